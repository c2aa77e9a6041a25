// Portable tile scoring and gated split-K decode for every power-of-two
// head_dim (1..512) and tile size (1..256): the reference's own contract
// (head_dim and tile_size are asserted to be powers of two,
// fused_eviction.py:609-610 and :738-739, gqa_eviction.py:551-552,
// paged_eviction.py:345-347).  The tuned kernels of oc_kernels.h cover
// head_dim 64 and 128 with 64-token tiles, every BASELINE configuration;
// these cover the rest with the same semantics:
//   * tile t of a row holds tokens [t*TS, t*TS + TS); its spectrum is the
//     natural-order (Sylvester) Walsh-Hadamard transform along the tokens,
//     X = (H_TS / sqrt(TS)) K_tile, and the bands are the reference's fixed
//     row ranges [1, 8) and [32, 64) clipped to the TS rows
//     (fused_eviction.py:424-427 slices energy_per_seq[1:8] and [32:64]);
//   * the zeta, Cauchy-Schwarz and mask gates, the cached / single-pass
//     modes, the K / V scale modes, paged block tables and row lengths are
//     those of oc_decode (gate_keep and friends are shared);
//   * split s of a row owns tiles {s + kP} (fused_eviction.py:259); a
//     workgroup takes splits_per_group consecutive splits and writes their
//     merged float32 state (m, l, acc[head_dim]) as one partial, which
//     merge_kernel (oc_api.hip) combines.
// Layout of the work: one 256-thread workgroup per (split group, row, chunk
// of up to 8 query heads).  A tile is staged through LDS as float32 in
// column chunks of at most 8192 values (32 KiB): K for the logits (and, in a
// single-pass gated decode, the in-place transform and band energies), then
// V for p.V, with every thread owning one or two output columns.  The path
// is VALU-only and element-wise in its loads; the tuned kernels are the ones
// the bench lines time.

#include "oc_kernels.h"
#include "oc_generic.h"

namespace oc {
namespace {

constexpr int kGenThreads = 256;
constexpr int kGenChunk = 8192;  // floats of one staged chunk of a tile
constexpr int kGenHeads = 8;     // query heads per workgroup
constexpr int kGenMaxTS = 256;
constexpr int kGenMaxD = 512;

// Element of K or V as float32 (fp8-e4m3fn decoded exactly)
template <int DT>
__device__ __forceinline__ float gen_elem(const char* p) {
  if constexpr (DT == OC_F32) {
    return *reinterpret_cast<const float*>(p);
  } else if constexpr (DT == OC_FP8_E4M3FN) {
    const auto f = __builtin_amdgcn_cvt_pk_f32_fp8((int)*reinterpret_cast<const uint8_t*>(p), false);
    return f[0];
  } else {
    return load_scalar(p, DT);
  }
}

// Tokens of row r (its length clamped to num_tiles * TS), as row_tokens
__device__ __forceinline__ int gen_row_tokens(const DecodeArgs& a, int r) {
  const int cap = a.num_tiles * a.ts;
  int n = a.row_tok > 0 ? a.row_tok : cap;
  if (a.lengths) {
    const int len = a.lengths[r / a.rows_per_length];
    n = len < 0 ? 0 : (len < n ? len : n);
  }
  return n;
}

// Byte offsets (from the pool base) of the K and V rows of tokens
// [tok0, tok0 + TS) of row `row`, or -1 past the row's tokens or for a
// block id outside the pool (which raises the error flag); thread j < TS
// fills entry j.
__device__ __forceinline__ void gen_row_offsets(const DecodeArgs& a, int row, int tok0, int n_tok, int64_t* koff,
                                                int64_t* voff) {
  const int j = threadIdx.x;
  if (j >= a.ts) return;
  const int tok = tok0 + j;
  int64_t ko = -1, vo = -1;
  if (tok < n_tok) {
    if (a.paged) {
      const int seq = row / a.nkv, head = row - (row / a.nkv) * a.nkv;
      const int id = a.bt[(int64_t)seq * a.bt_stride + (tok >> a.bs_log2)];
      if (id >= 0 && id < a.num_blocks) {
        const int64_t in = (int64_t)(tok & ((1 << a.bs_log2) - 1));
        ko = (int64_t)id * a.k_blk_stride + (int64_t)head * a.k_head_stride + in * a.k_tok_stride;
        vo = (int64_t)id * a.v_blk_stride + (int64_t)head * a.v_head_stride + in * a.v_tok_stride;
      } else if (a.error_flag) {
        atomicOr(a.error_flag, 1);
      }
    } else {
      ko = (int64_t)row * a.k_row_stride + (int64_t)tok * a.k_tok_stride;
      vo = (int64_t)row * a.v_row_stride + (int64_t)tok * a.v_tok_stride;
    }
  }
  koff[j] = ko;
  voff[j] = vo;
}

// Stage columns [c0, c0 + cw) of the tile's rows into s[tt * sp + c]
// (zeros for rows without an offset).  vmul: V's tile scale (V staging) or
// 1; ks: K's tile scale (K staging).  With a.gen_vec (every row offset and
// the column chunk 16-byte aligned, set by the host) each thread moves
// 16-byte pieces; otherwise one element at a time.
template <int DT, bool ISK>
__device__ __forceinline__ void gen_stage(const DecodeArgs& a, const char* base, const int64_t* off, int c0, int cw,
                                          int sp, float* s, float ks, float vmul) {
  constexpr int es = Elem<DT>::size;
  constexpr int EP = 16 / es;  // elements per 16-byte piece
  auto val = [&](float x) {
    if constexpr (ISK) {
      if (a.k_scale_mode == OC_KSCALE_TILE) return x * ks;
      if (a.k_scale_mode == OC_KSCALE_DEQUANT) return round_bf16(x * a.k_scale);
      return x;
    } else {
      return x * vmul;
    }
  };
  if (a.gen_vec && cw >= EP) {
    typedef uint32_t v4u __attribute__((ext_vector_type(4)));
    const int ppr = cw / EP;  // pieces per row
    const int pl = __builtin_ctz((unsigned)ppr);
    const int n = a.ts * ppr;
    for (int e = threadIdx.x; e < n; e += kGenThreads) {
      const int tt = e >> pl, pc = e & (ppr - 1);
      const int64_t o = off[tt];
      v4u w = v4u{0u, 0u, 0u, 0u};
      if (o >= 0) w = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(base + o + (int64_t)(c0 + pc * EP) * es));
      const uint32_t ww[4] = {w[0], w[1], w[2], w[3]};
      float* dst = s + tt * sp + pc * EP;
#pragma unroll
      for (int i = 0; i < EP; ++i) dst[i] = o >= 0 ? val(elem<DT>(ww, i)) : 0.f;
    }
    return;
  }
  const int n = a.ts * cw;
  const int cl = __builtin_ctz((unsigned)cw);
  for (int e = threadIdx.x; e < n; e += kGenThreads) {
    const int tt = e >> cl, c = e & (cw - 1);
    const int64_t o = off[tt];
    float x = 0.f;
    if (o >= 0) x = val(gen_elem<DT>(base + o + (int64_t)(c0 + c) * es));
    s[tt * sp + c] = x;
  }
}

// In-place natural-order Walsh-Hadamard butterflies (a, b) -> (a + b, a - b)
// along the TS rows of every staged column (unscaled: H_TS x)
__device__ __forceinline__ void gen_fwht(float* s, int ts, int cw, int sp) {
  const int cl = __builtin_ctz((unsigned)cw);
  const int n = (ts >> 1) * cw;
  for (int h = 1; h < ts; h <<= 1) {
    for (int e = threadIdx.x; e < n; e += kGenThreads) {
      const int pi = e >> cl, c = e & (cw - 1);
      const int r = ((pi & ~(h - 1)) << 1) | (pi & (h - 1));
      const float x = s[r * sp + c], y = s[(r + h) * sp + c];
      s[r * sp + c] = x + y;
      s[(r + h) * sp + c] = x - y;
    }
    __syncthreads();
  }
}

// Band energies of the staged (transformed) chunk, this thread's share
__device__ __forceinline__ void gen_bands(const float* s, int ts, int cw, int sp, float& el, float& eh) {
  const int cl = __builtin_ctz((unsigned)cw);
  const int lo_end = min(8, ts), hi_end = min(64, ts);
  for (int e = threadIdx.x; e < ts * cw; e += kGenThreads) {
    const int tt = e >> cl, c = e & (cw - 1);
    const float x = s[tt * sp + c];
    if (tt >= 1 && tt < lo_end) el = __builtin_fmaf(x, x, el);
    if (tt >= 32 && tt < hi_end) eh = __builtin_fmaf(x, x, eh);
  }
}

__device__ __forceinline__ float gen_block_sum(float x, float* red) {
  x = wave_sum(x);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[w] = x;
  __syncthreads();
  x = red[0] + red[1] + red[2] + red[3];
  __syncthreads();
  return x;
}

__device__ __forceinline__ int gen_chunk_cols(int ts, int d) { return min(d, kGenChunk / ts); }

// Scores (and, with o_fwht, the full transform) of tiles [t0, t0 + tcnt) of
// every row: one workgroup per (row, tile).  A partial tail tile gets zero
// energies and keep = 1, as score_kernel.
template <int DT>
__global__ __launch_bounds__(kGenThreads) void gen_score_kernel(const DecodeArgs a, int D) {
  __shared__ float sk[kGenChunk + kGenMaxTS];
  __shared__ int64_t koff[kGenMaxTS], voff[kGenMaxTS];
  __shared__ float red[4];
  const int TS = a.ts;
  const int64_t job = blockIdx.x;
  const int row = (int)(job / a.tcnt);
  const int t = a.t0 + (int)(job - (int64_t)row * a.tcnt);
  const int n_tok = gen_row_tokens(a, row);
  const int n_tiles = (n_tok + TS - 1) / TS;
  const bool full = (int64_t)(t + 1) * TS <= n_tok;
  float el = 0.f, eh = 0.f;
  if (full || a.o_fwht) {
    gen_row_offsets(a, row, t * TS, n_tok, koff, voff);
    const float ks = a.k_scale_mode == OC_KSCALE_TILE ? a.k_scales[(int64_t)row * a.ks_stride + t] : 1.f;
    __syncthreads();
    const int cw = gen_chunk_cols(TS, D), sp = cw + 1;
    const float inv = 1.f / __builtin_sqrtf((float)TS);
    for (int c0 = 0; c0 < D; c0 += cw) {
      gen_stage<DT, true>(a, a.k, koff, c0, cw, sp, sk, ks, 1.f);
      __syncthreads();
      gen_fwht(sk, TS, cw, sp);
      gen_bands(sk, TS, cw, sp, el, eh);
      if (a.o_fwht) {
        const int cl = __builtin_ctz((unsigned)cw);
        float* o = a.o_fwht + (((int64_t)row * a.num_tiles + t) * TS) * D;
        for (int e = threadIdx.x; e < TS * cw; e += kGenThreads) {
          const int tt = e >> cl, c = e & (cw - 1);
          o[(int64_t)tt * D + c0 + c] = sk[tt * sp + c] * inv;
        }
      }
      __syncthreads();
    }
    el = gen_block_sum(el, red) / (float)TS;
    eh = gen_block_sum(eh, red) / (float)TS;
    if (!full) el = eh = 0.f;
  }
  if (threadIdx.x == 0 && (a.o_el || a.o_eh || a.o_z || a.o_keep)) {
    const int64_t o = (int64_t)row * a.o_stride + t;
    float z = 0.f;
    uint8_t keep = 0;
    if (full) {
      z = eh / (el + 1e-6f);
      keep = gate_keep(OC_GATE_ZETA, a.thr, el, eh, 0.f, false) ? 1 : 0;
    } else if (t < n_tiles) {
      keep = 1;
    }
    if (a.o_el) a.o_el[o] = el;
    if (a.o_eh) a.o_eh[o] = eh;
    if (a.o_z) a.o_z[o] = z;
    if (a.o_keep) a.o_keep[o] = keep;
  }
}

// The gated decode.  grid = (Pg, rows, ceil(G / GT)), GT = min(G, 8) query
// heads per workgroup (heads_per_group's chunks of up to 8).
template <int DT, int VT>
__global__ __launch_bounds__(kGenThreads) void gen_decode_kernel(const DecodeArgs a, int D, int GT) {
  __shared__ float sk[kGenChunk + kGenMaxTS];          // staged K, then V, chunk
  __shared__ float sq[kGenHeads * kGenMaxD];            // this chunk's q heads
  __shared__ float sp[kGenHeads * kGenMaxTS];           // logits, then probabilities
  __shared__ int64_t koff[kGenMaxTS], voff[kGenMaxTS];
  __shared__ float s_m[kGenHeads], s_l[kGenHeads], s_alpha[kGenHeads];
  __shared__ float red[4];
  __shared__ int s_keep, s_qnan;
  __shared__ float s_qmax;
  const int TS = a.ts;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int gidx = blockIdx.x, row = blockIdx.y;
  const int g0 = blockIdx.z * GT;
  const int gn = min(GT, a.G - g0);
  const int n_tok = gen_row_tokens(a, row);
  const int n_tiles = (n_tok + TS - 1) / TS;
  const bool cached = a.mode == OC_MODE_CACHED;
  const bool sp_gate = !cached && (a.gate == OC_GATE_ZETA || a.gate == OC_GATE_CS);
  const int qes = a.q_dtype == OC_F32 ? 4 : 2;

  // q of this chunk's heads (q * k_scale rounded in q's dtype for Q_FOLD)
  auto q_at = [&](int g, int c) {
    float x = load_scalar(a.q + ((int64_t)row * a.G + g) * a.q_row_stride + (int64_t)c * qes, a.q_dtype);
    if (a.k_scale_mode == OC_KSCALE_Q_FOLD) x = round_to(x * a.k_scale, a.q_dtype);
    return x;
  };
  for (int e = tid; e < gn * D; e += kGenThreads) sq[e] = q_at(g0 + e / D, e % D);
  // max over all G heads of the row of ||q_g||_2 (CS gate; below 1e-38 as 0)
  if (a.gate == OC_GATE_CS) {
    float qmax = 0.f;
    bool qnan = false;
    for (int g = wave; g < a.G; g += kGenThreads / 64) {
      float ss = 0.f;
      for (int c = lane; c < D; c += 64) {
        const float x = q_at(g, c);
        ss = __builtin_fmaf(x, x, ss);
      }
      float qn = __builtin_sqrtf(wave_sum(ss));
      if ((double)qn < 1e-38) qn = 0.f;
      if (__builtin_isnan(qn)) qnan = true;
      else qmax = fmaxf(qmax, qn);
    }
    if (lane == 0) red[wave] = qnan ? __builtin_nanf("") : qmax;
    __syncthreads();
    if (tid == 0) {
      float m = 0.f;
      int nan = 0;
      for (int w = 0; w < 4; ++w) {
        if (__builtin_isnan(red[w])) nan = 1;
        else m = fmaxf(m, red[w]);
      }
      s_qmax = m;
      s_qnan = nan;
    }
  }
  if (tid < kGenHeads) {
    s_m[tid] = kM0;
    s_l[tid] = 0.f;
  }
  __syncthreads();
  const float qmax = a.gate == OC_GATE_CS ? s_qmax : 0.f;
  const bool qnan = a.gate == OC_GATE_CS && s_qnan != 0;

  // output columns of this thread: tid and tid + 256
  float acc[kGenHeads][2];
#pragma unroll
  for (int g = 0; g < kGenHeads; ++g) acc[g][0] = acc[g][1] = 0.f;
  const int cw = gen_chunk_cols(TS, D), spd = cw + 1;
  const int ts_log = __builtin_ctz((unsigned)TS);
  const int npair = gn * TS;  // (head, token) logits, up to 2048: 8 per thread
  int kept = 0;
  const int s_lo = gidx * a.spw, s_hi = min(a.P, s_lo + a.spw);
  for (int s = s_lo; s < s_hi; ++s) {
    for (int t = s; t < n_tiles; t += a.P) {
      const int tok0 = t * TS;
      const int valid = min(TS, n_tok - tok0);
      const bool full = valid == TS;
      // the gate where it needs no K (uniform over the workgroup)
      bool keep = true;
      if (a.gate == OC_GATE_MASK) {
        keep = a.tmask[(int64_t)row * a.tmask_stride + t] != 0;
      } else if (cached && a.gate != OC_GATE_NONE && full) {
        const float eh = a.sc_eh[(int64_t)row * a.sc_stride + t];
        const float el = a.gate == OC_GATE_ZETA ? a.sc_el[(int64_t)row * a.sc_stride + t] : 0.f;
        keep = gate_keep(a.gate, a.thr, el, eh, qmax, qnan);
      }
      if (!keep) {
        if (a.keep_out && blockIdx.z == 0 && tid == 0) a.keep_out[(int64_t)row * a.keep_stride + t] = 0;
        continue;
      }
      gen_row_offsets(a, row, tok0, n_tok, koff, voff);
      const float ks = a.k_scale_mode == OC_KSCALE_TILE ? a.k_scales[(int64_t)row * a.ks_stride + t] : 1.f;
      const float vmul = a.v_scale_mode == OC_VSCALE_TILE ? a.v_scales[(int64_t)row * a.vs_stride + t] : 1.f;
      __syncthreads();
      // K: logits (and the single-pass gate's band energies)
      float lg[kGenHeads * kGenMaxTS / kGenThreads];
#pragma unroll
      for (int i = 0; i < kGenHeads * kGenMaxTS / kGenThreads; ++i) lg[i] = 0.f;
      float el = 0.f, eh = 0.f;
      for (int c0 = 0; c0 < D; c0 += cw) {
        gen_stage<DT, true>(a, a.k, koff, c0, cw, spd, sk, ks, 1.f);
        __syncthreads();
#pragma unroll
        for (int i = 0; i < kGenHeads * kGenMaxTS / kGenThreads; ++i) {
          const int pr = tid + i * kGenThreads;
          if (pr < npair) {
            const int g = pr >> ts_log, tt = pr & (TS - 1);
            const float* qg = sq + g * D + c0;
            const float* kr = sk + tt * spd;
            float x = lg[i];
            for (int c = 0; c < cw; ++c) x = __builtin_fmaf(qg[c], kr[c], x);
            lg[i] = x;
          }
        }
        if (sp_gate) {
          __syncthreads();
          gen_fwht(sk, TS, cw, spd);
          gen_bands(sk, TS, cw, spd, el, eh);
        }
        __syncthreads();
      }
      if (sp_gate) {
        el = gen_block_sum(el, red) / (float)TS;
        eh = gen_block_sum(eh, red) / (float)TS;
        keep = full ? gate_keep(a.gate, a.thr, el, eh, qmax, qnan) : true;
      }
      if (a.keep_out && blockIdx.z == 0 && tid == 0) a.keep_out[(int64_t)row * a.keep_stride + t] = keep ? 1 : 0;
      if (!keep) continue;
      ++kept;
      // online softmax per head: logits to LDS, then one wave per head
#pragma unroll
      for (int i = 0; i < kGenHeads * kGenMaxTS / kGenThreads; ++i) {
        const int pr = tid + i * kGenThreads;
        if (pr < npair) sp[pr] = (pr & (TS - 1)) < valid ? lg[i] * a.scale : -__builtin_inff();
      }
      __syncthreads();
      for (int g = wave; g < gn; g += kGenThreads / 64) {
        float* pg = sp + g * TS;
        float mt = -__builtin_inff();
        for (int tt = lane; tt < TS; tt += 64) mt = fmaxf(mt, pg[tt]);
        mt = wave_max(mt);
        const float mo = s_m[g];
        const float mn = fmaxf(mo, mt);
        float ls = 0.f;
        for (int tt = lane; tt < TS; tt += 64) {
          const float p = __expf(pg[tt] - mn);
          pg[tt] = p;
          ls += p;
        }
        ls = wave_sum(ls);
        const float alpha = __expf(mo - mn);
        if (lane == 0) {
          s_alpha[g] = alpha;
          s_m[g] = mn;
          s_l[g] = __builtin_fmaf(s_l[g], alpha, ls);
        }
      }
      __syncthreads();
#pragma unroll
      for (int g = 0; g < kGenHeads; ++g) {
        if (g < gn) {
          acc[g][0] *= s_alpha[g];
          acc[g][1] *= s_alpha[g];
        }
      }
      // V: p . V over the staged column chunks
      for (int c0 = 0; c0 < D; c0 += cw) {
        gen_stage<VT, false>(a, a.v, voff, c0, cw, spd, sk, 1.f, vmul);
        __syncthreads();
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int c = tid + j * kGenThreads;
          if (c >= c0 && c < c0 + cw && c < D) {
            const float* vc = sk + (c - c0);
#pragma unroll
            for (int g = 0; g < kGenHeads; ++g) {
              if (g < gn) {
                const float* pg = sp + g * TS;
                float x = acc[g][j];
                for (int tt = 0; tt < TS; ++tt) x = __builtin_fmaf(pg[tt], vc[tt * spd], x);
                acc[g][j] = x;
              }
            }
          }
        }
        __syncthreads();
      }
    }
  }
  // the group's partial state: index ((row * G + g) * Pg + gidx)
  const int64_t pbase = (int64_t)row * a.G * a.Pg;
  for (int g = 0; g < gn; ++g) {
    const int64_t pidx = pbase + (int64_t)(g0 + g) * a.Pg + gidx;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int c = tid + j * kGenThreads;
      if (c < D) a.pacc[pidx * D + c] = acc[g][j];
    }
    if (tid == 0) {
      a.pm[pidx] = s_m[g];
      a.pl[pidx] = s_l[g];
    }
  }
  if (a.split_counts && blockIdx.z == 0 && tid == 0) a.split_counts[(int64_t)row * a.Pg + gidx] = kept;
}

}  // namespace

bool generic_shape(int head_dim, int tile_size) {
  return !(tile_size == 64 && (head_dim == 64 || head_dim == 128));
}

bool generic_supported(int head_dim, int tile_size) {
  auto pow2 = [](int x) { return x > 0 && (x & (x - 1)) == 0; };
  return pow2(head_dim) && head_dim <= kGenMaxD && pow2(tile_size) && tile_size <= kGenMaxTS;
}

hipError_t gen_launch_score(int dt, const DecodeArgs& a, int D, hipStream_t st) {
  const dim3 grid((unsigned)((int64_t)a.num_rows * a.tcnt)), block(kGenThreads);
  switch (dt) {
    case OC_F32: hipLaunchKernelGGL(gen_score_kernel<OC_F32>, grid, block, 0, st, a, D); break;
    case OC_F16: hipLaunchKernelGGL(gen_score_kernel<OC_F16>, grid, block, 0, st, a, D); break;
    case OC_BF16: hipLaunchKernelGGL(gen_score_kernel<OC_BF16>, grid, block, 0, st, a, D); break;
    default: hipLaunchKernelGGL(gen_score_kernel<OC_FP8_E4M3FN>, grid, block, 0, st, a, D); break;
  }
  return hipGetLastError();
}

hipError_t gen_launch_decode(int dt, const DecodeArgs& a, int D, int gt, int gchunks, hipStream_t st) {
  const dim3 grid(a.Pg, a.num_rows, gchunks), block(kGenThreads);
  switch (dt) {
    case OC_F32: hipLaunchKernelGGL((gen_decode_kernel<OC_F32, OC_F32>), grid, block, 0, st, a, D, gt); break;
    case OC_F16: hipLaunchKernelGGL((gen_decode_kernel<OC_F16, OC_F16>), grid, block, 0, st, a, D, gt); break;
    case OC_BF16: hipLaunchKernelGGL((gen_decode_kernel<OC_BF16, OC_BF16>), grid, block, 0, st, a, D, gt); break;
    default:
      if (a.v_bf16) hipLaunchKernelGGL((gen_decode_kernel<OC_FP8_E4M3FN, OC_BF16>), grid, block, 0, st, a, D, gt);
      else hipLaunchKernelGGL((gen_decode_kernel<OC_FP8_E4M3FN, OC_FP8_E4M3FN>), grid, block, 0, st, a, D, gt);
      break;
  }
  return hipGetLastError();
}

}  // namespace oc
