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
constexpr int kGenDynLds = 57 * 1024;  // dynamic LDS of a decode workgroup: with its static arrays <= 64 KiB

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
    // the chunk's loads go out in rounds of up to four per thread (at most
    // kGenChunk / EP / kGenThreads pieces: 8, 4 or 2), each round's before
    // its first LDS store
    typedef uint32_t v4u __attribute__((ext_vector_type(4)));
    constexpr int kMaxPieces = kGenChunk / EP / kGenThreads < 4 ? kGenChunk / EP / kGenThreads : 4;
    const int ppr = cw / EP;  // pieces per row
    const int pl = __builtin_ctz((unsigned)ppr);
    const int n = a.ts * ppr;
    for (int e0 = threadIdx.x; e0 < n; e0 += kMaxPieces * kGenThreads) {
      v4u w[kMaxPieces];
#pragma unroll
      for (int i = 0; i < kMaxPieces; ++i) {
        const int e = e0 + i * kGenThreads;
        w[i] = v4u{0u, 0u, 0u, 0u};
        if (e < n) {
          const int64_t o = off[e >> pl];
          if (o >= 0)
            w[i] = __builtin_nontemporal_load(
                reinterpret_cast<const v4u*>(base + o + (int64_t)(c0 + (e & (ppr - 1)) * EP) * es));
        }
      }
#pragma unroll
      for (int i = 0; i < kMaxPieces; ++i) {
        const int e = e0 + i * kGenThreads;
        if (e < n) {
          const int tt = e >> pl, pc = e & (ppr - 1);
          const bool ok = off[tt] >= 0;
          const uint32_t ww[4] = {w[i][0], w[i][1], w[i][2], w[i][3]};
          float* dst = s + tt * sp + pc * EP;
          if ((sp & 3) == 0) {
            // 16-byte aligned rows (the decode's pitch): 128-bit stores
#pragma unroll
            for (int k = 0; k < EP; k += 4)
              *reinterpret_cast<float4*>(dst + k) =
                  ok ? make_float4(val(elem<DT>(ww, k)), val(elem<DT>(ww, k + 1)), val(elem<DT>(ww, k + 2)),
                                   val(elem<DT>(ww, k + 3)))
                     : make_float4(0.f, 0.f, 0.f, 0.f);
          } else {
#pragma unroll
            for (int k = 0; k < EP; ++k) dst[k] = ok ? val(elem<DT>(ww, k)) : 0.f;
          }
        }
      }
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

// Band energies of a staged 64-token, 128-column chunk (unscaled, this
// thread's share) with the transform's butterflies (those of gen_fwht, in
// its stage order) in registers.  Thread tid works on column tid mod 128:
// stages 1..8 (row bits 0..3) on its two 16-row blocks 32 h and 32 h + 16
// (h = tid / 128), stored back; after one barrier, stages 16 and 32 as
// 4-point butterflies of rows (q, q + 16, q + 32, q + 48) for its eight
// q = 8 h .. 8 h + 7, summing X[q]^2 over q = 1..7 and X[q + 32]^2,
// X[q + 48]^2.  sk is left changed.
__device__ __forceinline__ void gen_bands_64x128(float* sk, float& el, float& eh) {
  constexpr int spd = 132;  // gen_pitch(128): constant LDS offsets
  const int c = threadIdx.x & 127, h = threadIdx.x >> 7;
#pragma unroll
  for (int blk = 0; blk < 2; ++blk) {
    float* col = sk + (32 * h + 16 * blk) * spd + c;
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) x[i] = col[i * spd];
#pragma unroll
    for (int st = 0; st < 4; ++st)
#pragma unroll
      for (int i = 0; i < 16; ++i)
        if (!(i & (1 << st))) {
          const float a = x[i], b = x[i + (1 << st)];
          x[i] = a + b;
          x[i + (1 << st)] = a - b;
        }
#pragma unroll
    for (int i = 0; i < 16; ++i) col[i * spd] = x[i];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int q = 8 * h + i;
    const float y0 = sk[q * spd + c], y1 = sk[(q + 16) * spd + c];
    const float y2 = sk[(q + 32) * spd + c], y3 = sk[(q + 48) * spd + c];
    const float a = y0 + y1, b = y0 - y1, d = y2 + y3, e = y2 - y3;
    if (q >= 1 && q < 8) el = __builtin_fmaf(a + d, a + d, el);
    eh = __builtin_fmaf(a - d, a - d, eh);
    eh = __builtin_fmaf(b - e, b - e, eh);
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

__host__ __device__ __forceinline__ int gen_chunk_cols(int ts, int d) { return min(d, kGenChunk / ts); }

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

// Row pitch (floats) of a staged decode chunk (gen_bands_64x128 assumes 132
// for 128 columns): cw + 4 keeps every row
// 16-byte aligned for 128-bit LDS reads and puts the rows' starts 4 banks
// apart; chunks narrower than 4 columns (head_dim 1 or 2) use cw + 1.
__host__ __device__ __forceinline__ int gen_pitch(int cw) { return (cw & 3) ? cw + 1 : cw + 4; }

// Dynamic LDS floats of one decode workgroup (gen_decode_kernel's layout)
__host__ __device__ __forceinline__ int gen_decode_floats(int ts, int d, int gt, int cw) {
  return ts * gen_pitch(cw) + 2 * gt * d + gt * ts;
}

// Logits of one staged K chunk, 128-bit reads: lg[m] += q_g . k over the
// chunk's columns for the thread's heads g = min(gq + nq m, gmax), m < HG
// (kr: the thread's token row; columns in order, as the scalar path).
template <int HG, int M0 = 0>
__device__ __forceinline__ void gen_logits4(const float* kr, const float* sq, int D, int c0, int cw, int gq, int nq,
                                            int gmax, float (&lg)[kGenHeads]) {
  constexpr int kU = HG <= 2 ? 2 : 1;  // column steps in flight
  const float* qh[HG];
#pragma unroll
  for (int m = 0; m < HG; ++m) qh[m] = sq + min(gq + nq * (M0 + m), gmax) * D + c0;
#pragma unroll kU
  for (int c = 0; c < cw; c += 4) {
    const float4 k4 = *reinterpret_cast<const float4*>(kr + c);
#pragma unroll
    for (int m = 0; m < HG; ++m) {
      const float4 q4 = *reinterpret_cast<const float4*>(qh[m] + c);
      float x = __builtin_fmaf(q4.x, k4.x, lg[M0 + m]);
      x = __builtin_fmaf(q4.y, k4.y, x);
      x = __builtin_fmaf(q4.z, k4.z, x);
      lg[M0 + m] = __builtin_fmaf(q4.w, k4.w, x);
    }
  }
}

// p.V of one staged V column for the thread's heads g = min(gv + nv m,
// gmax), m < HG: cur[m] += sum_tt p_g[tt] v[tt], 128-bit reads of p, tokens
// in order
template <int HG, int M0 = 0>
__device__ __forceinline__ void gen_pv4(const float* vc, int spd, const float* sp, int TS, int gv, int nv, int gmax,
                                        float (&cur)[kGenHeads]) {
  constexpr int kU = HG <= 2 ? 2 : 1;  // token steps in flight
  const float* ph[HG];
#pragma unroll
  for (int m = 0; m < HG; ++m) ph[m] = sp + min(gv + nv * (M0 + m), gmax) * TS;
#pragma unroll kU
  for (int tt = 0; tt < TS; tt += 4) {
    const float v0 = vc[tt * spd], v1 = vc[(tt + 1) * spd], v2 = vc[(tt + 2) * spd], v3 = vc[(tt + 3) * spd];
#pragma unroll
    for (int m = 0; m < HG; ++m) {
      const float4 p4 = *reinterpret_cast<const float4*>(ph[m] + tt);
      float x = __builtin_fmaf(p4.x, v0, cur[M0 + m]);
      x = __builtin_fmaf(p4.y, v1, x);
      x = __builtin_fmaf(p4.z, v2, x);
      cur[M0 + m] = __builtin_fmaf(p4.w, v3, x);
    }
  }
}

__device__ __forceinline__ int gen_pow2_ceil(int x) { return x <= 1 ? 1 : (x <= 2 ? 2 : (x <= 4 ? 4 : 8)); }

// The gated decode.  grid = (Pg, rows, ceil(G / GT)), GT = min(G, 8) query
// heads per workgroup (heads_per_group's chunks of up to 8), cw the columns
// of a staged chunk (chosen by the host so that the LDS below fits 64 KiB).
// LDS of one workgroup (gen_decode_floats): the staged chunk (TS rows at
// pitch gen_pitch(cw)), the group's q heads (GT x D), its logits, then
// probabilities (GT x TS), and its p.V accumulators (GT x D).
// Work of thread tid:
//   logits: token tq = tid mod TS of heads qs + nq m (qs = tid / TS,
//           nq = 256 / TS);
//   p.V:    column tid mod cw of each chunk (and + 256 in 512-column
//           chunks) for heads vs + nv m (vs = tid / cw, nv = 256 / cw; 0 and
//           1 for chunks of 256 columns or more); accumulator (g, column)
//           belongs to one thread, so it needs no barrier.
template <int DT, int VT>
__global__ __launch_bounds__(kGenThreads) __attribute__((amdgpu_waves_per_eu(3)))
void gen_decode_kernel(const DecodeArgs a, int D, int GT, int cw) {
  extern __shared__ __align__(16) float gen_lds[];
  __shared__ int64_t koff[kGenMaxTS], voff[kGenMaxTS];
  __shared__ float s_m[kGenHeads], s_l[kGenHeads], s_alpha[kGenHeads];
  __shared__ float red[4];
  __shared__ int s_qnan;
  __shared__ float s_qmax;
  __shared__ float s_ks[kGenThreads], s_vs[kGenThreads];  // tile scales of a batch of tiles
  __shared__ uint8_t s_flag[kGenThreads];                  // their keep flags (gates without K)
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
  const int spd = gen_pitch(cw);
  const bool vec = (cw & 3) == 0 && (TS & 3) == 0;  // the 128-bit paths
  float* sk = gen_lds;        // staged K, then V, chunk
  float* sq = sk + TS * spd;  // the group's q heads
  float* sp = sq + GT * D;    // logits, then probabilities
  float* sacc = sp + GT * TS; // p.V accumulators, (head, column)

  // q of this group's heads (q * k_scale rounded in q's dtype for Q_FOLD)
  auto q_at = [&](int g, int c) {
    float x = load_scalar(a.q + ((int64_t)row * a.G + g) * a.q_row_stride + (int64_t)c * qes, a.q_dtype);
    if (a.k_scale_mode == OC_KSCALE_Q_FOLD) x = round_to(x * a.k_scale, a.q_dtype);
    return x;
  };
  // (four loads in flight per thread)
  for (int e0 = tid; e0 < gn * D; e0 += 4 * kGenThreads) {
    float x[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = e0 + i * kGenThreads;
      x[i] = e < gn * D ? q_at(g0 + e / D, e % D) : 0.f;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = e0 + i * kGenThreads;
      if (e < gn * D) {
        sq[e] = x[i];
        sacc[e] = 0.f;
      }
    }
  }
  // max over all G heads of the row of ||q_g||_2 (CS gate; below 1e-38 as
  // 0), from the staged q when the group holds every head of the row
  if (a.gate == OC_GATE_CS) {
    const bool staged = gn == a.G;
    if (staged) __syncthreads();
    float qmax = 0.f;
    bool qnan = false;
    for (int g = wave; g < a.G; g += kGenThreads / 64) {
      float ss = 0.f;
      for (int c = lane; c < D; c += 64) {
        const float x = staged ? sq[g * D + c] : q_at(g, c);
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

  // the thread's logits work
  const int ts_log = __builtin_ctz((unsigned)TS);
  const int nq = kGenThreads >> ts_log;  // TS <= 256
  const int tq = tid & (TS - 1), qs = tid >> ts_log;
  const int hq = (gn + nq - 1) / nq;  // heads per thread (some past gn: clamped, dropped)
  const int hq2 = gen_pow2_ceil(hq);
  // the thread's p.V work
  const int cl = __builtin_ctz((unsigned)cw);
  const int cpt = cw > kGenThreads ? cw / kGenThreads : 1;  // columns per chunk
  const int nv = cw >= kGenThreads ? 1 : kGenThreads >> cl;
  const int vs = cw >= kGenThreads ? 0 : tid >> cl;
  const int vcol = tid & (min(cw, kGenThreads) - 1);
  const int hv = (gn + nv - 1) / nv;
  const int hv2 = gen_pow2_ceil(hv);
  int kept = 0;
  const int s_lo = gidx * a.spw, s_hi = min(a.P, s_lo + a.spw);
  // gates that need no K (mask, cached scores, none) and the tile scales are
  // read for up to 256 tiles of a split at once, one tile per thread, into
  // LDS ahead of the tiles' loop (instead of one dependent load per tile)
  const bool pre_gate = a.gate == OC_GATE_MASK || (cached && a.gate != OC_GATE_NONE);
  const bool ks_tile = a.k_scale_mode == OC_KSCALE_TILE, vs_tile = a.v_scale_mode == OC_VSCALE_TILE;
  for (int s = s_lo; s < s_hi; ++s) {
    const int nt_s = s < n_tiles ? (n_tiles - 1 - s) / a.P + 1 : 0;  // tiles s + kP of the row
    for (int k0 = 0; k0 < nt_s; k0 += kGenThreads) {
      const int kn = min(nt_s - k0, kGenThreads);
      __syncthreads();  // the previous batch's flags and scales are consumed
      if (tid < kn) {
        const int t = s + (k0 + tid) * a.P;
        bool keep = true;
        if (a.gate == OC_GATE_MASK) {
          keep = a.tmask[(int64_t)row * a.tmask_stride + t] != 0;
        } else if (pre_gate && (int64_t)(t + 1) * TS <= n_tok) {
          const float eh = a.sc_eh[(int64_t)row * a.sc_stride + t];
          const float el = a.gate == OC_GATE_ZETA ? a.sc_el[(int64_t)row * a.sc_stride + t] : 0.f;
          keep = gate_keep(a.gate, a.thr, el, eh, qmax, qnan);
        }
        s_flag[tid] = keep ? 1 : 0;
        if (!keep && a.keep_out && blockIdx.z == 0) a.keep_out[(int64_t)row * a.keep_stride + t] = 0;
        if (keep && ks_tile) s_ks[tid] = a.k_scales[(int64_t)row * a.ks_stride + t];
        if (keep && vs_tile) s_vs[tid] = a.v_scales[(int64_t)row * a.vs_stride + t];
      }
      __syncthreads();
      for (int kk = 0; kk < kn; ++kk) {
        const int t = s + (k0 + kk) * a.P;
        const int tok0 = t * TS;
        const int valid = min(TS, n_tok - tok0);
        const bool full = valid == TS;
        bool keep = s_flag[kk] != 0;
        if (!keep) continue;
        gen_row_offsets(a, row, tok0, n_tok, koff, voff);
        const float ks = ks_tile ? s_ks[kk] : 1.f;
        const float vmul = vs_tile ? s_vs[kk] : 1.f;
        __syncthreads();
        // K: logits (and the single-pass gate's band energies)
        float lg[kGenHeads];
  #pragma unroll
        for (int m = 0; m < kGenHeads; ++m) lg[m] = 0.f;
        float el = 0.f, eh = 0.f;
        for (int c0 = 0; c0 < D; c0 += cw) {
          gen_stage<DT, true>(a, a.k, koff, c0, cw, spd, sk, ks, 1.f);
          __syncthreads();
          const float* kr = sk + tq * spd;
          if (vec) {
            switch (hq2) {
              case 1: gen_logits4<1>(kr, sq, D, c0, cw, qs, nq, gn - 1, lg); break;
              case 2: gen_logits4<2>(kr, sq, D, c0, cw, qs, nq, gn - 1, lg); break;
              case 4: gen_logits4<4>(kr, sq, D, c0, cw, qs, nq, gn - 1, lg); break;
              default:  // eight heads in two passes of four (the register budget)
                gen_logits4<4, 0>(kr, sq, D, c0, cw, qs, nq, gn - 1, lg);
                gen_logits4<4, 4>(kr, sq, D, c0, cw, qs, nq, gn - 1, lg);
                break;
            }
          } else {
  #pragma unroll
            for (int m = 0; m < kGenHeads; ++m) {
              if (m < hq) {
                const float* qg = sq + min(qs + nq * m, gn - 1) * D + c0;
                float x = lg[m];
                for (int c = 0; c < cw; ++c) x = __builtin_fmaf(qg[c], kr[c], x);
                lg[m] = x;
              }
            }
          }
          if (sp_gate) {
            __syncthreads();
            if (TS == 64 && cw == 128) {
              gen_bands_64x128(sk, el, eh);
            } else {
              gen_fwht(sk, TS, cw, spd);
              gen_bands(sk, TS, cw, spd, el, eh);
            }
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
        for (int m = 0; m < kGenHeads; ++m) {
          const int g = qs + nq * m;
          if (m < hq && g < gn) sp[g * TS + tq] = tq < valid ? lg[m] * a.scale : -__builtin_inff();
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
        // V: p . V over the staged column chunks; each accumulator is
        // rescaled by its head's alpha as it is read (every chunk is visited
        // once per retained tile)
        for (int c0 = 0; c0 < D; c0 += cw) {
          gen_stage<VT, false>(a, a.v, voff, c0, cw, spd, sk, 1.f, vmul);
          __syncthreads();
          for (int u = 0; u < cpt; ++u) {
            const int c = vcol + u * kGenThreads;
            float cur[kGenHeads];
  #pragma unroll
            for (int m = 0; m < kGenHeads; ++m) {
              const int g = min(vs + nv * m, gn - 1);
              cur[m] = m < hv ? sacc[g * D + c0 + c] * s_alpha[g] : 0.f;
            }
            if (vec) {
              switch (hv2) {
                case 1: gen_pv4<1>(sk + c, spd, sp, TS, vs, nv, gn - 1, cur); break;
                case 2: gen_pv4<2>(sk + c, spd, sp, TS, vs, nv, gn - 1, cur); break;
                case 4: gen_pv4<4>(sk + c, spd, sp, TS, vs, nv, gn - 1, cur); break;
                default:
                  gen_pv4<4, 0>(sk + c, spd, sp, TS, vs, nv, gn - 1, cur);
                  gen_pv4<4, 4>(sk + c, spd, sp, TS, vs, nv, gn - 1, cur);
                  break;
              }
            } else {
  #pragma unroll
              for (int m = 0; m < kGenHeads; ++m) {
                if (m < hv) {
                  const float* pg = sp + min(vs + nv * m, gn - 1) * TS;
                  float x = cur[m];
                  for (int tt = 0; tt < TS; ++tt) x = __builtin_fmaf(pg[tt], sk[tt * spd + c], x);
                  cur[m] = x;
                }
              }
            }
  #pragma unroll
            for (int m = 0; m < kGenHeads; ++m) {
              const int g = vs + nv * m;
              if (m < hv && g < gn) sacc[g * D + c0 + c] = cur[m];
            }
          }
          __syncthreads();
        }
      }
    }
  }
  // the group's partial state: index ((row * G + g) * Pg + gidx); the
  // accumulators were last written by their owners before a barrier
  const int64_t pbase = (int64_t)row * a.G * a.Pg;
  for (int e = tid; e < gn * D; e += kGenThreads) {
    const int g = e / D;
    a.pacc[(pbase + (int64_t)(g0 + g) * a.Pg + gidx) * D + (e - g * D)] = sacc[e];
  }
  if (tid < gn) {
    const int64_t pidx = pbase + (int64_t)(g0 + tid) * a.Pg + gidx;
    a.pm[pidx] = s_m[tid];
    a.pl[pidx] = s_l[tid];
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
  // the widest power-of-two chunk (at most kGenChunk staged values) whose
  // LDS, with the kernel's static arrays (under 4.5 KiB), fits 64 KiB
  const int ts = a.ts;
  if (gt > kGenHeads || ts > kGenMaxTS || D > kGenMaxD) return hipErrorInvalidValue;
  int cw = gen_chunk_cols(ts, D);
  while (cw > 1 && gen_decode_floats(ts, D, gt, cw) * (int)sizeof(float) > kGenDynLds) cw >>= 1;
  const size_t lds = sizeof(float) * (size_t)gen_decode_floats(ts, D, gt, cw);
  if (lds > (size_t)kGenDynLds) return hipErrorInvalidValue;
  switch (dt) {
    case OC_F32: hipLaunchKernelGGL((gen_decode_kernel<OC_F32, OC_F32>), grid, block, lds, st, a, D, gt, cw); break;
    case OC_F16: hipLaunchKernelGGL((gen_decode_kernel<OC_F16, OC_F16>), grid, block, lds, st, a, D, gt, cw); break;
    case OC_BF16: hipLaunchKernelGGL((gen_decode_kernel<OC_BF16, OC_BF16>), grid, block, lds, st, a, D, gt, cw); break;
    default:
      if (a.v_bf16) hipLaunchKernelGGL((gen_decode_kernel<OC_FP8_E4M3FN, OC_BF16>), grid, block, lds, st, a, D, gt, cw);
      else hipLaunchKernelGGL((gen_decode_kernel<OC_FP8_E4M3FN, OC_FP8_E4M3FN>), grid, block, lds, st, a, D, gt, cw);
      break;
  }
  return hipGetLastError();
}

}  // namespace oc
