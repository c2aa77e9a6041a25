// The model-side attention hook's device work (declared in
// include/orthocache_hip.h): causal GQA prefill attention that skips the
// evicted 64-token tiles, the per-row q norms, an exact k-th-smallest
// selection (the median of those norms) and the per-kv-head gate over cached
// K band norms.
//
// Prefill attention is a flash-attention forward pass on the matrix cores.
// A wave owns 16 consecutive query positions of one q head (the 16 rows of
// the 16x16 MFMA tiles) and walks the 64-token K/V tiles its causal window
// reaches, skipping the tiles the mask evicts: S = q.K^T, online softmax with
// a per-row causal limit, O += P.V.  A workgroup is 8 waves = 128 positions
// of one head sharing each K/V tile through LDS; the workgroups of one kv
// group run next to each other on one XCD, so the K/V tiles they share stay
// in that XCD's L2.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "oc_kernels.h"
#include "oc_status.h"
#include "orthocache_hip.h"

namespace oc {
namespace {

constexpr int kPfWaves = 8;
constexpr int kPfRows = 16 * kPfWaves;  // query positions per workgroup
constexpr int kPfThreads = kPfWaves * kWave;
constexpr int kPfPvGroup = 4;  // p.V column pairs whose V reads are in flight together
// work items of a call that splits its longest causal windows (beyond: no split)
constexpr int kPfMaxItems = 512;
// -(1e-10) * ln(1e-10): what one zero probability adds to the entropy of a
// softmax row whose probabilities are clamped to >= 1e-10 before the log
constexpr float kZeroPTerm = 2.302585093e-9f;

struct PrefillArgs {
  const char* q;
  const char* k;
  const char* v;
  char* out;
  int64_t q_sb, q_sh, q_ss;  // byte strides (batch, head, position)
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_sh, o_ss;
  int32_t B, Hq, Hkv, G, Sq, Skv, T;  // T: full tiles the mask covers
  const uint8_t* mask;                // (B, Hkv, >= T) evict flags or null
  int64_t m_sb, m_sh;
  float scale;
  float* entropy;  // (B, Hq, Sq) or null
  int32_t qblocks;
  int32_t dtype;
  // split windows (nitems > 0): work item e is query block items[e] >> 2,
  // part items[e] & 3 (0: its whole window; 1, 2: the first and second half
  // of its tiles).  Blocks >= q0 are split: (block, head) pair k of them keeps
  // the two halves' per-lane states at part + (2 k + half) * 512 * (4 + D/4)
  // floats and its ticket at ctr[k * ctr_stride].
  int32_t nitems, q0, ctr_stride;
  float* part;
  int32_t* ctr;
  uint16_t items[kPfMaxItems];
};

// Online-softmax state in the transposed layout: lane 16r + x works on
// query x (scores of tokens 16tb + 4r + i, i = 0..3, in c[tb][i]); m is
// shared by the query's four lanes x, x + 16, x + 32, x + 48, and l, e are
// their partial sums.  Scores are kept in base-2 units (s * log2 e), so
// that each probability is one exp2.
struct PfState {
  float m;  // running max, base-2 units
  float l;
  float e;  // sum of 2^(s2 - m) * s2 (entropy), base-2 units
  int n;    // attended tokens of the query (entropy)
};

// Causal online-softmax update of one tile's raw scores c (transposed
// layout); token tok0 + j is visible to the lane's query when tok0 + j <
// nvis.  full (wave-uniform): every token of the tile is visible to every
// query of the wave (no mask needed).  scale2 = softmax scale * log2 e.
// c becomes 2^(s2 - m) and the accumulators are rescaled.
template <int D, bool ENT>
__device__ __forceinline__ void pf_softmax(PfState& st, f32x4 (&acc)[D / 16], f32x4 (&c)[4], float scale2, int nvis,
                                           int tok0, bool full, int lane) {
  (void)lane;  // lane / 16 (the row group r) is formed from the thread index below
  float mt = -__builtin_inff();
  if (full) {
#pragma unroll
    for (int tb = 0; tb < 4; ++tb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float v = c[tb][i] * scale2;
        c[tb][i] = v;
        mt = fmaxf(mt, v);
      }
  } else {
    // 4 r formed here from the thread index (lane = threadIdx.x mod 64; the
    // empty asm keeps the compiler from keeping it in a register across the
    // tile loop, where the bfloat16 entropy kernels would spill it)
    int tx = threadIdx.x;
    asm volatile("" : "+v"(tx));
    const int r4 = (tx >> 2) & 12;
#pragma unroll
    for (int tb = 0; tb < 4; ++tb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float v = tok0 + 16 * tb + r4 + i < nvis ? c[tb][i] * scale2 : -__builtin_inff();
        c[tb][i] = v;
        mt = fmaxf(mt, v);
      }
  }
  mt = fmaxf(mt, xpair<16>(mt));
  mt = fmaxf(mt, xpair<32>(mt));
  const float mn = fmaxf(st.m, mt);
  const float alpha = __builtin_amdgcn_exp2f(st.m - mn);
  st.m = mn;
  float ls = 0.f, es = 0.f;
#pragma unroll
  for (int tb = 0; tb < 4; ++tb)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float v = c[tb][i];
      const float pp = __builtin_amdgcn_exp2f(v - mn);
      ls += pp;
      if constexpr (ENT) es = pp > 0.f ? __builtin_fmaf(pp, v, es) : es;
      c[tb][i] = pp;
    }
  st.l = __builtin_fmaf(st.l, alpha, ls);
  if constexpr (ENT) {
    st.e = __builtin_fmaf(st.e, alpha, es);
    st.n += min(max(nvis - tok0, 0), 64);
  }
  // most tiles leave every running max unchanged (alpha == 1 in every lane)
  if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {
#pragma unroll
    for (int nc = 0; nc < D / 16; ++nc) acc[nc] *= alpha;
  }
}

// q of the wave's 16 rows as MFMA A operands.  16-bit: lane 16kg + x holds
// elements 32dc + 8kg .. +8 of row x for instruction dc.  float32 (16x16x4
// instructions): lane 16kg + x holds column kg*D/4 + dc of row x for
// instruction dc.  Rows past q_len read as zero.
template <int DT, int D>
struct PfQ {
  static constexpr bool F32 = DT == OC_F32;
  uint32_t w[F32 ? D / 4 : D / 8];
};

template <int DT, int D>
__device__ __forceinline__ void pf_load_q(const PrefillArgs& a, const char* qh, int pos0, int lane, PfQ<DT, D>& q) {
  const int x = lane & 15;
  const int kg = lane >> 4;
  const bool ok = pos0 + x < a.Sq;
  const char* rowp = qh + (int64_t)(pos0 + x) * a.q_ss;
  if constexpr (DT == OC_F32) {
#pragma unroll
    for (int j = 0; j < D / 16; ++j) {
      uint4 u = {0u, 0u, 0u, 0u};
      if (ok) u = *reinterpret_cast<const uint4*>(rowp + 4 * (kg * (D / 4) + 4 * j));
      q.w[4 * j] = u.x;
      q.w[4 * j + 1] = u.y;
      q.w[4 * j + 2] = u.z;
      q.w[4 * j + 3] = u.w;
    }
  } else {
#pragma unroll
    for (int dc = 0; dc < D / 32; ++dc) {
      uint4 u = {0u, 0u, 0u, 0u};
      if (ok) u = *reinterpret_cast<const uint4*>(rowp + 2 * (32 * dc + 8 * kg));
      q.w[4 * dc] = u.x;
      q.w[4 * dc + 1] = u.y;
      q.w[4 * dc + 2] = u.z;
      q.w[4 * dc + 3] = u.w;
    }
  }
}

// The workgroup's shared K/V tiles: K and V of one 64-token tile, row-major
// [token][D], in STAGES LDS stages.  The 256 threads stage the next tile
// through registers: each loads its 16-byte chunks while the waves compute
// the current tile, and stores them once that compute is done.  K's chunks
// are XOR-swizzled per row (chunk c of row r sits at c ^ swz(r)) so that the
// 16 rows one B-operand read touches fall in distinct LDS banks.
template <int DT, int D>
struct PfTile {
  static constexpr int ES = DT == OC_F32 ? 4 : 2;
  static constexpr int ROW = D * ES;                      // bytes per token row
  static constexpr int LPT = ROW / 16;                    // 16-byte chunks per row
  static constexpr int RB = ROW >= 256 ? 1 : 256 / ROW;   // rows per 256-byte bank line
  static constexpr int KV = 64 * ROW;                     // bytes of one K (or V) tile
  static constexpr int NL = KV / (kPfThreads * 16);       // chunks per thread per matrix
  static constexpr int STAGES = 2 * KV <= 32768 ? 2 : 1;
  static constexpr int LDS = STAGES * 2 * KV;
  __device__ static int swz(int r) { return (r / RB) % LPT; }
  // 16-bit V: the 32-byte column pair p of LDS row r is stored at pair
  // p ^ vswz(r).  A transposing read takes one pair of the 16 rows
  // 8g + i (+ 4h), g, i < 4; vswz gives those rows distinct pairs (each
  // bank slot used twice) instead of one pair 16 times over.
  static constexpr int PAIRS = ROW / 32;
  __device__ static int vswz(int r) {
    return PAIRS >= 8 ? (r & 3) + 4 * ((r >> 3) & 1) : ((r & 3) >> 1) + 2 * ((r >> 3) & 1);
  }
};

template <int DT, int D>
struct PfStage {
  uint4 k[PfTile<DT, D>::NL];
  uint4 v[PfTile<DT, D>::NL];
};

// a wave-uniform pointer as scalar registers
__device__ __forceinline__ const char* pf_uniform(const char* p) {
  const uint64_t u = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)u);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(u >> 32));
  return reinterpret_cast<const char*>(((uint64_t)hi << 32) | lo);
}

// global -> registers: chunk g = tid + 256 j of the tile is row g / LPT,
// chunk g % LPT; rows at or past kv_len read as zero (buffer range check)
template <int DT, int D>
__device__ __forceinline__ void pf_fetch(const PrefillArgs& a, const char* kh, const char* vh, int t, int tid,
                                         PfStage<DT, D>& st) {
  using L = PfTile<DT, D>;
  // every value of the resources is wave-uniform; saying so keeps the
  // compiler from wrapping each load in a readfirstlane loop
  t = __builtin_amdgcn_readfirstlane(t);
  const int nvalid = min(a.Skv - t * 64, 64);
  const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
      (void*)pf_uniform(kh + (int64_t)t * 64 * a.k_ss), (short)0,
      __builtin_amdgcn_readfirstlane(nvalid * (int)a.k_ss), 0x00020000);
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
      (void*)pf_uniform(vh + (int64_t)t * 64 * a.v_ss), (short)0,
      __builtin_amdgcn_readfirstlane(nvalid * (int)a.v_ss), 0x00020000);
#pragma unroll
  for (int j = 0; j < L::NL; ++j) {
    const int g = tid + kPfThreads * j;
    const int r = g / L::LPT, c = g % L::LPT;
    const auto uk = __builtin_amdgcn_raw_buffer_load_b128(rk, r * (int)a.k_ss + 16 * c, 0, 0);
    const auto uv = __builtin_amdgcn_raw_buffer_load_b128(rv, r * (int)a.v_ss + 16 * c, 0, 0);
    st.k[j] = uint4{uk[0], uk[1], uk[2], uk[3]};
    st.v[j] = uint4{uv[0], uv[1], uv[2], uv[3]};
  }
}

// 16 bytes per lane from a buffer straight to LDS: lane i's bytes land at
// dst + 16 i (dst wave-uniform)
__device__ __forceinline__ void pf_load_lds16(__amdgpu_buffer_rsrc_t r, char* dst, int voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 16, voff, 0, 0, 0);
}

// Token kept in LDS row r of a 16-bit V stage: within each 32-token block,
// token 16a + 4g + b sits in row 8g + 4a + b, so that the transposing read
// of rows 8g .. 8g + 7 hands lane group g the tokens 4g + b and 16 + 4g + b
// -- the tokens whose scores the lane holds (pf_pv).
__device__ __forceinline__ int pf_vtok(int r) {
  return (r & ~31) + 16 * ((r >> 2) & 1) + 4 * ((r >> 3) & 3) + (r & 3);
}

// global -> an LDS stage directly (two-stage tiles): each wave's load
// instruction fills a contiguous 1 KiB of the stage, slot g = tid + 512 j
// (row g / LPT, chunk g % LPT), so the lane filling a slot loads the chunk
// that the layout keeps there: K chunk c ^ swz(row); 16-bit V the token
// pf_vtok(row), chunk c ^ 2 vswz(row).  Rows at or past kv_len read as zero
// (buffer range check).  Default cache policy: the G query heads' workgroups
// of a kv head read the same tiles.
template <int DT, int D>
__device__ __forceinline__ void pf_fetch_lds(const PrefillArgs& a, const char* kh, const char* vh, int t, int tid,
                                             char* sk, char* sv) {
  using L = PfTile<DT, D>;
  t = __builtin_amdgcn_readfirstlane(t);
  const int nvalid = min(a.Skv - t * 64, 64);
  const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
      (void*)pf_uniform(kh + (int64_t)t * 64 * a.k_ss), (short)0,
      __builtin_amdgcn_readfirstlane(nvalid * (int)a.k_ss), 0x00020000);
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
      (void*)pf_uniform(vh + (int64_t)t * 64 * a.v_ss), (short)0,
      __builtin_amdgcn_readfirstlane(nvalid * (int)a.v_ss), 0x00020000);
  const int wbase = __builtin_amdgcn_readfirstlane(tid & ~63);  // the wave's first slot
#pragma unroll
  for (int j = 0; j < L::NL; ++j) {
    const int g = tid + kPfThreads * j;
    const int r = g / L::LPT, c = g % L::LPT;
    const int slot0 = 16 * (wbase + kPfThreads * j);
    pf_load_lds16(rk, sk + slot0, r * (int)a.k_ss + 16 * (c ^ L::swz(r)));
    int vt = r, vc = c;
    if constexpr (DT != OC_F32) {
      vt = pf_vtok(r);
      vc = c ^ (2 * L::vswz(r));
    }
    pf_load_lds16(rv, sv + slot0, vt * (int)a.v_ss + 16 * vc);
  }
}

// registers -> the LDS stage (single-stage tiles: float32 at head_dim 128;
// 16-bit tiles always have two stages and load straight into LDS): K
// swizzled, V in token order
template <int DT, int D>
__device__ __forceinline__ void pf_stash(const PfStage<DT, D>& st, int tid, char* sk, char* sv) {
  using L = PfTile<DT, D>;
  static_assert(DT == OC_F32, "only float32 tiles are staged through registers");
#pragma unroll
  for (int j = 0; j < L::NL; ++j) {
    const int g = tid + kPfThreads * j;
    const int r = g / L::LPT, c = g % L::LPT;
    *reinterpret_cast<uint4*>(sk + r * L::ROW + 16 * (c ^ L::swz(r))) = st.k[j];
    *reinterpret_cast<uint4*>(sv + r * L::ROW + 16 * c) = st.v[j];
  }
}

// S^T = K.q^T of one tile from the LDS stage: c[tb][i] is the score of
// token 16tb + 4r + i for query x in lane 16r + x.  K is the A operand:
// 16-bit instruction dc takes row 16tb + x, logical chunk 4dc + kg; float32
// reads 4 columns kg*D/4 + 4j .. for instructions 4j .. 4j + 3; q (the B
// operand) is in the same registers as before.
template <int DT, int D>
__device__ __forceinline__ void pf_logits(const PfQ<DT, D>& q, const char* sk, int lane, f32x4 (&c)[4]) {
  using L = PfTile<DT, D>;
  const int x = lane & 15;
  const int kg = lane >> 4;
#pragma unroll
  for (int tb = 0; tb < 4; ++tb) {
    c[tb] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int r = 16 * tb + x;
    const char* rowp = sk + r * L::ROW;
    const int sw = L::swz(r);
    if constexpr (DT == OC_F32) {
#pragma unroll
      for (int j = 0; j < D / 16; ++j) {
        const uint4 u = *reinterpret_cast<const uint4*>(rowp + 16 * ((kg * (D / 16) + j) ^ sw));
        const uint32_t uw[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int e = 0; e < 4; ++e)
          c[tb] = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(uw[e]), __uint_as_float(q.w[4 * j + e]),
                                                       c[tb], 0, 0, 0);
      }
    } else {
#pragma unroll
      for (int dc = 0; dc < D / 32; ++dc) {
        const uint4 u = *reinterpret_cast<const uint4*>(rowp + 16 * ((4 * dc + kg) ^ sw));
        const uint32_t aq[4] = {q.w[4 * dc], q.w[4 * dc + 1], q.w[4 * dc + 2], q.w[4 * dc + 3]};
        const uint32_t bk[4] = {u.x, u.y, u.z, u.w};
        c[tb] = mfma_qk<DT>(bk, aq, c[tb]);
      }
    }
  }
}

// O^T += V^T P^T on the matrix cores (transposed layout): acc[nc][i] is
// output column 16nc + 4r + i of query x in lane 16r + x.  16-bit: per
// 32-token block j, A = V^T read with ds_read_b64_tr_b16 from the permuted
// rows (lane group g gets tokens 32j + 4g + b and 32j + 16 + 4g + b), B =
// the lane's own eight probabilities c[2j][b], c[2j + 1][b]: float16 rounds
// them once (relative error at most 2^-12); bfloat16 sends a 16-bit high
// part plus the 16-bit rounding of the remainder (two instructions), since
// one rounding (2^-9) moves short causal rows past the output tolerance.
// float32: 16x16x4 steps over (tb, i), A = V[16tb + 4r + i][16nc + x], B =
// c[tb][i], exact.
template <int DT, int D>
__device__ __forceinline__ void pf_pv(f32x4 (&acc)[D / 16], const f32x4 (&c)[4], const char* svb, int lane) {
  const int x = lane & 15;
  const int kg = lane >> 4;
  if constexpr (DT == OC_F32) {
    const float* sv = reinterpret_cast<const float*>(svb);
#pragma unroll
    for (int tb = 0; tb < 4; ++tb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float* vr = sv + (16 * tb + 4 * kg + i) * D + x;
#pragma unroll
        for (int nc = 0; nc < D / 16; ++nc)
          acc[nc] = __builtin_amdgcn_mfma_f32_16x16x4f32(vr[16 * nc], c[tb][i], acc[nc], 0, 0, 0);
      }
  } else {
    typedef short s16x4 __attribute__((ext_vector_type(4)));
    const uint16_t* sv = reinterpret_cast<const uint16_t*>(svb);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      float pv[8];
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        pv[b] = c[2 * j][b];
        pv[4 + b] = c[2 * j + 1][b];
      }
      uint32_t bhi[4], blo[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if constexpr (DT == OC_BF16) {
          const __bf16 h0 = (__bf16)pv[2 * e], h1 = (__bf16)pv[2 * e + 1];
          const __bf16 l0 = (__bf16)(pv[2 * e] - (float)h0), l1 = (__bf16)(pv[2 * e + 1] - (float)h1);
          bhi[e] = (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
          blo[e] = (uint32_t)__builtin_bit_cast(uint16_t, l0) | ((uint32_t)__builtin_bit_cast(uint16_t, l1) << 16);
        } else {
          const _Float16 h0 = (_Float16)pv[2 * e], h1 = (_Float16)pv[2 * e + 1];
          bhi[e] = (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
        }
      }
      // lane x of group kg reads rows 32j + 8kg + 4h + x/4 (h = 0, 1), column
      // pair nc stored at nc ^ vswz(row) (the same for h = 0, 1 and every j)
      const int vrow = 32 * j + 8 * kg + (x >> 2);
      const int vt = PfTile<DT, D>::vswz(vrow);
      const uint16_t* rowp = sv + vrow * D + 4 * (x & 3);
      // the transposing reads of GS column pairs are issued before their
      // products, so that their latencies overlap
#pragma unroll
      for (int n0 = 0; n0 < D / 16; n0 += kPfPvGroup) {
        uint32_t av[kPfPvGroup][4];
#pragma unroll
        for (int g = 0; g < kPfPvGroup; ++g) {
          const int nc = n0 + g;
          const s16x4 b0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) s16x4*)(rowp + 16 * (nc ^ vt)));
          const s16x4 b1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) s16x4*)(rowp + 4 * D + 16 * (nc ^ vt)));
          typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
          const u32x2 w0 = __builtin_bit_cast(u32x2, b0), w1 = __builtin_bit_cast(u32x2, b1);
          av[g][0] = w0[0];
          av[g][1] = w0[1];
          av[g][2] = w1[0];
          av[g][3] = w1[1];
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int g = 0; g < kPfPvGroup; ++g) {
          acc[n0 + g] = mfma_qk<DT>(av[g], bhi, acc[n0 + g]);
          if constexpr (DT == OC_BF16) acc[n0 + g] = mfma_qk<DT>(av[g], blo, acc[n0 + g]);
        }
      }
    }
  }
}

template <int DT, int D, bool ENT, bool SPLIT>
__global__ __launch_bounds__(kPfThreads) __attribute__((amdgpu_waves_per_eu(DT == OC_F32 && D == 128 ? 1 : 4))) void prefill_kernel(
    const PrefillArgs a) {
  using L = PfTile<DT, D>;
  __shared__ __attribute__((aligned(16))) char sh[L::LDS];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  // XCD-aware order: workgroup i runs on XCD i % 8.  Each XCD takes a
  // contiguous eighth of the (batch, head) pairs -- whole kv groups or equal
  // parts of one, whose K/V tiles then stay in that XCD's L2 -- over every
  // query block, dispatched from the last block (longest causal window) to
  // the first, heads fastest.  So every XCD gets the same mix of window
  // lengths, longest first.  (Without eight equal parts: the same order over
  // the whole grid.)
  // With split windows the items come from the host's table, longest first.
  const int nbh = a.B * a.Hq;
  const int i = blockIdx.x;
  int bh, e;
  if (nbh % 8 == 0) {
    const int hpx = nbh / 8, j = i / 8;
    bh = (i % 8) * hpx + j % hpx;
    e = j / hpx;
  } else {
    bh = i % nbh;
    e = i / nbh;
  }
  int qb = a.qblocks - 1 - e, part = 0;
  if constexpr (SPLIT) {
    qb = a.items[e] >> 2;
    part = a.items[e] & 3;
  }
  const int b = bh / a.Hq;
  const int h = bh % a.Hq;
  const int kv = h / a.G;
  const int pos0 = qb * kPfRows + 16 * wave;

  const int off = a.Skv - a.Sq;  // query s sees keys j <= s + off
  const int r = lane >> 4;
  const int x = lane & 15;
  const int qpos = pos0 + x;  // this lane's query
  const int nvis = qpos < a.Sq ? min(max(qpos + off + 1, 0), a.Skv) : 0;
  // the wave's smallest window (its first query's); lanes past Sq are not
  // masked on full tiles, their results are never written
  const int nvis_w = min(max(pos0 + off + 1, 0), a.Skv);
  const float scale2 = a.scale * 1.4426950408889634f;  // log2 e
  // this wave's tiles, and the workgroup's (its last query's window)
  const int tend = pos0 < a.Sq ? (min(max(min(pos0 + 15, a.Sq - 1) + off + 1, 0), a.Skv) + 63) / 64 : 0;
  const int wg_tend = (min(max(min(qb * kPfRows + kPfRows - 1, a.Sq - 1) + off + 1, 0), a.Skv) + 63) / 64;
  // this item's tiles: the window, or one half of it
  const int tsplit = (wg_tend + 1) / 2;
  const int t_lo = part == 2 ? tsplit : 0;
  const int t_hi = part == 1 ? tsplit : wg_tend;

  PfQ<DT, D> q;
  pf_load_q<DT, D>(a, a.q + (int64_t)b * a.q_sb + (int64_t)h * a.q_sh, pos0, lane, q);
  const char* kh = a.k + (int64_t)b * a.k_sb + (int64_t)kv * a.k_sh;
  const char* vh = a.v + (int64_t)b * a.v_sb + (int64_t)kv * a.v_sh;
  const uint8_t* mrow = a.mask ? a.mask + (int64_t)b * a.m_sb + (int64_t)kv * a.m_sh : nullptr;
  auto next_kept = [&](int t) {  // first retained tile >= t (uniform over the workgroup)
    while (t < t_hi && mrow && t < a.T && mrow[t]) ++t;
    return t;
  };

  PfState st{kM0, 0.f, 0.f, 0};
  f32x4 accp[D / 16];
#pragma unroll
  for (int nc = 0; nc < D / 16; ++nc) accp[nc] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto stage_k = [&](int s) { return sh + s * 2 * L::KV; };
  auto stage_v = [&](int s) { return sh + s * 2 * L::KV + L::KV; };
  int t = next_kept(t_lo);
  if constexpr (L::STAGES == 2) {
    // two stages: the next tile goes straight to the other stage while this
    // one is used; each wave waits for its own loads before the barrier
    // that opens the stage to the workgroup
    if (t < t_hi) pf_fetch_lds<DT, D>(a, kh, vh, t, tid, stage_k(0), stage_v(0));
    __builtin_amdgcn_s_waitcnt(0);
    int s = 0;
    // one tile: the next one requested into the other stage, this one
    // computed.  The stages are restrict parameters, so the compiler knows
    // that the direct-to-LDS loads into one do not write what is read from
    // the other, and issues no wait for them before the reads.
    auto step = [&](int tn, char* __restrict__ nk, char* __restrict__ nv, const char* __restrict__ ck,
                    const char* __restrict__ cv) {
      if (tn < t_hi) pf_fetch_lds<DT, D>(a, kh, vh, tn, tid, nk, nv);
      if (t < tend) {
        f32x4 c[4];
        pf_logits<DT, D>(q, ck, lane, c);
        pf_softmax<D, ENT>(st, accp, c, scale2, nvis, t * 64, t * 64 + 64 <= nvis_w, lane);
        pf_pv<DT, D>(accp, c, cv, lane);
      }
    };
    while (t < t_hi) {
      // stage s is complete; every wave is done with the tile before (stage s ^ 1)
      __syncthreads();
      const int tn = next_kept(t + 1);
      step(tn, stage_k(1 - s), stage_v(1 - s), stage_k(s), stage_v(s));
      __builtin_amdgcn_s_waitcnt(0);
      s = 1 - s;
      t = tn;
    }
  } else {
    // one stage (float32, head_dim 128): the next tile waits in registers
    // and is written to the stage once every wave is done with it
    PfStage<DT, D> reg;
    if (t < t_hi) {
      pf_fetch<DT, D>(a, kh, vh, t, tid, reg);
      pf_stash<DT, D>(reg, tid, stage_k(0), stage_v(0));
    }
    while (t < t_hi) {
      __syncthreads();  // the stage is complete
      const int tn = next_kept(t + 1);
      if (tn < t_hi) pf_fetch<DT, D>(a, kh, vh, tn, tid, reg);  // in flight during this tile
      if (t < tend) {
        f32x4 c[4];
        pf_logits<DT, D>(q, stage_k(0), lane, c);
        pf_softmax<D, ENT>(st, accp, c, scale2, nvis, t * 64, t * 64 + 64 <= nvis_w, lane);
        pf_pv<DT, D>(accp, c, stage_v(0), lane);
      }
      __syncthreads();  // the stage is free again
      if (tn < t_hi) pf_stash<DT, D>(reg, tid, stage_k(0), stage_v(0));
      t = tn;
    }
  }

  if (SPLIT && part != 0) {
    // one half of a split window: this workgroup's per-lane state goes out
    // (agent-scope stores, written through to memory), then a ticket; the
    // workgroup that takes the second ticket merges the other half's state
    // into its own, in the order first half, second half whichever it is,
    // and writes the output.  Per lane: m, l, e, n, then the accumulators.
    constexpr int NF = 4 + D / 4;
    const int64_t k = (int64_t)(qb - a.q0) * nbh + bh;
    float* mine = a.part + (2 * k + part - 1) * NF * kPfThreads + tid;
    auto put = [&](int f, float v) {
      __hip_atomic_store(mine + f * kPfThreads, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };
    put(0, st.m);
    put(1, st.l);
    put(2, st.e);
    put(3, __int_as_float(st.n));
#pragma unroll
    for (int nc = 0; nc < D / 16; ++nc)
#pragma unroll
      for (int u = 0; u < 4; ++u) put(4 + 4 * nc + u, accp[nc][u]);
    // The hand-off below relies on gfx950's cache behaviour rather than on a
    // release / acquire pair of the HIP memory model, as the decode's fused
    // merge does: an agent-scope store is written through this XCD's L2
    // (sc1), its vmcnt acknowledgement comes back once memory holds it, and
    // an agent-scope load in the other workgroup (sc1) is served from memory,
    // not from a stale line of that XCD's L2.  So once every thread's stores
    // are acknowledged and the barrier has passed, the ticket can be taken
    // relaxed.  The formal pair (release on the ticket: an L2 write-back of
    // the whole XCD; acquire in the merging workgroup: an L2 invalidate)
    // costs more than the merge it protects.
    __shared__ int sh_last;
    __builtin_amdgcn_s_waitcnt(0);  // this thread's stores are acknowledged
    __syncthreads();
    if (tid == 0) {
      int* c = a.ctr + k * a.ctr_stride;
      const int done = atomicAdd(c, 1) + 1;
      sh_last = done == 2;
      if (done == 2) atomicExch(c, 0);
    }
    __syncthreads();
    if (!sh_last) return;
    const float* other = a.part + (2 * k + 2 - part) * NF * kPfThreads + tid;
    auto get = [&](int f) { return __hip_atomic_load(other + f * kPfThreads, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
    const float m2 = get(0), l2 = get(1), e2 = get(2);
    const int n2 = __float_as_int(get(3));
    const float mm = fmaxf(st.m, m2);
    const float w1 = __builtin_amdgcn_exp2f(st.m - mm), w2 = __builtin_amdgcn_exp2f(m2 - mm);
    // (first half's w, value; second half's w, value)
    auto mix = [&](float own, float oth) {
      return part == 1 ? __builtin_fmaf(own, w1, oth * w2) : __builtin_fmaf(oth, w2, own * w1);
    };
    st.l = mix(st.l, l2);
    st.e = mix(st.e, e2);
    st.n += n2;
    st.m = mm;
#pragma unroll
    for (int nc = 0; nc < D / 16; ++nc)
#pragma unroll
      for (int u = 0; u < 4; ++u) accp[nc][u] = mix(accp[nc][u], get(4 + 4 * nc + u));
  }

  // sums over the query's four lanes, then out = acc / max(l, 1e-9): lane
  // 16r + x writes columns 16nc + 4r .. + 4 of query x
  float l = st.l;
  l += xpair<16>(l);
  l += xpair<32>(l);
  const float inv = 1.f / fmaxf(l, 1e-9f);
  // this lane's query again, formed from the thread index after the loop
  // instead of kept in a register across it (the empty asm keeps the
  // compiler from reusing the value from before the loop): that register
  // would be the one spilled to scratch in the bfloat16 entropy kernels
  int tid_late = tid;
  asm volatile("" : "+v"(tid_late));
  const int qpos_o = pos0 + (tid_late & 15);
  if (qpos_o < a.Sq) {
    char* orow = a.out + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh + (int64_t)qpos_o * a.o_ss;
#pragma unroll
    for (int nc = 0; nc < D / 16; ++nc) {
      const int col = 16 * nc + 4 * r;
      if constexpr (DT == OC_F32) {
        *reinterpret_cast<float4*>(orow + 4 * col) =
            float4{accp[nc][0] * inv, accp[nc][1] * inv, accp[nc][2] * inv, accp[nc][3] * inv};
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) store_scalar(orow + 2 * (col + e), a.dtype, accp[nc][e] * inv);
      }
    }
  }
  if constexpr (ENT) {
    float e = st.e;
    e += xpair<16>(e);
    e += xpair<32>(e);
    if (qpos_o < a.Sq && r == 0) {
      // H = -sum p ln p with p = e^(s - m) / l: m + ln l - (sum e^(s-m) s) / l,
      // plus the clamp term of the probabilities that are exactly zero
      const float hz = (float)(a.Skv - st.n) * kZeroPTerm;
      constexpr float kLn2 = 0.6931471805599453f;
      const float H = l > 0.f ? kLn2 * (st.m - e / l) + logf(l) + hz : (float)a.Skv * kZeroPTerm;
      a.entropy[((int64_t)b * a.Hq + h) * a.Sq + qpos_o] = H;
    }
  }
}

// ------------------------------------------------------------ gate helpers

__device__ __forceinline__ float pf_load_elem(const char* p, int dtype) {
  if (dtype == OC_F32) return *reinterpret_cast<const float*>(p);
  const uint16_t u = *reinterpret_cast<const uint16_t*>(p);
  if (dtype == OC_BF16) return __uint_as_float((uint32_t)u << 16);
  return (float)__builtin_bit_cast(_Float16, u);
}

// ||row||_2 of one head_dim row by one wave, or with low_band > 0 its
// Walsh-subspace high part sqrt(max(0, ||row||^2 - sum_i S_i^2 / bs)) (S_i:
// sums of blocks of bs = d / low_band elements).  shrow: d floats of LDS of
// this wave.  The result is in every lane.
__device__ float row_norm_wave(const char* p, int dtype, int d, int low_band, float* shrow, int lane) {
  const int es = dtype == OC_F32 ? 4 : 2;
  float ss = 0.f;
  for (int c = lane; c < d; c += 64) {
    const float v = pf_load_elem(p + (int64_t)c * es, dtype);
    shrow[c] = v;
    ss = __builtin_fmaf(v, v, ss);
  }
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
  if (low_band > 0) {
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int bs = d / low_band;
    float lo = 0.f;
    for (int i = lane; i < low_band; i += 64) {
      float s = 0.f;
      for (int k = 0; k < bs; ++k) s += shrow[i * bs + k];
      lo = __builtin_fmaf(s, s, lo);
    }
    for (int o = 32; o > 0; o >>= 1) lo += __shfl_xor(lo, o, 64);
    lo /= (float)bs;
    ss = ss - lo;
    ss = ss < 0.f ? 0.f : ss;
  }
  return __builtin_sqrtf(ss);
}

// One wave per row of a 3-index view (row_norm_wave).
__global__ __launch_bounds__(256) void row_norms_kernel(const char* x, int dtype, int64_t n0, int64_t n1,
                                                        int64_t n2, int64_t s0, int64_t s1, int64_t s2, int d,
                                                        int low_band, float* out) {
  __shared__ float sh[4][1024];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + wave;
  if (r >= n0 * n1 * n2) return;
  const int64_t i2 = r % n2, i1 = (r / n2) % n1, i0 = r / (n1 * n2);
  const float n = row_norm_wave(x + i0 * s0 + i1 * s1 + i2 * s2, dtype, d, low_band, sh[wave], lane);
  if (lane == 0) out[r] = n;
}

// k-th smallest (0-based) of n non-negative floats per row by a radix
// select over their bit patterns (monotone for x >= 0; NaN sorts last):
// four 8-bit passes, each a 256-bin LDS histogram, then the bin holding
// rank k.  One workgroup per row.
__global__ __launch_bounds__(256) void kth_smallest_kernel(const float* x, int64_t n, int64_t row_stride, int64_t k,
                                                           float* out) {
  __shared__ uint32_t hist[256];
  __shared__ uint32_t sel[2];
  const float* row = x + (int64_t)blockIdx.x * row_stride;
  uint32_t prefix = 0, pmask = 0;
  uint64_t rank = (uint64_t)k;
  for (int shift = 24; shift >= 0; shift -= 8) {
    hist[threadIdx.x] = 0;
    __syncthreads();
    for (int64_t j = threadIdx.x; j < n; j += 256) {
      const uint32_t u = __float_as_uint(row[j]);
      if ((u & pmask) == prefix) atomicAdd(&hist[(u >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      uint64_t acc = 0;
      int bin = 255;
      for (int i = 0; i < 256; ++i) {
        if (acc + hist[i] > rank) {
          bin = i;
          break;
        }
        acc += hist[i];
      }
      sel[0] = (uint32_t)bin;
      sel[1] = (uint32_t)(rank - acc);
    }
    __syncthreads();
    prefix |= sel[0] << shift;
    pmask |= 255u << shift;
    rank = sel[1];
    __syncthreads();
  }
  if (threadIdx.x == 0) out[blockIdx.x] = __uint_as_float(prefix);
}

// The group norm of G per-head norms: their max (NaN-propagating) or the
// element of rank G/2 of their sorted order (ties counted by index).
__device__ float group_norm(const float* qh, int G, int reduce) {
  if (reduce == OC_GROUP_MAX) {
    bool nan = false;
    float best = -__builtin_inff();
    for (int g = 0; g < G; ++g) {
      nan = nan || __builtin_isnan(qh[g]);
      best = qh[g] > best ? qh[g] : best;
    }
    return nan ? __builtin_nanf("") : best;
  }
  const int want = G / 2;
  float qn = 0.f;
  for (int g = 0; g < G; ++g) {
    int below = 0;
    for (int j = 0; j < G; ++j) below += (qh[j] < qh[g] || (qh[j] == qh[g] && j < g)) ? 1 : 0;
    if (below == want) qn = qh[g];
  }
  return qn;
}

// The tile gate of one (batch, kv head) by a 256-thread workgroup:
// mask[t] = qn * kn[t] <= tau_norm for t < num_tiles and 0 up to mask_cols
// (keep_pol: 1 = attend instead); with stats, the evicted count, qn and the
// largest kn of the complete tiles (NaN if any is NaN, -inf if none).
__device__ void gate_tiles(float qn, const float* knr, int num_tiles, int mask_cols, double tau_norm, int keep_pol,
                           uint8_t* mr, float* stats) {
  __shared__ float s_red[2][4];
  float nev = 0.f, kmax = -__builtin_inff();
  bool knan = false;
  for (int t = threadIdx.x; t < mask_cols; t += 256) {
    const bool full = t < num_tiles;
    // the reference compares (qn * kn) / (64 d) <= tau in float64 with
    // float32 norms; 64 d is a power of two, so that is qn * kn <= tau * 64 d
    // with an exact product (two float32 factors fit a double)
    const bool ev = full && (double)qn * (double)knr[t] <= tau_norm;
    mr[t] = (ev != (keep_pol != 0)) ? 1 : 0;
    if (full) {
      nev += ev ? 1.f : 0.f;
      kmax = fmaxf(kmax, knr[t]);
      knan = knan || __builtin_isnan(knr[t]);
    }
  }
  if (stats) {
    // unclamped: the hook clamps after its reductions over heads
    nev = wave_sum(nev);
    kmax = wave_max(kmax);
    const bool wnan = __ballot(knan) != 0;
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
      s_red[0][w] = nev;
      s_red[1][w] = wnan ? __builtin_nanf("") : kmax;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      stats[0] = s_red[0][0] + s_red[0][1] + s_red[0][2] + s_red[0][3];
      stats[1] = qn;
      float m = s_red[1][0];
      for (int i = 1; i < 4; ++i) m = (__builtin_isnan(m) || __builtin_isnan(s_red[1][i])) ? __builtin_nanf("") : fmaxf(m, s_red[1][i]);
      stats[2] = m;
    }
  }
}

// One workgroup per (batch, kv head): qn = group_norm of the group's G
// per-head norms, then gate_tiles.
__global__ __launch_bounds__(256) void group_gate_kernel(const float* qn_heads, int Hkv, int G, int reduce,
                                                         const float* kn, int64_t kn_sb, int64_t kn_sh,
                                                         int num_tiles, int mask_cols, double tau_norm, int keep_pol,
                                                         uint8_t* mask, int64_t m_sb, int64_t m_sh, float* qn_out,
                                                         float* stats) {
  __shared__ float s_qn;
  const int bk = blockIdx.x;
  const int b = bk / Hkv;
  const int kv = bk % Hkv;
  if (threadIdx.x == 0) {
    const float qn = group_norm(qn_heads + ((int64_t)b * Hkv + kv) * G, G, reduce);
    s_qn = qn;
    if (qn_out) qn_out[bk] = qn;
  }
  __syncthreads();
  gate_tiles(s_qn, kn + (int64_t)b * kn_sb + (int64_t)kv * kn_sh, num_tiles, mask_cols, tau_norm, keep_pol,
             mask + (int64_t)b * m_sb + (int64_t)kv * m_sh, stats ? stats + (int64_t)bk * 3 : nullptr);
}

// The hook's decode gate in one launch: per (batch, kv head) the Walsh-
// subspace high norms of the group's G query rows (row_norm_wave, four
// waves), their median and the tile gate with the partial tail attended
// (keep polarity).
__global__ __launch_bounds__(256) void hook_gate_kernel(const char* q, int dtype, int64_t q_row_bytes, int Hkv, int G,
                                                        int d, int low_band, const float* kn, int64_t kn_sh,
                                                        int num_tiles, int mask_cols, double tau_norm, uint8_t* mask,
                                                        int64_t m_sh, float* stats) {
  __shared__ float sh[4][1024];
  __shared__ float s_qh[64];
  __shared__ float s_qn;
  const int bk = blockIdx.x;
  const int kv = bk % Hkv;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  for (int g = wave; g < G; g += 4) {
    const float n = row_norm_wave(q + ((int64_t)bk * G + g) * q_row_bytes, dtype, d, low_band, sh[wave], lane);
    if (lane == 0) s_qh[g] = n;
  }
  __syncthreads();
  if (threadIdx.x == 0) s_qn = group_norm(s_qh, G, OC_GROUP_MEDIAN);
  __syncthreads();
  gate_tiles(s_qn, kn + (int64_t)kv * kn_sh, num_tiles, mask_cols, tau_norm, 1, mask + (int64_t)bk * m_sh,
             stats ? stats + (int64_t)bk * 3 : nullptr);
}

bool pf_float_dtype(int dt) { return dt == OC_F32 || dt == OC_F16 || dt == OC_BF16; }

template <int DT, int D>
int launch_prefill(const PrefillArgs& a, hipStream_t s, unsigned blocks) {
  const dim3 grid(blocks), block(kPfThreads);
  if (a.nitems) {
    if (a.entropy) hipLaunchKernelGGL((prefill_kernel<DT, D, true, true>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((prefill_kernel<DT, D, false, true>), grid, block, 0, s, a);
  } else {
    if (a.entropy) hipLaunchKernelGGL((prefill_kernel<DT, D, true, false>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((prefill_kernel<DT, D, false, false>), grid, block, 0, s, a);
  }
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? OC_OK : hip_fail(e, "prefill launch");
}

template <int DT>
int launch_prefill_d(const PrefillArgs& a, int d, hipStream_t s, unsigned blocks) {
  return d == 64 ? launch_prefill<DT, 64>(a, s, blocks) : launch_prefill<DT, 128>(a, s, blocks);
}

// Workgroups of prefill_kernel<DT, D> that one CU holds at once (the
// entropy variant's budget is the same), times the device's CUs.
template <int DT, int D>
int pf_slots_t() {
  static int per_cu[64] = {0};
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (!per_cu[dev]) {
    int n = 0, c = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, prefill_kernel<DT, D, false, false>, kPfThreads, 0) !=
        hipSuccess)
      n = 0;
    if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) c = 0;
    per_cu[dev] = n > 0 ? n : -1;
    cus[dev] = c;
  }
  return per_cu[dev] > 0 ? per_cu[dev] * cus[dev] : 0;
}

int pf_slots(int dtype, int d) {
  switch (dtype) {
    case OC_F32: return d == 64 ? pf_slots_t<OC_F32, 64>() : pf_slots_t<OC_F32, 128>();
    case OC_F16: return d == 64 ? pf_slots_t<OC_F16, 64>() : pf_slots_t<OC_F16, 128>();
    default: return d == 64 ? pf_slots_t<OC_BF16, 64>() : pf_slots_t<OC_BF16, 128>();
  }
}

constexpr size_t kPfCounterBytes = 64 << 10;

// The split of a call's longest causal windows: when the call's workgroups
// fit on the device at once (one round) and no tiles are evicted, its time
// is the longest window's;
// blocks whose window is over half the longest (and at least 4 tiles) then
// run as two workgroups of half the tiles each.  Items are ordered longest
// first (ties: later block first, first half first).  False: no split.
struct PfPlan {
  int nitems = 0, q0 = 0, ctr_stride = 1;
  size_t part_bytes = 0;
  uint16_t items[kPfMaxItems];
};

bool pf_plan(const oc_prefill_params* p, PfPlan* pl) {
  // with evicted tiles the windows' work shrinks and the merge's fixed cost
  // no longer pays (half the tiles evicted, TinyLlama layer, bfloat16: 43
  // unsplit against 47 us split; float32 even)
  if (p->tile_mask) return false;
  const int qblocks = (p->q_len + kPfRows - 1) / kPfRows;
  const int64_t nbh = (int64_t)p->batch * p->num_q_heads;
  if (qblocks < 1 || nbh < 1) return false;
  const int slots = pf_slots(p->dtype, p->head_dim);
  if (slots <= 0 || nbh * qblocks > slots) return false;
  const int off = p->kv_len - p->q_len;
  auto window = [&](int qb) {
    return (std::min(std::max(std::min(qb * kPfRows + kPfRows - 1, p->q_len - 1) + off + 1, 0), p->kv_len) + 63) / 64;
  };
  const int wmax = window(qblocks - 1);
  int q0 = 0;
  while (q0 < qblocks && (2 * window(q0) <= wmax || window(q0) < 4)) ++q0;
  const int nsplit = qblocks - q0;
  if (nsplit == 0 || qblocks + nsplit > kPfMaxItems) return false;
  const int64_t npairs = (int64_t)nsplit * nbh;
  if (npairs * (int64_t)sizeof(int32_t) > (int64_t)kPfCounterBytes) return false;
  pl->ctr_stride = 32;
  while (pl->ctr_stride > 1 && npairs * pl->ctr_stride * (int64_t)sizeof(int32_t) > (int64_t)kPfCounterBytes)
    pl->ctr_stride >>= 1;
  pl->q0 = q0;
  pl->part_bytes = (size_t)npairs * 2 * (4 + p->head_dim / 4) * kPfThreads * sizeof(float);
  struct Item {
    int len, qb, part;
  };
  Item it[kPfMaxItems];
  int n = 0;
  for (int qb = 0; qb < qblocks; ++qb) {
    const int w = window(qb);
    if (qb >= q0) {
      const int ts = (w + 1) / 2;
      it[n++] = {ts, qb, 1};
      it[n++] = {w - ts, qb, 2};
    } else {
      it[n++] = {w, qb, 0};
    }
  }
  std::stable_sort(it, it + n, [](const Item& x, const Item& y) {
    if (x.len != y.len) return x.len > y.len;
    if (x.qb != y.qb) return x.qb > y.qb;
    return x.part < y.part;
  });
  for (int e = 0; e < n; ++e) pl->items[e] = (uint16_t)((it[e].qb << 2) | it[e].part);
  pl->nitems = n;
  return true;
}

}  // namespace
}  // namespace oc

using namespace oc;

extern "C" int oc_prefill_attention(const oc_prefill_params* p, void* stream) {
  if (!p) return fail(OC_ERR_INVALID, "NULL params");
  if (!p->q || !p->k || !p->v || !p->out) return fail(OC_ERR_INVALID, "NULL tensor pointer");
  if (!pf_float_dtype(p->dtype)) return fail(OC_ERR_UNSUPPORTED, "prefill dtype %d (float32, float16, bfloat16)",
                                             p->dtype);
  if (p->head_dim != 64 && p->head_dim != 128) return fail(OC_ERR_UNSUPPORTED, "head_dim %d (64 or 128)", p->head_dim);
  if (p->batch < 0 || p->num_q_heads < 0 || p->num_kv_heads < 1 || p->q_len < 0 || p->kv_len < 0)
    return fail(OC_ERR_INVALID, "bad sizes");
  if (p->num_q_heads % p->num_kv_heads) return fail(OC_ERR_INVALID, "num_q_heads %d not a multiple of num_kv_heads %d",
                                                    p->num_q_heads, p->num_kv_heads);
  const int es = p->dtype == OC_F32 ? 4 : 2;
  // 16-byte vector loads: rows and bases 16-byte aligned
  const int64_t strides[] = {p->q_stride_b, p->q_stride_h, p->q_stride_s, p->k_stride_b, p->k_stride_h,
                             p->k_stride_s, p->v_stride_b, p->v_stride_h, p->v_stride_s};
  for (int64_t st : strides)
    if ((st * es) % 16) return fail(OC_ERR_INVALID, "q/k/v strides must be multiples of 16 bytes");
  if (((uintptr_t)p->q | (uintptr_t)p->k | (uintptr_t)p->v) % 16) return fail(OC_ERR_INVALID, "q/k/v not 16-byte aligned");
  if (p->dtype == OC_F32 && ((uintptr_t)p->out % 16 || (p->out_stride_b * es) % 16 || (p->out_stride_h * es) % 16 ||
                             (p->out_stride_s * es) % 16))
    return fail(OC_ERR_INVALID, "float32 out rows must be 16-byte aligned");
  if (p->k_stride_s * es * 64 > 0x7FFFFFFF || p->v_stride_s * es * 64 > 0x7FFFFFFF)
    return fail(OC_ERR_UNSUPPORTED, "token stride too large");
  if (p->k_stride_s < p->head_dim || p->v_stride_s < p->head_dim)
    return fail(OC_ERR_INVALID, "token stride smaller than head_dim");
  if (p->tile_mask && p->tile_mask_cols < p->kv_len / 64)
    return fail(OC_ERR_INVALID, "tile_mask has %d columns, kv_len needs %d", p->tile_mask_cols, p->kv_len / 64);
  if (p->batch == 0 || p->num_q_heads == 0 || p->q_len == 0) return OC_OK;
  PrefillArgs a{};
  a.q = (const char*)p->q;
  a.k = (const char*)p->k;
  a.v = (const char*)p->v;
  a.out = (char*)p->out;
  a.q_sb = p->q_stride_b * es, a.q_sh = p->q_stride_h * es, a.q_ss = p->q_stride_s * es;
  a.k_sb = p->k_stride_b * es, a.k_sh = p->k_stride_h * es, a.k_ss = p->k_stride_s * es;
  a.v_sb = p->v_stride_b * es, a.v_sh = p->v_stride_h * es, a.v_ss = p->v_stride_s * es;
  a.o_sb = p->out_stride_b * es, a.o_sh = p->out_stride_h * es, a.o_ss = p->out_stride_s * es;
  a.B = p->batch, a.Hq = p->num_q_heads, a.Hkv = p->num_kv_heads, a.G = p->num_q_heads / p->num_kv_heads;
  a.Sq = p->q_len, a.Skv = p->kv_len, a.T = p->kv_len / 64;
  a.mask = p->tile_mask, a.m_sb = p->tile_mask_stride_b, a.m_sh = p->tile_mask_stride_h;
  a.scale = p->scale;
  a.entropy = p->entropy;
  a.qblocks = (p->q_len + kPfRows - 1) / kPfRows;
  a.dtype = p->dtype;
  int64_t items = a.qblocks;
  if (p->workspace) {
    PfPlan pl;
    if (pf_plan(p, &pl)) {
      const size_t need = kPfCounterBytes + pl.part_bytes + 256;
      if (p->workspace_bytes < need)
        return fail(OC_ERR_WORKSPACE, "prefill workspace of %zu bytes needed, %zu given", need, p->workspace_bytes);
      char* w = (char*)(((uintptr_t)p->workspace + 255) & ~(uintptr_t)255);
      a.ctr = (int32_t*)w;
      a.part = (float*)(w + kPfCounterBytes);
      a.nitems = pl.nitems;
      a.q0 = pl.q0;
      a.ctr_stride = pl.ctr_stride;
      std::copy(pl.items, pl.items + pl.nitems, a.items);
      items = pl.nitems;
    }
  }
  const int64_t blocks = items * a.B * a.Hq;
  if (blocks > 0x7FFFFFFF) return fail(OC_ERR_UNSUPPORTED, "too many query blocks");
  const hipStream_t s = (hipStream_t)stream;
  switch (p->dtype) {
    case OC_F32: return launch_prefill_d<OC_F32>(a, p->head_dim, s, (unsigned)blocks);
    case OC_F16: return launch_prefill_d<OC_F16>(a, p->head_dim, s, (unsigned)blocks);
    default: return launch_prefill_d<OC_BF16>(a, p->head_dim, s, (unsigned)blocks);
  }
}

extern "C" size_t oc_prefill_workspace_size(const oc_prefill_params* p) {
  if (!p || !pf_float_dtype(p->dtype) || (p->head_dim != 64 && p->head_dim != 128) || p->batch <= 0 ||
      p->num_q_heads <= 0 || p->q_len <= 0 || p->kv_len < 0)
    return 0;
  PfPlan pl;
  return pf_plan(p, &pl) ? kPfCounterBytes + pl.part_bytes + 256 : 0;
}

extern "C" int oc_row_norms(const void* x, int32_t dtype, int64_t n0, int64_t n1, int64_t n2, int64_t stride0,
                            int64_t stride1, int64_t stride2, int32_t head_dim, int32_t low_band, float* out,
                            void* stream) {
  if (!x || !out) return fail(OC_ERR_INVALID, "NULL pointer");
  if (!pf_float_dtype(dtype)) return fail(OC_ERR_INVALID, "dtype %d", dtype);
  if (n0 < 0 || n1 < 0 || n2 < 0 || head_dim < 1 || head_dim > 1024) return fail(OC_ERR_INVALID, "bad sizes");
  if (low_band < 0 || (low_band > 0 && head_dim % low_band))
    return fail(OC_ERR_INVALID, "head_dim %d not divisible by low_band %d", head_dim, low_band);
  const int64_t rows = n0 * n1 * n2;
  if (rows == 0) return OC_OK;
  const int64_t blocks = (rows + 3) / 4;
  if (blocks > 0x7FFFFFFF) return fail(OC_ERR_UNSUPPORTED, "too many rows");
  const int es = dtype == OC_F32 ? 4 : 2;
  hipLaunchKernelGGL(row_norms_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, (const char*)x,
                     dtype, n0, n1, n2, stride0 * es, stride1 * es, stride2 * es, head_dim, low_band, out);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? OC_OK : hip_fail(e, "row-norm launch");
}

extern "C" int oc_kth_smallest(const float* x, int64_t rows, int64_t n, int64_t row_stride, int64_t k, float* out,
                               void* stream) {
  if (!x || !out) return fail(OC_ERR_INVALID, "NULL pointer");
  if (rows < 0 || n < 1 || k < 0 || k >= n || row_stride < n) return fail(OC_ERR_INVALID, "bad sizes (k must be < n)");
  if (rows > 0x7FFFFFFF) return fail(OC_ERR_UNSUPPORTED, "too many rows");
  if (rows == 0) return OC_OK;
  hipLaunchKernelGGL(kth_smallest_kernel, dim3((unsigned)rows), dim3(256), 0, (hipStream_t)stream, x, n, row_stride,
                     k, out);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? OC_OK : hip_fail(e, "select launch");
}

extern "C" int oc_group_gate(const float* q_norms, int32_t batch, int32_t num_kv_heads, int32_t G, int32_t reduce,
                             const float* k_norms, int64_t k_norms_stride_b, int64_t k_norms_stride_h,
                             int32_t num_tiles, int32_t mask_cols, double tau_norm, int32_t keep_polarity,
                             uint8_t* mask, int64_t mask_stride_b, int64_t mask_stride_h, float* group_norms,
                             float* gate_stats, void* stream) {
  if (!q_norms || !k_norms || !mask) return fail(OC_ERR_INVALID, "NULL pointer");
  if (batch < 0 || num_kv_heads < 0 || G < 1 || num_tiles < 0 || mask_cols < num_tiles)
    return fail(OC_ERR_INVALID, "bad sizes");
  if (reduce != OC_GROUP_MAX && reduce != OC_GROUP_MEDIAN) return fail(OC_ERR_INVALID, "reduce %d", reduce);
  const int64_t wgs = (int64_t)batch * num_kv_heads;
  if (wgs == 0) return OC_OK;
  if (wgs > 0x7FFFFFFF) return fail(OC_ERR_UNSUPPORTED, "too many heads");
  hipLaunchKernelGGL(group_gate_kernel, dim3((unsigned)wgs), dim3(256), 0, (hipStream_t)stream, q_norms,
                     num_kv_heads, G, reduce, k_norms, k_norms_stride_b, k_norms_stride_h, num_tiles, mask_cols,
                     tau_norm, keep_polarity, mask, mask_stride_b, mask_stride_h, group_norms, gate_stats);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? OC_OK : hip_fail(e, "group-gate launch");
}

// The hook decode's gate launch (oc_hook_decode); q_row_stride in elements.
__attribute__((visibility("hidden"))) int oc_internal_hook_gate(
    const void* q, int32_t dtype, int64_t q_row_stride, int32_t batch, int32_t num_kv_heads, int32_t G,
    int32_t head_dim, int32_t low_band, const float* k_norms, int64_t k_norms_stride, int32_t num_tiles,
    int32_t mask_cols, double tau_norm, uint8_t* mask, int64_t mask_stride, float* gate_stats, void* stream) {
  const int64_t wgs = (int64_t)batch * num_kv_heads;
  if (wgs == 0) return OC_OK;
  const int es = dtype == OC_F32 ? 4 : 2;
  hipLaunchKernelGGL(hook_gate_kernel, dim3((unsigned)wgs), dim3(256), 0, (hipStream_t)stream, (const char*)q, dtype,
                     q_row_stride * es, num_kv_heads, G, head_dim, low_band, k_norms, k_norms_stride, num_tiles,
                     mask_cols, tau_norm, mask, mask_stride, gate_stats);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? OC_OK : hip_fail(e, "hook-gate launch");
}

extern "C" size_t oc_prefill_params_bytes(void) { return sizeof(oc_prefill_params); }
