// Device-side kernels of liborthocache_hip: tile scoring (64-point Walsh-
// Hadamard transform along the token axis), gated split-K flash-decode and
// the log-sum-exp merge, written for gfx950 (CDNA4, wave64).
//
// Wavefront layout of one 64-token tile (all dtypes, head_dim D = 16*CPL):
//   lane  = 16*gamma + j            (gamma = 0..3, j = 0..15)
//   token = 4*i + gamma             (i = 0..15, one "register row" per i)
//   dims  = CPL*j .. CPL*j + CPL-1  (CPL = D/16 consecutive elements)
// One load instruction of the wave therefore covers 4 whole token rows
// (64 lanes x CPL elements), so every global load is fully coalesced.
// Token bits t2..t5 live in the register index i, t0..t1 in the lane bits
// 4..5.  The 16 lanes that share a token row form one DPP row, so the
// q.k reduction and the p broadcast stay inside DPP rows.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "orthocache_hip.h"

namespace oc {

constexpr int kWave = 64;
constexpr int kWaves = 4;
constexpr int kThreads = kWave * kWaves;
constexpr float kM0 = -1e9f;

// Kernel arguments (byte strides).  Built by oc_api.hip from oc_decode_params.
struct DecodeArgs {
  const char* k;
  const char* v;
  int64_t k_row_stride, k_tok_stride, v_row_stride, v_tok_stride;
  int32_t paged, bs_log2, nkv, rows_per_length;
  const int32_t* bt;
  int64_t bt_stride, num_blocks;
  int64_t k_blk_stride, k_head_stride, v_blk_stride, v_head_stride;
  const int32_t* lengths;
  int32_t num_rows, num_tiles;
  int32_t k_scale_mode, v_scale_mode;
  float k_scale;
  int32_t q_dtype;
  const float* k_scales;
  int64_t ks_stride;
  const float* v_scales;
  int64_t vs_stride;
  int32_t* error_flag;
  const char* q;
  int64_t q_row_stride;
  int32_t G;
  int32_t gate, mode;
  double thr;
  const float* sc_el;
  const float* sc_eh;
  int64_t sc_stride;
  int32_t P;
  float* pm;
  float* pl;
  float* pacc;
  uint8_t* keep_out;
  int64_t keep_stride;
  int32_t* split_counts;
  float scale;
  // score kernel outputs
  float* o_el;
  float* o_eh;
  float* o_z;
  uint8_t* o_keep;
  int64_t o_stride;
  float* o_fwht;
};

template <int DT>
struct Elem {
  static constexpr int size = DT == OC_F32 ? 4 : (DT == OC_FP8_E4M3FN ? 1 : 2);
};

template <int DT, int D>
struct Lay {
  static constexpr int CPL = D / 16;               // columns per lane
  static constexpr int NI = 16;                    // register rows per lane
  static constexpr int LB = CPL * Elem<DT>::size;  // bytes per lane per register row
  static constexpr int LW = LB / 4;                // 32-bit words
  static_assert(LB >= 4 && LB <= 32, "unsupported lane width");
};

// ---------------------------------------------------------------- lane ops

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xF, 0xF, true));
}

// Partner exchange inside a 16-lane DPP row: M=8 pairs lane k with 15-k
// (row_mirror), M=4 with k^7 (row_half_mirror), M=2 and M=1 with k^2 and
// k^1 (quad_perm).  Each pairing flips bit log2(M) of the lane index, which
// is all a butterfly needs.  M >= 16 crosses DPP rows.
template <int M>
__device__ __forceinline__ float xpair(float x) {
  if constexpr (M == 8) return dpp<0x140>(x);
  else if constexpr (M == 4) return dpp<0x141>(x);
  else if constexpr (M == 2) return dpp<0x4E>(x);
  else if constexpr (M == 1) return dpp<0xB1>(x);
  else return __shfl_xor(x, M, kWave);
}

// value of lane 16*gamma + I for every lane of DPP row gamma (row_newbcast)
template <int I>
__device__ __forceinline__ float row_bcast(float x) {
  return dpp<0x150 + I>(x);
}

__device__ __forceinline__ float wave_sum(float x) {
  x += xpair<8>(x);
  x += xpair<4>(x);
  x += xpair<2>(x);
  x += xpair<1>(x);
  x += xpair<16>(x);
  x += xpair<32>(x);
  return x;
}

__device__ __forceinline__ float wave_max(float x) {
  x = fmaxf(x, xpair<8>(x));
  x = fmaxf(x, xpair<4>(x));
  x = fmaxf(x, xpair<2>(x));
  x = fmaxf(x, xpair<1>(x));
  x = fmaxf(x, xpair<16>(x));
  x = fmaxf(x, xpair<32>(x));
  return x;
}

// One transpose-reduce step: the lane keeps half of its n = 2M values (the
// upper half if lane bit log2(M) is set) and adds its partner's copy of
// that half.
template <int M, int N>
__device__ __forceinline__ void tr_step(float (&v)[N], int lane) {
  const bool up = (lane & M) != 0;
#pragma unroll
  for (int k = 0; k < M; ++k) {
    const float keep = up ? v[k + M] : v[k];
    const float send = up ? v[k] : v[k + M];
    v[k] = keep + xpair<M>(send);
  }
}

// v[i] (i = 0..15) are partial dot products of token 4i+gamma over the
// lane's columns.  Returns, in lane 16*gamma + j, the full dot product of
// token 4j+gamma (15 DPP adds instead of 64 for a full all-reduce).
__device__ __forceinline__ float transpose_reduce16(float (&v)[16], int lane) {
  tr_step<8>(v, lane);
  tr_step<4>(v, lane);
  tr_step<2>(v, lane);
  tr_step<1>(v, lane);
  return v[0];
}

// ---------------------------------------------------------------- elements

template <int LB>
__device__ __forceinline__ void load_lane_row(const char* p, uint32_t* w) {
  if constexpr (LB == 32) {
    const uint4 a = *reinterpret_cast<const uint4*>(p);
    const uint4 b = *reinterpret_cast<const uint4*>(p + 16);
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
    w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
  } else if constexpr (LB == 16) {
    const uint4 a = *reinterpret_cast<const uint4*>(p);
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
  } else if constexpr (LB == 8) {
    const uint2 a = *reinterpret_cast<const uint2*>(p);
    w[0] = a.x; w[1] = a.y;
  } else {
    w[0] = *reinterpret_cast<const uint32_t*>(p);
  }
}

template <int DT>
__device__ __forceinline__ float elem(const uint32_t* w, int c) {
  if constexpr (DT == OC_F32) {
    return __uint_as_float(w[c]);
  } else if constexpr (DT == OC_BF16) {
    const uint32_t x = w[c >> 1];
    return (c & 1) ? __uint_as_float(x & 0xFFFF0000u) : __uint_as_float(x << 16);
  } else if constexpr (DT == OC_F16) {
    const uint32_t x = w[c >> 1];
    const uint16_t h = (c & 1) ? (uint16_t)(x >> 16) : (uint16_t)(x & 0xFFFFu);
    return (float)__builtin_bit_cast(_Float16, h);
  } else {
    const int x = (int)w[c >> 2];
    if ((c >> 1) & 1) {
      const auto f = __builtin_amdgcn_cvt_pk_f32_fp8(x, true);
      return (c & 1) ? f[1] : f[0];
    } else {
      const auto f = __builtin_amdgcn_cvt_pk_f32_fp8(x, false);
      return (c & 1) ? f[1] : f[0];
    }
  }
}

// float32 -> nearest bf16 / f16 value (ties to even), returned as float32
__device__ __forceinline__ float round_bf16(float x) {
  uint32_t u = __float_as_uint(x);
  if ((u & 0x7F800000u) == 0x7F800000u) return x;  // inf / nan unchanged
  u += 0x7FFFu + ((u >> 16) & 1u);
  return __uint_as_float(u & 0xFFFF0000u);
}
__device__ __forceinline__ float round_f16(float x) { return (float)(_Float16)x; }

__device__ __forceinline__ float round_to(float x, int dtype) {
  if (dtype == OC_BF16) return round_bf16(x);
  if (dtype == OC_F16) return round_f16(x);
  return x;
}

__device__ __forceinline__ float load_scalar(const char* p, int dtype) {
  if (dtype == OC_F32) return *reinterpret_cast<const float*>(p);
  const uint16_t h = *reinterpret_cast<const uint16_t*>(p);
  if (dtype == OC_BF16) return __uint_as_float((uint32_t)h << 16);
  return (float)__builtin_bit_cast(_Float16, h);
}

__device__ __forceinline__ void store_scalar(char* p, int dtype, float x) {
  if (dtype == OC_F32) {
    *reinterpret_cast<float*>(p) = x;
  } else if (dtype == OC_BF16) {
    *reinterpret_cast<uint16_t*>(p) = (uint16_t)(__float_as_uint(round_bf16(x)) >> 16);
  } else {
    *reinterpret_cast<uint16_t*>(p) = __builtin_bit_cast(uint16_t, (_Float16)x);
  }
}

// ---------------------------------------------------------------- addressing

struct RowInfo {
  int n_tok;       // tokens of this row
  int n_tiles;     // ceil(n_tok / 64)
  int seq, head;   // paged: sequence and kv head of the row
};

__device__ __forceinline__ RowInfo row_info(const DecodeArgs& a, int row) {
  RowInfo ri;
  int n = a.num_tiles * 64;
  if (a.lengths) {
    const int len = a.lengths[row / a.rows_per_length];
    n = len < 0 ? 0 : (len < n ? len : n);
  }
  ri.n_tok = n;
  ri.n_tiles = (n + 63) >> 6;
  if (a.paged) {
    ri.seq = row / a.nkv;
    ri.head = row - ri.seq * a.nkv;
  } else {
    ri.seq = row;
    ri.head = 0;
  }
  return ri;
}

// Loads one tile (K or V) of `row` into w[i][*] for this lane.  Register
// rows whose first token is at or past n_tok are zero-filled without a
// load; a paged block id outside the pool raises error_flag and reads zeros.
template <int DT, int D>
__device__ __forceinline__ void load_tile(const DecodeArgs& a, const RowInfo& ri, int row, int t,
                                          bool is_v, int lane, uint32_t (&w)[16][Lay<DT, D>::LW]) {
  using L = Lay<DT, D>;
  const int gamma = lane >> 4;
  const int j = lane & 15;
  const int64_t lane_off = (int64_t)j * L::LB;
  const int tok0 = t * 64;
  if (!a.paged) {
    const char* base = (is_v ? a.v : a.k) + (int64_t)row * (is_v ? a.v_row_stride : a.k_row_stride);
    const int64_t ts = is_v ? a.v_tok_stride : a.k_tok_stride;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if (tok0 + 4 * i < ri.n_tok) {
        load_lane_row<L::LB>(base + (int64_t)(tok0 + 4 * i + gamma) * ts + lane_off, w[i]);
      } else {
#pragma unroll
        for (int x = 0; x < L::LW; ++x) w[i][x] = 0u;
      }
    }
  } else {
    const char* base = is_v ? a.v : a.k;
    const int64_t bstride = is_v ? a.v_blk_stride : a.k_blk_stride;
    const int64_t hoff = (int64_t)ri.head * (is_v ? a.v_head_stride : a.k_head_stride);
    const int64_t ts = is_v ? a.v_tok_stride : a.k_tok_stride;
    const int32_t* btrow = a.bt + (int64_t)ri.seq * a.bt_stride;
    const int bmask = (1 << a.bs_log2) - 1;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int tok = tok0 + 4 * i;  // uniform; block_size >= 4 keeps tok..tok+3 in one block
      bool ok = tok < ri.n_tok;
      int64_t blk = 0;
      if (ok) {
        blk = btrow[tok >> a.bs_log2];
        if (blk < 0 || blk >= a.num_blocks) {
          if (a.error_flag && lane == 0) atomicOr(a.error_flag, 1);
          ok = false;
        }
      }
      if (ok) {
        load_lane_row<L::LB>(base + blk * bstride + hoff + (int64_t)((tok & bmask) + gamma) * ts + lane_off,
                             w[i]);
      } else {
#pragma unroll
        for (int x = 0; x < L::LW; ++x) w[i][x] = 0u;
      }
    }
  }
}

// Dequantisation of one tile: value = round_to(float(elem) * mul, rnd) when
// `scaled`, float(elem) otherwise.
struct Deq {
  float mul;
  int rnd;
  bool scaled;
};

// The CPL values of one register row of this lane as float32.
template <int DT, int D>
__device__ __forceinline__ void row_vals(const uint32_t* w, float (&f)[D / 16], const Deq& dq) {
#pragma unroll
  for (int c = 0; c < D / 16; ++c) f[c] = elem<DT>(w, c);
  if (dq.scaled) {
#pragma unroll
    for (int c = 0; c < D / 16; ++c) f[c] = round_to(f[c] * dq.mul, dq.rnd);
  }
}

// Whole tile as float32 (used by the full-transform kernel).
template <int DT, int D>
__device__ __forceinline__ void decode_tile(const uint32_t (&w)[16][Lay<DT, D>::LW],
                                            float (&f)[16][Lay<DT, D>::CPL], const Deq& dq) {
#pragma unroll
  for (int i = 0; i < 16; ++i) row_vals<DT, D>(w[i], f[i], dq);
}

// ---------------------------------------------------------------- tile score

// Band energies of the 64-point Walsh-Hadamard transform along the token
// axis, X = W64 @ K_tile with W64[s,t] = (-1)^popcount(s&t) / 8 (natural
// order), summed over head_dim:
//   E_low  = sum_{s=1..7}  sum_c X[s,c]^2
//   E_high = sum_{s=32..63} sum_c X[s,c]^2
// The transform is evaluated only where the bands need it:
//  * rows 32..63 are the difference branch of the first butterfly stage
//    (token bit t5: pairs u, u+32, i.e. register rows i, i+8) followed by a
//    32-point transform that is orthogonal up to the 1/8 scale; its output
//    energy is therefore (1/64)*32*sum d^2 = 1/2 sum_{u<32} |k_u - k_{u+32}|^2
//    (Parseval);
//  * rows 0..7 only see the sum branches of stages t5, t4, t3, i.e. the
//    residue sums S_r = sum_{t = r mod 8} k_t, followed by the full 8-point
//    butterfly over t0..t2 (t2 in registers, t0 and t1 across lanes).
// The summation order is fixed, so every kernel that calls this function
// (scoring, single-pass decode) produces the same bits.
template <int DT, int D>
__device__ __forceinline__ void tile_energies(const uint32_t (&kw)[16][Lay<DT, D>::LW], const Deq& dq,
                                              int lane, float& e_low, float& e_high) {
  constexpr int CPL = D / 16;
  float h = 0.f;
  float s0[CPL], s1[CPL];  // residue sums for token parity t2 = 0 / 1
#pragma unroll
  for (int c = 0; c < CPL; ++c) s0[c] = s1[c] = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float fa[CPL], fb[CPL];
    row_vals<DT, D>(kw[i], fa, dq);
    row_vals<DT, D>(kw[i + 8], fb, dq);
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const float d = fa[c] - fb[c];
      h = __builtin_fmaf(d, d, h);
      if (i & 1) {
        s1[c] += fa[c];
        s1[c] += fb[c];
      } else {
        s0[c] += fa[c];
        s0[c] += fb[c];
      }
    }
  }
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    // butterfly on t2 (register parity)
    const float a0 = s0[c], a1 = s1[c];
    s0[c] = a0 + a1;
    s1[c] = a0 - a1;
    // butterflies on t0 (lane bit 4) and t1 (lane bit 5)
    {
      const float y0 = xpair<16>(s0[c]), y1 = xpair<16>(s1[c]);
      const bool up = (lane & 16) != 0;
      s0[c] = up ? (y0 - s0[c]) : (s0[c] + y0);
      s1[c] = up ? (y1 - s1[c]) : (s1[c] + y1);
    }
    {
      const float y0 = xpair<32>(s0[c]), y1 = xpair<32>(s1[c]);
      const bool up = (lane & 32) != 0;
      s0[c] = up ? (y0 - s0[c]) : (s0[c] + y0);
      s1[c] = up ? (y1 - s1[c]) : (s1[c] + y1);
    }
  }
  // lane holds X rows s = gamma (s0) and 4 + gamma (s1); skip the DC row
  float lo = 0.f;
  const bool dc_lane = (lane >> 4) == 0;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const float x0 = s0[c] * 0.125f;
    const float x1 = s1[c] * 0.125f;
    lo = dc_lane ? lo : __builtin_fmaf(x0, x0, lo);
    lo = __builtin_fmaf(x1, x1, lo);
  }
  e_low = wave_sum(lo);
  e_high = wave_sum(h) * 0.5f;
}

// Gate decision from a tile's band energies; true = retain.
//   zeta gate (fused_eviction.py:428-432): evict iff e_high/(e_low+1e-6) > zeta_max
//   CS gate (gqa_eviction.py:222-239): evict iff max_g ||q_g|| * ||X_high||_F <= tau,
//   with norms below 1e-38 clamped to 0; qmax = max_g ||q_g|| (fl(q*k) is
//   monotone in q for k >= 0, so max_g fl(q_g*k) = fl(qmax*k)).
__device__ __forceinline__ bool gate_keep(int gate, double thr, float e_low, float e_high,
                                          float qmax, bool qnan) {
  if (gate == OC_GATE_ZETA) {
    const float z = e_high / (e_low + 1e-6f);
    return !((double)z > thr);
  }
  if (gate == OC_GATE_CS) {
    float kn = __builtin_sqrtf(e_high);
    if ((double)kn < 1e-38) kn = 0.f;
    const float cs = qmax * kn;
    if (qnan || __builtin_isnan(cs)) return true;
    return !((double)cs <= thr);
  }
  return true;
}

// ---------------------------------------------------------------- decode

template <int DT, int D, int GT>
struct WaveState {
  static constexpr int CPL = Lay<DT, D>::CPL;
  float q[GT][CPL];
  float m[GT];
  float l[GT];      // per-lane partial sums
  float acc[GT][CPL];
};

// Online-softmax update of the wave's G states with one retained tile
// (fused_eviction.py:280-299 per head; gqa_eviction.py:409-451 per g).
// Token rows are processed in pairs (i, i+8) so that the first step of the
// transpose-reduce happens before the next pair is decoded.
template <int DT, int D, int GT>
__device__ __forceinline__ void attend_tile(WaveState<DT, D, GT>& st,
                                            const uint32_t (&kw)[16][Lay<DT, D>::LW], const Deq& kdq,
                                            const uint32_t (&vw)[16][Lay<DT, D>::LW], const Deq& vdq,
                                            int g_active, float scale, int valid, int lane) {
  constexpr int CPL = D / 16;
  float red[GT][8];
  const bool up8 = (lane & 8) != 0;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    float fa[CPL], fb[CPL];
    row_vals<DT, D>(kw[k], fa, kdq);
    row_vals<DT, D>(kw[k + 8], fb, kdq);
#pragma unroll
    for (int g = 0; g < GT; ++g) {
      float da = fa[0] * st.q[g][0];
      float db = fb[0] * st.q[g][0];
#pragma unroll
      for (int c = 1; c < CPL; ++c) {
        da = __builtin_fmaf(fa[c], st.q[g][c], da);
        db = __builtin_fmaf(fb[c], st.q[g][c], db);
      }
      const float keep = up8 ? db : da;
      const float send = up8 ? da : db;
      red[g][k] = keep + xpair<8>(send);
    }
  }
  float p[GT];
#pragma unroll
  for (int g = 0; g < GT; ++g) {
    tr_step<4>(red[g], lane);
    tr_step<2>(red[g], lane);
    tr_step<1>(red[g], lane);
    // lane 16*gamma + j holds token 4j + gamma
    float logit = red[g][0] * scale;
    if (valid < 64) {
      const int tok = 4 * (lane & 15) + (lane >> 4);
      if (tok >= valid) logit = -__builtin_inff();
    }
    if (g >= g_active) {
      p[g] = 0.f;
      continue;
    }
    const float mt = wave_max(logit);
    const float mn = fmaxf(st.m[g], mt);
    const float alpha = __expf(st.m[g] - mn);
    const float pg = __expf(logit - mn);
    st.l[g] = __builtin_fmaf(st.l[g], alpha, pg);
    st.m[g] = mn;
    p[g] = pg;
#pragma unroll
    for (int c = 0; c < CPL; ++c) st.acc[g][c] *= alpha;
  }
  // acc[g][c] += sum_i p(token 4i+gamma) * v[i][c]; p of that token sits
  // in lane 16*gamma + i of the same DPP row.
#define OC_PV_STEP(I)                                                        \
  {                                                                          \
    float fv[CPL];                                                           \
    row_vals<DT, D>(vw[I], fv, vdq);                                         \
    _Pragma("unroll") for (int g = 0; g < GT; ++g) {                         \
      const float pb = row_bcast<I>(p[g]);                                   \
      _Pragma("unroll") for (int c = 0; c < CPL; ++c) st.acc[g][c] =         \
          __builtin_fmaf(pb, fv[c], st.acc[g][c]);                           \
    }                                                                        \
  }
  OC_PV_STEP(0) OC_PV_STEP(1) OC_PV_STEP(2) OC_PV_STEP(3)
  OC_PV_STEP(4) OC_PV_STEP(5) OC_PV_STEP(6) OC_PV_STEP(7)
  OC_PV_STEP(8) OC_PV_STEP(9) OC_PV_STEP(10) OC_PV_STEP(11)
  OC_PV_STEP(12) OC_PV_STEP(13) OC_PV_STEP(14) OC_PV_STEP(15)
#undef OC_PV_STEP
}

__device__ __forceinline__ Deq tile_kdeq(const DecodeArgs& a, int row, int t) {
  if (a.k_scale_mode == OC_KSCALE_ELEM_QDTYPE) return Deq{a.k_scale, a.q_dtype, true};
  if (a.k_scale_mode == OC_KSCALE_TILE) return Deq{a.k_scales[(int64_t)row * a.ks_stride + t], OC_F32, true};
  return Deq{1.f, OC_F32, false};
}

__device__ __forceinline__ Deq tile_vdeq(const DecodeArgs& a, int row, int t) {
  if (a.v_scale_mode == OC_VSCALE_TILE) return Deq{a.v_scales[(int64_t)row * a.vs_stride + t], OC_F32, true};
  return Deq{1.f, OC_F32, false};
}

// Retain decision for tile t of a row in cached mode (scores precomputed by
// the scoring kernel).  A partial tail tile is always retained.
__device__ __forceinline__ bool cached_keep(const DecodeArgs& a, const RowInfo& ri, int row, int t,
                                            float qmax, bool qnan) {
  if ((t + 1) * 64 > ri.n_tok || a.gate == OC_GATE_NONE) return true;
  const int64_t o = (int64_t)row * a.sc_stride + t;
  const float el = a.gate == OC_GATE_ZETA ? a.sc_el[o] : 0.f;
  return gate_keep(a.gate, a.thr, el, a.sc_eh[o], qmax, qnan);
}

// Main decode kernel.  grid = (P, num_rows, ceil(G / GT)); block = 4 waves.
// Workgroup (s, row, chunk) forms the online-softmax state of query heads
// [chunk*GT, chunk*GT + GT) over the retained tiles {s + kP} of the row:
// the four waves take those tiles round-robin (single-pass) or take the
// retained ones round-robin (cached), and their states are merged in LDS
// into the split's partial (m, l, acc).
template <int DT, int D, int GT>
__global__ __launch_bounds__(kThreads) void decode_kernel(const DecodeArgs a) {
  constexpr int CPL = D / 16;
  using L = Lay<DT, D>;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int s = blockIdx.x;
  const int row = blockIdx.y;
  const int g0 = blockIdx.z * GT;
  const int g_active = min(GT, a.G - g0);
  const RowInfo ri = row_info(a, row);
  const int j = lane & 15;

  __shared__ float sh_m[kWaves][GT];
  __shared__ float sh_l[kWaves][GT];
  __shared__ float sh_acc[kWaves][GT][D];
  __shared__ int sh_cnt[kWaves];

  WaveState<DT, D, GT> st;
  // q rows of this chunk (q := round(q * k_scale) for the Q_FOLD mode)
  const float qmul = a.k_scale_mode == OC_KSCALE_Q_FOLD ? a.k_scale : 1.f;
#pragma unroll
  for (int g = 0; g < GT; ++g) {
    st.m[g] = kM0;
    st.l[g] = 0.f;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      st.acc[g][c] = 0.f;
      float x = 0.f;
      if (g < g_active) {
        const char* qp = a.q + (int64_t)(row * a.G + g0 + g) * a.q_row_stride +
                         (int64_t)(j * CPL + c) * (a.q_dtype == OC_F32 ? 4 : 2);
        x = load_scalar(qp, a.q_dtype);
        if (a.k_scale_mode == OC_KSCALE_Q_FOLD) x = round_to(x * qmul, a.q_dtype);
      }
      st.q[g][c] = x;
    }
  }
  // max_g ||q_g|| over all G query heads of the row (CS gate)
  float qmax = 0.f;
  bool qnan = false;
  if (a.gate == OC_GATE_CS) {
    for (int g = 0; g < a.G; ++g) {
      float ss = 0.f;
      if (lane < 16) {
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
          const char* qp = a.q + (int64_t)(row * a.G + g) * a.q_row_stride +
                           (int64_t)(j * CPL + c) * (a.q_dtype == OC_F32 ? 4 : 2);
          float x = load_scalar(qp, a.q_dtype);
          if (a.k_scale_mode == OC_KSCALE_Q_FOLD) x = round_to(x * qmul, a.q_dtype);
          ss = __builtin_fmaf(x, x, ss);
        }
      }
      float qn = __builtin_sqrtf(wave_sum(ss));
      if ((double)qn < 1e-38) qn = 0.f;
      if (__builtin_isnan(qn)) qnan = true;
      qmax = fmaxf(qmax, qn);
    }
  }

  const int n_split = s < ri.n_tiles ? (ri.n_tiles - s + a.P - 1) / a.P : 0;
  int kept = 0;
  uint32_t kw[16][L::LW];
  uint32_t vw[16][L::LW];

  if (a.mode == OC_MODE_SINGLE_PASS || a.gate == OC_GATE_NONE) {
    for (int kk = wave; kk < n_split; kk += kWaves) {
      const int t = s + kk * a.P;
      const int valid = min(64, ri.n_tok - t * 64);
      load_tile<DT, D>(a, ri, row, t, false, lane, kw);
      const Deq kdq = tile_kdeq(a, row, t);
      bool keep = true;
      if (a.gate != OC_GATE_NONE && valid == 64) {
        float el, eh;
        tile_energies<DT, D>(kw, kdq, lane, el, eh);
        keep = gate_keep(a.gate, a.thr, el, eh, qmax, qnan);
      }
      if (a.keep_out && lane == 0 && blockIdx.z == 0)
        a.keep_out[(int64_t)row * a.keep_stride + t] = keep ? 1 : 0;
      if (keep) {
        ++kept;
        load_tile<DT, D>(a, ri, row, t, true, lane, vw);
        attend_tile<DT, D, GT>(st, kw, kdq, vw, tile_vdeq(a, row, t), g_active, a.scale, valid, lane);
      }
    }
  } else {
    // cached scores: find the retained tiles of the split, 64 at a time
    int base_rank = 0;
    for (int c0 = 0; c0 < n_split; c0 += 64) {
      const int kk = c0 + lane;
      const int t = s + kk * a.P;
      const bool in = kk < n_split;
      const bool keep = in && cached_keep(a, ri, row, t, qmax, qnan);
      if (a.keep_out && in && wave == 0 && blockIdx.z == 0)
        a.keep_out[(int64_t)row * a.keep_stride + t] = keep ? 1 : 0;
      uint64_t mask = __ballot(keep);
      int rank = base_rank;
      base_rank += __popcll(mask);
      while (mask) {
        const int bit = __ffsll((unsigned long long)mask) - 1;
        mask &= mask - 1;
        if ((rank++ & (kWaves - 1)) != wave) continue;
        const int tt = s + (c0 + bit) * a.P;
        const int valid = min(64, ri.n_tok - tt * 64);
        load_tile<DT, D>(a, ri, row, tt, false, lane, kw);
        load_tile<DT, D>(a, ri, row, tt, true, lane, vw);
        ++kept;
        attend_tile<DT, D, GT>(st, kw, tile_kdeq(a, row, tt), vw, tile_vdeq(a, row, tt), g_active, a.scale,
                               valid, lane);
      }
    }
  }

  // wave -> LDS: l summed over lanes, acc summed over the 4 token groups
#pragma unroll
  for (int g = 0; g < GT; ++g) {
    const float lt = wave_sum(st.l[g]);
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      float x = st.acc[g][c];
      x += xpair<16>(x);
      x += xpair<32>(x);
      if (lane < 16) sh_acc[wave][g][j * CPL + c] = x;
    }
    if (lane == 0) {
      sh_m[wave][g] = st.m[g];
      sh_l[wave][g] = lt;
    }
  }
  if (lane == 0) sh_cnt[wave] = kept;
  __syncthreads();

  // merge the four wave states into the split's partial
  for (int idx = threadIdx.x; idx < g_active * D; idx += kThreads) {
    const int g = idx / D;
    const int c = idx - g * D;
    float mx = sh_m[0][g];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) mx = fmaxf(mx, sh_m[w][g]);
    float acc = 0.f, l = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float e = __expf(sh_m[w][g] - mx);
      acc = __builtin_fmaf(sh_acc[w][g][c], e, acc);
      l = __builtin_fmaf(sh_l[w][g], e, l);
    }
    const int64_t qh = (int64_t)row * a.G + g0 + g;
    a.pacc[(qh * a.P + s) * D + c] = acc;
    if (c == 0) {
      a.pm[qh * a.P + s] = mx;
      a.pl[qh * a.P + s] = l;
    }
  }
  if (a.split_counts && threadIdx.x == 0 && blockIdx.z == 0)
    a.split_counts[(int64_t)row * a.P + s] = sh_cnt[0] + sh_cnt[1] + sh_cnt[2] + sh_cnt[3];
}

// Tile scoring: one wave per (row, tile); block = 4 waves.
template <int DT, int D>
__global__ __launch_bounds__(kThreads) void score_kernel(const DecodeArgs a) {
  constexpr int CPL = D / 16;
  using L = Lay<DT, D>;
  const int lane = threadIdx.x & 63;
  const int64_t job = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (job >= (int64_t)a.num_rows * a.num_tiles) return;
  const int row = (int)(job / a.num_tiles);
  const int t = (int)(job - (int64_t)row * a.num_tiles);
  const RowInfo ri = row_info(a, row);
  const int64_t o = (int64_t)row * a.o_stride + t;
  float el = 0.f, eh = 0.f, z = 0.f;
  uint8_t keep = 0;
  if ((t + 1) * 64 <= ri.n_tok) {
    uint32_t kw[16][L::LW];
    load_tile<DT, D>(a, ri, row, t, false, lane, kw);
    tile_energies<DT, D>(kw, tile_kdeq(a, row, t), lane, el, eh);
    z = eh / (el + 1e-6f);
    keep = gate_keep(OC_GATE_ZETA, a.thr, el, eh, 0.f, false) ? 1 : 0;
  } else if (t < ri.n_tiles) {
    keep = 1;
  }
  if (lane == 0) {
    if (a.o_el) a.o_el[o] = el;
    if (a.o_eh) a.o_eh[o] = eh;
    if (a.o_z) a.o_z[o] = z;
    if (a.o_keep) a.o_keep[o] = keep;
  }
}

// Full 64-point transform X = W64 @ K_tile of every tile (float32 out):
// in-register butterflies over token bits t2..t5, cross-lane over t0, t1.
template <int DT, int D>
__global__ __launch_bounds__(kThreads) void fwht_kernel(const DecodeArgs a) {
  constexpr int CPL = D / 16;
  using L = Lay<DT, D>;
  const int lane = threadIdx.x & 63;
  const int64_t job = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (job >= (int64_t)a.num_rows * a.num_tiles) return;
  const int row = (int)(job / a.num_tiles);
  const int t = (int)(job - (int64_t)row * a.num_tiles);
  RowInfo ri = row_info(a, row);
  ri.n_tok = a.num_tiles * 64;  // the transform covers whole tiles
  uint32_t kw[16][L::LW];
  float f[16][CPL];
  load_tile<DT, D>(a, ri, row, t, false, lane, kw);
  decode_tile<DT, D>(kw, f, tile_kdeq(a, row, t));
#pragma unroll
  for (int h = 1; h < 16; h <<= 1) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if (i & h) continue;
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        const float x = f[i][c], y = f[i + h][c];
        f[i][c] = x + y;
        f[i + h][c] = x - y;
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) {
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      float x = f[i][c];
      float y = xpair<16>(x);
      x = (lane & 16) ? (y - x) : (x + y);
      y = xpair<32>(x);
      x = (lane & 32) ? (y - x) : (x + y);
      f[i][c] = x * 0.125f;
    }
  }
  const int gamma = lane >> 4, j = lane & 15;
  float* out = a.o_fwht + ((int64_t)row * a.num_tiles + t) * 64 * D;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
#pragma unroll
    for (int c = 0; c < CPL; ++c) out[(int64_t)(4 * i + gamma) * D + j * CPL + c] = f[i][c];
  }
}

// Launchers instantiated per element type (oc_kernels_<dtype>.hip).
template <int DT>
hipError_t launch_decode(const DecodeArgs& a, int head_dim, int gt, int gchunks, hipStream_t st);
template <int DT>
hipError_t launch_score(const DecodeArgs& a, int head_dim, hipStream_t st);
template <int DT>
hipError_t launch_fwht(const DecodeArgs& a, int head_dim, hipStream_t st);

#define OC_DEFINE_LAUNCHERS(DT)                                                                   \
  template <>                                                                                     \
  hipError_t launch_decode<DT>(const DecodeArgs& a, int head_dim, int gt, int gchunks,            \
                               hipStream_t st) {                                                  \
    const dim3 grid(a.P, a.num_rows, gchunks), block(kThreads);                                   \
    if (head_dim == 128) {                                                                        \
      switch (gt) {                                                                               \
        case 1: hipLaunchKernelGGL((decode_kernel<DT, 128, 1>), grid, block, 0, st, a); break;    \
        case 2: hipLaunchKernelGGL((decode_kernel<DT, 128, 2>), grid, block, 0, st, a); break;    \
        case 4: hipLaunchKernelGGL((decode_kernel<DT, 128, 4>), grid, block, 0, st, a); break;    \
        default: hipLaunchKernelGGL((decode_kernel<DT, 128, 8>), grid, block, 0, st, a); break;   \
      }                                                                                           \
    } else {                                                                                      \
      switch (gt) {                                                                               \
        case 1: hipLaunchKernelGGL((decode_kernel<DT, 64, 1>), grid, block, 0, st, a); break;     \
        case 2: hipLaunchKernelGGL((decode_kernel<DT, 64, 2>), grid, block, 0, st, a); break;     \
        case 4: hipLaunchKernelGGL((decode_kernel<DT, 64, 4>), grid, block, 0, st, a); break;     \
        default: hipLaunchKernelGGL((decode_kernel<DT, 64, 8>), grid, block, 0, st, a); break;    \
      }                                                                                           \
    }                                                                                             \
    return hipGetLastError();                                                                     \
  }                                                                                               \
  template <>                                                                                     \
  hipError_t launch_score<DT>(const DecodeArgs& a, int head_dim, hipStream_t st) {                \
    const int64_t jobs = (int64_t)a.num_rows * a.num_tiles;                                       \
    const dim3 grid((unsigned)((jobs + kWaves - 1) / kWaves)), block(kThreads);                   \
    if (head_dim == 128) hipLaunchKernelGGL((score_kernel<DT, 128>), grid, block, 0, st, a);      \
    else hipLaunchKernelGGL((score_kernel<DT, 64>), grid, block, 0, st, a);                       \
    return hipGetLastError();                                                                     \
  }                                                                                               \
  template <>                                                                                     \
  hipError_t launch_fwht<DT>(const DecodeArgs& a, int head_dim, hipStream_t st) {                 \
    const int64_t jobs = (int64_t)a.num_rows * a.num_tiles;                                       \
    const dim3 grid((unsigned)((jobs + kWaves - 1) / kWaves)), block(kThreads);                   \
    if (head_dim == 128) hipLaunchKernelGGL((fwht_kernel<DT, 128>), grid, block, 0, st, a);       \
    else hipLaunchKernelGGL((fwht_kernel<DT, 64>), grid, block, 0, st, a);                        \
    return hipGetLastError();                                                                     \
  }

}  // namespace oc
