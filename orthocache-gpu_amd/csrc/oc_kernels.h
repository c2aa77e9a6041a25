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

#include <type_traits>

#include "orthocache_hip.h"

namespace oc {

constexpr int kWave = 64;
constexpr int kWaves = 4;  // scoring / transform kernels: one tile per wave
constexpr int kThreads = kWave * kWaves;
// Decode kernel workgroup: 8 waves (one workgroup per CU at two waves per
// SIMD) except float32 K/V at head_dim 128, which runs one wave per SIMD.
// waves of a decode_kernel workgroup: 8 (two per SIMD, <= 256 registers
// each), or 4 at one per SIMD (512 registers) where 256 do not hold a
// wave's state: float32 K/V at head_dim 128 (the raw K and V tile alone take
// 256), the VALU path at head_dim 128 with two or more heads per workgroup
// (its tile words, heads' accumulators and states), and head_dim 256 (the K
// tile alone takes 128, the 32 KiB V slots fill the LDS at four waves)
template <int DT, int D, bool MQK = true, int GT = 1>
struct DecWaves {
  static constexpr int value = (D >= 256 || (D == 128 && (DT == OC_F32 || (!MQK && GT >= 2)))) ? 4 : 8;
};
constexpr float kM0 = -1e9f;
constexpr int kMaxBalTiles = 16384;  // tiles per row for the balanced cached decode (1M tokens)
constexpr int kKeepLds = kMaxBalTiles / 8;  // keep flags staged in LDS (bytes of the bitmask array)
// decode_fast's gate of the model hook's decode step (internal, set by
// oc_hook_decode): Walsh-subspace q norms, their group median and the cached
// tile norms, compared in float64
constexpr int kGateHook = 16;
constexpr int kFastChunks = 32;  // decode_fast: at most 64 * kFastChunks tiles per row
constexpr int kMergeFew = 8;     // fused merge: rows of at most this many partials take the one-pass form

// Kernel arguments (byte strides).  Built by oc_api.hip from oc_decode_params.
struct DecodeArgs {
  const char* k;
  const char* v;
  int64_t k_row_stride, k_tok_stride, v_row_stride, v_tok_stride;
  int32_t v_bf16;  // fp8 K with bf16 V (decode_fast only; strides above in bytes)
  int32_t ctr_stride;  // int32 words between the fused merge's (row, chunk) counters
  int32_t paged, bs_log2, nkv, rows_per_length;
  const int32_t* bt;
  int64_t bt_stride, num_blocks;
  int64_t k_blk_stride, k_head_stride, v_blk_stride, v_head_stride;
  const int32_t* lengths;
  int32_t num_rows, num_tiles;
  int32_t row_tok;  // tokens of every row without lengths (0: num_tiles * ts)
  int32_t ts;       // tokens per tile (64 in every kernel of this file; any power of two in oc_generic.hip)
  int32_t gen_vec;  // oc_generic.hip: K and V rows are read in 16-byte pieces (offsets 16-byte aligned)
  // kGateHook: tile norms of kv head (row % hk_rows) at hk_norms[h * hk_stride
  // + t] for the hk_full complete tiles, threshold hk_tau, per-row
  // statistics (evicted tiles, group norm, largest tile norm) to hk_stats
  const float* hk_norms;
  int64_t hk_stride;
  int32_t hk_rows, hk_full;
  double hk_tau;
  float* hk_stats;
  int32_t k_scale_mode, v_scale_mode;
  float k_scale;  // OC_KSCALE_Q_FOLD and OC_KSCALE_DEQUANT
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
  const uint8_t* tmask;  // OC_GATE_MASK: given (rows, T) tile mask
  int64_t tmask_stride;
  int64_t sc_stride;
  int32_t P;    // logical splits: split s owns tiles {s + kP}
  int32_t spw;  // logical splits per workgroup (group g owns splits [g*spw, g*spw + spw))
  int32_t Pg;   // workgroups (partial states) per row and query head: ceil(P / spw)
  float* pm;
  float* pl;
  float* pacc;
  uint8_t* keep_out;
  int64_t keep_stride;
  int32_t* split_counts;
  float scale;
  // fused merge: the last workgroup of each (row, head chunk) to finish
  // merges the row's Pg partials into out (counters: one per (row, chunk),
  // zero on entry and left zero)
  int32_t fuse;
  int32_t out_dtype;
  // balanced cached decode: the workgroups of a row split the row's retained
  // tiles evenly by rank (set when cached, spw > 1 and T <= kMaxBalTiles)
  int32_t bal;
  // variable-length rows (lengths given, merge fused): blockIdx.x is a flat
  // workgroup slot; row r gets q_r workgroups in proportion to its tiles
  // (flat_map) and its partials live at slots [first slot of r, + q_r)
  int32_t flat;
  int32_t flat_target;  // workgroups the flat layout aims at (slots = flat_target + num_rows)
  // decode_fast_kernel's flat layout (flat_map_lpt): percent of each row's
  // tiles in long shares, the short shares' size divisor, and the slot
  // bound (flat_lpt_slots) that sizes its grid and partials
  int32_t flat_pct, flat_div, flat_slots;
  // the per-wave prologue of decode_fast_kernel (set by the host when it
  // applies) and that kernel's waves per workgroup (4 or 8)
  int32_t fast, fast_waves;
  int32_t* counters;
  char* out;
  int64_t out_stride;  // bytes between query-head rows of out
  // score kernel outputs
  float* o_el;
  float* o_eh;
  float* o_z;
  uint8_t* o_keep;
  int64_t o_stride;
  float* o_fwht;
  // tile range of the scoring / band-norm kernels: tiles [t0, t0 + tcnt) of
  // every row
  int32_t t0, tcnt;
  // band-norm kernel: ||(W64 K)[band_lo, band_hi)||_F per tile, and the
  // per-row count of scored tiles raised to t + 1 (atomic max), if given
  int32_t band_lo, band_hi;
  float* o_norm;
  int32_t* o_valid;
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

// Cross-row exchange with the gfx950 lane swaps: with both operands x,
// v_permlane16_swap returns the even 16-lane rows of x in [0] and the odd
// rows in [1] (each duplicated over its row pair); v_permlane32_swap does
// the same for the two 32-lane halves.
template <int M>
__device__ __forceinline__ void row_pair(float x, float& lo, float& hi) {
  static_assert(M == 16 || M == 32, "cross-row exchange");
  if constexpr (M == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    lo = __uint_as_float(r[0]);
    hi = __uint_as_float(r[1]);
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    lo = __uint_as_float(r[0]);
    hi = __uint_as_float(r[1]);
  }
}

// Partner exchange: M=8 pairs lane k with 15-k inside its 16-lane DPP row
// (row_mirror), M=4 with k^7 (row_half_mirror), M=2 and M=1 with k^2 and
// k^1 (quad_perm); each pairing flips bit log2(M) of the lane index, which
// is all a butterfly needs.  M=16 and M=32 return the lane ^ M value.
template <int M>
__device__ __forceinline__ float xpair(float x) {
  if constexpr (M == 8) return dpp<0x140>(x);
  else if constexpr (M == 4) return dpp<0x141>(x);
  else if constexpr (M == 2) return dpp<0x4E>(x);
  else if constexpr (M == 1) return dpp<0xB1>(x);
  else {
    float lo, hi;
    row_pair<M>(x, lo, hi);
    return (__lane_id() & M) ? lo : hi;
  }
}

// Butterfly across lane bit log2(M) (16 or 32): the lower lane of each pair
// gets x_lo + x_hi, the upper lane x_lo - x_hi.
template <int M>
__device__ __forceinline__ float butterfly_rows(float x) {
  float lo, hi;
  row_pair<M>(x, lo, hi);
  return (__lane_id() & M) ? (lo - hi) : (lo + hi);
}

// value of lane 16*gamma + I for every lane of DPP row gamma (row_newbcast)
template <int I>
__device__ __forceinline__ float row_bcast(float x) {
  return dpp<0x150 + I>(x);
}

// Sum over the 16 lanes of each DPP row (identical bits in every lane).
__device__ __forceinline__ float row16_sum(float x) {
  x += xpair<8>(x);
  x += xpair<4>(x);
  x += xpair<2>(x);
  x += xpair<1>(x);
  return x;
}

__device__ __forceinline__ float wave_sum(float x) {
  x = row16_sum(x);
  float lo, hi;
  row_pair<16>(x, lo, hi);
  x = lo + hi;
  row_pair<32>(x, lo, hi);
  return lo + hi;
}

__device__ __forceinline__ float wave_max(float x) {
  x = fmaxf(x, xpair<8>(x));
  x = fmaxf(x, xpair<4>(x));
  x = fmaxf(x, xpair<2>(x));
  x = fmaxf(x, xpair<1>(x));
  float lo, hi;
  row_pair<16>(x, lo, hi);
  x = fmaxf(lo, hi);
  row_pair<32>(x, lo, hi);
  return fmaxf(lo, hi);
}

// Sum over the four 16-lane rows for each lane position j.
__device__ __forceinline__ float rows4_sum(float x) {
  float lo, hi;
  row_pair<16>(x, lo, hi);
  x = lo + hi;
  row_pair<32>(x, lo, hi);
  return lo + hi;
}

// Inclusive prefix sum over the 64 lanes: row_shr 1, 2, 4, 8 inside each
// 16-lane row, then lane 15 added to row 1 and row 3 (row_bcast:15) and
// lane 31 to rows 2 and 3 (row_bcast:31).  Lanes whose DPP source does not
// exist add 0.
__device__ __forceinline__ int wave_incl_scan(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, false);
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, false);
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, false);
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, false);
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false);
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false);
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

// Non-temporal loads of one lane's row piece (paged VALU path; the K/V
// tiles are streamed once, as with kStreamAux on the buffer loads).
template <int LB>
__device__ __forceinline__ void load_lane_row(const char* p, uint32_t* w) {
  typedef uint32_t v4u __attribute__((ext_vector_type(4)));
  typedef uint32_t v2u __attribute__((ext_vector_type(2)));
  if constexpr (LB == 32) {
    const v4u a = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p));
    const v4u b = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p + 16));
    w[0] = a[0]; w[1] = a[1]; w[2] = a[2]; w[3] = a[3];
    w[4] = b[0]; w[5] = b[1]; w[6] = b[2]; w[7] = b[3];
  } else if constexpr (LB == 16) {
    const v4u a = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p));
    w[0] = a[0]; w[1] = a[1]; w[2] = a[2]; w[3] = a[3];
  } else if constexpr (LB == 8) {
    const v2u a = __builtin_nontemporal_load(reinterpret_cast<const v2u*>(p));
    w[0] = a[0]; w[1] = a[1];
  } else {
    w[0] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p));
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

// tokens of row r: its length clamped to the row capacity
__device__ __forceinline__ int row_tokens(const DecodeArgs& a, int r) {
  int n = a.row_tok > 0 ? a.row_tok : a.num_tiles * 64;
  if (a.lengths) {
    const int len = a.lengths[r / a.rows_per_length];
    n = len < 0 ? 0 : (len < n ? len : n);
  }
  return n;
}

// row info from the row's token count n (row_tokens)
__device__ __forceinline__ RowInfo row_info_n(const DecodeArgs& a, int row, int n) {
  RowInfo ri;
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

__device__ __forceinline__ RowInfo row_info(const DecodeArgs& a, int row) { return row_info_n(a, row, row_tokens(a, row)); }

// Cache policy of the K/V tile loads: non-temporal (the buffer instructions'
// nt bit).  K and V are streamed once per decode step; on MI355X nt loads
// of the decode's 16 KiB K/V chunk pattern reach 6.86 TB/s against 6.0 for
// the default policy (7.15 against 6.33 for a plain stream).
constexpr int kStreamAux = 2;

template <int LB>
__device__ __forceinline__ void buffer_load_lane_row(__amdgpu_buffer_rsrc_t r, int voff, int soff, uint32_t* w) {
  if constexpr (LB == 32) {
    const auto x = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, kStreamAux);
    const auto y = __builtin_amdgcn_raw_buffer_load_b128(r, voff + 16, soff, kStreamAux);
    w[0] = x[0]; w[1] = x[1]; w[2] = x[2]; w[3] = x[3];
    w[4] = y[0]; w[5] = y[1]; w[6] = y[2]; w[7] = y[3];
  } else if constexpr (LB == 16) {
    const auto x = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, kStreamAux);
    w[0] = x[0]; w[1] = x[1]; w[2] = x[2]; w[3] = x[3];
  } else if constexpr (LB == 8) {
    const auto x = __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, kStreamAux);
    w[0] = x[0]; w[1] = x[1];
  } else {
    w[0] = __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, kStreamAux);
  }
}

// Loads one tile (K or V) of `row` into w[i][*] for this lane; tokens at or
// past n_tok read as zero.
// Contiguous rows (PAGED = false) use branch-free buffer loads: one SGPR
// descriptor at the tile start whose size is the valid part of the tile
// (the buffer unit returns zeros past it), one per-lane byte offset per
// 4-token row.
// Paged rows resolve a block id per 4-token group (block_size >= 4); rows at
// or past n_tok are zero-filled without a load, and a block id outside the
// pool raises error_flag and reads zeros.
template <int DT, int D, bool PAGED>
__device__ __forceinline__ void load_tile(const DecodeArgs& a, const RowInfo& ri, int row, int t,
                                          bool is_v, int lane, uint32_t (&w)[16][Lay<DT, D>::LW]) {
  using L = Lay<DT, D>;
  const int gamma = lane >> 4;
  const int j = lane & 15;
  const int tok0 = t * 64;
  const int valid = ri.n_tok - tok0;
  if constexpr (!PAGED) {
    const int64_t ts = is_v ? a.v_tok_stride : a.k_tok_stride;
    const char* base = (is_v ? a.v : a.k) + (int64_t)row * (is_v ? a.v_row_stride : a.k_row_stride) + tok0 * ts;
    const int nbytes = (int)(min(valid, 64) * ts);
    const int voff = gamma * (int)ts + j * L::LB;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      // one descriptor per 4-token row keeps the lane offset in one VGPR; the
      // range check (offset >= num_records) zero-fills tokens past n_tok
      const int rb = 4 * i * (int)ts;
      const __amdgpu_buffer_rsrc_t rs =
          __builtin_amdgcn_make_buffer_rsrc((void*)(base + rb), (short)0, max(nbytes - rb, 0), 0x00020000);
      buffer_load_lane_row<L::LB>(rs, voff, 0, w[i]);
    }
  } else {
    const char* base = is_v ? a.v : a.k;
    const int64_t bstride = is_v ? a.v_blk_stride : a.k_blk_stride;
    const int64_t hoff = (int64_t)ri.head * (is_v ? a.v_head_stride : a.k_head_stride);
    const int64_t ts = is_v ? a.v_tok_stride : a.k_tok_stride;
    const int64_t lane_off = (int64_t)j * L::LB;
    const int32_t* btrow = a.bt + (int64_t)ri.seq * a.bt_stride;
    const int bmask = (1 << a.bs_log2) - 1;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int tok = tok0 + 4 * i;  // uniform; block_size >= 4 keeps tok..tok+3 in one block
      bool ok = 4 * i < valid;
      int64_t blk = 0;
      if (ok) {
        blk = btrow[tok >> a.bs_log2];
        if (blk < 0 || blk >= a.num_blocks) {
          if (a.error_flag && lane == 0) atomicOr(a.error_flag, 1);
          ok = false;
        }
      }
      if (ok) {
        load_lane_row<L::LB>(base + blk * bstride + hoff + (int64_t)((tok & bmask) + gamma) * ts + lane_off, w[i]);
      } else {
#pragma unroll
        for (int x = 0; x < L::LW; ++x) w[i][x] = 0u;
      }
    }
    if (valid < 64) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        if (4 * i + gamma >= valid) {
#pragma unroll
          for (int x = 0; x < L::LW; ++x) w[i][x] = 0u;
        }
      }
    }
  }
}

// bf16 round to nearest even of a float32 (NaN stays NaN)
__device__ __forceinline__ uint32_t bf16_bits(float x) { return __builtin_bit_cast(uint16_t, (__bf16)x); }

// Per-tile dequantisation scale: value = float(elem) * mul when `scaled`.
struct Deq {
  float mul;
  bool scaled;
};

// The CPL values of one register row of this lane as float32.
template <int DT, int D>
__device__ __forceinline__ void row_vals(const uint32_t* w, float (&f)[D / 16]) {
#pragma unroll
  for (int c = 0; c < D / 16; ++c) f[c] = elem<DT>(w, c);
}

// Whole tile as float32 (used by the full-transform kernel).
template <int DT, int D>
__device__ __forceinline__ void decode_tile(const uint32_t (&w)[16][Lay<DT, D>::LW],
                                            float (&f)[16][Lay<DT, D>::CPL], const Deq& dq) {
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    row_vals<DT, D>(w[i], f[i]);
    if (dq.scaled) {
#pragma unroll
      for (int c = 0; c < D / 16; ++c) f[i][c] *= dq.mul;
    }
  }
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
// Elements are dequantised first (float(elem) * scale) as the reference
// does before its W @ K.  The summation order is fixed, so every kernel that
// calls this function (scoring, single-pass decode) produces the same bits.
// `mul` is the tile's dequantisation scale (1 when unscaled: exact).  The
// multiply is unconditional: a branch here lets the compiler hoist the
// element conversions of both arms and keep the whole tile live as floats.
// RND (OC_KSCALE_DEQUANT): each scaled element is rounded to bf16, as the
// reference's k.to(bfloat16) * k_scale before its transform.
template <int DT, int D, bool RND = false>
__device__ __forceinline__ void tile_energies(const uint32_t (&kw)[16][Lay<DT, D>::LW], const Deq& dq, int lane,
                                              float& e_low, float& e_high) {
  const float mul = dq.mul;
  constexpr int CPL = D / 16;
  float h = 0.f;
  float s0[CPL], s1[CPL];  // residue sums for token parity t2 = 0 / 1
#pragma unroll
  for (int c = 0; c < CPL; ++c) s0[c] = s1[c] = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    __builtin_amdgcn_sched_barrier(0);
    float fa[CPL], fb[CPL];
    row_vals<DT, D>(kw[i], fa);
    row_vals<DT, D>(kw[i + 8], fb);
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      fa[c] *= mul;
      fb[c] *= mul;
      if constexpr (RND) {
        fa[c] = __builtin_bit_cast(float, bf16_bits(fa[c]) << 16);
        fb[c] = __builtin_bit_cast(float, bf16_bits(fb[c]) << 16);
      }
    }
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
    s0[c] = butterfly_rows<16>(s0[c]);
    s1[c] = butterfly_rows<16>(s1[c]);
    s0[c] = butterfly_rows<32>(s0[c]);
    s1[c] = butterfly_rows<32>(s1[c]);
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
  if (gate == OC_GATE_MASK) return e_high != 0.f;  // the given mask, read as 0 / 1
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

__device__ __forceinline__ Deq tile_kdeq(const DecodeArgs& a, int row, int t) {
  if (a.k_scale_mode == OC_KSCALE_TILE) return Deq{a.k_scales[(int64_t)row * a.ks_stride + t], true};
  return Deq{1.f, false};
}

__device__ __forceinline__ float tile_vmul(const DecodeArgs& a, int row, int t) {
  if (a.v_scale_mode == OC_VSCALE_TILE) return a.v_scales[(int64_t)row * a.vs_stride + t];
  return 1.f;
}

// ---------------------------------------------------------------- decode

// q . k for the token rows of register row `w`, over this lane's CPL columns.
// Two-element 16-bit dot products (v_dot2_f32_bf16 / v_dot2_f32_f16) when K
// and q share a 16-bit type, float32 FMAs otherwise.
template <int DT, int D, bool DOT2>
__device__ __forceinline__ float row_dot(const uint32_t* w, const uint32_t (&qp)[D / 32 > 0 ? D / 32 : 1],
                                         const float (&qf)[D / 16]) {
  constexpr int CPL = D / 16;
  if constexpr (DOT2 && DT == OC_BF16) {
    typedef __attribute__((ext_vector_type(2))) __bf16 bf2;
    float s = 0.f;
#pragma unroll
    for (int x = 0; x < CPL / 2; ++x)
      s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2, w[x]), __builtin_bit_cast(bf2, qp[x]), s, false);
    return s;
  } else if constexpr (DOT2 && DT == OC_F16) {
    typedef __attribute__((ext_vector_type(2))) _Float16 h2;
    float s = 0.f;
#pragma unroll
    for (int x = 0; x < CPL / 2; ++x)
      s = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, w[x]), __builtin_bit_cast(h2, qp[x]), s, false);
    return s;
  } else {
    float f[CPL];
    row_vals<DT, D>(w, f);
    float s = f[0] * qf[0];
#pragma unroll
    for (int c = 1; c < CPL; ++c) s = __builtin_fmaf(f[c], qf[c], s);
    return s;
  }
}

template <int GT>
struct WaveState {
  float m[GT];
  float l[GT];  // per-lane partial sums of p
};

// logits of query head g for the 64 tokens of a tile: lane 16*gamma + j
// receives token 4j + gamma.  Token rows are taken in pairs (i, i+8) so the
// first transpose-reduce step happens as soon as a pair is done.
template <int DT, int D, bool DOT2>
__device__ __forceinline__ float tile_logit(const uint32_t (&kw)[16][Lay<DT, D>::LW],
                                            const uint32_t (&qp)[D / 32 > 0 ? D / 32 : 1],
                                            const float (&qf)[D / 16], int lane) {
  float v[8];
  const bool up8 = (lane & 8) != 0;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    __builtin_amdgcn_sched_barrier(0);
    const float da = row_dot<DT, D, DOT2>(kw[k], qp, qf);
    const float db = row_dot<DT, D, DOT2>(kw[k + 8], qp, qf);
    const float keep = up8 ? db : da;
    const float send = up8 ? da : db;
    v[k] = keep + xpair<8>(send);
  }
  tr_step<4>(v, lane);
  tr_step<2>(v, lane);
  tr_step<1>(v, lane);
  return v[0];
}

// Online-softmax update of the wave's G states with one retained tile
// (fused_eviction.py:280-299 per head; gqa_eviction.py:409-451 per g), in
// two phases so that the next tile's K can be requested as soon as this
// tile's K registers are free:
//   tile_softmax: logits from K, new max, p = e^(logit - m), l and the acc
//                 rescale;  lscale = 1/sqrt(d) * k_scale(tile) and
//                 vmul = v_scale(tile) fold the per-tile dequantisation
//                 scales into the logits and p;
//   tile_pv:      acc[g][c] += sum_i p(token 4i+gamma) * v[i][c].
template <int DT, int D, int GT, bool DOT2>
__device__ __forceinline__ void tile_softmax(WaveState<GT>& st, float (&acc)[GT][D / 16], float (&p)[GT],
                                             const uint32_t (&kw)[16][Lay<DT, D>::LW], const float* sh_qf,
                                             const uint32_t* sh_qp, float lscale, float vmul, int valid, int lane) {
  constexpr int CPL = D / 16;
  constexpr int QW = D / 32 > 0 ? D / 32 : 1;
  const int j = lane & 15;
  const bool tok_ok = 4 * j + (lane >> 4) < valid;
#pragma unroll
  for (int g = 0; g < GT; ++g) {
    // heads past g_active run on zeroed q and are never written out
    uint32_t qp[QW];
    float qf[CPL];
    if constexpr (DOT2) {
#pragma unroll
      for (int x = 0; x < QW; ++x) qp[x] = sh_qp[g * (D / 2) + j * QW + x];
    } else {
#pragma unroll
      for (int c = 0; c < CPL; ++c) qf[c] = sh_qf[g * D + j * CPL + c];
    }
    // computed in every lane (the transpose-reduce reads all lanes), then masked
    float logit = tile_logit<DT, D, DOT2>(kw, qp, qf, lane) * lscale;
    logit = tok_ok ? logit : -__builtin_inff();
    const float mt = wave_max(logit);
    const float mn = fmaxf(st.m[g], mt);
    const float alpha = __expf(st.m[g] - mn);
    const float pg = __expf(logit - mn);
    st.l[g] = __builtin_fmaf(st.l[g], alpha, pg);
    st.m[g] = mn;
    p[g] = pg * vmul;
#pragma unroll
    for (int c = 0; c < CPL; ++c) acc[g][c] *= alpha;
  }
}

template <int DT, int D, int GT>
__device__ __forceinline__ void tile_pv(float (&acc)[GT][D / 16], const float (&p)[GT],
                                        const uint32_t (&vw)[16][Lay<DT, D>::LW]) {
  constexpr int CPL = D / 16;
  // p of token 4i+gamma sits in lane 16*gamma + i of the same DPP row
#define OC_PV_STEP(I)                                                                       \
  {                                                                                         \
    __builtin_amdgcn_sched_barrier(0);                                                      \
    float fv[CPL];                                                                          \
    row_vals<DT, D>(vw[I], fv);                                                             \
    _Pragma("unroll") for (int g = 0; g < GT; ++g) {                                        \
      const float pb = row_bcast<I>(p[g]);                                                  \
      _Pragma("unroll") for (int c = 0; c < CPL; ++c) acc[g][c] = __builtin_fmaf(pb, fv[c], acc[g][c]); \
    }                                                                                       \
  }
  OC_PV_STEP(0) OC_PV_STEP(1) OC_PV_STEP(2) OC_PV_STEP(3)
  OC_PV_STEP(4) OC_PV_STEP(5) OC_PV_STEP(6) OC_PV_STEP(7)
  OC_PV_STEP(8) OC_PV_STEP(9) OC_PV_STEP(10) OC_PV_STEP(11)
  OC_PV_STEP(12) OC_PV_STEP(13) OC_PV_STEP(14) OC_PV_STEP(15)
#undef OC_PV_STEP
}

// ------------------------------------------------- q.k on the matrix cores
//
// Cached and dense decode with 16-bit K and q of the same type form the
// logits of a 64-token tile with v_mfma_f32_16x16x32_{bf16,f16}:
// D[m][n] = sum_k A[m][k] B[k][n] with A = q (m = query head, zero rows past
// GT), B = K^T of one 16-token block (n = token) and k = 32 head-dim columns
// per instruction, fp32 accumulation (the same products and accumulation
// type as v_dot2_f32).  Lane layouts (lane = 16*kg + x):
//   A: q[head x][32*dc + 8*kg .. +8]        B: K[token 16*tb + x][32*dc + 8*kg .. +8]
//   D: lane 16*r + x, register i -> head 4*r + i, token 16*tb + x
// so the K tile is read as 16-byte row pieces (tb, dc) of one token per lane.
// The probabilities go to the wave's LDS slot as p[head][token] and p.V runs
// on the matrix cores too, with V staged in LDS (tile_pv_mfma).

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// 16-bit type the matrix cores run in for K of type DT: the type itself, or
// bf16 for fp8-e4m3 K, whose values bf16 holds exactly (widened with
// v_cvt_scalef32_pk_bf16_fp8 at scale 1; all 256 codes checked on the GPU
// against the float32 decode).
template <int DT>
struct MfmaT {
  static constexpr int value = DT == OC_FP8_E4M3FN ? OC_BF16 : DT;
};

// four fp8 values (one word) -> two words of bf16 pairs
__device__ __forceinline__ void fp8x4_to_bf16(uint32_t w, uint32_t& lo, uint32_t& hi) {
  lo = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false));
  hi = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true));
}


// OC_KSCALE_DEQUANT: four fp8 values -> bf16(float32(float(k) * s)), the
// reference's k.to(bfloat16) * k_scale (a float32 product rounded once more to
// bfloat16).  v_cvt_scalef32_pk_bf16_fp8 cannot do it: it applies only the
// exponent of its scale operand (measured on the GPU over all 256 codes).
__device__ __forceinline__ void fp8x4_to_bf16_scaled(uint32_t w, float sc, uint32_t& lo, uint32_t& hi) {
  const auto p0 = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
  const auto p1 = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
  lo = bf16_bits(p0[0] * sc) | (bf16_bits(p0[1] * sc) << 16);
  hi = bf16_bits(p1[0] * sc) | (bf16_bits(p1[1] * sc) << 16);
}

// how K enters the matrix cores: fp8 widened exactly, or (OC_KSCALE_DEQUANT)
// scaled and rounded to bf16
struct KDq {
  bool on;
  float s;
};
__device__ __forceinline__ KDq k_dq(const DecodeArgs& a) {
  return KDq{a.k_scale_mode == OC_KSCALE_DEQUANT, a.k_scale};
}

template <int DT>
__device__ __forceinline__ f32x4 mfma_qk(const uint32_t (&aq)[4], const uint32_t (&bk)[4], f32x4 c) {
  const u32x4 av = {aq[0], aq[1], aq[2], aq[3]};
  const u32x4 bv = {bk[0], bk[1], bk[2], bk[3]};
  if constexpr (DT == OC_BF16) {
    typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, av), __builtin_bit_cast(bf16x8, bv),
                                                   c, 0, 0, 0);
  } else {
    typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, av), __builtin_bit_cast(f16x8, bv), c,
                                                  0, 0, 0);
  }
}

// A operand: q of head (lane & 15) from the packed LDS copy (zero past GT).
// Instruction dc takes head-dim columns 32*dc + 8*kg .. +8 from lane group
// kg; for fp8 K, whose lanes hold D/4 consecutive columns (kg*D/4 ..),
// columns kg*D/4 + 8*dc .. +8 (any column order works if q and K agree).
template <int DT, int D, int GT>
__device__ __forceinline__ void load_q_mfma(const uint32_t* sh_qp, int lane, uint32_t (&aq)[D / 32][4]) {
  const int x = lane & 15;
  const int kg = lane >> 4;
#pragma unroll
  for (int dc = 0; dc < D / 32; ++dc)
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const int pair = DT == OC_FP8_E4M3FN ? kg * (D / 8) + 4 * dc + w : 16 * dc + 4 * kg + w;
      aq[dc][w] = x < GT ? sh_qp[x * (D / 2) + pair] : 0u;
    }
}

// B operand (eight 16-bit values) of instruction (tb, dc) from the K
// registers: kb[tb][dc] for 16-bit K; for fp8 K the lane's bytes 8*dc .. +8
// of its D/4-byte row piece (words 2dc, 2dc + 1), widened to bf16.
template <int DT, int D>
__device__ __forceinline__ void k_operand(const uint32_t (&kb)[4][D / 32][4], int tb, int dc, uint32_t (&b)[4],
                                          bool dq = false, float sc = 1.f) {
  if constexpr (DT == OC_FP8_E4M3FN) {
    if (dq) {
      fp8x4_to_bf16_scaled(kb[tb][(2 * dc) >> 2][(2 * dc) & 3], sc, b[0], b[1]);
      fp8x4_to_bf16_scaled(kb[tb][(2 * dc + 1) >> 2][(2 * dc + 1) & 3], sc, b[2], b[3]);
    } else {
      fp8x4_to_bf16(kb[tb][(2 * dc) >> 2][(2 * dc) & 3], b[0], b[1]);
      fp8x4_to_bf16(kb[tb][(2 * dc + 1) >> 2][(2 * dc + 1) & 3], b[2], b[3]);
    }
  } else {
#pragma unroll
    for (int w = 0; w < 4; ++w) b[w] = kb[tb][dc][w];
  }
}

// Pages of the four 16-token blocks of a tile (paged K/V on the matrix-core
// path, block_size >= 16, so each block lies in one page): the block id
// (-1: no valid token, or an id outside the pool, which sets `bad` and
// reads as zeros) and the block's valid tokens.  Wave-uniform.
struct TilePages {
  int id[4];
  int n[4];
};

__device__ __forceinline__ TilePages tile_pages(const DecodeArgs& a, const RowInfo& ri, int t, bool& bad) {
  TilePages pg;
  const int32_t* btrow = a.bt + (int64_t)ri.seq * a.bt_stride;
#pragma unroll
  for (int tb = 0; tb < 4; ++tb) {
    const int tok = t * 64 + 16 * tb;
    int n = min(max(ri.n_tok - tok, 0), 16);
    int id = -1;
    if (n > 0) {
      id = btrow[tok >> a.bs_log2];
      if (id < 0 || id >= a.num_blocks) {
        bad = true;
        id = -1;
        n = 0;
      }
    }
    pg.id[tb] = id;
    pg.n[tb] = n;
  }
  return pg;
}

// Byte address of token `tok` of block id `id` (paged pool, kv head of the
// row; the pool start for id -1, whose descriptor then covers no bytes).
__device__ __forceinline__ const char* page_row(const char* pool, int64_t blk_stride, int64_t head_off, int64_t ts,
                                                int id, int tok, int bmask) {
  return pool + (id >= 0 ? (int64_t)id * blk_stride + head_off + (int64_t)(tok & bmask) * ts : 0);
}

// B operand pieces of one K tile (16-bit elements): lane 16*kg + x reads
// token 16*tb + x, columns 32*dc + 8*kg .. +8.  One buffer descriptor per
// 16-token block (contiguous rows: at the block; paged: at the block's
// place in its page) whose size is the valid part of the block, so tokens
// at or past n_tok read as zero.
//
// fp8 K: lane 16*kg + x reads the D/4 bytes kg*D/4 .. of token 16*tb + x
// (D/64 128-bit loads per block) into kb[tb][0..D/64).
template <int DT, int D, bool PAGED>
__device__ __forceinline__ void load_k_mfma(const DecodeArgs& a, const RowInfo& ri, int row, int t, int lane,
                                            uint32_t (&kb)[4][D / 32][4], const TilePages& pg) {
  constexpr bool F8 = DT == OC_FP8_E4M3FN;
  const int x = lane & 15;
  const int kg = lane >> 4;
  const int tok0 = t * 64;
  const int64_t ts = a.k_tok_stride;
  const char* base = a.k + (int64_t)row * a.k_row_stride + tok0 * ts;
  const int nbytes = (int)(min(ri.n_tok - tok0, 64) * ts);
  const int voff = x * (int)ts + (F8 ? kg * (D / 4) : 16 * kg);
#pragma unroll
  for (int tb = 0; tb < 4; ++tb) {
    const int rb = 16 * tb * (int)ts;
    __amdgpu_buffer_rsrc_t rs;
    if constexpr (PAGED) {
      const char* pb = page_row(a.k, a.k_blk_stride, (int64_t)ri.head * a.k_head_stride, ts, pg.id[tb],
                                tok0 + 16 * tb, (1 << a.bs_log2) - 1);
      rs = __builtin_amdgcn_make_buffer_rsrc((void*)pb, (short)0, pg.n[tb] * (int)ts, 0x00020000);
    } else {
      rs = __builtin_amdgcn_make_buffer_rsrc((void*)(base + rb), (short)0, max(nbytes - rb, 0), 0x00020000);
    }
#pragma unroll
    for (int dc = 0; dc < (F8 ? D / 64 : D / 32); ++dc) {
      const auto v = __builtin_amdgcn_raw_buffer_load_b128(rs, voff + (F8 ? 16 : 64) * dc, 0, kStreamAux);
      kb[tb][dc][0] = v[0];
      kb[tb][dc][1] = v[1];
      kb[tb][dc][2] = v[2];
      kb[tb][dc][3] = v[3];
    }
  }
}

// Online-softmax state in the MFMA output layout: lane 16*r + x keeps heads
// 4*r + i (i = 0..3); l is the lane's partial sum over its tokens.
struct MState {
  float m[4];
  float l[4];
};

// LDS layout of the matrix-core decode's V tile: the 16-byte chunk c of row
// r is stored at chunk c ^ v_xor(r).  A transposing read (tile_pv_mfma)
// takes one column piece of 16 rows (16-bit) or 32 rows (fp8) whose stride
// is a multiple of the bank line; the XOR gives them distinct bank slots
// (each slot used twice) instead of one slot 16 times over.
template <int DT, int D>
__host__ __device__ constexpr int v_xor(int r) {
  if constexpr (DT == OC_FP8_E4M3FN) {
    if constexpr (D == 256) return r & 15;
    else if constexpr (D == 128) return (r >> 1) & 7;
    else if constexpr (D == 64) return (r >> 2) & 3;
    else return 0;
  } else {
    // 128 and 256 (512-byte rows: the same pairs of rows share a bank line)
    if constexpr (D == 128 || D == 256) return 2 * ((r & 3) + 4 * ((r >> 3) & 1));
    else if constexpr (D == 64) return 2 * (((r & 3) >> 1) + 2 * ((r >> 3) & 1));
    // 32 (64-byte rows, four to a bank line): rows r and r + 8 of one read
    // take the two halves of the line in opposite order
    else if constexpr (D == 32) return 2 * ((r >> 3) & 1);
    else return 0;
  }
}

// Compile-time pin of v_xor: every chunk stays inside its row, and each
// transposing read of tile_pv_t (16-bit: 16 rows x 32 bytes, rows 32 tb2 +
// 8 kg + 4 h + m; fp8: 32 rows x 16 bytes, rows 32 tb2 + 8 kg + m) puts at
// most two 16-byte pieces on any of the 16 bank slots of a 256-byte line.
template <int DT, int D>
constexpr bool v_xor_pin() {
  constexpr bool F8 = DT == OC_FP8_E4M3FN;
  constexpr int es = F8 ? 1 : 2, row_bytes = D * es, chunks = row_bytes / 16;
  for (int r = 0; r < 64; ++r)
    for (int c = 0; c < chunks; ++c)
      if ((c ^ v_xor<DT, D>(r)) < 0 || (c ^ v_xor<DT, D>(r)) >= chunks) return false;
  for (int tb2 = 0; tb2 < 2; ++tb2)
    for (int nc = 0; nc < D / 16; ++nc)
      for (int h = 0; h < (F8 ? 1 : 2); ++h) {
        int use[16] = {};
        for (int kg = 0; kg < 4; ++kg)
          for (int m = 0; m < (F8 ? 8 : 4); ++m) {
            const int r = F8 ? 32 * tb2 + 8 * kg + m : 32 * tb2 + 8 * kg + 4 * h + m;
            const int o = F8 ? 16 * (nc ^ v_xor<DT, D>(r)) : 32 * (nc ^ (v_xor<DT, D>(r) >> 1));
            for (int piece = 0; piece < (F8 ? 16 : 32); piece += 16)
              if (++use[((r * row_bytes + o + piece) % 256) / 16] > 2) return false;
          }
      }
  return true;
}
static_assert(v_xor_pin<OC_BF16, 256>() && v_xor_pin<OC_BF16, 128>() && v_xor_pin<OC_BF16, 64>() &&
                  v_xor_pin<OC_BF16, 32>() && v_xor_pin<OC_FP8_E4M3FN, 256>() && v_xor_pin<OC_FP8_E4M3FN, 128>() &&
                  v_xor_pin<OC_FP8_E4M3FN, 64>(),
              "v_xor: a transposing V read uses a bank slot more than twice, or a chunk leaves its row");

// 16 bytes per lane from a buffer straight to LDS (non-temporal): lane i's
// bytes land at dst + 16 i (dst wave-uniform)
__device__ __forceinline__ void v_load_lds16(__amdgpu_buffer_rsrc_t r, uint16_t* dst, int voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 16, voff, 0, 0,
                                           kStreamAux);
}

// V tile of one 64-token tile into the wave's LDS slot, row-major
// [token][D] with the chunk order of v_xor, by direct-to-LDS buffer loads
// (16 bytes per lane, one 1 KiB instruction per 1024 / (es D) tokens: the
// lane filling slot (row, chunk c) loads chunk c ^ v_xor(row)); tokens at
// or past n_tok read as zero through the descriptor's range check.
template <int DT, int D, bool PAGED>
__device__ __forceinline__ void load_v_lds(const DecodeArgs& a, const RowInfo& ri, int row, int t, int lane,
                                           uint16_t* sv, const TilePages& pg) {
  constexpr int TPI = 1024 / (Elem<DT>::size * D);  // tokens per instruction
  constexpr int LPT = 64 / TPI;        // lanes per token
  const int64_t ts = a.v_tok_stride;
  const int tok0 = t * 64;
  const int rl = lane / LPT, cl = lane % LPT;
  const int voff = rl * (int)ts;
  // byte offset of the lane's chunk in instruction i (rows i * TPI + rl)
  auto chunk = [&](int i) { return 16 * (cl ^ v_xor<DT, D>(i * TPI + rl)); };
  if constexpr (PAGED) {
    // one descriptor per 16-token block (in one page), 16 / TPI instructions each
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
      const char* pb = page_row(a.v, a.v_blk_stride, (int64_t)ri.head * a.v_head_stride, ts, pg.id[tb],
                                tok0 + 16 * tb, (1 << a.bs_log2) - 1);
      const __amdgpu_buffer_rsrc_t rs =
          __builtin_amdgcn_make_buffer_rsrc((void*)pb, (short)0, pg.n[tb] * (int)ts, 0x00020000);
#pragma unroll
      for (int j = 0; j < 16 / TPI; ++j)
        v_load_lds16(rs, sv + (tb * (16 / TPI) + j) * 512, voff + chunk(tb * (16 / TPI) + j) + j * TPI * (int)ts);
    }
  } else {
    const char* base = a.v + (int64_t)row * a.v_row_stride + tok0 * ts;
    const int nbytes = (int)(min(ri.n_tok - tok0, 64) * ts);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, nbytes, 0x00020000);
#pragma unroll
    for (int i = 0; i < 64 / TPI; ++i)
      v_load_lds16(rs, sv + i * 512, voff + chunk(i) + i * TPI * (int)ts);
  }
}

// Raw logits q.k of one tile on the matrix cores: c[tb] in the D layout
// above (head 4r + i, token 16 tb + x in lane 16r + x, register i).
template <int DT, int D>
__device__ __forceinline__ void tile_logits_mfma(const uint32_t (&aq)[D / 32][4], const uint32_t (&kb)[4][D / 32][4],
                                                 f32x4 (&c)[4]) {
#pragma unroll
  for (int tb = 0; tb < 4; ++tb) {
    c[tb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int dc = 0; dc < D / 32; ++dc) {
      uint32_t b[4];
      k_operand<DT, D>(kb, tb, dc, b);
      c[tb] = mfma_qk<MfmaT<DT>::value>(aq[dc], b, c[tb]);
    }
  }
}

// Online-softmax update of the heads' states from a tile's raw logits; p
// (times vmul) goes to the wave's LDS slot as sp[head * 64 + token] and the
// p.V accumulators are rescaled by e^(m_old - m_new) (same lane layout as
// the state).
template <int DT, int D, int GT>
__device__ __forceinline__ void tile_softmax_regs(MState& ms, f32x4 (&accp)[D / 16], const f32x4 (&c)[4], float* sp,
                                                  float lscale, float vmul, int valid, int lane) {
  const int x = lane & 15;
  const int r = lane >> 4;
  // the state is kept in base-2 units (logit * log2 e), so each
  // probability is one exp2; it is converted back where it leaves the wave
  const float lscale2 = lscale * 1.4426950408889634f;
  float v[4][4];
  if (valid >= 64) {
#pragma unroll
    for (int tb = 0; tb < 4; ++tb)
#pragma unroll
      for (int i = 0; i < 4; ++i) v[tb][i] = c[tb][i] * lscale2;
  } else {
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
      const bool tok_ok = 16 * tb + x < valid;
#pragma unroll
      for (int i = 0; i < 4; ++i) v[tb][i] = tok_ok ? c[tb][i] * lscale2 : -__builtin_inff();
    }
  }
  float alpha[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float mt = fmaxf(fmaxf(v[0][i], v[1][i]), fmaxf(v[2][i], v[3][i]));
    mt = fmaxf(mt, xpair<8>(mt));
    mt = fmaxf(mt, xpair<4>(mt));
    mt = fmaxf(mt, xpair<2>(mt));
    mt = fmaxf(mt, xpair<1>(mt));
    const float mn = fmaxf(ms.m[i], mt);
    alpha[i] = __builtin_amdgcn_exp2f(ms.m[i] - mn);
    ms.m[i] = mn;
    float ls = 0.f;
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
      const float pp = __builtin_amdgcn_exp2f(v[tb][i] - mn);
      ls += pp;
      v[tb][i] = pp;
    }
    ms.l[i] = __builtin_fmaf(ms.l[i], alpha[i], ls);
  }
  // most tiles leave every running max unchanged (alpha == 1 in every lane)
  if (__builtin_amdgcn_ballot_w64(alpha[0] != 1.f || alpha[1] != 1.f || alpha[2] != 1.f || alpha[3] != 1.f)) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int nc = 0; nc < D / 16; ++nc) accp[nc][i] *= alpha[i];
  }
  // V's per-tile scale (fp8 V) folded into the probabilities p.V uses
  if (vmul != 1.f) {
#pragma unroll
    for (int tb = 0; tb < 4; ++tb)
#pragma unroll
      for (int i = 0; i < 4; ++i) v[tb][i] *= vmul;
  }
  if (r < (GT + 3) / 4) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) sp[(4 * r + i) * 64 + 16 * tb + x] = v[tb][i];
  }
}

template <int DT, int D, int GT>
__device__ __forceinline__ void tile_softmax_mfma(MState& ms, f32x4 (&accp)[D / 16], const uint32_t (&aq)[D / 32][4],
                                                  const uint32_t (&kb)[4][D / 32][4], float* sp, float lscale,
                                                  float vmul, int valid, int lane) {
  f32x4 c[4];
  tile_logits_mfma<DT, D>(aq, kb, c);
  tile_softmax_regs<DT, D, GT>(ms, accp, c, sp, lscale, vmul, valid, lane);
}

template <int DT>
__device__ __forceinline__ void unpack16x2(uint32_t u, float& lo, float& hi) {
  if constexpr (DT == OC_BF16) {
    lo = __uint_as_float(u << 16);
    hi = __uint_as_float(u & 0xffff0000u);
  } else {
    lo = (float)__builtin_bit_cast(_Float16, (uint16_t)(u & 0xffffu));
    hi = (float)__builtin_bit_cast(_Float16, (uint16_t)(u >> 16));
  }
}

// Band energies of a 16-bit K tile held in the matrix-core layout (lane
// 16*kg + x: tokens 16*tb + x, columns 32*dc + 8*kg .. +8), for the
// single-pass gate of the matrix-core decode:
//   E_high = 1/2 sum_{u<32} ||k_u - k_{u+32}||^2 (W64 rows 32..63, as in
//     tile_energies); the pairs (tb, tb + 2) sit in the same lane.
//   E_low = sum_{i=1..7} ||X_i||^2, X_i = 1/8 sum_r h8_i(r) S_r over the
//     residue sums S_r = sum_{t = r mod 8} k_t.  A lane sums its four tokens
//     (residue r = x & 7), adds lane x ^ 8 (row_ror:8; lanes x and x ^ 8 then
//     hold identical copies) and runs an 8-point butterfly over lane bits 0
//     and 1 (quad_perm) and 2 (row_ror:4, which reaches residue r ^ 4 in
//     either direction thanks to the copies).  A stage is y += s * partner
//     with s = -1 where the lane's bit is set, so the upper lane of a pair
//     holds -(lo - hi): the transform is exact up to per-lane signs, which
//     the squares drop.  The lane with r = 0 holds the DC row (no sign
//     flips), which E_low leaves out; lanes x >= 8 are the copies.
// The summation order is not that of tile_energies, so the two can differ
// in the last bits.
//
// fp8 K (a lane holds D/4 columns per token, kb[tb][0..D/64)) with a
// per-tile scale s: the energies of the stored values times s^2 (the
// energies of the dequantised tile s*k up to float rounding).
template <int DT, int D, bool LOW>
__device__ __forceinline__ void tile_energies_mfma(const uint32_t (&kb)[4][D / 32][4], int lane, float mul,
                                                   float& e_low, float& e_high) {
  constexpr bool F8 = DT == OC_FP8_E4M3FN;
  constexpr int NW = F8 ? D / 16 : D / 8;  // words of one token's row piece
  constexpr int EPW = F8 ? 4 : 2;          // values per word
  const int x = lane & 15;
  const float s0 = (x & 1) ? -1.f : 1.f;
  const float s1 = (x & 2) ? -1.f : 1.f;
  const float s2 = (x & 4) ? -1.f : 1.f;
  const bool low_lane = (x & 7) != 0 && x < 8;
  float h = 0.f, lo = 0.f;
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    // one word per token at a time: keeps the unpacked floats of the whole
    // tile from being live at once
    __builtin_amdgcn_sched_barrier(0);
    float f[4][EPW];
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
      const uint32_t u = kb[tb][i >> 2][i & 3];
      if constexpr (F8) {
        const auto p0 = __builtin_amdgcn_cvt_pk_f32_fp8((int)u, false);
        const auto p1 = __builtin_amdgcn_cvt_pk_f32_fp8((int)u, true);
        f[tb][0] = p0[0];
        f[tb][1] = p0[1];
        f[tb][2] = p1[0];
        f[tb][3] = p1[1];
      } else {
        unpack16x2<DT>(u, f[tb][0], f[tb][1]);
      }
    }
#pragma unroll
    for (int e = 0; e < EPW; ++e) {
      const float d0 = f[0][e] - f[2][e];
      const float d1 = f[1][e] - f[3][e];
      h = __builtin_fmaf(d0, d0, h);
      h = __builtin_fmaf(d1, d1, h);
      if constexpr (LOW) {
        float y = (f[0][e] + f[1][e]) + (f[2][e] + f[3][e]);
        y += dpp<0x128>(y);                         // row_ror:8
        y = __builtin_fmaf(dpp<0xB1>(y), s0, y);    // quad_perm [1,0,3,2]
        y = __builtin_fmaf(dpp<0x4E>(y), s1, y);    // quad_perm [2,3,0,1]
        y = __builtin_fmaf(dpp<0x124>(y), s2, y);   // row_ror:4
        lo = low_lane ? __builtin_fmaf(y, y, lo) : lo;
      }
    }
  }
  const float m2 = mul * mul;
  e_high = wave_sum(h) * 0.5f * m2;
  e_low = LOW ? wave_sum(lo) * (1.f / 64.f) * m2 : 0.f;
}

// s_waitcnt immediate that waits until at most n vector-memory operations
// are outstanding (gfx9 encoding; export and LDS counts left at their maxima)
constexpr int vmcnt_imm(int n) { return (n & 15) | (7 << 4) | (15 << 8) | ((n >> 4) << 14); }
// s_waitcnt immediate: outstanding LDS / scalar-memory operations done, vector
// memory operations left in flight
constexpr int kLgkmOnly = 15 | (7 << 4) | (0 << 8) | (3 << 14);

// p.V on the matrix cores: D[head][d] += sum_token P[head][token] V[token][d]
// per 32-token block and 16-column chunk.  A = P of head (lane & 15), tokens
// 8*kg .. +8 of the block, as a 16-bit high part plus the 16-bit rounding
// of the remainder (two instructions, so the products keep about 16
// mantissa bits of p; V is exact); B = V read from the LDS tile with the
// transposing ds_read_b64_tr_b16 (lane x of group kg gets V[8kg + e][16nc + x]
// from the four lanes that address rows 8kg + e, columns 16nc + 4(x%4) ..).
template <int DT, int D, int GT>
__device__ __forceinline__ void tile_pv_mfma(f32x4 (&accp)[D / 16], const float* sp, const uint16_t* sv, int lane) {
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  const int x = lane & 15;
  const int kg = lane >> 4;
#pragma unroll
  for (int tb2 = 0; tb2 < 2; ++tb2) {
    float pv[8];
    if (x < GT) {
      const float4 p0 = *reinterpret_cast<const float4*>(sp + x * 64 + 32 * tb2 + 8 * kg);
      const float4 p1 = *reinterpret_cast<const float4*>(sp + x * 64 + 32 * tb2 + 8 * kg + 4);
      pv[0] = p0.x; pv[1] = p0.y; pv[2] = p0.z; pv[3] = p0.w;
      pv[4] = p1.x; pv[5] = p1.y; pv[6] = p1.z; pv[7] = p1.w;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) pv[e] = 0.f;
    }
    uint32_t ahi[4], alo[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if constexpr (MfmaT<DT>::value == OC_BF16) {
        const __bf16 h0 = (__bf16)pv[2 * e], h1 = (__bf16)pv[2 * e + 1];
        const __bf16 l0 = (__bf16)(pv[2 * e] - (float)h0), l1 = (__bf16)(pv[2 * e + 1] - (float)h1);
        ahi[e] = (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
        alo[e] = (uint32_t)__builtin_bit_cast(uint16_t, l0) | ((uint32_t)__builtin_bit_cast(uint16_t, l1) << 16);
      } else {
        const _Float16 h0 = (_Float16)pv[2 * e], h1 = (_Float16)pv[2 * e + 1];
        const _Float16 l0 = (_Float16)(pv[2 * e] - (float)h0), l1 = (_Float16)(pv[2 * e + 1] - (float)h1);
        ahi[e] = (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
        alo[e] = (uint32_t)__builtin_bit_cast(uint16_t, l0) | ((uint32_t)__builtin_bit_cast(uint16_t, l1) << 16);
      }
    }
    // rows of this lane's transposing reads: 32*tb2 + 8*kg + 4*h + x/4; the
    // column pieces sit at the chunk order of v_xor, whose XOR is the same
    // for h = 0 and 1
    const int vrow = 32 * tb2 + 8 * kg + (x >> 2);
    const int vx = v_xor<DT, D>(vrow) >> 1;  // 16-bit: XOR of the 32-byte column pair
    const uint16_t* rowp = sv + vrow * D + 4 * (x & 3);
    // fp8 V: ds_read_b64_tr_b8 with lane x addressing row 32*tb2 + 8*kg +
    // x/2, bytes 16*nc + 8*(x%2) .. +8 returns V[32*tb2 + 8*kg + e][16*nc + x]
    // in byte e (e = 0..7; checked on the GPU with an in-bounds probe)
    const int vrow8 = 32 * tb2 + 8 * kg + (x >> 1);
    const int vx8 = v_xor<DT, D>(vrow8);  // fp8: XOR of the 16-byte chunk
    const uint8_t* rowp8 = reinterpret_cast<const uint8_t*>(sv) + vrow8 * D + 8 * (x & 1);
#pragma unroll
    for (int nc = 0; nc < D / 16; ++nc) {
      uint32_t bk[4];
      if constexpr (DT == OC_FP8_E4M3FN) {
        typedef int i32x2 __attribute__((ext_vector_type(2)));
        const i32x2 b8 = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
            (__attribute__((address_space(3))) i32x2*)(rowp8 + 16 * (nc ^ vx8)));
        fp8x4_to_bf16((uint32_t)b8[0], bk[0], bk[1]);
        fp8x4_to_bf16((uint32_t)b8[1], bk[2], bk[3]);
      } else {
        const s16x4 b0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) s16x4*)(rowp + 16 * (nc ^ vx)));
        const s16x4 b1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) s16x4*)(rowp + 4 * D + 16 * (nc ^ vx)));
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        const u32x2 w0 = __builtin_bit_cast(u32x2, b0), w1 = __builtin_bit_cast(u32x2, b1);
        bk[0] = w0[0];
        bk[1] = w0[1];
        bk[2] = w1[0];
        bk[3] = w1[1];
      }
      accp[nc] = mfma_qk<MfmaT<DT>::value>(ahi, bk, accp[nc]);
      accp[nc] = mfma_qk<MfmaT<DT>::value>(alo, bk, accp[nc]);
    }
  }
}

// ---- transposed matrix-core step (attend-every-tile loop, contiguous rows)
//
// S^T = K.q^T: with K as the A operand, lane 16r + x register i of c[tb]
// holds the logit of head x for K row 4r + i of 16-token block tb, so each
// head's online softmax is per lane (two cross-lane steps) and the
// probabilities are already the B operand of O^T += V^T.P^T: no P round trip
// through LDS.  For that, A-row a of the tile holds token kperm(a): within
// each 32-token block, a = 16h + 4r + i holds token 8r + 4h + i, so the eight
// probabilities a lane holds for block j are tokens 32j + 8kg .. + 7 in order,
// the k index of the p.V instruction (V stays in token order).
__host__ __device__ constexpr int kperm(int a) {
  return (a & ~31) + 8 * ((a >> 2) & 3) + 4 * ((a >> 4) & 1) + (a & 3);
}

// Compile-time pin of kperm: a permutation of the tile's 64 rows under which
// lane group kg's registers c[2j][i], c[2j + 1][i] (A rows 32j + 4kg + i and
// 32j + 16 + 4kg + i) hold tokens 32j + 8kg .. + 7 in order.
constexpr bool kperm_pin() {
  bool seen[64] = {};
  for (int a = 0; a < 64; ++a) {
    const int t = kperm(a);
    if (t < 0 || t >= 64 || seen[t]) return false;
    seen[t] = true;
  }
  for (int j = 0; j < 2; ++j)
    for (int kg = 0; kg < 4; ++kg)
      for (int e = 0; e < 8; ++e)
        if (kperm(32 * j + 16 * (e >> 2) + 4 * kg + (e & 3)) != 32 * j + 8 * kg + e) return false;
  return true;
}
static_assert(kperm_pin(), "kperm: the transposed step's K row order no longer matches the p.V operand");

struct MStateT {
  float m;  // running max of the lane's head, base-2 units
  float l;  // partial sum over the lane's tokens
};

// K rows of tile t in kperm order (one descriptor for the tile; rows at or
// past n_tok read as zero through its range check)
template <int DT, int D>
__device__ __forceinline__ void load_k_mfma_t(const DecodeArgs& a, const RowInfo& ri, int row, int t, int lane,
                                              uint32_t (&kb)[4][D / 32][4]) {
  constexpr bool F8 = DT == OC_FP8_E4M3FN;
  const int x = lane & 15;
  const int kg = lane >> 4;
  const int tok0 = t * 64;
  const int64_t ts = a.k_tok_stride;
  const char* base = a.k + (int64_t)row * a.k_row_stride + tok0 * ts;
  const int nbytes = (int)(min(ri.n_tok - tok0, 64) * ts);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, nbytes, 0x00020000);
  const int cofs = F8 ? kg * (D / 4) : 16 * kg;
#pragma unroll
  for (int tb = 0; tb < 4; ++tb) {
    const int voff = kperm(16 * tb + x) * (int)ts + cofs;
#pragma unroll
    for (int dc = 0; dc < (F8 ? D / 64 : D / 32); ++dc) {
      const auto v = __builtin_amdgcn_raw_buffer_load_b128(rs, voff + (F8 ? 16 : 64) * dc, 0, kStreamAux);
      kb[tb][dc][0] = v[0];
      kb[tb][dc][1] = v[1];
      kb[tb][dc][2] = v[2];
      kb[tb][dc][3] = v[3];
    }
  }
}

// Paged K rows of tile t in kperm order (pages of >= 16 tokens, tile_pages'
// ids).  The sixteen A-rows 16 tb .. +15 hold tokens of 16-token blocks
// 2 (tb / 2) (lanes x < 8) and 2 (tb / 2) + 1 (x >= 8), each in one page, so
// the loads are per-lane global loads (non-temporal) at the token's place in
// its page; tokens past the block's valid count or of an invalid page read
// as zero (their lanes load the pool's first row and drop it, so that every
// load is unconditional and the compiler's wait counts stay exact).
template <int DT, int D>
__device__ __forceinline__ void load_k_mfma_t_paged(const DecodeArgs& a, const RowInfo& ri, int t, int lane,
                                                    uint32_t (&kb)[4][D / 32][4], const TilePages& pg) {
  typedef uint32_t v4u __attribute__((ext_vector_type(4)));
  constexpr bool F8 = DT == OC_FP8_E4M3FN;
  const int x = lane & 15;
  const int kg = lane >> 4;
  const int64_t ts = a.k_tok_stride;
  const int cofs = F8 ? kg * (D / 4) : 16 * kg;
  const int bmask = (1 << a.bs_log2) - 1;
  const int64_t head_off = (int64_t)ri.head * a.k_head_stride;
#pragma unroll
  for (int tb = 0; tb < 4; ++tb) {
    const int tok = kperm(16 * tb + x);
    const int hi = x >> 3;  // block 2 (tb / 2) + hi
    const int id = hi ? pg.id[2 * (tb >> 1) + 1] : pg.id[2 * (tb >> 1)];
    const int n = hi ? pg.n[2 * (tb >> 1) + 1] : pg.n[2 * (tb >> 1)];
    const bool ok = (tok & 15) < n;
    const char* rp = page_row(a.k, a.k_blk_stride, head_off, ts, ok ? id : -1, t * 64 + tok, bmask) + cofs;
#pragma unroll
    for (int dc = 0; dc < (F8 ? D / 64 : D / 32); ++dc) {
      const v4u v = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(rp + (F8 ? 16 : 64) * dc));
      kb[tb][dc][0] = ok ? v[0] : 0u;
      kb[tb][dc][1] = ok ? v[1] : 0u;
      kb[tb][dc][2] = ok ? v[2] : 0u;
      kb[tb][dc][3] = ok ? v[3] : 0u;
    }
  }
}

template <int DT, int D>
__device__ __forceinline__ void tile_logits_t(const uint32_t (&aq)[D / 32][4], const uint32_t (&kb)[4][D / 32][4],
                                              f32x4 (&c)[4], KDq kd = KDq{false, 1.f}) {
  auto run = [&](auto dq_tag) {
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
      c[tb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int dc = 0; dc < D / 32; ++dc) {
        uint32_t b[4];
        k_operand<DT, D>(kb, tb, dc, b, decltype(dq_tag)::value, kd.s);
        c[tb] = mfma_qk<MfmaT<DT>::value>(b, aq[dc], c[tb]);
      }
    }
  };
  if (DT == OC_FP8_E4M3FN && kd.on) run(std::true_type{});
  else run(std::false_type{});
}

// Online-softmax update of the lane's head from the tile's raw logits (c
// becomes the probabilities times vmul); base-2 units, as tile_softmax_regs
template <int D>
__device__ __forceinline__ void tile_softmax_t(MStateT& ms, f32x4 (&accp)[D / 16], f32x4 (&c)[4], float lscale,
                                               float vmul, int valid, int lane) {
  const int r = lane >> 4;
  const float lscale2 = lscale * 1.4426950408889634f;
  if (valid >= 64) {
#pragma unroll
    for (int tb = 0; tb < 4; ++tb)
#pragma unroll
      for (int i = 0; i < 4; ++i) c[tb][i] *= lscale2;
  } else {
#pragma unroll
    for (int tb = 0; tb < 4; ++tb)
#pragma unroll
      for (int i = 0; i < 4; ++i) c[tb][i] = kperm(16 * tb + 4 * r + i) < valid ? c[tb][i] * lscale2 : -__builtin_inff();
  }
  float mt = -__builtin_inff();
#pragma unroll
  for (int tb = 0; tb < 4; ++tb) mt = fmaxf(mt, fmaxf(fmaxf(c[tb][0], c[tb][1]), fmaxf(c[tb][2], c[tb][3])));
  mt = fmaxf(mt, xpair<16>(mt));
  mt = fmaxf(mt, xpair<32>(mt));
  const float mn = fmaxf(ms.m, mt);
  const float alpha = __builtin_amdgcn_exp2f(ms.m - mn);
  ms.m = mn;
  float ls = 0.f;
#pragma unroll
  for (int tb = 0; tb < 4; ++tb)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float pp = __builtin_amdgcn_exp2f(c[tb][i] - mn);
      ls += pp;
      c[tb][i] = pp;
    }
  ms.l = __builtin_fmaf(ms.l, alpha, ls);
  if (__builtin_amdgcn_ballot_w64(alpha != 1.f)) {
#pragma unroll
    for (int nc = 0; nc < D / 16; ++nc) accp[nc] *= alpha;
  }
  if (vmul != 1.f) {
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) c[tb] *= vmul;
  }
}

// O^T += V^T.P^T: A = V^T from the LDS tile (transposing reads, as
// tile_pv_mfma's B operand), B = the lane's own probabilities of block j
// (c[2j][0..3], c[2j + 1][0..3]: tokens 32j + 8kg .. + 7) as a 16-bit high
// part plus the 16-bit rounding of the remainder; accp[nc] lane 16r + x
// register i = output column 16nc + 4r + i of head x.
template <int DT, int D>
__device__ __forceinline__ void tile_pv_t(f32x4 (&accp)[D / 16], const f32x4 (&c)[4], const uint16_t* sv, int lane) {
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  const int x = lane & 15;
  const int kg = lane >> 4;
#pragma unroll
  for (int tb2 = 0; tb2 < 2; ++tb2) {
    float pv[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      pv[e] = c[2 * tb2][e];
      pv[4 + e] = c[2 * tb2 + 1][e];
    }
    uint32_t phi[4], plo[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if constexpr (MfmaT<DT>::value == OC_BF16) {
        const __bf16 h0 = (__bf16)pv[2 * e], h1 = (__bf16)pv[2 * e + 1];
        const __bf16 l0 = (__bf16)(pv[2 * e] - (float)h0), l1 = (__bf16)(pv[2 * e + 1] - (float)h1);
        phi[e] = (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
        plo[e] = (uint32_t)__builtin_bit_cast(uint16_t, l0) | ((uint32_t)__builtin_bit_cast(uint16_t, l1) << 16);
      } else {
        const _Float16 h0 = (_Float16)pv[2 * e], h1 = (_Float16)pv[2 * e + 1];
        const _Float16 l0 = (_Float16)(pv[2 * e] - (float)h0), l1 = (_Float16)(pv[2 * e + 1] - (float)h1);
        phi[e] = (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
        plo[e] = (uint32_t)__builtin_bit_cast(uint16_t, l0) | ((uint32_t)__builtin_bit_cast(uint16_t, l1) << 16);
      }
    }
    const int vrow = 32 * tb2 + 8 * kg + (x >> 2);
    const int vx = v_xor<DT, D>(vrow) >> 1;
    const uint16_t* rowp = sv + vrow * D + 4 * (x & 3);
    const int vrow8 = 32 * tb2 + 8 * kg + (x >> 1);
    const int vx8 = v_xor<DT, D>(vrow8);
    const uint8_t* rowp8 = reinterpret_cast<const uint8_t*>(sv) + vrow8 * D + 8 * (x & 1);
    // the transposing reads of four column blocks are issued before their
    // products, so that their latencies overlap (one read ahead of each
    // product left a wave waiting on LDS latency for most of the step; all
    // eight blocks of head_dim 128 ahead needed more than 256 registers)
    constexpr int NW = DT == OC_FP8_E4M3FN ? 2 : 4;
    constexpr int GS = D / 16 < 4 ? D / 16 : 4;
#pragma unroll
    for (int n0 = 0; n0 < D / 16; n0 += GS) {
      uint32_t raw[GS][NW];
#pragma unroll
      for (int j = 0; j < GS; ++j) {
        const int nc = n0 + j;
        if constexpr (DT == OC_FP8_E4M3FN) {
          typedef int i32x2 __attribute__((ext_vector_type(2)));
          const i32x2 b8 = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
              (__attribute__((address_space(3))) i32x2*)(rowp8 + 16 * (nc ^ vx8)));
          raw[j][0] = (uint32_t)b8[0];
          raw[j][1] = (uint32_t)b8[1];
        } else {
          const s16x4 b0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) s16x4*)(rowp + 16 * (nc ^ vx)));
          const s16x4 b1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) s16x4*)(rowp + 4 * D + 16 * (nc ^ vx)));
          typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
          const u32x2 w0 = __builtin_bit_cast(u32x2, b0), w1 = __builtin_bit_cast(u32x2, b1);
          raw[j][0] = w0[0];
          raw[j][1] = w0[1];
          raw[j][2] = w1[0];
          raw[j][3] = w1[1];
        }
      }
      __builtin_amdgcn_sched_barrier(0);  // keep the reads ahead of the products
#pragma unroll
      for (int j = 0; j < GS; ++j) {
        const int nc = n0 + j;
        uint32_t va[4];
        if constexpr (DT == OC_FP8_E4M3FN) {
          fp8x4_to_bf16(raw[j][0], va[0], va[1]);
          fp8x4_to_bf16(raw[j][1], va[2], va[3]);
        } else {
#pragma unroll
          for (int w = 0; w < 4; ++w) va[w] = raw[j][w];
        }
        accp[nc] = mfma_qk<MfmaT<DT>::value>(va, phi, accp[nc]);
        accp[nc] = mfma_qk<MfmaT<DT>::value>(va, plo, accp[nc]);
      }
    }
  }
}

// Retain decision for tile t of a row in cached mode from its stored
// energies; a partial tail tile is always retained.
__device__ __forceinline__ bool cached_keep(const DecodeArgs& a, const RowInfo& ri, int t, float el, float eh,
                                            float qmax, bool qnan) {
  if ((t + 1) * 64 > ri.n_tok && a.gate != OC_GATE_MASK) return true;
  return gate_keep(a.gate, a.thr, el, eh, qmax, qnan);
}

// The cached scores of tile t of a row (cached mode): (e_low, e_high) from
// the score cache, or for OC_GATE_MASK the given mask byte as e_high = 0 / 1.
__device__ __forceinline__ void cached_scores(const DecodeArgs& a, int row, int t, float& el, float& eh) {
  if (a.gate == OC_GATE_MASK) {
    eh = a.tmask[(int64_t)row * a.tmask_stride + t] ? 1.f : 0.f;
    el = 0.f;
    return;
  }
  const int64_t o = (int64_t)row * a.sc_stride + t;
  eh = a.sc_eh[o];
  el = a.gate == OC_GATE_ZETA ? a.sc_el[o] : 0.f;
}

// A workgroup's tile list: index x < n -> tile s + (x / w) * P + x % w
// (logical splits s .. s + w - 1 of P; or, with P = w = 1, the tile range
// [s, s + n)).
struct TileList {
  int s, w, P, n;
};

__device__ __forceinline__ TileList split_list(const DecodeArgs& a, const RowInfo& ri, int s) {
  TileList tl;
  tl.s = s;
  tl.P = a.P;
  tl.w = min(a.spw, a.P - s);
  tl.n = s < ri.n_tiles ? tl.w * ((ri.n_tiles - s + a.P - 1) / a.P) : 0;
  return tl;
}

__device__ __forceinline__ int row_tiles(const DecodeArgs& a, int r) { return (row_tokens(a, r) + 63) >> 6; }

// Flat workgroup layout for rows of different lengths.  With N tiles in all
// and n_max in the longest row, U = max(ceil(N / flat_target),
// ceil(n_max / qcap), 1) and row r gets q_r = max(1, ceil(n_r / U))
// workgroups; the rows' workgroups are numbered row after row over
// blockIdx.x.  Every workgroup recomputes the table (two passes over the
// rows' lengths) and finds its row, its index g among the row's q_r
// workgroups and the row's first slot.  Returns false for the slots past
// the last row's.  sh_i: 2 kDW + 8 ints of LDS.
template <int kDW>
__device__ __forceinline__ bool flat_map(const DecodeArgs& a, int qcap, int* sh_i, int& row, int& g, int& q,
                                         int& slot0) {
  constexpr int kDT = kDW * kWave;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int bid = blockIdx.x;
  int sum = 0, mx = 0;
  for (int r = threadIdx.x; r < a.num_rows; r += kDT) {
    const int n = row_tiles(a, r);
    sum += n;
    mx = max(mx, n);
  }
  sum = wave_incl_scan(sum);
  mx = (int)wave_max((float)mx);  // exact: a row has < 2^24 tiles
  if (threadIdx.x == 0) sh_i[2 * kDW + 4] = -1;
  if (lane == 63) sh_i[wave] = sum;
  if (lane == 0) sh_i[kDW + wave] = mx;
  __syncthreads();
  int total = 0, nmax = 0;
#pragma unroll
  for (int w = 0; w < kDW; ++w) {
    total += sh_i[w];
    nmax = max(nmax, sh_i[kDW + w]);
  }
  const int U = max(1, max((total + a.flat_target - 1) / a.flat_target, (nmax + qcap - 1) / qcap));
  int carry = 0;
  for (int c = 0; c < a.num_rows; c += kDT) {
    __syncthreads();  // sh_i[0 .. kDW) is reused
    const int r = c + threadIdx.x;
    const int qr = r < a.num_rows ? max(1, (row_tiles(a, r) + U - 1) / U) : 0;
    const int incl = wave_incl_scan(qr);
    if (lane == 63) sh_i[wave] = incl;
    __syncthreads();
    int before = carry, all = 0;
#pragma unroll
    for (int w = 0; w < kDW; ++w) {
      const int x = sh_i[w];
      before += w < wave ? x : 0;
      all += x;
    }
    const int first = before + incl - qr;
    if (qr > 0 && first <= bid && bid < first + qr) {
      sh_i[2 * kDW + 4] = r;
      sh_i[2 * kDW + 5] = bid - first;
      sh_i[2 * kDW + 6] = qr;
      sh_i[2 * kDW + 7] = first;
    }
    carry += all;
  }
  __syncthreads();
  row = sh_i[2 * kDW + 4];
  g = sh_i[2 * kDW + 5];
  q = sh_i[2 * kDW + 6];
  slot0 = sh_i[2 * kDW + 7];
  return row >= 0;
}

// Slots of flat_map_lpt's layout, a bound on its share count for w =
// flat_target and `rows` rows: the long shares number at most w pct / 100 and
// the short ones fewer than w (100 - pct) div / 100 + rows (div + 1).
__host__ __device__ inline int flat_lpt_slots(int w, int rows, int pct, int div) {
  return (int)((int64_t)w * pct / 100 + ((int64_t)w * (100 - pct) * div + 99) / 100 + (int64_t)rows * (div + 1) + 1);
}

// The flat layout of decode_fast_kernel, longest shares first.  With N
// tiles in all, n_max in the longest row and W = flat_target, shares are
// cut from U = max(ceil(N / W), ceil(n_max f / (qcap - div - 1)), 1) tiles,
// f = (pct + (100 - pct) div) / 100.  Row r (n_r tiles) gets
// b_r = floor(n_r pct / (100 U)) long shares, tiles [g U, (g + 1) U), and its
// other L_r = n_r - b_r U tiles are cut into s_r = ceil(L_r / V) short shares
// of about V = ceil(U / div) tiles (tiles b_r U + floor(L_r h / s_r) ..; an
// empty row gets one empty share).  blockIdx.x numbers every row's long
// shares, row after row, then every row's short shares, so the hardware
// dispatches the long shares first and the short ones fill the end of the
// step.  A workgroup gets its row, its share index g among the row's
// q = b_r + s_r shares (its partials' slot, <= qcap), the row's first slot
// and its tile range [b0, b1); false for the slots past the last share.
// Three passes over the rows: totals, long-share count, lookup; the
// lengths are read once (rows threadIdx.x + k kDT, k < 4, kept in
// registers; the rows past those are read again in each pass).  ntok: the
// row's tokens.  sh_i: 4 kDW + 9 ints of LDS.
template <int kDW>
__device__ __forceinline__ bool flat_map_lpt(const DecodeArgs& a, int qcap, int* sh_i, int& row, int& g, int& q,
                                             int& slot0, int& b0, int& b1, int& ntok) {
  constexpr int kDT = kDW * kWave;
  constexpr int kKeep = 4;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int bid = blockIdx.x;
  const int pct = a.flat_pct, div = a.flat_div;
  int kept_tok[kKeep];
#pragma unroll
  for (int k = 0; k < kKeep; ++k) {
    const int r = threadIdx.x + k * kDT;
    kept_tok[k] = r < a.num_rows ? row_tokens(a, r) : 0;
  }
  // tokens of row r = threadIdx.x + k kDT (0 past the last row)
  auto tokens = [&](int k, int r) -> int {
    if (r >= a.num_rows) return 0;
    if (k >= kKeep) return row_tokens(a, r);
    int n = kept_tok[0];
#pragma unroll
    for (int j = 1; j < kKeep; ++j) n = k == j ? kept_tok[j] : n;
    return n;
  };
  int sum = 0, mx = 0;
  for (int k = 0, r = threadIdx.x; r < a.num_rows; r += kDT, ++k) {
    const int n = (tokens(k, r) + 63) >> 6;
    sum += n;
    mx = max(mx, n);
  }
  sum = wave_incl_scan(sum);
  mx = (int)wave_max((float)mx);  // exact: a row has < 2^24 tiles
  if (threadIdx.x == 0) sh_i[4 * kDW + 4] = -1;
  if (lane == 63) sh_i[wave] = sum;
  if (lane == 0) sh_i[kDW + wave] = mx;
  __syncthreads();
  int total = 0, nmax = 0;
#pragma unroll
  for (int w = 0; w < kDW; ++w) {
    total += sh_i[w];
    nmax = max(nmax, sh_i[kDW + w]);
  }
  const int64_t f100 = pct + (int64_t)(100 - pct) * div;
  const int ucap = (int)(((int64_t)nmax * f100 + 100LL * (qcap - div - 1) - 1) / (100LL * (qcap - div - 1)));
  const int U = max(1, max((total + a.flat_target - 1) / a.flat_target, ucap));
  const int V = (U + div - 1) / div;
  auto cut = [&](int k, int r, int& nb, int& ns, int& n) {
    n = (tokens(k, r) + 63) >> 6;
    nb = (int)((int64_t)n * pct / (100LL * U));
    ns = r < a.num_rows ? (n == 0 ? 1 : (n - nb * U + V - 1) / V) : 0;
  };
  // pass 2: the number of long shares
  int nbs = 0;
  for (int k = 0, r = threadIdx.x; r < a.num_rows; r += kDT, ++k) {
    int nb, ns, n;
    cut(k, r, nb, ns, n);
    nbs += nb;
  }
  nbs = wave_incl_scan(nbs);
  __syncthreads();  // sh_i[0 .. 2 kDW) is reused
  if (lane == 63) sh_i[wave] = nbs;
  __syncthreads();
  int NB = 0;
#pragma unroll
  for (int w = 0; w < kDW; ++w) NB += sh_i[w];
  // pass 3: this slot's share
  int cb = 0, cs = 0, ca = 0;  // long, short and all shares of the rows before the chunk
  for (int c = 0; c < a.num_rows; c += kDT) {
    __syncthreads();  // sh_i[0 .. 3 kDW) is reused
    const int r = c + threadIdx.x;
    int nb, ns, n;
    cut(c / kDT, r, nb, ns, n);
    const int ib = wave_incl_scan(nb), is = wave_incl_scan(ns), ia = wave_incl_scan(nb + ns);
    if (lane == 63) {
      sh_i[wave] = ib;
      sh_i[kDW + wave] = is;
      sh_i[2 * kDW + wave] = ia;
    }
    __syncthreads();
    int pb = cb, ps = cs, pa = ca, tb = 0, ts = 0, ta = 0;
#pragma unroll
    for (int w = 0; w < kDW; ++w) {
      const int xb = sh_i[w], xs = sh_i[kDW + w], xa = sh_i[2 * kDW + w];
      pb += w < wave ? xb : 0;
      ps += w < wave ? xs : 0;
      pa += w < wave ? xa : 0;
      tb += xb;
      ts += xs;
      ta += xa;
    }
    const int fb = pb + ib - nb, fs = NB + ps + is - ns;  // first blockIdx of the row's long / short shares
    int gi = -1, lo = 0, hi = 0;
    if (nb > 0 && fb <= bid && bid < fb + nb) {
      gi = bid - fb;
      lo = gi * U;
      hi = lo + U;
    } else if (ns > 0 && fs <= bid && bid < fs + ns) {
      const int h = bid - fs;
      const int L = n - nb * U;
      gi = nb + h;
      lo = nb * U + (int)((int64_t)L * h / ns);
      hi = nb * U + (int)((int64_t)L * (h + 1) / ns);
    }
    if (gi >= 0) {
      sh_i[4 * kDW + 4] = r;
      sh_i[4 * kDW + 5] = gi;
      sh_i[4 * kDW + 6] = nb + ns;
      sh_i[4 * kDW + 7] = pa + ia - nb - ns;
      sh_i[3 * kDW] = lo;
      sh_i[3 * kDW + 1] = hi;
      sh_i[4 * kDW + 8] = tokens(c / kDT, r);
    }
    cb += tb;
    cs += ts;
    ca += ta;
  }
  __syncthreads();
  row = sh_i[4 * kDW + 4];
  g = sh_i[4 * kDW + 5];
  q = sh_i[4 * kDW + 6];
  slot0 = sh_i[4 * kDW + 7];
  b0 = sh_i[3 * kDW];
  b1 = sh_i[3 * kDW + 1];
  ntok = sh_i[4 * kDW + 8];
  return row >= 0;
}

// The tile loop, the wave merge and the partial-state write of one
// workgroup (see decode_kernel).
template <int DT, int D, int GT, bool DOT2, bool PAGED, bool MQK, bool LOOP>
__device__ __forceinline__ void decode_body(const DecodeArgs& a, const RowInfo& ri, int row, const TileList& tl, int g0,
                                            float qmax, bool qnan, const float* sh_qf,
                                            const uint32_t* sh_qp, float (*sh_m)[GT], float (*sh_l)[GT],
                                            float (*sh_acc)[GT][D], int* sh_cnt, float pre_el, float pre_eh,
                                            const uint64_t* sh_bits, int wpre, int r0, int r1, float* sh_p,
                                            uint16_t* sh_v, uint8_t* sh_keep) {
  constexpr int CPL = D / 16;
  constexpr int kDW = DecWaves<DT, D, MQK, GT>::value;
  constexpr int kPH = GT > 4 ? 8 : 4;  // heads per P slot row block (MQK)
  using L = Lay<DT, D>;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int j = lane & 15;
  const bool cached = a.mode == OC_MODE_CACHED && a.gate != OC_GATE_NONE;
  // this workgroup's tile list: index x < n -> tile s + (x / w) * P + x % w
  const int s = tl.s, w = tl.w, n_split = tl.n;

  WaveState<GT> st;
  float acc[GT][CPL];
#pragma unroll
  for (int g = 0; g < GT; ++g) {
    st.m[g] = kM0;
    st.l[g] = 0.f;
#pragma unroll
    for (int c = 0; c < CPL; ++c) acc[g][c] = 0.f;
  }

  MState ms;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    ms.m[i] = kM0;
    ms.l[i] = 0.f;
  }
  // the transposed step: matrix cores, every listed tile attended, contiguous rows
  constexpr bool kT = MQK && LOOP && !PAGED;
  MStateT mst{kM0, 0.f};
  uint32_t aq[MQK ? D / 32 : 1][4];
  if constexpr (MQK) load_q_mfma<DT, D, GT>(sh_qp, lane, aq);
  float* sp = sh_p + wave * 64 * kPH;     // this wave's p[head][token] slot (MQK)
  uint16_t* sv = sh_v + wave * 64 * D;    // this wave's V tile slot (MQK)
  f32x4 accp[MQK ? D / 16 : 1];
#pragma unroll
  for (int nc = 0; nc < (MQK ? D / 16 : 1); ++nc) accp[nc] = f32x4{0.f, 0.f, 0.f, 0.f};

  uint32_t vw[16][L::LW];
  int kept = 0;
  int kk = wave - kDW;  // single-pass position in the group's tile list
  uint64_t cmask = 0;      // cached: retained tiles of the current 64-entry chunk
  int c0 = -64, rank = 0;
  int rb = r0 + wave - kDW, wc = 0;  // balanced: retained rank, bitmask word
  // next tile of this wave, or -1: every tile of the list round-robin
  // (single-pass, dense), every retained tile round-robin (cached), or the
  // retained tiles of ranks r0 + wave, r0 + wave + 4, ... < r1 (balanced)
  auto next_tile = [&]() -> int {
    int t = -1;
    if (a.bal) {
      if (rb < r0) {
        rb += kDW;  // the wave's first rank: r0 + wave
      } else {
        // later ranks from the workgroup's LDS counter, so that waves whose
        // tiles arrived sooner take more of them
        int x = 0;
        if (lane == 0) x = atomicAdd(&sh_cnt[kDW], 1);
        rb = r0 + __builtin_amdgcn_readfirstlane(x);
      }
      if (rb < r1) {
        // lane group holding rank rb: the first lane whose inclusive prefix
        // exceeds rb; then the word inside its four
        const int lg = __popcll((unsigned long long)__ballot(wpre <= rb));
        int base = __builtin_amdgcn_readlane(wpre, lg);
        wc = 4 * lg + 3;
        uint64_t bits = sh_bits[wc];
        base -= __popcll((unsigned long long)bits);
        for (int q = 2; q >= 0 && base > rb; --q) {
          bits = sh_bits[4 * lg + q];
          wc = 4 * lg + q;
          base -= __popcll((unsigned long long)bits);
        }
        const int k = rb - base;
        // the k-th set bit of bits: the lane whose bit is set with k set bits below it
        const int below = __builtin_amdgcn_mbcnt_hi((uint32_t)(bits >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bits, 0u));
        const bool hit = ((bits >> lane) & 1ull) && below == k;
        t = wc * 64 + __ffsll((unsigned long long)__ballot(hit)) - 1;
      }
    } else if (!cached) {
      for (;;) {
        if (MQK && kk >= 0) {
          // matrix-core single pass and dense: after the wave's first tile
          // (position `wave`), list positions are handed out in LDS, so a
          // wave whose tiles arrived sooner (or were evicted, cheaper) takes
          // more of them
          int x = 0;
          if (lane == 0) x = atomicAdd(&sh_cnt[kDW], 1);
          kk = __builtin_amdgcn_readfirstlane(x);
        } else {
          kk += kDW;
        }
        if (kk >= n_split) break;
        t = s + (kk / w) * tl.P + kk % w;
        if (t < ri.n_tiles) break;
        t = -1;
      }
    } else {
      for (;;) {
        if (cmask) {
          const int bit = __ffsll((unsigned long long)cmask) - 1;
          cmask &= cmask - 1;
          if ((rank++ & (kDW - 1)) == wave) {
            const int x = c0 + bit;
            t = s + (x / w) * tl.P + x % w;
            break;
          }
          continue;
        }
        c0 += 64;
        if (c0 >= n_split) break;
        const int kx = c0 + lane;
        const int tx = s + (kx / w) * tl.P + kx % w;
        const bool in = kx < n_split && tx < ri.n_tiles;
        float el = pre_el, eh = pre_eh;
        if (c0 > 0 && in) cached_scores(a, row, tx, el, eh);
        const bool keep = in && cached_keep(a, ri, tx, el, eh, qmax, qnan);
        if (a.keep_out && in && wave == 0 && blockIdx.z == 0)
          a.keep_out[(int64_t)row * a.keep_stride + tx] = keep ? 1 : 0;
        cmask = __ballot(keep);
      }
    }
    return __builtin_amdgcn_readfirstlane(t);  // the tile index is wave-uniform
  };
  auto lscale_of = [&](int t) -> float {
    return a.scale * (a.k_scale_mode == OC_KSCALE_TILE ? a.k_scales[(int64_t)row * a.ks_stride + t] : 1.f);
  };

  if constexpr (MQK) {
    static_assert(GT <= 8, "the matrix-core path keeps the heads in lane rows 0 and 1");
    uint32_t kb[4][D / 32][4];
    // a block id outside the pool (paged): raised once after the loop, so no
    // global atomic sits among the tile loads
    bool bad_page = false;
    if constexpr (kT) {
      // cached or dense decode on contiguous rows: the transposed step
      for (int t = next_tile(); t >= 0; t = next_tile()) {
        const int valid = min(64, ri.n_tok - t * 64);
        load_k_mfma_t<DT, D>(a, ri, row, t, lane, kb);
        load_v_lds<DT, D, PAGED>(a, ri, row, t, lane, sv, TilePages{});
        f32x4 c[4];
        tile_logits_t<DT, D>(aq, kb, c);
        tile_softmax_t<D>(mst, accp, c, lscale_of(t), tile_vmul(a, row, t), valid, lane);
        // the V tile's direct-to-LDS loads (issued after K) have landed
        __builtin_amdgcn_s_waitcnt(0);
        tile_pv_t<DT, D>(accp, c, sv, lane);
        ++kept;
      }
    } else if constexpr (LOOP) {
      // cached or dense decode (LOOP, fixed at launch: the same condition as
      // cached || gate == NONE): every listed tile is attended
      for (int t = next_tile(); t >= 0; t = next_tile()) {
        const int valid = min(64, ri.n_tok - t * 64);
        TilePages pg{};
        if constexpr (PAGED) pg = tile_pages(a, ri, t, bad_page);
        load_k_mfma<DT, D, PAGED>(a, ri, row, t, lane, kb, pg);
        load_v_lds<DT, D, PAGED>(a, ri, row, t, lane, sv, pg);
        tile_softmax_mfma<DT, D, GT>(ms, accp, aq, kb, sp, lscale_of(t), tile_vmul(a, row, t), valid, lane);
        // the V tile's direct-to-LDS loads (issued after K) have landed
        __builtin_amdgcn_s_waitcnt(0);
        tile_pv_mfma<DT, D, GT>(accp, sp, sv, lane);
        ++kept;
      }
    } else {
      // single pass: gate every K tile of the list; V only for retained
      // tiles.  The next K tile is requested as soon as the current one has
      // been consumed (logits and energies), so it streams in while this
      // tile's V lands and p.V runs.  Keep flags go to LDS (sh_keep, list
      // order) and are written out after the loop: a global store pending
      // among the loads would make every wait a full one.
      constexpr int kNK = 4 * (D / 32);  // K loads per tile
      const bool keep_lds = n_split <= kKeepLds;
      // one copy of the loop per gate (E_low only for the zeta gate): the
      // two in one loop body overflow the register budget
      auto single_pass = [&](auto low_tag) {
        constexpr bool LOW = decltype(low_tag)::value;
        int t = next_tile();
        TilePages pg{};
        if (t >= 0) {
          if constexpr (PAGED) pg = tile_pages(a, ri, t, bad_page);
          load_k_mfma<DT, D, PAGED>(a, ri, row, t, lane, kb, pg);
        }
        while (t >= 0) {
          const int valid = min(64, ri.n_tok - t * 64);
          // per-tile scales first: a load issued after the V and K requests
          // below would make its wait a wait for all of them
          const float kmul = tile_kdeq(a, row, t).mul;
          const float lsc = a.scale * kmul;  // = lscale_of(t)
          const float vmul = tile_vmul(a, row, t);
          f32x4 lg[4];
          tile_logits_mfma<DT, D>(aq, kb, lg);
          bool keep = true;
          if (valid == 64) {
            float el, eh;
            tile_energies_mfma<DT, D, LOW>(kb, lane, kmul, el, eh);
            keep = gate_keep(a.gate, a.thr, el, eh, qmax, qnan);
          }
          keep = __builtin_amdgcn_readfirstlane(keep ? 1 : 0) != 0;
          if (a.keep_out && blockIdx.z == 0) {
            if (keep_lds) {
              if (lane == 0) sh_keep[kk] = keep ? 1 : 0;
            } else if (lane == 0) {
              a.keep_out[(int64_t)row * a.keep_stride + t] = keep ? 1 : 0;
            }
          }
          if (keep) load_v_lds<DT, D, PAGED>(a, ri, row, t, lane, sv, pg);
          __builtin_amdgcn_sched_barrier(0);
          const int tn = next_tile();
          if (tn >= 0) {
            if constexpr (PAGED) pg = tile_pages(a, ri, tn, bad_page);
            load_k_mfma<DT, D, PAGED>(a, ri, row, tn, lane, kb, pg);
          }
          __builtin_amdgcn_sched_barrier(0);
          if (keep) {
            tile_softmax_regs<DT, D, GT>(ms, accp, lg, sp, lsc, vmul, valid, lane);
            // the V tile has landed once at most the next tile's K loads
            // (issued after it) are outstanding
            if (tn >= 0) __builtin_amdgcn_s_waitcnt(vmcnt_imm(kNK));
            else __builtin_amdgcn_s_waitcnt(0);
            tile_pv_mfma<DT, D, GT>(accp, sp, sv, lane);
            ++kept;
          }
          t = tn;
        }
      };
      if (a.gate == OC_GATE_ZETA) single_pass(std::true_type{});
      else single_pass(std::false_type{});
    }
    if (PAGED && bad_page && a.error_flag && lane == 0) atomicOr(a.error_flag, 1);
  } else {
    uint32_t kw[16][L::LW];
    float p[GT];
    for (int t = next_tile(); t >= 0; t = next_tile()) {
      const int valid = min(64, ri.n_tok - t * 64);
      load_tile<DT, D, PAGED>(a, ri, row, t, false, lane, kw);
      bool keep = true;
      if (!cached && a.gate != OC_GATE_NONE) {
        // single pass: gate on the K tile just read; V is read only if kept
        if (valid == 64) {
          float el, eh;
          tile_energies<DT, D>(kw, tile_kdeq(a, row, t), lane, el, eh);
          keep = gate_keep(a.gate, a.thr, el, eh, qmax, qnan);
        }
        if (a.keep_out && lane == 0 && blockIdx.z == 0)
          a.keep_out[(int64_t)row * a.keep_stride + t] = keep ? 1 : 0;
      }
      if (keep) {
        load_tile<DT, D, PAGED>(a, ri, row, t, true, lane, vw);
        tile_softmax<DT, D, GT, DOT2>(st, acc, p, kw, sh_qf, sh_qp, lscale_of(t), tile_vmul(a, row, t), valid, lane);
        tile_pv<DT, D, GT>(acc, p, vw);
        ++kept;
      }
    }
  }

  // wave -> LDS: l summed over lanes, acc summed over the 4 token groups
  float lsum_t = 0.f;
  if constexpr (kT) {
    // head x's state in lanes x, x + 16, x + 32, x + 48; its output
    // columns 16nc + 4r + i in lane 16r + x, register i
    lsum_t = mst.l + xpair<16>(mst.l);
    lsum_t += xpair<32>(lsum_t);
    float* ao = reinterpret_cast<float*>(sv);
    const int x = lane & 15;
    const int r = lane >> 4;
    if (x < GT) {
#pragma unroll
      for (int nc = 0; nc < D / 16; ++nc)
#pragma unroll
        for (int i = 0; i < 4; ++i) ao[x * D + 16 * nc + 4 * r + i] = accp[nc][i];
    }
  }
#pragma unroll
  for (int g = 0; g < GT; ++g) {
    float mg, lt;
    if constexpr (kT) {
      mg = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mst.m), g));
      if (mg != kM0) mg *= 0.6931471805599453f;
      lt = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lsum_t), g));
    } else if constexpr (MQK) {
      // head g: register g % 4 of the lanes of row g / 4; the p.V result of
      // head g, column 16nc + x sits in lane 16 (g / 4) + x, register g % 4 of
      // accp[nc].  It goes to the wave's (now idle) V slot.
      mg = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ms.m[g & 3]), 16 * (g >> 2)));
      // base-2 units back to natural ones; an empty state keeps kM0
      if (mg != kM0) mg *= 0.6931471805599453f;
      lt = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(row16_sum(ms.l[g & 3])), 16 * (g >> 2)));
      float* ao = reinterpret_cast<float*>(sv);
#pragma unroll
      for (int nc = 0; nc < D / 16; ++nc)
        if ((lane >> 4) == (g >> 2)) ao[g * D + 16 * nc + (lane & 15)] = accp[nc][g & 3];
    } else {
      mg = st.m[g];
      lt = wave_sum(st.l[g]);
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        const float x = rows4_sum(acc[g][c]);
        if (lane < 16) sh_acc[wave][g][j * CPL + c] = x;
      }
    }
    if (lane == 0) {
      sh_m[wave][g] = mg;
      sh_l[wave][g] = lt;
    }
  }
  if (lane == 0) sh_cnt[wave] = kept;
}

// The attend-every-tile transposed step on contiguous rows, or on pages of
// >= 16 tokens (block-table entries of a wave's next tile requested before
// its current tile is computed), with a short prologue (a.fast):
// cached decode with a score gate (at most
// 64 * kFastChunks tiles per row) or dense decode, q of the matrix-core type,
// all G <= GT query heads of a row in one workgroup.  Every wave loads the
// matrix-core q operand and forms the row's q norms; cached, wave w gates the
// 64-tile chunks w, w + kDW, ... of the tile range [b0, b1) and publishes
// their keep bits in LDS, and after one barrier every wave holds the range's
// retained-tile bitmask (lane c: the bits of tiles b0 + 64c .. + 63, with
// their inclusive prefix counts over the lanes).  From it each wave forms the
// workgroup's even share [r0, r1) of the range's retained tiles (dense: of
// its tiles; share gidx of npg) and its first rank r0 + wave.  It issues that
// tile's K and V loads before a second barrier, which publishes the LDS
// counter the later ranks are drawn from (a wave whose tiles arrived sooner
// takes more).
// The wave's state goes to LDS as decode_body leaves it.
template <int DT, int D, int GT, bool PAGED, int kDW, int VT>
__device__ __forceinline__ void decode_fast(const DecodeArgs& a, const RowInfo& ri, int row, int gidx, int npg, int b0, int b1,
                                            float (*sh_m)[GT], float (*sh_l)[GT], int* sh_cnt, uint16_t* sh_v) {
  constexpr bool F8 = DT == OC_FP8_E4M3FN;
  constexpr int QT = MfmaT<DT>::value;  // q's 16-bit type
  static_assert(GT <= 16, "one q head per 16-lane group of the operand");
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int x = lane & 15, kg = lane >> 4;
  const bool cached = a.mode == OC_MODE_CACHED && a.gate != OC_GATE_NONE;

  // q operand (B of S^T = K.q^T): lane 16 kg + x holds q[head x] columns
  // 32 dc + 8 kg .. + 8 (fp8 K: kg D / 4 + 8 dc ..), zero past G; one 16-byte
  // load per instruction column block, straight from q
  uint32_t aq[D / 32][4];
  auto load_q = [&]() {
    const char* qh = a.q + ((int64_t)row * a.G + x) * a.q_row_stride;
#pragma unroll
    for (int dc = 0; dc < D / 32; ++dc) {
      const int e0 = F8 ? kg * (D / 4) + 8 * dc : 32 * dc + 8 * kg;
      uint4 v = make_uint4(0u, 0u, 0u, 0u);
      if (x < a.G) v = *reinterpret_cast<const uint4*>(qh + 2 * e0);
      aq[dc][0] = v.x;
      aq[dc][1] = v.y;
      aq[dc][2] = v.z;
      aq[dc][3] = v.w;
    }
  };

  // cached: the row's keep flags, lane c holding the bits of chunk c.  One
  // copy of the pass per gate, with the gate's tests compiled in.  On ranges
  // of more than two chunks (shared) wave w gates chunks w + k kDW (k <
  // kCPW), whose scores are all requested before q, so that their latency
  // overlaps q's (indices clamped into the row), and writes each chunk's 64
  // keep bits to sh_keep; one barrier then publishes them to every wave.
  // (Every wave gating the whole range by itself, with no barrier, read each
  // score line kDW times per workgroup and took about 1.8 us longer per
  // workgroup at 512 tiles per row.)  On one or two chunks every wave gates
  // them all itself, with no barrier.
  const int nch = (b1 - b0 + 63) >> 6;
  uint32_t wlo = 0u, whi = 0u;
  __shared__ uint64_t sh_keep[kFastChunks];
  __shared__ float sh_hk[kDW][3];
  auto score_pass = [&](auto gate_tag) {
    constexpr int GATE = decltype(gate_tag)::value;
    constexpr bool HOOK = GATE == kGateHook;
    constexpr int kCPW = (kFastChunks + kDW - 1) / kDW;
    static_assert(kCPW >= 2, "the unshared pass gates two chunks");
    const bool shared = nch > 2;
    const int64_t so = (int64_t)row * a.sc_stride;
    float el[kCPW], eh[kCPW];
#pragma unroll
    for (int k = 0; k < kCPW; ++k) {
      const int c = shared ? wave + k * kDW : k;
      el[k] = 0.f;
      eh[k] = 0.f;
      if (c < nch) {
        const int t = min(b0 + c * 64 + lane, b1 - 1);
        if constexpr (HOOK) {
          // the complete tiles' norms (a partial tail reads the last one's)
          eh[k] = a.hk_norms[(int64_t)(row % a.hk_rows) * a.hk_stride + min(t, a.hk_full - 1)];
        } else if constexpr (GATE == OC_GATE_MASK) {
          eh[k] = a.tmask[(int64_t)row * a.tmask_stride + t] ? 1.f : 0.f;
        } else {
          eh[k] = a.sc_eh[so + t];
          if constexpr (GATE == OC_GATE_ZETA) el[k] = a.sc_el[so + t];
        }
      }
    }
    load_q();
    // max over the row's G heads of ||q_g||_2 (CS gate; norms below 1e-38
    // count as 0): head x's squares summed over its four lane groups
    float qmax = 0.f;
    bool qnan = false;
    if constexpr (GATE == OC_GATE_CS) {
      float ss = 0.f;
#pragma unroll
      for (int dc = 0; dc < D / 32; ++dc)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          float lo, hi;
          unpack16x2<QT>(aq[dc][w], lo, hi);
          ss = __builtin_fmaf(lo, lo, __builtin_fmaf(hi, hi, ss));
        }
      ss += xpair<16>(ss);
      ss += xpair<32>(ss);
      float qn = __builtin_sqrtf(ss);
      if ((double)qn < 1e-38) qn = 0.f;
      const bool head = x < a.G;
      qnan = __ballot(head && __builtin_isnan(qn)) != 0;
      float qv = head && !__builtin_isnan(qn) ? qn : 0.f;
      qv = fmaxf(qv, xpair<8>(qv));
      qv = fmaxf(qv, xpair<4>(qv));
      qv = fmaxf(qv, xpair<2>(qv));
      qv = fmaxf(qv, xpair<1>(qv));
      qmax = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(qv)));
    }
    float qn = 0.f;  // hook: the group's median Walsh-subspace norm
    if constexpr (HOOK) {
      static_assert(!F8, "the hook gate reads q in K's 16-bit layout");
      // head x: ||q||^2 - sum_i S_i^2 / bs over the 8 blocks of bs = D / 8
      // columns (S_i: block sums), from the lane's columns 32 dc + 8 kg .. +8
      float ss = 0.f, sp[D / 32];
#pragma unroll
      for (int dc = 0; dc < D / 32; ++dc) {
        float s = 0.f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          float lo, hi;
          unpack16x2<QT>(aq[dc][w], lo, hi);
          s += lo + hi;
          ss = __builtin_fmaf(lo, lo, __builtin_fmaf(hi, hi, ss));
        }
        sp[dc] = s;
      }
      ss += xpair<16>(ss);
      ss += xpair<32>(ss);
      float lsq = 0.f;
      if constexpr (D == 128) {
        // block 2 dc + kg / 2: lane groups kg and kg ^ 1 hold its halves
#pragma unroll
        for (int dc = 0; dc < D / 32; ++dc) {
          const float s = sp[dc] + xpair<16>(sp[dc]);
          lsq = __builtin_fmaf(s, s, lsq);
        }
        lsq += xpair<32>(lsq);
      } else {
        // block 4 dc + kg: the lane's eight columns
#pragma unroll
        for (int dc = 0; dc < D / 32; ++dc) lsq = __builtin_fmaf(sp[dc], sp[dc], lsq);
        lsq += xpair<16>(lsq);
        lsq += xpair<32>(lsq);
      }
      float h2 = ss - lsq / (float)(D / 8);
      h2 = h2 < 0.f ? 0.f : h2;
      const float qh = __builtin_sqrtf(h2);
      // the element of rank G / 2 of the G norms (ties by head index), as
      // oc_group_gate's median
      int below = 0;
      for (int g = 0; g < a.G; ++g) {
        const float v = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(qh), g));
        below += (v < qh || (v == qh && g < x)) ? 1 : 0;
      }
      const uint64_t pick = __ballot(kg == 0 && x < a.G && below == a.G / 2);
      // none when a NaN breaks the ranks: 0, as oc_group_gate
      qn = pick ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(qh), __ffsll((unsigned long long)pick) - 1))
                : 0.f;
    }
    float nev = 0.f, kmax = -__builtin_inff();
    bool knan = false;
    const bool keep_wr = a.keep_out && gidx == 0;
#pragma unroll
    for (int k = 0; k < kCPW; ++k) {
      const int c = shared ? wave + k * kDW : k;
      if (c < nch) {
        const int t = b0 + c * 64 + lane;
        // cached_keep with the gate fixed: a partial last tile is kept
        // (score gates), the mask byte decides (mask gate)
        bool keep;
        if constexpr (HOOK) {
          const bool full = t < a.hk_full;
          const bool ev = full && (double)qn * (double)eh[k] <= a.hk_tau;
          keep = !ev && t < b1;
          if (full) {
            nev += ev ? 1.f : 0.f;
            kmax = fmaxf(kmax, eh[k]);
            knan = knan || __builtin_isnan(eh[k]);
          }
        } else {
          keep = gate_keep(GATE, a.thr, el[k], eh[k], qmax, qnan);
          if constexpr (GATE != OC_GATE_MASK) keep = keep || (t + 1) * 64 > ri.n_tok;
          keep = keep && t < b1;
        }
        const uint64_t m = __ballot(keep);
        if (shared) {
          if (lane == 0) sh_keep[c] = m;
        } else if (lane == c) {
          wlo = (uint32_t)m;
          whi = (uint32_t)(m >> 32);
        }
        // the keep flags, by the row's first workgroup (unshared: chunk c by
        // wave c)
        if (keep_wr && (shared || c == wave) && t < b1) a.keep_out[(int64_t)row * a.keep_stride + t] = keep ? 1 : 0;
      }
    }
    // the wave's statistics (hook gate): evicted complete tiles, the largest
    // complete tile's norm, whether one is NaN; shared: of its chunks
    bool wnan = false;
    if constexpr (HOOK) {
      nev = wave_sum(nev);
      kmax = wave_max(kmax);
      wnan = __ballot(knan) != 0;
      if (shared && lane == 0) {
        sh_hk[wave][0] = nev;
        sh_hk[wave][1] = kmax;
        sh_hk[wave][2] = wnan ? 1.f : 0.f;
      }
    }
    if (shared) {
      // publish the chunks' keep bits with a bare barrier after the LDS
      // stores have completed (loads still in flight, such as the paged
      // block-table entries, stay in flight across it); the signal fences
      // keep the compiler from moving LDS accesses across it
      __builtin_amdgcn_s_waitcnt(kLgkmOnly);
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      __builtin_amdgcn_s_barrier();
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      if (lane < min(nch, kFastChunks)) {
        const uint64_t m = sh_keep[lane];
        wlo = (uint32_t)m;
        whi = (uint32_t)(m >> 32);
      }
    }
    if constexpr (HOOK) {
      // the row's statistics, by wave 0 of its first workgroup: evicted
      // complete tiles, the group norm and the largest complete tile's norm
      // (NaN if one is NaN, -inf if there are none)
      if (a.hk_stats && gidx == 0 && wave == 0 && lane == 0) {
        float ev = nev, mx = kmax;
        bool nan = wnan;
        if (shared) {
          ev = 0.f;
          mx = -__builtin_inff();
          nan = false;
          for (int w = 0; w < kDW; ++w) {
            ev += sh_hk[w][0];
            mx = fmaxf(mx, sh_hk[w][1]);
            nan = nan || sh_hk[w][2] != 0.f;
          }
        }
        float* o = a.hk_stats + (int64_t)row * 3;
        o[0] = ev;
        o[1] = qn;
        o[2] = nan ? __builtin_nanf("") : mx;
      }
    }
  };
  // paged: the block-table entries of the range's first 16 tiles (lane 4 d
  // + j: tile b0 + d, 16-token block j; tokens past the row read its last
  // block's entry), requested with the scores, so that a wave whose first
  // tile is among them needs no further round trip before its K and V
  int spec_ids = 0;
  if constexpr (PAGED) {
    if (ri.n_tok > 0) {
      const int tok = min(b0 * 64 + 16 * lane, ri.n_tok - 1);
      spec_ids = a.bt[(int64_t)ri.seq * a.bt_stride + (tok >> a.bs_log2)];
    }
  }
  if (!cached) load_q();
  else if (a.gate == OC_GATE_CS) score_pass(std::integral_constant<int, OC_GATE_CS>{});
  else if (!F8 && (D == 64 || D == 128) && a.gate == kGateHook)
    score_pass(std::integral_constant<int, (F8 || (D != 64 && D != 128)) ? OC_GATE_CS : kGateHook>{});
  else if (a.gate == OC_GATE_ZETA) score_pass(std::integral_constant<int, OC_GATE_ZETA>{});
  else score_pass(std::integral_constant<int, OC_GATE_MASK>{});
  const int cnt = __popc(wlo) + __popc(whi);
  const int pre = wave_incl_scan(cnt);
  const int total = cached ? __builtin_amdgcn_readlane(pre, 63) : b1 - b0;
  const int r0 = (int)((int64_t)total * gidx / npg);
  const int r1 = (int)((int64_t)total * (gidx + 1) / npg);
  // the tile of retained rank rb (cached) or tile rb (dense); wave-uniform
  auto tile_of_rank = [&](int rb) -> int {
    if (!cached) return b0 + rb;
    const int lg = __popcll((unsigned long long)__ballot(pre <= rb));  // chunk holding rank rb
    const int base = __builtin_amdgcn_readlane(pre, lg) - __builtin_amdgcn_readlane(cnt, lg);
    const uint64_t bits = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)whi, lg) << 32) |
                          (uint32_t)__builtin_amdgcn_readlane((int)wlo, lg);
    const int k = rb - base;
    const int below = __builtin_amdgcn_mbcnt_hi((uint32_t)(bits >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bits, 0u));
    const bool hit = ((bits >> lane) & 1ull) && below == k;
    return __builtin_amdgcn_readfirstlane(b0 + lg * 64 + __ffsll((unsigned long long)__ballot(hit)) - 1);
  };
  // One tile per wave step.  (Two fp8 tiles per step, which fill the
  // register and LDS footprint of one 16-bit tile, measured slower on 32 rows
  // of 2048 fp8 tiles: 110.6 us cached and 174.9 dense against 104.0 and
  // 166.6.)
  // A tile's per-tile K and V scales (fp8) are requested before its K and V,
  // so the wait for K covers them; without per-tile scales a valid word (q)
  // is read and 1 selected, keeping the loads unconditional.
  const bool ks_tile = a.k_scale_mode == OC_KSCALE_TILE, vs_tile = a.v_scale_mode == OC_VSCALE_TILE;
  const float* qword = reinterpret_cast<const float*>(a.q);
  float ks_raw = 1.f, vs_raw = 1.f;
  uint32_t kb[4][D / 32][4];
  uint16_t* sv = sh_v + wave * 64 * D;  // this wave's V slot
  TilePages pg{};
  bool bad_page = false;
  // paged: the block-table entries of tile tt's four 16-token blocks, one
  // unconditional vector load (lane j < 4: block j; blocks past the row read
  // its last block's entry, unused), which the caller waits for
  auto request_pages = [&](int tt) -> int {
    if constexpr (PAGED) {
      const int tok = min(tt * 64 + 16 * min(lane, 3), ri.n_tok - 1);
      return a.bt[(int64_t)ri.seq * a.bt_stride + (tok >> a.bs_log2)];
    }
    return 0;
  };
  auto take_pages = [&](int tt, int ids) {
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
      const int tok = tt * 64 + 16 * tb;
      int n = min(max(ri.n_tok - tok, 0), 16);
      int id = __builtin_amdgcn_readlane(ids, tb);
      if (n > 0 && (id < 0 || id >= a.num_blocks)) {
        bad_page = true;
        n = 0;
      }
      pg.id[tb] = n > 0 ? id : -1;
      pg.n[tb] = n;
    }
  };
  auto issue = [&](int tt) {
    ks_raw = *(ks_tile ? a.k_scales + (int64_t)row * a.ks_stride + tt : qword);
    vs_raw = *(vs_tile ? a.v_scales + (int64_t)row * a.vs_stride + tt : qword);
    if constexpr (PAGED) {
      load_k_mfma_t_paged<DT, D>(a, ri, tt, lane, kb, pg);
      load_v_lds<VT, D, true>(a, ri, row, tt, lane, sv, pg);
    } else {
      load_k_mfma_t<DT, D>(a, ri, row, tt, lane, kb);
      load_v_lds<VT, D, false>(a, ri, row, tt, lane, sv, TilePages{});
    }
  };
  MStateT mst{kM0, 0.f};
  f32x4 accp[D / 16];
#pragma unroll
  for (int nc = 0; nc < D / 16; ++nc) accp[nc] = f32x4{0.f, 0.f, 0.f, 0.f};
  int kept = 0;
  int t = r0 + wave < r1 ? tile_of_rank(r0 + wave) : -1;
  if (t >= 0) {
    if constexpr (PAGED) {
      int ids;
      if (t - b0 < 16) {
        ids = __shfl(spec_ids, 4 * (t - b0) + (lane & 3));
      } else {
        ids = request_pages(t);
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
      }
      take_pages(t, ids);
    }
    issue(t);
  }
  // publish the LDS rank counter with a bare barrier after the counter's
  // store has completed, so that the first tile's K and V loads stay in
  // flight across it (a fenced barrier, even an LDS-only one, waits for them:
  // V is loaded straight into LDS).  The signal fences keep the compiler from
  // moving LDS accesses across the barrier.
  if (threadIdx.x == 0) sh_cnt[kDW] = kDW;
  __builtin_amdgcn_s_waitcnt(kLgkmOnly);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  while (t >= 0) {
    // paged: the next rank is claimed first and its block-table entries
    // requested, so that they arrive while this tile is computed
    int tn = -1, ids = 0;
    if constexpr (PAGED) {
      int xr = 0;
      if (lane == 0) xr = atomicAdd(&sh_cnt[kDW], 1);
      const int rb = r0 + __builtin_amdgcn_readfirstlane(xr);
      tn = rb < r1 ? tile_of_rank(rb) : -1;
      if (tn >= 0) ids = request_pages(tn);
    }
    const int valid = min(64, ri.n_tok - t * 64);
    f32x4 c[4];
    tile_logits_t<DT, D>(aq, kb, c, k_dq(a));
    tile_softmax_t<D>(mst, accp, c, a.scale * (ks_tile ? ks_raw : 1.f), vs_tile ? vs_raw : 1.f, valid, lane);
    // the V tile's direct-to-LDS loads (issued after K) have landed; paged,
    // the next tile's block-table load (issued last) may still be in flight
    if (PAGED && tn >= 0) __builtin_amdgcn_s_waitcnt(vmcnt_imm(1));
    else __builtin_amdgcn_s_waitcnt(0);
    tile_pv_t<VT, D>(accp, c, sv, lane);
    ++kept;
    if constexpr (PAGED) {
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
      if (tn >= 0) take_pages(tn, ids);
    } else {
      int xr = 0;
      if (lane == 0) xr = atomicAdd(&sh_cnt[kDW], 1);
      const int rb = r0 + __builtin_amdgcn_readfirstlane(xr);
      tn = rb < r1 ? tile_of_rank(rb) : -1;
    }
    t = tn;
    if (t >= 0) issue(t);
  }
  if (PAGED && bad_page && a.error_flag && lane == 0) atomicOr(a.error_flag, 1);

  // wave -> LDS in decode_body's layout: head x's state in lanes x, x + 16,
  // x + 32, x + 48; its output columns 16 nc + 4 r + i in lane 16 r + x,
  // register i, to the wave's (now idle) V slot
  float lsum = mst.l + xpair<16>(mst.l);
  lsum += xpair<32>(lsum);
  float* ao = reinterpret_cast<float*>(sv);
  if (x < GT) {
#pragma unroll
    for (int nc = 0; nc < D / 16; ++nc)
#pragma unroll
      for (int i = 0; i < 4; ++i) ao[x * D + 16 * nc + 4 * kg + i] = accp[nc][i];
  }
#pragma unroll
  for (int g = 0; g < GT; ++g) {
    float mg = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mst.m), g));
    if (mg != kM0) mg *= 0.6931471805599453f;
    const float lt = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lsum), g));
    if (lane == 0) {
      sh_m[wave][g] = mg;
      sh_l[wave][g] = lt;
    }
  }
  if (lane == 0) sh_cnt[wave] = kept;
}

// Fused split merge.  Every workgroup waits until its partial stores (agent
// scope, written through to memory) are complete and takes a ticket on its
// (row, chunk) counter; the workgroup that takes the last ticket resets the
// counter, invalidates its L2 (agent-scope acquire) and forms
//   out = sum_p e^(m_p - M) acc_p / max(sum_p e^(m_p - M) l_p, 1e-9)
// for the chunk's query heads, the formula of the stand-alone merge kernel.
// No full write-back fence is needed in the other workgroups.
// sh_w (>= GT * Pg floats) and sh_inv (>= GT floats) reuse the wave-merge
// LDS, which is dead by now.
template <int D, int GT, int kDW>
__device__ __forceinline__ void merge_if_last(const DecodeArgs& a, int row, int g0, int g_active, float* sh_w,
                                              float* sh_inv, float4* sh_red, int Pg, int64_t pbase, int hstride,
                                              int qstride) {
  __shared__ int sh_last;
  __builtin_amdgcn_s_waitcnt(0);  // this thread's partial stores are acknowledged
  __syncthreads();
  if (threadIdx.x == 0) {
    int* ctr = a.counters + ((int64_t)row * gridDim.z + blockIdx.z) * a.ctr_stride;
    const int done = atomicAdd(ctr, 1) + 1;
    sh_last = done == Pg;
    if (done == Pg) atomicExch(ctr, 0);
  }
  __syncthreads();
  if (!sh_last) return;
  Pg = __builtin_amdgcn_readfirstlane(Pg);  // uniform (the flat layout's comes through LDS)
  // the other workgroups' partials are read with agent-scope (sc1) loads,
  // which are coherent across the XCDs' L2s without an L2 invalidate.  All
  // first-round loads (m, l of partials 0..63 and the first PF accumulator
  // quads of every thread) are issued before any of them is used.
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  constexpr int CQ = D / 4;
  constexpr int kDT = kDW * kWave;
  // the (head, column quad) pairs in NPASS passes of NPAIR, each pair of a
  // pass summed by NSLICE threads (two passes at head_dim 256 with 8 heads,
  // one otherwise)
  constexpr int NPASS = (GT * CQ + kDT - 1) / kDT;
  constexpr int NPAIR = GT * CQ / NPASS;
  constexpr int NSLICE = kDT / NPAIR;
  static_assert(NPAIR * NPASS == GT * CQ && NPAIR * NSLICE == kDT, "merge passes");
  constexpr int PF = D >= 128 ? 32 : 8;  // the D = 64 kernels keep more waves per SIMD
  const int sl = threadIdx.x / NPAIR;
  int gp = (threadIdx.x % NPAIR) / CQ;
  int cq = (threadIdx.x % NPAIR) - gp * CQ;
  // one buffer descriptor over the Pg partial accumulators (D floats each,
  // qstride * D floats apart) of heads g0 .. g0 + g_active - 1 (hstride * D
  // floats apart), at a base made wave-uniform, so that each load is one
  // instruction (a per-thread descriptor is applied one distinct value at a
  // time); the thread's head is in its offset
  const uint64_t hpa = (uint64_t)(uintptr_t)(a.pacc + (pbase + (int64_t)g0 * hstride) * D);
  const float* hp = reinterpret_cast<const float*>(
      (uintptr_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(hpa >> 32)) << 32) |
                  (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)hpa)));
  int hoff = min(gp, g_active - 1) * hstride * D;
  const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)hp, (short)0, ((g_active - 1) * hstride + (Pg - 1) * qstride + 1) * D * (int)sizeof(float), 0x00020000);
  // partial q's column quad, or zeros when !ok (an offset past the
  // descriptor's range, which the buffer load answers with zeros: no branch)
  auto ld4 = [&](int q, bool ok) -> float4 {
    const int off = ok ? (hoff + q * qstride * D + 4 * cq) * (int)sizeof(float) : 0x7ffffff0;
    const auto x = __builtin_amdgcn_raw_buffer_load_b128(pr, off, 0, 16 /* sc1 */);
    return make_float4(__uint_as_float(x[0]), __uint_as_float(x[1]), __uint_as_float(x[2]), __uint_as_float(x[3]));
  };
  auto ldc = [](const float* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
  if (Pg <= kMergeFew) {
    // few partials (a uniform test): one thread per (head, column quad)
    // pair requests every partial's m, l and quad at once and forms the
    // output itself (no LDS weights, wave reductions or slice sums); N load
    // slots, 4 when they hold every partial
    auto few = [&](auto n_tag) {
      constexpr int N = decltype(n_tag)::value;
#pragma unroll
      for (int p0 = 0; p0 < GT * CQ; p0 += kDT) {
        const int pr0 = p0 + (int)threadIdx.x;
        const int hg = pr0 / CQ;
        const int hq = pr0 - hg * CQ;
        if (pr0 < GT * CQ && hg < g_active) {
          const int64_t base = pbase + (int64_t)(g0 + hg) * hstride;
          float mq[N], lq[N];
          float4 xq[N];
#pragma unroll
          for (int q = 0; q < N; ++q) {
            const bool ok = q < Pg;
            mq[q] = ok ? ldc(a.pm + base + q * qstride) : -__builtin_inff();
            lq[q] = ok ? ldc(a.pl + base + q * qstride) : 0.f;
            const int off = ok ? ((hg * hstride + q * qstride) * D + 4 * hq) * (int)sizeof(float) : 0x7ffffff0;
            const auto x = __builtin_amdgcn_raw_buffer_load_b128(pr, off, 0, 16 /* sc1 */);
            xq[q] = make_float4(__uint_as_float(x[0]), __uint_as_float(x[1]), __uint_as_float(x[2]),
                                __uint_as_float(x[3]));
          }
          float mx = mq[0];
#pragma unroll
          for (int q = 1; q < N; ++q) mx = fmaxf(mx, mq[q]);
          float ls = 0.f;
          float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
          for (int q = 0; q < N; ++q) {
            if (q < Pg) {
              const float w = __expf(mq[q] - mx);
              ls = __builtin_fmaf(w, lq[q], ls);
              acc.x = __builtin_fmaf(xq[q].x, w, acc.x);
              acc.y = __builtin_fmaf(xq[q].y, w, acc.y);
              acc.z = __builtin_fmaf(xq[q].z, w, acc.z);
              acc.w = __builtin_fmaf(xq[q].w, w, acc.w);
            }
          }
          const float inv = fmaxf(ls, 1e-9f);
          const int es = a.out_dtype == OC_F32 ? 4 : 2;
          char* o = a.out + ((int64_t)row * a.G + g0 + hg) * a.out_stride + (int64_t)(4 * hq) * es;
          store_scalar(o, a.out_dtype, acc.x / inv);
          store_scalar(o + es, a.out_dtype, acc.y / inv);
          store_scalar(o + 2 * es, a.out_dtype, acc.z / inv);
          store_scalar(o + 3 * es, a.out_dtype, acc.w / inv);
        }
      }
    };
    if (Pg <= 4) few(std::integral_constant<int, 4>{});
    else few(std::integral_constant<int, kMergeFew>{});
    return;
  }
  static_assert(GT <= 2 * kDW, "a wave merges at most two heads");
  float m0[2], l0[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int g = wave + k * kDW;
    const int64_t base = pbase + (int64_t)(g0 + g) * hstride;
    const bool ok = g < g_active && lane < Pg;
    m0[k] = ok ? ldc(a.pm + base + lane * qstride) : -__builtin_inff();
    l0[k] = ok ? ldc(a.pl + base + lane * qstride) : 0.f;
  }
  // (round i is issued only when some thread of the workgroup has a
  // partial in it: a uniform test)
  float4 pf[PF];
  auto prefetch = [&]() {
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      const int q = sl + i * NSLICE;
      pf[i] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (i * NSLICE < Pg) pf[i] = ld4(q, gp < g_active && q < Pg);
    }
  };
  prefetch();
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int g = wave + k * kDW;
    if (g >= g_active) break;
    const int64_t base = pbase + (int64_t)(g0 + g) * hstride;
    float mx = m0[k];
    for (int q = lane + 64; q < Pg; q += 64) mx = fmaxf(mx, ldc(a.pm + base + q * qstride));
    mx = wave_max(mx);
    float ls = 0.f;
    if (lane < Pg) {
      const float w = __expf(m0[k] - mx);
      sh_w[g * Pg + lane] = w;
      ls = w * l0[k];
    }
    for (int q = lane + 64; q < Pg; q += 64) {
      const float w = __expf(ldc(a.pm + base + q * qstride) - mx);
      sh_w[g * Pg + q] = w;
      ls = __builtin_fmaf(w, ldc(a.pl + base + q * qstride), ls);
    }
    ls = wave_sum(ls);
    if (lane == 0) sh_inv[g] = fmaxf(ls, 1e-9f);
  }
  __syncthreads();
  for (int ps = 0; ps < NPASS; ++ps) {
    if (ps > 0) {
      // the next pass's pairs, once every thread has read the last pass's
      // slices from sh_red
      __syncthreads();
      const int pair = ps * NPAIR + threadIdx.x % NPAIR;
      gp = pair / CQ;
      cq = pair - gp * CQ;
      hoff = min(gp, g_active - 1) * hstride * D;
      prefetch();
    }
    // weighted sum over the Pg partials: thread (slice, g, column quad) adds
    // partials q = slice, slice + nslice, ... with all its loads independent;
    // the slices are then added in a fixed order (deterministic result)
    const int g = gp;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    if (g < g_active) {
      const float* wg = sh_w + g * Pg;
#pragma unroll
      for (int i = 0; i < PF; ++i) {
        if (i * NSLICE < Pg) {
          const int q = sl + i * NSLICE;
          const float w = q < Pg ? wg[min(q, Pg - 1)] : 0.f;
          acc.x = __builtin_fmaf(pf[i].x, w, acc.x);
          acc.y = __builtin_fmaf(pf[i].y, w, acc.y);
          acc.z = __builtin_fmaf(pf[i].z, w, acc.z);
          acc.w = __builtin_fmaf(pf[i].w, w, acc.w);
        }
      }
      // the rest in rounds of RB independent loads (the same order of
      // additions as one partial at a time)
      constexpr int RB = 16;
#pragma unroll 1
      for (int q0 = sl + PF * NSLICE; q0 < Pg; q0 += RB * NSLICE) {
        float4 x[RB];
#pragma unroll
        for (int i = 0; i < RB; ++i) {
          const int q = q0 + i * NSLICE;
          x[i] = ld4(q, q < Pg);
        }
#pragma unroll
        for (int i = 0; i < RB; ++i) {
          const int q = q0 + i * NSLICE;
          const float w = q < Pg ? wg[q] : 0.f;
          acc.x = __builtin_fmaf(x[i].x, w, acc.x);
          acc.y = __builtin_fmaf(x[i].y, w, acc.y);
          acc.z = __builtin_fmaf(x[i].z, w, acc.z);
          acc.w = __builtin_fmaf(x[i].w, w, acc.w);
        }
      }
    }
    sh_red[threadIdx.x] = acc;
    __syncthreads();
    if (threadIdx.x < NPAIR && g < g_active) {
      auto add = [&](const float4 y) {
        acc.x += y.x;
        acc.y += y.y;
        acc.z += y.z;
        acc.w += y.w;
      };
      if constexpr (NSLICE > 32) {
        // (head_dim 32, one head: 64 slices) rounds of 16 reads, the same
        // order of additions; all 63 reads at once would take 252 registers
        constexpr int RS = 16;
#pragma unroll 1
        for (int k0 = 1; k0 < NSLICE; k0 += RS) {
          float4 y[RS];
#pragma unroll
          for (int j = 0; j < RS; ++j)
            if (k0 + j < NSLICE) y[j] = sh_red[(k0 + j) * NPAIR + threadIdx.x];
#pragma unroll
          for (int j = 0; j < RS; ++j)
            if (k0 + j < NSLICE) add(y[j]);
        }
      } else {
#pragma unroll
        for (int k = 1; k < NSLICE; ++k) add(sh_red[k * NPAIR + threadIdx.x]);
      }
      const float inv = sh_inv[g];
      const int es = a.out_dtype == OC_F32 ? 4 : 2;
      char* o = a.out + ((int64_t)row * a.G + g0 + g) * a.out_stride + (int64_t)(4 * cq) * es;
      store_scalar(o, a.out_dtype, acc.x / inv);
      store_scalar(o + es, a.out_dtype, acc.y / inv);
      store_scalar(o + 2 * es, a.out_dtype, acc.z / inv);
      store_scalar(o + 3 * es, a.out_dtype, acc.w / inv);
    }
  }
}

// Main decode kernel.  grid = (Pg, num_rows, ceil(G / GT)); block = 8 waves.
// Workgroup (g, row, chunk) forms the online-softmax state of query heads
// [chunk*GT, chunk*GT + GT) over the retained tiles of the logical splits
// s = g*spw .. g*spw + spw - 1 of the row (split s owns tiles {s + kP}):
// the eight waves take those tiles round-robin (single-pass) or take the
// retained ones round-robin (cached), and their states are merged in LDS
// into the workgroup's partial (m, l, acc).  With spw = 1 every partial is
// exactly one logical split's state.
// Two waves per SIMD (<= 256 VGPRs) except for float32 K/V, whose raw K and
// V tiles alone take 256 registers.
// The kDW wave states of a workgroup merged into its split partial.  Partial
// index of query head h in slot p of the row: pbase + h * hstride + p *
// qstride ((row * G + h) * Pg + p, or with the flat layout (slot0 + p) * G +
// h).  acc_of(w, g, c): wave w's accumulator of head g, column c.
template <int D, int GT, int kDW, typename AccOf>
__device__ __forceinline__ void write_partial(const DecodeArgs& a, int g0, int g_active, int gidx, int64_t pbase,
                                              int hstride, int qstride, const float (*sh_m)[GT],
                                              const float (*sh_l)[GT], AccOf acc_of) {
  for (int idx = threadIdx.x; idx < g_active * D; idx += kDW * kWave) {
    const int g = idx / D;
    const int c = idx - g * D;
    float mx = sh_m[0][g];
#pragma unroll
    for (int w = 1; w < kDW; ++w) mx = fmaxf(mx, sh_m[w][g]);
    float acc = 0.f, l = 0.f;
#pragma unroll
    for (int w = 0; w < kDW; ++w) {
      const float e = __expf(sh_m[w][g] - mx);
      acc = __builtin_fmaf(acc_of(w, g, c), e, acc);
      l = __builtin_fmaf(sh_l[w][g], e, l);
    }
    const int64_t pidx = pbase + (int64_t)(g0 + g) * hstride + (int64_t)gidx * qstride;
    // agent-scope stores write through this XCD's L2, so the fused merge
    // (possibly on another XCD) reads them without a cache write-back
    __hip_atomic_store(a.pacc + pidx * D + c, acc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (c == 0) {
      __hip_atomic_store(a.pm + pidx, mx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(a.pl + pidx, l, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

template <int DT, int D, int GT, bool DOT2, bool PAGED, bool MQK, bool LOOP>
__global__ __launch_bounds__((DecWaves<DT, D, MQK, GT>::value * kWave)) __attribute__((amdgpu_waves_per_eu(DecWaves<DT, D, MQK, GT>::value == 4 ? 1 : 2))) void decode_kernel(
    const DecodeArgs a) {
  constexpr int kDW = DecWaves<DT, D, MQK, GT>::value;
  constexpr int kDT = kDW * kWave;
  const int lane = threadIdx.x & 63;
  const int g0 = blockIdx.z * GT;
  const int g_active = min(GT, a.G - g0);
  // the row, this workgroup's index among the row's workgroups, their
  // number and (flat layout) the row's first partial slot
  int row = blockIdx.y, gidx = blockIdx.x, npg = a.Pg, slot0 = 0;
  // flat layout: single pass and dense take tile-range shares, longest
  // first (flat_map_lpt); a cached decode splits each row's retained ranks
  // over its workgroups (a.bal) on flat_map's layout
  const bool lpt = a.flat && !a.bal;
  int fb0 = 0, fb1 = 0, fntok = 0;
  if (a.flat) {
    __shared__ int sh_fm[4 * kDW + 9];
    if (lpt ? !flat_map_lpt<kDW>(a, 4 * D, sh_fm, row, gidx, npg, slot0, fb0, fb1, fntok)
            : !flat_map<kDW>(a, 4 * D, sh_fm, row, gidx, npg, slot0))
      return;
  }
  const RowInfo ri = lpt ? row_info_n(a, row, fntok) : row_info(a, row);
  TileList tl;
  if (lpt) {
    tl.s = fb0;
    tl.n = fb1 - fb0;
    tl.w = tl.P = 1;
  } else if (a.flat) {
    // a contiguous share of the row's tiles (unused by the balanced split)
    tl.s = (int)((int64_t)ri.n_tiles * gidx / npg);
    tl.n = (int)((int64_t)ri.n_tiles * (gidx + 1) / npg) - tl.s;
    tl.w = tl.P = 1;
  } else {
    tl = split_list(a, ri, blockIdx.x * a.spw);
  }

  __shared__ float sh_qf[GT * D];
  __shared__ uint32_t sh_qp[GT * D / 2];
  __shared__ float sh_m[kDW][GT];
  __shared__ float sh_l[kDW][GT];
  __shared__ float sh_acc[MQK ? 1 : kDW][GT][D];  // MQK: the wave states go to the V slots
  __shared__ float4 sh_red_own[MQK ? 1 : kDT];     // merge reduction (MQK: inside the V slots)
  __shared__ int sh_cnt[kDW + 1];  // per-wave retained counts; [kDW]: single-pass list position
  __shared__ uint64_t sh_bits[kMaxBalTiles / 64];  // balanced: retained-tile bitmask of the row;
                                                   // matrix-core single pass: keep flags
  __shared__ float sh_p[MQK ? kDW * 64 * (GT > 4 ? 8 : 4) : 1];  // per wave p[head][token] of the current tile (MQK)
  __shared__ __attribute__((aligned(16))) uint16_t sh_v[MQK ? kDW * 64 * D : 8];  // per wave V tile (MQK)

  {
    // cached mode: fetch the scores before anything else (balanced: tiles
    // threadIdx.x + 256k of the first kPreChunks chunks; otherwise the lane's
    // entry of the first chunk of the split list)
    constexpr int kPreChunks = 4;
    float pre_el[kPreChunks], pre_eh[kPreChunks];
  #pragma unroll
    for (int k = 0; k < kPreChunks; ++k) pre_el[k] = pre_eh[k] = 0.f;
    if (a.mode == OC_MODE_CACHED && a.gate != OC_GATE_NONE) {
  #pragma unroll
      for (int k = 0; k < kPreChunks; ++k) {
        int t;
        bool in;
        if (a.bal) {
          t = k * kDT + threadIdx.x;
          in = t < ri.n_tiles;
        } else {
          t = tl.s + (lane / tl.w) * tl.P + lane % tl.w;
          in = k == 0 && lane < tl.n && t < ri.n_tiles;
        }
        if (in) cached_scores(a, row, t, pre_el[k], pre_eh[k]);
      }
    }

    // stage q of this chunk in LDS (float and packed 16-bit); q := round(q *
    // k_scale) in q's dtype for the Q_FOLD mode (fused_eviction.py:619-621)
    const int qes = a.q_dtype == OC_F32 ? 4 : 2;
    float qss = 0.f;  // x0^2 + x1^2 of this thread's pair (head norms below)
    for (int idx = threadIdx.x; idx < GT * D / 2; idx += kDT) {
      const int e0 = 2 * idx;
      const int g = e0 / D;
      const int c = e0 - g * D;
      float x0 = 0.f, x1 = 0.f;
      if (g < g_active) {
        const char* qp = a.q + (int64_t)(row * a.G + g0 + g) * a.q_row_stride + (int64_t)c * qes;
        x0 = load_scalar(qp, a.q_dtype);
        x1 = load_scalar(qp + qes, a.q_dtype);
        if (a.k_scale_mode == OC_KSCALE_Q_FOLD) {
          x0 = round_to(x0 * a.k_scale, a.q_dtype);
          x1 = round_to(x1 * a.k_scale, a.q_dtype);
        }
      }
      sh_qf[e0] = x0;
      sh_qf[e0 + 1] = x1;
      qss = __builtin_fmaf(x1, x1, x0 * x0);
      if constexpr (DOT2) {
        // x0, x1 are exact in the 16-bit q dtype, so the narrowing is exact
        uint32_t lo, hi;
        if (MfmaT<DT>::value == OC_BF16) {
          lo = __float_as_uint(x0) >> 16;
          hi = __float_as_uint(x1) >> 16;
        } else {
          lo = __builtin_bit_cast(uint16_t, (_Float16)x0);
          hi = __builtin_bit_cast(uint16_t, (_Float16)x1);
        }
        sh_qp[idx] = lo | (hi << 16);
      }
    }
    // max_g ||q_g|| over all G query heads of the row (CS gate).  When all G
    // heads are in this workgroup (and GT * D / 2 <= threads), the D / 2
    // threads of a head (one wave at D = 128, half a wave at D = 64) add their
    // pairs' squares right away; otherwise wave w forms the norms of heads w,
    // w + 8, ... from LDS and global memory after the barrier.  The wave
    // maxima are combined after the next barrier.
    __shared__ float sh_qn[kDW];
    __shared__ int sh_qnan[kDW];
    if (threadIdx.x == 0) sh_cnt[kDW] = kDW;
    const bool fast_norms = (D == 64 || D == 128) && a.gate == OC_GATE_CS && a.G <= GT && GT * D / 2 <= kDT;
    if (fast_norms) {
      const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
      float ss;
      if constexpr (D == 128) {
        ss = wave_sum(qss);
      } else {
        float lo, hi;
        row_pair<16>(row16_sum(qss), lo, hi);
        ss = lo + hi;  // the 32-lane half of this lane
      }
      float qn = __builtin_sqrtf(ss);
      if ((double)qn < 1e-38) qn = 0.f;
      const int hpw = 128 / D;  // heads per wave
      float wmax = 0.f;
      bool wnan = false;
  #pragma unroll
      for (int h = 0; h < 128 / D; ++h) {
        const int g = wave * hpw + h;
        const float x = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(qn), h * (64 / hpw)));
        if (g < a.G) {
          if (__builtin_isnan(x)) wnan = true;
          wmax = fmaxf(wmax, x);
        }
      }
      if (lane == 0) {
        sh_qn[wave] = wmax;
        sh_qnan[wave] = wnan ? 1 : 0;
      }
    }
    __syncthreads();
    float qmax = 0.f;
    bool qnan = false;
    if (a.gate == OC_GATE_CS && !fast_norms) {
      const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
      float wmax = 0.f;
      bool wnan = false;
      for (int g = wave; g < a.G; g += kDW) {
        float ss = 0.f;
        if (lane < 16) {
          const int gl = g - g0;
  #pragma unroll
          for (int c = 0; c < D / 16; ++c) {
            const int col = (lane & 15) * (D / 16) + c;
            float x;
            if (gl >= 0 && gl < GT) {
              x = sh_qf[gl * D + col];
            } else {
              x = load_scalar(a.q + (int64_t)(row * a.G + g) * a.q_row_stride + (int64_t)col * qes, a.q_dtype);
              if (a.k_scale_mode == OC_KSCALE_Q_FOLD) x = round_to(x * a.k_scale, a.q_dtype);
            }
            ss = __builtin_fmaf(x, x, ss);
          }
        }
        float qn = __builtin_sqrtf(wave_sum(ss));
        if ((double)qn < 1e-38) qn = 0.f;
        if (__builtin_isnan(qn)) wnan = true;
        wmax = fmaxf(wmax, qn);
      }
      if (lane == 0) {
        sh_qn[wave] = wmax;
        sh_qnan[wave] = wnan ? 1 : 0;
      }
      __syncthreads();
    }
    if (a.gate == OC_GATE_CS) {
  #pragma unroll
      for (int w = 0; w < kDW; ++w) {
        qmax = fmaxf(qmax, sh_qn[w]);
        qnan = qnan || sh_qnan[w] != 0;
      }
    }

    // balanced cached decode: retained-tile bitmask of the whole row and its
    // prefix counts, then this workgroup's even share [r0, r1) of the ranks
    int r0 = 0, r1 = 0, wpre = 0;
    if (a.bal) {
      const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
      const int nw = (ri.n_tiles + 63) / 64;
  #pragma unroll
      for (int c = 0; c < kPreChunks * kDT; c += kDT) {
        if (c < ri.n_tiles) {
          const int t = c + threadIdx.x;
          const bool keep = t < ri.n_tiles && cached_keep(a, ri, t, pre_el[c / kDT], pre_eh[c / kDT], qmax, qnan);
          if (a.keep_out && t < ri.n_tiles && gidx == 0 && blockIdx.z == 0)
            a.keep_out[(int64_t)row * a.keep_stride + t] = keep ? 1 : 0;
          const uint64_t m = __ballot(keep);
          const int wi = (c >> 6) + wave;
          if (lane == 0 && wi < nw) sh_bits[wi] = m;
        }
      }
      for (int c = kPreChunks * kDT; c < ri.n_tiles; c += kDT) {
        const int t = c + threadIdx.x;
        const bool in = t < ri.n_tiles;
        float el = 0.f, eh = 0.f;
        if (in) cached_scores(a, row, t, el, eh);
        const bool keep = in && cached_keep(a, ri, t, el, eh, qmax, qnan);
        if (a.keep_out && in && gidx == 0 && blockIdx.z == 0)
          a.keep_out[(int64_t)row * a.keep_stride + t] = keep ? 1 : 0;
        const uint64_t m = __ballot(keep);
        const int wi = (c >> 6) + wave;
        if (lane == 0 && wi < nw) sh_bits[wi] = m;
      }
      // words nw .. (nw rounded up to 4) read as empty in the lookups below
      if (threadIdx.x < 4 && nw + (int)threadIdx.x < ((nw + 3) & ~3)) sh_bits[nw + threadIdx.x] = 0;
      __syncthreads();
      // every wave: lane l counts the retained tiles of bitmask words
      // 4l .. 4l+3; wpre = inclusive prefix of those counts over the lanes
      int x = 0;
  #pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int wi = 4 * lane + k;
        x += wi < nw ? __popcll((unsigned long long)sh_bits[wi]) : 0;
      }
      wpre = wave_incl_scan(x);
      const uint32_t total = (uint32_t)__builtin_amdgcn_readlane(wpre, 63);
      r0 = (int)((uint64_t)total * gidx / (uint32_t)npg);
      r1 = (int)((uint64_t)total * (gidx + 1) / (uint32_t)npg);
    }

    decode_body<DT, D, GT, DOT2, PAGED, MQK, LOOP>(a, ri, row, tl, g0, qmax, qnan, sh_qf, sh_qp, sh_m, sh_l, sh_acc, sh_cnt,
                                             pre_el[0], pre_eh[0], sh_bits, wpre, r0, r1, sh_p, sh_v,
                                             reinterpret_cast<uint8_t*>(sh_bits));
  }
  __syncthreads();
  // matrix-core single pass: the keep flags staged in LDS in list order
  if (MQK && !LOOP && a.keep_out && blockIdx.z == 0) {
    if (tl.n <= kKeepLds) {
      const uint8_t* sh_keep = reinterpret_cast<const uint8_t*>(sh_bits);
      for (int x = threadIdx.x; x < tl.n; x += kDT) {
        const int t = tl.s + (x / tl.w) * tl.P + x % tl.w;
        if (t < ri.n_tiles) a.keep_out[(int64_t)row * a.keep_stride + t] = sh_keep[x];
      }
    }
  }

  const int64_t pbase = a.flat ? (int64_t)slot0 * a.G : (int64_t)row * a.G * a.Pg;
  const int hstride = a.flat ? 1 : a.Pg;
  const int qstride = a.flat ? a.G : 1;
  write_partial<D, GT, kDW>(a, g0, g_active, gidx, pbase, hstride, qstride, sh_m, sh_l, [&](int w, int g, int c) {
    return MQK ? reinterpret_cast<const float*>(sh_v + w * 64 * D)[g * D + c] : sh_acc[MQK ? 0 : w][g][c];
  });
  if (a.split_counts && threadIdx.x == 0 && blockIdx.z == 0)
  {
    int n = 0;
#pragma unroll
    for (int w = 0; w < kDW; ++w) n += sh_cnt[w];
    a.split_counts[(int64_t)row * a.Pg + blockIdx.x] = n;
  }
  // merge scratch: GT * Pg weights in the wave-state area, idle by now, and
  // one float4 per thread (MQK: both inside the V slots)
  float* sh_w = MQK ? reinterpret_cast<float*>(sh_v) : &sh_acc[0][0][0];
  float4* sh_red = MQK ? reinterpret_cast<float4*>(sh_v + kDW * 64 * D / 2) : sh_red_own;
  if (a.fuse) merge_if_last<D, GT, kDW>(a, row, g0, g_active, sh_w, &sh_l[0][0], sh_red, npg, pbase, hstride, qstride);
}

// The decode with the per-wave prologue (decode_fast; a.fast, set by the
// host): kDW waves per workgroup, every query head of a row in one
// workgroup (GT >= G).  kDW = 8 fills a CU with one workgroup; kDW = 4 (the
// flat layout's many small workgroups) lets two share a CU, so that one's
// prologue overlaps the other's tile loop.  VT: V's element type (DT, or
// bf16 V beside fp8 K).
template <int DT, int D, int GT, bool PAGED, int kDW, int VT = DT>
// Two waves per SIMD (<= 256 registers) at head_dim 64 and 128; at head_dim
// 256 (4-wave workgroups, a 32 KiB V slot per wave) one wave per SIMD: the K
// tile alone takes 128 registers and the accumulators 64.
__global__ __launch_bounds__(kDW * kWave) __attribute__((amdgpu_waves_per_eu(D >= 256 ? 1 : 2))) void decode_fast_kernel(
    const DecodeArgs a) {
  const int g_active = min(GT, a.G);
  int row = blockIdx.y, gidx = blockIdx.x, npg = a.Pg, slot0 = 0, b0 = 0, b1 = 0, ntok = 0;
  if (a.flat) {
    __shared__ int sh_fm[4 * kDW + 9];
    if (!flat_map_lpt<kDW>(a, 4 * D, sh_fm, row, gidx, npg, slot0, b0, b1, ntok)) return;
  }
  const RowInfo ri = a.flat ? row_info_n(a, row, ntok) : row_info(a, row);
  if (!a.flat) b1 = ri.n_tiles;
  __shared__ float sh_m[kDW][GT];
  __shared__ float sh_l[kDW][GT];
  __shared__ int sh_cnt[kDW + 1];
  __shared__ __attribute__((aligned(16))) uint16_t sh_v[kDW * 64 * D];  // per wave V tile, then its state
  // flat: the share is the tile range [b0, b1), all of whose retained tiles
  // the workgroup takes (one split of one); otherwise an even split of the
  // row's retained ranks (dense: tiles) over its npg workgroups
  decode_fast<DT, D, GT, PAGED, kDW, VT>(a, ri, row, a.flat ? 0 : gidx, a.flat ? 1 : npg, b0, b1, sh_m, sh_l, sh_cnt,
                                     sh_v);
  __syncthreads();
  const int64_t pbase = a.flat ? (int64_t)slot0 * a.G : (int64_t)row * a.G * a.Pg;
  const int hstride = a.flat ? 1 : a.Pg;
  const int qstride = a.flat ? a.G : 1;
  write_partial<D, GT, kDW>(a, 0, g_active, gidx, pbase, hstride, qstride, sh_m, sh_l, [&](int w, int g, int c) {
    return reinterpret_cast<const float*>(sh_v + w * 64 * D)[g * D + c];
  });
  // merge scratch inside the (idle) V slots: GT * Pg weights, one float4 per thread
  if (a.fuse)
    merge_if_last<D, GT, kDW>(a, row, 0, g_active, reinterpret_cast<float*>(sh_v), &sh_l[0][0],
                              reinterpret_cast<float4*>(sh_v + kDW * 64 * D / 2), npg, pbase, hstride, qstride);
}

// Tile scoring: one wave per (row, tile); block = 4 waves.
template <int DT, int D, bool PAGED>
__global__ __launch_bounds__(kThreads) void score_kernel(const DecodeArgs a) {
  using L = Lay<DT, D>;
  const int lane = threadIdx.x & 63;
  const int64_t job = (int64_t)blockIdx.x * kWaves + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (job >= (int64_t)a.num_rows * a.tcnt) return;
  const int row = (int)(job / a.tcnt);
  const int t = a.t0 + (int)(job - (int64_t)row * a.tcnt);
  const RowInfo ri = row_info(a, row);
  const int64_t o = (int64_t)row * a.o_stride + t;
  float el = 0.f, eh = 0.f, z = 0.f;
  uint8_t keep = 0;
  if ((t + 1) * 64 <= ri.n_tok) {
    uint32_t kw[16][L::LW];
    load_tile<DT, D, PAGED>(a, ri, row, t, false, lane, kw);
    if (DT == OC_FP8_E4M3FN && a.k_scale_mode == OC_KSCALE_DEQUANT) {
      if constexpr (DT == OC_FP8_E4M3FN) tile_energies<DT, D, true>(kw, Deq{a.k_scale, true}, lane, el, eh);
    } else {
      tile_energies<DT, D>(kw, tile_kdeq(a, row, t), lane, el, eh);
    }
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
template <int DT, int D, bool PAGED>
__global__ __launch_bounds__(kThreads) void fwht_kernel(const DecodeArgs a) {
  constexpr int CPL = D / 16;
  using L = Lay<DT, D>;
  const int lane = threadIdx.x & 63;
  const int64_t job = (int64_t)blockIdx.x * kWaves + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (job >= (int64_t)a.num_rows * a.num_tiles) return;
  const int row = (int)(job / a.num_tiles);
  const int t = (int)(job - (int64_t)row * a.num_tiles);
  RowInfo ri = row_info(a, row);
  ri.n_tok = a.num_tiles * 64;  // the transform covers whole tiles
  uint32_t kw[16][L::LW];
  float f[16][CPL];
  load_tile<DT, D, PAGED>(a, ri, row, t, false, lane, kw);
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
      float x = butterfly_rows<16>(f[i][c]);
      x = butterfly_rows<32>(x);
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

// Band norms ||(W64 K_t)[band_lo, band_hi)||_F of tiles [t0, t0 + tcnt) of
// every row (norm_cache.py:58-117), float32, clamped to 0 below 1e-38 as
// the reference does; the full 64-point transform in registers as in
// fwht_kernel, then the squares of the band's rows.  Tiles not wholly
// inside the row's length are not written.
template <int DT, int D, bool PAGED>
__global__ __launch_bounds__(kThreads) void band_norm_kernel(const DecodeArgs a) {
  constexpr int CPL = D / 16;
  using L = Lay<DT, D>;
  const int lane = threadIdx.x & 63;
  const int64_t job = (int64_t)blockIdx.x * kWaves + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (job >= (int64_t)a.num_rows * a.tcnt) return;
  const int row = (int)(job / a.tcnt);
  const int t = a.t0 + (int)(job - (int64_t)row * a.tcnt);
  const RowInfo ri = row_info(a, row);
  if ((t + 1) * 64 > ri.n_tok) return;
  uint32_t kw[16][L::LW];
  float f[16][CPL];
  load_tile<DT, D, PAGED>(a, ri, row, t, false, lane, kw);
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
  // lane (gamma, j) holds spectral rows 4i + gamma, columns j*CPL ..
  const int gamma = lane >> 4;
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const bool in = 4 * i + gamma >= a.band_lo && 4 * i + gamma < a.band_hi;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      float x = butterfly_rows<16>(f[i][c]);
      x = butterfly_rows<32>(x) * 0.125f;
      ss = in ? __builtin_fmaf(x, x, ss) : ss;
    }
  }
  float n = __builtin_sqrtf(wave_sum(ss));
  if ((double)n < 1e-38) n = 0.f;
  if (lane == 0) {
    a.o_norm[(int64_t)row * a.o_stride + t] = n;
    if (a.o_valid) atomicMax(a.o_valid + row, t + 1);
  }
}

// Launchers instantiated per element type (oc_kernels_<dtype>.hip).
template <int DT>
hipError_t launch_decode(const DecodeArgs& a, int head_dim, int gt, int gchunks, hipStream_t st);
template <int DT>
hipError_t launch_score(const DecodeArgs& a, int head_dim, hipStream_t st);
template <int DT>
hipError_t launch_fwht(const DecodeArgs& a, int head_dim, hipStream_t st);
template <int DT>
hipError_t launch_band(const DecodeArgs& a, int head_dim, hipStream_t st);

template <int DT, int HD, bool PG, int W, int VT = DT>
inline void launch_fast_gt(const DecodeArgs& a, int gt, dim3 grid, hipStream_t st) {
  const dim3 block(W * kWave);
  switch (gt) {
    case 1: hipLaunchKernelGGL((decode_fast_kernel<DT, HD, 1, PG, W, VT>), grid, block, 0, st, a); break;
    case 2: hipLaunchKernelGGL((decode_fast_kernel<DT, HD, 2, PG, W, VT>), grid, block, 0, st, a); break;
    case 4: hipLaunchKernelGGL((decode_fast_kernel<DT, HD, 4, PG, W, VT>), grid, block, 0, st, a); break;
    default: hipLaunchKernelGGL((decode_fast_kernel<DT, HD, 8, PG, W, VT>), grid, block, 0, st, a); break;
  }
}

template <int DT, int HD, bool DOT2, bool PG, bool MQ, bool LOOP>
inline void launch_decode_gt(const DecodeArgs& a, int gt, dim3 grid, hipStream_t st) {
  if constexpr (MQ && LOOP) {
    if (a.fast) {
      if constexpr (DT == OC_FP8_E4M3FN) {
        if (a.v_bf16) {
          if (a.fast_waves == 4) launch_fast_gt<DT, HD, PG, 4, OC_BF16>(a, gt, grid, st);
          else launch_fast_gt<DT, HD, PG, 8, OC_BF16>(a, gt, grid, st);
          return;
        }
      }
      if (a.fast_waves == 4) launch_fast_gt<DT, HD, PG, 4>(a, gt, grid, st);
      else launch_fast_gt<DT, HD, PG, 8>(a, gt, grid, st);
      return;
    }
  }
  auto block = [](int w) { return dim3(w * kWave); };
  switch (gt) {
    case 1: hipLaunchKernelGGL((decode_kernel<DT, HD, 1, DOT2, PG, MQ, LOOP>), grid, block(DecWaves<DT, HD, MQ, 1>::value), 0, st, a); break;
    case 2: hipLaunchKernelGGL((decode_kernel<DT, HD, 2, DOT2, PG, MQ, LOOP>), grid, block(DecWaves<DT, HD, MQ, 2>::value), 0, st, a); break;
    case 4: hipLaunchKernelGGL((decode_kernel<DT, HD, 4, DOT2, PG, MQ, LOOP>), grid, block(DecWaves<DT, HD, MQ, 4>::value), 0, st, a); break;
    default: hipLaunchKernelGGL((decode_kernel<DT, HD, 8, DOT2, PG, MQ, LOOP>), grid, block(DecWaves<DT, HD, MQ, 8>::value), 0, st, a); break;
  }
}

// matrix-core kernels come in two variants: every listed tile attended
// (cached or dense decode) or the single-pass gate, so that each carries
// only its own loop's registers
template <int DT, int HD, bool PG>
inline void launch_decode_mq(const DecodeArgs& a, int gt, dim3 grid, hipStream_t st) {
  const bool loop = (a.mode == OC_MODE_CACHED && a.gate != OC_GATE_NONE) || a.gate == OC_GATE_NONE;
  if (loop) launch_decode_gt<DT, HD, true, PG, true, true>(a, gt, grid, st);
  else launch_decode_gt<DT, HD, true, PG, true, false>(a, gt, grid, st);
}

// q . k on the matrix cores for contiguous 16-bit K (q of the same type)
template <int DT, int HD, bool DOT2>
inline void launch_decode_hd(const DecodeArgs& a, int gt, dim3 grid, hipStream_t st) {
  // matrix cores whenever q has the 16-bit type K runs in (bf16 q for fp8
  // K, which is widened exactly): contiguous K/V, or pages of >= 16 tokens
  // (a 16-token block inside one page)
  if constexpr (DOT2) {
    if (!a.paged) {
      launch_decode_mq<DT, HD, false>(a, gt, grid, st);
      return;
    }
    if (a.bs_log2 >= 4) {
      launch_decode_mq<DT, HD, true>(a, gt, grid, st);
      return;
    }
  }
  // VALU path (v_dot2 q.k for 16-bit K and q of the same type)
  constexpr bool VDOT2 = DOT2 && DT != OC_FP8_E4M3FN;
  if (a.paged) launch_decode_gt<DT, HD, VDOT2, true, false, false>(a, gt, grid, st);
  else launch_decode_gt<DT, HD, VDOT2, false, false, false>(a, gt, grid, st);
}

// head_dim 256: the matrix-core kernels only (the per-wave-prologue one,
// or the general one: attend-every-tile or single-pass gate), 16-bit K/V
// with q of K's type or fp8 K/V with bf16 q (bf16 V beside fp8 K in the
// per-wave-prologue kernel), 4-wave workgroups, up to 8 query heads per
// workgroup (the fused merge gives each of its 256 threads one column quad
// of one head per pass: two passes for 8 heads); the host routes every
// other head_dim-256 decode to the portable kernels
template <int DT>
inline void launch_decode256(const DecodeArgs& a, int gt, dim3 grid, hipStream_t st) {
  if constexpr (DT == OC_BF16 || DT == OC_F16 || DT == OC_FP8_E4M3FN) {
    const dim3 block(4 * kWave);
    const bool loop = (a.mode == OC_MODE_CACHED && a.gate != OC_GATE_NONE) || a.gate == OC_GATE_NONE;
    auto fast = [&](auto pg, auto vt) {
      constexpr bool PG = decltype(pg)::value;
      constexpr int VT = decltype(vt)::value;
      switch (gt) {
        case 1: hipLaunchKernelGGL((decode_fast_kernel<DT, 256, 1, PG, 4, VT>), grid, block, 0, st, a); break;
        case 2: hipLaunchKernelGGL((decode_fast_kernel<DT, 256, 2, PG, 4, VT>), grid, block, 0, st, a); break;
        case 4: hipLaunchKernelGGL((decode_fast_kernel<DT, 256, 4, PG, 4, VT>), grid, block, 0, st, a); break;
        default: hipLaunchKernelGGL((decode_fast_kernel<DT, 256, 8, PG, 4, VT>), grid, block, 0, st, a); break;
      }
    };
    auto go = [&](auto pg) {
      constexpr bool PG = decltype(pg)::value;
      if (a.fast) {
        if constexpr (DT == OC_FP8_E4M3FN) {
          if (a.v_bf16) fast(pg, std::integral_constant<int, OC_BF16>{});
          else fast(pg, std::integral_constant<int, DT>{});
        } else {
          fast(pg, std::integral_constant<int, DT>{});
        }
      } else if (loop) {
        switch (gt) {
          case 1: hipLaunchKernelGGL((decode_kernel<DT, 256, 1, true, PG, true, true>), grid, block, 0, st, a); break;
          case 2: hipLaunchKernelGGL((decode_kernel<DT, 256, 2, true, PG, true, true>), grid, block, 0, st, a); break;
          case 4: hipLaunchKernelGGL((decode_kernel<DT, 256, 4, true, PG, true, true>), grid, block, 0, st, a); break;
          default: hipLaunchKernelGGL((decode_kernel<DT, 256, 8, true, PG, true, true>), grid, block, 0, st, a); break;
        }
      } else {
        switch (gt) {
          case 1: hipLaunchKernelGGL((decode_kernel<DT, 256, 1, true, PG, true, false>), grid, block, 0, st, a); break;
          case 2: hipLaunchKernelGGL((decode_kernel<DT, 256, 2, true, PG, true, false>), grid, block, 0, st, a); break;
          case 4: hipLaunchKernelGGL((decode_kernel<DT, 256, 4, true, PG, true, false>), grid, block, 0, st, a); break;
          default: hipLaunchKernelGGL((decode_kernel<DT, 256, 8, true, PG, true, false>), grid, block, 0, st, a); break;
        }
      }
    };
    if (a.paged) go(std::true_type{});
    else go(std::false_type{});
  }
}

// head_dim 32: the matrix-core kernels only, 16-bit K/V with q of K's type
// (8-wave workgroups as at head_dim 64, a 4 KiB V slot per wave); the host
// routes every other head_dim-32 decode (fp8 or float32 K/V, another q type)
// to the portable kernels
template <int DT>
constexpr bool kNarrowMfma = DT == OC_BF16 || DT == OC_F16;
template <int DT>
inline void launch_decode32(const DecodeArgs& a, int gt, dim3 grid, hipStream_t st) {
  if constexpr (kNarrowMfma<DT>) {
    if (a.paged) launch_decode_mq<DT, 32, true>(a, gt, grid, st);
    else launch_decode_mq<DT, 32, false>(a, gt, grid, st);
  }
}

#define OC_DECODE_CASES(DT, DOT2)                                 \
  if (head_dim == 256) launch_decode256<DT>(a, gt, grid, st);     \
  else if (head_dim == 128) launch_decode_hd<DT, 128, DOT2>(a, gt, grid, st); \
  else if (head_dim == 32) launch_decode32<DT>(a, gt, grid, st);  \
  else launch_decode_hd<DT, 64, DOT2>(a, gt, grid, st);

// q . k on 16-bit operands (matrix cores, or v_dot2 on the VALU path) when
// q has K's 16-bit type; for fp8 K when q is bf16
template <int DT>
constexpr bool kHasDot2 = DT == OC_BF16 || DT == OC_F16 || DT == OC_FP8_E4M3FN;
template <int DT>
constexpr int kDot2Q = DT == OC_FP8_E4M3FN ? OC_BF16 : DT;

#define OC_DEFINE_LAUNCHERS(DT)                                                                   \
  template <>                                                                                     \
  hipError_t launch_decode<DT>(const DecodeArgs& a, int head_dim, int gt, int gchunks,            \
                               hipStream_t st) {                                                  \
    const dim3 grid = a.flat ? dim3(a.fast || !a.bal ? a.flat_slots : a.flat_target + a.num_rows, 1, gchunks)      \
                             : dim3(a.Pg, a.num_rows, gchunks);                                   \
    /* head_dim 32: 16-bit K/V with q of K's type only */                                        \
    if (head_dim == 32 && !(kNarrowMfma<DT> && a.q_dtype == DT)) return hipErrorInvalidValue;    \
    if (kHasDot2<DT> && a.q_dtype == kDot2Q<DT>) {                                               \
      OC_DECODE_CASES(DT, kHasDot2<DT>)                                                           \
    } else {                                                                                      \
      OC_DECODE_CASES(DT, false)                                                                  \
    }                                                                                             \
    return hipGetLastError();                                                                     \
  }                                                                                               \
  template <>                                                                                     \
  hipError_t launch_score<DT>(const DecodeArgs& a, int head_dim, hipStream_t st) {                \
    const int64_t jobs = (int64_t)a.num_rows * a.tcnt;                                            \
    const dim3 grid((unsigned)((jobs + kWaves - 1) / kWaves)), block(kThreads);                   \
    if (head_dim == 128) {                                                                        \
      if (a.paged) hipLaunchKernelGGL((score_kernel<DT, 128, true>), grid, block, 0, st, a);      \
      else hipLaunchKernelGGL((score_kernel<DT, 128, false>), grid, block, 0, st, a);             \
    } else {                                                                                      \
      if (a.paged) hipLaunchKernelGGL((score_kernel<DT, 64, true>), grid, block, 0, st, a);       \
      else hipLaunchKernelGGL((score_kernel<DT, 64, false>), grid, block, 0, st, a);              \
    }                                                                                             \
    return hipGetLastError();                                                                     \
  }                                                                                               \
  template <>                                                                                     \
  hipError_t launch_fwht<DT>(const DecodeArgs& a, int head_dim, hipStream_t st) {                 \
    const int64_t jobs = (int64_t)a.num_rows * a.num_tiles;                                       \
    const dim3 grid((unsigned)((jobs + kWaves - 1) / kWaves)), block(kThreads);                   \
    if (head_dim == 128) {                                                                        \
      if (a.paged) hipLaunchKernelGGL((fwht_kernel<DT, 128, true>), grid, block, 0, st, a);       \
      else hipLaunchKernelGGL((fwht_kernel<DT, 128, false>), grid, block, 0, st, a);              \
    } else {                                                                                      \
      if (a.paged) hipLaunchKernelGGL((fwht_kernel<DT, 64, true>), grid, block, 0, st, a);        \
      else hipLaunchKernelGGL((fwht_kernel<DT, 64, false>), grid, block, 0, st, a);               \
    }                                                                                             \
    return hipGetLastError();                                                                     \
  }                                                                                               \
  template <>                                                                                     \
  hipError_t launch_band<DT>(const DecodeArgs& a, int head_dim, hipStream_t st) {                 \
    const int64_t jobs = (int64_t)a.num_rows * a.tcnt;                                            \
    const dim3 grid((unsigned)((jobs + kWaves - 1) / kWaves)), block(kThreads);                   \
    if (head_dim == 128) {                                                                        \
      if (a.paged) hipLaunchKernelGGL((band_norm_kernel<DT, 128, true>), grid, block, 0, st, a);  \
      else hipLaunchKernelGGL((band_norm_kernel<DT, 128, false>), grid, block, 0, st, a);         \
    } else {                                                                                      \
      if (a.paged) hipLaunchKernelGGL((band_norm_kernel<DT, 64, true>), grid, block, 0, st, a);   \
      else hipLaunchKernelGGL((band_norm_kernel<DT, 64, false>), grid, block, 0, st, a);          \
    }                                                                                             \
    return hipGetLastError();                                                                     \
  }

}  // namespace oc
