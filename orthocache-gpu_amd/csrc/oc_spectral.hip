// The 512-token block spectra of orthocache_forward(mode='compact') and its
// stream compaction (declared in include/orthocache_hip.h).
//
// The normalised 512-point Walsh-Hadamard transform along tokens, X =
// H512 K / sqrt(512) in natural (Hadamard) order, factors over the token
// index t = 64 th + tl and the sequency u = 64 uh + ul as H512[u, t] =
// H8[uh, th] H64[ul, tl].  With Z_uh[tl] = sum_th H8[uh, th] K[64 th + tl]
// (an 8-point transform across the block's eight 64-token chunks),
// X[64 uh + ul] = (H64 Z_uh)[ul] / sqrt(512), and by Parseval over ul
//   sum_ul ||X[64 uh + ul]||^2 = ||Z_uh||_F^2 / 8.
// So the bands [64, 256) (uh = 1..3) and [256, 512) (uh = 4..7) are sums of
// squares of the 8-point outputs, computed in registers as the block
// streams in; the band [1, 64) and the DC row need the 64-point transform
// of Z_0 along tl, done per column from LDS.  Every band energy is a sum of
// squares, so near-zero bands stay exact-ish instead of cancelling.
#include <hip/hip_runtime.h>

#include <cmath>

#include "oc_kernels.h"
#include "oc_status.h"
#include "orthocache_hip.h"

namespace oc {
namespace {

constexpr int kSpThreads = 256;
constexpr int kBlock = 512;
constexpr int kMaxD = 256;

struct SpecArgs {
  const char* k;
  int64_t k_ts, k_hs;  // byte strides: token, head
  int32_t H, d, nb, dtype;
  const char* q;       // (Sq, H, d) or null
  int64_t q_ss, q_hs;  // byte strides
  int32_t Sq, q_dtype;
  float* e_low;
  float* e_mid;
  float* e_high;
  float* zeta;
  float* e_ac;
  float* energy;
  float* mean;        // (nb, H, d) block mean = DC / sqrt(512), or null
  float* bounds;      // (Sq, nb, H) or null
  float* max_bound;   // (nb, H) or null
  float* q_norm_max;  // (H,) max_s ||q_s|| or null
};

// 16-byte pieces of one token position: the eight chunk values (th) of a
// thread's eight columns, fetched raw so that no use of the loaded words
// (no wait) sits among the loads
template <int DT>
struct SpRaw {
  static constexpr int N = DT == OC_F32 ? 16 : 8;
  uint4 w[N];
};

template <int DT>
__device__ __forceinline__ void sp_fetch(const char* p, int64_t th_stride, SpRaw<DT>& r) {
#pragma unroll
  for (int th = 0; th < 8; ++th) {
    const char* pt = p + th * th_stride;
    if constexpr (DT == OC_F32) {
      r.w[2 * th] = *reinterpret_cast<const uint4*>(pt);
      r.w[2 * th + 1] = *reinterpret_cast<const uint4*>(pt + 16);
    } else {
      r.w[th] = *reinterpret_cast<const uint4*>(pt);
    }
  }
}

// column c of chunk th as float
template <int DT>
__device__ __forceinline__ float sp_elem(const SpRaw<DT>& r, int th, int c) {
  if constexpr (DT == OC_F32) {
    const uint4 u = r.w[2 * th + c / 4];
    const uint32_t x = (c & 3) == 0 ? u.x : (c & 3) == 1 ? u.y : (c & 3) == 2 ? u.z : u.w;
    return __uint_as_float(x);
  } else {
    const uint4 u = r.w[th];
    const uint32_t x = (c >> 1) == 0 ? u.x : (c >> 1) == 1 ? u.y : (c >> 1) == 2 ? u.z : u.w;
    if constexpr (DT == OC_BF16) return __uint_as_float((c & 1) ? (x & 0xFFFF0000u) : (x << 16));
    else return (float)__builtin_bit_cast(_Float16, (uint16_t)((c & 1) ? (x >> 16) : (x & 0xFFFFu)));
  }
}

__device__ __forceinline__ float block_max(float v, float* sh_red) {
  v = wave_max(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh_red[w] = v;
  __syncthreads();
  float s = sh_red[0];
  for (int i = 1; i < kSpThreads / 64; ++i) s = fmaxf(s, sh_red[i]);
  return s;
}

// a q element's raw bits (zero-extended 16-bit, or float32) and its value
__device__ __forceinline__ float sp_q_value(uint32_t bits, int dtype) {
  if (dtype == OC_F32) return __uint_as_float(bits);
  if (dtype == OC_BF16) return __uint_as_float(bits << 16);
  return (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
}

template <int DT, int D>
__global__ __launch_bounds__(kSpThreads) void block_spectrum_kernel(const SpecArgs a) {
  constexpr int DMAX = D ? D : kMaxD;
  // Z_0[tl][c]; once the transform has read it (after the barrier that
  // follows), row 0 holds the block mean (each thread writes its own
  // column) and entries d .. d + 20 the reduction scratch, so the whole
  // workgroup's LDS is 32 KiB at d = 128 (five workgroups per CU)
  __shared__ float sh_z[64 * DMAX];
  float* sh_mean = sh_z;
  float (*sh_sum)[4] = reinterpret_cast<float (*)[4]>(sh_z + (D ? D : a.d));
  float* sh_red = sh_z + (D ? D : a.d) + 4 * (kSpThreads / 64);
  // consecutive workgroups take the heads of one block, so the workgroups
  // in flight together read whole token rows of the (S, H, d) cache
  const int h = blockIdx.x;
  const int blk = blockIdx.y;
  const int d = D ? D : a.d;
  const int CG = d / 8;
  const int TG = kSpThreads / CG;
  const int tid = threadIdx.x;
  const int cg = tid % CG;
  const int tg = tid / CG;
  const char* kb = a.k + (int64_t)blk * kBlock * a.k_ts + (int64_t)h * a.k_hs + (int64_t)cg * 8 * (DT == OC_F32 ? 4 : 2);
  // the bounds: wave w takes queries w, w + 4, ..., lane l columns l, l + 64, ...;
  // the wave's first query is requested before the block streams in
  constexpr int QPL = (DMAX + 63) / 64;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  // raw bits, converted where used: columns past d read column d - 1 (in
  // bounds) and are zeroed at the conversion
  auto load_q = [&](int s, uint32_t (&qr_bits)[QPL]) {
    const char* qr = a.q + (int64_t)s * a.q_ss + (int64_t)h * a.q_hs;
    if (a.q_dtype == OC_F32) {
#pragma unroll
      for (int k = 0; k < QPL; ++k)
        qr_bits[k] = *reinterpret_cast<const uint32_t*>(qr + (int64_t)min(lane + 64 * k, d - 1) * 4);
    } else {
#pragma unroll
      for (int k = 0; k < QPL; ++k)
        qr_bits[k] = *reinterpret_cast<const uint16_t*>(qr + (int64_t)min(lane + 64 * k, d - 1) * 2);
    }
  };
  uint32_t q0[QPL];
#pragma unroll
  for (int k = 0; k < QPL; ++k) q0[k] = 0u;
  if (a.q && wave < a.Sq) load_q(wave, q0);
  float e_mid = 0.f, e_high = 0.f, energy = 0.f;
  // one token position tl of the thread: energies, the 8-point transform
  // over the chunks th, Z_0 to LDS
  auto consume = [&](int tl, const SpRaw<DT>& r) {
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      float z[8];
#pragma unroll
      for (int th = 0; th < 8; ++th) {
        z[th] = sp_elem<DT>(r, th, c);
        energy = __builtin_fmaf(z[th], z[th], energy);
      }
      // natural-order 8-point Walsh-Hadamard transform over th (unnormalised)
#pragma unroll
      for (int m = 1; m < 8; m <<= 1)
#pragma unroll
        for (int i = 0; i < 8; ++i)
          if (!(i & m)) {
            const float u = z[i], v = z[i + m];
            z[i] = u + v;
            z[i + m] = u - v;
          }
#pragma unroll
      for (int uh = 1; uh < 4; ++uh) e_mid = __builtin_fmaf(z[uh], z[uh], e_mid);
#pragma unroll
      for (int uh = 4; uh < 8; ++uh) e_high = __builtin_fmaf(z[uh], z[uh], e_high);
      sh_z[tl * d + 8 * cg + c] = z[0];
    }
  };
  const int64_t th_stride = 64 * a.k_ts;
  if constexpr (D != 0) {
    // TG divides 64: 64 / TG positions per thread, the next position's
    // loads issued before the current one is consumed
    constexpr int TPT = 64 / (kSpThreads / (D / 8));
    SpRaw<DT> rb[2];
    sp_fetch<DT>(kb + (int64_t)tg * a.k_ts, th_stride, rb[0]);
#pragma unroll
    for (int i = 0; i < TPT; ++i) {
      if (i + 1 < TPT) sp_fetch<DT>(kb + (int64_t)(tg + (i + 1) * TG) * a.k_ts, th_stride, rb[(i + 1) & 1]);
      consume(tg + i * TG, rb[i & 1]);
    }
  } else if (tg < TG) {
    // any other head_dim: positions tg, tg + TG, ... < 64; the threads past
    // TG * CG (when CG does not divide 256) take none
    for (int tl = tg; tl < 64; tl += TG) {
      SpRaw<DT> r;
      sp_fetch<DT>(kb + (int64_t)tl * a.k_ts, th_stride, r);
      consume(tl, r);
    }
  }
  __syncthreads();
  // 64-point transform of Z_0 along tl, one column per thread
  float e_low = 0.f, dc2 = 0.f;
  if (tid < d) {
    float y[64];
#pragma unroll
    for (int i = 0; i < 64; ++i) y[i] = sh_z[i * d + tid];  // consecutive threads, consecutive words
#pragma unroll
    for (int m = 1; m < 64; m <<= 1)
#pragma unroll
      for (int i = 0; i < 64; ++i)
        if (!(i & m)) {
          const float u = y[i], v = y[i + m];
          y[i] = u + v;
          y[i + m] = u - v;
        }
#pragma unroll
    for (int i = 1; i < 64; ++i) e_low = __builtin_fmaf(y[i], y[i], e_low);
    dc2 = y[0] * y[0];
    sh_mean[tid] = y[0] * (1.0f / 512.0f);  // DC / sqrt(512) with DC = sum_t k_t / sqrt(512)
  }
  // the four band sums in one reduction: lanes, then the four waves in LDS
  float r4[4] = {e_mid, e_high, e_low, energy};
#pragma unroll
  for (int j = 0; j < 4; ++j) r4[j] = wave_sum(r4[j]);
  __syncthreads();  // every column of Z_0 has been read: the scratch entries are free
  if (lane == 0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) sh_sum[wave][j] = r4[j];
  }
  __syncthreads();  // also: sh_mean complete
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    r4[j] = sh_sum[0][j];
    for (int w = 1; w < kSpThreads / 64; ++w) r4[j] += sh_sum[w][j];
  }
  const float s_mid = r4[0] * 0.125f;
  const float s_high = r4[1] * 0.125f;
  const float s_low = r4[2] * (1.0f / 512.0f);
  const float s_energy = r4[3];
  (void)dc2;
  const float s_ac = s_low + s_mid + s_high;
  const int64_t o = (int64_t)blk * a.H + h;
  if (tid == 0) {
    if (a.e_low) a.e_low[o] = s_low;
    if (a.e_mid) a.e_mid[o] = s_mid;
    if (a.e_high) a.e_high[o] = s_high;
    if (a.zeta) a.zeta[o] = s_high / (s_low + 1e-6f);
    if (a.e_ac) a.e_ac[o] = s_ac;
    if (a.energy) a.energy[o] = s_energy;
  }
  if (a.mean && tid < d) a.mean[o * d + tid] = sh_mean[tid];
  if (!a.q) return;
  // query-aware bounds: (q . mean + ||q|| sqrt(E_ac)) / sqrt(d)
  const float inv_sd = 1.0f / __builtin_sqrtf((float)d);
  const float sq_ac = __builtin_sqrtf(fmaxf(s_ac, 0.f));
  float best = -__builtin_inff();
  float qbest = 0.f;
  for (int s = wave; s < a.Sq; s += kSpThreads / 64) {
    uint32_t qb[QPL];
    if (s == wave) {
#pragma unroll
      for (int k = 0; k < QPL; ++k) qb[k] = q0[k];
    } else {
      load_q(s, qb);
    }
    float dot = 0.f, nn = 0.f;
#pragma unroll
    for (int k = 0; k < QPL; ++k) {
      const int c = lane + 64 * k;
      if (c < d) {
        const float qv = sp_q_value(qb[k], a.q_dtype);
        dot = __builtin_fmaf(qv, sh_mean[c], dot);
        nn = __builtin_fmaf(qv, qv, nn);
      }
    }
    dot = wave_sum(dot);
    nn = wave_sum(nn);
    const float qn = __builtin_sqrtf(nn);
    const float bnd = dot * inv_sd + qn * sq_ac * inv_sd;
    if (a.bounds && lane == 0) a.bounds[((int64_t)s * a.nb + blk) * a.H + h] = bnd;
    best = fmaxf(best, bnd);
    qbest = fmaxf(qbest, qn);
  }
  best = block_max(best, sh_red);
  if (tid == 0 && a.max_bound) a.max_bound[o] = best;
  if (blk == 0 && a.q_norm_max) {
    qbest = block_max(qbest, sh_red);
    if (tid == 0) a.q_norm_max[h] = qbest;
  }
}

constexpr int kGateLds = 2048;   // (block, head) entries staged in LDS by the gate kernel
constexpr int kGateHeads = 256;  // query norms staged with them
constexpr int kGateBlocks = 2048;  // blocks whose per-block results the gate kernel keeps in LDS
constexpr int kGateWaves = 16;

// N values reduced over the 1024-thread workgroup at once: a DPP reduction
// per wave, then the 16 wave results from LDS (bit j of max_mask: maximum,
// else sum; identical result in every thread, fixed order).
template <int N>
__device__ __forceinline__ void gate_reduce(float (&v)[N], unsigned max_mask, float (*sh)[8]) {
  static_assert(N <= 8, "at most eight values per reduction");
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int j = 0; j < N; ++j) v[j] = ((max_mask >> j) & 1) ? wave_max(v[j]) : wave_sum(v[j]);
  __syncthreads();  // the previous reduction's reads of sh are done
  if (lane == 0) {
#pragma unroll
    for (int j = 0; j < N; ++j) sh[wave][j] = v[j];
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < N; ++j) {
    float t = sh[0][j];
    for (int w = 1; w < kGateWaves; ++w) t = ((max_mask >> j) & 1) ? fmaxf(t, sh[w][j]) : t + sh[w][j];
    v[j] = t;
  }
}

// The compact pipeline's gates and statistics in one workgroup over the
// (block, head) table (pipeline.py:458-527): tau (given, or mean - unbiased
// std of the max bounds), the two-gate mask, the any-head block mask and its
// tile expansion, the zeta statistics of the per-block head means, the
// retained count, the largest retained bound and the perfect / statistical
// regimes of the evicted blocks.  stats: [tau, zeta mean, zeta std, zeta
// min, zeta max, retained, perfect, statistical, z_max].
__global__ __launch_bounds__(1024) void compact_gate_kernel(const float* mb, const float* zeta, const float* energy,
                                                            const float* qmax, int nb, int H, int d, float tau_in,
                                                            int tau_auto, float zeta_max, float underflow,
                                                            int tiles_per_block, uint8_t* unified,
                                                            uint8_t* tile_mask, float* stats) {
  __shared__ float sh_f[kGateWaves][8];
  // the (block, head) tables and the query norms staged in LDS when they
  // fit, every load in flight at once; otherwise read from global memory
  __shared__ float sh_mb[kGateLds], sh_zeta[kGateLds], sh_en[kGateLds], sh_qmax[kGateHeads];
  // per-block results of the first pass (any head kept, head-mean zeta, beta)
  __shared__ float sh_za[kGateBlocks], sh_beta[kGateBlocks];
  __shared__ uint8_t sh_any[kGateBlocks];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int n = nb * H;
  const bool staged = n <= kGateLds && H <= kGateHeads;
  const bool cache_blk = nb <= kGateBlocks;
  if (staged) {
#pragma unroll
    for (int k = 0; k < kGateLds / 1024; ++k) {
      const int i = tid + 1024 * k;
      if (i < n) {
        sh_mb[i] = mb[i];
        sh_zeta[i] = zeta[i];
        sh_en[i] = energy[i];
      }
    }
    if (tid < H) sh_qmax[tid] = qmax[tid];
    __syncthreads();
    mb = sh_mb;
    zeta = sh_zeta;
    energy = sh_en;
    qmax = sh_qmax;
  }
  float tau = tau_in;
  if (tau_auto) {
    float s[1] = {0.f};
    for (int i = tid; i < n; i += 1024) s[0] += mb[i];
    gate_reduce<1>(s, 0u, sh_f);
    const float mean = s[0] / (float)n;
    float v[1] = {0.f};
    for (int i = tid; i < n; i += 1024) v[0] = __builtin_fmaf(mb[i] - mean, mb[i] - mean, v[0]);
    gate_reduce<1>(v, 0u, sh_f);
    const float var = v[0] / (float)(n - 1);  // n = 1: NaN, as torch.std
    tau = mean - __builtin_sqrtf(var);
  }
  // per block (one wave per block, lanes over heads): any head retained,
  // head-mean zeta, largest bound, beta = max_h qmax_h sqrt(E) / sqrt(d)
  const float isd = 1.0f / __builtin_sqrtf((float)d);
  struct Blk {
    bool any;
    float za, bmx, beta;
  };
  auto block_stats = [&](int b) {
    bool any = false;
    float zsum = 0.f, bmx = -__builtin_inff(), beta = -__builtin_inff();
    for (int h = lane; h < H; h += 64) {
      const float m = mb[(int64_t)b * H + h], z = zeta[(int64_t)b * H + h];
      any = any || (m >= tau && z <= zeta_max);
      zsum += z;
      bmx = fmaxf(bmx, m);
      beta = fmaxf(beta, qmax[h] * __builtin_sqrtf(fmaxf(energy[(int64_t)b * H + h], 0.f)) * isd);
    }
    return Blk{__ballot(any) != 0, wave_sum(zsum) / (float)H, wave_max(bmx), wave_max(beta)};
  };
  // r1: zeta sum, retained (sums); -zeta min, zeta max, best retained bound (maxima)
  float r1[5] = {0.f, 0.f, -__builtin_inff(), -__builtin_inff(), -__builtin_inff()};
  for (int b = wave; b < nb; b += kGateWaves) {
    const Blk k = block_stats(b);
    for (int t = lane; t < tiles_per_block; t += 64) tile_mask[(int64_t)b * tiles_per_block + t] = k.any ? 1 : 0;
    if (lane == 0) {
      unified[b] = k.any ? 1 : 0;
      if (cache_blk) {
        sh_any[b] = k.any ? 1 : 0;
        sh_za[b] = k.za;
        sh_beta[b] = k.beta;
      }
      r1[0] += k.za;
      r1[1] += k.any ? 1.f : 0.f;
      r1[2] = fmaxf(r1[2], -k.za);
      r1[3] = fmaxf(r1[3], k.za);
      if (k.any) r1[4] = fmaxf(r1[4], k.bmx);
    }
  }
  gate_reduce<5>(r1, 0x1Cu, sh_f);  // its barriers also publish sh_any / sh_za / sh_beta
  const float zmean = r1[0] / (float)nb;
  const float retained = r1[1];
  const float zmin = -r1[2], zmx = r1[3];
  const float zmax_ret = retained == 0.f ? 0.f : r1[4];
  // r2: squared zeta deviations, perfect and statistical evictions
  float r2[3] = {0.f, 0.f, 0.f};
  auto regime = [&](bool any, float za, float beta) {
    r2[0] = __builtin_fmaf(za - zmean, za - zmean, r2[0]);
    if (!any) {
      if (zmax_ret - beta >= underflow) r2[1] += 1.f;
      else r2[2] += 1.f;
    }
  };
  if (cache_blk) {
    for (int b = tid; b < nb; b += 1024) regime(sh_any[b] != 0, sh_za[b], sh_beta[b]);
  } else {
    for (int b = wave; b < nb; b += kGateWaves) {
      const Blk k = block_stats(b);
      if (lane == 0) regime(k.any, k.za, k.beta);
    }
  }
  gate_reduce<3>(r2, 0u, sh_f);
  if (tid == 0) {
    stats[0] = tau;
    stats[1] = zmean;
    stats[2] = __builtin_sqrtf(r2[0] / (float)(nb - 1));
    stats[3] = zmin;
    stats[4] = zmx;
    stats[5] = retained;
    stats[6] = r2[1];
    stats[7] = r2[2];
    stats[8] = zmax_ret;
  }
}

// NaN-propagating maximum (torch.max semantics): a NaN operand wins
__device__ __forceinline__ float nan_max(float a, float b) { return (a != a || a >= b) ? a : b; }

// Eviction regimes of a block table (perfect_eviction.py:75-186 as
// orthocache_forward and its callers use it), one workgroup:
//   qn[h]   = max_s q_norms[s, h]                       (NaN propagates)
//   b[b, h] = qn[h] * sqrt(E[b, h] clamped at 0) / sqrt_d  (float32, NaN kept)
//   beta[b] = max_h b[b, h];  gap[b] = z - beta[b]
//   regime  = 0 when any of the block's mask entries is set (retained);
//             else 1 when gap >= underflow, 2 when gap < underflow, and 0
//             when gap is NaN (neither compare holds)
// counts = (regime-1 blocks, regime-2 blocks, retained blocks).  z is the
// largest of z_vec[0 .. z_count) when given (NaN propagates), else z_scalar.
__global__ __launch_bounds__(1024) void block_regimes_kernel(const float* qnorms, int sq, int H, const float* energy,
                                                             int nb, float sqrt_d, float z_scalar, const float* z_vec,
                                                             int z_count, const uint8_t* mask, int mask_heads,
                                                             float underflow, int32_t* regime, float* beta,
                                                             float* gap, float* beta_full, int32_t* counts) {
  __shared__ float sh_qn[kGateHeads];
  __shared__ float sh_f[kGateWaves][8];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // z: the reduction runs in every wave over the same lanes, so each wave
  // ends with the same value (no barrier needed)
  float z = z_scalar;
  if (z_vec) {
    float m = -__builtin_inff();
    for (int i = lane; i < z_count; i += 64) m = nan_max(m, z_vec[i]);
    for (int o = 32; o > 0; o >>= 1) m = nan_max(m, __shfl_xor(m, o, 64));
    z = m;
  }
  // per-head query norm maxima; heads past the LDS table are re-derived
  // where they are used
  auto head_qmax = [&](int h) {
    float m = -__builtin_inff();
    for (int s = 0; s < sq; ++s) m = nan_max(m, qnorms[(int64_t)s * H + h]);
    return m;
  };
  for (int h = threadIdx.x; h < H && h < kGateHeads; h += 1024) sh_qn[h] = head_qmax(h);
  __syncthreads();
  // one wave per block, lanes over heads
  float cnt[3] = {0.f, 0.f, 0.f};
  for (int b = wave; b < nb; b += kGateWaves) {
    float bm = -__builtin_inff();
    bool kept = false;
    for (int h = lane; h < H; h += 64) {
      const float e = energy[(int64_t)b * H + h];
      const float qn = h < kGateHeads ? sh_qn[h] : head_qmax(h);
      const float x = qn * __builtin_sqrtf(e < 0.f ? 0.f : e) / sqrt_d;
      if (beta_full) beta_full[(int64_t)b * H + h] = x;
      bm = nan_max(bm, x);
      if (mask_heads > 1) kept = kept || mask[(int64_t)b * mask_heads + h] != 0;
    }
    for (int o = 32; o > 0; o >>= 1) bm = nan_max(bm, __shfl_xor(bm, o, 64));
    kept = mask_heads > 1 ? __ballot(kept) != 0 : mask[b] != 0;
    if (lane == 0) {
      const float g = z - bm;
      const int r = kept ? 0 : (g >= underflow ? 1 : (g < underflow ? 2 : 0));
      regime[b] = r;
      beta[b] = bm;
      gap[b] = g;
      cnt[0] += r == 1 ? 1.f : 0.f;
      cnt[1] += r == 2 ? 1.f : 0.f;
      cnt[2] += kept ? 1.f : 0.f;
    }
  }
  gate_reduce<3>(cnt, 0u, sh_f);  // exact: counts below 2^24
  if (threadIdx.x == 0) {
    counts[0] = (int32_t)cnt[0];
    counts[1] = (int32_t)cnt[1];
    counts[2] = (int32_t)cnt[2];
  }
}

// Active-first stable order of n blocks (stream compaction): out[r] = the
// r-th retained block, then the evicted ones in order; *num_active = the
// retained count.  One workgroup of 1024 threads, chunked prefix sums.
__global__ __launch_bounds__(1024) void stream_compact_kernel(const uint8_t* mask, int n, int64_t* out,
                                                              int32_t* num_active) {
  __shared__ int sh[1024];
  __shared__ int sh_total;
  const int tid = threadIdx.x;
  int cnt = 0;
  for (int i = tid; i < n; i += 1024) cnt += mask[i] ? 1 : 0;
  for (int o = 32; o > 0; o >>= 1) cnt += __shfl_xor(cnt, o, 64);
  if (tid == 0) sh_total = 0;
  __syncthreads();
  if ((tid & 63) == 0) atomicAdd(&sh_total, cnt);
  __syncthreads();
  const int total = sh_total;
  int base_a = 0;
  for (int c0 = 0; c0 < n; c0 += 1024) {
    const int i = c0 + tid;
    const int f = (i < n && mask[i]) ? 1 : 0;
    sh[tid] = f;
    __syncthreads();
    for (int off = 1; off < 1024; off <<= 1) {  // inclusive Hillis-Steele scan
      const int v = tid >= off ? sh[tid - off] : 0;
      __syncthreads();
      sh[tid] += v;
      __syncthreads();
    }
    const int incl = sh[tid];
    const int chunk_a = sh[1023];
    if (i < n) {
      const int ra = base_a + incl - f;           // retained before i
      const int r = f ? ra : total + (i - ra);     // evicted before i: i - ra
      out[r] = i;
    }
    base_a += chunk_a;
    __syncthreads();
  }
  if (tid == 0 && num_active) *num_active = total;
}

template <int DT>
int launch_spectrum(const SpecArgs& a, hipStream_t s) {
  if (a.d == 128)
    hipLaunchKernelGGL((block_spectrum_kernel<DT, 128>), dim3(a.H, a.nb), dim3(kSpThreads), 0, s, a);
  else if (a.d == 64)
    hipLaunchKernelGGL((block_spectrum_kernel<DT, 64>), dim3(a.H, a.nb), dim3(kSpThreads), 0, s, a);
  else
    hipLaunchKernelGGL((block_spectrum_kernel<DT, 0>), dim3(a.H, a.nb), dim3(kSpThreads), 0, s, a);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? OC_OK : hip_fail(e, "block-spectrum launch");
}

}  // namespace
}  // namespace oc

using namespace oc;

extern "C" int oc_block_spectra(const oc_spectra_params* p, void* stream) {
  if (!p || !p->k) return fail(OC_ERR_INVALID, "NULL pointer");
  if (p->dtype != OC_F32 && p->dtype != OC_F16 && p->dtype != OC_BF16) return fail(OC_ERR_INVALID, "dtype %d", p->dtype);
  if (p->block_size != kBlock) return fail(OC_ERR_UNSUPPORTED, "block_size %d (the transform is 512-point)", p->block_size);
  if (p->head_dim < 8 || p->head_dim > kMaxD || p->head_dim % 8)
    return fail(OC_ERR_UNSUPPORTED, "head_dim %d (a multiple of 8 up to %d)", p->head_dim, kMaxD);
  if (p->num_blocks < 0 || p->num_heads < 0 || p->q_len < 0) return fail(OC_ERR_INVALID, "bad sizes");
  const int es = p->dtype == OC_F32 ? 4 : 2;
  if ((p->k_token_stride * es) % 16 || (p->k_head_stride * es) % 16 || ((uintptr_t)p->k % 16))
    return fail(OC_ERR_INVALID, "K rows must be 16-byte aligned");
  if (p->q && p->q_dtype != OC_F32 && p->q_dtype != OC_F16 && p->q_dtype != OC_BF16)
    return fail(OC_ERR_INVALID, "q dtype %d", p->q_dtype);
  if ((p->bounds || p->max_bound || p->q_norm_max) && !p->q) return fail(OC_ERR_INVALID, "bounds need q");
  if (p->num_blocks == 0 || p->num_heads == 0) return OC_OK;
  if (p->num_blocks > 65535) return fail(OC_ERR_UNSUPPORTED, "num_blocks > 65535 (33553920 tokens)");
  SpecArgs a{};
  a.k = (const char*)p->k;
  a.k_ts = p->k_token_stride * es, a.k_hs = p->k_head_stride * es;
  a.H = p->num_heads, a.d = p->head_dim, a.nb = p->num_blocks, a.dtype = p->dtype;
  a.q = (const char*)p->q;
  const int qes = p->q_dtype == OC_F32 ? 4 : 2;
  a.q_ss = p->q_token_stride * qes, a.q_hs = p->q_head_stride * qes;
  a.Sq = p->q ? p->q_len : 0;
  a.q_dtype = p->q_dtype;
  a.e_low = p->e_low, a.e_mid = p->e_mid, a.e_high = p->e_high, a.zeta = p->zeta;
  a.e_ac = p->e_ac, a.energy = p->energy, a.mean = p->block_mean;
  a.bounds = p->bounds, a.max_bound = p->max_bound, a.q_norm_max = p->q_norm_max;
  const hipStream_t s = (hipStream_t)stream;
  switch (p->dtype) {
    case OC_F32: return launch_spectrum<OC_F32>(a, s);
    case OC_F16: return launch_spectrum<OC_F16>(a, s);
    default: return launch_spectrum<OC_BF16>(a, s);
  }
}

extern "C" int oc_stream_compact(const uint8_t* block_mask, int32_t num_blocks, int64_t* indices,
                                 int32_t* num_active, void* stream) {
  if (!block_mask || !indices) return fail(OC_ERR_INVALID, "NULL pointer");
  if (num_blocks < 0) return fail(OC_ERR_INVALID, "bad sizes");
  if (num_blocks == 0) return OC_OK;
  hipLaunchKernelGGL(stream_compact_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, block_mask, num_blocks,
                     indices, num_active);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? OC_OK : hip_fail(e, "stream-compact launch");
}

extern "C" int oc_compact_gate(const float* max_bound, const float* zeta, const float* energy, const float* q_norm_max,
                               int32_t num_blocks, int32_t num_heads, int32_t head_dim, double tau, int32_t tau_auto,
                               double zeta_max, double underflow, int32_t tiles_per_block, uint8_t* block_mask,
                               uint8_t* tile_mask, float* stats, void* stream) {
  if (!max_bound || !zeta || !energy || !q_norm_max || !block_mask || !tile_mask || !stats)
    return fail(OC_ERR_INVALID, "NULL pointer");
  if (num_blocks < 1 || num_heads < 1 || head_dim < 1 || tiles_per_block < 1) return fail(OC_ERR_INVALID, "bad sizes");
  hipLaunchKernelGGL(compact_gate_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, max_bound, zeta, energy,
                     q_norm_max, num_blocks, num_heads, head_dim, (float)tau, tau_auto, (float)zeta_max,
                     (float)underflow, tiles_per_block, block_mask, tile_mask, stats);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? OC_OK : hip_fail(e, "compact-gate launch");
}

extern "C" int oc_block_regimes(const float* q_norms, int32_t q_len, int32_t num_heads, const float* energy,
                                int32_t num_blocks, int32_t head_dim, double z_max, const float* z_values,
                                int32_t z_count, const uint8_t* block_mask, int32_t mask_heads, double underflow,
                                int32_t* regime, float* beta, float* gap, float* beta_full, int32_t* counts,
                                void* stream) {
  if (!q_norms || !energy || !block_mask || !regime || !beta || !gap || !counts)
    return fail(OC_ERR_INVALID, "NULL pointer");
  if (q_len < 1 || num_heads < 1 || num_blocks < 0 || head_dim < 1 || (z_values && z_count < 1))
    return fail(OC_ERR_INVALID, "bad sizes");
  if (mask_heads != 1 && mask_heads != num_heads)
    return fail(OC_ERR_INVALID, "mask_heads %d must be 1 or num_heads %d", mask_heads, num_heads);
  if (num_blocks >= (1 << 24)) return fail(OC_ERR_UNSUPPORTED, "num_blocks %d >= 2^24", num_blocks);
  // the divisor as the reference forms it: math.sqrt(head_dim) taken to float32
  const float sqrt_d = (float)std::sqrt((double)head_dim);
  hipLaunchKernelGGL(block_regimes_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, q_norms, q_len, num_heads,
                     energy, num_blocks, sqrt_d, (float)z_max, z_values, z_count, block_mask, mask_heads,
                     (float)underflow, regime, beta, gap, beta_full, counts);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? OC_OK : hip_fail(e, "block-regimes launch");
}

extern "C" size_t oc_spectra_params_bytes(void) { return sizeof(oc_spectra_params); }
