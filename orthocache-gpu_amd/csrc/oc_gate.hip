// The O(1) decode gate from cached K band norms, the Walsh-subspace q norm
// and the tile mask on attention logits (declared in
// include/orthocache_hip.h).  These are small per-head kernels: the gate
// reads one float per tile, so it is bound by launch latency and the q
// loads, not by HBM bandwidth.
#include <hip/hip_runtime.h>

#include <cmath>

#include "oc_status.h"
#include "orthocache_hip.h"

namespace oc {
namespace {

constexpr int kGateThreads = 256;
constexpr int kMaxHeadDim = 1024;

__device__ __forceinline__ float load_q(const char* p, int dtype) {
  if (dtype == OC_F32) return *reinterpret_cast<const float*>(p);
  const uint16_t h = *reinterpret_cast<const uint16_t*>(p);
  if (dtype == OC_BF16) return __uint_as_float((uint32_t)h << 16);
  return (float)__builtin_bit_cast(_Float16, h);
}

__device__ __forceinline__ float wave_sum64(float x) {
  for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off, 64);
  return x;
}

// Squared norm of one q row and, with low_band > 0, its Walsh-subspace
// high part ||q||^2 - sum_i S_i^2 / bs (compute_q_high_norm_exact,
// decode_gate.py:86-98): S_i sums blocks of bs = d / low_band elements.
// One wave; lane l takes elements l, l + 64, ...; the block sums go
// through LDS (sh: >= d floats for this wave).
__device__ float q_row_sq(const char* q, int dtype, int d, int low_band, float* sh, int lane) {
  const int es = dtype == OC_F32 ? 4 : 2;
  float ss = 0.f;
  for (int c = lane; c < d; c += 64) {
    const float x = load_q(q + (int64_t)c * es, dtype);
    sh[c] = x;
    ss = __builtin_fmaf(x, x, ss);
  }
  ss = wave_sum64(ss);
  if (low_band <= 0) return ss;
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const int bs = d / low_band;
  float lo = 0.f;
  for (int i = lane; i < low_band; i += 64) {
    float s = 0.f;
    for (int k = 0; k < bs; ++k) s += sh[i * bs + k];
    lo = __builtin_fmaf(s, s, lo);
  }
  lo = wave_sum64(lo) / (float)bs;
  const float hi = ss - lo;
  return hi < 0.f ? 0.f : hi;  // clamp(min=0); NaN stays NaN
}

// One workgroup per kv head (decode_gate.py:108-181): q norm = max over the
// head's G query rows (spatial: the largest ||q_g||^2, then sqrt, as the
// Triton kernel does; Walsh high: the NaN-propagating max of the norms, as
// torch.max does), then one compare per tile.
__global__ __launch_bounds__(kGateThreads) void decode_gate_kernel(
    const char* q, int q_dtype, int64_t q_row_bytes, int G, int d, const float* nc, int64_t nc_stride,
    int num_tiles, int max_tiles, float tau_norm, int mode, int low_band, uint8_t* mask, int64_t mask_stride,
    float* q_norms) {
  __shared__ float sh_q[kGateThreads / 64][kMaxHeadDim];
  __shared__ float sh_n[kGateThreads / 64];
  const int h = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  float best = 0.f;
  bool nan = false;
  for (int g = wave; g < G; g += kGateThreads / 64) {
    const char* qr = q + (int64_t)(h * G + g) * q_row_bytes;
    const float sq = q_row_sq(qr, q_dtype, d, mode == OC_QNORM_WALSH_HIGH ? low_band : 0, sh_q[wave], lane);
    if (mode == OC_QNORM_WALSH_HIGH) {
      const float n = __builtin_sqrtf(sq);
      nan = nan || __builtin_isnan(n);
      best = n > best ? n : best;
    } else {
      best = sq > best ? sq : best;
    }
  }
  if (lane == 0) sh_n[wave] = nan ? __builtin_nanf("") : best;
  __syncthreads();
  float qn = 0.f;
  bool any_nan = false;
  for (int w = 0; w < kGateThreads / 64; ++w) {
    const float x = sh_n[w];
    any_nan = any_nan || __builtin_isnan(x);
    qn = x > qn ? x : qn;
  }
  if (mode == OC_QNORM_WALSH_HIGH) {
    if (any_nan) qn = __builtin_nanf("");
  } else {
    qn = __builtin_sqrtf(qn);
  }
  if (threadIdx.x == 0 && q_norms) q_norms[h] = qn;
  for (int t = threadIdx.x; t < max_tiles; t += kGateThreads) {
    uint8_t ev = 0;
    if (t < num_tiles) ev = (qn * nc[(int64_t)h * nc_stride + t] <= tau_norm) ? 1 : 0;
    mask[(int64_t)h * mask_stride + t] = ev;
  }
}

// One wave per q row.
__global__ __launch_bounds__(kGateThreads) void q_high_norm_kernel(const char* q, int q_dtype, int64_t rows,
                                                                   int d, int64_t q_row_bytes, int low_band,
                                                                   float* out) {
  __shared__ float sh_q[kGateThreads / 64][kMaxHeadDim];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * (kGateThreads / 64) + wave;
  if (r >= rows) return;
  const float sq = q_row_sq(q + r * q_row_bytes, q_dtype, d, low_band, sh_q[wave], lane);
  if (lane == 0) out[r] = __builtin_sqrtf(sq);
}

// grid (ceil(seq_len / 256), num_q_heads)
__global__ __launch_bounds__(kGateThreads) void apply_mask_kernel(char* logits, int dtype, int64_t seq_len,
                                                                  int64_t row_elems, const uint8_t* mask,
                                                                  int64_t mask_stride, int G, int tile,
                                                                  int num_tiles) {
  const int64_t s = (int64_t)blockIdx.x * kGateThreads + threadIdx.x;
  const int h = blockIdx.y;
  if (s >= seq_len) return;
  const int64_t t = s / tile;
  if (t >= num_tiles || !mask[(int64_t)(h / G) * mask_stride + t]) return;
  const int64_t i = (int64_t)h * row_elems + s;
  if (dtype == OC_F32) reinterpret_cast<float*>(logits)[i] = -__builtin_inff();
  else if (dtype == OC_BF16) reinterpret_cast<uint16_t*>(logits)[i] = 0xFF80u;
  else reinterpret_cast<uint16_t*>(logits)[i] = 0xFC00u;
}

// tile mask of a block mask (block_mask given) or zeros (indices given)
__global__ __launch_bounds__(kGateThreads) void block_tile_mask_kernel(const uint8_t* block_mask, int64_t n_tiles,
                                                                       int tpb, uint8_t* tile_mask) {
  const int64_t t = (int64_t)blockIdx.x * kGateThreads + threadIdx.x;
  if (t >= n_tiles) return;
  tile_mask[t] = block_mask ? (block_mask[t / tpb] ? 1 : 0) : 0;
}

// set the tiles of every listed block; indices outside the range raise the flag
__global__ __launch_bounds__(kGateThreads) void index_tile_mask_kernel(const int32_t* indices, int count,
                                                                       int num_blocks, int tpb, uint8_t* tile_mask,
                                                                       int32_t* error_flag) {
  const int i = blockIdx.x * kGateThreads + threadIdx.x;
  if (i >= count) return;
  const int b = indices[i];
  if (b < 0 || b >= num_blocks) {
    if (error_flag) atomicOr(error_flag, 1);
    return;
  }
  for (int k = 0; k < tpb; ++k) tile_mask[(int64_t)b * tpb + k] = 1;
}

bool float_dtype(int dt) { return dt == OC_F32 || dt == OC_F16 || dt == OC_BF16; }

}  // namespace
}  // namespace oc

using namespace oc;

extern "C" int oc_decode_gate(const void* q, int32_t q_dtype, int64_t q_row_stride, int32_t num_kv_heads, int32_t G,
                              int32_t head_dim, const float* norm_cache, int64_t norm_row_stride, int32_t num_tiles,
                              int32_t max_tiles, double tau_norm, int32_t q_norm_mode, int32_t low_band,
                              uint8_t* mask, int64_t mask_row_stride, float* q_norms, void* stream) {
  if (!q || !norm_cache || !mask) return fail(OC_ERR_INVALID, "NULL pointer");
  if (!float_dtype(q_dtype)) return fail(OC_ERR_INVALID, "q dtype %d", q_dtype);
  if (num_kv_heads < 0 || G < 1 || head_dim < 1 || head_dim > kMaxHeadDim || num_tiles < 0 || max_tiles < 0 ||
      num_tiles > max_tiles)
    return fail(OC_ERR_INVALID, "bad sizes");
  if (q_norm_mode != OC_QNORM_SPATIAL && q_norm_mode != OC_QNORM_WALSH_HIGH)
    return fail(OC_ERR_INVALID, "q_norm_mode %d", q_norm_mode);
  if (q_norm_mode == OC_QNORM_WALSH_HIGH && (low_band < 1 || head_dim % low_band))
    return fail(OC_ERR_INVALID, "head_dim %d not divisible by low_band %d", head_dim, low_band);
  if (num_kv_heads == 0) return OC_OK;
  const int es = q_dtype == OC_F32 ? 4 : 2;
  hipLaunchKernelGGL(decode_gate_kernel, dim3(num_kv_heads), dim3(kGateThreads), 0, (hipStream_t)stream,
                     (const char*)q, q_dtype, q_row_stride * es, G, head_dim, norm_cache, norm_row_stride, num_tiles,
                     max_tiles, (float)tau_norm, q_norm_mode, low_band, mask, mask_row_stride, q_norms);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? OC_OK : hip_fail(e, "decode-gate launch");
}

extern "C" int oc_q_high_norms(const void* q, int32_t q_dtype, int64_t rows, int32_t head_dim, int64_t q_row_stride,
                               int32_t low_band, float* out, void* stream) {
  if (!q || !out) return fail(OC_ERR_INVALID, "NULL pointer");
  if (!float_dtype(q_dtype)) return fail(OC_ERR_INVALID, "q dtype %d", q_dtype);
  if (rows < 0 || head_dim < 1 || head_dim > kMaxHeadDim) return fail(OC_ERR_INVALID, "bad sizes");
  if (low_band < 1 || head_dim % low_band)
    return fail(OC_ERR_INVALID, "head_dim %d not divisible by low_band %d", head_dim, low_band);
  if (rows == 0) return OC_OK;
  const int es = q_dtype == OC_F32 ? 4 : 2;
  const int64_t blocks = (rows + kGateThreads / 64 - 1) / (kGateThreads / 64);
  if (blocks > 0x7FFFFFFF) return fail(OC_ERR_UNSUPPORTED, "too many rows");
  hipLaunchKernelGGL(q_high_norm_kernel, dim3((unsigned)blocks), dim3(kGateThreads), 0, (hipStream_t)stream,
                     (const char*)q, q_dtype, rows, head_dim, q_row_stride * es, low_band, out);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? OC_OK : hip_fail(e, "q-norm launch");
}

extern "C" int oc_apply_tile_mask(void* logits, int32_t dtype, int32_t num_q_heads, int64_t seq_len,
                                  int64_t logits_row_stride, const uint8_t* mask, int64_t mask_row_stride, int32_t G,
                                  int32_t tile_size, int32_t num_tiles, void* stream) {
  if (!logits || !mask) return fail(OC_ERR_INVALID, "NULL pointer");
  if (!float_dtype(dtype)) return fail(OC_ERR_INVALID, "logits dtype %d", dtype);
  if (num_q_heads < 0 || seq_len < 0 || G < 1 || tile_size < 1 || num_tiles < 0 || num_q_heads > 65535)
    return fail(OC_ERR_INVALID, "bad sizes");
  if (num_q_heads == 0 || seq_len == 0 || num_tiles == 0) return OC_OK;
  const int64_t blocks = (seq_len + kGateThreads - 1) / kGateThreads;
  if (blocks > 0x7FFFFFFF) return fail(OC_ERR_UNSUPPORTED, "seq_len too large");
  hipLaunchKernelGGL(apply_mask_kernel, dim3((unsigned)blocks, num_q_heads), dim3(kGateThreads), 0,
                     (hipStream_t)stream, (char*)logits, dtype, seq_len, logits_row_stride, mask, mask_row_stride, G,
                     tile_size, num_tiles);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? OC_OK : hip_fail(e, "mask launch");
}

extern "C" int oc_tile_mask_from_blocks(const uint8_t* block_mask, const int32_t* indices, int32_t count,
                                        int32_t num_blocks, int32_t tiles_per_block, uint8_t* tile_mask,
                                        int32_t* error_flag, void* stream) {
  if (!tile_mask || (!block_mask && !indices) || (block_mask && indices))
    return fail(OC_ERR_INVALID, "give exactly one of block_mask and indices, and tile_mask");
  if (num_blocks < 0 || tiles_per_block < 1 || count < 0) return fail(OC_ERR_INVALID, "bad sizes");
  const int64_t n_tiles = (int64_t)num_blocks * tiles_per_block;
  if (n_tiles == 0) return OC_OK;
  const int64_t blocks = (n_tiles + kGateThreads - 1) / kGateThreads;
  if (blocks > 0x7FFFFFFF) return fail(OC_ERR_UNSUPPORTED, "too many tiles");
  hipLaunchKernelGGL(block_tile_mask_kernel, dim3((unsigned)blocks), dim3(kGateThreads), 0, (hipStream_t)stream,
                     block_mask, n_tiles, tiles_per_block, tile_mask);
  if (indices && count > 0)
    hipLaunchKernelGGL(index_tile_mask_kernel, dim3((unsigned)((count + kGateThreads - 1) / kGateThreads)),
                       dim3(kGateThreads), 0, (hipStream_t)stream, indices, count, num_blocks, tiles_per_block,
                       tile_mask, error_flag);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? OC_OK : hip_fail(e, "tile-mask launch");
}
