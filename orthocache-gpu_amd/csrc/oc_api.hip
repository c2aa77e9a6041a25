// C ABI of liborthocache_hip (declared in include/orthocache_hip.h):
// argument validation, workspace carving, kernel dispatch and the
// log-sum-exp merge kernel.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <algorithm>
#include <cstring>
#include <mutex>
#include <string>

#include "oc_generic.h"
#include "oc_kernels.h"
#include "oc_status.h"
#include "orthocache_hip.h"

namespace oc {

static thread_local std::string g_last_error;

void set_last_error(const char* msg) { g_last_error = msg; }

static int elem_size(int dt) {
  switch (dt) {
    case OC_F32: return 4;
    case OC_F16: case OC_BF16: return 2;
    case OC_FP8_E4M3FN: return 1;
    default: return 0;
  }
}

static bool aligned(const void* p, int64_t a) { return ((uintptr_t)p % (uintptr_t)a) == 0; }

// Validates the KV descriptor and fills the layout part of DecodeArgs.
// allow_dq: the entry point implements OC_KSCALE_DEQUANT (decode, scoring)
static int fill_kv(const oc_kv_desc* kv, DecodeArgs& a, bool allow_dq = false) {
  if (!kv) return fail(OC_ERR_INVALID, "kv descriptor is NULL");
  const int es = elem_size(kv->dtype);
  if (!es) return fail(OC_ERR_INVALID, "unknown K/V dtype %d", kv->dtype);
  // V's own element type: K's, or bf16 beside fp8 K
  const bool v_bf16 = kv->v_dtype != 0 && kv->v_dtype != kv->dtype;
  if (v_bf16 && (kv->dtype != OC_FP8_E4M3FN || kv->v_dtype != OC_BF16))
    return fail(OC_ERR_UNSUPPORTED, "V dtype %d beside K dtype %d (a different V type is bf16 beside fp8 K only)",
                kv->v_dtype, kv->dtype);
  const int ves = v_bf16 ? 2 : es;
  const int ts = kv->tile_size > 0 ? kv->tile_size : 64;
  if (kv->tile_size < 0 || !generic_supported(kv->head_dim, ts))
    return fail(OC_ERR_UNSUPPORTED, "head_dim %d with %d-token tiles not supported (powers of two, head_dim <= 512, "
                "tile_size <= 256)", kv->head_dim, ts);
  const bool tuned = !generic_shape(kv->head_dim, ts);
  if (kv->num_rows < 0 || kv->num_tiles < 0) return fail(OC_ERR_INVALID, "negative sizes");
  if (kv->num_rows > 65535) return fail(OC_ERR_UNSUPPORTED, "num_rows %d > 65535", kv->num_rows);
  if (!kv->k) return fail(OC_ERR_INVALID, "K pointer is NULL");
  // bytes per lane per token row, and the alignment of every K (V) offset
  // (the portable kernels read element by element: element alignment)
  auto align_of = [&](int e) -> int64_t {
    if (!tuned) return e;
    const int64_t lb = (int64_t)(kv->head_dim / 16) * e;
    return lb < 16 ? lb : 16;
  };
  const int64_t al = align_of(es), val = align_of(ves);
  auto chk = [&](int64_t stride_el, const char* what, bool is_v) -> int {
    const int64_t e = is_v ? ves : es, x = is_v ? val : al;
    if ((stride_el * e) % x) return fail(OC_ERR_INVALID, "%s stride %lld not a multiple of %lld bytes",
                                         what, (long long)stride_el, (long long)x);
    return OC_OK;
  };
  if (!aligned(kv->k, al) || (kv->v && !aligned(kv->v, val)))
    return fail(OC_ERR_INVALID, "K/V base pointers must be %lld/%lld-byte aligned", (long long)al, (long long)val);
  int rc;
  if ((rc = chk(kv->k_token_stride, "K token", false))) return rc;
  if (kv->k_token_stride * es * ts >= ((int64_t)1 << 31) || kv->v_token_stride * ves * ts >= ((int64_t)1 << 31))
    return fail(OC_ERR_UNSUPPORTED, "token stride too large (a tile must span < 2 GiB)");
  if ((rc = chk(kv->v_token_stride, "V token", true))) return rc;
  memset(&a, 0, sizeof a);
  a.k = (const char*)kv->k;
  a.v = (const char*)kv->v;
  a.v_bf16 = v_bf16 ? 1 : 0;
  a.k_tok_stride = kv->k_token_stride * es;
  a.v_tok_stride = kv->v_token_stride * ves;
  a.paged = kv->paged ? 1 : 0;
  if (!a.paged) {
    if ((rc = chk(kv->k_row_stride, "K row", false))) return rc;
    if ((rc = chk(kv->v_row_stride, "V row", true))) return rc;
    a.k_row_stride = kv->k_row_stride * es;
    a.v_row_stride = kv->v_row_stride * ves;
  } else {
    const int bs = kv->block_size;
    if (bs < 4 || (bs & (bs - 1))) return fail(OC_ERR_INVALID, "block_size %d must be a power of 2 >= 4", bs);
    if (kv->num_kv_heads <= 0 || kv->num_rows % kv->num_kv_heads)
      return fail(OC_ERR_INVALID, "num_rows %d not a multiple of num_kv_heads %d", kv->num_rows, kv->num_kv_heads);
    if (!kv->block_tables) return fail(OC_ERR_INVALID, "block_tables is NULL");
    if ((rc = chk(kv->k_block_stride, "K block", false))) return rc;
    if ((rc = chk(kv->k_head_stride, "K head", false))) return rc;
    if ((rc = chk(kv->v_block_stride, "V block", true))) return rc;
    if ((rc = chk(kv->v_head_stride, "V head", true))) return rc;
    int l2 = 0;
    while ((1 << l2) < bs) ++l2;
    a.bs_log2 = l2;
    a.nkv = kv->num_kv_heads;
    a.bt = kv->block_tables;
    a.bt_stride = kv->bt_stride;
    a.num_blocks = kv->num_blocks;
    a.k_blk_stride = kv->k_block_stride * es;
    a.k_head_stride = kv->k_head_stride * es;
    a.v_blk_stride = kv->v_block_stride * ves;
    a.v_head_stride = kv->v_head_stride * ves;
  }
  a.rows_per_length = kv->rows_per_length > 0 ? kv->rows_per_length : 1;
  a.lengths = kv->lengths;
  a.num_rows = kv->num_rows;
  a.num_tiles = kv->num_tiles;
  if (kv->num_tokens < 0 || (int64_t)kv->num_tokens > (int64_t)kv->num_tiles * ts)
    return fail(OC_ERR_INVALID, "num_tokens %d outside 0..num_tiles * tile_size", kv->num_tokens);
  if ((int64_t)kv->num_tiles * ts > 0x7FFFFFFF) return fail(OC_ERR_UNSUPPORTED, "rows longer than 2^31 tokens");
  a.ts = ts;
  // the portable kernels' 16-byte staging: every K / V offset and row chunk
  // 16-byte aligned (also set for the tuned shapes, which a caller can send
  // to the portable kernels with the params' portable flag)
  {
    auto a16 = [](int64_t bytes) { return bytes % 16 == 0; };
    bool vec = aligned(kv->k, 16) && (!kv->v || aligned(kv->v, 16)) && a16(a.k_tok_stride) &&
               a16(a.v_tok_stride);
    if (a.paged) vec = vec && a16(a.k_blk_stride) && a16(a.k_head_stride) && a16(a.v_blk_stride) && a16(a.v_head_stride);
    else vec = vec && a16(a.k_row_stride) && a16(a.v_row_stride);
    a.gen_vec = vec ? 1 : 0;
  }
  a.row_tok = kv->lengths ? 0 : kv->num_tokens;
  a.k_scale_mode = kv->k_scale_mode;
  a.v_scale_mode = kv->v_scale_mode;
  a.k_scale = kv->k_scale;
  a.k_scales = kv->k_scales;
  a.ks_stride = kv->k_scales_row_stride;
  a.v_scales = kv->v_scales;
  a.vs_stride = kv->v_scales_row_stride;
  a.error_flag = kv->error_flag;
  if (a.k_scale_mode == OC_KSCALE_DEQUANT) {
    if (!allow_dq)
      return fail(OC_ERR_UNSUPPORTED, "k_scale_mode OC_KSCALE_DEQUANT is implemented by the decode and scoring only");
    if (kv->dtype != OC_FP8_E4M3FN) return fail(OC_ERR_INVALID, "OC_KSCALE_DEQUANT needs fp8 K");
  } else if (a.k_scale_mode != OC_KSCALE_NONE && a.k_scale_mode != OC_KSCALE_Q_FOLD &&
             a.k_scale_mode != OC_KSCALE_TILE) {
    return fail(OC_ERR_INVALID, "k_scale_mode %d", a.k_scale_mode);
  }
  if (a.k_scale_mode == OC_KSCALE_TILE && !a.k_scales) return fail(OC_ERR_INVALID, "k_scales is NULL");
  if (a.v_scale_mode == OC_VSCALE_TILE && !a.v_scales) return fail(OC_ERR_INVALID, "v_scales is NULL");
  if (a.v_scale_mode != OC_VSCALE_NONE && a.v_scale_mode != OC_VSCALE_TILE)
    return fail(OC_ERR_INVALID, "v_scale_mode %d", a.v_scale_mode);
  return OC_OK;
}

template <int DT>
hipError_t launch_decode(const DecodeArgs& a, int head_dim, int gt, int gchunks, hipStream_t st);
template <int DT>
hipError_t launch_score(const DecodeArgs& a, int head_dim, hipStream_t st);
template <int DT>
hipError_t launch_fwht(const DecodeArgs& a, int head_dim, hipStream_t st);

static hipError_t dispatch_decode(int dt, const DecodeArgs& a, int hd, int gt, int gc, hipStream_t st) {
  switch (dt) {
    case OC_F32: return launch_decode<OC_F32>(a, hd, gt, gc, st);
    case OC_F16: return launch_decode<OC_F16>(a, hd, gt, gc, st);
    case OC_BF16: return launch_decode<OC_BF16>(a, hd, gt, gc, st);
    default: return launch_decode<OC_FP8_E4M3FN>(a, hd, gt, gc, st);
  }
}

static hipError_t dispatch_score(int dt, const DecodeArgs& a, int hd, hipStream_t st) {
  switch (dt) {
    case OC_F32: return launch_score<OC_F32>(a, hd, st);
    case OC_F16: return launch_score<OC_F16>(a, hd, st);
    case OC_BF16: return launch_score<OC_BF16>(a, hd, st);
    default: return launch_score<OC_FP8_E4M3FN>(a, hd, st);
  }
}

static hipError_t dispatch_band(int dt, const DecodeArgs& a, int hd, hipStream_t st) {
  switch (dt) {
    case OC_F32: return launch_band<OC_F32>(a, hd, st);
    case OC_F16: return launch_band<OC_F16>(a, hd, st);
    case OC_BF16: return launch_band<OC_BF16>(a, hd, st);
    default: return launch_band<OC_FP8_E4M3FN>(a, hd, st);
  }
}

static hipError_t dispatch_fwht(int dt, const DecodeArgs& a, int hd, hipStream_t st) {
  switch (dt) {
    case OC_F32: return launch_fwht<OC_F32>(a, hd, st);
    case OC_F16: return launch_fwht<OC_F16>(a, hd, st);
    case OC_BF16: return launch_fwht<OC_BF16>(a, hd, st);
    default: return launch_fwht<OC_FP8_E4M3FN>(a, hd, st);
  }
}

// ---------------------------------------------------------------- merge

__device__ __forceinline__ float block_reduce(float x, bool is_max, float* red) {
  x = is_max ? wave_max(x) : wave_sum(x);
  const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  if ((threadIdx.x & 63) == 0) red[w] = x;
  __syncthreads();
  x = red[0];
  for (int i = 1; i < nw; ++i) x = is_max ? fmaxf(x, red[i]) : x + red[i];
  __syncthreads();
  return x;
}

// out = sum_s e^(m_s-M) acc_s / max(sum_s e^(m_s-M) l_s, 1e-9) per query-head
// row.  grid = (rows, ceil(D / 64)): workgroup (r, cb) forms the weights of
// row r and merges columns 64 cb .. + 63, wave w summing the partials
// s = w, w + 4, ... (eight loads in flight per lane), the four wave sums
// added in wave order.
__global__ __launch_bounds__(256) void merge_kernel(const float* __restrict__ m, const float* __restrict__ l,
                                                    const float* __restrict__ acc, int P, int D, char* out,
                                                    int out_dtype, int64_t out_row_stride) {
  extern __shared__ float sw[];
  __shared__ float red[4];
  __shared__ float part[4][64];
  const int64_t r = blockIdx.x;
  const float* mr = m + r * P;
  const float* lr = l + r * P;
  float mx = -__builtin_inff();
  for (int s = threadIdx.x; s < P; s += blockDim.x) mx = fmaxf(mx, mr[s]);
  mx = block_reduce(mx, true, red);
  float ls = 0.f;
  for (int s = threadIdx.x; s < P; s += blockDim.x) {
    const float w = __expf(mr[s] - mx);
    sw[s] = w;
    ls = __builtin_fmaf(w, lr[s], ls);
  }
  ls = block_reduce(ls, false, red);  // contains the barrier that publishes sw
  const float inv_l = fmaxf(ls, 1e-9f);
  const int es = out_dtype == OC_F32 ? 4 : 2;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = blockIdx.y * 64 + lane;
  float x = 0.f;
  if (c < D) {
    const float* ap = acc + r * P * D + c;
    int s = wave;
    for (; s + 28 < P; s += 32) {
      float v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = ap[(int64_t)(s + 4 * i) * D];
#pragma unroll
      for (int i = 0; i < 8; ++i) x = __builtin_fmaf(v[i], sw[s + 4 * i], x);
    }
    for (; s < P; s += 4) x = __builtin_fmaf(ap[(int64_t)s * D], sw[s], x);
  }
  part[wave][lane] = x;
  __syncthreads();
  if (wave == 0 && c < D)
    store_scalar(out + r * out_row_stride + (int64_t)c * es, out_dtype,
                 (((part[0][lane] + part[1][lane]) + part[2][lane]) + part[3][lane]) / inv_l);
}

static int launch_merge(const float* m, const float* l, const float* acc, int rows, int P, int D, void* out,
                        int out_dtype, int64_t out_row_stride_el, hipStream_t st) {
  if (rows == 0) return OC_OK;
  const int es = out_dtype == OC_F32 ? 4 : 2;
  hipLaunchKernelGGL(merge_kernel, dim3(rows, (D + 63) / 64), dim3(256), (size_t)P * sizeof(float), st, m, l, acc, P,
                     D, (char*)out, out_dtype, out_row_stride_el * es);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? OC_OK : hip_fail(e, "merge launch");
}

// dst[i] = round_out(float(fp8 src[i]) * scale), 16 elements per thread
__global__ __launch_bounds__(256) void dequant_fp8_kernel(const uint4* __restrict__ src, int64_t n16, float scale,
                                                          int out_dtype, char* __restrict__ dst) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int es = out_dtype == OC_F32 ? 4 : 2;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) {
    const uint4 w = src[i];
    const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
    char* o = dst + i * 16 * es;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const float x = elem<OC_FP8_E4M3FN>(ww, e) * scale;
      store_scalar(o + e * es, out_dtype, x);
    }
  }
}

// Streaming read: each thread keeps four 128-bit loads in flight per step.
__global__ __launch_bounds__(256) void read_probe_kernel(const uint4* __restrict__ src, int64_t n16, float* sink) {
  typedef uint32_t v4u __attribute__((ext_vector_type(4)));
  const v4u* p = reinterpret_cast<const v4u*>(src);
  uint32_t s = 0u;
  const int64_t stride = (int64_t)gridDim.x * 256 * 4;
  for (int64_t base = (int64_t)blockIdx.x * 256 * 4 + threadIdx.x; base < n16; base += stride) {
    v4u v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      // non-temporal, the cache policy of the decode's K/V loads
      const int64_t i = base + (int64_t)u * 256;
      v[u] = i < n16 ? __builtin_nontemporal_load(p + i) : v4u{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) s ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  // a data-dependent store the compiler cannot remove keeps the loads live
  if (s == 0x9E3779B9u) sink[blockIdx.x] = 1.0f;
}

}  // namespace oc

using namespace oc;

extern "C" int oc_hbm_read_probe(const void* src, size_t bytes, float* sink, int32_t blocks, void* stream) {
  if (!src || !sink) return fail(OC_ERR_INVALID, "NULL pointer");
  if (bytes % 16 || !aligned(src, 16)) return fail(OC_ERR_INVALID, "bytes and src must be 16-byte multiples");
  if (blocks < 1 || blocks > 65536) return fail(OC_ERR_INVALID, "blocks %d outside 1..65536", blocks);
  if (bytes == 0) return OC_OK;
  hipLaunchKernelGGL(read_probe_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream, (const uint4*)src,
                     (int64_t)(bytes / 16), sink);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? OC_OK : hip_fail(e, "read probe launch");
}

// Gather probe: the decode's tile access pattern without its arithmetic.
// Every step reads `pps` pieces of LPS / pps KiB each at the given byte
// offsets (one 1 KiB load instruction per 16 bytes a lane, non-temporal,
// the decode's cache policy), all of a step's loads in flight before any
// is used, as the decode requests one tile's K and V.  Workgroup b takes
// steps [b n / blocks, (b + 1) n / blocks), its 8 waves interleaved; the
// offsets of a wave's next step are fetched while its current step's data
// is in flight.
template <int LPS>
__global__ __launch_bounds__(512) void gather_probe_kernel(const char* __restrict__ base,
                                                           const int64_t* __restrict__ offs, int64_t n_steps, int pps,
                                                           float* sink) {
  typedef uint32_t v4u __attribute__((ext_vector_type(4)));
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t s1 = n_steps * (blockIdx.x + 1) / gridDim.x;
  int64_t s = n_steps * blockIdx.x / gridDim.x + wave;
  const int kib = LPS / pps;  // 1 KiB loads per piece
  uint32_t acc = 0u;
  int64_t o[8];
#pragma unroll
  for (int p = 0; p < 8; ++p) o[p] = (s < s1 && p < pps) ? offs[s * pps + p] : 0;
  while (s < s1) {
    v4u v[LPS];
#pragma unroll
    for (int i = 0; i < LPS; ++i) {
      const int p = i / kib;
      v[i] = __builtin_nontemporal_load(
          reinterpret_cast<const v4u*>(base + o[p < 8 ? p : 7] + (int64_t)(i - p * kib) * 1024 + lane * 16));
    }
    s += 8;
#pragma unroll
    for (int p = 0; p < 8; ++p) o[p] = (s < s1 && p < pps) ? offs[s * pps + p] : 0;
#pragma unroll
    for (int i = 0; i < LPS; ++i) acc ^= v[i][0] ^ v[i][1] ^ v[i][2] ^ v[i][3];
  }
  // a data-dependent store the compiler cannot remove keeps the loads live
  if (acc == 0x9E3779B9u) sink[blockIdx.x] = 1.0f;
}

extern "C" int oc_hbm_gather_probe(const void* base, const int64_t* piece_offsets, int64_t n_steps,
                                   int32_t pieces_per_step, int32_t loads_per_step, float* sink, int32_t blocks,
                                   void* stream) {
  if (!base || !piece_offsets || !sink) return fail(OC_ERR_INVALID, "NULL pointer");
  if (pieces_per_step < 1 || pieces_per_step > 8 || n_steps < 0 || blocks < 1)
    return fail(OC_ERR_INVALID, "bad sizes (1..8 pieces a step)");
  if ((loads_per_step != 16 && loads_per_step != 32) || loads_per_step % pieces_per_step)
    return fail(OC_ERR_INVALID, "loads_per_step must be 16 or 32 and a multiple of pieces_per_step");
  if (n_steps == 0) return OC_OK;
  const hipStream_t st = (hipStream_t)stream;
  if (loads_per_step == 16)
    hipLaunchKernelGGL(gather_probe_kernel<16>, dim3(blocks), dim3(512), 0, st, (const char*)base, piece_offsets,
                       n_steps, pieces_per_step, sink);
  else
    hipLaunchKernelGGL(gather_probe_kernel<32>, dim3(blocks), dim3(512), 0, st, (const char*)base, piece_offsets,
                       n_steps, pieces_per_step, sink);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? OC_OK : hip_fail(e, "gather probe launch");
}

extern "C" int oc_dequant_fp8(const void* src, int64_t n, float scale, int32_t out_dtype, void* dst, void* stream) {
  if (!src || !dst) return fail(OC_ERR_INVALID, "NULL pointer");
  if (out_dtype != OC_F32 && out_dtype != OC_F16 && out_dtype != OC_BF16)
    return fail(OC_ERR_INVALID, "out dtype %d", out_dtype);
  if (n < 0 || n % 16) return fail(OC_ERR_INVALID, "element count %lld must be a multiple of 16", (long long)n);
  if (!aligned(src, 16) || !aligned(dst, 16)) return fail(OC_ERR_INVALID, "src/dst must be 16-byte aligned");
  if (n == 0) return OC_OK;
  const int64_t n16 = n / 16;
  const int blocks = (int)std::min<int64_t>((n16 + 255) / 256, 4096);
  hipLaunchKernelGGL(dequant_fp8_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream, (const uint4*)src, n16,
                     scale, out_dtype, (char*)dst);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? OC_OK : hip_fail(e, "dequant launch");
}

// CU count of the current device, cached per device index.
static int device_cus() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cache[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev] = n;
  }
  return cache[dev];
}

// query heads per decode workgroup for G heads per kv row (chunks of up to 8)
static int heads_per_group(const oc_decode_params* p) {
  const int G = p->G;
  return G >= 8 ? 8 : (G >= 4 ? (G == 4 ? 4 : 8) : (G == 3 ? 4 : G));
}

// Splits per workgroup: as many as keep the workgroup count at or below the
// CU count, so that the decode runs as one round of workgroups (one
// 512-thread workgroup is resident per CU at the decode kernel's register
// budget).  A second round would pay the prologue (q, scores, retained-tile
// bitmask) and the merge tail twice and leave its own imbalance (config 4,
// 32 rows of 2048 tiles: 512 workgroups took 121 us cached and 162 us single
// pass, 256 take 115 and 147).
static bool portable_path(const oc_decode_params* p);

// Whether a score-gated cached decode of p meets every condition of the
// per-wave-prologue kernel (decode_fast) other than its split grouping: q of
// K's 16-bit type (bf16 for fp8 K) in 16-byte rows, pages of >= 16 tokens,
// all query heads of a row in one workgroup, rows of at most 64 *
// kFastChunks tiles, output merged inside (no partials or per-split counts
// asked for), no q-folded K scale.
static bool fast_cached_shape(const oc_decode_params* p) {
  const oc_kv_desc& kv = p->kv;
  const int dt = kv.dtype;
  const bool mq = (dt == OC_BF16 && p->q_dtype == OC_BF16) || (dt == OC_F16 && p->q_dtype == OC_F16) ||
                  (dt == OC_FP8_E4M3FN && p->q_dtype == OC_BF16);
  const int qes = p->q_dtype == OC_F32 ? 4 : 2;
  const bool partials_given = p->partial_m && p->partial_l && p->partial_acc;
  return p->mode == OC_MODE_CACHED && p->gate != OC_GATE_NONE && mq && (!kv.paged || kv.block_size >= 16) &&
         p->G <= heads_per_group(p) && aligned(p->q, 16) && (p->q_row_stride * qes) % 16 == 0 &&
         kv.k_scale_mode != OC_KSCALE_Q_FOLD && p->out && !partials_given && !p->split_counts &&
         kv.num_tiles <= 64 * kFastChunks;
}

// splits per workgroup of the tuned kernels
static int choose_spw_tuned(const oc_decode_params* p) {
  if (p->splits_per_group > 0) return std::min(p->splits_per_group, p->num_splits);
  const int P = p->num_splits;
  const int64_t cus = device_cus();
  const int64_t groups = (int64_t)p->kv.num_rows * ((p->G + heads_per_group(p) - 1) / heads_per_group(p));
  int64_t spw = (P * groups + cus - 1) / cus;
  // A short cached decode whose splits alone fill the CUs (one split per
  // workgroup) still takes two per workgroup, which puts it on the
  // per-wave-prologue kernel: config 1 at 1K / 2K tokens (32 rows, 4 / 8
  // splits) took 14.3 / 14.9 us on one split per workgroup and 11.3 / 11.8
  // on two.
  if (spw <= 1 && P >= 2 && fast_cached_shape(p)) spw = 2;
  return (int)std::max<int64_t>(1, std::min<int64_t>(spw, P));
}

static int choose_spw(const oc_decode_params* p) {
  if (p->splits_per_group > 0) return std::min(p->splits_per_group, p->num_splits);
  // the portable kernels: one split per workgroup (several workgroups per
  // CU hide each other's staging round trips)
  if (portable_path(p)) return 1;
  return choose_spw_tuned(p);
}

static int num_groups(const oc_decode_params* p, int spw) { return (p->num_splits + spw - 1) / spw; }

static size_t partial_floats(const oc_decode_params* p, int pg) {
  const size_t rq = (size_t)p->kv.num_rows * (size_t)p->G * (size_t)pg;
  return rq * (2 + (size_t)p->kv.head_dim);
}

extern "C" int32_t oc_decode_num_groups(const oc_decode_params* p) {
  if (!p || p->num_splits <= 0) return 0;
  return num_groups(p, choose_spw(p));
}


// Workspace layout: [0, kCounterBytes) merge counters (zero before the first
// call, left zero by every call), then the partial states unless the caller
// gives its own.
static constexpr size_t kCounterBytes = 64 << 10;

// The split merge runs inside the decode kernel when the counters and the
// merge weights (GT * Pg floats in the kernel's 4 * GT * D wave-merge LDS)
// fit; otherwise merge_kernel runs after it.
static int gchunks_of(const oc_decode_params* p) {
  return (p->G + heads_per_group(p) - 1) / heads_per_group(p);
}

static bool fused_merge(const oc_decode_params* p, int pg) {
  const int gchunks = gchunks_of(p);
  return p->out && (size_t)p->kv.num_rows * gchunks * sizeof(int32_t) <= kCounterBytes && pg <= 4 * p->kv.head_dim;
}

// Rows of different lengths (a lengths array) are laid out flat: row r gets
// workgroups in proportion to its tiles, about per_cu per CU in all
// (flat_map in the kernel; flat_map_lpt, long shares first, in the
// per-wave-prologue kernel and the single-pass and dense decodes, with pct
// percent of each row's tiles in long shares and short shares 1 / div as
// long), with the merge fused.  Not with partials requested (their layout is
// the per-split one), per-split counts, or a cached decode too long for the
// in-LDS retained-tile bitmask.  A single-pass gated decode scores every tile
// inside its loop, and runs best with fewer, longer shares (config 3: 437-441
// us at 2 per CU and 95%, against 451-468 at 4 and 90%, where the cached and
// dense decodes are fastest).
struct FlatCfg {
  int per_cu, pct, div;
};
static constexpr FlatCfg kFlat = {4, 90, 4}, kFlatSinglePass = {2, 95, 4};

static FlatCfg flat_cfg(const oc_decode_params* p) {
  return p->mode == OC_MODE_SINGLE_PASS && p->gate != OC_GATE_NONE ? kFlatSinglePass : kFlat;
}

// The portable kernels (oc_generic.hip): head_dim other than 64 / 128 (and
// 32 / 256 outside the matrix-core routes below), tiles other than 64
// tokens, or asked for (p->portable).  They write one partial per split
// group and merge_kernel combines them.
static bool flat_layout_tuned(const oc_decode_params* p);

// head_dim 256 with 64-token tiles on the matrix-core kernels (4-wave
// workgroups at one wave per SIMD, a 32 KiB V slot per wave): bf16 or f16
// K/V with q of K's type, or fp8 K (fp8 or bf16 V) with bf16 q, contiguous
// rows or pages of >= 16 tokens, 16-byte aligned q, K, V and strides.  The
// per-wave-prologue kernel takes what it takes at head_dim 64 / 128 (a.fast,
// G <= 8), the general matrix-core kernel the rest (single-pass gate,
// partials, one split per workgroup, G > 8 in chunks of 8 heads).  bf16 V
// beside fp8 K and the in-kernel K dequantisation, which only the
// per-wave-prologue kernel does, need G <= 8.  Every other head_dim-256
// decode runs on the portable kernels.
static bool wide_route(const oc_decode_params* p) {
  const oc_kv_desc& kv = p->kv;
  const int ts = kv.tile_size > 0 ? kv.tile_size : 64;
  if (p->portable != 0 || kv.head_dim != 256 || ts != 64) return false;
  const bool f8 = kv.dtype == OC_FP8_E4M3FN;
  const bool mq = (kv.dtype == OC_BF16 && p->q_dtype == OC_BF16) || (kv.dtype == OC_F16 && p->q_dtype == OC_F16) ||
                  (f8 && p->q_dtype == OC_BF16);
  const bool v_ok = kv.v_dtype == 0 || kv.v_dtype == kv.dtype || (f8 && kv.v_dtype == OC_BF16);
  if (!mq || !v_ok || p->G < 1 || p->G > 64) return false;
  if (kv.paged && kv.block_size < 16) return false;
  if (kv.k_scale_mode == OC_KSCALE_DEQUANT && !f8) return false;
  const bool v_bf16 = f8 && kv.v_dtype == OC_BF16;
  if (p->G > 8 && (v_bf16 || kv.k_scale_mode == OC_KSCALE_DEQUANT)) return false;
  const int es = f8 ? 1 : 2, ves = f8 && kv.v_dtype == OC_BF16 ? 2 : es;
  auto a16 = [](int64_t el) { return (el * 2) % 16 == 0; };
  auto k16 = [es](int64_t el) { return (el * es) % 16 == 0; };
  auto v16 = [ves](int64_t el) { return (el * ves) % 16 == 0; };
  if (!aligned(p->q, 16) || !a16(p->q_row_stride) || !aligned(kv.k, 16) || !aligned(kv.v, 16) ||
      !k16(kv.k_token_stride) || !v16(kv.v_token_stride))
    return false;
  return kv.paged ? k16(kv.k_block_stride) && k16(kv.k_head_stride) && v16(kv.v_block_stride) &&
                        v16(kv.v_head_stride)
                  : k16(kv.k_row_stride) && v16(kv.v_row_stride);
}

// head_dim 32 with 64-token tiles on the matrix-core kernels of head_dim 64
// / 128 (8-wave workgroups, the per-wave-prologue kernel where a.fast, the
// general one otherwise): bf16 or f16 K/V with q of K's type (no fp8 or
// float32 K/V: a lane's 64-byte row piece holds 2 fp8 bytes), contiguous
// rows or pages of >= 16 tokens, 16-byte aligned q, K, V and strides.
// Every other head_dim-32 decode runs on the portable kernels.
static bool narrow_route(const oc_decode_params* p) {
  const oc_kv_desc& kv = p->kv;
  const int ts = kv.tile_size > 0 ? kv.tile_size : 64;
  if (p->portable != 0 || kv.head_dim != 32 || ts != 64) return false;
  const bool mq = (kv.dtype == OC_BF16 && p->q_dtype == OC_BF16) || (kv.dtype == OC_F16 && p->q_dtype == OC_F16);
  if (!mq || (kv.v_dtype != 0 && kv.v_dtype != kv.dtype)) return false;
  if (kv.paged && kv.block_size < 16) return false;
  auto a16 = [](int64_t el) { return (el * 2) % 16 == 0; };
  if (!aligned(p->q, 16) || !a16(p->q_row_stride) || !aligned(kv.k, 16) || !aligned(kv.v, 16) ||
      !a16(kv.k_token_stride) || !a16(kv.v_token_stride))
    return false;
  return kv.paged ? a16(kv.k_block_stride) && a16(kv.k_head_stride) && a16(kv.v_block_stride) &&
                        a16(kv.v_head_stride)
                  : a16(kv.k_row_stride) && a16(kv.v_row_stride);
}

static bool portable_path(const oc_decode_params* p) {
  return (p->portable == 1 || generic_shape(p->kv.head_dim, p->kv.tile_size > 0 ? p->kv.tile_size : 64)) &&
         !wide_route(p) && !narrow_route(p);
}

static bool flat_layout(const oc_decode_params* p) {
  if (portable_path(p)) return false;
  return flat_layout_tuned(p);
}

static bool flat_layout_tuned(const oc_decode_params* p) {
  const bool partials_given = p->partial_m && p->partial_l && p->partial_acc;
  const bool cached = p->mode == OC_MODE_CACHED && p->gate != OC_GATE_NONE;
  return p->kv.lengths && p->out && !partials_given && !p->split_counts && p->splits_per_group != 1 &&
         (!cached || p->kv.num_tiles <= kMaxBalTiles) && (int64_t)p->kv.num_rows * p->kv.num_tiles < (1 << 30) &&
         fused_merge(p, 1);
}

static int flat_target(const oc_decode_params* p) { return flat_cfg(p).per_cu * device_cus(); }

// partial slots of the flat layout: flat_map_lpt's bound, which also covers
// flat_map's flat_target + rows
static size_t flat_slots(const oc_decode_params* p) {
  const FlatCfg c = flat_cfg(p);
  return (size_t)flat_lpt_slots(flat_target(p), p->kv.num_rows, c.pct, c.div);
}

extern "C" size_t oc_decode_workspace_size(const oc_decode_params* p) {
  if (!p || p->num_splits <= 0 || p->G <= 0) return 0;
  const bool partials_given = p->partial_m && p->partial_l && p->partial_acc;
  if (partials_given && !p->out) return 0;
  size_t n = 256 + (p->out ? kCounterBytes : 0);
  if (flat_layout(p)) {
    // one partial per (slot, query head)
    return n + flat_slots(p) * (size_t)p->G * (2 + (size_t)p->kv.head_dim) * sizeof(float);
  }
  const int pg = num_groups(p, choose_spw(p));
  if (!partials_given) n += partial_floats(p, pg) * sizeof(float);
  return n;
}

// The model hook's gate, fused into the decode's prologue (oc_hook_decode):
// tile norms of kv head (row % rows), complete tiles, threshold, statistics.
struct HookGate {
  const float* norms;
  int64_t stride;
  int rows, full;
  double tau;
  float* stats;
};
// decode_impl's answer when a hook gate cannot be fused (the caller then
// gates with its own kernel); no error message is recorded for it
static constexpr int kHookNotFused = -1;

// oc_decode with the workspace (`ws`, `ws_bytes`) given separately from p,
// so that oc_decode_static can bring its own; with `hk` the decode gates
// with the hook's norms instead of p's gate (p's tile mask unused).
static int decode_impl(const oc_decode_params* p, void* ws, size_t ws_bytes, void* stream,
                       const HookGate* hk = nullptr) {
  if (!p) return fail(OC_ERR_INVALID, "params is NULL");
  DecodeArgs a{};
  int rc = fill_kv(&p->kv, a, true);
  if (rc) return rc;
  if (!p->kv.v) return fail(OC_ERR_INVALID, "V pointer is NULL");
  // in-kernel dequantisation runs where fp8 K is widened for the matrix cores
  if (a.k_scale_mode == OC_KSCALE_DEQUANT && !portable_path(p) && (p->q_dtype != OC_BF16 || (a.paged && a.bs_log2 < 4)))
    return fail(OC_ERR_UNSUPPORTED, "OC_KSCALE_DEQUANT needs bf16 q and contiguous rows or pages of >= 16 tokens");
  const int D = p->kv.head_dim;
  if (p->G < 1 || p->G > 64) return fail(OC_ERR_UNSUPPORTED, "G=%d outside 1..64", p->G);
  if (p->num_splits < 1 || p->num_splits > 8192) return fail(OC_ERR_INVALID, "num_splits %d outside 1..8192", p->num_splits);
  if (p->q_dtype != OC_F32 && p->q_dtype != OC_F16 && p->q_dtype != OC_BF16)
    return fail(OC_ERR_INVALID, "q dtype %d", p->q_dtype);
  if (p->out_dtype != OC_F32 && p->out_dtype != OC_F16 && p->out_dtype != OC_BF16)
    return fail(OC_ERR_INVALID, "out dtype %d", p->out_dtype);
  const bool partials_given = p->partial_m && p->partial_l && p->partial_acc;
  if (!p->q) return fail(OC_ERR_INVALID, "q pointer is NULL");
  if (!p->out && !partials_given) return fail(OC_ERR_INVALID, "out is NULL and no partial buffers are given");
  if (p->gate < OC_GATE_NONE || p->gate > OC_GATE_MASK) return fail(OC_ERR_INVALID, "gate %d", p->gate);
  if (p->gate == OC_GATE_MASK && (p->mode != OC_MODE_CACHED || !p->tile_mask))
    return fail(OC_ERR_INVALID, "the mask gate needs cached mode and a tile_mask");
  if (p->mode != OC_MODE_SINGLE_PASS && p->mode != OC_MODE_CACHED) return fail(OC_ERR_INVALID, "mode %d", p->mode);
  if (p->mode == OC_MODE_CACHED && p->gate != OC_GATE_NONE && p->gate != OC_GATE_MASK) {
    if (!p->score_e_high || (p->gate == OC_GATE_ZETA && !p->score_e_low))
      return fail(OC_ERR_INVALID, "cached mode needs score_e_high (and score_e_low for the zeta gate)");
  }
  const int qes = p->q_dtype == OC_F32 ? 4 : 2;
  a.q = (const char*)p->q;
  a.q_row_stride = p->q_row_stride * qes;
  a.q_dtype = p->q_dtype;
  a.G = p->G;
  a.gate = p->gate;
  a.mode = p->mode;
  a.thr = p->threshold;
  a.sc_el = p->score_e_low;
  a.sc_eh = p->score_e_high;
  a.tmask = p->tile_mask;
  a.tmask_stride = p->tile_mask_row_stride;
  a.sc_stride = p->score_row_stride;
  a.P = p->num_splits;
  if (p->splits_per_group < 0) return fail(OC_ERR_INVALID, "splits_per_group %d", p->splits_per_group);
  a.spw = choose_spw(p);
  a.Pg = num_groups(p, a.spw);
  a.flat = flat_layout(p) ? 1 : 0;
  a.flat_target = flat_target(p);
  a.flat_pct = flat_cfg(p).pct;
  a.flat_div = flat_cfg(p).div;
  a.flat_slots = a.flat ? (int)flat_slots(p) : 0;
  a.keep_out = p->keep_out;
  a.keep_stride = p->keep_row_stride;
  a.split_counts = p->split_counts;
  a.scale = (float)(1.0 / std::sqrt((double)D));
  const size_t need = oc_decode_workspace_size(p);
  char* w = nullptr;
  if (need) {
    if (!ws || ws_bytes < need)
      return fail(OC_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given", need, ws_bytes);
    w = (char*)(((uintptr_t)ws + 255) & ~(uintptr_t)255);
  }
  if (p->out) {
    a.counters = (int32_t*)w;
    w += kCounterBytes;
    // one 128-byte line per (row, chunk) counter where they fit: the tickets
    // of different rows then do not queue on one line
    const int64_t nctr = (int64_t)p->kv.num_rows * gchunks_of(p);
    a.ctr_stride = 32;
    while (a.ctr_stride > 1 && nctr * a.ctr_stride * (int64_t)sizeof(int32_t) > (int64_t)kCounterBytes) a.ctr_stride >>= 1;
  }
  if (partials_given) {
    if (!aligned(p->partial_acc, 16)) return fail(OC_ERR_INVALID, "partial_acc must be 16-byte aligned");
    a.pm = p->partial_m;
    a.pl = p->partial_l;
    a.pacc = p->partial_acc;
  } else {
    const size_t rq = a.flat ? flat_slots(p) * p->G : (size_t)p->kv.num_rows * p->G * a.Pg;
    a.pacc = (float*)w;
    a.pm = a.pacc + rq * D;
    a.pl = a.pm + rq;
  }
  const int oes = p->out_dtype == OC_F32 ? 4 : 2;
  const bool portable = portable_path(p);
  if (p->portable != 0 && p->portable != 1) return fail(OC_ERR_INVALID, "portable %d (0 or 1)", p->portable);
  a.fuse = !portable && (a.flat || fused_merge(p, a.Pg)) ? 1 : 0;
  // split the retained tiles of a row evenly over its workgroups (cached
  // mode); with one split per workgroup each partial stays the state of
  // exactly one logical split {s + kP}
  a.bal = (!portable && p->mode == OC_MODE_CACHED && p->gate != OC_GATE_NONE && (a.spw > 1 || a.flat) &&
           p->kv.num_tiles <= kMaxBalTiles) ? 1 : 0;
  a.out = (char*)p->out;
  a.out_dtype = p->out_dtype;
  a.out_stride = p->out_row_stride * oes;
  if (a.num_rows == 0) return OC_OK;
  const int gt = heads_per_group(p);
  const int gchunks = (p->G + gt - 1) / gt;
  if (portable) {
    // every gate, mode, scale mode and layout, in float32 on the VALU; the
    // model hook's fused gate is not (its caller then gates with its own
    // kernel and decodes with the mask gate)
    if (hk) return kHookNotFused;
    hipStream_t st = (hipStream_t)stream;
    hipError_t e = gen_launch_decode(p->kv.dtype, a, D, gt, gchunks, st);
    if (e != hipSuccess) return hip_fail(e, "portable decode launch");
    if (!p->out) return OC_OK;
    return launch_merge(a.pm, a.pl, a.pacc, p->kv.num_rows * p->G, a.Pg, D, p->out, p->out_dtype,
                        p->out_row_stride, st);
  }
  // the barrier-free prologue (decode_fast): the transposed matrix-core step
  // on contiguous rows or pages of >= 16 tokens (q of K's 16-bit type, bf16
  // for fp8 K), every query head of a row in one workgroup, q rows readable
  // as 16-byte pieces, partials internal; a score-gated cached decode whose
  // rows have at most 64 * kFastChunks tiles (their ranks split evenly over
  // the row's workgroups), or a dense decode over more than one split per
  // workgroup (or the flat layout of rows of different lengths)
  {
    const int dt = p->kv.dtype;
    const bool mq = (dt == OC_BF16 && p->q_dtype == OC_BF16) || (dt == OC_F16 && p->q_dtype == OC_F16) ||
                    (dt == OC_FP8_E4M3FN && p->q_dtype == OC_BF16);
    const bool cached_gate = p->mode == OC_MODE_CACHED && p->gate != OC_GATE_NONE;
    const bool q16 = aligned(p->q, 16) && (a.q_row_stride % 16) == 0;
    a.fast = (mq && (!a.paged || a.bs_log2 >= 4) && gchunks == 1 && q16 &&
              p->kv.k_scale_mode != OC_KSCALE_Q_FOLD && !partials_given && !p->split_counts &&
              ((cached_gate && a.bal && p->kv.num_tiles <= 64 * kFastChunks) ||
               (p->gate == OC_GATE_NONE && (a.spw > 1 || a.flat)))) ? 1 : 0;
    // the flat layout runs several rounds of small workgroups: two 4-wave
    // workgroups per CU, so that one's prologue overlaps the other's loop
    a.fast_waves = a.flat ? 4 : 8;
    // in-kernel K dequantisation and bf16 V beside fp8 K: in the
    // per-wave-prologue kernel only
    if (a.k_scale_mode == OC_KSCALE_DEQUANT && !a.fast)
      return fail(OC_ERR_UNSUPPORTED, "OC_KSCALE_DEQUANT: the decode of this shape or mode does not dequantise "
                                      "K itself (dequantise the pool, or decode cached / dense)");
    if (a.v_bf16 && !a.fast)
      return fail(OC_ERR_UNSUPPORTED, "bf16 V beside fp8 K: the decode of this shape or mode reads K and V in one "
                                      "type (convert one of them, or decode cached / dense)");
    if (hk) {
      // the row statistics come from a pass over the whole row (not flat)
      if (!a.fast || a.flat || dt == OC_FP8_E4M3FN || hk->full < 1 || (D != 64 && D != 128)) return kHookNotFused;
      a.gate = kGateHook;
      a.hk_norms = hk->norms;
      a.hk_stride = hk->stride;
      a.hk_rows = hk->rows;
      a.hk_full = hk->full;
      a.hk_tau = hk->tau;
      a.hk_stats = hk->stats;
    }
  }
  hipStream_t st = (hipStream_t)stream;
  hipError_t e = dispatch_decode(p->kv.dtype, a, D, gt, gchunks, st);
  if (e != hipSuccess) return hip_fail(e, "decode launch");
  if (!p->out || a.fuse) return OC_OK;
  return launch_merge(a.pm, a.pl, a.pacc, p->kv.num_rows * p->G, a.Pg, D, p->out, p->out_dtype,
                      p->out_row_stride, st);
}

extern "C" int oc_decode(const oc_decode_params* p, void* stream) {
  if (!p) return fail(OC_ERR_INVALID, "params is NULL");
  return decode_impl(p, p->workspace, p->workspace_bytes, stream);
}

// ------------------------------------------------ oc_hook_decode
//
// Workspace: [the decode's own workspace (merge counters first, so they stay
// at the start whatever the shapes)] [mask: rows x T bytes], each part
// 256-byte aligned.  A partial last tile is the descriptor's num_tokens (one
// length for every row), so the decode keeps its contiguous-row layout.

int oc_internal_hook_gate(const void* q, int32_t dtype, int64_t q_row_stride, int32_t batch, int32_t num_kv_heads,
                          int32_t G, int32_t head_dim, int32_t low_band, const float* k_norms,
                          int64_t k_norms_stride, int32_t num_tiles, int32_t mask_cols, double tau_norm,
                          uint8_t* mask, int64_t mask_stride, float* gate_stats, void* stream);

static size_t round256(size_t n) { return (n + 255) & ~(size_t)255; }

// The oc_decode parameters of a hook decode step (the mask pointer may be
// null when only sizes are wanted).
static int hook_to_decode(const oc_hook_decode_params* h, uint8_t* mask, oc_decode_params* d) {
  if (!h) return fail(OC_ERR_INVALID, "params is NULL");
  if (h->dtype != OC_F32 && h->dtype != OC_F16 && h->dtype != OC_BF16) return fail(OC_ERR_INVALID, "dtype %d", h->dtype);
  if (h->batch < 0 || h->num_kv_heads < 0 || h->G < 1 || h->G > 64 || h->kv_len < 64)
    return fail(OC_ERR_INVALID, "bad sizes (G in 1..64, kv_len >= 64)");
  if (h->low_band < 1 || h->head_dim % h->low_band) return fail(OC_ERR_INVALID, "low_band %d", h->low_band);
  const int64_t rows = (int64_t)h->batch * h->num_kv_heads;
  if (rows > 0x7FFFFFFF) return fail(OC_ERR_UNSUPPORTED, "too many rows");
  const int T = (h->kv_len + 63) / 64;
  std::memset(d, 0, sizeof(*d));
  d->kv.k = h->k;
  d->kv.v = h->v;
  d->kv.dtype = h->dtype;
  d->kv.head_dim = h->head_dim;
  d->kv.num_rows = (int32_t)rows;
  d->kv.num_tiles = T;
  d->kv.k_row_stride = h->k_row_stride;
  d->kv.k_token_stride = h->k_token_stride;
  d->kv.v_row_stride = h->v_row_stride;
  d->kv.v_token_stride = h->v_token_stride;
  d->kv.num_tokens = h->kv_len;
  d->q = h->q;
  d->q_dtype = h->dtype;
  d->G = h->G;
  d->q_row_stride = h->q_row_stride;
  d->gate = OC_GATE_MASK;
  d->mode = OC_MODE_CACHED;
  if (h->num_splits > 0) {
    d->num_splits = std::min(h->num_splits, T);
  } else {
    // about one workgroup per CU, two logical splits each (the retained
    // tiles of a row are split evenly over its workgroups)
    const int64_t wpr = std::max<int64_t>(1, std::min<int64_t>(device_cus() / std::max<int64_t>(rows, 1), T / 2));
    d->num_splits = (int)(2 * wpr);
    d->splits_per_group = 2;
  }
  d->out_dtype = h->dtype;
  d->out = h->out;
  d->out_row_stride = h->out_row_stride;
  d->tile_mask = mask;
  d->tile_mask_row_stride = T;
  return OC_OK;
}

extern "C" size_t oc_hook_decode_workspace_size(const oc_hook_decode_params* p) {
  oc_decode_params d;
  if (hook_to_decode(p, nullptr, &d)) return 0;
  d.out = (void*)1;  // sized as the call with an output
  return round256(oc_decode_workspace_size(&d)) + round256((size_t)d.kv.num_rows * d.kv.num_tiles) + 256;
}

extern "C" int oc_hook_decode(const oc_hook_decode_params* p, void* stream) {
  oc_decode_params d;
  int rc = hook_to_decode(p, nullptr, &d);
  if (rc) return rc;
  if (!p->q || !p->k || !p->v || !p->out || !p->k_norms) return fail(OC_ERR_INVALID, "NULL pointer");
  if (d.kv.num_rows == 0) return OC_OK;
  const size_t need = oc_hook_decode_workspace_size(p);
  if (!p->workspace || p->workspace_bytes < need)
    return fail(OC_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given", need, p->workspace_bytes);
  char* w = (char*)(((uintptr_t)p->workspace + 255) & ~(uintptr_t)255);
  d.out = p->out;
  const size_t dec = round256(oc_decode_workspace_size(&d));
  uint8_t* mask = (uint8_t*)(w + dec);
  d.workspace = w;
  d.workspace_bytes = dec;
  d.tile_mask = mask;
  if (p->low_band == 8 && (p->dtype == OC_BF16 || p->dtype == OC_F16)) {
    // one launch: the gate runs in the decode's prologue
    const HookGate hg{p->k_norms, p->k_norms_stride, p->num_kv_heads, p->kv_len / 64, p->tau_norm, p->gate_stats};
    rc = decode_impl(&d, d.workspace, d.workspace_bytes, stream, &hg);
    if (rc != kHookNotFused) return rc;
  }
  rc = oc_internal_hook_gate(p->q, p->dtype, p->q_row_stride, p->batch, p->num_kv_heads, p->G, p->head_dim,
                             p->low_band, p->k_norms, p->k_norms_stride, p->kv_len / 64, d.kv.num_tiles, p->tau_norm,
                             mask, d.kv.num_tiles, p->gate_stats, stream);
  if (rc) return rc;
  return decode_impl(&d, d.workspace, d.workspace_bytes, stream);
}

extern "C" size_t oc_hook_decode_params_bytes(void) { return sizeof(oc_hook_decode_params); }

// ------------------------------------------------ oc_decode_static scratch
//
// The split partials and merge counters of oc_decode_static live in this
// array: one copy per GPU, held until the process ends.  Its name is only a
// host-side stand-in in host code; the device address comes from
// hipGetSymbolAddress, once per device, and is what every kernel gets.
static constexpr size_t kScratchBytes = (size_t)16 << 20;
static __device__ __align__(256) char scratch[kScratchBytes];

// Zeroes n 32-bit words (the merge counters at set-up): a fill kernel, not
// hipMemsetAsync, so that a caller may capture the call in a graph.
__global__ __launch_bounds__(256) void zero_words_kernel(uint32_t* p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) p[i] = 0u;
}

static constexpr int kMaxDevices = 64;
static void* g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_mu;

// The current device's scratch address; at the first call on a device its
// merge counters are cleared on `st` (the array starts zeroed as well; the
// clear makes that independent of the loader), after which every call
// leaves them zero.
static int scratch_of_device(hipStream_t st, char** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail(OC_ERR_UNSUPPORTED, "device index %d >= %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) return hip_fail(e != hipSuccess ? e : hipErrorInvalidSymbol, "hipGetSymbolAddress");
    const int64_t words = (int64_t)(kCounterBytes + 256) / 4;
    hipLaunchKernelGGL(zero_words_kernel, dim3(64), dim3(256), 0, st, (uint32_t*)ptr, words);
    e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, "scratch clear launch");
    g_scratch_ptr[dev] = ptr;
  }
  *out = (char*)g_scratch_ptr[dev];
  return OC_OK;
}

extern "C" size_t oc_decode_static_scratch_bytes(void) { return kScratchBytes; }

extern "C" int oc_decode_static(const oc_decode_params* p, void* stream) {
  if (!p) return fail(OC_ERR_INVALID, "params is NULL");
  const size_t need = oc_decode_workspace_size(p);
  // the workspace is aligned up to 256 bytes inside; the array already is
  if (need > kScratchBytes)
    return fail(OC_ERR_WORKSPACE, "oc_decode_static: %zu bytes of split partials and counters needed, the static "
                "scratch holds %zu (use oc_decode with a workspace)", need, kScratchBytes);
  char* ptr = nullptr;
  if (need) {
    const int rc = scratch_of_device((hipStream_t)stream, &ptr);
    if (rc) return rc;
  }
  return decode_impl(p, ptr, need ? kScratchBytes : 0, stream);
}

extern "C" int oc_score_tiles(const oc_kv_desc* kv, double zeta_max, float* e_low, float* e_high, float* zeta,
                              uint8_t* keep, int64_t out_row_stride, void* stream) {
  DecodeArgs a{};
  int rc = fill_kv(kv, a, true);
  if (rc) return rc;
  a.thr = zeta_max;
  a.o_el = e_low;
  a.o_eh = e_high;
  a.o_z = zeta;
  a.o_keep = keep;
  a.o_stride = out_row_stride;
  a.q_dtype = OC_F32;
  a.t0 = 0;
  a.tcnt = kv->num_tiles;
  if ((int64_t)kv->num_rows * kv->num_tiles == 0) return OC_OK;
  const hipError_t e = generic_shape(kv->head_dim, a.ts) ? gen_launch_score(kv->dtype, a, kv->head_dim, (hipStream_t)stream)
                                                         : dispatch_score(kv->dtype, a, kv->head_dim, (hipStream_t)stream);
  return e == hipSuccess ? OC_OK : hip_fail(e, "score launch");
}

extern "C" int oc_score_tile_range(const oc_kv_desc* kv, int32_t first_tile, int32_t count, double zeta_max,
                                   float* e_low, float* e_high, float* zeta, uint8_t* keep, int64_t out_row_stride,
                                   void* stream) {
  DecodeArgs a{};
  int rc = fill_kv(kv, a, true);
  if (rc) return rc;
  if (first_tile < 0 || count < 0 || (int64_t)first_tile + count > kv->num_tiles)
    return fail(OC_ERR_INVALID, "tile range [%d, %d) outside 0..%d", first_tile, first_tile + count, kv->num_tiles);
  a.thr = zeta_max;
  a.o_el = e_low;
  a.o_eh = e_high;
  a.o_z = zeta;
  a.o_keep = keep;
  a.o_stride = out_row_stride;
  a.q_dtype = OC_F32;
  a.t0 = first_tile;
  a.tcnt = count;
  if ((int64_t)kv->num_rows * count == 0) return OC_OK;
  const hipError_t e = generic_shape(kv->head_dim, a.ts) ? gen_launch_score(kv->dtype, a, kv->head_dim, (hipStream_t)stream)
                                                         : dispatch_score(kv->dtype, a, kv->head_dim, (hipStream_t)stream);
  return e == hipSuccess ? OC_OK : hip_fail(e, "score launch");
}

extern "C" int oc_band_norms(const oc_kv_desc* kv, int32_t first_tile, int32_t count, int32_t band_lo,
                             int32_t band_hi, float* out, int64_t out_row_stride, int32_t* valid_tiles,
                             void* stream) {
  DecodeArgs a{};
  int rc = fill_kv(kv, a);
  if (rc) return rc;
  if (generic_shape(kv->head_dim, a.ts))
    return fail(OC_ERR_UNSUPPORTED, "band norms take head_dim 64 or 128 with 64-token tiles");
  if (!out) return fail(OC_ERR_INVALID, "out is NULL");
  if (first_tile < 0 || count < 0 || (int64_t)first_tile + count > kv->num_tiles)
    return fail(OC_ERR_INVALID, "tile range [%d, %d) outside 0..%d", first_tile, first_tile + count, kv->num_tiles);
  if (band_lo < 0 || band_hi > 64 || band_lo > band_hi)
    return fail(OC_ERR_INVALID, "band [%d, %d) outside the 64 Walsh rows", band_lo, band_hi);
  a.t0 = first_tile;
  a.tcnt = count;
  a.band_lo = band_lo;
  a.band_hi = band_hi;
  a.o_norm = out;
  a.o_stride = out_row_stride;
  a.o_valid = valid_tiles;
  if ((int64_t)kv->num_rows * count == 0) return OC_OK;
  const hipError_t e = dispatch_band(kv->dtype, a, kv->head_dim, (hipStream_t)stream);
  return e == hipSuccess ? OC_OK : hip_fail(e, "band-norm launch");
}

extern "C" int oc_fwht_tiles(const oc_kv_desc* kv, float* out, void* stream) {
  DecodeArgs a{};
  int rc = fill_kv(kv, a);
  if (rc) return rc;
  if (!out) return fail(OC_ERR_INVALID, "out is NULL");
  a.lengths = nullptr;
  a.o_fwht = out;
  if ((int64_t)kv->num_rows * kv->num_tiles == 0) return OC_OK;
  if (generic_shape(kv->head_dim, a.ts)) {
    a.t0 = 0;
    a.tcnt = kv->num_tiles;
    const hipError_t e = gen_launch_score(kv->dtype, a, kv->head_dim, (hipStream_t)stream);
    return e == hipSuccess ? OC_OK : hip_fail(e, "fwht launch");
  }
  const hipError_t e = dispatch_fwht(kv->dtype, a, kv->head_dim, (hipStream_t)stream);
  return e == hipSuccess ? OC_OK : hip_fail(e, "fwht launch");
}

extern "C" int oc_lse_merge(const float* m, const float* l, const float* acc, int32_t rows, int32_t num_splits,
                            int32_t head_dim, void* out, int32_t out_dtype, int64_t out_row_stride, void* stream) {
  if (!m || !l || !acc || !out) return fail(OC_ERR_INVALID, "NULL pointer");
  if (rows < 0 || num_splits < 1 || num_splits > 8192 || head_dim < 1 || head_dim > 1024)
    return fail(OC_ERR_INVALID, "bad sizes");
  if (out_dtype != OC_F32 && out_dtype != OC_F16 && out_dtype != OC_BF16)
    return fail(OC_ERR_INVALID, "out dtype %d", out_dtype);
  return launch_merge(m, l, acc, rows, num_splits, head_dim, out, out_dtype, out_row_stride,
                      (hipStream_t)stream);
}

extern "C" int oc_abi_sizes(size_t* kv_desc_bytes, size_t* decode_params_bytes) {
  if (kv_desc_bytes) *kv_desc_bytes = sizeof(oc_kv_desc);
  if (decode_params_bytes) *decode_params_bytes = sizeof(oc_decode_params);
  return OC_OK;
}

extern "C" int oc_device_cu_count(int32_t* cus) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  int n = 0;
  e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return hip_fail(e, "hipDeviceGetAttribute");
  if (cus) *cus = n;
  return OC_OK;
}

extern "C" int oc_device_props(oc_device_info* info) {
  if (!info) return fail(OC_ERR_INVALID, "info is NULL");
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  hipDeviceProp_t pr;
  e = hipGetDeviceProperties(&pr, dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDeviceProperties");
  memset(info, 0, sizeof *info);
  info->compute_units = pr.multiProcessorCount;
  info->memory_clock_khz = pr.memoryClockRate;
  info->memory_bus_bits = pr.memoryBusWidth;
  info->lds_per_cu_bytes = (int64_t)pr.maxSharedMemoryPerMultiProcessor;
  info->total_memory_bytes = (int64_t)pr.totalGlobalMem;
  info->wave_size = pr.warpSize;
  strncpy(info->arch, pr.gcnArchName, sizeof info->arch - 1);
  strncpy(info->name, pr.name, sizeof info->name - 1);
  return OC_OK;
}

extern "C" const char* oc_version(void) { return "orthocache_hip 0.1.0 (gfx950, abi 1)"; }

extern "C" const char* oc_last_error(void) { return g_last_error.c_str(); }
