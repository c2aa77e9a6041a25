/*
 * orthocache_hip.h -- C ABI of liborthocache_hip.so, the MI355X (gfx950)
 * implementation of OrthoCache's spectral-gated decode attention.
 *
 * Every entry point takes plain device pointers, element strides and sizes,
 * returns an int status (OC_OK = 0) and never lets a C++ exception or a
 * host allocation cross the boundary.  Work is enqueued on the hipStream_t
 * passed in (`stream`, NULL = the default stream); nothing synchronises.
 * oc_last_error() returns a thread-local message for the last failure.
 *
 * Reference interfaces replaced (paths relative to
 * src/orthocache_gpu/triton_kernels/ of the reference tree):
 *   oc_score_tiles  <- _fwht_eviction_kernel launch of triton_fwht_eviction
 *                      (fwht_fused_prototype.py:255-322, launch :305-318)
 *   oc_fwht_tiles   <- the W @ K_tile product that every kernel computes
 *                      (fwht_fused_prototype.py:160-162, fused_eviction.py:268)
 *   oc_decode       <- the main-kernel + reduce-kernel pair of
 *                      fused_orthocache_attention (fused_eviction.py:773-786),
 *                      fused_orthocache_attention_v2 (fused_eviction.py:657-680),
 *                      fused_orthocache_attention_v3_gqa (gqa_eviction.py:603-625),
 *                      fused_orthocache_attention_paged (paged_eviction.py:404-433)
 *   oc_lse_merge    <- _splitk_reduce_kernel (fused_eviction.py:316-373),
 *                      _gqa_splitk_reduce_kernel (gqa_eviction.py:458-495),
 *                      _paged_splitk_reduce_kernel (paged_eviction.py:195-237)
 *   oc_device_cu_count <- torch.cuda.get_device_properties(...).multi_processor_count
 *                      as read by _auto_num_splits (fused_eviction.py:556-570)
 *   oc_band_norms   <- SpectralNormCache.update_prefill / populate_from_keys
 *                      (src/orthocache_gpu/norm_cache.py:58-117)
 *   oc_decode_gate  <- _decode_gate_kernel + decode_gate (decode_gate.py:108-245);
 *                      with the Walsh-subspace q norm, _pytorch_decode_gate
 *                      (decode_gate.py:248-295)
 *   oc_q_high_norms <- compute_q_high_norm_exact (decode_gate.py:54-100)
 *   oc_apply_tile_mask <- apply_decode_mask / apply_decode_mask_vectorized
 *                      (decode_gate.py:302-374)
 *   oc_score_tile_range: no reference counterpart (the append path of the
 *                      score cache: rescore the tiles a decode step completed)
 *   oc_tile_mask_from_blocks + oc_decode(OC_GATE_MASK) <- the kernels of
 *                      triton_block_sparse_attention (sparse_attention.py:208-279)
 *                      and triton_indirect_attention (indirect_attention.py:200-286)
 * Model-side attention hook (eval/perplexity_eval.py of the reference tree):
 *   oc_prefill_attention <- the prefill branch of
 *                      OrthoCache_GQA_Attention.orthocache_attention (logits,
 *                      causal mask, tile eviction, softmax, entropy, P @ V;
 *                      perplexity_eval.py:399-545) and _dense_attention
 *                      (perplexity_eval.py:675-689)
 *   oc_row_norms + oc_kth_smallest <- torch.norm(q_group, dim=-1) and its
 *                      .median(dim=1) (perplexity_eval.py:454-456);
 *                      _compute_q_high_norm (perplexity_eval.py:547-573)
 *   oc_group_gate   <- the per-(kv head, tile) Cauchy-Schwarz compares of the
 *                      prefill and decode branches (perplexity_eval.py:476-491,
 *                      :639-657)
 * orthocache_forward(mode='compact') (src/orthocache_gpu/ of the reference tree):
 *   oc_block_spectra <- fwht_512 (fwht.py:6-45) with compute_spectral_bands,
 *                      compute_spectral_decay_ratio, compute_block_energy and
 *                      compute_query_aware_bounds (spectral_energy.py:26-200)
 *   oc_stream_compact <- stream_compact (adaptive_attention.py:33-45)
 *   oc_compact_gate  <- compute_multiband_mask, _compute_auto_tau, the zeta
 *                      statistics and classify_eviction as orthocache_forward
 *                      runs them (pipeline.py:458-527)
 *   oc_block_regimes <- compute_block_beta + classify_eviction
 *                      (perfect_eviction.py:75-186)
 *   oc_device_props  <- torch.cuda.get_device_properties as _detect_gpu_profile
 *                      reads it (pipeline.py:209-280)
 */
#ifndef ORTHOCACHE_HIP_H
#define ORTHOCACHE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OC_ABI_VERSION 1

/* status codes */
#define OC_OK 0
#define OC_ERR_INVALID 1      /* bad argument (shape, dtype, stride, size) */
#define OC_ERR_UNSUPPORTED 2  /* valid but not implemented by these kernels */
#define OC_ERR_HIP 3          /* a HIP runtime call failed */
#define OC_ERR_WORKSPACE 4    /* workspace too small */

/* element types of K/V (all four) and of q/out (the first three) */
#define OC_F32 0
#define OC_F16 1
#define OC_BF16 2
#define OC_FP8_E4M3FN 3

/* tile gates */
#define OC_GATE_NONE 0  /* dense decode: every tile retained                    */
#define OC_GATE_ZETA 1  /* retain iff !(e_high/(e_low+1e-6) > threshold)        */
#define OC_GATE_CS 2    /* retain iff !(max_g ||q_g|| * sqrt(e_high) <= threshold) */
#define OC_GATE_MASK 3  /* retain iff tile_mask[row, tile] != 0 (cached mode)      */

/* where tile scores come from */
#define OC_MODE_SINGLE_PASS 0 /* scores computed from K inside the decode kernel  */
#define OC_MODE_CACHED 1      /* scores read from score_e_low/score_e_high; K and
                                 V are read for retained tiles only               */

/* K dequantisation */
#define OC_KSCALE_NONE 0     /* k = float(k_elem)                                   */
#define OC_KSCALE_Q_FOLD 1   /* q := round_qdtype(float(q) * k_scale), k = float(k_elem)
                                (fused_eviction.py:619-621, gqa_eviction.py:565-567) */
#define OC_KSCALE_TILE 3     /* k = float(k_elem) * k_scales[row, tile]   (extension) */
#define OC_KSCALE_DEQUANT 4  /* k = round_bf16(float(k_elem) * k_scale): the reference's
                                k_cache.to(q.dtype) * k_scale (paged_eviction.py:354-357)
                                done in-kernel, for fp8 K: by oc_score_tiles /
                                oc_score_tile_range, and by oc_decode / oc_decode_static
                                for bf16 q in cached or dense decodes that take the
                                per-wave-prologue kernel (else OC_ERR_UNSUPPORTED);
                                other entry points refuse it */

/* V dequantisation */
#define OC_VSCALE_NONE 0
#define OC_VSCALE_TILE 1     /* v = float(v_elem) * v_scales[row, tile]   (extension) */

/*
 * KV layout.  A "row" is one (sequence, kv head) pair; rows are decoded
 * independently.  Tiles are 64 consecutive tokens of a row.
 *
 * paged == 0: element (row r, token t, dim c) of K is at
 *             k + (r * k_row_stride + t * k_token_stride + c) elements.
 * paged == 1: row r = b * num_kv_heads + h; token t of sequence b lives in
 *             physical block p = block_tables[b * bt_stride + t / block_size]
 *             at k + (p * k_block_stride + h * k_head_stride
 *                     + (t % block_size) * k_token_stride + c) elements.
 *             Block ids outside [0, num_blocks) make the call fail with
 *             OC_ERR_INVALID reported through `error_flag`.
 * lengths:    NULL, or int32 token counts indexed by r / rows_per_length;
 *             a row has ceil(len/64) tiles (at most num_tiles).  Full tiles
 *             are scored; a partial tail tile is always retained and its
 *             tokens past len are masked.  (extension)
 */
typedef struct oc_kv_desc {
  const void* k;
  const void* v;
  int32_t dtype;        /* OC_F32 .. OC_FP8_E4M3FN: K's, and V's unless v_dtype says otherwise */
  int32_t head_dim;     /* a power of two <= 512 (64 and 128: the tuned kernels) */
  int32_t num_rows;
  int32_t num_tiles;    /* tiles per row (upper bound when lengths != NULL) */
  int64_t k_row_stride, k_token_stride;
  int64_t v_row_stride, v_token_stride;
  int32_t paged;
  int32_t block_size;   /* power of two >= 8 */
  int32_t num_kv_heads;
  int32_t rows_per_length;
  const int32_t* block_tables;
  int64_t bt_stride;
  int64_t num_blocks;
  int64_t k_block_stride, k_head_stride;
  int64_t v_block_stride, v_head_stride;
  const int32_t* lengths;
  int32_t k_scale_mode;     /* OC_KSCALE_* */
  float k_scale;            /* scalar for Q_FOLD */
  const float* k_scales;    /* (num_rows, >= num_tiles) for OC_KSCALE_TILE */
  int64_t k_scales_row_stride;
  int32_t v_scale_mode;     /* OC_VSCALE_* */
  int32_t num_tokens;       /* lengths == NULL: tokens of every row, 1 .. num_tiles * 64
                               (0 = num_tiles * 64); a partial last tile without a
                               lengths array */
  const float* v_scales;
  int64_t v_scales_row_stride;
  int32_t* error_flag;      /* optional int32 set non-zero on a bad block id */
  int32_t v_dtype;          /* 0: V has K's dtype; OC_BF16 with fp8 K: bf16 V read as it
                               is (extension; the reference's fp8 caches pair an fp8 K
                               with a wider V, test_fp8.py:43-57).  Entry points that
                               read no V accept it; oc_decode / oc_decode_static take it
                               for bf16 q in the per-wave-prologue kernel's cached and
                               dense decodes, else OC_ERR_UNSUPPORTED */
  int32_t tile_size;        /* tokens per spectral tile: 0 (= 64) or a power of two <= 256
                               (fused_eviction.py:610, gqa_eviction.py:552,
                               paged_eviction.py:346: any power of two; the bands stay
                               the Walsh rows [1, 8) and [32, 64) clipped to the tile).
                               Tiles other than 64 tokens, and head_dim other than 64
                               and 128, run the portable kernels (oc_generic.hip),
                               except oc_decode at head_dim 256 with 64-token tiles,
                               bf16/f16 K/V with q of K's type or fp8 K/V with bf16
                               q (bf16 V beside fp8 K and in-kernel dequantisation:
                               G <= 8), pages of >= 16 tokens and 16-byte aligned
                               q, K, V and strides, and at head_dim 32 with 64-token
                               tiles, bf16/f16 K/V with q of K's type under the same
                               page and alignment conditions (the matrix-core kernels);
                               num_tiles and num_tokens count these tiles. */
} oc_kv_desc;

/*
 * oc_score_tiles -- per-(row, tile) band energies of the 64-point Walsh-
 * Hadamard transform along the token axis (natural-order rows [1,8) and
 * [32,64), fwht_fused_prototype.py:44-50), zeta = e_high/(e_low+1e-6) and
 * keep = !(zeta > zeta_max).  Outputs are (num_rows, num_tiles) row-major
 * with row stride `out_row_stride`; any output pointer may be NULL.
 * A partial tail tile gets e_low = e_high = zeta = 0 and keep = 1; tiles
 * past a row's length get keep = 0.
 * Replaces the launch in triton_fwht_eviction (fwht_fused_prototype.py:305-318).
 */
int oc_score_tiles(const oc_kv_desc* kv, double zeta_max, float* e_low, float* e_high,
                   float* zeta, uint8_t* keep, int64_t out_row_stride, void* stream);

/*
 * oc_fwht_tiles -- the full transform X = W64 @ K_tile (float32) of every
 * tile of every row, written to out[((r * num_tiles + t) * 64 + s) * head_dim + c].
 * Replaces the W @ K products (fwht_fused_prototype.py:160-162).
 */
int oc_fwht_tiles(const oc_kv_desc* kv, float* out, void* stream);

/*
 * oc_score_tile_range -- oc_score_tiles for tiles [first_tile, first_tile +
 * count) of every row only, written at those columns of the outputs.  The
 * append path of a score cache: after a decode step completes a tile, only
 * that tile is rescored.  No reference counterpart.
 */
int oc_score_tile_range(const oc_kv_desc* kv, int32_t first_tile, int32_t count, double zeta_max,
                        float* e_low, float* e_high, float* zeta, uint8_t* keep,
                        int64_t out_row_stride, void* stream);

/*
 * oc_band_norms -- ||(W64 @ K_t)[band_lo:band_hi]||_F (float32, 0 when below
 * 1e-38) of tiles [first_tile, first_tile + count) of every row, written to
 * out[r * out_row_stride + t]; tiles not wholly inside a row's length are
 * skipped.  valid_tiles (optional, int32 per row) is raised to t + 1 for
 * every tile written.  Replaces SpectralNormCache.update_prefill and
 * populate_from_keys (norm_cache.py:58-117; their band is [48, 64)).
 */
int oc_band_norms(const oc_kv_desc* kv, int32_t first_tile, int32_t count, int32_t band_lo,
                  int32_t band_hi, float* out, int64_t out_row_stride, int32_t* valid_tiles,
                  void* stream);

/* q-norm of the decode gate */
#define OC_QNORM_SPATIAL 0     /* ||q||_2 (the GPU path of decode_gate) */
#define OC_QNORM_WALSH_HIGH 1  /* Walsh-subspace ||q_high||_2 (compute_q_high_norm_exact) */

/*
 * oc_decode_gate -- the O(1) decode gate from cached K band norms.  For kv
 * head h: qn = max over its G query heads of the q norm (`q_norm_mode`;
 * q rows h*G .. h*G+G-1 of (num_kv_heads*G, head_dim), q_dtype F32/F16/BF16),
 * q_norms[h] = qn, and for t < num_tiles
 *   mask[h, t] = (qn * norm_cache[h, t] <= (float)tau_norm)   (1 = evict),
 * mask[h, t] = 0 for num_tiles <= t < max_tiles.  tau_norm = tau * tile_size
 * * head_dim, as decode_gate pre-multiplies it (decode_gate.py:210-212).
 * Replaces _decode_gate_kernel and its launch (decode_gate.py:108-245).
 */
int oc_decode_gate(const void* q, int32_t q_dtype, int64_t q_row_stride, int32_t num_kv_heads, int32_t G,
                   int32_t head_dim, const float* norm_cache, int64_t norm_row_stride, int32_t num_tiles,
                   int32_t max_tiles, double tau_norm, int32_t q_norm_mode, int32_t low_band,
                   uint8_t* mask, int64_t mask_row_stride, float* q_norms, void* stream);

/*
 * oc_q_high_norms -- out[r] = sqrt(max(||q_r||^2 - sum_i S_i^2 / bs, 0)),
 * S_i the sums of the low_band blocks of bs = head_dim / low_band elements
 * (float32).  Replaces compute_q_high_norm_exact (decode_gate.py:54-100).
 */
int oc_q_high_norms(const void* q, int32_t q_dtype, int64_t rows, int32_t head_dim, int64_t q_row_stride,
                    int32_t low_band, float* out, void* stream);

/*
 * oc_apply_tile_mask -- in place, logits[h, s] = -inf for every query head
 * h < num_q_heads and token s < seq_len whose tile t = s / tile_size is
 * below num_tiles with mask[h / G, t] != 0.  logits dtype F32/F16/BF16,
 * rows `logits_row_stride` elements apart, tokens contiguous.  Replaces
 * apply_decode_mask and apply_decode_mask_vectorized (decode_gate.py:302-374).
 */
/*
 * oc_tile_mask_from_blocks -- the 64-token tile mask (count = num_blocks *
 * tiles_per_block bytes) of a block mask or an index list: with block_mask,
 * tile_mask[t] = block_mask[t / tiles_per_block]; with indices (count
 * int32), tile_mask = 1 exactly on the tiles of the listed blocks, and an
 * index outside [0, num_blocks) is skipped and sets *error_flag (if given).
 * For the block-sparse and indirect attention wrappers
 * (sparse_attention.py:208-279, indirect_attention.py:200-286), which run
 * oc_decode with OC_GATE_MASK on the result.
 */
int oc_tile_mask_from_blocks(const uint8_t* block_mask, const int32_t* indices, int32_t count, int32_t num_blocks,
                             int32_t tiles_per_block, uint8_t* tile_mask, int32_t* error_flag, void* stream);

int oc_apply_tile_mask(void* logits, int32_t dtype, int32_t num_q_heads, int64_t seq_len,
                       int64_t logits_row_stride, const uint8_t* mask, int64_t mask_row_stride, int32_t G,
                       int32_t tile_size, int32_t num_tiles, void* stream);

/* group reductions of oc_group_gate */
#define OC_GROUP_MAX 0     /* largest of the G per-head norms (NaN propagates) */
#define OC_GROUP_MEDIAN 1  /* element of rank G/2 (0-based) of their ascending order */

/*
 * oc_row_norms -- out[(i0 * n1 + i1) * n2 + i2] = ||x[i0, i1, i2, :]||_2 over
 * head_dim elements (dtype F32/F16/BF16, element strides stride0..2, the
 * last dimension contiguous), accumulated in float32; with low_band > 0 the
 * Walsh-subspace high part sqrt(max(||x||^2 - sum_i S_i^2 / bs, 0)) as in
 * oc_q_high_norms.  Replaces torch.norm(q_group, p=2, dim=-1) of the hook's
 * prefill gate (perplexity_eval.py:454) and _compute_q_high_norm
 * (perplexity_eval.py:547-573).
 */
int oc_row_norms(const void* x, int32_t dtype, int64_t n0, int64_t n1, int64_t n2, int64_t stride0,
                 int64_t stride1, int64_t stride2, int32_t head_dim, int32_t low_band, float* out, void* stream);

/*
 * oc_kth_smallest -- out[r] = the k-th smallest (0-based) of the n floats
 * x[r * row_stride .. + n), for non-negative inputs (norms; NaN sorts
 * last).  Exact (radix select over the bit patterns).  k = (n - 1) / 2 is
 * torch.median's lower median (perplexity_eval.py:456).
 */
int oc_kth_smallest(const float* x, int64_t rows, int64_t n, int64_t row_stride, int64_t k, float* out,
                    void* stream);

/*
 * oc_group_gate -- for every (batch b, kv head h): qn = reduce over the G
 * per-head norms q_norms[(b * num_kv_heads + h) * G + g] (OC_GROUP_MAX or
 * OC_GROUP_MEDIAN), group_norms[b * num_kv_heads + h] = qn (if given), and
 * for t < mask_cols
 *   evict(t) = t < num_tiles && qn * k_norms[b * k_norms_stride_b + h * k_norms_stride_h + t]
 *              <= tau_norm      (product and compare in float64)
 *   mask[b * mask_stride_b + h * mask_stride_h + t] = keep_polarity ? !evict(t) : evict(t)
 * (keep_polarity 0: 1 = evict, the prefill kernel's convention; 1: 1 =
 * attend, oc_decode's OC_GATE_MASK convention).  tau_norm = tau * 64 *
 * head_dim: the hook compares qn * ||K_high|| / (64 * head_dim) with tau
 * (perplexity_eval.py:476-491 with the max of the per-head medians,
 * :639-657 with the median of the Walsh-subspace norms).  gate_stats (if
 * given, float32 (batch * num_kv_heads, 3)): per (b, h) the number of
 * evicted tiles t < num_tiles, qn and the largest k_norms entry of the
 * tiles t < num_tiles (NaN if one is NaN, -inf if there are none) -- the
 * hook's per-call statistics (evicted tiles, q and K information density)
 * before its reductions over heads and its clamp at 0.
 */
int oc_group_gate(const float* q_norms, int32_t batch, int32_t num_kv_heads, int32_t G, int32_t reduce,
                  const float* k_norms, int64_t k_norms_stride_b, int64_t k_norms_stride_h, int32_t num_tiles,
                  int32_t mask_cols, double tau_norm, int32_t keep_polarity, uint8_t* mask, int64_t mask_stride_b,
                  int64_t mask_stride_h, float* group_norms, float* gate_stats, void* stream);

/*
 * oc_prefill_attention -- causal GQA attention of q_len queries over kv_len
 * keys (query s sees keys j <= s + kv_len - q_len), skipping the 64-token
 * tiles t < kv_len / 64 whose tile_mask byte is set (1 = evict, for every
 * query of the kv head's G query heads):
 *   out[b, h, s] = sum_j softmax_j(q[b, h, s] . k[b, h / G, j] * scale) v[b, h / G, j]
 * over the visible, retained j; a query with none gets zeros (the hook's
 * nan_to_num).  float32 accumulation; out in dtype (round to nearest even).
 * With entropy given, entropy[(b * num_q_heads + h) * q_len + s] =
 * -sum_j p_j ln max(p_j, 1e-10) over all kv_len keys (evicted and masked
 * keys count as p = 0), the attention entropy the hook's EntropyGovernor
 * reads (perplexity_eval.py:522-531).  dtype F32/F16/BF16, head_dim 64 or
 * 128; q/k/v rows 16-byte aligned.
 */
typedef struct oc_prefill_params {
  const void* q;                  /* (batch, num_q_heads, q_len, head_dim) */
  int64_t q_stride_b, q_stride_h, q_stride_s;  /* elements; head_dim contiguous */
  const void* k;                  /* (batch, num_kv_heads, kv_len, head_dim) */
  int64_t k_stride_b, k_stride_h, k_stride_s;
  const void* v;
  int64_t v_stride_b, v_stride_h, v_stride_s;
  void* out;                      /* (batch, num_q_heads, q_len, head_dim) */
  int64_t out_stride_b, out_stride_h, out_stride_s;
  int32_t dtype;                  /* of q, k, v and out */
  int32_t batch, num_q_heads, num_kv_heads, q_len, kv_len, head_dim;
  const uint8_t* tile_mask;       /* (batch, num_kv_heads, tile_mask_cols) or NULL */
  int64_t tile_mask_stride_b, tile_mask_stride_h;
  int32_t tile_mask_cols;         /* >= kv_len / 64 */
  float scale;                    /* logit scale, 1/sqrt(head_dim) in the hook */
  float* entropy;                 /* (batch, num_q_heads, q_len) or NULL */
  void* workspace;                /* optional (extension): when the call's workgroups fit in one round,
                                     the longest causal windows run as two workgroups each, one of which
                                     merges the two states; NULL: one workgroup per query block */
  size_t workspace_bytes;         /* >= oc_prefill_workspace_size(p); its first 64 KiB hold counters that
                                     are zero before the first call (every call leaves them zero) */
} oc_prefill_params;

int oc_prefill_attention(const oc_prefill_params* p, void* stream);

/* bytes of workspace that lets oc_prefill_attention split the longest causal
 * windows (0: this call would not split).  No reference counterpart. */
size_t oc_prefill_workspace_size(const oc_prefill_params* p);

/* sizeof(oc_prefill_params) as compiled, for binding checks */
size_t oc_prefill_params_bytes(void);

/*
 * oc_block_spectra -- statistics of the normalised natural-order 512-point
 * Walsh-Hadamard transform X = H512 K_b / sqrt(512) of every 512-token
 * block b and head h of K (seq, num_heads, head_dim), as written by
 * fwht_512 (fwht.py:6-45), accumulated in float32:
 *   e_low  = sum_{u in [1, 64)}    ||X[u]||^2    e_mid = sum_{u in [64, 256)} ||X[u]||^2
 *   e_high = sum_{u in [256, 512)} ||X[u]||^2    zeta  = e_high / (e_low + 1e-6)
 *   e_ac   = e_low + e_mid + e_high (all rows but DC)
 *   energy = sum_t ||k_t||^2 (compute_block_energy)
 *   block_mean[b, h, :] = X[0] / sqrt(512)
 * each (num_blocks, num_heads) float32, any may be NULL.  With q (q_len,
 * num_heads, head_dim) given, the query-aware bounds of
 * compute_query_aware_bounds (spectral_energy.py:140-180)
 *   bound[s, b, h] = (q_s . block_mean + ||q_s|| sqrt(e_ac)) / sqrt(head_dim)
 * go to bounds (q_len, num_blocks, num_heads) and their max over s to
 * max_bound (num_blocks, num_heads), each if given.  block_size must be
 * 512; head_dim a multiple of 8 up to 256; K rows 16-byte aligned.
 */
typedef struct oc_spectra_params {
  const void* k;
  int32_t dtype;                  /* OC_F32 / OC_F16 / OC_BF16 */
  int32_t num_blocks, num_heads, head_dim, block_size;
  int64_t k_token_stride, k_head_stride;  /* elements */
  const void* q;                  /* (q_len, num_heads, head_dim) or NULL */
  int32_t q_dtype, q_len;
  int64_t q_token_stride, q_head_stride;  /* elements */
  float* e_low;
  float* e_mid;
  float* e_high;
  float* zeta;
  float* e_ac;
  float* energy;
  float* block_mean;              /* (num_blocks, num_heads, head_dim) */
  float* bounds;                  /* (q_len, num_blocks, num_heads) */
  float* max_bound;               /* (num_blocks, num_heads) */
  float* q_norm_max;              /* (num_heads,) max over queries of ||q_s|| */
} oc_spectra_params;

int oc_block_spectra(const oc_spectra_params* p, void* stream);

/* sizeof(oc_spectra_params) as compiled, for binding checks */
size_t oc_spectra_params_bytes(void);

/*
 * oc_compact_gate -- the compact pipeline's gates and statistics from
 * oc_block_spectra's outputs, in one workgroup (pipeline.py:458-527):
 * tau = the given value, or with tau_auto mean - std (unbiased) of
 * max_bound (_compute_auto_tau, pipeline.py:571-583); (b, h) is retained iff
 * max_bound >= tau and zeta <= zeta_max (compute_multiband_mask);
 * block_mask[b] = any head retained; tile_mask[b * tiles_per_block + i] =
 * block_mask[b]; stats[0..8] = tau, mean / std (unbiased) / min / max over
 * blocks of the head-mean zeta, the retained count, and the perfect and
 * statistical counts of the evicted blocks: beta_b = max_h q_norm_max[h]
 * sqrt(energy[b, h]) / sqrt(head_dim), z_max = the largest max_bound of a
 * retained block (0 if none), perfect iff z_max - beta_b >= underflow
 * (classify_eviction, perfect_eviction.py:107-186); stats[8] = z_max.
 */
int oc_compact_gate(const float* max_bound, const float* zeta, const float* energy, const float* q_norm_max,
                    int32_t num_blocks, int32_t num_heads, int32_t head_dim, double tau, int32_t tau_auto,
                    double zeta_max, double underflow, int32_t tiles_per_block, uint8_t* block_mask,
                    uint8_t* tile_mask, float* stats, void* stream);

/*
 * oc_block_regimes -- the eviction regime of every block of a compact-mode
 * block table.  With qn[h] = max over s of q_norms[s * num_heads + h] (the
 * (q_len, num_heads) spatial query norms, e.g. from oc_row_norms) and
 * E = energy (num_blocks, num_heads):
 *   beta_full[b, h] = qn[h] * sqrt(max(E[b, h], 0)) / sqrt(head_dim)
 *   beta[b] = max_h beta_full[b, h],  gap[b] = z - beta[b]
 *   regime[b] = 0 (retained: any of block_mask[b * mask_heads + 0 ..
 *               mask_heads) set), 1 (evicted, gap >= underflow: exp of
 *               every logit underflows, "perfect"), 2 (evicted, gap <
 *               underflow, "statistical"); 0 as well for a NaN gap
 *   counts = (regime-1 blocks, regime-2 blocks, retained blocks)  (int32)
 * z = max(z_values[0 .. z_count)) when z_values is given, else z_max.
 * float32 arithmetic, NaN propagating through every maximum; mask_heads 1
 * or num_heads; beta_full may be NULL.  Replaces compute_block_beta and
 * classify_eviction (perfect_eviction.py:75-186).
 */
int oc_block_regimes(const float* q_norms, int32_t q_len, int32_t num_heads, const float* energy,
                     int32_t num_blocks, int32_t head_dim, double z_max, const float* z_values, int32_t z_count,
                     const uint8_t* block_mask, int32_t mask_heads, double underflow, int32_t* regime,
                     float* beta, float* gap, float* beta_full, int32_t* counts, void* stream);

/*
 * oc_stream_compact -- the active-first stable permutation of num_blocks
 * blocks (block_mask != 0 = retained): indices[r] (int64) is the r-th
 * retained block, followed by the evicted blocks in order, and
 * *num_active the retained count (device int32).  Replaces stream_compact
 * (adaptive_attention.py:33-45), an argsort of where(mask, i, n + i).
 */
int oc_stream_compact(const uint8_t* block_mask, int32_t num_blocks, int64_t* indices, int32_t* num_active,
                      void* stream);

/* decode parameters; see oc_decode */
typedef struct oc_decode_params {
  oc_kv_desc kv;
  const void* q;            /* (num_rows * G, head_dim) */
  int32_t q_dtype;          /* OC_F32 / OC_F16 / OC_BF16 */
  int32_t G;                /* query heads per row, 1..64 */
  int64_t q_row_stride;     /* elements */
  int32_t gate;             /* OC_GATE_* */
  int32_t mode;             /* OC_MODE_* */
  double threshold;         /* zeta_max or tau */
  const float* score_e_low; /* cached mode: (num_rows, num_tiles) */
  const float* score_e_high;
  int64_t score_row_stride;
  int32_t num_splits;       /* P >= 1: split s owns tiles {s + kP} */
  int32_t splits_per_group; /* logical splits per workgroup (0 = choose); the
                               partial states are per group of splits */
  int32_t out_dtype;        /* OC_F32 / OC_F16 / OC_BF16 */
  int32_t portable;         /* 1: run the portable kernels whatever the shape (they
                               take every shape; for testing them against the tuned
                               kernels on the same inputs); 0: the tuned kernels where
                               they apply */
  void* out;                /* (num_rows * G, head_dim) */
  int64_t out_row_stride;
  uint8_t* keep_out;        /* optional (num_rows, num_tiles): 1 = retained */
  int64_t keep_row_stride;
  int32_t* split_counts;    /* optional (num_rows, Pg): retained tiles per group */
  float* partial_m;         /* optional (num_rows * G, Pg); NULL = workspace */
  float* partial_l;         /* optional (num_rows * G, Pg) */
  float* partial_acc;       /* optional (num_rows * G, Pg, head_dim);
                               Pg = oc_decode_num_groups(p) */
  void* workspace;          /* device memory, oc_decode_workspace_size() bytes */
  size_t workspace_bytes;
  const uint8_t* tile_mask; /* OC_GATE_MASK: (num_rows, num_tiles), 1 = attend */
  int64_t tile_mask_row_stride;
} oc_decode_params;

/* number of partial states per (row, query head): ceil(P / spw), with spw
 * the effective splits_per_group of `p` */
int32_t oc_decode_num_groups(const oc_decode_params* p);

/* bytes of device workspace oc_decode needs for `p` (0 when partials are given) */
size_t oc_decode_workspace_size(const oc_decode_params* p);

/*
 * oc_decode -- gated split-K flash-decode plus the log-sum-exp merge.
 * For every row r and split s, the online-softmax state of each of its G
 * query heads over the retained tiles {s + kP} (fused_eviction.py:259) is
 * formed in float32 (m0 = -1e9), then the P states are merged and
 * out = acc / max(l, 1e-9) is written in out_dtype.  One workgroup handles
 * splits_per_group consecutive splits and writes their merged state (the
 * merge is associative); with splits_per_group = 1 the partials are exactly
 * the per-split states.
 * With out == NULL (and the three partial_* buffers given) only the
 * partial states are written; the caller merges them with oc_lse_merge,
 * e.g. after gathering the partials of a sequence split across devices.
 */
int oc_decode(const oc_decode_params* p, void* stream);

/*
 * oc_decode_static -- oc_decode that allocates nothing and takes no
 * workspace: p->workspace / workspace_bytes are ignored, and the split
 * partials and merge counters live in a static device array of
 * oc_decode_static_scratch_bytes() bytes (16 MiB), one per GPU, held until
 * the process ends.  No counterpart in the reference: for callers that
 * cannot allocate device memory (code under HIP graph capture, serving
 * loops, harnesses that forbid hipMalloc).  Same results as oc_decode.
 * A call needing more than the array (oc_decode_workspace_size(p) > the
 * scratch bytes) fails with OC_ERR_WORKSPACE.  Every call on a GPU shares
 * its array: calls that overlap on one GPU (other streams or threads) race
 * and must be serialised by the caller.  The first call on a device clears
 * the merge counters with a small kernel on `stream`; every call leaves them
 * zero.
 */
int oc_decode_static(const oc_decode_params* p, void* stream);

/* bytes of the static device scratch of oc_decode_static */
size_t oc_decode_static_scratch_bytes(void);

/*
 * oc_hook_decode -- the model hook's decode step (q_len 1, norm cache
 * populated) in one call: for every batch element b and kv head h, the
 * Walsh-subspace high norms of the group's G query rows (as oc_row_norms
 * with low_band), their median qn (rank G/2), the gate
 *   evict(t) = qn * k_norms[h * k_norms_stride + t] <= tau_norm   (float64)
 * over the complete tiles t < kv_len / 64 (a partial last tile is always
 * attended), then attention of the G heads over the retained tiles
 * (oc_decode with OC_GATE_MASK, cached mode) written to out in `dtype`.
 * Two launches (gate, decode).  Replaces the per-batch loop of the
 * reference's decode branch (perplexity_eval.py:580-662): its per-head
 * _compute_q_high_norm (:547-573), the median, the norm-cache lookups and
 * compares, the -inf logit masking and the float32 softmax(q K^T) V.
 * tau_norm = tau * 64 * head_dim.  k_norms (cached ||(H64 K_t)[48:64]||_F,
 * float32, (num_kv_heads, >= kv_len / 64) with row stride k_norms_stride)
 * is shared by the batch, as the reference's norm cache.  gate_stats
 * (optional, float32 (batch * num_kv_heads, 3)) as oc_group_gate's.
 * The workspace (oc_hook_decode_workspace_size bytes) must be zero before
 * its first use and is left so; calls on one stream may share it.
 */
typedef struct oc_hook_decode_params {
  const void* q;                 /* (batch * num_kv_heads * G, head_dim), row stride q_row_stride */
  int64_t q_row_stride;          /* elements */
  const void* k;                 /* rows (batch * num_kv_heads) of kv_len tokens */
  const void* v;
  int64_t k_row_stride, k_token_stride;  /* elements; head_dim contiguous */
  int64_t v_row_stride, v_token_stride;
  int32_t dtype;                 /* of q, K, V and out: OC_F32 / OC_F16 / OC_BF16 */
  int32_t batch, num_kv_heads, G, head_dim, kv_len;
  const float* k_norms;
  int64_t k_norms_stride;        /* elements between kv heads */
  double tau_norm;
  int32_t low_band;              /* Walsh bands of q (the hook's 8) */
  int32_t num_splits;            /* 0: min(#CU, max(1, T / 4), T) over T = ceil(kv_len / 64) tiles */
  void* out;                     /* (batch * num_kv_heads * G, head_dim), row stride out_row_stride */
  int64_t out_row_stride;
  float* gate_stats;
  void* workspace;
  size_t workspace_bytes;
} oc_hook_decode_params;

size_t oc_hook_decode_workspace_size(const oc_hook_decode_params* p);
int oc_hook_decode(const oc_hook_decode_params* p, void* stream);

/* sizeof(oc_hook_decode_params) as compiled, for binding checks */
size_t oc_hook_decode_params_bytes(void);

/*
 * oc_lse_merge -- out[r, :] = merge over s of (m[r,s], l[r,s], acc[r,s,:]),
 * acc/max(l, 1e-9), written in out_dtype with row stride out_row_stride.
 */
int oc_lse_merge(const float* m, const float* l, const float* acc, int32_t rows,
                 int32_t num_splits, int32_t head_dim, void* out, int32_t out_dtype,
                 int64_t out_row_stride, void* stream);

/*
 * oc_dequant_fp8 -- dst[i] = round_out(float(src[i]) * scale) for n
 * fp8-e4m3fn elements, written as out_dtype (OC_F32 / OC_F16 / OC_BF16, ties
 * to even).  This is the reference's paged fp8 key dequantisation,
 * k_cache.to(q.dtype) * k_scale (paged_eviction.py:354-357); src and dst
 * must be 16-byte aligned.
 */
int oc_dequant_fp8(const void* src, int64_t n, float scale, int32_t out_dtype, void* dst, void* stream);

/* oc_hbm_read_probe -- measurement aid with no counterpart in the
 * reference: streams `bytes` (a multiple of 16, src 16-byte aligned) from
 * device memory with 128-bit loads over `blocks` 256-thread workgroups and
 * XOR-folds them per thread (sink[0..blocks) is written only when a
 * thread's fold equals a fixed sentinel, which keeps the loads live).  Timed by bench.py to state the achievable read bandwidth
 * next to the 8 TB/s peak. */
int oc_hbm_read_probe(const void* src, size_t bytes, float* sink, int32_t blocks, void* stream);

/* oc_hbm_gather_probe -- measurement aid with no counterpart in the
 * reference: the decode's tile access pattern without its arithmetic.
 * n_steps steps of pieces_per_step (1..8) pieces each, piece i of step s at
 * byte offset piece_offsets[s * pieces_per_step + i] from base (1 KiB
 * aligned), loads_per_step (16 or 32) KiB a step split evenly over its
 * pieces; blocks 512-thread workgroups, each taking an even share of the
 * steps, one step in flight per wave (non-temporal 128-bit loads).  Timed by
 * bench.py to state the read bandwidth of the decode's patterns (contiguous
 * 16-bit and fp8 tiles, 4 KiB pages) beside the decode's own. */
int oc_hbm_gather_probe(const void* base, const int64_t* piece_offsets, int64_t n_steps, int32_t pieces_per_step,
                        int32_t loads_per_step, float* sink, int32_t blocks, void* stream);

/* sizeof(oc_kv_desc) and sizeof(oc_decode_params) as compiled into the
 * library, so that a binding can check its own struct layout (no
 * counterpart in the reference, which has no native ABI) */
int oc_abi_sizes(size_t* kv_desc_bytes, size_t* decode_params_bytes);

/* number of compute units of the current device (256 on MI355X) */
int oc_device_cu_count(int32_t* cus);

/* properties of the current device that the host side sizes its dispatch
 * and its crossover model by (no counterpart in the reference, which reads
 * torch.cuda.get_device_properties, pipeline.py:209-280) */
typedef struct oc_device_info {
  char arch[64];               /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
  char name[128];
  int32_t compute_units;
  int32_t wave_size;
  int32_t memory_clock_khz;    /* peak memory clock */
  int32_t memory_bus_bits;     /* memory interface width */
  int64_t lds_per_cu_bytes;
  int64_t total_memory_bytes;
} oc_device_info;

int oc_device_props(oc_device_info* info);

const char* oc_version(void);
const char* oc_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* ORTHOCACHE_HIP_H */
