"""CPU tests of the boundary: the C-ABI library loads and exports every
function include/orthocache_hip.h declares, the binding's struct layout
matches, and the drop-in entry points raise the reference's assertion
messages (these checks run before any GPU work).  No kernel is launched."""

import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "orthocache_hip.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(oc_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_expected_api():
    names = _declared()
    for n in ("oc_score_tiles", "oc_fwht_tiles", "oc_decode", "oc_decode_workspace_size", "oc_lse_merge",
              "oc_device_cu_count", "oc_version", "oc_last_error", "oc_abi_sizes"):
        assert n in names


def test_library_exports_every_declared_symbol():
    import ctypes
    from orthocache_gpu import _native as N
    lib = ctypes.CDLL(N.LIB_PATH)
    for name in _declared():
        assert hasattr(lib, name), name
        assert name in N.SIGNATURES, f"binding lacks {name}"


def test_struct_layout_matches_library():
    import ctypes
    from orthocache_gpu import _native as N
    N.lib()  # raises on a mismatch
    kv, p = ctypes.c_size_t(), ctypes.c_size_t()
    assert N.lib().oc_abi_sizes(ctypes.byref(kv), ctypes.byref(p)) == 0
    assert kv.value == ctypes.sizeof(N.OcKvDesc)
    assert p.value == ctypes.sizeof(N.OcDecodeParams)
    assert "gfx950" in N.version()


def test_invalid_arguments_return_status_and_message():
    """Validation runs on the host; a bad call returns OC_ERR_* and a message."""
    import ctypes
    from orthocache_gpu import _native as N
    p = N.OcDecodeParams()
    p.kv.head_dim = 128
    rc = N.lib().oc_decode(ctypes.byref(p), None)
    assert rc == N.OC_ERR_INVALID
    assert b"NULL" in N.lib().oc_last_error()
    p.kv.dtype, p.kv.head_dim, p.kv.k = N.OC_BF16, 96, 256
    assert N.lib().oc_decode(ctypes.byref(p), None) == N.OC_ERR_UNSUPPORTED
    assert b"head_dim" in N.lib().oc_last_error()
    with pytest.raises(N.OrthoCacheHIPError, match="oc_decode"):
        N.check("oc_decode", N.lib().oc_decode(ctypes.byref(p), None))


def test_gate_and_norm_cache_argument_checks():
    """The score-cache and decode-gate entry points validate on the host
    (no launch happens for these calls)."""
    import ctypes
    from orthocache_gpu import _native as N
    L = N.lib()
    kv = N.OcKvDesc()
    kv.k, kv.dtype, kv.head_dim, kv.num_rows, kv.num_tiles = 256, N.OC_BF16, 128, 2, 4
    kv.k_token_stride = 128
    assert L.oc_band_norms(ctypes.byref(kv), 0, 4, 40, 70, 256, 4, None, None) == N.OC_ERR_INVALID
    assert b"band" in L.oc_last_error()
    assert L.oc_band_norms(ctypes.byref(kv), 2, 3, 48, 64, 256, 4, None, None) == N.OC_ERR_INVALID
    assert b"tile range" in L.oc_last_error()
    assert L.oc_score_tile_range(ctypes.byref(kv), -1, 1, 0.0, 256, 256, None, None, 4, None) == N.OC_ERR_INVALID
    assert L.oc_decode_gate(None, N.OC_F32, 64, 2, 4, 64, 256, 8, 8, 8, 1.0, 0, 8, 256, 8, None,
                            None) == N.OC_ERR_INVALID
    assert L.oc_decode_gate(256, N.OC_F32, 64, 2, 4, 60, 256, 8, 8, 8, 1.0, N.OC_QNORM_WALSH_HIGH, 8, 256, 8,
                            None, None) == N.OC_ERR_INVALID
    assert b"low_band" in L.oc_last_error()
    assert L.oc_q_high_norms(256, N.OC_FP8_E4M3FN, 4, 64, 64, 8, 256, None) == N.OC_ERR_INVALID
    assert L.oc_apply_tile_mask(256, N.OC_F32, 4, 100, 100, None, 4, 2, 64, 1, None) == N.OC_ERR_INVALID


def test_hook_entry_point_argument_checks():
    """oc_prefill_attention, oc_row_norms, oc_kth_smallest and oc_group_gate
    validate on the host; none of these calls launches."""
    import ctypes
    from orthocache_gpu import _native as N
    L = N.lib()
    assert L.oc_prefill_params_bytes() == ctypes.sizeof(N.OcPrefillParams)
    p = N.OcPrefillParams()
    assert L.oc_prefill_attention(ctypes.byref(p), None) == N.OC_ERR_INVALID
    assert b"NULL" in L.oc_last_error()
    p.q = p.k = p.v = p.out = 256
    p.dtype, p.head_dim, p.batch, p.num_q_heads, p.num_kv_heads, p.q_len, p.kv_len = N.OC_BF16, 96, 1, 4, 2, 8, 64
    assert L.oc_prefill_attention(ctypes.byref(p), None) == N.OC_ERR_UNSUPPORTED
    assert b"head_dim" in L.oc_last_error()
    p.head_dim, p.dtype = 64, N.OC_FP8_E4M3FN
    assert L.oc_prefill_attention(ctypes.byref(p), None) == N.OC_ERR_UNSUPPORTED
    p.dtype, p.num_kv_heads = N.OC_F16, 3
    assert L.oc_prefill_attention(ctypes.byref(p), None) == N.OC_ERR_INVALID
    assert b"multiple" in L.oc_last_error()
    p.num_kv_heads, p.k_stride_s = 2, 65  # 130-byte token stride breaks the 16-byte loads
    assert L.oc_prefill_attention(ctypes.byref(p), None) == N.OC_ERR_INVALID
    assert b"16 bytes" in L.oc_last_error()
    p.k_stride_s, p.v_stride_s, p.q_stride_s = 64, 64, 64
    p.tile_mask, p.tile_mask_cols, p.kv_len = 256, 1, 200
    assert L.oc_prefill_attention(ctypes.byref(p), None) == N.OC_ERR_INVALID
    assert b"tile_mask" in L.oc_last_error()
    assert L.oc_row_norms(256, N.OC_F32, 1, 1, 4, 0, 0, 64, 60, 8, 256, None) == N.OC_ERR_INVALID
    assert b"low_band" in L.oc_last_error()
    assert L.oc_kth_smallest(256, 2, 5, 5, 5, 256, None) == N.OC_ERR_INVALID
    assert L.oc_kth_smallest(256, 2, 5, 4, 1, 256, None) == N.OC_ERR_INVALID
    assert L.oc_group_gate(256, 1, 2, 4, 7, 256, 0, 8, 4, 4, 1.0, 0, 256, 8, 4, None, None, None) == N.OC_ERR_INVALID
    assert L.oc_group_gate(256, 1, 2, 4, N.OC_GROUP_MAX, 256, 0, 8, 5, 4, 1.0, 0, 256, 8, 4, None, None,
                           None) == N.OC_ERR_INVALID


def test_spectra_argument_checks():
    import ctypes
    from orthocache_gpu import _native as N
    L = N.lib()
    assert L.oc_spectra_params_bytes() == ctypes.sizeof(N.OcSpectraParams)
    p = N.OcSpectraParams()
    assert L.oc_block_spectra(ctypes.byref(p), None) == N.OC_ERR_INVALID
    p.k, p.dtype, p.num_blocks, p.num_heads, p.head_dim, p.block_size = 256, N.OC_BF16, 2, 2, 64, 256
    p.k_token_stride, p.k_head_stride = 128, 64
    assert L.oc_block_spectra(ctypes.byref(p), None) == N.OC_ERR_UNSUPPORTED
    assert b"512" in L.oc_last_error()
    p.block_size, p.head_dim = 512, 12
    assert L.oc_block_spectra(ctypes.byref(p), None) == N.OC_ERR_UNSUPPORTED
    p.head_dim, p.max_bound = 64, 256
    assert L.oc_block_spectra(ctypes.byref(p), None) == N.OC_ERR_INVALID
    assert b"need q" in L.oc_last_error()
    assert L.oc_stream_compact(None, 4, 256, None, None) == N.OC_ERR_INVALID


def test_reference_assertion_messages():
    """test_fp8.py:128-158 and test_paged_eviction.py:139-159 of the reference."""
    from orthocache_gpu import (fused_orthocache_attention, fused_orthocache_attention_paged,
                                fused_orthocache_attention_v2, fused_orthocache_attention_v3_gqa)
    q = torch.randn(1, 128)
    keys = torch.randn(256, 128)
    with pytest.raises(AssertionError, match="head_dim.*must be a power of 2"):
        fused_orthocache_attention(torch.randn(1, 100), torch.randn(256, 100), torch.randn(256, 100), 5.0)
    with pytest.raises(AssertionError, match="tile_size.*must be a power of 2"):
        fused_orthocache_attention(q, keys, keys, zeta_max=5.0, tile_size=50)
    with pytest.raises(AssertionError, match="not divisible by tile_size"):
        fused_orthocache_attention(q, torch.randn(250, 128), torch.randn(250, 128), 5.0, tile_size=64)
    with pytest.raises(AssertionError, match="num_splits.*greater than 0"):
        fused_orthocache_attention_v2(torch.randn(2, 128), torch.randn(2, 256, 128), torch.randn(2, 256, 128),
                                      5.0, num_splits=0)
    with pytest.raises(AssertionError, match="num_query_heads"):
        fused_orthocache_attention_v3_gqa(torch.randn(16, 128), torch.randn(4, 256, 128),
                                          torch.randn(4, 256, 128), tau=1.0, num_query_groups=8)
    bt = torch.tensor([[0, 1]], dtype=torch.int32)
    with pytest.raises(AssertionError, match="head_dim.*power of 2"):
        fused_orthocache_attention_paged(torch.randn(1, 2, 63), torch.randn(4, 2, 32, 63),
                                         torch.randn(4, 2, 32, 63), bt, zeta_max=5.0)
    with pytest.raises(AssertionError, match="block_size.*power of 2"):
        fused_orthocache_attention_paged(torch.randn(1, 2, 64), torch.randn(4, 2, 31, 64),
                                         torch.randn(4, 2, 31, 64), bt, zeta_max=5.0)


def test_cpu_tensors_fail_loudly():
    """No CPU fallback: the product path refuses host tensors."""
    from orthocache_gpu import fused_orthocache_attention_v2, triton_fwht_eviction
    with pytest.raises(RuntimeError, match="GPU"):
        fused_orthocache_attention_v2(torch.randn(2, 128), torch.randn(2, 256, 128), torch.randn(2, 256, 128), 5.0)
    with pytest.raises(RuntimeError, match="GPU"):
        triton_fwht_eviction(torch.randn(256, 128), 5.0)


def test_pipeline_host_logic():
    from orthocache_gpu import BypassFlag, TelemetryLevel, format_bypass_reason, get_hardware_profile
    from orthocache_gpu.pipeline import _GPU_PROFILES, orthocache_forward
    assert _GPU_PROFILES["MI355X"].sm_count == 256
    if not torch.cuda.is_available():
        assert get_hardware_profile().name == "RTX 4060 Laptop"
    assert "crossover" in format_bypass_reason(BypassFlag.CROSSOVER_BYPASS, 100, 4096)
    # the reference's telemetry strings, order and separator (pipeline.py:87-117)
    assert format_bypass_reason(BypassFlag.NONE) == "no flags set"
    assert format_bypass_reason(BypassFlag.CROSSOVER_BYPASS, 100, 4096) == "seq_len_k=100 < crossover=4096"
    assert (format_bypass_reason(BypassFlag.CROSSOVER_BYPASS, 512, 2048, _GPU_PROFILES["MI355X"])
            == "seq_len_k=512 < crossover=2048 on MI355X (256 CUs, 8000 GB/s)")
    allf = BypassFlag(0xFF)
    assert format_bypass_reason(allf, 1, 2).split("; ") == [
        "seq_len_k=1 < crossover=2", "mode=dense (explicit)", "mode=triton_fused (God Kernel)",
        "full spectral eviction path", "all blocks evicted", "tau auto-computed (mean - 1σ)",
        "GPU auto-detected via bandwidth-ratio model"]
    assert format_bypass_reason(BypassFlag.PERFECT_EVICTION) == "no flags set"
    assert TelemetryLevel.SILENT < TelemetryLevel.FLAGS < TelemetryLevel.VERBOSE
    q = torch.randn(1, 2, 64)
    k = torch.randn(1024, 2, 64)
    with pytest.raises(RuntimeError, match="GPU"):  # no CPU fallback
        orthocache_forward(q, k, k, mode="compact")
    with pytest.raises(ValueError, match="Unknown mode"):
        orthocache_forward(q, k, k, mode="bogus")


def test_walsh_matrix_api():
    from orthocache_gpu import generate_walsh_matrix
    w = generate_walsh_matrix(64)
    assert torch.allclose(w @ w.T, torch.eye(64), atol=1e-6)
    assert torch.all(w[0] == 0.125)


def test_split_grouping_of_short_cached_decodes():
    """oc_decode_num_groups (host logic only): a cached decode whose splits
    alone fill the CUs (one split per workgroup) takes two splits per
    workgroup, which puts it on the per-wave-prologue kernel; partials asked
    for, a dense decode, or a caller's own grouping keep one split per
    group."""
    import ctypes
    from orthocache_gpu import _native as N
    lib = N.lib()

    def params(**kw):
        p = N.OcDecodeParams()
        p.kv.k, p.kv.v = 1 << 20, 1 << 21
        p.kv.dtype, p.kv.head_dim, p.kv.num_rows, p.kv.num_tiles = N.OC_BF16, 128, 32, 16
        p.kv.k_row_stride = p.kv.v_row_stride = 16 * 64 * 128
        p.kv.k_token_stride = p.kv.v_token_stride = 128
        p.q, p.q_dtype, p.G, p.q_row_stride = 1 << 22, N.OC_BF16, 1, 128
        p.gate, p.mode = N.OC_GATE_CS, N.OC_MODE_CACHED
        p.score_e_low, p.score_e_high, p.score_row_stride = 1 << 23, 1 << 24, 16
        p.num_splits, p.out_dtype, p.out = 4, N.OC_BF16, 1 << 25
        for k, v in kw.items():
            setattr(p, k, v)
        return p

    groups = lambda p: lib.oc_decode_num_groups(ctypes.byref(p))
    assert groups(params()) == 2                                   # 32 rows x 4 splits: two per workgroup
    assert groups(params(num_splits=8)) == 4
    assert groups(params(gate=N.OC_GATE_NONE, mode=N.OC_MODE_SINGLE_PASS)) == 4   # dense: one per group
    assert groups(params(mode=N.OC_MODE_SINGLE_PASS)) == 4         # single pass: one per group
    assert groups(params(splits_per_group=1)) == 4                 # the caller's grouping
    assert groups(params(partial_m=1 << 26, partial_l=1 << 27, partial_acc=1 << 28)) == 4
    assert groups(params(q=(1 << 22) + 2)) == 4                    # q rows not 16-byte pieces
    assert groups(params(num_splits=1)) == 1


def test_head_dim_32_and_256_routes():
    """oc_decode_num_groups (host logic only): head_dim 32 and 256 decodes
    of 16-bit K/V with q of K's type take the matrix-core kernels' split
    grouping (fewer groups than splits); fp8 K at head_dim 32, float32 K/V,
    another q type, q rows that are not 16-byte pieces, tiles other than 64
    tokens or the portable switch keep the portable kernels' one split per
    group."""
    import ctypes
    from orthocache_gpu import _native as N
    lib = N.lib()

    def params(d, **kw):
        p = N.OcDecodeParams()
        p.kv.k, p.kv.v = 1 << 20, 1 << 21
        p.kv.dtype, p.kv.head_dim, p.kv.num_rows, p.kv.num_tiles = N.OC_BF16, d, 32, 160
        p.kv.k_row_stride = p.kv.v_row_stride = 160 * 64 * d
        p.kv.k_token_stride = p.kv.v_token_stride = d
        p.q, p.q_dtype, p.G, p.q_row_stride = 1 << 22, N.OC_BF16, 1, d
        p.gate, p.mode = N.OC_GATE_CS, N.OC_MODE_CACHED
        p.score_e_low, p.score_e_high, p.score_row_stride = 1 << 23, 1 << 24, 160
        p.num_splits, p.out_dtype, p.out = 40, N.OC_BF16, 1 << 25
        for k, v in kw.items():
            if k.startswith("kv_"):
                setattr(p.kv, k[3:], v)
            else:
                setattr(p, k, v)
        return p

    groups = lambda p: lib.oc_decode_num_groups(ctypes.byref(p))
    for d in (32, 256):
        assert groups(params(d)) < 40, d                                     # matrix cores
        assert groups(params(d, kv_dtype=N.OC_F16, q_dtype=N.OC_F16)) < 40, d
        assert groups(params(d, portable=1)) == 40, d
        assert groups(params(d, q_dtype=N.OC_F32)) == 40, d                  # q not of K's type
        assert groups(params(d, kv_dtype=N.OC_F32, q_dtype=N.OC_F32)) == 40, d
        assert groups(params(d, q=(1 << 22) + 2)) == 40, d                    # q rows not 16-byte pieces
    assert groups(params(32, kv_dtype=N.OC_FP8_E4M3FN)) == 40                # fp8 K: portable at 32
    assert groups(params(256, kv_dtype=N.OC_FP8_E4M3FN)) < 40                # (matrix cores at 256)
    # head_dim 256 with G > 8: the general matrix-core kernel in chunks of 8
    # heads, except bf16 V beside fp8 K (per-wave-prologue kernel only)
    assert groups(params(256, G=8)) < 40 and groups(params(256, G=12)) < 40
    assert groups(params(256, G=8, kv_dtype=N.OC_FP8_E4M3FN, kv_v_dtype=N.OC_BF16)) < 40
    assert groups(params(256, G=12, kv_dtype=N.OC_FP8_E4M3FN, kv_v_dtype=N.OC_BF16)) == 40
    assert groups(params(32, kv_tile_size=32, kv_num_tiles=320, score_row_stride=320)) == 40
    assert groups(params(16)) == 40 and groups(params(512)) == 40            # portable head dims
