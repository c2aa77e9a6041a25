"""ctypes binding of liborthocache_hip.so (include/orthocache_hip.h).

The library is loaded from orthocache_gpu/_lib/ (built in-tree by
`make -C orthocache-gpu_amd`).  A missing library is an error: there is no
CPU or eager fallback behind the public API.
"""

from __future__ import annotations

import ctypes
import os
import threading

_LIB_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib")
LIB_PATH = os.path.join(_LIB_DIR, "liborthocache_hip.so")

# status codes
OC_OK = 0
OC_ERR_INVALID = 1
OC_ERR_UNSUPPORTED = 2
OC_ERR_HIP = 3
OC_ERR_WORKSPACE = 4

# element types
OC_F32, OC_F16, OC_BF16, OC_FP8_E4M3FN = 0, 1, 2, 3
# gates / modes / scale modes
OC_GATE_NONE, OC_GATE_ZETA, OC_GATE_CS, OC_GATE_MASK = 0, 1, 2, 3
OC_MODE_SINGLE_PASS, OC_MODE_CACHED = 0, 1
OC_KSCALE_NONE, OC_KSCALE_Q_FOLD, OC_KSCALE_TILE, OC_KSCALE_DEQUANT = 0, 1, 3, 4
OC_VSCALE_NONE, OC_VSCALE_TILE = 0, 1
# q norm of the decode gate
OC_QNORM_SPATIAL, OC_QNORM_WALSH_HIGH = 0, 1
OC_GROUP_MAX, OC_GROUP_MEDIAN = 0, 1

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64


class OcKvDesc(ctypes.Structure):
    _fields_ = [
        ("k", _p), ("v", _p),
        ("dtype", _i32), ("head_dim", _i32), ("num_rows", _i32), ("num_tiles", _i32),
        ("k_row_stride", _i64), ("k_token_stride", _i64),
        ("v_row_stride", _i64), ("v_token_stride", _i64),
        ("paged", _i32), ("block_size", _i32), ("num_kv_heads", _i32), ("rows_per_length", _i32),
        ("block_tables", _p), ("bt_stride", _i64), ("num_blocks", _i64),
        ("k_block_stride", _i64), ("k_head_stride", _i64),
        ("v_block_stride", _i64), ("v_head_stride", _i64),
        ("lengths", _p),
        ("k_scale_mode", _i32), ("k_scale", ctypes.c_float),
        ("k_scales", _p), ("k_scales_row_stride", _i64),
        ("v_scale_mode", _i32), ("num_tokens", _i32),
        ("v_scales", _p), ("v_scales_row_stride", _i64),
        ("error_flag", _p),
        ("v_dtype", _i32), ("tile_size", _i32),
    ]


class OcDecodeParams(ctypes.Structure):
    _fields_ = [
        ("kv", OcKvDesc),
        ("q", _p), ("q_dtype", _i32), ("G", _i32), ("q_row_stride", _i64),
        ("gate", _i32), ("mode", _i32), ("threshold", ctypes.c_double),
        ("score_e_low", _p), ("score_e_high", _p), ("score_row_stride", _i64),
        ("num_splits", _i32), ("splits_per_group", _i32), ("out_dtype", _i32), ("portable", _i32),
        ("out", _p), ("out_row_stride", _i64),
        ("keep_out", _p), ("keep_row_stride", _i64),
        ("split_counts", _p),
        ("partial_m", _p), ("partial_l", _p), ("partial_acc", _p),
        ("workspace", _p), ("workspace_bytes", ctypes.c_size_t),
        ("tile_mask", _p), ("tile_mask_row_stride", _i64),
    ]


class OcPrefillParams(ctypes.Structure):
    _fields_ = [
        ("q", _p), ("q_stride_b", _i64), ("q_stride_h", _i64), ("q_stride_s", _i64),
        ("k", _p), ("k_stride_b", _i64), ("k_stride_h", _i64), ("k_stride_s", _i64),
        ("v", _p), ("v_stride_b", _i64), ("v_stride_h", _i64), ("v_stride_s", _i64),
        ("out", _p), ("out_stride_b", _i64), ("out_stride_h", _i64), ("out_stride_s", _i64),
        ("dtype", _i32), ("batch", _i32), ("num_q_heads", _i32), ("num_kv_heads", _i32),
        ("q_len", _i32), ("kv_len", _i32), ("head_dim", _i32),
        ("tile_mask", _p), ("tile_mask_stride_b", _i64), ("tile_mask_stride_h", _i64),
        ("tile_mask_cols", _i32), ("scale", ctypes.c_float),
        ("entropy", _p),
        ("workspace", _p), ("workspace_bytes", ctypes.c_size_t),
    ]


class OcSpectraParams(ctypes.Structure):
    _fields_ = [
        ("k", _p), ("dtype", _i32), ("num_blocks", _i32), ("num_heads", _i32), ("head_dim", _i32),
        ("block_size", _i32), ("k_token_stride", _i64), ("k_head_stride", _i64),
        ("q", _p), ("q_dtype", _i32), ("q_len", _i32), ("q_token_stride", _i64), ("q_head_stride", _i64),
        ("e_low", _p), ("e_mid", _p), ("e_high", _p), ("zeta", _p), ("e_ac", _p), ("energy", _p),
        ("block_mean", _p), ("bounds", _p), ("max_bound", _p), ("q_norm_max", _p),
    ]


class OcHookDecodeParams(ctypes.Structure):
    _fields_ = [
        ("q", _p), ("q_row_stride", _i64), ("k", _p), ("v", _p),
        ("k_row_stride", _i64), ("k_token_stride", _i64), ("v_row_stride", _i64), ("v_token_stride", _i64),
        ("dtype", _i32), ("batch", _i32), ("num_kv_heads", _i32), ("G", _i32), ("head_dim", _i32), ("kv_len", _i32),
        ("k_norms", _p), ("k_norms_stride", _i64), ("tau_norm", ctypes.c_double),
        ("low_band", _i32), ("num_splits", _i32),
        ("out", _p), ("out_row_stride", _i64), ("gate_stats", _p),
        ("workspace", _p), ("workspace_bytes", ctypes.c_size_t),
    ]


class OcDeviceInfo(ctypes.Structure):
    _fields_ = [
        ("arch", ctypes.c_char * 64), ("name", ctypes.c_char * 128), ("compute_units", _i32), ("wave_size", _i32),
        ("memory_clock_khz", _i32), ("memory_bus_bits", _i32), ("lds_per_cu_bytes", _i64),
        ("total_memory_bytes", _i64),
    ]


# every function declared in include/orthocache_hip.h: name -> (restype, argtypes)
SIGNATURES = {
    "oc_score_tiles": (_i32, [ctypes.POINTER(OcKvDesc), ctypes.c_double, _p, _p, _p, _p, _i64, _p]),
    "oc_fwht_tiles": (_i32, [ctypes.POINTER(OcKvDesc), _p, _p]),
    "oc_score_tile_range": (_i32, [ctypes.POINTER(OcKvDesc), _i32, _i32, ctypes.c_double, _p, _p, _p, _p, _i64,
                                   _p]),
    "oc_band_norms": (_i32, [ctypes.POINTER(OcKvDesc), _i32, _i32, _i32, _i32, _p, _i64, _p, _p]),
    "oc_decode_gate": (_i32, [_p, _i32, _i64, _i32, _i32, _i32, _p, _i64, _i32, _i32, ctypes.c_double, _i32, _i32,
                              _p, _i64, _p, _p]),
    "oc_q_high_norms": (_i32, [_p, _i32, _i64, _i32, _i64, _i32, _p, _p]),
    "oc_apply_tile_mask": (_i32, [_p, _i32, _i32, _i64, _i64, _p, _i64, _i32, _i32, _i32, _p]),
    "oc_tile_mask_from_blocks": (_i32, [_p, _p, _i32, _i32, _i32, _p, _p, _p]),
    "oc_row_norms": (_i32, [_p, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i32, _i32, _p, _p]),
    "oc_kth_smallest": (_i32, [_p, _i64, _i64, _i64, _i64, _p, _p]),
    "oc_group_gate": (_i32, [_p, _i32, _i32, _i32, _i32, _p, _i64, _i64, _i32, _i32, ctypes.c_double, _i32, _p,
                             _i64, _i64, _p, _p, _p]),
    "oc_prefill_attention": (_i32, [ctypes.POINTER(OcPrefillParams), _p]),
    "oc_prefill_workspace_size": (ctypes.c_size_t, [ctypes.POINTER(OcPrefillParams)]),
    "oc_prefill_params_bytes": (ctypes.c_size_t, []),
    "oc_block_spectra": (_i32, [ctypes.POINTER(OcSpectraParams), _p]),
    "oc_spectra_params_bytes": (ctypes.c_size_t, []),
    "oc_stream_compact": (_i32, [_p, _i32, _p, _p, _p]),
    "oc_compact_gate": (_i32, [_p, _p, _p, _p, _i32, _i32, _i32, ctypes.c_double, _i32, ctypes.c_double,
                               ctypes.c_double, _i32, _p, _p, _p, _p]),
    "oc_block_regimes": (_i32, [_p, _i32, _i32, _p, _i32, _i32, ctypes.c_double, _p, _i32, _p, _i32,
                                ctypes.c_double, _p, _p, _p, _p, _p, _p]),
    "oc_decode_workspace_size": (ctypes.c_size_t, [ctypes.POINTER(OcDecodeParams)]),
    "oc_decode_num_groups": (_i32, [ctypes.POINTER(OcDecodeParams)]),
    "oc_decode": (_i32, [ctypes.POINTER(OcDecodeParams), _p]),
    "oc_decode_static": (_i32, [ctypes.POINTER(OcDecodeParams), _p]),
    "oc_decode_static_scratch_bytes": (ctypes.c_size_t, []),
    "oc_hook_decode": (_i32, [ctypes.POINTER(OcHookDecodeParams), _p]),
    "oc_hook_decode_workspace_size": (ctypes.c_size_t, [ctypes.POINTER(OcHookDecodeParams)]),
    "oc_hook_decode_params_bytes": (ctypes.c_size_t, []),
    "oc_lse_merge": (_i32, [_p, _p, _p, _i32, _i32, _i32, _p, _i32, _i64, _p]),
    "oc_dequant_fp8": (_i32, [_p, _i64, ctypes.c_float, _i32, _p, _p]),
    "oc_hbm_read_probe": (_i32, [_p, ctypes.c_size_t, _p, _i32, _p]),
    "oc_hbm_gather_probe": (_i32, [_p, _p, _i64, _i32, _i32, _p, _i32, _p]),
    "oc_abi_sizes": (_i32, [ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)]),
    "oc_device_cu_count": (_i32, [ctypes.POINTER(_i32)]),
    "oc_device_props": (_i32, [ctypes.POINTER(OcDeviceInfo)]),
    "oc_version": (ctypes.c_char_p, []),
    "oc_last_error": (ctypes.c_char_p, []),
}


class OrthoCacheHIPError(RuntimeError):
    """A liborthocache_hip call returned a non-zero status."""

    def __init__(self, func: str, code: int, message: str):
        super().__init__(f"{func} failed (status {code}): {message}")
        self.func, self.code, self.message = func, code, message


_lock = threading.Lock()
_lib = None


def lib():
    """The loaded library (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"orthocache_gpu: native library {LIB_PATH} is missing; build it with "
                    "`make -C orthocache-gpu_amd` (or __graft_entry__.build()). There is no "
                    "CPU fallback.")
            handle = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype, fn.argtypes = res, args
            kv_sz, p_sz = ctypes.c_size_t(), ctypes.c_size_t()
            handle.oc_abi_sizes(ctypes.byref(kv_sz), ctypes.byref(p_sz))
            if kv_sz.value != ctypes.sizeof(OcKvDesc) or p_sz.value != ctypes.sizeof(OcDecodeParams):
                raise RuntimeError(
                    "orthocache_gpu: struct layout mismatch between the binding and "
                    f"{LIB_PATH} ({kv_sz.value}/{p_sz.value} vs "
                    f"{ctypes.sizeof(OcKvDesc)}/{ctypes.sizeof(OcDecodeParams)} bytes)")
            for fn, st in (("oc_prefill_params_bytes", OcPrefillParams), ("oc_spectra_params_bytes", OcSpectraParams),
                           ("oc_hook_decode_params_bytes", OcHookDecodeParams)):
                if getattr(handle, fn)() != ctypes.sizeof(st):
                    raise RuntimeError(f"orthocache_gpu: {st.__name__} layout mismatch between the binding and "
                                       f"{LIB_PATH}")
            _lib = handle
    return _lib


def check(func: str, rc: int) -> None:
    if rc != OC_OK:
        msg = lib().oc_last_error()
        raise OrthoCacheHIPError(func, rc, msg.decode() if msg else "")


def version() -> str:
    return lib().oc_version().decode()


def device_cu_count() -> int:
    n = _i32()
    check("oc_device_cu_count", lib().oc_device_cu_count(ctypes.byref(n)))
    return int(n.value)


def device_props() -> OcDeviceInfo:
    """hipDeviceProp_t fields of the current device (oc_device_props)."""
    info = OcDeviceInfo()
    check("oc_device_props", lib().oc_device_props(ctypes.byref(info)))
    return info
