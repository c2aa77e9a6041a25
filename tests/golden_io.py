"""Loader for the golden vectors written by tests/golden/make_golden.py."""

import json
import os

import numpy as np

GOLDEN_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _fp8_table():
    from oracle.orthocache_oracle import fp8_e4m3fn_table
    return fp8_e4m3fn_table()


def decode(arr: np.ndarray, dtype: str) -> np.ndarray:
    """Stored bits -> float32 values (exact)."""
    if dtype == "f32":
        return arr.astype(np.float32)
    if dtype == "f16":
        return arr.view(np.float16).astype(np.float32)
    if dtype == "bf16":
        return (arr.astype(np.uint32) << 16).view(np.float32)
    if dtype == "fp8":
        return _fp8_table()[arr]
    if dtype == "i32":
        return arr
    if dtype == "bool":
        return arr.astype(bool)
    raise ValueError(dtype)


def load(name: str):
    """Returns (raw arrays, decoded float arrays, dtypes, meta, params, reference_function)."""
    with open(os.path.join(GOLDEN_DIR, name + ".json")) as f:
        info = json.load(f)
    z = np.load(os.path.join(GOLDEN_DIR, name + ".npz"))
    raw = {k: z[k] for k in z.files}
    dec = {k: decode(raw[k], info["dtypes"][k]) for k in raw}
    meta = {}
    for k, v in info["meta"].items():
        if isinstance(v, dict) and "npz" in v:
            a = np.load(os.path.join(GOLDEN_DIR, v["npz"]))["a"]
            meta[k] = decode(a, v["dtype"])
        else:
            meta[k] = v
    return raw, dec, info["dtypes"], meta, info["params"], info["reference_function"]


def cases():
    with open(os.path.join(GOLDEN_DIR, "MANIFEST.json")) as f:
        return json.load(f)["cases"]
