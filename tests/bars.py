"""Output bars of the GPU parity tests, and the record of what each check
achieved.

The north-star bars are max-abs errors: 1e-5 (float32), 2e-3 (float16 /
bfloat16), 2e-2 (fp8 K/V).  An output stored in a 16-bit type carries its
own rounding: the reference returns out.to(q.dtype) as well, so a value v
is off its float32 result by up to half a unit in the last place of v in
that type.  assert_out therefore checks, element by element,

    |got - ref| <= bar + h(ref)     ref = the unrounded float32/64 oracle,
                                    h = half an output ulp of ref
    |got - ref| <= bar + 2 h(ref)   ref = a stored (already rounded) output
                                    of the reference (golden vectors)

and records the achieved max-abs error beside the plain bar.  h is at
most 2^-9 |ref| in bfloat16 and 2^-12 |ref| in float16, so for outputs
below 0.5 in magnitude (nearly all decode outputs: averages of many value
rows) the check is the plain bar; the terminal summary lists the worst
error per bar and every check whose plain max-abs error exceeded its bar.
"""

from __future__ import annotations

import json
import os

import numpy as np
import torch

TOL = {"f32": 1e-5, "f16": 2e-3, "bf16": 2e-3, "fp8": 2e-2}
_OUT_NAMES = {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16"}
RECORDS: list = []


def half_ulp(ref: np.ndarray, out_dtype: str) -> np.ndarray:
    """Half a unit in the last place of |ref| in out_dtype (0 for float32,
    whose own rounding is inside the 1e-5 bar)."""
    a = np.abs(np.asarray(ref, dtype=np.float64))
    if out_dtype == "f32":
        return np.zeros_like(a)
    mant = {"bf16": 8, "f16": 11}[out_dtype]
    min_exp = {"bf16": -126, "f16": -14}[out_dtype]
    e = np.floor(np.log2(np.where(a > 0, a, 1.0)))
    e = np.maximum(e, min_exp)
    return np.where(a > 0, 2.0 ** (e - mant), 2.0 ** (min_exp - mant))


def assert_out(got, ref, bar: str, what: str = "", *, ref_rounded: bool = False, out_dtype: str | None = None):
    """got: device tensor or array; ref: the oracle (unrounded) or, with
    ref_rounded, the reference's own stored output; bar
    ('f32', 'f16', 'bf16' or 'fp8')."""
    if isinstance(got, torch.Tensor):
        if out_dtype is None:
            out_dtype = _OUT_NAMES[got.dtype]
        got = got.detach().double().cpu().numpy()
    if out_dtype is None:
        out_dtype = "f32"
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64).reshape(got.shape)
    err = np.abs(got - ref)
    tol = TOL[bar] + (2.0 if ref_rounded else 1.0) * half_ulp(ref, out_dtype)
    worst = float(np.nanmax(err)) if err.size else 0.0
    RECORDS.append({"check": what, "bar": bar, "out": out_dtype, "max_abs": worst, "bar_value": TOL[bar],
                    "vs": "reference output" if ref_rounded else "oracle", "max_ref": float(np.abs(ref).max())
                    if ref.size else 0.0})
    bad = ~(err <= tol)
    assert not bad.any(), (f"{what}: max err {worst:.3g} (bar {TOL[bar]:g} + output rounding) at "
                           f"{np.argwhere(bad)[:4].tolist()}")


def summary_lines() -> list:
    if not RECORDS:
        return []
    lines = ["output parity: achieved max-abs error per north-star bar (plain max-abs, no rounding slack)"]
    for bar in ("f32", "f16", "bf16", "fp8"):
        rs = [r for r in RECORDS if r["bar"] == bar]
        if not rs:
            continue
        w = max(rs, key=lambda r: r["max_abs"])
        over = [r for r in rs if r["max_abs"] > r["bar_value"]]
        lines.append(f"  bar {bar} ({TOL[bar]:g}): {len(rs)} checks, worst {w['max_abs']:.3g} "
                     f"({w['check']}, |out| <= {w['max_ref']:.3g}), over the plain bar: {len(over)}")
        for r in over:
            lines.append(f"    over: {r['check']} ({r['out']} out, |out| <= {r['max_ref']:.3g}): {r['max_abs']:.3g}")
    path = os.environ.get("OC_PARITY_REPORT")
    if path:
        with open(path, "w") as f:
            json.dump(RECORDS, f, indent=0)
    return lines
