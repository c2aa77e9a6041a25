"""Register, LDS and scratch use of every compiled kernel (CPU).

Reads the AMDGPU metadata of the gfx950 code objects in the built
liborthocache_hip.so (orthocache_gpu.kernel_metadata; the counterpart of the
reference's print_kernel_metadata, triton_kernels/fwht_fused_prototype.py:
329-385) and holds the build to:
  * no scratch memory traffic in any kernel: no register spilled to memory
    (VGPR spills that the compiler places in AGPRs cost none and are
    allowed), checked in the disassembly of every kernel that carries a
    stack frame, and no frame at all in the kernels the bench times;
  * at most 256 registers per lane (VGPRs and AGPRs together: gfx950's
    unified file, which the metadata's vgpr_count already totals) for
    kernels of 8 or more waves per workgroup (two waves per SIMD), 512 for
    the rest, and at most the CU's 160 KiB of LDS per workgroup;
  * the headline decode kernel (bf16, head_dim 128, G = 4, contiguous rows,
    8 waves) at two waves per SIMD.
"""

import os

import pytest

from orthocache_gpu import kernel_metadata as KM

LIB = KM.library_path()
pytestmark = pytest.mark.skipif(not os.path.exists(LIB), reason="liborthocache_hip.so is not built")


@pytest.fixture(scope="module")
def rows():
    return KM.kernel_metadata(LIB)


def test_every_kernel_listed(rows):
    names = [r["name"] for r in rows]
    assert len(rows) > 300
    for k in ("decode_fast_kernel", "decode_kernel", "score_kernel", "prefill_kernel", "merge_kernel",
              "block_spectrum_kernel"):
        assert any(k in n for n in names), k


def test_no_scratch_traffic(rows):
    """No kernel reads or writes scratch memory.  A few SGPR-spill-heavy
    decode kernels carry a stack frame of 20-68 bytes that the register
    allocator reserved and then left unused (a spill slot emptied later);
    their disassembly must show no scratch instruction."""
    framed = [r for r in rows if r["scratch_bytes"]]
    assert len(framed) <= 24, [r["name"] for r in framed]
    if not framed:
        return
    counts = KM.scratch_instructions([r["symbol"] for r in framed], LIB)
    assert set(counts) == {r["symbol"] for r in framed}
    used = {s: n for s, n in counts.items() if n}
    assert not used, f"kernels with scratch traffic: {used}"


def test_hot_kernels_have_no_frame(rows):
    """The kernels the bench lines time: no stack frame at all."""
    hot = ["void oc::decode_fast_kernel<2, 128, 4, false, 8, 2>",   # BASELINE configs 2 and the metric
           "void oc::decode_fast_kernel<3, 128, 8, false, 8, 3>",   # config 4 (fp8, G = 8)
           "void oc::decode_fast_kernel<2, 128, 4, true, 4, 2>",    # config 3 (paged, flat layout)
           "void oc::decode_fast_kernel<1, 128, 1, false, 8, 1>",   # config 1 (float16, G = 1)
           "void oc::score_kernel<2, 128, false>", "oc::merge_kernel("]
    for h in hot:
        k = [r for r in rows if r["name"].startswith(h)]
        assert k, h
        assert all(r["scratch_bytes"] == 0 for r in k), h


def test_register_and_lds_budgets(rows):
    for r in rows:
        assert r["lds_bytes"] <= 160 * 1024, r["name"]
        regs = r["vgpr"]  # arch VGPRs + AGPRs (unified register file)
        assert r["agpr"] <= regs <= 512, r["name"]
        waves = max(1, r["max_workgroup"] // 64)
        if waves >= 8:  # two or more waves per SIMD
            assert regs <= 256, (r["name"], regs)


def test_headline_kernel(rows):
    k = [r for r in rows if r["name"].startswith("void oc::decode_fast_kernel<2, 128, 4, false, 8, 2>")]
    assert len(k) == 1
    r = k[0]
    assert r["vgpr"] <= 256 and r["scratch_bytes"] == 0 and r["max_workgroup"] == 512


def test_print_kernel_metadata(capsys):
    from orthocache_gpu.triton_kernels.fwht_fused_prototype import print_kernel_metadata
    got = print_kernel_metadata()
    out = capsys.readouterr().out
    assert got and all("score_kernel" in r["name"] for r in got)
    assert out.count("\n") == len(got)
    assert all(" scratch   0 B/lane" in line for line in out.splitlines())
