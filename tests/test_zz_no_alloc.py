"""GPU test of oc_decode_static, the decode entry point that allocates
nothing (split partials and merge counters in the library's static device
scratch), called through the C ABI: its keep flags must equal oc_decode's
and its outputs agree with them to the north-star bar, on two
calls in a row with the second one smaller, for the contiguous cached
decode, the flat layout (rows of different lengths over a paged pool) and
the dense decode; a call whose partials exceed the scratch is refused
before anything is launched."""

import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import orthocache_gpu._native as N
    N.lib()
    yield


def _params(kv, q, G, gate, mode, tau, scores, out, keep, P):
    from orthocache_gpu import _native as N
    p = N.OcDecodeParams()
    p.kv = kv.struct()
    p.q = q.data_ptr()
    p.q_dtype = N.OC_BF16
    p.G = G
    p.q_row_stride = q.stride(0)
    p.gate, p.mode, p.threshold = gate, mode, float(tau)
    if scores is not None:
        p.score_e_low, p.score_e_high = scores.e_low.data_ptr(), scores.e_high.data_ptr()
        p.score_row_stride = scores.e_high.stride(0)
    p.num_splits = P
    p.out_dtype = N.OC_BF16
    p.out, p.out_row_stride = out.data_ptr(), out.stride(0)
    p.keep_out, p.keep_row_stride = keep.data_ptr(), keep.stride(0)
    return p


def _run_both(kv, q, G, gate, mode, tau, scores):
    """(out, keep) of oc_decode with a fresh zeroed workspace and of
    oc_decode_static, on the same inputs."""
    from orthocache_gpu import _launch as X
    from orthocache_gpu import _native as N
    lib = N.lib()
    stream = ctypes.c_void_p(X.current_stream(q.device))
    P = X.auto_num_splits(kv.num_tiles, q.device)
    res = []
    for static in (False, True):
        out = torch.full((q.shape[0], q.shape[1]), float("nan"), dtype=torch.bfloat16, device=DEV)
        keep = torch.full((kv.num_rows, kv.num_tiles), 7, dtype=torch.uint8, device=DEV)
        p = _params(kv, q, G, gate, mode, tau, scores, out, keep, P)
        if static:
            rc = lib.oc_decode_static(ctypes.byref(p), stream)
            N.check("oc_decode_static", rc)
        else:
            need = lib.oc_decode_workspace_size(ctypes.byref(p))
            ws = torch.zeros(max(need, 1), dtype=torch.uint8, device=DEV)
            p.workspace, p.workspace_bytes = ws.data_ptr(), ws.numel()
            N.check("oc_decode", lib.oc_decode(ctypes.byref(p), stream))
        torch.cuda.synchronize()
        res.append((out.cpu(), keep.cpu()))
    return res


def _assert_same(res, what):
    """Keep flags bit for bit; outputs to the bfloat16 bar: the cached
    decode's waves draw tiles from an LDS counter, so which wave sums which
    tiles (and the float32 summation order) varies from call to call, in
    oc_decode as much as between the two entry points."""
    from tests.bars import assert_out
    (o0, k0), (o1, k1) = res
    assert not torch.isnan(o0.float()).any(), f"{what}: oc_decode left outputs unwritten"
    assert not torch.isnan(o1.float()).any(), f"{what}: oc_decode_static left outputs unwritten"
    assert_out(o1, o0.float().numpy(), "bf16", f"static vs workspace {what}", ref_rounded=True)
    if (k0 != 7).any():
        assert torch.equal(k0, k1), f"{what}: keep flags differ"


@pytest.mark.parametrize("rows,tiles", [(16, 512), (6, 200)])
def test_static_cached_equals_workspace_twice(rows, tiles):
    """Two rounds: the larger call first, then a smaller one (the scratch
    keeps the first call's contents)."""
    from orthocache_gpu import _native as N
    from orthocache_gpu.triton_kernels.fwht_fused_prototype import score_tiles
    from orthocache_gpu.workloads import calibrate_tau, make_kv, make_q
    from orthocache_gpu import _launch as X
    for it, (r, t) in enumerate(((rows, tiles), (max(1, rows // 2), max(1, tiles // 3)))):
        wl = make_kv(r, t * 64, 128, dtype=torch.bfloat16, device=DEV, seed=11 + it)
        q = make_q(r, 4, 128, dtype=torch.bfloat16, device=DEV, seed=12 + it)
        sc = score_tiles(wl.keys)
        tau = calibrate_tau(sc.e_high, q, 4)
        kv = X.rows_layout(wl.keys, wl.values)
        print(f"cached rows={r} tiles={t} call {it}", flush=True)
        res = _run_both(kv, q, 4, N.OC_GATE_CS, N.OC_MODE_CACHED, tau, sc)
        _assert_same(res, f"cached {r}x{t}")
        print(f"dense rows={r} tiles={t} call {it}", flush=True)
        res = _run_both(kv, q, 4, N.OC_GATE_NONE, N.OC_MODE_SINGLE_PASS, 0.0, None)
        _assert_same(res, f"dense {r}x{t}")


def test_static_flat_paged_equals_workspace_twice():
    """Rows of different lengths over a shuffled page pool (flat workgroup
    layout: one partial per slot), a long batch then a short one."""
    from orthocache_gpu import _launch as X
    from orthocache_gpu import _native as N
    from orthocache_gpu.triton_kernels.paged_eviction import score_paged_tiles
    from orthocache_gpu.workloads import calibrate_tau, make_kv, make_q, paged_pool
    hkv, G, bs = 2, 4, 16
    for it, lens in enumerate(([4096, 960, 2112, 64], [640, 128])):
        B = len(lens)
        s_max = max(lens)
        wl = make_kv(B * hkv, s_max, 128, noise_frac=0.4, dtype=torch.bfloat16, device=DEV, seed=40 + it)
        kc, vc, bt = paged_pool(wl.keys, wl.values, hkv, bs, lens, seed=41 + it)
        lens_t = torch.tensor(lens, dtype=torch.int32, device=DEV)
        sc = score_paged_tiles(kc, bt, context_lens=lens_t)
        kv = X.paged_layout(kc, vc, bt, s_max // 64)
        kv.lengths = lens_t
        q = make_q(B * hkv, G, 128, dtype=torch.bfloat16, device=DEV, seed=42 + it)
        live = torch.arange(sc.e_high.shape[1], device=DEV)[None, :] < \
            torch.tensor([n // 64 for n in lens for _ in range(hkv)], device=DEV)[:, None]
        tau = calibrate_tau(sc.e_high, q, G, live=live)
        print(f"paged flat lens={lens} call {it}", flush=True)
        res = _run_both(kv, q, G, N.OC_GATE_CS, N.OC_MODE_CACHED, tau, sc)
        _assert_same(res, f"paged {lens}")


def test_static_refuses_oversized_request():
    """512 rows x 64 heads x 1 split of (128 + 2) floats is 17 MB of partials,
    more than the 16 MiB scratch: refused with OC_ERR_WORKSPACE before any
    launch, and the library keeps working afterwards."""
    from orthocache_gpu import _launch as X
    from orthocache_gpu import _native as N
    lib = N.lib()
    assert lib.oc_decode_static_scratch_bytes() == 16 << 20
    rows, G = 512, 64
    k = torch.zeros((rows, 64, 128), dtype=torch.bfloat16, device=DEV)
    q = torch.zeros((rows * G, 128), dtype=torch.bfloat16, device=DEV)
    out = torch.zeros((rows * G, 128), dtype=torch.bfloat16, device=DEV)
    keep = torch.zeros((rows, 1), dtype=torch.uint8, device=DEV)
    kv = X.rows_layout(k, k)
    p = _params(kv, q, G, N.OC_GATE_NONE, N.OC_MODE_SINGLE_PASS, 0.0, None, out, keep, 1)
    assert lib.oc_decode_workspace_size(ctypes.byref(p)) > (16 << 20)
    rc = lib.oc_decode_static(ctypes.byref(p), ctypes.c_void_p(X.current_stream(q.device)))
    assert rc == N.OC_ERR_WORKSPACE
    assert b"static scratch" in lib.oc_last_error()
    # a call that fits still runs afterwards
    q1 = torch.ones((2 * 4, 128), dtype=torch.bfloat16, device=DEV)
    k1 = torch.ones((2, 128, 128), dtype=torch.bfloat16, device=DEV)
    res = _run_both(X.rows_layout(k1, k1), q1, 4, N.OC_GATE_NONE, N.OC_MODE_SINGLE_PASS, 0.0, None)
    _assert_same(res, "ones")
    assert np.allclose(res[1][0].float().numpy(), 1.0)
