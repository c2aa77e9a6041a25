"""Write the golden vectors of the paths around the decode (score cache,
decode gate, mask-given attention, compact pipeline, eviction regimes,
model hook) from the reference's own CPU code.

Run in the development container only (the reference tree is not present on
the GPU box):

    python tests/golden/make_golden_8f.py /root/reference

It imports the reference's CPU entry points in a process whose sys.path
holds only the reference tree, feeds them small seeded inputs and stores
inputs and outputs as data (npz + json) beside the other golden vectors.
Which reference function produced each case is recorded in its json:

* _pytorch_decode_gate            (triton_kernels/decode_gate.py:248-295),
  with tight=True (Walsh-subspace q norm) and tight=False (spatial norm)
* SpectralNormCache.populate_from_keys / update_prefill (norm_cache.py:58-117)
* _pytorch_block_sparse_attention (triton_kernels/sparse_attention.py:144-203)
* _pytorch_indirect_attention     (triton_kernels/indirect_attention.py:136-197)
* orthocache_forward(mode='compact') on CPU (pipeline.py:312-555), auto and
  given tau
* compute_block_beta + classify_eviction (perfect_eviction.py:75-186)
* OrthoCache_GQA_Attention prefill then decode, with the residual and the
  entropy governor (eval/perplexity_eval.py:239-689)

These pin the decisions the restated oracle makes for these paths: the gate
thresholds (tau * 64 * d), the q-norm forms, the median and max group
reductions, the auto-tau statistics, the regime split and the hook's
statistics, on the reference's own float32 bits.
"""

import importlib.util
import json
import os
import sys


def main():
    ref_root = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    sys.path[:] = [p for p in sys.path if "orthocache-gpu_amd" not in p and os.path.abspath(p) !=
                   os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))]
    sys.path.insert(0, os.path.join(ref_root, "src"))
    import numpy as np
    import torch

    torch.set_num_threads(1)
    try:
        torch.set_flush_denormal(True)
    except ValueError:
        pass

    from orthocache_gpu.norm_cache import SpectralNormCache
    from orthocache_gpu.perfect_eviction import classify_eviction, compute_block_beta
    from orthocache_gpu.pipeline import orthocache_forward
    from orthocache_gpu.triton_kernels.decode_gate import _pytorch_decode_gate
    from orthocache_gpu.triton_kernels.fwht_fused_prototype import generate_walsh_matrix
    from orthocache_gpu.triton_kernels.indirect_attention import _pytorch_indirect_attention
    from orthocache_gpu.triton_kernels.sparse_attention import _pytorch_block_sparse_attention
    spec = importlib.util.spec_from_file_location("ref_perplexity_eval",
                                                  os.path.join(ref_root, "eval", "perplexity_eval.py"))
    pe = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(pe)

    out_dir = os.path.dirname(os.path.abspath(__file__))
    W = generate_walsh_matrix(64)

    def raw(t):
        t = t.detach().cpu().contiguous()
        if t.dtype == torch.float32:
            return t.numpy(), "f32"
        if t.dtype == torch.float16:
            return t.view(torch.int16).numpy().view(np.uint16), "f16"
        if t.dtype == torch.bfloat16:
            return t.view(torch.int16).numpy().view(np.uint16), "bf16"
        if t.dtype == torch.int32:
            return t.numpy(), "i32"
        if t.dtype == torch.int64:
            return t.numpy().astype(np.int32), "i32"
        if t.dtype == torch.bool:
            return t.numpy().astype(np.uint8), "bool"
        raise TypeError(t.dtype)

    names = []

    def save(name, fn_ref, arrays, meta, params):
        npz, dtypes = {}, {}
        for k, v in arrays.items():
            npz[k], dtypes[k] = raw(v)
        np.savez_compressed(os.path.join(out_dir, name + ".npz"), **npz)
        with open(os.path.join(out_dir, name + ".json"), "w") as f:
            json.dump({"reference_function": fn_ref, "params": params, "dtypes": dtypes, "meta": meta}, f,
                      indent=1, sort_keys=True)
        names.append(name)

    def mixed_tiles(g, n_tiles, d, noise_every=2):
        """smooth tiles W @ C (rows 1..4 of C) + 0.05 N(0, 1); noise tiles
        W @ C (rows 32..63)"""
        tiles = []
        for i in range(n_tiles):
            c = torch.zeros(64, d)
            if i % noise_every == 1:
                c[32:64] = torch.randn(32, d, generator=g)
                tiles.append(W @ c)
            else:
                c[1:5] = torch.randn(4, d, generator=g)
                tiles.append(W @ c + 0.05 * torch.randn(64, d, generator=g))
        return torch.cat(tiles)

    def gap_threshold(values):
        """a threshold in the middle of the widest gap between sorted values"""
        v = np.sort(np.asarray(values, dtype=np.float64).ravel())
        v = v[np.isfinite(v)]
        i = int(np.argmax(np.diff(v)))
        return float((v[i] + v[i + 1]) / 2)

    # 1. the O(1) decode gate: spatial and Walsh-subspace q norms, G = 4
    g = torch.Generator().manual_seed(801)
    hkv, G, d, max_tiles, n_tiles = 3, 4, 128, 12, 9
    q = torch.randn(hkv * G, d, generator=g)
    q[1::G] *= 0.2
    nc = torch.rand(hkv, max_tiles, generator=g) * 40.0
    for tight in (False, True):
        # a tau between two of the bounds, so the gate both keeps and evicts
        _, qmax = _pytorch_decode_gate(q, nc, 0.0, n_tiles, G, tight=tight)
        tau = gap_threshold((qmax[:, None] * nc[:, :n_tiles]).numpy()) / (64.0 * d)
        mask, q_norms = _pytorch_decode_gate(q, nc, tau, n_tiles, G, tight=tight)
        save("gate_%s" % ("high" if tight else "spatial"),
             "decode_gate.py:248-295 _pytorch_decode_gate (tight=%s)" % tight,
             {"q": q, "norm_cache": nc, "mask": mask, "q_norms": q_norms}, {},
             {"tau": tau, "num_tiles": n_tiles, "G": G, "tile_size": 64, "low_band": 8})

    # 2. the norm cache: bulk population from keys (a partial tail tile is
    #    skipped), then one tile rewritten through update_prefill
    g = torch.Generator().manual_seed(802)
    hkv, d = 3, 64
    keys = torch.stack([torch.cat([mixed_tiles(g, 5, d), torch.randn(20, d, generator=g)]) for _ in range(hkv)])
    cache = SpectralNormCache(hkv, 8, torch.device("cpu"))
    cache.populate_from_keys(keys, W, 64, 48, 64)
    bulk = cache.cache.clone()
    valid = cache.valid_tiles.clone()
    tile = torch.randn(64, d, generator=g) * 3.0
    cache.update_prefill(1, 6, tile, W, 48, 64)
    save("norm_cache", "norm_cache.py:58-117 SpectralNormCache.populate_from_keys + update_prefill",
         {"keys": keys, "bulk": bulk, "valid_tiles": valid, "tile": tile, "after": cache.cache,
          "valid_after": cache.valid_tiles}, {}, {"band": [48, 64], "max_tiles": 8, "update": [1, 6]})

    # 3. block-sparse and indirect attention on the same inputs, float32
    #    with 64-token blocks and bfloat16 with 512-token blocks
    for dt_name, dt, bs, nb in (("f32", torch.float32, 64, 12), ("bf16", torch.bfloat16, 512, 6)):
        g = torch.Generator().manual_seed(803 + bs)
        d = 64
        q = torch.randn(1, d, generator=g).to(dt)
        k = torch.randn(nb * bs, d, generator=g).to(dt)
        v = torch.randn(nb * bs, d, generator=g).to(dt)
        bm = torch.rand(nb, generator=g) < 0.5
        bm[0] = True
        out_bs = _pytorch_block_sparse_attention(q, k, v, bm, bs)
        idx = torch.randperm(nb, generator=g)[:5].to(torch.int32)
        out_ind = _pytorch_indirect_attention(q, k, v, idx, 4, bs)
        save("sparse_%s" % dt_name, "sparse_attention.py:144-203 _pytorch_block_sparse_attention + "
             "indirect_attention.py:136-197 _pytorch_indirect_attention",
             {"q": q, "keys": k, "values": v, "block_mask": bm, "out_block_sparse": out_bs, "active_indices": idx,
              "out_indirect": out_ind}, {}, {"block_size": bs, "num_active": 4})

    # 4. orthocache_forward(mode='compact') on CPU: 8 blocks of 512 tokens, 2
    #    heads, d 64, bfloat16 caches, smooth and noise blocks; auto and a
    #    given tau on the same inputs
    g = torch.Generator().manual_seed(804)
    nb, H, d = 8, 2, 64
    i = torch.arange(512)
    x = i[:, None] & i[None, :]
    pc = torch.zeros_like(x)
    for b in range(9):
        pc += (x >> b) & 1
    w512 = (1.0 - 2.0 * (pc % 2).float()) / 512 ** 0.5
    k = torch.zeros(nb * 512, H, d)
    for b in range(nb):
        for h in range(H):
            c = torch.zeros(512, d)
            if b in (2, 5, 6):
                c[256:] = torch.randn(256, d, generator=g)
            else:
                c[0] = torch.randn(d, generator=g)
                c[1:5] = 4 * torch.randn(4, d, generator=g)
            k[512 * b:512 * (b + 1), h] = w512 @ c + 0.05 * torch.randn(512, d, generator=g)
    k = k.to(torch.bfloat16)
    v = torch.randn(nb * 512, H, d, generator=g).to(torch.bfloat16)
    q = torch.randn(2, H, d, generator=g).to(torch.bfloat16)
    arrays, meta = {"q": q, "keys": k, "values": v}, {}
    for tau_name, tau in (("auto", None), ("given", 9.0)):
        out, m = orthocache_forward(q, k, v, block_size=512, zeta_max=5.0, tau=tau, mode="compact")
        arrays["out_" + tau_name] = out
        meta[tau_name] = {kk: vv for kk, vv in m.items() if isinstance(vv, (int, float, bool, str)) and
                          not kk.endswith("_ms")}
    save("compact", "pipeline.py:312-555 orthocache_forward(mode='compact') (CPU)", arrays, meta,
         {"tau_given": 9.0, "zeta_max": 5.0, "block_size": 512})

    # 4b. the same pipeline in float32 on 4 blocks: the reference's CPU
    #     profile bypasses contexts under 4096 tokens, so its cached profile
    #     is replaced by one with a 1024-token crossover for this call
    import dataclasses
    import orthocache_gpu.pipeline as ref_pipeline
    ref_pipeline._cached_profile = dataclasses.replace(ref_pipeline._REFERENCE_PROFILE, crossover_seq_len=1024)
    nb = 4
    k4 = torch.cat([k[:512 * 2], k[512 * 5:512 * 7]]).float()  # two smooth and two noise blocks
    v4 = torch.randn(nb * 512, H, d, generator=g)
    q4 = torch.randn(3, H, d, generator=g)
    arrays, meta = {"q": q4, "keys": k4, "values": v4}, {}
    for tau_name, tau in (("auto", None), ("given", 7.5)):
        out, m = orthocache_forward(q4, k4, v4, block_size=512, zeta_max=5.0, tau=tau, mode="compact")
        arrays["out_" + tau_name] = out
        meta[tau_name] = {kk: vv for kk, vv in m.items() if isinstance(vv, (int, float, bool, str)) and
                          not kk.endswith("_ms")}
    ref_pipeline._cached_profile = None
    save("compact_f32", "pipeline.py:312-555 orthocache_forward(mode='compact') (CPU, float32, crossover 1024)",
         arrays, meta, {"tau_given": 7.5, "zeta_max": 5.0, "block_size": 512})

    # 5. eviction regimes: per-head and per-block masks, a tensor z_max
    g = torch.Generator().manual_seed(805)
    q = torch.randn(3, 4, 64, generator=g)
    e = torch.rand(10, 4, generator=g) * torch.logspace(-4, 4, 10)[:, None]
    m = torch.rand(10, 4, generator=g) < 0.15
    z = torch.tensor([60.0, 95.0, 80.0, 91.0])
    beta = compute_block_beta(q, e, 64)
    meta = classify_eviction(q, e, z, m, 64)
    meta1 = classify_eviction(q, e, torch.tensor(130.0), m.any(dim=1), 64, accumulator_dtype="bfloat16")
    save("regimes", "perfect_eviction.py:75-186 compute_block_beta + classify_eviction",
         {"q": q, "energy": e, "mask": m, "z_max": z, "beta_full": beta, "regime": meta.regime, "beta": meta.beta,
          "gap": meta.logit_gap, "regime_b": meta1.regime, "gap_b": meta1.logit_gap},
         {"counts": [meta.num_perfect, meta.num_statistical, meta.num_retained],
          "counts_b": [meta1.num_perfect, meta1.num_statistical, meta1.num_retained],
          "threshold": meta.underflow_threshold, "threshold_b": meta1.underflow_threshold},
         {"z_max_b": 130.0, "head_dim": 64})

    # 6. the model hook: prefill then one decode step, float32, G = 4, with
    #    the residual governor (alpha 0.5) and the entropy governor
    for gov_name in ("residual", "entropy"):
        g = torch.Generator().manual_seed(806)
        B, Hq, Hkv, S, d = 2, 4, 2, 4 * 64, 64
        Gq = Hq // Hkv
        qp = torch.randn(B, Hq, S, d, generator=g)
        kp = torch.stack([torch.stack([mixed_tiles(g, 4, d) for _ in range(Hkv)]) for _ in range(B)])
        vp = torch.randn(B, Hkv, S, d, generator=g)
        # bounds of the prefill gate (tau = -1 evicts nothing), for a tau in a gap
        probe = pe.OrthoCache_GQA_Attention(tau=-1.0)
        probe.norm_cache = SpectralNormCache(Hkv, 16, torch.device("cpu"))
        probe.orthocache_attention(qp, kp, vp, Gq)
        qn = torch.norm(qp.view(B, Hkv, Gq, S, d), dim=-1).median(dim=-1).values.amax(dim=-1)  # (B, Hkv)
        kn = probe.norm_cache.cache[:, :4]
        tau = gap_threshold((qn[:, :, None] * kn[None]).numpy() / (64.0 * d))
        gov = pe.ResidualGovernor(alpha=0.5) if gov_name == "residual" else \
            pe.EntropyGovernor(alpha=0.5, beta=1.0, h_median=1.56)
        hook = pe.OrthoCache_GQA_Attention(tau=tau, governor=gov)
        hook.norm_cache = SpectralNormCache(Hkv, 16, torch.device("cpu"))
        out_p = hook.orthocache_attention(qp, kp, vp, Gq)
        tau_after_prefill = gov.get_tau_effective(tau)
        # decode: one more token (a partial fifth tile), q of length 1
        q1 = torch.randn(B, Hq, 1, d, generator=g)
        k1 = torch.cat([kp, torch.randn(B, Hkv, 1, d, generator=g)], dim=2)
        v1 = torch.cat([vp, torch.randn(B, Hkv, 1, d, generator=g)], dim=2)
        out_d = hook.orthocache_attention(q1, k1, v1, Gq)
        st = hook.stats
        meta = {kk: st[kk] for kk in ("total_tiles", "evicted_tiles", "layers_processed", "decode_steps",
                                      "decode_tiles_skipped", "decode_tiles_total", "hallucination_scores",
                                      "q_search_intensity", "k_info_density")}
        if "entropy" in st:
            meta["entropy"] = st["entropy"]
        meta["layer_history"] = list(gov.layer_history)
        meta["tau_after_prefill"] = tau_after_prefill
        meta["tau_after_decode"] = gov.get_tau_effective(tau)
        arrays = {"out_prefill": out_p, "out_decode": out_d, "norm_cache": hook.norm_cache.cache,
                  "valid_tiles": hook.norm_cache.valid_tiles}
        params = {"tau": tau, "G": Gq, "alpha": 0.5, "beta": 1.0, "h_median": 1.56}
        if gov_name == "residual":
            arrays.update({"q_prefill": qp, "k_prefill": kp, "v_prefill": vp, "q_decode": q1, "k_decode": k1,
                           "v_decode": v1})
        else:
            params["inputs_from"] = "hook_residual"  # the same seeded inputs
        save("hook_%s" % gov_name, "perplexity_eval.py:320-689 OrthoCache_GQA_Attention prefill + decode "
             "(%s governor)" % gov_name, arrays, meta, params)

    man = os.path.join(out_dir, "MANIFEST_8f.json")
    with open(man, "w") as f:
        json.dump({"cases": names, "torch": torch.__version__, "generator": "tests/golden/make_golden_8f.py"}, f,
                  indent=1)
    print("wrote", len(names), "cases to", out_dir)


if __name__ == "__main__":
    main()
