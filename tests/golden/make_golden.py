"""Write the golden vectors under tests/golden/ from the reference's own CPU code.

Run in the development container only (the reference tree is not present on
the GPU box):

    python tests/golden/make_golden.py /root/reference/src

It imports the reference's CPU ("PyTorch fallback") entry points in a
process whose sys.path holds only the reference tree, feeds them small
seeded inputs and stores inputs and outputs as data (npz + json).  Which
reference function produced each case is recorded in the case's json:

* triton_fwht_eviction CPU path   (fwht_fused_prototype.py:199-248)
* fused_orthocache_attention      (fused_eviction.py:698-755, :460-549)
* fused_orthocache_attention_v2   (fused_eviction.py:573-628, :380-457)
* fused_orthocache_attention_v3_gqa (gqa_eviction.py:511-574, :87-276)
* fused_orthocache_attention_paged  (paged_eviction.py:323-368, :244-316)

These vectors pin what neither closed forms nor known-answer tiles fix:
the metadata counts, the q*k_scale rounding in q's dtype, the paged fp8
path's double rounding and the reference's float32 bits.
"""

import json
import os
import sys


def _setup(ref_src):
    sys.path[:] = [p for p in sys.path if "orthocache-gpu_amd" not in p]
    sys.path.insert(0, ref_src)


def main():
    ref_src = sys.argv[1] if len(sys.argv) > 1 else "/root/reference/src"
    _setup(ref_src)
    import numpy as np
    import torch

    torch.set_num_threads(1)
    try:
        torch.set_flush_denormal(True)
    except ValueError:
        pass

    from orthocache_gpu.triton_kernels.fwht_fused_prototype import (
        _pytorch_fwht_eviction, generate_walsh_matrix)
    from orthocache_gpu.triton_kernels.fused_eviction import (
        fused_orthocache_attention, fused_orthocache_attention_v2)
    from orthocache_gpu.triton_kernels.gqa_eviction import fused_orthocache_attention_v3_gqa
    from orthocache_gpu.triton_kernels.paged_eviction import fused_orthocache_attention_paged

    out_dir = os.path.dirname(os.path.abspath(__file__))
    W = generate_walsh_matrix(64)

    def raw(t):
        """Tensor -> (numpy array of the stored bits/values, dtype name)."""
        t = t.detach().cpu().contiguous()
        if t.dtype == torch.float32:
            return t.numpy(), "f32"
        if t.dtype == torch.float16:
            return t.view(torch.int16).numpy().view(np.uint16), "f16"
        if t.dtype == torch.bfloat16:
            return t.view(torch.int16).numpy().view(np.uint16), "bf16"
        if t.dtype == torch.float8_e4m3fn:
            return t.view(torch.uint8).numpy(), "fp8"
        if t.dtype == torch.int32:
            return t.numpy(), "i32"
        if t.dtype == torch.bool:
            return t.numpy().astype(np.uint8), "bool"
        raise TypeError(t.dtype)

    def mixed_tiles(g, n_tiles, d, noise_every=2, scale=1.0):
        """Config-0 recipe in the reference's natural-order band semantics:
        smooth tiles = W @ C with rows 1..4 of C ~ N(0,1) plus 0.05 N(0,1);
        noise tiles = W @ C with rows 32..63 of C ~ N(0,1)."""
        tiles = []
        for i in range(n_tiles):
            c = torch.zeros(64, d)
            if i % noise_every == 1:
                c[32:64] = torch.randn(32, d, generator=g)
                tiles.append(W @ c)
            else:
                c[1:5] = torch.randn(4, d, generator=g)
                tiles.append(W @ c + 0.05 * torch.randn(64, d, generator=g))
        return torch.cat(tiles) * scale

    def quant_fp8(x):
        amax = x.abs().max().item()
        s = amax / 448.0 if amax > 0 else 1.0
        return (x / s).clamp(-448.0, 448.0).to(torch.float8_e4m3fn), s

    manifest = []

    def save(name, fn_ref, arrays, meta, params):
        npz = {}
        dtypes = {}
        for k, v in arrays.items():
            if isinstance(v, torch.Tensor):
                a, dt = raw(v)
            else:
                a, dt = np.asarray(v), "np"
            npz[k] = a
            dtypes[k] = dt
        np.savez_compressed(os.path.join(out_dir, name + ".npz"), **npz)
        clean = {}
        for k, v in meta.items():
            if isinstance(v, torch.Tensor):
                a, dt = raw(v)
                npz_key = "meta_" + k
                np.savez_compressed(os.path.join(out_dir, name + "." + npz_key + ".npz"), a=a)
                clean[k] = {"npz": name + "." + npz_key + ".npz", "dtype": dt}
            else:
                clean[k] = v
        with open(os.path.join(out_dir, name + ".json"), "w") as f:
            json.dump({"reference_function": fn_ref, "params": params,
                       "dtypes": dtypes, "meta": clean}, f, indent=1, sort_keys=True)
        manifest.append(name)

    # 1. tile scores (mask + zeta), reference test recipe + random tiles.
    g = torch.Generator().manual_seed(123)
    t = torch.linspace(0, 2 * np.pi, 64)
    blocks = [torch.sin(t).unsqueeze(1).expand(64, 128) + 0.01 * torch.randn(64, 128, generator=g)
              for _ in range(4)]
    blocks += [torch.randn(64, 128, generator=g) * 5.0 for _ in range(4)]
    keys = torch.cat([torch.cat(blocks), mixed_tiles(g, 8, 128),
                      torch.randn(4 * 64, 128, generator=g)])
    mask, zeta = _pytorch_fwht_eviction(keys, 5.0, 64, True)
    save("fwht_scores", "fwht_fused_prototype.py:199-248 _pytorch_fwht_eviction",
         {"keys": keys, "mask": mask, "zeta": zeta}, {}, {"zeta_max": 5.0})

    # 2. v1, fp32, mixed tiles, return_mask.
    g = torch.Generator().manual_seed(0)
    q = torch.randn(1, 128, generator=g)
    k = mixed_tiles(g, 6, 128)
    v = torch.randn(6 * 64, 128, generator=g)
    out, meta = fused_orthocache_attention(q, k, v, 5.0, return_mask=True)
    save("v1_f32", "fused_eviction.py:698-755 fused_orthocache_attention (CPU path)",
         {"q": q, "keys": k, "values": v, "out": out}, meta, {"zeta_max": 5.0})

    # 3. v1 with fp8 keys and a scalar k_scale, q in bf16.
    k8, ks = quant_fp8(k)
    qb = q.to(torch.bfloat16)
    out, meta = fused_orthocache_attention(qb, k8, v, 5.0, return_mask=True, k_scale=ks)
    save("v1_fp8k_bf16q", "fused_eviction.py:698-755 fused_orthocache_attention (CPU path, k_scale)",
         {"q": qb, "keys": k8, "values": v, "out": out}, meta, {"zeta_max": 5.0, "k_scale": ks})

    # 4. v2 multi-head in three dtypes, d=64 and d=128.
    for dt_name, dt, d in (("f32", torch.float32, 64), ("f16", torch.float16, 64),
                           ("bf16", torch.bfloat16, 128)):
        g = torch.Generator().manual_seed(7)
        hh, tt = 2, 8
        q = torch.randn(hh, d, generator=g).to(dt)
        k = torch.stack([mixed_tiles(g, tt, d) for _ in range(hh)])
        perm = [torch.randperm(tt, generator=g) for _ in range(hh)]
        k = torch.stack([k[h].view(tt, 64, d)[perm[h]].reshape(tt * 64, d) for h in range(hh)]).to(dt)
        v = torch.randn(hh, tt * 64, d, generator=g).to(dt)
        out, meta = fused_orthocache_attention_v2(q, k, v, 5.0)
        save("v2_" + dt_name, "fused_eviction.py:573-628 fused_orthocache_attention_v2 (CPU path)",
             {"q": q, "keys": k, "values": v, "out": out}, meta, {"zeta_max": 5.0})

    # 5. v3 GQA, CS gate with a tau between the two tile clusters.
    for dt_name, dt, d in (("f32", torch.float32, 64), ("bf16", torch.bfloat16, 128)):
        g = torch.Generator().manual_seed(11)
        hkv, G, tt = 2, 4, 6
        q = torch.randn(hkv * G, d, generator=g)
        q[1::G] *= 0.01
        q[0] *= 0.01
        q = q.to(dt)
        k = torch.stack([mixed_tiles(g, tt, d) for _ in range(hkv)]).to(dt)
        v = torch.randn(hkv, tt * 64, d, generator=g).to(dt)
        out, meta = fused_orthocache_attention_v3_gqa(q, k, v, 160.0, G)
        save("v3_" + dt_name, "gqa_eviction.py:511-574 fused_orthocache_attention_v3_gqa (CPU path)",
             {"q": q, "keys": k, "values": v, "out": out}, meta, {"tau": 160.0, "G": G})

    # 6. v3 with fp8 keys and scalar k_scale, bf16 q.
    g = torch.Generator().manual_seed(12)
    q = torch.randn(8, 128, generator=g).to(torch.bfloat16)
    kf = torch.stack([mixed_tiles(g, 4, 128) for _ in range(2)])
    k8, ks = quant_fp8(kf)
    v = torch.randn(2, 4 * 64, 128, generator=g).to(torch.bfloat16)
    out, meta = fused_orthocache_attention_v3_gqa(q, k8, v, 160.0, 4, k_scale=ks)
    save("v3_fp8k", "gqa_eviction.py:511-574 fused_orthocache_attention_v3_gqa (CPU path, k_scale)",
         {"q": q, "keys": k8, "values": v, "out": out}, meta, {"tau": 160.0, "G": 4, "k_scale": ks})

    # 7. paged, shuffled pool, block sizes 16 and 32, fp32.
    for bs in (16, 32):
        g = torch.Generator().manual_seed(21 + bs)
        B, H, d, tt = 2, 2, 64, 3
        nb = tt * 64 // bs
        q = torch.randn(B, H, d, generator=g)
        kc = torch.stack([torch.stack([mixed_tiles(g, tt, d) for _ in range(H)]) for _ in range(B)])
        vc = torch.randn(B, H, tt * 64, d, generator=g)
        pool = B * nb + 3
        perm = torch.randperm(pool, generator=g)
        bt = perm[:B * nb].view(B, nb).to(torch.int32)
        k_cache = torch.zeros(pool, H, bs, d)
        v_cache = torch.zeros(pool, H, bs, d)
        for b in range(B):
            for j in range(nb):
                k_cache[bt[b, j]] = kc[b, :, j * bs:(j + 1) * bs]
                v_cache[bt[b, j]] = vc[b, :, j * bs:(j + 1) * bs]
        out, meta = fused_orthocache_attention_paged(q, k_cache, v_cache, bt, 5.0)
        save("paged_bs%d" % bs, "paged_eviction.py:323-368 fused_orthocache_attention_paged (CPU path)",
             {"q": q, "k_cache": k_cache, "v_cache": v_cache, "block_tables": bt, "out": out},
             meta, {"zeta_max": 5.0})

    # 8. paged with an fp8 key cache, bf16 q and cache values, k_scale.
    g = torch.Generator().manual_seed(31)
    B, H, d, bs, tt = 1, 2, 128, 64, 4
    q = torch.randn(B, H, d, generator=g).to(torch.bfloat16)
    kc = torch.stack([mixed_tiles(g, tt, d) for _ in range(H)])
    k_cache = kc.view(H, tt, 64, d).permute(1, 0, 2, 3).contiguous()
    v_cache = torch.randn(tt, H, bs, d, generator=g).to(torch.bfloat16)
    k8, ks = quant_fp8(k_cache)
    bt = torch.arange(tt, dtype=torch.int32).view(1, tt)
    out, meta = fused_orthocache_attention_paged(q, k8, v_cache, bt, 5.0, k_scale=ks)
    save("paged_fp8k", "paged_eviction.py:323-368 fused_orthocache_attention_paged (CPU path, fp8 k_cache)",
         {"q": q, "k_cache": k8, "v_cache": v_cache, "block_tables": bt, "out": out},
         meta, {"zeta_max": 5.0, "k_scale": ks})

    with open(os.path.join(out_dir, "MANIFEST.json"), "w") as f:
        json.dump({"cases": manifest, "torch": torch.__version__,
                   "generator": "tests/golden/make_golden.py"}, f, indent=1)
    print("wrote", len(manifest), "cases to", out_dir)


if __name__ == "__main__":
    main()
