"""Write golden vectors for head dims other than 64 / 128 and tiles other
than 64 tokens, from the reference's own CPU code.

Run in the development container only (the reference tree is not present on
the GPU box):

    python tests/golden/make_golden_shapes.py /root/reference/src

Like make_golden.py, it imports the reference's CPU entry points in a
process whose sys.path holds only the reference tree, feeds them small
seeded inputs and stores inputs and outputs as data (npz + json), with the
producing function recorded in each case's json.  The reference asserts
only that head_dim and tile_size are powers of two
(fused_eviction.py:609-610, gqa_eviction.py:551-552, paged_eviction.py:
345-347); its bands stay the rows [1, 8) and [32, 64) of the tile's
spectrum, clipped to the tile (fused_eviction.py:424-427).  These cases pin
the oracle and the portable kernels at such shapes:

* triton_fwht_eviction CPU path at 16, 32, 128 and 256-token tiles
  (fwht_fused_prototype.py:199-248)
* fused_orthocache_attention at head_dim 32, and at 128-token tiles
  (fused_eviction.py:698-755, :460-549)
* fused_orthocache_attention_v2 at head_dim 16 / 32 / 256 and 32 / 128-token
  tiles (fused_eviction.py:573-628, :380-457)
* fused_orthocache_attention_v3_gqa at head_dim 256 and 128-token tiles, and
  at 32-token tiles, whose empty high band evicts every tile
  (gqa_eviction.py:511-574, :87-276)
* fused_orthocache_attention_paged at head_dim 256, 128-token tiles over
  32-token blocks, head_dim 32 with 32-token tiles (paged_eviction.py:323-368,
  :244-316)
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
        if t.dtype == torch.bool:
            return t.numpy().astype(np.uint8), "bool"
        raise TypeError(t.dtype)

    def mixed_tiles(g, n_tiles, d, ts, noise_every=2):
        """The config-0 recipe at ts-token tiles: smooth tiles W_ts C with
        rows 1..4 of C ~ N(0, 1) plus 0.05 N(0, 1); noise tiles W_ts C with
        rows [min(32, ts / 2), ts) of C ~ N(0, 1)."""
        W = generate_walsh_matrix(ts)
        lo_end = min(5, ts)
        hi0 = min(32, ts // 2)
        tiles = []
        for i in range(n_tiles):
            c = torch.zeros(ts, d)
            if i % noise_every == 1:
                c[hi0:] = torch.randn(ts - hi0, d, generator=g)
                tiles.append(W @ c)
            else:
                c[1:lo_end] = torch.randn(lo_end - 1, d, generator=g)
                tiles.append(W @ c + 0.05 * torch.randn(ts, d, generator=g))
        return torch.cat(tiles)

    manifest = []

    def save(name, fn_ref, arrays, meta, params):
        npz, dtypes = {}, {}
        for k, v in arrays.items():
            a, dt = raw(v) if isinstance(v, torch.Tensor) else (np.asarray(v), "np")
            npz[k] = a
            dtypes[k] = dt
        np.savez_compressed(os.path.join(out_dir, name + ".npz"), **npz)
        clean = {}
        for k, v in meta.items():
            if isinstance(v, torch.Tensor):
                a, dt = raw(v)
                key = "meta_" + k
                np.savez_compressed(os.path.join(out_dir, name + "." + key + ".npz"), a=a)
                clean[k] = {"npz": name + "." + key + ".npz", "dtype": dt}
            else:
                clean[k] = v
        with open(os.path.join(out_dir, name + ".json"), "w") as f:
            json.dump({"reference_function": fn_ref, "params": params, "dtypes": dtypes, "meta": clean}, f,
                      indent=1, sort_keys=True)
        manifest.append(name)

    # 1. tile scores at other tile sizes (d = 64)
    for ts in (16, 32, 128, 256):
        g = torch.Generator().manual_seed(300 + ts)
        keys = torch.cat([mixed_tiles(g, 6, 64, ts), torch.randn(2 * ts, 64, generator=g)])
        mask, zeta = _pytorch_fwht_eviction(keys, 5.0, ts, True)
        save(f"shapes_fwht_ts{ts}", "fwht_fused_prototype.py:199-248 _pytorch_fwht_eviction",
             {"keys": keys, "mask": mask, "zeta": zeta}, {}, {"zeta_max": 5.0, "tile_size": ts})

    # 2. v1: head_dim 32 (64-token tiles) and 128-token tiles (head_dim 64)
    for name, d, ts in (("shapes_v1_d32", 32, 64), ("shapes_v1_ts128", 64, 128)):
        g = torch.Generator().manual_seed(400 + d + ts)
        q = torch.randn(1, d, generator=g)
        k = mixed_tiles(g, 6, d, ts)
        v = torch.randn(6 * ts, d, generator=g)
        out, meta = fused_orthocache_attention(q, k, v, 5.0, tile_size=ts, return_mask=True)
        save(name, "fused_eviction.py:698-755 fused_orthocache_attention (CPU path)",
             {"q": q, "keys": k, "values": v, "out": out}, meta, {"zeta_max": 5.0, "tile_size": ts})

    # 3. v2 multi-head
    for name, dt, d, ts in (("shapes_v2_d256_bf16", torch.bfloat16, 256, 64),
                            ("shapes_v2_d32_f16", torch.float16, 32, 64),
                            ("shapes_v2_d16_ts16_f32", torch.float32, 16, 16),
                            ("shapes_v2_ts32_f32", torch.float32, 128, 32),
                            ("shapes_v2_ts128_bf16", torch.bfloat16, 128, 128)):
        g = torch.Generator().manual_seed(500 + d + ts)
        hh, tt = 2, 8
        q = torch.randn(hh, d, generator=g).to(dt)
        k = torch.stack([mixed_tiles(g, tt, d, ts) for _ in range(hh)])
        perm = [torch.randperm(tt, generator=g) for _ in range(hh)]
        k = torch.stack([k[h].view(tt, ts, d)[perm[h]].reshape(tt * ts, d) for h in range(hh)]).to(dt)
        v = torch.randn(hh, tt * ts, d, generator=g).to(dt)
        out, meta = fused_orthocache_attention_v2(q, k, v, 5.0, tile_size=ts)
        save(name, "fused_eviction.py:573-628 fused_orthocache_attention_v2 (CPU path)",
             {"q": q, "keys": k, "values": v, "out": out}, meta, {"zeta_max": 5.0, "tile_size": ts})

    # 4. v3 GQA with the Cauchy-Schwarz gate; tau between the tile clusters
    #    (32-token tiles: the high band is empty, every tile is evicted)
    for name, dt, d, ts, tau in (("shapes_v3_d256_f32", torch.float32, 256, 64, 230.0),
                                 ("shapes_v3_ts128_bf16", torch.bfloat16, 64, 128, 110.0),
                                 ("shapes_v3_ts32_f32", torch.float32, 128, 32, 1.0)):
        g = torch.Generator().manual_seed(600 + d + ts)
        hkv, G, tt = 2, 4, 6
        q = torch.randn(hkv * G, d, generator=g)
        q[1::G] *= 0.01
        q = q.to(dt)
        k = torch.stack([mixed_tiles(g, tt, d, ts) for _ in range(hkv)]).to(dt)
        v = torch.randn(hkv, tt * ts, d, generator=g).to(dt)
        out, meta = fused_orthocache_attention_v3_gqa(q, k, v, tau, G, tile_size=ts)
        save(name, "gqa_eviction.py:511-574 fused_orthocache_attention_v3_gqa (CPU path)",
             {"q": q, "keys": k, "values": v, "out": out}, meta, {"tau": tau, "G": G, "tile_size": ts})

    # 5. paged, shuffled pool
    for name, d, ts, bs in (("shapes_paged_d256", 256, 64, 16), ("shapes_paged_ts128", 64, 128, 32),
                            ("shapes_paged_d32_ts32", 32, 32, 16)):
        g = torch.Generator().manual_seed(700 + d + ts + bs)
        B, H, tt = 2, 2, 3
        nb = tt * ts // bs
        q = torch.randn(B, H, d, generator=g)
        kc = torch.stack([torch.stack([mixed_tiles(g, tt, d, ts) for _ in range(H)]) for _ in range(B)])
        vc = torch.randn(B, H, tt * ts, d, generator=g)
        pool = B * nb + 3
        perm = torch.randperm(pool, generator=g)
        bt = perm[:B * nb].view(B, nb).to(torch.int32)
        k_cache = torch.zeros(pool, H, bs, d)
        v_cache = torch.zeros(pool, H, bs, d)
        for b in range(B):
            for j in range(nb):
                k_cache[bt[b, j]] = kc[b, :, j * bs:(j + 1) * bs]
                v_cache[bt[b, j]] = vc[b, :, j * bs:(j + 1) * bs]
        out, meta = fused_orthocache_attention_paged(q, k_cache, v_cache, bt, 5.0, tile_size=ts)
        save(name, "paged_eviction.py:323-368 fused_orthocache_attention_paged (CPU path)",
             {"q": q, "k_cache": k_cache, "v_cache": v_cache, "block_tables": bt, "out": out},
             meta, {"zeta_max": 5.0, "tile_size": ts})

    with open(os.path.join(out_dir, "MANIFEST_shapes.json"), "w") as f:
        json.dump({"cases": manifest, "torch": torch.__version__,
                   "generator": "tests/golden/make_golden_shapes.py"}, f, indent=1)
    print("wrote", len(manifest), "cases to", out_dir)


if __name__ == "__main__":
    main()
