"""Helpers shared by the GPU parity tests (test infrastructure)."""
from __future__ import annotations

import numpy as np
import torch

from oracle import oracle as orc
from rvllm_amd.kv_storage import HipKvStorage


def dev_u32(a) -> torch.Tensor:
    arr = np.ascontiguousarray(np.asarray(a, dtype=np.uint32)).view(np.int32)
    return torch.from_numpy(arr.copy()).cuda()


def fill_layer(store: HipKvStorage, layer: int, seed: int,
               scale: float = 1.0, chunk_tokens: int = 1 << 17) -> None:
    """Writes N(0,1)*scale f16 values into every slot of `layer` through
    rvkv_append (f16 source), drawn on the device from a seeded generator."""
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    bs, nkv, hd = store.block_size, store.n_kv_heads, store.head_dim
    total = store.num_blocks * bs
    for t0 in range(0, total, chunk_tokens):
        n = min(chunk_tokens, total - t0)
        slots = torch.arange(t0, t0 + n, device="cuda", dtype=torch.int64)
        blk = (slots // bs).to(torch.int32)
        off = (slots % bs).to(torch.int32)
        k = (torch.randn((n, nkv, hd), generator=g, device="cuda") * scale
             ).to(torch.float16)
        v = (torch.randn((n, nkv, hd), generator=g, device="cuda") * scale
             ).to(torch.float16)
        store.write_tokens(layer, blk, off, k, v)


def oracle_subset(store: HipKvStorage, layer: int, tables, ctx_lens):
    """Copies the blocks the given sequences read into a compact oracle
    cache (f16 bits) and returns (cache, remapped padded tables, max_blocks)."""
    uniq = np.unique(np.concatenate([np.asarray(t, np.uint32)
                                     for t in tables]))
    remap = {int(b): i for i, b in enumerate(uniq)}
    ids = dev_u32(uniq)
    kb = store.read_blocks(layer, 0, ids).cpu().numpy().view(np.uint16)
    vb = store.read_blocks(layer, 1, ids).cpu().numpy().view(np.uint16)
    cache = orc.KvCache(len(uniq), store.block_size, store.n_kv_heads,
                        store.head_dim, orc.F16)
    cache.k[:] = kb
    cache.v[:] = vb
    mb = max(len(t) for t in tables)
    padded = np.zeros((len(tables), mb), np.uint32)
    for i, t in enumerate(tables):
        r = [remap[int(x)] for x in t]
        padded[i, :len(r)] = r
        padded[i, len(r):] = r[-1] if r else 0
    return cache, padded, mb
