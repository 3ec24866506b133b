"""Shared helpers for the tests: oracle evaluation of GPU workloads on host copies."""
from __future__ import annotations

import numpy as np
import torch

from oracle import attention as ora


def to_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def decode_oracle(wl, layer: int = 0, rows=None, acc=np.float32):
    """Oracle output [len(rows), Hq, D] for the given rows of a q3attn DecodeWorkload.

    Only the pages the selected rows reference are copied to the host (a compact pool with a
    renumbered table), so this stays cheap for the full-size pools."""
    L = wl.layers[layer]
    B = wl.batch
    rows = list(range(B)) if rows is None else list(rows)
    page = wl.page_size
    bt = L.block_table.cpu().numpy().astype(np.int64)
    ctx = wl.ctx[rows]
    need = [bt[b, : (int(c) + page - 1) // page] for b, c in zip(rows, ctx)]
    flat = np.concatenate(need) if need else np.zeros(0, np.int64)
    uniq = np.unique(flat) if flat.size else np.zeros(1, np.int64)
    remap = {int(p): i for i, p in enumerate(uniq)}
    idx = torch.from_numpy(uniq).to(wl.k_cache.device)
    k = to_np(wl.k_cache.index_select(0, idx))
    v = to_np(wl.v_cache.index_select(0, idx))
    P = max(1, max((len(n) for n in need), default=1))
    table = np.zeros((len(rows), P), np.int64)
    for i, n in enumerate(need):
        table[i, : len(n)] = [remap[int(p)] for p in n]
    q = to_np(L.q[rows])
    return ora.paged_decode(q, k, v, ctx, table, wl.scale, acc=acc)
