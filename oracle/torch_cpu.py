"""PyTorch-CPU restatement of the reference's fp32 attention paths, used as the CPU baseline.

TEST INFRASTRUCTURE ONLY: imported by ``bench.py``'s ``cpu_baseline`` leg and by ``tests/``.  It
times the reference's own CPU-capable formulation (torch fp32 matmul -> softmax -> matmul, one row
at a time), never the product.
"""
from __future__ import annotations

import torch


def paged_decode_rows(q, k_cache, v_cache, seqlens, block_table, scale):
    """Per-row loop of ``Talker._attn_ref`` (engine/talker.py:82-88) with the page-table gather of
    ``flash_attn_with_kvcache`` (engine/talker.py:77).

    q [B, Hq, D] fp32; k_cache, v_cache [num_pages, page, Hkv, D] fp32; seqlens [B] int;
    block_table [B, P] int.  Returns [B, Hq, D] fp32 (ctx == 0 rows are zeros).
    """
    B, Hq, D = q.shape
    page, Hkv = k_cache.shape[1], k_cache.shape[2]
    G = Hq // Hkv
    out = []
    for b in range(B):
        ctx = int(seqlens[b])
        if ctx <= 0:
            out.append(torch.zeros(Hq, D, dtype=q.dtype))
            continue
        npg = (ctx + page - 1) // page
        pages = block_table[b, :npg].long()
        k = k_cache[pages].reshape(npg * page, Hkv, D)[:ctx].transpose(0, 1)        # [Hkv, ctx, D]
        v = v_cache[pages].reshape(npg * page, Hkv, D)[:ctx].transpose(0, 1)
        a = torch.matmul(q[b].view(Hkv, G, D), k.transpose(-1, -2)) * scale
        out.append(torch.matmul(torch.softmax(a, dim=-1), v).reshape(Hq, D))
    return torch.stack(out, 0)
