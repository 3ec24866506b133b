"""PyTorch restatement of the reference's fp32 attention paths (the CPU baseline) and of its q/k producers.

TEST INFRASTRUCTURE ONLY: imported by ``bench.py``'s ``cpu_baseline`` leg and by ``tests/``.  It
times the reference's own CPU-capable formulation (torch fp32 matmul -> softmax -> matmul, one row
at a time), never the product.  ``rms`` and ``rope`` are the reference's producers as torch ops on
any device (the synthetic models and the tests run them on the GPU as the engine does); on the CPU
they are pinned bit for bit to ``oracle.attention.norm_rope`` (tests/test_producers.py).
"""
from __future__ import annotations

import torch


def rms(x, w, eps=1e-6):
    """Qwen3 qk/hidden RMSNorm as engine/ops.py:51-55 writes it: normalise in float32, cast back to x's dtype, scale."""
    xf = x.float()
    xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return w * xf.to(x.dtype)


def rope(x, cos, sin):
    """Rotate-half RoPE as engine/ops.py:58-60 writes it."""
    h = x.shape[-1] // 2
    return x * cos + torch.cat((-x[..., h:], x[..., :h]), dim=-1) * sin


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


def cp_attn_rows(q, K, V, n_live, scale):
    """``CodePredictor._post``'s attention exactly as the reference writes it (engine/code_predictor.py:46-47),
    on CPU bf16 tensors: q [B, 16, 128], K/V [B, 8, 16, 128] -> [B, 2048]."""
    B, Hkv, S, D = K.shape
    mask = torch.full((S, S), float("-inf")).triu(1).to(q.dtype)[n_live - 1]
    att = torch.matmul(q.view(B, Hkv, q.shape[1] // Hkv, D), K.transpose(-1, -2)) * scale + mask
    return torch.matmul(torch.softmax(att.float(), dim=-1).to(q.dtype), V).reshape(B, -1)


def prefill_rows(q, k, v, cu_seqlens, scale):
    """The fp32 single-sequence prefill of ``Talker.prefill_hidden`` (engine/talker.py:165-167), looped over
    the packed sequences: q [T, 16, 128], k/v [T, 8, 128] fp32 -> [T, 16, 128]."""
    T, Hq, D = q.shape
    Hkv = k.shape[1]
    out = torch.empty_like(q)
    for i in range(len(cu_seqlens) - 1):
        s0, s1 = int(cu_seqlens[i]), int(cu_seqlens[i + 1])
        L = s1 - s0
        qh = q[s0:s1].transpose(0, 1).reshape(Hkv, Hq // Hkv, L, D)
        kh = k[s0:s1].transpose(0, 1)[:, None]
        vh = v[s0:s1].transpose(0, 1)[:, None]
        a = torch.matmul(qh, kh.transpose(-1, -2)) * scale + torch.full((L, L), float("-inf")).triu(1)
        out[s0:s1] = torch.matmul(torch.softmax(a, dim=-1), vh).reshape(Hq, L, D).transpose(0, 1)
    return out


def prefill_prefix_rows(q, K, V, scale):
    """``FastAdmit._attn_ref`` (engine/arrivals.py:125-131) on CPU fp32 tensors: q [S, R, 16, 128] attends over
    K/V [S, n, 8, 128], query i seeing the n - R prefix keys and the new keys <= i (mask triu(n - R + 1)).
    Returns [S, R, 16, 128]."""
    S, R, Hq, D = q.shape
    n, Hkv = K.shape[1], K.shape[2]
    m = torch.full((R, n), float("-inf")).triu(n - R + 1)
    qh = q.permute(0, 2, 1, 3).reshape(S, Hkv, Hq // Hkv, R, D)
    Kh = K.permute(0, 2, 1, 3)[:, :, None]
    Vh = V.permute(0, 2, 1, 3)[:, :, None]
    a = torch.matmul(qh, Kh.transpose(-1, -2)) * scale + m
    return torch.matmul(torch.softmax(a, dim=-1), Vh).reshape(S, Hq, R, D).permute(0, 2, 1, 3)
