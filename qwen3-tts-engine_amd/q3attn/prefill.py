"""Talker prefill attention (packed variable-length, MFMA) as torch custom ops over the q3attn C ABI.

``flash_attn_varlen_func`` keeps the signature the talker uses at engine/talker.py:169 and ``flash_attn_func``
the one at engine/arrivals.py:148 (bottom-right causal for a K/V prefix longer than the queries).  Both also
accept the paged KV pool through ``block_table`` (the layout the talker writes at engine/talker.py:161-162),
so prefill can read K/V back from the pool.  ``prefill_append`` also writes the prompt's K/V into the pool
(engine/talker.py:161-162) in the same launch.  GPU only.
"""
from __future__ import annotations

from typing import Optional

import torch

from ._lib import check, lib


def _req(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


@torch.library.custom_op("q3attn::prefill", mutates_args=())
def prefill(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu_seqlens_q: torch.Tensor,
            cu_seqlens_k: torch.Tensor, block_table: Optional[torch.Tensor], max_seqlen_q: int,
            softmax_scale: float, causal: bool) -> torch.Tensor:
    """q [T, Hq, D]; k, v packed [Tk, Hkv, D] (block_table None) or the paged pool
    [num_pages, page, Hkv, D]; cu_seqlens int32 [n+1].  Returns [T, Hq, D] bf16."""
    _req(q.is_cuda, "q3attn.prefill: tensors must be on a GPU (there is no CPU path)")
    for name, t in (("k", k), ("v", v), ("cu_seqlens_q", cu_seqlens_q), ("cu_seqlens_k", cu_seqlens_k)):
        _req(t.device == q.device, f"q3attn.prefill: {name} is on {t.device}, q on {q.device}")
    _req(q.dtype == torch.bfloat16 and k.dtype == torch.bfloat16 and v.dtype == torch.bfloat16,
         "q3attn.prefill: q, k, v must be bfloat16")
    _req(q.dim() == 3 and q.stride(-1) == 1, "q3attn.prefill: q must be [tokens, heads, head_dim], dim contiguous")
    # k and v may differ in strides: the talker passes a fresh k and v as a view of the qkv projection
    # (engine/talker.py:158-160).
    _req(k.shape == v.shape, "q3attn.prefill: k and v must have the same shape")
    _req(k.stride(-1) == 1 and v.stride(-1) == 1, "q3attn.prefill: k/v head_dim must be contiguous")
    _req(cu_seqlens_q.dtype == torch.int32 and cu_seqlens_k.dtype == torch.int32,
         "q3attn.prefill: cu_seqlens must be int32")
    _req(cu_seqlens_q.is_contiguous() and cu_seqlens_k.is_contiguous() and cu_seqlens_q.shape == cu_seqlens_k.shape,
         "q3attn.prefill: cu_seqlens_q/k must be contiguous [n+1]")
    T, Hq, D = q.shape
    n = cu_seqlens_q.shape[0] - 1
    out = torch.empty_like(q, memory_format=torch.contiguous_format)
    if n <= 0 or T == 0:
        return out.zero_() if T else out
    if block_table is None:
        _req(k.dim() == 3 and k.shape[2] == D, "q3attn.prefill: packed k/v must be [tokens, kv_heads, head_dim]")
        Hkv = k.shape[1]
        ks, vs = (0, k.stride(0), k.stride(1)), (0, v.stride(0), v.stride(1))
        num_pages, page, bt_ptr, bt_sb, max_pages = 0, 0, None, 0, 0
    else:
        _req(k.dim() == 4 and k.shape[3] == D, "q3attn.prefill: paged k/v must be [num_pages, page, kv_heads, head_dim]")
        _req(block_table.dtype == torch.int32 and block_table.dim() == 2 and block_table.shape[0] == n
             and block_table.stride(1) == 1 and block_table.device == q.device,
             "q3attn.prefill: block_table must be int32 [n, max_pages] with contiguous rows")
        num_pages, page, Hkv = k.shape[0], k.shape[1], k.shape[2]
        ks, vs = (k.stride(0), k.stride(1), k.stride(2)), (v.stride(0), v.stride(1), v.stride(2))
        bt_ptr, bt_sb, max_pages = block_table.data_ptr(), block_table.stride(0), block_table.shape[1]
    rc = lib().q3a_prefill(
        q.data_ptr(), q.stride(0), q.stride(1), cu_seqlens_q.data_ptr(),
        k.data_ptr(), *ks, v.data_ptr(), *vs, num_pages, page, bt_ptr, bt_sb, max_pages,
        cu_seqlens_k.data_ptr(), out.data_ptr(), out.stride(0), out.stride(1),
        n, int(max_seqlen_q), Hq, Hkv, D, float(softmax_scale), 1 if causal else 0,
        torch.cuda.current_stream(q.device).cuda_stream)
    check(rc, "q3a_prefill")
    return out


@prefill.register_fake
def _prefill_fake(q, k, v, cu_seqlens_q, cu_seqlens_k, block_table, max_seqlen_q, softmax_scale, causal):
    return torch.empty_like(q, memory_format=torch.contiguous_format)


def _unsupported(dropout_p, window_size, softcap, alibi_slopes, return_attn_probs):
    if dropout_p or tuple(window_size) != (-1, -1) or softcap or alibi_slopes is not None or return_attn_probs:
        raise NotImplementedError("q3attn: dropout, windows, softcap, alibi and returned probabilities are unsupported")


def flash_attn_varlen_func(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, dropout_p=0.0,
                           softmax_scale=None, causal=False, window_size=(-1, -1), softcap=0.0, alibi_slopes=None,
                           deterministic=False, return_attn_probs=False, block_table=None):
    """Drop-in for ``flash_attn.flash_attn_varlen_func`` as the talker calls it (engine/talker.py:169):
    q [T, Hq, D], k/v [Tk, Hkv, D] (or the paged pool with ``block_table``), int32 cumulative lengths.
    Returns [T, Hq, D]."""
    _unsupported(dropout_p, window_size, softcap, alibi_slopes, return_attn_probs)
    scale = softmax_scale if softmax_scale is not None else q.shape[-1] ** -0.5
    return prefill(q, k, v, cu_seqlens_q, cu_seqlens_k, block_table, int(max_seqlen_q), float(scale), bool(causal))


@torch.library.custom_op("q3attn::prefill_append", mutates_args=("k_cache", "v_cache"))
def prefill_append(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu_seqlens_q: torch.Tensor,
                   cu_seqlens_k: torch.Tensor, max_seqlen_q: int, k_cache: torch.Tensor, v_cache: torch.Tensor,
                   block_table: torch.Tensor, softmax_scale: float, causal: bool = True) -> torch.Tensor:
    """The talker's prompt step in one launch: the K and V rows of every query token (packed k/v [Tk, Hkv, D]) go
    into the paged pool [num_pages, page, Hkv, D] at the token's position in its sequence, through block_table
    [n, max_pages] (engine/talker.py:161-162 scatters them with index_copy_ at seat * seat_len + position), and the
    result is flash_attn_varlen_func(q, k, v, ...) over the packed k/v (engine/talker.py:169), bit for bit."""
    _req(q.is_cuda, "q3attn.prefill_append: tensors must be on a GPU (there is no CPU path)")
    for name, t in (("k", k), ("v", v), ("cu_seqlens_q", cu_seqlens_q), ("cu_seqlens_k", cu_seqlens_k),
                    ("k_cache", k_cache), ("v_cache", v_cache), ("block_table", block_table)):
        _req(t.device == q.device, f"q3attn.prefill_append: {name} is on {t.device}, q on {q.device}")
    _req(all(t.dtype == torch.bfloat16 for t in (q, k, v, k_cache, v_cache)),
         "q3attn.prefill_append: q, k, v and the caches must be bfloat16")
    _req(q.dim() == 3 and q.stride(-1) == 1, "q3attn.prefill_append: q must be [tokens, heads, head_dim], dim contiguous")
    _req(k.dim() == 3 and k.shape == v.shape and k.stride(-1) == 1 and v.stride(-1) == 1,
         "q3attn.prefill_append: k and v must be packed [tokens, kv_heads, head_dim] with a contiguous head_dim")
    _req(k_cache.dim() == 4 and k_cache.shape == v_cache.shape and k_cache.stride() == v_cache.stride()
         and k_cache.stride(-1) == 1 and k_cache.shape[2:] == k.shape[1:],
         "q3attn.prefill_append: k_cache and v_cache must be [num_pages, page, kv_heads, head_dim] with equal strides")
    _req(cu_seqlens_q.dtype == torch.int32 and cu_seqlens_k.dtype == torch.int32 and cu_seqlens_q.is_contiguous()
         and cu_seqlens_k.is_contiguous() and cu_seqlens_q.shape == cu_seqlens_k.shape,
         "q3attn.prefill_append: cu_seqlens_q/k must be contiguous int32 [n+1]")
    n = cu_seqlens_q.shape[0] - 1
    _req(block_table.dtype == torch.int32 and block_table.dim() == 2 and block_table.shape[0] == max(n, 0)
         and block_table.stride(1) == 1, "q3attn.prefill_append: block_table must be int32 [n, max_pages] with contiguous rows")
    T, Hq, D = q.shape
    out = torch.empty_like(q, memory_format=torch.contiguous_format)
    if n <= 0 or T == 0:
        return out.zero_() if T else out
    num_pages, page, Hkv, _ = k_cache.shape
    rc = lib().q3a_prefill_append(
        q.data_ptr(), q.stride(0), q.stride(1), cu_seqlens_q.data_ptr(),
        k.data_ptr(), k.stride(0), k.stride(1), v.data_ptr(), v.stride(0), v.stride(1), cu_seqlens_k.data_ptr(),
        k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(0), k_cache.stride(1), k_cache.stride(2),
        num_pages, page, block_table.data_ptr(), block_table.stride(0), block_table.shape[1],
        out.data_ptr(), out.stride(0), out.stride(1),
        n, int(max_seqlen_q), Hq, Hkv, D, float(softmax_scale), 1 if causal else 0,
        torch.cuda.current_stream(q.device).cuda_stream)
    check(rc, "q3a_prefill_append")
    return out


@prefill_append.register_fake
def _prefill_append_fake(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, k_cache, v_cache, block_table,
                         softmax_scale, causal=True):
    return torch.empty_like(q, memory_format=torch.contiguous_format)


@torch.library.custom_op("q3attn::prefill_dense", mutates_args=())
def prefill_dense(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, softmax_scale: float,
                  causal: bool) -> torch.Tensor:
    """q [S, R, Hq, D]; k, v [S, n, Hkv, D] (any strides with a contiguous head dim).  Returns [S, R, Hq, D] bf16."""
    _req(q.is_cuda, "q3attn.flash_attn_func: tensors must be on a GPU (there is no CPU path)")
    _req(k.device == q.device and v.device == q.device, "q3attn.flash_attn_func: q, k, v must share a device")
    _req(q.dtype == torch.bfloat16 and k.dtype == torch.bfloat16 and v.dtype == torch.bfloat16,
         "q3attn.flash_attn_func: q, k, v must be bfloat16")
    _req(q.dim() == 4 and k.dim() == 4 and k.shape == v.shape
         and q.shape[0] == k.shape[0] and q.shape[3] == k.shape[3],
         "q3attn.flash_attn_func: q [S,R,H,D], k/v [S,n,Hkv,D]")
    _req(q.stride(3) == 1 and k.stride(3) == 1 and v.stride(3) == 1, "q3attn.flash_attn_func: head_dim must be contiguous")
    S, R, Hq, D = q.shape
    n, Hkv = k.shape[1], k.shape[2]
    out = torch.empty((S, R, Hq, D), dtype=q.dtype, device=q.device)
    if S == 0 or R == 0:
        return out
    rc = lib().q3a_prefill_dense(
        q.data_ptr(), q.stride(0), q.stride(1), q.stride(2), k.data_ptr(), k.stride(0), k.stride(1), k.stride(2),
        v.data_ptr(), v.stride(0), v.stride(1), v.stride(2), out.data_ptr(), out.stride(0), out.stride(1),
        out.stride(2), S, R, n, Hq, Hkv, D,
        float(softmax_scale), 1 if causal else 0, torch.cuda.current_stream(q.device).cuda_stream)
    check(rc, "q3a_prefill_dense")
    return out


@prefill_dense.register_fake
def _prefill_dense_fake(q, k, v, softmax_scale, causal):
    return q.new_empty(q.shape)


@torch.library.custom_op("q3attn::prefill_dense_append", mutates_args=("k_cache", "v_cache"))
def prefill_dense_append(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, k_cache: torch.Tensor,
                         v_cache: torch.Tensor, block_table: torch.Tensor, softmax_scale: float, causal: bool = True,
                         first_row: int = 0) -> torch.Tensor:
    """The fast-admission layer step in one launch: rows first_row .. n-1 of every sequence's K and V (dense
    [S, n, Hkv, D]) go into the paged pool [num_pages, page, Hkv, D] at positions first_row .. n-1 of the sequence,
    through block_table [S, max_pages] (engine/arrivals.py:144-145 scatters all n rows with index_copy_ at
    seat * seat_len + position), and the result is flash_attn_func(q, k, v, softmax_scale, causal) on the dense
    k/v (engine/arrivals.py:148), bit for bit.  first_row = 0 is the engine's call; n - R writes only the new rows
    (a prefix already in the pool)."""
    who = "q3attn.prefill_dense_append"
    _req(q.is_cuda, f"{who}: tensors must be on a GPU (there is no CPU path)")
    for name, t in (("k", k), ("v", v), ("k_cache", k_cache), ("v_cache", v_cache), ("block_table", block_table)):
        _req(t.device == q.device, f"{who}: {name} is on {t.device}, q on {q.device}")
    _req(all(t.dtype == torch.bfloat16 for t in (q, k, v, k_cache, v_cache)),
         f"{who}: q, k, v and the caches must be bfloat16")
    _req(q.dim() == 4 and k.dim() == 4 and k.shape == v.shape and q.shape[0] == k.shape[0] and q.shape[3] == k.shape[3],
         f"{who}: q [S,R,H,D], k/v [S,n,Hkv,D]")
    _req(q.stride(3) == 1 and k.stride(3) == 1 and v.stride(3) == 1, f"{who}: head_dim must be contiguous")
    _req(k_cache.dim() == 4 and k_cache.shape == v_cache.shape and k_cache.stride() == v_cache.stride()
         and k_cache.stride(-1) == 1 and k_cache.shape[2:] == k.shape[2:],
         f"{who}: k_cache and v_cache must be [num_pages, page, kv_heads, head_dim] with equal strides")
    S, R, Hq, D = q.shape
    n, Hkv = k.shape[1], k.shape[2]
    _req(block_table.dtype == torch.int32 and block_table.dim() == 2 and block_table.shape[0] == S
         and block_table.stride(1) == 1, f"{who}: block_table must be int32 [S, max_pages] with contiguous rows")
    _req(0 <= first_row <= max(0, n - R), f"{who}: first_row {first_row} must lie in [0, max(0, n - R)]")
    out = torch.empty((S, R, Hq, D), dtype=q.dtype, device=q.device)
    if S == 0 or R == 0:
        return out
    num_pages, page = k_cache.shape[0], k_cache.shape[1]
    rc = lib().q3a_prefill_dense_append(
        q.data_ptr(), q.stride(0), q.stride(1), q.stride(2), k.data_ptr(), k.stride(0), k.stride(1), k.stride(2),
        v.data_ptr(), v.stride(0), v.stride(1), v.stride(2),
        k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(0), k_cache.stride(1), k_cache.stride(2),
        num_pages, page, block_table.data_ptr(), block_table.stride(0), block_table.shape[1], int(first_row),
        out.data_ptr(), out.stride(0), out.stride(1), out.stride(2), S, R, n, Hq, Hkv, D,
        float(softmax_scale), 1 if causal else 0, torch.cuda.current_stream(q.device).cuda_stream)
    check(rc, "q3a_prefill_dense_append")
    return out


@prefill_dense_append.register_fake
def _prefill_dense_append_fake(q, k, v, k_cache, v_cache, block_table, softmax_scale, causal=True, first_row=0):
    return q.new_empty(q.shape)


@torch.library.custom_op("q3attn::prefill_append_rope", mutates_args=("k_cache", "v_cache"))
def prefill_append_rope(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, q_norm_w: torch.Tensor,
                        k_norm_w: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, cu_seqlens: torch.Tensor,
                        max_seqlen: int, k_cache: torch.Tensor, v_cache: torch.Tensor, block_table: torch.Tensor,
                        softmax_scale: float, causal: bool = True, eps: float = 1e-6) -> torch.Tensor:
    """The talker's prompt step with its producers (engine/talker.py:157-169) in two launches: q [T, Hq, D] and k
    [T, Hkv, D] arrive raw (views of the qkv projection), are RMS-normalised and rotated with each token's cos/sin row
    ([T, D], or [T, 1, D] as the engine gathers them) with the rounding of eager bf16 ops (engine/ops.py:51-60), k and
    v go into the pool at each token's position through block_table [n, max_pages], and the result is
    flash_attn_varlen_func(q, k, v, cu_seqlens, cu_seqlens, ...) over the normalised q and k [T, Hq, D].  Causal, the
    first launch normalises k straight into the pool and the attention kernel reads K back from there and normalises
    q itself (a key whose table entry is invalid or missing attends with zeros for K); otherwise the first launch
    normalises both into a workspace."""
    who = "q3attn.prefill_append_rope"
    _req(q.is_cuda, f"{who}: tensors must be on a GPU (there is no CPU path)")
    dev = q.device
    for name, t in (("k", k), ("v", v), ("q_norm_w", q_norm_w), ("k_norm_w", k_norm_w), ("cos", cos), ("sin", sin),
                    ("cu_seqlens", cu_seqlens), ("k_cache", k_cache), ("v_cache", v_cache),
                    ("block_table", block_table)):
        _req(t.device == dev, f"{who}: {name} is on {t.device}, q on {dev}")
    _req(all(t.dtype == torch.bfloat16 for t in (q, k, v, q_norm_w, k_norm_w, cos, sin, k_cache, v_cache)),
         f"{who}: q, k, v, the weights, cos/sin and the caches must be bfloat16")
    _req(q.dim() == 3 and k.dim() == 3 and k.shape == v.shape and q.shape[0] == k.shape[0] and q.shape[2] == k.shape[2],
         f"{who}: q [T, Hq, D], k/v [T, Hkv, D]")
    T, Hq, D = q.shape
    Hkv = k.shape[1]
    _req(all(t.stride(-1) == 1 for t in (q, k, v)), f"{who}: head_dim must be contiguous")
    for name, w in (("q_norm_w", q_norm_w), ("k_norm_w", k_norm_w)):
        _req(tuple(w.shape) == (D,) and w.is_contiguous(), f"{who}: {name} must be a contiguous [{D}] tensor")
    c2, s2 = cos.reshape(-1, D), sin.reshape(-1, D)
    _req(c2.shape[0] == T and s2.shape[0] == T and c2.stride(1) == 1 and c2.stride(0) == s2.stride(0),
         f"{who}: cos/sin must hold T = {T} rows of {D} with a contiguous last dim and a shared row stride")
    _req(cu_seqlens.dtype == torch.int32 and cu_seqlens.dim() == 1 and cu_seqlens.is_contiguous(),
         f"{who}: cu_seqlens must be contiguous int32 [n+1]")
    n = cu_seqlens.shape[0] - 1
    _req(k_cache.dim() == 4 and k_cache.shape == v_cache.shape and k_cache.stride() == v_cache.stride()
         and k_cache.stride(-1) == 1 and k_cache.shape[2:] == k.shape[1:],
         f"{who}: k_cache and v_cache must be [num_pages, page, kv_heads, head_dim] with equal strides")
    _req(block_table.dtype == torch.int32 and block_table.dim() == 2 and block_table.shape[0] == max(n, 0)
         and block_table.stride(1) == 1, f"{who}: block_table must be int32 [n, max_pages] with contiguous rows")
    out = torch.empty((T, Hq, D), dtype=q.dtype, device=dev)
    if n <= 0 or T == 0:
        return out.zero_() if T else out
    L = lib()
    # causal: the k rows go straight into the pool and q is normalised in the attention, so no workspace
    ws_bytes = 0 if causal else L.q3a_prefill_append_rope_workspace_bytes(T, Hq, Hkv, D)
    ws = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=dev) if ws_bytes else None
    num_pages, page = k_cache.shape[0], k_cache.shape[1]
    rc = L.q3a_prefill_append_rope(
        q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), k.stride(0), k.stride(1), v.data_ptr(), v.stride(0),
        v.stride(1), q_norm_w.data_ptr(), k_norm_w.data_ptr(), c2.data_ptr(), s2.data_ptr(), c2.stride(0), float(eps),
        cu_seqlens.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(0), k_cache.stride(1),
        k_cache.stride(2), num_pages, page, block_table.data_ptr(), block_table.stride(0), block_table.shape[1],
        out.data_ptr(), out.stride(0), out.stride(1), ws.data_ptr() if ws is not None else None, ws_bytes, n, T,
        int(max_seqlen), Hq, Hkv, D, float(softmax_scale), 1 if causal else 0, torch.cuda.current_stream(dev).cuda_stream)
    check(rc, "q3a_prefill_append_rope")
    return out


@prefill_append_rope.register_fake
def _prefill_append_rope_fake(q, k, v, q_norm_w, k_norm_w, cos, sin, cu_seqlens, max_seqlen, k_cache, v_cache,
                              block_table, softmax_scale, causal=True, eps=1e-6):
    return torch.empty_like(q, memory_format=torch.contiguous_format)


@torch.library.custom_op("q3attn::prefill_dense_append_rope", mutates_args=("k_cache", "v_cache"))
def prefill_dense_append_rope(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, prefix_k: torch.Tensor,
                              prefix_v: torch.Tensor, q_norm_w: torch.Tensor, k_norm_w: torch.Tensor,
                              cos: torch.Tensor, sin: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                              block_table: torch.Tensor, softmax_scale: float,
                              prefix_index: Optional[torch.Tensor] = None, causal: bool = True, eps: float = 1e-6,
                              first_row: int = 0) -> torch.Tensor:
    """The fast-admission layer's attention block (engine/arrivals.py:112-118, 144-148), one launch when P + R <= 128
    and R <= 112, else two: q and the
    new k arrive raw (views of the qkv projection [S, R, ...]) and are RMS-normalised and rotated with the new tokens'
    cos/sin rows ([R, D], or any view with R*D elements and a contiguous last dim such as [1, R, 1, D]), with the
    rounding of eager bf16 torch ops (engine/ops.py:51-60); K = cat(prefix_k, k) and V = cat(prefix_v, v) with
    prefix_k/prefix_v [num_prefixes, P, Hkv, D] taken at prefix_index[s] (int64 [S], as engine/arrivals.py:143 gathers
    self.pK[l][slot]) or at s; rows first_row .. P+R-1 of K and V go into the pool through block_table [S, max_pages]
    and the result is flash_attn_func(q, K, V, softmax_scale, causal) [S, R, Hq, D]."""
    who = "q3attn.prefill_dense_append_rope"
    _req(q.is_cuda, f"{who}: tensors must be on a GPU (there is no CPU path)")
    dev = q.device
    for name, t in (("k", k), ("v", v), ("prefix_k", prefix_k), ("prefix_v", prefix_v), ("q_norm_w", q_norm_w),
                    ("k_norm_w", k_norm_w), ("cos", cos), ("sin", sin), ("k_cache", k_cache), ("v_cache", v_cache),
                    ("block_table", block_table)):
        _req(t.device == dev, f"{who}: {name} is on {t.device}, q on {dev}")
    _req(all(t.dtype == torch.bfloat16 for t in (q, k, v, prefix_k, prefix_v, q_norm_w, k_norm_w, cos, sin, k_cache,
                                                  v_cache)), f"{who}: all tensors but the table and index must be bfloat16")
    _req(q.dim() == 4 and k.dim() == 4 and k.shape == v.shape and q.shape[:2] == k.shape[:2]
         and q.shape[3] == k.shape[3], f"{who}: q [S,R,Hq,D], k/v [S,R,Hkv,D]")
    S, R, Hq, D = q.shape
    Hkv = k.shape[2]
    _req(prefix_k.dim() == 4 and prefix_k.shape == prefix_v.shape and prefix_k.shape[2:] == k.shape[2:],
         f"{who}: prefix_k/prefix_v must be [num_prefixes, P, Hkv, D]")
    P = prefix_k.shape[1]
    _req(all(t.stride(-1) == 1 for t in (q, k, v, prefix_k, prefix_v)), f"{who}: head_dim must be contiguous")
    for name, w in (("q_norm_w", q_norm_w), ("k_norm_w", k_norm_w)):
        _req(tuple(w.shape) == (D,) and w.is_contiguous(), f"{who}: {name} must be a contiguous [{D}] tensor")
    c2, s2 = cos.reshape(-1, D), sin.reshape(-1, D)
    _req(c2.shape[0] == R and s2.shape[0] == R and c2.stride(1) == 1 and c2.stride(0) == s2.stride(0),
         f"{who}: cos/sin must hold R = {R} rows of {D} with a contiguous last dim and a shared row stride")
    if prefix_index is not None:
        _req(prefix_index.device == dev and prefix_index.dtype == torch.int64 and prefix_index.shape == (S,)
             and prefix_index.is_contiguous(), f"{who}: prefix_index must be a contiguous int64 [S] tensor")
    else:
        _req(prefix_k.shape[0] == S, f"{who}: without prefix_index, prefix_k needs one prefix per sequence")
    _req(k_cache.dim() == 4 and k_cache.shape == v_cache.shape and k_cache.stride() == v_cache.stride()
         and k_cache.stride(-1) == 1 and k_cache.shape[2:] == k.shape[2:],
         f"{who}: k_cache and v_cache must be [num_pages, page, kv_heads, head_dim] with equal strides")
    _req(block_table.dtype == torch.int32 and block_table.dim() == 2 and block_table.shape[0] == S
         and block_table.stride(1) == 1, f"{who}: block_table must be int32 [S, max_pages] with contiguous rows")
    _req(0 <= first_row <= P, f"{who}: first_row {first_row} must lie in [0, prefix length {P}]")
    out = torch.empty((S, R, Hq, D), dtype=q.dtype, device=dev)
    if S == 0 or R == 0:
        return out
    L = lib()
    ws_bytes = L.q3a_prefill_dense_append_rope_workspace_bytes(S, R, P, Hq, Hkv, D)
    ws = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=dev)
    num_pages, page = k_cache.shape[0], k_cache.shape[1]
    rc = L.q3a_prefill_dense_append_rope(
        q.data_ptr(), q.stride(0), q.stride(1), q.stride(2), k.data_ptr(), k.stride(0), k.stride(1), k.stride(2),
        v.data_ptr(), v.stride(0), v.stride(1), v.stride(2),
        prefix_k.data_ptr(), prefix_k.stride(0), prefix_k.stride(1), prefix_k.stride(2),
        prefix_v.data_ptr(), prefix_v.stride(0), prefix_v.stride(1), prefix_v.stride(2),
        prefix_index.data_ptr() if prefix_index is not None else None, prefix_k.shape[0],
        q_norm_w.data_ptr(), k_norm_w.data_ptr(), c2.data_ptr(), s2.data_ptr(), c2.stride(0), float(eps),
        k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(0), k_cache.stride(1), k_cache.stride(2),
        num_pages, page, block_table.data_ptr(), block_table.stride(0), block_table.shape[1], int(first_row),
        out.data_ptr(), out.stride(0), out.stride(1), out.stride(2), ws.data_ptr(), ws_bytes,
        S, R, P, Hq, Hkv, D, float(softmax_scale), 1 if causal else 0, torch.cuda.current_stream(dev).cuda_stream)
    check(rc, "q3a_prefill_dense_append_rope")
    return out


@prefill_dense_append_rope.register_fake
def _prefill_dense_append_rope_fake(q, k, v, prefix_k, prefix_v, q_norm_w, k_norm_w, cos, sin, k_cache, v_cache,
                                    block_table, softmax_scale, prefix_index=None, causal=True, eps=1e-6,
                                    first_row=0):
    return q.new_empty(q.shape)


def flash_attn_func(q, k, v, dropout_p=0.0, softmax_scale=None, causal=False, window_size=(-1, -1), softcap=0.0,
                    alibi_slopes=None, deterministic=False, return_attn_probs=False):
    """Drop-in for ``flash_attn.flash_attn_func`` as the fast-admission path calls it (engine/arrivals.py:148):
    q [S, R, Hq, D], k/v [S, n, Hkv, D]; with ``causal`` query i sees the n - R prefix keys and the new keys
    <= i (bottom-right).  Returns [S, R, Hq, D]."""
    _unsupported(dropout_p, window_size, softcap, alibi_slopes, return_attn_probs)
    scale = softmax_scale if softmax_scale is not None else q.shape[-1] ** -0.5
    return prefill_dense(q, k, v, float(scale), bool(causal))
