"""Attention entry points of the talker, as torch custom ops over the q3attn C ABI.

``flash_attn_with_kvcache`` keeps the call signature and tensor layouts the engine uses at
engine/talker.py:77, so the talker's import line (engine/talker.py:13) can point here instead.
The ops are registered with ``torch.library.custom_op`` (opaque to torch.compile, with fake
implementations for tracing), enqueue on the current HIP stream, allocate only through torch's
caching allocator and never synchronise, so they can be captured into HIP graphs.  They run on
the GPU only: CPU tensors raise.
"""
from __future__ import annotations

import math
from typing import Optional

import torch

from ._lib import check, lib


# Fixed-split limits of q3a_paged_decode (split_tokens <= 1024, at most 64 splits per row).
_MAX_SPLIT_TOKENS = 1024
_MAX_SPLITS = 64

# Decomposition codes, passed as split_tokens (include/q3attn.h): 0 lets the library choose from the batch and the
# table capacity; these force one kernel (tests and benchmarks run each on the same shapes).
DECODE_ROW = -1        # one workgroup per (row, KV head), one launch (tables <= 2,048 tokens)
DECODE_CHUNKS = -2     # chunks of each row over many workgroups, then a combine (small batches of long rows)
DECODE_STREAMK = -3    # stream-K over all rows' tiles, then a combine (batch <= 4096)
DECODE_PLANNED = -4    # stream-K read from a per-frame plan (decode_plan); the plan is the call's workspace

# Plan forms (include/q3attn.h): which entry point a plan serves.
_PLAN_FORMS = {"plain": 0, "append": 1, "append_rope": 2}


def _req(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _check_decode_inputs(q, k_cache, v_cache, cache_seqlens, block_table):
    _req(q.is_cuda, "q3attn.paged_decode: tensors must be on a GPU (there is no CPU path)")
    dev = q.device
    for name, t in (("k_cache", k_cache), ("v_cache", v_cache), ("cache_seqlens", cache_seqlens),
                    ("block_table", block_table)):
        _req(t.device == dev, f"q3attn.paged_decode: {name} is on {t.device}, q on {dev}")
    _req(q.dtype == torch.bfloat16, f"q3attn.paged_decode: q must be bfloat16, got {q.dtype}")
    _req(k_cache.dtype == torch.bfloat16 and v_cache.dtype == torch.bfloat16,
         "q3attn.paged_decode: k_cache/v_cache must be bfloat16")
    _req(q.dim() == 3, f"q3attn.paged_decode: q must be [batch, heads, head_dim], got {tuple(q.shape)}")
    _req(k_cache.dim() == 4, "q3attn.paged_decode: k_cache must be [num_pages, page_size, kv_heads, head_dim]")
    _req(k_cache.shape == v_cache.shape and k_cache.stride() == v_cache.stride(),
         "q3attn.paged_decode: k_cache and v_cache must have the same shape and strides")
    _req(q.stride(-1) == 1 and k_cache.stride(-1) == 1, "q3attn.paged_decode: last dimension must be contiguous")
    B, Hq, D = q.shape
    _req(k_cache.shape[3] == D, "q3attn.paged_decode: head_dim mismatch between q and k_cache")
    _req(cache_seqlens.dtype == torch.int32 and cache_seqlens.shape == (B,),
         "q3attn.paged_decode: cache_seqlens must be int32 [batch]")
    _req(cache_seqlens.is_contiguous(), "q3attn.paged_decode: cache_seqlens must be contiguous")
    _req(block_table.dtype == torch.int32 and block_table.dim() == 2 and block_table.shape[0] == B,
         "q3attn.paged_decode: block_table must be int32 [batch, max_pages]")
    _req(block_table.stride(1) == 1, "q3attn.paged_decode: block_table rows must be contiguous")


def decode_plan(cache_seqlens: torch.Tensor, block_table: torch.Tensor, page_size: int, num_kv_heads: int = 8,
                form: str = "plain"):
    """The stream-K decomposition of the decode calls that share ``cache_seqlens`` and ``block_table``, built once
    (one launch on the current stream) and passed to each of them as ``plan=`` (``scheduler_metadata=`` in
    ``flash_attn_with_kvcache``).  The talker's 28 calls of a frame all take the frame's ctx and block table
    (engine/talker.py:77, 107-112), so one plan per frame serves them all: a planned call's waves read their tile
    lists and page ids in one memory round trip instead of scanning cache_seqlens and looking pages up in the table.

    ``block_table`` is [batch, max_pages] (one plan, a uint8 tensor) or [tables, batch, max_pages] (one plan per
    table, stacked: plan t serves table t).  ``form``: "plain" (paged_decode), "append" (paged_decode_append) or
    "append_rope" (paged_decode_append_rope); ``cache_seqlens`` as those calls take it.  Returns None for shapes the
    library does not decode with stream-K (small batches, narrow tables): pass the None on, the calls then take their
    usual path.  The plan holds the lengths and table entries of the moment the plan kernel runs: build it again
    after either changes.  Calls that share a plan must not run concurrently (each uses the buffer behind the plan
    as scratch for its partial records); calls on one stream never do.  Build it outside a torch.compile'd region
    (it is a host call that allocates its result), as flash-attn 3's get_scheduler_metadata is used."""
    _req(cache_seqlens.is_cuda, "q3attn.decode_plan: tensors must be on a GPU")
    _req(form in _PLAN_FORMS, f"q3attn.decode_plan: form must be one of {sorted(_PLAN_FORMS)}, got {form!r}")
    _req(cache_seqlens.dtype == torch.int32 and cache_seqlens.dim() == 1 and cache_seqlens.is_contiguous(),
         "q3attn.decode_plan: cache_seqlens must be a contiguous int32 [batch] tensor")
    _req(block_table.device == cache_seqlens.device and block_table.dtype == torch.int32,
         "q3attn.decode_plan: block_table must be int32 on cache_seqlens' device")
    stacked = block_table.dim() == 3
    bt = block_table if stacked else block_table.unsqueeze(0)
    _req(bt.dim() == 3 and bt.shape[1] == cache_seqlens.shape[0] and bt.stride(2) == 1,
         "q3attn.decode_plan: block_table must be [batch, max_pages] or [tables, batch, max_pages] with contiguous rows")
    T, B, max_pages = bt.shape
    L = lib()
    nbytes = L.q3a_paged_decode_plan_bytes(B, int(num_kv_heads), max_pages, int(page_size))
    if nbytes == 0 or T == 0:
        return None
    stride = (nbytes + 255) // 256 * 256
    plans = torch.empty((T, stride), dtype=torch.uint8, device=cache_seqlens.device)
    rc = L.q3a_paged_decode_plan(cache_seqlens.data_ptr(), bt.data_ptr(), bt.stride(1), bt.stride(0), T, max_pages,
                                 int(page_size), B, int(num_kv_heads), _PLAN_FORMS[form], plans.data_ptr(), stride,
                                 plans.numel(), _stream(cache_seqlens.device))
    check(rc, "q3a_paged_decode_plan")
    return plans if stacked else plans[0]


def _plan_ws(plan, q, what):
    """(workspace, bytes, split code) of a planned call."""
    _req(plan.device == q.device and plan.dtype == torch.uint8 and plan.dim() == 1 and plan.is_contiguous(),
         f"q3attn.{what}: plan must be a uint8 plan from q3attn.decode_plan on q's device")
    return plan, plan.numel(), DECODE_PLANNED


@torch.library.custom_op("q3attn::paged_decode", mutates_args=())
def paged_decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                 cache_seqlens: torch.Tensor, block_table: torch.Tensor, softmax_scale: float,
                 split_tokens: int = 0, plan: Optional[torch.Tensor] = None) -> torch.Tensor:
    """o[b, h] = softmax(q[b, h] . K_b^T * scale) . V_b over the ctx = cache_seqlens[b] tokens of
    row b, gathered through ``block_table``; query head h reads KV head h // (Hq / Hkv).

    q [B, Hq, D] bf16; k_cache, v_cache [num_pages, page_size, Hkv, D] bf16; cache_seqlens [B]
    int32; block_table [B, max_pages] int32.  Returns [B, Hq, D] bf16.  fp32 semantics:
    engine/talker.py:82-88; the call it replaces: engine/talker.py:77.  ``plan``: a decode_plan(form="plain") of
    these cache_seqlens and block_table (the call then ignores split_tokens).  The plan buffer is also the call's
    scratch for its partial records, which it writes and reads within the call; the plan itself is left as it was,
    so the op is declared free of mutation and calls in one stream may share a plan.
    """
    _check_decode_inputs(q, k_cache, v_cache, cache_seqlens, block_table)
    B, Hq, D = q.shape
    num_pages, page, Hkv, _ = k_cache.shape
    max_pages = block_table.shape[1]
    out = torch.empty((B, Hq, D), dtype=q.dtype, device=q.device)
    if B == 0:
        return out
    L = lib()
    if plan is not None:
        ws, ws_bytes, split = _plan_ws(plan, q, "paged_decode")
    else:
        split = int(split_tokens)            # 0: the library's default decomposition (stream-K)
        ws_bytes = L.q3a_paged_decode_workspace_bytes(B, Hq, Hkv, D, max_pages, page, split)
        ws = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=q.device)
    rc = L.q3a_paged_decode(
        q.data_ptr(), q.stride(0), q.stride(1),
        k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(0), k_cache.stride(1), k_cache.stride(2),
        num_pages, page,
        cache_seqlens.data_ptr(), block_table.data_ptr(), block_table.stride(0), max_pages,
        out.data_ptr(), out.stride(0), out.stride(1),
        ws.data_ptr(), ws_bytes,
        B, Hq, Hkv, D, float(softmax_scale), split, _stream(q.device))
    check(rc, "q3a_paged_decode")
    return out


@paged_decode.register_fake
def _paged_decode_fake(q, k_cache, v_cache, cache_seqlens, block_table, softmax_scale, split_tokens=0, plan=None):
    return q.new_empty(q.shape)


def _new_rows(x, B, Hkv, D, name):
    """k/v of this step as [B, Hkv, D] with packed heads: accepts [B, Hkv, D], [B, 1, Hkv, D] or [B, Hkv*D]
    views (e.g. the v slice of a fused qkv projection)."""
    if x.dim() == 4:
        _req(x.shape[1] == 1, f"q3attn.paged_decode_append: {name} must hold one new token per row")
        x = x[:, 0]
    elif x.dim() == 2:
        x = x.view(x.shape[0], Hkv, D)
    _req(x.dtype == torch.bfloat16, f"q3attn.paged_decode_append: {name} must be bfloat16")
    _req(tuple(x.shape) == (B, Hkv, D), f"q3attn.paged_decode_append: {name} must be [B, {Hkv}, {D}]")
    _req(x.stride(2) == 1 and x.stride(1) == D, f"q3attn.paged_decode_append: {name} heads must be packed")
    return x


@torch.library.custom_op("q3attn::paged_decode_append", mutates_args=("k_cache", "v_cache"))
def paged_decode_append(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, k_cache: torch.Tensor,
                        v_cache: torch.Tensor, cache_seqlens: torch.Tensor, block_table: torch.Tensor,
                        softmax_scale: float, split_tokens: int = 0,
                        plan: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Append + attend in one pass: writes k[b], v[b] at position p = cache_seqlens[b] of row b (page
    block_table[b][p // page], offset p % page) and returns the attention of q[b] over tokens 0..p
    (engine/talker.py:72-73 then :77).  Rows with cache_seqlens < 0 give zeros and write nothing.  ``plan``: a
    decode_plan(form="append") of these cache_seqlens and block_table."""
    _check_decode_inputs(q, k_cache, v_cache, cache_seqlens, block_table)
    B, Hq, D = q.shape
    num_pages, page, Hkv, _ = k_cache.shape
    _req(k.device == q.device and v.device == q.device, "q3attn.paged_decode_append: k, v must be on q's device")
    k3 = _new_rows(k, B, Hkv, D, "k")
    v3 = _new_rows(v, B, Hkv, D, "v")
    max_pages = block_table.shape[1]
    out = torch.empty((B, Hq, D), dtype=q.dtype, device=q.device)
    if B == 0:
        return out
    L = lib()
    if plan is not None:
        ws, ws_bytes, split = _plan_ws(plan, q, "paged_decode_append")
    else:
        split = int(split_tokens)
        ws_bytes = L.q3a_paged_decode_workspace_bytes(B, Hq, Hkv, D, max_pages, page, split)
        ws = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=q.device)
    rc = L.q3a_paged_decode_append(
        q.data_ptr(), q.stride(0), q.stride(1),
        k3.data_ptr(), k3.stride(0), v3.data_ptr(), v3.stride(0),
        k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(0), k_cache.stride(1), k_cache.stride(2),
        num_pages, page,
        cache_seqlens.data_ptr(), block_table.data_ptr(), block_table.stride(0), max_pages,
        out.data_ptr(), out.stride(0), out.stride(1),
        ws.data_ptr(), ws_bytes,
        B, Hq, Hkv, D, float(softmax_scale), split, _stream(q.device))
    check(rc, "q3a_paged_decode_append")
    return out


@paged_decode_append.register_fake
def _paged_decode_append_fake(q, k, v, k_cache, v_cache, cache_seqlens, block_table, softmax_scale,
                              split_tokens=0, plan=None):
    return q.new_empty(q.shape)


def _rope_rows(x: torch.Tensor, B: int, D: int, dev, name: str) -> torch.Tensor:
    """cos/sin of each row's new position: [B, D] or the talker's [B, 1, D] (engine/talker.py:108)."""
    _req(x.device == dev and x.dtype == torch.bfloat16, f"q3attn.paged_decode_append_rope: {name} must be bfloat16 "
         "on q's device")
    if x.dim() == 3:
        _req(x.shape[1] == 1, f"q3attn.paged_decode_append_rope: {name} must be [B, {D}] or [B, 1, {D}]")
        x = x[:, 0]
    _req(tuple(x.shape) == (B, D) and x.stride(1) == 1,
         f"q3attn.paged_decode_append_rope: {name} must be [B, {D}] with contiguous rows")
    _req(x.stride(0) % 8 == 0 and x.data_ptr() % 16 == 0,
         f"q3attn.paged_decode_append_rope: {name} rows must be 16-byte aligned")
    return x


@torch.library.custom_op("q3attn::paged_decode_append_rope", mutates_args=("k_cache", "v_cache"))
def paged_decode_append_rope(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, q_norm_w: torch.Tensor,
                             k_norm_w: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, k_cache: torch.Tensor,
                             v_cache: torch.Tensor, cache_seqlens: torch.Tensor, block_table: torch.Tensor,
                             softmax_scale: float, eps: float = 1e-6, split_tokens: int = 0,
                             plan: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The talker's per-layer attention block in one launch (engine/talker.py:69-77): q and k arrive as the raw
    projections (views of the qkv output), are RMS-normalised with q_norm_w / k_norm_w and rotated with each row's
    cos/sin (engine/ops.py:51-60), k and v are written at position p = cache_seqlens[b] of row b, and the attention of
    q[b] over tokens 0..p is returned, as paged_decode_append does for already-normalised q and k.  split_tokens: 0
    (the library's choice) or one of the DECODE_* codes; fixed splits do not take this form.  ``plan``: a
    decode_plan(form="append_rope") of these cache_seqlens and block_table."""
    _check_decode_inputs(q, k_cache, v_cache, cache_seqlens, block_table)
    B, Hq, D = q.shape
    num_pages, page, Hkv, _ = k_cache.shape
    dev = q.device
    _req(k.device == dev and v.device == dev, "q3attn.paged_decode_append_rope: k, v must be on q's device")
    k3 = _new_rows(k, B, Hkv, D, "k")
    v3 = _new_rows(v, B, Hkv, D, "v")
    for name, w in (("q_norm_w", q_norm_w), ("k_norm_w", k_norm_w)):
        _req(w.device == dev and w.dtype == torch.bfloat16 and tuple(w.shape) == (D,) and w.is_contiguous()
             and w.data_ptr() % 16 == 0, f"q3attn.paged_decode_append_rope: {name} must be a contiguous, "
             f"16-byte aligned bfloat16 [{D}] tensor on q's device")
    c2 = _rope_rows(cos, B, D, dev, "cos")
    s2 = _rope_rows(sin, B, D, dev, "sin")
    _req(c2.stride(0) == s2.stride(0), "q3attn.paged_decode_append_rope: cos and sin must share a row stride")
    max_pages = block_table.shape[1]
    out = torch.empty((B, Hq, D), dtype=q.dtype, device=dev)
    if B == 0:
        return out
    L = lib()
    if plan is not None:
        ws, ws_bytes, split = _plan_ws(plan, q, "paged_decode_append_rope")
    else:
        split = int(split_tokens)
        ws_bytes = L.q3a_paged_decode_workspace_bytes(B, Hq, Hkv, D, max_pages, page, split)
        ws = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=dev)
    rc = L.q3a_paged_decode_append_rope(
        q.data_ptr(), q.stride(0), q.stride(1),
        k3.data_ptr(), k3.stride(0), v3.data_ptr(), v3.stride(0),
        q_norm_w.data_ptr(), k_norm_w.data_ptr(), c2.data_ptr(), s2.data_ptr(), c2.stride(0), float(eps),
        k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(0), k_cache.stride(1), k_cache.stride(2),
        num_pages, page,
        cache_seqlens.data_ptr(), block_table.data_ptr(), block_table.stride(0), max_pages,
        out.data_ptr(), out.stride(0), out.stride(1),
        ws.data_ptr(), ws_bytes,
        B, Hq, Hkv, D, float(softmax_scale), split, _stream(dev))
    check(rc, "q3a_paged_decode_append_rope")
    return out


@paged_decode_append_rope.register_fake
def _paged_decode_append_rope_fake(q, k, v, q_norm_w, k_norm_w, cos, sin, k_cache, v_cache, cache_seqlens,
                                   block_table, softmax_scale, eps=1e-6, split_tokens=0, plan=None):
    return q.new_empty(q.shape)


def flash_attn_with_kvcache(q, k_cache, v_cache, k=None, v=None, rotary_cos=None, rotary_sin=None,
                            cache_seqlens=None, cache_batch_idx=None, cache_leftpad=None,
                            block_table=None, softmax_scale=None, causal=False, window_size=(-1, -1),
                            softcap=0.0, rotary_interleaved=True, alibi_slopes=None, num_splits=0,
                            return_softmax_lse=False, scheduler_metadata=None):
    """Drop-in for the paged-decode subset of ``flash_attn.flash_attn_with_kvcache`` that the talker
    calls (engine/talker.py:77): q [B, 1, Hq, D], paged caches, int32 ``cache_seqlens`` and
    ``block_table``, ``softmax_scale``, ``causal`` (a no-op for one query token).  Returns
    [B, 1, Hq, D].

    With ``k``/``v`` ([B, 1, Hkv, D], one new token per row) the flash-attn append semantics apply:
    the new token is written into the caches at position ``cache_seqlens[b]`` and attention runs over
    ``cache_seqlens[b] + 1`` tokens, in one pass (replacing engine/talker.py:72-73 + :77);
    ``cache_seqlens`` itself is not updated.  ``scheduler_metadata``: a plan from q3attn.decode_plan for these
    cache_seqlens and block_table (form "append" with k/v, else "plain"), built once for the calls that share them;
    None decodes without one.  Arguments the talker does not use raise NotImplementedError."""
    _req((k is None) == (v is None), "q3attn.flash_attn_with_kvcache: pass both k and v, or neither")
    unsupported = {"rotary_cos": rotary_cos, "rotary_sin": rotary_sin,
                   "cache_batch_idx": cache_batch_idx, "cache_leftpad": cache_leftpad,
                   "alibi_slopes": alibi_slopes}
    for name, val in unsupported.items():
        if val is not None:
            raise NotImplementedError(f"q3attn.flash_attn_with_kvcache: argument {name!r} is not supported")
    if tuple(window_size) != (-1, -1) or softcap != 0.0 or return_softmax_lse:
        raise NotImplementedError("q3attn.flash_attn_with_kvcache: window_size/softcap/return_softmax_lse unsupported")
    _req(cache_seqlens is not None and block_table is not None,
         "q3attn.flash_attn_with_kvcache: cache_seqlens and block_table are required")
    _req(q.dim() == 4 and q.shape[1] == 1,
         f"q3attn.flash_attn_with_kvcache: q must be [batch, 1, heads, head_dim], got {tuple(q.shape)}")
    if isinstance(cache_seqlens, int):
        cache_seqlens = torch.full((q.shape[0],), cache_seqlens, dtype=torch.int32, device=q.device)
    scale = softmax_scale if softmax_scale is not None else q.shape[-1] ** -0.5
    split = 0
    if num_splits and num_splits > 0:
        # flash-attn's split count maps to a fixed split length, kept inside the library's limits: at most
        # _MAX_SPLITS splits per row and _MAX_SPLIT_TOKENS tokens per split (beyond both: stream-K).
        max_ctx = block_table.shape[1] * k_cache.shape[1]
        ceil16 = lambda n: 16 * math.ceil(n / 16)
        lo = max(16, ceil16(math.ceil(max_ctx / _MAX_SPLITS)))
        split = min(max(lo, ceil16(math.ceil(max_ctx / num_splits))), _MAX_SPLIT_TOKENS)
        if lo > _MAX_SPLIT_TOKENS:
            split = 0
    if k is not None:
        _req(k.dim() == 4 and v.dim() == 4, "q3attn.flash_attn_with_kvcache: k/v must be [batch, new, kv_heads, head_dim]")
        if k.shape[1] != 1 or v.shape[1] != 1:
            raise NotImplementedError("q3attn.flash_attn_with_kvcache: one new token per row is supported")
        o = paged_decode_append(q[:, 0], k[:, 0], v[:, 0], k_cache, v_cache, cache_seqlens, block_table,
                                float(scale), split, scheduler_metadata)
    else:
        o = paged_decode(q[:, 0], k_cache, v_cache, cache_seqlens, block_table, float(scale), split,
                         scheduler_metadata)
    return o.unsqueeze(1)
