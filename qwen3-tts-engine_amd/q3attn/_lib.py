"""Loader for the q3attn C-ABI library (``libq3attn.so``, built from ``csrc/`` for gfx950).

torch is imported first on purpose: the library's ``libamdhip64.so.7`` dependency then binds to
the HIP runtime torch already loaded, so both share one runtime, one device context and the
same stream handles.  There is no fallback: a missing library raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (must precede the library load, see above)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libq3attn.so")
ABI_VERSION = 8

_c_i64 = ctypes.c_int64
_c_int = ctypes.c_int
_c_vp = ctypes.c_void_p
_c_size = ctypes.c_size_t
_c_float = ctypes.c_float

# Exported symbols and their C signatures (include/q3attn.h).
SIGNATURES = {
    "q3a_abi_version": (_c_int, []),
    "q3a_last_error": (ctypes.c_char_p, []),
    "q3a_paged_decode": (_c_int, [
        _c_vp, _c_i64, _c_i64,                      # q, q_stride_b, q_stride_h
        _c_vp, _c_vp, _c_i64, _c_i64, _c_i64,       # k_cache, v_cache, kv strides (page, tok, head)
        _c_int, _c_int,                             # num_pages, page_size
        _c_vp, _c_vp, _c_i64, _c_int,               # cache_seqlens, block_table, bt_stride_b, max_pages
        _c_vp, _c_i64, _c_i64,                      # out, o_stride_b, o_stride_h
        _c_vp, _c_size,                             # workspace, workspace_bytes
        _c_int, _c_int, _c_int, _c_int,             # batch, Hq, Hkv, D
        _c_float, _c_int, _c_vp,                    # softmax_scale, split_tokens, stream
    ]),
    "q3a_paged_decode_append": (_c_int, [
        _c_vp, _c_i64, _c_i64,                      # q, q_stride_b, q_stride_h
        _c_vp, _c_i64, _c_vp, _c_i64,               # k_new, kn_stride_b, v_new, vn_stride_b
        _c_vp, _c_vp, _c_i64, _c_i64, _c_i64,       # k_cache, v_cache, kv strides (page, tok, head)
        _c_int, _c_int,                             # num_pages, page_size
        _c_vp, _c_vp, _c_i64, _c_int,               # cache_seqlens, block_table, bt_stride_b, max_pages
        _c_vp, _c_i64, _c_i64,                      # out, o_stride_b, o_stride_h
        _c_vp, _c_size,                             # workspace, workspace_bytes
        _c_int, _c_int, _c_int, _c_int,             # batch, Hq, Hkv, D
        _c_float, _c_int, _c_vp,                    # softmax_scale, split_tokens, stream
    ]),
    "q3a_paged_decode_append_rope": (_c_int, [
        _c_vp, _c_i64, _c_i64,                      # q, q_stride_b, q_stride_h
        _c_vp, _c_i64, _c_vp, _c_i64,               # k_new, kn_stride_b, v_new, vn_stride_b
        _c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_float,  # q_norm_w, k_norm_w, cos, sin, cs_stride_b, eps
        _c_vp, _c_vp, _c_i64, _c_i64, _c_i64,       # k_cache, v_cache, kv strides (page, tok, head)
        _c_int, _c_int,                             # num_pages, page_size
        _c_vp, _c_vp, _c_i64, _c_int,               # cache_seqlens, block_table, bt_stride_b, max_pages
        _c_vp, _c_i64, _c_i64,                      # out, o_stride_b, o_stride_h
        _c_vp, _c_size,                             # workspace, workspace_bytes
        _c_int, _c_int, _c_int, _c_int,             # batch, Hq, Hkv, D
        _c_float, _c_int, _c_vp,                    # softmax_scale, split_tokens, stream
    ]),
    "q3a_paged_decode_noalloc": (_c_int, [
        _c_vp, _c_i64, _c_i64,                      # q, q_stride_b, q_stride_h
        _c_vp, _c_vp, _c_i64, _c_i64, _c_i64,       # k_cache, v_cache, kv strides (page, tok, head)
        _c_int, _c_int,                             # num_pages, page_size
        _c_vp, _c_vp, _c_i64, _c_int,               # cache_seqlens, block_table, bt_stride_b, max_pages
        _c_vp, _c_i64, _c_i64,                      # out, o_stride_b, o_stride_h
        _c_int, _c_int, _c_int, _c_int,             # batch, Hq, Hkv, D
        _c_float, _c_int, _c_vp,                    # softmax_scale, split_tokens, stream
    ]),
    "q3a_paged_decode_workspace_bytes": (_c_size, [_c_int] * 7),
    "q3a_paged_decode_plan_bytes": (_c_size, [_c_int] * 4),
    "q3a_paged_decode_plan": (_c_int, [
        _c_vp, _c_vp, _c_i64, _c_i64, _c_int,       # cache_seqlens, block_table, bt strides (row, table), num_tables
        _c_int, _c_int, _c_int, _c_int, _c_int,     # max_pages, page_size, batch, Hkv, form
        _c_vp, _c_i64, _c_size, _c_vp,              # plans, plan_stride, plans_bytes, stream
    ]),
    "q3a_paged_decode_default_split": (_c_int, [_c_int] * 4),
    "q3a_cp_attn": (_c_int, [
        _c_vp, _c_i64,                                         # q, q_stride_b
        _c_vp, _c_i64, _c_i64, _c_i64,                         # k, k strides (b, h, s)
        _c_vp, _c_i64, _c_i64, _c_i64,                         # v, v strides (b, h, s)
        _c_vp, _c_i64,                                         # out, o_stride_b
        _c_int, _c_int, _c_int, _c_int, _c_int,                # batch, Hq, Hkv, D, n_live
        _c_float, _c_vp,                                       # softmax_scale, stream
    ]),
    "q3a_cp_attn_append": (_c_int, [
        _c_vp, _c_i64, _c_vp, _c_i64, _c_vp, _c_i64,           # q, q_sb, k_new, kn_sb, v_new, vn_sb
        _c_vp, _c_i64, _c_i64, _c_i64,                         # k, k strides (b, h, s)
        _c_vp, _c_i64, _c_i64, _c_i64,                         # v, v strides (b, h, s)
        _c_vp, _c_i64,                                         # out, o_stride_b
        _c_int, _c_int, _c_int, _c_int, _c_int,                # batch, Hq, Hkv, D, n_live
        _c_float, _c_vp,                                       # softmax_scale, stream
    ]),
    "q3a_prefill": (_c_int, [
        _c_vp, _c_i64, _c_i64, _c_vp,                          # q, q_stride_t, q_stride_h, cu_seqlens_q
        _c_vp, _c_i64, _c_i64, _c_i64,                         # k, k strides (page, tok, head)
        _c_vp, _c_i64, _c_i64, _c_i64,                         # v, v strides (page, tok, head)
        _c_int, _c_int, _c_vp, _c_i64, _c_int,                 # num_pages, page_size, block_table, bt stride, max pages
        _c_vp, _c_vp, _c_i64, _c_i64,                          # cu_seqlens_k, out, o_stride_t, o_stride_h
        _c_int, _c_int, _c_int, _c_int, _c_int,                # num_seqs, max_seqlen_q, Hq, Hkv, D
        _c_float, _c_int, _c_vp,                               # softmax_scale, causal, stream
    ]),
    "q3a_prefill_append": (_c_int, [
        _c_vp, _c_i64, _c_i64, _c_vp,                          # q, q_stride_t, q_stride_h, cu_seqlens_q
        _c_vp, _c_i64, _c_i64, _c_vp, _c_i64, _c_i64,          # k, k strides (tok, head), v, v strides (tok, head)
        _c_vp,                                                 # cu_seqlens_k
        _c_vp, _c_vp, _c_i64, _c_i64, _c_i64,                  # k_cache, v_cache, cache strides (page, tok, head)
        _c_int, _c_int, _c_vp, _c_i64, _c_int,                 # num_pages, page_size, block_table, bt stride, max pages
        _c_vp, _c_i64, _c_i64,                                 # out, o_stride_t, o_stride_h
        _c_int, _c_int, _c_int, _c_int, _c_int,                # num_seqs, max_seqlen_q, Hq, Hkv, D
        _c_float, _c_int, _c_vp,                               # softmax_scale, causal, stream
    ]),
    "q3a_prefill_dense": (_c_int, [
        _c_vp, _c_i64, _c_i64, _c_i64,                         # q, q strides (seq, tok, head)
        _c_vp, _c_i64, _c_i64, _c_i64,                         # k, k strides (seq, tok, head)
        _c_vp, _c_i64, _c_i64, _c_i64,                         # v, v strides (seq, tok, head)
        _c_vp, _c_i64, _c_i64, _c_i64,                         # out, o strides (seq, tok, head)
        _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,        # num_seqs, seqlen_q, seqlen_k, Hq, Hkv, D
        _c_float, _c_int, _c_vp,                               # softmax_scale, causal, stream
    ]),
    "q3a_prefill_dense_append_rope_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int, _c_int, _c_int, _c_int]),
    "q3a_prefill_dense_append_rope": (_c_int, [
        _c_vp, _c_i64, _c_i64, _c_i64,                         # q (raw), strides (seq, tok, head)
        _c_vp, _c_i64, _c_i64, _c_i64,                         # k (raw new keys), strides
        _c_vp, _c_i64, _c_i64, _c_i64,                         # v (new values), strides
        _c_vp, _c_i64, _c_i64, _c_i64,                         # prefix_k, strides (prefix, tok, head)
        _c_vp, _c_i64, _c_i64, _c_i64,                         # prefix_v, strides
        _c_vp, _c_i64,                                         # prefix_index (int64 or NULL), num_prefixes
        _c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_float,          # q/k norm weights, cos, sin, rope row stride, eps
        _c_vp, _c_vp, _c_i64, _c_i64, _c_i64,                  # k_cache, v_cache, cache strides (page, tok, head)
        _c_int, _c_int, _c_vp, _c_i64, _c_int,                 # num_pages, page_size, block_table, bt stride, max pages
        _c_int,                                                # first_row
        _c_vp, _c_i64, _c_i64, _c_i64,                         # out, o strides (seq, tok, head)
        _c_vp, _c_size,                                        # workspace, workspace bytes
        _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,        # num_seqs, seqlen_q, prefix_len, Hq, Hkv, D
        _c_float, _c_int, _c_vp,                               # softmax_scale, causal, stream
    ]),
    "q3a_cp_attn_append_rope": (_c_int, [
        _c_vp, _c_i64, _c_vp, _c_i64, _c_vp, _c_i64,          # q (raw), row stride, k_new (raw), stride, v_new, stride
        _c_vp, _c_vp, _c_vp, _c_vp, _c_float,                  # q/k norm weights, cos, sin rows, eps
        _c_vp, _c_i64, _c_i64, _c_i64,                         # K scratch, strides (row, head, slot)
        _c_vp, _c_i64, _c_i64, _c_i64,                         # V scratch, strides
        _c_vp, _c_i64,                                         # out, row stride
        _c_int, _c_int, _c_int, _c_int, _c_int, _c_float, _c_vp,  # B, Hq, Hkv, D, n_live, scale, stream
    ]),
    "q3a_prefill_append_rope_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int, _c_int]),
    "q3a_prefill_append_rope": (_c_int, [
        _c_vp, _c_i64, _c_i64, _c_vp, _c_i64, _c_i64,          # q (raw), strides (tok, head), k (raw), strides
        _c_vp, _c_i64, _c_i64,                                 # v, strides
        _c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_float,          # q/k norm weights, cos, sin, rope row stride, eps
        _c_vp,                                                 # cu_seqlens
        _c_vp, _c_vp, _c_i64, _c_i64, _c_i64,                  # k_cache, v_cache, cache strides (page, tok, head)
        _c_int, _c_int, _c_vp, _c_i64, _c_int,                 # num_pages, page_size, block_table, bt stride, max pages
        _c_vp, _c_i64, _c_i64,                                 # out, o_stride_t, o_stride_h
        _c_vp, _c_size,                                        # workspace, workspace bytes
        _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,        # num_seqs, total_tokens, max_seqlen, Hq, Hkv, D
        _c_float, _c_int, _c_vp,                               # softmax_scale, causal, stream
    ]),
    "q3a_prefill_dense_append": (_c_int, [
        _c_vp, _c_i64, _c_i64, _c_i64,                         # q, q strides (seq, tok, head)
        _c_vp, _c_i64, _c_i64, _c_i64,                         # k, k strides (seq, tok, head)
        _c_vp, _c_i64, _c_i64, _c_i64,                         # v, v strides (seq, tok, head)
        _c_vp, _c_vp, _c_i64, _c_i64, _c_i64,                  # k_cache, v_cache, cache strides (page, tok, head)
        _c_int, _c_int, _c_vp, _c_i64, _c_int,                 # num_pages, page_size, block_table, bt stride, max pages
        _c_int,                                                # first_row
        _c_vp, _c_i64, _c_i64, _c_i64,                         # out, o strides (seq, tok, head)
        _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,        # num_seqs, seqlen_q, seqlen_k, Hq, Hkv, D
        _c_float, _c_int, _c_vp,                               # softmax_scale, causal, stream
    ]),
}

_lock = threading.Lock()
_lib = None


class Q3AttnError(RuntimeError):
    pass


def lib() -> ctypes.CDLL:
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise Q3AttnError(
                    f"q3attn: HIP library not found at {LIB_PATH}; build it first "
                    "(python qwen3-tts-engine_amd/build.py or __graft_entry__.build())")
            handle = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            ver = handle.q3a_abi_version()
            if ver != ABI_VERSION:
                raise Q3AttnError(f"q3attn: library ABI {ver} != expected {ABI_VERSION}; rebuild")
            _lib = handle
    return _lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().q3a_last_error().decode(errors="replace")
        raise Q3AttnError(f"{what} failed ({rc}): {msg}")
