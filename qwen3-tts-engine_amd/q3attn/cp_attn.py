"""The code predictor's 16-slot causal attention as one HIP kernel per call.

``cp_attn(q, K, V, n_live, scale)`` keeps the signature and layouts of engine/cp_attn.py:33-39
(the attention of ``CodePredictor._post``, engine/code_predictor.py:46-47): q [B, 16, 128] or
[B, 2048], K/V [B, 8, 16, 128] bf16 whose batch stride may exceed the live batch, ``n_live`` =
p + 1 live slots -> o [B, 2048] bf16.  Scores and softmax are float32, probabilities are rounded
to bf16 before P.V, P.V accumulates in float32.  GPU only.
"""
from __future__ import annotations

import torch

from ._lib import check, lib


def _req(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


@torch.library.custom_op("q3attn::cp_attn", mutates_args=())
def cp_attn_op(q: torch.Tensor, K: torch.Tensor, V: torch.Tensor, n_live: int, scale: float) -> torch.Tensor:
    _req(q.is_cuda, "q3attn.cp_attn: tensors must be on a GPU (there is no CPU path)")
    _req(K.device == q.device and V.device == q.device, "q3attn.cp_attn: q, K, V must share a device")
    _req(q.dtype == torch.bfloat16 and K.dtype == torch.bfloat16 and V.dtype == torch.bfloat16,
         "q3attn.cp_attn: q, K, V must be bfloat16")
    _req(K.dim() == 4 and K.shape == V.shape and K.stride() == V.stride(),
         "q3attn.cp_attn: K and V must be [B, kv_heads, slots, head_dim] with equal strides")
    B, Hkv, S, D = K.shape
    _req(K.stride(3) == 1, "q3attn.cp_attn: K/V head_dim must be contiguous")
    _req(1 <= n_live <= S, f"q3attn.cp_attn: n_live {n_live} outside [1, {S}]")
    q2 = q.reshape(q.shape[0], -1)
    _req(q2.shape[0] == B and q2.shape[1] % D == 0, "q3attn.cp_attn: q and K batch/head_dim mismatch")
    _req(q2.stride(1) == 1, "q3attn.cp_attn: q rows must be contiguous")
    Hq = q2.shape[1] // D
    out = torch.empty((B, Hq * D), dtype=q.dtype, device=q.device)
    if B == 0:
        return out
    rc = lib().q3a_cp_attn(
        q2.data_ptr(), q2.stride(0), K.data_ptr(), V.data_ptr(), K.stride(0), K.stride(1), K.stride(2),
        out.data_ptr(), out.stride(0), B, Hq, Hkv, D, int(n_live), float(scale),
        torch.cuda.current_stream(q.device).cuda_stream)
    check(rc, "q3a_cp_attn")
    return out


@cp_attn_op.register_fake
def _cp_attn_fake(q, K, V, n_live, scale):
    B = q.shape[0]
    return q.new_empty((B, q.numel() // max(B, 1) if B else K.shape[1] * 2 * K.shape[3]))


def cp_attn(q, K, V, n_live, scale):
    """q [B,16,128] (or [B,2048]), K/V [B,8,16,128] (row stride may exceed the live batch),
    n_live = p + 1 -> o [B,2048].  engine/cp_attn.py:33-39."""
    return cp_attn_op(q, K, V, int(n_live), float(scale))
