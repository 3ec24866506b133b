"""The code predictor's 16-slot causal attention as one HIP kernel per call.

``cp_attn(q, K, V, n_live, scale)`` keeps the signature and layouts of engine/cp_attn.py:33-39
(the attention of ``CodePredictor._post``, engine/code_predictor.py:46-47): q [B, 16, 128] or
[B, 2048], K/V [B, 8, 16, 128] bf16 whose batch stride may exceed the live batch, ``n_live`` =
p + 1 live slots -> o [B, 2048] bf16.  Scores and softmax are float32, probabilities are rounded
to bf16 before P.V, P.V accumulates in float32.  GPU only.

``cp_attn_append(q, k, v, K, V, p, scale)`` is the slot write of engine/code_predictor.py:58
(``K.index_copy_(2, p, k.unsqueeze(2))`` and the same for V) fused with that attention over
n_live = p + 1 slots: one launch instead of three.  ``cp_attn_append_rope`` takes q and k raw and applies the
q/k RMSNorm + RoPE of ``_pre`` (engine/code_predictor.py:38-43) in the same launch.
"""
from __future__ import annotations

import torch

from ._lib import check, lib


def _req(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


@torch.library.custom_op("q3attn::cp_attn", mutates_args=())
def cp_attn_op(q: torch.Tensor, K: torch.Tensor, V: torch.Tensor, n_live: int, scale: float) -> torch.Tensor:
    q2, B, Hkv, D, Hq = _check_common(q, K, V, n_live, "cp_attn")
    out = torch.empty((B, Hq * D), dtype=q.dtype, device=q.device)
    if B == 0:
        return out
    rc = lib().q3a_cp_attn(
        q2.data_ptr(), q2.stride(0), K.data_ptr(), K.stride(0), K.stride(1), K.stride(2),
        V.data_ptr(), V.stride(0), V.stride(1), V.stride(2),
        out.data_ptr(), out.stride(0), B, Hq, Hkv, D, int(n_live), float(scale),
        torch.cuda.current_stream(q.device).cuda_stream)
    check(rc, "q3a_cp_attn")
    return out


def _check_common(q, K, V, n_live, who):
    _req(q.is_cuda, f"q3attn.{who}: tensors must be on a GPU (there is no CPU path)")
    _req(K.device == q.device and V.device == q.device, f"q3attn.{who}: q, K, V must share a device")
    _req(q.dtype == torch.bfloat16 and K.dtype == torch.bfloat16 and V.dtype == torch.bfloat16,
         f"q3attn.{who}: q, K, V must be bfloat16")
    _req(K.dim() == 4 and K.shape == V.shape, f"q3attn.{who}: K and V must be [B, kv_heads, slots, head_dim]")
    B, Hkv, S, D = K.shape
    _req(K.stride(3) == 1 and V.stride(3) == 1, f"q3attn.{who}: K/V head_dim must be contiguous")
    _req(1 <= n_live <= S, f"q3attn.{who}: n_live {n_live} outside [1, {S}]")
    q2 = q.reshape(q.shape[0], -1)
    _req(q2.shape[0] == B and q2.shape[1] % D == 0, f"q3attn.{who}: q and K batch/head_dim mismatch")
    _req(q2.stride(1) == 1, f"q3attn.{who}: q rows must be contiguous")
    return q2, B, Hkv, D, q2.shape[1] // D


def _new_rows(x, B, Hkv, D, name):
    if x.dim() == 2:
        x = x.view(x.shape[0], Hkv, D)
    _req(x.dtype == torch.bfloat16, f"q3attn.cp_attn_append: {name} must be bfloat16")
    _req(tuple(x.shape) == (B, Hkv, D), f"q3attn.cp_attn_append: {name} must be [B, {Hkv}, {D}]")
    _req(x.stride(2) == 1 and x.stride(1) == D, f"q3attn.cp_attn_append: {name} heads must be packed rows")
    return x


@torch.library.custom_op("q3attn::cp_attn_append", mutates_args=("K", "V"))
def cp_attn_append_op(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, K: torch.Tensor, V: torch.Tensor,
                      p: int, scale: float) -> torch.Tensor:
    q2, B, Hkv, D, Hq = _check_common(q, K, V, int(p) + 1, "cp_attn_append")
    _req(k.device == q.device and v.device == q.device, "q3attn.cp_attn_append: k, v must share q's device")
    k3 = _new_rows(k, B, Hkv, D, "k")
    v3 = _new_rows(v, B, Hkv, D, "v")
    out = torch.empty((B, Hq * D), dtype=q.dtype, device=q.device)
    if B == 0:
        return out
    rc = lib().q3a_cp_attn_append(
        q2.data_ptr(), q2.stride(0), k3.data_ptr(), k3.stride(0), v3.data_ptr(), v3.stride(0),
        K.data_ptr(), K.stride(0), K.stride(1), K.stride(2), V.data_ptr(), V.stride(0), V.stride(1), V.stride(2),
        out.data_ptr(), out.stride(0), B, Hq, Hkv, D, int(p) + 1, float(scale),
        torch.cuda.current_stream(q.device).cuda_stream)
    check(rc, "q3a_cp_attn_append")
    return out


@cp_attn_append_op.register_fake
def _cp_attn_append_fake(q, k, v, K, V, p, scale):
    return q.new_empty((q.shape[0], K.shape[1] * 2 * K.shape[3]))


@cp_attn_op.register_fake
def _cp_attn_fake(q, K, V, n_live, scale):
    B = q.shape[0]
    return q.new_empty((B, q.numel() // max(B, 1) if B else K.shape[1] * 2 * K.shape[3]))


def cp_attn(q, K, V, n_live, scale):
    """q [B,16,128] (or [B,2048]), K/V [B,8,16,128] (row stride may exceed the live batch),
    n_live = p + 1 -> o [B,2048].  engine/cp_attn.py:33-39."""
    return cp_attn_op(q, K, V, int(n_live), float(scale))


def cp_attn_append(q, k, v, K, V, p, scale):
    """Slot write + attention of one code-predictor step (engine/code_predictor.py:58 then :46-47):
    K[:, :, p] = k, V[:, :, p] = v (k, v [B, 8, 128], v may be a view into the qkv projection), then
    attention over slots 0..p -> o [B, 2048]."""
    return cp_attn_append_op(q, k, v, K, V, int(p), float(scale))


@torch.library.custom_op("q3attn::cp_attn_append_rope", mutates_args=("K", "V"))
def cp_attn_append_rope_op(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, K: torch.Tensor, V: torch.Tensor,
                           p: int, scale: float, q_norm_w: torch.Tensor, k_norm_w: torch.Tensor, cos: torch.Tensor,
                           sin: torch.Tensor, eps: float) -> torch.Tensor:
    q2, B, Hkv, D, Hq = _check_common(q, K, V, int(p) + 1, "cp_attn_append_rope")
    dev = q.device
    for name, t in (("k", k), ("v", v), ("q_norm_w", q_norm_w), ("k_norm_w", k_norm_w), ("cos", cos), ("sin", sin)):
        _req(t.device == dev, f"q3attn.cp_attn_append_rope: {name} must be on q's device")
    k3 = _new_rows(k, B, Hkv, D, "k")
    v3 = _new_rows(v, B, Hkv, D, "v")
    for name, t in (("q_norm_w", q_norm_w), ("k_norm_w", k_norm_w), ("cos", cos), ("sin", sin)):
        _req(t.dtype == torch.bfloat16 and t.numel() == D and t.is_contiguous(),
             f"q3attn.cp_attn_append_rope: {name} must be a contiguous bfloat16 row of {D}")
    out = torch.empty((B, Hq * D), dtype=q.dtype, device=dev)
    if B == 0:
        return out
    rc = lib().q3a_cp_attn_append_rope(
        q2.data_ptr(), q2.stride(0), k3.data_ptr(), k3.stride(0), v3.data_ptr(), v3.stride(0),
        q_norm_w.data_ptr(), k_norm_w.data_ptr(), cos.data_ptr(), sin.data_ptr(), float(eps),
        K.data_ptr(), K.stride(0), K.stride(1), K.stride(2), V.data_ptr(), V.stride(0), V.stride(1), V.stride(2),
        out.data_ptr(), out.stride(0), B, Hq, Hkv, D, int(p) + 1, float(scale), torch.cuda.current_stream(dev).cuda_stream)
    check(rc, "q3a_cp_attn_append_rope")
    return out


@cp_attn_append_rope_op.register_fake
def _cp_attn_append_rope_fake(q, k, v, K, V, p, scale, q_norm_w, k_norm_w, cos, sin, eps):
    return q.new_empty((q.shape[0], K.shape[1] * 2 * K.shape[3]))


def cp_attn_append_rope(q, k, v, K, V, p, scale, q_norm_w, k_norm_w, cos, sin, eps=1e-6):
    """One code-predictor step's attention block (engine/code_predictor.py:38-43, 58, 46-47) in one launch: q
    [B, 16, 128] and k [B, 8, 128] arrive raw (views of the qkv projection), are RMS-normalised with q_norm_w /
    k_norm_w and rotated with slot p's cos/sin row ([128], W.cp_cos[p]) as the compiled _pre evaluates them (the rope
    rounded once), k and v go into slot p of K/V [B, 8, 16, 128], and the attention over slots 0..p -> o [B, 2048]."""
    return cp_attn_append_rope_op(q, k, v, K, V, int(p), float(scale), q_norm_w, k_norm_w, cos.reshape(-1),
                                  sin.reshape(-1), float(eps))
