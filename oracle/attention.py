"""CPU oracle for the Qwen3-TTS attention hot path.

TEST INFRASTRUCTURE ONLY.  This module is the checker, never the product: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may import it.  The
product path (``q3attn``) never calls it and raises when its HIP library is missing.

Every function restates the arithmetic of one reference function (cited ``file:line`` in the
reference engine) in plain numpy, on float32 arrays that hold bf16-exact values.  ``acc`` selects
the accumulation precision (float32, like the reference's fp32 parity path, or float64 for
brute-force checks).

Pinning (what independent check fixes each function; see tests/test_oracle.py):

* ``paged_decode``      -- float64 scalar-loop brute force on tiny shapes; torch CPU
                           ``scaled_dot_product_attention(enable_gqa=True)`` (a library routine);
                           closed forms: ctx=1 -> V[tok0], constant V -> V, identical keys ->
                           mean(V); page-table permutation invariance; identity table of
                           page size 256 == the reference's contiguous-slot gather.
* ``cp_attn_torch_path``-- torch CPU bf16 ops executing the same op sequence (bf16 matmul,
                           bf16 scale, bf16 mask add, fp32 softmax, bf16 P, bf16 matmul);
                           n_live=1 -> V[slot 0]; within tolerance of the float64 closed form.
* ``cp_attn_triton_path``-- n_live=1 -> V[slot 0]; NaN-poisoned stale slots leave the output
                           unchanged; within tolerance of the float64 closed form.
* ``prefill_varlen``    -- torch CPU SDPA ``is_causal=True`` per sequence; float64 brute force.
* ``prefill_prefix``    -- R == n reduces to ``prefill_varlen``; brute force float64; causal=False
                           against torch CPU SDPA without a mask.
* ``rms`` / ``rope``    -- unit-RMS invariant; RoPE at position 0 is the identity; RoPE preserves
                           the norm of each rotated pair; relative-position invariance of q.k.
* ``norm_rope``         -- eager form: bit for bit against torch's CPU bf16 kernels running
                           engine/ops.py:51-60 (rows of RMS 1e-4..10, so eps matters); planted
                           mistakes (weight before the cast, no eps, swapped halves, cos/sin
                           swapped) fail that check.  Compiled form: equal to the same chain in
                           float64 rounded once up to double roundings, within one bf16 unit.
* ``rope_tables``       -- closed-form frequencies (theta**(-2i/D)) checked at chosen indices.
"""
from __future__ import annotations

import math

import numpy as np

NEG_INF = np.float32(-np.inf)


# ----------------------------------------------------------------------------- bf16 helpers
def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round float32 -> bf16 (round to nearest, ties to even); returns the uint16 bit patterns."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    lsb = (u >> np.uint32(16)) & np.uint32(1)
    r = ((u + np.uint32(0x7FFF) + lsb) >> np.uint32(16)).astype(np.uint16)
    nan = np.isnan(np.asarray(x, dtype=np.float32))
    if nan.any():
        r = np.where(nan, ((u >> np.uint32(16)) | np.uint32(0x40)).astype(np.uint16), r)
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 values rounded onto the bf16 grid (what ``tensor.to(torch.bfloat16)`` stores)."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


# ----------------------------------------------------------------------------- input producers
def rope_tables(n_pos: int, head_dim: int = 128, theta: float = 1.0e6):
    """cos/sin tables [n_pos, head_dim] in float32.

    The reference takes them from the upstream rotary module (engine/model_load.py:48-52, 62-63):
    inv_freq[i] = theta**(-2i/D), angle = pos * inv_freq, table = cat(angle, angle).
    """
    inv = 1.0 / (theta ** (np.arange(0, head_dim, 2, dtype=np.float64) / head_dim))
    ang = np.arange(n_pos, dtype=np.float64)[:, None] * inv[None, :]
    emb = np.concatenate([ang, ang], axis=-1)
    return np.cos(emb).astype(np.float32), np.sin(emb).astype(np.float32)


def rms(x: np.ndarray, w: np.ndarray | None = None, eps: float = 1e-6, to_bf16: bool = True) -> np.ndarray:
    """Qwen3 RMSNorm (engine/ops.py:51-55): normalise in float32, cast back, then scale."""
    xf = x.astype(np.float32)
    y = xf / np.sqrt((xf * xf).mean(-1, keepdims=True) + np.float32(eps))
    y = y.astype(np.float32)
    if to_bf16:
        y = bf16_round(y)
    return y if w is None else (w * y).astype(np.float32)


def rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """Rotate-half RoPE (engine/ops.py:58-60): x*cos + cat(-x[h:], x[:h])*sin."""
    h = x.shape[-1] // 2
    rot = np.concatenate([-x[..., h:], x[..., :h]], axis=-1)
    return (x * cos + rot * sin).astype(np.float32)


def _rsqrt_mean_sq(xf: np.ndarray, eps: float) -> np.ndarray:
    """1 / sqrt(mean(x^2) + eps) over the last axis in float32 (``torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) +
    eps)``, engine/ops.py:53), numpy's summation order."""
    ms = (xf * xf).mean(-1, keepdims=True, dtype=np.float32)
    return np.float32(1.0) / np.sqrt(ms + np.float32(eps), dtype=np.float32)


def _normalise(xf: np.ndarray, r: np.ndarray) -> np.ndarray:
    """``(xf * r).to(x.dtype)`` (engine/ops.py:53-54): the product rounded to bf16."""
    return bf16_round(xf * r)


def _rotate_half(y: np.ndarray) -> np.ndarray:
    """``torch.cat((-y[..., h:], y[..., :h]), dim=-1)`` (engine/ops.py:59)."""
    h = y.shape[-1] // 2
    return np.concatenate([-y[..., h:], y[..., :h]], axis=-1)


def norm_rope(x: np.ndarray, w: np.ndarray, cos: np.ndarray, sin: np.ndarray, eps: float = 1e-6,
              eager: bool = True) -> np.ndarray:
    """The talker's q/k producers on bf16 head rows: ``rope(rms(x, w), cos, sin)`` (engine/ops.py:51-60, called at
    engine/talker.py:69-70, 158-159 and engine/arrivals.py:112-118).  x, w, cos, sin hold bf16 values; the result is
    bf16 values in float32.

    rms: r = 1 / sqrt(mean(x^2) + eps) in float32, n = (x * r).to(bf16) (the explicit cast), y = w * n.
    rope: y * cos + cat(-y[h:], y[:h]) * sin.
    * eager=True -- eager torch bf16 ops (``prefill_hidden`` and the admission layer are not compiled,
      engine/arrivals.py:57-61): every op rounds its result, y = bf16(w * bf16(x * r)),
      o = bf16(bf16(y cos) + bf16(rot(y) sin)).  Torch's CPU bf16 kernels give these bits exactly.
    * eager=False -- the chain as torch.compile's GPU kernels evaluate it for the compiled callers (``Talker._decode``,
      ``CodePredictor._pre``, engine/talker.py:56-59, engine/code_predictor.py:25-29): every intermediate stays in
      float32, the cast inside rms included, and the result is rounded once: y = w * (x * r),
      o = bf16(y cos + rot(y) sin), each product and the sum a separate float32 operation (measured on MI355X: the
      compiled producers equal this on every element of 262,144).
    The mean of squares is summed in numpy's order; another order moves mean(x^2) by an fp32 unit, which can move the
    result by a bf16 unit on rare elements."""
    xf = np.asarray(x, np.float32)
    r = _rsqrt_mean_sq(xf, eps)
    if eager:
        y = bf16_round(np.asarray(w, np.float32) * _normalise(xf, r))
        return bf16_round(bf16_round(y * cos) + bf16_round(_rotate_half(y) * sin))
    y = (np.asarray(w, np.float32) * (xf * r).astype(np.float32)).astype(np.float32)
    return bf16_round((y * cos + _rotate_half(y) * sin).astype(np.float32))


# ----------------------------------------------------------------------------- talker decode
def gather_seat(cache: np.ndarray, block_table_row: np.ndarray, ctx: int) -> np.ndarray:
    """Tokens 0..ctx-1 of one seat: token t lives at page bt[t // page], offset t % page.

    The reference's identity table (engine/talker.py:42) makes this the contiguous slot range
    [seat*seat_len, seat*seat_len + ctx) that ``_attn_ref`` slices (engine/talker.py:85).
    """
    page = cache.shape[1]
    t = np.arange(ctx)
    pages = np.asarray(block_table_row, dtype=np.int64)[t // page]
    return cache[pages, t % page]                    # [ctx, Hkv, D]


def paged_decode(q, k_cache, v_cache, seqlens, block_table, scale, acc=np.float32):
    """Single-query attention of every row over its paged context.

    Restates ``Talker._attn_ref`` (engine/talker.py:82-88): per row b, q[b] viewed as
    [Hkv, Hq/Hkv, D] (q head h reads kv head h // (Hq/Hkv)), a = q.K^T * scale, softmax over the
    ctx tokens, o = softmax(a).V -- here with the tokens gathered through ``block_table`` as
    flash_attn_with_kvcache does at engine/talker.py:77.  Rows with ctx == 0 produce zeros (a
    convention of this build; the reference never issues them).

    q [B, Hq, D]; k_cache, v_cache [num_pages, page, Hkv, D]; seqlens [B]; block_table [B, P].
    Returns [B, Hq, D] in ``acc``.
    """
    B, Hq, D = q.shape
    Hkv = k_cache.shape[2]
    G = Hq // Hkv
    out = np.zeros((B, Hq, D), dtype=acc)
    for b in range(B):
        ctx = int(seqlens[b])
        if ctx <= 0:
            continue
        K = gather_seat(k_cache, block_table[b], ctx).astype(acc).transpose(1, 0, 2)   # [Hkv, ctx, D]
        V = gather_seat(v_cache, block_table[b], ctx).astype(acc).transpose(1, 0, 2)
        qb = q[b].astype(acc).reshape(Hkv, G, D)
        a = np.matmul(qb, K.transpose(0, 2, 1)) * acc(scale)                          # [Hkv, G, ctx]
        a = a - a.max(-1, keepdims=True)
        p = np.exp(a)
        p = p / p.sum(-1, keepdims=True)
        out[b] = np.matmul(p, V).reshape(Hq, D)
    return out


def paged_decode_bruteforce(q, k_cache, v_cache, seqlens, block_table, scale):
    """float64 scalar-loop restatement (math.exp, explicit sums) for tiny shapes only."""
    B, Hq, D = q.shape
    Hkv = k_cache.shape[2]
    page = k_cache.shape[1]
    G = Hq // Hkv
    out = np.zeros((B, Hq, D), dtype=np.float64)
    for b in range(B):
        ctx = int(seqlens[b])
        for h in range(Hq):
            g = h // G
            s = []
            for t in range(ctx):
                pg = int(block_table[b][t // page])
                k = k_cache[pg, t % page, g]
                s.append(sum(float(q[b, h, d]) * float(k[d]) for d in range(D)) * scale)
            if not s:
                continue
            m = max(s)
            e = [math.exp(x - m) for x in s]
            z = sum(e)
            for d in range(D):
                out[b, h, d] = sum(e[t] * float(v_cache[int(block_table[b][t // page]), t % page, g, d])
                                   for t in range(ctx)) / z
    return out


# ----------------------------------------------------------------------------- code predictor
def cp_attn_torch_path(q, K, V, n_live, scale):
    """The 16-slot causal attention exactly as ``CodePredictor._post`` computes it in bf16.

    engine/code_predictor.py:46-47 with mask row p = n_live - 1 (engine/code_predictor.py:22-23):
      att = bf16(q . K^T)          -- bf16 matmul, fp32 accumulate, bf16 result
      att = bf16(att * scale)      -- bf16 tensor times a Python float
      att = bf16(att + mask)       -- -inf at slots > p
      P   = bf16(softmax(float32(att)))
      o   = bf16(P . V)            -- bf16 matmul, fp32 accumulate
    q [B, Hq, D]; K, V [B, Hkv, S, D] (S = 16 slots).  Returns o [B, Hq*D] (float32 on the bf16 grid).
    """
    B, Hq, D = q.shape
    Hkv, S = K.shape[1], K.shape[2]
    G = Hq // Hkv
    qh = q.astype(np.float32).reshape(B, Hkv, G, D)
    att = bf16_round(np.matmul(qh, K.astype(np.float32).transpose(0, 1, 3, 2)))        # [B,Hkv,G,S]
    att = bf16_round(att * np.float32(scale))
    mask = np.where(np.arange(S) > (n_live - 1), NEG_INF, np.float32(0.0))
    att = bf16_round(att + mask)
    att = att - att.max(-1, keepdims=True)
    e = np.exp(att)
    p = bf16_round((e / e.sum(-1, keepdims=True)).astype(np.float32))
    o = bf16_round(np.matmul(p, V.astype(np.float32)))                                 # [B,Hkv,G,D]
    return o.reshape(B, Hq * D)


def cp_attn_triton_path(q, K, V, n_live, scale):
    """``_cp_attn_kernel`` (engine/cp_attn.py:13-30): scores and softmax in float32 over the n_live
    live slots (loads masked with 0, scores masked with -inf), P rounded to bf16, P.V in float32,
    output rounded to bf16.  Returns o [B, Hq*D]."""
    B, Hq, D = q.shape
    Hkv, S = K.shape[1], K.shape[2]
    G = Hq // Hkv
    live = np.arange(S) < n_live
    Kl = np.where(live[None, None, :, None], K.astype(np.float32), np.float32(0.0))
    Vl = np.where(live[None, None, :, None], V.astype(np.float32), np.float32(0.0))
    qh = q.astype(np.float32).reshape(B, Hkv, G, D)
    att = np.matmul(qh, Kl.transpose(0, 1, 3, 2)) * np.float32(scale)
    att = np.where(live, att, NEG_INF)
    att = att - att.max(-1, keepdims=True)
    e = np.exp(att)
    p = bf16_round((e / e.sum(-1, keepdims=True)).astype(np.float32))
    o = bf16_round(np.matmul(p, Vl))
    return o.reshape(B, Hq * D)


def cp_attn_exact(q, K, V, n_live, scale):
    """float64 closed form of the same attention (no intermediate rounding)."""
    B, Hq, D = q.shape
    Hkv = K.shape[1]
    G = Hq // Hkv
    qh = q.astype(np.float64).reshape(B, Hkv, G, D)
    Kl = K[:, :, :n_live].astype(np.float64)
    Vl = V[:, :, :n_live].astype(np.float64)
    a = np.matmul(qh, Kl.transpose(0, 1, 3, 2)) * scale
    a = a - a.max(-1, keepdims=True)
    p = np.exp(a)
    p /= p.sum(-1, keepdims=True)
    return np.matmul(p, Vl).reshape(B, Hq * D)


# ----------------------------------------------------------------------------- prefill
def prefill_varlen(q, k, v, cu_seqlens, scale, acc=np.float32):
    """Packed causal self-attention, one block per sequence.

    Restates the fp32 single-sequence path of ``Talker.prefill_hidden`` (engine/talker.py:163-167,
    mask triu(1)) for every packed sequence of ``flash_attn_varlen_func`` (engine/talker.py:169).
    q [T, Hq, D], k/v [T, Hkv, D], cu_seqlens [n+1].  Returns [T, Hq, D].
    """
    T, Hq, D = q.shape
    Hkv = k.shape[1]
    G = Hq // Hkv
    out = np.zeros((T, Hq, D), dtype=acc)
    for i in range(len(cu_seqlens) - 1):
        s0, s1 = int(cu_seqlens[i]), int(cu_seqlens[i + 1])
        L = s1 - s0
        if L <= 0:
            continue
        qh = q[s0:s1].astype(acc).transpose(1, 0, 2).reshape(Hkv, G, L, D)
        kh = k[s0:s1].astype(acc).transpose(1, 0, 2)[:, None]                  # [Hkv,1,L,D]
        vh = v[s0:s1].astype(acc).transpose(1, 0, 2)[:, None]
        a = np.matmul(qh, kh.transpose(0, 1, 3, 2)) * acc(scale)
        a = a + np.triu(np.full((L, L), -np.inf, dtype=acc), 1)
        a = a - a.max(-1, keepdims=True)
        p = np.exp(a)
        p = p / p.sum(-1, keepdims=True)
        out[s0:s1] = np.matmul(p, vh).reshape(Hq, L, D).transpose(1, 0, 2)
    return out


def prefill_prefix(q, K, V, scale, acc=np.float32, causal=True):
    """Prefix + new tokens with bottom-right-aligned causal mask.

    Restates ``FastAdmit._attn_ref`` (engine/arrivals.py:125-131): query i (of R new) sees the
    n - R prefix keys and the new keys <= i; mask = triu(n - R + 1).  causal=False: every query sees
    all n keys (flash_attn_func's causal=False, which the engine never passes).
    q [S, R, Hq, D]; K, V [S, n, Hkv, D].  Returns [S, R, Hq, D].
    """
    S, R, Hq, D = q.shape
    n, Hkv = K.shape[1], K.shape[2]
    G = Hq // Hkv
    m = np.triu(np.full((R, n), -np.inf, dtype=acc), n - R + 1) if causal else np.zeros((R, n), dtype=acc)
    qh = q.astype(acc).transpose(0, 2, 1, 3).reshape(S, Hkv, G, R, D)
    Kh = K.astype(acc).transpose(0, 2, 1, 3)[:, :, None]
    Vh = V.astype(acc).transpose(0, 2, 1, 3)[:, :, None]
    a = np.matmul(qh, Kh.transpose(0, 1, 2, 4, 3)) * acc(scale) + m
    a = a - a.max(-1, keepdims=True)
    p = np.exp(a)
    p = p / p.sum(-1, keepdims=True)
    return np.matmul(p, Vh).reshape(S, Hq, R, D).transpose(0, 2, 1, 3)


# ----------------------------------------------------------------------------- tolerance
def compare(out, ref, max_abs=2e-2, mean_abs=2e-3):
    """The bf16 parity bar for this path: max-abs <= 2e-2 and mean-abs <= 2e-3."""
    out = np.asarray(out, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    if out.shape != ref.shape:
        return False, {"error": f"shape {out.shape} != {ref.shape}"}
    if out.size == 0:
        return True, {"max_abs": 0.0, "mean_abs": 0.0}
    if not np.isfinite(out).all():
        return False, {"error": "non-finite output"}
    d = np.abs(out - ref)
    st = {"max_abs": float(d.max()), "mean_abs": float(d.mean())}
    return (st["max_abs"] <= max_abs and st["mean_abs"] <= mean_abs), st
