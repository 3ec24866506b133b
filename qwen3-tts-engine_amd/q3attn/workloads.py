"""Seeded synthetic inputs for the attention hot path, at the engine's real shapes.

q and k are drawn N(0, 1), scaled to unit RMS per head (the role of the qk-RMSNorm,
engine/ops.py:51-55) and rotated by rotate-half RoPE with theta = 1e6 (engine/ops.py:58-60) at
each token's position; v is N(0, 1).  Everything is generated on the target device with a seeded
``torch.Generator``; integer draws (context lengths, page permutations) use numpy's seeded PCG64.

Decode workloads (16 query heads over 8 KV heads, head_dim 128, pages of 16 tokens):
  * ``c1``: 1 row, ctx 64, identity page table (the CPU-runnable case);
  * ``c3``: 256 rows, ctx ~ U[200, 1200], random table over a 65,536-page pool;
  * ``c5``: 576 rows, 518 live with ctx = round(exp(U[ln 64, ln 1800])) and 58 padded rows with
    ctx = 0 at the tail, random table over a 131,072-page pool.
The code-predictor workload ``c2`` is 512 rows with dense 16-slot K/V buffers (5 layers x 16 steps).
Prefill workload ``c4``: 32 sequences of U[150, 400] tokens packed, causal, K/V through the page pool.
Admission workload (``make_admit``): the fast-admission prefill of engine/arrivals.py:133-152, S sequences of R new
tokens over a shared prefix, q [S, R, 16, 128] against K/V [S, n, 8, 128] (n = prefix + R), bottom-right causal.
"""
from __future__ import annotations

import dataclasses
import math

import numpy as np
import torch

HQ, HKV, HEAD_DIM, PAGE = 16, 8, 128, 16
ROPE_THETA = 1.0e6


def rope_tables(n_pos: int, device, head_dim: int = HEAD_DIM, theta: float = ROPE_THETA):
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float64, device=device) / head_dim))
    ang = torch.arange(n_pos, dtype=torch.float64, device=device)[:, None] * inv[None, :]
    emb = torch.cat([ang, ang], dim=-1)
    return emb.cos().float(), emb.sin().float()


def _unit_rms(x: torch.Tensor) -> torch.Tensor:
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6)


def _rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    h = x.shape[-1] // 2
    return x * cos + torch.cat((-x[..., h:], x[..., :h]), dim=-1) * sin


@dataclasses.dataclass
class DecodeLayer:
    q: torch.Tensor              # [B, Hq, D] bf16
    block_table: torch.Tensor    # [B, max_pages] int32


@dataclasses.dataclass
class DecodeWorkload:
    name: str
    k_cache: torch.Tensor        # [num_pages, page, Hkv, D] bf16
    v_cache: torch.Tensor
    cache_seqlens: torch.Tensor  # [B] int32
    layers: list                 # list[DecodeLayer]
    ctx: np.ndarray              # host copy of the context lengths
    scale: float = HEAD_DIM ** -0.5

    @property
    def batch(self) -> int:
        return int(self.ctx.shape[0])

    @property
    def page_size(self) -> int:
        return int(self.k_cache.shape[1])

    def algorithmic_bytes(self) -> int:
        """Bytes one decode call must move: K+V of every attended token, q in, o out, the page-table
        entries read and the context lengths."""
        return decode_bytes(self.ctx, self.page_size, HQ, int(self.k_cache.shape[2]), int(self.k_cache.shape[3]))


def decode_bytes(ctx, page: int, hq: int = HQ, hkv: int = HKV, d: int = HEAD_DIM) -> int:
    ctx = np.asarray(ctx, dtype=np.int64)
    kv = 2 * hkv * d * 2 * int(ctx.sum())
    qo = 2 * hq * d * 2 * int(ctx.shape[0])
    pages = 4 * int(((ctx + page - 1) // page).sum())
    return kv + qo + pages + 4 * int(ctx.shape[0])


def draw_contexts(name: str, seed: int = 0) -> np.ndarray:
    rng = np.random.default_rng(seed)
    if name == "decode1x64":
        return np.array([64], dtype=np.int64)
    if name == "decode256":
        return rng.integers(200, 1201, size=256).astype(np.int64)
    if name == "decode576":
        n_rows, n_pad = 576, 58
        live = np.rint(np.exp(rng.uniform(math.log(64), math.log(1800), size=n_rows - n_pad))).astype(np.int64)
        return np.concatenate([live, np.zeros(n_pad, dtype=np.int64)])
    raise ValueError(f"unknown decode workload {name!r}")


POOL_PAGES = {"decode1x64": 4, "decode256": 65536, "decode576": 131072}
MAX_CTX = {"decode1x64": 64, "decode256": 1200, "decode576": 1800}


def make_decode(name: str, device, layers: int = 1, seed: int = 0, ctx: np.ndarray | None = None,
                num_pages: int | None = None, max_ctx: int | None = None, page: int = PAGE,
                identity: bool | None = None, chunk_pages: int = 4096) -> DecodeWorkload:
    """Build a decode workload.  ``ctx``/``num_pages``/``max_ctx`` override the named config (used
    by the tests for small ragged cases)."""
    device = torch.device(device)
    ctx = draw_contexts(name, seed) if ctx is None else np.asarray(ctx, dtype=np.int64)
    num_pages = POOL_PAGES.get(name) if num_pages is None else num_pages
    max_ctx = MAX_CTX.get(name, int(ctx.max(initial=1))) if max_ctx is None else max_ctx
    identity = (name == "decode1x64") if identity is None else identity
    B = int(ctx.shape[0])
    P = max(1, -(-max_ctx // page))
    if B * P > num_pages:
        raise ValueError(f"pool of {num_pages} pages cannot hold {B} rows x {P} pages")
    rng = np.random.default_rng(seed + 1)
    tables = []
    for layer in range(layers):
        if identity:
            bt = np.arange(B * P, dtype=np.int64).reshape(B, P)
        else:
            bt = rng.permutation(num_pages)[: B * P].reshape(B, P)
        tables.append(bt)

    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    # Token positions of each pool page under layer 0's table (unreferenced pages: position 0).
    pos_base = np.zeros(num_pages, dtype=np.int64)
    pos_base[tables[0].reshape(-1)] = np.tile(np.arange(P, dtype=np.int64) * page, B)
    pos_base_t = torch.from_numpy(pos_base).to(device)
    cos, sin = rope_tables(max(P * page, 1), device)

    k_cache = torch.empty((num_pages, page, HKV, HEAD_DIM), dtype=torch.bfloat16, device=device)
    v_cache = torch.empty_like(k_cache)
    ar = torch.arange(page, device=device)
    for c0 in range(0, num_pages, chunk_pages):
        n = min(chunk_pages, num_pages - c0)
        x = _unit_rms(torch.randn((n, page, HKV, HEAD_DIM), generator=gen, device=device))
        pos = pos_base_t[c0:c0 + n, None] + ar[None, :]
        x = _rope(x, cos[pos][:, :, None, :], sin[pos][:, :, None, :])
        k_cache[c0:c0 + n] = x.to(torch.bfloat16)
        v_cache[c0:c0 + n] = torch.randn((n, page, HKV, HEAD_DIM), generator=gen, device=device).to(torch.bfloat16)
        del x

    qpos = torch.from_numpy(np.maximum(ctx - 1, 0)).to(device)
    out_layers = []
    for layer in range(layers):
        q = _unit_rms(torch.randn((B, HQ, HEAD_DIM), generator=gen, device=device))
        q = _rope(q, cos[qpos][:, None, :], sin[qpos][:, None, :]).to(torch.bfloat16)
        out_layers.append(DecodeLayer(q=q, block_table=torch.from_numpy(tables[layer]).to(torch.int32).to(device)))
    seqlens = torch.from_numpy(ctx).to(torch.int32).to(device)
    return DecodeWorkload(name=name, k_cache=k_cache, v_cache=v_cache, cache_seqlens=seqlens,
                          layers=out_layers, ctx=ctx)


def make_cp(batch: int, device, seed: int = 0, steps: int = 16, kv_pad: int = 0) -> tuple:
    """Dense 16-slot K/V scratch (engine/code_predictor.py:20-21) filled for all 16 slots and one
    query per step p (RoPE at position p).  ``kv_pad`` > 0 allocates the slot rows wider than
    head_dim to exercise non-trivial strides.  Returns (qs: list of [B, Hq, D], K, V)."""
    device = torch.device(device)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    cos, sin = rope_tables(16, device)
    Kb = torch.zeros((batch, HKV, 16, HEAD_DIM + kv_pad), dtype=torch.bfloat16, device=device)
    Vb = torch.zeros_like(Kb)
    k = _unit_rms(torch.randn((batch, HKV, 16, HEAD_DIM), generator=gen, device=device))
    k = _rope(k, cos[None, None], sin[None, None])
    Kb[..., :HEAD_DIM] = k.to(torch.bfloat16)
    Vb[..., :HEAD_DIM] = torch.randn((batch, HKV, 16, HEAD_DIM), generator=gen, device=device).to(torch.bfloat16)
    qs = []
    for p in range(steps):
        q = _unit_rms(torch.randn((batch, HQ, HEAD_DIM), generator=gen, device=device))
        qs.append(_rope(q, cos[p], sin[p]).to(torch.bfloat16))
    return qs, Kb[..., :HEAD_DIM], Vb[..., :HEAD_DIM]


def cp_bytes(batch: int, n_live: int, hq: int = HQ, hkv: int = HKV, d: int = HEAD_DIM, append: bool = False) -> int:
    """Bytes of one cp_attn call: K+V of the live slots, q in, o out; with ``append`` also the write of
    the new slot's K+V (its reads are already counted as live slots)."""
    return batch * (2 * hkv * n_live * d * 2 + 2 * hq * d * 2 + (2 * hkv * d * 2 if append else 0))


@dataclasses.dataclass
class PrefillWorkload:
    q: torch.Tensor              # [T, Hq, D] bf16, packed sequences
    k: torch.Tensor              # [T, Hkv, D] bf16, packed
    v: torch.Tensor
    cu_seqlens: torch.Tensor     # [n + 1] int32
    lens: np.ndarray
    k_cache: torch.Tensor | None = None   # paged pool holding the same K/V
    v_cache: torch.Tensor | None = None
    block_table: torch.Tensor | None = None
    scale: float = HEAD_DIM ** -0.5

    @property
    def max_len(self) -> int:
        return int(self.lens.max(initial=0))

    def flops(self) -> int:
        """Causal attention flops (QK^T and PV over the keys each query sees)."""
        L = self.lens.astype(np.int64)
        return int((4 * HEAD_DIM * HQ * (L * (L + 1) // 2)).sum())

    def algorithmic_bytes(self) -> int:
        """q read + o write + K/V read once per sequence and KV head + cu_seqlens and table entries."""
        T = int(self.lens.sum())
        pages = int(((self.lens + PAGE - 1) // PAGE).sum()) if self.block_table is not None else 0
        return 2 * T * HQ * HEAD_DIM * 2 + 2 * T * HKV * HEAD_DIM * 2 + 4 * (len(self.lens) + 1) + 4 * pages


def prefill_lengths(name: str, seed: int = 0) -> np.ndarray:
    rng = np.random.default_rng(seed)
    if name == "prefill32":
        return rng.integers(150, 401, size=32).astype(np.int64)
    raise ValueError(f"unknown prefill workload {name!r}")


def make_prefill(device, lens, seed: int = 0, paged: bool = True, page: int = PAGE, num_pages: int | None = None,
                 identity: bool = False) -> PrefillWorkload:
    """Prompt prefill: each sequence's q/k get RoPE at positions 0..L-1; with ``paged`` the K/V are also
    written into a pool through a seeded random (or identity) page table, as the talker does before it
    attends (engine/talker.py:161-162)."""
    device = torch.device(device)
    lens = np.asarray(lens, dtype=np.int64)
    T = int(lens.sum())
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    cos, sin = rope_tables(max(int(lens.max(initial=1)), 1), device)
    pos = torch.from_numpy(np.concatenate([np.arange(L) for L in lens]) if T else np.zeros(0, np.int64)).to(device)
    q = _rope(_unit_rms(torch.randn((T, HQ, HEAD_DIM), generator=gen, device=device)), cos[pos][:, None], sin[pos][:, None])
    k = _rope(_unit_rms(torch.randn((T, HKV, HEAD_DIM), generator=gen, device=device)), cos[pos][:, None], sin[pos][:, None])
    v = torch.randn((T, HKV, HEAD_DIM), generator=gen, device=device)
    cu = torch.from_numpy(np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)).to(device)
    wl = PrefillWorkload(q=q.to(torch.bfloat16), k=k.to(torch.bfloat16), v=v.to(torch.bfloat16), cu_seqlens=cu,
                         lens=lens)
    if paged:
        n = len(lens)
        P = max(1, -(-int(lens.max(initial=1)) // page))
        num_pages = n * P if num_pages is None else num_pages
        rng = np.random.default_rng(seed + 7)
        bt = np.arange(n * P).reshape(n, P) if identity else rng.permutation(num_pages)[: n * P].reshape(n, P)
        slots = np.concatenate([bt[s, np.arange(L) // page] * page + np.arange(L) % page for s, L in enumerate(lens)])
        slots_t = torch.from_numpy(slots.astype(np.int64)).to(device)
        kc = torch.zeros((num_pages, page, HKV, HEAD_DIM), dtype=torch.bfloat16, device=device)
        vc = torch.zeros_like(kc)
        kc.view(-1, HKV, HEAD_DIM).index_copy_(0, slots_t, wl.k)
        vc.view(-1, HKV, HEAD_DIM).index_copy_(0, slots_t, wl.v)
        wl.k_cache, wl.v_cache = kc, vc
        wl.block_table = torch.from_numpy(bt.astype(np.int32)).to(device)
    return wl


@dataclasses.dataclass
class AdmitWorkload:
    q: torch.Tensor              # [S, R, Hq, D] bf16: the new tokens, positions n - R .. n - 1
    k: torch.Tensor              # [S, n, Hkv, D] bf16: prefix + new tokens, positions 0 .. n - 1
    v: torch.Tensor
    scale: float = HEAD_DIM ** -0.5

    def flops(self) -> int:
        """QK^T and PV over the keys each new token sees (n - R prefix keys plus the new ones up to itself)."""
        S, R = self.q.shape[0], self.q.shape[1]
        n = self.k.shape[1]
        seen = R * (n - R) + R * (R + 1) // 2
        return 4 * HEAD_DIM * HQ * S * seen


def make_admit(device, S: int, R: int, n: int, seed: int = 0) -> AdmitWorkload:
    """Fast-admission prefill inputs (engine/arrivals.py:112-118, 148): each sequence's K carries RoPE at positions
    0..n-1 and q at the new tokens' positions n-R..n-1."""
    device = torch.device(device)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    cos, sin = rope_tables(n, device)
    q = _rope(_unit_rms(torch.randn((S, R, HQ, HEAD_DIM), generator=gen, device=device)),
              cos[n - R:][None, :, None], sin[n - R:][None, :, None])
    k = _rope(_unit_rms(torch.randn((S, n, HKV, HEAD_DIM), generator=gen, device=device)),
              cos[None, :, None], sin[None, :, None])
    v = torch.randn((S, n, HKV, HEAD_DIM), generator=gen, device=device)
    return AdmitWorkload(q=q.to(torch.bfloat16), k=k.to(torch.bfloat16), v=v.to(torch.bfloat16))
