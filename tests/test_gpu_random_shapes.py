"""Seeded random shapes for the decode forms (plain, KV append, q/k norm + RoPE + append) and the prefill, each against
the oracle at the 2e-2 / 2e-3 bar.  Every case draws its own batch, KV-head count, page size, table width, context
lengths (zeros and full tables included), split mode and page table, so the kernel choices (row-parallel, stream-K,
fixed split) and their boundary cases are exercised beyond the fixed sweep.  Pools are random bf16; only the pages a
case references are copied to the host for the oracle."""
import numpy as np
import pytest
import torch

import q3attn
from helpers import to_np
from oracle import attention as ora

pytestmark = pytest.mark.gpu

EPS = 1e-6


def _bf16(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(dev).to(torch.bfloat16)


def _draw(seed):
    rng = np.random.default_rng(1000 + seed)
    mode = ("plain", "append", "rope")[seed % 3]
    hkv = 8 if mode == "rope" else int(rng.choice([1, 2, 4, 8, 16]))
    page = int(rng.choice([16, 32, 64, 256]))
    B = int(rng.choice([1, 2, 3, 7, 16, 33, 64, 65, 130, 200]))
    max_ctx = int(rng.choice([16, 100, 128, 129, 600, 2048, 2064, 3000]))
    split = 0 if mode == "rope" or rng.random() < 0.7 else int(rng.choice([16, 64, 256, 1024]))
    if split:                                                # at most 64 splits per row
        split = max(split, -(-max_ctx // (64 * 16)) * 16)
    P = -(-max_ctx // page)
    while B > 1 and B * P * page * hkv * 128 > (1 << 27):    # pools of at most 256 MiB
        B //= 2
    lo = 1 if mode != "plain" else 0
    ctx = rng.integers(lo, max_ctx + 1, size=B)
    if rng.random() < 0.5:                                   # log-uniform, as the talker's seats are
        ctx = np.maximum(lo, np.rint(np.exp(rng.uniform(0, np.log(max_ctx), size=B)))).astype(np.int64)
    ctx[rng.random(B) < 0.1] = lo
    ctx[0] = max_ctx
    return rng, mode, hkv, page, B, max_ctx, split, ctx


def _compact(kc, vc, bt, ctx, page):
    """The pages rows reference, on the host, and the table renumbered onto them."""
    need = [bt[b, : (int(c) + page - 1) // page] for b, c in enumerate(ctx)]
    flat = np.concatenate([n for n in need if len(n)]) if any(len(n) for n in need) else np.zeros(1, np.int64)
    uniq = np.unique(flat)
    remap = {int(p): i for i, p in enumerate(uniq)}
    idx = torch.from_numpy(uniq).to(kc.device)
    k = to_np(kc.index_select(0, idx))
    v = to_np(vc.index_select(0, idx))
    table = np.zeros((len(ctx), max(1, bt.shape[1])), np.int64)
    for i, n in enumerate(need):
        table[i, : len(n)] = [remap[int(p)] for p in n]
    return k, v, table


@pytest.mark.parametrize("seed", range(24))
def test_decode_random_shapes(cuda_device, seed):
    rng, mode, hkv, page, B, max_ctx, split, ctx = _draw(seed)
    dev = cuda_device
    P = -(-max_ctx // page)
    num_pages = B * P + 5
    g = torch.Generator(device=dev).manual_seed(seed)
    kc = torch.randn(num_pages, page, hkv, 128, generator=g, device=dev).to(torch.bfloat16)
    vc = torch.randn(num_pages, page, hkv, 128, generator=g, device=dev).to(torch.bfloat16)
    bt = rng.permutation(num_pages)[: B * P].reshape(B, P).astype(np.int64)
    bt_d = torch.from_numpy(bt.astype(np.int32)).to(dev)
    q = rng.standard_normal((B, 2 * hkv, 128)) * (1.0 if mode != "rope" else rng.uniform(0.3, 3.0, (B, 2 * hkv, 1)))
    q = ora.bf16_round(q.astype(np.float32))
    scale = 128 ** -0.5
    label = f"{mode} hkv={hkv} page={page} B={B} max_ctx={max_ctx} split={split}"
    if mode == "plain":
        seq = torch.from_numpy(ctx.astype(np.int32)).to(dev)
        out = q3attn.paged_decode(_bf16(q, dev), kc, vc, seq, bt_d, scale, split)
        torch.cuda.synchronize()
        k, v, table = _compact(kc, vc, bt, ctx, page)
        ref = ora.paged_decode(q, k, v, ctx, table, scale)
        # the same inputs through each decomposition the shape allows (the path codes force one kernel)
        for code in (q3attn.DECODE_ROW, q3attn.DECODE_CHUNKS, q3attn.DECODE_STREAMK):
            if code == q3attn.DECODE_ROW and P * page > 2048:
                continue
            o = q3attn.paged_decode(_bf16(q, dev), kc, vc, seq, bt_d, scale, code)
            torch.cuda.synchronize()
            ok, st = ora.compare(to_np(o), ref)
            print(f"[random] decode {label} path {code} {st}", flush=True)
            assert ok, (label, code, st)
            assert not o[torch.from_numpy(ctx == 0).to(dev)].float().abs().sum().item(), (label, code)
    else:
        kn = ora.bf16_round(rng.standard_normal((B, hkv, 128)).astype(np.float32) *
                            (1.0 if mode == "append" else rng.uniform(0.3, 3.0, (B, hkv, 1)).astype(np.float32)))
        vn = ora.bf16_round(rng.standard_normal((B, hkv, 128)).astype(np.float32))
        old = torch.from_numpy((ctx - 1).astype(np.int32)).to(dev)
        if mode == "append":
            out = q3attn.paged_decode_append(_bf16(q, dev), _bf16(kn, dev), _bf16(vn, dev), kc, vc, old, bt_d, scale,
                                             split)
            qq, kk = q, kn
        else:
            qn = ora.bf16_round(rng.uniform(0.5, 1.5, 128).astype(np.float32))
            knw = ora.bf16_round(rng.uniform(0.5, 1.5, 128).astype(np.float32))
            cos_t, sin_t = ora.rope_tables(max_ctx)
            pos = np.maximum(ctx - 1, 0)
            cos, sin = ora.bf16_round(cos_t[pos]), ora.bf16_round(sin_t[pos])
            out = q3attn.paged_decode_append_rope(_bf16(q, dev), _bf16(kn, dev), _bf16(vn, dev), _bf16(qn, dev),
                                                  _bf16(knw, dev), _bf16(cos, dev), _bf16(sin, dev), kc, vc, old,
                                                  bt_d, scale, EPS)
            qq = ora.norm_rope(q, qn, cos[:, None], sin[:, None], EPS, eager=False)
            kk = ora.norm_rope(kn, knw, cos[:, None], sin[:, None], EPS, eager=False)
        torch.cuda.synchronize()
        # The oracle's pool: the kernel's own writes are checked against kk / vn, then replaced by them.
        k, v, table = _compact(kc, vc, bt, ctx, page)
        live = np.where(ctx > 0)[0]
        pos = ctx[live] - 1
        pg, off = table[live, pos // page], pos % page
        got_k, got_v = k[pg, off], v[pg, off]
        assert np.array_equal(got_v, vn[live]), f"{label}: v rows"
        if mode == "append":
            assert np.array_equal(got_k, kk[live]), f"{label}: k rows"
        else:
            y = ora.rms(kn[live], knw, eps=EPS)
            rot = np.concatenate([-y[..., 64:], y[..., :64]], axis=-1)
            bound = 2.0 ** -8 * (np.abs(y) + np.abs(rot)) + 2.0 ** -7 * np.abs(kk[live]) + 1e-30
            assert (np.abs(got_k - kk[live]) <= bound).all(), f"{label}: k rows"
        k[pg, off] = kk[live]
        ref = ora.paged_decode(qq, k, v, ctx, table, scale)
    ok, st = ora.compare(to_np(out), ref)
    print(f"[random] decode {label} {st}", flush=True)
    assert ok, (label, st)
    assert not out[torch.from_numpy(ctx == 0).to(dev)].float().abs().sum().item(), f"{label}: ctx 0 rows"


@pytest.mark.parametrize("seed", range(12))
def test_prefill_random_shapes(cuda_device, seed):
    rng = np.random.default_rng(2000 + seed)
    dev = cuda_device
    hkv = int(rng.choice([1, 2, 8, 16]))
    n = int(rng.integers(1, 40))
    lens = rng.integers(1, int(rng.choice([20, 64, 300, 700])) + 1, size=n)
    if rng.random() < 0.3:
        lens[0] = 1
    causal = bool(rng.random() < 0.8)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T = int(cu[-1])
    q = ora.bf16_round(rng.standard_normal((T, 2 * hkv, 128)).astype(np.float32))
    k = ora.bf16_round(rng.standard_normal((T, hkv, 128)).astype(np.float32))
    v = ora.bf16_round(rng.standard_normal((T, hkv, 128)).astype(np.float32))
    cu_d = torch.from_numpy(cu).to(dev)
    out = q3attn.flash_attn_varlen_func(_bf16(q, dev), _bf16(k, dev), _bf16(v, dev), cu_d, cu_d, int(lens.max()),
                                        int(lens.max()), softmax_scale=128 ** -0.5, causal=causal)
    torch.cuda.synchronize()
    if causal:
        ref = ora.prefill_varlen(q, k, v, cu, 128 ** -0.5)
    else:
        ref = np.zeros_like(q)
        for s in range(n):
            a, b = cu[s], cu[s + 1]
            for h in range(2 * hkv):
                sc = (q[a:b, h] @ k[a:b, h // 2].T) * (128 ** -0.5)
                p = np.exp(sc - sc.max(-1, keepdims=True))
                ref[a:b, h] = (p / p.sum(-1, keepdims=True)) @ v[a:b, h // 2]
    ok, st = ora.compare(to_np(out), ref)
    label = f"hkv={hkv} n={n} max_len={int(lens.max())} causal={causal}"
    print(f"[random] prefill {label} {st}", flush=True)
    assert ok, (label, st)


@pytest.mark.parametrize("seed", range(12))
def test_dense_append_random_shapes(cuda_device, seed):
    """The admission forms (q3a_prefill_dense_append and, on every other seed, the producer form
    q3a_prefill_dense_append_rope) on random S, R, n, first_row, page size and table: output against the oracle,
    pool rows first_row .. n-1 at their table positions and nothing else written (NaN-poisoned pool)."""
    dev = cuda_device
    rng = np.random.default_rng(2000 + seed)
    rope = seed % 2 == 1
    S = int(rng.choice([1, 2, 3, 5, 8]))
    R = int(rng.choice([1, 7, 16, 42, 65, 130]))
    P = int(rng.choice([0, 1, 35, 64, 90, 200]))
    n = P + R
    page = int(rng.choice([16, 32, 64, 256]))
    first = int(rng.integers(0, P + 1))
    Pn = -(-n // page)
    num_pages = 2 * S * Pn + 3
    bt = rng.permutation(num_pages)[: S * Pn].reshape(S, Pn).astype(np.int32)
    scale = 128 ** -0.5
    print(f"[case] dense append seed={seed} rope={rope} S={S} R={R} P={P} page={page} first={first}", flush=True)
    kc = torch.full((num_pages, page, 8, 128), float("nan"), dtype=torch.bfloat16, device=dev)
    vc = torch.full_like(kc, float("nan"))
    btd = torch.from_numpy(bt).to(dev)
    g = torch.Generator(device=dev)
    g.manual_seed(3000 + seed)
    if rope:
        qkv = torch.randn((S, R, 4096), generator=g, device=dev).to(torch.bfloat16)
        pk = torch.randn((S, P, 8, 128), generator=g, device=dev).to(torch.bfloat16)
        pv = torch.randn((S, P, 8, 128), generator=g, device=dev).to(torch.bfloat16)
        qn = (1.0 + 0.1 * torch.randn(128, generator=g, device=dev)).to(torch.bfloat16)
        kn = (1.0 + 0.1 * torch.randn(128, generator=g, device=dev)).to(torch.bfloat16)
        ang = np.arange(P, n)[:, None] * (1e6 ** (-np.arange(0, 128, 2) / 128))[None, :]
        emb = np.concatenate([ang, ang], -1)
        cos, sin = _bf16(np.cos(emb), dev), _bf16(np.sin(emb), dev)
        q, k, v = qkv[..., :2048].view(S, R, 16, 128), qkv[..., 2048:3072].view(S, R, 8, 128), qkv[..., 3072:].view(S, R, 8, 128)
        out = q3attn.prefill_dense_append_rope(q, k, v, pk, pv, qn, kn, cos, sin, kc, vc, btd, scale, None, True,
                                               EPS, first)
        c, s = to_np(cos)[None, :, None], to_np(sin)[None, :, None]

        def prod(x, w):   # eager rounding points (engine/ops.py:51-60 as bf16 torch ops)
            y = ora.bf16_round(to_np(w) * ora.rms(to_np(x), None, EPS, to_bf16=True))
            rot = np.concatenate([-y[..., 64:], y[..., :64]], axis=-1)
            return ora.bf16_round(ora.bf16_round(y * c) + ora.bf16_round(rot * s))
        qo = prod(q, qn)
        K = np.concatenate([to_np(pk), prod(k, kn)], 1)
        V = np.concatenate([to_np(pv), to_np(v)], 1)
    else:
        qo = rng.standard_normal((S, R, 16, 128)).astype(np.float32)
        K = rng.standard_normal((S, n, 8, 128)).astype(np.float32)
        V = rng.standard_normal((S, n, 8, 128)).astype(np.float32)
        qd, Kd, Vd = _bf16(qo, dev), _bf16(K, dev), _bf16(V, dev)
        qo, K, V = to_np(qd), to_np(Kd), to_np(Vd)
        out = q3attn.prefill_dense_append(qd, Kd, Vd, kc, vc, btd, scale, True, first)
    torch.cuda.synchronize()
    ref = ora.prefill_prefix(qo, K, V, scale)
    ok, st = ora.compare(to_np(out), ref)
    print(f"[parity] dense append seed={seed}: {st}", flush=True)
    assert ok, st
    kp, vp = to_np(kc), to_np(vc)
    j = np.arange(first, n)
    pages, offs = bt[:, j // page], j % page
    assert np.array_equal(vp[pages, offs], V[:, first:])
    diff = np.abs(kp[pages, offs] - K[:, first:])
    assert (diff <= np.maximum(np.abs(K[:, first:]), 0.5) * 2.0 ** -6).all()
    if not rope:
        assert not diff.any()
    written = np.zeros(kc.shape[:2], dtype=bool)
    written[pages, offs] = True
    assert np.isnan(kp[~written]).all() and np.isnan(vp[~written]).all()
