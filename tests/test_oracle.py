"""Pins the CPU oracle (oracle/attention.py) with checks that do not restate its own formulas:
library routines (torch CPU SDPA, torch bf16 ops), float64 brute force, closed forms, invariants,
and planted mistakes that those checks must catch."""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as ora

RNG = np.random.default_rng(1234)


def _bf16(x):
    return ora.bf16_round(np.asarray(x, np.float32))


def _decode_case(B=4, Hq=4, Hkv=2, D=16, page=4, ctx=(1, 5, 9, 12), num_pages=32, seed=0):
    r = np.random.default_rng(seed)
    P = max(1, -(-max(ctx) // page))
    q = _bf16(r.standard_normal((B, Hq, D)))
    k = _bf16(r.standard_normal((num_pages, page, Hkv, D)))
    v = _bf16(r.standard_normal((num_pages, page, Hkv, D)))
    bt = r.permutation(num_pages)[: B * P].reshape(B, P)
    return q, k, v, np.array(ctx), bt


# ----------------------------------------------------------------------------- bf16 helpers
def test_bf16_round_matches_torch():
    x = np.concatenate([
        RNG.standard_normal(10000).astype(np.float32) * 10,
        np.array([0.0, -0.0, 1.0, 1.00390625, 1.01171875, 3.0e38, -3.0e38, 1e-40, -1e-40,
                  np.inf, -np.inf], np.float32),
        # exact ties between two bf16 neighbours (round half to even)
        (np.arange(1, 200, dtype=np.uint32) << 16 | 0x8000).view(np.float32),
    ])
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    got = ora.bf16_round(x)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    nan = ora.bf16_round(np.array([np.nan], np.float32))
    assert np.isnan(nan).all()


# ----------------------------------------------------------------------------- paged decode
def test_paged_decode_matches_bruteforce():
    q, k, v, ctx, bt = _decode_case(B=3, Hq=4, Hkv=2, D=8, page=4, ctx=(1, 6, 11), num_pages=16)
    got = ora.paged_decode(q, k, v, ctx, bt, 0.3, acc=np.float64)
    want = ora.paged_decode_bruteforce(q, k, v, ctx, bt, 0.3)
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-12)


def _sdpa_decode(q, k, v, ctx, bt, scale):
    """torch CPU scaled_dot_product_attention with its own GQA convention, per row."""
    page = k.shape[1]
    out = np.zeros_like(q, dtype=np.float64)
    for b in range(q.shape[0]):
        c = int(ctx[b])
        if c == 0:
            continue
        t = np.arange(c)
        K = torch.from_numpy(k[bt[b][t // page], t % page].astype(np.float64)).transpose(0, 1)[None]
        V = torch.from_numpy(v[bt[b][t // page], t % page].astype(np.float64)).transpose(0, 1)[None]
        Q = torch.from_numpy(q[b].astype(np.float64))[None, :, None, :]
        o = F.scaled_dot_product_attention(Q, K, V, scale=scale, enable_gqa=True)
        out[b] = o[0, :, 0].numpy()
    return out


def test_paged_decode_matches_sdpa():
    q, k, v, ctx, bt = _decode_case(B=5, Hq=16, Hkv=8, D=128, page=16, ctx=(1, 16, 17, 100, 300),
                                    num_pages=128, seed=3)
    got = ora.paged_decode(q, k, v, ctx, bt, 128 ** -0.5)
    want = _sdpa_decode(q, k, v, ctx, bt, 128 ** -0.5)
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-6)


def test_paged_decode_closed_forms():
    q, k, v, ctx, bt = _decode_case(B=3, Hq=4, Hkv=2, D=16, page=4, ctx=(1, 7, 13), num_pages=32, seed=5)
    page = k.shape[1]
    # ctx == 1: the output is exactly the first token's V row of the mapped KV head.
    o = ora.paged_decode(q, k, v, np.array([1, 1, 1]), bt, 0.25)
    for b in range(3):
        for h in range(4):
            assert np.array_equal(o[b, h], v[bt[b][0], 0, h // 2])
    # constant V along tokens -> output equals that row
    vc = np.broadcast_to(v[:, :1], v.shape).copy()
    vc[:] = v[0, 0]
    o = ora.paged_decode(q, k, vc, ctx, bt, 0.25)
    np.testing.assert_allclose(o, np.broadcast_to(v[0, 0][None, [0, 0, 1, 1]], o.shape), atol=1e-6)
    # identical keys -> uniform weights -> mean of the context's V rows
    kc = np.broadcast_to(k[0, 0], k.shape).copy()
    o = ora.paged_decode(q, kc, v, ctx, bt, 0.25, acc=np.float64)
    for b in range(3):
        t = np.arange(ctx[b])
        V = v[bt[b][t // page], t % page]                       # [ctx, Hkv, D]
        for h in range(4):
            np.testing.assert_allclose(o[b, h], V[:, h // 2].mean(0), atol=1e-12)
    # ctx == 0 -> zeros
    o = ora.paged_decode(q, k, v, np.array([0, 0, 0]), bt, 0.25)
    assert not o.any()


def test_paged_decode_page_table_permutation_invariance():
    q, k, v, ctx, bt = _decode_case(B=3, Hq=4, Hkv=2, D=16, page=4, ctx=(3, 8, 14), num_pages=24, seed=7)
    perm = np.random.default_rng(9).permutation(k.shape[0])          # new page p holds old page perm[p]
    inv = np.argsort(perm)
    o1 = ora.paged_decode(q, k, v, ctx, bt, 0.2)
    o2 = ora.paged_decode(q, k[perm], v[perm], ctx, inv[bt], 0.2)
    assert np.array_equal(o1, o2)


def test_paged_decode_identity_table_is_reference_slot_slice():
    """With 256-token pages and the identity table (engine/talker.py:23-25, 42) the gather is the
    contiguous slot range that ``_attn_ref`` slices: K[slot-ctx+1 : slot+1] with
    slot = seat*seat_len + pos and ctx = pos + 1 (engine/talker.py:85, 109-110)."""
    r = np.random.default_rng(11)
    seats, seat_len, page, Hkv, D, Hq = 3, 512, 256, 2, 8, 4
    P = seat_len // page
    k = _bf16(r.standard_normal((seats * P, page, Hkv, D)))
    v = _bf16(r.standard_normal((seats * P, page, Hkv, D)))
    q = _bf16(r.standard_normal((seats, Hq, D)))
    pos = np.array([0, 255, 300])
    bt = (np.arange(seats)[:, None] * P + np.arange(P)[None, :])
    got = ora.paged_decode(q, k, v, pos + 1, bt, 0.35, acc=np.float64)
    Kf = k.reshape(-1, Hkv, D)
    Vf = v.reshape(-1, Hkv, D)
    for b in range(seats):
        slot = b * seat_len + pos[b]
        s0 = slot - pos[b]
        K = Kf[s0:slot + 1].astype(np.float64).transpose(1, 0, 2)
        V = Vf[s0:slot + 1].astype(np.float64).transpose(1, 0, 2)
        a = np.matmul(q[b].astype(np.float64).reshape(Hkv, Hq // Hkv, D), K.transpose(0, 2, 1)) * 0.35
        p = np.exp(a - a.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
        np.testing.assert_allclose(got[b], np.matmul(p, V).reshape(Hq, D), atol=1e-12)


def test_planted_mistakes_are_caught():
    """Mutated oracles (wrong GQA map, dropped scale, off-by-one page offset) must fail the SDPA check."""
    q, k, v, ctx, bt = _decode_case(B=3, Hq=16, Hkv=8, D=32, page=16, ctx=(5, 20, 40), num_pages=16, seed=13)
    want = _sdpa_decode(q, k, v, ctx, bt, 0.2)

    def gqa_mod(q, k, v, ctx, bt, s):           # q head h reads kv head h % Hkv
        qq = q.reshape(q.shape[0], 2, 8, -1).transpose(0, 2, 1, 3).reshape(q.shape)
        o = ora.paged_decode(qq, k, v, ctx, bt, s)
        return o.reshape(o.shape[0], 8, 2, -1).transpose(0, 2, 1, 3).reshape(o.shape)

    def no_scale(q, k, v, ctx, bt, s):
        return ora.paged_decode(q, k, v, ctx, bt, 1.0)

    def page_shift(q, k, v, ctx, bt, s):       # token t read from offset (t+1) % page
        return ora.paged_decode(q, np.roll(k, -1, axis=1), np.roll(v, -1, axis=1), ctx, bt, s)

    for bad in (gqa_mod, no_scale, page_shift):
        got = bad(q, k, v, ctx, bt, 0.2)
        assert np.abs(got - want).max() > 1e-3, bad.__name__


# ----------------------------------------------------------------------------- code predictor
def _cp_case(B=6, seed=0, nan_stale=False):
    r = np.random.default_rng(seed)
    q = _bf16(r.standard_normal((B, 16, 128)))
    K = _bf16(r.standard_normal((B, 8, 16, 128)))
    V = _bf16(r.standard_normal((B, 8, 16, 128)))
    return q, K, V


@pytest.mark.parametrize("n_live", [1, 2, 7, 16])
def test_cp_torch_path_matches_torch_bf16_ops(n_live):
    """The numpy rounding sequence against torch's own bf16 CPU kernels running the op sequence of
    engine/code_predictor.py:46-47 (bf16 matmul, *scale, +mask, fp32 softmax, bf16 P, bf16 matmul)."""
    q, K, V = _cp_case(B=6, seed=n_live)
    scale = 128 ** -0.5
    qt = torch.from_numpy(q).to(torch.bfloat16)
    Kt = torch.from_numpy(K).to(torch.bfloat16)
    Vt = torch.from_numpy(V).to(torch.bfloat16)
    mask = torch.full((16, 16), float("-inf")).triu(1).to(torch.bfloat16)[n_live - 1]
    att = torch.matmul(qt.view(6, 8, 2, 128), Kt.transpose(-1, -2).contiguous()) * scale + mask
    o = torch.matmul(torch.softmax(att.float(), dim=-1).to(torch.bfloat16), Vt).reshape(6, 2048).float().numpy()
    got = ora.cp_attn_torch_path(q, K, V, n_live, scale)
    d = np.abs(got - o)
    # Identical op sequence; only the fp32 accumulation order inside the matmuls may differ.
    assert d.max() <= 2 ** -7 * np.abs(o).max() and (d == 0).mean() > 0.95


@pytest.mark.parametrize("n_live", [1, 3, 16])
def test_cp_paths_within_tolerance_of_exact(n_live):
    q, K, V = _cp_case(B=8, seed=100 + n_live)
    exact = ora.cp_attn_exact(q, K, V, n_live, 128 ** -0.5)
    for fn in (ora.cp_attn_torch_path, ora.cp_attn_triton_path):
        ok, st = ora.compare(fn(q, K, V, n_live, 128 ** -0.5), exact)
        assert ok, (fn.__name__, st)


def test_cp_closed_forms_and_stale_slots():
    q, K, V = _cp_case(B=4, seed=21)
    for fn in (ora.cp_attn_torch_path, ora.cp_attn_triton_path):
        o = fn(q, K, V, 1, 128 ** -0.5).reshape(4, 8, 2, 128)
        assert np.array_equal(o, np.broadcast_to(V[:, :, 0][:, :, None], o.shape))
    for n_live in (1, 5, 15):
        Kp, Vp = K.copy(), V.copy()
        Kp[:, :, n_live:] = np.nan
        Vp[:, :, n_live:] = np.nan
        a = ora.cp_attn_triton_path(q, K, V, n_live, 0.1)
        b = ora.cp_attn_triton_path(q, Kp, Vp, n_live, 0.1)
        assert np.array_equal(a, b)


# ----------------------------------------------------------------------------- prefill
def test_prefill_varlen_matches_sdpa_causal():
    r = np.random.default_rng(31)
    lens = [1, 7, 20]
    T = sum(lens)
    cu = np.concatenate([[0], np.cumsum(lens)])
    q = _bf16(r.standard_normal((T, 16, 32)))
    k = _bf16(r.standard_normal((T, 8, 32)))
    v = _bf16(r.standard_normal((T, 8, 32)))
    got = ora.prefill_varlen(q, k, v, cu, 0.17, acc=np.float64)
    for i, L in enumerate(lens):
        s = slice(cu[i], cu[i + 1])
        Q = torch.from_numpy(q[s].astype(np.float64)).transpose(0, 1)[None]
        K = torch.from_numpy(k[s].astype(np.float64)).transpose(0, 1)[None]
        V = torch.from_numpy(v[s].astype(np.float64)).transpose(0, 1)[None]
        o = F.scaled_dot_product_attention(Q, K, V, is_causal=True, scale=0.17, enable_gqa=True)
        np.testing.assert_allclose(got[s], o[0].transpose(0, 1).numpy(), atol=1e-12)


def test_prefill_prefix_reduces_and_bruteforce():
    r = np.random.default_rng(41)
    S, R, n, Hq, Hkv, D = 2, 5, 9, 4, 2, 8
    q = _bf16(r.standard_normal((S, R, Hq, D)))
    K = _bf16(r.standard_normal((S, n, Hkv, D)))
    V = _bf16(r.standard_normal((S, n, Hkv, D)))
    got = ora.prefill_prefix(q, K, V, 0.3, acc=np.float64)
    # brute force: query i sees keys j <= (n - R) + i
    for s in range(S):
        for i in range(R):
            for h in range(Hq):
                sc = [float(np.dot(q[s, i, h].astype(np.float64), K[s, j, h // 2])) * 0.3 for j in range(n - R + i + 1)]
                m = max(sc)
                e = np.exp(np.array(sc) - m)
                o = (e[:, None] * V[s, : len(sc), h // 2].astype(np.float64)).sum(0) / e.sum()
                np.testing.assert_allclose(got[s, i, h], o, atol=1e-12)
    # R == n: standard causal attention of one packed sequence
    q2 = q[:, :R]
    K2, V2 = K[:, :R], V[:, :R]
    a = ora.prefill_prefix(q2, K2, V2, 0.3, acc=np.float64)
    b = ora.prefill_varlen(q2[0], K2[0], V2[0], np.array([0, R]), 0.3, acc=np.float64)
    np.testing.assert_allclose(a[0], b, atol=1e-12)


def test_prefill_prefix_non_causal_is_sdpa_without_mask():
    r = np.random.default_rng(43)
    S, R, n, Hq, Hkv, D = 3, 6, 11, 8, 4, 16
    q = _bf16(r.standard_normal((S, R, Hq, D)))
    K = _bf16(r.standard_normal((S, n, Hkv, D)))
    V = _bf16(r.standard_normal((S, n, Hkv, D)))
    got = ora.prefill_prefix(q, K, V, 0.25, acc=np.float64, causal=False)
    t = lambda x: torch.from_numpy(x.astype(np.float64)).transpose(1, 2)
    want = torch.nn.functional.scaled_dot_product_attention(t(q), t(K), t(V), scale=0.25, enable_gqa=True)
    np.testing.assert_allclose(got, want.transpose(1, 2).numpy(), atol=1e-12)
    # and differs from the causal form wherever a query has keys past its diagonal
    assert np.abs(got - ora.prefill_prefix(q, K, V, 0.25, acc=np.float64)).max() > 1e-3


# ----------------------------------------------------------------------------- rms / rope
def test_rms_rope_invariants():
    x = RNG.standard_normal((64, 128)).astype(np.float32) * 3
    y = ora.rms(x, to_bf16=False)
    np.testing.assert_allclose((y.astype(np.float64) ** 2).mean(-1), 1.0, rtol=1e-5)
    cos, sin = ora.rope_tables(1024)
    # position 0 is the identity
    np.testing.assert_array_equal(ora.rope(y, cos[0], sin[0]), y)
    # each (i, i+64) pair is rotated: its norm is preserved
    r = ora.rope(y, cos[777], sin[777])
    n0 = y[:, :64] ** 2 + y[:, 64:] ** 2
    n1 = r[:, :64] ** 2 + r[:, 64:] ** 2
    np.testing.assert_allclose(n1, n0, rtol=1e-5, atol=1e-6)
    # q(m).k(n) depends only on m - n
    a, b = y[0].astype(np.float64), y[1].astype(np.float64)
    cos64, sin64 = [t.astype(np.float64) for t in ora.rope_tables(1024)]
    d1 = ora.rope(a, cos64[100], sin64[100]) @ ora.rope(b, cos64[90], sin64[90])
    d2 = ora.rope(a, cos64[510], sin64[510]) @ ora.rope(b, cos64[500], sin64[500])
    assert abs(d1 - d2) < 1e-4


def test_rope_table_closed_form():
    cos, sin = ora.rope_tables(2000, theta=1.0e6)
    for pos, i in ((0, 0), (1, 0), (1799, 5), (1500, 63), (37, 40)):
        ang = pos * (1.0e6 ** (-2 * i / 128))
        assert math.isclose(cos[pos, i], math.cos(ang), abs_tol=1e-6)
        assert math.isclose(sin[pos, i + 64], math.sin(ang), abs_tol=1e-6)


def test_cpu_baseline_ports_agree_with_oracle():
    """oracle/torch_cpu.py (timed as the CPU baseline) computes what the numpy oracle computes."""
    from oracle import torch_cpu as tc
    q, k, v, ctx, bt = _decode_case(B=4, Hq=16, Hkv=8, D=128, page=16, ctx=(0, 1, 40, 77), num_pages=32, seed=23)
    got = tc.paged_decode_rows(torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v), ctx,
                               torch.from_numpy(bt), 0.09).numpy()
    np.testing.assert_allclose(got, ora.paged_decode(q, k, v, ctx, bt, 0.09), atol=2e-6)
    qc, K, V = _cp_case(B=5, seed=29)
    bf = lambda x: torch.from_numpy(x).to(torch.bfloat16)
    got = tc.cp_attn_rows(bf(qc), bf(K), bf(V), 6, 128 ** -0.5).float().numpy()
    d = np.abs(got - ora.cp_attn_torch_path(qc, K, V, 6, 128 ** -0.5))
    assert d.max() <= 2 ** -7 * np.abs(got).max() and (d == 0).mean() > 0.95
    r = np.random.default_rng(31)
    lens = [3, 20]
    cu = np.array([0, 3, 23])
    qp = _bf16(r.standard_normal((23, 16, 32)))
    kp = _bf16(r.standard_normal((23, 8, 32)))
    vp = _bf16(r.standard_normal((23, 8, 32)))
    got = tc.prefill_rows(torch.from_numpy(qp), torch.from_numpy(kp), torch.from_numpy(vp), cu, 0.2).numpy()
    np.testing.assert_allclose(got, ora.prefill_varlen(qp, kp, vp, cu, 0.2), atol=2e-6)
    qa = _bf16(r.standard_normal((2, 5, 16, 32)))
    Ka = _bf16(r.standard_normal((2, 9, 8, 32)))
    Va = _bf16(r.standard_normal((2, 9, 8, 32)))
    got = tc.prefill_prefix_rows(torch.from_numpy(qa), torch.from_numpy(Ka), torch.from_numpy(Va), 0.2).numpy()
    np.testing.assert_allclose(got, ora.prefill_prefix(qa, Ka, Va, 0.2), atol=2e-6)
