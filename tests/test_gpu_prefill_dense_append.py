"""GPU parity of the fused fast-admission layer step (q3a_prefill_dense_append through the C ABI).

engine/arrivals.py:144-145 scatters every row of K = cat(prefix, new) and of V into the seat's cache positions
0 .. n-1 with index_copy_, then engine/arrivals.py:148 runs flash_attn_func(q, K, V, causal=True) on the dense
tensors.  Against that two-step sequence (index_copy_ + q3attn.prefill_dense) the fused call's output and pool must
be bit-identical.  The pool starts NaN-filled, so every slot the call should write is checked and every other slot
must stay NaN.  The causal outputs are also checked against the oracle (engine/arrivals.py:125-131's fp32 form).
Shapes with n <= 128 keys take the short-key kernel (whole K/V range in LDS, rows stored from there), longer ones
the tiled kernel (rows in 64-row chunks spread over a sequence's query-tile workgroups)."""
import numpy as np
import pytest
import torch

import q3attn
from helpers import to_np
from oracle import attention as ora
from q3attn import workloads as W

pytestmark = pytest.mark.gpu


def _table(S, P, num_pages, identity, seed):
    if identity:
        return np.arange(S * P, dtype=np.int32).reshape(S, P)
    return np.random.default_rng(seed).permutation(num_pages)[: S * P].reshape(S, P).astype(np.int32)


def _slots(S, n, first, bt, page, num_pages):
    """Flat pool slot and (sequence, row) of every row the call writes: rows first .. n-1 of each sequence that have
    a valid page."""
    slots, seqs, rows = [], [], []
    for s in range(S):
        for p in range(first, n):
            if p // page >= bt.shape[1] or not 0 <= bt[s, p // page] < num_pages:
                continue
            slots.append(int(bt[s, p // page]) * page + p % page)
            seqs.append(s)
            rows.append(p)
    return (np.array(slots, dtype=np.int64), np.array(seqs, dtype=np.int64), np.array(rows, dtype=np.int64))


def _run_both(dev, q, k, v, bt_np, page, num_pages, scale, causal=True, first=0):
    S, n, Hkv, _ = k.shape
    kc = torch.full((num_pages, page, Hkv, 128), float("nan"), dtype=torch.bfloat16, device=dev)
    vc = torch.full_like(kc, float("nan"))
    bt = torch.from_numpy(bt_np).to(dev)
    print(f"[case] prefill_dense_append S={S} R={q.shape[1]} n={n} page={page} first={first} causal={causal}",
          flush=True)
    out = q3attn.prefill_dense_append(q, k, v, kc, vc, bt, scale, causal, first)
    torch.cuda.synchronize()
    # the two-step reference: index_copy_ of the rows, then the dense prefill
    rk, rv = torch.full_like(kc, float("nan")), torch.full_like(vc, float("nan"))
    slots, seqs, rows = _slots(S, n, first, bt_np, page, num_pages)
    si = torch.from_numpy(slots).to(dev)
    sq, sr = torch.from_numpy(seqs).to(dev), torch.from_numpy(rows).to(dev)
    if len(slots):
        rk.view(-1, Hkv, 128).index_copy_(0, si, k[sq, sr])
        rv.view(-1, Hkv, 128).index_copy_(0, si, v[sq, sr])
    ref = q3attn.flash_attn_func(q, k, v, softmax_scale=scale, causal=causal)
    torch.cuda.synchronize()
    assert torch.equal(out, ref), "output differs from the dense prefill"
    # NaN-aware pool comparison: written slots equal, untouched slots still NaN in both
    assert torch.equal(torch.isnan(kc), torch.isnan(rk)) and torch.equal(torch.isnan(vc), torch.isnan(rv))
    assert torch.equal(torch.nan_to_num(kc), torch.nan_to_num(rk))
    assert torch.equal(torch.nan_to_num(vc), torch.nan_to_num(rv))
    return out, kc, vc, len(slots)


def _oracle_check(out, w_q, w_k, w_v, scale, what):
    ok, st = ora.compare(to_np(out), ora.prefill_prefix(to_np(w_q), to_np(w_k), to_np(w_v), scale))
    print(f"[parity] {what} vs oracle {st}", flush=True)
    assert ok, st


@pytest.mark.parametrize("S,R,n,page,identity,first", [
    (8, 42, 77, 16, False, 0),       # the admission shape, the engine's call (every row)
    (8, 42, 77, 16, False, 35),      # prefix already in the pool: the new rows only
    (8, 42, 77, 16, False, 20),      # part of the prefix
    (4, 42, 77, 256, True, 0),       # the reference's own pool: 256-token pages, identity seats
    (3, 20, 20, 16, False, 0),       # no prefix
    (2, 50, 128, 32, False, 0),      # the short-key kernel's largest key range
    (2, 300, 100, 16, False, 0),     # more queries than keys: two query blocks, the first 200 tokens see nothing
    (2, 100, 300, 16, False, 0),     # tiled: 5 row chunks over 2 query tiles
    (3, 130, 150, 16, False, 0),     # tiled: 3 query tiles, a 20-row prefix
    (2, 40, 700, 64, False, 0),      # tiled: one query tile writes all 11 chunks
    (2, 40, 700, 16, False, 660),    # tiled, new rows only
    (2, 40, 690, 16, False, 600),    # tiled, part of the prefix
])
def test_dense_append_matches_scatter_then_prefill(cuda_device, S, R, n, page, identity, first):
    if R <= n:
        w = W.make_admit(cuda_device, S, R, n, seed=21 + n)
        q = w.q
    else:                                        # q of R new tokens over only n keys
        w = W.make_admit(cuda_device, S, n, n, seed=21 + n)
        q = W.make_admit(cuda_device, S, R, R, seed=20).q
    P = -(-n // page)
    num_pages = max(2 * S * P, 64)
    bt = _table(S, P, num_pages, identity, seed=22)
    out, _, _, nw = _run_both(cuda_device, q, w.k, w.v, bt, page, num_pages, w.scale, True, first)
    assert nw == S * (n - first)
    if R <= n:
        _oracle_check(out, q, w.k, w.v, w.scale, f"prefill_dense_append S={S} R={R} n={n} first={first}")
    else:                                        # the first R - n tokens see no key: zeros; the rest as the oracle
        assert not out[:, : R - n].float().abs().sum().item()
        _oracle_check(out[:, R - n:], q[:, R - n:], w.k, w.v, w.scale, f"prefill_dense_append S={S} R={R} n={n}")


@pytest.mark.parametrize("S,R,n", [(4, 42, 77), (2, 100, 300)])
def test_dense_append_non_causal(cuda_device, S, R, n):
    w = W.make_admit(cuda_device, S, R, n, seed=23)
    P = -(-n // 16)
    bt = _table(S, P, 64, False, seed=24)
    _, _, _, nw = _run_both(cuda_device, w.q, w.k, w.v, bt, 16, 64, w.scale, causal=False)
    assert nw == S * n


@pytest.mark.parametrize("n", [77, 300])
def test_dense_append_short_table_and_invalid_pages(cuda_device, n):
    """A table with fewer pages than the key range and invalid entries: those positions are not written (and
    nothing faults); the attention still sees every key of the dense K/V."""
    S, R = 3, 42
    w = W.make_admit(cuda_device, S, R, n, seed=25)
    P = -(-n // 16) - 2                          # the last 17-32 positions of every sequence have no page
    bt = _table(S, P, 128, False, seed=26)
    bt[0, 1] = -1                                # positions 16..31 of sequence 0
    bt[2, 0] = 1 << 20                           # past num_pages: positions 0..15 of sequence 2
    out, _, _, nw = _run_both(cuda_device, w.q, w.k, w.v, bt, 16, 128, w.scale)
    assert nw == S * min(n, 16 * P) - 32
    _oracle_check(out, w.q, w.k, w.v, w.scale, f"prefill_dense_append short table n={n}")


@pytest.mark.parametrize("n", [77, 300])
def test_dense_append_strided_inputs(cuda_device, n):
    """q, K and V as views with their own strides (V as the second half of a [S, n, 16, 128] buffer, K with a padded
    sequence stride), as producers other than torch.cat would hand them over."""
    S, R = 3, 42
    w = W.make_admit(cuda_device, S, R, n, seed=27)
    vbuf = torch.zeros(S, n, 16, 128, dtype=torch.bfloat16, device=cuda_device)
    vbuf[:, :, 8:] = w.v
    v = vbuf[:, :, 8:]
    kbuf = torch.zeros(S, n + 5, 8, 128, dtype=torch.bfloat16, device=cuda_device)
    kbuf[:, :n] = w.k
    k = kbuf[:, :n]
    qbuf = torch.zeros(S, R, 24, 128, dtype=torch.bfloat16, device=cuda_device)
    qbuf[:, :, 4:20] = w.q
    q = qbuf[:, :, 4:20]
    bt = _table(S, -(-n // 16), 96, False, seed=28)
    out, _, _, nw = _run_both(cuda_device, q, k, v, bt, 16, 96, w.scale)
    assert nw == S * n
    _oracle_check(out, w.q, w.k, w.v, w.scale, f"prefill_dense_append strided n={n}")


@pytest.mark.parametrize("n", [77, 300])
def test_dense_append_in_graph_replays(cuda_device, n):
    S, R = 8, 42
    w = W.make_admit(cuda_device, S, R, n, seed=29)
    P = -(-n // 16)
    bt = torch.from_numpy(_table(S, P, 256, False, seed=30)).to(cuda_device)
    kc = torch.zeros(256, 16, 8, 128, dtype=torch.bfloat16, device=cuda_device)
    vc = torch.zeros_like(kc)
    eager = q3attn.prefill_dense_append(w.q, w.k, w.v, kc, vc, bt, w.scale, True, 0)
    torch.cuda.synchronize()
    k_ref, v_ref = kc.clone(), vc.clone()
    s = torch.cuda.Stream(cuda_device)
    s.wait_stream(torch.cuda.current_stream(cuda_device))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        static = q3attn.prefill_dense_append(w.q, w.k, w.v, kc, vc, bt, w.scale, True, 0)
    for _ in range(3):
        kc.fill_(float("nan"))
        vc.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(static, eager)
        assert torch.equal(torch.nan_to_num(kc), torch.nan_to_num(k_ref))
        assert torch.equal(torch.nan_to_num(vc), torch.nan_to_num(v_ref))
