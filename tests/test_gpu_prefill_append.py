"""GPU parity of the fused prompt step (q3a_prefill_append through the C ABI): the K and V rows of every prompt token
go into the paged pool (engine/talker.py:161-162 scatters them with index_copy_ at seat * seat_len + position) and the
attention runs over the packed k/v (engine/talker.py:169).  Against that two-step sequence the output and the pool
must be bit-identical; the pool starts NaN-filled, so every slot the call should write is checked, and every other
slot must stay NaN.  The output is also checked against the oracle."""
import numpy as np
import pytest
import torch

import q3attn
from helpers import to_np
from oracle import attention as ora
from q3attn import workloads as W

pytestmark = pytest.mark.gpu


def _table(n, P, num_pages, identity, seed):
    if identity:
        return np.arange(n * P, dtype=np.int32).reshape(n, P)
    return np.random.default_rng(seed).permutation(num_pages)[: n * P].reshape(n, P).astype(np.int32)


def _slots(cu_q, cu_k, bt, page, max_pages):
    """Flat pool slot and packed k row of every written token: positions Lk - Lq .. Lk - 1 of each sequence."""
    slots, rows = [], []
    for s in range(len(cu_q) - 1):
        Lq, Lk = cu_q[s + 1] - cu_q[s], cu_k[s + 1] - cu_k[s]
        for i in range(Lq):
            p = Lk - Lq + i
            if p < 0 or p // page >= max_pages or bt[s, p // page] < 0:
                continue
            slots.append(int(bt[s, p // page]) * page + p % page)
            rows.append(int(cu_k[s]) + p)
    return np.array(slots, dtype=np.int64), np.array(rows, dtype=np.int64)


def _run_both(dev, q, k, v, cu_q, cu_k, max_q, bt_np, page, num_pages, scale, causal=True):
    Hkv = k.shape[1]
    kc = torch.full((num_pages, page, Hkv, 128), float("nan"), dtype=torch.bfloat16, device=dev)
    vc = torch.full_like(kc, float("nan"))
    bt = torch.from_numpy(bt_np).to(dev)
    cq, ck = torch.from_numpy(cu_q).to(dev), torch.from_numpy(cu_k).to(dev)
    out = q3attn.prefill_append(q, k, v, cq, ck, max_q, kc, vc, bt, scale, causal)
    torch.cuda.synchronize()
    # the two-step reference: index_copy_ of the rows, then the packed prefill
    rk, rv = torch.full_like(kc, float("nan")), torch.full_like(vc, float("nan"))
    slots, rows = _slots(cu_q, cu_k, bt_np, page, bt_np.shape[1])
    si, ri = torch.from_numpy(slots).to(dev), torch.from_numpy(rows).to(dev)
    rk.view(-1, Hkv, 128).index_copy_(0, si, k[ri])
    rv.view(-1, Hkv, 128).index_copy_(0, si, v[ri])
    ref = q3attn.flash_attn_varlen_func(q, k, v, cq, ck, max_q, int((cu_k[1:] - cu_k[:-1]).max()),
                                        softmax_scale=scale, causal=causal)
    torch.cuda.synchronize()
    assert torch.equal(out, ref), "output differs from the packed prefill"
    # NaN-aware pool comparison: written slots equal, untouched slots still NaN in both
    assert torch.equal(torch.isnan(kc), torch.isnan(rk)) and torch.equal(torch.isnan(vc), torch.isnan(rv))
    assert torch.equal(torch.nan_to_num(kc), torch.nan_to_num(rk)) and torch.equal(torch.nan_to_num(vc), torch.nan_to_num(rv))
    return out, kc, vc, len(slots)


@pytest.mark.parametrize("lens,page,identity", [
    ([1, 7, 16, 17, 33, 64, 65, 150, 3], 16, False),
    ([77, 300, 5], 256, True),                 # the reference's own pool: 256-token pages, identity seats
    (None, 16, False),                         # the 32-sequence prefill workload (U[150, 400] tokens)
    ("grouped", 16, False),                    # 48 sequences of up to 500 tokens: the grouped work order
])
def test_prefill_append_matches_scatter_then_prefill(cuda_device, lens, page, identity):
    if lens == "grouped":
        lens = np.random.default_rng(13).integers(1, 500, 48)
        lens[0] = 499
    lens = W.prefill_lengths("prefill32") if lens is None else np.array(lens)
    wl = W.make_prefill(cuda_device, lens, seed=11, paged=False)
    cu = wl.cu_seqlens.cpu().numpy()
    P = int(-(-lens.max() // page))
    num_pages = max(len(lens) * P * 2, 64)
    bt = _table(len(lens), P, num_pages, identity, seed=12)
    out, kc, _, nw = _run_both(cuda_device, wl.q, wl.k, wl.v, cu, cu, wl.max_len, bt, page, num_pages, wl.scale)
    assert nw == int(lens.sum())
    ok, st = ora.compare(to_np(out), ora.prefill_varlen(to_np(wl.q), to_np(wl.k), to_np(wl.v), cu, wl.scale))
    print(f"[parity] prefill_append {len(lens)} seqs page {page} vs oracle {st}", flush=True)
    assert ok, st


def test_prefill_append_prefix_writes_only_new_tokens(cuda_device):
    """cu_seqlens_k != cu_seqlens_q (a K/V prefix before the new tokens): positions Lk - Lq .. Lk - 1 are written,
    the prefix slots are left alone."""
    S, R, n = 4, 42, 77
    w = W.make_admit(cuda_device, S, R, n, seed=13)
    q = w.q.reshape(S * R, 16, 128)
    k = w.k.reshape(S * n, 8, 128)
    v = w.v.reshape(S * n, 8, 128)
    cu_q = np.arange(0, S * R + 1, R, dtype=np.int32)
    cu_k = np.arange(0, S * n + 1, n, dtype=np.int32)
    bt = _table(S, 5, 64, False, seed=14)
    out, kc, _, nw = _run_both(cuda_device, q, k, v, cu_q, cu_k, R, bt, 16, 64, w.scale)
    assert nw == S * R
    prefix = [int(bt[s, p // 16]) * 16 + p % 16 for s in range(S) for p in range(n - R)]
    assert torch.isnan(kc.view(-1, 8, 128)[torch.tensor(prefix, device=cuda_device)]).all()


def test_prefill_append_strided_v_and_short_table(cuda_device):
    """v as a view of a fused qkv projection (token stride 4096, engine/talker.py:160); a table with fewer pages than
    the longest sequence and an invalid entry: those positions are not written (and nothing faults)."""
    lens = np.array([40, 100, 64])
    wl = W.make_prefill(cuda_device, lens, seed=15, paged=False)
    T = int(lens.sum())
    qkv = torch.zeros(T, 4096, dtype=torch.bfloat16, device=cuda_device)
    qkv[:, 3072:] = wl.v.reshape(T, 1024)
    v = qkv[:, 3072:].view(T, 8, 128)
    cu = wl.cu_seqlens.cpu().numpy()
    bt = _table(3, 5, 64, False, seed=16)       # 5 pages = 80 positions: sequence 1 keeps 20 tokens unwritten
    bt[2, 1] = -1                               # positions 16..31 of sequence 2 have no page
    out, kc, _, nw = _run_both(cuda_device, wl.q, wl.k, v, cu, cu, wl.max_len, bt, 16, 64, wl.scale)
    assert nw == 40 + 80 + 48


def test_prefill_append_in_graph_replays(cuda_device):
    lens = np.array([150, 33, 260, 1, 97])
    wl = W.make_prefill(cuda_device, lens, seed=17, paged=False)
    cu = wl.cu_seqlens.to(cuda_device)
    P = int(-(-lens.max() // 16))
    bt = torch.from_numpy(_table(len(lens), P, 256, False, seed=18)).to(cuda_device)
    kc = torch.zeros(256, 16, 8, 128, dtype=torch.bfloat16, device=cuda_device)
    vc = torch.zeros_like(kc)
    eager = q3attn.prefill_append(wl.q, wl.k, wl.v, cu, cu, wl.max_len, kc, vc, bt, wl.scale, True)
    torch.cuda.synchronize()
    k_ref, v_ref = kc.clone(), vc.clone()
    s = torch.cuda.Stream(cuda_device)
    s.wait_stream(torch.cuda.current_stream(cuda_device))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        static = q3attn.prefill_append(wl.q, wl.k, wl.v, cu, cu, wl.max_len, kc, vc, bt, wl.scale, True)
    for _ in range(3):
        kc.fill_(float("nan"))
        vc.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(static, eager)
        written = ~torch.isnan(kc)
        assert torch.equal(kc[written], k_ref[written]) and torch.equal(vc[written], v_ref[written])
        assert int(written.view(-1, 8 * 128).all(dim=1).sum()) == int(lens.sum())
