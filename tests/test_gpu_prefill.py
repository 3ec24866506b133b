"""GPU parity of the MFMA prefill (q3a_prefill through the C ABI) against the oracle: packed varlen causal
(engine/talker.py:169), read back from the paged pool (32 sequences of U[150,400] tokens), the prefix + new bottom-right form
(engine/arrivals.py:148), non-causal, and query rows that see no key."""
import numpy as np
import pytest
import torch

import q3attn
from helpers import to_np
from oracle import attention as ora
from q3attn import workloads as W

pytestmark = pytest.mark.gpu


def oracle_varlen(wl):
    cu = wl.cu_seqlens.cpu().numpy()
    return ora.prefill_varlen(to_np(wl.q), to_np(wl.k), to_np(wl.v), cu, wl.scale)


def check(out, ref, what):
    ok, st = ora.compare(to_np(out), ref)
    print(f"[parity] {what} {st}", flush=True)
    assert ok, (what, st)


def test_packed_varlen_causal(cuda_device):
    lens = [1, 7, 16, 17, 33, 64, 65, 150, 3]
    wl = W.make_prefill(cuda_device, lens, seed=1, paged=False)
    out = q3attn.flash_attn_varlen_func(wl.q, wl.k, wl.v, wl.cu_seqlens, wl.cu_seqlens, wl.max_len, wl.max_len,
                                        softmax_scale=wl.scale, causal=True)
    torch.cuda.synchronize()
    check(out, oracle_varlen(wl), "packed varlen")


def test_paged_prefill32_full(cuda_device):
    lens = W.prefill_lengths("prefill32")
    wl = W.make_prefill(cuda_device, lens, seed=0, paged=True, num_pages=4096)
    out = q3attn.flash_attn_varlen_func(wl.q, wl.k_cache, wl.v_cache, wl.cu_seqlens, wl.cu_seqlens, wl.max_len,
                                        wl.max_len, softmax_scale=wl.scale, causal=True, block_table=wl.block_table)
    torch.cuda.synchronize()
    ref = oracle_varlen(wl)
    check(out, ref, "c4 paged")
    packed = q3attn.flash_attn_varlen_func(wl.q, wl.k, wl.v, wl.cu_seqlens, wl.cu_seqlens, wl.max_len, wl.max_len,
                                           softmax_scale=wl.scale, causal=True)
    torch.cuda.synchronize()
    assert torch.equal(out, packed), "paged and packed K/V sources must give identical results"


def test_reference_layout_page256_identity(cuda_device):
    wl = W.make_prefill(cuda_device, [77, 300, 5], seed=2, paged=True, page=256, identity=True)
    out = q3attn.flash_attn_varlen_func(wl.q, wl.k_cache, wl.v_cache, wl.cu_seqlens, wl.cu_seqlens, wl.max_len,
                                        wl.max_len, softmax_scale=wl.scale, causal=True, block_table=wl.block_table)
    torch.cuda.synchronize()
    check(out, oracle_varlen(wl), "page256")


@pytest.mark.parametrize("S,R,n", [(4, 42, 77), (1, 5, 5), (8, 42, 77), (2, 70, 200)])
def test_prefix_bottom_right(cuda_device, S, R, n):
    """FastAdmit's dense form (engine/arrivals.py:118, 148): the k = n - R prefix keys plus R new keys."""
    g = torch.Generator(device=cuda_device).manual_seed(S * 1000 + R)
    q = torch.randn(S, R, 16, 128, generator=g, device=cuda_device).to(torch.bfloat16)
    K = torch.randn(S, n, 8, 128, generator=g, device=cuda_device).to(torch.bfloat16)
    V = torch.randn(S, n, 8, 128, generator=g, device=cuda_device).to(torch.bfloat16)
    out = q3attn.flash_attn_func(q, K, V, softmax_scale=128 ** -0.5, causal=True)
    torch.cuda.synchronize()
    check(out, ora.prefill_prefix(to_np(q), to_np(K), to_np(V), 128 ** -0.5), f"prefix S={S} R={R} n={n}")


def test_non_causal(cuda_device):
    lens = [9, 40, 129]
    wl = W.make_prefill(cuda_device, lens, seed=3, paged=False)
    out = q3attn.flash_attn_varlen_func(wl.q, wl.k, wl.v, wl.cu_seqlens, wl.cu_seqlens, wl.max_len, wl.max_len,
                                        softmax_scale=wl.scale, causal=False)
    torch.cuda.synchronize()
    q, k, v = to_np(wl.q), to_np(wl.k), to_np(wl.v)
    cu = wl.cu_seqlens.cpu().numpy()
    ref = np.zeros_like(q)
    for i in range(len(lens)):
        s = slice(cu[i], cu[i + 1])
        ref[s] = _dense(q[s], k[s], v[s], wl.scale)
    check(out, ref, "non-causal")


def _dense(q, k, v, scale):
    G = q.shape[1] // k.shape[1]
    kk = np.repeat(k, G, axis=1).astype(np.float64)
    vv = np.repeat(v, G, axis=1).astype(np.float64)
    a = np.einsum("thd,shd->hts", q.astype(np.float64), kk) * scale
    a -= a.max(-1, keepdims=True)
    p = np.exp(a)
    p /= p.sum(-1, keepdims=True)
    return np.einsum("hts,shd->thd", p, vv)


def test_query_rows_without_keys_are_zero(cuda_device):
    """Lq > Lk with bottom-right alignment: the first Lq - Lk queries see no key."""
    g = torch.Generator(device=cuda_device).manual_seed(5)
    q = torch.randn(1, 20, 16, 128, generator=g, device=cuda_device).to(torch.bfloat16)
    K = torch.randn(1, 12, 8, 128, generator=g, device=cuda_device).to(torch.bfloat16)
    V = torch.randn(1, 12, 8, 128, generator=g, device=cuda_device).to(torch.bfloat16)
    out = q3attn.flash_attn_func(q, K, V, softmax_scale=0.1, causal=True)
    torch.cuda.synchronize()
    assert not out[0, :8].float().abs().sum().item()
    ref = ora.prefill_prefix(to_np(q[:, 8:]), to_np(K), to_np(V), 0.1)
    check(out[:, 8:], ref, "rows with keys")


def test_graph_capture_prefill(cuda_device):
    wl = W.make_prefill(cuda_device, [33, 100], seed=4, paged=True, num_pages=64)
    f = lambda: q3attn.flash_attn_varlen_func(wl.q, wl.k_cache, wl.v_cache, wl.cu_seqlens, wl.cu_seqlens, 100, 100,
                                              softmax_scale=wl.scale, causal=True, block_table=wl.block_table)
    eager = f().clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        f()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        static = f()
    for _ in range(3):
        torch.randn(1 << 18, device=cuda_device)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(static, eager)


def test_flash_attn_func_strided_views(cuda_device):
    """q, K, V as views into wider tensors (the engine slices them out of projection outputs): the dense entry
    point reads them through their strides, no copies."""
    g = torch.Generator(device=cuda_device).manual_seed(11)
    S, R, n = 3, 42, 77
    qbig = torch.randn(S, R, 24, 128, generator=g, device=cuda_device).to(torch.bfloat16)
    kvbig = torch.randn(S, n + 5, 2, 12, 128, generator=g, device=cuda_device).to(torch.bfloat16)
    q, K, V = qbig[:, :, 4:20], kvbig[:, 5:, 0, 2:10], kvbig[:, 5:, 1, 2:10]
    assert not q.is_contiguous() and not K.is_contiguous()
    out = q3attn.flash_attn_func(q, K, V, softmax_scale=128 ** -0.5, causal=True)
    torch.cuda.synchronize()
    check(out, ora.prefill_prefix(to_np(q), to_np(K), to_np(V), 128 ** -0.5), "strided prefix views")
    out_c = q3attn.flash_attn_func(q.contiguous(), K.contiguous(), V.contiguous(), softmax_scale=128 ** -0.5,
                                   causal=True)
    assert torch.equal(out, out_c)


def test_graph_capture_flash_attn_func(cuda_device):
    """The admission path captures flash_attn_func in graphs (engine/arrivals.py:133-166): replays equal the eager
    result, with other work between replays."""
    wl = W.make_admit(cuda_device, 4, 42, 77, seed=12)
    f = lambda: q3attn.flash_attn_func(wl.q, wl.k, wl.v, softmax_scale=wl.scale, causal=True)
    eager = f().clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        f()
    torch.cuda.current_stream().wait_stream(s)
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr, stream=s):
        static = f()
    for _ in range(3):
        torch.randn(1 << 18, device=cuda_device)
        gr.replay()
        torch.cuda.synchronize()
        assert torch.equal(static, eager)
    check(eager, ora.prefill_prefix(to_np(wl.q), to_np(wl.k), to_np(wl.v), wl.scale), "admission shape")


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("R,n", [(1, 1), (1, 77), (16, 16), (17, 32), (17, 33), (42, 64), (42, 77), (5, 100),
                                 (42, 128), (42, 129), (33, 20)])
def test_flash_attn_func_short_key_ranges(cuda_device, R, n, causal):
    """Key ranges of at most 128 go to the short-key kernel (the whole K/V range in LDS, one wave per 16 query tokens
    and query head); 129 keys and more to the tiled kernel.  Both must agree with the oracle on either side of the boundary, causal (bottom-right)
    or not; with R > n the first R - n queries see no key under the causal mask and are zeros."""
    g = torch.Generator(device=cuda_device).manual_seed(R * 1000 + n)
    S = 3
    q = torch.randn(S, R, 16, 128, generator=g, device=cuda_device).to(torch.bfloat16)
    K = torch.randn(S, n, 8, 128, generator=g, device=cuda_device).to(torch.bfloat16)
    V = torch.randn(S, n, 8, 128, generator=g, device=cuda_device).to(torch.bfloat16)
    out = q3attn.flash_attn_func(q, K, V, softmax_scale=128 ** -0.5, causal=causal)
    torch.cuda.synchronize()
    qn, Kn, Vn = to_np(q), to_np(K), to_np(V)
    if causal:
        skip = max(0, R - n)
        if skip:
            assert not out[:, :skip].float().abs().sum().item()
        ref = ora.prefill_prefix(qn[:, skip:], Kn, Vn, 128 ** -0.5)
        check(out[:, skip:], ref, f"short keys R={R} n={n} causal")
    else:
        ref = np.stack([_dense(qn[i], Kn[i], Vn[i], 128 ** -0.5) for i in range(S)])
        check(out, ref, f"short keys R={R} n={n} non-causal")


@pytest.mark.parametrize("hkv", [8, 4, 16])
@pytest.mark.parametrize("causal", [True, False])
def test_varlen_many_sequences(cuda_device, hkv, causal):
    """120 packed sequences of 0..299 tokens (zero-length and one-token ones included) with 4, 8 or 16 KV heads:
    more workgroups than the GPU holds at once.  Within the bar of the oracle, and graph replays equal the eager
    call."""
    rng = np.random.default_rng(hkv * 10 + int(causal))
    lens = rng.integers(0, 300, size=120)
    lens[:4] = [0, 1, 299, 0]
    T = int(lens.sum())
    g = torch.Generator(device=cuda_device).manual_seed(hkv)
    q = torch.randn(T, 2 * hkv, 128, generator=g, device=cuda_device).to(torch.bfloat16)
    k = torch.randn(T, hkv, 128, generator=g, device=cuda_device).to(torch.bfloat16)
    v = torch.randn(T, hkv, 128, generator=g, device=cuda_device).to(torch.bfloat16)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32, device=cuda_device)
    max_q = int(lens.max())
    scale = 128 ** -0.5
    f = lambda: q3attn.flash_attn_varlen_func(q, k, v, cu, cu, max_q, max_q, softmax_scale=scale, causal=causal)
    out = f()
    torch.cuda.synchronize()
    qn, kn, vn, cun = to_np(q), to_np(k), to_np(v), cu.cpu().numpy()
    if causal:
        ref = ora.prefill_varlen(qn, kn, vn, cun, scale)
    else:
        ref = np.zeros_like(qn)
        for i in range(len(lens)):
            sl = slice(cun[i], cun[i + 1])
            if lens[i]:
                ref[sl] = _dense(qn[sl], kn[sl], vn[sl], scale)
    check(out, ref, f"varlen 120 seqs hkv={hkv} causal={causal}")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        f()
    torch.cuda.current_stream().wait_stream(s)
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr, stream=s):
        static = f()
    for _ in range(3):
        torch.randn(1 << 18, device=cuda_device)
        gr.replay()
        torch.cuda.synchronize()
        assert torch.equal(static, out)


@pytest.mark.parametrize("case", ["64 seqs", "ties", "one long", "grouped", "grouped, max_seqlen above longest"])
def test_varlen_work_orders(cuda_device, case):
    """Both work orders of the tiled kernel: all sequences' query tiles longest first (grids of up to about three
    rounds of resident workgroups), and groups of sequences one after another (larger grids: 45 sequences of up
    to 500 tokens, a partial last group, zero-length sequences, and a max_seqlen_q above every length so that
    whole query-tile rows are empty).  Equal lengths and one long sequence among short ones.  Within the bar of
    the oracle."""
    rng = np.random.default_rng(len(case))
    lens = {"64 seqs": rng.integers(0, 200, 64),
            "ties": np.array([128, 64, 128, 1, 128, 64, 0, 65] * 3),
            "one long": np.array([5, 17, 700, 3, 64, 1]),
            "grouped": rng.integers(0, 500, 45),
            "grouped, max_seqlen above longest": rng.integers(1, 300, 45)}[case]
    lens[0] = max(lens[0], 1)
    hkv = 8
    T = int(lens.sum())
    g = torch.Generator(device=cuda_device).manual_seed(len(case))
    q = torch.randn(T, 2 * hkv, 128, generator=g, device=cuda_device).to(torch.bfloat16)
    k = torch.randn(T, hkv, 128, generator=g, device=cuda_device).to(torch.bfloat16)
    v = torch.randn(T, hkv, 128, generator=g, device=cuda_device).to(torch.bfloat16)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32, device=cuda_device)
    max_q = int(lens.max()) + (200 if "above" in case else 0)
    out = q3attn.flash_attn_varlen_func(q, k, v, cu, cu, max_q, max_q, softmax_scale=128 ** -0.5, causal=True)
    torch.cuda.synchronize()
    ref = ora.prefill_varlen(to_np(q), to_np(k), to_np(v), cu.cpu().numpy(), 128 ** -0.5)
    check(out, ref, f"work order: {case}")


@pytest.mark.parametrize("S,L", [(5, 300), (40, 640)])
def test_dense_work_order(cuda_device, S, L):
    """The dense form with key ranges past the short-range kernel, in both work orders (40 x 640 runs in groups of
    4 sequences), against the oracle."""
    g = torch.Generator(device=cuda_device).manual_seed(S * 100 + L)
    q = torch.randn(S, L, 16, 128, generator=g, device=cuda_device).to(torch.bfloat16)
    K = torch.randn(S, L, 8, 128, generator=g, device=cuda_device).to(torch.bfloat16)
    V = torch.randn(S, L, 8, 128, generator=g, device=cuda_device).to(torch.bfloat16)
    out = q3attn.flash_attn_func(q, K, V, softmax_scale=128 ** -0.5, causal=True)
    torch.cuda.synchronize()
    check(out, ora.prefill_prefix(to_np(q), to_np(K), to_np(V), 128 ** -0.5), f"dense S={S} L={L}")
