"""GPU parity of the fused q/k norm + RoPE + KV append + decode (q3a_paged_decode_append_rope via the C ABI).

The reference block is engine/talker.py:69-77: q = rope(rms(q_raw, qn)), k = rope(rms(k_raw, kn)) (engine/ops.py:51-60),
k and v written into the pool with index_copy_, then the paged attention.  Expected values come from the oracle's
restatement of the producers as the compiled talker evaluates them (oracle.attention.norm_rope, eager=False: float32
throughout, one rounding) and its decode attention.

Two kinds of check:
* exact inputs: head rows of +-1 entries with eps = 0 have mean(x^2) = 1 and 1/sqrt of it 1, so the normalised row is
  exactly +-w and the rope products are exact; the fused call must then match paged_decode_append on the oracle's q
  and k bit for bit, output and pool (this also proves the slot receives the k the new token was attended with);
* random inputs: output within the 2e-2 / 2e-3 bar of the oracle, the written k rows within the bound a one-unit
  change of the normalised value allows (fp32 sums of squares in another order, _k_rows_close) and at least 99 %
  bit-identical."""
import numpy as np
import pytest
import torch

import q3attn
from helpers import decode_oracle, to_np
from oracle import attention as ora
from q3attn import workloads as W

pytestmark = pytest.mark.gpu

RAGGED = [0, 1, 2, 3, 4, 5, 15, 16, 17, 31, 32, 33, 63, 64, 65, 100, 127, 128, 129, 200, 255, 256, 257, 511,
          700, 1023, 1800]
SK_CTX = 2064   # tables wider than 2,048 tokens take stream-K at any batch; narrower ones up to 64 rows the row kernel
EPS = 1e-6


def _bf16(x: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(dev).to(torch.bfloat16)


def _slots(wl):
    """Flat slot of each live row's new token (position ctx - 1), -1 for ctx 0."""
    page = wl.page_size
    bt = wl.layers[0].block_table.cpu().numpy().astype(np.int64)
    pos = wl.ctx - 1
    s = np.full(wl.batch, -1, np.int64)
    live = pos >= 0
    s[live] = bt[np.arange(wl.batch)[live], pos[live] // page] * page + pos[live] % page
    return s


def _inputs(wl, seed, exact):
    """Raw q/k/v, norm weights and per-row cos/sin (bf16 tables at each row's new position)."""
    rng = np.random.default_rng(seed)
    B = wl.batch
    if exact:
        q = rng.choice([-1.0, 1.0], size=(B, W.HQ, W.HEAD_DIM))
        k = rng.choice([-1.0, 1.0], size=(B, W.HKV, W.HEAD_DIM))
    else:
        q = rng.standard_normal((B, W.HQ, W.HEAD_DIM)) * rng.uniform(0.2, 5.0, size=(B, W.HQ, 1))
        k = rng.standard_normal((B, W.HKV, W.HEAD_DIM)) * rng.uniform(0.2, 5.0, size=(B, W.HKV, 1))
    v = rng.standard_normal((B, W.HKV, W.HEAD_DIM))
    qn = rng.uniform(0.5, 1.5, size=W.HEAD_DIM)
    kn = rng.uniform(0.5, 1.5, size=W.HEAD_DIM)
    cos_t, sin_t = ora.rope_tables(int(max(wl.ctx.max(), 1)))
    pos = np.maximum(wl.ctx - 1, 0)
    r = lambda x: ora.bf16_round(np.asarray(x, np.float32))
    return r(q), r(k), r(v), r(qn), r(kn), r(cos_t[pos]), r(sin_t[pos])


def _k_rows_close(got, k, kn, kk):
    """The written k rows against the oracle's: a sum of squares taken in another order moves r by an fp32 unit, which
    moves y*cos + rot(y)*sin by far less than 2^-8 (|y| + |rot(y)|) before its own rounding (2^-8 |k'|); beyond that
    bound a row is wrong.  Returns (all within, fraction bit-identical)."""
    y = ora.rms(k, kn, eps=EPS)
    rot = np.concatenate([-y[..., 64:], y[..., :64]], axis=-1)
    bound = 2.0 ** -8 * (np.abs(y) + np.abs(rot)) + 2.0 ** -7 * np.abs(kk) + 1e-30
    d = np.abs(got - kk)
    return bool((d <= bound).all()), float((d == 0).mean())


def _oracle_qk(q, k, qn, kn, cos, sin, eps=EPS):
    """q' and k' as the oracle computes them (bf16 values in float32)."""
    qq = ora.norm_rope(q, qn, cos[:, None, :], sin[:, None, :], eps, eager=False)
    kk = ora.norm_rope(k, kn, cos[:, None, :], sin[:, None, :], eps, eager=False)
    return qq, kk


def _run(wl, seed, exact, qkv_views=False, cs3=False):
    eps = 0.0 if exact else EPS
    dev = wl.k_cache.device
    q, k, v, qn, kn, cos, sin = _inputs(wl, seed, exact)
    B = wl.batch
    slots = _slots(wl)
    live = slots >= 0
    kflat = wl.k_cache.view(-1, W.HKV, W.HEAD_DIM)
    vflat = wl.v_cache.view(-1, W.HKV, W.HEAD_DIM)
    pristine_k, pristine_v = wl.k_cache.clone(), wl.v_cache.clone()
    live_idx = torch.from_numpy(slots[live]).to(dev)
    kflat.index_fill_(0, live_idx, float("nan"))
    vflat.index_fill_(0, live_idx, float("nan"))
    old = torch.from_numpy(wl.ctx - 1).to(torch.int32).to(dev)
    if qkv_views:   # q, k, v as views of one fused [B, 4096] projection, as engine/talker.py:68-71 slices them
        qkv = torch.cat([_bf16(q.reshape(B, -1), dev), _bf16(k.reshape(B, -1), dev), _bf16(v.reshape(B, -1), dev)], 1)
        qt = qkv[:, :2048].view(B, W.HQ, W.HEAD_DIM)
        kt = qkv[:, 2048:3072].view(B, W.HKV, W.HEAD_DIM)
        vt = qkv[:, 3072:].view(B, W.HKV, W.HEAD_DIM)
    else:
        qt, kt, vt = _bf16(q, dev), _bf16(k, dev), _bf16(v, dev)
    ct, st = _bf16(cos, dev), _bf16(sin, dev)
    if cs3:         # the talker's [B, 1, 128] rows (engine/talker.py:108)
        ct, st = ct[:, None, :], st[:, None, :]
    L = wl.layers[0]
    out = q3attn.paged_decode_append_rope(qt, kt, vt, _bf16(qn, dev), _bf16(kn, dev), ct, st, wl.k_cache, wl.v_cache,
                                          old, L.block_table, wl.scale, eps)
    torch.cuda.synchronize()
    qq, kk = _oracle_qk(q, k, qn, kn, cos, sin, eps)
    return out, qq, kk, v, old, pristine_k, pristine_v, slots


def _expected_pool(wl, pristine_k, pristine_v, kk, v, slots):
    dev = wl.k_cache.device
    live = slots >= 0
    ek, ev = pristine_k.clone(), pristine_v.clone()
    idx = torch.from_numpy(slots[live]).to(dev)
    ek.view(-1, W.HKV, W.HEAD_DIM).index_copy_(0, idx, _bf16(kk[live], dev))
    ev.view(-1, W.HKV, W.HEAD_DIM).index_copy_(0, idx, _bf16(v[live], dev))
    return ek, ev


@pytest.mark.parametrize("max_ctx", [1800, SK_CTX])
def test_exact_inputs_match_append_on_oracle_qk(cuda_device, max_ctx):
    """+-1 rows: q', k' are exact, so the fused call equals paged_decode_append(q', k', v) bit for bit."""
    wl = W.make_decode("rope", cuda_device, ctx=np.array(RAGGED), num_pages=4096, max_ctx=max_ctx, seed=31)
    out, qq, kk, v, old, pk, pv, slots = _run(wl, 5, exact=True)
    ek, ev = _expected_pool(wl, pk, pv, kk, v, slots)
    assert torch.equal(wl.k_cache, ek) and torch.equal(wl.v_cache, ev), "pool differs from the oracle's k', v"
    # The unfused path on the oracle's q', k' over a pristine pool (its own slot writes give the same pool).
    wl.k_cache.copy_(pk)
    wl.v_cache.copy_(pv)
    dev = cuda_device
    L = wl.layers[0]
    ref = q3attn.paged_decode_append(_bf16(qq, dev), _bf16(kk, dev), _bf16(v, dev), wl.k_cache, wl.v_cache, old,
                                     L.block_table, wl.scale)
    torch.cuda.synchronize()
    assert torch.equal(out, ref), f"fused output differs from append on the oracle's q', k' (max_ctx {max_ctx})"
    assert not out[0].float().abs().sum().item(), "row with ctx 0 must be zeros"


@pytest.mark.parametrize("max_ctx,views,cs3", [(1800, False, False), (SK_CTX, False, False), (SK_CTX, True, True),
                                               (1800, True, True)])
def test_random_inputs_vs_oracle(cuda_device, max_ctx, views, cs3):
    wl = W.make_decode("rope", cuda_device, ctx=np.array(RAGGED), num_pages=4096, max_ctx=max_ctx, seed=32)
    out, qq, kk, v, old, pk, pv, slots = _run(wl, 6, exact=False, qkv_views=views, cs3=cs3)
    live = slots >= 0
    dev = cuda_device
    idx = torch.from_numpy(slots[live]).to(dev)
    got_k = to_np(wl.k_cache.view(-1, W.HKV, W.HEAD_DIM).index_select(0, idx))
    got_v = to_np(wl.v_cache.view(-1, W.HKV, W.HEAD_DIM).index_select(0, idx))
    assert np.array_equal(got_v, v[live]), "v rows must be stored as given"
    inp = _inputs(wl, 6, exact=False)
    within, exact = _k_rows_close(got_k, inp[1][live], inp[4], kk[live])
    print(f"[parity] rope k rows bit-identical to the oracle: {exact:.4f}", flush=True)
    assert within and exact >= 0.99
    # Every other slot is untouched.
    keep = torch.ones(wl.k_cache.shape[0] * wl.page_size, dtype=torch.bool, device=dev)
    keep[idx] = False
    kf, pkf = wl.k_cache.view(-1, W.HKV, W.HEAD_DIM), pk.view(-1, W.HKV, W.HEAD_DIM)
    assert torch.equal(kf[keep], pkf[keep]) and torch.equal(wl.v_cache.view(-1, W.HKV, W.HEAD_DIM)[keep],
                                                            pv.view(-1, W.HKV, W.HEAD_DIM)[keep])
    # Oracle attention over the pool as the oracle would leave it, with its own q'.
    ek, ev = _expected_pool(wl, pk, pv, kk, v, slots)
    wl.k_cache.copy_(ek)
    wl.v_cache.copy_(ev)
    wl.layers[0].q = _bf16(qq, dev)
    ok, st = ora.compare(to_np(out), decode_oracle(wl))
    print(f"[parity] rope max_ctx={max_ctx} views={views} vs oracle {st}", flush=True)
    assert ok, st
    assert not out[0].float().abs().sum().item()


def test_full_size_576_rows_vs_oracle(cuda_device):
    """The 576-row workload (stream-K), every row against the oracle."""
    wl = W.make_decode("decode576", cuda_device, layers=1, seed=7)
    out, qq, kk, v, old, pk, pv, slots = _run(wl, 8, exact=False, qkv_views=True, cs3=True)
    ek, ev = _expected_pool(wl, pk, pv, kk, v, slots)
    live = slots >= 0
    idx = torch.from_numpy(slots[live]).to(cuda_device)
    inp = _inputs(wl, 8, exact=False)
    within, exact = _k_rows_close(to_np(wl.k_cache.view(-1, W.HKV, W.HEAD_DIM).index_select(0, idx)), inp[1][live],
                                  inp[4], kk[live])
    print(f"[parity] rope 576 rows: k rows bit-identical to the oracle: {exact:.4f}", flush=True)
    assert within and exact >= 0.99
    wl.k_cache.copy_(ek)
    wl.v_cache.copy_(ev)
    wl.layers[0].q = _bf16(qq, cuda_device)
    ok, st = ora.compare(to_np(out), decode_oracle(wl))
    print(f"[parity] rope 576 rows vs oracle {st}", flush=True)
    assert ok, st
    assert not out[wl.ctx == 0].float().abs().sum().item(), "padded rows must be zeros"


@pytest.mark.parametrize("max_ctx", [1800, SK_CTX])
def test_graph_replays_match_eager(cuda_device, max_ctx):
    wl = W.make_decode("rope", cuda_device, ctx=np.array(RAGGED), num_pages=4096, max_ctx=max_ctx, seed=33)
    dev = cuda_device
    q, k, v, qn, kn, cos, sin = _inputs(wl, 9, exact=False)
    args = [_bf16(x, dev) for x in (q, k, v, qn, kn, cos, sin)]
    old = torch.from_numpy(wl.ctx - 1).to(torch.int32).to(dev)
    L = wl.layers[0]
    f = lambda: q3attn.paged_decode_append_rope(*args, wl.k_cache, wl.v_cache, old, L.block_table, wl.scale, EPS)
    eager = f()
    pool = wl.k_cache.clone()
    s = torch.cuda.Stream(dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        f()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        o = f()
    for rep in range(4):
        o.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(o, eager), f"replay {rep} differs"
        assert torch.equal(wl.k_cache, pool), f"replay {rep} changed the pool"
