"""GPU parity of planned decode calls (q3attn.decode_plan + Q3A_DECODE_PLANNED through the C ABI).

A plan holds the stream-K decomposition of the calls that share cache_seqlens and a block table (the 28 calls of a
talker frame, engine/talker.py:77 with ctx and bt of engine/talker.py:107-112): the tile ranges, each wave's first
tile list and every tile's row, offset, valid tokens and page id.  Each workgroup of a planned call claims one of
the plan's ranges from its XCD's queue, and with enough tiles per range the plan weights the ranges by XCD, so the
partition differs from the unplanned call's equal ranges: the outputs are checked against the oracle (max-abs 2e-2,
mean-abs 2e-3) and against the unplanned call within the spread of fp32 reduction orders (one bf16 step), the slot
rows of the append forms bit for bit, and repeated planned calls against each other bit for bit (the ranges are
fixed by the plan; which workgroup claims which does not change the output).  With few tiles per range the plan
keeps equal ranges and the planned call is bit-identical to the unplanned one."""
import numpy as np
import pytest
import torch

import q3attn
from helpers import decode_oracle, to_np
from oracle import attention as ora
from q3attn import workloads as W

pytestmark = pytest.mark.gpu

SK = q3attn.DECODE_STREAMK


def _eq(a, b, what):
    same = torch.equal(a.view(torch.int16), b.view(torch.int16))
    if not same:
        d = (a.float() - b.float()).abs()
        print(f"[plan] {what}: {int((d > 0).sum())} elements differ, max {float(d.max())}", flush=True)
    assert same, what


def _near(a, b, what, tol=1.6e-2):
    """Two decompositions of the same attention: equal up to the order of the fp32 reductions and the rounding of
    the bf16 output (a bf16 step at |o| ~ 1 is 2^-8)."""
    d = (a.float() - b.float()).abs()
    print(f"[plan] {what}: max |planned - unplanned| {float(d.max()):.3g}, {int((d > 0).sum())} of {d.numel()} differ",
          flush=True)
    assert float(d.max()) <= tol, what


def _parity(out, ref, what):
    ok, st = ora.compare(to_np(out), ref)
    print(f"[parity] {what} {st}", flush=True)
    assert ok, (what, st)


def _tables(wl):
    return torch.stack([L.block_table for L in wl.layers])


def test_planned_576_rows_two_tables(cuda_device):
    """The 576-row peak-load workload with two layers' tables in one stacked plan: each layer's planned call equals
    its unplanned stream-K call bit for bit, and layer 0 matches the oracle on every row."""
    print("[case] decode576 planned, two tables", flush=True)
    wl = W.make_decode("decode576", cuda_device, layers=2, seed=3)
    bts = _tables(wl)
    plans = q3attn.decode_plan(wl.cache_seqlens, bts, wl.page_size)
    assert plans is not None and plans.shape[0] == 2
    for li, L in enumerate(wl.layers):
        ref = q3attn.paged_decode(L.q, wl.k_cache, wl.v_cache, wl.cache_seqlens, bts[li], wl.scale, SK)
        out = q3attn.paged_decode(L.q, wl.k_cache, wl.v_cache, wl.cache_seqlens, bts[li], wl.scale,
                                  plan=plans[li])
        torch.cuda.synchronize()
        _near(out, ref, f"layer {li}")
        if li == 0:
            _parity(out, decode_oracle(wl), "decode576 planned layer 0")
    # The same plan serves repeated calls (the partial records it holds are rewritten by each, the claim counters are
    # left at zero), with the same output bits whatever workgroup claims which range.
    for rep in range(4):
        again = q3attn.paged_decode(wl.layers[1].q, wl.k_cache, wl.v_cache, wl.cache_seqlens, bts[1], wl.scale,
                                    plan=plans[1])
        torch.cuda.synchronize()
        _eq(again, out, f"repeated call {rep}")


@pytest.mark.parametrize("seed,B,max_ctx,page", [(1, 65, 2064, 16), (2, 200, 1800, 16), (3, 700, 600, 32),
                                                 (4, 90, 4096, 64), (5, 1000, 300, 16), (6, 17, 4096, 256)])
def test_planned_random_shapes(cuda_device, seed, B, max_ctx, page):
    """Ragged batches (empty rows, one-token rows, rows ending on and off tile and page boundaries) on several page
    sizes: planned equals unplanned stream-K bit for bit, and the oracle on a sample of rows."""
    print(f"[case] planned seed={seed} B={B} max_ctx={max_ctx} page={page}", flush=True)
    rng = np.random.default_rng(seed)
    ctx = rng.integers(0, max_ctx + 1, B)
    ctx[rng.random(B) < 0.1] = 0
    ctx[: min(B, 4)] = [1, 16, max_ctx, 17][: min(B, 4)]
    P = -(-max_ctx // page)
    wl = W.make_decode("plan", cuda_device, ctx=ctx, num_pages=B * P + 64, max_ctx=max_ctx, page=page, seed=seed)
    L = wl.layers[0]
    plan = q3attn.decode_plan(wl.cache_seqlens, L.block_table, page)
    assert plan is not None
    ref = q3attn.paged_decode(L.q, wl.k_cache, wl.v_cache, wl.cache_seqlens, L.block_table, wl.scale, SK)
    out = q3attn.paged_decode(L.q, wl.k_cache, wl.v_cache, wl.cache_seqlens, L.block_table, wl.scale, plan=plan)
    again = q3attn.paged_decode(L.q, wl.k_cache, wl.v_cache, wl.cache_seqlens, L.block_table, wl.scale, plan=plan)
    torch.cuda.synchronize()
    _near(out, ref, f"seed {seed}")
    _eq(again, out, f"seed {seed} repeated")
    rows = sorted(set(rng.choice(B, min(B, 48), replace=False).tolist()) | {0, 1, 2, 3})
    _parity(out[rows], decode_oracle(wl, rows=rows), f"planned seed {seed}")


def test_planned_equal_ranges_are_bit_identical(cuda_device):
    """With fewer than 32 tiles per range (70 rows of 400 tokens: 1,750 tiles over 256 ranges) the plan keeps the
    unplanned call's equal ranges, and the planned call equals the unplanned one bit for bit."""
    wl = W.make_decode("plan", cuda_device, ctx=np.full(70, 400), num_pages=70 * 26, max_ctx=416, seed=8)
    L = wl.layers[0]
    plan = q3attn.decode_plan(wl.cache_seqlens, L.block_table, wl.page_size)
    ref = q3attn.paged_decode(L.q, wl.k_cache, wl.v_cache, wl.cache_seqlens, L.block_table, wl.scale, SK)
    out = q3attn.paged_decode(L.q, wl.k_cache, wl.v_cache, wl.cache_seqlens, L.block_table, wl.scale, plan=plan)
    torch.cuda.synchronize()
    _eq(out, ref, "equal ranges")


def test_planned_long_waves(cuda_device):
    """Waves that hold more than one 64-tile list (70 rows of 16,384 tokens: ~140 tiles per wave), so later lists come
    from the plan's per-tile entries; planned equals unplanned bit for bit and the oracle on sampled rows."""
    print("[case] planned long waves 70 x 16384", flush=True)
    ctx = np.full(70, 16384)
    ctx[::7] = 16000
    wl = W.make_decode("plan-long", cuda_device, ctx=ctx, num_pages=70 * 64 + 8, max_ctx=16384, page=256, seed=9)
    L = wl.layers[0]
    plan = q3attn.decode_plan(wl.cache_seqlens, L.block_table, 256)
    ref = q3attn.paged_decode(L.q, wl.k_cache, wl.v_cache, wl.cache_seqlens, L.block_table, wl.scale, SK)
    out = q3attn.paged_decode(L.q, wl.k_cache, wl.v_cache, wl.cache_seqlens, L.block_table, wl.scale, plan=plan)
    torch.cuda.synchronize()
    _near(out, ref, "long waves")
    _parity(out[[0, 1, 35, 69]], decode_oracle(wl, rows=[0, 1, 35, 69]), "planned long waves")


def _new_rows(wl, seed):
    g = torch.Generator(device=wl.k_cache.device)
    g.manual_seed(seed)
    k = torch.randn((wl.batch, W.HKV, W.HEAD_DIM), generator=g, device=wl.k_cache.device).to(torch.bfloat16)
    v = torch.randn((wl.batch, W.HKV, W.HEAD_DIM), generator=g, device=wl.k_cache.device).to(torch.bfloat16)
    return k, v


def _slot_index(wl, pos):
    """Flat pool row of each row's new-token slot (position pos[b]), 0 for rows that write nothing."""
    bt = wl.layers[0].block_table.cpu().numpy().astype(np.int64)
    page = wl.page_size
    ok = (pos >= 0) & (pos < bt.shape[1] * page)
    idx = np.where(ok, bt[np.arange(wl.batch), np.clip(pos, 0, None) // page] * page + np.clip(pos, 0, None) % page, 0)
    return torch.from_numpy(idx[ok]).to(wl.k_cache.device)


@pytest.mark.parametrize("form", ["append", "append_rope"])
def test_planned_append_forms_576(cuda_device, form):
    """The append and norm/rope forms at 576 rows: the planned call's output equals the unplanned stream-K call's bit
    for bit, and so do the slot rows it writes (poisoned with NaN between the two calls)."""
    print(f"[case] decode576 planned {form}", flush=True)
    wl = W.make_decode("decode576", cuda_device, seed=4)
    L = wl.layers[0]
    pos = wl.ctx - 1                                # tokens already cached; -1: rows with nothing to append
    seqlens = torch.from_numpy(pos).to(torch.int32).to(wl.k_cache.device)
    k, v = _new_rows(wl, 11)
    dev = wl.k_cache.device
    g = torch.Generator(device=dev)
    g.manual_seed(12)
    qn = (1 + 0.1 * torch.randn(W.HEAD_DIM, generator=g, device=dev)).to(torch.bfloat16)
    kn = (1 + 0.1 * torch.randn(W.HEAD_DIM, generator=g, device=dev)).to(torch.bfloat16)
    cos, sin = W.rope_tables(4096, dev)
    p = torch.from_numpy(np.clip(pos, 0, None)).to(dev)
    c, s = cos[p].to(torch.bfloat16).contiguous(), sin[p].to(torch.bfloat16).contiguous()

    def call(plan=None):
        if form == "append":
            return q3attn.paged_decode_append(L.q, k, v, wl.k_cache, wl.v_cache, seqlens, L.block_table, wl.scale,
                                              SK, plan=plan)
        return q3attn.paged_decode_append_rope(L.q, k, v, qn, kn, c, s, wl.k_cache, wl.v_cache, seqlens,
                                               L.block_table, wl.scale, 1e-6, SK, plan=plan)

    idx = _slot_index(wl, pos)
    kflat = wl.k_cache.view(-1, W.HKV, W.HEAD_DIM)
    vflat = wl.v_cache.view(-1, W.HKV, W.HEAD_DIM)
    ref = call()
    ref_k, ref_v = kflat.index_select(0, idx), vflat.index_select(0, idx)
    kflat.index_fill_(0, idx, float("nan"))
    vflat.index_fill_(0, idx, float("nan"))
    plan = q3attn.decode_plan(seqlens, L.block_table, wl.page_size, form=form)
    out = call(plan)
    torch.cuda.synchronize()
    _near(out, ref, form)
    _eq(kflat.index_select(0, idx), ref_k, f"{form} k slots")
    _eq(vflat.index_select(0, idx), ref_v, f"{form} v slots")
    assert torch.isfinite(out.float()).all()
    again = call(plan)
    torch.cuda.synchronize()
    _eq(again, out, f"{form} repeated")


def test_plan_refuses_other_calls(cuda_device):
    """A plan serves only the calls it was built for: another cache_seqlens tensor, another table or another form
    raise; shapes the library does not decode with stream-K get no plan (None) and the call takes its usual path."""
    wl = W.make_decode("plan", cuda_device, ctx=np.full(80, 300), num_pages=80 * 20, max_ctx=320, seed=2)
    L = wl.layers[0]
    plan = q3attn.decode_plan(wl.cache_seqlens, L.block_table, wl.page_size)
    other = wl.cache_seqlens.clone()
    with pytest.raises(RuntimeError, match="another call"):
        q3attn.paged_decode(L.q, wl.k_cache, wl.v_cache, other, L.block_table, wl.scale, plan=plan)
    with pytest.raises(RuntimeError, match="another call"):
        q3attn.paged_decode(L.q, wl.k_cache, wl.v_cache, wl.cache_seqlens, L.block_table.clone(), wl.scale, plan=plan)
    k, v = _new_rows(wl, 1)
    with pytest.raises(RuntimeError, match="another call"):
        q3attn.paged_decode_append(L.q, k, v, wl.k_cache, wl.v_cache, wl.cache_seqlens, L.block_table, wl.scale,
                                   plan=plan)
    junk = torch.zeros_like(plan)
    with pytest.raises(RuntimeError, match="not a decode plan"):
        q3attn.paged_decode(L.q, wl.k_cache, wl.v_cache, wl.cache_seqlens, L.block_table, wl.scale, plan=junk)
    small = W.make_decode("plan", cuda_device, ctx=np.full(8, 300), num_pages=8 * 20, max_ctx=320, seed=2)
    assert q3attn.decode_plan(small.cache_seqlens, small.layers[0].block_table, small.page_size) is None
    o = q3attn.flash_attn_with_kvcache(small.layers[0].q.unsqueeze(1), small.k_cache, small.v_cache,
                                       cache_seqlens=small.cache_seqlens, block_table=small.layers[0].block_table,
                                       softmax_scale=small.scale, causal=True, scheduler_metadata=None)
    torch.cuda.synchronize()
    _parity(o[:, 0], decode_oracle(small), "no plan for 8 rows")


def test_planned_graph_replays_follow_new_lengths(cuda_device):
    """A graph that builds the plan and then runs planned calls (the frame's order) follows the lengths written into
    its cache_seqlens tensor before each replay; every replay equals the eager unplanned call on those lengths, with
    eager work and synchronisations between the replays."""
    print("[case] planned graph replays", flush=True)
    rng = np.random.default_rng(21)
    wl = W.make_decode("plan", cuda_device, ctx=rng.integers(0, 1800, 300), num_pages=300 * 116, max_ctx=1856,
                       layers=2, seed=21)
    bts = _tables(wl)
    seqlens = wl.cache_seqlens.clone()
    outs = [torch.empty_like(wl.layers[0].q) for _ in range(2)]

    def frame():
        plans = q3attn.decode_plan(seqlens, bts, wl.page_size)
        for li, L in enumerate(wl.layers):
            outs[li].copy_(q3attn.flash_attn_with_kvcache(
                L.q.unsqueeze(1), wl.k_cache, wl.v_cache, cache_seqlens=seqlens, block_table=bts[li],
                softmax_scale=wl.scale, causal=True, scheduler_metadata=plans[li])[:, 0])

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        frame()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        frame()
    for rep in range(4):
        new = rng.integers(0, 1857, 300).astype(np.int32)
        new[rng.random(300) < 0.1] = 0
        seqlens.copy_(torch.from_numpy(new))
        g.replay()
        torch.cuda.synchronize()
        for li, L in enumerate(wl.layers):
            ref = q3attn.paged_decode(L.q, wl.k_cache, wl.v_cache, seqlens, bts[li], wl.scale, SK)
            plans = q3attn.decode_plan(seqlens, bts, wl.page_size)
            eager = q3attn.paged_decode(L.q, wl.k_cache, wl.v_cache, seqlens, bts[li], wl.scale, plan=plans[li])
            torch.cuda.synchronize()
            _eq(outs[li], eager, f"replay {rep} layer {li}")
            _near(outs[li], ref, f"replay {rep} layer {li} against unplanned")
