"""GPU parity of the chunked (split-KV) decode: q3a_paged_decode with split_tokens = Q3A_DECODE_CHUNKS, the kernel the
library picks for small batches of long rows (the talker's frame graphs at buckets 1, 2, 4, 8, 16, engine/engine.py:65,
each calling flash_attn_with_kvcache at engine/talker.py:77).

Each workgroup reduces one chunk of a (row, KV head) -- 128 tokens as 8 waves of one 16-token tile for tables up to
2,048 tokens, 256 tokens as 16 waves up to 4,096, then 8 waves of several tiles -- to an fp32 record (o = sum p.v,
m, l); a second kernel merges a row's records.  Checked here:
* against the oracle (bf16 output within max-abs 2e-2 and mean-abs 2e-3 of the fp32-softmax restatement of
  engine/talker.py:82-88) for contexts on both sides of every chunk boundary and each chunk geometry;
* against the row-parallel and stream-K kernels on the same inputs (another fp32 reduction order: within 8e-3 /
  2e-4);
* exact cases: ctx = 1 gives the V row bit for bit, ctx = 0 gives zeros, NaN in stale slots and garbage table
  entries past a row's pages are never read, a page-table permutation changes no bit;
* the append form bit-identical to index_copy_ x2 + the plain chunked decode (the same decomposition), with the
  target slots NaN-poisoned; the norm/rope form on +-1 rows bit-identical to the append form on the oracle's q, k;
* HIP-graph replays equal to eager calls.
"""
import numpy as np
import pytest
import torch

import q3attn
from helpers import decode_oracle, to_np
from oracle import attention as ora
from q3attn import workloads as W

pytestmark = pytest.mark.gpu

CHUNKS, ROW, SK = q3attn.DECODE_CHUNKS, q3attn.DECODE_ROW, q3attn.DECODE_STREAMK


def decode(wl, split=CHUNKS, layer=0, q=None, k=None, v=None, bt=None):
    L = wl.layers[layer]
    out = q3attn.paged_decode(L.q if q is None else q, wl.k_cache if k is None else k,
                              wl.v_cache if v is None else v, wl.cache_seqlens,
                              L.block_table if bt is None else bt, wl.scale, split)
    torch.cuda.synchronize()
    return out


def parity(out, ref, what):
    ok, st = ora.compare(to_np(out), ref)
    print(f"[parity] chunks {what} {st}", flush=True)
    assert ok, (what, st)


# Contexts on both sides of the 128- and 256-token chunk boundaries, a full table, and the empty and one-token rows.
EDGES_2048 = [0, 1, 16, 127, 128, 129, 255, 256, 257, 1000, 1024, 1800, 2047, 2048]


@pytest.mark.parametrize("max_ctx,ctx", [
    (2048, EDGES_2048),                                  # 8 waves x 1 tile: 16 chunks of 128 tokens
    (2048, [1800]),                                      # one row (bucket 1)
    (304, [304, 300, 129, 128, 5]),                      # 3 chunks, the last one partial
    (4096, [4096, 2049, 256, 257, 3000, 1]),             # 16 waves x 1 tile: 16 chunks of 256 tokens
    (8192, [8192, 4097, 513, 511, 7000, 0, 1]),          # 8 waves x 4 tiles: 16 chunks of 512 tokens
])
def test_chunks_vs_oracle(cuda_device, max_ctx, ctx):
    ctx = np.array(ctx)
    wl = W.make_decode("chunks", cuda_device, ctx=ctx, num_pages=max(1024, 2 * len(ctx) * (max_ctx // 16 + 1)),
                       max_ctx=max_ctx, seed=max_ctx + len(ctx))
    out = decode(wl)
    parity(out, decode_oracle(wl), f"{max_ctx} {ctx.tolist()}")
    assert not out[ctx == 0].float().abs().sum().item(), "ctx == 0 rows must be zeros"
    assert torch.equal(out, decode(wl)), "not deterministic"


@pytest.mark.parametrize("B,ctx_hi", [(1, 1800), (4, 1024), (8, 1800), (16, 2048)])
def test_chunks_random_batches_vs_oracle_and_other_kernels(cuda_device, B, ctx_hi):
    rng = np.random.default_rng(B * 1000 + ctx_hi)
    ctx = rng.integers(1, ctx_hi + 1, size=B)
    ctx[0] = ctx_hi
    wl = W.make_decode("chunks_rand", cuda_device, ctx=ctx, num_pages=4 * B * 130 + 64, max_ctx=2048, seed=B)
    out = decode(wl)
    parity(out, decode_oracle(wl), f"B={B} ctx<={ctx_hi}")
    for other in (ROW, SK, 0):
        ok, st = ora.compare(to_np(decode(wl, split=other)), to_np(out), max_abs=8e-3, mean_abs=2e-4)
        assert ok, (other, st)


@pytest.mark.parametrize("max_ctx", [2048, 4096])
def test_chunks_ctx1_is_exact_v_row(cuda_device, max_ctx):
    wl = W.make_decode("one", cuda_device, ctx=np.array([1, 1, 1, 1]), num_pages=1024, max_ctx=max_ctx, seed=3)
    out = decode(wl)
    bt = wl.layers[0].block_table[:, 0].long()
    assert torch.equal(out, wl.v_cache[bt, 0].repeat_interleave(2, dim=1))


def test_chunks_stale_slots_garbage_entries_and_permutation(cuda_device):
    ctx = np.array(EDGES_2048)
    wl = W.make_decode("dirty", cuda_device, ctx=ctx, num_pages=4096, max_ctx=2048, seed=41)
    clean = decode(wl)
    bt = wl.layers[0].block_table.clone()
    k, v = wl.k_cache.clone(), wl.v_cache.clone()
    page = wl.page_size
    for b, c in enumerate(ctx):
        used = (c + page - 1) // page
        if c % page:
            pg = int(bt[b, used - 1])
            k[pg, c % page:] = float("nan")
            v[pg, c % page:] = float("nan")
        bt[b, used:] = -7 if b % 2 else 1 << 30
    assert torch.equal(clean, decode(wl, k=k, v=v, bt=bt)), "stale slots or table entries were read"
    perm = torch.randperm(4096, generator=torch.Generator().manual_seed(2)).to(cuda_device)
    inv = torch.argsort(perm)
    permuted = decode(wl, k=wl.k_cache[perm], v=wl.v_cache[perm], bt=inv[wl.layers[0].block_table.long()].int())
    assert torch.equal(clean, permuted)


def test_chunks_out_of_range_page_ids(cuda_device):
    """A page id outside the pool contributes no tokens (its chunk's record carries l = 0)."""
    wl = W.make_decode("oob", cuda_device, ctx=np.array([600, 600]), num_pages=512, max_ctx=2048, seed=4)
    bt = wl.layers[0].block_table.clone()
    bt[0, 9] = -1            # a whole 16-token page inside chunk 1 of row 0
    bt[1, 0:8] = 1 << 30     # every page of row 1's chunk 0
    out = decode(wl, bt=bt)
    assert torch.isfinite(out.float()).all()
    # The same attention with those tokens gone: the oracle over the remaining pages.
    keep_k, keep_v = wl.k_cache.clone(), wl.v_cache.clone()
    ref_bt = bt.clone()
    ref_bt[ref_bt >= 512] = -1
    oracle_rows = []
    for b in range(2):
        pages = [int(p) for p in ref_bt[b, :600 // 16 + 1].tolist()]
        toks = [(p, o) for i, p in enumerate(pages) for o in range(16) if p >= 0 and i * 16 + o < 600]
        kk = torch.stack([keep_k[p, o] for p, o in toks]).float().cpu().numpy()   # [n, 8, 128]
        vv = torch.stack([keep_v[p, o] for p, o in toks]).float().cpu().numpy()
        q = to_np(wl.layers[0].q[b])                                              # [16, 128]
        o = np.zeros((16, 128), np.float32)
        for h in range(16):
            s = kk[:, h // 2] @ q[h] * wl.scale
            p_ = np.exp(s - s.max())
            o[h] = (p_ / p_.sum()) @ vv[:, h // 2]
        oracle_rows.append(o)
    ok, st = ora.compare(to_np(out), np.stack(oracle_rows))
    assert ok, st


def _split_step(wl):
    """Each live row's last token as this step's (k, v); its slot poisoned with NaN; the pristine pools kept."""
    page = wl.page_size
    bt = wl.layers[0].block_table.cpu().numpy().astype(np.int64)
    pos = wl.ctx - 1
    live = pos >= 0
    slots = np.full(wl.batch, -1, np.int64)
    slots[live] = bt[np.arange(wl.batch)[live], pos[live] // page] * page + pos[live] % page
    idx = torch.from_numpy(np.where(live, slots, 0)).to(wl.k_cache.device)
    kflat = wl.k_cache.view(-1, W.HKV, W.HEAD_DIM)
    vflat = wl.v_cache.view(-1, W.HKV, W.HEAD_DIM)
    k, v = kflat.index_select(0, idx), vflat.index_select(0, idx)
    ref_k, ref_v = wl.k_cache.clone(), wl.v_cache.clone()
    live_idx = torch.from_numpy(slots[live]).to(idx.device)
    kflat.index_fill_(0, live_idx, float("nan"))
    vflat.index_fill_(0, live_idx, float("nan"))
    old = torch.from_numpy(wl.ctx - 1).to(torch.int32).to(idx.device)
    return k, v, old, ref_k, ref_v


@pytest.mark.parametrize("max_ctx,ctx", [(2048, EDGES_2048), (4096, [4096, 257, 1, 2049]),
                                         (8192, [8192, 513, 1, 0])])
def test_chunks_append_bit_identical_to_index_copy(cuda_device, max_ctx, ctx):
    wl = W.make_decode("chunks_append", cuda_device, ctx=np.array(ctx), num_pages=4 * len(ctx) * (max_ctx // 16),
                       max_ctx=max_ctx, seed=max_ctx + 7)
    k, v, old, ref_k, ref_v = _split_step(wl)
    L = wl.layers[0]
    ref = q3attn.paged_decode(L.q, ref_k, ref_v, wl.cache_seqlens, L.block_table, wl.scale, CHUNKS)
    out = q3attn.paged_decode_append(L.q, k, v, wl.k_cache, wl.v_cache, old, L.block_table, wl.scale, CHUNKS)
    torch.cuda.synchronize()
    assert torch.equal(out, ref), "append output differs from index_copy_ + decode"
    assert torch.equal(wl.k_cache, ref_k) and torch.equal(wl.v_cache, ref_v), "pool differs from index_copy_"
    parity(out, decode_oracle(wl), f"append {max_ctx}")


def test_chunks_rope_form_exact_rows(cuda_device):
    """+-1 head rows with eps = 0: mean(x^2) = 1 and 1/sqrt of it 1, the normalised rows are exactly +-w and the rope
    products exact, so the norm/rope form equals the append form on the oracle's q', k' bit for bit (output and
    pool)."""
    EPS = 0.0
    ctx = np.array([1, 129, 1800, 256, 2048, 0])
    wl = W.make_decode("chunks_rope", cuda_device, ctx=ctx, num_pages=2048, max_ctx=2048, seed=77)
    dev = cuda_device
    rng = np.random.default_rng(5)
    B = wl.batch
    r = lambda x: ora.bf16_round(np.asarray(x, np.float32))
    q = r(rng.choice([-1.0, 1.0], size=(B, W.HQ, W.HEAD_DIM)))
    k = r(rng.choice([-1.0, 1.0], size=(B, W.HKV, W.HEAD_DIM)))
    v = r(rng.standard_normal((B, W.HKV, W.HEAD_DIM)))
    qn, kn = r(rng.uniform(0.5, 1.5, W.HEAD_DIM)), r(rng.uniform(0.5, 1.5, W.HEAD_DIM))
    cos_t, sin_t = ora.rope_tables(2048)
    pos = np.maximum(ctx - 1, 0)
    cos, sin = r(cos_t[pos]), r(sin_t[pos])
    qq = ora.norm_rope(q, qn, cos[:, None], sin[:, None], EPS, eager=False)
    kk = ora.norm_rope(k, kn, cos[:, None], sin[:, None], EPS, eager=False)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(dev).to(torch.bfloat16)
    old = torch.from_numpy(ctx - 1).to(torch.int32).to(dev)
    L = wl.layers[0]
    pk, pv = wl.k_cache.clone(), wl.v_cache.clone()
    out = q3attn.paged_decode_append_rope(t(q), t(k), t(v), t(qn), t(kn), t(cos), t(sin), wl.k_cache, wl.v_cache,
                                          old, L.block_table, wl.scale, EPS, CHUNKS)
    got_k, got_v = wl.k_cache.clone(), wl.v_cache.clone()
    wl.k_cache.copy_(pk)
    wl.v_cache.copy_(pv)
    ref = q3attn.paged_decode_append(t(qq), t(kk), t(v), wl.k_cache, wl.v_cache, old, L.block_table, wl.scale, CHUNKS)
    torch.cuda.synchronize()
    assert torch.equal(out, ref), "norm/rope chunked output differs from append on the oracle's q', k'"
    assert torch.equal(got_k, wl.k_cache) and torch.equal(got_v, wl.v_cache), "pool differs"
    assert not out[ctx == 0].float().abs().sum().item()


def test_chunks_graph_replays_match_eager(cuda_device):
    ctx = np.array([1800, 5, 1024, 0, 2048, 300, 129, 77])
    wl = W.make_decode("chunks_graph", cuda_device, ctx=ctx, num_pages=4096, max_ctx=2048, layers=3, seed=12)
    f = lambda: [q3attn.paged_decode(L.q, wl.k_cache, wl.v_cache, wl.cache_seqlens, L.block_table, wl.scale, 0)
                 for L in wl.layers]
    eager = [o.clone() for o in f()]
    s = torch.cuda.Stream(cuda_device)
    s.wait_stream(torch.cuda.current_stream(cuda_device))
    with torch.cuda.stream(s):
        f()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        outs = f()
    for rep in range(4):
        for o in outs:
            o.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(a, b) for a, b in zip(outs, eager)), f"replay {rep} differs"
    parity(eager[0], decode_oracle(wl, 0), "graph layer 0")
