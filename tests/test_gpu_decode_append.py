"""GPU parity of the fused KV append + decode (q3a_paged_decode_append through the C ABI).

The reference sequence is the engine's: write this step's k/v into the paged pool with index_copy_
(engine/talker.py:72-73), then attend over ctx = pos + 1 tokens (engine/talker.py:77).  The fused call must
give the same output bit for bit (it runs the same tile arithmetic) and leave the pool identical, while never
reading the slot it overwrites (those slots are poisoned with NaN before the call).  The outputs are also
checked against the oracle at the 2e-2 / 2e-3 bar."""
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


def _new_token_slots(wl, layer=0):
    """Flat slot (page * page_size + offset) of each row's last token, -1 for rows with ctx 0."""
    page = wl.page_size
    bt = wl.layers[layer].block_table.cpu().numpy().astype(np.int64)
    pos = wl.ctx - 1
    slots = np.full(wl.batch, -1, np.int64)
    live = pos >= 0
    slots[live] = bt[np.arange(wl.batch)[live], pos[live] // page] * page + pos[live] % page
    return slots


def _split_step(wl, layer=0, v_view=False):
    """Take each live row's last token out of the workload's pool as this step's (k, v), poison its slot
    with NaN, and return (k, v, cache_seqlens before the append, pristine pools)."""
    slots = _new_token_slots(wl, layer)
    live = slots >= 0
    idx = torch.from_numpy(np.where(live, slots, 0)).to(wl.k_cache.device)
    kflat = wl.k_cache.view(-1, W.HKV, W.HEAD_DIM)
    vflat = wl.v_cache.view(-1, W.HKV, W.HEAD_DIM)
    k = kflat.index_select(0, idx)
    v = vflat.index_select(0, idx)
    if v_view:                                   # v as a slice of a fused [B, 4096] qkv projection
        qkv = torch.zeros(wl.batch, 4096, dtype=torch.bfloat16, device=v.device)
        qkv[:, 3072:] = v.reshape(wl.batch, -1)
        v = qkv[:, 3072:].view(wl.batch, W.HKV, W.HEAD_DIM)
    ref_k, ref_v = wl.k_cache.clone(), wl.v_cache.clone()
    live_idx = torch.from_numpy(slots[live]).to(idx.device)
    kflat.index_fill_(0, live_idx, float("nan"))
    vflat.index_fill_(0, live_idx, float("nan"))
    old = torch.from_numpy(wl.ctx - 1).to(torch.int32).to(idx.device)
    return k, v, old, ref_k, ref_v


def _reference(wl, ref_k, ref_v, layer=0, split=0):
    L = wl.layers[layer]
    return q3attn.paged_decode(L.q, ref_k, ref_v, wl.cache_seqlens, L.block_table, wl.scale, split)


# Tables wider than 2,048 tokens take stream-K at any batch; up to 64 rows of narrower tables take the
# row-parallel kernel.
SK_CTX = 2064


@pytest.mark.parametrize("split,max_ctx", [(0, 1800), (0, SK_CTX), (32, 1800), (1024, 1800)])
def test_append_matches_index_copy_then_decode(cuda_device, split, max_ctx):
    wl = W.make_decode("append", cuda_device, ctx=np.array(RAGGED), num_pages=4096, max_ctx=max_ctx, seed=21)
    k, v, old, ref_k, ref_v = _split_step(wl)
    ref = _reference(wl, ref_k, ref_v, split=split)
    L = wl.layers[0]
    out = q3attn.paged_decode_append(L.q, k, v, wl.k_cache, wl.v_cache, old, L.block_table, wl.scale, split)
    torch.cuda.synchronize()
    assert torch.equal(out, ref), f"split={split}"
    assert torch.equal(wl.k_cache, ref_k) and torch.equal(wl.v_cache, ref_v), "pool differs from index_copy_"
    assert not out[0].float().abs().sum().item(), "row with cache_seqlens -1 must be zeros"
    ok, st = ora.compare(to_np(out), decode_oracle(wl))
    print(f"[parity] append split={split} vs oracle {st}", flush=True)
    assert ok, st


@pytest.mark.parametrize("max_ctx", [1800, SK_CTX])
def test_flash_attn_kvcache_k_v_form_strided_v(cuda_device, max_ctx):
    """The flash-attn call form (k=, v= with cache_seqlens = tokens before the append), v a strided view."""
    wl = W.make_decode("append", cuda_device, ctx=np.array(RAGGED[1:]), num_pages=4096, max_ctx=max_ctx, seed=22)
    k, v, old, ref_k, ref_v = _split_step(wl, v_view=True)
    ref = _reference(wl, ref_k, ref_v)
    L = wl.layers[0]
    out = q3attn.flash_attn_with_kvcache(L.q.unsqueeze(1), wl.k_cache, wl.v_cache, k=k.unsqueeze(1),
                                         v=v.unsqueeze(1), cache_seqlens=old, block_table=L.block_table,
                                         softmax_scale=wl.scale, causal=True)
    torch.cuda.synchronize()
    assert out.shape == (wl.batch, 1, 16, 128)
    assert torch.equal(out[:, 0], ref)
    assert torch.equal(wl.k_cache, ref_k) and torch.equal(wl.v_cache, ref_v)


@pytest.mark.parametrize("rows", [2000, 4000])
def test_append_many_short_rows_stream_k(cuda_device, rows):
    """Thousands of rows of 1..40 tokens: many rows end inside each stream-K range; at 4,000 rows a wave holds more
    whole rows than the four whose outputs wait in LDS until after its tile loop."""
    rng = np.random.default_rng(23)
    ctx = rng.integers(1, 41, size=rows)
    wl = W.make_decode("short", cuda_device, ctx=ctx, num_pages=rows * 10 + 480, max_ctx=144, seed=23)
    k, v, old, ref_k, ref_v = _split_step(wl)
    ref = _reference(wl, ref_k, ref_v)
    L = wl.layers[0]
    out = q3attn.paged_decode_append(L.q, k, v, wl.k_cache, wl.v_cache, old, L.block_table, wl.scale, 0)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    assert torch.equal(wl.k_cache, ref_k) and torch.equal(wl.v_cache, ref_v)


@pytest.mark.parametrize("max_ctx", [16, 64, 128])
def test_append_narrow_tables_single_pass(cuda_device, max_ctx):
    """Tables of at most 128 tokens take the single-pass kernel, whose tail wave stores the new rows itself (no
    second kernel): bitwise equal to index_copy_ + decode, pool included, and within the bar of the oracle."""
    rng = np.random.default_rng(40 + max_ctx)
    ctx = rng.integers(1, max_ctx + 1, size=45)
    ctx[:3] = [1, max_ctx, max_ctx - 1]
    wl = W.make_decode("narrow_append", cuda_device, ctx=ctx, num_pages=4096, max_ctx=max_ctx, seed=max_ctx)
    k, v, old, ref_k, ref_v = _split_step(wl)
    ref = _reference(wl, ref_k, ref_v)
    L = wl.layers[0]
    out = q3attn.paged_decode_append(L.q, k, v, wl.k_cache, wl.v_cache, old, L.block_table, wl.scale, 0)
    torch.cuda.synchronize()
    assert torch.equal(out, ref), f"max_ctx={max_ctx}"
    assert torch.equal(wl.k_cache, ref_k) and torch.equal(wl.v_cache, ref_v), "pool differs from index_copy_"
    ok, st = ora.compare(to_np(out), decode_oracle(wl))
    print(f"[parity] append narrow table {max_ctx} vs oracle {st}", flush=True)
    assert ok, st


@pytest.mark.parametrize("max_ctx,ctx", [(272, [272, 17, 1]), (2048, [1, 17, 1000, 2048, 640])])
def test_append_row_parallel_small_batches(cuda_device, max_ctx, ctx):
    """Small batches of long tables: the row-parallel kernel with 8 waves of several tiles each, the same
    decomposition as the plain form; the wave owning each row's last tile stores the new rows.  Bitwise equal to
    index_copy_ + decode, pool included, and within the bar of the oracle."""
    wl = W.make_decode("row_append", cuda_device, ctx=np.array(ctx), num_pages=4096, max_ctx=max_ctx, seed=max_ctx)
    k, v, old, ref_k, ref_v = _split_step(wl)
    ref = _reference(wl, ref_k, ref_v)
    L = wl.layers[0]
    out = q3attn.paged_decode_append(L.q, k, v, wl.k_cache, wl.v_cache, old, L.block_table, wl.scale, 0)
    torch.cuda.synchronize()
    assert torch.equal(out, ref), f"max_ctx={max_ctx}"
    assert torch.equal(wl.k_cache, ref_k) and torch.equal(wl.v_cache, ref_v), "pool differs from index_copy_"
    ok, st = ora.compare(to_np(out), decode_oracle(wl))
    print(f"[parity] append row path {max_ctx} vs oracle {st}", flush=True)
    assert ok, st


def test_append_decode576_full_size(cuda_device):
    """576 rows (58 padded, 131,072-page pool): bitwise equal to index_copy_ + decode; every row against the oracle."""
    wl = W.make_decode("decode576", cuda_device, layers=1, seed=24)
    k, v, old, ref_k, ref_v = _split_step(wl)
    ref = _reference(wl, ref_k, ref_v)
    del ref_k, ref_v
    L = wl.layers[0]
    out = q3attn.paged_decode_append(L.q, k, v, wl.k_cache, wl.v_cache, old, L.block_table, wl.scale, 0)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    ok, st = ora.compare(to_np(out), decode_oracle(wl))
    print(f"[parity] append decode576 all {wl.batch} rows vs oracle {st}", flush=True)
    assert ok, st


def test_append_rows_past_capacity_are_skipped(cuda_device):
    """cache_seqlens == max_pages * page_size (no room for the new token) and -1 both give zeros, write nothing."""
    wl = W.make_decode("cap", cuda_device, ctx=np.array([32, 32, 32]), num_pages=64, max_ctx=32, seed=25)
    L = wl.layers[0]
    k = torch.randn(3, 8, 128, device=cuda_device).to(torch.bfloat16)
    v = torch.randn(3, 8, 128, device=cuda_device).to(torch.bfloat16)
    before_k, before_v = wl.k_cache.clone(), wl.v_cache.clone()
    old = torch.tensor([32, -1, 31], dtype=torch.int32, device=cuda_device)
    out = q3attn.paged_decode_append(L.q, k, v, wl.k_cache, wl.v_cache, old, L.block_table, wl.scale, 0)
    torch.cuda.synchronize()
    assert not out[:2].float().abs().sum().item()
    slot = int(L.block_table[2, 1]) * 16 + 15
    kflat, bk = wl.k_cache.view(-1, 8, 128), before_k.view(-1, 8, 128)
    assert torch.equal(kflat[slot], k[2])
    keep = torch.ones(kflat.shape[0], dtype=torch.bool, device=cuda_device)
    keep[slot] = False
    assert torch.equal(kflat[keep], bk[keep])
    assert torch.equal(wl.v_cache.view(-1, 8, 128)[keep], before_v.view(-1, 8, 128)[keep])
    assert out[2].float().abs().sum().item() > 0


@pytest.mark.parametrize("max_ctx", [1800, SK_CTX])
def test_append_in_graph_replays(cuda_device, max_ctx):
    """Captured into a HIP graph (as the talker frame is) and replayed: every replay equals the eager call."""
    wl = W.make_decode("append", cuda_device, ctx=np.array(RAGGED), num_pages=4096, max_ctx=max_ctx, seed=26)
    k, v, old, ref_k, ref_v = _split_step(wl)
    L = wl.layers[0]
    eager = q3attn.paged_decode_append(L.q, k, v, wl.k_cache, wl.v_cache, old, L.block_table, wl.scale, 0)
    torch.cuda.synchronize()
    s = torch.cuda.Stream(cuda_device)
    s.wait_stream(torch.cuda.current_stream(cuda_device))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        static = q3attn.paged_decode_append(L.q, k, v, wl.k_cache, wl.v_cache, old, L.block_table, wl.scale, 0)
    for _ in range(3):
        wl.k_cache.view(-1, 8, 128)[torch.from_numpy(_new_token_slots(wl)[1:]).to(cuda_device)] = float("nan")
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(static, eager)
        assert torch.equal(wl.k_cache, ref_k)
