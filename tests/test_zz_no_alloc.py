"""q3a_paged_decode_noalloc (the allocation-free decode entry point) through the C ABI against q3a_paged_decode.

Two calls in a row on one stream, the second with a smaller input, must each equal the workspace entry point's
output bit for bit (the static scratch keeps the first call's contents; nothing in it needs to start at zero).  A shape
whose workspace exceeds the static scratch is rejected before any launch, leaving the output untouched."""
import numpy as np
import pytest
import torch

import q3attn
from q3attn import _lib
from q3attn import workloads as W

pytestmark = pytest.mark.gpu


def _noalloc(q, kc, vc, seqlens, bt, out, scale, split=0):
    B, Hq, D = q.shape
    rc = _lib.lib().q3a_paged_decode_noalloc(
        q.data_ptr(), q.stride(0), q.stride(1), kc.data_ptr(), vc.data_ptr(), kc.stride(0), kc.stride(1), kc.stride(2),
        kc.shape[0], kc.shape[1], seqlens.data_ptr(), bt.data_ptr(), bt.stride(0), bt.shape[1], out.data_ptr(),
        out.stride(0), out.stride(1), B, Hq, kc.shape[2], D, scale, split,
        torch.cuda.current_stream(q.device).cuda_stream)
    return rc


def _case(wl, layer=0):
    L = wl.layers[layer]
    want = q3attn.paged_decode(L.q, wl.k_cache, wl.v_cache, wl.cache_seqlens, L.block_table, wl.scale, 0)
    out = torch.full_like(want, float("nan"))
    rc = _noalloc(L.q, wl.k_cache, wl.v_cache, wl.cache_seqlens, L.block_table, out, wl.scale)
    torch.cuda.synchronize()
    assert rc == 0, _lib.lib().q3a_last_error().decode()
    return out, want


def test_noalloc_matches_workspace_entry_point_twice(cuda_device):
    big = W.make_decode("decode576", cuda_device, layers=1, seed=31)
    print(f"[noalloc] call 1: {big.batch} rows, {int(big.ctx.sum())} tokens", flush=True)
    out1, want1 = _case(big)
    assert torch.equal(out1, want1)
    del big
    torch.cuda.empty_cache()
    rng = np.random.default_rng(32)
    ctx = rng.integers(0, 700, size=80)    # more than 64 rows: the stream-K path, which uses the scratch
    small = W.make_decode("small", cuda_device, ctx=ctx, num_pages=4096, max_ctx=700, seed=32)
    print(f"[noalloc] call 2: {small.batch} rows, {int(small.ctx.sum())} tokens", flush=True)
    out2, want2 = _case(small)
    assert torch.equal(out2, want2)
    assert not out2[ctx == 0].float().abs().sum().item()


def test_noalloc_chunked_path_twice(cuda_device):
    """Small batches of long tables take the chunked kernel, whose fp32 chunk records live in the scratch: two calls
    in a row (8 rows, then 2 rows with shorter contexts, so the second call's combine meets the first call's stale
    records past its rows' ends) each equal the workspace entry point bit for bit."""
    for B, hi, seed in ((8, 2048, 41), (2, 700, 42)):
        rng = np.random.default_rng(seed)
        ctx = rng.integers(1, hi + 1, size=B)
        ctx[0] = hi
        wl = W.make_decode("small", cuda_device, ctx=ctx, num_pages=4 * B * 128 + 64, max_ctx=2048, seed=seed)
        print(f"[noalloc] chunked path: {B} rows, {int(ctx.sum())} tokens", flush=True)
        out, want = _case(wl)
        assert torch.equal(out, want)
        del wl
        torch.cuda.empty_cache()


def test_noalloc_rejects_shapes_beyond_the_scratch(cuda_device):
    B, P = 5000, 128                       # fixed splits: 5000 rows x 32 splits x 8 heads x 528 B >> 8 MiB
    q = torch.zeros(B, 16, 128, dtype=torch.bfloat16, device=cuda_device)
    kc = torch.zeros(64, 16, 8, 128, dtype=torch.bfloat16, device=cuda_device)
    seqlens = torch.ones(B, dtype=torch.int32, device=cuda_device)
    bt = torch.zeros(B, P, dtype=torch.int32, device=cuda_device)
    out = torch.full_like(q, 7.0)
    rc = _noalloc(q, kc, kc, seqlens, bt, out, 0.1)
    torch.cuda.synchronize()
    assert rc == -28 and "static scratch" in _lib.lib().q3a_last_error().decode()
    assert (out == 7.0).all()
