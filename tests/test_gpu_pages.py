"""GPU: a talker-style decode loop over the shared page pool.

Seats join at staggered frames, some leave and their pages are handed to seats that join later (recycled pages
still hold the previous owner's K/V).  Every frame appends each active seat's new token and attends, once with
the fused append form (paged_decode_append, cache_seqlens = tokens already cached) and once the reference's way
(index_copy_ into PagePool.slot, then paged_decode over ctx = pos + 1); both must match each other bit for bit and
the oracle over each seat's own token history (engine/talker.py:72-77, 107-112)."""
import numpy as np
import pytest
import torch

import q3attn
from helpers import to_np
from oracle import attention as ora
from q3attn.pages import PagePool

pytestmark = pytest.mark.gpu


def test_decode_loop_over_shared_pool(cuda_device):
    rng = np.random.default_rng(3)
    max_seats, max_pages, page = 6, 8, 16
    pool = PagePool(num_pages=40, max_seats=max_seats, max_pages_per_seat=max_pages, device=cuda_device)
    shape = (pool.num_pages, page, 8, 128)
    kc_a, vc_a = torch.randn(shape, device=cuda_device).to(torch.bfloat16), torch.randn(shape, device=cuda_device).to(torch.bfloat16)
    kc_b, vc_b = kc_a.clone(), vc_a.clone()
    # (seat, first frame, frames): seats 0-3 start early; 1 and 2 leave and 4, 5 reuse their pages
    sched = [(0, 0, 70), (1, 2, 30), (2, 5, 25), (3, 9, 60), (4, 40, 35), (5, 45, 20)]
    hist = {s: [] for s in range(max_seats)}
    scale = 128 ** -0.5
    worst = {"max_abs": 0.0, "mean_abs": 0.0}
    for f in range(75):
        for s, f0, n in sched:
            if f == f0 + n:
                pool.release(s)
                hist[s] = []
        act = [s for s, f0, n in sched if f0 <= f < f0 + n]
        if not act:
            continue
        B = len(act)
        seat = torch.tensor(act, dtype=torch.long, device=cuda_device)
        pos_h = np.array([len(hist[s]) for s in act])
        pool.grow(act, pos_h + 1)
        pos = torch.from_numpy(pos_h).to(cuda_device)
        q = torch.randn(B, 16, 128, device=cuda_device).to(torch.bfloat16)
        k = torch.randn(B, 8, 128, device=cuda_device).to(torch.bfloat16)
        v = torch.randn(B, 8, 128, device=cuda_device).to(torch.bfloat16)
        bt = pool.block_table(seat)
        out_a = q3attn.paged_decode_append(q, k, v, kc_a, vc_a, pos.to(torch.int32), bt, scale, 0)
        slot = pool.slot(seat, pos)
        kc_b.view(-1, 8, 128).index_copy_(0, slot, k)
        vc_b.view(-1, 8, 128).index_copy_(0, slot, v)
        out_b = q3attn.paged_decode(q, kc_b, vc_b, (pos + 1).to(torch.int32), bt, scale, 0)
        torch.cuda.synchronize()
        assert torch.equal(out_a, out_b), f"frame {f}"
        kh, vh = to_np(k), to_np(v)
        for i, s in enumerate(act):
            hist[s].append((kh[i], vh[i]))
        # oracle over each seat's own history (a compact identity-table pool per row)
        ctx = np.array([len(hist[s]) for s in act])
        P = int(-(-ctx.max() // page))
        kk = np.zeros((B * P, page, 8, 128), np.float32)
        vv = np.zeros_like(kk)
        for i, s in enumerate(act):
            for t, (a, b) in enumerate(hist[s]):
                kk[i * P + t // page, t % page], vv[i * P + t // page, t % page] = a, b
        table = np.arange(B * P).reshape(B, P)
        ref = ora.paged_decode(to_np(q), kk, vv, ctx, table, scale)
        ok, st = ora.compare(to_np(out_a), ref)
        assert ok, (f, st)
        worst = {k_: max(worst[k_], st[k_]) for k_ in worst}
    pool.check()
    assert torch.equal(kc_a, kc_b) and torch.equal(vc_a, vc_b)
    print(f"[parity] shared-pool decode loop, 75 frames, worst {worst}", flush=True)
