"""The entry points inside a captured HIP graph (the reference replays its frame as one CUDA graph,
engine/talker.py:115-137): replays with eager work and synchronisations between them must equal
the eager result every time."""
import numpy as np
import pytest
import torch

import q3attn
from q3attn import workloads as W

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("max_ctx", [1800, 2064])     # the row-parallel and the stream-K decode
def test_graph_replay_matches_eager(cuda_device, max_ctx):
    wl = W.make_decode("g", cuda_device, ctx=np.array([0, 1, 33, 200, 700, 64, 1500, 3]), num_pages=2048,
                       max_ctx=max_ctx, layers=3, seed=12)
    qs, K, V = W.make_cp(32, cuda_device, seed=12)

    def frame():
        outs = []
        for L in wl.layers:
            outs.append(q3attn.flash_attn_with_kvcache(L.q.unsqueeze(1), wl.k_cache, wl.v_cache,
                                                       cache_seqlens=wl.cache_seqlens, block_table=L.block_table,
                                                       softmax_scale=wl.scale, causal=True))
        for p in range(16):
            outs.append(q3attn.cp_attn(qs[p], K, V, p + 1, 0.088))
        return outs

    eager = [o.clone() for o in frame()]
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        frame()                                  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        static = frame()
    for rep in range(4):
        junk = torch.randn(1 << 20, device=cuda_device) * 3          # eager work between replays
        g.replay()
        torch.cuda.synchronize()
        for a, b in zip(static, eager):
            assert torch.equal(a, b), rep
        del junk


def test_two_streams_concurrently(cuda_device):
    """The engine replays its frame graph and the fast-admission graphs on two streams at once
    (engine/engine.py:104, engine/arrivals.py:183-200): the ops keep no state between calls, so two graphs replayed
    concurrently on two default-priority streams, and eager calls interleaved on both, give the eager results
    bit for bit."""
    ctx_a = np.random.default_rng(3).integers(1, 900, 96)
    ctx_b = np.random.default_rng(4).integers(1, 600, 40)
    wa = W.make_decode("a", cuda_device, ctx=ctx_a, num_pages=8192, max_ctx=1024, layers=4, seed=21)
    wb = W.make_decode("b", cuda_device, ctx=ctx_b, num_pages=4096, max_ctx=1024, layers=2, seed=22)
    qs, K, V = W.make_cp(64, cuda_device, seed=23)
    adm = W.make_admit(cuda_device, 4, 42, 77, seed=24)
    kb = torch.randn(40, 8, 128, device=cuda_device).to(torch.bfloat16)
    vb = torch.randn(40, 8, 128, device=cuda_device).to(torch.bfloat16)
    old_b = (wb.cache_seqlens - 1).clamp(min=0)

    def frame_a():
        return [q3attn.paged_decode(L.q, wa.k_cache, wa.v_cache, wa.cache_seqlens, L.block_table, wa.scale, 0)
                for L in wa.layers]

    def frame_b():
        outs = [q3attn.paged_decode(L.q, wb.k_cache, wb.v_cache, wb.cache_seqlens, L.block_table, wb.scale, 0)
                for L in wb.layers]
        # the append rewrites each row's last cached token with the same rows every time: idempotent
        outs.append(q3attn.paged_decode_append(wb.layers[0].q, kb, vb, wb.k_cache, wb.v_cache, old_b,
                                               wb.layers[0].block_table, wb.scale, 0))
        outs += [q3attn.cp_attn(qs[p], K, V, p + 1, 0.088) for p in (0, 7, 15)]
        outs.append(q3attn.flash_attn_func(adm.q, adm.k, adm.v, softmax_scale=adm.scale, causal=True))
        return outs

    frame_b()                                   # the append's first call writes the rows; later calls rewrite them
    torch.cuda.synchronize()
    ref_a = [o.clone() for o in frame_a()]
    ref_b = [o.clone() for o in frame_b()]
    torch.cuda.synchronize()

    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    # eager calls interleaved on the two streams
    for _ in range(3):
        with torch.cuda.stream(sa):
            out_a = frame_a()
        with torch.cuda.stream(sb):
            out_b = frame_b()
        torch.cuda.synchronize()
        assert all(torch.equal(x, y) for x, y in zip(out_a, ref_a))
        assert all(torch.equal(x, y) for x, y in zip(out_b, ref_b))

    graphs = []
    for s, fn in ((sa, frame_a), (sb, frame_b)):
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            fn()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            static = fn()
        graphs.append((g, static))
    torch.cuda.synchronize()
    for rep in range(10):
        with torch.cuda.stream(sa):
            graphs[0][0].replay()
        with torch.cuda.stream(sb):
            graphs[1][0].replay()
        torch.cuda.synchronize()
        assert all(torch.equal(x, y) for x, y in zip(graphs[0][1], ref_a)), rep
        assert all(torch.equal(x, y) for x, y in zip(graphs[1][1], ref_b)), rep
