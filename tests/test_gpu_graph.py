"""The entry points inside a captured HIP graph (the reference replays its frame as one CUDA graph,
engine/talker.py:115-137): replays with eager work and synchronisations between them must equal
the eager result every time."""
import numpy as np
import pytest
import torch

import q3attn
from q3attn import workloads as W

pytestmark = pytest.mark.gpu


def test_graph_replay_matches_eager(cuda_device):
    wl = W.make_decode("g", cuda_device, ctx=np.array([0, 1, 33, 200, 700, 64, 1500, 3]), num_pages=1024,
                       max_ctx=1800, layers=3, seed=12)
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
