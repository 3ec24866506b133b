"""GPU parity of the code predictor's step attention block in one launch (q3a_cp_attn_append_rope).

engine/code_predictor.py:38-43 (`_pre`, compiled by default) normalises and rotates q and k with slot p's cos/sin
row, :58 writes k and v into slot p of the layer's K/V scratch, :46-47 attends over slots 0..p.  Against that:
  * the same step through q3a_cp_attn_append on q and k normalised by the oracle's producers with the compiled
    rounding (one rounding after the rope; every product is exact in fp32) agrees within the max-abs bar and a tenth
    of the mean-abs bar
    (the normalised rows can differ in a rare last bit: the mean of squares is summed in another order);
  * slot p holds the normalised k (up to a rare last-bit difference from the summation order of the mean of squares)
    and v exactly; no other slot changes;
  * the output is within the bar of the oracle attention over the oracle's producers (engine/cp_attn.py:19-30).
"""
import numpy as np
import pytest
import torch

import q3attn
from helpers import to_np
from oracle import attention as ora
from q3attn import workloads as W

pytestmark = pytest.mark.gpu

D = 128


def _compiled_norm_rope_np(x, w, cos, sin, eps=1e-6):
    """engine/ops.py:51-60 as the compiled step evaluates it (the oracle's compiled form: float32 throughout, one
    rounding at the end)."""
    return ora.norm_rope(x, w, cos, sin, eps, eager=False)


def _step_inputs(dev, B, seed):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    qkv = torch.randn((B, 4096), generator=g, device=dev).to(torch.bfloat16)
    qn = (1.0 + 0.1 * torch.randn(D, generator=g, device=dev)).to(torch.bfloat16)
    kn = (1.0 + 0.1 * torch.randn(D, generator=g, device=dev)).to(torch.bfloat16)
    K = torch.randn((B, 8, 16, D), generator=g, device=dev).to(torch.bfloat16)
    V = torch.randn((B, 8, 16, D), generator=g, device=dev).to(torch.bfloat16)
    cos, sin = W.rope_tables(16, dev)
    return qkv, qn, kn, K, V, cos.to(torch.bfloat16), sin.to(torch.bfloat16)


@pytest.mark.parametrize("B", [1, 64, 512])
def test_cp_rope_step_matches_normalised_append(cuda_device, B):
    dev = cuda_device
    qkv, qn, kn, K0, V0, cos, sin = _step_inputs(dev, B, seed=60 + B)
    q, k, v = qkv[:, :2048].view(B, 16, D), qkv[:, 2048:3072].view(B, 8, D), qkv[:, 3072:].view(B, 8, D)
    scale = D ** -0.5
    flips = 0
    for p in range(16):
        # slots past p hold NaN: the kernel must not read them
        K, V = K0.clone(), V0.clone()
        K[:, :, p + 1:] = float("nan")
        V[:, :, p + 1:] = float("nan")
        Kr, Vr = K.clone(), V.clone()
        print(f"[case] cp_attn_append_rope B={B} p={p}", flush=True)
        out = q3attn.cp_attn_append_rope(q, k, v, K, V, p, scale, qn, kn, cos[p], sin[p])
        c, s = to_np(cos[p]), to_np(sin[p])
        qo = _compiled_norm_rope_np(to_np(q), to_np(qn), c, s)
        ko = _compiled_norm_rope_np(to_np(k), to_np(kn), c, s)
        ref = q3attn.cp_attn_append(torch.from_numpy(qo).to(dev, torch.bfloat16),
                                    torch.from_numpy(ko).to(dev, torch.bfloat16), v, Kr, Vr, p, scale)
        torch.cuda.synchronize()
        # slot p: k as normalised (within a bf16 step on rare elements), v exactly; every other slot unchanged
        kp = to_np(K[:, :, p])
        diff = np.abs(kp - ko)
        assert (diff <= np.maximum(np.abs(ko), 0.5) * 2.0 ** -6).all(), f"p={p}: slot p beyond a bf16 step"
        flips += int((diff > 0).sum())
        assert torch.equal(V[:, :, p], v)
        others = [i for i in range(16) if i != p]   # untouched by either call: compare the two NaN-poisoned copies
        assert torch.equal(torch.nan_to_num(K[:, :, others]), torch.nan_to_num(Kr[:, :, others]))
        assert torch.equal(torch.nan_to_num(V[:, :, others]), torch.nan_to_num(Vr[:, :, others]))
        assert torch.isnan(K[:, :, p + 1:]).all()
        ok, st = ora.compare(to_np(out), to_np(ref), max_abs=2e-2, mean_abs=2e-4)
        assert ok, (p, st)
        Kn = to_np(K0).copy()
        Kn[:, :, p] = ko
        Vn = to_np(V0).copy()
        Vn[:, :, p] = to_np(v)
        ok, st = ora.compare(to_np(out), ora.cp_attn_triton_path(qo, Kn, Vn, p + 1, scale))
        assert ok, (p, st)
    print(f"[parity] cp_attn_append_rope B={B}: all 16 steps within the bar; {flips} slot elements a bf16 step from "
          f"the oracle's producers", flush=True)
    assert flips <= 2e-3 * B * 8 * D * 16


def test_cp_rope_step_in_graph_replays(cuda_device):
    dev = cuda_device
    B = 64
    qkv, qn, kn, K, V, cos, sin = _step_inputs(dev, B, seed=61)
    q, k, v = qkv[:, :2048].view(B, 16, D), qkv[:, 2048:3072].view(B, 8, D), qkv[:, 3072:].view(B, 8, D)
    scale = D ** -0.5
    eager = [q3attn.cp_attn_append_rope(q, k, v, K, V, p, scale, qn, kn, cos[p], sin[p]) for p in range(16)]
    torch.cuda.synchronize()
    K_ref, V_ref = K.clone(), V.clone()
    s = torch.cuda.Stream(dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        static = [q3attn.cp_attn_append_rope(q, k, v, K, V, p, scale, qn, kn, cos[p], sin[p]) for p in range(16)]
    for _ in range(3):
        K.fill_(float("nan"))
        V.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(a, b) for a, b in zip(static, eager))
        assert torch.equal(K, K_ref) and torch.equal(V, V_ref)
