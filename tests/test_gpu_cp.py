"""GPU parity of the code-predictor attention (q3a_cp_attn through the C ABI) against the oracle's
two reference rounding sequences (engine/cp_attn.py:19-30 and engine/code_predictor.py:46-47)."""
import numpy as np
import pytest
import torch

import q3attn
from helpers import to_np
from oracle import attention as ora
from q3attn import workloads as W

pytestmark = pytest.mark.gpu


def _np(qs, K, V):
    return [to_np(q) for q in qs], to_np(K), to_np(V)


@pytest.mark.parametrize("kv_pad", [0, 8])
def test_all_steps_c2(cuda_device, kv_pad):
    B = 512
    qs, K, V = W.make_cp(B, cuda_device, seed=kv_pad, kv_pad=kv_pad)
    qn, Kn, Vn = _np(qs, K, V)
    for p in range(16):
        n_live = p + 1
        o = q3attn.cp_attn(qs[p], K, V, n_live, W.HEAD_DIM ** -0.5)
        torch.cuda.synchronize()
        got = to_np(o)
        scale = W.HEAD_DIM ** -0.5
        exact = ora.cp_attn_exact(qn[p], Kn, Vn, n_live, scale)
        # fp32-score reference (engine/cp_attn.py:19-30) and the exact result: the parity bar
        for name, ref in (("triton_path", ora.cp_attn_triton_path(qn[p], Kn, Vn, n_live, scale)), ("exact", exact)):
            ok, st = ora.compare(got, ref)
            print(f"[parity] cp n_live={n_live} pad={kv_pad} vs {name} {st}", flush=True)
            assert ok, (n_live, name, st)
        # bf16-score torch path (engine/code_predictor.py:46-47): it rounds the scores to bf16 before
        # the softmax, so its own distance from the exact result can exceed 2e-2.  The kernel must
        # be no further from exact than that path and agree with it on average.
        torch_path = ora.cp_attn_torch_path(qn[p], Kn, Vn, n_live, scale)
        _, st_t = ora.compare(got, torch_path)
        _, st_ref = ora.compare(torch_path, exact)
        _, st_ours = ora.compare(got, exact)
        print(f"[parity] cp n_live={n_live} vs torch_path {st_t}; torch_path vs exact {st_ref}", flush=True)
        assert st_t["mean_abs"] <= 2e-3, st_t
        assert st_ours["max_abs"] <= st_ref["max_abs"] and st_ours["mean_abs"] <= st_ref["mean_abs"]


def test_n_live_1_is_exact(cuda_device):
    qs, K, V = W.make_cp(64, cuda_device, seed=3)
    o = q3attn.cp_attn(qs[0], K, V, 1, 0.088).reshape(64, 8, 2, 128)
    torch.cuda.synchronize()
    assert torch.equal(o, V[:, :, 0:1].expand(-1, -1, 2, -1))


def test_stale_slots_never_read(cuda_device):
    qs, K, V = W.make_cp(128, cuda_device, seed=4)
    for n_live in (1, 6, 15):
        a = q3attn.cp_attn(qs[n_live - 1], K, V, n_live, 0.088)
        Kp, Vp = K.clone(), V.clone()
        Kp[:, :, n_live:] = float("nan")
        Vp[:, :, n_live:] = float("nan")
        b = q3attn.cp_attn(qs[n_live - 1], Kp, Vp, n_live, 0.088)
        torch.cuda.synchronize()
        assert torch.equal(a, b)


def test_batch_stride_wider_than_live_batch(cuda_device):
    """K/V are slices [l, :B] of a [layers, max_bs, 8, 16, 128] scratch (engine/code_predictor.py:56)."""
    max_bs, B = 96, 40
    qs, K, V = W.make_cp(max_bs, cuda_device, seed=5)
    Kbig = torch.stack([torch.zeros_like(K), K])
    Vbig = torch.stack([torch.zeros_like(V), V])
    o = q3attn.cp_attn(qs[9][:B].reshape(B, 2048), Kbig[1, :B], Vbig[1, :B], 10, 0.088)
    full = q3attn.cp_attn(qs[9], K, V, 10, 0.088)
    torch.cuda.synchronize()
    assert torch.equal(o, full[:B])


def test_odd_batch_sizes(cuda_device):
    for B in (1, 3, 5, 272, 577):
        qs, K, V = W.make_cp(B, cuda_device, seed=B, steps=4)
        o = q3attn.cp_attn(qs[3], K, V, 4, 0.088)
        torch.cuda.synchronize()
        ok, st = ora.compare(to_np(o), ora.cp_attn_triton_path(to_np(qs[3]), to_np(K), to_np(V), 4, 0.088))
        assert ok, (B, st)


def _step_rows(B, device, seed):
    """This step's k (contiguous [B, 8, 128]) and v as a view into a [B, 4096] qkv projection, the layouts
    engine/code_predictor.py:38-42 hands to the slot write."""
    g = torch.Generator(device=device).manual_seed(seed)
    k = torch.randn(B, 8, 128, generator=g, device=device).to(torch.bfloat16)
    qkv = torch.randn(B, 4096, generator=g, device=device).to(torch.bfloat16)
    return k, qkv[:, 3072:].view(B, 8, 128)


@pytest.mark.parametrize("kv_pad", [0, 8])
def test_append_matches_index_copy_then_attn(cuda_device, kv_pad):
    """cp_attn_append == K.index_copy_ + V.index_copy_ + cp_attn, bit for bit, for every slot p, and leaves
    the scratch exactly as the index_copy_ pair does (engine/code_predictor.py:58)."""
    B = 300
    qs, K, V = W.make_cp(B, cuda_device, seed=11, kv_pad=kv_pad)
    _, K2, V2 = W.make_cp(B, cuda_device, seed=11, kv_pad=kv_pad, steps=0)
    for t in (K, V, K2, V2):
        t.zero_()
    scale = W.HEAD_DIM ** -0.5
    for p in range(16):
        k, v = _step_rows(B, cuda_device, 100 + p)
        pidx = torch.tensor([p], device=cuda_device)
        K.index_copy_(2, pidx, k.unsqueeze(2))
        V.index_copy_(2, pidx, v.unsqueeze(2))
        ref = q3attn.cp_attn(qs[p], K, V, p + 1, scale)
        got = q3attn.cp_attn_append(qs[p], k, v, K2, V2, p, scale)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), p
        assert torch.equal(K2, K) and torch.equal(V2, V), p
        if p in (0, 7, 15):
            ok, st = ora.compare(to_np(got), ora.cp_attn_triton_path(to_np(qs[p]), to_np(K), to_np(V), p + 1, scale))
            print(f"[parity] cp_append p={p} pad={kv_pad} vs triton_path {st}", flush=True)
            assert ok, (p, st)


def test_append_writes_only_slot_p(cuda_device):
    B = 64
    qs, K, V = W.make_cp(B, cuda_device, seed=12)
    k, v = _step_rows(B, cuda_device, 7)
    K0, V0 = K.clone(), V.clone()
    q3attn.cp_attn_append(qs[5], k, v, K, V, 5, 0.088)
    torch.cuda.synchronize()
    keep = [s for s in range(16) if s != 5]
    assert torch.equal(K[:, :, keep], K0[:, :, keep]) and torch.equal(V[:, :, keep], V0[:, :, keep])
    assert torch.equal(K[:, :, 5], k) and torch.equal(V[:, :, 5], v)


def test_append_batch_slice_of_wider_scratch(cuda_device):
    """K/V are [l, :B] slices of the [layers, max_bs, 8, 16, 128] scratch: rows >= B stay untouched."""
    max_bs, B, p = 96, 40, 3
    qs, K, V = W.make_cp(max_bs, cuda_device, seed=13)
    Kbig, Vbig = torch.stack([K.clone(), K.clone()]), torch.stack([V.clone(), V.clone()])
    before = Kbig.clone(), Vbig.clone()
    k, v = _step_rows(B, cuda_device, 8)
    got = q3attn.cp_attn_append(qs[p][:B], k, v, Kbig[1, :B], Vbig[1, :B], p, 0.088)
    K[:B, :, p] = k
    V[:B, :, p] = v
    ref = q3attn.cp_attn(qs[p][:B], K[:B], V[:B], p + 1, 0.088)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
    assert torch.equal(Kbig[0], before[0][0]) and torch.equal(Vbig[0], before[1][0])
    assert torch.equal(Kbig[1, B:], before[0][1, B:]) and torch.equal(Vbig[1, B:], before[1][1, B:])
    assert torch.equal(Kbig[1, :B], K[:B]) and torch.equal(Vbig[1, :B], V[:B])
