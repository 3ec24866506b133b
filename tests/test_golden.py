"""The committed golden fixtures (tests/golden/*.npz): the oracle must still reproduce them (CPU), and the HIP
kernels must match them through the C ABI (GPU)."""
import os

import numpy as np
import pytest
import torch

from oracle import attention as ora

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return dict(np.load(os.path.join(GOLD, name), allow_pickle=False))


def f32(bits):
    return ora.bf16_bits_to_f32(bits)


def test_oracle_reproduces_decode_fixture():
    d = load("decode_small.npz")
    bt = np.where(d["block_table"] < 0, 0, d["block_table"])
    out = ora.paged_decode(f32(d["q"]), f32(d["k_cache"]), f32(d["v_cache"]), d["cache_seqlens"], bt,
                           float(d["scale"]), acc=np.float64)
    np.testing.assert_allclose(out, d["out"], rtol=0, atol=1e-6)


def test_oracle_reproduces_cp_fixture():
    d = load("cp_small.npz")
    for n in d["n_live"]:
        q = f32(d[f"q{n}"])
        assert np.array_equal(ora.cp_attn_triton_path(q, f32(d["K"]), f32(d["V"]), int(n), float(d["scale"])),
                              d[f"out_triton{n}"])
        assert np.array_equal(ora.cp_attn_torch_path(q, f32(d["K"]), f32(d["V"]), int(n), float(d["scale"])),
                              d[f"out_torch{n}"])


def _bf16_tensor(bits, dev):
    return torch.from_numpy(bits.astype(np.int16)).view(torch.bfloat16).to(dev)


@pytest.mark.gpu
def test_decode_kernel_matches_fixture(cuda_device):
    import q3attn
    d = load("decode_small.npz")
    q = _bf16_tensor(d["q"], cuda_device)
    kc = _bf16_tensor(d["k_cache"], cuda_device)
    vc = _bf16_tensor(d["v_cache"], cuda_device)
    sl = torch.from_numpy(d["cache_seqlens"]).to(cuda_device)
    bt = torch.from_numpy(d["block_table"]).to(cuda_device)
    for split in (0, 16, 64):
        o = q3attn.paged_decode(q, kc, vc, sl, bt, float(d["scale"]), split)
        torch.cuda.synchronize()
        ok, st = ora.compare(o.float().cpu().numpy(), d["out"])
        assert ok, (split, st)


@pytest.mark.gpu
def test_cp_kernel_matches_fixture(cuda_device):
    import q3attn
    d = load("cp_small.npz")
    K = _bf16_tensor(d["K"], cuda_device)
    V = _bf16_tensor(d["V"], cuda_device)
    for n in d["n_live"]:
        o = q3attn.cp_attn(_bf16_tensor(d[f"q{n}"], cuda_device), K, V, int(n), float(d["scale"]))
        torch.cuda.synchronize()
        got = o.float().cpu().numpy()
        for ref in ("out_triton", "out_exact"):
            ok, st = ora.compare(got, d[f"{ref}{n}"])
            assert ok, (int(n), ref, st)
