"""CPU checks that the GPU tests' and the benchmark's input generators (q3attn.workloads) compute what the pinned
oracle producers compute: the RoPE tables (engine/model_load.py:48-52), the unit-RMS scaling that stands in for the
qk-RMSNorm (engine/ops.py:51-55, no weight, kept in float32) and rotate-half RoPE (engine/ops.py:58-60).  The oracle's
rms/rope/rope_tables are themselves pinned by invariants in test_oracle.py; this ties the generators to them, so a
mistake in either copy (a swapped half, a wrong exponent, a dropped epsilon) fails here."""
import numpy as np
import pytest
import torch

from oracle import attention as ora
from q3attn import workloads as W


def test_rope_tables_match_oracle():
    cos_w, sin_w = W.rope_tables(1800, "cpu")
    cos_o, sin_o = ora.rope_tables(1800)
    assert cos_w.dtype == torch.float32
    # both evaluate the angles in float64 and round once to float32
    np.testing.assert_allclose(cos_w.numpy(), cos_o, rtol=0, atol=6e-8)
    np.testing.assert_allclose(sin_w.numpy(), sin_o, rtol=0, atol=6e-8)


@pytest.mark.parametrize("shape", [(7, 128), (3, 16, 128), (2, 5, 8, 128)])
def test_unit_rms_matches_oracle(shape):
    g = torch.Generator().manual_seed(sum(shape))
    x = torch.randn(shape, generator=g) * 3.0
    got = W._unit_rms(x).numpy()
    want = ora.rms(x.numpy(), to_bf16=False)
    np.testing.assert_allclose(got, want, rtol=4e-7, atol=0)
    np.testing.assert_allclose(np.sqrt((got * got).mean(-1)), 1.0, rtol=1e-5)


def test_rope_matches_oracle():
    g = torch.Generator().manual_seed(3)
    pos = torch.tensor([0, 1, 17, 399, 1799])
    cos, sin = W.rope_tables(1800, "cpu")
    x = torch.randn(5, 8, 128, generator=g)
    got = W._rope(x, cos[pos][:, None], sin[pos][:, None]).numpy()
    c, s = ora.rope_tables(1800)
    want = ora.rope(x.numpy(), c[pos.numpy()][:, None], s[pos.numpy()][:, None])
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-6)
    np.testing.assert_array_equal(got[0], x[0].numpy())          # position 0 is the identity


def test_decode_workload_keys_are_the_oracle_producers_output():
    """A small decode workload built on the CPU: every live token's K row and every q row is rope(unit_rms(.)), so it
    has unit RMS per head (RoPE preserves pair norms) up to the bf16 rounding."""
    ctx = np.array([5, 33, 0, 16])
    wl = W.make_decode("cpu", "cpu", ctx=ctx, num_pages=32, max_ctx=48, seed=4)
    L = wl.layers[0]
    bt = L.block_table.numpy()
    for b, c in enumerate(ctx):
        if c == 0:
            continue
        k = ora.gather_seat(wl.k_cache.float().numpy(), bt[b], int(c))       # [c, 8, 128]
        r = np.sqrt((k * k).mean(-1))
        np.testing.assert_allclose(r, 1.0, atol=1e-2)
    q = L.q.float().numpy()
    assert np.allclose(np.sqrt((q * q).mean(-1)), 1.0, atol=1e-2)


def test_prefill_workload_pool_holds_the_packed_rows():
    lens = np.array([3, 20, 17])
    wl = W.make_prefill("cpu", lens, seed=5, paged=True, num_pages=16)
    bt = wl.block_table.numpy()
    cu = wl.cu_seqlens.numpy()
    for s, n in enumerate(lens):
        got = ora.gather_seat(wl.k_cache.float().numpy(), bt[s], int(n))
        np.testing.assert_array_equal(got, wl.k[cu[s]:cu[s + 1]].float().numpy())
