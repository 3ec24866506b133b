"""CPU pins of the talker's q/k producers, ``rope(rms(x, w), cos, sin)`` (engine/ops.py:51-60), as the oracle restates
them (oracle.attention.norm_rope) and as the tests' torch copies run them (oracle.torch_cpu.rms / rope).

* Eager form (every torch op rounds to bf16; the prompt step and the admission layer run this way): the oracle equals
  torch's own CPU bf16 kernels running the reference's code bit for bit, on rows whose RMS spans 1e-4..10 (eps = 1e-6
  matters at the low end), random weights and RoPE rows of positions 0..2047.
* Mistakes planted in the oracle (the weight applied before the bf16 cast, eps dropped, the rotate-half halves
  swapped, cos and sin swapped, the sum of squares in place of the mean) each fail that check.
* Compiled form (every intermediate in float32 and one rounding at the end, as torch.compile's GPU kernels evaluate
  the chain; what the HIP kernels of the compiled callers compute): within one bf16 unit of the float64 evaluation of
  the same chain rounded once, equal on all but the elements its fp32 roundings move across a bf16 rounding boundary,
  and within the eager form's per-term roundings of it.
"""
import numpy as np
import pytest
import torch

from oracle import attention as ora
from oracle import torch_cpu as tc

D = 128


def _bf16(a):
    return ora.bf16_round(np.asarray(a, np.float32))


def _inputs(seed, n=96, heads=8):
    rng = np.random.default_rng(seed)
    scales = 10.0 ** rng.uniform(-4, 1, size=(n, heads, 1))
    x = _bf16(rng.standard_normal((n, heads, D)) * scales)
    w = _bf16(1.0 + 0.1 * rng.standard_normal(D))
    cos_t, sin_t = ora.rope_tables(2048)
    pos = rng.integers(0, 2048, size=n)
    return x, w, _bf16(cos_t[pos])[:, None, :], _bf16(sin_t[pos])[:, None, :]


def _torch_eager(x, w, cos, sin):
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(torch.bfloat16)
    return tc.rope(tc.rms(t(x), t(w)), t(cos), t(sin)).float().numpy()


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_eager_form_is_torch_bf16_ops_bit_for_bit(seed):
    x, w, cos, sin = _inputs(seed)
    want = _torch_eager(x, w, cos, sin)
    got = ora.norm_rope(x, w, cos, sin, eager=True)
    assert np.array_equal(got, want), f"{(got != want).mean():.4%} of elements differ"


def _plant_weight_before_cast(mp):
    mp.setattr(ora, "_normalise", lambda xf, r: (xf * r).astype(np.float32))


def _plant_no_eps(mp):
    f = ora._rsqrt_mean_sq
    mp.setattr(ora, "_rsqrt_mean_sq", lambda xf, eps: f(xf, 0.0))


def _plant_swapped_halves(mp):
    mp.setattr(ora, "_rotate_half", lambda y: np.concatenate([y[..., D // 2:], -y[..., : D // 2]], axis=-1))


def _plant_sum_not_mean(mp):
    mp.setattr(ora, "_rsqrt_mean_sq",
               lambda xf, eps: np.float32(1.0) / np.sqrt((xf * xf).sum(-1, keepdims=True, dtype=np.float32) +
                                                         np.float32(eps), dtype=np.float32))


PLANTED = {"weight before the cast": _plant_weight_before_cast, "eps dropped": _plant_no_eps,
           "halves swapped": _plant_swapped_halves, "sum of squares for the mean": _plant_sum_not_mean,
           "cos and sin swapped": None}


@pytest.mark.parametrize("name", sorted(PLANTED))
def test_planted_mistakes_fail_the_torch_check(monkeypatch, name):
    x, w, cos, sin = _inputs(11)
    want = _torch_eager(x, w, cos, sin)
    if PLANTED[name] is None:
        got = ora.norm_rope(x, w, sin, cos, eager=True)
    else:
        PLANTED[name](monkeypatch)
        got = ora.norm_rope(x, w, cos, sin, eager=True)
    same = float((got == want).mean())
    print(f"[producers] planted '{name}': {same:.4f} of elements still equal", flush=True)
    assert same < 0.99


def test_compiled_form_is_the_chain_rounded_once():
    x, w, cos, sin = _inputs(5)
    got = ora.norm_rope(x, w, cos, sin, eager=False)
    # the same chain in float64: y = w * x * r with r from the float64 mean, one rounding at the end
    xd = x.astype(np.float64)
    r = 1.0 / np.sqrt((xd * xd).mean(-1, keepdims=True) + 1e-6)
    y = w.astype(np.float64) * xd * r
    rot = np.concatenate([-y[..., D // 2:], y[..., : D // 2]], axis=-1)
    ref = _bf16((y * cos + rot * sin).astype(np.float32))
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(ref), 1e-30))) - 7)
    d = np.abs(got - ref)
    bound_terms = 2.0 ** -22 * (np.abs(y * cos) + np.abs(rot * sin))   # the fp32 products' and sum's rounding
    assert (d <= ulp + bound_terms).all() and (d == 0).mean() > 0.99, (d.max(), (d == 0).mean())
    # eager rounds y, y cos and rot(y) sin separately: where the two terms cancel the difference is bounded by the
    # terms' rounding, not the result's
    eager = ora.norm_rope(x, w, cos, sin, eager=True)
    de = np.abs(got - eager)
    bound = 2.0 ** -6 * (np.abs(y * cos) + np.abs(rot * sin)) + ulp
    assert (de <= bound).all() and (de == 0).mean() > 0.5, ((de / bound).max(), (de == 0).mean())
    print(f"[producers] compiled form: {(d == 0).mean():.5f} equal to the float64 chain, "
          f"{(de == 0).mean():.4f} equal to the eager form", flush=True)


def test_torch_copies_run_the_reference_rounding():
    """oracle.torch_cpu.rms / rope (the copies the synthetic models and GPU tests run) on the CPU: their composition is
    the eager form, and rms alone is the oracle's normalised-and-scaled row rounded by the product w * n."""
    x, w, cos, sin = _inputs(3)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(torch.bfloat16)
    n = tc.rms(t(x), t(w)).float().numpy()
    xf = x.astype(np.float32)
    assert np.array_equal(n, _bf16(w * ora._normalise(xf, ora._rsqrt_mean_sq(xf, 1e-6))))
    assert np.array_equal(_torch_eager(x, w, cos, sin), ora.norm_rope(x, w, cos, sin, eager=True))
