"""Code-0 criterion on a seeded synthetic 28-layer talker.

The same frames run with every op identical except attention: the HIP decode kernel, the fp32 oracle (rounded to
bf16 like any kernel output), the same oracle accumulating in float64, and an independent bf16 attention written the
reference's torch way.  Seats join at staggered frames (ragged contexts); pages are 16 tokens through a random table.
Teacher-forced: all runs consume the fp32 oracle run's sampled code-0, so differences never compound through the
inputs.  The comparisons run on the processed scores the sampler sees (engine/talker.py:90-98): every path's raw
codec-head logits go through the same per-seat state (repetition penalty over the seat's generated ids, specials
suppressed except EOS, EOS blocked for the first two frames), updated with the oracle's codes.

Each layer's attention output is rounded to bf16, and over 28 layers those roundings accumulate into a ~1% relative
difference of the codebook-0 logits between any two correct implementations: the float64 oracle, whose outputs differ
from the float32 oracle's only in the last bf16 bit here and there, already flips some near-tie argmaxes and seeded
samples.  That disagreement is the floor, and it is measured in the same run.  The HIP kernel must stay within it (and
within the reference's own bf16 recipe's), keep the argmax identical wherever the oracle's top-1 margin clears the
guard, and stay under explicit bounds on flips and sample mismatches (printed, so a regression shows as a count).
Two o-projection scales run: the standard init (gain 1) and gain 4, where the attention output dominates each layer's
update (the difference in the logits is of the same order at both, which shows it is accumulated rounding, not the
gain).
"""
import numpy as np
import pytest
import torch

import q3attn
from synthetic_talker import (PAGE, Cb0State, SyntheticTalker, oracle64_attention, oracle_attention, sample_topk,
                              torch_bf16_attention)

pytestmark = pytest.mark.gpu

MARGIN_GUARD = 0.25      # logit units (the synthetic logits have std ~4)


def hip_attention(q, kc, vc, ctx, bt, scale):
    return q3attn.flash_attn_with_kvcache(q.unsqueeze(1), kc, vc, cache_seqlens=ctx, block_table=bt,
                                          softmax_scale=scale, causal=True)[:, 0]


# o_gain -> (max argmax flips, max seeded-sample mismatches) of the HIP path on the processed scores, as fractions of
# the cases.  Measured on MI355X (788 cases, flips / sample mismatches): gain 1: HIP 28 / 133, float64 oracle 19 / 122,
# torch bf16 recipe 21 / 131; gain 4: HIP 18 / 94, float64 oracle 14 / 97, torch bf16 20 / 108.
BOUNDS = {1.0: (0.04, 0.22), 4.0: (0.025, 0.15)}


@pytest.mark.parametrize("o_gain", sorted(BOUNDS))
def test_code0_against_oracle_talker(cuda_device, o_gain):
    seats, frames, prompt = 24, 40, 12
    T = SyntheticTalker(cuda_device, layers=28, seed=7, o_gain=o_gain)
    P = (frames + PAGE - 1) // PAGE
    rng = np.random.default_rng(7)
    num_pages = 4 * seats * P
    bt = torch.from_numpy(rng.permutation(num_pages)[: seats * P].reshape(seats, P).astype(np.int32)).to(cuda_device)
    start = np.array([(3 * b) % 16 for b in range(seats)])
    paths = {"hip": hip_attention, "oracle": oracle_attention, "oracle_f64": oracle64_attention,
             "torch_bf16": torch_bf16_attention}
    pools = {k: T.new_pools(num_pages) for k in paths}
    gens = {k: torch.Generator(device=cuda_device) for k in paths}
    for g in gens.values():
        g.manual_seed(123)
    emb_gen = torch.Generator(device=cuda_device).manual_seed(99)
    text = torch.randn(seats, frames, 1024, generator=emb_gen, device=cuda_device).to(torch.bfloat16)
    prev = torch.zeros(seats, dtype=torch.long, device=cuda_device)
    cb0 = Cb0State(seats, cuda_device)
    stats = {k: dict(agree=0, agree_guarded=0, sampled=0, rel=[]) for k in ("hip", "oracle_f64", "torch_bf16")}
    total = guarded = 0
    for f in range(frames):
        act = np.nonzero(f >= start)[0]
        if len(act) == 0:
            continue
        a = torch.from_numpy(act).to(cuda_device)
        pos = torch.from_numpy(f - start[act]).to(cuda_device)
        x = text[a, pos]
        x = torch.where((pos >= prompt)[:, None], x + T.codec_emb[prev[a]], x)
        out = {}
        for name, attn in paths.items():
            kc, vc = pools[name]
            raw = T.logits(T.decode(x, pos, bt[a], kc, vc, attn))
            lg = cb0.process(raw, a)
            out[name] = (raw, lg, sample_topk(lg, 0.9, 50, gens[name]))
        ro, lo, so = out["oracle"]
        top2 = lo.topk(2, dim=-1).values
        clear = (top2[:, 0] - top2[:, 1]) > MARGIN_GUARD
        total += len(act)
        guarded += int(clear.sum())
        for name in stats:
            raw, lg, smp = out[name]
            same = lg.argmax(-1) == lo.argmax(-1)
            stats[name]["agree"] += int(same.sum())
            stats[name]["agree_guarded"] += int(same[clear].sum())
            stats[name]["sampled"] += int((smp == so).sum())
            stats[name]["rel"].append(float((raw - ro).norm() / ro.norm()))
        cb0.update(a, so)
        prev[a] = so
    for name, st in stats.items():
        rel = np.array(st["rel"])
        print(f"[code0] o_gain={o_gain} {name}: argmax {st['agree']}/{total} (flips {total - st['agree']}), "
              f"argmax on clear margins {st['agree_guarded']}/{guarded}, seeded samples {st['sampled']}/{total} "
              f"(mismatches {total - st['sampled']}), raw logit rel mean {rel.mean():.2e} max {rel.max():.2e}",
              flush=True)
    hip, ref, f64 = stats["hip"], stats["torch_bf16"], stats["oracle_f64"]
    max_flips, max_mismatch = BOUNDS[o_gain]
    assert total - hip["agree"] <= max_flips * total, "too many code-0 argmax flips against the oracle"
    assert total - hip["sampled"] <= max_mismatch * total, "too many seeded-sample mismatches against the oracle"
    assert hip["agree_guarded"] == guarded, "code-0 argmax flips where the oracle's margin is clear"
    floor_flips = max(total - f64["agree"], total - ref["agree"])
    floor_mismatch = max(total - f64["sampled"], total - ref["sampled"])
    assert total - hip["agree"] <= floor_flips + 0.01 * total
    assert total - hip["sampled"] <= floor_mismatch + 0.02 * total
    assert np.mean(hip["rel"]) <= 1.25 * np.mean(ref["rel"]) + 1e-3
    assert hip["agree"] >= ref["agree"] - 0.01 * total
    assert hip["sampled"] >= ref["sampled"] - 0.02 * total
