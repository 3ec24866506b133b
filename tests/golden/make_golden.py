"""Writes the small golden fixtures of this directory from the oracle (run: python tests/golden/make_golden.py).

Inputs are seeded numpy draws rounded to bf16 (stored as uint16 bit patterns); expected outputs are the oracle's
float64 results stored as float32.  The fixtures freeze the oracle's answers so later changes to it, or to the
kernels, are checked against fixed vectors.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle import attention as ora  # noqa: E402


def bf16(x):
    return ora.f32_to_bf16_bits(np.asarray(x, np.float32))


def decode_fixture(rng):
    # 2 query heads over 1 KV head, head_dim 128, 16-token pages, 12-page pool, ragged rows incl. ctx 0 and 1.
    ctx = np.array([0, 1, 15, 16, 17, 70], np.int32)
    page, num_pages, P = 16, 12, 5
    q = bf16(rng.standard_normal((6, 2, 128)))
    k = bf16(rng.standard_normal((num_pages, page, 1, 128)))
    v = bf16(rng.standard_normal((num_pages, page, 1, 128)))
    bt = np.full((6, P), -1, np.int32)
    perm = rng.permutation(num_pages)
    used = 0
    for b, c in enumerate(ctx):
        n = -(-int(c) // page)
        bt[b, :n] = perm[used:used + n]
        used += n
    scale = 128 ** -0.5
    out = ora.paged_decode(ora.bf16_bits_to_f32(q), ora.bf16_bits_to_f32(k), ora.bf16_bits_to_f32(v), ctx,
                           np.where(bt < 0, 0, bt), scale, acc=np.float64)
    return dict(q=q, k_cache=k, v_cache=v, cache_seqlens=ctx, block_table=bt, scale=np.float64(scale),
                out=out.astype(np.float32))


def cp_fixture(rng):
    # 2 query heads over 1 KV head, 3 rows, the 16-slot scratch, steps n_live = 1, 5, 16.
    B, scale = 3, 128 ** -0.5
    K = bf16(rng.standard_normal((B, 1, 16, 128)))
    V = bf16(rng.standard_normal((B, 1, 16, 128)))
    d = dict(K=K, V=V, scale=np.float64(scale), n_live=np.array([1, 5, 16], np.int32))
    Kf, Vf = ora.bf16_bits_to_f32(K), ora.bf16_bits_to_f32(V)
    for n in (1, 5, 16):
        q = bf16(rng.standard_normal((B, 2, 128)))
        qf = ora.bf16_bits_to_f32(q)
        d[f"q{n}"] = q
        d[f"out_triton{n}"] = ora.cp_attn_triton_path(qf, Kf, Vf, n, scale)
        d[f"out_torch{n}"] = ora.cp_attn_torch_path(qf, Kf, Vf, n, scale)
        d[f"out_exact{n}"] = ora.cp_attn_exact(qf, Kf, Vf, n, scale).astype(np.float32)
    return d


def main():
    rng = np.random.default_rng(20261201)
    np.savez_compressed(os.path.join(HERE, "decode_small.npz"), **decode_fixture(rng))
    np.savez_compressed(os.path.join(HERE, "cp_small.npz"), **cp_fixture(rng))


if __name__ == "__main__":
    main()
