"""Seeded randomized sweep of the kernels' general shapes against the oracle: KV-head counts 1..16 (the model uses
8), page sizes 16/32/256, stream-K and fixed splits, the append form, padded cache rows (non-trivial token/head
strides), q and out as strided views, prefill with q as a slice of a fused qkv tensor, and the CP kernel with other
head counts.  Bar: max-abs 2e-2, mean-abs 2e-3 against the fp32-softmax oracle on the same bf16 inputs."""
import numpy as np
import pytest
import torch

import q3attn
from helpers import to_np
from oracle import attention as ora

pytestmark = pytest.mark.gpu


def _bf16(rng, shape, dev):
    return torch.from_numpy(rng.standard_normal(shape).astype(np.float32)).to(dev).to(torch.bfloat16)


def _check(out, ref, what):
    ok, st = ora.compare(to_np(out), ref)
    print(f"[sweep] {what} {st}", flush=True)
    assert ok, (what, st)


DECODE_CASES = [
    dict(hkv=1, page=16, B=5, max_ctx=300, split=0, append=False, pad=0),
    dict(hkv=2, page=32, B=17, max_ctx=500, split=0, append=True, pad=8),
    dict(hkv=4, page=16, B=33, max_ctx=200, split=64, append=False, pad=8),
    dict(hkv=16, page=16, B=9, max_ctx=400, split=0, append=False, pad=0),
    dict(hkv=16, page=256, B=4, max_ctx=700, split=0, append=True, pad=0),
    dict(hkv=8, page=32, B=100, max_ctx=120, split=16, append=True, pad=8),
    dict(hkv=4, page=256, B=3, max_ctx=1000, split=1024, append=False, pad=0),
    dict(hkv=8, page=16, B=1, max_ctx=2000, split=0, append=True, pad=0),
    # stream-K at small batches (tables past 2,048 tokens) and past 64 rows
    dict(hkv=2, page=32, B=17, max_ctx=2100, split=0, append=True, pad=8),
    dict(hkv=16, page=16, B=9, max_ctx=2100, split=0, append=False, pad=0),
    dict(hkv=1, page=16, B=70, max_ctx=300, split=0, append=False, pad=0),
]


@pytest.mark.parametrize("case", DECODE_CASES, ids=lambda c: "-".join(f"{k}{v}" for k, v in c.items()))
def test_decode_shapes(cuda_device, case):
    rng = np.random.default_rng(hash(tuple(case.values())) % (1 << 31))
    hkv, page, B, max_ctx, split = case["hkv"], case["page"], case["B"], case["max_ctx"], case["split"]
    P = -(-max_ctx // page)
    num_pages = B * P + 8
    D = 128 + case["pad"]                                     # padded head rows -> head/token strides != 128
    kpool = _bf16(rng, (num_pages, page, hkv, D), cuda_device)[..., :128]
    vpool = _bf16(rng, (num_pages, page, hkv, D), cuda_device)[..., :128]
    lo = 1 if case["append"] else 0
    ctx = rng.integers(lo, max_ctx + 1, size=B)
    ctx[0] = max_ctx
    if not case["append"] and B > 2:
        ctx[1] = 0
    bt = rng.permutation(num_pages)[: B * P].reshape(B, P).astype(np.int32)
    qkv = _bf16(rng, (B, 4 * hkv + 1, 128), cuda_device)      # q as a strided view of a wider row
    q = qkv[:, : 2 * hkv]
    scale = 128 ** -0.5
    bt_d = torch.from_numpy(bt).to(cuda_device)
    if case["append"]:
        k_new = _bf16(rng, (B, hkv, 128), cuda_device)
        v_new = _bf16(rng, (B, hkv, 128), cuda_device)
        old = torch.from_numpy(ctx - 1).to(torch.int32).to(cuda_device)
        out = q3attn.paged_decode_append(q, k_new, v_new, kpool, vpool, old, bt_d, scale, split)
        torch.cuda.synchronize()
        kh, vh = to_np(kpool), to_np(vpool)                   # pools after the append
        for b in range(B):
            pos = int(ctx[b]) - 1
            pg, off = bt[b, pos // page], pos % page
            assert np.array_equal(kh[pg, off], to_np(k_new[b])) and np.array_equal(vh[pg, off], to_np(v_new[b]))
    else:
        out = q3attn.paged_decode(q, kpool, vpool, torch.from_numpy(ctx).to(torch.int32).to(cuda_device), bt_d,
                                  scale, split)
        torch.cuda.synchronize()
        kh, vh = to_np(kpool), to_np(vpool)
    ref = ora.paged_decode(to_np(q), kh, vh, ctx, bt, scale)
    _check(out, ref, f"decode {case}")


PREFILL_CASES = [
    dict(hkv=1, paged=False, page=0, causal=True, lens=[1, 70, 129]),
    dict(hkv=2, paged=True, page=64, causal=True, lens=[200, 33, 64, 5]),
    dict(hkv=4, paged=True, page=16, causal=False, lens=[48, 300]),
    dict(hkv=8, paged=True, page=256, causal=True, lens=[513, 17]),
    dict(hkv=16, paged=False, page=0, causal=True, lens=[90, 64, 1]),
]


@pytest.mark.parametrize("case", PREFILL_CASES, ids=lambda c: f"hkv{c['hkv']}-paged{c['paged']}-page{c['page']}-causal{c['causal']}")
def test_prefill_shapes(cuda_device, case):
    rng = np.random.default_rng(7 + case["hkv"])
    hkv, lens = case["hkv"], np.array(case["lens"])
    T = int(lens.sum())
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    qkv = _bf16(rng, (T, 4 * hkv, 128), cuda_device)          # engine-style fused projection, q/k/v are views
    q, k, v = qkv[:, : 2 * hkv], qkv[:, 2 * hkv: 3 * hkv], qkv[:, 3 * hkv:]
    cu_d = torch.from_numpy(cu).to(cuda_device)
    scale = 128 ** -0.5
    if case["paged"]:
        page = case["page"]
        P = int((-(-lens // page)).max())
        num_pages = int((-(-lens // page)).sum()) + 5
        bt = np.full((len(lens), P), -1, np.int32)
        perm = rng.permutation(num_pages)
        kc = torch.zeros((num_pages, page, hkv, 128), dtype=torch.bfloat16, device=cuda_device)
        vc = torch.zeros_like(kc)
        i = 0
        for s, L in enumerate(lens):
            for j in range(-(-L // page)):
                bt[s, j] = perm[i]
                i += 1
                n = min(page, L - j * page)
                kc[bt[s, j], :n] = k[cu[s] + j * page: cu[s] + j * page + n]
                vc[bt[s, j], :n] = v[cu[s] + j * page: cu[s] + j * page + n]
        out = q3attn.flash_attn_varlen_func(q, kc, vc, cu_d, cu_d, int(lens.max()), int(lens.max()),
                                            softmax_scale=scale, causal=case["causal"],
                                            block_table=torch.from_numpy(bt).to(cuda_device))
    else:
        out = q3attn.flash_attn_varlen_func(q, k, v, cu_d, cu_d, int(lens.max()), int(lens.max()),
                                            softmax_scale=scale, causal=case["causal"])
    torch.cuda.synchronize()
    qn, kn, vn = to_np(q), to_np(k), to_np(v)
    if case["causal"]:
        ref = ora.prefill_varlen(qn, kn, vn, cu, scale)
    else:
        ref = np.zeros_like(qn)
        G = 2
        for s in range(len(lens)):
            sl = slice(cu[s], cu[s + 1])
            a = np.einsum("thd,shd->hts", qn[sl], np.repeat(kn[sl], G, axis=1)) * scale
            a -= a.max(-1, keepdims=True)
            p = np.exp(a)
            p /= p.sum(-1, keepdims=True)
            ref[sl] = np.einsum("hts,shd->thd", p, np.repeat(vn[sl], G, axis=1))
    _check(out, ref, f"prefill {case}")


@pytest.mark.parametrize("hkv,B,n_live", [(1, 7, 16), (4, 40, 3), (16, 9, 11), (2, 130, 1)])
def test_cp_shapes(cuda_device, hkv, B, n_live):
    rng = np.random.default_rng(hkv * 100 + B)
    K = _bf16(rng, (B + 3, hkv, 16, 136), cuda_device)[:B, :, :, :128]     # padded slots, batch slice
    V = _bf16(rng, (B + 3, hkv, 16, 136), cuda_device)[:B, :, :, :128]
    q = _bf16(rng, (B, 2 * hkv, 128), cuda_device)
    o = q3attn.cp_attn(q, K, V, n_live, 0.088)
    torch.cuda.synchronize()
    _check(o, ora.cp_attn_triton_path(to_np(q), to_np(K), to_np(V), n_live, 0.088), f"cp hkv={hkv} B={B} n={n_live}")
