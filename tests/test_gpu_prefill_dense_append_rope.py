"""GPU parity of the attention blocks with their q/k producers in one call: the fast-admission layer
(q3a_prefill_dense_append_rope) and, at the end of the file, the talker's prompt step (q3a_prefill_append_rope).

engine/arrivals.py:112-118 normalises and rotates q and the new keys (engine/ops.py:51-60, eager bf16 ops by default:
the admission layer is not compiled, engine/arrivals.py:57-61), concatenates the registered voice's prefix K/V
before the new rows, scatters every K/V row into the seat's cache (:144-145) and attends (:148).  Against that:
  * the output is within the bar of the oracle attention (engine/arrivals.py:125-131) over the oracle's producers,
    which restate engine/ops.py:51-60 with the eager rounding points (every op rounds to bf16);
  * the pool holds the prefix rows and the new V rows bit for bit, and the new K rows as the oracle's producers
    give them up to the last bf16 bit of a rare row (the mean of squares is summed in another order);
  * positions outside first_row .. n-1 of the NaN-filled pool stay NaN;
  * against the same producers as eager torch ops on the GPU followed by prefill_dense_append, outputs and pools
    agree to the same last-bit allowance.
Shapes with n <= 128 keys take the short-key attention kernel, longer ones the tiled kernel."""
import numpy as np
import pytest
import torch

import q3attn
from helpers import to_np
from oracle import attention as ora
from oracle import torch_cpu as tc
from q3attn import workloads as W

pytestmark = pytest.mark.gpu

D = 128


def _eager_norm_rope_np(x, w, cos, sin, eps=1e-6):
    """engine/ops.py:51-60 as eager bf16 ops (the oracle's eager form, pinned to torch's bf16 kernels on the CPU)."""
    return ora.norm_rope(x, w, cos, sin, eps, eager=True)


def _eager_norm_rope_torch(x, w, cos, sin, eps=1e-6):
    """The same producers as the engine runs them: the reference's torch ops, here on the GPU."""
    return tc.rope(tc.rms(x, w, eps), cos, sin)


def _inputs(dev, S, R, P, n_prefixes, seed):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    qkv = torch.randn((S, R, 4096), generator=g, device=dev).to(torch.bfloat16)
    pre = W.make_admit(dev, n_prefixes, 1, P, seed=seed + 1) if P > 0 else None
    pk = pre.k if pre is not None else torch.zeros(n_prefixes, 0, 8, D, dtype=torch.bfloat16, device=dev)
    pv = pre.v if pre is not None else torch.zeros_like(pk)
    qn = (1.0 + 0.1 * torch.randn(D, generator=g, device=dev)).to(torch.bfloat16)
    kn = (1.0 + 0.1 * torch.randn(D, generator=g, device=dev)).to(torch.bfloat16)
    cos, sin = W.rope_tables(P + R, dev)
    return qkv, pk, pv, qn, kn, cos[P:].to(torch.bfloat16).contiguous(), sin[P:].to(torch.bfloat16).contiguous()


def _views(qkv):
    S, R = qkv.shape[:2]
    return (qkv[..., :2048].view(S, R, 16, D), qkv[..., 2048:3072].view(S, R, 8, D), qkv[..., 3072:].view(S, R, 8, D))


def _table(S, P, num_pages, seed):
    return np.random.default_rng(seed).permutation(num_pages)[: S * P].reshape(S, P).astype(np.int32)


def _pool_rows(cache, bt, n, page):
    """[S, n, Hkv, D] rows 0..n-1 of every sequence read back through its table."""
    S = bt.shape[0]
    j = np.arange(n)
    return cache[bt[:, j // page], j % page]


def _assert_last_bit(a, b, what, frac=2e-3):
    """Equal except for rare elements a bf16 step or two apart: the mean of squares summed in another order can move
    one normalised value by one bf16 step, and the rope's sum can then land a step or two away (more where its two
    products cancel, so the bound is relative to the normalised rows' unit scale as well)."""
    diff = np.abs(a.astype(np.float32) - b.astype(np.float32))
    bad = diff > 0
    tol = np.maximum(np.abs(b).astype(np.float32), 0.5) * 2.0 ** -6
    assert (diff <= tol).all(), f"{what}: a difference beyond two bf16 steps ({diff.max():.3e})"
    assert bad.mean() <= frac, f"{what}: {bad.mean():.2e} of the elements differ"
    print(f"[parity] {what}: {int(bad.sum())} of {bad.size} elements one bf16 step apart", flush=True)


@pytest.mark.parametrize("S,R,P,page,first,indexed,causal", [
    (8, 42, 35, 16, 0, True, True),       # the admission shape: 8 seats, 42 new tokens after a 35-token voice prefix
    (8, 42, 35, 16, 35, True, True),      # prefix already in the pool: the new rows only
    (4, 42, 35, 256, 0, False, True),     # the reference's 256-token pages, one prefix per sequence
    (3, 20, 0, 16, 0, False, True),       # no prefix
    (5, 70, 50, 16, 3, True, True),       # one launch, 5 query groups, part of the prefix into the pool
    (2, 120, 5, 16, 0, True, True),       # 125 keys but 8 query groups: the two-launch form on the short-key kernel
    (2, 100, 200, 16, 0, True, True),     # 300 keys: the tiled attention kernel
    (2, 40, 660, 32, 600, True, True),    # tiled, part of a long prefix
    (4, 42, 35, 16, 0, True, False),      # non-causal, one launch (the last key tile's masking only)
    (2, 120, 5, 16, 0, True, False),      # non-causal, the two-launch form
])
def test_dense_append_rope_matches_oracle(cuda_device, S, R, P, page, first, indexed, causal):
    dev = cuda_device
    n = P + R
    nvoices = 3 if indexed else S
    qkv, pk, pv, qn, kn, cos, sin = _inputs(dev, S, R, P, nvoices, seed=40 + n)
    q, k, v = _views(qkv)
    pidx = torch.tensor([(2 * s + 1) % nvoices for s in range(S)], dtype=torch.int64, device=dev) if indexed else None
    Pn = -(-n // page)
    num_pages = max(2 * S * Pn, 64)
    bt = _table(S, Pn, num_pages, seed=41)
    kc = torch.full((num_pages, page, 8, D), float("nan"), dtype=torch.bfloat16, device=dev)
    vc = torch.full_like(kc, float("nan"))
    scale = D ** -0.5
    print(f"[case] prefill_dense_append_rope S={S} R={R} P={P} page={page} first={first} indexed={indexed} "
          f"causal={causal}", flush=True)
    out = q3attn.prefill_dense_append_rope(q, k, v, pk, pv, qn, kn, cos, sin, kc, vc,
                                           torch.from_numpy(bt).to(dev), scale, pidx, causal, 1e-6, first)
    torch.cuda.synchronize()
    # the oracle's producers and attention
    sel = pidx.cpu().numpy() if indexed else np.arange(S)
    cn, sn = to_np(cos)[None, :, None], to_np(sin)[None, :, None]
    q_o = _eager_norm_rope_np(to_np(q), to_np(qn), cn, sn)
    k_o = _eager_norm_rope_np(to_np(k), to_np(kn), cn, sn)
    K = np.concatenate([to_np(pk)[sel], k_o], axis=1)
    V = np.concatenate([to_np(pv)[sel], to_np(v)], axis=1)
    ok, st = ora.compare(to_np(out), ora.prefill_prefix(q_o, K, V, scale, causal=causal))
    print(f"[parity] prefill_dense_append_rope S={S} R={R} P={P} causal={causal} vs oracle {st}", flush=True)
    assert ok, st
    # the pool: rows first..n-1 as the producers give them, every other slot still NaN
    kp, vp = _pool_rows(to_np(kc), bt, n, page), _pool_rows(to_np(vc), bt, n, page)
    assert np.isnan(kp[:, :first]).all() and np.isnan(vp[:, :first]).all()
    assert np.array_equal(kp[:, first:P], K[:, first:P]) and np.array_equal(vp[:, first:], V[:, first:])
    _assert_last_bit(kp[:, max(first, P):], k_o, "pool new K rows vs oracle producers")
    written = np.zeros(kc.shape[:2], dtype=bool)
    j = np.arange(first, n)
    written[bt[:, j // page], j % page] = True
    assert torch.isnan(kc[torch.from_numpy(~written).to(dev)]).all()
    assert torch.isnan(vc[torch.from_numpy(~written).to(dev)]).all()


@pytest.mark.parametrize("P", [35, 200])
def test_dense_append_rope_matches_torch_producers(cuda_device, P):
    """The engine's own sequence on the GPU: eager torch producers, torch.cat, then prefill_dense_append (the fused
    scatters + attention); the one-call form agrees up to rare last-bit differences of the normalised rows."""
    dev = cuda_device
    S, R = 8, 42
    n = P + R
    qkv, pk, pv, qn, kn, cos, sin = _inputs(dev, S, R, P, S, seed=43)
    q, k, v = _views(qkv)
    Pn = -(-n // 16)
    bt = torch.from_numpy(_table(S, Pn, 256, seed=44)).to(dev)
    pools = [torch.zeros(256, 16, 8, D, dtype=torch.bfloat16, device=dev) for _ in range(4)]
    scale = D ** -0.5
    out = q3attn.prefill_dense_append_rope(q, k, v, pk, pv, qn, kn, cos, sin, pools[0], pools[1], bt, scale)
    c4, s4 = cos[None, :, None], sin[None, :, None]
    qe = _eager_norm_rope_torch(q, qn, c4, s4)
    K = torch.cat((pk, _eager_norm_rope_torch(k, kn, c4, s4)), 1)
    V = torch.cat((pv, v), 1)
    ref = q3attn.prefill_dense_append(qe, K, V, pools[2], pools[3], bt, scale, True, 0)
    torch.cuda.synchronize()
    _assert_last_bit(to_np(pools[0]), to_np(pools[2]), f"pool K, P={P}")
    assert torch.equal(pools[1], pools[3])
    ok, st = ora.compare(to_np(out), to_np(ref), max_abs=2e-2, mean_abs=2e-4)
    print(f"[parity] rope form vs torch producers + dense append, P={P}: {st}", flush=True)
    assert ok, st


def test_dense_append_rope_invalid_prefix_index_reads_zeros(cuda_device):
    """A prefix index outside [0, num_prefixes) contributes zero rows (no fault), like an empty voice."""
    dev = cuda_device
    S, R, P = 2, 42, 35
    qkv, pk, pv, qn, kn, cos, sin = _inputs(dev, S, R, P, 2, seed=45)
    q, k, v = _views(qkv)
    pidx = torch.tensor([1, 7], dtype=torch.int64, device=dev)
    bt = torch.from_numpy(_table(S, 5, 64, seed=46)).to(dev)
    kc = torch.full((64, 16, 8, D), float("nan"), dtype=torch.bfloat16, device=dev)
    vc = torch.full_like(kc, float("nan"))
    q3attn.prefill_dense_append_rope(q, k, v, pk, pv, qn, kn, cos, sin, kc, vc, bt, D ** -0.5, pidx)
    torch.cuda.synchronize()
    kp = _pool_rows(to_np(kc), bt.cpu().numpy(), P + R, 16)
    assert np.array_equal(kp[0, :P], to_np(pk)[1]) and not np.abs(kp[1, :P]).any()


def test_dense_append_rope_in_graph_replays(cuda_device):
    dev = cuda_device
    S, R, P = 8, 42, 35
    qkv, pk, pv, qn, kn, cos, sin = _inputs(dev, S, R, P, 4, seed=47)
    q, k, v = _views(qkv)
    pidx = torch.tensor([s % 4 for s in range(S)], dtype=torch.int64, device=dev)
    bt = torch.from_numpy(_table(S, 5, 128, seed=48)).to(dev)
    kc = torch.zeros(128, 16, 8, D, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    eager = q3attn.prefill_dense_append_rope(q, k, v, pk, pv, qn, kn, cos, sin, kc, vc, bt, D ** -0.5, pidx)
    torch.cuda.synchronize()
    k_ref, v_ref = kc.clone(), vc.clone()
    s = torch.cuda.Stream(dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        static = q3attn.prefill_dense_append_rope(q, k, v, pk, pv, qn, kn, cos, sin, kc, vc, bt, D ** -0.5, pidx)
    for _ in range(3):
        kc.fill_(float("nan"))
        vc.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(static, eager)
        assert torch.equal(torch.nan_to_num(kc), torch.nan_to_num(k_ref))
        assert torch.equal(torch.nan_to_num(vc), torch.nan_to_num(v_ref))


# ------------------------------------------------------------------ the talker's prompt step (engine/talker.py:157-169)
def _prompt_inputs(dev, lens, seed):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    T = int(lens.sum())
    qkv = torch.randn((T, 4096), generator=g, device=dev).to(torch.bfloat16)
    qn = (1.0 + 0.1 * torch.randn(D, generator=g, device=dev)).to(torch.bfloat16)
    kn = (1.0 + 0.1 * torch.randn(D, generator=g, device=dev)).to(torch.bfloat16)
    pos = torch.cat([torch.arange(int(L), device=dev) for L in lens])
    cos, sin = W.rope_tables(int(lens.max()), dev)
    # gathered per token as engine/talker.py:154 does: [T, 1, D]
    cos_t, sin_t = cos.to(torch.bfloat16)[pos][:, None, :], sin.to(torch.bfloat16)[pos][:, None, :]
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32, device=dev)
    q, k, v = qkv[:, :2048].view(T, 16, D), qkv[:, 2048:3072].view(T, 8, D), qkv[:, 3072:].view(T, 8, D)
    return q, k, v, qn, kn, cos_t, sin_t, cu


@pytest.mark.parametrize("lens", [[1, 7, 16, 33, 150, 400], "prefill32", [300, 5], "70seqs"])
def test_prompt_step_rope_matches_oracle(cuda_device, lens):
    """"70seqs": more sequences than one 64-lane load of cu_seqlens holds (the producer's search loops over them),
    with empty sequences among them."""
    dev = cuda_device
    if lens == "prefill32":
        lens = W.prefill_lengths("prefill32")
    elif lens == "70seqs":
        lens = np.random.default_rng(7).integers(0, 40, size=70)
        lens[[3, 64, 65]] = 0
        lens[-1] = 97
    else:
        lens = np.array(lens)
    q, k, v, qn, kn, cos_t, sin_t, cu = _prompt_inputs(dev, lens, seed=50 + len(lens))
    n, page = len(lens), 16
    Pn = int(-(-lens.max() // page))
    num_pages = max(2 * n * Pn, 64)
    bt = _table(n, Pn, num_pages, seed=51)
    kc = torch.full((num_pages, page, 8, D), float("nan"), dtype=torch.bfloat16, device=dev)
    vc = torch.full_like(kc, float("nan"))
    scale = D ** -0.5
    print(f"[case] prefill_append_rope {n} sequences, {int(lens.sum())} tokens", flush=True)
    out = q3attn.prefill_append_rope(q, k, v, qn, kn, cos_t, sin_t, cu, int(lens.max()), kc, vc,
                                     torch.from_numpy(bt).to(dev), scale)
    torch.cuda.synchronize()
    cn, sn = to_np(cos_t), to_np(sin_t)
    q_o = _eager_norm_rope_np(to_np(q), to_np(qn), cn, sn)
    k_o = _eager_norm_rope_np(to_np(k), to_np(kn), cn, sn)
    cu_np = cu.cpu().numpy()
    ok, st = ora.compare(to_np(out), ora.prefill_varlen(q_o, k_o, to_np(v), cu_np, scale))
    print(f"[parity] prefill_append_rope {n} sequences vs oracle {st}", flush=True)
    assert ok, st
    # every token's K (normalised) and V rows at its position; no other slot written
    kcn, vcn = to_np(kc), to_np(vc)
    rows = np.concatenate([np.arange(L) for L in lens])
    seq = np.repeat(np.arange(n), lens)
    pages, offs = bt[seq, rows // page], rows % page
    assert np.array_equal(vcn[pages, offs], to_np(v))
    _assert_last_bit(kcn[pages, offs], k_o, f"prompt pool K rows, {n} sequences")
    written = np.zeros(kc.shape[:2], dtype=bool)
    written[pages, offs] = True
    assert np.isnan(kcn[~written]).all() and np.isnan(vcn[~written]).all()


@pytest.mark.parametrize("causal", [True, False])
def test_prompt_step_rope_matches_torch_producers(cuda_device, causal):
    """The talker's own sequence on the GPU (engine/talker.py:157-169): eager torch producers, then prefill_append
    (the fused scatters + attention).  Causal, q is normalised inside the attention kernel; otherwise by the
    producer pass with k."""
    dev = cuda_device
    lens = W.prefill_lengths("prefill32")
    q, k, v, qn, kn, cos_t, sin_t, cu = _prompt_inputs(dev, lens, seed=52)
    n = len(lens)
    Pn = int(-(-lens.max() // 16))
    bt = torch.from_numpy(_table(n, Pn, 2 * n * Pn, seed=53)).to(dev)
    pools = [torch.zeros(2 * n * Pn, 16, 8, D, dtype=torch.bfloat16, device=dev) for _ in range(4)]
    scale = D ** -0.5
    L = int(lens.max())
    print(f"[case] prefill_append_rope vs torch producers, causal={causal}", flush=True)
    out = q3attn.prefill_append_rope(q, k, v, qn, kn, cos_t, sin_t, cu, L, pools[0], pools[1], bt, scale, causal)
    qe = _eager_norm_rope_torch(q, qn, cos_t, sin_t)
    ke = _eager_norm_rope_torch(k, kn, cos_t, sin_t)
    ref = q3attn.prefill_append(qe, ke, v, cu, cu, L, pools[2], pools[3], bt, scale, causal)
    torch.cuda.synchronize()
    _assert_last_bit(to_np(pools[0]), to_np(pools[2]), "prompt pool K vs torch producers")
    assert torch.equal(pools[1], pools[3])
    ok, st = ora.compare(to_np(out), to_np(ref), max_abs=2e-2, mean_abs=2e-4)
    print(f"[parity] prompt rope form vs torch producers + prefill_append: {st}", flush=True)
    assert ok, st


def test_prompt_step_rope_invalid_pages_attend_zero_keys(cuda_device):
    """Causal, the attention reads K back from the pool where the producer pass stored it: a key whose table entry is
    outside [0, num_pages) (-1, num_pages) or past the table (sequence 0 needs 10 pages of a 9-entry table) is not
    stored and attends with zero K, while its V comes from the packed values.  (The engine's index_copy_ would raise
    on such a slot.)  Every other row is stored and attended as usual."""
    dev = cuda_device
    lens = np.array([150, 40, 64])
    q, k, v, qn, kn, cos_t, sin_t, cu = _prompt_inputs(dev, lens, seed=56)
    n, page, Pn, num_pages = len(lens), 16, 9, 64
    bt = _table(n, Pn, num_pages, seed=57)
    bt[0, 3] = -1            # keys 48..63 of sequence 0
    bt[2, 1] = num_pages     # keys 16..31 of sequence 2
    kc = torch.full((num_pages, page, 8, D), float("nan"), dtype=torch.bfloat16, device=dev)
    vc = torch.full_like(kc, float("nan"))
    scale = D ** -0.5
    print(f"[case] prefill_append_rope with invalid table entries, lens {lens.tolist()}", flush=True)
    out = q3attn.prefill_append_rope(q, k, v, qn, kn, cos_t, sin_t, cu, int(lens.max()), kc, vc,
                                     torch.from_numpy(bt).to(dev), scale)
    torch.cuda.synchronize()
    cn, sn = to_np(cos_t), to_np(sin_t)
    q_o = _eager_norm_rope_np(to_np(q), to_np(qn), cn, sn)
    k_o = _eager_norm_rope_np(to_np(k), to_np(kn), cn, sn)
    rows = np.concatenate([np.arange(L) for L in lens])
    seq = np.repeat(np.arange(n), lens)
    pi = rows // page
    page_id = np.where(pi < Pn, bt[seq, np.minimum(pi, Pn - 1)], -1)
    valid = (page_id >= 0) & (page_id < num_pages)
    assert (~valid).sum() == 16 + 6 + 16
    k_eff = np.where(valid[:, None, None], k_o, 0.0).astype(np.float32)
    ok, st = ora.compare(to_np(out), ora.prefill_varlen(q_o, k_eff, to_np(v), cu.cpu().numpy(), scale))
    print(f"[parity] prefill_append_rope, invalid entries, vs oracle with zero keys {st}", flush=True)
    assert ok, st
    kcn, vcn = to_np(kc), to_np(vc)
    pages, offs = page_id[valid], rows[valid] % page
    assert np.array_equal(vcn[pages, offs], to_np(v)[valid])
    _assert_last_bit(kcn[pages, offs], k_o[valid], "pool K rows with valid entries")
    written = np.zeros(kc.shape[:2], dtype=bool)
    written[pages, offs] = True
    assert np.isnan(kcn[~written]).all() and np.isnan(vcn[~written]).all()


def test_prompt_step_rope_in_graph_replays(cuda_device):
    dev = cuda_device
    lens = np.array([150, 33, 260, 1, 97])
    q, k, v, qn, kn, cos_t, sin_t, cu = _prompt_inputs(dev, lens, seed=54)
    Pn = int(-(-lens.max() // 16))
    bt = torch.from_numpy(_table(len(lens), Pn, 128, seed=55)).to(dev)
    kc = torch.zeros(128, 16, 8, D, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    L = int(lens.max())
    eager = q3attn.prefill_append_rope(q, k, v, qn, kn, cos_t, sin_t, cu, L, kc, vc, bt, D ** -0.5)
    torch.cuda.synchronize()
    k_ref, v_ref = kc.clone(), vc.clone()
    s = torch.cuda.Stream(dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        static = q3attn.prefill_append_rope(q, k, v, qn, kn, cos_t, sin_t, cu, L, kc, vc, bt, D ** -0.5)
    for _ in range(3):
        kc.fill_(float("nan"))
        vc.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(static, eager)
        assert torch.equal(torch.nan_to_num(kc), torch.nan_to_num(k_ref))
        assert torch.equal(torch.nan_to_num(vc), torch.nan_to_num(v_ref))
