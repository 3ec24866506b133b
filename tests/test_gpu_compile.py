"""The ops inside torch.compile(dynamic=False) and HIP-graph capture, the way the reference runs its attention.

The talker compiles its per-frame decode, K/V scatters included (engine/talker.py:56-59, 63-77), and captures the
compiled frame into a graph on a side stream (engine/talker.py:115-129); the code predictor compiles _pre/_post around
an eager slot write (engine/code_predictor.py:25-29, 52-60).  The ops are opaque custom ops with fake implementations;
the mutating ones (the fused append forms) declare the pool/scratch they write.  These tests check that:
  * a compiled call's result matches the oracle and its writes land in the caller's pool tensor (no copy);
  * the compiled call allocates far less than the pool it mutates, so the mutation is not functionalised into a
    clone of the pool or scratch (engine/code_predictor.py:73-74 measured that cost for an in-graph index_copy_),
    and the generated code allocates no buffer of the pool's size;
  * a graph captured from the compiled function replays bit for bit equal to the compiled eager call.
The reference's own in-graph index_copy_ scatters (engine/talker.py:72-73 inside the compiled _decode) are lowered by
inductor into a copy of the whole pool and a copy back; the first test measures and prints that, the fused form's
test shows the op that replaces them adds none.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import q3attn
from helpers import to_np
from oracle import attention as ora
from synthetic_talker import rms, rope
from test_gpu_reference_layouts import HD, NH, NK, NKV, NQ, SCALE, Proj, check, rope_bf16

pytestmark = pytest.mark.gpu

NUM_PAGES, PAGE = 4096, 16           # 128 MiB per pool


def _pools(dev, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    kc = torch.randn(NUM_PAGES, PAGE, NKV, HD, generator=g, device=dev).to(torch.bfloat16)
    vc = torch.randn(NUM_PAGES, PAGE, NKV, HD, generator=g, device=dev).to(torch.bfloat16)
    return kc, vc


def _frame_inputs(dev, B, seed):
    rng = np.random.default_rng(seed)
    P = 64
    bt = torch.from_numpy(rng.permutation(NUM_PAGES)[: B * P].reshape(B, P).astype(np.int32)).to(dev)
    pos = torch.from_numpy(rng.integers(0, P * PAGE - 1, size=B)).to(dev)
    pos[0] = 0
    slot = (bt.gather(1, (pos // PAGE)[:, None].to(torch.int64))[:, 0].to(torch.int64) * PAGE + pos % PAGE)
    g = torch.Generator(device=dev).manual_seed(seed)
    x = torch.randn(B, 1024, generator=g, device=dev).to(torch.bfloat16)
    return x, pos, slot, (pos + 1).to(torch.int32), bt


def _peak_delta(fn):
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    out = fn()
    torch.cuda.synchronize()
    return out, torch.cuda.max_memory_allocated() - base


def _capture(fn, dev):
    """Warm on a side stream, capture there, as engine/talker.py:115-129 does."""
    s = torch.cuda.Stream(dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        for _ in range(3):
            fn()
    torch.cuda.current_stream(dev).wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        static = fn()
    return g, static


def _big_allocations(codes, min_numel):
    """Allocations of at least min_numel elements in the compiled module's call path.  The module's trailing
    benchmark harness (benchmark_compiled_module) builds random inputs of every graph input's shape, so only the
    code before it is searched."""
    import re

    found = []
    for code in codes:
        body = code.split("def benchmark_compiled_module")[0]
        for m in re.finditer(r"empty_strided\w*\(\(([\d, ]*)\)", body):
            dims = [int(d) for d in m.group(1).split(",") if d.strip()]
            if int(np.prod(dims)) >= min_numel:
                found.append(m.group(0))
    return found


def test_compiled_decode_plain_form(cuda_device):
    """One layer of Talker._decode compiled whole, as the reference writes it: projection, the two index_copy_ scatters
    and the flash_attn_with_kvcache call (engine/talker.py:66-77).  The attention op itself mutates nothing and adds no
    pool-sized buffer; the in-graph index_copy_ scatters are functionalised by inductor into a copy of each pool (this
    is the reference's own pattern, measured and printed here; the fused append form below avoids it)."""
    from torch._inductor.utils import run_and_get_code

    dev = cuda_device
    torch._dynamo.reset()
    kc, vc = _pools(dev, 1)
    proj = Proj(dev, 2)
    cos_t, sin_t = rope_bf16(64 * PAGE, dev)
    B = 24
    x, pos, slot, ctx, bt = _frame_inputs(dev, B, 3)
    cos, sin = cos_t[pos][:, None, :], sin_t[pos][:, None, :]

    def layer(x, cos, sin, slot, ctx, bt):
        q, k, v = proj(x, cos, sin)
        kc.view(-1, NKV, HD).index_copy_(0, slot, k)
        vc.view(-1, NKV, HD).index_copy_(0, slot, v)
        o = q3attn.flash_attn_with_kvcache(q.unsqueeze(1), kc, vc, cache_seqlens=ctx, block_table=bt,
                                           softmax_scale=SCALE, causal=True)
        return o, q, k, v

    step = torch.compile(layer, dynamic=False)
    (o, q, k, v), codes = run_and_get_code(step, x, cos, sin, slot, ctx, bt)
    torch.cuda.synchronize()
    print(f"[compile] decode plain (in-graph index_copy_): pool-sized buffers {_big_allocations(codes, kc.numel())}",
          flush=True)
    assert torch.equal(kc.view(-1, NKV, HD)[slot], k) and torch.equal(vc.view(-1, NKV, HD)[slot], v)
    ref = ora.paged_decode(to_np(q), to_np(kc), to_np(vc), ctx.cpu().numpy(), bt.cpu().numpy(), SCALE)
    check(o[:, 0], ref, "compiled decode")
    (o2, *_), delta = _peak_delta(lambda: step(x, cos, sin, slot, ctx, bt))
    print(f"[compile] decode plain (in-graph index_copy_): peak allocation {delta / 2**20:.1f} MiB "
          f"(pool {kc.numel() * 2 / 2**20:.0f} MiB)", flush=True)
    assert torch.equal(o2, o)

    # the attention op alone, compiled with the scatters left eager (engine/code_predictor.py:73-74's structure)
    def attend(q, ctx, bt):
        return q3attn.flash_attn_with_kvcache(q.unsqueeze(1), kc, vc, cache_seqlens=ctx, block_table=bt,
                                              softmax_scale=SCALE, causal=True)

    catt = torch.compile(attend, dynamic=False)
    o3, codes = run_and_get_code(catt, q, ctx, bt)
    assert not _big_allocations(codes, kc.numel() // 4)
    assert torch.equal(o3, o)
    o4, delta = _peak_delta(lambda: catt(q, ctx, bt))
    print(f"[compile] decode attention op alone: peak allocation {delta / 2**20:.1f} MiB", flush=True)
    assert delta < kc.numel() * 2 // 16
    g, static = _capture(lambda: catt(q, ctx, bt), dev)
    for _ in range(3):
        torch.randn(1 << 18, device=dev)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(static, o)


def test_compiled_decode_with_a_plan(cuda_device):
    """The frame's plan built outside the compiled layers and passed in as scheduler_metadata (the way flash-attn 3's
    get_scheduler_metadata is used): two compiled layer calls sharing the plan equal the eager planned calls bit for
    bit and the oracle, the compiled module allocates nothing of the plan's size (the op declares no mutation of it:
    it only uses the buffer behind the plan as scratch within a call), and a graph of the plan launch and the compiled
    layers replays bit for bit."""
    from torch._inductor.utils import run_and_get_code

    dev = cuda_device
    torch._dynamo.reset()
    kc, vc = _pools(dev, 7)
    B, P = 80, 32                      # 80 rows of 512-token tables: the library decodes them with stream-K
    rng = np.random.default_rng(8)
    bt = torch.from_numpy(rng.permutation(NUM_PAGES)[: B * P].reshape(B, P).astype(np.int32)).to(dev)
    ctx = torch.from_numpy(rng.integers(1, P * PAGE + 1, B).astype(np.int32)).to(dev)
    g = torch.Generator(device=dev).manual_seed(9)
    q1 = torch.randn(B, NH, HD, generator=g, device=dev).to(torch.bfloat16)
    q2 = torch.randn(B, NH, HD, generator=g, device=dev).to(torch.bfloat16)

    def two_layers(q1, q2, ctx, bt, plan):
        o1 = q3attn.flash_attn_with_kvcache(q1.unsqueeze(1), kc, vc, cache_seqlens=ctx, block_table=bt,
                                            softmax_scale=SCALE, causal=True, scheduler_metadata=plan)
        o2 = q3attn.flash_attn_with_kvcache(q2.unsqueeze(1), kc, vc, cache_seqlens=ctx, block_table=bt,
                                            softmax_scale=SCALE, causal=True, scheduler_metadata=plan)
        return o1, o2

    plan = q3attn.decode_plan(ctx, bt, PAGE)
    assert plan is not None
    step = torch.compile(two_layers, dynamic=False)
    (o1, o2), codes = run_and_get_code(step, q1, q2, ctx, bt, plan)
    e1, e2 = two_layers(q1, q2, ctx, bt, plan)
    torch.cuda.synchronize()
    assert torch.equal(o1, e1) and torch.equal(o2, e2)
    assert not _big_allocations(codes, plan.numel() // 8)
    ref = ora.paged_decode(to_np(q1), to_np(kc), to_np(vc), ctx.cpu().numpy(), bt.cpu().numpy(), SCALE)
    check(o1[:, 0], ref, "compiled planned decode")
    gr, static = _capture(lambda: step(q1, q2, ctx, bt, q3attn.decode_plan(ctx, bt, PAGE)), dev)
    for _ in range(3):
        torch.randn(1 << 18, device=dev)
        gr.replay()
        torch.cuda.synchronize()
        assert torch.equal(static[0], o1) and torch.equal(static[1], o2)


def test_compiled_decode_append_form(cuda_device):
    """The same layer with the scatters folded into the call (flash-attn's k=/v= form): compiled, the op mutates the
    caller's pools in place; bitwise equal to index_copy_ + decode on the same q/k/v."""
    from torch._inductor.utils import run_and_get_code

    dev = cuda_device
    torch._dynamo.reset()
    kc, vc = _pools(dev, 4)
    kc_ref, vc_ref = kc.clone(), vc.clone()
    proj = Proj(dev, 5)
    cos_t, sin_t = rope_bf16(64 * PAGE, dev)
    B = 24
    x, pos, slot, ctx, bt = _frame_inputs(dev, B, 6)
    cos, sin = cos_t[pos][:, None, :], sin_t[pos][:, None, :]

    def layer(x, cos, sin, ctx, bt):
        q, k, v = proj(x, cos, sin)
        o = q3attn.flash_attn_with_kvcache(q.unsqueeze(1), kc, vc, k=k.unsqueeze(1), v=v.unsqueeze(1),
                                           cache_seqlens=ctx - 1, block_table=bt, softmax_scale=SCALE, causal=True)
        return o, q, k, v

    step = torch.compile(layer, dynamic=False)
    (o, q, k, v), codes = run_and_get_code(step, x, cos, sin, ctx, bt)
    torch.cuda.synchronize()
    assert not _big_allocations(codes, kc.numel() // 4), "the fused append op must not be functionalised into a copy"
    kc_ref.view(-1, NKV, HD).index_copy_(0, slot, k)
    vc_ref.view(-1, NKV, HD).index_copy_(0, slot, v)
    assert torch.equal(kc, kc_ref) and torch.equal(vc, vc_ref), "the compiled op must write the caller's pools"
    eager = q3attn.flash_attn_with_kvcache(q.unsqueeze(1), kc_ref, vc_ref, cache_seqlens=ctx, block_table=bt,
                                           softmax_scale=SCALE, causal=True)
    assert torch.equal(o, eager)
    (o2, *_), delta = _peak_delta(lambda: step(x, cos, sin, ctx, bt))
    print(f"[compile] decode append: peak allocation {delta / 2**20:.1f} MiB (pool {kc.numel() * 2 / 2**20:.0f} MiB)",
          flush=True)
    assert delta < kc.numel() * 2 // 4
    assert torch.equal(o2, o)
    g, static = _capture(lambda: step(x, cos, sin, ctx, bt), dev)
    for _ in range(3):
        kc.view(-1, NKV, HD)[slot] = float("nan")          # the replay must rewrite the slots
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(static[0], o)
        assert torch.equal(kc, kc_ref)


def test_compiled_code_predictor_post_with_fused_slot_write(cuda_device):
    """A _post-style compiled function (engine/code_predictor.py:44-50) that takes the step's q/k/v and the scratch
    slices K = self.K[l, :B], V = self.V[l, :B] and calls cp_attn_append (slot write + attention) before the
    o-projection.  The scratch is mutated in place (no functionalised copy of it)."""
    from torch._inductor.utils import run_and_get_code

    dev = cuda_device
    torch._dynamo.reset()
    L, max_bs, B = 5, 512, 400
    Ks = torch.zeros(L, max_bs, NKV, 16, HD, dtype=torch.bfloat16, device=dev)
    Vs = torch.zeros_like(Ks)
    g = torch.Generator(device=dev).manual_seed(8)
    o_w = (torch.randn(1024, NQ, generator=g, device=dev) * NQ ** -0.5).to(torch.bfloat16)
    proj = Proj(dev, 9)
    cos_t, sin_t = rope_bf16(16, dev)

    def post(x, q, k, v, K, V, p: int):
        o = q3attn.cp_attn_append(q, k, v, K, V, p, SCALE)
        return x + F.linear(o, o_w), o

    cpost = torch.compile(post, dynamic=False)
    for p in (0, 5, 15):
        x = torch.randn(B, 1024, generator=g, device=dev).to(torch.bfloat16)
        q, k, v = proj(x, cos_t[p], sin_t[p])
        l = p % L
        K, V = Ks[l, :B], Vs[l, :B]
        before_k, before_v = Ks.clone(), Vs.clone()
        (y, o), codes = run_and_get_code(cpost, x, q, k, v, K, V, p)
        torch.cuda.synchronize()
        assert not _big_allocations(codes, K.numel() // 4), "cp_attn_append must not copy the scratch"
        assert torch.equal(Ks[l, :B, :, p], k) and torch.equal(Vs[l, :B, :, p], v)
        before_k[l, :B, :, p] = k
        before_v[l, :B, :, p] = v
        assert torch.equal(Ks, before_k) and torch.equal(Vs, before_v)
        check(o, ora.cp_attn_triton_path(to_np(q), to_np(K), to_np(V), p + 1, SCALE), f"compiled cp p={p}")
        (y2, o2), delta = _peak_delta(lambda: cpost(x, q, k, v, K, V, p))
        print(f"[compile] cp post p={p}: peak allocation {delta / 2**20:.2f} MiB "
              f"(scratch slice {K.numel() * 2 / 2**20:.1f} MiB)", flush=True)
        assert delta < K.numel() * 2 // 4
        assert torch.equal(o2, o) and torch.equal(y2, y)
        gr, static = _capture(lambda: cpost(x, q, k, v, K, V, p), dev)
        for _ in range(2):
            Ks[l, :B, :, p] = float("nan")
            gr.replay()
            torch.cuda.synchronize()
            assert torch.equal(static[1], o) and torch.equal(static[0], y)
            assert torch.equal(Ks[l, :B, :, p], k)


def test_compiled_decode_rope_form(cuda_device):
    """engine/talker.py:66-77 with the q/k producers, the scatters and the attention in paged_decode_append_rope: the
    compiled layer projects, then hands the raw q/k/v views of the projection to the op.  The op writes the caller's
    pools in place (no pool-sized buffer); the output is within the parity bar of the oracle fed with the reference's
    own producers (engine/ops.py:51-60 via the test's restatement), the written k rows within the rounding bound of
    those producers, and a graph captured from the compiled function replays bit for bit."""
    from torch._inductor.utils import run_and_get_code

    dev = cuda_device
    torch._dynamo.reset()
    kc, vc = _pools(dev, 10)
    kc_before = kc.clone()
    proj = Proj(dev, 11)
    cos_t, sin_t = rope_bf16(64 * PAGE, dev)
    B = 24
    x, pos, slot, ctx, bt = _frame_inputs(dev, B, 12)
    cos, sin = cos_t[pos][:, None, :], sin_t[pos][:, None, :]

    def layer(x, cos, sin, ctx, bt):
        qkv = F.linear(rms(x, proj.ln1), proj.qkv)
        o = q3attn.paged_decode_append_rope(qkv[:, :NQ].view(B, NH, HD), qkv[:, NQ:NQ + NK].view(B, NKV, HD),
                                            qkv[:, NQ + NK:].view(B, NKV, HD), proj.qn, proj.kn, cos, sin, kc, vc,
                                            ctx - 1, bt, SCALE)
        return o, qkv

    step = torch.compile(layer, dynamic=False)
    (o, qkv), codes = run_and_get_code(step, x, cos, sin, ctx, bt)
    torch.cuda.synchronize()
    assert not _big_allocations(codes, kc.numel() // 4), "the fused op must not be functionalised into a copy"
    # the reference's producers (engine/ops.py:51-60 as eager torch ops) on the compiled layer's own projection
    q_ref = rope(rms(qkv[:, :NQ].view(B, NH, HD), proj.qn), cos, sin)
    k_ref = rope(rms(qkv[:, NQ:NQ + NK].view(B, NKV, HD), proj.kn), cos, sin)
    v_ref = qkv[:, NQ + NK:].view(B, NKV, HD)
    assert torch.equal(vc.view(-1, NKV, HD)[slot], v_ref), "v rows must be stored as given"
    got_k = kc.view(-1, NKV, HD)[slot].float()
    dk = (got_k - k_ref.float()).abs()
    assert bool((dk <= k_ref.float().abs() * 2.0 ** -6 + 2.0 ** -6).all()), float(dk.max())
    untouched = torch.ones(NUM_PAGES * PAGE, dtype=torch.bool, device=dev)
    untouched[slot] = False
    assert torch.equal(kc.view(-1, NKV, HD)[untouched], kc_before.view(-1, NKV, HD)[untouched])
    kc_ref = kc.clone()
    kc_ref.view(-1, NKV, HD)[slot] = k_ref
    ref = ora.paged_decode(to_np(q_ref), to_np(kc_ref), to_np(vc), ctx.cpu().numpy(), bt.cpu().numpy(), SCALE)
    check(o, ref, "compiled norm/rope decode")
    (o2, _), delta = _peak_delta(lambda: step(x, cos, sin, ctx, bt))
    print(f"[compile] decode norm/rope: peak allocation {delta / 2**20:.1f} MiB (pool {kc.numel() * 2 / 2**20:.0f} MiB)",
          flush=True)
    assert delta < kc.numel() * 2 // 4
    assert torch.equal(o2, o)
    pool = kc.clone()
    g, static = _capture(lambda: step(x, cos, sin, ctx, bt), dev)
    for _ in range(3):
        kc.view(-1, NKV, HD)[slot] = float("nan")          # the replay must rewrite the slots
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(static[0], o)
        assert torch.equal(kc, pool)


def test_compiled_code_predictor_step_with_fused_producers(cuda_device):
    """The code-predictor step with _pre's producers folded in (engine/code_predictor.py:38-47, 58): a compiled
    function takes the raw qkv projection, calls cp_attn_append_rope on its views (q/k norm + RoPE, slot write,
    attention) and applies the o-projection.  Compiled, the call mutates the scratch slice in place (no
    functionalised copy), its output matches the eager op's bit for bit and it replays from a graph."""
    from torch._inductor.utils import run_and_get_code

    dev = cuda_device
    torch._dynamo.reset()
    L, max_bs, B = 5, 512, 400
    Ks = torch.zeros(L, max_bs, NKV, 16, HD, dtype=torch.bfloat16, device=dev)
    Vs = torch.zeros_like(Ks)
    g = torch.Generator(device=dev).manual_seed(10)
    qkv_w = (torch.randn(4096, 1024, generator=g, device=dev) * 1024 ** -0.5).to(torch.bfloat16)
    o_w = (torch.randn(1024, NQ, generator=g, device=dev) * NQ ** -0.5).to(torch.bfloat16)
    qn = (1.0 + 0.1 * torch.randn(HD, generator=g, device=dev)).to(torch.bfloat16)
    kn = (1.0 + 0.1 * torch.randn(HD, generator=g, device=dev)).to(torch.bfloat16)
    cos_t, sin_t = rope_bf16(16, dev)

    def step(x, K, V, c, s, p: int):
        qkv = F.linear(x, qkv_w)
        o = q3attn.cp_attn_append_rope(qkv[:, :NQ].view(-1, 16, HD), qkv[:, NQ:NQ + 1024].view(-1, NKV, HD),
                                       qkv[:, NQ + 1024:].view(-1, NKV, HD), K, V, p, SCALE, qn, kn, c, s)
        return x + F.linear(o, o_w), o

    cstep = torch.compile(step, dynamic=False)
    for p in (0, 5, 15):
        x = torch.randn(B, 1024, generator=g, device=dev).to(torch.bfloat16)
        l = p % L
        K, V = Ks[l, :B], Vs[l, :B]
        Ke, Ve = K.clone(), V.clone()
        y_e, o_e = step(x, Ke, Ve, cos_t[p], sin_t[p], p)          # eager reference on copies of the slices
        (y, o), codes = run_and_get_code(cstep, x, K, V, cos_t[p], sin_t[p], p)
        torch.cuda.synchronize()
        # the qkv projection's own output (B x 4096) is a quarter of the slice; a copy of the slice would be all of it
        assert not _big_allocations(codes, K.numel() // 2), "cp_attn_append_rope must not copy the scratch"
        assert torch.equal(o, o_e)                       # the op's output, bit for bit
        # the compiled o-projection + residual rounds its fused add differently from eager addmm: torch's own numerics
        assert torch.allclose(y.float(), y_e.float(), atol=3e-2, rtol=1e-2)
        assert torch.equal(K, Ke) and torch.equal(V, Ve)
        gr, static = _capture(lambda: cstep(x, K, V, cos_t[p], sin_t[p], p), dev)
        for _ in range(2):
            Ks[l, :B, :, p] = float("nan")
            gr.replay()
            torch.cuda.synchronize()
            assert torch.equal(static[1], o) and torch.equal(static[0], y)
            assert torch.equal(K, Ke)
        print(f"[compile] cp step with fused producers p={p}: equal to eager, no scratch copy", flush=True)


def test_compiled_producers_against_fused_norm_rope_rows(cuda_device):
    """The reference's producers compiled as the engine compiles them (rope(rms(k, kn), cos, sin), engine/ops.py:51-60,
    under torch.compile like Talker._decode and CodePredictor._pre) against the k rows the fused norm/rope kernels write
    into the pool (paged_decode_append_rope) and into the CP scratch slot (cp_attn_append_rope).  Inductor keeps the
    whole chain in fp32 (the cast inside rms is not materialised) and rounds once; the kernels evaluate the same chain.
    Printed: the fraction of equal elements for both kernels, and how the compiled producers compare with the chain
    with the cast kept (every intermediate fp32 but n = bf16(x r)) and with the oracle's compiled form (cast
    dropped).  Asserted: every element within the rounding of the two rope products, and all but rare elements (a
    sum of squares taken in another order) equal."""
    dev = cuda_device
    torch._dynamo.reset()
    g = torch.Generator(device=dev).manual_seed(21)
    B = 256
    k_raw = (torch.randn(B, NKV, HD, generator=g, device=dev) *
             (0.2 + 3.0 * torch.rand(B, NKV, 1, generator=g, device=dev))).to(torch.bfloat16)
    q_raw = torch.randn(B, NH, HD, generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn(B, NKV, HD, generator=g, device=dev).to(torch.bfloat16)
    qn = (1.0 + 0.1 * torch.randn(HD, generator=g, device=dev)).to(torch.bfloat16)
    kn = (1.0 + 0.1 * torch.randn(HD, generator=g, device=dev)).to(torch.bfloat16)
    cos_t, sin_t = rope_bf16(1024, dev)
    rng = np.random.default_rng(21)
    pos = torch.from_numpy(rng.integers(0, 255, size=B)).to(dev)
    produce = torch.compile(lambda x, w, c, s: rope(rms(x, w), c, s), dynamic=False)

    # decode: each row's new k goes to position pos of its own 256-token table
    P = 16
    bt = torch.from_numpy(rng.permutation(NUM_PAGES)[: B * P].reshape(B, P).astype(np.int32)).to(dev)
    kc = torch.zeros(NUM_PAGES, PAGE, NKV, HD, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    c, s = cos_t[pos], sin_t[pos]
    q3attn.paged_decode_append_rope(q_raw, k_raw, v, qn, kn, c, s, kc, vc, pos.to(torch.int32), bt, SCALE, 1e-6)
    slot = bt.gather(1, (pos // PAGE)[:, None].to(torch.int64))[:, 0].to(torch.int64) * PAGE + pos % PAGE
    got_dec = kc.view(-1, NKV, HD)[slot]
    want_dec = produce(k_raw, kn, c[:, None, :], s[:, None, :])

    # code predictor: step p's k goes to slot p of every row (cos/sin of position p)
    p = 9
    K = torch.zeros(B, NKV, 16, HD, dtype=torch.bfloat16, device=dev)
    V = torch.zeros_like(K)
    q3attn.cp_attn_append_rope(q_raw, k_raw, v, K, V, p, SCALE, qn, kn, cos_t[p], sin_t[p])
    got_cp = K[:, :, p]
    want_cp = produce(k_raw, kn, cos_t[p], sin_t[p])
    torch.cuda.synchronize()

    xk, w = to_np(k_raw), to_np(kn)
    for name, got, want, cs, sn in (("paged_decode_append_rope", got_dec, want_dec, to_np(c)[:, None], to_np(s)[:, None]),
                                     ("cp_attn_append_rope", got_cp, want_cp, to_np(cos_t[p]), to_np(sin_t[p]))):
        got, want = to_np(got), to_np(want)
        same = float((got == want).mean())
        dropped = ora.norm_rope(xk, w, cs, sn, eager=False)
        xf = xk.astype(np.float32)
        yk = w * ora._normalise(xf, ora._rsqrt_mean_sq(xf, 1e-6))   # the cast kept
        kept = ora.bf16_round(yk * cs + ora._rotate_half(yk) * sn)
        terms = np.abs(yk * cs) + np.abs(ora._rotate_half(yk) * sn)
        d = np.abs(got - want)
        print(f"[compile] {name}: k rows equal to the compiled producers on {same:.4f} of elements (max diff "
              f"{d.max():.3e}); compiled producers equal the cast-kept chain on {float((want == kept).mean()):.4f}, "
              f"the oracle's compiled form (cast dropped) on {float((want == dropped).mean()):.4f}; kernel rows equal "
              f"the oracle's compiled form on {float((got == dropped).mean()):.4f}", flush=True)
        assert (d <= 2.0 ** -7 * terms + 2.0 ** -7 * np.abs(want) + 1e-30).all()
        assert same >= 0.999
