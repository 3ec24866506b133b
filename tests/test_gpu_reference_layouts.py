"""Every drop-in fed exactly as the reference engine feeds it.

The reference builds q/k/v from one fused projection: qkv = linear(rms(x)), q and k through the per-head qk-RMSNorm and
rotate-half RoPE (fresh tensors), v a strided view of qkv (engine/talker.py:66-71, 155-160; engine/arrivals.py:112-118;
engine/code_predictor.py:38-43).  The caches are the reference's own layouts: the talker's pools with 256-token pages
and the identity seat table (engine/talker.py:23-31, 42), the code predictor's [5, max_bs, 8, 16, 128] scratch sliced to
the live batch (engine/code_predictor.py:20-21, 55).  Each call site is reproduced with its own arguments and checked
against the oracle; the fused forms are checked bit for bit against the reference's scatter + attention sequence.
Bar: max-abs 2e-2 and mean-abs 2e-3 against the fp32-softmax oracle on the same bf16 inputs."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import q3attn
from helpers import to_np
from oracle import attention as ora
from synthetic_talker import rms, rope

pytestmark = pytest.mark.gpu

H, NH, NKV, HD = 1024, 16, 8, 128
NQ, NK = NH * HD, NKV * HD
SCALE = HD ** -0.5


class Proj:
    """One layer's qkv projection and qk-norm weights (random, the 0.6B geometry)."""

    def __init__(self, dev, seed):
        g = torch.Generator(device=dev).manual_seed(seed)
        self.ln1 = (1 + 0.1 * torch.randn(H, generator=g, device=dev)).to(torch.bfloat16)
        self.qkv = (torch.randn(NQ + 2 * NK, H, generator=g, device=dev) * H ** -0.5).to(torch.bfloat16)
        self.qn = (1 + 0.1 * torch.randn(HD, generator=g, device=dev)).to(torch.bfloat16)
        self.kn = (1 + 0.1 * torch.randn(HD, generator=g, device=dev)).to(torch.bfloat16)

    def __call__(self, x, cos, sin):
        """engine/talker.py:66-71: q, k fresh from rope(rms(.)), v a view of the projection."""
        lead = x.shape[:-1]
        qkv = F.linear(rms(x, self.ln1), self.qkv)
        q = rope(rms(qkv[..., :NQ].view(*lead, NH, HD), self.qn), cos, sin)
        k = rope(rms(qkv[..., NQ:NQ + NK].view(*lead, NKV, HD), self.kn), cos, sin)
        v = qkv[..., NQ + NK:].view(*lead, NKV, HD)
        return q, k, v


def rope_bf16(n_pos, dev):
    """bf16 cos/sin tables [n_pos, 128] (the talker keeps its tables in the model dtype)."""
    c, s = ora.rope_tables(n_pos)
    return torch.from_numpy(c).to(dev).to(torch.bfloat16), torch.from_numpy(s).to(dev).to(torch.bfloat16)


def check(out, ref, what):
    ok, st = ora.compare(to_np(out), ref)
    print(f"[reference-layout] {what} {st}", flush=True)
    assert ok, (what, st)


def test_talker_decode_reference_pool_and_producers(cuda_device):
    """Talker._frame + _decode (engine/talker.py:107-112, 63-77): 256-token pages, identity seat table, slot =
    seat * seat_len + pos, ctx = pos + 1, two padded rows on the scratch seat at position 0."""
    dev = cuda_device
    n_seats, seat_len, page = 6, 768, 256
    P = seat_len // page
    S1 = n_seats + 1
    kc = torch.zeros(S1 * P, page, NKV, HD, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    seat_pages = (torch.arange(S1, dtype=torch.int32, device=dev)[:, None] * P
                  + torch.arange(P, dtype=torch.int32, device=dev)[None, :]).contiguous()
    g = torch.Generator(device=dev).manual_seed(1)
    # history already in the seats (what earlier frames wrote)
    kc.normal_(generator=g)
    vc.normal_(generator=g)
    cos_t, sin_t = rope_bf16(seat_len, dev)
    proj = Proj(dev, 2)
    seat = torch.tensor([3, 0, 5, 1, n_seats, n_seats], device=dev)
    pos = torch.tensor([700, 0, 255, 256, 0, 0], device=dev)
    B = seat.shape[0]
    x = torch.randn(B, H, generator=g, device=dev).to(torch.bfloat16)
    q, k, v = proj(x, cos_t[pos][:, None, :], sin_t[pos][:, None, :])
    assert v.stride(0) == NQ + 2 * NK and k.is_contiguous()
    slot = seat * seat_len + pos
    ctx = (pos + 1).to(torch.int32)
    bt = seat_pages[seat]
    kc2, vc2 = kc.clone(), vc.clone()
    # the reference's sequence: two scatters, then the attention call (engine/talker.py:72-77)
    kc.view(-1, NKV, HD).index_copy_(0, slot, k)
    vc.view(-1, NKV, HD).index_copy_(0, slot, v)
    o = q3attn.flash_attn_with_kvcache(q.unsqueeze(1), kc, vc, cache_seqlens=ctx, block_table=bt, softmax_scale=SCALE,
                                       causal=True)
    torch.cuda.synchronize()
    assert o.shape == (B, 1, NH, HD)
    ref = ora.paged_decode(to_np(q), to_np(kc), to_np(vc), ctx.cpu().numpy(), bt.cpu().numpy(), SCALE)
    check(o[:, 0], ref, "talker decode")
    # the fused append form on the pools as they were before the scatters (flash-attn's k=/v= semantics)
    o2 = q3attn.flash_attn_with_kvcache(q.unsqueeze(1), kc2, vc2, k=k.unsqueeze(1), v=v.unsqueeze(1),
                                        cache_seqlens=ctx - 1, block_table=bt, softmax_scale=SCALE, causal=True)
    torch.cuda.synchronize()
    live = slice(0, 4)
    assert torch.equal(o2[live], o[live])
    # the two padded rows share the scratch seat's slot 0: each attends its own new row in the fused form
    for r in (4, 5):
        assert torch.equal(o2[r, 0], v[r].repeat_interleave(2, dim=0))
    keep = torch.ones(kc.shape[0] * page, dtype=torch.bool, device=dev)
    keep[n_seats * seat_len] = False
    assert torch.equal(kc2.view(-1, NKV, HD)[keep], kc.view(-1, NKV, HD)[keep])
    assert torch.equal(vc2.view(-1, NKV, HD)[keep], vc.view(-1, NKV, HD)[keep])
    # both padded rows store into that slot (as both index_copy_ rows do): each element holds one of the two rows
    scratch_k = kc2.view(-1, NKV, HD)[n_seats * seat_len]
    assert ((scratch_k == k[4]) | (scratch_k == k[5])).all()


def test_talker_prefill_reference_producers(cuda_device):
    """Talker.prefill_hidden (engine/talker.py:147-169): k is a fresh [T, 8, 128] tensor (token stride 1024), v a view
    of the [T, 4096] projection (token stride 4096); the call passes them as they are."""
    dev = cuda_device
    lens = [37, 150, 5, 64, 220]
    T = sum(lens)
    g = torch.Generator(device=dev).manual_seed(3)
    x = torch.randn(T, H, generator=g, device=dev).to(torch.bfloat16)
    pos = torch.cat([torch.arange(L, device=dev) for L in lens])
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32, device=dev)
    cos_t, sin_t = rope_bf16(max(lens), dev)
    q, k, v = Proj(dev, 4)(x, cos_t[pos][:, None, :], sin_t[pos][:, None, :])
    assert k.stride() == (NK, HD, 1) and v.stride() == (NQ + 2 * NK, HD, 1)
    o = q3attn.flash_attn_varlen_func(q, k, v, cu_seqlens_q=cu, cu_seqlens_k=cu, max_seqlen_q=max(lens),
                                      max_seqlen_k=max(lens), softmax_scale=SCALE, causal=True)
    torch.cuda.synchronize()
    check(o, ora.prefill_varlen(to_np(q), to_np(k), to_np(v), cu.cpu().numpy(), SCALE), "talker prefill")
    # the same K/V scattered into the reference's pools (engine/talker.py:152, 161-162) and read back through the
    # identity seat table: bitwise the same result
    seat_len, page = 256, 256
    seats = [2, 0, 4, 1, 3]
    kc = torch.full((6, page, NKV, HD), float("nan"), dtype=torch.bfloat16, device=dev)
    vc = torch.full_like(kc, float("nan"))
    slot = torch.cat([s * seat_len + torch.arange(L, device=dev) for s, L in zip(seats, lens)])
    kc.view(-1, NKV, HD).index_copy_(0, slot, k)
    vc.view(-1, NKV, HD).index_copy_(0, slot, v)
    bt = torch.tensor(seats, dtype=torch.int32, device=dev)[:, None].contiguous()
    o2 = q3attn.flash_attn_varlen_func(q, kc, vc, cu, cu, max(lens), max(lens), softmax_scale=SCALE, causal=True,
                                       block_table=bt)
    torch.cuda.synchronize()
    assert torch.equal(o, o2)


def test_admission_prefill_reference_producers(cuda_device):
    """FastAdmit._layer + _run (engine/arrivals.py:112-118, 141-148): K = cat(prefix K of the voice slot, new k),
    V = cat(prefix V, v view); q at the new tokens' positions k..k+R-1; bottom-right causal."""
    dev = cuda_device
    S, R, kpre, voices = 8, 42, 35, 3
    g = torch.Generator(device=dev).manual_seed(5)
    pK = torch.randn(voices, kpre, NKV, HD, generator=g, device=dev).to(torch.bfloat16)
    pV = torch.randn(voices, kpre, NKV, HD, generator=g, device=dev).to(torch.bfloat16)
    slot = torch.tensor([0, 2, 1, 1, 0, 2, 2, 1], device=dev)
    cos_t, sin_t = rope_bf16(kpre + R, dev)
    x = torch.randn(S, R, H, generator=g, device=dev).to(torch.bfloat16)
    q, kk, v = Proj(dev, 6)(x, cos_t[kpre:kpre + R][None, :, None, :], sin_t[kpre:kpre + R][None, :, None, :])
    K, V = torch.cat((pK[slot], kk), 1), torch.cat((pV[slot], v), 1)
    o = q3attn.flash_attn_func(q, K, V, softmax_scale=SCALE, causal=True)
    torch.cuda.synchronize()
    check(o, ora.prefill_prefix(to_np(q), to_np(K), to_np(V), SCALE), "admission prefill")


def test_code_predictor_reference_scratch_and_producers(cuda_device):
    """CodePredictor._s (engine/code_predictor.py:52-60): K = self.K[l, :B] of the [5, max_bs, 8, 16, 128] scratch,
    the slot write K.index_copy_(2, p, k) before each step's attention, 16 steps.  cp_attn is checked against the
    oracle's fp32-score sequence (engine/cp_attn.py:19-30) and cp_attn_append bit for bit against index_copy_ +
    cp_attn, with v a view of the projection."""
    dev = cuda_device
    L, max_bs, B = 5, 64, 48
    Ks = torch.zeros(L, max_bs, NKV, 16, HD, dtype=torch.bfloat16, device=dev)
    Vs = torch.zeros_like(Ks)
    Ks2, Vs2 = Ks.clone(), Vs.clone()
    # stale contents past the live batch and in future slots (the scratch is reused across frames)
    Ks[:, B:] = float("nan")
    Ks2[:, B:] = float("nan")
    cos_t, sin_t = rope_bf16(16, dev)
    projs = [Proj(dev, 10 + l) for l in range(L)]
    g = torch.Generator(device=dev).manual_seed(7)
    for p in range(16):
        pidx = torch.tensor([p], device=dev)
        for l in range(L):
            x = torch.randn(B, H, generator=g, device=dev).to(torch.bfloat16)
            q, k, v = projs[l](x, cos_t[p], sin_t[p])
            K, V = Ks[l, :B], Vs[l, :B]
            K.index_copy_(2, pidx, k.unsqueeze(2))
            V.index_copy_(2, pidx, v.unsqueeze(2))
            o = q3attn.cp_attn(q, K, V, p + 1, SCALE)
            o2 = q3attn.cp_attn_append(q, k, v, Ks2[l, :B], Vs2[l, :B], p, SCALE)
            torch.cuda.synchronize()
            assert torch.equal(o, o2), (p, l)
            if l == 0 or p in (0, 15):
                check(o, ora.cp_attn_triton_path(to_np(q), to_np(K), to_np(V), p + 1, SCALE), f"cp p={p} l={l}")
    assert torch.equal(Ks[:, :B], Ks2[:, :B]) and torch.equal(Vs, Vs2)
    assert torch.isnan(Ks2[:, B:].float()).all()
