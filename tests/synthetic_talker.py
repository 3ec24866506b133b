"""Seeded synthetic talker for the code-0 criterion (test infrastructure).

It restates the talker's per-frame decode (engine/talker.py:63-80: qkv projection, qk-RMSNorm, RoPE, K/V
append into the paged pool, attention, o-projection, MLP, final norm), the processed codebook-0 scores with their
per-seat state (``Cb0State``: engine/talker.py:90-94 and 99-101 -- repetition penalty over the seat's own generated
ids, special ids suppressed except EOS, EOS blocked for the first frames) and the top-k sampler (engine/ops.py:68-76)
with random weights of the 0.6B geometry (hidden 1024, 28 layers, 16/8 heads of 128, ffn 3072, 3072 codes).
The attention call is injected so the identical stack runs once with the HIP kernel and once with the
oracle.  The page table is a seeded random permutation of 16-token pages; the append slot goes through it.
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from oracle.torch_cpu import rms, rope  # noqa: F401  (engine/ops.py:51-60; re-exported for the GPU tests)

H, NH, NKV, HD, FFN, VOCAB, PAGE = 1024, 16, 8, 128, 3072, 3072, 16


def sample_topk(logits, temperature, k, gen):
    """engine/ops.py:68-76 (HF order: temperature, top-k, sample)."""
    vals, idx = torch.topk(logits, k, dim=-1)
    p = torch.softmax(vals / temperature, dim=-1)
    j = torch.multinomial(p, 1, generator=gen)
    return idx.gather(1, j).squeeze(1)


class Cb0State:
    """Per-seat sampling state of the talker's codebook-0 head (engine/talker.py:36-45) and the processing of its
    scores (``_cb0_logits``, engine/talker.py:90-94): ids a seat has generated are penalised (negative scores times
    ``rep``, positive ones divided by it), the last 1,024 ids (specials) are suppressed except EOS, and EOS is blocked
    until the seat has generated ``min_new`` codes.  ``update`` records a frame's codes (engine/talker.py:99-101).
    Defaults are the engine's (temperature 0.9, top-k 50, rep 1.05, min_new 2, engine/talker.py:22); EOS is one id
    of the special range, as the codec's is."""

    def __init__(self, seats, device, rep=1.05, min_new=2, eos=VOCAB - 1024 + 126):
        self.rep, self.min_new = rep, min_new
        self.seen = torch.zeros(seats, VOCAB, dtype=torch.bool, device=device)
        self.ngen = torch.zeros(seats, dtype=torch.long, device=device)
        self.suppress = torch.zeros(VOCAB, device=device)
        self.suppress[VOCAB - 1024:] = float("-inf")
        self.suppress[eos] = 0.0
        self.eos_col = torch.zeros(VOCAB, dtype=torch.bool, device=device)
        self.eos_col[eos] = True

    def process(self, lg, seat):
        lg = torch.where(self.seen[seat], torch.where(lg < 0, lg * self.rep, lg / self.rep), lg) + self.suppress
        return lg.masked_fill((self.ngen[seat] < self.min_new)[:, None] & self.eos_col[None, :], float("-inf"))

    def update(self, seat, c0):
        self.seen.index_put_((seat, c0), self.eos_col.new_ones(()).expand_as(c0))
        self.ngen.index_copy_(0, seat, self.ngen[seat] + 1)


class SyntheticTalker:
    def __init__(self, device, layers=28, seed=0, max_pos=1024, dtype=torch.bfloat16, o_gain=4.0):
        """``o_gain`` scales the o-projection's init std.  At 1.0 (the standard 1/sqrt(fan_in)) a random stack's
        residual stream is dominated by the embeddings and MLPs, and attention moves the logits little; at 4.0 the
        attention output carries a large share of each layer's update, so a rounding difference in attention
        reaches the codebook-0 logits at full strength (the harder test of the criterion)."""
        self.device, self.dtype = torch.device(device), dtype
        g = torch.Generator(device=self.device)
        g.manual_seed(seed)

        def w(*shape, std):
            return (torch.randn(*shape, generator=g, device=self.device) * std).to(dtype)

        def norm_w():
            return (1.0 + 0.1 * torch.randn(H, generator=g, device=self.device)).to(dtype)

        def head_norm_w():
            return (1.0 + 0.1 * torch.randn(HD, generator=g, device=self.device)).to(dtype)

        self.layers = []
        for _ in range(layers):
            self.layers.append(dict(
                ln1=norm_w(), ln2=norm_w(), qn=head_norm_w(), kn=head_norm_w(),
                qkv=w((NH + 2 * NKV) * HD, H, std=H ** -0.5),
                o=w(H, NH * HD, std=(NH * HD) ** -0.5 * o_gain),
                gu=w(2 * FFN, H, std=H ** -0.5),
                down=w(H, FFN, std=FFN ** -0.5 * 0.5)))
        self.norm = norm_w()
        self.codec_head = w(VOCAB, H, std=H ** -0.5 * 4)
        self.codec_emb = w(VOCAB, H, std=1.0)
        inv = 1.0 / (1.0e6 ** (torch.arange(0, HD, 2, dtype=torch.float64, device=self.device) / HD))
        ang = torch.arange(max_pos, dtype=torch.float64, device=self.device)[:, None] * inv[None, :]
        emb = torch.cat([ang, ang], -1)
        self.cos, self.sin = emb.cos().to(dtype), emb.sin().to(dtype)
        self.scale = HD ** -0.5

    def new_pools(self, num_pages):
        shape = (num_pages, PAGE, NKV, HD)
        return ([torch.zeros(shape, dtype=self.dtype, device=self.device) for _ in self.layers],
                [torch.zeros(shape, dtype=self.dtype, device=self.device) for _ in self.layers])

    @torch.inference_mode()
    def decode(self, x, pos, bt, kc, vc, attn):
        """x [B, H] bf16, pos [B] int64 (this token's position), bt [B, P] int32 -> post-norm hidden [B, H].
        The token's K/V go to slot bt[b, pos//16]*16 + pos%16 before attention over ctx = pos + 1."""
        B = x.shape[0]
        nq, nk = NH * HD, NKV * HD
        cos, sin = self.cos[pos][:, None, :], self.sin[pos][:, None, :]
        slot = bt.long().gather(1, (pos // PAGE)[:, None])[:, 0] * PAGE + pos % PAGE
        ctx = (pos + 1).to(torch.int32)
        for l, w in enumerate(self.layers):
            qkv = F.linear(rms(x, w["ln1"]), w["qkv"])
            q = rope(rms(qkv[:, :nq].view(B, NH, HD), w["qn"]), cos, sin)
            k = rope(rms(qkv[:, nq:nq + nk].view(B, NKV, HD), w["kn"]), cos, sin)
            v = qkv[:, nq + nk:].view(B, NKV, HD)
            kc[l].view(-1, NKV, HD).index_copy_(0, slot, k)
            vc[l].view(-1, NKV, HD).index_copy_(0, slot, v)
            o = attn(q.contiguous(), kc[l], vc[l], ctx, bt, self.scale)
            x = x + F.linear(o.reshape(B, nq), w["o"])
            gu = F.linear(rms(x, w["ln2"]), w["gu"])
            x = x + F.linear(F.silu(gu[..., :FFN]) * gu[..., FFN:], w["down"])
        return rms(x, self.norm)

    def logits(self, h):
        """Raw codebook-0 scores (engine/talker.py:92), before Cb0State.process."""
        return F.linear(h, self.codec_head).float()


def oracle_attention(q, kc, vc, ctx, bt, scale, acc=np.float32):
    """The oracle's paged decode on host copies of the pages the rows reference, back as bf16 (accumulating in
    ``acc``)."""
    from oracle import attention as ora
    page = kc.shape[1]
    ctx_h = ctx.cpu().numpy().astype(np.int64)
    bt_h = bt.cpu().numpy().astype(np.int64)
    need = np.unique(np.concatenate([bt_h[b, : (c + page - 1) // page] for b, c in enumerate(ctx_h)]))
    remap = np.zeros(int(bt_h.max()) + 1, np.int64)
    remap[need] = np.arange(len(need))
    idx = torch.from_numpy(need).to(kc.device)
    k = kc.index_select(0, idx).float().cpu().numpy()
    v = vc.index_select(0, idx).float().cpu().numpy()
    tab = remap[np.where(bt_h < len(remap), bt_h, 0)]
    out = ora.paged_decode(q.float().cpu().numpy(), k, v, ctx_h, tab, scale, acc=acc)
    return torch.from_numpy(out.astype(np.float32)).to(q.device).to(q.dtype)


def oracle64_attention(q, kc, vc, ctx, bt, scale):
    """The same oracle accumulating in float64: a second correct implementation whose bf16 outputs differ from the
    float32 oracle's only by rounding, so its code-0 disagreement with it is the floor any bf16 kernel meets."""
    return oracle_attention(q, kc, vc, ctx, bt, scale, acc=np.float64)


def torch_bf16_attention(q, kc, vc, ctx, bt, scale):
    """An independent bf16 attention: the reference's torch recipe (engine/code_predictor.py:46-47 applied to
    decode) -- bf16 matmul for the scores, fp32 softmax, probabilities rounded to bf16, bf16 matmul with V --
    one row at a time over its gathered pages.  Operands are made contiguous before each product."""
    B, Hq, D = q.shape
    page, Hkv = kc.shape[1], kc.shape[2]
    out = torch.zeros_like(q)
    for b in range(B):
        c = int(ctx[b])
        if c <= 0:
            continue
        npg = (c + page - 1) // page
        pages = bt[b, :npg].long()
        K = kc[pages].reshape(npg * page, Hkv, D)[:c].transpose(0, 1).contiguous()      # [Hkv, c, D]
        V = vc[pages].reshape(npg * page, Hkv, D)[:c].transpose(0, 1).contiguous()
        Kt = K.transpose(1, 2).contiguous()                                               # [Hkv, D, c]
        att = torch.matmul(q[b].view(Hkv, Hq // Hkv, D).contiguous(), Kt) * scale
        p = torch.softmax(att.float(), dim=-1).to(q.dtype)
        out[b] = torch.matmul(p, V).reshape(Hq, D)
    return out
