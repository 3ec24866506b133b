"""Seeded synthetic code predictor for the CP logit criterion (test infrastructure).

It restates the 16-step, 5-layer code-predictor frame of engine/code_predictor.py:37-82 (qkv projection,
qk-RMSNorm, RoPE at slot p, the slot-p K/V write, attention over slots 0..p, o-projection, MLP, final norm, the 15
codebook heads) with random weights of the 0.6B geometry (hidden 1024, 16/8 heads of 128, ffn 3072, 2048 codes per
codebook, 3072 talker codes for the step-1 embedding).  The slot write + attention is injected, so the identical
stack runs with the HIP kernel, the oracle and the reference's own torch recipe (engine/code_predictor.py:46-47).
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from synthetic_talker import rms, rope

H, NH, NKV, HD, FFN, CPV, TV, STEPS = 1024, 16, 8, 128, 3072, 2048, 3072, 16


class SyntheticCodePredictor:
    def __init__(self, device, layers=5, seed=0, dtype=torch.bfloat16):
        self.device, self.dtype = torch.device(device), dtype
        g = torch.Generator(device=self.device)
        g.manual_seed(seed)

        def w(*shape, std):
            return (torch.randn(*shape, generator=g, device=self.device) * std).to(dtype)

        def norm_w(n):
            return (1.0 + 0.1 * torch.randn(n, generator=g, device=self.device)).to(dtype)

        self.layers = [dict(ln1=norm_w(H), ln2=norm_w(H), qn=norm_w(HD), kn=norm_w(HD),
                            qkv=w((NH + 2 * NKV) * HD, H, std=H ** -0.5),
                            o=w(H, NH * HD, std=(NH * HD) ** -0.5 * 4.0),
                            gu=w(2 * FFN, H, std=H ** -0.5),
                            down=w(H, FFN, std=FFN ** -0.5 * 0.5)) for _ in range(layers)]
        self.norm = norm_w(H)
        self.codec_emb = w(TV, H, std=1.0)                  # talker's codebook-0 embedding (step 1 input)
        self.cp_emb = w(STEPS - 1, CPV, H, std=1.0)         # engine/code_predictor.py:76 (W.cp_emb[i])
        self.cp_head = w(STEPS - 1, CPV, H, std=H ** -0.5 * 4)
        inv = 1.0 / (1.0e6 ** (torch.arange(0, HD, 2, dtype=torch.float64, device=self.device) / HD))
        ang = torch.arange(STEPS, dtype=torch.float64, device=self.device)[:, None] * inv[None, :]
        emb = torch.cat([ang, ang], -1)
        self.cos, self.sin = emb.cos().to(dtype), emb.sin().to(dtype)
        self.scale = HD ** -0.5

    def new_scratch(self, B):
        shape = (len(self.layers), B, NKV, STEPS, HD)
        return torch.zeros(shape, dtype=self.dtype, device=self.device), torch.zeros(shape, dtype=self.dtype, device=self.device)

    @torch.inference_mode()
    def step(self, x, p, K, V, attn):
        """x [B, H] at slot p -> normed hidden [B, H]; attn(q, k, v, K_l, V_l, p) writes slot p and attends over 0..p."""
        B = x.shape[0]
        nq, nk = NH * HD, NKV * HD
        cos, sin = self.cos[p], self.sin[p]
        for l, w in enumerate(self.layers):
            qkv = F.linear(rms(x, w["ln1"]), w["qkv"])
            q = rope(rms(qkv[:, :nq].view(B, NH, HD), w["qn"]), cos, sin)
            k = rope(rms(qkv[:, nq:nq + nk].view(B, NKV, HD), w["kn"]), cos, sin)
            v = qkv[:, nq + nk:].view(B, NKV, HD)
            o = attn(q.contiguous(), k.contiguous(), v, K[l], V[l], p)
            x = x + F.linear(o.reshape(B, nq), w["o"])
            gu = F.linear(rms(x, w["ln2"]), w["gu"])
            x = x + F.linear(F.silu(gu[..., :FFN]) * gu[..., FFN:], w["down"])
        return rms(x, self.norm)

    @torch.inference_mode()
    def frame_logits(self, h, c0, codes, K, V, attn):
        """One frame (engine/code_predictor.py:62-82): h [B, H] talker hidden, c0 [B] codebook-0 ids.  With codes
        [B, 15] the ids fed back after each head are those (teacher forcing); with codes None each head's argmax is
        fed back.  Returns (the 15 logits [B, 15, 2048] float32, the codes fed back [B, 15])."""
        self.step(h, 0, K, V, attn)
        e = self.codec_emb[c0]
        out, fed = [], []
        for i in range(STEPS - 1):
            hid = self.step(e, i + 1, K, V, attn)
            lg = F.linear(hid, self.cp_head[i]).float()
            out.append(lg)
            c = lg.argmax(-1) if codes is None else codes[:, i]
            fed.append(c)
            e = self.cp_emb[i][c]
        return torch.stack(out, 1), torch.stack(fed, 1)


def hip_slot_attn(q, k, v, K, V, p):
    import q3attn
    return q3attn.cp_attn_append(q, k, v, K, V, p, HD ** -0.5)


def _write_slot(k, v, K, V, p):
    K[:, :, p] = k
    V[:, :, p] = v


def oracle_slot_attn(q, k, v, K, V, p):
    """Slot write, then the oracle's fp32-score sequence (engine/cp_attn.py:19-30) on host copies, back as bf16."""
    from oracle import attention as ora
    _write_slot(k, v, K, V, p)
    out = ora.cp_attn_triton_path(q.float().cpu().numpy(), K.float().cpu().numpy(), V.float().cpu().numpy(), p + 1,
                                  HD ** -0.5)
    return torch.from_numpy(np.ascontiguousarray(out)).to(q.device).to(q.dtype)


def torch_slot_attn(q, k, v, K, V, p):
    """The reference's in-graph torch sequence (engine/code_predictor.py:46-47): bf16 scores + mask, fp32 softmax,
    probabilities to bf16, bf16 P.V.  Right operands are made contiguous before each product."""
    _write_slot(k, v, K, V, p)
    B = q.shape[0]
    mask = torch.full((STEPS, STEPS), float("-inf"), device=q.device).triu(1).to(q.dtype)[p]
    Kt = K.transpose(-1, -2).contiguous()
    att = torch.matmul(q.view(B, NKV, NH // NKV, HD), Kt) * (HD ** -0.5) + mask
    return torch.matmul(torch.softmax(att.float(), dim=-1).to(q.dtype), V.contiguous()).reshape(B, NH * HD)
