"""Llama-shaped decoder stack with every linear on the W4A16 kernels (measurement harness).

Used to measure prefill and greedy-decode throughput on the shapes of the W4A16
workloads: Llama-2-7B (32 layers, hidden 4096, 32 heads, FFN 11008, vocab 32000)
and Llama-3-70B (80 layers, hidden 8192, 64 q / 8 kv heads, FFN 28672, vocab 128256).
Weights are random W4 g128 codes with fp16 scales / zeros (a random init of the
quantized model; no checkpoint is loaded).  q/k/v and gate/up are fused into one
W4A16 GEMM each (row concatenation of the packed weight is exact).

``decode_step`` runs one greedy step as 7-8 launches per layer: fused residual-add
+ RMSNorm, the W4A16 GEMVs, split-K decode attention with RoPE and the KV append
fused in (plus the split merge), and the gate/up GEMV with SiLU-mul in its epilogue.
With one row (and hidden 2048 / 4096) each add-RMSNorm runs in the prologue of the
GEMV that consumes it: 6 launches per layer.
The KV cache has a fixed capacity ``[L, B, kvh, T, 128]`` and every kernel reads
the current position from device memory, so a step is shape-static and can be
captured into a HIP graph.  ``decode_step_torch`` is the same step in PyTorch ops
(masked attention over the whole cache), kept as the numerical reference.  Prefill
uses PyTorch attention (SDPA) around the same W4A16 linears and fused norm / SiLU-mul kernels.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import ops


@dataclass
class DecoderConfig:
    layers: int = 32
    hidden: int = 4096
    heads: int = 32
    kv_heads: int = 32
    ffn: int = 11008
    vocab: int = 32000
    group: int = 128
    rope_theta: float = 10000.0
    eps: float = 1e-5

    @staticmethod
    def llama2_7b():
        return DecoderConfig()

    @staticmethod
    def llama3_70b():
        return DecoderConfig(layers=80, hidden=8192, heads=64, kv_heads=8, ffn=28672, vocab=128256,
                             rope_theta=500000.0)

    @property
    def head_dim(self):
        return self.hidden // self.heads


class _W4:
    """Random W4 g128 linear held as packed codes + fp16 scales / zeros."""

    def __init__(self, n, k, group, gen, device):
        self.n, self.k, self.group = n, k, group
        self.packed = torch.randint(-2**31, 2**31 - 1, (n, k // 8), generator=gen, device=device, dtype=torch.int32)
        # dequantised values (u - z) * s with s ~ 0.0027: weights of std ~0.012 over [-0.02, 0.02]
        self.scales = (torch.rand(n, k // group, generator=gen, device=device) * 0.001 + 0.0022).half()
        self.zeros = torch.full((n, k // group), 8.0, device=device, dtype=torch.float16)

    def __call__(self, x):
        return ops.w4a16_gemm(x, self.packed, self.scales, self.zeros, self.group, None)

    def swiglu(self, x):
        """silu(gate) * up of this fused gate/up linear in one launch."""
        return ops.w4a16_gemm_swiglu(x, self.packed, self.scales, self.zeros, self.group, None)

    def nbytes(self):
        return self.packed.numel() * 4 + self.scales.numel() * 2 + self.zeros.numel() * 2

    def dequantized(self):
        """The pseudo-quantized fp16 weight ``(u - z) * s`` (each op rounded to fp16, as the reference's
        dequantised tensor), unpacked with torch bit operations: the reference path shares no kernel
        with the W4A16 GEMMs it checks.  Cached."""
        w = getattr(self, "_deq", None)
        if w is None:
            shifts = torch.arange(0, 32, 4, device=self.packed.device, dtype=torch.int32)
            u = ((self.packed.unsqueeze(-1) >> shifts) & 0xF).reshape(self.n, self.k).to(torch.float16)
            s = self.scales.repeat_interleave(self.group, dim=1)
            z = self.zeros.repeat_interleave(self.group, dim=1)
            w = (u - z) * s
            self._deq = w
        return w

    def reference(self, x):
        """``F.linear`` on the pseudo-quantized weight with fp32 accumulation, one rounding to fp16."""
        return (x.float() @ self.dequantized().float().t()).half()


def _rms(x, w, eps):
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)).half() * w


class W4Decoder:
    def __init__(self, cfg: DecoderConfig, max_batch: int, max_len: int, device="cuda", seed: int = 1):
        self.cfg, self.max_batch, self.max_len = cfg, max_batch, max_len
        self.fuse_norm = True  # one-row decode steps: add-RMSNorm inside the next GEMV
        gen = torch.Generator(device=device).manual_seed(seed)
        h, hd, kvh = cfg.hidden, cfg.head_dim, cfg.kv_heads
        self.embed = (torch.randn(cfg.vocab, h, generator=gen, device=device) * 0.02).half()
        self.layers = []
        for _ in range(cfg.layers):
            self.layers.append({
                "ln1": torch.ones(h, device=device, dtype=torch.float16),
                "ln2": torch.ones(h, device=device, dtype=torch.float16),
                "qkv": _W4((cfg.heads + 2 * kvh) * hd, h, cfg.group, gen, device),
                "o": _W4(h, cfg.heads * hd, cfg.group, gen, device),
                "gate_up": _W4(2 * cfg.ffn, h, cfg.group, gen, device),
                "down": _W4(h, cfg.ffn, cfg.group, gen, device),
            })
        self.norm = torch.ones(h, device=device, dtype=torch.float16)
        self.lm_head = _W4(cfg.vocab, h, cfg.group, gen, device)
        # KV cache [L, B, kvh, T, hd]: one 256-byte row per position
        self.k_cache = torch.zeros(cfg.layers, max_batch, kvh, max_len, hd, device=device, dtype=torch.float16)
        self.v_cache = torch.zeros(cfg.layers, max_batch, kvh, max_len, hd, device=device, dtype=torch.float16)
        self.attn_ws = {}
        inv = 1.0 / (cfg.rope_theta ** (torch.arange(0, hd, 2, device=device).float() / hd))
        t = torch.arange(max_len, device=device).float()
        freqs = torch.outer(t, inv)
        self.cos = freqs.cos().half()
        self.sin = freqs.sin().half()

    def weight_bytes(self):
        return sum(l[n].nbytes() for l in self.layers for n in ("qkv", "o", "gate_up", "down")) + self.lm_head.nbytes()

    def _rope(self, x, pos):
        # x [B, heads, T, hd]; pos [T] (or [B, T] for decode)
        cos = self.cos[pos].unsqueeze(-3) if pos.dim() == 1 else self.cos[pos].unsqueeze(1)
        sin = self.sin[pos].unsqueeze(-3) if pos.dim() == 1 else self.sin[pos].unsqueeze(1)
        x1, x2 = x[..., 0::2], x[..., 1::2]
        out = torch.empty_like(x)
        out[..., 0::2] = x1 * cos - x2 * sin
        out[..., 1::2] = x1 * sin + x2 * cos
        return out

    @torch.no_grad()
    def prefill(self, tokens, return_logits=False):
        """tokens [B, T] int64; fills the cache at positions [0, T); returns next-token ids [B]
        (or the last position's logits).  The residual adds and RMSNorms run on the fused
        kernels (one launch each), the SiLU-mul in the gate/up GEMM's epilogue, RoPE and the
        cache writes in one launch; attention is PyTorch SDPA."""
        cfg = self.cfg
        b, t = tokens.shape
        hd, nh, kvh = cfg.head_dim, cfg.heads, cfg.kv_heads
        x = self.embed[tokens].reshape(b * t, -1)                  # [B*T, H] residual stream
        delta = None
        for li, l in enumerate(self.layers):
            if delta is None:
                hn = ops.add_rms_norm_quant(x, None, l["ln1"], cfg.eps, quant=False)[0]
            else:
                hn, _, _, x = ops.add_rms_norm_quant(delta, x, l["ln1"], cfg.eps, quant=False)
            # one launch: RoPE on q / k, q to [B, nh, T, hd], k / v into the cache rows 0 .. T-1
            q = ops.prefill_rope_split(l["qkv"](hn), b, nh, kvh, self.cos, self.sin, self.k_cache[li, :b],
                                       self.v_cache[li, :b])
            k, v = self.k_cache[li, :b, :, :t], self.v_cache[li, :b, :, :t]
            kk = k.repeat_interleave(nh // kvh, dim=1) if kvh != nh else k
            vv = v.repeat_interleave(nh // kvh, dim=1) if kvh != nh else v
            att = torch.nn.functional.scaled_dot_product_attention(q, kk.contiguous(), vv.contiguous(), is_causal=True)
            o = l["o"](att.transpose(1, 2).reshape(b * t, nh * hd))
            hn, _, _, x = ops.add_rms_norm_quant(o, x, l["ln2"], cfg.eps, quant=False)
            delta = l["down"](l["gate_up"].swiglu(hn))  # gate/up GEMM with SiLU-mul in its epilogue
        # the last position of each sequence only
        d_last = delta.reshape(b, t, -1)[:, -1].contiguous()
        x_last = x.reshape(b, t, -1)[:, -1].contiguous()
        hn = ops.add_rms_norm_quant(d_last, x_last, self.norm, cfg.eps, quant=False)[0]
        logits = self.lm_head(hn)
        return logits if return_logits else logits.argmax(-1)

    @torch.no_grad()
    def prefill_torch(self, tokens, return_logits=False):
        """The prefill in PyTorch ops (reference path): every linear is F.linear on the
        pseudo-quantized fp16 weight (fp32 accumulation), attention in fp32."""
        cfg = self.cfg
        b, t = tokens.shape
        hd, nh, kvh = cfg.head_dim, cfg.heads, cfg.kv_heads
        x = self.embed[tokens]
        pos = torch.arange(t, device=tokens.device)
        for li, l in enumerate(self.layers):
            hn = _rms(x, l["ln1"], cfg.eps)
            qkv = l["qkv"].reference(hn.reshape(b * t, -1)).reshape(b, t, nh + 2 * kvh, hd).transpose(1, 2)
            q, k, v = qkv[:, :nh], qkv[:, nh:nh + kvh], qkv[:, nh + kvh:]
            q, k = self._rope(q, pos), self._rope(k, pos)
            self.k_cache[li, :b, :, :t] = k
            self.v_cache[li, :b, :, :t] = v
            kk = k.repeat_interleave(nh // kvh, dim=1) if kvh != nh else k
            vv = v.repeat_interleave(nh // kvh, dim=1) if kvh != nh else v
            att = torch.nn.functional.scaled_dot_product_attention(q.float(), kk.float(), vv.float(),
                                                                   is_causal=True).half()
            x = x + l["o"].reference(att.transpose(1, 2).reshape(b * t, nh * hd)).reshape(b, t, -1)
            hn = _rms(x, l["ln2"], cfg.eps)
            gu = l["gate_up"].reference(hn.reshape(b * t, -1))
            act = torch.nn.functional.silu(gu[:, :cfg.ffn]) * gu[:, cfg.ffn:]
            x = x + l["down"].reference(act.contiguous()).reshape(b, t, -1)
        logits = self.lm_head.reference(_rms(x[:, -1], self.norm, cfg.eps).contiguous())
        return logits if return_logits else logits.argmax(-1)

    def attn_splits(self, b):
        """Workgroups per (row, kv head) for the decode attention: ~1024 in all for one head per
        kv head, ~512 (at most 32 splits) for head groups, whose MFMA scoring makes longer
        chunks pay (70B, measured: B = 1 9.38 -> 9.23 ms with 32 splits instead of 64, B = 16
        17.80 -> 17.57 ms with 4 instead of 8), and a score buffer of at most 64 KB per
        workgroup."""
        cfg = self.cfg
        grp = cfg.heads // cfg.kv_heads
        if grp >= 4:
            splits = max(1, min(32, 512 // (b * cfg.kv_heads)))
        else:
            splits = max(1, min(64, 1024 // (b * cfg.kv_heads)))
        while -(-self.max_len // splits) * grp * 4 > 64 * 1024:
            splits += 1
        return splits

    def _attn_workspace(self, b):
        splits = self.attn_splits(b)
        key = (b, splits)
        if key not in self.attn_ws:
            self.attn_ws[key] = ops.decode_attention_workspace(b, self.cfg.heads, splits, self.k_cache.device)
        return splits, self.attn_ws[key]

    @torch.no_grad()
    def decode_step(self, tokens, cur_len, return_logits=False):
        """One greedy step for a batch on the fused kernels.  tokens [B] int64 (the last
        token), cur_len [1] int64 device tensor = position of that token; writes its K/V
        and returns the next ids (or the logits)."""
        cfg = self.cfg
        b = tokens.shape[0]
        hd, nh, kvh = cfg.head_dim, cfg.heads, cfg.kv_heads
        splits, ws = self._attn_workspace(b)
        scale = 1.0 / math.sqrt(hd)
        x = self.embed[tokens]                                    # [B, H] residual stream
        # one row of width <= 4096: each add-RMSNorm runs inside the next GEMV (at 8192 every
        # workgroup's 48 KB prologue costs more than the launch it saves: 70B 9.37 -> 9.80 ms/step)
        fused = self.fuse_norm and b == 1 and cfg.hidden in (2048, 4096) and cfg.group == 128

        def norm_linear(delta, x, w, lin, swiglu=False):
            """(lin(RMSNorm(delta + x) * w), delta + x); delta None: no residual add."""
            if fused:
                src, res = (x, None) if delta is None else (delta, x)
                y, rsum = ops.w4a16_gemv_add_rms_norm(src, res, w, cfg.eps, lin.packed, lin.scales, lin.zeros,
                                                      lin.group, None, swiglu)
                return y, (x if rsum is None else rsum)
            if delta is None:
                hn = ops.add_rms_norm_quant(x, None, w, cfg.eps, quant=False)[0]
            else:
                hn, _, _, x = ops.add_rms_norm_quant(delta, x, w, cfg.eps, quant=False)
            return (lin.swiglu(hn) if swiglu else lin(hn)), x

        delta = None
        for li, l in enumerate(self.layers):
            qkv, x = norm_linear(delta, x, l["ln1"], l["qkv"])
            att = ops.decode_rope_attention(qkv, nh, kvh, self.cos, self.sin, cur_len, self.k_cache[li, :b],
                                            self.v_cache[li, :b], splits, scale, ws)
            act, x = norm_linear(l["o"](att.reshape(b, nh * hd)), x, l["ln2"], l["gate_up"], swiglu=True)
            delta = l["down"](act)
        logits, x = norm_linear(delta, x, self.norm, self.lm_head)
        return logits if return_logits else ops.argmax_rows(logits)

    @torch.no_grad()
    def decode_step_torch(self, tokens, cur_len, return_logits=False):
        """The decode step in PyTorch ops (reference path): RMSNorm on the rounded residual, every
        linear F.linear on the pseudo-quantized fp16 weight (fp32 accumulation), fp32 attention over the
        whole cache masked by the current length."""
        cfg = self.cfg
        b = tokens.shape[0]
        hd, nh, kvh = cfg.head_dim, cfg.heads, cfg.kv_heads
        grp = nh // kvh
        x = self.embed[tokens]                                    # [B, H]
        pos = cur_len.expand(b).unsqueeze(1)                      # [B, 1]
        mask = torch.where(torch.arange(self.max_len, device=tokens.device) > cur_len, float("-inf"), 0.0)
        scale = 1.0 / math.sqrt(hd)
        for li, l in enumerate(self.layers):
            hn = _rms(x, l["ln1"], cfg.eps)
            qkv = l["qkv"].reference(hn).reshape(b, nh + 2 * kvh, 1, hd)
            q, k, v = qkv[:, :nh], qkv[:, nh:nh + kvh], qkv[:, nh + kvh:]
            q, k = self._rope(q, pos), self._rope(k, pos)
            self.k_cache[li, :b].index_copy_(2, cur_len, k.contiguous())
            self.v_cache[li, :b].index_copy_(2, cur_len, v.contiguous())
            qg = q.reshape(b, kvh, grp, hd).float()                # heads grouped by kv head
            kt = self.k_cache[li, :b].float().transpose(-1, -2).contiguous()
            s = torch.matmul(qg, kt) * scale + mask                # [B, kvh, grp, T]
            p = torch.softmax(s, dim=-1)
            att = torch.matmul(p, self.v_cache[li, :b].float()).half()
            x = x + l["o"].reference(att.reshape(b, nh * hd))
            hn = _rms(x, l["ln2"], cfg.eps)
            gu = l["gate_up"].reference(hn)
            act = torch.nn.functional.silu(gu[:, :cfg.ffn]) * gu[:, cfg.ffn:]
            x = x + l["down"].reference(act.contiguous())
        logits = self.lm_head.reference(_rms(x, self.norm, cfg.eps).contiguous())
        return logits if return_logits else logits.argmax(-1)
