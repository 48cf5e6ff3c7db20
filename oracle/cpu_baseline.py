"""Timed CPU baselines: the reference's fake-quant forward restated with torch CPU ops.

TEST AND MEASUREMENT INFRASTRUCTURE ONLY.  Imported by ``bench.py``'s ``cpu_baseline`` leg
(the reported CPU figures) and by ``tests/`` (which check these restatements against the numpy
oracle); nothing in ``mindpipe_amd`` imports it.

What is timed (the reference's CPU path, torch ops in fp16 as the reference runs them):
  * W4A16: ``F.linear(x, w_deq)`` on the AWQ pseudo-quantized weight
    (``pseudo_quantize_tensor``, ``algorithm/quantization/ptq/awq/source/awq/quantize/quantizer.py:63-105``,
    then the HF forward); the one-off dequant is reported separately.
  * W8A8: ``F.linear(fq_token(x), fq_channel(W))`` (``SmoothQuantLinear.forward``,
    ``smoothquant/source/smoothquant/fake_quant.py:85-88``; quantizers ``:10-31``).
  * MoE: the per-expert loop of ``SmoothQuantPackedMoeExperts.forward`` (``fake_quant.py:166-191``).
  * Decoder stacks: one decoder layer's W4A16 linears at the decode batch, extrapolated over the
    layers (a full fp16 70B model does not fit a CPU run).
Protocol: median of 10 timed runs after 3 warmups, ``torch.get_num_threads()`` threads (the
host's OMP setting), the CPU model read from ``/proc/cpuinfo``.
"""
from __future__ import annotations

import os
import time

import torch
import torch.nn.functional as F


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def host_info() -> dict:
    try:
        nproc = len(os.sched_getaffinity(0))
    except AttributeError:
        nproc = os.cpu_count()
    return {"threads": torch.get_num_threads(), "nproc": nproc, "cpu_model": cpu_model()}


def median_ms(fn, runs: int = 10, warmup: int = 3) -> float:
    for _ in range(warmup):
        fn()
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    ts.sort()
    return 1e3 * (ts[runs // 2 - 1] + ts[runs // 2]) / 2 if runs % 2 == 0 else 1e3 * ts[runs // 2]


# ---------------------------------------------------------------- restated reference ops
@torch.no_grad()
def fake_quant_rows(t: torch.Tensor, n_bits: int = 8) -> torch.Tensor:
    """Per-row symmetric abs-max fake quant in t's dtype: the arithmetic of both
    ``quantize_activation_per_token_absmax`` and ``quantize_weight_per_channel_absmax``
    (``fake_quant.py:10-31``): s = max|t|.clamp(1e-5) / (2^(b-1) - 1); round(t / s) * s."""
    s = t.abs().amax(dim=-1, keepdim=True).clamp(min=1e-5) / (2 ** (n_bits - 1) - 1)
    return torch.round(t / s) * s


@torch.no_grad()
def awq_pseudo_quantize(w: torch.Tensor, group: int = 128) -> torch.Tensor:
    """Asymmetric 4-bit group pseudo-quantization in w's dtype (``quantizer.py:63-105``)."""
    n, k = w.shape
    g = w.reshape(-1, group)
    mx, mn = g.amax(dim=1, keepdim=True), g.amin(dim=1, keepdim=True)
    s = (mx - mn).clamp(min=1e-5) / 15
    z = (-torch.round(mn / s)).clamp(0, 15)
    return ((torch.clamp(torch.round(g / s) + z, 0, 15) - z) * s).reshape(n, k)


@torch.no_grad()
def moe_fake_forward(x, ids, w_topk, gu_fq, dn_fq):
    """The per-expert loop of ``SmoothQuantPackedMoeExperts.forward`` (``fake_quant.py:166-191``)
    on fake-quantized expert weights: for each hit expert in ascending order, per-token fake
    quant, gate/up linear, SiLU * up, per-token fake quant, down linear, router weight,
    ``index_add_``."""
    out = torch.zeros_like(x)
    inter = dn_fq.shape[2]
    for e in torch.unique(ids).tolist():
        slot, tok = torch.nonzero((ids == e).T, as_tuple=True)
        cur = fake_quant_rows(x[tok])
        gu = F.linear(cur, gu_fq[e])
        h = fake_quant_rows(F.silu(gu[:, :inter]) * gu[:, inter:])
        y = F.linear(h, dn_fq[e]) * w_topk[tok, slot, None]
        out.index_add_(0, tok, y.to(out.dtype))
    return out


# ---------------------------------------------------------------- timed baselines
def w4a16_linear(m=1, n=4096, k=4096, group=128, seed=1) -> dict:
    """C1: F.linear on the AWQ pseudo-quantized fp16 weight, M x K by N x K."""
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(n, k, generator=g) * 0.02).half()
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(0)).half()
    t0 = time.perf_counter()
    wd = awq_pseudo_quantize(w, group)
    t_deq = time.perf_counter() - t0
    ms = median_ms(lambda: F.linear(x, wd))
    nbytes = n * k // 2 + 2 * n * (k // group) * 2 + m * k * 2 + m * n * 2
    return {"value": round(nbytes / (ms * 1e-3) / 1e12, 6), "unit": "TB/s", "ms_per_call": ms,
            "sample": f"full workload: F.linear(x [{m},{k}] fp16, AWQ-dequantized W [{n},{k}] fp16), "
                      f"median of 10 after 3 warmups; one-off AWQ dequant {t_deq * 1e3:.0f} ms excluded",
            "dequant_ms": t_deq * 1e3}


def w8a8_fake_linear(m=16, n=11008, k=4096, max_rows=512, seed=1) -> dict:
    """C2: F.linear(fq_token(x), fq_channel(W)) in fp16.  Above ``max_rows`` rows a row sample is
    timed and the per-row time scaled to M (the rows are independent)."""
    g = torch.Generator().manual_seed(seed)
    wq = fake_quant_rows((torch.randn(n, k, generator=g) * 0.02).half())
    ms_rows = min(m, max_rows)
    x = torch.randn(ms_rows, k, generator=torch.Generator().manual_seed(0))
    x[:, torch.randperm(k, generator=torch.Generator().manual_seed(2))[: max(1, round(k * 0.01))]] *= 20
    x = x.half()
    ms = median_ms(lambda: F.linear(fake_quant_rows(x), wq)) * (m / ms_rows)
    ops = 2.0 * m * n * k
    return {"value": round(ops / (ms * 1e-3) / 1e12, 6), "unit": "TOPS", "ms_per_call": ms,
            "gb_s": (n * k + m * k + m * n * 2) / (ms * 1e-3) / 1e9,
            "sample": (f"F.linear(fq(x) [{ms_rows},{k}], fq(W) [{n},{k}]) fp16" +
                       (f", {ms_rows} of {m} rows timed, per-row time x{m / ms_rows:g}" if ms_rows < m else
                        ", full workload") + "; median of 10 after 3 warmups")}


def moe_fake(t=512, h=4096, inter=14336, e=8, top_k=2, t_sample=64, seed=1) -> dict:
    """C4: the per-expert loop on ``t_sample`` of the ``t`` tokens (same routing statistics),
    time scaled by t / t_sample (the expert GEMMs are compute-bound on the CPU at these row
    counts; stated as an extrapolation)."""
    g = torch.Generator().manual_seed(seed)
    gu = torch.empty(e, 2 * inter, h, dtype=torch.float16)
    dn = torch.empty(e, h, inter, dtype=torch.float16)
    for i in range(e):
        gu[i] = fake_quant_rows((torch.randn(2 * inter, h, generator=g) * 0.02).half())
        dn[i] = fake_quant_rows((torch.randn(h, inter, generator=g) * 0.02).half())
    x = torch.randn(t_sample, h, generator=torch.Generator().manual_seed(0)).half()
    p = torch.softmax(torch.randn(t_sample, e, generator=torch.Generator().manual_seed(3)), -1)
    w, ids = torch.topk(p, top_k, dim=-1)
    w = w / w.sum(-1, keepdim=True)
    ms = median_ms(lambda: moe_fake_forward(x, ids, w, gu, dn)) * (t / t_sample)
    wbytes = e * (2 * inter * h + h * inter)
    return {"value": round(wbytes / (ms * 1e-3) / 1e12, 6), "unit": "TB/s (expert weight bytes)",
            "ms_per_call": ms,
            "sample": f"per-expert fake-quant loop on {t_sample} of {t} tokens (top-{top_k} of {e} experts, "
                      f"H={h}, I={inter}), time x{t / t_sample:g}; median of 10 after 3 warmups"}


def decoder_layer_decode(hidden, inter, heads, kv_heads, layers, batch=1, group=128, seed=1) -> dict:
    """C3 / C5: one decoder layer's W4A16 linears (q/k/v, o, gate/up, down) as F.linear on
    AWQ-dequantized fp16 weights at the decode batch; tokens/s = batch / (layers x layer time)
    (attention, norms and lm_head excluded: a lower bound on the CPU step time)."""
    hd = hidden // heads
    shapes = {"qkv": ((heads + 2 * kv_heads) * hd, hidden), "o": (hidden, heads * hd),
              "gate_up": (2 * inter, hidden), "down": (hidden, inter)}
    g = torch.Generator().manual_seed(seed)
    ws = {k: awq_pseudo_quantize((torch.randn(*s, generator=g) * 0.02).half(), group) for k, s in shapes.items()}
    x = torch.randn(batch, hidden, generator=torch.Generator().manual_seed(0)).half()
    xi = torch.randn(batch, inter, generator=torch.Generator().manual_seed(0)).half()
    xa = torch.randn(batch, heads * hd, generator=torch.Generator().manual_seed(0)).half()

    def layer():
        F.linear(x, ws["qkv"])
        F.linear(xa, ws["o"])
        F.linear(x, ws["gate_up"])
        F.linear(xi, ws["down"])

    ms = median_ms(layer)
    return {"value": round(batch / (ms * layers * 1e-3), 4), "unit": "tok/s", "ms_per_layer": ms,
            "sample": f"one layer's 4 W4A16 linears (AWQ-dequantized fp16, F.linear) at batch {batch}, "
                      f"median of 10 after 3 warmups, x{layers} layers (attention, norms, lm_head excluded)"}
