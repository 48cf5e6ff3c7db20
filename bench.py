"""Benchmark of the quantized-linear forward path on one MI355X.

Prints ONE JSON line.  ``value`` is the headline W4A16 g128 GEMV at M=1 (K=N=4096, the
BASELINE metric's first figure) in TB/s of algorithmic bytes.  A step is one pass over 64
distinct W4A16 linears of that shape (64 rotated weight copies, 571 MB, so the 256 MB Infinity
Cache cannot serve them): one HIP graph of 64 GEMV launches, replayed ``--steps`` times after
``--warmup`` untimed replays; inputs are resident in HBM before timing.  The other legs of the
metric (W8A8 int8 GEMM TOPS at M=4096, the W8A8 sweep, W4A16 M=16 and the 70B GEMV shapes, the
Mixtral-shaped MoE chain, the Llama-2-7B-shaped decode at B = 1 / 8 / 32 with its 2048-token
prefill, and the Llama-3-70B-shaped decode at B = 1 / 16 / 64 over a 4096-token context) are
reported under ``legs``, each with its roofline fraction and its CPU baseline.  Timing uses HIP
events recorded on the stream the kernels are launched on (torch's current stream), bracketed
by ``torch.cuda.synchronize()``.

``cpu_baseline``: the reference's CPU fake-quant forward restated with torch CPU ops
(``oracle/cpu_baseline.py``), timed on this host's cores on the same workload (bounded samples
stated in each ``sample``).

``--profile NAME`` runs one kernel mix for rocprofv3 (the commands in ``profiles/``):
``w4gemv`` (the headline loop), ``readfloor`` (one-launch reads of 8.9 MB, rotated), ``readsweep``
(read probes of several launch shapes at 8.9 MB and 1 GiB), ``curead`` (per-CU read rates from L2 and
from HBM, into registers or LDS), ``cufew`` (the HBM read rate of one CU when 8 to 128 read), ``mfmabread`` (the MoE weights read in an MFMA B operand's lane order), ``w8sweep`` (the W8A8 sweep's GEMMs), ``moe`` (the Mixtral MoE
chain), ``moesmall`` (the same chain at an expert FFN of 1792), ``prefill`` (the 7B prefill linears at
M = 2048), ``w4shapes`` (M=16 and the 70B GEMV shapes), ``w4bf16`` (the bf16 W4A16 legs),
``w4batch8`` (7B gate/up and down at M = 1 and 8), ``dec7b`` (the 7B decode step), ``dec70b`` (four
layers of the 70B decode step), ``decsteps`` (two full-depth steps of every decode leg, for their
traffic) and ``w8big`` (the M=4096 int8 GEMM); ``--traffic-probe`` runs the kernel mix of
``profiles/traffic.json``.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np
import torch

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, published
INT8_PEAK_TOPS = 5000.0        # MI355X dense int8 MFMA, published (POPS x 1000)
FP16_PEAK_TFLOPS = 2500.0      # MI355X dense fp16 MFMA, published

METRIC = "qlinear HBM TB/s (W4A16, M=1) & int8 TOPS (W8A8, M=4096); 7B decode tok/s"


def _log(*a):
    print(*a, file=sys.stderr, flush=True)


def _time_graph(fn, per_graph, steps, warmup):
    """Milliseconds per step: a step is one replay of a HIP graph holding ``per_graph`` launches
    ``fn(0) .. fn(per_graph - 1)`` (each on its own rotated input); ``warmup`` untimed replays,
    then exactly ``steps`` timed replays between HIP events on the current stream."""
    for i in range(per_graph):
        fn(i)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(min(2, per_graph)):
            fn(i)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(per_graph):
            fn(i)
    for _ in range(max(1, warmup)):
        graph.replay()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(steps):
        graph.replay()
    e1.record(st)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    del graph
    return ms


def _traffic(key):
    """HBM bytes per launch measured by rocprofv3 FETCH_SIZE / WRITE_SIZE (profiles/traffic.json)."""
    try:
        with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic.json")) as f:
            return json.load(f)[key]["bytes"]
    except (OSError, KeyError, ValueError):
        return None


def _roof(bound, achieved, peak, unit, traffic=None):
    return {"bound": bound, "achieved": round(achieved, 3), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 4), "traffic": traffic}


def _w4_copies(ops, n, k, copies, g=128, dtype=torch.float16):
    gen = torch.Generator(device="cuda").manual_seed(1)
    w = (torch.randn(n, k, generator=gen, device="cuda") * 0.02).to(dtype)
    packed, s, z, _ = ops.w4_quantize_awq(w, g, True, return_deq=False)
    del w
    return [packed.clone() for _ in range(copies)], [s.clone() for _ in range(copies)], \
        [z.clone() for _ in range(copies)]


def leg_w4a16(ops, m, n, k, steps, warmup, copies=64, g=128, dtype=torch.float16):
    """W4A16 at M x K x N: one step = ``copies`` launches, each on its own weight copy.  ``dtype``:
    the activation / scale / zero / output dtype (bf16: weights quantized in bf16 arithmetic)."""
    pk, sc, zr = _w4_copies(ops, n, k, copies, g, dtype)
    gx = torch.Generator(device="cuda").manual_seed(0)
    x = torch.randn(m, k, generator=gx, device="cuda").to(dtype)
    y = ops.w4a16_gemm(x, pk[0], sc[0], zr[0], g, None)
    ms_step = _time_graph(lambda i: ops.w4a16_gemm(x, pk[i], sc[i], zr[i], g, None), copies, steps, warmup)
    ms = ms_step / copies
    nbytes = n * k // 2 + 2 * n * (k // g) * 2 + m * k * 2 + m * n * 2
    gbs = nbytes / (ms * 1e-3) / 1e9
    del pk, sc, zr
    torch.cuda.empty_cache()
    return {"m": m, "n": n, "k": k, "group": g, "dtype": "u4*bf16->bf16" if dtype == torch.bfloat16 else "u4*f16->f16",
            "ms_per_call": ms, "ms_per_step": ms_step,
            "bytes_per_call": nbytes, "tb_s": gbs / 1000.0, "roofline": _roof("hbm", gbs, HBM_PEAK_GBS, "GB/s"),
            "weight_copies": copies, "working_set_bytes": copies * (n * k // 2 + 2 * n * (k // g) * 2)}, y


def leg_w8a8(ops, m, n, k, steps, warmup):
    """C2: X [M, K] ~ N(0, 1) with 1% of the channels x20, W [N, K] ~ N(0, 0.02); smoothed with
    alpha = 0.5 (s_j = max|X_j|^0.5 / max|W_j|^0.5: X / s, W * s) on the library's smoothing kernels,
    then W per-channel int8 (export rule) and X per-token int8 (runtime rule)."""
    gen = torch.Generator(device="cuda").manual_seed(1)
    w = (torch.randn(n, k, generator=gen, device="cuda") * 0.02).half()
    gx = torch.Generator(device="cuda").manual_seed(0)
    x = torch.randn(m, k, generator=gx, device="cuda")
    idx = torch.randperm(k, generator=torch.Generator().manual_seed(2))[: max(1, round(k * 0.01))]
    x[:, idx.cuda()] *= 20
    x = x.half()
    smooth = ops.smooth_scales(ops.colmax_abs(x), ops.colmax_abs(w), 0.5, torch.float16)
    ops.scale_columns_(x, smooth, divide=True)
    ops.scale_columns_(w, smooth)
    qw, sw, _ = ops.w8_quantize_per_channel(w, "export")
    del w
    # HBM-bound shapes rotate distinct weight copies past the Infinity Cache (>= 600 MB); the
    # MFMA-bound M = 4096 GEMM runs 4 launches per step on one copy
    copies = max(1, min(16, int(600e6 // (n * k)))) if m <= 256 else 4
    qws = [qw.clone() for _ in range(copies)] if m <= 256 else [qw] * copies
    q, st = ops.quant_per_token_i8(x)
    ms = _time_graph(lambda i: ops.w8a8_gemm(q, st, qws[i], sw, None, torch.float16), copies, steps, warmup) / copies
    ms_q = _time_graph(lambda i: ops.quant_per_token_i8(x), 4, steps, warmup) / 4
    ops_count = 2.0 * m * n * k
    nbytes = n * k + m * k + m * n * 2 + 4 * n + 4 * m
    tops = ops_count / (ms * 1e-3) / 1e12
    gbs = nbytes / (ms * 1e-3) / 1e9
    out = {"m": m, "n": n, "k": k, "smoothing_alpha": 0.5, "ms_gemm": ms, "ms_quant": ms_q, "ms_e2e": ms + ms_q, "tops": tops,
           "tops_e2e": ops_count / ((ms + ms_q) * 1e-3) / 1e12, "gb_s": gbs,
           "weight_copies": len({id(t) for t in qws})}
    traffic = _traffic(f"w8a8_gemm_m{m}_k{k}_n{n}")
    if m >= 1024:
        out["roofline"] = _roof("mfma", tops, INT8_PEAK_TOPS, "TOPS", traffic)
    elif m <= 16:
        out["roofline"] = _roof("hbm", gbs, HBM_PEAK_GBS, "GB/s", traffic)
    else:
        out["roofline"] = _roof("hbm", gbs, HBM_PEAK_GBS, "GB/s", traffic)
        out["roofline_mfma"] = _roof("mfma", tops, INT8_PEAK_TOPS, "TOPS", traffic)
    del qws
    torch.cuda.empty_cache()
    return out


def _moe_inputs(ops, t=512, h=4096, inter=14336, e=8, top_k=2):
    """Config 4's inputs: tokens ~ N(0, 1), router logits ~ N(0, 1) routed by fp32 softmax -> top-k
    -> renormalise, expert weights ~ N(0, 0.02) quantized per row to int8 (export rule)."""
    gen = torch.Generator(device="cuda").manual_seed(1)
    q13 = torch.empty((e, 2 * inter, h), dtype=torch.int8, device="cuda")
    s13 = torch.empty((e, 2 * inter), dtype=torch.float32, device="cuda")
    q2 = torch.empty((e, h, inter), dtype=torch.int8, device="cuda")
    s2 = torch.empty((e, h), dtype=torch.float32, device="cuda")
    for i in range(e):
        w = (torch.randn(2 * inter, h, generator=gen, device="cuda") * 0.02).half()
        q13[i], s13[i], _ = ops.w8_quantize_per_channel(w, "export")
        w = (torch.randn(h, inter, generator=gen, device="cuda") * 0.02).half()
        q2[i], s2[i], _ = ops.w8_quantize_per_channel(w, "export")
    del w
    gx = torch.Generator(device="cuda").manual_seed(0)
    x = torch.randn(t, h, generator=gx, device="cuda").half()
    logits = torch.randn(t, e, generator=torch.Generator().manual_seed(3)).float()
    p = torch.softmax(logits, dim=-1)
    tw, ids = torch.topk(p, top_k, dim=-1)
    tw = (tw / tw.sum(-1, keepdim=True)).float().cuda()
    ids = ids.to(torch.int32).cuda()
    return x, ids, tw, q13, s13, q2, s2


def _moe_chain_ms(ops, steps, warmup=3):
    x, ids, tw, q13, s13, q2, s2 = _moe_inputs(ops)
    return _time_graph(lambda i: ops.moe_w8a8_forward(x, ids, tw, q13, s13, q2, s2), 1, steps, warmup)


def leg_moe(ops, steps, warmup, t=512, h=4096, inter=14336, e=8, top_k=2):
    ms = _moe_chain_ms(ops, steps, warmup)
    wbytes = e * (2 * inter * h + h * inter)
    ops_count = 2.0 * t * top_k * (2 * inter * h + h * inter)
    gbs = wbytes / (ms * 1e-3) / 1e9
    tops = ops_count / (ms * 1e-3) / 1e12
    chain = _traffic("moe_chain_mixtral_t512")
    return {"tokens": t, "experts": e, "top_k": top_k, "hidden": h, "inter": inter, "ms_chain": ms,
            "weight_bytes": wbytes, "gb_s": gbs, "tops": tops,
            "roofline": _roof("hbm", gbs, HBM_PEAK_GBS, "GB/s", chain),
            "roofline_mfma": _roof("mfma", tops, INT8_PEAK_TOPS, "TOPS", chain)}


def leg_decoder(cfg_name, batches, prompt, gen_tokens, prefill_batch=1):
    """Llama-shaped W4A16 stack: prefill tok/s at B=prefill_batch and greedy decode tok/s
    at each batch size.  For decode the KV cache holds a `prompt`-token context (random
    values: decode cost does not depend on them); one step is captured in a HIP graph
    that also feeds the argmax back as the next token, and is replayed gen_tokens times."""
    from mindpipe_amd.decoder import DecoderConfig, W4Decoder
    cfg = getattr(DecoderConfig, cfg_name)()
    out = {"model": cfg_name, "prompt": prompt, "gen_tokens": gen_tokens, "decode": {}}
    max_len = prompt + gen_tokens
    kv_per_tok_layer = 2 * cfg.kv_heads * cfg.head_dim * 2
    for b in batches:
        model = W4Decoder(cfg, max_batch=b, max_len=max_len)
        wbytes = model.weight_bytes()
        if b == prefill_batch:
            toks = torch.randint(0, cfg.vocab, (b, prompt), device="cuda",
                                 generator=torch.Generator(device="cuda").manual_seed(4))
            model.prefill(toks)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            model.prefill(toks)
            e1.record()
            torch.cuda.synchronize()
            ms = e0.elapsed_time(e1)
            n_params = sum(l[n].n * l[n].k for l in model.layers for n in ("qkv", "o", "gate_up", "down"))
            lin_flops = 2.0 * b * prompt * n_params
            out["prefill"] = {"batch": b, "tokens": prompt, "ms": ms, "tok_s": b * prompt / (ms * 1e-3),
                              "linear_tflops": lin_flops / (ms * 1e-3) / 1e12,
                              "roofline": _roof("mfma", lin_flops / (ms * 1e-3) / 1e12, FP16_PEAK_TFLOPS, "TFLOP/s")}
        g = torch.Generator(device="cuda").manual_seed(5)
        model.k_cache.normal_(0, 1, generator=g)
        model.v_cache.normal_(0, 1, generator=g)
        tok = torch.randint(0, cfg.vocab, (b,), device="cuda", generator=g)
        cur = torch.tensor([prompt], device="cuda", dtype=torch.int64)

        def step():
            nxt = model.decode_step(tok, cur)
            tok.copy_(nxt)
            cur.add_(1)

        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            step()
        torch.cuda.current_stream().wait_stream(side)
        cur.fill_(prompt)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        cur.fill_(prompt)
        graph.replay()
        cur.fill_(prompt)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(gen_tokens):
            graph.replay()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / gen_tokens
        avg_len = prompt + (gen_tokens + 1) / 2       # positions [0, pos] read by the attention kernel
        kv_bytes = b * avg_len * cfg.layers * kv_per_tok_layer
        alg_bytes = wbytes + kv_bytes
        out["decode"][str(b)] = {"ms_per_step": ms, "tok_s": b / (ms * 1e-3), "weight_bytes": wbytes,
                                 "kv_bytes_per_step_read": kv_bytes,
                                 "roofline": _roof("hbm", alg_bytes / (ms * 1e-3) / 1e9, HBM_PEAK_GBS, "GB/s",
                                                   _traffic(f"decode_{cfg_name}_b{b}"))}
        del graph, model
        torch.cuda.empty_cache()
    return out


def cpu_baselines(legs):
    """The reference's CPU path (oracle/cpu_baseline.py) on each leg's workload."""
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import cpu_baseline as CB
    info = CB.host_info()
    out = {}
    _log("cpu baseline: W4A16 M=1")
    out["head"] = CB.w4a16_linear(m=1)
    if "w4" in legs:
        _log("cpu baseline: W4A16 M=16")
        out["w4a16_m16_k4096_n4096"] = CB.w4a16_linear(m=16)
    if "w8" in legs:
        _log("cpu baseline: W8A8 M=16 / 4096")
        out["w8a8_m16_k4096_n11008"] = CB.w8a8_fake_linear(m=16)
        out["w8a8_m4096_k4096_n11008"] = CB.w8a8_fake_linear(m=4096)
    if "moe" in legs:
        _log("cpu baseline: MoE")
        out["moe_w8a8_mixtral_t512"] = CB.moe_fake()
    if "dec7b" in legs:
        _log("cpu baseline: 7B layer")
        out["llama2_7b_w4a16"] = CB.decoder_layer_decode(4096, 11008, 32, 32, 32)
    if "dec70b" in legs:
        _log("cpu baseline: 70B layer")
        out["llama3_70b_w4a16"] = CB.decoder_layer_decode(8192, 28672, 64, 8, 80)
    for v in out.values():
        v.update({"cores": info["threads"], "nproc": info["nproc"], "cpu_model": info["cpu_model"],
                  "kind": "port"})
    return out


def profile_mix(ops, name, steps):
    """Kernel mixes that the rocprofv3 summaries in profiles/ were taken from."""
    if name == "w4gemv":
        pk, sc, zr = _w4_copies(ops, 4096, 4096, 64)
        x = torch.randn(1, 4096, device="cuda").half()
        ms = _time_graph(lambda i: ops.w4a16_gemm(x, pk[i], sc[i], zr[i], 128, None), 64, steps, 5)
        print(f"w4gemv: {ms / 64 * 1e3:.3f} us per launch")
    elif name == "readfloor":
        # the measurement library's read probe over the headline GEMV's 8,929,280 bytes (64 rotated
        # buffers): launch + latency + transfer with no dequant or dot work
        from mindpipe_amd.measure import probe_read
        bufs = [torch.ones(8929280 // 4, dtype=torch.int32, device="cuda") for _ in range(64)]
        sinks = [probe_read(b) for b in bufs]
        ms = _time_graph(lambda i: probe_read(bufs[i], sinks[i]), 64, steps, 5)
        print(f"readfloor: {ms / 64 * 1e3:.3f} us per 8.9 MB read launch")
    elif name == "readsweep":
        # read probes of several launch shapes (threads per workgroup, 16-byte loads per lane,
        # one-shot workgroups or a fixed strided grid), graph-replayed: at the headline's 8.9 MB over
        # 64 rotated buffers and at 1 GiB (one buffer, four times the Infinity Cache)
        from mindpipe_amd.measure import probe_read
        small = [torch.ones(8929280 // 4, dtype=torch.int32, device="cuda") for _ in range(64)]
        shapes_small = [(256, 1, 0), (256, 2, 0), (256, 4, 0), (256, 8, 0), (512, 2, 0), (512, 4, 0),
                        (256, 4, 256), (256, 8, 256), (512, 4, 256), (512, 4, 512), (256, 4, 1024), (512, 2, 1024)]
        for th, ld, gr in shapes_small:
            sinks = [probe_read(b, None, th, ld, gr) for b in small]
            ms = _time_graph(lambda i: probe_read(small[i], sinks[i], th, ld, gr), 64, steps, 3)
            us = ms / 64 * 1e3
            print(f"readsweep 8.9MB threads={th} loads={ld} grid={gr or 'one-shot'}: {us:.3f} us per launch, "
                  f"{8929280 / (us * 1e-6) / 1e12:.2f} TB/s", flush=True)
        del small
        torch.cuda.empty_cache()
        big = torch.ones((1 << 30) // 4, dtype=torch.int32, device="cuda")
        shapes_big = [(256, 4, 0), (512, 8, 0), (512, 4, 256), (512, 8, 256), (512, 4, 512), (512, 8, 512),
                      (512, 4, 1024), (512, 4, 2048), (256, 4, 4096)]
        for th, ld, gr in shapes_big:
            sink = probe_read(big, None, th, ld, gr)
            ms = _time_graph(lambda i: probe_read(big, sink, th, ld, gr), 4, steps, 3)
            us = ms / 4 * 1e3
            print(f"readsweep 1GiB threads={th} loads={ld} grid={gr or 'one-shot'}: {us:.1f} us per launch, "
                  f"{(1 << 30) / (us * 1e-6) / 1e12:.2f} TB/s", flush=True)
    elif name == "tileread":
        # the W8A8 weight operand (N = 11008 rows of K = 4096 bytes, 13 rotated copies) read in a
        # tiled GEMM's order (a workgroup per tile of rows, step_bytes of each row per step, depth steps
        # in flight) against the same bytes read contiguously
        from mindpipe_amd.measure import probe_read, probe_read_tiles
        n, kb = 11008, 4096
        bufs = [torch.ones(n * kb // 4, dtype=torch.int32, device="cuda") for _ in range(13)]
        sinks = [probe_read(b, None, 256, 4, 0) for b in bufs]
        ms = _time_graph(lambda i: probe_read(bufs[i], sinks[i], 256, 4, 0), 13, steps, 3) / 13
        print(f"tileread contiguous: {ms * 1e3:.2f} us, {n * kb / (ms * 1e-3) / 1e12:.2f} TB/s", flush=True)
        for tr, sb, d in ((128, 128, 1), (128, 128, 4), (64, 256, 4), (32, 512, 4), (16, 1024, 4), (8, 2048, 2),
                          (32, 128, 4), (16, 256, 4), (128, 512, 1), (64, 1024, 1), (16, 4096, 1)):
            tsinks = [probe_read_tiles(b, n, kb, tr, sb, d) for b in bufs]
            ms = _time_graph(lambda i: probe_read_tiles(bufs[i], n, kb, tr, sb, d, tsinks[i]), 13, steps, 3) / 13
            print(f"tileread tile_rows={tr} step_bytes={sb} depth={d}: {ms * 1e3:.2f} us, "
                  f"{n * kb / (ms * 1e-3) / 1e12:.2f} TB/s", flush=True)
    elif name == "curead":
        # per-CU read rate: every workgroup re-reads a 1 MB region shared by its XCD (L2 hits after
        # the first pass; 32 passes), or one workgroup per distinct 4 MB / 2 MB region of 1 GiB (HBM),
        # into registers or straight into LDS, at several launch shapes
        from mindpipe_amd.measure import probe_cu_read
        buf = torch.ones(1 << 28, dtype=torch.int32, device="cuda")
        for mode in ("l2", "hbm"):
            for grid in (256, 512):
                for threads, loads in ((256, 4), (256, 8), (512, 4), (512, 8)):
                    for dma in (False, True):
                        if dma and threads * loads * 32 > 65536:
                            continue
                        if mode == "l2":
                            region, nreg, passes = 1 << 20, 8, 32
                        else:
                            region, nreg, passes = (1 << 30) // grid, grid, 1
                        sink = probe_cu_read(buf, region, nreg, passes, grid, threads, loads, dma)
                        ms = _time_graph(lambda i: probe_cu_read(buf, region, nreg, passes, grid, threads, loads, dma,
                                                                 sink), 1, steps, 2)
                        total = region * passes * grid
                        print(f"curead {mode} grid={grid} threads={threads} loads={loads} dma={int(dma)}: "
                              f"{ms * 1e3:.1f} us, {total / (ms * 1e-3) / 1e12:.2f} TB/s, "
                              f"{total / (ms * 1e-3) / 1e9 / 256:.1f} GB/s per CU", flush=True)
    elif name == "cufew":
        # the HBM read rate one workgroup (one CU) reaches when few CUs read: 8 to 128 workgroups, each
        # streaming its own region of 1 GiB (at most 64 MB) once, into registers or straight into LDS
        from mindpipe_amd.measure import probe_cu_read
        buf = torch.ones(1 << 28, dtype=torch.int32, device="cuda")
        for grid in (8, 32, 64, 128):
            for threads, loads, dma in ((256, 4, False), (256, 8, False), (512, 8, False), (256, 8, True)):
                region = min((1 << 30) // grid, 64 << 20)
                sink = probe_cu_read(buf, region, grid, 1, grid, threads, loads, dma)
                ms = _time_graph(lambda i: probe_cu_read(buf, region, grid, 1, grid, threads, loads, dma, sink), 1,
                                 steps, 2)
                total = region * grid
                print(f"cufew grid={grid} threads={threads} loads={loads} dma={int(dma)}: {ms * 1e3:.1f} us, "
                      f"{total / (ms * 1e-3) / 1e12:.2f} TB/s, {total / (ms * 1e-3) / 1e9 / grid:.1f} GB/s per "
                      f"workgroup", flush=True)
    elif name == "mfmabread":
        # the MoE expert weights read in an MFMA B operand's lane order straight from memory (32 rows x
        # 32 bytes per load instruction), against the same bytes read contiguously: GEMM1's
        # [8 x 28672, 4096] and GEMM2's [8 x 4096, 14336]
        from mindpipe_amd.measure import probe_read, probe_read_mfma_b
        for rows, kb, kps in ((8 * 28672, 4096, (1, 2, 4)), (8 * 4096, 14336, (1, 2, 4, 7))):
            buf = torch.ones(rows * kb // 4, dtype=torch.int32, device="cuda")
            sink = probe_read(buf, None, 256, 4, 0)
            ms = _time_graph(lambda i: probe_read(buf, sink, 256, 4, 0), 1, steps, 2)
            print(f"mfmabread [{rows}, {kb}] contiguous: {ms * 1e3:.1f} us, {rows * kb / (ms * 1e-3) / 1e12:.2f} TB/s",
                  flush=True)
            for kp in kps:
                for d in (1, 2, 4, 8):
                    bs = probe_read_mfma_b(buf, rows, kb, kp, d)
                    ms = _time_graph(lambda i: probe_read_mfma_b(buf, rows, kb, kp, d, bs), 1, steps, 2)
                    print(f"mfmabread [{rows}, {kb}] kparts={kp} depth={d}: {ms * 1e3:.1f} us, "
                          f"{rows * kb / (ms * 1e-3) / 1e12:.2f} TB/s", flush=True)
            del buf
            torch.cuda.empty_cache()
    elif name == "w8sweep":
        # the W8A8 sweep legs' GEMMs (M = 1, 16, 256, 4096; N = 11008, K = 4096) on random int8 data,
        # M <= 256 over 13 rotated weight copies as in the bench
        gen = torch.Generator(device="cuda").manual_seed(1)
        copies = [torch.randint(-127, 128, (11008, 4096), dtype=torch.int8, device="cuda", generator=gen)
                  for _ in range(13)]
        sw = torch.rand(11008, device="cuda") * 1e-3
        for m in (1, 16, 256, 4096):
            qx = torch.randint(-127, 128, (m, 4096), dtype=torch.int8, device="cuda", generator=gen)
            st = torch.rand(m, device="cuda") * 1e-2
            c = 13 if m <= 256 else 1
            ms = _time_graph(lambda i: ops.w8a8_gemm(qx, st, copies[i], sw, None, torch.float16), c, steps, 3) / c
            print(f"w8sweep m={m}: {ms * 1e3:.2f} us per launch", flush=True)
    elif name == "moe":
        # the Mixtral MoE leg's chain (route + quant, GEMM1 + SwiGLU + requant, GEMM2, combine) on the
        # bench leg's inputs
        ms = _moe_chain_ms(ops, steps)
        print(f"moe chain: {ms * 1e3:.1f} us per call", flush=True)
    elif name == "moesmall":
        # the same chain with an expert FFN of 1792 (8x smaller): its 176 MB of expert weights stay in
        # the Infinity Cache across calls, so the GEMMs' rate per byte shows whether HBM sets it
        x, ids, tw, q13, s13, q2, s2 = _moe_inputs(ops, inter=1792)
        ms = _time_graph(lambda i: ops.moe_w8a8_forward(x, ids, tw, q13, s13, q2, s2), 1, steps, 3)
        print(f"moe chain (I = 1792): {ms * 1e3:.1f} us per call", flush=True)
    elif name == "prefill":
        # the 7B prefill linears at M = 2048 (fp16): q/k/v (N = 12288), o (4096), fused gate/up with
        # SiLU-mul (2 x 11008), down (K = 11008)
        for n, k, swi in ((12288, 4096, False), (4096, 4096, False), (2 * 11008, 4096, True), (4096, 11008, False)):
            pk, sc, zr = _w4_copies(ops, n, k, 1)
            x = torch.randn(2048, k, device="cuda").half()
            if swi:
                f = lambda i: ops.w4a16_gemm_swiglu(x, pk[0], sc[0], zr[0], 128, None)  # noqa: E731
            else:
                f = lambda i: ops.w4a16_gemm(x, pk[0], sc[0], zr[0], 128, None)  # noqa: E731
            ms = _time_graph(f, 2, steps, 3) / 2
            print(f"prefill n={n} k={k}{' swiglu' if swi else ''}: {ms * 1e3:.1f} us, "
                  f"{2 * 2048 * n * k / (ms * 1e-3) / 1e12:.0f} TFLOP/s", flush=True)
            del pk, sc, zr
            torch.cuda.empty_cache()
    elif name == "w4shapes":
        for m, n, k, c in ((16, 4096, 4096, 64), (1, 28672, 8192, 8), (1, 8192, 28672, 8), (16, 28672, 8192, 8),
                           (64, 28672, 8192, 8)):
            pk, sc, zr = _w4_copies(ops, n, k, c)
            x = torch.randn(m, k, device="cuda").half()
            ms = _time_graph(lambda i: ops.w4a16_gemm(x, pk[i], sc[i], zr[i], 128, None), c, steps, 3)
            print(f"w4 m={m} n={n} k={k}: {ms / c * 1e3:.3f} us per launch")
            del pk, sc, zr
            torch.cuda.empty_cache()
    elif name == "w4bf16":
        # bf16 W4A16 (the matrix-core small-M kernel) at the bench's bf16 legs: M = 1 and 16 at
        # 4096 x 4096 (64 rotated copies) and the 70B gate/up GEMV (8 copies)
        for m, n, k, c in ((1, 4096, 4096, 64), (16, 4096, 4096, 64), (1, 28672, 8192, 8)):
            pk, sc, zr = _w4_copies(ops, n, k, c, dtype=torch.bfloat16)
            x = torch.randn(m, k, device="cuda").bfloat16()
            ms = _time_graph(lambda i: ops.w4a16_gemm(x, pk[i], sc[i], zr[i], 128, None), c, steps, 3)
            print(f"w4bf16 m={m} n={n} k={k}: {ms / c * 1e3:.3f} us per launch")
            del pk, sc, zr
            torch.cuda.empty_cache()
    elif name == "w4batch8":
        # the 7B gate/up (fused SiLU-up, N = 2 x 11008, K = 4096) and down (N = 4096, K = 11008)
        # linears at M = 1 (one-row GEMV) and M = 8 (batched kernel), 4 eager launches each
        for n, k, swiglu in ((2 * 11008, 4096, True), (4096, 11008, False)):
            pk, sc, zr = _w4_copies(ops, n, k, 1)
            for m in (1, 8):
                x = torch.randn(m, k, device="cuda").half()
                for _ in range(4):
                    if swiglu:
                        ops.w4a16_gemm_swiglu(x, pk[0], sc[0], zr[0], 128, None)
                    else:
                        ops.w4a16_gemm(x, pk[0], sc[0], zr[0], 128, None)
            del pk, sc, zr
        print("w4batch8 done")
    elif name == "dec7b":
        # the Llama-2-7B decode step at B = 1 and B = 8 with a 2048-token context (random KV values),
        # 4 eager steps each: the kernels of the bench's decode leg, one launch at a time
        from mindpipe_amd.decoder import DecoderConfig, W4Decoder
        cfg = DecoderConfig.llama2_7b()
        for b in (1, 8):
            model = W4Decoder(cfg, max_batch=b, max_len=2048 + 8)
            g = torch.Generator(device="cuda").manual_seed(5)
            model.k_cache.normal_(0, 1, generator=g)
            model.v_cache.normal_(0, 1, generator=g)
            tok = torch.randint(0, cfg.vocab, (b,), device="cuda", generator=g)
            cur = torch.tensor([2048], device="cuda", dtype=torch.int64)
            for _ in range(4):
                tok = model.decode_step(tok, cur)
                cur.add_(1)
            torch.cuda.synchronize()
            del model
            torch.cuda.empty_cache()
        print("dec7b done")
    elif name == "dec70b":
        # four layers of the Llama-3-70B decode step at B = 1 and B = 16 with a 4096-token context
        # (random KV values), 4 eager steps each: the per-layer kernels of the bench's 70B leg
        import dataclasses
        from mindpipe_amd.decoder import DecoderConfig, W4Decoder
        cfg = dataclasses.replace(DecoderConfig.llama3_70b(), layers=4)
        for b in (1, 16):
            model = W4Decoder(cfg, max_batch=b, max_len=4096 + 8)
            g = torch.Generator(device="cuda").manual_seed(5)
            model.k_cache.normal_(0, 1, generator=g)
            model.v_cache.normal_(0, 1, generator=g)
            tok = torch.randint(0, cfg.vocab, (b,), device="cuda", generator=g)
            cur = torch.tensor([4096], device="cuda", dtype=torch.int64)
            for _ in range(4):
                tok = model.decode_step(tok, cur)
                cur.add_(1)
            torch.cuda.synchronize()
            del model
            torch.cuda.empty_cache()
        print("dec70b done")
    elif name == "decsteps":
        # the bench's decode legs at full depth (Llama-2-7B at B = 1 / 8 / 32 after a 2048-token prompt,
        # Llama-3-70B at B = 1 / 16 / 64 after 4096 tokens; random KV), two eager steps each at the leg's
        # middle position (prompt + half the generated tokens: the leg's mean KV length), every step
        # preceded by a one-row silu_mul launch (a kernel no decode step runs) that marks the step's
        # first dispatch for the FETCH_SIZE / WRITE_SIZE passes of profiles/decode_step_traffic.md
        from mindpipe_amd.decoder import DecoderConfig, W4Decoder
        mark = torch.zeros(1, 2, dtype=torch.float16, device="cuda")
        for cfg_name, batches, prompt, gen in (("llama2_7b", (1, 8, 32), 2048, 256),
                                               ("llama3_70b", (1, 16, 64), 4096, 64)):
            cfg = getattr(DecoderConfig, cfg_name)()
            for b in batches:
                model = W4Decoder(cfg, max_batch=b, max_len=prompt + gen + 8)
                g = torch.Generator(device="cuda").manual_seed(5)
                model.k_cache.normal_(0, 1, generator=g)
                model.v_cache.normal_(0, 1, generator=g)
                tok = torch.randint(0, cfg.vocab, (b,), device="cuda", generator=g)
                cur = torch.tensor([prompt + gen // 2], device="cuda", dtype=torch.int64)
                torch.cuda.synchronize()
                for _ in range(2):
                    ops.silu_mul(mark)
                    tok = model.decode_step(tok, cur)
                    cur.add_(1)
                ops.silu_mul(mark)
                torch.cuda.synchronize()
                print(f"decsteps {cfg_name} B={b} done", flush=True)
                del model
                torch.cuda.empty_cache()
    elif name == "w8big":
        gen = torch.Generator(device="cuda").manual_seed(1)
        qx = torch.randint(-127, 128, (4096, 4096), dtype=torch.int8, device="cuda", generator=gen)
        qw = torch.randint(-127, 128, (11008, 4096), dtype=torch.int8, device="cuda", generator=gen)
        st = torch.rand(4096, device="cuda") * 0.01
        sw = torch.rand(11008, device="cuda") * 0.001
        ms = _time_graph(lambda i: ops.w8a8_gemm(qx, st, qw, sw, None, torch.float16), 4, steps, 3) / 4
        print(f"w8big: {ms * 1e3:.1f} us per launch, {2 * 4096 * 11008 * 4096 / (ms * 1e-3) / 1e12:.1f} TOPS")
    else:
        raise SystemExit(f"unknown profile mix {name!r}")
    torch.cuda.synchronize()


def traffic_probe(ops):
    """Kernel mix for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE passes: a plain 256 MiB
    device copy (calibration of the counters) and the headline kernels."""
    src = torch.empty(256 * 1024 * 1024 // 4, dtype=torch.float32, device="cuda").fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    del src, dst
    gen = torch.Generator(device="cuda").manual_seed(1)
    w = (torch.randn(4096, 4096, generator=gen, device="cuda") * 0.02).half()
    packed, s, z, _ = ops.w4_quantize_awq(w, 128, True, return_deq=False)
    pk = [packed.clone() for _ in range(64)]
    sc = [s.clone() for _ in range(64)]
    zr = [z.clone() for _ in range(64)]
    x = torch.randn(1, 4096, device="cuda").half()
    for i in range(128):
        ops.w4a16_gemm(x, pk[i % 64], sc[i % 64], zr[i % 64], 128, None)
    x16 = torch.randn(16, 4096, device="cuda").half()
    for i in range(64):
        ops.w4a16_gemm(x16, pk[i], sc[i], zr[i], 128, None)
    del pk, sc, zr
    # the 70B decode GEMVs (M = 1): K = 8192, N = 28672 and K = 28672, N = 8192, 4 rotated copies each
    for n, k in ((28672, 8192), (8192, 28672)):
        pk, sc, zr = _w4_copies(ops, n, k, 4)
        xk = torch.randn(1, k, device="cuda").half()
        for i in range(8):
            ops.w4a16_gemm(xk, pk[i % 4], sc[i % 4], zr[i % 4], 128, None)
        del pk, sc, zr
    # the bf16 legs: M = 1 and M = 16 at K = N = 4096 (64 launches over 64 copies each), then
    # K = 8192, N = 28672 (8 launches over 4 copies)
    pk, sc, zr = _w4_copies(ops, 4096, 4096, 64, dtype=torch.bfloat16)
    for m in (1, 16):
        xb = torch.randn(m, 4096, device="cuda").bfloat16()
        for i in range(64):
            ops.w4a16_gemm(xb, pk[i], sc[i], zr[i], 128, None)
    del pk, sc, zr
    pk, sc, zr = _w4_copies(ops, 28672, 8192, 4, dtype=torch.bfloat16)
    xb = torch.randn(1, 8192, device="cuda").bfloat16()
    for i in range(8):
        ops.w4a16_gemm(xb, pk[i % 4], sc[i % 4], zr[i % 4], 128, None)
    del pk, sc, zr
    # the W8A8 sweep: M = 1, 16, 256 over 13 rotated weight copies (3 rounds), M = 4096 three times
    gen8 = torch.Generator(device="cuda").manual_seed(1)
    wcopies = [torch.randint(-127, 128, (11008, 4096), dtype=torch.int8, device="cuda", generator=gen8)
               for _ in range(13)]
    sw = torch.rand(11008, device="cuda")
    for m in (1, 16, 256, 4096):
        qx = torch.randint(-127, 128, (m, 4096), dtype=torch.int8, device="cuda", generator=gen8)
        st = torch.rand(m, device="cuda")
        for i in range(39 if m <= 256 else 3):
            ops.w8a8_gemm(qx, st, wcopies[i % 13], sw, None, torch.float16)
    del wcopies, qx
    # the 7B prefill's fused gate/up + SiLU-mul at M = 2048 (the prefill kernel's SwiGLU form)
    pk, sc, zr = _w4_copies(ops, 2 * 11008, 4096, 1)
    xp = torch.randn(2048, 4096, device="cuda").half()
    for _ in range(3):
        ops.w4a16_gemm_swiglu(xp, pk[0], sc[0], zr[0], 128, None)
    del pk, sc, zr, xp
    # the Mixtral MoE leg's whole chain on the bench leg's inputs (route + quant, GEMM1 + SwiGLU +
    # requant, GEMM2, combine), three calls
    mx = _moe_inputs(ops)
    for _ in range(3):
        ops.moe_w8a8_forward(*mx)
    del mx
    torch.cuda.synchronize()
    print("traffic probe done")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--legs", default="w4,w8,moe,dec7b,dec70b")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="run the kernel mix profiled for HBM traffic (profiles/traffic.json) and exit")
    ap.add_argument("--profile", default=None, help="run one kernel mix for rocprofv3 and exit")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the kernels run on one GPU's shard; no collectives are built)", file=sys.stderr)
        sys.exit(2)
    from mindpipe_amd import ops

    if args.traffic_probe:
        traffic_probe(ops)
        return
    if args.profile:
        profile_mix(ops, args.profile, args.steps)
        return
    legs = set(args.legs.split(","))
    steps, warmup = args.steps, args.warmup
    torch.cuda.init()
    dev = torch.cuda.get_device_properties(0)
    _log(f"device {dev.name} CUs={dev.multi_processor_count}")
    out_legs = {}
    _log("leg w4a16 M=1")
    head, _ = leg_w4a16(ops, 1, 4096, 4096, steps, warmup)
    head["roofline"]["traffic"] = _traffic("w4a16_gemv_m1_k4096_n4096")
    if "w4" in legs:
        _log("leg w4a16 M=16")
        out_legs["w4a16_m16_k4096_n4096"], _ = leg_w4a16(ops, 16, 4096, 4096, steps, warmup)
        out_legs["w4a16_m16_k4096_n4096"]["roofline"]["traffic"] = _traffic("w4a16_m16_k4096_n4096")
        _log("leg w4a16 70B shapes")
        small = max(2, steps // 4)
        for m, n, k in ((1, 28672, 8192), (1, 8192, 28672)):
            key = f"w4a16_m{m}_k{k}_n{n}"
            out_legs[key], _ = leg_w4a16(ops, m, n, k, small, max(1, warmup // 2), copies=8)
            out_legs[key]["roofline"]["traffic"] = _traffic(key)
        _log("leg w4a16 bf16")
        for m, n, k in ((1, 4096, 4096), (16, 4096, 4096), (1, 28672, 8192)):
            key = f"w4a16_bf16_m{m}_k{k}_n{n}"
            cp = 64 if n * k <= 4096 * 4096 else 8
            out_legs[key], _ = leg_w4a16(ops, m, n, k, steps if cp == 64 else small, max(1, warmup // 2), copies=cp,
                                         dtype=torch.bfloat16)
            out_legs[key]["roofline"]["traffic"] = _traffic(key)
    if "w8" in legs:
        for m in (4096, 256, 16, 1):
            _log(f"leg w8a8 M={m}")
            out_legs[f"w8a8_m{m}_k4096_n11008"] = leg_w8a8(ops, m, 11008, 4096, steps, max(1, warmup // 2))
    if "moe" in legs:
        _log("leg moe")
        out_legs["moe_w8a8_mixtral_t512"] = leg_moe(ops, max(3, steps // 2), max(1, warmup // 4))
    dec = None
    if "dec7b" in legs:
        _log("leg llama-2-7b-shaped W4A16 decode")
        dec = leg_decoder("llama2_7b", (1, 8, 32), prompt=2048, gen_tokens=256)
        out_legs["llama2_7b_w4a16"] = dec
    if "dec70b" in legs:
        _log("leg llama-3-70b-shaped W4A16 decode")
        out_legs["llama3_70b_w4a16"] = leg_decoder("llama3_70b", (1, 16, 64), prompt=4096, gen_tokens=64,
                                                   prefill_batch=0)
    cpu = None
    if not args.no_cpu_baseline:
        cpus = cpu_baselines(legs)
        cpu = cpus.pop("head")
        for key, v in cpus.items():
            if key in out_legs:
                out_legs[key]["cpu_baseline"] = v
    w8 = out_legs.get("w8a8_m4096_k4096_n11008")
    res = {
        "metric": METRIC,
        "value": round(head["tb_s"], 4),
        "unit": "TB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(head["ms_per_step"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u4*f16->f16",
        "data": "synthetic",
        "config": {"workload": "W4A16 g128 asym GEMV, M=1, K=N=4096, fp16 activations; a step is one pass over "
                               "64 distinct linears (64 rotated weight copies, one launch each)",
                   "m": 1, "k": 4096, "n": 4096, "group_size": 128, "launches_per_step": 64,
                   "working_set_bytes": head["working_set_bytes"], "us_per_launch": round(head["ms_per_call"] * 1e3, 3)},
        "roofline": head["roofline"],
        "cpu_baseline": cpu,
        "int8_tops_m4096": round(w8["tops"], 2) if w8 else None,
        "decode_7b_tok_s": {k: round(v["tok_s"], 1) for k, v in dec["decode"].items()} if dec else None,
        "decode_70b_tok_s": ({k: round(v["tok_s"], 1) for k, v in out_legs["llama3_70b_w4a16"]["decode"].items()}
                             if "llama3_70b_w4a16" in out_legs else None),
        "legs": out_legs,
        "device": dev.name,
    }
    print(json.dumps(res))


if __name__ == "__main__":
    main()
