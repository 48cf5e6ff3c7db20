"""Write golden vectors of the reference quantizers at code widths other than W8A8 / W4.

Run in the build container only (the reference tree is not present on GPU boxes):
``python tests/golden/make_width_vectors.py /root/reference``.  It imports the reference's
own functions and modules, feeds them small seeded inputs and stores inputs and outputs in
``tests/golden/reference_width_vectors.npz``.  Only data is written; no reference source
is copied.

Functions exercised (reference paths):
* ``pseudo_quantize_tensor`` at n_bit 2, 3 and 8, with and without a zero point, fp16 and
  bf16, group 128 and per row
  (algorithm/quantization/ptq/awq/source/awq/quantize/quantizer.py:63-105);
* ``quantize_weight_per_channel_absmax`` / ``quantize_activation_per_token_absmax`` at
  n_bits 3, 4 and 6 in fp16 and bf16 (algorithm/quantization/ptq/smoothquant/source/
  smoothquant/fake_quant.py:10-31);
* ``SmoothQuantLinear.from_float`` + ``forward`` at W4A8, W8A4, W6A6 (output quant), W8A16,
  W16A8, W16A16 and W4A4 (output quant), fp16 and bf16 (fake_quant.py:38-121);
* ``SmoothQuantPackedMoeExperts`` at W4A4 / SiLU, W8A8 / tanh-GELU, W8A16 / SiLU and
  W6A6 / tanh-GELU, fp16 and bf16 (fake_quant.py:124-198).
"""
import sys
from pathlib import Path

import numpy as np
import torch


def bits(t):
    t = t.detach()
    return t.view(torch.int16).numpy() if t.dtype == torch.bfloat16 else t.numpy()


def main(ref_root):
    ref = Path(ref_root)
    sys.path.insert(0, str(ref))
    from torch import nn
    from algorithm.quantization.ptq.awq.source.awq.quantize.quantizer import pseudo_quantize_tensor
    from algorithm.quantization.ptq.smoothquant.source.smoothquant.fake_quant import (
        SmoothQuantLinear, SmoothQuantPackedMoeExperts, quantize_activation_per_token_absmax,
        quantize_weight_per_channel_absmax)

    gen = torch.Generator().manual_seed(2468)
    out = {}
    dts = ((torch.float16, "f16"), (torch.bfloat16, "bf16"))

    # AWQ at other widths: a constant group and a linear ramp among N(0, 0.02) rows
    for dt, tag in dts:
        w = torch.randn(24, 256, generator=gen) * 0.02
        w[0, :128] = 0.0
        w[1, 128:] = torch.linspace(-0.5, 0.5, 128)
        w = w.to(dt)
        out[f"awq_{tag}_w"] = bits(w)
        for n_bit in (2, 3, 8):
            for zp in (True, False):
                for g in (128, -1):
                    if g == -1 and n_bit != 3:
                        continue
                    key = f"awq_{tag}_n{n_bit}_zp{int(zp)}_g{g}"
                    if zp:
                        d, s, z = pseudo_quantize_tensor(w.clone(), n_bit=n_bit, zero_point=True, q_group_size=g,
                                                         get_scale_zp=True)
                        out[key + "_s"] = bits(s)
                        out[key + "_z"] = bits(z)
                    else:
                        d = pseudo_quantize_tensor(w.clone(), n_bit=n_bit, zero_point=False, q_group_size=g)
                    out[key + "_deq"] = bits(d)

    # per-channel / per-token fake quant at 3, 4 and 6 bits (outlier channels, a zero row)
    for dt, tag in dts:
        x = torch.randn(17, 192, generator=gen)
        x[:, torch.randperm(192, generator=gen)[:3]] *= 20
        x[2] = 0.0
        x = x.to(dt)
        wq = (torch.randn(40, 192, generator=gen) * 0.02).to(dt)
        out[f"fq_{tag}_x"] = bits(x)
        out[f"fq_{tag}_w"] = bits(wq)
        for n in (3, 4, 6):
            out[f"fq_{tag}_x_n{n}"] = bits(quantize_activation_per_token_absmax(x.clone(), n))
            out[f"fq_{tag}_w_n{n}"] = bits(quantize_weight_per_channel_absmax(wq.clone(), n))

    # SmoothQuantLinear at other widths
    cfgs = ((4, 8, False), (8, 4, False), (6, 6, True), (8, 16, False), (16, 8, False), (16, 16, False),
            (4, 4, True))
    for dt, tag in dts:
        lin = nn.Linear(256, 96, bias=True).to(dt)
        with torch.no_grad():
            lin.weight.copy_((torch.randn(96, 256, generator=gen) * 0.02).to(dt))
            lin.bias.copy_((torch.randn(96, generator=gen) * 0.1).to(dt))
        xi = torch.randn(2, 7, 256, generator=gen)
        xi[..., torch.randperm(256, generator=gen)[:3]] *= 20
        xi = xi.to(dt)
        out[f"lin_{tag}_w"] = bits(lin.weight)
        out[f"lin_{tag}_b"] = bits(lin.bias)
        out[f"lin_{tag}_x"] = bits(xi)
        for wb, ab, qo in cfgs:
            mod = SmoothQuantLinear.from_float(lin, wb, ab, quantize_output=qo)
            out[f"lin_{tag}_w{wb}a{ab}q{int(qo)}_y"] = bits(mod(xi.clone()))

    # packed MoE experts: E = 4, top-2, T = 24, H = 128, I = 64
    e, t, h, inter = 4, 24, 128, 64
    acts = {"silu": nn.SiLU(), "gelu_tanh": nn.GELU(approximate="tanh")}
    mcfgs = ((4, 4, "silu"), (8, 8, "gelu_tanh"), (8, 16, "silu"), (6, 6, "gelu_tanh"))
    for dt, tag in dts:
        gu = (torch.randn(e, 2 * inter, h, generator=gen) * 0.02).to(dt)
        dn = (torch.randn(e, h, inter, generator=gen) * 0.02).to(dt)
        x = torch.randn(t, h, generator=gen)
        x[:, torch.randperm(h, generator=gen)[:3]] *= 20
        x = x.to(dt)
        probs = torch.softmax(torch.randn(t, e, generator=gen), dim=-1)
        top_w, top_i = torch.topk(probs, 2, dim=-1)
        top_w = (top_w / top_w.sum(dim=-1, keepdim=True)).to(dt)
        out.update({f"moe_{tag}_gu": bits(gu), f"moe_{tag}_dn": bits(dn), f"moe_{tag}_x": bits(x),
                    f"moe_{tag}_ids": top_i.numpy().astype(np.int32), f"moe_{tag}_tw": bits(top_w)})
        for wb, ab, act in mcfgs:
            mod = SmoothQuantPackedMoeExperts(gu.clone(), dn.clone(), acts[act], weight_bits=wb, activation_bits=ab)
            out[f"moe_{tag}_w{wb}a{ab}_{act}_y"] = bits(mod(x.clone(), top_i.clone(), top_w.clone()))

    dst = Path(__file__).with_name("reference_width_vectors.npz")
    np.savez_compressed(dst, **out)
    print("wrote", dst, len(out), "arrays")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
