"""Write golden vectors by running the reference's own Python quantizers.

Run in the build container only (the reference tree is not present on GPU
boxes):  ``python tests/golden/make_reference_vectors.py /root/reference``.
It imports the reference functions named below, feeds them small seeded
inputs (plus tie-heavy rows), and stores inputs and outputs in
``tests/golden/reference_vectors.npz``.  Only data is written; no reference
source is copied.

Functions exercised (reference paths):
* ``pseudo_quantize_tensor``  algorithm/quantization/ptq/awq/source/awq/quantize/quantizer.py:63-105
* ``quantize_activation_per_token_absmax`` / ``quantize_weight_per_channel_absmax``
  algorithm/quantization/ptq/smoothquant/source/smoothquant/fake_quant.py:10-31
* ``quantize_weight_per_channel``  scripts/repro/export_fp16_to_ascend_w8a8_dynamic_probe.py:175-195
* ``pack_int4_for_vllm``  algorithm/quantization/exporters/vllm.py:89-111
* ``Quantizer`` + ``quantize_with_qint``  algorithm/quantization/ptq/gptq/source/quant.py:6-137

A second file, ``reference_ext_vectors.npz`` (``write_ext``), holds what the
checks above leave open:
* ``SmoothQuantPackedMoeExperts`` construction + ``forward`` in fp16 and bf16
  (fake_quant.py:124-191), the MoE forward the oracle's ``moe_fake`` restates;
* the bf16 arithmetic of ``pseudo_quantize_tensor`` (quantizer.py:63-105) and of
  ``quantize_activation_per_token_absmax`` / ``quantize_weight_per_channel_absmax``
  (fake_quant.py:10-31), and ``SmoothQuantLinear`` forward in fp16 / bf16
  (fake_quant.py:85-113);
* ``_compute_smooth_scales`` (smooth.py:7-25) on fp16 and bf16 weights.
"""
import importlib.util
import sys
from pathlib import Path

import numpy as np
import torch


def _load(path, name):
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def main(ref_root):
    ref = Path(ref_root)
    sys.path.insert(0, str(ref))
    from algorithm.quantization.ptq.awq.source.awq.quantize.quantizer import pseudo_quantize_tensor
    from algorithm.quantization.ptq.smoothquant.source.smoothquant.fake_quant import (
        quantize_activation_per_token_absmax, quantize_weight_per_channel_absmax)
    from algorithm.quantization.exporters.vllm import pack_int4_for_vllm
    probe = _load(ref / "scripts/repro/export_fp16_to_ascend_w8a8_dynamic_probe.py", "w8probe")
    gq = _load(ref / "algorithm/quantization/ptq/gptq/source/quant.py", "gptq_quant")

    gen = torch.Generator().manual_seed(1234)
    out = {}
    # AWQ asym g128 on N(0, 0.02) plus rows with ties / constant groups / per-row fallback
    w = (torch.randn(48, 512, generator=gen) * 0.02).half()
    w[0, :128] = 0.0                       # constant group
    w[1, :128] = torch.linspace(-1, 1, 128).half()
    w[2, 128:256] = (torch.arange(128) % 16).half() * 0.0625
    wd, s, z = pseudo_quantize_tensor(w.clone(), n_bit=4, zero_point=True, q_group_size=128, get_scale_zp=True)
    out.update(awq_w=w.numpy(), awq_deq=wd.numpy(), awq_s=s.numpy(), awq_z=z.numpy())
    w2 = (torch.randn(8, 200, generator=gen) * 0.02).half()   # 200 % 128 != 0 -> per-row
    wd2, s2, z2 = pseudo_quantize_tensor(w2.clone(), n_bit=4, zero_point=True, q_group_size=128, get_scale_zp=True)
    out.update(awq_w_row=w2.numpy(), awq_deq_row=wd2.numpy(), awq_s_row=s2.numpy(), awq_z_row=z2.numpy())
    wd3 = pseudo_quantize_tensor(w.clone(), n_bit=4, zero_point=False, q_group_size=128)
    out.update(awq_sym_deq=wd3.numpy())

    # SmoothQuant fake per-token / per-channel, with outliers and exact-tie rows
    x = torch.randn(32, 384, generator=gen)
    x[:, torch.randperm(384, generator=gen)[:4]] *= 20
    x = x.half()
    x[3] = (torch.arange(384) - 192).half() * 0.5     # many .5 ties after scaling
    x[4] = 0.0
    out.update(sq_x=x.numpy(), sq_x_fq=quantize_activation_per_token_absmax(x.clone(), 8).numpy())
    wsq = (torch.randn(40, 384, generator=gen) * 0.02).half()
    out.update(sq_w=wsq.numpy(), sq_w_fq=quantize_weight_per_channel_absmax(wsq.clone(), 8).numpy())

    # Ascend export quantizer, fp16 and bf16 sources
    q, sc, off = probe.quantize_weight_per_channel(wsq.clone())
    out.update(ex_q=q.numpy(), ex_s=sc.numpy(), ex_off=off.numpy())
    wb = (torch.randn(24, 256, generator=gen) * 0.05).bfloat16()
    qb, sb, _ = probe.quantize_weight_per_channel(wb.clone())
    out.update(ex_wb_bits=wb.view(torch.int16).numpy(), ex_qb=qb.numpy(), ex_sb_bits=sb.view(torch.int16).numpy())

    # pack_int4_for_vllm on random signed ints with padding
    iw = torch.randint(-8, 8, (16, 77), generator=gen, dtype=torch.int8)
    out.update(pack_in=iw.numpy(), pack_out=pack_int4_for_vllm(iw).numpy())

    # GPTQ RTN: Quantizer(perchannel, sym) per 128-column group + quantize_with_qint
    wg = torch.randn(12, 256, generator=gen) * 0.03
    wg[0, :128] = wg[0, :128].abs()        # all-positive group keeps xmin = 0
    wg[1, 128:] = 0.0                      # all-zero group
    ints, scales = [], []
    for gi in range(2):
        quant = gq.Quantizer()
        quant.configure(4, perchannel=True, sym=True, mse=False)
        quant.find_params(wg[:, gi * 128:(gi + 1) * 128], weight=True)
        _, qint = gq.quantize_with_qint(wg[:, gi * 128:(gi + 1) * 128], quant.scale, quant.zero, quant.maxq)
        ints.append((qint.float() - quant.zero).to(torch.int8))
        scales.append(quant.scale.reshape(-1).float())
    out.update(gptq_w=wg.numpy(), gptq_int=torch.cat(ints, 1).numpy(),
               gptq_scale=torch.stack(scales, 1).half().numpy())

    dst = Path(__file__).with_name("reference_vectors.npz")
    np.savez_compressed(dst, **out)
    print("wrote", dst, {k: v.shape for k, v in out.items()})


def write_ext(ref_root):
    ref = Path(ref_root)
    if str(ref) not in sys.path:
        sys.path.insert(0, str(ref))
    from torch import nn
    from algorithm.quantization.ptq.awq.source.awq.quantize.quantizer import pseudo_quantize_tensor
    from algorithm.quantization.ptq.smoothquant.source.smoothquant.fake_quant import (
        SmoothQuantLinear, SmoothQuantPackedMoeExperts, quantize_activation_per_token_absmax,
        quantize_weight_per_channel_absmax)
    from algorithm.quantization.ptq.smoothquant.source.smoothquant.smooth import _compute_smooth_scales

    gen = torch.Generator().manual_seed(4321)
    out = {}

    def bits(t):
        t = t.detach()
        return t.view(torch.int16).numpy() if t.dtype == torch.bfloat16 else t.numpy()

    # MoE forward: E = 4 experts, top-2, T = 48 tokens, H = 128, I = 96, SiLU; router weights
    # fp32 (softmax -> top-k -> renormalise, as the HF router returns them).  Token 0 is all
    # zeros; expert 3 is hit by one token only.
    e, t, h, inter = 4, 48, 128, 96
    for dt, tag in ((torch.float16, "f16"), (torch.bfloat16, "bf16")):
        gu = (torch.randn(e, 2 * inter, h, generator=gen) * 0.02).to(dt)
        dn = (torch.randn(e, h, inter, generator=gen) * 0.02).to(dt)
        x = torch.randn(t, h, generator=gen)
        x[:, torch.randperm(h, generator=gen)[:3]] *= 20
        x[0] = 0.0
        x = x.to(dt)
        logits = torch.randn(t, e, generator=gen)
        probs = torch.softmax(logits, dim=-1)
        top_w, top_i = torch.topk(probs[:, :3], 2, dim=-1)
        top_i[5, 1] = 3                      # the only token of expert 3
        top_w = top_w / top_w.sum(dim=-1, keepdim=True)
        mod = SmoothQuantPackedMoeExperts(gu.clone(), dn.clone(), nn.SiLU())
        y = mod(x.clone(), top_i.clone(), top_w.clone())
        out.update({f"moe_{tag}_gu": bits(gu), f"moe_{tag}_dn": bits(dn), f"moe_{tag}_x": bits(x),
                    f"moe_{tag}_ids": top_i.numpy().astype(np.int32), f"moe_{tag}_w": top_w.numpy(),
                    f"moe_{tag}_y": bits(y)})

    # bf16 AWQ asym g128 (plus a constant group) and the symmetric branch
    w = (torch.randn(32, 512, generator=gen) * 0.02).bfloat16()
    w[0, :128] = 0.0
    w[1, :128] = torch.linspace(-1, 1, 128).bfloat16()
    wd, s, z = pseudo_quantize_tensor(w.clone(), n_bit=4, zero_point=True, q_group_size=128, get_scale_zp=True)
    out.update(awqb_w=bits(w), awqb_deq=bits(wd), awqb_s=bits(s), awqb_z=bits(z))
    out.update(awqb_sym_deq=bits(pseudo_quantize_tensor(w.clone(), n_bit=4, zero_point=False, q_group_size=128)))

    # bf16 fake per-token / per-channel quantizers (outliers, ties, a zero row)
    x = torch.randn(32, 384, generator=gen)
    x[:, torch.randperm(384, generator=gen)[:4]] *= 20
    x = x.bfloat16()
    x[3] = ((torch.arange(384) - 192) * 0.5).bfloat16()
    x[4] = 0.0
    out.update(sqb_x=bits(x), sqb_x_fq=bits(quantize_activation_per_token_absmax(x.clone(), 8)))
    wsq = (torch.randn(40, 384, generator=gen) * 0.02).bfloat16()
    out.update(sqb_w=bits(wsq), sqb_w_fq=bits(quantize_weight_per_channel_absmax(wsq.clone(), 8)))

    # SmoothQuantLinear.from_float + forward (fake path) in fp16 and bf16, with bias
    for dt, tag in ((torch.float16, "f16"), (torch.bfloat16, "bf16")):
        lin = nn.Linear(384, 200, bias=True).to(dt)
        with torch.no_grad():
            lin.weight.copy_((torch.randn(200, 384, generator=gen) * 0.02).to(dt))
            lin.bias.copy_((torch.randn(200, generator=gen) * 0.1).to(dt))
        xi = torch.randn(24, 384, generator=gen)
        xi[:, torch.randperm(384, generator=gen)[:4]] *= 20
        xi = xi.to(dt)
        sq = SmoothQuantLinear.from_float(lin, 8, 8, quantize_output=False)
        sqo = SmoothQuantLinear.from_float(lin, 8, 8, quantize_output=True)
        out.update({f"sql_{tag}_w": bits(lin.weight.detach()), f"sql_{tag}_b": bits(lin.bias.detach()),
                    f"sql_{tag}_x": bits(xi), f"sql_{tag}_y": bits(sq(xi.clone())),
                    f"sql_{tag}_yq": bits(sqo(xi.clone()))})

    # _compute_smooth_scales: two fcs sharing a norm, calibration abs-max in fp32 (with outliers)
    for dt, tag in ((torch.float16, "f16"), (torch.bfloat16, "bf16")):
        fcs = [nn.Linear(256, 96, bias=False).to(dt), nn.Linear(256, 64, bias=False).to(dt)]
        with torch.no_grad():
            for fc in fcs:
                fc.weight.copy_((torch.randn(fc.weight.shape, generator=gen) * 0.02).to(dt))
            fcs[0].weight[:, 7] = 0.0     # a column whose weight max hits the 1e-5 clamp
            fcs[1].weight[:, 7] = 0.0
        a = torch.randn(256, generator=gen).abs() * 3
        a[torch.randperm(256, generator=gen)[:5]] *= 30
        _, sc = _compute_smooth_scales(fcs, a.clone(), 0.5)
        out.update({f"smooth_{tag}_w0": bits(fcs[0].weight.detach()), f"smooth_{tag}_w1": bits(fcs[1].weight.detach()),
                    f"smooth_{tag}_a": a.numpy(), f"smooth_{tag}_s": bits(sc)})

    dst = Path(__file__).with_name("reference_ext_vectors.npz")
    np.savez_compressed(dst, **out)
    print("wrote", dst, {k: v.shape for k, v in out.items()})


if __name__ == "__main__":
    root = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    main(root)
    write_ext(root)
