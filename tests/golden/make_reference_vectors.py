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


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
