"""GPU tests of the reference-compatible module API (SmoothQuant, AWQ/GPTQ W4, runtime
contract, export/load) against the numpy oracle.  Bars: codes bit-exact; outputs
rel. Frobenius error <= 1e-3 against the oracle's dequant -> matmul."""
import json
import sys
from pathlib import Path

import numpy as np
import pytest
import torch
from torch import nn

from oracle import quant as O

pytestmark = pytest.mark.gpu
GOLD = np.load(Path(__file__).parent / "golden" / "reference_vectors.npz")
EXT = np.load(Path(__file__).parent / "golden" / "reference_ext_vectors.npz")
DEV = "cuda:0"


def _say(*a):
    print(*a, flush=True)


def _rel(y, ref):
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.linalg.norm(y - ref) / max(np.linalg.norm(ref), 1e-30))


def _lin(n, k, bias=True, seed=1):
    torch.manual_seed(seed)
    lin = nn.Linear(k, n, bias=bias)
    with torch.no_grad():
        lin.weight.normal_(0, 0.02)
        if bias:
            lin.bias.normal_(0, 0.1)
    return lin.half().to(DEV)


# ------------------------------------------------------------------ SmoothQuant
def test_fake_quant_functions_match_reference_values():
    _say("fake quant fns")
    from mindpipe_amd.smoothquant import quantize_activation_per_token_absmax, quantize_weight_per_channel_absmax
    fx = quantize_activation_per_token_absmax(torch.from_numpy(GOLD["sq_x"]).to(DEV)).cpu().numpy()
    assert np.array_equal(fx, GOLD["sq_x_fq"])
    fw = quantize_weight_per_channel_absmax(torch.from_numpy(GOLD["sq_w"]).to(DEV)).cpu().numpy()
    assert np.array_equal(fw, GOLD["sq_w_fq"])
    x = torch.randn(3, 8, device=DEV).half()
    assert quantize_activation_per_token_absmax(x, 16) is x


@pytest.mark.parametrize("m,bias,qout", [(1, True, False), (16, False, False), (7, True, True), (300, True, False)])
def test_smoothquant_linear_matches_reference_fake_path(m, bias, qout):
    _say("SmoothQuantLinear", m, bias, qout)
    from mindpipe_amd.smoothquant import SmoothQuantLinear
    lin = _lin(384, 512, bias)
    mod = SmoothQuantLinear.from_float(lin, quantize_output=qout)
    assert repr(mod) == ("SmoothQuantLinear(512, 384, bias=%s, weight_bits=8, activation_bits=8, "
                         "weight_quant=per_channel, act_quant=per_token, output_quant=%s)"
                         % (bias, "per_token" if qout else "none"))
    w = lin.weight.detach().cpu().numpy()
    qw, _, _ = O.quantize_weight_per_channel_fake(w)
    assert np.array_equal(mod.weight.cpu().numpy(), qw)
    x = torch.randn(m, 512, generator=torch.Generator().manual_seed(0)).half()
    ref = O.w8a8_linear_fake(x.numpy(), w, lin.bias.detach().cpu().numpy() if bias else None)
    if qout:
        # output fake-quant re-rounds y: a 1-ulp difference in y can move a code by one
        # step, so check the linear before it (<= 1e-3) and the output quantizer
        # bit-exactly on the module's own pre-quant output
        mod.output_quant_name = "none"
        y_pre = mod(x.to(DEV))
        mod.output_quant_name = "per_token"
        assert _rel(y_pre.float().cpu().numpy(), ref.astype(np.float32)) <= 1e-3
        y = mod(x.to(DEV)).cpu().numpy()
        assert np.array_equal(y, O.quantize_activation_per_token_fake(y_pre.cpu().numpy())[2])
    else:
        y = mod(x.to(DEV)).float().cpu().numpy()
        assert _rel(y, ref.astype(np.float32)) <= 1e-3
    # 3-D input keeps its leading shape
    y3 = mod(x.to(DEV).reshape(1, m, 512))
    assert y3.shape == (1, m, 384)


def test_quantize_model_tiny_llama_names_and_forward():
    _say("quantize_model llama")
    from transformers import LlamaConfig, LlamaForCausalLM
    from mindpipe_amd.smoothquant import SmoothQuantLinear, quantize_model
    torch.manual_seed(0)
    cfg = LlamaConfig(hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=4,
                      num_key_value_heads=4, vocab_size=512)
    model = LlamaForCausalLM(cfg).half().to(DEV).eval()
    ids = torch.randint(0, 512, (1, 12), device=DEV)
    with torch.no_grad():
        ref = model(ids).logits.float()
    names = quantize_model(model)
    exp = []
    for i in range(2):
        exp += [f"model.layers.{i}.self_attn.{p}" for p in ("q_proj", "k_proj", "v_proj", "o_proj")]
        exp += [f"model.layers.{i}.mlp.{p}" for p in ("gate_proj", "up_proj", "down_proj")]
    assert names == exp
    assert isinstance(model.model.layers[0].self_attn.q_proj, SmoothQuantLinear)
    assert model.model.layers[0].self_attn.q_proj.output_quant_name == "per_token"
    assert model.model.layers[0].self_attn.o_proj.output_quant_name == "none"
    with torch.no_grad():
        out = model(ids).logits.float()
    cos = torch.nn.functional.cosine_similarity(out.flatten(), ref.flatten(), dim=0).item()
    assert cos > 0.99, cos


def test_quantize_model_tiny_mixtral_packed_experts():
    """Mixtral is outside the reference's allow-list: rejected by default, accepted as an
    extension (packed experts like qwen3_moe).  The packed experts follow the reference
    module's fake-quant forward (oracle.moe_fake) by default and the fp32 runtime chain
    (oracle.moe_runtime) with scale_rule="export"."""
    _say("quantize_model mixtral")
    from transformers import MixtralConfig, MixtralForCausalLM
    from mindpipe_amd.smoothquant import SmoothQuantPackedMoeExperts, quantize_model
    torch.manual_seed(0)
    cfg = MixtralConfig(hidden_size=256, intermediate_size=384, num_hidden_layers=1, num_attention_heads=4,
                        num_key_value_heads=2, vocab_size=512, num_local_experts=4, num_experts_per_tok=2)
    model = MixtralForCausalLM(cfg).half().to(DEV).eval()
    with pytest.raises(ValueError, match="Unsupported model type"):
        quantize_model(model)
    experts = model.model.layers[0].mlp.experts
    gu = experts.gate_up_proj.detach().clone()
    dn = experts.down_proj.detach().clone()
    names = quantize_model(model, allow_extension_models=True)
    assert names[-2:] == ["model.layers.0.mlp.experts.gate_up_proj", "model.layers.0.mlp.experts.down_proj"]
    mod = model.model.layers[0].mlp.experts
    assert isinstance(mod, SmoothQuantPackedMoeExperts)
    assert repr(mod) == ("SmoothQuantPackedMoeExperts(num_experts=4, hidden_dim=256, intermediate_dim=384, "
                         "weight_bits=8, activation_bits=8)")
    t = 40
    x = torch.randn(t, 256, generator=torch.Generator().manual_seed(1)).half()
    ids, tw = O.mixtral_router(np.random.default_rng(2).standard_normal((t, 4)).astype(np.float32), 2)
    y = mod(x.to(DEV), torch.from_numpy(ids).to(DEV), torch.from_numpy(tw).to(DEV)).float().cpu().numpy()
    gun, dnn = gu.cpu().numpy(), dn.cpu().numpy()
    gq, dq = mod.dequantized_weights()   # values (int8 codes carry no sign of zero)
    assert np.array_equal(gq.float().cpu().numpy(),
                          np.stack([O.quantize_weight_per_channel_fake(gun[e])[2] for e in range(4)]).astype(np.float32))
    ref = O.moe_fake(x.numpy(), ids, tw, gun, dnn)
    assert _rel(y, ref.astype(np.float32)) <= 1e-3
    # the runtime rule: export-rule codes and the fp32 chain
    modr = SmoothQuantPackedMoeExperts(gu, dn, torch.nn.SiLU(), scale_rule="export")
    yr = modr(x.to(DEV), torch.from_numpy(ids).to(DEV), torch.from_numpy(tw).to(DEV)).float().cpu().numpy()
    q13 = np.stack([O.quantize_weight_per_channel_export(gun[e])[0] for e in range(4)])
    s13 = np.stack([O.quantize_weight_per_channel_export(gun[e])[1] for e in range(4)])
    q2 = np.stack([O.quantize_weight_per_channel_export(dnn[e])[0] for e in range(4)])
    s2 = np.stack([O.quantize_weight_per_channel_export(dnn[e])[1] for e in range(4)])
    assert np.array_equal(modr.gate_up_proj.cpu().numpy(), q13)
    assert _rel(yr, O.moe_runtime(x.numpy(), ids, tw, q13, s13, q2, s2).astype(np.float32)) <= 1e-3
    with torch.no_grad():
        model(torch.randint(0, 512, (1, 9), device=DEV))


@pytest.mark.parametrize("tag,dt", [("f16", "fp16"), ("bf16", "bf16")])
def test_smoothquant_linear_matches_reference_outputs(tag, dt):
    """SmoothQuantLinear.from_float + forward in fp16 and bf16 against the outputs the
    reference module wrote (fake_quant.py:85-113): rel. Frobenius error <= 1e-3; with the
    output fake-quant, the module's output is the fake rule applied to its own linear output."""
    _say("SmoothQuantLinear fixture", dt)
    from mindpipe_amd.smoothquant import SmoothQuantLinear
    tdt = torch.float16 if dt == "fp16" else torch.bfloat16

    def cv(a):
        t = torch.from_numpy(np.ascontiguousarray(a))
        return (t if dt == "fp16" else t.view(torch.bfloat16)).to(DEV)

    def f32(t):
        return t.float().cpu().numpy()

    w, b, x = cv(EXT[f"sql_{tag}_w"]), cv(EXT[f"sql_{tag}_b"]), cv(EXT[f"sql_{tag}_x"])
    lin = nn.Linear(w.shape[1], w.shape[0], bias=True).to(device=DEV, dtype=tdt)
    with torch.no_grad():
        lin.weight.copy_(w)
        lin.bias.copy_(b)
    ref = cv(EXT[f"sql_{tag}_y"])
    mod = SmoothQuantLinear.from_float(lin)
    y = mod(x)
    assert y.dtype == tdt
    assert _rel(f32(y), f32(ref)) <= 1e-3     # bar: rel. Frobenius error <= 1e-3
    modq = SmoothQuantLinear.from_float(lin, quantize_output=True)
    yq = modq(x)
    from mindpipe_amd.smoothquant import quantize_activation_per_token_absmax
    assert torch.equal(yq, quantize_activation_per_token_absmax(y))
    assert _rel(f32(yq), f32(cv(EXT[f"sql_{tag}_yq"]))) <= 1e-2   # re-quantized: a code step is 1/127


def test_runtime_fused_experts_contract():
    """fused_experts_w8a8 on the runtime's loaded layout (w13 [E,H,2I], w2 [E,I,H], bf16 scales),
    a pre-quantized input with pertoken_scale, and an expert_map; grouped_apply_mlp_w8a8 with
    group_list types 0 and 1 (vllm_ascend.patch:2015-2031, 2278-2291, 4447-4468)."""
    _say("runtime fused_experts")
    from mindpipe_amd.runtime import dynamic_quant, fused_experts_w8a8, grouped_apply_mlp_w8a8
    from mindpipe_amd import ops
    rng = np.random.default_rng(8)
    t, h, inter, e = 64, 256, 192, 4
    x = rng.standard_normal((t, h)).astype(np.float16)
    ids, tw = O.mixtral_router(rng.standard_normal((t, e)).astype(np.float32), 2)
    gu = (rng.standard_normal((e, 2 * inter, h)) * 0.02).astype(np.float16)
    dn = (rng.standard_normal((e, h, inter)) * 0.02).astype(np.float16)
    q13 = np.stack([O.quantize_weight_per_channel_export(gu[i])[0] for i in range(e)])
    s13 = np.stack([O.quantize_weight_per_channel_export(gu[i])[1] for i in range(e)])
    q2 = np.stack([O.quantize_weight_per_channel_export(dn[i])[0] for i in range(e)])
    s2 = np.stack([O.quantize_weight_per_channel_export(dn[i])[1] for i in range(e)])
    # runtime layout with bf16 scales: the oracle sees the bf16-rounded scales
    s13b = O.bf16_bits_to_f32(O.f32_to_bf16_bits(s13))
    s2b = O.bf16_bits_to_f32(O.f32_to_bf16_bits(s2))
    w13_rt = torch.from_numpy(np.ascontiguousarray(q13.transpose(0, 2, 1))).to(DEV)
    w2_rt = torch.from_numpy(np.ascontiguousarray(q2.transpose(0, 2, 1))).to(DEV)
    sc13 = torch.from_numpy(s13).to(DEV).bfloat16()
    sc2 = torch.from_numpy(s2).to(DEV).bfloat16()
    xt, idt, twt = torch.from_numpy(x).to(DEV), torch.from_numpy(ids).to(DEV), torch.from_numpy(tw).to(DEV)
    y = fused_experts_w8a8(xt, w13_rt, sc13, w2_rt, sc2, twt, idt)
    ref = O.moe_runtime(x, ids, tw, q13, s13b, q2, s2b)
    assert np.array_equal(y.cpu().numpy().view(np.uint16), ref.view(np.uint16)) or \
        _rel(y.float().cpu().numpy(), ref.astype(np.float32)) <= 1e-3
    # pre-quantized input: the same bits as quantizing inside
    qx, sx = dynamic_quant(xt)
    y2 = fused_experts_w8a8(qx, w13_rt, sc13, w2_rt, sc2, twt, idt, pertoken_scale=sx, output_dtype=torch.float16)
    assert torch.equal(y, y2)
    # expert_map: experts 2, 3 live elsewhere (-1); their assignments contribute nothing
    emap = torch.tensor([0, 1, -1, -1], dtype=torch.int32, device=DEV)
    y3 = fused_experts_w8a8(xt, w13_rt[:2], sc13[:2], w2_rt[:2], sc2[:2], twt, idt, expert_map=emap)
    tw_loc = np.where(ids < 2, tw, 0).astype(np.float32)
    ref3 = O.moe_runtime(x, np.where(ids < 2, ids, 0).astype(np.int32), tw_loc, q13, s13b, q2, s2b)
    assert _rel(y3.float().cpu().numpy(), ref3.astype(np.float32)) <= 1e-3
    # grouped MLP over pre-permuted rows, group_list as cumulative endpoints (0) or counts (1)
    routed, rscale, row_of_slot, offs = ops.moe_permute_quant(xt, idt, e)
    counts = torch.diff(offs)
    outs = [grouped_apply_mlp_w8a8(routed, w13_rt, sc13, w2_rt, sc2, gl, glt, dynamic_scale=rscale,
                                   output_dtype=torch.float32)
            for gl, glt in ((offs[1:], 0), (counts, 1))]
    assert torch.equal(outs[0], outs[1])
    yk = ops.moe_gmm2(*ops.moe_gmm1_swiglu_quant(routed, rscale, torch.from_numpy(q13).to(DEV),
                                                 torch.from_numpy(s13b).to(DEV), offs, inter),
                      torch.from_numpy(q2).to(DEV), torch.from_numpy(s2b).to(DEV), offs)
    assert torch.equal(outs[0], yk)
    with pytest.raises(ValueError):
        grouped_apply_mlp_w8a8(routed, w13_rt, sc13, w2_rt, sc2, counts, 2, dynamic_scale=rscale)


def test_runtime_moe_layers_convert_each_weight_once():
    """48 MoE layers' worth of distinct weights (Qwen3-30B-A3B has 48), called as the reference
    runtime calls ``fused_experts`` (``vllm_ascend.patch:4447-4468``: ``w1 [E,H,2I]``,
    ``w2 [E,I,H]``, no layout argument), twice per layer: each weight is re-laid at most once
    and every output is bit-exact against the oracle's runtime chain.  Layers processed by
    ``W8A8DynamicFusedMoEMethod.process_weights_after_loading`` (loaded ``[E,2I,H]`` /
    ``[E,H,I]``) convert nothing, and their ``apply`` gives the same bits."""
    _say("runtime moe 48 layers")
    from mindpipe_amd.runtime import W8A8DynamicFusedMoEMethod, fused_experts_w8a8, layout_conversions
    rng = np.random.default_rng(48)
    t, h, inter, e, layers = 40, 128, 192, 4, 48
    x = rng.standard_normal((t, h)).astype(np.float16)
    ids, tw = O.mixtral_router(rng.standard_normal((t, e)).astype(np.float32), 2)
    xt, idt, twt = torch.from_numpy(x).to(DEV), torch.from_numpy(ids).to(DEV), torch.from_numpy(tw).to(DEV)

    class Layer(nn.Module):
        pass

    stack = []
    for li in range(layers):
        gu = (rng.standard_normal((e, 2 * inter, h)) * 0.02).astype(np.float16)
        dn = (rng.standard_normal((e, h, inter)) * 0.02).astype(np.float16)
        q13, s13 = (np.stack(v) for v in zip(*[O.quantize_weight_per_channel_export(gu[i])[:2] for i in range(e)]))
        q2, s2 = (np.stack(v) for v in zip(*[O.quantize_weight_per_channel_export(dn[i])[:2] for i in range(e)]))
        stack.append((q13, s13, q2, s2))
    base = layout_conversions()
    w_rt = [(torch.from_numpy(np.ascontiguousarray(q13.transpose(0, 2, 1))).to(DEV),
             torch.from_numpy(np.ascontiguousarray(q2.transpose(0, 2, 1))).to(DEV)) for q13, _, q2, _ in stack]
    first, exact = [], 0
    for rep in range(2):
        for li, (q13, s13, q2, s2) in enumerate(stack):
            w13, w2 = w_rt[li]
            y = fused_experts_w8a8(xt, w13, torch.from_numpy(s13).to(DEV), w2, torch.from_numpy(s2).to(DEV), twt, idt)
            yn = y.cpu().numpy()
            if rep == 0:
                ref = O.moe_runtime(x, ids, tw, q13, s13, q2, s2)
                # silu's exp is correctly rounded on neither side: a requant code may differ by one
                same = np.array_equal(yn.view(np.uint16), ref.view(np.uint16))
                exact += same
                assert same or _rel(yn.astype(np.float32), ref.astype(np.float32)) <= 1e-3, li
                first.append(yn)
            else:   # the re-laid weights give the same bits as the first call
                assert np.array_equal(yn.view(np.uint16), first[li].view(np.uint16)), li
            assert w13.shape == (e, h, 2 * inter) and torch.equal(w13.cpu(), torch.from_numpy(q13.transpose(0, 2, 1)))
        assert layout_conversions() - base == 2 * layers
    _say("bit-exact layers", exact, "of", layers)
    assert exact >= layers // 2
    # the method's own loading path: no conversion at all
    meth = W8A8DynamicFusedMoEMethod(torch.float16)
    base = layout_conversions()
    for li, (q13, s13, q2, s2) in enumerate(stack[:4]):
        layer = Layer()
        layer.w13_weight = nn.Parameter(torch.from_numpy(q13).to(DEV), requires_grad=False)
        layer.w2_weight = nn.Parameter(torch.from_numpy(q2).to(DEV), requires_grad=False)
        layer.w13_weight_scale = nn.Parameter(torch.from_numpy(s13).half().reshape(e, -1, 1).to(DEV),
                                              requires_grad=False)
        layer.w2_weight_scale = nn.Parameter(torch.from_numpy(s2).half().reshape(e, -1, 1).to(DEV),
                                             requires_grad=False)
        layer.w13_weight_offset = nn.Parameter(torch.zeros(e, 2 * inter, 1, device=DEV), requires_grad=False)
        layer.w2_weight_offset = nn.Parameter(torch.zeros(e, h, 1, device=DEV), requires_grad=False)
        meth.process_weights_after_loading(layer)
        assert layer.w13_weight.shape == (e, h, 2 * inter) and layer.w2_weight.shape == (e, inter, h)
        assert layer.w13_weight_scale.shape == (e, 2 * inter) and layer.w2_weight_scale_fp32.dtype == torch.float32
        y = meth.apply(layer, xt, twt, idt)
        s13h = layer.w13_weight_scale_fp32.cpu().numpy()
        s2h = layer.w2_weight_scale_fp32.cpu().numpy()
        ref = O.moe_runtime(x, ids, tw.astype(np.float16).astype(np.float32), q13, s13h, q2, s2h)
        yn = y.cpu().numpy()
        assert np.array_equal(yn.view(np.uint16), ref.view(np.uint16)) or \
            _rel(yn.astype(np.float32), ref.astype(np.float32)) <= 1e-3, li
    assert layout_conversions() == base
    with pytest.raises(ValueError):   # kernel-layout weights are not the runtime contract
        fused_experts_w8a8(xt, torch.from_numpy(stack[0][0]).to(DEV), torch.from_numpy(stack[0][1]).to(DEV),
                           torch.from_numpy(stack[0][2]).to(DEV), torch.from_numpy(stack[0][3]).to(DEV), twt, idt)


def test_runtime_apply_contract():
    _say("runtime apply")
    from mindpipe_amd.runtime import W8A8DynamicLinearMethod, dynamic_quant, fused_experts_w8a8
    w = torch.randn(256, 512, generator=torch.Generator().manual_seed(1)) * 0.02
    q, s32, s16, off = O.quantize_weight_per_channel_export(w.half().numpy())

    class Layer(nn.Module):
        pass

    layer = Layer()
    layer.weight = nn.Parameter(torch.from_numpy(q).to(DEV), requires_grad=False)
    layer.weight_scale = nn.Parameter(torch.from_numpy(s16).reshape(-1, 1).to(DEV), requires_grad=False)
    layer.weight_offset = nn.Parameter(torch.zeros(256, 1, dtype=torch.float16, device=DEV), requires_grad=False)
    meth = W8A8DynamicLinearMethod()
    meth.process_weights_after_loading(layer)
    assert layer.weight_scale.shape == (256,) and layer.weight_scale_fp32.dtype == torch.float32
    x = torch.randn(2, 5, 512, generator=torch.Generator().manual_seed(0)).half()
    y = meth.apply(layer, x.to(DEV))
    assert y.shape == (2, 5, 256) and y.dtype == torch.float16
    rq, rs = O.quantize_per_token_runtime(x.reshape(10, 512).numpy())
    ref = O.w8a8_linear_runtime(rq, rs, q, s16.astype(np.float32))
    assert np.array_equal(y.reshape(10, 256).cpu().numpy().view(np.uint16), ref.view(np.uint16))
    # pre-quantized tuple input + return_scale
    layer._ascend_quant_config = {"return_scale": True, "output_dtype": torch.bfloat16}
    qx, sx = dynamic_quant(x.reshape(10, 512).to(DEV))
    out, sc = meth.apply(layer, (qx, sx))
    assert out.dtype == torch.bfloat16 and sc.shape == (10,)
    assert np.array_equal(qx.cpu().numpy(), rq)


# ------------------------------------------------------------------ W4A16
def test_w4_module_paths():
    _say("w4 modules")
    from mindpipe_amd.w4a16 import (W4A16Linear, gptq_rtn_quantize, pack_int4_for_vllm, pseudo_quantize_tensor,
                                    unpack_int4)
    w = torch.from_numpy(GOLD["awq_w"]).to(DEV)
    deq, s, z = pseudo_quantize_tensor(w, n_bit=4, zero_point=True, q_group_size=128, get_scale_zp=True)
    assert np.array_equal(deq.cpu().numpy().view(np.uint16), GOLD["awq_deq"].view(np.uint16))
    assert np.array_equal(z.cpu().numpy().view(np.uint16), GOLD["awq_z"].view(np.uint16))
    art = gptq_rtn_quantize("proj", torch.from_numpy(GOLD["gptq_w"]).to(DEV), 4, 128)
    assert np.array_equal(art.int_weight.cpu().numpy(), GOLD["gptq_int"])
    vals = torch.tensor([[-8, -7, -1, 0, 1, 6, 7, -3, 4, 2]], dtype=torch.int8)
    p = pack_int4_for_vllm(vals)           # CPU tensor in, CPU tensor out
    assert p.device.type == "cpu" and p.tolist() == [[1609139984, 172]]
    assert torch.equal(unpack_int4(p, 10), vals)
    lin = _lin(512, 1024, True)
    for zp in (True, False):
        mod = W4A16Linear.from_float(lin, 128, zp)
        x = torch.randn(3, 1024, generator=torch.Generator().manual_seed(0)).half()
        y = mod(x.to(DEV)).float().cpu().numpy()
        wn = lin.weight.detach().cpu().numpy()
        rdeq = O.pseudo_quantize_tensor(wn, 4, zp, 128)[0]
        ref = O.w4a16_linear(x.numpy(), rdeq, lin.bias.detach().cpu().numpy())
        assert _rel(y, ref.astype(np.float32)) <= 1e-3
        assert np.array_equal(mod.dequantized_weight().cpu().numpy().view(np.uint16), rdeq.view(np.uint16)) or not zp


class _Bundle:
    """Tokenizer bundle of the export contract: ``save_pretrained`` and an optional ``source_path``."""

    def __init__(self, source_path=None):
        self.source_path = source_path

    def save_pretrained(self, output_dir):
        Path(output_dir, "tokenizer_config.json").write_text("{}", encoding="utf-8")


class _TinyExport(nn.Module):
    """A model with the ``save_pretrained(dir, safe_serialization=True)`` contract of HF models."""

    def __init__(self, k=256, n=64, config=None):
        super().__init__()
        self.proj = nn.Linear(k, n, bias=True)
        self.ignored = nn.Linear(k, n, bias=False)
        self.config_dict = config or {"model_type": "tiny"}

    def save_pretrained(self, output_dir, *, safe_serialization):
        from safetensors.torch import save_file
        assert safe_serialization is True
        out = Path(output_dir)
        out.mkdir(parents=True, exist_ok=True)
        save_file({k: v.detach().cpu().contiguous() for k, v in self.state_dict().items()}, str(out / "model.safetensors"))
        (out / "config.json").write_text(json.dumps(self.config_dict), encoding="utf-8")


def test_export_vllm_gptq_w4a16_reference_kat(tmp_path):
    """The reference's export case (tests/test_vllm_real_quant_export.py:105-152): K = 8, g = 4, the
    signed codes packed to [[1609139984], [-1340634641]], scale (2, 2), ignore == ["ignored"], the
    model's own module restored afterwards, and the rope_theta -> rope_parameters fix-up."""
    _say("export kat")
    from safetensors import safe_open
    from mindpipe_amd.w4a16 import RealQuantLinearArtifact, export_vllm_gptq_w4a16, unpack_int4
    model = _TinyExport(8, 2, {"model_type": "tiny", "rope_theta": 10000.0})
    orig = model.proj
    iw = torch.tensor([[-8, -7, -1, 0, 1, 6, 7, -3], [7, 6, 1, 0, -1, -7, -8, 3]], dtype=torch.int8)
    art = RealQuantLinearArtifact(name="proj", bits=4, group_size=4, symmetric=True, original_shape=(2, 8),
                                  int_weight=iw, scale=torch.tensor([[0.1, 0.2], [0.3, 0.4]], dtype=torch.float16))
    summary = export_vllm_gptq_w4a16(model=model, tokenizer_bundle=_Bundle(), artifacts={"proj": art},
                                     export_dir=tmp_path, group_size=4)
    assert model.proj is orig
    assert summary["backend"] == "vllm" and summary["format"] == "compressed-tensors"
    assert summary["quantized_linear_count"] == 1 and summary["ignored_layers"] == ["ignored"]
    with safe_open(str(tmp_path / "model.safetensors"), framework="pt", device="cpu") as f:
        assert f.get_tensor("proj.weight_packed").tolist() == [[1609139984], [-1340634641]]
        assert torch.equal(unpack_int4(f.get_tensor("proj.weight_packed"), 8), iw)
        assert tuple(f.get_tensor("proj.weight_scale").shape) == (2, 2)
        assert f.get_tensor("proj.weight_shape").tolist() == [2, 8]
    cfg = json.loads((tmp_path / "config.json").read_text())
    assert cfg["compression_config"]["format"] == "pack-quantized"
    assert cfg["compression_config"]["config_groups"]["group_0"]["weights"]["group_size"] == 4
    assert cfg["compression_config"]["ignore"] == ["ignored"]
    assert cfg["rope_parameters"] == {"rope_theta": 10000.0, "rope_type": "default"}
    assert (tmp_path / "tokenizer_config.json").exists()


def test_export_vllm_gptq_w4a16_checks_and_inference_files(tmp_path):
    """Argument checks of the export (each raises before anything is written or swapped) and the copy
    of the source checkpoint's inference files (weights and config.json never copied)."""
    _say("export checks")
    from mindpipe_amd.w4a16 import RealQuantLinearArtifact, export_vllm_gptq_w4a16
    iw = torch.zeros(2, 8, dtype=torch.int8)
    sc = torch.ones(2, 2, dtype=torch.float16)
    good = dict(name="proj", bits=4, group_size=4, symmetric=True, original_shape=(2, 8), int_weight=iw, scale=sc)
    model = _TinyExport(8, 2)
    orig = model.proj
    cases = [({}, ValueError), ({"missing": RealQuantLinearArtifact(**good)}, KeyError),
             ({"proj": RealQuantLinearArtifact(**{**good, "symmetric": False})}, ValueError),
             ({"proj": RealQuantLinearArtifact(**{**good, "group_size": 2})}, ValueError),
             ({"proj": RealQuantLinearArtifact(**{**good, "original_shape": (2, 16)})}, ValueError),
             ({"proj": RealQuantLinearArtifact(**{**good, "scale": torch.ones(2, 3, dtype=torch.float16)})}, ValueError)]
    for arts, exc in cases:
        with pytest.raises(exc):
            export_vllm_gptq_w4a16(model=model, tokenizer_bundle=_Bundle(), artifacts=arts, export_dir=tmp_path / "x",
                                   group_size=4)
        assert model.proj is orig
    src = tmp_path / "src"
    src.mkdir()
    for name in ("tokenizer.json", "generation_config.json", "chat_template.jinja", "model.safetensors",
                 "config.json", "notes.txt", "modeling_tiny.py"):
        (src / name).write_text("{}")
    out = tmp_path / "out"
    summary = export_vllm_gptq_w4a16(model=_TinyExport(8, 2, {"model_type": "tiny",
                                                             "rope_parameters": {"rope_theta": 5e5, "rope_type": "llama3"}}),
                                     tokenizer_bundle=_Bundle(str(src)), artifacts={"proj": RealQuantLinearArtifact(**good)},
                                     export_dir=out, group_size=4)
    assert summary["copied_inference_files"] == ["chat_template.jinja", "generation_config.json", "modeling_tiny.py",
                                                 "tokenizer.json"]
    cfg = json.loads((out / "config.json").read_text())
    assert cfg["rope_theta"] == 5e5 and cfg["rope_parameters"]["rope_type"] == "llama3"


def test_export_then_load_round_trip(tmp_path):
    _say("export/load")
    from mindpipe_amd.w4a16 import VllmPackedInt4Linear, export_vllm_gptq_w4a16, gptq_rtn_quantize, load_vllm_w4a16
    torch.manual_seed(0)
    m = _TinyExport().half().to(DEV)
    art = gptq_rtn_quantize("proj", m.proj.weight.float(), 4, 128)
    summary = export_vllm_gptq_w4a16(model=m, tokenizer_bundle=_Bundle(), artifacts={"proj": art}, export_dir=tmp_path,
                                     group_size=128)
    assert summary["ignored_layers"] == ["ignored"] and summary["quantized_linear_count"] == 1
    cfg = json.loads((tmp_path / "config.json").read_text())["compression_config"]
    assert cfg["format"] == "pack-quantized" and cfg["config_groups"]["group_0"]["weights"]["group_size"] == 128
    m2 = _TinyExport().half().to(DEV)
    names = load_vllm_w4a16(m2, tmp_path)
    assert names == ["proj"] and isinstance(m2.proj, VllmPackedInt4Linear)
    assert torch.equal(m2.ignored.weight, m.ignored.weight)
    x = torch.randn(4, 256, device=DEV).half()
    iw = art.int_weight.float().cpu().numpy()
    deq = (iw * np.repeat(art.scale.float().cpu().numpy(), 128, 1)).astype(np.float16)
    ref = O.w4a16_linear(x.cpu().numpy(), deq, m.proj.bias.detach().cpu().numpy())
    assert _rel(m2.proj(x).float().cpu().numpy(), ref.astype(np.float32)) <= 1e-3


def _tiny_llama(seed=0, dtype=torch.float16):
    from transformers import LlamaConfig, LlamaForCausalLM
    torch.manual_seed(seed)
    cfg = LlamaConfig(hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=4,
                      num_key_value_heads=2, vocab_size=512)
    return LlamaForCausalLM(cfg).to(dtype).to(DEV).eval()


@pytest.mark.parametrize("zero_point", [True, False])
def test_pseudo_quantize_model_weight_router(zero_point):
    """The AWQ router rewrites exactly the block linears (q/k/v/o/gate/up/down of every layer, not the
    embeddings or lm_head), each bit-identical to the oracle's pseudo_quantize_tensor of its weight."""
    _say("pseudo_quantize_model_weight", zero_point)
    from mindpipe_amd.w4a16 import get_blocks, pseudo_quantize_model_weight
    model = _tiny_llama()
    before = {n: p.detach().clone() for n, p in model.named_parameters()}
    pseudo_quantize_model_weight(model, w_bit=4, q_config={"zero_point": zero_point, "q_group_size": 128})
    assert len(get_blocks(model)) == 2
    changed = sorted(n for n, p in model.named_parameters() if not torch.equal(p, before[n]))
    exp = sorted(f"model.layers.{i}.{p}.weight" for i in range(2)
                 for p in ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
                           "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj"))
    assert changed == exp
    for n in exp:
        ref = O.pseudo_quantize_tensor(before[n].cpu().numpy(), 4, zero_point, 128)[0]
        got = dict(model.named_parameters())[n].detach().cpu().numpy()
        assert np.array_equal(got.view(np.uint16), ref.view(np.uint16)), n


def test_quantize_model_w4a16_swaps_block_linears():
    """Real-int4 swap of the router's linears: the same names, W4A16Linear modules, and logits within
    1e-3 of the pseudo-quantized model's (the same codes; fp32 accumulation in both)."""
    _say("quantize_model_w4a16")
    from mindpipe_amd.w4a16 import W4A16Linear, pseudo_quantize_model_weight, quantize_model_w4a16
    ids = torch.randint(0, 512, (2, 16), device=DEV, generator=torch.Generator(device=DEV).manual_seed(1))
    ref_model = _tiny_llama()
    pseudo_quantize_model_weight(ref_model, 4, {"zero_point": True, "q_group_size": 128})
    model = _tiny_llama()
    names = quantize_model_w4a16(model, 128, True)
    assert len(names) == 14 and names[0] == "model.layers.0.self_attn.q_proj"
    assert all(isinstance(model.get_submodule(n), W4A16Linear) for n in names)
    assert isinstance(model.lm_head, nn.Linear)
    with torch.no_grad():
        a = model(ids).logits.float()
        b = ref_model(ids).logits.float()
    assert _rel(a.cpu().numpy(), b.cpu().numpy()) <= 1e-3


# ------------------------------------------------------------------ add-RMSNorm fusion, dense MLP chain
def _w8_layer(n, k, seed):
    from mindpipe_amd.runtime import W8A8DynamicLinearMethod
    w = torch.randn(n, k, generator=torch.Generator().manual_seed(seed)) * 0.02
    q, s32, s16, _ = O.quantize_weight_per_channel_export(w.half().numpy())

    class Layer(nn.Module):
        pass

    layer = Layer()
    layer.weight = nn.Parameter(torch.from_numpy(q).to(DEV), requires_grad=False)
    layer.weight_scale = nn.Parameter(torch.from_numpy(s16).reshape(-1, 1).to(DEV), requires_grad=False)
    layer.quant_method = W8A8DynamicLinearMethod()
    layer.quant_method.process_weights_after_loading(layer)
    return layer, q, s16


def test_add_rms_norm_forward_fused_equals_unfused():
    _say("add_rms_norm_forward")
    from mindpipe_amd.runtime import add_rms_norm_forward
    h, t = 512, 6
    layer, q, s16 = _w8_layer(384, h, seed=4)
    norm = nn.Module()
    norm.weight = nn.Parameter((torch.rand(h, generator=torch.Generator().manual_seed(2)) + 0.5).half().to(DEV),
                               requires_grad=False)
    norm.variance_epsilon = 1e-6
    g = torch.Generator().manual_seed(3)
    x = torch.randn(t, h, generator=g).half().to(DEV)
    res = torch.randn(t, h, generator=g).half().to(DEV)
    fused, rsum = add_rms_norm_forward(norm, x, res, layer)        # (int8, scale) tuple for a W8A8 linear
    assert isinstance(fused, tuple) and fused[0].dtype == torch.int8
    plain, rsum2 = add_rms_norm_forward(norm, x, res, None)        # normalised fp16 activations
    assert plain.dtype == torch.float16 and torch.equal(rsum, rsum2)
    assert torch.equal(rsum, (x.float() + res.float()).half())
    # the W8A8 linear gives the same bits from the fused tuple and from the unfused activations
    y_f = layer.quant_method.apply(layer, fused)
    y_u = layer.quant_method.apply(layer, plain)
    assert torch.equal(y_f, y_u)
    yr, qr, sr, _ = O.add_rms_norm_quant(x.cpu().numpy(), res.cpu().numpy(), norm.weight.cpu().numpy(), 1e-6)
    assert np.abs(plain.cpu().numpy().view(np.int16).astype(int) - yr.view(np.int16).astype(int)).max() <= 2


@pytest.mark.parametrize("chunks,tuple_in", [(1, False), (2, False), (4, True)])
def test_dense_mlp_w8a8_matches_oracle(chunks, tuple_in):
    _say("dense mlp", chunks, tuple_in)
    from mindpipe_amd.runtime import dense_mlp_w8a8, dynamic_quant, prepare_dense_mlp_w8a8
    h, inter, t = 512, 768, 20
    gate_up, q13, s13 = _w8_layer(2 * inter, h, seed=5)
    down, q2, s2 = _w8_layer(h, inter, seed=6)
    prepare_dense_mlp_w8a8(gate_up, down, chunks)
    x = torch.randn(t, h, generator=torch.Generator().manual_seed(7)).half()
    xin = dynamic_quant(x.to(DEV)) if tuple_in else x.to(DEV)
    y = dense_mlp_w8a8(gate_up, down, xin)
    assert y.shape == (t, h) and y.dtype == torch.float16
    ref = O.dense_mlp_runtime(x.numpy(), q13, s13.astype(np.float32), q2, s2.astype(np.float32), chunks=chunks)
    yn = y.cpu().numpy()
    err = _rel(yn, ref)
    assert err <= 1e-3, err   # bar: rel. Frobenius error <= 1e-3
    # bit-identical except where silu's exp puts a requant code on a rounding boundary
    assert np.mean(yn.view(np.uint16) == ref.view(np.uint16)) >= 0.99


# ------------------------------------------------------------------ method adapters (base.py:20-21)
def test_smoothquant_method_adapter_on_tiny_llama(tmp_path):
    """apply_fake_quantization: statistics from calibration batches, smoothing, int8 swap; the
    artifact dict of the reference; logits close to the fp16 model's; statistics saved and reused."""
    _say("SmoothQuantMethod")
    from types import SimpleNamespace
    from mindpipe_amd.methods import SmoothQuantMethod
    from mindpipe_amd.smoothquant import SmoothQuantLinear
    model = _tiny_llama()
    g = torch.Generator().manual_seed(5)
    batches = [(torch.randint(0, 512, (2, 32), generator=g), None) for _ in range(2)]
    ids = batches[0][0].to(DEV)
    with torch.no_grad():
        ref = model(ids).logits.float()
    args = SimpleNamespace(weight_bits=8, activation_bits=8, query_bits=16, key_bits=16, value_bits=16,
                           smoothquant_alpha=0.85, calibration_batches=batches, smoothquant_save_act_scales=True,
                           model_path=str(tmp_path / "tiny"), output_root=str(tmp_path / "runs"), sequence_length=32)
    art = SmoothQuantMethod().apply_fake_quantization(model, None, args)
    assert art["quantized_linear_count"] == 14 and art["smoothquant_config"]["alpha"] == 0.85
    assert art["smoothquant_config"]["model_type"] == "llama" and Path(art["act_scales_path"]).exists()
    assert isinstance(model.model.layers[1].mlp.down_proj, SmoothQuantLinear)
    with torch.no_grad():
        out = model(ids).logits.float()
    cos = torch.nn.functional.cosine_similarity(out.flatten(), ref.flatten(), dim=0).item()
    assert cos > 0.99, cos
    # reuse of the saved statistics on a fresh model gives the same quantized weights
    model2 = _tiny_llama()
    args2 = SimpleNamespace(**{**vars(args), "calibration_batches": None,
                               "smoothquant_act_scales_from": art["act_scales_path"]})
    SmoothQuantMethod().apply_fake_quantization(model2, None, args2)
    assert torch.equal(model2.model.layers[0].self_attn.q_proj.weight, model.model.layers[0].self_attn.q_proj.weight)


def test_awq_method_adapter_equals_router():
    _say("AWQMethod")
    from types import SimpleNamespace
    from mindpipe_amd.methods import AWQMethod
    from mindpipe_amd.w4a16 import pseudo_quantize_model_weight
    a, b = _tiny_llama(), _tiny_llama()
    args = SimpleNamespace(weight_bits=4, activation_bits=16, weight_symmetric=False, weight_group_size=128)
    art = AWQMethod().apply_fake_quantization(a, None, args)
    assert art["quantization_config"] == {"zero_point": True, "q_group_size": 128}
    pseudo_quantize_model_weight(b, 4, {"zero_point": True, "q_group_size": 128})
    for (n, p), (_, q) in zip(a.named_parameters(), b.named_parameters()):
        assert torch.equal(p, q), n
