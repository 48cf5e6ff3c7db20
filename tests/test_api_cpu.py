"""CPU-side behaviour of the host API: argument checks, loud failure without a GPU path,
config builders.  No kernel runs here."""
import pytest
import torch
from torch import nn

from mindpipe_amd import w4a16 as W4
from mindpipe_amd import smoothquant as SQ


def test_compression_config_matches_reference_schema():
    cfg = W4.build_compression_config(group_size=128, ignored_layers=["lm_head"])
    assert cfg["format"] == "pack-quantized"
    assert cfg["ignore"] == ["lm_head"]
    wq = cfg["config_groups"]["group_0"]["weights"]
    assert wq == {"dynamic": False, "group_size": 128, "num_bits": 4, "observer": "minmax", "observer_kwargs": {},
                  "strategy": "group", "symmetric": True, "type": "int"}
    assert cfg["quant_method"] == "compressed-tensors"


def test_smoothquant_linear_rejects_bad_args():
    with pytest.raises(ValueError):
        SQ.SmoothQuantLinear(8, 8, act_quant="per_tensor")
    with pytest.raises(NotImplementedError):
        SQ.SmoothQuantLinear(8, 8, weight_bits=12)  # codes wider than int8
    with pytest.raises(NotImplementedError):
        SQ.SmoothQuantLinear(8, 8, activation_bits=1)
    with pytest.raises(ValueError):
        SQ.SmoothQuantLinear(8, 8, scale_rule="other")
    with pytest.raises(ValueError):
        SQ.SmoothQuantLinear(8, 8, weight_bits=4, scale_rule="export")
    assert "weight_bits=4, activation_bits=16" in repr(SQ.SmoothQuantLinear(8, 8, weight_bits=4, activation_bits=16))


def test_module_forward_refuses_cpu_tensors():
    mod = SQ.SmoothQuantLinear(16, 8)
    with pytest.raises(RuntimeError, match="GPU"):
        mod(torch.zeros(2, 16, dtype=torch.float16))
    with pytest.raises(RuntimeError, match="GPU"):
        SQ.quantize_activation_per_token_absmax(torch.zeros(2, 16, dtype=torch.float16))
    w4 = W4.W4A16Linear(128, 16)
    with pytest.raises(RuntimeError, match="GPU"):
        w4(torch.zeros(1, 128, dtype=torch.float16))


def test_quantize_model_rejects_unknown_model_type():
    class M(nn.Module):
        config = type("C", (), {"model_type": "gpt2"})()
    with pytest.raises(ValueError, match="Unsupported model type"):
        SQ.quantize_model(M())
    with pytest.raises(ValueError):
        SQ.quantize_model(M(), weight_quant="per_tensor")


def test_w4_module_buffers_and_shapes():
    mod = W4.W4A16Linear(256, 64, group_size=128, zero_point=True)
    assert mod.weight_packed.shape == (64, 32) and mod.weight_packed.dtype == torch.int32
    assert mod.weight_scale.shape == (64, 2) and mod.weight_zero_point.shape == (64, 2)
    assert mod.weight_shape.tolist() == [64, 256]
    with pytest.raises(ValueError):
        W4.W4A16Linear(100, 8, group_size=128)
    with pytest.raises(NotImplementedError):  # codes wider than 8 bits
        W4.pseudo_quantize_tensor(torch.zeros(4, 128, dtype=torch.float16), n_bit=9)
    with pytest.raises(RuntimeError, match="GPU"):  # other widths run on the GPU too
        W4.pseudo_quantize_tensor(torch.zeros(4, 128, dtype=torch.float16), n_bit=8)


def test_smoothing_refuses_cpu_weights():
    """Smoothing runs on the GPU kernels only: CPU weights raise instead of falling back."""
    fc = nn.Linear(3, 2, bias=False).half()
    with pytest.raises(RuntimeError):
        SQ.compute_smooth_scales(fc, torch.tensor([4.0, 9.0, 0.0]), 0.5)
    with pytest.raises(AssertionError):  # the reference's width check comes first
        SQ.compute_smooth_scales(fc, torch.tensor([4.0, 9.0]), 0.5)

def test_method_adapters_validate_like_the_reference():
    """apply_fake_quantization's argument checks (smoothquant/method.py:85-108): unsupported model type,
    non-W8A8 bits, quantized Q/K/V caches, missing calibration data; AWQ's search is refused."""
    from types import SimpleNamespace
    from mindpipe_amd.methods import AWQMethod, BaseQuantizationMethod, METHODS, SmoothQuantMethod
    assert issubclass(SmoothQuantMethod, BaseQuantizationMethod) and set(METHODS) == {"smoothquant", "awq"}

    class M(nn.Module):
        def __init__(self, t):
            super().__init__()
            self.config = SimpleNamespace(model_type=t)

    ok = dict(weight_bits=8, activation_bits=8, query_bits=16, key_bits=16, value_bits=16, smoothquant_alpha=0.85)
    with pytest.raises(NotImplementedError):
        SmoothQuantMethod().apply_fake_quantization(M("gpt2"), None, SimpleNamespace(**ok))
    with pytest.raises(ValueError):
        SmoothQuantMethod().apply_fake_quantization(M("llama"), None, SimpleNamespace(**{**ok, "weight_bits": 4}))
    with pytest.raises(ValueError):
        SmoothQuantMethod().apply_fake_quantization(M("llama"), None, SimpleNamespace(**{**ok, "key_bits": 8}))
    with pytest.raises(ValueError):  # no calibration_batches / act scales
        SmoothQuantMethod().apply_fake_quantization(M("llama"), None, SimpleNamespace(**ok))
    with pytest.raises(NotImplementedError):
        AWQMethod().apply_fake_quantization(M("llama"), None, SimpleNamespace(awq_search=True))


@pytest.mark.parametrize("model_type", ["qwen2_vl", "qwen3", "qwen3_moe"])
def test_ascend_export_rejects_non_dense_qwen2(tmp_path, model_type):
    """read_config of the W8A8_DYNAMIC export (export_fp16_to_ascend_w8a8_dynamic_probe.py:75-101):
    only dense Qwen2 / Qwen2.5 checkpoints."""
    import json
    from mindpipe_amd.ascend_w8a8 import read_config
    (tmp_path / "config.json").write_text(json.dumps({"architectures": ["Qwen2ForCausalLM"], "model_type": model_type,
                                                      "num_hidden_layers": 1}))
    with pytest.raises(ValueError, match="Expected dense Qwen2/Qwen2.5"):
        read_config(tmp_path)


def _ascend_source(path, dtype=torch.float16, drop=None):
    """The reference test's tiny dense-Qwen2 source (one layer, every projection
    ``arange(6).reshape(2, 3) - index``; test_export_fp16_to_ascend_w8a8_dynamic_probe.py:27-45)."""
    import json
    from safetensors.torch import save_file
    from mindpipe_amd.ascend_w8a8 import LINEAR_SUFFIXES
    path.mkdir(parents=True)
    (path / "config.json").write_text(json.dumps({"architectures": ["Qwen2ForCausalLM"], "model_type": "qwen2",
                                                  "num_hidden_layers": 1}))
    t = {"model.embed_tokens.weight": torch.arange(12, dtype=dtype).reshape(4, 3),
         "lm_head.weight": torch.arange(12, dtype=dtype).reshape(4, 3)}
    for i, suf in enumerate(LINEAR_SUFFIXES, start=1):
        name = f"model.layers.0.{suf}.weight"
        if name != drop:
            t[name] = torch.arange(6, dtype=dtype).reshape(2, 3) - i
    save_file(t, str(path / "model.safetensors"))
    return t


def _ascend_output(path, src_tensors, scale_dtype=None):
    """An export written by hand from the oracle's export quantizer (no GPU): what the writer must
    produce, for the verifier."""
    import json
    from safetensors.torch import save_file
    from oracle import quant as O
    from mindpipe_amd.ascend_w8a8 import LINEAR_SUFFIXES
    path.mkdir(parents=True)
    out, desc = {}, {"model.embed_tokens.weight": "FLOAT", "lm_head.weight": "FLOAT"}
    for n, v in src_tensors.items():
        if any(n.endswith(s + ".weight") for s in LINEAR_SUFFIXES):
            q, _, s16, _ = O.quantize_weight_per_channel_export(v.numpy())
            base = n[:-len(".weight")]
            sc = torch.from_numpy(s16).reshape(-1, 1).to(scale_dtype or v.dtype)
            out.update({n: torch.from_numpy(q), f"{base}.weight_scale": sc, f"{base}.weight_offset": torch.zeros_like(sc)})
            desc[n] = "W8A8_DYNAMIC"
        else:
            out[n] = v
    save_file(out, str(path / "model.safetensors"))
    (path / "quant_model_description.json").write_text(json.dumps(desc))


def test_ascend_export_checks_before_any_gpu_work(tmp_path):
    """The source checks of the W8A8_DYNAMIC export, with the message fragments the reference's tests
    match (tests/repro/test_export_fp16_to_ascend_w8a8_dynamic_probe.py:107-171)."""
    from mindpipe_amd.ascend_w8a8 import export_w8a8_dynamic
    src = tmp_path / "src"
    _ascend_source(src)
    for out in (src, src / "out", tmp_path):
        with pytest.raises(ValueError, match="separate, non-nested"):
            export_w8a8_dynamic(src, out)
    src2 = tmp_path / "src2"
    _ascend_source(src2, drop="model.layers.0.mlp.down_proj.weight")
    with pytest.raises(ValueError, match="missing 1 required"):
        export_w8a8_dynamic(src2, tmp_path / "o2")
    src3 = tmp_path / "src3"
    _ascend_source(src3, dtype=torch.int8)
    with pytest.raises(ValueError, match="floating-point"):
        export_w8a8_dynamic(src3, tmp_path / "o3")
    assert not (tmp_path / "o2").exists() and not (tmp_path / "o3").exists()


def test_ascend_verifier_on_a_hand_written_export(tmp_path):
    """verify_w8a8_dynamic accepts an export holding the format (with and without the index) and
    names every mismatch: a scale in another dtype than its source weight ("expected source weight
    dtype F16", the reference test's fragment), a missing offset, a wrong description entry."""
    import json
    from mindpipe_amd.ascend_w8a8 import verify_w8a8_dynamic
    src, out = tmp_path / "src", tmp_path / "out"
    t = _ascend_source(src)
    _ascend_output(out, t)
    rep = verify_w8a8_dynamic(out, src)
    assert rep["validated_linear_weights"] == 7 and rep["output_index_present"] is False
    from safetensors import safe_open
    with safe_open(str(out / "model.safetensors"), framework="pt") as f:
        wm = {n: "model.safetensors" for n in f.keys()}
    (out / "model.safetensors.index.json").write_text(json.dumps({"weight_map": wm}))
    assert verify_w8a8_dynamic(out, src)["output_index_present"] is True
    wm["lm_head.weight"] = "other.safetensors"
    (out / "model.safetensors.index.json").write_text(json.dumps({"weight_map": wm}))
    with pytest.raises(ValueError, match="index maps lm_head.weight"):
        verify_w8a8_dynamic(out, src)
    (out / "model.safetensors.index.json").unlink()
    bad = tmp_path / "bad"
    _ascend_output(bad, t, scale_dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="expected source weight dtype F16"):
        verify_w8a8_dynamic(bad, src)
    d = json.loads((out / "quant_model_description.json").read_text())
    d["lm_head.weight"] = "W8A8_DYNAMIC"
    (out / "quant_model_description.json").write_text(json.dumps(d))
    with pytest.raises(ValueError, match="lm_head.weight"):
        verify_w8a8_dynamic(out, src)
