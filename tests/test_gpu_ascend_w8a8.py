"""Ascend W8A8_DYNAMIC writer / verifier / loader on the reference's tiny dense-Qwen2 fixture
(tests/repro/test_export_fp16_to_ascend_w8a8_dynamic_probe.py:27-99: one layer, H = 3, every
projection W = arange(6).reshape(2, 3) - index in fp16).

Pins: the reference test's assertions (7 converted linears, 7 validated, index present, int8 q_proj,
weight_scale [2, 1], verify-only with and without the index) and the closed-form codes of projections
1 and 2 (q = [[-127, 0, 127], [64, 95, 127]] with scale fp16 [0.00787353515625, 0.031494140625];
q = [[-127, -64, 0], [42, 85, 127]]; the 63.5 -> 64 and -63.5 -> -64 ties).  The round trip loads the
export into a model with no requantization and runs the runtime linear: bit-exact against the oracle's
runtime W8A8 linear on the stored codes and scales."""
import json
import sys

import numpy as np
import pytest
import torch
from torch import nn

from oracle import quant as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _write_source(path, model_type="qwen2"):
    from safetensors.torch import save_file
    from mindpipe_amd.ascend_w8a8 import LINEAR_SUFFIXES
    path.mkdir(parents=True)
    cfg = {"architectures": ["Qwen2ForCausalLM"], "model_type": model_type, "num_hidden_layers": 1,
           "tie_word_embeddings": False, "quantization_config": {"drop": True}}
    (path / "config.json").write_text(json.dumps(cfg), encoding="utf-8")
    (path / "tokenizer_config.json").write_text("{}", encoding="utf-8")
    t = {"model.embed_tokens.weight": torch.arange(12, dtype=torch.float16).reshape(4, 3),
         "model.layers.0.input_layernorm.weight": torch.ones(3, dtype=torch.float16),
         "lm_head.weight": torch.arange(12, dtype=torch.float16).reshape(4, 3)}
    for i, suf in enumerate(LINEAR_SUFFIXES, start=1):
        t[f"model.layers.0.{suf}.weight"] = torch.arange(6, dtype=torch.float16).reshape(2, 3) - i
    save_file(t, str(path / "model.safetensors"))


class _Attn(nn.Module):
    def __init__(self):
        super().__init__()
        for p in ("q_proj", "k_proj", "v_proj", "o_proj"):
            setattr(self, p, nn.Linear(3, 2, bias=False))


class _Mlp(nn.Module):
    def __init__(self):
        super().__init__()
        for p in ("gate_proj", "up_proj", "down_proj"):
            setattr(self, p, nn.Linear(3, 2, bias=False))


class _Norm(nn.Module):
    def __init__(self):
        super().__init__()
        self.weight = nn.Parameter(torch.zeros(3))


class _Layer(nn.Module):
    def __init__(self):
        super().__init__()
        self.self_attn, self.mlp, self.input_layernorm = _Attn(), _Mlp(), _Norm()


class _Inner(nn.Module):
    def __init__(self):
        super().__init__()
        self.embed_tokens = nn.Embedding(4, 3)
        self.layers = nn.ModuleList([_Layer()])


class _Model(nn.Module):
    """The module tree of the fixture's tensor names (a format-level stand-in for Qwen2ForCausalLM)."""

    def __init__(self):
        super().__init__()
        self.model = _Inner()
        self.lm_head = nn.Linear(3, 4, bias=False)


def test_export_verify_and_reference_assertions(tmp_path):
    _say("ascend export")
    from safetensors import safe_open
    from mindpipe_amd.ascend_w8a8 import export_w8a8_dynamic, verify_w8a8_dynamic
    src, out = tmp_path / "source", tmp_path / "output"
    _write_source(src)
    summary = export_w8a8_dynamic(src, out)
    assert summary["converted_linear_modules"] == 7
    assert summary["validation"]["validated_linear_weights"] == 7
    assert summary["validation"]["output_index_present"] is True
    index = json.loads((out / "model.safetensors.index.json").read_text())
    assert "model.layers.0.self_attn.q_proj.weight_scale" in index["weight_map"]
    with safe_open(str(out / "model.safetensors"), framework="pt", device="cpu") as f:
        assert str(f.get_slice("model.layers.0.self_attn.q_proj.weight").get_dtype()).upper() in {"I8", "INT8"}
        assert f.get_slice("model.layers.0.self_attn.q_proj.weight_scale").get_shape() == [2, 1]
        q1 = f.get_tensor("model.layers.0.self_attn.q_proj.weight")
        s1 = f.get_tensor("model.layers.0.self_attn.q_proj.weight_scale")
        q2 = f.get_tensor("model.layers.0.self_attn.k_proj.weight")
        assert q1.tolist() == [[-127, 0, 127], [64, 95, 127]]
        assert s1.dtype == torch.float16 and s1.flatten().tolist() == [0.00787353515625, 0.031494140625]
        assert q2.tolist() == [[-127, -64, 0], [42, 85, 127]]
        assert torch.equal(f.get_tensor("model.layers.0.self_attn.q_proj.weight_offset"), torch.zeros(2, 1).half())
        assert torch.equal(f.get_tensor("lm_head.weight"), torch.arange(12, dtype=torch.float16).reshape(4, 3))
    desc = json.loads((out / "quant_model_description.json").read_text())
    assert desc["lm_head.weight"] == "FLOAT" and desc["model.layers.0.mlp.gate_up_proj.weight"] == "W8A8_DYNAMIC"
    cfg = json.loads((out / "config.json").read_text())
    assert "quantization_config" not in cfg and (out / "tokenizer_config.json").exists()
    assert verify_w8a8_dynamic(out, src)["output_index_present"] is True
    (out / "model.safetensors.index.json").unlink()   # the index-less exports stay verifiable
    assert verify_w8a8_dynamic(out, src)["output_index_present"] is False
    with pytest.raises(FileExistsError):
        export_w8a8_dynamic(src, out)
    assert export_w8a8_dynamic(src, out, overwrite=True)["converted_linear_modules"] == 7


@pytest.mark.parametrize("target", ["runtime", "smoothquant"])
def test_round_trip_into_model_without_requantization(tmp_path, target):
    _say("ascend load", target)
    from safetensors import safe_open
    from mindpipe_amd.ascend_w8a8 import export_w8a8_dynamic, load_w8a8_dynamic
    src, out = tmp_path / "source", tmp_path / "output"
    _write_source(src)
    export_w8a8_dynamic(src, out)
    model = _Model().half().to(DEV)
    names = load_w8a8_dynamic(model, out, target=target)
    assert len(names) == 7 and names[0].startswith("model.layers.0.")
    assert torch.equal(model.lm_head.weight.cpu(), torch.arange(12, dtype=torch.float16).reshape(4, 3))
    assert torch.equal(model.model.layers[0].input_layernorm.weight.cpu(), torch.ones(3, dtype=torch.float16))
    x = torch.randn(5, 3, generator=torch.Generator().manual_seed(0)).half()
    qx, sx = O.quantize_per_token_runtime(x.numpy())
    with safe_open(str(out / "model.safetensors"), framework="pt", device="cpu") as f:
        for n in names:
            lin = model.get_submodule(n)
            q = f.get_tensor(f"{n}.weight")
            s = f.get_tensor(f"{n}.weight_scale").float().flatten()
            assert torch.equal(lin.weight.cpu(), q)                 # the stored codes, not requantized
            y = lin(x.to(DEV))
            ref = O.w8a8_linear_runtime(qx, sx, q.numpy(), s.numpy(), None, "fp16")
            assert np.array_equal(y.cpu().numpy().view(np.uint16), np.asarray(ref).view(np.uint16)), n
