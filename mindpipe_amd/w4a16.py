"""W4A16 group-quantized linear: AWQ / GPTQ quantizers, the vLLM compressed-tensors
pack format and a real-int4 linear module, backed by the gfx950 kernels.

Mirrors:
  * ``pseudo_quantize_tensor`` / ``pseudo_quantize_model_weight``
    (``algorithm/quantization/ptq/awq/source/awq/quantize/quantizer.py:63-130``);
  * GPTQ's symmetric group quantizer in its round-to-nearest form
    (``algorithm/quantization/ptq/gptq/source/quant.py:13-17,44-82``, signed export
    ``gptq.py:157-161``) producing ``RealQuantLinearArtifact`` (``exporters/schema.py:10-20``);
  * ``pack_int4_for_vllm`` / ``VllmPackedInt4Linear`` / the compression config
    (``algorithm/quantization/exporters/vllm.py:57-190``), with a working ``forward``;
  * the export dequant of ``scripts/repro/evaluate_real_quant_export_dequant.py:36-64``.
"""
from __future__ import annotations

import contextlib
import json
import shutil
from dataclasses import dataclass
from pathlib import Path
from typing import Dict, Iterable, List, Optional

import torch
from torch import nn

from . import ops

__all__ = [
    "pseudo_quantize_tensor",
    "gptq_rtn_quantize",
    "RealQuantLinearArtifact",
    "pack_int4_for_vllm",
    "unpack_int4",
    "W4A16Linear",
    "VllmPackedInt4Linear",
    "build_compression_config",
    "get_blocks",
    "get_named_linears",
    "pseudo_quantize_model_weight",
    "quantize_model_w4a16",
    "export_vllm_gptq_w4a16",
    "load_vllm_w4a16",
]


def _gpu(t: torch.Tensor) -> torch.Tensor:
    if t.is_cuda:
        return t
    if not torch.cuda.is_available():
        raise RuntimeError("mindpipe_amd runs on the GPU only; no GPU is visible")
    return t.cuda()


@dataclass
class RealQuantLinearArtifact:
    """Integer weight and qparams of one quantized Linear (``exporters/schema.py:10-20``)."""

    name: str
    bits: int
    group_size: int
    symmetric: bool
    original_shape: tuple
    int_weight: torch.Tensor
    scale: torch.Tensor


@torch.no_grad()
def pseudo_quantize_tensor(w, n_bit=8, zero_point=True, q_group_size=-1, inplace=False, get_scale_zp=False):
    """AWQ pseudo-quantization on the GPU, same signature and results as the reference.

    Code widths ``n_bit`` 1..8 (2..8 without a zero point); fp16 and bf16 weights are quantized
    in their own arithmetic.  Returns the dequantized weight (bit-identical to the reference's),
    plus ``scales``/``zeros`` ``[N, K/g]`` when ``get_scale_zp`` (zero_point only, as in the
    reference).  ``n_bit=4`` runs the quantizer that also packs the codes for the W4A16 GEMMs.
    """
    n_bit = int(n_bit)
    if not (1 <= n_bit <= 8) or (n_bit == 1 and not zero_point):
        raise NotImplementedError(f"n_bit={n_bit}: this build's AWQ quantizer takes 1..8-bit codes "
                                  "(2..8 without a zero point)")
    if get_scale_zp and not zero_point:
        raise ValueError("get_scale_zp needs zero_point=True (the reference's symmetric branch has no zeros)")
    src = _gpu(w.detach())
    shape = src.shape
    w2 = src.reshape(-1, shape[-1]).contiguous()
    if w2.dtype not in (torch.float16, torch.bfloat16):
        raise NotImplementedError("the AWQ quantizer takes fp16 or bf16 weights (the reference's arithmetic)")
    if n_bit == 4:
        _, s, z, deq = ops.w4_quantize_awq(w2, q_group_size, zero_point, return_deq=True)
    else:
        s, z, deq = ops.awq_pseudo_quantize(w2, n_bit, q_group_size, zero_point)
    deq = deq.reshape(shape).to(w.device)
    if inplace:
        w.data.copy_(deq)
        deq = w
    if get_scale_zp:
        return deq, s.to(w.device), z.to(w.device)
    return deq


@torch.no_grad()
def gptq_rtn_quantize(name: str, weight: torch.Tensor, bits: int = 4, group_size: int = 128) -> RealQuantLinearArtifact:
    """GPTQ symmetric group quantizer without Hessian error feedback (its RTN case):
    ``int_weight`` int8 ``[N,K]`` in ``[-8,7]`` and fp16 ``scale`` ``[N, K/g]``."""
    if bits != 4:
        raise NotImplementedError("mindpipe_amd implements the 4-bit GPTQ export")
    iw, _, scale = ops.w4_quantize_gptq_rtn(_gpu(weight.detach()).contiguous(), group_size)
    return RealQuantLinearArtifact(name=name, bits=4, group_size=group_size, symmetric=True,
                                   original_shape=tuple(int(d) for d in weight.shape), int_weight=iw,
                                   scale=scale)


def pack_int4_for_vllm(int_weight: torch.Tensor) -> torch.Tensor:
    """``exporters/vllm.py:89-111`` on the GPU; returns the packed tensor on the input's device."""
    if int_weight.ndim != 2:
        raise ValueError(f"Expected 2D int_weight, got shape {tuple(int_weight.shape)}.")
    packed = ops.pack_int4(_gpu(int_weight.to(torch.int8)).contiguous())
    return packed.to(int_weight.device)


def unpack_int4(packed: torch.Tensor, columns: int) -> torch.Tensor:
    return ops.unpack_int4(_gpu(packed).contiguous(), columns).to(packed.device)


class W4A16Linear(nn.Module):
    """Real int4 linear: ``weight_packed`` int32 ``[N, K/8]``, ``weight_scale`` ``[N, K/g]``,
    ``weight_zero_point`` ``[N, K/g]`` (AWQ asymmetric) or ``None`` (symmetric, zero point 8),
    ``weight_shape`` int64 ``[2]``, ``bias``; scales, zeros and bias in the module dtype (fp16
    or bf16, the dtype of the activations); ``forward`` runs the W4A16 kernel."""

    def __init__(self, in_features: int, out_features: int, group_size: int = 128, bias: bool = True,
                 zero_point: bool = True, dtype=torch.float16, device=None):
        super().__init__()
        if in_features % 8 or in_features % group_size:
            raise ValueError("in_features must be a multiple of 8 and of group_size")
        if dtype not in (torch.float16, torch.bfloat16):
            raise ValueError("W4A16Linear computes in fp16 or bf16")
        self.in_features, self.out_features, self.group_size = in_features, out_features, group_size
        self.dtype = dtype
        g = in_features // group_size
        self.register_buffer("weight_packed", torch.zeros((out_features, in_features // 8), dtype=torch.int32, device=device))
        self.register_buffer("weight_scale", torch.ones((out_features, g), dtype=dtype, device=device))
        self.register_buffer("weight_zero_point", torch.full((out_features, g), 8.0, dtype=dtype, device=device)
                             if zero_point else None)
        self.register_buffer("weight_shape", torch.tensor([out_features, in_features], dtype=torch.int64))
        self.register_buffer("bias", torch.zeros(out_features, dtype=dtype, device=device) if bias else None)

    @classmethod
    @torch.no_grad()
    def from_float(cls, linear: nn.Linear, group_size: int = 128, zero_point: bool = True) -> "W4A16Linear":
        """AWQ codes of ``linear.weight`` in its own dtype (bf16 stays bf16, anything else is
        quantized in fp16)."""
        dt = linear.weight.dtype if linear.weight.dtype in (torch.float16, torch.bfloat16) else torch.float16
        w = _gpu(linear.weight.detach()).to(dt).contiguous()
        n, k = w.shape
        mod = cls(k, n, group_size, linear.bias is not None, zero_point, dtype=dt, device=w.device)
        packed, s, z, _ = ops.w4_quantize_awq(w, group_size, zero_point, return_deq=False)
        if s.shape[1] != k // group_size:
            raise ValueError("group_size must divide in_features")
        mod.weight_packed.copy_(packed)
        mod.weight_scale.copy_(s)
        if zero_point:
            mod.weight_zero_point.copy_(z)
        if linear.bias is not None:
            mod.bias.copy_(linear.bias.detach().to(dt))
        return mod

    @classmethod
    def from_artifact(cls, art: RealQuantLinearArtifact, bias: Optional[torch.Tensor] = None) -> "W4A16Linear":
        n, k = art.original_shape
        mod = cls(k, n, art.group_size, bias is not None, zero_point=False,
                  device=torch.device("cuda") if torch.cuda.is_available() else None)
        mod.weight_packed.copy_(pack_int4_for_vllm(art.int_weight).to(mod.weight_packed.device))
        mod.weight_scale.copy_(art.scale.to(torch.float16))
        if bias is not None:
            mod.bias.copy_(bias)
        return mod

    def dequantized_weight(self) -> torch.Tensor:
        """``(u - z) * s`` in the module dtype (the reference's pseudo-quantized weight for AWQ
        codes)."""
        u = ops.unpack_int4(self.weight_packed, self.in_features).to(torch.int16) + 8
        s = self.weight_scale.repeat_interleave(self.group_size, dim=1)
        z = (self.weight_zero_point.repeat_interleave(self.group_size, dim=1) if self.weight_zero_point is not None
             else torch.full_like(s, 8.0))
        return ((u.to(s.dtype) - z) * s).to(s.dtype)

    @torch.no_grad()
    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if not x.is_cuda:
            raise RuntimeError("W4A16Linear runs on the GPU only")
        if x.dtype != self.weight_scale.dtype:
            raise RuntimeError(f"W4A16Linear holds {self.weight_scale.dtype} scales; got {x.dtype} activations")
        return ops.w4a16_gemm(x.contiguous(), self.weight_packed, self.weight_scale, self.weight_zero_point,
                              self.group_size, self.bias)

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, group_size={self.group_size}, "
                f"zero_point={self.weight_zero_point is not None}, bias={self.bias is not None}")


class VllmPackedInt4Linear(W4A16Linear):
    """The export module of ``exporters/vllm.py:57-86`` (same buffer names), with a forward."""

    def __init__(self, *, packed_weight, scale, bias, in_features, out_features):
        g = in_features // scale.shape[1]
        super().__init__(in_features, out_features, g, bias is not None, zero_point=False,
                         device=packed_weight.device)
        self.weight_packed.copy_(packed_weight)
        self.weight_scale.copy_(scale.to(torch.float16))
        if bias is not None:
            self.bias.copy_(bias)


def build_compression_config(*, group_size: int, ignored_layers: List[str],
                             quant_method: str = "compressed-tensors") -> dict:
    """``_build_compression_config`` (``exporters/vllm.py:139-165``)."""
    return {
        "config_groups": {"group_0": {"targets": ["Linear"], "input_activations": None,
                                      "weights": {"dynamic": False, "group_size": int(group_size), "num_bits": 4,
                                                  "observer": "minmax", "observer_kwargs": {}, "strategy": "group",
                                                  "symmetric": True, "type": "int"}}},
        "format": "pack-quantized",
        "ignore": list(ignored_layers),
        "quant_method": quant_method,
    }


def _named_linears(model: nn.Module) -> Dict[str, nn.Linear]:
    return {n: m for n, m in model.named_modules() if isinstance(m, nn.Linear)}


def _set_module(model: nn.Module, name: str, new: nn.Module) -> None:
    parent_name, _, child = name.rpartition(".")
    parent = model.get_submodule(parent_name) if parent_name else model
    setattr(parent, child, new)


def _is_qwen3_5(model) -> bool:
    return str(getattr(getattr(model, "config", None), "model_type", None)) in {"qwen3_5", "qwen3_5_text"}


def get_blocks(model: nn.Module):
    """The decoder blocks whose linears the AWQ router rewrites (``get_blocks``,
    ``awq/source/awq/quantize/pre_quant.py:47-76``): the language model's ``layers`` for HF decoders
    and VL wrappers, ``decoder.layers`` (OPT), ``transformer.h`` (BLOOM / Falcon / BigCode),
    ``transformer.blocks`` (MPT), ``gpt_neox.layers``, ``llm.model.layers`` (LLaVA-Llama)."""
    inner = getattr(model, "model", None)
    if inner is not None and hasattr(inner, "language_model"):
        return inner.language_model.layers
    lm = getattr(model, "language_model", None)
    if lm is not None and hasattr(lm, "layers"):
        return lm.layers
    cls = model.__class__.__name__
    if cls == "InternVL3":
        return model.language_model.model.layers
    if inner is not None and hasattr(inner, "layers"):
        return inner.layers
    if inner is not None and hasattr(inner, "decoder") and hasattr(inner.decoder, "layers"):
        return inner.decoder.layers
    low = str(model.__class__).lower()
    tr = getattr(model, "transformer", None)
    if tr is not None:
        if "mpt" in low and hasattr(tr, "blocks"):
            return tr.blocks
        if hasattr(tr, "h"):
            return tr.h
    if "neox" in low:
        return model.gpt_neox.layers
    if cls == "LlavaLlamaModel":
        return model.llm.model.layers
    raise NotImplementedError(type(model))


def get_named_linears(module: nn.Module, model: Optional[nn.Module] = None,
                      qwen3_5_quantize_linear_attn: bool = True) -> Dict[str, nn.Linear]:
    """Every ``nn.Linear`` of a block by qualified name (``pre_quant.py:34-44``).  In a Qwen3.5 model
    a full-attention block keeps only its ``mlp.*`` linears, and so does a linear-attention block when
    ``qwen3_5_quantize_linear_attn`` is off."""
    found = {name: m for name, m in module.named_modules() if isinstance(m, nn.Linear)}
    if model is not None and _is_qwen3_5(model):
        kind = getattr(module, "layer_type", None)
        if kind == "full_attention" or (kind == "linear_attention" and not qwen3_5_quantize_linear_attn):
            found = {name: m for name, m in found.items() if name.startswith("mlp.")}
    return found


@torch.no_grad()
def pseudo_quantize_model_weight(model: nn.Module, w_bit: int, q_config: dict,
                                 qwen3_5_quantize_linear_attn: bool = True, device=None) -> None:
    """The AWQ router (``quantizer.py:108-130``): every block linear's weight is replaced in place by
    its pseudo-quantized value, computed by the GPU quantizer in the weight's dtype.  ``q_config``
    holds ``zero_point`` and ``q_group_size``; ``device`` is accepted for the reference's signature
    (each weight is quantized where it lives, staged through the GPU when it lives on the host)."""
    del device
    for layer in get_blocks(model):
        for _, lin in get_named_linears(layer, model=model,
                                        qwen3_5_quantize_linear_attn=qwen3_5_quantize_linear_attn).items():
            lin.weight.data = pseudo_quantize_tensor(lin.weight.data, n_bit=w_bit, **q_config)


@torch.no_grad()
def quantize_model_w4a16(model: nn.Module, group_size: int = 128, zero_point: bool = True,
                         qwen3_5_quantize_linear_attn: bool = True) -> List[str]:
    """Real-int4 counterpart of ``pseudo_quantize_model_weight``: the same block linears
    (``get_blocks`` / ``get_named_linears``) become ``W4A16Linear`` modules holding the AWQ codes the
    router would round the weights to.  Returns the qualified names of the swapped linears."""
    blocks = get_blocks(model)
    prefix = {id(m): n for n, m in model.named_modules()}
    names = []
    for layer in blocks:
        lp = prefix[id(layer)]
        for name, lin in get_named_linears(layer, model=model,
                                           qwen3_5_quantize_linear_attn=qwen3_5_quantize_linear_attn).items():
            _set_module(layer, name, W4A16Linear.from_float(lin, group_size, zero_point))
            names.append(f"{lp}.{name}" if lp else name)
    return names


# What a vLLM export directory takes over from the source checkpoint (tokenizer, chat template,
# generation and processor configs, remote-code modules) and what it never copies from it (weights,
# weight indexes, the config it rewrites): the on-disk format of ``exporters/vllm.py:18-54``.
_CARRIED_FILES = ("tokenizer.json", "tokenizer_config.json", "special_tokens_map.json", "added_tokens.json",
                  "vocab.*", "merges.txt", "*.model", "spiece.model", "sentencepiece.bpe.model",
                  "chat_template*.jinja", "generation_config*.json", "preprocessor_config.json",
                  "processor_config.json", "image_processor_config.json", "video_processor_config.json",
                  "feature_extractor_config.json", "configuration.json", "configuration*.py", "modeling*.py",
                  "processing*.py", "tokenization*.py", "image_processing*.py", "video_processing*.py")
_NEVER_CARRIED = ("config.json", "*.safetensors", "*.bin", "*.pt", "*.pth", "*.ckpt", "*.gguf", "*.onnx",
                  "model.safetensors.index.json", "pytorch_model.bin.index.json")


def _carried_files(source_dir) -> List[Path]:
    """The files of ``source_dir`` an export carries over, in name order."""
    if not source_dir or not Path(source_dir).is_dir():
        return []
    hit = lambda name, pats: any(Path(name).match(p) for p in pats)  # noqa: E731
    return [f for f in sorted(Path(source_dir).iterdir())
            if f.is_file() and hit(f.name, _CARRIED_FILES) and not hit(f.name, _NEVER_CARRIED)]


def export_config(config: dict, group_size: int, ignored_layers: List[str]) -> dict:
    """The export's ``config.json`` from the saved model config (``vllm.py:168-190``): no
    ``quantization_config``; ``rope_theta`` and ``rope_parameters`` each present when the other is
    (a top-level ``rope_theta`` becomes ``{"rope_theta": .., "rope_type": "default"}``, a
    ``rope_parameters["rope_theta"]`` is mirrored at top level); the compressed-tensors
    ``compression_config``."""
    cfg = {k: v for k, v in config.items() if k != "quantization_config"}
    rope = cfg.get("rope_parameters")
    theta = cfg.get("rope_theta")
    if isinstance(rope, dict):
        if theta is None and rope.get("rope_theta") is not None:
            cfg["rope_theta"] = rope["rope_theta"]
    elif theta is not None:
        cfg["rope_parameters"] = {"rope_theta": theta, "rope_type": "default"}
    cfg["compression_config"] = build_compression_config(group_size=group_size, ignored_layers=ignored_layers)
    return cfg


def _check_artifact(name: str, art: "RealQuantLinearArtifact", mod, g: int) -> None:
    """Raise if ``art`` cannot be exported as the packed weight of module ``mod`` (``None`` when the
    model has no module of that name) with group size ``g``."""
    if mod is None:
        raise KeyError(f"the model has no module {name!r} for its quantized artifact")
    if not isinstance(mod, nn.Linear):
        raise TypeError(f"artifact {name!r} targets a {type(mod).__name__}; only nn.Linear modules are exported")
    shape = tuple(mod.weight.shape)
    n, k = shape
    checks = (
        (art.bits == 4 and art.symmetric, f"{name!r} is a {art.bits}-bit "
                                          f"{'symmetric' if art.symmetric else 'asymmetric'} artifact; the "
                                          f"compressed-tensors W4A16 format holds symmetric 4-bit codes"),
        (int(art.group_size) == g, f"{name!r} was quantized with group size {art.group_size}, the export uses {g}"),
        (tuple(art.original_shape) == shape, f"{name!r} was quantized from a {tuple(art.original_shape)} weight; "
                                             f"the module's weight is {shape}"),
        (tuple(art.int_weight.shape) == shape, f"{name!r} holds {tuple(art.int_weight.shape)} codes for a "
                                               f"{shape} weight"),
        (k % g == 0, f"{name!r}: in_features {k} is not a multiple of the group size {g} (the packed format "
                     f"needs whole groups)"),
        (tuple(art.scale.shape) == (n, k // g), f"{name!r} has scales {tuple(art.scale.shape)}, the format "
                                                f"needs {(n, k // g)}"),
    )
    for ok, msg in checks:
        if not ok:
            raise ValueError(msg)


@contextlib.contextmanager
def _modules_swapped(model: nn.Module, replacements: Dict[str, nn.Module]):
    """Replace the named submodules for the duration of the block; the originals come back on exit,
    also when the block raises."""
    saved = []
    try:
        for name, new in replacements.items():
            parent_name, _, child = name.rpartition(".")
            parent = model.get_submodule(parent_name) if parent_name else model
            saved.append((parent, child, parent._modules[child]))
            parent._modules[child] = new
        yield
    finally:
        for parent, child, orig in reversed(saved):
            parent._modules[child] = orig


@torch.no_grad()
def export_vllm_gptq_w4a16(*, model: nn.Module, tokenizer_bundle, artifacts: Dict[str, RealQuantLinearArtifact],
                           export_dir, group_size: int) -> dict:
    """Write GPTQ W4A16 artifacts as a vLLM compressed-tensors ``pack-quantized`` checkpoint: the
    keyword-only interface, files and summary keys of ``exporters/vllm.py:224-327``.

    Every artifact is checked against its module first (``_check_artifact``), so a bad one raises
    before anything is written or swapped.  The model is then saved by its own
    ``save_pretrained(..., safe_serialization=True)`` while the quantized linears are swapped for
    ``VllmPackedInt4Linear`` (codes packed by the GPU packer; the model's modules come back
    afterwards); the tokenizer bundle saves itself, the source checkpoint's inference files are
    carried over, and ``config.json`` is rewritten by ``export_config``, with every unquantized
    ``nn.Linear`` in ``ignore``."""
    if not artifacts:
        raise ValueError("export_vllm_gptq_w4a16 got no quantized artifacts to export")
    g = int(group_size)
    modules = dict(model.named_modules())
    for name, art in artifacts.items():
        _check_artifact(name, art, modules.get(name), g)
    ignored = sorted(n for n, m in modules.items() if isinstance(m, nn.Linear) and n not in artifacts)
    packed = {}
    for name, art in artifacts.items():
        mod = modules[name]
        packed[name] = VllmPackedInt4Linear(
            packed_weight=pack_int4_for_vllm(art.int_weight).cpu(), scale=art.scale.detach().cpu(),
            bias=None if mod.bias is None else mod.bias.detach().cpu(), in_features=mod.in_features,
            out_features=mod.out_features)
    out = Path(export_dir)
    out.mkdir(parents=True, exist_ok=True)
    with _modules_swapped(model, packed):
        model.save_pretrained(out, safe_serialization=True)
    tokenizer_bundle.save_pretrained(str(out))
    carried = []
    for f in _carried_files(getattr(tokenizer_bundle, "source_path", None)):
        if f.resolve() != (out / f.name).resolve():
            shutil.copy2(f, out / f.name)
            carried.append(f.name)
    cfg_path = out / "config.json"
    cfg = export_config(json.loads(cfg_path.read_text(encoding="utf-8")), g, ignored)
    cfg_path.write_text(json.dumps(cfg, ensure_ascii=False, indent=2), encoding="utf-8")
    return {"backend": "vllm", "format": "compressed-tensors", "precision": "W4A16", "path": str(out),
            "quantized_linear_count": len(artifacts), "ignored_linear_count": len(ignored),
            "ignored_layers": ignored, "copied_inference_files": carried}


@torch.no_grad()
def load_vllm_w4a16(model: nn.Module, export_dir) -> List[str]:
    """Load a compressed-tensors ``pack-quantized`` export straight into ``W4A16Linear``
    modules (no re-quantization); returns the replaced module names."""
    from safetensors import safe_open
    path = Path(export_dir)
    cfg = json.loads((path / "config.json").read_text())["compression_config"]
    if cfg.get("format") != "pack-quantized":
        raise ValueError(f"unsupported compression format {cfg.get('format')!r}")
    g = int(cfg["config_groups"]["group_0"]["weights"]["group_size"])
    names = []
    dev = torch.device("cuda")
    with safe_open(str(path / "model.safetensors"), framework="pt", device="cpu") as f:
        keys = set(f.keys())
        for k_ in sorted(keys):
            if not k_.endswith(".weight_packed"):
                continue
            name = k_[: -len(".weight_packed")]
            n, kk = (int(v) for v in f.get_tensor(f"{name}.weight_shape").tolist())
            bias = f.get_tensor(f"{name}.bias").to(dev) if f"{name}.bias" in keys else None
            mod = VllmPackedInt4Linear(packed_weight=f.get_tensor(k_).to(dev),
                                       scale=f.get_tensor(f"{name}.weight_scale").to(dev),
                                       bias=bias, in_features=kk, out_features=n)
            _set_module(model, name, mod)
            names.append(name)
        for k_ in keys:
            if k_.rsplit(".", 1)[0] in names:
                continue
            try:
                t = model.get_parameter(k_)
            except AttributeError:
                try:
                    t = model.get_buffer(k_)
                except AttributeError:
                    continue
            t.data.copy_(f.get_tensor(k_).to(t.device))
    if g <= 0:
        raise ValueError("bad group size in compression_config")
    return names
