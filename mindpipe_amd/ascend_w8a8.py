"""Ascend ``W8A8_DYNAMIC`` checkpoints: writer, verifier and loader.

The on-disk format is the one the reference's dense-Qwen2 export writes
(``scripts/repro/export_fp16_to_ascend_w8a8_dynamic_probe.py:175-257``) and the vLLM-Ascend
``W8A8_DYNAMIC`` linear method reads (``vllm_ascend.patch:3935-4033``):

* each decoder linear ``model.layers.{i}.self_attn.{q,k,v,o}_proj`` / ``mlp.{gate,up,down}_proj``
  stores ``.weight`` int8 ``[N, K]`` (per output channel: ``s = fp32(max|w|) / 127`` clamped at
  1e-8, ``q = round(w / s)`` clamped to +-127), ``.weight_scale`` ``[N, 1]`` and ``.weight_offset``
  ``[N, 1]`` (zeros), both in the source weight's dtype;
* every other tensor keeps its name, shard, dtype and values;
* ``quant_model_description.json`` marks each quantized weight, and the fused ``qkv_proj`` /
  ``gate_up_proj`` names the runtime packs them into, ``"W8A8_DYNAMIC"``, and ``embed_tokens`` /
  ``lm_head`` ``"FLOAT"``; ``model.safetensors.index.json`` maps every tensor to its shard; the
  config loses ``quantization_config`` / ``compression_config``; tokenizer files come along.

How this module is organised.  A checkpoint is handled as a *manifest*: for every tensor name, its
shard, dtype and shape, read from the safetensors headers (eight-byte length, then JSON) without
loading any tensor data.  The export is planned from the source manifest as the manifest the output
must have (``_expected_output``); the writer streams the source shard by shard on the GPU export
quantizer; the verifier reads the output's manifest back and compares it with the planned one,
together with the description and the index, and reports every mismatch it finds at once.  The
loader puts an export into a model from the same manifest.
"""
from __future__ import annotations

import json
import shutil
from dataclasses import dataclass
from pathlib import Path
from typing import Dict, Iterable, List, Optional, Tuple

import torch
from torch import nn

from . import ops
from .runtime import W8A8DynamicLinearMethod

__all__ = ["QUANT_TYPE", "FLOAT_TYPE", "LINEAR_SUFFIXES", "read_config", "export_w8a8_dynamic",
           "verify_w8a8_dynamic", "load_w8a8_dynamic", "W8A8DynamicLinear"]

# ------------------------------------------------------------------ the format
QUANT_TYPE = "W8A8_DYNAMIC"
FLOAT_TYPE = "FLOAT"
LINEAR_SUFFIXES = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
                   "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj")
PACKED_SUFFIXES = ("self_attn.qkv_proj", "mlp.gate_up_proj")   # the runtime's fused module names
TERMINAL_WEIGHTS = ("model.embed_tokens.weight", "lm_head.weight")
TOKENIZER_FILES = ("added_tokens.json", "chat_template.json", "chat_template.jinja", "generation_config.json",
                   "merges.txt", "special_tokens_map.json", "tokenizer.json", "tokenizer.model",
                   "tokenizer_config.json", "vocab.json")
INDEX_FILE = "model.safetensors.index.json"
DESCRIPTION_FILE = "quant_model_description.json"
_DENSE_QWEN2 = ("qwen2", "Qwen2ForCausalLM")
_INT8 = "I8"
_FLOATS = frozenset({"F16", "BF16", "F32", "F64"})
_SIDE_TENSORS = ("weight_scale", "weight_offset")


def _json(path: Path):
    return json.loads(path.read_text(encoding="utf-8"))


def _write_json(path: Path, obj) -> None:
    path.write_text(json.dumps(obj, ensure_ascii=False, indent=2) + "\n", encoding="utf-8")


# ------------------------------------------------------------------ manifests
@dataclass(frozen=True)
class TensorInfo:
    shard: str
    dtype: str        # safetensors dtype tag ("F16", "BF16", "I8", ...)
    shape: Tuple[int, ...]


def _header(shard: Path) -> Dict[str, Tuple[str, Tuple[int, ...]]]:
    """``{tensor: (dtype, shape)}`` of one safetensors file, from its JSON header alone."""
    with open(shard, "rb") as f:
        size = int.from_bytes(f.read(8), "little")
        if size <= 0 or size > (1 << 27):
            raise ValueError(f"{shard} is not a safetensors file (header size {size})")
        head = json.loads(f.read(size))
    return {k: (v["dtype"].upper(), tuple(int(d) for d in v["shape"])) for k, v in head.items() if k != "__metadata__"}


def _headers_of(directory: Path, shards: Iterable[str]) -> Dict[str, TensorInfo]:
    man: Dict[str, TensorInfo] = {}
    for shard in sorted(set(shards)):
        for name, (dt, shape) in _header(directory / shard).items():
            if name in man:
                raise ValueError(f"tensor {name} appears in both {man[name].shard} and {shard}")
            man[name] = TensorInfo(shard, dt, shape)
    return man


def _index(directory: Path) -> Optional[Dict[str, str]]:
    """The index's ``weight_map`` (tensor -> shard file), checked for plain file names, or None."""
    path = directory / INDEX_FILE
    if not path.is_file():
        return None
    wm = _json(path).get("weight_map")
    if not isinstance(wm, dict) or not wm:
        raise ValueError(f"{path} has no weight_map")
    for name, shard in wm.items():
        if not isinstance(name, str) or not name or not isinstance(shard, str) or Path(shard).name != shard \
                or shard in ("", ".", ".."):
            raise ValueError(f"{path} maps {name!r} to an unsafe shard name {shard!r}")
    return wm


def _manifest(directory: Path) -> Dict[str, TensorInfo]:
    """A checkpoint's manifest: the shards its index names, or every ``*.safetensors`` file."""
    wm = _index(directory)
    if wm is None:
        shards = [p.name for p in directory.glob("*.safetensors")]
        if not shards:
            raise FileNotFoundError(f"no safetensors checkpoint in {directory}")
        return _headers_of(directory, shards)
    missing = sorted({s for s in wm.values() if not (directory / s).is_file()})
    if missing:
        raise FileNotFoundError(f"{directory} lacks shard file(s) named by its index: {', '.join(missing)}")
    man = _headers_of(directory, wm.values())
    absent = sorted(n for n, s in wm.items() if n not in man or man[n].shard != s)
    if absent:
        raise ValueError(f"{len(absent)} indexed tensor(s) are not in their shard; first: {', '.join(absent[:8])}")
    return {n: man[n] for n in wm}


_ELEM_BYTES = {"F64": 8, "I64": 8, "F32": 4, "I32": 4, "F16": 2, "BF16": 2, "I16": 2, "I8": 1, "U8": 1, "BOOL": 1}


def _nbytes(info: TensorInfo) -> int:
    n = 1
    for d in info.shape:
        n *= d
    return n * _ELEM_BYTES.get(info.dtype, 1)


def _by_shard(names: Iterable[str], man: Dict[str, TensorInfo]) -> Dict[str, List[str]]:
    out: Dict[str, List[str]] = {}
    for n in sorted(names):
        out.setdefault(man[n].shard, []).append(n)
    return out


# ------------------------------------------------------------------ the source
def _directories(source, output) -> Tuple[Path, Path]:
    src, out = Path(source).expanduser().resolve(), Path(output).expanduser().resolve()
    if not src.is_dir():
        raise FileNotFoundError(f"source checkpoint directory {src} does not exist")
    nested = src == out or src in out.parents or out in src.parents
    if nested:
        raise ValueError(f"export needs separate, non-nested source and output directories (source {src}, "
                         f"output {out})")
    return src, out


def read_config(source) -> dict:
    """``config.json`` of the source, which must describe a dense Qwen2 / Qwen2.5 causal LM with at
    least one decoder layer (the one family the format is defined for)."""
    path = Path(source) / "config.json"
    if not path.is_file():
        raise FileNotFoundError(f"{path} does not exist")
    cfg = _json(path)
    if not isinstance(cfg, dict):
        raise ValueError(f"{path} does not hold a JSON object")
    mt, arch = _DENSE_QWEN2
    if cfg.get("model_type") != mt or arch not in (cfg.get("architectures") or []):
        raise ValueError(f"Expected dense Qwen2/Qwen2.5 checkpoint (model_type {mt!r}, architecture {arch!r}); "
                         f"{path} has model_type {cfg.get('model_type')!r}, architectures {cfg.get('architectures')!r}")
    layers = cfg.get("num_hidden_layers")
    if isinstance(layers, bool) or not isinstance(layers, int) or layers < 1:
        raise ValueError(f"{path}: num_hidden_layers must be a positive integer, got {layers!r}")
    return cfg


def _linear_weights(cfg: dict) -> List[str]:
    return [f"model.layers.{i}.{s}.weight" for i in range(cfg["num_hidden_layers"]) for s in LINEAR_SUFFIXES]


def _description(cfg: dict, quantized: Iterable[str]) -> Dict[str, str]:
    desc = {t: FLOAT_TYPE for t in TERMINAL_WEIGHTS}
    desc.update({t: QUANT_TYPE for t in quantized})
    for i in range(cfg["num_hidden_layers"]):
        desc.update({f"model.layers.{i}.{s}.weight": QUANT_TYPE for s in PACKED_SUFFIXES})
    return dict(sorted(desc.items()))


def _expected_output(src_man: Dict[str, TensorInfo], quantized: List[str]) -> Dict[str, TensorInfo]:
    """The manifest the export must have: every source tensor in its shard, each quantized weight as
    int8 of its shape with ``[N, 1]`` scale and offset in the source weight's dtype beside it."""
    missing = [t for t in quantized if t not in src_man]
    if missing:
        raise ValueError(f"source checkpoint is missing {len(missing)} required linear weight(s) of its decoder "
                         f"layers: {', '.join(missing[:8])}")
    exp = dict(src_man)
    for t in quantized:
        info = src_man[t]
        if len(info.shape) != 2:
            raise ValueError(f"{t} has shape {info.shape}; a linear weight is [N, K]")
        if info.dtype not in _FLOATS:
            raise ValueError(f"{t} is {info.dtype}: the export quantizes a floating-point weight")
        base = t[: -len(".weight")]
        exp[t] = TensorInfo(info.shard, _INT8, info.shape)
        for side in _SIDE_TENSORS:
            exp[f"{base}.{side}"] = TensorInfo(info.shard, info.dtype, (info.shape[0], 1))
    return exp


# ------------------------------------------------------------------ writer
def _quantize(name: str, w: torch.Tensor) -> Dict[str, torch.Tensor]:
    """One linear weight through the GPU export quantizer (bit-exact to the fp32 rule,
    ``export_fp16_to_ascend_w8a8_dynamic_probe.py:175-195``): its int8 codes, scale and zero offset."""
    if not w.is_floating_point():
        raise ValueError(f"{name}: the export needs a floating-point weight, got {w.dtype}")
    if w.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError(f"{name}: the GPU export quantizer takes fp16 or bf16 weights, got {w.dtype}")
    if not torch.cuda.is_available():
        raise RuntimeError("the W8A8 export quantizer runs on the GPU; none is visible")
    q, _, scale = ops.w8_quantize_per_channel(w.cuda().contiguous(), "export")
    scale = scale.reshape(-1, 1).cpu()
    base = name[: -len(".weight")]
    return {name: q.cpu(), f"{base}.weight_scale": scale, f"{base}.weight_offset": torch.zeros_like(scale)}


def export_w8a8_dynamic(source, output, *, overwrite: bool = False) -> dict:
    """Write the ``W8A8_DYNAMIC`` export of a dense fp16 / bf16 Qwen2 checkpoint into ``output``,
    then verify it.  Returns (and stores as ``conversion_summary.json``) the export summary:
    ``converted_linear_modules``, ``output_tensors``, ``quant_description_entries`` and the
    verifier's report under ``validation``."""
    from safetensors import safe_open
    from safetensors.torch import save_file
    src, out = _directories(source, output)
    cfg = read_config(src)
    src_man = _manifest(src)
    quantized = _linear_weights(cfg)
    expected = _expected_output(src_man, quantized)
    if out.exists():
        if not overwrite:
            raise FileExistsError(f"{out} exists; pass overwrite=True to replace it")
        shutil.rmtree(out)
    out.mkdir(parents=True)
    qset = set(quantized)
    for shard, names in _by_shard(src_man, src_man).items():
        written: Dict[str, torch.Tensor] = {}
        with safe_open(str(src / shard), framework="pt", device="cpu") as f:
            for n in names:
                t = f.get_tensor(n)
                written.update(_quantize(n, t) if n in qset else {n: t})
        save_file(written, str(out / shard))
        del written
    total = sum(_nbytes(i) for i in expected.values())
    _write_json(out / INDEX_FILE, {"metadata": {"total_size": total},
                                   "weight_map": {n: i.shard for n, i in sorted(expected.items())}})
    desc = _description(cfg, quantized)
    _write_json(out / DESCRIPTION_FILE, desc)
    _write_json(out / "config.json",
                {k: v for k, v in cfg.items() if k not in ("quantization_config", "compression_config")})
    for fname in TOKENIZER_FILES:
        if (src / fname).is_file():
            shutil.copy2(src / fname, out / fname)
    summary = {"source": str(src), "output": str(out), "quant_type": QUANT_TYPE,
               "converted_linear_modules": len(quantized), "output_tensors": len(expected),
               "quant_description_entries": len(desc), "validation": verify_w8a8_dynamic(out, src)}
    _write_json(out / "conversion_summary.json", summary)
    return summary


# ------------------------------------------------------------------ verifier
def verify_w8a8_dynamic(output, source) -> dict:
    """Compare an export with the manifest planned from its source.  Checked: every planned tensor
    is in the output's shards with the planned dtype and shape (int8 ``[N, K]`` weights,
    ``[N, 1]`` scales and offsets in the source weight's dtype, the rest unchanged); the index, when
    present, maps each planned tensor to the shard that holds it; the description marks each
    quantized weight ``W8A8_DYNAMIC`` and the terminal weights ``FLOAT``.  Every mismatch is
    reported in one ``ValueError``."""
    src, out = Path(source).resolve(), Path(output).resolve()
    if not out.is_dir():
        raise FileNotFoundError(f"export directory {out} does not exist")
    cfg = read_config(src)
    src_man = _manifest(src)
    quantized = _linear_weights(cfg)
    expected = _expected_output(src_man, quantized)
    shards = [p.name for p in out.glob("*.safetensors")]
    if not shards:
        raise FileNotFoundError(f"no safetensors shards in {out}")
    actual = _headers_of(out, shards)
    problems: List[str] = []
    for n, want in expected.items():
        got = actual.get(n)
        if got is None:
            problems.append(f"{n} is missing")
            continue
        if got.dtype != want.dtype:
            kind = "expected source weight dtype" if n.endswith(_SIDE_TENSORS) else "expected"
            problems.append(f"{n}: dtype {got.dtype}, {kind} {want.dtype}")
        if got.shape != want.shape:
            problems.append(f"{n}: shape {got.shape}, expected {want.shape}")
    index = _index(out)
    if index is not None:
        for n in expected:
            if n in actual and index.get(n) != actual[n].shard:
                problems.append(f"index maps {n} to {index.get(n)!r}, but it is in {actual[n].shard!r}")
    desc_path = out / DESCRIPTION_FILE
    desc = _json(desc_path) if desc_path.is_file() else None
    if not isinstance(desc, dict):
        problems.append(f"{DESCRIPTION_FILE} is missing or not a JSON object")
        desc = {}
    problems += [f"description marks {t} {desc.get(t)!r}, not {QUANT_TYPE}" for t in quantized
                 if desc.get(t) != QUANT_TYPE]
    terminals = [t for t in TERMINAL_WEIGHTS if t in src_man]
    problems += [f"description marks {t} {desc.get(t)!r}, not {FLOAT_TYPE}" for t in terminals
                 if desc.get(t) != FLOAT_TYPE]
    if problems:
        head = "; ".join(problems[:8])
        raise ValueError(f"W8A8_DYNAMIC export {out} fails {len(problems)} check(s): {head}")
    return {"validated_linear_weights": len(quantized), "validated_scale_offset_pairs": len(quantized),
            "validated_float_terminal_weights": len(terminals), "checked_tensors": len(expected),
            "output_index_present": index is not None}


# ------------------------------------------------------------------ loader
class W8A8DynamicLinear(nn.Module):
    """A linear layer in the runtime method's form: ``weight`` int8 ``[N, K]``, ``weight_scale`` /
    ``weight_offset`` as stored, ``weight_scale_fp32`` after ``process_weights_after_loading``; the
    forward is ``W8A8DynamicLinearMethod.apply`` (per-token int8 quant, int8 GEMM, per-token x
    per-channel epilogue) in ``params_dtype``."""

    def __init__(self, weight: torch.Tensor, weight_scale: torch.Tensor, weight_offset: torch.Tensor,
                 bias: Optional[torch.Tensor], params_dtype: torch.dtype):
        super().__init__()
        self.out_features, self.in_features = (int(d) for d in weight.shape)
        self.weight = nn.Parameter(weight, requires_grad=False)
        self.weight_scale = nn.Parameter(weight_scale, requires_grad=False)
        self.weight_offset = nn.Parameter(weight_offset, requires_grad=False)
        self.bias = nn.Parameter(bias, requires_grad=False) if bias is not None else None
        self.params_dtype = params_dtype
        self.quant_method = W8A8DynamicLinearMethod()
        self.quant_method.process_weights_after_loading(self)

    def forward(self, x):
        b = None if self.bias is None else self.bias.to(x.dtype if not isinstance(x, tuple) else self.params_dtype)
        return self.quant_method.apply(self, x, b)


def _quantized_module(lin: nn.Linear, q, scale, bias, target: str) -> nn.Module:
    from .smoothquant import SmoothQuantLinear
    dev, pdt = lin.weight.device, lin.weight.dtype
    if target == "runtime":
        off = torch.zeros_like(scale)
        return W8A8DynamicLinear(q.to(dev), scale.to(dev), off.to(dev), None if bias is None else bias.to(dev), pdt)
    new = SmoothQuantLinear(lin.in_features, lin.out_features, bias is not None, dtype=pdt,
                            scale_rule="export").to(dev)
    new.weight = q.to(dev)
    new.weight_scale = scale.reshape(-1).to(device=dev, dtype=torch.float32)
    if bias is not None:
        new.bias = bias.to(device=dev, dtype=pdt)
    return new


@torch.no_grad()
def load_w8a8_dynamic(model: nn.Module, export_dir, *, target: str = "runtime") -> List[str]:
    """Load a ``W8A8_DYNAMIC`` export into ``model`` without requantizing.  Each weight the
    description marks ``W8A8_DYNAMIC`` and the checkpoint holds replaces its ``nn.Linear`` with a
    ``W8A8DynamicLinear`` (``target="runtime"``) or a ``SmoothQuantLinear`` on the export scale
    rule (``target="smoothquant"``): the stored codes, the fp32 value of the stored scale and the
    linear's bias (the checkpoint's, else the module's).  Every other checkpoint tensor is copied
    into the model's parameter or buffer of that name.  Returns the replaced module names."""
    from safetensors import safe_open
    if target not in ("runtime", "smoothquant"):
        raise ValueError(f"unknown target {target!r}")
    d = Path(export_dir)
    man = _manifest(d)
    desc = _json(d / DESCRIPTION_FILE)
    modules = sorted(t[: -len(".weight")] for t, kind in desc.items() if kind == QUANT_TYPE and t in man)
    consumed = set()
    for base in modules:
        consumed |= {f"{base}.weight", f"{base}.weight_scale", f"{base}.weight_offset", f"{base}.bias"}
    replaced: List[str] = []
    for shard, names in _by_shard(man, man).items():
        with safe_open(str(d / shard), framework="pt", device="cpu") as f:
            mine = [b for b in modules if man[f"{b}.weight"].shard == shard]
            for base in mine:
                lin = model.get_submodule(base)
                if not isinstance(lin, nn.Linear):
                    raise TypeError(f"{base} is a {type(lin).__name__}, not an nn.Linear")
                q = f.get_tensor(f"{base}.weight")
                if q.dtype != torch.int8 or q.shape != lin.weight.shape:
                    raise ValueError(f"{base}.weight is {q.dtype} {tuple(q.shape)}; the model needs int8 "
                                     f"{tuple(lin.weight.shape)}")
                if torch.count_nonzero(f.get_tensor(f"{base}.weight_offset")):
                    raise ValueError(f"{base}.weight_offset is not zero; W8A8_DYNAMIC weights are symmetric")
                bname = f"{base}.bias"
                bias = f.get_tensor(bname) if man.get(bname) is not None and man[bname].shard == shard else \
                    (None if lin.bias is None else lin.bias.detach().clone())
                parent, _, child = base.rpartition(".")
                setattr(model.get_submodule(parent) if parent else model, child,
                        _quantized_module(lin, q, f.get_tensor(f"{base}.weight_scale"), bias, target))
                replaced.append(base)
            for n in names:
                if n in consumed:
                    continue
                try:
                    dst = model.get_parameter(n)
                except AttributeError:
                    try:
                        dst = model.get_buffer(n)
                    except AttributeError:
                        continue
                dst.data.copy_(f.get_tensor(n).to(dst.device))
    return replaced
