"""Ascend ``W8A8_DYNAMIC`` checkpoints: writer, verifier and loader.

The on-disk format is the one ``scripts/repro/export_fp16_to_ascend_w8a8_dynamic_probe.py`` writes for
a dense Qwen2 / Qwen2.5 model (``:175-257``) and the vLLM-Ascend ``W8A8_DYNAMIC`` linear method reads
(``vllm_ascend.patch:3935-4033``):

* each decoder linear ``model.layers.{i}.{q,k,v,o}_proj`` / ``mlp.{gate,up,down}_proj`` stores
  ``.weight`` int8 ``[N, K]`` (per-output-channel, the fp32 rule
  ``s = max|w| / 127`` clamped at 1e-8, ``q = round(w / s).clamp(-127, 127)``), ``.weight_scale``
  ``[N, 1]`` and ``.weight_offset`` ``[N, 1]`` (zeros), both in the source weight's dtype;
* every other tensor is copied unchanged;
* ``quant_model_description.json`` maps each quantized weight (and the fused ``qkv_proj`` /
  ``gate_up_proj`` names the runtime packs) to ``"W8A8_DYNAMIC"`` and ``embed_tokens`` / ``lm_head``
  to ``"FLOAT"``; ``model.safetensors.index.json`` indexes the shards; the config loses its
  ``quantization_config`` / ``compression_config``; tokenizer files are copied.

``export_w8a8_dynamic`` quantizes with the GPU export quantizer (bit-exact to the fp32 rule) and
verifies what it wrote; ``verify_w8a8_dynamic`` is the verify-only check; ``load_w8a8_dynamic`` puts
an export into a model as ``W8A8DynamicLinear`` (the runtime method's layer) or ``SmoothQuantLinear``
modules holding the stored int8 codes and scales -- no requantization.
"""
from __future__ import annotations

import gc
import json
import shutil
from pathlib import Path
from typing import Dict, List, Optional, Set, Tuple

import torch
from torch import nn

from . import ops
from .runtime import W8A8DynamicLinearMethod

__all__ = ["QUANT_TYPE", "FLOAT_TYPE", "LINEAR_SUFFIXES", "export_w8a8_dynamic", "verify_w8a8_dynamic",
           "load_w8a8_dynamic", "W8A8DynamicLinear"]

QUANT_TYPE = "W8A8_DYNAMIC"
FLOAT_TYPE = "FLOAT"
MODEL_TYPE = "qwen2"
ARCHITECTURE = "Qwen2ForCausalLM"
# the tokenizer / generation files an export carries over from its source
INFERENCE_FILE_NAMES = ("added_tokens.json", "chat_template.json", "chat_template.jinja", "generation_config.json",
                        "merges.txt", "special_tokens_map.json", "tokenizer.json", "tokenizer.model",
                        "tokenizer_config.json", "vocab.json")
LINEAR_SUFFIXES = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
                   "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj")
_FLOAT_DTYPES = {"BF16", "F16", "F32", "F64"}
_TERMINALS = ("model.embed_tokens.weight", "lm_head.weight")


# ------------------------------------------------------------------ source checks
def _paths(source, output) -> Tuple[Path, Path]:
    src, out = Path(source).expanduser().resolve(), Path(output).expanduser().resolve()
    if not src.is_dir():
        raise FileNotFoundError(f"Source checkpoint directory does not exist: {src}")
    if src == out or src in out.parents or out in src.parents:
        raise ValueError(f"source and output must be separate, non-nested directories: source={src}, output={out}")
    return src, out


def read_config(source) -> dict:
    """``config.json`` of a dense Qwen2 / Qwen2.5 checkpoint (the only family the format covers)."""
    path = Path(source) / "config.json"
    if not path.is_file():
        raise FileNotFoundError(f"Missing config.json in {source}")
    cfg = json.loads(path.read_text(encoding="utf-8"))
    if not isinstance(cfg, dict):
        raise ValueError(f"Invalid JSON object in {path}")
    if cfg.get("model_type") != MODEL_TYPE:
        raise ValueError(f"Expected dense Qwen2/Qwen2.5 model_type={MODEL_TYPE!r}, got {cfg.get('model_type')!r}.")
    if ARCHITECTURE not in (cfg.get("architectures") or []):
        raise ValueError(f"Expected architectures to contain {ARCHITECTURE!r}, got {cfg.get('architectures')!r}.")
    try:
        layers = int(cfg["num_hidden_layers"])
    except (KeyError, TypeError, ValueError) as exc:
        raise ValueError("config.json has no valid num_hidden_layers") from exc
    if layers <= 0:
        raise ValueError("num_hidden_layers must be positive")
    return cfg


def _shard_name(name, where) -> str:
    if not isinstance(name, str) or not name or Path(name).name != name:
        raise ValueError(f"Invalid or unsafe shard name in {where}: {name!r}")
    return name


def _read_index(directory: Path) -> Optional[Dict[str, str]]:
    idx = directory / "model.safetensors.index.json"
    if not idx.is_file():
        return None
    data = json.loads(idx.read_text(encoding="utf-8"))
    wm = data.get("weight_map") if isinstance(data, dict) else None
    if not isinstance(wm, dict) or not wm:
        raise ValueError(f"Invalid weight_map in {idx}")
    out = {}
    for t, f in wm.items():
        if not isinstance(t, str) or not t:
            raise ValueError(f"Invalid tensor name in {idx}: {t!r}")
        out[t] = _shard_name(f, idx)
    return out


def _scan_shards(directory: Path) -> Dict[str, str]:
    from safetensors import safe_open
    shards = sorted(directory.glob("*.safetensors"))
    if not shards:
        raise FileNotFoundError(f"No safetensors checkpoint found in {directory}")
    wm: Dict[str, str] = {}
    for sp in shards:
        with safe_open(str(sp), framework="pt", device="cpu") as f:
            for t in f.keys():
                if t in wm:
                    raise ValueError(f"Duplicate tensor across shards: {t}")
                wm[t] = sp.name
    return wm


def _source_map(source: Path) -> Dict[str, str]:
    wm = _read_index(source)
    if wm is None:
        if not (source / "model.safetensors").is_file():
            raise FileNotFoundError(f"No safetensors checkpoint found in {source}")
        return _scan_shards(source)
    for f in set(wm.values()):
        if not (source / f).is_file():
            raise FileNotFoundError(f"Source shard missing: {source / f}")
    return wm


def quantized_weight_names(cfg: dict) -> Set[str]:
    return {f"model.layers.{i}.{s}.weight" for i in range(int(cfg["num_hidden_layers"])) for s in LINEAR_SUFFIXES}


def _by_file(wm: Dict[str, str]) -> Dict[str, List[str]]:
    out: Dict[str, List[str]] = {}
    for t, f in wm.items():
        out.setdefault(f, []).append(t)
    return out


# ------------------------------------------------------------------ writer
def _quantize_export(w: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """The export quantizer of one weight on the GPU: ``(int8 [N, K], scale [N, 1], offset [N, 1])``,
    scale and offset in the weight's dtype (``export_fp16_to_ascend_w8a8_dynamic_probe.py:175-195``)."""
    if w.ndim != 2:
        raise ValueError(f"Expected a two-dimensional Linear weight, got {tuple(w.shape)}")
    if not w.is_floating_point():
        raise ValueError(f"Expected a floating-point source weight, got {w.dtype}")
    if w.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError(f"the GPU export quantizer takes fp16 / bf16 weights, got {w.dtype}")
    if not torch.cuda.is_available():
        raise RuntimeError("the W8A8 export quantizer runs on the GPU only; no GPU is visible")
    q, _s32, ssrc = ops.w8_quantize_per_channel(w.cuda().contiguous(), "export")
    scale = ssrc.reshape(-1, 1).cpu().contiguous()
    return q.cpu().contiguous(), scale, torch.zeros_like(scale)


def export_w8a8_dynamic(source, output, *, overwrite: bool = False) -> dict:
    """Convert a dense fp16 / bf16 Qwen2 checkpoint to ``W8A8_DYNAMIC``, then verify it.  Returns the
    conversion summary (also written to ``conversion_summary.json``)."""
    from safetensors import safe_open
    from safetensors.torch import save_file
    src, out = _paths(source, output)
    cfg = read_config(src)
    src_map = _source_map(src)
    qnames = quantized_weight_names(cfg)
    missing = sorted(qnames - set(src_map))
    if missing:
        raise ValueError(f"Source checkpoint is missing {len(missing)} required dense Qwen2 Linear weights; "
                         f"first entries: {', '.join(missing[:8])}")
    if out.exists():
        if not overwrite:
            raise FileExistsError(f"{out} already exists; pass overwrite=True to replace it")
        shutil.rmtree(out)
    out.mkdir(parents=True)
    for name in INFERENCE_FILE_NAMES:
        if (src / name).is_file():
            shutil.copy2(src / name, out / name)
    clean = {k: v for k, v in cfg.items() if k not in ("compression_config", "quantization_config")}
    (out / "config.json").write_text(json.dumps(clean, ensure_ascii=False, indent=2) + "\n", encoding="utf-8")
    desc = {t: FLOAT_TYPE for t in _TERMINALS}
    for t in sorted(qnames):
        desc[t] = QUANT_TYPE
    for i in range(int(cfg["num_hidden_layers"])):
        desc[f"model.layers.{i}.self_attn.qkv_proj.weight"] = QUANT_TYPE
        desc[f"model.layers.{i}.mlp.gate_up_proj.weight"] = QUANT_TYPE
    (out / "quant_model_description.json").write_text(json.dumps(desc, ensure_ascii=False, indent=2) + "\n",
                                                      encoding="utf-8")
    out_map: Dict[str, str] = {}
    converted = n_tensors = total = 0
    for fname, names in sorted(_by_file(src_map).items()):
        tensors: Dict[str, torch.Tensor] = {}
        with safe_open(str(src / fname), framework="pt", device="cpu") as f:
            avail = set(f.keys())
            lost = sorted(set(names) - avail)
            if lost:
                raise ValueError(f"{fname} misses {len(lost)} indexed tensors; first: {', '.join(lost[:8])}")
            for t in sorted(names):
                v = f.get_tensor(t)
                if t in qnames:
                    q, sc, off = _quantize_export(v)
                    p = t[: -len(".weight")]
                    tensors.update({t: q, f"{p}.weight_scale": sc, f"{p}.weight_offset": off})
                    converted += 1
                else:
                    tensors[t] = v
        save_file(tensors, str(out / fname))
        for t, v in tensors.items():
            out_map[t] = fname
            total += v.numel() * v.element_size()
        n_tensors += len(tensors)
        del tensors
        gc.collect()
    (out / "model.safetensors.index.json").write_text(
        json.dumps({"metadata": {"total_size": total}, "weight_map": dict(sorted(out_map.items()))},
                   ensure_ascii=False, indent=2) + "\n", encoding="utf-8")
    report = verify_w8a8_dynamic(out, src)
    summary = {"source": str(src), "output": str(out), "model_type": cfg["model_type"], "architecture": ARCHITECTURE,
               "converted_linear_modules": converted, "output_tensors": n_tensors,
               "quant_description_entries": len(desc), "format": "ascend_w8a8_dynamic_probe_from_fp16",
               "validation": report,
               "notes": "Dense transformer block Linear weights are W8A8_DYNAMIC; embed_tokens and lm_head remain FLOAT."}
    (out / "conversion_summary.json").write_text(json.dumps(summary, ensure_ascii=False, indent=2) + "\n",
                                                 encoding="utf-8")
    return summary


# ------------------------------------------------------------------ verifier
def verify_w8a8_dynamic(output, source) -> dict:
    """Check an export against its source: every source tensor present, each quantized weight int8
    ``[N, K]`` with ``weight_scale`` / ``weight_offset`` ``[N, 1]`` in the source weight's dtype, the
    description's ``W8A8_DYNAMIC`` / ``FLOAT`` entries, and (when present) the index against the shards."""
    from safetensors import safe_open
    src, out = Path(source).resolve(), Path(output).resolve()
    if not out.is_dir():
        raise FileNotFoundError(f"Output checkpoint directory does not exist: {out}")
    cfg = read_config(src)
    src_map = _source_map(src)
    qnames = quantized_weight_names(cfg)
    indexed = _read_index(out)
    actual = _scan_shards(out)
    expected = set(src_map)
    for t in qnames:
        p = t[: -len(".weight")]
        expected |= {f"{p}.weight_scale", f"{p}.weight_offset"}
    missing = sorted(expected - set(actual))
    if missing:
        raise ValueError(f"Output misses {len(missing)} required tensors; first: {', '.join(missing[:8])}")
    if indexed is not None:
        lost = sorted(expected - set(indexed))
        if lost:
            raise ValueError(f"Output index misses {len(lost)} required tensors; first: {', '.join(lost[:8])}")
        wrong = sorted(t for t in expected if indexed[t] != actual[t])
        if wrong:
            raise ValueError(f"Output index maps {len(wrong)} tensors to the wrong shard; first: {', '.join(wrong[:8])}")
    dpath = out / "quant_model_description.json"
    if not dpath.is_file():
        raise FileNotFoundError(f"Missing quantization description: {dpath}")
    desc = json.loads(dpath.read_text(encoding="utf-8"))
    if not isinstance(desc, dict):
        raise ValueError(f"Invalid quantization description: {dpath}")
    bad = sorted(t for t in qnames if desc.get(t) != QUANT_TYPE)
    if bad:
        raise ValueError(f"Description has {len(bad)} invalid W8A8_DYNAMIC entries; first: {', '.join(bad[:8])}")
    terminals = set(_TERMINALS) & set(src_map)
    bad = sorted(t for t in terminals if desc.get(t) != FLOAT_TYPE)
    if bad:
        raise ValueError("Description does not keep terminal weights FLOAT: " + ", ".join(bad))
    src_dtypes = {}
    for fname, names in _by_file(src_map).items():
        want = qnames.intersection(names)
        if want:
            with safe_open(str(src / fname), framework="pt", device="cpu") as f:
                for t in want:
                    src_dtypes[t] = str(f.get_slice(t).get_dtype()).upper()
    checked = 0
    for fname, names in _by_file({t: actual[t] for t in qnames}).items():
        with safe_open(str(out / fname), framework="pt", device="cpu") as f:
            for t in sorted(names):
                if str(f.get_slice(t).get_dtype()).upper() not in {"I8", "INT8"}:
                    raise ValueError(f"{t} has dtype {f.get_slice(t).get_dtype()}, expected int8")
                shape = tuple(f.get_slice(t).get_shape())
                if len(shape) != 2:
                    raise ValueError(f"{t} has invalid shape {shape}")
                p = t[: -len(".weight")]
                for suf in ("weight_scale", "weight_offset"):
                    pn = f"{p}.{suf}"
                    dt = str(f.get_slice(pn).get_dtype()).upper()
                    if dt != src_dtypes[t]:
                        raise ValueError(f"{pn} has dtype {dt}, expected source weight dtype {src_dtypes[t]}")
                    if tuple(f.get_slice(pn).get_shape()) != (shape[0], 1):
                        raise ValueError(f"{pn} has shape {tuple(f.get_slice(pn).get_shape())}, expected ({shape[0]}, 1)")
                checked += 1
    for t in sorted(terminals):
        with safe_open(str(out / actual[t]), framework="pt", device="cpu") as f:
            if str(f.get_slice(t).get_dtype()).upper() not in _FLOAT_DTYPES:
                raise ValueError(f"{t} is not floating point")
    if checked != len(qnames):
        raise AssertionError(f"Validated {checked} quantized weights, expected {len(qnames)}")
    return {"validated_linear_weights": checked, "validated_scale_offset_pairs": checked,
            "validated_float_terminal_weights": len(terminals), "all_linear_weights_int8": True,
            "all_scale_offset_shapes_valid": True, "all_scale_offset_dtypes_match_source": True,
            "output_index_present": indexed is not None}


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


def _set_module(model: nn.Module, name: str, new: nn.Module) -> None:
    parent, _, child = name.rpartition(".")
    setattr(model.get_submodule(parent) if parent else model, child, new)


@torch.no_grad()
def load_w8a8_dynamic(model: nn.Module, export_dir, *, target: str = "runtime") -> List[str]:
    """Load a ``W8A8_DYNAMIC`` export into ``model`` without requantizing: each quantized weight's
    ``nn.Linear`` becomes a ``W8A8DynamicLinear`` (``target="runtime"``) or a ``SmoothQuantLinear``
    with the export scale rule (``target="smoothquant"``) holding the stored codes, the fp32 copy of
    the stored scale and the linear's bias; every other tensor is copied into the model's parameter
    or buffer of that name.  Returns the replaced module names."""
    from safetensors import safe_open
    from .smoothquant import SmoothQuantLinear
    if target not in ("runtime", "smoothquant"):
        raise ValueError(f"unknown target {target!r}")
    d = Path(export_dir)
    desc = json.loads((d / "quant_model_description.json").read_text(encoding="utf-8"))
    wm = _read_index(d) or _scan_shards(d)
    qset = {t for t, kind in desc.items() if kind == QUANT_TYPE and t in wm}
    done: List[str] = []
    handled: Set[str] = set()
    for fname, names in sorted(_by_file(wm).items()):
        with safe_open(str(d / fname), framework="pt", device="cpu") as f:
            for t in sorted(set(names) & qset):
                p = t[: -len(".weight")]
                lin = model.get_submodule(p)
                if not isinstance(lin, nn.Linear):
                    raise TypeError(f"{p} is {type(lin).__name__}, expected nn.Linear")
                q = f.get_tensor(t)
                if q.dtype != torch.int8 or tuple(q.shape) != tuple(lin.weight.shape):
                    raise ValueError(f"{t}: int8 {tuple(lin.weight.shape)} expected, got {q.dtype} {tuple(q.shape)}")
                sc, off = f.get_tensor(f"{p}.weight_scale"), f.get_tensor(f"{p}.weight_offset")
                if torch.any(off != 0):
                    raise ValueError(f"{p}.weight_offset is not zero: W8A8_DYNAMIC is symmetric")
                bname = f"{p}.bias"
                bias = (f.get_tensor(bname) if bname in wm and wm[bname] == fname else
                        (lin.bias.detach().clone() if lin.bias is not None else None))
                dev, pdt = lin.weight.device, lin.weight.dtype
                if target == "runtime":
                    new = W8A8DynamicLinear(q.to(dev), sc.to(dev), off.to(dev),
                                            None if bias is None else bias.to(dev), pdt)
                else:
                    new = SmoothQuantLinear(lin.in_features, lin.out_features, bias is not None, dtype=pdt,
                                            scale_rule="export").to(dev)
                    new.weight = q.to(dev)
                    new.weight_scale = sc.reshape(-1).to(device=dev, dtype=torch.float32)
                    if bias is not None:
                        new.bias = bias.to(device=dev, dtype=pdt)
                _set_module(model, p, new)
                done.append(p)
                handled |= {t, f"{p}.weight_scale", f"{p}.weight_offset", bname}
    for fname, names in sorted(_by_file(wm).items()):
        rest = [t for t in names if t not in handled]
        if not rest:
            continue
        with safe_open(str(d / fname), framework="pt", device="cpu") as f:
            for t in rest:
                try:
                    dst = model.get_parameter(t)
                except AttributeError:
                    try:
                        dst = model.get_buffer(t)
                    except AttributeError:
                        continue
                dst.data.copy_(f.get_tensor(t).to(dst.device))
    return done
