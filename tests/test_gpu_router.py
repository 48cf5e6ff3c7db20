"""GPU tests of the SmoothQuant module-swap router against the reference router's own results.

``tests/golden/router_fixtures.json`` holds, for a tiny random model of each model type the
reference accepts (``fake_quant.py:226-242``), the qualified names the reference
``quantize_model`` returned, which modules it swapped and which it left in floating point, and
the ``repr`` of every swapped module (``make_router_fixtures.py`` wrote them by running the
reference in the build container).  Here the same models (``golden/router_models.py``, the same
configs and seeds) go through this build's router on the GPU, and every fixture must match
exactly: names and their order, module kinds, reprs, and the rejection of model types outside the
allow-list.
"""
import json
import sys
from pathlib import Path

import pytest
import torch

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).parent / "golden"
sys.path.insert(0, str(GOLD))
from router_models import MODEL_TYPES, module_kinds, tiny_model  # noqa: E402

FIX = json.loads((GOLD / "router_fixtures.json").read_text())
DEV = "cuda:0"
CASES = sorted(FIX)


def _say(*a):
    print(*a, flush=True)


def _run(key, layer_type_alias=True, **kw):
    mt, bits, bmm = key.split("/")
    model = tiny_model(mt, torch.float16, layer_type_alias=layer_type_alias).to(DEV)
    from mindpipe_amd.smoothquant import quantize_model
    names = quantize_model(model, weight_bits=8, activation_bits=8, quantize_bmm_input=bmm == "bmm1", **kw)
    return model, names


def test_fixture_covers_every_model_type():
    assert {k.split("/")[0] for k in FIX} == set(MODEL_TYPES)


@pytest.mark.parametrize("key", CASES)
def test_router_matches_reference(key):
    _say("router", key)
    want = FIX[key]
    if "error" in want:
        etype, msg = want["error"]
        with pytest.raises(ValueError) as ei:
            _run(key)
        assert etype == "ValueError" and str(ei.value) == msg
        return
    model, names = _run(key)
    assert names == want["names"]
    kinds = module_kinds(model)
    assert kinds == want["kinds"]
    mods = dict(model.named_modules())
    assert {n: repr(mods[n]) for n, c in kinds.items() if c.startswith("SmoothQuant")} == want["reprs"]
    torch.cuda.synchronize()


@pytest.mark.parametrize("mt", ["qwen3_5", "qwen3_5_moe", "qwen3_5_moe_text"])
def test_router_reads_block_type_of_later_transformers(mt):
    """Without the ``layer_type`` alias (the installed transformers' own layers) the router reads
    ``block_type`` and swaps the same modules as the reference does on the alias."""
    _say("router block_type", mt)
    key = f"{mt}/w8a8/bmm1"
    model, names = _run(key, layer_type_alias=False)
    assert names == FIX[key]["names"]
    assert module_kinds(model) == FIX[key]["kinds"]


def test_router_extension_model_types():
    """Mixtral is refused like the reference unless ``allow_extension_models``; then its packed
    experts and attention are swapped and the router's names follow the reference's order."""
    _say("router mixtral extension")
    model, names = _run("mixtral/w8a8/bmm1", allow_extension_models=True)
    want = []
    for li in range(4):
        lp = f"model.layers.{li}"
        want += [f"{lp}.self_attn.{p}" for p in ("q_proj", "k_proj", "v_proj", "o_proj")]
        want += [f"{lp}.mlp.experts.gate_up_proj", f"{lp}.mlp.experts.down_proj"]
    assert names == want
    assert type(model.model.layers[0].mlp.experts).__name__ == "SmoothQuantPackedMoeExperts"


@pytest.mark.parametrize("mt", ["llama", "qwen3_moe", "qwen3_5_moe_text"])
def test_routed_model_forward_runs(mt):
    """The swapped model runs its forward on the GPU and gives finite logits."""
    _say("routed forward", mt)
    model, _ = _run(f"{mt}/w8a8/bmm1")
    ids = torch.randint(0, 128, (2, 9), generator=torch.Generator().manual_seed(4)).to(DEV)
    with torch.no_grad():
        out = model(input_ids=ids).logits
    assert out.shape == (2, 9, 128) and torch.isfinite(out.float()).all()
