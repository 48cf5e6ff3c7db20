"""Write the router fixture by running the reference's SmoothQuant router on tiny models.

Run in the build container only (the reference tree is not present on GPU boxes):
``python tests/golden/make_router_fixtures.py /root/reference``.

For each model type in ``router_models.MODEL_TYPES`` it builds the tiny random model of
``router_models.tiny_model``, calls the reference ``quantize_model`` on it
(``algorithm/quantization/ptq/smoothquant/source/smoothquant/fake_quant.py:441-457``, which
routes through ``quantize_llama_like`` ``:226-438``) and stores, in
``tests/golden/router_fixtures.json``:

* ``names``: the qualified names the router returns, in its order;
* ``kinds``: ``{module name: class name}`` for every linear / quantized linear / expert block
  after the swap (which linears were swapped and which were left in floating point);
* ``reprs``: ``repr()`` of every swapped module (bit widths and ``output_quant``);
* ``error``: the exception type and message when the router rejects the model type.

Only data is written; no reference source is copied.
"""
import json
import sys
from pathlib import Path

import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE))
from router_models import MODEL_TYPES, module_kinds, tiny_model  # noqa: E402


def main(ref_root):
    sys.path.insert(0, str(Path(ref_root)))
    from algorithm.quantization.ptq.smoothquant.source.smoothquant.fake_quant import quantize_model
    out = {}
    for mt in MODEL_TYPES:
        for wb, ab, qbmm in ((8, 8, True), (8, 8, False)):
            model = tiny_model(mt, torch.float16)
            key = f"{mt}/w{wb}a{ab}/bmm{int(qbmm)}"
            try:
                names = quantize_model(model, weight_bits=wb, activation_bits=ab, quantize_bmm_input=qbmm)
            except Exception as e:  # the reference's rejection is part of the contract
                out[key] = {"error": [type(e).__name__, str(e)]}
                continue
            kinds = module_kinds(model)
            mods = dict(model.named_modules())
            reprs = {n: repr(mods[n]) for n, c in kinds.items() if c.startswith("SmoothQuant")}
            out[key] = {"names": names, "kinds": kinds, "reprs": reprs}
            print(key, len(names), "names")
    (HERE / "router_fixtures.json").write_text(json.dumps(out, indent=1, sort_keys=True) + "\n")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
