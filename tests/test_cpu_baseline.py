"""The torch CPU restatements timed as bench.py's cpu_baseline, checked against the outputs
the reference's own functions wrote (tests/golden): the baseline times the reference's path,
not a different computation."""
from pathlib import Path

import numpy as np
import torch

from oracle import cpu_baseline as CB

GOLD = np.load(Path(__file__).parent / "golden" / "reference_vectors.npz")
EXT = np.load(Path(__file__).parent / "golden" / "reference_ext_vectors.npz")


def test_awq_restatement_matches_reference_vectors():
    w = torch.from_numpy(GOLD["awq_w"])
    assert np.array_equal(CB.awq_pseudo_quantize(w, 128).numpy().view(np.uint16), GOLD["awq_deq"].view(np.uint16))


def test_fake_quant_rows_matches_reference_vectors():
    fx = CB.fake_quant_rows(torch.from_numpy(GOLD["sq_x"])).numpy()
    assert np.array_equal(fx.view(np.uint16), GOLD["sq_x_fq"].view(np.uint16))
    fw = CB.fake_quant_rows(torch.from_numpy(GOLD["sq_w"])).numpy()
    assert np.array_equal(fw.view(np.uint16), GOLD["sq_w_fq"].view(np.uint16))


def test_moe_loop_matches_reference_module():
    gu = CB.fake_quant_rows(torch.from_numpy(EXT["moe_f16_gu"]))
    dn = CB.fake_quant_rows(torch.from_numpy(EXT["moe_f16_dn"]))
    y = CB.moe_fake_forward(torch.from_numpy(EXT["moe_f16_x"]), torch.from_numpy(EXT["moe_f16_ids"]).long(),
                            torch.from_numpy(EXT["moe_f16_w"]), gu, dn)
    assert np.array_equal(y.numpy().view(np.uint16), EXT["moe_f16_y"].view(np.uint16))


def test_host_info_and_median():
    info = CB.host_info()
    assert info["threads"] >= 1 and info["nproc"] >= 1 and isinstance(info["cpu_model"], str)
    calls = []
    assert CB.median_ms(lambda: calls.append(1), runs=4, warmup=2) >= 0 and len(calls) == 6
