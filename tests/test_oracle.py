"""Pins the numpy oracle against the reference's known answers and golden vectors.

Sources of truth used here (never the oracle's own formula retyped):
* known answers held in the reference's tests (pack KAT, export KAT, tiny
  Qwen2 W8A8 export values), restated as literal data;
* ``tests/golden/reference_vectors.npz`` and ``reference_ext_vectors.npz``,
  written by running the reference's own quantizers, ``SmoothQuantLinear``,
  ``SmoothQuantPackedMoeExperts`` and ``_compute_smooth_scales``
  (``tests/golden/make_reference_vectors.py``);
* brute-force loops and closed-form invariants.
"""
import json
from pathlib import Path

import numpy as np
import pytest

from oracle import quant as O

GOLD = np.load(Path(__file__).parent / "golden" / "reference_vectors.npz")
EXT = np.load(Path(__file__).parent / "golden" / "reference_ext_vectors.npz")
KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())


def test_pack_kat_round_trip():
    # tests/test_vllm_real_quant_export.py:30-40
    k = KATS["pack_round_trip"]
    packed = O.pack_int4_signed(np.array(k["values"], np.int8))
    assert packed.dtype == np.int32 and packed.shape == (1, 2)
    assert packed.tolist() == k["packed"]
    assert O.unpack_int4_signed(packed, 10).tolist() == k["values"]


def test_export_kat_words():
    # tests/test_vllm_real_quant_export.py:105-152
    k = KATS["export_int_weight"]
    packed = O.pack_int4_signed(np.array(k["int_weight"], np.int8))
    assert packed.tolist() == k["packed"]
    assert O.unpack_int4_signed(packed, 8).tolist() == k["int_weight"]


def test_pack_matches_reference_vectors_and_bruteforce():
    iw = GOLD["pack_in"]
    packed = O.pack_int4_signed(iw)
    assert np.array_equal(packed, GOLD["pack_out"])
    # brute force bit loop
    for r in range(iw.shape[0]):
        for c in range(iw.shape[1]):
            word = int(packed[r, c // 8]) & 0xFFFFFFFF
            assert ((word >> (4 * (c % 8))) & 0xF) == int(iw[r, c]) + 8
        for c in range(iw.shape[1], packed.shape[1] * 8):
            assert ((int(packed[r, c // 8]) & 0xFFFFFFFF) >> (4 * (c % 8))) & 0xF == 0


def test_pack_rejects_out_of_range():
    with pytest.raises(ValueError):
        O.pack_int4_signed(np.array([[8]], np.int8))
    with pytest.raises(ValueError):
        O.pack_int4_signed(np.array([1, 2], np.int8))


def test_w8_export_tiny_qwen2_kat():
    # tests/repro/test_export_fp16_to_ascend_w8a8_dynamic_probe.py:27-99 fixture
    for case in KATS["w8_export"]:
        w = np.array(case["w"], np.float16)
        q, s32, s16, off = O.quantize_weight_per_channel_export(w)
        assert q.dtype == np.int8 and q.tolist() == case["q"]
        assert s16.dtype == np.float16 and s16.tolist() == case["scale_fp16"]
        assert off.shape == (2,) and not off.any()


def test_w8_export_rejects_non_finite():
    with pytest.raises(ValueError):
        O.quantize_weight_per_channel_export(np.array([[1.0, np.inf]], np.float16))


def test_w8_export_matches_reference_vectors():
    q, s32, s16, _ = O.quantize_weight_per_channel_export(GOLD["sq_w"])
    assert np.array_equal(q, GOLD["ex_q"])
    assert np.array_equal(s16.view(np.uint16), GOLD["ex_s"][:, 0].view(np.uint16))
    qb, _, sb, _ = O.quantize_weight_per_channel_export(GOLD["ex_wb_bits"].view(np.uint16), in_dtype="bf16")
    assert np.array_equal(qb, GOLD["ex_qb"])
    assert np.array_equal(sb, GOLD["ex_sb_bits"][:, 0].view(np.uint16))


def test_awq_matches_reference_vectors_bitwise():
    deq, s, z, codes = O.pseudo_quantize_tensor(GOLD["awq_w"], 4, True, 128)
    assert np.array_equal(deq.view(np.uint16), GOLD["awq_deq"].view(np.uint16))
    assert np.array_equal(s.view(np.uint16), GOLD["awq_s"].view(np.uint16))
    assert np.array_equal(z.view(np.uint16), GOLD["awq_z"].view(np.uint16))
    deq, s, z, _ = O.pseudo_quantize_tensor(GOLD["awq_w_row"], 4, True, 128)
    assert s.shape == (8, 1)
    assert np.array_equal(deq.view(np.uint16), GOLD["awq_deq_row"].view(np.uint16))
    assert np.array_equal(s.view(np.uint16), GOLD["awq_s_row"].view(np.uint16))
    assert np.array_equal(z.view(np.uint16), GOLD["awq_z_row"].view(np.uint16))
    deq, _, _, _ = O.pseudo_quantize_tensor(GOLD["awq_w"], 4, False, 128)
    assert np.array_equal(deq.view(np.uint16), GOLD["awq_sym_deq"].view(np.uint16))


def test_awq_invariants_and_packed_dequant():
    rng = np.random.default_rng(0)
    w = (rng.standard_normal((16, 384)) * 0.02).astype(np.float16)
    deq, s, z, codes = O.pseudo_quantize_tensor(w, 4, True, 128)
    assert codes.min() >= 0 and codes.max() <= 15
    assert np.all((z >= 0) & (z <= 15)) and np.all(z == np.rint(z))
    # the group's min maps to code 0 or 1 (one rounding step) and max to 14 or 15
    g = codes.reshape(-1, 128)
    assert np.all(g.min(axis=1) <= 1) and np.all(g.max(axis=1) >= 14)
    # reconstruction inside the representable range: |w - deq| <= s/2 (+ fp16 rounding)
    srep = np.repeat(s.astype(np.float32), 128, axis=1)
    err = np.abs(w.astype(np.float32) - deq.astype(np.float32))
    assert np.all(err <= srep * 0.5 + np.abs(deq.astype(np.float32)) * 2**-10 + 1e-7)
    # packed path reproduces the same fp16 weights bit for bit
    packed = O.pack_uint4(codes)
    deq2 = O.dequant_w4_fp16(packed, s, z, 384, 128)
    assert np.array_equal(deq2.view(np.uint16), deq.view(np.uint16))


def test_gptq_rtn_matches_reference_vectors():
    iw, scale, fake = O.gptq_rtn_quantize(GOLD["gptq_w"], 4, 128)
    assert np.array_equal(iw, GOLD["gptq_int"])
    assert np.array_equal(scale.view(np.uint16), GOLD["gptq_scale"].view(np.uint16))
    # reconstruction invariant of tests/test_vllm_real_quant_export.py:43-78
    assert iw.min() >= -8 and iw.max() <= 7
    rec = iw.astype(np.float32) * np.repeat(scale.astype(np.float32), 128, axis=1)
    np.testing.assert_allclose(rec, fake, atol=1e-3 * np.abs(fake).max())


def test_gptq_export_dequant_round_trip():
    iw, scale, _ = O.gptq_rtn_quantize(GOLD["gptq_w"], 4, 128)
    packed = O.pack_int4_signed(iw)
    deq = O.dequant_w4_export_fp32(packed, scale, (12, 256))
    assert np.array_equal(deq, iw.astype(np.float32) * np.repeat(scale.astype(np.float32), 128, 1))
    # fp16 path with z = 8 equals the fp32 path rounded to fp16
    d16 = O.dequant_w4_fp16(packed, scale, None, 256, 128)
    assert np.array_equal(d16, deq.astype(np.float16))


def test_fake_quant_matches_reference_vectors_bitwise():
    _, _, fx = O.quantize_activation_per_token_fake(GOLD["sq_x"])
    assert np.array_equal(fx.view(np.uint16), GOLD["sq_x_fq"].view(np.uint16))
    _, _, fw = O.quantize_weight_per_channel_fake(GOLD["sq_w"])
    assert np.array_equal(fw.view(np.uint16), GOLD["sq_w_fq"].view(np.uint16))


def test_runtime_per_token_bruteforce_and_invariants():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((6, 40)).astype(np.float16)
    x[2] = 0
    x[3, :] = np.arange(40, dtype=np.float16) - 20
    q, s = O.quantize_per_token_runtime(x)
    for r in range(x.shape[0]):
        amax = max(abs(float(v)) for v in x[r])
        sr = np.float32(np.float32(amax) / np.float32(127))
        assert s[r] == sr
        for c in range(x.shape[1]):
            if sr == 0:
                assert q[r, c] == 0
                continue
            v = float(np.float32(np.float32(x[r, c]) / sr))
            lo = np.floor(v)
            frac = v - lo
            exp = lo + 1 if frac > 0.5 or (frac == 0.5 and lo % 2 == 1) else lo
            assert q[r, c] == int(max(-127, min(127, exp)))
    nz = s > 0
    assert np.all(np.abs(q[nz]).max(axis=1) == 127)


def test_w8a8_runtime_linear_bruteforce():
    rng = np.random.default_rng(2)
    qx = rng.integers(-127, 128, (3, 7)).astype(np.int8)
    qw = rng.integers(-127, 128, (5, 7)).astype(np.int8)
    sx = rng.random(3).astype(np.float32)
    sw = rng.random(5).astype(np.float32)
    b = rng.standard_normal(5).astype(np.float16)
    y = O.w8a8_linear_runtime(qx, sx, qw, sw, b)
    for m in range(3):
        for n in range(5):
            acc = sum(int(qx[m, k]) * int(qw[n, k]) for k in range(7))
            v = np.float32(np.float32(np.float32(acc) * sx[m]) * sw[n]) + np.float32(b[n])
            assert y[m, n] == np.float16(np.float32(v))
    yb = O.w8a8_linear_runtime(qx, sx, qw, sw, None, out_dtype="bf16")
    ref = O.w8a8_linear_runtime(qx, sx, qw, sw, None, out_dtype="fp32")
    assert np.all(np.abs(O.bf16_bits_to_f32(yb) - ref) <= np.abs(ref) * 2**-8 + 1e-30)


def test_bf16_rounding_closed_form():
    x = np.array([1.0, 1.00390625, 1.005859375, 1.0 + 2**-8 + 2**-9, -3.0, 0.0], np.float32)
    bits = O.f32_to_bf16_bits(x)
    assert O.bf16_bits_to_f32(bits).tolist() == [1.0, 1.0, 1.0078125, 1.0078125, -3.0, 0.0]


def test_smooth_scales_closed_form():
    a = np.array([4.0, 9.0, 0.0], np.float32)
    w = np.array([[1.0, -0.25, 0.0], [0.5, 0.0625, 0.0]], np.float16)
    s = O.compute_smooth_scales(a, w, 0.5)
    assert s.dtype == np.float16
    assert s.tolist()[:2] == [2.0, 6.0]              # sqrt(4)/sqrt(1), sqrt(9)/sqrt(0.25)
    assert s[2] == np.float16(1e-5)                   # clamp


def test_router_invariants():
    rng = np.random.default_rng(3)
    logits = rng.standard_normal((64, 8)).astype(np.float32)
    idx, w = O.mixtral_router(logits, 2)
    assert np.allclose(w.sum(1), 1, atol=1e-6)
    assert np.all(idx[:, 0] == logits.argmax(1))
    assert np.all(idx[:, 0] != idx[:, 1])
    assert np.all(w[:, 0] >= w[:, 1])


def _moe_bruteforce(x, ids, w, qw13, s13, qw2, s2):
    t_count, hdim = x.shape
    inter = qw2.shape[2]
    out = np.zeros((t_count, hdim), np.float32)
    qx, sx = O.quantize_per_token_runtime(x)
    ys = np.zeros((t_count, ids.shape[1], hdim), np.float32)
    for t in range(t_count):
        for j in range(ids.shape[1]):
            e = ids[t, j]
            acc = qw13[e].astype(np.int64) @ qx[t].astype(np.int64)
            g = (acc.astype(np.float32) * sx[t]).astype(np.float32) * s13[e]
            gate, up = g[:inter], g[inter:]
            h = (gate / (np.float32(1) + np.exp(-gate))).astype(np.float32) * up
            qh, sh = O.quantize_per_token_runtime(h[None].astype(np.float32), in_dtype="fp32")
            acc2 = qw2[e].astype(np.int64) @ qh[0].astype(np.int64)
            ys[t, j] = (acc2.astype(np.float32) * sh[0]).astype(np.float32) * s2[e]
    for j in range(ids.shape[1]):
        out = (out + w[:, j][:, None] * ys[:, j]).astype(np.float32)
    return out.astype(np.float16)


def test_moe_runtime_matches_bruteforce_and_fake_path():
    rng = np.random.default_rng(4)
    t_count, hdim, inter, n_exp = 12, 32, 24, 4
    x = rng.standard_normal((t_count, hdim)).astype(np.float16)
    ids, w = O.mixtral_router(rng.standard_normal((t_count, n_exp)).astype(np.float32), 2)
    ids[0] = [3, 1]                     # make sure expert 0 can go unhit
    ids[ids == 0] = 2
    ids[1] = [2, 3]
    wgu = (rng.standard_normal((n_exp, 2 * inter, hdim)) * 0.2).astype(np.float16)
    wdn = (rng.standard_normal((n_exp, hdim, inter)) * 0.2).astype(np.float16)
    q13 = np.stack([O.quantize_weight_per_channel_export(wgu[e])[0] for e in range(n_exp)])
    s13 = np.stack([O.quantize_weight_per_channel_export(wgu[e])[1] for e in range(n_exp)])
    q2 = np.stack([O.quantize_weight_per_channel_export(wdn[e])[0] for e in range(n_exp)])
    s2 = np.stack([O.quantize_weight_per_channel_export(wdn[e])[1] for e in range(n_exp)])
    y = O.moe_runtime(x, ids, w, q13, s13, q2, s2)
    yb = _moe_bruteforce(x, ids, w, q13, s13, q2, s2)
    assert np.array_equal(y.view(np.uint16), yb.view(np.uint16))


def _u16(a):
    return np.ascontiguousarray(a).view(np.uint16)


def _cv(dt):
    return (lambda a: a) if dt == "fp16" else (lambda a: np.ascontiguousarray(a).view(np.uint16))


@pytest.mark.parametrize("tag,dt", [("f16", "fp16"), ("bf16", "bf16")])
def test_moe_fake_matches_reference_module_forward(tag, dt):
    """``SmoothQuantPackedMoeExperts(gate_up, down, SiLU)(x, ids, w)`` as the reference computes it
    (fake_quant.py:124-191; vectors written by the reference module): bit-exact, fp16 and bf16,
    including an all-zero token and an expert hit by one token."""
    cv = _cv(dt)
    y = O.moe_fake(cv(EXT[f"moe_{tag}_x"]), EXT[f"moe_{tag}_ids"], EXT[f"moe_{tag}_w"], cv(EXT[f"moe_{tag}_gu"]),
                   cv(EXT[f"moe_{tag}_dn"]), dt)
    assert np.array_equal(_u16(y), _u16(EXT[f"moe_{tag}_y"]))


def test_moe_fake_differs_from_runtime_rule_by_rounding_only():
    """The fake rule (fp16 scales and fp16 roundings) and the runtime rule (fp32 scales, fp32
    SwiGLU) describe the same layer: within a few 1e-3 of each other on the reference's case,
    and a planted mistake (gate/up swapped) is far from both."""
    x, ids, w = EXT["moe_f16_x"], EXT["moe_f16_ids"], EXT["moe_f16_w"]
    gu, dn = EXT["moe_f16_gu"], EXT["moe_f16_dn"]
    e = gu.shape[0]
    q13 = np.stack([O.quantize_weight_per_channel_export(gu[i])[0] for i in range(e)])
    s13 = np.stack([O.quantize_weight_per_channel_export(gu[i])[1] for i in range(e)])
    q2 = np.stack([O.quantize_weight_per_channel_export(dn[i])[0] for i in range(e)])
    s2 = np.stack([O.quantize_weight_per_channel_export(dn[i])[1] for i in range(e)])
    yr = O.moe_runtime(x, ids, w, q13, s13, q2, s2).astype(np.float64)
    yf = EXT["moe_f16_y"].astype(np.float64)
    assert np.linalg.norm(yr - yf) / np.linalg.norm(yf) < 2e-2
    inter = dn.shape[2]
    swapped = np.concatenate([gu[:, inter:], gu[:, :inter]], axis=1)
    ys = O.moe_fake(x, ids, w, swapped, dn).astype(np.float64)
    assert np.linalg.norm(ys - yf) / np.linalg.norm(yf) > 0.3


def test_bf16_awq_and_fake_quant_match_reference():
    """bf16 arithmetic of pseudo_quantize_tensor (asym with a constant group, and sym) and of
    the per-token / per-channel fake quantizers: bit-exact to the reference's outputs."""
    w = _u16(EXT["awqb_w"])
    d, s, z, c = O.pseudo_quantize_tensor(w, 4, True, 128, dtype="bf16")
    assert np.array_equal(d, _u16(EXT["awqb_deq"]))
    assert np.array_equal(s, _u16(EXT["awqb_s"])) and np.array_equal(z, _u16(EXT["awqb_z"]))
    assert c.min() >= 0 and c.max() <= 15
    d2, s2, _, c2 = O.pseudo_quantize_tensor(w, 4, False, 128, dtype="bf16")
    assert np.array_equal(d2, _u16(EXT["awqb_sym_deq"]))
    # the packed codes dequantize to the reference's bf16 weights bit for bit (both zero-point forms)
    k = w.shape[1]
    assert np.array_equal(O.dequant_w4_bf16(O.pack_uint4(c), s, z, k, 128), _u16(EXT["awqb_deq"]))
    assert np.array_equal(O.dequant_w4_bf16(O.pack_int4_signed(c2), s2, None, k, 128), _u16(EXT["awqb_sym_deq"]))
    _, _, fx = O.quantize_activation_per_token_fake(_u16(EXT["sqb_x"]), 8, "bf16")
    assert np.array_equal(fx, _u16(EXT["sqb_x_fq"]))
    _, _, fw = O.quantize_weight_per_channel_fake(_u16(EXT["sqb_w"]), 8, "bf16")
    assert np.array_equal(fw, _u16(EXT["sqb_w_fq"]))


def test_bf16_packed_dequant_matches_pseudo_quantize_on_random_groups():
    """dequant_w4_bf16 of the packed codes equals pseudo_quantize_tensor's bf16 weight bit for bit on
    random rows (every group its own scale / zero, wide scale range), and a planted mistake (the
    product not rounded to bf16) does not."""
    rng = np.random.default_rng(5)
    w32 = (rng.standard_normal((24, 512)) * np.exp(rng.uniform(-6, 2, (24, 1)))).astype(np.float32)
    w = O.f32_to_bf16_bits(w32)
    for zp in (True, False):
        d, s, z, c = O.pseudo_quantize_tensor(w, 4, zp, 128, dtype="bf16")
        packed = O.pack_uint4(c) if zp else O.pack_int4_signed(c)
        assert np.array_equal(O.dequant_w4_bf16(packed, s, z, 512, 128), d)
    u = O.unpack_uint4(packed, 512).astype(np.float32)
    unrounded = (u - 8.0) * np.repeat(O.bf16_bits_to_f32(s), 128, axis=1)
    assert not np.array_equal(unrounded, O.bf16_bits_to_f32(d))


@pytest.mark.parametrize("tag,dt", [("f16", "fp16"), ("bf16", "bf16")])
def test_smoothquant_linear_fake_forward_matches_reference(tag, dt):
    """SmoothQuantLinear.from_float + forward (fake_quant.py:85-113), with and without the
    output fake-quant: bit-exact in fp16 and bf16."""
    cv = _cv(dt)
    y = O.w8a8_linear_fake(cv(EXT[f"sql_{tag}_x"]), cv(EXT[f"sql_{tag}_w"]), cv(EXT[f"sql_{tag}_b"]), dt)
    assert np.array_equal(_u16(y), _u16(EXT[f"sql_{tag}_y"]))
    yq = O.quantize_activation_per_token_fake(y, 8, dt)[2]
    assert np.array_equal(_u16(yq), _u16(EXT[f"sql_{tag}_yq"]))


@pytest.mark.parametrize("tag,dt", [("f16", "fp16"), ("bf16", "bf16")])
def test_smooth_scales_match_reference(tag, dt):
    """_compute_smooth_scales (smooth.py:7-25) over two fcs sharing a norm, with a clamped
    weight column and activation outliers: bit-exact."""
    cv = _cv(dt)
    s = O.compute_smooth_scales(EXT[f"smooth_{tag}_a"], [cv(EXT[f"smooth_{tag}_w0"]), cv(EXT[f"smooth_{tag}_w1"])],
                                0.5, dt)
    assert np.array_equal(_u16(s), _u16(EXT[f"smooth_{tag}_s"]))


def test_add_rms_norm_closed_forms_and_invariants():
    h = 64
    w1 = np.ones(h, np.float16)
    # constant rows: rstd = 1/|c| (eps negligible) -> y = sign(c); the codes are +-127
    x = np.stack([np.full(h, 3.0), np.full(h, -0.25), np.full(h, 1024.0)]).astype(np.float16)
    y, q, s, r = O.add_rms_norm_quant(x, None, w1, 1e-12)
    assert r is None
    assert y.tolist() == np.sign(x.astype(np.float32)).astype(np.float16).tolist()
    assert (np.abs(q) == 127).all() and np.allclose(s, 1.0 / 127.0)
    # +-a rows: rms = a, so y = +-1 * weight (weight a power of two keeps it exact)
    xa = np.tile(np.array([2.0, -2.0], np.float16), (2, h // 2))
    wp = np.full(h, 0.5, np.float16)
    y2, _, _, _ = O.add_rms_norm_quant(xa, None, wp, 0.0, quant=False)
    assert y2.tolist() == (np.sign(xa.astype(np.float32)) * 0.5).astype(np.float16).tolist()
    # a mean over h (not h - 1): one non-zero entry v in h gives y = sqrt(h) at that place
    xo = np.zeros((1, h), np.float16)
    xo[0, 5] = 0.75
    y3, _, _, _ = O.add_rms_norm_quant(xo, None, w1, 0.0, quant=False)
    assert float(y3[0, 5]) == 8.0 and float(np.abs(y3).sum()) == 8.0
    # scale invariance: x and 4x normalise to the same y (eps 0)
    g = np.random.default_rng(3)
    xr = (g.standard_normal((5, h)) * 0.7).astype(np.float16)
    wr = (g.standard_normal(h) * 0.5 + 1).astype(np.float16)
    ya, _, _, _ = O.add_rms_norm_quant(xr, None, wr, 0.0, quant=False)
    yb, _, _, _ = O.add_rms_norm_quant((xr.astype(np.float32) * 4).astype(np.float16), None, wr, 0.0, quant=False)
    assert ya.tolist() == yb.tolist()
    # residual identity: exact sums (multiples of 1/64 in a small range)
    xi = (g.integers(-64, 64, (3, h)) / 64).astype(np.float16)
    ri = (g.integers(-64, 64, (3, h)) / 64).astype(np.float16)
    yc, qc, sc, rc = O.add_rms_norm_quant(xi, ri, wr, 1e-6)
    yd, qd, sd, _ = O.add_rms_norm_quant((xi.astype(np.float32) + ri).astype(np.float16), None, wr, 1e-6)
    assert rc.tolist() == (xi.astype(np.float32) + ri).astype(np.float16).tolist()
    assert yc.tolist() == yd.tolist() and qc.tolist() == qd.tolist() and sc.tolist() == sd.tolist()
    # q / s are the per-token runtime quant of y
    q2, s2 = O.quantize_per_token_runtime(yc)
    assert q2.tolist() == qc.tolist() and s2.tolist() == sc.tolist()


def test_dense_mlp_single_chunk_equals_one_expert_moe():
    g = np.random.default_rng(11)
    t, h, inter = 6, 64, 32
    x = (g.standard_normal((t, h))).astype(np.float16)
    qw13 = g.integers(-127, 128, (2 * inter, h)).astype(np.int8)
    qw2 = g.integers(-127, 128, (h, inter)).astype(np.int8)
    s13 = (g.random(2 * inter) * 0.01 + 1e-3).astype(np.float32)
    s2 = (g.random(h) * 0.01 + 1e-3).astype(np.float32)
    y1 = O.dense_mlp_runtime(x, qw13, s13, qw2, s2, chunks=1)
    ym = O.moe_runtime(x, np.zeros((t, 1), np.int32), np.ones((t, 1), np.float32), qw13[None], s13[None], qw2[None],
                       s2[None])
    assert y1.tobytes() == ym.tobytes()
    # chunks split the intermediate dimension: every chunk alone is a one-chunk MLP on its slice
    cs = inter // 2
    parts = []
    for c in range(2):
        rows = np.r_[c * cs:(c + 1) * cs, inter + c * cs:inter + (c + 1) * cs]
        parts.append(O.dense_mlp_runtime(x, qw13[rows], s13[rows], np.ascontiguousarray(qw2[:, c * cs:(c + 1) * cs]),
                                         O.bf16_bits_to_f32(O.f32_to_bf16_bits(s2)), chunks=1, out_dtype="fp32"))
    y2 = O.dense_mlp_runtime(x, qw13, s13, qw2, s2, chunks=2, out_dtype="fp32")
    assert y2.tobytes() == (np.float32(0) + parts[0] + parts[1]).astype(np.float32).tobytes()


WID = np.load(Path(__file__).parent / "golden" / "reference_width_vectors.npz")


@pytest.mark.parametrize("tag,dt", [("f16", "fp16"), ("bf16", "bf16")])
def test_quantizers_match_reference_at_other_widths(tag, dt):
    """AWQ at 2, 3 and 8 bits (zero point and symmetric, group 128 and per row) and the
    per-token / per-channel fake quantizers at 3, 4 and 6 bits, against the reference's own
    outputs (``make_width_vectors.py``): bit-exact in fp16 and bf16."""
    cv = _cv(dt)
    w = cv(WID[f"awq_{tag}_w"])
    checked = 0
    for n_bit in (2, 3, 8):
        for zp in (True, False):
            for g in (128, -1):
                key = f"awq_{tag}_n{n_bit}_zp{int(zp)}_g{g}"
                if key + "_deq" not in WID.files:
                    continue
                d, s, z, _ = O.pseudo_quantize_tensor(w, n_bit, zp, g, dt)
                assert np.array_equal(_u16(d), _u16(WID[key + "_deq"])), key
                if zp:
                    assert np.array_equal(_u16(s), _u16(WID[key + "_s"])), key
                    assert np.array_equal(_u16(z), _u16(WID[key + "_z"])), key
                checked += 1
    assert checked == 8
    for n in (3, 4, 6):
        _, _, fx = O.quantize_activation_per_token_fake(cv(WID[f"fq_{tag}_x"]), n, dt)
        assert np.array_equal(_u16(fx), _u16(WID[f"fq_{tag}_x_n{n}"])), n
        _, _, fw = O.quantize_weight_per_channel_fake(cv(WID[f"fq_{tag}_w"]), n, dt)
        assert np.array_equal(_u16(fw), _u16(WID[f"fq_{tag}_w_n{n}"])), n
