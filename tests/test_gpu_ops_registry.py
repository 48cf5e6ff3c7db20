"""The torch.library registrations: every ``torch.ops.mindpipe_amd.*`` op passes opcheck's schema and
fake-tensor checks (the fake implementation gives the real op's output shapes, dtypes and devices),
the registration contract of the reference's ``torch.ops.vllm.*`` bridge op (vllm.patch:171-228,
291-306).  Numerics of each op are covered by the parity tests."""
import sys

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
CHECKS = ("test_schema", "test_faketensor")


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _g(seed):
    return torch.Generator(device=DEV).manual_seed(seed)


def _cases():
    from mindpipe_amd import ops  # noqa: F401  (registers the ops)
    mp = torch.ops.mindpipe_amd
    g = _g(0)
    t, h, i, n = 24, 256, 128, 192
    x = torch.randn(t, h, device=DEV, generator=g).half()
    r = torch.randn(t, h, device=DEV, generator=g).half()
    nw = (1 + 0.1 * torch.randn(h, device=DEV, generator=g)).half()
    qx = torch.randint(-127, 128, (t, h), dtype=torch.int8, device=DEV, generator=g)
    sx = torch.rand(t, device=DEV, generator=g) * 0.01
    w8 = torch.randint(-127, 128, (n, h), dtype=torch.int8, device=DEV, generator=g)
    s8 = torch.rand(n, device=DEV, generator=g) * 0.01
    w13 = torch.randint(-127, 128, (1, 2 * i, h), dtype=torch.int8, device=DEV, generator=g)
    s13 = torch.rand(1, 2 * i, device=DEV, generator=g) * 1e-3
    w2 = torch.randint(-127, 128, (1, h, i), dtype=torch.int8, device=DEV, generator=g)
    s2 = torch.rand(h, device=DEV, generator=g) * 1e-3
    offs = torch.tensor([0, t], dtype=torch.int64, device=DEV)
    pk = torch.randint(-2**31, 2**31 - 1, (n, h // 8), dtype=torch.int32, device=DEV, generator=g)
    gs = (torch.rand(n, h // 128, device=DEV, generator=g) * 0.01).half()
    gz = torch.randint(0, 16, (n, h // 128), device=DEV, generator=g).half()
    e, topk = 4, 2
    ids = torch.randint(0, e, (t, topk), dtype=torch.int32, device=DEV, generator=g)
    tw = torch.softmax(torch.randn(t, topk, device=DEV, generator=g), -1)
    mw13 = torch.randint(-127, 128, (e, 2 * i, h), dtype=torch.int8, device=DEV, generator=g)
    ms13 = torch.rand(e, 2 * i, device=DEV, generator=g) * 1e-3
    mw2 = torch.randint(-127, 128, (e, h, i), dtype=torch.int8, device=DEV, generator=g)
    ms2 = torch.rand(e, h, device=DEV, generator=g) * 1e-3
    return {
        "add_rms_norm_dynamic_quant": (mp.add_rms_norm_dynamic_quant.default, (x, r, nw, 1e-6)),
        "rms_norm_dynamic_quant": (mp.rms_norm_dynamic_quant.default, (x, nw, 1e-6)),
        "add_rms_norm": (mp.add_rms_norm.default, (x, r, nw, 1e-6)),
        "dense_mlp_w8a8": (mp.dense_mlp_w8a8.default, (qx, sx, offs, [w13[:, :]], [s13], w2, s2, i, torch.float16)),
        "quant_per_token_i8": (mp.quant_per_token_i8.default, (x,)),
        "w8a8_gemm": (mp.w8a8_gemm.default, (qx, sx, w8, s8, None, torch.float16)),
        "w8a8_gemm_fake": (mp.w8a8_gemm_fake.default, (qx, sx.half().float(), w8, s8.half().float(), None,
                                                       torch.float16)),
        "w4a16_gemm": (mp.w4a16_gemm.default, (x, pk, gs, gz, 128, None)),
        "w8a8_gemm_quant_out": (mp.w8a8_gemm_quant_out.default, (qx, sx, w8, s8, None, torch.float16, False)),
        "i8_gemm_swiglu_requant": (mp.i8_gemm_swiglu_requant.default, (qx, sx, w13, s13, offs, i)),
        "moe_w8a8_forward": (mp.moe_w8a8_forward.default, (x, ids, tw, mw13, ms13, mw2, ms2)),
    }


NAMES = ["add_rms_norm_dynamic_quant", "rms_norm_dynamic_quant", "add_rms_norm", "dense_mlp_w8a8",
         "quant_per_token_i8", "w8a8_gemm", "w8a8_gemm_fake", "w8a8_gemm_quant_out", "w4a16_gemm",
         "i8_gemm_swiglu_requant", "moe_w8a8_forward"]


@pytest.mark.parametrize("name", NAMES)
def test_registered_op_passes_opcheck(name):
    _say("opcheck", name)
    op, args = _cases()[name]
    torch.library.opcheck(op, args, test_utils=CHECKS)


def test_every_registered_op_is_checked():
    from mindpipe_amd import ops  # noqa: F401
    regs = sorted(n for n in dir(torch.ops.mindpipe_amd) if not n.startswith("_") and n != "name")
    assert regs == sorted(NAMES), regs
