"""The allocation-free GMM1 entry point (mp_i8_gemm_swiglu_requant_noalloc) against the
workspace entry point, through the C ABI: the same int8 codes and fp32 scales bit for bit, on
two calls in a row (the second smaller, over the scratch the first call left), for the runtime
and the fake rule; shapes past the 64 MiB scratch are refused before any launch."""
import sys

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _case(t, h, inter, e, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    rows = t * 2
    counts = torch.multinomial(torch.ones(e), rows, replacement=True, generator=torch.Generator().manual_seed(seed))
    counts = torch.bincount(counts, minlength=e)
    offs = torch.cat([torch.zeros(1, dtype=torch.int64), torch.cumsum(counts, 0)]).to(DEV)
    routed = torch.randint(-127, 128, (rows, h), generator=g, device=DEV, dtype=torch.int8)
    rscale = torch.rand(rows, generator=g, device=DEV) * 0.01 + 1e-3
    w13 = torch.randint(-127, 128, (e, 2 * inter, h), generator=g, device=DEV, dtype=torch.int8)
    s13 = torch.rand(e, 2 * inter, generator=g, device=DEV) * 1e-3 + 1e-4
    return routed, rscale, w13, s13, offs


def _run(lib, args, rule, act, noalloc):
    from mindpipe_amd import _lib
    routed, rscale, w13, s13, offs = args
    rows, h = routed.shape
    e, two_i, _ = w13.shape
    inter = two_i // 2
    q = torch.empty((rows, inter), dtype=torch.int8, device=DEV)
    s = torch.empty((rows,), dtype=torch.float32, device=DEV)
    stream = torch.cuda.current_stream().cuda_stream
    if noalloc:
        rc = lib.mp_i8_gemm_swiglu_requant_noalloc(routed.data_ptr(), rscale.data_ptr(), w13.data_ptr(),
                                                   s13.data_ptr(), offs.data_ptr(), e, rows, h, inter, rule, act,
                                                   q.data_ptr(), s.data_ptr(), stream)
    else:
        wsb = lib.mp_moe_gmm1_workspace_bytes(rows, inter)
        ws = torch.empty((wsb,), dtype=torch.uint8, device=DEV)
        rc = lib.mp_i8_gemm_swiglu_requant(routed.data_ptr(), rscale.data_ptr(), w13.data_ptr(), s13.data_ptr(),
                                           offs.data_ptr(), e, rows, h, inter, rule, act, q.data_ptr(),
                                           s.data_ptr(), ws.data_ptr(), wsb, stream)
    _lib.check(rc, "gmm1")
    torch.cuda.synchronize()
    return q, s


@pytest.mark.parametrize("rule,act", [(0, 0), (1, 0), (1, 1)])
def test_noalloc_gmm1_matches_workspace_entry(rule, act):
    from mindpipe_amd import _lib
    lib = _lib.load()
    for t, h, inter, e, seed in ((300, 512, 768, 8, 1), (40, 256, 384, 4, 2)):
        _say("noalloc gmm1", rule, act, t, h, inter, e)
        args = _case(t, h, inter, e, seed)
        q_ref, s_ref = _run(lib, args, rule, act, False)
        q_na, s_na = _run(lib, args, rule, act, True)
        assert torch.equal(q_na, q_ref)        # bar: bit-exact (same kernels, same arithmetic)
        assert torch.equal(s_na.view(torch.int32), s_ref.view(torch.int32))


def test_noalloc_gmm1_refuses_oversized_shape():
    from mindpipe_amd import _lib
    lib = _lib.load()
    # 4096 rows x 8192 intermediate columns of fp32 rows: 128 MiB > 64 MiB; refused on the host before
    # any launch.  Every operand is a real buffer of its full size, so only the scratch is too small.
    t, h, inter, e = 4096, 128, 8192, 8
    dev = "cuda:0"
    routed = torch.zeros((t, h), dtype=torch.int8, device=dev)
    rscale = torch.ones((t,), dtype=torch.float32, device=dev)
    w13 = torch.zeros((e, 2 * inter, h), dtype=torch.int8, device=dev)
    s13 = torch.ones((e, 2 * inter), dtype=torch.float32, device=dev)
    offsets = torch.arange(0, t + 1, t // e, dtype=torch.int64, device=dev)
    q = torch.empty((t, inter), dtype=torch.int8, device=dev)
    s = torch.empty((t,), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    rc = lib.mp_i8_gemm_swiglu_requant_noalloc(routed.data_ptr(), rscale.data_ptr(), w13.data_ptr(), s13.data_ptr(),
                                               offsets.data_ptr(), e, t, h, inter, 0, 0, q.data_ptr(), s.data_ptr(),
                                               torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == 6   # MP_ERR_WORKSPACE
    assert lib.mp_moe_gmm1_workspace_bytes(4096, 8192) > (64 << 20)
