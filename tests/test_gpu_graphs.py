"""HIP-graph capture and dynamo tracing of the forward path.

Each forward op is captured once in a ``torch.cuda.CUDAGraph`` and replayed several times.  Between
replays new inputs are copied into the captured input tensors (eager work on the program's stream), the
eager op runs on those inputs, and the device is synchronised; every replay must give the eager op's
bits.  The entry points allocate nothing, record no memset and never synchronise with the host in their
forward path, so they capture as they are (a serving loop replays them this way).  The registered ops
also trace through ``torch.compile`` (fullgraph, ``aot_eager`` backend: dynamo and AOT autograd run the
fake implementations, the kernels run the compiled graph) with the eager result."""
import sys

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
REPLAYS = 3


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _flat(out):
    return list(out) if isinstance(out, (tuple, list)) else [out]


def _case(name, seed=0):
    """(fn, inputs refreshed between replays, refresh function)"""
    from mindpipe_amd import ops
    g = torch.Generator(device=DEV).manual_seed(seed)

    def randn(*s, dt=torch.float16):
        return torch.randn(*s, device=DEV, generator=g).to(dt)

    def i8(*s):
        return torch.randint(-127, 128, s, dtype=torch.int8, device=DEV, generator=g)

    if name.startswith("w4a16"):
        m, dt = {"w4a16_m1": (1, torch.float16), "w4a16_m16": (16, torch.float16),
                 "w4a16_m300": (300, torch.float16), "w4a16_bf16_m1": (1, torch.bfloat16)}[name]
        n, k = 512, 1024
        w = randn(n, k, dt=dt) * 0.05
        pk, sc, zr, _ = ops.w4_quantize_awq(w, 128, True, return_deq=False)
        x = randn(m, k, dt=dt)
        return (lambda: ops.w4a16_gemm(x, pk, sc, zr, 128, None)), [x]
    if name.startswith("w8a8"):
        m = {"w8a8_m1": 1, "w8a8_m16": 16, "w8a8_m256": 256, "w8a8_m600": 600}[name]
        n, k = 768, 1024
        qx, sx = i8(m, k), torch.rand(m, device=DEV, generator=g) * 0.01
        w, sw = i8(n, k), torch.rand(n, device=DEV, generator=g) * 0.01
        return (lambda: ops.w8a8_gemm(qx, sx, w, sw, None, torch.float16)), [qx, sx]
    if name == "quant_per_token":
        x = randn(200, 1024)
        return (lambda: ops.quant_per_token_i8(x)), [x]
    if name == "add_rms_norm_quant":
        x, r = randn(64, 1024), randn(64, 1024)
        nw = (1 + 0.1 * randn(1024, dt=torch.float32)).half()
        return (lambda: ops.add_rms_norm_dynamic_quant(x, r, nw, 1e-6)), [x, r]
    if name == "moe_chain":
        t, h, inter, e, topk = 96, 512, 256, 8, 2
        x = randn(t, h)
        ids = torch.stack([torch.randperm(e, device=DEV, generator=g)[:topk] for _ in range(t)]).to(torch.int32)
        tw = torch.softmax(randn(t, topk, dt=torch.float32), -1)
        w13 = i8(e, 2 * inter, h)
        s13 = torch.rand(e, 2 * inter, device=DEV, generator=g) * 1e-3
        w2 = i8(e, h, inter)
        s2 = torch.rand(e, h, device=DEV, generator=g) * 1e-3
        return (lambda: ops.moe_w8a8_forward(x, ids, tw, w13, s13, w2, s2)), [x, ids, tw]
    if name == "gmm1_swiglu_requant":
        rows, h, inter = 300, 512, 192
        q, s = i8(rows, h), torch.rand(rows, device=DEV, generator=g) * 0.01
        w13 = i8(3, 2 * inter, h)
        s13 = torch.rand(3, 2 * inter, device=DEV, generator=g) * 1e-3
        offs = torch.tensor([0, 90, 90, rows], dtype=torch.int64, device=DEV)
        return (lambda: ops.moe_gmm1_swiglu_quant(q, s, w13, s13, offs, inter)), [q, s]
    raise KeyError(name)


def _refresh(t, g):
    """new values of t's kind, in place (routing ids stay a permutation prefix per token)"""
    if t.dtype == torch.int8:
        t.copy_(torch.randint(-127, 128, t.shape, dtype=torch.int8, device=DEV, generator=g))
    elif t.dtype == torch.int32:
        e = 8
        t.copy_(torch.stack([torch.randperm(e, device=DEV, generator=g)[:t.shape[1]] for _ in range(t.shape[0])]))
    elif t.dtype == torch.float32 and t.dim() == 2:  # top-k weights
        t.copy_(torch.softmax(torch.randn(t.shape, device=DEV, generator=g), -1))
    elif t.dtype == torch.float32:  # per-token scales
        t.copy_(torch.rand(t.shape, device=DEV, generator=g) * 0.01)
    else:
        t.copy_(torch.randn(t.shape, device=DEV, generator=g).to(t.dtype))


NAMES = ["w4a16_m1", "w4a16_m16", "w4a16_m300", "w4a16_bf16_m1", "w8a8_m1", "w8a8_m16", "w8a8_m256", "w8a8_m600",
         "quant_per_token", "add_rms_norm_quant", "moe_chain", "gmm1_swiglu_requant"]


@pytest.mark.parametrize("name", NAMES)
def test_graph_replays_match_eager(name):
    _say("graph", name)
    fn, inputs = _case(name)
    g = torch.Generator(device=DEV).manual_seed(99)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()  # warm-up on a side stream (library load, allocator pools)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = _flat(fn())
    torch.cuda.synchronize()
    for rep in range(REPLAYS):
        for t in inputs:
            _refresh(t, g)
        expect = [o.clone() for o in _flat(fn())]
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(out, expect)):
            assert a.shape == b.shape and a.dtype == b.dtype
            assert torch.equal(a, b), f"{name}: replay {rep} output {i} differs from the eager op"
    del graph


COMPILED = ["w4a16_m16", "w8a8_m256", "quant_per_token", "add_rms_norm_quant", "moe_chain"]


@pytest.mark.parametrize("name", COMPILED)
def test_compiled_ops_match_eager(name):
    _say("compile", name)
    import torch._dynamo
    fn, _ = _case(name, seed=3)
    expect = [o.clone() for o in _flat(fn())]
    torch._dynamo.reset()
    compiled = torch.compile(fn, backend="aot_eager", fullgraph=True)
    got = _flat(compiled())
    torch.cuda.synchronize()
    for a, b in zip(got, expect):
        assert torch.equal(a, b), f"{name}: compiled output differs from the eager op"
