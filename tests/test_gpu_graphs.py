"""The ops inside a captured HIP graph and under torch.compile, on the GPU.

The C ABI launches only kernels on the caller's stream (fills are kernels, no memsets, no
host synchronisation) and the torch layer takes every buffer from the caching allocator, so a
forward + backward can be captured once and replayed. Each replay runs on inputs rewritten in
place between replays (with eager work and synchronisations in between) and is checked
against the float64 oracle on the same inputs (and against the eager ops).
"""
import pytest
import torch

import tvdcn
from oracle import oracle
from helpers import make_case, oracle_conv, rel_err

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _ops(dim, transposed):
    if transposed:
        return (getattr(torch.ops.tvdcn, f"deform_conv_transpose{dim}d"),
                getattr(torch.ops.tvdcn, f"_deform_conv_transpose{dim}d_backward"))
    return (getattr(torch.ops.tvdcn, f"deform_conv{dim}d"),
            getattr(torch.ops.tvdcn, f"_deform_conv{dim}d_backward"))


@pytest.mark.parametrize("dim,transposed", [(2, False), (2, True), (3, False)])
def test_hip_graph_capture_and_replay_fp32(dim, transposed):
    in_size = {2: [14, 12], 3: [5, 8, 7]}[dim]
    case = make_case(dim, transposed, batch=2, cin=32, cout=32, kernel=[3] * dim, stride=[1] * dim,
                     padding=[1] * dim, dilation=[1] * dim, in_size=in_size, out_pad=[0] * dim, seed=600 + dim)
    fwd, bwd = _ops(dim, transposed)
    params = ([1] * dim, [1] * dim, [0] * dim, [1] * dim, 1) if transposed else ([1] * dim, [1] * dim, [1] * dim, 1)
    names = ("input", "weight", "offset", "mask", "bias")
    st = {n: case[n].to(DEV, torch.float32).contiguous() for n in names}

    def run():
        y = fwd(st["input"], st["weight"], st["offset"], st["mask"], st["bias"], *params)
        gs = bwd(gy, st["input"], st["weight"], st["offset"], st["mask"], st["bias"], *params)
        return [y] + list(gs)

    gy = torch.rand(fwd(st["input"], st["weight"], st["offset"], st["mask"], st["bias"], *params).shape, device=DEV)

    # warm-up on a side stream (plans, kernel attributes), then capture
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            run()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = run()
    torch.cuda.synchronize()

    g = torch.Generator(device=DEV).manual_seed(601)
    for rep in range(3):
        # new inputs, written in place (eager work between replays)
        st["input"].copy_(torch.randn(st["input"].shape, device=DEV, generator=g))
        st["offset"].copy_(2.0 * torch.randn(st["offset"].shape, device=DEV, generator=g))
        st["mask"].copy_(torch.rand(st["mask"].shape, device=DEV, generator=g))
        gy.copy_(torch.randn(gy.shape, device=DEV, generator=g))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        ref = run()
        torch.cuda.synchronize()
        host = [st[n].double().cpu() for n in names]
        kw = dict(stride=[1] * dim, padding=[1] * dim, dilation=[1] * dim, groups=1, transposed=transposed,
                  output_padding=[0] * dim)
        o_ref = [oracle.forward(dim, *host, **kw)] + list(oracle.backward(dim, gy.double().cpu(), *host, **kw))
        for i, (name, a, r, o) in enumerate(zip(("output",) + tuple("grad_" + n for n in names), outs, ref, o_ref)):
            assert r is not None and a is not None, name
            e = rel_err(a.double().cpu(), o)
            assert e < (1e-5 if i == 0 else 1e-4), f"replay {rep}: {name} rel err {e} (oracle)"
            e = rel_err(a.double().cpu(), r.double().cpu())
            assert e < 1e-5, f"replay {rep}: {name} rel err {e} (eager)"


def test_torch_compile_on_gpu_fp32():
    """torch.compile (aot_eager, fullgraph) of a forward + backward runs the same HIP kernels as
    eager execution: the loss gradients against the float64 oracle (differentiable through
    helpers.oracle_conv) and against eager execution."""
    torch._dynamo.reset()
    case = make_case(2, False, batch=2, cin=32, cout=32, kernel=[3, 3], stride=[1, 1], padding=[1, 1],
                     dilation=[1, 1], in_size=[14, 12], out_pad=[0, 0], seed=610)
    names = ("input", "weight", "offset", "mask", "bias")

    def f(x, w, o, m, b):
        return (tvdcn.deform_conv2d(x, w, o, m, b, padding=1) ** 2).sum()

    def leaves():
        return [case[n].to(DEV, torch.float32).requires_grad_(True) for n in names]

    eager = leaves()
    f(*eager).backward()
    comp = leaves()
    torch.compile(f, backend="aot_eager", fullgraph=True)(*comp).backward()
    torch.cuda.synchronize()
    ref = [case[n].to(torch.float32).double().requires_grad_(True) for n in names]
    (oracle_conv(2, *ref, [1, 1], [1, 1], [1, 1], 1) ** 2).sum().backward()
    for n, a, r, o in zip(names, comp, eager, ref):
        e = rel_err(a.grad.double().cpu(), o.grad)
        assert e < 1e-4, f"grad_{n} rel err {e} (oracle)"
        e = rel_err(a.grad.double().cpu(), r.grad.double().cpu())
        assert e < 1e-5, f"grad_{n} rel err {e} (eager)"
