"""GPU parity: tvdcn's HIP kernels against the float64 oracle (a C restatement of
tvdcn's CPU algorithm, itself pinned to the reference build and the golden fixtures).

Tolerances (norm-wise, see helpers.rel_err): float64 1e-9; float32 forward 1e-5 and
backward 1e-4 (atomic ordering); float16 / bfloat16 1e-2 against the oracle run on
the same rounded inputs. The oracle samples at the positions the kernels form: base + offset
rounded once to float32 (float32, bfloat16) or to half precision (float16), as the reference's
own float32 and c10::Half arithmetic rounds them (helpers.rounded_position_offsets).
"""
import itertools

import pytest
import torch

import tvdcn
from oracle import oracle
from helpers import make_case, oracle_offsets, rel_err

pytestmark = pytest.mark.gpu

DEV = "cuda"
TOL = {torch.float64: (1e-9, 1e-9), torch.float32: (1e-5, 1e-4), torch.float16: (1e-2, 1e-2),
       torch.bfloat16: (1e-2, 1e-2)}


def run_gpu(case, dtype, grad_out=None):
    """forward + autograd backward on the GPU; returns (out, [grads...], grad_out used)."""
    names = ("input", "weight", "offset", "mask", "bias")
    ts = [case[n].to(DEV, dtype).requires_grad_(True) if case[n] is not None else None for n in names]
    if case["transposed"]:
        fn = getattr(tvdcn, f"deform_conv_transpose{case['dim']}d")
        out = fn(*ts, stride=case["stride"], padding=case["padding"], output_padding=case["output_padding"],
                 dilation=case["dilation"], groups=case["groups"])
    else:
        fn = getattr(tvdcn, f"deform_conv{case['dim']}d")
        out = fn(*ts, stride=case["stride"], padding=case["padding"], dilation=case["dilation"],
                 groups=case["groups"])
    if grad_out is None:
        g = torch.Generator().manual_seed(7)
        grad_out = torch.rand(out.shape, generator=g, dtype=torch.float64)
    out.backward(grad_out.to(DEV, dtype))
    torch.cuda.synchronize()
    return out, [t.grad if t is not None else None for t in ts], grad_out


def run_oracle(case, grad_out, dtype):
    cast = (lambda t: None if t is None else t.to(dtype).double())
    args = [cast(case[n]) for n in ("input", "weight", "offset", "mask", "bias")]
    args[2] = oracle_offsets(case, args[2], dtype)
    kw = dict(stride=case["stride"], padding=case["padding"], dilation=case["dilation"], groups=case["groups"],
              transposed=case["transposed"], output_padding=case["output_padding"])
    out = oracle.forward(case["dim"], *args, **kw)
    grads = oracle.backward(case["dim"], grad_out.to(dtype).double(), *args, **kw)
    return out, grads


def check(case, dtype):
    out, grads, gout = run_gpu(case, dtype)
    ref_out, ref_grads = run_oracle(case, gout, dtype)
    tf, tb = TOL[dtype]
    assert list(out.shape) == case["out_shape"]
    e = rel_err(out, ref_out)
    assert e < tf, f"forward rel err {e}"
    for name, g, r in zip(("input", "weight", "offset", "mask", "bias"), grads, ref_grads):
        if r is None:
            assert g is None
            continue
        e = rel_err(g, r)
        assert e < tb, f"grad_{name} rel err {e}"


# flag / group combinations at the reference's test sizes (generic, scalar-channel path)
COMBOS = list(itertools.product([1, 2, 3], [False, True], [(True, True), (True, False), (False, True),
                                                              (False, False)]))


@pytest.mark.parametrize("dim,transposed,flags", COMBOS)
def test_small_fp64(dim, transposed, flags):
    deformable, modulated = flags
    case = make_case(dim, transposed, cin=4, cout=6, groups=2, og=2, mg=1, deformable=deformable,
                     modulated=modulated, seed=dim * 10 + int(transposed))
    check(case, torch.float64)


@pytest.mark.parametrize("dim,transposed", list(itertools.product([1, 2, 3], [False, True])))
def test_small_fp32(dim, transposed):
    case = make_case(dim, transposed, cin=4, cout=6, groups=2, og=2, mg=2, seed=100 + dim)
    check(case, torch.float32)


@pytest.mark.parametrize("dim,transposed,og,mg,groups", [
    (2, False, 1, 1, 1), (2, False, 2, 4, 1), (2, False, 4, 2, 2), (1, False, 4, 4, 1), (3, False, 1, 1, 1),
    (2, True, 2, 2, 1), (2, True, 1, 1, 2), (1, True, 2, 1, 1), (3, True, 1, 1, 1)])
def test_vector_path_fp32(dim, transposed, og, mg, groups):
    """channel counts that are multiples of 16/64: exercises the 4-channel vector gather and the
    wave-reduced offset/mask gradients"""
    in_size = {1: [40], 2: [12, 11], 3: [5, 6, 7]}[dim]
    case = make_case(dim, transposed, batch=2, cin=64, cout=128 if not transposed else 64, groups=groups, og=og,
                     mg=mg, kernel=[3] * dim, stride=[1] * dim, padding=[1] * dim, dilation=[1] * dim,
                     in_size=in_size, out_pad=[0] * dim, seed=200 + dim)
    check(case, torch.float32)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("transposed", [False, True])
def test_half_precision(dtype, transposed):
    case = make_case(2, transposed, batch=2, cin=32, cout=32, og=2, mg=2, kernel=[3, 3], stride=[1, 1],
                     padding=[1, 1], dilation=[1, 1], in_size=[9, 10], out_pad=[0, 0], seed=300)
    check(case, dtype)


def test_unbatched_and_no_bias():
    case = make_case(2, False, batch=1, cin=4, cout=4, bias=False, seed=400)
    x = case["input"][0].to(DEV).requires_grad_(True)
    w = case["weight"].to(DEV)
    o = case["offset"][0].to(DEV)
    m = case["mask"][0].to(DEV)
    out = tvdcn.deform_conv2d(x, w, o, m, None, case["stride"], case["padding"], case["dilation"])
    ref = oracle.forward(2, case["input"], case["weight"], case["offset"], case["mask"], None,
                         case["stride"], case["padding"], case["dilation"])
    assert out.shape == ref.shape[1:]
    assert rel_err(out, ref[0]) < 1e-9


def test_zero_offset_unit_mask_is_conv2d():
    """closed form: zero offsets and unit mask reduce to F.conv2d (torch's own GPU convolution)"""
    g = torch.Generator().manual_seed(5)
    x = torch.randn(2, 16, 13, 13, generator=g, dtype=torch.float64).to(DEV)
    w = torch.randn(32, 8, 3, 3, generator=g, dtype=torch.float64).to(DEV)
    b = torch.randn(32, generator=g, dtype=torch.float64).to(DEV)
    off = torch.zeros(2, 2 * 9, 7, 7, dtype=torch.float64, device=DEV)
    msk = torch.ones(2, 9, 7, 7, dtype=torch.float64, device=DEV)
    out = tvdcn.deform_conv2d(x, w, off, msk, b, stride=2, padding=1, dilation=1, groups=2)
    ref = torch.nn.functional.conv2d(x, w, b, stride=2, padding=1, groups=2)
    assert rel_err(out, ref) < 1e-10


def test_mask_softmax_matches_torch_softmax():
    g = torch.Generator().manual_seed(9)
    for dim, ks, shape in [(1, (5,), (3, 20, 33)), (2, (4, 4), (2, 32, 6, 7)), (3, (3, 3, 3), (2, 27, 3, 4, 5)),
                           (2, (7, 7), (1, 98, 5, 5))]:
        x = torch.randn(*shape, generator=g, dtype=torch.float64).to(DEV).requires_grad_(True)
        y = getattr(tvdcn, f"mask_softmax{dim}d")(x, ks)
        kn = 1
        for k in ks:
            kn *= k
        xr = x.detach().clone().requires_grad_(True)
        yr = torch.softmax(xr.view(shape[0], shape[1] // kn, kn, -1), dim=2).view(shape)
        assert rel_err(y, yr) < 1e-12
        gy = torch.randn(*shape, generator=g, dtype=torch.float64).to(DEV)
        y.backward(gy)
        yr.backward(gy)
        assert rel_err(x.grad, xr.grad) < 1e-12


@pytest.mark.parametrize("K,shape", [(3, (2, 6, 37)), (4, (3, 8, 130)), (7, (2, 14, 65)), (9, (1, 18, 4097)),
                                     (25, (2, 50, 99)), (9, (4, 36, 20000)), (16, (2, 32, 70001)),
                                     (9, (70000, 9, 1)), (40, (2, 80, 33))])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_mask_softmax_tap_counts_and_ragged_columns(K, shape, dtype):
    """every tap-count instantiation of the softmax kernels (3, 4, 9, 25 compiled in, 7 and 40 at
    run time, 40 on the re-reading kernel), one and four columns per thread, column counts that
    are not multiples of the 64-lane wavefront, and more (batch, group) rows than one grid axis
    holds: against torch.softmax on the same view, forward and backward"""
    g = torch.Generator().manual_seed(K + shape[-1])
    x = torch.randn(*shape, generator=g).to(DEV, dtype).requires_grad_(True)
    y = torch.ops.tvdcn.mask_softmax(x, K)
    xr = x.detach().double().requires_grad_(True)
    yr = torch.softmax(xr.view(shape[0], shape[1] // K, K, -1), dim=2).view(shape)
    tol = 1e-6 if dtype == torch.float32 else 1e-2
    assert rel_err(y, yr) < tol
    gy = torch.randn(*shape, generator=g).to(DEV, dtype)
    y.backward(gy)
    yr.backward(gy.double())
    assert rel_err(x.grad, xr.grad) < (1e-5 if dtype == torch.float32 else 2e-2)


@pytest.mark.parametrize("dim,transposed", [(2, False), (2, True), (1, False), (3, False)])
def test_autocast_runs_in_float32_and_casts_back(dim, transposed):
    """Under torch.autocast("cuda"), float16 inputs run in float32 and the result is cast back to the
    input's type (autocast/deform_conv2d_kernel.cpp:9-38): the same numbers as the float32 op on the
    widened inputs, cast to float16; gradients reach the float16 leaves; float32 against the oracle."""
    case = make_case(dim, transposed, batch=2, cin=16, cout=16, seed=700 + dim)
    names = ("input", "weight", "offset", "mask", "bias")
    fn = getattr(tvdcn, f"deform_conv_transpose{dim}d" if transposed else f"deform_conv{dim}d")
    kw = dict(stride=case["stride"], padding=case["padding"], dilation=case["dilation"], groups=case["groups"])
    if transposed:
        kw["output_padding"] = case["output_padding"]
    ts16 = [case[n].to(DEV, torch.float16).requires_grad_(True) for n in names]
    with torch.autocast("cuda", dtype=torch.float16):
        y = fn(*ts16, **kw)
    assert y.dtype == torch.float16
    ts32 = [t.detach().float().requires_grad_(True) for t in ts16]
    y32 = fn(*ts32, **kw)
    assert torch.equal(y, y32.half())
    g = torch.rand(y.shape, generator=torch.Generator().manual_seed(7), dtype=torch.float64)
    y.backward(g.to(DEV, torch.float16))
    y32.backward(g.to(DEV, torch.float16).float())
    torch.cuda.synchronize()
    for n, a, b in zip(names, ts16, ts32):
        assert a.grad is not None and a.grad.dtype == torch.float16, n
        # float atomics in the offset / mask gradients: not bit-reproducible from run to run
        assert rel_err(a.grad, b.grad.half()) < 1e-3, n
    rounded = {k: (v.half().double() if isinstance(v, torch.Tensor) else v) for k, v in case.items()}
    ref_out, _ = run_oracle(rounded, g, torch.float64)
    assert rel_err(y32, ref_out) < 1e-5
