"""The CPU dispatch key: tvdcn's ops on host tensors (tvdcn_amd/csrc/torch/cpu_kernels.cpp), the
counterpart of the reference's CPU kernels (tvdcn/csrc/ops/cpu/deform_conv2d_kernel.cpp:645 and
twins).

Checked like the GPU path: against the float64 oracle (every op, rank, flag and group combination;
float32 / float16 / bfloat16 at the same tolerances as the GPU tests), against the golden fixtures
that the reference's own CPU build wrote (tests/golden), against the closed forms (zero offsets and
a unit mask are plain convolutions), and by torch.autograd.gradcheck in float64. No GPU.
"""
import glob
import itertools
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import tvdcn
from oracle import oracle
from helpers import make_case, oracle_offsets, rel_err

NAMES = ("input", "weight", "offset", "mask", "bias")
TOL = {torch.float64: (1e-10, 1e-10), torch.float32: (1e-5, 1e-4), torch.float16: (1e-2, 1e-2),
       torch.bfloat16: (1e-2, 1e-2)}


def op_of(case):
    return getattr(tvdcn, f"deform_conv_transpose{case['dim']}d" if case["transposed"] else f"deform_conv{case['dim']}d")


def kwargs_of(case):
    kw = dict(stride=case["stride"], padding=case["padding"], dilation=case["dilation"], groups=case["groups"])
    if case["transposed"]:
        kw["output_padding"] = case["output_padding"]
    return kw


def run_cpu(case, dtype, grad_out=None):
    ts = [case[n].detach().to(dtype).clone().requires_grad_(True) if case[n] is not None else None for n in NAMES]
    out = op_of(case)(*ts, **kwargs_of(case))
    if grad_out is None:
        grad_out = torch.rand(out.shape, generator=torch.Generator().manual_seed(7), dtype=torch.float64)
    out.backward(grad_out.to(dtype))
    return out, [t.grad if t is not None else None for t in ts], grad_out


def run_oracle(case, grad_out, dtype):
    args = [None if case[n] is None else case[n].to(dtype).double() for n in NAMES]
    args[2] = oracle_offsets(case, args[2], dtype)
    kw = dict(stride=case["stride"], padding=case["padding"], dilation=case["dilation"], groups=case["groups"],
              transposed=case["transposed"], output_padding=case["output_padding"])
    return oracle.forward(case["dim"], *args, **kw), oracle.backward(case["dim"], grad_out.to(dtype).double(),
                                                                     *args, **kw)


def check(case, dtype):
    out, grads, gout = run_cpu(case, dtype)
    assert out.device.type == "cpu" and out.dtype == dtype
    ref_out, ref_grads = run_oracle(case, gout, dtype)
    tf, tb = TOL[dtype]
    assert list(out.shape) == case["out_shape"]
    assert rel_err(out, ref_out) < tf, "forward"
    for name, g, r in zip(NAMES, grads, ref_grads):
        if r is None:
            assert g is None
            continue
        assert g.dtype == dtype
        assert rel_err(g, r) < tb, f"grad_{name}"


COMBOS = list(itertools.product([1, 2, 3], [False, True], [(True, True), (True, False), (False, True),
                                                            (False, False)]))


@pytest.mark.parametrize("dim,transposed,flags", COMBOS)
def test_cpu_fp64_against_oracle(dim, transposed, flags):
    deformable, modulated = flags
    case = make_case(dim, transposed, cin=4, cout=6, groups=2, og=2, mg=1, deformable=deformable,
                     modulated=modulated, seed=dim * 10 + int(transposed))
    check(case, torch.float64)


@pytest.mark.parametrize("dim,transposed", list(itertools.product([1, 2, 3], [False, True])))
def test_cpu_fp32_groups_against_oracle(dim, transposed):
    case = make_case(dim, transposed, cin=8, cout=12, groups=2, og=4, mg=2, seed=100 + dim)
    check(case, torch.float32)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("transposed", [False, True])
def test_cpu_half_precision(dtype, transposed):
    case = make_case(2, transposed, batch=2, cin=16, cout=16, og=2, mg=2, kernel=[3, 3], stride=[1, 1],
                     padding=[1, 1], dilation=[1, 1], in_size=[9, 10], out_pad=[0, 0], seed=300)
    check(case, dtype)


@pytest.mark.parametrize("transposed", [False, True])
def test_cpu_chunked_columns(transposed):
    """more column pixels than one chunk of the sampling table (several chunks per image); float64,
    where no float32 rounding of a sampling position near a cell boundary flips its corner cell"""
    case = make_case(2, transposed, batch=2, cin=4, cout=8, og=2, mg=2, kernel=[3, 3], stride=[1, 1],
                     padding=[1, 1], dilation=[1, 1], in_size=[96, 120], out_pad=[0, 0], seed=310)
    check(case, torch.float64)


GOLDEN = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "*.npz")))


@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p)[:-4] for p in GOLDEN])
def test_cpu_golden_fixture(path):
    """the reference CPU build's own outputs and gradients (float64, float32, float16) through the
    public functions on host tensors"""
    z = np.load(path, allow_pickle=False)
    t = {k: torch.from_numpy(z[k]) for k in z.files}
    dim, tr, G = int(t["dim"]), bool(int(t["transposed"])), int(t["groups"])
    s, p, d, op = (t[k].tolist() for k in ("stride", "padding", "dilation", "output_padding"))
    dtype = t["input"].dtype
    ts = [t[n].clone().requires_grad_(True) if n in t else None for n in NAMES]
    if tr:
        out = getattr(tvdcn, f"deform_conv_transpose{dim}d")(*ts, s, p, op, d, G)
    else:
        out = getattr(tvdcn, f"deform_conv{dim}d")(*ts, s, p, d, G)
    out.backward(t["grad_out"])
    tf, tb = TOL[dtype]
    assert rel_err(out, t["out"]) < tf
    for n, ten in zip(NAMES, ts):
        if ten is not None:
            assert rel_err(ten.grad, t["g_" + n]) < tb, n


CONV = {1: F.conv1d, 2: F.conv2d, 3: F.conv3d}
CONVT = {1: F.conv_transpose1d, 2: F.conv_transpose2d, 3: F.conv_transpose3d}


@pytest.mark.parametrize("dim,transposed", list(itertools.product([1, 2, 3], [False, True])))
def test_cpu_zero_offset_unit_mask_is_plain_convolution(dim, transposed):
    """closed form, independent of the reference: forward and every gradient equal torch's own
    convolution's"""
    case = make_case(dim, transposed, batch=2, cin=4, cout=6, groups=2, seed=5 + dim)
    x, w, o, m, b = (case[n].clone().requires_grad_(True) for n in NAMES)
    with torch.no_grad():
        o.zero_()
        m.fill_(1.0)
    out = op_of(case)(x, w, o, m, b, **kwargs_of(case))
    xr, wr, br = (t.detach().clone().requires_grad_(True) for t in (x, w, b))
    if transposed:
        ref = CONVT[dim](xr, wr, br, case["stride"], case["padding"], case["output_padding"], case["groups"],
                         case["dilation"])
    else:
        ref = CONV[dim](xr, wr, br, case["stride"], case["padding"], case["dilation"], case["groups"])
    assert rel_err(out, ref) < 1e-12
    gout = torch.rand(out.shape, generator=torch.Generator().manual_seed(1), dtype=torch.float64)
    out.backward(gout)
    ref.backward(gout)
    for a, r in ((x, xr), (w, wr), (b, br)):
        assert rel_err(a.grad, r.grad) < 1e-12


@pytest.mark.parametrize("dim,transposed", [(1, False), (2, False), (3, False), (2, True)])
def test_cpu_gradcheck(dim, transposed):
    """torch.autograd.gradcheck in float64, as the reference's tests/test_grad.py:34-40 does"""
    case = make_case(dim, transposed, batch=1, cin=2, cout=2, seed=60 + dim,
                     in_size={1: [5], 2: [4, 5], 3: [3, 4, 3]}[dim], offset_scale=0.7)
    ts = tuple(case[n].clone().requires_grad_(True) for n in NAMES)
    kw = kwargs_of(case)
    assert torch.autograd.gradcheck(lambda *a: op_of(case)(*a, **kw), ts, eps=1e-6, atol=1e-5, nondet_tol=1e-5)


def test_cpu_unbatched_channels_last_and_empty():
    case = make_case(2, False, batch=1, cin=4, cout=4, bias=False, seed=400)
    x, w, o, m = (case[n] for n in ("input", "weight", "offset", "mask"))
    out = tvdcn.deform_conv2d(x[0], w, o[0], m[0], None, case["stride"], case["padding"], case["dilation"])
    ref = oracle.forward(2, x, w, o, m, None, case["stride"], case["padding"], case["dilation"])
    assert out.shape == ref.shape[1:] and rel_err(out, ref[0]) < 1e-10
    xc = torch.rand(2, 8, 9, 9, dtype=torch.float64).to(memory_format=torch.channels_last)
    wc = torch.rand(8, 8, 3, 3, dtype=torch.float64)
    oc = torch.randn(2, 18, 9, 9, dtype=torch.float64)
    got = tvdcn.deform_conv2d(xc, wc, oc, None, None, padding=1)
    assert rel_err(got, oracle.forward(2, xc.contiguous(), wc, oc, None, None, padding=1)) < 1e-10
    xe = torch.zeros(0, 4, 6, 6, requires_grad=True)
    we = torch.rand(5, 4, 3, 3, requires_grad=True)
    oe = torch.zeros(0, 18, 4, 4, requires_grad=True)
    oute = tvdcn.deform_conv2d(xe, we, oe, None, torch.rand(5))
    oute.sum().backward()
    assert oute.shape == (0, 5, 4, 4) and we.grad.abs().sum().item() == 0.0


def test_cpu_validation_messages_match_gpu_layer():
    """the CPU key runs the same shape checks (reference wording) as the GPU key"""
    x = torch.rand(1, 4, 5, 5)
    w = torch.rand(6, 3, 3, 3)
    with pytest.raises(RuntimeError, match="weight.size\\(1\\) \\* groups == in_channels"):
        tvdcn.deform_conv2d(x, w)
    with pytest.raises(RuntimeError, match="offset output dims"):
        tvdcn.deform_conv2d(x, torch.rand(6, 4, 3, 3), torch.rand(1, 18, 4, 4))


def test_cpu_mask_softmax_matches_torch_softmax():
    g = torch.Generator().manual_seed(9)
    for dim, ks, shape in [(1, (5,), (3, 20, 33)), (2, (4, 4), (2, 32, 6, 7)), (3, (3, 3, 3), (2, 27, 3, 4, 5))]:
        x = torch.randn(*shape, generator=g, dtype=torch.float64).requires_grad_(True)
        y = getattr(tvdcn, f"mask_softmax{dim}d")(x, ks)
        kn = int(np.prod(ks))
        xr = x.detach().clone().requires_grad_(True)
        yr = torch.softmax(xr.view(shape[0], shape[1] // kn, kn, -1), dim=2).view(shape)
        assert rel_err(y, yr) < 1e-14
        gy = torch.randn(*shape, generator=g, dtype=torch.float64)
        y.backward(gy)
        yr.backward(gy)
        assert rel_err(x.grad, xr.grad) < 1e-13
        assert rel_err(y, oracle.mask_softmax_forward(x.detach(), kn)) < 1e-14


@pytest.mark.parametrize("activation", ["sigmoid", "softmax"])
@pytest.mark.parametrize("dim,transposed", [(2, False), (1, True), (3, False)])
def test_cpu_packed_modules_fused_mask_activation(activation, dim, transposed):
    """the packed modules' fused mask activation on host tensors: the same numbers as the
    unfused composition (the activation as its own op, then the convolution), float64"""
    torch.manual_seed(20 + dim)
    if transposed:
        mod = getattr(tvdcn, f"PackedDeformConvTranspose{dim}d")(4, 6, 3, stride=1, padding=1, modulated=True,
                                                                  offset_groups=2, mask_groups=2,
                                                                  mask_activation=activation).double()
    else:
        mod = getattr(tvdcn, f"PackedDeformConv{dim}d")(4, 6, 3, padding=1, modulated=True, offset_groups=2,
                                                        mask_groups=2, mask_activation=activation).double()
    for gen in (mod.offset_generator, mod.mask_generator):
        torch.nn.init.normal_(gen.weight, std=0.3)
    x = torch.rand(2, 4, *([6, 5, 4][:dim]), dtype=torch.float64, requires_grad=True)
    y = mod(x)
    assert mod._mask_fusion()[0] != 0
    gy = torch.rand(y.shape, dtype=torch.float64)
    y.backward(gy)
    fused = [x.grad.clone()] + [p.grad.clone() for p in mod.parameters()]
    # unfused: the module's own pieces composed in Python
    x.grad = None
    mod.zero_grad()
    off = mod.offset_generator(x)
    msk = mod.mask_activation(mod.mask_generator(x))
    fn = getattr(tvdcn, f"deform_conv_transpose{dim}d" if transposed else f"deform_conv{dim}d")
    kw = dict(stride=mod.stride, padding=mod.padding, dilation=mod.dilation, groups=mod.groups)
    if transposed:
        kw["output_padding"] = mod.output_padding
    y2 = fn(x, mod.weight, off, msk, mod.bias, **kw)
    assert rel_err(y, y2) < 1e-12
    y2.backward(gy)
    for a, b in zip(fused, [x.grad] + [p.grad for p in mod.parameters()]):
        assert rel_err(a, b) < 1e-11
