"""Mask activations folded into the kernels' mask load (op tvdcn::deform_conv_mask_activation):
``scale * sigmoid`` (tvdcn's MaskSigmoid) and the softmax over the kernel taps of each mask
group (MaskSoftmax{N}d).

Reference: the float64 oracle, differentiable through ``helpers.OracleDeformConv``, applied to
the mask activated in float64 torch ops on the CPU, so that the logits' gradient comes from
torch's float64 chain rule: forward and every gradient, for the op and through the packed
modules (their generator convolutions run in float64 on the CPU too).
"""
import pytest
import torch

import tvdcn
from tvdcn.ops.deform_conv import _deform_conv_mask_activation
from helpers import make_case, mask_activation_f64, oracle_conv, oracle_offsets, rel_err
from test_gpu_parity import TOL

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
NAMES = ("input", "weight", "offset", "mask", "bias")


def _oracle_activated(case, dim, transposed, vals, activation, scale):
    """float64 reference on CPU leaves; returns (out, leaves)"""
    leaves = [None if v is None else v.detach().double().cpu().requires_grad_(True) for v in vals]
    x, w, o, logits, b = leaves
    if o is not None:
        # sampling positions rounded as the kernels form them (float16: to half precision, as the
        # reference's c10::Half; float32 / bfloat16: to float32)
        o = o + (oracle_offsets(case, o.detach(), vals[2].dtype) - o.detach())
    kn = 1
    for k in w.shape[2:]:
        kn *= k
    mask = mask_activation_f64(logits, activation, kn, scale)
    out = oracle_conv(dim, x, w, o, mask, b, case["stride"], case["padding"], case["dilation"], case["groups"],
                      transposed, case["output_padding"] if transposed else 0)
    return out, leaves


@pytest.mark.parametrize("activation", [1, 2], ids=["sigmoid", "softmax"])
@pytest.mark.parametrize("dim,transposed,dtype", [
    (2, False, torch.float32), (1, False, torch.float32), (3, False, torch.float32), (2, True, torch.float32),
    (3, True, torch.float32), (2, False, torch.bfloat16), (2, False, torch.float16), (2, False, torch.float64),
    (1, True, torch.float64)])
def test_fused_mask_activation_matches_oracle(dim, transposed, dtype, activation):
    in_size = {1: [40], 2: [14, 12], 3: [5, 8, 7]}[dim]
    case = make_case(dim, transposed, batch=2, cin=32, cout=32, kernel=[3] * dim, stride=[1] * dim,
                     padding=[1] * dim, dilation=[1] * dim, in_size=in_size, out_pad=[0] * dim, seed=620 + dim,
                     mg=2)
    scale = 2.0
    g = torch.Generator().manual_seed(621)
    logits = torch.randn(case["mask"].shape, generator=g, dtype=torch.float64) * 2.0   # mask slot holds logits
    vals = [(case[n] if n != "mask" else logits).to(dtype) for n in NAMES]   # inputs rounded to dtype

    ts = [v.to(DEV).requires_grad_(True) for v in vals]
    op_pad = case["output_padding"] if transposed else [0] * dim
    y = _deform_conv_mask_activation(ts[0], ts[1], ts[2], ts[3], ts[4], case["stride"], case["padding"], op_pad,
                                     case["dilation"], case["groups"], transposed, activation, scale)
    gout = torch.randn(y.shape, generator=g, dtype=torch.float64).to(dtype)
    y.backward(gout.to(DEV))
    torch.cuda.synchronize()

    y_ref, leaves = _oracle_activated(case, dim, transposed, vals, activation, scale)
    y_ref.backward(gout.double())
    tf, tb = TOL[dtype]
    assert rel_err(y, y_ref) < tf
    for n, a, r in zip(NAMES, ts, leaves):
        e = rel_err(a.grad, r.grad)
        assert e < tb, f"grad_{n} rel err {e}"


def _module_ref_f64(m, x, transposed):
    """the packed module's computation in float64 on the CPU, the oracle for the deformable part;
    returns (out, {parameter name: float64 leaf})"""
    dim = m.weight.dim() - 2
    params = {n: p.detach().double().cpu().requires_grad_(True) for n, p in m.named_parameters()}
    conv = {1: torch.nn.functional.conv1d, 2: torch.nn.functional.conv2d, 3: torch.nn.functional.conv3d}[dim]
    xo = x.detach().double().cpu()
    og, mg = m.offset_generator, m.mask_generator
    off = conv(xo, params["offset_generator.weight"], None, og.stride, og.padding, og.dilation, og.groups)
    logits = conv(xo, params["mask_generator.weight"], None, mg.stride, mg.padding, mg.dilation, mg.groups)
    kn = 1
    for k in m.kernel_size:
        kn *= k
    act = 1 if isinstance(m.mask_activation, tvdcn.MaskSigmoid) else 2
    mask = mask_activation_f64(logits, act, kn, getattr(m.mask_activation, "scale", 2.0))
    y = oracle_conv(dim, xo, params["weight"], off, mask, params.get("bias"), list(m.stride), list(m.padding),
                    list(m.dilation), m.groups, transposed, list(m.output_padding) if transposed else 0)
    return y, params


@pytest.mark.parametrize("activation", ["sigmoid", "softmax"])
@pytest.mark.parametrize("transposed", [False, True])
def test_packed_module_fused_activation_matches_oracle(transposed, activation):
    """PackedDeformConv2d / PackedDeformConvTranspose2d with a fusable mask activation: forward and every
    parameter gradient against the float64 composition (generators given random weights so that offsets
    and masks are not trivial)."""
    torch.manual_seed(630)
    if transposed:
        m = tvdcn.PackedDeformConvTranspose2d(32, 16, 4, stride=2, padding=1, modulated=True, mask_groups=2,
                                              mask_activation=activation)
    else:
        m = tvdcn.PackedDeformConv2d(32, 16, 3, padding=1, modulated=True, mask_groups=2,
                                     mask_activation=activation)
    with torch.no_grad():
        m.offset_generator.weight.normal_(0, 0.05)
        m.mask_generator.weight.normal_(0, 0.3)
    m = m.to(DEV)
    assert m._mask_fusion()[0] == (1 if activation == "sigmoid" else 2)
    x = torch.randn(2, 32, 12, 10, device=DEV)
    y = m(x)
    gy = torch.randn(y.shape, generator=torch.Generator().manual_seed(631), dtype=torch.float64)
    y.backward(gy.to(DEV, y.dtype))
    torch.cuda.synchronize()

    y_ref, params = _module_ref_f64(m, x, transposed)
    y_ref.backward(gy)
    assert rel_err(y, y_ref) < 1e-5
    for name, p in m.named_parameters():
        e = rel_err(p.grad, params[name].grad)
        assert e < 1e-4, f"{name} grad rel err {e}"


def test_fused_mask_activation_without_offsets_and_empty_batch():
    """Offset-free sampling with a logit mask (both activations), and an empty batch (zero gradients)."""
    case = make_case(2, False, batch=2, cin=32, cout=32, kernel=[3, 3], stride=[1, 1], padding=[1, 1],
                     dilation=[1, 1], in_size=[14, 12], out_pad=[0, 0], seed=640, deformable=False)
    g = torch.Generator().manual_seed(641)
    logits = torch.randn(case["mask"].shape, generator=g, dtype=torch.float64)
    vals = [case["input"], case["weight"], None, logits, case["bias"]]
    for activation in (1, 2):
        ts = [None if v is None else v.to(DEV, torch.float32).requires_grad_(True) for v in vals]
        y = _deform_conv_mask_activation(ts[0], ts[1], None, ts[3], ts[4], [1, 1], [1, 1], [0, 0], [1, 1], 1,
                                         False, activation, 2.0)
        gout = torch.randn(y.shape, generator=g, dtype=torch.float64)
        y.backward(gout.to(DEV, torch.float32))
        torch.cuda.synchronize()
        y_ref, leaves = _oracle_activated(case, 2, False, [v.float() if v is not None else None for v in vals],
                                          activation, 2.0)
        y_ref.backward(gout)
        assert rel_err(y, y_ref) < 1e-5
        for a, r in zip(ts, leaves):
            if a is not None:
                assert rel_err(a.grad, r.grad) < 1e-4
    # empty batch
    x = torch.zeros(0, 32, 14, 12, device=DEV, requires_grad=True)
    w = torch.rand(32, 32, 3, 3, device=DEV, requires_grad=True)
    lg = torch.zeros(0, 9, 14, 12, device=DEV, requires_grad=True)
    for activation in (1, 2):
        y0 = _deform_conv_mask_activation(x, w, None, lg, None, [1, 1], [1, 1], [0, 0], [1, 1], 1, False,
                                          activation, 2.0)
        assert y0.shape == (0, 32, 14, 12)
        y0.sum().backward()
        assert w.grad is not None and float(w.grad.abs().sum()) == 0.0 and lg.grad.shape == lg.shape
