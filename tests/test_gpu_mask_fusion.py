"""The sigmoid mask activation folded into the kernels' mask load (deform_conv_sigmoid_mask).

Checked against the unfused composition the reference runs — ``mask_scale * sigmoid(logits)``
(tvdcn/ops/activations/mask_sigmoid.py:11-21) as a separate torch pass, then the deformable
op — forward and every gradient, the logits' gradient included, and through the packed
modules, whose default mask activation now takes the fused path.
"""
import pytest
import torch

import tvdcn_amd
from tvdcn_amd.ops.deform_conv import _deform_conv_sigmoid_mask
from helpers import make_case, rel_err
from test_gpu_parity import TOL

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _unfused(case, dim, transposed, ts, scale):
    x, w, o, logits, b = ts
    mask = scale * torch.sigmoid(logits)
    if transposed:
        fn = getattr(tvdcn_amd, f"deform_conv_transpose{dim}d")
        return fn(x, w, o, mask, b, stride=case["stride"], padding=case["padding"],
                  output_padding=case["output_padding"], dilation=case["dilation"], groups=case["groups"])
    fn = getattr(tvdcn_amd, f"deform_conv{dim}d")
    return fn(x, w, o, mask, b, stride=case["stride"], padding=case["padding"], dilation=case["dilation"],
              groups=case["groups"])


@pytest.mark.parametrize("dim,transposed,dtype", [
    (2, False, torch.float32), (1, False, torch.float32), (3, False, torch.float32), (2, True, torch.float32),
    (2, False, torch.bfloat16), (2, False, torch.float64), (1, True, torch.float64)])
def test_fused_sigmoid_mask_matches_unfused(dim, transposed, dtype):
    in_size = {1: [40], 2: [14, 12], 3: [5, 8, 7]}[dim]
    case = make_case(dim, transposed, batch=2, cin=32, cout=32, kernel=[3] * dim, stride=[1] * dim,
                     padding=[1] * dim, dilation=[1] * dim, in_size=in_size, out_pad=[0] * dim, seed=620 + dim,
                     mg=2)
    scale = 2.0
    names = ("input", "weight", "offset", "mask", "bias")
    g = torch.Generator().manual_seed(621)
    logits = torch.randn(case["mask"].shape, generator=g, dtype=torch.float64) * 2.0   # mask slot holds logits

    def leaves():
        vals = [case[n] if n != "mask" else logits for n in names]
        return [v.to(DEV, dtype).requires_grad_(True) for v in vals]

    ref_ts = leaves()
    y_ref = _unfused(case, dim, transposed, ref_ts, scale)
    gout = torch.randn(y_ref.shape, generator=g, dtype=torch.float64).to(DEV, dtype)
    y_ref.backward(gout)

    ts = leaves()
    op_pad = case["output_padding"] if transposed else [0] * dim
    y = _deform_conv_sigmoid_mask(dim, ts[0], ts[1], ts[2], ts[3], ts[4], case["stride"], case["padding"], op_pad,
                                  case["dilation"], case["groups"], transposed, scale)
    y.backward(gout)
    torch.cuda.synchronize()
    tf, tb = TOL[dtype]
    assert rel_err(y, y_ref) < tf
    for n, a, r in zip(names, ts, ref_ts):
        e = rel_err(a.grad, r.grad)
        assert e < tb, f"grad_{n} rel err {e}"


@pytest.mark.parametrize("transposed", [False, True])
def test_packed_module_default_sigmoid_is_fused(transposed):
    """PackedDeformConv2d / PackedDeformConvTranspose2d with the default mask activation give the
    numbers of the unfused composition (generators given random weights so that offsets and
    masks are not trivial)."""
    torch.manual_seed(630)
    if transposed:
        m = tvdcn_amd.PackedDeformConvTranspose2d(32, 16, 4, stride=2, padding=1, modulated=True, mask_groups=2)
    else:
        m = tvdcn_amd.PackedDeformConv2d(32, 16, 3, padding=1, modulated=True, mask_groups=2)
    m = m.to(DEV)
    with torch.no_grad():
        m.offset_generator.weight.normal_(0, 0.05)
        m.mask_generator.weight.normal_(0, 0.1)
    x = torch.randn(2, 32, 12, 10, device=DEV)

    offset, logits, scale = m._generate(x)
    assert scale == 2.0 and isinstance(m.mask_activation, tvdcn_amd.MaskSigmoid)
    y = m(x)
    y.square().sum().backward()
    fused = [p.grad.clone() for p in m.parameters()]
    m.zero_grad()

    offset = m.offset_generator(x)
    mask = m.mask_activation(m.mask_generator(x))
    if transposed:
        y_ref = tvdcn_amd.deform_conv_transpose2d(x, m.weight, offset, mask, m.bias, m.stride, m.padding,
                                                  m.output_padding, m.dilation, m.groups)
    else:
        y_ref = tvdcn_amd.deform_conv2d(x, m.weight, offset, mask, m.bias, m.stride, m.padding, m.dilation, m.groups)
    y_ref.square().sum().backward()
    torch.cuda.synchronize()
    assert rel_err(y, y_ref) < 1e-5
    for (name, p), a in zip(m.named_parameters(), fused):
        e = rel_err(a, p.grad)
        assert e < 1e-4, f"{name} grad rel err {e}"


def test_fused_sigmoid_mask_without_offsets_and_empty_batch():
    """Offset-free sampling with a logit mask, and an empty batch (zero gradients)."""
    case = make_case(2, False, batch=2, cin=32, cout=32, kernel=[3, 3], stride=[1, 1], padding=[1, 1],
                     dilation=[1, 1], in_size=[14, 12], out_pad=[0, 0], seed=640, deformable=False)
    g = torch.Generator().manual_seed(641)
    logits = torch.randn(case["mask"].shape, generator=g, dtype=torch.float64)
    vals = [case["input"], case["weight"], None, logits, case["bias"]]
    ref = [None if v is None else v.to(DEV, torch.float32).requires_grad_(True) for v in vals]
    fus = [None if v is None else v.to(DEV, torch.float32).requires_grad_(True) for v in vals]
    y_ref = tvdcn_amd.deform_conv2d(ref[0], ref[1], None, 2.0 * torch.sigmoid(ref[3]), ref[4], padding=1)
    gout = torch.randn(y_ref.shape, generator=g, dtype=torch.float64).to(DEV, torch.float32)
    y_ref.backward(gout)
    y = _deform_conv_sigmoid_mask(2, fus[0], fus[1], None, fus[3], fus[4], 1, 1, 0, 1, 1, False, 2.0)
    y.backward(gout)
    torch.cuda.synchronize()
    assert rel_err(y, y_ref) < 1e-5
    for a, r in zip(fus, ref):
        if a is not None:
            assert rel_err(a.grad, r.grad) < 1e-4
    # empty batch
    x = torch.zeros(0, 32, 14, 12, device=DEV, requires_grad=True)
    w = fus[1].detach().clone().requires_grad_(True)
    lg = torch.zeros(0, 9, 14, 12, device=DEV, requires_grad=True)
    y0 = _deform_conv_sigmoid_mask(2, x, w, None, lg, None, 1, 1, 0, 1, 1, False, 2.0)
    assert y0.shape == (0, 32, 14, 12)
    y0.sum().backward()
    assert w.grad is not None and float(w.grad.abs().sum()) == 0.0 and lg.grad.shape == lg.shape
