"""Shared test helpers: case construction, norm-wise error metrics, the C ABI descriptor."""
import ctypes
import itertools

import torch


class Desc(ctypes.Structure):
    """tvdcn_conv_desc of include/tvdcn_hip.h"""
    _fields_ = [("dim", ctypes.c_int32), ("transposed", ctypes.c_int32), ("dtype", ctypes.c_int32),
                ("flags", ctypes.c_int32), ("batch", ctypes.c_int64), ("in_channels", ctypes.c_int64),
                ("out_channels", ctypes.c_int64), ("groups", ctypes.c_int64), ("offset_groups", ctypes.c_int64),
                ("mask_groups", ctypes.c_int64), ("in_size", ctypes.c_int64 * 3), ("kernel", ctypes.c_int64 * 3),
                ("stride", ctypes.c_int64 * 3), ("padding", ctypes.c_int64 * 3), ("dilation", ctypes.c_int64 * 3),
                ("output_padding", ctypes.c_int64 * 3), ("mask_scale", ctypes.c_double)]


def rel_err(a, ref):
    """max(relative L2 error, max-abs error / max|ref|), computed in float64."""
    a = a.detach().double().cpu()
    ref = ref.detach().double().cpu()
    if ref.numel() == 0:
        return 0.0
    scale = ref.abs().max().item()
    if scale == 0:
        return a.abs().max().item()
    l2 = ((a - ref).norm() / ref.norm().clamp_min(1e-300)).item()
    mx = ((a - ref).abs().max() / scale).item()
    return max(l2, mx)


def out_size(dim, transposed, in_size, k, s, p, d, op):
    if transposed:
        return [(in_size[i] - 1) * s[i] - 2 * p[i] + d[i] * (k[i] - 1) + 1 + op[i] for i in range(dim)]
    return [(in_size[i] + 2 * p[i] - (d[i] * (k[i] - 1) + 1)) // s[i] + 1 for i in range(dim)]


def make_case(dim, transposed=False, batch=2, cin=4, cout=6, groups=1, og=1, mg=1, deformable=True,
              modulated=True, bias=True, kernel=None, stride=None, padding=None, dilation=None, out_pad=None,
              in_size=None, dtype=torch.float64, seed=0, offset_scale=2.0):
    """Random problem like the reference's DeformConvTestArgs (tests/utils/deform_conv_test_args.py:19-80):
    returns dict of CPU tensors + params."""
    g = torch.Generator().manual_seed(seed)
    kernel = kernel or [2, 3, 2][:dim]
    stride = stride or [1, 2, 1][:dim]
    padding = padding or [0, 1, 1][:dim]
    dilation = dilation or [1, 2, 1][:dim]
    out_pad = out_pad or [0, 1, 0][:dim] if transposed else [0] * dim
    in_size = in_size or [5, 6, 7][:dim]
    o = out_size(dim, transposed, in_size, kernel, stride, padding, dilation, out_pad)
    grid = in_size if transposed else o
    kn = 1
    for k in kernel:
        kn *= k
    x = torch.rand(batch, cin, *in_size, generator=g, dtype=torch.float64)
    if transposed:
        w = torch.rand(cin, cout // groups, *kernel, generator=g, dtype=torch.float64)
    else:
        w = torch.rand(cout, cin // groups, *kernel, generator=g, dtype=torch.float64)
    off = (torch.rand(batch, og * dim * kn, *grid, generator=g, dtype=torch.float64) - 0.5) * 2 * offset_scale \
        if deformable else None
    msk = torch.rand(batch, mg * kn, *grid, generator=g, dtype=torch.float64) if modulated else None
    b = torch.rand(cout, generator=g, dtype=torch.float64) if bias else None
    cast = (lambda t: None if t is None else t.to(dtype))
    return dict(dim=dim, transposed=transposed, input=cast(x), weight=cast(w), offset=cast(off), mask=cast(msk),
                bias=cast(b), stride=stride, padding=padding, dilation=dilation, output_padding=out_pad,
                groups=groups, out_shape=[batch, cout] + o)


def position_type(dtype):
    """The float type in which the kernels form a sampling position `base + offset` for inputs of
    `dtype`: the reference's own arithmetic for float32 and float16 (an integer base plus a scalar_t
    offset, one rounding to scalar_t: cpu/deform_conv2d_common_kernels.cpp:407-411,
    cuda/deform_conv2d_common_kernels.cu:170-178); float32 for bfloat16, which the reference lacks;
    None for float64 (the oracle's own precision)."""
    return {torch.float32: torch.float32, torch.float16: torch.float16, torch.bfloat16: torch.float32}.get(dtype)


def rounded_position_offsets(case, offset, ptype):
    """Offsets (float64) that put the float64 oracle's sampling positions where `ptype` arithmetic
    puts them: base + offset rounded once to `ptype`, base = p * stride - padding + tap * dilation on
    each axis of the column grid. The gradient reported for an offset is the one at that position.
    Where the exact position lies within half a unit in the last place of an integer, the rounded
    one is that integer: the sample then takes the other cell, and the offset gradient the other
    one-sided derivative, as the reference's float path does."""
    dim = case["dim"]
    ks = list(case["weight"].shape[2:])
    grid = list(offset.shape[2:])
    B, ch = offset.shape[:2]
    kn = 1
    for k in ks:
        kn *= k
    og = ch // (dim * kn)
    taps = torch.tensor(list(itertools.product(*[range(k) for k in ks])))   # (kn, dim)
    pos = offset.double().reshape(B, og, kn, dim, *grid).clone()
    for a in range(dim):
        shape = [1] * dim
        shape[a] = grid[a]
        p = torch.arange(grid[a], dtype=torch.float64).reshape(shape)
        base = p * case["stride"][a] - case["padding"][a] + \
            taps[:, a].double().reshape([kn] + [1] * dim) * case["dilation"][a]   # (kn, *grid)
        exact = pos[:, :, :, a] + base
        pos[:, :, :, a] = exact.to(ptype).double() - base
    return pos.reshape(offset.shape)


def oracle_offsets(case, offset, dtype):
    """The offsets to hand the float64 oracle for a run of the kernels in `dtype` (see
    rounded_position_offsets); float64 offsets unchanged."""
    ptype = position_type(dtype)
    if offset is None or ptype is None:
        return offset
    return rounded_position_offsets(case, offset, ptype)


class OracleDeformConv(torch.autograd.Function):
    """The float64 oracle as an autograd function on CPU tensors: a reference for compositions
    (generator convolutions, mask activations) whose other parts torch differentiates in float64."""

    @staticmethod
    def forward(ctx, x, w, o, m, b, dim, params):
        from oracle import oracle
        ctx.save_for_backward(x, w, o, m, b)
        ctx.dim, ctx.params = dim, params
        return oracle.forward(dim, x, w, o, m, b, **params)

    @staticmethod
    def backward(ctx, g):
        from oracle import oracle
        x, w, o, m, b = ctx.saved_tensors
        grads = oracle.backward(ctx.dim, g.contiguous(), x, w, o, m, b, **ctx.params)
        return tuple(grads) + (None, None)


def oracle_conv(dim, x, w, o, m, b, stride, padding, dilation, groups, transposed=False, output_padding=0):
    """deform_conv{dim}d / deform_conv_transpose{dim}d through the float64 oracle, differentiable"""
    params = dict(stride=stride, padding=padding, dilation=dilation, groups=groups, transposed=transposed,
                  output_padding=output_padding)
    return OracleDeformConv.apply(x, w, o, m, b, dim, params)


def mask_activation_f64(logits, activation, kernel_numel, scale=2.0):
    """the packed modules' mask activations in float64 torch ops: 1 = scale * sigmoid, 2 = softmax over the
    kernel taps of each mask group (tvdcn/ops/activations/mask_sigmoid.py:11-21, mask_softmax.py:19-126)"""
    if activation == 1:
        return scale * torch.sigmoid(logits)
    B, ch = logits.shape[:2]
    v = logits.reshape(B, ch // kernel_numel, kernel_numel, -1)
    return torch.softmax(v, dim=2).reshape(logits.shape)
