"""Images whose own tensors exceed the kernels' 32-bit indexing (the C ABI refuses them with
TVDCN_STATUS_NOT_SUPPORTED; the reference indexes them in 64 bits, ops/utils/dispatch.h:52-60): the
operator layer runs the problem as sub-problems over channel ranges (a conv group's range of sampled
channels times a range of GEMM-side channels) and sums the partial results in float32.

The limit is forced below one image's tensors with tvdcn_set_max_block_elements on problems the
float64 oracle checks: ranges on both channel sides, conv groups, offset / mask groups inside one range
and spanning several, conv and transposed, ranks 1-3, float32 / float16, and the fused mask
activations. Each test first asserts that the C ABI refuses the whole problem at that limit, so the
split path is the one that ran."""
import ctypes

import pytest
import torch

import tvdcn
from helpers import Desc, make_case, rel_err
from test_gpu_parity import TOL, check, run_oracle

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
NOT_SUPPORTED = 3


def _lib():
    lib = ctypes.CDLL(tvdcn.extension.HIP_LIB_PATH)
    lib.tvdcn_set_max_block_elements.argtypes = [ctypes.c_int64]
    lib.tvdcn_set_max_block_elements.restype = ctypes.c_int
    lib.tvdcn_conv_batch_block.argtypes = [ctypes.POINTER(Desc), ctypes.POINTER(ctypes.c_int64)]
    lib.tvdcn_conv_batch_block.restype = ctypes.c_int
    return lib


def _desc(case):
    d = Desc()
    dim = case["dim"]
    x, w = case["input"], case["weight"]
    d.dim, d.transposed, d.dtype, d.flags = dim, int(case["transposed"]), 0, 0
    d.batch, d.in_channels = x.shape[0], x.shape[1]
    d.out_channels = case["out_shape"][1]
    d.groups = case["groups"]
    kn = w[0, 0].numel()
    d.offset_groups = case["offset"].shape[1] // (dim * kn) if case["offset"] is not None else 0
    d.mask_groups = case["mask"].shape[1] // kn if case["mask"] is not None else 0
    for i in range(3):
        d.in_size[i] = d.kernel[i] = d.stride[i] = d.dilation[i] = 1
        d.padding[i] = d.output_padding[i] = 0
    for i in range(dim):
        d.in_size[i] = x.shape[2 + i]
        d.kernel[i] = w.shape[2 + i]
        d.stride[i] = case["stride"][i]
        d.padding[i] = case["padding"][i]
        d.dilation[i] = case["dilation"][i]
        d.output_padding[i] = case["output_padding"][i]
    return d


def _limit(case, og, mg):
    """A block limit under one image's input or output but above one offset / mask group's tensors
    (the smallest sub-problem still takes a whole offset group)."""
    x, out = case["input"], case["out_shape"]
    per_image = max(x[0].numel(), torch.Size(out[1:]).numel())
    floor = 1
    if case["offset"] is not None:
        floor = max(floor, case["offset"][0].numel() // og)
    if case["mask"] is not None:
        floor = max(floor, case["mask"][0].numel() // mg)
    return max(floor, per_image // 3)


CASES = [
    # dim, transposed, cin, cout, groups, og, mg, in_size
    (2, False, 32, 48, 1, 1, 1, [16, 16]),
    (2, False, 32, 48, 2, 2, 1, [16, 14]),
    (2, False, 64, 32, 1, 4, 2, [12, 12]),   # ranges inside one offset group
    (2, True, 48, 32, 1, 2, 2, [9, 8]),
    (2, True, 32, 32, 2, 1, 2, [10, 9]),
    (1, False, 32, 48, 1, 4, 4, [90]),
    # (3D: 27 taps make one offset group's tensor the largest but for wide channel counts)
    (3, False, 64, 96, 1, 1, 1, [4, 6, 5]),
    (3, True, 128, 96, 1, 1, 1, [3, 4, 4]),
]


def _case(dim, transposed, cin, cout, groups, og, mg, in_size, seed):
    return make_case(dim, transposed, batch=2, cin=cin, cout=cout, groups=groups, og=og, mg=mg,
                     kernel=[3] * dim, stride=[1] * dim, padding=[1] * dim, dilation=[1] * dim,
                     in_size=in_size, out_pad=[0] * dim, seed=seed)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("dim,transposed,cin,cout,groups,og,mg,in_size", CASES)
def test_channel_split_matches_oracle(dim, transposed, cin, cout, groups, og, mg, in_size, dtype):
    case = _case(dim, transposed, cin, cout, groups, og, mg, in_size, seed=900 + 10 * dim + int(transposed))
    lib = _lib()
    limit = _limit(case, og, mg)
    print(f"dim {dim} transposed {transposed} C {cin}->{cout} groups {groups} og {og} mg {mg} {dtype} "
          f"limit {limit}", flush=True)
    assert lib.tvdcn_set_max_block_elements(limit) == 0
    try:
        images = ctypes.c_int64()
        assert lib.tvdcn_conv_batch_block(ctypes.byref(_desc(case)), ctypes.byref(images)) == NOT_SUPPORTED
        check(case, dtype)
    finally:
        assert lib.tvdcn_set_max_block_elements(2 ** 31 - 1) == 0


@pytest.mark.parametrize("activation", ["sigmoid", "softmax"])
def test_channel_split_with_fused_mask_activation(activation):
    """The fused mask activations on split problems: the logit gradient is linear in the mask
    gradient, so the sub-problems' logit gradients sum to the whole problem's (against the same
    problem run whole, at the default limit)."""
    case = _case(2, False, 32, 48, 1, 2, 2, [14, 12], seed=950)
    x, w, o, m, b = (case[n].to(DEV, torch.float32) for n in ("input", "weight", "offset", "mask", "bias"))
    logits = (m * 4 - 2).contiguous()
    act = 1 if activation == "sigmoid" else 2
    # stride, padding, output_padding, dilation, groups, transposed, activation, mask_scale
    params = ([1, 1], [1, 1], [0, 0], [1, 1], 1, False, act, 2.0)
    op = torch.ops.tvdcn.deform_conv_mask_activation
    bwd = torch.ops.tvdcn._deform_conv_mask_activation_backward
    y_ref = op(x, w, o, logits, b, *params)
    gy = torch.randn(y_ref.shape, device=DEV, generator=torch.Generator(device=DEV).manual_seed(3))
    g_ref = bwd(gy, x, w, o, logits, b, *params)
    lib = _lib()
    limit = _limit(case, 2, 2)
    assert lib.tvdcn_set_max_block_elements(limit) == 0
    try:
        images = ctypes.c_int64()
        assert lib.tvdcn_conv_batch_block(ctypes.byref(_desc(case)), ctypes.byref(images)) == NOT_SUPPORTED
        y = op(x, w, o, logits, b, *params)
        g = bwd(gy, x, w, o, logits, b, *params)
        torch.cuda.synchronize()
    finally:
        assert lib.tvdcn_set_max_block_elements(2 ** 31 - 1) == 0
    tf, tb = TOL[torch.float32]
    assert rel_err(y, y_ref) < tf
    for name, a, r in zip(("input", "weight", "offset", "mask", "bias"), g, g_ref):
        assert rel_err(a, r) < tb, name


def test_channel_split_channels_last_input():
    """A channels-last input on the split path: its gradient comes back channels-last, with the
    oracle's numbers."""
    case = _case(2, False, 32, 48, 1, 1, 1, [16, 16], seed=960)
    names = ("input", "weight", "offset", "mask", "bias")
    lib = _lib()
    assert lib.tvdcn_set_max_block_elements(_limit(case, 1, 1)) == 0
    try:
        ts = [case[n].to(DEV, torch.float32) for n in names]
        ts[0] = ts[0].contiguous(memory_format=torch.channels_last)
        ts = [t.requires_grad_(True) for t in ts]
        y = tvdcn.deform_conv2d(*ts, stride=1, padding=1, dilation=1)
        gout = torch.rand(y.shape, generator=torch.Generator().manual_seed(7), dtype=torch.float64)
        y.backward(gout.to(DEV, torch.float32))
        torch.cuda.synchronize()
    finally:
        assert lib.tvdcn_set_max_block_elements(2 ** 31 - 1) == 0
    assert ts[0].grad.is_contiguous(memory_format=torch.channels_last)
    ref_out, ref_grads = run_oracle(case, gout, torch.float32)
    tf, tb = TOL[torch.float32]
    assert rel_err(y, ref_out) < tf
    for n, t, r in zip(names, ts, ref_grads):
        assert rel_err(t.grad, r) < tb, n


def test_image_above_2_31_elements():
    """One (1, 512, 2048, 2048) float32 image: 2^31 input elements, run as channel-range sub-problems at
    the default limit. Checked against the float64 oracle on a crop: with offsets below one pixel, an
    8 x 8 block of outputs depends only on the 14 x 14 input patch around it, so the oracle on that patch
    (no padding; the block's offsets moved to the float32-rounded positions of the whole image, which
    sit near 1000 where float32 steps are 2^-14) gives the block's outputs; with grad_out zero outside the
    block, the input gradient (zero outside the patch), the block's offset / mask gradients and the
    weight / bias gradients must match the oracle's on the patch too."""
    from oracle import oracle
    g = torch.Generator(device=DEV).manual_seed(970)
    C, H, W, K = 512, 2048, 2048, 3
    x = torch.randn(1, C, H, W, device=DEV, generator=g)
    assert x.numel() >= 2 ** 31
    w = torch.randn(C, C, K, K, device=DEV, generator=g) * (2.0 / (K * K * C)) ** 0.5
    off = (torch.rand(1, 2 * K * K, H, W, device=DEV, generator=g) - 0.5) * 1.8
    msk = torch.rand(1, K * K, H, W, device=DEV, generator=g)
    bias = torch.randn(C, device=DEV, generator=g)
    r0, c0, n, h = 1000, 1500, 8, 3
    rows, cols = slice(r0, r0 + n), slice(c0, c0 + n)
    prow, pcol = slice(r0 - h, r0 + n + h), slice(c0 - h, c0 + n + h)
    blk = slice(h - 1, h - 1 + n)   # the block inside the patch's 12 x 12 outputs
    # the patch's oracle operands: the block's offsets at the whole image's float32 positions
    off_blk = off[0, :, rows, cols].cpu()
    off_model = torch.zeros(2 * K * K, n, n, dtype=torch.float64)
    ys = torch.arange(r0, r0 + n).view(n, 1).expand(n, n)
    xs = torch.arange(c0, c0 + n).view(1, n).expand(n, n)
    for t in range(K * K):
        by, bx = (ys - 1 + t // K).float(), (xs - 1 + t % K).float()
        off_model[2 * t] = (by + off_blk[2 * t]).double() - by.double()
        off_model[2 * t + 1] = (bx + off_blk[2 * t + 1]).double() - bx.double()
    pn = n + 2 * h - 2
    o_p = torch.zeros(1, 2 * K * K, pn, pn, dtype=torch.float64)
    m_p = torch.zeros(1, K * K, pn, pn, dtype=torch.float64)
    o_p[0, :, blk, blk] = off_model
    m_p[0, :, blk, blk] = msk[0, :, rows, cols].double().cpu()
    x_p, w64, b64 = x[:, :, prow, pcol].double().cpu(), w.double().cpu(), bias.double().cpu()
    kw = dict(stride=[1, 1], padding=[0, 0], dilation=[1, 1], groups=1)
    print("forward over the whole image", flush=True)
    y = torch.ops.tvdcn.deform_conv2d(x, w, off, msk, bias, [1, 1], [1, 1], [1, 1], 1)
    y_blk = y[:, :, rows, cols].double().cpu()
    del y
    ref = oracle.forward(2, x_p, w64, o_p, m_p, b64, **kw)
    assert rel_err(y_blk, ref[:, :, blk, blk]) < 1e-5
    gy = torch.zeros(1, C, H, W, device=DEV)
    gy[:, :, rows, cols] = torch.randn(1, C, n, n, device=DEV, generator=g)
    g_p = torch.zeros(1, C, pn, pn, dtype=torch.float64)
    g_p[:, :, blk, blk] = gy[:, :, rows, cols].double().cpu()
    print("backward over the whole image", flush=True)
    gx, gw, goff, gmsk, gb = torch.ops.tvdcn._deform_conv2d_backward(gy, x, w, off, msk, bias, [1, 1], [1, 1],
                                                                      [1, 1], 1)
    torch.cuda.synchronize()
    del gy
    gx_p = gx[:, :, prow, pcol].double().cpu()
    gx[:, :, prow, pcol] = 0.0
    assert float(gx.abs().max()) == 0.0
    del gx
    r_gx, r_gw, r_goff, r_gmsk, r_gb = oracle.backward(2, g_p, x_p, w64, o_p, m_p, b64, **kw)
    assert rel_err(gx_p, r_gx) < 1e-4
    assert rel_err(goff[0, :, rows, cols].double().cpu(), r_goff[0, :, blk, blk]) < 1e-4
    assert rel_err(gmsk[0, :, rows, cols].double().cpu(), r_gmsk[0, :, blk, blk]) < 1e-4
    assert rel_err(gw.double().cpu(), r_gw) < 1e-4
    assert rel_err(gb.double().cpu(), r_gb) < 1e-4
