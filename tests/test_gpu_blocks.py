"""Batch blocks: the kernels index in 32 bits, so the C ABI runs a batch whose tensors exceed
2^31 - 1 elements in blocks of images and accumulates the weight gradient over them (the
reference's n_parallel_imgs blocking, cuda/deform_conv2d_kernel.cpp:149).

* forced small blocks (tvdcn_set_max_block_elements) on modest problems, against the float64
  oracle: full blocks, a remainder block, conv and transposed, ranks 1-3, float32 / float16;
* one problem above 2^31 elements (B=128, C=256, 256x256 float32), against size-independent
  properties: every image's output and input gradient equal those of the image run alone, and
  the weight / bias gradients equal the sum over the two halves of the batch run separately.
"""
import ctypes

import pytest
import torch

import tvdcn
from helpers import make_case, rel_err
from test_gpu_parity import check, run_oracle

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _lib():
    lib = ctypes.CDLL(tvdcn.extension.HIP_LIB_PATH)
    lib.tvdcn_set_max_block_elements.argtypes = [ctypes.c_int64]
    lib.tvdcn_set_max_block_elements.restype = ctypes.c_int
    return lib


def _per_image(case):
    x, w, o, m = case["input"], case["weight"], case["offset"], case["mask"]
    out = case["out_shape"]
    sizes = [x[0].numel(), torch.Size(out[1:]).numel()]
    sizes += [t[0].numel() for t in (o, m) if t is not None]
    return max(sizes)


@pytest.mark.parametrize("images", [1, 2])
@pytest.mark.parametrize("dim,transposed,dtype", [
    (2, False, torch.float32), (2, True, torch.float32), (1, False, torch.float32), (3, False, torch.float32),
    (2, False, torch.float16)])
def test_forced_batch_blocks_match_oracle(dim, transposed, dtype, images):
    in_size = {1: [60], 2: [18, 16], 3: [5, 8, 7]}[dim]
    case = make_case(dim, transposed, batch=5, cin=32, cout=48, kernel=[3] * dim, stride=[1] * dim,
                     padding=[1] * dim, dilation=[1] * dim, in_size=in_size, out_pad=[0] * dim, seed=800 + dim)
    lib = _lib()
    print(f"blocks of {images} image(s): dim {dim} transposed {transposed} {dtype}", flush=True)
    assert lib.tvdcn_set_max_block_elements(images * _per_image(case)) == 0
    try:
        check(case, dtype)
    finally:
        assert lib.tvdcn_set_max_block_elements(2 ** 31 - 1) == 0


def test_problem_above_2_31_elements():
    """B=128, C=256, 256x256 float32: 2^31 input elements, run in two blocks (127 + 1 images)."""
    g = torch.Generator(device=DEV).manual_seed(810)
    B, C, H = 128, 256, 256
    x = torch.randn(B, C, H, H, device=DEV, generator=g)
    assert x.numel() >= 2 ** 31
    w = torch.randn(C, C, 3, 3, device=DEV, generator=g) * (2.0 / (9 * C)) ** 0.5
    off = torch.randn(B, 18, H, H, device=DEV, generator=g)
    msk = torch.rand(B, 9, H, H, device=DEV, generator=g)
    bias = torch.randn(C, device=DEV, generator=g)
    print("forward over the full batch", flush=True)
    y = tvdcn.deform_conv2d(x, w, off, msk, bias, padding=1)
    torch.cuda.synchronize()
    for b in (0, 126, 127):
        yb = tvdcn.deform_conv2d(x[b:b + 1], w, off[b:b + 1], msk[b:b + 1], bias, padding=1)
        assert rel_err(y[b:b + 1], yb) < 1e-6, b
    gy = torch.randn(y.shape, device=DEV, generator=g)
    del y
    print("backward over the full batch", flush=True)
    gx, gw, goff, gmsk, gb = torch.ops.tvdcn._deform_conv2d_backward(gy, x, w, off, msk, bias, [1, 1], [1, 1],
                                                                      [1, 1], 1)
    torch.cuda.synchronize()
    for b in (0, 127):
        r = torch.ops.tvdcn._deform_conv2d_backward(gy[b:b + 1], x[b:b + 1], w, off[b:b + 1], msk[b:b + 1], bias,
                                                    [1, 1], [1, 1], [1, 1], 1)
        for name, full, one in zip(("input", "offset", "mask"), (gx, goff, gmsk), (r[0], r[2], r[3])):
            assert rel_err(full[b:b + 1], one) < 1e-5, (b, name)
    del gx, goff, gmsk
    print("backward over the two halves", flush=True)
    parts = []
    for lo, hi in ((0, 64), (64, 128)):
        r = torch.ops.tvdcn._deform_conv2d_backward(gy[lo:hi], x[lo:hi], w, off[lo:hi], msk[lo:hi], bias, [1, 1],
                                                    [1, 1], [1, 1], 1)
        parts.append((r[1], r[4]))
        del r
    torch.cuda.synchronize()
    # sums over 8.4M pixels per weight element in two float32 orders: the backward's 1e-4
    assert rel_err(gw, parts[0][0] + parts[1][0]) < 1e-4
    assert rel_err(gb, parts[0][1] + parts[1][1]) < 1e-4


@pytest.mark.parametrize("images", [1, 3, 5])
@pytest.mark.parametrize("transposed,dtype,channels_last", [
    (False, torch.float32, False), (True, torch.float32, False), (False, torch.float16, False),
    (True, torch.bfloat16, False), (False, torch.float32, True)])
def test_forced_batch_blocks_with_unaligned_image_sizes(transposed, dtype, channels_last, images):
    """C = 3 on a 7 x 7 grid: no batch-sized tensor's per-image bytes are a multiple of 16 (float32
    input 588 B), so blocks of 1 or 3 images put later blocks' pointers off 16-byte boundaries (2- or
    4-byte aligned), which every kernel accepts; blocks of 5 images round down to 4, a multiple of 16
    bytes for every tensor. Batch 7: full blocks and a remainder, against the float64 oracle (float32
    channels-last: the input sampled in place at the block's offset)."""
    case = make_case(2, transposed, batch=7, cin=3, cout=5, kernel=[3, 3], stride=[1, 1], padding=[1, 1],
                     dilation=[1, 1], in_size=[7, 7], out_pad=[0, 0], seed=830 + images)
    lib = _lib()
    print(f"blocks of {images} image(s): transposed {transposed} {dtype} channels_last {channels_last}", flush=True)
    assert lib.tvdcn_set_max_block_elements(images * _per_image(case)) == 0
    try:
        if not channels_last:
            check(case, dtype)
            return
        names = ("input", "weight", "offset", "mask", "bias")
        ts = [case[n].to(DEV, dtype) for n in names]
        ts[0] = ts[0].contiguous(memory_format=torch.channels_last)
        ts = [t.requires_grad_(True) for t in ts]
        y = tvdcn.deform_conv2d(*ts, stride=1, padding=1, dilation=1)
        gout = torch.rand(y.shape, generator=torch.Generator().manual_seed(7), dtype=torch.float64)
        y.backward(gout.to(DEV, dtype))
        torch.cuda.synchronize()
        assert ts[0].grad.is_contiguous(memory_format=torch.channels_last)
        ref_out, ref_grads = run_oracle(case, gout, dtype)
        assert rel_err(y, ref_out) < 1e-5
        for n, t, r in zip(names, ts, ref_grads):
            assert rel_err(t.grad, r) < 1e-4, n
    finally:
        assert lib.tvdcn_set_max_block_elements(2 ** 31 - 1) == 0
