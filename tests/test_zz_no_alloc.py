"""The allocation-free forward (tvdcn_deform_conv_forward_noalloc) through the C ABI.

Checked against the workspace entry point (tvdcn_deform_conv_forward, same kernels: the same
numbers) and against the float64 oracle (float32 forward 1e-5, bfloat16 1e-2), on calls in a
row whose later problems are smaller, so that the library's scratch array holds the previous
call's data when the next one starts; the workspace entry point gets a workspace filled with
NaN bytes. A problem above the scratch size is refused with a message naming both sizes.
"""
import ctypes

import pytest
import torch

import tvdcn
from helpers import Desc, make_case, rel_err
from test_gpu_parity import run_oracle

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
DTYPE = {torch.float32: 0, torch.float64: 1, torch.float16: 2, torch.bfloat16: 3}
SCRATCH_BYTES = 64 << 20


def _lib():
    lib = ctypes.CDLL(tvdcn.extension.HIP_LIB_PATH)
    vp = ctypes.c_void_p
    lib.tvdcn_deform_conv_forward.argtypes = [ctypes.POINTER(Desc)] + [vp] * 7 + [ctypes.c_size_t, vp]
    lib.tvdcn_deform_conv_forward_noalloc.argtypes = [ctypes.POINTER(Desc)] + [vp] * 6 + [vp]
    lib.tvdcn_deform_conv_forward_workspace_size.argtypes = [ctypes.POINTER(Desc)]
    lib.tvdcn_deform_conv_forward_workspace_size.restype = ctypes.c_size_t
    lib.tvdcn_last_error.restype = ctypes.c_char_p
    return lib


def _desc(case, dtype):
    dim, tr = case["dim"], case["transposed"]
    x, w = case["input"], case["weight"]
    kn = 1
    for k in w.shape[2:]:
        kn *= k
    d = Desc(dim=dim, transposed=int(tr), dtype=DTYPE[dtype], flags=0, batch=x.shape[0], in_channels=x.shape[1],
             out_channels=w.shape[1] * case["groups"] if tr else w.shape[0], groups=case["groups"],
             offset_groups=case["offset"].shape[1] // (dim * kn) if case["offset"] is not None else 0,
             mask_groups=case["mask"].shape[1] // kn if case["mask"] is not None else 0)
    for i in range(3):
        d.in_size[i] = d.kernel[i] = d.stride[i] = d.dilation[i] = 1
    for i in range(dim):
        d.in_size[i], d.kernel[i] = x.shape[2 + i], w.shape[2 + i]
        d.stride[i], d.padding[i], d.dilation[i] = case["stride"][i], case["padding"][i], case["dilation"][i]
        d.output_padding[i] = case["output_padding"][i] if tr else 0
    return d


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _run(lib, case, dtype, noalloc):
    ts = [case[n].to(DEV, dtype).contiguous() if case[n] is not None else None
          for n in ("input", "weight", "offset", "mask", "bias")]
    d = _desc(case, dtype)
    out = torch.full(case["out_shape"], float("nan"), device=DEV, dtype=dtype)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    if noalloc:
        st = lib.tvdcn_deform_conv_forward_noalloc(ctypes.byref(d), *map(_ptr, ts), _ptr(out), stream)
    else:
        nbytes = lib.tvdcn_deform_conv_forward_workspace_size(ctypes.byref(d))
        ws = torch.full((max(nbytes, 16) // 4 + 1,), float("nan"), device=DEV, dtype=torch.float32)
        st = lib.tvdcn_deform_conv_forward(ctypes.byref(d), *map(_ptr, ts), _ptr(out), _ptr(ws),
                                           ctypes.c_size_t(nbytes), stream)
    assert st == 0, lib.tvdcn_last_error()
    torch.cuda.synchronize()
    return out


CASES = [
    # (dim, transposed, dtype, batch, channels, spatial): each call smaller than the one before
    (2, False, torch.float32, 4, 64, [24, 20]),
    (2, False, torch.float32, 2, 32, [12, 10]),
    (1, False, torch.float32, 3, 48, [40]),
    (3, False, torch.float32, 1, 16, [5, 6, 7]),
    (2, True, torch.float32, 2, 32, [9, 8]),
    (2, False, torch.bfloat16, 1, 32, [10, 9]),
]


def test_noalloc_forward_matches_workspace_forward():
    lib = _lib()
    for i, (dim, tr, dtype, b, ch, size) in enumerate(CASES):
        print(f"noalloc case {i}: dim {dim} transposed {tr} {dtype} batch {b} channels {ch} size {size}",
              flush=True)
        case = make_case(dim, tr, batch=b, cin=ch, cout=ch, kernel=[3] * dim, stride=[1] * dim,
                         padding=[1] * dim, dilation=[1] * dim, out_pad=[0] * dim, in_size=size, seed=900 + i,
                         og=2, mg=2)
        y_ws = _run(lib, case, dtype, noalloc=False)
        y_na = _run(lib, case, dtype, noalloc=True)
        assert not torch.isnan(y_na).any()
        assert rel_err(y_na, y_ws) < (1e-6 if dtype == torch.float32 else 1e-2)
        ref, _ = run_oracle(case, torch.zeros(case["out_shape"], dtype=torch.float64), dtype)
        assert rel_err(y_na, ref) < (1e-5 if dtype == torch.float32 else 1e-2)


def test_noalloc_forward_refuses_problems_above_the_scratch():
    lib = _lib()
    d = Desc(dim=1, transposed=0, dtype=0, flags=0, batch=16, in_channels=512, out_channels=512, groups=1,
             offset_groups=4, mask_groups=4)
    for i in range(3):
        d.in_size[i] = d.kernel[i] = d.stride[i] = d.dilation[i] = 1
    d.in_size[0], d.kernel[0], d.padding[0] = 4096, 5, 2
    assert lib.tvdcn_deform_conv_forward_workspace_size(ctypes.byref(d)) > SCRATCH_BYTES
    st = lib.tvdcn_deform_conv_forward_noalloc(ctypes.byref(d), *([ctypes.c_void_p(16)] * 6), None)
    assert st == 2
    msg = lib.tvdcn_last_error().decode()
    assert "scratch" in msg and str(SCRATCH_BYTES) in msg
