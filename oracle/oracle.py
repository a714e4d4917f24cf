"""Python access to the CPU checkers. TEST INFRASTRUCTURE ONLY.

Two checkers live under oracle/:

* ``liboracle.so`` -- this repo's float64 C restatement of tvdcn's CPU algorithm
  (``deform_oracle.c``); wrapped by :func:`forward`, :func:`backward`,
  :func:`mask_softmax_forward`, :func:`mask_softmax_backward`.
* ``_ref/libtvdcn_ref.so`` -- the reference's own CPU path compiled from its
  sources by ``oracle/Makefile``. It registers the ``torch.ops.tvdcn`` namespace,
  as the product library does, so :func:`run_reference` runs it in a child
  process (``oracle/ref_child.py``).

Only tests/, ``__graft_entry__.smoke()`` and bench.py's cpu_baseline leg import
this module. Product code (tvdcn_amd/) never does.
"""
import ctypes
import os
import subprocess
import sys
import tempfile

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_LIB = os.path.join(_HERE, "_build", "liboracle.so")
REF_LIB = os.path.join(_HERE, "_ref", "libtvdcn_ref.so")

_lib = None


class _Desc(ctypes.Structure):
    _fields_ = [
        ("dim", ctypes.c_int32),
        ("transposed", ctypes.c_int32),
        ("batch", ctypes.c_int64),
        ("in_channels", ctypes.c_int64),
        ("out_channels", ctypes.c_int64),
        ("groups", ctypes.c_int64),
        ("offset_groups", ctypes.c_int64),
        ("mask_groups", ctypes.c_int64),
        ("in_size", ctypes.c_int64 * 3),
        ("kernel", ctypes.c_int64 * 3),
        ("stride", ctypes.c_int64 * 3),
        ("padding", ctypes.c_int64 * 3),
        ("dilation", ctypes.c_int64 * 3),
        ("output_padding", ctypes.c_int64 * 3),
    ]


def build(force=False):
    """Compile liboracle.so (and, when /root/reference exists, the reference CPU build)."""
    if force or not os.path.exists(ORACLE_LIB):
        subprocess.check_call(["make", "-s", "-C", _HERE, "oracle"])


def build_reference():
    """Compile oracle/_ref from the reference sources; a no-op without /root/reference."""
    if os.path.isdir("/root/reference/tvdcn/csrc"):
        subprocess.check_call(["make", "-s", "-j8", "-C", _HERE, "ref"])
    return os.path.exists(REF_LIB)


def _load():
    global _lib
    if _lib is None:
        build()
        lib = ctypes.CDLL(ORACLE_LIB)
        dp = ctypes.POINTER(ctypes.c_double)
        lib.oracle_deform_conv_forward.argtypes = [ctypes.POINTER(_Desc)] + [dp] * 6
        lib.oracle_deform_conv_backward.argtypes = [ctypes.POINTER(_Desc)] + [dp] * 10
        lib.oracle_mask_softmax_forward.argtypes = [ctypes.c_int64] * 4 + [dp] * 2
        lib.oracle_mask_softmax_backward.argtypes = [ctypes.c_int64] * 4 + [dp] * 3
        lib.oracle_output_size.argtypes = [ctypes.POINTER(_Desc), ctypes.c_int64 * 3]
        lib.oracle_output_size.restype = ctypes.c_int64
        _lib = lib
    return _lib


def have_reference():
    """True when the reference's CPU build (oracle/_ref) exists."""
    return os.path.exists(REF_LIB)


def run_reference(requests, env=None):
    """Runs requests (see oracle/ref_child.py) against the reference build in a child process;
    returns the list of results. CPU tensors only."""
    if not have_reference():
        raise RuntimeError(f"{REF_LIB} is not built")
    root = os.path.dirname(_HERE)
    with tempfile.TemporaryDirectory() as tmp:
        src, dst = os.path.join(tmp, "req.pt"), os.path.join(tmp, "res.pt")
        torch.save(list(requests), src)
        proc = subprocess.run([sys.executable, "-m", "oracle.ref_child", src, dst], cwd=root, env=env,
                              stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
        if proc.returncode != 0:
            raise RuntimeError(f"reference child process failed ({proc.returncode}):\n{proc.stdout}")
        return torch.load(dst, weights_only=True)


def _ptr(t):
    if t is None:
        return None
    return ctypes.cast(t.data_ptr(), ctypes.POINTER(ctypes.c_double))


def _f64(t):
    if t is None:
        return None
    return t.detach().to(device="cpu", dtype=torch.float64).contiguous()


def _tuple(v, dim):
    if isinstance(v, int):
        return (v,) * dim
    v = tuple(int(x) for x in v)
    return v if len(v) == dim else v * dim


def make_desc(dim, transposed, input, weight, offset, mask, stride, padding, dilation, groups,
              output_padding=0):
    d = _Desc()
    d.dim = dim
    d.transposed = int(bool(transposed))
    d.batch = input.shape[0]
    d.in_channels = input.shape[1]
    kernel = tuple(weight.shape[2:])
    kn = 1
    for k in kernel:
        kn *= k
    d.out_channels = weight.shape[1] * groups if transposed else weight.shape[0]
    d.groups = groups
    d.offset_groups = offset.shape[1] // (dim * kn) if offset is not None else 0
    d.mask_groups = mask.shape[1] // kn if mask is not None else 0
    for i, (s, k, st, p, dl, op) in enumerate(zip(
            input.shape[2:], kernel, _tuple(stride, dim), _tuple(padding, dim), _tuple(dilation, dim),
            _tuple(output_padding, dim))):
        d.in_size[i] = s
        d.kernel[i] = k
        d.stride[i] = st
        d.padding[i] = p
        d.dilation[i] = dl
        d.output_padding[i] = op
    return d


def output_shape(desc):
    sz = (ctypes.c_int64 * 3)()
    _load().oracle_output_size(ctypes.byref(desc), sz)
    return tuple(sz[i] for i in range(desc.dim))


def forward(dim, input, weight, offset=None, mask=None, bias=None, stride=1, padding=0, dilation=1,
            groups=1, transposed=False, output_padding=0):
    """float64 forward of deform_conv{dim}d / deform_conv_transpose{dim}d (batched inputs)."""
    lib = _load()
    x, w, o, m, b = (_f64(t) for t in (input, weight, offset, mask, bias))
    d = make_desc(dim, transposed, x, w, o, m, stride, padding, dilation, groups, output_padding)
    out = torch.empty((x.shape[0], d.out_channels) + output_shape(d), dtype=torch.float64)
    lib.oracle_deform_conv_forward(ctypes.byref(d), _ptr(x), _ptr(w), _ptr(o), _ptr(m), _ptr(b), _ptr(out))
    return out


def backward(dim, grad_out, input, weight, offset=None, mask=None, bias=None, stride=1, padding=0,
             dilation=1, groups=1, transposed=False, output_padding=0):
    """float64 (grad_input, grad_weight, grad_offset, grad_mask, grad_bias); None where absent."""
    lib = _load()
    g, x, w, o, m = (_f64(t) for t in (grad_out, input, weight, offset, mask))
    d = make_desc(dim, transposed, x, w, o, m, stride, padding, dilation, groups, output_padding)
    gx = torch.empty_like(x)
    gw = torch.empty_like(w)
    go = torch.empty_like(o) if o is not None else None
    gm = torch.empty_like(m) if m is not None else None
    gb = torch.empty(d.out_channels, dtype=torch.float64) if bias is not None else None
    lib.oracle_deform_conv_backward(ctypes.byref(d), _ptr(g), _ptr(x), _ptr(w), _ptr(o), _ptr(m),
                                    _ptr(gx), _ptr(gw), _ptr(go), _ptr(gm), _ptr(gb))
    return gx, gw, go, gm, gb


def mask_softmax_forward(mask, kernel_numel):
    lib = _load()
    x = _f64(mask)
    B, ch = x.shape[:2]
    S = x[0, 0].numel()
    groups = ch // kernel_numel
    y = torch.empty_like(x)
    lib.oracle_mask_softmax_forward(B, groups, kernel_numel, S, _ptr(x), _ptr(y))
    return y


def mask_softmax_backward(y, grad_y, kernel_numel):
    lib = _load()
    y64, g64 = _f64(y), _f64(grad_y)
    B, ch = y64.shape[:2]
    S = y64[0, 0].numel()
    groups = ch // kernel_numel
    gx = torch.empty_like(y64)
    lib.oracle_mask_softmax_backward(B, groups, kernel_numel, S, _ptr(y64), _ptr(g64), _ptr(gx))
    return gx
