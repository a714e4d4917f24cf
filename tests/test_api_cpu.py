"""CPU tests of the drop-in boundary and the host logic (no GPU compute).

* the C ABI library loads and exports every function declared in include/tvdcn_hip.h;
  its host-only entry points (output size, workspace and batch-block queries, argument checks) work;
* the C++ API of include/tvdcn_ops.h: the reference's exported symbols, and a C++ caller built
  against the header and linked with _C.so gets the Python API's results;
* the operator schemas match the reference's (names, argument order, defaults);
* shape inference and validation run on meta tensors, with the reference's error
  texts (checked side by side with the reference build when oracle/_ref exists);
* autograd and double-backward behaviour, on meta tensors;
* CPU tensors go to the CPU dispatch key (host kernels; tests/test_cpu_kernels.py checks their
  numbers), GPU tensors never do;
* the nn.Module wrappers and mask activations keep the reference's API and errors.
"""
import ctypes
import math
import os
import re

import pytest
import torch

import tvdcn
from tvdcn import extension
from oracle import oracle
from helpers import Desc

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "tvdcn_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tvdcn_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    return ctypes.CDLL(extension.HIP_LIB_PATH)


def test_native_library_loaded():
    assert tvdcn.has_ops()
    assert tvdcn.with_cuda()
    assert tvdcn.cuda_arch_list() == ["gfx950"]
    assert tvdcn.cuda_version() > 60000000


def test_operator_library_found_by_the_extension_finder():
    """The operator library is located as the reference locates its _C (tvdcn/extension.py:19-51): the
    import system's extension finder over the package directory, so _C + any of the interpreter's
    extension suffixes is taken; a name without a library raises ImportError."""
    import importlib.machinery
    path = extension._get_extension_path("_C")
    assert os.path.dirname(path) == os.path.dirname(extension.__file__)
    base = os.path.basename(path)
    assert base.startswith("_C") and base[2:] in importlib.machinery.EXTENSION_SUFFIXES
    with pytest.raises(ImportError):
        extension._get_extension_path("_no_such_library")


def test_c_abi_exports_every_declared_function(lib):
    names = declared_functions()
    assert len(names) >= 11
    for n in names:
        assert hasattr(lib, n), n


def cfg2_desc(**over):
    d = Desc(dim=2, transposed=0, dtype=0, batch=8, in_channels=256, out_channels=256, groups=1, offset_groups=1,
             mask_groups=1)
    for i in range(3):
        d.in_size[i], d.kernel[i], d.stride[i], d.padding[i], d.dilation[i], d.output_padding[i] = 64, 3, 1, 1, 1, 0
    for k, v in over.items():
        setattr(d, k, v)
    return d


def test_c_abi_host_queries(lib):
    lib.tvdcn_conv_output_size.restype = ctypes.c_int
    lib.tvdcn_deform_conv_forward_workspace_size.restype = ctypes.c_size_t
    lib.tvdcn_deform_conv_backward_workspace_size.restype = ctypes.c_size_t
    lib.tvdcn_last_error.restype = ctypes.c_char_p
    d = cfg2_desc()
    out = (ctypes.c_int64 * 3)()
    assert lib.tvdcn_conv_output_size(ctypes.byref(d), out) == 0
    assert list(out)[:2] == [64, 64]
    fw = lib.tvdcn_deform_conv_forward_workspace_size(ctypes.byref(d))
    bw = lib.tvdcn_deform_conv_backward_workspace_size(ctypes.byref(d))
    # forward: channels-last copy of the input (33.5 MB) + the re-laid-out weight, fp32 (2.4 MB) and
    # as the 16-bit MFMA operand (two fp16 pieces: 2.4 MB)
    assert 8 * 256 * 64 * 64 * 4 <= fw < 8 * 256 * 64 * 64 * 4 + 8 * 2**20
    assert bw > fw
    # transposed output size (cfg5): 32 -> 64 with k4 s2 p1
    t = cfg2_desc(transposed=1, in_channels=256, out_channels=128, offset_groups=2, mask_groups=2)
    for i in range(2):
        t.in_size[i], t.kernel[i], t.stride[i] = 32, 4, 2
    assert lib.tvdcn_conv_output_size(ctypes.byref(t), out) == 0
    assert list(out)[:2] == [64, 64]


def test_c_abi_argument_errors(lib):
    lib.tvdcn_conv_output_size.restype = ctypes.c_int
    lib.tvdcn_deform_conv_forward.restype = ctypes.c_int
    lib.tvdcn_last_error.restype = ctypes.c_char_p
    out = (ctypes.c_int64 * 3)()
    bad = cfg2_desc()
    bad.stride[0] = 0
    assert lib.tvdcn_conv_output_size(ctypes.byref(bad), out) == 1
    assert b"stride" in lib.tvdcn_last_error()
    small = cfg2_desc()
    small.in_size[0] = 1
    small.padding[0] = 0
    assert lib.tvdcn_conv_output_size(ctypes.byref(small), out) == 1
    assert b"too small" in lib.tvdcn_last_error()
    # argument checks fail before any device work: workspace too small, mismatched offset pointer
    d = cfg2_desc()
    st = lib.tvdcn_deform_conv_forward(ctypes.byref(d), None, None, None, None, None, None, None,
                                       ctypes.c_size_t(0), None)
    assert st == 1 and b"offset" in lib.tvdcn_last_error()
    d = cfg2_desc(offset_groups=0, mask_groups=0)
    st = lib.tvdcn_deform_conv_forward(ctypes.byref(d), None, None, None, None, None, None, None,
                                       ctypes.c_size_t(16), None)
    assert st == 2
    d = cfg2_desc(offset_groups=3)
    assert lib.tvdcn_conv_output_size(ctypes.byref(d), out) == 0
    st = lib.tvdcn_deform_conv_forward(ctypes.byref(d), None, None, ctypes.c_void_p(16), ctypes.c_void_p(16), None,
                                       None, None, ctypes.c_size_t(0), None)
    assert st == 1 and b"offset_groups" in lib.tvdcn_last_error()
    # descriptor flags: unknown bits, and channels-last input on the transposed op
    for d, msg in ((cfg2_desc(flags=8), b"unknown flags"),
                   (cfg2_desc(flags=6, mask_scale=2.0), b"exclude each other"),
                   (cfg2_desc(flags=4, mask_groups=0), b"softmax mask"),
                   (cfg2_desc(flags=1, transposed=1, out_channels=128, offset_groups=2, mask_groups=2),
                    b"channels-last"),
                   (cfg2_desc(flags=2, mask_scale=0.0), b"sigmoid mask"),
                   (cfg2_desc(flags=2, mask_scale=2.0, mask_groups=0), b"sigmoid mask")):
        st = lib.tvdcn_deform_conv_forward(ctypes.byref(d), None, None, ctypes.c_void_p(16), ctypes.c_void_p(16),
                                           None, None, None, ctypes.c_size_t(0), None)
        assert st == 1 and msg in lib.tvdcn_last_error()


def test_batch_blocks_keep_pointers_aligned(lib):
    """With a forced block limit the batch runs in blocks of images; for C = 3 on a 7 x 7 input every
    batch-sized tensor's per-image bytes leave a remainder mod 16 (float32 input 588 B, offset 392 B x
    18 / 9 ...), so the block is rounded down to a multiple of the image count m that makes all of them
    multiples of 16: each block's pointers stay 16-byte aligned. With room for fewer than m images per
    block the block is not rounded (the kernels accept less aligned block pointers)."""
    lib.tvdcn_conv_batch_block.restype = ctypes.c_int
    lib.tvdcn_set_max_block_elements.restype = ctypes.c_int
    d = Desc(dim=2, transposed=0, dtype=0, batch=37, in_channels=3, out_channels=5, groups=1, offset_groups=1,
             mask_groups=1)
    for i in range(2):
        d.in_size[i], d.kernel[i], d.stride[i], d.padding[i], d.dilation[i] = 7, 3, 1, 1, 1
    es_of = {0: 4, 1: 8, 2: 2, 3: 2}
    try:
        for dtype in (0, 1, 2, 3):
            d.dtype = dtype
            es = es_of[dtype]
            per_image = [3 * 49, 5 * 49, 18 * 49, 9 * 49]   # input, output, offset, mask
            m = max(16 // math.gcd(n * es % 16, 16) if n * es % 16 else 1 for n in per_image)
            for limit in (20 * 18 * 49, 18 * 49 * 3, 2 ** 31 - 1):
                assert lib.tvdcn_set_max_block_elements(ctypes.c_int64(limit)) == 0
                blk = ctypes.c_int64(0)
                assert lib.tvdcn_conv_batch_block(ctypes.byref(d), ctypes.byref(blk)) == 0
                raw = min(37, limit // (18 * 49))
                if raw >= 37:
                    assert blk.value == 37
                elif raw >= m:
                    assert blk.value == raw - raw % m and blk.value % m == 0
                    for n in per_image:
                        assert blk.value * n * es % 16 == 0
                else:
                    assert blk.value == raw
    finally:
        lib.tvdcn_set_max_block_elements(ctypes.c_int64(2 ** 31 - 1))


def test_c_abi_rejects_misaligned_tensor_pointers(lib):
    """The C ABI takes 16-byte aligned tensor pointers (a batch block's own pointers may be less
    aligned; the caller's are checked at the entry, before any device work)."""
    lib.tvdcn_deform_conv_forward.restype = ctypes.c_int
    lib.tvdcn_deform_conv_backward.restype = ctypes.c_int
    lib.tvdcn_last_error.restype = ctypes.c_char_p
    d = cfg2_desc()
    big = ctypes.c_size_t(1 << 40)
    p, q = ctypes.c_void_p(1 << 20), ctypes.c_void_p((1 << 20) + 4)
    st = lib.tvdcn_deform_conv_forward(ctypes.byref(d), p, p, q, p, None, p, p, big, None)
    assert st == 1 and b"16-byte aligned" in lib.tvdcn_last_error()
    st = lib.tvdcn_deform_conv_backward(ctypes.byref(d), p, p, p, p, p, p, p, p, q, None, p, big, None)
    assert st == 1 and b"16-byte aligned" in lib.tvdcn_last_error()


REF_SCHEMAS = {
    "deform_conv1d": "(Tensor input, Tensor weight, Tensor? offset=None, Tensor? mask=None, Tensor? bias=None, "
                     "SymInt[1] stride=[1], SymInt[1] padding=[0], SymInt[1] dilation=[1], SymInt groups=1) -> Tensor",
    "deform_conv2d": "(Tensor input, Tensor weight, Tensor? offset=None, Tensor? mask=None, Tensor? bias=None, "
                     "SymInt[2] stride=[1, 1], SymInt[2] padding=[0, 0], SymInt[2] dilation=[1, 1], "
                     "SymInt groups=1) -> Tensor",
    "deform_conv_transpose2d": "(Tensor input, Tensor weight, Tensor? offset=None, Tensor? mask=None, "
                               "Tensor? bias=None, SymInt[2] stride=[1, 1], SymInt[2] padding=[0, 0], "
                               "SymInt[2] output_padding=[0, 0], SymInt[2] dilation=[1, 1], SymInt groups=1) -> Tensor",
}


TWELVE = [n for dim in (1, 2, 3) for base in (f"deform_conv{dim}d", f"deform_conv_transpose{dim}d")
          for n in (base, f"_{base}_backward")]


@pytest.fixture(scope="module")
def reference_schemas():
    """schema strings of the reference build (run in a child process: it registers torch.ops.tvdcn too)"""
    if not oracle.have_reference():
        return None
    return dict(zip(TWELVE, oracle.run_reference([{"schema": n} for n in TWELVE])))


@pytest.mark.parametrize("name", sorted(REF_SCHEMAS))
def test_schemas_match_reference(name):
    schema = str(getattr(torch.ops.tvdcn, name).default._schema)
    assert schema == f"tvdcn::{name}{REF_SCHEMAS[name]}"


def test_all_twelve_ops_and_backward_schemas_exist(reference_schemas):
    for name in TWELVE:
        schema = str(getattr(torch.ops.tvdcn, name).default._schema)
        assert schema.endswith("-> (Tensor, Tensor, Tensor, Tensor, Tensor)" if name.startswith("_") else "-> Tensor")
        if reference_schemas is not None:
            assert schema == reference_schemas[name]


def meta(*shape):
    return torch.empty(*shape, device="meta")


@pytest.mark.parametrize("dim", [1, 2, 3])
def test_meta_shapes(dim):
    sz = [9, 10, 11][:dim]
    k = [3, 2, 3][:dim]
    kn = 1
    for kk in k:
        kn *= kk
    out = [s - kk + 1 for s, kk in zip(sz, k)]
    y = getattr(tvdcn, f"deform_conv{dim}d")(meta(2, 4, *sz), meta(6, 2, *k), meta(2, 2 * dim * kn, *out),
                                                 meta(2, 3 * kn, *out)[:, :kn], meta(6), groups=2)
    assert list(y.shape) == [2, 6] + out
    yt = getattr(tvdcn, f"deform_conv_transpose{dim}d")(meta(2, 4, *sz), meta(4, 3, *k), meta(2, dim * kn, *sz),
                                                            None, meta(6), stride=2, padding=1, output_padding=1,
                                                            groups=2)
    assert list(yt.shape) == [2, 6] + [(s - 1) * 2 - 2 + kk + 1 for s, kk in zip(sz, k)]
    # unbatched
    y1 = getattr(tvdcn, f"deform_conv{dim}d")(meta(4, *sz), meta(6, 4, *k), meta(dim * kn, *out))
    assert list(y1.shape) == [6] + out


INVALID = [
    ("offset channels", (meta(2, 4, 8, 8), meta(5, 4, 3, 3), meta(2, 17, 6, 6), None, None),
     "The shape of the offset tensor at dimension 1 is not valid"),
    ("offset multiple", (meta(2, 4, 8, 8), meta(5, 4, 3, 3), meta(2, 36 + 18, 6, 6), None, None),
     "% offset_groups == 0"),
    ("offset batch", (meta(2, 4, 8, 8), meta(5, 4, 3, 3), meta(3, 18, 6, 6), None, None),
     "invalid batch size of offset"),
    ("offset grid", (meta(2, 4, 8, 8), meta(5, 4, 3, 3), meta(2, 18, 5, 6), None, None), "offset output dims"),
    ("mask channels", (meta(2, 4, 8, 8), meta(5, 4, 3, 3), None, meta(2, 8, 6, 6), None),
     "The shape of the mask tensor at dimension 1 is not valid"),
    ("mask batch", (meta(2, 4, 8, 8), meta(5, 4, 3, 3), None, meta(1, 9, 6, 6), None), "invalid batch size of mask"),
    ("mask grid", (meta(2, 4, 8, 8), meta(5, 4, 3, 3), None, meta(2, 9, 6, 7), None), "mask output dims"),
    ("input ndim", (meta(2, 4, 8, 8, 1), meta(5, 4, 3, 3), None, None, None), "Expected 3D (unbatched) or 4D"),
    ("weight ndim", (meta(2, 4, 8, 8), meta(5, 4, 3), None, None, None), "Expected 4D weight"),
    ("too small", (meta(2, 4, 2, 2), meta(5, 4, 3, 3), None, None, None), "Calculated output size too small"),
]


@pytest.fixture(scope="module")
def reference_errors():
    """message the reference build raises for each INVALID case on CPU zeros of the same shapes"""
    if not oracle.have_reference():
        return None
    reqs = [{"error": "deform_conv2d",
             "args": [torch.zeros(a.shape) if isinstance(a, torch.Tensor) else a for a in args] +
                     [[1, 1], [0, 0], [1, 1], 1]} for _, args, _ in INVALID]
    return dict(zip((c[0] for c in INVALID), oracle.run_reference(reqs)))


@pytest.mark.parametrize("label,args,msg", INVALID, ids=[c[0] for c in INVALID])
def test_validation_errors_match_reference(label, args, msg, reference_errors):
    with pytest.raises(RuntimeError) as ei:
        torch.ops.tvdcn.deform_conv2d(*args, [1, 1], [0, 0], [1, 1], 1)
    assert msg in str(ei.value)
    if reference_errors is not None:
        ref = reference_errors[label]
        assert ref is not None and msg in ref, ref


@pytest.mark.parametrize("what", ["stride", "pad", "dilation"])
def test_parameter_errors(what):
    s, p, d = [1, 1], [0, 0], [1, 1]
    {"stride": s, "pad": p, "dilation": d}[what][0] = -1 if what == "pad" else 0
    with pytest.raises(RuntimeError, match=what + "_h"):
        torch.ops.tvdcn.deform_conv2d(meta(2, 4, 8, 8), meta(5, 4, 3, 3), None, None, None, s, p, d, 1)


def test_groups_error():
    with pytest.raises(RuntimeError, match="groups"):
        torch.ops.tvdcn.deform_conv2d(meta(2, 4, 8, 8), meta(5, 4, 3, 3), None, None, None, [1, 1], [0, 0],
                                          [1, 1], 2)


def test_dtype_mismatch_error():
    with pytest.raises(RuntimeError):
        torch.ops.tvdcn.deform_conv2d(meta(2, 4, 8, 8), meta(5, 4, 3, 3).double(), None, None, None, [1, 1],
                                          [0, 0], [1, 1], 1)


def test_cpu_key_registered_for_every_op():
    """every schema has a CPU kernel (the reference registers CPU twins of its CUDA drivers,
    ops/cpu/deform_conv2d_kernel.cpp:645) besides the CUDA (HIP) one"""
    ops = ["deform_conv1d", "deform_conv2d", "deform_conv3d", "deform_conv_transpose1d", "deform_conv_transpose2d",
           "deform_conv_transpose3d"]
    names = ops + [f"_{o}_backward" for o in ops] + ["mask_softmax", "_mask_softmax_backward",
                                                      "deform_conv_mask_activation",
                                                      "_deform_conv_mask_activation_backward"]
    for n in names:
        for key in ("CPU", "CUDA", "Meta"):
            assert torch._C._dispatch_has_kernel_for_dispatch_key(f"tvdcn::{n}", key), (n, key)
    y = tvdcn.deform_conv2d(torch.rand(1, 2, 5, 5), torch.rand(2, 2, 3, 3), torch.rand(1, 18, 3, 3))
    assert y.device.type == "cpu" and y.shape == (1, 2, 3, 3)
    assert tvdcn.mask_softmax2d(torch.rand(1, 9, 3, 3), (3, 3)).device.type == "cpu"


def test_meta_autograd_and_double_backward():
    x = meta(2, 4, 8, 8).requires_grad_(True)
    w = meta(5, 4, 3, 3).requires_grad_(True)
    o = meta(2, 18, 6, 6).requires_grad_(True)
    m = meta(2, 9, 6, 6).requires_grad_(True)
    b = meta(5).requires_grad_(True)
    y = tvdcn.deform_conv2d(x, w, o, m, b)
    gx, gw, go, gm, gb = torch.autograd.grad(y.sum(), (x, w, o, m, b), create_graph=True)
    assert gx.shape == x.shape and gw.shape == w.shape and go.shape == o.shape and gm.shape == m.shape
    assert gb.shape == b.shape
    with pytest.raises(RuntimeError, match="double backwards on deform_conv2d not supported"):
        gx.sum().backward()


def test_meta_autograd_without_offset_mask_bias():
    x = meta(2, 4, 8, 8).requires_grad_(True)
    w = meta(5, 4, 3, 3).requires_grad_(True)
    y = tvdcn.deform_conv2d(x, w)
    y.sum().backward()
    assert x.grad.shape == x.shape and w.grad.shape == w.shape
    gs = torch.ops.tvdcn._deform_conv2d_backward(meta(2, 5, 6, 6), meta(2, 4, 8, 8), meta(5, 4, 3, 3), None,
                                                     None, None, [1, 1], [0, 0], [1, 1], 1)
    assert gs[2] is None and gs[3] is None and gs[4] is None


def test_modules_api():
    m = tvdcn.DeformConv2d(4, 6, 3, padding=1, groups=2, bias=False)
    assert m.weight.shape == (6, 2, 3, 3) and m.bias is None
    assert "bias=False" in repr(m) and "groups=2" in repr(m)
    p = tvdcn.PackedDeformConv2d(4, 8, 3, padding=1, offset_groups=2, mask_groups=4, modulated=True,
                                     mask_activation="softmax")
    assert p.offset_generator.weight.shape == (2 * 9 * 2, 2, 3, 3)
    assert p.mask_generator.weight.shape == (9 * 4, 1, 3, 3)
    assert float(p.offset_generator.weight.detach().abs().sum()) == 0.0
    assert isinstance(p.mask_activation, tvdcn.MaskSoftmax2d)
    t = tvdcn.PackedDeformConvTranspose2d(4, 6, 4, stride=2, padding=1, modulated=True)
    assert t.offset_generator.kernel_size == (1, 1) and t.mask_generator.out_channels == 16
    assert isinstance(t.mask_activation, tvdcn.MaskSigmoid) and t.mask_activation.scale == 2.0
    for cls in (tvdcn.PackedDeformConv1d, tvdcn.PackedDeformConv3d, tvdcn.PackedDeformConvTranspose1d,
                tvdcn.PackedDeformConvTranspose3d):
        assert cls(4, 4, 3).deformable
    with pytest.raises(ValueError, match="in_channels must be divisible by offset_groups"):
        tvdcn.PackedDeformConv2d(4, 8, 3, offset_groups=3)
    with pytest.raises(ValueError, match="out_channels must be divisible by mask_groups"):
        tvdcn.PackedDeformConv2d(4, 6, 3, mask_groups=4)
    with pytest.raises(ValueError, match="no activation is supported for offset"):
        tvdcn.PackedDeformConv2d(4, 8, 3, offset_activation="tanh")
    with pytest.raises(ValueError, match="only"):
        tvdcn.PackedDeformConv2d(4, 8, 3, mask_activation="relu")


def test_module_forward_on_meta():
    m = tvdcn.PackedDeformConv2d(4, 6, 3, padding=1, modulated=True, device="meta")
    assert m(meta(2, 4, 8, 8)).shape == (2, 6, 8, 8)
    r = tvdcn.DeformConv2d(4, 6, 3, padding=1, padding_mode="reflect", device="meta")
    assert r(meta(2, 4, 8, 8), meta(2, 18, 8, 8)).shape == (2, 6, 8, 8)
    t = tvdcn.DeformConvTranspose2d(4, 6, 3, stride=2, padding=1, device="meta")
    assert t(meta(2, 4, 5, 5), None, output_size=[10, 10]).shape == (2, 6, 10, 10)
    with pytest.raises(ValueError, match="requested an output size"):
        t(meta(2, 4, 5, 5), None, output_size=[20, 20])
    bad = tvdcn.DeformConvTranspose2d(4, 6, 3, padding_mode="reflect", device="meta")
    with pytest.raises(ValueError, match="zeros"):
        bad(meta(2, 4, 5, 5), None)


def test_output_padding_matches_torch_rule():
    ours = tvdcn.DeformConvTranspose2d(4, 6, 3, stride=3, padding=1, dilation=2)
    ref = torch.nn.ConvTranspose2d(4, 6, 3, stride=3, padding=1, dilation=2)
    x = torch.empty(1, 4, 7, 5)
    for size in ([21, 15], [22, 16], [23, 17]):
        assert ours._output_padding(x, size, [3, 3], [1, 1], [3, 3], 2, [2, 2]) == \
            ref._output_padding(x, size, [3, 3], [1, 1], [3, 3], 2, [2, 2])


def test_mask_activation_errors():
    with pytest.raises(ValueError, match="scale must be positive"):
        tvdcn.mask_sigmoid(torch.zeros(2), scale=0.0)
    assert torch.allclose(tvdcn.mask_sigmoid(torch.zeros(3)), torch.ones(3))
    with pytest.raises(RuntimeError, match="mask tensor at dimension 1 is not valid"):
        tvdcn.mask_softmax2d(meta(2, 5, 3, 3), (3, 3))
    y = tvdcn.mask_softmax3d(meta(2, 54, 2, 3, 4), 3)
    assert y.shape == (2, 54, 2, 3, 4)
    assert tvdcn.MaskSoftmax1d(5)(meta(2, 10, 7)).shape == (2, 10, 7)


def fastdiv(n, d):
    """Python restatement of FastDiv (tvdcn_amd/csrc/hip/common.h) for checking the constants"""
    s = 0
    while (1 << s) < d:
        s += 1
    m = ((1 << 32) * ((1 << s) - d)) // d + 1
    t = (n * m) >> 32
    return (t + n) >> s


def test_fastdiv_constants_are_exact():
    import random
    rng = random.Random(0)
    for d in list(range(1, 300)) + [4096, 4097, 12544, 50176, 65536, 1 << 20, (1 << 31) - 1]:
        for n in [0, 1, d - 1, d, d + 1, 2 * d - 1, (1 << 31) - 1, (1 << 31) - 2] + \
                 [rng.randrange(0, 1 << 31) for _ in range(200)]:
            if 0 <= n < (1 << 31):
                assert fastdiv(n, d) == n // d, (n, d)


@pytest.mark.parametrize("dim,transposed", [(1, False), (2, False), (3, False), (1, True), (2, True), (3, True)])
def test_torch_compile_fullgraph_on_meta(dim, transposed):
    """torch.compile traces the ops without graph breaks (fullgraph=True): the Meta kernels serve
    as the fake-tensor implementations, forward and backward."""
    from torch._dynamo.testing import CompileCounterWithBackend
    torch._dynamo.reset()
    k = 3
    S = [6] * dim
    if transposed:
        fn = getattr(tvdcn, f"deform_conv_transpose{dim}d")
        x = meta(2, 4, *S)
        w = meta(4, 3, *[k] * dim)                    # (Cin, Cout, k...)
        out_sz = [s + k - 1 for s in S]
        o = meta(2, dim * k ** dim, *S)                # offsets on the input grid
        m = meta(2, k ** dim, *S)
    else:
        fn = getattr(tvdcn, f"deform_conv{dim}d")
        x = meta(2, 4, *S)
        w = meta(5, 4, *[k] * dim)
        out_sz = [s - k + 1 for s in S]
        o = meta(2, dim * k ** dim, *out_sz)
        m = meta(2, k ** dim, *out_sz)
    b = meta(w.shape[1] if transposed else w.shape[0])
    leaves = [t.requires_grad_(True) for t in (x, w, o, m, b)]

    def f(x, w, o, m, b):
        return torch.relu(fn(x, w, o, m, b)).sum()

    cnt = CompileCounterWithBackend("aot_eager")
    out = torch.compile(f, backend=cnt, fullgraph=True)(*leaves)
    out.backward()
    assert cnt.frame_count == 1
    for t in leaves:
        assert t.grad is not None and t.grad.shape == t.shape
    if transposed:
        assert list(fn(x, w, o, m, b).shape[2:]) == out_sz


@pytest.mark.parametrize("activation", [1, 2])
def test_mask_activation_op_on_meta(activation):
    """The fused mask-activation op: shapes, gradients to the logits, double-backward refusal, argument
    errors, and the packed modules' choice of the fused path."""
    x = meta(2, 4, 8, 8).requires_grad_(True)
    w = meta(5, 4, 3, 3).requires_grad_(True)
    o = meta(2, 18, 6, 6).requires_grad_(True)
    lg = meta(2, 9, 6, 6).requires_grad_(True)
    op = torch.ops.tvdcn.deform_conv_mask_activation
    y = op(x, w, o, lg, None, [1, 1], [0, 0], [0, 0], [1, 1], 1, False, activation, 2.0)
    assert y.shape == (2, 5, 6, 6)
    gx, gw, go, gl = torch.autograd.grad(y.sum(), (x, w, o, lg), create_graph=True)
    assert gl.shape == lg.shape and go.shape == o.shape
    with pytest.raises(RuntimeError, match="double backwards on deform_conv_mask_activation not supported"):
        gl.sum().backward()
    with pytest.raises(RuntimeError, match="activation must be"):
        op(x, w, o, lg, None, [1, 1], [0, 0], [0, 0], [1, 1], 1, False, 3, 2.0)
    if activation == 1:
        with pytest.raises(RuntimeError, match="mask_scale"):
            op(x, w, o, lg, None, [1, 1], [0, 0], [0, 0], [1, 1], 1, False, 1, 0.0)


def test_packed_modules_choose_the_fused_mask_activation():
    name = "sigmoid"
    for cls, ks in ((tvdcn.PackedDeformConv2d, (3, 3)), (tvdcn.PackedDeformConvTranspose1d, (3,))):
        for name, code in (("sigmoid", 1), ("softmax", 2)):
            m = cls(4, 6, 3, modulated=True, mask_activation=name, device="meta")
            assert m._mask_fusion()[0] == code
            offset, logits, fused, scale = m._generate(meta(2, 4, *([8] * len(ks))))
            assert fused == code and logits.shape[1] == len(ks) and (scale == 2.0 or code == 2) or \
                logits.shape[1] == 3 ** len(ks)
    m = tvdcn.PackedDeformConv2d(4, 6, 3, modulated=True, device="meta")
    m.mask_activation = torch.nn.Sigmoid()            # any other activation runs as a module
    assert m._mask_fusion() == (0, 0.0)
    m.mask_activation = tvdcn.MaskSoftmax2d((3, 1))   # a softmax over other taps is not fused
    assert m._mask_fusion() == (0, 0.0)
    m.mask_activation = tvdcn.MaskSigmoid(0.5)
    assert m._mask_fusion() == (1, 0.5)
    m.mask_activation = tvdcn.MaskSigmoid(-1.0)       # left to MaskSigmoid, which raises ValueError
    assert m._mask_fusion() == (0, 0.0)
    with pytest.raises(ValueError, match="scale must be positive"):
        m(meta(2, 4, 8, 8))


@pytest.mark.parametrize("kind", ["hook", "pre_hook", "global_hook"])
def test_mask_activation_hooks_run(kind):
    """A forward hook or pre-hook on the mask activation (or a global one) runs as in the reference,
    which calls the activation module: the fused mask load is not taken while one is registered, and
    what the hook does to the mask shows in the output."""
    torch.manual_seed(0)
    m = tvdcn.PackedDeformConv2d(4, 6, 3, padding=1, modulated=True)
    for gen in (m.offset_generator, m.mask_generator):
        torch.nn.init.normal_(gen.weight, std=0.3)
    x = torch.randn(2, 4, 7, 8)
    calls = []
    if kind == "hook":
        h = m.mask_activation.register_forward_hook(lambda mod, inp, out: calls.append(1) or out * 0.25)
    elif kind == "pre_hook":
        h = m.mask_activation.register_forward_pre_hook(lambda mod, inp: calls.append(1) or (inp[0] - 3.0,))
    else:
        h = torch.nn.modules.module.register_module_forward_hook(
            lambda mod, inp, out: (calls.append(1) or out * 0.25) if isinstance(mod, tvdcn.MaskSigmoid) else None)
    try:
        assert m._mask_fusion() == (0, 0.0)
        y = m(x)
    finally:
        h.remove()
    assert calls, "the hook did not run"
    assert m._mask_fusion() == (1, 2.0)       # fused again once the hook is gone
    offset = m.offset_generator(x)
    logits = m.mask_generator(x)
    mask = 2.0 * torch.sigmoid(logits - 3.0 if kind == "pre_hook" else logits)
    if kind != "pre_hook":
        mask = mask * 0.25
    ref = tvdcn.deform_conv2d(x, m.weight, offset, mask, m.bias, padding=1)
    assert torch.allclose(y, ref, rtol=1e-5, atol=1e-6)


MODULES = [
    ("DeformConv1d", (4, 6, 3), (2, 4, 9)), ("DeformConv2d", (4, 6, 3), (2, 4, 9, 8)),
    ("DeformConv3d", (4, 6, 3), (2, 4, 5, 6, 7)),
    ("DeformConvTranspose1d", (4, 6, 3), (2, 4, 9)), ("DeformConvTranspose2d", (4, 6, 3), (2, 4, 9, 8)),
    ("DeformConvTranspose3d", (4, 6, 3), (2, 4, 5, 6, 7)),
    ("PackedDeformConv1d", (4, 6, 3), (2, 4, 9)), ("PackedDeformConv2d", (4, 6, 3), (2, 4, 9, 8)),
    ("PackedDeformConv3d", (4, 6, 3), (2, 4, 5, 6, 7)),
    ("PackedDeformConvTranspose1d", (4, 6, 3), (2, 4, 9)),
    ("PackedDeformConvTranspose2d", (4, 6, 3), (2, 4, 9, 8)),
    ("PackedDeformConvTranspose3d", (4, 6, 3), (2, 4, 5, 6, 7)),
    ("MaskSoftmax1d", (3,), (2, 6, 9)), ("MaskSoftmax2d", (3,), (2, 18, 9, 8)),
    ("MaskSoftmax3d", (3,), (2, 54, 5, 6, 7)), ("MaskSigmoid", (), (2, 9, 8)),
]


@pytest.mark.parametrize("packed_kw", [{}, {"modulated": True}, {"modulated": True, "mask_activation": "softmax"},
                                       {"deformable": False, "modulated": True}, {"padding_mode": "reflect"}])
@pytest.mark.parametrize("name,args,shape", MODULES, ids=[m[0] for m in MODULES])
def test_torchscript_modules(name, args, shape, packed_kw):
    """Every module class compiles with torch.jit.script, as tvdcn's examples do
    (examples/deform_conv_modules_example.py:8,23), and the scripted module computes the eager
    module's shapes (meta tensors: the Meta kernels run the same validation)."""
    cls = getattr(tvdcn, name)
    kw = {}
    if name.startswith("Packed"):
        kw = dict(packed_kw)
        if "Transpose" in name and kw.get("padding_mode", "zeros") != "zeros":
            kw.pop("padding_mode")
    elif packed_kw:
        pytest.skip("packed-module options")
    if name.startswith("Deform") and "Transpose" not in name:
        kw["padding"] = 1
    m = cls(*args, **kw, device="meta") if not name.startswith("Mask") else cls(*args)
    sm = torch.jit.script(m)
    x = meta(*shape)
    if name.startswith("Packed") or name.startswith("Mask"):
        ins = (x,)
    else:
        dim = len(shape) - 2
        k = 3 ** dim
        grid = shape[2:]
        ins = (x, meta(shape[0], dim * k, *grid), meta(shape[0], k, *grid))
    assert sm(*ins).shape == m(*ins).shape


def test_torchscript_functional_defaults():
    """The functional ops script with their int defaults (int-or-tuple parameters)"""
    f = torch.jit.script(tvdcn.deform_conv2d)
    y = f(meta(2, 4, 9, 8), meta(6, 4, 3, 3))
    assert y.shape == (2, 6, 7, 6)
    y = f(meta(2, 4, 9, 8), meta(6, 4, 3, 3), padding=1, stride=(2, 1))
    assert y.shape == (2, 6, 5, 8)
    ft = torch.jit.script(tvdcn.deform_conv_transpose1d)
    assert ft(meta(2, 4, 9), meta(4, 6, 3), stride=2, output_padding=1).shape == (2, 6, 20)


def test_drop_in_package_layout():
    """import tvdcn gives the reference's package layout (tvdcn/__init__.py, tvdcn/ops/__init__.py,
    tvdcn/ops/activations/__init__.py) on the MI355X implementation"""
    import importlib
    import tvdcn_amd
    for mod in ("tvdcn.ops", "tvdcn.ops.activations", "tvdcn.ops.activations.mask_softmax",
                "tvdcn.ops.activations.mask_sigmoid", "tvdcn.ops.deform_conv", "tvdcn.ops.deform_conv_transpose",
                "tvdcn.extension", "tvdcn.utils"):
        assert importlib.import_module(mod) is importlib.import_module(mod.replace("tvdcn", "tvdcn_amd", 1))
    from tvdcn.ops import deform_conv2d, PackedDeformConvTranspose3d  # noqa: F401
    from tvdcn.ops.activations import MaskSigmoid, mask_softmax2d  # noqa: F401
    public = [n for n in dir(tvdcn_amd) if not n.startswith("_")]
    for n in public:
        assert getattr(tvdcn, n) is getattr(tvdcn_amd, n)
    assert tvdcn.deform_conv2d is tvdcn.ops.deform_conv2d
    assert torch.ops.tvdcn.deform_conv2d.default._schema.name == "tvdcn::deform_conv2d"


@pytest.mark.parametrize("dim,transposed", [(1, 0), (2, 0), (3, 0), (2, 1)])
def test_c_abi_empty_batch_queries(lib, dim, transposed):
    """Workspace queries of an empty batch (host planning only): GEMM sides of 16 rows and more
    once divided by a zero split count."""
    lib.tvdcn_deform_conv_forward_workspace_size.restype = ctypes.c_size_t
    lib.tvdcn_deform_conv_backward_workspace_size.restype = ctypes.c_size_t
    for ch in (4, 32, 256):
        d = Desc(dim=dim, transposed=transposed, dtype=0, batch=0, in_channels=ch, out_channels=ch, groups=1,
                 offset_groups=1, mask_groups=1)
        for i in range(3):
            d.in_size[i], d.kernel[i], d.stride[i], d.padding[i], d.dilation[i] = 7, 3, 1, 1, 1
        assert lib.tvdcn_deform_conv_forward_workspace_size(ctypes.byref(d)) > 0
        assert lib.tvdcn_deform_conv_backward_workspace_size(ctypes.byref(d)) > 0


def test_c_abi_planning_fuzz(lib):
    """Host planning over random valid descriptors (ranks, conv / transposed, strides, paddings,
    dilations, groups, offset / mask groups, dtypes, flags, empty batches): every workspace
    query returns without crashing, and a positive size exactly when the output size query
    accepts the descriptor."""
    import random
    rnd = random.Random(2024)
    lib.tvdcn_conv_output_size.restype = ctypes.c_int
    lib.tvdcn_deform_conv_forward_workspace_size.restype = ctypes.c_size_t
    lib.tvdcn_deform_conv_backward_workspace_size.restype = ctypes.c_size_t
    out = (ctypes.c_int64 * 3)()
    for _ in range(400):
        dim = rnd.choice((1, 2, 3))
        tr = rnd.random() < 0.4
        groups = rnd.choice((1, 1, 2, 4))
        cin = groups * rnd.choice((1, 2, 3, 4, 8, 12, 16, 20, 32, 48))
        cout = groups * rnd.choice((1, 2, 3, 4, 8, 16, 24, 40, 64))
        cols = cout if tr else cin
        og = rnd.choice([g for g in (0, 1, 2, 4) if g == 0 or (cin % g == 0 and cols % g == 0)])
        mg = rnd.choice([g for g in (0, 1, 2, 4) if g == 0 or (cin % g == 0 and cols % g == 0)])
        flags = 0
        if not tr and dim > 1 and rnd.random() < 0.2:
            flags |= 1
        if mg and rnd.random() < 0.2:
            flags |= 2
        d = Desc(dim=dim, transposed=int(tr), dtype=rnd.choice((0, 1, 2, 3)), flags=flags,
                 batch=rnd.choice((0, 1, 2, 3)), in_channels=cin, out_channels=cout, groups=groups,
                 offset_groups=og, mask_groups=mg, mask_scale=2.0)
        for i in range(3):
            d.in_size[i] = rnd.choice((1, 2, 5, 9, 17, 33)) if i < dim else 1
            d.kernel[i] = rnd.choice((1, 2, 3, 4)) if i < dim else 1
            d.stride[i] = rnd.choice((1, 1, 2, 3)) if i < dim else 1
            d.padding[i] = rnd.choice((0, 1, 2)) if i < dim else 0
            d.dilation[i] = rnd.choice((1, 1, 2)) if i < dim else 1
            d.output_padding[i] = rnd.choice((0, 1)) if (tr and i < dim and d.stride[i] > 1) else 0
        ok = lib.tvdcn_conv_output_size(ctypes.byref(d), out) == 0
        fw = lib.tvdcn_deform_conv_forward_workspace_size(ctypes.byref(d))
        bw = lib.tvdcn_deform_conv_backward_workspace_size(ctypes.byref(d))
        if not ok:
            assert fw == 0 and bw == 0
        else:
            assert bw > 0


def test_c_abi_layout_copy_argument_checks(lib):
    """tvdcn_to_channels_last / tvdcn_from_channels_last: float32 only, sizes checked on the host,
    empty tensors succeed without touching the device."""
    lib.tvdcn_last_error.restype = ctypes.c_char_p
    for fn in (lib.tvdcn_to_channels_last, lib.tvdcn_from_channels_last):
        fn.restype = ctypes.c_int
        fn.argtypes = [ctypes.c_int32, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p,
                       ctypes.c_void_p, ctypes.c_void_p]
        assert fn(1, 2, 3, 4, None, None, None) != 0                          # float64
        assert b"float32 only" in lib.tvdcn_last_error()
        assert fn(0, -1, 3, 4, None, None, None) != 0
        assert b"negative size" in lib.tvdcn_last_error()
        assert fn(0, 1 << 20, 1 << 10, 1 << 10, None, None, None) != 0       # 2^40 elements
        assert b"32-bit indexing" in lib.tvdcn_last_error()
        assert fn(0, 0, 3, 4, None, None, None) == 0                          # empty batch
        assert lib.tvdcn_last_error() == b""
        assert fn(0, 2, 3, 4, None, None, None) != 0                          # null pointers
        assert b"null pointer" in lib.tvdcn_last_error()


def test_c_abi_batch_blocks_beyond_32_bit_indexing(lib):
    """A descriptor above 2^31 elements (B=128, C=256, 256x256 float32: 2^31 input elements) plans
    in batch blocks: the workspace queries succeed and serve one block; lowering the block limit
    shrinks the workspace; one image above the limit is refused; the limit's range is checked."""
    lib.tvdcn_deform_conv_forward_workspace_size.restype = ctypes.c_size_t
    lib.tvdcn_deform_conv_backward_workspace_size.restype = ctypes.c_size_t
    lib.tvdcn_set_max_block_elements.argtypes = [ctypes.c_int64]
    lib.tvdcn_set_max_block_elements.restype = ctypes.c_int
    lib.tvdcn_last_error.restype = ctypes.c_char_p
    big = cfg2_desc(batch=128)
    for i in range(2):
        big.in_size[i] = 256
    assert 128 * 256 * 256 * 256 >= 2 ** 31
    fw = lib.tvdcn_deform_conv_forward_workspace_size(ctypes.byref(big))
    bw = lib.tvdcn_deform_conv_backward_workspace_size(ctypes.byref(big))
    half = cfg2_desc(batch=64)   # the largest block below 2^31 elements: 127 images, a remainder of 1
    for i in range(2):
        half.in_size[i] = 256
    assert fw > 0 and bw > 0
    assert fw <= lib.tvdcn_deform_conv_forward_workspace_size(ctypes.byref(half)) * 2
    try:
        per_image = 256 * 256 * 256
        assert lib.tvdcn_set_max_block_elements(4 * per_image) == 0
        fw4 = lib.tvdcn_deform_conv_forward_workspace_size(ctypes.byref(big))
        assert 0 < fw4 < fw / 16
        assert lib.tvdcn_set_max_block_elements(per_image - 1) == 0
        assert lib.tvdcn_deform_conv_forward_workspace_size(ctypes.byref(big)) == 0
        out = (ctypes.c_int64 * 3)()
        st = lib.tvdcn_deform_conv_forward(ctypes.byref(big), None, None, ctypes.c_void_p(16), ctypes.c_void_p(16),
                                           None, None, None, ctypes.c_size_t(0), None)
        assert st == 3 and b"32 bits" in lib.tvdcn_last_error()
        assert lib.tvdcn_set_max_block_elements(0) == 1
        assert lib.tvdcn_set_max_block_elements(2 ** 31) == 1
    finally:
        assert lib.tvdcn_set_max_block_elements(2 ** 31 - 1) == 0
    assert lib.tvdcn_deform_conv_forward_workspace_size(ctypes.byref(big)) == fw


CPP_CALLER = os.path.join(ROOT, "tests", "cpp", "cpp_api_caller.cpp")


@pytest.fixture(scope="module")
def cpp_caller_output(tmp_path_factory):
    """builds tests/cpp/cpp_api_caller.cpp against include/tvdcn_ops.h and tvdcn_amd/_C.so (g++, torch's
    headers and libraries), runs it, returns {name: values}"""
    import subprocess
    from tvdcn_amd import _build
    tdir, incs = _build._torch_paths()
    libdir = os.path.join(tdir, "lib")
    exe = str(tmp_path_factory.mktemp("cpp_api") / "caller")
    cmd = ["g++", "-O1", "-std=c++17", f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
           "-I", os.path.join(ROOT, "include")]
    for i in incs:
        cmd += ["-isystem", i]
    cmd += [CPP_CALLER, "-o", exe, os.path.join(ROOT, "tvdcn_amd", "_C.so"), "-L", libdir, "-lc10", "-ltorch",
            "-ltorch_cpu",
            f"-Wl,-rpath,{libdir}", f"-Wl,-rpath,{os.path.join(ROOT, 'tvdcn_amd')}"]
    subprocess.run(cmd, check=True, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    proc = subprocess.run([exe], stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, timeout=120)
    assert proc.returncode == 0, proc.stderr[-2000:]
    out = {}
    for line in proc.stdout.splitlines():
        name, *vals = line.split()
        out[name] = vals
    return out


def _filled(shape, phase):
    n = 1
    for v in shape:
        n *= v
    return torch.sin(torch.arange(n, dtype=torch.float32) * 0.37 + phase).reshape(shape)


def test_cpp_api_exports_the_reference_symbols():
    """The C++ API's functions have the reference's mangled names (namespace, name, argument types):
    every public tvdcn:: function the reference's own build exports (its CPU kernels' internals aside),
    _C.so exports too, so C++ code linked against the reference links against this library."""
    import subprocess
    if not oracle.have_reference():
        pytest.skip("reference CPU build (oracle/_ref) not available")

    def exported(path):
        out = subprocess.run(["nm", "-D", "--defined-only", path], stdout=subprocess.PIPE, text=True,
                             check=True).stdout
        return {ln.split()[-1] for ln in out.splitlines() if ln.split() and ln.split()[-1].startswith("_ZN5tvdcn")}

    ref = {s for s in exported(oracle.REF_LIB) if not s.startswith("_ZN5tvdcn3ops3cpu")}
    ours = exported(os.path.join(ROOT, "tvdcn_amd", "_C.so"))
    assert len(ref) == 26
    assert ref <= ours, sorted(ref - ours)


def test_cpp_api_caller(cpp_caller_output):
    """A C++ program calling tvdcn::ops (include/tvdcn_ops.h) on host tensors gets what the Python API
    computes from the same inputs: forward (int and SymInt argument forms), the backward schema, a
    transposed op with output_padding, default arguments, and the library information."""
    out = cpp_caller_output
    val = lambda name: torch.tensor([float(v) for v in out[name]], dtype=torch.float64)
    assert int(out["cuda_version"][0]) == tvdcn.cuda_version()
    assert out["cuda_arch_flags"] == tvdcn.cuda_arch_list()
    x, w, b = _filled((2, 4, 5, 6), 0.1), _filled((3, 4, 3, 3), 0.2), _filled((3,), 0.3)
    off, msk = _filled((2, 36, 5, 6), 0.4) * 1.5, _filled((2, 9, 5, 6), 0.5).abs()
    y = tvdcn.deform_conv2d(x, w, off, msk, b, stride=1, padding=1, dilation=1)
    close = lambda name, t: torch.allclose(val(name), t.detach().double().flatten(), rtol=1e-6, atol=1e-6)
    assert close("conv2d", y) and close("conv2d_symint", y)
    gy = _filled(tuple(y.shape), 0.6)
    grads = torch.ops.tvdcn._deform_conv2d_backward(gy, x, w, off, msk, b, [1, 1], [1, 1], [1, 1], 1)
    for name, g in zip(("input", "weight", "offset", "mask", "bias"), grads):
        assert close(f"conv2d_grad_{name}", g), name
    x1, w1, off1 = _filled((2, 4, 7), 0.7), _filled((4, 2, 3), 0.8), _filled((2, 3, 7), 0.9)
    assert close("transpose1d", tvdcn.deform_conv_transpose1d(x1, w1, off1, None, None, stride=2, padding=1,
                                                                output_padding=1))
    x3, w3, off3 = _filled((1, 2, 3, 4, 4), 1.0), _filled((2, 2, 2, 2, 2), 1.1), _filled((1, 24, 2, 3, 3), 1.2)
    assert close("conv3d_defaults", tvdcn.deform_conv3d(x3, w3, off3))
