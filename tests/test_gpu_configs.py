"""GPU parity at the BASELINE.json configurations' full sizes and on the golden fixtures.

Full-size checks compare the HIP kernels with the reference's own CPU implementation
(oracle/_ref, tvdcn 1.1.0 compiled from its sources) run on the same seeded fp32
inputs: forward within 1e-5 and every gradient within 1e-4 (norm-wise: max of the
relative L2 error and max-abs error / max |ref|). float16 runs are compared with the
reference's own float16 path, bfloat16 runs (no reference path) with the fp32 reference
evaluated on the same rounded inputs, both within 1e-2. Inputs follow the configs'
distributions (seed 1000 + config number).

The golden fixtures (tests/golden, written by the reference build) are replayed through
the public API on the GPU.
"""
import glob
import os

import numpy as np
import pytest
import torch

import tvdcn
from oracle import oracle
from helpers import rel_err

pytestmark = pytest.mark.gpu
DEV = "cuda"
HAVE_REF = oracle.have_reference()


def kaiming(shape, fan_in, g):
    return torch.randn(*shape, generator=g) * (2.0 / fan_in) ** 0.5


def config(n):
    """tensors + params of BASELINE.json configs[n-1] (CPU, fp32)"""
    g = torch.Generator().manual_seed(1000 + n)
    if n == 2:
        x = torch.randn(8, 256, 64, 64, generator=g)
        w = kaiming((256, 256, 3, 3), 2304, g)
        o = torch.randn(8, 18, 64, 64, generator=g) * 2
        m = torch.sigmoid(torch.randn(8, 9, 64, 64, generator=g))
        b = torch.zeros(256)
        return dict(dim=2, tr=False, x=x, w=w, o=o, m=m, b=b, s=[1, 1], p=[1, 1], d=[1, 1], op=[0, 0], G=1)
    if n == 3:
        x = torch.randn(16, 512, 4096, generator=g)
        w = kaiming((512, 512, 5), 2560, g)
        o = torch.randn(16, 20, 4096, generator=g) * 3
        logits = torch.randn(16, 20, 4096, generator=g)
        m = torch.softmax(logits.view(16, 4, 5, 4096), 2).view(16, 20, 4096)
        return dict(dim=1, tr=False, x=x, w=w, o=o, m=m, b=None, s=[1], p=[2], d=[1], op=[0], G=1, logits=logits,
                    kn=5)
    if n == 4:
        x = torch.randn(2, 64, 16, 56, 56, generator=g)
        w = kaiming((64, 64, 3, 3, 3), 1728, g)
        o = torch.randn(2, 81, 16, 56, 56, generator=g) * 1.5
        m = torch.sigmoid(torch.randn(2, 27, 16, 56, 56, generator=g))
        return dict(dim=3, tr=False, x=x, w=w, o=o, m=m, b=None, s=[1, 1, 1], p=[1, 1, 1], d=[1, 1, 1],
                    op=[0, 0, 0], G=1)
    if n == 5:
        # offsets / masks on the input grid (32 x 32): tvdcn rejects the output-grid shapes
        x = torch.randn(8, 256, 32, 32, generator=g)
        w = kaiming((256, 128, 4, 4), 128 * 16, g)
        o = torch.randn(8, 64, 32, 32, generator=g)
        logits = torch.randn(8, 32, 32, 32, generator=g)
        m = torch.softmax(logits.view(8, 2, 16, 32, 32), 2).view(8, 32, 32, 32)
        return dict(dim=2, tr=True, x=x, w=w, o=o, m=m, b=None, s=[2, 2], p=[1, 1], d=[1, 1], op=[0, 0], G=1,
                    logits=logits, kn=16)
    raise ValueError(n)


def reference(c, gout):
    """forward and the five gradients from the reference's CPU build (child process)"""
    dim = c["dim"]
    args = [c["x"], c["w"], c["o"], c["m"], c["b"]]
    name = f"deform_conv_transpose{dim}d" if c["tr"] else f"deform_conv{dim}d"
    params = [c["s"], c["p"], c["op"], c["d"], c["G"]] if c["tr"] else [c["s"], c["p"], c["d"], c["G"]]
    out, grads = oracle.run_reference([{"op": name, "args": args + params},
                                       {"op": f"_{name}_backward", "args": [gout] + args + params}])
    return out, grads


def ours(c, gout, dtype):
    ts = [t.to(DEV, dtype).requires_grad_(True) if t is not None else None
          for t in (c["x"], c["w"], c["o"], c["m"], c["b"])]
    dim = c["dim"]
    if c["tr"]:
        out = getattr(tvdcn, f"deform_conv_transpose{dim}d")(*ts, c["s"], c["p"], c["op"], c["d"], c["G"])
    else:
        out = getattr(tvdcn, f"deform_conv{dim}d")(*ts, c["s"], c["p"], c["d"], c["G"])
    out.backward(gout.to(DEV, dtype))
    torch.cuda.synchronize()
    return out, [t.grad if t is not None else None for t in ts]


def upstream(c, n):
    g = torch.Generator().manual_seed(2000 + n)
    dim = c["dim"]
    if c["tr"]:
        sz = [(c["x"].shape[2 + i] - 1) * c["s"][i] - 2 * c["p"][i] + c["d"][i] * (c["w"].shape[2 + i] - 1) + 1 +
              c["op"][i] for i in range(dim)]
        cout = c["w"].shape[1] * c["G"]
    else:
        sz = [(c["x"].shape[2 + i] + 2 * c["p"][i] - (c["d"][i] * (c["w"].shape[2 + i] - 1) + 1)) // c["s"][i] + 1
              for i in range(dim)]
        cout = c["w"].shape[0]
    return torch.randn(c["x"].shape[0], cout, *sz, generator=g)


@pytest.mark.skipif(not HAVE_REF, reason="reference CPU build (oracle/_ref) not available")
@pytest.mark.parametrize("n", [2, 3, 4, 5])
def test_full_config_fp32_matches_reference(n):
    c = config(n)
    gout = upstream(c, n)
    out, grads = ours(c, gout, torch.float32)
    ref_out, ref_grads = reference(c, gout)
    e = rel_err(out, ref_out)
    print(f"cfg{n} forward rel err {e:.2e}", flush=True)
    assert e < 1e-5
    for name, gr, r in zip(("input", "weight", "offset", "mask", "bias"), grads, ref_grads):
        if r is None:
            continue
        e = rel_err(gr, r)
        print(f"cfg{n} grad_{name} rel err {e:.2e}", flush=True)
        assert e < 1e-4, name


@pytest.mark.skipif(not HAVE_REF, reason="reference CPU build (oracle/_ref) not available")
@pytest.mark.parametrize("n", [3, 5])
def test_full_config_fused_softmax_matches_reference(n):
    """Configs 3 and 5 as bench.py times them: the mask is the softmax of the logits over each mask
    group's taps, applied in the kernels' mask load (tvdcn::deform_conv_mask_activation, what
    PackedDeformConv*(mask_activation="softmax") runs), and its gradient flows to the logits. Against
    the reference's CPU build run on mask = mask_softmax(logits) (its own composition), the mask
    gradient carried to the logits through the softmax in float64: forward within 1e-5, every gradient
    (the logits' included) within 1e-4."""
    from tvdcn.ops.deform_conv import _deform_conv_mask_activation
    c = config(n)
    gout = upstream(c, n)
    ref_out, ref_grads = reference(c, gout)
    dim = c["dim"]
    ts = [t.to(DEV).requires_grad_(True) if t is not None else None
          for t in (c["x"], c["w"], c["o"], c["logits"], c["b"])]
    out = _deform_conv_mask_activation(ts[0], ts[1], ts[2], ts[3], ts[4], c["s"], c["p"], c["op"], c["d"], c["G"],
                                       c["tr"], 2, 0.0)
    out.backward(gout.to(DEV))
    torch.cuda.synchronize()
    e = rel_err(out, ref_out)
    print(f"cfg{n} fused softmax forward rel err {e:.2e}", flush=True)
    assert e < 1e-5
    # d loss / d logits = y * (g - sum_taps g * y), y = softmax over each group's taps (float64)
    B, ch = c["logits"].shape[:2]
    y = torch.softmax(c["logits"].double().view(B, ch // c["kn"], c["kn"], -1), 2)
    gm = ref_grads[3].double().view(y.shape)
    ref_glogits = (y * (gm - (gm * y).sum(2, keepdim=True))).view(c["logits"].shape)
    for name, t, r in zip(("input", "weight", "offset", "logits"), ts, (*ref_grads[:3], ref_glogits)):
        e = rel_err(t.grad, r)
        print(f"cfg{n} fused softmax grad_{name} rel err {e:.2e}", flush=True)
        assert e < 1e-4, name


@pytest.mark.skipif(not HAVE_REF, reason="reference CPU build (oracle/_ref) not available")
@pytest.mark.parametrize("dtype", [torch.bfloat16])
def test_cfg5_bfloat16_matches_reference(dtype):
    """bfloat16 has no reference path (its dispatch excludes the type): against the float32 reference
    on the same rounded inputs, within 1e-2 (float16: test_cfg5_float16_matches_reference_float16_path)."""
    c = config(5)
    gout = upstream(c, 5)
    rounded = {k: (v.to(dtype).float() if isinstance(v, torch.Tensor) else v) for k, v in c.items()}
    out, grads = ours(rounded, gout.to(dtype).float(), dtype)
    ref_out, ref_grads = reference(rounded, gout.to(dtype).float())
    assert rel_err(out, ref_out) < 1e-2
    for gr, r in zip(grads, ref_grads):
        if r is not None:
            assert rel_err(gr, r) < 1e-2


@pytest.mark.skipif(not HAVE_REF, reason="reference CPU build (oracle/_ref) not available")
def test_cfg5_float16_matches_reference_float16_path():
    """cfg5 in float16 against the reference's own float16 path on the same half inputs: its c10::Half
    arithmetic rounds every intermediate (sampling positions included) to half precision; the kernels
    round the positions the same way and compute the rest in float32. Forward and every gradient
    within 1e-2."""
    c = config(5)
    gout = upstream(c, 5).half()
    half = {k: (v.half() if isinstance(v, torch.Tensor) else v) for k, v in c.items()}
    ref_out, ref_grads = reference(half, gout)
    out, grads = ours({k: (v.float() if isinstance(v, torch.Tensor) else v) for k, v in half.items()},
                      gout.float(), torch.float16)
    e = rel_err(out, ref_out.double())
    print(f"cfg5 float16 forward rel err {e:.2e}", flush=True)
    assert e < 1e-2
    for name, gr, r in zip(("input", "weight", "offset", "mask", "bias"), grads, ref_grads):
        if r is None:
            continue
        e = rel_err(gr, r.double())
        print(f"cfg5 float16 grad_{name} rel err {e:.2e}", flush=True)
        assert e < 1e-2, name


def test_cfg2_zero_offset_is_miopen_conv():
    """size-independent closed form at full size: zero offsets, unit mask == torch's own conv2d"""
    c = config(2)
    x, w = c["x"].to(DEV), c["w"].to(DEV)
    out = tvdcn.deform_conv2d(x, w, torch.zeros_like(c["o"]).to(DEV), torch.ones_like(c["m"]).to(DEV),
                                  None, 1, 1, 1)
    ref = torch.nn.functional.conv2d(x.double(), w.double(), padding=1)
    assert rel_err(out, ref) < 1e-5


GOLDEN = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "*.npz")))


@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p)[:-4] for p in GOLDEN])
def test_golden_fixture_on_gpu(path):
    z = np.load(path, allow_pickle=False)
    t = {k: torch.from_numpy(z[k]) for k in z.files}
    dim, tr, G = int(t["dim"]), bool(int(t["transposed"])), int(t["groups"])
    s, p, d, op = (t[k].tolist() for k in ("stride", "padding", "dilation", "output_padding"))
    dtype = t["input"].dtype
    names = ("input", "weight", "offset", "mask", "bias")
    ts = [t[n].to(DEV).requires_grad_(True) if n in t else None for n in names]
    if tr:
        out = getattr(tvdcn, f"deform_conv_transpose{dim}d")(*ts, s, p, op, d, G)
    else:
        out = getattr(tvdcn, f"deform_conv{dim}d")(*ts, s, p, d, G)
    out.backward(t["grad_out"].to(DEV))
    torch.cuda.synchronize()
    tf, tb = {torch.float64: (1e-9, 1e-9), torch.float32: (1e-5, 1e-4), torch.float16: (1e-2, 1e-2)}[dtype]
    assert rel_err(out, t["out"]) < tf
    for n, ten in zip(names, ts):
        key = "g_" + n
        if ten is None:
            continue
        assert rel_err(ten.grad, t[key]) < tb, n


@pytest.mark.parametrize("transposed", [False, True])
def test_empty_batch(transposed):
    x = torch.zeros(0, 4, 6, 6, device=DEV, requires_grad=True)
    if transposed:
        w = torch.rand(4, 3, 3, 3, device=DEV, requires_grad=True)
        o = torch.zeros(0, 18, 6, 6, device=DEV, requires_grad=True)
        out = tvdcn.deform_conv_transpose2d(x, w, o, None, torch.rand(3, device=DEV))
    else:
        w = torch.rand(5, 4, 3, 3, device=DEV, requires_grad=True)
        o = torch.zeros(0, 18, 4, 4, device=DEV, requires_grad=True)
        out = tvdcn.deform_conv2d(x, w, o, None, torch.rand(5, device=DEV))
    assert out.shape[0] == 0
    out.sum().backward()
    torch.cuda.synchronize()
    assert w.grad.abs().sum().item() == 0.0 and x.grad.shape == x.shape


def test_empty_batch_wide_gemm_side():
    """An empty batch whose GEMM side takes the windowed weight gradient (>= 16 rows): its split
    count once divided by zero on the host."""
    x = torch.zeros(0, 32, 6, 6, device=DEV, requires_grad=True)
    w = torch.rand(32, 32, 3, 3, device=DEV, requires_grad=True)
    o = torch.zeros(0, 18, 4, 4, device=DEV, requires_grad=True)
    m = torch.zeros(0, 9, 4, 4, device=DEV, requires_grad=True)
    out = tvdcn.deform_conv2d(x, w, o, m)
    out.sum().backward()
    torch.cuda.synchronize()
    assert out.shape == (0, 32, 4, 4) and w.grad.abs().sum().item() == 0.0


def test_mask_softmax_cfg3_shape_and_half():
    g = torch.Generator().manual_seed(3)
    logits = torch.randn(16, 20, 4096, generator=g)
    for dtype, tol in [(torch.float32, 1e-6), (torch.float16, 1e-2), (torch.bfloat16, 1e-2)]:
        x = logits.to(DEV, dtype).requires_grad_(True)
        y = tvdcn.mask_softmax1d(x, 5)
        ref = torch.softmax(logits.to(dtype).double().view(16, 4, 5, 4096), 2).view(16, 20, 4096)
        assert rel_err(y, ref) < tol
        gy = torch.randn(16, 20, 4096, generator=g)
        y.backward(gy.to(DEV, dtype))
        xr = logits.to(dtype).double().requires_grad_(True)
        torch.softmax(xr.view(16, 4, 5, 4096), 2).view(16, 20, 4096).backward(gy.double())
        assert rel_err(x.grad, xr.grad) < max(tol, 1e-5)
