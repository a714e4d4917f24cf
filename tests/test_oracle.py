"""CPU tests that pin the float64 oracle (oracle/deform_oracle.c).

* against the golden fixtures made by the reference's own CPU build (tests/golden);
* against the reference build directly, when oracle/_ref is present;
* against what the mathematics fixes, independently of the reference:
  zero offsets + unit mask == torch.nn.functional.conv{N}d / conv_transpose{N}d
  (forward and all gradients), a whole-pixel offset == convolution of the shifted
  input, linearity in the mask, block-diagonal groups, central finite differences
  of the oracle's own forward (pins every backward formula: a dropped term, a sign
  or a swapped index shows up as a mismatch), and torch.softmax for mask_softmax.
"""
import glob
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle
from helpers import make_case, rel_err, rounded_position_offsets

GOLDEN = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "*.npz")))
NAMES = ("input", "weight", "offset", "mask", "bias")
GNAMES = ("g_input", "g_weight", "g_offset", "g_mask", "g_bias")


def load_fixture(path):
    z = np.load(path, allow_pickle=False)
    t = {k: torch.from_numpy(z[k]) for k in z.files}
    return t


def fixture_kwargs(t):
    return dict(stride=t["stride"].tolist(), padding=t["padding"].tolist(), dilation=t["dilation"].tolist(),
                groups=int(t["groups"]), transposed=bool(int(t["transposed"])),
                output_padding=t["output_padding"].tolist())


def tol_for(dtype):
    return {torch.float64: (1e-10, 1e-10), torch.float32: (2e-6, 2e-5), torch.float16: (5e-3, 1e-2)}[dtype]


@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p)[:-4] for p in GOLDEN])
def test_oracle_matches_reference_fixtures(path):
    t = load_fixture(path)
    dim = int(t["dim"])
    kw = fixture_kwargs(t)
    unb = bool(int(t["unbatched"]))
    args = [t.get(n) for n in NAMES]
    gout = t["grad_out"]
    if unb:   # the oracle takes batched tensors
        args = [a.unsqueeze(0) if (a is not None and i in (0, 2, 3)) else a for i, a in enumerate(args)]
        gout = gout.unsqueeze(0)
    dtype = t["input"].dtype
    if dtype != torch.float64 and args[2] is not None:
        # The reference forms each sample position y + offset in the input's type (c10::Half or
        # float arithmetic, cpu/deform_conv2d_common_kernels.cpp:407-411): floor() can then land on
        # the neighbouring cell (its own fp16 grad_offset is ~13% (L2) from the value at the exact
        # positions on the float16 fixture); the oracle samples at the same rounded positions
        geo = dict(dim=dim, weight=args[1], stride=kw["stride"], padding=kw["padding"], dilation=kw["dilation"])
        args[2] = rounded_position_offsets(geo, args[2], dtype)
    args = [None if a is None else a.double() for a in args]
    out = oracle.forward(dim, *args, **kw)
    grads = oracle.backward(dim, gout.double(), *args, **kw)
    tf, tb = tol_for(dtype)
    ref_out = t["out"].unsqueeze(0) if unb else t["out"]
    assert rel_err(out, ref_out) < tf
    for gname, g, a in zip(GNAMES, grads, args):
        if a is None:
            assert gname not in t
            continue
        ref = t[gname].unsqueeze(0) if (unb and gname in ("g_input", "g_offset", "g_mask")) else t[gname]
        assert rel_err(g, ref) < tb, gname


def test_fixture_count():
    assert len(GOLDEN) >= 40


@pytest.mark.skipif(not os.path.exists(oracle.REF_LIB), reason="reference CPU build (oracle/_ref) not built")
@pytest.mark.parametrize("dim,transposed", [(1, False), (2, False), (3, False), (1, True), (2, True), (3, True)])
def test_oracle_matches_reference_build_random(dim, transposed):
    """fresh random cases (larger channel counts, og != mg) straight through the reference build"""
    case = make_case(dim, transposed, batch=3, cin=8, cout=12, groups=2, og=4, mg=2, seed=77 + dim,
                     in_size={1: [9], 2: [6, 7], 3: [4, 5, 4]}[dim])
    x, w, o, m, b = (case[n] for n in NAMES)
    s, p, d, op, G = case["stride"], case["padding"], case["dilation"], case["output_padding"], case["groups"]
    gout = torch.rand(case["out_shape"], dtype=torch.float64, generator=torch.Generator().manual_seed(3))
    name = f"deform_conv_transpose{dim}d" if transposed else f"deform_conv{dim}d"
    params = [s, p, op, d, G] if transposed else [s, p, d, G]
    ref, rg = oracle.run_reference([{"op": name, "args": [x, w, o, m, b] + params},
                                    {"op": f"_{name}_backward", "args": [gout, x, w, o, m, b] + params}])
    kw = dict(stride=s, padding=p, dilation=d, groups=G, transposed=transposed, output_padding=op)
    assert rel_err(oracle.forward(dim, x, w, o, m, b, **kw), ref) < 1e-12
    for g, r in zip(oracle.backward(dim, gout, x, w, o, m, b, **kw), rg):
        assert rel_err(g, r) < 1e-12


def _near_integer_offsets(shape, seed):
    """float32 offsets one float32 step from an integer (k = -2 .. 2), on the side of k - 1 or k + 1: a
    position base + offset then lies within half a float32 step of the integer base + k, so its float32
    rounding is that integer while the exact value is not; a third of the offsets stay random"""
    g = torch.Generator().manual_seed(seed)
    k = torch.randint(-2, 3, shape, generator=g).float()
    side = torch.where(torch.rand(shape, generator=g) < 0.5, k - 1, k + 1)
    near = torch.nextafter(k, side)
    rand = (torch.rand(shape, generator=g) - 0.5) * 4
    return torch.where(torch.rand(shape, generator=g) < 1 / 3, rand, near)


@pytest.mark.skipif(not os.path.exists(oracle.REF_LIB), reason="reference CPU build (oracle/_ref) not built")
@pytest.mark.parametrize("dim,transposed", [(1, False), (2, False), (3, False), (1, True), (2, True), (3, True)])
def test_float32_position_model_matches_reference_build(dim, transposed):
    """The reference's float32 path forms a sampling position as integer base + float offset, rounded
    once to float32 (cpu/deform_conv2d_common_kernels.cpp:407-411; the CUDA twin
    cuda/deform_conv2d_common_kernels.cu:170-178). Offsets one float32 step from an integer put most
    positions within half a step of a cell boundary: rounded, they sit on the boundary and take the other
    cell and the other one-sided offset derivative. The float64 oracle sampling at those rounded positions
    (helpers.rounded_position_offsets, what the GPU parity tests hand the oracle for float32 runs) must
    match the reference's own float32 results at float32 accuracy, and the oracle at the exact positions
    must not (the model is what closes the gap)."""
    case = make_case(dim, transposed, batch=2, cin=8, cout=6, groups=1, og=2, mg=1, seed=131 + dim,
                     in_size={1: [23], 2: [9, 11], 3: [5, 6, 7]}[dim], dtype=torch.float32)
    case["offset"] = _near_integer_offsets(case["offset"].shape, 17 + dim)
    x, w, o, m, b = (case[n] for n in NAMES)
    s, p, d, op, G = case["stride"], case["padding"], case["dilation"], case["output_padding"], case["groups"]
    gout = torch.rand(case["out_shape"], generator=torch.Generator().manual_seed(5)).float()
    name = f"deform_conv_transpose{dim}d" if transposed else f"deform_conv{dim}d"
    params = [s, p, op, d, G] if transposed else [s, p, d, G]
    ref, rg = oracle.run_reference([{"op": name, "args": [x, w, o, m, b] + params},
                                    {"op": f"_{name}_backward", "args": [gout, x, w, o, m, b] + params}])
    kw = dict(stride=s, padding=p, dilation=d, groups=G, transposed=transposed, output_padding=op)
    x64, w64, m64, b64, g64 = (t.double() for t in (x, w, m, b, gout))
    o_model = rounded_position_offsets(case, o.double(), torch.float32)
    moved = float((o_model != o.double()).double().mean())
    assert moved > 0.3, f"only {moved:.2f} of the positions round onto a boundary"
    out = oracle.forward(dim, x64, w64, o_model, m64, b64, **kw)
    grads = oracle.backward(dim, g64, x64, w64, o_model, m64, b64, **kw)
    assert rel_err(out, ref) < 1e-5
    for gname, gr, r in zip(GNAMES, grads, rg):
        assert rel_err(gr, r) < 1e-4, gname
    exact = oracle.backward(dim, g64, x64, w64, o.double(), m64, b64, **kw)
    assert rel_err(exact[2], rg[2]) > 1e-2, "the exact positions should take other one-sided derivatives"


CONV = {1: F.conv1d, 2: F.conv2d, 3: F.conv3d}
CONVT = {1: F.conv_transpose1d, 2: F.conv_transpose2d, 3: F.conv_transpose3d}


@pytest.mark.parametrize("dim,transposed", [(1, False), (2, False), (3, False), (1, True), (2, True), (3, True)])
def test_zero_offset_unit_mask_is_plain_convolution(dim, transposed):
    case = make_case(dim, transposed, batch=2, cin=4, cout=6, groups=2, seed=5 + dim)
    x, w, o, m, b = (case[n] for n in NAMES)
    o = torch.zeros_like(o)
    m = torch.ones_like(m)
    s, p, d, op, G = case["stride"], case["padding"], case["dilation"], case["output_padding"], case["groups"]
    kw = dict(stride=s, padding=p, dilation=d, groups=G, transposed=transposed, output_padding=op)
    out = oracle.forward(dim, x, w, o, m, b, **kw)
    xr, wr, br = (t.clone().requires_grad_(True) for t in (x, w, b))
    if transposed:
        ref = CONVT[dim](xr, wr, br, stride=s, padding=p, output_padding=op, groups=G, dilation=d)
    else:
        ref = CONV[dim](xr, wr, br, stride=s, padding=p, dilation=d, groups=G)
    assert rel_err(out, ref) < 1e-12
    gout = torch.rand(ref.shape, dtype=torch.float64, generator=torch.Generator().manual_seed(1))
    ref.backward(gout)
    gx, gw, _, _, gb = oracle.backward(dim, gout, x, w, o, m, b, **kw)
    assert rel_err(gx, xr.grad) < 1e-12
    assert rel_err(gw, wr.grad) < 1e-12
    assert rel_err(gb, br.grad) < 1e-12


def test_no_offset_no_mask_is_plain_convolution():
    case = make_case(2, False, batch=2, cin=4, cout=6, deformable=False, modulated=False, seed=9)
    x, w, _, _, b = (case[n] for n in NAMES)
    s, p, d = case["stride"], case["padding"], case["dilation"]
    out = oracle.forward(2, x, w, None, None, b, stride=s, padding=p, dilation=d)
    assert rel_err(out, F.conv2d(x, w, b, stride=s, padding=p, dilation=d)) < 1e-12


def test_whole_pixel_offset_is_shifted_convolution():
    """offset (dy, dx) = (1, -2) on every tap and pixel == convolving the input shifted by that amount"""
    g = torch.Generator().manual_seed(4)
    x = torch.rand(2, 3, 9, 10, generator=g, dtype=torch.float64)
    w = torch.rand(4, 3, 3, 3, generator=g, dtype=torch.float64)
    out_hw = (7, 8)
    off = torch.zeros(2, 18, *out_hw, dtype=torch.float64)
    off[:, 0::2] = 1.0     # dy
    off[:, 1::2] = -2.0    # dx
    out = oracle.forward(2, x, w, off, None, None)
    shifted = torch.zeros_like(x)
    # sample at (y + 1, x - 2): shifted[y, x] = x[y + 1, x - 2]
    shifted[:, :, :-1, 2:] = x[:, :, 1:, :-2]
    assert rel_err(out, F.conv2d(shifted, w)) < 1e-12


def test_mask_linearity():
    case = make_case(2, False, batch=2, cin=4, cout=6, seed=11)
    x, w, o, m, b = (case[n] for n in NAMES)
    kw = dict(stride=case["stride"], padding=case["padding"], dilation=case["dilation"])
    a = oracle.forward(2, x, w, o, m, b, **kw) - b.view(1, -1, 1, 1)
    a3 = oracle.forward(2, x, w, o, 3 * m, b, **kw) - b.view(1, -1, 1, 1)
    assert rel_err(a3, 3 * a) < 1e-12


def test_groups_are_block_diagonal():
    case = make_case(2, False, batch=2, cin=4, cout=6, groups=2, og=2, mg=2, seed=12)
    x, w, o, m, b = (case[n] for n in NAMES)
    kw = dict(stride=case["stride"], padding=case["padding"], dilation=case["dilation"])
    out = oracle.forward(2, x, w, o, m, b, groups=2, **kw)
    # offset group g covers input channels [2g, 2g+2) == conv group g; same for the mask groups here
    kn = 6
    halves = []
    for gi in range(2):
        halves.append(oracle.forward(2, x[:, 2 * gi:2 * gi + 2], w[3 * gi:3 * gi + 3], o[:, gi * 2 * kn:(gi + 1) * 2 * kn],
                                     m[:, gi * kn:(gi + 1) * kn], b[3 * gi:3 * gi + 3], **kw))
    assert rel_err(out, torch.cat(halves, 1)) < 1e-12


@pytest.mark.parametrize("dim,transposed", [(1, False), (2, False), (3, False), (1, True), (2, True), (3, True)])
def test_backward_matches_finite_differences(dim, transposed):
    """<grad_i, v_i> == d/de <gout, f(args + e v_i)> for a random direction v_i of each input"""
    case = make_case(dim, transposed, batch=2, cin=4, cout=4, groups=2, og=2, mg=1, seed=21 + dim,
                     in_size={1: [6], 2: [5, 6], 3: [4, 4, 5]}[dim])
    args = [case[n] for n in NAMES]
    kw = dict(stride=case["stride"], padding=case["padding"], dilation=case["dilation"], groups=case["groups"],
              transposed=transposed, output_padding=case["output_padding"])
    gen = torch.Generator().manual_seed(99)
    gout = torch.rand(case["out_shape"], dtype=torch.float64, generator=gen)
    grads = oracle.backward(dim, gout, *args, **kw)
    eps = 1e-6
    for i, (a, gr) in enumerate(zip(args, grads)):
        v = torch.rand(a.shape, dtype=torch.float64, generator=gen) - 0.5
        plus = list(args)
        minus = list(args)
        plus[i] = a + eps * v
        minus[i] = a - eps * v
        fd = ((oracle.forward(dim, *plus, **kw) - oracle.forward(dim, *minus, **kw)) * gout).sum() / (2 * eps)
        an = (gr * v).sum()
        assert abs(fd - an) <= 1e-6 * max(1.0, abs(an)), (NAMES[i], float(fd), float(an))


@pytest.mark.parametrize("K,shape", [(5, (3, 20, 33)), (16, (2, 32, 6, 7)), (27, (2, 27, 3, 4, 5)), (49, (1, 98, 5, 5))])
def test_oracle_mask_softmax(K, shape):
    g = torch.Generator().manual_seed(2)
    x = torch.randn(*shape, generator=g, dtype=torch.float64) * 3
    y = oracle.mask_softmax_forward(x, K)
    ref = torch.softmax(x.view(shape[0], shape[1] // K, K, -1), dim=2).view(shape)
    assert rel_err(y, ref) < 1e-14
    gy = torch.randn(*shape, generator=g, dtype=torch.float64)
    xr = x.clone().requires_grad_(True)
    torch.softmax(xr.view(shape[0], shape[1] // K, K, -1), dim=2).view(shape).backward(gy)
    assert rel_err(oracle.mask_softmax_backward(y, gy, K), xr.grad) < 1e-13
