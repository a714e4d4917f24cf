"""GPU parity of the windowed kernels' less common paths, against the float64 oracle.

* offsets far larger than the window margin: bilinear corners outside the LDS window
  take the general path (global reads in the forward and weight gradient, global
  atomics in the data gradient);
* a GEMM side that is not a multiple of 16 rows (zero-padded rows in the data gradient);
* a non-finite upstream gradient: the data gradient's fixed-point window cannot bound
  the pass and falls back to global float atomics, so inf / nan propagate as in the
  reference.
"""
import itertools

import pytest
import torch

import tvdcn
from oracle import oracle
from helpers import make_case, oracle_offsets, rel_err
from test_gpu_parity import TOL, check, run_gpu, run_oracle

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dim,transposed", [(2, False), (2, True), (1, False), (3, False)])
def test_offsets_beyond_window_fp32(dim, transposed):
    in_size = {1: [300], 2: [40, 36], 3: [6, 12, 12]}[dim]
    case = make_case(dim, transposed, batch=2, cin=32, cout=64, kernel=[3] * dim, stride=[1] * dim,
                     padding=[1] * dim, dilation=[1] * dim, in_size=in_size, out_pad=[0] * dim, seed=500 + dim,
                     offset_scale=12.0)
    check(case, torch.float32)


def test_gemm_side_not_multiple_of_16_fp32():
    case = make_case(2, False, batch=2, cin=32, cout=40, kernel=[3, 3], stride=[1, 1], padding=[1, 1],
                     dilation=[1, 1], in_size=[20, 18], out_pad=[0, 0], seed=510)
    check(case, torch.float32)


def test_nonfinite_grad_out_fp32():
    case = make_case(2, False, batch=2, cin=32, cout=64, kernel=[3, 3], stride=[1, 1], padding=[1, 1],
                     dilation=[1, 1], in_size=[20, 18], out_pad=[0, 0], seed=520)
    g = torch.Generator().manual_seed(521)
    gout = torch.rand(case["out_shape"], generator=g, dtype=torch.float64)
    gout[1, 5, 7, 9] = float("nan")
    _, grads, _ = run_gpu(case, torch.float32, grad_out=gout)
    _, ref_grads = run_oracle(case, gout, torch.float32)
    for name, gr, r in zip(("input", "weight", "offset", "mask", "bias"), grads, ref_grads):
        gr = gr.detach().double().cpu()
        assert torch.equal(torch.isnan(gr), torch.isnan(r)), f"grad_{name}: nan pattern differs"
        assert torch.equal(torch.isinf(gr), torch.isinf(r)), f"grad_{name}: inf pattern differs"
        fin = torch.isfinite(r)
        if fin.any():
            e = rel_err(gr[fin], r[fin])
            assert e < TOL[torch.float32][1], f"grad_{name} rel err {e}"


@pytest.mark.parametrize("dim", [2, 3])
def test_offset_free_nonfinite_input_fp32(dim):
    """Integer sampling (offset None) touches only the sampled pixel: an inf in the input must
    reach exactly the outputs / gradients the reference's integer sampling reaches."""
    in_size = {2: [20, 18], 3: [6, 10, 9]}[dim]
    case = make_case(dim, False, batch=2, cin=32, cout=32, kernel=[3] * dim, stride=[1] * dim, padding=[1] * dim,
                     dilation=[1] * dim, in_size=in_size, out_pad=[0] * dim, seed=530 + dim, deformable=False)
    case["input"] = case["input"].clone()
    case["input"][1, 3][(2,) * dim] = float("inf")
    g = torch.Generator().manual_seed(531)
    gout = torch.rand(case["out_shape"], generator=g, dtype=torch.float64)
    out, grads, _ = run_gpu(case, torch.float32, grad_out=gout)
    ref_out, ref_grads = run_oracle(case, gout, torch.float32)
    for name, gr, r in zip(("output", "input", "weight", "offset", "mask", "bias"), [out] + list(grads), [ref_out] + list(ref_grads)):
        if r is None:
            continue
        gr = gr.detach().double().cpu()
        assert torch.equal(torch.isnan(gr), torch.isnan(r)), f"{name}: nan pattern differs"
        assert torch.equal(torch.isinf(gr), torch.isinf(r)), f"{name}: inf pattern differs"
        fin = torch.isfinite(r)
        if fin.any():
            e = rel_err(gr[fin], r[fin])
            assert e < TOL[torch.float32][1], f"{name} rel err {e}"


@pytest.mark.parametrize("dim", [1, 2, 3])
def test_deformable_nonfinite_input_fp32(dim):
    """An inf in the input under fractional sampling: the offset gradients of the taps whose
    corners hold it are +-inf in the reference's corner sums (nan only where a corner weight
    is zero), and the mask gradient is +-inf; forms that take differences of corners first
    would give inf - inf = nan there."""
    in_size = {1: [40], 2: [20, 18], 3: [6, 10, 9]}[dim]
    case = make_case(dim, False, batch=2, cin=32, cout=32, kernel=[3] * dim, stride=[1] * dim, padding=[1] * dim,
                     dilation=[1] * dim, in_size=in_size, out_pad=[0] * dim, seed=550 + dim)
    case["input"] = case["input"].clone()
    case["input"][1, 3][(2,) * dim] = float("inf")
    g = torch.Generator().manual_seed(551)
    gout = torch.rand(case["out_shape"], generator=g, dtype=torch.float64)
    out, grads, _ = run_gpu(case, torch.float32, grad_out=gout)
    ref_out, ref_grads = run_oracle(case, gout, torch.float32)
    assert torch.isinf(ref_grads[2]).any(), "the inf must reach some offset gradient"
    for name, gr, r in zip(("output", "input", "weight", "offset", "mask", "bias"), [out] + list(grads), [ref_out] + list(ref_grads)):
        if r is None:
            continue
        gr = gr.detach().double().cpu()
        assert torch.equal(torch.isnan(gr), torch.isnan(r)), f"{name}: nan pattern differs"
        assert torch.equal(torch.isinf(gr), torch.isinf(r)), f"{name}: inf pattern differs"
        fin = torch.isfinite(r)
        if fin.any():
            e = rel_err(gr[fin], r[fin])
            assert e < TOL[torch.float32][1], f"{name} rel err {e}"


def test_nonfinite_bound_in_a_later_pass_fp32():
    """25 taps = three passes of the data gradient's window: an inf weight at tap 12 makes only
    the second pass's bound non-finite, so the window flushes what the first pass accumulated
    and the second pass scatters through global atomics."""
    case = make_case(2, False, batch=2, cin=32, cout=32, kernel=[5, 5], stride=[1, 1], padding=[2, 2],
                     dilation=[1, 1], in_size=[20, 18], out_pad=[0, 0], seed=540)
    case["weight"] = case["weight"].clone()
    case["weight"][3, 5, 2, 2] = float("inf")   # tap 12 = (2, 2)
    g = torch.Generator().manual_seed(541)
    gout = torch.rand(case["out_shape"], generator=g, dtype=torch.float64)
    _, grads, _ = run_gpu(case, torch.float32, grad_out=gout)
    _, ref_grads = run_oracle(case, gout, torch.float32)
    for name, gr, r in zip(("input", "weight", "offset", "mask", "bias"), grads, ref_grads):
        gr = gr.detach().double().cpu()
        assert torch.equal(torch.isnan(gr), torch.isnan(r)), f"grad_{name}: nan pattern differs"
        assert torch.equal(torch.isinf(gr), torch.isinf(r)), f"grad_{name}: inf pattern differs"
        fin = torch.isfinite(r)
        if fin.any():
            e = rel_err(gr[fin], r[fin])
            assert e < TOL[torch.float32][1], f"grad_{name} rel err {e}"


def test_many_taps_multi_pass_fp32():
    """25 taps: the window accumulates three passes and is rescaled as the bound grows."""
    case = make_case(2, False, batch=2, cin=32, cout=64, kernel=[5, 5], stride=[1, 1], padding=[2, 2],
                     dilation=[1, 1], in_size=[24, 22], out_pad=[0, 0], seed=545, offset_scale=3.0)
    check(case, torch.float32)


@pytest.mark.parametrize("dim,dtype", [(2, torch.float32), (2, torch.bfloat16), (3, torch.float32)])
def test_channels_last_input(dim, dtype):
    """A channels-last conv input is sampled in place (fp32) or widened in place (half types), and
    its gradient comes back channels-last; forward and gradients against the float64 oracle (and
    the NC<spatial> path's numbers)."""
    in_size = {2: [20, 18], 3: [6, 10, 9]}[dim]
    case = make_case(dim, False, batch=2, cin=32, cout=48, kernel=[3] * dim, stride=[1] * dim, padding=[1] * dim,
                     dilation=[1] * dim, in_size=in_size, out_pad=[0] * dim, seed=560 + dim)
    out, grads, gout = run_gpu(case, dtype)
    ref_out, ref_grads = run_oracle(case, gout, dtype)
    fmt = torch.channels_last if dim == 2 else torch.channels_last_3d
    names = ("input", "weight", "offset", "mask", "bias")
    ts = [case[n].to("cuda:0", dtype) for n in names]
    ts[0] = ts[0].contiguous(memory_format=fmt)
    assert not ts[0].is_contiguous()
    ts = [t.requires_grad_(True) for t in ts]
    fn = getattr(tvdcn, f"deform_conv{dim}d")
    y = fn(*ts, stride=case["stride"], padding=case["padding"], dilation=case["dilation"], groups=case["groups"])
    y.backward(gout.to("cuda:0", dtype))
    torch.cuda.synchronize()
    assert ts[0].grad.is_contiguous(memory_format=fmt)
    tf, tb = TOL[dtype]
    assert rel_err(y, ref_out) < tf
    assert rel_err(y, out) < tf
    for n, t, r, r_nc in zip(names, ts, ref_grads, grads):
        e = rel_err(t.grad, r)
        assert e < tb, f"grad_{n} rel err {e} (oracle)"
        assert rel_err(t.grad, r_nc) < tb, f"grad_{n} (NC<spatial> path)"


@pytest.mark.parametrize("dim,transposed,cin,cout,k,size", [
    (1, False, 32, 256, 5, [300]), (2, False, 32, 160, 2, [20, 18]), (1, True, 256, 32, 3, [150]),
    (2, False, 48, 144, 2, [9, 33])])
def test_weight_gradient_short_passes_fp32(dim, transposed, cin, cout, k, size):
    """Passes of at most 5 taps on GEMM sides above 128 rows take the weight gradient's
    (5 tap slots, 64-pixel chunk) shape; ragged tiles and GEMM sides that are not multiples of
    256 rows included."""
    case = make_case(dim, transposed, batch=2, cin=cin, cout=cout, kernel=[k] * dim, stride=[1] * dim,
                     padding=[1] * dim, dilation=[1] * dim, in_size=size, out_pad=[0] * dim, seed=570 + dim)
    check(case, torch.float32)


def test_layout_copies_through_c_abi():
    """tvdcn_to_channels_last / tvdcn_from_channels_last on the GPU: bit-exact permutations
    (ragged sizes, off the 32 x 32 tile of the copy kernels), and their round trip."""
    import ctypes
    from tvdcn import extension
    lib = ctypes.CDLL(extension.HIP_LIB_PATH)
    for fn in (lib.tvdcn_to_channels_last, lib.tvdcn_from_channels_last):
        fn.restype = ctypes.c_int
        fn.argtypes = [ctypes.c_int32, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p,
                       ctypes.c_void_p, ctypes.c_void_p]
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for B, C, S in ((3, 37, 1000), (1, 256, 4096), (2, 5, 33)):
        print(f"layout copy B={B} C={C} S={S}", flush=True)
        x = torch.randn(B, C, S, device="cuda:0")
        cl = torch.empty(B, S, C, device="cuda:0")
        back = torch.empty_like(x)
        assert lib.tvdcn_to_channels_last(0, B, C, S, x.data_ptr(), cl.data_ptr(), stream) == 0
        assert lib.tvdcn_from_channels_last(0, B, C, S, cl.data_ptr(), back.data_ptr(), stream) == 0
        torch.cuda.synchronize()
        assert torch.equal(cl, x.permute(0, 2, 1))
        assert torch.equal(back, x)


@pytest.mark.parametrize("dim", [1, 2, 3])
def test_forward_copy_kept_for_backward(dim):
    """float32 NC<spatial> inputs with the opt-in kept copy (set_keep_channels_last_copy): the
    forward's channels-last copy serves the backward, and
    grad_input comes back in the input's own (NC<spatial>) order with the numbers of the
    backward op called on the original input, and of the float64 oracle."""
    in_size = {1: [70], 2: [20, 18], 3: [6, 10, 9]}[dim]
    case = make_case(dim, False, batch=2, cin=32, cout=48, kernel=[3] * dim, stride=[1] * dim, padding=[1] * dim,
                     dilation=[1] * dim, in_size=in_size, out_pad=[0] * dim, seed=570 + dim)
    names = ("input", "weight", "offset", "mask", "bias")
    ts = [case[n].to("cuda:0", torch.float32) for n in names]
    params = ([1] * dim, [1] * dim, [1] * dim, 1)
    fwd = getattr(torch.ops.tvdcn, f"deform_conv{dim}d")
    bwd = getattr(torch.ops.tvdcn, f"_deform_conv{dim}d_backward")
    with torch.no_grad():
        y_ref = fwd(*ts, *params)
    gy = torch.randn(y_ref.shape, device="cuda:0")
    ref = bwd(gy, *ts, *params)
    leaves = [t.clone().requires_grad_(True) for t in ts]
    previous = tvdcn.set_keep_channels_last_copy(True)
    try:
        y = fwd(*leaves, *params)
    finally:
        tvdcn.set_keep_channels_last_copy(previous)
    y.backward(gy)
    torch.cuda.synchronize()
    assert leaves[0].grad.is_contiguous()
    assert rel_err(y, y_ref) < 1e-6
    for n, t, r in zip(names, leaves, ref):
        e = rel_err(t.grad, r)
        assert e < 1e-6, f"grad_{n} rel err {e}"
    o_out, o_grads = run_oracle(case, gy.double().cpu(), torch.float32)
    assert rel_err(y, o_out) < TOL[torch.float32][0]
    for n, t, r in zip(names, leaves, o_grads):
        assert rel_err(t.grad, r) < TOL[torch.float32][1], f"grad_{n} (oracle)"


def test_weight_splits_across_pass_boundaries_fp32():
    """3D, 27 taps (three passes) over 135 spatial tiles: the windowed weight gradient's splits
    run over (pass, tile) units two at a time, so split 67 holds the last tile of pass 0 and
    the first of pass 1, and the reduction sums per tap only the splits that meet its pass.
    Every quantity at the usual bounds (the oracle samples at the float32 positions, so the
    samples that round onto a cell boundary take the same one-sided offset derivative)."""
    case = make_case(3, False, batch=3, cin=16, cout=32, kernel=[3, 3, 3], stride=[1, 1, 1], padding=[1, 1, 1],
                     dilation=[1, 1, 1], in_size=[12, 24, 40], out_pad=[0, 0, 0], seed=590)
    check(case, torch.float32)


def test_channels_last_1d_input():
    """A 1D conv input in (batch, length, channels) order, seen as (B, C, L) with strides
    (L * C, 1, C) (a permuted tensor; torch has no 1D channels-last format), is sampled in
    place; its gradient comes back in the same order, with the numbers of the float64 oracle (and
    of the NC<spatial> path)."""
    case = make_case(1, False, batch=2, cin=32, cout=48, kernel=[3], stride=[1], padding=[1], dilation=[1],
                     in_size=[70], out_pad=[0], seed=580)
    out, grads, gout = run_gpu(case, torch.float32)
    ref_out, ref_grads = run_oracle(case, gout, torch.float32)
    names = ("input", "weight", "offset", "mask", "bias")
    ts = [case[n].to("cuda:0", torch.float32) for n in names]
    ts[0] = ts[0].permute(0, 2, 1).contiguous().permute(0, 2, 1)
    assert ts[0].stride() == (70 * 32, 1, 32)
    ts = [t.requires_grad_(True) for t in ts]
    y = tvdcn.deform_conv1d(*ts, stride=1, padding=1, dilation=1)
    y.backward(gout.to("cuda:0", torch.float32))
    torch.cuda.synchronize()
    assert ts[0].grad.stride() == (70 * 32, 1, 32)
    assert rel_err(y, ref_out) < 1e-5 and rel_err(y, out) < 1e-5
    for n, t, r, r_nc in zip(names, ts, ref_grads, grads):
        e = rel_err(t.grad, r)
        assert e < 1e-4, f"grad_{n} rel err {e} (oracle)"
        assert rel_err(t.grad, r_nc) < 1e-5, f"grad_{n} (NC<spatial> path)"


def scatter_magnitude(case, gout, dtype):
    """A[b, c, s] = sum over the scatter terms landing on input element (b, c, s) of |G * mask| * corner
    weight, G = W^T grad_out (the grad-columns): the float64 oracle's transposed forward scatters
    |G| with |mask| through a selection weight (input channel c * K + t -> output channel c at tap t),
    which is the conv backward's col2im geometry on the same offsets (conv only, groups 1)."""
    from oracle import oracle
    dim = case["dim"]
    w = case["weight"].to(dtype).double()
    M, C = w.shape[:2]
    k = list(w.shape[2:])
    K = w[0, 0].numel()
    g = gout.to(dtype).double()
    B, P = g.shape[0], list(g.shape[2:])
    G = torch.einsum("mck,bmp->bckp", w.reshape(M, C, K), g.reshape(B, M, -1))   # (B, C, K, P)
    X = G.abs().reshape(B, C * K, *P)
    sel = torch.zeros(C * K, C, K, dtype=torch.float64)
    idx = torch.arange(C)
    for t in range(K):
        sel[idx * K + t, idx, t] = 1.0
    sel = sel.reshape(C * K, C, *k)
    off = case["offset"].to(dtype).double()
    msk = case["mask"].to(dtype).double().abs()
    S = list(case["input"].shape[2:])
    s, p, d = case["stride"], case["padding"], case["dilation"]
    op = [S[i] - ((P[i] - 1) * s[i] - 2 * p[i] + d[i] * (k[i] - 1) + 1) for i in range(dim)]
    return oracle.forward(dim, X, sel, off, msk, None, stride=s, padding=p, dilation=d, groups=1,
                          transposed=True, output_padding=op)


def transposed_forward_magnitude(case, dtype):
    """A[b, c, s] = sum over the scatter terms landing on output element (b, c, s) of the transposed
    forward of |cols * mask| * corner weight, cols = W^T input (groups 1): the float64 oracle's transposed
    forward of |cols| through a selection weight (channel c * K + t -> output channel c at tap t)"""
    from oracle import oracle
    dim = case["dim"]
    w = case["weight"].to(dtype).double()   # (Cin, Cout, k...)
    M, C = w.shape[:2]
    k = list(w.shape[2:])
    K = w[0, 0].numel()
    x = case["input"].to(dtype).double()
    B, P = x.shape[0], list(x.shape[2:])
    cols = torch.einsum("mck,bmp->bckp", w.reshape(M, C, K), x.reshape(B, M, -1))   # (B, C, K, P)
    X = cols.abs().reshape(B, C * K, *P)
    sel = torch.zeros(C * K, C, K, dtype=torch.float64)
    idx = torch.arange(C)
    for t in range(K):
        sel[idx * K + t, idx, t] = 1.0
    sel = sel.reshape(C * K, C, *k)
    off = oracle_offsets(case, case["offset"].to(dtype).double(), dtype)
    msk = case["mask"].to(dtype).double().abs() if case["mask"] is not None else None
    return oracle.forward(dim, X, sel, off, msk, None, stride=case["stride"], padding=case["padding"],
                          dilation=case["dilation"], groups=1, transposed=True,
                          output_padding=case["output_padding"])


def elementwise_err(a, ref, mag):
    """max over elements of |a - ref| / (mag + median mag): the error relative to the summed magnitude of
    the element's own terms, plus that of a typical element (float64)"""
    a = a.detach().double().cpu()
    return float(((a - ref).abs() / (mag + mag.median())).max())


@pytest.mark.skipif(not oracle.have_reference(), reason="reference CPU build (oracle/_ref) not available")
@pytest.mark.parametrize("dim,spike,dense", [(2, 0.0, False), (2, 1e4, False), (2, 1e6, False), (1, 1e6, False),
                                             (3, 0.0, False), (3, 1e4, False), (3, 1e6, False), (2, 1e4, True),
                                             (2, 1e2, True)])
def test_scatter_elementwise_under_gradient_spikes_fp32(dim, spike, dense):
    """grad_input element by element when grad_out holds one spike pixel (all channels x `spike`) in
    every 256-pixel tile of the data-gradient kernel (dense: 16, every 4th row and column). The
    fixed-point window's unit is relative to its tile's bound, so spike terms (above 2^6 x the typical
    term of their pass) take global float atomics. Error of an element = |x - x64| /
    (A + median A), A = the summed magnitude of the element's own scatter terms, x64 the float64 oracle.
    Bound: 4x the largest error of the reference's own float32 path on the same inputs (oracle/_ref) +
    1e-5. Measured (MI355X): no spike 4e-6 / 6e-6 (2D / 3D; float atomics 2e-7: the window's unit is
    ~2^-28 of its tile's bound); at 1e4 and 1e6 spikes within 1.3x / 4.2x of the reference (whose own
    float32 GEMM rounding of the spike dominates); the window kept at the spike's scale was 200x it."""
    in_size = {1: [600], 2: [40, 36], 3: [8, 16, 16]}[dim]
    case = make_case(dim, False, batch=2, cin=16 if dim == 3 else 32, cout=64, kernel=[3] * dim,
                     stride=[1] * dim, padding=[1] * dim, dilation=[1] * dim, in_size=in_size, out_pad=[0] * dim,
                     seed=540 + dim)
    # offsets on a 2^-8 grid: sampling positions and bilinear weights are exact in float32, so that
    # the float32 rounding of positions stays out of what this test measures
    case["offset"] = (case["offset"] * 256).round() / 256
    g = torch.Generator().manual_seed(541)
    gout = torch.randn(case["out_shape"], generator=g, dtype=torch.float64)
    if dense:
        gout[..., ::4, ::4] *= spike
    elif spike:
        box = {1: (256,), 2: (16, 16), 3: (4, 8, 8)}[dim]
        grid = case["out_shape"][2:]
        origins = [range(0, n, bx) for n, bx in zip(grid, box)]
        for org in itertools.product(*origins):
            pix = tuple(min(o + bx // 2, n - 1) for o, bx, n in zip(org, box, grid))
            gout[(slice(None), slice(None)) + pix] *= spike
    _, grads, _ = run_gpu(case, torch.float32, grad_out=gout)
    _, ref = run_oracle(case, gout, torch.float32)
    mag = scatter_magnitude(case, gout, torch.float32)
    e = elementwise_err(grads[0], ref[0], mag)
    args = [case[n].float() if case[n] is not None else None for n in ("input", "weight", "offset", "mask", "bias")]
    params = [case["stride"], case["padding"], case["dilation"], case["groups"]]
    ref32 = oracle.run_reference([{"op": f"_deform_conv{dim}d_backward", "args": [gout.float()] + args + params}])
    e_ref = elementwise_err(ref32[0][0], ref[0], mag)
    print(f"dim {dim} spike {spike:g} dense {dense}: grad_input elementwise error {e:.2e} "
          f"(reference float32 path {e_ref:.2e})", flush=True)
    assert e <= 4 * e_ref + 1e-5
    for name, gr, r in zip(("weight", "offset", "mask", "bias"), grads[1:], ref[1:]):
        assert rel_err(gr, r) < TOL[torch.float32][1], name


@pytest.mark.skipif(not oracle.have_reference(), reason="reference CPU build (oracle/_ref) not available")
@pytest.mark.parametrize("dim", [1, 2, 3])
def test_scatter_elementwise_graded_grad_out_fp32(dim):
    """grad_input element by element when grad_out falls smoothly from 1 to 1e-3 across every 256-pixel
    tile of the data-gradient kernel (log-linear along the tile's last axis): the quiet end of a tile
    accumulates in the same fixed-point window, at a unit set by the tile's bound, as its loud end. Error
    of an element as in the spike test: |x - x64| / (A + median A), bound 4x the reference's own float32
    path (oracle/_ref) + 1e-5. Also printed: the error relative to the element's own magnitude A alone
    over the quietest tenth of the elements, ours and the reference's."""
    in_size = {1: [600], 2: [40, 36], 3: [8, 16, 16]}[dim]
    case = make_case(dim, False, batch=2, cin=16 if dim == 3 else 32, cout=64, kernel=[3] * dim,
                     stride=[1] * dim, padding=[1] * dim, dilation=[1] * dim, in_size=in_size, out_pad=[0] * dim,
                     seed=545 + dim)
    case["offset"] = (case["offset"] * 256).round() / 256
    g = torch.Generator().manual_seed(546)
    gout = torch.randn(case["out_shape"], generator=g, dtype=torch.float64)
    span = {1: 256, 2: 16, 3: 8}[dim]   # the tile's extent along the last axis
    n = case["out_shape"][-1]
    u = (torch.arange(n, dtype=torch.float64) % span) / (span - 1)
    gout = gout * torch.pow(10.0, -3.0 * u)
    _, grads, _ = run_gpu(case, torch.float32, grad_out=gout)
    _, ref = run_oracle(case, gout, torch.float32)
    mag = scatter_magnitude(case, gout, torch.float32)
    e = elementwise_err(grads[0], ref[0], mag)
    args = [case[n].float() if case[n] is not None else None for n in ("input", "weight", "offset", "mask", "bias")]
    params = [case["stride"], case["padding"], case["dilation"], case["groups"]]
    ref32 = oracle.run_reference([{"op": f"_deform_conv{dim}d_backward", "args": [gout.float()] + args + params}])
    e_ref = elementwise_err(ref32[0][0], ref[0], mag)
    quiet = (mag > 0) & (mag <= mag[mag > 0].quantile(0.1))

    def own(a):
        return float(((a.detach().double().cpu() - ref[0]).abs()[quiet] / mag[quiet]).max())

    print(f"dim {dim} graded grad_out: grad_input elementwise error {e:.2e} (reference float32 path {e_ref:.2e}); "
          f"quietest tenth, relative to their own magnitude: {own(grads[0]):.2e} "
          f"(reference {own(ref32[0][0]):.2e})", flush=True)
    assert e <= 4 * e_ref + 1e-5
    for name, gr, r in zip(("weight", "offset", "mask", "bias"), grads[1:], ref[1:]):
        assert rel_err(gr, r) < TOL[torch.float32][1], name


def test_saved_input_version_check_by_default():
    """By default the autograd node saves the input itself, as the reference does
    (autograd/deform_conv2d_kernel.cpp:35): changing it in place after the forward makes the backward
    raise torch's version-counter error."""
    case = make_case(2, False, batch=2, cin=32, cout=48, kernel=[3, 3], stride=[1, 1], padding=[1, 1],
                     dilation=[1, 1], in_size=[12, 10], out_pad=[0, 0], seed=590)
    ts = [case[n].to("cuda:0", torch.float32).requires_grad_(n != "input")
          for n in ("input", "weight", "offset", "mask", "bias")]
    x = ts[0].clone().requires_grad_(True)
    xin = x * 1.0    # a non-leaf input that can be changed in place
    y = tvdcn.deform_conv2d(xin, *ts[1:], padding=1)
    xin.add_(1.0)
    with pytest.raises(RuntimeError, match="modified by an inplace operation"):
        y.sum().backward()


@pytest.mark.parametrize("what", ["input", "mask", "grad_out"])
def test_large_fp32_operands_take_the_fp32_loop(what):
    """fp32 operands go into the 16-bit MFMA loops as scaled fp16 pieces only when their products and
    scales stay in the float range: an input at or above 2^96, a plain mask at or above 2^30 or a
    grad_out past the bf16 range sets the device flag, and the kernels run their fp32 MFMA loops. Results against the
    float64 oracle at the fp32 tolerances (forward and every gradient)."""
    case = make_case(2, False, batch=2, cin=32, cout=32, kernel=[3, 3], stride=[1, 1], padding=[1, 1],
                     dilation=[1, 1], in_size=[14, 12], out_pad=[0, 0], seed=560)
    g = torch.Generator().manual_seed(561)
    gout = torch.randn(case["out_shape"], generator=g, dtype=torch.float64)
    if what == "input":
        case["input"] = case["input"] * 1e30
    elif what == "mask":
        case["mask"] = case["mask"] * 1e10
    else:
        # one value rounds past the largest bf16; the input is scaled down so that no gradient
        # overflows fp32
        case["input"] = case["input"] * 1e-3
        gout[0, 0, 0, 0] = 3.3999e38
    out, grads, _ = run_gpu(case, torch.float32, grad_out=gout)
    ref_out, ref_grads = run_oracle(case, gout, torch.float32)
    assert rel_err(out, ref_out) < TOL[torch.float32][0]
    for name, gr, r in zip(("input", "weight", "offset", "mask", "bias"), grads, ref_grads):
        e = rel_err(gr, r)
        assert e < TOL[torch.float32][1], f"grad_{name} rel err {e}"


@pytest.mark.parametrize("dim,transposed,dtype", [(1, False, torch.float32), (1, True, torch.float32),
                                                  (1, False, torch.float16), (2, False, torch.bfloat16)])
def test_staged_weight_blocks_nine_tap_passes(dim, transposed, dtype):
    """Nine-tap passes stage the data gradient's weight blocks in LDS (double-buffered, one
    barrier per 32-channel step): several steps, a GEMM side off the step size (zero rows),
    the conv backward and the transposed forward (scatter-only plan)."""
    kernel = [9] if dim == 1 else [3, 3]
    in_size = [200] if dim == 1 else [20, 18]
    case = make_case(dim, transposed, batch=2, cin=48, cout=80, kernel=kernel, stride=[1] * dim,
                     padding=[k // 2 for k in kernel], dilation=[1] * dim, in_size=in_size, out_pad=[0] * dim,
                     seed=610 + dim + 2 * transposed, offset_scale=2.0)
    check(case, dtype)


@pytest.mark.skipif(not oracle.have_reference(), reason="reference CPU build (oracle/_ref) not available")
@pytest.mark.parametrize("dim", [2, 3])
def test_transposed_forward_elementwise_fp32(dim):
    """The transposed forward is the scatter-only plan of the data-gradient kernel: its output accumulates
    in the LDS fixed-point window. With many taps (2D 5 x 5 at stride 2; 3D 4 x 4 x 4 on few channels,
    64 taps) the unit of a window tied to the summed bound of its tile lost float32 accuracy (forward
    rel err 1e-5 .. 2.3e-5 on 48 / 64-tap 3D problems); the unit follows the largest kept term of the pass
    instead. Each element against the float64 oracle, relative to the summed magnitude of its own terms
    plus that of a typical element (elementwise_err), within 4x the reference's own float32 path on the
    same inputs (oracle/_ref) + 1e-6; norm-wise within the float32 forward bound."""
    if dim == 2:
        case = make_case(2, True, batch=2, cin=32, cout=48, kernel=[5, 5], stride=[2, 2], padding=[2, 2],
                         dilation=[1, 1], in_size=[20, 18], out_pad=[1, 1], seed=611, offset_scale=2.0)
    else:
        case = make_case(3, True, batch=2, cin=16, cout=32, kernel=[4, 4, 4], stride=[1, 2, 1], padding=[2, 1, 2],
                         dilation=[1, 1, 1], in_size=[7, 6, 7], out_pad=[0, 1, 0], seed=612, offset_scale=2.0)
    out, _, _ = run_gpu(case, torch.float32)
    ref_out, _ = run_oracle(case, torch.zeros(case["out_shape"], dtype=torch.float64), torch.float32)
    mag = transposed_forward_magnitude(case, torch.float32)
    e = elementwise_err(out, ref_out, mag)
    args = [case[n].float() if case[n] is not None else None for n in ("input", "weight", "offset", "mask", "bias")]
    params = [case["stride"], case["padding"], case["output_padding"], case["dilation"], case["groups"]]
    ref32 = oracle.run_reference([{"op": f"deform_conv_transpose{dim}d", "args": args + params}])
    e_ref = elementwise_err(ref32[0], ref_out, mag)
    n = rel_err(out, ref_out)
    print(f"dim {dim}: transposed forward elementwise error {e:.2e} (reference float32 path {e_ref:.2e}), "
          f"norm-wise {n:.2e}", flush=True)
    assert n < TOL[torch.float32][0]
    assert e <= 4 * e_ref + 1e-6


@pytest.mark.parametrize("kind", ["tiny", "large", "wide", "transposed_tiny"])
def test_fp32_pieces_scaled_per_tensor(kind):
    """fp32 operands enter the 16-bit MFMA loops as two fp16 pieces of the value times a per-tensor
    power of two that puts the tensor's largest magnitude in [2^14, 2^15): magnitudes far outside
    fp16's range (tiny: inputs near 1e-6 and an upstream gradient near 1e-8, whose unscaled fp16
    pieces would underflow; large: inputs near 1e4 with weights near 1e-4) and a wide range inside
    one tensor (input magnitudes log-uniform over 1e-4 .. 1e2) keep float32 accuracy: forward and
    every gradient against the float64 oracle at the float32 bounds."""
    transposed = kind.startswith("transposed")
    case = make_case(2, transposed, batch=2, cin=32, cout=48, kernel=[3, 3], stride=[1, 1] if not transposed else [2, 2],
                     padding=[1, 1], dilation=[1, 1], in_size=[14, 12], out_pad=[1, 1] if transposed else [0, 0],
                     seed=620)
    g = torch.Generator().manual_seed(621)
    gout = torch.randn(case["out_shape"], generator=g, dtype=torch.float64)
    if kind in ("tiny", "transposed_tiny"):
        case["input"] = case["input"] * 1e-6
        gout = gout * 1e-8
    elif kind == "large":
        case["input"] = case["input"] * 1e4
        case["weight"] = case["weight"] * 1e-4
    else:
        mag = torch.exp(torch.empty(case["input"].shape, dtype=torch.float64).uniform_(
            float(torch.log(torch.tensor(1e-4))), float(torch.log(torch.tensor(1e2))), generator=g))
        case["input"] = torch.where(torch.rand(case["input"].shape, generator=g) < 0.5, -mag, mag)
    out, grads, _ = run_gpu(case, torch.float32, grad_out=gout)
    ref_out, ref_grads = run_oracle(case, gout, torch.float32)
    e = rel_err(out, ref_out)
    print(f"{kind}: forward rel err {e:.2e}", flush=True)
    assert e < TOL[torch.float32][0]
    for name, gr, r in zip(("input", "weight", "offset", "mask", "bias"), grads, ref_grads):
        if r is not None:
            e = rel_err(gr, r)
            print(f"{kind}: grad_{name} rel err {e:.2e}", flush=True)
            assert e < TOL[torch.float32][1], name


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("dim,transposed,in_size", [
    (2, False, [20, 24]), (2, False, [20, 22]), (1, False, [320]), (1, False, [322]),
    (3, False, [6, 8, 16]), (3, False, [6, 8, 12]), (2, True, [16, 16])])
def test_weight_gradient_a_fragments(dim, transposed, in_size, dtype):
    """The weight gradient's 16-bit loop reads its A fragments (Z, 8 pixels of a row) as 16-bit values
    when the column grid's rows are a multiple of 8 wide (fp32: Z's pieces written beside the data
    gradient's split; fp16 / bf16: Z itself), and forms them from fp32 loads otherwise: both widths,
    every rank, conv and transposed, against the float64 oracle."""
    k = [5] if dim == 1 else [3] * dim
    case = make_case(dim, transposed, batch=2, cin=32, cout=48, kernel=k, stride=[1] * dim,
                     padding=[kk // 2 for kk in k], dilation=[1] * dim, in_size=in_size, out_pad=[0] * dim,
                     seed=630 + dim + 3 * transposed + in_size[-1])
    check(case, dtype)
