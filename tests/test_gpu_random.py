"""Seeded random problems against the float64 oracle (fp32 on the GPU): ranks 1-3, conv and
transposed, groups, offset / mask groups, kernel sizes, strides, paddings, dilations, output
paddings, channel counts on and off the 4- and 16-channel granularity of the windowed kernels,
offset scales from sub-pixel to far beyond the LDS windows. Each case prints its parameters."""
import random

import pytest
import torch

from helpers import make_case, rel_err
from test_gpu_parity import check, run_gpu, run_oracle

pytestmark = pytest.mark.gpu


def random_case(seed):
    rnd = random.Random(seed)
    dim = rnd.choice((1, 2, 2, 3))
    transposed = rnd.random() < 0.35
    groups = rnd.choice((1, 1, 1, 2))
    cin = groups * rnd.choice((2, 4, 8, 16, 20, 32))
    cout = groups * rnd.choice((3, 4, 16, 24, 32, 48))
    cols = cout if transposed else cin
    divs = [g for g in (1, 2, 4) if cin % g == 0 and cols % g == 0]
    og, mg = rnd.choice(divs), rnd.choice(divs)
    kernel = [rnd.choice((1, 2, 3, 4)) for _ in range(dim)]
    stride = [rnd.choice((1, 1, 2, 3)) for _ in range(dim)]
    padding = [rnd.choice((0, 1, 2)) for _ in range(dim)]
    dilation = [rnd.choice((1, 1, 2)) for _ in range(dim)]
    out_pad = [rnd.randrange(0, max(s, d)) if transposed else 0 for s, d in zip(stride, dilation)]
    hi = {1: 40, 2: 14, 3: 7}[dim]
    in_size = []
    for a in range(dim):
        span = dilation[a] * (kernel[a] - 1)
        if transposed:   # (in - 1) * stride - 2 * padding + span + out_pad + 1 >= 1
            lo = 1 + max(0, -(-(2 * padding[a] - span - out_pad[a]) // stride[a]))
        else:            # in + 2 * padding >= span + 1
            lo = max(1, span + 1 - 2 * padding[a])
        in_size.append(rnd.randint(lo, max(lo, hi)))
    params = dict(batch=rnd.choice((1, 2)), cin=cin, cout=cout, groups=groups, og=og, mg=mg,
                  deformable=rnd.random() < 0.85, modulated=rnd.random() < 0.7, bias=rnd.random() < 0.7,
                  kernel=kernel, stride=stride, padding=padding, dilation=dilation, out_pad=out_pad,
                  in_size=in_size, seed=seed, offset_scale=rnd.choice((0.5, 2.0, 6.0)))
    return dim, transposed, params


@pytest.mark.parametrize("seed", range(700, 764))
def test_random_problem_fp32(seed):
    dim, transposed, params = random_case(seed)
    print(f"seed {seed}: dim {dim} transposed {transposed} {params}", flush=True)
    case = make_case(dim, transposed, **params)
    check(case, torch.float32)


@pytest.mark.parametrize("seed", range(800, 816))
def test_random_problem_half_and_double(seed):
    dim, transposed, params = random_case(seed)
    dtype = (torch.float16, torch.bfloat16, torch.float64)[seed % 3]
    print(f"seed {seed}: {dtype} dim {dim} transposed {transposed} {params}", flush=True)
    case = make_case(dim, transposed, **params)
    check(case, dtype)


@pytest.mark.parametrize("seed", range(900, 912))
def test_random_medium_problem_fp32(seed):
    """Larger channel counts and grids (several channel slices and spatial tiles, multi-pass tap
    sets, split forward grids) on the windowed kernels."""
    rnd = random.Random(seed)
    dim = rnd.choice((1, 2, 2, 3))
    transposed = rnd.random() < 0.3
    cin = rnd.choice((64, 96, 128))
    cout = rnd.choice((64, 128, 144))
    cols = cout if transposed else cin
    og = rnd.choice([g for g in (1, 2, 4) if cin % g == 0 and cols % g == 0 and (cols // g) % 16 == 0])
    mg = rnd.choice([g for g in (1, 2, 4) if cin % g == 0 and cols % g == 0 and (cols // g) % 16 == 0])
    k = rnd.choice((2, 3, 4)) if dim < 3 else rnd.choice((2, 3))
    stride = rnd.choice((1, 1, 2)) if not transposed else 2
    size = {1: [rnd.randint(200, 600)], 2: [rnd.randint(16, 40), rnd.randint(16, 40)],
            3: [rnd.randint(4, 9), rnd.randint(8, 16), rnd.randint(8, 16)]}[dim]
    params = dict(batch=2, cin=cin, cout=cout, groups=1, og=og, mg=mg, kernel=[k] * dim, stride=[stride] * dim,
                  padding=[k // 2] * dim, dilation=[1] * dim, out_pad=[1 if transposed else 0] * dim,
                  in_size=size, seed=seed, offset_scale=rnd.choice((1.0, 3.0)))
    print(f"seed {seed}: dim {dim} transposed {transposed} {params}", flush=True)
    case = make_case(dim, transposed, **params)
    # Sampling positions of up to ~700 (1D grids): a float32 position (integer base + offset,
    # rounded once, as the reference's fp32 kernels compute it) is off by up to half an ulp,
    # 3e-5 at 512..1024, which moves bilinear weights by that much against the float64 oracle.
    # Structural mistakes show as errors of 1e-3 and more; the bound below leaves room for the
    # rounding only.
    out, grads, gout = run_gpu(case, torch.float32)
    ref_out, ref_grads = run_oracle(case, gout, torch.float32)
    assert rel_err(out, ref_out) < 1e-4, "forward"
    for name, gr, r in zip(("input", "weight", "offset", "mask", "bias"), grads, ref_grads):
        if r is not None:
            e = rel_err(gr, r)
            assert e < 1e-3 if name == "offset" else e < 2e-4, f"grad_{name} rel err {e}"


@pytest.mark.parametrize("seed", [6391, 11239, 12803])
def test_random_problem_without_a_window_fp32(seed):
    """3D transposed problems on tiny input grids (an axis of 1 or 2 cells): the 256-pixel tile box
    stretches along the long axis and no window fits its footprint. Such plans take the unwindowed
    kernels (a zero-cell window still counted a corner at its origin cell as inside and read LDS that
    was never filled)."""
    dim, transposed, params = random_case(seed)
    print(f"seed {seed}: dim {dim} transposed {transposed} {params}", flush=True)
    check(make_case(dim, transposed, **params), torch.float32)
