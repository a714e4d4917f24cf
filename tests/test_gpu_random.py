"""Seeded random problems against the float64 oracle (fp32 on the GPU): ranks 1-3, conv and
transposed, groups, offset / mask groups, kernel sizes, strides, paddings, dilations, output
paddings, channel counts on and off the 4- and 16-channel granularity of the windowed kernels,
offset scales from sub-pixel to far beyond the LDS windows. Each case prints its parameters."""
import random

import pytest
import torch

from helpers import make_case
from test_gpu_parity import check

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
    # (sampling positions up to ~700 on the 1D grids: the oracle samples at their float32 roundings,
    # as the kernels and the reference form them)
    check(make_case(dim, transposed, **params), torch.float32)


@pytest.mark.parametrize("seed", [6391, 11239, 12803])
def test_random_problem_without_a_window_fp32(seed):
    """3D transposed problems on tiny input grids (an axis of 1 or 2 cells): the 256-pixel tile box
    stretches along the long axis and no window fits its footprint. Such plans take the unwindowed
    kernels (a zero-cell window still counted a corner at its origin cell as inside and read LDS that
    was never filled)."""
    dim, transposed, params = random_case(seed)
    print(f"seed {seed}: dim {dim} transposed {transposed} {params}", flush=True)
    check(make_case(dim, transposed, **params), torch.float32)


# Problems from wider random sweeps (random_case above, and a generator of larger kernels: up to 11
# taps in 1D, 5 x 5 in 2D) that once failed, with the parameters they were drawn with. Each is
# checked at the full bounds: the oracle samples at the float32 positions the kernels and the
# reference form (a position within half a float32 step of a cell boundary takes the other cell and
# the other one-sided offset derivative), and the transposed forward's scatter keeps float32 accuracy
# on many-tap problems.
SWEEP_CASES = [
    # many-tap 3D transposed forwards (48 and 64 taps on few channels)
    (11069, "float32", 3, True, {'batch': 2, 'cin': 4, 'cout': 64, 'groups': 2, 'og': 4, 'mg': 1, 'deformable': True,
                                 'modulated': True, 'bias': False, 'kernel': [4, 4, 4], 'stride': [1, 3, 1],
                                 'padding': [2, 0, 2], 'dilation': [1, 1, 1], 'out_pad': [0, 2, 0],
                                 'in_size': [7, 4, 7], 'seed': 11069, 'offset_scale': 2.0}),
    (37015, "float32", 3, True, {'batch': 1, 'cin': 16, 'cout': 48, 'groups': 1, 'og': 1, 'mg': 2, 'deformable': True,
                                 'modulated': False, 'bias': True, 'kernel': [4, 3, 4], 'stride': [1, 3, 2],
                                 'padding': [2, 0, 1], 'dilation': [2, 1, 1], 'out_pad': [1, 1, 1],
                                 'in_size': [4, 7, 6], 'seed': 37015, 'offset_scale': 0.5}),
    # a 3D transposed problem on a 1-cell axis (no window fits its footprint)
    (10836, "bfloat16", 3, True, {'batch': 1, 'cin': 16, 'cout': 48, 'groups': 1, 'og': 1, 'mg': 2,
                                  'deformable': True, 'modulated': False, 'bias': False, 'kernel': [2, 2, 3],
                                  'stride': [3, 3, 3], 'padding': [0, 0, 1], 'dilation': [1, 1, 1],
                                  'out_pad': [0, 2, 1], 'in_size': [5, 4, 1], 'seed': 10836, 'offset_scale': 0.5}),
    # bfloat16 2D problems with larger kernels
    (35764, "bfloat16", 2, False, {'batch': 1, 'cin': 16, 'cout': 4, 'groups': 1, 'og': 2, 'mg': 2,
                                   'deformable': True, 'modulated': False, 'bias': True, 'kernel': [2, 2],
                                   'stride': [2, 1], 'padding': [0, 2], 'dilation': [1, 1], 'out_pad': [0, 0],
                                   'in_size': [9, 14], 'seed': 35764, 'offset_scale': 0.5}),
    (40692, "bfloat16", 2, False, {'batch': 1, 'cin': 64, 'cout': 48, 'groups': 1, 'og': 2, 'mg': 1, 'kernel': [3, 5],
                                   'stride': [2, 2], 'padding': [1, 4], 'dilation': [1, 2], 'out_pad': [0, 0],
                                   'in_size': [18, 26], 'seed': 40692, 'offset_scale': 0.5, 'modulated': False,
                                   'bias': False}),
    (41412, "bfloat16", 2, False, {'batch': 2, 'cin': 64, 'cout': 16, 'groups': 1, 'og': 2, 'mg': 1, 'kernel': [5, 4],
                                   'stride': [1, 1], 'padding': [4, 1], 'dilation': [2, 1], 'out_pad': [0, 0],
                                   'in_size': [25, 28], 'seed': 41412, 'offset_scale': 5.0, 'modulated': True,
                                   'bias': False}),
    # float32 positions on cell boundaries (single offset-gradient elements against the exact positions)
    (14539, "float32", 2, False, {'batch': 1, 'cin': 32, 'cout': 80, 'groups': 1, 'og': 2, 'mg': 1, 'kernel': [5, 4],
                                  'stride': [1, 1], 'padding': [4, 1], 'dilation': [2, 1], 'out_pad': [0, 0],
                                  'in_size': [22, 22], 'seed': 14539, 'offset_scale': 0.5, 'modulated': True,
                                  'bias': True}),
    (40039, "float32", 1, False, {'batch': 2, 'cin': 32, 'cout': 32, 'groups': 1, 'og': 2, 'mg': 1, 'kernel': [10],
                                  'stride': [1], 'padding': [4], 'dilation': [1], 'out_pad': [0], 'in_size': [123],
                                  'seed': 40039, 'offset_scale': 0.5, 'modulated': True, 'bias': True}),
    (40271, "float32", 1, False, {'batch': 1, 'cin': 64, 'cout': 32, 'groups': 1, 'og': 2, 'mg': 2, 'kernel': [11],
                                  'stride': [2], 'padding': [10], 'dilation': [2], 'out_pad': [0], 'in_size': [273],
                                  'seed': 40271, 'offset_scale': 2.0, 'modulated': True, 'bias': False}),
    (40573, "float32", 3, False, {'batch': 2, 'cin': 48, 'cout': 48, 'groups': 1, 'og': 1, 'mg': 1,
                                  'kernel': [3, 2, 2], 'stride': [1, 1, 1], 'padding': [1, 0, 0],
                                  'dilation': [1, 1, 1], 'out_pad': [0, 0, 0], 'in_size': [5, 11, 12], 'seed': 40573,
                                  'offset_scale': 5.0, 'modulated': False, 'bias': False}),
    (40615, "float32", 2, True, {'batch': 2, 'cin': 64, 'cout': 80, 'groups': 1, 'og': 1, 'mg': 1, 'kernel': [4, 5],
                                 'stride': [2, 2], 'padding': [3, 4], 'dilation': [2, 2], 'out_pad': [1, 1],
                                 'in_size': [9, 21], 'seed': 40615, 'offset_scale': 0.5, 'modulated': False,
                                 'bias': False}),
    (41309, "float32", 1, False, {'batch': 2, 'cin': 32, 'cout': 80, 'groups': 1, 'og': 2, 'mg': 2, 'kernel': [8],
                                  'stride': [2], 'padding': [3], 'dilation': [1], 'out_pad': [0], 'in_size': [211],
                                  'seed': 41309, 'offset_scale': 2.0, 'modulated': True, 'bias': False}),
    (7219, "float32", 2, True, {'batch': 2, 'cin': 16, 'cout': 80, 'groups': 1, 'og': 1, 'mg': 1, 'kernel': [4, 3],
                                'stride': [1, 2], 'padding': [1, 2], 'dilation': [1, 2], 'out_pad': [0, 0],
                                'in_size': [13, 27], 'seed': 7219, 'offset_scale': 0.5, 'modulated': True,
                                'bias': True}),
    (6097, "float32", 2, True, {'batch': 2, 'cin': 16, 'cout': 4, 'groups': 1, 'og': 4, 'mg': 4, 'deformable': True,
                                'modulated': False, 'bias': True, 'kernel': [3, 2], 'stride': [1, 3],
                                'padding': [2, 1], 'dilation': [2, 1], 'out_pad': [0, 0], 'in_size': [6, 13],
                                'seed': 6097, 'offset_scale': 0.5}),
    (6391, "float32", 3, True, {'batch': 2, 'cin': 32, 'cout': 48, 'groups': 2, 'og': 2, 'mg': 1, 'deformable': True,
                                'modulated': True, 'bias': True, 'kernel': [4, 1, 4], 'stride': [2, 1, 1],
                                'padding': [1, 0, 1], 'dilation': [1, 1, 2], 'out_pad': [1, 0, 0],
                                'in_size': [7, 1, 5], 'seed': 6391, 'offset_scale': 6.0}),
]


@pytest.mark.parametrize("seed,dtype,dim,transposed,params", SWEEP_CASES, ids=[str(c[0]) for c in SWEEP_CASES])
def test_sweep_case(seed, dtype, dim, transposed, params):
    dtype = getattr(torch, dtype)
    print(f"seed {seed}: {dtype} dim {dim} transposed {transposed} {params}", flush=True)
    check(make_case(dim, transposed, **params), dtype)
