"""Generate the golden fixtures under tests/golden/*.npz from the reference's own CPU
implementation (tvdcn 1.1.0 compiled from its sources into oracle/_ref by oracle/Makefile).

Run in a container where /root/reference exists:
    make -C oracle ref && python tests/golden/make_golden.py

Each fixture holds the inputs of one call and the reference's outputs: the forward
result (`out`) and the five gradients of the backward op for a fixed upstream
gradient (`g_input`, `g_weight`, `g_offset`, `g_mask`, `g_bias`; absent ones are
omitted), plus the integer parameters. Inputs follow the reference's own test
generator (tests/utils/deform_conv_test_args.py:19-92: uniform [0,1) tensors, small
shapes, offset_groups != mask_groups) with offsets shifted to [-1.5, 1.5) so that
boundary corners are exercised; seed 12 as in tests/test_grad.py:11.

The reference's autograd wrapper fails under the torch in this image ("cannot call
get_autograd_meta() on undefined tensor"), so the backward op is called directly
below autograd (torch.inference_mode), which runs the same CPU kernel.
"""
import itertools
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)


def out_size(dim, transposed, in_size, k, s, p, d, op):
    if transposed:
        return [(in_size[i] - 1) * s[i] - 2 * p[i] + d[i] * (k[i] - 1) + 1 + op[i] for i in range(dim)]
    return [(in_size[i] + 2 * p[i] - (d[i] * (k[i] - 1) + 1)) // s[i] + 1 for i in range(dim)]


def cases():
    """(name, dim, transposed, deformable, modulated, batch, cin, cout, groups, og, mg, kernel, stride, pad,
    dil, out_pad, in_size, unbatched, dtype)"""
    out = []
    for dim, tr in itertools.product([1, 2, 3], [False, True]):
        k = [2, 3, 2][:dim]
        s = [1, 2, 1][:dim]
        p = [0, 1, 1][:dim]
        d = [1, 2, 1][:dim]
        op = [0, 1, 0][:dim] if tr else [0] * dim
        sz = [5, 6, 7][:dim] if dim < 3 else ([3, 4, 4] if tr else [4, 5, 5])
        kind = f"{'tr' if tr else 'conv'}{dim}d"
        for deform, mod in [(True, True), (True, False), (False, True), (False, False)]:
            out.append((f"{kind}_d{int(deform)}m{int(mod)}", dim, tr, deform, mod, 2, 4, 6, 2, 2, 1, k, s, p, d,
                        op, sz, False, torch.float64))
        out.append((f"{kind}_og1mg2_g1", dim, tr, True, True, 2, 4, 4, 1, 1, 2, k, s, p, d, op, sz, False,
                    torch.float64))
        out.append((f"{kind}_unbatched", dim, tr, True, True, 1, 4, 6, 1, 2, 2, k, s, p, d, op, sz, True,
                    torch.float64))
        out.append((f"{kind}_fp32", dim, tr, True, True, 2, 4, 6, 2, 2, 2, k, s, p, d, op, sz, False, torch.float32))
    # the reference's plumbing case (uniform [0,1) inputs incl. offsets)
    out.append(("cfg1_conv2d_fp32", 2, False, True, True, 4, 3, 5, 1, 1, 1, [3, 3], [1, 1], [0, 0], [1, 1],
                [0, 0], [10, 10], False, torch.float32))
    out.append(("conv2d_fp16", 2, False, True, True, 2, 4, 4, 1, 2, 2, [3, 3], [1, 1], [1, 1], [1, 1], [0, 0],
                [6, 6], False, torch.float16))
    return out


def make_inputs(c, gen):
    (name, dim, tr, deform, mod, B, cin, cout, G, og, mg, k, s, p, d, op, sz, unbatched, dtype) = c
    o = out_size(dim, tr, sz, k, s, p, d, op)
    grid = sz if tr else o
    kn = int(np.prod(k))
    x = torch.rand(B, cin, *sz, generator=gen, dtype=torch.float64)
    w = torch.rand(*((cin, cout // G) if tr else (cout, cin // G)), *k, generator=gen, dtype=torch.float64)
    if name.startswith("cfg1"):
        off = torch.rand(B, og * dim * kn, *grid, generator=gen, dtype=torch.float64) if deform else None
    else:
        off = torch.rand(B, og * dim * kn, *grid, generator=gen, dtype=torch.float64) * 3 - 1.5 if deform else None
    msk = torch.rand(B, mg * kn, *grid, generator=gen, dtype=torch.float64) if mod else None
    b = torch.rand(cout, generator=gen, dtype=torch.float64)
    gout = torch.rand(B, cout, *o, generator=gen, dtype=torch.float64)
    if name.startswith("cfg1"):
        gout = torch.ones_like(gout)   # backward of sum(out)
    ts = [t.to(dtype) if t is not None else None for t in (x, w, off, msk, b, gout)]
    if unbatched:
        ts = [t[0] if (t is not None and i in (0, 2, 3, 5)) else t for i, t in enumerate(ts)]
    return ts


def run_reference(c, ts):
    (name, dim, tr, *_rest) = c
    s, p, d, op = c[12], c[13], c[14], c[15]
    G = c[8]
    x, w, off, msk, b, gout = ts
    ops = torch.ops.tvdcn
    with torch.inference_mode():
        if tr:
            out = getattr(ops, f"deform_conv_transpose{dim}d")(x, w, off, msk, b, s, p, op, d, G)
            grads = getattr(ops, f"_deform_conv_transpose{dim}d_backward")(gout, x, w, off, msk, b, s, p, op, d, G)
        else:
            out = getattr(ops, f"deform_conv{dim}d")(x, w, off, msk, b, s, p, d, G)
            grads = getattr(ops, f"_deform_conv{dim}d_backward")(gout, x, w, off, msk, b, s, p, d, G)
    return out, grads


def main():
    from oracle import oracle
    if not oracle.have_reference():
        raise SystemExit("oracle/_ref/libtvdcn_ref.so is missing: run `make -C oracle ref` first")
    # this script loads the reference build only (never the product library, which registers
    # the same torch.ops.tvdcn namespace)
    torch.ops.load_library(oracle.REF_LIB)
    gen = torch.Generator().manual_seed(12)
    n = 0
    for c in cases():
        ts = make_inputs(c, gen)
        out, grads = run_reference(c, ts)
        (name, dim, tr, deform, mod, B, cin, cout, G, og, mg, k, s, p, d, op, sz, unbatched, dtype) = c
        arrays = dict(dim=np.int64(dim), transposed=np.int64(tr), groups=np.int64(G), stride=np.array(s),
                      padding=np.array(p), dilation=np.array(d), output_padding=np.array(op),
                      unbatched=np.int64(unbatched))
        for key, t in zip(("input", "weight", "offset", "mask", "bias", "grad_out"), ts):
            if t is not None:
                arrays[key] = t.numpy()
        arrays["out"] = out.numpy()
        for key, t in zip(("g_input", "g_weight", "g_offset", "g_mask", "g_bias"), grads):
            if t is not None and t.numel() > 0:
                arrays[key] = t.numpy()
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **arrays)
        n += 1
    print(f"wrote {n} fixtures to {HERE}")


if __name__ == "__main__":
    main()
