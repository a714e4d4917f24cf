#!/usr/bin/env python3
"""Benchmark of the deformable-convolution hot path on one MI355X.

Default workload (the north-star metric): deform_conv2d
DCNv2 backbone layer, fp32, input (8,256,64,64), weight (256,256,3,3), stride 1,
pad 1, dilation 1, one offset/mask group, offset N(0, 2^2) px, mask sigmoid(N(0,1)),
forward + backward with upstream gradient N(0,1). One "step" = forward + backward
through autograd on inputs already resident in HBM.

Printed JSON line (rank 0): the driver contract plus
  roofline      -- the kernel family with the most time in the timed region: its
                   algorithmic flops per launch / its average launch duration, the
                   duration measured with HIP events recorded on the launch stream
                   (tvdcn_kernel_timer_* in the C ABI), against MI355X peak;
  cpu_baseline  -- the reference's own CPU path (oracle/_ref, compiled from the
                   reference sources) timed on this host on the full workload, in a
                   child process (oracle/ref_child.py);
  kernels       -- every kernel family's average launch time and roofline fraction.
"""
import argparse
import ctypes
import hashlib
import json
import os
import statistics
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "deform_conv2d fwd+bwd ms and % HBM/MFMA roofline, B8 C256 64x64 k3 fp32"
PEAK_FP32_MFMA = 157.3e12      # MI355X dense fp32 matrix, FLOP/s
PEAK_HBM = 8.0e12              # MI355X HBM3E, B/s
PEAK_16BIT_MFMA = 2.5e15       # MI355X dense fp16 / bf16 matrix, FLOP/s


def mfma_path(dtype=torch.float32):
    """(MFMA instruction, MFMA products per algorithmic product, its dense peak) of the MFMA kernel
    families' K loops: 16x16x32 MFMAs in every rank, fp32 operands as two fp16 pieces at a per-tensor
    power-of-two scale, of which three cross products are summed (fp32-accurate), fp16/bf16 operands
    as they are. A launch whose fp32 operands were flagged (not finite) runs the fp32 loop instead.
    The fp32 path's own ceiling is the 16-bit peak over the products per product (2.5 PFLOP/s / 3 =
    833 TFLOP/s fp32-equivalent), above the fp32 MFMA peak."""
    if dtype == torch.float32:
        return "v_mfma_f32_16x16x32_f16 (2 fp16 pieces per fp32 value, 3 products)", 3, PEAK_16BIT_MFMA
    return f"v_mfma_f32_16x16x32_{'f16' if dtype == torch.float16 else 'bf16'}", 1, PEAK_16BIT_MFMA
FAMILIES = ["layout", "gather_gemm", "data_grad", "weight_grad", "bias_grad", "mask_softmax"]


def make_inputs(batch=8, seed=1002):
    """cfg2 tensors in the order input, weight, offset, mask-logits, bias, grad_out (CPU, fp32)."""
    g = torch.Generator().manual_seed(seed)
    C, H, W, K = 256, 64, 64, 3
    x = torch.randn(batch, C, H, W, generator=g)
    w = torch.randn(C, C, K, K, generator=g) * (2.0 / (C * K * K)) ** 0.5   # Kaiming normal, fan_in 2304
    off = torch.randn(batch, 2 * K * K, H, W, generator=g) * 2.0
    mask = torch.sigmoid(torch.randn(batch, K * K, H, W, generator=g))
    bias = torch.zeros(C)
    gout = torch.randn(batch, C, H, W, generator=g)
    return dict(input=x, weight=w, offset=off, mask=mask, bias=bias, grad_out=gout)


def sha(t):
    return hashlib.sha256(t.contiguous().numpy().tobytes()).hexdigest()[:16]


def flops_fwd(batch=8):
    return 2.0 * batch * 256 * 256 * 9 * 64 * 64


def _kernel_lib():
    import tvdcn
    lib = ctypes.CDLL(tvdcn.extension.HIP_LIB_PATH)
    lib.tvdcn_kernel_timer_enable.argtypes = [ctypes.c_int32]
    lib.tvdcn_kernel_timer_read.argtypes = [ctypes.c_int32, ctypes.POINTER(ctypes.c_double),
                                            ctypes.POINTER(ctypes.c_int64)]
    return lib


def time_path(params, fwd, gout, steps, warmup):
    """Times fwd() alone and fwd().backward(gout) (grads of `params` cleared each step) with host
    clocks around synchronised loops, then per-kernel-family durations from HIP events on the
    launch stream. Returns (fwd_ms, step_ms, {family: totals})."""
    lib = _kernel_lib()

    def step():
        for p in params:
            p.grad = None
        fwd().backward(gout)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()

    # forward only
    with torch.no_grad():
        for _ in range(2):
            fwd()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            fwd()
        torch.cuda.synchronize()
        fwd_ms = (time.perf_counter() - t0) * 1e3 / steps

    # forward + backward
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    step_ms = (time.perf_counter() - t0) * 1e3 / steps

    # per-kernel durations from HIP events on the launch stream
    lib.tvdcn_kernel_timer_enable(1)
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    kern = {}
    for i, name in enumerate(FAMILIES):
        tot, n = ctypes.c_double(0), ctypes.c_int64(0)
        lib.tvdcn_kernel_timer_read(i, ctypes.byref(tot), ctypes.byref(n))
        if n.value:
            kern[name] = dict(total_ms=tot.value, launches=n.value, avg_ms=tot.value / n.value)
    lib.tvdcn_kernel_timer_enable(0)
    return fwd_ms, step_ms, kern


def gpu_bench(inp, steps, warmup):
    import tvdcn
    dev = torch.device("cuda:0")
    params = [inp[k].to(dev).requires_grad_(True) for k in ("input", "weight", "offset", "mask", "bias")]
    gout = inp["grad_out"].to(dev)

    def fwd():
        return tvdcn.deform_conv2d(*params, stride=1, padding=1, dilation=1, groups=1)

    return time_path(params, fwd, gout, steps, warmup)


def family_rooflines(kern, contraction_flops, grad_out_bytes, mask_bytes=0, dtype=torch.float32):
    """Algorithmic work per launch of each kernel family against the bound that applies: each of
    the three MFMA families performs one contraction of `contraction_flops` per launch (its fraction
    taken of the fp32 MFMA peak, the arithmetic the path delivers; `mfma` names the instruction its
    K loop runs on and `hw_frac` that instruction's use of its own dense peak); the bias gradient
    reads grad_out once; mask_softmax reads + writes the mask (forward) or reads two tensors and
    writes one (backward): 2.5 passes over `mask_bytes` on average."""
    work = {
        "gather_gemm": ("mfma", contraction_flops, PEAK_FP32_MFMA, "TFLOP/s"),
        "data_grad": ("mfma", contraction_flops, PEAK_FP32_MFMA, "TFLOP/s"),
        "weight_grad": ("mfma", contraction_flops, PEAK_FP32_MFMA, "TFLOP/s"),
        "bias_grad": ("hbm", grad_out_bytes, PEAK_HBM, "GB/s"),
        "mask_softmax": ("hbm", 2.5 * mask_bytes, PEAK_HBM, "GB/s"),
    }
    out = {}
    for name, k in kern.items():
        if name in work and work[name][1] > 0:
            bound, amount, peak, unit = work[name]
            achieved = amount / (k["avg_ms"] * 1e-3)
            scale = 1e12 if unit == "TFLOP/s" else 1e9
            out[name] = dict(avg_ms=round(k["avg_ms"], 4), launches=k["launches"], bound=bound,
                             achieved=round(achieved / scale, 2), peak=round(peak / scale, 1), unit=unit,
                             frac=round(achieved / peak, 4))
            if bound == "mfma":
                # hw_frac: the instruction's use of its own dense peak, which is also the fraction of
                # the path's ceiling (hw_peak / products in algorithmic FLOP/s)
                instr, products, hw_peak = mfma_path(dtype)
                out[name].update(mfma=instr, hw_frac=round(products * achieved / hw_peak, 4),
                                 ceiling=round(hw_peak / products / scale, 1))
        else:
            # layout family: several small launches (channels-last copies, weight re-layouts, zero fills)
            out[name] = dict(avg_ms=round(k["avg_ms"], 4), launches=k["launches"], total_ms=round(k["total_ms"], 4))
    return out


def kernel_rooflines(kern, batch=8):
    """cfg2 work per launch for each family."""
    return family_rooflines(kern, flops_fwd(batch), 4 * batch * 256 * 64 * 64)


# ---- per-config suite ------------------------------------------

def _kaiming(shape, fan_in, g):
    return torch.randn(*shape, generator=g) * (2.0 / fan_in) ** 0.5


def suite_case(n):
    """Tensors (CPU, fp32) and parameters of BASELINE.json configs[n - 1], n = 2..5, with that
    config's distributions. For configs 3 and 5 the mask is the op's mask_softmax of N(0,1)
    logits, applied inside the timed layer (it is part of the path)."""
    g = torch.Generator().manual_seed(3000 + n)
    if n == 2:
        t = make_inputs()
        return dict(name="cfg2 deform_conv2d B8 C256 64x64 k3", op="deform_conv2d", tr=False,
                    x=t["input"], w=t["weight"], o=t["offset"], m=t["mask"], b=t["bias"], logits=None, ks=None,
                    kw=dict(stride=1, padding=1, dilation=1, groups=1))
    if n == 3:
        return dict(name="cfg3 deform_conv1d B16 C512 L4096 k5 og4 mg4", op="deform_conv1d", tr=False,
                    x=torch.randn(16, 512, 4096, generator=g), w=_kaiming((512, 512, 5), 2560, g),
                    o=torch.randn(16, 20, 4096, generator=g) * 3, m=None, b=None,
                    logits=torch.randn(16, 20, 4096, generator=g), ks=(5,),
                    kw=dict(stride=1, padding=2, dilation=1, groups=1))
    if n == 4:
        return dict(name="cfg4 deform_conv3d B2 C64 16x56x56 k3", op="deform_conv3d", tr=False,
                    x=torch.randn(2, 64, 16, 56, 56, generator=g), w=_kaiming((64, 64, 3, 3, 3), 1728, g),
                    o=torch.randn(2, 81, 16, 56, 56, generator=g) * 1.5,
                    m=torch.sigmoid(torch.randn(2, 27, 16, 56, 56, generator=g)), b=None, logits=None, ks=None,
                    kw=dict(stride=1, padding=1, dilation=1, groups=1))
    if n == 5:
        # offsets / masks on the input grid (32 x 32), where the transposed op defines them
        return dict(name="cfg5 deform_conv_transpose2d B8 C256->128 32x32->64x64 k4 s2 og2 mg2",
                    op="deform_conv_transpose2d", tr=True,
                    x=torch.randn(8, 256, 32, 32, generator=g), w=_kaiming((256, 128, 4, 4), 128 * 16, g),
                    o=torch.randn(8, 64, 32, 32, generator=g), m=None, b=None,
                    logits=torch.randn(8, 32, 32, 32, generator=g), ks=(4, 4),
                    kw=dict(stride=2, padding=1, output_padding=0, dilation=1, groups=1))
    raise ValueError(n)


def suite_flops(c):
    """Algorithmic flops of one contraction (= the forward's GEMM work)."""
    x, w = c["x"], c["w"]
    kn = 1
    for k in w.shape[2:]:
        kn *= k
    B, groups = x.shape[0], c["kw"]["groups"]
    if c["tr"]:
        # columns over the input pixels: (Cin) x (Cout/groups * Kn) per group
        return 2.0 * B * x[0, 0].numel() * x.shape[1] * w.shape[1] * kn
    out_px = 1
    for i, S in enumerate(x.shape[2:]):
        K = w.shape[2 + i]
        out_px *= (S + 2 * c["kw"]["padding"] - (c["kw"]["dilation"] * (K - 1) + 1)) // c["kw"]["stride"] + 1
    return 2.0 * B * out_px * w.shape[0] * (x.shape[1] // groups) * kn


def run_suite_case(n, dtype, steps, warmup, cpu=False):
    """One config of the suite. Configs 3 and 5 take their softmax mask the way
    PackedDeformConv*(mask_activation="softmax") does: the softmax of the logits applied in the kernels'
    mask load (tvdcn::deform_conv_mask_activation), its gradient flowing to the logits."""
    import tvdcn
    from tvdcn.ops.deform_conv import _deform_conv_mask_activation
    c = suite_case(n)
    dev = torch.device("cuda:0")
    mk = lambda t: None if t is None else t.to(dev, dtype).requires_grad_(True)
    x, w, o, m, b, logits = (mk(c[k]) for k in ("x", "w", "o", "m", "b", "logits"))
    params = [t for t in (x, w, o, m, b, logits) if t is not None]
    op = getattr(tvdcn, c["op"])
    dim = x.dim() - 2
    kw = c["kw"]
    lst = lambda v: [v] * dim

    def fwd():
        if logits is not None:
            return _deform_conv_mask_activation(x, w, o, logits, b, lst(kw["stride"]), lst(kw["padding"]),
                                                lst(kw.get("output_padding", 0)), lst(kw["dilation"]),
                                                kw["groups"], c["tr"], 2, 0.0)
        return op(x, w, o, m, b, **kw)

    with torch.no_grad():
        out_shape = fwd().shape
    gout = torch.randn(out_shape, generator=torch.Generator().manual_seed(4000 + n)).to(dev, dtype)
    fwd_ms, step_ms, kern = time_path(params, fwd, gout, steps, warmup)
    F = suite_flops(c)
    # backward contractions: conv grad-columns + grad-weight; transposed also recomputes Wᵀ·X for the
    # offset / mask gradients (3 contractions)
    nb = 3 if c["tr"] else 2
    es = torch.finfo(dtype).bits // 8
    mask_bytes = es * (logits.numel() if logits is not None else 0)
    roof = family_rooflines(kern, F, es * gout.numel(), mask_bytes, dtype=dtype)
    row = {
        "case": c["name"], "dtype": str(dtype).replace("torch.", ""),
        "compute": ("fp32-accurate: scaled fp16 pieces on 16x16x32 MFMAs, fp32 accumulate" if dtype == torch.float32 else
                    f"{str(dtype).replace('torch.', '')} operands on 16x16x32 MFMAs, fp32 accumulate"),
        "mask": "softmax of logits in the mask load" if logits is not None else "given",
        "fwd_ms": round(fwd_ms, 4), "bwd_ms": round(step_ms - fwd_ms, 4), "fwd_bwd_ms": round(step_ms, 4),
        "gflop_fwd": round(F / 1e9, 3), "gflop_bwd": round(nb * F / 1e9, 3),
        "gflop_fwd_bwd": round((1 + nb) * F / 1e9, 3),
        "fwd_tflops": round(F / (fwd_ms * 1e-3) / 1e12, 2),
        "fwd_frac_mfma_fp32": round(F / (fwd_ms * 1e-3) / PEAK_FP32_MFMA, 4),
        "bwd_tflops": round(nb * F / ((step_ms - fwd_ms) * 1e-3) / 1e12, 2),
        "bwd_frac_mfma_fp32": round(nb * F / ((step_ms - fwd_ms) * 1e-3) / PEAK_FP32_MFMA, 4),
        "fwd_bwd_tflops": round((1 + nb) * F / (step_ms * 1e-3) / 1e12, 2),
        "fwd_bwd_frac_mfma_fp32": round((1 + nb) * F / (step_ms * 1e-3) / PEAK_FP32_MFMA, 4),
        "kernels": roof,
    }
    if cpu and dtype == torch.float32:
        row["cpu_baseline"] = cpu_baseline_case(c, gout.cpu(), reps=1)
    return row


SUITE = [(2, torch.float32), (3, torch.float32), (4, torch.float32), (5, torch.float32), (5, torch.float16),
         (5, torch.bfloat16)]


TRAFFIC_KERNELS = {"gather_gemm": "fwd_win_kernel<2, float, 8, true>",
                   "data_grad": "bwd_data_win_kernel<2, float, true, true>",
                   "weight_grad": "bwd_weight_win_kernel<2, float, true, 2, 1, 9, 32, true>"}


def load_traffic(family):
    """HBM bytes per launch of `family`'s kernel, read from the committed rocprofv3 --pmc summary
    (profiles/traffic_deform_conv2d_cfg2.md: calibrated FETCH_SIZE + WRITE_SIZE per dispatch), or None."""
    path = os.path.join(ROOT, "profiles", "traffic_deform_conv2d_cfg2.md")
    prefix = TRAFFIC_KERNELS.get(family)
    try:
        with open(path) as f:
            for row in f:
                cells = [c.strip() for c in row.strip().strip("|").split("|")]
                if len(cells) == 4 and prefix and cells[0].strip("`").startswith(prefix):
                    return int(round(float(cells[3]) * 1e6))
    except (OSError, ValueError):
        pass
    return None


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            return next(l.split(":", 1)[1].strip() for l in f if l.startswith("model name"))
    except (OSError, StopIteration):
        return "unknown CPU"


def _reference_times(name, args, bwd_args, reps):
    """(forward seconds, backward seconds) per call of the reference's CPU ops, median of `reps` calls
    after one warm-up call each, in a child process (oracle/ref_child.py: the reference build registers
    the torch.ops.tvdcn namespace, as this build's library does)."""
    from oracle import oracle
    res = oracle.run_reference([{"threads": None},
                                {"op": name, "args": args, "repeat": reps + 1},
                                {"op": f"_{name}_backward", "args": bwd_args, "repeat": reps + 1}])
    fwd = statistics.median(res[1]["times"][1:])
    bwd = statistics.median(res[2]["times"][1:])
    return fwd, bwd, res[0]


def cpu_baseline(inp, reps=3):
    """The reference's CPU implementation (oracle/_ref) on the full workload: forward + backward of all
    8 images, the same tensors the GPU run uses."""
    from oracle import oracle
    if not oracle.have_reference():
        return None
    args = [inp[k] for k in ("input", "weight", "offset", "mask", "bias")] + [[1, 1], [1, 1], [1, 1], 1]
    fwd, bwd, threads = _reference_times("deform_conv2d", args, [inp["grad_out"]] + args, reps)
    return dict(value=round((fwd + bwd) * 1e3, 1), unit="ms", cores=len(os.sched_getaffinity(0)),
                kind="reference", fwd_ms=round(fwd * 1e3, 1), bwd_ms=round(bwd * 1e3, 1),
                sample=f"reference CPU path (oracle/_ref: tvdcn 1.1.0 cpu/ kernels + ATen addmm_), forward and "
                       f"backward of the full workload (8 of 8 images), each the median of {reps} calls after 1 "
                       f"warm-up call; {_cpu_model()}; torch threads {threads['torch']}, reference OpenMP loops "
                       f"32 threads")


def cpu_baseline_case(c, gout, reps=1):
    """The reference's CPU path on a suite config's full tensors (mask given as its softmax / sigmoid
    values; the reference runs the activation in torch, not timed here)."""
    from oracle import oracle
    if not oracle.have_reference():
        return None
    dim = c["x"].dim() - 2
    m = c["m"]
    if c["logits"] is not None:
        B, ch = c["logits"].shape[:2]
        kn = 1
        for k in c["ks"]:
            kn *= k
        m = torch.softmax(c["logits"].view(B, ch // kn, kn, -1), 2).view(c["logits"].shape)
    kw = c["kw"]
    lst = lambda v: [v] * dim
    params = [lst(kw["stride"]), lst(kw["padding"])] + ([lst(kw["output_padding"])] if c["tr"] else []) + \
        [lst(kw["dilation"]), kw["groups"]]
    args = [c["x"], c["w"], c["o"], m, c["b"]] + params
    fwd, bwd, threads = _reference_times(c["op"], args, [gout] + args, reps)
    return dict(fwd_ms=round(fwd * 1e3, 1), fwd_bwd_ms=round((fwd + bwd) * 1e3, 1),
                cores=len(os.sched_getaffinity(0)), kind="reference", torch_threads=threads["torch"],
                sample=f"full workload, {reps} call(s) each after 1 warm-up call")


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--cpu-reps", type=int, default=3, help="timed reference CPU calls (after one warm-up call)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--configs", action="store_true",
                    help="instead of the metric line, print one JSON line per BASELINE config 2-5 (cfg5 also in "
                         "fp16 / bf16): forward and forward+backward ms, TFLOP/s, fraction of fp32 MFMA peak and "
                         "per-kernel-family rooflines")
    ap.add_argument("--only", type=int, default=0, metavar="N",
                    help="with --configs: only BASELINE config N (2-5; cfg5 in all three dtypes)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB 5 times (reference for the rocprofv3 "
                         "FETCH_SIZE / WRITE_SIZE scale) and exit")
    args = ap.parse_args()
    if args.copy_calibration:
        src = torch.empty(args.copy_calibration * 2**20 // 4, dtype=torch.float32, device="cuda").uniform_()
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": args.copy_calibration * 2**20}))
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported in this build "
              f"(the path would shard over the batch: independent images, one all-reduce of the weight and "
              f"bias gradients)", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)

    if args.configs:
        for n, dt in SUITE:
            if args.only and n != args.only:
                continue
            print(f"[bench] suite cfg{n} {dt}", file=sys.stderr, flush=True)
            print(json.dumps(run_suite_case(n, dt, args.steps, args.warmup, cpu=not args.no_cpu_baseline)),
                  flush=True)
            torch.cuda.empty_cache()
        return

    inp = make_inputs()
    hashes = {k: sha(v) for k, v in inp.items()}
    print(f"[bench] inputs sha256/16: {hashes}", file=sys.stderr, flush=True)
    fwd_ms, step_ms, kern = gpu_bench(inp, args.steps, args.warmup)
    print(f"[bench] fwd {fwd_ms:.3f} ms, fwd+bwd {step_ms:.3f} ms", file=sys.stderr, flush=True)
    roof = kernel_rooflines(kern)
    mfma = {k: v for k, v in roof.items() if "frac" in v}
    dom = max(mfma, key=lambda k: kern[k]["total_ms"])
    d = roof[dom]
    roofline = dict(kernel=dom, bound=d["bound"], achieved=d["achieved"], peak=d["peak"], unit=d["unit"],
                    frac=d["frac"], traffic=load_traffic(dom), mfma=d.get("mfma"), hw_frac=d.get("hw_frac"),
                    ceiling=d.get("ceiling"))

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(inp, args.cpu_reps)
        if cpu:
            print(f"[bench] cpu baseline {cpu['value']} ms ({cpu['cores']} cores)", file=sys.stderr, flush=True)

    total_flops = 3 * flops_fwd()
    line = {
        "metric": METRIC, "value": round(step_ms, 4), "unit": "ms", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(step_ms, 4), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "deform_conv2d DCNv2 layer fwd+bwd (BASELINE configs[1])", "batch": 8,
                   "channels": 256, "spatial": [64, 64], "kernel": [3, 3], "stride": 1, "padding": 1,
                   "offset_groups": 1, "mask_groups": 1, "parallelism": "none (1 GPU)"},
        "fwd_ms": round(fwd_ms, 4), "bwd_ms": round(step_ms - fwd_ms, 4),
        "fwd_bwd_tflops": round(total_flops / (step_ms * 1e-3) / 1e12, 2),
        "roofline": roofline, "cpu_baseline": cpu, "kernels": roof,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
