"""Runs the reference's own CPU build (oracle/_ref/libtvdcn_ref.so) in a child process.
TEST INFRASTRUCTURE ONLY.

The reference registers its operators as ``torch.ops.tvdcn``, the namespace the product
library (tvdcn_amd/_C.so) registers too, so the two never share a process: the parent
(tests, bench.py's cpu_baseline leg) writes the calls to a file, this script loads the
reference build, runs them under ``torch.inference_mode()`` and writes the results back.

Request file (torch.save, read with weights_only=True): a list of dicts, each one of
  {"op": name, "args": [...]}                      -> the op's result (tensor or tuple),
  {"op": name, "args": [...], "repeat": n}         -> {"times": [seconds per call]},
  {"schema": name}                                 -> str of the op's schema,
  {"error": name, "args": [...]}                   -> the RuntimeError text the op raises (or None),
  {"threads": None}                                -> {"torch": torch threads, "omp": OMP_NUM_THREADS}.
Usage: python -m oracle.ref_child <request.pt> <result.pt>
"""
import os
import sys
import time

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
REF_LIB = os.path.join(_HERE, "_ref", "libtvdcn_ref.so")


def _run(req):
    ops = torch.ops.tvdcn
    if "schema" in req:
        return str(getattr(ops, req["schema"]).default._schema)
    if "threads" in req:
        return {"torch": torch.get_num_threads(), "omp": os.environ.get("OMP_NUM_THREADS")}
    if "error" in req:
        try:
            getattr(ops, req["error"])(*req["args"])
        except RuntimeError as e:
            return str(e)
        return None
    fn = getattr(ops, req["op"])
    if "repeat" in req:
        times = []
        for _ in range(int(req["repeat"])):
            t0 = time.perf_counter()
            fn(*req["args"])
            times.append(time.perf_counter() - t0)
        return {"times": times}
    return fn(*req["args"])


def main(argv):
    src, dst = argv[1], argv[2]
    torch.ops.load_library(REF_LIB)
    reqs = torch.load(src, weights_only=True)
    out = []
    with torch.inference_mode():
        for req in reqs:
            out.append(_run(req))
    torch.save(out, dst)


if __name__ == "__main__":
    main(sys.argv)
