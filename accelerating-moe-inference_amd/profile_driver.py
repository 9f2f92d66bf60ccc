"""Workloads to run under rocprofv3 for counter collection.

    rocprofv3 --pmc FETCH_SIZE -d OUT -o copy -- python3 profile_driver.py copy --mib 1024
    rocprofv3 --pmc FETCH_SIZE -d OUT -o c3   -- python3 profile_driver.py layer --config c3
    rocprofv3 --pmc FETCH_SIZE -d OUT -o c2   -- python3 profile_driver.py sgemm

`copy` launches one elementwise kernel that reads and writes exactly
--mib MiB (torch.neg into a second buffer): the calibration of the TCC byte
counters against a known traffic.  `layer` runs --steps MoE layer forwards
of a bench configuration (same seeded data as bench.py) after one warm-up;
with --block, as the decoder's MoE block (the norm in front, the residual
added).
`sgemm` runs every config-2 SGEMM shape twice, NN then NT (bench.py's
SGEMM_SHAPES, A and B ~ U[-1, 1]), printing each shape before its calls so
dispatches can be matched to shapes.
"""
from __future__ import annotations

import argparse
import importlib.util
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("what", choices=["copy", "layer", "sgemm"])
    ap.add_argument("--mib", type=int, default=1024)
    ap.add_argument("--config", default="c3", choices=["c1", "c3", "c4", "c5", "ref"])
    ap.add_argument("--steps", type=int, default=2)
    ap.add_argument("--block", action="store_true",
                    help="layer: the MoE block (norm in front, residual added)")
    args = ap.parse_args()

    import torch

    if args.what == "copy":
        n = args.mib * (1 << 20) // 4
        a = torch.ones(n, device="cuda")
        b = torch.empty_like(a)
        torch.cuda.synchronize()
        torch.neg(a, out=b)
        torch.cuda.synchronize()
        print(f"copy: read {args.mib} MiB, wrote {args.mib} MiB", flush=True)
        return

    spec = importlib.util.spec_from_file_location("bench", os.path.join(ROOT, "bench.py"))
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    pkg = bench.load_pkg()
    if args.what == "sgemm":
        ctx = pkg.Context(0)
        g = torch.Generator(device="cuda").manual_seed(0)
        for layout in ("nn", "nt"):
            for M, N, K in bench.SGEMM_SHAPES:
                a = torch.rand((M, K), device="cuda", generator=g) * 2 - 1
                b = torch.rand((K, N) if layout == "nn" else (N, K), device="cuda", generator=g) * 2 - 1
                c = torch.empty((M, N), device="cuda")
                torch.cuda.synchronize()
                print(f"sgemm {layout} {M} {N} {K}", flush=True)
                for _ in range(2):
                    (ctx.sgemm_nn if layout == "nn" else ctx.sgemm_nt)(a, b, c)
                torch.cuda.synchronize()
                del a, b, c
        ctx.close()
        return
    cfg = bench.CONFIGS[args.config]
    x, weights, y, idx, w, desc = bench.build_layer(pkg, cfg, cfg["T"], args.block,
                                                    torch.device("cuda:0"))
    ctx = pkg.Context(0)
    ctx.reserve(desc)
    for i in range(1 + args.steps):
        ctx.layer_forward(desc, weights, x, y)
        torch.cuda.synchronize()
        print(f"layer {args.config} step {i} done", flush=True)
    ctx.close()


if __name__ == "__main__":
    sys.exit(main())
