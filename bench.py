"""Benchmark: Cut Cross-Entropy fwd+bwd on one MI355X.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload c3] [--filter on|off] [--quantize BITS]

A step is one forward + backward (dE and dC, dBias when the workload has a bias)
of linear_cross_entropy over one batch of synthetic input already resident in
HBM.  Default workload: c3, the Llama-3.1-8B head (N=8192 tokens, D=4096,
V=128256, bf16), the configuration the headline metric is quoted on.

Prints one JSON line.  `value` is tokens/s of the whole job; `roofline` is the
forward kernel pair (tile kernel + lse combine, timed with HIP events on the
stream they run on) against the bf16 MFMA peak; `step_roofline` is the whole step
against the peak for the MFMA work it performed (forward + the backward's three
products over the tiles it computed: the metric's fwd+bwd fraction); `dense` is the
same step with the tile filter off (every tile: 8 N D V FLOPs, 16-bit G as the
fp32-accurate hi + lo pair, and again rounded once), timed in the same run;
`cpu_baseline` is the float32 torch-CPU restatement of the reference's
materialised-logits path timed on a bounded slice of the same workload on this host.

--quantize BITS (2, 4 or 8; not the default) stores the classifier rows in affine
groups of 64 and passes them to the loss quantized (the frozen-head case: dE and dBias,
no dC); the library dequantizes a bounded chunk of rows at a time.
"""

import argparse
import json
import math
import os
import re
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "mlx-cross-entropy_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "fwd+bwd tokens/sec and % bf16 MFMA roofline, Llama-3-8B head, 1 MI355X"
PEAK_TFLOPS = {"bf16": 2500.0, "f16": 2500.0, "f32": 157.3}
HBM_PEAK_GBS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def traffic_from_profiles(workload, filter_mode):
    """HBM bytes per forward launch from the committed rocprofv3 --pmc summary, if present."""
    path = os.path.join(ROOT, "profiles", f"fwd_tile_{workload}_traffic.txt")
    if not os.path.exists(path):
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", open(path).read())
    return float(m.group(1)) if m else None


def cpu_baseline(w, rows, budget_s):
    from oracle import cpu_baseline as CB

    N = w["N"]
    rows = min(rows, N)
    r = CB.time_tokens_per_s(w["e"].detach(), w["c"].detach(), w["targets"].detach(), w["bias"], w["reduction"],
                             w["ignore_index"], rows=rows, budget_s=budget_s)
    return {"value": r["value"], "unit": "tokens/s", "cores": r["cores"], "kind": "port",
            "sample": (f"first {r['rows']} of {N} tokens of {w['name']} (full D={w['D']}, V={w['V']}), "
                       f"float32 torch CPU, materialised logits + autograd (reference/_reference.py), "
                       f"{r['reps']} reps in {r['seconds']:.1f} s")}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="c3", choices=["c1", "c2", "c3", "c4", "c5"])
    ap.add_argument("--filter", default="on", choices=["on", "off"])
    ap.add_argument("--cpu-baseline", default="on", choices=["on", "off"])
    ap.add_argument("--quantize", type=int, default=0, choices=[0, 2, 4, 8],
                    help="classifier rows in BITS-bit affine groups of 64 (frozen head: no dC)")
    ap.add_argument("--dense-steps", type=int, default=3,
                    help="steps of the filter-off (dense) leg timed after the main ones (0: skip it)")
    ap.add_argument("--cpu-rows", type=int, default=1024)
    ap.add_argument("--cpu-budget", type=float, default=12.0)
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="after the timed steps, run one device-to-device copy of this many MiB: the known-size "
                         "kernel that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings to bytes")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": f"this build measures one GPU only (asked for --gpus {args.gpus}, "
                                   f"WORLD_SIZE={world}); run with --gpus 1"}))
        log("bench.py: multi-GPU runs are not part of this build; use --gpus 1")
        sys.exit(1)

    import torch

    import mlx_cce_amd as cce
    import workloads
    from mlx_cce_amd import _ext

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    log(f"bench: {_ext.version()} on {torch.cuda.get_device_name(dev)}; building {args.workload}")
    w = workloads.make(args.workload, device=dev)
    N, D, V = w["N"], w["D"], w["V"]
    dt = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}[w["dtype"]]
    e = w["e"].reshape(N, D).detach().requires_grad_(True)
    qw = cce.quantize(w["c"].detach(), group_size=64, bits=args.quantize) if args.quantize else None
    c = qw if qw is not None else w["c"].detach().requires_grad_(True)
    b = w["bias"].detach().requires_grad_(True) if w["bias"] is not None else None
    t = w["targets"].reshape(N)
    red = w["reduction"]
    feps = cce.FILTER_LOG_EPS if args.filter == "on" else None
    up = torch.ones(N, device=dev) if red == "none" else None

    def step(filter_eps=feps):
        e.grad = None
        if qw is None:
            c.grad = None
        if b is not None:
            b.grad = None
        loss = cce.linear_cross_entropy(e, c, t, b, reduction=red, ignore_index=w["ignore_index"],
                                        filter_eps=filter_eps)
        loss.backward(up)
        return loss

    torch.cuda.synchronize()
    for i in range(args.warmup):
        step()
    torch.cuda.synchronize()
    log(f"bench: warmup {args.warmup} done")
    fs = cce.last_filter_stats(dev)
    kept, total, kept_in = fs["kept"], fs["total"], fs["kept_input_order"]
    skip = 1.0 - kept / total
    skip_in = 1.0 - kept_in / total

    # Timed steps: HIP events bracket the forward pair (the roofline kernels) on the
    # stream it runs on; the backward is timed in a few extra steps after the timed
    # region, so that only two event records fall inside it per step.
    torch.cuda.reset_peak_memory_stats(dev)
    _ext.set_timing(True, kinds=("forward",))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    tm = _ext.timings_ms()
    peak_mem = torch.cuda.max_memory_allocated(dev)
    log(f"bench: {args.steps} steps in {elapsed:.3f} s")
    _ext.set_timing(True, kinds=("backward",))
    for i in range(min(args.steps, 5)):
        step()
    tm["backward"] = _ext.timings_ms()["backward"]
    _ext.set_timing(False)
    dense = None
    if args.dense_steps > 0 and feps is not None:
        # The conservative figure: every tile computed (filter off), same inputs, with
        # the library's default for it -- 16-bit G carried as a hi + lo pair (fp32-
        # accurate, the reference's precision) -- and again with G rounded once to the
        # input dtype (CCE_BWD_G_SINGLE) for the cost of that precision.
        def dense_leg(precision):
            with _ext.backward_options(g_precision=precision):
                _ext.set_timing(True)
                step(None)
                torch.cuda.synchronize()
                _ext.set_timing(True)
                td0 = time.perf_counter()
                for i in range(args.dense_steps):
                    step(None)
                torch.cuda.synchronize()
                d_ms = (time.perf_counter() - td0) * 1e3 / args.dense_steps
                tmd = _ext.timings_ms()
                _ext.set_timing(False)
            return d_ms, statistics.mean(tmd["forward"]), statistics.mean(tmd["backward"])

        dfl = workloads.flops(N, D, V, 0.0, qw is None)
        pair = dt != "f32"
        dense_ms, dfwd, dbwd = dense_leg(None)
        # MFMA work the hardware does: the pair's lo halves take a second MFMA in each sum
        hw = dfl + (2.0 if qw is None else 1.0) * 2.0 * N * D * V if pair else dfl
        dense = {"ms_per_step": dense_ms, "tokens_per_s": N / (dense_ms * 1e-3), "flops": dfl,
                 "tflops": dfl / (dense_ms * 1e-3) / 1e12,
                 "mfma_frac": dfl / (dense_ms * 1e-3) / 1e12 / PEAK_TFLOPS[dt],
                 "g_precision": "hi+lo pair (fp32-accurate)" if pair else "fp32",
                 "mfma_instr_flops": hw, "mfma_instr_frac": hw / (dense_ms * 1e-3) / 1e12 / PEAK_TFLOPS[dt],
                 "fwd_ms": dfwd, "bwd_ms": dbwd,
                 "steps": args.dense_steps, "note": "filter off: every 128x128 tile, 8NDV (6NDV without dC)"}
        log(f"bench: dense leg {dense_ms:.2f} ms/step")
        if pair:
            s_ms, s_fwd, s_bwd = dense_leg("single")
            dense["single_rounded_g"] = {"ms_per_step": s_ms, "tokens_per_s": N / (s_ms * 1e-3),
                                         "mfma_frac": dfl / (s_ms * 1e-3) / 1e12 / PEAK_TFLOPS[dt],
                                         "fwd_ms": s_fwd, "bwd_ms": s_bwd,
                                         "note": "CCE_BWD_G_SINGLE: G rounded to the input dtype before the products"}
            log(f"bench: dense leg, single-rounded G {s_ms:.2f} ms/step")
    if args.calib_copy_mib > 0:
        src = torch.empty(args.calib_copy_mib << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"bench: calibration copy of {args.calib_copy_mib} MiB done")
        del src, dst

    ms = elapsed * 1e3 / args.steps
    fwd_ms = statistics.mean(tm["forward"])
    bwd_ms = statistics.mean(tm["backward"])
    peak = PEAK_TFLOPS[dt]
    fwd_flops = 2.0 * N * D * V
    achieved = fwd_flops / (fwd_ms * 1e-3) / 1e12
    # MFMA work of the step as performed: the forward plus the backward's three GEMMs
    # over the tiles it computed (the 2^-12 filter's kept tiles, with the rows grouped
    # by target tile when that keeps fewer).  The non-filtered FLOPs of the metric's
    # definition with token blocks in input order (more tiles kept, never computed
    # when the rows are grouped) are reported beside it, labelled.
    want_dc = qw is None
    performed_flops = workloads.flops(N, D, V, skip, want_dc)
    input_order_flops = workloads.flops(N, D, V, skip_in, want_dc)
    dense_flops = workloads.flops(N, D, V, 0.0, want_dc)

    out = {
        "metric": METRIC,
        "value": N / (ms * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dt,
        "data": "synthetic (seeded torch.Generator on device; random-init classifier rows)",
        "config": {"workload": f"{w['name']}: {w['description']}", "N": N, "D": D, "V": V, "reduction": red,
                   "bias": b is not None,
                   "grads": ("dE,dC" if qw is None else "dE") + (",dBias" if b is not None else ""),
                   "classifier_rows": (f"{args.quantize}-bit affine groups of 64, dequantized in chunks of 32768 rows"
                                       if qw is not None else "dense"),
                   "filter": "2^-12 (128x128 tiles)" if feps is not None else "off",
                   "backward_token_order": "grouped by target tile when it keeps >=10% fewer tiles"},
        "roofline": {"bound": "mfma",
                     "kernel": ("cce forward (fwd_tile_kernel + lse_kernel)" if qw is None else
                                "cce forward (dequant_kernel per chunk + fwd_tile_kernel + lse_kernel)"),
                     "achieved": achieved, "peak": peak, "unit": "TFLOP/s", "frac": achieved / peak,
                     "traffic": traffic_from_profiles(args.workload, args.filter) if qw is None else None,
                     "flops_per_launch": fwd_flops, "avg_launch_ms": fwd_ms},
        # The whole step against the peak for the MFMA work it performed: the metric's
        # fwd + bwd fraction (roofline above is the dominant kernel's alone).
        "step_roofline": {"bound": "mfma", "achieved": performed_flops / (ms * 1e-3) / 1e12, "peak": peak,
                          "unit": "TFLOP/s", "frac": performed_flops / (ms * 1e-3) / 1e12 / peak,
                          "flops": performed_flops, "ms_per_step": ms,
                          "flops_formula": "2NDV + 6NDV(1 - tile_skip) (4NDV without dC)"},
        "step": {"fwd_ms": fwd_ms, "bwd_ms": bwd_ms, "total_tiles": total,
                 "rows_grouped_by_target": bool(fs["sorted_rows"]), "tile_skip": skip, "kept_tiles": kept,
                 "performed_flops": performed_flops, "tflops": performed_flops / (ms * 1e-3) / 1e12,
                 "mfma_frac": performed_flops / (ms * 1e-3) / 1e12 / peak,
                 "kept_tiles_input_order": kept_in, "tile_skip_input_order": skip_in,
                 "input_order_flops": input_order_flops,
                 "mfma_frac_input_order_flops": input_order_flops / (ms * 1e-3) / 1e12 / peak,
                 "dense_flops": dense_flops,
                 "peak_mem_gb": peak_mem / 2 ** 30, "logits_bytes_if_materialised": 4.0 * N * V},
        "dense": dense,
        "cpu_baseline": None,
    }
    if args.cpu_baseline == "on":
        log("bench: timing CPU baseline")
        out["cpu_baseline"] = cpu_baseline(w, args.cpu_rows, args.cpu_budget)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
