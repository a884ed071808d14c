"""MoE layer forward benchmark on one MI355X.

    python bench.py [--steps K] [--warmup W] [--config 2] [--no-cpu-baseline]

A step is one full MoE layer forward (router -> histogram/scan -> permute plan -> grouped
SwiGLU GEMMs -> combine + aux loss) over one batch of synthetic input already resident in HBM.
Default workload: config 2 of BASELINE.json (T=16384 = 8 x 2048, d=1024, 32 experts, top-4
softmax, SwiGLU H=512, bf16, dropless). Prints ONE JSON line.

roofline: the dominant kernel is the grouped up-projection GEMM (gate/value GEMM with the fused
SwiGLU epilogue, 2/3 of the layer's FLOP). Its algorithmic FLOP per launch = 2 * (T k) * d * 2H;
its average launch duration is measured with HIP events recorded on the launch stream around
every launch inside the timed region. `traffic` (HBM bytes per launch) comes from the rocprofv3
FETCH_SIZE / WRITE_SIZE summary committed in profiles/traffic.json, when present.

cpu_baseline: the CPU oracle (a restatement of the reference's eager per-expert PyTorch loop,
fp32) timed on this host's cores on the same workload, on rank 0 only.
"""
import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "MoE layer tokens/s; grouped-GEMM % MFMA peak (32e top-4, T=16K, bf16)"
PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawTextHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=50)
    p.add_argument("--config", type=int, default=2, choices=[1, 2, 3, 4])
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--permute-rows", action="store_true",
                   help="move token rows with the permute kernel instead of gathering in the GEMM")
    p.add_argument("--cpu-budget-s", type=float, default=20.0)
    p.add_argument("--calibrate-copy", action="store_true",
                   help="only run a plain 1 GiB device-to-device copy (known HBM bytes), used to "
                        "scale rocprofv3 FETCH_SIZE / WRITE_SIZE readings")
    return p.parse_args()


def calibrate_copy(reps=20, nbytes=1 << 30):
    """A plain copy of known size: reads and writes `nbytes` per launch."""
    import torch
    src = torch.empty(nbytes // 2, device="cuda", dtype=torch.bfloat16).normal_()
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        dst.copy_(src)
    b.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / reps
    print(json.dumps({"copy_bytes_read": nbytes, "copy_bytes_written": nbytes,
                      "avg_launch_ms": round(ms, 5),
                      "GB_per_s": round(2 * nbytes / (ms * 1e-3) / 1e9, 1)}), flush=True)


def gpu_inputs(case):
    import torch
    from tests.moe_cases import make_inputs
    cpu = make_inputs(case)
    dev = torch.device("cuda")
    bf = lambda t: None if t is None else t.to(torch.bfloat16).to(dev)
    return cpu, dict(x=cpu["x"].to(dev), wt=cpu["router"].t().contiguous().to(dev),
                     w1=bf(cpu["w1"]), w2=bf(cpu["w2"]), sw1=bf(cpu["shared_w1"]),
                     sw2=bf(cpu["shared_w2"]),
                     bias=None if cpu["bias"] is None else cpu["bias"].to(dev))


def layer_flops(case):
    from oracle.moe_oracle import tflops
    return tflops(case.T, case.d, case.E, case.k, case.H, case.shared_H)


def load_traffic(case_key):
    path = ROOT / "profiles" / "traffic.json"
    if not path.exists():
        return None
    try:
        return json.loads(path.read_text()).get(case_key, {}).get("gemm_up_bytes")
    except (OSError, ValueError):
        return None


def cpu_baseline(case, cpu, budget_s):
    """The oracle's eager per-expert fp32 forward (reference semantics) on the host cores."""
    import torch
    from oracle import moe_oracle as orc
    threads = min(len(os.sched_getaffinity(0)), 16)
    torch.set_num_threads(threads)
    weights = orc.Weights(router=cpu["router"], w1=cpu["w1"], w2=cpu["w2"],
                          shared_w1=None if cpu["shared_w1"] is None else cpu["shared_w1"][0],
                          shared_w2=None if cpu["shared_w2"] is None else cpu["shared_w2"][0],
                          bias=cpu["bias"])
    x = cpu["x"]

    def run(tokens):
        t0 = time.perf_counter()
        orc.moe_forward(x[:tokens], weights, case.k, score_fn=case.score_fn,
                        activation=case.activation, router="reference")
        return time.perf_counter() - t0

    first = run(case.T)  # warm-up, also sizes the sample
    reps = max(1, min(5, int(budget_s / max(first, 1e-3))))
    times = sorted(run(case.T) for _ in range(reps))
    med = times[len(times) // 2]
    return dict(value=case.T / med, unit="tokens/s", cores=threads, kind="port",
                sample=f"full workload ({case.T} tokens), oracle eager per-expert fp32 loop with "
                       f"the reference's F.linear router, median of {reps} after 1 warm-up",
                ms_per_step=med * 1e3)


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        log("bench.py: this build is single-GPU only (one MI355X, no collectives); "
            f"--gpus {args.gpus} / WORLD_SIZE {world} is not supported.")
        sys.exit(2)

    if args.calibrate_copy:
        calibrate_copy()
        return

    import torch
    from nexttransformer_amd import ops
    from tests.moe_cases import CONFIGS

    case = CONFIGS[args.config]
    log(f"[bench] config {args.config}: {case}")
    cpu, g = gpu_inputs(case)
    torch.cuda.synchronize()

    def forward(mark=None):
        return ops.moe_forward(g["x"], g["wt"], g["w1"], g["w2"], top_k=case.k,
                               score_fn=case.score_fn, activation=case.activation,
                               logit_bias=g["bias"], shared_w1=g["sw1"], shared_w2=g["sw2"],
                               permute_rows=args.permute_rows, mark=mark)

    for _ in range(args.warmup):
        forward()
    torch.cuda.synchronize()
    log(f"[bench] warm-up done ({args.warmup} steps)")

    # Timed region: K full forwards; HIP events bracket every up-projection GEMM launch.
    stream = torch.cuda.current_stream()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        def mark(name, i=i):
            if name == "route_plan":
                ev[i][0].record(stream)
            elif name == "gemm_up":
                ev[i][1].record(stream)
        forward(mark)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms = (t1 - t0) * 1e3 / args.steps
    up_ms = sum(a.elapsed_time(b) for a, b in ev) / args.steps
    log(f"[bench] timed {args.steps} steps: {ms:.4f} ms/step, gemm_up {up_ms:.4f} ms")

    # Per-stage breakdown (separate instrumented pass, outside the timed region).
    names = ["router", "route_plan", "gemm_up", "gemm_down", "shared", "combine"]
    reps = 10
    stage = {n: 0.0 for n in names}
    for _ in range(reps):
        evs = [("start", torch.cuda.Event(enable_timing=True))]
        evs[0][1].record(stream)

        def mark(name):
            e = torch.cuda.Event(enable_timing=True)
            e.record(stream)
            evs.append((name, e))
        forward(mark)
        torch.cuda.synchronize()
        for (_, a), (n, b) in zip(evs, evs[1:]):
            stage[n] += a.elapsed_time(b) / reps
    stage = {n: round(v, 5) for n, v in stage.items() if v > 0}

    A = case.T * case.k
    F = 2 * case.H if case.activation == 0 else case.H
    up_flop = 2.0 * A * case.d * F
    achieved = up_flop / (up_ms * 1e-3) / 1e12
    traffic = load_traffic(f"config{args.config}")
    result = {
        "metric": METRIC,
        "value": round(case.T / (ms * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: hidden ~N(0,1), router/expert weights ~N(0,0.02) random init, seed 0",
        "config": {
            "workload": f"MoE layer forward, config {args.config}: T={case.T}, d={case.d}, "
                        f"E={case.E}, top-{case.k} {'softmax' if case.score_fn == 0 else 'sigmoid'}, "
                        f"{'SwiGLU' if case.activation == 0 else 'ReLU2'} H={case.H}"
                        + (f", shared H={case.shared_H}" if case.shared_H else "")
                        + (f", Zipf({case.zipf_bias}) logit bias" if case.zipf_bias else "")
                        + ", dropless",
            "tokens": case.T, "d_model": case.d, "experts": case.E, "top_k": case.k,
            "expert_hidden": case.H, "rows_gathered_in_gemm": not args.permute_rows,
        },
        "roofline": {
            "kernel": "grouped_gemm_kernel (up-projection + SwiGLU epilogue)",
            "bound": "mfma",
            "achieved": round(achieved, 2),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
            "traffic": traffic,
            "flop_per_launch": up_flop,
            "avg_launch_ms": round(up_ms, 5),
        },
        "layer_tflops": round(layer_flops(case) / (ms * 1e-3) / 1e12, 2),
        "stages_ms": stage,
    }
    if not args.no_cpu_baseline:
        log("[bench] cpu baseline ...")
        result["cpu_baseline"] = cpu_baseline(case, cpu, args.cpu_budget_s)
        log(f"[bench] cpu baseline {result['cpu_baseline']['value']:.1f} tokens/s")
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
