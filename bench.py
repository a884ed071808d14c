"""MoE layer forward benchmark on one MI355X.

    python bench.py [--steps K] [--warmup W] [--config 2] [--no-cpu-baseline]

A step is one full MoE layer forward (router -> histogram/scan -> permute plan -> grouped
expert GEMMs -> combine + aux loss) over one batch of synthetic input already resident in HBM.
Before the W warm-up steps, untimed forwards run for --settle-ms of wall time (default 300 ms):
the GPU raises its clocks only under sustained load, and without them a short run such as
--steps 20 --warmup 5 times its forwards 8-11 % slower than a settled one (measured side by side).
Default workload: config 2 (T=16384 = 8 x 2048, d=1024, 32 experts, top-4 softmax, SwiGLU H=512,
bf16, dropless). Configs 1-4 run the bf16 path; config 5 (T=64, d=4096, 128 experts, top-8,
H=1536) runs the fp8 path (e4m3 weights with 128 x 128 block scales, activations quantised per
row on the fly). Prints ONE JSON line.

roofline: the dominant kernel is the grouped up-projection GEMM (gate/value GEMM with the fused
SwiGLU epilogue, 2/3 of the layer's FLOP). bf16 configs: bound "mfma", algorithmic FLOP per
launch = 2 * (T k) * d * 2H. Config 5: bound "hbm", algorithmic bytes per launch = the e4m3
weights and scales of the experts that received tokens + the quantised token rows once + h
written. The average launch duration is measured with HIP events recorded on the launch stream
around the launches of every --event-every-th forward (default 8) inside the timed region: an
event record writes back the L2 of every XCD and idles the stream for about 6 us, so events
around every launch would add 12 us to every step. With --graph the timed forwards replay HIP graphs
captured from the forward (three segments, so the events sit between replays), and the replays'
output is checked bit for bit against an eager forward. `traffic` (HBM bytes per launch) comes from the
rocprofv3 FETCH_SIZE / WRITE_SIZE summary in profiles/traffic.json, when present.

cpu_baseline: the reference's eager CPU layer restated with torch's own ops (oracle/, the
RoutedFFN loop of reference_blocks.py:35-45 in fp32) timed on this host on the same workload,
with every core of the affinity mask and with one thread.
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


class DeviceEvent:
    """A HIP timing event recorded with a device-scope release (hipEventReleaseToDevice).
    torch.cuda.Event's record releases to system scope: the L2 is written back and invalidated
    at every record, which idles the GPU for about 6 us between the kernels the event separates
    and starts the next kernel on a cold L2. The events here only time work on this GPU."""
    _hip = None
    _RELEASE_TO_DEVICE = 0x40000000

    @classmethod
    def _lib(cls):
        if cls._hip is None:
            import ctypes
            import torch
            torch.cuda.init()
            # the HIP runtime torch loaded (the native library binds to the same one)
            with open("/proc/self/maps") as f:
                path = next(line.split()[-1] for line in f if "libamdhip64" in line)
            lib = ctypes.CDLL(path)
            vp = ctypes.c_void_p
            lib.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(vp), ctypes.c_uint]
            lib.hipEventRecord.argtypes = [vp, vp]
            lib.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), vp, vp]
            cls._hip = lib
        return cls._hip

    def __init__(self):
        import ctypes
        self._ctypes = ctypes
        self.ev = ctypes.c_void_p()
        rc = self._lib().hipEventCreateWithFlags(ctypes.byref(self.ev), self._RELEASE_TO_DEVICE)
        if rc != 0:
            raise RuntimeError(f"hipEventCreateWithFlags failed: {rc}")

    def record(self, stream=None):
        import torch
        stream = stream if stream is not None else torch.cuda.current_stream()
        rc = self._lib().hipEventRecord(self.ev, self._ctypes.c_void_p(stream.cuda_stream))
        if rc != 0:
            raise RuntimeError(f"hipEventRecord failed: {rc}")

    def elapsed_time(self, end):
        ms = self._ctypes.c_float()
        rc = self._lib().hipEventElapsedTime(self._ctypes.byref(ms), self.ev, end.ev)
        if rc != 0:
            raise RuntimeError(f"hipEventElapsedTime failed: {rc}")
        return ms.value
    # (no destructor: the few events of a run live until the process ends, and destroying them
    # during interpreter shutdown could run after the HIP runtime is gone)


def parse():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawTextHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--event-every", type=int, default=8,
                   help="time the up-projection launch with HIP events in every N-th timed "
                        "forward (each event record idles the stream about 6 us)")
    p.add_argument("--warmup", type=int, default=50)
    p.add_argument("--settle-ms", type=float, default=300.0,
                   help="before the warm-up steps, run forwards for at least this long (wall "
                        "time): the GPU raises its clocks only after some milliseconds of load, "
                        "so without it a short run (--steps 20 --warmup 5) times the first "
                        "forwards at low clocks, 8-11 %% slower than a settled run")
    p.add_argument("--config", type=int, default=2, choices=[1, 2, 3, 4, 5, 6],
                   help="1-5: the benchmark configurations; 6: the registered T3 expert cell "
                        "(moe-T3-L20 shapes) on 16384 tokens")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--permute-rows", action="store_true",
                   help="move token rows with the permute kernel instead of gathering in the GEMM")
    p.add_argument("--graph", action="store_true",
                   help="replay HIP graphs captured from the forward in the timed region instead of "
                        "launching every kernel from Python (slower on ROCm 7 at config 2: "
                        "0.323 vs 0.301 ms per forward)")
    p.add_argument("--train", action="store_true",
                   help="time forward + backward (bf16 configs) instead of the forward")
    p.add_argument("--gemms", action="store_true",
                   help="time the grouped GEMMs alone (bf16 configs) on the configuration's "
                        "routing: packed weights (where the widths allow) and plain ones, up and "
                        "down projection, --steps launches each; prints one JSON line")
    p.add_argument("--cpu-budget-s", type=float, default=30.0)
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
    a, b = DeviceEvent(), DeviceEvent()
    a.record()
    for _ in range(reps):
        dst.copy_(src)
    b.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / reps
    print(json.dumps({"copy_bytes_read": nbytes, "copy_bytes_written": nbytes,
                      "avg_launch_ms": round(ms, 5),
                      "GB_per_s": round(2 * nbytes / (ms * 1e-3) / 1e9, 1)}), flush=True)


def train_layer(case, cpu):
    """An MoELayer (aux gradient injected at scale 1) holding the case's weights as its fp32
    masters (and the case's logit bias, if any)."""
    import torch
    from nexttransformer_amd.moe import MoELayer
    from nexttransformer_amd.moe_recipe import MoERecipe
    recipe = MoERecipe(layers=2, width=case.d, heads=max(1, case.d // 64), sequence_len=case.T,
                       global_batch_tokens=case.T, routed_experts=case.E, top_k=case.k,
                       expert_width=case.H, score_function=("softmax", "sigmoid")[case.score_fn],
                       activation=("swiglu", "relu2")[case.activation],
                       shared_experts=1 if case.shared_H else 0,
                       shared_expert_width=case.shared_H or None, allow_any_expert_width=True)
    layer = MoELayer(recipe, 1)
    with torch.no_grad():
        layer.router.weight.copy_(cpu["router"])
        for i, e in enumerate(layer.experts.local_experts):
            e.linear_fc1.weight.copy_(cpu["w1"][i])
            e.linear_fc2.weight.copy_(cpu["w2"][i])
        if case.shared_H:
            layer.shared_experts.linear_fc1.weight.copy_(cpu["shared_w1"][0])
            layer.shared_experts.linear_fc2.weight.copy_(cpu["shared_w2"][0])
    if cpu["bias"] is not None:
        layer.logit_bias = cpu["bias"].cuda()
    return layer


def train_bench(args, case, cpu, g):
    """Training steps of the module: MoELayer forward + backward through autograd (loss = <out, G>
    with a fixed random G, the aux-loss gradient injected at scale 1), bf16 experts. A step's
    time is the forward + backward on the layer's cached operands plus the rebuild of those
    operands from the fp32 masters that every optimizer update triggers (bf16 cast / pack, the
    backward's transposed operands), timed on its own after bumping every master's version
    (gradient-accumulation micro-steps skip the rebuild). Prints one JSON line; the per-stage
    split comes from a separate instrumented pass of ops.moe_forward / ops.moe_backward on the
    same cached operands."""
    import torch
    from nexttransformer_amd import ops
    from nexttransformer_amd.moe import set_aux_loss_scale
    if g["w1_scale"] is not None:
        log("bench.py --train: the backward covers bf16 experts")
        sys.exit(2)
    set_aux_loss_scale(1.0, device="cuda")
    layer = train_layer(case, cpu)
    params = list(layer.parameters())
    x = g["x"]
    G = torch.randn(case.T, case.d, generator=torch.Generator().manual_seed(1)).to(
        torch.bfloat16).cuda()

    def step():
        for p in params:
            p.grad = None
        out, _ = layer(x)
        out.backward(G)

    def prepare():
        """Rebuilds every operand the kernels read from the masters (as after an optimizer
        step): the bf16 cast / pack, the backward's transposed operands and the router's."""
        w = layer.packed_weights(keep_plain=True)
        bw = layer.backward_weights(w)
        bw.w1t, bw.w2t, bw.shared, bw.first(w["router_t"])
        w1 = w["w1"]
        n_out = w1.shape[1] // 2 if case.activation == 0 else w1.shape[1]
        packed_up = w["packed"] if isinstance(w["packed"], bool) else w["packed"][0]
        if not packed_up and not ops.plain_keep_supported(w1.shape[2], n_out):
            bw.w1  # the fc1 recompute operand: the forward keeps no fc1 then

    for _ in range(max(1, args.warmup)):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    ms_step = (time.perf_counter() - t0) * 1e3 / args.steps
    prep = []
    for _ in range(5):
        with torch.no_grad():
            for p in params:
                p.add_(0.0)  # a new version of every master
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        prepare()
        torch.cuda.synchronize()
        prep.append((time.perf_counter() - t0) * 1e3)
    prep_ms = sorted(prep)[len(prep) // 2]
    # Steps as a training loop runs them, each after a weight update: every master's version
    # counter is bumped before the step (as an optimizer's in-place update bumps it; no kernel
    # runs), so each forward first rebuilds the operands, its host work overlapping the kernels
    # still queued from the step before. This loop's time per step is ms_per_step; the parts
    # above, timed apart (the rebuild behind a synchronize), sum to ms_sum_of_parts.
    bump = torch.autograd.graph.increment_version
    for _ in range(2):
        bump(params)
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        bump(params)
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps

    # per-stage split on the layer's cached operands
    w = layer.packed_weights(keep_plain=True)
    bw = layer.backward_weights(w)
    stream = torch.cuda.current_stream()
    stage, reps, kept = {}, 5, None
    for _ in range(reps):
        evs = [("start", DeviceEvent())]
        evs[0][1].record(stream)

        def mark(name):
            e = DeviceEvent()
            e.record(stream)
            evs.append((name, e))
        _, _, st = ops.moe_forward(x, w["router_t"], w["w1"], w["w2"], top_k=case.k,
                                   score_fn=case.score_fn, activation=case.activation,
                                   logit_bias=layer.logit_bias, shared_w1=w["shared_w1"],
                                   shared_w2=w["shared_w2"], packed=w["packed"],
                                   want_logits=True, keep=True, mark=lambda n: mark("fwd_" + n))
        kept = st["fc1"] is not None
        kept_shared = st["shared_fc1"] is not None
        ops.moe_backward(G, torch.tensor([1.0, 0.0, 0.0], device="cuda"), x, w["router_t"], bw,
                         st, top_k=case.k, score_fn=case.score_fn, activation=case.activation,
                         mark=lambda n: mark("bwd_" + n))
        torch.cuda.synchronize()
        for (_, a), (n, b) in zip(evs, evs[1:]):
            stage[n] = stage.get(n, 0.0) + a.elapsed_time(b) / reps
    A = case.T * case.k
    F = 2 * case.H if case.activation == 0 else case.H
    Fs = 2 * case.shared_H if case.activation == 0 else case.shared_H
    up, down = 2.0 * A * case.d * F, 2.0 * A * case.H * case.d
    sup, sdown = 2.0 * case.T * case.d * Fs, 2.0 * case.T * case.shared_H * case.d
    router = 2.0 * case.T * case.d * case.E
    # forward: up + down; backward: dgrad and wgrad of both (+ the fc1 recompute when the forward
    # kept no pre-activations); the shared expert likewise; the router GEMM once forward and its
    # two gradient products
    flops = ((3 if kept else 4) * up + 3 * down + (3 if kept_shared else 4) * sup + 3 * sdown
             + 3 * router)
    wg_ms = stage.get("bwd_wgrad", 0.0)
    wg_flop = up + down + sup + sdown
    wg_tflops = wg_flop / (wg_ms * 1e-3) / 1e12 if wg_ms > 0 else None
    result = {"metric": "MoE layer training step (forward + backward) tokens/s",
              "value": round(case.T / (ms * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1,
              "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 5),
              "ms_forward_backward": round(ms_step, 5),
              "ms_weight_preparation": round(prep_ms, 5),
              "ms_sum_of_parts": round(ms_step + prep_ms, 5),
              "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
              "data": "synthetic, seed 0", "config": describe(case, args.config, False, False),
              "path": "MoELayer forward + autograd backward, each step after a weight "
                      "update (the operands rebuilt from the fp32 masters in every step); "
                      "apart: the steps on cached operands and the rebuild alone (median of 5)",
              "fc1_kept_by_forward": kept,
              "layer_tflops": round(flops / (ms * 1e-3) / 1e12, 2),
              "stages_ms": {n: round(v, 5) for n, v in stage.items()},
              "roofline": None if wg_tflops is None else {
                  "kernel": "grouped_wgrad_kernel (dW1 + dW2, shared expert's)", "bound": "mfma",
                  "achieved": round(wg_tflops, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                  "frac": round(wg_tflops / PEAK_BF16_TFLOPS, 4), "traffic": None,
                  "flop_per_step": wg_flop, "ms_per_step": round(wg_ms, 5)}}
    print(json.dumps(result), flush=True)


class Segments(list):
    """HIP graphs of consecutive pieces of one forward (replayed in order), with its outputs."""
    out = None
    aux = None


def capture_segments(forward, cuts):
    """Captures forward(mark) into len(cuts) + 1 HIP graphs that share one memory pool: a new
    graph starts after each stage named in `cuts` (mark is called once a stage is enqueued).
    The forward must have run eagerly before (the library's lazy set-up stays out of capture)."""
    import torch
    graphs = Segments([torch.cuda.CUDAGraph()])
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    pool = torch.cuda.graph_pool_handle()
    with torch.cuda.stream(side):
        graphs[0].capture_begin(pool=pool)

        def mark(name):
            if name in cuts:
                graphs[-1].capture_end()
                graphs.append(torch.cuda.CUDAGraph())
                graphs[-1].capture_begin(pool=pool)
        graphs.out, graphs.aux, _ = forward(mark)
        graphs[-1].capture_end()
    torch.cuda.current_stream().wait_stream(side)
    if len(graphs) != len(cuts) + 1:
        raise RuntimeError(f"capture_segments: the forward marked {len(graphs) - 1} of the "
                           f"{len(cuts)} cut points")
    return graphs


def gpu_inputs(case, fp8):
    import torch
    from nexttransformer_amd import ops
    from tests.moe_cases import make_inputs
    cpu = make_inputs(case)
    dev = torch.device("cuda")
    g = dict(x=cpu["x"].to(dev), wt=cpu["router"].t().contiguous().to(dev),
             bias=None if cpu["bias"] is None else cpu["bias"].to(dev))
    for name in ("w1", "w2", "shared_w1", "shared_w2"):
        g[name], g[name + "_scale"] = None, None
        if cpu[name] is None:
            continue
        if fp8:
            g[name], g[name + "_scale"] = ops.quantize_fp8_blockwise(cpu[name].to(dev))
        else:
            g[name] = cpu[name].to(torch.bfloat16).to(dev)
    # the packed-weight grouped GEMMs: always for fp8; for bf16 the up projections' weights
    # when every up projection (routed, shared) qualifies, the down projections' likewise
    g["packed"] = False
    if fp8:
        from nexttransformer_amd import _native as nat
        up = nat.EPI_SWIGLU if case.activation == 0 else nat.EPI_RELU2
        for n, e in (("w1", up), ("w2", nat.EPI_NONE), ("shared_w1", up), ("shared_w2", nat.EPI_NONE)):
            if g[n] is not None:
                g[n] = ops.pack_expert_weights_fp8(g[n], e)
        g["packed"] = True
    else:
        from nexttransformer_amd import _native as nat
        up = nat.EPI_SWIGLU if case.activation == 0 else nat.EPI_RELU2
        names = [["w1"], ["w2"]]
        if g["shared_w1"] is not None:
            names[0].append("shared_w1")
            names[1].append("shared_w2")
        pk = []
        for group, e in zip(names, (up, nat.EPI_NONE)):
            ok = all(ops.prefers_packed(g[n].shape[2],
                                        g[n].shape[1] // (2 if e == nat.EPI_SWIGLU else 1), e,
                                        repacked_each_step=False)  # packed once, as inference
                     for n in group)
            if ok:
                for n in group:
                    g[n] = ops.pack_expert_weights(g[n], e)
            pk.append(ok)
        g["packed"] = tuple(pk)
    torch.cuda.synchronize()
    return cpu, g


def layer_flops(case):
    """Algorithmic FLOP of one forward: router 2 T d E + routed experts 2 (T k) d F + 2 (T k) H d
    (F = 2H for SwiGLU, H for ReLU^2) + the shared expert's 2 T d Fs + 2 T Hs d."""
    F = 2 * case.H if case.activation == 0 else case.H
    Fs = 2 * case.shared_H if case.activation == 0 else case.shared_H
    A = case.T * case.k
    return (2 * case.T * case.d * case.E + 2 * A * case.d * (F + case.H)
            + 2 * case.T * case.d * (Fs + case.shared_H))


def load_traffic(case_key):
    path = ROOT / "profiles" / "traffic.json"
    if not path.exists():
        return None
    try:
        return json.loads(path.read_text()).get(case_key, {}).get("gemm_up_bytes")
    except (OSError, ValueError):
        return None


def cpu_baseline(case, cpu, budget_s):
    """The reference's eager CPU layer (torch ops: F.linear router, topk, softmax over the
    selected, per-expert torch.where / index_add loop, shared expert; fp32) timed on the host:
    with every core of this process's affinity mask and with one thread (the reference CI's
    OMP_NUM_THREADS=1). Median of up to 5 runs after 2 warm-ups per thread count. The sample is
    the full workload when a run fits the budget, else its first T' tokens (scaled to tokens/s)."""
    import torch
    from oracle import moe_oracle as orc
    weights = orc.Weights(router=cpu["router"], w1=cpu["w1"], w2=cpu["w2"],
                          shared_w1=None if cpu["shared_w1"] is None else cpu["shared_w1"][0],
                          shared_w2=None if cpu["shared_w2"] is None else cpu["shared_w2"][0],
                          bias=cpu["bias"])
    threads_all = len(os.sched_getaffinity(0))
    before = torch.get_num_threads()

    def measure(threads, tokens, share):
        torch.set_num_threads(threads)
        x = cpu["x"][:tokens]

        def run():
            t0 = time.perf_counter()
            orc.reference_eager_forward(x, weights, case.k, score_fn=case.score_fn,
                                        activation=case.activation)
            return time.perf_counter() - t0
        first = run()
        # the second warm-up, then as many timed runs (<= 5) as this thread count's share allows
        reps = max(1, min(5, int((share - 2 * first) / max(first, 1e-3))))
        run()
        times = sorted(run() for _ in range(reps))
        med = times[len(times) // 2]
        return dict(value=round(tokens / med, 1), unit="tokens/s", cores=threads,
                    ms_per_sample=round(med * 1e3, 3), sample_tokens=tokens, runs=reps)
    try:
        multi = measure(threads_all, case.T, budget_s / 3)
        # one thread: size the sample so that one run takes about 1/8 of its share
        torch.set_num_threads(1)
        probe = min(case.T, 1024)
        t0 = time.perf_counter()
        orc.reference_eager_forward(cpu["x"][:probe], weights, case.k, score_fn=case.score_fn,
                                    activation=case.activation)
        per_token_1t = (time.perf_counter() - t0) / probe
        tokens_1t = int(min(case.T, max(64, (2 * budget_s / 3) / 8 / per_token_1t)))
        single = measure(1, tokens_1t, 2 * budget_s / 3)
    finally:
        torch.set_num_threads(before)
    out = dict(multi, kind="port",
               sample=f"reference eager CPU layer (torch ops, fp32) on {multi['sample_tokens']} "
                      f"tokens of the workload, {threads_all} threads (this process's affinity "
                      f"mask), median of {multi['runs']} after 2 warm-ups",
               single_thread=dict(single, sample=f"same path, 1 thread, first "
                                                 f"{single['sample_tokens']} tokens, median of "
                                                 f"{single['runs']} after 2 warm-ups"))
    return out


def describe(case, cfg, permute_rows, fp8):
    act = "SwiGLU" if case.activation == 0 else "ReLU2"
    score = "softmax" if case.score_fn == 0 else "sigmoid (normalised over top-k)"
    text = (f"MoE layer forward, config {cfg}: T={case.T}, d={case.d}, E={case.E}, "
            f"top-{case.k} {score}, {act} H={case.H}")
    if case.shared_H:
        text += f", shared expert H={case.shared_H}"
    if case.zipf_bias:
        text += f", Zipf({case.zipf_bias}) logit bias"
    if fp8:
        text += ", fp8 e4m3 experts (128x128 block scales, per-row activation scales)"
    return {"workload": text + ", dropless", "tokens": case.T, "d_model": case.d,
            "experts": case.E, "top_k": case.k, "expert_hidden": case.H,
            "shared_hidden": case.shared_H, "rows_gathered_in_gemm": not permute_rows,
            "expert_weights": "fp8 e4m3 + block scales" if fp8 else "bf16"}


def gemm_bench(args, case, cpu):
    """Median launch time of each grouped GEMM of the layer on the configuration's routing."""
    import torch
    from nexttransformer_amd import _native as nat, ops
    dev = torch.device("cuda")
    x = cpu["x"].to(dev)
    wt = cpu["router"].t().contiguous().to(dev)
    bias = None if cpu["bias"] is None else cpu["bias"].to(dev)
    _, ids, w, _, _ = ops.router(x, wt, bias, case.k, case.score_fn, False)
    _, offsets, src, _, _, _, _ = ops.route_plan(ids, w, case.E, None, False)
    A = case.T * case.k
    up = nat.EPI_SWIGLU if case.activation == 0 else nat.EPI_RELU2
    w1 = cpu["w1"].to(torch.bfloat16).to(dev)
    w2 = cpu["w2"].to(torch.bfloat16).to(dev)
    h = ops.grouped_gemm(x, src, offsets, w1, up, A)
    F = w1.shape[1]
    runs = {"plain_up": lambda: ops.grouped_gemm(x, src, offsets, w1, up, A),
            "plain_down": lambda: ops.grouped_gemm(h, None, offsets, w2, nat.EPI_NONE, A)}
    if ops.packable(case.d, F // 2 if up == nat.EPI_SWIGLU else F, up):
        w1p = ops.pack_expert_weights(w1, up)
        runs["packed_up"] = lambda: ops.grouped_gemm_packed(x, src, offsets, w1p, up, A)
    if ops.packable(case.H, case.d, nat.EPI_NONE):
        w2p = ops.pack_expert_weights(w2, nat.EPI_NONE)
        runs["packed_down"] = lambda: ops.grouped_gemm_packed(h, None, offsets, w2p, nat.EPI_NONE, A)
    flop = {"up": 2.0 * A * case.d * F, "down": 2.0 * A * case.H * case.d}
    out = {"config": args.config, "launches": args.steps}
    for name, fn in runs.items():
        fn()
        torch.cuda.synchronize()
        evs = []
        for _ in range(args.steps):
            a, b = DeviceEvent(), DeviceEvent()
            a.record()
            fn()
            b.record()
            evs.append((a, b))
        torch.cuda.synchronize()
        ms = sorted(a.elapsed_time(b) for a, b in evs)[len(evs) // 2]
        tf = flop[name.split("_")[1]] / (ms * 1e-3) / 1e12
        out[name] = {"median_us": round(ms * 1e3, 2), "TFLOP/s": round(tf, 1),
                     "frac_of_bf16_peak": round(tf / PEAK_BF16_TFLOPS, 4)}
    print(json.dumps(out), flush=True)


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
    fp8 = args.config == 5
    log(f"[bench] config {args.config}: {case}")
    if args.gemms:
        if fp8:
            log("bench.py --gemms: bf16 configurations only")
            sys.exit(2)
        from tests.moe_cases import make_inputs
        gemm_bench(args, case, make_inputs(case))
        return
    cpu, g = gpu_inputs(case, fp8)

    def forward(mark=None):
        return ops.moe_forward(g["x"], g["wt"], g["w1"], g["w2"], top_k=case.k,
                               score_fn=case.score_fn, activation=case.activation,
                               logit_bias=g["bias"], shared_w1=g["shared_w1"],
                               shared_w2=g["shared_w2"], w1_scale=g["w1_scale"],
                               w2_scale=g["w2_scale"], shared_w1_scale=g["shared_w1_scale"],
                               shared_w2_scale=g["shared_w2_scale"],
                               permute_rows=args.permute_rows, packed=g["packed"], mark=mark)

    if args.train:
        train_bench(args, case, cpu, g)
        return

    state = None
    settle_n = 0
    if args.settle_ms > 0:
        t_settle = time.perf_counter()
        while (time.perf_counter() - t_settle) * 1e3 < args.settle_ms:
            for _ in range(10):
                forward()
            settle_n += 10
            torch.cuda.synchronize()
    for _ in range(max(1, args.warmup)):
        _, _, state = forward()
    torch.cuda.synchronize()
    counts = state["counts"].cpu()
    load_ratio = counts.max().item() / counts.float().mean().item()
    log(f"[bench] warm-up done ({args.warmup} steps); expert load max/mean {load_ratio:.2f}")

    # Timed region: K full forwards, every kernel launched from Python, with HIP events recorded
    # on the launch stream around the up-projection launch of every --event-every-th forward
    # (an event record releases the memory model's device scope, which on this GPU writes back
    # the L2 of every XCD and idles the stream about 6 us; recording around every launch would
    # add 12 us to every step). With --graph each forward instead replays three HIP graphs
    # captured from it (routing, the up-projection GEMM, the rest), the events recorded between
    # the replays of the sampled forwards.
    before_up = "quantize" if fp8 else "route_plan"
    stream = torch.cuda.current_stream()
    every = max(1, args.event_every)
    sampled = list(range(0, args.steps, every))
    ev = {i: (DeviceEvent(), DeviceEvent()) for i in sampled}
    graphs = capture_segments(forward, (before_up, "gemm_up")) if args.graph else None
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        pair = ev.get(i)
        if graphs is None:
            if pair is None:
                forward()
            else:
                def mark(name, pair=pair):
                    if name == before_up:
                        pair[0].record(stream)
                    elif name == "gemm_up":
                        pair[1].record(stream)
                forward(mark)
        else:
            graphs[0].replay()
            if pair is not None:
                pair[0].record(stream)
            graphs[1].replay()
            if pair is not None:
                pair[1].record(stream)
            graphs[2].replay()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms = (t1 - t0) * 1e3 / args.steps
    up_ms = sum(a.elapsed_time(b) for a, b in ev.values()) / len(ev)
    log(f"[bench] timed {args.steps} steps ({'eager' if graphs is None else 'graph replay'}): "
        f"{ms:.4f} ms/step, gemm_up {up_ms:.4f} ms")
    replay_ok = None
    if graphs is not None:  # the replays' results equal an eager forward's, bit for bit
        out_e, aux_e, _ = forward()
        torch.cuda.synchronize()
        replay_ok = bool(torch.equal(graphs.out.view(torch.int16), out_e.view(torch.int16))
                         and torch.equal(graphs.aux, aux_e))
        if not replay_ok:
            log("[bench] graph replay differs from the eager forward")
            sys.exit(1)

    # Per-stage breakdown (separate instrumented pass, outside the timed region).
    reps = 10
    stage = {}
    for _ in range(reps):
        evs = [("start", DeviceEvent())]
        evs[0][1].record(stream)

        def mark(name):
            e = DeviceEvent()
            e.record(stream)
            evs.append((name, e))
        forward(mark)
        torch.cuda.synchronize()
        for (_, a), (n, b) in zip(evs, evs[1:]):
            stage[n] = stage.get(n, 0.0) + a.elapsed_time(b) / reps
    stage = {n: round(v, 5) for n, v in stage.items()}

    A = case.T * case.k
    F = 2 * case.H if case.activation == 0 else case.H
    if fp8:
        touched = int((counts > 0).sum())
        up_bytes = (touched * F * case.d + touched * (F // 128) * (case.d // 128) * 4
                    + case.T * case.d + case.T * 4 + A * case.H * 2)
        achieved = up_bytes / (up_ms * 1e-3) / 1e9
        roofline = {"kernel": "fp8_grouped_gemm_kernel (up-projection, e4m3 weight streaming)",
                    "bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS,
                    "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4),
                    "traffic": load_traffic(f"config{args.config}"),
                    "bytes_per_launch": up_bytes, "experts_touched": touched,
                    "avg_launch_ms": round(up_ms, 5), "launches_timed": len(ev)}
    else:
        up_flop = 2.0 * A * case.d * F
        achieved = up_flop / (up_ms * 1e-3) / 1e12
        # the plain-weight entry point takes the 256x256 kernel when K >= 128 and the output
        # width is a multiple of 8 (nt_moe_grouped_gemm_bf16)
        n_out = case.H
        plain = "grouped_gemm_t256_kernel" if case.d >= 128 and n_out % 8 == 0 else "grouped_gemm_kernel"
        epi = "SwiGLU" if case.activation == 0 else "ReLU^2"
        roofline = {"kernel": ("grouped_gemm_packed_kernel" if g["packed"][0] else plain)
                              + f" (up-projection + {epi} epilogue)",
                    "bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
                    "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                    "traffic": load_traffic(f"config{args.config}"),
                    "flop_per_launch": up_flop, "avg_launch_ms": round(up_ms, 5),
                    "launches_timed": len(ev)}
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
        "dtype": "fp8-e4m3 (fp32 accumulate)" if fp8 else "bf16",
        "data": "synthetic: hidden ~N(0,1), router/expert weights ~N(0,0.02) random init, seed 0",
        "config": dict(describe(case, args.config, args.permute_rows, fp8),
                       weights_packed=(g["packed"] if fp8 else
                                       dict(up=g["packed"][0], down=g["packed"][1]))),
        "roofline": roofline,
        "layer_tflops": round(layer_flops(case) / (ms * 1e-3) / 1e12, 2),
        "expert_load_max_over_mean": round(load_ratio, 3),
        "stages_ms": stage,
        "launch": "eager" if graphs is None else "hip_graph_replay",
        "settle": {"ms": args.settle_ms, "forwards": settle_n},
        "graph_replay_matches_eager": replay_ok,
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
