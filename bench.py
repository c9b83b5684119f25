"""Benchmark of the Qwen3-30B-A3B Q8_0 MoE FFN path on one MI355X.

Default workload: the 48-layer MoE-only stack at decode batch 1 (each layer
RMSNorm -> MoE FFN -> residual, all 48 x 128 Q8_0 experts resident in HBM),
the configuration the HBM-roofline target is stated on. A step is one token
through the 48 layers; inputs and weights are synthetic (seeded, generated in
HBM) and resident before the timed region starts.

Prints one JSON line: throughput (tokens/s), the whole-step HBM rate, the
roofline of the dominant kernel (timed live with HIP events on the library's
stream) and the reference C path (the CPU oracle, one thread) timed on a
bounded sample of the same workload on this host.
"""
import argparse
import json
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import motoria_amd as M  # noqa: E402
from motoria_amd import workloads as W  # noqa: E402

HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense fp16/bf16 matrix peak
METRIC = "MoE tokens/s + achieved HBM GB/s (% of peak), Qwen3-30B-A3B shape, 1 GPU"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def profiled_traffic(workload, kernel):
    """HBM bytes per launch of `kernel` on `workload` from the committed
    rocprofv3 counter summary (FETCH_SIZE + WRITE_SIZE, each scaled by the
    same counter's reading over a copy of known size), or None."""
    path = os.path.join(ROOT, "profiles", "%s_%s_traffic.md" % (workload, kernel))
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def routing_census(moe, d_x, d_x0, layers, T, nbytes, d_bias):
    """One untimed pass layer by layer: distinct experts touched per layer."""
    moe.sync()
    M.lib().mhip_d2d(moe.gpu, d_x, d_x0, nbytes)
    touched = []
    for l in range(layers):
        moe.layer_dev(l, d_x, T, d_bias)
        moe.sync()
        touched.append(int(moe.d2h(moe.scratch().groups, 1, np.int32)[0]))
    return touched


def gateup_bytes(n_touched, T, shape):
    """Algorithmic bytes of one gate/up launch: the touched experts' gate and
    up Q8_0 blocks (36 B per 32 weights), the Q8 activations read, h written."""
    d, eh, K = shape["dim"], shape["expert_hidden"], shape["n_active"]
    w = n_touched * 2 * eh * (d // 32) * 36
    return w + T * d + T * (d // 32) * 4 + T * K * eh * 4


def gateup_flops(T, shape):
    """Algorithmic flops of one gate/up launch: 2 * assignments * (gate + up
    rows) * dim multiply-adds."""
    d, eh, K = shape["dim"], shape["expert_hidden"], shape["n_active"]
    return 2.0 * T * K * 2 * eh * d


def cpu_baseline(moe, wl, shape, sample_layers, sample_tokens):
    """The oracle (the reference C path restated, gcc -O3, one thread) on
    `sample_layers` layers x `sample_tokens` tokens of the same model; tokens
    are independent, so tokens/s of the full stack = 1 / (L * t_token_layer)."""
    import oracle as O

    d = O.dims(**shape)
    x = O.synth_x(W.X_SEED, sample_tokens, d.dim)
    norm = np.ones(d.dim, np.float32)
    t_cpu = 0.0
    for l in range(sample_layers):
        blobs = [moe.read_expert(l, e) for e in range(d.n_experts)]
        router = O.synth_router(W.WEIGHT_SEED, l, d)
        t0 = time.perf_counter()
        x, _, _, _, _ = O.moe_layer(d, x, norm, router, blobs, nthreads=1)
        t_cpu += time.perf_counter() - t0
        del blobs
    t_tl = t_cpu / (sample_layers * sample_tokens)
    tokens_per_s = 1.0 / (wl["layers"] * t_tl)
    return {
        "value": tokens_per_s,
        "unit": "tokens/s",
        "cores": 1,
        "kind": "port",
        "sample": ("oracle/mia_oracle.c (reference C path restated; gcc -std=c99 -O3 "
                   "-ffp-contract=off, 1 thread) on %d layers x %d tokens of the same "
                   "synthetic model = %.1f s CPU, %.2f ms per token-layer, scaled to %d "
                   "layers; host: %s, %d cpus visible"
                   % (sample_layers, sample_tokens, t_cpu, t_tl * 1e3, wl["layers"],
                      cpu_model(), os.cpu_count() or 0)),
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="decode48", choices=sorted(W.WORKLOADS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-layers", type=int, default=4)
    ap.add_argument("--cpu-tokens", type=int, default=768)
    ap.add_argument("--multi-kernel", action="store_true",
                    help="batch-1 workloads: one launch per stage instead of the "
                         "persistent decode kernel")
    args = ap.parse_args()

    if args.gpus != 1:
        print("bench.py: this build runs on one GPU only; multi-GPU sharding of the MoE "
              "path (expert-parallel all-to-all) is designed but not built. Use --gpus 1.",
              file=sys.stderr)
        sys.exit(2)
    if M.device_count() < 1:
        print("bench.py: no HIP device visible", file=sys.stderr)
        sys.exit(1)

    wl = W.WORKLOADS[args.workload]
    shape = dict(W.SHAPE)
    L, T = wl["layers"], wl["tokens"]
    d = shape["dim"]
    log("workload %s: %s" % (args.workload, wl["doc"]))

    t0 = time.perf_counter()
    moe = M.Moe(n_layers=L, max_tokens=T, device=0, **shape)
    moe.synth(W.WEIGHT_SEED)
    moe.sync()
    log("expert table (%d layers, %.2f GiB) generated in HBM in %.2f s"
        % (L, L * 128 * 5308416 / 2**30, time.perf_counter() - t0))
    nbytes = T * d * 4
    d_x0 = moe.malloc(nbytes)
    d_x = moe.malloc(nbytes)
    d_bias = None
    if wl["skew"]:
        d_bias = moe.malloc(shape["n_experts"] * 4)
        moe.h2d(d_bias, W.zipf_bias(shape["n_experts"]))
    moe.synth_f32(d_x0, T * d, W.X_SEED, 1 << 40, 1.0)

    persistent = T == 1 and not args.multi_kernel

    def step():
        if persistent:
            # decode: each step takes the previous step's output as its
            # token (K experts per layer whatever x is, so the bytes per step
            # do not depend on it)
            moe.decode_dev(0, L, d_x, d_bias)
            return
        M.lib().mhip_d2d(moe.gpu, d_x, d_x0, nbytes)
        if d_bias is None:
            moe.stack_dev(0, L, d_x, T)
        else:
            for l in range(L):
                moe.layer_dev(l, d_x, T, d_bias)

    touched = routing_census(moe, d_x, d_x0, L, T, nbytes, d_bias)
    step_bytes = W.bytes_per_step(L, T, touched, shape)
    step_ops = W.ops_per_step(L, T, shape)

    M.lib().mhip_d2d(moe.gpu, d_x, d_x0, nbytes)
    for _ in range(args.warmup):
        step()
    moe.sync()

    # Timed region: host clock between two stream synchronisations, HIP events
    # on the library stream, and events around every launch of the dominant
    # kernel (k_gateup per layer). A persistent decode step is one launch of
    # the dominant kernel, so the two region events time it (launch gaps
    # included); per-launch events would add their own gaps to the step.
    dom = "decode" if persistent else "gateup"
    moe.stage_timing([] if persistent else [dom], max_launches=L * args.steps + 16)
    moe.sync()
    t0 = time.perf_counter()
    moe.mark(0)
    for _ in range(args.steps):
        step()
    moe.mark(1)
    moe.sync()
    t1 = time.perf_counter()
    ev_ms = moe.elapsed_ms(0, 1)
    stage = {dom: (ev_ms, args.steps) if persistent else moe.stage_time(dom)}
    dstat = moe.decode_status() if persistent else None
    # Untimed diagnostic pass: every stage bracketed by events.
    diag_steps = min(args.steps, 5)
    moe.stage_timing(M.STAGES, max_launches=len(M.STAGES) * L * diag_steps + 16)
    for _ in range(diag_steps):
        step()
    moe.sync()
    diag = {s: moe.stage_time(s) for s in M.STAGES}
    moe.stage_timing([], 0)

    ms_step = (t1 - t0) * 1e3 / args.steps
    tokens_per_s = T / (ms_step / 1e3)
    hbm_gbs = step_bytes / (ms_step / 1e3) / 1e9
    dom_ms, dom_n = stage[dom]
    dom_avg_s = dom_ms / max(dom_n, 1) / 1e3
    if persistent:
        dom_bytes = step_bytes
        dom_name = ("k_decode_stack (persistent: %d layers of rmsnorm, router/top-8, "
                    "gate/up+SwiGLU, down, combine in one launch)" % L)
    else:
        dom_bytes = sum(gateup_bytes(n, T, shape) for n in touched) / len(touched)
        dom_name = "k_gateup (gate/up Q8_0 grouped GEMV + SwiGLU)"
    achieved = dom_bytes / dom_avg_s / 1e9
    # Large batches run the expert products on the matrix cores: the gate/up
    # kernel is then priced against the fp16 matrix peak.
    matrix = not persistent and T * shape["n_active"] >= M.GEMM_MIN_A
    if matrix:
        dom_name = ("k_gateup_mfma (gate/up on fp16 MFMA with the exact per-block Q8_0 "
                    "epilogue, SwiGLU, Q8(h))")
        dom_flops = gateup_flops(T, shape)
        achieved_tf = dom_flops / dom_avg_s / 1e12
    for s in M.STAGES:
        ms, n = diag[s]
        if n:
            log("  stage %-8s %4d launches, avg %8.2f us, %5.1f %% of step (diagnostic pass)"
                % (s, n, ms / max(n, 1) * 1e3, 100.0 * ms / (ms_step * diag_steps)))
    if dstat is not None:
        log("decode status %s (abort bits, rmsnorm fallbacks, exact-router layers)" % dstat)
        if dstat[0]:
            print("bench.py: the decode kernel aborted (%s)" % dstat, file=sys.stderr)
            sys.exit(1)
    log("step %.3f ms (events %.3f ms), %.1f tokens/s, %.1f GB/s algorithmic"
        % (ms_step, ev_ms / args.steps, tokens_per_s, hbm_gbs))

    cpu = None
    if not args.no_cpu:
        t0 = time.perf_counter()
        cpu = cpu_baseline(moe, wl, shape, min(args.cpu_layers, L), args.cpu_tokens)
        log("cpu baseline: %.2f tokens/s (%.1f s)" % (cpu["value"], time.perf_counter() - t0))

    out = {
        "metric": METRIC,
        "value": tokens_per_s,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 x int8 -> int32 block dots, fp32 scales/accumulation (Q8_0)",
        "data": "synthetic: seeded N(0,0.02) weights quantized to Q8_0, x ~ N(0,1), "
                "generated in HBM (no checkpoint offline)"
                + ("; each decode step continues from the previous step's x" if persistent else ""),
        "config": {
            "workload": "%s: %s" % (args.workload, wl["doc"]),
            "layers": L, "tokens_per_step": T, "hidden": d,
            "experts": shape["n_experts"], "top_k": shape["n_active"],
            "expert_hidden": shape["expert_hidden"], "weights": "Q8_0 (36-byte blocks)",
            "zipf_bias": bool(wl["skew"]), "experts_touched_per_layer": touched[:4] + (
                ["..."] if len(touched) > 4 else []),
        },
        "hbm": {"bytes_per_step": step_bytes, "achieved_gbs": hbm_gbs,
                "frac": hbm_gbs / HBM_PEAK_GBS, "ops_per_step": step_ops},
        "roofline": ({
            "kernel": dom_name,
            "bound": "mfma",
            "achieved": achieved_tf,
            "peak": MFMA_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": achieved_tf / MFMA_PEAK_TFLOPS,
            "traffic": None,
            "flops_per_launch": dom_flops,
            "avg_launch_us": dom_avg_s * 1e6,
            "layer_ops_tflops": step_ops / (ms_step / 1e3) / 1e12,
        } if matrix else {
            "kernel": dom_name,
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": profiled_traffic(args.workload, "k_decode_stack" if persistent else "k_gateup"),
            "bytes_per_launch": dom_bytes,
            "avg_launch_us": dom_avg_s * 1e6,
        }),
        "path": ("persistent decode kernel" if persistent else
                 "one launch per stage, expert products on the matrix cores" if matrix else
                 "one launch per stage"),
        "cpu_baseline": cpu,
    }
    print(json.dumps(out))
    moe.free(d_x)
    moe.free(d_x0)
    if d_bias:
        moe.free(d_bias)
    moe.close()


if __name__ == "__main__":
    main()
