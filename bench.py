"""Benchmark of the causal RACE hot path on one MI355X.

Headline (BASELINE.json metric "RACE layer fwd+bwd tokens/sec at 1M ctx"):
one causal RACE layer forward+backward, B=1, H=4, T=2^20, D=64, L=8, K=4,
bf16 q/k/v ~ N(0, 1/sqrt(D)) and upstream grad ~ N(0,1), planes seed 0, inputs
drawn from torch.Generator(cuda).manual_seed(1) in the order q, k, v, go and
resident in HBM before the timed region. A step is forward + backward of the
layer; value = B*T / seconds per step.

The same JSON line also carries:
  roofline       dominant kernel of the step: algorithmic HBM bytes per launch over
                 its average launch time (HIP events inside librace_amd, on the
                 launch stream), against 8 TB/s
  layer_roofline the whole step against t_bound = max(F_alg/2.5e15, B_alg/8e12)
  cfg2           the same layer step at B=4, H=16, T=65536, L=16 (S=256), q/k/v ~ N(0,1)
  decode         fused decode tokens/s (256 sequences, 32 q / 8 kv heads, 512-token
                 prefill, 1024 steps; its 69.5 MB state stays in the 256 MB Infinity Cache)
  decode_hbm_streaming  the same decode kernel on 2048 sequences (0.55 GB of state, streamed
                 from HBM every step), 256 steps
  cpu_baseline   the reference CPU path (faithful port, oracle/race_cpu_port.py)
                 timed on this host on a bounded sample of the same layer
"""
import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK = 8.0e12      # B/s
BF16_PEAK = 2.5e15     # dense MFMA flop/s
FP32_PEAK = 157.3e12   # dense fp32 MFMA flop/s


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--T", type=int, default=1 << 20)
    ap.add_argument("--B", type=int, default=1)
    ap.add_argument("--H", type=int, default=4)
    ap.add_argument("--L", type=int, default=8)
    ap.add_argument("--decode-steps", type=int, default=1024)
    ap.add_argument("--decode-seqs", type=int, default=256,
                    help="sequences of the decode line (cfg4: 256; e.g. 2048 puts the carried state beyond "
                         "the 256 MB Infinity Cache)")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-cfg2", action="store_true", help="leave the cfg2 layer line out of the default run")
    ap.add_argument("--streaming-decode-seqs", type=int, default=2048,
                    help="sequences of the second decode line, whose carried state (0.55 GB at 2048) exceeds the "
                         "256 MB Infinity Cache and streams from HBM every step (0: leave it out)")
    ap.add_argument("--streaming-decode-steps", type=int, default=256)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-T", type=int, default=16384)
    ap.add_argument("--sweep", action="store_true",
                    help="cfg3 long-context sweep instead of the headline line: tokens/s for "
                         "T = 2^20 .. --sweep-max, GPU and CPU-path memory per token and the "
                         "largest T each fits")
    ap.add_argument("--sweep-max", type=int, default=1 << 24)
    ap.add_argument("--max-context", action="store_true",
                    help="measure the longest cfg3 sequence (B=1, H=4, D=64, L=8, K=4) one layer fwd+bwd "
                         "runs at on this GPU (T doubled, then bisected, until torch reports out of memory) "
                         "and, in the same run, the longest the CPU path runs within a host-memory budget")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a plain 1 GiB device copy (x3), the reference kernel for scaling "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE counters to bytes")
    ap.add_argument("--workload", default="cfg3",
                    choices=["cfg1", "cfg2", "cfg3", "cfg5", "op", "noncausal", "linear"],
                    help="cfg1: the reference's fp32 op path (soft_hash_probs + RaceCausalFn) fwd+bwd at "
                         "B=2, H=8, T=2048, D=64, L=8, K=4, scale sqrt(D) and 1.0, with the CPU path on the same "
                         "inputs; cfg2: the same layer step at B=4, H=16, T=65536, L=16 (S=256), q/k/v ~ N(0,1); "
                         "cfg5: Llama-3.2-1B-shaped hybrid LM (random init), B=8, T=8192 prefill "
                         "forward+backward, then 256-token greedy decode through the RACE state cache")
    return ap.parse_args()


# ---------------------------------------------------------------- algorithmic counts
def layer_counts(S, D, L, K, elt=2):
    """Per (token, head) of one layer fwd+bwd: flops and compulsory HBM bytes."""
    R = 1 << K
    f_scan = 14 * S * D + 9 * S
    f_hash = 6 * (2 * D * L * K + 2 * L * K * R + 4 * S)
    return f_scan + f_hash, 11 * D * elt


def kernel_bytes(name, Hq, Hkv, D, elt=2):
    """Algorithmic HBM bytes per kv-head token of one fused kernel launch."""
    G = Hq // Hkv
    row = D * elt
    return {
        "qkv_fwd_totals": 2 * row,                    # k, v
        "qkv_fwd_readout": 2 * row + 2 * G * row,     # k, v, q, out
        "qkv_bwd_totals": 2 * row + 3 * G * row,      # k, v, q, go, dq
        "qkv_bwd_main": 4 * row + 2 * G * row,        # k, v, dk, dv, q, go
    }.get(name)


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` at the default cfg3 shape, measured with rocprofv3
    FETCH_SIZE / WRITE_SIZE (calibrated on a plain copy) and recorded in
    profiles/race_layer_cfg3_T1M_hbm_traffic.md; None when not recorded."""
    path = os.path.join(ROOT, "profiles", "race_layer_cfg3_T1M_hbm_traffic.md")
    try:
        for line in open(path):
            if line.strip().startswith("traffic_bytes_per_launch"):
                return json.loads(line.split("traffic_bytes_per_launch", 1)[1]).get(kernel)
    except OSError:
        pass
    return None


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported in this build "
              "(the hot path would shard over kv heads and sequence blocks, with one exchange of block states)", file=sys.stderr)
        sys.exit(2)

    import torch

    from race_attention_amd import RaceDecodeState, build_planes_protos, race_causal_attention
    from race_attention_amd import _lib

    if args.copy_calibration:
        a = torch.empty(1 << 28, device="cuda").uniform_()
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes_per_launch": a.numel() * 4, "launches": 3}))
        return
    if args.sweep:
        print(json.dumps(bench_sweep(torch, args, build_planes_protos, race_causal_attention)))
        return
    if args.max_context:
        print(json.dumps(bench_max_context(torch, args, build_planes_protos, race_causal_attention)))
        return
    if args.workload == "cfg5":
        print(json.dumps(bench_hybrid(torch, args)))
        return
    if args.workload == "cfg1":
        print(json.dumps(bench_cfg1(torch, args)))
        return
    if args.workload == "op":  # the fp32 op path at 2^20 (token, head) pairs
        print(json.dumps(bench_cfg1(torch, args, B=1, H=4, T=1 << 18, name="op", cpu_T=1 << 13)))
        return
    if args.workload == "noncausal":
        print(json.dumps(bench_noncausal(torch, args)))
        return
    if args.workload == "linear":
        print(json.dumps(bench_linear(torch, args)))
        return
    dev = torch.device("cuda:0")
    B, H, T, L, std = args.B, args.H, args.T, args.L, 1.0 / math.sqrt(64)
    if args.workload == "cfg2":
        B, H, T, L, std = 4, 16, 65536, 16, 1.0
    lay = bench_layer(torch, args, B, H, T, L, std, build_planes_protos, race_causal_attention, _lib)

    result = {
        "metric": "RACE layer fwd+bwd tokens/sec at 1M ctx; fused-decode tokens/sec",
        "value": lay["value"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": lay["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": f"{args.workload}: one causal RACE layer fwd+bwd", **lay["config"],
                   "parallelism": "single GPU"},
        "roofline": lay["roofline"],
        "layer_roofline": lay["layer_roofline"],
        "wall_s_timed": lay["wall_s_timed"],
    }
    torch.cuda.empty_cache()
    if args.workload == "cfg3" and not args.no_cfg2:
        # cfg2 on the same clock: B=4, H=16, T=65536, L=16 (S=256, two bucket tiles), q/k/v ~ N(0,1)
        c2 = bench_layer(torch, args, 4, 16, 65536, 16, 1.0, build_planes_protos, race_causal_attention, _lib)
        result["cfg2"] = {"value": c2["value"], "unit": "tokens/s", "ms_per_step": c2["ms_per_step"],
                          "config": {"workload": "cfg2: one causal RACE layer fwd+bwd", **c2["config"]},
                          "roofline": c2["roofline"], "layer_roofline": c2["layer_roofline"]}
        torch.cuda.empty_cache()
    if not args.no_decode:
        result["decode"] = bench_decode(torch, dev, RaceDecodeState, build_planes_protos, _lib, args.decode_steps,
                                        args.decode_seqs)
        torch.cuda.empty_cache()
        if args.decode_seqs == 256 and args.streaming_decode_seqs:
            # the same kernel with a carried state larger than the 256 MB Infinity Cache, so every step
            # streams it from HBM
            result["decode_hbm_streaming"] = bench_decode(torch, dev, RaceDecodeState, build_planes_protos, _lib,
                                                          args.streaming_decode_steps, args.streaming_decode_seqs)
            torch.cuda.empty_cache()
    if not args.no_cpu:
        result["cpu_baseline"] = bench_cpu(torch, args.cpu_T, H, 64, L, 4)
    print(json.dumps(result))


def bench_layer(torch, args, B, H, T, L, std, build_planes_protos, race_causal_attention, _lib, D=64, K=4):
    """One causal RACE layer fwd+bwd on bf16 inputs resident in HBM: `args.warmup` untimed steps, then
    `args.steps` timed back to back between two HIP events on the launch stream, then the same number
    of steps with the library's per-kernel HIP events for the kernel split and the dominant kernel's
    roofline."""
    dev = torch.device("cuda:0")
    S = L << K
    planes_T, _ = build_planes_protos(D, K, L, 1, device=dev, seed=0)
    g = torch.Generator(device=dev).manual_seed(1)
    q = (torch.randn(B, H, T, D, generator=g, device=dev) * std).to(torch.bfloat16).requires_grad_(True)
    k = (torch.randn(B, H, T, D, generator=g, device=dev) * std).to(torch.bfloat16).requires_grad_(True)
    v = (torch.randn(B, H, T, D, generator=g, device=dev) * std).to(torch.bfloat16).requires_grad_(True)
    go = torch.randn(B, H, T, D, generator=g, device=dev).to(torch.bfloat16)

    def step():
        q.grad = k.grad = v.grad = None
        out = race_causal_attention(q, k, v, planes_T, L, K)
        out.backward(go)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = e0.elapsed_time(e1) / args.steps
    tokens_per_s = B * T / (ms_per_step / 1e3)

    # per-kernel launch times (HIP events recorded by the library on the launch stream)
    _lib.profile(True)
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    kern = _lib.profile_read()
    _lib.profile(False)
    dom = max(kern, key=lambda n: kern[n][0])
    dom_ms = kern[dom][0] / kern[dom][1]
    per_tok = kernel_bytes(dom, H, H, D)
    roofline = None
    if per_tok is not None:
        # the pass's compulsory bytes over its time per step: with S > 128 a pass is one launch per
        # 128-bucket tile, each re-reading the rows (cfg2: two); at S <= 128 one launch
        launches = kern[dom][1] / args.steps
        traffic_bytes = per_tok * B * H * T
        achieved = traffic_bytes / (dom_ms * launches / 1e3) / 1e9
        default_shape = (B, H, T, L) == (1, 4, 1 << 20, 8)
        roofline = {"kernel": dom, "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK / 1e9,
                    "unit": "GB/s", "frac": round(achieved / (HBM_PEAK / 1e9), 4),
                    "traffic": measured_traffic(dom) if default_shape else None,
                    "algorithmic_bytes_per_launch": round(traffic_bytes / launches),
                    "avg_launch_ms": round(dom_ms, 4), "launches_per_step": round(launches, 2)}
    f_alg, b_alg = layer_counts(S, D, L, K)
    n_tok = B * H * T
    t_bound = max(f_alg * n_tok / BF16_PEAK, b_alg * n_tok / HBM_PEAK)
    layer_roofline = {"t_bound_ms": round(t_bound * 1e3, 4), "frac": round(t_bound * 1e3 / ms_per_step, 4),
                      "bound": "hbm" if b_alg / HBM_PEAK > f_alg / BF16_PEAK else "mfma",
                      "kernels_ms_per_step": {n: round(v[0] / args.steps, 4) for n, v in kern.items()}}
    del q, k, v, go
    return {"value": round(tokens_per_s, 1), "ms_per_step": round(ms_per_step, 4),
            "config": {"B": B, "H": H, "T": T, "D": D, "L": L, "K": K, "S": S,
                       "inputs": f"bf16 q,k,v ~ N(0,{'1' if std == 1.0 else '1/sqrt(D)'}), go ~ N(0,1), seed 1; "
                                 "planes seed 0"},
            "roofline": roofline, "layer_roofline": layer_roofline, "wall_s_timed": round(wall, 3)}


def bench_sweep(torch, args, build_planes_protos, race_causal_attention):
    """cfg3 over T = 2^20 .. sweep_max (B=1, H=4, D=64, L=8, K=4): tokens/s of one layer
    fwd+bwd and peak HBM per token; the largest T that fits in this GPU's memory at that
    rate; the CPU path's (oracle/race_cpu_port.py) peak host memory per token at a small
    T and the largest T the host memory would hold."""
    import resource
    dev = torch.device("cuda:0")
    B, H, D, L, K = 1, args.H, 64, args.L, 4
    planes_T, _ = build_planes_protos(D, K, L, 1, device=dev, seed=0)
    rows = []
    T = 1 << 20
    per_tok = None
    while T <= args.sweep_max:
        torch.cuda.empty_cache()
        torch.cuda.reset_peak_memory_stats(dev)
        base = torch.cuda.memory_allocated(dev)
        g = torch.Generator(device=dev).manual_seed(1)
        std = 1.0 / math.sqrt(D)
        q, k, v = ((torch.randn(B, H, T, D, generator=g, device=dev) * std).to(torch.bfloat16).requires_grad_(True)
                   for _ in range(3))
        go = torch.randn(B, H, T, D, generator=g, device=dev).to(torch.bfloat16)

        def step():
            q.grad = k.grad = v.grad = None
            race_causal_attention(q, k, v, planes_T, L, K).backward(go)

        for _ in range(3):  # (the first T also warms the device's clocks)
            step()
        torch.cuda.synchronize()
        reps = 5
        t0 = time.perf_counter()
        for _ in range(reps):
            step()
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) / reps * 1e3
        peak = torch.cuda.max_memory_allocated(dev) - base
        per_tok = peak / (B * T)
        rows.append({"T": T, "ms_per_step": round(ms, 3), "tokens_per_s": round(B * T / (ms / 1e3), 1),
                     "peak_hbm_bytes": peak, "hbm_bytes_per_token": round(per_tok, 1)})
        print(json.dumps(rows[-1]), file=sys.stderr, flush=True)
        del q, k, v, go
        T *= 2
    total = torch.cuda.get_device_properties(dev).total_memory
    gpu_max_T = int(total // per_tok)
    # CPU path: peak resident memory of one layer fwd+bwd at a small T
    from oracle import race_cpu_port
    from oracle import race_oracle as orc
    planes_c, protos_c = orc.build_planes_protos(D, K, L, seed=0)
    Tc = args.cpu_T
    rss0 = resource.getrusage(resource.RUSAGE_SELF).ru_maxrss * 1024
    gc = torch.Generator().manual_seed(1)
    qc, kc, vc = ((torch.randn(1, H, Tc, D, generator=gc) / math.sqrt(D)).requires_grad_(True) for _ in range(3))
    race_cpu_port.race_layer_cpu(qc, kc, vc, planes_c, protos_c, L, K).backward(torch.randn(1, H, Tc, D, generator=gc))
    rss1 = resource.getrusage(resource.RUSAGE_SELF).ru_maxrss * 1024
    cpu_per_tok = max(rss1 - rss0, 1) / Tc
    host = os.sysconf("SC_PAGE_SIZE") * os.sysconf("SC_PHYS_PAGES")
    return {"workload": "cfg3 long-context sweep (one layer fwd+bwd, B=1, H=4, D=64, L=8, K=4, bf16)",
            "sweep": rows, "gpu_total_bytes": total, "gpu_max_T_estimate": gpu_max_T,
            "cpu_path": {"T": Tc, "peak_rss_growth_bytes": rss1 - rss0, "bytes_per_token": round(cpu_per_tok, 1),
                         "host_bytes": host, "cpu_max_T_estimate": int(host // cpu_per_tok)}}


def _randn_bf16(torch, shape, gen, std, dev, chunk=1 << 26):
    """bf16 tensor of N(0, std^2) values drawn in fp32 chunks (no full-size fp32 temporary)."""
    t = torch.empty(shape, dtype=torch.bfloat16, device=dev)
    flat = t.view(-1)
    for i in range(0, flat.numel(), chunk):
        n = min(chunk, flat.numel() - i)
        flat[i:i + n] = (torch.randn(n, generator=gen, device=dev) * std).to(torch.bfloat16)
    return t


def bench_max_context(torch, args, build_planes_protos, race_causal_attention):
    """Longest sequence of one cfg3 layer fwd+bwd (B=1, H=4, D=64, L=8, K=4, bf16; q, k, v, go, out,
    dq, dk, dv resident in HBM, plus the library's block state and scratch) that runs on this GPU:
    T doubles from 2^22 until torch's allocator reports out of memory (an ordinary Python
    exception: nothing is launched on memory that was not allocated), then bisects to 2^20 tokens.
    In the same run the CPU path (oracle/race_cpu_port.py, the reference's memory behaviour) runs
    doubling T while its projected peak stays within a host-memory budget (half of the host, at
    most 160 GiB), and its largest T and the host-memory limit implied by its bytes per token are
    reported beside the GPU's."""
    import resource
    dev = torch.device("cuda:0")
    B, H, D, L, K = 1, args.H, 64, args.L, 4
    planes_T, _ = build_planes_protos(D, K, L, 1, device=dev, seed=0)
    std = 1.0 / math.sqrt(D)

    def try_T(T):
        torch.cuda.empty_cache()
        torch.cuda.reset_peak_memory_stats(dev)
        box = {}
        try:
            g = torch.Generator(device=dev).manual_seed(1)
            for name, sd in (("q", std), ("k", std), ("v", std), ("go", 1.0)):
                box[name] = _randn_bf16(torch, (B, H, T, D), g, sd, dev)
            for name in ("q", "k", "v"):
                box[name].requires_grad_(True)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            box["out"] = race_causal_attention(box["q"], box["k"], box["v"], planes_T, L, K)
            box["out"].backward(box["go"])
            torch.cuda.synchronize()
            ms = (time.perf_counter() - t0) * 1e3
            ok = bool(torch.isfinite(box["q"].grad[0, 0, -1].float()).all())
            row = {"T": T, "ok": ok, "ms_fwd_bwd": round(ms, 1), "tokens_per_s": round(B * T / (ms / 1e3), 1),
                   "peak_hbm_bytes": torch.cuda.max_memory_allocated(dev)}
        except torch.cuda.OutOfMemoryError:
            row = {"T": T, "ok": False, "oom": True}
        box.clear()
        torch.cuda.empty_cache()
        print(json.dumps(row), file=sys.stderr, flush=True)
        return row

    rows = []
    T, good, bad = 1 << 22, None, None
    while T <= (1 << 30):
        r = try_T(T)
        rows.append(r)
        if r["ok"]:
            good = T
            T *= 2
        else:
            bad = T
            break
    step = 1 << 20
    while good is not None and bad is not None and bad - good > step:
        mid = (good + bad) // 2 // step * step
        if mid <= good:
            break
        r = try_T(mid)
        rows.append(r)
        if r["ok"]:
            good = mid
        else:
            bad = mid
    gpu = {"max_T_ran": good, "first_T_out_of_memory": bad,
           "gpu_total_bytes": torch.cuda.get_device_properties(dev).total_memory, "trials": rows}

    from oracle import race_cpu_port
    from oracle import race_oracle as orc
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    host = os.sysconf("SC_PAGE_SIZE") * os.sysconf("SC_PHYS_PAGES")
    budget = min(host // 2, 160 << 30)
    pl_c, pr_c = orc.build_planes_protos(D, K, L, seed=0)
    base = resource.getrusage(resource.RUSAGE_SELF).ru_maxrss * 1024
    cpu_rows, per_tok, Tc = [], None, 4096
    while per_tok is None or per_tok * Tc * 1.25 <= budget:
        gc = torch.Generator().manual_seed(1)
        qc, kc, vc = ((torch.randn(1, H, Tc, D, generator=gc) * std).requires_grad_(True) for _ in range(3))
        goc = torch.randn(1, H, Tc, D, generator=gc)
        t0 = time.perf_counter()
        race_cpu_port.race_layer_cpu(qc, kc, vc, pl_c, pr_c, L, K).backward(goc)
        sec = time.perf_counter() - t0
        peak = resource.getrusage(resource.RUSAGE_SELF).ru_maxrss * 1024 - base
        per_tok = peak / Tc
        cpu_rows.append({"T": Tc, "seconds_fwd_bwd": round(sec, 3), "tokens_per_s": round(Tc / sec, 1),
                         "peak_rss_growth_bytes": peak})
        print(json.dumps(cpu_rows[-1]), file=sys.stderr, flush=True)
        del qc, kc, vc, goc
        Tc *= 2
    cpu = {"max_T_ran": cpu_rows[-1]["T"], "bytes_per_token": round(per_tok, 1), "host_bytes": host,
           "budget_bytes": budget, "host_limit_T": int(host // per_tok), "cores": cores, "runs": cpu_rows}
    return {"workload": "cfg3 maximum context: one causal RACE layer fwd+bwd, B=1, H=4, D=64, L=8, K=4, bf16 "
                        "(GPU) / fp32 reference CPU path (host)",
            "gpu": gpu, "cpu_path": cpu,
            "gpu_over_cpu_max_T": round(good / cpu["host_limit_T"], 1) if good else None}


def bench_hybrid(torch, args, B=8, T=8192, n_new=256):
    """cfg5: HybridLM (16 layers, hidden 2048, 32/8 heads of 64, SwiGLU 8192, vocab 128256,
    RACE L=8 K=4), bf16 random-init weights, uniform synthetic token ids (seed 1).
    prefill: forward + cross-entropy backward over B x T tokens; decode: prefill the
    RACE state cache with the B x T prompt, then n_new greedy tokens, one fused decode
    kernel per layer per token: eagerly, and replaying one captured HIP graph per token step."""
    from race_attention_amd.hybrid import GraphedDecoder, HybridConfig, HybridLM
    dev = torch.device("cuda:0")
    cfg = HybridConfig()
    model = HybridLM(cfg).to(dev).init_weights(seed=0)
    g = torch.Generator(device=dev).manual_seed(1)
    idx = torch.randint(0, cfg.vocab_size, (B, T + 1), generator=g, device=dev)

    def train_step():
        model.zero_grad(set_to_none=True)
        model(idx[:, :-1], targets=idx[:, 1:]).backward()

    for _ in range(max(1, args.warmup)):
        train_step()
    torch.cuda.synchronize()
    steps = max(1, min(args.steps, 3))
    t0 = time.perf_counter()
    for _ in range(steps):
        train_step()
    torch.cuda.synchronize()
    train_s = (time.perf_counter() - t0) / steps
    model.zero_grad(set_to_none=True)
    torch.cuda.empty_cache()
    with torch.no_grad():
        cache = model.make_cache(B)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        logits = model(idx[:, :T], cache)[:, -1]
        torch.cuda.synchronize()
        prefill_s = time.perf_counter() - t0
        t0 = time.perf_counter()
        for i in range(n_new):
            nxt = logits.argmax(-1, keepdim=True)
            logits = model(nxt, cache)[:, -1]
        torch.cuda.synchronize()
        decode_s = time.perf_counter() - t0
        del cache, logits
        dec = GraphedDecoder(model, idx[:, :T])  # prefill and capture, not timed
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(n_new):
            dec.step(keep=False)
        torch.cuda.synchronize()
        graph_s = time.perf_counter() - t0
    return {"metric": "cfg5 hybrid LM tokens/sec", "workload": "cfg5", "B": B, "T": T, "params": sum(
                p.numel() for p in model.parameters()),
            "train_fwd_bwd": {"value": round(B * T / train_s, 1), "unit": "tokens/s", "seconds": round(train_s, 4)},
            "prefill_fwd": {"value": round(B * T / prefill_s, 1), "unit": "tokens/s", "seconds": round(prefill_s, 4)},
            "greedy_decode": {"value": round(B * n_new / decode_s, 1), "unit": "tokens/s", "steps": n_new,
                              "ms_per_token_step": round(decode_s / n_new * 1e3, 3)},
            "greedy_decode_graphed": {"value": round(B * n_new / graph_s, 1), "unit": "tokens/s", "steps": n_new,
                                      "ms_per_token_step": round(graph_s / n_new * 1e3, 3),
                                      "how": "one captured HIP graph per token step (GraphedDecoder)"},
            "dtype": "bf16", "data": "synthetic uniform token ids, random-init weights"}


def bench_cfg1(torch, args, B=2, H=8, T=2048, D=64, L=8, K=4, eps=1e-6, name="cfg1", cpu_T=None):
    """cfg1: fp32 q/k/v/go ~ N(0,1) drawn on the CPU (the same bits on both devices), planes seed 0.
    GPU: the reference's fp32 op path (soft_hash_probs + RaceCausalFn, forward and backward) at the
    reference's scale sqrt(D) and at 1.0; CPU: the reference CPU path (the port, whose soft-hash
    fixes sqrt(D)) on the same inputs (their first cpu_T tokens when given), all host cores,
    median of 10 after 2 warm-ups. The same function serves the `op` workload (the op path at 2^20 (token, head)
    pairs) with per-kernel times from the library's HIP events."""
    from oracle import race_cpu_port
    from oracle import race_oracle as orc
    from race_attention_amd.race_causal_cuda import RaceCausalFn
    from race_attention_amd.race_common import build_planes_protos, soft_hash_probs
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(1)
    Q, Kt, V, go = (torch.randn(B, H, T, D, generator=g) for _ in range(4))
    planes_T, protos_T = build_planes_protos(D, K, L, 1, device=dev, seed=0)
    q, k, v = (x.to(dev).requires_grad_(True) for x in (Q, Kt, V))
    gd = go.to(dev)
    S = L << K
    f_alg, _ = layer_counts(S, D, L, K, elt=4)
    n_tok = B * H * T
    t_bound = max(f_alg * n_tok / FP32_PEAK, 11 * D * 4 * n_tok / HBM_PEAK)
    gpu = {}
    for sname, scale in (("scale_sqrt_D", math.sqrt(D)), ("scale_1", 1.0)):
        def step():
            q.grad = k.grad = v.grad = None
            pK, pQ, V2, _ = soft_hash_probs(q, k, v, planes_T, protos_T, L, K, 1, True, scale=scale)
            RaceCausalFn.apply(pK, pQ, V2, eps).view(B, H, T, D).backward(gd)

        for _ in range(max(1, args.warmup)):
            step()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(args.steps):
            step()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / args.steps
        gpu[sname] = {"value": round(B * T / (ms / 1e3), 1), "unit": "tokens/s", "ms_per_step": round(ms, 4),
                     "layer_roofline": {"bound": "fp32 compute", "t_bound_ms": round(t_bound * 1e3, 4),
                                        "frac": round(t_bound * 1e3 / ms, 4)}}
    split = None
    if cpu_T is not None:  # per-kernel times at scale 1.0 (the last configuration timed)
        from race_attention_amd import _lib
        split = _kernel_split(torch, _lib, step, 3)
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    pl_c, pr_c = orc.build_planes_protos(D, K, L, seed=0)
    Tc = T if cpu_T is None else min(T, cpu_T)
    qc, kc, vc = (x[:, :, :Tc].clone().requires_grad_(True) for x in (Q, Kt, V))
    goc = go[:, :, :Tc].contiguous()

    def run_cpu():
        qc.grad = kc.grad = vc.grad = None
        race_cpu_port.race_layer_cpu(qc, kc, vc, pl_c, pr_c, L, K).backward(goc)

    sec = _cpu_median(run_cpu)
    sample = (f"the whole {name} layer fwd+bwd (scale sqrt(D)), median of 10 after 2 warm-ups" if Tc == T else
              f"the {name} layer fwd+bwd on its first {Tc} tokens (scale sqrt(D)), median of 10 after 2 warm-ups")
    r = {"metric": f"{name} fp32 layer fwd+bwd tokens/sec", "workload": name, "dtype": "f32",
         "config": {"B": B, "H": H, "T": T, "D": D, "L": L, "K": K, "S": S, "path": "soft_hash_probs + RaceCausalFn"},
         "gpu": gpu,
         "cpu_baseline": {"value": round(B * Tc / sec, 1), "unit": "tokens/s", "cores": cores, "kind": "port",
                          "sample": sample, "seconds_per_step": round(sec, 3)}}
    if split is not None:
        r["kernels_ms_per_step"] = split
    return r


def _time_steps(torch, step, warmup, steps):
    for _ in range(max(1, warmup)):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def _kernel_split(torch, _lib, step, steps):
    """Per-kernel ms per step from the library's HIP events on its launch stream."""
    _lib.profile(True)
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    kern = _lib.profile_read()
    _lib.profile(False)
    return {n: round(v[0] / steps, 4) for n, v in kern.items()}


def _cpu_median(fn, reps=10, warmup=2):
    """Median wall time of `reps` runs of fn after `warmup` untimed ones (the reference's
    bench_cpu_kernels.py:27-35 method, with the repetition counts of the CPU-baseline plan)."""
    for _ in range(warmup):
        fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return sorted(ts)[len(ts) // 2]


def bench_noncausal(torch, args, B=1, H=4, T=1 << 20, D=128, L=3, K=3, M=1, eps=1e-6):
    """Non-causal BatchedACE (scaling/benchmark_time.py:77-166) at that benchmark's defaults (B=1,
    H=4, D=128, race_L=3, race_Kbits=3, race_M=1; :357-372) and T = 2^20: fp32 inputs
    [M,B,T,H,D] ~ N(0,1), one step = forward + backward incl. d loss / d temperature.
    Per (token, head): 12 S D flops for the state contractions plus the soft-hash term of the layer
    count; 11 fp32 rows of HBM traffic (q, k, v, out, go, dq, dk, dv with q, k, v read twice).
    CPU: the reference's BatchedACE sequence (soft-hash, pK^T V, normalisation, pQ E; torch
    autograd) in fp32 on all host cores, on a T = 2^16 sample."""
    from oracle import race_oracle as orc
    from race_attention_amd import _lib
    from race_attention_amd.noncausal import BatchedACE
    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    ace = BatchedACE(D, K, L, M, device=dev, share_planes=True)
    g = torch.Generator(device=dev).manual_seed(1)
    Kh, Vh, Qh = (torch.randn(M, B, T, H, D, generator=g, device=dev).requires_grad_(True) for _ in range(3))
    go = torch.randn(M, B, T, H, D, generator=g, device=dev)

    def step():
        for x in (Kh, Vh, Qh):
            x.grad = None
        ace.logit_temp.grad = None
        ace(Kh, Vh, Qh, eps).backward(go)

    ms = _time_steps(torch, step, args.warmup, args.steps)
    split = _kernel_split(torch, _lib, step, 3)
    S = L << K
    n = M * B * H * T
    flops = (12 * S * D + 6 * (2 * D * L * K + 2 * L * K * (1 << K) + 4 * S)) * n
    nbytes = 11 * D * 4 * n
    t_bound = max(flops / FP32_PEAK, nbytes / HBM_PEAK)
    Tc = 1 << 16
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    gc = torch.Generator().manual_seed(1)
    Kc, Vc, Qc = (torch.randn(M, B, Tc, H, D, generator=gc).requires_grad_(True) for _ in range(3))
    goc = torch.randn(M, B, Tc, H, D, generator=gc)
    lt = torch.zeros((), requires_grad=True)
    pl, pr = ace.planes_T.cpu(), ace.protos_T.cpu()

    def run_cpu():
        for x in (Kc, Vc, Qc, lt):
            x.grad = None
        orc.batched_ace_nc_ref(Kc, Vc, Qc, pl, pr, L, K, True, lt, eps, dtype=torch.float32).backward(goc)

    sec = _cpu_median(run_cpu)
    return {"metric": "non-causal RACE (BatchedACE) fwd+bwd tokens/sec", "value": round(B * T / (ms / 1e3), 1),
            "unit": "tokens/s", "ms_per_step": round(ms, 4), "higher_is_better": True, "dtype": "f32",
            "data": "synthetic", "vs_baseline": None,
            "config": {"workload": "noncausal", "B": B, "H": H, "T": T, "D": D, "L": L, "K": K, "M": M, "S": S},
            "layer_roofline": {"bound": "hbm" if nbytes / HBM_PEAK >= flops / FP32_PEAK else "fp32 compute",
                               "t_bound_ms": round(t_bound * 1e3, 4), "frac": round(t_bound * 1e3 / ms, 4)},
            "kernels_ms_per_step": split,
            "cpu_baseline": {"value": round(B * Tc / sec, 1), "unit": "tokens/s", "cores": cores, "kind": "port",
                             "sample": "the reference's fp32 BatchedACE sequence fwd+bwd (torch autograd) at T = 2^16 "
                                       "(same B, H, D, L, K), median of 10 after 2 warm-ups",
                             "seconds_per_step": round(sec, 3)}}


def bench_linear(torch, args, B=1, H=4, T=1 << 20, D=64):
    """Causal linear attention (kernels/cpu/linear_pref.cpp:87-226, the comparison baseline) on the
    chunked scan kernels: Q, K, V [B,H,T,D] fp32, Q, K ~ U(0,1) (positive features), V ~ N(0,1);
    one step = forward + backward. Per (token, head): 12 D^2 flops, 11 fp32 rows of HBM traffic.
    CPU: the reference's own kernels/cpu/linear_pref.cpp (causal_dot_product + causal_dot_backward,
    compiled from its source into oracle/_ref, fp32, OpenMP over the B*H sequences) on a T = 2^17
    sample; the fp64 cumulative-sum restatement (oracle) at T = 2^12 where that build is absent."""
    from oracle import race_oracle as orc
    from race_attention_amd import _lib
    from race_attention_amd.linear_attention import causal_linear_attention
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(1)
    Q = torch.rand(B, H, T, D, generator=g, device=dev).requires_grad_(True)
    Kk = torch.rand(B, H, T, D, generator=g, device=dev).requires_grad_(True)
    V = torch.randn(B, H, T, D, generator=g, device=dev).requires_grad_(True)
    go = torch.randn(B, H, T, D, generator=g, device=dev)

    def step():
        for x in (Q, Kk, V):
            x.grad = None
        causal_linear_attention(Q, Kk, V).backward(go)

    ms = _time_steps(torch, step, args.warmup, args.steps)
    split = _kernel_split(torch, _lib, step, 3)
    n = B * H * T
    flops = 12 * D * D * n
    nbytes = 11 * D * 4 * n
    t_bound = max(flops / FP32_PEAK, nbytes / HBM_PEAK)
    from oracle import oracle_c
    ext = oracle_c.ref_linear_ext()
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    os.environ.setdefault("OMP_NUM_THREADS", str(cores))
    gc = torch.Generator().manual_seed(1)
    if ext is not None:
        Tc = 1 << 17
        Qc, Kc = torch.rand(B, H, Tc, D, generator=gc), torch.rand(B, H, Tc, D, generator=gc)
        Vc, goc = torch.randn(B, H, Tc, D, generator=gc), torch.randn(B, H, Tc, D, generator=gc)
        outc, gq, gk, gv = (torch.zeros(B, H, Tc, D) for _ in range(4))

        def run_cpu():
            outc.zero_()
            ext.causal_dot_product(Qc, Kc, Vc, outc)
            for t in (gq, gk, gv):
                t.zero_()
            ext.causal_dot_backward(Qc, Kc, Vc, goc, gq, gk, gv)

        kind, what = "reference", "the reference's compiled linear_pref.cpp fwd+bwd (fp32)"
    else:
        Tc = 1 << 12
        Qc = torch.rand(B, H, Tc, D, generator=gc, dtype=torch.float64).requires_grad_(True)
        Kc = torch.rand(B, H, Tc, D, generator=gc, dtype=torch.float64).requires_grad_(True)
        Vc = torch.randn(B, H, Tc, D, generator=gc, dtype=torch.float64).requires_grad_(True)
        goc = torch.randn(B, H, Tc, D, generator=gc, dtype=torch.float64)

        def run_cpu():
            for x in (Qc, Kc, Vc):
                x.grad = None
            orc.causal_linear_ref(Qc, Kc, Vc).backward(goc)

        kind, what = "port", "fp64 cumulative-sum restatement fwd+bwd"
    sec = _cpu_median(run_cpu)
    return {"metric": "causal linear attention fwd+bwd tokens/sec", "value": round(B * T / (ms / 1e3), 1),
            "unit": "tokens/s", "ms_per_step": round(ms, 4), "higher_is_better": True, "dtype": "f32",
            "data": "synthetic", "vs_baseline": None,
            "config": {"workload": "linear", "B": B, "H": H, "T": T, "D": D},
            "layer_roofline": {"bound": "hbm" if nbytes / HBM_PEAK >= flops / FP32_PEAK else "fp32 compute",
                               "t_bound_ms": round(t_bound * 1e3, 4), "frac": round(t_bound * 1e3 / ms, 4)},
            "kernels_ms_per_step": split,
            "cpu_baseline": {"value": round(B * Tc / sec, 1), "unit": "tokens/s", "cores": cores, "kind": kind,
                             "sample": f"{what} at T = {Tc} (same B, H, D), median of 10 after 2 warm-ups",
                             "seconds_per_step": round(sec, 4)}}


def bench_decode(torch, dev, RaceDecodeState, build_planes_protos, _lib, steps, Bs=256):
    """cfg4: `Bs` (256) sequences with a 512-token prefilled state, 32 q / 8 kv heads, D=64,
    L=8, K=4; `steps` single-token decode steps updating the fp32 state in place."""
    Hq, Hkv, D, L, K, T0 = 32, 8, 64, 8, 4, 512
    S = L << K
    planes_T, _ = build_planes_protos(D, K, L, 1, device=dev, seed=0)
    g = torch.Generator(device=dev).manual_seed(1)
    st = RaceDecodeState(Bs, Hq, Hkv, D, L, K, planes_T, device=dev)
    qp = torch.randn(Bs, Hq, T0, D, generator=g, device=dev).to(torch.bfloat16)
    kp = torch.randn(Bs, Hkv, T0, D, generator=g, device=dev).to(torch.bfloat16)
    vp = torch.randn(Bs, Hkv, T0, D, generator=g, device=dev).to(torch.bfloat16)
    st.prefill(qp, kp, vp)
    del qp, kp, vp
    qs = torch.randn(steps, Bs, Hq, D, generator=g, device=dev).to(torch.bfloat16)
    ks = torch.randn(steps, Bs, Hkv, D, generator=g, device=dev).to(torch.bfloat16)
    vs = torch.randn(steps, Bs, Hkv, D, generator=g, device=dev).to(torch.bfloat16)
    out = torch.empty(Bs, Hq, D, dtype=torch.bfloat16, device=dev)
    for i in range(4):
        st.step(qs[i], ks[i], vs[i], out)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(steps):
        st.step(qs[i], ks[i], vs[i], out)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1)
    _lib.profile(True)
    for i in range(min(steps, 64)):
        st.step(qs[i], ks[i], vs[i], out)
    torch.cuda.synchronize()
    kern = _lib.profile_read()
    _lib.profile(False)
    ev_ms = kern["decode_step"][0] / kern["decode_step"][1]
    # A step is one kernel launch, so the back-to-back step period bounds the kernel's duration from
    # above; the per-launch HIP-event bracket adds the event records around a ~25 us kernel and
    # reads longer, so it is reported beside it but not used.
    k_ms = ms / steps
    bytes_step = 2 * 4 * Bs * Hkv * S * (D + 1) + 2 * Bs * (2 * Hq + 2 * Hkv) * D
    achieved = bytes_step / (k_ms / 1e3) / 1e9
    state_bytes = 4 * Bs * Hkv * S * (D + 1)
    return {"value": round(Bs * steps / (ms / 1e3), 1), "unit": "tokens/s", "ms_per_step": round(ms / steps, 5),
            "config": {"workload": "cfg4 fused decode" if Bs == 256 else f"fused decode, cfg4 heads, {Bs} sequences",
                       "sequences": Bs, "Hq": Hq, "Hkv": Hkv, "D": D, "L": L, "K": K, "prefill": T0,
                       "steps": steps, "state_bytes": state_bytes,
                       "state_vs_256MB_infinity_cache": "fits" if state_bytes < 256e6 else "exceeds"},
            "roofline": {"kernel": "decode_step", "bound": "hbm", "achieved": round(achieved, 1),
                         "peak": HBM_PEAK / 1e9, "unit": "GB/s", "frac": round(achieved / (HBM_PEAK / 1e9), 4),
                         "algorithmic_bytes_per_launch": bytes_step, "avg_launch_ms": round(k_ms, 5),
                         "how": "step period of back-to-back launches (one kernel per step)",
                         "event_bracket_ms": round(ev_ms, 5)}}


def bench_cpu(torch, T, H, D, L, K, reps=10, warmup=2):
    """The reference CPU path (soft-hash + RaceCausalCPUFn, fp32, fp64 prefix-mean
    kernel on OpenMP threads) on the same layer shape with a bounded T: median of `reps`
    timed runs after `warmup` untimed ones."""
    from oracle import race_cpu_port
    from oracle import race_oracle as orc
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    planes_T, protos_T = orc.build_planes_protos(D, K, L, seed=0)
    g = torch.Generator().manual_seed(1)
    std = 1.0 / math.sqrt(D)
    q, k, v = ((torch.randn(1, H, T, D, generator=g) * std).requires_grad_(True) for _ in range(3))
    go = torch.randn(1, H, T, D, generator=g)

    def run():
        q.grad = k.grad = v.grad = None
        out = race_cpu_port.race_layer_cpu(q, k, v, planes_T, protos_T, L, K)
        out.backward(go)

    sec = _cpu_median(run, reps, warmup)
    return {"value": round(T / sec, 1), "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"one layer fwd+bwd, B=1 H={H} T={T} D={D} L={L} K={K} fp32, median of {reps} "
                      f"after {warmup} warm-up runs",
            "seconds_per_step": round(sec, 3)}


if __name__ == "__main__":
    main()
