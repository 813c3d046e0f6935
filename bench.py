#!/usr/bin/env python3
"""Benchmark of the MoE expert hot path on one MI355X.

Default workload (the headline decode configuration): a Qwen3-30B-A3B-shaped
MoE stack, 48 layers of H=2048, I=768, 128 Q4_0 experts, top-8 with
renormalised softmax, decode batch 1.  One step = one token through all 48
layers (x <- x + MoE_l(rms_norm(x))).  Weights are synthetic N(0, 0.02)
quantized to Q4_0 (16.3 GB resident in HBM) with fp32 N(0, 0.02) routers;
every step copies a fresh N(0, 1) token into the stack's hidden-state
buffer and runs the stack (one launch per layer).  The timed region starts
with all inputs in HBM.  Step times are also reported as the median of the
timed steps.  The same line carries one object per other configuration,
each with its own roofline and CPU baseline:
  prefill       2048 tokens through the same 48-layer stack on the grouped
                int8-MFMA path: int8 TOPS against the MFMA peak, nominal and
                at the shader clock measured under MFMA load.
  batched       64 tokens per step through one layer, steps rotating over 16
                of the stack's layers, routers skewed to Zipf(1.1).
  decode_235b   the Qwen3-235B-A22B-shaped stack (H=4096, I=1536, 94 layers,
                127.7 GB resident; built after the 30B arena is released),
                one token per step.
  batched_235b  the same stack, 32 tokens per step, routers skewed to
                Zipf(1.1).

Other workloads (--workload):
  batched      one layer per step, 64 tokens per step, router skewed so that
               expert popularity follows Zipf(1.1); steps rotate over 16
               layers (5.4 GB) so no step finds its experts in the 256 MB MALL.
  prefill      2048 tokens through the 48-layer stack on the grouped int8
               MFMA path; int8 TOPS against the MFMA peak.
  decode-235b  the Qwen3-235B-A22B-shaped stack (H=4096, I=1536, 94 layers,
               127.7 GB resident), one token per step.
  batched-235b the same stack, 32 tokens per step with Zipf(1.1) routing.
  hbm-ceiling  what one launch of plain 128-bit loads reads from HBM.
  legacy-moe   the reference's own legacy call, tg_moe_forward: 8 Q4_K experts
               of the 30B shape on caller-owned host buffers (operands copied
               in per call, as the reference's ABI hands them over).
  legacy-expert the reference engine's own MoE loop on the same buffers: one
               tg_expert_forward_mixed call per expert into a zeroed output.
  legacy-layer the reference's tg_transformer_layer on the same buffers: f32
               attention (32 heads / 4 kv heads of 128, 1024 cached positions)
               and 8 Q4_K experts, one token.
  output-head  the step after the layers: logits of the 151936 x 2048 fp32
               head (resident) and the greedy token, one call per step.
  sample       temperature / top-p sampling of the next token over 151936
               resident logits, one call per step.

Prints one JSON line: tok/s (value), expert-weight HBM GB/s, the roofline
of the dominant kernel (HIP events on its launch stream) and the CPU oracle
timed on this host on a bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import platform
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

H, I, E, K_TOP = 2048, 768, 128, 8
HBM_PEAK = 8.0e12            # MI355X HBM3E, bytes/s
EXPERT_Q4_BYTES = 3 * I * (H // 32) * 18          # 2,654,208
ROUTER_BYTES = E * H * 4                           # 1,048,576 (fp32 router of one layer)
DECODE_PATHS = {"auto": 0, "per-layer": 2, "fused": 3, "routed": 4}
GATEUP_BYTES_PER_EXPERT = 2 * I * (H // 32) * 18  # 1,769,472


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor()


def profiled_traffic(kernel):
    """HBM bytes per launch (read + write) of `kernel` as measured by the
    FETCH_SIZE / WRITE_SIZE counter runs summarised under profiles/ (line
    `traffic_bytes_per_launch <kernel> <bytes>`), or None."""
    root = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles")
    if not os.path.isdir(root):
        return None
    for name in sorted(os.listdir(root)):
        if not name.endswith(".md"):
            continue
        with open(os.path.join(root, name)) as f:
            for line in f:
                parts = line.split()
                if len(parts) == 3 and parts[0] == "traffic_bytes_per_launch" and parts[1] == kernel:
                    return int(parts[2])
    return None


def kernel_times(call, names):
    """(launches, total ms) per kernel name from the library's event timing."""
    out = {}
    for name in names:
        n = ctypes.c_int()
        ms = ctypes.c_double()
        call("tg_prof_read", name.encode(), ctypes.byref(n), ctypes.byref(ms))
        if n.value:
            out[name] = (n.value, ms.value)
    return out


def step_stats(events):
    """Median / min / max step time (ms) from HIP events recorded before each
    step and after the last one, on the stream the steps run on."""
    ms = np.array([events[i].elapsed_time(events[i + 1]) for i in range(len(events) - 1)])
    return {"median": round(float(np.median(ms)), 4), "min": round(float(ms.min()), 4),
            "max": round(float(ms.max()), 4), "n": int(ms.size)}


def host_copy_gbps(threads, nbytes=1 << 30, reps=5):
    """STREAM-style copy on this host's cores: dst[:] = src[:] over nbytes,
    split over `threads` threads (numpy releases the GIL for the copy);
    bytes read + written per second, best of `reps`."""
    from concurrent.futures import ThreadPoolExecutor
    src = np.ones(nbytes // 4, np.float32)
    dst = np.zeros_like(src)
    cuts = np.linspace(0, src.size, threads + 1).astype(np.int64)
    parts = [(int(cuts[i]), int(cuts[i + 1])) for i in range(threads)]
    best = float("inf")
    with ThreadPoolExecutor(threads) as ex:
        for _ in range(reps):
            t0 = time.perf_counter()
            list(ex.map(lambda ab: np.copyto(dst[ab[0]:ab[1]], src[ab[0]:ab[1]]), parts))
            best = min(best, time.perf_counter() - t0)
    return 2 * nbytes / best / 1e9


def cpu_roofline(value_gbps, cores):
    """The CPU baseline's expert-byte rate against this host's copy rate."""
    copy_n = host_copy_gbps(cores)
    copy_1 = host_copy_gbps(1)
    return {"expert_gbps": round(value_gbps, 2), "host_copy_gbps": round(copy_n, 1),
            "host_copy_gbps_1thread": round(copy_1, 1), "frac": round(value_gbps / copy_n, 4),
            "note": "STREAM-style copy (read + write bytes) on the same cores"}


# ----------------------------------------------------------------- CPU legs

def cpu_baseline_stack(arena, seed, n_layers_total, seconds, gpu_check, shape=(H, I, E, K_TOP), n_sample=4):
    """The C oracle on this host: one token at a time through a sample of
    layers read back from the arena; extrapolated to the full stack."""
    from oracle import oracle as O
    H, I, E, K_TOP = shape
    n_s = min(n_sample, n_layers_total)
    layers = [arena.read_layer(l) for l in range(n_s)]
    routers = [O.synth_normal(seed, O.stream_id(l, 0, 3), 0.02, E * H).reshape(E, H) for l in range(n_s)]
    x_ref, x_gpu = gpu_check
    got, _ = O.moe_stack(layers, routers, H, I, E, K_TOP, x_ref)
    parity = "bit-exact" if np.array_equal(got.view(np.uint32), x_gpu.view(np.uint32)) else "MISMATCH"
    cores = O.cpu_count()
    res = {}
    for threads in (1, cores):
        O.set_threads(threads)
        tok = 0
        t0 = time.perf_counter()
        while True:
            x = O.synth_normal(seed + 7, O.stream_id(0, tok, 4), 1.0, H)
            O.moe_stack(layers, routers, H, I, E, K_TOP, x)
            tok += 1
            dt = time.perf_counter() - t0
            if dt >= seconds / 2 and tok >= 2:
                break
        per_layer = dt / (tok * n_s)
        res[threads] = (1.0 / (per_layer * n_layers_total), tok, dt)
    O.set_threads(cores)
    v1, tok1, dt1 = res[1]
    vn, tokn, dtn = res[cores]
    EBt = 3 * I * (H // 32) * 18
    return {
        "value": round(vn, 3), "unit": "tok/s", "cores": cores, "kind": "port",
        "roofline": cpu_roofline(vn * n_layers_total * K_TOP * EBt / 1e9, cores),
        "sample": (f"C oracle, {tokn} tokens x {n_s} of {n_layers_total} layers "
                   f"({dtn:.1f} s, {cores} OpenMP threads), per-layer time extrapolated to "
                   f"{n_layers_total} layers"),
        "single_thread": {"value": round(v1, 3), "unit": "tok/s", "cores": 1,
                          "sample": f"{tok1} tokens x {n_s} layers ({dt1:.1f} s)"},
        "cpu_model": cpu_model(),
        "sample_parity_vs_gpu": parity,
    }


def cpu_baseline_layer(layer_bytes, router, X, seconds, gpu_check, shape=(H, I, E, K_TOP)):
    """The C oracle on this host over the batched workload: steps of T tokens
    through one layer, as many as fit in the time budget."""
    from oracle import oracle as O
    H, I, E, K_TOP = shape
    x0, out_gpu = gpu_check
    ref, _, _, _ = O.moe_layer(layer_bytes, router, H, I, E, K_TOP, x0)
    parity = "bit-exact" if np.array_equal(ref.view(np.uint32), out_gpu.view(np.uint32)) else "MISMATCH"
    cores = O.cpu_count()
    res = {}
    for threads in (1, cores):
        O.set_threads(threads)
        steps, tok = 0, 0
        t0 = time.perf_counter()
        while True:
            xs = X[steps % len(X)]
            O.moe_layer(layer_bytes, router, H, I, E, K_TOP, xs)
            steps += 1
            tok += xs.shape[0]
            dt = time.perf_counter() - t0
            if dt >= seconds / 2 and steps >= 1:
                break
        res[threads] = (tok / dt, steps, dt)
    O.set_threads(cores)
    vn, sn, dn = res[cores]
    v1, s1, d1 = res[1]
    T = X[0].shape[0]
    return {
        "value": round(vn, 2), "unit": "tok/s", "cores": cores, "kind": "port",
        "sample": f"C oracle, {sn} steps of {T} tokens through one layer ({dn:.1f} s, {cores} OpenMP threads)",
        "single_thread": {"value": round(v1, 2), "unit": "tok/s", "cores": 1,
                          "sample": f"{s1} steps of {T} tokens ({d1:.1f} s)"},
        "cpu_model": cpu_model(),
        "sample_parity_vs_gpu": parity,
    }


# ----------------------------------------------------------------- workloads

def run_decode_stack(args, torch, call):
    from tinygiant_amd.arena import HBMExpertArena
    from tinygiant_amd.moe import MoEBlock
    from tinygiant_amd.synth import stream_id

    L, K, W = args.layers, args.steps or 256, 16 if args.warmup is None else args.warmup
    log(f"arena: {L} layers x {E} experts ({L * E * EXPERT_Q4_BYTES / 1e9:.2f} GB Q4_0)")
    arena = HBMExpertArena(L, E, H, I, K_TOP)
    for l in range(L):
        arena.synth_layer(l, args.seed)
    arena.set_decode_path(DECODE_PATHS[args.path])
    stream = torch.cuda.current_stream().cuda_stream
    X = torch.empty((W + K, H), dtype=torch.float32, device="cuda")
    call("tg_synth_normal_dev", args.seed, stream_id(0, 0, 4), 1.0, X.numel(), X.data_ptr(), stream)
    X0 = X.clone()
    xt = torch.empty((1, H), dtype=torch.float32, device="cuda")  # the token's hidden state
    torch.cuda.synchronize()
    blk = MoEBlock(arena)

    # every step copies its token into the same buffer (with graphs on, the
    # stack call replays the one HIP graph captured in the warmup)
    log(f"warmup {W} tokens")
    for i in range(W):
        xt.copy_(X[i:i + 1])
        blk.step(xt)
    torch.cuda.synchronize()
    log(f"timing {K} tokens x {L} layers")
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(K + 1)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(W, W + K):
        evs[i - W].record()
        xt.copy_(X[i:i + 1])
        blk.step(xt)
    evs[K].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    arena.status()
    steps_ms = step_stats(evs)
    ms_step = wall * 1e3 / K
    tok_s = K / wall
    bytes_per_tok = L * K_TOP * EXPERT_Q4_BYTES
    gbps = tok_s * bytes_per_tok / 1e9

    # roofline of the dominant kernel: HIP events around each launch on its stream
    log("kernel timing pass")
    X.copy_(X0)
    torch.cuda.synchronize()
    call("tg_prof_enable", 1)
    for i in range(W, W + K):
        xt.copy_(X[i:i + 1])
        blk.step(xt)
    torch.cuda.synchronize()
    call("tg_prof_enable", 0)
    arena.status()
    kern = kernel_times(call, ("dec_part", "layer", "route", "experts", "gateup", "down"))
    kern_us = {k: round(v[1] / max(v[0], 1) * 1e3, 3) for k, v in kern.items()}
    router_bytes = None
    if "layer" in kern:
        # one launch = routing, gate/up and down of one layer: the expert
        # weights (the roofline's bytes) and the next layer's router columns
        # (reported apart)
        n_x, ms_x = kern["layer"]
        avg = ms_x / max(n_x, 1) * 1e-3
        roof_kernel, roof_bytes, router_bytes = "k_layer_dec", K_TOP * EXPERT_Q4_BYTES, ROUTER_BYTES
        path = "routed"
    elif "experts" in kern:
        # one launch = gate/up and down of the token's k experts in one layer
        n_x, ms_x = kern["experts"]
        avg = ms_x / max(n_x, 1) * 1e-3
        roof_kernel, roof_bytes = "k_experts", K_TOP * EXPERT_Q4_BYTES
        path = "fused"
    else:
        path = "per-layer"
        n_gu, ms_gu = kern["gateup"]
        avg = ms_gu / max(n_gu, 1) * 1e-3
        roof_kernel, roof_bytes = "k_gateup", K_TOP * GATEUP_BYTES_PER_EXPERT
    achieved = roof_bytes / avg

    cpu = None
    if not args.no_cpu:
        log("cpu baseline (oracle)")
        from oracle import oracle as O  # the checker, timed as the CPU baseline
        n_s = min(4, L)
        xt = O.synth_normal(args.seed + 99, O.stream_id(0, 1, 4), 1.0, H).reshape(1, H)
        xg = torch.from_numpy(xt).cuda()
        MoEBlock(arena).step(xg, 0, n_s)
        torch.cuda.synchronize()
        cpu = cpu_baseline_stack(arena, args.seed, L, args.cpu_seconds, (xt, xg.cpu().numpy()))

    prefill = None
    if not args.no_prefill:
        log("prefill leg: 2048 tokens through the same stack")
        prefill = prefill_leg(args, torch, call, arena, L, K=20, W=2)
        clk = measure_clock(call)
        prefill["clock"] = clk
        prefill["roofline"]["peak_at_measured_clock"] = clk["int8_peak_tops"]
        prefill["roofline"]["frac_at_measured_clock"] = round(prefill["roofline"]["achieved"] / clk["int8_peak_tops"], 4)
        prefill["mfma_frac_at_measured_clock"] = round(prefill["value"] / clk["int8_peak_tops"], 4)

    batched = None
    if not args.no_batched and L >= 16:
        log("batched leg: 64 tokens per step over 16 of the stack's layers, Zipf(1.1) routers")
        batched = batched_leg(args, torch, call, arena, 16, K=256, W=16)
    arena.close()

    d235 = b235 = None
    if not args.no_235b:
        log("235B legs: the 30B arena closed, the 94-layer 235B-shaped arena filled")
        a5 = synth_235b_arena(args, L5)
        d235 = leg_235b(args, torch, call, a5, 1, K=64, W=8)
        b235 = leg_235b(args, torch, call, a5, 32, K=16, W=2)
        a5.close()

    roofline = {"bound": "hbm", "kernel": roof_kernel, "bytes_per_launch": roof_bytes,
                "achieved": round(achieved / 1e9, 1), "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK, 4), "traffic": profiled_traffic(roof_kernel)}
    if router_bytes:
        roofline.update({"router_bytes_per_launch": router_bytes,
                         "frac_with_router": round((roof_bytes + router_bytes) / avg / HBM_PEAK, 4)})

    out = {
        "metric": "MoE-layer decode tok/s (48-layer Q4_0 stack, batch 1)",
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_0 x q8_0 (int8 dot, fp32 accumulate)",
        "data": "synthetic (N(0,0.02) Q4_0 experts and fp32 routers, N(0,1) tokens)",
        "config": {"workload": "qwen3-30b-a3b-moe-stack-decode", "layers": L, "hidden": H,
                   "experts": E, "moe_intermediate": I, "top_k": K_TOP, "batch": 1, "tokens": K},
        "hbm_gbps_expert_weights": round(gbps, 1),
        "hbm_frac_expert_weights": round(gbps * 1e9 / HBM_PEAK, 4),
        "event_ms_per_step": round(evs[0].elapsed_time(evs[K]) / K, 4),
        "step_ms": steps_ms,
        "kernel_avg_us": kern_us,
        "decode_path": path,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "prefill": prefill,
        "batched": batched,
        "decode_235b": d235,
        "batched_235b": b235,
    }
    return out


ZIPF_TARGET = 1.1
ZIPF_BETA0 = 0.54 / 0.905  # bias scale (per unit of logit noise) that gave ~1.1 at the 30B shape


def calibrate_zipf(build, measure, beta=ZIPF_BETA0, iters=4, tol=0.02):
    """Scales the per-expert router bias until the fitted rank-frequency
    exponent of the routing is within tol of 1.1: build(beta) loads the
    routers, measure() routes sample tokens and fits the exponent.  The
    exponent grows about in proportion to the bias, so each step multiplies
    beta by 1.1 / fit.  Returns (beta, fit) of the routers left loaded."""
    fit = float("nan")
    for it in range(iters):
        build(beta)
        fit = measure()
        log(f"zipf calibration {it}: bias scale {beta:.4f} -> fitted exponent {fit:.3f}")
        if abs(fit - ZIPF_TARGET) <= tol or it == iters - 1:
            break
        beta *= ZIPF_TARGET / fit
    return beta, fit


def batched_leg(args, torch, call, arena, LR=16, K=256, W=16, T=64):
    """Config 3 on the first LR layers of a 30B-shaped arena: T tokens per
    step through one layer, steps rotating over the LR layers (LR * 340 MB,
    more than the 256 MB MALL), the router of each layer skewed so that
    expert popularity follows Zipf(1.1): a per-expert bias along a direction
    u that every token shares (tokens N(0, 1) + c u), scaled until the fitted
    exponent of the routing is 1.1.  Returns the batched object of the bench
    line."""
    from tinygiant_amd.moe import MoEBlock
    from tinygiant_amd.synth import fit_zipf_exponent, stream_id, zipf_router_bias

    H_, E_ = arena.embed_dim, arena.n_experts
    rng = np.random.default_rng(args.seed)
    u = rng.standard_normal(H_)
    u /= np.linalg.norm(u)
    c = 0.5 * np.sqrt(H_)                       # token component along u
    rms = np.sqrt(1.0 + c * c / H_)
    noise_std = 0.02 * np.sqrt(H_) / rms         # std of the unskewed logits
    routers = []

    def build(beta):
        r2 = np.random.default_rng(args.seed + 17)
        bias = zipf_router_bias(E_, beta * noise_std)
        routers.clear()
        for l in range(LR):
            Wr = (r2.standard_normal((E_, H_)) * 0.02).astype(np.float32)
            Wr += (bias[:, None] * (rms / c) * u[None, :]).astype(np.float32)
            arena.load_router(l, Wr)
            routers.append(Wr)

    arena.set_batch_path(arena.BATCH_GROUPED)
    stream = torch.cuda.current_stream().cuda_stream
    # at least one input per layer: the calibration routes one step through every layer
    X = torch.empty((max(W + K, LR), T, H_), dtype=torch.float32, device="cuda")
    call("tg_synth_normal_dev", args.seed, stream_id(0, 0, 4), 1.0, X.numel(), X.data_ptr(), stream)
    X += torch.from_numpy((c * u).astype(np.float32)).cuda()
    torch.cuda.synchronize()
    blk = MoEBlock(arena)

    def measure():
        idx = [blk.forward(i % LR, X[i], return_routing=True)[1].cpu().numpy() for i in range(LR)]
        return fit_zipf_exponent(np.concatenate(idx), E_)

    beta, _ = calibrate_zipf(build, measure)

    log(f"batched: warmup {W} steps")
    for i in range(W):
        blk.forward(i % LR, X[i])
    torch.cuda.synchronize()
    log(f"batched: timing {K} steps of {T} tokens over {LR} layers")
    t0 = time.perf_counter()
    for i in range(W, W + K):
        blk.forward(i % LR, X[i])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = wall * 1e3 / K
    tok_s = T * K / wall

    # routing of every timed step (untimed): unique experts and the skew
    uniq, all_idx = [], []
    for i in range(W, W + K):
        _, idx, _ = blk.forward(i % LR, X[i], return_routing=True)
        ih = idx.cpu().numpy()
        uniq.append(len(np.unique(ih)))
        all_idx.append(ih)
    n_uniq = float(np.mean(uniq))
    zipf_s = fit_zipf_exponent(np.concatenate(all_idx), E_)
    bytes_step = n_uniq * EXPERT_Q4_BYTES
    gbps = bytes_step / (ms_step * 1e-3) / 1e9

    log("batched: kernel timing pass")
    call("tg_prof_enable", 1)
    for i in range(W, W + K):
        blk.forward(i % LR, X[i])
    torch.cuda.synchronize()
    call("tg_prof_enable", 0)
    names = ("route", "route_q8", "place", "group", "gateup_mfma", "down_mfma", "gu_down_mfma", "gateup_grouped",
             "down_grouped", "combine")
    kern = kernel_times(call, names)
    kern_us = {k: round(v[1] / max(v[0], 1) * 1e3, 3) for k, v in kern.items()}
    if "gu_down_mfma" in kern:  # gate/up and down of the one-tile items in one launch
        gu_name, gu_kernel, part = "gu_down_mfma", "k_mfma_small_gd", "gate/up + down"
        roof_bytes = n_uniq * EXPERT_Q4_BYTES
    else:
        gu_name = "gateup_mfma" if "gateup_mfma" in kern else "gateup_grouped"
        # one M-tile per expert (k_mfma_small) while T*top_k/E averages <= 16 entries
        gu_kernel = (("k_mfma_small" if T * K_TOP <= 16 * E else "k_mfma_grouped") if gu_name == "gateup_mfma"
                     else "k_gateup_grouped")
        part, roof_bytes = "gate/up", n_uniq * GATEUP_BYTES_PER_EXPERT
    n_gu, ms_gu = kern[gu_name]
    achieved = roof_bytes / (ms_gu / n_gu * 1e-3)

    cpu = None
    if not args.no_cpu:
        log("batched: cpu baseline (oracle)")
        l0 = W % LR
        lb = arena.read_layer(l0)
        Xh = [X[W + j].cpu().numpy() for j in range(0, K, LR)][:4]
        out = blk.forward(l0, X[W])
        cpu = cpu_baseline_layer(lb, routers[l0], Xh, args.cpu_seconds, (X[W].cpu().numpy(), out.cpu().numpy()))
    arena.set_batch_path(arena.BATCH_AUTO)
    del X
    return {
        "metric": "MoE-layer batched decode tok/s (64 tokens/step, Zipf(1.1) routing)",
        "value": round(tok_s, 1), "unit": "tok/s", "steps": K, "warmup": W, "ms_per_step": round(ms_step, 4),
        "dtype": "q4_0 x q8_0 (int8 MFMA, fp32 accumulate)",
        "data": "synthetic (N(0,0.02) Q4_0 experts, Zipf-skewed fp32 routers, N(0,1) tokens + shared direction)",
        "config": {"workload": "qwen3-30b-a3b-moe-layer-batched-decode", "hidden": H_, "experts": E_,
                   "moe_intermediate": arena.inter_dim, "top_k": K_TOP, "tokens_per_step": T, "layers_rotated": LR,
                   "zipf_target": ZIPF_TARGET, "zipf_fit": round(zipf_s, 3), "zipf_bias_scale": round(beta, 4),
                   "unique_experts_per_step": round(n_uniq, 2)},
        "hbm_gbps_expert_weights": round(gbps, 1),
        "hbm_frac_expert_weights": round(gbps * 1e9 / HBM_PEAK, 4),
        "kernel_avg_us": kern_us,
        "roofline": {"bound": "hbm", "kernel": f"{gu_kernel} ({part})",
                     "bytes_per_launch": round(roof_bytes),
                     "achieved": round(achieved / 1e9, 1), "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK, 4),
                     "traffic": profiled_traffic(gu_kernel + ("/gate_up" if part == "gate/up" else ""))},
        "cpu_baseline": cpu,
    }


def run_batched(args, torch, call):
    """Config 3 alone: a 16-layer 30B-shaped arena, 64 tokens per step."""
    from tinygiant_amd.arena import HBMExpertArena

    LR = 16
    log(f"arena: {LR} layers x {E} experts ({LR * E * EXPERT_Q4_BYTES / 1e9:.2f} GB Q4_0)")
    arena = HBMExpertArena(LR, E, H, I, K_TOP)
    for l in range(LR):
        arena.synth_layer(l, args.seed)
    b = batched_leg(args, torch, call, arena, LR, K=args.steps or 256, W=16 if args.warmup is None else args.warmup)
    arena.close()
    return headline(b)


def headline(leg):
    """A leg's object as a bench line of its own."""
    out = {"metric": leg.pop("metric"), "value": leg.pop("value"), "unit": leg.pop("unit"), "n_gpus": 1,
           "steps": leg.pop("steps"), "warmup": leg.pop("warmup"), "ms_per_step": leg.pop("ms_per_step"),
           "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": leg.pop("dtype"),
           "data": leg.pop("data"), "config": leg.pop("config")}
    out.update(leg)
    return out


# Qwen3-235B-A22B MoE shape (config 5)
H5, I5, E5, K5, L5 = 4096, 1536, 128, 8, 94
EXPERT5_BYTES = 3 * I5 * (H5 // 32) * 18          # 10,616,832
GATEUP5_BYTES = 2 * I5 * (H5 // 32) * 18          # 7,077,888
ROUTER5_BYTES = E5 * H5 * 4                        # 2,097,152


def skewed_stack_routers(arena, blk, x0, u, c, beta, seed, torch):
    """Routers of a stack whose expert popularity follows a power law at
    every depth: a per-expert component along the direction u that tokens
    share.  Layer l's component is scaled by rms(x_l) / (u . x_l) measured on
    the hidden states that reach it (x0 pushed through the layers before
    it), so the logit bias stays the same although the residual stream
    grows.  beta: the bias per unit of logit noise."""
    from tinygiant_amd.synth import zipf_router_bias
    Hs, Es = arena.embed_dim, arena.n_experts
    rms0 = np.sqrt(1.0 + c * c / Hs)
    noise_std = 0.02 * np.sqrt(Hs) / rms0
    bias = zipf_router_bias(Es, beta * noise_std)
    ut = torch.from_numpy(u.astype(np.float32)).cuda()
    rng = np.random.default_rng(seed + 29)
    x = x0.clone()
    routers = []
    for l in range(arena.n_layers):
        rms_l = float(torch.sqrt((x * x).mean(dim=1)).mean())
        proj_l = float((x @ ut).mean())
        Wr = (rng.standard_normal((Es, Hs)) * 0.02).astype(np.float32)
        Wr += (bias[:, None] * (rms_l / proj_l) * u[None, :]).astype(np.float32)
        arena.load_router(l, Wr)
        routers.append(Wr)
        x += blk.forward(l, x)
    torch.cuda.synchronize()
    return routers


def synth_235b_arena(args, L):
    from tinygiant_amd.arena import HBMExpertArena
    log(f"arena: {L} layers x {E5} experts ({L * E5 * EXPERT5_BYTES / 1e9:.1f} GB Q4_0)")
    t0 = time.perf_counter()
    arena = HBMExpertArena(L, E5, H5, I5, K5)
    for l in range(L):
        arena.synth_layer(l, args.seed)
    arena.status()
    log(f"arena filled in {time.perf_counter() - t0:.1f} s")
    return arena


def leg_235b(args, torch, call, arena, T, K, W):
    """Config 5 on a 235B-shaped arena (H=4096, I=1536, 128 experts, top-8;
    94 layers, 127.7 GB of Q4_0 resident in HBM); one step = T tokens
    through every layer.  T = 1: the synthetic N(0, 0.02) routers, one-token
    decode path.  T = 32: routers skewed to a fitted Zipf exponent of 1.1,
    grouped path.  Returns the leg's object of the bench line."""
    from tinygiant_amd.moe import MoEBlock
    from tinygiant_amd.synth import fit_zipf_exponent, stream_id

    L = arena.n_layers
    rng = np.random.default_rng(args.seed)
    stream = torch.cuda.current_stream().cuda_stream
    X = torch.empty((max(W + K, 3), T, H5), dtype=torch.float32, device="cuda")  # the calibration routes X[1], X[2]
    call("tg_synth_normal_dev", args.seed, stream_id(0, 0, 4), 1.0, X.numel(), X.data_ptr(), stream)
    blk = MoEBlock(arena)
    routers, beta = None, None
    if T > 1:
        u = rng.standard_normal(H5)
        u /= np.linalg.norm(u)
        c = 0.5 * np.sqrt(H5)
        X += torch.from_numpy((c * u).astype(np.float32)).cuda()
        holder = []

        def build(b):
            holder[:] = [skewed_stack_routers(arena, blk, X[0], u, c, b, args.seed, torch)]

        def measure():
            idx = []
            for i in (1, 2):
                x = X[i].clone()
                for l in range(L):
                    out, ix, _ = blk.forward(l, x, return_routing=True)
                    idx.append(ix.cpu().numpy())
                    x += out
            return fit_zipf_exponent(np.concatenate(idx), E5)

        log("235B batched: router calibration through the stack")
        beta, _ = calibrate_zipf(build, measure)
        routers = holder[0]
    X0 = X.clone()
    torch.cuda.synchronize()

    log(f"235B: warmup {W} steps")
    for i in range(W):
        blk.step(X[i])
    torch.cuda.synchronize()
    log(f"235B: timing {K} steps of {T} token(s) x {L} layers")
    t0 = time.perf_counter()
    for i in range(W, W + K):
        blk.step(X[i])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    arena.status()
    ms_step = wall * 1e3 / K
    tok_s = T * K / wall

    # distinct experts per layer-step and the skew (untimed, layer by layer)
    n_uniq, zipf_s = float(K5), None
    if T > 1:
        uniq, all_idx = [], []
        for i in range(W, min(W + K, W + 4)):
            x = X0[i].clone()
            for l in range(L):
                out, idx, _ = blk.forward(l, x, return_routing=True)
                ih = idx.cpu().numpy()
                uniq.append(len(np.unique(ih)))
                all_idx.append(ih)
                x += out
        n_uniq = float(np.mean(uniq))
        zipf_s = fit_zipf_exponent(np.concatenate(all_idx), E5)
    bytes_step = L * n_uniq * EXPERT5_BYTES
    gbps = bytes_step / (ms_step * 1e-3) / 1e9

    log("235B: kernel timing pass")
    X.copy_(X0)
    torch.cuda.synchronize()
    call("tg_prof_enable", 1)
    for i in range(W, W + min(K, 8)):
        blk.step(X[i])
    torch.cuda.synchronize()
    call("tg_prof_enable", 0)
    names = ("dec_part", "layer", "route", "experts", "gateup", "down", "route_q8", "group", "gateup_mfma", "down_mfma",
             "gu_down_mfma", "combine")
    kern = kernel_times(call, names)
    kern_us = {k: round(v[1] / max(v[0], 1) * 1e3, 3) for k, v in kern.items()}
    router_bytes = None
    if "layer" in kern:  # expert bytes only; the next layer's router columns it also reads are reported apart
        rk, rb, roof, router_bytes = "layer", K5 * EXPERT5_BYTES, "k_layer_dec", ROUTER5_BYTES
    elif "experts" in kern:
        rk, rb = "experts", K5 * EXPERT5_BYTES
        roof = "k_experts"
    elif "gateup" in kern:
        rk, rb = "gateup", K5 * GATEUP5_BYTES
        roof = "k_gateup"
    elif "gu_down_mfma" in kern:  # gate/up and down of the one-tile items in one launch
        rk, rb, roof = "gu_down_mfma", round(n_uniq * EXPERT5_BYTES), "k_mfma_small_gd"
    else:
        rk, rb = "gateup_mfma", round(n_uniq * GATEUP5_BYTES)
        # one M-tile per expert (k_mfma_small) while T*top_k/E averages <= 16 entries
        roof = "k_mfma_small/gate_up" if T * K5 <= 16 * E5 else "k_mfma_grouped/gate_up"
    n_r, ms_r = kern[rk]
    avg_s = ms_r / n_r * 1e-3
    achieved = rb / avg_s
    roofline = {"bound": "hbm", "kernel": roof, "bytes_per_launch": rb, "achieved": round(achieved / 1e9, 1),
                "peak": HBM_PEAK / 1e9, "unit": "GB/s", "frac": round(achieved / HBM_PEAK, 4),
                "traffic": profiled_traffic(roof + "@235b")}  # this shape's own counter run
    if router_bytes:
        roofline.update({"router_bytes_per_launch": router_bytes,
                         "frac_with_router": round((rb + router_bytes) / avg_s / HBM_PEAK, 4)})

    cpu = None
    if not args.no_cpu:
        log("235B: cpu baseline (oracle)")
        if T == 1:
            xt = X0[W, :1].cpu().numpy()
            xg = X0[W, :1].clone()
            blk.step(xg, 0, 2)
            torch.cuda.synchronize()
            cpu = cpu_baseline_stack(arena, args.seed, L, args.cpu_seconds, (xt, xg.cpu().numpy()),
                                     (H5, I5, E5, K5), 2)
        else:
            lb = arena.read_layer(0)
            out = blk.forward(0, X0[W])
            cpu = cpu_baseline_layer(lb, routers[0], [X0[W].cpu().numpy()], args.cpu_seconds,
                                     (X0[W].cpu().numpy(), out.cpu().numpy()), (H5, I5, E5, K5))
            cpu["sample"] += f"; the stack rate is this over {L} layers"
            cpu["value"] = round(cpu["value"] / L, 3)
            cpu["single_thread"]["value"] = round(cpu["single_thread"]["value"] / L, 3)

    cfg = {"workload": f"qwen3-235b-a22b-moe-stack-{'decode' if T == 1 else 'batched-decode'}", "layers": L,
           "hidden": H5, "experts": E5, "moe_intermediate": I5, "top_k": K5, "tokens_per_step": T}
    if zipf_s is not None:
        cfg.update({"zipf_target": ZIPF_TARGET, "zipf_fit": round(zipf_s, 3), "zipf_bias_scale": round(beta, 4),
                    "unique_experts_per_layer_step": round(n_uniq, 2)})
    del X, X0
    return {
        "metric": f"MoE stack decode tok/s (94-layer 235B-shaped Q4_0 stack, {T} token(s)/step)",
        "value": round(tok_s, 2), "unit": "tok/s", "steps": K, "warmup": W, "ms_per_step": round(ms_step, 4),
        "dtype": "q4_0 x q8_0 (int8 dot / int8 MFMA, fp32 accumulate)",
        "data": "synthetic (N(0,0.02) Q4_0 experts, fp32 routers" + (", Zipf-skewed" if T > 1 else "") +
                ", N(0,1) tokens)",
        "config": cfg,
        "hbm_gbps_expert_weights": round(gbps, 1),
        "hbm_frac_expert_weights": round(gbps * 1e9 / HBM_PEAK, 4),
        "kernel_avg_us": kern_us,
        "roofline": roofline,
        "cpu_baseline": cpu,
    }


def run_235b(args, torch, call, T):
    """Config 5 alone, at batch T."""
    L = args.layers if args.layers != 48 else L5
    arena = synth_235b_arena(args, L)
    K = args.steps or (64 if T == 1 else 16)
    W = (8 if T == 1 else 2) if args.warmup is None else args.warmup
    leg = leg_235b(args, torch, call, arena, T, K, W)
    arena.close()
    return headline(leg)


MFMA_INT8_PEAK = 5.0e15  # MI355X dense int8 MFMA, ops/s (256 CUs x 8192 ops/clk x 2.4 GHz)
MFMA_INT8_OPS_PER_CLK_CU = 8192


def measure_clock(call):
    """The shader clock while every CU runs int8 MFMA chains (the library's
    clock probe: shader-cycle and 100 MHz real-time counters of each block),
    and the int8 MFMA peak at that clock beside the nominal 2.4 GHz one."""
    import torch
    md, mn, mx = ctypes.c_double(), ctypes.c_double(), ctypes.c_double()
    call("tg_clock_mfma_mhz", 20000, ctypes.byref(md), ctypes.byref(mn), ctypes.byref(mx))  # warm
    call("tg_clock_mfma_mhz", 200000, ctypes.byref(md), ctypes.byref(mn), ctypes.byref(mx))
    n_cu = torch.cuda.get_device_properties(0).multi_processor_count
    peak = n_cu * MFMA_INT8_OPS_PER_CLK_CU * md.value * 1e6
    return {"mhz_median": round(md.value, 1), "mhz_min": round(mn.value, 1), "mhz_max": round(mx.value, 1),
            "cus": n_cu, "int8_peak_tops": round(peak / 1e12, 1),
            "nominal": {"mhz": 2400.0, "int8_peak_tops": MFMA_INT8_PEAK / 1e12},
            "method": "s_memtime / s_memrealtime around 200k rounds of four v_mfma_i32_16x16x32_i8 chains per wave, "
                      "4 blocks of 256 threads per CU, median over blocks; HBM peak is not clock-scaled"}


def prefill_leg(args, torch, call, arena, L, K=20, W=2):
    """Config 4 on an arena that holds L synthetic 30B layers: 2048 tokens
    through the stack on the grouped int8-MFMA path (routing uniform-ish from
    the N(0, 0.02) routers).  Returns the prefill object of the bench line:
    int8 TOPS (median step), the MFMA fraction, the roofline of the gate/up
    MFMA kernel and the CPU oracle on a one-layer sample."""
    from tinygiant_amd.moe import MoEBlock
    from tinygiant_amd.synth import stream_id

    T = 2048
    ops_layer = 2 * T * K_TOP * 3 * H * I  # 154,618,822,656
    arena.set_batch_path(arena.BATCH_GROUPED)
    stream = torch.cuda.current_stream().cuda_stream
    X = torch.empty((W + K, T, H), dtype=torch.float32, device="cuda")
    call("tg_synth_normal_dev", args.seed, stream_id(0, 1, 4), 1.0, X.numel(), X.data_ptr(), stream)
    xb = torch.empty((T, H), dtype=torch.float32, device="cuda")  # the batch's hidden states
    torch.cuda.synchronize()
    blk = MoEBlock(arena)
    log(f"warmup {W} prefills")
    for i in range(W):
        xb.copy_(X[i])
        blk.step(xb)
    torch.cuda.synchronize()
    log(f"timing {K} prefills of {T} tokens x {L} layers")
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(K + 1)]
    t0 = time.perf_counter()
    for i in range(W, W + K):
        evs[i - W].record()
        xb.copy_(X[i])
        blk.step(xb)
    evs[K].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    steps_ms = step_stats(evs)
    tops_mean = ops_layer * L / (wall / K) / 1e12
    tops = ops_layer * L / (steps_ms["median"] * 1e-3) / 1e12

    log("kernel timing pass")
    call("tg_prof_enable", 1)
    for i in range(W, W + min(K, 4)):
        xb.copy_(X[i])
        blk.step(xb)
    torch.cuda.synchronize()
    call("tg_prof_enable", 0)
    names = ("route", "route_q8", "place", "group", "gateup_mfma", "down_mfma", "gu_down_mfma", "combine")
    kern = kernel_times(call, names)
    kern_us = {k: round(v[1] / max(v[0], 1) * 1e3, 3) for k, v in kern.items()}
    if "gu_down_mfma" in kern:  # gate/up and down in one launch: the roofline covers both products
        n_gu, ms_gu = kern["gu_down_mfma"]
        gu_ops = 2 * T * K_TOP * 3 * H * I
        roof_kernel, roof_traffic = "k_mfma16_gd (gate/up + down)", profiled_traffic("k_mfma16_gd")
    else:
        n_gu, ms_gu = kern["gateup_mfma"]
        gu_ops = 2 * T * K_TOP * 2 * H * I
        roof_kernel, roof_traffic = "k_mfma16<true> (gate/up)", profiled_traffic("k_mfma16/gate_up")
    achieved = gu_ops / (ms_gu / n_gu * 1e-3)
    layer_us = sum(kern_us.values())

    cpu = None
    if not args.no_cpu:
        log("prefill cpu baseline (oracle, one layer, 64 tokens)")
        from oracle import oracle as O  # the checker, timed as the CPU baseline
        lb = arena.read_layer(0)
        router = O.synth_normal(args.seed, O.stream_id(0, 0, 3), 0.02, E * H).reshape(E, H)
        Xs = X[W][:64].cpu().numpy()
        out = blk.forward(0, X[W][:64].contiguous())
        c = cpu_baseline_layer(lb, router, [Xs], args.cpu_seconds / 2, (Xs, out.cpu().numpy()))
        c["value_int_ops"] = round(c["value"] * 2 * K_TOP * 3 * H * I / 1e12, 4)
        c["unit_int_ops"] = "TOPS"
        cpu = c

    arena.set_batch_path(arena.BATCH_AUTO)
    return {
        "metric": "MoE prefill int8 TOPS (2048 tokens x 48-layer Q4_0 stack, grouped int8 MFMA)",
        "value": round(tops, 2), "unit": "TOPS", "steps": K, "warmup": W,
        "ms_per_step": round(wall * 1e3 / K, 3), "step_ms": steps_ms, "value_mean_steps": round(tops_mean, 2),
        "dtype": "q4_0 x q8_0 (int8 MFMA, fp32 accumulate)",
        "config": {"workload": "qwen3-30b-a3b-moe-prefill", "tokens": T, "layers": L, "hidden": H,
                   "experts": E, "moe_intermediate": I, "top_k": K_TOP, "ops_per_layer": ops_layer,
                   "us_per_layer": round(steps_ms["median"] * 1e3 / L, 2)},
        "mfma_frac": round(tops * 1e12 / MFMA_INT8_PEAK, 4),
        "kernel_avg_us": kern_us,
        "layer_kernel_us": round(layer_us, 2),
        "roofline": {"bound": "mfma", "kernel": roof_kernel, "ops_per_launch": gu_ops,
                     "achieved": round(achieved / 1e12, 1), "peak": MFMA_INT8_PEAK / 1e12, "unit": "TOPS",
                     "frac": round(achieved / MFMA_INT8_PEAK, 4), "traffic": roof_traffic},
        "cpu_baseline": cpu,
    }


def run_prefill(args, torch, call):
    """Config 4 alone: 2048 tokens through the 48-layer stack."""
    from tinygiant_amd.arena import HBMExpertArena

    L = args.layers
    K, W = args.steps or 20, 2 if args.warmup is None else args.warmup
    log(f"arena: {L} layers x {E} experts ({L * E * EXPERT_Q4_BYTES / 1e9:.2f} GB Q4_0)")
    arena = HBMExpertArena(L, E, H, I, K_TOP)
    for l in range(L):
        arena.synth_layer(l, args.seed)
    p = prefill_leg(args, torch, call, arena, L, K=K, W=W)
    arena.close()
    clk = measure_clock(call)
    p["clock"] = clk
    p["roofline"]["peak_at_measured_clock"] = clk["int8_peak_tops"]
    p["roofline"]["frac_at_measured_clock"] = round(p["roofline"]["achieved"] / clk["int8_peak_tops"], 4)
    p["data"] = "synthetic (N(0,0.02) Q4_0 experts and fp32 routers, N(0,1) tokens)"
    return headline(p)


def q4k_blocks(rng, n):
    """n random Q4_K blocks (144 bytes): finite fp16 d and dmin, any 6-bit
    scale/min field, random nibbles."""
    b = rng.integers(0, 256, (n, 144), dtype=np.uint8)
    b[:, 0:2] = rng.uniform(0.0005, 0.004, n).astype(np.float16).view(np.uint8).reshape(n, 2)
    b[:, 2:4] = rng.uniform(0.0, 0.004, n).astype(np.float16).view(np.uint8).reshape(n, 2)
    return b.reshape(-1)


def readonly_views(arrays):
    """The arrays written to one temporary file and mapped back read-only,
    one uint8 view per array: the form in which the reference's cache holds
    its experts (np.frombuffer over an ACCESS_READ mmap of the layer file,
    cache.py:31-55).  Returns the views and the mapping (kept open by the
    caller while the views are in use)."""
    import mmap
    import tempfile
    with tempfile.TemporaryFile() as f:
        for a in arrays:
            f.write(a.tobytes())
        f.flush()
        mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
    views, off = [], 0
    for a in arrays:
        views.append(np.frombuffer(mm, np.uint8, count=a.nbytes, offset=off))
        off += a.nbytes
    return views, mm


def run_legacy_moe(args, torch, call):
    """The legacy entry point tg_moe_forward (libtinygiant.c:647-655) as the
    reference's engine would call it: 8 Q4_K experts of the 30B shape
    (gate | up | down, 2,654,208 bytes each) in host memory, one call per
    layer; rotates over 16 sets of experts.  The call copies its operands to
    the device, so the rate is bound by the host-to-device copy; "pinned"
    times the same calls after tg_mlock of every expert, which keeps an HBM
    copy (the reference's cache locks its pinned experts the same way).  The
    roofline is the Q4_K row-dot kernel's on its device operands."""
    from tinygiant_amd._lib import require_lib
    lib = require_lib()
    rng = np.random.default_rng(args.seed)
    gb = I * (H // 256) * 144
    eb = 2 * gb + H * (I // 256) * 144
    NSET = 16
    flat, mm = readonly_views([q4k_blocks(rng, eb // 144) for _ in range(K_TOP * NSET)])
    sets = [flat[i * K_TOP:(i + 1) * K_TOP] for i in range(NSET)]
    ptrs = [(ctypes.c_void_p * K_TOP)(*[e.ctypes.data for e in st]) for st in sets]
    w = np.array([0.15, 0.14, 0.13, 0.13, 0.12, 0.11, 0.11, 0.11], np.float32)  # tools/nws_q8dot_bench.c:369
    x = rng.normal(0.0, 1.0, H).astype(np.float32)
    out = np.zeros(H, np.float32)
    K, W = args.steps or 64, 4 if args.warmup is None else args.warmup

    def step(i):
        lib.tg_moe_forward(ptrs[i % NSET], w.ctypes.data, K_TOP, x.ctypes.data, out.ctypes.data, H, I)

    log(f"warmup {W} calls")
    for i in range(W):
        step(i)
    log(f"timing {K} calls")
    t0 = time.perf_counter()
    for i in range(K):
        step(i)
    wall = time.perf_counter() - t0
    # the same calls with every expert locked, as the reference's cache locks its pinned experts
    # (cache.py:59-67): the views are read-only mappings, so tg_mlock keeps an HBM copy by default
    # and the calls read the experts from it
    for st in sets:
        for e in st:
            lib.tg_mlock(ctypes.c_void_p(e.ctypes.data), ctypes.c_size_t(e.nbytes))
    for i in range(W):
        step(i)
    t0 = time.perf_counter()
    for i in range(K):
        step(i)
    wall_pin = time.perf_counter() - t0
    mb, mr, mh, mm = ctypes.c_size_t(), ctypes.c_int(), ctypes.c_uint64(), ctypes.c_uint64()
    lib.tg_mirror_stats(ctypes.byref(mb), ctypes.byref(mr), ctypes.byref(mh), ctypes.byref(mm))
    call("tg_prof_enable", 1)
    for i in range(8):
        step(i)
    call("tg_prof_enable", 0)
    kern = kernel_times(call, ("lg_quant", "lg_q4k", "lg_silu", "lg_q4k_down", "lg_acc", "lg_moe_gateup",
                               "lg_moe_silu", "lg_moe_down"))
    kern_us = {k: round(v[1] / max(v[0], 1) * 1e3, 3) for k, v in kern.items()}
    if "lg_moe_gateup" in kern:  # every expert's gate and up rows in one launch
        n_q, ms_q = kern["lg_moe_gateup"]
        q_bytes = K_TOP * 2 * gb + (H // 256) * 264
        roof_name, roof_traffic = "k_moe_gateup_q4k", profiled_traffic("k_moe_gateup_q4k")
    else:
        n_q, ms_q = kern["lg_q4k"]
        q_bytes = gb + (H // 256) * 264  # one gate (or up) matrix and its Q8 activations
        roof_name, roof_traffic = "k_matmul_q4k (gate/up)", profiled_traffic("k_matmul_q4k/gate_up")
    achieved = q_bytes / (ms_q / n_q * 1e-3)

    cpu = None
    if not args.no_cpu:
        log("cpu baseline (oracle)")
        from oracle import oracle as O  # the checker, timed as the CPU baseline
        ref = O.moe_forward_q4k(sets[0], w, x, H, I)
        step(0)
        assert np.array_equal(ref.view(np.uint32), out.view(np.uint32)), "GPU legacy MoE differs from the oracle"
        n, t1 = 0, time.perf_counter()
        while time.perf_counter() - t1 < min(args.cpu_seconds, 10.0):
            O.moe_forward_q4k(sets[n % NSET], w, x, H, I)
            n += 1
        cpu_s = (time.perf_counter() - t1) / n
        cpu = {"value": round(1.0 / cpu_s, 2), "unit": "layer/s", "cores": 1, "kind": "port",
               "sample": f"{n} tg_moe_forward calls (8 Q4_K experts, 2048x768) through the C oracle, one thread; "
                         "bit-identical to the GPU call on the first set"}

    lib.tg_mirror_drop(None, 0)  # before the mapping goes with the views
    return {
        "metric": "legacy tg_moe_forward calls/s (8 Q4_K experts, 30B shape, host pointers)",
        "value": round(K / wall, 2), "unit": "layer/s", "n_gpus": 1, "steps": K, "warmup": W,
        "ms_per_step": round(wall * 1e3 / K, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "q4_k x q8 (int dot, fp32 accumulate)",
        "data": "synthetic (random Q4_K blocks, N(0,1) input)",
        "config": {"workload": "legacy-q4k-moe-forward", "hidden": H, "moe_intermediate": I, "experts": K_TOP,
                   "expert_bytes": eb, "note": "experts in read-only mmap views of one file, as the reference's "
                                               "cache maps them; each call copies 21.2 MB of them to the device"},
        "pinned": {"value": round(K / wall_pin, 2), "unit": "layer/s", "ms_per_step": round(wall_pin * 1e3 / K, 4),
                   "note": f"after tg_mlock of every expert: {mb.value / 1e6:.1f} MB in {mr.value} HBM copies, "
                           f"{mh.value} operand reads from them, {mm.value} copied"},
        "kernel_avg_us": kern_us,
        "roofline": {"bound": "hbm", "kernel": roof_name, "bytes_per_launch": q_bytes,
                     "achieved": round(achieved / 1e9, 1), "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK, 4), "traffic": roof_traffic},
        "cpu_baseline": cpu,
    }


def run_legacy_expert(args, torch, call):
    """The reference engine's own MoE loop (engine.py:240-257): moe_out
    zeroed, then one tg_expert_forward_mixed call per selected expert
    (libtinygiant.c:599-643; 8 Q4_K experts of the 30B shape, down format 0)
    adding weight * expert(x) into it; rotates over 16 sets of experts, first
    with the operands copied per call, then ("pinned") after tg_mlock of every
    expert, as the reference's cache locks its pinned experts."""
    from tinygiant_amd._lib import require_lib
    lib = require_lib()
    rng = np.random.default_rng(args.seed)
    gb = I * (H // 256) * 144
    eb = 2 * gb + H * (I // 256) * 144
    NSET = 16
    flat, mm = readonly_views([q4k_blocks(rng, eb // 144) for _ in range(K_TOP * NSET)])
    sets = [flat[i * K_TOP:(i + 1) * K_TOP] for i in range(NSET)]
    w = np.array([0.15, 0.14, 0.13, 0.13, 0.12, 0.11, 0.11, 0.11], np.float32)
    x = rng.normal(0.0, 1.0, H).astype(np.float32)
    out = np.zeros(H, np.float32)
    K, W = args.steps or 64, 4 if args.warmup is None else args.warmup

    def step(i):
        out[:] = 0.0
        for j, e in enumerate(sets[i % NSET]):
            base = e.ctypes.data
            lib.tg_expert_forward_mixed(ctypes.c_void_p(base), ctypes.c_void_p(base + gb),
                                        ctypes.c_void_p(base + 2 * gb), 0, x.ctypes.data, out.ctypes.data,
                                        ctypes.c_float(float(w[j])), H, I)

    def timed():
        for i in range(W):
            step(i)
        t0 = time.perf_counter()
        for i in range(K):
            step(i)
        return time.perf_counter() - t0

    log(f"timing {K} layers (8 calls each), operands copied per call")
    wall = timed()
    for st in sets:
        for e in st:
            lib.tg_mlock(ctypes.c_void_p(e.ctypes.data), ctypes.c_size_t(e.nbytes))
    log(f"timing {K} layers after tg_mlock")
    wall_pin = timed()
    call("tg_prof_enable", 1)
    for i in range(4):
        step(i)
    call("tg_prof_enable", 0)
    kern = kernel_times(call, ("lg_quant", "lg_moe_gateup", "lg_moe_silu", "lg_moe_down", "lg_q4k", "lg_silu",
                               "lg_q4k_down", "lg_acc"))
    kern_us = {k: round(v[1] / max(v[0], 1) * 1e3, 3) for k, v in kern.items()}
    if "lg_moe_gateup" in kern:  # one expert's gate and up rows in one launch
        n_q, ms_q = kern["lg_moe_gateup"]
        q_bytes, roof_name = 2 * gb + (H // 256) * 264, "k_moe_gateup_q4k (one expert)"
    else:  # the per-expert chain (TG_LEGACY_MOE_ALL=0)
        n_q, ms_q = kern["lg_q4k"]
        q_bytes, roof_name = gb + (H // 256) * 264, "k_matmul_q4k (gate/up)"
    achieved = q_bytes / (ms_q / n_q * 1e-3)

    cpu = None
    if not args.no_cpu:
        log("cpu baseline (oracle)")
        from oracle import oracle as O  # the checker, timed as the CPU baseline
        step(0)
        ref = O.moe_forward_q4k(sets[0], w, x, H, I)  # zero, then out += w * expert(x) expert by expert
        assert np.array_equal(ref.view(np.uint32), out.view(np.uint32)), "GPU expert loop differs from the oracle"
        n, t1 = 0, time.perf_counter()
        while time.perf_counter() - t1 < min(args.cpu_seconds, 10.0):
            O.moe_forward_q4k(sets[n % NSET], w, x, H, I)
            n += 1
        cpu_s = (time.perf_counter() - t1) / n
        cpu = {"value": round(1.0 / cpu_s, 2), "unit": "layer/s", "cores": 1, "kind": "port",
               "sample": f"{n} layers of 8 Q4_K experts (2048x768) through the C oracle, one thread; the GPU loop "
                         "bit-identical to it on the first set"}
    lib.tg_mirror_drop(None, 0)  # before the mapping goes with the views
    return {
        "metric": "legacy engine MoE loop layers/s (8 tg_expert_forward_mixed calls, 30B shape, host pointers)",
        "value": round(K / wall, 2), "unit": "layer/s", "n_gpus": 1, "steps": K, "warmup": W,
        "ms_per_step": round(wall * 1e3 / K, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "q4_k x q8 (int dot, fp32 accumulate)",
        "data": "synthetic (random Q4_K blocks, N(0,1) input)",
        "config": {"workload": "legacy-engine-expert-loop", "hidden": H, "moe_intermediate": I, "experts": K_TOP,
                   "expert_bytes": eb, "note": "experts in read-only mmap views of one file, as the reference's "
                                               "cache maps them"},
        "pinned": {"value": round(K / wall_pin, 2), "unit": "layer/s", "ms_per_step": round(wall_pin * 1e3 / K, 4)},
        "kernel_avg_us": kern_us,
        "roofline": {"bound": "hbm", "kernel": roof_name, "bytes_per_launch": q_bytes,
                     "achieved": round(achieved / 1e9, 1), "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK, 4), "traffic": None},
        "cpu_baseline": cpu,
    }


def run_legacy_layer(args, torch, call):
    """The legacy entry point tg_transformer_layer (libtinygiant.c:662-702)
    with host buffers, as the reference's engine calls it: a 30B-shaped layer
    (embed 2048, 32 query heads and 4 kv heads of 128, f32 attention weights,
    a cache of kv_max 2048 rows of which 1024 are filled) and 8 Q4_K experts.
    Each call copies its operands (about 105 MB) to the device."""
    from tinygiant_amd._lib import require_lib
    lib = require_lib()
    rng = np.random.default_rng(args.seed)
    Hh, KV, hd, kv_max, kv_len = 32, 4, 128, 2048, 1024
    qd, kvd = Hh * hd, KV * hd
    w = [rng.normal(0, 0.02, n).astype(np.float32) for n in (qd * H, kvd * H, kvd * H, H * qd)]
    an, fn_ = (rng.normal(1.0, 0.1, H).astype(np.float32) for _ in range(2))
    qn, kn = (rng.normal(1.0, 0.1, hd).astype(np.float32) for _ in range(2))
    ang = np.arange(kv_max)[:, None] * (10000.0 ** (-np.arange(hd // 2) / (hd // 2)))[None, :]
    cos_t, sin_t = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    kv_k = rng.normal(0, 1, (KV, kv_max, hd)).astype(np.float32)
    kv_v = rng.normal(0, 1, (KV, kv_max, hd)).astype(np.float32)
    gb = I * (H // 256) * 144
    experts, mm = readonly_views([q4k_blocks(rng, (2 * gb + H * (I // 256) * 144) // 144) for _ in range(K_TOP)])
    gp = (ctypes.c_void_p * K_TOP)(*[e.ctypes.data for e in experts])
    up = (ctypes.c_void_p * K_TOP)(*[e.ctypes.data + gb for e in experts])
    dp = (ctypes.c_void_p * K_TOP)(*[e.ctypes.data + 2 * gb for e in experts])
    dif = np.zeros(K_TOP, np.int32)
    ew = np.array([0.15, 0.14, 0.13, 0.13, 0.12, 0.11, 0.11, 0.11], np.float32)
    x0 = rng.normal(0, 1, H).astype(np.float32)
    x = x0.copy()
    K, W = args.steps or 32, 2 if args.warmup is None else args.warmup

    def step():
        x[:] = x0
        lib.tg_transformer_layer(*(a.ctypes.data for a in w), an.ctypes.data, qn.ctypes.data, kn.ctypes.data,
                                 fn_.ctypes.data, kv_k.ctypes.data, kv_v.ctypes.data, kv_len, kv_max,
                                 cos_t.ctypes.data, sin_t.ctypes.data, gp, up, dp, dif.ctypes.data, ew.ctypes.data,
                                 K_TOP, x.ctypes.data, H, I, Hh, KV, hd, kv_len)

    log(f"warmup {W} calls")
    for _ in range(W):
        step()
    log(f"timing {K} calls")
    t0 = time.perf_counter()
    for _ in range(K):
        step()
    wall = time.perf_counter() - t0
    # the same calls after tg_mlock of every weight, as the reference's engine locks its attention weights
    # (engine.py:134-139) and its cache the pinned experts (cache.py:59-67): the weights are then read from
    # HBM copies; the KV rows, x and the rope rows are still copied per call.  The attention weights are
    # writable numpy arrays, copied only in TG_MIRROR_ALL (they are never written after the lock)
    lib.tg_mirror_mode(2)
    for a in (*w, an, fn_, qn, kn, *experts):
        lib.tg_mlock(ctypes.c_void_p(a.ctypes.data), ctypes.c_size_t(a.nbytes))
    for _ in range(W):
        step()
    log(f"timing {K} calls after tg_mlock")
    t0 = time.perf_counter()
    for _ in range(K):
        step()
    wall_pin = time.perf_counter() - t0
    call("tg_prof_enable", 1)
    for _ in range(4):
        step()
    call("tg_prof_enable", 0)
    kern = kernel_times(call, ("lg_f32", "lg_rms", "lg_rope", "lg_kv", "lg_attn_sc", "lg_attn_sm", "lg_attn", "lg_add",
                               "lg_quant", "lg_q4k", "lg_silu", "lg_q4k_down", "lg_acc", "lg_moe_gateup",
                               "lg_moe_silu", "lg_moe_down"))
    kern_us = {k: round(v[1] / max(v[0], 1) * 1e3, 3) for k, v in kern.items()}
    # dominant kernel: the f32 q / k / v / o projections (k_matvec_two_acc),
    # bytes per launch = weights + input averaged over the four launches
    n_f, ms_f = kern["lg_f32"]
    proj_shapes = ((Hh * hd, H), (KV * hd, H), (KV * hd, H), (H, Hh * hd))
    proj_bytes = sum(4 * (r * c + c + r) for r, c in proj_shapes) / len(proj_shapes)
    achieved = proj_bytes / (ms_f / n_f * 1e-3)
    # attention proper: scores, softmax weights, weighted sum of V
    attn_bytes = 2 * KV * (kv_len + 1) * hd * 4  # the K and V cache rows, each read once
    attn_us = sum(kern[k][1] / kern[k][0] * 1e3 for k in ("lg_attn_sc", "lg_attn_sm", "lg_attn") if k in kern)

    cpu = None
    if not args.no_cpu:
        log("cpu baseline (oracle)")
        from oracle import oracle as O  # the checker, timed as the CPU baseline
        rk, rv, rx = kv_k.copy(), kv_v.copy(), x0.copy()
        O.transformer_layer(*w, an, qn, kn, fn_, rk, rv, kv_len, kv_max, cos_t, sin_t, [e for e in experts],
                            [e[gb:] for e in experts], [e[2 * gb:] for e in experts], list(dif), ew, rx, H, I, Hh,
                            KV, hd, kv_len)
        step()
        assert np.array_equal(rx.view(np.uint32), x.view(np.uint32)), "GPU legacy layer differs from the oracle"
        n, t1 = 0, time.perf_counter()
        while time.perf_counter() - t1 < min(args.cpu_seconds, 10.0):
            O.transformer_layer(*w, an, qn, kn, fn_, kv_k.copy(), kv_v.copy(), kv_len, kv_max, cos_t, sin_t,
                                [e for e in experts], [e[gb:] for e in experts], [e[2 * gb:] for e in experts],
                                list(dif), ew, x0.copy(), H, I, Hh, KV, hd, kv_len)
            n += 1
        cpu_s = (time.perf_counter() - t1) / n
        cpu = {"value": round(1.0 / cpu_s, 2), "unit": "layer/s", "cores": 1, "kind": "port",
               "sample": f"{n} tg_transformer_layer calls through the C oracle, one thread; bit-identical to the "
                         "GPU call"}

    lib.tg_mirror_drop(None, 0)  # before the mapping goes with the views
    lib.tg_mirror_mode(1)
    return {
        "metric": "legacy tg_transformer_layer calls/s (30B-shaped layer, 1024 cached positions, host pointers)",
        "value": round(K / wall, 2), "unit": "layer/s", "n_gpus": 1, "steps": K, "warmup": W,
        "ms_per_step": round(wall * 1e3 / K, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32 attention, q4_k x q8 experts", "data": "synthetic",
        "config": {"workload": "legacy-transformer-layer", "hidden": H, "heads": Hh, "kv_heads": KV, "head_dim": hd,
                   "kv_len": kv_len, "experts": K_TOP, "moe_intermediate": I},
        "pinned": {"value": round(K / wall_pin, 2), "unit": "layer/s", "ms_per_step": round(wall_pin * 1e3 / K, 4),
                   "note": "after tg_mlock of every weight (attention, norms, experts; tg_mirror_mode "
                           "TG_MIRROR_ALL, since the attention weights are writable arrays); the KV rows still copied"},
        "kernel_avg_us": kern_us,
        "roofline": {"bound": "hbm", "kernel": "k_matvec_two_acc (f32 projections)",
                     "bytes_per_launch": round(proj_bytes), "achieved": round(achieved / 1e9, 1),
                     "peak": HBM_PEAK / 1e9, "unit": "GB/s", "frac": round(achieved / HBM_PEAK, 4),
                     "traffic": profiled_traffic("k_matvec_two_acc/f32")},
        "attention": {"kernels": "k_attn_scores + k_attn_softmax + k_attn_wv", "us": round(attn_us, 3),
                      "cache_bytes": attn_bytes, "gbps": round(attn_bytes / (attn_us * 1e-6) / 1e9, 1)},
        "cpu_baseline": cpu,
    }


def run_hbm_ceiling(args, torch, call):
    """What one launch can read from HBM: plain 128-bit loads over regions of
    the sizes the MoE kernels stream, rotating over a 16 GiB buffer so no
    launch finds its bytes in the caches."""
    total = 16 << 30
    buf = torch.empty(total, dtype=torch.uint8, device="cuda")
    buf.fill_(1)
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    rows = []
    sizes = {"gate+up, 8 experts": 8 * GATEUP_BYTES_PER_EXPERT, "one layer, 8 experts": 8 * EXPERT_Q4_BYTES,
             "235B layer, 8 experts": 84934656, "one layer, all 128 experts": E * EXPERT_Q4_BYTES}
    for name, nbytes in sizes.items():
        nreg = min(total // nbytes, 400)
        best = None
        for grid in (256, 512, 1024, 2048):
            for w in range(4):
                call("tg_stream_read_dev", buf.data_ptr() + (w % nreg) * nbytes, nbytes, grid, sink.data_ptr(), st)
            ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            R = args.steps or 200
            ev0.record()
            for r in range(R):
                call("tg_stream_read_dev", buf.data_ptr() + ((r * 7) % nreg) * nbytes, nbytes, grid, sink.data_ptr(),
                     st)
            ev1.record()
            torch.cuda.synchronize()
            us = ev0.elapsed_time(ev1) * 1e3 / R
            if best is None or us < best[1]:
                best = (grid, us)
        rows.append({"region": name, "bytes": nbytes, "grid": best[0], "us_per_launch": round(best[1], 2),
                     "gbps": round(nbytes / best[1] / 1e3, 1)})
        log(f"{name}: {rows[-1]}")
    top = max(rows, key=lambda r: r["gbps"])
    return {"metric": "HBM read ceiling of one launch (back-to-back launches, plain 128-bit loads)",
            "value": top["gbps"], "unit": "GB/s", "n_gpus": 1, "steps": args.steps or 200, "warmup": 4,
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "u8",
            "data": "synthetic", "config": {"workload": "hbm-read-ceiling", "regions": rows},
            "roofline": {"bound": "hbm", "achieved": top["gbps"], "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                         "frac": round(top["gbps"] * 1e9 / HBM_PEAK, 4), "traffic": None},
            "cpu_baseline": None}


def run_output_head(args, torch, call):
    """The output head after the layers (engine.py:262-266,359): logits =
    W @ rms_norm(x) with the Qwen3-30B-A3B head W 151936 x 2048 fp32 (1.24 GB,
    resident in HBM behind tg_head_create), then the greedy token.  One step =
    one tg_head_forward call: the 8 KB input copied in, norm, matvec, argmax,
    the token copied back (the logits stay on the device)."""
    from tinygiant_amd._lib import require_lib
    lib = require_lib()
    V = 151936
    rng = np.random.default_rng(args.seed)
    log(f"head weights {V} x {H} fp32 ({V * H * 4 / 1e9:.2f} GB)")
    W = rng.standard_normal((V, H), dtype=np.float32) * np.float32(0.02)
    nw = rng.normal(1.0, 0.1, H).astype(np.float32)
    xs = [rng.normal(0, 1, H).astype(np.float32) for _ in range(8)]
    h = lib.tg_head_create(W.ctypes.data, nw.ctypes.data, V, H)
    if not h:
        raise RuntimeError(f"tg_head_create: {lib.tg_last_error().decode()}")
    tok = ctypes.c_int32()
    K, W_ = args.steps or 200, 10 if args.warmup is None else args.warmup

    def step(i):
        rc = lib.tg_head_forward(h, xs[i % len(xs)].ctypes.data, 1e-6, None, ctypes.byref(tok))
        if rc:
            raise RuntimeError(f"tg_head_forward: {lib.tg_last_error().decode()}")

    log(f"warmup {W_} calls")
    for i in range(W_):
        step(i)
    log(f"timing {K} calls")
    t0 = time.perf_counter()
    for i in range(K):
        step(i)
    wall = time.perf_counter() - t0
    call("tg_prof_enable", 1)
    for i in range(16):
        step(i)
    call("tg_prof_enable", 0)
    kern = kernel_times(call, ("head_rms", "head_mv", "head_argmax"))
    kern_us = {k: round(v[1] / max(v[0], 1) * 1e3, 3) for k, v in kern.items()}
    n_m, ms_m = kern["head_mv"]
    mv_bytes = 4 * (V * H + H + V)
    achieved = mv_bytes / (ms_m / n_m * 1e-3)

    cpu = None
    if not args.no_cpu:
        log("cpu baseline (oracle)")
        from oracle import oracle as O  # the checker, timed as the CPU baseline
        logits, ref_tok = O.output_head(W, nw, xs[0], 1e-6)
        step(0)
        assert tok.value == ref_tok, "GPU head token differs from the oracle"
        n, t1 = 0, time.perf_counter()
        while time.perf_counter() - t1 < min(args.cpu_seconds, 10.0):
            O.output_head(W, nw, xs[n % len(xs)], 1e-6)
            n += 1
        cpu_s = (time.perf_counter() - t1) / n
        cpu = {"value": round(1.0 / cpu_s, 2), "unit": "tok/s", "cores": 1, "kind": "port",
               "sample": f"{n} output-head calls (norm + 151936 x 2048 fp32 matvec + argmax) through the C oracle, "
                         "one thread; same token as the GPU call"}
    lib.tg_head_destroy(h)
    return {
        "metric": "output head tok/s (151936 x 2048 fp32 logits + greedy token, weights resident)",
        "value": round(K / wall, 2), "unit": "tok/s", "n_gpus": 1, "steps": K, "warmup": W_,
        "ms_per_step": round(wall * 1e3 / K, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic (N(0, 0.02) fp32 head, N(0, 1) inputs)",
        "config": {"workload": "qwen3-30b-a3b-output-head", "vocab": V, "hidden": H},
        "kernel_avg_us": kern_us,
        "roofline": {"bound": "hbm", "kernel": "k_matvec_two_acc (head)", "bytes_per_launch": mv_bytes,
                     "achieved": round(achieved / 1e9, 1), "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK, 4), "traffic": profiled_traffic("k_matvec_two_acc/head")},
        "cpu_baseline": cpu,
    }


def run_sample(args, torch, call):
    """Next-token sampling after the head (engine.py:348-357 with the
    reference's defaults T 0.7, top_p 0.9) at the Qwen3 vocabulary 151936, on
    logits resident in HBM: one step = one tg_sampler_run (its launches and
    the token copied back).  Logits N(0, 2.5): about a hundred candidates.
    The same call with top_p 1.0 (every token a candidate: the global-memory
    sort) is timed beside it."""
    from tinygiant_amd._lib import require_lib
    from oracle import sample as S  # the checker, timed as the CPU baseline
    lib = require_lib()
    V, T, TOP_P = 151936, 0.7, 0.9
    rng = np.random.default_rng(args.seed)
    logits = [(rng.standard_normal(V) * 2.5).astype(np.float32) for _ in range(8)]
    dl = [torch.from_numpy(l).to("cuda:0") for l in logits]
    torch.cuda.synchronize()
    s = lib.tg_sampler_create(V)
    if not s:
        raise RuntimeError(f"tg_sampler_create: {lib.tg_last_error().decode()}")
    tok = ctypes.c_int32()
    us = rng.random(64)

    def step(i, top_p=TOP_P):
        rc = lib.tg_sampler_run(s, ctypes.c_void_p(dl[i % 8].data_ptr()), 1, np.float32(T), top_p, us[i % 64],
                                ctypes.byref(tok), None)
        if rc:
            raise RuntimeError(f"tg_sampler_run: {lib.tg_last_error().decode()}")
        return tok.value

    for i in range(8):  # the same tokens as the numpy restatement
        ref = S.sample(logits[i], T, TOP_P, us[i])[0]
        assert step(i) == ref, "GPU token differs from the restatement"
    K, W_ = args.steps or 200, 10 if args.warmup is None else args.warmup
    log(f"warmup {W_} calls")
    for i in range(W_):
        step(i)
    log(f"timing {K} calls")
    times = []
    for i in range(K):
        t0 = time.perf_counter()
        step(i)
        times.append(time.perf_counter() - t0)
    times_all = []
    for i in range(max(K // 4, 10)):
        t0 = time.perf_counter()
        step(i, 1.0)
        times_all.append(time.perf_counter() - t0)
    call("tg_prof_enable", 1)
    for i in range(16):
        step(i)
    call("tg_prof_enable", 0)
    kern = kernel_times(call, ("sample",))
    n_k, ms_k = kern["sample"]
    med = float(np.median(times))
    cpu = None
    if not args.no_cpu:
        log("cpu baseline (numpy, the reference's sampling code restated)")
        n, t1 = 0, time.perf_counter()
        while time.perf_counter() - t1 < min(args.cpu_seconds, 10.0):
            S.sample(logits[n % 8], T, TOP_P, us[n % 64], exp="numpy")
            n += 1
        cpu_s = (time.perf_counter() - t1) / n
        cpu = {"value": round(1.0 / cpu_s, 2), "unit": "tok/s", "cores": 1, "kind": "port",
               "sample": f"{n} draws of engine.py:348-357 in numpy (float32 exp, argsort of 151936) on this host"}
    lib.tg_sampler_destroy(s)
    return {
        "metric": "next-token sampling tok/s (T 0.7, top_p 0.9, vocab 151936, logits resident)",
        "value": round(1.0 / med, 2), "unit": "tok/s", "n_gpus": 1, "steps": K, "warmup": W_,
        "ms_per_step": round(med * 1e3, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic (N(0, 2.5) logits, uniform draws)",
        "config": {"workload": "qwen3-sampling", "vocab": V, "temperature": T, "top_p": TOP_P},
        "launches_us": round(ms_k / max(n_k, 1) * 1e3, 2),
        "top_p_1_ms": round(float(np.median(times_all)) * 1e3, 4),
        "cpu_baseline": cpu,
    }


WORKLOADS = {"decode-stack": run_decode_stack, "batched": run_batched, "prefill": run_prefill,
             "decode-235b": lambda a, t, c: run_235b(a, t, c, 1),
             "batched-235b": lambda a, t, c: run_235b(a, t, c, 32),
             "hbm-ceiling": run_hbm_ceiling, "legacy-moe": run_legacy_moe, "legacy-layer": run_legacy_layer,
             "legacy-expert": run_legacy_expert,
             "output-head": run_output_head, "sample": run_sample}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="decode-stack")
    ap.add_argument("--layers", type=int, default=48)
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill", action="store_true", help="default workload: skip the prefill leg")
    ap.add_argument("--no-batched", action="store_true", help="default workload: skip the batched leg")
    ap.add_argument("--no-235b", action="store_true", help="default workload: skip the two 235B-shaped legs")
    ap.add_argument("--path", choices=list(DECODE_PATHS), default="auto",
                    help="decode path of one-token stack calls")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures a single GPU (one MI355X); --gpus must be 1. "
              "Expert-parallel sharding over several GPUs is designed but not built.",
              file=sys.stderr)
        return 2

    import torch
    from tinygiant_amd._lib import call, require_lib

    require_lib()
    call("tg_gpu_init", 0)
    out = WORKLOADS[args.workload](args, torch, call)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
