#!/usr/bin/env python3
"""Benchmark of the fused tile-local Strassen GEMM on one MI355X.

Workload (one "step"): the GEMM sites of one Qwen3-32B-shaped decoder block
at 8 x 1024 tokens, each with its fused epilogue, on synthetic bf16 data
already resident in HBM:

  q     X[8192,5120]  . Wq[5120,8192]   + per-head RMSNorm + RoPE (qk_norm_rope)
  k     X[8192,5120]  . Wk[5120,1024]   + qk_norm_rope
  v     X[8192,5120]  . Wv[5120,1024]
  o     O[8192,8192]  . Wo[8192,5120]   + residual (residual_add)
  gate|up Y[8192,5120] . Wgu[5120,51200] -> silu(gate)*up (swiglu) -> H[8192,25600]
  down  H[8192,25600] . Wd[25600,5120]  + residual (residual_add)

7.989 TFLOP per step (2*M*N*K summed over the sites, the classical count for
every arm). Arms: "strassen" (the 7-product kernels: the product-major
kernel on the whole rounds of a call's tiles, the split kernel on the rest),
"cubic" (matched 8-product kernel, identical tiling and epilogues) and
"hipblaslt" (torch.matmul, with the epilogues as separate torch ops);
"strassen_split" and "strassen_product_major" are the Strassen weights on one
of its kernels alone. Printed value: effective TFLOP/s of the Strassen arm.
The pure GEMMs at the same shapes (no epilogue) are reported in "pure_gemm".

One JSON line on stdout; progress on stderr.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

METRIC = "block ms + effective TFLOP/s vs matched cubic MFMA, Qwen3-32B shapes, 8x1024 tok"
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA (AMD spec)

TOKENS, HIDDEN, FFN = 8192, 5120, 25600
HEADS, KV_HEADS, HEAD_DIM = 64, 8, 128
BATCH, SEQ = 8, 1024
THETA, EPS = 1e6, 1e-6
TILE = (1024, 1024, 512)
COPY_BYTES = 256 << 20
# The default Strassen arm's packed weights on the library's other Strassen
# kernels (the default runs the product-major kernel on whole rounds of its
# tiles and the split kernel on the rest).
KERNEL_ARMS = {"strassen_split": "split", "strassen_product_major": "product_major"}


def log(*args):
    print(*args, file=sys.stderr, flush=True)


def site_shapes():
    q, kv = HEADS * HEAD_DIM, KV_HEADS * HEAD_DIM
    return {
        "q": (TOKENS, HIDDEN, q),
        "k": (TOKENS, HIDDEN, kv),
        "v": (TOKENS, HIDDEN, kv),
        "o": (TOKENS, q, HIDDEN),
        "gate_up": (TOKENS, HIDDEN, 2 * FFN),
        "down": (TOKENS, FFN, HIDDEN),
    }


def flops(shape):
    m, k, n = shape
    return 2.0 * m * n * k


def make_block(torch, dev, seed=0):
    """Random-init weights and activations of the block's GEMM sites."""
    import strassen_tpu_amd as smx

    bm, bn, bk = TILE
    g = torch.Generator(device=dev).manual_seed(seed)

    def randn(*shape, std=1.0):
        return (torch.randn(*shape, device=dev, generator=g) * std).to(torch.bfloat16)

    d = {}
    d["x"] = randn(TOKENS, HIDDEN)            # normalised attention input
    d["attn"] = randn(TOKENS, HEADS * HEAD_DIM)
    d["y"] = randn(TOKENS, HIDDEN)            # normalised MLP input
    d["res1"] = randn(TOKENS, HIDDEN)
    d["res2"] = randn(TOKENS, HIDDEN)
    # Weights stored [out, in]; the GEMM's B operand is the [in, out] view.
    for name, (out_f, in_f) in {"wq": (HEADS * HEAD_DIM, HIDDEN), "wk": (KV_HEADS * HEAD_DIM, HIDDEN),
                                "wv": (KV_HEADS * HEAD_DIM, HIDDEN), "wo": (HIDDEN, HEADS * HEAD_DIM),
                                "wgu": (2 * FFN, HIDDEN), "wd": (HIDDEN, FFN)}.items():
        d[name] = randn(out_f, in_f, std=0.02).t()
    gamma_q = (1.0 + 0.1 * torch.randn(HEAD_DIM, device=dev, generator=g)).to(torch.bfloat16)
    gamma_k = (1.0 + 0.1 * torch.randn(HEAD_DIM, device=dev, generator=g)).to(torch.bfloat16)
    pos = torch.arange(SEQ, dtype=torch.float32, device=dev)[:, None]
    inv = 1.0 / (THETA ** (torch.arange(0, HEAD_DIM, 2, dtype=torch.float32, device=dev) / HEAD_DIM))
    ang = torch.cat([pos * inv[None, :]] * 2, dim=-1)
    cos, sin = torch.cos(ang).to(torch.bfloat16), torch.sin(ang).to(torch.bfloat16)
    d["cos"], d["sin"], d["gamma_q"], d["gamma_k"] = cos, sin, gamma_q, gamma_k
    # Offline relayouts (strassen_pallas.py:1315-1411), done once.
    d["wq_laid"] = smx.rope_weight_layout(d["wq"], bn, HEAD_DIM)
    d["wk_laid"] = smx.rope_weight_layout(d["wk"], bn, HEAD_DIM)
    d["wgu_laid"] = smx.swiglu_weight_layout(d["wgu"], bn)
    tcos, tsin = smx.rope_layout_tables(cos.repeat(BATCH, 1), sin.repeat(BATCH, 1), bn // 2, HEAD_DIM)
    d["tcos"], d["tsin"] = tcos, tsin
    d["scale_q"] = smx.rope_scale_layout(gamma_q, bn, HEAD_DIM)
    d["scale_k"] = smx.rope_scale_layout(gamma_k, bn, HEAD_DIM)
    # Packed weights (offline, like the relayouts above): the seven Strassen
    # B operand sums ("_sw") and the cubic's four quadrants ("_cw").
    d["wup"] = d["wgu"][:, :FFN]
    for name in ("wq_laid", "wk_laid", "wv", "wo", "wgu_laid", "wd", "wup"):
        d[name + "_sw"] = smx.strassen_weight_layout(d[name], bn, bk)
        d[name + "_cw"] = smx.cubic_weight_layout(d[name], bn, bk)
    return d


# The six block sites' weights (B operands) as make_block names them.
SITE_WEIGHTS = ("wq_laid", "wk_laid", "wv", "wo", "wgu_laid", "wd")


def weight_memory(d):
    """HBM bytes the block's six weights occupy in each arm's form: plain
    bf16, the seven packed Strassen operand sums (7/4 of plain) and the
    cubic's four packed quadrants (the plain size)."""
    def total(suffix):
        return int(sum((d[n + suffix].data if suffix else d[n]).numel() * 2 for n in SITE_WEIGHTS))

    plain, strassen, cubic = total(""), total("_sw"), total("_cw")
    gu = d["wgu_laid"].numel() * 2
    return {"plain_bytes": plain, "strassen_packed_bytes": strassen, "cubic_packed_bytes": cubic,
            "strassen_over_plain": round(strassen / plain, 4),
            "gate_up_bytes": {"plain": gu, "strassen_packed": int(d["wgu_laid_sw"].data.numel() * 2),
                              "cubic_packed": int(d["wgu_laid_cw"].data.numel() * 2)}}


# Weight suffix and algorithm id of each kernel arm.
ARM_WEIGHTS = {"strassen": ("_sw", 7), "cubic": ("_cw", 8), "strassen_plain": ("", 7), "cubic_plain": ("", 8)}


def fused_sites(torch, d, algo):
    """Callables for a fused arm, keyed by site. algo: "strassen" / "cubic"
    (packed weights; each activation is packed once per step, inside the
    step, and shared by the GEMMs that read it) or "strassen_plain" /
    "cubic_plain" (ordinary [in, out] weights, as a drop-in caller passes
    them: every call packs its weight and its activation, then runs the same
    packed kernel)."""
    import strassen_tpu_amd as smx

    bm, bn, bk = TILE
    suffix, algo_id = ARM_WEIGHTS[algo]
    fn = smx.cubic_matmul if algo.startswith("cubic") else smx.strassen_matmul
    packed = suffix != ""
    kw = dict(bm=bm, bn=bn, bk=bk)
    if not algo.startswith("cubic"):
        kw["interleave_products"] = True
    qk = dict(epilogue="qk_norm_rope", rope_cos=d["tcos"], rope_sin=d["tsin"], rope_head_dim=HEAD_DIM,
              rope_eps=EPS)
    act = {}

    def operand(name, fresh):
        """The activation as the arm consumes it (packed once when fresh)."""
        if not packed:
            return d[name]
        if fresh or name not in act:
            act[name] = smx.pack_activation(d[name], algo_id, bm, bk)
        return act[name]

    out = {}
    out["q"] = lambda: fn(operand("x", True), d["wq_laid" + suffix], rope_scale=d["scale_q"], **qk, **kw)
    out["k"] = lambda: fn(operand("x", False), d["wk_laid" + suffix], rope_scale=d["scale_k"], **qk, **kw)
    out["v"] = lambda: fn(operand("x", False), d["wv" + suffix], **kw)
    out["o"] = lambda: fn(operand("attn", True), d["wo" + suffix], epilogue="residual_add", residual=d["res1"],
                          **kw)

    def gate_up():
        d["h"] = fn(operand("y", True), d["wgu_laid" + suffix], epilogue="swiglu", **kw)
        return d["h"]

    out["gate_up"] = gate_up
    out["down"] = lambda: fn(operand("h", True), d["wd" + suffix], epilogue="residual_add", residual=d["res2"],
                             **kw)
    return out


def vendor_sites(torch, d):
    """hipBLASLt GEMMs with the same epilogues as separate torch ops."""
    f32 = torch.float32

    def qk_norm_rope(y, gamma, heads):
        t = y.view(TOKENS, heads, HEAD_DIM).float()
        t = t * torch.rsqrt(t.pow(2).mean(-1, keepdim=True) + EPS) * gamma.float()
        c = d["cos"].float().repeat(BATCH, 1)[:, None, :]
        s = d["sin"].float().repeat(BATCH, 1)[:, None, :]
        x1, x2 = t.chunk(2, dim=-1)
        return (t * c + torch.cat([-x2, x1], dim=-1) * s).to(torch.bfloat16)

    out = {}
    out["q"] = lambda: qk_norm_rope(torch.matmul(d["x"], d["wq"]), d["gamma_q"], HEADS)
    out["k"] = lambda: qk_norm_rope(torch.matmul(d["x"], d["wk"]), d["gamma_k"], KV_HEADS)
    out["v"] = lambda: torch.matmul(d["x"], d["wv"])
    out["o"] = lambda: (torch.matmul(d["attn"], d["wo"]).to(f32) + d["res1"].to(f32)).to(torch.bfloat16)

    def gate_up():
        gu = torch.matmul(d["y"], d["wgu"])
        g, u = gu.chunk(2, dim=-1)
        d["h_v"] = (torch.nn.functional.silu(g.float()) * u.float()).to(torch.bfloat16)
        return d["h_v"]

    out["gate_up"] = gate_up
    out["down"] = lambda: (torch.matmul(d["h_v"], d["wd"]).to(f32) + d["res2"].to(f32)).to(torch.bfloat16)
    return out


def pure_sites(torch, d, algo):
    """The pure GEMMs (no epilogue) at gate/up, down and o (activation
    packing included for the packed arms)."""
    import strassen_tpu_amd as smx

    bm, bn, bk = TILE
    if algo == "hipblaslt":
        fn = lambda a, b: torch.matmul(a, d[b])
    else:
        suffix, _ = ARM_WEIGHTS[algo]
        base = smx.cubic_matmul if algo.startswith("cubic") else smx.strassen_matmul
        fn = lambda a, b: base(a, d[b + suffix], bm=bm, bn=bn, bk=bk)
    return {
        "gate_up": lambda: fn(d["y"], "wup"),
        "down": lambda: fn(d["h_any"], "wd"),
        "o": lambda: fn(d["attn"], "wo"),
        # the whole gate|up weight (a column permutation of [gate | up]), no
        # epilogue: the shape of the reference's pure-GEMM confirmation run
        "gate_up_full": lambda: fn(d["y"], "wgu_laid"),
    }


def gate_up_gemm(d, algo):
    """The dominant kernel alone: the fused gate|up SwiGLU GEMM launch on an
    activation packed beforehand (algo 7 Strassen, 8 cubic)."""
    import strassen_tpu_amd as smx

    bm, bn, bk = TILE
    packed = smx.pack_activation(d["y"], algo, bm, bk)
    if algo == 7:
        return lambda: smx.strassen_matmul(packed, d["wgu_laid_sw"], bm=bm, bn=bn, bk=bk, epilogue="swiglu",
                                           interleave_products=True)
    return lambda: smx.cubic_matmul(packed, d["wgu_laid_cw"], bm=bm, bn=bn, bk=bk, epilogue="swiglu")


def head_columns(m, k, n, bn, cus):
    """Columns of an (m, k, n) Strassen call that the default kernel choice
    runs on the product-major kernel: its 128 x 256 product tiles in whole
    rounds of the CUs, ending on a bn tile boundary, and none below K = 4096
    (the library's pm_round_columns)."""
    if k < 4096:
        return 0
    tiles_m, tiles_n = (m // 2) // 128, (n // 2) // 256
    per_round = cus // math.gcd(tiles_m, cus)
    per_bn = (bn // 2) // 256
    step = per_round * per_bn // math.gcd(per_round, per_bn)
    return 2 * 256 * (tiles_n // step * step)


def gate_up_head_gemm(d, cus):
    """The dominant kernel alone: the product-major head of the fused gate|up
    SwiGLU call (the columns head_columns gives), on an activation packed
    beforehand. Returns (head columns, callable)."""
    import strassen_tpu_amd as smx
    from strassen_tpu_amd.packing import PackedOperand

    bm, bn, bk = TILE
    n = head_columns(TOKENS, HIDDEN, 2 * FFN, bn, cus)
    w = d["wgu_laid_sw"]
    # A packed weight's leading n columns are its first n/2 / 128 packed
    # tiles: (n/2) (K/2) seven operands of bf16.
    head = PackedOperand(w.data[:(n // 2) * (w.k // 2) * 7], algo=7, side="rhs", rows=n, k=w.k,
                         tile_rows=w.tile_rows, bk=w.bk)
    packed = smx.pack_activation(d["y"], 7, bm, bk)
    return n, lambda: smx.strassen_matmul(packed, head, bm=bm, bn=bn, bk=bk, epilogue="swiglu",
                                          interleave_products=True)


def full_block_times(torch, dev, steps, warmup):
    """Median ms of one whole Qwen3-32B decoder block (RMSNorms, q/k with
    fused qk_norm_rope, v on hipBLASLt, causal SDPA attention, o + residual,
    gate|up + SwiGLU, down + residual) per arm, same weights and input. The
    cubic_unfused arm is the cubic arm of the reference's published block
    run: cubic GEMMs for o, gate|up and down with torch epilogues, q, k and v
    on hipBLASLt with torch norms and RoPE."""
    from strassen_tpu_amd import qwen3_block as qb

    weights = qb.BlockWeights.random_init(qb.QWEN3_32B, dev, seed=1)
    x = torch.randn(TOKENS, HIDDEN, device=dev, generator=torch.Generator(device=dev).manual_seed(2))
    x = x.to(torch.bfloat16)
    out = {}
    for arm in qb.ARMS:
        log(f"timing full block, {arm} arm")
        block = qb.PreparedBlock(weights, qb.QWEN3_32B, arm, batch=BATCH, seq=SEQ, tile=TILE)
        _, ev = time_steps(torch, lambda: qb.block_forward(x, block), steps, warmup)
        out[arm] = statistics.median(ev)
        del block
    return out


def time_steps(torch, step, steps, warmup):
    """Warm up, then time exactly `steps` calls between two synchronisations.
    Returns (total wall ms, per-step event ms list)."""
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    t0 = time.perf_counter()
    for e0, e1 in events:
        e0.record()
        step()
        e1.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3
    return wall, [e0.elapsed_time(e1) for e0, e1 in events]


def run_block(sites):
    order = ("q", "k", "v", "o", "gate_up", "down")

    def step():
        for name in order:
            sites[name]()
    return step


def cpu_threads():
    """Host threads for the CPU baseline: the CPUs this process may run on,
    capped by OMP_NUM_THREADS when the environment sets a share."""
    n = len(os.sched_getaffinity(0))
    cap = os.environ.get("OMP_NUM_THREADS")
    if cap and cap.isdigit() and int(cap) > 0:
        n = min(n, int(cap))
    return max(n, 1)


def cpu_baseline(seconds):
    """The reference's Strassen path restated in torch on the host cores,
    at the reference's CPU-runnable configuration: A[1024,1024] ~ N(0,1),
    B[1024,1024] ~ N(0, 1/32), bf16, seed 0, tile (1024, 1024, 512).
    Warm-up, then alternating timed calls of the Strassen restatement and the
    FP32 cubic torch.matmul for about `seconds` in all."""
    import numpy as np
    import torch

    import oracle as o
    from oracle import strassen_torch_cpu as tc

    threads = cpu_threads()
    torch.set_num_threads(threads)
    rng = np.random.default_rng(0)
    a = torch.from_numpy(o.bf16_round(rng.standard_normal((1024, 1024)).astype(np.float32))).to(torch.bfloat16)
    b = torch.from_numpy(o.bf16_round((rng.standard_normal((1024, 1024)) / 32).astype(np.float32)))
    b = b.to(torch.bfloat16)
    a32, b32 = a.float(), b.float()
    bm, bn, bk = 1024, 1024, 512
    for _ in range(2):
        tc.strassen_matmul(a, b, bm=bm, bn=bn, bk=bk)
        torch.matmul(a32, b32)
    strassen_s, cubic_s = [], []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(strassen_s) < 3:
        t0 = time.perf_counter()
        tc.strassen_matmul(a, b, bm=bm, bn=bn, bk=bk)
        t1 = time.perf_counter()
        torch.matmul(a32, b32)
        t2 = time.perf_counter()
        strassen_s.append(t1 - t0)
        cubic_s.append(t2 - t1)
    flop = 2.0 * 1024 ** 3
    median = statistics.median(strassen_s)
    cpu_model = None
    try:
        with open("/proc/cpuinfo") as f:
            cpu_model = next((line.split(":", 1)[1].strip() for line in f if line.startswith("model name")), None)
    except OSError:
        pass
    ms = [x * 1e3 for x in strassen_s]
    return {
        "value": round(flop / median / 1e12, 5), "unit": "TFLOP/s", "cores": threads, "kind": "port",
        "sample": f"{len(strassen_s)} calls of the torch-CPU restatement of the reference Strassen path at "
                  "1024x1024x1024 (bf16, A~N(0,1), B~N(0,1/32), seed 0, tile 1024x1024x512), "
                  f"interleaved with FP32 torch.matmul, {sum(strassen_s) + sum(cubic_s):.1f} s",
        "ms_per_call": {"mean": round(statistics.mean(ms), 3), "median": round(statistics.median(ms), 3),
                        "std": round(statistics.stdev(ms), 3) if len(ms) > 1 else 0.0, "n": len(ms)},
        "cubic_fp32_matmul_tflops": round(flop / statistics.median(cubic_s) / 1e12, 5),
        "affinity_cpus": len(os.sched_getaffinity(0)),
        "cpu_model": cpu_model,
    }


def summary(samples):
    """mean / median / std (ms) of per-step event times."""
    return {"mean": round(statistics.mean(samples), 4), "median": round(statistics.median(samples), 4),
            "std": round(statistics.stdev(samples), 4) if len(samples) > 1 else 0.0, "n": len(samples)}


def paired_ci95(numerator, denominator):
    """Mean and 95% t-interval of the per-round ratios numerator_i /
    denominator_i (rounds paired: both arms timed back to back)."""
    ratios = [x / y for x, y in zip(numerator, denominator)]
    n = len(ratios)
    mean = statistics.mean(ratios)
    t975 = {2: 12.706, 3: 4.303, 4: 3.182, 5: 2.776, 6: 2.571, 7: 2.447, 8: 2.365}.get(n, 2.0)
    half = t975 * statistics.stdev(ratios) / n ** 0.5 if n > 1 else float("nan")
    return {"mean": round(mean, 4), "lo": round(mean - half, 4), "hi": round(mean + half, 4), "rounds": n}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only", default=None,
                    help="profiling runs: time only ARM:SITE (ARM strassen|cubic|strassen_plain|cubic_plain|"
                         "hipblaslt|strassen_split|strassen_product_major; SITE q|k|v|o|gate_up|down|pure_gate_up|pure_down|pure_o|pure_gate_up_full, gate_up_gemm "
                         "for the packed GEMM call alone, or gate_up_head for its product-major head alone), or \"copy\" (a 256 MiB copy, counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: the Strassen GEMM path runs on one MI355X "
              "(no collectives). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch

    import strassen_tpu_amd as smx  # noqa: F401  (loads the HIP library; fails loudly if missing)
    from strassen_tpu_amd import _lib

    _lib.load()
    dev = torch.device("cuda:0")
    torch.backends.cuda.matmul.allow_tf32 = False
    if args.only == "copy":
        # Counter calibration: one 256 MiB device-to-device copy per step.
        src = torch.ones(COPY_BYTES // 2, dtype=torch.bfloat16, device=dev)
        dst = torch.empty_like(src)
        _, ev = time_steps(torch, lambda: dst.copy_(src), args.steps, args.warmup)
        log(f"copy {COPY_BYTES >> 20} MiB: {statistics.mean(ev):.3f} ms/call")
        return
    log(f"device: {torch.cuda.get_device_name(0)}, CUs {torch.cuda.get_device_properties(0).multi_processor_count}")
    d = make_block(torch, dev)
    shapes = site_shapes()
    block_flops = sum(flops(s) for s in shapes.values())

    arms = {arm: fused_sites(torch, d, arm) for arm in ARM_WEIGHTS}
    arms["hipblaslt"] = vendor_sites(torch, d)
    # H for the pure down GEMM (any bf16 activations of the right shape).
    arms["strassen"]["gate_up"]()
    d["h_any"] = d["h"]
    arms["hipblaslt"]["gate_up"]()
    torch.cuda.synchronize()

    if args.only:
        arm, site = args.only.split(":")
        if arm in KERNEL_ARMS:
            with smx.strassen_kernel(KERNEL_ARMS[arm]):
                fn = arms["strassen"][site] if not site.startswith("pure_") else \
                    pure_sites(torch, d, "strassen")[site.replace("pure_", "")]
                _, ev = time_steps(torch, fn, args.steps, args.warmup)
            log(f"{args.only}: {statistics.mean(ev):.3f} ms/call")
            return
        if site == "gate_up_head":
            _, fn = gate_up_head_gemm(d, torch.cuda.get_device_properties(0).multi_processor_count)
            _, ev = time_steps(torch, fn, args.steps, args.warmup)
            log(f"{args.only}: {statistics.mean(ev):.3f} ms/call")
            return
        if site == "gate_up_gemm":
            fn = gate_up_gemm(d, 7 if arm == "strassen" else 8)
            _, ev = time_steps(torch, fn, args.steps, args.warmup)
            log(f"{args.only}: {statistics.mean(ev):.3f} ms/call")
            return
        table = arms[arm] if site in arms[arm] and not site.startswith("pure_") else \
            pure_sites(torch, d, arm)
        fn = table[site.replace("pure_", "")]
        wall, ev = time_steps(torch, fn, args.steps, args.warmup)
        log(f"{args.only}: {statistics.mean(ev):.3f} ms/call")
        return

    # Headline: exactly `steps` Strassen block steps between synchronisations.
    log("timing strassen block")
    wall_s, ev_s = time_steps(torch, run_block(arms["strassen"]), args.steps, args.warmup)
    results = {"strassen": statistics.median(ev_s)}
    stats = {"strassen": summary(ev_s)}
    for arm in ("cubic", "hipblaslt", "strassen_plain", "cubic_plain"):
        log(f"timing {arm} block")
        _, ev = time_steps(torch, run_block(arms[arm]), args.steps, args.warmup)
        results[arm] = statistics.median(ev)
        stats[arm] = summary(ev)
    # Interleaved rounds (rotated arm order) to check the comparison is not
    # an ordering artefact; the paired per-round ratios give the speedup CI.
    names = ["strassen", "cubic", "hipblaslt"]
    rounds = {a: [] for a in names}
    for r in range(5):
        order = names[r % 3:] + names[:r % 3]
        for arm in order:
            _, ev = time_steps(torch, run_block(arms[arm]), max(3, args.steps // 4), 1)
            rounds[arm].append(statistics.median(ev))

    # Per-site times (events on the launching stream) for every arm.
    per_site = {}
    for arm, sites in arms.items():
        per_site[arm] = {}
        for name in ("q", "k", "v", "o", "gate_up", "down"):
            _, ev = time_steps(torch, sites[name], args.steps, 2)
            per_site[arm][name] = statistics.median(ev)
    pure = {}
    for arm in ("strassen", "strassen_plain", "cubic", "cubic_plain", "hipblaslt"):
        table = pure_sites(torch, d, arm)
        pure[arm] = {}
        for name, fn in table.items():
            _, ev = time_steps(torch, fn, args.steps, 2)
            pure[arm][name] = statistics.median(ev)
    # The other Strassen kernels on the same packed weights: the split kernel
    # alone, and the product-major kernel on every tile (it does not take the
    # q/k epilogue: the q and k sites then run the split kernel).
    for kernel_arm, kind in KERNEL_ARMS.items():
        with smx.strassen_kernel(kind):
            per_site[kernel_arm] = {}
            for name in ("q", "k", "v", "o", "gate_up", "down"):
                _, ev = time_steps(torch, arms["strassen"][name], args.steps, 2)
                per_site[kernel_arm][name] = statistics.median(ev)
            pure[kernel_arm] = {}
            for name, fn in pure_sites(torch, d, "strassen").items():
                _, ev = time_steps(torch, fn, args.steps, 2)
                pure[kernel_arm][name] = statistics.median(ev)
    pure_shapes = {"gate_up": (TOKENS, HIDDEN, FFN), "down": (TOKENS, FFN, HIDDEN),
                   "o": (TOKENS, HEADS * HEAD_DIM, HIDDEN), "gate_up_full": (TOKENS, HIDDEN, 2 * FFN)}

    # Roofline of the dominant kernel: the product-major head of the fused
    # gate|up SwiGLU Strassen call (its whole rounds of 128 x 256 product
    # tiles) alone, activation already packed, timed with events on the
    # stream it is launched on. The whole call adds the split kernel's rest.
    bm, bn, bk = TILE
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    head_n, head_fn = gate_up_head_gemm(d, cus)
    head_tiles = (TOKENS // 2 // 128) * (head_n // 2 // 256)
    _, ev = time_steps(torch, head_fn, args.steps, 2)
    head_ms = statistics.mean(ev)
    head_tflops = 2.0 * TOKENS * HIDDEN * head_n / (head_ms * 1e-3) / 1e12
    _, ev = time_steps(torch, gate_up_gemm(d, 7), args.steps, 2)
    gu_ms = statistics.mean(ev)
    _, ev = time_steps(torch, gate_up_gemm(d, 8), args.steps, 2)
    gu_cubic_ms = statistics.mean(ev)
    _, ev = time_steps(torch, lambda: smx.pack_activation(d["y"], 7, bm, bk), args.steps, 2)
    pack_ms = statistics.mean(ev)
    traffic, traffic_note = None, None
    measured = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "gate_up_swiglu_qwen3_32b_traffic.json")
    if os.path.exists(measured):
        rec = json.load(open(measured))["strassen"]
        if rec.get("columns") == head_n:
            traffic = round(rec["traffic_bytes"])
            traffic_note = (f"L2-miss bytes per launch (reads and writes between the XCDs' L2 and the memory side, "
                            f"which the 256 MB MALL or HBM serves: rocprofv3 exposes no counter that tells them "
                            f"apart on this image) from rocprofv3 FETCH_SIZE/WRITE_SIZE passes scaled by a "
                            f"copy-kernel calibration (profiles/gemm_pm_strassen_swiglu_qwen3_32b_gate_up_head.md); "
                            f"algorithmic {rec['algorithmic_bytes']} B")
    roofline = {
        "bound": "mfma", "achieved": round(head_tflops, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
        "frac": round(head_tflops / PEAK_BF16_TFLOPS, 4), "traffic": traffic, "traffic_note": traffic_note,
        "kernel": f"smx::pm::gemm_pm<SMX_EPI_SWIGLU> (product-major Strassen): the head of the gate|up call, "
                  f"M=8192 K=5120 N={head_n} of 51200, {head_tiles} tiles of 128 x 256 product space "
                  f"({head_tiles // cus} whole rounds on {cus} CUs), packed operands",
        "mfma_executed_frac": round(head_tflops * 7 / 8 / PEAK_BF16_TFLOPS, 4),
        "avg_launch_ms": round(head_ms, 4),
        "gate_up_call_ms": round(gu_ms, 4),
        "gate_up_call_tflops": round(flops(shapes["gate_up"]) / (gu_ms * 1e-3) / 1e12, 2),
        "cubic_same_site_ms": round(gu_cubic_ms, 4),
        "activation_pack_ms": round(pack_ms, 4),
    }

    # The whole decoder block (norms, attention, v on hipBLASLt) per arm.
    full_block = full_block_times(torch, dev, args.steps, args.warmup)

    ms = results["strassen"]
    value = block_flops / (ms * 1e-3) / 1e12
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "wall_ms_per_step": round(wall_s / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init bf16 weights ~N(0,0.02), activations ~N(0,1))",
        "config": {
            "workload": "qwen3_32b_block_gemm_sites_fused",
            "tokens": TOKENS, "batch": BATCH, "seq": SEQ, "hidden": HIDDEN, "ffn": FFN,
            "heads": HEADS, "kv_heads": KV_HEADS, "head_dim": HEAD_DIM,
            "tile_bm_bn_bk": list(TILE), "block_tflop": round(block_flops / 1e12, 4),
            "sites": {k: list(v) for k, v in shapes.items()},
        },
        "arms_ms": {k: round(v, 4) for k, v in results.items()},
        "arms_stats_ms": stats,
        "arms_interleaved_ms": {k: [round(x, 4) for x in v] for k, v in rounds.items()},
        "speedup_vs_cubic": round(results["cubic"] / ms, 4),
        "speedup_vs_hipblaslt": round(results["hipblaslt"] / ms, 4),
        "speedup_vs_cubic_ci95": paired_ci95(rounds["cubic"], rounds["strassen"]),
        "speedup_vs_hipblaslt_ci95": paired_ci95(rounds["hipblaslt"], rounds["strassen"]),
        "sites_ms": {arm: {k: round(v, 4) for k, v in s.items()} for arm, s in per_site.items()},
        "sites_tflops": {arm: {k: round(flops(shapes[k]) / (v * 1e-3) / 1e12, 1) for k, v in s.items()}
                         for arm, s in per_site.items()},
        "pure_gemm_ms": {arm: {k: round(v, 4) for k, v in s.items()} for arm, s in pure.items()},
        "pure_gemm_tflops": {arm: {k: round(flops(pure_shapes[k]) / (v * 1e-3) / 1e12, 1) for k, v in s.items()}
                             for arm, s in pure.items()},
        # The reference's pure-GEMM confirmation shape, 8192 x 5120 x 51200
        # with no epilogue (strassen_qwen3_32b_v6e_pure_gemm.jsonl:17).
        "pure_gate_up_full_speedup": {"vs_cubic": round(pure["cubic"]["gate_up_full"] / pure["strassen"]["gate_up_full"], 4),
                                      "vs_hipblaslt": round(pure["hipblaslt"]["gate_up_full"]
                                                            / pure["strassen"]["gate_up_full"], 4)},
        "roofline": roofline,
        "full_block_ms": {k: round(v, 4) for k, v in full_block.items()},
        "full_block_speedup_vs_cubic": round(full_block["cubic"] / full_block["strassen"], 4),
        # The arm policy of the reference's published block comparison: its
        # cubic arm has no fused epilogues (benchmark_qwen3_32b_full_layer_
        # product_inference.py:63-76, :146-170).
        "full_block_speedup_vs_cubic_unfused": round(full_block["cubic_unfused"] / full_block["strassen"], 4),
        "weight_memory": weight_memory(d),
    }
    if not args.no_cpu_baseline:
        log("timing CPU baseline (oracle)")
        line["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
