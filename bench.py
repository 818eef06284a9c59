"""Benchmark of the NF4 frozen-weight path on one MI355X.

Default workload (the shape the throughput targets are quoted at): a LoRA
training step on an NF4 base, W [14336, 4096] (fp16 N(0, 0.02) source,
blocksize 64, dequantized to bf16), X bf16 [8192, 4096] N(0, 1), LoRA rank 16
(A, B bf16 N(0, 0.01), scale 1). One step = fused forward
Y = X.W^T + X.A^T.B^T and fused backward dX = dY.W (+ LoRA), plus the LoRA
weight gradients. ``value`` counts the two frozen-base GEMMs only
(2 x 2.M.N.K = 1924.1 GFLOP per step); the LoRA flops are reported apart.

Also measured, each with HIP events on the stream the kernels run on:
  * the fused forward kernel alone (the roofline line, dense-bf16 MFMA bound);
  * the NF4 dequantize kernel on the same W to bf16 (HBM bound, 2.5625 B/element);
  * the unfused path the reference uses (dequantize + torch.matmul);
  * the CPU oracle (C restatement, all host threads) on a bounded sample.

    python bench.py [--steps K] [--warmup W] [--workload lora_step|layer_stream]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "NF4 dequant GB/s (% HBM peak); fused NF4-GEMM TFLOP/s (% MFMA peak)"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
EV_EVERY = 3  # timed steps per sampled one (HIP events around its fused GEMM launches)


def seeded(torch, shape, seed, std, dtype, device):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * std).to(dtype).to(device)


def graph_time_ms(torch, fn, reps):
    """Average device time of fn() with the host taken out: reps launches are
    captured into one HIP graph (torch.cuda.graph), which is replayed and timed
    with events. For kernels of a few microseconds, where launching from Python
    costs more than the kernel."""
    fn()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()  # warm up on the capture stream (allocator pool, cached tables)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(reps):
            fn()
    g.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(3):
        g.replay()
    end.record()
    end.synchronize()
    ms = start.elapsed_time(end) / (3 * reps)
    del g
    return ms


def event_time_ms(torch, fn, reps):
    """Average duration of fn() over reps launches, timed with HIP events on the
    current stream (where the library launches its kernels)."""
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for _ in range(3):  # warm-up: library heuristics, allocator growth
        fn()
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(reps):
        fn()
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) / reps


def cpu_baseline(torch, w_half, N, K, sample_rows):
    """Oracle on the host: C-restatement dequantize of the whole W (all threads),
    then an fp32 torch matmul of `sample_rows` rows of X with it."""
    import numpy as np

    from oracle import c_oracle as C
    from oracle import nf4_oracle as O

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    wbits = w_half.cpu().view(torch.int16).numpy().view(np.uint16)
    packed, absmax = C.quantize(wbits, O.DT_F16, 64, "argmin", threads)
    n = N * K
    t0 = time.perf_counter()
    reps = 0
    while True:
        wd = C.dequantize(packed, absmax, n, 64, O.DT_BF16, threads)
        reps += 1
        if time.perf_counter() - t0 > 3.0:
            break
    deq_s = (time.perf_counter() - t0) / reps
    w32 = torch.from_numpy(wd.view(np.int16).reshape(N, K)).view(torch.bfloat16).float()
    x = torch.randn(sample_rows, K)
    t0 = time.perf_counter()
    y = x @ w32.t()
    mm_s = time.perf_counter() - t0
    del y
    flops = 2.0 * sample_rows * N * K
    # vectorised torch on the same cores: the reference's own CPU formulation
    tp, ta = torch.from_numpy(packed), torch.from_numpy(absmax)
    tdeq_s, wt = _timed_loop(lambda: _torch_cpu_dequantize(tp, ta, torch.bfloat16), 3.0)
    if not torch.equal(wt.view(torch.int16), torch.from_numpy(wd.view(np.int16))):
        raise RuntimeError("torch CPU dequantize disagrees with the oracle")
    torch_leg = {"value": round(flops / (tdeq_s + mm_s) / 1e12, 4), "unit": "TFLOP/s",
                 "what": "vectorised torch dequantize of W (bit-identical to the oracle's) + the same matmul",
                 "dequant_gbs": round(2.5625 * n / tdeq_s / 1e9, 3)}
    return {
        "value": round(flops / (deq_s + mm_s) / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"oracle C dequantize of W [{N},{K}] to bf16 + fp32 torch matmul of {sample_rows} "
                   f"rows of X (of 8192)"),
        "dequant_gbs": round(2.5625 * n / deq_s / 1e9, 3),
        "cpu_model": _cpu_model(),
        "torch_vectorised": torch_leg,
    }


def _torch_cpu_quantize(w, blocksize=64, chunk=1 << 20):
    """bitsandbytes' CPU quantize_4bit restated in vectorised torch (the path
    the reference runs at staging time, stratum/upload.py:360-369): blockwise
    absmax, s = x * (1 / absmax) in fp32, the nearest level by argmin (first
    index on ties), two codes per byte (even element in the high nibble)."""
    import torch
    from stratum_amd.functional import NF4_LEVELS
    code = torch.tensor(NF4_LEVELS, dtype=torch.float32)
    xf = w.reshape(-1, blocksize).float()
    absmax = xf.abs().amax(1)
    s = (xf * (1.0 / absmax).unsqueeze(1)).reshape(-1)
    codes = torch.empty(s.numel(), dtype=torch.uint8)
    for i in range(0, s.numel(), chunk):
        codes[i:i + chunk] = (s[i:i + chunk, None] - code).abs().argmin(1).to(torch.uint8)
    pairs = codes.view(-1, 2)
    return (pairs[:, 0] << 4) | pairs[:, 1], absmax


def _torch_cpu_dequantize(packed, absmax, dtype, blocksize=64):
    """bitsandbytes' CPU dequantize_4bit restated in vectorised torch: level *
    absmax in fp32, one rounding to dtype."""
    import torch
    from stratum_amd.functional import NF4_LEVELS
    code = torch.tensor(NF4_LEVELS, dtype=torch.float32)
    vals = torch.stack([code[(packed >> 4).long()], code[(packed & 15).long()]], 1).reshape(-1, blocksize)
    return (vals * absmax.unsqueeze(1)).reshape(-1).to(dtype)


def _timed_loop(fn, seconds):
    t0 = time.perf_counter()
    reps = 0
    while True:
        out = fn()
        reps += 1
        if time.perf_counter() - t0 > seconds:
            return (time.perf_counter() - t0) / reps, out


def _profiled_traffic():
    """HBM bytes per launch from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
    summary of this workload (calibrated against a 1 GiB elementwise kernel)."""
    path = os.path.join(ROOT, "profiles", "traffic_lora_step_w14336x4096_x8192.json")
    try:
        with open(path) as f:
            d = json.load(f)
        return {k: v["read_bytes"] + v["write_bytes"] for k, v in d["kernels"].items()}
    except (OSError, KeyError, ValueError):
        return {}


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _forced_fused(fn):
    """fn() with the fused kernels forced at every row count."""
    policy = os.environ.get("STRATUM_NF4_FUSED_MAX_ROWS")
    os.environ["STRATUM_NF4_FUSED_MAX_ROWS"] = "-1"
    try:
        return fn()
    finally:
        if policy is None:
            del os.environ["STRATUM_NF4_FUSED_MAX_ROWS"]
        else:
            os.environ["STRATUM_NF4_FUSED_MAX_ROWS"] = policy


def check_step_output(torch, step_once, x, A, B, dy, w):
    """One untimed run of the timed step, its y, dX, dA and dB against fp32
    torch on the dequantized weight (relative Frobenius error, bf16 bar 1e-2).
    Raises if any is off: a throughput of wrong results is not reported."""
    x.grad = A.grad = B.grad = None
    y = step_once()
    y.backward(dy)
    got = {"y": y.detach(), "dX": x.grad, "dA": A.grad, "dB": B.grad}
    xr = x.detach().float().requires_grad_(True)
    Ar = A.detach().float().requires_grad_(True)
    Br = B.detach().float().requires_grad_(True)
    yr = xr @ w.float().t().contiguous() + (xr @ Ar.t().contiguous()) @ Br.t().contiguous()
    yr.backward(dy.float())
    ref = {"y": yr.detach(), "dX": xr.grad, "dA": Ar.grad, "dB": Br.grad}
    rel = {k: ((got[k].float() - ref[k]).norm() / ref[k].norm()).item() for k in got}
    x.grad = A.grad = B.grad = None
    del y, yr, got, ref
    torch.cuda.empty_cache()
    bad = {k: v for k, v in rel.items() if not v <= 1e-2}
    if bad:
        raise SystemExit(f"bench: the timed step's output is off the fp32 reference: {bad}")
    return {"rel_err": {k: float(f"{v:.3e}") for k, v in rel.items()}, "tol": 1e-2,
            "what": "one untimed run of the timed step (fused kernels forced) against fp32 torch on the "
                    "dequantized weight"}


def run_lora_step(args):
    import torch

    from stratum_amd.functional import dequantize_4bit, nf4_gemm_bwd_dx, nf4_gemm_fwd, quantize_4bit
    from stratum_amd.nf4_linear import nf4_linear

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    N, K, M, R = 14336, 4096, 8192, 16
    w = seeded(torch, (N, K), 0, 0.02, torch.float16, dev)
    packed, state = quantize_4bit(w)
    state.dtype = torch.bfloat16
    absmax = state.absmax
    x = seeded(torch, (M, K), 1, 1.0, torch.bfloat16, dev).requires_grad_(True)
    A = seeded(torch, (R, K), 2, 0.01, torch.bfloat16, dev).requires_grad_(True)
    B = seeded(torch, (N, R), 3, 0.01, torch.bfloat16, dev).requires_grad_(True)
    dy = seeded(torch, (M, N), 4, 1.0, torch.bfloat16, dev)

    def step():
        y = nf4_linear(x, packed, state, None, A, B, 1.0)
        y.backward(dy)
        x.grad = None
        A.grad = None
        B.grad = None

    # every EV_EVERY-th timed step (from the first) is a sampled one: its fused GEMM
    # launches are bracketed by HIP events (see below)
    sampled = {"on": False}

    def timed_steps(n):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(n):
            sampled["on"] = i % EV_EVERY == 0
            step()
        sampled["on"] = False
        torch.cuda.synchronize()
        return time.perf_counter() - t0

    # The headline measures the fused dequant-GEMMs (forced for every row count);
    # the library default for this M (dequantize + hipBLASLt) is reported beside it.
    # During the sampled timed steps each fused GEMM launch is bracketed by HIP
    # events on the stream it is launched on: the roofline's kernel duration is the
    # mean over those launches of the timed region itself. Only every EV_EVERY-th
    # step is sampled because each timing event holds the next launch back by
    # about 5 us (four per step cost 0.8 % of the step, A/B-timed).
    import importlib
    NL = importlib.import_module("stratum_amd.nf4_linear")  # the package also exports a function of that name
    spans = {"fwd": [], "bwd": []}

    def bracketed(fn, key):
        def call(*a, **kw):
            if not sampled["on"]:
                return fn(*a, **kw)
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
            out = fn(*a, **kw)
            end.record()
            spans[key].append((start, end))
            return out
        return call

    policy = os.environ.get("STRATUM_NF4_FUSED_MAX_ROWS")
    os.environ["STRATUM_NF4_FUSED_MAX_ROWS"] = "-1"
    try:
        for _ in range(args.warmup):
            step()
        NL.nf4_gemm_fwd, NL.nf4_gemm_bwd_dx = bracketed(nf4_gemm_fwd, "fwd"), bracketed(nf4_gemm_bwd_dx, "bwd")
        try:
            elapsed = timed_steps(args.steps)
        finally:
            NL.nf4_gemm_fwd, NL.nf4_gemm_bwd_dx = nf4_gemm_fwd, nf4_gemm_bwd_dx
    finally:
        if policy is None:
            del os.environ["STRATUM_NF4_FUSED_MAX_ROWS"]
        else:
            os.environ["STRATUM_NF4_FUSED_MAX_ROWS"] = policy
    # each side measurement gets warm-up steps of its own: the first steps after
    # a switch of path run 10-15 % slow (allocator growth for the temporary
    # weight), which one warm-up step does not absorb
    side_warmup, side_steps = max(5, args.warmup), max(10, args.steps // 3)
    for _ in range(side_warmup):
        step()
    default_ms = timed_steps(side_steps) * 1e3 / side_steps

    # the reference's architecture for the same work: the frozen weight is
    # dequantized for the forward (ensure_weights), freed after it, and
    # dequantized again for the backward; the frozen F.linear and a PEFT LoRA
    # (lora_B(lora_A(x)) * scaling) run in torch; autograd takes dX, dA, dB
    import torch.nn.functional as F

    class _ReferenceFrozenLinear(torch.autograd.Function):
        @staticmethod
        def forward(ctx, inp):
            return F.linear(inp, dequantize_4bit(packed, state))

        @staticmethod
        def backward(ctx, gy):
            return gy @ dequantize_4bit(packed, state)

    def reference_step():
        y = _ReferenceFrozenLinear.apply(x) + F.linear(F.linear(x, A), B) * 1.0
        y.backward(dy)
        x.grad = None
        A.grad = None
        B.grad = None

    for _ in range(side_warmup):
        reference_step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(side_steps):
        reference_step()
    torch.cuda.synchronize()
    ref_ms = (time.perf_counter() - t0) * 1e3 / side_steps
    ms = elapsed * 1e3 / args.steps
    output_check = check_step_output(torch, step_once=lambda: _forced_fused(lambda: nf4_linear(x, packed, state, None,
                                                                                               A, B, 1.0)),
                                     x=x, A=A, B=B, dy=dy, w=dequantize_4bit(packed, state))
    base_flops = 2 * 2.0 * M * N * K
    lora_flops = 2.0 * M * K * R + 2.0 * M * R * N           # forward rank-16 path
    lora_flops += 2.0 * M * N * R + 2.0 * M * R * K          # dX rank-16 term
    lora_flops += 2.0 * R * M * K + 2.0 * N * M * R          # dA, dB
    value = base_flops / (elapsed / args.steps) / 1e12

    xd = x.detach()
    reps = max(5, args.kernel_reps)
    n_sampled = (args.steps + EV_EVERY - 1) // EV_EVERY
    assert len(spans["fwd"]) == len(spans["bwd"]) == n_sampled, {k: len(v) for k, v in spans.items()}
    fwd_ms = sum(a.elapsed_time(b) for a, b in spans["fwd"]) / n_sampled
    bwd_ms = sum(a.elapsed_time(b) for a, b in spans["bwd"]) / n_sampled
    gemm_flops = 2.0 * M * N * K
    fwd_tf = gemm_flops / (fwd_ms * 1e-3) / 1e12
    bwd_tf = gemm_flops / (bwd_ms * 1e-3) / 1e12

    out = torch.empty((N, K), dtype=torch.bfloat16, device=dev)
    deq_ms = event_time_ms(torch, lambda: dequantize_4bit(packed, state, out=out), reps * 4)
    deq_bytes = 2.5625 * N * K
    deq_gbs = deq_bytes / (deq_ms * 1e-3) / 1e9

    def unfused():
        wt = dequantize_4bit(packed, state, out=out)
        return xd @ wt.t()

    unf_ms = event_time_ms(torch, unfused, reps)

    # fp16, the reference's production training dtype: the same GEMMs
    x16, dy16 = xd.half(), dy.half()
    out16 = torch.empty((N, K), dtype=torch.float16, device=dev)
    fwd16_ms = event_time_ms(torch, lambda: nf4_gemm_fwd(x16, packed, absmax, (N, K), 64), reps)
    bwd16_ms = event_time_ms(torch, lambda: nf4_gemm_bwd_dx(dy16, packed, absmax, (N, K), 64), reps)

    def unfused16():
        state.dtype = torch.float16
        wt = dequantize_4bit(packed, state, out=out16)
        state.dtype = torch.bfloat16
        return x16 @ wt.t()

    unf16_ms = event_time_ms(torch, unfused16, reps)
    del x16, dy16, out16
    fp16 = {"fwd": {"kernel": "k_gemm_fwd_rw<F16>", "tflops": round(gemm_flops / (fwd16_ms * 1e-3) / 1e12, 2),
                    "frac": round(gemm_flops / (fwd16_ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
                    "avg_kernel_ms": round(fwd16_ms, 4)},
            "bwd_dx": {"kernel": "k_gemm_bwd_rw<F16>", "tflops": round(gemm_flops / (bwd16_ms * 1e-3) / 1e12, 2),
                       "frac": round(gemm_flops / (bwd16_ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
                       "avg_kernel_ms": round(bwd16_ms, 4)},
            "unfused_fwd": {"what": "dequantize kernel + torch.matmul (hipBLASLt), fp16",
                            "tflops": round(gemm_flops / (unf16_ms * 1e-3) / 1e12, 2), "ms": round(unf16_ms, 4)},
            "peak_note": "fp16 dense MFMA peak is the same 2.5 PFLOP/s as bf16"}
    traffic = _profiled_traffic()
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,0.02) fp16 weight quantized to NF4, N(0,1) bf16 activations)",
        "config": {"workload": "lora_step_nf4_w14336x4096_x8192", "M": M, "N": N, "K": K, "lora_rank": R,
                   "blocksize": 64, "parallelism": "single-gpu"},
        "roofline": {"bound": "mfma", "kernel": "k_gemm_fwd_rw<BF16>", "achieved": round(fwd_tf, 2),
                     "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(fwd_tf / MFMA_BF16_PEAK_TFLOPS, 4), "traffic": traffic.get("k_gemm_fwd_rw"),
                     "traffic_source": "profiles/traffic_lora_step_w14336x4096_x8192.json (rocprofv3 "
                                       "FETCH_SIZE + WRITE_SIZE per launch, calibrated; not measured in this run)",
                     "avg_kernel_ms": round(fwd_ms, 4), "flops_per_launch": gemm_flops,
                     "timing": f"HIP events around each launch on its stream, mean over one timed step in "
                               f"{EV_EVERY} ({n_sampled} of {args.steps}, from the first)"},
        "bwd_dx": {"kernel": "k_gemm_bwd_rw<BF16>", "achieved": round(bwd_tf, 2), "unit": "TFLOP/s",
                   "frac": round(bwd_tf / MFMA_BF16_PEAK_TFLOPS, 4), "avg_kernel_ms": round(bwd_ms, 4)},
        "dequant": {"kernel": "k_dequantize<BF16>", "value": round(deq_gbs, 1), "unit": "GB/s",
                    "frac": round(deq_gbs / HBM_PEAK_GBS, 4), "peak": HBM_PEAK_GBS,
                    "avg_kernel_ms": round(deq_ms, 4), "bytes_per_launch": deq_bytes,
                    "traffic": traffic.get("k_dequantize")},
        "unfused_fwd": {"what": "dequantize kernel + torch.matmul (hipBLASLt)",
                        "tflops": round(gemm_flops / (unf_ms * 1e-3) / 1e12, 2), "ms": round(unf_ms, 4)},
        "output_check": output_check,
        "default_policy_step": {"what": "NF4LoRALinear default above 1024 rows: dequantize + hipBLASLt, "
                                        "the backward reuses the forward's dequantized temporary",
                                "ms_per_step": round(default_ms, 4),
                                "tflops": round(base_flops / (default_ms * 1e-3) / 1e12, 2)},
        "reference_architecture_step": {"what": "dequantize for the forward and again for the backward, torch "
                                                "F.linear + PEFT-style LoRA, autograd backward",
                                        "ms_per_step": round(ref_ms, 4),
                                        "tflops": round(base_flops / (ref_ms * 1e-3) / 1e12, 2),
                                        "fused_speedup": round(ref_ms / ms, 3)},
        "lora_gflop_per_step": round(lora_flops / 1e9, 2),
        "fp16": fp16,
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(torch, w, N, K, args.cpu_rows)
    if not args.main_only:
        del x, A, B, dy, out, w
        torch.cuda.empty_cache()
        line["configs"] = {name: fn(torch, args) for name, fn in SECONDARY_CONFIGS.items()}
    return line


# ---------------------------------------------------------------- other configs
def _gpu_quantized(torch, shape, seed, dev):
    """fp16 N(0, 0.02) weight generated on the GPU and quantized there."""
    from stratum_amd.functional import quantize_4bit
    g = torch.Generator(device=dev).manual_seed(seed)
    w = (torch.randn(*shape, generator=g, device=dev) * 0.02).half()
    packed, state = quantize_4bit(w.reshape(-1, shape[-1]))
    del w
    return packed, state


def run_roundtrip(torch, args):
    """fp16 [5632, 2048] N(0, 0.02): GPU quantize + dequantize vs the C oracle on the host."""
    import numpy as np

    from stratum_amd.functional import dequantize_4bit, quantize_4bit
    dev = torch.device("cuda:0")
    w = seeded(torch, (5632, 2048), 0, 0.02, torch.float16, dev)
    n = w.numel()
    packed, state = quantize_4bit(w)
    out = torch.empty_like(w)
    q_ms = graph_time_ms(torch, lambda: quantize_4bit(w), 50)
    d_ms = graph_time_ms(torch, lambda: dequantize_4bit(packed, state, out=out), 50)
    q_call_ms = event_time_ms(torch, lambda: quantize_4bit(w), 50)
    byt = 2.5625 * n
    res = {"shape": [5632, 2048], "quantize_gbs": round(byt / q_ms / 1e6, 1), "quantize_us": round(q_ms * 1e3, 2),
           "dequantize_gbs": round(byt / d_ms / 1e6, 1), "dequantize_us": round(d_ms * 1e3, 2),
           "timing": "device time: 50 launches captured in one HIP graph, replayed",
           "quantize_call_us_from_python": round(q_call_ms * 1e3, 2),
           "aggregate": _roundtrip_aggregate(torch, dev)}
    if not args.no_cpu:
        from oracle import c_oracle as C
        from oracle import nf4_oracle as O
        threads = os.cpu_count() or 1
        bits = w.cpu().view(torch.int16).numpy().view(np.uint16)
        t0 = time.perf_counter()
        reps = 0
        while time.perf_counter() - t0 < 2.0:
            p_, a_ = C.quantize(bits, O.DT_F16, 64, "argmin", threads)
            C.dequantize(p_, a_, n, 64, O.DT_F16, threads)
            reps += 1
        cpu_s = (time.perf_counter() - t0) / reps
        res["cpu_roundtrip_ms"] = round(cpu_s * 1e3, 2)
        res["cpu_threads"] = threads
        torch.set_num_threads(threads)
        wc = w.cpu()
        tq_s, (tp, ta) = _timed_loop(lambda: _torch_cpu_quantize(wc), 2.0)
        td_s, _ = _timed_loop(lambda: _torch_cpu_dequantize(tp, ta, torch.float16), 1.0)
        if not (np.array_equal(tp.numpy(), p_) and np.array_equal(ta.numpy(), a_)):
            raise RuntimeError("torch CPU quantize disagrees with the oracle")
        res["torch_cpu_roundtrip_ms"] = round((tq_s + td_s) * 1e3, 2)
        res["gpu_roundtrip_ms"] = round(q_ms + d_ms, 4)
    return res


def _roundtrip_aggregate(torch, dev):
    """The matrices of one TinyLlama-1.1B decoder layer (q/o [2048,2048], k/v
    [256,2048], gate/up [5632,2048], down [2048,5632]; fp16 N(0, 0.02)) quantized
    and dequantized in one batched launch each, against one launch per matrix."""
    from stratum_amd.functional import dequantize_4bit, dequantize_4bit_many, quantize_4bit, quantize_4bit_many
    shapes = [(2048, 2048), (256, 2048), (256, 2048), (2048, 2048), (5632, 2048), (5632, 2048), (2048, 5632)]
    ws = [seeded(torch, sh, 60 + i, 0.02, torch.float16, dev) for i, sh in enumerate(shapes)]
    qs = quantize_4bit_many(ws)
    outs = [torch.empty_like(w) for w in ws]
    n = sum(w.numel() for w in ws)
    byt = 2.5625 * n

    def per_matrix_q():
        for w in ws:
            quantize_4bit(w)

    def per_matrix_d():
        for (p, st), o in zip(qs, outs):
            dequantize_4bit(p, st, out=o)

    qm = graph_time_ms(torch, lambda: quantize_4bit_many(ws), 20)
    dm = graph_time_ms(torch, lambda: dequantize_4bit_many(qs, out=outs), 20)
    q1 = graph_time_ms(torch, per_matrix_q, 20)
    d1 = graph_time_ms(torch, per_matrix_d, 20)
    return {"tensors": len(ws), "elements": n,
            "quantize_many_us": round(qm * 1e3, 2), "quantize_many_gbs": round(byt / qm / 1e6, 1),
            "dequantize_many_us": round(dm * 1e3, 2), "dequantize_many_gbs": round(byt / dm / 1e6, 1),
            "one_launch_per_matrix": {"quantize_us": round(q1 * 1e3, 2), "dequantize_us": round(d1 * 1e3, 2)}}


def run_qwen06(torch, args):
    """Qwen3-0.6B layer projections at M = 4096 tokens: fused NF4 forward, and
    beside it dequantize + hipBLASLt per projection (the reference's
    architecture, bitsandbytes dequantize then a cuBLAS matmul)."""
    from stratum_amd.functional import dequantize_4bit, nf4_gemm_fwd, stack_nf4
    dev = torch.device("cuda:0")
    M = 4096
    shapes = {"q": (2048, 1024), "k": (1024, 1024), "v": (1024, 1024), "o": (1024, 2048),
              "gate": (3072, 1024), "up": (3072, 1024), "down": (1024, 3072)}
    ws = {k: _gpu_quantized(torch, s, i, dev) for i, (k, s) in enumerate(shapes.items())}
    xs = {K: seeded(torch, (M, K), 100 + K, 1.0, torch.bfloat16, dev) for K in {s[1] for s in shapes.values()}}

    outs = {k: torch.empty((M, N), dtype=torch.bfloat16, device=dev) for k, (N, K) in shapes.items()}
    dense = {k: torch.empty(s, dtype=torch.bfloat16, device=dev) for k, s in shapes.items()}

    def layer():
        for k, (N, K) in shapes.items():
            p, st = ws[k]
            nf4_gemm_fwd(xs[K], p, st.absmax, (N, K), 64, out=outs[k])

    def library():  # the reference's architecture: dequantize each weight, then a plain matmul
        for k, (N, K) in shapes.items():
            p, st = ws[k]
            st.dtype = torch.bfloat16
            torch.matmul(xs[K], dequantize_4bit(p, st, out=dense[k]).t(), out=outs[k])

    # the projections that read the same input stacked into one NF4 weight
    # each (q|k|v, gate|up: payload bytes back to back, stack_nf4), so the
    # layer is 4 GEMMs; the outputs are column slices of the stacked results
    groups = {"qkv": ["q", "k", "v"], "o": ["o"], "gate_up": ["gate", "up"], "down": ["down"]}
    stacked = {g: stack_nf4([ws[k] for k in ks]) if len(ks) > 1 else ws[ks[0]] for g, ks in groups.items()}
    sshape = {g: (sum(shapes[k][0] for k in ks), shapes[ks[0]][1]) for g, ks in groups.items()}
    souts = {g: torch.empty((M, n), dtype=torch.bfloat16, device=dev) for g, (n, _) in sshape.items()}
    sdense = {g: torch.empty(sh, dtype=torch.bfloat16, device=dev) for g, sh in sshape.items()}

    def layer_stacked():
        for g, (N, K) in sshape.items():
            p, st = stacked[g]
            nf4_gemm_fwd(xs[K], p, st.absmax, (N, K), 64, out=souts[g])

    def library_stacked():
        for g, (N, K) in sshape.items():
            p, st = stacked[g]
            st.dtype = torch.bfloat16
            torch.matmul(xs[K], dequantize_4bit(p, st, out=sdense[g]).t(), out=souts[g])

    ms = event_time_ms(torch, layer, 20)
    lib_ms = event_time_ms(torch, library, 20)
    sms = event_time_ms(torch, layer_stacked, 20)
    slib_ms = event_time_ms(torch, library_stacked, 20)
    flops = sum(2.0 * M * N * K for N, K in shapes.values())
    return {"tokens": M, "layer_ms": round(ms, 4), "tflops": round(flops / ms / 1e9, 1),
            "gflop_per_layer": round(flops / 1e9, 2),
            "dequantize_plus_hipblaslt": {"layer_ms": round(lib_ms, 4), "tflops": round(flops / lib_ms / 1e9, 1)},
            "fused_speedup": round(lib_ms / ms, 3),
            "stacked_qkv_gate_up": {"what": "q|k|v and gate|up as one NF4 weight each: 4 GEMMs per layer",
                                    "fused_layer_ms": round(sms, 4), "fused_tflops": round(flops / sms / 1e9, 1),
                                    "dequantize_plus_hipblaslt_layer_ms": round(slib_ms, 4),
                                    "fused_vs_reference_architecture": round(lib_ms / sms, 3)}}


def run_layer_stream(torch, args):
    """8B-class decoder layers (q/o 4096x4096, k/v 1024x4096, gate/up 14336x4096,
    down 4096x14336) streamed from pinned host payloads: H2D alone, dequantize
    alone, serial (upload then dequantize per layer, one stream) and overlapped
    (NF4LayerStream: copy stream + dequant stream)."""
    import torch.nn as nn

    from stratum_amd.functional import dequantize_4bit
    from stratum_amd.stream import NF4LayerStream
    from stratum_amd.upload import NF4_ATTR, NF4Payload, _pin_cpu, ensure_weights, free_weights
    dev = torch.device("cuda:0")
    shapes = {"q": (4096, 4096), "k": (1024, 4096), "v": (1024, 4096), "o": (4096, 4096),
              "gate": (14336, 4096), "up": (14336, 4096), "down": (4096, 14336)}
    layers = []
    for li in range(args.layers):
        m = nn.Module()
        for j, (name, shp) in enumerate(shapes.items()):
            packed, st = _gpu_quantized(torch, shp, 1000 * li + j, dev)
            p = nn.Parameter(torch.empty(0, dtype=torch.float16), requires_grad=False)
            setattr(p, NF4_ATTR, NF4Payload(quantized=_pin_cpu(packed), absmax=_pin_cpu(st.absmax),
                                            code=_pin_cpu(st.code), shape=shp, dtype=torch.float16, blocksize=64,
                                            quant_type="nf4", source_numel=shp[0] * shp[1],
                                            source_bytes=2 * shp[0] * shp[1],
                                            payload_bytes=packed.numel() + 4 * st.absmax.numel() + 64))
            m.register_parameter(name, p)
        layers.append(m)
    payload = sum(getattr(p, NF4_ATTR).quantized.numel() + 4 * getattr(p, NF4_ATTR).absmax.numel()
                  for p in layers[0].parameters())
    elems = sum(a * b for a, b in shapes.values())
    L = len(layers)

    def timed(fn):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        fn()
        torch.cuda.synchronize()
        return time.perf_counter() - t0

    dev_payloads = [[(getattr(p, NF4_ATTR).quantized.to(dev), getattr(p, NF4_ATTR).absmax.to(dev))
                     for p in m.parameters()] for m in layers[:2]]

    def h2d_only():
        for m in layers:
            for p in m.parameters():
                pay = getattr(p, NF4_ATTR)
                pay.quantized.to(dev, non_blocking=True)
                pay.absmax.to(dev, non_blocking=True)

    outs = {name: torch.empty(shp, dtype=torch.float16, device=dev) for name, shp in shapes.items()}

    def deq_only():
        for li in range(L):
            for (q, a), (name, shp) in zip(dev_payloads[li % 2], shapes.items()):
                dequantize_4bit(q, absmax=a, shape=shp, blocksize=64, dtype=torch.float16, out=outs[name])

    def serial():
        for m in layers:
            ensure_weights(m, 0)
            free_weights(m)

    def overlapped():
        for _i, _m in NF4LayerStream(layers, 0, lookahead=1):
            pass

    serial()
    overlapped()
    t_h2d = min(timed(h2d_only) for _ in range(2))
    t_deq = min(timed(deq_only) for _ in range(2))
    t_ser = min(timed(serial) for _ in range(2))
    t_ovl = min(timed(overlapped) for _ in range(2))
    return {"layers": L, "payload_mb_per_layer": round(payload / 1e6, 1),
            "h2d_gbs": round(payload * L / t_h2d / 1e9, 2),
            "dequant_gbs": round(2.5625 * elems * L / t_deq / 1e9, 1),
            "serial_ms": round(t_ser * 1e3, 2), "overlapped_ms": round(t_ovl * 1e3, 2),
            "h2d_ms": round(t_h2d * 1e3, 2), "dequant_ms": round(t_deq * 1e3, 2),
            "overlap_efficiency": round(t_ser / t_ovl, 3),
            "overlapped_vs_h2d_bound": round(t_h2d / t_ovl, 3)}


def run_moe(torch, args):
    """Qwen3-30B-A3B-like expert bank: 128 experts, gate_up [1536, 2048] and
    down [2048, 768] in NF4; 8192 tokens, top-8 of softmax(N(0,1) logits).
    Fused grouped GEMMs against dequantize + a per-expert matmul loop; and the
    same layer at a decode size (16 tokens)."""
    from stratum_amd.functional import dequantize_4bit, nf4_grouped_gemm
    dev = torch.device("cuda:0")
    E, H, I, T, TOPK = 128, 2048, 768, 8192, 8
    gu_p, gu_s = _gpu_quantized(torch, (E, 2 * I, H), 7, dev)
    dn_p, dn_s = _gpu_quantized(torch, (E, H, I), 8, dev)
    g = torch.Generator(device=dev).manual_seed(9)
    logits = torch.randn(T, E, generator=g, device=dev)
    top = torch.topk(torch.softmax(logits, -1), TOPK, dim=-1).indices.reshape(-1)
    counts = torch.bincount(top, minlength=E)
    offsets = torch.zeros(E + 1, dtype=torch.int32, device=dev)
    offsets[1:] = torch.cumsum(counts, 0).to(torch.int32)
    rows = int(offsets[-1].item())
    max_rows = int(counts.max().item())
    x = seeded(torch, (rows, H), 10, 1.0, torch.bfloat16, dev)
    h = seeded(torch, (rows, I), 11, 1.0, torch.bfloat16, dev)

    offsets = offsets.cpu()  # the host copy: validated and uploaded per call without a device sync
    y_gu = torch.empty((rows, 2 * I), dtype=torch.bfloat16, device=dev)
    y_dn = torch.empty((rows, H), dtype=torch.bfloat16, device=dev)

    def layer():
        nf4_grouped_gemm(x, gu_p, gu_s.absmax, offsets, (2 * I, H), 64, max_rows=max_rows, out=y_gu)
        nf4_grouped_gemm(h, dn_p, dn_s.absmax, offsets, (H, I), 64, max_rows=max_rows, out=y_dn)

    # the reference's architecture: the staged bank is dequantized whole, then
    # the experts run one F.linear each per projection (transformers'
    # Qwen3MoeExperts loop over the experts that received tokens)
    bounds = offsets.tolist()
    hit = [e for e in range(E) if bounds[e + 1] > bounds[e]]
    gu_s.dtype = dn_s.dtype = torch.bfloat16
    gu_w = torch.empty((E * 2 * I, H), dtype=torch.bfloat16, device=dev)
    dn_w = torch.empty((E * H, I), dtype=torch.bfloat16, device=dev)

    def expert_loop(gu, dn):
        for e in hit:
            r0, r1 = bounds[e], bounds[e + 1]
            torch.matmul(x[r0:r1], gu[e * 2 * I:(e + 1) * 2 * I].t(), out=y_gu[r0:r1])
            torch.matmul(h[r0:r1], dn[e * H:(e + 1) * H].t(), out=y_dn[r0:r1])

    def library():
        expert_loop(dequantize_4bit(gu_p, gu_s, out=gu_w), dequantize_4bit(dn_p, dn_s, out=dn_w))

    ms = event_time_ms(torch, layer, 20)
    lib_ms = event_time_ms(torch, library, 10)
    loop_ms = event_time_ms(torch, lambda: expert_loop(gu_w, dn_w), 10)
    flops = 2.0 * rows * (2 * I * H + H * I)

    # decode size: the first 16 tokens' routing (at most a few rows per expert:
    # the grouped weight-streaming kernel), against the tile path pinned
    from stratum_amd import _lib
    TD = 16
    cd = torch.bincount(top.reshape(T, TOPK)[:TD].reshape(-1), minlength=E)
    off_d = torch.zeros(E + 1, dtype=torch.int32)
    off_d[1:] = torch.cumsum(cd.cpu(), 0).to(torch.int32)
    rows_d, max_d = int(off_d[-1]), int(cd.max().item())
    x_d, h_d = x[:rows_d].contiguous(), h[:rows_d].contiguous()
    yg_d = torch.empty((rows_d, 2 * I), dtype=torch.bfloat16, device=dev)
    yd_d = torch.empty((rows_d, H), dtype=torch.bfloat16, device=dev)

    def layer_d():
        nf4_grouped_gemm(x_d, gu_p, gu_s.absmax, off_d, (2 * I, H), 64, max_rows=max_d, out=yg_d)
        nf4_grouped_gemm(h_d, dn_p, dn_s.absmax, off_d, (H, I), 64, max_rows=max_d, out=yd_d)

    dec_ms = event_time_ms(torch, layer_d, 20)
    _lib.lib().stm_nf4_gemm_set_tile(0)
    try:
        dec_tile_ms = event_time_ms(torch, layer_d, 20)
    finally:
        _lib.lib().stm_nf4_gemm_set_tile(-1)
    return {"experts": E, "tokens": T, "top_k": TOPK, "rows": rows, "max_rows_per_expert": max_rows,
            "layer_ms": round(ms, 4), "tflops": round(flops / ms / 1e9, 1), "gflop_per_layer": round(flops / 1e9, 1),
            "dequantize_plus_expert_loop": {"layer_ms": round(lib_ms, 4), "tflops": round(flops / lib_ms / 1e9, 1),
                                            "what": "k_dequantize over both banks + one hipBLASLt matmul per "
                                                    "expert and projection"},
            "expert_loop_dense_only_ms": round(loop_ms, 4),
            "fused_speedup": round(lib_ms / ms, 3),
            "decode_16tok": {"rows": rows_d, "max_rows_per_expert": max_d, "layer_ms": round(dec_ms, 4),
                             "tile_path_layer_ms": round(dec_tile_ms, 4),
                             "what": "gate_up + down for the first 16 tokens' top-8 routing: the grouped "
                                     "weight-streaming kernel (at most 64 rows per expert) against the 256-row "
                                     "tiles pinned; eager launches, HIP events"}}


def run_mlp(torch, args):
    """Frozen 8B SwiGLU MLP (H 4096, I 14336), 8192 tokens in chunks of 2048:
    forward + input gradient through MemoryFlatFrozenMLP with NF4 projections
    (library default, and fused kernels forced), against the reference's
    architecture: the same wrapper over a dense module holding the dequantized
    bf16 weights (chunked forward and torch.autograd.grad recompute)."""
    import torch.nn as nn
    from stratum_amd.functional import dequantize_4bit
    from stratum_amd.mlp import MemoryFlatFrozenMLP, quantize_mlp_
    dev = torch.device("cuda:0")
    H, I, T, CH = 4096, 14336, 8192, 2048

    class Mlp(nn.Module):
        def __init__(self):
            super().__init__()
            self.gate_proj = nn.Linear(H, I, bias=False, device=dev, dtype=torch.bfloat16)
            self.up_proj = nn.Linear(H, I, bias=False, device=dev, dtype=torch.bfloat16)
            self.down_proj = nn.Linear(I, H, bias=False, device=dev, dtype=torch.bfloat16)
            self.act_fn = nn.SiLU()
            for i, lin in enumerate((self.gate_proj, self.up_proj, self.down_proj)):
                lin.weight.requires_grad_(False)
                lin.weight.copy_(seeded(torch, tuple(lin.weight.shape), 30 + i, 0.02, torch.float16, dev))

    with torch.no_grad():
        dense = Mlp()
    nf4 = quantize_mlp_(Mlp())
    with torch.no_grad():  # the reference runs on the dequantized weights
        for name in ("gate_proj", "up_proj", "down_proj"):
            lin = getattr(nf4, name)
            getattr(dense, name).weight.copy_(dequantize_4bit(lin.quantized, lin.quant_state, dtype=torch.bfloat16))
    x = seeded(torch, (1, T, H), 33, 1.0, torch.bfloat16, dev)
    dy = seeded(torch, (1, T, H), 34, 1.0, torch.bfloat16, dev)

    def run(module):
        w = MemoryFlatFrozenMLP(module, token_chunk_size=CH)

        def go():
            xi = x.detach().requires_grad_(True)
            w(xi).backward(dy)
        return go

    out = {}
    flops = 2.0 * T * H * I * 3 * 2  # forward (3 projections) + input gradient (3)
    for name, fn in (("reference_arch_dense", run(dense)), ("nf4_default", run(nf4))):
        ms = event_time_ms(torch, fn, 5)
        out[name] = {"ms": round(ms, 3), "tflops": round(flops / ms / 1e9, 1)}
    policy = os.environ.get("STRATUM_NF4_FUSED_MAX_ROWS")
    os.environ["STRATUM_NF4_FUSED_MAX_ROWS"] = "-1"
    try:
        ms = event_time_ms(torch, run(nf4), 5)
    finally:
        if policy is None:
            del os.environ["STRATUM_NF4_FUSED_MAX_ROWS"]
        else:
            os.environ["STRATUM_NF4_FUSED_MAX_ROWS"] = policy
    out["nf4_fused_forced"] = {"ms": round(ms, 3), "tflops": round(flops / ms / 1e9, 1)}
    out["model_gflop"] = round(flops / 1e9, 1)
    out["tokens"], out["chunk"] = T, CH
    return out


def run_small_m(torch, args):
    """M = 16 rows on the 14336 x 4096 weight (decode-sized): fused forward (the
    split-free weight-streaming small-M kernel, one launch) and input gradient
    (the weight-streaming small-M input-gradient kernel over ranges of weight
    rows, plus the split reduce), against dequantize + hipBLASLt; the fused
    forward of a single row (batch-1 decode); and both at 64 rows (the 64-row
    layouts of the two weight-streaming kernels, ranges + split reduce)."""
    from stratum_amd.functional import dequantize_4bit, nf4_gemm_bwd_dx, nf4_gemm_fwd
    dev = torch.device("cuda:0")
    N, K, M = 14336, 4096, 16
    p, st = _gpu_quantized(torch, (N, K), 40, dev)
    st.dtype = torch.bfloat16
    x = seeded(torch, (M, K), 41, 1.0, torch.bfloat16, dev)
    dy = seeded(torch, (M, N), 42, 1.0, torch.bfloat16, dev)
    f = graph_time_ms(torch, lambda: nf4_gemm_fwd(x, p, st.absmax, (N, K), 64), 20)
    b = graph_time_ms(torch, lambda: nf4_gemm_bwd_dx(dy, p, st.absmax, (N, K), 64), 20)
    uf = graph_time_ms(torch, lambda: x @ dequantize_4bit(p, st).t(), 20)
    ub = graph_time_ms(torch, lambda: dy @ dequantize_4bit(p, st), 20)
    x1 = x[:1].contiguous()
    f1 = graph_time_ms(torch, lambda: nf4_gemm_fwd(x1, p, st.absmax, (N, K), 64), 20)
    x64 = seeded(torch, (64, K), 43, 1.0, torch.bfloat16, dev)
    dy64 = seeded(torch, (64, N), 44, 1.0, torch.bfloat16, dev)
    f64 = graph_time_ms(torch, lambda: nf4_gemm_fwd(x64, p, st.absmax, (N, K), 64), 20)
    b64 = graph_time_ms(torch, lambda: nf4_gemm_bwd_dx(dy64, p, st.absmax, (N, K), 64), 20)
    uf64 = graph_time_ms(torch, lambda: x64 @ dequantize_4bit(p, st).t(), 20)
    ub64 = graph_time_ms(torch, lambda: dy64 @ dequantize_4bit(p, st), 20)
    wbytes = N * K / 2 + 4 * N * K / 64
    return {"M": M, "fused_fwd_ms": round(f, 4), "fused_bwd_ms": round(b, 4), "unfused_fwd_ms": round(uf, 4),
            "unfused_bwd_ms": round(ub, 4), "fused_fwd_weight_gbs": round(wbytes / f / 1e6, 1),
            "fused_bwd_weight_gbs": round(wbytes / b / 1e6, 1),
            "fused_fwd_m1_ms": round(f1, 4), "fused_fwd_m1_weight_gbs": round(wbytes / f1 / 1e6, 1),
            "m64": {"fused_fwd_ms": round(f64, 4), "fused_bwd_ms": round(b64, 4),
                    "unfused_fwd_ms": round(uf64, 4), "unfused_bwd_ms": round(ub64, 4)},
            "timing": "device time: 20 launches captured in one HIP graph, replayed (the input gradient's "
                      "split reduce included)"}


SECONDARY_CONFIGS = {
    "roundtrip_f16_5632x2048": run_roundtrip,
    "qwen3_0.6b_layer_fwd_m4096": run_qwen06,
    "moe_128x_gate_up_down_8192tok_top8": run_moe,
    "stream_8b_layers_pinned_h2d_dequant": run_layer_stream,
    "mlp_8b_swiglu_8192tok_chunk2048_fwd_bwd": run_mlp,
    "small_m16_w14336x4096_split_reduction": run_small_m,
}


def run_profile(args):
    """Kernel-only pass for rocprofv3 (kernel trace / PMC): each kernel of the
    step launched `--kernel-reps` times on the default workload, the quantize
    kernel on the same weight, the batched quantize / dequantize on one
    TinyLlama-1.1B layer's matrices, plus a plain 1 GiB device copy whose
    FETCH_SIZE / WRITE_SIZE calibrate the counters."""
    import torch

    from stratum_amd.functional import dequantize_4bit, nf4_gemm_bwd_dx, nf4_gemm_fwd, quantize_4bit

    dev = torch.device("cuda:0")
    N, K, M = 14336, 4096, 8192
    w = seeded(torch, (N, K), 0, 0.02, torch.float16, dev)
    packed, state = quantize_4bit(w)
    state.dtype = torch.bfloat16
    x = seeded(torch, (M, K), 1, 1.0, torch.bfloat16, dev)
    dy = seeded(torch, (M, N), 4, 1.0, torch.bfloat16, dev)
    out = torch.empty((N, K), dtype=torch.bfloat16, device=dev)
    # the quantize kernel on the same weight, and the batched kernels on the
    # matrices of one TinyLlama-1.1B layer
    from stratum_amd.functional import dequantize_4bit_many, quantize_4bit_many
    layer = [seeded(torch, sh, 60 + i, 0.02, torch.float16, dev) for i, sh in enumerate(
        [(2048, 2048), (256, 2048), (256, 2048), (2048, 2048), (5632, 2048), (5632, 2048), (2048, 5632)])]
    layer_q = quantize_4bit_many(layer)
    layer_out = [torch.empty_like(t) for t in layer]
    # calibration: an elementwise kernel that reads 1 GiB and writes 1 GiB
    src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(args.kernel_reps):
        nf4_gemm_fwd(x, packed, state.absmax, (N, K), 64)
        nf4_gemm_bwd_dx(dy, packed, state.absmax, (N, K), 64)
        dequantize_4bit(packed, state, out=out)
        quantize_4bit(w)
        quantize_4bit_many(layer)
        dequantize_4bit_many(layer_q, out=layer_out)
        torch.mul(src, 2.0, out=dst)
    torch.cuda.synchronize()
    print(json.dumps({"profile": "done", "reps": args.kernel_reps, "copy_bytes": 4 * src.numel()}), flush=True)


def run_profile_small_m(args):
    """Kernel-only pass for rocprofv3 at decode size: the fused forward (the
    split-free small-M kernel) and input gradient (small-M kernel + split reduce)
    at M = 16 on the 14336 x 4096 weight, each launched --kernel-reps times."""
    import torch

    from stratum_amd.functional import nf4_gemm_bwd_dx, nf4_gemm_fwd

    dev = torch.device("cuda:0")
    N, K, M = 14336, 4096, 16
    p, st = _gpu_quantized(torch, (N, K), 40, dev)
    x = seeded(torch, (M, K), 41, 1.0, torch.bfloat16, dev)
    dy = seeded(torch, (M, N), 42, 1.0, torch.bfloat16, dev)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    dx = torch.empty((M, K), dtype=torch.bfloat16, device=dev)
    for _ in range(args.kernel_reps):
        nf4_gemm_fwd(x, p, st.absmax, (N, K), 64, out=y)
    for _ in range(args.kernel_reps):
        nf4_gemm_bwd_dx(dy, p, st.absmax, (N, K), 64, out=dx)
    torch.cuda.synchronize()
    print(json.dumps({"profile": "small_m16 done", "reps": args.kernel_reps}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="lora_step", choices=["lora_step"])
    ap.add_argument("--kernel-reps", type=int, default=20)
    ap.add_argument("--cpu-rows", type=int, default=256)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--main-only", action="store_true", help="skip the secondary configs")
    ap.add_argument("--layers", type=int, default=32, help="decoder layers in the stream-in config")
    ap.add_argument("--profile", action="store_true",
                    help="launch each kernel --kernel-reps times for rocprofv3; prints no bench line")
    ap.add_argument("--profile-small-m", action="store_true",
                    help="as --profile, for the M = 16 forward and input gradient")
    ap.add_argument("--config", choices=sorted(SECONDARY_CONFIGS),
                    help="run one secondary config alone and print its JSON (e.g. under rocprofv3)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}, WORLD_SIZE {world}); "
              "the NF4 path is sharded by weight rows with no collective on one GPU's share -- "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if args.profile:
        run_profile(args)
        return
    if args.profile_small_m:
        run_profile_small_m(args)
        return
    if args.config:
        import torch
        torch.cuda.set_device(0)
        print(json.dumps({args.config: SECONDARY_CONFIGS[args.config](torch, args)}), flush=True)
        return
    line = run_lora_step(args)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
