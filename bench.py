"""Benchmark of the NF4 QLoRA gated-MLP hot path on one MI355X.

Headline (value): tokens/s of one NF4-LoRA gated MLP forward+backward at the
Llama-3-8B MLP shape (BASELINE cfg4: H=4096, I=14336, r=64, alpha=128,
M=8192 tokens), including every adapter gradient. Inputs are synthetic, seeded
and already resident in HBM. Also reported: the roofline of the dominant
kernel (the fused gate/up NF4 GEMM) from HIP events recorded around its
launches on its own stream during the timed steps, the frozen RMSNorm kernels
and the RMSNorm-replay recipe step, every NF4-LoRA projection shape of the
cfg3 decoder (attention and MLP, forward + backward), the frozen LM head with
its chunked cross-entropy, the skinny-M NF4 GEMV sweep (cfg5, HBM
GB/s), and the CPU baseline (the oracle's restatement of MOLT's
eager CPU path, cfg1, numpy fp32 on the host cores).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_BF16_TFLOPS = 2516.6   # MI355X dense bf16 MFMA (256 CU x 2.4 GHz x 4096 FLOP/clk)
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
METRIC = "QLoRA gated-MLP fwd+bwd tokens/s @1 GPU; MFMA util %; NF4 GEMV HBM GB/s"
NF4_BYTES_PER_ELEM = 0.5 + 1 / 64 + 4 / 16384


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def make_mlp(H, I, r, alpha, M, seed, dev):
    import torch
    import molt_amd

    g = torch.Generator(device="cpu").manual_seed(seed)
    projs = []
    for out_f, in_f in ((I, H), (I, H), (H, I)):
        w = (torch.randn(out_f, in_f, generator=g) * 0.02).to(dev)
        packed, qs = molt_amd.quantize_4bit(w, blocksize=64, compress_statistics=True)
        del w
        bound = 1.0 / math.sqrt(in_f)
        a = ((torch.rand(r, in_f, generator=g) * 2 - 1) * bound).to(dev).requires_grad_()
        b = (torch.randn(out_f, r, generator=g) * 0.01).to(dev).requires_grad_()
        molt_amd.resolved_nf4_scales(qs)
        projs.append((packed, qs, a, b))
    x = torch.randn(M, H, generator=g).to(dev, torch.bfloat16).requires_grad_()
    dy = torch.randn(M, H, generator=g).to(dev, torch.bfloat16)
    return projs, x, dy, alpha / r


def mlp_step(projs, x, dy, s):
    from molt_amd.methods import fused_gated_nf4_lora_mlp

    (pg, qg, ag, bg), (pu, qu, au, bu), (pd, qd, ad, bd) = projs
    for t in (x, ag, bg, au, bu, ad, bd):
        t.grad = None
    y = fused_gated_nf4_lora_mlp(x, pg, ag, bg, pu, au, bu, pd, ad, bd, qg, qu, qd, s, s, s)
    y.backward(dy)


def gemv_sweep(dev, reps: int = 20):
    """cfg5: NF4 GEMV at Llama-3-8B projection shapes, M in {1..16}, r=16 LoRA
    add-on. Each launch reads a different copy of the weight (>= 512 MiB of
    distinct copies per shape, beyond the 256 MB Infinity Cache); launches
    are captured in a HIP graph so host launch cost is not timed."""
    import ctypes
    import torch
    import molt_amd
    from molt_amd import _lib, ops

    lib = _lib.load()
    out = []
    g = torch.Generator(device="cpu").manual_seed(5)
    for n, k in ((4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)):
        w = (torch.randn(n, k, generator=g) * 0.02).to(dev)
        packed, qs = molt_amd.quantize_4bit(w, blocksize=64, compress_statistics=True)
        del w
        wbytes = n * k // 2
        copies = max(2, math.ceil(512 * 2**20 / wbytes))
        packs = [packed.reshape(-1).clone() for _ in range(copies)]
        qcopies = [qs.absmax.clone() for _ in range(copies)]
        r = 16
        a = ((torch.rand(r, k, generator=g) * 2 - 1) / math.sqrt(k)).to(dev)
        b = (torch.randn(n, r, generator=g) * 0.01).to(dev)
        descs = []
        for pk, qq in zip(packs, qcopies):
            d = ops._weight(pk, None, qs.code, n, k, 64, 1, qq, qs.state2.absmax, qs.state2.code,
                            float(qs.offset), 256)
            descs.append(d)
        for m in (1, 2, 4, 8, 16):
            log(f"gemv N={n} K={k} M={m} ...")
            x = torch.randn(m, k, generator=g).to(dev, torch.bfloat16)
            t = ops.lora_project(x, None, 0, 1.0, a, 0)
            y = torch.empty(m, n, device=dev, dtype=torch.bfloat16)
            ws_bytes = int(lib.molt_nf4_gemv_workspace(m, n, k))
            ws = torch.zeros(max(ws_bytes, 256), device=dev, dtype=torch.uint8)   # unused when 0 bytes
            torch.cuda.synchronize()

            def launch_all():
                st = torch.cuda.current_stream().cuda_stream
                for d in descs:
                    _lib.check(lib.molt_nf4_gemv(x.data_ptr(), k, m, ctypes.byref(d), t.data_ptr(), r,
                                                 b.data_ptr(), r, 2.0, y.data_ptr(), n, ws.data_ptr(),
                                                 ws_bytes, st))

            launch_all()   # warm (and validates arguments outside capture)
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                launch_all()
            graph.replay()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                graph.replay()
            e1.record()
            e1.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / (reps * len(descs))
            alg = n * k * NF4_BYTES_PER_ELEM + m * k * 2 + m * n * 2 + r * (k + n) * 2
            gbs = alg / (us * 1e-6) / 1e9
            out.append({"N": n, "K": k, "M": m, "us": round(us, 3), "GB_s": round(gbs, 1),
                        "frac_hbm": round(gbs / PEAK_HBM_GBS, 4)})
            log(f"gemv N={n} K={k} M={m}: {us:.2f} us/launch, {gbs:.0f} GB/s ({100 * gbs / PEAK_HBM_GBS:.1f}%)")
            del graph
        del packs, qcopies, descs
        torch.cuda.empty_cache()
    return out


def rmsnorm_bench(dev, projs, dy, s, M, H, steps: int, reps: int = 5):
    """Frozen RMSNorm at the cfg4 residual shape ([M, H] bf16, bf16 weight):
    forward and backward kernel time (HIP events over `reps` rounds of
    launches over distinct input copies) against their algorithmic bytes, and the gated-MLP step through the RMSNorm-replay
    recipe (norm forward + _ResidualRecipeGatedNF4LoRA + norm backward), which
    saves the residual instead of the normalised input."""
    import torch
    from molt_amd import ops
    from molt_amd.kernels.frozen_rmsnorm import _FrozenRMSNormFunction
    from molt_amd.methods.gated_replay import _ResidualRecipeGatedNF4LoRA

    g = torch.Generator(device="cpu").manual_seed(7)
    src = torch.randn(M, H, generator=g).to(dev, torch.bfloat16)
    w = (1.0 + 0.2 * torch.randn(H, generator=g)).to(dev, torch.bfloat16)
    gy = torch.randn(M, H, generator=g).to(dev, torch.bfloat16)
    eps = 1e-6
    # rotate over distinct copies (>= 512 MiB of inputs) so that the kernels
    # read HBM, not the 256 MB Infinity Cache
    copies = max(2, math.ceil(512 * 2**20 / (M * H * 2)))
    srcs = [src.clone() for _ in range(copies)]
    gys = [gy.clone() for _ in range(copies)]
    out = {}
    for name, fn, nbytes in (("forward", lambda j: ops.rmsnorm_forward(srcs[j], w, eps, 0.0), 2 * M * H * 2 + H * 2),
                             ("backward", lambda j: ops.rmsnorm_backward(gys[j], srcs[j], w, eps, 0.0),
                              3 * M * H * 2 + H * 2)):
        for j in range(copies):
            fn(j)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for j in range(reps * copies):
            fn(j % copies)
        e1.record()
        e1.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / (reps * copies)
        gbs = nbytes / (us * 1e-6) / 1e9
        out[name] = {"us": round(us, 2), "bytes": nbytes, "GB_s": round(gbs, 1), "frac_hbm": round(gbs / PEAK_HBM_GBS, 4)}
        log(f"rmsnorm {name} M={M} H={H}: {us:.2f} us, {gbs:.0f} GB/s ({100 * gbs / PEAK_HBM_GBS:.1f}% of HBM)")

    del srcs, gys
    (pg, qg, ag, bg), (pu, qu, au, bu), (pd, qd, ad, bd) = projs
    source = src.clone().requires_grad_()

    def step():
        for t in (source, ag, bg, au, bu, ad, bd):
            t.grad = None
        normalized = _FrozenRMSNormFunction.apply(source, w, eps, 0.0)
        y = _ResidualRecipeGatedNF4LoRA.apply(source, normalized, pg, ag, bg, pu, au, bu, pd, ad, bd, qg, qu, qd,
                                              s, s, s, w, eps, 0.0)
        y.backward(dy)

    for _ in range(2):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    out["recipe_step_ms"] = round(ms, 4)
    out["recipe_tokens_s"] = round(M / (ms * 1e-3), 1)
    log(f"RMSNorm-replay recipe step (norm fwd + gated MLP fwd/bwd + norm bwd): {ms:.3f} ms, {M / (ms * 1e-3):.0f} tok/s")
    return out


def projection_sweep(dev, reps: int = 10):
    """Every NF4-LoRA projection of the cfg3 decoder (Qwen2.5-1.5B shapes:
    H=1536, 12 q heads / 2 kv heads x 128, I=8960, r=16, M=4096 tokens)
    through scheduled_nf4_lora, forward + backward (dX, dA, dB), with the
    algorithmic FLOPs 4*M*N*K + 6*M*r*(N+K) per projection."""
    import torch
    import molt_amd
    from molt_amd.methods import scheduled_nf4_lora

    M, r, s = 4096, 16, 2.0
    g = torch.Generator(device="cpu").manual_seed(9)
    out = []
    for name, n, k in (("q_proj/o_proj", 1536, 1536), ("k_proj/v_proj", 256, 1536), ("gate_proj/up_proj", 8960, 1536),
                       ("down_proj", 1536, 8960)):
        w = (torch.randn(n, k, generator=g) * 0.02).to(dev)
        packed, qs = molt_amd.quantize_4bit(w, blocksize=64, compress_statistics=True)
        del w
        a = ((torch.rand(r, k, generator=g) * 2 - 1) / math.sqrt(k)).to(dev).requires_grad_()
        b = (torch.randn(n, r, generator=g) * 0.01).to(dev).requires_grad_()
        x = torch.randn(M, k, generator=g).to(dev, torch.bfloat16).requires_grad_()
        dy = torch.randn(M, n, generator=g).to(dev, torch.bfloat16)

        def run():
            for t in (x, a, b):
                t.grad = None
            with torch.autocast("cuda", dtype=torch.bfloat16):
                y = scheduled_nf4_lora(x, packed, a, b, qs, s)
            y.backward(dy)

        for _ in range(3):
            run()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            run()
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / reps
        flop = 4 * M * n * k + 6 * M * r * (n + k)
        tf = flop / (ms * 1e-3) / 1e12
        out.append({"proj": name, "N": n, "K": k, "M": M, "r": r, "ms_fwd_bwd": round(ms, 4), "TFLOP_s": round(tf, 1),
                    "frac_bf16_peak": round(tf / PEAK_BF16_TFLOPS, 4)})
        log(f"cfg3 {name} N={n} K={k} M={M}: fwd+bwd {ms:.3f} ms, {tf:.0f} TFLOP/s ({100 * tf / PEAK_BF16_TFLOPS:.1f}%)")
    return out


def lm_head_bench(dev, steps: int = 5):
    """The frozen LM head of the cfg3 decoder (Qwen2.5-1.5B: vocabulary
    151,936 x hidden 1,536, bf16) over M=4096 tokens in chunks of 256 through
    frozen_linear_cross_entropy: loss and hidden gradient (two hipBLASLt GEMMs
    per chunk, 4*M*V*H FLOPs in all, plus the HIP row reduction). The row
    kernel alone is timed on one [256, V] chunk against its algorithmic bytes
    (read the logits once, write the gradient once)."""
    import torch
    from molt_amd import ops
    from molt_amd.kernels.frozen_linear_cross_entropy import frozen_linear_cross_entropy

    V, H, M, chunk = 151936, 1536, 4096, 256
    g = torch.Generator(device="cpu").manual_seed(11)
    w = (torch.randn(V, H, generator=g) * 0.02).to(dev, torch.bfloat16)
    h = torch.randn(M, H, generator=g).to(dev, torch.bfloat16).requires_grad_()
    t = torch.randint(0, V, (M,), generator=g).to(dev)

    def run():
        h.grad = None
        frozen_linear_cross_entropy(h, w, t, chunk).backward()

    for _ in range(2):
        run()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        run()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    flop = 4 * M * V * H
    tf = flop / (ms * 1e-3) / 1e12
    logits = torch.randn(chunk, V, generator=g).to(dev, torch.bfloat16)
    tc = t[:chunk].contiguous()
    copies = [logits.clone() for _ in range(8)]
    for c in copies:
        ops.cross_entropy_rows(c, tc, float(M), True)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for c in copies:
        ops.cross_entropy_rows(c, tc, float(M), True)
    e1.record()
    e1.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / len(copies)
    nbytes = 2 * chunk * V * 2
    gbs = nbytes / (us * 1e-6) / 1e9
    log(f"LM head V={V} H={H} M={M} chunk={chunk}: loss+grad {ms:.3f} ms, {tf:.0f} TFLOP/s "
        f"({100 * tf / PEAK_BF16_TFLOPS:.1f}%); row kernel {us:.1f} us per chunk, {gbs:.0f} GB/s "
        f"({100 * gbs / PEAK_HBM_GBS:.1f}% of HBM)")
    return {"vocab": V, "hidden": H, "tokens": M, "chunk": chunk, "ms_loss_and_grad": round(ms, 4),
            "TFLOP_s": round(tf, 1), "frac_bf16_peak": round(tf / PEAK_BF16_TFLOPS, 4),
            "row_kernel_us_per_chunk": round(us, 2), "row_kernel_GB_s": round(gbs, 1),
            "row_kernel_frac_hbm": round(gbs / PEAK_HBM_GBS, 4)}


TRAFFIC_FILE = ROOT / "profiles" / "gateup_fwd_cfg4_hbm_traffic.txt"


def measured_traffic():
    """HBM bytes per launch of the gate/up kernel, from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE passes (each scaled by the same counter's reading
    for a copy of known size); None when no such summary is present."""
    try:
        for line in TRAFFIC_FILE.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch:"):
                return int(float(line.split(":", 1)[1]))
    except OSError:
        pass
    return None


def profile_kernel(which: str, reps: int) -> int:
    """Run one kernel `reps` times at cfg4 shapes, for rocprofv3 counter passes:
    'gateup' = the fused gate/up NF4-LoRA GEMM, 'copy' = a 1 GiB device copy
    (1 GiB read + 1 GiB written) that calibrates FETCH_SIZE / WRITE_SIZE."""
    import torch
    from molt_amd import ops

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if which == "copy":
        src = torch.ones(2**30, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(reps):
            dst.copy_(src)
    else:
        H, I, r, alpha, M = 4096, 14336, 64, 128.0, 8192
        projs, x, _dy, s = make_mlp(H, I, r, alpha, M, 1337, dev)
        (pg, qg, ag, bg), (pu, qu, au, bu) = projs[0], projs[1]
        import molt_amd
        sg, su = molt_amd.resolved_nf4_scales(qg), molt_amd.resolved_nf4_scales(qu)
        with torch.no_grad():
            t = ops.lora_project(x.detach(), None, 0, 1.0, torch.cat([ag, au]).detach(), 0)
            for _ in range(reps):
                ops.nf4_gateup_forward(x.detach(), pg.reshape(-1), sg, pu.reshape(-1), su, qg.code, I, H, 1, t,
                                       bg.detach(), bu.detach(), s, s)
    torch.cuda.synchronize()
    log(f"profile-kernel {which}: {reps} launches done")
    return 0


def cpu_baseline(seconds_budget: float = 20.0):
    """Oracle restatement of MOLT's eager CPU path on cfg1 (numpy fp32)."""
    import numpy as np
    import torch

    from oracle import nf4_oracle as O
    from oracle.cpu_baseline import gated_mlp_step_f32

    H, I, r, M, s = 896, 4864, 16, 1024, 2.0
    rng = np.random.default_rng(1337)
    weights = []
    for out_f, in_f in ((I, H), (I, H), (H, I)):
        w = (rng.standard_normal((out_f, in_f), dtype=np.float32) * np.float32(0.02))
        weights.append(O.quantize_bnb_layout(w, 64, nested=True))
    adapters = []
    for out_f, in_f in ((I, H), (I, H), (H, I)):
        bound = 1.0 / math.sqrt(in_f)
        a = rng.uniform(-bound, bound, (r, in_f)).astype(np.float32)
        b = (rng.standard_normal((out_f, r)) * 0.01).astype(np.float32)
        adapters.append((a, b))
    x = O.bf16_round(rng.standard_normal((M, H)).astype(np.float32))
    dy = O.bf16_round(rng.standard_normal((M, H)).astype(np.float32))
    times = []
    started = time.perf_counter()
    for i in range(2 + 20):
        t0 = time.perf_counter()
        gated_mlp_step_f32(x, weights, adapters, s, dy)
        dt = time.perf_counter() - t0
        if i >= 2:
            times.append(dt)
        if i >= 6 and time.perf_counter() - started > seconds_budget:
            break
    med = statistics.median(times)
    try:
        from threadpoolctl import threadpool_info
        threads = max((p.get("num_threads", 1) for p in threadpool_info()), default=1)
    except Exception:
        threads = os.cpu_count() or 1
    cpu_model = platform.processor() or ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(M / med, 1), "unit": "tokens/s", "cores": int(threads), "kind": "port",
            "sample": f"cfg1 gated MLP H=896 I=4864 r=16 M=1024 fwd+bwd, numpy fp32 with per-step NF4 decode, "
                      f"median of {len(times)} steps ({med * 1e3:.0f} ms/step)",
            "host_cpus": os.cpu_count(), "cpu_model": cpu_model,
            "gflops": round((12 * H * I + 18 * r * (H + I)) * M / med / 1e9, 1)}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--tokens", type=int, default=8192, help="M (default: cfg4's 8 x 1024)")
    ap.add_argument("--no-gemv", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-norm", action="store_true", help="skip the RMSNorm / norm-replay recipe measurement")
    ap.add_argument("--no-proj", action="store_true", help="skip the cfg3 projection sweep")
    ap.add_argument("--no-head", action="store_true", help="skip the LM head + cross-entropy measurement")
    ap.add_argument("--profile-kernel", choices=("gateup", "copy"),
                    help="only launch one kernel (for rocprofv3 --pmc passes) and exit")
    ap.add_argument("--reps", type=int, default=3, help="launches for --profile-kernel")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the data-parallel sharding design is described in DESIGN.md). Run with --gpus 1.",
              file=sys.stderr)
        return 2

    if args.profile_kernel:
        return profile_kernel(args.profile_kernel, args.reps)

    import torch
    from molt_amd import ops

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    H, I, r, alpha, M = 4096, 14336, 64, 128.0, args.tokens
    log(f"building cfg4 workload H={H} I={I} r={r} M={M}")
    projs, x, dy, s = make_mlp(H, I, r, alpha, M, 1337, dev)
    for _ in range(args.warmup):
        mlp_step(projs, x, dy, s)
    torch.cuda.synchronize()
    log("warmup done")
    pairs = ops.probe_events("molt_nf4_gateup_forward")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        mlp_step(projs, x, dy, s)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ops.probe_events("molt_nf4_gateup_forward", enable=False)
    ms_step = elapsed * 1e3 / args.steps
    tok_s = M * args.steps / elapsed
    flop_step = (12 * H * I + 18 * r * (H + I)) * M
    step_tflops = flop_step / (ms_step * 1e-3) / 1e12
    k_ms = statistics.mean(a.elapsed_time(b) for a, b in pairs)
    k_flop = 2 * (2 * M * H * I) + 2 * (2 * M * I * r)      # gate+up base GEMMs + their LoRA B GEMMs
    k_tflops = k_flop / (k_ms * 1e-3) / 1e12
    log(f"step {ms_step:.3f} ms, {tok_s:.0f} tok/s, {step_tflops:.1f} TFLOP/s ({100 * step_tflops / PEAK_BF16_TFLOPS:.1f}% of bf16 peak); "
        f"gate/up kernel {k_ms:.3f} ms = {k_tflops:.1f} TFLOP/s")

    result = {
        "metric": METRIC, "value": round(tok_s, 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic (seeded N(0,0.02) weights NF4-quantised, N(0,1) X/dY)",
        "config": {"workload": "cfg4: Llama-3-8B-shaped NF4-LoRA gated MLP fwd+bwd incl. dA/dB",
                   "hidden": H, "intermediate": I, "lora_rank": r, "lora_alpha": alpha, "tokens": M,
                   "nf4_block": 64, "double_quant": True, "parallelism": "single GPU"},
        "mfma_util_pct": round(100 * step_tflops / PEAK_BF16_TFLOPS, 2),
        "step_tflops": round(step_tflops, 1),
        "roofline": {"kernel": "big::fwd_kernel<true> (fused gate/up NF4-LoRA GEMM)", "bound": "mfma",
                     "achieved": round(k_tflops, 1), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(k_tflops / PEAK_BF16_TFLOPS, 4), "traffic": measured_traffic(),
                     "traffic_unit": "bytes/launch (rocprofv3 FETCH_SIZE+WRITE_SIZE, copy-calibrated)",
                     "avg_launch_ms": round(k_ms, 4), "launches": len(pairs),
                     "flop_per_launch": k_flop},
    }
    if not args.no_norm:
        result["rmsnorm"] = rmsnorm_bench(dev, projs, dy, s, M, H, args.steps)
    if not args.no_proj:
        result["cfg3_projections"] = projection_sweep(dev)
    if not args.no_head:
        result["lm_head"] = lm_head_bench(dev)
    if not args.no_gemv:
        sweep = gemv_sweep(dev)
        result["gemv"] = sweep
        result["gemv_best_frac_hbm"] = max(e["frac_hbm"] for e in sweep)
    if not args.no_cpu:
        log("cpu baseline (cfg1, oracle restatement, numpy fp32)")
        result["cpu_baseline"] = cpu_baseline()
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
