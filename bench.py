"""Benchmark of the NF4 QLoRA gated-MLP hot path on one MI355X.

Headline (value): tokens/s of one NF4-LoRA gated MLP forward+backward at the
Llama-3-8B MLP shape (BASELINE cfg4: H=4096, I=14336, r=64, alpha=128,
M=8192 tokens), including every adapter gradient. Inputs are synthetic, seeded
and already resident in HBM. Also reported: every NF4 GEMM of the step with
its algorithmic TFLOP/s from HIP events recorded around its launches on the
launch stream, and the roofline of the longest of them (the gate/up forward,
timed during the timed steps; the other three in as many steps again after
them, since each pair of timing events leaves the GPU idle for a few µs);
the standalone NF4 dequant (HBM GB/s); the frozen RMSNorm kernels
and the RMSNorm-replay recipe step, every NF4-LoRA projection shape of the
cfg3 decoder (attention and MLP, forward + backward), the frozen LM head with
its chunked cross-entropy, the 28-layer cfg3 decoder stack, the skinny-M NF4
GEMV sweep (cfg5, HBM GB/s), cfg1 on the GPU and, beside it, the CPU baseline
(the oracle's restatement of MOLT's eager CPU path, cfg1, numpy fp32 on the
host cores).

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


GEMV_CFG5 = ((4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336))
# Qwen2.5-1.5B decode shapes (the reference's generate_qlora, training/qlora.py:1332-1358):
# q/o 1536 x 1536, k/v 256 x 1536, gate/up 8960 x 1536, down 1536 x 8960
GEMV_QWEN = ((1536, 1536), (256, 1536), (8960, 1536), (1536, 8960))


def gemv_sweep(dev, reps: int = 20, shapes=GEMV_CFG5 + GEMV_QWEN):
    """cfg5: NF4 GEMV at Llama-3-8B projection shapes, M in {1..16}, r=16 LoRA
    add-on, plus the Qwen2.5-1.5B decode shapes as extra rows. Each launch
    reads a different copy of the weight (>= 512 MiB of distinct copies per
    shape, beyond the 256 MB Infinity Cache); launches are captured in a HIP
    graph so host launch cost is not timed."""
    import ctypes
    import torch
    import molt_amd
    from molt_amd import _lib, ops

    lib = _lib.load()
    out = []
    g = torch.Generator(device="cpu").manual_seed(5)
    for n, k in shapes:
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
                        "frac_hbm": round(gbs / PEAK_HBM_GBS, 4),
                        "set": "cfg5" if (n, k) in GEMV_CFG5 else "qwen2.5-1.5b"})
            log(f"gemv N={n} K={k} M={m}: {us:.2f} us/launch, {gbs:.0f} GB/s ({100 * gbs / PEAK_HBM_GBS:.1f}%)")
            del graph
        del packs, qcopies, descs
        torch.cuda.empty_cache()
    return out


def dequant_bench(dev, n: int = 14336, k: int = 4096, reps: int = 10):
    """Standalone NF4 dequant (molt_nf4_dequantize, nested statistics, bf16
    out) of an n x k weight: 2.515869 algorithmic bytes per element (read the
    packed codes and the statistics, write bf16). Each launch reads a distinct
    copy (>= 512 MiB in all) and writes one of four outputs (470 MB), so
    neither side stays in the 256 MB Infinity Cache; launches are replayed from
    a HIP graph."""
    import ctypes
    import torch
    import molt_amd
    from molt_amd import _lib, ops

    lib = _lib.load()
    g = torch.Generator(device="cpu").manual_seed(13)
    w = (torch.randn(n, k, generator=g) * 0.02).to(dev)
    packed, qs = molt_amd.quantize_4bit(w, blocksize=64, compress_statistics=True)
    del w
    per_copy = n * k // 2 + qs.absmax.numel()
    copies = max(2, math.ceil(512 * 2**20 / per_copy))
    packs = [packed.reshape(-1).clone() for _ in range(copies)]
    qcopies = [qs.absmax.clone() for _ in range(copies)]
    outs = [torch.empty(n, k, device=dev, dtype=torch.bfloat16) for _ in range(4)]
    code, a2, c2 = qs.code.float().contiguous(), qs.state2.absmax.float().contiguous(), qs.state2.code.float().contiguous()
    descs = [ops._weight(pk, None, code, n, k, 64, 1, qq, a2, c2, float(qs.offset), 256)
             for pk, qq in zip(packs, qcopies)]

    def launch_all():
        st = torch.cuda.current_stream().cuda_stream
        for i, d in enumerate(descs):
            _lib.check(lib.molt_nf4_dequantize(ctypes.byref(d), outs[i % 4].data_ptr(), _lib.DTYPE_BF16, st))

    launch_all()
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
    us = e0.elapsed_time(e1) * 1e3 / (reps * copies)
    alg = n * k * (NF4_BYTES_PER_ELEM + 2)
    gbs = alg / (us * 1e-6) / 1e9
    log(f"dequant {n}x{k}: {us:.2f} us, {gbs:.0f} GB/s ({100 * gbs / PEAK_HBM_GBS:.1f}% of HBM)")
    return {"N": n, "K": k, "us": round(us, 3), "bytes": int(alg), "GB_s": round(gbs, 1),
            "frac_hbm": round(gbs / PEAK_HBM_GBS, 4), "copies": copies}


def cfg1_gpu(dev, steps: int = 20):
    """cfg1 (the CPU baseline's workload: H=896, I=4864, r=16, alpha=32,
    M=1024) on the GPU through the same fused gated-MLP node as the headline."""
    import torch

    H, I, r, alpha, M = 896, 4864, 16, 32.0, 1024
    projs, x, dy, s = make_mlp(H, I, r, alpha, M, 1337, dev)
    for _ in range(3):
        mlp_step(projs, x, dy, s)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        mlp_step(projs, x, dy, s)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    tf = (12 * H * I + 18 * r * (H + I)) * M / (ms * 1e-3) / 1e12
    log(f"cfg1 on the GPU: {ms:.3f} ms/step, {M / (ms * 1e-3):.0f} tok/s, {tf:.1f} TFLOP/s")
    return {"tokens_s": round(M / (ms * 1e-3), 1), "ms_per_step": round(ms, 4), "TFLOP_s": round(tf, 1),
            "frac_bf16_peak": round(tf / PEAK_BF16_TFLOPS, 4)}


def cfg3_stack(dev, steps: int = 3):
    """cfg3: the 28-layer Qwen2.5-1.5B-shaped decoder stack (hidden 1536,
    12/2 heads of 128, intermediate 8960, RMSNorm; transformers' Llama decoder
    with those shapes, bias-free projections), NF4 QLoRA r=16 alpha=32 on all
    seven projections, fwd+bwd over bf16 embeddings N(0,1) at 4 x 1024 tokens,
    with the gated MLP's RMSNorm replay. Attention is torch SDPA. FLOPs per token
    and layer: the projections' forward GEMMs twice (forward and input
    gradient; the frozen weights have none), 6 r (K + N) per LoRA adapter, and
    causal attention 6 * seq * H (QK^T and PV, forward and twice that backward,
    halved for causality)."""
    import torch
    from transformers import LlamaConfig, LlamaModel

    from molt_amd.kernels import enable_frozen_rmsnorm_bf16
    from molt_amd.loading import prepare_nf4_qlora
    from molt_amd.methods import (enable_fused_gated_nf4_lora, enable_rmsnorm_replay, enable_scheduled_nf4_lora,
                                  enable_stacked_nf4_lora)

    H, I, L, heads, kv, hd, r, B, S = 1536, 8960, 28, 12, 2, 128, 16, 4, 1024
    cfg = LlamaConfig(hidden_size=H, intermediate_size=I, num_hidden_layers=L, num_attention_heads=heads,
                      num_key_value_heads=kv, head_dim=hd, vocab_size=256, rms_norm_eps=1e-6,
                      max_position_embeddings=S, attention_bias=False, mlp_bias=False)
    cfg._attn_implementation = "sdpa"
    torch.manual_seed(1337)
    with torch.device(dev):
        model = LlamaModel(cfg)
    prepare_nf4_qlora(model, r, 32.0)
    enable_frozen_rmsnorm_bf16(model)
    enable_scheduled_nf4_lora(model, module_suffixes=("q_proj", "k_proj", "v_proj", "o_proj"))
    enable_stacked_nf4_lora(model)          # q, k and v of each layer as one node
    enable_fused_gated_nf4_lora(model)
    enable_rmsnorm_replay(model)
    g = torch.Generator(device="cpu").manual_seed(3)
    x = torch.randn(B, S, H, generator=g).to(dev, torch.bfloat16).requires_grad_()
    dy = torch.randn(B, S, H, generator=g).to(dev, torch.bfloat16)
    params = [p for p in model.parameters() if p.requires_grad]

    def step():
        x.grad = None
        for p in params:
            p.grad = None
        with torch.autocast("cuda", dtype=torch.bfloat16):
            out = model(inputs_embeds=x).last_hidden_state
        out.backward(dy)

    for _ in range(2):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    proj = 2 * H * (H + 2 * kv * hd) + 2 * H * H + 3 * 2 * H * I       # forward GEMMs per token
    lora = 6 * r * ((H + H) + 2 * (H + kv * hd) + (H + H) + 3 * (H + I))  # 6 r (K + N) per projection
    attn = 6 * S * H                                                    # causal QK^T, PV: fwd + 2x bwd
    flop_tok = L * (2 * proj + lora + attn)                             # fwd + dX, frozen weights
    tok = B * S
    tf = flop_tok * tok / (ms * 1e-3) / 1e12
    log(f"cfg3 stack: {ms:.2f} ms/step, {tok / (ms * 1e-3):.0f} tok/s, {tf:.0f} TFLOP/s "
        f"({100 * tf / PEAK_BF16_TFLOPS:.1f}% of bf16 peak)")
    del model
    torch.cuda.empty_cache()
    return {"layers": L, "tokens": tok, "ms_per_step": round(ms, 3), "tokens_s": round(tok / (ms * 1e-3), 1),
            "gflop_per_token": round(flop_tok / 1e9, 3), "TFLOP_s": round(tf, 1),
            "frac_bf16_peak": round(tf / PEAK_BF16_TFLOPS, 4)}


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
    algorithmic FLOPs 4*M*N*K + 6*M*r*(N+K) per projection. Timed twice: eager
    through autograd (host-inclusive; the small shapes are host-bound) and as
    the GPU work alone (the same kernels replayed from a HIP graph)."""
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
        gpu_ms = _graph_ms(lambda: _projection_ops(x, packed, qs, a, b, dy, s))
        flop = 4 * M * n * k + 6 * M * r * (n + k)
        tf = flop / (ms * 1e-3) / 1e12
        gtf = flop / (gpu_ms * 1e-3) / 1e12
        out.append({"proj": name, "N": n, "K": k, "M": M, "r": r, "ms_fwd_bwd": round(ms, 4), "TFLOP_s": round(tf, 1),
                    "frac_bf16_peak": round(tf / PEAK_BF16_TFLOPS, 4), "gpu_ms_fwd_bwd": round(gpu_ms, 4),
                    "gpu_TFLOP_s": round(gtf, 1), "gpu_frac_bf16_peak": round(gtf / PEAK_BF16_TFLOPS, 4)})
        log(f"cfg3 {name} N={n} K={k} M={M}: fwd+bwd {ms:.3f} ms eager ({tf:.0f} TFLOP/s, "
            f"{100 * tf / PEAK_BF16_TFLOPS:.1f}%), {gpu_ms:.3f} ms of GPU work ({gtf:.0f} TFLOP/s, "
            f"{100 * gtf / PEAK_BF16_TFLOPS:.1f}%)")
    out.append(_stacked_qkv(dev, M, r, s, reps, g))
    return out


def _stacked_qkv(dev, M, r, s, reps, g):
    """cfg3's q, k and v projections (1536, 256 and 256 outputs of 1536) as one
    stacked node (methods.stacked_lora) against the three scheduled nodes:
    forward + backward, eager and as GPU work alone."""
    import torch
    import molt_amd
    from molt_amd.methods import scheduled_nf4_lora
    from molt_amd.methods.stacked_lora import stacked_nf4_lora

    k, rows = 1536, (1536, 256, 256)
    projs = []
    for n in rows:
        w = (torch.randn(n, k, generator=g) * 0.02).to(dev)
        packed, qs = molt_amd.quantize_4bit(w, blocksize=64, compress_statistics=True)
        a = ((torch.rand(r, k, generator=g) * 2 - 1) / math.sqrt(k)).to(dev).requires_grad_()
        b = (torch.randn(n, r, generator=g) * 0.01).to(dev).requires_grad_()
        projs.append((packed, qs, a, b))
    x = torch.randn(M, k, generator=g).to(dev, torch.bfloat16).requires_grad_()
    dys = [torch.randn(M, n, generator=g).to(dev, torch.bfloat16) for n in rows]
    leaves = [x] + [t for p in projs for t in p[2:]]

    def stacked():
        for t in leaves:
            t.grad = None
        with torch.autocast("cuda", dtype=torch.bfloat16):
            ys = stacked_nf4_lora(x, [p[0] for p in projs], [p[2] for p in projs], [p[3] for p in projs],
                                  [p[1] for p in projs], s)
        torch.autograd.backward(ys, dys)

    def separate():
        for t in leaves:
            t.grad = None
        with torch.autocast("cuda", dtype=torch.bfloat16):
            ys = [scheduled_nf4_lora(x, p[0], p[2], p[3], p[1], s) for p in projs]
        torch.autograd.backward(ys, dys)

    res = {"proj": "q/k/v stacked", "N": sum(rows), "K": k, "M": M, "r": r}
    flop = sum(4 * M * n * k + 6 * M * r * (n + k) for n in rows)
    for name, fn in (("separate", separate), ("stacked", stacked)):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            fn()
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / reps
        gpu_ms = _graph_ms(fn)
        res[f"{name}_ms_fwd_bwd"] = round(ms, 4)
        res[f"{name}_gpu_ms_fwd_bwd"] = round(gpu_ms, 4)
        log(f"cfg3 q/k/v {name} (N=1536+256+256 K={k} M={M}): fwd+bwd {ms:.3f} ms eager, {gpu_ms:.3f} ms of GPU "
            f"work ({flop / (gpu_ms * 1e-3) / 1e12:.0f} TFLOP/s)")
    return res


def _projection_ops(x, packed, qs, a, b, dy, s):
    """The kernels of one scheduled NF4-LoRA projection, forward and backward,
    as _ScheduledNF4LoRA issues them (methods/nf4_lora.py forward/backward)."""
    from molt_amd import ops
    from molt_amd.nf4 import nibble_order, resolved_nf4_scales

    n, k = b.shape[0], x.shape[1]
    sc, order = resolved_nf4_scales(qs), nibble_order(qs)
    t = ops.direct.lora_project(x, None, 0, 1.0, a, 0)
    ops.direct.nf4_lora_forward(x, packed.reshape(-1), sc, qs.code, n, k, order, 64, t, b, s)
    u = ops.direct.lora_project(dy, None, 2, s, b, 1)
    ops.direct.nf4_lora_backward_input(dy, packed.reshape(-1), sc, qs.code, n, k, order, 64, u, a, 1.0)
    ops.direct.lora_grad(x, None, 0, u, 1.0, 1)
    ops.direct.lora_grad(dy, None, 0, t, s, 0)


def _graph_ms(fn, reps: int = 10, replays: int = 5) -> float:
    """GPU time per call of `fn` with the host out of the way: `reps` calls
    captured in one HIP graph, replayed `replays` times between HIP events."""
    import torch

    fn()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            for _ in range(reps):
                fn()
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(replays):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / (reps * replays)
    del graph
    return ms


def lm_head_bench(dev, steps: int = 5):
    """The frozen LM head of the cfg3 decoder (Qwen2.5-1.5B: vocabulary
    151,936 x hidden 1,536, bf16) over M=4096 tokens in chunks of 256 through
    frozen_linear_cross_entropy: loss and hidden gradient (two hipBLASLt GEMMs
    per chunk, 4*M*V*H FLOPs in all, plus the HIP row reduction); also in one
    chunk of all 4096 rows (1.2 GB of bf16 logits, which the GPU's 288 GB
    hold; the reference's default is no chunking). The row kernel alone is
    timed on one [256, V] chunk against its algorithmic bytes (read the logits
    once, write the gradient once)."""
    import torch
    from molt_amd import ops
    from molt_amd.kernels.frozen_linear_cross_entropy import frozen_linear_cross_entropy

    V, H, M, chunk = 151936, 1536, 4096, 256
    g = torch.Generator(device="cpu").manual_seed(11)
    w = (torch.randn(V, H, generator=g) * 0.02).to(dev, torch.bfloat16)
    h = torch.randn(M, H, generator=g).to(dev, torch.bfloat16).requires_grad_()
    t = torch.randint(0, V, (M,), generator=g).to(dev)

    def run(c):
        h.grad = None
        frozen_linear_cross_entropy(h, w, t, c).backward()

    flop = 4 * M * V * H
    timed = {}
    for c in (chunk, M):
        for _ in range(2):
            run(c)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            run(c)
        torch.cuda.synchronize()
        timed[c] = (time.perf_counter() - t0) * 1e3 / steps
    ms, ms_one = timed[chunk], timed[M]
    tf, tf_one = flop / (ms * 1e-3) / 1e12, flop / (ms_one * 1e-3) / 1e12
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
        f"({100 * gbs / PEAK_HBM_GBS:.1f}% of HBM); one chunk of {M}: {ms_one:.3f} ms, {tf_one:.0f} TFLOP/s "
        f"({100 * tf_one / PEAK_BF16_TFLOPS:.1f}%)")
    return {"vocab": V, "hidden": H, "tokens": M, "chunk": chunk, "ms_loss_and_grad": round(ms, 4),
            "TFLOP_s": round(tf, 1), "frac_bf16_peak": round(tf / PEAK_BF16_TFLOPS, 4),
            "ms_loss_and_grad_one_chunk": round(ms_one, 4), "TFLOP_s_one_chunk": round(tf_one, 1),
            "row_kernel_us_per_chunk": round(us, 2), "row_kernel_GB_s": round(gbs, 1),
            "row_kernel_frac_hbm": round(gbs / PEAK_HBM_GBS, 4)}


# (C entry point, the GEMM kernel it launches at cfg4 (the staged-weight variants), algorithmic FLOPs
# per launch at (M, H, I, r))
GEMMS = (
    ("molt_nf4_gateup_forward", "big::fwd_kernel<true, true> (gate/up forward)",
     lambda M, H, I, r: 2 * (2 * M * H * I) + 2 * (2 * M * I * r)),
    ("molt_nf4_lora_forward", "big::fwd_kernel<false, true> (down forward)",
     lambda M, H, I, r: 2 * M * I * H + 2 * M * H * r),
    ("molt_nf4_swiglu_backward", "big::bwd_kernel<2, true> (down dX + SwiGLU backward)",
     lambda M, H, I, r: 2 * M * H * I + 2 * M * r * I),
    ("molt_nf4_lora_backward_input_pair", "big::bwd_kernel<0, true> (paired gate/up dX)",
     lambda M, H, I, r: 2 * (2 * M * I * H) + 2 * (2 * M * r * H)),
)
TRAFFIC_FILE = ROOT / "profiles" / "gemm_cfg4_hbm_traffic.txt"
COUNTER_FILE = ROOT / "profiles" / "gemm_cfg4_counters.txt"


def _summary_rows(path: Path) -> dict:
    """``kernel | key=value ...`` lines of a committed profile summary, by kernel."""
    rows = {}
    try:
        for line in path.read_text().splitlines():
            if "|" not in line or line.startswith("#"):
                continue
            name, _, rest = line.partition("|")
            rows[name.strip()] = dict(kv.split("=", 1) for kv in rest.split())
    except OSError:
        pass
    return rows


def measured_traffic(kernel: str):
    """HBM bytes per launch of ``kernel`` from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE passes (each scaled by the same counter's reading
    for a copy of known size); None when no such summary is present."""
    row = _summary_rows(TRAFFIC_FILE).get(kernel)
    return int(float(row["traffic_bytes"])) if row and "traffic_bytes" in row else None


def measured_counters() -> dict:
    """MFMA busy fraction per GEMM kernel from the committed rocprofv3 counter
    summary: SQ_VALU_MFMA_BUSY_CYCLES / (SIMDs x GRBM_GUI_ACTIVE per XCD)."""
    return {k: float(v["mfma_busy"]) for k, v in _summary_rows(COUNTER_FILE).items() if "mfma_busy" in v}


PROFILE_DECODE = tuple((n, k, m) for n, k in GEMV_CFG5 for m in (1, 16))


def profile_decode(dev, reps: int) -> None:
    """Decode kernels for counter passes: the NF4 GEMV (r=16 LoRA add-on) at
    each cfg5 shape with M in (1, 16), then the standalone 14336 x 4096
    dequant, `reps` launches each, in that order, one synchronised launch at a
    time. Every launch reads its own copy of the packed weight and absmax
    (copies totalling >= 512 MiB per shape, beyond the 256 MB Infinity Cache),
    so no launch finds another's operands in a cache. Prints one line per
    launch, in dispatch order, naming the case."""
    import ctypes
    import torch
    import molt_amd
    from molt_amd import _lib, ops

    lib = _lib.load()
    g = torch.Generator(device="cpu").manual_seed(5)
    r = 16
    cases = [("gemv", n, k, m) for n, k, m in PROFILE_DECODE] + [("dequant", 14336, 4096, 0)]
    for kind, n, k, m in cases:
        w = (torch.randn(n, k, generator=g) * 0.02).to(dev)
        packed, qs = molt_amd.quantize_4bit(w, blocksize=64, compress_statistics=True)
        del w
        copies = max(reps, math.ceil(512 * 2**20 / (n * k // 2)))
        packs = [packed.reshape(-1).clone() for _ in range(copies)]
        qcopies = [qs.absmax.clone() for _ in range(copies)]
        code, a2, c2 = (qs.code.float().contiguous(), qs.state2.absmax.float().contiguous(),
                        qs.state2.code.float().contiguous())
        descs = [ops._weight(pk, None, code, n, k, 64, 1, qq, a2, c2, float(qs.offset), 256)
                 for pk, qq in zip(packs, qcopies)]
        st = torch.cuda.current_stream().cuda_stream
        if kind == "gemv":
            x = torch.randn(m, k, generator=g).to(dev, torch.bfloat16)
            a = ((torch.rand(r, k, generator=g) * 2 - 1) / math.sqrt(k)).to(dev)
            b = (torch.randn(n, r, generator=g) * 0.01).to(dev)
            t = ops.lora_project(x, None, 0, 1.0, a, 0)
            y = torch.empty(m, n, device=dev, dtype=torch.bfloat16)
            ws_bytes = int(lib.molt_nf4_gemv_workspace(m, n, k))
            ws = torch.zeros(max(ws_bytes, 256), device=dev, dtype=torch.uint8)
        else:
            out = torch.empty(n, k, device=dev, dtype=torch.bfloat16)
        torch.cuda.synchronize()
        for i in range(reps):
            d = descs[(i * (copies // reps)) % copies]   # spread over the copies
            if kind == "gemv":
                _lib.check(lib.molt_nf4_gemv(x.data_ptr(), k, m, ctypes.byref(d), t.data_ptr(), r, b.data_ptr(),
                                             r, 2.0, y.data_ptr(), n, ws.data_ptr(), ws_bytes, st))
            else:
                _lib.check(lib.molt_nf4_dequantize(ctypes.byref(d), out.data_ptr(), _lib.DTYPE_BF16, st))
            torch.cuda.synchronize()
            log(f"decode-case {kind} N={n} K={k} M={m} launch {i}")
        del packs, qcopies, descs
        torch.cuda.empty_cache()


def profile_kernel(which: str, reps: int) -> int:
    """Run one kernel `reps` times at cfg4 shapes, for rocprofv3 passes:
    'gateup' = the fused gate/up NF4-LoRA GEMM, 'step' = whole gated-MLP steps,
    'decode' = the NF4 GEMV at the cfg5 shapes and the standalone dequant,
    'stack' = cfg3 decoder-stack steps, 'hipblaslt' = plain bf16 GEMMs of the
    step's four shapes (the vendor-library ceiling), 'copy' = a 1 GiB device
    copy (1 GiB read + 1 GiB written) that calibrates FETCH_SIZE / WRITE_SIZE."""
    import torch
    from molt_amd import ops

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if which == "copy":
        src = torch.ones(2**30, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(reps):
            dst.copy_(src)
    elif which == "step":
        projs, x, dy, s = make_mlp(4096, 14336, 64, 128.0, 8192, 1337, dev)
        for _ in range(reps):
            mlp_step(projs, x, dy, s)
    elif which == "stack":
        cfg3_stack(dev, steps=reps)
    elif which == "decode":
        profile_decode(dev, reps)
    elif which == "hipblaslt":
        # plain bf16 GEMMs of the cfg4 step's four contractions (hipBLASLt through torch.mm):
        # the vendor-library ceiling for these shapes, without NF4 decode or LoRA
        M, H, I = 8192, 4096, 14336
        g = torch.Generator(device="cpu").manual_seed(21)
        x = torch.randn(M, H, generator=g).to(dev, torch.bfloat16)
        w_gu = torch.randn(H, 2 * I, generator=g).to(dev, torch.bfloat16)      # [K, N] row-major
        h = torch.randn(M, I, generator=g).to(dev, torch.bfloat16)
        w_d = torch.randn(I, H, generator=g).to(dev, torch.bfloat16)
        dy = torch.randn(M, H, generator=g).to(dev, torch.bfloat16)
        w_dt = torch.randn(H, I, generator=g).to(dev, torch.bfloat16)
        dgu = torch.randn(M, 2 * I, generator=g).to(dev, torch.bfloat16)
        w_gut = torch.randn(2 * I, H, generator=g).to(dev, torch.bfloat16)
        shapes = (("gate/up forward", x, w_gu), ("down forward", h, w_d), ("down dX", dy, w_dt),
                  ("paired gate/up dX", dgu, w_gut))
        for _ in range(reps):
            for name, a, b in shapes:
                torch.mm(a, b)
        torch.cuda.synchronize()
        for name, a, b in shapes:
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                torch.mm(a, b)
            e1.record()
            e1.synchronize()
            ms = e0.elapsed_time(e1) / reps
            tf = 2 * a.shape[0] * a.shape[1] * b.shape[1] / (ms * 1e-3) / 1e12
            log(f"hipBLASLt bf16 {name} [{a.shape[0]}x{a.shape[1]}]x[{b.shape[0]}x{b.shape[1]}]: {ms:.3f} ms, "
                f"{tf:.0f} TFLOP/s ({100 * tf / PEAK_BF16_TFLOPS:.1f}% of bf16 peak)")
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
    ap.add_argument("--no-dequant", action="store_true", help="skip the standalone dequant measurement")
    ap.add_argument("--no-stack", action="store_true", help="skip the cfg3 28-layer decoder stack")
    ap.add_argument("--profile-kernel", choices=("gateup", "step", "decode", "stack", "hipblaslt", "copy"),
                    help="only launch one kernel or one gated-MLP step (for rocprofv3 --pmc passes) and exit")
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
    # Events around a launch cost a few µs of GPU idle each (≈ 12 µs a step per
    # timed GEMM with four markers, half that with the two of pre-made event
    # pairs), so the timed steps carry them only for the gate/up forward,
    # the step's longest kernel (twice the FLOPs of any other); the other
    # GEMMs are timed over as many steps again after the timed region.
    lead = GEMMS[0][0]
    probes = {lead: ops.probe_events(lead, reserve=args.steps)}
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        mlp_step(projs, x, dy, s)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ops.probe_events(lead, enable=False)
    rest = {entry: ops.probe_events(entry, reserve=args.steps) for entry, _, _ in GEMMS[1:]}
    for i in range(args.steps):
        mlp_step(projs, x, dy, s)
    torch.cuda.synchronize()
    for entry in rest:
        ops.probe_events(entry, enable=False)
    probes.update(rest)
    ms_step = elapsed * 1e3 / args.steps
    tok_s = M * args.steps / elapsed
    flop_step = (12 * H * I + 18 * r * (H + I)) * M
    step_tflops = flop_step / (ms_step * 1e-3) / 1e12
    counters = measured_counters()
    gemms = []
    for entry, kernel, flop_fn in GEMMS:
        k_ms = statistics.mean(a.elapsed_time(b) for a, b in probes[entry])
        k_flop = flop_fn(M, H, I, r)
        k_tflops = k_flop / (k_ms * 1e-3) / 1e12
        gemms.append({"entry": entry, "kernel": kernel, "avg_launch_ms": round(k_ms, 4),
                      "launches": len(probes[entry]), "flop_per_launch": k_flop, "achieved": round(k_tflops, 1),
                      "frac": round(k_tflops / PEAK_BF16_TFLOPS, 4), "mfma_busy": counters.get(kernel)})
        log(f"{kernel}: {k_ms:.3f} ms = {k_tflops:.1f} TFLOP/s ({100 * k_tflops / PEAK_BF16_TFLOPS:.1f}%)")
    dominant = max(gemms, key=lambda g: g["avg_launch_ms"])
    log(f"step {ms_step:.3f} ms, {tok_s:.0f} tok/s, {step_tflops:.1f} TFLOP/s "
        f"({100 * step_tflops / PEAK_BF16_TFLOPS:.1f}% of bf16 peak); dominant kernel {dominant['kernel']}")

    result = {
        "metric": METRIC, "value": round(tok_s, 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic (seeded N(0,0.02) weights NF4-quantised, N(0,1) X/dY)",
        "config": {"workload": "cfg4: Llama-3-8B-shaped NF4-LoRA gated MLP fwd+bwd incl. dA/dB",
                   "hidden": H, "intermediate": I, "lora_rank": r, "lora_alpha": alpha, "tokens": M,
                   "nf4_block": 64, "double_quant": True, "parallelism": "single GPU"},
        "step_frac_of_bf16_peak": round(step_tflops / PEAK_BF16_TFLOPS, 4),
        "step_tflops": round(step_tflops, 1),
        "roofline": {"kernel": dominant["kernel"], "bound": "mfma", "achieved": dominant["achieved"],
                     "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s", "frac": dominant["frac"],
                     "traffic": measured_traffic(dominant["kernel"]),
                     "traffic_unit": "bytes/launch (rocprofv3 FETCH_SIZE+WRITE_SIZE, copy-calibrated)",
                     "avg_launch_ms": dominant["avg_launch_ms"], "launches": dominant["launches"],
                     "flop_per_launch": dominant["flop_per_launch"], "mfma_busy": dominant["mfma_busy"]},
        "gemm_kernels": gemms,
    }
    del probes
    if not args.no_dequant:
        result["dequant"] = dequant_bench(dev)
    if not args.no_norm:
        result["rmsnorm"] = rmsnorm_bench(dev, projs, dy, s, M, H, args.steps)
    if not args.no_proj:
        result["cfg3_projections"] = projection_sweep(dev)
    if not args.no_head:
        result["lm_head"] = lm_head_bench(dev)
    if not args.no_stack:
        del projs, x, dy
        torch.cuda.empty_cache()
        result["cfg3_stack"] = cfg3_stack(dev)
    if not args.no_gemv:
        sweep = gemv_sweep(dev)
        result["gemv"] = sweep
        result["gemv_best_frac_hbm"] = max(e["frac_hbm"] for e in sweep if e["set"] == "cfg5")
    if not args.no_cpu:
        result["cfg1_gpu"] = cfg1_gpu(dev)
        log("cpu baseline (cfg1, oracle restatement, numpy fp32)")
        result["cpu_baseline"] = cpu_baseline()
        result["cpu_baseline"]["gpu_speedup_cfg1"] = round(result["cfg1_gpu"]["tokens_s"] /
                                                           result["cpu_baseline"]["value"], 1)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
