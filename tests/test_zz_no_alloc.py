"""molt_nf4_gemv_noalloc (the GEMV entry point that allocates nothing: its
split-K partials live in a static per-device array) against molt_nf4_gemv with
a caller workspace, both called through the C ABI: bitwise equal outputs on two
calls in a row, the second with a smaller problem, plus the fp64 oracle on the
first. The shapes use the split-K path (K = 14336), which is the one that needs
scratch memory."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest
import torch

from tests._util import assert_close_fro, bf16_values, np_f32, oracle_weight, seeded, uniform

import molt_amd
from molt_amd import _lib, ops

pytestmark = pytest.mark.gpu


def _problem(m, n, k, r, seed):
    w = seeded((n, k), seed, std=0.02, dtype=torch.float32)
    packed, qs = molt_amd.quantize_4bit(w, blocksize=64, compress_statistics=True)
    del w
    x = seeded((m, k), seed + 1)
    a = uniform((r, k), seed + 2, 1.0 / np.sqrt(k))
    b = seeded((n, r), seed + 3, std=0.01, dtype=torch.float32)
    t = ops.lora_project(x, None, 0, 1.0, a, 0)
    return packed.reshape(-1), qs, x, t, b


def _descriptor(packed, qs):
    s2 = qs.state2
    return ops._weight(packed, None, qs.code.float().contiguous(), int(qs.shape[0]), int(qs.shape[1]), 64, 1,
                       qs.absmax.contiguous(), s2.absmax.float().contiguous(), s2.code.float().contiguous(),
                       float(qs.offset), int(s2.blocksize))


def _run(noalloc, packed, qs, x, t, b, s):
    lib = _lib.load()
    m, k = x.shape
    n, r = b.shape
    w = _descriptor(packed, qs)
    y = torch.empty((m, n), device="cuda", dtype=torch.bfloat16)
    stream = torch.cuda.current_stream().cuda_stream
    if noalloc:
        rc = lib.molt_nf4_gemv_noalloc(x.data_ptr(), k, m, C.byref(w), t.data_ptr(), r, b.data_ptr(), r, s,
                                       y.data_ptr(), n, stream)
    else:
        need = int(lib.molt_nf4_gemv_workspace(m, n, k))
        ws = torch.empty(max(need, 16), device="cuda", dtype=torch.uint8)
        rc = lib.molt_nf4_gemv(x.data_ptr(), k, m, C.byref(w), t.data_ptr(), r, b.data_ptr(), r, s, y.data_ptr(),
                               n, ws.data_ptr(), need, stream)
    _lib.check(rc)
    torch.cuda.synchronize()
    return y


def test_noalloc_gemv_matches_workspace_gemv_on_two_calls():
    lib = _lib.load()
    s = 2.0
    cases = [(16, 4096, 14336, 16, 700), (3, 1024, 14336, 16, 710), (1, 2048, 4096, 16, 720)]
    assert int(lib.molt_nf4_gemv_workspace(16, 4096, 14336)) > int(lib.molt_nf4_gemv_workspace(3, 1024, 14336)) > 0
    for i, (m, n, k, r, seed) in enumerate(cases):
        print(f"no-alloc GEMV call {i}: M={m} N={n} K={k} r={r}", flush=True)
        packed, qs, x, t, b = _problem(m, n, k, r, seed)
        got = _run(True, packed, qs, x, t, b, s)
        want = _run(False, packed, qs, x, t, b, s)
        assert torch.equal(got, want), f"call {i}: the no-alloc GEMV differs from the workspace GEMV"
        if i == 0:
            wo = oracle_weight(packed, qs).dequant_bf16().astype(np.float64)
            ref = bf16_values(x) @ wo.T + s * (bf16_values(t) @ bf16_values(b).T)
            assert_close_fro(np_f32(got), ref, what="no-alloc GEMV vs oracle")
    # the first shape again after the smaller ones: the shared scratch keeps no state that matters
    packed, qs, x, t, b = _problem(*cases[0][:4], 730)
    assert torch.equal(_run(True, packed, qs, x, t, b, s), _run(False, packed, qs, x, t, b, s))


def test_noalloc_gemv_calls_on_two_streams_are_ordered():
    """No-alloc calls alternating between two streams with no host
    synchronisation between them all use the one scratch array; the entry point
    orders each call after the previous one from another stream, so every
    output equals its workspace-path result bit for bit."""
    lib = _lib.load()
    s = 2.0
    probs = [_problem(16, 4096, 14336, 16, 740 + 10 * i) for i in range(4)]
    want = [_run(False, *p, s) for p in probs]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    torch.cuda.synchronize()
    descs, outs = [], []
    for i, (packed, qs, x, t, b) in enumerate(probs):
        m, k = x.shape
        n, r = b.shape
        print(f"no-alloc GEMV on stream {i % 2}: M={m} N={n} K={k}", flush=True)
        w = _descriptor(packed, qs)
        y = torch.empty((m, n), device="cuda", dtype=torch.bfloat16)
        descs.append(w)
        outs.append(y)
        _lib.check(lib.molt_nf4_gemv_noalloc(x.data_ptr(), k, m, C.byref(w), t.data_ptr(), r, b.data_ptr(), r, s,
                                             y.data_ptr(), n, streams[i % 2].cuda_stream))
    torch.cuda.synchronize()
    for i, (got, ref) in enumerate(zip(outs, want)):
        assert torch.equal(got, ref), f"call {i} on stream {i % 2} differs from the workspace GEMV"
