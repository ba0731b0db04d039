"""CPU baseline (TEST INFRASTRUCTURE, used only by bench.py's cpu_baseline leg).

One gated NF4-LoRA MLP forward+backward in numpy float32 on the host, as
MOLT's only CPU-capable NF4 path computes it: every step decodes the NF4
weights to fp32 (streaming/engine.py:36; streaming/nf4.py:29-35) and runs the
eager LoRA algebra of streaming/engine.py:21-48 around the SwiGLU of
kernels/gated_activation.py:29-51.
"""
from __future__ import annotations

import numpy as np

from . import nf4_oracle as O


def _silu(g):
    return g / (np.float32(1.0) + np.exp(-g))


def gated_mlp_step_f32(x, weights, adapters, s, dy):
    """weights: three OracleNF4 (gate, up, down); adapters: three (A, B) fp32.
    Returns dX and the six adapter gradients (all fp32)."""
    s = np.float32(s)
    wg, wu, wd = (w.dequant_f32() for w in weights)
    (ag, bg), (au, bu), (ad, bd) = adapters
    tg, tu = x @ ag.T, x @ au.T
    g = x @ wg.T + s * (tg @ bg.T)
    u = x @ wu.T + s * (tu @ bu.T)
    sg = _silu(g)
    h = sg * u
    td = h @ ad.T
    _y = h @ wd.T + s * (td @ bd.T)
    wg, wu, wd = (w.dequant_f32() for w in weights)   # the eager backward re-decodes
    ud = s * (dy @ bd)
    dh = dy @ wd + ud @ ad
    sig = np.float32(1.0) / (np.float32(1.0) + np.exp(-g))
    dgate = dh * u * sig * (np.float32(1.0) + g * (np.float32(1.0) - sig))
    dup = dh * sg
    ug, uu = s * (dgate @ bg), s * (dup @ bu)
    dx = dgate @ wg + ug @ ag + dup @ wu + uu @ au
    grads = (ug.T @ x, s * (dgate.T @ tg), uu.T @ x, s * (dup.T @ tu), ud.T @ h, s * (dy.T @ td))
    return dx, grads
