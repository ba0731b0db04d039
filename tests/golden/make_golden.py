"""Writes the golden fixtures under tests/golden/ from the CPU oracle.

Run from the repository root: ``python tests/golden/make_golden.py``.

The reference (PraveenNimilka/MOLT) stores no vectors for this path: its
hot-path tests are differential against bitsandbytes on CUDA at run time. These
fixtures are therefore produced by this repository's oracle, itself pinned by
``tests/test_oracle.py``, and freeze its outputs on small seeded cases. The
shapes follow the reference tests: the 64 x 64 NF4 storage test
(tests/test_molt_stream_nf4.py:9-15), the 70 x 65-style tails
(tests/kernels/test_nf4_lora.py:106-121), the (in, out) = (64, 96), r = 8
linear (tests/kernels/test_nf4_lora.py:14-45) and the (hidden, intermediate) =
(64, 96), M = 32, r = 8, s = 2 gated MLP (tests/kernels/test_gated_replay.py:11-114).

Each fixture records the nibble order and the state2 code table it uses.
Inputs are drawn with numpy's PCG64 from fixed seeds; activations are stored
as bf16 bit patterns, expected results as fp32 (rounded once from fp64).
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import nf4_oracle as O  # noqa: E402

CODEC_CASES = [
    # name, shape, block, layout ("bnb" nested / high nibble first, "clean" fp32 absmax / low first)
    ("bnb_64x64", (64, 64), 64, "bnb"),
    ("clean_70x66", (70, 66), 64, "clean"),
    ("bnb_32x1024", (32, 1024), 64, "bnb"),
    ("clean_48x40_b16", (48, 40), 16, "clean"),
]


def _quantize(w: np.ndarray, block: int, layout: str) -> O.OracleNF4:
    if layout == "bnb":
        return O.quantize_bnb_layout(w, block, nested=True)
    idx, absmax = O.quantize_blocks(w, block)
    return O.OracleNF4(O.pack_nibbles(idx, O.NIBBLE_LOW_FIRST), tuple(w.shape), block,
                       O.NIBBLE_LOW_FIRST, O.NF4_CODE.copy(), absmax, absmax)


def codec_arrays(name: str, shape, block: int, layout: str, rng) -> dict:
    w = (rng.standard_normal(shape, dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    t = _quantize(w, block, layout)
    out = {
        f"{name}/w": w,
        f"{name}/block": np.int32(block),
        f"{name}/order": np.int32(t.order),
        f"{name}/packed": t.packed,
        f"{name}/absmax": t.absmax,
        f"{name}/scales": t.scales,
        f"{name}/dequant_bf16_bits": t.dequant_bf16_bits(),
    }
    if t.nested:
        out.update({f"{name}/q": t.q, f"{name}/absmax2": t.absmax2, f"{name}/code2": t.code2,
                    f"{name}/offset": np.float32(t.offset)})
    return out


def _bf16_bits(x: np.ndarray) -> np.ndarray:
    return O.bf16_rne_bits(np.asarray(x, np.float32))


def _weight(rng, out_f: int, in_f: int) -> tuple[np.ndarray, O.OracleNF4]:
    w = (rng.standard_normal((out_f, in_f), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    return w, O.quantize_bnb_layout(w, 64, nested=True)


def _adapter(rng, out_f: int, in_f: int, r: int):
    bound = 1.0 / np.sqrt(in_f)
    a = rng.uniform(-bound, bound, (r, in_f)).astype(np.float32)
    b = (rng.standard_normal((out_f, r)) * 0.01).astype(np.float32)
    return a, b


def linear_arrays(rng) -> dict:
    """One NF4+LoRA linear: in 64, out 96, r 8, s 2, M 37 (a row tail)."""
    m, k, n, r, s = 37, 64, 96, 8, 2.0
    _, t = _weight(rng, n, k)
    a, b = _adapter(rng, n, k, r)
    x = _bf16_bits(rng.standard_normal((m, k)).astype(np.float32))
    dy = _bf16_bits(rng.standard_normal((m, n)).astype(np.float32))
    xv, dyv = O.bf16_bits_to_f32(x), O.bf16_bits_to_f32(dy)
    wv = t.dequant_bf16().astype(np.float64)
    a16, b16 = O.bf16_round(a), O.bf16_round(b)
    y = O.lora_linear_forward(xv, wv, a16, b16, s)
    dx, da, db = O.lora_linear_backward(xv, wv, a16, b16, s, dyv)
    return {
        "linear/packed": t.packed, "linear/q": t.q, "linear/absmax2": t.absmax2,
        "linear/code2": t.code2, "linear/offset": np.float32(t.offset),
        "linear/lora_a": a, "linear/lora_b": b, "linear/scaling": np.float32(s),
        "linear/x_bf16_bits": x, "linear/dy_bf16_bits": dy,
        "linear/y": y.astype(np.float32), "linear/dx": dx.astype(np.float32),
        "linear/da": da.astype(np.float32), "linear/db": db.astype(np.float32),
    }


def mlp_arrays(rng) -> dict:
    """Gated MLP: hidden 64, intermediate 96, r 8, s 2, M 32."""
    h, i, r, m, s = 64, 96, 8, 32, 2.0
    out = {"mlp/scaling": np.float32(s)}
    deq, adapters = [], []
    for name, (o, k) in (("gate", (i, h)), ("up", (i, h)), ("down", (h, i))):
        _, t = _weight(rng, o, k)
        a, b = _adapter(rng, o, k, r)
        out.update({f"mlp/{name}/packed": t.packed, f"mlp/{name}/q": t.q,
                    f"mlp/{name}/absmax2": t.absmax2, f"mlp/{name}/code2": t.code2,
                    f"mlp/{name}/offset": np.float32(t.offset), f"mlp/{name}/lora_a": a,
                    f"mlp/{name}/lora_b": b})
        deq.append(t.dequant_bf16().astype(np.float64))
        adapters.append((O.bf16_round(a), O.bf16_round(b)))
    x = _bf16_bits(rng.standard_normal((m, h)).astype(np.float32))
    dy = _bf16_bits(rng.standard_normal((m, h)).astype(np.float32))
    xv, dyv = O.bf16_bits_to_f32(x), O.bf16_bits_to_f32(dy)
    (ag, bg), (au, bu), (ad, bd) = adapters
    y, saved = O.gated_mlp_forward(xv, deq[0], deq[1], deq[2], ag, bg, au, bu, ad, bd, s)
    dx, grads = O.gated_mlp_backward(xv, deq[0], deq[1], deq[2], ag, bg, au, bu, ad, bd, s, dyv, saved)
    out.update({"mlp/x_bf16_bits": x, "mlp/dy_bf16_bits": dy, "mlp/y": y.astype(np.float32),
                "mlp/dx": dx.astype(np.float32)})
    for key, g in zip(("da_gate", "db_gate", "da_up", "db_up", "da_down", "db_down"), grads):
        out[f"mlp/{key}"] = g.astype(np.float32)
    return out


def build() -> dict[str, dict]:
    codec: dict = {}
    for seed, (name, shape, block, layout) in enumerate(CODEC_CASES):
        codec.update(codec_arrays(name, shape, block, layout, np.random.default_rng(1000 + seed)))
    return {"nf4_codec.npz": codec,
            "nf4_lora_linear.npz": linear_arrays(np.random.default_rng(2000)),
            "gated_mlp.npz": mlp_arrays(np.random.default_rng(3000))}


def main() -> None:
    for fname, arrays in build().items():
        np.savez_compressed(HERE / fname, **arrays)
        print(f"wrote {fname}: {len(arrays)} arrays, {(HERE / fname).stat().st_size} bytes")


if __name__ == "__main__":
    main()
