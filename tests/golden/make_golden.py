"""Writes the golden fixtures of this directory: seeded inputs of each config
at small shapes and the expected outputs, computed in float64 by the numpy
restatement under ``oracle/`` (never by importing the reference).

Run from the repository root: ``python tests/golden/make_golden.py``.
``generate(name)`` returns a fixture's arrays without writing, so the tests
can check that the committed files still follow from their seeds.

Storage: fp32 arrays as float32; bf16 arrays as their raw 16-bit patterns
(uint16, suffix ``__bf16``); expected outputs as float32 (the rounding of the
float64 result is 6e-8 relative, far inside the 1e-5 / 2e-2 gates).

Fixtures (the small shapes of the five configs, plus the dense affine scan
and the deferred-affine attention):

* ``c1_weight_chain``: 8 stacked ``Linear(128, 128)``, ``x (64, 128)``, fp32;
* ``c2_swiglu``: rms_norm + SwiGLU, ``x (1, 64, 256)``, F = 512, bf16;
* ``c3_causal_attention``: ``q, k, v (1, 1, 256, 128)``, causal, bf16;
* ``c4_retention``: ``q, k, v (1, 2, 256, 128)``, C = 64 (K = 4), γ fp32, bf16;
* ``c5_ssm``: ``a (2, 256, 16, 16)``, ``bx, c (2, 256, 16)``, ``x (2, 256, 16)``,
  ``h (2, 16, 16)``, fp32;
* ``aff_linear_recurrence``: shared ``A (16, 16)``, ``b (32, 4, 16, 1)``, ``h (4, 16, 1)``, fp32;
* ``omd_scan_attention``: 16 queries over the 128 states of a diagonal scan
  (d = 16, 4 key blocks, dk = 16), fp32.
"""

from __future__ import annotations

import math
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

import oracle  # noqa: E402

BF16 = "__bf16"


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 → bf16 bit patterns, round to nearest even (NaN-free inputs)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    rounded = u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))
    return (rounded >> np.uint32(16)).astype(np.uint16)


def from_bf16_bits(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def _bf16(x: np.ndarray) -> np.ndarray:
    """The bf16 value of ``x`` as float32 (what the fixture stores)."""
    return from_bf16_bits(to_bf16_bits(x))


def _f32(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, dtype=np.float32)


def _c1(rng):
    L, d, rows = 8, 128, 64
    bound = 1.0 / math.sqrt(d)  # nn.Linear's default U(±1/√in) for W and b
    ins = {"x": _f32(rng.standard_normal((rows, d)))}
    for i in range(L):
        ins[f"W{i + 1}"] = _f32(rng.uniform(-bound, bound, (d, d)))
        ins[f"b{i + 1}"] = _f32(rng.uniform(-bound, bound, d))
    y = oracle.linear_chain(ins["x"].astype(np.float64), [ins[f"W{i + 1}"].astype(np.float64) for i in range(L)],
                            [ins[f"b{i + 1}"].astype(np.float64) for i in range(L)])
    return ins, {"y": y}, {"L": L, "d": d, "rows": rows}, ()


def _c2(rng):
    rows, D, F = (1, 64), 256, 512
    ins = {"x": _bf16(rng.standard_normal((*rows, D))),
           "gamma": _bf16(1.0 + 0.02 * rng.standard_normal(D)),
           "W_gate": _bf16(0.02 * rng.standard_normal((F, D))),
           "W_up": _bf16(0.02 * rng.standard_normal((F, D))),
           "W_down": _bf16(0.02 * rng.standard_normal((D, F)))}
    f64 = {k: v.astype(np.float64) for k, v in ins.items()}
    h = oracle.rms_norm(f64["x"], f64["gamma"], 1e-6)
    y = oracle.swiglu_fused(h, f64["W_gate"], f64["W_up"], f64["W_down"])
    return ins, {"y": y}, {"rows": rows, "D": D, "F": F, "eps": 1e-6}, tuple(ins)


def _c3(rng):
    B, H, T, d = 1, 1, 256, 128
    ins = {n: _bf16(rng.standard_normal((B, H, T, d))) for n in "qkv"}
    y = oracle.attention_om(*(ins[n].astype(np.float64) for n in "qkv"), 1.0 / math.sqrt(d), causal=True)
    return ins, {"y": y}, {"B": B, "H": H, "T": T, "d": d}, tuple(ins)


def _c4(rng):
    B, H, T, d, C = 1, 2, 256, 128, 64
    ins = {n: _bf16(rng.standard_normal((B, H, T, d)) / math.sqrt(d)) for n in "qkv"}
    ins["gamma"] = _f32([1.0 - 2.0 ** (-5 - h / 2) for h in range(H)])
    y = oracle.retention_kway(*(ins[n].astype(np.float64) for n in "qkv"), ins["gamma"].astype(np.float64), T // C)
    return ins, {"y": y}, {"B": B, "H": H, "T": T, "d": d, "C": C}, ("q", "k", "v")


def _c5(rng):
    B, T, D, N = 2, 256, 16, 16
    z = rng.standard_normal((B, T, D, N))
    ins = {"a": _f32(1.0 / (1.0 + np.exp(z))),  # exp(-softplus(z))
           "bx": _f32(rng.standard_normal((B, T, N))), "c": _f32(rng.standard_normal((B, T, N))),
           "x": _f32(rng.standard_normal((B, T, D))), "h": _f32(rng.standard_normal((B, D, N)))}
    y, _ = oracle.ssm_serial(*(ins[n].astype(np.float64) for n in ("a", "bx", "c", "x", "h")))
    return ins, {"y": y}, {"B": B, "T": T, "D": D, "N": N}, ()


def _aff(rng):
    T, d, B = 32, 16, 4
    ins = {"A": _f32(rng.standard_normal((d, d)) * (0.9 / math.sqrt(d))),
           "b": _f32(rng.standard_normal((T, B, d, 1))), "h": _f32(rng.standard_normal((B, d, 1)))}
    states = oracle.serial_aff_scan(ins["A"].astype(np.float64), ins["b"][..., 0].astype(np.float64),
                                    ins["h"].astype(np.float64))
    return ins, {"y": states[-1]}, {"T": T, "d": d, "B": B}, ()


def _omd(rng):
    T, d, Tq, blocks, dk = 128, 16, 16, 4, 16
    ins = {"q": _f32(rng.standard_normal((Tq, dk)) * 0.5), "k": _f32(rng.standard_normal((T, dk)) * 0.5),
           "a": _f32(rng.uniform(0.6, 1.0, (T, d))), "x": _f32(rng.standard_normal((T, d))),
           "h": _f32(rng.standard_normal(d))}
    f64 = {k: v.astype(np.float64) for k, v in ins.items()}
    states = oracle.serial_affd_scan(f64["a"], f64["x"], f64["h"])
    s = f64["q"] @ f64["k"].T
    w = np.exp(s - s.max(-1, keepdims=True))
    y = (w / w.sum(-1, keepdims=True)) @ states
    return ins, {"y": y}, {"T": T, "d": d, "Tq": Tq, "blocks": blocks, "dk": dk}, ()


#: name → (seed, builder)
FIXTURES = {
    "c1_weight_chain": (101, _c1),
    "c2_swiglu": (102, _c2),
    "c3_causal_attention": (103, _c3),
    "c4_retention": (104, _c4),
    "c5_ssm": (105, _c5),
    "aff_linear_recurrence": (106, _aff),
    "omd_scan_attention": (107, _omd),
}


def generate(name: str) -> dict:
    """``{"inputs": {name: float32 array}, "expected": {...}, "meta": {...},
    "bf16": (input names held in bf16), "seed": int}``."""
    seed, build = FIXTURES[name]
    ins, exp, meta, bf16 = build(np.random.default_rng(seed))
    return {"inputs": ins, "expected": {k: _f32(v) for k, v in exp.items()}, "meta": meta,
            "bf16": tuple(bf16), "seed": seed}


def path_of(name: str) -> Path:
    return HERE / f"{name}.npz"


def save(name: str, fx: dict) -> None:
    arrays = {"seed": np.asarray(fx["seed"], dtype=np.int64),
              "meta": np.asarray(repr(fx["meta"]))}
    for k, v in fx["inputs"].items():
        if k in fx["bf16"]:
            arrays[f"in_{k}{BF16}"] = to_bf16_bits(v)
        else:
            arrays[f"in_{k}"] = _f32(v)
    for k, v in fx["expected"].items():
        arrays[f"out_{k}"] = _f32(v)
    np.savez_compressed(path_of(name), **arrays)


def load(name: str) -> dict:
    """A committed fixture, with bf16 inputs widened to float32 (exact)."""
    with np.load(path_of(name), allow_pickle=False) as z:
        ins, exp, bf16 = {}, {}, []
        for key in z.files:
            if key.startswith("in_"):
                k = key[3:]
                if k.endswith(BF16):
                    k = k[:-len(BF16)]
                    bf16.append(k)
                    ins[k] = from_bf16_bits(z[key])
                else:
                    ins[k] = z[key]
            elif key.startswith("out_"):
                exp[key[4:]] = z[key]
        return {"inputs": ins, "expected": exp, "bf16": tuple(bf16), "seed": int(z["seed"]),
                "meta": str(z["meta"])}


def main() -> None:
    for name in FIXTURES:
        fx = generate(name)
        save(name, fx)
        print(f"{path_of(name).relative_to(ROOT)}: {path_of(name).stat().st_size} bytes")


if __name__ == "__main__":
    main()
