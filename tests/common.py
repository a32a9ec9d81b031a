"""Shared helpers for the tests: seeded synthetic blocks and the oracle view of them.

Weights are drawn from N(0, 0.02) and activations from N(0, 1) with numpy's PCG64
(`np.random.default_rng(seed)`), which gives the same stream on every platform.
"""
from __future__ import annotations

import numpy as np

from oracle import oracle as O

KEYS = ("router", "gate", "up", "down", "sgate", "sup", "sdown", "seg")


def shapes(H, E, I, Is):
    s = {"router": (E, H), "gate": (E, I, H), "up": (E, I, H), "down": (E, H, I)}
    if Is > 0:
        s.update({"sgate": (Is, H), "sup": (Is, H), "sdown": (H, Is), "seg": (1, H)})
    return s


def make_f32_block(seed, H, E, I, Is, std=0.02):
    rng = np.random.default_rng(seed)
    return {k: (rng.standard_normal(shp, dtype=np.float32) * np.float32(std)) for k, shp in shapes(H, E, I, Is).items()}


def make_x(seed, T, H):
    rng = np.random.default_rng(seed + 7919)
    return rng.standard_normal((T, H), dtype=np.float32)


def bf16_bits(a: np.ndarray) -> np.ndarray:
    """round-to-nearest-even f32 -> bf16 bits (vectorised; NaN-free inputs)"""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = u + 0x7FFF + ((u >> 16) & 1)
    return (u >> 16).astype(np.uint16)


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return O.bf16_bits_to_f32(b)


def store(w: dict, formats: dict) -> dict:
    """Convert f32 weights to their storage formats. formats maps key -> dtype."""
    out = {}
    for k, a in w.items():
        dt = formats.get(k, O.F32)
        if dt == O.F32:
            out[k] = (dt, np.ascontiguousarray(a, dtype=np.float32))
        elif dt == O.BF16:
            out[k] = (dt, bf16_bits(a))
        else:
            out[k] = (dt, O.quantize(dt, a))
    return out


def oracle_block(cfg, stored, act_dtype):
    H, E, k, I, Is, norm = cfg
    return O.OracleMoe(H, E, k, I, Is, norm, act_dtype, stored)


C1 = dict(H=256, E=16, k=4, I=128, Is=128, norm=True, T=32)


def rel_err(got, ref):
    """normwise max|got-ref| / max|ref| (the parity gate)"""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30))


def errors(got, ref):
    """the three figures reported for a float output: normwise
    max|y-r| / max|r| (the gate), cosine, and elementwise
    max |y-r| / (|r| + 1e-3 max|r|)"""
    got = np.asarray(got, np.float64).ravel()
    ref = np.asarray(ref, np.float64).ravel()
    m = max(np.abs(ref).max(), 1e-30)
    return {"normwise": float(np.abs(got - ref).max() / m),
            "cosine": float(got @ ref / max(np.linalg.norm(got) * np.linalg.norm(ref), 1e-300)),
            "elementwise": float((np.abs(got - ref) / (np.abs(ref) + 1e-3 * m)).max())}


def report(tag, got, ref):
    e = errors(got, ref)
    print(f"[err] {tag}: normwise {e['normwise']:.3e} cosine {e['cosine']:.7f} elementwise {e['elementwise']:.3e}",
          flush=True)
    return e


def mfma_routing(T, H, E, k, norm, act_bf16, router_bf16):
    """whether a route / forward of T tokens takes the prefill routing whose
    router GEMM runs on MFMA: ids and permutation bit-exact, the renormalised
    weights exp(l_r - max) / sum over the selected (the softmax denominator
    cancels) within a few ulps of the reference's p_r / sum p"""
    return (T > 8 and act_bf16 and router_bf16 and norm and H % 32 == 0 and 32 <= H <= 4096
            and E <= 1024 and k <= 64)


def assert_topk_w(got, ref, k, exact):
    """routing weights: bit-exact, or (MFMA routing) within (4k + 8) u of the
    reference relative to each weight, u = 2^-24 -- twice the rounding steps
    of the two formulas"""
    got = np.asarray(got, np.float32)
    ref = np.asarray(ref, np.float32)
    if exact:
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
        return
    rel = np.abs(got.astype(np.float64) - ref) / np.maximum(np.abs(ref.astype(np.float64)), 1e-30)
    assert float(rel.max()) <= (4 * k + 8) * 2.0 ** -24, float(rel.max())
