"""CPU check of the error bound the MFMA prefill routing relies on
(csrc/hx_route_mfma.hip, header): for bf16 token rows x and router rows r,

    |c - m| <= eps = 1.01 u (130 + H/32 + 8 ceil(H/512)) |x| |r|,   u = 2^-24,

where c is the canonical logit (the oracle's fmaf chain over groups of 8 in
lane order plus the xor butterfly, before the bf16 rounding) and m the MFMA
router's value: each K chunk of 32 exact products summed by the matrix unit
from zero (each internal addition allowed a relative error of 4u), the chunk
results added to an f32 running sum.

The matrix unit is simulated here by accumulators at least as bad as the
bound allows: one that truncates every partial sum toward zero, and one that
moves every partial sum by 4u of its magnitude in one direction (products
ordered so the partial sums are as large as possible). The bound must hold
for both on random and cancellation-heavy inputs; a bound without the chunk
term or without the running-sum term must fail for some input, so the check
pins each term of the derivation rather than restating the formula."""
import math

import numpy as np
import pytest

from oracle import oracle as O

U = 2.0 ** -24


def bf16_round(a):
    return O.bf16_bits_to_f32(O.f32_to_bf16_bits(np.asarray(a, dtype=np.float32)))


def canonical(x, r):
    """the oracle's canonical logits [T][E] (f32 activations, so no bf16 rounding
    of the sum; the inputs are bf16 values, as on the MFMA path)"""
    H, E = x.shape[1], r.shape[0]
    blk = O.OracleMoe(H, E, 1, 8, 0, True, O.F32, {"router": (O.F32, r.astype(np.float32))})
    return blk.logits(x.astype(np.float32)).astype(np.float64)


def f32_rtz(s):
    """round float64 values to f32 toward zero"""
    f = s.astype(np.float32)
    over = np.abs(f.astype(np.float64)) > np.abs(s)
    f[over] = np.nextafter(f[over], np.float32(0))
    return f


def mfma_sim(x, r, mode):
    """the router's m for every (token, row): chunks of 32 products summed from
    zero by a simulated matrix unit, then added to an f32 running sum (RNE)"""
    T, H = x.shape
    E = r.shape[0]
    p = x.astype(np.float64)[:, None, :] * r.astype(np.float64)[None, :, :]   # exact bf16 products
    p = p.reshape(T, E, H // 32, 32)
    if mode == "adverse":
        # largest magnitudes first, signs kept: partial sums as large as possible
        order = np.argsort(-np.abs(p), axis=-1)
        p = np.take_along_axis(p, order, axis=-1)
    acc = np.zeros(p.shape[:-1], dtype=np.float64)
    for j in range(32):
        s = acc + p[..., j]
        if mode == "truncate":
            acc = f32_rtz(s).astype(np.float64)
        else:   # every partial sum moved up by 4u of its magnitude
            acc = (s + 4.0 * U * np.abs(s)).astype(np.float64)
    run = np.zeros((T, E), dtype=np.float32)
    for c in range(H // 32):
        run = (run + acc[:, :, c].astype(np.float32)).astype(np.float32)
    return run.astype(np.float64)


def bound(x, r, chunk_term=130.0, running_term=True):
    H = x.shape[1]
    k = chunk_term + (H / 32 if running_term else 0.0) + 8 * math.ceil(H / 512)
    nx = np.linalg.norm(x.astype(np.float64), axis=1)
    nr = np.linalg.norm(r.astype(np.float64), axis=1)
    return 1.01 * U * k * nx[:, None] * nr[None, :]


def inputs(kind, T, E, H, seed):
    rng = np.random.default_rng(seed)
    if kind == "random":
        x = rng.standard_normal((T, H))
        r = rng.normal(0, 0.02, (E, H))
    elif kind == "aligned":
        # router rows parallel to the tokens, positive products: no cancellation,
        # the running sum grows over the whole row
        x = np.abs(rng.standard_normal((T, H))) + 0.5
        r = np.repeat((x[:1] * 0.02), E, axis=0) * (1 + 0.01 * rng.standard_normal((E, H)))
    else:   # "cancel": pairs of large opposite products and a small remainder
        x = rng.standard_normal((T, H))
        r = rng.normal(0, 0.02, (E, H))
        r[:, 1::2] = -r[:, 0::2] * x[:1, 0::2] / np.where(x[:1, 1::2] == 0, 1, x[:1, 1::2])
    return bf16_round(x), bf16_round(r)


@pytest.mark.parametrize("H", [1024, 2048, 4096])
@pytest.mark.parametrize("kind", ["random", "aligned", "cancel"])
def test_bound_holds_for_adversarial_accumulators(H, kind):
    x, r = inputs(kind, 6, 12, H, 100 + H)
    c = canonical(x, r)
    eps = bound(x, r)
    for mode in ("truncate", "adverse"):
        m = mfma_sim(x, r, mode)
        assert np.all(np.abs(c - m) <= eps), (mode, float(np.max(np.abs(c - m) / eps)))


def test_each_term_of_the_bound_is_needed():
    """the chunk term: with one dominant product at the head of every chunk (and
    router rows parallel to the token, so S = |x| |r|), the 4u-per-addition
    accumulator breaks a bound that keeps only the canonical chain's term; the
    running-sum term: the f32 sum of H/32 chunk results is off by at most
    u (H/32) S, and by all of it for chunk results that tie at every addition"""
    rng = np.random.default_rng(8)
    H = 1024
    x = np.abs(rng.standard_normal((6, H))) * 0.05 + 0.01
    x[:, ::32] = 4.0   # one dominant element per chunk
    x = bf16_round(x)
    spikes = bf16_round(np.repeat(0.02 * x[:1], 12, axis=0))   # parallel to token 0: S = |x| |r|
    c = canonical(x, spikes)
    m = mfma_sim(x, spikes, "adverse")
    err = np.abs(c - m)
    assert np.all(err <= bound(x, spikes))
    assert np.any(err > bound(x, spikes, chunk_term=6.0))
    H = 4096
    x, r = inputs("aligned", 6, 12, H, 7)
    # running sum alone: exact chunk sums added in f32
    p = (x.astype(np.float64)[:, None, :] * r.astype(np.float64)[None, :, :]).reshape(6, 12, H // 32, 32)
    chunks = p.sum(axis=-1)
    run = np.zeros((6, 12), dtype=np.float32)
    for k in range(H // 32):
        run = (run + chunks[:, :, k].astype(np.float32)).astype(np.float32)
    exact = chunks.sum(axis=-1)
    S = np.abs(p).sum(axis=(-1, -2))
    rerr = np.abs(run.astype(np.float64) - exact)
    assert np.all(rerr <= U * (H / 32) * S)
    # and it is tight: a first chunk of 1 and H/32 - 1 chunks of 2^-24, each
    # addition an exact tie that rounds back to 1
    ties = np.full(H // 32, 2.0 ** -24)
    ties[0] = 1.0
    run1 = np.float32(0.0)
    for v in ties:
        run1 = np.float32(run1 + np.float32(v))
    assert abs(float(run1) - ties.sum()) > 0.95 * U * (H / 32) * ties.sum()


def test_canonical_logits_are_the_oracles_router():
    """the canonical value used above is the oracle's router logit: its bf16
    rounding equals the bf16-activation oracle's logits bit for bit"""
    x, r = inputs("random", 3, 8, 1024, 3)
    c = canonical(x, r).astype(np.float32)
    blk = O.OracleMoe(1024, 8, 1, 8, 0, True, O.BF16, {"router": (O.BF16, O.f32_to_bf16_bits(r))})
    lb = blk.logits(O.f32_to_bf16_bits(x))
    assert np.array_equal(bf16_round(c), lb)
