"""Pins for the CPU oracle (oracle/hx_oracle.c): each oracle function is checked
against a known answer, a closed form, an independent library routine or brute
force, chosen so that a plausible slip (a dropped term, a swapped field, a wrong
index or tie rule) fails here. CPU only."""
import numpy as np
import pytest

from oracle import oracle as O
from tests.common import bf16_bits, bf16_to_f32, make_f32_block, make_x, oracle_block, rel_err, store

L = O.lib()


# ------------------------------------------------------------------ scalars
def test_f16_to_f32_exhaustive():
    h = np.arange(65536, dtype=np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = np.array([L.hxo_f16_to_f32(int(v)) for v in h], np.float32)
    same = (got.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(got) & np.isnan(ref))
    assert same.all()


def test_f32_to_f16_matches_numpy_rne():
    rng = np.random.default_rng(1)
    parts = [rng.standard_normal(4000).astype(np.float32) * s for s in (1e-9, 1e-7, 6e-5, 1e-3, 1.0, 3e4, 7e4)]
    # exact ties of the 10-bit mantissa, the overflow edge and the subnormal edge
    ties = (np.arange(1, 2000, dtype=np.float32) + 0.5) * np.float32(2.0 ** -10)
    edges = np.array([65504, 65519.99, 65520, 65536, 6.103515625e-05, 6.0975552e-05,
                      5.9604645e-08, 2.9802322e-08, 2.9802326e-08, 0.0, -0.0], np.float32)
    x = np.concatenate(parts + [ties, -ties, edges])
    got = np.array([L.hxo_f32_to_f16(float(v)) for v in x], np.uint16)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    assert (got == ref).all()


def test_bf16_round_trip_matches_torch():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(2)
    x = np.concatenate([rng.standard_normal(20000).astype(np.float32) * s for s in (1e-30, 1e-3, 1, 1e30)])
    ties = ((np.arange(1, 1000, dtype=np.uint32) << 16) | 0x8000).view(np.float32)
    x = np.concatenate([x, ties, -ties])
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = O.f32_to_bf16_bits(x)
    assert (got == ref).all()
    assert (bf16_bits(x) == ref).all()  # the vectorised test helper agrees too
    back = bf16_to_f32(ref)
    assert (back == torch.from_numpy(x).to(torch.bfloat16).float().numpy()).all()


def test_expf_error_bound_and_special_values():
    xs = np.concatenate([np.linspace(-87.0, 0.0, 400001, dtype=np.float32),
                         np.linspace(0.0, 88.0, 20001, dtype=np.float32)])
    got = np.array([O.expf(v) for v in xs], np.float64)
    ref = np.exp(xs.astype(np.float64))
    ulp = np.spacing(ref.astype(np.float32)).astype(np.float64)
    assert (np.abs(got - ref) / ulp).max() <= 2.0
    assert O.expf(0.0) == 1.0
    assert O.expf(-87.5) == 0.0 and O.expf(-1000.0) == 0.0
    assert np.isinf(O.expf(89.0))


# ------------------------------------------------------------------ GGUF blocks
def f16b(v):
    return np.array([v], np.float16).view(np.uint8)


def test_q8_0_known_answer():
    blk = np.zeros(34, np.uint8)
    blk[0:2] = f16b(0.5)
    q = np.array([-127, -64, -1, 0, 1, 2, 63, 127] * 4, np.int8)
    blk[2:] = q.view(np.uint8)
    got = O.dequantize(O.Q8_0, blk, 32)
    assert (got == 0.5 * q.astype(np.float32)).all()


def pack_q4k_scales(sc, mn):
    """12-byte scale field written from the GGUF description: sub-blocks 0-3 keep
    their 6-bit scale in bytes 0-3 and 6-bit min in bytes 4-7; sub-blocks 4-7 keep
    the low 4 bits of scale|min as the low|high nibble of bytes 8-11 and their top
    2 bits in the top 2 bits of bytes 0-3 (scale) and 4-7 (min)."""
    b = [0] * 12
    for j in range(4):
        b[j] = sc[j] | ((sc[j + 4] >> 4) << 6)
        b[j + 4] = mn[j] | ((mn[j + 4] >> 4) << 6)
        b[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    return np.array(b, np.uint8)


def test_q4_k_known_answer_every_subblock():
    rng = np.random.default_rng(3)
    sc = [5, 17, 33, 63, 16, 48, 1, 62]          # high bits set on the j>=4 half
    mn = [60, 2, 31, 0, 63, 20, 47, 15]
    q = rng.integers(0, 16, 256)
    blk = np.zeros(144, np.uint8)
    blk[0:2] = f16b(0.25)
    blk[2:4] = f16b(0.125)
    blk[4:16] = pack_q4k_scales(sc, mn)
    qs = np.zeros(128, np.uint8)
    for e in range(256):       # element 64c+l: low nibble of byte 32c+l; 64c+32+l: high nibble
        c, r = divmod(e, 64)
        if r < 32:
            qs[32 * c + r] |= q[e]
        else:
            qs[32 * c + r - 32] |= q[e] << 4
    blk[16:] = qs
    got = O.dequantize(O.Q4_K, blk, 256)
    j = np.arange(256) // 32
    want = 0.25 * np.array(sc)[j] * q - 0.125 * np.array(mn)[j]
    assert np.array_equal(got, want.astype(np.float32))


def test_q6_k_known_answer_every_subblock():
    rng = np.random.default_rng(4)
    q = rng.integers(0, 64, 256)               # stored q, value is d*sc*(q-32)
    sc = rng.integers(-128, 128, 16)
    d = 0.0625
    blk = np.zeros(210, np.uint8)
    ql = np.zeros(128, np.uint8)
    qh = np.zeros(64, np.uint8)
    for e in range(256):
        # element 128n + 32s + l: low nibble source ql[64n + 32(s&1) + l], nibble s>>1;
        # high 2 bits in qh[32n + l] at bit 2s
        n, r = divmod(e, 128)
        s, l = divmod(r, 32)
        byte = 64 * n + 32 * (s & 1) + l
        ql[byte] |= (q[e] & 15) << (4 * (s >> 1))
        qh[32 * n + l] |= (q[e] >> 4) << (2 * s)
    blk[0:128] = ql
    blk[128:192] = qh
    blk[192:208] = sc.astype(np.int8).view(np.uint8)
    blk[208:210] = f16b(d)
    got = O.dequantize(O.Q6_K, blk, 256)
    want = d * sc[np.arange(256) // 16] * (q - 32)
    assert np.array_equal(got, want.astype(np.float32))


def test_row_bytes_and_divisibility():
    assert O.row_bytes(O.Q8_0, 2048) == 64 * 34
    assert O.row_bytes(O.Q4_K, 2048) == 8 * 144
    assert O.row_bytes(O.Q6_K, 512) == 2 * 210
    assert O.row_bytes(O.Q6_K, 100) == -1        # isq.rs:62-68 rejects a ragged last dim
    with pytest.raises(ValueError):
        O.quantize(O.Q4_K, np.zeros((4, 100), np.float32))


@pytest.mark.parametrize("dt,rel_rms", [(O.Q8_0, 0.007), (O.Q4_K, 0.09), (O.Q6_K, 0.022)])
def test_quantizer_round_trip_error(dt, rel_rms):
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((16, 2048)) * 0.02).astype(np.float32)
    d = O.dequantize(dt, O.quantize(dt, w), 2048)
    err = d - w
    assert np.sqrt((err ** 2).mean() / (w ** 2).mean()) < rel_rms
    if dt == O.Q8_0:
        # per element: half a step, plus |q| <= 127 times the f16 rounding of the scale
        d = np.abs(w.reshape(-1, 32)).max(1, keepdims=True) / 127
        assert (np.abs(err.reshape(-1, 32)) <= d * (0.5 + 127 * 2.0 ** -11) * 1.0001).all()


def test_quantizer_is_exact_on_representable_q8_0():
    q = np.tile(np.arange(-127, 128, 8, dtype=np.float32), 2)[:32]
    q[0] = 127
    w = (q * np.float32(0.5)).reshape(1, 32)
    blk = O.quantize(O.Q8_0, w)
    assert np.array_equal(O.dequantize(O.Q8_0, blk, 32), w)


# ------------------------------------------- quantiser rules (candle's from_float)
def test_q8_0_rounds_half_away_from_zero():
    """BlockQ8_0::from_float rounds x / d with f32::round: with amax 127 (d = 1)
    the halves go away from zero (round-half-even would give 0, 4, -2, -0)"""
    x = np.zeros((1, 32), np.float32)
    x[0, :5] = [127.0, 0.5, 4.5, -2.5, -0.5]
    blk = O.quantize(O.Q8_0, x)[0]
    assert blk[:2].view(np.uint16)[0] == 0x3C00            # f16 1.0
    assert list(blk[2:7].view(np.int8)) == [127, 1, 5, -3, -1]


def test_q4_k_constant_subblock_quantises_to_zero():
    """make_qkx1_quants returns (scale 0, min 0) when a sub-block's max equals its
    min -- before min is clamped to <= 0 -- so a sub-block holding one positive
    constant dequantises to 0, and a whole block of it stores nothing but zeros"""
    assert not O.quantize(O.Q4_K, np.full((1, 256), 0.3, np.float32)).any()
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((1, 256)) * 0.02).astype(np.float32)
    x[0, 64:96] = 0.01
    d = O.dequantize(O.Q4_K, O.quantize(O.Q4_K, x), 256)[0]
    assert not d[64:96].any() and np.abs(d[:64] - x[0, :64]).max() < 0.01


def test_q4_k_lattice_round_trip_is_exact():
    """sub-block j holding s_j l - m_j (l = 0..15, both ends present) with
    s_j = sc_j 2^-10, m_j = mm_j 2^-12 and the largest sc, mm equal to 63: the
    search converges to (s_j, m_j), d = 2^-10, dmin = 2^-12 and the 6-bit
    scales/mins are sc_j, mm_j (ones above 15 use the high-bit packing of
    sub-blocks 4-7), so dequantisation gives x back exactly"""
    sc = [63, 17, 40, 5, 33, 63, 18, 50]
    mm = [0, 63, 21, 7, 48, 16, 63, 31]
    rng = np.random.default_rng(8)
    x = np.empty(256, np.float32)
    for j in range(8):
        l = rng.integers(0, 16, 32)
        l[0], l[1] = 0, 15
        x[32 * j:32 * j + 32] = (sc[j] * l * 4.0 - mm[j]) / 4096.0
    blk = O.quantize(O.Q4_K, x.reshape(1, 256))[0]
    assert blk[:4].view(np.uint16).tolist() == [0x1400, 0x0C00]     # 2^-10, 2^-12
    assert np.array_equal(O.dequantize(O.Q4_K, blk, 256), x)


def test_q6_k_lattice_round_trip_is_exact():
    """sub-block i holding n_i 2^-12 l (l in [-32, 31], -32 present so it is the
    largest-|x| element): make_qx_quants keeps the lattice codes, the largest
    scale (n = 128) sets iscale = -4096, d = -2^-12 and the int8 scales -n_i"""
    n = [128, 1, 77, 3, 100, 64, 9, 128, 31, 2, 127, 50, 12, 90, 45, 7]
    rng = np.random.default_rng(9)
    x = np.empty(256, np.float32)
    for i in range(16):
        l = rng.integers(-32, 32, 16)
        l[0] = -32
        x[16 * i:16 * i + 16] = n[i] * l / 4096.0
    blk = O.quantize(O.Q6_K, x.reshape(1, 256))[0]
    assert blk[208:210].view(np.uint16)[0] == 0x8C00                # -2^-12
    assert list(blk[192:208].view(np.int8)) == [-v for v in n]
    assert np.array_equal(O.dequantize(O.Q6_K, blk, 256), x)


def test_make_qx_quants_improves_on_its_start_and_returns_the_fit_scale():
    """on random sub-blocks: the returned scale is the x^2-weighted least-squares
    scale of the returned codes, the codes lie in [-32, 31], and the weighted
    error is no larger than that of the starting codes (round(-32 x / max))
    with their own least-squares scale"""
    rng = np.random.default_rng(11)
    for _ in range(200):
        x = (rng.standard_normal(16) * 0.02).astype(np.float32)
        scale, l = O.make_qx(x, 32)
        assert l.min() >= -32 and l.max() <= 31
        w = x.astype(np.float64) ** 2
        ls = (w * x * l).sum() / (w * l * l).sum()
        assert abs(scale - ls) <= 1e-5 * abs(ls)
        mx = x[np.argmax(np.abs(x))]
        l0 = np.clip(np.floor(-32.0 / mx * x.astype(np.float64) + 0.5), -32, 31)
        s0 = (w * x * l0).sum() / (w * l0 * l0).sum()
        assert (w * (x - scale * l) ** 2).sum() <= (w * (x - s0 * l0) ** 2).sum() * (1 + 1e-6)


def test_make_qkx1_quants_closed_forms():
    """two-valued sub-blocks: {a, b} with a < 0 < b converges to scale (b - a) / 15
    and min -a (codes 0 and 15 fit exactly); an all-positive sub-block keeps min 0
    and its scale is the least-squares fit of codes against x; equal values give
    (0, 0)"""
    x = np.array([-0.3, 0.6] * 16, np.float32)
    s, m = O.make_qkx1(x, 15, 5)
    assert abs(s - 0.06) < 1e-6 and abs(m - 0.3) < 1e-6
    x = np.linspace(0.1, 0.7, 32).astype(np.float32)
    s, m = O.make_qkx1(x, 15, 5)
    assert m == 0.0
    l = np.clip(np.floor(x / s + 0.5), 0, 15)
    assert abs(s - (x * l).sum() / (l * l).sum()) < 1e-6
    assert O.make_qkx1(np.full(32, -0.2, np.float32), 15, 5) == (0.0, 0.0)


# ------------------------------------------- candle's quantised-matmul arithmetic
def _round_away(v):
    """f32::round on float32 values: half away from zero (exact)"""
    v = np.asarray(v, np.float32)
    t = np.trunc(v)
    return (t + np.sign(v) * (np.abs(v - t) >= 0.5)).astype(np.float32)


def _q8k_np(x):
    """BlockQ8K::from_float restated in numpy float32 ops"""
    x = np.asarray(x, np.float32).reshape(-1, 256)
    d = np.zeros(len(x), np.float32)
    qs = np.zeros(x.shape, np.int32)
    for b, row in enumerate(x):
        i = int(np.argmax(np.abs(row)))           # first largest |x|
        if row[i] == 0:
            continue
        iscale = np.float32(-128.0) / row[i]
        qs[b] = np.minimum(_round_away(iscale * row), 127).astype(np.int32)
        d[b] = np.float32(1.0) / iscale
    return d, qs, qs.reshape(-1, 16, 16).sum(-1)


def test_quant_q8_k_known_answer():
    """iscale = -128 / (signed largest-|x| value), q = min(round(iscale x), 127):
    the largest element maps to -128 and its negation saturates at 127;
    bsums are sums of 16"""
    x = np.zeros(256, np.float32)
    x[:6] = [2.0, -2.0, 1.0, 0.0078125, -0.01171875, 0.5]
    d, qs, bs = O.quant_q8_k(x)
    assert d[0] == np.float32(-1.0 / 64.0)
    assert list(qs[:6]) == [-128, 127, -64, -1, 1, -32]       # 0.5 and -0.75 round away from zero
    assert bs[0, 0] == -128 + 127 - 64 - 1 + 1 - 32 and not bs[0, 1:].any()
    x = np.random.default_rng(4).standard_normal(1024).astype(np.float32)
    d2, q2, b2 = O.quant_q8_k(x)
    dn, qn, bn = _q8k_np(x)
    assert np.array_equal(d2, dn) and np.array_equal(q2.astype(np.int32), qn.ravel()) and np.array_equal(b2, bn)
    assert not O.quant_q8_k(np.zeros(256, np.float32))[1].any()


def _f16(b):
    return np.frombuffer(np.ascontiguousarray(b).tobytes(), np.float16).astype(np.float32)


def _vec_dot_np(dt, wrow, xrow):
    """candle's vec_dot_unopt (weights GGUF row, activations f32 row) restated
    with numpy float32 scalar ops in the published order"""
    f32 = np.float32
    if dt == O.Q8_0:
        xb = O.quantize(O.Q8_0, xrow.reshape(1, -1))[0].reshape(-1, 34)
        wb = wrow.reshape(-1, 34)
        sumf = f32(0)
        for bw, bx in zip(wb, xb):
            si = int((bw[2:].view(np.int8).astype(np.int64) * bx[2:].view(np.int8).astype(np.int64)).sum())
            sumf = f32(sumf + f32(f32(f32(si) * _f16(bw[:2])[0]) * _f16(bx[:2])[0]))
        return sumf
    d_x, q_x, bs_x = _q8k_np(xrow)
    if dt == O.Q4_K:
        wb = wrow.reshape(-1, 144)
        sums = np.zeros(8, np.float32)
        sumf = f32(0)
        for b, blk in enumerate(wb):
            sc = blk[4:16].astype(np.int64)
            scale = [(sc[j] & 63) if j < 4 else ((sc[j + 4] & 0xF) | ((sc[j - 4] >> 6) << 4)) for j in range(8)]
            mins = [(sc[j + 4] & 63) if j < 4 else ((sc[j + 4] >> 4) | ((sc[j] >> 6) << 4)) for j in range(8)]
            qs = blk[16:].astype(np.int64).reshape(4, 32)
            a = np.concatenate([np.concatenate([q & 0xF, q >> 4]) for q in qs])
            q8 = q_x[b].astype(np.int64)
            aux = np.zeros(8, np.int64)
            for j in range(8):
                aux += scale[j] * (q8[32 * j:32 * j + 32] * a[32 * j:32 * j + 32]).reshape(4, 8).sum(0)
            sumi = sum(int(bs_x[b][j]) * mins[j // 2] for j in range(16))
            d = f32(_f16(blk[0:2])[0] * d_x[b])
            for l in range(8):
                sums[l] = f32(sums[l] + f32(d * f32(aux[l])))
            sumf = f32(sumf - f32(f32(_f16(blk[2:4])[0] * d_x[b]) * f32(sumi)))
        s = f32(-0.0)
        for l in range(8):
            s = f32(s + sums[l])
        return f32(sumf + s)
    wb = wrow.reshape(-1, 210)
    sums = np.zeros(8, np.float32)
    for b, blk in enumerate(wb):
        ql, qh = blk[:128].astype(np.int64), blk[128:192].astype(np.int64)
        a = np.zeros(256, np.int64)
        for n in range(2):
            for l in range(32):
                a[128 * n + l] = ((ql[64 * n + l] & 0xF) | ((qh[32 * n + l] & 3) << 4)) - 32
                a[128 * n + l + 32] = ((ql[64 * n + l + 32] & 0xF) | (((qh[32 * n + l] >> 2) & 3) << 4)) - 32
                a[128 * n + l + 64] = ((ql[64 * n + l] >> 4) | (((qh[32 * n + l] >> 4) & 3) << 4)) - 32
                a[128 * n + l + 96] = ((ql[64 * n + l + 32] >> 4) | (((qh[32 * n + l] >> 6) & 3) << 4)) - 32
        sc = blk[192:208].view(np.int8).astype(np.int64)
        q8 = q_x[b].astype(np.int64)
        aux = np.zeros(8, np.int64)
        for j in range(16):
            aux += sc[j] * (q8[16 * j:16 * j + 16] * a[16 * j:16 * j + 16]).reshape(2, 8).sum(0)
        d = f32(_f16(blk[208:210])[0] * d_x[b])
        for l in range(8):
            sums[l] = f32(sums[l] + f32(f32(aux[l]) * d))
    s = f32(-0.0)
    for l in range(8):
        s = f32(s + sums[l])
    return s


@pytest.mark.parametrize("dt", [O.Q8_0, O.Q4_K, O.Q6_K])
def test_candle_vec_dot_matches_independent_restatement(dt):
    """m <= 64: the oracle's vectorised vec_dot equals a plain numpy restatement
    of candle's vec_dot_unopt bit for bit, and (the integer identity) agrees with
    the f64 dot of the dequantised weights and dequantised activations"""
    rng = np.random.default_rng(20 + dt)
    K, N, m = 512, 6, 3
    w = O.quantize(dt, (rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    x = rng.standard_normal((m, K)).astype(np.float32)
    got = O.qlinear(dt, w, x)
    for r in range(m):
        for n in range(N):
            assert got[r, n].view(np.uint32) == np.float32(_vec_dot_np(dt, w[n], x[r])).view(np.uint32)
    wd = O.dequantize(dt, w, K).astype(np.float64)
    if dt == O.Q8_0:
        xd = O.dequantize(O.Q8_0, O.quantize(O.Q8_0, x), K).astype(np.float64)
    else:
        xd = np.stack([np.concatenate([(d * q).astype(np.float64) for d, q in zip(*_q8k_np(row)[:2])])
                       for row in x])
    ref = xd @ wd.T
    assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()


def test_candle_f16_path_above_64_rows():
    """m > 64 (forward_via_f16): weights and x rounded to f16, an f32 fmaf chain
    over k, the output rounded to f16"""
    rng = np.random.default_rng(31)
    K, N, m = 256, 3, 70
    w = O.quantize(O.Q4_K, (rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    x = rng.standard_normal((m, K)).astype(np.float32)
    got = O.qlinear(O.Q4_K, w, x)
    wh = O.dequantize(O.Q4_K, w, K).astype(np.float16).astype(np.float64)
    xh = x.astype(np.float16).astype(np.float64)
    for r in (0, 33, 69):
        for n in range(N):
            acc = np.float32(0)
            for kk in range(K):                      # fmaf: one rounding of an exact f64 a*b + c
                acc = np.float32(xh[r, kk] * wh[n, kk] + np.float64(acc))
            assert got[r, n] == np.float32(np.float16(acc))


@pytest.mark.parametrize("fmt", [O.Q8_0, O.Q4_K])
def test_candle_mode_close_to_exact_mode(fmt):
    """the two forward modes share the routing and differ only by candle's
    activation quantisation / f16 rounding: close (within 3e-2: 8-bit
    activations move single outputs by a few tenths of a percent of max|y|,
    more at small H), not equal"""
    H, E, k, I, Is = 512, 16, 4, 256, 256
    w = make_f32_block(40, H, E, I, Is)
    fm = {"gate": fmt, "up": fmt, "down": O.Q6_K if fmt == O.Q4_K else fmt, "router": O.BF16, "seg": O.BF16}
    fm.update({"sgate": fm["gate"], "sup": fm["up"], "sdown": fm["down"]})
    orc = oracle_block((H, E, k, I, Is, True), store(w, fm), O.BF16)
    for T in (1, 80):
        x = bf16_bits(make_x(41, T, H))
        a, c = orc.forward(x), orc.forward_candle(x)
        assert 0 < rel_err(c, a) <= 3e-2


def test_candle_mode_sampled_tokens_equal_the_full_forward():
    """forward_candle_tokens (what the GPU tests compare sampled prefill tokens
    with) equals the full candle forward's rows bit for bit: every expert call
    keeps the arm of its full row count (here some experts get more than 64
    rows, so both arms occur), and each arm computes rows independently"""
    H, E, k, I, Is = 256, 8, 2, 256, 256
    w = make_f32_block(42, H, E, I, Is)
    fm = {"gate": O.Q4_K, "up": O.Q4_K, "down": O.Q6_K, "router": O.BF16, "seg": O.BF16}
    fm.update({"sgate": O.Q4_K, "sup": O.Q4_K, "sdown": O.Q6_K})
    orc = oracle_block((H, E, k, I, Is, True), store(w, fm), O.BF16)
    T = 400
    x = bf16_bits(make_x(43, T, H))
    counts = np.bincount(orc.route(x)[2].ravel(), minlength=E)
    assert counts.max() > 64
    full = orc.forward_candle(x)
    sel = np.array([0, 7, 150, 399, 8])
    part = orc.forward_candle_tokens(x, sel)
    assert np.array_equal(part.view(np.uint32), full[sel].view(np.uint32))
    with pytest.raises(ValueError):
        orc.forward_candle_tokens(x, np.array([3, 3]))
    # and the arm really follows the full count: on the sampled tokens alone
    # every call has m <= 5 and takes the quantised arm, which differs
    alone = orc.forward_candle(x[sel])
    assert not np.array_equal(alone, part)


# ------------------------------------------------------------------ router
def tiny(seed=0, H=64, E=8, k=2, I=16, Is=16, norm=True, act=O.F32, fmt=None):
    w = make_f32_block(seed, H, E, I, Is, std=0.5)
    st = store(w, fmt or {})
    return w, oracle_block((H, E, k, I, Is, norm), st, act)


def stable_desc(p):
    return np.argsort(-p, axis=-1, kind="stable")


def test_router_zero_weights_closed_form():
    H, E, k = 32, 16, 4
    w = make_f32_block(0, H, E, 8, 0)
    w["router"][:] = 0
    m = oracle_block((H, E, k, 8, 0, True), store(w, {}), O.F32)
    lg, pr, ix, wt = m.route(make_x(0, 5, H))
    assert (lg == 0).all() and (pr == np.float32(1 / 16)).all()
    assert (ix == np.arange(k)).all()            # all tied: lowest ids win
    assert (wt == np.float32(0.25)).all()


@pytest.mark.parametrize("act", [O.F32, O.BF16])
@pytest.mark.parametrize("H", [8, 64, 100, 520, 2048])
def test_router_brute_force(act, H):
    E, k = 24, 5
    w = make_f32_block(H, H, E, 8, 0, std=0.1)
    m = oracle_block((H, E, k, 8, 0, True), store(w, {"router": act}), act)
    x = make_x(H, 9, H)
    xs = bf16_bits(x) if act == O.BF16 else x
    lg, pr, ix, wt = m.route(xs)
    xf = bf16_to_f32(xs) if act == O.BF16 else x
    wr = bf16_to_f32(bf16_bits(w["router"])) if act == O.BF16 else w["router"]
    exact = xf.astype(np.float64) @ wr.astype(np.float64).T
    if act == O.BF16:   # logits are bf16 values, one rounding from the f32 sum
        assert (bf16_to_f32(bf16_bits(lg)) == lg).all()
        assert np.abs(lg - exact).max() <= 2.0 ** -8 * np.abs(exact).max() + 1e-6
    else:
        assert np.abs(lg - exact).max() <= 1e-5 * np.abs(exact).max()
    ref_p = np.exp(lg.astype(np.float64) - lg.max(1, keepdims=True))
    ref_p /= ref_p.sum(1, keepdims=True)
    assert np.abs(pr - ref_p).max() <= 4 * np.spacing(np.float32(1.0))
    assert (ix == stable_desc(pr)[:, :k]).all()
    sel = np.take_along_axis(pr.astype(np.float64), ix.astype(np.int64), 1)
    assert np.abs(wt - sel / sel.sum(1, keepdims=True)).max() < 1e-6


def test_router_ties_go_to_lower_id_and_no_renorm():
    H, E, k = 16, 6, 3
    w = make_f32_block(1, H, E, 8, 0, std=0.3)
    w["router"][4] = w["router"][1]              # experts 1 and 4 tie exactly
    w["router"][5] = w["router"][2]
    m = oracle_block((H, E, k, 8, 0, False), store(w, {}), O.F32)
    x = make_x(1, 50, H)
    lg, pr, ix, wt = m.route(x)
    assert (pr[:, 1] == pr[:, 4]).all() and (pr[:, 2] == pr[:, 5]).all()
    assert (ix == stable_desc(pr)[:, :k]).all()
    both = (ix == 1).any(1) & (ix == 4).any(1)
    # whenever only one of a tied pair is picked it is the lower id
    only = ((ix == 1).any(1) ^ (ix == 4).any(1))
    assert not (ix[only] == 4).any()
    assert both.any() or only.any()
    assert np.array_equal(wt, np.take_along_axis(pr, ix, 1))   # norm_topk_prob=false: raw softmax


def test_router_bias_is_added_after_rounding():
    _, m = tiny(act=O.BF16, fmt={"router": O.BF16}, H=64, E=8)
    x = bf16_bits(make_x(3, 4, 64))
    b = np.linspace(-1, 1, 8).astype(np.float32)
    assert np.array_equal(m.logits(x, b), m.logits(x) + b)


# ------------------------------------------------------------------ dispatch
def test_dispatch_invariants_and_brute_force():
    rng = np.random.default_rng(6)
    T, k, E = 300, 7, 40
    ix = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    perm, offs, inv = O.dispatch(ix, E)
    flat = ix.ravel()
    assert np.array_equal(np.sort(perm), np.arange(T * k))
    assert np.array_equal(offs, np.concatenate([[0], np.cumsum(np.bincount(flat, minlength=E))]))
    assert np.array_equal(perm, np.argsort(flat, kind="stable"))
    assert np.array_equal(inv[perm], np.arange(T * k))
    # moe.rs:152-160: each expert's rows are its tokens in ascending order
    for e in range(E):
        toks = perm[offs[e]:offs[e + 1]] // k
        assert np.array_equal(toks, np.nonzero((ix == e).any(1))[0])


def test_dispatch_empty_and_single_expert():
    perm, offs, inv = O.dispatch(np.zeros((0, 3), np.int32), 5)
    assert (offs == 0).all() and perm.size == 0
    ix = np.full((4, 1), 2, np.int32)
    perm, offs, _ = O.dispatch(ix, 5)
    assert list(offs) == [0, 0, 0, 4, 4, 4] and list(perm) == [0, 1, 2, 3]


# ------------------------------------------------------------------ forward
def np_swiglu(wg, wu, wd, x):
    g = x.astype(np.float64) @ wg.T.astype(np.float64)
    u = x.astype(np.float64) @ wu.T.astype(np.float64)
    return (g / (1 + np.exp(-g)) * u) @ wd.T.astype(np.float64)


def per_token_reference(w, x, k, norm, shared=True, bf16_logits=False):
    """moe.rs:245-294: route each token on its own (host softmax, stable descending
    sort, renorm) and mix its experts one by one, then the shared expert. With bf16
    activations the router Linear returns bf16 logits (moe.rs:134)."""
    out = np.zeros(x.shape, np.float64)
    lg = x.astype(np.float64) @ w["router"].T.astype(np.float64)
    if bf16_logits:
        lg = bf16_to_f32(bf16_bits(lg.astype(np.float32))).astype(np.float64)
    for t in range(x.shape[0]):
        p = np.exp(lg[t] - lg[t].max())
        p /= p.sum()
        sel = np.argsort(-p, kind="stable")[:k]
        den = p[sel].sum() if norm else 1.0
        for e in sel:
            out[t] += p[e] / den * np_swiglu(w["gate"][e], w["up"][e], w["down"][e], x[t:t + 1])[0]
        if shared:
            mix = 1 / (1 + np.exp(-(x[t].astype(np.float64) @ w["seg"][0].astype(np.float64))))
            out[t] += mix * np_swiglu(w["sgate"], w["sup"], w["sdown"], x[t:t + 1])[0]
    return out


def test_forward_matches_reference_unit_test_shapes():
    # moe.rs:223-303 (hidden 8, inter 4, 6 experts, top-2, 2x3 tokens, tol 1e-4)
    H, I, E, k = 8, 4, 6, 2
    w = make_f32_block(11, H, E, I, I, std=0.5)
    m = oracle_block((H, E, k, I, I, True), store(w, {}), O.F32)
    x = make_x(11, 6, H) * np.float32(0.5)
    assert np.abs(m.forward(x) - per_token_reference(w, x, k, True)).max() < 1e-4
    # moe.rs:309-359 (hidden 4, inter 2, 3 experts, top-1, no shared, no renorm)
    H, I, E, k = 4, 2, 3, 1
    w = make_f32_block(12, H, E, I, 0, std=0.5)
    m = oracle_block((H, E, k, I, 0, False), store(w, {}), O.F32)
    x = make_x(12, 1, H) * np.float32(0.5)
    assert np.abs(m.forward(x) - per_token_reference(w, x, k, False, shared=False)).max() < 1e-5


def test_forward_uniform_routing_is_mean_of_experts():
    H, E, I = 32, 4, 16
    w = make_f32_block(13, H, E, I, I, std=0.2)
    w["router"][:] = 0
    w["seg"][:] = 0                                  # sigmoid(0) = 1/2
    m = oracle_block((H, E, E, I, I, True), store(w, {}), O.F32)
    x = make_x(13, 3, H)
    want = sum(np_swiglu(w["gate"][e], w["up"][e], w["down"][e], x) for e in range(E)) / E
    want += 0.5 * np_swiglu(w["sgate"], w["sup"], w["sdown"], x)
    assert rel_err(m.forward(x), want) < 1e-6


def test_forward_tp_partial_sums_reproduce_full_block():
    """tp_qwen3_5.rs:2460-2496: column-split gate/up and row-split down along the
    intermediate dim; the two partial blocks sum to the single-device block."""
    H, E, k, I = 64, 8, 3, 32
    w = make_f32_block(14, H, E, I, I, std=0.2)
    full = oracle_block((H, E, k, I, I, True), store(w, {}), O.F32)
    x = make_x(14, 7, H)
    parts = []
    for r in range(2):
        sl = slice(r * I // 2, (r + 1) * I // 2)
        wr = dict(w)
        wr["gate"], wr["up"] = w["gate"][:, sl].copy(), w["up"][:, sl].copy()
        wr["down"] = w["down"][:, :, sl].copy()
        wr["sgate"], wr["sup"], wr["sdown"] = w["sgate"][sl].copy(), w["sup"][sl].copy(), w["sdown"][:, sl].copy()
        parts.append(oracle_block((H, E, k, I // 2, I // 2, True), store(wr, {}), O.F32).forward(x))
    assert rel_err(parts[0] + parts[1], full.forward(x)) < 1e-6


@pytest.mark.parametrize("fmt", [
    {"gate": O.Q8_0, "up": O.Q8_0, "down": O.Q8_0, "sgate": O.Q8_0, "sup": O.Q8_0, "sdown": O.Q8_0},
    {"gate": O.Q4_K, "up": O.Q4_K, "down": O.Q6_K, "sgate": O.Q4_K, "sup": O.Q4_K, "sdown": O.Q6_K},
])
def test_forward_quantised_equals_forward_on_dequantised_weights(fmt):
    H, E, k, I = 256, 8, 3, 256
    w = make_f32_block(15, H, E, I, I)
    st = store(w, dict(fmt, router=O.BF16, seg=O.BF16))
    deq = {}
    for key, (dt, a) in st.items():
        cols = a.shape[-1] if dt in (O.F32,) else (H if key in ("router", "gate", "up", "sgate", "sup", "seg") else I)
        deq[key] = bf16_to_f32(a) if dt == O.BF16 else (a if dt == O.F32 else O.dequantize(dt, a, cols))
    x = bf16_bits(make_x(15, 6, H))
    mq = oracle_block((H, E, k, I, I, True), st, O.BF16)
    mf = oracle_block((H, E, k, I, I, True), store(deq, {"router": O.BF16, "seg": O.BF16}), O.BF16)
    assert np.array_equal(mq.route(x)[2], mf.route(x)[2])
    assert rel_err(mq.forward(x), mf.forward(x)) < 1e-6
    assert rel_err(mq.forward(x), per_token_reference(deq, bf16_to_f32(x), k, True, bf16_logits=True)) < 1e-5


def test_forward_tokens_are_independent():
    H, E, k, I = 64, 8, 2, 16
    w = make_f32_block(16, H, E, I, I)
    m = oracle_block((H, E, k, I, I, True), store(w, {}), O.F32)
    x = make_x(16, 10, H)
    full = m.forward(x)
    assert np.array_equal(m.forward(x[3:7]), full[3:7])


def test_rmsnorm_closed_forms():
    H = 64
    w = np.linspace(-0.5, 0.5, H).astype(np.float32)
    x = np.full((2, H), 3.0, np.float32)
    y = O.rmsnorm(x, w, 1e-6, O.F32)
    assert np.allclose(y, 3.0 / np.sqrt(9.0 + 1e-6) * (1 + w), rtol=1e-6)
    xr = make_x(17, 4, H)
    y0 = O.rmsnorm(xr, np.zeros(H, np.float32), 1e-6, O.F32)
    assert np.allclose(np.sqrt((y0.astype(np.float64) ** 2).mean(1)), 1.0, rtol=1e-5)


# ------------------------------------------------------------------ C1 vs HF transformers
def c1_oracle(seed):
    from tests.common import C1
    H, E, k, I, Is = C1["H"], C1["E"], C1["k"], C1["I"], C1["Is"]
    w = make_f32_block(seed, H, E, I, Is)
    return oracle_block((H, E, k, I, Is, True), store(w, {}), O.F32), make_x(seed, C1["T"], H)


def test_c1_matches_transformers_golden():
    """tests/golden/c1_transformers.npz holds HF Qwen3NextSparseMoeBlock's outputs
    on the C1 block (make_c1_golden.py); the oracle must reproduce its routing
    exactly and its output within the f32 tolerance (max rel err 1e-4)."""
    import os
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "c1_transformers.npz"))
    m, x = c1_oracle(int(g["seed"]))
    _, _, ix, wt = m.route(x)
    assert np.array_equal(ix, g["topk_idx"])
    assert np.abs(wt - g["topk_w"]).max() < 1e-6
    assert rel_err(m.forward(x), g["y"]) < 1e-5


def test_c1_matches_transformers_live_other_seed():
    pytest.importorskip("transformers")
    import importlib.util
    import os
    spec = importlib.util.spec_from_file_location(
        "make_c1_golden", os.path.join(os.path.dirname(__file__), "golden", "make_c1_golden.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    ref = mod.run(seed=77)
    m, x = c1_oracle(77)
    assert np.array_equal(m.route(x)[2], ref["topk_idx"])
    assert rel_err(m.forward(x), ref["y"]) < 1e-5
