"""ctypes view of the CPU oracle (oracle/libhxoracle.so) -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this
module, and only as the checker. It restates helexa neuron's Qwen3-Next
sparse-MoE block; the C source (oracle/hx_oracle.c) cites the reference lines it
follows. Arrays are numpy; bf16 tensors travel as uint16 arrays of raw bits.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libhxoracle.so")

F32, F16, Q8_0, Q4_K, Q6_K, BF16 = 0, 1, 8, 12, 14, 30
BLOCK_ELEMS = {F32: 1, F16: 1, BF16: 1, Q8_0: 32, Q4_K: 256, Q6_K: 256}
BLOCK_BYTES = {F32: 4, F16: 2, BF16: 2, Q8_0: 34, Q4_K: 144, Q6_K: 210}


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE, "-B"], check=True)


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        vp, i64, i32 = C.c_void_p, C.c_int64, C.c_int
        L.hxo_f32_to_bf16.restype = C.c_uint16
        L.hxo_f32_to_bf16.argtypes = [C.c_float]
        L.hxo_bf16_to_f32.restype = C.c_float
        L.hxo_bf16_to_f32.argtypes = [C.c_uint16]
        L.hxo_f32_to_f16.restype = C.c_uint16
        L.hxo_f32_to_f16.argtypes = [C.c_float]
        L.hxo_f16_to_f32.restype = C.c_float
        L.hxo_f16_to_f32.argtypes = [C.c_uint16]
        L.hxo_expf.restype = C.c_float
        L.hxo_expf.argtypes = [C.c_float]
        L.hxo_row_bytes.restype = i64
        L.hxo_row_bytes.argtypes = [i32, i64]
        L.hxo_dequant.restype = i32
        L.hxo_dequant.argtypes = [i32, vp, i64, vp]
        L.hxo_quantize.restype = i32
        L.hxo_quantize.argtypes = [i32, vp, i64, i64, vp, i32]
        L.hxo_router_logits.restype = i32
        L.hxo_router_logits.argtypes = [vp, vp, i64, vp, vp]
        L.hxo_route.restype = i32
        L.hxo_route.argtypes = [vp, vp, i64, vp, vp, vp, vp, vp]
        L.hxo_dispatch.restype = i32
        L.hxo_dispatch.argtypes = [vp, i64, i32, i64, vp, vp, vp]
        L.hxo_moe_forward.restype = i32
        L.hxo_moe_forward.argtypes = [vp, vp, i64, vp, vp, i32]
        L.hxo_moe_forward_candle.restype = i32
        L.hxo_moe_forward_candle.argtypes = [vp, vp, i64, vp, vp, i32]
        L.hxo_moe_forward_candle_sel.restype = i32
        L.hxo_moe_forward_candle_sel.argtypes = [vp, vp, i64, vp, vp, i64, vp, i32]
        L.hxo_qlinear.restype = i32
        L.hxo_qlinear.argtypes = [i32, vp, i64, i64, vp, i64, vp, i32]
        L.hxo_quant_q8_k.restype = i32
        L.hxo_quant_q8_k.argtypes = [vp, i64, vp, vp, vp]
        L.hxo_make_qx.restype = C.c_float
        L.hxo_make_qx.argtypes = [i32, i32, vp, vp]
        L.hxo_make_qkx1.restype = None
        L.hxo_make_qkx1.argtypes = [i32, i32, i32, vp, C.POINTER(C.c_float), C.POINTER(C.c_float)]
        L.hxo_rmsnorm.restype = i32
        L.hxo_rmsnorm.argtypes = [i32, vp, i64, i64, vp, C.c_float, vp]
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


# ---------------------------------------------------------------- scalars
def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    L = lib()
    return np.array([L.hxo_f32_to_bf16(float(v)) for v in x.ravel()], dtype=np.uint16).reshape(x.shape)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def expf(x: float) -> float:
    return lib().hxo_expf(float(x))


# ---------------------------------------------------------------- blocks
def row_bytes(dtype: int, n: int) -> int:
    return int(lib().hxo_row_bytes(dtype, n))


def quantize(dtype: int, w: np.ndarray, nthreads: int = 0) -> np.ndarray:
    """f32 [..., cols] -> GGUF rows as uint8 [..., row_bytes]."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    cols = w.shape[-1]
    rows = w.size // cols
    rb = row_bytes(dtype, cols)
    if rb < 0:
        raise ValueError(f"cols {cols} do not tile into dtype {dtype} blocks")
    out = np.empty(w.shape[:-1] + (rb,), dtype=np.uint8)
    rc = lib().hxo_quantize(dtype, _p(w), rows, cols, _p(out), nthreads)
    if rc:
        raise ValueError(f"hxo_quantize rc={rc}")
    return out


def dequantize(dtype: int, q: np.ndarray, cols: int) -> np.ndarray:
    """GGUF rows uint8 [..., row_bytes] -> f32 [..., cols]."""
    q = np.ascontiguousarray(q, dtype=np.uint8)
    rb = row_bytes(dtype, cols)
    rows = q.size // rb
    out = np.empty(q.shape[:-1] + (cols,), dtype=np.float32)
    rc = lib().hxo_dequant(dtype, _p(q), rows * cols, _p(out))
    if rc:
        raise ValueError(f"hxo_dequant rc={rc}")
    return out


def qlinear(dtype: int, w: np.ndarray, x: np.ndarray, nthreads: int = 0) -> np.ndarray:
    """one MaybeQuantLinear call in candle's arithmetic: w GGUF rows [N, row_bytes]
    (or f32 [N, K]), x f32 [m, K] -> [m, N]"""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w)
    m, K = x.shape
    N = w.shape[0]
    out = np.empty((m, N), np.float32)
    rc = lib().hxo_qlinear(dtype, _p(w), N, K, _p(x), m, _p(out), nthreads)
    if rc:
        raise ValueError(f"hxo_qlinear rc={rc}")
    return out


def quant_q8_k(x: np.ndarray):
    """candle's BlockQ8K::from_float over a row -> (d [nb], qs int8 [n], bsums int16 [nb, 16])"""
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    nb = x.size // 256
    d = np.empty(nb, np.float32)
    qs = np.empty(x.size, np.int8)
    bs = np.empty((nb, 16), np.int16)
    if lib().hxo_quant_q8_k(_p(x), x.size, _p(d), _p(qs), _p(bs)):
        raise ValueError("row length must be a multiple of 256")
    return d, qs, bs


def make_qx(x: np.ndarray, nmax: int):
    """candle's make_qx_quants(n, nmax, x, L, 1) -> (scale, L - nmax as int32)"""
    x = np.ascontiguousarray(x, dtype=np.float32)
    L = np.empty(x.size, np.int8)
    sc = lib().hxo_make_qx(x.size, nmax, _p(x), _p(L))
    return float(np.float32(sc)), L.astype(np.int32) - nmax


def make_qkx1(x: np.ndarray, nmax: int, ntry: int):
    """candle's make_qkx1_quants(nmax, ntry, x) -> (scale, -min)"""
    x = np.ascontiguousarray(x, dtype=np.float32)
    sc, mn = C.c_float(), C.c_float()
    lib().hxo_make_qkx1(x.size, nmax, ntry, _p(x), C.byref(sc), C.byref(mn))
    return sc.value, mn.value


# ---------------------------------------------------------------- block
class _Moe(C.Structure):
    _fields_ = [
        ("hidden", C.c_int32), ("num_experts", C.c_int32), ("top_k", C.c_int32),
        ("inter", C.c_int32), ("shared_inter", C.c_int32), ("norm_topk_prob", C.c_int32),
        ("act_dtype", C.c_int32),
        ("router_dtype", C.c_int32), ("router", C.c_void_p),
        ("gate_dtype", C.c_int32), ("gate", C.c_void_p),
        ("up_dtype", C.c_int32), ("up", C.c_void_p),
        ("down_dtype", C.c_int32), ("down", C.c_void_p),
        ("sgate_dtype", C.c_int32), ("sgate", C.c_void_p),
        ("sup_dtype", C.c_int32), ("sup", C.c_void_p),
        ("sdown_dtype", C.c_int32), ("sdown", C.c_void_p),
        ("seg_dtype", C.c_int32), ("seg", C.c_void_p),
    ]


class OracleMoe:
    """Holds numpy weights (already in their storage format) and runs the oracle.

    weights: dict with keys router, gate, up, down, sgate, sup, sdown, seg; each a
    (dtype, ndarray) pair. Float formats are float32 arrays (F32) or uint16 bf16
    bits (BF16); quantised formats are uint8 GGUF rows.
    """

    def __init__(self, hidden, num_experts, top_k, inter, shared_inter, norm_topk_prob,
                 act_dtype, weights):
        self.cfg = (hidden, num_experts, top_k, inter, shared_inter, norm_topk_prob, act_dtype)
        self.w = {k: (dt, np.ascontiguousarray(a)) for k, (dt, a) in weights.items()}
        s = _Moe()
        s.hidden, s.num_experts, s.top_k, s.inter, s.shared_inter = hidden, num_experts, top_k, inter, shared_inter
        s.norm_topk_prob, s.act_dtype = int(bool(norm_topk_prob)), act_dtype
        for name in ("router", "gate", "up", "down", "sgate", "sup", "sdown", "seg"):
            if name in self.w:
                dt, a = self.w[name]
                setattr(s, name + "_dtype", dt)
                setattr(s, name, a.ctypes.data)
        self.s = s
        self.T_bytes = hidden * (2 if act_dtype == BF16 else 4)

    def _x(self, x):
        x = np.ascontiguousarray(x)
        want = np.uint16 if self.cfg[6] == BF16 else np.float32
        if x.dtype != want:
            raise TypeError(f"x must be {want} for act dtype {self.cfg[6]}")
        return x, x.size // self.cfg[0]

    def logits(self, x, bias=None):
        x, T = self._x(x)
        out = np.empty((T, self.cfg[1]), dtype=np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        rc = lib().hxo_router_logits(C.byref(self.s), _p(x), T, _p(b), _p(out))
        if rc:
            raise ValueError(f"hxo_router_logits rc={rc}")
        return out

    def route(self, x, bias=None):
        """-> (logits, probs, topk_idx int32 [T,k], topk_w f32 [T,k])"""
        x, T = self._x(x)
        E, k = self.cfg[1], self.cfg[2]
        lg = np.empty((T, E), np.float32)
        pr = np.empty((T, E), np.float32)
        ix = np.empty((T, k), np.int32)
        wt = np.empty((T, k), np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        rc = lib().hxo_route(C.byref(self.s), _p(x), T, _p(b), _p(lg), _p(pr), _p(ix), _p(wt))
        if rc:
            raise ValueError(f"hxo_route rc={rc}")
        return lg, pr, ix, wt

    def forward(self, x, bias=None, nthreads=0):
        """exact mode: dequantised weights, products accumulated in double"""
        x, T = self._x(x)
        y = np.empty((T, self.cfg[0]), np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        rc = lib().hxo_moe_forward(C.byref(self.s), _p(x), T, _p(b), _p(y), nthreads)
        if rc:
            raise ValueError(f"hxo_moe_forward rc={rc}")
        return y

    def forward_candle(self, x, bias=None, nthreads=0):
        """candle-arithmetic mode: the reference's CPU path for quantised experts
        (Q8_0 / Q8_K activation quantisation and integer vec_dot at m <= 64, the
        f16 path above), same routing as forward()"""
        x, T = self._x(x)
        y = np.empty((T, self.cfg[0]), np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        rc = lib().hxo_moe_forward_candle(C.byref(self.s), _p(x), T, _p(b), _p(y), nthreads)
        if rc:
            raise ValueError(f"hxo_moe_forward_candle rc={rc}")
        return y

    def forward_candle_tokens(self, x, tokens, bias=None, nthreads=0):
        """candle-arithmetic mode for the tokens `tokens` of a forward of all of x:
        each expert call takes the arm of its full row count (so a sample of a
        prefill is computed as in the full forward), only the sampled rows are
        computed; -> [len(tokens), H]"""
        x, T = self._x(x)
        sel = np.ascontiguousarray(tokens, dtype=np.int32)
        y = np.empty((sel.size, self.cfg[0]), np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        rc = lib().hxo_moe_forward_candle_sel(C.byref(self.s), _p(x), T, _p(b), _p(sel), sel.size, _p(y), nthreads)
        if rc:
            raise ValueError(f"hxo_moe_forward_candle_sel rc={rc}")
        return y


def dispatch(topk_idx: np.ndarray, num_experts: int):
    """-> (perm [T*k], offsets [E+1], inv [T*k]) int32"""
    ix = np.ascontiguousarray(topk_idx, dtype=np.int32)
    T, k = ix.shape
    perm = np.empty(T * k, np.int32)
    offs = np.empty(num_experts + 1, np.int32)
    inv = np.empty(T * k, np.int32)
    rc = lib().hxo_dispatch(_p(ix), T, k, num_experts, _p(perm), _p(offs), _p(inv))
    if rc:
        raise ValueError(f"hxo_dispatch rc={rc}")
    return perm, offs, inv


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float, act_dtype: int) -> np.ndarray:
    x = np.ascontiguousarray(x)
    H = w.shape[-1]
    T = x.size // H
    y = np.empty((T, H), np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    lib().hxo_rmsnorm(act_dtype, _p(x), T, H, _p(w), float(eps), _p(y))
    return y
