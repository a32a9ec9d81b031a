"""Host-side mirror of neuron's Qwen3-Next MoE block over libhxmoe.so's C ABI.

Names follow the reference so callers and tests read like neuron's own:

    TextConfig           crates/neuron/src/harness/arch/qwen3_5/mod.rs:227-314 (MoE fields)
    Qwen3_5MoeBlock      crates/neuron/src/harness/arch/qwen3_5/moe.rs:39-199
      .load(cfg, weights)      moe.rs:55 (validation moe.rs:56-69)
      .forward(xs)             moe.rs:164-199, input (b, l, hidden), same shape/dtype out
      .route(xs)               route_scatter moe.rs:124-162 + the dispatch sort of
                               tp_qwen3_5.rs:1189
    quantize                   isq.rs:39-55 (on the device)

Errors: every nonzero status from the library becomes HxError carrying
hx_last_error(), the way neuron maps candle errors to anyhow (moe.rs:56-76).
The library is required: there is no CPU fallback, and importing this module on
a machine without libhxmoe.so raises at first use.
"""
from __future__ import annotations

import ctypes as C
import json
import os
from dataclasses import dataclass, field
from typing import Optional

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libhxmoe.so")

# storage formats (GGML type ids) and status codes, as in include/hx_moe.h
F32, F16, Q8_0, Q4_K, Q6_K, BF16 = 0, 1, 8, 12, 14, 30
HX_HOST, HX_DEVICE = 0, 1
STATUS = {0: "HX_OK", 1: "HX_ERR_INVALID_ARGUMENT", 2: "HX_ERR_UNSUPPORTED", 3: "HX_ERR_DEVICE",
          4: "HX_ERR_WORKSPACE_TOO_SMALL", 5: "HX_ERR_OUT_OF_MEMORY"}

# every entry point include/hx_moe.h declares
EXPORTS = ("hx_moe_create", "hx_moe_destroy", "hx_moe_workspace_size", "hx_moe_forward", "hx_moe_forward_noalloc",
           "hx_moe_forward_host",
           "hx_moe_route", "hx_moe_router_logits", "hx_moe_decoder_mlp", "hx_quantize", "hx_dequantize",
           "hx_row_bytes", "hx_quantize_activations", "hx_moe_timing_begin", "hx_moe_timing_read", "hx_moe_timing_end",
           "hx_moe_timing_name", "hx_last_error")


class HxError(RuntimeError):
    def __init__(self, code: int, what: str):
        super().__init__(f"{what}: {STATUS.get(code, code)}: {last_error()}")
        self.code = code


class HxConfig(C.Structure):
    _fields_ = [("hidden_size", C.c_int32), ("num_experts", C.c_int32), ("num_experts_per_tok", C.c_int32),
                ("moe_intermediate_size", C.c_int32), ("shared_expert_intermediate_size", C.c_int32),
                ("norm_topk_prob", C.c_int32), ("act_dtype", C.c_int32)]


class HxWeights(C.Structure):
    _fields_ = [("location", C.c_int32),
                ("router_dtype", C.c_int32), ("router", C.c_void_p),
                ("gate_dtype", C.c_int32), ("experts_gate", C.c_void_p),
                ("up_dtype", C.c_int32), ("experts_up", C.c_void_p),
                ("down_dtype", C.c_int32), ("experts_down", C.c_void_p),
                ("shared_gate_dtype", C.c_int32), ("shared_gate", C.c_void_p),
                ("shared_up_dtype", C.c_int32), ("shared_up", C.c_void_p),
                ("shared_down_dtype", C.c_int32), ("shared_down", C.c_void_p),
                ("shared_expert_gate_dtype", C.c_int32), ("shared_expert_gate", C.c_void_p)]


_lib: Optional[C.CDLL] = None


def lib() -> C.CDLL:
    """Load libhxmoe.so (built in-tree by helexa_amd.build). Raises if absent."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m helexa_amd.build`")
        L = C.CDLL(LIB_PATH)
        vp, i64, i32 = C.c_void_p, C.c_int64, C.c_int
        sig = {
            "hx_moe_create": (i32, [C.POINTER(HxConfig), C.POINTER(HxWeights), i32, C.POINTER(vp)]),
            "hx_moe_destroy": (i32, [vp]),
            "hx_moe_workspace_size": (i32, [vp, i64, C.POINTER(C.c_size_t)]),
            "hx_moe_forward": (i32, [vp, vp, i64, vp, vp, C.c_size_t, vp, vp]),
            "hx_moe_forward_noalloc": (i32, [vp, vp, i64, vp, vp, vp]),
            "hx_moe_forward_host": (i32, [vp, vp, i64, vp, vp]),
            "hx_moe_route": (i32, [vp, vp, i64, vp, vp, vp, vp, vp, vp, vp, C.c_size_t, vp]),
            "hx_moe_router_logits": (i32, [vp, vp, i64, vp, vp, vp]),
            "hx_moe_decoder_mlp": (i32, [vp, vp, i64, vp, C.c_float, vp, C.c_size_t, vp]),
            "hx_quantize": (i32, [i32, vp, i64, i64, vp, vp]),
            "hx_dequantize": (i32, [i32, vp, i64, i64, vp, vp]),
            "hx_row_bytes": (i64, [i32, i64]),
            "hx_quantize_activations": (i32, [i32, vp, i32, i64, i64, vp, vp, vp]),
            "hx_moe_timing_begin": (i32, [vp, i32]),
            "hx_moe_timing_read": (i32, [vp, C.POINTER(C.c_double), C.POINTER(C.c_int64), C.POINTER(C.c_int)]),
            "hx_moe_timing_end": (i32, [vp, C.POINTER(C.c_double), C.POINTER(C.c_int64), C.POINTER(C.c_int)]),
            "hx_moe_timing_name": (C.c_char_p, [i32]),
            "hx_last_error": (C.c_char_p, []),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype, fn.argtypes = res, args
        _lib = L
    return _lib


def last_error() -> str:
    return lib().hx_last_error().decode(errors="replace")


def check(code: int, what: str) -> None:
    if code != 0:
        raise HxError(code, what)


def row_bytes(dtype: int, n: int) -> int:
    return int(lib().hx_row_bytes(dtype, n))


# ---------------------------------------------------------------------------- config
@dataclass
class TextConfig:
    """MoE fields of neuron's TextConfig (mod.rs:270-302) plus what the block needs."""
    hidden_size: int
    num_experts: int = 0
    num_experts_per_tok: int = 0
    moe_intermediate_size: int = 0
    shared_expert_intermediate_size: int = 0
    decoder_sparse_step: int = 1
    mlp_only_layers: list = field(default_factory=list)
    norm_topk_prob: bool = False
    num_hidden_layers: int = 1
    rms_norm_eps: float = 1e-6

    @classmethod
    def from_config_json(cls, text: str) -> "TextConfig":
        """Config::from_config_json (mod.rs:147-198): flat qwen3_next configs carry the
        fields at the top level, nested qwen3_5 ones under text_config."""
        v = json.loads(text)
        t = v.get("text_config", v) if v.get("model_type") != "qwen3_next" else v
        return cls(hidden_size=int(t["hidden_size"]), num_experts=int(t.get("num_experts", 0)),
                   num_experts_per_tok=int(t.get("num_experts_per_tok", 0)),
                   moe_intermediate_size=int(t.get("moe_intermediate_size", 0)),
                   shared_expert_intermediate_size=int(t.get("shared_expert_intermediate_size", 0)),
                   decoder_sparse_step=int(t.get("decoder_sparse_step", 1)),
                   mlp_only_layers=list(t.get("mlp_only_layers", [])),
                   norm_topk_prob=bool(t.get("norm_topk_prob", False)),
                   num_hidden_layers=int(t.get("num_hidden_layers", 1)),
                   rms_norm_eps=float(t.get("rms_norm_eps", 1e-6)))

    def layer_uses_moe(self, layer_idx: int) -> bool:
        """mod.rs:309-314"""
        return (self.num_experts > 0 and self.decoder_sparse_step > 0
                and layer_idx not in self.mlp_only_layers
                and (layer_idx + 1) % self.decoder_sparse_step == 0)


# ---------------------------------------------------------------------------- block
def _ptr(t) -> int:
    return 0 if t is None else int(t.data_ptr())


def _stream(stream=None) -> int:
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return int(s.cuda_stream)


def _check_bias(bias, E: int, device) -> None:
    """router_bias: None or a contiguous float32 [E] tensor on the block's device"""
    import torch
    if bias is None:
        return
    if bias.dtype != torch.float32 or tuple(bias.shape) != (E,) or not bias.is_contiguous() or bias.device != device:
        raise ValueError(f"router_bias must be a contiguous float32 [{E}] tensor on {device}")


def _check_acts(x, H: int, act: int, what: str = "xs") -> None:
    """activations: a CUDA tensor of the block's dtype with last dim H"""
    if not getattr(x, "is_cuda", False):
        raise ValueError(f"{what} must be a CUDA tensor")
    if x.shape[-1] != H:
        raise ValueError(f"{what}: last dim {x.shape[-1]} != hidden {H}")
    if _act_dtype(x.dtype) != act:
        raise TypeError(f"{what}: activation dtype differs from the block's")


def _act_dtype(torch_dtype) -> int:
    import torch
    if torch_dtype == torch.bfloat16:
        return BF16
    if torch_dtype == torch.float32:
        return F32
    raise TypeError(f"activations must be float32 or bfloat16, got {torch_dtype}")


class Qwen3_5MoeBlock:
    """One sparse-MoE block resident on a GPU.

    weights: dict name -> (dtype, torch tensor) with names router, gate, up, down,
    sgate, sup, sdown, seg (mlp.gate, experts.*.{gate,up,down}_proj,
    shared_expert.{gate,up,down}_proj, shared_expert_gate). Float tensors are
    float32 / bfloat16; quantised ones are uint8 GGUF rows. All on the same
    device (cuda) or all on the CPU.
    """

    def __init__(self, handle: int, cfg: TextConfig, act_dtype: int, device: int):
        self._h = C.c_void_p(handle)
        self.cfg = cfg
        self.act_dtype = act_dtype
        self.device = device

    @classmethod
    def load(cls, cfg: TextConfig, weights: dict, act_dtype: int = BF16, device: int = 0) -> "Qwen3_5MoeBlock":
        c = HxConfig(cfg.hidden_size, cfg.num_experts, cfg.num_experts_per_tok, cfg.moe_intermediate_size,
                     cfg.shared_expert_intermediate_size, int(bool(cfg.norm_topk_prob)), act_dtype)
        w = HxWeights()
        tensors = [t for _, t in weights.values()]
        on_dev = any(getattr(t, "is_cuda", False) for t in tensors)
        w.location = HX_DEVICE if on_dev else HX_HOST
        for key, field_ in (("router", "router"), ("gate", "experts_gate"), ("up", "experts_up"),
                            ("down", "experts_down"), ("sgate", "shared_gate"), ("sup", "shared_up"),
                            ("sdown", "shared_down"), ("seg", "shared_expert_gate")):
            if key in weights:
                dt, t = weights[key]
                if not t.is_contiguous():
                    raise ValueError(f"weight {key} must be contiguous")
                dname = {"experts_gate": "gate_dtype", "experts_up": "up_dtype", "experts_down": "down_dtype",
                         "router": "router_dtype"}.get(field_, field_ + "_dtype")
                setattr(w, dname, dt)
                setattr(w, field_, _ptr(t))
        out = C.c_void_p()
        check(lib().hx_moe_create(C.byref(c), C.byref(w), device, C.byref(out)), "hx_moe_create")
        return cls(out.value, cfg, act_dtype, device)

    def close(self) -> None:
        if self._h:
            lib().hx_moe_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def handle(self):
        return self._h

    def workspace_size(self, n_tokens: int) -> int:
        n = C.c_size_t()
        check(lib().hx_moe_workspace_size(self._h, n_tokens, C.byref(n)), "hx_moe_workspace_size")
        return n.value

    def forward(self, xs, router_bias=None, workspace=None, stream=None, out=None):
        """Module::forward: xs (b, l, hidden) or (T, hidden) on this GPU -> same shape.
        `out`, if given, is a contiguous tensor of xs's shape and dtype to write."""
        import torch
        _check_acts(xs, self.cfg.hidden_size, self.act_dtype)
        x = xs.contiguous()
        _check_bias(router_bias, self.cfg.num_experts, x.device)
        if out is None:
            y = torch.empty_like(x)
        else:
            if out.shape != x.shape or out.dtype != x.dtype or not out.is_contiguous():
                raise ValueError("out must be contiguous with the input's shape and dtype")
            y = out
        T = x.numel() // self.cfg.hidden_size
        ws_ptr, ws_n = (None, 0) if workspace is None else (_ptr(workspace), workspace.numel() * workspace.element_size())
        check(lib().hx_moe_forward(self._h, _ptr(x), T, _ptr(y), ws_ptr, ws_n, _ptr(router_bias), _stream(stream)),
              "hx_moe_forward")
        return y

    def forward_noalloc(self, xs, out, router_bias=None, stream=None):
        """forward() through hx_moe_forward_noalloc: no workspace argument and no
        allocation inside the library (its per-GPU scratch is the workspace). `out`
        is required, a contiguous tensor of xs's shape and dtype."""
        _check_acts(xs, self.cfg.hidden_size, self.act_dtype)
        _check_bias(router_bias, self.cfg.num_experts, xs.device)
        if not xs.is_contiguous():
            raise ValueError("xs must be contiguous (no copy is made here)")
        if out.shape != xs.shape or out.dtype != xs.dtype or not out.is_contiguous():
            raise ValueError("out must be contiguous with the input's shape and dtype")
        T = xs.numel() // self.cfg.hidden_size
        check(lib().hx_moe_forward_noalloc(self._h, _ptr(xs), T, _ptr(out), _ptr(router_bias), _stream(stream)),
              "hx_moe_forward_noalloc")
        return out

    def route(self, xs, router_bias=None, stream=None):
        """-> dict(topk_idx [T,k] i32, topk_w [T,k] f32, perm [T*k], offsets [E+1], inv [T*k])"""
        import torch
        _check_acts(xs, self.cfg.hidden_size, self.act_dtype)
        x = xs.contiguous()
        _check_bias(router_bias, self.cfg.num_experts, x.device)
        T = x.numel() // self.cfg.hidden_size
        k, E = self.cfg.num_experts_per_tok, self.cfg.num_experts
        dev = x.device
        out = dict(topk_idx=torch.empty((T, k), dtype=torch.int32, device=dev),
                   topk_w=torch.empty((T, k), dtype=torch.float32, device=dev),
                   perm=torch.empty(T * k, dtype=torch.int32, device=dev),
                   offsets=torch.empty(E + 1, dtype=torch.int32, device=dev),
                   inv=torch.empty(T * k, dtype=torch.int32, device=dev))
        check(lib().hx_moe_route(self._h, _ptr(x), T, _ptr(router_bias), _ptr(out["topk_idx"]), _ptr(out["topk_w"]),
                                 _ptr(out["perm"]), _ptr(out["offsets"]), _ptr(out["inv"]), None, 0,
                                 _stream(stream)), "hx_moe_route")
        return out

    def router_logits(self, xs, router_bias=None, stream=None):
        import torch
        _check_acts(xs, self.cfg.hidden_size, self.act_dtype)
        x = xs.contiguous()
        _check_bias(router_bias, self.cfg.num_experts, x.device)
        T = x.numel() // self.cfg.hidden_size
        out = torch.empty((T, self.cfg.num_experts), dtype=torch.float32, device=x.device)
        check(lib().hx_moe_router_logits(self._h, _ptr(x), T, _ptr(router_bias), _ptr(out), _stream(stream)),
              "hx_moe_router_logits")
        return out

    def decoder_mlp_(self, x, norm_w, eps: float, workspace=None, stream=None):
        """x <- x + moe(rmsnorm(x)) in place (decoder.rs:129-132). x: contiguous
        CUDA tensor [..., hidden] of the block's dtype; norm_w: contiguous float32
        [hidden] on the same device."""
        import torch
        H = self.cfg.hidden_size
        _check_acts(x, H, self.act_dtype, "x")
        if not x.is_contiguous():
            raise ValueError("x must be contiguous (it is updated in place)")
        if (norm_w.dtype != torch.float32 or tuple(norm_w.shape) != (H,) or not norm_w.is_contiguous()
                or norm_w.device != x.device):
            raise ValueError(f"norm_w must be a contiguous float32 [{H}] tensor on {x.device}")
        T = x.numel() // H
        ws_ptr, ws_n = (None, 0) if workspace is None else (_ptr(workspace), workspace.numel() * workspace.element_size())
        check(lib().hx_moe_decoder_mlp(self._h, _ptr(x), T, _ptr(norm_w), float(eps), ws_ptr, ws_n, _stream(stream)),
              "hx_moe_decoder_mlp")
        return x

    def timing_begin(self, max_calls: int) -> None:
        check(lib().hx_moe_timing_begin(self._h, max_calls), "hx_moe_timing_begin")

    def _timing(self, fn) -> dict:
        n = C.c_int(16)
        ms = (C.c_double * 16)()
        cnt = (C.c_int64 * 16)()
        check(fn(self._h, ms, cnt, C.byref(n)), fn.__name__)
        return {lib().hx_moe_timing_name(i).decode(): (ms[i], cnt[i]) for i in range(n.value)}

    def timing_read(self) -> dict:
        """{kernel slot: (summed ms, timed launches)} over the armed forwards"""
        return self._timing(lib().hx_moe_timing_read)

    def timing_end(self) -> dict:
        return self._timing(lib().hx_moe_timing_end)


def quantize(dtype: int, w, stream=None):
    """quantize_parallel on the device: float32 cuda tensor [..., cols] -> uint8 GGUF rows."""
    import torch
    w = w.contiguous()
    if w.dtype != torch.float32 or not w.is_cuda:
        raise TypeError("quantize needs a float32 cuda tensor")
    cols = w.shape[-1]
    rb = row_bytes(dtype, cols)
    if rb < 0:
        raise ValueError(f"{cols} columns do not tile into dtype {dtype} blocks")
    out = torch.empty(w.shape[:-1] + (rb,), dtype=torch.uint8, device=w.device)
    check(lib().hx_quantize(dtype, _ptr(w), w.numel() // cols, cols, _ptr(out), _stream(stream)), "hx_quantize")
    return out


def dequantize(dtype: int, q, cols: int, stream=None):
    import torch
    q = q.contiguous()
    rb = row_bytes(dtype, cols)
    rows = q.numel() // rb
    out = torch.empty(q.shape[:-1] + (cols,), dtype=torch.float32, device=q.device)
    check(lib().hx_dequantize(dtype, _ptr(q), rows, cols, _ptr(out), _stream(stream)), "hx_dequantize")
    return out


def quantize_activations(weight_dtype: int, x, stream=None):
    """The activation quantisation of the reference's quantised arm (the rows of
    an expert call of at most 64 rows, quantised to the weight type's vec_dot
    type: Q8_0 blocks for Q8_0 weights, Q8_K for Q4_K / Q6_K) on the device:
    float32 or bfloat16 cuda tensor [rows, cols] -> (int8 codes [rows, cols],
    float32 d [rows, cols / block])."""
    import torch
    x = x.contiguous()
    if not x.is_cuda or x.dim() != 2:
        raise TypeError("quantize_activations needs a 2-d cuda tensor")
    act = _act_dtype(x.dtype)
    rows, cols = x.shape
    blk = 32 if weight_dtype == Q8_0 else 256
    codes = torch.empty((rows, cols), dtype=torch.int8, device=x.device)
    d = torch.empty((rows, max(cols // blk, 1)), dtype=torch.float32, device=x.device)
    check(lib().hx_quantize_activations(weight_dtype, _ptr(x), act, rows, cols, _ptr(codes), _ptr(d), _stream(stream)),
          "hx_quantize_activations")
    return codes, d
