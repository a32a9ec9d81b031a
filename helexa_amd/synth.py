"""Seeded synthetic MoE blocks generated on the device (benchmarks and GPU tests).

Weights are N(0, std) f32 drawn with a seeded torch generator on the target
device, then stored in the requested format: float32, bfloat16 (round to
nearest even) or GGUF rows quantised on the device by hx_quantize. Activations
are N(0, 1). The configurations mirror the benchmark's:

    C1  hidden 256, 16 experts, top-4 renormalised, intermediate 128, shared 128, f32
    C2  Qwen3-Next-80B-A3B layer: hidden 2048, 512 experts, top-10, intermediate 512,
        shared 512; experts Q8_0, router and shared gate bf16, activations bf16
    C3  same shape, Q4_K_M: gate/up Q4_K, down Q6_K (routed and shared experts)
"""
from __future__ import annotations

from .moe import BF16, F32, Q4_K, Q6_K, Q8_0, TextConfig, quantize

C1 = TextConfig(hidden_size=256, num_experts=16, num_experts_per_tok=4, moe_intermediate_size=128,
                shared_expert_intermediate_size=128, norm_topk_prob=True)
A3B = TextConfig(hidden_size=2048, num_experts=512, num_experts_per_tok=10, moe_intermediate_size=512,
                 shared_expert_intermediate_size=512, norm_topk_prob=True, num_hidden_layers=48)

FMT_F32 = dict(router=F32, gate=F32, up=F32, down=F32, sgate=F32, sup=F32, sdown=F32, seg=F32)
FMT_Q8_0 = dict(router=BF16, gate=Q8_0, up=Q8_0, down=Q8_0, sgate=Q8_0, sup=Q8_0, sdown=Q8_0, seg=BF16)
FMT_Q4_K_M = dict(router=BF16, gate=Q4_K, up=Q4_K, down=Q6_K, sgate=Q4_K, sup=Q4_K, sdown=Q6_K, seg=BF16)
FMT_BF16 = dict(router=BF16, gate=BF16, up=BF16, down=BF16, sgate=BF16, sup=BF16, sdown=BF16, seg=BF16)


def shapes(cfg: TextConfig) -> dict:
    H, E, I, Is = cfg.hidden_size, cfg.num_experts, cfg.moe_intermediate_size, cfg.shared_expert_intermediate_size
    s = {"router": (E, H), "gate": (E, I, H), "up": (E, I, H), "down": (E, H, I)}
    if Is > 0:
        s.update({"sgate": (Is, H), "sup": (Is, H), "sdown": (H, Is), "seg": (1, H)})
    return s


def make_weights(cfg: TextConfig, formats: dict, seed: int, device="cuda", std: float = 0.02) -> dict:
    import torch
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    out = {}
    for key, shp in shapes(cfg).items():
        w = torch.randn(shp, generator=g, device=device, dtype=torch.float32).mul_(std)
        dt = formats[key]
        if dt == F32:
            out[key] = (F32, w)
        elif dt == BF16:
            out[key] = (BF16, w.to(torch.bfloat16))
        else:
            out[key] = (dt, quantize(dt, w))
        del w
    return out


def make_x(cfg: TextConfig, T: int, seed: int, act_dtype: int = BF16, device="cuda"):
    import torch
    g = torch.Generator(device=device)
    g.manual_seed(seed + 7919)
    x = torch.randn((T, cfg.hidden_size), generator=g, device=device, dtype=torch.float32)
    return x.to(torch.bfloat16) if act_dtype == BF16 else x


def zipf_bias(E: int, s: float, alpha: float, seed: int, device="cuda"):
    """router_bias[e] = alpha * ln(p_{pi(e)}), p_r proportional to r^-s, pi a seeded
    permutation of the ranks (the skewed-routing benchmark's hook)."""
    import torch
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    ranks = torch.randperm(E, generator=g) + 1
    p = ranks.double() ** (-s)
    p = p / p.sum()
    return (alpha * torch.log(p)).float().to(device)


def to_numpy(weights: dict) -> dict:
    """device weights -> numpy (bf16 as uint16 bits, GGUF as uint8) for the CPU checker"""
    import numpy as np
    import torch
    out = {}
    for k, (dt, t) in weights.items():
        t = t.detach().cpu().contiguous()
        if t.dtype == torch.bfloat16:
            out[k] = (dt, t.view(torch.int16).numpy().view(np.uint16))
        else:
            out[k] = (dt, t.numpy())
    return out
