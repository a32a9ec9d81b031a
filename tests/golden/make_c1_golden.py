"""Writes tests/golden/c1_transformers.npz: the C1 block (hidden 256, 16 experts,
top-4 renormalised, intermediate 128, shared expert 128 with sigmoid gate, f32,
32 tokens) evaluated by HF transformers' Qwen3NextSparseMoeBlock -- the upstream
implementation neuron's qwen3_next parity test pins against
(crates/neuron/tests/qwen3_next_parity.rs:1-12). Inputs come from the seeded
numpy generator in tests/common.py, so only outputs are stored.

Run: python tests/golden/make_c1_golden.py   (CPU; needs transformers + torch)
"""
import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from tests.common import C1, make_f32_block, make_x  # noqa: E402

SEED = 2024


def hf_block(w, H, E, k, I, Is, norm):
    from transformers.models.qwen3_next.configuration_qwen3_next import Qwen3NextConfig
    from transformers.models.qwen3_next.modeling_qwen3_next import Qwen3NextSparseMoeBlock

    cfg = Qwen3NextConfig(hidden_size=H, num_experts=E, num_experts_per_tok=k, moe_intermediate_size=I,
                          shared_expert_intermediate_size=Is, norm_topk_prob=norm, hidden_act="silu")
    blk = Qwen3NextSparseMoeBlock(cfg).eval()
    with torch.no_grad():
        blk.gate.weight.copy_(torch.from_numpy(w["router"]))
        blk.experts.gate_up_proj.copy_(torch.from_numpy(np.concatenate([w["gate"], w["up"]], axis=1)))
        blk.experts.down_proj.copy_(torch.from_numpy(w["down"]))
        blk.shared_expert.gate_proj.weight.copy_(torch.from_numpy(w["sgate"]))
        blk.shared_expert.up_proj.weight.copy_(torch.from_numpy(w["sup"]))
        blk.shared_expert.down_proj.weight.copy_(torch.from_numpy(w["sdown"]))
        blk.shared_expert_gate.weight.copy_(torch.from_numpy(w["seg"]))
    return blk


def run(seed=SEED):
    H, E, k, I, Is, T = C1["H"], C1["E"], C1["k"], C1["I"], C1["Is"], C1["T"]
    w = make_f32_block(seed, H, E, I, Is)
    x = make_x(seed, T, H)
    blk = hf_block(w, H, E, k, I, Is, True)
    with torch.no_grad():
        xt = torch.from_numpy(x).reshape(1, T, H)
        y = blk(xt)
        y = y[0] if isinstance(y, tuple) else y
        _, scores, idx = blk.gate(xt.reshape(T, H))
    return dict(seed=np.int64(seed), y=y.reshape(T, H).numpy().astype(np.float32),
                topk_idx=idx.numpy().astype(np.int32), topk_w=scores.numpy().astype(np.float32))


if __name__ == "__main__":
    out = run()
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c1_transformers.npz")
    np.savez_compressed(path, **out)
    print("wrote", path, {k: v.shape for k, v in out.items()})
