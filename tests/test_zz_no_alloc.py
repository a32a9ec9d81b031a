"""hx_moe_forward_noalloc (the entry point that allocates nothing: its workspace
is the library's per-GPU scratch) against hx_moe_forward on the same inputs.
Both run the same kernels, so the outputs must agree bit for bit; two calls in a
row, the second on a smaller input, so a stale scratch from the first call
would show in the second."""
import ctypes as C

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import oracle as O  # noqa: E402
from tests.common import rel_err  # noqa: E402

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 64 << 20      # HX_NOALLOC_SCRATCH_BYTES in include/hx_moe.h


def _block(fmt_name, seed):
    import helexa_amd as hx
    from helexa_amd import synth
    cfg = synth.A3B
    print(f"[no_alloc] A3B {fmt_name} seed={seed}", flush=True)
    w = synth.make_weights(cfg, getattr(synth, fmt_name), seed)
    return hx.Qwen3_5MoeBlock.load(cfg, w, act_dtype=hx.BF16), w


@pytest.fixture(scope="module")
def q4km():
    blk, w = _block("FMT_Q4_K_M", 4101)
    yield blk, w
    blk.close()


@pytest.fixture(scope="module")
def q8():
    blk, w = _block("FMT_Q8_0", 4102)
    yield blk, w
    blk.close()


def _pair(blk, T, seed, bias=None):
    from helexa_amd import synth
    x = synth.make_x(blk.cfg, T, seed)
    ref = blk.forward(x, router_bias=bias)
    out = torch.full_like(x, float("nan"))
    blk.forward_noalloc(x, out, router_bias=bias)
    torch.cuda.synchronize()
    return x, ref, out


@pytest.mark.parametrize("sizes", [(512, 37), (8, 1), (300, 4)])
def test_noalloc_matches_forward_q4_k_m(q4km, sizes):
    blk, _ = q4km
    for i, T in enumerate(sizes):
        print(f"[no_alloc] Q4_K_M T={T} (call {i + 1} of {len(sizes)})", flush=True)
        _, ref, out = _pair(blk, T, 900 + 10 * T + i)
        assert torch.equal(out, ref), f"T={T}: noalloc output differs from hx_moe_forward"


def test_noalloc_matches_forward_q8_0_decode_and_oracle(q8):
    """C2 decode (T=1) after a T=8 call; the T=1 output also checked against the oracle"""
    from helexa_amd import synth
    blk, w = q8
    for T in (8, 1):
        print(f"[no_alloc] Q8_0 T={T}", flush=True)
        x, ref, out = _pair(blk, T, 1700 + T)
        assert torch.equal(out, ref)
    wnp = synth.to_numpy(w)
    cfg = blk.cfg
    orc = O.OracleMoe(cfg.hidden_size, cfg.num_experts, cfg.num_experts_per_tok, cfg.moe_intermediate_size,
                      cfg.shared_expert_intermediate_size, cfg.norm_topk_prob, O.BF16, wnp)
    xn = x.detach().cpu().view(torch.int16).numpy().view(np.uint16)
    r = orc.forward_candle(xn)   # the reference's arithmetic for GGUF experts
    got = out.float().cpu().numpy()
    assert rel_err(got, r) <= 1e-2


def test_noalloc_router_bias(q4km):
    from helexa_amd import synth
    blk, _ = q4km
    bias = synth.zipf_bias(blk.cfg.num_experts, 1.1, 0.5, 3)
    for T in (64, 2):
        print(f"[no_alloc] bias T={T}", flush=True)
        _, ref, out = _pair(blk, T, 40 + T, bias)
        assert torch.equal(out, ref)


def test_noalloc_limit_rejected(q4km):
    """the largest token count whose workspace fits the scratch runs; one more is
    refused with HX_ERR_WORKSPACE_TOO_SMALL (4) before anything is launched"""
    import helexa_amd as hx
    from helexa_amd import synth
    blk, _ = q4km
    lo, hi = 1, 1 << 16
    while lo < hi:
        mid = (lo + hi + 1) // 2
        if blk.workspace_size(mid) <= SCRATCH_BYTES:
            lo = mid
        else:
            hi = mid - 1
    t_max = lo
    print(f"[no_alloc] largest T in the scratch: {t_max}", flush=True)
    assert t_max >= 700      # the header's figure for the 80B-A3B shape
    x = synth.make_x(blk.cfg, t_max + 1, 5)
    out = torch.empty_like(x)
    with pytest.raises(hx.HxError) as ei:
        blk.forward_noalloc(x, out)
    assert ei.value.code == 4 and "scratch" in str(ei.value)
    # the refused call left the scratch usable
    _, ref, got = _pair(blk, 3, 77)
    assert torch.equal(got, ref)


def test_noalloc_on_a_side_stream_and_in_a_graph(q4km):
    """on a caller stream, and captured into a HIP graph replayed three times with
    eager forwards (own workspace) between the replays; every replay equals the
    eager result"""
    from helexa_amd import synth
    blk, _ = q4km
    x = synth.make_x(blk.cfg, 4, 321)
    ref = blk.forward(x)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    out = torch.zeros_like(x)
    with torch.cuda.stream(s):
        blk.forward_noalloc(x, out, stream=s)
    s.synchronize()
    assert torch.equal(out, ref)
    g = torch.cuda.CUDAGraph()
    gout = torch.zeros_like(x)
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            blk.forward_noalloc(x, gout, stream=s)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    for r in range(3):
        print(f"[no_alloc] graph replay {r}", flush=True)
        gout.fill_(float("nan"))
        other = synth.make_x(blk.cfg, 9, 600 + r)
        blk.forward(other)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(gout, ref), f"replay {r}"


def test_noalloc_bad_arguments(q4km):
    import helexa_amd as hx
    blk, _ = q4km
    L = hx.lib()
    assert L.hx_moe_forward_noalloc(None, None, 1, None, None, None) == 1
    assert L.hx_moe_forward_noalloc(blk.handle, None, 0, None, None, None) == 0   # zero tokens: no-op
    assert L.hx_moe_forward_noalloc(blk.handle, None, 2, None, None, None) == 1
    assert L.hx_moe_forward_noalloc(blk.handle, C.c_void_p(16), (1 << 24) + 1, C.c_void_p(16), None, None) == 2
