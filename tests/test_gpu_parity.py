"""GPU parity: libhxmoe.so (through its C ABI) against the CPU oracle on the same
seeded inputs. Routing (logits, top-k ids and weights, dispatch permutation) is
bit-exact; the activation codes of the reference's quantised arm are bit-exact;
outputs are within max|y-r|/max|r| <= 1e-2 for bf16 activations and <= 1e-4 for
f32 of the reference's arithmetic: for GGUF experts
the oracle's candle mode (expert calls of m <= 64 rows on Q8_0 / Q8_K activation
codes and integer block products, larger calls in f16), for f32 / bf16 experts
its exact mode (the reference's f32 Linear)."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import oracle as O  # noqa: E402
from tests.common import assert_topk_w, rel_err, report  # noqa: E402

pytestmark = pytest.mark.gpu

TOL_BF16, TOL_F32 = 1e-2, 1e-4
# GGUF experts against the oracle's candle-arithmetic mode (the reference's CPU
# path: its 8-bit activation quantisation alone puts it 0.7-2.2 % of max|y|
# from exact arithmetic): the same 1e-2 bar, and a cosine floor
TOL_CANDLE, COS_CANDLE = 1e-2, 0.9999


def _hx():
    import helexa_amd as hx
    from helexa_amd import synth
    return hx, synth


def oracle_for(cfg, wnp, act):
    return O.OracleMoe(cfg.hidden_size, cfg.num_experts, cfg.num_experts_per_tok, cfg.moe_intermediate_size,
                       cfg.shared_expert_intermediate_size, cfg.norm_topk_prob, act, wnp)


def x_np(x):
    x = x.detach().cpu().contiguous()
    return x.view(torch.int16).numpy().view(np.uint16) if x.dtype == torch.bfloat16 else x.numpy()


class Case:
    def __init__(self, cfg, fmt, seed, act):
        hx, synth = _hx()
        print(f"[case] H={cfg.hidden_size} E={cfg.num_experts} k={cfg.num_experts_per_tok} "
              f"I={cfg.moe_intermediate_size} fmt={fmt['gate']}/{fmt['down']} seed={seed}", flush=True)
        self.cfg, self.act, self.seed = cfg, act, seed
        self.w = synth.make_weights(cfg, fmt, seed)
        self.block = hx.Qwen3_5MoeBlock.load(cfg, self.w, act_dtype=act)
        self.wnp = synth.to_numpy(self.w)
        self.oracle = oracle_for(cfg, self.wnp, act)
        self.quant = gguf_experts(self.w)

    def x(self, T, seed=0):
        _, synth = _hx()
        return synth.make_x(self.cfg, T, self.seed * 1000 + seed, self.act)

    def ref(self, xin, bias=None):
        """the reference's output for x (numpy): candle arithmetic for GGUF experts, else exact"""
        return self.oracle.forward_candle(xin, bias=bias) if self.quant else self.oracle.forward(xin, bias=bias)

    def ref_tokens(self, xin, sel, bias=None):
        """the reference's output for the tokens sel of a forward of all of x"""
        if self.quant:
            return self.oracle.forward_candle_tokens(xin, sel, bias=bias)
        return self.oracle.forward(xin[sel], bias=bias)


def gguf_experts(w):
    """whether the expert projections are GGUF (the reference's MaybeQuantLinear arms apply)"""
    hx, _ = _hx()
    return any(w[k][0] in (hx.Q8_0, hx.Q4_K, hx.Q6_K) for k in ("gate", "up", "down") if k in w)


@pytest.fixture(scope="module")
def c1():
    _, synth = _hx()
    return Case(synth.C1, synth.FMT_F32, 2024, O.F32)


@pytest.fixture(scope="module")
def router_case():
    """A3B router shape (hidden 2048, 512 experts, top-10) with thin bf16 experts"""
    hx, synth = _hx()
    cfg = hx.TextConfig(hidden_size=2048, num_experts=512, num_experts_per_tok=10, moe_intermediate_size=64,
                        shared_expert_intermediate_size=64, norm_topk_prob=True)
    return Case(cfg, synth.FMT_BF16, 31, O.BF16)


@pytest.fixture(scope="module")
def c2():
    _, synth = _hx()
    return Case(synth.A3B, synth.FMT_Q8_0, 7, O.BF16)


# ------------------------------------------------------------------ weights
@pytest.mark.parametrize("dt", [O.Q8_0, O.Q4_K, O.Q6_K, O.BF16])
def test_device_quantiser_matches_oracle_bytes(dt):
    hx, _ = _hx()
    g = torch.Generator(device="cuda").manual_seed(5)
    w = torch.randn((96, 2048), generator=g, device="cuda") * 0.02
    w[3, :256] = 0.0                                  # all-zero blocks
    w[4, :32] = 1e-3                                  # constant block
    w[5, :256] = 0.3                                  # positive-constant superblock
    w[6, 32:64] = -0.01                               # negative-constant sub-block
    w[7, :32] = torch.tensor([127.0, 0.5, 4.5, -2.5, -0.5] + [0.0] * 27)   # Q8_0 halves
    lat = torch.arange(256, device="cuda", dtype=torch.float32)
    w[8, :256] = ((lat % 16) * 63.0 * 4.0 - 21.0) / 4096.0                 # Q4_K lattice
    w[9, :256] = ((lat % 64) - 32.0) * 77.0 / 4096.0                       # Q6_K lattice
    w[10, :] = torch.randn((2048,), generator=g, device="cuda") * 3.0      # large magnitudes
    q = hx.quantize(dt, w).cpu().numpy()
    ref = O.quantize(dt, w.cpu().numpy())
    assert np.array_equal(q.reshape(-1), ref.reshape(-1))


@pytest.mark.parametrize("dt", [O.Q8_0, O.Q4_K, O.Q6_K])
def test_device_dequantiser_matches_oracle(dt):
    hx, _ = _hx()
    g = torch.Generator(device="cuda").manual_seed(6)
    w = torch.randn((64, 512), generator=g, device="cuda") * 0.02
    q = hx.quantize(dt, w)
    got = hx.dequantize(dt, q, 512).cpu().numpy()
    ref = O.dequantize(dt, q.cpu().numpy(), 512)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("wdt", [O.Q8_0, O.Q4_K])
@pytest.mark.parametrize("xdt", ["bf16", "f32"])
def test_activation_codes_match_the_reference_quantiser(wdt, xdt):
    """hx_quantize_activations -- the quantisation every kernel of the
    quantised arm performs -- equals the oracle's restatement of candle's Q8_0 /
    Q8_K from_float bit for bit (codes and d): random rows, all-zero blocks,
    ties in |x| of opposite sign (the first one's sign decides iscale's), an
    all-negative block, values on the .5 rounding boundary (half away from
    zero), large and tiny magnitudes"""
    hx, _ = _hx()
    g = torch.Generator(device="cuda").manual_seed(31)
    rows, cols = 64, 2048
    x = torch.randn((rows, cols), generator=g, device="cuda")
    x[1, :256] = 0.0
    x[2, :256] = torch.randn((256,), generator=g, device="cuda") * 0.1
    x[2, 10], x[2, 200] = 5.0, -5.0          # tie in |x|, positive first
    x[3, :256] = torch.randn((256,), generator=g, device="cuda") * 0.1
    x[3, 10], x[3, 200] = -5.0, 5.0          # tie in |x|, negative first
    x[4, :256] = -x[4, :256].abs()
    x[5, :32] = torch.tensor([127.0, 2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 126.5] + [0.0] * 24)   # Q8_0: d = 1
    x[6, :256] = 0.0
    x[6, :8] = torch.tensor([-128.0, 2.5, -2.5, 0.5, -0.5, 127.5, -127.5, 128.0])           # Q8_K: iscale = 1
    x[7] *= 1e4
    x[8] *= 1e-6
    x[9, :32] = 0.0
    x[9, 5] = 1.0
    if xdt == "bf16":
        x = x.to(torch.bfloat16)
    codes, d = hx.quantize_activations(wdt, x)
    codes, d = codes.cpu().numpy(), d.cpu().numpy()
    xf = x.float().cpu().numpy()
    if wdt == O.Q8_0:
        blk = O.quantize(O.Q8_0, xf).reshape(rows, cols // 32, 34)
        ref_d = blk[:, :, :2].copy().view(np.float16).astype(np.float32).reshape(rows, cols // 32)
        ref_q = blk[:, :, 2:].copy().view(np.int8).reshape(rows, cols)
    else:
        ref_d, ref_q, _ = O.quant_q8_k(xf)
        ref_d, ref_q = ref_d.reshape(rows, cols // 256), ref_q.reshape(rows, cols)
    assert np.array_equal(codes, ref_q)
    assert np.array_equal(d.view(np.uint32), ref_d.astype(np.float32).view(np.uint32))
    if wdt != O.Q8_0:   # the first of two equal |x| sets the sign of iscale
        assert (codes[2, 10], codes[2, 200], codes[3, 10], codes[3, 200]) == (-128, 127, -128, 127)


# ------------------------------------------------------------------ routing
@pytest.mark.parametrize("T", [1, 3, 8, 9, 300])
def test_router_logits_bit_exact(router_case, T):
    c = router_case
    x = c.x(T, seed=T)
    got = c.block.router_logits(x).cpu().numpy()
    ref = c.oracle.logits(x_np(x))
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("T", [1, 2, 4, 5, 8, 9, 64, 1000, 2048, 3000])
def test_routing_and_dispatch_bit_exact(router_case, T):
    """Above 8 tokens the MFMA router splits K over 4 logit planes up to 1,984
    tokens and over 2 from there (2048, and the ragged 3000) at 512 experts; the
    4096-token C5 test takes 1."""
    c = router_case
    x = c.x(T, seed=100 + T)
    r = c.block.route(x)
    _, _, ix, wt = c.oracle.route(x_np(x))
    assert np.array_equal(r["topk_idx"].cpu().numpy(), ix)
    assert_topk_w(r["topk_w"].cpu().numpy(), wt, 10, exact=T <= 8)
    perm, offs, inv = O.dispatch(ix, c.cfg.num_experts)
    assert np.array_equal(r["perm"].cpu().numpy(), perm)
    assert np.array_equal(r["offsets"].cpu().numpy(), offs)
    assert np.array_equal(r["inv"].cpu().numpy(), inv)


@pytest.mark.parametrize("H,fmt,act", [(1032, "FMT_BF16", O.BF16), (2048, "FMT_F32", O.F32),
                                       (200, "FMT_F32", O.F32), (520, "FMT_BF16", O.BF16)])
def test_prefill_router_logits_bit_exact_shapes(H, fmt, act):
    """Prefill router tiles (more than 8 tokens): hidden sizes whose groups of 8
    leave the last pass of 64 lanes partly empty, and f32 inputs and weights."""
    hx, synth = _hx()
    cfg = hx.TextConfig(hidden_size=H, num_experts=40, num_experts_per_tok=4, moe_intermediate_size=32,
                        shared_expert_intermediate_size=32, norm_topk_prob=True)
    w = synth.make_weights(cfg, getattr(synth, fmt), 5)
    blk = hx.Qwen3_5MoeBlock.load(cfg, w, act_dtype=act)
    o = oracle_for(cfg, synth.to_numpy(w), act)
    for T in (9, 301):
        x = synth.make_x(cfg, T, 17 + T, act)
        got = blk.router_logits(x).cpu().numpy()
        ref = o.logits(x_np(x))
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (H, T)


def test_routing_ties_break_to_lower_id():
    """Duplicate router rows give exactly tied logits; the lower id must win."""
    hx, synth = _hx()
    cfg = hx.TextConfig(hidden_size=256, num_experts=64, num_experts_per_tok=6, moe_intermediate_size=32,
                        shared_expert_intermediate_size=0, norm_topk_prob=True)
    w = synth.make_weights(cfg, synth.FMT_BF16, 9)
    r = w["router"][1]
    r[32:] = r[:32]                                   # expert 32+i ties expert i
    blk = hx.Qwen3_5MoeBlock.load(cfg, w, act_dtype=hx.BF16)
    x = synth.make_x(cfg, 200, 9)
    got = blk.route(x)["topk_idx"].cpu().numpy()
    o = oracle_for(cfg, synth.to_numpy(w), O.BF16)
    ref = o.route(x_np(x))[2]
    assert np.array_equal(got, ref)
    # a twin 32+i is only ever picked together with i, and ranks right after it
    for row in got:
        for j, e in enumerate(row):
            if e >= 32:
                assert e - 32 in row[:j], row


@pytest.mark.parametrize("E", [40, 128])
def test_mfma_routing_all_tied_tokens_mixed_with_others(E):
    """prefill routing on MFMA: all-zero token rows give logits that tie
    everywhere (every interval straddles 0: all E experts are candidates, which
    above 64 sends the token to the exact path inside the routing wave) in the
    same launch as ordinary tokens; ids, permutation bit-exact either way"""
    hx, synth = _hx()
    cfg = hx.TextConfig(hidden_size=256, num_experts=E, num_experts_per_tok=6, moe_intermediate_size=32,
                        shared_expert_intermediate_size=32, norm_topk_prob=True)
    w = synth.make_weights(cfg, synth.FMT_BF16, 21)
    blk = hx.Qwen3_5MoeBlock.load(cfg, w, act_dtype=hx.BF16)
    o = oracle_for(cfg, synth.to_numpy(w), O.BF16)
    x = synth.make_x(cfg, 64, 21)
    x[32:] = 0
    x[40] = -x[3]
    r = blk.route(x)
    _, _, ix, wt = o.route(x_np(x))
    assert np.array_equal(r["topk_idx"].cpu().numpy(), ix)
    assert (ix[32:39] == np.arange(6)).all()
    assert_topk_w(r["topk_w"].cpu().numpy(), wt, 6, exact=False)
    perm, offs, inv = O.dispatch(ix, E)
    assert np.array_equal(r["perm"].cpu().numpy(), perm)
    assert np.array_equal(r["offsets"].cpu().numpy(), offs)


@pytest.mark.parametrize("H,E,k", [(1024, 64, 4), (1024, 1024, 1)])
def test_mfma_routing_split_planes(H, E, k):
    """the MFMA router's K split: H = 1024, E = 64, k = 4 sums four logit planes
    (4 K steps of 64 per workgroup); H = 1024, E = 1024, k = 1 has no room for
    the extra planes in front of the shared rows and runs one plane of 16 steps"""
    hx, synth = _hx()
    cfg = hx.TextConfig(hidden_size=H, num_experts=E, num_experts_per_tok=k, moe_intermediate_size=32,
                        shared_expert_intermediate_size=32, norm_topk_prob=True)
    w = synth.make_weights(cfg, synth.FMT_BF16, 23)
    blk = hx.Qwen3_5MoeBlock.load(cfg, w, act_dtype=hx.BF16)
    o = oracle_for(cfg, synth.to_numpy(w), O.BF16)
    for T in (9, 200):
        x = synth.make_x(cfg, T, 23 + T)
        r = blk.route(x)
        _, _, ix, wt = o.route(x_np(x))
        assert np.array_equal(r["topk_idx"].cpu().numpy(), ix), (H, E, k, T)
        assert_topk_w(r["topk_w"].cpu().numpy(), wt, k, exact=False)
        perm, offs, inv = O.dispatch(ix, E)
        assert np.array_equal(r["perm"].cpu().numpy(), perm)
        got = blk.forward(x).float().cpu().numpy()
        assert rel_err(got, o.forward(x_np(x))) <= TOL_BF16


@pytest.mark.parametrize("fmt,act,norm", [("FMT_F32", O.F32, True), ("FMT_BF16", O.BF16, False)])
def test_multi_block_dispatch_after_generic_routing(fmt, act, norm):
    """prefills routed by the per-token kernel (f32 tokens, or no
    renormalisation): the dispatch's own kernel builds the chunk counts and the
    token bitmap; T = 300 and 1000 leave the last bitmap word and the last
    256-token chunk partly filled"""
    hx, synth = _hx()
    cfg = hx.TextConfig(hidden_size=256, num_experts=96, num_experts_per_tok=8, moe_intermediate_size=32,
                        shared_expert_intermediate_size=32, norm_topk_prob=norm)
    w = synth.make_weights(cfg, getattr(synth, fmt), 41)
    blk = hx.Qwen3_5MoeBlock.load(cfg, w, act_dtype=act)
    o = oracle_for(cfg, synth.to_numpy(w), act)
    for T in (300, 1000):
        x = synth.make_x(cfg, T, 41 + T, act)
        r = blk.route(x)
        _, _, ix, wt = o.route(x_np(x))
        assert np.array_equal(r["topk_idx"].cpu().numpy(), ix), (fmt, norm, T)
        assert_topk_w(r["topk_w"].cpu().numpy(), wt, cfg.num_experts_per_tok, exact=True)
        perm, offs, inv = O.dispatch(ix, cfg.num_experts)
        assert np.array_equal(r["perm"].cpu().numpy(), perm), (fmt, norm, T)
        assert np.array_equal(r["offsets"].cpu().numpy(), offs)
        assert np.array_equal(r["inv"].cpu().numpy(), inv)
        got = blk.forward(x).float().cpu().numpy()
        assert rel_err(got, o.forward(x_np(x))) <= (TOL_F32 if act == O.F32 else TOL_BF16), (fmt, norm, T)


def test_mfma_routing_underflowing_probabilities():
    """a bias of -150 on 12 of 16 experts: their probabilities underflow to 0
    and the top 8 takes them by id; the MFMA routing must notice (selected exps
    below 2^-100) and route those tokens by the exact path"""
    hx, synth = _hx()
    cfg = hx.TextConfig(hidden_size=512, num_experts=16, num_experts_per_tok=8, moe_intermediate_size=32,
                        shared_expert_intermediate_size=0, norm_topk_prob=True)
    w = synth.make_weights(cfg, synth.FMT_BF16, 22)
    blk = hx.Qwen3_5MoeBlock.load(cfg, w, act_dtype=hx.BF16)
    o = oracle_for(cfg, synth.to_numpy(w), O.BF16)
    bias = torch.zeros(16, device="cuda")
    bias[[1, 2, 3, 5, 6, 8, 9, 10, 12, 13, 14, 15]] = -150.0
    x = synth.make_x(cfg, 50, 22)
    r = blk.route(x, router_bias=bias)
    _, _, ix, wt = o.route(x_np(x), bias=bias.cpu().numpy())
    assert np.array_equal(r["topk_idx"].cpu().numpy(), ix)
    assert set(ix[0, :4]) == {0, 4, 7, 11} and (ix[:, 4:] == [1, 2, 3, 5]).all()
    assert_topk_w(r["topk_w"].cpu().numpy(), wt, 8, exact=False)
    got = blk.forward(x, router_bias=bias).float().cpu().numpy()
    assert rel_err(got, o.forward(x_np(x), bias=bias.cpu().numpy())) <= TOL_BF16


def test_router_bias_hook(router_case):
    c = router_case
    _, synth = _hx()
    bias = synth.zipf_bias(c.cfg.num_experts, 1.1, 1.0, 3)
    x = c.x(40, seed=77)
    r = c.block.route(x, router_bias=bias)
    _, _, ix, wt = c.oracle.route(x_np(x), bias=bias.cpu().numpy())
    assert np.array_equal(r["topk_idx"].cpu().numpy(), ix)
    assert_topk_w(r["topk_w"].cpu().numpy(), wt, 10, exact=False)


# ------------------------------------------------------------------ forward
@pytest.mark.parametrize("T", [1, 4, 8, 32])
def test_forward_c1_f32(c1, T):
    x = c1.x(T, seed=T)
    got = c1.block.forward(x).cpu().numpy()
    ref = c1.oracle.forward(x_np(x))
    assert rel_err(got, ref) <= TOL_F32


def test_forward_c1_matches_transformers_golden(c1):
    """the C1 block at the golden fixture's seed, end to end on the GPU"""
    import os
    hx, synth = _hx()
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "c1_transformers.npz"))
    from tests.common import make_f32_block, make_x
    cfg = synth.C1
    w = make_f32_block(int(g["seed"]), cfg.hidden_size, cfg.num_experts, cfg.moe_intermediate_size,
                       cfg.shared_expert_intermediate_size)
    dev = {k: (hx.F32, torch.from_numpy(v).cuda()) for k, v in w.items()}
    blk = hx.Qwen3_5MoeBlock.load(cfg, dev, act_dtype=hx.F32)
    x = torch.from_numpy(make_x(int(g["seed"]), 32, cfg.hidden_size)).cuda()
    r = blk.route(x)
    assert np.array_equal(r["topk_idx"].cpu().numpy(), g["topk_idx"])
    assert rel_err(blk.forward(x).cpu().numpy(), g["y"]) <= TOL_F32
    xs3 = x.reshape(1, 32, cfg.hidden_size)                     # (b, l, hidden) in, same shape out
    assert blk.forward(xs3).shape == xs3.shape


@pytest.mark.parametrize("T", [1, 4, 8])
def test_forward_c2_decode_q8_0(c2, T):
    x = c2.x(T, seed=T)
    got = c2.block.forward(x).float().cpu().numpy()
    ref = c2.ref(x_np(x))
    assert rel_err(got, ref) <= TOL_BF16


@pytest.mark.parametrize("H,I,gfmt,dfmt", [(256, 96, "Q4_K", "Q8_0"), (512, 96, "Q4_K", "Q8_0"),
                                          (288, 256, "Q8_0", "Q6_K")])
def test_blocked_layouts_partial_row_groups(H, I, gfmt, dfmt):
    """Q4_K and Q6_K matrices are stored in row groups of the largest power of
    two up to 64 / 128 that divides the row count: gate/up with 96 rows and
    down with 288 rows use 32-row groups (every prefill MFMA shape uses full
    64 / 128-row groups); decode (the fast one-token kernels at H = 512) and
    the generic prefill read them through the same address functions"""
    hx, synth = _hx()
    cfg = hx.TextConfig(hidden_size=H, num_experts=16, num_experts_per_tok=4, moe_intermediate_size=I,
                        shared_expert_intermediate_size=I, norm_topk_prob=True)
    g, d = getattr(hx, gfmt), getattr(hx, dfmt)
    fmt = dict(router=hx.BF16, gate=g, up=g, down=d, sgate=g, sup=g, sdown=d, seg=hx.BF16)
    c = Case(cfg, fmt, 57, O.BF16)
    for T in (1, 4, 40):
        x = c.x(T, seed=T)
        got = c.block.forward(x).float().cpu().numpy()
        assert rel_err(got, c.ref(x_np(x))) <= TOL_BF16, (H, I, gfmt, dfmt, T)


@pytest.mark.parametrize("pattern", [[0] * 8, [0, 0, 0, 0, 0, 1, 1, 2], [0, 1, 0, 1, 0, 1, 0, 1]])
def test_forward_c2_decode_repeated_tokens(c2, pattern):
    """tokens that share experts: slots of several rows, which for T = 8 and
    k = 10 (80 assignments) cross the 64-entry boundary of the dispatch"""
    base = c2.x(3, seed=77)
    x = base[torch.tensor(pattern, device=base.device)].contiguous()
    r = c2.block.route(x)
    _, _, ix, wt = c2.oracle.route(x_np(x))
    assert np.array_equal(r["topk_idx"].cpu().numpy(), ix)
    assert np.array_equal(r["topk_w"].cpu().numpy().view(np.uint32), wt.view(np.uint32))
    perm, offs, inv = O.dispatch(ix, c2.cfg.num_experts)
    assert np.array_equal(r["perm"].cpu().numpy(), perm)
    assert np.array_equal(r["offsets"].cpu().numpy(), offs)
    got = c2.block.forward(x).float().cpu().numpy()
    assert rel_err(got, c2.ref(x_np(x))) <= TOL_BF16


@pytest.mark.parametrize("T", [2, 8])
def test_decode_tokens_isolated_from_an_overflowing_token(c2, T):
    """a token whose activations are huge (1e38: its gate / up products and
    down rows overflow to inf / NaN) leaves the other tokens' outputs finite
    and bit for bit what they are beside an ordinary token: each token's
    output sums its own rows only"""
    x = c2.x(T, seed=31)
    y0 = c2.block.forward(x).float().cpu().numpy()
    xb = x.clone()
    xb[T - 1] = 1e38
    y1 = c2.block.forward(xb).float().cpu().numpy()
    assert np.isfinite(y1[:T - 1]).all()
    assert np.array_equal(y1[:T - 1].view(np.uint32), y0[:T - 1].view(np.uint32))
    assert not np.isfinite(y1[T - 1]).all()   # the overflow did happen


def test_prefill_tokens_isolated_from_an_overflowing_token(q4km):
    """the same at a prefill size (64 tokens, MFMA routing and GEMM tiles): the
    other tokens keep their routing bit for bit and finite outputs within the
    bar of those beside an ordinary token (an expert that gains the bad
    token's row may cross the 64-row arm threshold, so not bit for bit)"""
    T = 64
    x = q4km.x(T, seed=32)
    r0 = q4km.block.route(x)
    y0 = q4km.block.forward(x).float().cpu().numpy()
    xb = x.clone()
    xb[T - 1] = 1e38
    r1 = q4km.block.route(xb)
    y1 = q4km.block.forward(xb).float().cpu().numpy()
    assert np.array_equal(r1["topk_idx"].cpu().numpy()[:T - 1], r0["topk_idx"].cpu().numpy()[:T - 1])
    assert np.isfinite(y1[:T - 1]).all()
    assert rel_err(y1[:T - 1], y0[:T - 1]) <= TOL_BF16


@pytest.mark.parametrize("T", [1, 4])
def test_route_after_forward_publishes_everything(c2, T):
    """a decode forward writes only its plan into the handle's workspace; a
    route() on the same workspace right after must still publish the whole
    routing (ids, weights, permutation, offsets), bit-exact"""
    x = c2.x(T, seed=90 + T)
    c2.block.forward(x)
    r = c2.block.route(x)
    _, _, ix, wt = c2.oracle.route(x_np(x))
    assert np.array_equal(r["topk_idx"].cpu().numpy(), ix)
    assert np.array_equal(r["topk_w"].cpu().numpy().view(np.uint32), wt.view(np.uint32))
    perm, offs, inv = O.dispatch(ix, c2.cfg.num_experts)
    assert np.array_equal(r["perm"].cpu().numpy(), perm)
    assert np.array_equal(r["offsets"].cpu().numpy(), offs)
    assert np.array_equal(r["inv"].cpu().numpy(), inv)


@pytest.mark.parametrize("T", [1, 4])
def test_forward_decode_with_router_bias(q4km, T):
    """decode with the router-bias hook: the logits are no longer bf16 values
    (bias added after the rounding); routing through the fast decode kernels
    against the oracle with the same bias, and the routing itself bit-exact"""
    _, synth = _hx()
    bias = synth.zipf_bias(q4km.cfg.num_experts, 1.1, 2.0, 11)
    x = q4km.x(T, seed=40 + T)
    r = q4km.block.route(x, router_bias=bias)
    _, _, ix, wt = q4km.oracle.route(x_np(x), bias=bias.cpu().numpy())
    assert np.array_equal(r["topk_idx"].cpu().numpy(), ix)
    assert np.array_equal(r["topk_w"].cpu().numpy().view(np.uint32), wt.view(np.uint32))
    got = q4km.block.forward(x, router_bias=bias).float().cpu().numpy()
    assert rel_err(got, q4km.ref(x_np(x), bias=bias.cpu().numpy())) <= TOL_BF16


@pytest.fixture(scope="module")
def q4km_raw():
    """the A3B shape with norm_topk_prob = false (raw softmax weights)"""
    hx, synth = _hx()
    cfg = hx.TextConfig(hidden_size=2048, num_experts=512, num_experts_per_tok=10, moe_intermediate_size=512,
                        shared_expert_intermediate_size=512, norm_topk_prob=False)
    return Case(cfg, synth.FMT_Q4_K_M, 17, O.BF16)


@pytest.mark.parametrize("T", [1, 4, 8])
def test_forward_decode_without_renormalisation(q4km_raw, T):
    """norm_topk_prob = false through the fast decode kernels, Q4_K_M"""
    x = q4km_raw.x(T, seed=60 + T)
    got = q4km_raw.block.forward(x).float().cpu().numpy()
    assert rel_err(got, q4km_raw.ref(x_np(x))) <= TOL_BF16


@pytest.fixture(scope="module")
def q4km():
    _, synth = _hx()
    return Case(synth.A3B, synth.FMT_Q4_K_M, 13, O.BF16)


@pytest.mark.parametrize("T", [2, 3, 5, 7])
def test_forward_q4_k_m_decode_batches(q4km, T):
    """decode for T > 1 at every group count of the pipelined down kernel (rows
    of h = T (k + 1) in groups of 24: one to four groups)"""
    x = q4km.x(T, seed=T)
    got = q4km.block.forward(x).float().cpu().numpy()
    assert rel_err(got, q4km.ref(x_np(x))) <= TOL_BF16


@pytest.mark.parametrize("T", [9, 24, 40])
def test_forward_q4_k_m_prefill_small_tiles(q4km, T):
    """prefill tiles with 1, 2 and 3 sixteen-row sub-tiles in use (routed tiles of
    a row or two; the shared expert's tile holds all T rows)"""
    x = q4km.x(T, seed=100 + T)
    got = q4km.block.forward(x).float().cpu().numpy()
    assert rel_err(got, q4km.ref(x_np(x))) <= TOL_BF16


def test_forward_q4_k_m_prefill_sampled_tokens():
    hx, synth = _hx()
    c = Case(synth.A3B, synth.FMT_Q4_K_M, 11, O.BF16)
    T = 2048
    x = c.x(T, seed=5)
    y = c.block.forward(x)
    r = c.block.route(x)
    _, _, ix, _ = c.oracle.route(x_np(x))
    assert np.array_equal(r["topk_idx"].cpu().numpy(), ix)
    sample = np.linspace(0, T - 1, 12).astype(int)
    ref = c.ref_tokens(x_np(x), sample)
    assert rel_err(y.float().cpu().numpy()[sample], ref) <= TOL_BF16
    # the decode path on the same block
    xd = c.x(3, seed=6)
    assert rel_err(c.block.forward(xd).float().cpu().numpy(), c.ref(x_np(xd))) <= TOL_BF16


def test_forward_host_entry_matches_device(c1):
    import ctypes as C
    hx, _ = _hx()
    x = c1.x(5, seed=3)
    dev = c1.block.forward(x).cpu().numpy()
    xh = x.cpu().numpy()
    yh = np.empty_like(xh)
    hx.moe.check(hx.lib().hx_moe_forward_host(c1.block.handle, xh.ctypes.data_as(C.c_void_p), 5,
                                              yh.ctypes.data_as(C.c_void_p), None), "forward_host")
    assert np.array_equal(dev, yh)


def test_decoder_mlp_residual(c1):
    hx, _ = _hx()
    x = c1.x(6, seed=4)
    w = torch.linspace(-0.5, 0.5, c1.cfg.hidden_size, device="cuda")
    ref_n = O.rmsnorm(x_np(x), w.cpu().numpy(), 1e-6, O.F32)
    ref = x_np(x) + c1.oracle.forward(ref_n)
    got = c1.block.decoder_mlp_(x.clone(), w, 1e-6).cpu().numpy()
    assert rel_err(got, ref) <= TOL_F32


# ------------------------------------------------------------------ edges / errors
def test_zero_tokens_is_noop(c1):
    x = torch.empty((0, c1.cfg.hidden_size), device="cuda")
    assert c1.block.forward(x).shape == (0, c1.cfg.hidden_size)


def test_workspace_too_small_is_an_error(c1):
    hx, _ = _hx()
    ws = torch.empty(16, dtype=torch.uint8, device="cuda")
    with pytest.raises(hx.HxError) as e:
        c1.block.forward(c1.x(4), workspace=ws)
    assert e.value.code == 4


def test_caller_workspace_and_stream(c1):
    x = c1.x(20, seed=8)
    ref = c1.block.forward(x)
    ws = torch.empty(c1.block.workspace_size(20), dtype=torch.uint8, device="cuda")
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        y = c1.block.forward(x, workspace=ws, stream=s)
    s.synchronize()
    assert torch.equal(y, ref)


def test_invalid_configs_are_rejected():
    hx, synth = _hx()
    w = synth.make_weights(synth.C1, synth.FMT_F32, 1)
    bad = hx.TextConfig(hidden_size=256, num_experts=16, num_experts_per_tok=17, moe_intermediate_size=128,
                        shared_expert_intermediate_size=128, norm_topk_prob=True)
    with pytest.raises(hx.HxError) as e:
        hx.Qwen3_5MoeBlock.load(bad, w, act_dtype=hx.F32)
    assert e.value.code == 1 and "exceeds num_experts" in str(e.value)
    qcfg = hx.TextConfig(hidden_size=256, num_experts=16, num_experts_per_tok=4, moe_intermediate_size=128,
                         shared_expert_intermediate_size=128, norm_topk_prob=True)
    wq = dict(w)
    wq["down"] = (hx.Q6_K, torch.zeros((16, 256, 10), dtype=torch.uint8, device="cuda"))  # I=128 not /256
    with pytest.raises(hx.HxError) as e:
        hx.Qwen3_5MoeBlock.load(qcfg, wq, act_dtype=hx.F32)
    assert e.value.code == 1


def test_forward_q8_0_prefill_sampled_tokens(c2):
    """prefill (MFMA grouped GEMMs) on the C2 block: 300 tokens, ragged M tiles"""
    x = c2.x(300, seed=9)
    y = c2.block.forward(x).float().cpu().numpy()
    sample = np.array([0, 1, 57, 150, 299])
    assert rel_err(y[sample], c2.ref_tokens(x_np(x), sample)) <= TOL_BF16


@pytest.mark.parametrize("T", [2048, 2049])
def test_forward_prefill_stream_threshold(c2, T):
    """Up to 2048 tokens the shared expert's tiles run inside the routed
    launches on one stream; from 2049 its GEMMs run on the side stream, here
    with a last shared tile of one row."""
    x = c2.x(T, seed=21)
    y = c2.block.forward(x).float().cpu().numpy()
    sample = np.unique([0, 777, 2047, T - 1])
    assert rel_err(y[sample], c2.ref_tokens(x_np(x), sample)) <= TOL_BF16


def test_forward_skewed_routing_prefill(c2):
    """Zipf router bias: a few experts take most rows, so their segments span
    several 64-row M tiles (the skewed-prefill shape)."""
    _, synth = _hx()
    bias = synth.zipf_bias(c2.cfg.num_experts, 1.1, 8.0, 5)
    x = c2.x(700, seed=10)
    r = c2.block.route(x, router_bias=bias)
    counts = np.diff(r["offsets"].cpu().numpy())
    assert counts.max() > 128                       # at least one expert spans 3+ tiles
    y = c2.block.forward(x, router_bias=bias).float().cpu().numpy()
    sample = np.array([3, 100, 350, 699])
    ref = c2.ref_tokens(x_np(x), sample, bias=bias.cpu().numpy())
    assert rel_err(y[sample], ref) <= TOL_BF16


# ------------------------------------------------------------------ C4 / C5 shapes
def test_c4_stack_layers_q4_k_m():
    """Two Q4_K_M layers of the C4 stack (x <- x + moe(rmsnorm(x)), the (1 + w)
    RMSNorm scaling with a per-channel weight, attention skipped) at B = 1, 3, 4,
    7, 8 (an odd B leaves the router's last token pair one token): each layer's
    output against the oracle applied to that layer's bf16 input."""
    _, synth = _hx()
    layers = [Case(synth.A3B, synth.FMT_Q4_K_M, 40 + i, O.BF16) for i in range(2)]
    w = torch.linspace(-0.5, 0.5, synth.A3B.hidden_size, device="cuda")   # per-channel norm weights
    wn = w.cpu().numpy()
    for B in (1, 3, 4, 7, 8):
        x = layers[0].x(B, seed=20 + B)
        for c in layers:
            xin = x_np(x)
            xn = O.f32_to_bf16_bits(O.rmsnorm(xin, wn, 1e-6, O.BF16))
            moe = O.bf16_bits_to_f32(O.f32_to_bf16_bits(c.ref(xn)))
            ref = O.bf16_bits_to_f32(xin) + moe
            print(f"[c4] B={B} layer seed={c.seed}", flush=True)
            x = c.block.decoder_mlp_(x, w, 1e-6)
            assert rel_err(x.float().cpu().numpy(), ref) <= TOL_BF16


def test_c5_skewed_prefill_4096():
    """C5 shape: 4096 tokens, Q4_K_M, Zipf(1.1) router bias scaled so the top 8
    experts take roughly 40% of the assignments. Routing bit-exact for every
    token, outputs on sampled tokens."""
    _, synth = _hx()
    c = Case(synth.A3B, synth.FMT_Q4_K_M, 13, O.BF16)
    T = 4096
    base = synth.zipf_bias(c.cfg.num_experts, 1.1, 1.0, 11)
    bias = base * 0.58
    x = c.x(T, seed=12)
    r = c.block.route(x, router_bias=bias)
    _, _, ix, wt = c.oracle.route(x_np(x), bias=bias.cpu().numpy())
    got_ix = r["topk_idx"].cpu().numpy()
    assert np.array_equal(got_ix, ix)
    assert_topk_w(r["topk_w"].cpu().numpy(), wt, 10, exact=False)
    top8 = torch.argsort(base, descending=True)[:8].cpu().numpy()
    share = np.isin(got_ix, top8).mean()
    assert 0.3 < share < 0.5
    perm, offsets, inv = O.dispatch(ix, c.cfg.num_experts)
    assert np.array_equal(r["perm"].cpu().numpy(), perm)
    assert np.array_equal(r["offsets"].cpu().numpy(), offsets)
    y = c.block.forward(x, router_bias=bias).float().cpu().numpy()
    sample = np.linspace(0, T - 1, 10).astype(int)
    ref = c.ref_tokens(x_np(x), sample, bias=bias.cpu().numpy())
    ex = c.oracle.forward(x_np(x)[sample], bias=bias.cpu().numpy())
    report("C5 Q4_K_M T=4096 sampled tokens vs candle arithmetic", y[sample], ref)
    report("C5 Q4_K_M T=4096 sampled tokens vs exact", y[sample], ex)
    assert rel_err(y[sample], ref) <= TOL_BF16


# ------------------------------------------------------------------ both oracle modes
def _both(tag, got, c, xin, bias=None):
    """GPU output against the candle-arithmetic mode (the reference's arithmetic
    for these GGUF experts: the gate, TOL_CANDLE and COS_CANDLE) and the exact
    mode (reported: the reference's own distance from exact arithmetic is the
    8-bit quantisation of its activations); prints the three error figures of
    each"""
    assert c.quant
    ref = c.oracle.forward(xin, bias=bias)
    cnd = c.oracle.forward_candle(xin, bias=bias)
    report(f"{tag} vs exact", got, ref)
    ec = report(f"{tag} vs candle arithmetic", got, cnd)
    report(f"{tag} exact vs candle arithmetic", ref, cnd)
    assert ec["normwise"] <= TOL_CANDLE and ec["cosine"] >= COS_CANDLE


@pytest.mark.parametrize("T", [1, 4, 8])
def test_c2_against_both_oracle_modes(c2, T):
    x = c2.x(T, seed=300 + T)
    _both(f"C2 Q8_0 T={T}", c2.block.forward(x).float().cpu().numpy(), c2, x_np(x))


def test_c3_against_both_oracle_modes():
    """C3: the full 2048-token Q4_K_M prefill in both modes (candle's m <= 64
    vec_dot path for the routed experts, its f16 path for the shared expert)"""
    _, synth = _hx()
    c = Case(synth.A3B, synth.FMT_Q4_K_M, 19, O.BF16)
    x = c.x(2048, seed=7)
    _both("C3 Q4_K_M T=2048", c.block.forward(x).float().cpu().numpy(), c, x_np(x))


def test_c4_layers_against_both_oracle_modes():
    """two C4 layers at B = 1, 4, 8 (RMSNorm weight linspace(-0.5, 0.5) under the
    (1 + w) scaling): each layer's MoE output on its RMSNorm'd bf16 input, in both
    modes (the stack's residual outputs are checked against the exact mode by
    test_c4_stack_layers_q4_k_m; here the MoE term alone, which the residual
    would dwarf)"""
    _, synth = _hx()
    layers = [Case(synth.A3B, synth.FMT_Q4_K_M, 60 + i, O.BF16) for i in range(2)]
    w = torch.linspace(-0.5, 0.5, synth.A3B.hidden_size, device="cuda")
    wn = w.cpu().numpy()
    for B in (1, 4, 8):
        x = layers[0].x(B, seed=70 + B)
        for c in layers:
            xn = O.f32_to_bf16_bits(O.rmsnorm(x_np(x), wn, 1e-6, O.BF16))
            xnd = torch.from_numpy(xn.view(np.int16)).cuda().view(torch.bfloat16)
            _both(f"C4 B={B} layer seed={c.seed}", c.block.forward(xnd).float().cpu().numpy(), c, xn)
            x = c.block.decoder_mlp_(x, w, 1e-6)
