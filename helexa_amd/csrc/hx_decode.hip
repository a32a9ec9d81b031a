// Decode expert kernels for bf16 activations (T <= HX_DECODE_MAX_T).
//
// Reference: Qwen3_5MLP::forward (crates/neuron/src/harness/arch/qwen3_5/mlp.rs:54-60)
// inside the scatter loop of Module::forward (moe.rs:177-195) and
// MaybeQuantLinear's GGUF GEMV arm (crates/neuron/src/harness/tp/tp_linear.rs:120-137):
// every expert call of a decode step has m = T <= 8 <= 64 rows, so the
// reference quantises each activation row to the weight type's vec_dot type
// (Q8_0 or Q8_K, hx_quant.h) and sums integer products of codes per block.
//
// Arithmetic: the activation codes (integers in [-128, 127]) come as int8 in
// chunk records (hx_quant.h): the tokens' records are written by the router
// kernel, those of the SwiGLU rows h (stored as f32) by the down kernel itself
// (one token) or by k_hrec. Each quantised weight becomes an int8 byte -- Q8_0
// its code, Q4_K its nibble, Q6_K its 6-bit code (unsigned), assembled four at
// a time by masks -- and v_dot4_i32_i8 sums four products into an int32, so
// the block dot products are exact integers, as in the reference:
// sum((u - bias) q) = sum(u q) - bias sum(q) with the record's code sums. Per
// chunk the float steps follow: Q8_0 (d_w isum) d_x; Q4_K (d_w d_x) S -
// (dmin_w d_x) M with S the scaled sums and M the mins times the code sums;
// Q6_K (d_w d_x) S, S the int32 sum of the scaled sub-block sums.
#include "hx_internal.h"
#include "hx_quant.h"
#include "hx_route_small.h"
#include "hx_router_dev.h"

namespace hx {

typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) u32x4v lds_v4;

// v_dot4_i32_i8: acc + the sum of the four products of the signed bytes of w and x
HX_DEV int dot4(uint32_t w, uint32_t x, int acc) { return __builtin_amdgcn_sdot4((int)w, (int)x, acc, false); }

// DChunk<FMT>: one lane's chunk of 32 weights of a row and its dot product
// with the chunk's activation codes. xp: the record's 16 f16 code pairs; xs:
// the code sums the format's offset correction needs (rec_sums); dx: the
// activation block's d. Slot g of a chunk (xp[4g .. 4g + 3]) holds elements
// x_group_off(c, g) .. + 7 of the row.
template <int FMT>
struct DChunk;

// Q8_0 planar: chunk = one 32-weight block: 32 int8 + f16 scale
template <>
struct DChunk<HX_Q8_0> {
  static constexpr int NX = 8;   // words of activation codes per chunk
  static constexpr int NS = 1;   // code sums per chunk (unused: the weights are signed)
  using Raw = Chunk<HX_Q8_0>::Raw;
  HX_DEV static void load(const uint8_t* mat, int R, int K, int row, int c, Raw& r) {
    Chunk<HX_Q8_0>::load(mat, R, K, row, c, r);
  }
  // activation positions: elements 32c .. 32c+31; slot g of 8 -> words xp[2g ..]
  HX_DEV static int x_group_off(int c, int g) { return 32 * c + 8 * g; }
  HX_DEV static void rec_sums(const int (&s)[4], int* xs) { xs[0] = (s[0] + s[1]) + (s[2] + s[3]); }
  // isum = sum(q x) over the block, exact; then (d_w isum) d_x
  HX_DEV static float dot(const Raw& r, const uint32_t* xp, const int* xs, float dx) {
    const uint32_t q[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
    int acc = 0;
#pragma unroll
    for (int j = 0; j < 8; j++) acc = dot4(q[j], xp[j], acc);
    return (f16_to_f32((uint16_t)r.d) * (float)acc) * dx;
  }
};

// Q4_K (GGUF): chunk = 16 bytes of nibbles: low run (sub-block 2p) and high run (2p+1)
template <>
struct DChunk<HX_Q4_K> {
  static constexpr int NX = 8, NS = 2;
  using Raw = Chunk<HX_Q4_K>::Raw;
  HX_DEV static void load(const uint8_t* mat, int R, int K, int row, int c, Raw& r) {
    Chunk<HX_Q4_K>::load(mat, R, K, row, c, r);
  }
  // activation positions: the low run (slots 0, 1) and the high run (2, 3)
  HX_DEV static int x_group_off(int c, int g) {
    const int sb = c >> 3, cc = c & 7, p = cc >> 1, h = cc & 1;
    return sb * 256 + 64 * p + 16 * h + 8 * (g & 1) + 32 * (g >> 1);
  }
  HX_DEV static void rec_sums(const int (&s)[4], int* xs) {
    xs[0] = s[0] + s[1];
    xs[1] = s[2] + s[3];
  }
  // byte i of the chunk: low nibble = low-run element i, high nibble =
  // high-run element i. Scales and mins of the two runs without branches (the
  // lanes of a wave hold different sub-blocks). S = sc0 D0 + sc1 D1 and
  // M = m0 X0 + m1 X1 are exact integers (D the code dot products, X the code
  // sums of the two runs); the reference's superblock step is
  // (d d_x) sum S - (dmin d_x) sum M.
  HX_DEV static float dot(const Raw& r, const uint32_t* xp, const int* xs, float dx) {
    const uint32_t q[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
    int lo = 0, hi = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      lo = dot4(q[j] & 0x0F0F0F0Fu, xp[j], lo);
      hi = dot4((q[j] >> 4) & 0x0F0F0F0Fu, xp[4 + j], hi);
    }
    const float d = f16_to_f32((uint16_t)(r.hdr.x & 0xffffu)), dmin = f16_to_f32((uint16_t)(r.hdr.x >> 16));
    // sub-blocks 2p, 2p + 1: bytes (2p) & 3, +1 of the 6-bit fields (p < 2), or
    // of the split fields (p >= 2)
    const int p = r.cc >> 1;
    const uint32_t sh = 16u * (uint32_t)(p & 1);
    const uint32_t a0 = r.hdr.y >> sh, a1 = r.hdr.z >> sh, a2 = r.hdr.w >> sh;
    const uint32_t scp = p < 2 ? a0 & 0x3F3Fu : (a2 & 0x0F0Fu) | ((a0 >> 2) & 0x3030u);
    const uint32_t mp = p < 2 ? a1 & 0x3F3Fu : ((a2 >> 4) & 0x0F0Fu) | ((a1 >> 2) & 0x3030u);
    const int sc0 = (int)(scp & 0xffu), sc1 = (int)((scp >> 8) & 0xffu);
    const int m0 = (int)(mp & 0xffu), m1 = (int)((mp >> 8) & 0xffu);
    const int S = sc0 * lo + sc1 * hi;
    const int M = m0 * xs[0] + m1 * xs[1];
    return (d * dx) * (float)S - (dmin * dx) * (float)M;
  }
};

// Q6_K planar: chunk = quarters 0..3 of l = 8a .. 8a+7 in half n of a superblock
template <>
struct DChunk<HX_Q6_K> {
  static constexpr int NX = 8, NS = 4;
  using Raw = Chunk<HX_Q6_K>::Raw;
  HX_DEV static void load(const uint8_t* mat, int R, int K, int row, int c, Raw& r) {
    Chunk<HX_Q6_K>::load(mat, R, K, row, c, r);
  }
  // activation positions: quarter g of the chunk's half superblock
  HX_DEV static int x_group_off(int c, int g) {
    const int sb = c >> 3, cc = c & 7, n = cc >> 2, a = cc & 3;
    return sb * 256 + 128 * n + 8 * a + 32 * g;
  }
  HX_DEV static void rec_sums(const int (&s)[4], int* xs) {
#pragma unroll
    for (int q = 0; q < 4; q++) xs[q] = s[q];
  }
  // the unsigned 6-bit code of quarter q, four elements a byte: its low
  // nibble (ql of quarters 0 / 1: low nibble, 2 / 3: high nibble) and the two
  // qh bits of the quarter (bits 2q, 2q + 1) moved to bits 4, 5. Per quarter
  // the int32 sum of (code - 32) x = D - 32 X; S = sum of sc (D - 32 X) is
  // the reference's exact integer, and its step (d d_x) S.
  HX_DEV static float dot(const Raw& r, const uint32_t* xp, const int* xs, float dx) {
    const uint32_t l0[2] = {r.l0.x, r.l0.y}, l1[2] = {r.l1.x, r.l1.y}, hh[2] = {r.h.x, r.h.y};
    int acc[4] = {0, 0, 0, 0};
#pragma unroll
    for (int w = 0; w < 2; w++) {
      const uint32_t h = hh[w];
      const uint32_t q0 = (l0[w] & 0x0F0F0F0Fu) | ((h << 4) & 0x30303030u);
      const uint32_t q1 = (l1[w] & 0x0F0F0F0Fu) | ((h << 2) & 0x30303030u);
      const uint32_t q2 = ((l0[w] >> 4) & 0x0F0F0F0Fu) | (h & 0x30303030u);
      const uint32_t q3 = ((l1[w] >> 4) & 0x0F0F0F0Fu) | ((h >> 2) & 0x30303030u);
      acc[0] = dot4(q0, xp[0 + w], acc[0]);
      acc[1] = dot4(q1, xp[2 + w], acc[1]);
      acc[2] = dot4(q2, xp[4 + w], acc[2]);
      acc[3] = dot4(q3, xp[6 + w], acc[3]);
    }
    int S = 0;
#pragma unroll
    for (int q = 0; q < 4; q++) S += (int)(int8_t)((r.sc >> (8 * q)) & 0xffu) * (acc[q] - 32 * xs[q]);
    return (f16_to_f32((uint16_t)r.d) * dx) * (float)S;
  }
};

// one chunk record (HX_REC_VECS x 16 bytes, hx_quant.h) -> the dot's code
// words, sums and d
template <class D>
HX_DEV void unpack_record(const u32x4v (&v)[HX_REC_VECS], uint32_t* xp, int* xs, float& dx) {
#pragma unroll
  for (int g = 0; g < 2; g++) {
    xp[4 * g] = v[g][0]; xp[4 * g + 1] = v[g][1]; xp[4 * g + 2] = v[g][2]; xp[4 * g + 3] = v[g][3];
  }
  const uint32_t t[4] = {v[2][0], v[2][1], v[2][2], v[2][3]};
  int s[4];
  record_tail(t, s, dx);
  D::rec_sums(s, xs);
}
template <class P>
HX_DEV void load_record(P src, u32x4v (&v)[HX_REC_VECS]) {
#pragma unroll
  for (int g = 0; g < HX_REC_VECS; g++) v[g] = src[g];
}
// keeps every word of a loaded record live up to this point: a word the
// format does not read is otherwise free at once, and the compiler reused its
// register right after the load, which made the wave wait for that load (and
// for every load issued before it) on the spot
HX_DEV void hold_record(u32x4v (&v)[HX_REC_VECS]) {
#pragma unroll
  for (int g = 0; g < HX_REC_VECS; g++) asm volatile("" : "+v"(v[g]));
}

// the decode plan, pulled into LDS by the whole workgroup in one pass
// the plan's first per-row word, 4 + 4 max_slots, taken from the kernel
// arguments at the kernel's start, together with the others (left to itself
// the compiler read max_slots only where the plan's rows are addressed: one
// more scalar round trip ahead of the plan loads and the weight loads that
// wait for them)
HX_DEV int plan_rows_at(const ExpertArgs& a) {
  int v = 4 + 4 * a.max_slots;
  asm volatile("" : "+s"(v));
  return v;
}

HX_DEV void load_plan(const ExpertArgs& a, int32_t* splan) {
  const int np = plan_ints(a.max_slots, a.F, a.T);
  for (int i = threadIdx.x; i < np; i += blockDim.x) splan[i] = a.plan[i];
  __syncthreads();
}

// NR (gate, up) row pairs of one expert for a list of tokens: the tokens'
// chunk records come from a.xcv (written by the router kernel); h = silu(g) u
// is stored as f32 for the down kernels' quantisation. tok_of(j) is token j of
// the list (tok_of(0) known before any load); pre() issues whatever loads
// tok_of(j > 0) reads, after the weight loads and before token 0's record.
template <int FMT, int LPR, int NR, class TokF, class PreF>
HX_DEV void gate_up_rows_f(const ExpertArgs& a, const uint8_t* G, const uint8_t* U, int rows, int row0, int count,
                           TokF tok_of, PreF pre, const int* hrow) {
  using D = DChunk<FMT>;
  constexpr int RG = 64 / LPR;
  const int c = lane_id() % LPR, K = a.H;
  typename D::Raw rgt[NR], rup[NR];
#pragma unroll
  for (int g = 0; g < NR; g++) {   // rows past the end read the last row (dropped)
    const int row = min(row0 + g * RG, rows - 1);
    D::load(G, rows, K, row, c, rgt[g]);
    D::load(U, rows, K, row, c, rup[g]);
  }
  pre();
  // token j's record is loaded before token j - 1's dot products (token 0's
  // together with the weights), so each load overlaps work
  u32x4v xr[HX_REC_VECS];
  auto xload = [&](int t) __attribute__((always_inline)) {
    load_record((const u32x4v*)(a.xcv + ((int64_t)t * (K / 32) + c) * HX_XCV_WORDS), xr);
  };
  xload(tok_of(0));
  __builtin_amdgcn_sched_barrier(0);   // no weight arithmetic above these loads
  for (int j = 0; j < count; j++) {
    uint32_t xp[D::NX];
    int xs[D::NS];
    float dx;
    unpack_record<D>(xr, xp, xs, dx);
    if (j + 1 < count) xload(tok_of(j + 1));
#pragma unroll
    for (int g = 0; g < NR; g++) {
      const int row = row0 + g * RG;
      float pg = row < rows ? D::dot(rgt[g], xp, xs, dx) : 0.f;
      float pu = row < rows ? D::dot(rup[g], xp, xs, dx) : 0.f;
      pg = wave_sum<LPR>(pg);
      pu = wave_sum<LPR>(pu);
      if (c == 0 && row < rows) a.hbuf[(int64_t)hrow[j] * a.hstride + row] = siluf_(pg) * pu;
    }
  }
}
template <int FMT, int LPR, int NR>
HX_DEV void gate_up_rows(const ExpertArgs& a, const uint8_t* G, const uint8_t* U, int rows, int row0, int count,
                         const int* tok, const int* hrow) {
  gate_up_rows_f<FMT, LPR, NR>(a, G, U, rows, row0, count, [&](int j) { return tok[j]; }, [] {}, hrow);
}

// ----------------------------------------------------------------------------
// K1: router logits (blocks [0, nrb)) and the tokens' chunk records (blocks
// nrb.., one workgroup per token, wave w quantising elements 512 w .. 512 w +
// 511, whole Q8_0 / Q8_K blocks): the token row in the router's canonical
// layout -- with the decoder RMSNorm applied by the same code as in the
// router waves when it is fused, so the normalised row is the same bits --
// quantised to the vec_dot type of the expert weights (hx_quant.h). (One
// wave per token quantising the whole row was the kernel's last wave to
// finish.)
// ----------------------------------------------------------------------------
template <int FMT, int NG>
HX_DEV void x_records(const RouterArgs& r, const ExpertArgs& a, int t, int part) {
  const int lane = lane_id(), H = r.H;
  uint32_t xr[1][NG][4];
#pragma unroll
  for (int i = 0; i < NG; i++) {
    const uint4 v = *(const uint4*)((const uint16_t*)r.x + (int64_t)t * H + 8 * (lane + 64 * i));
    xr[0][i][0] = v.x; xr[0][i][1] = v.y; xr[0][i][2] = v.z; xr[0][i][3] = v.w;
  }
  if (r.norm_w) rmsnorm_regs<1, NG>(r, xr, t);
  uint32_t* rec = a.xcv + (int64_t)t * (H / 32) * HX_XCV_WORDS;
#pragma unroll
  for (int i = 0; i < NG; i++) {
    if (i != part) continue;   // wave-uniform: this wave's 512 elements (whole Q8_0 / Q8_K blocks)
    float x[8];
#pragma unroll
    for (int q = 0; q < 4; q++) {
      x[2 * q] = __uint_as_float(xr[0][i][q] << 16);
      x[2 * q + 1] = __uint_as_float(xr[0][i][q] & 0xffff0000u);
    }
    group_to_record<FMT>(x, lane + 64 * i, rec);
  }
}

template <int FMT, bool RBF, int TT>
__global__ __launch_bounds__(256) void k_router_dec(RouterArgs r, ExpertArgs a, int nrb) {
  const int wave = threadIdx.x >> 6;
  const int ng = (a.T + TT - 1) / TT;   // token groups of TT
  if ((int)blockIdx.x < nrb * ng) {
    // router rows of workgroup rb (one a wave) for token group g
    const int rb = (int)blockIdx.x % nrb, g = (int)blockIdx.x / nrb;
    if (TT > 1 && r.norm_w && (r.H & 7) == 0 && r.H <= 8 * 256)   // at most 4 groups of 8 a lane
      router_rows_norm<RBF, TT, 1, 4>(r, rb * 4 + wave, g * TT, rb == 0);
    else
      router_rows<true, RBF, TT, 1>(r, rb * 4 + wave, g * TT);
    return;
  }
  // one workgroup per token: wave w quantises the token's elements 512 w ..
  // 512 w + 511 (each wave holds the whole row for the RMSNorm's sum)
  const int t = (int)blockIdx.x - nrb * ng;
  if (t >= a.T || wave >= (a.H >> 9)) return;
  switch (a.H >> 9) {   // groups of 8 per lane: H / 512 (H = 512, 1024, 2048)
    case 1: x_records<FMT, 1>(r, a, t, wave); break;
    case 2: x_records<FMT, 2>(r, a, t, wave); break;
    default: x_records<FMT, 4>(r, a, t, wave); break;
  }
}

// ----------------------------------------------------------------------------
// K2 (T == 1): routed gate/up + SwiGLU. Every workgroup routes the token from
// the logits in LDS (wave 0) while its other waves compute shared-expert rows.
// The last grid row's workgroup 0 only publishes the plan (and the routing
// unless the forward asks for the plan only); workgroup
// (x, u < last row) computes rows of slot u's expert. (Pulling the expert's
// down projection into the caches here as well was measured to cost more in
// this kernel than it saved in the next.)
// ----------------------------------------------------------------------------
template <int FMT, int LPR, int NR>
__global__ __launch_bounds__(256) void k_gate_up_dec(RouterArgs r, ExpertArgs a) {
  constexpr int RG = 64 / LPR;
  __shared__ RouteSmem sm;
  const bool publisher = blockIdx.y == gridDim.y - 1;
  const int wave = threadIdx.x >> 6;
  if (wave > 0 && a.Is > 0) {
    // waves 1..3 compute the shared expert's gate/up rows (RG * NR per wave, in
    // linear workgroup order) while wave 0 routes
    const int task = (blockIdx.y * gridDim.x + blockIdx.x) * 3 + wave - 1;
    const int r0 = task * (RG * NR);
    if (r0 < a.Is) {
      int tok[HX_DECODE_MAX_T], hrow[HX_DECODE_MAX_T];
      for (int j = 0; j < a.T; j++) {
        tok[j] = j;
        hrow[j] = a.F + j;
      }
      gate_up_rows<FMT, LPR, NR>(a, a.sgate.base, a.sup.base, a.Is, r0 + lane_id() / LPR, a.T, tok, hrow);
    }
  }
  if (publisher && blockIdx.x > 0) return;
  route_small_lds(r.logits, r.E1, r.E, r.k, r.norm, publisher && r.has_shared, r.T, sm, 256);
  if (publisher) {
    publish_route(r.d, r.topk_w, r.sgw, sm);
    return;
  }
  const int u = blockIdx.y;
  if (u >= sm.nroute) return;
  const int e = sm.slots[3 * u], start = sm.slots[3 * u + 1], count = sm.slots[3 * u + 2];
  int tok[HX_DECODE_MAX_T], hrow[HX_DECODE_MAX_T];
  for (int j = 0; j < count; j++) {
    hrow[j] = start + j;
    tok[j] = sm.perm[start + j] / a.k;
  }
  const int row0 = (blockIdx.x * 4 + wave) * (RG * NR) + lane_id() / LPR;
  if (row0 - lane_id() / LPR < a.I)
    gate_up_rows<FMT, LPR, NR>(a, a.gate.mat(e), a.up.mat(e), a.I, row0, count, tok, hrow);
}

// ----------------------------------------------------------------------------
// The routing and decode plan of one token, written by the wave that routed it
// straight from its registers (lane j < k: rank j's expert e, weight w and
// dispatch position pos): the words publish_route writes from RouteSmem for
// T = 1. The k experts are distinct, so each is a slot of one row at its
// dispatch position, and offsets[x] is the number of them below x.
// ----------------------------------------------------------------------------
HX_DEV void publish_one_token(const DispatchArgs& d, float* topk_w, float* sgw, int e, float w, int pos, float sg) {
  const int lane = lane_id(), k = d.k, E = d.E;
  const bool all = !d.plan_only;
  const int tok0 = 4 + 4 * d.max_slots, w0 = tok0 + k + 1, e0 = w0 + k + 1;   // F = k, T = 1
  if (lane < k) {
    if (all) {
      d.topk_idx[lane] = e;
      topk_w[lane] = w;
      d.perm[pos] = lane;
      if (d.inv) d.inv[lane] = pos;
      d.slots[3 * pos + 0] = e;
      d.slots[3 * pos + 1] = pos;
      d.slots[3 * pos + 2] = 1;
    }
    d.plan[tok0 + pos] = 0;
    d.plan[w0 + pos] = __float_as_int(w);
    d.plan[e0 + pos] = e;
    *(int4*)(d.plan + 4 + 4 * pos) = make_int4(e, pos, 1, 0);
  }
  if (lane == 0) {
    if (all) sgw[0] = sg;
    d.plan[tok0 + k] = 0;
    d.plan[w0 + k] = __float_as_int(sg);
    d.plan[e0 + k] = E;
    if (d.has_shared) {
      if (all) {
        d.slots[3 * k + 0] = E;
        d.slots[3 * k + 1] = k;
        d.slots[3 * k + 2] = 1;
      }
      *(int4*)(d.plan + 4 + 4 * k) = make_int4(E, k, 1, 0);
    }
    const int ns = k + (d.has_shared ? 1 : 0);
    if (all) {
      d.counts[0] = ns;
      d.counts[1] = 0;
    }
    d.plan[0] = ns;
  }
  if (all) {
    for (int x = lane; x <= E; x += 64) {
      int c = 0;
      for (int j = 0; j < k; j++) c += __builtin_amdgcn_readlane(e, j) < x;
      d.offsets[x] = c;
    }
  }
}

// ----------------------------------------------------------------------------
// K2 for one token with H = 64 chunks of 32 and k = KR: a wave owns one row
// of the gate or of the up projection (waves 2i and 2i + 1: row 2b + i of
// workgroup b) for the KR routed experts and the shared expert. Every wave
// routes the token itself (same arithmetic as route_token_core, so all waves
// agree; no barrier) and issues the loads of its row of the rank-r expert right
// after round r, so the weight stream overlaps the rest of the selection; the
// shared expert's row and the token's chunk record are loaded before routing
// starts. The KR + 1 dot products of a wave are summed by one reduce-scatter,
// and wave 2i combines them with wave 2i + 1's into h = silu(gate) * up,
// stored (f32) at the row of h of the expert's dispatch position. Wave 0 of
// workgroup 0 also publishes the plan (and, unless the forward asks for the
// plan only, the routing) from its registers as soon as the selection ends
// (measured on MI355X: 0.4 us shorter than a whole-workgroup publication
// after the dot products).
// ----------------------------------------------------------------------------
template <int FMT, int EPL, int KR>
__global__ __launch_bounds__(256) void k_gate_up_dec1(RouterArgs r, ExpertArgs a) {
  using D = DChunk<FMT>;
  static_assert(KR < 16, "the rank-r sums and the shared one fit 16 values");
  __shared__ float sums[4][16];
  const int wave = threadIdx.x >> 6, lane = lane_id();
  const int mat = wave & 1;                       // 0: gate, 1: up
  const int row = blockIdx.x * 2 + (wave >> 1);   // row of I (and of the shared expert's Is)
  const int K = a.H;
  // the logits first: a wait for them then leaves the later loads in flight
  float lv[EPL];
  route_logits_load<EPL>(r.logits, r.E, lv);
  // the shared gate's logit: a vector load (its index held in a VGPR) issued
  // with the logits and counted with them, not a scalar load that the next
  // wait for kernel arguments would wait for too; used only at publication
  int sgi = r.has_shared ? r.E : 0;
  asm volatile("" : "+v"(sgi));
  const float sg = r.logits[sgi];
  u32x4v xr[HX_REC_VECS];
  load_record((const u32x4v*)(a.xcv + (int64_t)lane * HX_XCV_WORDS), xr);
  const bool shrow = a.Is > 0 && row < a.Is, rrow = row < a.I;
  // loads are unconditional (out-of-range rows read row 0 and are dropped at
  // the end), and a scheduling barrier after each round's loads keeps the
  // compiler from pulling the dot products' first instructions up to them,
  // which would wait for every load on the spot
  typename D::Raw rsh;
  const bool hs = a.Is > 0;   // without a shared expert, read routed matrix 0
  D::load(hs ? (mat ? a.sup.base : a.sgate.base) : (mat ? a.up.mat(0) : a.gate.mat(0)),
          hs ? a.Is : a.I, K, shrow ? row : 0, lane, rsh);
  __builtin_amdgcn_sched_barrier(0);
  typename D::Raw raw[KR];
  int my_e;
  float my_w;
  // rounds -1 .. -SPEC: the experts of the SPEC largest logits (lowest id
  // first), almost always ranks 0 .. SPEC - 1: their rows are loaded before the
  // softmax and sort, and reloaded only if the round of that rank selects
  // another expert (measured on MI355X: SPEC = 1 is fastest; each further
  // guess delays the softmax by one more pair of wave reductions)
  constexpr int SPEC = 1;
  int es[SPEC];
  route_token_core_hook<EPL, KR, SPEC>(lv, r.E, r.norm, my_e, my_w, [&](int j, int e) {
    if (j < 0) {
      const int sp = -1 - j;
      es[sp] = e;
      D::load(mat ? a.up.mat(e >= 0 ? e : 0) : a.gate.mat(e >= 0 ? e : 0), a.I, K, rrow ? row : 0, lane, raw[sp]);
    } else if (j >= SPEC || e != es[j]) {
      D::load(mat ? a.up.mat(e) : a.gate.mat(e), a.I, K, rrow ? row : 0, lane, raw[j]);
    }
    __builtin_amdgcn_sched_barrier(0);
  });
  // dispatch position of rank `lane`: the k experts are distinct
  int pos = 0;
#pragma unroll
  for (int j = 0; j < KR; j++) pos += __builtin_amdgcn_readlane(my_e, j) < my_e;
  if (blockIdx.x == 0 && wave == 0)
    publish_one_token(r.d, r.topk_w, r.sgw, my_e, my_w, pos, r.has_shared ? sigmoidf_(sg_late(sg)) : 0.0f);
  uint32_t xp[D::NX];
  int xs[D::NS];
  float dx;
  hold_record(xr);
  unpack_record<D>(xr, xp, xs, dx);
  float v[16];
#pragma unroll
  for (int j = 0; j < KR; j++) v[j] = D::dot(raw[j], xp, xs, dx);
  const float vs = D::dot(rsh, xp, xs, dx);
  v[KR] = hs ? vs : 0.f;
#pragma unroll
  for (int j = KR + 1; j < 16; j++) v[j] = 0.f;
  rs_vals64<16>(v);   // lane l: value l / 4
  if ((lane & 3) == 0) sums[wave][lane >> 2] = v[0];
  __syncthreads();
  if (mat == 0 && lane <= KR) {
    const float g = sums[wave][lane], u = sums[wave + 1][lane];
    const float h = siluf_(g) * u;
    if (lane < KR && rrow) a.hbuf[(int64_t)pos * a.hstride + row] = h;
    if (lane == KR && shrow) a.hbuf[(int64_t)a.F * a.hstride + row] = h;
  }
}

// ----------------------------------------------------------------------------
// K2 for T > 1: the routing and plan were published by one workgroup
// (k_route_small); grid row y computes rows of one slot's expert from the
// plan: row 0 the shared expert's slot (the plan's last; its T tokens make
// its workgroups the longest, so they are dispatched first), rows 1.. the
// routed slots.
// ----------------------------------------------------------------------------
template <int FMT, int LPR, int NR>
__global__ __launch_bounds__(256) void k_gate_up_plan(ExpertArgs a) {
  constexpr int RG = 64 / LPR;
  // the shared expert's slot needs no plan: expert E, rows F .. F + T - 1 of
  // h, row F + t for token t; a routed slot's record is read together with
  // the slot count (one round trip before the weight loads, not two)
  const bool sh = a.Is > 0 && blockIdx.y == 0;
  int4 sr = make_int4(a.E, a.F, a.T, 0);   // expert, first row, rows, first row's token
  if (!sh) {
    const int u = (int)blockIdx.y - (a.Is > 0 ? 1 : 0);   // < max_slots - 1: a record of the plan
    const int nslots = a.plan[0];
    sr = *(const int4*)(a.plan + 4 + 4 * u);
    if (u >= nslots - (a.Is > 0 ? 1 : 0)) return;
  }
  const int e = sr.x, start = sr.y, count = sr.z;
  const int tok0 = 4 + 4 * a.max_slots;
  int hrow[HX_DECODE_MAX_T];
  for (int j = 0; j < count; j++) hrow[j] = start + j;
  const int rows = sh ? a.Is : a.I;
  const int wave = threadIdx.x >> 6;
  const int row0 = (blockIdx.x * 4 + wave) * (RG * NR) + lane_id() / LPR;
  // a routed slot's tokens after the first: one vector load (lane j holds
  // token j), issued behind the weight loads, so neither waits for the other
  // (a loop of dependent scalar loads here delayed the weight stream by a
  // round trip per token)
  int tl = 0;
  auto tok_of = [&](int j) __attribute__((always_inline)) {
    return sh ? j : j == 0 ? sr.w : __builtin_amdgcn_readlane(tl, j);
  };
  auto pre = [&]() __attribute__((always_inline)) {
    if (!sh && count > 1) tl = a.plan[tok0 + start + min(lane_id(), count - 1)];
  };
  if (row0 - lane_id() / LPR < rows)
    gate_up_rows_f<FMT, LPR, NR>(a, sh ? a.sgate.base : a.gate.mat(e), sh ? a.sup.base : a.up.mat(e), rows, row0, count,
                                 tok_of, pre, hrow);
}

// ----------------------------------------------------------------------------
// Rows of h (f32) -> chunk records for the down projection: one wave per row,
// the row in the canonical layout (group g of 8 in lane g % 64, register
// g / 64), quantised to the vec_dot type of the down weights.
// ----------------------------------------------------------------------------
template <int NG>
HX_DEV void h_row_load(const float* hrow, float (&x)[NG][8]) {
  const int lane = lane_id();
#pragma unroll
  for (int i = 0; i < NG; i++) {
    const float4 p = *(const float4*)(hrow + 8 * (lane + 64 * i)), q = *(const float4*)(hrow + 8 * (lane + 64 * i) + 4);
    x[i][0] = p.x; x[i][1] = p.y; x[i][2] = p.z; x[i][3] = p.w;
    x[i][4] = q.x; x[i][5] = q.y; x[i][6] = q.z; x[i][7] = q.w;
  }
}
template <int FMT, int NG>
HX_DEV void h_regs_records(const float (&x)[NG][8], uint32_t* rec) {
#pragma unroll
  for (int i = 0; i < NG; i++) group_to_record<FMT>(x[i], lane_id() + 64 * i, rec);
}
template <int FMT, int NG>
HX_DEV void h_row_records(const float* hrow, uint32_t* rec) {
  float x[NG][8];
  h_row_load<NG>(hrow, x);
  h_regs_records<FMT, NG>(x, rec);
}

// the rows of h of a forward (routed, then the shared expert's) into a.hrec
template <int FMT, int NG>
__global__ __launch_bounds__(256) void k_hrec(ExpertArgs a, int nrows) {
  // the kernel arguments all read in one round trip before the bound check
  // (which otherwise split them in two, ahead of the row's loads); the asm
  // only uses them (one that rewrote the pointers would hide their address
  // space and turn the row's loads and stores into flat ones)
  const float* hb = a.hbuf;
  uint32_t* hr = a.hrec;
  const int hs = a.hstride;
  asm volatile("" ::"s"(hb), "s"(hr), "s"(hs));
  const int row = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6);
  if (row >= nrows) return;
  h_row_records<FMT, NG>(hb + (int64_t)row * hs, hr + (int64_t)row * (16 * NG) * HX_XCV_WORDS);
}

// the residual element a down kernel loaded at its start, as f32 in its
// epilogue: the empty asm keeps the conversion (and so the wait for the load)
// from being hoisted up to the load
HX_DEV float resid_f32(uint16_t rx) {
  uint32_t v = rx;
  asm volatile("" : "+v"(v));
  return __uint_as_float(v << 16);
}

// ----------------------------------------------------------------------------
// down + combine: block = RG output rows; the NW waves take the group's rows
// of h SPW at a time (groups of ROWS = NW SPW rows, grid.y of them); each row's
// contribution w * (row . h) goes to LDS, and each token's output is the sum
// of its rows in row order (slots by ascending expert, then the shared
// expert), as the reference's combine order; with several groups, the group's
// partial sum, which k_down_reduce adds up in group order. The chunk records
// of the rows of h come from k_hrec; each wave loads those of a row right
// before its dot product.
// ----------------------------------------------------------------------------
template <int FMT, int LPR, int SPW, int NW>
__global__ __launch_bounds__(64 * NW) void k_down_dec(ExpertArgs a) {
  using D = DChunk<FMT>;
  constexpr int RG = 64 / LPR;
  constexpr int ROWS = NW * SPW;   // rows of h per group (one pass per wave)
  static_assert(ROWS <= HX_DOWN_ROWS, "groups of at most HX_DOWN_ROWS rows of h");
  // LDS: per row of h its token, weight and expert; then the contributions
  // [ROWS][RG]
  extern __shared__ __attribute__((aligned(16))) uint16_t xl[];
  int* stok = (int*)xl;
  float* swt = (float*)(stok + ROWS);
  int* sexp = (int*)(swt + ROWS);
  float* contrib = (float*)(sexp + ROWS);
  const int T = a.T, NH = a.F + T;
  const int nh_all = a.F + (a.Is > 0 ? T : 0);   // rows of h in use
  const int h0 = blockIdx.y * ROWS;              // this workgroup's group of rows
  const int nh = min(nh_all - h0, ROWS);
  {
    // thread 32 part + r < 96 loads row r's token (part 0), weight (1) or
    // expert (2); one load each, clamped to a valid row, so one round trip.
    // Rows r in [nh, ROWS) get token -1 (no token's row).
    static_assert(ROWS <= 32, "a part of the plan per 32 threads");
    const int tok0 = 4 + 4 * a.max_slots + h0;
    const int i = threadIdx.x, part = i >> 5, r = i & 31;
    if (i < 96) {
      const int v = a.plan[tok0 + part * NH + min(r, nh - 1)];
      int* dst = part == 0 ? stok : part == 1 ? (int*)swt : sexp;
      if (r < nh) dst[r] = v;
      else if (part == 0 && r < ROWS) dst[r] = -1;
    }
  }
  __syncthreads();
  const int lane = lane_id(), wave = threadIdx.x >> 6, rg = lane / LPR, c = lane % LPR;
  const int n0 = blockIdx.x * RG, row = n0 + rg;
  // every weight load of the wave first, all unconditional (rows past the
  // group's end, and chunks past a shorter shared expert's K, read valid data
  // that is dropped)
  typename D::Raw raw[SPW];
#pragma unroll
  for (int s = 0; s < SPW; s++) {
    const int hr = wave + NW * s;
    const int hq = hr < nh ? hr : 0;
    const int e = sexp[hq];
    const bool sh = e == a.E;
    const int K = sh ? a.Is : a.I;
    const int cc = c < K / 32 ? c : 0;
    D::load(sh ? a.sdown.base : a.down.mat(e), a.H, K, row < a.H ? row : 0, cc, raw[s]);
  }
#pragma unroll
  for (int s = 0; s < SPW; s++) {
    const int hr = wave + NW * s;
    if (hr >= nh) {   // every contribution slot is defined (zero past the group's rows)
      if (c == 0 && row < a.H) contrib[hr * RG + rg] = 0.f;
      continue;
    }
    const int K = sexp[hr] == a.E ? a.Is : a.I;
    float p = 0.f;
    if (c < K / 32) {
      u32x4v v[HX_REC_VECS];
      load_record((const u32x4v*)(a.hrec + ((int64_t)(h0 + hr) * LPR + c) * HX_XCV_WORDS), v);
      uint32_t xp[D::NX];
      int xs[D::NS];
    float dx;
      unpack_record<D>(v, xp, xs, dx);
      p = D::dot(raw[s], xp, xs, dx);
    }
    p = wave_sum<LPR>(p);
    if (c == 0 && row < a.H) contrib[hr * RG + rg] = swt[hr] * p;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < T * RG; i += 64 * NW) {
    const int t = i / RG, r = i % RG;
    if (n0 + r >= a.H) continue;
    float y = 0.f;
    // unrolled, and the row selection a multiplication by 1 or 0 (exact), so
    // the LDS reads are unconditional and go out together
#pragma unroll
    for (int hr = 0; hr < ROWS; hr++) y += contrib[hr * RG + r] * (stok[hr] == t ? 1.f : 0.f);
    if (gridDim.y > 1) {
      a.dpart[((int64_t)blockIdx.y * T + t) * a.H + n0 + r] = y;
    } else if (a.resid) {
      uint16_t* px = a.resid + (int64_t)t * a.H + n0 + r;
      *px = f32_to_bf16(bf16_to_f32(*px) + bf16_to_f32(f32_to_bf16(y)));
    } else {
      ((uint16_t*)a.y)[(int64_t)t * a.H + n0 + r] = f32_to_bf16(y);
    }
  }
}

// ----------------------------------------------------------------------------
// down + combine for one token with at most 12 rows of h (k <= 11): OG groups
// of four waves per workgroup, group o owning output rows RG o .. + RG - 1 of
// the workgroup's RG OG; wave q of a group takes rows of h q, q + 4, q + 8.
// The workgroup quantises each row of h once into chunk records in LDS (wave
// w rows w, w + 4 OG), whose loads it issues first of all (they need no plan)
// so the quantisation can start once they have arrived while the weight loads
// issued after them are still in flight; more output rows per workgroup read
// and quantise the rows of h fewer times over the grid. Each output is the sum
// of its rows' contributions in row order (slots by ascending expert, then the
// shared expert), as the reference's combine order.
// ----------------------------------------------------------------------------
template <int FMT, int LPR, int OG, int WPG>
__global__ __launch_bounds__(64 * WPG * OG) void k_down_one(ExpertArgs a) {
  using D = DChunk<FMT>;
  constexpr int RG = 64 / LPR, NG = LPR / 16;   // K = 32 LPR: groups of 8 per lane of a row
  constexpr int NW = WPG * OG, ROWS = 12, SPW = ROWS / WPG, QS = (ROWS + NW - 1) / NW;
  static_assert(ROWS % WPG == 0, "each wave of a group takes ROWS / WPG rows of h");
  constexpr int NO = RG * OG;   // output rows of the workgroup
  // LDS: chunk records [ROWS][LPR]; per row its token, weight and expert; the
  // contributions [ROWS][NO]
  extern __shared__ __attribute__((aligned(16))) uint16_t xl[];
  uint32_t* srec = (uint32_t*)xl;
  int* stok = (int*)(srec + ROWS * LPR * HX_XCV_WORDS);
  float* swt = (float*)(stok + ROWS);
  int* sexp = (int*)(swt + ROWS);
  float* contrib = (float*)(sexp + ROWS);
  const int tok0 = plan_rows_at(a);
  const int NH = a.F + 1;
  const int nh = a.F + (a.Is > 0 ? 1 : 0);   // rows of h in use (<= ROWS)
  const int w = threadIdx.x >> 6;
  // the residual this thread adds in the epilogue, loaded first (the
  // epilogue then waits on no memory round trip)
  // (every thread loads an in-bounds element, so no lane-dependent branch
  // makes the wave wait for the load where it is issued; only the epilogue's
  // threads use theirs)
  const int n_out = blockIdx.x * NO + (int)threadIdx.x;
  const uint16_t rx = a.resid ? a.resid[min(n_out, a.H - 1)] : 0;
  // the plan's words first (thread 32 part + r < 96 stores row r's token
  // (part 0), weight (1) or expert (2); every thread loads an in-bounds word,
  // so no branch surrounds the load): loads complete in order, so the wait
  // for the plan, which the weight loads need, leaves the rows of h in flight
  const int pi = threadIdx.x, part = min(pi >> 5, 2), pr = pi & 31;
  const int pv = a.plan[tok0 + part * NH + min(pr, nh - 1)];
  __builtin_amdgcn_sched_barrier(0);
  float hx[QS][NG][8];
#pragma unroll
  for (int s = 0; s < QS; s++)   // rows past the end read row 0 (not quantised)
    h_row_load<NG>(a.hbuf + (int64_t)(w + NW * s < nh ? w + NW * s : 0) * a.hstride, hx[s]);
  __builtin_amdgcn_sched_barrier(0);
  if (pi < 96) {   // rows r in [nh, ROWS) get token -1 (no token's row)
    int* dst = part == 0 ? stok : part == 1 ? (int*)swt : sexp;
    if (pr < nh) dst[pr] = pv;
    else if (part == 0 && pr < ROWS) dst[pr] = -1;
  }
  lds_barrier();   // LDS only: the rows of h stay in flight
  const int lane = lane_id(), og = w / WPG, wq = w % WPG, rg = lane / LPR, c = lane % LPR;
  const int row = (blockIdx.x * OG + og) * RG + rg;
  // every weight load of the wave, unconditional (rows past the end, and
  // chunks past a shorter shared expert's K, read valid data that is dropped)
  typename D::Raw raw[SPW];
#pragma unroll
  for (int s = 0; s < SPW; s++) {
    const int hr = wq + WPG * s, hq = hr < nh ? hr : 0;
    const int e = sexp[hq];
    const bool sh = e == a.E;
    const int K = sh ? a.Is : a.I;
    D::load(sh ? a.sdown.base : a.down.mat(e), a.H, K, row < a.H ? row : 0, c < K / 32 ? c : 0, raw[s]);
  }
  __builtin_amdgcn_sched_barrier(0);   // the weight loads go out before the quantisation
#pragma unroll
  for (int s = 0; s < QS; s++)
    if (w + NW * s < nh) h_regs_records<FMT, NG>(hx[s], srec + (w + NW * s) * LPR * HX_XCV_WORDS);
  lds_barrier();   // LDS only: the weight loads stay in flight for the dot products
#pragma unroll
  for (int s = 0; s < SPW; s++) {
    const int hr = wq + WPG * s;
    if (hr >= nh) {   // every contribution slot is defined (zero past the rows of h)
      if (c == 0) contrib[hr * NO + og * RG + rg] = 0.f;
      continue;
    }
    const int K = sexp[hr] == a.E ? a.Is : a.I;
    float p = 0.f;
    if (c < K / 32) {
      u32x4v v[HX_REC_VECS];
      load_record((const lds_v4*)(srec + (hr * LPR + c) * HX_XCV_WORDS), v);
      uint32_t xp[D::NX];
      int xs[D::NS];
      float dx;
      unpack_record<D>(v, xp, xs, dx);
      p = D::dot(raw[s], xp, xs, dx);
    }
    p = wave_sum<LPR>(p);
    if (c == 0) contrib[hr * NO + og * RG + rg] = swt[hr] * p;
  }
  __syncthreads();
  const int i = threadIdx.x;
  const int n = blockIdx.x * NO + i;
  if (i < NO && n < a.H) {
    float y = 0.f;
#pragma unroll
    for (int hr = 0; hr < ROWS; hr++) y += contrib[hr * NO + i] * (stok[hr] == 0 ? 1.f : 0.f);
    if (a.resid) {
      a.resid[n] = f32_to_bf16(resid_f32(rx) + bf16_to_f32(f32_to_bf16(y)));
    } else {
      ((uint16_t*)a.y)[n] = f32_to_bf16(y);
    }
  }
}

// ----------------------------------------------------------------------------
// Q6_K down rows read two chunks a lane: chunks 2 p and 2 p + 1 of a row (the
// same superblock half, l-blocks a and a + 1 with a even) share their scale
// bytes and d, and their ql / qh pieces are adjacent, 16-byte aligned: one
// lane loads both in five loads (ql 2 x 16 B, qh 16 B, the half's 8 scale
// bytes, d) instead of ten.
// ----------------------------------------------------------------------------
struct Q6Pair {
  uint4 l0, l1, h;
  uint32_t sc, d;
  HX_DEV static void load(const uint8_t* mat, int R, int K, int row, int p, Q6Pair& r) {
    const int c = 2 * p, sb = c >> 3, cc = c & 7, n = cc >> 2, a = cc & 3;   // a even
    const int o = sb * 128 + 64 * n + 8 * a;
    const uint2 sc8 = *(const uint2*)q6k_sc(mat, R, K, row, sb * 16 + 8 * n);
    r.l0 = *(const uint4*)q6k_ql(mat, R, K, row, o);
    r.l1 = *(const uint4*)q6k_ql(mat, R, K, row, o + 32);
    r.h = *(const uint4*)q6k_qh(mat, R, K, row, sb * 64 + 32 * n + 8 * a);
    r.sc = __builtin_amdgcn_perm(sc8.y, sc8.x, 0x06040200u + 0x01010101u * (uint32_t)(a >> 1));
    r.d = *((const uint16_t*)(mat + (int64_t)R * (K / 2 + K / 4 + K / 16)) + (int64_t)row * (K / 256) + sb);
  }
  // the two chunks as the one-chunk form DChunk<HX_Q6_K> takes
  HX_DEV void split(Chunk<HX_Q6_K>::Raw& c0, Chunk<HX_Q6_K>::Raw& c1) const {
    c0.l0 = make_uint2(l0.x, l0.y); c0.l1 = make_uint2(l1.x, l1.y); c0.h = make_uint2(h.x, h.y);
    c1.l0 = make_uint2(l0.z, l0.w); c1.l1 = make_uint2(l1.z, l1.w); c1.h = make_uint2(h.z, h.w);
    c0.sc = c1.sc = sc;
    c0.d = c1.d = d;
  }
};

// k_down_one for Q6_K down weights with K = 512, two chunks a lane (Q6Pair):
// 8 lanes a row, the workgroup's 8 output rows in every wave, NW waves a
// workgroup, wave w taking rows of h w, w + NW, .. (12 / NW of them) and
// quantising the same rows; otherwise as k_down_one (each row of h quantised
// once a workgroup into records in LDS; row-order sums per token, the lane's
// two chunks added first)
template <int NW>
__global__ __launch_bounds__(64 * NW) void k_down_one_q6p(ExpertArgs a) {
  using D = DChunk<HX_Q6_K>;
  constexpr int LPR = 8, RG = 8, NG = 1, ROWS = 12, SPW = ROWS / NW, QS = SPW, NC = 16;
  extern __shared__ __attribute__((aligned(16))) uint16_t xl[];
  uint32_t* srec = (uint32_t*)xl;
  int* stok = (int*)(srec + ROWS * NC * HX_XCV_WORDS);
  float* swt = (float*)(stok + ROWS);
  int* sexp = (int*)(swt + ROWS);
  float* contrib = (float*)(sexp + ROWS);
  const int tok0 = plan_rows_at(a);
  const int NH = a.F + 1;
  const int nh = a.F + (a.Is > 0 ? 1 : 0);
  const int w = threadIdx.x >> 6;
  // the epilogue's residual, loaded first (an in-bounds element for every
  // thread: no lane-dependent branch around the load)
  const int n_out = blockIdx.x * RG + (int)threadIdx.x;
  const uint16_t rx = a.resid ? a.resid[min(n_out, a.H - 1)] : 0;
  // the plan's words first (thread 32 part + r < 96 stores row r's token
  // (part 0), weight (1) or expert (2); every thread loads an in-bounds word,
  // so no branch surrounds the load): loads complete in order, so the wait
  // for the plan, which the weight loads need, leaves the rows of h in flight
  const int pi = threadIdx.x, part = min(pi >> 5, 2), pr = pi & 31;
  const int pv = a.plan[tok0 + part * NH + min(pr, nh - 1)];
  __builtin_amdgcn_sched_barrier(0);
  float hx[QS][NG][8];
#pragma unroll
  for (int s = 0; s < QS; s++)
    h_row_load<NG>(a.hbuf + (int64_t)(w + NW * s < nh ? w + NW * s : 0) * a.hstride, hx[s]);
  __builtin_amdgcn_sched_barrier(0);
  if (pi < 96) {   // rows r in [nh, ROWS) get token -1 (no token's row)
    int* dst = part == 0 ? stok : part == 1 ? (int*)swt : sexp;
    if (pr < nh) dst[pr] = pv;
    else if (part == 0 && pr < ROWS) dst[pr] = -1;
  }
  lds_barrier();   // LDS only: the rows of h stay in flight
  const int lane = lane_id(), rg = lane / LPR, pc = lane % LPR;
  const int row = blockIdx.x * RG + rg;
  Q6Pair raw[SPW];
#pragma unroll
  for (int s = 0; s < SPW; s++) {
    const int hr = w + NW * s, hq = hr < nh ? hr : 0;
    const int e = sexp[hq];
    const bool sh = e == a.E;
    const int K = sh ? a.Is : a.I;
    Q6Pair::load(sh ? a.sdown.base : a.down.mat(e), a.H, K, row < a.H ? row : 0, 2 * pc < K / 32 ? pc : 0, raw[s]);
  }
  __builtin_amdgcn_sched_barrier(0);   // the weight loads go out before the quantisation
#pragma unroll
  for (int s = 0; s < QS; s++)
    if (w + NW * s < nh) h_regs_records<HX_Q6_K, NG>(hx[s], srec + (w + NW * s) * NC * HX_XCV_WORDS);
  lds_barrier();   // LDS only: the weight loads stay in flight for the dot products
#pragma unroll
  for (int s = 0; s < SPW; s++) {
    const int hr = w + NW * s;
    if (hr >= nh) {
      if (pc == 0) contrib[hr * RG + rg] = 0.f;
      continue;
    }
    const int K = sexp[hr] == a.E ? a.Is : a.I;
    float p = 0.f;
    if (2 * pc < K / 32) {
      Chunk<HX_Q6_K>::Raw c0, c1;
      raw[s].split(c0, c1);
#pragma unroll
      for (int h = 0; h < 2; h++) {
        u32x4v v[HX_REC_VECS];
        load_record((const lds_v4*)(srec + (hr * NC + 2 * pc + h) * HX_XCV_WORDS), v);
        uint32_t xp[D::NX];
        int xs[D::NS];
        float dx;
        unpack_record<D>(v, xp, xs, dx);
        p += D::dot(h ? c1 : c0, xp, xs, dx);
      }
    }
    p = wave_sum<LPR>(p);
    if (pc == 0) contrib[hr * RG + rg] = swt[hr] * p;
  }
  __syncthreads();
  const int i = threadIdx.x;
  const int n = blockIdx.x * RG + i;
  if (i < RG && n < a.H) {
    float y = 0.f;
#pragma unroll
    for (int hr = 0; hr < ROWS; hr++) y += contrib[hr * RG + i] * (stok[hr] == 0 ? 1.f : 0.f);
    if (a.resid) {
      a.resid[n] = f32_to_bf16(resid_f32(rx) + bf16_to_f32(f32_to_bf16(y)));
    } else {
      ((uint16_t*)a.y)[n] = f32_to_bf16(y);
    }
  }
}

// ----------------------------------------------------------------------------
// The rows of h of each token as bit masks (row hr of token t: bit hr % 64 of
// word hr / 64 of m[t]), built by ballots, wave w taking tokens w, w + waves;
// and a token's sum of its rows' contributions (column r of RG) in row order
// from them: the same additions as summing contrib * (token == t) over every
// row, without the products by zero.
// ----------------------------------------------------------------------------
template <int NWORD>
HX_DEV void token_row_masks(const int* stok, int nh, int T, unsigned long long (*m)[NWORD]) {
  const int wave = threadIdx.x >> 6, lane = lane_id();
  for (int t = wave; t < T; t += blockDim.x >> 6) {
#pragma unroll
    for (int q = 0; q < NWORD; q++) {
      const int hr = 64 * q + lane;
      const unsigned long long b = __ballot(hr < nh && stok[hr < nh ? hr : 0] == t);
      if (lane == 0) m[t][q] = b;
    }
  }
}
template <int NWORD>
HX_DEV float token_row_sum(const float* contrib, int RG, int r, const unsigned long long (&m)[NWORD]) {
  float y = 0.f;
#pragma unroll
  for (int q = 0; q < NWORD; q++) {
    for (unsigned long long b = m[q]; b; b &= b - 1) y += contrib[(64 * q + __builtin_ctzll(b)) * RG + r];
  }
  return y;
}

// ----------------------------------------------------------------------------
// down + combine for T > 1 and K = 512, pipelined: workgroup = RG output rows
// over every row of h, taken in groups of 24 (24 / NW per wave; NW = 8 keeps
// the registers under 128, so 4 waves share each SIMD). The weights of
// group g + 1 (registers, two buffers) and its chunk records (registers, then
// LDS, two buffers) are loaded while group g's dot products run, so memory
// and arithmetic overlap; the contributions of all rows stay in LDS and each
// token's output is their sum in row order (slots by ascending expert, then
// the shared expert), written directly, with no partial sums to reduce.
// ----------------------------------------------------------------------------
constexpr int DP_K = 512;
// output groups of four waves per workgroup of k_down_one (measured on MI355X,
// paired: 2 against 1 saves 1.1 us a layer at C2 and 1.3 at C4 B = 1; 4 less)
constexpr int HX_DOWN_ONE_OG = 2;
// waves per output group of k_down_one: 12 (one row of h a wave) measured no
// faster for Q4_K and 0.3 us a layer slower at C2 (Q8_0), in groups of one or
// two; k_down_one_q6p's single group of 12 waves is 1.1 us a layer faster at
// C4 B = 1 than that kernel with 4 waves (and 6 no faster than 4)
constexpr int HX_DOWN_ONE_WPG = 4, HX_DOWN_Q6P_NW = 12;
template <int FMT, int LPR, int NW>
__global__ __launch_bounds__(64 * NW, 4) void k_down_pipe(ExpertArgs a) {
  using D = DChunk<FMT>;
  using Raw = typename D::Raw;
  constexpr int ROWS = 24, SPW = ROWS / NW, RG = 64 / LPR, NC = DP_K / 32;
  static_assert(SPW * NW == ROWS, "the waves split a group's rows of h evenly");
  static_assert(ROWS * NC <= 64 * NW, "one chunk of a group's rows of h per thread");
  constexpr int REC = HX_XCV_WORDS / 4;   // 16-byte words per chunk record
  // LDS: chunk records of the rows of h [2][ROWS][NC], then per row of h its
  // token, weight and expert, then the contributions [rows of h][RG]
  extern __shared__ __attribute__((aligned(16))) uint16_t xl[];
  const int T = a.T, NH = a.F + T;
  const int nh_all = a.F + (a.Is > 0 ? T : 0);
  const int ng = (nh_all + ROWS - 1) / ROWS;
  lds_v4* const rec = (lds_v4*)xl;
  int* stok = (int*)((uint8_t*)xl + 2 * ROWS * NC * HX_XCV_WORDS * 4);
  float* swt = (float*)(stok + nh_all);
  int* sexp = (int*)(swt + nh_all);
  float* contrib = (float*)(sexp + nh_all);
  {
    // the plan's tokens, weights and experts of all rows: PL loads per
    // thread (3 nh_all <= 512), all issued before any is stored
    constexpr int PL = 512 / (64 * NW);
    const int tok0 = 4 + 4 * a.max_slots, n3 = 3 * nh_all;
    int v[PL];
#pragma unroll
    for (int b = 0; b < PL; b++) {
      const int i = min(b * 64 * NW + (int)threadIdx.x, n3 - 1), part = i / nh_all, r = i - part * nh_all;
      v[b] = a.plan[tok0 + part * NH + r];
    }
#pragma unroll
    for (int b = 0; b < PL; b++) {
      const int i = b * 64 * NW + (int)threadIdx.x, part = i / nh_all, r = i - part * nh_all;
      if (i < n3) (part == 0 ? stok : part == 1 ? (int*)swt : sexp)[r] = v[b];
    }
  }
  __syncthreads();
  __shared__ unsigned long long smask[HX_DECODE_MAX_T][3];   // nh_all <= 170
  token_row_masks<3>(stok, nh_all, T, smask);   // read after the loop's last barrier
  const int lane = lane_id(), wave = threadIdx.x >> 6, rg = lane / LPR, c = lane % LPR;
  const int n0 = blockIdx.x * RG, row = n0 + rg;
  Raw ra[SPW], rb[SPW];
  u32x4v xv[REC];   // a native vector type, so the array stays in registers across the loop
  // loads of group g: this thread's chunk record (item q = thread: row
  // q / NC, chunk q % NC; past the end, the group's last row), then the
  // wave's SPW weight rows (rows past the end read row 0 of the group,
  // dropped later). The record goes first: the memory counter retires loads
  // in issue order, so staging the record waits for it alone and the
  // weights stay in flight until the group's dot products.
  auto issue = [&](int g, Raw(&raw)[SPW]) __attribute__((always_inline)) {
    const int h0 = g * ROWS, nh = min(nh_all - h0, ROWS);
    {
      const int q = min((int)threadIdx.x, nh * NC - 1), hr = q / NC, cc = q % NC;
      load_record((const u32x4v*)(a.hrec + ((int64_t)(h0 + hr) * NC + cc) * HX_XCV_WORDS), xv);
    }
#pragma unroll
    for (int s = 0; s < SPW; s++) {
      const int hr = wave + NW * s, hq = hr < nh ? hr : 0;
      const int e = sexp[h0 + hq];
      const bool sh = e == a.E;
      const int K = sh ? a.Is : a.I;
      D::load(sh ? a.sdown.base : a.down.mat(e), a.H, K, row < a.H ? row : 0, c < K / 32 ? c : 0, raw[s]);
    }
  };
  // records past the group's rows land in slots that are not read
  auto stage = [&](int g) __attribute__((always_inline)) {
    if ((int)threadIdx.x < ROWS * NC) {
      lds_v4* dst = rec + ((g & 1) * ROWS * NC + (int)threadIdx.x) * REC;
#pragma unroll
      for (int w = 0; w < REC; w++) dst[w] = xv[w];
    }
  };
  auto compute = [&](int g, const Raw(&raw)[SPW]) __attribute__((always_inline)) {
    const int h0 = g * ROWS, nh = min(nh_all - h0, ROWS);
    const lds_v4* xb = rec + (g & 1) * ROWS * NC * REC;
#pragma unroll
    for (int s = 0; s < SPW; s++) {
      const int hr = wave + NW * s;
      if (hr >= nh) continue;
      const int K = sexp[h0 + hr] == a.E ? a.Is : a.I;
      float p = 0.f;
      if (c < K / 32) {
        u32x4v v[REC];
        load_record(xb + (hr * NC + c) * REC, v);
        uint32_t xp[D::NX];
        int xs[D::NS];
    float dx;
        unpack_record<D>(v, xp, xs, dx);
        p = D::dot(raw[s], xp, xs, dx);
      }
      p = wave_sum<LPR>(p);
      if (c == 0 && row < a.H) contrib[(h0 + hr) * RG + rg] = swt[h0 + hr] * p;
    }
  };
  // group g's records go to LDS buffer g & 1 once they have arrived; every
  // wave has finished group g - 1 (the other user of that buffer) before any
  // passes the barrier that precedes group g's dot products
  issue(0, ra);
  for (int g = 0; g < ng; g += 2) {
    stage(g);
    if (g + 1 < ng) issue(g + 1, rb);
    __syncthreads();
    compute(g, ra);
    if (g + 1 >= ng) break;
    stage(g + 1);
    if (g + 2 < ng) issue(g + 2, ra);
    __syncthreads();
    compute(g + 1, rb);
  }
  __syncthreads();
  for (int i = threadIdx.x; i < T * RG; i += 64 * NW) {
    const int t = i / RG, r = i % RG;
    if (n0 + r >= a.H) continue;
    const float y = token_row_sum<3>(contrib, RG, r, smask[t]);
    if (a.resid) {
      uint16_t* px = a.resid + (int64_t)t * a.H + n0 + r;
      *px = f32_to_bf16(bf16_to_f32(*px) + bf16_to_f32(f32_to_bf16(y)));
    } else {
      ((uint16_t*)a.y)[(int64_t)t * a.H + n0 + r] = f32_to_bf16(y);
    }
  }
}

// ----------------------------------------------------------------------------
// down + combine for T > 1, K = 512 and at most DP3_ROWS rows of h: like
// k_down_pipe, but every chunk record of the rows of h is moved into LDS once
// in the prologue (with the plan), so the loop over groups of 24 rows streams
// only weights, three register buffers deep: group g + 2's weights are issued
// before group g's dot products, and the loop has no barrier. (k_down_pipe
// stages each group's records through registers; the memory counter retires
// loads in issue order, so a record load issued behind a deeper weight
// prefetch would wait for it.)
// ----------------------------------------------------------------------------
constexpr int DP3_ROWS = 96;
static_assert(DP3_ROWS <= 128, "two mask words a token");
template <int FMT, int LPR, int NW>
__global__ __launch_bounds__(64 * NW, 4) void k_down_pipe3(ExpertArgs a) {
  using D = DChunk<FMT>;
  using Raw = typename D::Raw;
  constexpr int ROWS = 24, SPW = ROWS / NW, RG = 64 / LPR, NC = DP_K / 32, REC = HX_REC_VECS;
  static_assert(SPW * NW == ROWS, "the waves split a group's rows of h evenly");
  constexpr int MAXR = (DP3_ROWS * NC * REC + 64 * NW - 1) / (64 * NW);   // 16-byte record pieces a thread moves
  // LDS: the records of every row of h [nh_all][NC], then per row its token,
  // weight and expert, then the contributions [rows of h][RG]
  extern __shared__ __attribute__((aligned(16))) uint16_t xl[];
  const int T = a.T, NH = a.F + T;
  const int nh_all = a.F + (a.Is > 0 ? T : 0);
  const int ng = (nh_all + ROWS - 1) / ROWS;
  lds_v4* const rec = (lds_v4*)xl;
  int* stok = (int*)((uint8_t*)xl + (size_t)nh_all * NC * HX_XCV_WORDS * 4);
  float* swt = (float*)(stok + nh_all);
  int* sexp = (int*)(swt + nh_all);
  float* contrib = (float*)(sexp + nh_all);
  const int tid = threadIdx.x;
  const int tok0 = plan_rows_at(a);
  // thread t RG + r (wave 0) adds token t's residual at output row n0 + r in
  // the epilogue; wave 0 moves the dwords holding them into LDS first (an
  // LDS-DMA: no register held across the loop, no wait until the epilogue)
  static_assert(HX_DECODE_MAX_T * RG <= 64, "the epilogue's outputs in wave 0");
  const int n0 = blockIdx.x * RG;
  const bool out_thread = tid < T * RG && n0 + tid % RG < a.H;
  uint32_t* const rsl = (uint32_t*)(contrib + nh_all * RG);   // 64 dwords
  if (a.resid && tid < 64) {
    const int64_t i = (int64_t)min(tid / RG, T - 1) * a.H + min(n0 + tid % RG, a.H - 1);   // H even
    dma4(a.resid + (i & ~(int64_t)1), (uint32_t)(uintptr_t)(lds_u8*)rsl);
  }
  u32x4v rv[MAXR];
  {
    // the plan's tokens, weights and experts of all rows (PL loads a thread),
    // then the records (MAXR 16-byte pieces a thread), all issued before any
    // is stored; the plan's loads first, so storing them waits for them alone
    constexpr int PL = (3 * DP3_ROWS + 64 * NW - 1) / (64 * NW);
    const int n3 = 3 * nh_all, n16 = nh_all * NC * REC;
    int v[PL];
#pragma unroll
    for (int b = 0; b < PL; b++) {
      const int i = min(b * 64 * NW + tid, n3 - 1), part = i / nh_all, r = i - part * nh_all;
      v[b] = a.plan[tok0 + part * NH + r];
    }
    __builtin_amdgcn_sched_barrier(0);   // the plan's loads go out before the records'
#pragma unroll
    for (int b = 0; b < MAXR; b++) rv[b] = ((const u32x4v*)a.hrec)[min(b * 64 * NW + tid, n16 - 1)];
#pragma unroll
    for (int b = 0; b < PL; b++) {
      const int i = b * 64 * NW + tid, part = i / nh_all, r = i - part * nh_all;
      if (i < n3) (part == 0 ? stok : part == 1 ? (int*)swt : sexp)[r] = v[b];
    }
  }
  // the records stay in flight across this barrier: the weight loads behind
  // it wait for the plan alone
  lds_barrier();
  __shared__ unsigned long long smask[HX_DECODE_MAX_T][2];   // nh_all <= DP3_ROWS <= 128
  const int lane = lane_id(), wave = tid >> 6, rg = lane / LPR, c = lane % LPR;
  const int row = n0 + rg;
  Raw ra[SPW], rb[SPW], rc[SPW];
  // the wave's SPW weight rows of group g (rows past the end read row 0 of
  // the group, dropped later)
  // the experts of group g's rows (LDS reads), then their weight loads
  auto experts = [&](int g, int (&ev)[SPW]) __attribute__((always_inline)) {
    const int h0 = g * ROWS, nh = min(nh_all - h0, ROWS);
#pragma unroll
    for (int s = 0; s < SPW; s++) {
      const int hr = wave + NW * s;
      ev[s] = sexp[h0 + (hr < nh ? hr : 0)];
    }
  };
  auto issue_e = [&](const int (&ev)[SPW], Raw(&raw)[SPW]) __attribute__((always_inline)) {
#pragma unroll
    for (int s = 0; s < SPW; s++) {
      const int e = ev[s];
      const bool sh = e == a.E;
      const int K = sh ? a.Is : a.I;
      D::load(sh ? a.sdown.base : a.down.mat(e), a.H, K, row < a.H ? row : 0, c < K / 32 ? c : 0, raw[s]);
    }
  };
  auto issue = [&](int g, Raw(&raw)[SPW]) __attribute__((always_inline)) {
    int ev[SPW];
    experts(g, ev);
    issue_e(ev, raw);
  };
  issue(0, ra);
  if (ng > 1) issue(1, rb);
  token_row_masks<2>(stok, nh_all, T, smask);   // read after the loop's last barrier
  {
    const int n16 = nh_all * NC * REC;
#pragma unroll
    for (int b = 0; b < MAXR; b++) {
      const int i = b * 64 * NW + tid;
      if (i < n16) rec[i] = rv[b];
    }
  }
  lds_barrier();   // the first groups' weight loads stay in flight
  auto compute = [&](int g, const Raw(&raw)[SPW]) __attribute__((always_inline)) {
    const int h0 = g * ROWS, nh = min(nh_all - h0, ROWS);
#pragma unroll
    for (int s = 0; s < SPW; s++) {
      const int hr = wave + NW * s;
      if (hr >= nh) continue;
      const int K = sexp[h0 + hr] == a.E ? a.Is : a.I;
      float p = 0.f;
      if (c < K / 32) {
        u32x4v v[REC];
        load_record(rec + ((h0 + hr) * NC + c) * REC, v);
        uint32_t xp[D::NX];
        int xs[D::NS];
        float dx;
        unpack_record<D>(v, xp, xs, dx);
        p = D::dot(raw[s], xp, xs, dx);
      }
      p = wave_sum<LPR>(p);
      if (c == 0 && row < a.H) contrib[(h0 + hr) * RG + rg] = swt[h0 + hr] * p;
    }
  };
  for (int g = 0; g < ng; g += 3) {
    if (g + 2 < ng) issue(g + 2, rc);
    compute(g, ra);
    if (g + 1 >= ng) break;
    if (g + 3 < ng) issue(g + 3, ra);
    compute(g + 1, rb);
    if (g + 2 >= ng) break;
    if (g + 4 < ng) issue(g + 4, rb);
    compute(g + 2, rc);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // wave 0's residual DMA has landed
  __syncthreads();
  if (out_thread) {
    const int t = tid / RG, r = tid % RG;
    const float y = token_row_sum<2>(contrib, RG, r, smask[t]);
    const int64_t o = (int64_t)t * a.H + n0 + r;
    if (a.resid) {
      const uint32_t w = rsl[tid];
      const float rx = __uint_as_float((o & 1) ? (w & 0xffff0000u) : (w << 16));
      a.resid[o] = f32_to_bf16(rx + bf16_to_f32(f32_to_bf16(y)));
    } else {
      ((uint16_t*)a.y)[o] = f32_to_bf16(y);
    }
  }
}

// sum of the down kernel's per-group partials, in group order, for T tokens
__global__ __launch_bounds__(256) void k_down_reduce(ExpertArgs a, int groups) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)a.T * a.H) return;
  const int64_t TH = (int64_t)a.T * a.H;
  float y = 0.f;
  for (int g = 0; g < groups; g++) y += a.dpart[g * TH + i];
  if (a.resid) a.resid[i] = f32_to_bf16(bf16_to_f32(a.resid[i]) + bf16_to_f32(f32_to_bf16(y)));
  else ((uint16_t*)a.y)[i] = f32_to_bf16(y);
}

// ----------------------------------------------------------------------------
// launchers: used for bf16 activations with Q8_0 / Q4_K / Q6_K weights whose
// input dims give 16, 32 or 64 chunks of 32 per row (K = 512, 1024, 2048)
// ----------------------------------------------------------------------------
bool decode_fast_ok(const ExpertArgs& a) {
  auto ok = [](int fmt, int K) {
    return (fmt == HX_Q8_0 || fmt == HX_Q4_K || fmt == HX_Q6_K) && (K == 512 || K == 1024 || K == 2048);
  };
  const int Kd = a.I > a.Is ? a.I : a.Is;
  // one vec_dot type for the tokens (gate and up) and one for h (down)
  const bool same = a.up.fmt == a.gate.fmt &&
                    (a.Is == 0 || (a.sgate.fmt == a.gate.fmt && a.sup.fmt == a.gate.fmt && a.sdown.fmt == a.down.fmt));
  return a.xbf && same && ok(a.gate.fmt, a.H) && ok(a.down.fmt, Kd) && (a.Is == 0 || a.Is == a.I);
}

template <int FMT>
static hipError_t router_dec_fmt(const RouterArgs& r, const ExpertArgs& a, bool rbf, hipStream_t s) {
  // One router row a wave, the tokens in pairs: each pair's router
  // workgroups after the previous pair's, so 8 tokens take 4 x 129 workgroups
  // (measured on MI355X, paired: 3.4 us a layer less at 8 tokens than 65
  // workgroups of two rows x 8 tokens a wave; pairs 0.4-0.6 us less than
  // groups of 4 at 4 and 8 tokens, and 0.3-1.3 us less than one token a
  // group). The blocks after the router's quantise the tokens (one workgroup
  // each).
#define RD(RB, TT)                                                                          \
  {                                                                                         \
    const int nrb = (r.E1 + 3) / 4, ng = (a.T + TT - 1) / TT, ncb = a.T;                    \
    hx_launch(k_router_dec<FMT, RB, TT>, dim3(nrb * ng + ncb), dim3(256), 0, s, r, a, nrb); \
  }
#define RD_T(RB) { if (r.T <= 1) RD(RB, 1) else RD(RB, 2) }
  if (rbf) RD_T(true) else RD_T(false)
#undef RD_T
#undef RD
  return hipGetLastError();
}

template <int FMT>
static hipError_t gate_up_dec_fmt(const RouterArgs& r, const ExpertArgs& a, hipStream_t s) {
  const int nch = a.H / 32;
  const int nroute = a.F < a.E ? a.F : a.E;
  constexpr int NR = 2;
#define GUD(LPR)                                                                          \
  {                                                                                       \
    constexpr int RG = 64 / LPR;                                                          \
    dim3 grid((a.I + 4 * RG * NR - 1) / (4 * RG * NR), nroute + 1);                       \
    hipLaunchKernelGGL((k_gate_up_dec<FMT, LPR, NR>), grid, dim3(256), 0, s, r, a);       \
  }
  if (nch == 64) GUD(64) else if (nch == 32) GUD(32) else GUD(16)
#undef GUD
  return hipGetLastError();
}

template <int FMT>
static hipError_t gate_up_plan_fmt(const ExpertArgs& a, hipStream_t s) {
  const int nch = a.H / 32;
  const int rows = a.I > a.Is ? a.I : a.Is;
  constexpr int NR = 2;
  // grid rows: the shared expert's slot, then one per routed slot
  // (max_slots = min(F, E) + 1 covers both)
#define GUP(LPR)                                                                          \
  {                                                                                       \
    constexpr int RG = 64 / LPR;                                                          \
    dim3 grid((rows + 4 * RG * NR - 1) / (4 * RG * NR), a.max_slots);                     \
    hipLaunchKernelGGL((k_gate_up_plan<FMT, LPR, NR>), grid, dim3(256), 0, s, a);         \
  }
  if (nch == 64) GUP(64) else if (nch == 32) GUP(32) else GUP(16)
#undef GUP
  return hipGetLastError();
}

template <int FMT>
static hipError_t down_dec_fmt(const ExpertArgs& a, hipStream_t s) {
  const int K = a.I > a.Is ? a.I : a.Is, nch = K / 32;
  const int nh_all = a.F + (a.Is > 0 ? a.T : 0);
  const int groups = down_groups(a.F, a.Is > 0 ? a.T : 0);
  if (a.hstride != K) return hipErrorInvalidValue;   // rows of h contiguous
  if (a.T > HX_DECODE_MAX_T) return hipErrorInvalidValue;   // the per-token row masks
  // one token with at most 12 rows of h (k <= 11): the workgroup quantises the
  // rows of h itself; otherwise k_hrec writes their records first
  const bool qh = a.T == 1 && nh_all <= 12;
  if (!qh) {
    const dim3 g((unsigned)((nh_all + 3) / 4));
    if (nch == 64) hipLaunchKernelGGL((k_hrec<FMT, 4>), g, dim3(256), 0, s, a, nh_all);
    else if (nch == 32) hipLaunchKernelGGL((k_hrec<FMT, 2>), g, dim3(256), 0, s, a, nh_all);
    else hipLaunchKernelGGL((k_hrec<FMT, 1>), g, dim3(256), 0, s, a, nh_all);
  }
  // every row of h in one workgroup per RG output rows, pipelined over groups
  // (measured on MI355X at T = 4 and 8: faster than the grouped kernel + the
  // partial-sum pass, and than one workgroup per (slot, output rows) writing
  // per-row results that a second pass sums per token: +4.0 / +2.9 us a layer
  // at B = 4 / 8); up to DP3_ROWS rows of h with every record in LDS and the
  // weights three groups deep, else the plan of all rows in one pass
  // (3 rows <= 512) and records staged per group
  if (a.T > 1 && nch == DP_K / 32 && nh_all <= DP3_ROWS) {
    constexpr int LPR = DP_K / 32, RG = 64 / LPR;
    const size_t lds = (size_t)nh_all * (DP_K / 32) * HX_XCV_WORDS * 4 + (size_t)nh_all * (3 + RG) * 4 + 64 * 4;
    hipLaunchKernelGGL((k_down_pipe3<FMT, LPR, 8>), dim3((a.H + RG - 1) / RG), dim3(512), lds, s, a);
    return hipGetLastError();
  }
  if (a.T > 1 && nch == DP_K / 32 && 3 * nh_all <= 512) {
    constexpr int LPR = DP_K / 32, RG = 64 / LPR;
    const size_t lds = (size_t)2 * 24 * (DP_K / 32) * HX_XCV_WORDS * 4 + (size_t)nh_all * (3 + RG) * 4;
    hipLaunchKernelGGL((k_down_pipe<FMT, LPR, 8>), dim3((a.H + RG - 1) / RG), dim3(512), lds, s, a);
    return hipGetLastError();
  }
#define DD(LPR)                                                                                       \
  {                                                                                                   \
    constexpr int RG = 64 / LPR, OG = HX_DOWN_ONE_OG;                                                 \
    if (qh && FMT == HX_Q6_K && LPR == 16) {                                                          \
      const size_t lds = (size_t)12 * 16 * HX_XCV_WORDS * 4 + (size_t)12 * (3 + 8) * 4;               \
      hx_launch(k_down_one_q6p<HX_DOWN_Q6P_NW>, dim3((a.H + 7) / 8), dim3(64 * HX_DOWN_Q6P_NW), (uint32_t)lds, s, a); \
    } else if (qh) {                                                                                  \
      const size_t lds = (size_t)12 * LPR * HX_XCV_WORDS * 4 + (size_t)12 * (3 + RG * OG) * 4;        \
      hx_launch(k_down_one<FMT, LPR, OG, HX_DOWN_ONE_WPG>, dim3((a.H + RG * OG - 1) / (RG * OG)), dim3(64 * HX_DOWN_ONE_WPG * OG), (uint32_t)lds, s, a); \
    } else {                                                                                          \
      const size_t lds = (size_t)HX_DOWN_ROWS * (3 + RG) * 4;                                         \
      hipLaunchKernelGGL((k_down_dec<FMT, LPR, 6, 4>), dim3((a.H + RG - 1) / RG, groups), dim3(256), lds, s, a); \
    }                                                                                                 \
  }
  if (nch == 64) DD(64) else if (nch == 32) DD(32) else DD(16)
#undef DD
  if (!qh && groups > 1)
    hipLaunchKernelGGL(k_down_reduce, dim3((unsigned)(((int64_t)a.T * a.H + 255) / 256)), dim3(256), 0, s, a, groups);
  return hipGetLastError();
}

hipError_t launch_router_dec(const RouterArgs& r, const ExpertArgs& a, bool rbf, hipStream_t s) {
  switch (a.gate.fmt) {
    case HX_Q8_0: return router_dec_fmt<HX_Q8_0>(r, a, rbf, s);
    case HX_Q4_K: return router_dec_fmt<HX_Q4_K>(r, a, rbf, s);
    case HX_Q6_K: return router_dec_fmt<HX_Q6_K>(r, a, rbf, s);
    default: return hipErrorInvalidValue;
  }
}

template <int FMT>
static hipError_t gate_up_dec1_fmt(const RouterArgs& r, const ExpertArgs& a, hipStream_t s) {
  const int rows = a.I > a.Is ? a.I : a.Is;
  hx_launch(k_gate_up_dec1<FMT, 8, 10>, dim3((rows + 1) / 2), dim3(256), 0, s, r, a);
  return hipGetLastError();
}

hipError_t launch_gate_up_dec(const RouterArgs& r, const ExpertArgs& a, hipStream_t s) {
  // one token, H = 2048, top-10 of 257..512 experts: the overlapped kernel
  if (a.T == 1 && a.H == 64 * 32 && a.k == 10 && r.E > 256 && r.E <= 512) {
    switch (a.gate.fmt) {
      case HX_Q8_0: return gate_up_dec1_fmt<HX_Q8_0>(r, a, s);
      case HX_Q4_K: return gate_up_dec1_fmt<HX_Q4_K>(r, a, s);
      case HX_Q6_K: return gate_up_dec1_fmt<HX_Q6_K>(r, a, s);
      default: break;
    }
  }
  switch (a.gate.fmt) {
    case HX_Q8_0: return gate_up_dec_fmt<HX_Q8_0>(r, a, s);
    case HX_Q4_K: return gate_up_dec_fmt<HX_Q4_K>(r, a, s);
    case HX_Q6_K: return gate_up_dec_fmt<HX_Q6_K>(r, a, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_gate_up_plan(const ExpertArgs& a, hipStream_t s) {
  switch (a.gate.fmt) {
    case HX_Q8_0: return gate_up_plan_fmt<HX_Q8_0>(a, s);
    case HX_Q4_K: return gate_up_plan_fmt<HX_Q4_K>(a, s);
    case HX_Q6_K: return gate_up_plan_fmt<HX_Q6_K>(a, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_down_dec(const ExpertArgs& a, hipStream_t s) {
  switch (a.down.fmt) {
    case HX_Q8_0: return down_dec_fmt<HX_Q8_0>(a, s);
    case HX_Q4_K: return down_dec_fmt<HX_Q4_K>(a, s);
    case HX_Q6_K: return down_dec_fmt<HX_Q6_K>(a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace hx
