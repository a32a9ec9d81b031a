// Prefill routing with the router GEMM on MFMA and an exact finish.
//
// The routing contract fixes every logit as the canonical fmaf chain (groups
// of 8 inputs, group g in lane g % 64, the 64 partials by the xor butterfly),
// rounded to bf16, plus the optional bias. The top-k ids and the dispatch
// permutation must equal the ones those logits give (route_scatter,
// crates/neuron/src/harness/arch/qwen3_5/moe.rs:124-162; dispatch sort,
// crates/neuron/src/harness/tp/tp_qwen3_5.rs:1189). Computing all T x E
// canonical logits costs a VALU pass over 2 T H E flop; here:
//
// 1. k_router_mfma: m[t][e] = x_t . r_e on v_mfma_f32_16x16x32_bf16 (bf16
//    products are exact in f32). Each MFMA starts from a zero accumulator and
//    its results are added to the running f32 sums, so the distance to the
//    exact dot product is bounded whatever order the MFMA sums its 32 products
//    in: with S = sum |x_i r_i| <= |x| |r| and u = 2^-24,
//      |m - exact| <= 4u * 31 S    (one K chunk: 31 additions, each allowed a
//                                   relative error of 4u -- a probe of this
//                                   MFMA found at most 8u per 32 products --
//                                   on partial sums below the chunk's S)
//                   + u * H/32 S   (the running sum over the H/32 chunks)
//    and the canonical value c has |c - exact| <= u (8 ceil(H/512) + 6) S (its
//    fmaf chain of at most 8 ceil(H/512) steps per lane, and the butterfly).
//    So |c - m| <= u (130 + H/32 + 8 ceil(H/512)) |x| |r| (to first order; a
//    factor 1.01 covers the rest) plus an absolute slack for flushed denormal
//    inputs, products and sums.
// 2. k_route_mfma, one wave per token: each logit lies in [lo, hi] = bf16 of
//    m -/+ that bound (monotone rounding), plus the bias. tau = the k-th
//    largest of the 64 lanes' largest lo (expert e in lane e % 64): at least k
//    experts have a logit >= tau, so only the candidates with hi >= tau can be
//    among the top k.
//    Candidates whose lo != hi get their canonical logit recomputed exactly
//    (the token row is held in registers in the canonical layout); the shared
//    expert's gate logit is always recomputed. The top k of the candidates by
//    (logit desc, id asc) are the reference's top k by (probability desc, id
//    asc) when equal logits are the only equal probabilities that matter:
//    exp(l - max) is computed with the same expf_route as the reference path,
//    and every adjacent pair of distinct logits among the first k + 1 (the
//    best excluded candidate, or the largest hi of the excluded experts) must
//    have exps at least 2^-20 apart (relative) and >= 2^-100, so dividing by
//    any softmax denominator keeps them strictly ordered. A token that fails
//    any check (more than 64 candidates, non-finite values, near-equal exps)
//    is routed by the exact path inside the same wave: all E canonical
//    logits, then the softmax / top-k of route_token_regs.
//    Weights: exp(l_r - max) / sum over the k selected (renormalisation, which
//    this path requires: the softmax denominator cancels), within a few ulps
//    of the reference's p_r / sum p.
#include "hx_internal.h"
#include "hx_quant.h"
#include "hx_route_small.h"

namespace hx {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// K chunks (of 32) per pair of K steps: H is a multiple of 32 RM_GROUP
constexpr int RM_GROUP = 4;
// K steps of 64 whose loads are in flight (a ring of RM_AHEAD + 1 register
// buffers of 16 VGPRs). Measured on MI355X at 2048 tokens over 4 logit
// planes: 8 steps 19.0 us, 6 18.8, 4 16.7, 3 16.2, 2 16.1 -- the registers buy
// more resident waves than the deeper look-ahead saves; with 2 planes at 2048
// tokens and 1 at 4096 (16 and 32 steps per workgroup) 3 and 4 steps ahead
// measured the same as 2.
constexpr int RM_AHEAD = 2;

// Grid (E / 64 expert blocks, token blocks of 64 rounded up to 8); workgroup =
// 64 tokens x 64 experts, all expert blocks of one token block on one XCD
// (workgroup L runs on XCD L % 8). K goes in NST steps of 64: each step's
// operand tiles (64 token rows and 64 router rows x 128 bytes) are read with
// coalesced 16-byte loads (8 lanes per 128-byte row segment), RM_AHEAD steps
// ahead, into registers, and written to one of two LDS buffers; wave w then computes
// tokens 32 (w & 1) .., experts 32 (w >> 1) .. as 2 x 2 MFMA tiles from
// fragments read out of LDS (lane l: row l % 16, K elements 8 (l / 16) ..).
// Slot s (16 bytes) of row r is stored at slot s ^ ((r >> 1) & 7): the 16
// rows a fragment read touches then fall in 16 distinct bank groups. The K
// loop is unrolled (NST is a template argument), so the compiler's waits
// count exactly the loads in flight.
//
// Two jobs ride along (each a null pointer when not wanted): the workgroups
// write the f16 copy of the tokens the MFMA expert kernels read, K step s by
// the workgroup of expert block s % (expert blocks)
// (xh: each group of 8 elements converted exactly and stored at its own place,
// in natural order when xnat is set, else in the swizzled order
// (e0,e2)(e1,e3)(e4,e6)(e5,e7)), and the dispatch
// histogram and token bitmap the routing kernel fills are cleared (ndmap ints).
//
// Split K: grid z = s < S takes K steps s NST .. s NST + NST - 1 (NST steps of
// 64 per workgroup, H = 64 NST S) and writes its sums to logit plane s (plane
// 0: m, plane s >= 1: mp + (s - 1) T E1); the routing kernel adds the planes
// in order.
// With S planes each running sum covers H / (32 S) chunks and the planes add
// S - 1 roundings: fewer than the H / 32 of one running sum, so the bound
// below holds as stated.
template <int NST>
__global__ __launch_bounds__(256) void k_router_mfma(const uint16_t* __restrict__ x, const uint16_t* __restrict__ R,
                                                     int T, int H, int E, int E1, float* __restrict__ m,
                                                     float* __restrict__ mp, uint16_t* __restrict__ xh, int xnat,
                                                     int32_t* __restrict__ dmap, int ndmap) {
  static_assert(NST % 2 == 0, "K steps come in pairs");
  __shared__ __attribute__((aligned(16))) uint8_t lds[2][2][64 * 128];   // [buffer][A / B][row * 128 + slot * 16]
  const int NX = gridDim.x, L = blockIdx.y * NX + blockIdx.x, z = blockIdx.z;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  if (dmap) {
    const int nwg = NX * gridDim.y * gridDim.z, lz = z * NX * gridDim.y + L;
    for (int i = lz * 256 + tid; i < ndmap; i += nwg * 256) dmap[i] = 0;
  }
  const int eb = (L >> 3) % NX, tb = (L / (8 * NX)) * 8 + (L & 7);
  if (tb * 64 >= T) return;   // whole workgroups
  const int ks0 = z * NST;     // this workgroup's first K step
  if (z > 0) m = mp + (int64_t)(z - 1) * T * E1;
  // loads: this thread's two 16-byte slots of each operand tile per step
  // (slot u = q * 256 + tid: row u / 8, 16-byte slot u % 8) as buffer loads
  // (a 32-bit byte offset and the step's scalar offset) from descriptors over
  // this workgroup's token block (at most 64 x 8 KB) and the router; rows past
  // the end are clamped
  const int nrows = min(64, T - tb * 64);
  int goff[2][2], soff[2];
#pragma unroll
  for (int q = 0; q < 2; q++) {
    const int u = q * 256 + tid, r = u >> 3, sl = u & 7;
    goff[0][q] = (min(r, nrows - 1) * H + 8 * sl) * 2;
    goff[1][q] = (min(eb * 64 + r, E - 1) * H + 8 * sl) * 2;
    soff[q] = r * 128 + ((sl ^ ((r >> 1) & 7)) << 4);
  }
  const __amdgpu_buffer_rsrc_t rsa =
      __builtin_amdgcn_make_buffer_rsrc((void*)(x + (int64_t)tb * 64 * H), 0, nrows * H * 2, 0x00020000);
  const __amdgpu_buffer_rsrc_t rsb = __builtin_amdgcn_make_buffer_rsrc((void*)R, 0, E * H * 2, 0x00020000);
  u32x4_t st[RM_AHEAD + 1][2][2];   // [step % (RM_AHEAD + 1)][A / B][q]
  auto load = [&](int step, int b) {
#pragma unroll
    for (int q = 0; q < 2; q++) {
      st[b][0][q] = __builtin_amdgcn_raw_buffer_load_b128(rsa, goff[0][q], (ks0 + step) * 128, 0);
      st[b][1][q] = __builtin_amdgcn_raw_buffer_load_b128(rsb, goff[1][q], (ks0 + step) * 128, 0);
    }
  };
  auto store = [&](int b, int buf, int step) {
#pragma unroll
    for (int o = 0; o < 2; o++)
#pragma unroll
      for (int q = 0; q < 2; q++) *(u32x4_t*)(&lds[buf][o][soff[q]]) = st[b][o][q];
    // the f16 tokens of K step s are written by the token block's workgroup of
    // expert block s % NX (every one of them loads every step of its K range)
    if (xh && (ks0 + step) % NX == eb) {
#pragma unroll
      for (int q = 0; q < 2; q++) {
        const int u = q * 256 + tid, r = u >> 3, sl = u & 7;
        if (r < nrows) {
          const u32x4_t v = st[b][0][q];
          uint32_t h[4];
#pragma unroll
          for (int j2 = 0; j2 < 4; j2++) {
            const _Float16 lo16 = (_Float16)__uint_as_float(v[j2] << 16);
            const _Float16 hi16 = (_Float16)__uint_as_float(v[j2] & 0xffff0000u);
            h[j2] = (uint32_t)__builtin_bit_cast(uint16_t, lo16) | ((uint32_t)__builtin_bit_cast(uint16_t, hi16) << 16);
          }
          u32x4_t o;
          if (xnat) {
            o[0] = h[0]; o[1] = h[1]; o[2] = h[2]; o[3] = h[3];
          } else {
            o[0] = __builtin_amdgcn_perm(h[1], h[0], 0x05040100u);
            o[1] = __builtin_amdgcn_perm(h[1], h[0], 0x07060302u);
            o[2] = __builtin_amdgcn_perm(h[3], h[2], 0x05040100u);
            o[3] = __builtin_amdgcn_perm(h[3], h[2], 0x07060302u);
          }
          *(u32x4_t*)(xh + ((int64_t)tb * 64 + r) * H + 64 * (ks0 + step) + 8 * sl) = o;
        }
      }
    }
  };
  // fragment reads: row rowbase + l % 16, logical slot c * 4 + l / 16
  const int r16 = lane & 15, kq = lane >> 4;
  int fo[2][2];   // [A / B][i]: LDS byte offset of this lane's row, slot applied per chunk
  int rsw[2][2];
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const int ra = 32 * (wave & 1) + 16 * i + r16, rb = 32 * (wave >> 1) + 16 * i + r16;
    fo[0][i] = ra * 128;
    fo[1][i] = rb * 128;
    rsw[0][i] = (ra >> 1) & 7;
    rsw[1][i] = (rb >> 1) & 7;
  }
  f32x4_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  auto compute = [&](int buf) {
#pragma unroll
    for (int c = 0; c < 2; c++) {
      u32x4_t fa[2], fb[2];
#pragma unroll
      for (int i = 0; i < 2; i++) {
        fa[i] = *(const u32x4_t*)(&lds[buf][0][fo[0][i] + (((c * 4 + kq) ^ rsw[0][i]) << 4)]);
        fb[i] = *(const u32x4_t*)(&lds[buf][1][fo[1][i] + (((c * 4 + kq) ^ rsw[1][i]) << 4)]);
      }
      // the empty asm makes each sum live here, so the compiler cannot sink
      // the additions (and keep every chunk's MFMA results) to the end
#pragma unroll
      for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
          const f32x4_t z = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              __builtin_bit_cast(bf16x8_t, fa[i]), __builtin_bit_cast(bf16x8_t, fb[j]), f32x4_t{0.f, 0.f, 0.f, 0.f},
              0, 0, 0);
          acc[i][j] = acc[i][j] + z;
          asm volatile("" : "+v"(acc[i][j]));
        }
    }
  };
  constexpr int NB = RM_AHEAD + 1;
#pragma unroll
  for (int s = 0; s < RM_AHEAD && s < NST; s++) load(s, s);
  store(0, 0, 0);
  __syncthreads();
#pragma unroll
  for (int s = 0; s < NST; s++) {
    // slot (s + RM_AHEAD) % NB last held step s - 1, stored to LDS before now
    if (s + RM_AHEAD < NST) load(s + RM_AHEAD, (s + RM_AHEAD) % NB);
    if (s + 1 < NST) store((s + 1) % NB, (s + 1) & 1, s + 1);
    compute(s & 1);
    __syncthreads();
  }
  // D: lane l holds rows 4 (l / 16) + q of column l % 16
  const int t0 = tb * 64 + 32 * (wave & 1), e0 = eb * 64 + 32 * (wave >> 1);
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int e = e0 + 16 * j + r16;
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const int t = t0 + 16 * i + 4 * (lane >> 4) + q;
        if (t < T && e < E) m[(int64_t)t * E1 + e] = acc[i][j][q];
      }
    }
}

HX_DEV float bf16r(float v) { return bf16_to_f32(f32_to_bf16(v)); }

// B canonical logit sums (before the bf16 rounding) of router rows rows[b]
// against the token row held in xr (group g = lane + 64 i in xr[i]): the
// fmaf chain over the lane's groups in order, then the butterfly.
template <int NG>
HX_DEV void canon_load(const uint16_t* R, int H, int row, uint32_t (&wr)[NG][4]) {
  const int lane = lane_id(), G = H / 8;
#pragma unroll
  for (int i = 0; i < NG; i++) {
    const int g = min(lane + 64 * i, G - 1);
    const uint4 v = *(const uint4*)(R + (int64_t)row * H + 8 * g);
    wr[i][0] = v.x; wr[i][1] = v.y; wr[i][2] = v.z; wr[i][3] = v.w;
  }
}
template <int NG, int B>
HX_DEV void canon_dots_regs(const uint32_t (&xr)[NG][4], const uint32_t (&wr)[B][NG][4], int H, float* out) {
  const int lane = lane_id(), G = H / 8;
  float acc[B];
#pragma unroll
  for (int b = 0; b < B; b++) acc[b] = 0.0f;
#pragma unroll
  for (int i = 0; i < NG; i++) {
    if (lane + 64 * i >= G) break;
#pragma unroll
    for (int q = 0; q < 8; q++) {
      const float xv = __uint_as_float(q & 1 ? xr[i][q / 2] & 0xffff0000u : xr[i][q / 2] << 16);
#pragma unroll
      for (int b = 0; b < B; b++) {
        const float wv = __uint_as_float(q & 1 ? wr[b][i][q / 2] & 0xffff0000u : wr[b][i][q / 2] << 16);
        acc[b] = __builtin_fmaf(xv, wv, acc[b]);
      }
    }
  }
#pragma unroll
  for (int b = 0; b < B; b++) out[b] = wave_sum<64>(acc[b]);
}
template <int NG, int B>
HX_DEV void canon_dots(const uint32_t (&xr)[NG][4], const uint16_t* R, int H, const int* rows, float* out) {
  uint32_t wr[B][NG][4];
#pragma unroll
  for (int b = 0; b < B; b++) canon_load<NG>(R, H, rows[b], wr[b]);
  canon_dots_regs<NG, B>(xr, wr, H, out);
}

struct alignas(16) RouteMfmaSmem {
  int ce[4][64];      // candidate experts of each wave's token
  float cl[4][64];    // their logits (exact once the recomputations are in)
  float sl[4][64];    // logits in rank order
  int se[4][64];      // experts in rank order
};

// absolute slack of |canonical - MFMA| per unit of (sqrt(H) (|x| + |r|) + 3 H):
// every term, product or partial sum that a denormal flush can change is below
// 2^-126 times that
#define HX_RM_ABS 0x1p-100f

// the token's xq from its row in the canonical layout (group g of 8 in lane
// g % 64, register g / 64): the Q8 codes of the m <= 64 expert calls (a Q8_K
// block is 32 consecutive lanes of a register, a Q8_0 block 4), stored as f16
// d q in xh's element order; lanes past the row hold whole zero blocks
template <int FMT, int NG>
HX_DEV void route_xq(const RouterArgs& a, const uint32_t (&xr)[NG][4], int t) {
  const int G = a.H / 8, lane = lane_id();
  uint16_t* dst = a.xq + (int64_t)t * a.H;
#pragma unroll
  for (int i = 0; i < NG; i++) {
    const int g = lane + 64 * i;
    float x[8], q[8], d;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      x[2 * j] = g < G ? __uint_as_float(xr[i][j] << 16) : 0.0f;
      x[2 * j + 1] = g < G ? __uint_as_float(xr[i][j] & 0xffff0000u) : 0.0f;
    }
    quant_group<FMT>(x, q, d);
    if (g < G) {
      _Float16 h[8];
#pragma unroll
      for (int j = 0; j < 8; j++) h[j] = fq_f16(q[j], d);
      auto pk = [&](int u, int v) {
        return (uint32_t)__builtin_bit_cast(uint16_t, h[u]) | ((uint32_t)__builtin_bit_cast(uint16_t, h[v]) << 16);
      };
      *(uint4*)(dst + 8 * g) = a.xq_nat ? make_uint4(pk(0, 1), pk(2, 3), pk(4, 5), pk(6, 7))
                                        : make_uint4(pk(0, 2), pk(1, 3), pk(4, 6), pk(5, 7));
    }
  }
}

template <int EPL, int NG>
__global__ __launch_bounds__(256) void k_route_mfma(RouterArgs a) {
  __shared__ RouteMfmaSmem sm;
  const int wave = threadIdx.x >> 6, lane = lane_id();
  // workgroup L runs on XCD L % 8, as did the MFMA logits of token block tb
  // (64 tokens) on XCD tb % 8: workgroup L takes 4 tokens of a block on its own
  // XCD, so the logits row and the token row are in that XCD's L2
  const int L = blockIdx.x, jb = L >> 3;
  const int t = ((jb >> 4) * 8 + (L & 7)) * 64 + (jb & 15) * 4 + wave;
  if (t >= a.T) return;   // whole waves; no workgroup barrier below
  const int H = a.H, G = H / 8, E = a.E, k = a.k;
  const uint16_t* R = (const uint16_t*)a.R;
  // the shared expert's gate row (its logit is always computed exactly)
  uint32_t wsh[1][NG][4];
  if (a.has_shared) canon_load<NG>(R, H, E, wsh[0]);
  // the token row in the canonical layout, the MFMA logits, row norms, bias
  uint32_t xr[NG][4];
#pragma unroll
  for (int i = 0; i < NG; i++) {
    const int g = min(lane + 64 * i, G - 1);
    const uint4 v = *(const uint4*)((const uint16_t*)a.x + (int64_t)t * H + 8 * g);
    xr[i][0] = v.x; xr[i][1] = v.y; xr[i][2] = v.z; xr[i][3] = v.w;
  }
  // the MFMA logits: the sum of the split-K planes, in plane order
  const float* mrow = a.logits + (int64_t)t * a.E1;
  const int64_t plane = (int64_t)a.T * a.E1;   // floats per logit plane
  float mv[EPL], nw[EPL], bv[EPL];
#pragma unroll
  for (int j = 0; j < EPL; j++) {
    const int e = min(lane + 64 * j, E - 1);
    mv[j] = mrow[e];
    nw[j] = a.rnorm[e];
    bv[j] = a.bias ? a.bias[e] : 0.0f;
  }
  {
    // every plane's loads first (one memory round trip), then the sums in plane order
    float pv[HX_RM_SPLITS - 1][EPL];
#pragma unroll
    for (int z = 1; z < HX_RM_SPLITS; z++) {
      const float* prow = a.mplanes + (z - 1) * plane + (int64_t)t * a.E1;
#pragma unroll
      for (int j = 0; j < EPL; j++) pv[z - 1][j] = z < a.msplit ? prow[min(lane + 64 * j, E - 1)] : 0.0f;
    }
#pragma unroll
    for (int z = 1; z < HX_RM_SPLITS; z++)
#pragma unroll
      for (int j = 0; j < EPL; j++)
        if (z < a.msplit) mv[j] = mv[j] + pv[z - 1][j];
  }
  // |x| from above: the f32 sum of squares is within 40 u of the exact one
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < NG; i++) {
    if (lane + 64 * i >= G) break;
#pragma unroll
    for (int q = 0; q < 8; q++) {
      const float v = __uint_as_float(q & 1 ? xr[i][q / 2] & 0xffff0000u : xr[i][q / 2] << 16);
      ss = __builtin_fmaf(v, v, ss);
    }
  }
  ss = wave_sum<64>(ss);
  if (a.xq) {   // wave-uniform
    if (a.xq_q80) route_xq<HX_Q8_0, NG>(a, xr, t);
    else route_xq<HX_Q4_K, NG>(a, xr, t);
  }
  const float nx = sqrtf(ss * (1.0f + 0x1p-16f)) * (1.0f + 0x1p-20f);
  float lsh = 0.0f;   // the shared expert's gate logit
  if (a.has_shared) {
    float sh[1];
    canon_dots_regs<NG, 1>(xr, wsh, H, sh);
    lsh = bf16r(sh[0]);
  }
  const float sqh = sqrtf((float)H) * 1.001f;
  // relative bound of |canonical - MFMA| per |x| |r| (see the top of the file)
  const float rel = (130.0f + (float)(H / 32) + 8.0f * (float)((H + 511) / 512)) * 0x1p-24f * 1.01f;
  // logit intervals
  float lo[EPL], hi[EPL];
  bool ok = true;
#pragma unroll
  for (int j = 0; j < EPL; j++) {
    const bool real = lane + 64 * j < E;
    float eps = rel * nx * nw[j];
    eps = eps + HX_RM_ABS * (sqh * (nx + nw[j]) + 3.0f * (float)H);
    eps = eps * (1.0f + 0x1p-20f) + fabsf(mv[j]) * 0x1p-22f;   // covers the rounding of m -/+ eps
    const float l0 = bf16r(mv[j] - eps) + bv[j], h0 = bf16r(mv[j] + eps) + bv[j];
    ok = ok && (!real || (__builtin_isfinite(l0) && __builtin_isfinite(h0)));
    lo[j] = real ? l0 : -__builtin_inff();
    hi[j] = real ? h0 : -__builtin_inff();
  }
  ok = __all(ok);
  int nc = 0;
  float hx_nc = -__builtin_inff();   // largest hi among the experts that are not candidates
  if (ok) {
    // tau: the k-th largest lane head (the largest lo of each lane), <= the
    // k-th largest lo: the lanes whose head has fewer than k larger heads are at
    // least k, and tau is the smallest of their heads
    float hd = -__builtin_inff();
#pragma unroll
    for (int j = 0; j < EPL; j++) hd = fmaxf(hd, lo[j]);
    int above = 0;
#pragma unroll
    for (int l2 = 0; l2 < 64; l2++)
      above += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(hd), l2)) > hd ? 1 : 0;
    const float tau = -wave_max_dpp(above < k ? -hd : -__builtin_inff());
    // candidates into LDS (any order); the largest excluded hi
#pragma unroll
    for (int j = 0; j < EPL; j++) {
      const int e = lane + 64 * j;
      const bool c = e < E && hi[j] >= tau;
      const unsigned long long bal = __ballot(c);
      const int pos = nc + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
      if (c && pos < 64) {
        sm.ce[wave][pos] = e;
        sm.cl[wave][pos] = lo[j] == hi[j] ? lo[j] : __builtin_nanf("");
      }
      nc += __popcll(bal);
      if (e < E && !c) hx_nc = fmaxf(hx_nc, hi[j]);
    }
    hx_nc = wave_max_dpp(hx_nc);
    ok = nc <= 64;
  }
  __builtin_amdgcn_wave_barrier();
  if (ok) {
    // exact logits of the ambiguous candidates
    const float my_l = lane < nc ? sm.cl[wave][lane] : 0.0f;
    unsigned long long amb = __ballot(lane < nc && my_l != my_l);
    while (amb) {
      int rows[4], idx[4];
#pragma unroll
      for (int b = 0; b < 4; b++) {
        if (amb) {
          const int i = __ffsll((long long)amb) - 1;
          amb &= amb - 1;
          rows[b] = sm.ce[wave][i];
          idx[b] = i;
        } else {
          rows[b] = E - 1;   // padding: computed and dropped
          idx[b] = -2;
        }
      }
      float s[4];
      canon_dots<NG, 4>(xr, R, H, rows, s);
#pragma unroll
      for (int b = 0; b < 4; b++) {
        const float v = bf16r(s[b]);
        if (idx[b] >= 0 && lane == 0) sm.cl[wave][idx[b]] = v + (a.bias ? a.bias[rows[b]] : 0.0f);
      }
    }
  }
  __builtin_amdgcn_wave_barrier();
  int out_e = 0;
  float out_w = 0.0f;
  if (ok) {
    // rank the candidates by (logit desc, id asc)
    const float li = lane < nc ? sm.cl[wave][lane] : -__builtin_inff();
    const int ei = lane < nc ? sm.ce[wave][lane] : 0x7fffffff;
    int rank = 0;
    for (int j = 0; j < nc; j++) {   // wave-uniform j: readlane, not a permute through LDS
      const float lj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(li), j));
      const int ej = __builtin_amdgcn_readlane(ei, j);
      rank += (lj > li || (lj == li && ej < ei)) ? 1 : 0;
    }
    if (lane < nc) {
      sm.sl[wave][rank] = li;
      sm.se[wave][rank] = ei;
    }
    __builtin_amdgcn_wave_barrier();
    const float lmax = sm.sl[wave][0];
    // positions 0 .. k: the selected ones and the best excluded candidate
    const float lr = lane <= k && lane < nc ? sm.sl[wave][lane] : -__builtin_inff();
    const int er = lane < nc ? sm.se[wave][min(lane, nc - 1)] : 0;
    const float xr_ = lr - lmax;
    const float ex = expf_route(xr_);
    const float ex_next = __shfl(ex, min(lane + 1, 63), 64);
    const float lr_next = __shfl(lr, min(lane + 1, 63), 64);
    bool good = true;
    if (lane < k) {
      good = ex >= 0x1p-100f;
      // the next position: a selected one (lane + 1 < k) or the best excluded candidate
      if (lane + 1 < nc && lane + 1 <= k && lr_next != lr) good = good && ex >= ex_next * (1.0f + 0x1p-20f);
      // the excluded experts that are not candidates (logits <= hx_nc < tau)
      if (lane == k - 1 && nc < E && hx_nc > -__builtin_inff())
        good = good && ex >= expf_route(hx_nc - lmax) * (1.0f + 0x1p-20f);
    }
    ok = __all(good);
    if (ok) {
      float tot = 0.0f;
      for (int r = 0; r < k; r++) tot = tot + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ex), r));
      out_e = er;
      out_w = ex / tot;
    }
  }
  if (!ok) {
    // the exact path: every canonical logit, then the reference softmax / top-k
    float v[EPL];
#pragma unroll
    for (int j = 0; j < EPL; j++) v[j] = -__builtin_inff();
#pragma unroll
    for (int j = 0; j < EPL; j++) {
      for (int l0 = 0; l0 < 64; l0 += 4) {
        if (64 * j + l0 >= E) break;
        int rows[4];
#pragma unroll
        for (int b = 0; b < 4; b++) rows[b] = min(64 * j + l0 + b, E - 1);
        float s[4];
        canon_dots<NG, 4>(xr, R, H, rows, s);
#pragma unroll
        for (int b = 0; b < 4; b++) {
          const int e = 64 * j + l0 + b;
          const float vv = bf16r(s[b]) + (a.bias ? a.bias[rows[b]] : 0.0f);
          if (lane == l0 + b && e < E) v[j] = vv;
        }
      }
    }
    const float mx = route_logits_max<EPL>(v);
    route_token_regs<EPL>(v, mx, k, a.norm, out_e, out_w);
  }
  if (lane < k) {
    const int64_t f = (int64_t)t * k + lane;
    a.d.topk_idx[f] = out_e;
    a.topk_w[f] = out_w;
    // the dispatch histogram of token t's chunk and t's bit of its expert in
    // the bitmap (both cleared by k_router_mfma)
    if (a.d.hist) {
      atomicAdd(&a.d.hist[(int64_t)(t / HX_DISPATCH_TOK) * E + out_e], 1);
      atomicOr(&a.d.bits[(int64_t)(t >> 5) * E + out_e], 1u << (t & 31));
    }
  }
  if (a.has_shared && lane == 0) a.sgw[t] = sigmoidf_(lsh);
}

// router row norms from above: |r_e| in double, rounded up to f32
__global__ __launch_bounds__(256) void k_row_norms(const uint16_t* R, int E1, int H, float* out) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = lane_id();
  if (row >= E1) return;
  double s = 0.0;
  for (int h = lane; h < H; h += 64) {
    const double v = (double)bf16_to_f32(R[(int64_t)row * H + h]);
    s += v * v;
  }
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
  if (lane == 0) out[row] = __double2float_ru(sqrt(s) * (1.0 + 0x1p-40));
}

// gfx950: the device is gfx950, whose v_mfma_f32_16x16x32_f16 accumulation
// the logit error bound (alpha) was measured on; any other target is refused
bool route_mfma_ok(const RouterArgs& a, bool xbf, bool rbf, bool gfx950) {
  const int ngr = a.H / (32 * RM_GROUP);   // accumulation groups of 128 (two K steps of 64)
  const bool shape = a.H % (32 * RM_GROUP) == 0 &&
                     (ngr == 1 || ngr == 2 || ngr == 3 || ngr == 4 || ngr == 6 || ngr == 8 || ngr == 12 ||
                      ngr == 16 || ngr == 24 || ngr == 32);
  return gfx950 && shape && xbf && rbf && a.rnorm && a.norm && a.T > HX_DECODE_MAX_T && a.H <= 4096 &&
         a.E >= 1 && a.E <= 1024 && a.k >= 1 && a.k <= 64 && a.k <= a.E;
}

// K splits of the MFMA router (logit planes): the fewest of 1, 2, 4 ..
// HX_RM_SPLITS that gives at least 512 workgroups (two per CU), among the
// splits whose K steps of 64 divide into that many runs of at least 4 and
// whose planes 1.. fit in front of the shared expert's rows of the
// weighted-rows buffer (row F of bf16 rows of H: 2 k H bytes per token).
// Measured on MI355X (E = 512, H = 2048): 512 tokens take 4 planes (256
// workgroups; 2 planes were 3.6 us slower), 2048 tokens 2 (router + routing
// 32.1 -> 30.6 us against 4), 4096 tokens 1 (56.4 -> 51.0 us); more
// planes add plane traffic to both kernels, fewer leave CUs idle.
int route_mfma_splits(const RouterArgs& a) {
  const int nst = a.H / 64;
  const int64_t nwg1 = (int64_t)((a.E + 63) / 64) * (((a.T + 63) / 64 + 7) / 8 * 8);
  auto ok = [&](int S) {
    return S == 1 || (nst % S == 0 && nst >= 4 * S && a.mplanes &&
                      (int64_t)4 * (S - 1) * a.E1 <= (int64_t)2 * a.k * a.H);
  };
  int best = 1;
  for (int S = 1; S <= HX_RM_SPLITS; S *= 2) {
    if (!ok(S)) break;
    best = S;
    if (nwg1 * S >= 512) break;
  }
  return best;
}

hipError_t launch_router_mfma(const RouterArgs& a, uint16_t* xh, bool xnat, hipStream_t s) {
  int32_t* dmap = a.d.hist;
  const int ndmap = dmap ? (dispatch_chunks(a.T) + dispatch_words(a.T)) * a.E : 0;
  const int S = route_mfma_splits(a), nsw = a.H / 64 / S;
  const int NX = (a.E + 63) / 64;
  const dim3 grid(NX, ((a.T + 63) / 64 + 7) / 8 * 8, S);
#define RM(N)                                                                                                    \
  case N:                                                                                                        \
    hx_launch(k_router_mfma<N>, grid, dim3(256), 0, s, (const uint16_t*)a.x, (const uint16_t*)a.R, a.T, a.H, a.E, \
              a.E1, a.logits, a.mplanes, xh, xnat ? 1 : 0, dmap, ndmap);                                         \
    break;
  switch (nsw) {   // steps per workgroup: every size route_mfma_ok admits, split or not
    RM(2) RM(4) RM(6) RM(8) RM(12) RM(16) RM(24) RM(32) RM(48) RM(64)
    default: return hipErrorInvalidValue;   // route_mfma_ok admits only the sizes above
  }
#undef RM
  return hipGetLastError();
}

template <int EPL>
static void route_mfma_ng(const RouterArgs& a0, hipStream_t s) {
  RouterArgs a = a0;
  a.msplit = route_mfma_splits(a);
  const dim3 g(((a.T + 63) / 64 + 7) / 8 * 8 * 16), b(256);   // 16 workgroups per token block of 64
  if (a.H <= 512) hx_launch(k_route_mfma<EPL, 1>, g, b, 0, s, a);
  else if (a.H <= 1024) hx_launch(k_route_mfma<EPL, 2>, g, b, 0, s, a);
  else if (a.H <= 2048) hx_launch(k_route_mfma<EPL, 4>, g, b, 0, s, a);
  else hx_launch(k_route_mfma<EPL, 8>, g, b, 0, s, a);
}

void launch_route_mfma(const RouterArgs& a, hipStream_t s) {
  if (a.E <= 64) route_mfma_ng<1>(a, s);
  else if (a.E <= 128) route_mfma_ng<2>(a, s);
  else if (a.E <= 256) route_mfma_ng<4>(a, s);
  else if (a.E <= 512) route_mfma_ng<8>(a, s);
  else route_mfma_ng<16>(a, s);
}

hipError_t launch_row_norms(const void* R, int E1, int H, float* out, hipStream_t s) {
  hipLaunchKernelGGL(k_row_norms, dim3((E1 + 3) / 4), dim3(256), 0, s, (const uint16_t*)R, E1, H, out);
  return hipGetLastError();
}

}  // namespace hx
