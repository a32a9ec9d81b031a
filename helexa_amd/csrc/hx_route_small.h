// Routing of a few tokens (T <= HX_DECODE_MAX_T) inside one workgroup, all in
// LDS: softmax / top-k / renormalisation per token and the stable dispatch
// permutation. Decode kernels run it as a prologue (every workgroup computes
// the same routing from the router logits, so no separate routing kernel and
// no cross-workgroup synchronisation is needed); one workgroup publishes the
// result to global memory.
//
// Reference: route_scatter (crates/neuron/src/harness/arch/qwen3_5/moe.rs:124-162),
// dispatch sort (crates/neuron/src/harness/tp/tp_qwen3_5.rs:1189).
#pragma once
#include "hx_internal.h"

namespace hx {

constexpr int HX_SMALL_F = HX_DECODE_MAX_T * HX_MAX_TOPK;

constexpr int HX_SMALL_W = HX_MAX_EXPERTS / 64;   // expert-mask words
struct alignas(16) RouteSmem {
  unsigned long long emask[HX_DECODE_MAX_T][HX_SMALL_W];   // token t's experts: bit e % 64 of word e / 64
  unsigned long long wuni[HX_SMALL_W];   // the union over the tokens
  int wpre[HX_SMALL_W];                  // entries in the words below, over the tokens
  int upre[HX_SMALL_W];                  // distinct experts in the words below
  int idx[HX_SMALL_F];       // expert of flat entry f = t*k + j
  float w[HX_SMALL_F];       // routing weight of entry f
  int pos[HX_SMALL_F];       // permuted position of entry f
  int perm[HX_SMALL_F];      // entry at permuted position p
  uint8_t first[HX_SMALL_F]; // entry f is its expert's first
  int slots[3 * HX_SMALL_F]; // routed slot u: expert, start, count
  float sgw[HX_DECODE_MAX_T];
  int nroute;
};
// the dispatch reads perm four ints at a time
static_assert(offsetof(RouteSmem, perm) % 16 == 0 && HX_SMALL_F % 4 == 0, "RouteSmem.perm alignment");

// Descending sort of one lane's EPL keys (hi = probability bits, lo = ~expert):
// comparing (hi, lo) as one 64-bit value orders by probability, then by lower
// expert id. Sorting networks: Batcher's odd-even merge sort for 8, bitonic
// otherwise.
HX_DEV void key_cas(uint32_t& ah, uint32_t& al, uint32_t& bh, uint32_t& bl) {
  const uint64_t a = ((uint64_t)ah << 32) | al, b = ((uint64_t)bh << 32) | bl;
  const bool sw = b > a;
  const uint32_t th = sw ? bh : ah, tl = sw ? bl : al;
  bh = sw ? ah : bh;
  bl = sw ? al : bl;
  ah = th;
  al = tl;
}

template <int EPL>
HX_DEV void sort_keys_desc(uint32_t* h, uint32_t* l) {
  if (EPL == 8) {
    constexpr int P[19][2] = {{0, 1}, {2, 3}, {4, 5}, {6, 7}, {0, 2}, {1, 3}, {4, 6}, {5, 7}, {1, 2}, {5, 6},
                              {0, 4}, {1, 5}, {2, 6}, {3, 7}, {2, 4}, {3, 5}, {1, 2}, {3, 4}, {5, 6}};
#pragma unroll
    for (int c = 0; c < 19; c++) key_cas(h[P[c][0]], l[P[c][0]], h[P[c][1]], l[P[c][1]]);
    return;
  }
#pragma unroll
  for (int kk = 2; kk <= EPL; kk *= 2)
#pragma unroll
    for (int jj = kk / 2; jj > 0; jj /= 2)
#pragma unroll
      for (int i = 0; i < EPL; i++) {
        const int q = i ^ jj;
        if (q > i) {
          if ((i & kk) == 0) key_cas(h[i], l[i], h[q], l[q]);
          else key_cas(h[q], l[q], h[i], l[i]);
        }
      }
}

// this lane's logits (expert lane + 64 j; padding -inf)
template <int EPL>
HX_DEV void route_logits_load(const float* lg, int E, float* v) {
  const int lane = lane_id();
#pragma unroll
  for (int j = 0; j < EPL; j++) {
    const int e = lane + 64 * j;
    const float x = lg[e < E ? e : E - 1];
    v[j] = e < E ? x : -__builtin_inff();
  }
}
// the wave-wide max of the loaded logits
template <int EPL>
HX_DEV float route_logits_max(const float* v) {
  float mx = -__builtin_inff();
#pragma unroll
  for (int j = 0; j < EPL; j++) mx = v[j] > mx ? v[j] : mx;
  return wave_max_dpp(mx);
}
template <int EPL>
HX_DEV float route_logits(const float* lg, int E, float* v) {
  route_logits_load<EPL>(lg, E, v);
  return route_logits_max<EPL>(v);
}

// the lowest expert id whose logit is the maximum (wave-uniform; -1 if none):
// rank 0 of the routing unless rounding gives a smaller logit the same
// probability, so a caller may start work on it before the softmax
template <int EPL>
HX_DEV int route_argmax(const float* v, float mx, int E) {
  const int lane = lane_id();
  uint32_t cand = 0u;   // ~id of this lane's lowest id holding mx
#pragma unroll
  for (int j = EPL - 1; j >= 0; j--)
    cand = v[j] == mx && lane + 64 * j < E ? ~(uint32_t)(lane + 64 * j) : cand;
  return (int)~wave_max_u32(cand);
}

// softmax over the E logits of a token and this lane's keys, sorted
template <int EPL>
HX_DEV void route_keys_from(float* v, float mx, uint32_t* h, uint32_t* l) {
  const int lane = lane_id();
#pragma unroll
  for (int j = 0; j < EPL; j++) v[j] = v[j] - mx;
  expf_route_n<EPL>(v);   // padding: exp(-inf) = 0
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < EPL; j++) s = s + v[j];
  s = wave_sum<64>(s);
#pragma unroll
  for (int j = 0; j < EPL; j++) {
    h[j] = __float_as_uint(v[j] / s);   // padding: 0 / s = +0
    l[j] = ~(uint32_t)(lane + 64 * j);
  }
  sort_keys_desc<EPL>(h, l);
}
template <int EPL>
HX_DEV void route_keys(const float* lg, int E, uint32_t* h, uint32_t* l) {
  float v[EPL];
  const float mx = route_logits<EPL>(lg, E, v);
  route_keys_from<EPL>(v, mx, h, l);
}

// One selection round: the wave-wide largest head probability m; when several
// heads hold it, the lowest expert id among them. Returns that expert (wave-
// uniform) and its probability bits in m; pops it. The rest of the previous
// pop's shift (pend) is applied alongside the reduction.
template <int EPL>
HX_DEV int route_round(uint32_t* h, uint32_t* l, uint32_t& pend, uint32_t& m) {
  uint32_t x = h[0];
  x = max(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0xB1, 0xf, 0xf, false));
#pragma unroll
  for (int j = 1; j + 1 < EPL; j++) h[j] = (h[j] & ~pend) | (h[j + 1] & pend);
  x = max(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x4E, 0xf, 0xf, false));
  if (EPL > 1) h[EPL - 1] &= ~pend;
  x = max(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x141, 0xf, 0xf, false));
#pragma unroll
  for (int j = 0; j + 1 < EPL; j++) l[j] = (l[j] & ~pend) | (l[j + 1] & pend);
  x = max(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x140, 0xf, 0xf, false));
  l[EPL - 1] &= ~pend;
  x = max(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x142, 0xa, 0xf, false));
  x = max(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x143, 0xc, 0xf, false));
  m = (uint32_t)__builtin_amdgcn_readlane((int)x, 63);
  bool hit = h[0] == m;
  unsigned long long hold = __ballot(hit);
  if (hold & (hold - 1)) {   // several heads hold m: the lowest expert id goes first
    const uint32_t lo = wave_max_u32(hit ? l[0] : 0u);
    hit = hit && l[0] == lo;
    hold = __ballot(hit);
  }
  pend = hit ? 0xffffffffu : 0u;
  const int e = (int)~(uint32_t)__builtin_amdgcn_readlane((int)l[0], __ffsll((long long)hold) - 1);
  h[0] = EPL > 1 ? ((h[0] & ~pend) | (h[1] & pend)) : (h[0] & ~pend);
  return e;
}

// One wave routes one token: softmax over E with expf_route and the
// lane-strided butterfly sum, then the k largest probabilities, ties to the
// lowest expert id, and the sequential renormalisation in rank order. Lane
// j < k returns rank j's (expert, weight).
//
// Selection: expert e lives in lane e % 64; each lane sorts its EPL keys
// (probability bits, ~e) in descending order once (so a lane's equal
// probabilities are ordered by expert id, and its head is its best entry).
// Probabilities are >= 0, so their bit patterns order like the values; padding
// (e >= E) has key (0, ~e). Round r takes the wave-wide largest head
// probability m (one DPP reduction). When one lane holds m, its head is rank r.
// When several do (equal probabilities are common: the logits are rounded to
// the activation dtype), the next entry in rank order is the lowest expert id
// among their heads -- every lane's lowest id of probability m is its head --
// found by a second reduction over ~e; that branch is wave-uniform. Only the
// chosen lane pops. The pop is split: the head is replaced at once (the next
// reduction needs it); the rest of the shift is applied during the next
// round's reduction, which does not depend on it.
// v: this lane's logits (expert lane + 64 j in v[j], padding -inf); mx: their
// wave-wide maximum.
template <int EPL>
HX_DEV void route_token_regs(float* v, float mx, int k, bool norm, int& out_e, float& out_w) {
  const int lane = lane_id();
  uint32_t h[EPL], l[EPL];
  route_keys_from<EPL>(v, mx, h, l);
  float my_p = 0.0f, tot = 0.0f;
  int my_e = 0;
  uint32_t pend = 0u;   // all-ones in the lane popped by the previous round
  for (int r = 0; r < k; r++) {
    uint32_t m;
    const int e = route_round<EPL>(h, l, pend, m);
    const float pm = __uint_as_float(m);
    tot = tot + pm;
    my_p = lane == r ? pm : my_p;
    my_e = lane == r ? e : my_e;
  }
  out_e = my_e;
  out_w = norm ? my_p / tot : my_p;
}

// the same from the token's logits row lg (E values) in memory
template <int EPL>
HX_DEV void route_token_core(const float* lg, int E, int k, bool norm, int& out_e, float& out_w) {
  float v[EPL];
  const float mx = route_logits<EPL>(lg, E, v);
  route_token_regs<EPL>(v, mx, k, norm, out_e, out_w);
}

// route_token_core with K rounds unrolled and hook(r, e) called right after
// round r picks expert e (wave-uniform), so a caller can start loading that
// expert's weights while the later rounds run; before the softmax, hook(-1 - s,
// e) for s < SPEC with the expert of the s-th largest logit. v: this lane's
// logits from route_logits_load (the caller issues those loads first, so that
// waiting for them does not wait for its other loads).
template <int EPL, int K, int SPEC, class Hook>
HX_DEV void route_token_core_hook(float* v, int E, bool norm, int& out_e, float& out_w, Hook&& hook) {
  const int lane = lane_id();
  uint32_t h[EPL], l[EPL];
  {
    // hook(-1 - s, e), s < SPEC: the likely rank-s expert (the s-th largest
    // logit, lowest id first), as soon as the logits are in
    const float mx = route_logits_max<EPL>(v);
    int e = route_argmax<EPL>(v, mx, E);
    hook(-1, e);
    if constexpr (SPEC > 1) {
      float w[EPL];
#pragma unroll
      for (int j = 0; j < EPL; j++) w[j] = v[j];
#pragma unroll
      for (int sp = 1; sp < SPEC; sp++) {
#pragma unroll
        for (int j = 0; j < EPL; j++) w[j] = lane + 64 * j == e ? -__builtin_inff() : w[j];
        e = route_argmax<EPL>(w, route_logits_max<EPL>(w), E);
        hook(-1 - sp, e);
      }
    }
    route_keys_from<EPL>(v, mx, h, l);
  }
  float my_p = 0.0f, tot = 0.0f;
  int my_e = 0;
  uint32_t pend = 0u;
#pragma unroll
  for (int r = 0; r < K; r++) {
    uint32_t m;
    const int e = route_round<EPL>(h, l, pend, m);
    hook(r, e);
    const float pm = __uint_as_float(m);
    tot = tot + pm;
    my_p = lane == r ? pm : my_p;
    my_e = lane == r ? e : my_e;
  }
  out_e = my_e;
  out_w = norm ? my_p / tot : my_p;
}

// a value loaded early and used late: the empty asm keeps the compiler from
// starting its arithmetic (and so waiting for its load) where it is loaded
HX_DEV float sg_late(float v) {
  asm volatile("" : "+v"(v));
  return v;
}

template <int EPL>
HX_DEV void route_token_lds_t(const float* lg, int E, int k, bool norm, bool want_sgw, int t, RouteSmem& sm) {
  // the shared gate's logit, issued with the logits (no branch around the
  // load) and used at the end (sg_late: its sigmoid is not started at the load)
  const float sg = lg[want_sgw ? E : 0];
  int e;
  float w;
  route_token_core<EPL>(lg, E, k, norm, e, w);
  const int lane = lane_id();
  if (lane < k) {
    sm.idx[t * k + lane] = e;
    sm.w[t * k + lane] = w;
  }
  if (lane == 0) sm.sgw[t] = want_sgw ? sigmoidf_(sg_late(sg)) : 0.0f;
  // the token's expert mask: cleared, then one bit per selected expert (the
  // wave's LDS operations take effect in program order)
  if (lane < HX_SMALL_W) sm.emask[t][lane] = 0ull;
  if (lane < k) atomicOr(&sm.emask[t][e >> 6], 1ull << (e & 63));
}

// One token in wave 0 of the workgroup, dispatch included: the k experts of a
// token are distinct, so expert-sorted position = rank of the expert id, every
// entry starts its own slot, and slot = position.
template <int EPL>
HX_DEV void route_one_token(const float* lg, int E, int k, bool norm, bool want_sgw, RouteSmem& sm) {
  const float sg = lg[want_sgw ? E : 0];   // as in route_token_lds_t
  int e;
  float w;
  route_token_core<EPL>(lg, E, k, norm, e, w);
  const int lane = lane_id();
  int pos = 0;
  for (int j = 0; j < k; j++) pos += __builtin_amdgcn_readlane(e, j) < e;
  if (lane < k) {
    sm.idx[lane] = e;
    sm.w[lane] = w;
    sm.pos[lane] = pos;
    sm.perm[pos] = lane;
    sm.first[lane] = 1;
    sm.slots[3 * pos + 0] = e;
    sm.slots[3 * pos + 1] = pos;
    sm.slots[3 * pos + 2] = 1;
  }
  if (lane == 0) {
    sm.sgw[0] = want_sgw ? sigmoidf_(sg_late(sg)) : 0.0f;
    sm.nroute = k;
  }
}

HX_DEV void route_token_lds(const float* lg, int E, int k, bool norm, bool want_sgw, int t, RouteSmem& sm) {
  if (E <= 64) route_token_lds_t<1>(lg, E, k, norm, want_sgw, t, sm);
  else if (E <= 128) route_token_lds_t<2>(lg, E, k, norm, want_sgw, t, sm);
  else if (E <= 256) route_token_lds_t<4>(lg, E, k, norm, want_sgw, t, sm);
  else if (E <= 512) route_token_lds_t<8>(lg, E, k, norm, want_sgw, t, sm);
  else route_token_lds_t<16>(lg, E, k, norm, want_sgw, t, sm);
}

HX_DEV void route_one_token_lds(const float* lg, int E, int k, bool norm, bool want_sgw, RouteSmem& sm) {
  if (E <= 64) route_one_token<1>(lg, E, k, norm, want_sgw, sm);
  else if (E <= 128) route_one_token<2>(lg, E, k, norm, want_sgw, sm);
  else if (E <= 256) route_one_token<4>(lg, E, k, norm, want_sgw, sm);
  else if (E <= 512) route_one_token<8>(lg, E, k, norm, want_sgw, sm);
  else route_one_token<16>(lg, E, k, norm, want_sgw, sm);
}

// threads of the k_route_small workgroup for T tokens (one wave a token, at
// least four waves)
__host__ __device__ inline int route_small_threads(int T) { return T > 4 ? 512 : 256; }

// Full routing of T tokens from logits [T][E1] into RouteSmem; ends with a
// barrier. The shared-expert gate sigmoid is computed only when want_sgw.
// nt: the workgroup's threads (blockDim.x), passed in: read from the
// kernel's hidden arguments it cost a scalar round trip ahead of the logits
HX_DEV void route_small_lds(const float* logits, int E1, int E, int k, bool norm, bool want_sgw, int T,
                            RouteSmem& sm, int nt) {
  const int tid = threadIdx.x, wave = tid >> 6;
  const int F = T * k;
  if (T == 1) {
    if (wave == 0) route_one_token_lds(logits, E, k, norm, want_sgw, sm);
    __syncthreads();
    return;
  }
  const int nw = nt >> 6;
  for (int t = wave; t < T; t += nw) route_token_lds(logits + (int64_t)t * E1, E, k, norm, want_sgw, t, sm);
  __syncthreads();
  // dispatch from the tokens' expert masks (a token's k experts are distinct):
  // entry f = (token t, expert e) goes to position pos = (entries with a
  // smaller expert) + (tokens before t that also chose e) -- the stable sort
  // by (expert, f); expert e's slot is the number of distinct experts below
  // it, starting at the position of its first entry, with one row per token
  // that chose it
  static_assert(HX_SMALL_W <= 16, "the word scan runs in one row of 16 lanes");
  if (wave == 0) {
    // lane q < 16: word q's union and entry count, then exclusive prefix sums
    // over the words (inclusive scans along row 0 by DPP row_shr)
    const int q = tid, NWD = (E + 63) >> 6;
    unsigned long long u = 0ull;
    int c = 0;
#pragma unroll
    for (int t = 0; t < HX_DECODE_MAX_T; t++) {
      const unsigned long long m = q < NWD && t < T ? sm.emask[t][q] : 0ull;
      u |= m;
      c += __popcll(m);
    }
    const int cu = __popcll(u);
    int ic = c, iu = cu;
#define HX_SCAN(CTRL)                                                       \
    ic += __builtin_amdgcn_update_dpp(0, ic, CTRL, 0xf, 0xf, true);         \
    iu += __builtin_amdgcn_update_dpp(0, iu, CTRL, 0xf, 0xf, true);
    HX_SCAN(0x111) HX_SCAN(0x112) HX_SCAN(0x114) HX_SCAN(0x118)
#undef HX_SCAN
    if (q < HX_SMALL_W) {
      sm.wuni[q] = u;
      sm.wpre[q] = ic - c;
      sm.upre[q] = iu - cu;
    }
    if (q == 15) sm.nroute = iu;
  }
  __syncthreads();
  for (int f = tid; f < F; f += nt) {
    const int t = f / k, e = sm.idx[f], wd = e >> 6, b = e & 63;
    const unsigned long long below = (1ull << b) - 1ull;
    int less = sm.wpre[wd], before = 0, cnt = 0;
    const int slot = sm.upre[wd] + __popcll(sm.wuni[wd] & below);
#pragma unroll
    for (int u = 0; u < HX_DECODE_MAX_T; u++) {
      const unsigned long long m = u < T ? sm.emask[u][wd] : 0ull;
      const int bit = (int)((m >> b) & 1ull);
      less += __popcll(m & below);
      cnt += bit;
      before += u < t ? bit : 0;
    }
    const int pos = less + before;
    sm.pos[f] = pos;
    sm.perm[pos] = f;
    sm.first[f] = before == 0;
    if (before == 0) {
      sm.slots[3 * slot + 0] = e;
      sm.slots[3 * slot + 1] = pos;
      sm.slots[3 * slot + 2] = cnt;
    }
  }
  __syncthreads();
}

// write the routing (and the decode plan) of RouteSmem to global memory; with
// d.plan_only the decode plan and nothing else
HX_DEV void publish_route(const DispatchArgs& d, float* topk_w, float* sgw, const RouteSmem& sm) {
  const int tid = threadIdx.x, nt = blockDim.x, F = d.F, T = d.T, E = d.E;
  const bool all = !d.plan_only;
  const int ns = sm.nroute + (d.has_shared ? 1 : 0);
  const int tok0 = 4 + 4 * d.max_slots, w0 = tok0 + F + T, e0 = w0 + F + T;
  for (int f = tid; f < F; f += nt) {
    const int p = sm.pos[f];
    if (all) {
      d.topk_idx[f] = sm.idx[f];
      topk_w[f] = sm.w[f];
      d.perm[p] = f;
      if (d.inv) d.inv[f] = p;
    }
    d.plan[tok0 + p] = f / d.k;
    d.plan[w0 + p] = __float_as_int(sm.w[f]);
    d.plan[e0 + p] = sm.idx[f];
  }
  for (int t = tid; t < T; t += nt) {
    if (all) sgw[t] = sm.sgw[t];
    d.plan[tok0 + F + t] = t;
    d.plan[w0 + F + t] = __float_as_int(sm.sgw[t]);
    d.plan[e0 + F + t] = E;
  }
  for (int u = tid; u < sm.nroute; u += nt) {
#pragma unroll
    for (int q = 0; q < 3; q++) {
      if (all) d.slots[3 * u + q] = sm.slots[3 * u + q];
      d.plan[4 + 4 * u + q] = sm.slots[3 * u + q];
    }
    d.plan[4 + 4 * u + 3] = sm.perm[sm.slots[3 * u + 1]] / d.k;   // token of the slot's first row
  }
  if (all) {
    // offsets[e] = number of entries routed to experts below e = start of the
    // first slot whose expert is >= e (F if none): binary search of the slots,
    // which are in ascending expert order
    for (int e = tid; e <= E; e += nt) {
      int lo = 0, hi = sm.nroute;
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (sm.slots[3 * mid] < e) lo = mid + 1;
        else hi = mid;
      }
      d.offsets[e] = lo < sm.nroute ? sm.slots[3 * lo + 1] : F;
    }
  }
  if (tid == 0) {
    if (d.has_shared) {
      const int u = sm.nroute;
      if (all) {
        d.slots[3 * u + 0] = E;
        d.slots[3 * u + 1] = F;
        d.slots[3 * u + 2] = T;
      }
      d.plan[4 + 4 * u + 0] = E;
      d.plan[4 + 4 * u + 1] = F;
      d.plan[4 + 4 * u + 2] = T;
      d.plan[4 + 4 * u + 3] = 0;
    }
    if (all) {
      d.counts[0] = ns;
      d.counts[1] = 0;
    }
    d.plan[0] = ns;
  }
}

}  // namespace hx
