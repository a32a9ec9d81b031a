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

struct RouteSmem {
  int idx[HX_SMALL_F];       // expert of flat entry f = t*k + j
  float w[HX_SMALL_F];       // routing weight of entry f
  int pos[HX_SMALL_F];       // permuted position of entry f
  int perm[HX_SMALL_F];      // entry at permuted position p
  uint8_t first[HX_SMALL_F]; // entry f is its expert's first
  int slots[3 * HX_SMALL_F]; // routed slot u: expert, start, count
  float sgw[HX_DECODE_MAX_T];
  int nroute;
};

// One wave routes one token: softmax over E with expf_route and the
// lane-strided butterfly sum, then k rounds of selection -- the largest
// probability not yet taken, ties to the lowest expert id (a DPP max of the
// per-lane best, then a DPP min of the ids holding it) -- and the sequential
// renormalisation in rank order. Lane j < k returns rank j's (expert, weight).
template <int EPL>
HX_DEV void route_token_core(const float* lg, int E, int k, bool norm, int& out_e, float& out_w) {
  const int lane = lane_id();
  float v[EPL];
  float mx = -__builtin_inff();
#pragma unroll
  for (int j = 0; j < EPL; j++) {
    const int e = lane + 64 * j;
    v[j] = e < E ? lg[e] : -__builtin_inff();
    mx = v[j] > mx ? v[j] : mx;
  }
  mx = wave_max_dpp(mx);
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < EPL; j++) {
    if (lane + 64 * j < E) {
      v[j] = expf_route(v[j] - mx);
      s = s + v[j];
    }
  }
  s = wave_sum<64>(s);
#pragma unroll
  for (int j = 0; j < EPL; j++) v[j] = lane + 64 * j < E ? v[j] / s : -1.0f;
  float my_p = 0.0f, tot = 0.0f;
  int my_e = 0;
  uint32_t taken = 0;
  for (int r = 0; r < k; r++) {
    float bm = -2.0f;
    int bj = 0;
#pragma unroll
    for (int j = 0; j < EPL; j++)
      if (!((taken >> j) & 1u) && v[j] > bm) {
        bm = v[j];
        bj = j;
      }
    const float m = wave_max_dpp(bm);
    const unsigned long long holders = __ballot(bm == m);
    int e;
    if (__popcll(holders) == 1)   // the usual case: one lane holds the maximum
      e = __builtin_amdgcn_readlane(lane + 64 * bj, __ffsll((long long)holders) - 1);
    else                          // equal probabilities: the lowest expert id
      e = wave_min_dpp(bm == m ? lane + 64 * bj : 0x7fffffff);
    if ((e & 63) == lane) taken |= 1u << (e >> 6);
    tot = tot + m;
    if (lane == r) {
      my_p = m;
      my_e = e;
    }
  }
  out_e = my_e;
  out_w = norm ? my_p / tot : my_p;
}

template <int EPL>
HX_DEV void route_token_lds_t(const float* lg, int E, int k, bool norm, bool has_shared, int t, RouteSmem& sm) {
  int e;
  float w;
  route_token_core<EPL>(lg, E, k, norm, e, w);
  const int lane = lane_id();
  if (lane < k) {
    sm.idx[t * k + lane] = e;
    sm.w[t * k + lane] = w;
  }
  if (lane == 0) sm.sgw[t] = has_shared ? sigmoidf_(lg[E]) : 0.0f;
}

HX_DEV void route_token_lds(const float* lg, int E, int k, bool norm, bool has_shared, int t, RouteSmem& sm) {
  if (E <= 64) route_token_lds_t<1>(lg, E, k, norm, has_shared, t, sm);
  else if (E <= 128) route_token_lds_t<2>(lg, E, k, norm, has_shared, t, sm);
  else if (E <= 256) route_token_lds_t<4>(lg, E, k, norm, has_shared, t, sm);
  else if (E <= 512) route_token_lds_t<8>(lg, E, k, norm, has_shared, t, sm);
  else route_token_lds_t<16>(lg, E, k, norm, has_shared, t, sm);
}

// full routing of T tokens from logits [T][E1]; ends with a barrier
HX_DEV void route_small_lds(const float* logits, int E1, int E, int k, bool norm, bool has_shared, int T,
                            RouteSmem& sm) {
  const int tid = threadIdx.x, wave = tid >> 6;
  const int F = T * k;
  if (tid == 0) sm.nroute = 0;
  for (int t = wave; t < T; t += 4) route_token_lds(logits + (int64_t)t * E1, E, k, norm, has_shared, t, sm);
  __syncthreads();
  if (F <= 64) {
    // one wave: entry f in lane f, the other entries' experts via readlane
    if (wave == 0) {
      const int lane = lane_id();
      const int e = lane < F ? sm.idx[lane] : 0x7fffffff;
      int less = 0, before = 0;
      for (int j = 0; j < F; j++) {
        const int ej = __builtin_amdgcn_readlane(e, j);
        less += ej < e;
        before += (ej == e) & (j < lane);
      }
      const bool first = lane < F && before == 0;
      int slot = 0, count = 0;
      for (int j = 0; j < F; j++) {
        const int ej = __builtin_amdgcn_readlane(e, j);
        const int fj = __builtin_amdgcn_readlane((int)first, j);
        slot += fj & (ej < e);
        count += ej == e;
      }
      if (lane < F) {
        sm.pos[lane] = less + before;
        sm.perm[less + before] = lane;
        sm.first[lane] = first;
      }
      if (first) {
        sm.slots[3 * slot + 0] = e;
        sm.slots[3 * slot + 1] = less;
        sm.slots[3 * slot + 2] = count;
      }
      const int nfirst = __popcll(__ballot(first));
      if (lane == 0) sm.nroute = nfirst;
    }
    __syncthreads();
    return;
  }
  // stable sort by expert: pos(f) = #{e_j < e_f} + #{j < f, e_j == e_f}
  for (int f = tid; f < F; f += 256) {
    const int e = sm.idx[f];
    int less = 0, before = 0;
    for (int j = 0; j < F; j++) {
      const int ej = sm.idx[j];
      less += ej < e;
      before += (ej == e) & (j < f);
    }
    sm.pos[f] = less + before;
    sm.perm[less + before] = f;
    sm.first[f] = before == 0;
  }
  __syncthreads();
  for (int f = tid; f < F; f += 256) {
    if (!sm.first[f]) continue;
    const int e = sm.idx[f];
    int slot = 0, count = 0;
    for (int j = 0; j < F; j++) {
      const int ej = sm.idx[j];
      slot += sm.first[j] & (ej < e);
      count += ej == e;
    }
    sm.slots[3 * slot + 0] = e;
    sm.slots[3 * slot + 1] = sm.pos[f];
    sm.slots[3 * slot + 2] = count;
    atomicAdd(&sm.nroute, 1);
  }
  __syncthreads();
}

// write the routing (and the decode plan) of RouteSmem to global memory
HX_DEV void publish_route(const DispatchArgs& d, float* topk_w, float* sgw, const RouteSmem& sm) {
  const int tid = threadIdx.x, F = d.F, T = d.T, E = d.E;
  const int ns = sm.nroute + (d.has_shared ? 1 : 0);
  const int tok0 = 4 + 4 * d.max_slots, w0 = tok0 + F + T;
  for (int f = tid; f < F; f += 256) {
    const int p = sm.pos[f];
    d.topk_idx[f] = sm.idx[f];
    topk_w[f] = sm.w[f];
    d.perm[p] = f;
    if (d.inv) d.inv[f] = p;
    d.plan[tok0 + p] = f / d.k;
    d.plan[w0 + p] = __float_as_int(sm.w[f]);
  }
  for (int t = tid; t < T; t += 256) {
    sgw[t] = sm.sgw[t];
    d.plan[tok0 + F + t] = t;
    d.plan[w0 + F + t] = __float_as_int(sm.sgw[t]);
  }
  for (int u = tid; u < sm.nroute; u += 256) {
    for (int q = 0; q < 3; q++) {
      d.slots[3 * u + q] = sm.slots[3 * u + q];
      d.plan[4 + 4 * u + q] = sm.slots[3 * u + q];
    }
  }
  // offsets[e] = number of entries routed to experts below e
  for (int e = tid; e <= E; e += 256) {
    int less = 0;
    for (int j = 0; j < F; j++) less += sm.idx[j] < e;
    d.offsets[e] = less;
  }
  if (tid == 0) {
    if (d.has_shared) {
      const int u = sm.nroute;
      d.slots[3 * u + 0] = E;
      d.slots[3 * u + 1] = F;
      d.slots[3 * u + 2] = T;
      d.plan[4 + 4 * u + 0] = E;
      d.plan[4 + 4 * u + 1] = F;
      d.plan[4 + 4 * u + 2] = T;
    }
    d.counts[0] = ns;
    d.counts[1] = 0;
    d.plan[0] = ns;
  }
}

}  // namespace hx
