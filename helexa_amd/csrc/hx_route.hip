// Routing kernels: router logits, per-token softmax / top-k / renormalisation,
// and the stable dispatch permutation.
//
// Reference: route_scatter (crates/neuron/src/harness/arch/qwen3_5/moe.rs:124-162)
// and forward_fused's on-device routing + sort
// (crates/neuron/src/harness/tp/tp_qwen3_5.rs:1179-1189).
#include "hx_internal.h"

namespace hx {

// ----------------------------------------------------------------------------
// per-token routing: one wave per token.
// lg: logits row [E1] (E1 = E + has_shared; column E is the shared-expert gate)
// ----------------------------------------------------------------------------
HX_DEV void route_one_token(const float* lg, int E, int k, bool norm, bool has_shared, int t,
                            int32_t* topk_idx, float* topk_w, float* sgw) {
  const int lane = lane_id();
  constexpr int EPL = HX_MAX_EXPERTS / 64;
  float mx = -__builtin_inff();
  float v[EPL];
#pragma unroll
  for (int j = 0; j < EPL; j++) {
    int e = lane + 64 * j;
    v[j] = e < E ? lg[e] : -__builtin_inff();
    mx = v[j] > mx ? v[j] : mx;
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    float o = __shfl_xor(mx, off, 64);
    mx = o > mx ? o : mx;
  }
  // exp and the lane-strided sum (expert e -> lane e % 64, increasing e)
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < EPL; j++) {
    int e = lane + 64 * j;
    if (e < E) {
      v[j] = expf_route(v[j] - mx);
      s = s + v[j];
    }
  }
  s = wave_sum<64>(s);
  unsigned long long key[EPL];
#pragma unroll
  for (int j = 0; j < EPL; j++) {
    int e = lane + 64 * j;
    float p = v[j] / s;
    key[j] = e < E ? (((unsigned long long)__float_as_uint(p) << 32) | (unsigned long long)(0xffffffffu - (uint32_t)e))
                   : 0ull;
  }
  // k rounds of a wave arg-max; the key orders by probability, then lower id
  float my_p = 0.0f, tot = 0.0f;
  int my_e = 0;
  uint32_t taken = 0;
  for (int r = 0; r < k; r++) {
    unsigned long long best = 0ull;
#pragma unroll
    for (int j = 0; j < EPL; j++)
      if (!((taken >> j) & 1u) && key[j] > best) best = key[j];
    best = wave_max_u64(best);
    int e = (int)(0xffffffffu - (uint32_t)(best & 0xffffffffull));
    float p = __uint_as_float((uint32_t)(best >> 32));
    if ((e & 63) == lane) taken |= 1u << (e >> 6);
    tot = tot + p;
    if (lane == r) {
      my_p = p;
      my_e = e;
    }
  }
  if (lane < k) {
    topk_idx[(int64_t)t * k + lane] = my_e;
    topk_w[(int64_t)t * k + lane] = norm ? my_p / tot : my_p;
  }
  if (has_shared && lane == 0) sgw[t] = sigmoidf_(lg[E]);
}

// ----------------------------------------------------------------------------
// block-level stable dispatch (NT threads). Writes perm, inv, offsets, the slot
// list (non-empty experts ascending, then the shared expert) and the M-tile
// list for the grouped GEMMs.
// ----------------------------------------------------------------------------
struct DispatchSmem {
  int cnt[HX_MAX_EXPERTS + 1];
  int aux[HX_MAX_EXPERTS + 1];
  int flag[HX_MAX_EXPERTS + 1];
  int ntile[HX_MAX_EXPERTS + 1];
  int scan[1024 + 1];
  uint8_t whist[16][HX_MAX_EXPERTS];
};

// exclusive scan of a[0..n) in place (NT threads, contiguous segments); returns total
template <int NT>
HX_DEV int block_exclusive_scan(int* a, int n, int* scratch) {
  const int tid = threadIdx.x;
  const int seg = (n + NT - 1) / NT;
  int b = tid * seg, e = b + seg < n ? b + seg : n;
  int local = 0;
  for (int i = b; i < e; i++) local += a[i];
  scratch[tid] = local;
  __syncthreads();
  if (tid == 0) {
    int run = 0;
    for (int i = 0; i < NT; i++) {
      int c = scratch[i];
      scratch[i] = run;
      run += c;
    }
    scratch[NT] = run;   // scratch has NT+1 slots
  }
  __syncthreads();
  int run = scratch[tid];
  for (int i = b; i < e; i++) {
    int c = a[i];
    a[i] = run;
    run += c;
  }
  int total = scratch[NT];
  __syncthreads();
  return total;
}

template <int NT>
HX_DEV void dispatch_block(const DispatchArgs& a, DispatchSmem& sm) {
  const int tid = threadIdx.x, lane = lane_id(), wave = tid >> 6;
  const int E = a.E, F = a.F;
  for (int e = tid; e <= E; e += NT) sm.cnt[e] = 0;
  for (int i = tid; i < (NT / 64) * E; i += NT) sm.whist[i / E][i % E] = 0;
  __syncthreads();
  for (int f = tid; f < F; f += NT) atomicAdd(&sm.cnt[a.topk_idx[f]], 1);
  __syncthreads();
  // per-expert counts -> aux (kept), cnt -> exclusive offsets
  for (int e = tid; e < E; e += NT) sm.aux[e] = sm.cnt[e];
  __syncthreads();
  block_exclusive_scan<NT>(sm.cnt, E, sm.scan);
  for (int e = tid; e < E; e += NT) a.offsets[e] = sm.cnt[e];
  if (tid == 0) a.offsets[E] = F;
  __syncthreads();
  {
    // slot index = exclusive scan of (count > 0); tile index = exclusive scan of
    // ceil(count / tile_m)
    int* flag = sm.flag;
    int* ntile = sm.ntile;
    for (int e = tid; e < E; e += NT) {
      flag[e] = sm.aux[e] > 0 ? 1 : 0;
      ntile[e] = (sm.aux[e] + a.tile_m - 1) / a.tile_m;
    }
    __syncthreads();
    int nslot = block_exclusive_scan<NT>(flag, E, sm.scan);
    int ntl = block_exclusive_scan<NT>(ntile, E, sm.scan);
    for (int e = tid; e < E; e += NT) {
      int c = sm.aux[e];
      if (c > 0) {
        int s = flag[e];
        a.slots[3 * s + 0] = e;
        a.slots[3 * s + 1] = sm.cnt[e];
        a.slots[3 * s + 2] = c;
        int t0 = ntile[e];
        for (int m0 = 0, i = 0; m0 < c; m0 += a.tile_m, i++) {
          a.tiles[4 * (t0 + i) + 0] = s;
          a.tiles[4 * (t0 + i) + 1] = e;
          a.tiles[4 * (t0 + i) + 2] = sm.cnt[e] + m0;
          a.tiles[4 * (t0 + i) + 3] = c - m0 < a.tile_m ? c - m0 : a.tile_m;
        }
      }
    }
    if (tid == 0) {
      int ns = nslot, nt = ntl;
      if (a.has_shared) {
        a.slots[3 * ns + 0] = E;
        a.slots[3 * ns + 1] = F;
        a.slots[3 * ns + 2] = a.T;
        for (int m0 = 0; m0 < a.T; m0 += a.tile_m, nt++) {
          a.tiles[4 * nt + 0] = ns;
          a.tiles[4 * nt + 1] = E;
          a.tiles[4 * nt + 2] = F + m0;
          a.tiles[4 * nt + 3] = a.T - m0 < a.tile_m ? a.T - m0 : a.tile_m;
        }
        ns++;
      }
      a.counts[0] = ns;
      a.counts[1] = nt;
    }
  }
  __syncthreads();
  // stable scatter, NT entries at a time
  const int nbits = 32 - __clz(E);
  const unsigned long long lt = (1ull << lane) - 1ull;
  for (int base = 0; base < F; base += NT) {
    int f = base + tid;
    bool valid = f < F;
    int e = valid ? a.topk_idx[f] : 0;
    unsigned long long mask = __ballot(valid);
    for (int b = 0; b < nbits; b++) {
      int bit = (e >> b) & 1;
      unsigned long long m = __ballot(bit);
      mask &= bit ? m : ~m;
    }
    int rank = __popcll(mask & lt);
    int wcount = __popcll(mask);
    bool leader = valid && rank == 0;
    if (leader) sm.whist[wave][e] = (uint8_t)wcount;
    __syncthreads();
    if (valid) {
      int pre = 0;
      for (int w = 0; w < wave; w++) pre += sm.whist[w][e];
      int pos = sm.cnt[e] + pre + rank;
      a.perm[pos] = f;
      if (a.inv) a.inv[f] = pos;
    }
    __syncthreads();
    if (leader) {
      atomicAdd(&sm.cnt[e], wcount);
      sm.whist[wave][e] = 0;
    }
    __syncthreads();
  }
}

__global__ __launch_bounds__(1024) void k_dispatch(DispatchArgs a) {
  __shared__ DispatchSmem sm;
  dispatch_block<1024>(a, sm);
}

__global__ __launch_bounds__(256) void k_route_tokens(const float* logits, int E1, int T, int E, int k, bool norm,
                                                       bool has_shared, int32_t* topk_idx, float* topk_w, float* sgw) {
  int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  route_one_token(logits + (int64_t)t * E1, E, k, norm, has_shared, t, topk_idx, topk_w, sgw);
}

// ----------------------------------------------------------------------------
// router logits. Each wave owns TT tokens x TE router rows; lane l accumulates
// groups g = l, l+64, ... (8 inputs each) with fmaf, then the butterfly.
// With TAIL, the last block to finish runs the per-token routing and the
// dispatch for all T tokens (small T only).
// ----------------------------------------------------------------------------
template <bool XBF, bool RBF>
HX_DEV void load8(const void* base, int64_t row_elems, int64_t row, int h0, int H, bool vec, float* out) {
  if (vec) {
    if (XBF) {
      uint4 q = *(const uint4*)((const uint16_t*)base + row * row_elems + h0);
      const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int j = 0; j < 4; j++) {
        out[2 * j] = __uint_as_float(w[j] << 16);
        out[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
      }
    } else {
      const float4* p = (const float4*)((const float*)base + row * row_elems + h0);
      float4 a = p[0], b = p[1];
      out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
      out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; i++) {
      int h = h0 + i;
      out[i] = h < H ? (XBF ? bf16_to_f32(((const uint16_t*)base)[row * row_elems + h])
                            : ((const float*)base)[row * row_elems + h])
                     : 0.0f;
    }
  }
}

template <bool XBF, bool RBF, int TT, int TE, bool TAIL>
__global__ __launch_bounds__(256) void k_router(RouterArgs a) {
  const int lane = lane_id(), wave = threadIdx.x >> 6;
  const int e0 = (blockIdx.x * 4 + wave) * TE;
  const int t0 = blockIdx.y * TT;
  const int H = a.H, G = (H + 7) / 8;
  const bool vec = (H & 7) == 0;
  if (e0 < a.E1) {
    float acc[TT][TE];
#pragma unroll
    for (int i = 0; i < TT; i++)
#pragma unroll
      for (int j = 0; j < TE; j++) acc[i][j] = 0.0f;
    for (int g = lane; g < G; g += 64) {
      const int h0 = 8 * g;
      float xv[TT][8], wv[TE][8];
#pragma unroll
      for (int i = 0; i < TT; i++) {
        if (t0 + i < a.T) load8<XBF, XBF>(a.x, H, t0 + i, h0, H, vec, xv[i]);
        else
#pragma unroll
          for (int q = 0; q < 8; q++) xv[i][q] = 0.0f;
      }
#pragma unroll
      for (int j = 0; j < TE; j++) {
        if (e0 + j < a.E1) load8<RBF, RBF>(a.R, H, e0 + j, h0, H, vec, wv[j]);
        else
#pragma unroll
          for (int q = 0; q < 8; q++) wv[j][q] = 0.0f;
      }
      const int n = H - h0 < 8 ? H - h0 : 8;
#pragma unroll
      for (int q = 0; q < 8; q++) {
        if (q < n) {
#pragma unroll
          for (int i = 0; i < TT; i++)
#pragma unroll
            for (int j = 0; j < TE; j++) acc[i][j] = __builtin_fmaf(xv[i][q], wv[j][q], acc[i][j]);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < TT; i++)
#pragma unroll
      for (int j = 0; j < TE; j++) {
        float v = wave_sum<64>(acc[i][j]);
        const int t = t0 + i, e = e0 + j;
        if (lane == i * TE + j && t < a.T && e < a.E1) {
          if (XBF) v = bf16_to_f32(f32_to_bf16(v));
          if (a.bias && e < a.E) v = v + a.bias[e];
          a.logits[(int64_t)t * a.E1 + e] = v;
        }
      }
  }
  if constexpr (TAIL) {
    __shared__ int last;
    __syncthreads();
    if (threadIdx.x == 0) {
      __threadfence();
      unsigned total = gridDim.x * gridDim.y;
      unsigned prev = atomicAdd(a.counter, 1u);
      last = prev == total - 1;
    }
    __syncthreads();
    if (!last) return;
    __threadfence();
    for (int t = wave; t < a.T; t += 4)
      route_one_token(a.logits + (int64_t)t * a.E1, a.E, a.k, a.norm, a.has_shared, t, a.d.topk_idx,
                      a.topk_w, a.sgw);
    __threadfence();
    __syncthreads();
    __shared__ DispatchSmem sm;
    dispatch_block<256>(a.d, sm);
    if (threadIdx.x == 0) *a.counter = 0u;
  }
}

// ----------------------------------------------------------------------------
// launchers
// ----------------------------------------------------------------------------
template <bool XBF, bool RBF>
static void launch_router_t(const RouterArgs& a, bool tail, hipStream_t s) {
  if (tail) {
    dim3 grid((a.E1 + 3) / 4, a.T);
    hipLaunchKernelGGL((k_router<XBF, RBF, 1, 1, true>), grid, dim3(256), 0, s, a);
  } else {
    constexpr int TT = 8, TE = 4;
    dim3 grid((a.E1 + 4 * TE - 1) / (4 * TE), (a.T + TT - 1) / TT);
    hipLaunchKernelGGL((k_router<XBF, RBF, TT, TE, false>), grid, dim3(256), 0, s, a);
  }
}

void launch_router(const RouterArgs& a, bool xbf, bool rbf, bool tail, hipStream_t s) {
  if (xbf && rbf) launch_router_t<true, true>(a, tail, s);
  else if (xbf) launch_router_t<true, false>(a, tail, s);
  else if (rbf) launch_router_t<false, true>(a, tail, s);
  else launch_router_t<false, false>(a, tail, s);
}

void launch_route_tokens(const RouterArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(k_route_tokens, dim3((a.T + 3) / 4), dim3(256), 0, s, a.logits, a.E1, a.T, a.E, a.k, a.norm,
                     a.has_shared, a.d.topk_idx, a.topk_w, a.sgw);
}

void launch_dispatch(const DispatchArgs& d, hipStream_t s) {
  hipLaunchKernelGGL(k_dispatch, dim3(1), dim3(1024), 0, s, d);
}

}  // namespace hx
