// Routing kernels: router logits, per-token softmax / top-k / renormalisation,
// and the stable dispatch permutation.
//
// Reference: route_scatter (crates/neuron/src/harness/arch/qwen3_5/moe.rs:124-162)
// and forward_fused's on-device routing + sort
// (crates/neuron/src/harness/tp/tp_qwen3_5.rs:1179-1189).
#include "hx_internal.h"
#include "hx_route_small.h"
#include "hx_router_dev.h"

namespace hx {

// ----------------------------------------------------------------------------
// Prefill dispatch: perm, inv, offsets, the slot list (non-empty experts
// ascending, then the shared expert) and the M-tile list for the grouped
// GEMMs. The order is by expert, then token (each token's experts are
// distinct, so this is the stable order by entry index). (One workgroup
// sorting the entries in LDS took ~35 µs at any size from 90 to 5,120
// entries, against 10-15 µs for these three kernels.)
//   k_disp_maps    (routing paths other than the MFMA one, which fills both
//                  maps itself) block c counts the experts of the tokens of
//                  chunk c (HX_DISPATCH_TOK tokens) and sets their bits
//   k_disp_scan    one block: per expert, the exclusive prefix over chunks and
//                  the total; offsets = exclusive scan of the totals; slots and
//                  M-tiles
//   k_disp_scatter one thread per entry (token t, expert e): position = the
//                  base of e in t's chunk + the set bits of e's bitmap words
//                  from the chunk's first token up to t
// ----------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_disp_maps(DispatchArgs a) {
  constexpr int WPC = HX_DISPATCH_TOK / 32;   // bitmap words a chunk
  __shared__ int cnt[HX_MAX_EXPERTS];
  __shared__ uint32_t row[WPC][HX_MAX_EXPERTS];
  const int c = blockIdx.x, E = a.E, k = a.k, W = dispatch_words(a.T);
  for (int e = threadIdx.x; e < E; e += 256) {
    cnt[e] = 0;
#pragma unroll
    for (int i = 0; i < WPC; i++) row[i][e] = 0u;
  }
  __syncthreads();
  const int t0 = c * HX_DISPATCH_TOK, n = min(HX_DISPATCH_TOK, a.T - t0) * k;
  for (int i = threadIdx.x; i < n; i += 256) {
    const int e = a.topk_idx[(int64_t)t0 * k + i], t = i / k;
    atomicAdd(&cnt[e], 1);
    atomicOr(&row[t >> 5][e], 1u << (t & 31));
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += 256) {
    a.hist[(int64_t)c * E + e] = cnt[e];
#pragma unroll
    for (int i = 0; i < WPC; i++)
      if (c * WPC + i < W) a.bits[(int64_t)(c * WPC + i) * E + e] = row[i][e];
  }
}

// exclusive scans of three values per thread over a 1024-thread block in one
// pass (three barriers); tot[i] gets the sums (sh: 3 x 17 ints of LDS)
HX_DEV void block_scan3_1024(const int (&v)[3], int (&r)[3], int (&tot)[3], int (*sh)[17]) {
  const int lane = lane_id(), wave = threadIdx.x >> 6;
  int x[3] = {v[0], v[1], v[2]};
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
#pragma unroll
    for (int i = 0; i < 3; i++) {
      const int y = __shfl_up(x[i], off, 64);
      if (lane >= off) x[i] += y;
    }
  }
  if (lane == 63)
#pragma unroll
    for (int i = 0; i < 3; i++) sh[i][wave] = x[i];
  __syncthreads();
  if (threadIdx.x < 3) {
    int run = 0;
    for (int w = 0; w < 16; w++) {
      const int c = sh[threadIdx.x][w];
      sh[threadIdx.x][w] = run;
      run += c;
    }
    sh[threadIdx.x][16] = run;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 3; i++) {
    r[i] = sh[i][wave] + x[i] - v[i];
    tot[i] = sh[i][16];
  }
}

// k_disp_scan: one block, thread e = expert e. The per-chunk bases are
// written once (prefix over chunks + the expert's offset) when the chunk
// count is at most SCAN_REG (registers), else in a second pass; the M tiles
// are written in parallel, tile i's expert found by an upper-bound search
// over the experts' first tiles (experts without tiles share the next one's
// first tile, so the largest e with first[e] <= i is the owner).
constexpr int SCAN_REG = 32;
__global__ __launch_bounds__(1024) void k_disp_scan(DispatchArgs a) {
  __shared__ int sh[3][17];
  __shared__ int s_first[HX_MAX_EXPERTS], s_slot[HX_MAX_EXPERTS], s_off[HX_MAX_EXPERTS], s_cnt[HX_MAX_EXPERTS];
  const int e = threadIdx.x, E = a.E, nb = dispatch_chunks(a.T);
  int count = 0;
  int pre[SCAN_REG];   // entries of e in chunks before c (nb <= SCAN_REG)
  if (e < E) {
    if (nb <= SCAN_REG) {
      int h[SCAN_REG];
#pragma unroll
      for (int i = 0; i < SCAN_REG; i++) h[i] = i < nb ? a.hist[(int64_t)i * E + e] : 0;
#pragma unroll
      for (int i = 0; i < SCAN_REG; i++) {
        pre[i] = count;
        count += h[i];
      }
    } else {
      // the expert's per-chunk counts, PB at a time: all loads of a batch
      // issued before the first is used (one memory round trip per batch)
      constexpr int PB = 16;
      for (int b0 = 0; b0 < nb; b0 += PB) {
        int h[PB];
#pragma unroll
        for (int i = 0; i < PB; i++) h[i] = b0 + i < nb ? a.hist[(int64_t)(b0 + i) * E + e] : 0;
#pragma unroll
        for (int i = 0; i < PB; i++) {
          if (b0 + i < nb) a.hist[(int64_t)(b0 + i) * E + e] = count;
          count += h[i];
        }
      }
    }
  }
  const int in[3] = {e < E ? count : 0, e < E && count > 0 ? 1 : 0, e < E ? (count + a.tile_m - 1) / a.tile_m : 0};
  int ex[3], tot[3];
  block_scan3_1024(in, ex, tot, sh);
  const int off = ex[0], slot = ex[1], nslot = tot[1], ntile = tot[2];
  if (e < E) {
    a.offsets[e] = off;
    s_first[e] = ex[2];
    s_slot[e] = slot;
    s_off[e] = off;
    s_cnt[e] = count;
    // per-chunk bases: offsets[e] + entries of e in earlier chunks
    if (nb <= SCAN_REG) {
#pragma unroll
      for (int i = 0; i < SCAN_REG; i++)
        if (i < nb) a.hist[(int64_t)i * E + e] = pre[i] + off;
    } else {
      for (int b = 0; b < nb; b++) a.hist[(int64_t)b * E + e] += off;
    }
    if (count > 0) {
      a.slots[3 * slot + 0] = e;
      a.slots[3 * slot + 1] = off;
      a.slots[3 * slot + 2] = count;
    }
  }
  __syncthreads();
  for (int t = threadIdx.x; t < ntile; t += 1024) {
    int lo = 0, hi = E - 1;   // the largest e with s_first[e] <= t
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (s_first[mid] <= t) lo = mid;
      else hi = mid - 1;
    }
    const int m0 = (t - s_first[lo]) * a.tile_m, c = s_cnt[lo];
    a.tiles[4 * t + 0] = s_slot[lo];
    a.tiles[4 * t + 1] = lo;
    a.tiles[4 * t + 2] = s_off[lo] + m0;
    a.tiles[4 * t + 3] = c - m0 < a.tile_m ? c - m0 : a.tile_m;
  }
  if (e == 0) a.offsets[E] = a.F;
  int ns = nslot, nt = ntile;
  if (a.has_shared) {
    const int nst = (a.T + a.tile_m - 1) / a.tile_m;
    for (int i = threadIdx.x; i < nst; i += 1024) {
      const int m0 = i * a.tile_m;
      a.tiles[4 * (ntile + i) + 0] = nslot;
      a.tiles[4 * (ntile + i) + 1] = E;
      a.tiles[4 * (ntile + i) + 2] = a.F + m0;
      a.tiles[4 * (ntile + i) + 3] = a.T - m0 < a.tile_m ? a.T - m0 : a.tile_m;
    }
    if (threadIdx.x == 0) {
      a.slots[3 * nslot + 0] = E;
      a.slots[3 * nslot + 1] = a.F;
      a.slots[3 * nslot + 2] = a.T;
    }
    ns++;
    nt += nst;
  }
  if (threadIdx.x == 0) {
    a.counts[0] = ns;
    a.counts[1] = nt;
  }
}

// one thread per entry: the chunk's base and the (at most HX_DISPATCH_TOK / 32)
// bitmap words from the chunk's first token to t, all loaded before the first
// is used; threads t < T also copy the shared expert's sigmoid gate to its
// rows' weights (wpos[F + t])
__global__ __launch_bounds__(256) void k_disp_scatter(DispatchArgs a) {
  constexpr int WPC = HX_DISPATCH_TOK / 32;
  const int f = blockIdx.x * 256 + threadIdx.x;
  if (a.wpos && a.has_shared && f < a.T) a.wpos[a.F + f] = a.sgw[f];
  if (f >= a.F) return;
  const int E = a.E, e = a.topk_idx[f], t = f / a.k, w = t >> 5, w0 = (t / HX_DISPATCH_TOK) * WPC;
  const float wv = a.wpos ? a.topk_w[f] : 0.0f;
  int pos = a.hist[(int64_t)(t / HX_DISPATCH_TOK) * E + e];
  uint32_t b[WPC];
#pragma unroll
  for (int i = 0; i < WPC; i++) b[i] = w0 + i <= w ? a.bits[(int64_t)(w0 + i) * E + e] : 0u;
#pragma unroll
  for (int i = 0; i < WPC; i++) pos += __popc(w0 + i < w ? b[i] : w0 + i == w ? b[i] & ((1u << (t & 31)) - 1u) : 0u);
  a.perm[pos] = f;
  if (a.inv) a.inv[f] = pos;
  if (a.wpos) a.wpos[pos] = wv;
}

// per-token routing for any T: one wave per token
template <int EPL>
__global__ __launch_bounds__(256) void k_route_tokens(const float* logits, int E1, int T, int E, int k, bool norm,
                                                       bool has_shared, int32_t* topk_idx, float* topk_w, float* sgw) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const float* lg = logits + (int64_t)t * E1;
  int e;
  float w;
  route_token_core<EPL>(lg, E, k, norm, e, w);
  const int lane = lane_id();
  if (lane < k) {
    topk_idx[(int64_t)t * k + lane] = e;
    topk_w[(int64_t)t * k + lane] = w;
  }
  if (has_shared && lane == 0) sgw[t] = sigmoidf_(lg[E]);
}

// router logits for any T: each wave owns TT tokens x TE router rows. Grid
// (row groups, token groups rounded up to 8); the linear workgroup id is mapped
// so that all row groups of one token group run on the same XCD (workgroups go
// to XCD id % 8): the token group's rows are fetched into that XCD's L2 once.
template <bool XBF, bool RBF, int TT, int TE>
__global__ __launch_bounds__(256) void k_router(RouterArgs a) {
  const int wave = threadIdx.x >> 6;
  const int NX = gridDim.x, L = blockIdx.y * NX + blockIdx.x;
  const int rg = (L >> 3) % NX, tg = (L / (8 * NX)) * 8 + (L & 7);
  if (tg * TT >= a.T) return;
  router_rows<XBF, RBF, TT, TE>(a, (rg * 4 + wave) * TE, tg * TT);
}

// prefill router: one wave per 8 tokens x 8 router rows, four waves per
// workgroup along the rows; XCD-aware order as in k_router
template <bool XBF, bool RBF, int NG>
__global__ __launch_bounds__(256) void k_router88(RouterArgs a) {
  const int wave = threadIdx.x >> 6;
  const int NX = gridDim.x, L = blockIdx.y * NX + blockIdx.x;
  const int rg = (L >> 3) % NX, tg = (L / (8 * NX)) * 8 + (L & 7);
  const int e0 = (rg * 4 + wave) * 8;
  if (tg * 8 >= a.T || e0 >= a.E1) return;
  router_tile88<XBF, RBF, NG>(a, e0, tg * 8);
}

// routing of a few tokens in one workgroup (256 or 512 threads: one wave per
// token up to 8), published to global memory
__global__ __launch_bounds__(512) void k_route_small(RouterArgs a) {
  __shared__ RouteSmem sm;
  route_small_lds(a.logits, a.E1, a.E, a.k, a.norm, a.has_shared, a.T, sm);
  publish_route(a.d, a.topk_w, a.sgw, sm);
}

template <bool XBF, bool RBF>
static void launch_router_t(const RouterArgs& a, hipStream_t s) {
  if (a.T <= 2) {
    dim3 grid((a.E1 + 3) / 4, ((a.T + 1) / 2 + 7) / 8 * 8);
    hx_launch(k_router<XBF, RBF, 2, 1>, grid, dim3(256), 0, s, a);
  } else if (a.T <= HX_DECODE_MAX_T) {
    dim3 grid((a.E1 + 3) / 4, ((a.T + 7) / 8 + 7) / 8 * 8);
    hx_launch(k_router<XBF, RBF, 8, 1>, grid, dim3(256), 0, s, a);
  } else if (a.H % 8 == 0 && a.H <= 8 * 256) {
    dim3 grid((a.E1 + 31) / 32, ((a.T + 7) / 8 + 7) / 8 * 8);
    if (a.H <= 8 * 64) hx_launch(k_router88<XBF, RBF, 1>, grid, dim3(256), 0, s, a);
    else if (a.H <= 8 * 128) hx_launch(k_router88<XBF, RBF, 2>, grid, dim3(256), 0, s, a);
    else hx_launch(k_router88<XBF, RBF, 4>, grid, dim3(256), 0, s, a);
  } else {
    constexpr int TT = 8, TE = 4;
    dim3 grid((a.E1 + 4 * TE - 1) / (4 * TE), ((a.T + TT - 1) / TT + 7) / 8 * 8);
    hx_launch(k_router<XBF, RBF, TT, TE>, grid, dim3(256), 0, s, a);
  }
}

void launch_router(const RouterArgs& a, bool xbf, bool rbf, hipStream_t s) {
  if (xbf && rbf) launch_router_t<true, true>(a, s);
  else if (xbf) launch_router_t<true, false>(a, s);
  else if (rbf) launch_router_t<false, true>(a, s);
  else launch_router_t<false, false>(a, s);
}

void launch_route_small(const RouterArgs& a, hipStream_t s) {
  hx_launch(k_route_small, dim3(1), dim3(a.T > 4 ? 512 : 256), 0, s, a);
}

void launch_route_tokens(const RouterArgs& a, hipStream_t s) {
  const dim3 g((a.T + 3) / 4), b(256);
#define RT(EPL)                                                                                           \
  hx_launch(k_route_tokens<EPL>, g, b, 0, s, (const float*)a.logits, a.E1, a.T, a.E, a.k, a.norm, a.has_shared, \
            a.d.topk_idx, a.topk_w, a.sgw)
  if (a.E <= 64) RT(1);
  else if (a.E <= 128) RT(2);
  else if (a.E <= 256) RT(4);
  else if (a.E <= 512) RT(8);
  else RT(16);
#undef RT
}

hipError_t launch_dispatch(const DispatchArgs& d, hipStream_t s, bool maps_ready) {
  if (!d.hist || d.E > HX_MAX_EXPERTS) return hipErrorInvalidValue;   // a prefill workspace holds the maps
  if (!maps_ready) hipLaunchKernelGGL(k_disp_maps, dim3(dispatch_chunks(d.T)), dim3(256), 0, s, d);
  hipLaunchKernelGGL(k_disp_scan, dim3(1), dim3(1024), 0, s, d);
  hipLaunchKernelGGL(k_disp_scatter, dim3((d.F + 255) / 256), dim3(256), 0, s, d);
  return hipGetLastError();
}

}  // namespace hx
