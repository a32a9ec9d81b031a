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
// entries.)
//   k_disp_maps    (routing paths other than the MFMA one, which fills both
//                  maps itself) block c counts the experts of the tokens of
//                  chunk c (HX_DISPATCH_TOK tokens) and sets their bits
//   k_disp_fused   one workgroup per 1024 entries: per expert, the prefix over
//                  chunks and the total; offsets = exclusive scan of the totals;
//                  slots and M-tiles (workgroup 0); then one thread per entry
//                  (token t, expert e): position = offset of e + the prefix of e
//                  at t's chunk + the set bits of e's bitmap words from the
//                  chunk's first token up to t
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

// k_disp_fused: the scan and the scatter in one launch, one workgroup per
// DISP_EPB entries. The per-chunk counts are complete before it starts, so
// every workgroup scans them itself: thread e sums expert e's counts over all
// chunks, keeping the prefix at the (at most DISP_MAXC) chunks its own entries
// come from; the three-value block scan gives the offsets, slots and M tiles.
// Workgroup 0 writes offsets, slots, tiles and counts; every workgroup places
// its own entries (one thread each). The entry's expert and its bitmap words
// are loaded before the scan, so their latency overlaps it. (A one-block scan
// kernel followed by a per-entry scatter kernel took 6.0 + 4.6 us at 2048
// tokens, plus the gap between the two launches.)
constexpr int DISP_EPB = 1024;
constexpr int DISP_MAXC = DISP_EPB / HX_DISPATCH_TOK + 2;
__global__ __launch_bounds__(1024) void k_disp_fused(DispatchArgs a) {
  constexpr int WPC = HX_DISPATCH_TOK / 32, PB = 16;
  __shared__ int sh[3][17];
  __shared__ int s_first[HX_MAX_EXPERTS], s_off[HX_MAX_EXPERTS], s_cnt[HX_MAX_EXPERTS];
  __shared__ int s_base[DISP_MAXC][HX_MAX_EXPERTS];
  const int e = threadIdx.x, E = a.E, nb = dispatch_chunks(a.T), k = a.k;
  const int f0 = blockIdx.x * DISP_EPB, f1 = min(a.F, f0 + DISP_EPB);
  const int c_lo = (f0 / k) / HX_DISPATCH_TOK, c_hi = ((f1 - 1) / k) / HX_DISPATCH_TOK;
  // this thread's entry, then its bitmap words (the chunk's first word up to t's)
  const int f = f0 + (int)threadIdx.x;
  const bool has_f = f < f1;
  const int fe = has_f ? a.topk_idx[f] : 0;
  const float wv = has_f && a.wpos ? a.topk_w[f] : 0.0f;
  const int t = f / k, w = t >> 5, w0 = (t / HX_DISPATCH_TOK) * WPC;
  uint32_t b[WPC];
#pragma unroll
  for (int i = 0; i < WPC; i++) b[i] = has_f && w0 + i <= w ? a.bits[(int64_t)(w0 + i) * E + fe] : 0u;
  // expert e's total and its prefix at chunks c_lo .. c_hi, PB counts per memory round trip
  int count = 0;
  int pre[DISP_MAXC];
#pragma unroll
  for (int j = 0; j < DISP_MAXC; j++) pre[j] = 0;
  if (e < E) {
    for (int c0 = 0; c0 < nb; c0 += PB) {
      int h[PB];
#pragma unroll
      for (int i = 0; i < PB; i++) h[i] = c0 + i < nb ? a.hist[(int64_t)(c0 + i) * E + e] : 0;
#pragma unroll
      for (int i = 0; i < PB; i++) {
#pragma unroll
        for (int j = 0; j < DISP_MAXC; j++)
          if (c0 + i == c_lo + j) pre[j] = count;
        count += h[i];
      }
    }
  }
  const int in[3] = {e < E ? count : 0, e < E && count > 0 ? 1 : 0, e < E ? (count + a.tile_m - 1) / a.tile_m : 0};
  int ex[3], tot[3];
  block_scan3_1024(in, ex, tot, sh);
  const int off = ex[0], nslot = tot[1], ntile = tot[2];
  if (e < E) {
#pragma unroll
    for (int j = 0; j < DISP_MAXC; j++)
      if (c_lo + j <= c_hi) s_base[j][e] = off + pre[j];
    if (blockIdx.x == 0) {
      a.offsets[e] = off;
      s_first[e] = ex[2];
      s_off[e] = off;
      s_cnt[e] = count;
      if (count > 0) {
        a.slots[3 * ex[1] + 0] = e;
        a.slots[3 * ex[1] + 1] = off;
        a.slots[3 * ex[1] + 2] = count;
      }
    }
  }
  __syncthreads();
  if (blockIdx.x == 0) {
    for (int i = threadIdx.x; i < ntile; i += 1024) {
      int lo = 0, hi = E - 1;   // the largest e with s_first[e] <= i
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (s_first[mid] <= i) lo = mid;
        else hi = mid - 1;
      }
      const int m0 = (i - s_first[lo]) * a.tile_m, c = s_cnt[lo];
      a.tiles[4 * i + 0] = c;   // the rows of the expert's call: its arithmetic arm
      a.tiles[4 * i + 1] = lo;
      a.tiles[4 * i + 2] = s_off[lo] + m0;
      a.tiles[4 * i + 3] = c - m0 < a.tile_m ? c - m0 : a.tile_m;
    }
    if (threadIdx.x == 0) a.offsets[E] = a.F;
    int ns = nslot, nt = ntile;
    if (a.has_shared) {
      const int nst = (a.T + a.tile_m - 1) / a.tile_m;
      for (int i = threadIdx.x; i < nst; i += 1024) {
        const int m0 = i * a.tile_m;
        a.tiles[4 * (ntile + i) + 0] = a.T;
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
  // the shared expert's rows take its sigmoid gate as their weight
  if (a.wpos && a.has_shared && f < a.T) a.wpos[a.F + f] = a.sgw[f];
  const int cl = t / HX_DISPATCH_TOK - c_lo;
  if (has_f && cl >= 0 && cl < DISP_MAXC) {
    int pos = s_base[cl][fe];
#pragma unroll
    for (int i = 0; i < WPC; i++) pos += __popc(w0 + i < w ? b[i] : w0 + i == w ? b[i] & ((1u << (t & 31)) - 1u) : 0u);
    a.perm[pos] = f;
    if (a.inv) a.inv[f] = pos;
    if (a.wpos) a.wpos[pos] = wv;
  }
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
  route_small_lds(a.logits, a.E1, a.E, a.k, a.norm, a.has_shared, a.T, sm, route_small_threads(a.T));
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
  hx_launch(k_route_small, dim3(1), dim3(route_small_threads(a.T)), 0, s, a);
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
  hipLaunchKernelGGL(k_disp_fused, dim3((d.F + DISP_EPB - 1) / DISP_EPB), dim3(1024), 0, s, d);
  return hipGetLastError();
}

}  // namespace hx
