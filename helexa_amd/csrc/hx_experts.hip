// Expert kernels: SwiGLU gate/up GEMV, down GEMV with the weighted combine
// (every shape outside the fast decode and prefill MFMA kernels). For GGUF
// weights the expert calls of m <= 64 rows read the f32 d q of the Q8 codes
// of their tokens (k_xq_f32) and of their rows of h (k_hq_f32, in place),
// the reference's quantised arm up to f32 rounding; larger calls compute
// exactly in f32 (the reference's f16 arm within f16 operand rounding).
//
// Reference: Qwen3_5MLP::forward (crates/neuron/src/harness/arch/qwen3_5/mlp.rs:54-60),
// the scatter loop of Module::forward (moe.rs:177-195: experts ascending,
// then the sigmoid-gated shared expert) and the fused path's weighted down
// GEMM + sum over k (crates/neuron/src/harness/tp/tp_qwen3_5.rs:1192-1225).
//
// Work is described by the slot list the dispatch wrote: slot u = (expert e,
// start position in the permuted order, token count); the shared expert is
// the last slot with e == E, start F and all T tokens. SwiGLU activations of
// slot u's j-th token live in row start+j of hbuf (shared: row F+t).
#include "hx_internal.h"

namespace hx {

// load n (multiple of 8, 8-aligned offset) activations as f32
HX_DEV void load_run(const void* base, bool bf, int64_t off, float* out, int n) {
  if (bf) {
    const uint4* p = (const uint4*)((const uint16_t*)base + off);
    for (int v = 0; v < n / 8; v++) {
      uint4 q = p[v];
      const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int j = 0; j < 4; j++) {
        out[8 * v + 2 * j] = __uint_as_float(w[j] << 16);
        out[8 * v + 2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
      }
    }
  } else {
    const float4* p = (const float4*)((const float*)base + off);
    for (int v = 0; v < n / 4; v++) {
      float4 q = p[v];
      out[4 * v] = q.x; out[4 * v + 1] = q.y; out[4 * v + 2] = q.z; out[4 * v + 3] = q.w;
    }
  }
}

// the CH activations of chunk c of a row, in chunk order
template <int FMT>
HX_DEV void load_chunk_x(const void* row, bool bf, int c, float* xv) {
  using CK = Chunk<FMT>;
#pragma unroll
  for (int r = 0; r < CK::CH / CK::RUN; r++) load_run(row, bf, CK::pos(c, r * CK::RUN), xv + r * CK::RUN, CK::RUN);
}

// ----------------------------------------------------------------------------
// gate/up + SwiGLU. grid = (row blocks, slots). Each wave owns NRG row groups of
// RG = 64 / LPR rows; lane ll of a row group owns chunks ll + LPR * ci.
// ----------------------------------------------------------------------------
template <int FMT, int LPR, int CPL, int NTOK, int NRG>
__global__ __launch_bounds__(256) void k_gate_up(ExpertArgs a) {
  using CK = Chunk<FMT>;
  constexpr int CH = CK::CH, RG = 64 / LPR, NS = CK::NSUM > 0 ? CK::NSUM : 1;
  const int u = blockIdx.y;
  if (u >= a.counts[0]) return;
  const int e = a.slots[3 * u], start = a.slots[3 * u + 1], count = a.slots[3 * u + 2];
  const bool sh = e == a.E;
  const uint8_t* G = sh ? a.sgate.base : a.gate.mat(e);
  const uint8_t* U = sh ? a.sup.base : a.up.mat(e);
  const int rows = sh ? a.Is : a.I;
  const int K = a.H, nch = K / CH;
  const int lane = lane_id(), wave = threadIdx.x >> 6, rg = lane / LPR, ll = lane % LPR;
  const int row_base = (blockIdx.x * 4 + wave) * (RG * NRG);
  if (row_base >= rows) return;
  // GGUF weights, a call of m <= HX_QUANT_M rows: the reference quantises the
  // tokens to the vec_dot type (MaybeQuantLinear, tp_linear.rs:120-137); they
  // come as the f32 d q of their codes (k_xq_f32)
  const bool qa = a.xq32 && count <= HX_QUANT_M;

  // weights first: every load of the wave is in flight before any math
  typename CK::Raw rgt[NRG][CPL], rup[NRG][CPL];
#pragma unroll
  for (int g = 0; g < NRG; g++) {
    const int row = row_base + g * RG + rg;
#pragma unroll
    for (int ci = 0; ci < CPL; ci++) {
      const int c = ll + LPR * ci;
      if (row < rows && c < nch) {
        CK::load(G, rows, K, row, c, rgt[g][ci]);
        CK::load(U, rows, K, row, c, rup[g][ci]);
      }
    }
  }
  for (int tg = 0; tg < count; tg += NTOK) {
    float xv[NTOK][CPL][CH], xs[NTOK][CPL][NS];
    int hrow[NTOK];
#pragma unroll
    for (int tok = 0; tok < NTOK; tok++) {
      const int j = tg + tok < count ? tg + tok : count - 1;
      const int t = sh ? j : a.perm[start + j] / a.k;
      hrow[tok] = sh ? a.F + j : start + j;
      const bool xb = a.xbf && !qa;
      const void* xr = qa ? (const void*)(a.xq32 + (int64_t)t * K)
                          : xb ? (const void*)((const uint16_t*)a.x + (int64_t)t * K)
                               : (const void*)((const float*)a.x + (int64_t)t * K);
#pragma unroll
      for (int ci = 0; ci < CPL; ci++) {
        const int c = ll + LPR * ci;
        if (c < nch) {
          load_chunk_x<FMT>(xr, xb, c, xv[tok][ci]);
          CK::sums(xv[tok][ci], xs[tok][ci]);
        }
      }
    }
#pragma unroll
    for (int g = 0; g < NRG; g++) {
      const int row = row_base + g * RG + rg;
#pragma unroll
      for (int tok = 0; tok < NTOK; tok++) {
        float pg = 0.f, pu = 0.f;
#pragma unroll
        for (int ci = 0; ci < CPL; ci++) {
          const int c = ll + LPR * ci;
          if (row < rows && c < nch) {
            pg += CK::dot(rgt[g][ci], xv[tok][ci], xs[tok][ci]);
            pu += CK::dot(rup[g][ci], xv[tok][ci], xs[tok][ci]);
          }
        }
        pg = wave_sum<LPR>(pg);
        pu = wave_sum<LPR>(pu);
        if (ll == 0 && row < rows && tg + tok < count) {
          float h = siluf_(pg) * pu;
          a.hbuf[(int64_t)hrow[tok] * a.hstride + row] = h;
          if (a.hbf) a.hbf[(int64_t)hrow[tok] * a.hstride + row] = f32_to_bf16(h);
        }
      }
    }
  }
}

// ----------------------------------------------------------------------------
// decode down projection + combine. Block = RG output rows (one wave-row-group);
// its 4 waves split the slots; contrib[u][t][r] collects w * (down_e row . h)
// in LDS and the final sum runs over u in slot order (experts ascending, then
// the shared expert), as moe.rs:178-194 does.
// ----------------------------------------------------------------------------
template <int FMT, int LPR, int CPL, int SPW>
__global__ __launch_bounds__(256) void k_down_combine(ExpertArgs a) {
  using CK = Chunk<FMT>;
  constexpr int CH = CK::CH, RG = 64 / LPR, NS = CK::NSUM > 0 ? CK::NSUM : 1;
  extern __shared__ float contrib[];
  const int nslots = a.counts[0], T = a.T;
  const int lane = lane_id(), wave = threadIdx.x >> 6, rg = lane / LPR, ll = lane % LPR;
  const int n0 = blockIdx.x * RG, row = n0 + rg;
  for (int i = threadIdx.x; i < nslots * T * RG; i += 256) contrib[i] = 0.f;
  __syncthreads();
  for (int ub = wave; ub < nslots; ub += 4 * SPW) {
    typename CK::Raw raw[SPW][CPL];
#pragma unroll
    for (int s = 0; s < SPW; s++) {
      const int u = ub + 4 * s;
      if (u < nslots) {
        const int e = a.slots[3 * u];
        const bool sh = e == a.E;
        const uint8_t* W = sh ? a.sdown.base : a.down.mat(e);
        const int K = sh ? a.Is : a.I;
#pragma unroll
        for (int ci = 0; ci < CPL; ci++) {
          const int c = ll + LPR * ci;
          if (row < a.H && c < K / CH) CK::load(W, a.H, K, row, c, raw[s][ci]);
        }
      }
    }
#pragma unroll
    for (int s = 0; s < SPW; s++) {
      const int u = ub + 4 * s;
      if (u >= nslots) break;
      const int e = a.slots[3 * u], start = a.slots[3 * u + 1], count = a.slots[3 * u + 2];
      const bool sh = e == a.E;
      const int K = sh ? a.Is : a.I;
      for (int j = 0; j < count; j++) {
        int t, hrow;
        float wgt;
        if (sh) {
          t = j;
          hrow = a.F + j;
          wgt = a.sgw[j];
        } else {
          const int f = a.perm[start + j];
          t = f / a.k;
          hrow = start + j;
          wgt = a.topk_w[f];
        }
        float p = 0.f;
#pragma unroll
        for (int ci = 0; ci < CPL; ci++) {
          const int c = ll + LPR * ci;
          if (c < K / CH) {
            float xv[CH], xs[NS];
            load_chunk_x<FMT>(a.hbuf + (int64_t)hrow * a.hstride, false, c, xv);
            CK::sums(xv, xs);
            p += CK::dot(raw[s][ci], xv, xs);
          }
        }
        p = wave_sum<LPR>(p);
        if (ll == 0 && row < a.H) contrib[((int64_t)u * T + t) * RG + rg] = wgt * p;
      }
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < T * RG; i += 256) {
    const int t = i / RG, r = i % RG;
    if (n0 + r >= a.H) continue;
    float y = 0.f;
    for (int u = 0; u < nslots; u++) y += contrib[((int64_t)u * T + t) * RG + r];
    const int64_t o = (int64_t)t * a.H + n0 + r;
    if (a.xbf) ((uint16_t*)a.y)[o] = f32_to_bf16(y);
    else ((float*)a.y)[o] = y;
  }
}

// ----------------------------------------------------------------------------
// prefill fallback down projection: obuf[hrow][n] = w * (down_e row n . h[hrow])
// grid = (row blocks, slots)
// ----------------------------------------------------------------------------
template <int FMT, int LPR, int CPL, int NTOK, int NRG>
__global__ __launch_bounds__(256) void k_down_rows(ExpertArgs a) {
  using CK = Chunk<FMT>;
  constexpr int CH = CK::CH, RG = 64 / LPR, NS = CK::NSUM > 0 ? CK::NSUM : 1;
  const int u = blockIdx.y;
  if (u >= a.counts[0]) return;
  const int e = a.slots[3 * u], start = a.slots[3 * u + 1], count = a.slots[3 * u + 2];
  const bool sh = e == a.E;
  const uint8_t* W = sh ? a.sdown.base : a.down.mat(e);
  const int K = sh ? a.Is : a.I, nch = K / CH, rows = a.H;
  const int lane = lane_id(), wave = threadIdx.x >> 6, rg = lane / LPR, ll = lane % LPR;
  const int row_base = (blockIdx.x * 4 + wave) * (RG * NRG);
  if (row_base >= rows) return;
  typename CK::Raw raw[NRG][CPL];
#pragma unroll
  for (int g = 0; g < NRG; g++) {
    const int row = row_base + g * RG + rg;
#pragma unroll
    for (int ci = 0; ci < CPL; ci++) {
      const int c = ll + LPR * ci;
      if (row < rows && c < nch) CK::load(W, rows, K, row, c, raw[g][ci]);
    }
  }
  for (int tg = 0; tg < count; tg += NTOK) {
    float xv[NTOK][CPL][CH], xs[NTOK][CPL][NS], wgt[NTOK];
    int hrow[NTOK];
#pragma unroll
    for (int tok = 0; tok < NTOK; tok++) {
      const int j = tg + tok < count ? tg + tok : count - 1;
      hrow[tok] = sh ? a.F + j : start + j;
      wgt[tok] = sh ? a.sgw[j] : a.topk_w[a.perm[start + j]];
#pragma unroll
      for (int ci = 0; ci < CPL; ci++) {
        const int c = ll + LPR * ci;
        if (c < nch) {
          load_chunk_x<FMT>(a.hbuf + (int64_t)hrow[tok] * a.hstride, false, c, xv[tok][ci]);
          CK::sums(xv[tok][ci], xs[tok][ci]);
        }
      }
    }
#pragma unroll
    for (int g = 0; g < NRG; g++) {
      const int row = row_base + g * RG + rg;
#pragma unroll
      for (int tok = 0; tok < NTOK; tok++) {
        float p = 0.f;
#pragma unroll
        for (int ci = 0; ci < CPL; ci++) {
          const int c = ll + LPR * ci;
          if (row < rows && c < nch) p += CK::dot(raw[g][ci], xv[tok][ci], xs[tok][ci]);
        }
        p = wave_sum<LPR>(p);
        if (ll == 0 && row < rows && tg + tok < count) {
          const int64_t o = (int64_t)hrow[tok] * a.H + row;
          if (a.xbf) ((uint16_t*)a.obuf)[o] = f32_to_bf16(wgt[tok] * p);
          else ((float*)a.obuf)[o] = wgt[tok] * p;
        }
      }
    }
  }
}

// ----------------------------------------------------------------------------
// combine: y[t] = sum of the token's k weighted expert rows in ascending expert
// order (= ascending permuted position), then the shared expert's row.
// Grid (T, ceil(H / 2048)): a block serves one token and up to 2048 outputs,
// 8 per thread. Wave 0 sorts the token's k positions once (rank of each among
// the k, into LDS); every thread then issues all k + 1 row loads together.
// ----------------------------------------------------------------------------
// (the bound of 8 workgroups per CU holds it to 64 registers, so the T
// workgroups of a prefill are all resident at once instead of in two rounds)
__global__ __launch_bounds__(256, 8) void k_combine(ExpertArgs a) {
  __shared__ int spos[HX_MAX_TOPK + 1];
  const int t = blockIdx.x, k = a.k;
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    const int p = lane < k ? a.inv[(int64_t)t * k + lane] : 0x7fffffff;
    int rank = 0;
    for (int j = 0; j < k; j++) rank += __builtin_amdgcn_readlane(p, j) < p;
    if (lane < k) spos[rank] = p;
    if (lane == 0) spos[k] = a.F + t;   // the shared expert's row (used when Is > 0)
  }
  __syncthreads();
  const int n0 = (blockIdx.y * 256 + threadIdx.x) * 8;
  if (n0 >= a.H) return;
  const int nrows = k + (a.Is > 0 ? 1 : 0);
  // the shared expert's row (row k) scaled here when the down GEMM stored it
  // unweighted; the routed rows are multiplied by 1 (exact)
  const float shs = a.shared_raw && a.Is > 0 ? a.sgw[t] : 1.f;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (a.xbf) {
    // rows loaded B at a time without branches: indices past the last row are
    // clamped to it and their values masked to +0 (adding +0 changes nothing)
    constexpr int B = 12;
    for (int j0 = 0; j0 < nrows; j0 += B) {
      uint4 q[B];
#pragma unroll
      for (int j = 0; j < B; j++) {
        const int r = spos[min(j0 + j, nrows - 1)];
        q[j] = *(const uint4*)((const uint16_t*)a.obuf + (int64_t)r * a.H + n0);
      }
#pragma unroll
      for (int j = 0; j < B; j++) {
        const uint32_t m = j0 + j < nrows ? 0xffffffffu : 0u;
        const uint32_t w[4] = {q[j].x & m, q[j].y & m, q[j].z & m, q[j].w & m};
        const float sc = j0 + j == k ? shs : 1.f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
          acc[2 * i] += __uint_as_float(w[i] << 16) * sc;
          acc[2 * i + 1] += __uint_as_float(w[i] & 0xffff0000u) * sc;
        }
      }
    }
    uint4 o;
    o.x = f32_to_bf16(acc[0]) | ((uint32_t)f32_to_bf16(acc[1]) << 16);
    o.y = f32_to_bf16(acc[2]) | ((uint32_t)f32_to_bf16(acc[3]) << 16);
    o.z = f32_to_bf16(acc[4]) | ((uint32_t)f32_to_bf16(acc[5]) << 16);
    o.w = f32_to_bf16(acc[6]) | ((uint32_t)f32_to_bf16(acc[7]) << 16);
    *(uint4*)((uint16_t*)a.y + (int64_t)t * a.H + n0) = o;
  } else {
    for (int j = 0; j < nrows; j++) {
      const float4* q = (const float4*)((const float*)a.obuf + (int64_t)spos[j] * a.H + n0);
      const float4 u = q[0], v = q[1];
      const float sc = j == k ? shs : 1.f;
      acc[0] += u.x * sc; acc[1] += u.y * sc; acc[2] += u.z * sc; acc[3] += u.w * sc;
      acc[4] += v.x * sc; acc[5] += v.y * sc; acc[6] += v.z * sc; acc[7] += v.w * sc;
    }
    float4* p = (float4*)((float*)a.y + (int64_t)t * a.H + n0);
    p[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
    p[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
  }
}

// ----------------------------------------------------------------------------
// launchers: pick LPR / CPL from K and the chunk size
// ----------------------------------------------------------------------------
template <int FMT>
static int chunks_per_row(int K) { return K / Chunk<FMT>::CH; }

// chunks per row -> (lanes per row, chunks per lane); rows longer than 512
// chunks are rejected when the block is created
#define HX_LPR_CASES(MACRO, NCH)                       \
  if ((NCH) > 512) { return hipErrorInvalidValue; }    \
  else if ((NCH) > 256) { MACRO(64, 8); }              \
  else if ((NCH) > 128) { MACRO(64, 4); }              \
  else if ((NCH) > 64) { MACRO(64, 2); }               \
  else if ((NCH) > 32) { MACRO(64, 1); }               \
  else if ((NCH) > 16) { MACRO(32, 1); }               \
  else if ((NCH) > 8) { MACRO(16, 1); }                \
  else { MACRO(8, 1); }

template <int FMT>
static hipError_t gate_up_fmt(const ExpertArgs& a, bool decode, hipStream_t s) {
  const int nch = chunks_per_row<FMT>(a.H);
  const int maxrows = a.I > a.Is ? a.I : a.Is;
  const int nslot = a.max_slots;
#define GU(LPR, CPL)                                                                          \
  {                                                                                           \
    constexpr int RG = 64 / LPR, NRG = (CPL >= 2 ? 1 : 2);                                    \
    dim3 grid((maxrows + 4 * RG * NRG - 1) / (4 * RG * NRG), nslot);                          \
    if (decode && a.T == 1)                                                                   \
      hipLaunchKernelGGL((k_gate_up<FMT, LPR, CPL, 1, NRG>), grid, dim3(256), 0, s, a);       \
    else                                                                                      \
      hipLaunchKernelGGL((k_gate_up<FMT, LPR, CPL, 2, NRG>), grid, dim3(256), 0, s, a);       \
  }
  HX_LPR_CASES(GU, nch)
#undef GU
  return hipGetLastError();
}

template <int FMT>
static hipError_t down_combine_fmt(const ExpertArgs& a, hipStream_t s) {
  const int K = a.I > a.Is ? a.I : a.Is;
  const int nch = chunks_per_row<FMT>(K);
#define DC(LPR, CPL)                                                                            \
  {                                                                                             \
    constexpr int RG = 64 / LPR;                                                                \
    size_t lds = (size_t)a.max_slots * a.T * RG * sizeof(float);                                \
    hipLaunchKernelGGL((k_down_combine<FMT, LPR, CPL, 4>), dim3((a.H + RG - 1) / RG), dim3(256), \
                       lds, s, a);                                                              \
  }
  HX_LPR_CASES(DC, nch)
#undef DC
  return hipGetLastError();
}

template <int FMT>
static hipError_t down_rows_fmt(const ExpertArgs& a, hipStream_t s) {
  const int K = a.I > a.Is ? a.I : a.Is;
  const int nch = chunks_per_row<FMT>(K);
#define DR(LPR, CPL)                                                                          \
  {                                                                                           \
    constexpr int RG = 64 / LPR, NRG = (CPL >= 2 ? 1 : 2);                                    \
    dim3 grid((a.H + 4 * RG * NRG - 1) / (4 * RG * NRG), a.max_slots);                        \
    hipLaunchKernelGGL((k_down_rows<FMT, LPR, CPL, 2, NRG>), grid, dim3(256), 0, s, a);       \
  }
  HX_LPR_CASES(DR, nch)
#undef DR
  return hipGetLastError();
}

hipError_t launch_gate_up_gemv(const ExpertArgs& a, hipStream_t s) {
  switch (a.gate.fmt) {
    case HX_F32: return gate_up_fmt<HX_F32>(a, true, s);
    case HX_BF16: return gate_up_fmt<HX_BF16>(a, true, s);
    case HX_Q8_0: return gate_up_fmt<HX_Q8_0>(a, true, s);
    case HX_Q4_K: return gate_up_fmt<HX_Q4_K>(a, true, s);
    case HX_Q6_K: return gate_up_fmt<HX_Q6_K>(a, true, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_gate_up_prefill(const ExpertArgs& a, hipStream_t s) {
  switch (a.gate.fmt) {
    case HX_F32: return gate_up_fmt<HX_F32>(a, false, s);
    case HX_BF16: return gate_up_fmt<HX_BF16>(a, false, s);
    case HX_Q8_0: return gate_up_fmt<HX_Q8_0>(a, false, s);
    case HX_Q4_K: return gate_up_fmt<HX_Q4_K>(a, false, s);
    case HX_Q6_K: return gate_up_fmt<HX_Q6_K>(a, false, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_down_gemv_combine(const ExpertArgs& a, hipStream_t s) {
  switch (a.down.fmt) {
    case HX_F32: return down_combine_fmt<HX_F32>(a, s);
    case HX_BF16: return down_combine_fmt<HX_BF16>(a, s);
    case HX_Q8_0: return down_combine_fmt<HX_Q8_0>(a, s);
    case HX_Q4_K: return down_combine_fmt<HX_Q4_K>(a, s);
    case HX_Q6_K: return down_combine_fmt<HX_Q6_K>(a, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_down_prefill(const ExpertArgs& a, hipStream_t s) {
  switch (a.down.fmt) {
    case HX_F32: return down_rows_fmt<HX_F32>(a, s);
    case HX_BF16: return down_rows_fmt<HX_BF16>(a, s);
    case HX_Q8_0: return down_rows_fmt<HX_Q8_0>(a, s);
    case HX_Q4_K: return down_rows_fmt<HX_Q4_K>(a, s);
    case HX_Q6_K: return down_rows_fmt<HX_Q6_K>(a, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_combine(const ExpertArgs& a, hipStream_t s) {
  // H % 8 == 0 holds for every block this library creates with a combine step
  hx_launch(k_combine, dim3((unsigned)a.T, (unsigned)((a.H / 8 + 255) / 256)), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace hx
