// Activation quantisation kernels: the rows the reference quantises before its
// integer vec_dot (expert calls of m <= 64 rows, MaybeQuantLinear::forward,
// crates/neuron/src/harness/tp/tp_linear.rs:120-137), for the prefill MFMA
// kernels and the generic GEMV kernels; and hx_quantize_activations, which
// exposes the codes for tests.
//
// A row is quantised by one wave in passes of 512 elements: group g of 8 of
// the pass in lane g % 64 (the layout of hx_quant.h, whose quant_group gives
// the reference's codes). Outputs:
//   * f16 d q (the prefill MFMA kernels' operand; one rounding of the exact
//     dequantised value), in the element order of their A operands;
//   * f32 d q (the generic kernels' f32 dot products);
//   * int8 codes and per-block d (tests).
#include "hx_internal.h"
#include "hx_quant.h"

namespace hx {

// groups g0 .. g0 + 63 of a row of G groups of 8 (one pass of a wave; G % 4 ==
// 0, % 32 for Q8_K, so a block lies wholly inside or past the row): load(g, x)
// fills the 8 values of group g, emit(g, q, d) takes its codes and block d
template <int FMT, class Load, class Emit>
HX_DEV void quant_pass(int g0, int G, Load load, Emit emit) {
  const int g = g0 + lane_id();
  float x[8];
  if (g < G) {
    load(g, x);
  } else {
#pragma unroll
    for (int j = 0; j < 8; j++) x[j] = 0.f;
  }
  float q[8], d;
  quant_group<FMT>(x, q, d);
  if (g < G) emit(g, q, d);
}
// a row of K elements (K % 256 == 0 for Q8_K, % 32 for Q8_0) in passes
template <int FMT, class Load, class Emit>
HX_DEV void quant_row(int K, Load load, Emit emit) {
  for (int g0 = 0; g0 < K / 8; g0 += 64) quant_pass<FMT>(g0, K / 8, load, emit);   // wave-uniform
}

HX_DEV void load_bf16x8(const uint16_t* p, float (&x)[8]) {
  const uint4 v = *(const uint4*)p;
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int j = 0; j < 4; j++) {
    x[2 * j] = __uint_as_float(w[j] << 16);
    x[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
  }
}
HX_DEV void load_f32x8(const float* p, float (&x)[8]) {
  const float4 a = *(const float4*)p, b = *(const float4*)(p + 4);
  x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
  x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
}

// f16 d q of a group into 8 f16 at p: natural order, or (0, 2, 1, 3) within
// each group of 4 (the prefill kernels' swizzled K order)
HX_DEV void store_fq8(uint16_t* p, const float (&q)[8], float d, bool nat) {
  _Float16 h[8];
#pragma unroll
  for (int j = 0; j < 8; j++) h[j] = fq_f16(q[j], d);
  auto pk = [&](int i, int j) { return (uint32_t)__builtin_bit_cast(uint16_t, h[i]) | ((uint32_t)__builtin_bit_cast(uint16_t, h[j]) << 16); };
  *(uint4*)p = nat ? make_uint4(pk(0, 1), pk(2, 3), pk(4, 5), pk(6, 7)) : make_uint4(pk(0, 2), pk(1, 3), pk(4, 6), pk(5, 7));
}

// ---------------------------------------------------------------- prefill
// tokens (bf16) -> xq: the f16 operand of the m <= 64 expert calls, in the
// order of xh (natural for Q4_K gate/up, else swizzled); one wave per token
// and 512 elements (grid.y: the row's passes)
template <int FMT>
__global__ __launch_bounds__(256) void k_xq_fq(ExpertArgs a, int nat) {
  const int t = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6);
  if (t >= a.T) return;
  const uint16_t* src = (const uint16_t*)a.x + (int64_t)t * a.H;
  uint16_t* dst = a.xq + (int64_t)t * a.H;
  quant_pass<FMT>(64 * (int)blockIdx.y, a.H / 8, [&](int g, float (&x)[8]) { load_bf16x8(src + 8 * g, x); },
                  [&](int g, const float (&q)[8], float d) { store_fq8(dst + 8 * g, q, d, nat != 0); });
}

// rows of h (f32, written by the gate/up kernels for the m <= 64 expert calls)
// -> hbf as f16 d q in the swizzled order; workgroup (x, y) = rows 4 y .. 4 y + 3
// of M tile x of the dispatch list (or, for the shared expert's own launch,
// of T), one row per wave; tiles of the f16 arm (m > 64) are skipped. (Placing
// each tile's workgroups on the XCD of its gate/up and down workgroups was
// measured slower: C3 15.5 -> 17.1 us; so were four rows a wave with their
// loads issued together, a quarter of the workgroups: C3 +4.1 us paired.)
template <int FMT>
__global__ __launch_bounds__(256) void k_hq_fq(ExpertArgs a) {
  const int tile = blockIdx.x, nt = blockIdx.y;
  int m, p0, rows, K;
  if (a.tsel == HX_TILES_SHARED) {
    const int m0 = tile * HX_TILE_M;
    if (m0 >= a.T) return;
    m = a.T;
    p0 = a.F + m0;
    rows = min(HX_TILE_M, a.T - m0);
    K = a.Is;
  } else {
    if (tile >= a.counts[1]) return;
    m = a.tiles[4 * tile + 0];
    const int e = a.tiles[4 * tile + 1];
    if (a.tsel == HX_TILES_ROUTED && e == a.E) return;
    p0 = a.tiles[4 * tile + 2];
    rows = a.tiles[4 * tile + 3];
    K = e == a.E ? a.Is : a.I;
  }
  const int r = 4 * nt + (int)(threadIdx.x >> 6);
  if (m > HX_QUANT_M || r >= rows) return;
  const float* src = a.hbuf + (int64_t)(p0 + r) * a.hstride;
  uint16_t* dst = a.hbf + (int64_t)(p0 + r) * a.hstride;
  quant_row<FMT>(K, [&](int g, float (&x)[8]) { load_f32x8(src + 8 * g, x); },
                 [&](int g, const float (&q)[8], float d) { store_fq8(dst + 8 * g, q, d, false); });
}

// ---------------------------------------------------------------- generic paths
// tokens -> xq32 (f32 d q, for the m <= 64 calls of the generic gate/up kernel)
template <int FMT>
__global__ __launch_bounds__(256) void k_xq_f32(ExpertArgs a) {
  const int t = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6);
  if (t >= a.T) return;
  float* dst = a.xq32 + (int64_t)t * a.H;
  auto emit = [&](int g, const float (&q)[8], float d) {
    *(float4*)(dst + 8 * g) = make_float4(d * q[0], d * q[1], d * q[2], d * q[3]);
    *(float4*)(dst + 8 * g + 4) = make_float4(d * q[4], d * q[5], d * q[6], d * q[7]);
  };
  if (a.xbf) {
    const uint16_t* src = (const uint16_t*)a.x + (int64_t)t * a.H;
    quant_row<FMT>(a.H, [&](int g, float (&x)[8]) { load_bf16x8(src + 8 * g, x); }, emit);
  } else {
    const float* src = (const float*)a.x + (int64_t)t * a.H;
    quant_row<FMT>(a.H, [&](int g, float (&x)[8]) { load_f32x8(src + 8 * g, x); }, emit);
  }
}

// rows of h of the m <= 64 slots -> f32 d q in place (workgroup = one slot)
template <int FMT>
__global__ __launch_bounds__(256) void k_hq_f32(ExpertArgs a) {
  const int u = blockIdx.x;
  if (u >= a.counts[0]) return;
  const int e = a.slots[3 * u], start = a.slots[3 * u + 1], count = a.slots[3 * u + 2];
  if (count > HX_QUANT_M) return;
  const bool sh = e == a.E;
  const int K = sh ? a.Is : a.I, h0 = sh ? a.F : start;
  for (int r = (int)(threadIdx.x >> 6); r < count; r += 4) {
    float* row = a.hbuf + (int64_t)(h0 + r) * a.hstride;
    quant_row<FMT>(K, [&](int g, float (&x)[8]) { load_f32x8(row + 8 * g, x); },
                   [&](int g, const float (&q)[8], float d) {
                     *(float4*)(row + 8 * g) = make_float4(d * q[0], d * q[1], d * q[2], d * q[3]);
                     *(float4*)(row + 8 * g + 4) = make_float4(d * q[4], d * q[5], d * q[6], d * q[7]);
                   });
  }
}

// ---------------------------------------------------------------- test entry
// rows -> int8 codes [rows][cols] and d [rows][cols / block]
template <int FMT>
__global__ __launch_bounds__(256) void k_actq_codes(const void* x, int xbf, int64_t rows, int cols, int8_t* codes,
                                                    float* dout) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  constexpr int BG = FMT == HX_Q8_0 ? 4 : 32;   // groups of 8 per block
  int8_t* cr = codes + r * cols;
  float* dr = dout + r * (cols / (8 * BG));
  auto emit = [&](int g, const float (&q)[8], float d) {
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      lo |= ((uint32_t)(int)q[j] & 0xffu) << (8 * j);
      hi |= ((uint32_t)(int)q[4 + j] & 0xffu) << (8 * j);
    }
    *(uint2*)(cr + 8 * g) = make_uint2(lo, hi);
    if (g % BG == 0) dr[g / BG] = d;
  };
  if (xbf) {
    const uint16_t* src = (const uint16_t*)x + r * cols;
    quant_row<FMT>(cols, [&](int g, float (&v)[8]) { load_bf16x8(src + 8 * g, v); }, emit);
  } else {
    const float* src = (const float*)x + r * cols;
    quant_row<FMT>(cols, [&](int g, float (&v)[8]) { load_f32x8(src + 8 * g, v); }, emit);
  }
}

// ---------------------------------------------------------------- launchers
// the vec_dot type of a weight format: Q8_0 blocks for Q8_0, Q8_K otherwise
#define HX_VD_SWITCH(FMT_VAL, CALL) \
  switch (FMT_VAL) {                \
    case HX_Q8_0: CALL(HX_Q8_0); break; \
    case HX_Q4_K: case HX_Q6_K: CALL(HX_Q4_K); break; \
    default: return hipErrorInvalidValue; \
  }

bool gguf_fmt(int fmt) { return fmt == HX_Q8_0 || fmt == HX_Q4_K || fmt == HX_Q6_K; }

hipError_t launch_xq_fq(const ExpertArgs& a, hipStream_t s) {
  const dim3 g((unsigned)((a.T + 3) / 4), (unsigned)((a.H + 511) / 512));
  const int nat = xh_natural(a.gate.fmt) ? 1 : 0;
#define L(F) hipLaunchKernelGGL((k_xq_fq<F>), g, dim3(256), 0, s, a, nat)
  HX_VD_SWITCH(a.gate.fmt, L)
#undef L
  return hipGetLastError();
}

hipError_t launch_hq_fq(const ExpertArgs& a, int ntiles, hipStream_t s) {
  const dim3 g((unsigned)ntiles, (unsigned)(HX_TILE_M / 4));
#define L(F) hipLaunchKernelGGL((k_hq_fq<F>), g, dim3(256), 0, s, a)
  HX_VD_SWITCH(a.down.fmt, L)
#undef L
  return hipGetLastError();
}

hipError_t launch_xq_f32(const ExpertArgs& a, hipStream_t s) {
  const dim3 g((unsigned)((a.T + 3) / 4));
#define L(F) hipLaunchKernelGGL((k_xq_f32<F>), g, dim3(256), 0, s, a)
  HX_VD_SWITCH(a.gate.fmt, L)
#undef L
  return hipGetLastError();
}

hipError_t launch_hq_f32(const ExpertArgs& a, hipStream_t s) {
  const dim3 g((unsigned)a.max_slots);
#define L(F) hipLaunchKernelGGL((k_hq_f32<F>), g, dim3(256), 0, s, a)
  HX_VD_SWITCH(a.down.fmt, L)
#undef L
  return hipGetLastError();
}

hipError_t launch_actq_codes(int wfmt, const void* x, bool xbf, int64_t rows, int cols, int8_t* codes, float* d,
                             hipStream_t s) {
  const dim3 g((unsigned)((rows + 3) / 4));
#define L(F) hipLaunchKernelGGL((k_actq_codes<F>), g, dim3(256), 0, s, x, xbf ? 1 : 0, rows, cols, codes, d)
  HX_VD_SWITCH(wfmt, L)
#undef L
  return hipGetLastError();
}

}  // namespace hx
