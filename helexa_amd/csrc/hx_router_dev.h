// Router GEMV core shared by the routing and decode kernels.
//
// Canonical order of a router logit (restated by the CPU checker): the H inputs
// are cut into groups of 8 (the last may be shorter); group g belongs to lane
// g % 64; each lane runs an fmaf chain over its groups in increasing order; the
// 64 partials are combined by the xor butterfly 32,16,8,4,2,1; the sum is
// rounded to the activation dtype (candle's Linear returns the input dtype,
// crates/neuron/src/harness/arch/qwen3_5/moe.rs:134); then the optional bias.
#pragma once
#include "hx_internal.h"

namespace hx {

template <bool BF>
HX_DEV void load8(const void* base, int64_t row_elems, int64_t row, int h0, int H, bool vec, float* out) {
  if (vec) {
    if (BF) {
      const uint4 q = *(const uint4*)((const uint16_t*)base + row * row_elems + h0);
      const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int j = 0; j < 4; j++) {
        out[2 * j] = __uint_as_float(w[j] << 16);
        out[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
      }
    } else {
      const float4* p = (const float4*)((const float*)base + row * row_elems + h0);
      const float4 a = p[0], b = p[1];
      out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
      out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const int h = h0 + i;
      out[i] = h < H ? (BF ? bf16_to_f32(((const uint16_t*)base)[row * row_elems + h])
                           : ((const float*)base)[row * row_elems + h])
                     : 0.0f;
    }
  }
}

// The decoder RMSNorm on the bf16 token rows a wave holds in registers (group
// g = lane + 64 i of token t in xr[t][i]): per token, an fmaf chain of squares
// over the lane's groups in order, the 64-lane butterfly, inv = 1 / sqrt(ss / H
// + eps), then x * inv * (1 + w) rounded to bf16 in place. Every wave of the
// router does the same arithmetic, so all hold the same rows; wave 0 of
// workgroup 0 writes them to xn_out.
template <int TT, int NG>
HX_DEV void rmsnorm_regs(const RouterArgs& a, uint32_t (&xr)[TT][NG][4], int t0,
                         bool writer = blockIdx.x == 0 && threadIdx.x < 64) {
  const int lane = lane_id(), H = a.H, G = H / 8;
  float w[NG][8];
#pragma unroll
  for (int i = 0; i < NG; i++) {
    const int g = min(lane + 64 * i, G - 1);
    const float4 w0 = *(const float4*)(a.norm_w + 8 * g), w1 = *(const float4*)(a.norm_w + 8 * g + 4);
    w[i][0] = w0.x; w[i][1] = w0.y; w[i][2] = w0.z; w[i][3] = w0.w;
    w[i][4] = w1.x; w[i][5] = w1.y; w[i][6] = w1.z; w[i][7] = w1.w;
  }
  // the tokens' sums of squares, their wave reductions and scales in three
  // passes, so the TT dependent chains run side by side; per token the same
  // operations in the same order as for one token
  float ss[TT], inv[TT];
#pragma unroll
  for (int t = 0; t < TT; t++) {
    ss[t] = 0.f;
#pragma unroll
    for (int i = 0; i < NG; i++) {
      if (lane + 64 * i >= G) break;
#pragma unroll
      for (int q = 0; q < 8; q++) {
        const float v = __uint_as_float(q & 1 ? xr[t][i][q / 2] & 0xffff0000u : xr[t][i][q / 2] << 16);
        ss[t] = __builtin_fmaf(v, v, ss[t]);
      }
    }
  }
#pragma unroll
  for (int t = 0; t < TT; t++) ss[t] = wave_sum<64>(ss[t]);
#pragma unroll
  for (int t = 0; t < TT; t++) inv[t] = 1.0f / sqrtf(ss[t] / (float)H + a.eps);
#pragma unroll
  for (int t = 0; t < TT; t++) {
#pragma unroll
    for (int i = 0; i < NG; i++) {
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const float lo = __uint_as_float(xr[t][i][q] << 16) * inv[t] * (1.0f + w[i][2 * q]);
        const float hi = __uint_as_float(xr[t][i][q] & 0xffff0000u) * inv[t] * (1.0f + w[i][2 * q + 1]);
        xr[t][i][q] = (uint32_t)f32_to_bf16(lo) | ((uint32_t)f32_to_bf16(hi) << 16);
      }
      if (writer && t0 + t < a.T && lane + 64 * i < G)
        *(uint4*)(a.xn_out + (int64_t)(t0 + t) * H + 8 * (lane + 64 * i)) =
            make_uint4(xr[t][i][0], xr[t][i][1], xr[t][i][2], xr[t][i][3]);
    }
  }
}

// One wave: logits of tokens t0 .. t0+TT-1 for router rows e0 .. e0+TE-1, for
// H % 8 == 0 and at most 64 * NG groups of 8. Every load of the wave is issued
// before the first multiply-add (addresses are clamped into range and the
// values of out-of-range groups, rows and tokens replaced by zeros afterwards),
// so a wave waits for memory once. Same arithmetic order as the loop version.
template <bool XBF, bool RBF, int TT, int TE, int NG>
HX_DEV void router_rows_u(const RouterArgs& a, int e0, int t0) {
  constexpr int RW = RBF ? 4 : 8, XW = XBF ? 4 : 8;   // dwords per group of 8 values
  const int lane = lane_id();
  const int H = a.H, G = H / 8;
  uint32_t wr[TE][NG][RW], xr[TT][NG][XW];
#pragma unroll
  for (int i = 0; i < NG; i++) {
    const int g = min(lane + 64 * i, G - 1);
#pragma unroll
    for (int j = 0; j < TE; j++) {
      const int64_t row = min(e0 + j, a.E1 - 1);
      const uint4* p = (const uint4*)((const uint8_t*)a.R + (row * H + 8 * g) * (RBF ? 2 : 4));
#pragma unroll
      for (int q = 0; q < RW / 4; q++) {
        const uint4 v = p[q];
        wr[j][i][4 * q] = v.x; wr[j][i][4 * q + 1] = v.y; wr[j][i][4 * q + 2] = v.z; wr[j][i][4 * q + 3] = v.w;
      }
    }
#pragma unroll
    for (int t = 0; t < TT; t++) {
      const int64_t tok = min(t0 + t, a.T - 1);
      const uint4* p = (const uint4*)((const uint8_t*)a.x + (tok * H + 8 * g) * (XBF ? 2 : 4));
#pragma unroll
      for (int q = 0; q < XW / 4; q++) {
        const uint4 v = p[q];
        xr[t][i][4 * q] = v.x; xr[t][i][4 * q + 1] = v.y; xr[t][i][4 * q + 2] = v.z; xr[t][i][4 * q + 3] = v.w;
      }
    }
  }
  if constexpr (XBF) {
    if (a.norm_w) rmsnorm_regs<TT, NG>(a, xr, t0);
  }
  float acc[TT][TE];
#pragma unroll
  for (int t = 0; t < TT; t++)
#pragma unroll
    for (int j = 0; j < TE; j++) acc[t][j] = 0.0f;
#pragma unroll
  for (int i = 0; i < NG; i++) {
    if (lane + 64 * i >= G) break;   // this lane's remaining groups are past the end
#pragma unroll
    for (int q = 0; q < 8; q++) {
#pragma unroll
      for (int t = 0; t < TT; t++) {
        const float xv = XBF ? __uint_as_float(q & 1 ? xr[t][i][q / 2] & 0xffff0000u : xr[t][i][q / 2] << 16)
                             : __uint_as_float(xr[t][i][q]);
#pragma unroll
        for (int j = 0; j < TE; j++) {
          const float wv = RBF ? __uint_as_float(q & 1 ? wr[j][i][q / 2] & 0xffff0000u : wr[j][i][q / 2] << 16)
                               : __uint_as_float(wr[j][i][q]);
          acc[t][j] = __builtin_fmaf(xv, wv, acc[t][j]);
        }
      }
    }
  }
#pragma unroll
  for (int t = 0; t < TT; t++)
#pragma unroll
    for (int j = 0; j < TE; j++) {
      float v = wave_sum<64>(acc[t][j]);
      const int tt = t0 + t, e = e0 + j;
      if (lane == t * TE + j && tt < a.T && e < a.E1) {
        if (XBF) v = bf16_to_f32(f32_to_bf16(v));
        if (a.bias && e < a.E) v = v + a.bias[e];
        a.logits[(int64_t)tt * a.E1 + e] = v;
      }
    }
}

// router_rows_u for bf16 tokens with the decoder RMSNorm and TT > 1, all four
// waves of the workgroup taking part: wave w normalises tokens w, w + 4, ..
// (the arithmetic of rmsnorm_regs for one token, so the bits the record waves
// compute) into LDS, and after one barrier every wave reads the TT normalised
// rows from there for its router rows. Each token is normalised once per
// workgroup instead of once per wave (the waves run one per SIMD, so the
// repeated normalisation was serial VALU work on the kernel's critical path).
// Same multiply-add order per logit as router_rows_u.
// Tokens t0 .. t0 + TT - 1; writer: this workgroup writes the normalised rows.
template <bool RBF, int TT, int TE, int NG>
HX_DEV void router_rows_norm(const RouterArgs& a, int e0, int t0, bool writer) {
  constexpr int RW = RBF ? 4 : 8, TW = (TT + 3) / 4;
  __shared__ uint4 sxn[TT][NG][64];   // normalised rows, canonical layout
  const int lane = lane_id(), wave = threadIdx.x >> 6;
  const int H = a.H, G = H / 8;
  uint32_t wr[TE][NG][RW], xr[TW][NG][4];
#pragma unroll
  for (int i = 0; i < NG; i++) {
    const int g = min(lane + 64 * i, G - 1);
#pragma unroll
    for (int j = 0; j < TE; j++) {
      const int64_t row = min(e0 + j, a.E1 - 1);
      const uint4* p = (const uint4*)((const uint8_t*)a.R + (row * H + 8 * g) * (RBF ? 2 : 4));
#pragma unroll
      for (int q = 0; q < RW / 4; q++) {
        const uint4 v = p[q];
        wr[j][i][4 * q] = v.x; wr[j][i][4 * q + 1] = v.y; wr[j][i][4 * q + 2] = v.z; wr[j][i][4 * q + 3] = v.w;
      }
    }
#pragma unroll
    for (int s = 0; s < TW; s++) {
      const int64_t tok = min(t0 + wave + 4 * s, a.T - 1);
      const uint4 v = *(const uint4*)((const uint16_t*)a.x + tok * H + 8 * g);
      xr[s][i][0] = v.x; xr[s][i][1] = v.y; xr[s][i][2] = v.z; xr[s][i][3] = v.w;
    }
  }
#pragma unroll
  for (int s = 0; s < TW; s++) {
    const int t = wave + 4 * s;
    if (t >= TT) continue;   // wave-uniform
    uint32_t one[1][NG][4];
#pragma unroll
    for (int i = 0; i < NG; i++)
#pragma unroll
      for (int q = 0; q < 4; q++) one[0][i][q] = xr[s][i][q];
    rmsnorm_regs<1, NG>(a, one, t0 + t, writer && t0 + t < a.T);
#pragma unroll
    for (int i = 0; i < NG; i++) sxn[t][i][lane] = make_uint4(one[0][i][0], one[0][i][1], one[0][i][2], one[0][i][3]);
  }
  __syncthreads();
  float acc[TT][TE];
#pragma unroll
  for (int t = 0; t < TT; t++)
#pragma unroll
    for (int j = 0; j < TE; j++) acc[t][j] = 0.0f;
#pragma unroll
  for (int i = 0; i < NG; i++) {
    if (lane + 64 * i >= G) break;   // this lane's remaining groups are past the end
    uint32_t xg[TT][4];
#pragma unroll
    for (int t = 0; t < TT; t++) {
      const uint4 v = sxn[t][i][lane];
      xg[t][0] = v.x; xg[t][1] = v.y; xg[t][2] = v.z; xg[t][3] = v.w;
    }
#pragma unroll
    for (int q = 0; q < 8; q++) {
#pragma unroll
      for (int t = 0; t < TT; t++) {
        const float xv = __uint_as_float(q & 1 ? xg[t][q / 2] & 0xffff0000u : xg[t][q / 2] << 16);
#pragma unroll
        for (int j = 0; j < TE; j++) {
          const float wv = RBF ? __uint_as_float(q & 1 ? wr[j][i][q / 2] & 0xffff0000u : wr[j][i][q / 2] << 16)
                               : __uint_as_float(wr[j][i][q]);
          acc[t][j] = __builtin_fmaf(xv, wv, acc[t][j]);
        }
      }
    }
  }
#pragma unroll
  for (int t = 0; t < TT; t++)
#pragma unroll
    for (int j = 0; j < TE; j++) {
      float v = wave_sum<64>(acc[t][j]);
      const int e = e0 + j;
      if (lane == t * TE + j && t0 + t < a.T && e < a.E1) {
        v = bf16_to_f32(f32_to_bf16(v));
        if (a.bias && e < a.E) v = v + a.bias[e];
        a.logits[(int64_t)(t0 + t) * a.E1 + e] = v;
      }
    }
}

// One wave: logits of tokens t0 .. t0+7 for router rows e0 .. e0+7, for
// H % 8 == 0 and at most 64 * NG groups of 8; same arithmetic order as
// router_rows_u. The loads of group i + 1 are issued before the multiply-adds
// of group i; the 64 partial sums of a lane are combined by reduce_scatter64,
// after which lane l holds the logit of token t0 + l / 8, row e0 + l % 8.
template <bool XBF, bool RBF, int NG>
HX_DEV void router_tile88(const RouterArgs& a, int e0, int t0) {
  constexpr int RW = RBF ? 4 : 8, XW = XBF ? 4 : 8;   // dwords per group of 8 values
  const int lane = lane_id();
  const int H = a.H, G = H / 8;
  uint32_t wr[2][8][RW], xr[2][8][XW];
  auto load = [&](int i, int b) {
    const int g = min(lane + 64 * i, G - 1);
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const int64_t row = min(e0 + j, a.E1 - 1);
      const uint4* p = (const uint4*)((const uint8_t*)a.R + (row * H + 8 * g) * (RBF ? 2 : 4));
#pragma unroll
      for (int q = 0; q < RW / 4; q++) {
        const uint4 v = p[q];
        wr[b][j][4 * q] = v.x; wr[b][j][4 * q + 1] = v.y; wr[b][j][4 * q + 2] = v.z; wr[b][j][4 * q + 3] = v.w;
      }
    }
#pragma unroll
    for (int t = 0; t < 8; t++) {
      const int64_t tok = min(t0 + t, a.T - 1);
      const uint4* p = (const uint4*)((const uint8_t*)a.x + (tok * H + 8 * g) * (XBF ? 2 : 4));
#pragma unroll
      for (int q = 0; q < XW / 4; q++) {
        const uint4 v = p[q];
        xr[b][t][4 * q] = v.x; xr[b][t][4 * q + 1] = v.y; xr[b][t][4 * q + 2] = v.z; xr[b][t][4 * q + 3] = v.w;
      }
    }
  };
  float acc[64];
#pragma unroll
  for (int k = 0; k < 64; k++) acc[k] = 0.0f;
  load(0, 0);
#pragma unroll
  for (int i = 0; i < NG; i++) {
    const int b = i & 1;
    if (i + 1 < NG) load(i + 1, b ^ 1);
    if (lane + 64 * i < G) {   // lanes past the end have no group i
#pragma unroll
      for (int q = 0; q < 8; q++) {
        float wv[8];
#pragma unroll
        for (int j = 0; j < 8; j++)
          wv[j] = RBF ? __uint_as_float(q & 1 ? wr[b][j][q / 2] & 0xffff0000u : wr[b][j][q / 2] << 16)
                      : __uint_as_float(wr[b][j][q]);
#pragma unroll
        for (int t = 0; t < 8; t++) {
          const float xv = XBF ? __uint_as_float(q & 1 ? xr[b][t][q / 2] & 0xffff0000u : xr[b][t][q / 2] << 16)
                               : __uint_as_float(xr[b][t][q]);
#pragma unroll
          for (int j = 0; j < 8; j++) acc[8 * t + j] = __builtin_fmaf(xv, wv[j], acc[8 * t + j]);
        }
      }
    }
  }
  float v = reduce_scatter64(acc);
  const int tt = t0 + (lane >> 3), e = e0 + (lane & 7);
  if (tt < a.T && e < a.E1) {
    if (XBF) v = bf16_to_f32(f32_to_bf16(v));
    if (a.bias && e < a.E) v = v + a.bias[e];
    a.logits[(int64_t)tt * a.E1 + e] = v;
  }
}

// any H: groups loaded one at a time
template <bool XBF, bool RBF, int TT, int TE>
HX_DEV void router_rows_loop(const RouterArgs& a, int e0, int t0) {
  const int lane = lane_id();
  const int H = a.H, G = (H + 7) / 8;
  const bool vec = (H & 7) == 0;
  if (e0 >= a.E1) return;
  float acc[TT][TE];
#pragma unroll
  for (int i = 0; i < TT; i++)
#pragma unroll
    for (int j = 0; j < TE; j++) acc[i][j] = 0.0f;
  for (int g = lane; g < G; g += 64) {
    const int h0 = 8 * g;
    float xv[TT][8], wv[TE][8];
#pragma unroll
    for (int j = 0; j < TE; j++) {
      if (e0 + j < a.E1) load8<RBF>(a.R, H, e0 + j, h0, H, vec, wv[j]);
      else
#pragma unroll
        for (int q = 0; q < 8; q++) wv[j][q] = 0.0f;
    }
#pragma unroll
    for (int i = 0; i < TT; i++) {
      if (t0 + i < a.T) load8<XBF>(a.x, H, t0 + i, h0, H, vec, xv[i]);
      else
#pragma unroll
        for (int q = 0; q < 8; q++) xv[i][q] = 0.0f;
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

// one wave: logits of tokens t0 .. t0+TT-1 for router rows e0 .. e0+TE-1
template <bool XBF, bool RBF, int TT, int TE>
HX_DEV void router_rows(const RouterArgs& a, int e0, int t0) {
  if (e0 >= a.E1) return;
  if ((a.H & 7) == 0) {
    const int G = a.H / 8;
    if (G <= 64) { router_rows_u<XBF, RBF, TT, TE, 1>(a, e0, t0); return; }
    if (G <= 128) { router_rows_u<XBF, RBF, TT, TE, 2>(a, e0, t0); return; }
    if (G <= 256) { router_rows_u<XBF, RBF, TT, TE, 4>(a, e0, t0); return; }
  }
  router_rows_loop<XBF, RBF, TT, TE>(a, e0, t0);
}

}  // namespace hx
