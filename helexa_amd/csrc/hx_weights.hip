// Weight preparation on the device: GGUF quantiser (the ISQ step), dequantiser,
// repack of GGUF rows into the kernels' planar layouts; plus the decoder-layer
// RMSNorm and residual add.
//
// Reference: quantize_parallel / quantize_blocks
// (crates/neuron/src/harness/tp/isq.rs:39-113): f32 rows, last dim tiled by the
// block size, blocks independent, each quantised by candle's from_float block
// rule (restated below); Qwen3_5RmsNorm
// (crates/neuron/src/harness/arch/qwen3_5/rmsnorm.rs:67-80).
#include "hx_internal.h"

namespace hx {

int64_t gguf_block_elems(int fmt) {
  switch (fmt) {
    case HX_F32: case HX_F16: case HX_BF16: return 1;
    case HX_Q8_0: return 32;
    case HX_Q4_K: case HX_Q6_K: return 256;
    default: return 0;
  }
}

int64_t gguf_block_bytes(int fmt) {
  switch (fmt) {
    case HX_F32: return 4;
    case HX_F16: case HX_BF16: return 2;
    case HX_Q8_0: return 34;
    case HX_Q4_K: return 144;
    case HX_Q6_K: return 210;
    default: return 0;
  }
}

HX_DEV void st_u16(uint8_t* p, uint16_t v) {
  p[0] = (uint8_t)(v & 0xff);
  p[1] = (uint8_t)(v >> 8);
}
HX_DEV uint16_t ld_u16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

// ---------------------------------------------------------------- quantiser
// The block rules of candle's GgmlType::from_float, which quantize_parallel
// calls per block (isq.rs:98, 104-112; isq.rs:1-19 and 123-161 hold it
// byte-identical to candle's QTensor::quantize). candle's k_quants port of
// ggml's first k_quants.c reference quantisers, restated from the published
// algorithms: one thread per block, every float operation in the published
// order (no contraction), so the bytes equal the CPU restatement's.

// candle's nearest_int: f32::round (half away from zero), then Rust's
// saturating float -> i32 cast (NaN -> 0)
HX_DEV int rs_nearest(float v) {
  const float r = roundf(v);
  if (r != r) return 0;
  if (r >= 2147483648.0f) return 2147483647;
  if (r < -2147483648.0f) return -2147483647 - 1;
  return (int)r;
}
HX_DEV int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

// Q8_0 (BlockQ8_0::from_float): d = amax / 127, q = (i8)round(x * (1 / d))
HX_DEV void qz_q8_0(const float* x, uint8_t* b) {
  float amax = 0.0f;
  for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(x[j]));
  const float d = amax / 127.0f;
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  st_u16(b, f32_to_f16(d));
  for (int j = 0; j < 32; j++) {
    const float r = roundf(x[j] * id);   // Rust `as i8`: saturating, NaN -> 0
    const int q = r != r ? 0 : (r >= 127.0f ? 127 : (r <= -128.0f ? -128 : (int)r));
    b[2 + j] = (uint8_t)(int8_t)q;
  }
}

// make_qkx1_quants(nmax, ntry, x[n]) -> (scale, -min): codes
// clamp(round((x - min) / scale), 0, nmax) alternated with the least-squares
// scale and the mean-residual min (<= 0), from min = min(0, min x) and
// scale = (max - min) / nmax, until the codes stop changing or ntry rounds
HX_DEV void make_qkx1(const float* x, int n, int nmax, int ntry, float& scale_out, float& min_out) {
  float mn = x[0], mx = x[0];
  for (int i = 1; i < n; i++) {
    const float v = x[i];
    mn = v < mn ? v : mn;
    mx = v > mx ? v : mx;
  }
  if (mx == mn) {
    scale_out = 0.0f;
    min_out = 0.0f;
    return;
  }
  if (mn > 0.0f) mn = 0.0f;
  float iscale = (float)nmax / (mx - mn);
  float scale = 1.0f / iscale;
  uint8_t L[32];
  for (int i = 0; i < n; i++) L[i] = 0;
  for (int t = 0; t < ntry; t++) {
    float sumlx = 0.0f;
    int suml2 = 0;
    bool changed = false;
    for (int i = 0; i < n; i++) {
      const int li = clampi(rs_nearest(iscale * (x[i] - mn)), 0, nmax);
      if ((uint8_t)li != L[i]) {
        L[i] = (uint8_t)li;
        changed = true;
      }
      sumlx += (x[i] - mn) * (float)li;
      suml2 += li * li;
    }
    scale = sumlx / (float)suml2;
    float sum = -0.0f;
    for (int i = 0; i < n; i++) sum += x[i] - scale * (float)L[i];
    mn = sum / (float)n;
    if (mn > 0.0f) mn = 0.0f;
    iscale = 1.0f / scale;
    if (!changed) break;
  }
  scale_out = scale;
  min_out = -mn;
}

// Q4_K (BlockQ4K::from_float): make_qkx1_quants(15, 5) per 32 elements; scales
// and mins to 6 bits against their maxima; codes re-fitted with the stored ones
HX_DEV void qz_q4_k(const float* x, uint8_t* b) {
  float scales[8], mins[8];
  for (int j = 0; j < 8; j++) make_qkx1(x + 32 * j, 32, 15, 5, scales[j], mins[j]);
  float max_scale = 0.0f, max_min = 0.0f;
  for (int j = 0; j < 8; j++) {
    max_scale = fmaxf(scales[j], max_scale);
    max_min = fmaxf(mins[j], max_min);
  }
  const float inv_scale = max_scale > 0.0f ? 63.0f / max_scale : 0.0f;
  const float inv_min = max_min > 0.0f ? 63.0f / max_min : 0.0f;
  uint8_t s[12];
  for (int j = 0; j < 12; j++) s[j] = 0;
  for (int j = 0; j < 8; j++) {
    const int a = rs_nearest(inv_scale * scales[j]), m = rs_nearest(inv_min * mins[j]);
    const uint8_t ls = (uint8_t)(a < 63 ? a : 63), lm = (uint8_t)(m < 63 ? m : 63);
    if (j < 4) {
      s[j] = ls;
      s[j + 4] = lm;
    } else {
      s[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
      s[j - 4] |= (uint8_t)((ls >> 4) << 6);
      s[j] |= (uint8_t)((lm >> 4) << 6);
    }
  }
  const uint16_t dh = f32_to_f16(max_scale / 63.0f), mh = f32_to_f16(max_min / 63.0f);
  st_u16(b, dh);
  st_u16(b + 2, mh);
  for (int j = 0; j < 12; j++) b[4 + j] = s[j];
  const float d = f16_to_f32(dh), dmin = f16_to_f32(mh);
  uint8_t* qs = b + 16;
  for (int c = 0; c < 4; c++) {
    int code[2][32];
    for (int h = 0; h < 2; h++) {
      const int j = 2 * c + h;
      int sc, m;
      if (j < 4) {
        sc = s[j] & 63;
        m = s[j + 4] & 63;
      } else {
        sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
        m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
      }
      const float dd = d * (float)sc, dm = dmin * (float)m;
      for (int l = 0; l < 32; l++)
        code[h][l] = dd == 0.0f ? 0 : clampi(rs_nearest((x[32 * j + l] + dm) / dd), 0, 15);
    }
    for (int l = 0; l < 32; l++) qs[32 * c + l] = (uint8_t)(code[0][l] | (code[1][l] << 4));
  }
}

// make_qx_quants(n, nmax, x, L, rmse_type = 1), weights x^2: codes from the
// largest-|x| element, up to 3 rounds re-deriving them from the least-squares
// scale while the weighted fit improves, up to 5 rounds of single-code moves
// that improve it. Returns the scale; L holds code + nmax.
HX_DEV float make_qx(int n, int nmax, const float* x, int8_t* L) {
  float max = 0.0f, amax = 0.0f;
  for (int i = 0; i < n; i++) {
    const float ax = fabsf(x[i]);
    if (ax > amax) {
      amax = ax;
      max = x[i];
    }
  }
  if (amax == 0.0f) {
    for (int i = 0; i < n; i++) L[i] = 0;
    return 0.0f;
  }
  const float iscale = -(float)nmax / max;
  float sumlx = 0.0f, suml2 = 0.0f;
  for (int i = 0; i < n; i++) {
    const int l = clampi(rs_nearest(iscale * x[i]), -nmax, nmax - 1);
    L[i] = (int8_t)(l + nmax);
    const float w = x[i] * x[i];
    sumlx += w * x[i] * (float)l;
    suml2 += w * (float)l * (float)l;
  }
  float scale = sumlx / suml2;
  float best = scale * sumlx;
  for (int t = 0; t < 3; t++) {
    const float is = 1.0f / scale;
    float slx = 0.0f, sl2 = 0.0f;
    bool changed = false;
    for (int i = 0; i < n; i++) {
      const int l = clampi(rs_nearest(is * x[i]), -nmax, nmax - 1);
      if (l + nmax != (int)L[i]) changed = true;
      const float w = x[i] * x[i];
      slx += w * x[i] * (float)l;
      sl2 += w * (float)l * (float)l;
    }
    if (!changed || sl2 == 0.0f || slx * slx <= best * sl2) break;
    for (int i = 0; i < n; i++) L[i] = (int8_t)(nmax + clampi(rs_nearest(is * x[i]), -nmax, nmax - 1));
    sumlx = slx;
    suml2 = sl2;
    scale = sumlx / suml2;
    best = scale * sumlx;
  }
  for (int t = 0; t < 5; t++) {
    int n_changed = 0;
    for (int i = 0; i < n; i++) {
      const float w = x[i] * x[i];
      const int l = (int)L[i] - nmax;
      float slx = sumlx - w * x[i] * (float)l;
      if (slx > 0.0f) {
        float sl2 = suml2 - w * (float)l * (float)l;
        const int new_l = clampi(rs_nearest(x[i] * sl2 / slx), -nmax, nmax - 1);
        if (new_l != l) {
          slx += w * x[i] * (float)new_l;
          sl2 += w * (float)new_l * (float)new_l;
          if (sl2 > 0.0f && slx * slx * suml2 > sumlx * sumlx * sl2) {
            L[i] = (int8_t)(nmax + new_l);
            sumlx = slx;
            suml2 = sl2;
            scale = sumlx / suml2;
            best = scale * sumlx;
            n_changed++;
          }
        }
      }
    }
    if (!n_changed) break;
  }
  return scale;
}

// Q6_K (BlockQ6K::from_float): make_qx_quants(16, 32, rmse 1) per 16 elements;
// scales to int8 against -128 / (largest-|.| scale); codes re-fitted to [-32, 31]
HX_DEV void qz_q6_k(const float* x, uint8_t* b) {
  int8_t L[256];
  float scales[16];
  float max_scale = 0.0f, max_abs_scale = 0.0f;
  for (int ib = 0; ib < 16; ib++) {
    const float sc = make_qx(16, 32, x + 16 * ib, L + 16 * ib);
    scales[ib] = sc;
    if (fabsf(sc) > max_abs_scale) {
      max_abs_scale = fabsf(sc);
      max_scale = sc;
    }
  }
  const float iscale = -128.0f / max_scale;
  const uint16_t dh = f32_to_f16(1.0f / iscale);
  int8_t ysc[16];
  for (int i = 0; i < 16; i++) {
    const int v = rs_nearest(iscale * scales[i]);
    ysc[i] = (int8_t)(uint8_t)(v < 127 ? v : 127);
  }
  const float d = f16_to_f32(dh);
  for (int j = 0; j < 16; j++) {
    const float dj = d * (float)ysc[j];
    if (dj == 0.0f) continue;
    for (int l = 0; l < 16; l++) L[16 * j + l] = (int8_t)(clampi(rs_nearest(x[16 * j + l] / dj), -32, 31) + 32);
  }
  uint8_t* ql = b;
  uint8_t* qh = b + 128;
  for (int n = 0; n < 2; n++) {
    for (int l = 0; l < 32; l++) {
      const uint8_t q1 = (uint8_t)L[128 * n + l], q2 = (uint8_t)L[128 * n + 32 + l];
      const uint8_t q3 = (uint8_t)L[128 * n + 64 + l], q4 = (uint8_t)L[128 * n + 96 + l];
      ql[64 * n + l] = (uint8_t)((q1 & 0xF) | ((q3 & 0xF) << 4));
      ql[64 * n + 32 + l] = (uint8_t)((q2 & 0xF) | ((q4 & 0xF) << 4));
      qh[32 * n + l] = (uint8_t)(((q1 >> 4) & 3) | (((q2 >> 4) & 3) << 2) | (((q3 >> 4) & 3) << 4) |
                                 (((q4 >> 4) & 3) << 6));
    }
  }
  for (int i = 0; i < 16; i++) b[192 + i] = (uint8_t)ysc[i];
  st_u16(b + 208, dh);
}

template <int FMT>
__global__ __launch_bounds__(256) void k_quantize(const float* src, int64_t nblocks, uint8_t* dst) {
  const int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (b >= nblocks) return;
  if (FMT == HX_Q8_0) {
    float x[32];
    for (int j = 0; j < 32; j++) x[j] = src[b * 32 + j];
    qz_q8_0(x, dst + b * 34);
  } else if (FMT == HX_Q4_K) {
    qz_q4_k(src + b * 256, dst + b * 144);
  } else if (FMT == HX_Q6_K) {
    qz_q6_k(src + b * 256, dst + b * 210);
  } else if (FMT == HX_BF16) {
    uint16_t h = f32_to_bf16(src[b]);
    st_u16(dst + 2 * b, h);
  } else if (FMT == HX_F16) {
    st_u16(dst + 2 * b, f32_to_f16(src[b]));
  }
}

// ---------------------------------------------------------------- dequantiser
template <int FMT>
__global__ __launch_bounds__(256) void k_dequantize(const uint8_t* src, int64_t nblocks, float* dst) {
  const int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (b >= nblocks) return;
  if (FMT == HX_Q8_0) {
    const uint8_t* p = src + b * 34;
    float d = f16_to_f32(ld_u16(p));
    for (int j = 0; j < 32; j++) dst[b * 32 + j] = d * (float)(int8_t)p[2 + j];
  } else if (FMT == HX_Q4_K) {
    const uint8_t* p = src + b * 144;
    float d = f16_to_f32(ld_u16(p)), dmin = f16_to_f32(ld_u16(p + 2));
    const uint8_t* s = p + 4;
    for (int c = 0; c < 4; c++) {
      int sc[2], m[2];
      for (int h = 0; h < 2; h++) {
        int j = 2 * c + h;
        if (j < 4) {
          sc[h] = s[j] & 63;
          m[h] = s[j + 4] & 63;
        } else {
          sc[h] = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
          m[h] = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
        }
      }
      float d0 = d * (float)sc[0], m0 = dmin * (float)m[0], d1 = d * (float)sc[1], m1 = dmin * (float)m[1];
      for (int l = 0; l < 32; l++) {
        uint8_t q = p[16 + 32 * c + l];
        dst[b * 256 + 64 * c + l] = d0 * (float)(q & 0xF) - m0;
        dst[b * 256 + 64 * c + 32 + l] = d1 * (float)(q >> 4) - m1;
      }
    }
  } else if (FMT == HX_Q6_K) {
    const uint8_t* p = src + b * 210;
    const uint8_t* ql = p;
    const uint8_t* qh = p + 128;
    const int8_t* sc = (const int8_t*)(p + 192);
    float d = f16_to_f32(ld_u16(p + 208));
    for (int n = 0; n < 2; n++)
      for (int l = 0; l < 32; l++) {
        int is = l / 16;
        int q1 = (int)((ql[64 * n + l] & 0xF) | (((qh[32 * n + l] >> 0) & 3) << 4)) - 32;
        int q2 = (int)((ql[64 * n + l + 32] & 0xF) | (((qh[32 * n + l] >> 2) & 3) << 4)) - 32;
        int q3 = (int)((ql[64 * n + l] >> 4) | (((qh[32 * n + l] >> 4) & 3) << 4)) - 32;
        int q4 = (int)((ql[64 * n + l + 32] >> 4) | (((qh[32 * n + l] >> 6) & 3) << 4)) - 32;
        float* y = dst + b * 256 + 128 * n;
        y[l] = d * (float)sc[8 * n + is] * (float)q1;
        y[l + 32] = d * (float)sc[8 * n + is + 2] * (float)q2;
        y[l + 64] = d * (float)sc[8 * n + is + 4] * (float)q3;
        y[l + 96] = d * (float)sc[8 * n + is + 6] * (float)q4;
      }
  } else if (FMT == HX_BF16) {
    dst[b] = bf16_to_f32(ld_u16(src + 2 * b));
  } else if (FMT == HX_F16) {
    dst[b] = f16_to_f32(ld_u16(src + 2 * b));
  } else if (FMT == HX_F32) {
    dst[b] = ((const float*)src)[b];
  }
}

// ---------------------------------------------------------------- repack
// one thread per GGUF block of one [rows][K] matrix in a stack of `count`
__global__ __launch_bounds__(256) void k_repack_q8_0(const uint8_t* src, int64_t count, int64_t rows, int64_t K,
                                                     uint8_t* dst, int64_t dst_stride) {
  const int64_t nb_row = K / 32, nb_mat = rows * nb_row;
  const int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (b >= count * nb_mat) return;
  const int64_t m = b / nb_mat, r = (b % nb_mat) / nb_row, j = b % nb_row;
  const uint8_t* s = src + b * 34;
  uint8_t* mat = dst + m * dst_stride;
  uint8_t* qs = mat + r * K + j * 32;
  for (int i = 0; i < 32; i++) qs[i] = s[2 + i];
  uint8_t* d = mat + rows * K + (r * nb_row + j) * 2;
  d[0] = s[0];
  d[1] = s[1];
}

__global__ __launch_bounds__(256) void k_repack_q6_k(const uint8_t* src, int64_t count, int64_t rows, int64_t K,
                                                     uint8_t* dst, int64_t dst_stride) {
  const int64_t nb_row = K / 256, nb_mat = rows * nb_row;
  const int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (b >= count * nb_mat) return;
  const int64_t m = b / nb_mat, r = (b % nb_mat) / nb_row, j = b % nb_row;
  const uint8_t* s = src + b * 210;
  uint8_t* mat = dst + m * dst_stride;
  const int R = (int)rows, KK = (int)K, row = (int)r, o = (int)j;
  uint8_t* d = mat + rows * (K / 2 + K / 4 + K / 16) + (r * nb_row + j) * 2;
  // planes in the stored layout of q6k_at (pieces of 32, 32 and 16 bytes)
  for (int p = 0; p < 4; p++) {
    uint8_t* ql = (uint8_t*)q6k_ql(mat, R, KK, row, 128 * o + 32 * p);
    for (int i = 0; i < 32; i++) ql[i] = s[32 * p + i];
  }
  for (int p = 0; p < 2; p++) {
    uint8_t* qh = (uint8_t*)q6k_qh(mat, R, KK, row, 64 * o + 32 * p);
    for (int i = 0; i < 32; i++) qh[i] = s[128 + 32 * p + i];
  }
  uint8_t* sc = (uint8_t*)q6k_sc(mat, R, KK, row, 16 * o);
  for (int i = 0; i < 16; i++) sc[i] = s[192 + i];
  d[0] = s[208];
  d[1] = s[209];
}

// GGUF Q4_K rows -> the stored layout of q4k_sb: one thread per superblock
__global__ __launch_bounds__(256) void k_repack_q4_k(const uint8_t* src, int64_t count, int64_t rows, int64_t K,
                                                     uint8_t* dst, int64_t dst_stride) {
  const int64_t nb_row = K / 256, nb_mat = rows * nb_row;
  const int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (b >= count * nb_mat) return;
  const int64_t m = b / nb_mat, r = (b % nb_mat) / nb_row, j = b % nb_row;
  const uint8_t* s = src + b * 144;   // the caller's rows: any alignment
  uint8_t* d = (uint8_t*)q4k_sb(dst + m * dst_stride, (int)rows, (int)K, (int)r, (int)j);
  for (int i = 0; i < 144; i++) d[i] = s[i];
}

hipError_t launch_quantize(int fmt, const float* src, int64_t rows, int64_t cols, void* dst, hipStream_t s) {
  const int64_t nb = rows * (cols / gguf_block_elems(fmt));
  const dim3 grid((unsigned)((nb + 255) / 256));
  uint8_t* d = (uint8_t*)dst;
  switch (fmt) {
    case HX_Q8_0: hipLaunchKernelGGL(k_quantize<HX_Q8_0>, grid, dim3(256), 0, s, src, nb, d); break;
    case HX_Q4_K: hipLaunchKernelGGL(k_quantize<HX_Q4_K>, grid, dim3(256), 0, s, src, nb, d); break;
    case HX_Q6_K: hipLaunchKernelGGL(k_quantize<HX_Q6_K>, grid, dim3(256), 0, s, src, nb, d); break;
    case HX_BF16: hipLaunchKernelGGL(k_quantize<HX_BF16>, grid, dim3(256), 0, s, src, nb, d); break;
    case HX_F16: hipLaunchKernelGGL(k_quantize<HX_F16>, grid, dim3(256), 0, s, src, nb, d); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_dequantize(int fmt, const void* src, int64_t rows, int64_t cols, float* dst, hipStream_t s) {
  const int64_t nb = rows * (cols / gguf_block_elems(fmt));
  const dim3 grid((unsigned)((nb + 255) / 256));
  const uint8_t* p = (const uint8_t*)src;
  switch (fmt) {
    case HX_Q8_0: hipLaunchKernelGGL(k_dequantize<HX_Q8_0>, grid, dim3(256), 0, s, p, nb, dst); break;
    case HX_Q4_K: hipLaunchKernelGGL(k_dequantize<HX_Q4_K>, grid, dim3(256), 0, s, p, nb, dst); break;
    case HX_Q6_K: hipLaunchKernelGGL(k_dequantize<HX_Q6_K>, grid, dim3(256), 0, s, p, nb, dst); break;
    case HX_BF16: hipLaunchKernelGGL(k_dequantize<HX_BF16>, grid, dim3(256), 0, s, p, nb, dst); break;
    case HX_F16: hipLaunchKernelGGL(k_dequantize<HX_F16>, grid, dim3(256), 0, s, p, nb, dst); break;
    case HX_F32: hipLaunchKernelGGL(k_dequantize<HX_F32>, grid, dim3(256), 0, s, p, nb, dst); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_repack(int fmt, const void* src, int64_t count, int64_t rows, int64_t K, void* dst,
                         int64_t dst_stride, hipStream_t s) {
  const uint8_t* p = (const uint8_t*)src;
  uint8_t* d = (uint8_t*)dst;
  if (fmt == HX_Q8_0) {
    const int64_t nb = count * rows * (K / 32);
    hipLaunchKernelGGL(k_repack_q8_0, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0, s, p, count, rows, K, d,
                       dst_stride);
  } else if (fmt == HX_Q6_K) {
    const int64_t nb = count * rows * (K / 256);
    hipLaunchKernelGGL(k_repack_q6_k, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0, s, p, count, rows, K, d,
                       dst_stride);
  } else if (fmt == HX_Q4_K) {
    const int64_t nb = count * rows * (K / 256);
    hipLaunchKernelGGL(k_repack_q4_k, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0, s, p, count, rows, K, d,
                       dst_stride);
  } else {
    const int64_t packed = rows * (K / gguf_block_elems(fmt)) * gguf_block_bytes(fmt);
    return hipMemcpy2DAsync(d, dst_stride, p, packed, packed, count, hipMemcpyDeviceToDevice, s);
  }
  return hipGetLastError();
}

// ---------------------------------------------------------------- RMSNorm
// one block per token; f32 sum of squares (per-thread strided, then a fixed
// tree), y = x * rsqrt(mean + eps) * (1 + w) rounded to the activation dtype
__global__ __launch_bounds__(256) void k_rmsnorm(const void* x, bool bf, int64_t H, const float* w, float eps,
                                                 void* y) {
  __shared__ float red[256];
  const int64_t t = blockIdx.x;
  float ss = 0.f;
  for (int64_t i = threadIdx.x; i < H; i += 256) {
    float v = ld_act(x, t * H + i, bf);
    ss = __builtin_fmaf(v, v, ss);
  }
  red[threadIdx.x] = ss;
  __syncthreads();
  for (int off = 128; off >= 1; off >>= 1) {
    if ((int)threadIdx.x < off) red[threadIdx.x] += red[threadIdx.x + off];
    __syncthreads();
  }
  const float inv = 1.0f / sqrtf(red[0] / (float)H + eps);
  for (int64_t i = threadIdx.x; i < H; i += 256) {
    float v = ld_act(x, t * H + i, bf) * inv * (1.0f + w[i]);
    if (bf) ((uint16_t*)y)[t * H + i] = f32_to_bf16(v);
    else ((float*)y)[t * H + i] = v;
  }
}

__global__ __launch_bounds__(256) void k_residual_add(void* x, const void* y, bool bf, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  if (bf) {
    uint16_t* px = (uint16_t*)x;
    px[i] = f32_to_bf16(bf16_to_f32(px[i]) + bf16_to_f32(((const uint16_t*)y)[i]));
  } else {
    ((float*)x)[i] += ((const float*)y)[i];
  }
}

hipError_t launch_rmsnorm(const void* x, bool xbf, int64_t T, int64_t H, const float* w, float eps, void* y,
                          hipStream_t s) {
  hipLaunchKernelGGL(k_rmsnorm, dim3((unsigned)T), dim3(256), 0, s, x, xbf, H, w, eps, y);
  return hipGetLastError();
}

hipError_t launch_residual_add(void* x, const void* y, bool bf, int64_t n, hipStream_t s) {
  hipLaunchKernelGGL(k_residual_add, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, y, bf, n);
  return hipGetLastError();
}

}  // namespace hx
