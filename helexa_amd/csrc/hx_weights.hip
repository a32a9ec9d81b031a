// Weight preparation on the device: GGUF quantiser (the ISQ step), dequantiser,
// repack of GGUF rows into the kernels' planar layouts; plus the decoder-layer
// RMSNorm and residual add.
//
// Reference: quantize_parallel / quantize_blocks
// (crates/neuron/src/harness/tp/isq.rs:39-113): f32 rows, last dim tiled by the
// block size, blocks independent. The per-block search here is our own
// (documented in the quantiser below) and is byte-identical to the library's
// CPU quantiser; Qwen3_5RmsNorm (crates/neuron/src/harness/arch/qwen3_5/rmsnorm.rs:67-80).
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

HX_DEV int nearest_int(float v) { return (int)__builtin_rintf(v); }

HX_DEV void st_u16(uint8_t* p, uint16_t v) {
  p[0] = (uint8_t)(v & 0xff);
  p[1] = (uint8_t)(v >> 8);
}
HX_DEV uint16_t ld_u16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

// Q8_0: d = amax / 127, q = round-to-nearest-even(x / d)
HX_DEV void qz_q8_0(const float* x, uint8_t* b) {
  float amax = 0.0f;
  for (int j = 0; j < 32; j++) {
    float a = fabsf(x[j]);
    if (a > amax) amax = a;
  }
  float d = amax / 127.0f;
  float id = d != 0.0f ? 1.0f / d : 0.0f;
  st_u16(b, f32_to_f16(d));
  for (int j = 0; j < 32; j++) {
    int q = nearest_int(x[j] * id);
    q = q > 127 ? 127 : (q < -127 ? -127 : q);
    b[2 + j] = (uint8_t)(int8_t)q;
  }
}

// Q4_K: per 32-element sub-block, min = min(0, min x), scale = (max - min) / 15;
// the 8 scales and 8 mins quantised to 6 bits against their maxima; then each
// element re-fitted to 4 bits with the stored (f16, 6-bit) scale and min.
HX_DEV void qz_q4_k(const float* x, uint8_t* b) {
  float scale[8], mins[8];
  float max_scale = 0.0f, max_min = 0.0f;
  for (int j = 0; j < 8; j++) {
    float mn = 0.0f, mx = x[32 * j];
    for (int l = 0; l < 32; l++) {
      float v = x[32 * j + l];
      if (v < mn) mn = v;
      if (v > mx) mx = v;
    }
    scale[j] = (mx - mn) / 15.0f;
    mins[j] = -mn;
    if (scale[j] > max_scale) max_scale = scale[j];
    if (mins[j] > max_min) max_min = mins[j];
  }
  float inv_scale = max_scale > 0.0f ? 63.0f / max_scale : 0.0f;
  float inv_min = max_min > 0.0f ? 63.0f / max_min : 0.0f;
  uint8_t ls[8], lm[8];
  for (int j = 0; j < 8; j++) {
    int a = nearest_int(inv_scale * scale[j]), m = nearest_int(inv_min * mins[j]);
    ls[j] = (uint8_t)(a > 63 ? 63 : a);
    lm[j] = (uint8_t)(m > 63 ? 63 : m);
  }
  uint16_t dh = f32_to_f16(max_scale / 63.0f), mh = f32_to_f16(max_min / 63.0f);
  st_u16(b, dh);
  st_u16(b + 2, mh);
  uint8_t* s = b + 4;
  for (int j = 0; j < 4; j++) {
    s[j] = (uint8_t)((ls[j] & 63) | ((ls[j + 4] >> 4) << 6));
    s[j + 4] = (uint8_t)((lm[j] & 63) | ((lm[j + 4] >> 4) << 6));
    s[j + 8] = (uint8_t)((ls[j + 4] & 0xF) | ((lm[j + 4] & 0xF) << 4));
  }
  float d = f16_to_f32(dh), dmin = f16_to_f32(mh);
  uint8_t* qs = b + 16;
  for (int c = 0; c < 4; c++) {
    float dd0 = d * (float)ls[2 * c], dm0 = dmin * (float)lm[2 * c];
    float dd1 = d * (float)ls[2 * c + 1], dm1 = dmin * (float)lm[2 * c + 1];
    for (int l = 0; l < 32; l++) {
      int v0 = 0, v1 = 0;
      if (dd0 != 0.0f) {
        v0 = nearest_int((x[64 * c + l] + dm0) / dd0);
        v0 = v0 < 0 ? 0 : (v0 > 15 ? 15 : v0);
      }
      if (dd1 != 0.0f) {
        v1 = nearest_int((x[64 * c + 32 + l] + dm1) / dd1);
        v1 = v1 < 0 ? 0 : (v1 > 15 ? 15 : v1);
      }
      qs[32 * c + l] = (uint8_t)(v0 | (v1 << 4));
    }
  }
}

// Q6_K: per 16-element sub-block, scale = (signed max-|x| element) / -32; the 16
// scales quantised to int8 against the largest-|.| one (-128 / max); elements
// re-fitted to [-32, 31] with the stored scales.
HX_DEV void qz_q6_k(const float* x, uint8_t* b) {
  float scale[16];
  float max_scale = 0.0f, max_abs_scale = 0.0f;
  for (int i = 0; i < 16; i++) {
    float vmax = 0.0f, amax = 0.0f;
    for (int l = 0; l < 16; l++) {
      float v = x[16 * i + l], a = fabsf(v);
      if (a > amax) {
        amax = a;
        vmax = v;
      }
    }
    scale[i] = vmax != 0.0f ? vmax / -32.0f : 0.0f;
    float as = fabsf(scale[i]);
    if (as > max_abs_scale) {
      max_abs_scale = as;
      max_scale = scale[i];
    }
  }
  float iscale = max_scale != 0.0f ? -128.0f / max_scale : 0.0f;
  int8_t sc[16];
  for (int i = 0; i < 16; i++) {
    int v = nearest_int(iscale * scale[i]);
    v = v > 127 ? 127 : (v < -128 ? -128 : v);
    sc[i] = (int8_t)v;
  }
  uint16_t dh = f32_to_f16(iscale != 0.0f ? 1.0f / iscale : 0.0f);
  float d = f16_to_f32(dh);
  uint8_t* ql = b;
  uint8_t* qh = b + 128;
  for (int n = 0; n < 2; n++) {
    for (int l = 0; l < 32; l++) {
      uint8_t q[4];
      for (int s = 0; s < 4; s++) {
        int e = 128 * n + 32 * s + l;
        float di = d * (float)sc[e / 16];
        int v = 0;
        if (di != 0.0f) {
          v = nearest_int(x[e] / di);
          v = v < -32 ? -32 : (v > 31 ? 31 : v);
        }
        q[s] = (uint8_t)(v + 32);
      }
      ql[64 * n + l] = (uint8_t)((q[0] & 0xF) | ((q[2] & 0xF) << 4));
      ql[64 * n + 32 + l] = (uint8_t)((q[1] & 0xF) | ((q[3] & 0xF) << 4));
      qh[32 * n + l] = (uint8_t)((q[0] >> 4) | ((q[1] >> 4) << 2) | ((q[2] >> 4) << 4) | ((q[3] >> 4) << 6));
    }
  }
  for (int i = 0; i < 16; i++) b[192 + i] = (uint8_t)sc[i];
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
  uint8_t* ql = mat + r * (K / 2) + j * 128;
  uint8_t* qh = mat + rows * (K / 2) + r * (K / 4) + j * 64;
  uint8_t* sc = mat + rows * (K / 2 + K / 4) + r * (K / 16) + j * 16;
  uint8_t* d = mat + rows * (K / 2 + K / 4 + K / 16) + (r * nb_row + j) * 2;
  for (int i = 0; i < 128; i++) ql[i] = s[i];
  for (int i = 0; i < 64; i++) qh[i] = s[128 + i];
  for (int i = 0; i < 16; i++) sc[i] = s[192 + i];
  d[0] = s[208];
  d[1] = s[209];
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
