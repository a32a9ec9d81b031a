// Device-side helpers shared by the hx_moe kernels (gfx950, wave64).
//
// Numeric contract for routing (restated independently by the CPU checker):
//   * router logit: the H inputs are cut into groups of 8 (the last may be
//     shorter); group g belongs to lane g % 64; each lane runs an fmaf chain
//     over its groups in increasing order; the 64 partials are combined by the
//     xor butterfly 32,16,8,4,2,1; the sum is rounded to the activation dtype.
//   * softmax: hx_expf below, lane-strided sum (expert e -> lane e % 64, in
//     increasing e) + the same butterfly, IEEE division.
//   * top-k: largest probability first, ties to the lower expert id.
//   * renormalisation: sequential sum in rank order, IEEE division.
// All kernels are compiled with -ffp-contract=off: no multiply-add is fused
// unless __builtin_fmaf is written.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define HX_DEV __device__ __forceinline__

namespace hx {

HX_DEV float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

HX_DEV uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// exact for every f16 value (normal, subnormal, inf, nan)
HX_DEV float f16_to_f32(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  if (e == 0) {
    float v = (float)m * 5.9604644775390625e-8f;
    return sign ? -v : v;
  }
  if (e == 31) return __uint_as_float(sign | 0x7f800000u | (m << 13));
  return __uint_as_float(sign | ((e + 112u) << 23) | (m << 13));
}

// round-to-nearest-even f32 -> f16 bits, subnormals kept, overflow -> inf
HX_DEV uint16_t f32_to_f16(float f) {
  uint32_t x = __float_as_uint(f);
  uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  uint32_t ax = x & 0x7fffffffu;
  if (ax > 0x7f800000u) return sign | 0x7e00u;
  if (ax >= 0x38800000u) {
    uint32_t m = ax + 0xfffu + ((ax >> 13) & 1u);
    m -= (112u << 23);
    if (m >= 0x0f800000u) return sign | 0x7c00u;
    return (uint16_t)(sign | (m >> 13));
  }
  float v = __uint_as_float(ax) * 16777216.0f;
  float q = (v + 8388608.0f) - 8388608.0f;
  return (uint16_t)(sign | (uint16_t)q);
}

// exp for the router softmax: Cody-Waite split of ln2 (0.693145751953125 +
// 1.42860682030941723212e-6, the Cephes constants), degree-7 Taylor
// polynomial in Horner form with fmaf, exact 2^n scaling. x < -87 -> 0,
// x > 88.5 -> +inf.
HX_DEV float expf_route(float x) {
  if (x != x) return x;
  if (x < -87.0f) return 0.0f;
  if (x > 88.5f) return __builtin_inff();
  float n = __builtin_rintf(x * 1.44269504088896341f);
  float r = __builtin_fmaf(n, -0.693145751953125f, x);
  r = __builtin_fmaf(n, -1.42860682030941723212e-6f, r);
  float p = 1.98412698412698413e-4f;
  p = __builtin_fmaf(p, r, 1.38888888888888889e-3f);
  p = __builtin_fmaf(p, r, 8.33333333333333333e-3f);
  p = __builtin_fmaf(p, r, 4.16666666666666667e-2f);
  p = __builtin_fmaf(p, r, 1.66666666666666667e-1f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  int ni = (int)n;
  if (ni > 127) return p * __uint_as_float((uint32_t)(127 + 127) << 23) * 2.0f;
  return p * __uint_as_float((uint32_t)(ni + 127) << 23);
}

HX_DEV float sigmoidf_(float v) { return 1.0f / (1.0f + __expf(-v)); }
HX_DEV float siluf_(float g) { return g / (1.0f + __expf(-g)); }

// xor butterfly over the low `width` lanes (width a power of two <= 64)
template <int WIDTH>
HX_DEV float wave_sum(float v) {
#pragma unroll
  for (int off = WIDTH / 2; off >= 1; off >>= 1) v = v + __shfl_xor(v, off, 64);
  return v;
}

HX_DEV unsigned long long wave_max_u64(unsigned long long v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    unsigned long long o = __shfl_xor(v, off, 64);
    v = o > v ? o : v;
  }
  return v;
}

HX_DEV int lane_id() { return (int)(threadIdx.x & 63); }

// DPP move of v from the lane picked by CTRL; rows outside ROWMASK keep v
template <int CTRL, int ROWMASK = 0xf>
HX_DEV int dpp_mov(int v) {
  return __builtin_amdgcn_update_dpp(v, v, CTRL, ROWMASK, 0xf, false);
}

// Wave-wide max / min through DPP (quad swaps, half-row and row mirrors, then
// the row 15 / row 31 broadcasts); exact for max and min, so the order of the
// combination does not matter. The result is read from lane 63 and returned
// to every lane.
HX_DEV float wave_max_dpp(float v) {
  v = fmaxf(v, __int_as_float(dpp_mov<0xB1>(__float_as_int(v))));   // quad_perm 1,0,3,2
  v = fmaxf(v, __int_as_float(dpp_mov<0x4E>(__float_as_int(v))));   // quad_perm 2,3,0,1
  v = fmaxf(v, __int_as_float(dpp_mov<0x141>(__float_as_int(v))));  // row_half_mirror
  v = fmaxf(v, __int_as_float(dpp_mov<0x140>(__float_as_int(v))));  // row_mirror
  v = fmaxf(v, __int_as_float(dpp_mov<0x142, 0xA>(__float_as_int(v))));  // row_bcast15
  v = fmaxf(v, __int_as_float(dpp_mov<0x143, 0xC>(__float_as_int(v))));  // row_bcast31
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

HX_DEV int wave_min_dpp(int v) {
  v = min(v, dpp_mov<0xB1>(v));
  v = min(v, dpp_mov<0x4E>(v));
  v = min(v, dpp_mov<0x141>(v));
  v = min(v, dpp_mov<0x140>(v));
  v = min(v, dpp_mov<0x142, 0xA>(v));
  v = min(v, dpp_mov<0x143, 0xC>(v));
  return __builtin_amdgcn_readlane(v, 63);
}

// activation element loads
HX_DEV float ld_act(const void* p, int64_t i, bool bf16) {
  return bf16 ? bf16_to_f32(((const uint16_t*)p)[i]) : ((const float*)p)[i];
}

}  // namespace hx
