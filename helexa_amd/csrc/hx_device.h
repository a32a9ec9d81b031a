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

typedef __attribute__((address_space(3))) uint8_t lds_u8;

// global_load_lds_dwordx4: lane l's 16 bytes at g land at LDS byte lds_base +
// 16 l, no registers involved; issued from inline assembly with M0 saved and
// restored around it (the compiler does not know which LDS bytes it writes, so
// the waits for it are placed by hand)
HX_DEV void dma16(const void* g, uint32_t lds_base) {
  uint32_t save;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
               : "=&s"(save) : "v"(g), "s"(lds_base) : "memory");
}
// a workgroup barrier that orders LDS accesses only: global loads still in
// flight stay in flight across it (__syncthreads' fence waits for all of them)
HX_DEV void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// global_load_lds_dword: lane l's 4 bytes at g land at LDS byte lds_base + 4 l
HX_DEV void dma4(const void* g, uint32_t lds_base) {
  uint32_t save;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\tglobal_load_lds_dword %1, off\n\ts_mov_b32 m0, %0"
               : "=&s"(save) : "v"(g), "s"(lds_base) : "memory");
}

// v_and_or_b32 with its two constants in registers (a VOP3 instruction on this
// target takes no literal operand; left to itself the compiler splits the
// operation into an and and an or, each with a literal)
HX_DEV uint32_t and_or(uint32_t x, uint32_t m, uint32_t o) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "v"(m), "v"(o));
  return r;
}
// a register holding the constant C (not volatile: repeated uses merge and the
// move leaves loops)
template <uint32_t C>
HX_DEV uint32_t vconst() {
  uint32_t r;
  asm("v_mov_b32 %0, %1" : "=v"(r) : "i"(C));
  return r;
}

HX_DEV float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// f32 -> bf16, round to nearest even, a NaN kept with its sign and upper
// payload and quieted (bit 6 of the bf16 set): one v_cvt_pk_bf16_f32, whose
// result equals that bit-level rule (u + 0x7fff + ((u >> 16) & 1)) >> 16 for
// every one of the 2^32 f32 inputs (checked exhaustively on MI355X); two
// conversions packed into one word compile to a single instruction
HX_DEV uint16_t f32_to_bf16(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

// exact for every f16 value (normal, subnormal, inf, nan): v_cvt_f32_f16 with
// f16 denormals kept (the default mode of HIP kernels)
HX_DEV float f16_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

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
// x > 88.5 -> +inf, NaN -> NaN. Written with selects only (no branches): the
// special cases are computed alongside and picked at the end.
HX_DEV float expf_route(float x) {
  float n = __builtin_rintf(x * 1.44269504088896341f);
  n = fminf(fmaxf(n, -127.0f), 128.0f);   // only reached for |x| outside the range handled below
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
  const int ni = (int)n;
  float res = p * __uint_as_float((uint32_t)((ni > 127 ? 127 : ni) + 127) << 23);
  res = ni > 127 ? res * 2.0f : res;
  res = x < -87.0f ? 0.0f : res;
  res = x > 88.5f ? __builtin_inff() : res;
  return x != x ? x : res;
}

// expf_route over N values, step by step across the N values so that the N
// independent dependency chains interleave (a single wave is latency-bound on
// one chain). Same arithmetic as expf_route.
template <int N>
HX_DEV void expf_route_n(float* x) {
  float n[N], r[N], p[N];
#pragma unroll
  for (int i = 0; i < N; i++) n[i] = fminf(fmaxf(__builtin_rintf(x[i] * 1.44269504088896341f), -127.0f), 128.0f);
#pragma unroll
  for (int i = 0; i < N; i++) r[i] = __builtin_fmaf(n[i], -0.693145751953125f, x[i]);
#pragma unroll
  for (int i = 0; i < N; i++) r[i] = __builtin_fmaf(n[i], -1.42860682030941723212e-6f, r[i]);
#pragma unroll
  for (int i = 0; i < N; i++) p[i] = __builtin_fmaf(1.98412698412698413e-4f, r[i], 1.38888888888888889e-3f);
#pragma unroll
  for (int i = 0; i < N; i++) p[i] = __builtin_fmaf(p[i], r[i], 8.33333333333333333e-3f);
#pragma unroll
  for (int i = 0; i < N; i++) p[i] = __builtin_fmaf(p[i], r[i], 4.16666666666666667e-2f);
#pragma unroll
  for (int i = 0; i < N; i++) p[i] = __builtin_fmaf(p[i], r[i], 1.66666666666666667e-1f);
#pragma unroll
  for (int i = 0; i < N; i++) p[i] = __builtin_fmaf(p[i], r[i], 0.5f);
#pragma unroll
  for (int i = 0; i < N; i++) p[i] = __builtin_fmaf(p[i], r[i], 1.0f);
#pragma unroll
  for (int i = 0; i < N; i++) p[i] = __builtin_fmaf(p[i], r[i], 1.0f);
#pragma unroll
  for (int i = 0; i < N; i++) {
    const int ni = (int)n[i];
    float res = p[i] * __uint_as_float((uint32_t)((ni > 127 ? 127 : ni) + 127) << 23);
    res = ni > 127 ? res * 2.0f : res;
    res = x[i] < -87.0f ? 0.0f : res;
    res = x[i] > 88.5f ? __builtin_inff() : res;
    x[i] = x[i] != x[i] ? x[i] : res;
  }
}

HX_DEV float sigmoidf_(float v) { return 1.0f / (1.0f + __expf(-v)); }
HX_DEV float siluf_(float g) { return g / (1.0f + __expf(-g)); }
// the same with the division by one v_rcp_f32 (1 ulp): g -> -inf gives
// rcp(inf) = 0, so -0 as the quotient; for the prefill SwiGLU epilogue, whose
// result is rounded to f16
HX_DEV float silu_rcp(float g) { return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)); }

// Xor butterfly over aligned groups of WIDTH lanes (WIDTH a power of two <= 64):
// for off = WIDTH/2 .. 1, every lane adds the value of lane (lane ^ off). Float
// addition is commutative, so both lanes of a pair hold the same sum and the
// result is the same in every lane of a group. Register-only exchanges:
//   off 32 / 16: v_permlane32_swap / v_permlane16_swap of v with itself; the two
//     results hold (own, partner) in some order in every lane;
//   off 8: DPP row_ror:8, which is lane ^ 8 within a row of 16;
//   off 4: DPP row_ror:4 reads lane (r - 4) mod 16, which is r ^ 4 or r ^ 4 ^ 8;
//     once the off-8 step is done, lanes r ^ 4 and r ^ 4 ^ 8 hold equal values;
//   off 2 / 1: DPP quad_perm [2,3,0,1] / [1,0,3,2].
// Groups of 8 lanes use __shfl_xor for the off-4 step.
template <int CTRL>
HX_DEV float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, true));
}

template <int WIDTH>
HX_DEV float wave_sum(float v) {
  if (WIDTH >= 64) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  if (WIDTH >= 32) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  if (WIDTH >= 16) v = v + dpp_f<0x128>(v);   // row_ror:8
  if (WIDTH >= 16) v = v + dpp_f<0x124>(v);   // row_ror:4 (see above)
  else if (WIDTH >= 8) v = v + __shfl_xor(v, 4, 64);
  if (WIDTH >= 4) v = v + dpp_f<0x4E>(v);     // quad_perm [2,3,0,1]
  if (WIDTH >= 2) v = v + dpp_f<0xB1>(v);     // quad_perm [1,0,3,2]
  return v;
}

// One step of the butterfly over lane ^ OFF (OFF a power of two <= 32).
// rs_keep: a lane keeps the sum of lo (lane bit clear) or hi (bit set) with
// its partner's copy of the same value; bf_add: v + partner's v. Exact xor
// partners throughout (lane ^ 4 via row_ror:12 or :4 by bit 2).
template <int OFF>
HX_DEV float rs_keep(float lo, float hi) {
  const int l = __lane_id();
  if (OFF == 32) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(lo), __float_as_uint(hi), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  } else if (OFF == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(lo), __float_as_uint(hi), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  } else if (OFF == 8) {
    const float s1 = lo + dpp_f<0x128>(lo), s2 = hi + dpp_f<0x128>(hi);
    return (l & 8) ? s2 : s1;
  } else if (OFF == 4) {
    const float s1 = lo + dpp_f<0x12C>(lo), s2 = hi + dpp_f<0x124>(hi);
    return (l & 4) ? s2 : s1;
  } else if (OFF == 2) {
    const float s1 = lo + dpp_f<0x4E>(lo), s2 = hi + dpp_f<0x4E>(hi);
    return (l & 2) ? s2 : s1;
  } else {
    const float s1 = lo + dpp_f<0xB1>(lo), s2 = hi + dpp_f<0xB1>(hi);
    return (l & 1) ? s2 : s1;
  }
}
template <int OFF>
HX_DEV float bf_add(float v) {
  const int l = __lane_id();
  if (OFF == 32 || OFF == 16) {
    const auto r = OFF == 32 ? __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false)
                             : __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  } else if (OFF == 8) {
    return v + dpp_f<0x128>(v);
  } else if (OFF == 4) {
    // both reads with the whole wave active (a DPP read of a lane that is off
    // in the current exec mask yields 0), then the select
    const float a = dpp_f<0x124>(v), b = dpp_f<0x12C>(v);
    return v + ((l & 4) ? a : b);
  } else if (OFF == 2) {
    return v + dpp_f<0x4E>(v);
  } else {
    return v + dpp_f<0xB1>(v);
  }
}

// Wave-wide sums of M (gate, up) pairs (M a power of two <= 64): the first
// log2 M steps of the butterfly are a reduce-scatter over the pairs, the rest
// plain butterfly steps; lane l ends with the sums of pair l >> (6 - log2 M).
template <int M, int STEP = 0>
HX_DEV void rs_pairs64(float* g, float* u) {
  if constexpr (STEP < 6) {
    constexpr int OFF = 32 >> STEP, LIVE = M >> STEP;
    if constexpr (LIVE >= 2) {
#pragma unroll
      for (int k = 0; k < LIVE / 2; k++) {
        g[k] = rs_keep<OFF>(g[k], g[k + LIVE / 2]);
        u[k] = rs_keep<OFF>(u[k], u[k + LIVE / 2]);
      }
    } else {
      g[0] = bf_add<OFF>(g[0]);
      u[0] = bf_add<OFF>(u[0]);
    }
    rs_pairs64<M, STEP + 1>(g, u);
  }
}

// Wave-wide sums of M values (M a power of two <= 64), as rs_pairs64 for
// single values: lane l ends with the sum of value l >> (6 - log2 M) in v[0].
template <int M, int STEP = 0>
HX_DEV void rs_vals64(float* v) {
  if constexpr (STEP < 6) {
    constexpr int OFF = 32 >> STEP, LIVE = M >> STEP;
    if constexpr (LIVE >= 2) {
#pragma unroll
      for (int k = 0; k < LIVE / 2; k++) v[k] = rs_keep<OFF>(v[k], v[k + LIVE / 2]);
    } else {
      v[0] = bf_add<OFF>(v[0]);
    }
    rs_vals64<M, STEP + 1>(v);
  }
}

// The butterfly of wave_sum<64> applied to 64 values at once, as a
// reduce-scatter: at each step a lane adds its partner's copy of only the half
// of its live values it keeps (the half selected by the lane's bit for that
// step), so every addition is one the butterfly performs and the sums are the
// same bit for bit; lane l ends with the sum of v[l]. 141 instructions instead
// of 64 butterflies. Lane semantics used: permlane32_swap(x, y) returns
// (own x, x of lane + 32) in lanes 0..31 and (y of lane - 32, own y) in lanes
// 32..63, permlane16_swap the same for rows 0/1 and 2/3; DPP row_ror:N reads
// lane (r - N) mod 16 of the row.
HX_DEV float reduce_scatter64(float (&v)[64]) {
  const int l = __lane_id();
#pragma unroll
  for (int k = 0; k < 32; k++) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[k]), __float_as_uint(v[k + 32]), false, false);
    v[k] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
#pragma unroll
  for (int k = 0; k < 16; k++) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[k]), __float_as_uint(v[k + 16]), false, false);
    v[k] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
#pragma unroll
  for (int k = 0; k < 8; k++) {   // lane ^ 8: row_ror:8
    const float s1 = v[k] + dpp_f<0x128>(v[k]), s2 = v[k + 8] + dpp_f<0x128>(v[k + 8]);
    v[k] = (l & 8) ? s2 : s1;
  }
#pragma unroll
  for (int k = 0; k < 4; k++) {   // lane ^ 4: lane + 4 (row_ror:12) where bit 2 is clear, lane - 4 (row_ror:4) where set
    const float s1 = v[k] + dpp_f<0x12C>(v[k]), s2 = v[k + 4] + dpp_f<0x124>(v[k + 4]);
    v[k] = (l & 4) ? s2 : s1;
  }
#pragma unroll
  for (int k = 0; k < 2; k++) {   // lane ^ 2: quad_perm [2,3,0,1]
    const float s1 = v[k] + dpp_f<0x4E>(v[k]), s2 = v[k + 2] + dpp_f<0x4E>(v[k + 2]);
    v[k] = (l & 2) ? s2 : s1;
  }
  const float s1 = v[0] + dpp_f<0xB1>(v[0]), s2 = v[1] + dpp_f<0xB1>(v[1]);   // lane ^ 1: quad_perm [1,0,3,2]
  return (l & 1) ? s2 : s1;
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

// wave-wide max of unsigned values (identity 0, so the DPP moves fold into
// v_max_u32_dpp), returned to every lane
HX_DEV uint32_t wave_max_u32(uint32_t v) {
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xf, 0xf, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xf, 0xf, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xf, 0xf, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xf, 0xf, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xa, 0xf, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xc, 0xf, false));
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
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
