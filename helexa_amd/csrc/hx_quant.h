// Activation quantisation of the reference's quantised matmul, on the device.
//
// Reference: MaybeQuantLinear::forward (crates/neuron/src/harness/tp/tp_linear.rs:120-137):
// an expert projection called on m <= 64 rows casts x to f32 and calls
// QMatMul::forward, whose CPU arithmetic (candle-core 0.11 k_quants, a third-
// party crate) quantises every activation row to the weight type's vec_dot
// type and sums integer products of codes block by block:
//   Q8_0 weights -> Q8_0 rows (blocks of 32): d = amax / 127, id = 1 / d (0 when
//     d == 0), q = round(x id), round half away from zero; d is stored as f16;
//   Q4_K / Q6_K weights -> Q8_K rows (blocks of 256): max = the signed value of
//     the first element of largest |x|, iscale = -128 / max,
//     q = min(round(iscale x), 127), d = 1 / iscale; an all-zero block is zero.
// The codes computed here are those codes bit for bit (the same IEEE
// operations: -ffp-contract=off keeps iscale x a rounded product, the
// divisions are correctly rounded).
//
// Chunk records. The decode GEMV kernels give each lane chunks of 32 weights
// of a row (Chunk<FMT>::pos) and need the 32 matching activation codes as the
// int8 bytes their v_dot4_i32_i8 products take. A record holds one chunk:
//   words 0..7   the codes as int8, slot s (elements x_group_off(c, s) .. + 7,
//                see hx_decode.hip) in words 2 s, 2 s + 1, in element order;
//                every product sum of codes and weights is an exact int32;
//   words 8, 9   the sums of the eight codes of slots 0, 1 | 2, 3 as int16
//                (|sum| <= 1024);
//   word 10      the block's d (f32; Q8_0: its f16 value);
//   word 11      0.
// Every chunk lies inside one quantisation block (Q8_0: the chunk is the
// block; Q8_K: chunk c is in superblock c / 8).
//
// Producers work on rows in the canonical layout of the router kernels: the
// K elements cut into groups of 8, group g held by lane g % 64 in register
// g / 64. A group is one slot of one chunk, and the groups of a block are
// consecutive lanes (4 for Q8_0, 32 for Q8_K), in element order.
#pragma once
#include "hx_internal.h"

namespace hx {

constexpr int HX_REC_SUMS = 8, HX_REC_D = 10;
constexpr int HX_REC_VECS = HX_XCV_WORDS / 4;   // 16-byte words per record
static_assert(HX_XCV_WORDS == 12, "record layout: 8 code words, 2 sum words, d, 0");

// round half away from zero, for |y| <= 130: trunc(y + copysign(pred(0.5), y))
// equals roundf(y) on every f32 in that range (checked exhaustively); the
// products quantised here are at most 128.00002 in magnitude
HX_DEV float round_away(float y) { return __builtin_truncf(y + __builtin_copysignf(0.49999997f, y)); }

// the chunk c and slot s of group g of a row (the K layout of the weight
// format FMT, which is also what selects the vec_dot type)
template <int FMT>
HX_DEV void group_slot(int g, int& c, int& s) {
  if constexpr (FMT == HX_Q8_0) {
    c = g >> 2;
    s = g & 3;
  } else if constexpr (FMT == HX_Q4_K) {
    // superblock g / 32; 64-element group p; r8 = group in p: low run of
    // chunk 2p + h (r8 = 2h, 2h + 1) or high run (r8 = 4 + 2h, 5 + 2h)
    const int r8 = g & 7, p = (g >> 3) & 3, h = (r8 >> 1) & 1, hi = r8 >> 2;
    c = 8 * (g >> 5) + 2 * p + h;
    s = 2 * hi + (r8 & 1);
  } else {
    // Q6_K: superblock g / 32; half n, quarter q, l-block a: chunk 4n + a, slot q
    const int gg = g & 31, n = gg >> 4, q = (gg >> 2) & 3, a = gg & 3;
    c = 8 * (g >> 5) + 4 * n + a;
    s = q;
  }
}

// Reductions over a block of W consecutive lanes (W = 4 or 32) by register
// moves, every lane of the wave taking part. Quads by DPP quad_perm (lane ^ 1,
// lane ^ 2). A row of 16 by two DPP row rotations, 4 and then 8 lanes: after
// the quad step each lane holds its quad's value, the rotation by 4 adds a
// neighbouring quad and the rotation by 8 the other two, whichever way the
// rotation turns. Two rows by permlane16_swap, whose two results hold the
// values of rows 2i and 2i + 1 in both rows; the reduction takes both.
template <typename Op>
HX_DEV uint32_t lanes_reduce4(uint32_t v, Op op) {
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xf, 0xf, true));   // quad_perm [1,0,3,2]
  return op(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xf, 0xf, true));   // quad_perm [2,3,0,1]
}
template <typename Op>
HX_DEV uint32_t lanes_reduce32(uint32_t v, Op op) {
  v = lanes_reduce4(v, op);
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x124, 0xf, 0xf, true));   // row_ror:4
  v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x128, 0xf, 0xf, true));   // row_ror:8
  const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  return op(r[0], r[1]);
}

// max over the W consecutive lanes of a block (W = 4 or 32)
template <int W>
HX_DEV float block_max(float v) {
  const auto op = [](uint32_t a, uint32_t b) { return __float_as_uint(fmaxf(__uint_as_float(a), __uint_as_float(b))); };
  const uint32_t u = __float_as_uint(v);
  return __uint_as_float(W == 32 ? lanes_reduce32(u, op) : lanes_reduce4(u, op));
}
template <int W>
HX_DEV int block_min(int v) {
  const auto op = [](uint32_t a, uint32_t b) { return (uint32_t)min((int)a, (int)b); };
  return (int)(W == 32 ? lanes_reduce32((uint32_t)v, op) : lanes_reduce4((uint32_t)v, op));
}

// Quantise one group of 8 (this lane's) of a block spread over consecutive
// lanes; every lane of the wave must take part (cross-lane reductions).
// Q8_0 (FMT == HX_Q8_0): blocks of 4 lanes; Q8_K (Q4_K / Q6_K): 32 lanes.
// q: the codes as floats (exact integers); d: the block's d as the vec_dot
// uses it.
template <int FMT>
HX_DEV void quant_group(const float (&x)[8], float (&q)[8], float& d) {
  float am = fabsf(x[0]);
#pragma unroll
  for (int j = 1; j < 8; j++) am = fmaxf(am, fabsf(x[j]));
  if constexpr (FMT == HX_Q8_0) {
    am = block_max<4>(am);
    const float dd = am / 127.0f;
    const float id = dd != 0.0f ? 1.0f / dd : 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j++) q[j] = round_away(x[j] * id);
    d = (float)(_Float16)dd;
  } else {
    const float bam = block_max<32>(am);
    // the first element of the block with |x| == bam: its position, then its
    // signed value from the lane holding it
    const int lb = lane_id() & 31;
    int pos = 0x7fff;
#pragma unroll
    for (int j = 7; j >= 0; j--) pos = fabsf(x[j]) == bam ? 8 * lb + j : pos;
    pos = block_min<32>(pos);
    const int pj = pos & 7;
    float mine = x[0];
#pragma unroll
    for (int j = 1; j < 8; j++) mine = pj == j ? x[j] : mine;
    const float mx = __shfl(mine, (lane_id() & 32) | ((pos >> 3) & 31), 64);
    const bool nz = bam != 0.0f;
    const float iscale = nz ? -128.0f / mx : 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j++) q[j] = fminf(round_away(iscale * x[j]), 127.0f);
    d = nz ? 1.0f / iscale : 0.0f;
  }
}

// four codes (exact integers in [-128, 127], as floats) -> one word of int8
HX_DEV uint32_t pk_i8(float a, float b, float c, float d) {
  const uint32_t lo = ((uint32_t)(int)a & 0xffu) | (((uint32_t)(int)b & 0xffu) << 8);
  const uint32_t hi = ((uint32_t)(int)c & 0xffu) | ((uint32_t)(int)d << 8);
  return lo | (hi << 16);
}

// quantise group g (this lane's 8 values) and write its part of the record of
// its chunk into rec (the row's records, HX_XCV_WORDS words each)
template <int FMT>
HX_DEV void group_to_record(const float (&x)[8], int g, uint32_t* rec) {
  float q[8], d;
  quant_group<FMT>(x, q, d);
  int c, s;
  group_slot<FMT>(g, c, s);
  uint32_t* r = rec + (int64_t)c * HX_XCV_WORDS;
  *(uint2*)(r + 2 * s) = make_uint2(pk_i8(q[0], q[1], q[2], q[3]), pk_i8(q[4], q[5], q[6], q[7]));
  const float sum = ((q[0] + q[1]) + (q[2] + q[3])) + ((q[4] + q[5]) + (q[6] + q[7]));   // exact integers
  ((int16_t*)(r + HX_REC_SUMS))[s] = (int16_t)(int)sum;
  if (s == 0) *(uint2*)(r + HX_REC_D) = make_uint2(__float_as_uint(d), 0u);
}

// the four slot sums and d of a record's last four words
HX_DEV void record_tail(const uint32_t (&w)[4], int (&s)[4], float& d) {
  s[0] = (int)(int16_t)(w[0] & 0xffffu);
  s[1] = (int)w[0] >> 16;
  s[2] = (int)(int16_t)(w[1] & 0xffffu);
  s[3] = (int)w[1] >> 16;
  d = __uint_as_float(w[2]);
}

// Fake-quantised f16 value of a code: f16(d q), the operand the prefill MFMA
// kernels take for expert calls of m <= 64 rows (one rounding of the
// dequantised Q8 value; the codes themselves are candle's)
HX_DEV _Float16 fq_f16(float q, float d) { return (_Float16)(d * q); }

}  // namespace hx
