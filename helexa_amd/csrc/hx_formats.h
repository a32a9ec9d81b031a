// Weight formats as the kernels see them.
//
// The library keeps each expert projection as E matrices of [rows][K]:
//   F32 / BF16 : row-major, as in the checkpoint.
//   Q4_K       : GGUF superblocks, unchanged (144 B, already 16 B aligned).
//   Q8_0       : GGUF blocks split into planes so every load is aligned:
//                qs plane [rows][K] int8, then d plane [rows][K/32] f16.
//   Q6_K       : GGUF superblocks split into planes:
//                ql [rows][K/2], qh [rows][K/4], scales [rows][K/16] int8,
//                d [rows][K/256] f16.
// The planar forms hold exactly the GGUF bytes, reordered (same size).
//
// A "chunk" is the unit one lane owns in a GEMV: CH weights of one row, loaded
// with a few aligned vector loads. Chunk c of a row covers element positions
// given by pos(c, i) for i in [0, CH); runs of RUN consecutive elements.
#pragma once
#include "hx_device.h"

#define HX_F32 0
#define HX_F16 1
#define HX_Q8_0 8
#define HX_Q4_K 12
#define HX_Q6_K 14
#define HX_BF16 30

namespace hx {

template <int FMT>
struct Chunk;

// ---------------------------------------------------------------- F32
template <>
struct Chunk<HX_F32> {
  static constexpr int CH = 8, RUN = 8;
  struct Raw { float4 a, b; };
  HX_DEV static int pos(int c, int i) { return c * 8 + i; }
  HX_DEV static void load(const uint8_t* mat, int R, int K, int row, int c, Raw& r) {
    const float4* p = (const float4*)(mat + ((int64_t)row * K + c * 8) * 4);
    r.a = p[0];
    r.b = p[1];
  }
  // sum over the chunk of w*x; xs unused
  HX_DEV static float dot(const Raw& r, const float* x, const float* xs) {
    float s = 0.f;
    s = __builtin_fmaf(r.a.x, x[0], s); s = __builtin_fmaf(r.a.y, x[1], s);
    s = __builtin_fmaf(r.a.z, x[2], s); s = __builtin_fmaf(r.a.w, x[3], s);
    s = __builtin_fmaf(r.b.x, x[4], s); s = __builtin_fmaf(r.b.y, x[5], s);
    s = __builtin_fmaf(r.b.z, x[6], s); s = __builtin_fmaf(r.b.w, x[7], s);
    return s;
  }
  static constexpr int NSUM = 0;
  HX_DEV static void sums(const float* x, float* xs) {}
};

// ---------------------------------------------------------------- BF16
template <>
struct Chunk<HX_BF16> {
  static constexpr int CH = 8, RUN = 8;
  struct Raw { uint4 a; };
  HX_DEV static int pos(int c, int i) { return c * 8 + i; }
  HX_DEV static void load(const uint8_t* mat, int R, int K, int row, int c, Raw& r) {
    r.a = *(const uint4*)(mat + ((int64_t)row * K + c * 8) * 2);
  }
  HX_DEV static float dot(const Raw& r, const float* x, const float* xs) {
    const uint32_t w[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      s = __builtin_fmaf(__uint_as_float(w[j] << 16), x[2 * j], s);
      s = __builtin_fmaf(__uint_as_float(w[j] & 0xffff0000u), x[2 * j + 1], s);
    }
    return s;
  }
  static constexpr int NSUM = 0;
  HX_DEV static void sums(const float* x, float* xs) {}
};

// ---------------------------------------------------------------- Q8_0 (planar)
template <>
struct Chunk<HX_Q8_0> {
  static constexpr int CH = 32, RUN = 32;
  struct Raw { uint4 a, b; uint32_t d; };
  HX_DEV static int pos(int c, int i) { return c * 32 + i; }
  HX_DEV static void load(const uint8_t* mat, int R, int K, int row, int c, Raw& r) {
    const uint4* p = (const uint4*)(mat + (int64_t)row * K + c * 32);
    r.a = p[0];
    r.b = p[1];
    r.d = ((const uint16_t*)(mat + (int64_t)R * K))[(int64_t)row * (K / 32) + c];
  }
  HX_DEV static float dot(const Raw& r, const float* x, const float* xs) {
    const uint32_t q[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < 8; j++) {
#pragma unroll
      for (int b = 0; b < 4; b++) {
        int v = ((int)(q[j] << (24 - 8 * b))) >> 24;
        s = __builtin_fmaf((float)v, x[4 * j + b], s);
      }
    }
    return f16_to_f32((uint16_t)r.d) * s;
  }
  static constexpr int NSUM = 0;
  HX_DEV static void sums(const float* x, float* xs) {}
};

// ---------------------------------------------------------------- Q4_K (GGUF)
// Stored layout of a Q4_K matrix of R rows: the GGUF superblocks (144 B) in
// groups of G rows, superblock-major inside a group -- superblock sb of row r
// at ((r / G) G nsb + sb G + r % G) 144, G = the largest power of two up to
// HX_Q4K_GROUP that divides R (64 for every shape the prefill MFMA kernels
// take; every group full, so the offsets are shifts). The same bytes as the
// GGUF rows, reordered at load so that one superblock of a group's rows (what
// a prefill tile's K chunk reads from its 64 weight rows) is one contiguous
// run: read row by row, the chunks touched DRAM pages 80 bytes at a time
// (measured on MI355X: 4.6 against 6.2 TB/s for the same bytes blocked).
#define HX_Q4K_GROUP 64
HX_DEV int q4k_group_log2(int R) { return min(__builtin_ctz((unsigned)R), 6); }
HX_DEV const uint8_t* q4k_sb(const uint8_t* mat, int R, int K, int row, int sb) {
  static_assert(HX_Q4K_GROUP == 64, "q4k_group_log2 caps at 2^6");
  const int lg = q4k_group_log2(R), g0 = (row >> lg) << lg;
  return mat + ((int64_t)g0 * (K / 256) + ((int64_t)sb << lg) + (row - g0)) * 144;
}

// Chunk c of a row: superblock sb = c / 8, cc = c % 8, pair p = cc / 2, half
// h = cc % 2. It holds the 16 bytes qs[32p + 16h .. +15]: low nibbles are
// elements 64p + 16h + i (sub-block 2p), high nibbles 64p + 32 + 16h + i
// (sub-block 2p+1).
template <>
struct Chunk<HX_Q4_K> {
  static constexpr int CH = 32, RUN = 16;
  struct Raw { uint4 q; uint4 hdr; int cc; };
  HX_DEV static int pos(int c, int i) {
    int sb = c >> 3, cc = c & 7, p = cc >> 1, h = cc & 1;
    return sb * 256 + 64 * p + 16 * h + (i < 16 ? i : 32 + (i - 16));
  }
  HX_DEV static void load(const uint8_t* mat, int R, int K, int row, int c, Raw& r) {
    const uint8_t* sb = q4k_sb(mat, R, K, row, c >> 3);
    int cc = c & 7;
    r.hdr = *(const uint4*)sb;
    r.q = *(const uint4*)(sb + 16 + 32 * (cc >> 1) + 16 * (cc & 1));
    r.cc = cc;
  }
  HX_DEV static void scale_min(const uint4& hdr, int j, int& sc, int& m) {
    const uint32_t s0 = hdr.y, s1 = hdr.z, s2 = hdr.w;  // scales bytes 0-3, 4-7, 8-11
    if (j < 4) {
      sc = (s0 >> (8 * j)) & 63;
      m = (s1 >> (8 * j)) & 63;
    } else {
      int jj = j - 4;
      sc = ((s2 >> (8 * jj)) & 0xF) | (((s0 >> (8 * jj + 6)) & 3) << 4);
      m = ((s2 >> (8 * jj + 4)) & 0xF) | (((s1 >> (8 * jj + 6)) & 3) << 4);
    }
  }
  // xs[0] = sum of x over the low run, xs[1] = over the high run
  static constexpr int NSUM = 2;
  HX_DEV static void sums(const float* x, float* xs) {
    float a = 0.f, b = 0.f;
#pragma unroll
    for (int i = 0; i < 16; i++) { a += x[i]; b += x[16 + i]; }
    xs[0] = a;
    xs[1] = b;
  }
  HX_DEV static float dot(const Raw& r, const float* x, const float* xs) {
    const uint32_t q[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
    float lo = 0.f, hi = 0.f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
#pragma unroll
      for (int b = 0; b < 4; b++) {
        uint32_t byte = (q[j] >> (8 * b)) & 0xffu;
        lo = __builtin_fmaf((float)(byte & 0xF), x[4 * j + b], lo);
        hi = __builtin_fmaf((float)(byte >> 4), x[16 + 4 * j + b], hi);
      }
    }
    float d = f16_to_f32((uint16_t)(r.hdr.x & 0xffffu)), dmin = f16_to_f32((uint16_t)(r.hdr.x >> 16));
    int p = r.cc >> 1, sc0, m0, sc1, m1;
    scale_min(r.hdr, 2 * p, sc0, m0);
    scale_min(r.hdr, 2 * p + 1, sc1, m1);
    return d * ((float)sc0 * lo + (float)sc1 * hi) - dmin * ((float)m0 * xs[0] + (float)m1 * xs[1]);
  }
};

// ---------------------------------------------------------------- Q6_K (planar)
// Stored layout of a Q6_K matrix of R rows and K columns: four planes, ql
// (K / 2 bytes a row), qh (K / 4), scales (K / 16) and d (K / 128); the first
// three in groups of G rows, piece-major inside a group -- byte o of row r's
// part of a plane whose rows hold Wp bytes in pieces of Sp at
//   (r / G) G Wp + (o / Sp) G Sp + (r % G) Sp + o % Sp,
// G = the largest power of two up to HX_Q6K_GROUP that divides R (128 for
// every shape the prefill MFMA kernels take; every group full, so the piece
// offset is a shift by a uniform amount -- a multiply per load there cost the
// multi-token decode kernels 7-9 %), so that the pieces a prefill down tile's
// K chunk reads from its 128 weight rows (32 ql and 32 qh bytes, 8 scale
// bytes each) are contiguous runs; Sp = 32 for ql and qh, 16 for the scales
// (every read stays inside one piece). d is row-major.
#define HX_Q6K_GROUP 128
HX_DEV int q6k_group_log2(int R) { return min(__builtin_ctz((unsigned)R), 7); }
HX_DEV const uint8_t* q6k_at(const uint8_t* plane, int R, int Wp, int Sp, int row, int o) {
  static_assert(HX_Q6K_GROUP == 128, "q6k_group_log2 caps at 2^7");
  const int lg = q6k_group_log2(R), g0 = (row >> lg) << lg;
  return plane + (int64_t)g0 * Wp + ((int64_t)(o / Sp) << lg) * Sp + (int64_t)(row - g0) * Sp + o % Sp;
}
HX_DEV const uint8_t* q6k_ql(const uint8_t* mat, int R, int K, int row, int o) {
  return q6k_at(mat, R, K / 2, 32, row, o);
}
HX_DEV const uint8_t* q6k_qh(const uint8_t* mat, int R, int K, int row, int o) {
  return q6k_at(mat + (int64_t)R * (K / 2), R, K / 4, 32, row, o);
}
HX_DEV const uint8_t* q6k_sc(const uint8_t* mat, int R, int K, int row, int o) {
  return q6k_at(mat + (int64_t)R * (K / 2 + K / 4), R, K / 16, 16, row, o);
}

// Chunk c: superblock sb = c / 8, cc = c % 8, half n = cc / 4, a = cc % 4.
// It covers l = 8a .. 8a+7 of the four quarters s = 0..3 of half n: elements
// 128n + 32s + l. Bytes: ql[64n + 8a ..] (quarters 0, 2), ql[64n + 32 + 8a ..]
// (quarters 1, 3), qh[32n + 8a ..] (2 bits per quarter), scale
// sc[8n + 2s + a/2].
template <>
struct Chunk<HX_Q6_K> {
  static constexpr int CH = 32, RUN = 8;
  struct Raw { uint2 l0, l1, h; uint32_t sc; uint32_t d; };
  HX_DEV static int pos(int c, int i) {
    int sb = c >> 3, cc = c & 7, n = cc >> 2, a = cc & 3;
    return sb * 256 + 128 * n + 32 * (i >> 3) + 8 * a + (i & 7);
  }
  HX_DEV static void load(const uint8_t* mat, int R, int K, int row, int c, Raw& r) {
    int sb = c >> 3, cc = c & 7, n = cc >> 2, a = cc & 3;
    const int o = sb * 128 + 64 * n + 8 * a;
    const uint8_t* qh = q6k_qh(mat, R, K, row, sb * 64 + 32 * n + 8 * a);
    // the half's 8 scales as one 8-byte load; the chunk's are bytes
    // (a >> 1) + 0, 2, 4, 6 of it
    const uint2 sc8 = *(const uint2*)q6k_sc(mat, R, K, row, sb * 16 + 8 * n);
    const uint16_t* d = (const uint16_t*)(mat + (int64_t)R * (K / 2 + K / 4 + K / 16)) + (int64_t)row * (K / 256) + sb;
    r.l0 = *(const uint2*)q6k_ql(mat, R, K, row, o);
    r.l1 = *(const uint2*)q6k_ql(mat, R, K, row, o + 32);
    r.h = *(const uint2*)qh;
    r.sc = __builtin_amdgcn_perm(sc8.y, sc8.x, 0x06040200u + 0x01010101u * (uint32_t)(a >> 1));
    r.d = *d;
  }
  static constexpr int NSUM = 4;
  HX_DEV static void sums(const float* x, float* xs) {
#pragma unroll
    for (int s = 0; s < 4; s++) {
      float a = 0.f;
#pragma unroll
      for (int i = 0; i < 8; i++) a += x[8 * s + i];
      xs[s] = a;
    }
  }
  HX_DEV static float dot(const Raw& r, const float* x, const float* xs) {
    const uint32_t l0[2] = {r.l0.x, r.l0.y}, l1[2] = {r.l1.x, r.l1.y}, hh[2] = {r.h.x, r.h.y};
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < 2; w++) {
#pragma unroll
      for (int b = 0; b < 4; b++) {
        int i = 4 * w + b;
        uint32_t a0 = (l0[w] >> (8 * b)) & 0xffu, a1 = (l1[w] >> (8 * b)) & 0xffu, h = (hh[w] >> (8 * b)) & 0xffu;
        uint32_t q0 = (a0 & 0xF) | ((h & 3) << 4);
        uint32_t q1 = (a1 & 0xF) | (((h >> 2) & 3) << 4);
        uint32_t q2 = (a0 >> 4) | (((h >> 4) & 3) << 4);
        uint32_t q3 = (a1 >> 4) | (((h >> 6) & 3) << 4);
        acc[0] = __builtin_fmaf((float)q0, x[i], acc[0]);
        acc[1] = __builtin_fmaf((float)q1, x[8 + i], acc[1]);
        acc[2] = __builtin_fmaf((float)q2, x[16 + i], acc[2]);
        acc[3] = __builtin_fmaf((float)q3, x[24 + i], acc[3]);
      }
    }
    float s = 0.f;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      float sc = (float)(int8_t)((r.sc >> (8 * q)) & 0xffu);
      s = __builtin_fmaf(sc, acc[q] - 32.0f * xs[q], s);
    }
    return f16_to_f32((uint16_t)r.d) * s;
  }
};

}  // namespace hx
