// Prefill grouped GEMMs on the matrix cores (bf16 activations, GGUF experts).
//
// Reference: MaybeQuantLinear's prefill arm (dequantise W, then a GEMM;
// crates/neuron/src/harness/tp/tp_linear.rs:111-118) inside the fused MoE path
// (three grouped GEMMs over expert-sorted rows, the routing weights folded into
// the down GEMM, then the sum over k; crates/neuron/src/harness/tp/tp_qwen3_5.rs:1192-1225).
//
// Work unit: one M tile of the dispatch tile list (<= 64 permuted rows of one
// expert, or of the shared expert) x one N tile. The reference computes an
// expert call of m rows in one of two arms (tp_linear.rs:107-137), and so does
// each tile, by its expert's m (the tile record's first word):
//   * m <= HX_QUANT_M (= 64): the rows quantised to the weights' vec_dot type
//     (Q8_0 / Q8_K codes, exactly the reference's, hx_quant.h) and integer
//     block products. Here the operand is the f16 value d q of each code
//     (one rounding of the dequantised code; the weights are f16 as well), so
//     the products equal the reference's to f16 operand rounding. Tokens come
//     from xq (k_xq_fq); h leaves the gate/up epilogue in f32 and k_hq_fq
//     quantises it into hbf before the down GEMM.
//   * m > 64 (forward_via_f16): f16 weights and activations, f32 sums, and the
//     products rounded to f16 in the epilogues, as the reference's f16 output.
// Operands are f16: the tokens are converted once (bf16 -> f16 is exact in
// f16's normal range), the SwiGLU activations are stored as f16, and weights
// are dequantised to f16 with the
// 0x6400 pattern (f16 1024 + u, exact) and packed f16 arithmetic. Along K the
// elements of every group of 4 are stored in the order (0, 2, 1, 3) -- in the
// activations and in the weights alike, so the dot products are unchanged --
// which lets two 4-bit / 8-bit codes become an f16 pair in one operation;
// the Q4_K gate/up kernel converts adjacent codes instead (FP8 conversion, see
// q4k_compute), so with Q4_K gate/up weights the f16 tokens are in natural
// order (xh_natural).
//
// Per K chunk of 128 the workgroup stages both operands in LDS (rows padded by
// 16 bytes: the 16 lanes of a fragment read hit distinct banks) and issues
// v_mfma_f32_16x16x32_f16 (gfx950 layout: lane l holds A[l%16][8(l/16)+i],
// B[8(l/16)+i][l%16] and D rows 4(l/16)+i of column l%16). The next chunk's
// global loads are issued before the current chunk's MFMAs. 52 KB of LDS per
// workgroup: three workgroups per CU.
#include "hx_internal.h"
#include <type_traits>

namespace hx {

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int PM = 64;            // rows of an M tile
constexpr int PKC = 128;          // K chunk (f16 elements)
constexpr int PLD = PKC + 8;      // LDS row pitch (f16 elements)

HX_DEV h2_t h2(uint32_t v) { return __builtin_bit_cast(h2_t, v); }
HX_DEV uint32_t u32(h2_t v) { return __builtin_bit_cast(uint32_t, v); }
HX_DEV h2_t h2s(float f) {
  const _Float16 h = (_Float16)f;
  return h2_t{h, h};
}
// position of element i of a row in the swizzled storage order
HX_DEV int swz(int i) { return (i & ~3) | ((i & 1) << 1) | ((i >> 1) & 1); }

// (1024 + u) code pairs -> f16 weights a * u - b, two per operation
HX_DEV uint32_t fma_pair(uint32_t codes, h2_t a, h2_t nb, h2_t off) {
  return u32(__builtin_elementwise_fma(h2(codes) + off, a, nb));
}
HX_DEV uint32_t mul_pair(uint32_t codes, h2_t a, h2_t off) { return u32((h2(codes) + off) * a); }

// ---------------------------------------------------------------- weight chunks
// PRaw<FMT>: one thread's raw data for 64 weights (half of a 128-wide K chunk)
// of one row; to_lds writes them, dequantised and swizzled, into the row.
template <int FMT>
struct PRaw;

// Q4_K (GGUF): chunk kc = half (kc & 1) of superblock kc >> 1; part pt holds
// the 32 qs bytes of 64-element group c = 2 (kc & 1) + pt: low nibbles are
// sub-block 2c, high nibbles sub-block 2c + 1.
template <>
struct PRaw<HX_Q4_K> {
  uint4 hdr, q0, q1;
  int c;
  HX_DEV void load(const uint8_t* mat, int R, int K, int row, int kc, int pt) {
    const uint8_t* p = q4k_sb(mat, R, K, row, kc >> 1);
    c = 2 * (kc & 1) + pt;
    hdr = *(const uint4*)p;
    q0 = *(const uint4*)(p + 16 + 32 * c);
    q1 = *(const uint4*)(p + 32 + 32 * c);
  }
  HX_DEV void to_lds(uint16_t* dst) const {
    const float d = f16_to_f32((uint16_t)(hdr.x & 0xffffu)), dmin = f16_to_f32((uint16_t)(hdr.x >> 16));
    int sc0, m0, sc1, m1;
    Chunk<HX_Q4_K>::scale_min(hdr, 2 * c, sc0, m0);
    Chunk<HX_Q4_K>::scale_min(hdr, 2 * c + 1, sc1, m1);
    const h2_t a0 = h2s(d * (float)sc0), nb0 = h2s(-dmin * (float)m0);
    const h2_t a1 = h2s(d * (float)sc1), nb1 = h2s(-dmin * (float)m1);
    const h2_t off = h2s(-1024.0f);
    const uint32_t w[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
    uint32_t lo[16], hi[16];
#pragma unroll
    for (int j = 0; j < 8; j++) {
      lo[2 * j] = fma_pair((w[j] & 0x000F000Fu) | 0x64006400u, a0, nb0, off);
      lo[2 * j + 1] = fma_pair(((w[j] >> 8) & 0x000F000Fu) | 0x64006400u, a0, nb0, off);
      hi[2 * j] = fma_pair(((w[j] >> 4) & 0x000F000Fu) | 0x64006400u, a1, nb1, off);
      hi[2 * j + 1] = fma_pair(((w[j] >> 12) & 0x000F000Fu) | 0x64006400u, a1, nb1, off);
    }
    uint4* o = (uint4*)dst;
#pragma unroll
    for (int v = 0; v < 4; v++) {
      o[v] = make_uint4(lo[4 * v], lo[4 * v + 1], lo[4 * v + 2], lo[4 * v + 3]);
      o[4 + v] = make_uint4(hi[4 * v], hi[4 * v + 1], hi[4 * v + 2], hi[4 * v + 3]);
    }
  }
};

// Q8_0 planar: part pt holds blocks 4 kc + 2 pt and + 1 (64 int8 + 2 scales)
template <>
struct PRaw<HX_Q8_0> {
  uint4 q[4];
  uint32_t d;
  HX_DEV void load(const uint8_t* mat, int R, int K, int row, int kc, int pt) {
    const int b0 = 4 * kc + 2 * pt;
    const uint4* p = (const uint4*)(mat + (int64_t)row * K + 32 * b0);
#pragma unroll
    for (int v = 0; v < 4; v++) q[v] = p[v];
    d = *(const uint32_t*)((const uint16_t*)(mat + (int64_t)R * K) + (int64_t)row * (K / 32) + b0);
  }
  HX_DEV void to_lds(uint16_t* dst) const {
    const h2_t off = h2s(-1152.0f);
    uint4* o = (uint4*)dst;
#pragma unroll
    for (int b = 0; b < 2; b++) {
      const h2_t s = h2s(f16_to_f32((uint16_t)(d >> (16 * b))));
      const uint32_t w[8] = {q[2 * b].x, q[2 * b].y, q[2 * b].z, q[2 * b].w,
                             q[2 * b + 1].x, q[2 * b + 1].y, q[2 * b + 1].z, q[2 * b + 1].w};
      uint32_t r[16];
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const uint32_t u = w[j] ^ 0x80808080u;                     // int8 -> q + 128
        r[2 * j] = mul_pair(__builtin_amdgcn_perm(u, 0x64646464u, 0x00060004u), s, off);
        r[2 * j + 1] = mul_pair(__builtin_amdgcn_perm(u, 0x64646464u, 0x00070005u), s, off);
      }
#pragma unroll
      for (int v = 0; v < 4; v++) o[4 * b + v] = make_uint4(r[4 * v], r[4 * v + 1], r[4 * v + 2], r[4 * v + 3]);
    }
  }
};

// Q6_K planar: chunk kc = half n = kc & 1 of superblock kc >> 1 (quarters
// s = 0..3 of 32 elements each); part pt holds quarters pt and pt + 2: ql bytes
// 32 pt .. +31 of the half (low / high nibble) and the half's 32 qh bytes.
template <>
struct PRaw<HX_Q6_K> {
  uint4 l0, l1, h0, h1;
  uint32_t sc;
  uint32_t d;
  int pt;
  HX_DEV void load(const uint8_t* mat, int R, int K, int row, int kc, int p) {
    const int sb = kc >> 1, n = kc & 1;
    pt = p;
    const uint8_t* ql = q6k_ql(mat, R, K, row, sb * 128 + 64 * n + 32 * pt);
    const uint8_t* qh = q6k_qh(mat, R, K, row, sb * 64 + 32 * n);
    const uint8_t* s = q6k_sc(mat, R, K, row, sb * 16 + 8 * n);
    l0 = *(const uint4*)ql;
    l1 = *(const uint4*)(ql + 16);
    h0 = *(const uint4*)qh;
    h1 = *(const uint4*)(qh + 16);
    // scales of quarter pt (2pt, 2pt+1) and quarter pt+2 (2pt+4, 2pt+5)
    sc = (uint32_t)s[2 * pt] | ((uint32_t)s[2 * pt + 1] << 8) | ((uint32_t)s[2 * pt + 4] << 16) |
         ((uint32_t)s[2 * pt + 5] << 24);
    d = *((const uint16_t*)(mat + (int64_t)R * (K / 2 + K / 4 + K / 16)) + (int64_t)row * (K / 256) + sb);
  }
  HX_DEV void to_lds(uint16_t* dst) const {
    const float dd = f16_to_f32((uint16_t)d);
    const h2_t off = h2s(-1056.0f);
    const uint32_t L[8] = {l0.x, l0.y, l0.z, l0.w, l1.x, l1.y, l1.z, l1.w};
    const uint32_t Hq[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
#pragma unroll
    for (int qq = 0; qq < 2; qq++) {       // quarter pt + 2 qq
      const int s = pt + 2 * qq, hs = 2 * s;
      uint32_t r[16];
#pragma unroll
      for (int j = 0; j < 8; j++) {        // elements l = 4j .. 4j+3
        const h2_t a = h2s(dd * (float)(int8_t)((sc >> (16 * qq + 8 * (j >> 2))) & 0xffu));
        const uint32_t lq = qq ? L[j] >> 4 : L[j];
        const uint32_t hq = hs >= 4 ? Hq[j] >> (hs - 4) : Hq[j] << (4 - hs);   // bits hs..hs+1 -> 4..5
        r[2 * j] = mul_pair((lq & 0x000F000Fu) | (hq & 0x00300030u) | 0x64006400u, a, off);
        r[2 * j + 1] = mul_pair(((lq >> 8) & 0x000F000Fu) | ((hq >> 8) & 0x00300030u) | 0x64006400u, a, off);
      }
      uint4* o = (uint4*)(dst + 32 * s - 64 * pt);   // quarter s starts at element 32 s of the chunk
#pragma unroll
      for (int v = 0; v < 4; v++) o[v] = make_uint4(r[4 * v], r[4 * v + 1], r[4 * v + 2], r[4 * v + 3]);
    }
  }
};

// ---------------------------------------------------------------- A tile
// 64 gathered f16 rows x 128 of K chunk kc, as 1024 16-byte pieces: piece
// q = thread + 256 i is row q / 16, piece q % 16. Sixteen consecutive lanes
// cover one row (coalesced 256-byte reads) and any 8 consecutive lanes write
// 8 different bank groups of LDS.
struct ARaw {
  uint4 v[4];
  HX_DEV void load(const uint16_t* src, int64_t stride, const int* rowsrc, int rows, int kc) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int q = threadIdx.x + 256 * i, r = q >> 4, seg = q & 15;
      v[i] = r < rows ? *(const uint4*)(src + (int64_t)rowsrc[r] * stride + kc * PKC + 8 * seg)
                      : make_uint4(0u, 0u, 0u, 0u);
    }
  }
  HX_DEV void to_lds(uint16_t* As) const {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int q = threadIdx.x + 256 * i, r = q >> 4, seg = q & 15;
      *(uint4*)(As + r * PLD + 8 * seg) = v[i];
    }
  }
};


HX_DEV f16x8_t frag(const uint16_t* base) { return __builtin_bit_cast(f16x8_t, *(const uint4*)base); }

// the M tile of a workgroup (expert, first permuted row, rows): from the
// dispatch list, or for a shared-expert-only launch computed from T; false if
// the workgroup has no tile (past the end, or a tile the launch skips). TS is
// the launch's tile selection (HX_TILES_*), a template parameter so that each
// selection is a kernel of its own name in traces and counter runs.
// m: the rows of the expert's call (the reference's arm: m <= HX_QUANT_M
// quantised activations, else f16)
template <int TS>
HX_DEV bool get_tile(const ExpertArgs& a, int tile, int& e, int& p0, int& rows, int& m) {
  if (TS == HX_TILES_SHARED) {
    const int m0 = tile * PM;
    if (m0 >= a.T) return false;
    e = a.E;
    p0 = a.F + m0;
    rows = min(PM, a.T - m0);
    m = a.T;
    return true;
  }
  if (tile >= a.counts[1]) return false;
  m = a.tiles[4 * tile + 0];
  e = a.tiles[4 * tile + 1];
  p0 = a.tiles[4 * tile + 2];
  rows = a.tiles[4 * tile + 3];
  return !(TS == HX_TILES_ROUTED && e == a.E);
}

// ---------------------------------------------------------------- Q4_K gate/up, streamed
// k_gate_up_q4k<FPW, NW>: the gate/up GEMM for Q4_K weights, operands
// streamed into LDS by the memory unit (global_load_lds_dwordx4: lane l's 16
// bytes land at the wave's LDS base + 16 l, no registers involved) through a
// ring of NST K-chunk stages, NST - 1 chunks ahead of the MFMAs.
// Tile: 64 gathered rows x 16 FPW NW gate + as many up columns; wave w owns
// gate and up columns 16 (FPW w + j) .. + 15, j < FPW.
//   stage: A = 64 token rows x 128 K (f16, 16 KB), the 16-byte pieces of row r
//          stored at piece p ^ (r % 16) so the 16 rows of an MFMA fragment read
//          hit different LDS banks;
//          B = the raw GGUF bytes the chunk needs of each of the 32 FPW NW
//          weight rows (gate rows, then up rows): the superblock header (16 B) and the
//          64 qs bytes of the chunk's half superblock, 80 B per row.
// Each wave dequantises its own B fragments from the raw bytes in LDS, so the
// activations are the only operand every wave reads in full.
// LDS: FPW = 1 with 4 waves, 2 stages of 26 KB, so 3 workgroups per CU.
// Measured on MI355X for the A3B shapes, this beats 3 stages with 2
// workgroups per CU (the kernel waits more on its own LDS reads, dequantisation
// and MFMA chains than on memory, so waves per SIMD matter more than a second
// chunk of look-ahead), 4 waves with FPW = 2, and 8 waves over 128 + 128
// columns: fewer waves per SIMD hide less of the LDS and dequantisation
// latency than the halved activation traffic saves.
// The DMA instructions are issued from inline assembly (M0 saved and restored
// around them) because the compiler, not knowing which LDS bytes a DMA writes,
// would otherwise wait for every outstanding one before each LDS read; the
// waits are placed by hand: before the barrier of chunk kc, a wave waits until
// only its DMAs of the chunks after kc are outstanding.
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

HX_DEV uint4 lds_ld16(const lds_u8* p) {
  const u32x4_t v = *(const __attribute__((address_space(3))) u32x4_t*)p;
  return make_uint4(v.x, v.y, v.z, v.w);
}
HX_DEV uint2 lds_ld8(const lds_u8* p) {
  const u32x2_t v = *(const __attribute__((address_space(3))) u32x2_t*)p;
  return make_uint2(v.x, v.y);
}

constexpr int QA_BYTES = PM * 128 * 2;   // A stage
constexpr int QB_ROW = 80;                // B bytes per weight row per chunk

// FPW: B fragments per matrix per wave; NW: waves per workgroup
template <int FPW, int NW>
struct Q4k {
  static constexpr int FPW_ = FPW;
  static constexpr int NT = 64 * NW;
  static constexpr int COLS = 16 * FPW * NW;             // gate (and up) columns of a tile
  static constexpr int BROWS = 2 * COLS;                 // gate + up weight rows
  static constexpr int STAGE = QA_BYTES + BROWS * QB_ROW;
  static constexpr int NST = 2;                          // ring stages
  static constexpr int NA = 1024 / NT;                   // A DMA rounds
  static constexpr int BPIECES = 5 * BROWS;              // 16-byte pieces of B per chunk
  static constexpr int NBI = (BPIECES + NT - 1) / NT;    // B DMA rounds
  // DMA instructions per chunk of wave w for a tile of MT sub-tiles
  HX_DEV static int per_wave(int w, int MT) {
    return (MT < NA ? MT : NA) + (BPIECES - NT * (NBI - 1) > 64 * w ? NBI : NBI - 1);
  }
};

// Ring layout for tiles of MT sub-tiles: tiles of at most 16 rows (most of
// them at the 512-token prefill chunk) need 4 KB of A per stage, so their ring
// has 3 stages, two chunks ahead, in the LDS of the 2-stage ring of the rest.
template <class Q, int MT>
struct QStage {
  static constexpr int A = MT == 1 ? 16 * 128 * 2 : QA_BYTES;
  static constexpr int SIZE = A + Q::BROWS * QB_ROW;
  static constexpr int NST = MT == 1 ? 3 : 2;
  static_assert(NST * SIZE <= Q::NST * Q::STAGE, "the stages fit the ring");
};

// Per-thread DMA sources of chunk 0; chunk kc adds 256 kc bytes to the A
// sources and (kc / 2) 64 * 144 bytes (+ 64 for odd kc on qs pieces) to the B
// ones (the weight rows n0 .. n0 + 63 are one full group of the stored layout:
// each superblock of the 64 rows one contiguous 9,216-byte run).
// A: thread t moves piece t % 16 (stored at slot t % 16, holding K segment
// (t % 16) ^ (row % 16)) of rows t / 16 + (NT / 16) i.  B: piece q = NT i + t
// is part q % 5 of weight row q / 5: the header (part 0) or 16 qs bytes
// (parts 1..4).
template <class Q>
struct Q4kSrc {
  const uint8_t* a[Q::NA];
  const uint8_t* b[Q::NBI];
  uint32_t bq;   // bit i: b[i] is a qs piece
};

template <class Q>
HX_DEV Q4kSrc<Q> q4k_sources(const uint16_t* xh, int H, const int* rowsrc, const uint8_t* G, const uint8_t* U,
                             int n0, int R, int K) {
  const int tid = threadIdx.x;
  Q4kSrc<Q> src;
  const int sl = tid & 15, r0 = tid >> 4, seg = sl ^ (r0 & 15);
#pragma unroll
  for (int i = 0; i < Q::NA; i++) src.a[i] = (const uint8_t*)(xh + (int64_t)rowsrc[r0 + (Q::NT / 16) * i] * H + 8 * seg);
  src.bq = 0;
#pragma unroll
  for (int i = 0; i < Q::NBI; i++) {
    const int q = i * Q::NT + tid < Q::BPIECES ? i * Q::NT + tid : 0, row = q / 5, part = q - 5 * row;
    const uint8_t* mat = row < Q::COLS ? G : U;
    const uint8_t* sbp = q4k_sb(mat, R, K, n0 + (row < Q::COLS ? row : row - Q::COLS), 0);
    src.b[i] = part == 0 ? sbp : sbp + 16 * part;
    src.bq |= (part != 0 ? 1u : 0u) << i;
  }
  return src;
}

// DMA of chunk kc into stage st; A round i moves token rows 16 i .. 16 i + 15
// (sub-tile i), so a tile of MT sub-tiles needs the first MT rounds only
template <class Q, int MT>
HX_DEV void q4k_issue(uint32_t lds0, int st, const Q4kSrc<Q>& src, int kc, int wave_u) {
  static_assert(Q::NT == 256, "A round i = rows 16 i .. 16 i + 15");
  using S = QStage<Q, MT>;
  const uint32_t sbase = lds0 + (uint32_t)(st * S::SIZE + wave_u * 64 * 16);
#pragma unroll
  for (int i = 0; i < (MT < Q::NA ? MT : Q::NA); i++) dma16(src.a[i] + 256 * kc, sbase + (uint32_t)(i * Q::NT * 16));
  static_assert(Q::COLS == HX_Q4K_GROUP, "a tile's weight rows are one group of the stored layout");
  const int hdr_off = (kc >> 1) * (HX_Q4K_GROUP * 144), qs_off = hdr_off + 64 * (kc & 1);
#pragma unroll
  for (int i = 0; i < Q::NBI; i++) {
    if (i * Q::NT + 64 * wave_u >= Q::BPIECES) break;   // the last round may cover fewer waves
    dma16(src.b[i] + ((src.bq >> i) & 1 ? qs_off : hdr_off), sbase + (uint32_t)(S::A + i * Q::NT * 16));
  }
}

// f16 (a, nb) of sub-blocks 4 PAR .. 4 PAR + 3 of a Q4_K superblock header:
// a = d sc, nb = -dmin m, each one f16 rounding of the exact product (as in
// h2s(d * (float)sc)); the 6-bit sc and m of the four sub-blocks are
// gathered into the bytes of one word, turned into exact f16 integers by the
// 1024 magic and scaled two at a time.
template <int PAR>
HX_DEV void q4k_scales(const uint4& hdr, uint32_t kbyte, uint32_t kmagic, h2_t* a, h2_t* nb) {
  uint32_t scb, mb;
  if (PAR == 0) {
    scb = hdr.y & 0x3F3F3F3Fu;
    mb = hdr.z & 0x3F3F3F3Fu;
  } else {
    scb = (hdr.w & 0x0F0F0F0Fu) | ((hdr.y >> 2) & 0x30303030u);
    mb = ((hdr.w >> 4) & 0x0F0F0F0Fu) | ((hdr.z >> 2) & 0x30303030u);
  }
  const h2_t dm = h2(hdr.x), off = h2s(-1024.0f);
  const h2_t d2 = __builtin_shufflevector(dm, dm, 0, 0), nm2 = -__builtin_shufflevector(dm, dm, 1, 1);
  // (1024 + v) d + (-1024 d) = v d exactly inside the fused multiply-add
  // (-1024 d is exact: a power-of-two scale), so one rounding of v d, as from
  // subtracting the magic first and multiplying
  const h2_t cd = d2 * off, cm = nm2 * off;
  const h2_t s02 = __builtin_elementwise_fma(h2(and_or(scb, kbyte, kmagic)), d2, cd);
  const h2_t s13 = __builtin_elementwise_fma(h2(and_or(scb >> 8, kbyte, kmagic)), d2, cd);
  const h2_t m02 = __builtin_elementwise_fma(h2(and_or(mb, kbyte, kmagic)), nm2, cm);
  const h2_t m13 = __builtin_elementwise_fma(h2(and_or(mb >> 8, kbyte, kmagic)), nm2, cm);
  a[0] = __builtin_shufflevector(s02, s02, 0, 0);
  a[1] = __builtin_shufflevector(s13, s13, 0, 0);
  a[2] = __builtin_shufflevector(s02, s02, 1, 1);
  a[3] = __builtin_shufflevector(s13, s13, 1, 1);
  nb[0] = __builtin_shufflevector(m02, m02, 0, 0);
  nb[1] = __builtin_shufflevector(m13, m13, 0, 0);
  nb[2] = __builtin_shufflevector(m02, m02, 1, 1);
  nb[3] = __builtin_shufflevector(m13, m13, 1, 1);
}

// MT: 16-row M sub-tiles in use (the tile's rows rounded up to 16)
template <class Q, int PAR, int MT>   // chunk parity: sub-blocks 4 PAR .. 4 PAR + 3 of the superblock
HX_DEV void q4k_compute(const lds_u8* st, f32x4_t (*accg)[Q::FPW_], f32x4_t (*accu)[Q::FPW_], int wave, int l16, int kq,
                        uint32_t knib, uint32_t kbyte, uint32_t kmagic) {
  constexpr int NF = Q::FPW_;
  const lds_u8* B = st + QStage<Q, MT>::A;
  constexpr int NB = 2 * NF;   // B fragments of the wave: gate j, then up j
  uint4 hdr[NB];
  uint2 qs[NB][2];
#pragma unroll
  for (int f = 0; f < NB; f++) {
    const int row = (f < NF ? 0 : Q::COLS) + 16 * (NF * wave + f % NF) + l16;
    hdr[f] = lds_ld16(B + row * QB_ROW);
    // two 8-byte reads: the compiler would merge them into one ds_read2_b64,
    // whose two addresses 32 B apart in rows 80 B apart conflict in the LDS
    // banks (measured ~3x the cycles of the two reads); the empty asm hides
    // the relation between the addresses
    uint32_t q0 = row * QB_ROW + 16 + 8 * kq, q1 = q0 + 32;
    asm volatile("" : "+v"(q1));
    qs[f][0] = lds_ld8(B + q0);
    qs[f][1] = lds_ld8(B + q1);
  }
  h2_t a[NB][4], nb[NB][4];
#pragma unroll
  for (int f = 0; f < NB; f++) q4k_scales<PAR>(hdr[f], kbyte, kmagic, a[f], nb[f]);
  // the four nibbles of a word, one per byte (the high ones shifted down), are
  // FP8 E4M3 codes 0x0u, whose value is u 2^-9 for every u < 16 (denormal
  // below 8), so v_cvt_scalef32_pk_f16_fp8 with scale 2^9 gives the codes of
  // two adjacent bytes as the exact f16 pair (u, u'); then a u + nb with one
  // rounding, as before. K is in natural order here (the tokens are stored so).
#pragma unroll
  for (int s = 0; s < 4; s++) {
    const int g = s >> 1, hi = s & 1;
    f16x8_t bf[NB];
#pragma unroll
    for (int f = 0; f < NB; f++) {
      const uint32_t w0 = qs[f][g].x, w1 = qs[f][g].y;
      const uint32_t n0 = (hi ? w0 >> 4 : w0) & 0x0F0F0F0Fu, n1 = (hi ? w1 >> 4 : w1) & 0x0F0F0F0Fu;
      const h2_t u0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(n0, 512.0f, false);
      const h2_t u1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(n0, 512.0f, true);
      const h2_t u2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(n1, 512.0f, false);
      const h2_t u3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(n1, 512.0f, true);
      bf[f] = __builtin_bit_cast(f16x8_t, make_uint4(u32(__builtin_elementwise_fma(u0, a[f][s], nb[f][s])),
                                                     u32(__builtin_elementwise_fma(u1, a[f][s], nb[f][s])),
                                                     u32(__builtin_elementwise_fma(u2, a[f][s], nb[f][s])),
                                                     u32(__builtin_elementwise_fma(u3, a[f][s], nb[f][s]))));
    }
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
      const int row = 16 * mt + l16, seg = 4 * s + kq;
      const f16x8_t av = __builtin_bit_cast(f16x8_t, *(const __attribute__((address_space(3))) u32x4_t*)(st + row * 256 + ((seg ^ l16) << 4)));
#pragma unroll
      for (int j = 0; j < NF; j++) {
        accg[mt][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bf[j], accg[mt][j], 0, 0, 0);
        accu[mt][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bf[NF + j], accu[mt][j], 0, 0, 0);
      }
    }
  }
}

// wait until at most `ahead` chunks of this wave's DMAs are outstanding;
// `ahead` and the count are wave-uniform, so the branches are scalar
template <class Q, int MT>
HX_DEV void q4k_wait(int ahead, int wave_u) {
  const int n = ahead * Q::per_wave(wave_u, MT);
  switch (n) {   // counts not listed wait for everything (correct, only later)
    case 3: asm volatile("s_waitcnt vmcnt(3)" ::: "memory"); break;
    case 4: asm volatile("s_waitcnt vmcnt(4)" ::: "memory"); break;
    case 5: asm volatile("s_waitcnt vmcnt(5)" ::: "memory"); break;
    case 6: asm volatile("s_waitcnt vmcnt(6)" ::: "memory"); break;
    case 7: asm volatile("s_waitcnt vmcnt(7)" ::: "memory"); break;
    case 8: asm volatile("s_waitcnt vmcnt(8)" ::: "memory"); break;
    case 9: asm volatile("s_waitcnt vmcnt(9)" ::: "memory"); break;
    case 10: asm volatile("s_waitcnt vmcnt(10)" ::: "memory"); break;
    case 18: asm volatile("s_waitcnt vmcnt(18)" ::: "memory"); break;
    default: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
  }
}

// the K loop and epilogue of k_gate_up_q4k for tiles of at most 16 MT rows:
// DMAs, activation-fragment reads and MFMAs only for the sub-tiles in use
// qa: the tile's expert call takes the quantised arm (m <= HX_QUANT_M): its
// tokens are the f16 d q operands and h goes out in f32 for quantisation;
// otherwise the f16 arm: gate and up rounded to f16 (the reference's
// forward_via_f16 output), h = silu(g) u rounded to f16 as the down input
template <class Q, int MT>
HX_DEV void q4k_main(const ExpertArgs& a, uint8_t* ring, const Q4kSrc<Q>& src, int nk, int rows, int p0, int n0,
                     int wave, int wave_u, int l16, int kq, uint32_t knib, uint32_t kbyte, uint32_t kmagic, bool qa) {
  constexpr int FPW = Q::FPW_;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_u8*)ring;
  f32x4_t accg[MT][FPW], accu[MT][FPW];
#pragma unroll
  for (int i = 0; i < MT; i++)
#pragma unroll
    for (int j = 0; j < FPW; j++) {
      accg[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      accu[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
  using S = QStage<Q, MT>;
#pragma unroll
  for (int c = 0; c < S::NST - 1; c++)
    if (c < nk) q4k_issue<Q, MT>(lds0, c, src, c, wave_u);
  // chunk kc: wait for its DMAs, issue chunk kc + NST - 1's, then its MFMAs;
  // the loop takes the two chunks of a superblock per iteration (nk is even),
  // so both parities are straight-line code and the accumulators stay in place
  // (one parity branch per chunk made the compiler copy them back each time)
  auto step = [&](int kc, auto par) __attribute__((always_inline)) {
    const int ahead = min(S::NST - 2, nk - 1 - kc);
    q4k_wait<Q, MT>(ahead, wave_u);
    __syncthreads();   // chunk kc is in LDS for every wave; stage (kc - 1) % NST is free
    if (kc + S::NST - 1 < nk) q4k_issue<Q, MT>(lds0, (kc + S::NST - 1) % S::NST, src, kc + S::NST - 1, wave_u);
    const lds_u8* st = (const lds_u8*)ring + (kc % S::NST) * S::SIZE;
    q4k_compute<Q, decltype(par)::value, MT>(st, accg, accu, wave, l16, kq, knib, kbyte, kmagic);
  };
  for (int kc = 0; kc < nk; kc += 2) {
    step(kc, std::integral_constant<int, 0>{});
    step(kc + 1, std::integral_constant<int, 1>{});
  }
  __syncthreads();   // every wave is done with the ring
  if (qa) {
    // the 16 MT x COLS f32 rows of h (natural column order, row pitch
    // COLS + 4) through LDS, out as 16-byte pieces into hbuf
    constexpr int OP = Q::COLS + 4;
    float* ot = (float*)ring;
#pragma unroll
    for (int j = 0; j < FPW; j++) {
      const int col = 16 * (FPW * wave + j) + l16;
#pragma unroll
      for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int i = 0; i < 4; i++) ot[(16 * mt + 4 * kq + i) * OP + col] = silu_rcp(accg[mt][j][i]) * accu[mt][j][i];
    }
    __syncthreads();
    constexpr int PER_ROW = Q::COLS / 4;
    constexpr int RSTEP = Q::NT / PER_ROW;
    const int m0 = threadIdx.x / PER_ROW, c4 = (threadIdx.x % PER_ROW) * 4;
    float* hrow = a.hbuf + (int64_t)(p0 + m0) * a.hstride + n0 + c4;
#pragma unroll
    for (int m = m0; m < 16 * MT; m += RSTEP, hrow += (int64_t)RSTEP * a.hstride)
      if (m < rows) *(float4*)hrow = *(const float4*)(ot + m * OP + c4);
    return;
  }
  // the 16 MT x COLS f16 rows of h go through LDS (columns in the swizzled
  // order, row pitch COLS + 8) and out as 16-byte pieces
  constexpr int OP = Q::COLS + 8;
  _Float16* ot = (_Float16*)ring;
#pragma unroll
  for (int j = 0; j < FPW; j++) {
    const int col = swz(16 * (FPW * wave + j) + l16);
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int m = 16 * mt + 4 * kq + i;
        const float g = (float)(_Float16)accg[mt][j][i], u = (float)(_Float16)accu[mt][j][i];
        ot[m * OP + col] = (_Float16)(silu_rcp(g) * u);
      }
  }
  __syncthreads();
  constexpr int PER_ROW = Q::COLS / 8;
  static_assert(Q::NT % PER_ROW == 0, "a thread keeps its column piece");
  constexpr int RSTEP = Q::NT / PER_ROW;   // rows one pass of the workgroup stores
  const int m0 = threadIdx.x / PER_ROW, c8 = (threadIdx.x % PER_ROW) * 8;
  _Float16* hrow = (_Float16*)a.hbf + (int64_t)(p0 + m0) * a.hstride + n0 + c8;
#pragma unroll
  for (int m = m0; m < 16 * MT; m += RSTEP, hrow += (int64_t)RSTEP * a.hstride)
    if (m < rows) *(uint4*)hrow = *(const uint4*)(ot + m * OP + c8);
}

// grid (I / COLS, tiles rounded up to 8), mapped by xcd_tile
// (the second bound is waves per SIMD: 3 workgroups of 4 waves per CU)
template <int FPW, int NW, int TS>
__global__ __launch_bounds__(64 * NW, 3) void k_gate_up_q4k(ExpertArgs a) {
  using Q = Q4k<FPW, NW>;
  __shared__ __attribute__((aligned(16))) uint8_t ring[Q::NST * Q::STAGE];
  __shared__ int rowsrc[PM];
  int nt, tile;
  xcd_tile(nt, tile);
  int e, p0, rows, mc;
  if (!get_tile<TS>(a, tile, e, p0, rows, mc)) return;
  const bool sh = e == a.E, qa = mc <= HX_QUANT_M;
  const int n0 = nt * Q::COLS;
  const uint8_t* G = sh ? a.sgate.base : a.gate.mat(e);
  const uint8_t* U = sh ? a.sup.base : a.up.mat(e);
  const int K = a.H, nk = K / 128;
  if (threadIdx.x < PM) {
    const int p = p0 + (threadIdx.x < rows ? threadIdx.x : 0);   // padding rows repeat row 0
    rowsrc[threadIdx.x] = sh ? p - a.F : a.perm[p] / a.k;
  }
  __syncthreads();
  const int lane = lane_id(), wave = threadIdx.x >> 6, l16 = lane & 15, kq = lane >> 4;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  const Q4kSrc<Q> src = q4k_sources<Q>(qa ? a.xq : a.xh, a.H, rowsrc, G, U, n0, sh ? a.Is : a.I, K);
  // dequantisation constants, kept in registers for v_and_or_b32
  const uint32_t knib = __builtin_amdgcn_readfirstlane(0x000F000Fu), kbyte = __builtin_amdgcn_readfirstlane(0x00FF00FFu);
  uint32_t kmagic;
  asm("v_mov_b32 %0, 0x64006400" : "=v"(kmagic));
  switch ((rows + 15) >> 4) {   // uniform over the workgroup
    case 1: q4k_main<Q, 1>(a, ring, src, nk, rows, p0, n0, wave, wave_u, l16, kq, knib, kbyte, kmagic, qa); break;
    case 2: q4k_main<Q, 2>(a, ring, src, nk, rows, p0, n0, wave, wave_u, l16, kq, knib, kbyte, kmagic, qa); break;
    case 3: q4k_main<Q, 3>(a, ring, src, nk, rows, p0, n0, wave, wave_u, l16, kq, knib, kbyte, kmagic, qa); break;
    default: q4k_main<Q, 4>(a, ring, src, nk, rows, p0, n0, wave, wave_u, l16, kq, knib, kbyte, kmagic, qa); break;
  }
}

// ---------------------------------------------------------------- Q6_K down, streamed
// k_down_q6k: h . W_d^T for Q6_K down projections with K = I = 512, the
// operands streamed into LDS by global_load_lds_{dwordx4,dword} through a
// 3-stage ring, two chunks ahead (3 workgroups per CU: about 100 KB in flight
// per CU). Tile: 64 rows of h (contiguous in the dispatch order, f16, K
// swizzled as the gate/up epilogue wrote it) x 128 output columns; wave w owns
// columns 32w .. 32w + 31 (two B fragments).
// K chunk c (8 per row) = the quarters {p, p + 2} (p = c & 1) of half
// n = (c >> 1) & 1 of superblock c >> 2: those two quarters share their ql
// bytes (low and high nibbles) and the half's qh bytes, so a chunk needs per
// weight row 32 ql + 32 qh bytes, with the half's 8 scales beside them.
//   stage: A = 64 rows x 64 K (8 KB; the row's 8 16-byte pieces stored at
//          slot piece ^ ((row >> 1) & 7)); B = 64 B per weight row (its four
//          16-byte parts stored at slot part ^ ((row >> 2) & 3)); S = 8 B per row;
//   once per tile: d of both superblocks of each weight row (4 B).
// The two swizzles make the fragment reads conflict-free: the 16 rows of an
// A fragment (128 B apart, so rows 2 apart share banks) read 16 different
// 16-byte bank groups, and the 32 lanes of a B read (16 rows 64 B apart, two
// 8-byte halves) cover the 64 banks once. (With slot piece ^ (row % 8) and
// unswizzled B rows, bank conflicts took 2/3 of the kernel's LDS cycles and
// the kernel 5-8 % longer.)
// Dequantisation in registers: q = ql nibble | (qh bits << 4) under the 0x6400
// f16 pattern (1024 + q, exact), (x - 1056) * (d * sc) with packed f16 ops.
// Rows are scaled by their routing weight by position (the shared expert's
// rows by its sigmoid gate) and written as bf16 to the per-assignment rows.
constexpr int DQ_A = PM * 64 * 2;
constexpr int DQ_BROW = 64;
constexpr int DQ_B = 128 * DQ_BROW;
constexpr int DQ_S = 128 * 8;
constexpr int DQ_STAGE = DQ_A + DQ_B + DQ_S;
constexpr int DQ_NST = 3;
constexpr int DQ_K = 512;
constexpr int DQ_NC = DQ_K / 64;


// first K column of chunk c: 256 (c >> 2) + 128 ((c >> 1) & 1) + 32 (c & 1)
HX_DEV int dq_col(int c) { return 256 * (c >> 2) + 128 * ((c >> 1) & 1) + 32 * (c & 1); }

// Per-thread DMA sources of chunk 0. Chunk c adds 2 dq_col(c) bytes to the A
// sources; the 128 weight rows n0 .. n0 + 127 are whole groups of G rows in the
// stored layout, so in each group chunk c's ql pieces (piece c of each row) are
// the run c of 32 G bytes, its qh pieces (piece c / 2) the run c / 2, and its
// scales 8 n bytes into the run sb of 16-byte pieces.
// A piece q = 256 i + t: row q / 8, slot q % 8 holding segment
// (q % 8) ^ ((row / 2) % 8): segments 0..3 are K columns 8 s .. of quarter p,
// 4..7 of quarter p + 2 (64 columns further). B piece q = 256 i + t: slot q % 4
// of weight row q / 4, holding part (q % 4) ^ ((row / 4) % 4) (ql bytes
// 16 part for parts 0, 1; qh bytes 16 (part - 2)).
// Scale dword t: row t / 2, half t % 2.
struct DqSrc {
  const uint8_t* a[2];
  const uint8_t* b[2];
  const uint8_t* s;
  uint32_t bqh;   // bit i: b[i] is a qh piece
};

HX_DEV DqSrc dq_sources(const uint16_t* hbf, int hstride, int p0, int rows, const uint8_t* W, int R, int n0) {
  const int tid = threadIdx.x;
  DqSrc src;
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const int q = i * 256 + tid, row = q >> 3, seg = (q & 7) ^ ((row >> 1) & 7);
    const int r = min(row, rows - 1);   // padding rows repeat the last row
    src.a[i] = (const uint8_t*)(hbf + (int64_t)(p0 + r) * hstride + 64 * (seg >> 2) + 8 * (seg & 3));
  }
  src.bqh = 0;
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const int q = i * 256 + tid, row = q >> 2, part = (q & 3) ^ ((row >> 2) & 3);
    src.b[i] = part < 2 ? q6k_ql(W, R, DQ_K, n0 + row, 16 * part) : q6k_qh(W, R, DQ_K, n0 + row, 16 * (part - 2));
    src.bqh |= (part >= 2 ? 1u : 0u) << i;
  }
  src.s = q6k_sc(W, R, DQ_K, n0 + (tid >> 1), 4 * (tid & 1));
  return src;
}

// NA + 3 DMA instructions per wave and chunk: A round i moves rows
// 32 i .. 32 i + 31 of h, so tiles of at most 32 rows (NA = 1) skip round 1
template <int NA>
HX_DEV void dq_issue(uint32_t lds0, int st, const DqSrc& src, int c, int wave_u) {
  const uint32_t sbase = lds0 + (uint32_t)(st * DQ_STAGE);
  const int sb = c >> 2, n = (c >> 1) & 1;
  static_assert(128 % HX_Q6K_GROUP == 0, "a down tile's weight rows are whole groups of the stored layout");
  const int aoff = 2 * dq_col(c), qloff = c * (HX_Q6K_GROUP * 32), qhoff = (c >> 1) * (HX_Q6K_GROUP * 32);
#pragma unroll
  for (int i = 0; i < NA; i++) dma16(src.a[i] + aoff, sbase + (uint32_t)(i * 4096 + wave_u * 1024));
#pragma unroll
  for (int i = 0; i < 2; i++)
    dma16(src.b[i] + ((src.bqh >> i) & 1 ? qhoff : qloff), sbase + (uint32_t)(DQ_A + i * 4096 + wave_u * 1024));
  dma4(src.s + sb * (HX_Q6K_GROUP * 16) + 8 * n, sbase + (uint32_t)(DQ_A + DQ_B + wave_u * 256));
}

// (lo4 & 0x000F000F) | 0x64006400 | (hi2 & 0x00300030): two 6-bit codes as 1024 + q
HX_DEV uint32_t q6_pair(uint32_t lo4, uint32_t hi2, uint32_t knib, uint32_t kmagic, uint32_t k30) {
  return and_or(hi2, k30, and_or(lo4, knib, kmagic));
}

// MT: 16-row M sub-tiles in use
template <int P, int MT>   // chunk parity: quarters P and P + 2 of the half
HX_DEV void dq_compute(const lds_u8* st, const uint16_t* dl, int sb, f32x4_t (*acc)[4], int wave, int l16, int kq,
                       uint32_t knib, uint32_t kmagic, uint32_t k30) {
  const h2_t off = h2s(-1056.0f);
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int brow = 32 * wave + 16 * j + l16;
    const lds_u8* B = st + DQ_A + brow * DQ_BROW;
    // ql bytes 8 kq .. (part kq / 2) and qh bytes 8 kq .. (part 2 + kq / 2); brow / 4 % 4 = l16 / 4
    const int sw = (l16 >> 2) & 3, hk = 8 * (kq & 1);
    const uint2 ql = lds_ld8(B + 16 * ((kq >> 1) ^ sw) + hk), qh = lds_ld8(B + 16 * ((2 + (kq >> 1)) ^ sw) + hk);
    const uint2 sc = lds_ld8(st + DQ_A + DQ_B + brow * 8);
    const float d = f16_to_f32(dl[2 * brow + sb]);
    const int sh = 8 * (kq >> 1);
#pragma unroll
    for (int t = 0; t < 2; t++) {   // MFMA step t: quarter q = P + 2 t, ql nibble t
      constexpr int Q0 = P;
      const int q = Q0 + 2 * t;
      const uint32_t sw = q < 2 ? sc.x : sc.y;   // scale 2 q + kq / 2 of the half
      const h2_t a = h2s(d * (float)(int8_t)((sw >> (16 * (q & 1) + sh)) & 0xffu));
      const uint32_t wx = ql.x >> (4 * t), wy = ql.y >> (4 * t);
      const uint32_t hx_ = q < 3 ? qh.x << (4 - 2 * q) : qh.x >> 2, hy = q < 3 ? qh.y << (4 - 2 * q) : qh.y >> 2;
      const f16x8_t bf = __builtin_bit_cast(
          f16x8_t, make_uint4(u32((h2(q6_pair(wx, hx_, knib, kmagic, k30)) + off) * a),
                              u32((h2(q6_pair(wx >> 8, hx_ >> 8, knib, kmagic, k30)) + off) * a),
                              u32((h2(q6_pair(wy, hy, knib, kmagic, k30)) + off) * a),
                              u32((h2(q6_pair(wy >> 8, hy >> 8, knib, kmagic, k30)) + off) * a)));
#pragma unroll
      for (int mt = 0; mt < MT; mt++) {
        const int row = 16 * mt + l16, seg = 4 * t + kq;
        const f16x8_t av = __builtin_bit_cast(
            f16x8_t, *(const __attribute__((address_space(3))) u32x4_t*)(st + row * 128 + ((seg ^ ((l16 >> 1) & 7)) << 4)));
        acc[j][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bf, acc[j][mt], 0, 0, 0);
      }
    }
  }
}

// grid (H / 128, tiles rounded up to 8), mapped by xcd_tile
// the K loop and epilogue of k_down_q6k for tiles of at most 16 MT rows (MFMAs,
// activation-fragment reads and A DMA rounds for the sub-tiles in use)
// fa: the f16 arm (m > HX_QUANT_M): the products rounded to f16 (the
// reference's forward_via_f16 output) before the routing weight
template <int MT>
HX_DEV void dq_main(const ExpertArgs& a, uint8_t* ring, float* rws, const DqSrc& src, float rw, int rows, int p0,
                    int n0, int wave, int wave_u, int l16, int kq, bool fa) {
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_u8*)ring;
  const uint16_t* dl = (const uint16_t*)(ring + DQ_NST * DQ_STAGE);
  constexpr int NA = MT <= 2 ? 1 : 2;   // A rounds (32 rows each) the tile needs
#pragma unroll
  for (int c = 0; c < DQ_NST - 1; c++) dq_issue<NA>(lds0, c, src, c, wave_u);
  const uint32_t knib = __builtin_amdgcn_readfirstlane(0x000F000Fu), k30 = __builtin_amdgcn_readfirstlane(0x00300030u);
  uint32_t kmagic;
  asm("v_mov_b32 %0, 0x64006400" : "=v"(kmagic));
  f32x4_t acc[2][4];
#pragma unroll
  for (int j = 0; j < 2; j++)
#pragma unroll
    for (int i = 0; i < MT; i++) acc[j][i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // two chunks per iteration (DQ_NC is even), so both parities are
  // straight-line code and the accumulators stay in place
  auto step = [&](int c, auto par) __attribute__((always_inline)) {
    // chunk c (and, before chunk 0, the d dwords) has landed once at most the
    // NA + 3 DMAs of chunk c + 1 are outstanding
    if (c + 1 < DQ_NC) {
      if (NA == 1) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
      else asm volatile("s_waitcnt vmcnt(5)" ::: "memory");
    } else {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    __syncthreads();   // chunk c is in LDS for every wave; stage (c - 1) % NST is free
    if (c + DQ_NST - 1 < DQ_NC) dq_issue<NA>(lds0, (c + DQ_NST - 1) % DQ_NST, src, c + DQ_NST - 1, wave_u);
    const lds_u8* st = (const lds_u8*)ring + (c % DQ_NST) * DQ_STAGE;
    dq_compute<decltype(par)::value, MT>(st, dl, c >> 2, acc, wave, l16, kq, knib, kmagic, k30);
  };
  static_assert(DQ_NC % 2 == 0, "chunks come in pairs");
  for (int c = 0; c < DQ_NC; c += 2) {
    step(c, std::integral_constant<int, 0>{});
    step(c + 1, std::integral_constant<int, 1>{});
  }
  if (threadIdx.x < PM) rws[threadIdx.x] = rw;
  __syncthreads();   // also: every wave is done with the ring
  // the 16 MT x 128 bf16 output rows go through LDS (row pitch 272 B, so the
  // 16 lanes of a row group write different banks) and out as 16-byte pieces
  constexpr int OP = 136;   // pitch in bf16
  uint16_t* ot = (uint16_t*)ring;
#pragma unroll
  for (int mt = 0; mt < MT; mt++) {
    // the weights of this lane's rows 16 mt + 4 kq .. + 3, one 16-byte read
    const float4 w4 = *(const float4*)(rws + 16 * mt + 4 * kq);
    const float wv[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int col = 32 * wave + 16 * j + l16;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float v = fa ? (float)(_Float16)acc[j][mt][i] : acc[j][mt][i];
        ot[(16 * mt + 4 * kq + i) * OP + col] = f32_to_bf16(wv[i] * v);
      }
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0, m = threadIdx.x >> 4; i < MT; i++, m += 16) {
    const int c8 = (threadIdx.x & 15) * 8;
    if (m < rows)
      *(uint4*)((uint16_t*)a.obuf + (int64_t)(p0 + (threadIdx.x >> 4)) * a.H + (int64_t)(16 * i) * a.H + n0 + c8) =
          *(const uint4*)(ot + m * OP + c8);
  }
}

template <int TS>
__global__ __launch_bounds__(256, 3) void k_down_q6k(ExpertArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t ring[DQ_NST * DQ_STAGE + 128 * 4];
  __shared__ __attribute__((aligned(16))) float rws[PM];
  int nt, tile;
  xcd_tile(nt, tile);
  int e, p0, rows, mc;
  if (!get_tile<TS>(a, tile, e, p0, rows, mc)) return;
  const bool fa = mc > HX_QUANT_M;
  const bool sh = e == a.E;
  const int n0 = nt * 128;
  const uint8_t* W = sh ? a.sdown.base : a.down.mat(e);
  const int lane = lane_id(), wave = threadIdx.x >> 6, l16 = lane & 15, kq = lane >> 4;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  // routing weights, loaded before the DMAs and first used after the last one
  const float rw = threadIdx.x >= PM ? 0.f : e == a.E && a.shared_raw ? 1.f : a.wpos[p0 + min((int)threadIdx.x, rows - 1)];
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_u8*)ring;
  // d of both superblocks of the 128 weight rows (waves 0 and 1, one dword each)
  if (wave_u < 2)
    dma4(W + (int64_t)a.H * (DQ_K / 2 + DQ_K / 4 + DQ_K / 16) + (int64_t)(n0 + 64 * wave_u + lane) * 4,
         lds0 + (uint32_t)(DQ_NST * DQ_STAGE + wave_u * 256));
  const DqSrc src = dq_sources(a.hbf, a.hstride, p0, rows, W, a.H, n0);
  switch ((rows + 15) >> 4) {   // uniform over the workgroup
    case 1: dq_main<1>(a, ring, rws, src, rw, rows, p0, n0, wave, wave_u, l16, kq, fa); break;
    case 2: dq_main<2>(a, ring, rws, src, rw, rows, p0, n0, wave, wave_u, l16, kq, fa); break;
    case 3: dq_main<3>(a, ring, rws, src, rw, rows, p0, n0, wave, wave_u, l16, kq, fa); break;
    default: dq_main<4>(a, ring, rws, src, rw, rows, p0, n0, wave, wave_u, l16, kq, fa); break;
  }
}

// ---------------------------------------------------------------- gate/up
// grid (I / 64, tiles rounded up to 8), mapped by xcd_tile: 64 rows x 64
// intermediate columns; wave w owns columns
// 16w .. 16w+15 of gate and of up for all 64 rows. Quantised arm (m <=
// HX_QUANT_M): the tokens are the f16 d q operands and h = silu(gate) * up goes
// to hbuf in f32; f16 arm: gate and up rounded to f16, h written as f16 in the
// swizzled order.
template <int FMT, int TS>
__global__ __launch_bounds__(256) void k_gate_up_mfma(ExpertArgs a) {
  __shared__ uint16_t As[PM * PLD];
  __shared__ uint16_t Bs[128 * PLD];
  __shared__ int rowsrc[PM];
  int nt, tile;
  xcd_tile(nt, tile);
  int e, p0, rows, mc;
  if (!get_tile<TS>(a, tile, e, p0, rows, mc)) return;
  const bool sh = e == a.E, qa = mc <= HX_QUANT_M;
  const uint16_t* X = qa ? a.xq : a.xh;
  const int I = sh ? a.Is : a.I, n0 = nt * 64;
  if (n0 >= I) return;
  const uint8_t* G = sh ? a.sgate.base : a.gate.mat(e);
  const uint8_t* U = sh ? a.sup.base : a.up.mat(e);
  const int K = a.H, nk = K / PKC;
  if (threadIdx.x < PM) {
    const int p = p0 + threadIdx.x;
    rowsrc[threadIdx.x] = threadIdx.x < rows ? (sh ? p - a.F : a.perm[p] / a.k) : 0;
  }
  __syncthreads();
  const int lane = lane_id(), wave = threadIdx.x >> 6, l16 = lane & 15, kq = lane >> 4;
  // B rows: thread t dequantises half t % 2 of row t / 2 (rows 0..63 gate,
  // 64..127 up): the two threads of a row read adjacent bytes
  const int brow = threadIdx.x >> 1, bpt = threadIdx.x & 1;
  const uint8_t* Wm = brow < 64 ? G : U;
  const int wrow = n0 + (brow & 63);
  f32x4_t accg[4], accu[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    accg[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    accu[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
  ARaw ar;
  PRaw<FMT> br;
  ar.load(X, K, rowsrc, rows, 0);
  br.load(Wm, I, K, wrow, 0, bpt);
  for (int kc = 0; kc < nk; kc++) {
    ar.to_lds(As);
    br.to_lds(Bs + brow * PLD + 64 * bpt);
    if (kc + 1 < nk) {
      ar.load(X, K, rowsrc, rows, kc + 1);
      br.load(Wm, I, K, wrow, kc + 1, bpt);
    }
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < PKC / 32; ks++) {
      const int ko = 32 * ks + 8 * kq;
      const f16x8_t bg = frag(Bs + (16 * wave + l16) * PLD + ko);
      const f16x8_t bu = frag(Bs + (64 + 16 * wave + l16) * PLD + ko);
#pragma unroll
      for (int mt = 0; mt < 4; mt++) {
        const f16x8_t av = frag(As + (16 * mt + l16) * PLD + ko);
        accg[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bg, accg[mt], 0, 0, 0);
        accu[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bu, accu[mt], 0, 0, 0);
      }
    }
    __syncthreads();
  }
  const int coln = n0 + 16 * wave + l16, col = swz(coln);
#pragma unroll
  for (int mt = 0; mt < 4; mt++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int m = 16 * mt + 4 * kq + i;
      if (m >= rows) continue;
      if (qa) {
        a.hbuf[(int64_t)(p0 + m) * a.hstride + coln] = siluf_(accg[mt][i]) * accu[mt][i];
      } else {
        const float g = (float)(_Float16)accg[mt][i], u = (float)(_Float16)accu[mt][i];
        ((_Float16*)a.hbf)[(int64_t)(p0 + m) * a.hstride + col] = (_Float16)(siluf_(g) * u);
      }
    }
}

// ---------------------------------------------------------------- down
// grid (H / 128, tiles rounded up to 8), mapped by xcd_tile: 64 rows x 128
// output columns; wave w owns columns
// 32w .. 32w+31. Rows are scaled by their routing weight (shared expert: the
// sigmoid gate) and written to the per-assignment output rows; in the f16 arm
// (m > HX_QUANT_M) the products are rounded to f16 first.
template <int FMT, int TS>
__global__ __launch_bounds__(256) void k_down_mfma(ExpertArgs a) {
  __shared__ uint16_t As[PM * PLD];
  __shared__ uint16_t Bs[128 * PLD];
  __shared__ int rowsrc[PM];
  __shared__ float rw[PM];
  int nt, tile;
  xcd_tile(nt, tile);
  int e, p0, rows, mc;
  if (!get_tile<TS>(a, tile, e, p0, rows, mc)) return;
  const bool fa = mc > HX_QUANT_M;
  const bool sh = e == a.E;
  const int K = sh ? a.Is : a.I, n0 = nt * 128, nk = K / PKC;
  const uint8_t* W = sh ? a.sdown.base : a.down.mat(e);
  if (threadIdx.x < PM) {
    const int p = p0 + threadIdx.x;
    rowsrc[threadIdx.x] = p0 + (threadIdx.x < rows ? threadIdx.x : 0);
    rw[threadIdx.x] = threadIdx.x < rows ? (sh ? (a.shared_raw ? 1.f : a.sgw[p - a.F]) : a.topk_w[a.perm[p]]) : 0.f;
  }
  __syncthreads();
  const int lane = lane_id(), wave = threadIdx.x >> 6, l16 = lane & 15, kq = lane >> 4;
  const int brow = threadIdx.x >> 1, bpt = threadIdx.x & 1;   // as in the gate/up kernel
  f32x4_t acc[2][4];
#pragma unroll
  for (int j = 0; j < 2; j++)
#pragma unroll
    for (int i = 0; i < 4; i++) acc[j][i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  ARaw ar;
  PRaw<FMT> br;
  ar.load(a.hbf, a.hstride, rowsrc, rows, 0);
  br.load(W, a.H, K, n0 + brow, 0, bpt);
  for (int kc = 0; kc < nk; kc++) {
    ar.to_lds(As);
    br.to_lds(Bs + brow * PLD + 64 * bpt);
    if (kc + 1 < nk) {
      ar.load(a.hbf, a.hstride, rowsrc, rows, kc + 1);
      br.load(W, a.H, K, n0 + brow, kc + 1, bpt);
    }
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < PKC / 32; ks++) {
      const int ko = 32 * ks + 8 * kq;
      f16x8_t bv[2];
#pragma unroll
      for (int j = 0; j < 2; j++) bv[j] = frag(Bs + (32 * wave + 16 * j + l16) * PLD + ko);
#pragma unroll
      for (int mt = 0; mt < 4; mt++) {
        const f16x8_t av = frag(As + (16 * mt + l16) * PLD + ko);
#pragma unroll
        for (int j = 0; j < 2; j++) acc[j][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv[j], acc[j][mt], 0, 0, 0);
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int col = n0 + 32 * wave + 16 * j + l16;
#pragma unroll
    for (int mt = 0; mt < 4; mt++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int m = 16 * mt + 4 * kq + i;
        if (m < rows)
          ((uint16_t*)a.obuf)[(int64_t)(p0 + m) * a.H + col] =
              f32_to_bf16(rw[m] * (fa ? (float)(_Float16)acc[j][mt][i] : acc[j][mt][i]));
      }
  }
}

// ---------------------------------------------------------------- tokens -> f16
// bf16 [T][H] -> f16 [T][H] in the swizzled element order; one thread per 8
__global__ __launch_bounds__(256) void k_x_to_f16(const uint16_t* x, int64_t n8, uint16_t* xh, int nat) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n8) return;
  const uint4 v = ((const uint4*)x)[i];
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  uint32_t h[4];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const h2_t p = {(_Float16)__uint_as_float(w[j] << 16), (_Float16)__uint_as_float(w[j] & 0xffff0000u)};
    h[j] = u32(p);
  }
  uint4 o;   // natural, or (e0,e1)(e2,e3) -> (e0,e2)(e1,e3)
  if (nat) {
    o = make_uint4(h[0], h[1], h[2], h[3]);
  } else {
    o.x = __builtin_amdgcn_perm(h[1], h[0], 0x05040100u);
    o.y = __builtin_amdgcn_perm(h[1], h[0], 0x07060302u);
    o.z = __builtin_amdgcn_perm(h[3], h[2], 0x05040100u);
    o.w = __builtin_amdgcn_perm(h[3], h[2], 0x07060302u);
  }
  ((uint4*)xh)[i] = o;
}

// ---------------------------------------------------------------- launchers
bool prefill_mfma_ok(const ExpertArgs& a) {
  auto q = [](int f) { return f == HX_Q4_K || f == HX_Q8_0 || f == HX_Q6_K; };
  return a.xbf && q(a.gate.fmt) && q(a.down.fmt) && a.H % 256 == 0 && a.I % 256 == 0 && (a.Is == 0 || a.Is == a.I);
}

hipError_t launch_x_to_f16(const ExpertArgs& a, hipStream_t s) {
  const int64_t n8 = (int64_t)a.T * a.H / 8;
  hx_launch(k_x_to_f16, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, s, (const uint16_t*)a.x, n8, a.xh,
            xh_natural(a.gate.fmt) ? 1 : 0);
  return hipGetLastError();
}

// M tiles a launch's grid covers
static int grid_tiles(const ExpertArgs& a) {
  const int n = a.tsel == HX_TILES_SHARED ? (a.T + PM - 1) / PM : a.max_tiles;
  return (n + 7) / 8 * 8;
}

// reads the f16 tokens launch_x_to_f16 wrote
template <int TS>
static hipError_t gate_up_mfma_ts(const ExpertArgs& a, hipStream_t s) {
  const dim3 grid(a.I / 64, grid_tiles(a));
  switch (a.gate.fmt) {
    case HX_Q4_K: hx_launch(k_gate_up_q4k<1, 4, TS>, grid, dim3(256), 0, s, a); break;
    case HX_Q8_0: hx_launch(k_gate_up_mfma<HX_Q8_0, TS>, grid, dim3(256), 0, s, a); break;
    case HX_Q6_K: hx_launch(k_gate_up_mfma<HX_Q6_K, TS>, grid, dim3(256), 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_gate_up_mfma(const ExpertArgs& a, hipStream_t s) {
  switch (a.tsel) {
    case HX_TILES_ROUTED: return gate_up_mfma_ts<HX_TILES_ROUTED>(a, s);
    case HX_TILES_SHARED: return gate_up_mfma_ts<HX_TILES_SHARED>(a, s);
    default: return gate_up_mfma_ts<HX_TILES_ALL>(a, s);
  }
}

template <int TS>
static hipError_t down_mfma_ts(const ExpertArgs& a, hipStream_t s) {
  const dim3 grid(a.H / 128, grid_tiles(a));
  switch (a.down.fmt) {
    case HX_Q4_K: hx_launch(k_down_mfma<HX_Q4_K, TS>, grid, dim3(256), 0, s, a); break;
    case HX_Q8_0: hx_launch(k_down_mfma<HX_Q8_0, TS>, grid, dim3(256), 0, s, a); break;
    case HX_Q6_K:
      if (a.I == DQ_K && (a.wpos || TS == HX_TILES_SHARED)) hx_launch(k_down_q6k<TS>, grid, dim3(256), 0, s, a);
      else hx_launch(k_down_mfma<HX_Q6_K, TS>, grid, dim3(256), 0, s, a);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_down_mfma(const ExpertArgs& a, hipStream_t s) {
  switch (a.tsel) {
    case HX_TILES_ROUTED: return down_mfma_ts<HX_TILES_ROUTED>(a, s);
    case HX_TILES_SHARED: return down_mfma_ts<HX_TILES_SHARED>(a, s);
    default: return down_mfma_ts<HX_TILES_ALL>(a, s);
  }
}

}  // namespace hx
