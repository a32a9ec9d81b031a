// Internal declarations of libhxmoe: kernel argument blocks, launchers and the
// handle. Not part of the C ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <stdint.h>

#include <string>
#include <vector>

#include "hx_formats.h"

// Largest expert count the routing kernels hold in registers / LDS.
#define HX_MAX_EXPERTS 1024
// Largest k (top-k) supported: one lane per selected expert.
#define HX_MAX_TOPK 64
// Token count up to which the decode path (fused routing tail, GEMV experts,
// in-register combine) is used.
#define HX_DECODE_MAX_T 8
// Rows of a grouped-GEMM M tile.
#define HX_TILE_M 64
// Largest row count of an expert call that takes the reference's quantised
// arm (activations quantised to the vec_dot type, integer block products):
// QUANT_PREFILL_M_THRESHOLD (crates/neuron/src/harness/tp/tp_linear.rs:96);
// larger calls take its f16 arm (forward_via_f16, tp_linear.rs:111-118).
#define HX_QUANT_M 64

namespace hx {

// XCD-aware work mapping of the prefill kernels. Workgroups are dealt to the 8
// XCDs round-robin by linear id (XCD = id % 8), each with its own L2. The
// launch grid is (NX, tiles rounded up to 8); linear id L is mapped so that the
// NX workgroups of one M tile land on the same XCD, XCD tile % 8: the tile's
// gathered activation rows are fetched into one L2 and read from there by all
// NX workgroups, and every kernel of a forward that works on a tile's rows
// (gate/up, the quantisation of h, down) finds them in that L2.
__device__ __forceinline__ void xcd_tile(int& nt, int& tile) {
  const int NX = gridDim.x, L = blockIdx.y * NX + blockIdx.x;
  const int group = L / (8 * NX), xcd = L & 7;
  nt = (L >> 3) % NX;
  tile = group * 8 + xcd;
}

struct DispatchArgs {
  int32_t* topk_idx;   // [T*k] (input)
  int T, k, E, F;
  bool has_shared;
  int tile_m;
  int32_t* perm;       // [F]
  int32_t* inv;        // [F] or null
  int32_t* offsets;    // [E+1]
  int32_t* slots;      // [(min(F,E)+1) * 3]: expert, start position, count
  int32_t* tiles;      // [max_tiles * 4]: rows of the expert's call (its count; T for the
                       // shared expert), expert, start position, rows of the tile
  int32_t* counts;     // [2]: number of slots, number of tiles
  int32_t* plan;       // decode plan (written by the decode routing tail), see plan_ints()
  int max_slots;
  // the decode routing tail writes the plan only (a forward reads nothing else;
  // topk_idx, perm, inv, offsets, slots and counts are left as they were)
  bool plan_only = false;
  // prefill dispatch: hist[c][e] = entries of
  // expert e among the tokens of chunk c (HX_DISPATCH_TOK tokens), which the
  // scan turns into the position in perm of the chunk's first such entry; bit
  // j of bits[w][e] is set when token 32 w + j has expert e among its top k.
  // The two are one block of (dispatch_chunks(T) + dispatch_words(T)) E ints,
  // hist first.
  int32_t* hist;       // [dispatch_chunks(T)][E]
  uint32_t* bits;      // [dispatch_words(T)][E]
  // prefill: routing weight by permuted position, wpos[p] = topk_w[perm[p]],
  // and the shared expert's sigmoid gate at wpos[F + t]
  const float* topk_w = nullptr;
  const float* sgw = nullptr;
  float* wpos = nullptr;
};

// Prefill dispatch maps: the per-chunk histogram (HX_DISPATCH_TOK tokens a
// chunk) and the token bitmap (32 tokens a word).
#define HX_DISPATCH_TOK 256
__host__ __device__ inline int dispatch_words(int T) { return (T + 31) / 32; }
__host__ __device__ inline int dispatch_chunks(int T) { return (T + HX_DISPATCH_TOK - 1) / HX_DISPATCH_TOK; }

// Decode plan: everything the decode expert kernels need about the routing, in
// one contiguous int32 block they pull into LDS with a single coalesced load.
//   [0]                         number of slots S (routed experts + shared)
//   [4 + 4u + {0,1,2}]          slot u: expert (E = shared), start position, count
//   [4 + 4*max_slots + p]       token of permuted position p (p < F + T; shared: F + t)
//   [4 + 4*max_slots + F+T + p] routing weight of position p (f32 bits)
//   [4 + 4*max_slots + 2(F+T) + p] expert of position p (E for the shared rows)
// decode plan: [0] slots used; [4 + 4u ..] slot u's (expert, first row, row count);
// then per row of h (routed rows in dispatch order, then the shared expert's T
// rows): token, weight bits, expert (E for the shared expert)
__host__ __device__ inline int plan_ints(int max_slots, int F, int T) { return 4 + 4 * max_slots + 3 * (F + T); }

struct RouterArgs {
  const void* x;       // [T, H] act dtype
  int T, H;
  const void* R;       // [E1, H] router rows (+ shared-expert gate row)
  int E1, E, k;
  bool norm, has_shared;
  const float* bias;   // [E] or null
  float* logits;       // [T, E1]
  float* topk_w;       // [T*k]
  float* sgw;          // [T] sigmoid of the shared-expert gate
  DispatchArgs d;
  // decoder RMSNorm folded into the router (decode, bf16): x is the layer input,
  // the logits use x * rsqrt(mean(x^2) + eps) * (1 + norm_w) rounded to bf16,
  // and workgroup 0 writes that row to xn_out for the expert kernels
  const float* norm_w = nullptr;
  float eps = 0.f;
  uint16_t* xn_out = nullptr;
  // |r_e| rounded up, per router row (bf16 router rows): the MFMA prefill
  // routing bounds each logit with it
  const float* rnorm = nullptr;
  // MFMA prefill routing: logit planes (split K) the routing kernel adds;
  // plane 0 is `logits`, plane z >= 1 at mplanes + (z - 1) T (E + 1)
  int msplit = 1;
  float* mplanes = nullptr;
  // MFMA prefill routing: each routing wave also writes its token's xq (the
  // f16 d q of its Q8 codes for the m <= 64 expert calls, ExpertArgs::xq):
  // Q8_0 codes when xq_q80, else Q8_K; natural element order when xq_nat
  uint16_t* xq = nullptr;
  bool xq_q80 = false, xq_nat = false;
};
// most logit planes of the MFMA prefill router
#define HX_RM_SPLITS 4

// One projection stack: E matrices of [rows][K] in the internal layout.
struct WMat {
  int fmt = -1;        // HX_F32 / HX_BF16 / HX_Q8_0 (planar) / HX_Q4_K / HX_Q6_K (planar)
  int rows = 0, K = 0, count = 0;
  int64_t mat_bytes = 0;
  uint8_t* base = nullptr;
  __host__ __device__ const uint8_t* mat(int e) const { return base + (int64_t)e * mat_bytes; }
};

struct ExpertArgs {
  // routed stacks
  WMat gate, up, down;
  // shared expert (count 1) - fmt -1 if absent
  WMat sgate, sup, sdown;
  int E, k, H, I, Is, T, F;
  const void* x;
  bool xbf;
  const int32_t* perm;
  const float* topk_w;
  const float* sgw;
  const int32_t* slots;
  const int32_t* tiles;
  const int32_t* counts;
  float* hbuf;         // [(F+T), hstride] SwiGLU activations, f32
  int hstride;
  uint16_t* hbf;       // [(F+T), hstride] f16 copy (prefill: elements swizzled in groups of 4)
  uint16_t* xh;        // [T, H] f16 tokens in the swizzled order (prefill)
  uint16_t* xq;        // [T, H] prefill: f16 d q of the tokens' Q8 codes (the operand of the
                       // m <= 64 expert calls), in the order of xh
  float* xq32;         // [T, H] generic paths: f32 d q of the tokens' Q8 codes
  uint32_t* xcv;       // [T][H / 32][HX_XCV_WORDS] decode: each 32-wide chunk of a token quantised
                       // to the gate/up weights' vec_dot type, as a chunk record (hx_quant.h)
  uint32_t* hrec;      // [(F+T)][I / 32][HX_XCV_WORDS] decode: the rows of h as chunk records
                       // (the down weights' vec_dot type)
  void* obuf;          // [(F+T), H] weighted expert outputs (prefill): bf16 for bf16
                       // activations, f32 for f32 ones
  const int32_t* inv;
  const int32_t* topk_idx;
  void* y;             // [T, H] act dtype
  int max_slots, max_tiles;
  const int32_t* plan;
  // decoder residual folded into the decode down kernel: resid[t] becomes
  // bf16(resid[t] + bf16(y[t])) in place of writing y (bf16 activations)
  uint16_t* resid = nullptr;
  const float* wpos = nullptr;   // prefill: routing weight by permuted position (see DispatchArgs)
  // decode down partial sums [groups of HX_DOWN_ROWS rows of h][T][H] when the
  // rows of h take more than one group
  float* dpart = nullptr;
  // prefill MFMA kernels: which M tiles a launch covers -- HX_TILES_ALL: every
  // tile of the dispatch list; HX_TILES_ROUTED: the routed experts' tiles of
  // the list; HX_TILES_SHARED: the shared expert's tiles, computed from T (no
  // list: such a launch needs no routing)
  int tsel = 0;
  // prefill: the shared expert's rows of the down GEMM are stored unweighted
  // and the combine applies its sigmoid gate (the shared expert then runs
  // before the routing has computed that gate)
  bool shared_raw = false;
};
#define HX_TILES_ALL 0
#define HX_TILES_ROUTED 1
#define HX_TILES_SHARED 2

// prefill forwards of more tokens than this run the shared expert's GEMMs on
// the handle's side stream; smaller ones fold its tiles into the routed
// launches on the caller's stream. Measured on MI355X (A3B, Q4_K_M), one
// stream against the side stream, paired forwards: 512 tokens -5 to -9 us,
// 1024 -7.0, 1536 -4.2, 2048 -0.5, skewed 4096 -1.2, uniform 3072 +6.2 us.
#define HX_SIDE_STREAM_T 2048

// words of a chunk record (hx_quant.h); rows of h one decode down workgroup
// takes (4 waves x 6 rows each)
constexpr int HX_XCV_WORDS = 12;
constexpr int HX_DOWN_ROWS = 24;
__host__ __device__ inline int down_groups(int F, int T) { return (F + T + HX_DOWN_ROWS - 1) / HX_DOWN_ROWS; }

void launch_router(const RouterArgs& a, bool xbf, bool rbf, hipStream_t s);
void launch_route_small(const RouterArgs& a, hipStream_t s);   // T <= HX_DECODE_MAX_T, one workgroup
void launch_route_tokens(const RouterArgs& a, hipStream_t s);
// maps_ready: d.hist and d.bits are already filled (the MFMA routing does it)
hipError_t launch_dispatch(const DispatchArgs& d, hipStream_t s, bool maps_ready = false);
// prefill routing with the router GEMM on MFMA (bf16 tokens and router rows,
// renormalised top-k): approximate logits, then per token the exact top-k
bool route_mfma_ok(const RouterArgs& a, bool xbf, bool rbf, bool gfx950);
int route_mfma_splits(const RouterArgs& a);
// also writes the f16 tokens for the MFMA expert kernels when xh is not null,
// and clears the dispatch histogram and bitmap that launch_route_mfma fills
hipError_t launch_router_mfma(const RouterArgs& a, uint16_t* xh, bool xnat, hipStream_t s);
// the f16 tokens of the prefill MFMA kernels keep K in natural order for Q4_K
// gate/up weights (their dequantisation pairs adjacent elements) and in the
// order (0, 2, 1, 3) per group of 4 for the other formats
inline bool xh_natural(int gate_fmt) { return gate_fmt == HX_Q4_K; }
void launch_route_mfma(const RouterArgs& a, hipStream_t s);
hipError_t launch_row_norms(const void* R, int E1, int H, float* out, hipStream_t s);

// decode (T <= HX_DECODE_MAX_T)
bool decode_fast_ok(const ExpertArgs& a);   // bf16 activations, GGUF weights: f16 dot2 kernels
hipError_t launch_router_dec(const RouterArgs& r, const ExpertArgs& a, bool rbf, hipStream_t s);  // router + shared gate/up
hipError_t launch_gate_up_dec(const RouterArgs& r, const ExpertArgs& a, hipStream_t s);   // T == 1: routes in its prologue
hipError_t launch_gate_up_plan(const ExpertArgs& a, hipStream_t s);   // T > 1: reads the published plan
hipError_t launch_down_dec(const ExpertArgs& a, hipStream_t s);
hipError_t launch_gate_up_gemv(const ExpertArgs& a, hipStream_t s);
hipError_t launch_down_gemv_combine(const ExpertArgs& a, hipStream_t s);
// prefill
bool prefill_mfma_ok(const ExpertArgs& a);   // bf16 activations, GGUF experts: MFMA grouped GEMMs
hipError_t launch_x_to_f16(const ExpertArgs& a, hipStream_t s);       // tokens -> f16 for the MFMA kernels
hipError_t launch_gate_up_mfma(const ExpertArgs& a, hipStream_t s);
hipError_t launch_down_mfma(const ExpertArgs& a, hipStream_t s);
hipError_t launch_gate_up_prefill(const ExpertArgs& a, hipStream_t s);
hipError_t launch_down_prefill(const ExpertArgs& a, hipStream_t s);
hipError_t launch_combine(const ExpertArgs& a, hipStream_t s);

// activation quantisation (hx_actq.hip): the reference's Q8 codes of the rows
// of the m <= 64 expert calls
bool gguf_fmt(int fmt);
hipError_t launch_xq_fq(const ExpertArgs& a, hipStream_t s);               // tokens -> xq (prefill)
hipError_t launch_hq_fq(const ExpertArgs& a, int ntiles, hipStream_t s);   // h rows of m <= 64 tiles -> hbf
hipError_t launch_xq_f32(const ExpertArgs& a, hipStream_t s);              // tokens -> xq32 (generic)
hipError_t launch_hq_f32(const ExpertArgs& a, hipStream_t s);              // h rows of m <= 64 slots, in place
hipError_t launch_actq_codes(int wfmt, const void* x, bool xbf, int64_t rows, int cols, int8_t* codes, float* d,
                             hipStream_t s);

// weights
hipError_t launch_quantize(int fmt, const float* src, int64_t rows, int64_t cols, void* dst, hipStream_t s);
hipError_t launch_dequantize(int fmt, const void* src, int64_t rows, int64_t cols, float* dst, hipStream_t s);
// GGUF rows of `count` contiguous [rows][K] matrices -> internal layout, matrix m
// written at dst + m * dst_stride bytes
hipError_t launch_repack(int fmt, const void* src, int64_t count, int64_t rows, int64_t K, void* dst,
                         int64_t dst_stride, hipStream_t s);

hipError_t launch_rmsnorm(const void* x, bool xbf, int64_t T, int64_t H, const float* w, float eps, void* y,
                          hipStream_t s);
hipError_t launch_residual_add(void* x, const void* y, bool bf, int64_t n, hipStream_t s);

int64_t gguf_block_elems(int fmt);
int64_t gguf_block_bytes(int fmt);

// Per-kernel timing (hx_moe_timing_*): when start is set, the next launch
// through hx_launch has the runtime record the two events at that kernel's own
// dispatch start and end (hipExtLaunchKernel) -- the interval a kernel trace
// reports -- and clears them.
struct ExtTiming {
  hipEvent_t start = nullptr, stop = nullptr;
};
extern thread_local ExtTiming g_ext_timing;
template <typename K, typename... Args>
inline void hx_launch(K kernel, dim3 grid, dim3 block, uint32_t shm, hipStream_t s, Args... args) {
  ExtTiming& t = g_ext_timing;
  if (t.start) {
    const hipEvent_t a = t.start, b = t.stop;
    t.start = t.stop = nullptr;
    hipExtLaunchKernelGGL(kernel, grid, block, shm, s, a, b, 0u, args...);
  } else {
    hipLaunchKernelGGL(kernel, grid, block, shm, s, args...);
  }
}

}  // namespace hx
