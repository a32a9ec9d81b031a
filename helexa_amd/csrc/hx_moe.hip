// C ABI of libhxmoe (include/hx_moe.h): the block handle, weight upload and the
// forward orchestration.
//
// Reference: Qwen3_5MoeBlock::{load, forward} (crates/neuron/src/harness/arch/qwen3_5/moe.rs:55-199),
// TpQwen3_5MoeBlock::{load, forward_fused, forward}
// (crates/neuron/src/harness/tp/tp_qwen3_5.rs:1060-1275).
//
// Decode (T <= HX_DECODE_MAX_T, bf16 activations, GGUF experts; every expert
// call takes the reference's quantised arm): one token runs three kernels --
// router logits + the token's chunk records; routed + shared gate/up, each
// workgroup re-deriving the (small) routing from the logits; down + combine,
// which quantises the rows of h itself. Several tokens: router + records; one
// workgroup routes the tokens and publishes the plan; gate/up per slot of the
// plan (the shared expert's first); the records of the rows of h; down +
// combine. Prefill runs router (which also writes the f16 tokens), per-token
// routing (which also writes the Q8 operand of the quantised-arm tiles),
// dispatch, gate/up, the quantisation of h for the quantised-arm tiles, down
// (weighted rows) and combine.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "hx_moe.h"
#include "hx_internal.h"

using namespace hx;

static thread_local char g_err[512];

static int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

// ----------------------------------------------------------------------------
// scratch of hx_moe_forward_noalloc
// ----------------------------------------------------------------------------
// The workspace of the no-allocation forward: one copy per device, created with
// the code object and held until the process ends. On the host `scratch` names
// only a stand-in, not device memory: host code uses the address
// hipGetSymbolAddress returns for the current device, taken once per device by
// scratch_init (from hx_moe_create) and kept in g_scratch_ptr.
#define HX_SCRATCH_MAX_DEVICES 64
static __device__ __align__(256) uint8_t scratch[HX_NOALLOC_SCRATCH_BYTES];
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[HX_SCRATCH_MAX_DEVICES];

// device must be current
static int scratch_init(int device) {
  if (device < 0 || device >= HX_SCRATCH_MAX_DEVICES)
    return fail(HX_ERR_UNSUPPORTED, "device %d: at most %d devices", device, HX_SCRATCH_MAX_DEVICES);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[device]) return HX_OK;
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !p)
    return fail(HX_ERR_DEVICE, "hipGetSymbolAddress(scratch) on device %d failed: %s", device, hipGetErrorString(e));
  g_scratch_ptr[device] = p;
  return HX_OK;
}

static void* scratch_ptr(int device) {
  if (device < 0 || device >= HX_SCRATCH_MAX_DEVICES) return nullptr;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  return g_scratch_ptr[device];
}

#define HX_HIP(call)                                                                               \
  do {                                                                                             \
    hipError_t e_ = (call);                                                                        \
    if (e_ != hipSuccess) return fail(HX_ERR_DEVICE, "%s failed: %s (%s:%d)", #call, hipGetErrorString(e_), \
                                      __FILE__, __LINE__);                                         \
  } while (0)

extern "C" const char* hx_last_error(void) { return g_err; }

extern "C" int64_t hx_row_bytes(int dtype, int64_t n) {
  int64_t be = gguf_block_elems(dtype);
  if (be == 0 || n <= 0 || n % be) return -1;
  return n / be * gguf_block_bytes(dtype);
}

// ----------------------------------------------------------------------------
// timing slots
// ----------------------------------------------------------------------------
enum {
  SLOT_ROUTER = 0, SLOT_ROUTE_TOKENS, SLOT_DISPATCH, SLOT_GATE_UP, SLOT_DOWN, SLOT_COMBINE, SLOT_X_F16,
  SLOT_SH_GATE_UP, SLOT_SH_DOWN, N_SLOTS
};
static const char* kSlotNames[N_SLOTS] = {"router", "route_tokens", "dispatch", "gate_up", "down", "combine",
                                          "x_f16", "shared_gate_up", "shared_down"};

struct Timing {
  bool on = false;
  bool ext_armed = false;   // tm_ext handed this call's events to the next hx_launch
  int max_calls = 0, calls = 0;
  std::vector<hipEvent_t> ev;  // [max_calls][N_SLOTS][2]
  std::vector<int> used;       // [max_calls][N_SLOTS]
};

struct hx_moe {
  hx_moe_config cfg{};
  int device = 0;
  bool gfx950 = false;   // the device's architecture, checked at creation
  int E1 = 0;
  int rdt = HX_F32;   // dtype of the combined router rows
  void* router = nullptr;
  float* rnorm = nullptr;   // [E1] |router row| rounded up (bf16 router rows only)
  WMat gate, up, down, sgate, sup, sdown;
  void* own_ws = nullptr;
  size_t own_ws_bytes = 0;
  Timing tm;
  // prefill: the shared expert's GEMMs run on `side` (default priority) while
  // the caller's stream routes and dispatches; fork / join by the two events
  hipStream_t side = nullptr;
  hipEvent_t ev_fork = nullptr, ev_join = nullptr;
};

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// token counts above this are refused by every entry point: the kernels index
// the T * k assignments with 32-bit integers (k <= HX_MAX_TOPK)
#define HX_MAX_TOKENS ((int64_t)1 << 24)

struct WsLayout {
  size_t logits, topk_idx, topk_w, sgw, perm, inv, offsets, slots, tiles, counts, plan, dmap, hbuf, hbf, xh, xq, xq32, xcv,
      hrec, obuf, xn, ym, dpart, wpos, total;
  int hstride, max_slots, max_tiles;
};

// which expert kernels a forward of T tokens takes: the fast decode GEMVs,
// the prefill MFMA GEMMs, or the generic GEMVs (everything else)
static ExpertArgs shape_args(const hx_moe* m) {
  ExpertArgs a{};
  a.gate = m->gate; a.up = m->up; a.down = m->down;
  a.sgate = m->sgate; a.sup = m->sup; a.sdown = m->sdown;
  a.E = m->cfg.num_experts; a.k = m->cfg.num_experts_per_tok; a.H = m->cfg.hidden_size;
  a.I = m->cfg.moe_intermediate_size; a.Is = m->cfg.shared_expert_intermediate_size;
  a.xbf = m->cfg.act_dtype == HX_BF16;
  return a;
}
static bool generic_path(const hx_moe* m, int64_t T) {
  const ExpertArgs a = shape_args(m);
  return T <= HX_DECODE_MAX_T ? !decode_fast_ok(a) : !prefill_mfma_ok(a);
}

static WsLayout ws_layout(const hx_moe* m, int64_t T) {
  WsLayout L{};
  const int64_t E = m->cfg.num_experts, k = m->cfg.num_experts_per_tok, H = m->cfg.hidden_size;
  const int64_t F = T * k;
  const int64_t I = m->cfg.moe_intermediate_size, Is = m->cfg.shared_expert_intermediate_size;
  const bool decode = T <= HX_DECODE_MAX_T;
  L.hstride = (int)(((I > Is ? I : Is) + 7) / 8 * 8);
  L.max_slots = (int)((F < E ? F : E) + 1);
  L.max_tiles = (int)((F + HX_TILE_M - 1) / HX_TILE_M + (F < E ? F : E) + (T + HX_TILE_M - 1) / HX_TILE_M + 1);
  size_t o = 0;
  auto take = [&](size_t bytes) {
    size_t at = o;
    o += align256(bytes);
    return at;
  };
  L.logits = take(sizeof(float) * T * m->E1);
  L.topk_idx = take(sizeof(int32_t) * F);
  L.topk_w = take(sizeof(float) * F);
  L.sgw = take(sizeof(float) * T);
  L.perm = take(sizeof(int32_t) * F);
  L.inv = take(sizeof(int32_t) * F);
  L.offsets = take(sizeof(int32_t) * (E + 1));
  L.slots = take(sizeof(int32_t) * 3 * L.max_slots);
  L.tiles = take(sizeof(int32_t) * 4 * L.max_tiles);
  L.counts = take(sizeof(int32_t) * 4);
  L.plan = take(sizeof(int32_t) * plan_ints(L.max_slots, (int)F, (int)T));
  L.dmap = decode ? 0 : take(sizeof(int32_t) * (size_t)(dispatch_chunks((int)T) + dispatch_words((int)T)) * E);
  L.hbuf = take(sizeof(float) * (F + T) * L.hstride);
  L.hbf = take(sizeof(uint16_t) * (F + T) * L.hstride);
  const size_t act = m->cfg.act_dtype == HX_BF16 ? 2 : 4;
  L.obuf = decode ? 0 : take(act * (F + T) * H);
  L.xh = decode ? 0 : take(sizeof(uint16_t) * T * H);
  const bool generic = generic_path(m, T);
  // the MFMA path's xq lives in the routed rows of the weighted-rows buffer,
  // behind the router's logit planes: it is read by the gate/up kernels only,
  // before the down kernels write those rows (the shared expert's rows, which
  // the side stream may write meanwhile, start at row F)
  if (!decode && !generic) {
    const size_t at = align256(sizeof(float) * (HX_RM_SPLITS - 1) * T * m->E1), need = sizeof(uint16_t) * T * H;
    L.xq = at + need <= act * F * H ? L.obuf + at : take(need);
  }
  L.xq32 = generic && gguf_fmt(m->gate.fmt) ? take(sizeof(float) * T * H) : 0;
  L.xcv = decode ? take(sizeof(uint32_t) * (size_t)T * (H / 32) * HX_XCV_WORDS) : 0;
  L.hrec = decode ? take(sizeof(uint32_t) * (size_t)(F + T) * ((I > Is ? I : Is) / 32) * HX_XCV_WORDS) : 0;
  L.xn = take(act * T * H);
  L.ym = take(act * T * H);
  L.dpart = decode ? take(sizeof(float) * (size_t)down_groups((int)F, (int)T) * T * H) : 0;
  L.wpos = decode ? 0 : take(sizeof(float) * (F + T));
  L.total = o;
  return L;
}

// ----------------------------------------------------------------------------
// creation
// ----------------------------------------------------------------------------
static int chunk_elems(int fmt) {
  switch (fmt) {
    case HX_F32: case HX_BF16: return 8;
    case HX_Q8_0: case HX_Q4_K: case HX_Q6_K: return 32;
    default: return 0;
  }
}

static int check_proj(const char* name, int fmt, int64_t K) {
  if (fmt != HX_F32 && fmt != HX_BF16 && fmt != HX_Q8_0 && fmt != HX_Q4_K && fmt != HX_Q6_K)
    return fail(HX_ERR_UNSUPPORTED, "%s: unsupported storage dtype %d", name, fmt);
  if (hx_row_bytes(fmt, K) < 0)
    return fail(HX_ERR_INVALID_ARGUMENT, "%s: input dim %lld does not tile into dtype %d blocks", name,
                (long long)K, fmt);
  int ch = chunk_elems(fmt);
  if (K % ch || K / ch > 512)
    return fail(HX_ERR_UNSUPPORTED, "%s: input dim %lld must be a multiple of %d and at most %d", name,
                (long long)K, ch, 512 * ch);
  return HX_OK;
}

// upload one projection stack ([count][rows][K] GGUF rows) into the internal
// layout; every expert matrix starts on a 256-byte boundary
static int upload_proj(WMat& w, const char* name, int fmt, const void* src, int loc, int count, int rows, int K) {
  w.fmt = fmt;
  w.rows = rows;
  w.K = K;
  w.count = count;
  const int64_t packed = (int64_t)rows * hx_row_bytes(fmt, K);
  w.mat_bytes = (int64_t)align256((size_t)packed);
  const size_t bytes = (size_t)w.mat_bytes * count, src_bytes = (size_t)packed * count;
  if (!src) return fail(HX_ERR_INVALID_ARGUMENT, "%s: null weight pointer", name);
  if (hipMalloc(&w.base, bytes) != hipSuccess)
    return fail(HX_ERR_OUT_OF_MEMORY, "%s: cannot allocate %zu bytes", name, bytes);
  const void* dsrc = src;
  void* tmp = nullptr;
  if (loc == HX_HOST) {
    if (hipMalloc(&tmp, src_bytes) != hipSuccess)
      return fail(HX_ERR_OUT_OF_MEMORY, "%s: cannot allocate %zu staging bytes", name, src_bytes);
    hipError_t e = hipMemcpy(tmp, src, src_bytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
      (void)hipFree(tmp);
      return fail(HX_ERR_DEVICE, "%s: upload failed: %s", name, hipGetErrorString(e));
    }
    dsrc = tmp;
  }
  hipError_t e = launch_repack(fmt, dsrc, count, rows, K, w.base, w.mat_bytes, 0);
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (tmp) (void)hipFree(tmp);
  if (e != hipSuccess) return fail(HX_ERR_DEVICE, "%s: repack failed: %s", name, hipGetErrorString(e));
  return HX_OK;
}

static void free_mat(WMat& w) {
  if (w.base) (void)hipFree(w.base);
  w.base = nullptr;
}

extern "C" int hx_moe_destroy(hx_moe* m) {
  if (!m) return HX_OK;
  (void)hipSetDevice(m->device);
  (void)hipDeviceSynchronize();
  free_mat(m->gate); free_mat(m->up); free_mat(m->down);
  free_mat(m->sgate); free_mat(m->sup); free_mat(m->sdown);
  if (m->router) (void)hipFree(m->router);
  if (m->rnorm) (void)hipFree(m->rnorm);
  if (m->own_ws) (void)hipFree(m->own_ws);
  for (hipEvent_t e : m->tm.ev) (void)hipEventDestroy(e);
  if (m->ev_fork) (void)hipEventDestroy(m->ev_fork);
  if (m->ev_join) (void)hipEventDestroy(m->ev_join);
  if (m->side) (void)hipStreamDestroy(m->side);
  delete m;
  return HX_OK;
}

static int build_router(hx_moe* m, const hx_moe_weights* w) {
  const int E = m->cfg.num_experts, H = m->cfg.hidden_size;
  const bool sh = m->cfg.shared_expert_intermediate_size > 0;
  const int rd = w->router_dtype, sd = sh ? w->shared_expert_gate_dtype : rd;
  if ((rd != HX_F32 && rd != HX_BF16) || (sd != HX_F32 && sd != HX_BF16))
    return fail(HX_ERR_UNSUPPORTED, "router / shared_expert_gate must be F32 or BF16");
  if (!w->router || (sh && !w->shared_expert_gate))
    return fail(HX_ERR_INVALID_ARGUMENT, "null router or shared_expert_gate pointer");
  m->rdt = rd == sd ? rd : HX_F32;
  const size_t es = m->rdt == HX_BF16 ? 2 : 4;
  m->E1 = E + (sh ? 1 : 0);
  std::vector<uint8_t> host((size_t)m->E1 * H * es);
  auto fetch = [&](const void* src, int dt, int rows, uint8_t* dst) -> int {
    const size_t sbytes = (size_t)rows * H * (dt == HX_BF16 ? 2 : 4);
    std::vector<uint8_t> tmp(sbytes);
    if (w->location == HX_HOST) memcpy(tmp.data(), src, sbytes);
    else HX_HIP(hipMemcpy(tmp.data(), src, sbytes, hipMemcpyDeviceToHost));
    if (dt == m->rdt) {
      memcpy(dst, tmp.data(), sbytes);
    } else {  // bf16 -> f32, exact
      const uint16_t* s = (const uint16_t*)tmp.data();
      float* d = (float*)dst;
      for (size_t i = 0; i < (size_t)rows * H; i++) {
        uint32_t u = (uint32_t)s[i] << 16;
        memcpy(&d[i], &u, 4);
      }
    }
    return HX_OK;
  };
  int rc = fetch(w->router, rd, E, host.data());
  if (rc) return rc;
  if (sh && (rc = fetch(w->shared_expert_gate, sd, 1, host.data() + (size_t)E * H * es))) return rc;
  if (hipMalloc(&m->router, host.size()) != hipSuccess) return fail(HX_ERR_OUT_OF_MEMORY, "router allocation");
  HX_HIP(hipMemcpy(m->router, host.data(), host.size(), hipMemcpyHostToDevice));
  if (m->rdt == HX_BF16) {
    if (hipMalloc((void**)&m->rnorm, sizeof(float) * m->E1) != hipSuccess)
      return fail(HX_ERR_OUT_OF_MEMORY, "router norm allocation");
    HX_HIP(launch_row_norms(m->router, m->E1, H, m->rnorm, 0));
    HX_HIP(hipDeviceSynchronize());
  }
  return HX_OK;
}

extern "C" int hx_moe_create(const hx_moe_config* cfg, const hx_moe_weights* w, int device, hx_moe** out) {
  if (!cfg || !w || !out) return fail(HX_ERR_INVALID_ARGUMENT, "null argument");
  *out = nullptr;
  const hx_moe_config c = *cfg;
  // moe.rs:56-69
  if (c.num_experts <= 0 || c.num_experts_per_tok <= 0 || c.moe_intermediate_size <= 0)
    return fail(HX_ERR_INVALID_ARGUMENT,
                "MoE block needs num_experts (%d), num_experts_per_tok (%d) and moe_intermediate_size (%d) all > 0",
                c.num_experts, c.num_experts_per_tok, c.moe_intermediate_size);
  if (c.num_experts_per_tok > c.num_experts)
    return fail(HX_ERR_INVALID_ARGUMENT, "num_experts_per_tok (%d) exceeds num_experts (%d)",
                c.num_experts_per_tok, c.num_experts);
  if (c.hidden_size <= 0 || c.shared_expert_intermediate_size < 0)
    return fail(HX_ERR_INVALID_ARGUMENT, "bad hidden_size / shared_expert_intermediate_size");
  if (c.hidden_size % 8 != 0)   // the combine and router kernels move 8 elements per lane
    return fail(HX_ERR_UNSUPPORTED, "hidden_size (%d) must be a multiple of 8", c.hidden_size);
  if (c.num_experts > HX_MAX_EXPERTS || c.num_experts_per_tok > HX_MAX_TOPK)
    return fail(HX_ERR_UNSUPPORTED, "at most %d experts and top-%d are supported", HX_MAX_EXPERTS, HX_MAX_TOPK);
  if (c.act_dtype != HX_F32 && c.act_dtype != HX_BF16)
    return fail(HX_ERR_UNSUPPORTED, "act_dtype must be HX_F32 or HX_BF16");
  if (w->location != HX_HOST && w->location != HX_DEVICE)
    return fail(HX_ERR_INVALID_ARGUMENT, "weights.location must be HX_HOST or HX_DEVICE");
  const int H = c.hidden_size, I = c.moe_intermediate_size, Is = c.shared_expert_intermediate_size;
  const bool sh = Is > 0;
  int rc;
  if ((rc = check_proj("experts.gate_proj", w->gate_dtype, H)) || (rc = check_proj("experts.up_proj", w->up_dtype, H)) ||
      (rc = check_proj("experts.down_proj", w->down_dtype, I)))
    return rc;
  if (w->gate_dtype != w->up_dtype) return fail(HX_ERR_UNSUPPORTED, "gate_proj and up_proj must share a dtype");
  if (sh) {
    if ((rc = check_proj("shared_expert.gate_proj", w->shared_gate_dtype, H)) ||
        (rc = check_proj("shared_expert.up_proj", w->shared_up_dtype, H)) ||
        (rc = check_proj("shared_expert.down_proj", w->shared_down_dtype, Is)))
      return rc;
    if (w->shared_gate_dtype != w->gate_dtype || w->shared_up_dtype != w->up_dtype ||
        w->shared_down_dtype != w->down_dtype)
      return fail(HX_ERR_UNSUPPORTED, "the shared expert must use the routed experts' projection dtypes");
    if (chunk_elems(w->down_dtype) && (I > Is ? I : Is) / chunk_elems(w->down_dtype) > 512)
      return fail(HX_ERR_UNSUPPORTED, "intermediate size too large");
  }
  if (hipSetDevice(device) != hipSuccess) return fail(HX_ERR_DEVICE, "hipSetDevice(%d) failed", device);
  // the library holds gfx950 code objects only, and the MFMA routing's error
  // bound rests on gfx950's f16 MFMA accumulation
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess)
    return fail(HX_ERR_DEVICE, "hipGetDeviceProperties(%d) failed", device);
  const bool gfx950 = strncmp(prop.gcnArchName, "gfx950", 6) == 0 &&
                      (prop.gcnArchName[6] == '\0' || prop.gcnArchName[6] == ':');
  if (!gfx950) return fail(HX_ERR_UNSUPPORTED, "device %d is %s; libhxmoe is built for gfx950 only", device, prop.gcnArchName);
  if ((rc = scratch_init(device))) return rc;
  hx_moe* m = new hx_moe();
  m->gfx950 = gfx950;
  m->cfg = c;
  m->device = device;
  // the fork / join events order work of two streams on this one device: a
  // device-scope release / acquire is enough (no system-scope fence, which
  // writes back and invalidates the caches for the host at every record)
  const unsigned evf = hipEventDisableTiming | hipEventDisableSystemFence;
  if (hipStreamCreateWithFlags(&m->side, hipStreamNonBlocking) != hipSuccess ||
      hipEventCreateWithFlags(&m->ev_fork, evf) != hipSuccess ||
      hipEventCreateWithFlags(&m->ev_join, evf) != hipSuccess) {
    hx_moe_destroy(m);
    return fail(HX_ERR_DEVICE, "cannot create the handle's side stream / events");
  }
  const int E = c.num_experts;
  if ((rc = build_router(m, w)) || (rc = upload_proj(m->gate, "experts.gate_proj", w->gate_dtype, w->experts_gate, w->location, E, I, H)) ||
      (rc = upload_proj(m->up, "experts.up_proj", w->up_dtype, w->experts_up, w->location, E, I, H)) ||
      (rc = upload_proj(m->down, "experts.down_proj", w->down_dtype, w->experts_down, w->location, E, H, I))) {
    hx_moe_destroy(m);
    return rc;
  }
  if (sh && ((rc = upload_proj(m->sgate, "shared_expert.gate_proj", w->shared_gate_dtype, w->shared_gate, w->location, 1, Is, H)) ||
             (rc = upload_proj(m->sup, "shared_expert.up_proj", w->shared_up_dtype, w->shared_up, w->location, 1, Is, H)) ||
             (rc = upload_proj(m->sdown, "shared_expert.down_proj", w->shared_down_dtype, w->shared_down, w->location, 1, H, Is)))) {
    hx_moe_destroy(m);
    return rc;
  }
  *out = m;
  return HX_OK;
}

extern "C" int hx_moe_workspace_size(const hx_moe* m, int64_t n_tokens, size_t* bytes) {
  if (!m || !bytes || n_tokens < 0) return fail(HX_ERR_INVALID_ARGUMENT, "bad argument");
  *bytes = ws_layout(m, n_tokens).total;
  return HX_OK;
}

// ----------------------------------------------------------------------------
// forward
// ----------------------------------------------------------------------------
static int get_ws(hx_moe* m, int64_t T, void*& ws, size_t& ws_bytes, WsLayout& L) {
  L = ws_layout(m, T);
  if (ws) {
    if (ws_bytes < L.total)
      return fail(HX_ERR_WORKSPACE_TOO_SMALL, "workspace of %zu bytes, %zu needed for %lld tokens", ws_bytes,
                  L.total, (long long)T);
    return HX_OK;
  }
  if (m->own_ws_bytes < L.total) {
    if (m->own_ws) {
      HX_HIP(hipDeviceSynchronize());
      (void)hipFree(m->own_ws);
      m->own_ws = nullptr;
      m->own_ws_bytes = 0;
    }
    if (hipMalloc(&m->own_ws, L.total) != hipSuccess)
      return fail(HX_ERR_OUT_OF_MEMORY, "workspace allocation of %zu bytes", L.total);
    m->own_ws_bytes = L.total;
  }
  ws = m->own_ws;
  ws_bytes = m->own_ws_bytes;
  return HX_OK;
}

struct Plan {
  RouterArgs ra;
  ExpertArgs ea;
};

static void make_plan(hx_moe* m, const void* x, int64_t T, void* y, uint8_t* ws, const WsLayout& L,
                      const float* bias, Plan& p) {
  const hx_moe_config& c = m->cfg;
  const int k = c.num_experts_per_tok, E = c.num_experts;
  const int F = (int)(T * k);
  RouterArgs& r = p.ra;
  r = RouterArgs{};
  r.x = x;
  r.T = (int)T;
  r.H = c.hidden_size;
  r.R = m->router;
  r.E1 = m->E1;
  r.E = E;
  r.k = k;
  r.norm = c.norm_topk_prob != 0;
  r.has_shared = c.shared_expert_intermediate_size > 0;
  r.bias = bias;
  r.rnorm = m->rnorm;
  // logit planes 1.. of the MFMA router live at the start of the weighted-rows
  // buffer, which nothing writes before the down kernels (the shared expert's
  // rows, written beside the routing, start at row F, far past them)
  r.mplanes = L.obuf ? (float*)(ws + L.obuf) : nullptr;
  r.logits = (float*)(ws + L.logits);
  r.topk_w = (float*)(ws + L.topk_w);
  r.sgw = (float*)(ws + L.sgw);
  DispatchArgs& d = r.d;
  d.topk_idx = (int32_t*)(ws + L.topk_idx);
  d.T = (int)T;
  d.k = k;
  d.E = E;
  d.F = F;
  d.has_shared = r.has_shared;
  d.tile_m = HX_TILE_M;
  d.perm = (int32_t*)(ws + L.perm);
  d.inv = (int32_t*)(ws + L.inv);
  d.offsets = (int32_t*)(ws + L.offsets);
  d.slots = (int32_t*)(ws + L.slots);
  d.tiles = (int32_t*)(ws + L.tiles);
  d.counts = (int32_t*)(ws + L.counts);
  d.plan = (int32_t*)(ws + L.plan);
  d.max_slots = L.max_slots;
  d.hist = L.dmap ? (int32_t*)(ws + L.dmap) : nullptr;
  d.bits = L.dmap ? (uint32_t*)(ws + L.dmap) + (size_t)dispatch_chunks((int)T) * E : nullptr;
  d.topk_w = r.topk_w;
  d.sgw = r.sgw;
  d.wpos = L.wpos ? (float*)(ws + L.wpos) : nullptr;
  ExpertArgs& a = p.ea;
  a = ExpertArgs{};
  a.gate = m->gate; a.up = m->up; a.down = m->down;
  a.sgate = m->sgate; a.sup = m->sup; a.sdown = m->sdown;
  a.E = E; a.k = k; a.H = c.hidden_size; a.I = c.moe_intermediate_size; a.Is = c.shared_expert_intermediate_size;
  a.T = (int)T; a.F = F;
  a.x = x;
  a.xbf = c.act_dtype == HX_BF16;
  a.perm = d.perm;
  a.topk_w = r.topk_w;
  a.sgw = r.sgw;
  a.slots = d.slots;
  a.tiles = d.tiles;
  a.counts = d.counts;
  a.hbuf = (float*)(ws + L.hbuf);
  a.hstride = L.hstride;
  a.hbf = L.hbf ? (uint16_t*)(ws + L.hbf) : nullptr;
  a.obuf = L.obuf ? (void*)(ws + L.obuf) : nullptr;
  a.xh = L.xh ? (uint16_t*)(ws + L.xh) : nullptr;
  a.xq = L.xq ? (uint16_t*)(ws + L.xq) : nullptr;
  a.xq32 = L.xq32 ? (float*)(ws + L.xq32) : nullptr;
  a.xcv = L.xcv ? (uint32_t*)(ws + L.xcv) : nullptr;
  a.hrec = L.hrec ? (uint32_t*)(ws + L.hrec) : nullptr;
  a.inv = d.inv;
  a.topk_idx = d.topk_idx;
  a.y = y;
  a.max_slots = L.max_slots;
  a.max_tiles = L.max_tiles;
  a.plan = d.plan;
  a.dpart = L.dpart ? (float*)(ws + L.dpart) : nullptr;
  a.wpos = d.wpos;
}

namespace hx {
thread_local ExtTiming g_ext_timing;
}

// event helpers for the optional per-kernel timing
// forwards recorded under stream capture are not timed: no event is recorded
// into the graph, no slot is marked and the call is not counted
static bool capturing(hipStream_t s) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  (void)hipStreamIsCapturing(s, &st);
  return st != hipStreamCaptureStatusNone;
}

static void tm_mark(hx_moe* m, int slot, int which, hipStream_t s) {
  Timing& t = m->tm;
  if (!t.on || t.calls >= t.max_calls || capturing(s)) return;
  hipEvent_t ev = t.ev[((size_t)t.calls * N_SLOTS + slot) * 2 + which];
  (void)hipEventRecord(ev, s);
  if (which == 1) t.used[(size_t)t.calls * N_SLOTS + slot] = 1;
}

// timing of a slot launched as one kernel through hx_launch: the events are
// recorded by that kernel's dispatch itself (tm_ext before the launch,
// tm_ext_done after; a launcher that did not consume them leaves the slot
// untimed for this call)
static void tm_ext(hx_moe* m, int slot, hipStream_t s) {
  Timing& t = m->tm;
  t.ext_armed = false;
  if (!t.on || t.calls >= t.max_calls || capturing(s)) return;
  const size_t k = ((size_t)t.calls * N_SLOTS + slot) * 2;
  g_ext_timing.start = t.ev[k];
  g_ext_timing.stop = t.ev[k + 1];
  t.ext_armed = true;
}
static void tm_ext_done(hx_moe* m, int slot) {
  Timing& t = m->tm;
  if (!t.ext_armed) return;
  t.ext_armed = false;
  if (g_ext_timing.start) {   // no launch consumed the events
    g_ext_timing.start = g_ext_timing.stop = nullptr;
    return;
  }
  t.used[(size_t)t.calls * N_SLOTS + slot] = 1;
}

// the prefill routing on MFMA (approximate logits, exact top-k per token)
static bool route_mfma(const hx_moe* m, const Plan& p) {
  return route_mfma_ok(p.ra, m->cfg.act_dtype == HX_BF16, m->rdt == HX_BF16, m->gfx950);
}

// xh: where the MFMA router also writes the f16 tokens (or null)
static int run_router(hx_moe* m, Plan& p, hipStream_t s, uint16_t* xh = nullptr) {
  const bool xbf = m->cfg.act_dtype == HX_BF16, rbf = m->rdt == HX_BF16;
  tm_ext(m, SLOT_ROUTER, s);
  if (route_mfma(m, p)) HX_HIP(launch_router_mfma(p.ra, xh, xh_natural(p.ea.gate.fmt), s));
  else launch_router(p.ra, xbf, rbf, s);
  tm_ext_done(m, SLOT_ROUTER);
  HX_HIP(hipGetLastError());
  return HX_OK;
}

// per-token routing and dispatch from the router's logits
static int run_route_dispatch(hx_moe* m, Plan& p, hipStream_t s) {
  if (p.ra.T <= HX_DECODE_MAX_T) {
    tm_ext(m, SLOT_ROUTE_TOKENS, s);
    launch_route_small(p.ra, s);
    tm_ext_done(m, SLOT_ROUTE_TOKENS);
    HX_HIP(hipGetLastError());
  } else {
    tm_ext(m, SLOT_ROUTE_TOKENS, s);
    if (route_mfma(m, p)) launch_route_mfma(p.ra, s);
    else launch_route_tokens(p.ra, s);
    tm_ext_done(m, SLOT_ROUTE_TOKENS);
    HX_HIP(hipGetLastError());
    tm_mark(m, SLOT_DISPATCH, 0, s);
    HX_HIP(launch_dispatch(p.ra.d, s, route_mfma(m, p)));
    tm_mark(m, SLOT_DISPATCH, 1, s);
  }
  return HX_OK;
}

static int run_routing(hx_moe* m, Plan& p, hipStream_t s) {
  int rc = run_router(m, p, s);
  return rc ? rc : run_route_dispatch(m, p, s);
}

// the join of the side stream on every way out of a forward that forked it:
// the join event recorded on the side stream (if the forward had not got to
// it) and waited on by the caller's stream
struct SideJoin {
  hipStream_t s, side;
  hipEvent_t ev;
  bool armed = false, recorded = false;
  SideJoin(hipStream_t s_, hipStream_t side_, hipEvent_t ev_) : s(s_), side(side_), ev(ev_) {}
  ~SideJoin() {
    if (!armed) return;
    if (!recorded) (void)hipEventRecord(ev, side);
    (void)hipStreamWaitEvent(s, ev, 0);
  }
};

// the decoder's RMSNorm and residual around the block (hx_moe_decoder_mlp)
struct DecoderFuse {
  const float* norm_w;
  float eps;
  void* x;   // layer input; receives x + block(rmsnorm(x))
};

static int forward_impl(hx_moe* m, const void* x, int64_t T, void* y, void* ws, size_t ws_bytes,
                        const float* bias, hipStream_t s, const DecoderFuse* fz = nullptr) {
  WsLayout L;
  int rc = get_ws(m, T, ws, ws_bytes, L);
  if (rc) return rc;
  Plan p;
  make_plan(m, x, T, y, (uint8_t*)ws, L, bias, p);
  const bool decode = T <= HX_DECODE_MAX_T;
  const bool fast = decode && decode_fast_ok(p.ea);
  p.ra.d.plan_only = fast;   // the fast kernels read the plan only
  const bool bf = m->cfg.act_dtype == HX_BF16;
  const int H = m->cfg.hidden_size;
  uint16_t* xn = (uint16_t*)((uint8_t*)ws + L.xn);
  if (fz && fast && H <= 8 * 256) {
    // RMSNorm inside the router kernel (the router waves and the token-record
    // waves normalise each token with the same arithmetic, so both see the
    // same bits), residual inside the down kernel
    p.ra.norm_w = fz->norm_w;
    p.ra.eps = fz->eps;
    p.ra.xn_out = xn;
    p.ea.x = xn;
    p.ea.resid = (uint16_t*)fz->x;
  } else if (fz) {
    HX_HIP(launch_rmsnorm(fz->x, bf, T, H, fz->norm_w, fz->eps, xn, s));
    p.ra.x = p.ea.x = xn;
    if (fast) p.ea.resid = (uint16_t*)fz->x;   // the down kernel adds the residual
  }
  if (fast) {
    // router + shared gate/up; routed gate/up (one token: routing in its
    // prologue; more: routed once by one workgroup, then the plan); down + combine
    // one token: each slot is one kernel, timed by its own dispatch
    if (T == 1) tm_ext(m, SLOT_ROUTER, s);
    else tm_mark(m, SLOT_ROUTER, 0, s);
    HX_HIP(launch_router_dec(p.ra, p.ea, m->rdt == HX_BF16, s));
    if (T == 1) tm_ext_done(m, SLOT_ROUTER);
    else tm_mark(m, SLOT_ROUTER, 1, s);
    if (T == 1) {
      tm_ext(m, SLOT_GATE_UP, s);
      HX_HIP(launch_gate_up_dec(p.ra, p.ea, s));
      tm_ext_done(m, SLOT_GATE_UP);
    } else {
      tm_mark(m, SLOT_ROUTE_TOKENS, 0, s);
      launch_route_small(p.ra, s);
      HX_HIP(hipGetLastError());
      tm_mark(m, SLOT_ROUTE_TOKENS, 1, s);
      tm_mark(m, SLOT_GATE_UP, 0, s);
      HX_HIP(launch_gate_up_plan(p.ea, s));
      tm_mark(m, SLOT_GATE_UP, 1, s);
    }
    if (T == 1) tm_ext(m, SLOT_DOWN, s);
    else tm_mark(m, SLOT_DOWN, 0, s);
    HX_HIP(launch_down_dec(p.ea, s));
    if (T == 1) tm_ext_done(m, SLOT_DOWN);
    else tm_mark(m, SLOT_DOWN, 1, s);
  } else if (decode) {
    // generic GEMVs; for GGUF weights every expert call (m = T <= 8) takes the
    // quantised arm: the tokens and then the rows of h as f32 d q of their Q8
    // codes
    if ((rc = run_routing(m, p, s))) return rc;
    tm_mark(m, SLOT_GATE_UP, 0, s);
    if (p.ea.xq32) HX_HIP(launch_xq_f32(p.ea, s));
    HX_HIP(launch_gate_up_gemv(p.ea, s));
    tm_mark(m, SLOT_GATE_UP, 1, s);
    tm_mark(m, SLOT_DOWN, 0, s);
    if (gguf_fmt(p.ea.down.fmt)) HX_HIP(launch_hq_f32(p.ea, s));
    HX_HIP(launch_down_gemv_combine(p.ea, s));
    tm_mark(m, SLOT_DOWN, 1, s);
  } else {
    const bool mfma = prefill_mfma_ok(p.ea);
    // MFMA path: one kernel per slot, each timed by its own dispatch. With a
    // shared expert and more than HX_SIDE_STREAM_T tokens, its gate/up and
    // down need only the f16 tokens: after the router kernel (which keeps
    // every CU busy) they run on the side stream, next to the per-token
    // routing and the dispatch (small kernels that leave most CUs idle), their
    // down rows unweighted (the combine applies the sigmoid gate the routing
    // computes); the routed GEMMs follow the dispatch on the caller's stream
    // and the combine waits for both. Up to HX_SIDE_STREAM_T tokens the shared
    // tiles ride in the routed launches instead (the dispatch lists them after
    // the routed tiles, weighted by the sigmoid gate in the down epilogue):
    // there the fork and join cost more than the overlap gains.
    const bool split = mfma && m->cfg.shared_expert_intermediate_size > 0 && T > HX_SIDE_STREAM_T;
    // the MFMA router writes the f16 tokens itself
    const bool xh_in_router = mfma && route_mfma(m, p);
    if (mfma && !xh_in_router) {
      tm_ext(m, SLOT_X_F16, s);
      HX_HIP(launch_x_to_f16(p.ea, s));
      tm_ext_done(m, SLOT_X_F16);
    }
    if ((rc = run_router(m, p, s, xh_in_router ? p.ea.xh : nullptr))) return rc;
    // the m > 64 calls (the shared expert above 64 tokens, hot experts) read
    // xh; the m <= 64 ones the f16 d q of the tokens' Q8 codes
    const bool hq_shared = T <= HX_QUANT_M;   // the shared expert's call takes the quantised arm
    // once the side stream has forked, every return joins it back (so that a
    // failure under stream capture leaves no stream in capture state)
    SideJoin join(s, m->side, m->ev_join);
    if (split) {
      ExpertArgs sa = p.ea;
      sa.tsel = HX_TILES_SHARED;
      sa.shared_raw = true;
      HX_HIP(hipEventRecord(m->ev_fork, s));
      HX_HIP(hipStreamWaitEvent(m->side, m->ev_fork, 0));
      join.armed = true;
      tm_ext(m, SLOT_SH_GATE_UP, m->side);
      HX_HIP(launch_gate_up_mfma(sa, m->side));
      tm_ext_done(m, SLOT_SH_GATE_UP);
      if (hq_shared) HX_HIP(launch_hq_fq(sa, (int)((T + HX_TILE_M - 1) / HX_TILE_M), m->side));
      tm_ext(m, SLOT_SH_DOWN, m->side);
      HX_HIP(launch_down_mfma(sa, m->side));
      tm_ext_done(m, SLOT_SH_DOWN);
      HX_HIP(hipEventRecord(m->ev_join, m->side));
      join.recorded = true;
      p.ea.tsel = HX_TILES_ROUTED;
      p.ea.shared_raw = true;
    }
    // xq: written by the MFMA routing waves (which hold the token rows), else
    // by its own kernel
    if (mfma && xh_in_router) {
      p.ra.xq = p.ea.xq;
      p.ra.xq_q80 = p.ea.gate.fmt == HX_Q8_0;
      p.ra.xq_nat = xh_natural(p.ea.gate.fmt);
    } else if (mfma) {
      HX_HIP(launch_xq_fq(p.ea, s));
    }
    if ((rc = run_route_dispatch(m, p, s))) return rc;
    if (mfma) {
      tm_ext(m, SLOT_GATE_UP, s);
      HX_HIP(launch_gate_up_mfma(p.ea, s));
      tm_ext_done(m, SLOT_GATE_UP);
      HX_HIP(launch_hq_fq(p.ea, p.ea.max_tiles, s));
      tm_ext(m, SLOT_DOWN, s);
      HX_HIP(launch_down_mfma(p.ea, s));
      tm_ext_done(m, SLOT_DOWN);
      if (split) {
        join.armed = false;
        HX_HIP(hipStreamWaitEvent(s, m->ev_join, 0));
      }
    } else {
      // generic GEMVs: the m <= 64 slots read the f32 d q of the tokens' and
      // then of their rows of h's Q8 codes (GGUF weights)
      tm_mark(m, SLOT_GATE_UP, 0, s);
      if (p.ea.xq32) HX_HIP(launch_xq_f32(p.ea, s));
      HX_HIP(launch_gate_up_prefill(p.ea, s));
      tm_mark(m, SLOT_GATE_UP, 1, s);
      tm_mark(m, SLOT_DOWN, 0, s);
      if (gguf_fmt(p.ea.down.fmt)) HX_HIP(launch_hq_f32(p.ea, s));
      HX_HIP(launch_down_prefill(p.ea, s));
      tm_mark(m, SLOT_DOWN, 1, s);
    }
    tm_ext(m, SLOT_COMBINE, s);
    HX_HIP(launch_combine(p.ea, s));
    tm_ext_done(m, SLOT_COMBINE);
  }
  if (fz && !p.ea.resid) HX_HIP(launch_residual_add(fz->x, y, bf, T * H, s));
  if (m->tm.on && m->tm.calls < m->tm.max_calls && !capturing(s)) m->tm.calls++;
  return HX_OK;
}

extern "C" int hx_moe_forward(hx_moe* m, const void* x, int64_t n_tokens, void* y, void* workspace,
                              size_t workspace_bytes, const float* router_bias, void* stream) {
  if (!m || n_tokens < 0 || (n_tokens > 0 && (!x || !y))) return fail(HX_ERR_INVALID_ARGUMENT, "bad argument");
  if (n_tokens == 0) return HX_OK;
  if (n_tokens > HX_MAX_TOKENS) return fail(HX_ERR_UNSUPPORTED, "too many tokens in one call");
  HX_HIP(hipSetDevice(m->device));
  return forward_impl(m, x, n_tokens, y, workspace, workspace_bytes, router_bias, (hipStream_t)stream);
}

extern "C" int hx_moe_forward_noalloc(hx_moe* m, const void* x, int64_t n_tokens, void* y,
                                      const float* router_bias, void* stream) {
  if (!m || n_tokens < 0 || (n_tokens > 0 && (!x || !y))) return fail(HX_ERR_INVALID_ARGUMENT, "bad argument");
  if (n_tokens == 0) return HX_OK;
  if (n_tokens > HX_MAX_TOKENS) return fail(HX_ERR_UNSUPPORTED, "too many tokens in one call");
  const size_t need = ws_layout(m, n_tokens).total;
  if (need > HX_NOALLOC_SCRATCH_BYTES)
    return fail(HX_ERR_WORKSPACE_TOO_SMALL,
                "hx_moe_forward_noalloc: %lld tokens need %zu bytes of workspace, the scratch holds %zu",
                (long long)n_tokens, need, (size_t)HX_NOALLOC_SCRATCH_BYTES);
  void* ws = scratch_ptr(m->device);
  if (!ws) return fail(HX_ERR_DEVICE, "no scratch on device %d", m->device);
  HX_HIP(hipSetDevice(m->device));
  return forward_impl(m, x, n_tokens, y, ws, HX_NOALLOC_SCRATCH_BYTES, router_bias, (hipStream_t)stream);
}

extern "C" int hx_moe_forward_host(hx_moe* m, const void* x_host, int64_t n_tokens, void* y_host,
                                   const float* router_bias_host) {
  if (!m || n_tokens < 0 || (n_tokens > 0 && (!x_host || !y_host)))
    return fail(HX_ERR_INVALID_ARGUMENT, "bad argument");
  if (n_tokens == 0) return HX_OK;
  if (n_tokens > HX_MAX_TOKENS) return fail(HX_ERR_UNSUPPORTED, "too many tokens in one call");
  HX_HIP(hipSetDevice(m->device));
  const size_t bytes = (size_t)n_tokens * m->cfg.hidden_size * (m->cfg.act_dtype == HX_BF16 ? 2 : 4);
  void *dx = nullptr, *dy = nullptr;
  float* db = nullptr;
  int rc = HX_OK;
  if (hipMalloc(&dx, bytes) != hipSuccess || hipMalloc(&dy, bytes) != hipSuccess ||
      (router_bias_host && hipMalloc((void**)&db, sizeof(float) * m->cfg.num_experts) != hipSuccess)) {
    rc = fail(HX_ERR_OUT_OF_MEMORY, "staging allocation");
  } else if (hipMemcpy(dx, x_host, bytes, hipMemcpyHostToDevice) != hipSuccess ||
             (db && hipMemcpy(db, router_bias_host, sizeof(float) * m->cfg.num_experts, hipMemcpyHostToDevice) !=
                        hipSuccess)) {
    rc = fail(HX_ERR_DEVICE, "copy to device failed");
  } else if ((rc = forward_impl(m, dx, n_tokens, dy, nullptr, 0, db, 0)) == HX_OK) {
    if (hipMemcpy(y_host, dy, bytes, hipMemcpyDeviceToHost) != hipSuccess) rc = fail(HX_ERR_DEVICE, "copy to host failed");
  }
  if (dx) (void)hipFree(dx);
  if (dy) (void)hipFree(dy);
  if (db) (void)hipFree(db);
  return rc;
}

extern "C" int hx_moe_route(hx_moe* m, const void* x, int64_t n_tokens, const float* router_bias, int32_t* topk_idx,
                            float* topk_w, int32_t* perm, int32_t* offsets, int32_t* inv, void* workspace,
                            size_t workspace_bytes, void* stream) {
  if (!m || n_tokens < 0 || (n_tokens > 0 && !x)) return fail(HX_ERR_INVALID_ARGUMENT, "bad argument");
  if (n_tokens == 0) return HX_OK;
  if (n_tokens > HX_MAX_TOKENS) return fail(HX_ERR_UNSUPPORTED, "too many tokens in one call");
  HX_HIP(hipSetDevice(m->device));
  hipStream_t s = (hipStream_t)stream;
  WsLayout L;
  int rc = get_ws(m, n_tokens, workspace, workspace_bytes, L);
  if (rc) return rc;
  Plan p;
  make_plan(m, x, n_tokens, nullptr, (uint8_t*)workspace, L, router_bias, p);
  if ((rc = run_routing(m, p, s))) return rc;
  const int64_t F = n_tokens * m->cfg.num_experts_per_tok;
  if (topk_idx) HX_HIP(hipMemcpyAsync(topk_idx, p.ra.d.topk_idx, 4 * F, hipMemcpyDeviceToDevice, s));
  if (topk_w) HX_HIP(hipMemcpyAsync(topk_w, p.ra.topk_w, 4 * F, hipMemcpyDeviceToDevice, s));
  if (perm) HX_HIP(hipMemcpyAsync(perm, p.ra.d.perm, 4 * F, hipMemcpyDeviceToDevice, s));
  if (inv) HX_HIP(hipMemcpyAsync(inv, p.ra.d.inv, 4 * F, hipMemcpyDeviceToDevice, s));
  if (offsets)
    HX_HIP(hipMemcpyAsync(offsets, p.ra.d.offsets, 4 * (m->cfg.num_experts + 1), hipMemcpyDeviceToDevice, s));
  return HX_OK;
}

extern "C" int hx_moe_router_logits(hx_moe* m, const void* x, int64_t n_tokens, const float* router_bias,
                                    float* logits, void* stream) {
  if (!m || n_tokens < 0 || (n_tokens > 0 && (!x || !logits))) return fail(HX_ERR_INVALID_ARGUMENT, "bad argument");
  if (n_tokens == 0) return HX_OK;
  if (n_tokens > HX_MAX_TOKENS) return fail(HX_ERR_UNSUPPORTED, "too many tokens in one call");
  HX_HIP(hipSetDevice(m->device));
  hipStream_t s = (hipStream_t)stream;
  void* ws = nullptr;
  size_t wsb = 0;
  WsLayout L;
  int rc = get_ws(m, n_tokens, ws, wsb, L);
  if (rc) return rc;
  Plan p;
  make_plan(m, x, n_tokens, nullptr, (uint8_t*)ws, L, router_bias, p);
  launch_router(p.ra, m->cfg.act_dtype == HX_BF16, m->rdt == HX_BF16, s);
  HX_HIP(hipGetLastError());
  const int E = m->cfg.num_experts, E1 = m->E1;
  HX_HIP(hipMemcpy2DAsync(logits, sizeof(float) * E, p.ra.logits, sizeof(float) * E1, sizeof(float) * E, n_tokens,
                          hipMemcpyDeviceToDevice, s));
  return HX_OK;
}

extern "C" int hx_moe_decoder_mlp(hx_moe* m, void* x, int64_t n_tokens, const float* norm_w, float eps,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  if (!m || n_tokens < 0 || (n_tokens > 0 && (!x || !norm_w))) return fail(HX_ERR_INVALID_ARGUMENT, "bad argument");
  if (n_tokens == 0) return HX_OK;
  if (n_tokens > HX_MAX_TOKENS) return fail(HX_ERR_UNSUPPORTED, "too many tokens in one call");
  HX_HIP(hipSetDevice(m->device));
  hipStream_t s = (hipStream_t)stream;
  WsLayout L;
  int rc = get_ws(m, n_tokens, workspace, workspace_bytes, L);
  if (rc) return rc;
  uint8_t* ws = (uint8_t*)workspace;
  const DecoderFuse fz{norm_w, eps, x};
  return forward_impl(m, x, n_tokens, ws + L.ym, workspace, workspace_bytes, nullptr, s, &fz);
}

extern "C" int hx_quantize(int dtype, const float* src, int64_t rows, int64_t cols, void* dst, void* stream) {
  if (!src || !dst || rows < 0) return fail(HX_ERR_INVALID_ARGUMENT, "bad argument");
  if (dtype != HX_Q8_0 && dtype != HX_Q4_K && dtype != HX_Q6_K && dtype != HX_BF16 && dtype != HX_F16)
    return fail(HX_ERR_UNSUPPORTED, "hx_quantize: dtype %d", dtype);
  if (hx_row_bytes(dtype, cols) < 0)
    return fail(HX_ERR_INVALID_ARGUMENT, "hx_quantize: %lld columns do not tile into dtype %d blocks", (long long)cols, dtype);
  if (rows == 0) return HX_OK;
  HX_HIP(launch_quantize(dtype, src, rows, cols, dst, (hipStream_t)stream));
  return HX_OK;
}

extern "C" int hx_dequantize(int dtype, const void* src, int64_t rows, int64_t cols, float* dst, void* stream) {
  if (!src || !dst || rows < 0) return fail(HX_ERR_INVALID_ARGUMENT, "bad argument");
  if (hx_row_bytes(dtype, cols) < 0)
    return fail(HX_ERR_INVALID_ARGUMENT, "hx_dequantize: %lld columns do not tile into dtype %d blocks", (long long)cols, dtype);
  if (rows == 0) return HX_OK;
  HX_HIP(launch_dequantize(dtype, src, rows, cols, dst, (hipStream_t)stream));
  return HX_OK;
}

extern "C" int hx_quantize_activations(int weight_dtype, const void* x, int x_dtype, int64_t rows, int64_t cols,
                                       int8_t* codes, float* d, void* stream) {
  if (!x || !codes || !d || rows < 0 || cols <= 0 || cols > (1 << 20)) return fail(HX_ERR_INVALID_ARGUMENT, "bad argument");
  if (!gguf_fmt(weight_dtype)) return fail(HX_ERR_UNSUPPORTED, "hx_quantize_activations: weight dtype %d has no vec_dot type", weight_dtype);
  if (x_dtype != HX_F32 && x_dtype != HX_BF16) return fail(HX_ERR_UNSUPPORTED, "hx_quantize_activations: x dtype %d", x_dtype);
  const int64_t blk = weight_dtype == HX_Q8_0 ? 32 : 256;
  if (cols % blk)
    return fail(HX_ERR_INVALID_ARGUMENT, "hx_quantize_activations: %lld columns are not whole blocks of %lld",
                (long long)cols, (long long)blk);
  if (rows == 0) return HX_OK;
  HX_HIP(launch_actq_codes(weight_dtype, x, x_dtype == HX_BF16, rows, (int)cols, codes, d, (hipStream_t)stream));
  return HX_OK;
}

// ----------------------------------------------------------------------------
// timing
// ----------------------------------------------------------------------------
extern "C" int hx_moe_timing_begin(hx_moe* m, int max_calls) {
  if (!m || max_calls <= 0) return fail(HX_ERR_INVALID_ARGUMENT, "bad argument");
  HX_HIP(hipSetDevice(m->device));
  Timing& t = m->tm;
  const size_t need = (size_t)max_calls * N_SLOTS * 2;
  while (t.ev.size() < need) {
    hipEvent_t e;
    HX_HIP(hipEventCreate(&e));
    t.ev.push_back(e);
  }
  t.used.assign((size_t)max_calls * N_SLOTS, 0);
  t.max_calls = max_calls;
  t.calls = 0;
  t.on = true;
  return HX_OK;
}

extern "C" int hx_moe_timing_read(hx_moe* m, double* ms, int64_t* launches, int* n_slots) {
  if (!m || !ms || !launches || !n_slots) return fail(HX_ERR_INVALID_ARGUMENT, "bad argument");
  Timing& t = m->tm;
  const int cap = *n_slots;
  *n_slots = N_SLOTS;
  if (cap < N_SLOTS) return fail(HX_ERR_INVALID_ARGUMENT, "need room for %d slots", N_SLOTS);
  HX_HIP(hipSetDevice(m->device));
  for (int i = 0; i < N_SLOTS; i++) {
    ms[i] = 0.0;
    launches[i] = 0;
  }
  for (int c = 0; c < t.calls; c++)
    for (int i = 0; i < N_SLOTS; i++) {
      if (!t.used[(size_t)c * N_SLOTS + i]) continue;
      hipEvent_t a = t.ev[((size_t)c * N_SLOTS + i) * 2], b = t.ev[((size_t)c * N_SLOTS + i) * 2 + 1];
      HX_HIP(hipEventSynchronize(b));
      float v = 0.f;
      HX_HIP(hipEventElapsedTime(&v, a, b));
      ms[i] += v;
      launches[i]++;
    }
  return HX_OK;
}

extern "C" int hx_moe_timing_end(hx_moe* m, double* ms, int64_t* launches, int* n_slots) {
  int rc = hx_moe_timing_read(m, ms, launches, n_slots);
  if (m) {
    m->tm.on = false;
    m->tm.calls = 0;
  }
  return rc;
}

extern "C" const char* hx_moe_timing_name(int slot) {
  return slot >= 0 && slot < N_SLOTS ? kSlotNames[slot] : "";
}
