/*
 * hx_moe.h -- C ABI of libhxmoe.so, an MI355X (gfx950) implementation of
 * helexa neuron's Qwen3-Next sparse-MoE block.
 *
 * Reference interfaces replaced (paths relative to the helexa repository):
 *   Qwen3_5MoeBlock::load                   crates/neuron/src/harness/arch/qwen3_5/moe.rs:55
 *   TpQwen3_5MoeBlock::load                 crates/neuron/src/harness/tp/tp_qwen3_5.rs:1060-1103
 *   impl Module for Qwen3_5MoeBlock         moe.rs:164-199
 *   impl Module for TpQwen3_5MoeBlock       tp_qwen3_5.rs:1240-1275
 *   route_scatter                           moe.rs:115-162
 *   forward_fused routing + sort            tp_qwen3_5.rs:1179-1189
 *   quantize_parallel                       crates/neuron/src/harness/tp/isq.rs:39-55
 *   Qwen3_5RmsNorm::forward                 crates/neuron/src/harness/arch/qwen3_5/rmsnorm.rs:67-80
 *   Qwen3_5DecoderLayer::forward (MLP half) crates/neuron/src/harness/arch/qwen3_5/decoder.rs:129-132
 *
 * Conventions
 *   - Every function returns an int status (HX_OK on success). Nothing aborts
 *     or throws across the ABI; hx_last_error() describes the last failure on
 *     the calling thread.
 *   - A handle is bound to the device given at creation. Calls on one handle
 *     must be serialised (the reference drives a block from one owner thread,
 *     device_worker/mod.rs:103-111).
 *   - "stream" arguments are hipStream_t values passed as void*; NULL is the
 *     legacy default stream.
 *   - Tensors are row-major. Activations are HX_F32 or HX_BF16 (raw bf16 bits).
 *   - Quantised weights are GGUF rows ([out, in], blocked along in), exactly the
 *     bytes candle's QTensor holds (isq.rs:104-112).
 */
#ifndef HX_MOE_H
#define HX_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define HX_OK 0
#define HX_ERR_INVALID_ARGUMENT 1
#define HX_ERR_UNSUPPORTED 2
#define HX_ERR_DEVICE 3
#define HX_ERR_WORKSPACE_TOO_SMALL 4
#define HX_ERR_OUT_OF_MEMORY 5

/* storage formats: the GGML type ids */
#define HX_F32 0
#define HX_F16 1
#define HX_Q8_0 8
#define HX_Q4_K 12
#define HX_Q6_K 14
#define HX_BF16 30

/* where the pointers in hx_moe_weights live */
#define HX_HOST 0
#define HX_DEVICE 1

/* MoE fields of TextConfig (crates/neuron/src/harness/arch/qwen3_5/mod.rs:270-302) */
typedef struct hx_moe_config {
    int32_t hidden_size;                      /* H */
    int32_t num_experts;                      /* E */
    int32_t num_experts_per_tok;              /* k, 1 <= k <= E */
    int32_t moe_intermediate_size;            /* I */
    int32_t shared_expert_intermediate_size;  /* Is, 0 = no shared expert */
    int32_t norm_topk_prob;                   /* renormalise the top-k weights */
    int32_t act_dtype;                        /* HX_F32 or HX_BF16 */
} hx_moe_config;

/* Checkpoint tensors of one block (moe.rs:73-102, mlp.rs:43-45). The library
 * copies them into its own device memory (and may repack the quantised ones);
 * the caller may free them after hx_moe_create returns. */
typedef struct hx_moe_weights {
    int32_t location;                                  /* HX_HOST or HX_DEVICE */
    int32_t router_dtype;   const void* router;        /* mlp.gate.weight [E, H], F32 or BF16 */
    int32_t gate_dtype;     const void* experts_gate;  /* experts.{e}.gate_proj [E, I, H] */
    int32_t up_dtype;       const void* experts_up;    /* experts.{e}.up_proj   [E, I, H] */
    int32_t down_dtype;     const void* experts_down;  /* experts.{e}.down_proj [E, H, I] */
    int32_t shared_gate_dtype; const void* shared_gate;  /* shared_expert.gate_proj [Is, H] */
    int32_t shared_up_dtype;   const void* shared_up;    /* shared_expert.up_proj   [Is, H] */
    int32_t shared_down_dtype; const void* shared_down;  /* shared_expert.down_proj [H, Is] */
    int32_t shared_expert_gate_dtype; const void* shared_expert_gate; /* [1, H], F32 or BF16 */
} hx_moe_weights;

typedef struct hx_moe hx_moe;

/* Qwen3_5MoeBlock::load (moe.rs:55-112): validates E, k, I > 0, k <= E
 * (moe.rs:56-69) and the GGUF block divisibility of every quantised projection
 * (isq.rs:62-68), uploads the weights to `device`. */
int hx_moe_create(const hx_moe_config* cfg, const hx_moe_weights* w, int device, hx_moe** out);

/* Drop: frees the handle's device memory. NULL is accepted. */
int hx_moe_destroy(hx_moe* m);

/* Bytes of device workspace hx_moe_forward / hx_moe_route need for n_tokens. */
int hx_moe_workspace_size(const hx_moe* m, int64_t n_tokens, size_t* bytes);

/* Module::forward (moe.rs:164-199 / tp_qwen3_5.rs:1240-1275), device resident:
 * x and y are device pointers to [n_tokens, H] in act_dtype (the reference's
 * (b, l, H) input flattened, moe.rs:166-167). workspace may be NULL, in which
 * case the handle grows its own. router_bias is an optional device [E] f32 added
 * to the router logits before the softmax (a benchmark hook with no reference
 * counterpart; NULL in production). n_tokens == 0 is a no-op. */
int hx_moe_forward(hx_moe* m, const void* x, int64_t n_tokens, void* y,
                   void* workspace, size_t workspace_bytes, const float* router_bias, void* stream);

/* No counterpart in the reference: hx_moe_forward for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). Same arguments and results as
 * hx_moe_forward with a NULL workspace, but the workspace is a fixed scratch
 * array of HX_NOALLOC_SCRATCH_BYTES in the library's own device memory (one
 * copy per GPU, set up by hx_moe_create and held until the process ends), so
 * the call performs no allocation of any kind. n_tokens whose workspace
 * (hx_moe_workspace_size) exceeds HX_NOALLOC_SCRATCH_BYTES are rejected with
 * HX_ERR_WORKSPACE_TOO_SMALL; at the 80B-A3B shape the limit holds every
 * decode batch and prefill chunks of up to 700 tokens. Every call on one GPU
 * shares that GPU's scratch: calls that overlap on one GPU (other streams,
 * other threads, other handles) race and must be serialised by the caller. */
#define HX_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int hx_moe_forward_noalloc(hx_moe* m, const void* x, int64_t n_tokens, void* y, const float* router_bias,
                           void* stream);

/* Same, for host buffers (what a candle CPU-tensor wrapper calls): copies x in,
 * runs hx_moe_forward on the default stream, copies y out, synchronises. */
int hx_moe_forward_host(hx_moe* m, const void* x_host, int64_t n_tokens, void* y_host,
                        const float* router_bias_host);

/* route_scatter (moe.rs:124-162) plus the dispatch sort of forward_fused
 * (tp_qwen3_5.rs:1189), device resident. Outputs (device pointers, any may be
 * NULL):
 *   topk_idx [T, k] int32  -- descending probability, ties to the lower id
 *   topk_w   [T, k] f32    -- softmax probabilities, renormalised if configured
 *   perm     [T*k]  int32  -- flat index t*k+j stably sorted by expert id
 *   offsets  [E+1]  int32  -- exclusive scan of the per-expert counts
 *   inv      [T*k]  int32  -- inverse of perm */
int hx_moe_route(hx_moe* m, const void* x, int64_t n_tokens, const float* router_bias,
                 int32_t* topk_idx, float* topk_w, int32_t* perm, int32_t* offsets, int32_t* inv,
                 void* workspace, size_t workspace_bytes, void* stream);

/* Router logits [T, E] f32 exactly as the routing kernel computes them (rounded
 * to act_dtype, plus router_bias). For bit-exact checks. */
int hx_moe_router_logits(hx_moe* m, const void* x, int64_t n_tokens, const float* router_bias,
                         float* logits, void* stream);

/* Decoder-layer MLP half on a residual stream (decoder.rs:129-132 with the
 * attention half skipped): x <- x + moe(rmsnorm(x)), where rmsnorm is
 * Qwen3_5RmsNorm, x * rsqrt(mean(x^2) + eps) * (1 + norm_w) in f32
 * (rmsnorm.rs:67-80). x is device [T, H] act_dtype, norm_w device [H] f32. */
int hx_moe_decoder_mlp(hx_moe* m, void* x, int64_t n_tokens, const float* norm_w, float eps,
                       void* workspace, size_t workspace_bytes, void* stream);

/* quantize_parallel (isq.rs:39-113) on the device: f32 [rows, cols] -> GGUF
 * rows of dtype (HX_Q8_0, HX_Q4_K, HX_Q6_K, HX_BF16, HX_F16). cols must tile
 * into whole blocks. Each block follows the rule of candle's
 * GgmlType::from_float, which quantize_parallel calls (isq.rs:98): Q8_0
 * d = amax/127 with rounding half away from zero; Q4_K make_qkx1_quants
 * (5 tries) per 32 elements; Q6_K make_qx_quants (rmse_type 1) per 16. */
int hx_quantize(int dtype, const float* src, int64_t rows, int64_t cols, void* dst, void* stream);

/* GGUF rows of dtype -> f32 [rows, cols] on the device. */
int hx_dequantize(int dtype, const void* src, int64_t rows, int64_t cols, float* dst, void* stream);

/* Bytes of one GGUF row of n elements, or -1 if n does not tile into blocks. */
int64_t hx_row_bytes(int dtype, int64_t n);

/* The activation quantisation of MaybeQuantLinear's quantised arm
 * (crates/neuron/src/harness/tp/tp_linear.rs:120-137: an expert call of at
 * most 64 rows quantises each activation row to the weight type's vec_dot
 * type before candle's integer vec_dot), as the forward kernels compute it,
 * on the device: x [rows, cols] (x_dtype HX_F32 or HX_BF16) -> codes int8
 * [rows, cols] and d f32 [rows, cols / block]. weight_dtype HX_Q8_0 gives Q8_0
 * blocks of 32 (d = amax / 127, rounded to f16; codes round(x / d) half away
 * from zero); HX_Q4_K or HX_Q6_K gives Q8_K blocks of 256 (iscale = -128 /
 * the first largest-magnitude value, codes min(round(iscale x), 127),
 * d = 1 / iscale). cols must be a multiple of the block. */
int hx_quantize_activations(int weight_dtype, const void* x, int x_dtype, int64_t rows, int64_t cols, int8_t* codes,
                            float* d, void* stream);

/* Per-kernel timing (a measurement hook with no reference counterpart): HIP
 * events recorded on the forward's stream around each kernel it launches.
 * hx_moe_timing_begin arms it for the next max_calls forwards (forwards under
 * stream capture are not timed).
 * hx_moe_timing_read synchronises on the recorded events and returns, per
 * kernel slot, the summed milliseconds and the number of timed launches
 * (*n_slots: capacity in, slots used out); hx_moe_timing_end does the same and
 * disarms. hx_moe_timing_name names a slot. */
int hx_moe_timing_begin(hx_moe* m, int max_calls);
int hx_moe_timing_read(hx_moe* m, double* ms, int64_t* launches, int* n_slots);
int hx_moe_timing_end(hx_moe* m, double* ms, int64_t* launches, int* n_slots);
const char* hx_moe_timing_name(int slot);

/* Description of the last error on the calling thread ("" if none). */
const char* hx_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* HX_MOE_H */
