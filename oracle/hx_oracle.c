/*
 * hx_oracle.c -- TEST INFRASTRUCTURE ONLY.
 *
 * CPU restatement of helexa neuron's Qwen3-Next sparse-MoE block, used as the
 * checker for the HIP library (libhxmoe.so). Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load this library; the product path never
 * does.
 *
 * What it restates (reference paths are relative to the helexa repository):
 *   - route_scatter            crates/neuron/src/harness/arch/qwen3_5/moe.rs:124-162
 *       router Linear (moe.rs:134), f32 softmax (moe.rs:135), descending argsort
 *       top-k (moe.rs:140-142), renormalisation (moe.rs:143-146), per-expert
 *       ascending token lists (moe.rs:152-160)
 *   - dispatch permutation     crates/neuron/src/harness/tp/tp_qwen3_5.rs:1189
 *       (topk_ids.flatten_all().sort_last_dim(true), ties by flat index)
 *   - Module::forward          moe.rs:164-199 (experts ascending, then shared)
 *   - Qwen3_5MLP::forward      crates/neuron/src/harness/arch/qwen3_5/mlp.rs:54-60
 *   - MaybeQuantLinear         crates/neuron/src/harness/tp/tp_linear.rs:98-140
 *       (quantised weights: GGUF Q8_0 / Q4_K / Q6_K blocks, public ggml format)
 *   - quantize_blocks          crates/neuron/src/harness/tp/isq.rs:57-113
 *       (block layout and divisibility) with the block rules of candle's
 *       GgmlType::from_float, which isq.rs:98 calls (Q8_0, Q4_K, Q6_K; see the
 *       quantiser section)
 *   - Qwen3_5RmsNorm::forward  crates/neuron/src/harness/arch/qwen3_5/rmsnorm.rs:67-80
 *   - decoder residual         crates/neuron/src/harness/arch/qwen3_5/decoder.rs:129-132
 *
 * Numeric contract shared (by restatement, not by code) with the HIP library:
 *   - router logit = lane-strided dot product: the H inputs are cut into groups
 *     of 8 (the last one may be shorter); group g belongs to lane g % 64; each lane runs an fmaf chain over its
 *     groups in increasing order; the 64 lane partials are then combined by an
 *     xor butterfly (offsets 32,16,8,4,2,1). The result is rounded to the
 *     activation dtype (candle's Linear returns the input dtype, moe.rs:134).
 *   - softmax uses hxo_expf below (Cody-Waite reduction + degree-7 Taylor,
 *     evaluated with fmaf), a lane-strided sum with the same butterfly, and an
 *     IEEE division.
 *   - top-k: k largest probabilities, ties to the lower expert id.
 *   - renormalisation: sequential sum in rank order, IEEE division.
 * Everything here is compiled with -ffp-contract=off so that no multiply-add is
 * fused unless fmaf is written explicitly.
 *
 * How each part is pinned (tests/test_oracle.py):
 *   - f16 / bf16 conversions: exhaustive / numpy / torch comparisons.
 *   - hxo_expf: error bound against libm in double, special values.
 *   - GGUF dequantisation: hand-built known-answer blocks for every sub-block
 *     of Q8_0, Q4_K, Q6_K (the public ggml layout), row sizes, divisibility.
 *   - router / softmax / top-k / renorm: closed forms (zero weights), brute
 *     force in double on small shapes, tie and no-renorm cases, and the
 *     reference's own unit tests (moe.rs:223-303, 309-359) restated.
 *   - dispatch: permutation invariants and brute-force stable sort.
 *   - forward: uniform routing = mean of experts, TP partial-sum identity
 *     (tp_qwen3_5.rs:2460-2496), quantised == forward on dequantised weights,
 *     token independence, and an f32 golden from transformers'
 *     Qwen3NextSparseMoeBlock on the C1 shape.
 *   - rmsnorm: closed forms.
 *   - quantisers (candle's from_float rules): known-answer blocks (Q8_0
 *     halves rounded away from zero, Q4_K positive-constant sub-blocks stored
 *     as zero, exact Q4_K / Q6_K lattice round trips that fix d, dmin and the
 *     packed 6-bit / int8 scales), and invariants of the make_qx_quants /
 *     make_qkx1_quants searches (least-squares scale of the returned codes, no
 *     worse than the starting codes, closed forms on two-valued blocks).
 * Parity unpinned (no reference vector or buildable reference exists here):
 *   - hxo_quantize restates candle's from_float rules from the published
 *     algorithms; byte parity with candle itself is unpinned (forward parity
 *     never depends on it: both sides are fed the same GGUF bytes).
 *   - two forward modes: hxo_moe_forward (exact: dequantised weights, products
 *     accumulated in double) and hxo_moe_forward_candle (candle's CPU
 *     quantised-matmul arithmetic, restated in its own section below). The
 *     candle mode is pinned bit for bit against an independent numpy
 *     restatement of the integer vec_dot and against the f64 dot of the
 *     dequantised operands, but not against candle itself (its CPU build is
 *     not available here).
 */
#include <immintrin.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define HXO_F32 0
#define HXO_F16 1
#define HXO_Q8_0 8
#define HXO_Q4_K 12
#define HXO_Q6_K 14
#define HXO_BF16 30

/* ------------------------------------------------------------------------- */
/* scalar formats                                                            */
/* ------------------------------------------------------------------------- */
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

uint16_t hxo_f32_to_bf16(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float hxo_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

uint16_t hxo_f32_to_f16(float f) {
    uint32_t x = f2u(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return sign | 0x7e00u;           /* NaN */
    if (ax >= 0x38800000u) {                                /* f16 normal range */
        uint32_t m = ax + 0xfffu + ((ax >> 13) & 1u);       /* RNE to 10 bits */
        m -= (112u << 23);
        if (m >= 0x0f800000u) return sign | 0x7c00u;        /* overflow -> inf */
        return (uint16_t)(sign | (m >> 13));
    }
    /* f16 subnormal or zero: value * 2^24 rounded to an integer, RNE */
    float v = u2f(ax) * 16777216.0f;
    volatile float r = v + 8388608.0f;
    float q = r - 8388608.0f;
    return (uint16_t)(sign | (uint16_t)q);
}

float hxo_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0) {
        float v = (float)m * 5.9604644775390625e-8f;        /* m * 2^-24 */
        return sign ? -v : v;
    }
    if (e == 31) return u2f(sign | 0x7f800000u | (m << 13));
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

/* exp(x) for the router softmax. Cody-Waite split of ln2 (the Cephes
 * constants 0.693145751953125 + 1.42860682030941723212e-6), then the degree-7
 * Taylor polynomial of e^r on |r| <= ln2/2 in Horner form with fmaf, then an
 * exact scaling by 2^n. Inputs below -87 return 0 (the result would be within
 * a factor 2 of FLT_MIN); inputs above 88.5 return +inf. */
float hxo_expf(float x) {
    if (x != x) return x;
    if (x < -87.0f) return 0.0f;
    if (x > 88.5f) return INFINITY;
    float n = rintf(x * 1.44269504088896341f);
    float r = fmaf(n, -0.693145751953125f, x);
    r = fmaf(n, -1.42860682030941723212e-6f, r);
    float p = 1.98412698412698413e-4f;              /* 1/7! */
    p = fmaf(p, r, 1.38888888888888889e-3f);        /* 1/6! */
    p = fmaf(p, r, 8.33333333333333333e-3f);        /* 1/5! */
    p = fmaf(p, r, 4.16666666666666667e-2f);        /* 1/4! */
    p = fmaf(p, r, 1.66666666666666667e-1f);        /* 1/3! */
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    int ni = (int)n;
    if (ni > 127) return p * u2f((uint32_t)(127 + 127) << 23) * 2.0f;
    return p * u2f((uint32_t)(ni + 127) << 23);
}

/* ------------------------------------------------------------------------- */
/* GGUF blocks (public ggml format)                                          */
/* ------------------------------------------------------------------------- */
int64_t hxo_block_elems(int dtype) {
    switch (dtype) {
    case HXO_F32: case HXO_F16: case HXO_BF16: return 1;
    case HXO_Q8_0: return 32;
    case HXO_Q4_K: case HXO_Q6_K: return 256;
    default: return 0;
    }
}

int64_t hxo_block_bytes(int dtype) {
    switch (dtype) {
    case HXO_F32: return 4;
    case HXO_F16: case HXO_BF16: return 2;
    case HXO_Q8_0: return 34;
    case HXO_Q4_K: return 144;
    case HXO_Q6_K: return 210;
    default: return 0;
    }
}

/* bytes of one row of n elements; -1 if n does not tile into whole blocks */
int64_t hxo_row_bytes(int dtype, int64_t n) {
    int64_t be = hxo_block_elems(dtype);
    if (be == 0 || n % be) return -1;
    return n / be * hxo_block_bytes(dtype);
}

static inline float ld_f16(const uint8_t* p) { uint16_t h; memcpy(&h, p, 2); return hxo_f16_to_f32(h); }

static void dq_q8_0(const uint8_t* b, float* y) {
    float d = ld_f16(b);
    const int8_t* qs = (const int8_t*)(b + 2);
    for (int j = 0; j < 32; j++) y[j] = d * (float)qs[j];
}

/* Q4_K 6-bit scale/min of sub-block j from the 12 packed bytes */
static void q4k_scale_min(int j, const uint8_t* s, int* sc, int* m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
        *m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

static void dq_q4_k(const uint8_t* b, float* y) {
    float d = ld_f16(b), dmin = ld_f16(b + 2);
    const uint8_t* sc = b + 4;
    const uint8_t* qs = b + 16;
    for (int c = 0; c < 4; c++) {
        int s0, m0, s1, m1;
        q4k_scale_min(2 * c, sc, &s0, &m0);
        q4k_scale_min(2 * c + 1, sc, &s1, &m1);
        float d0 = d * (float)s0, mm0 = dmin * (float)m0;
        float d1 = d * (float)s1, mm1 = dmin * (float)m1;
        for (int l = 0; l < 32; l++) {
            uint8_t q = qs[32 * c + l];
            y[64 * c + l] = d0 * (float)(q & 0xF) - mm0;
            y[64 * c + 32 + l] = d1 * (float)(q >> 4) - mm1;
        }
    }
}

static void dq_q6_k(const uint8_t* b, float* y) {
    const uint8_t* ql = b;
    const uint8_t* qh = b + 128;
    const int8_t* sc = (const int8_t*)(b + 192);
    float d = ld_f16(b + 208);
    for (int n = 0; n < 2; n++) {
        for (int l = 0; l < 32; l++) {
            int is = l / 16;
            int q1 = (int)((ql[64 * n + l] & 0xF) | (((qh[32 * n + l] >> 0) & 3) << 4)) - 32;
            int q2 = (int)((ql[64 * n + l + 32] & 0xF) | (((qh[32 * n + l] >> 2) & 3) << 4)) - 32;
            int q3 = (int)((ql[64 * n + l] >> 4) | (((qh[32 * n + l] >> 4) & 3) << 4)) - 32;
            int q4 = (int)((ql[64 * n + l + 32] >> 4) | (((qh[32 * n + l] >> 6) & 3) << 4)) - 32;
            y[128 * n + l] = d * (float)sc[8 * n + is] * (float)q1;
            y[128 * n + l + 32] = d * (float)sc[8 * n + is + 2] * (float)q2;
            y[128 * n + l + 64] = d * (float)sc[8 * n + is + 4] * (float)q3;
            y[128 * n + l + 96] = d * (float)sc[8 * n + is + 6] * (float)q4;
        }
    }
}

/* dequantise n elements (a whole number of blocks) to f32 */
int hxo_dequant(int dtype, const void* src, int64_t n, float* dst) {
    const uint8_t* s = (const uint8_t*)src;
    int64_t be = hxo_block_elems(dtype), bb = hxo_block_bytes(dtype);
    if (be == 0 || n % be) return 1;
    for (int64_t b = 0; b < n / be; b++) {
        const uint8_t* blk = s + b * bb;
        float* y = dst + b * be;
        switch (dtype) {
        case HXO_F32: memcpy(y, blk, 4); break;
        case HXO_F16: *y = ld_f16(blk); break;
        case HXO_BF16: { uint16_t h; memcpy(&h, blk, 2); *y = hxo_bf16_to_f32(h); } break;
        case HXO_Q8_0: dq_q8_0(blk, y); break;
        case HXO_Q4_K: dq_q4_k(blk, y); break;
        case HXO_Q6_K: dq_q6_k(blk, y); break;
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------- */
/* quantisers: candle's GgmlType::from_float, which quantize_parallel calls   */
/* (isq.rs:98, 104-112) and which isq.rs:1-19, 123-161 hold byte-identical to  */
/* QTensor::quantize. candle-core 0.11's k_quants port of ggml's first         */
/* k_quants.c reference quantisers (third-party, not vendored in the          */
/* reference; restated from the published algorithms):                        */
/*   Q8_0  d = amax / 127, q = round-half-away(x / d)  (BlockQ8_0::from_float) */
/*   Q4_K  make_qkx1_quants(nmax 15, 5 tries) per 32 elements, scales / mins  */
/*         to 6 bits against their maxima, codes re-fitted (BlockQ4K)         */
/*   Q6_K  make_qx_quants(16, nmax 32, rmse_type 1) per 16 elements, scales   */
/*         to int8 against -128 / (largest-|.| scale), codes re-fitted        */
/* nearest_int is f32::round (half away from zero) followed by Rust's          */
/* saturating float -> int cast (NaN -> 0).                                   */
/* ------------------------------------------------------------------------- */
static inline int rs_nearest(float v) {
    float r = roundf(v);
    if (r != r) return 0;
    if (r >= 2147483648.0f) return INT32_MAX;
    if (r < -2147483648.0f) return INT32_MIN;
    return (int)r;
}

static inline int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* Rust `as i8` from f32: round toward zero, saturate, NaN -> 0 (the value here
 * is already rounded) */
static inline int8_t rs_f32_to_i8(float v) {
    if (v != v) return 0;
    if (v >= 127.0f) return 127;
    if (v <= -128.0f) return -128;
    return (int8_t)v;
}

static void qz_q8_0(const float* x, uint8_t* b) {
    float amax = 0.0f;
    for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(x[j]));
    float d = amax / 127.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint16_t dh = hxo_f32_to_f16(d);
    memcpy(b, &dh, 2);
    for (int j = 0; j < 32; j++) b[2 + j] = (uint8_t)rs_f32_to_i8(roundf(x[j] * id));
}

/* make_qkx1_quants(nmax, ntry, x[n]) -> (scale, -min): alternate the codes
 * l = clamp(round((x - min) / scale), 0, nmax) with the least-squares scale
 * sum((x - min) l) / sum(l^2) and the mean residual min (clamped to <= 0),
 * starting from min = min(0, min x), scale = (max - min) / nmax, until the
 * codes stop changing or ntry rounds ran. The codes start at 0. */
static void make_qkx1(const float* x, int n, int nmax, int ntry, float* scale_out, float* min_out) {
    float mn = x[0], mx = x[0];
    for (int i = 1; i < n; i++) {
        if (x[i] < mn) mn = x[i];
        if (x[i] > mx) mx = x[i];
    }
    if (mx == mn) {
        *scale_out = 0.0f;
        *min_out = 0.0f;
        return;
    }
    if (mn > 0.0f) mn = 0.0f;
    float iscale = (float)nmax / (mx - mn);
    float scale = 1.0f / iscale;
    uint8_t L[256];
    memset(L, 0, sizeof L);
    for (int t = 0; t < ntry; t++) {
        float sumlx = 0.0f;
        int suml2 = 0, changed = 0;
        for (int i = 0; i < n; i++) {
            int li = clampi(rs_nearest(iscale * (x[i] - mn)), 0, nmax);
            if ((uint8_t)li != L[i]) {
                L[i] = (uint8_t)li;
                changed = 1;
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
    *scale_out = scale;
    *min_out = -mn;
}

static void qz_q4_k(const float* x, uint8_t* b) {
    float scales[8], mins[8];
    for (int j = 0; j < 8; j++) make_qkx1(x + 32 * j, 32, 15, 5, &scales[j], &mins[j]);
    float max_scale = 0.0f, max_min = 0.0f;
    for (int j = 0; j < 8; j++) {
        max_scale = fmaxf(scales[j], max_scale);
        max_min = fmaxf(mins[j], max_min);
    }
    float inv_scale = max_scale > 0.0f ? 63.0f / max_scale : 0.0f;
    float inv_min = max_min > 0.0f ? 63.0f / max_min : 0.0f;
    uint8_t* s = b + 4;
    memset(s, 0, 12);
    for (int j = 0; j < 8; j++) {
        int a = rs_nearest(inv_scale * scales[j]), m = rs_nearest(inv_min * mins[j]);
        uint8_t ls = (uint8_t)(a < 63 ? a : 63), lm = (uint8_t)(m < 63 ? m : 63);
        if (j < 4) {
            s[j] = ls;
            s[j + 4] = lm;
        } else {
            s[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
            s[j - 4] |= (uint8_t)((ls >> 4) << 6);
            s[j] |= (uint8_t)((lm >> 4) << 6);
        }
    }
    uint16_t dh = hxo_f32_to_f16(max_scale / 63.0f), mh = hxo_f32_to_f16(max_min / 63.0f);
    memcpy(b, &dh, 2);
    memcpy(b + 2, &mh, 2);
    float d = hxo_f16_to_f32(dh), dmin = hxo_f16_to_f32(mh);
    uint8_t q[256];
    memset(q, 0, sizeof q);
    for (int j = 0; j < 8; j++) {
        int sc, m;
        q4k_scale_min(j, s, &sc, &m);
        float dd = d * (float)sc;
        if (dd == 0.0f) continue;
        float dm = dmin * (float)m;
        for (int l = 0; l < 32; l++) q[32 * j + l] = (uint8_t)clampi(rs_nearest((x[32 * j + l] + dm) / dd), 0, 15);
    }
    uint8_t* qs = b + 16;
    for (int c = 0; c < 4; c++)
        for (int l = 0; l < 32; l++)
            qs[32 * c + l] = (uint8_t)(q[64 * c + l] | (q[64 * c + 32 + l] << 4));
}

/* make_qx_quants(n, nmax, x, L, rmse_type) for rmse_type 1 (weights x^2):
 * codes l in [-nmax, nmax - 1] from the largest-|x| element's scale, then up to
 * 3 rounds re-deriving the codes from the least-squares scale while the
 * weighted fit improves, then up to 5 rounds of single-code moves that
 * improve it. Returns the scale; L holds l + nmax. */
static float make_qx(int n, int nmax, const float* x, int8_t* L) {
    float max = 0.0f, amax = 0.0f;
    for (int i = 0; i < n; i++) {
        float ax = fabsf(x[i]);
        if (ax > amax) {
            amax = ax;
            max = x[i];
        }
    }
    if (amax == 0.0f) {
        for (int i = 0; i < n; i++) L[i] = 0;
        return 0.0f;
    }
    float iscale = -(float)nmax / max;
    float sumlx = 0.0f, suml2 = 0.0f;
    for (int i = 0; i < n; i++) {
        int l = clampi(rs_nearest(iscale * x[i]), -nmax, nmax - 1);
        L[i] = (int8_t)(l + nmax);
        float w = x[i] * x[i];
        sumlx += w * x[i] * (float)l;
        suml2 += w * (float)l * (float)l;
    }
    float scale = sumlx / suml2;
    float best = scale * sumlx;
    for (int t = 0; t < 3; t++) {
        float is = 1.0f / scale;
        float slx = 0.0f, sl2 = 0.0f;
        int changed = 0;
        for (int i = 0; i < n; i++) {
            int l = clampi(rs_nearest(is * x[i]), -nmax, nmax - 1);
            if (l + nmax != (int)L[i]) changed = 1;
            float w = x[i] * x[i];
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
            float w = x[i] * x[i];
            int l = (int)L[i] - nmax;
            float slx = sumlx - w * x[i] * (float)l;
            if (slx > 0.0f) {
                float sl2 = suml2 - w * (float)l * (float)l;
                int new_l = clampi(rs_nearest(x[i] * sl2 / slx), -nmax, nmax - 1);
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

static void qz_q6_k(const float* x, uint8_t* b) {
    int8_t L[256];
    float scales[16];
    float max_scale = 0.0f, max_abs_scale = 0.0f;
    for (int ib = 0; ib < 16; ib++) {
        float sc = make_qx(16, 32, x + 16 * ib, L + 16 * ib);
        scales[ib] = sc;
        float as = fabsf(sc);
        if (as > max_abs_scale) {
            max_abs_scale = as;
            max_scale = sc;
        }
    }
    float iscale = -128.0f / max_scale;
    uint16_t dh = hxo_f32_to_f16(1.0f / iscale);
    int8_t* ysc = (int8_t*)(b + 192);
    for (int i = 0; i < 16; i++) {
        int v = rs_nearest(iscale * scales[i]);
        ysc[i] = (int8_t)(uint8_t)(v < 127 ? v : 127);
    }
    float d = hxo_f16_to_f32(dh);
    for (int j = 0; j < 16; j++) {
        float dj = d * (float)ysc[j];
        if (dj == 0.0f) continue;
        for (int l = 0; l < 16; l++) L[16 * j + l] = (int8_t)(clampi(rs_nearest(x[16 * j + l] / dj), -32, 31) + 32);
    }
    uint8_t* ql = b;
    uint8_t* qh = b + 128;
    for (int n = 0; n < 2; n++) {
        for (int l = 0; l < 32; l++) {
            uint8_t q1 = (uint8_t)L[128 * n + l], q2 = (uint8_t)L[128 * n + 32 + l];
            uint8_t q3 = (uint8_t)L[128 * n + 64 + l], q4 = (uint8_t)L[128 * n + 96 + l];
            ql[64 * n + l] = (uint8_t)((q1 & 0xF) | ((q3 & 0xF) << 4));
            ql[64 * n + 32 + l] = (uint8_t)((q2 & 0xF) | ((q4 & 0xF) << 4));
            qh[32 * n + l] = (uint8_t)(((q1 >> 4) & 3) | (((q2 >> 4) & 3) << 2) | (((q3 >> 4) & 3) << 4) |
                                       (((q4 >> 4) & 3) << 6));
        }
    }
    memcpy(b + 208, &dh, 2);
}

/* the per-sub-block searches on their own (test hooks) */
float hxo_make_qx(int n, int nmax, const float* x, int8_t* L) {
    return n > 0 && n <= 256 ? make_qx(n, nmax, x, L) : 0.0f;
}
void hxo_make_qkx1(int n, int nmax, int ntry, const float* x, float* scale, float* min) {
    if (n > 0 && n <= 256) make_qkx1(x, n, nmax, ntry, scale, min);
}

/* quantise a [rows, cols] f32 matrix into GGUF rows; cols must tile into blocks
 * (the same constraint as isq.rs:62-68). Returns 0 on success. */
int hxo_quantize(int dtype, const float* src, int64_t rows, int64_t cols, void* dst, int nthreads) {
    int64_t be = hxo_block_elems(dtype), bb = hxo_block_bytes(dtype);
    if (be == 0 || cols <= 0 || cols % be) return 1;
    int64_t nb = rows * (cols / be);
    uint8_t* d = (uint8_t*)dst;
#ifdef _OPENMP
    if (nthreads <= 0) nthreads = omp_get_max_threads();
#pragma omp parallel for schedule(static) num_threads(nthreads)
#endif
    for (int64_t b = 0; b < nb; b++) {
        const float* x = src + b * be;
        uint8_t* o = d + b * bb;
        switch (dtype) {
        case HXO_F32: memcpy(o, x, 4); break;
        case HXO_F16: { uint16_t h = hxo_f32_to_f16(*x); memcpy(o, &h, 2); } break;
        case HXO_BF16: { uint16_t h = hxo_f32_to_bf16(*x); memcpy(o, &h, 2); } break;
        case HXO_Q8_0: qz_q8_0(x, o); break;
        case HXO_Q4_K: qz_q4_k(x, o); break;
        case HXO_Q6_K: qz_q6_k(x, o); break;
        }
    }
    (void)nthreads;
    return 0;
}

/* ------------------------------------------------------------------------- */
/* router                                                                     */
/* ------------------------------------------------------------------------- */
static inline float ld_act(int dtype, const void* p, int64_t i) {
    if (dtype == HXO_BF16) return hxo_bf16_to_f32(((const uint16_t*)p)[i]);
    return ((const float*)p)[i];
}

/* 64 lane partials combined by the xor butterfly 32,16,8,4,2,1 */
static float butterfly64(float* p) {
    for (int off = 32; off >= 1; off >>= 1) {
        float q[64];
        for (int l = 0; l < 64; l++) q[l] = p[l] + p[l ^ off];
        memcpy(p, q, sizeof q);
    }
    return p[0];
}

/* canonical router dot product of x (act dtype) and one router row (router dtype) */
static float router_dot(int act_dtype, const void* x, int router_dtype, const void* w, int64_t H) {
    float acc[64];
    for (int l = 0; l < 64; l++) acc[l] = 0.0f;
    for (int64_t g = 0; 8 * g < H; g++) {
        int l = (int)(g % 64);
        for (int i = 0; i < 8 && 8 * g + i < H; i++) {
            int64_t h = 8 * g + i;
            acc[l] = fmaf(ld_act(act_dtype, x, h), ld_act(router_dtype, w, h), acc[l]);
        }
    }
    return butterfly64(acc);
}

typedef struct hxo_moe {
    int32_t hidden, num_experts, top_k, inter, shared_inter, norm_topk_prob, act_dtype;
    int32_t router_dtype; const void* router;        /* [E, H] */
    int32_t gate_dtype; const void* gate;            /* [E, I, H] GGUF rows */
    int32_t up_dtype; const void* up;                /* [E, I, H] */
    int32_t down_dtype; const void* down;            /* [E, H, I] */
    int32_t sgate_dtype; const void* sgate;          /* [Is, H] */
    int32_t sup_dtype; const void* sup;              /* [Is, H] */
    int32_t sdown_dtype; const void* sdown;          /* [H, Is] */
    int32_t seg_dtype; const void* seg;              /* shared_expert_gate [1, H] */
} hxo_moe;

/* logits [T, E] exactly as the router kernel produces them (rounded to the
 * activation dtype, then + bias if given) */
/* the same chains with the operands laid out lane-major, p[(g * 8 + i) * 64 + l]
 * = v[8 (64 g + l) + i] for H a multiple of 512: lane l's fmaf chain runs over
 * its groups g and their elements i in the canonical order, 64 lanes side by
 * side (one vector instruction per 8 lanes) */
static void lane_major(int dtype, const void* v, int64_t H, float* p) {
    for (int64_t g = 0; g < H / 512; g++)
        for (int i = 0; i < 8; i++)
            for (int l = 0; l < 64; l++) p[(g * 8 + i) * 64 + l] = ld_act(dtype, v, 8 * (64 * g + l) + i);
}

static float router_dot_lm(const float* xp, const float* wp, int64_t H) {
    float acc[64];
    for (int l = 0; l < 64; l++) acc[l] = 0.0f;
    for (int64_t gi = 0; gi < H / 64; gi++)
        for (int l = 0; l < 64; l++) acc[l] = fmaf(xp[gi * 64 + l], wp[gi * 64 + l], acc[l]);
    return butterfly64(acc);
}

int hxo_router_logits(const hxo_moe* m, const void* x, int64_t T, const float* bias, float* logits) {
    int64_t H = m->hidden, E = m->num_experts;
    int64_t wrow = H * (m->router_dtype == HXO_BF16 ? 2 : 4);
    int64_t xrow = H * (m->act_dtype == HXO_BF16 ? 2 : 4);
    if (H % 512 == 0) {
        float* wp = (float*)malloc(sizeof(float) * (size_t)(E * H));
        if (!wp) return 2;
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
        for (int64_t e = 0; e < E; e++) lane_major(m->router_dtype, (const uint8_t*)m->router + e * wrow, H, wp + e * H);
#ifdef _OPENMP
#pragma omp parallel
#endif
        {
            float* xp = (float*)malloc(sizeof(float) * (size_t)H);
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
            for (int64_t t = 0; t < T; t++) {
                lane_major(m->act_dtype, (const uint8_t*)x + t * xrow, H, xp);
                for (int64_t e = 0; e < E; e++) {
                    float v = router_dot_lm(xp, wp + e * H, H);
                    if (m->act_dtype == HXO_BF16) v = hxo_bf16_to_f32(hxo_f32_to_bf16(v));
                    if (bias) v = v + bias[e];
                    logits[t * E + e] = v;
                }
            }
            free(xp);
        }
        free(wp);
        return 0;
    }
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
    for (int64_t t = 0; t < T; t++) {
        const void* xt = (const uint8_t*)x + t * xrow;
        for (int64_t e = 0; e < E; e++) {
            float v = router_dot(m->act_dtype, xt, m->router_dtype, (const uint8_t*)m->router + e * wrow, H);
            if (m->act_dtype == HXO_BF16) v = hxo_bf16_to_f32(hxo_f32_to_bf16(v));
            if (bias) v = v + bias[e];
            logits[t * E + e] = v;
        }
    }
    return 0;
}

/* softmax over E with the lane-strided sum + butterfly */
static void softmax_row(const float* l, int64_t E, float* p) {
    float mx = l[0];
    for (int64_t e = 1; e < E; e++) if (l[e] > mx) mx = l[e];
    float acc[64];
    for (int i = 0; i < 64; i++) acc[i] = 0.0f;
    for (int64_t e = 0; e < E; e++) {
        p[e] = hxo_expf(l[e] - mx);
        acc[e % 64] = acc[e % 64] + p[e];
    }
    float s = butterfly64(acc);
    for (int64_t e = 0; e < E; e++) p[e] = p[e] / s;
}

/* k largest with ties to the lower index; selection by repeated scan */
static void topk_row(const float* p, int64_t E, int k, int32_t* idx, unsigned char* taken) {
    memset(taken, 0, (size_t)E);
    for (int j = 0; j < k; j++) {
        int64_t best = -1;
        for (int64_t e = 0; e < E; e++) {
            if (taken[e]) continue;
            if (best < 0 || p[e] > p[best]) best = e;
        }
        taken[best] = 1;
        idx[j] = (int32_t)best;
    }
}

/* route_scatter (moe.rs:124-162) up to the device->host copy: probs, top-k ids and
 * weights. Any of the outputs may be NULL. */
int hxo_route(const hxo_moe* m, const void* x, int64_t T, const float* bias,
              float* logits_out, float* probs_out, int32_t* topk_idx, float* topk_w) {
    int64_t E = m->num_experts;
    int k = m->top_k;
    if (k <= 0 || k > E || k > 1024 || E > 65536) return 1;
    float* logits = (float*)malloc(sizeof(float) * T * E);
    float* probs = (float*)malloc(sizeof(float) * T * E);
    if (!logits || !probs) { free(logits); free(probs); return 2; }
    int rc = hxo_router_logits(m, x, T, bias, logits);
    if (rc) { free(logits); free(probs); return rc; }
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
    for (int64_t t = 0; t < T; t++) {
        int32_t ids[1024];
        unsigned char taken[65536];
        softmax_row(logits + t * E, E, probs + t * E);
        topk_row(probs + t * E, E, k, ids, taken);
        float s = 0.0f;
        for (int j = 0; j < k; j++) s = s + probs[t * E + ids[j]];
        for (int j = 0; j < k; j++) {
            float w = probs[t * E + ids[j]];
            if (m->norm_topk_prob) w = w / s;
            if (topk_idx) topk_idx[t * k + j] = ids[j];
            if (topk_w) topk_w[t * k + j] = w;
        }
    }
    if (logits_out) memcpy(logits_out, logits, sizeof(float) * T * E);
    if (probs_out) memcpy(probs_out, probs, sizeof(float) * T * E);
    free(logits);
    free(probs);
    return 0;
}

/* dispatch permutation: flat index f = t*k + j stably sorted by expert id
 * (tp_qwen3_5.rs:1189; equals moe.rs:152-160's ascending-token lists).
 * perm[pos] = f, offsets[E+1] exclusive scan of the histogram, inv[f] = pos. */
int hxo_dispatch(const int32_t* topk_idx, int64_t T, int k, int64_t E,
                 int32_t* perm, int32_t* offsets, int32_t* inv) {
    int64_t F = T * k;
    int32_t* cnt = (int32_t*)calloc((size_t)E + 1, sizeof(int32_t));
    if (!cnt) return 2;
    for (int64_t f = 0; f < F; f++) {
        int32_t e = topk_idx[f];
        if (e < 0 || e >= E) { free(cnt); return 1; }
        cnt[e]++;
    }
    int32_t run = 0;
    for (int64_t e = 0; e < E; e++) { int32_t c = cnt[e]; offsets[e] = run; cnt[e] = run; run += c; }
    offsets[E] = run;
    for (int64_t f = 0; f < F; f++) {
        int32_t pos = cnt[topk_idx[f]]++;
        perm[pos] = (int32_t)f;
        if (inv) inv[f] = pos;
    }
    free(cnt);
    return 0;
}

/* ------------------------------------------------------------------------- */
/* forward                                                                    */
/* ------------------------------------------------------------------------- */
/* dot product with a fixed order: 8 interleaved double accumulators summed
 * pairwise at the end (deterministic, vectorisable without reassociation) */
static double dotd(const float* a, const float* b, int64_t K) {
    double s[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int64_t i = 0;
    for (; i + 8 <= K; i += 8)
        for (int j = 0; j < 8; j++) s[j] += (double)a[i + j] * (double)b[i + j];
    for (; i < K; i++) s[0] += (double)a[i] * (double)b[i];
    return ((s[0] + s[4]) + (s[1] + s[5])) + ((s[2] + s[6]) + (s[3] + s[7]));
}

static inline float silu_f(float g) { return g / (1.0f + expf(-g)); }

/* One SwiGLU expert (mlp.rs:54-60) over the n tokens rows[0..n) of xf:
 * acc[rows[p]] += scale[p] * down(silu(gate x) * up x).
 * gate/up are [I, H] GGUF rows, down is [H, I]. hbuf holds n*I floats. */
static void expert_rows(int gdt, const void* g, int udt, const void* u, int ddt, const void* d,
                        int64_t H, int64_t I, const float* xf, const int32_t* rows, const double* scale,
                        int64_t n, double* acc, float* hbuf, int nthreads) {
    int64_t grb = hxo_row_bytes(gdt, H), urb = hxo_row_bytes(udt, H), drb = hxo_row_bytes(ddt, I);
#ifdef _OPENMP
#pragma omp parallel num_threads(nthreads)
#endif
    {
        /* wg also holds a down row (I elements) in the second loop */
        float* wg = (float*)malloc(sizeof(float) * (H > I ? H : I));
        float* wu = (float*)malloc(sizeof(float) * H);
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
        for (int64_t i = 0; i < I; i++) {
            hxo_dequant(gdt, (const uint8_t*)g + i * grb, H, wg);
            hxo_dequant(udt, (const uint8_t*)u + i * urb, H, wu);
            for (int64_t p = 0; p < n; p++) {
                const float* xt = xf + (int64_t)rows[p] * H;
                float gv = (float)dotd(wg, xt, H), uv = (float)dotd(wu, xt, H);
                hbuf[p * I + i] = silu_f(gv) * uv;
            }
        }
        float* wd = wg;
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
        for (int64_t r = 0; r < H; r++) {
            hxo_dequant(ddt, (const uint8_t*)d + r * drb, I, wd);
            for (int64_t p = 0; p < n; p++)
                acc[(int64_t)rows[p] * H + r] += scale[p] * dotd(wd, hbuf + p * I, I);
        }
        free(wg);
        free(wu);
    }
}

/* Module::forward (moe.rs:164-199): the scatter loop over experts in ascending
 * id, each expert's tokens ascending (moe.rs:178-189), then the sigmoid-gated
 * shared expert (moe.rs:191-195). y is f32 [T, H], not rounded to the
 * activation dtype; products accumulate in double. */
int hxo_moe_forward(const hxo_moe* m, const void* x, int64_t T, const float* bias, float* y, int nthreads) {
    int64_t H = m->hidden, E = m->num_experts, I = m->inter, Is = m->shared_inter;
    int k = m->top_k;
    if (hxo_row_bytes(m->gate_dtype, H) < 0 || hxo_row_bytes(m->up_dtype, H) < 0 ||
        hxo_row_bytes(m->down_dtype, I) < 0)
        return 1;
    if (Is > 0 && (hxo_row_bytes(m->sgate_dtype, H) < 0 || hxo_row_bytes(m->sup_dtype, H) < 0 ||
                   hxo_row_bytes(m->sdown_dtype, Is) < 0 || !m->seg))
        return 1;
#ifdef _OPENMP
    if (nthreads <= 0) nthreads = omp_get_max_threads();
#else
    nthreads = 1;
#endif
    int64_t F = T * k, KM = I > Is ? I : Is;
    int32_t* idx = (int32_t*)malloc(sizeof(int32_t) * F);
    float* w = (float*)malloc(sizeof(float) * F);
    int32_t* perm = (int32_t*)malloc(sizeof(int32_t) * F);
    int32_t* offs = (int32_t*)malloc(sizeof(int32_t) * (E + 1));
    int32_t* rows = (int32_t*)malloc(sizeof(int32_t) * (T > F ? T : F));
    double* sc = (double*)malloc(sizeof(double) * (T > F ? T : F));
    float* xf = (float*)malloc(sizeof(float) * T * H);
    float* hbuf = (float*)malloc(sizeof(float) * (T > F ? T : F) * KM);
    double* acc = (double*)calloc((size_t)(T * H), sizeof(double));
    int rc = 0;
    if (!idx || !w || !perm || !offs || !rows || !sc || !xf || !hbuf || !acc) { rc = 2; goto done; }
    rc = hxo_route(m, x, T, bias, NULL, NULL, idx, w);
    if (rc) goto done;
    rc = hxo_dispatch(idx, T, k, E, perm, offs, NULL);
    if (rc) goto done;
    for (int64_t i = 0; i < T * H; i++) xf[i] = ld_act(m->act_dtype, x, i);
    {
        int64_t gb = hxo_row_bytes(m->gate_dtype, H) * I, ub = hxo_row_bytes(m->up_dtype, H) * I;
        int64_t db = hxo_row_bytes(m->down_dtype, I) * H;
        for (int64_t e = 0; e < E; e++) {
            int64_t n = offs[e + 1] - offs[e];
            if (n == 0) continue;
            for (int64_t p = 0; p < n; p++) {
                int32_t f = perm[offs[e] + p];
                rows[p] = f / k;
                sc[p] = (double)w[f];
            }
            expert_rows(m->gate_dtype, (const uint8_t*)m->gate + e * gb, m->up_dtype,
                        (const uint8_t*)m->up + e * ub, m->down_dtype, (const uint8_t*)m->down + e * db,
                        H, I, xf, rows, sc, n, acc, hbuf, nthreads);
        }
    }
    if (Is > 0) {
        float* wr = (float*)malloc(sizeof(float) * H);
        hxo_dequant(m->seg_dtype, m->seg, H, wr);
        for (int64_t t = 0; t < T; t++) {
            rows[t] = (int32_t)t;
            sc[t] = 1.0 / (1.0 + exp(-dotd(wr, xf + t * H, H)));
        }
        free(wr);
        expert_rows(m->sgate_dtype, m->sgate, m->sup_dtype, m->sup, m->sdown_dtype, m->sdown,
                    H, Is, xf, rows, sc, T, acc, hbuf, nthreads);
    }
    for (int64_t i = 0; i < T * H; i++) y[i] = (float)acc[i];
done:
    free(idx); free(w); free(perm); free(offs); free(rows); free(sc); free(xf); free(hbuf); free(acc);
    return rc;
}

/* Qwen3_5RmsNorm::forward (rmsnorm.rs:67-80): x * rsqrt(mean(x^2) + eps) * (1 + w),
 * computed in f32; output f32 (caller rounds). */
int hxo_rmsnorm(int act_dtype, const void* x, int64_t T, int64_t H, const float* w, float eps, float* y) {
    for (int64_t t = 0; t < T; t++) {
        double ss = 0.0;
        for (int64_t i = 0; i < H; i++) { double v = ld_act(act_dtype, x, t * H + i); ss += v * v; }
        float inv = (float)(1.0 / sqrt(ss / (double)H + (double)eps));
        for (int64_t i = 0; i < H; i++) y[t * H + i] = ld_act(act_dtype, x, t * H + i) * inv * (1.0f + w[i]);
    }
    return 0;
}

/* ------------------------------------------------------------------------- */
/* candle's quantised-matmul arithmetic: the second forward mode             */
/* ------------------------------------------------------------------------- */
/* hxo_moe_forward_candle restates the reference's CPU path for quantised
 * experts (the Scatter store, tp_qwen3_5.rs:1105-1138, each expert a TpExpert
 * at world size 1, tp_qwen3_5.rs:840-850, whose projections are
 * MaybeQuantLinear, tp_linear.rs:98-140) with candle's CPU arithmetic
 * (candle-core 0.11, third-party, not vendored; restated from the published
 * algorithms):
 *   - m = rows of the call (the tokens routed to the expert; T for the shared
 *     expert). m <= 64: x is quantised per row to the weight type's vec_dot
 *     type (Q8_0 for Q8_0 weights, Q8_K for Q4_K / Q6_K) and every output is
 *     candle's generic vec_dot (vec_dot_unopt: what x86-64 runs without
 *     target-cpu flags, which the reference's build does not set): integer
 *     block dot products, then the per-block float steps in candle's order.
 *   - m > 64 (forward_via_f16): weights dequantised and rounded to f16, x
 *     rounded to f16, f32 accumulation (an fmaf chain over k), the output
 *     rounded to f16 and cast back.
 *   - f32 / bf16 weights: an f32 fmaf chain over k.
 *   - SwiGLU silu(g) * u with silu(v) = v / (1 + exp(-v)), f32 (mlp.rs:54-60);
 *     ys[t] += out * w per expert ascending (index_add, moe.rs:178-189); then
 *     ys + shared * sigmoid(x . w_sg) (moe.rs:191-195).
 * Routing (ids, weights) is the canonical routing of hxo_route, so both modes
 * and the GPU combine the same experts with the same weights.
 * Parity unpinned against candle itself: its CPU build is not available here.
 * Pinned by tests/test_oracle.py: the Q8_K quantiser's invariants, the vec_dot
 * integer identities (each equals the f64 dot of the dequantised operands up
 * to float rounding), and agreement with the exact mode within tolerance. */

/* Q8_K block (the k-quants vec_dot type): f32 d, 256 int8, 16 sums of 16 */
typedef struct {
    float d;
    int8_t qs[256];
    int16_t bsums[16];
} q8k_t;

/* BlockQ8K::from_float: iscale = -128 / (signed largest-|x| value),
 * q = min(round(iscale x), 127), d = 1 / iscale; an all-zero block is zero */
static void quant_q8_k(const float* x, q8k_t* y) {
    float max = 0.0f, amax = 0.0f;
    for (int j = 0; j < 256; j++) {
        float ax = fabsf(x[j]);
        if (amax < ax) {
            amax = ax;
            max = x[j];
        }
    }
    memset(y, 0, sizeof *y);
    if (amax == 0.0f) return;
    float iscale = -128.0f / max;
    for (int j = 0; j < 256; j++) {
        float v = roundf(iscale * x[j]);
        y->qs[j] = rs_f32_to_i8(v < 127.0f ? v : 127.0f);
    }
    for (int j = 0; j < 16; j++) {
        int s = 0;
        for (int i = 0; i < 16; i++) s += y->qs[16 * j + i];
        y->bsums[j] = (int16_t)s;
    }
    y->d = 1.0f / iscale;
}

/* test hook: one row of Q8_K blocks, as (d, qs, bsums) arrays */
int hxo_quant_q8_k(const float* x, int64_t n, float* d, int8_t* qs, int16_t* bsums) {
    if (n <= 0 || n % 256) return 1;
    for (int64_t b = 0; b < n / 256; b++) {
        q8k_t y;
        quant_q8_k(x + 256 * b, &y);
        d[b] = y.d;
        memcpy(qs + 256 * b, y.qs, 256);
        memcpy(bsums + 16 * b, y.bsums, 32);
    }
    return 0;
}

/* one weight row decoded once for the vec_dot loop over the activation rows */
typedef struct {
    int8_t* a;       /* [K] codes: Q8_0 quants, Q4_K 0..15, Q6_K -32..31 */
    float* d;        /* per block: f16 d (Q8_0, Q4_K, Q6_K) */
    float* dmin;     /* per superblock: f16 dmin (Q4_K) */
    int32_t* sc;     /* per sub-block: 6-bit scale (Q4_K, 8 per superblock) or int8 scale (Q6_K, 16) */
    int32_t* mn;     /* per sub-block: 6-bit min (Q4_K) */
} wrow_t;

static void decode_row(int dt, const uint8_t* r, int64_t K, wrow_t* w) {
    if (dt == HXO_Q8_0) {
        for (int64_t b = 0; b < K / 32; b++) {
            const uint8_t* p = r + 34 * b;
            w->d[b] = ld_f16(p);
            memcpy(w->a + 32 * b, p + 2, 32);
        }
    } else if (dt == HXO_Q4_K) {
        for (int64_t b = 0; b < K / 256; b++) {
            const uint8_t* p = r + 144 * b;
            w->d[b] = ld_f16(p);
            w->dmin[b] = ld_f16(p + 2);
            for (int j = 0; j < 8; j++) {
                int s, m;
                q4k_scale_min(j, p + 4, &s, &m);
                w->sc[8 * b + j] = s;
                w->mn[8 * b + j] = m;
            }
            int8_t* a = w->a + 256 * b;
            for (int c = 0; c < 4; c++)
                for (int l = 0; l < 32; l++) {
                    a[64 * c + l] = (int8_t)(p[16 + 32 * c + l] & 0xF);
                    a[64 * c + 32 + l] = (int8_t)(p[16 + 32 * c + l] >> 4);
                }
        }
    } else {   /* Q6_K */
        for (int64_t b = 0; b < K / 256; b++) {
            const uint8_t* p = r + 210 * b;
            const uint8_t* ql = p;
            const uint8_t* qh = p + 128;
            w->d[b] = ld_f16(p + 208);
            for (int j = 0; j < 16; j++) w->sc[16 * b + j] = (int8_t)p[192 + j];
            int8_t* a = w->a + 256 * b;
            for (int n = 0; n < 2; n++)
                for (int l = 0; l < 32; l++) {
                    a[128 * n + l] = (int8_t)(((ql[64 * n + l] & 0xF) | ((qh[32 * n + l] & 3) << 4)) - 32);
                    a[128 * n + l + 32] = (int8_t)(((ql[64 * n + l + 32] & 0xF) | (((qh[32 * n + l] >> 2) & 3) << 4)) - 32);
                    a[128 * n + l + 64] = (int8_t)(((ql[64 * n + l] >> 4) | (((qh[32 * n + l] >> 4) & 3) << 4)) - 32);
                    a[128 * n + l + 96] = (int8_t)(((ql[64 * n + l + 32] >> 4) | (((qh[32 * n + l] >> 6) & 3) << 4)) - 32);
                }
        }
    }
}

/* The integer parts of the vec_dot products below are exact, so they are
 * computed with AVX2 integer vectors in whatever order is fast; only the
 * float steps follow candle's order. lane8(q, a, n) returns, for l = 0..7,
 * the sum over the n / 8 groups g of q[8g + l] * a[8g + l] (n = 16 or 32):
 * candle's per-lane aux16 / aux32 partial for one sub-block. */
static inline __m256i lane8_16(const int8_t* q, const int8_t* a) {
    const __m256i p = _mm256_mullo_epi16(_mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i*)q)),
                                         _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i*)a)));
    return _mm256_add_epi32(_mm256_cvtepi16_epi32(_mm256_castsi256_si128(p)),
                            _mm256_cvtepi16_epi32(_mm256_extracti128_si256(p, 1)));
}
static inline __m256i lane8_32(const int8_t* q, const int8_t* a) {
    const __m256i p = _mm256_add_epi16(
        _mm256_mullo_epi16(_mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i*)q)),
                           _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i*)a))),
        _mm256_mullo_epi16(_mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i*)(q + 16))),
                           _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i*)(a + 16)))));
    return _mm256_add_epi32(_mm256_cvtepi16_epi32(_mm256_castsi256_si128(p)),
                            _mm256_cvtepi16_epi32(_mm256_extracti128_si256(p, 1)));
}
static inline void store8(__m256i v, int32_t* o) { _mm256_storeu_si256((__m256i*)o, v); }

/* vec_dot_unopt of a Q8_0 weight row with a Q8_0 activation row:
 * sumf += (float)isum * d_w * d_x, block by block */
static float vd_q8_0(const wrow_t* w, const uint8_t* xq, const float* xd, int64_t K) {
    float sumf = 0.0f;
    for (int64_t b = 0; b < K / 32; b++) {
        int32_t t[8];
        store8(lane8_32((const int8_t*)(xq + 34 * b + 2), w->a + 32 * b), t);
        const int32_t s = t[0] + t[1] + t[2] + t[3] + t[4] + t[5] + t[6] + t[7];
        sumf += (float)s * w->d[b] * xd[b];
    }
    return sumf;
}

/* vec_dot_unopt Q4_K x Q8_K: per superblock, 8 lane sums
 * aux32[l] = sum_j scale_j sum_g q8 a (lane l of each 8-group of sub-block j),
 * sums[l] += (d_w d_x) aux32[l]; sumf -= (dmin_w d_x) sum_j bsums_j min_{j/2};
 * result sumf + sum_l sums[l] */
static float vd_q4_k(const wrow_t* w, const q8k_t* xq, int64_t K) {
    float sums[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    float sumf = 0.0f;
    for (int64_t b = 0; b < K / 256; b++) {
        const q8k_t* y = xq + b;
        const int8_t* a = w->a + 256 * b;
        __m256i aux = _mm256_setzero_si256();
        int32_t sumi = 0;
        for (int j = 0; j < 16; j++) sumi += (int32_t)y->bsums[j] * w->mn[8 * b + j / 2];
        for (int j = 0; j < 8; j++)
            aux = _mm256_add_epi32(aux, _mm256_mullo_epi32(_mm256_set1_epi32(w->sc[8 * b + j]),
                                                           lane8_32(y->qs + 32 * j, a + 32 * j)));
        int32_t a32[8];
        store8(aux, a32);
        const float d = w->d[b] * y->d;
        for (int l = 0; l < 8; l++) sums[l] += d * (float)a32[l];
        const float dmin = w->dmin[b] * y->d;
        sumf -= dmin * (float)sumi;
    }
    float s = -0.0f;
    for (int l = 0; l < 8; l++) s += sums[l];
    return sumf + s;
}

/* vec_dot_unopt Q6_K x Q8_K: per superblock, aux32[l] = sum_j scale_j sum_g q8 a
 * over the sixteen 16-element groups, sums[l] += aux32[l] d; result
 * sum_l sums[l]. candle accumulates aux32 in f32: every partial sum is an
 * integer of magnitude at most 2^24 (32 terms of at most 128 * 128 * 32), so
 * the int32 sums converted once are the same values. */
static float vd_q6_k(const wrow_t* w, const q8k_t* xq, int64_t K) {
    float sums[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int64_t b = 0; b < K / 256; b++) {
        const q8k_t* y = xq + b;
        const int8_t* a = w->a + 256 * b;
        __m256i aux = _mm256_setzero_si256();
        for (int j = 0; j < 16; j++)
            aux = _mm256_add_epi32(aux, _mm256_mullo_epi32(_mm256_set1_epi32(w->sc[16 * b + j]),
                                                           lane8_16(y->qs + 16 * j, a + 16 * j)));
        int32_t a32[8];
        store8(aux, a32);
        const float d = w->d[b] * y->d;
        for (int l = 0; l < 8; l++) sums[l] += (float)a32[l] * d;
    }
    float s = -0.0f;
    for (int l = 0; l < 8; l++) s += sums[l];
    return s;
}

/* f32 fmaf chain over k */
static float dot_chain(const float* a, const float* b, int64_t K) {
    float s = 0.0f;
    for (int64_t k = 0; k < K; k++) s = fmaf(a[k], b[k], s);
    return s;
}

/* out[r] = dot_chain(X row r, w) for 8 rows at once: the rows' chains run side
 * by side in the 8 lanes of one vector (each lane the same sequential fmaf
 * chain); xt holds the 8 rows transposed, xt[k][r] */
typedef float v8f __attribute__((vector_size(32)));
static void dot_chain8(const float* xt, const float* w, int64_t K, float* out) {
    v8f acc = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int64_t k = 0; k < K; k++) {
        v8f xv;
        memcpy(&xv, xt + 8 * k, sizeof xv);
        const v8f wv = {w[k], w[k], w[k], w[k], w[k], w[k], w[k], w[k]};
        for (int l = 0; l < 8; l++) acc[l] = fmaf(xv[l], wv[l], acc[l]);
    }
    memcpy(out, &acc, sizeof acc);
}

/* MaybeQuantLinear::forward over m rows: out[m][N] = X[m][K] . W[N][K]^T. The
 * arm follows marm, the rows of the reference's call (tp_linear.rs:107-109;
 * QUANT_PREFILL_M_THRESHOLD = 64, tp_linear.rs:96): a caller that evaluates
 * only some rows of a call passes the call's full row count (every arm
 * computes each row independently). */
static void qlinear(int dt, const void* W, int64_t N, int64_t K, const float* X, int64_t m, int64_t marm, float* out,
                    int nthreads) {
    const int64_t rb = hxo_row_bytes(dt, K);
    const int quant = dt == HXO_Q8_0 || dt == HXO_Q4_K || dt == HXO_Q6_K;
    if (!quant || marm > 64) {
        /* plain f32 Linear, or forward_via_f16: f16 weights and x, f16 output */
        const int f16 = quant;
        float* xr = (float*)malloc(sizeof(float) * m * K);
        for (int64_t i = 0; i < m * K; i++) xr[i] = f16 ? hxo_f16_to_f32(hxo_f32_to_f16(X[i])) : X[i];
        /* rows in blocks of 8, transposed: xt[blk][k][8] (padding rows zero) */
        const int64_t nblk = (m + 7) / 8;
        float* xt = (float*)calloc((size_t)(nblk * K * 8), sizeof(float));
        for (int64_t r = 0; r < m; r++)
            for (int64_t k = 0; k < K; k++) xt[((r / 8) * K + k) * 8 + (r % 8)] = xr[r * K + k];
#ifdef _OPENMP
#pragma omp parallel num_threads(nthreads)
#endif
        {
            float* wr = (float*)malloc(sizeof(float) * K);
            float o8[8];
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
            for (int64_t n = 0; n < N; n++) {
                hxo_dequant(dt, (const uint8_t*)W + n * rb, K, wr);
                if (f16)
                    for (int64_t k = 0; k < K; k++) wr[k] = hxo_f16_to_f32(hxo_f32_to_f16(wr[k]));
                for (int64_t b = 0; b < nblk; b++) {
                    dot_chain8(xt + b * K * 8, wr, K, o8);
                    for (int64_t r = 8 * b; r < m && r < 8 * b + 8; r++) {
                        const float v = o8[r - 8 * b];
                        out[r * N + n] = f16 ? hxo_f16_to_f32(hxo_f32_to_f16(v)) : v;
                    }
                }
            }
            free(wr);
        }
        free(xt);
        free(xr);
        return;
    }
    /* GGUF vec_dot: activations quantised per row to the vec_dot type */
    const int64_t nsb = K / 256, nb = K / 32;
    uint8_t* xq8 = NULL;
    float* xd8 = NULL;   /* the Q8_0 activation blocks' d as f32 */
    q8k_t* xqk = NULL;
    if (dt == HXO_Q8_0) {
        xq8 = (uint8_t*)malloc((size_t)(m * nb * 34));
        xd8 = (float*)malloc(sizeof(float) * (size_t)(m * nb));
        for (int64_t r = 0; r < m; r++)
            for (int64_t b = 0; b < nb; b++) {
                qz_q8_0(X + r * K + 32 * b, xq8 + (r * nb + b) * 34);
                xd8[r * nb + b] = ld_f16(xq8 + (r * nb + b) * 34);
            }
    } else {
        xqk = (q8k_t*)malloc(sizeof(q8k_t) * (size_t)(m * nsb));
        for (int64_t r = 0; r < m; r++)
            for (int64_t b = 0; b < nsb; b++) quant_q8_k(X + r * K + 256 * b, xqk + r * nsb + b);
    }
#ifdef _OPENMP
#pragma omp parallel num_threads(nthreads)
#endif
    {
        wrow_t w;
        w.a = (int8_t*)malloc((size_t)K);
        w.d = (float*)malloc(sizeof(float) * (size_t)nb);
        w.dmin = (float*)malloc(sizeof(float) * (size_t)(nsb + 1));
        w.sc = (int32_t*)malloc(sizeof(int32_t) * (size_t)(16 * nsb + 1));
        w.mn = (int32_t*)malloc(sizeof(int32_t) * (size_t)(8 * nsb + 1));
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
        for (int64_t n = 0; n < N; n++) {
            decode_row(dt, (const uint8_t*)W + n * rb, K, &w);
            for (int64_t r = 0; r < m; r++) {
                float v;
                if (dt == HXO_Q8_0) v = vd_q8_0(&w, xq8 + r * nb * 34, xd8 + r * nb, K);
                else if (dt == HXO_Q4_K) v = vd_q4_k(&w, xqk + r * nsb, K);
                else v = vd_q6_k(&w, xqk + r * nsb, K);
                out[r * N + n] = v;
            }
        }
        free(w.a); free(w.d); free(w.dmin); free(w.sc); free(w.mn);
    }
    free(xq8);
    free(xd8);
    free(xqk);
}

/* test hook: one MaybeQuantLinear call (m rows) */
int hxo_qlinear(int dt, const void* W, int64_t N, int64_t K, const float* X, int64_t m, float* out, int nthreads) {
    if (hxo_row_bytes(dt, K) < 0 || N <= 0 || m < 0) return 1;
#ifdef _OPENMP
    if (nthreads <= 0) nthreads = omp_get_max_threads();
#endif
    qlinear(dt, W, N, K, X, m, m, out, nthreads);
    return 0;
}

/* TpExpert::forward_partial at world size 1 over m rows of xf (gathered):
 * out[m][H] = down(silu(gate x) * up x) */
static void candle_expert(int gdt, const void* g, int udt, const void* u, int ddt, const void* d, int64_t H,
                          int64_t I, const float* X, int64_t m, int64_t marm, float* out, float* gbuf, float* ubuf,
                          int nthreads) {
    qlinear(gdt, g, I, H, X, m, marm, gbuf, nthreads);
    qlinear(udt, u, I, H, X, m, marm, ubuf, nthreads);
    for (int64_t i = 0; i < m * I; i++) {
        const float v = gbuf[i];
        gbuf[i] = (v / (1.0f + expf(-v))) * ubuf[i];
    }
    qlinear(ddt, d, H, I, gbuf, m, marm, out, nthreads);
}

static int forward_candle_impl(const hxo_moe* m, const void* x, int64_t T, const float* bias, const int32_t* sel,
                               int64_t nsel, float* y, int nthreads);

int hxo_moe_forward_candle(const hxo_moe* m, const void* x, int64_t T, const float* bias, float* y, int nthreads) {
    return forward_candle_impl(m, x, T, bias, NULL, 0, y, nthreads);
}

/* the outputs of the distinct tokens sel[0 .. nsel) of a forward of all T tokens, in
 * candle arithmetic: every expert call takes the arm of its full row count,
 * and only the selected tokens' rows are computed (y: [nsel][H]) */
int hxo_moe_forward_candle_sel(const hxo_moe* m, const void* x, int64_t T, const float* bias, const int32_t* sel,
                               int64_t nsel, float* y, int nthreads) {
    if (!sel || nsel <= 0) return 1;
    for (int64_t i = 0; i < nsel; i++) {   /* distinct tokens in [0, T) */
        if (sel[i] < 0 || sel[i] >= T) return 1;
        for (int64_t j = 0; j < i; j++)
            if (sel[j] == sel[i]) return 1;
    }
    return forward_candle_impl(m, x, T, bias, sel, nsel, y, nthreads);
}

static int forward_candle_impl(const hxo_moe* m, const void* x, int64_t T, const float* bias, const int32_t* sel,
                               int64_t nsel, float* y, int nthreads) {
    int64_t H = m->hidden, E = m->num_experts, I = m->inter, Is = m->shared_inter;
    int k = m->top_k;
    if (hxo_row_bytes(m->gate_dtype, H) < 0 || hxo_row_bytes(m->up_dtype, H) < 0 ||
        hxo_row_bytes(m->down_dtype, I) < 0)
        return 1;
    if (Is > 0 && (hxo_row_bytes(m->sgate_dtype, H) < 0 || hxo_row_bytes(m->sup_dtype, H) < 0 ||
                   hxo_row_bytes(m->sdown_dtype, Is) < 0 || !m->seg))
        return 1;
#ifdef _OPENMP
    if (nthreads <= 0) nthreads = omp_get_max_threads();
#else
    nthreads = 1;
#endif
    const int64_t F = T * k, KM = I > Is ? I : Is, R = T > F ? T : F, ny = sel ? nsel : T;
    int32_t* idx = (int32_t*)malloc(sizeof(int32_t) * F);
    float* w = (float*)malloc(sizeof(float) * F);
    int32_t* perm = (int32_t*)malloc(sizeof(int32_t) * F);
    int32_t* offs = (int32_t*)malloc(sizeof(int32_t) * (E + 1));
    int64_t* yrow = (int64_t*)malloc(sizeof(int64_t) * T);   /* output row of token t, or -1 */
    int32_t* rows = (int32_t*)malloc(sizeof(int32_t) * R);   /* the computed rows of a call */
    float* xf = (float*)malloc(sizeof(float) * T * H);
    float* xg = (float*)malloc(sizeof(float) * R * H);
    float* og = (float*)malloc(sizeof(float) * R * H);
    float* gbuf = (float*)malloc(sizeof(float) * R * KM);
    float* ubuf = (float*)malloc(sizeof(float) * R * KM);
    int rc = 0;
    if (!idx || !w || !perm || !offs || !yrow || !rows || !xf || !xg || !og || !gbuf || !ubuf) { rc = 2; goto done; }
    rc = hxo_route(m, x, T, bias, NULL, NULL, idx, w);
    if (rc) goto done;
    rc = hxo_dispatch(idx, T, k, E, perm, offs, NULL);
    if (rc) goto done;
    for (int64_t t = 0; t < T; t++) yrow[t] = sel ? -1 : t;
    if (sel)
        for (int64_t i = 0; i < nsel; i++) yrow[sel[i]] = i;
    for (int64_t i = 0; i < T * H; i++) xf[i] = ld_act(m->act_dtype, x, i);
    for (int64_t i = 0; i < ny * H; i++) y[i] = 0.0f;
    {
        const int64_t gb = hxo_row_bytes(m->gate_dtype, H) * I, ub = hxo_row_bytes(m->up_dtype, H) * I;
        const int64_t db = hxo_row_bytes(m->down_dtype, I) * H;
        for (int64_t e = 0; e < E; e++) {
            const int64_t n = offs[e + 1] - offs[e];
            int64_t nc = 0;   /* rows of the call computed here (all, or those of selected tokens) */
            for (int64_t p = 0; p < n; p++)
                if (yrow[perm[offs[e] + p] / k] >= 0) rows[nc++] = perm[offs[e] + p];
            if (nc == 0) continue;
            for (int64_t p = 0; p < nc; p++) memcpy(xg + p * H, xf + (int64_t)(rows[p] / k) * H, sizeof(float) * H);
            candle_expert(m->gate_dtype, (const uint8_t*)m->gate + e * gb, m->up_dtype, (const uint8_t*)m->up + e * ub,
                          m->down_dtype, (const uint8_t*)m->down + e * db, H, I, xg, nc, n, og, gbuf, ubuf, nthreads);
            for (int64_t p = 0; p < nc; p++) {
                const int32_t f = rows[p];
                float* yt = y + yrow[f / k] * H;
                for (int64_t h = 0; h < H; h++) yt[h] = yt[h] + og[p * H + h] * w[f];
            }
        }
    }
    if (Is > 0) {
        float* wr = (float*)malloc(sizeof(float) * H);
        hxo_dequant(m->seg_dtype, m->seg, H, wr);
        for (int64_t t = 0; t < T; t++)
            if (yrow[t] >= 0) memcpy(xg + yrow[t] * H, xf + t * H, sizeof(float) * H);
        candle_expert(m->sgate_dtype, m->sgate, m->sup_dtype, m->sup, m->sdown_dtype, m->sdown, H, Is, xg, ny, T, og,
                      gbuf, ubuf, nthreads);
        for (int64_t t = 0; t < T; t++) {
            const int64_t r = yrow[t];
            if (r < 0) continue;
            const float mix = 1.0f / (1.0f + expf(-dot_chain(xf + t * H, wr, H)));
            for (int64_t h = 0; h < H; h++) y[r * H + h] = y[r * H + h] + og[r * H + h] * mix;
        }
        free(wr);
    }
done:
    free(idx); free(w); free(perm); free(offs); free(yrow); free(rows); free(xf); free(xg); free(og); free(gbuf);
    free(ubuf);
    return rc;
}
