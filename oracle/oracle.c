/*
 * CPU ORACLE -- test infrastructure only (see oracle.h).  Nothing in the
 * product links or loads this file.
 *
 * Reference anchors (paths relative to the reference checkout):
 *   - op list and decode order: docs/BLOCKS.md, k0/compile_schedule.py:358-703
 *   - GDN math: k0/ops/gdn.cuh:66-383, docs/SEMANTICS.md:280-304
 *   - attention math: k0/ops/attn.cuh:109-488, tests/test_attn.cu:388-424
 *   - RMSNorm / glue: k0/ops/glue.cuh:25-152
 *   - argmax: k0/harness.cpp:1187-1195
 * The quantised block formats (Q8_0, Q4_K, Q6_K, Q8_K) and the activation
 * quantisers are ggml's public GGUF formats; ggml itself is not in the
 * reference (it is the un-vendored llama.cpp fork autoround @546eca8dc,
 * ggml 0.12.0), so these are restated from the published layouts.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------ conversions */

float or_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1f, man = h & 0x3ff, bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: value = man * 2^-24 */
            float v = (float)man * 5.9604644775390625e-8f;
            memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* IEEE binary32 -> binary16, round to nearest even (what F16C/`__float2half`
 * compute). */
uint16_t or_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000);
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) /* inf / nan */
        return sign | 0x7c00 | (ax > 0x7f800000u ? 0x200 : 0);
    if (ax >= 0x477ff000u) /* rounds to >= 65520 -> inf */
        return sign | 0x7c00;
    if (ax < 0x38800000u) { /* result is subnormal or zero: value/2^-24 */
        float a;
        memcpy(&a, &ax, 4);
        /* a * 2^24 is exact in fp32 range; nearbyintf rounds half-even */
        const float m = nearbyintf(a * 16777216.0f);
        return sign | (uint16_t)m;
    }
    /* normal: keep 10 mantissa bits, round half to even on the dropped 13 */
    uint32_t mant = ax + 0xfffu + ((ax >> 13) & 1u);
    return sign | (uint16_t)((mant - 0x38000000u) >> 13);
}

float or_bf16_to_f32(uint16_t h) {
    uint32_t b = (uint32_t)h << 16;
    float f;
    memcpy(&f, &b, 4);
    return f;
}

/* ggml GGML_FP32_TO_BF16: nan -> quiet nan, otherwise round half to even */
uint16_t or_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u)
        return (uint16_t)((u >> 16) | 64);
    return (uint16_t)((u + (0x7fffu + ((u >> 16) & 1u))) >> 16);
}

/* ggml nearest_int: the 1.5*2^23 magic-number round (half to even) */
int or_nearest_int(float fval) {
    float val = fval + 12582912.f;
    int i;
    memcpy(&i, &val, sizeof(int));
    return (i & 0x007fffff) - 0x00400000;
}

/* ------------------------------------------------------------ formats */

typedef struct { uint16_t d; int8_t qs[32]; } blk_q8_0;                          /* 34 B */
typedef struct { uint16_t d, dmin; uint8_t scales[12]; uint8_t qs[128]; } blk_q4_K; /* 144 B */
typedef struct { uint8_t ql[128]; uint8_t qh[64]; int8_t scales[16]; uint16_t d; } blk_q6_K; /* 210 B */
typedef struct { float d; int8_t qs[256]; int16_t bsums[16]; } blk_q8_K;          /* 292 B */

size_t or_type_block_elems(int t) {
    switch (t) {
    case OR_Q8_0: return 32;
    case OR_Q4_K: case OR_Q6_K: case OR_Q8_K: return 256;
    default: return 1;
    }
}

size_t or_type_block_bytes(int t) {
    switch (t) {
    case OR_F32: return 4;
    case OR_F16: case OR_BF16: return 2;
    case OR_Q8_0: return 34;
    case OR_Q4_K: return 144;
    case OR_Q6_K: return 210;
    case OR_Q8_K: return 292;
    default: return 0;
    }
}

size_t or_row_bytes(int t, int64_t k) {
    return (size_t)(k / (int64_t)or_type_block_elems(t)) * or_type_block_bytes(t);
}

/* Q4_K packed 6-bit scale/min pair j of 8 (ggml get_scale_min_k4) */
static void q4k_scale_min(int j, const uint8_t *q, int *sc, int *m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

/* Q4_K element e (0..255) code, 0..15: sub-block pair p = e/64 shares bytes
 * qs[32p .. 32p+32), low nibble for e%64 < 32, high nibble otherwise. */
static inline int q4k_code(const blk_q4_K *b, int e) {
    const int p = e >> 6, l = e & 31;
    const uint8_t byte = b->qs[32 * p + l];
    return (e & 32) ? (byte >> 4) : (byte & 0xF);
}

/* Q6_K element e code, -32..31: half n = e/128 uses ql[64n..], qh[32n..];
 * within a half, quarter t = (e%128)/32 selects {ql low, ql+32 low, ql high,
 * ql+32 high} and qh bit pair 2t. */
static inline int q6k_code(const blk_q6_K *b, int e) {
    const int n = e >> 7, r = e & 127, t = r >> 5, l = r & 31;
    const uint8_t *ql = b->ql + 64 * n, *qh = b->qh + 32 * n;
    const uint8_t lo = (t & 1) ? ql[l + 32] : ql[l];
    const int nib = (t & 2) ? (lo >> 4) : (lo & 0xF);
    const int hi = (qh[l] >> (2 * t)) & 3;
    return (nib | (hi << 4)) - 32;
}

void or_dequant_row(int t, const void *row, float *out, int64_t k) {
    if (t == OR_F32) { memcpy(out, row, (size_t)k * 4); return; }
    if (t == OR_F16) { for (int64_t i = 0; i < k; i++) out[i] = or_f16_to_f32(((const uint16_t *)row)[i]); return; }
    if (t == OR_BF16) { for (int64_t i = 0; i < k; i++) out[i] = or_bf16_to_f32(((const uint16_t *)row)[i]); return; }
    const int64_t nb = k / (int64_t)or_type_block_elems(t);
    for (int64_t ib = 0; ib < nb; ib++) {
        if (t == OR_Q8_0) {
            const blk_q8_0 *b = (const blk_q8_0 *)row + ib;
            const float d = or_f16_to_f32(b->d);
            for (int l = 0; l < 32; l++) out[ib * 32 + l] = d * (float)b->qs[l];
        } else if (t == OR_Q4_K) {
            /* ggml dequantize_row_q4_K: y = (d*sc)*q - (dmin*m), fp32 */
            const blk_q4_K *b = (const blk_q4_K *)row + ib;
            const float d = or_f16_to_f32(b->d), dmin = or_f16_to_f32(b->dmin);
            for (int s = 0; s < 8; s++) {
                int sc, m;
                q4k_scale_min(s, b->scales, &sc, &m);
                const float d1 = d * (float)sc, m1 = dmin * (float)m;
                for (int l = 0; l < 32; l++)
                    out[ib * 256 + 32 * s + l] = d1 * (float)q4k_code(b, 32 * s + l) - m1;
            }
        } else if (t == OR_Q6_K) {
            /* ggml dequantize_row_q6_K: y = d * sc * q, fp32 left to right */
            const blk_q6_K *b = (const blk_q6_K *)row + ib;
            const float d = or_f16_to_f32(b->d);
            for (int e = 0; e < 256; e++)
                out[ib * 256 + e] = d * (float)b->scales[e / 16] * (float)q6k_code(b, e);
        } else if (t == OR_Q8_K) {
            const blk_q8_K *b = (const blk_q8_K *)row + ib;
            for (int e = 0; e < 256; e++) out[ib * 256 + e] = b->d * (float)b->qs[e];
        }
    }
}

/* ------------------------------------------------------------ activation quant */

/* ggml-cpu x86 quantize_row_q8_0 (AVX2 branch): d = amax/127 stored as f16;
 * id = 127/amax (0 if amax == 0); q = round-half-even(x*id). */
void or_quant_q8_0(const float *x, void *vy, int64_t k) {
    blk_q8_0 *y = (blk_q8_0 *)vy;
    for (int64_t ib = 0; ib < k / 32; ib++) {
        const float *xb = x + ib * 32;
        float amax = 0.0f;
        for (int l = 0; l < 32; l++) amax = fmaxf(amax, fabsf(xb[l]));
        const float d = amax / 127.f;
        y[ib].d = or_f32_to_f16(d);
        const float id = (amax != 0.0f) ? 127.f / amax : 0.0f;
        for (int l = 0; l < 32; l++) y[ib].qs[l] = (int8_t)or_nearest_int(xb[l] * id);
    }
}

/* ggml quantize_row_q8_0_ref (ggml-quants.c), the form the KV-cache copy
 * kernels use too: d = amax/127 (f16), id = d ? 1/d : 0, q = roundf(x*id)
 * (half away from zero). */
void or_quant_q8_0_ref(const float *x, void *vy, int64_t k) {
    blk_q8_0 *y = (blk_q8_0 *)vy;
    for (int64_t ib = 0; ib < k / 32; ib++) {
        const float *xb = x + ib * 32;
        float amax = 0.0f;
        for (int l = 0; l < 32; l++) amax = fmaxf(amax, fabsf(xb[l]));
        const float d = amax / 127.f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        y[ib].d = or_f32_to_f16(d);
        for (int l = 0; l < 32; l++) y[ib].qs[l] = (int8_t)roundf(xb[l] * id);
    }
}

/* ggml quantize_row_q8_K_ref: max = signed element of largest |x| (first
 * wins); iscale = -127/max; q = min(127, nearest_int(iscale*x)); bsums over
 * 16; d = 1/iscale. */
void or_quant_q8_K(const float *x, void *vy, int64_t k) {
    blk_q8_K *y = (blk_q8_K *)vy;
    for (int64_t ib = 0; ib < k / 256; ib++) {
        const float *xb = x + ib * 256;
        float max = 0, amax = 0;
        for (int j = 0; j < 256; j++) {
            const float ax = fabsf(xb[j]);
            if (ax > amax) { amax = ax; max = xb[j]; }
        }
        if (amax == 0.0f) {
            y[ib].d = 0;
            memset(y[ib].qs, 0, 256);
            memset(y[ib].bsums, 0, sizeof(y[ib].bsums));
            continue;
        }
        const float iscale = -127.f / max;
        for (int j = 0; j < 256; j++) {
            const int v = or_nearest_int(iscale * xb[j]);
            y[ib].qs[j] = (int8_t)(v < 127 ? v : 127);
        }
        for (int j = 0; j < 16; j++) {
            int s = 0;
            for (int i = 0; i < 16; i++) s += y[ib].qs[16 * j + i];
            y[ib].bsums[j] = (int16_t)s;
        }
        y[ib].d = 1 / iscale;
    }
}

void or_quant_bf16(const float *x, uint16_t *y, int64_t k) {
    for (int64_t i = 0; i < k; i++) y[i] = or_f32_to_bf16(x[i]);
}

/* ------------------------------------------------------------ block terms */

double or_block_term(int t, const void *wb, const void *xb) {
    if (t == OR_Q8_0) {
        const blk_q8_0 *w = (const blk_q8_0 *)wb, *x = (const blk_q8_0 *)xb;
        int32_t isum = 0;
        for (int l = 0; l < 32; l++) isum += (int32_t)w->qs[l] * (int32_t)x->qs[l];
        return ((double)or_f16_to_f32(w->d) * (double)or_f16_to_f32(x->d)) * (double)isum;
    }
    if (t == OR_Q4_K) {
        const blk_q4_K *w = (const blk_q4_K *)wb;
        const blk_q8_K *x = (const blk_q8_K *)xb;
        int64_t isum = 0, imin = 0;
        for (int s = 0; s < 8; s++) {
            int sc, m;
            q4k_scale_min(s, w->scales, &sc, &m);
            int32_t dot = 0;
            for (int l = 0; l < 32; l++) dot += q4k_code(w, 32 * s + l) * (int32_t)x->qs[32 * s + l];
            isum += (int64_t)sc * dot;
            imin += (int64_t)m * ((int32_t)x->bsums[2 * s] + (int32_t)x->bsums[2 * s + 1]);
        }
        const double dx = (double)x->d;
        return ((double)or_f16_to_f32(w->d) * dx) * (double)isum -
               ((double)or_f16_to_f32(w->dmin) * dx) * (double)imin;
    }
    if (t == OR_Q6_K) {
        const blk_q6_K *w = (const blk_q6_K *)wb;
        const blk_q8_K *x = (const blk_q8_K *)xb;
        int64_t isum = 0;
        for (int j = 0; j < 16; j++) {
            int32_t dot = 0;
            for (int l = 0; l < 16; l++) dot += q6k_code(w, 16 * j + l) * (int32_t)x->qs[16 * j + l];
            isum += (int64_t)w->scales[j] * dot;
        }
        return ((double)or_f16_to_f32(w->d) * (double)x->d) * (double)isum;
    }
    return 0.0;
}

static int vec_dot_type(int t) {
    switch (t) {
    case OR_Q8_0: return OR_Q8_0;
    case OR_Q4_K: case OR_Q6_K: return OR_Q8_K;
    case OR_BF16: return OR_BF16;
    default: return OR_F32;
    }
}

/* fast per-row kernels (same arithmetic as or_block_term, unrolled so the
 * full-model oracle runs in reasonable time): an AVX-512 copy and a baseline
 * copy of oracle_rows.inc, the one the CPU supports chosen at first use. */
#pragma GCC push_options
#pragma GCC target("avx512f,avx512bw,avx512vl,avx2,fma,bmi2")
#define ROWFN(name) name##_avx512
#include "oracle_rows.inc"
#undef ROWFN
#pragma GCC pop_options
#define ROWFN(name) name##_base
#include "oracle_rows.inc"
#undef ROWFN

static int use_avx512(void) {
    static int v = -1;
    if (v < 0) {
        __builtin_cpu_init();
        v = __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
            __builtin_cpu_supports("avx512vl");
    }
    return v;
}

int or_row_isa(void) { return use_avx512() ? 512 : 0; }

void or_gemv_q(int t, const void *w, int64_t rows, int64_t k, const void *xq, float *y) {
    const size_t rb = or_row_bytes(t, k);
    const int64_t nb = k / (int64_t)or_type_block_elems(t);
    const int v512 = use_avx512();
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; r++) {
        const void *row = (const char *)w + (size_t)r * rb;
        double acc = 0.0;
        switch (t) {
        case OR_Q4_K:
            acc = v512 ? row_q4k_avx512((const blk_q4_K *)row, (const blk_q8_K *)xq, nb)
                       : row_q4k_base((const blk_q4_K *)row, (const blk_q8_K *)xq, nb);
            break;
        case OR_Q6_K:
            acc = v512 ? row_q6k_avx512((const blk_q6_K *)row, (const blk_q8_K *)xq, nb)
                       : row_q6k_base((const blk_q6_K *)row, (const blk_q8_K *)xq, nb);
            break;
        case OR_Q8_0:
            acc = v512 ? row_q8_0_avx512((const blk_q8_0 *)row, (const blk_q8_0 *)xq, nb)
                       : row_q8_0_base((const blk_q8_0 *)row, (const blk_q8_0 *)xq, nb);
            break;
        case OR_BF16:
            acc = v512 ? row_bf16_avx512((const uint16_t *)row, (const uint16_t *)xq, k)
                       : row_bf16_base((const uint16_t *)row, (const uint16_t *)xq, k);
            break;
        case OR_F32: {
            const float *wf = (const float *)row, *xf = (const float *)xq;
            for (int64_t g = 0; g < k / 64; g++) {
                double part = 0.0;
                for (int64_t i = 64 * g; i < 64 * g + 64; i++) part += (double)wf[i] * (double)xf[i];
                acc += part;
            }
        } break;
        default: break;
        }
        y[r] = (float)acc;
    }
}

void or_gemv(int t, const void *w, int64_t rows, int64_t k, const float *x, float *y) {
    const int vt = vec_dot_type(t);
    void *xq = malloc(or_row_bytes(vt, k) + 64);
    switch (vt) {
    case OR_Q8_0: or_quant_q8_0(x, xq, k); break;
    case OR_Q8_K: or_quant_q8_K(x, xq, k); break;
    case OR_BF16: or_quant_bf16(x, (uint16_t *)xq, k); break;
    default: memcpy(xq, x, (size_t)k * 4); break;
    }
    or_gemv_q(t, w, rows, k, xq, y);
    free(xq);
}

/* ------------------------------------------------------------ norms, unary */

/* ggml CPU rms_norm: sum of fp32 squares in double; mean -> float;
 * scale = 1/sqrtf(mean+eps); y = x*scale; then the separate MUL by w
 * (reference k0/ops/glue.cuh:56-152 is the same operator). */
void or_rmsnorm(const float *x, const float *w, float *y, int64_t n, float eps) {
    double sum = 0.0;
    for (int64_t i = 0; i < n; i++) sum += (double)(x[i] * x[i]);
    const float mean = (float)(sum / (double)n);
    const float scale = 1.0f / sqrtf(mean + eps);
    for (int64_t i = 0; i < n; i++) {
        const float t = x[i] * scale;
        y[i] = w ? t * w[i] : t;
    }
}

/* ggml CPU l2_norm: scale = 1/fmaxf(sqrtf(sum), eps) over fp32 squares summed
 * in double (the CUDA form rsqrtf(fmaxf(sum, eps^2)) in k0/ops/gdn.cuh:187-212
 * is the same operator up to rounding). */
void or_l2norm(const float *x, float *y, int64_t n, float eps) {
    double sum = 0.0;
    for (int64_t i = 0; i < n; i++) sum += (double)(x[i] * x[i]);
    const float scale = 1.0f / fmaxf(sqrtf((float)sum), eps);
    for (int64_t i = 0; i < n; i++) y[i] = x[i] * scale;
}

float or_silu(float x) { return x / (1.0f + (float)exp(-(double)x)); }
float or_sigmoid(float x) { return 1.0f / (1.0f + (float)exp(-(double)x)); }
float or_softplus(float x) {
    if (x > 20.0f) return x;
    const float e = (float)exp((double)x);
    return (float)log((double)(1.0f + e));
}

/* ------------------------------------------------------------ gated DeltaNet */

/* k0/ops/gdn.cuh:106-171: window {h0,h1,h2,x}, tap-contiguous weights
 * w[c*dconv + j]; history <- {h1,h2,x}; y = silu(sum_j win_j*w_j) with the
 * sum in fp64 rounded once. */
void or_conv_silu(const float *xnew, float *st, const float *cw, float *out,
                  int64_t channels, int dconv) {
    const int nh = dconv - 1;
    for (int64_t c = 0; c < channels; c++) {
        float win[8];
        for (int j = 0; j < nh; j++) win[j] = st[c * nh + j];
        win[nh] = xnew[c];
        double acc = 0.0;
        for (int j = 0; j < dconv; j++) acc += (double)win[j] * (double)cw[c * dconv + j];
        out[c] = or_silu((float)acc);
        for (int j = 0; j < nh; j++) st[c * nh + j] = win[j + 1];
    }
}

/* k0/ops/gdn.cuh:215-245: g = exp(softplus(alpha + dt_bias) * a);
 * beta = sigmoid(beta_raw). */
void or_gdn_gates(const float *alpha, const float *beta_raw, const float *dt_bias,
                  const float *ssm_a, float *g, float *beta, int nh) {
    for (int h = 0; h < nh; h++) {
        const float sp = or_softplus(alpha[h] + dt_bias[h]);
        g[h] = (float)exp((double)(sp * ssm_a[h]));
        beta[h] = or_sigmoid(beta_raw[h]);
    }
}

/* k0/ops/gdn.cuh:248-337 (delta rule, modulo head map hk = h % HK), with
 * the declared fp32 folds of k0/ops/gdn.cuh:19-28 over the kernel's thread
 * layout (csrc/gdn.h): a state column's D rows split over tpc = 256 / cols
 * threads, thread t holding rows [t rpt, (t + 1) rpt), rpt = D / tpc:
 *   kv    = tree_t (sum_r S[t rpt + r][col] k[t rpt + r])   per-thread sums
 *           sequential fp32 (a rounded product, then a rounded add), closed
 *           by the butterfly a[t] += a[t ^ m], m = 1, 2, 4, ... (or_lanes_tree)
 *   delta = (v[col] - g*kv) * beta                            (fp32 ops)
 *   S'    = g*S + k*delta                                     (fp32: mul, mul, add)
 *   o     = tree_t (sum_r S'[..][col] q[..]) * scale          (same fold, scale last) */
static float or_lanes_tree(float *a, int n) {
    for (int m = 1; m < n; m <<= 1) {
        float b[64];
        for (int t = 0; t < n; t++) b[t] = a[t] + a[t ^ m];
        memcpy(a, b, sizeof(float) * (size_t)n);
    }
    return a[0];
}

void or_gdn_step(const float *q, const float *k, const float *v, const float *g,
                 const float *beta, float *state, float *o, int hv, int hk, int d,
                 float scale, int cols) {
    const int tpc = 256 / cols, rpt = d / tpc;
    for (int h = 0; h < hv; h++) {
        const int kh = h % hk;
        const float *qh = q + (size_t)kh * d, *kk = k + (size_t)kh * d;
        const float gv = g[h], bv = beta[h];
        for (int col = 0; col < d; col++) {
            float *s = state + ((size_t)h * d + col) * d;
            float part[64];
            for (int t = 0; t < tpc; t++) {
                float acc = 0.0f;
                for (int r = 0; r < rpt; r++) {
                    const float pr = s[t * rpt + r] * kk[t * rpt + r];
                    acc = acc + pr;
                }
                part[t] = acc;
            }
            const float kvf = or_lanes_tree(part, tpc);
            const float t1 = gv * kvf;
            const float t2 = v[(size_t)h * d + col] - t1;
            const float delta = t2 * bv;
            for (int i = 0; i < d; i++) {
                const float a = gv * s[i];
                const float b = kk[i] * delta;
                s[i] = a + b;
            }
            for (int t = 0; t < tpc; t++) {
                float acc = 0.0f;
                for (int r = 0; r < rpt; r++) {
                    const float pr = s[t * rpt + r] * qh[t * rpt + r];
                    acc = acc + pr;
                }
                part[t] = acc;
            }
            o[(size_t)h * d + col] = or_lanes_tree(part, tpc) * scale;
        }
    }
}

/* the GDN step's columns per workgroup item for a head size (csrc/model.cpp) */
int or_gdn_cols(int d) { return d >= 128 ? 32 : 16; }

/* k0/ops/gdn.cuh:339-383: per head rms_norm(x)*w, then * silu(z). */
void or_gated_rmsnorm(const float *x, const float *z, const float *w, float *y,
                      int nh, int d, float eps) {
    for (int h = 0; h < nh; h++) {
        or_rmsnorm(x + (size_t)h * d, w, y + (size_t)h * d, d, eps);
        for (int i = 0; i < d; i++) y[(size_t)h * d + i] *= or_silu(z[(size_t)h * d + i]);
    }
}

/* ------------------------------------------------------------ attention */

/* theta_scale = powf(base, -2/n_dims), correctly rounded (k0/ops/attn.cuh:63
 * pins 1e7 -> 0x1.356656p-1). */
float or_rope_theta_scale(float base, int n_dims) {
    return (float)pow((double)base, -2.0 / (double)n_dims);
}

/* ggml rope cache: theta_0 = pos, theta_{i+1} = theta_i * theta_scale (fp32);
 * NEOX pairs (i, i + n_dims/2) for i < n_dims/2; dims >= n_dims pass through.
 * IMROPE with sections [11,11,10,0] and four equal position ids is this same
 * operator (k0/ops/attn.cuh:135-175, docs/SEMANTICS.md:500-523). */
void or_rope_neox(float *x, int hd, int n_dims, int pos, float theta_scale) {
    (void)hd;
    float theta = (float)pos;
    const int half = n_dims / 2;
    for (int i = 0; i < half; i++) {
        const float c = (float)cos((double)theta), s = (float)sin((double)theta);
        const float x0 = x[i], x1 = x[i + half];
        x[i] = x0 * c - x1 * s;
        x[i + half] = x0 * s + x1 * c;
        theta *= theta_scale;
    }
}

/* Exact-arithmetic decode attention (tests/test_attn.cu:388-424 computes the
 * same thing in double): scores s_j = scale * q.k_j with exact fp64 products,
 * softmax and the V sum in fp64, rounded to fp32 once.  GQA: q head h reads
 * kv head h / (nq/nkv).  Caches are rows of row_width f16 (all kv heads of a
 * position contiguous). */
void or_attn_decode(const float *q, const uint16_t *kc, const uint16_t *vc, int n_kv,
                    int nq, int nkv, int hd, int row_width, float scale, float *out) {
    const int gqa = nq / nkv;
    /* heads are independent: one thread per head (results do not depend on
     * the thread count) */
#pragma omp parallel for schedule(static)
    for (int h = 0; h < nq; h++) {
        double *s = (double *)malloc(sizeof(double) * (size_t)(n_kv > 0 ? n_kv : 1));
        double *acc = (double *)malloc(sizeof(double) * (size_t)hd);
        const int g = h / gqa;
        const float *qh = q + (size_t)h * hd;
        double m = -INFINITY;
        for (int j = 0; j < n_kv; j++) {
            const uint16_t *kr = kc + (size_t)j * row_width + (size_t)g * hd;
            double dot = 0.0;
            for (int d = 0; d < hd; d++) dot += (double)qh[d] * (double)or_f16_to_f32(kr[d]);
            s[j] = dot * (double)scale;
            if (s[j] > m) m = s[j];
        }
        double sum = 0.0;
        for (int d = 0; d < hd; d++) acc[d] = 0.0;
        for (int j = 0; j < n_kv; j++) {
            const double p = exp(s[j] - m);
            sum += p;
            const uint16_t *vr = vc + (size_t)j * row_width + (size_t)g * hd;
            for (int d = 0; d < hd; d++) acc[d] += p * (double)or_f16_to_f32(vr[d]);
        }
        for (int d = 0; d < hd; d++) out[(size_t)h * hd + d] = (float)(acc[d] / sum);
        free(s);
        free(acc);
    }
}

/* element e of cache row j (row of row_elems elements) as f32: f16, or a
 * Q8_0 code times its block's f16 scale (exact in f32) */
static float kv_elem(const void *cache, int kv_type, size_t row_elems, int j, size_t e) {
    if (kv_type == OR_Q8_0) {
        const blk_q8_0 *b = (const blk_q8_0 *)cache + ((size_t)j * row_elems + e) / 32;
        return (float)b->qs[e % 32] * or_f16_to_f32(b->d);
    }
    return or_f16_to_f32(((const uint16_t *)cache)[(size_t)j * row_elems + e]);
}

/* or_attn_decode with the cache element type a parameter (same arithmetic) */
void or_attn_decode_kv(const float *q, const void *kc, const void *vc, int kv_type, int n_kv,
                       int nq, int nkv, int hd, float scale, float *out) {
    const int gqa = nq / nkv;
    const size_t rw = (size_t)nkv * hd;
#pragma omp parallel for schedule(static)
    for (int h = 0; h < nq; h++) {
        double *s = (double *)malloc(sizeof(double) * (size_t)(n_kv > 0 ? n_kv : 1));
        double *acc = (double *)malloc(sizeof(double) * (size_t)hd);
        const int g = h / gqa;
        const float *qh = q + (size_t)h * hd;
        double m = -INFINITY;
        for (int j = 0; j < n_kv; j++) {
            double dot = 0.0;
            for (int d = 0; d < hd; d++) dot += (double)qh[d] * (double)kv_elem(kc, kv_type, rw, j, (size_t)g * hd + d);
            s[j] = dot * (double)scale;
            if (s[j] > m) m = s[j];
        }
        double sum = 0.0;
        for (int d = 0; d < hd; d++) acc[d] = 0.0;
        for (int j = 0; j < n_kv; j++) {
            const double p = exp(s[j] - m);
            sum += p;
            for (int d = 0; d < hd; d++) acc[d] += p * (double)kv_elem(vc, kv_type, rw, j, (size_t)g * hd + d);
        }
        for (int d = 0; d < hd; d++) out[(size_t)h * hd + d] = (float)(acc[d] / sum);
        free(s);
        free(acc);
    }
}

/* Split-K decode attention in fp32, the folds the GPU's attention op declares
 * (sinter attention op; the reference's fp32 FATTN fold discipline,
 * k0/ops/attn.cuh:33-42, restated for 64-wide waves):
 *   chunks: T = ceil(n_kv/32) tiles, tpc = max(ceil(T/C), ceil(chunk_min/32))
 *           tiles per chunk, ceil(T/tpc) chunks;
 *   score:  32 lane partials, lane p chaining fmaf over dims 8p..8p+7,
 *           added by the tree of lane masks 16, 15, 7, 2, 1, times scale;
 *   groups: a tile's rows split by row mod 8; each group runs its own online
 *           softmax per q head over its rows of the chunk's tiles:
 *           m' = max(m, the group's tile max); w = exp(s - m'), corr =
 *           exp(m - m') (0 before the group's first row, 1 if m is unchanged)
 *           in fp64 rounded to fp32; sum = (w0 + w1) + (w2 + w3) over the
 *           group's 4 tile rows (0 past n_kv); l = l*corr + sum;
 *           acc = acc*corr, then fmaf(w, v, acc) over the group's rows ascending;
 *   chunk:  M = max m_g, e_g = exp(m_g - M) (0 for an empty group), L and O
 *           fmaf chains over the groups ascending;
 *   merge:  M = max m_c, e_c = exp(m_c - M); L, O fmaf chains over chunks
 *           ascending; out = O / L (the un-gated attention).
 * Rows past n_kv contribute nothing. */
static float or_tree32(const float *v, const int masks[5]) {
    float a[32], b[32];
    memcpy(a, v, sizeof a);
    for (int lv = 0; lv < 5; lv++) {
        for (int p = 0; p < 32; p++) b[p] = a[p] + a[p ^ masks[lv]];
        memcpy(a, b, sizeof a);
    }
    return a[0];
}

static const int OR_ATT_SCORE_MASKS[5] = {16, 15, 7, 2, 1};

static float or_attn_exp(float x) { return (float)exp((double)x); }

/* one (kv head, chunk) item: acc[gqa][hd], m[gqa], l[gqa] */
static inline __attribute__((always_inline)) void or_attn_chunk_body(
        const float *q, const void *kc, const void *vc, int kv_type, int g, int gqa, int nkv, int hd,
        int kv0, int kv1, float scale, float *acc, float *mo, float *lo) {
    const size_t rw = (size_t)nkv * hd;
    float accr[8][8][256];
    float mrun[8][8], lrun[8][8];
    float kr[32][256], vr[32][256];
    for (int gr = 0; gr < 8; gr++)
        for (int s = 0; s < gqa; s++) { mrun[gr][s] = -INFINITY; lrun[gr][s] = 0.0f; }
    memset(accr, 0, sizeof accr);
    for (int t0 = kv0; t0 < kv1; t0 += 32) {
        const int nr = kv1 - t0 < 32 ? kv1 - t0 : 32;
        for (int r = 0; r < nr; r++)
            for (int d = 0; d < hd; d++) {
                kr[r][d] = kv_elem(kc, kv_type, rw, t0 + r, (size_t)g * hd + d);
                vr[r][d] = kv_elem(vc, kv_type, rw, t0 + r, (size_t)g * hd + d);
            }
        for (int s = 0; s < gqa; s++) {
            const float *qs = q + (size_t)(g * gqa + s) * hd;
            float sc[32];
            for (int r = 0; r < nr; r++) {
                float part[32];
                for (int p = 0; p < 32; p++) {
                    float a = 0.0f;
                    for (int d = 8 * p; d < 8 * p + 8; d++) a = fmaf(qs[d], kr[r][d], a);
                    part[p] = a;
                }
                sc[r] = or_tree32(part, OR_ATT_SCORE_MASKS) * scale;
            }
            for (int gr = 0; gr < 8; gr++) {
                float mt = -INFINITY, w[4];
                for (int i = 0; i < 4; i++)
                    if (gr + 8 * i < nr) mt = fmaxf(mt, sc[gr + 8 * i]);
                const float m0 = mrun[gr][s], mn = fmaxf(m0, mt);
                for (int i = 0; i < 4; i++) w[i] = gr + 8 * i < nr ? or_attn_exp(sc[gr + 8 * i] - mn) : 0.0f;
                const float ws = (w[0] + w[1]) + (w[2] + w[3]);
                const float cf = m0 == -INFINITY ? 0.0f : (m0 == mn ? 1.0f : or_attn_exp(m0 - mn));
                const float lc = lrun[gr][s] * cf;
                lrun[gr][s] = lc + ws;
                mrun[gr][s] = mn;
                for (int d = 0; d < hd; d++) accr[gr][s][d] = accr[gr][s][d] * cf;
                for (int i = 0; i < 4; i++)
                    if (gr + 8 * i < nr)
                        for (int d = 0; d < hd; d++) accr[gr][s][d] = fmaf(w[i], vr[gr + 8 * i][d], accr[gr][s][d]);
            }
        }
    }
    for (int s = 0; s < gqa; s++) {
        float M = -INFINITY, e[8], L = 0.0f;
        for (int gr = 0; gr < 8; gr++) M = fmaxf(M, mrun[gr][s]);
        for (int gr = 0; gr < 8; gr++) {
            e[gr] = mrun[gr][s] == -INFINITY ? 0.0f : or_attn_exp(mrun[gr][s] - M);
            L = fmaf(e[gr], lrun[gr][s], L);
        }
        for (int d = 0; d < hd; d++) {
            float o = 0.0f;
            for (int gr = 0; gr < 8; gr++) o = fmaf(e[gr], accr[gr][s][d], o);
            acc[(size_t)s * hd + d] = o;
        }
        mo[s] = M;
        lo[s] = L;
    }
}

__attribute__((target("avx2,fma"))) static void or_attn_chunk_fma(
        const float *q, const void *kc, const void *vc, int kv_type, int g, int gqa, int nkv, int hd,
        int kv0, int kv1, float scale, float *acc, float *mo, float *lo) {
    or_attn_chunk_body(q, kc, vc, kv_type, g, gqa, nkv, hd, kv0, kv1, scale, acc, mo, lo);
}
static void or_attn_chunk_base(
        const float *q, const void *kc, const void *vc, int kv_type, int g, int gqa, int nkv, int hd,
        int kv0, int kv1, float scale, float *acc, float *mo, float *lo) {
    or_attn_chunk_body(q, kc, vc, kv_type, g, gqa, nkv, hd, kv0, kv1, scale, acc, mo, lo);
}

void or_attn_geom(int n_kv, int n_chunks, int chunk_min, int *tiles, int *tpc, int *nch) {
    const int T = (n_kv + 31) / 32;
    const int a = (T + n_chunks - 1) / n_chunks, b = (chunk_min + 31) / 32;
    int t = a > b ? a : b;
    if (t < 1) t = 1;
    *tiles = T;
    *tpc = t;
    *nch = (T + t - 1) / t;
}

void or_attn_split(const float *q, const void *kc, const void *vc, int kv_type, int n_kv, int nq, int nkv,
                   int hd, float scale, int n_chunks, int chunk_min, float *out) {
    const int gqa = nq / nkv;
    int T, tpc, NC;
    or_attn_geom(n_kv, n_chunks, chunk_min, &T, &tpc, &NC);
    (void)T;
    float *acc = (float *)malloc(sizeof(float) * (size_t)nkv * NC * gqa * hd);
    float *m = (float *)malloc(sizeof(float) * (size_t)nkv * NC * gqa);
    float *l = (float *)malloc(sizeof(float) * (size_t)nkv * NC * gqa);
    const int fma_ok = __builtin_cpu_supports("fma");
#pragma omp parallel for schedule(dynamic, 1)
    for (int it = 0; it < nkv * NC; it++) {
        const int g = it / NC, c = it % NC;
        const int kv0 = c * tpc * 32, kv1 = kv0 + tpc * 32 < n_kv ? kv0 + tpc * 32 : n_kv;
        float *a = acc + (size_t)it * gqa * hd;
        if (fma_ok) or_attn_chunk_fma(q, kc, vc, kv_type, g, gqa, nkv, hd, kv0, kv1, scale, a, m + (size_t)it * gqa, l + (size_t)it * gqa);
        else or_attn_chunk_base(q, kc, vc, kv_type, g, gqa, nkv, hd, kv0, kv1, scale, a, m + (size_t)it * gqa, l + (size_t)it * gqa);
    }
    for (int g = 0; g < nkv; g++)
        for (int s = 0; s < gqa; s++) {
            float M = -INFINITY;
            for (int c = 0; c < NC; c++) M = fmaxf(M, m[((size_t)g * NC + c) * gqa + s]);
            float e[64], L = 0.0f;
            for (int c = 0; c < NC; c++) {
                e[c] = or_attn_exp(m[((size_t)g * NC + c) * gqa + s] - M);
                L = fmaf(e[c], l[((size_t)g * NC + c) * gqa + s], L);
            }
            for (int d = 0; d < hd; d++) {
                float O = 0.0f;
                for (int c = 0; c < NC; c++) O = fmaf(e[c], acc[(((size_t)g * NC + c) * gqa + s) * hd + d], O);
                out[(size_t)(g * gqa + s) * hd + d] = O / L;
            }
        }
    free(acc);
    free(m);
    free(l);
}

/* ------------------------------------------------------------ layers */

int or_is_attn_layer(const or_cfg *c, int il) {
    return c->attn_every > 0 && (il % c->attn_every) == c->attn_every - 1;
}

/* dbg (nullable) receives the GDN intermediates in this order:
 * qkv[C] | z[HV*D] | alpha[HV] | beta_raw[HV] | conv_out[C] | g[HV] | beta[HV]
 * | o[HV*D] | on[HV*D] */
void or_gdn_mixer(const or_cfg *c, const void *const *w, void *const *st,
                  const float *xn, float *out, float *dbg) {
    const int E = c->n_embd, HK = c->gdn_hk, HV = c->gdn_hv, D = c->gdn_d;
    const int C = (2 * HK + HV) * D, VD = HV * D;
    float *qkv = (float *)malloc(sizeof(float) * (size_t)C);
    float *z = (float *)malloc(sizeof(float) * (size_t)VD);
    float *al = (float *)malloc(sizeof(float) * (size_t)HV);
    float *br = (float *)malloc(sizeof(float) * (size_t)HV);
    float *cv = (float *)malloc(sizeof(float) * (size_t)C);
    float *g = (float *)malloc(sizeof(float) * (size_t)HV);
    float *be = (float *)malloc(sizeof(float) * (size_t)HV);
    float *o = (float *)malloc(sizeof(float) * (size_t)VD);
    float *on = (float *)malloc(sizeof(float) * (size_t)VD);
    const int t = c->t_default;
    or_gemv(t, w[OR_SLOT_QKV], C, E, xn, qkv);
    or_gemv(t, w[OR_SLOT_Z], VD, E, xn, z);
    or_gemv(t, w[OR_SLOT_ALPHA], HV, E, xn, al);
    or_gemv(t, w[OR_SLOT_BETA], HV, E, xn, br);
    or_conv_silu(qkv, (float *)st[OR_ST_CONV], (const float *)w[OR_SLOT_CONV_W], cv, C, c->conv_k);
    for (int h = 0; h < 2 * HK; h++) or_l2norm(cv + (size_t)h * D, cv + (size_t)h * D, D, c->eps);
    or_gdn_gates(al, br, (const float *)w[OR_SLOT_DT_BIAS], (const float *)w[OR_SLOT_SSM_A], g, be, HV);
    const float scale = 1.0f / sqrtf((float)D);
    or_gdn_step(cv, cv + (size_t)HK * D, cv + (size_t)2 * HK * D, g, be, (float *)st[OR_ST_SSM], o,
                HV, HK, D, scale, or_gdn_cols(D));
    or_gated_rmsnorm(o, z, (const float *)w[OR_SLOT_SSM_NORM], on, HV, D, c->eps);
    or_gemv(t, w[OR_SLOT_SSM_OUT], E, VD, on, out);
    if (dbg) {
        float *p = dbg;
        memcpy(p, qkv, sizeof(float) * C); p += C;
        memcpy(p, z, sizeof(float) * VD); p += VD;
        memcpy(p, al, sizeof(float) * HV); p += HV;
        memcpy(p, br, sizeof(float) * HV); p += HV;
        memcpy(p, cv, sizeof(float) * C); p += C;
        memcpy(p, g, sizeof(float) * HV); p += HV;
        memcpy(p, be, sizeof(float) * HV); p += HV;
        memcpy(p, o, sizeof(float) * VD); p += VD;
        memcpy(p, on, sizeof(float) * VD);
    }
    free(qkv); free(z); free(al); free(br); free(cv); free(g); free(be); free(o); free(on);
}

/* the split-K geometry of a configuration (0: the library defaults for a
 * 256-workgroup grid over attn_nkv kv heads, and SINTER_ATTN_CHUNK_MIN) */
static int or_chunks(const or_cfg *c) {
    if (c->attn_chunks > 0) return c->attn_chunks;
    const int n = 256 / c->attn_nkv;
    return n > 64 ? 64 : n < 1 ? 1 : n;
}
static int or_chunk_min(const or_cfg *c) { return c->attn_chunk_min > 0 ? c->attn_chunk_min : 128; }

/* dbg (nullable): qg[NQ*2*HD] | k[NKV*HD] | v[NKV*HD] | qr[NQ*HD] | kr[NKV*HD]
 * | att[NQ*HD] | gated[NQ*HD] */
void or_attn_mixer(const or_cfg *c, const void *const *w, void *const *st,
                   const float *xn, int pos, float *out, float *dbg) {
    const int E = c->n_embd, NQ = c->attn_nq, NKV = c->attn_nkv, HD = c->head_dim;
    const int RW = NKV * HD;
    float *qg = (float *)malloc(sizeof(float) * (size_t)NQ * 2 * HD);
    float *kk = (float *)malloc(sizeof(float) * (size_t)RW);
    float *vv = (float *)malloc(sizeof(float) * (size_t)RW);
    float *qr = (float *)malloc(sizeof(float) * (size_t)NQ * HD);
    float *kr = (float *)malloc(sizeof(float) * (size_t)RW);
    float *att = (float *)malloc(sizeof(float) * (size_t)NQ * HD);
    float *gt = (float *)malloc(sizeof(float) * (size_t)NQ * HD);
    or_gemv(c->t_default, w[OR_SLOT_WQ], (int64_t)NQ * 2 * HD, E, xn, qg);
    or_gemv(c->t_default, w[OR_SLOT_WK], RW, E, xn, kk);
    or_gemv(c->t_attn_v, w[OR_SLOT_WV], RW, E, xn, vv);
    const float ts = or_rope_theta_scale(c->rope_base, c->rope_dims);
    for (int h = 0; h < NQ; h++) {
        or_rmsnorm(qg + (size_t)h * 2 * HD, (const float *)w[OR_SLOT_Q_NORM], qr + (size_t)h * HD, HD, c->eps);
        or_rope_neox(qr + (size_t)h * HD, HD, c->rope_dims, pos, ts);
    }
    for (int g = 0; g < NKV; g++) {
        or_rmsnorm(kk + (size_t)g * HD, (const float *)w[OR_SLOT_K_NORM], kr + (size_t)g * HD, HD, c->eps);
        or_rope_neox(kr + (size_t)g * HD, HD, c->rope_dims, pos, ts);
    }
    if (c->t_kv == OR_Q8_0) {
        /* the appended rows as Q8_0 blocks (ggml's reference quantiser) */
        blk_q8_0 *K = (blk_q8_0 *)st[OR_ST_K], *V = (blk_q8_0 *)st[OR_ST_V];
        or_quant_q8_0_ref(kr, K + (size_t)pos * (RW / 32), RW);
        or_quant_q8_0_ref(vv, V + (size_t)pos * (RW / 32), RW);
        or_attn_split(qr, K, V, OR_Q8_0, pos + 1, NQ, NKV, HD, 1.0f / sqrtf((float)HD), or_chunks(c), or_chunk_min(c), att);
    } else {
        uint16_t *K = (uint16_t *)st[OR_ST_K], *V = (uint16_t *)st[OR_ST_V];
        for (int i = 0; i < RW; i++) {
            K[(size_t)pos * RW + i] = or_f32_to_f16(kr[i]);
            V[(size_t)pos * RW + i] = or_f32_to_f16(vv[i]);
        }
        or_attn_split(qr, K, V, OR_F16, pos + 1, NQ, NKV, HD, 1.0f / sqrtf((float)HD), or_chunks(c), or_chunk_min(c), att);
    }
    for (int h = 0; h < NQ; h++)
        for (int d = 0; d < HD; d++) {
            const float gv = qg[(size_t)h * 2 * HD + HD + d];
            gt[(size_t)h * HD + d] = att[(size_t)h * HD + d] * or_sigmoid(gv);
        }
    or_gemv(c->t_default, w[OR_SLOT_WO], E, (int64_t)NQ * HD, gt, out);
    if (dbg) {
        float *p = dbg;
        memcpy(p, qg, sizeof(float) * NQ * 2 * HD); p += NQ * 2 * HD;
        memcpy(p, kk, sizeof(float) * RW); p += RW;
        memcpy(p, vv, sizeof(float) * RW); p += RW;
        memcpy(p, qr, sizeof(float) * NQ * HD); p += NQ * HD;
        memcpy(p, kr, sizeof(float) * RW); p += RW;
        memcpy(p, att, sizeof(float) * NQ * HD); p += NQ * HD;
        memcpy(p, gt, sizeof(float) * NQ * HD);
    }
    free(qg); free(kk); free(vv); free(qr); free(kr); free(att); free(gt);
}

/* SwiGLU FFN: silu(gate.x) * (up.x), then down (k0/ops/gemv.cuh:327-347) */
void or_ffn(const or_cfg *c, const void *const *w, const float *xn, float *out) {
    const int E = c->n_embd, F = c->n_ff;
    float *gg = (float *)malloc(sizeof(float) * (size_t)F);
    float *uu = (float *)malloc(sizeof(float) * (size_t)F);
    or_gemv(c->t_default, w[OR_SLOT_FFN_GATE], F, E, xn, gg);
    or_gemv(c->t_default, w[OR_SLOT_FFN_UP], F, E, xn, uu);
    for (int i = 0; i < F; i++) gg[i] = or_silu(gg[i]) * uu[i];
    or_gemv(c->t_ffn_down, w[OR_SLOT_FFN_DOWN], E, F, gg, out);
    free(gg);
    free(uu);
}

int64_t or_argmax_first(const float *x, int64_t n) {
    int64_t best = 0;
    for (int64_t i = 1; i < n; i++)
        if (x[i] > x[best]) best = i;
    return best;
}

int or_decode_step(const or_cfg *c, const void *const *weights, void *const *state,
                   int token, int pos, float *logits, float *resid) {
    const int E = c->n_embd;
    const void *embd = weights[(size_t)c->n_layer * OR_NSLOT + 0];
    const float *onorm = (const float *)weights[(size_t)c->n_layer * OR_NSLOT + 1];
    const void *outw = weights[(size_t)c->n_layer * OR_NSLOT + 2];
    float *x = (float *)malloc(sizeof(float) * (size_t)E);
    float *xn = (float *)malloc(sizeof(float) * (size_t)E);
    float *a = (float *)malloc(sizeof(float) * (size_t)E);
    or_dequant_row(c->t_embd, (const char *)embd + (size_t)token * or_row_bytes(c->t_embd, E), x, E);
    for (int il = 0; il < c->n_layer; il++) {
        const void *const *w = weights + (size_t)il * OR_NSLOT;
        void *const *st = state + (size_t)il * OR_NST;
        or_rmsnorm(x, (const float *)w[OR_SLOT_ATTN_NORM], xn, E, c->eps);
        if (or_is_attn_layer(c, il))
            or_attn_mixer(c, w, st, xn, pos, a, NULL);
        else
            or_gdn_mixer(c, w, st, xn, a, NULL);
        for (int i = 0; i < E; i++) x[i] = x[i] + a[i];
        or_rmsnorm(x, (const float *)w[OR_SLOT_POST_NORM], xn, E, c->eps);
        or_ffn(c, w, xn, a);
        for (int i = 0; i < E; i++) x[i] = x[i] + a[i];
        if (resid) memcpy(resid + (size_t)il * E, x, sizeof(float) * E);
    }
    or_rmsnorm(x, onorm, xn, E, c->eps);
    or_gemv(c->t_output, outw, c->n_vocab, E, xn, logits);
    free(x);
    free(xn);
    free(a);
    return (int)or_argmax_first(logits, c->n_vocab);
}
