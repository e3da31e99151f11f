// SINTER_OP_GEMV: the weight-streaming matrix-vector product of the decode
// pass, fused with what surrounds it in the reference schedule:
//   prologue  RMSNorm / gated RMSNorm / embedding lookup   (k0/ops/glue.cuh:56-227,
//             k0/ops/gdn.cuh:339-383)
//             + activation quantisation to the vec_dot type (k0/ops/gemv.cuh:213-237,
//             there q8_1; here ggml's Q8_K / Q8_0 / BF16)
//   body      y = W a for Q4_K / Q6_K / Q8_0 / BF16 / F32 rows, several
//             matrices ("segments") sharing one activation        (gemv.cuh:256-492)
//   epilogue  store, residual add, SwiGLU pair, greedy argmax    (gemv.cuh:327-347,
//             k0/harness.cpp:1187-1195)
//
// Work split: the rows of all segments form one byte-weighted row space; the
// participating workgroups take contiguous, byte-balanced row ranges.  A
// workgroup streams its share through three 36 KiB LDS tiles with gfx950
// LDS-DMA (global_load_lds_dwordx4: 16 B per lane straight into LDS, no
// VGPRs), two tiles in flight while one is computed.  A tile is a run of
// whole items (ggml blocks) that ignores row boundaries, sized so that every
// lane of the workgroup has one item (or half of one) per tile; item terms go
// to an LDS ring, and one tile later the lanes that own the touched rows add
// them to per-row running sums.  One workgroup barrier per tile.  Row results
// stay in LDS; the epilogues run over the buffered rows.
//
// Declared numerics (oracle/oracle.c): integer block dots are exact; each
// item's term is an fp64 expression of exact integers and the f16/f32
// scales; a row is the ascending fp64 sum of its item terms, rounded to fp32
// once, so outputs are bit-identical to the oracle's.
#pragma once
#include "dev_common.h"

namespace sinter {

__device__ __forceinline__ int vec_dot_type(int t) {
    return (t == SINTER_Q4_K || t == SINTER_Q6_K) ? SINTER_Q8_K
         : (t == SINTER_Q8_0) ? SINTER_Q8_0
         : (t == SINTER_BF16) ? SINTER_BF16 : SINTER_F32;
}
// bytes of one 256-element group of a weight row
__device__ __forceinline__ uint32_t group_bytes(int t) {
    switch (t) {
    case SINTER_Q4_K: return 144;
    case SINTER_Q6_K: return 210;
    case SINTER_Q8_0: return 272;
    case SINTER_BF16: return 512;
    default: return 1024;
    }
}

// ------------------------------------------------------------ LDS helpers

// 4 bytes at an arbitrary 2-aligned LDS byte offset
__device__ __forceinline__ uint32_t lds_u32(const char *lds, uint32_t off) {
    const uint32_t *w = reinterpret_cast<const uint32_t *>(lds + (off & ~3u));
    const uint32_t lo = w[0];
    if ((off & 3u) == 0) return lo;
    return __builtin_amdgcn_alignbyte(w[1], lo, off & 3u);
}
__device__ __forceinline__ uint16_t lds_u16(const char *lds, uint32_t off) {
    return *reinterpret_cast<const uint16_t *>(lds + off);
}

// ------------------------------------------------------------ activation layout in LDS
// (ACT_* constants and act_bytes are in isa.h, shared with host validation)
struct ActView {
    const lds_char *q;   // codes / bf16 / f32 chunks
    const LDS float *d;
    const LDS int16_t *bs;
};
__device__ __forceinline__ ActView act_view(char *qg, uint32_t K, int vt) {
    const lds_char *q = (const lds_char *)qg;
    ActView v{};
    v.q = q;
    v.d = reinterpret_cast<const LDS float *>(q + (K / 256) * ACT_GSTRIDE);
    v.bs = reinterpret_cast<const LDS int16_t *>(q + act_bs_off(K));
    (void)vt;
    return v;
}
__device__ __forceinline__ uint32_t act_qoff(uint32_t e) { return (e >> 8) * ACT_GSTRIDE + (e & 255); }

// ------------------------------------------------------------ embedding dequant (4 elements)

// ggml dequantize_row_* for elements [e, e+4) of one row (e % 4 == 0)
__device__ __forceinline__ void dequant4(const void *row, int type, uint32_t e, float out[4]) {
    const char *r = static_cast<const char *>(row);
    if (type == SINTER_Q4_K) {
        const blk_q4_K *b = reinterpret_cast<const blk_q4_K *>(r) + (e >> 8);
        const uint32_t j = e & 255, s = j >> 5, p = j >> 6, l = j & 31;
        int sc, m;
        if (s < 4) { sc = b->scales[s] & 63; m = b->scales[s + 4] & 63; }
        else {
            sc = (b->scales[s + 4] & 0xF) | ((b->scales[s - 4] >> 6) << 4);
            m = (b->scales[s + 4] >> 4) | ((b->scales[s] >> 6) << 4);
        }
        const float d1 = h2f(b->d) * (float)sc, m1 = h2f(b->dmin) * (float)m;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint8_t byte = b->qs[32 * p + l + i];
            const int q = (j & 32) ? (byte >> 4) : (byte & 0xF);
            out[i] = d1 * (float)q - m1;
        }
    } else if (type == SINTER_Q6_K) {
        const blk_q6_K *b = reinterpret_cast<const blk_q6_K *>(r) + (e >> 8);
        const float d = h2f(b->d);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t ee = (e & 255) + i, n = ee >> 7, rr = ee & 127, t = rr >> 5, l = rr & 31;
            const uint8_t lo = (t & 1) ? b->ql[64 * n + l + 32] : b->ql[64 * n + l];
            const int nib = (t & 2) ? (lo >> 4) : (lo & 0xF);
            const int hi = (b->qh[32 * n + l] >> (2 * t)) & 3;
            out[i] = d * (float)b->scales[ee / 16] * (float)((nib | (hi << 4)) - 32);
        }
    } else if (type == SINTER_Q8_0) {
        const blk_q8_0 *b = reinterpret_cast<const blk_q8_0 *>(r) + (e >> 5);
        const float d = h2f(b->d);
#pragma unroll
        for (int i = 0; i < 4; i++) out[i] = d * (float)b->qs[(e & 31) + i];
    } else if (type == SINTER_BF16 || type == SINTER_F16) {
        const uint16_t *h = reinterpret_cast<const uint16_t *>(r) + e;
#pragma unroll
        for (int i = 0; i < 4; i++) out[i] = (type == SINTER_BF16) ? bf2f(h[i]) : h2f(h[i]);
    } else {
        const float *f = reinterpret_cast<const float *>(r) + e;
#pragma unroll
        for (int i = 0; i < 4; i++) out[i] = f[i];
    }
}

// ------------------------------------------------------------ prologue

// The prologue gives each 256-element chunk to one 16-lane DPP row, 16
// consecutive elements per lane: a per-chunk reduction is four in-VALU DPP
// steps and a Q8_K bsum (16 elements) is one lane's own sum.
constexpr uint32_t PRO_ROWS = BLOCK_THREADS / 16;
// chunks per row per round (all loads of a round are issued before any of
// them is used): one round up to K = 16 * 5 * 256 = 20480
constexpr uint32_t PRO_RC = 5;

__device__ __forceinline__ void lds_st16(lds_char *p, uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
    u32x4_t v = {a, b, c, d};
    *reinterpret_cast<LDS u32x4_t *>(p) = v;
}
__device__ __forceinline__ uint32_t pack4_i8(int a, int b, int c, int d) {
    return (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) | ((uint32_t)(c & 0xff) << 16) | ((uint32_t)(d & 0xff) << 24);
}

// Quantise this lane's 16 elements [e0, e0+16) of chunk c (every lane of the
// row calls this with the same c) into the activation layout at q.
__device__ __forceinline__ void quant16(int vt, uint32_t c, uint32_t r, uint32_t e0, const float t[16], lds_char *q,
                                        LDS float *qd, LDS int16_t *qb) {
    int qv[16];
    if (vt == SINTER_Q8_K) {
        // ggml quantize_row_q8_K_ref: the signed element of largest |x|, first
        // index wins; q = min(127, rne(x * -127/max)), d = 1/iscale.  The
        // lane's maximum, first index and its sign come from balanced trees
        // (short dependency chains); NaNs never win (v_max ignores them, and
        // they compare unequal).
        float ax[16];
#pragma unroll
        for (int i = 0; i < 16; i++) ax[i] = fabsf(t[i]);
        float m4[4];
#pragma unroll
        for (int i = 0; i < 4; i++) m4[i] = fmaxf(fmaxf(ax[4 * i], ax[4 * i + 1]), fmaxf(ax[4 * i + 2], ax[4 * i + 3]));
        const float am = fmaxf(fmaxf(m4[0], m4[1]), fmaxf(m4[2], m4[3]));
        const float A = row16_max(am);
        // (index, sign) keys of the elements reaching A; the smallest wins
        int key[16];
#pragma unroll
        for (int i = 0; i < 16; i++) key[i] = ax[i] == A ? ((i << 1) | (t[i] < 0.0f ? 1 : 0)) : 0x7fffffff;
#pragma unroll
        for (int w = 8; w > 0; w >>= 1)
#pragma unroll
            for (int i = 0; i < w; i++) key[i] = min(key[i], key[i + w]);
        const int lkey = key[0] == 0x7fffffff ? 0x7fffffff : (int)(r << 5) + key[0];
        const int gkey = row16_min(lkey);
        float dd = 0.0f;
        if (A != 0.0f) {
            const float bmax = (gkey & 1) ? -A : A;
            const float iscale = -127.f / bmax;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int v = (int)__builtin_rintf(iscale * t[i]);
                qv[i] = v < 127 ? v : 127;
            }
            dd = 1.0f / iscale;
        } else {
#pragma unroll
            for (int i = 0; i < 16; i++) qv[i] = 0;
        }
        const int bsum = (((qv[0] + qv[1]) + (qv[2] + qv[3])) + ((qv[4] + qv[5]) + (qv[6] + qv[7]))) +
                         (((qv[8] + qv[9]) + (qv[10] + qv[11])) + ((qv[12] + qv[13]) + (qv[14] + qv[15])));
        lds_st16(q + c * ACT_GSTRIDE + r * 16, pack4_i8(qv[0], qv[1], qv[2], qv[3]), pack4_i8(qv[4], qv[5], qv[6], qv[7]),
                 pack4_i8(qv[8], qv[9], qv[10], qv[11]), pack4_i8(qv[12], qv[13], qv[14], qv[15]));
        qb[e0 / 16] = (int16_t)bsum;
        if (r == 0) qd[c] = dd;
    } else if (vt == SINTER_Q8_0) {
        // ggml-cpu x86 quantize_row_q8_0: d = f16(amax/127), q = rne(x * 127/amax);
        // a 32-element block is two lanes
        float am = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; i++) am = fmaxf(am, fabsf(t[i]));
        am = fmaxf(am, dpp_f<DPP_XOR1>(am));
        const float d = am / 127.f;
        const float id = (am != 0.0f) ? 127.f / am : 0.0f;
#pragma unroll
        for (int i = 0; i < 16; i++) qv[i] = (int)__builtin_rintf(t[i] * id);
        lds_st16(q + c * ACT_GSTRIDE + r * 16, pack4_i8(qv[0], qv[1], qv[2], qv[3]), pack4_i8(qv[4], qv[5], qv[6], qv[7]),
                 pack4_i8(qv[8], qv[9], qv[10], qv[11]), pack4_i8(qv[12], qv[13], qv[14], qv[15]));
        if ((r & 1) == 0) qd[e0 / 32] = h2f(f2h(d));
    } else if (vt == SINTER_BF16) {
        uint32_t h[8];
#pragma unroll
        for (int i = 0; i < 8; i++) h[i] = (uint32_t)f2bf(t[2 * i]) | ((uint32_t)f2bf(t[2 * i + 1]) << 16);
        lds_char *p = q + (e0 >> 6) * ACT_BF_CSTRIDE + (e0 & 63) * 2;
        lds_st16(p, h[0], h[1], h[2], h[3]);
        lds_st16(p + 16, h[4], h[5], h[6], h[7]);
    } else {
        lds_char *p = q + (e0 >> 6) * ACT_F_CSTRIDE + (e0 & 63) * 4;
#pragma unroll
        for (int k = 0; k < 4; k++)
            lds_st16(p + 16 * k, __float_as_uint(t[4 * k]), __float_as_uint(t[4 * k + 1]), __float_as_uint(t[4 * k + 2]),
                     __float_as_uint(t[4 * k + 3]));
    }
}

// Build the quantised activation in LDS (g_qbuf).  Every thread of the block
// calls this.  `red` is 128 B of LDS scratch.  Row g of the block (16 lanes)
// owns chunks g, g+16, ... and reads them in rounds of PRO_RC chunks, so the
// prologue pays one memory latency per round (one round up to K = 20480; an
// RMSNorm with more chunks makes one extra pass for its sum of squares).
__device__ __forceinline__ void gemv_prologue(const sinter_gemv_args &a, int vt, bool write_x, double *red,
                                              unsigned *err) {
    const uint32_t K = a.K;
    const bool embed = a.pro == SINTER_PRO_EMBED, gated = a.pro == SINTER_PRO_GATED;
    const bool rms = a.pro == SINTER_PRO_RMSNORM || embed;
    const __amdgpu_buffer_rsrc_t xr = coh_rsrc(a.x, embed ? 0u : K * 4);
    const __amdgpu_buffer_rsrc_t zr = coh_rsrc(a.aux, gated ? K * 4 : 0u);
    const void *erow = nullptr;
    if (embed) {
        int32_t tok = ld_coh(a.token);
        if (tok < 0 || (uint32_t)tok >= a.aux_rows) {   // never read outside the table
            if (threadIdx.x == 0) raise_error(err, SINTER_E_BAD_SHAPE, 0xE0000000u);
            tok = 0;
        }
        erow = static_cast<const char *>(a.aux) + (size_t)tok * sinter_row_bytes_dev(a.aux_type, K);
    }
    const uint32_t gd = 1u << a.gn_log2d;  // gated-norm head width (4..256)
    // the lane's indices, opaque to the compiler so that the per-lane address
    // arithmetic below is not hoisted out of the interpreter loop (where it
    // would stay live, in registers, for the whole kernel)
    uint32_t tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    const uint32_t r = tid & 15, g = tid >> 4, nchunk = K / 256;
    const uint32_t mine = nchunk > g ? (nchunk - g + PRO_ROWS - 1) / PRO_ROWS : 0u;   // chunks of this row
    auto raw16 = [&](uint32_t e0, float v[16]) {
        if (embed) {
#pragma unroll
            for (int k = 0; k < 4; k++) dequant4(erow, a.aux_type, e0 + 4 * k, v + 4 * k);
        } else {
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const float4 t = ld_coh16(xr, (e0 + 4 * k) * 4);
                v[4 * k] = t.x; v[4 * k + 1] = t.y; v[4 * k + 2] = t.z; v[4 * k + 3] = t.w;
            }
        }
    };
    // the second per-element input: the gate z (gated) or the norm weights
    auto raw16b = [&](uint32_t e0, float y[16]) {
#pragma unroll
        for (int k = 0; k < 4; k++) {
            float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
            if (gated) t = ld_coh16(zr, (e0 + 4 * k) * 4);
            else if (rms) t = *reinterpret_cast<const float4 *>(a.norm_w + e0 + 4 * k);
            y[4 * k] = t.x; y[4 * k + 1] = t.y; y[4 * k + 2] = t.z; y[4 * k + 3] = t.w;
        }
    };
    // gated-norm weights: element i of this lane is norm_w[(16r + i) % gd] in every chunk
    float gw[16];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
        if (gated) t = *reinterpret_cast<const float4 *>(a.norm_w + ((r * 16 + 4 * k) & (gd - 1)));
        gw[4 * k] = t.x; gw[4 * k + 1] = t.y; gw[4 * k + 2] = t.z; gw[4 * k + 3] = t.w;
    }
    float xv[PRO_RC][16], yv[PRO_RC][16];
    auto load_round = [&](uint32_t j0, bool both) {
#pragma unroll
        for (uint32_t j = 0; j < PRO_RC; j++) {
            if (j0 + j < mine) {
                const uint32_t e0 = (g + PRO_ROWS * (j0 + j)) * 256 + r * 16;
                raw16(e0, xv[j]);
                if (both) raw16b(e0, yv[j]);
            }
        }
    };
    // global RMSNorm scale (ggml: fp32 squares summed in double, mean -> f32,
    // scale = 1/sqrtf(mean + eps))
    float gscale = 1.0f;
    const bool one_round = nchunk <= PRO_ROWS * PRO_RC;
    if (one_round) load_round(0, true);
    if (rms) {
        double s = 0.0;
        for (uint32_t j0 = 0; j0 < mine; j0 += PRO_RC) {
            if (!one_round) load_round(j0, false);
#pragma unroll
            for (uint32_t j = 0; j < PRO_RC; j++)
                if (j0 + j < mine)
#pragma unroll
                    for (int i = 0; i < 16; i++) s += (double)(xv[j][i] * xv[j][i]);
        }
        s = block_sum_f64(s, red);
        const float mean = (float)(s / (double)K);
        gscale = 1.0f / sqrtf(mean + a.eps);
    }
    lds_char *q = (lds_char *)g_qbuf;
    LDS float *qd = reinterpret_cast<LDS float *>(q + (K / 256) * ACT_GSTRIDE);
    LDS int16_t *qb = reinterpret_cast<LDS int16_t *>(q + act_bs_off(K));
    const bool has_y = gated || rms;
    for (uint32_t j0 = 0; j0 < mine; j0 += PRO_RC) {
        if (!one_round) load_round(j0, true);
        const uint32_t cnt = min(PRO_RC, mine - j0);
        // slot 0 is processed, then the slots shift down by one: the code of
        // a chunk exists once (a loop body, fetched once per op) rather than
        // once per slot -- straight-line code is fetched from L2 every time
#pragma unroll 1
        for (uint32_t j = 0; j < cnt; j++) {
            if (j) {
#pragma unroll
                for (uint32_t k = 0; k + 1 < PRO_RC; k++)
#pragma unroll
                    for (int i = 0; i < 16; i++) xv[k][i] = xv[k + 1][i];
                if (has_y)
#pragma unroll
                    for (uint32_t k = 0; k + 1 < PRO_RC; k++)
#pragma unroll
                        for (int i = 0; i < 16; i++) yv[k][i] = yv[k + 1][i];
            }
            const uint32_t c = g + PRO_ROWS * (j0 + j), e0 = c * 256 + r * 16;
            const float *v = xv[0], *y = yv[0];
            float t[16];
            if (write_x)
#pragma unroll
                for (int k = 0; k < 4; k++)
                    st_coh4(a.x_out + e0 + 4 * k, make_float4(v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]));
            if (a.pro == SINTER_PRO_PLAIN) {
#pragma unroll
                for (int i = 0; i < 16; i++) t[i] = v[i];
            } else if (gated) {
                // per-head sums of squares in double: heads of 4 or 8
                // elements inside the lane, wider heads over gd/16 lanes
                double s4[4];
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    double h = 0.0;
#pragma unroll
                    for (int i = 0; i < 4; i++) h += (double)(v[4 * k + i] * v[4 * k + i]);
                    s4[k] = h;
                }
                const double s8a = s4[0] + s4[1], s8b = s4[2] + s4[3];
                double s16 = s8a + s8b;
                if (gd >= 32) s16 += dpp_d<DPP_XOR1>(s16);
                if (gd >= 64) s16 += dpp_d<DPP_XOR2>(s16);
                if (gd >= 128) s16 += dpp_d<DPP_HALF_MIRROR>(s16);
                if (gd >= 256) s16 += dpp_d<DPP_MIRROR>(s16);
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const double hsum = gd == 4 ? s4[i / 4] : gd == 8 ? (i < 8 ? s8a : s8b) : s16;
                    const float mean = (float)(hsum / (double)gd);
                    const float hs = 1.0f / sqrtf(mean + a.eps);
                    const float nrm = v[i] * hs;
                    const float wn = nrm * gw[i];
                    t[i] = wn * dev_silu(y[i]);
                    if ((i & 3) == 3) sched_fence();   // bounds the live fp64 temporaries
                }
            } else {
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const float nrm = v[i] * gscale;
                    t[i] = nrm * y[i];
                }
            }
            quant16(vt, c, r, e0, t, q, qd, qb);
        }
    }
    __syncthreads();
}

// ------------------------------------------------------------ item terms
// A weight row is a sequence of items: one 256-element group for the
// quantised types (one Q4_K / Q6_K block, eight Q8_0 blocks), 64 elements
// for BF16 / F32.  An item's term is an fp64 expression of exact integer
// block dots and the f16/f32 scales (a float sum of exact products for
// BF16/F32).  A row is the ascending fp64 sum of its item terms, rounded to
// fp32 once -- the fold oracle/oracle.c declares.
//
// Lanes per item: one for Q4_K / BF16 / F32; two for Q6_K (one 128-element
// half each, integer partials added exactly) and Q8_0 (blocks 0-3 and 4-7;
// the second lane continues the first lane's ascending block sum).  The term
// ends up on the item's last lane.
//
// With one wave per SIMD nothing hides LDS latency, so each item function
// issues all of its LDS reads first and only then computes (a scheduling
// barrier keeps the compiler from interleaving loads into the arithmetic,
// which would expose one LDS round trip per use).

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x4 lds16(const lds_char *p) { return *reinterpret_cast<const LDS u32x4 *>(p); }
__device__ __forceinline__ f32x4 ldsf16(const lds_char *p) { return *reinterpret_cast<const LDS f32x4 *>(p); }
__device__ __forceinline__ uint16_t ld_u16(const lds_char *p) { return *reinterpret_cast<const LDS uint16_t *>(p); }

// The N+1 aligned dwords covering N words at a 2-aligned LDS address, and
// the byte shift that extracts them (unaligned LDS reads stall the LDS
// pipeline on gfx950, so reads stay dword-aligned).
template <int N>
__device__ __forceinline__ uint32_t ld_span(const lds_char *p, uint32_t d[N + 1]) {
    const uint32_t off = (uint32_t)(uintptr_t)p;
    const LDS uint32_t *q = reinterpret_cast<const LDS uint32_t *>(p - (off & 3u));
#pragma unroll
    for (int i = 0; i <= N; i++) d[i] = q[i];
    return off & 3u;
}
template <int N>
__device__ __forceinline__ void span_words(const uint32_t d[N + 1], uint32_t sh, uint32_t w[N]) {
#pragma unroll
    for (int i = 0; i < N; i++) w[i] = __builtin_amdgcn_alignbyte(d[i + 1], d[i], sh);
}

// Q4_K block (16-aligned in LDS) against Q8_K group g
__device__ __forceinline__ double term_q4k(const lds_char *blk, const ActView &x, uint32_t g) {
    u32x4 wv[9], xv[16], bsv[2];
#pragma unroll
    for (int i = 0; i < 9; i++) wv[i] = lds16(blk + 16 * i);
    const lds_char *xq = x.q + g * ACT_GSTRIDE;
#pragma unroll
    for (int i = 0; i < 16; i++) xv[i] = lds16(xq + 16 * i);
    const lds_char *bsp = reinterpret_cast<const lds_char *>(x.bs + g * 16);
    bsv[0] = lds16(bsp);
    bsv[1] = lds16(bsp + 16);
    const float dxf = x.d[g];
    sched_fence();
    const uint32_t sw[3] = {wv[0].y, wv[0].z, wv[0].w};   // scales[0..11]
    auto byte = [&](uint32_t i) -> int { return (int)((sw[i >> 2] >> (8 * (i & 3))) & 0xff); };
    auto bsum = [&](int j) -> int {                       // bsums[j], int16
        const uint32_t wd = bsv[j >> 3][(j >> 1) & 3];
        return (j & 1) ? ((int)wd >> 16) : (int)(int16_t)(wd & 0xffff);
    };
    int isum = 0, imin = 0;
#pragma unroll
    for (int p = 0; p < 4; p++) {
        const int s0 = 2 * p, s1 = 2 * p + 1;
        int sc0, m0, sc1, m1;
        if (p < 2) {
            sc0 = byte(s0) & 63; m0 = byte(s0 + 4) & 63;
            sc1 = byte(s1) & 63; m1 = byte(s1 + 4) & 63;
        } else {
            sc0 = (byte(s0 + 4) & 0xF) | ((byte(s0 - 4) >> 6) << 4); m0 = (byte(s0 + 4) >> 4) | ((byte(s0) >> 6) << 4);
            sc1 = (byte(s1 + 4) & 0xF) | ((byte(s1 - 4) >> 6) << 4); m1 = (byte(s1 + 4) >> 4) | ((byte(s1) >> 6) << 4);
        }
        const u32x4 qa = wv[1 + 2 * p], qb = wv[2 + 2 * p];
        const uint32_t w[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
        const u32x4 x0 = xv[4 * p], x1 = xv[4 * p + 1], x2 = xv[4 * p + 2], x3 = xv[4 * p + 3];
        const uint32_t xl[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        const uint32_t xh[8] = {x2.x, x2.y, x2.z, x2.w, x3.x, x3.y, x3.z, x3.w};
        int dlo = 0, dhi = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            dlo = sdot4(w[i] & 0x0F0F0F0Fu, xl[i], dlo);
            dhi = sdot4((w[i] >> 4) & 0x0F0F0F0Fu, xh[i], dhi);
        }
        isum += sc0 * dlo + sc1 * dhi;
        imin += m0 * (bsum(4 * p) + bsum(4 * p + 1)) + m1 * (bsum(4 * p + 2) + bsum(4 * p + 3));
    }
    const double dx = (double)dxf;
    const double dw = (double)h2f((uint16_t)(wv[0].x & 0xffff));
    const double dm = (double)h2f((uint16_t)(wv[0].x >> 16));
    return (dw * dx) * (double)isum - (dm * dx) * (double)imin;
}

// Half n (elements [128n, 128n+128)) of a Q6_K block at a 2-aligned LDS
// address against Q8_K group g: the exact integer sum over its 8 sub-blocks
// of scale * (code dot x).  Codes are taken unsigned (0..63) and the -32
// offset folds through the bsums: sum((c-32)*x) = sum(c*x) - 32*bsum.
__device__ __forceinline__ int q6k_half(const lds_char *blk, const ActView &x, uint32_t g, uint32_t n) {
    uint32_t dl[17], dh[9], ds[3];
    const uint32_t shl = ld_span<16>(blk + 64 * n, dl);          // ql[64n .. 64n+64)
    const uint32_t shh = ld_span<8>(blk + 128 + 32 * n, dh);     // qh[32n .. 32n+32)
    const uint32_t shs = ld_span<2>(blk + 192 + 8 * n, ds);      // int8 scales[8n .. 8n+8)
    const lds_char *xq = x.q + g * ACT_GSTRIDE + 128 * n;
    u32x4 xv[8];
#pragma unroll
    for (int i = 0; i < 8; i++) xv[i] = lds16(xq + 16 * i);
    const u32x4 bsv = lds16(reinterpret_cast<const lds_char *>(x.bs + g * 16 + 8 * n));
    sched_fence();
    uint32_t ql[16], qh[8], scw[2];
    span_words<16>(dl, shl, ql);
    span_words<8>(dh, shh, qh);
    span_words<2>(ds, shs, scw);
    uint32_t xw[32];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        xw[4 * i] = xv[i].x; xw[4 * i + 1] = xv[i].y; xw[4 * i + 2] = xv[i].z; xw[4 * i + 3] = xv[i].w;
    }
    int dot[4][2] = {{0, 0}, {0, 0}, {0, 0}, {0, 0}};  // [quarter][16-element half]
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const uint32_t qa = ql[i], qb = ql[8 + i];
        const uint32_t c0 = (qa & 0x0F0F0F0Fu) | ((qh[i] << 4) & 0x30303030u);
        const uint32_t c1 = (qb & 0x0F0F0F0Fu) | ((qh[i] << 2) & 0x30303030u);
        const uint32_t c2 = ((qa >> 4) & 0x0F0F0F0Fu) | (qh[i] & 0x30303030u);
        const uint32_t c3 = ((qb >> 4) & 0x0F0F0F0Fu) | ((qh[i] >> 2) & 0x30303030u);
        const int hf = i >> 2;                     // l = 4i.. : half hf of each quarter
        dot[0][hf] = sdot4(c0, xw[i], dot[0][hf]);
        dot[1][hf] = sdot4(c1, xw[8 + i], dot[1][hf]);
        dot[2][hf] = sdot4(c2, xw[16 + i], dot[2][hf]);
        dot[3][hf] = sdot4(c3, xw[24 + i], dot[3][hf]);
    }
    int isum = 0;
#pragma unroll
    for (int t = 0; t < 4; t++) {
#pragma unroll
        for (int hf = 0; hf < 2; hf++) {
            const int j = 2 * t + hf;              // 16-element sub-block within the half
            const int sc = (int)(int8_t)((scw[j >> 2] >> (8 * (j & 3))) & 0xff);
            const uint32_t bw = bsv[j >> 1];
            const int bs = (j & 1) ? ((int)bw >> 16) : (int)(int16_t)(bw & 0xffff);
            isum += sc * (dot[t][hf] - 32 * bs);
        }
    }
    return isum;
}

// Blocks 4h .. 4h+3 of an 8-block Q8_0 item (34-byte blocks, 2-aligned)
// against Q8_0 activation blocks 8g+4h ..: the four block terms.
__device__ __forceinline__ void q80_quad(const lds_char *item, const ActView &x, uint32_t g, uint32_t h, double t[4]) {
    uint32_t dw[4][9], sh[4];
    uint16_t dh[4];
    u32x4 xv[8];
    float dx[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t b = 4 * h + j;
        const lds_char *bo = item + 34 * b;
        sh[j] = ld_span<8>(bo + 2, dw[j]);
        dh[j] = ld_u16(bo);
        const lds_char *xq = x.q + g * ACT_GSTRIDE + 32 * b;
        xv[2 * j] = lds16(xq);
        xv[2 * j + 1] = lds16(xq + 16);
        dx[j] = x.d[8 * g + b];
    }
    sched_fence();
#pragma unroll
    for (int j = 0; j < 4; j++) {
        uint32_t w[8];
        span_words<8>(dw[j], sh[j], w);
        const u32x4 x0 = xv[2 * j], x1 = xv[2 * j + 1];
        const uint32_t xw[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        int isum = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) isum = sdot4(w[i], xw[i], isum);
        t[j] = ((double)h2f(dh[j]) * (double)dx[j]) * (double)isum;
    }
}

// 64 bf16 elements (128 B, 16-aligned), products exact in fp64, ascending
__device__ __forceinline__ double term_bf16(const lds_char *blk, const ActView &x, uint32_t k) {
    const lds_char *xx = x.q + k * ACT_BF_CSTRIDE;
    u32x4 av[8], bv[8];
#pragma unroll
    for (int i = 0; i < 8; i++) { av[i] = lds16(blk + 16 * i); bv[i] = lds16(xx + 16 * i); }
    sched_fence();
    double acc = 0.0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t aw = av[i][j], bw = bv[i][j];
            acc += (double)__uint_as_float(aw << 16) * (double)__uint_as_float(bw << 16);
            acc += (double)__uint_as_float(aw & 0xffff0000u) * (double)__uint_as_float(bw & 0xffff0000u);
        }
    }
    return acc;
}

// 64 f32 elements (256 B, 16-aligned), products exact in fp64, ascending
__device__ __forceinline__ double term_f32(const lds_char *blk, const ActView &x, uint32_t k) {
    const lds_char *xx = x.q + k * ACT_F_CSTRIDE;
    double acc = 0.0;
#pragma unroll
    for (int h = 0; h < 2; h++) {
        f32x4 av[8], bv[8];
#pragma unroll
        for (int i = 0; i < 8; i++) { av[i] = ldsf16(blk + 128 * h + 16 * i); bv[i] = ldsf16(xx + 128 * h + 16 * i); }
        sched_fence();
#pragma unroll
        for (int i = 0; i < 8; i++) {
            acc += (double)av[i].x * (double)bv[i].x;
            acc += (double)av[i].y * (double)bv[i].y;
            acc += (double)av[i].z * (double)bv[i].z;
            acc += (double)av[i].w * (double)bv[i].w;
        }
    }
    return acc;
}

// ------------------------------------------------------------ work split
// The host compiles each GEMV into a GemvPlan (isa.h): per-segment constants,
// the term ring geometry and the workgroups' row cuts.  The kernel reads it
// through the constant address space, so every field is a scalar load.
typedef const __attribute__((address_space(4))) GemvPlan cplan_t;
typedef const __attribute__((address_space(4))) uint32_t cu32_t;

__device__ __forceinline__ uint32_t uni(uint32_t v) { return __builtin_amdgcn_readfirstlane(v); }

// q = v / d, r = v % d from m = floor((2^32-1) / d): the estimate is q or
// q-1, one correction step makes it exact (v < 2^31)
__device__ __forceinline__ uint32_t divm(uint32_t v, uint32_t d, uint32_t m, uint32_t &r) {
    uint32_t q = __umulhi(v, m);
    r = v - q * d;
    if (r >= d) { r -= d; q += 1; }
    return q;
}

// The term ring: row-aligned.  The row of workgroup-local index lr owns
// slot lr % R; its term k sits at slot*P + k (P = ipr rounded up to RING_PAD, the
// pad slot holds -0.0, an exact no-op in the fold).  SwiGLU up terms use a
// second ring of R*P behind the first.  Rows are folded once, complete, in
// ascending k.  "Deferred" rings fold a tile's rows one tile later (no extra
// barrier; R covers the rows of two tiles); otherwise the rows are folded
// right after an extra barrier.
struct Ring {
    uint32_t ipr, mipr, P, R, mR, RP, defer;
};

// ------------------------------------------------------------ tiles
// A tile is a run of whole items of one segment: items [a, a+cnt) of its
// matrix (and the same items of w2 for a SwiGLU pair), a contiguous byte
// range of the row-major weights.  Tiles ignore row boundaries, so every lane
// has an item; a row's terms may span tiles.  a = ra*ipr + ka.
//
// The DMA cursor walks the tiles of this workgroup in order and keeps the
// current segment's constants in registers; consecutive tiles of a segment
// differ by constants, so creating a tile is a handful of scalar operations.
struct TD {                 // what compute and fold need of a tile
    uint32_t ok, a, cnt, ra, ka;
    uint32_t type, swig, lr0;           // weight type, SwiGLU pair, workgroup-local index of row ra
    uint32_t skew_a, base_b;            // LDS byte offsets of matrix A's and B's first item
};
struct Cursor {
    uint32_t ok, seg, a, ra, ka;        // next tile to create
    uint32_t end, T, qT, rT, ib, type, swig, lrb;   // current segment
    uintptr_t wa, wb;                   // weights of the current segment
    uint32_t n_seg, ipr, row_lo, row_hi;            // the op: this workgroup's global rows
    cplan_t *pl;
};

// Move the cursor to the first segment >= s with rows in [row_lo, row_hi).
__device__ __forceinline__ void cur_seg(Cursor &c, uint32_t s) {
    c.ok = 0;
    for (; s < c.n_seg; s++) {
        const uint32_t base = c.pl->seg[s].base, rows = c.pl->seg[s].rows;
        const uint32_t lo = min(max(c.row_lo, base), base + rows) - base;
        const uint32_t hi = min(max(c.row_hi, base), base + rows) - base;
        if (lo < hi) {
            c.ok = 1; c.seg = s; c.a = lo * c.ipr; c.ra = lo; c.ka = 0;
            c.end = hi * c.ipr; c.T = c.pl->seg[s].T; c.qT = c.pl->seg[s].qT; c.rT = c.pl->seg[s].rT;
            c.ib = c.pl->seg[s].ib; c.type = c.pl->seg[s].type; c.swig = c.pl->seg[s].swig; c.lrb = base - c.row_lo;
            c.wa = (uintptr_t)c.pl->seg[s].wa;
            c.wb = (uintptr_t)c.pl->seg[s].wb;
            return;
        }
    }
}

// One 1 KiB LDS-DMA chunk per wave: lane l's 16 bytes at base + voff land at
// lds_base + 16*l.  Issued from inline asm so the compiler does not treat the
// pending DMA as aliasing every later LDS read (it would insert vmcnt(0)
// before them and serialise the pipeline); the tile loop below waits for it
// explicitly.  M0 (the LDS base of the DMA) is restored before the asm ends;
// one wait state separates the M0 write from the DMA that reads it.
// Weights are read once per pass, so the load is non-temporal (nt): streamed
// through L2 without displacing the lines that are reused (the kernel's own
// code, which every instruction-cache miss refetches from L2, and the
// activations).
__device__ __forceinline__ void lds_dma16(uintptr_t base, uint32_t voff, uint32_t lds_base) {
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %2, %3 nt\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "s"(lds_base), "v"(voff), "s"(base)
        : "memory");
}

// Create the tile at the cursor, LDS-DMA it into a 36 KiB buffer and advance
// the cursor.  Every wave issues exactly TILE_CPW 1-KiB chunks, so the number
// of outstanding loads per wave is a compile-time constant and the tile waits
// can be partial.  Matrix A fills the first chunks; a SwiGLU matrix B starts
// at the next 1 KiB chunk boundary, so every chunk reads from one matrix;
// lanes past a matrix's end re-read its last 16 bytes into the unused tail.
__device__ __forceinline__ TD tile_next(Cursor &c, char *buf) {
    TD t;
    t.ok = c.ok;
    t.a = 0; t.cnt = 0; t.ra = 0; t.ka = 0; t.type = 0; t.swig = 0; t.lr0 = 0; t.skew_a = 0; t.base_b = 0;
    if (!c.ok) return t;
    t.a = c.a; t.ra = c.ra; t.ka = c.ka;
    t.cnt = min(c.T, c.end - c.a);
    t.type = c.type; t.swig = c.swig; t.lr0 = c.lrb + c.ra;
    const uint32_t bytes = t.cnt * c.ib;
    const uintptr_t A = c.wa + (uintptr_t)c.a * c.ib;
    t.skew_a = (uint32_t)(A & 15);
    const uintptr_t sa = A & ~(uintptr_t)15;
    const uint32_t last_a = ((t.skew_a + bytes - 1) >> 4) << 4;       // offset of A's last 16 B
    const uint32_t chunks_a = (t.skew_a + bytes + 1023) >> 10;
    uintptr_t sb = sa;
    uint32_t last_b = last_a;
    if (c.swig) {
        const uintptr_t B = c.wb + (uintptr_t)c.a * c.ib;
        sb = B & ~(uintptr_t)15;
        const uint32_t skew_b = (uint32_t)(B & 15);
        t.base_b = chunks_a * 1024 + skew_b;
        last_b = ((skew_b + bytes - 1) >> 4) << 4;
    }
    const uint32_t w = uni(wave_id()), lane16 = lane_id() * 16;
    const uint32_t lbase = (uint32_t)(uintptr_t)(lds_void *)buf;
    if (!c.swig) {
        // one matrix: chunk j of the tile is bytes [1024 j, 1024 j + 1024)
#pragma unroll
        for (uint32_t k = 0; k < TILE_CPW; k++) {
            const uint32_t j = w + 4 * k;
            lds_dma16(sa, min(j * 1024 + lane16, last_a), lbase + j * 1024);
        }
    } else {
#pragma unroll
        for (uint32_t k = 0; k < TILE_CPW; k++) {
            const uint32_t j = w + 4 * k;
            const bool in_a = j < chunks_a;
            const uintptr_t src = in_a ? sa : sb;
            const uint32_t j0 = in_a ? j : j - chunks_a;
            const uint32_t voff = min(j0 * 1024 + lane16, in_a ? last_a : last_b);
            lds_dma16(src, voff, lbase + j * 1024);
        }
    }
    // advance
    c.a += t.cnt;
    if (c.a >= c.end) {
        cur_seg(c, c.seg + 1);
    } else {
        c.ra += c.qT;
        c.ka += c.rT;
        if (c.ka >= c.ipr) { c.ka -= c.ipr; c.ra += 1; }
    }
    return t;
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ void wait_lgkm0() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Item terms of a landed tile into the term ring.
template <int TYPE>
__device__ __forceinline__ void tile_terms_t(const TD &t, const lds_char *buf, LDS double *ring, bool swig,
                                             const Ring &rg, const ActView &x) {
    constexpr uint32_t LPI = (TYPE == SINTER_Q6_K || TYPE == SINTER_Q8_0) ? 2u : 1u;
    constexpr uint32_t IB = TYPE == SINTER_Q4_K ? 144u : TYPE == SINTER_Q6_K ? 210u : TYPE == SINTER_Q8_0 ? 272u
                          : TYPE == SINTER_BF16 ? 128u : 256u;
    const uint32_t l = threadIdx.x;
    const uint32_t m = swig ? (l >> 7) : 0u;
    const uint32_t ll = swig ? (l & 127u) : l;
    const uint32_t u = ll / LPI, part = ll % LPI;
    if (u < t.cnt) {   // the lanes of one item are active together
        uint32_t k, slot;
        const uint32_t q = divm(t.ka + u, rg.ipr, rg.mipr, k);
        (void)divm(t.lr0 + q, rg.R, rg.mR, slot);
        const lds_char *blk = buf + (m ? t.base_b : t.skew_a) + u * IB;
        double term;
        if constexpr (TYPE == SINTER_Q4_K) {
            term = term_q4k(blk, x, k);
        } else if constexpr (TYPE == SINTER_Q6_K) {
            const uint16_t dh = ld_u16(blk + 208);
            const float dxf = x.d[k];
            int is = q6k_half(blk, x, k, part);
            is += __shfl_xor(is, 1, 64);
            term = ((double)h2f(dh) * (double)dxf) * (double)is;
        } else if constexpr (TYPE == SINTER_Q8_0) {
            double tt[4];
            q80_quad(blk, x, k, part, tt);
            const double lo4 = (((0.0 + tt[0]) + tt[1]) + tt[2]) + tt[3];   // blocks 0-3 (part 0)
            const double prev = __shfl_xor(lo4, 1, 64);
            term = (((prev + tt[0]) + tt[1]) + tt[2]) + tt[3];             // blocks 4-7 continue it (part 1)
        } else if constexpr (TYPE == SINTER_BF16) {
            term = term_bf16(blk, x, k);
        } else {
            term = term_f32(blk, x, k);
        }
        if (part == LPI - 1) ring[m * rg.RP + slot * rg.P + k] = term;
    }
}

__device__ __forceinline__ void tile_terms(const TD &t, const char *bufg, const Ring &rg, const ActView &x) {
    const bool swig = t.swig != 0;
    const lds_char *buf = (const lds_char *)bufg;
    LDS double *ring = (LDS double *)g_cb;
    switch (t.type) {
    case SINTER_Q4_K: tile_terms_t<SINTER_Q4_K>(t, buf, ring, swig, rg, x); break;
    case SINTER_Q6_K: tile_terms_t<SINTER_Q6_K>(t, buf, ring, swig, rg, x); break;
    case SINTER_Q8_0: tile_terms_t<SINTER_Q8_0>(t, buf, ring, swig, rg, x); break;
    case SINTER_BF16: tile_terms_t<SINTER_BF16>(t, buf, ring, swig, rg, x); break;
    default: tile_terms_t<SINTER_F32>(t, buf, ring, swig, rg, x); break;
    }
}

// workgroup-local rows completed once this tile is computed
__device__ __forceinline__ uint32_t td_done_after(const TD &t, const Ring &rg) {
    uint32_t r;
    return t.lr0 + divm(t.ka + t.cnt, rg.ipr, rg.mipr, r);
}

// One row's P ring terms summed in ascending order (fp64); pad terms are
// -0.0 and rows start 16-byte aligned.  With P a multiple of RING_PAD = 8:
// rows of up to 24 terms (K <= 6144 for 256-element items) issue every read
// before the first add -- one LDS round trip; longer rows run 8-term batches
// with the next batch's reads in flight.  Other P (short rows): pairs.
__device__ __forceinline__ double fold_row(const LDS double *g, uint32_t P) {
    typedef double f64x2 __attribute__((ext_vector_type(2)));
    const LDS f64x2 *v = reinterpret_cast<const LDS f64x2 *>(g);
    double s = 0.0;
    if ((P & 7u) != 0) {
        for (uint32_t k = 0; k < P / 2; k++) {
            const f64x2 b = v[k];
            s += b.x;
            s += b.y;
        }
        return s;
    }
    if (P <= 24) {
        f64x2 b[12];
#pragma unroll
        for (uint32_t i = 0; i < 4; i++) b[i] = v[i];
        if (P >= 16) {
#pragma unroll
            for (uint32_t i = 4; i < 8; i++) b[i] = v[i];
        }
        if (P >= 24) {
#pragma unroll
            for (uint32_t i = 8; i < 12; i++) b[i] = v[i];
        }
#pragma unroll
        for (uint32_t i = 0; i < 4; i++) { s += b[i].x; s += b[i].y; }
        if (P >= 16) {
#pragma unroll
            for (uint32_t i = 4; i < 8; i++) { s += b[i].x; s += b[i].y; }
        }
        if (P >= 24) {
#pragma unroll
            for (uint32_t i = 8; i < 12; i++) { s += b[i].x; s += b[i].y; }
        }
        return s;
    }
    f64x2 cur[4];
#pragma unroll
    for (uint32_t i = 0; i < 4; i++) cur[i] = v[i];
    for (uint32_t k = 0; k < P; k += 8) {
        f64x2 nxt[4];
        if (k + 8 < P) {
#pragma unroll
            for (uint32_t i = 0; i < 4; i++) nxt[i] = v[(k + 8) / 2 + i];
        }
#pragma unroll
        for (uint32_t i = 0; i < 4; i++) { s += cur[i].x; s += cur[i].y; }
#pragma unroll
        for (uint32_t i = 0; i < 4; i++) cur[i] = nxt[i];
    }
    return s;
}

// Fold the rows this tile completed: rows [t.lr0, done_after).  The row of
// workgroup-local index lr is folded by lane ((lr%4)<<6) | ((lr/4)%64) and
// rounded to fp32 into g_res.
__device__ __forceinline__ void tile_fold(const TD &t, const Ring &rg, uint32_t res_row0) {
    const LDS double *ring = (const LDS double *)g_cb;
    LDS float *res = (LDS float *)g_res;
    const uint32_t nf = td_done_after(t, rg) - t.lr0;
    const uint32_t l = threadIdx.x;
    const uint32_t c = ((l & 63u) << 2) | (l >> 6);
    const uint32_t d = (c - t.lr0) & 255u;
    if (d < nf) {
        const uint32_t lr = t.lr0 + d;
        uint32_t slot;
        (void)divm(lr, rg.R, rg.mR, slot);
        const uint32_t i = lr - res_row0;
        res[2 * i] = (float)fold_row(ring + slot * rg.P, rg.P);
        if (t.swig) res[2 * i + 1] = (float)fold_row(ring + rg.RP + slot * rg.P, rg.P);
    }
}

// ------------------------------------------------------------ the op

// Apply the epilogues to the buffered rows [row0, row0 + n) and store them;
// greedy-argmax candidates fold into (bv, bi).  All threads.
__device__ __forceinline__ void gemv_flush(const sinter_gemv_args &a, uint32_t row0, uint32_t n, float &bv, int32_t &bi) {
    for (uint32_t i = threadIdx.x; i < n; i += BLOCK_THREADS) {
        const uint32_t grow = row0 + i;
        uint32_t s = 0, base = 0;
        while (s + 1 < a.n_seg && grow >= base + a.seg[s].rows) { base += a.seg[s].rows; s++; }
        const sinter_gemv_seg &sg = a.seg[s];
        const uint32_t r = grow - base;
        const float dot = g_res[2 * i];
        float y = dot;
        if (sg.epi == SINTER_EPI_SWIGLU) {
            y = dev_silu(dot) * g_res[2 * i + 1];
        } else if (sg.epi == SINTER_EPI_RESID) {
            y = ld_coh(sg.aux + r) + dot;
        } else if (sg.epi == SINTER_EPI_CONV) {
            // causal conv over {state[0..dc-2], dot}, fp64 sum rounded once,
            // then silu; the state shifts by one tap (this block owns row r)
            const uint32_t dc = sg.dconv;
            float *st = sg.aux + (size_t)r * (dc - 1);
            const float *cw = static_cast<const float *>(sg.w2) + (size_t)r * dc;
            float win[8];
#pragma unroll
            for (uint32_t j = 0; j < 8; j++) win[j] = (j + 1 < dc) ? st[j] : 0.0f;
            double cacc = 0.0;
#pragma unroll
            for (uint32_t j = 0; j < 8; j++) {
                const float wv = (j + 1 < dc) ? win[j] : (j + 1 == dc ? dot : 0.0f);
                if (j < dc) cacc += (double)wv * (double)cw[j];
            }
            y = dev_silu((float)cacc);
#pragma unroll
            for (uint32_t j = 0; j < 7; j++)
                if (j + 1 < dc) st[j] = (j + 2 < dc) ? win[j + 1] : dot;
        } else if (sg.epi == SINTER_EPI_ARGMAX) {
            if (y > bv || (y == bv && (int32_t)r < bi)) { bv = y; bi = (int32_t)r; }
        }
        st_coh(sg.y + r, y);
    }
}

// What gemv_begin leaves for gemv_run (wave-uniform registers): the op can
// be begun before the grid barrier that precedes it -- its weights do not
// depend on the barrier -- so the first two tiles stream in while the
// workgroup waits.
struct GemvState {
    uint32_t ok, row_lo;
    Ring rg;
    Cursor cur;
    TD X, Y;
};

// Copy the payload to LDS, read the plan, clear the term ring and LDS-DMA the
// first two tiles.  Uses LDS (the GEMV buffers) only, so it may run as soon
// as the previous op of the pass has returned.
__device__ __forceinline__ void gemv_begin(const sinter_instr &ins, const GemvPlan *plan, const uint32_t *cuts,
                                           unsigned *err, GemvState &st) {
    if (threadIdx.x < sizeof(sinter_gemv_args) / 4)
        reinterpret_cast<uint32_t *>(g_args)[threadIdx.x] = reinterpret_cast<const uint32_t *>(ins.payload)[threadIdx.x];
    // every ring slot starts as -0.0 (pad slots keep it)
    for (uint32_t i = threadIdx.x; i < CB_CAP; i += BLOCK_THREADS) g_cb[i] = -0.0;
    cplan_t *pl = (cplan_t *)plan;
    cu32_t *cu = (cu32_t *)cuts;
    const uint32_t rel = uni(blockIdx.x - ins.block_lo);
    st.ok = pl->ok;
    if (!st.ok) {
        if (rel == 0 && threadIdx.x == 0) raise_error(err, SINTER_E_BAD_SHAPE, ins.dbg_node);
        __syncthreads();
        return;
    }
    st.rg.ipr = pl->ipr; st.rg.mipr = pl->mipr; st.rg.P = pl->P; st.rg.R = pl->R;
    st.rg.mR = pl->mR; st.rg.RP = pl->RP; st.rg.defer = pl->defer;
    Cursor &c = st.cur;
    c.pl = pl;
    c.n_seg = pl->n_seg;
    c.ipr = pl->ipr;
    c.row_lo = cu[rel];
    c.row_hi = cu[rel + 1];
    st.row_lo = c.row_lo;
    cur_seg(c, 0);
    st.X = tile_next(c, g_tiles);
    st.Y = tile_next(c, g_tiles + TILE_BYTES);
    __syncthreads();
}

// The rest of the op: prologue, tile pipeline, epilogues.
__device__ __forceinline__ void gemv_run(const sinter_instr &ins, unsigned *err, GemvState &st) {
    if (!st.ok) return;
    const sinter_gemv_args &a = *reinterpret_cast<const sinter_gemv_args *>(g_args);
    const uint32_t rel = uni(blockIdx.x - ins.block_lo), nblk = uni(ins.block_hi - ins.block_lo);
    const uint32_t K = a.K;
    const int vt = (int)st.cur.pl->vt;
    const bool any_argmax = st.cur.pl->any_argmax != 0;
    const uint32_t row_lo = st.row_lo;
    const Ring rg = st.rg;
    Cursor cur = st.cur;
    TD X = st.X, Y = st.Y;

    // The tile pipeline: X = tile being computed (buffer bx), Y = next (in
    // flight), the tile after Y is created and issued this iteration into the
    // buffer that X-1 occupied, P = the previous tile.  One barrier per tile
    // makes X's DMA and the previous terms visible to every wave and frees
    // P's buffer; a deferred ring folds P's rows in the same step, otherwise
    // X's rows are folded after a second barrier.
    const bool write_x = (a.pro == SINTER_PRO_EMBED) && rel == 0 && a.x_out != nullptr;
    gemv_prologue(a, vt, write_x, g_red, err);   // ends with __syncthreads()
    settle_vmem();
    const ActView x = act_view(g_qbuf, K, vt);

    float bv = -INFINITY;
    int32_t bi = 0x7fffffff;
    uint32_t res_row0 = 0;           // workgroup-local first row not yet flushed
    TD P;
    P.ok = 0; P.a = 0; P.cnt = 0; P.ra = 0; P.ka = 0; P.type = 0; P.swig = 0; P.lr0 = 0; P.skew_a = 0; P.base_b = 0;
    uint32_t bx = 0;
    while (X.ok) {
        if (Y.ok) wait_vmcnt<TILE_CPW>(); else wait_vmcnt<0>();
        wait_lgkm0();
        __builtin_amdgcn_s_barrier();
        const uint32_t bz = bx == 0 ? 2u : bx - 1;
        const TD Z = tile_next(cur, g_tiles + bz * TILE_BYTES);
        const TD &F = rg.defer ? P : X;       // the tile whose rows this step folds
        if (rg.defer && P.ok && td_done_after(P, rg) - res_row0 > RES_CAP) {
            gemv_flush(a, row_lo + res_row0, P.lr0 - res_row0, bv, bi);
            settle_vmem();
            res_row0 = P.lr0;
            __syncthreads();
        }
        tile_terms(X, g_tiles + bx * TILE_BYTES, rg, x);
        if (!rg.defer) {
            wait_lgkm0();
            __builtin_amdgcn_s_barrier();
            if (td_done_after(X, rg) - res_row0 > RES_CAP) {
                gemv_flush(a, row_lo + res_row0, X.lr0 - res_row0, bv, bi);
                settle_vmem();
                res_row0 = X.lr0;
                __syncthreads();
            }
        }
        if (F.ok) tile_fold(F, rg, res_row0);
        P = X; X = Y; Y = Z;
        bx = bx == 2 ? 0u : bx + 1;
    }
    wait_lgkm0();
    __syncthreads();
    uint32_t rows_total = 0;
    if (P.ok) {
        rows_total = td_done_after(P, rg);
        if (rg.defer) {
            if (rows_total - res_row0 > RES_CAP) {
                gemv_flush(a, row_lo + res_row0, P.lr0 - res_row0, bv, bi);
                res_row0 = P.lr0;
                __syncthreads();
            }
            tile_fold(P, rg, res_row0);
        }
    }
    __syncthreads();
    gemv_flush(a, row_lo + res_row0, rows_total - res_row0, bv, bi);

    // greedy argmax: block-local best, then the last-arriving block reduces
    if (any_argmax) {
        // block reduction of (value, index): larger value, then smaller index
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(bv, o, 64);
            const int32_t oi = __shfl_xor(bi, o, 64);
            if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
        }
        float *rv = reinterpret_cast<float *>(g_part);
        int32_t *ri = reinterpret_cast<int32_t *>(g_part + 4);
        __syncthreads();
        if (lane_id() == 0) { rv[wave_id()] = bv; ri[wave_id()] = bi; }
        __syncthreads();
        if (threadIdx.x == 0) {
            for (int w = 1; w < (int)(BLOCK_THREADS / 64); w++)
                if (rv[w] > bv || (rv[w] == bv && ri[w] < bi)) { bv = rv[w]; bi = ri[w]; }
        }
    }
    if (any_argmax && threadIdx.x == 0 && rel >= static_cast<sinter_argmax_ws *>(a.epi_ws)->capacity) {
        raise_error(err, SINTER_E_BAD_SHAPE, ins.dbg_node);
    } else if (any_argmax && threadIdx.x == 0) {
        sinter_argmax_ws *ws = static_cast<sinter_argmax_ws *>(a.epi_ws);
        st_coh(ws->part_val + rel, bv);
        st_coh(ws->part_idx + rel, bi);
        settle_vmem();
        const unsigned old = __hip_atomic_fetch_add(ws->count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old == nblk - 1) {
            float best = -INFINITY;
            int32_t bidx = 0x7fffffff;
            const __amdgpu_buffer_rsrc_t vr = coh_rsrc(ws->part_val, nblk * 4), ir = coh_rsrc(ws->part_idx, nblk * 4);
            for (uint32_t w = 0; w < nblk; w++) {
                const float v = ld_coh4b(vr, w * 4);
                const int32_t i = __float_as_int(ld_coh4b(ir, w * 4));
                if (v > best || (v == best && i < bidx)) { best = v; bidx = i; }
            }
            sinter_pass_cell *pc = reinterpret_cast<sinter_pass_cell *>(ws->pass_cell);
            const int32_t steps = ld_coh(&pc->steps);
            if (ws->history && (uint32_t)steps < ws->history_cap) st_coh(ws->history + steps, bidx);
            st_coh(&pc->steps, steps + 1);
            st_coh(&pc->token, bidx);
            st_coh(&pc->pos, ld_coh(&pc->pos) + 1);
            __hip_atomic_store(ws->count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    __syncthreads();
}

__device__ __forceinline__ void op_gemv(const sinter_instr &ins, const GemvPlan *plan, const uint32_t *cuts,
                                        unsigned *err) {
    GemvState st;
    gemv_begin(ins, plan, cuts, err, st);
    gemv_run(ins, err, st);
}

}  // namespace sinter
