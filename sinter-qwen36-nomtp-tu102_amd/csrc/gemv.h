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
// workgroup streams its rows in tiles: 16-byte coalesced global loads into
// registers, one tile ahead, stored into a double-buffered LDS tile; compute
// then reads the (arbitrarily aligned) ggml blocks from LDS.  One lane owns one
// (row, 256-element group) item and produces that group's exact term.
//
// Declared fold (identical in oracle/oracle.c): integer block dots are exact;
// each 256-element group contributes one fp64 term (for Q8_0 the sum of its
// 8 block terms in ascending order); the row is the ascending fp64 sum of its
// group terms, rounded to fp32 once.
#pragma once
#include "dev_common.h"

namespace sinter {

constexpr int MAX_LD = (int)(TILE_BYTES / 16 / BLOCK_THREADS);  // uint4 per thread per tile

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
// Q8_K: qs int8[K] | d f32[K/256] | bsums i16[K/16]
// Q8_0: qs int8[K] | d f32[K/32]  (d is the f16-rounded scale, as float)
// BF16: u16[K];  F32: f32[K]
struct ActView {
    const int8_t *qs;
    const float *d;
    const int16_t *bs;
    const uint16_t *bf;
    const float *f;
};
__device__ __forceinline__ ActView act_view(char *q, uint32_t K, int vt) {
    ActView v{};
    v.qs = reinterpret_cast<const int8_t *>(q);
    if (vt == SINTER_Q8_K) {
        v.d = reinterpret_cast<const float *>(q + K);
        v.bs = reinterpret_cast<const int16_t *>(q + K + (K / 256) * 4);
    } else if (vt == SINTER_Q8_0) {
        v.d = reinterpret_cast<const float *>(q + K);
    }
    v.bf = reinterpret_cast<const uint16_t *>(q);
    v.f = reinterpret_cast<const float *>(q);
    return v;
}

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

// Raw input value of elements [e, e+4): x, or the embedding row.
__device__ __forceinline__ void pro_raw4(const sinter_gemv_args &a, const void *erow, uint32_t e, float v[4]) {
    if (a.pro == SINTER_PRO_EMBED) {
        dequant4(erow, a.aux_type, e, v);
    } else {
        const float4 t = *reinterpret_cast<const float4 *>(a.x + e);
        v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
    }
}

// Build the quantised activation in LDS at `q`.  Every thread of the block
// calls this.  `red` is 128 B of LDS scratch.
__device__ void gemv_prologue(const sinter_gemv_args &a, int vt, bool write_x, char *q, double *red,
                              unsigned *err) {
    const uint32_t K = a.K;
    const void *erow = nullptr;
    if (a.pro == SINTER_PRO_EMBED) {
        int32_t tok = *a.token;
        if (tok < 0 || (uint32_t)tok >= a.aux_rows) {   // never read outside the table
            if (threadIdx.x == 0) raise_error(err, SINTER_E_BAD_SHAPE, 0xE0000000u);
            tok = 0;
        }
        erow = static_cast<const char *>(a.aux) + (size_t)tok * sinter_row_bytes_dev(a.aux_type, K);
    }
    // global RMSNorm scale (ggml: fp32 squares summed in double, mean -> f32,
    // scale = 1/sqrtf(mean + eps))
    float gscale = 1.0f;
    if (a.pro == SINTER_PRO_RMSNORM || a.pro == SINTER_PRO_EMBED) {
        double s = 0.0;
        for (uint32_t e = threadIdx.x * 4; e < K; e += blockDim.x * 4) {
            float v[4];
            pro_raw4(a, erow, e, v);
#pragma unroll
            for (int i = 0; i < 4; i++) s += (double)(v[i] * v[i]);
        }
        s = block_sum_f64(s, red);
        const float mean = (float)(s / (double)K);
        gscale = 1.0f / sqrtf(mean + a.eps);
    }
    const uint32_t gd = 1u << a.gn_log2d;  // gated-norm head width (64..256)
    const int lane = lane_id();
    const int nw = blockDim.x >> 6;
    int8_t *qs = reinterpret_cast<int8_t *>(q);
    float *qd = reinterpret_cast<float *>(q + K);
    int16_t *qb = reinterpret_cast<int16_t *>(q + K + (K / 256) * 4);
    // one wave per 256-element chunk, 4 consecutive elements per lane
    for (uint32_t c = wave_id(); c < K / 256; c += nw) {
        const uint32_t e = c * 256 + lane * 4;
        float v[4], t[4];
        pro_raw4(a, erow, e, v);
        if (write_x) *reinterpret_cast<float4 *>(a.x_out + e) = make_float4(v[0], v[1], v[2], v[3]);
        if (a.pro == SINTER_PRO_PLAIN) {
#pragma unroll
            for (int i = 0; i < 4; i++) t[i] = v[i];
        } else if (a.pro == SINTER_PRO_GATED) {
            // per-head sum over gd/4 lanes (heads never straddle a chunk)
            double s = 0.0;
#pragma unroll
            for (int i = 0; i < 4; i++) s += (double)(v[i] * v[i]);
            for (uint32_t o = 1; o < gd / 4; o <<= 1) s += __shfl_xor(s, (int)o, 64);
            const float mean = (float)(s / (double)gd);
            const float hs = 1.0f / sqrtf(mean + a.eps);
            const float4 z = *reinterpret_cast<const float4 *>(static_cast<const float *>(a.aux) + e);
            const float zz[4] = {z.x, z.y, z.z, z.w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float nrm = v[i] * hs;
                const float wn = nrm * a.norm_w[(e + i) & (gd - 1)];
                t[i] = wn * dev_silu(zz[i]);
            }
        } else {
            const float4 w = *reinterpret_cast<const float4 *>(a.norm_w + e);
            const float ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float nrm = v[i] * gscale;
                t[i] = nrm * ww[i];
            }
        }
        if (vt == SINTER_Q8_K) {
            // ggml quantize_row_q8_K_ref: signed element of largest |x|, first index wins
            float bmax = 0.0f, bamax = 0.0f;
            int bidx = 0x7fffffff;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float ax = fabsf(t[i]);
                if (ax > bamax) { bamax = ax; bmax = t[i]; bidx = lane * 4 + i; }
            }
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) {
                const float oa = __shfl_xor(bamax, o, 64);
                const float om = __shfl_xor(bmax, o, 64);
                const int oi = __shfl_xor(bidx, o, 64);
                if (oa > bamax || (oa == bamax && oi < bidx)) { bamax = oa; bmax = om; bidx = oi; }
            }
            int qv[4] = {0, 0, 0, 0};
            float dd = 0.0f;
            if (bamax != 0.0f) {
                const float iscale = -127.f / bmax;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int r = (int)__builtin_rintf(iscale * t[i]);
                    qv[i] = r < 127 ? r : 127;
                }
                dd = 1.0f / iscale;
            }
            const uint32_t packed = (uint32_t)(qv[0] & 0xff) | ((uint32_t)(qv[1] & 0xff) << 8) |
                                    ((uint32_t)(qv[2] & 0xff) << 16) | ((uint32_t)(qv[3] & 0xff) << 24);
            *reinterpret_cast<uint32_t *>(qs + e) = packed;
            int bsum = qv[0] + qv[1] + qv[2] + qv[3];
            bsum += __shfl_xor(bsum, 1, 64);
            bsum += __shfl_xor(bsum, 2, 64);
            if ((lane & 3) == 0) qb[e / 16] = (int16_t)bsum;
            if (lane == 0) qd[c] = dd;
        } else if (vt == SINTER_Q8_0) {
            // ggml-cpu x86 quantize_row_q8_0: d = f16(amax/127), q = rne(x * 127/amax)
            float am = fmaxf(fmaxf(fabsf(t[0]), fabsf(t[1])), fmaxf(fabsf(t[2]), fabsf(t[3])));
            am = fmaxf(am, __shfl_xor(am, 1, 64));
            am = fmaxf(am, __shfl_xor(am, 2, 64));
            am = fmaxf(am, __shfl_xor(am, 4, 64));
            const float d = am / 127.f;
            const float id = (am != 0.0f) ? 127.f / am : 0.0f;
            int qv[4];
#pragma unroll
            for (int i = 0; i < 4; i++) qv[i] = (int)__builtin_rintf(t[i] * id);
            const uint32_t packed = (uint32_t)(qv[0] & 0xff) | ((uint32_t)(qv[1] & 0xff) << 8) |
                                    ((uint32_t)(qv[2] & 0xff) << 16) | ((uint32_t)(qv[3] & 0xff) << 24);
            *reinterpret_cast<uint32_t *>(qs + e) = packed;
            if ((lane & 7) == 0) qd[e / 32] = h2f(f2h(d));
        } else if (vt == SINTER_BF16) {
            uint16_t *bf = reinterpret_cast<uint16_t *>(q);
#pragma unroll
            for (int i = 0; i < 4; i++) bf[e + i] = f2bf(t[i]);
        } else {
            float *f = reinterpret_cast<float *>(q);
#pragma unroll
            for (int i = 0; i < 4; i++) f[e + i] = t[i];
        }
    }
    __syncthreads();
}

// ------------------------------------------------------------ group terms

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// Q4_K block (16-aligned in LDS) against Q8_K group g
__device__ __forceinline__ double term_q4k(const char *blk, const ActView &x, uint32_t g) {
    const uint4 hdr = *reinterpret_cast<const uint4 *>(blk);
    const uint8_t *scb = reinterpret_cast<const uint8_t *>(blk) + 4;
    int sc[8], mn[8];
#pragma unroll
    for (int s = 0; s < 4; s++) {
        sc[s] = scb[s] & 63;
        mn[s] = scb[s + 4] & 63;
        sc[s + 4] = (scb[s + 8] & 0xF) | ((scb[s] >> 6) << 4);
        mn[s + 4] = (scb[s + 8] >> 4) | ((scb[s + 4] >> 6) << 4);
    }
    const uint32_t *xq = reinterpret_cast<const uint32_t *>(x.qs + g * 256);
    const int16_t *bs = x.bs + g * 16;
    int isum = 0, imin = 0;
#pragma unroll
    for (int p = 0; p < 4; p++) {
        const uint4 qa = *reinterpret_cast<const uint4 *>(blk + 16 + 32 * p);
        const uint4 qb = *reinterpret_cast<const uint4 *>(blk + 32 + 32 * p);
        const uint32_t w[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
        int dlo = 0, dhi = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            dlo = sdot4(w[i] & 0x0F0F0F0Fu, xq[16 * p + i], dlo);
            dhi = sdot4((w[i] >> 4) & 0x0F0F0F0Fu, xq[16 * p + 8 + i], dhi);
        }
        isum += sc[2 * p] * dlo + sc[2 * p + 1] * dhi;
        imin += mn[2 * p] * ((int)bs[4 * p] + (int)bs[4 * p + 1]) +
                mn[2 * p + 1] * ((int)bs[4 * p + 2] + (int)bs[4 * p + 3]);
    }
    const double dx = (double)x.d[g];
    const double dw = (double)h2f((uint16_t)(hdr.x & 0xffff));
    const double dm = (double)h2f((uint16_t)(hdr.x >> 16));
    return (dw * dx) * (double)isum - (dm * dx) * (double)imin;
}

// Q6_K block at a 2-aligned LDS offset against Q8_K group g.  Codes are
// taken unsigned (0..63) and the -32 offset is folded through the bsums:
// sum((c-32)*x) = sum(c*x) - 32*bsum, exact in integers.
__device__ __forceinline__ double term_q6k(const char *lds, uint32_t off, const ActView &x, uint32_t g) {
    const uint32_t *xq = reinterpret_cast<const uint32_t *>(x.qs + g * 256);
    const int16_t *bs = x.bs + g * 16;
    int isum = 0;
#pragma unroll
    for (int n = 0; n < 2; n++) {
#pragma unroll
        for (int h = 0; h < 2; h++) {          // lbase = 16h
            int dot[4] = {0, 0, 0, 0};          // quarters t = 0..3
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t qla = lds_u32(lds, off + 64 * n + 16 * h + 4 * i);
                const uint32_t qlb = lds_u32(lds, off + 64 * n + 32 + 16 * h + 4 * i);
                const uint32_t qh = lds_u32(lds, off + 128 + 32 * n + 16 * h + 4 * i);
                const uint32_t c0 = (qla & 0x0F0F0F0Fu) | ((qh << 4) & 0x30303030u);
                const uint32_t c1 = (qlb & 0x0F0F0F0Fu) | ((qh << 2) & 0x30303030u);
                const uint32_t c2 = ((qla >> 4) & 0x0F0F0F0Fu) | (qh & 0x30303030u);
                const uint32_t c3 = ((qlb >> 4) & 0x0F0F0F0Fu) | ((qh >> 2) & 0x30303030u);
                // element base of quarter t: 128n + 32t + 16h + 4i
                dot[0] = sdot4(c0, xq[(128 * n + 0 + 16 * h) / 4 + i], dot[0]);
                dot[1] = sdot4(c1, xq[(128 * n + 32 + 16 * h) / 4 + i], dot[1]);
                dot[2] = sdot4(c2, xq[(128 * n + 64 + 16 * h) / 4 + i], dot[2]);
                dot[3] = sdot4(c3, xq[(128 * n + 96 + 16 * h) / 4 + i], dot[3]);
            }
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const int j = 8 * n + 2 * t + h;  // 16-element sub-block
                const int sc = (int)(int8_t)(lds_u16(lds, off + 192 + (j & ~1)) >> (8 * (j & 1)));
                isum += sc * (dot[t] - 32 * (int)bs[j]);
            }
        }
    }
    const double dw = (double)h2f(lds_u16(lds, off + 208));
    return (dw * (double)x.d[g]) * (double)isum;
}

// 8 Q8_0 blocks (272 B, 16-aligned item) against Q8_0 activation blocks 8g..8g+7
__device__ __forceinline__ double term_q80(const char *lds, uint32_t off, const ActView &x, uint32_t g) {
    double acc = 0.0;
#pragma unroll
    for (int b = 0; b < 8; b++) {
        const uint32_t bo = off + 34 * b;
        const uint32_t *xq = reinterpret_cast<const uint32_t *>(x.qs + (8 * g + b) * 32);
        int isum = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) isum = sdot4(lds_u32(lds, bo + 2 + 4 * i), xq[i], isum);
        const double dw = (double)h2f(lds_u16(lds, bo));
        acc += (dw * (double)x.d[8 * g + b]) * (double)isum;
    }
    return acc;
}

__device__ __forceinline__ double term_bf16(const char *lds, uint32_t off, const ActView &x, uint32_t g) {
    const uint32_t *w = reinterpret_cast<const uint32_t *>(lds + off);
    const uint32_t *xx = reinterpret_cast<const uint32_t *>(x.bf + g * 256);
    double acc = 0.0;
    for (int i = 0; i < 128; i++) {
        const uint32_t ww = w[i], xv = xx[i];
        acc = fma((double)__uint_as_float(ww << 16), (double)__uint_as_float(xv << 16), acc);
        acc = fma((double)__uint_as_float(ww & 0xffff0000u), (double)__uint_as_float(xv & 0xffff0000u), acc);
    }
    return acc;
}

__device__ __forceinline__ double term_f32(const char *lds, uint32_t off, const ActView &x, uint32_t g) {
    const float *w = reinterpret_cast<const float *>(lds + off);
    const float *xx = x.f + g * 256;
    double acc = 0.0;
    for (int i = 0; i < 256; i++) acc = fma((double)w[i], (double)xx[i], acc);
    return acc;
}

__device__ __forceinline__ double group_term(int type, const char *lds, uint32_t off, const ActView &x, uint32_t g) {
    switch (type) {
    case SINTER_Q4_K: return term_q4k(lds + off, x, g);
    case SINTER_Q6_K: return term_q6k(lds, off, x, g);
    case SINTER_Q8_0: return term_q80(lds, off, x, g);
    case SINTER_BF16: return term_bf16(lds, off, x, g);
    default: return term_f32(lds, off, x, g);
    }
}

// ------------------------------------------------------------ row ranges

// Row cut for workgroup w of n: the global row nearest to byte w*T/n of the
// concatenated (byte-weighted) row space.
__device__ __forceinline__ uint32_t row_cut(const sinter_gemv_args &a, const uint32_t *rb_eff,
                                            uint64_t total, uint32_t w, uint32_t n) {
    if (w >= n) {
        uint32_t r = 0;
        for (int s = 0; s < a.n_seg; s++) r += a.seg[s].rows;
        return r;
    }
    const uint64_t target = total * w / n;
    uint64_t acc = 0;
    uint32_t rows = 0;
    for (int s = 0; s < a.n_seg; s++) {
        const uint64_t sb = (uint64_t)a.seg[s].rows * rb_eff[s];
        if (target < acc + sb) return rows + (uint32_t)((target - acc + rb_eff[s] / 2) / rb_eff[s]);
        acc += sb;
        rows += a.seg[s].rows;
    }
    return rows;
}

struct Tile {
    int seg;
    uint32_t r0, nr;           // output rows [r0, r0+nr) of segment seg
    uint32_t skew_a, n16_a;    // range A (w): byte skew in its first uint4, uint4 count
    uint32_t skew_b, n16_b;    // range B (w2, SwiGLU only)
    const uint4 *src_a, *src_b;
};

// ------------------------------------------------------------ the op

// Payload checks every block evaluates identically (so an error leaves no
// block behind at the next grid barrier).
__device__ __forceinline__ bool gemv_args_ok(const sinter_gemv_args &a) {
    if (a.n_seg < 1 || a.n_seg > SINTER_GEMV_MAX_SEG) return false;
    if (a.K == 0 || (a.K & 255u) != 0) return false;
    const int vt = vec_dot_type(a.seg[0].type);
    const uint32_t need = vt == SINTER_Q8_K ? a.K + (a.K / 256) * 4 + (a.K / 16) * 2
                        : vt == SINTER_Q8_0 ? a.K + (a.K / 32) * 4
                        : vt == SINTER_BF16 ? a.K * 2 : a.K * 4;
    if (need > QBUF_BYTES) return false;
    if (a.pro == SINTER_PRO_GATED && (a.gn_log2d < 2 || a.gn_log2d > 8)) return false;
    for (int s = 0; s < a.n_seg; s++) {
        const sinter_gemv_seg &g = a.seg[s];
        if (vec_dot_type(g.type) != vt) return false;
        const uint32_t rbe = (uint32_t)sinter_row_bytes_dev(g.type, a.K) * (g.epi == SINTER_EPI_SWIGLU ? 2u : 1u);
        if (rbe == 0 || rbe > TILE_BYTES - 64) return false;
        if ((a.K / 256) * (g.epi == SINTER_EPI_SWIGLU ? 2u : 1u) > BLOCK_THREADS) return false;
        if (g.epi == SINTER_EPI_CONV && (g.dconv < 2 || g.dconv > 8)) return false;
    }
    return true;
}

__device__ void op_gemv(const sinter_instr &ins, char *lds, unsigned *err) {
    const sinter_gemv_args &a = *reinterpret_cast<const sinter_gemv_args *>(ins.payload);
    const uint32_t rel = blockIdx.x - ins.block_lo, nblk = ins.block_hi - ins.block_lo;
    if (!gemv_args_ok(a)) {
        if (rel == 0 && threadIdx.x == 0) raise_error(err, SINTER_E_BAD_SHAPE, ins.dbg_node);
        return;
    }
    const uint32_t K = a.K, G = K / 256;
    double *red = reinterpret_cast<double *>(lds);
    char *qbuf = lds + RED_BYTES;
    char *tbuf0 = qbuf + QBUF_BYTES;
    char *tbuf1 = tbuf0 + TILE_BYTES;
    double *cb = reinterpret_cast<double *>(tbuf1 + TILE_BYTES);
    float *rowv = reinterpret_cast<float *>(cb + 256);      // per-tile row results
    const int vt = vec_dot_type(a.seg[0].type);

    // byte-weighted row space
    uint32_t rb[SINTER_GEMV_MAX_SEG], rb_eff[SINTER_GEMV_MAX_SEG];
    uint64_t total = 0;
    for (int s = 0; s < a.n_seg; s++) {
        rb[s] = (uint32_t)sinter_row_bytes_dev(a.seg[s].type, K);
        rb_eff[s] = rb[s] * (a.seg[s].epi == SINTER_EPI_SWIGLU ? 2u : 1u);
        total += (uint64_t)a.seg[s].rows * rb_eff[s];
    }
    const uint32_t row_lo = row_cut(a, rb_eff, total, rel, nblk);
    const uint32_t row_hi = row_cut(a, rb_eff, total, rel + 1, nblk);

    // tile iterator over [row_lo, row_hi) of the concatenated row space
    auto make_tile = [&](uint32_t grow, Tile &t) -> bool {
        if (grow >= row_hi) return false;
        uint32_t base = 0;
        int s = 0;
        while (s < a.n_seg && grow >= base + a.seg[s].rows) { base += a.seg[s].rows; s++; }
        const sinter_gemv_seg &sg = a.seg[s];
        const bool sw = sg.epi == SINTER_EPI_SWIGLU;
        const uint32_t items_per_row = G * (sw ? 2u : 1u);
        uint32_t nr = BLOCK_THREADS / items_per_row;
        const uint32_t by_bytes = (TILE_BYTES - 64) / rb_eff[s];
        if (by_bytes < nr) nr = by_bytes;
        const uint32_t seg_end = base + sg.rows < row_hi ? base + sg.rows : row_hi;
        if (grow + nr > seg_end) nr = seg_end - grow;
        t.seg = s;
        t.r0 = grow - base;
        t.nr = nr;
        const uintptr_t A = reinterpret_cast<uintptr_t>(sg.w) + (uintptr_t)t.r0 * rb[s];
        t.src_a = reinterpret_cast<const uint4 *>(A & ~(uintptr_t)15);
        t.skew_a = (uint32_t)(A & 15);
        t.n16_a = (t.skew_a + nr * rb[s] + 15) / 16;
        if (sw) {
            const uintptr_t B = reinterpret_cast<uintptr_t>(sg.w2) + (uintptr_t)t.r0 * rb[s];
            t.src_b = reinterpret_cast<const uint4 *>(B & ~(uintptr_t)15);
            t.skew_b = (uint32_t)(B & 15);
            t.n16_b = (t.skew_b + nr * rb[s] + 15) / 16;
        } else {
            t.src_b = nullptr; t.skew_b = 0; t.n16_b = 0;
        }
        return true;
    };

    uint4 stage[MAX_LD];
    auto issue = [&](const Tile &t) {
#pragma unroll
        for (int k = 0; k < MAX_LD; k++) {
            const uint32_t i = threadIdx.x + k * BLOCK_THREADS;
            if (i < t.n16_a) stage[k] = t.src_a[i];
            else if (i < t.n16_a + t.n16_b) stage[k] = t.src_b[i - t.n16_a];
        }
    };
    auto commit = [&](const Tile &t, char *buf) {
#pragma unroll
        for (int k = 0; k < MAX_LD; k++) {
            const uint32_t i = threadIdx.x + k * BLOCK_THREADS;
            if (i < t.n16_a + t.n16_b) reinterpret_cast<uint4 *>(buf)[i] = stage[k];
        }
    };

    Tile cur{}, nxt{};
    bool have = make_tile(row_lo, cur);
    if (have) issue(cur);   // first weight loads overlap the prologue

    const bool write_x = (a.pro == SINTER_PRO_EMBED) && rel == 0 && a.x_out != nullptr;
    gemv_prologue(a, vt, write_x, qbuf, red, err);
    const ActView xv = act_view(qbuf, K, vt);

    // greedy argmax state (thread 0 of the block)
    float best_v = -INFINITY;
    int32_t best_i = 0x7fffffff;

    if (have) commit(cur, tbuf0);
    __syncthreads();
    int bi = 0;
    uint32_t grow = row_lo;
    while (have) {
        char *buf = bi ? tbuf1 : tbuf0;
        const bool more = make_tile(grow + cur.nr, nxt);
        if (more) issue(nxt);
        const sinter_gemv_seg &sg = a.seg[cur.seg];
        const bool sw = sg.epi == SINTER_EPI_SWIGLU;
        const uint32_t per = G * (sw ? 2u : 1u);
        const uint32_t n_items = cur.nr * per;
        const uint32_t gb = group_bytes(sg.type);
        const uint32_t rbs = rb[cur.seg];
        for (uint32_t it = threadIdx.x; it < n_items; it += BLOCK_THREADS) {
            const uint32_t rr = it / per, k = it - rr * per;
            const bool up = k >= G;
            const uint32_t g = up ? k - G : k;
            const uint32_t off = up ? (cur.n16_a * 16 + cur.skew_b + rr * rbs + g * gb)
                                    : (cur.skew_a + rr * rbs + g * gb);
            cb[it] = group_term(sg.type, buf, off, xv, g);
        }
        __syncthreads();
        // row results: ascending fp64 sum of the group terms
        if (threadIdx.x < cur.nr) {
            const uint32_t rr = threadIdx.x, r = cur.r0 + rr;
            double acc = 0.0;
            for (uint32_t g = 0; g < G; g++) acc += cb[rr * per + g];
            const float dot = (float)acc;
            float y = dot;
            if (sw) {
                double acc2 = 0.0;
                for (uint32_t g = 0; g < G; g++) acc2 += cb[rr * per + G + g];
                y = dev_silu(dot) * (float)acc2;
            } else if (sg.epi == SINTER_EPI_RESID) {
                y = sg.aux[r] + dot;
            } else if (sg.epi == SINTER_EPI_CONV) {
                // causal conv over {state[0..dc-2], dot}, fp64 sum rounded once,
                // then silu; the state shifts by one tap (this block owns row r)
                const uint32_t dc = sg.dconv;
                float *st = sg.aux + (size_t)r * (dc - 1);
                const float *cw = static_cast<const float *>(sg.w2) + (size_t)r * dc;
                float win[8];
                for (uint32_t j = 0; j + 1 < dc; j++) win[j] = st[j];
                win[dc - 1] = dot;
                double cacc = 0.0;
                for (uint32_t j = 0; j < dc; j++) cacc += (double)win[j] * (double)cw[j];
                y = dev_silu((float)cacc);
                for (uint32_t j = 0; j + 1 < dc; j++) st[j] = win[j + 1];
            }
            sg.y[r] = y;
            rowv[rr] = y;
        }
        if (sg.epi == SINTER_EPI_ARGMAX) {
            __syncthreads();
            if (threadIdx.x == 0) {
                for (uint32_t rr = 0; rr < cur.nr; rr++) {
                    const float v = rowv[rr];
                    if (v > best_v) { best_v = v; best_i = (int32_t)(cur.r0 + rr); }
                }
            }
        }
        if (more) commit(nxt, bi ? tbuf0 : tbuf1);
        __syncthreads();
        grow += cur.nr;
        cur = nxt;
        have = more;
        bi ^= 1;
    }

    // greedy argmax: last-arriving block reduces the per-block partials
    bool any_argmax = false;
    for (int s = 0; s < a.n_seg; s++) any_argmax |= a.seg[s].epi == SINTER_EPI_ARGMAX;
    if (any_argmax && threadIdx.x == 0 && rel >= static_cast<sinter_argmax_ws *>(a.epi_ws)->capacity) {
        raise_error(err, SINTER_E_BAD_SHAPE, ins.dbg_node);
    } else if (any_argmax && threadIdx.x == 0) {
        sinter_argmax_ws *ws = static_cast<sinter_argmax_ws *>(a.epi_ws);
        ws->part_val[rel] = best_v;
        ws->part_idx[rel] = best_i;
        fence_release_agent();
        const unsigned old = __hip_atomic_fetch_add(ws->count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old == nblk - 1) {
            fence_acquire_agent();
            float bv = -INFINITY;
            int32_t bidx = 0x7fffffff;
            for (uint32_t w = 0; w < nblk; w++) {
                const float v = __hip_atomic_load(ws->part_val + w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                const int32_t i = __hip_atomic_load(ws->part_idx + w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (v > bv || (v == bv && i < bidx)) { bv = v; bidx = i; }
            }
            sinter_pass_cell *pc = reinterpret_cast<sinter_pass_cell *>(ws->pass_cell);
            if (ws->history && (uint32_t)pc->steps < ws->history_cap) ws->history[pc->steps] = bidx;
            pc->steps += 1;
            pc->token = bidx;
            pc->pos += 1;
            __hip_atomic_store(ws->count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            fence_release_agent();
        }
    }
    __syncthreads();
}

}  // namespace sinter
