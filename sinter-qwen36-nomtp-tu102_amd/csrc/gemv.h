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
// workgroup streams its rows through three 36 KiB LDS tiles with gfx950
// LDS-DMA (global_load_lds_dwordx4: 16 B per lane straight into LDS, no
// VGPRs), two tiles in flight while one is computed; compute reads the
// (arbitrarily aligned) ggml blocks from LDS, one wave per row, lanes over
// 32-element units, and a wave-wide fp64 sum per row.  Row results stay in
// LDS; the epilogues run once over the block's rows at the end.
//
// Declared numerics (oracle/oracle.c): integer block dots are exact; each
// unit's term is an fp64 expression of exact integers and the f16/f32
// scales; a row is the fp64 sum of its terms rounded to fp32 once.  The
// oracle sums in ascending order, the kernel in wave order; both round the
// same ~1e-16-accurate fp64 value, so outputs agree to the last bit except
// with probability ~1e-8 per row (1 ulp then).
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
// Padded so that lanes working on different groups/chunks start on
// different LDS banks (an unpadded 256-byte group stride puts every group on
// bank 0 and serialises the activation reads):
//   Q8_K: int8 codes, group g at g*ACT_GSTRIDE | d f32[G] | bsums i16[16G]
//   Q8_0: int8 codes, group g at g*ACT_GSTRIDE | d f32[K/32] (f16-rounded)
//   BF16: 64-element chunk c at c*ACT_BF_CSTRIDE (u16)
//   F32:  64-element chunk c at c*ACT_F_CSTRIDE
constexpr uint32_t ACT_GSTRIDE = 272;
constexpr uint32_t ACT_BF_CSTRIDE = 144;
constexpr uint32_t ACT_F_CSTRIDE = 272;
__host__ __device__ inline uint32_t act_bytes(int vt, uint32_t K) {
    if (vt == SINTER_Q8_K) return (K / 256) * ACT_GSTRIDE + (K / 256) * 4 + (K / 16) * 2;
    if (vt == SINTER_Q8_0) return (K / 256) * ACT_GSTRIDE + (K / 32) * 4;
    if (vt == SINTER_BF16) return (K / 64) * ACT_BF_CSTRIDE;
    return (K / 64) * ACT_F_CSTRIDE;
}
struct ActView {
    const char *q;       // codes / bf16 / f32 chunks
    const float *d;
    const int16_t *bs;
};
__device__ __forceinline__ ActView act_view(char *q, uint32_t K, int vt) {
    ActView v{};
    v.q = q;
    v.d = reinterpret_cast<const float *>(q + (K / 256) * ACT_GSTRIDE);
    v.bs = reinterpret_cast<const int16_t *>(q + (K / 256) * ACT_GSTRIDE + (K / 256) * 4);
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
    float *qd = reinterpret_cast<float *>(q + (K / 256) * ACT_GSTRIDE);
    int16_t *qb = reinterpret_cast<int16_t *>(q + (K / 256) * ACT_GSTRIDE + (K / 256) * 4);
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
            *reinterpret_cast<uint32_t *>(q + act_qoff(e)) = packed;
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
            *reinterpret_cast<uint32_t *>(q + act_qoff(e)) = packed;
            if ((lane & 7) == 0) qd[e / 32] = h2f(f2h(d));
        } else if (vt == SINTER_BF16) {
            uint16_t *bf = reinterpret_cast<uint16_t *>(q + (e >> 6) * ACT_BF_CSTRIDE) + (e & 63);
#pragma unroll
            for (int i = 0; i < 4; i++) bf[i] = f2bf(t[i]);
        } else {
            float *f = reinterpret_cast<float *>(q + (e >> 6) * ACT_F_CSTRIDE) + (e & 63);
#pragma unroll
            for (int i = 0; i < 4; i++) f[i] = t[i];
        }
    }
    __syncthreads();
}

// ------------------------------------------------------------ item terms
// A weight row is a sequence of items: one 256-element group for the
// quantised types (one Q4_K / Q6_K block, eight Q8_0 blocks), 64 elements
// for BF16 / F32.  One lane computes one item's term: an fp64 expression of
// exact integer block dots and the f16/f32 scales (a float sum of exact
// products for BF16/F32).  A row is the ascending fp64 sum of its item terms,
// rounded to fp32 once -- the fold oracle/oracle.c declares.

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// n words (4 bytes each) at a 2-aligned LDS byte offset
template <int N>
__device__ __forceinline__ void lds_words(const char *lds, uint32_t off, uint32_t w[N]) {
    const uint32_t *p = reinterpret_cast<const uint32_t *>(lds + (off & ~3u));
    const uint32_t sh = off & 3u;
    uint32_t d[N + 1];
#pragma unroll
    for (int i = 0; i <= N; i++) d[i] = p[i];
#pragma unroll
    for (int i = 0; i < N; i++) w[i] = __builtin_amdgcn_alignbyte(d[i + 1], d[i], sh);
}

__device__ __forceinline__ uint32_t item_elems(int t) { return (t == SINTER_BF16 || t == SINTER_F32) ? 64u : 256u; }
__device__ __forceinline__ uint32_t item_bytes(int t) {
    switch (t) {
    case SINTER_Q4_K: return 144;
    case SINTER_Q6_K: return 210;
    case SINTER_Q8_0: return 272;
    case SINTER_BF16: return 128;
    default: return 256;
    }
}

// Q4_K block (16-aligned in LDS) against Q8_K group g
__device__ __forceinline__ double term_q4k(const char *blk, const ActView &x, uint32_t g) {
    const uint4 hdr = *reinterpret_cast<const uint4 *>(blk);
    const uint32_t sw[3] = {hdr.y, hdr.z, hdr.w};   // scales[0..11]
    auto byte = [&](uint32_t i) -> int { return (int)((sw[i >> 2] >> (8 * (i & 3))) & 0xff); };
    const uint32_t *xq = reinterpret_cast<const uint32_t *>(x.q + g * ACT_GSTRIDE);
    const int16_t *bs = x.bs + g * 16;
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
        const uint4 qa = *reinterpret_cast<const uint4 *>(blk + 16 + 32 * p);
        const uint4 qb = *reinterpret_cast<const uint4 *>(blk + 32 + 32 * p);
        const uint32_t w[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
        int dlo = 0, dhi = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            dlo = sdot4(w[i] & 0x0F0F0F0Fu, xq[16 * p + i], dlo);
            dhi = sdot4((w[i] >> 4) & 0x0F0F0F0Fu, xq[16 * p + 8 + i], dhi);
        }
        isum += sc0 * dlo + sc1 * dhi;
        imin += m0 * ((int)bs[4 * p] + (int)bs[4 * p + 1]) + m1 * ((int)bs[4 * p + 2] + (int)bs[4 * p + 3]);
    }
    const double dx = (double)x.d[g];
    const double dw = (double)h2f((uint16_t)(hdr.x & 0xffff));
    const double dm = (double)h2f((uint16_t)(hdr.x >> 16));
    return (dw * dx) * (double)isum - (dm * dx) * (double)imin;
}

// Q6_K block at a 2-aligned LDS offset against Q8_K group g.  Codes are
// taken unsigned (0..63) and the -32 offset folds through the bsums:
// sum((c-32)*x) = sum(c*x) - 32*bsum, exact in integers.
__device__ __forceinline__ double term_q6k(const char *lds, uint32_t off, const ActView &x, uint32_t g) {
    const uint32_t *xq = reinterpret_cast<const uint32_t *>(x.q + g * ACT_GSTRIDE);
    const int16_t *bs = x.bs + g * 16;
    uint32_t scw[4];
    lds_words<4>(lds, off + 192, scw);                 // int8 scales[16]
    int isum = 0;
#pragma unroll
    for (int n = 0; n < 2; n++) {
        uint32_t qa[8], qb[8], qh[8];
        lds_words<8>(lds, off + 64 * n, qa);           // ql[64n .. 64n+32)
        lds_words<8>(lds, off + 64 * n + 32, qb);      // ql[64n+32 .. 64n+64)
        lds_words<8>(lds, off + 128 + 32 * n, qh);     // qh[32n .. 32n+32)
        int dot[4][2] = {{0, 0}, {0, 0}, {0, 0}, {0, 0}};  // [quarter][16-element half]
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t c0 = (qa[i] & 0x0F0F0F0Fu) | ((qh[i] << 4) & 0x30303030u);
            const uint32_t c1 = (qb[i] & 0x0F0F0F0Fu) | ((qh[i] << 2) & 0x30303030u);
            const uint32_t c2 = ((qa[i] >> 4) & 0x0F0F0F0Fu) | (qh[i] & 0x30303030u);
            const uint32_t c3 = ((qb[i] >> 4) & 0x0F0F0F0Fu) | ((qh[i] >> 2) & 0x30303030u);
            const int hf = i >> 2;                     // l = 4i.. : half hf of each quarter
            dot[0][hf] = sdot4(c0, xq[(128 * n + 0) / 4 + i], dot[0][hf]);
            dot[1][hf] = sdot4(c1, xq[(128 * n + 32) / 4 + i], dot[1][hf]);
            dot[2][hf] = sdot4(c2, xq[(128 * n + 64) / 4 + i], dot[2][hf]);
            dot[3][hf] = sdot4(c3, xq[(128 * n + 96) / 4 + i], dot[3][hf]);
        }
#pragma unroll
        for (int t = 0; t < 4; t++) {
#pragma unroll
            for (int hf = 0; hf < 2; hf++) {
                const int j = 8 * n + 2 * t + hf;      // 16-element sub-block
                const int sc = (int)(int8_t)((scw[j >> 2] >> (8 * (j & 3))) & 0xff);
                isum += sc * (dot[t][hf] - 32 * (int)bs[j]);
            }
        }
    }
    const double dw = (double)h2f(lds_u16(lds, off + 208));
    return (dw * (double)x.d[g]) * (double)isum;
}

// 8 Q8_0 blocks (272 B group) against Q8_0 activation blocks 8g..8g+7,
// block terms summed in ascending order inside the group
__device__ __forceinline__ double term_q80(const char *lds, uint32_t off, const ActView &x, uint32_t g) {
    double acc = 0.0;
#pragma unroll
    for (int b = 0; b < 8; b++) {
        const uint32_t bo = off + 34 * b;
        uint32_t w[8];
        lds_words<8>(lds, bo + 2, w);
        const uint32_t *xq = reinterpret_cast<const uint32_t *>(x.q + g * ACT_GSTRIDE + 32 * b);
        int isum = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) isum = sdot4(w[i], xq[i], isum);
        const double dw = (double)h2f(lds_u16(lds, bo));
        acc += (dw * (double)x.d[8 * g + b]) * (double)isum;
    }
    return acc;
}

// 64 bf16 elements (128 B, 16-aligned), products exact in fp64, ascending
__device__ __forceinline__ double term_bf16(const char *lds, uint32_t off, const ActView &x, uint32_t k) {
    const uint4 *w = reinterpret_cast<const uint4 *>(lds + off);
    const uint4 *xx = reinterpret_cast<const uint4 *>(x.q + k * ACT_BF_CSTRIDE);
    double acc = 0.0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const uint4 a = w[i], b = xx[i];
        const uint32_t aw[4] = {a.x, a.y, a.z, a.w}, bw[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            acc += (double)__uint_as_float(aw[j] << 16) * (double)__uint_as_float(bw[j] << 16);
            acc += (double)__uint_as_float(aw[j] & 0xffff0000u) * (double)__uint_as_float(bw[j] & 0xffff0000u);
        }
    }
    return acc;
}

// 64 f32 elements (256 B, 16-aligned), products exact in fp64, ascending
__device__ __forceinline__ double term_f32(const char *lds, uint32_t off, const ActView &x, uint32_t k) {
    const float4 *w = reinterpret_cast<const float4 *>(lds + off);
    const float4 *xx = reinterpret_cast<const float4 *>(x.q + k * ACT_F_CSTRIDE);
    double acc = 0.0;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const float4 a = w[i], b = xx[i];
        acc += (double)a.x * (double)b.x;
        acc += (double)a.y * (double)b.y;
        acc += (double)a.z * (double)b.z;
        acc += (double)a.w * (double)b.w;
    }
    return acc;
}

__device__ __forceinline__ double item_term(int type, const char *tile, uint32_t off, const ActView &x, uint32_t k) {
    switch (type) {
    case SINTER_Q4_K: return term_q4k(tile + off, x, k);
    case SINTER_Q6_K: return term_q6k(tile, off, x, k);
    case SINTER_Q8_0: return term_q80(tile, off, x, k);
    case SINTER_BF16: return term_bf16(tile, off, x, k);
    default: return term_f32(tile, off, x, k);
    }
}

// ------------------------------------------------------------ row ranges and tiles

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
#pragma unroll
    for (int s = 0; s < SINTER_GEMV_MAX_SEG; s++) {
        if (s < a.n_seg) {
            const uint64_t sb = (uint64_t)a.seg[s].rows * rb_eff[s];
            if (target < acc + sb) return rows + (uint32_t)((target - acc + rb_eff[s] / 2) / rb_eff[s]);
            acc += sb;
            rows += a.seg[s].rows;
        }
    }
    return rows;
}

struct Tile {
    uint32_t seg;
    uint32_t r0, nr;           // output rows [r0, r0+nr) of segment seg
    uint32_t skew_a, n16_a;    // range A (w): byte skew in its first uint4, uint4 count
    uint32_t skew_b, n16_b;    // range B (w2, SwiGLU only)
    const uint4 *src_a, *src_b;
};

__device__ __forceinline__ uint32_t uni(uint32_t v) { return __builtin_amdgcn_readfirstlane(v); }

// per-segment geometry, read from the payload (scalar loads; no private arrays)
__device__ __forceinline__ uint32_t seg_rb(const sinter_gemv_args &a, uint32_t s) {
    return (uint32_t)sinter_row_bytes_dev(a.seg[s].type, a.K);
}
__device__ __forceinline__ uint32_t seg_rb_eff(const sinter_gemv_args &a, uint32_t s) {
    return seg_rb(a, s) * (a.seg[s].epi == SINTER_EPI_SWIGLU ? 2u : 1u);
}
// segment holding global row grow, and its first global row
__device__ __forceinline__ uint32_t seg_of(const sinter_gemv_args &a, uint32_t grow, uint32_t &base) {
    uint32_t s = 0, b = 0;
    while (s + 1 < a.n_seg && grow >= b + a.seg[s].rows) { b += a.seg[s].rows; s++; }
    base = b;
    return s;
}

// Tile starting at global row grow (caller checks grow < row_hi).
__device__ __forceinline__ Tile tile_at(const sinter_gemv_args &a, uint32_t grow, uint32_t row_hi) {
    Tile t;
    uint32_t base;
    t.seg = uni(seg_of(a, grow, base));
    base = uni(base);
    const sinter_gemv_seg &sg = a.seg[t.seg];
    const uint32_t rb = seg_rb(a, t.seg);
    uint32_t nr = (TILE_BYTES - 64) / seg_rb_eff(a, t.seg);
    // one lane per item: at most BLOCK_THREADS items per tile (a longer row
    // still gets a tile of its own and is looped over)
    const uint32_t ipr = a.K / item_elems(sg.type) * (sg.epi == SINTER_EPI_SWIGLU ? 2u : 1u);
    nr = min(nr, max(1u, BLOCK_THREADS / ipr));
    const uint32_t seg_end = min(base + sg.rows, row_hi);
    if (nr > RES_CAP) nr = RES_CAP;
    if (grow + nr > seg_end) nr = seg_end - grow;
    nr = uni(nr);
    t.r0 = grow - base;
    t.nr = nr;
    const uintptr_t A = reinterpret_cast<uintptr_t>(sg.w) + (uintptr_t)t.r0 * rb;
    t.src_a = reinterpret_cast<const uint4 *>(A & ~(uintptr_t)15);
    t.skew_a = (uint32_t)(A & 15);
    t.n16_a = (t.skew_a + nr * rb + 15) / 16;
    if (sg.epi == SINTER_EPI_SWIGLU) {
        const uintptr_t B = reinterpret_cast<uintptr_t>(sg.w2) + (uintptr_t)t.r0 * rb;
        t.src_b = reinterpret_cast<const uint4 *>(B & ~(uintptr_t)15);
        t.skew_b = (uint32_t)(B & 15);
        t.n16_b = (t.skew_b + nr * rb + 15) / 16;
    } else {
        t.src_b = nullptr; t.skew_b = 0; t.n16_b = 0;
    }
    return t;
}

// One 1 KiB LDS-DMA chunk per wave: lane l's 16 bytes at src land at
// lds_base + 16*l.  Issued from inline asm so the compiler does not treat the
// pending DMA as aliasing every later LDS read (it would insert vmcnt(0)
// before them and serialise the pipeline); the tile loop below waits for it
// explicitly.  M0 (the LDS base of the DMA) is restored before the asm ends.
__device__ __forceinline__ void lds_dma16(const void *src, uint32_t lds_base) {
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "global_load_lds_dwordx4 %2, off\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "s"(lds_base), "v"(src)
        : "memory");
}

// LDS-DMA one tile into a 36 KiB buffer: every wave issues exactly
// TILE_CPW 1-KiB chunks (lanes past the tile re-read its first 16 bytes into
// the unused tail of the buffer), so the number of outstanding loads per wave
// is a compile-time constant and the tile waits below can be partial.
__device__ __forceinline__ void tile_issue(const Tile &t, char *buf) {
    const uint32_t w = uni(wave_id()), lane = lane_id();
    const uint32_t n16 = t.n16_a + t.n16_b;
    const uint32_t base = (uint32_t)(uintptr_t)(lds_void *)buf;
#pragma unroll
    for (uint32_t k = 0; k < TILE_CPW; k++) {
        const uint32_t j = w + 4 * k;
        const uint32_t idx = j * 64 + lane;
        const uint4 *src = idx < t.n16_a ? t.src_a + idx : (idx < n16 ? t.src_b + (idx - t.n16_a) : t.src_a);
        lds_dma16(src, uni(base + j * 1024));
    }
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ void wait_lgkm0() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// ------------------------------------------------------------ the op

// Payload checks every block evaluates identically (so an error leaves no
// block behind at the next grid barrier).
__device__ __forceinline__ bool gemv_args_ok(const sinter_gemv_args &a) {
    if (a.n_seg < 1 || a.n_seg > SINTER_GEMV_MAX_SEG) return false;
    if (a.K == 0 || (a.K & 255u) != 0) return false;
    const int vt = vec_dot_type(a.seg[0].type);
    if (act_bytes(vt, a.K) > QBUF_BYTES) return false;
    if (a.pro == SINTER_PRO_GATED && (a.gn_log2d < 2 || a.gn_log2d > 8)) return false;
    for (int s = 0; s < a.n_seg; s++) {
        const sinter_gemv_seg &g = a.seg[s];
        if (vec_dot_type(g.type) != vt) return false;
        const uint32_t rbe = (uint32_t)sinter_row_bytes_dev(g.type, a.K) * (g.epi == SINTER_EPI_SWIGLU ? 2u : 1u);
        if (rbe == 0 || rbe > TILE_BYTES - 64) return false;
        if ((a.K / item_elems(g.type)) * (g.epi == SINTER_EPI_SWIGLU ? 2u : 1u) > CB_CAP) return false;
        if (g.epi == SINTER_EPI_CONV && (g.dconv < 2 || g.dconv > 8)) return false;
    }
    return true;
}

// Apply the epilogues to the buffered rows [row0, row0 + n) and store them;
// greedy-argmax candidates fold into (bv, bi).  All threads.
__device__ void gemv_flush(const sinter_gemv_args &a, uint32_t row0, uint32_t n, float &bv, int32_t &bi) {
    for (uint32_t i = threadIdx.x; i < n; i += BLOCK_THREADS) {
        const uint32_t grow = row0 + i;
        uint32_t base;
        const uint32_t s = seg_of(a, grow, base);
        const sinter_gemv_seg &sg = a.seg[s];
        const uint32_t r = grow - base;
        const float dot = g_res[2 * i];
        float y = dot;
        if (sg.epi == SINTER_EPI_SWIGLU) {
            y = dev_silu(dot) * g_res[2 * i + 1];
        } else if (sg.epi == SINTER_EPI_RESID) {
            y = sg.aux[r] + dot;
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
        sg.y[r] = y;
    }
}

// Compute one landed tile: one lane per (virtual row, item) writes the item
// term to LDS, then one lane per virtual row sums its terms in ascending
// order.  A SwiGLU tile has nr gate rows then nr up rows.  Row results go to
// g_res[2*(slot0 + row) + {0: gate/plain, 1: up}].
template <int TYPE>
__device__ __forceinline__ void tile_compute_t(const Tile &t, const char *buf, uint32_t ipr, uint32_t nv,
                                               uint32_t rb, uint32_t slot0, const ActView &x) {
    const uint32_t ib = item_bytes(TYPE);
    const uint32_t n_items = nv * ipr;
    for (uint32_t it = threadIdx.x; it < n_items; it += BLOCK_THREADS) {
        const uint32_t v = it / ipr, k = it - v * ipr;
        const uint32_t roff = v < t.nr ? t.skew_a + v * rb : t.n16_a * 16 + t.skew_b + (v - t.nr) * rb;
        g_cb[it] = item_term(TYPE, buf, roff + k * ib, x, k);
    }
    wait_lgkm0();
    __builtin_amdgcn_s_barrier();
    // ascending fold of each row's terms; the terms are fetched 8 at a time
    // (one LDS round trip per 8) before the dependent fp64 adds
    for (uint32_t v = threadIdx.x; v < nv; v += BLOCK_THREADS) {
        const double *c = g_cb + v * ipr;
        double s = 0.0;
        uint32_t k = 0;
        for (; k + 8 <= ipr; k += 8) {
            double b[8];
#pragma unroll
            for (int i = 0; i < 8; i++) b[i] = c[k + i];
#pragma unroll
            for (int i = 0; i < 8; i++) s += b[i];
        }
        for (; k < ipr; k++) s += c[k];
        const uint32_t row = v < t.nr ? v : v - t.nr;
        g_res[2 * (slot0 + row) + (v < t.nr ? 0 : 1)] = (float)s;
    }
}

__device__ __forceinline__ void tile_compute(const sinter_gemv_args &a, const Tile &t, const char *buf,
                                          uint32_t slot0, const ActView &x) {
    const sinter_gemv_seg &sg = a.seg[t.seg];
    const int type = (int)uni(sg.type);
    const uint32_t ipr = a.K / item_elems(type);
    const uint32_t nv = t.nr * (sg.epi == SINTER_EPI_SWIGLU ? 2u : 1u);
    const uint32_t rb = uni(seg_rb(a, t.seg));
    switch (type) {
    case SINTER_Q4_K: tile_compute_t<SINTER_Q4_K>(t, buf, ipr, nv, rb, slot0, x); break;
    case SINTER_Q6_K: tile_compute_t<SINTER_Q6_K>(t, buf, ipr, nv, rb, slot0, x); break;
    case SINTER_Q8_0: tile_compute_t<SINTER_Q8_0>(t, buf, ipr, nv, rb, slot0, x); break;
    case SINTER_BF16: tile_compute_t<SINTER_BF16>(t, buf, ipr, nv, rb, slot0, x); break;
    default: tile_compute_t<SINTER_F32>(t, buf, ipr, nv, rb, slot0, x); break;
    }
}

__device__ void op_gemv(const sinter_instr &ins, unsigned *err) {
    if (threadIdx.x < sizeof(sinter_gemv_args) / 4)
        reinterpret_cast<uint32_t *>(g_args)[threadIdx.x] = reinterpret_cast<const uint32_t *>(ins.payload)[threadIdx.x];
    __syncthreads();
    const sinter_gemv_args &a = *reinterpret_cast<const sinter_gemv_args *>(g_args);
    const uint32_t rel = uni(blockIdx.x - ins.block_lo), nblk = uni(ins.block_hi - ins.block_lo);
    if (!gemv_args_ok(a)) {
        if (rel == 0 && threadIdx.x == 0) raise_error(err, SINTER_E_BAD_SHAPE, ins.dbg_node);
        return;
    }
    const uint32_t K = a.K;
    const int vt = vec_dot_type(a.seg[0].type);
    uint32_t rb_eff[SINTER_GEMV_MAX_SEG];
    uint64_t total = 0;
#pragma unroll
    for (int s = 0; s < SINTER_GEMV_MAX_SEG; s++) {
        rb_eff[s] = s < a.n_seg ? seg_rb_eff(a, s) : 0u;
        total += s < a.n_seg ? (uint64_t)a.seg[s].rows * rb_eff[s] : 0ull;
    }
    const uint32_t row_lo = uni(row_cut(a, rb_eff, total, rel, nblk));
    const uint32_t row_hi = uni(row_cut(a, rb_eff, total, rel + 1, nblk));

    // Three-buffer rotation over tiles identified by their first row (the
    // geometry is recomputed).  X = tile being computed (buffer bx), Y = the
    // next tile, already in flight.  Before computing X each wave waits for
    // its own DMA into X -- Y's TILE_CPW loads may stay outstanding -- and a
    // barrier makes every wave's chunks visible; after the compute a barrier
    // frees buffer bx+2 (computed last step) for the tile after Y.
    uint32_t gx = row_lo, gy = 0, next = row_lo, bx = 0;
    bool hx = gx < row_hi, hy = false;
    if (hx) { const Tile t = tile_at(a, gx, row_hi); next += t.nr; tile_issue(t, g_tiles); }
    if (hx && next < row_hi) {
        gy = next; hy = true;
        const Tile t = tile_at(a, gy, row_hi); next += t.nr; tile_issue(t, g_tiles + TILE_BYTES);
    }

    const bool write_x = (a.pro == SINTER_PRO_EMBED) && rel == 0 && a.x_out != nullptr;
    gemv_prologue(a, vt, write_x, g_qbuf, g_red, err);   // ends with __syncthreads()
    const ActView x = act_view(g_qbuf, K, vt);

    float bv = -INFINITY;
    int32_t bi = 0x7fffffff;
    uint32_t res_row0 = row_lo, res_n = 0;
    while (hx) {
        const Tile t = tile_at(a, gx, row_hi);
        if (res_n + t.nr > RES_CAP) {
            __syncthreads();
            gemv_flush(a, res_row0, res_n, bv, bi);
            res_row0 += res_n;
            res_n = 0;
            __syncthreads();
        }
        if (hy) wait_vmcnt<TILE_CPW>(); else wait_vmcnt<0>();
        __builtin_amdgcn_s_barrier();
        tile_compute(a, t, g_tiles + bx * TILE_BYTES, res_n, x);
        res_n += t.nr;
        wait_lgkm0();
        __builtin_amdgcn_s_barrier();
        const uint32_t bz = bx == 0 ? 2u : bx - 1;
        bool hz = hy && next < row_hi;
        uint32_t gz = 0;
        if (hz) { gz = next; const Tile tz = tile_at(a, gz, row_hi); next += tz.nr; tile_issue(tz, g_tiles + bz * TILE_BYTES); }
        gx = gy; hx = hy; gy = gz; hy = hz;
        bx = bx == 2 ? 0u : bx + 1;
    }
    __syncthreads();
    gemv_flush(a, res_row0, res_n, bv, bi);

    // greedy argmax: block-local best, then the last-arriving block reduces
    bool any_argmax = false;
    for (int s = 0; s < a.n_seg; s++) any_argmax |= a.seg[s].epi == SINTER_EPI_ARGMAX;
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
        ws->part_val[rel] = bv;
        ws->part_idx[rel] = bi;
        fence_release_agent();
        const unsigned old = __hip_atomic_fetch_add(ws->count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old == nblk - 1) {
            fence_acquire_agent();
            float best = -INFINITY;
            int32_t bidx = 0x7fffffff;
            for (uint32_t w = 0; w < nblk; w++) {
                const float v = __hip_atomic_load(ws->part_val + w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                const int32_t i = __hip_atomic_load(ws->part_idx + w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (v > best || (v == best && i < bidx)) { best = v; bidx = i; }
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
