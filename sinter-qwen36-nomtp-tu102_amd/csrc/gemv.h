// SINTER_OP_GEMV: the weight-streaming matrix-vector product of the decode
// pass, fused with what surrounds it in the reference schedule:
//   prologue  RMSNorm / gated RMSNorm / embedding lookup   (k0/ops/glue.cuh:56-227,
//             k0/ops/gdn.cuh:339-383)
//             + activation quantisation to the vec_dot type (k0/ops/gemv.cuh:213-237,
//             there q8_1; here ggml's Q8_K / Q8_0 / BF16)
//   body      y = W a for Q4_K / Q6_K / Q8_0 / BF16 / F32 rows, several
//             matrices ("segments") sharing one activation        (gemv.cuh:256-492)
//   epilogue  store, residual add, SwiGLU pair, conv, greedy argmax
//             (gemv.cuh:327-347, k0/harness.cpp:1187-1195)
//
// Work split: the rows of all segments form one byte-weighted row space; the
// host cuts it into one contiguous, byte-balanced row range per WAVE (four
// per workgroup).  A wave streams its range on its own -- no workgroup
// barrier inside the body: lane l takes items l, l+64, l+128, ... of the
// range (an item is one ggml block group; items ignore row boundaries, so
// every lane is busy), loads each item with 16-byte loads straight into
// registers, D items ahead (the first D are issued before the
// grid barrier that precedes the op, while the workgroup waits), computes its
// exact term against the quantised activation in LDS and writes it to the
// wave's term ring in LDS.  When the ring fills (and at the end) the lanes
// fold the completed rows -- lane i the i-th row -- in ascending item order
// and apply the row's epilogue.
//
// Declared numerics (oracle/oracle.c): integer block dots are exact; each
// item's term is an fp64 expression of exact integers and the f16/f32
// scales; a row is the ascending fp64 sum of its item terms, rounded to fp32
// once, so outputs are bit-identical to the oracle's.
#pragma once
#include <type_traits>

#include "dev_common.h"

namespace sinter {

__device__ __forceinline__ int vec_dot_type(int t) {
    return (t == SINTER_Q4_K || t == SINTER_Q6_K) ? SINTER_Q8_K
         : (t == SINTER_Q8_0) ? SINTER_Q8_0
         : (t == SINTER_BF16) ? SINTER_BF16 : SINTER_F32;
}
// wave-uniform copy of a value (its first active lane), kept in an SGPR
__device__ __forceinline__ uint32_t uni(uint32_t v) { return __builtin_amdgcn_readfirstlane(v); }

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

// Copy n floats (n a multiple of 256) from global p into LDS dst: the
// workgroup's waves take 1 KiB chunks round-robin.
template <bool COH>
__device__ __forceinline__ void dma_vec(const float *p, uint32_t n, char *dst) {
    // readfirstlane returns int: widen each word through uint32_t (a
    // sign-extended low word with bit 31 set would overwrite the high word)
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)p);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)((uintptr_t)p >> 32));
    const uintptr_t base = ((uintptr_t)hi << 32) | (uintptr_t)lo;
    const uint32_t lbase = (uint32_t)(uintptr_t)(lds_void *)dst;
    const uint32_t w = __builtin_amdgcn_readfirstlane(wave_id()), lane16 = lane_id() * 16;
    const uint32_t nch = n / 256;
    for (uint32_t j = w; j < nch; j += WAVES) lds_dma16<COH>(base, j * 1024 + lane16, lbase + j * 1024);
}

// ------------------------------------------------------------ prologue

// The prologue gives each 256-element chunk to one 16-lane DPP row, 16
// consecutive elements per lane: a per-chunk reduction is four in-VALU DPP
// steps and a Q8_K bsum (16 elements) is one lane's own sum.
constexpr uint32_t PRO_ROWS = BLOCK_THREADS / 16;

__device__ __forceinline__ void lds_st16(lds_char *p, uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
    u32x4_t v = {a, b, c, d};
    *reinterpret_cast<LDS u32x4_t *>(p) = v;
}
__device__ __forceinline__ uint32_t pack4_i8(int a, int b, int c, int d) {
    return (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) | ((uint32_t)(c & 0xff) << 16) | ((uint32_t)(d & 0xff) << 24);
}

// ggml quantize_row_q8_K_ref element by element for the lane's t[4q + i]
// (elements 64q + 4r + i of a chunk held by a 16-lane row): the first
// element reaching the row's max |x| (a (index, sign) key, smallest wins)
// gives bmax.  Writes b[i] = (int8 code) + 0x4B400000 and returns d.
__device__ __forceinline__ float quant_q8k_exact(uint32_t r, const float t[16], uint32_t b[16]) {
    float ax[16];
#pragma unroll
    for (int i = 0; i < 16; i++) ax[i] = fabsf(t[i]);
    float am = ax[0];
#pragma unroll
    for (int i = 1; i < 16; i++) am = fmaxf(am, ax[i]);
    const float A = row16_max(am);
    int key = 0x7fffffff;
#pragma unroll
    for (int qq = 0; qq < 4; qq++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int e = 64 * qq + 4 * (int)r + i;
            if (ax[4 * qq + i] == A) key = min(key, (e << 1) | (t[4 * qq + i] < 0.0f ? 1 : 0));
        }
    const int gkey = row16_min(key);
    if (!(A > 0.0f)) {    // max |x| == 0 (NaNs never win): all codes 0, d = 0
#pragma unroll
        for (int i = 0; i < 16; i++) b[i] = 0x4B400000u;
        return 0.0f;
    }
    const float bmax = (gkey & 1) ? -A : A;
    const float iscale = -127.f / bmax;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const float f = iscale * t[i];
        const int v = (int)(__float_as_uint(f + 12582912.f) & 0x007fffffu) - 0x00400000;
        b[i] = (uint32_t)(int32_t)(int8_t)(v < 127 ? v : 127) + 0x4B400000u;   // the stored int8
    }
    return 1.0f / iscale;
}

// Lane r of a 16-lane row holds elements 64q + 4r + i (q, i = 0..3) of its
// 256-element chunk c: four float4 at 64-element strides, so the 16 lanes of a
// row read 256 contiguous bytes per q (no LDS bank conflicts) and a Q8_K
// 16-element sub-block 4q + r/4 sits on the four lanes r/4 (two DPP steps).
// Quantise the lane's t[4q + i] into the activation layout at q.
__device__ __forceinline__ void quant_chunk(int vt, uint32_t c, uint32_t r, const float t[16], lds_char *q,
                                            LDS float *qd, LDS int16_t *qb) {
    if (vt == SINTER_Q8_K) {
        // ggml quantize_row_q8_K_ref: bmax = the signed element of largest |x|
        // (first index wins; NaNs never win), iscale = -127/bmax,
        // q = min(127, nearest_int(iscale * x)) with nearest_int's 1.5*2^23
        // magic add, d = 1/iscale; a chunk with max |x| = 0 gets q = 0, d = 0.
        // The chunk's signed max mx and min mn fix bmax's sign unless both +A
        // and -A occur.  For finite x, b = bits(iscale*x + 1.5*2^23) lies in
        // 0x4B400000 +- 127 and b - 0x4B400000 is the code, so the code byte
        // is b's low byte and the bsum is the sum of b's minus the bias.  A
        // wave in which any row has a +-A tie, a non-finite maximum or a b out
        // of that range (NaN or infinite inputs) recomputes its codes element
        // by element (quant_q8k_exact), which is exact for every input.
        float m2[8], n2[8];
#pragma unroll
        for (int i = 0; i < 8; i++) { m2[i] = fmaxf(t[2 * i], t[2 * i + 1]); n2[i] = fminf(t[2 * i], t[2 * i + 1]); }
#pragma unroll
        for (int w = 4; w > 0; w >>= 1)
#pragma unroll
            for (int i = 0; i < w; i++) { m2[i] = fmaxf(m2[i], m2[i + w]); n2[i] = fminf(n2[i], n2[i + w]); }
        const float mx = row16_max(m2[0]), mn = row16_minf(n2[0]);
        const float A = fmaxf(mx, -mn);
        const bool zero = A == 0.0f;
        const float bm = mx > -mn ? mx : mn;
        const float is = -127.f / bm;
        const float iscale = zero ? 0.0f : is;
        uint32_t b[16], hi = 0u, lo = 0xffffffffu;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const float f = iscale * t[i];
            b[i] = __float_as_uint(f + 12582912.f);
            hi = max(hi, b[i]);
            lo = min(lo, b[i]);
        }
        float dd = zero ? 0.0f : 1.0f / iscale;
        const bool bad = !(A <= 3.40282347e38f) || (mx == -mn && !zero) || hi > 0x4B40007Fu || lo < 0x4B3FFF81u;
        if (__builtin_amdgcn_ballot_w64(bad)) dd = quant_q8k_exact(r, t, b);
#pragma unroll
        for (int qq = 0; qq < 4; qq++) {
            const uint32_t w01 = __builtin_amdgcn_perm(b[4 * qq + 1], b[4 * qq], 0x0c0c0400u);
            const uint32_t w23 = __builtin_amdgcn_perm(b[4 * qq + 3], b[4 * qq + 2], 0x04000c0cu);
            *reinterpret_cast<LDS uint32_t *>(q + c * ACT_GSTRIDE + 64 * qq + 4 * r) = w01 | w23;
        }
        // bsum of sub-block 4qq + r/4: the four lanes r/4 hold it after two
        // DPP steps; lane r writes the one of qq = r & 3
        uint32_t s4[4];
#pragma unroll
        for (int qq = 0; qq < 4; qq++) {
            uint32_t s = (b[4 * qq] + b[4 * qq + 1]) + (b[4 * qq + 2] + b[4 * qq + 3]);
            s += (uint32_t)dpp_i<DPP_XOR1>((int)s);
            s += (uint32_t)dpp_i<DPP_XOR2>((int)s);
            s4[qq] = s;
        }
        const uint32_t j = r & 3;
        const uint32_t sj = j == 0 ? s4[0] : j == 1 ? s4[1] : j == 2 ? s4[2] : s4[3];
        qb[16 * c + 4 * j + r / 4] = (int16_t)(int32_t)(sj - 16u * 0x4B400000u);
        if (r == 0) qd[c] = dd;
    } else if (vt == SINTER_Q8_0) {
        int qv[16];
        // ggml-cpu x86 quantize_row_q8_0: d = f16(amax/127), q = rne(x * 127/amax);
        // 32-element block 2q + r/8 is the lane's four elements of each q on
        // the eight lanes r/8
        float dblk[4];
#pragma unroll
        for (int qq = 0; qq < 4; qq++) {
            float am = fmaxf(fmaxf(fabsf(t[4 * qq]), fabsf(t[4 * qq + 1])), fmaxf(fabsf(t[4 * qq + 2]), fabsf(t[4 * qq + 3])));
            am = fmaxf(am, dpp_f<DPP_XOR1>(am));
            am = fmaxf(am, dpp_f<DPP_XOR2>(am));
            am = fmaxf(am, dpp_f<DPP_HALF_MIRROR>(am));
            const float id = (am != 0.0f) ? 127.f / am : 0.0f;
#pragma unroll
            for (int i = 0; i < 4; i++) qv[4 * qq + i] = (int)__builtin_rintf(t[4 * qq + i] * id);
            dblk[qq] = am / 127.f;
            *reinterpret_cast<LDS uint32_t *>(q + c * ACT_GSTRIDE + 64 * qq + 4 * r) =
                pack4_i8(qv[4 * qq], qv[4 * qq + 1], qv[4 * qq + 2], qv[4 * qq + 3]);
            if ((r & 7) == 0) qd[8 * c + 2 * qq + r / 8] = h2f(f2h(dblk[qq]));
        }
    } else if (vt == SINTER_BF16) {
#pragma unroll
        for (int qq = 0; qq < 4; qq++) {
            const uint32_t h0 = (uint32_t)f2bf(t[4 * qq]) | ((uint32_t)f2bf(t[4 * qq + 1]) << 16);
            const uint32_t h1 = (uint32_t)f2bf(t[4 * qq + 2]) | ((uint32_t)f2bf(t[4 * qq + 3]) << 16);
            typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
            const u32x2_t v = {h0, h1};
            *reinterpret_cast<LDS u32x2_t *>(q + (4 * c + qq) * ACT_BF_CSTRIDE + 8 * r) = v;
        }
    } else {
#pragma unroll
        for (int qq = 0; qq < 4; qq++)
            lds_st16(q + (4 * c + qq) * ACT_F_CSTRIDE + 16 * r, __float_as_uint(t[4 * qq]), __float_as_uint(t[4 * qq + 1]),
                     __float_as_uint(t[4 * qq + 2]), __float_as_uint(t[4 * qq + 3]));
    }
}

// Q8_K with one sub-block per lane: lane r of a 16-lane row holds elements
// 16r + i (i = 0..15) of its chunk, i.e. Q8_K sub-block r, so its 16 codes
// are one 16-byte store and its bsum is the lane's own sum.  The row's
// signed max and min come from IEEE-2019 maximum / minimum (v_maximum3 /
// v_minimum3: NaNs propagate, so a chunk holding a NaN fails the finite-max
// test and takes the exact path).  Bit-identical to quant_chunk's Q8_K
// branch: the same bmax, iscale, codes, d and bsums.
__device__ __forceinline__ float fmax2019(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ float fmin2019(float a, float b) { return __builtin_elementwise_minimum(a, b); }

// quant_q8k_exact for the sub-block-per-lane layout (element 16r + i)
__device__ __forceinline__ float quant_q8k_exact_span(uint32_t r, const float t[16], uint32_t b[16]) {
    float ax[16];
#pragma unroll
    for (int i = 0; i < 16; i++) ax[i] = fabsf(t[i]);
    float am = ax[0];
#pragma unroll
    for (int i = 1; i < 16; i++) am = fmaxf(am, ax[i]);
    const float A = row16_max(am);
    int key = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int e = 16 * (int)r + i;
        if (ax[i] == A) key = min(key, (e << 1) | (t[i] < 0.0f ? 1 : 0));
    }
    const int gkey = row16_min(key);
    if (!(A > 0.0f)) {    // max |x| == 0 (NaNs never win): all codes 0, d = 0
#pragma unroll
        for (int i = 0; i < 16; i++) b[i] = 0x4B400000u;
        return 0.0f;
    }
    const float bmax = (gkey & 1) ? -A : A;
    const float iscale = -127.f / bmax;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const float f = iscale * t[i];
        const int v = (int)(__float_as_uint(f + 12582912.f) & 0x007fffffu) - 0x00400000;
        b[i] = (uint32_t)(int32_t)(int8_t)(v < 127 ? v : 127) + 0x4B400000u;   // the stored int8
    }
    return 1.0f / iscale;
}

// Fast path of quant_q8k_span: b[i] = bits(iscale*t[i] + 1.5*2^23) (the
// code is b's low byte) and d; returns true when the row must take the
// exact path instead.  With NaN-propagating max / min, a NaN or infinite
// element makes A non-finite; with A finite and non-zero and iscale =
// -127/bmax finite, every |iscale*t| <= 127 (1 + 2^-24)^2 < 127.5, so every
// code lies in [-127, 127] and min(127, .) is a no-op.  Left for the exact
// path: non-finite A, iscale overflow (denormal A) and +-A ties.
__device__ __forceinline__ bool q8k_fast(const float t[16], uint32_t b[16], float &dd) {
    float mx = fmax2019(t[0], t[1]), mn = fmin2019(t[0], t[1]);
#pragma unroll
    for (int i = 2; i < 16; i += 2) {
        mx = fmax2019(mx, fmax2019(t[i], t[i + 1]));
        mn = fmin2019(mn, fmin2019(t[i], t[i + 1]));
    }
    mx = fmax2019(mx, dpp_f<DPP_XOR1>(mx));
    mn = fmin2019(mn, dpp_f<DPP_XOR1>(mn));
    mx = fmax2019(mx, dpp_f<DPP_XOR2>(mx));
    mn = fmin2019(mn, dpp_f<DPP_XOR2>(mn));
    mx = fmax2019(mx, dpp_f<DPP_HALF_MIRROR>(mx));
    mn = fmin2019(mn, dpp_f<DPP_HALF_MIRROR>(mn));
    mx = fmax2019(mx, dpp_f<DPP_MIRROR>(mx));
    mn = fmin2019(mn, dpp_f<DPP_MIRROR>(mn));
    // as quant_chunk: bmax's sign from mx / mn unless +A and -A both occur
    const float A = fmax2019(mx, -mn);
    const bool zero = A == 0.0f;
    const float bm = mx > -mn ? mx : mn;
    const float is = -127.f / bm;
    const float iscale = zero ? 0.0f : is;
#pragma unroll
    for (int i = 0; i < 16; i++) b[i] = __float_as_uint(iscale * t[i] + 12582912.f);
    dd = zero ? 0.0f : 1.0f / iscale;
    return !(A <= 3.40282347e38f) || (!zero && (mx == -mn || !(fabsf(is) <= 3.40282347e38f)));
}

// Store chunk c's codes (b's low bytes), its sub-block bsum and d.
__device__ __forceinline__ void q8k_store(uint32_t c, uint32_t r, const uint32_t b[16], float dd, lds_char *q,
                                          LDS float *qd, LDS int16_t *qb) {
    uint32_t w[4];
#pragma unroll
    for (int qq = 0; qq < 4; qq++)
        w[qq] = __builtin_amdgcn_perm(b[4 * qq + 1], b[4 * qq], 0x0c0c0400u) |
                __builtin_amdgcn_perm(b[4 * qq + 3], b[4 * qq + 2], 0x04000c0cu);
    lds_st16(q + c * ACT_GSTRIDE + 16 * r, w[0], w[1], w[2], w[3]);
    // the bsum: the sub-block's 16 signed codes, summed exactly
    int bs = __builtin_amdgcn_sdot4((int)w[0], 0x01010101, 0, false);
    bs = __builtin_amdgcn_sdot4((int)w[1], 0x01010101, bs, false);
    bs = __builtin_amdgcn_sdot4((int)w[2], 0x01010101, bs, false);
    bs = __builtin_amdgcn_sdot4((int)w[3], 0x01010101, bs, false);
    qb[16 * c + r] = (int16_t)bs;
    if (r == 0) qd[c] = dd;
}

__device__ __forceinline__ void quant_q8k_span(uint32_t c, uint32_t r, const float t[16], lds_char *q, LDS float *qd,
                                               LDS int16_t *qb) {
    uint32_t b[16];
    float dd;
    const bool bad = q8k_fast(t, b, dd);
    if (__builtin_amdgcn_ballot_w64(bad)) dd = quant_q8k_exact_span(r, t, b);
    q8k_store(c, r, b, dd, q, qd, qb);
}

// Two chunks at once (independent chains the compiler interleaves).
__device__ __forceinline__ void quant_q8k_span2(uint32_t c0, uint32_t c1, uint32_t r, const float t0[16],
                                                const float t1[16], lds_char *q, LDS float *qd, LDS int16_t *qb) {
    uint32_t b0[16], b1[16];
    float d0, d1;
    const bool bad0 = q8k_fast(t0, b0, d0);
    const bool bad1 = q8k_fast(t1, b1, d1);
    if (__builtin_amdgcn_ballot_w64(bad0)) d0 = quant_q8k_exact_span(r, t0, b0);
    if (__builtin_amdgcn_ballot_w64(bad1)) d1 = quant_q8k_exact_span(r, t1, b1);
    q8k_store(c0, r, b0, d0, q, qd, qb);
    q8k_store(c1, r, b1, d1, q, qd, qb);
}

__device__ __forceinline__ u32x4 lds16(const lds_char *p) { return *reinterpret_cast<const LDS u32x4 *>(p); }
__device__ __forceinline__ f32x4 ldsf16(const lds_char *p) { return *reinterpret_cast<const LDS f32x4 *>(p); }

// Build the quantised activation in LDS (g_qbuf).  Every thread of the block
// calls this.  Phase 1 stages the f32 inputs in g_big with LDS-DMA -- x (and
// z for the gated norm) device-coherently, the norm weights cached --
// without holding any registers (the caller may hold prefetched weights).
// Phase 2: row g of the block (16 lanes) owns chunks g, g+16, ... and reads
// its elements from the staging area; RMSNorm first sums squares over its
// chunks for the block-wide scale.
template <class Post>
__device__ __forceinline__ void prologue_stage(const sinter_gemv_args &a, bool write_x, unsigned *err, Post &&post) {
    const uint32_t K = a.K;
    const bool embed = a.pro == SINTER_PRO_EMBED;
    const bool gpre = a.pro == SINTER_PRO_GATED_G, gated = a.pro == SINTER_PRO_GATED || gpre;
    const bool rms = a.pro == SINTER_PRO_RMSNORM || embed;
    char *xs_g = g_big, *ys_g = g_big + K * 4;
    const uint32_t gd = 1u << a.gn_log2d;  // gated-norm head width (4..256)
    // gated norms: the gd head-width norm weights go to the last KiB of the
    // staging area by one LDS-DMA (lanes past gd/4 re-read the last 16 bytes,
    // in bounds), so that no compiler-visible load precedes the weight slots
    // post() issues (a wait for it would wait for those too)
    char *ws_g = g_big + BIG_BYTES - 1024;
    if (gated && wave_id() == 0) {
        const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)a.norm_w);
        const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)((uintptr_t)a.norm_w >> 32));
        lds_dma16<false>(((uintptr_t)hi << 32) | lo, min((uint32_t)lane_id() * 16u, gd * 4u - 16u),
                         (uint32_t)(uintptr_t)(lds_void *)ws_g);
    }
    if (embed) {
        int32_t tok = ld_coh(a.token);
        if (tok < 0 || (uint32_t)tok >= a.aux_rows) {   // never read outside the table
            if (threadIdx.x == 0) raise_error(err, SINTER_E_BAD_SHAPE, 0xE0000000u);
            tok = 0;
        }
        const void *erow = static_cast<const char *>(a.aux) + (size_t)tok * sinter_row_bytes_dev(a.aux_type, K);
        dma_vec<false>(a.norm_w, K, ys_g);
        LDS float *xs = reinterpret_cast<LDS float *>((lds_char *)xs_g);
        for (uint32_t i = threadIdx.x; i < K / 4; i += BLOCK_THREADS) {
            float v[4];
            dequant4(erow, a.aux_type, 4 * i, v);
            if (write_x) st_coh4(a.x_out + 4 * i, make_float4(v[0], v[1], v[2], v[3]));
#pragma unroll
            for (int k = 0; k < 4; k++) xs[4 * i + k] = v[k];
        }
        post();
    } else {
        dma_vec<true>(a.x, K, xs_g);
        if (gated) dma_vec<true>(static_cast<const float *>(a.aux), K, ys_g);
        else if (rms) dma_vec<false>(a.norm_w, K, ys_g);
        post();
    }
    __syncthreads();
}

// The lane's 16 elements of chunk c from LDS: elements 16r + i (SPAN, the
// Q8_K sub-block-per-lane layout) or 64q + 4r + i (q, i = 0..3: the layout
// quant_chunk takes).
template <bool SPAN>
__device__ __forceinline__ void ld16(const LDS float *base, uint32_t c, uint32_t r, float v[16]) {
#pragma unroll
    for (int qq = 0; qq < 4; qq++) {
        const f32x4 t = *reinterpret_cast<const LDS f32x4 *>(base + c * 256 + (SPAN ? 16 * r + 4 * qq : 64 * qq + 4 * r));
        v[4 * qq] = t.x; v[4 * qq + 1] = t.y; v[4 * qq + 2] = t.z; v[4 * qq + 3] = t.w;
    }
}

// Norm + quantisation of the staged f32 inputs into the activation layout in
// g_qbuf, for one vec_dot type VT; the prologue kind and sizes are
// wave-uniform (scalar branches only).  Row g (16 lanes) owns chunks g,
// g+16, ...; the next chunk's inputs are read while the current one is
// quantised.
template <int VT>
__device__ __forceinline__ void prologue_quant(uint32_t K, uint32_t pro, uint32_t log2d, float eps, double *red) {
    constexpr bool SPAN = VT == SINTER_Q8_K;
    // the lane's indices, opaque to the compiler so that the per-lane address
    // arithmetic below is not hoisted out of the interpreter loop (where it
    // would stay live, in registers, for the whole kernel)
    uint32_t tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    const uint32_t r = tid & 15, g = tid >> 4, nchunk = K / 256;
    const LDS float *xs = reinterpret_cast<const LDS float *>((const lds_char *)g_big);
    const LDS float *ys = xs + K;
    lds_char *q = (lds_char *)g_qbuf;
    LDS float *qd = reinterpret_cast<LDS float *>(q + nchunk * ACT_GSTRIDE);
    LDS int16_t *qb = reinterpret_cast<LDS int16_t *>(q + act_bs_off(K));
    auto quantize = [&](uint32_t c, const float t[16]) {
        if constexpr (SPAN) quant_q8k_span(c, r, t, q, qd, qb);
        else quant_chunk(VT, c, r, t, q, qd, qb);
    };
    auto quantize2 = [&](uint32_t c0, uint32_t c1, const float t0[16], const float t1[16]) {
        if constexpr (SPAN) {
            quant_q8k_span2(c0, c1, r, t0, t1, q, qd, qb);
        } else {
            quant_chunk(VT, c0, r, t0, q, qd, qb);
            quant_chunk(VT, c1, r, t1, q, qd, qb);
        }
    };
    if (pro == SINTER_PRO_PLAIN) {
        // chunks in pairs (c, c + 16)
#pragma unroll 1
        for (uint32_t c = g; c < nchunk; c += 2 * PRO_ROWS) {
            float t0[16];
            ld16<SPAN>(xs, c, r, t0);
            if (c + PRO_ROWS < nchunk) {
                float t1[16];
                ld16<SPAN>(xs, c + PRO_ROWS, r, t1);
                quantize2(c, c + PRO_ROWS, t0, t1);
            } else {
                quantize(c, t0);
            }
        }
    } else if (pro == SINTER_PRO_RMSNORM || pro == SINTER_PRO_EMBED) {
        // global RMSNorm scale (ggml: fp32 squares summed in double, mean ->
        // f32, scale = 1/sqrtf(mean + eps)); the fp64 sum is a fixed tree:
        // per lane four partial sums over its chunks, then the 16-lane row,
        // the wave's rows and the waves in order.  The row's first two
        // chunks stay in registers for the second pass.
        float v0[16], v1[16];
#pragma unroll
        for (int i = 0; i < 16; i++) { v0[i] = 0.0f; v1[i] = 0.0f; }
        if (g < nchunk) ld16<SPAN>(xs, g, r, v0);
        if (g + PRO_ROWS < nchunk) ld16<SPAN>(xs, g + PRO_ROWS, r, v1);
        double s4[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll 1
        for (uint32_t c = g + 2 * PRO_ROWS; c < nchunk; c += PRO_ROWS) {
            float v[16];
            ld16<SPAN>(xs, c, r, v);
#pragma unroll
            for (int i = 0; i < 16; i++) s4[i / 4] += (double)(v[i] * v[i]);
        }
#pragma unroll
        for (int i = 0; i < 16; i++) s4[i / 4] += (double)(v0[i] * v0[i]);
#pragma unroll
        for (int i = 0; i < 16; i++) s4[i / 4] += (double)(v1[i] * v1[i]);
        double s = row16_sum_f64((s4[0] + s4[1]) + (s4[2] + s4[3]));
        s = ((readlane_f64(s, 0) + readlane_f64(s, 16)) + readlane_f64(s, 32)) + readlane_f64(s, 48);
        // every wave has passed the staging barrier, so no reader of an
        // earlier sum is left; the next writer is past this op's last barrier
        if (lane_id() == 0) red[wave_id()] = s;
        float y0[16], y1[16];
        if (g < nchunk) ld16<SPAN>(ys, g, r, y0);
        if (g + PRO_ROWS < nchunk) ld16<SPAN>(ys, g + PRO_ROWS, r, y1);
        __syncthreads();
        s = ((red[0] + red[1]) + red[2]) + red[3];
        const float mean = (float)(s / (double)K);
        const float gscale = 1.0f / sqrtf(mean + eps);
        // chunks in pairs (c, c + 16), the first pair from registers
#pragma unroll 1
        for (uint32_t c = g; c < nchunk; c += 2 * PRO_ROWS) {
            if (c != g) {
                ld16<SPAN>(xs, c, r, v0);
                ld16<SPAN>(ys, c, r, y0);
                if (c + PRO_ROWS < nchunk) {
                    ld16<SPAN>(xs, c + PRO_ROWS, r, v1);
                    ld16<SPAN>(ys, c + PRO_ROWS, r, y1);
                }
            }
            float t0[16];
#pragma unroll
            for (int i = 0; i < 16; i++) t0[i] = (v0[i] * gscale) * y0[i];
            if (c + PRO_ROWS < nchunk) {
                float t1[16];
#pragma unroll
                for (int i = 0; i < 16; i++) t1[i] = (v1[i] * gscale) * y1[i];
                quantize2(c, c + PRO_ROWS, t0, t1);
            } else {
                quantize(c, t0);
            }
        }
    } else {
        // gated norm per head of gd = 2^log2d elements: rmsnorm(x_h) * norm_w
        // * g_h, g = z (GATED_G) or silu(z) (GATED).  Element e of every chunk
        // uses norm_w[e % gd] (staged in the last KiB of g_big); each group
        // of four elements of the lane (e, .., e+3) lies in one head (gd >= 4).
        const bool gpre = pro == SINTER_PRO_GATED_G;
        const uint32_t gd = 1u << log2d;
        const double inv_gd = __longlong_as_double((long long)(1023 - log2d) << 52);   // 2^-log2d exactly
        const LDS float *ws = reinterpret_cast<const LDS float *>((const lds_char *)(g_big + BIG_BYTES - 1024));
        float gw[16];
#pragma unroll
        for (int qq = 0; qq < 4; qq++) {
            const uint32_t e = SPAN ? 16 * r + 4 * qq : 64 * qq + 4 * r;
            const f32x4 t = *reinterpret_cast<const LDS f32x4 *>(ws + (e & (gd - 1)));
            gw[4 * qq] = t.x; gw[4 * qq + 1] = t.y; gw[4 * qq + 2] = t.z; gw[4 * qq + 3] = t.w;
        }
#pragma unroll 1
        for (uint32_t c = g; c < nchunk; c += PRO_ROWS) {
            float v[16], y[16], t[16];
            ld16<SPAN>(xs, c, r, v);
            ld16<SPAN>(ys, c, r, y);
            // per-head sums of squares in double, s4[qq] for the lane's
            // elements of group qq
            double s4[4];
#pragma unroll
            for (int qq = 0; qq < 4; qq++) {
                double h = 0.0;
#pragma unroll
                for (int i = 0; i < 4; i++) h += (double)(v[4 * qq + i] * v[4 * qq + i]);
                s4[qq] = h;
            }
            if constexpr (SPAN) {
                // the lane's 16 elements are one head (gd >= 16; its sum then
                // spans gd/16 lanes), two (gd = 8) or four (gd = 4)
                if (gd == 8) {
                    const double a01 = s4[0] + s4[1], a23 = s4[2] + s4[3];
                    s4[0] = s4[1] = a01; s4[2] = s4[3] = a23;
                } else if (gd >= 16) {
                    double h = (s4[0] + s4[1]) + (s4[2] + s4[3]);
                    if (gd >= 32) h += dpp_d<DPP_XOR1>(h);
                    if (gd >= 64) h += dpp_d<DPP_XOR2>(h);
                    if (gd >= 128) h += dpp_d<DPP_HALF_MIRROR>(h);
                    if (gd >= 256) h += dpp_d<DPP_MIRROR>(h);
                    s4[0] = s4[1] = s4[2] = s4[3] = h;
                }
            } else {
                // head h of width gd holds, on lane r, the elements of each q
                // with (64q + 4r) / gd == h: its sum combines lanes (DPP)
                // and, for gd >= 128, q's
#pragma unroll
                for (int qq = 0; qq < 4; qq++) {
                    double h = s4[qq];
                    if (gd >= 8) h += dpp_d<DPP_XOR1>(h);
                    if (gd >= 16) h += dpp_d<DPP_XOR2>(h);
                    if (gd >= 32) h += dpp_d<DPP_HALF_MIRROR>(h);
                    if (gd >= 64) h += dpp_d<DPP_MIRROR>(h);
                    s4[qq] = h;
                }
                if (gd >= 128) { const double a01 = s4[0] + s4[1], a23 = s4[2] + s4[3]; s4[0] = s4[1] = a01; s4[2] = s4[3] = a23; }
                if (gd >= 256) { const double all = s4[0] + s4[2]; s4[0] = s4[1] = s4[2] = s4[3] = all; }
            }
            float hs[4];
#pragma unroll
            for (int qq = 0; qq < 4; qq++) hs[qq] = 1.0f / sqrtf((float)(s4[qq] * inv_gd) + eps);
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const float wn = (v[i] * hs[i / 4]) * gw[i];
                t[i] = wn * (gpre ? y[i] : dev_silu(y[i]));
                if ((i & 3) == 3) sched_fence();   // bounds the live fp64 temporaries
            }
            quantize(c, t);
        }
    }
    __syncthreads();
}

// (F: the interpreter's feature set; the op checked that vt is in it)
template <uint32_t F>
__device__ __forceinline__ void prologue_compute(const sinter_gemv_args &a, int vt, double *red) {
    const uint32_t K = uni(a.K), pro = uni(a.pro), log2d = uni(a.gn_log2d);
    const float eps = __uint_as_float(uni(__float_as_uint(a.eps)));
    constexpr uint32_t FX = F & (FEAT_X_Q8K | FEAT_X_Q80 | FEAT_X_BF16 | FEAT_X_F32);
    if constexpr (FX == FEAT_X_Q8K) {
        prologue_quant<SINTER_Q8_K>(K, pro, log2d, eps, red);
        return;
    } else if constexpr (FX == FEAT_X_BF16) {
        prologue_quant<SINTER_BF16>(K, pro, log2d, eps, red);
        return;
    }
    switch (vt) {
    case SINTER_Q8_K: if constexpr ((F & FEAT_X_Q8K) != 0) prologue_quant<SINTER_Q8_K>(K, pro, log2d, eps, red); break;
    case SINTER_Q8_0: if constexpr ((F & FEAT_X_Q80) != 0) prologue_quant<SINTER_Q8_0>(K, pro, log2d, eps, red); break;
    case SINTER_BF16: if constexpr ((F & FEAT_X_BF16) != 0) prologue_quant<SINTER_BF16>(K, pro, log2d, eps, red); break;
    case SINTER_F32: if constexpr ((F & FEAT_X_F32) != 0) prologue_quant<SINTER_F32>(K, pro, log2d, eps, red); break;
    default: break;
    }
}

template <uint32_t F, class Post>
__device__ __forceinline__ void gemv_prologue(const sinter_gemv_args &a, int vt, bool write_x, double *red,
                                              unsigned *err, Post &&post) {
    prologue_stage(a, write_x, err, post);
    prologue_compute<F>(a, vt, red);
}

// ------------------------------------------------------------ item terms
// A weight row is a sequence of items: one 256-element group for the
// quantised types (one Q4_K / Q6_K block, eight Q8_0 blocks), 64 elements
// for BF16 / F32.  An item's term is an fp64 expression of exact integer
// block dots and the f16/f32 scales (a float sum of exact products for
// BF16/F32).  A row is the ascending fp64 sum of its item terms, rounded to
// fp32 once -- the fold oracle/oracle.c declares.  Each term function takes
// the item's bytes from registers (one lane, one item) and the activation
// from LDS; it issues all of its LDS reads before computing.

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// Q4_K block (144 B = 9 x 16 B) against Q8_K group g
__device__ __forceinline__ double term_q4k(const u32x4 *wv, const ActView &x, uint32_t g) {
    u32x4 xv[16], bsv[2];
    const lds_char *xq = x.q + g * ACT_GSTRIDE;
#pragma unroll
    for (int i = 0; i < 16; i++) xv[i] = lds16(xq + 16 * i);
    const lds_char *bsp = reinterpret_cast<const lds_char *>(x.bs + g * 16);
    bsv[0] = lds16(bsp);
    bsv[1] = lds16(bsp + 16);
    const float dxf = x.d[g];
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

// Q6_K block (210 B at byte `sh` (0 or 2) of a 212-byte window -- 53 dwords
// -- read from a 4-aligned address) against Q8_K group g.  Codes are taken
// unsigned (0..63) and the -32 offset folds through the bsums:
// sum((c-32)*x) = sum(c*x) - 32*bsum; the block's integer sum is exact.
__device__ __forceinline__ double term_q6k(const u32x4 *wv, uint32_t sh, const ActView &x, uint32_t g) {
    const lds_char *xq = x.q + g * ACT_GSTRIDE;
    u32x4 xv[16], bsv[2];
#pragma unroll
    for (int i = 0; i < 16; i++) xv[i] = lds16(xq + 16 * i);
    const lds_char *bsp = reinterpret_cast<const lds_char *>(x.bs + g * 16);
    bsv[0] = lds16(bsp);
    bsv[1] = lds16(bsp + 16);
    const float dxf = x.d[g];
    uint32_t d[53];
#pragma unroll
    for (int i = 0; i < 13; i++) { d[4 * i] = wv[i].x; d[4 * i + 1] = wv[i].y; d[4 * i + 2] = wv[i].z; d[4 * i + 3] = wv[i].w; }
    d[52] = wv[13].x;
    auto W = [&](int j) -> uint32_t { return __builtin_amdgcn_alignbyte(d[j + 1], d[j], sh); };
    int isum = 0;
#pragma unroll
    for (int n = 0; n < 2; n++) {
        uint32_t xw[32];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const u32x4 t = xv[8 * n + i];
            xw[4 * i] = t.x; xw[4 * i + 1] = t.y; xw[4 * i + 2] = t.z; xw[4 * i + 3] = t.w;
        }
        int dot[4][2] = {{0, 0}, {0, 0}, {0, 0}, {0, 0}};  // [quarter][16-element half]
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t qa = W(16 * n + i), qb = W(16 * n + 8 + i), qh = W(32 + 8 * n + i);
            const uint32_t c0 = (qa & 0x0F0F0F0Fu) | ((qh << 4) & 0x30303030u);
            const uint32_t c1 = (qb & 0x0F0F0F0Fu) | ((qh << 2) & 0x30303030u);
            const uint32_t c2 = ((qa >> 4) & 0x0F0F0F0Fu) | (qh & 0x30303030u);
            const uint32_t c3 = ((qb >> 4) & 0x0F0F0F0Fu) | ((qh >> 2) & 0x30303030u);
            const int hf = i >> 2;                     // l = 4i.. : half hf of each quarter
            dot[0][hf] = sdot4(c0, xw[i], dot[0][hf]);
            dot[1][hf] = sdot4(c1, xw[8 + i], dot[1][hf]);
            dot[2][hf] = sdot4(c2, xw[16 + i], dot[2][hf]);
            dot[3][hf] = sdot4(c3, xw[24 + i], dot[3][hf]);
        }
        const uint32_t scw[2] = {W(48 + 2 * n), W(49 + 2 * n)};
        const u32x4 bs = bsv[n];
#pragma unroll
        for (int t = 0; t < 4; t++) {
#pragma unroll
            for (int hf = 0; hf < 2; hf++) {
                const int j = 2 * t + hf;              // 16-element sub-block within the half
                const int sc = (int)(int8_t)((scw[j >> 2] >> (8 * (j & 3))) & 0xff);
                const uint32_t bw = bs[j >> 1];
                const int b = (j & 1) ? ((int)bw >> 16) : (int)(int16_t)(bw & 0xffff);
                isum += sc * (dot[t][hf] - 32 * b);
            }
        }
    }
    const uint16_t dh = (uint16_t)((sh ? d[52] >> 16 : d[52]) & 0xffff);   // block bytes 208..209
    return ((double)h2f(dh) * (double)dxf) * (double)isum;
}

// Q8_0 item: eight 34-byte blocks (272 B = 17 x 16 B, 16-aligned) against
// Q8_0 activation blocks 8g ..; the block terms summed in ascending order.
__device__ __forceinline__ double term_q80(const u32x4 *wv, const ActView &x, uint32_t g) {
    const lds_char *xq = x.q + g * ACT_GSTRIDE;
    u32x4 xv[16];
#pragma unroll
    for (int i = 0; i < 16; i++) xv[i] = lds16(xq + 16 * i);
    float dx[8];
#pragma unroll
    for (int j = 0; j < 8; j++) dx[j] = x.d[8 * g + j];
    uint32_t d[68];
#pragma unroll
    for (int i = 0; i < 17; i++) { d[4 * i] = wv[i].x; d[4 * i + 1] = wv[i].y; d[4 * i + 2] = wv[i].z; d[4 * i + 3] = wv[i].w; }
    double acc = 0.0;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int b0 = 34 * j;                       // block start byte
        const uint32_t dw16 = __builtin_amdgcn_alignbyte(d[b0 / 4 + 1], d[b0 / 4], b0 % 4) & 0xffff;
        const int q0 = b0 + 2;                       // codes start byte
        int isum = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int bb = q0 + 4 * i;
            const uint32_t w = (bb % 4) == 0 ? d[bb / 4] : __builtin_amdgcn_alignbyte(d[bb / 4 + 1], d[bb / 4], bb % 4);
            isum = sdot4(w, xv[2 * j + i / 4][i % 4], isum);
        }
        acc += ((double)h2f((uint16_t)dw16) * (double)dx[j]) * (double)isum;
    }
    return acc;
}

// 64 bf16 elements (128 B = 8 x 16 B), products exact in fp64, ascending
__device__ __forceinline__ double term_bf16(const u32x4 *av, const ActView &x, uint32_t k) {
    const lds_char *xx = x.q + k * ACT_BF_CSTRIDE;
    u32x4 bv[8];
#pragma unroll
    for (int i = 0; i < 8; i++) bv[i] = lds16(xx + 16 * i);
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

// 64 f32 elements (256 B = 16 x 16 B), products exact in fp64, ascending
__device__ __forceinline__ double term_f32(const u32x4 *av, const ActView &x, uint32_t k) {
    const lds_char *xx = x.q + k * ACT_F_CSTRIDE;
    double acc = 0.0;
#pragma unroll
    for (int h = 0; h < 2; h++) {
        f32x4 bv[8];
#pragma unroll
        for (int i = 0; i < 8; i++) bv[i] = ldsf16(xx + 128 * h + 16 * i);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const u32x4 a = av[8 * h + i];
            acc += (double)__uint_as_float(a.x) * (double)bv[i].x;
            acc += (double)__uint_as_float(a.y) * (double)bv[i].y;
            acc += (double)__uint_as_float(a.z) * (double)bv[i].z;
            acc += (double)__uint_as_float(a.w) * (double)bv[i].w;
        }
    }
    return acc;
}

template <int T>
__device__ __forceinline__ double item_term(const u32x4 *wv, uint32_t sh, const ActView &x, uint32_t k) {
    if constexpr (T == SINTER_Q4_K) return term_q4k(wv, x, k);
    else if constexpr (T == SINTER_Q6_K) return term_q6k(wv, sh, x, k);
    else if constexpr (T == SINTER_Q8_0) return term_q80(wv, x, k);
    else if constexpr (T == SINTER_BF16) return term_bf16(wv, x, k);
    else return term_f32(wv, x, k);
}

// ------------------------------------------------------------ runs
// The host compiles each GEMV into a GemvPlan (isa.h): per-segment constants,
// the term ring geometry and the waves' row cuts.  The kernel reads it
// through the constant address space, so every field is a scalar load.
typedef const __attribute__((address_space(4))) GemvPlan cplan_t;
typedef const __attribute__((address_space(4))) uint32_t cu32_t;


// q = v / d, r = v % d from m = floor((2^32-1) / d): the estimate is q or
// q-1, one correction step makes it exact (v < 2^31)
__device__ __forceinline__ uint32_t divm(uint32_t v, uint32_t d, uint32_t m, uint32_t &r) {
    uint32_t q = __umulhi(v, m);
    r = v - q * d;
    if (r >= d) { r -= d; q += 1; }
    return q;
}

// A run: the rows of a wave's range that lie in one segment, streamed as one
// flat sequence of items.  Plain: lane l takes items l, l+64, ...; SwiGLU
// pair: even lanes take gate items l/2, l/2+32, ..., odd lanes the same up
// items, so a step covers 32 items of each matrix and every lane holds one
// item.  Item f of the run is item f + L of the segment (L = first item).
struct Run {
    uint32_t ok, s, type, swig;
    uint32_t g0, g1, n;                 // global rows [g0, g1); n = items (per matrix)
    uint64_t VA, VB;                    // address of the run's item 0 in matrix A, B
};

__device__ __forceinline__ bool epi_loads(uint32_t epi) { return epi == SINTER_EPI_RESID || epi == SINTER_EPI_CONV; }

// The run of rows [lo, hi) in the first segment >= s holding any of them
// (at most min(64, R) rows for an operand-reading epilogue).
__device__ __forceinline__ Run make_run(cplan_t *pl, uint32_t s, uint32_t lo, uint32_t hi) {
    Run r;
    r.ok = 0; r.s = 0; r.type = 0; r.swig = 0; r.g0 = lo; r.g1 = lo; r.n = 0; r.VA = 0; r.VB = 0;
    const uint32_t nseg = pl->n_seg;
    for (; s < nseg; s++) {
        const uint32_t base = pl->seg[s].base, rows = pl->seg[s].rows;
        if (max(lo, base) < min(hi, base + rows)) break;
    }
    if (s >= nseg) return r;
    const uint32_t base = pl->seg[s].base, rows = pl->seg[s].rows, ib = pl->seg[s].ib, ipr = pl->ipr;
    r.ok = 1; r.s = s; r.type = pl->seg[s].type; r.swig = pl->seg[s].swig;
    r.g0 = max(lo, base);
    r.g1 = min(hi, base + rows);
    if (epi_loads(pl->seg[s].epi)) r.g1 = min(r.g1, r.g0 + min(64u, pl->R));
    r.n = (r.g1 - r.g0) * ipr;
    const uint64_t off = (uint64_t)(r.g0 - base) * ipr * ib;
    r.VA = pl->seg[s].wa + off;
    r.VB = pl->seg[s].wb + off;
    return r;
}

// ------------------------------------------------------------ streaming

// Registers of the weight items in flight: D slots of NI 16-byte loads per
// lane.  The first DPRE slots are loaded across the grid barrier, slots up
// to DPRO during the prologue (issued behind its activation DMAs), the rest
// when the body starts -- at most PF_PRE registers of 16 B stay live through
// the prologue.  Measured on the 27B decode: Q4_K with D = 3 is 0.4 % faster
// than with a fourth slot in the body and 0.6 % faster than D = 2 (a lane's
// item is nine 16-byte loads 144 B apart, so each load instruction of a wave
// touches ~64 cache lines: a stream probe of that pattern reads 5.4 TB/s with
// two items in flight per lane and 4.5 with four); a third Q6_K slot is 1 %
// faster than two, a fourth 3.8 % slower; a fourth Q4_K slot across the
// barrier (DPRE = 4) was 0.6 % slower; moving a slot from across the barrier
// to the prologue (DPRE < DPRO), or more slots live through the prologue
// (which then spill), is slower -- loads issued behind the activation DMAs
// delay the activation reads of the workgroups released later.  A Q6_K block (210 B, 2-aligned) is read as 13 x 16 B + 4 B from the
// 4-aligned address at or below it: every byte read lies in
// [block - 2, block + 210), never past the end of the weights.
constexpr int PF_MAX = 42, PF_PRE = 28;
template <int T> struct TypeCfg;
template <> struct TypeCfg<SINTER_Q4_K> { static constexpr int NI = 9, IB = 144, D = 3, DPRE = 3, DPRO = 3; };
template <> struct TypeCfg<SINTER_Q6_K> { static constexpr int NI = 14, IB = 210, D = 3, DPRE = 2, DPRO = 2; };
template <> struct TypeCfg<SINTER_Q8_0> { static constexpr int NI = 17, IB = 272, D = 2, DPRE = 1, DPRO = 1; };
template <> struct TypeCfg<SINTER_BF16> { static constexpr int NI = 8, IB = 128, D = 4, DPRE = 3, DPRO = 3; };
template <> struct TypeCfg<SINTER_F32> { static constexpr int NI = 16, IB = 256, D = 2, DPRE = 1, DPRO = 1; };

// Weight loads use the default cache policy: a lane's item spans several
// 16-byte loads whose cache lines the other loads of the same step share,
// so the lines must stay in L1/L2 until all of them have read (measured: a
// non-temporal policy re-fetches them and halves the streaming rate).
__device__ __forceinline__ u32x4 ldw16(uint64_t p) { return *reinterpret_cast<const GLB u32x4 *>(p); }
__device__ __forceinline__ uint32_t ldw4(uint64_t p) { return *reinterpret_cast<const GLB uint32_t *>(p); }
typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));
__device__ __forceinline__ u32x4 ldw16a4(uint64_t p) {
    const u32x4a4 v = *reinterpret_cast<const GLB u32x4a4 *>(p);
    u32x4 o = {v.x, v.y, v.z, v.w};
    return o;
}

// the lane's matrix (SwiGLU pair: odd lanes read B) and its item within a step
__device__ __forceinline__ uint32_t lane_item(bool swig) { return swig ? (uint32_t)lane_id() >> 1 : (uint32_t)lane_id(); }

// Load item f of the run into slot S.  Every step loads unconditionally, so
// the compiler counts the loads in flight exactly and waits for a slot with
// a partial vmcnt (a load that might be skipped makes it wait for all of
// them): lanes past the run's end read the same bytes of `dummy` (the op's
// plan in device memory, L2-resident) instead.
template <int T, int S>
__device__ __forceinline__ void issue_item(u32x4 (&pf)[PF_MAX], uint32_t (&sh)[4], const Run &r, uint32_t f,
                                           uint64_t dummy) {
    constexpr int NI = TypeCfg<T>::NI, IB = TypeCfg<T>::IB;
    static_assert((S + 1) * NI <= PF_MAX, "prefetch slots");
    uint64_t A = ((r.swig && (lane_id() & 1)) ? r.VB : r.VA) + (uint64_t)f * IB;
    A = f < r.n ? A : dummy;
    if constexpr (T == SINTER_Q6_K) {
        sh[S] = (uint32_t)A & 3u;
        A &= ~(uint64_t)3;
#pragma unroll
        for (int i = 0; i < NI - 1; i++) pf[S * NI + i] = ldw16a4(A + 16 * i);
        pf[S * NI + NI - 1].x = ldw4(A + 16 * (NI - 1));
    } else {
#pragma unroll
        for (int i = 0; i < NI; i++) pf[S * NI + i] = ldw16(A + 16 * i);
    }
}

// Load slots [S0, S1) of the run's first steps.
template <int T, int S0, int S1>
__device__ __forceinline__ void issue_slots(u32x4 (&pf)[PF_MAX], uint32_t (&sh)[4], const Run &r, uint64_t dummy) {
    const uint32_t si = r.swig ? 32u : 64u, f0 = lane_item(r.swig != 0);
    if constexpr (S0 <= 0 && 0 < S1) issue_item<T, 0>(pf, sh, r, f0, dummy);
    if constexpr (S0 <= 1 && 1 < S1) issue_item<T, 1>(pf, sh, r, f0 + si, dummy);
    if constexpr (S0 <= 2 && 2 < S1) issue_item<T, 2>(pf, sh, r, f0 + 2 * si, dummy);
    if constexpr (S0 <= 3 && 3 < S1) issue_item<T, 3>(pf, sh, r, f0 + 3 * si, dummy);
}

// has_w<F, T>: whether the interpreter compiled for feature set F handles
// weight type T.  with_wtype<F>(t, f) calls f(integral_constant<int, T>) for
// run type t: a plain two-way choice in the K-quant interpreter, one case
// per handled type otherwise (types outside F: no call; the op checked the
// plan against F first).
template <uint32_t F, int T> constexpr bool has_w = (F & feat_w(T)) != 0;
template <uint32_t F, class Fn>
__device__ __forceinline__ void with_wtype(uint32_t t, Fn &&f) {
    constexpr uint32_t FW = F & (FEAT_W_Q4K | FEAT_W_Q6K | FEAT_W_Q80 | FEAT_W_BF16 | FEAT_W_F32);
    if constexpr (FW == (FEAT_W_Q4K | FEAT_W_Q6K)) {
        if (t == SINTER_Q6_K) f(std::integral_constant<int, SINTER_Q6_K>{});
        else f(std::integral_constant<int, SINTER_Q4_K>{});
    } else if constexpr (FW == FEAT_W_BF16) {
        f(std::integral_constant<int, SINTER_BF16>{});
    } else {
        switch (t) {
        case SINTER_Q4_K: if constexpr (has_w<F, SINTER_Q4_K>) f(std::integral_constant<int, SINTER_Q4_K>{}); break;
        case SINTER_Q6_K: if constexpr (has_w<F, SINTER_Q6_K>) f(std::integral_constant<int, SINTER_Q6_K>{}); break;
        case SINTER_Q8_0: if constexpr (has_w<F, SINTER_Q8_0>) f(std::integral_constant<int, SINTER_Q8_0>{}); break;
        case SINTER_BF16: if constexpr (has_w<F, SINTER_BF16>) f(std::integral_constant<int, SINTER_BF16>{}); break;
        case SINTER_F32: if constexpr (has_w<F, SINTER_F32>) f(std::integral_constant<int, SINTER_F32>{}); break;
        default: break;
        }
    }
}

// The slots loaded before the prologue (dispatch on the run's type).
template <uint32_t F>
__device__ __forceinline__ void issue_pre(u32x4 (&pf)[PF_MAX], uint32_t (&sh)[4], const Run &r, uint64_t dummy) {
    if (!r.ok) return;
    with_wtype<F>(r.type, [&](auto Tc) {
        constexpr int T = decltype(Tc)::value;
        issue_slots<T, 0, TypeCfg<T>::DPRE>(pf, sh, r, dummy);
    });
}

// Slots [DPRE, DPRO), issued right after the prologue's LDS-DMAs
// so that they stream while the activation is normalised and quantised;
// then the wait for those DMAs, which leaves exactly these loads in flight
// (vmcnt counts in order).  Without a run nothing is issued and the wait is
// for everything.  WAIT = false: issue only (a later run of the wave).
template <int T, bool WAIT>
__device__ __forceinline__ void issue_post_t(u32x4 (&pf)[PF_MAX], uint32_t (&sh)[4], const Run &r, uint64_t dummy) {
    constexpr int DPRO = TypeCfg<T>::DPRO, DPRE = TypeCfg<T>::DPRE, N = (DPRO - DPRE) * TypeCfg<T>::NI;
    static_assert(N < 64 && DPRO * TypeCfg<T>::NI <= PF_PRE && DPRE <= DPRO && DPRO <= TypeCfg<T>::D,
                  "vmcnt range, registers live through the prologue");
    issue_slots<T, DPRE, DPRO>(pf, sh, r, dummy);
    if constexpr (WAIT) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
template <uint32_t F, bool WAIT>
__device__ __forceinline__ void issue_post(u32x4 (&pf)[PF_MAX], uint32_t (&sh)[4], const Run &r, uint64_t dummy) {
    if (!r.ok) {
        if constexpr (WAIT) dma_wait();
        return;
    }
    with_wtype<F>(r.type, [&](auto Tc) { issue_post_t<decltype(Tc)::value, WAIT>(pf, sh, r, dummy); });
}

// Epilogues that read operands (residual add, conv) run only in the fold at
// the end of a run, whose rows are capped at 64 (longer ranges are split into
// runs): row q's operands are loaded into lane q right after the grid
// barrier, so they queue behind the weights loaded before it and have landed
// when the prologue's DMA wait returns -- a load inside the streaming loop
// would wait for every weight load in flight (vmcnt counts in order).
// RESID: v[0] = residual; CONV (dc <= 4 taps): v[0..dc-2] = state,
// v[3..3+dc) = conv weights.
struct EpiPre {
    float v[7];
};
__device__ __forceinline__ void epi_preload(cplan_t *pl, const Run &r, EpiPre &ev) {
#pragma unroll
    for (int j = 0; j < 7; j++) ev.v[j] = 0.0f;
    if (!r.ok) return;
    const uint32_t epi = pl->seg[r.s].epi, q = lane_id(), row = r.g0 + q - pl->seg[r.s].base;
    if (q >= r.g1 - r.g0) return;
    if (epi == SINTER_EPI_RESID) {
        const __amdgpu_buffer_rsrc_t ar = coh_rsrc(reinterpret_cast<const void *>(pl->seg[r.s].aux), 0x7fffffff);
        ev.v[0] = ld_coh4b(ar, row * 4);
    } else if (epi == SINTER_EPI_CONV) {
        const uint32_t dc = pl->seg[r.s].dconv;
        const GLB float *st = reinterpret_cast<const GLB float *>(pl->seg[r.s].aux) + (size_t)row * (dc - 1);
        const GLB float *cw = reinterpret_cast<const GLB float *>(pl->seg[r.s].w2) + (size_t)row * dc;
#pragma unroll
        for (uint32_t j = 0; j < 3; j++) if (j + 1 < dc) ev.v[j] = st[j];
#pragma unroll
        for (uint32_t j = 0; j < 4; j++) if (j < dc) ev.v[3 + j] = cw[j];
    }
}

// Row epilogue of segment row r (segment s of the plan): dot (and the up dot
// of a SwiGLU pair); greedy-argmax candidates fold into (bv, bi).  FULL: the
// end-of-run fold (every mode; RESID/CONV use this lane's preloaded
// operands); otherwise the in-loop fold (STORE / SWIGLU / ARGMAX only).
template <bool FULL>
__device__ __forceinline__ void epi_row(cplan_t *pl, uint32_t s, __amdgpu_buffer_rsrc_t yr, uint32_t r, float dot,
                                        float up, float &bv, int32_t &bi, const EpiPre &ev) {
    float y = dot;
    const uint32_t epi = pl->seg[s].epi;
    if (epi == SINTER_EPI_SWIGLU) {
        y = dev_silu(dot) * up;
    } else if (epi == SINTER_EPI_SILU) {
        y = dev_silu(dot);
    } else if (FULL && epi == SINTER_EPI_RESID) {
        y = ev.v[0] + dot;
    } else if (FULL && epi == SINTER_EPI_CONV) {
        // causal conv over {state[0..dc-2], dot}, fp64 sum rounded once,
        // then silu; the state shifts by one tap (this wave owns row r)
        const uint32_t dc = pl->seg[s].dconv;
        GLB float *st = reinterpret_cast<GLB float *>(pl->seg[s].aux) + (size_t)r * (dc - 1);
        double cacc = 0.0;
#pragma unroll
        for (uint32_t j = 0; j < 4; j++) {
            const float wv = (j + 1 < dc) ? ev.v[j < 3 ? j : 2] : dot;
            if (j < dc) cacc += (double)wv * (double)ev.v[3 + j];
        }
        y = dev_silu((float)cacc);
#pragma unroll
        for (uint32_t j = 0; j < 3; j++)
            if (j + 1 < dc) st[j] = (j + 2 < dc) ? ev.v[j + 1 < 3 ? j + 1 : 2] : dot;
    } else if (epi == SINTER_EPI_ARGMAX) {
        if (y > bv || (y == bv && (int32_t)r < bi)) { bv = y; bi = (int32_t)r; }
    }
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(y), yr, r * 4, 0, CPOL_SC1);
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

// What the streaming loop keeps of the op (wave-uniform).
struct GemvCtx {
    uint32_t ipr, mipr, P, R, mR;
    uint32_t qs, rs, qs2, rs2;          // a 64-item step (32 for SwiGLU pairs) in rows + items
    LDS double *ring;                   // this wave's ring (A); B = ring + RING_CAP/2
    uint64_t dummy;                     // readable device bytes for loads past a run's end
};

// Fold the run's rows [lo, hi) (run-local) -- row q on lane q % 64 -- and
// apply the epilogues.
template <bool FULL>
__device__ __forceinline__ void fold_rows(const GemvCtx &c, cplan_t *pl, const Run &r, uint32_t lo, uint32_t hi,
                                          float &bv, int32_t &bi, const EpiPre &ev) {
    const uint32_t lane = lane_id();
    const bool swig = r.swig != 0;
    const uint32_t seg_base = pl->seg[r.s].base;
    const __amdgpu_buffer_rsrc_t yr = coh_rsrc(reinterpret_cast<const void *>(pl->seg[r.s].y), 0x7fffffff);
    for (uint32_t b = lo & ~63u; b < hi; b += 64) {
        const uint32_t q = b + lane;
        if (q >= lo && q < hi) {
            uint32_t slot;
            (void)divm(q, c.R, c.mR, slot);
            const double s = fold_row(c.ring + slot * c.P, c.P);
            double u = 0.0;
            if (swig) u = fold_row(c.ring + RING_CAP / 2 + slot * c.P, c.P);
            epi_row<FULL>(pl, r.s, yr, r.g0 + q - seg_base, (float)s, (float)u, bv, bi, ev);
        }
    }
}

// The body of one run whose first DPRO slots were loaded: the remaining
// slots, then steps of terms into the ring, rows folded as the ring fills.
// FOLD_END: fold the run's last rows here; otherwise return the first row
// not folded yet and the caller folds the rest (one copy of the final fold
// and its epilogues for every weight type of an interpreter that handles
// several, so less code competes for the instruction cache).
template <int T, bool FOLD_END>
__device__ __forceinline__ uint32_t run_body(u32x4 (&pf)[PF_MAX], uint32_t (&sh)[4], const GemvCtx &c, cplan_t *pl,
                                             const Run &r, const ActView &x, float &bv, int32_t &bi,
                                             const EpiPre &ev) {
    constexpr int D = TypeCfg<T>::D, NI = TypeCfg<T>::NI;
    issue_slots<T, TypeCfg<T>::DPRO, D>(pf, sh, r, c.dummy);
    const bool swig = r.swig != 0;
    const uint32_t si = swig ? 32u : 64u, qs = swig ? c.qs2 : c.qs, rs = swig ? c.rs2 : c.rs;
    const uint32_t n = r.n, nJ = (n + si - 1) / si, nrows = r.g1 - r.g0;
    // lane state: item f = si*j + lane_item is item k of run-local row q (ring slot)
    const uint32_t f0 = lane_item(swig);
    uint32_t k, q = divm(f0, c.ipr, c.mipr, k), slot;
    (void)divm(q, c.R, c.mR, slot);
    uint32_t folded = 0;
    LDS double *ring = c.ring + ((swig && (lane_id() & 1)) ? RING_CAP / 2 : 0u);
    // every step computes (lanes past the end masked) and loads D steps
    // ahead (past the end: the dummy), whole groups of D steps
    auto step = [&](auto Sc, uint32_t j) {
        constexpr int S = decltype(Sc)::value;
        const uint32_t f = si * j + f0;
        if (f < n) ring[slot * c.P + k] = item_term<T>(&pf[S * NI], sh[S], x, k);
        // this lane's next item
        k += rs;
        q += qs;
        slot += qs;
        if (k >= c.ipr) { k -= c.ipr; q += 1; slot += 1; }
        if (slot >= c.R) slot -= c.R;
        issue_item<T, S>(pf, sh, r, f + si * D, c.dummy);
    };
    for (uint32_t j0 = 0; j0 < nJ; j0 += D) {
        // ring room for rows [folded, last row of this group of D steps]
        // (runs with operand-reading epilogues have at most R rows, so this
        // never fires for them)
        uint32_t rem;
        const uint32_t last = divm(min(n, si * (j0 + D)) - 1, c.ipr, c.mipr, rem);
        if (last - folded + 1 > c.R) {
            const uint32_t first = divm(si * j0, c.ipr, c.mipr, rem);
            fold_rows<false>(c, pl, r, folded, first, bv, bi, ev);
            folded = first;
        }
        step(std::integral_constant<int, 0>{}, j0);
        if constexpr (D > 1) step(std::integral_constant<int, 1>{}, j0 + 1);
        if constexpr (D > 2) step(std::integral_constant<int, 2>{}, j0 + 2);
        if constexpr (D > 3) step(std::integral_constant<int, 3>{}, j0 + 3);
    }
    if constexpr (FOLD_END) {
        fold_rows<true>(c, pl, r, folded, nrows, bv, bi, ev);
        return nrows;
    }
    return folded;
}

// (measured: the shared final fold is 1 % faster in the K-quant decode, and
// 4.5 % slower for the general interpreter's Q8_0 GEMV -- that interpreter
// and the bf16 one keep the fold in each type's body)
template <uint32_t F>
__device__ __forceinline__ void run_dispatch(u32x4 (&pf)[PF_MAX], uint32_t (&sh)[4], const GemvCtx &c, cplan_t *pl,
                                             const Run &r, const ActView &x, float &bv, int32_t &bi,
                                             const EpiPre &ev) {
    constexpr uint32_t FW = F & (FEAT_W_Q4K | FEAT_W_Q6K | FEAT_W_Q80 | FEAT_W_BF16 | FEAT_W_F32);
    constexpr bool shared = FW == (FEAT_W_Q4K | FEAT_W_Q6K);   // the K-quant interpreters
    if constexpr (shared) {
        uint32_t folded = 0;
        with_wtype<F>(r.type, [&](auto Tc) {
            folded = run_body<decltype(Tc)::value, false>(pf, sh, c, pl, r, x, bv, bi, ev);
        });
        fold_rows<true>(c, pl, r, folded, r.g1 - r.g0, bv, bi, ev);
    } else {
        with_wtype<F>(r.type, [&](auto Tc) { (void)run_body<decltype(Tc)::value, true>(pf, sh, c, pl, r, x, bv, bi, ev); });
    }
}

// Whether the interpreter compiled for F runs the planned GEMV: its
// activation type and every segment's weight type are in F (the host picks
// a kernel whose set covers the program, so this only guards against a
// mismatch: a run read with another type's item size would stream past its
// matrix).
template <uint32_t F>
__device__ __forceinline__ bool plan_in_set(cplan_t *pl) {
    if constexpr (F == FEAT_ALL) return true;
    else return (pl->feat & ~F) == 0;
}

// ------------------------------------------------------------ the op

// Returns false when the kernel must stop (barrier timeout, or an error seen
// at a pass end).
// ts (thread 0, or null): wall clock stamps [1] after the barrier wait,
// [2] after the prologue.  hdr: the instruction's header (ins_hdr).
template <uint32_t F>
__device__ __forceinline__ bool gemv_op(const sinter_instr &ins, const GemvPlan *plan, const uint32_t *cuts,
                                       unsigned *err, GridCross *gx, uint64_t *ts, uint64_t hdr) {
    cplan_t *pl = (cplan_t *)plan;
    cu32_t *cu = (cu32_t *)cuts;
    const uint32_t rel = uni(blockIdx.x - hdr_lo(hdr)), nblk = uni(hdr_hi(hdr) - hdr_lo(hdr));
    bool planned = false, ok = false;
    uint32_t row_hi = 0;
    Run run;
    u32x4 pf[PF_MAX];
    uint32_t sh[4] = {0, 0, 0, 0};
    // The op's reads of its payload and plan are memory round trips (the
    // program and the plans are far larger than the scalar cache): they run
    // between the barrier's arrival and its wait, so the last workgroup to
    // arrive does not wait for them before it arrives.  The payload goes to
    // LDS first (its wait then covers no weight load); then the plan, this
    // wave's run and the first weight slots.
    auto setup = [&] {
        if (threadIdx.x < sizeof(sinter_gemv_args) / 4)
            reinterpret_cast<uint32_t *>(g_args)[threadIdx.x] =
                reinterpret_cast<const uint32_t *>(ins.payload)[threadIdx.x];
        // (a plan outside this interpreter's feature set raises UNWIRED_KIND)
        planned = pl->ok != 0;
        ok = planned && plan_in_set<F>(pl);
        const uint32_t wv = rel * WAVES + uni(wave_id());
        const uint32_t row_lo = ok ? cu[wv] : 0u;
        row_hi = ok ? cu[wv + 1] : 0u;
        run = make_run(pl, 0, row_lo, row_hi);
        issue_pre<F>(pf, sh, run, (uint64_t)plan);
    };
    if (gx) {
        // (the wait's workgroup barrier publishes g_args)
        if (!cross_barrier(*gx, setup)) return false;
    } else {
        setup();
        __syncthreads();
    }
    if (ts) ts[1] = wall_clock64();
    EpiPre ev;
    epi_preload(pl, run, ev);
    if (!ok) {
        if (rel == 0 && threadIdx.x == 0)
            raise_error(err, planned ? SINTER_E_UNWIRED_KIND : SINTER_E_BAD_SHAPE, ins.dbg_node);
        settle_vmem();
        __syncthreads();
        return true;
    }
    const sinter_gemv_args &a = *reinterpret_cast<const sinter_gemv_args *>(g_args);
    const uint32_t K = a.K;
    const int vt = (int)pl->vt;
    const bool write_x = (a.pro == SINTER_PRO_EMBED) && rel == 0 && a.x_out != nullptr;
    // the remaining weight slots stream during the prologue (issued after
    // its activation DMAs, which the prologue then waits for)
    gemv_prologue<F>(a, vt, write_x, g_red, err, [&] { issue_post<F, true>(pf, sh, run, (uint64_t)plan); });
    if (ts) ts[2] = wall_clock64();
    const ActView x = act_view(g_qbuf, K, vt);

    // this wave's term ring (aliases the prologue's staging, done now): every
    // slot starts as -0.0 (pad slots keep it)
    GemvCtx c;
    c.ipr = pl->ipr; c.mipr = pl->mipr; c.P = pl->P; c.R = pl->R; c.mR = pl->mR;
    c.qs = pl->q64; c.rs = pl->r64; c.qs2 = pl->q32; c.rs2 = pl->r32;
    c.ring = reinterpret_cast<LDS double *>((lds_char *)g_big) + uni(wave_id()) * RING_CAP;
    c.dummy = (uint64_t)plan;
    {
        typedef double f64x2 __attribute__((ext_vector_type(2)));
        LDS f64x2 *rv = reinterpret_cast<LDS f64x2 *>(c.ring);
        const f64x2 mz = {-0.0, -0.0};
#pragma unroll
        for (uint32_t i = 0; i < RING_CAP / 128; i++) rv[i * 64 + lane_id()] = mz;
    }

    float bv = -INFINITY;
    int32_t bi = 0x7fffffff;
    while (run.ok) {
        run_dispatch<F>(pf, sh, c, pl, run, x, bv, bi, ev);
        run = make_run(pl, run.s, run.g1, row_hi);
        if (!run.ok) break;
        issue_pre<F>(pf, sh, run, (uint64_t)plan);
        issue_post<F, false>(pf, sh, run, (uint64_t)plan);
        epi_preload(pl, run, ev);
    }

    // greedy argmax: block-local best, then the last-arriving block reduces
    const bool any_argmax = pl->any_argmax != 0;
    if (any_argmax) {
        // block reduction of (value, index): larger value, then smaller index
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(bv, o, 64);
            const int32_t oi = __shfl_xor(bi, o, 64);
            if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
        }
        LDS float *rv = reinterpret_cast<LDS float *>((LDS double *)g_part);
        LDS int32_t *ri = reinterpret_cast<LDS int32_t *>((LDS double *)g_part + 4);
        if (lane_id() == 0) { rv[wave_id()] = bv; ri[wave_id()] = bi; }
        __syncthreads();
        if (threadIdx.x == 0) {
            for (int w = 1; w < (int)WAVES; w++)
                if (rv[w] > bv || (rv[w] == bv && ri[w] < bi)) { bv = rv[w]; bi = ri[w]; }
        }
    }
    if (any_argmax) {
        sinter_argmax_ws *ws = static_cast<sinter_argmax_ws *>(a.epi_ws);
        __shared__ unsigned am_last;
        if (threadIdx.x == 0) {
            am_last = 0;
            if (rel >= ws->capacity) {
                raise_error(err, SINTER_E_BAD_SHAPE, ins.dbg_node);
            } else {
                st_coh(ws->part_val + rel, bv);
                st_coh(ws->part_idx + rel, bi);
                settle_vmem();
                const unsigned old = __hip_atomic_fetch_add(gp(ws->count), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                am_last = old == nblk - 1 ? 1u : 0u;
            }
        }
        __syncthreads();
        if (am_last) {
            // the last arriver reduces the nblk partials: every load at once
            // (thread t takes t, t+256, ...), then lanes and waves combined;
            // larger value wins, then the smaller index (NaNs never win: each
            // lane starts from -inf)
            float best = -INFINITY;
            int32_t bidx = 0x7fffffff;
            const __amdgpu_buffer_rsrc_t vr = coh_rsrc(ws->part_val, nblk * 4), ir = coh_rsrc(ws->part_idx, nblk * 4);
            float pv[PLAN_MAX_BLOCKS / BLOCK_THREADS];
            int32_t pi[PLAN_MAX_BLOCKS / BLOCK_THREADS];
#pragma unroll
            for (uint32_t k = 0; k < PLAN_MAX_BLOCKS / BLOCK_THREADS; k++) {
                const uint32_t w = min(threadIdx.x + k * BLOCK_THREADS, nblk - 1);
                pv[k] = ld_coh4b(vr, w * 4);
                pi[k] = __float_as_int(ld_coh4b(ir, w * 4));
            }
#pragma unroll
            for (uint32_t k = 0; k < PLAN_MAX_BLOCKS / BLOCK_THREADS; k++) {
                const bool in = threadIdx.x + k * BLOCK_THREADS < nblk;
                if (in && (pv[k] > best || (pv[k] == best && pi[k] < bidx))) { best = pv[k]; bidx = pi[k]; }
            }
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) {
                const float ov = __shfl_xor(best, o, 64);
                const int32_t oi = __shfl_xor(bidx, o, 64);
                if (ov > best || (ov == best && oi < bidx)) { best = ov; bidx = oi; }
            }
            LDS float *rv = reinterpret_cast<LDS float *>((LDS double *)g_part);
            LDS int32_t *ri = reinterpret_cast<LDS int32_t *>((LDS double *)g_part + 4);
            __syncthreads();
            if (lane_id() == 0) { rv[wave_id()] = best; ri[wave_id()] = bidx; }
            __syncthreads();
            if (threadIdx.x == 0) {
                for (int w = 1; w < (int)WAVES; w++)
                    if (rv[w] > best || (rv[w] == best && ri[w] < bidx)) { best = rv[w]; bidx = ri[w]; }
                sinter_pass_cell *pc = reinterpret_cast<sinter_pass_cell *>(ws->pass_cell);
                const int32_t steps = ld_coh(&pc->steps);
                // prefill: the prompt's next token instead of the argmax
                if (ws->forced && (uint32_t)steps + 1u < ws->n_forced) bidx = ws->forced[steps + 1];
                if (ws->history && (uint32_t)steps < ws->history_cap) st_coh(ws->history + steps, bidx);
                st_coh(&pc->steps, steps + 1);
                st_coh(&pc->token, bidx);
                st_coh(&pc->pos, ld_coh(&pc->pos) + 1);
                __hip_atomic_store(gp(ws->count), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
    __syncthreads();
    return true;
}

}  // namespace sinter
