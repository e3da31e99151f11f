// Batched GEMV over a ubatch of tokens: the trunk GEMM of a batched prefill
// (docs/PREFILL-SEMANTICS.md:286-313 in the reference: the fork's prefill
// multiplies quantised weights by quantised activations on int8 tensor
// cores, MMQ, instead of running the single-token GEMV once per token).
//
//   y[t][r] = (float) sum_i term(W[r] item i, X[t] item i),  t < n_tokens
//
// W: rows x K of ggml Q4_K or Q6_K super-blocks (the GGUF layout as-is);
// X: n_tokens Q8_K activations (ggml block_q8_K {f32 d; i8 qs[256];
// i16 bsums[16]}, K/256 blocks per token).  The item terms and their fold
// are the single-token GEMV's (gemv.h: one fp64 term per 256-element
// super-block, summed in item order), so every output is bit-identical to
// the decode GEMV of the same token; only the integer dot products move to
// MFMA.
//
// A workgroup of four waves owns 64 rows (16 per wave) and up to 64 tokens
// (four 16-token tiles), so each weight byte is read from HBM once per 64
// tokens.  Item by item the workgroup stages the 64 tokens' Q8_K blocks in
// LDS (double-buffered: the next item's are loaded while this one is
// computed) and every wave streams its own rows' weights.  Per item
// and token tile it runs v_mfma_i32_16x16x32_i8 with the tokens' codes as A
// (16 x 32, lane l: token l%16, elements 8(l/16)..+7 of the 32) and the rows'
// codes as B (32 x 16, lane l: row l%16, the same elements); D (16 x 16
// int32, lane l: row l%16, tokens 4(l/16)+v) holds one exact 32-element dot
// per (token, row).  A Q4_K sub-block is 32 elements, and two of them go
// through one 64-deep v_mfma_i32_16x16x64_i8 (the pair's 8-byte operands side
// by side: the sums accumulate over all sub-blocks anyway); a Q6_K sub-block
// is 16, so a 32-element chunk runs two 32-deep MFMAs, each with the other
// sub-block's half of B zeroed.  Q4_K's min term sum_s m_s * (sum of the
// sub-block's activation codes) is one more MFMA per sub-block pair, against
// B = m_s in every byte, accumulated across the sub-blocks in D.  Each lane then
// forms the fp64 term of its four (token, row) pairs from its own row's
// scales and folds it into its accumulators.
#include "internal.h"
#include "dev_common.h"

namespace sinter {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr uint32_t UB_ROWS = 16;     // rows per wave: the MFMA's N
constexpr uint32_t UB_TOK = 16;      // tokens per tile: the MFMA's M
constexpr uint32_t UB_TILES = 4;     // token tiles per wave
constexpr uint32_t UB_TOKENS = UB_TOK * UB_TILES;
constexpr uint32_t UB_THREADS = 256;  // four waves: 64 rows of the workgroup's row tile
constexpr uint32_t UB_WG_ROWS = UB_ROWS * (UB_THREADS / 64u);
constexpr uint32_t UB_XSTRIDE = 68;   // LDS dwords per staged token (65 used)
// fewest workgroups a launch splits its token groups to reach: two per CU, so
// each SIMD holds two waves to hide the latency of its MFMA / fp64 chains
// (4096-token prefill: 1.076 s at one per CU, 1.021 s at 384 or 512, 1.153 s
// at 768 or 1024, where the 5120-row matrices drop to one token tile per
// workgroup and read their weights four times)
constexpr uint64_t UB_MIN_WGS = 512;
constexpr uint32_t UB_CONV_MAX = 8;    // conv taps
constexpr uint32_t Q8K_BYTES = 292;  // block_q8_K
constexpr uint32_t Q4K_BYTES = 144, Q6K_BYTES = 210;

__device__ __forceinline__ uint32_t ld32(const uint8_t *p) { return *(const uint32_t *)p; }
__device__ __forceinline__ long pack64(uint32_t lo, uint32_t hi) {
    return (long)(((unsigned long)hi << 32) | lo);
}
// two 8-byte MFMA operands as one 16-byte operand (x in bytes 0-7)
__device__ __forceinline__ v4i pack128(long x, long y) {
    const v4i r = {(int)(uint32_t)x, (int)(uint32_t)((unsigned long)x >> 32), (int)(uint32_t)y,
                   (int)(uint32_t)((unsigned long)y >> 32)};
    return r;
}
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}
// 8 bytes at block byte o of a 2-aligned block whose 4-aligned base is
// base4 = block - sh (sh = 0 or 2): the third dword is read only when the
// bytes straddle it, so no read leaves the block's own 4-aligned span
__device__ __forceinline__ void ld8u(const uint8_t *base4, uint32_t o, uint32_t sh, uint32_t &lo, uint32_t &hi) {
    const uint32_t *p = (const uint32_t *)(base4 + o);
    const uint32_t d0 = p[0], d1 = p[1];
    const uint32_t d2 = sh ? p[2] : 0u;
    // v_alignbyte_b32: ({d1, d0} >> 8 * sh)[31:0] -- the shift counts bytes
    lo = __builtin_amdgcn_alignbyte(d1, d0, sh);
    hi = __builtin_amdgcn_alignbyte(d2, d1, sh);
}
// bytewise x - 32 for bytes 0..63 (no borrow crosses a byte)
__device__ __forceinline__ uint32_t sub32b(uint32_t x) { return ((x | 0x80808080u) - 0x20202020u) ^ 0x80808080u; }

template <int WT>
struct WItem;

// Q4_K: the lane's row header (d, dmin, 12 scale bytes) and its four 8-byte
// slices of qs (bytes 32p + 8g..+7: sub-block 2p in the low nibbles, 2p + 1
// in the high ones)
template <>
struct WItem<SINTER_Q4_K> {
    uint32_t h[4];
    uint32_t q[8];
    __device__ __forceinline__ void load(const uint8_t *row, uint32_t i, uint32_t g) {
        const uint8_t *b = row + (size_t)i * Q4K_BYTES;
        const uint4 hv = *(const uint4 *)b;
        h[0] = hv.x; h[1] = hv.y; h[2] = hv.z; h[3] = hv.w;
#pragma unroll
        for (uint32_t p = 0; p < 4; p++) {
            const uint2 v = *(const uint2 *)(b + 16u + 32u * p + 8u * g);
            q[2 * p] = v.x; q[2 * p + 1] = v.y;
        }
    }
};

// Q6_K: the lane's slices of ql (bytes 64n + 8g and 64n + 32 + 8g), qh
// (bytes 32n + 8g) for both halves n, the 16 int8 scales and d
template <>
struct WItem<SINTER_Q6_K> {
    uint32_t l0[4], l1[4], hh[4];   // [2n], [2n + 1]: lo / hi dwords of half n
    uint32_t sc[4];
    uint32_t d;
    __device__ __forceinline__ void load(const uint8_t *row, uint32_t i, uint32_t g) {
        const uint8_t *b = row + (size_t)i * Q6K_BYTES;
        const uint32_t sh = (uint32_t)((uintptr_t)b & 3u);
        const uint8_t *b4 = b - sh;
#pragma unroll
        for (uint32_t n = 0; n < 2; n++) {
            ld8u(b4, 64u * n + 8u * g, sh, l0[2 * n], l0[2 * n + 1]);
            ld8u(b4, 64u * n + 32u + 8u * g, sh, l1[2 * n], l1[2 * n + 1]);
            ld8u(b4, 128u + 32u * n + 8u * g, sh, hh[2 * n], hh[2 * n + 1]);
        }
        ld8u(b4, 192u, sh, sc[0], sc[1]);
        ld8u(b4, 200u, sh, sc[2], sc[3]);
        d = *(const uint16_t *)(b + 208);
    }
};

// Stage item i of the workgroup's tokens in LDS: token j's Q8_K block i (its
// 256 codes at dwords 0..63 of LDS row j, its d at dword 64).  Wave w stages
// token tile w, four lanes per token, each lane 16 code dwords (and the
// first of the four, d), so the per-item work is one address update and
// loads at immediate offsets.  Tokens past the last repeat it (never
// stored).  ld: into registers; st: registers to LDS buffer xs.
struct ActStage {
    uint32_t v[16], d;
    const uint8_t *blk0;   // the lane's token's block 0
    uint32_t part, row;    // 16-dword quarter of the codes; LDS row (token within the group)
    __device__ __forceinline__ void init(const uint8_t *xq, uint32_t nb, uint32_t tok0, uint32_t n_tok) {
        const uint32_t lane = threadIdx.x & 63u;
        row = UB_TOK * (threadIdx.x >> 6) + (lane >> 2);
        part = lane & 3u;
        const uint32_t tok = min(tok0 + row, n_tok - 1u);
        blk0 = xq + (size_t)tok * nb * Q8K_BYTES;
    }
    __device__ __forceinline__ void ld(uint32_t i) {
        const uint8_t *b = blk0 + (size_t)i * Q8K_BYTES;
        const uint32_t *c = (const uint32_t *)(b + 4u + 64u * part);
#pragma unroll
        for (uint32_t k = 0; k < 16; k++) v[k] = c[k];
        if (part == 0) d = *(const uint32_t *)b;
    }
    __device__ __forceinline__ void st(uint32_t *xs) const {
        uint32_t *r = xs + row * UB_XSTRIDE;
#pragma unroll
        for (uint32_t k = 0; k < 4; k++)
            *(uint4 *)(r + 16u * part + 4u * k) = make_uint4(v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]);
        if (part == 0) r[64] = d;
    }
};
static_assert(UB_THREADS / 64u == UB_TILES, "one staging wave per token tile");
static_assert(UB_XSTRIDE % 4u == 0, "16-byte LDS row alignment");

template <int WT>
__global__ __launch_bounds__(UB_THREADS) void ubatch_gemv_kernel(const uint8_t *__restrict__ w, uint32_t rows,
                                                                uint32_t nb, const uint8_t *__restrict__ xq,
                                                                uint32_t n_tok, float *__restrict__ y, uint32_t n_tg,
                                                                uint32_t tpw, uint32_t accumulate) {
    __shared__ uint32_t xs[2][UB_TOKENS * UB_XSTRIDE];
    const uint32_t lane = threadIdx.x & 63u, wv = threadIdx.x >> 6, r = lane & 15u, g = lane >> 4;
    // adjacent workgroups share a row tile (their token groups): its weight
    // bytes come from HBM once and from the memory-side cache after
    const uint32_t rt = blockIdx.x / n_tg, tg = blockIdx.x % n_tg;
    const uint32_t row = rt * UB_WG_ROWS + wv * UB_ROWS + r;
    const uint32_t rowc = row < rows ? row : rows - 1u;
    const uint32_t tok0 = tg * UB_TOK * tpw;
    const uint32_t ntiles = min(tpw, (n_tok - tok0 + UB_TOK - 1u) / UB_TOK);   // block-uniform, 1..4
    const size_t row_bytes = (size_t)nb * (WT == SINTER_Q4_K ? Q4K_BYTES : Q6K_BYTES);
    const uint8_t *wrow = w + (size_t)rowc * row_bytes;

    double acc[UB_TILES][4];
#pragma unroll
    for (uint32_t t = 0; t < UB_TILES; t++)
#pragma unroll
        for (uint32_t v = 0; v < 4; v++) acc[t][v] = 0.0;

    ActStage stage;
    // wave w stages token tile w, when the group has it (wave-uniform)
    const bool stager = (threadIdx.x >> 6) < ntiles;
    stage.init(xq, nb, tok0, n_tok);
    if (stager) stage.ld(0);
    WItem<WT> cur, nxt;
    cur.load(wrow, 0, g);
    if (stager) stage.st(xs[0]);
    __syncthreads();
    for (uint32_t i = 0; i < nb; i++) {
        if (i + 1u < nb) {
            // activations first: vector loads complete in order, so the
            // staging store at the end of this item then waits for these
            // cache hits and not for the weights behind them
            if (stager) stage.ld(i + 1u);
            nxt.load(wrow, i + 1u, g);
        }
        const uint32_t *xb = xs[i & 1u];

        // B operands and the per-sub-block integer scales of the lane's row
        long b[8];       // Q4_K: codes x the scale's low 3 bits; Q6_K: codes
        long bh[8];      // Q4_K: codes x the scale's high 3 bits
        long bm[8];      // Q4_K: the min in every byte
        int scl[16];     // Q6_K: the 16 sub-block scales
        float dw, dmin = 0.0f;
        if constexpr (WT == SINTER_Q4_K) {
            // ggml get_scale_min_k4 for sub-blocks 0..7, four at a time
            const uint32_t s0 = cur.h[1], s1 = cur.h[2], s2 = cur.h[3];
            const uint32_t dlo = s0 & 0x3F3F3F3Fu, mlo = s1 & 0x3F3F3F3Fu;
            const uint32_t dhi = (s2 & 0x0F0F0F0Fu) | ((s0 >> 2) & 0x30303030u);
            const uint32_t mhi = ((s2 >> 4) & 0x0F0F0F0Fu) | ((s1 >> 2) & 0x30303030u);
#pragma unroll
            for (uint32_t s = 0; s < 8; s++) {
                const uint32_t sd = ((s < 4 ? dlo : dhi) >> (8u * (s & 3u))) & 0xFFu;
                const uint32_t sm = ((s < 4 ? mlo : mhi) >> (8u * (s & 3u))) & 0xFFu;
                const uint32_t mm = sm * 0x01010101u;
                bm[s] = pack64(mm, mm);
                const uint32_t p = s >> 1, sh = 4u * (s & 1u);
                const uint32_t q0 = (cur.q[2 * p] >> sh) & 0x0F0F0F0Fu, q1 = (cur.q[2 * p + 1] >> sh) & 0x0F0F0F0Fu;
                // scale = 8 hi + lo (hi, lo <= 7): a code (<= 15) times either
                // fits a byte (<= 105), so one 32-bit multiply scales four
                // codes with no carry between them, and the products are
                // int8 operands
                const uint32_t lo = sd & 7u, hi = sd >> 3;
                b[s] = pack64(q0 * lo, q1 * lo);
                bh[s] = pack64(q0 * hi, q1 * hi);
            }
            dw = f16_bits_to_f32(cur.h[0] & 0xFFFFu);
            dmin = f16_bits_to_f32(cur.h[0] >> 16);
        } else {
#pragma unroll
            for (uint32_t c = 0; c < 8; c++) {
                const uint32_t n = c >> 2, q = c & 3u;
                const uint32_t *L = (q & 1u) ? cur.l1 : cur.l0;
                const uint32_t ls = 4u * (q >> 1), hs = 2u * q;
                uint32_t lo = ((L[2 * n] >> ls) & 0x0F0F0F0Fu) | (((cur.hh[2 * n] >> hs) & 0x03030303u) << 4);
                uint32_t hi = ((L[2 * n + 1] >> ls) & 0x0F0F0F0Fu) | (((cur.hh[2 * n + 1] >> hs) & 0x03030303u) << 4);
                b[c] = pack64(sub32b(lo), sub32b(hi));
            }
#pragma unroll
            for (uint32_t j = 0; j < 16; j++) scl[j] = (int)(int8_t)((cur.sc[j >> 2] >> (8u * (j & 3u))) & 0xFFu);
            dw = f16_bits_to_f32(cur.d);
        }

#pragma unroll
        for (uint32_t t = 0; t < UB_TILES; t++) {
            if (t < ntiles) {
                // A: token 16t + r, elements 32c + 8g..+7 (row stride 68 dwords: the
                // 32 lanes of a half-wave read 32 distinct bank pairs)
                const uint32_t *xa = xb + (UB_TOK * t + r) * UB_XSTRIDE + 2u * g;
                long a[8];
#pragma unroll
                for (uint32_t c = 0; c < 8; c++) {
                    const uint2 v2 = *(const uint2 *)(xa + 8u * c);
                    a[c] = pack64(v2.x, v2.y);
                }
                float dx[4];
#pragma unroll
                for (uint32_t v = 0; v < 4; v++)
                    dx[v] = __builtin_bit_cast(float, xb[(UB_TOK * t + 4u * g + v) * UB_XSTRIDE + 64u]);
                const v4i z = {0, 0, 0, 0};
                int isum[4] = {0, 0, 0, 0};
                if constexpr (WT == SINTER_Q4_K) {
                    // sum_s scale_s dot_s = 8 sum_s hi_s dot_s + sum_s lo_s dot_s, all
                    // exact in int32 (|each| <= 256 * 105 * 128).  Sub-blocks s and
                    // s + 1 go through one 64-deep MFMA: A and B carry sub-block s in
                    // bytes 0-7 of each lane and s + 1 in bytes 8-15 (the MFMA pairs
                    // A and B bytes by the same lane-group / byte k index, so any
                    // common placement gives the same exact sums)
                    v4i cm = z, ch = z, cl = z;
#pragma unroll
                    for (uint32_t s = 0; s < 8; s += 2) {
                        const v4i a2 = pack128(a[s], a[s + 1]);
                        cl = __builtin_amdgcn_mfma_i32_16x16x64_i8(a2, pack128(b[s], b[s + 1]), cl, 0, 0, 0);
                        ch = __builtin_amdgcn_mfma_i32_16x16x64_i8(a2, pack128(bh[s], bh[s + 1]), ch, 0, 0, 0);
                        cm = __builtin_amdgcn_mfma_i32_16x16x64_i8(a2, pack128(bm[s], bm[s + 1]), cm, 0, 0, 0);
                    }
#pragma unroll
                    for (uint32_t v = 0; v < 4; v++) {
                        isum[v] = 8 * ch[v] + cl[v];
                        const double dxd = (double)dx[v];
                        const double t1 = ((double)dw * dxd) * (double)isum[v];
                        const double t2 = ((double)dmin * dxd) * (double)cm[v];
                        acc[t][v] += t1 - t2;
                    }
                } else {
                    const bool lo_half = g < 2u;
#pragma unroll
                    for (uint32_t c = 0; c < 8; c++) {
                        const long b0 = lo_half ? b[c] : 0l, b1 = lo_half ? 0l : b[c];
                        const v4i c0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[c], b0, z, 0, 0, 0);
                        const v4i c1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[c], b1, z, 0, 0, 0);
                        // |scale| <= 128, |dot| <= 16 * 32 * 128: 24-bit products
#pragma unroll
                        for (uint32_t v = 0; v < 4; v++)
                            isum[v] += __mul24(scl[2 * c], c0[v]) + __mul24(scl[2 * c + 1], c1[v]);
                    }
#pragma unroll
                    for (uint32_t v = 0; v < 4; v++) acc[t][v] += ((double)dw * (double)dx[v]) * (double)isum[v];
                }
            }
        }
        if (i + 1u < nb) {
            cur = nxt;
            // buffer (i + 1) & 1 was last read for item i - 1, before the
            // barrier that ended that item
            if (stager) stage.st(xs[(i + 1u) & 1u]);
        }
        __syncthreads();
    }

    if (row < rows) {
#pragma unroll
        for (uint32_t t = 0; t < UB_TILES; t++)
#pragma unroll
            for (uint32_t v = 0; v < 4; v++) {
                const uint32_t tok = tok0 + t * UB_TOK + 4u * g + v;
                if (t < ntiles && tok < n_tok) {
                    // accumulate: the residual add of the single-token GEMV's
                    // RESID epilogue (y = y + result, one fp32 add)
                    float *yp = y + (size_t)tok * rows + row;
                    *yp = accumulate ? *yp + (float)acc[t][v] : (float)acc[t][v];
                }
            }
    }
}

// ggml quantize_row_q8_K_ref over a ubatch (the oracle's or_quant_q8_K):
// one wave per 256-element block, lane l holding elements 4l..4l+3.  The
// block's scale comes from its first element of largest |x| (sequentially:
// `if (|x| > amax)`, so a tie keeps the lower index -- the wave reduction
// breaks ties by index), iscale = -127 / that element, codes
// min(127, rint(iscale * x)) (ggml's nearest_int: round half to even), d =
// 1 / iscale, bsums the 16-element sums of the codes; an all-zero block is
// all zeros.  Inputs are finite.
__device__ __forceinline__ void quant_block_q8k(const float e[4], uint32_t lane, uint8_t *ob) {
    float amax = 0.0f, mx = 0.0f;
    uint32_t idx = 0xFFFFFFFFu;
#pragma unroll
    for (uint32_t j = 0; j < 4; j++) {
        const float ax = fabsf(e[j]);
        if (ax > amax) { amax = ax; mx = e[j]; idx = 4u * lane + j; }
    }
#pragma unroll
    for (uint32_t o = 1; o < 64; o <<= 1) {
        const float a2 = __shfl_xor(amax, o), m2 = __shfl_xor(mx, o);
        const uint32_t i2 = __shfl_xor(idx, o);
        if (a2 > amax || (a2 == amax && i2 < idx)) { amax = a2; mx = m2; idx = i2; }
    }
    int q[4] = {0, 0, 0, 0};
    float d = 0.0f;
    if (amax != 0.0f) {
        const float iscale = -127.f / mx;
#pragma unroll
        for (uint32_t j = 0; j < 4; j++) {
            const int t = (int)rintf(iscale * e[j]);
            q[j] = t < 127 ? t : 127;
        }
        d = 1.0f / iscale;
    }
    *(uint32_t *)(ob + 4u + 4u * lane) =
        (uint32_t)(q[0] & 0xFF) | ((uint32_t)(q[1] & 0xFF) << 8) | ((uint32_t)(q[2] & 0xFF) << 16) | ((uint32_t)q[3] << 24);
    int bs = q[0] + q[1] + q[2] + q[3];
    bs += __shfl_xor(bs, 1);
    bs += __shfl_xor(bs, 2);
    if ((lane & 3u) == 0) *(int16_t *)(ob + 260u + 2u * (lane >> 2)) = (int16_t)bs;
    if (lane == 0) *(float *)ob = d;
}

__global__ __launch_bounds__(64) void quant_q8k_kernel(const float *__restrict__ x, uint8_t *__restrict__ xq) {
    const uint32_t lane = threadIdx.x;
    const size_t blk = blockIdx.x;   // token * (k / 256) + block: x and xq in the same order
    const float4 v = ((const float4 *)(x + blk * 256u))[lane];
    const float e[4] = {v.x, v.y, v.z, v.w};
    quant_block_q8k(e, lane, xq + blk * Q8K_BYTES);
}

// SwiGLU then the Q8_K quantiser over a ubatch: f = silu(gate) * up (the
// single-token GEMV's SWIGLU epilogue and the oracle's or_ffn: silu(x) =
// x / (1 + (float)exp(-(double)x))), quantised for the down projection.
__global__ __launch_bounds__(64) void swiglu_quant_q8k_kernel(const float *__restrict__ gate,
                                                             const float *__restrict__ up, uint8_t *__restrict__ xq) {
    const uint32_t lane = threadIdx.x;
    const size_t blk = blockIdx.x;
    const float4 g = ((const float4 *)(gate + blk * 256u))[lane];
    const float4 u = ((const float4 *)(up + blk * 256u))[lane];
    const float e[4] = {dev_silu(g.x) * u.x, dev_silu(g.y) * u.y, dev_silu(g.z) * u.z, dev_silu(g.w) * u.w};
    quant_block_q8k(e, lane, xq + blk * Q8K_BYTES);
}

// Gated RMSNorm per head then the Q8_K quantiser over a ubatch (the input of
// a gated-DeltaNet layer's ssm_out): for each head of d elements (d a power
// of two, 4..256), y = ((x * scale) * w[i]) * silu(z) with scale = 1 /
// sqrtf(mean + eps) from the head's fp32 squares summed in fp64 -- the
// single-token GEMV's GATED prologue and the oracle's or_gated_rmsnorm.  One
// wave per 256-element block: the d / 4 lanes of a head reduce its sum by xor
// shuffles (a fixed tree; the mean divides by a power of two, exactly).
__global__ __launch_bounds__(64) void gated_norm_quant_q8k_kernel(const float *__restrict__ x,
                                                                 const float *__restrict__ z,
                                                                 const float *__restrict__ w, uint32_t log2d,
                                                                 float eps, uint8_t *__restrict__ xq) {
    const uint32_t lane = threadIdx.x;
    const size_t blk = blockIdx.x;
    const float4 v = ((const float4 *)(x + blk * 256u))[lane];
    const float4 g = ((const float4 *)(z + blk * 256u))[lane];
    const uint32_t d = 1u << log2d, i0 = (4u * lane) & (d - 1u);   // element of the head
    double sq = (double)(v.x * v.x);
    sq += (double)(v.y * v.y);
    sq += (double)(v.z * v.z);
    sq += (double)(v.w * v.w);
    for (uint32_t o = 1; o < d / 4u; o <<= 1) sq += __shfl_xor(sq, o);
    const double inv_d = 1.0 / (double)d;   // a power of two: exact
    const float scale = 1.0f / sqrtf((float)(sq * inv_d) + eps);
    const float e[4] = {((v.x * scale) * w[i0]) * dev_silu(g.x), ((v.y * scale) * w[i0 + 1]) * dev_silu(g.y),
                        ((v.z * scale) * w[i0 + 2]) * dev_silu(g.z), ((v.w * scale) * w[i0 + 3]) * dev_silu(g.w)};
    quant_block_q8k(e, lane, xq + blk * Q8K_BYTES);
}

// The causal conv + silu of a gated-DeltaNet layer's qkv rows over a ubatch
// (the single-token GEMV's CONV epilogue and the oracle's or_conv_silu, token
// after token): with input(tau) = x[tau][c] for tau >= 0 and the conv state
// st[c][nh + tau] for -nh <= tau < 0 (nh = dconv - 1, oldest first),
// y[t][c] = silu(sum_j input(t - nh + j) * w[c][j]), the sum in fp64 in tap
// order rounded once.  Outputs do not depend on each other, so a thread
// takes channel c over UB_CONV_TOK consecutive tokens (blockIdx.y), its
// window in registers; the state moves on in conv_state_kernel, launched
// after this one.
constexpr uint32_t UB_CONV_TOK = 8;
__global__ __launch_bounds__(256) void conv_silu_kernel(const float *__restrict__ x, const float *__restrict__ st,
                                                       const float *__restrict__ cw, float *__restrict__ y,
                                                       uint32_t channels, uint32_t dconv, uint32_t n_tok) {
    const uint32_t c = blockIdx.x * 256u + threadIdx.x;
    if (c >= channels) return;
    const uint32_t nh = dconv - 1u, t0 = blockIdx.y * UB_CONV_TOK, t1 = min(t0 + UB_CONV_TOK, n_tok);
    float win[UB_CONV_MAX];
    float wt[UB_CONV_MAX];
#pragma unroll
    for (uint32_t j = 0; j < UB_CONV_MAX; j++) {
        const int tau = (int)t0 - (int)nh + (int)j;
        win[j] = j >= nh ? 0.0f : tau >= 0 ? x[(size_t)tau * channels + c] : st[(size_t)c * nh + (uint32_t)(tau + (int)nh)];
        wt[j] = j < dconv ? cw[(size_t)c * dconv + j] : 0.0f;
    }
    for (uint32_t t = t0; t < t1; t++) {
        const float xn = x[(size_t)t * channels + c];
        double acc = 0.0;
#pragma unroll
        for (uint32_t j = 0; j < UB_CONV_MAX; j++)
            if (j < dconv) acc += (double)(j < nh ? win[j] : xn) * (double)wt[j];
        y[(size_t)t * channels + c] = dev_silu((float)acc);
#pragma unroll
        for (uint32_t j = 0; j + 1 < UB_CONV_MAX; j++)
            if (j < nh) win[j] = (j + 1 < nh) ? win[j + 1] : xn;
    }
}

// The conv state after the ubatch: st[c][j] = input(n_tok - nh + j), the last
// nh inputs (old state entries when the ubatch is shorter than nh).
__global__ __launch_bounds__(256) void conv_state_kernel(const float *__restrict__ x, float *__restrict__ st,
                                                        uint32_t channels, uint32_t dconv, uint32_t n_tok) {
    const uint32_t c = blockIdx.x * 256u + threadIdx.x;
    if (c >= channels) return;
    const uint32_t nh = dconv - 1u;
    float nv[UB_CONV_MAX];
#pragma unroll
    for (uint32_t j = 0; j < UB_CONV_MAX; j++) {
        const int tau = (int)n_tok - (int)nh + (int)j;
        nv[j] = j >= nh ? 0.0f : tau >= 0 ? x[(size_t)tau * channels + c] : st[(size_t)c * nh + (uint32_t)(tau + (int)nh)];
    }
#pragma unroll
    for (uint32_t j = 0; j < UB_CONV_MAX; j++)
        if (j < nh) st[(size_t)c * nh + j] = nv[j];
}

// RMSNorm then the Q8_K quantiser, one workgroup per token: the norm of the
// single-token GEMV's SINTER_PRO_RMSNORM prologue (gemv.h) and of the
// oracle's or_rmsnorm (ggml: fp32 squares summed in fp64, the mean rounded
// to fp32, scale = 1 / sqrtf(mean + eps), y = (x * scale) * w).  The fp64 sum
// is the prologue's tree exactly, so prefill and decode normalise a row to
// the same bits: row g = t / 16 (16 lanes) owns the 256-element chunks g,
// g + 16, ..., lane r = t % 16 elements 16r..16r+15 of each; the lane keeps
// four partial sums (element i into sum i / 4) over its chunks g + 32,
// g + 48, ... and then g and g + 16; the row adds them as
// (s0 + s1) + (s2 + s3) and by its DPP butterfly, the wave its four rows in
// order, the workgroup its four waves in order.  Then wave v quantises
// blocks v, v + 4, ... of the normalised row.
__device__ __forceinline__ void ub_add_sq(const float *xr, uint32_t c, uint32_t r, double s4[4]) {
#pragma unroll
    for (uint32_t q = 0; q < 4; q++) {
        const float4 v = ((const float4 *)(xr + 256u * c + 16u * r))[q];
        s4[q] += (double)(v.x * v.x);
        s4[q] += (double)(v.y * v.y);
        s4[q] += (double)(v.z * v.z);
        s4[q] += (double)(v.w * v.w);
    }
}
__global__ __launch_bounds__(256) void rmsnorm_quant_q8k_kernel(const float *__restrict__ x, const float *__restrict__ w,
                                                               float eps, uint32_t k, uint8_t *__restrict__ xq) {
    __shared__ double red[4];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wv = tid >> 6, r = tid & 15u, g = tid >> 4, nchunk = k / 256u;
    const float *xr = x + (size_t)blockIdx.x * k;
    double s4[4] = {0.0, 0.0, 0.0, 0.0};
    for (uint32_t c = g + 32u; c < nchunk; c += 16u) ub_add_sq(xr, c, r, s4);
    if (g < nchunk) ub_add_sq(xr, g, r, s4);
    if (g + 16u < nchunk) ub_add_sq(xr, g + 16u, r, s4);
    double s = row16_sum_f64((s4[0] + s4[1]) + (s4[2] + s4[3]));
    s = ((readlane_f64(s, 0) + readlane_f64(s, 16)) + readlane_f64(s, 32)) + readlane_f64(s, 48);
    if (lane == 0) red[wv] = s;
    __syncthreads();
    s = ((red[0] + red[1]) + red[2]) + red[3];
    const float mean = (float)(s / (double)k);
    const float scale = 1.0f / sqrtf(mean + eps);
    uint8_t *orow = xq + (size_t)blockIdx.x * (k / 256u) * Q8K_BYTES;
    for (uint32_t b = wv; b < k / 256u; b += 4u) {
        const float4 v = ((const float4 *)(xr + 256u * b))[lane];
        float e[4] = {v.x * scale, v.y * scale, v.z * scale, v.w * scale};
        if (w) {
            const float4 g = ((const float4 *)(w + 256u * b))[lane];
            e[0] = e[0] * g.x; e[1] = e[1] * g.y; e[2] = e[2] * g.z; e[3] = e[3] * g.w;
        }
        quant_block_q8k(e, lane, orow + (size_t)b * Q8K_BYTES);
    }
}

}  // namespace
}  // namespace sinter

using namespace sinter;

extern "C" int sinter_op_gemv_ubatch(int type, const void *w, int64_t rows, int64_t k, const void *xq,
                                     uint32_t n_tokens, float *y, int accumulate, void *stream) {
    if (type != SINTER_Q4_K && type != SINTER_Q6_K)
        return set_error(SINTER_ERR_ARG, "gemv_ubatch: weight type %d (Q4_K or Q6_K)", type);
    if (rows <= 0 || rows > (int64_t)UINT32_MAX - UB_ROWS || k <= 0 || k % 256 != 0 || k / 256 > (int64_t)UINT32_MAX)
        return set_error(SINTER_ERR_ARG, "gemv_ubatch: rows %lld / k %lld (k a positive multiple of 256)",
                         (long long)rows, (long long)k);
    if (n_tokens == 0) return SINTER_OK;
    if (!w || !xq || !y) return set_error(SINTER_ERR_ARG, "gemv_ubatch: null pointer");
    const uintptr_t wa = type == SINTER_Q4_K ? 16u : 4u;
    if ((uintptr_t)w % wa || (uintptr_t)xq % 4u || (uintptr_t)y % 4u)
        return set_error(SINTER_ERR_ARG, "gemv_ubatch: alignment (weights %u B, activations and output 4 B)",
                         (unsigned)wa);
    const uint64_t n_rt = ((uint64_t)rows + UB_WG_ROWS - 1) / UB_WG_ROWS;
    // token tiles per workgroup: 4 (weights read once per 64 tokens) unless
    // that leaves fewer than UB_MIN_WGS workgroups; then fewer, the row
    // tile's token groups running side by side so its weights come from the
    // memory-side cache after the first
    uint32_t tpw = UB_TILES;
    while (tpw > 1 && n_rt * (((uint64_t)n_tokens + UB_TOK * tpw - 1) / (UB_TOK * tpw)) < UB_MIN_WGS) tpw /= 2;
    const uint64_t n_tg = ((uint64_t)n_tokens + UB_TOK * tpw - 1) / (UB_TOK * tpw);
    if (n_rt * n_tg > (uint64_t)INT32_MAX) return set_error(SINTER_ERR_ARG, "gemv_ubatch: grid too large");
    const uint32_t nb = (uint32_t)(k / 256);
    const dim3 grid((uint32_t)(n_rt * n_tg)), block(UB_THREADS);
    hipStream_t s = (hipStream_t)stream;
    if (type == SINTER_Q4_K)
        hipLaunchKernelGGL(ubatch_gemv_kernel<SINTER_Q4_K>, grid, block, 0, s, (const uint8_t *)w, (uint32_t)rows, nb,
                           (const uint8_t *)xq, n_tokens, y, (uint32_t)n_tg, tpw,
                           (uint32_t)(accumulate != 0));
    else
        hipLaunchKernelGGL(ubatch_gemv_kernel<SINTER_Q6_K>, grid, block, 0, s, (const uint8_t *)w, (uint32_t)rows, nb,
                           (const uint8_t *)xq, n_tokens, y, (uint32_t)n_tg, tpw,
                           (uint32_t)(accumulate != 0));
    return hip_ok(hipGetLastError(), "gemv_ubatch: launch") ? SINTER_OK : SINTER_ERR_HIP;
}

extern "C" int sinter_quant_q8k_ubatch(const float *x, int64_t k, uint32_t n_tokens, void *xq, void *stream) {
    if (k <= 0 || k % 256 != 0) return set_error(SINTER_ERR_ARG, "quant_q8k_ubatch: k %lld (a positive multiple of 256)",
                                                 (long long)k);
    if (n_tokens == 0) return SINTER_OK;
    if (!x || !xq) return set_error(SINTER_ERR_ARG, "quant_q8k_ubatch: null pointer");
    if ((uintptr_t)x % 16u || (uintptr_t)xq % 4u)
        return set_error(SINTER_ERR_ARG, "quant_q8k_ubatch: alignment (x 16 bytes, xq 4 bytes)");
    const uint64_t n_blk = (uint64_t)n_tokens * (uint64_t)(k / 256);
    if (n_blk > (uint64_t)INT32_MAX) return set_error(SINTER_ERR_ARG, "quant_q8k_ubatch: too many blocks");
    hipLaunchKernelGGL(quant_q8k_kernel, dim3((uint32_t)n_blk), dim3(64), 0, (hipStream_t)stream, x, (uint8_t *)xq);
    return hip_ok(hipGetLastError(), "quant_q8k_ubatch: launch") ? SINTER_OK : SINTER_ERR_HIP;
}

extern "C" int sinter_rmsnorm_quant_q8k_ubatch(const float *x, const float *w, float eps, int64_t k, uint32_t n_tokens,
                                               void *xq, void *stream) {
    if (k <= 0 || k % 256 != 0 || k > (int64_t)UINT32_MAX)
        return set_error(SINTER_ERR_ARG, "rmsnorm_quant_q8k_ubatch: k %lld (a positive multiple of 256)", (long long)k);
    if (n_tokens == 0) return SINTER_OK;
    if (!x || !xq) return set_error(SINTER_ERR_ARG, "rmsnorm_quant_q8k_ubatch: null pointer");
    if ((uintptr_t)x % 16u || (uintptr_t)w % 16u || (uintptr_t)xq % 4u)
        return set_error(SINTER_ERR_ARG, "rmsnorm_quant_q8k_ubatch: alignment (x, w 16 bytes, xq 4 bytes)");
    if (!(eps >= 0.0f)) return set_error(SINTER_ERR_ARG, "rmsnorm_quant_q8k_ubatch: eps must be >= 0");
    hipLaunchKernelGGL(rmsnorm_quant_q8k_kernel, dim3(n_tokens), dim3(256), 0, (hipStream_t)stream, x, w, eps,
                       (uint32_t)k, (uint8_t *)xq);
    return hip_ok(hipGetLastError(), "rmsnorm_quant_q8k_ubatch: launch") ? SINTER_OK : SINTER_ERR_HIP;
}

extern "C" int sinter_swiglu_quant_q8k_ubatch(const float *gate, const float *up, int64_t k, uint32_t n_tokens, void *xq,
                                              void *stream) {
    if (k <= 0 || k % 256 != 0)
        return set_error(SINTER_ERR_ARG, "swiglu_quant_q8k_ubatch: k %lld (a positive multiple of 256)", (long long)k);
    if (n_tokens == 0) return SINTER_OK;
    if (!gate || !up || !xq) return set_error(SINTER_ERR_ARG, "swiglu_quant_q8k_ubatch: null pointer");
    if ((uintptr_t)gate % 16u || (uintptr_t)up % 16u || (uintptr_t)xq % 4u)
        return set_error(SINTER_ERR_ARG, "swiglu_quant_q8k_ubatch: alignment (gate, up 16 bytes, xq 4 bytes)");
    const uint64_t n_blk = (uint64_t)n_tokens * (uint64_t)(k / 256);
    if (n_blk > (uint64_t)INT32_MAX) return set_error(SINTER_ERR_ARG, "swiglu_quant_q8k_ubatch: too many blocks");
    hipLaunchKernelGGL(swiglu_quant_q8k_kernel, dim3((uint32_t)n_blk), dim3(64), 0, (hipStream_t)stream, gate, up,
                       (uint8_t *)xq);
    return hip_ok(hipGetLastError(), "swiglu_quant_q8k_ubatch: launch") ? SINTER_OK : SINTER_ERR_HIP;
}

extern "C" int sinter_gated_rmsnorm_quant_q8k_ubatch(const float *x, const float *z, const float *w, uint32_t head_dim,
                                                     float eps, int64_t k, uint32_t n_tokens, void *xq, void *stream) {
    if (k <= 0 || k % 256 != 0)
        return set_error(SINTER_ERR_ARG, "gated_rmsnorm_quant_q8k_ubatch: k %lld (a positive multiple of 256)",
                         (long long)k);
    if (head_dim < 4 || head_dim > 256 || (head_dim & (head_dim - 1)))
        return set_error(SINTER_ERR_ARG, "gated_rmsnorm_quant_q8k_ubatch: head_dim %u (a power of two, 4..256)",
                         head_dim);
    if (n_tokens == 0) return SINTER_OK;
    if (!x || !z || !w || !xq) return set_error(SINTER_ERR_ARG, "gated_rmsnorm_quant_q8k_ubatch: null pointer");
    if ((uintptr_t)x % 16u || (uintptr_t)z % 16u || (uintptr_t)w % 4u || (uintptr_t)xq % 4u)
        return set_error(SINTER_ERR_ARG, "gated_rmsnorm_quant_q8k_ubatch: alignment (x, z 16 bytes, w, xq 4 bytes)");
    if (!(eps >= 0.0f)) return set_error(SINTER_ERR_ARG, "gated_rmsnorm_quant_q8k_ubatch: eps must be >= 0");
    const uint64_t n_blk = (uint64_t)n_tokens * (uint64_t)(k / 256);
    if (n_blk > (uint64_t)INT32_MAX) return set_error(SINTER_ERR_ARG, "gated_rmsnorm_quant_q8k_ubatch: too many blocks");
    hipLaunchKernelGGL(gated_norm_quant_q8k_kernel, dim3((uint32_t)n_blk), dim3(64), 0, (hipStream_t)stream, x, z, w,
                       (uint32_t)__builtin_ctz(head_dim), eps, (uint8_t *)xq);
    return hip_ok(hipGetLastError(), "gated_rmsnorm_quant_q8k_ubatch: launch") ? SINTER_OK : SINTER_ERR_HIP;
}

extern "C" int sinter_conv_silu_ubatch(const float *x, float *state, const float *conv_w, float *y, int64_t channels,
                                       uint32_t dconv, uint32_t n_tokens, void *stream) {
    if (channels <= 0 || channels > (int64_t)INT32_MAX || dconv < 1 || dconv > UB_CONV_MAX)
        return set_error(SINTER_ERR_ARG, "conv_silu_ubatch: channels %lld / dconv %u (1..%u)", (long long)channels,
                         dconv, UB_CONV_MAX);
    if (n_tokens == 0) return SINTER_OK;
    if (!x || !conv_w || !y || (dconv > 1 && !state)) return set_error(SINTER_ERR_ARG, "conv_silu_ubatch: null pointer");
    if ((uintptr_t)x % 4u || (uintptr_t)state % 4u || (uintptr_t)conv_w % 4u || (uintptr_t)y % 4u)
        return set_error(SINTER_ERR_ARG, "conv_silu_ubatch: alignment (4 bytes)");
    const uint32_t nblk = (uint32_t)((channels + 255) / 256);
    hipLaunchKernelGGL(conv_silu_kernel, dim3(nblk, (n_tokens + UB_CONV_TOK - 1) / UB_CONV_TOK), dim3(256), 0,
                       (hipStream_t)stream, x, state, conv_w, y, (uint32_t)channels, dconv, n_tokens);
    if (dconv > 1)
        hipLaunchKernelGGL(conv_state_kernel, dim3(nblk), dim3(256), 0, (hipStream_t)stream, x, state,
                           (uint32_t)channels, dconv, n_tokens);
    return hip_ok(hipGetLastError(), "conv_silu_ubatch: launch") ? SINTER_OK : SINTER_ERR_HIP;
}
