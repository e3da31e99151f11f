// The batched prefill's own kernels (sinter_model_prefill runs a prompt layer
// by layer over ubatches of tokens; docs/PREFILL-SEMANTICS.md:379-426 of the
// reference calls this the "(b)" stage: each layer once per ubatch, the
// recurrence looping over the ubatch's tokens inside one launch).  The trunk
// GEMMs, norms, quantisers, SwiGLU and the conv come from ubatch.hip; here:
//   embed_ubatch_kernel      token rows of the embedding, dequantised
//   gdn_prep_ubatch_kernel   the l2 norms of q and k and the gates of every
//                            token of the ubatch
//   gdn_scan_ubatch_kernel   the delta rule over the ubatch, token after
//                            token, the state slice in registers
//   attn_prep_ubatch_kernel  q/k RMSNorm + NEOX RoPE per token and head, the
//                            ubatch's K/V rows appended to the cache
//   attn_prefill_kernel      causal attention of the ubatch's queries over
//                            the cache, gated by sigmoid(gate)
// The first three compute what the decode ops compute, expression for
// expression (same helpers, same fp64 folds), so a prefilled state and KV
// cache are bit-identical to the decode program's.  The attention of a
// prefill query is the decode's declared fp32 fold over one chunk holding all
// its positions (the decode splits long contexts over chunks); the oracle's
// or_attn_prefill restates it.
#include "internal.h"
#include "gemv.h"
#include "attn.h"

namespace sinter {
namespace {

// ------------------------------------------------------------------ embedding

// x[t] = dequant(embd[tokens[t]]) (the decode's SINTER_PRO_EMBED rows, ggml's
// dequantize_row_*); blockIdx.y is the token
__global__ __launch_bounds__(256) void embed_ubatch_kernel(const char *__restrict__ embd, int type, uint32_t E,
                                                          uint64_t row_bytes, const int32_t *__restrict__ tokens,
                                                          float *__restrict__ x) {
    const uint32_t t = blockIdx.y;
    const char *row = embd + (size_t)tokens[t] * row_bytes;
    for (uint32_t i = blockIdx.x * 256u + threadIdx.x; i < E / 4u; i += gridDim.x * 256u) {
        float v[4];
        dequant4(row, type, 4u * i, v);
        reinterpret_cast<float4 *>(x + (size_t)t * E)[i] = make_float4(v[0], v[1], v[2], v[3]);
    }
}

// ------------------------------------------------------------------ GDN step over a ubatch

struct GdnUb {
    const float *qkv;     // [T][C] conv outputs: q[HK*D] | k[HK*D] | v[HV*D]
    const float *alpha;   // [T][HV]
    const float *beta;    // [T][HV]
    const float *dt_bias, *ssm_a;
    float *qn, *kn;       // [T][HK][D] l2-normalised q and k
    float *gate, *bgate;  // [T][HV] decay g and beta
    float *state;         // [HV][D][D] (column-major per head), updated in place
    float *o;             // [T][HV*D]
    uint32_t hk, hv, d, cols, n_tok, c_stride;
    float eps, scale;
};

// The per-token inputs of the recurrence, for every token at once: the l2
// norms of q and k head hk (blockIdx.y) of token blockIdx.x -- the decode
// op_gdn_step's block_sum2_f64 over the same 256-thread layout, scale
// 1/fmaxf(sqrtf(sum), eps) -- and, in the hk = 0 workgroup, the token's gates
// g = exp(softplus(alpha + dt_bias) * a) and beta = sigmoid(beta_raw).
__global__ __launch_bounds__(256) void gdn_prep_ubatch_kernel(GdnUb a) {
    __shared__ double red[16];
    const uint32_t t = blockIdx.x, hk = blockIdx.y, D = a.d, HK = a.hk;
    const float *qkv = a.qkv + (size_t)t * a.c_stride;
    const uint32_t tq = threadIdx.x & (D - 1);
    const float qv = qkv[(size_t)hk * D + tq], kv = qkv[(size_t)HK * D + (size_t)hk * D + tq];
    const bool mine = threadIdx.x < D;
    double sq = mine ? (double)(qv * qv) : 0.0, sk = mine ? (double)(kv * kv) : 0.0;
    block_sum2_f64(sq, sk, red);
    if (mine) {
        const size_t o = ((size_t)t * HK + hk) * D + threadIdx.x;
        a.qn[o] = qv * (1.0f / fmaxf(sqrtf((float)sq), a.eps));
        a.kn[o] = kv * (1.0f / fmaxf(sqrtf((float)sk), a.eps));
    }
    if (hk == 0) {
        for (uint32_t h = threadIdx.x; h < a.hv; h += 256u) {
            const float alpha = a.alpha[(size_t)t * a.hv + h], braw = a.beta[(size_t)t * a.hv + h];
            const float sp = dev_softplus(alpha + a.dt_bias[h]);
            a.gate[(size_t)t * a.hv + h] = (float)exp((double)(sp * a.ssm_a[h]));
            a.bgate[(size_t)t * a.hv + h] = dev_sigmoid(braw);
        }
    }
}

// The delta rule over the ubatch: one (v-head, slice of `cols` state
// columns) item per workgroup, the decode op_gdn_step's item (gdn.h) with its
// thread layout and folds -- kv and o as sequential fp32 sums over the
// thread's RPT rows then lanes_sum_f32 over the column's threads, delta and
// the update in the same fp32 expressions.  The state slice stays in registers from the first
// token to the last.  The per-token inputs (precomputed by
// gdn_prep_ubatch_kernel) move through LDS in stages of GDN_STAGE tokens,
// double-buffered: stage s + 1 is loaded into registers while stage s is
// computed, so a token waits on no memory and the workgroup meets at one
// barrier per stage.
constexpr uint32_t GDN_STAGE = 16;
template <uint32_t RPT>
__global__ __launch_bounds__(256) void gdn_scan_ubatch_kernel(GdnUb a) {
    // per buffer: k | q [GDN_STAGE][2][D], v [GDN_STAGE][cols], g [GDN_STAGE], beta [GDN_STAGE]
    constexpr uint32_t BUF = GDN_STAGE * (2 * 256 + 32 + 2);
    __shared__ __attribute__((aligned(16))) float lds[2 * BUF];
    const uint32_t D = a.d, HK = a.hk, HV = a.hv, cols = a.cols, tpc = 256u / cols;
    const uint32_t slices = D / cols, item = blockIdx.x, tid = threadIdx.x;
    const uint32_t h = item / slices, c0 = (item % slices) * cols, hk = h % HK;
    const uint32_t col = c0 + tid / tpc, i0 = (tid % tpc) * RPT;
    const uint32_t kq_f = GDN_STAGE * 2 * D, v_off = kq_f, g_off = v_off + GDN_STAGE * cols, b_off = g_off + GDN_STAGE;
    float *srow = a.state + ((size_t)h * D + col) * D + i0;
    float s[RPT];
#pragma unroll
    for (uint32_t r = 0; r < RPT; r += 4) {
        const f32x4 t = *reinterpret_cast<const f32x4 *>(srow + r);
        s[r] = t.x; s[r + 1] = t.y; s[r + 2] = t.z; s[r + 3] = t.w;
    }
    // stage loads into registers: thread tid takes float4 j = tid + 256 i of
    // the k|q block (token j / (D / 2), half (j / (D / 4)) % 2, element
    // 4 (j % (D / 4))); threads below GDN_STAGE cols / 4 one float4 of v;
    // threads 128 .. 128 + 2 GDN_STAGE one g or beta
    constexpr uint32_t KQ4 = GDN_STAGE * 2 * 256 / 4 / 256;   // float4 per thread at D = 256
    const uint32_t n_kq4 = kq_f / 4, n_v4 = GDN_STAGE * cols / 4;
    f32x4 rkq[KQ4];
    f32x4 rv = {0.0f, 0.0f, 0.0f, 0.0f};
    float rg = 0.0f;
    const uint32_t nst = (a.n_tok + GDN_STAGE - 1) / GDN_STAGE;
    auto issue = [&](uint32_t st) {
        const uint32_t tb = st * GDN_STAGE;
#pragma unroll
        for (uint32_t i = 0; i < KQ4; i++) {
            const uint32_t j = tid + 256u * i;
            if (j < n_kq4) {
                const uint32_t tk = j / (D / 2), half = (j / (D / 4)) & 1u, e = 4u * (j % (D / 4));
                const uint32_t t = min(tb + tk, a.n_tok - 1);
                const float *src = (half ? a.qn : a.kn) + ((size_t)t * HK + hk) * D + e;
                rkq[i] = *reinterpret_cast<const f32x4 *>(src);
            }
        }
        if (tid < n_v4) {
            const uint32_t tk = tid / (cols / 4), e = 4u * (tid % (cols / 4));
            const uint32_t t = min(tb + tk, a.n_tok - 1);
            rv = *reinterpret_cast<const f32x4 *>(a.qkv + (size_t)t * a.c_stride + (size_t)2 * HK * D +
                                                  (size_t)h * D + c0 + e);
        }
        if (tid >= 128 && tid < 128 + 2 * GDN_STAGE) {
            const uint32_t tk = (tid - 128) % GDN_STAGE, t = min(tb + tk, a.n_tok - 1);
            rg = tid < 128 + GDN_STAGE ? a.gate[(size_t)t * HV + h] : a.bgate[(size_t)t * HV + h];
        }
    };
    auto park = [&](uint32_t st) {
        float *L = lds + (st & 1u) * BUF;
#pragma unroll
        for (uint32_t i = 0; i < KQ4; i++) {
            const uint32_t j = tid + 256u * i;
            if (j < n_kq4) *reinterpret_cast<f32x4 *>(L + 4 * j) = rkq[i];
        }
        if (tid < n_v4) *reinterpret_cast<f32x4 *>(L + v_off + 4 * tid) = rv;
        if (tid >= 128 && tid < 128 + 2 * GDN_STAGE) L[g_off + (tid - 128)] = rg;
    };
    issue(0);
    park(0);
    if (nst > 1) issue(1);
    __syncthreads();
    // Token t's o sum and token t + 1's kv sum take the same updated state
    // and run in one loop, two independent chains; the kv sum of a stage's
    // first token runs alone after the stage barrier.
    auto load8 = [&](const float *p, float (&d)[RPT]) {
#pragma unroll
        for (uint32_t r = 0; r < RPT; r += 4) {
            const f32x4 v = *reinterpret_cast<const f32x4 *>(p + r);
            d[r] = v.x; d[r + 1] = v.y; d[r + 2] = v.z; d[r + 3] = v.w;
        }
    };
    for (uint32_t st = 0; st < nst; st++) {
        const float *L = lds + (st & 1u) * BUF;
        const uint32_t tb = st * GDN_STAGE, te = min(GDN_STAGE, a.n_tok - tb);
        float kk[RPT], qq[RPT], kn[RPT];
        load8(L + i0, kk);
        float dkv = 0.0f;
#pragma unroll
        for (uint32_t r = 0; r < RPT; r++) {
            const float pr = s[r] * kk[r];
            dkv = dkv + pr;
        }
        dkv = lanes_sum_f32(dkv, tpc);
        for (uint32_t tk = 0; tk < te; tk++) {
            const uint32_t tn = tk + 1 < te ? tk + 1 : tk;   // (the last token's "next" sum is dropped)
            load8(L + tk * 2 * D + D + i0, qq);
            load8(L + tn * 2 * D + i0, kn);
            const float vcol = L[v_off + tk * cols + (col - c0)];
            const float g = L[g_off + tk], beta = L[b_off + tk];
            const float kvf = dkv;
            const float t1 = g * kvf;
            const float t2 = vcol - t1;
            const float delta = t2 * beta;
            float dout = 0.0f, dkn = 0.0f;
#pragma unroll
            for (uint32_t r = 0; r < RPT; r++) {
                const float u1 = g * s[r];
                const float u2 = kk[r] * delta;
                s[r] = u1 + u2;
                const float po = s[r] * qq[r], pn = s[r] * kn[r];
                dout = dout + po;
                dkn = dkn + pn;
            }
            dout = lanes_sum_f32(dout, tpc);
            dkv = lanes_sum_f32(dkn, tpc);
            if ((tid % tpc) == 0) a.o[(size_t)(tb + tk) * HV * D + (size_t)h * D + col] = dout * a.scale;
#pragma unroll
            for (uint32_t r = 0; r < RPT; r++) kk[r] = kn[r];
        }
        if (st + 1 < nst) {
            park(st + 1);   // (its buffer was last read in stage st - 1, before the last barrier)
            if (st + 2 < nst) issue(st + 2);
        }
        __syncthreads();
    }
#pragma unroll
    for (uint32_t r = 0; r < RPT; r += 4) {
        const f32x4 v = {s[r], s[r + 1], s[r + 2], s[r + 3]};
        *reinterpret_cast<f32x4 *>(srow + r) = v;
    }
}

// ------------------------------------------------------------------ attention prep

struct AttnPrepUb {
    const float *qg;      // [T][NQ][2*HD]: q | gate
    const float *k, *v;   // [T][NKV*HD]
    const float *q_norm, *k_norm;
    void *kc, *vc;        // the cache: rows [n_ctx][NKV heads], f16 or Q8_0
    float *qr;            // [T][NQ][HD] normalised, rotated q
    int32_t pos0;
    uint32_t n_tok, nq, nkv, hd, rope_dims, kv_type;
    float theta_scale, eps;
};

// One wave per (token, head): heads j < NQ are the token's q heads (into qr),
// heads NQ + g its k head g, appended (with v head g, raw) at row pos0 + t.
// The decode's att_prep arithmetic: lane l holds elements 4l..4l+3; the sum
// of squares is the lane's four fp32 squares added in fp64 in order, then
// wave_sum_f64; y = (x * (1/sqrtf(mean + eps))) * w; rope pair (i, i + half)
// turns by theta_i = pos * theta_scale^i (repeated fp32 products), cos and
// sin evaluated in fp64 and rounded; the cache gets f16 (round to nearest
// even) or ggml's reference Q8_0 blocks (amax / 127, codes roundf(x * 1/d)).
__global__ __launch_bounds__(256) void attn_prep_ubatch_kernel(AttnPrepUb a) {
    const uint32_t t = blockIdx.x, lane = threadIdx.x & 63u;
    const uint32_t j = blockIdx.y * 4u + (threadIdx.x >> 6);
    if (j >= a.nq + a.nkv) return;   // (wave-uniform)
    const int pos = a.pos0 + (int)t;
    const uint32_t HD = a.hd, RW = a.nkv * HD, e0 = 4 * lane;
    const bool isq = j < a.nq;
    const uint32_t g = isq ? 0u : j - a.nq;
    const float *src = isq ? a.qg + ((size_t)t * a.nq + j) * 2 * HD : a.k + (size_t)t * RW + (size_t)g * HD;
    const float4 x = reinterpret_cast<const float4 *>(src)[lane];
    const float4 wt = reinterpret_cast<const float4 *>(isq ? a.q_norm : a.k_norm)[lane];
    double ss = (double)(x.x * x.x);
    ss += (double)(x.y * x.y);
    ss += (double)(x.z * x.z);
    ss += (double)(x.w * x.w);
    ss = wave_sum_f64(ss);
    const float hs = 1.0f / sqrtf((float)(ss / 256.0) + a.eps);
    const float xv[4] = {x.x, x.y, x.z, x.w}, wv[4] = {wt.x, wt.y, wt.z, wt.w};
    float y[4], o[4];
#pragma unroll
    for (uint32_t c = 0; c < 4; c++) {
        const float nrm = xv[c] * hs;
        y[c] = nrm * wv[c];
    }
    const uint32_t half = a.rope_dims / 2, pl = half / 4, partner = lane < pl ? lane + pl : lane - pl;
#pragma unroll
    for (uint32_t c = 0; c < 4; c++) o[c] = __shfl(y[c], (int)partner, 64);
#pragma unroll
    for (uint32_t c = 0; c < 4; c++) {
        const uint32_t i = e0 + c;
        if (i < 2 * half) {
            const uint32_t ri = i < half ? i : i - half;
            float th = (float)pos;
            for (uint32_t k = 0; k < ri; k++) th *= a.theta_scale;
            const float cs = (float)cos((double)th), sn = (float)sin((double)th);
            if (i < half) {
                const float a0 = y[c] * cs, a1 = o[c] * sn;
                y[c] = a0 - a1;
            } else {
                const float b0 = o[c] * sn, b1 = y[c] * cs;
                y[c] = b0 + b1;
            }
        }
    }
    if (isq) {
        reinterpret_cast<float4 *>(a.qr + ((size_t)t * a.nq + j) * HD)[lane] = make_float4(y[0], y[1], y[2], y[3]);
        return;
    }
    const float4 vr4 = reinterpret_cast<const float4 *>(a.v + (size_t)t * RW + (size_t)g * HD)[lane];
    const float vv[4] = {vr4.x, vr4.y, vr4.z, vr4.w};
    if (a.kv_type != SINTER_Q8_0) {
        uint16_t *kr = static_cast<uint16_t *>(a.kc) + (size_t)pos * RW + (size_t)g * HD + e0;
        uint16_t *vrow = static_cast<uint16_t *>(a.vc) + (size_t)pos * RW + (size_t)g * HD + e0;
#pragma unroll
        for (uint32_t c = 0; c < 4; c++) {
            kr[c] = f2h(y[c]);
            vrow[c] = f2h(vv[c]);
        }
        return;
    }
    // Q8_0: block b = lane / 8 of the head row holds the lane's 4 elements
    const size_t row_bytes = (size_t)a.nkv * ATT_Q8_HEAD;
    auto q8 = [&](const float val[4], unsigned char *row) {
        float am = fmaxf(fmaxf(fabsf(val[0]), fabsf(val[1])), fmaxf(fabsf(val[2]), fabsf(val[3])));
#pragma unroll
        for (int off = 1; off < 8; off <<= 1) am = fmaxf(am, __shfl_xor(am, off, 64));
        const float d = am / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        unsigned char *blk = row + (lane >> 3) * 34u;
#pragma unroll
        for (uint32_t c = 0; c < 4; c++) blk[2 + 4 * (lane & 7u) + c] = (unsigned char)(int8_t)roundf(val[c] * id);
        if ((lane & 7u) == 0) {
            const uint16_t dh = f2h(d);
            blk[0] = (unsigned char)(dh & 0xff);
            blk[1] = (unsigned char)(dh >> 8);
        }
    };
    q8(y, static_cast<unsigned char *>(a.kc) + (size_t)pos * row_bytes + (size_t)g * ATT_Q8_HEAD);
    q8(vv, static_cast<unsigned char *>(a.vc) + (size_t)pos * row_bytes + (size_t)g * ATT_Q8_HEAD);
}

// ------------------------------------------------------------------ causal attention of the ubatch

struct AttnPrefill {
    const float *qr;      // [T][NQ][HD]
    const float *qg;      // [T][NQ][2*HD] (the gate halves)
    const void *kc, *vc;
    float *part;          // [T][NQ][C][att_rec(HD)] chunk partials: O[HD], M, L
    float *out;           // [T][NQ*HD] gated attention output
    int32_t pos0;
    uint32_t n_tok, nq, nkv, hd, kv_type, n_chunks, chunk_min;
    float scale;
};

constexpr uint32_t PF_SLOTS = 8;   // queries per work item
// K/V tile buffers of the prefill attention: with PF_NBUF = 2 (tile j + 1
// loads while tile j is computed) the workgroup's LDS fits two workgroups
// per CU; 3 keeps two tiles in flight as the decode does.
#ifndef PF_NBUF
#define PF_NBUF 2
#endif
constexpr uint32_t PF_Q8_KC = 2 * PF_NBUF * ATT_Q8_RAWB, PF_Q8_VC = PF_Q8_KC + 32 * 256;
constexpr uint32_t PF_Q8_KS = PF_Q8_VC + 32 * 256, PF_Q8_VS = PF_Q8_KS + 32 * 8 * 4;
constexpr uint32_t PF_TILES = PF_NBUF * ATT_F16_BUF > 8u * PF_SLOTS * 256u * 4u ? PF_NBUF * ATT_F16_BUF
                                                                               : 8u * PF_SLOTS * 256u * 4u;
static_assert(PF_Q8_VS + 32 * 8 * 4 <= PF_TILES, "Q8_0 tiles fit the tile region");

// Work item = (kv head g, split chunk c, q head hh of g's group, block of 8
// consecutive queries), the block index running over the query blocks
// first, so the items that read one chunk of one kv head run side by side.  Query i of the ubatch (position pos0 + i) is split
// exactly as the decode splits it at that position: att_geom(pos0 + i + 1,
// C, chunk_min) chunks of tpc tiles, chunk c holding rows [c tpc 32,
// min((c + 1) tpc 32, pos0 + i + 1)).  The item runs the decode attention's
// tile loop (attn.h) over the union of its queries' chunk-c rows with the
// register slots holding 8 queries of one head instead of the 8 heads of one
// query, so every K/V tile is read once for 8 queries; a row outside a
// query's own range is masked out of its scores and enters its V sums as
// fmaf(0, v, acc) (no change but the sign of a zero sum, which the Q8_K
// quantisation of the attention output erases).  Per query the chunk partial
// -- the 8 row groups merged, O, M, L -- is the decode's, bit for bit.
template <bool Q8>
__global__ __launch_bounds__(256) void attn_prefill_split_kernel(AttnPrefill a, uint32_t cmax) {
    __shared__ __attribute__((aligned(16))) unsigned char tiles[PF_TILES];
    __shared__ __attribute__((aligned(16))) float wl[8 * (4 * PF_SLOTS + PF_SLOTS)];
    __shared__ __attribute__((aligned(16))) float gm[2 * 8 * PF_SLOTS];
    const uint32_t t = threadIdx.x, HD = a.hd, NQ = a.nq, NKV = a.nkv, gqa = NQ / NKV, C = a.n_chunks;
    const uint32_t n_qb = (a.n_tok + PF_SLOTS - 1) / PF_SLOTS;
    uint32_t it = blockIdx.x;
    const uint32_t qb = it % n_qb; it /= n_qb;
    const uint32_t hh = it % gqa; it /= gqa;
    const uint32_t c = it % cmax, g = it / cmax;
    const uint32_t head = g * gqa + hh, q0 = qb * PF_SLOTS, nqs = min(PF_SLOTS, a.n_tok - q0);
    // query s's chunk-c rows [k0, k1) (empty when its split has fewer chunks)
    auto range = [&](uint32_t s, uint32_t &k0, uint32_t &k1) {
        const uint32_t n_kv = (uint32_t)a.pos0 + q0 + s + 1u;
        const AttGeom geo = att_geom(n_kv, C, a.chunk_min);
        k0 = k1 = 0;
        if (s < nqs && c < geo.n) {
            k0 = c * geo.tpc * ATT_TILE;
            k1 = min(k0 + geo.tpc * ATT_TILE, n_kv);
        }
    };
    uint32_t U0 = 0xffffffffu, U1 = 0;
    for (uint32_t s = 0; s < nqs; s++) {
        uint32_t k0, k1;
        range(s, k0, k1);
        if (k1 > k0) {
            U0 = min(U0, k0);
            U1 = max(U1, k1);
        }
    }
    if (U1 == 0) return;   // (uniform) no query of the block has a chunk c
    const uint32_t ntile = (U1 - U0 + ATT_TILE - 1) / ATT_TILE;
    const uint32_t HB = Q8 ? ATT_Q8_HEAD : HD * 2u, RWB = NKV * HB;
    const uint32_t w = __builtin_amdgcn_readfirstlane(t >> 6), lane = t & 63u;
    LDS unsigned char *Lu = (LDS unsigned char *)tiles;
    const uint32_t kbase = (uint32_t)(uintptr_t)Lu;
    // tile j (rows U0 + 32 j ..) into buffer j % PF_NBUF, as the decode's
    // issue_tile; rows past U1 re-read row U1 - 1
    auto issue_tile = [&](uint32_t j) {
        const uint32_t t0 = U0 + j * ATT_TILE;
        if constexpr (!Q8) {
            const uint32_t bo = (j % PF_NBUF) * ATT_F16_BUF;
#pragma unroll
            for (uint32_t kk = 0; kk < 4; kk++) {
                const uint32_t k = w + 4 * kk, row = min(t0 + 2 * k + (lane >> 5), U1 - 1);
                const uint32_t voff = row * RWB + g * HB + (lane & 31) * 16;
                lds_dma16<false>((uintptr_t)a.kc, voff, kbase + bo + k * 1024);
                lds_dma16<false>((uintptr_t)a.vc, voff, kbase + bo + ATT_TILE * 512 + k * 1024);
            }
        } else {
            const uint32_t rb = (j % PF_NBUF) * 2 * ATT_Q8_RAWB;
#pragma unroll
            for (uint32_t kk = 0; kk < 3; kk++) {
                const uint32_t c0 = 136u * w + 64u * kk, ci = c0 + lane;
                const uint32_t row = min(t0 + ci / 17u, U1 - 1), voff = row * RWB + g * HB + (ci % 17u) * 16u;
                lds_dma16<false>((uintptr_t)a.kc, voff, kbase + rb + c0 * 16u);
                lds_dma16<false>((uintptr_t)a.vc, voff, kbase + rb + ATT_Q8_RAWB + c0 * 16u);
            }
        }
    };
    issue_tile(0);
    if (PF_NBUF > 2 && ntile > 1) issue_tile(1);
    const uint32_t rr = t >> 5, p = t & 31, mp = att_perm(p);
    // register slot s holds query q0 + (s ^ (mp & 7)) of head `head` (zero past the ubatch)
    float qv[PF_SLOTS][8], acc[PF_SLOTS][8];
#pragma unroll
    for (uint32_t s = 0; s < PF_SLOTS; s++) {
        const uint32_t qi = s ^ (mp & 7u);
        const bool ok = qi < nqs;
        const float *src = a.qr + ((size_t)(q0 + (ok ? qi : 0u)) * NQ + head) * HD + 8 * p;
        const float4 v0 = reinterpret_cast<const float4 *>(src)[0], v1 = reinterpret_cast<const float4 *>(src)[1];
        const float q8v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
        for (uint32_t d = 0; d < 8; d++) {
            qv[s][d] = ok ? q8v[d] : 0.0f;
            acc[s][d] = 0.0f;
        }
    }
    // softmax state of (row group rr, query my_s): the same in the group's 4 lanes of that query
    float mrun = -INFINITY, lrun = 0.0f;
    const uint32_t my_s = mp & 7u, my_i = mp >> 3;
    uint32_t my0, my1;
    range(my_s, my0, my1);
    LDS float *wgr = (LDS float *)wl + rr * (4 * PF_SLOTS + PF_SLOTS);
    LDS float *gml = (LDS float *)gm;

    for (uint32_t j = 0; j < ntile; j++) {
        const uint32_t t0 = U0 + j * ATT_TILE, b = j % PF_NBUF;
        if (PF_NBUF > 2 && j + 1 < ntile) {
            // tile j landed; tile j+1 may still fly
            if (Q8) asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
            else asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
        } else {
            dma_wait();
        }
        __syncthreads();   // tile j landed for every wave; every wave is past tile j - 1
        if (j + PF_NBUF - 1 < ntile) issue_tile(j + PF_NBUF - 1);   // into the buffer tile j - 1 used
        const LDS unsigned char *kt = Lu + b * ATT_F16_BUF, *vt = kt + ATT_TILE * 512;
        if constexpr (Q8) {
            const uint32_t rq = t >> 3, bb = t & 7u, rb = b * 2 * ATT_Q8_RAWB;
            const LDS unsigned char *raw = Lu + rb + rq * ATT_Q8_HEAD + 34u * bb;
            att_q8_split(raw, Lu + PF_Q8_KC + rq * 256 + 32u * bb, reinterpret_cast<LDS float *>(Lu + PF_Q8_KS) + t);
            sched_fence();
            att_q8_split(raw + ATT_Q8_RAWB, Lu + PF_Q8_VC + rq * 256 + 32u * bb,
                         reinterpret_cast<LDS float *>(Lu + PF_Q8_VS) + t);
            __syncthreads();
            kt = Lu + PF_Q8_KC;
            vt = Lu + PF_Q8_VC;
        }
        float part[4 * PF_SLOTS];
#pragma unroll
        for (uint32_t i = 0; i < 4; i++) {
            const uint32_t r = rr + 8 * (i ^ (mp >> 3));
            const LDS unsigned char *kr = kt + r * (Q8 ? 256u : 512u);
            const float ks = Q8 ? reinterpret_cast<const LDS float *>(Lu + PF_Q8_KS)[r * 8 + (p >> 2)] : 0.0f;
            float kd[8];
            att_row8<Q8>(kr, p, ks, kd);
#pragma unroll
            for (uint32_t s = 0; s < PF_SLOTS; s++) {
                float d = 0.0f;
#pragma unroll
                for (uint32_t dd = 0; dd < 8; dd++) d = fmaf(qv[s][dd], kd[dd], d);
                part[i * PF_SLOTS + s] = d;
            }
        }
        att_rs_step_x16(part);
        att_rs_step<DPP_MIRROR, 8>(part);
        att_rs_step<DPP_HALF_MIRROR, 4>(part);
        att_rs_step<DPP_XOR2, 2>(part);
        att_rs_step<DPP_XOR1, 1>(part);
        {
            const uint32_t row = t0 + rr + 8 * my_i;
            const bool valid = row >= my0 && row < my1;
            const float sv = valid ? part[0] * a.scale : -INFINITY;
            float mt = fmaxf(sv, dpp_f<DPP_MIRROR>(sv));
            mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
            const float mn = fmaxf(mrun, mt);
            const float wgt = valid ? att_exp(sv - mn) : 0.0f;
            float ws = wgt + dpp_f<DPP_MIRROR>(wgt);
            ws = ws + __shfl_xor(ws, 16, 64);
            const float cf = mrun == -INFINITY ? 0.0f : (mrun == mn ? 1.0f : att_exp(mrun - mn));
            const float lc = lrun * cf;
            lrun = lc + ws;
            mrun = mn;
            wgr[my_i * PF_SLOTS + my_s] = wgt;
            if (my_i == 0) wgr[4 * PF_SLOTS + my_s] = cf;
        }
        // (read back by this wave only: LDS accesses of a wave complete in order)
        {
            const f32x4 c0 = *reinterpret_cast<const LDS f32x4 *>(wgr + 4 * PF_SLOTS);
            const f32x4 c1 = *reinterpret_cast<const LDS f32x4 *>(wgr + 4 * PF_SLOTS + 4);
            const float cfv[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
#pragma unroll
            for (uint32_t s = 0; s < PF_SLOTS; s++)
#pragma unroll
                for (uint32_t dd = 0; dd < 8; dd++) acc[s][dd] = acc[s][dd] * cfv[s];
        }
#pragma unroll
        for (uint32_t i = 0; i < 4; i++) {
            const uint32_t r = rr + 8 * i;
            if (t0 + r < U1) {
                const LDS unsigned char *vr = vt + r * (Q8 ? 256u : 512u);
                const float vs = Q8 ? reinterpret_cast<const LDS float *>(Lu + PF_Q8_VS)[r * 8 + (p >> 2)] : 0.0f;
                float vd[8];
                att_row8<Q8>(vr, p, vs, vd);
                const f32x4 w0 = *reinterpret_cast<const LDS f32x4 *>(wgr + i * PF_SLOTS);
                const f32x4 w1 = *reinterpret_cast<const LDS f32x4 *>(wgr + i * PF_SLOTS + 4);
                const float w8[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
                for (uint32_t s = 0; s < PF_SLOTS; s++)
#pragma unroll
                    for (uint32_t dd = 0; dd < 8; dd++) acc[s][dd] = fmaf(w8[s], vd[dd], acc[s][dd]);
            }
        }
    }
    // the chunk's partial per query: the eight row groups merged (through
    // LDS, in the tile region) as the decode merges them
    LDS float *comb = reinterpret_cast<LDS float *>(Lu);   // [8 rr][8 slots][256]
    __syncthreads();
#pragma unroll
    for (uint32_t s = 0; s < PF_SLOTS; s++) {
        LDS float *d = comb + (rr * PF_SLOTS + s) * 256 + 8 * p;
        const f32x4 v0 = {acc[s][0], acc[s][1], acc[s][2], acc[s][3]};
        const f32x4 v1 = {acc[s][4], acc[s][5], acc[s][6], acc[s][7]};
        *reinterpret_cast<LDS f32x4 *>(d) = v0;
        *reinterpret_cast<LDS f32x4 *>(d + 4) = v1;
    }
    if (my_i == 0) {
        gml[rr * PF_SLOTS + my_s] = mrun;
        gml[8 * PF_SLOTS + rr * PF_SLOTS + my_s] = lrun;
    }
    __syncthreads();
    {
        const uint32_t s = t >> 5, po = t & 31;
        uint32_t k0, k1;
        range(s, k0, k1);
        float M = -INFINITY;
#pragma unroll
        for (uint32_t g2 = 0; g2 < 8; g2++) M = fmaxf(M, gml[g2 * PF_SLOTS + s]);
        float Lc = 0.0f, o[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (uint32_t g2 = 0; g2 < 8; g2++) {
            const float mg = gml[g2 * PF_SLOTS + s];
            const float e = mg != -INFINITY ? att_exp(mg - M) : 0.0f;
            Lc = fmaf(e, gml[8 * PF_SLOTS + g2 * PF_SLOTS + s], Lc);
            const f32x4 c0 = *reinterpret_cast<const LDS f32x4 *>(comb + (g2 * PF_SLOTS + s) * 256 + 8 * po);
            const f32x4 c1 = *reinterpret_cast<const LDS f32x4 *>(comb + (g2 * PF_SLOTS + s) * 256 + 8 * po + 4);
            const float cv[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
#pragma unroll
            for (uint32_t dd = 0; dd < 8; dd++) o[dd] = fmaf(e, cv[dd], o[dd]);
        }
        if (k1 > k0) {
            const uint32_t PS = att_rec(HD);
            float *d = a.part + (((size_t)(q0 + s) * NQ + head) * C + c) * PS;
            reinterpret_cast<float4 *>(d + 8 * po)[0] = make_float4(o[0], o[1], o[2], o[3]);
            reinterpret_cast<float4 *>(d + 8 * po)[1] = make_float4(o[4], o[5], o[6], o[7]);
            if (po == 0) {
                d[HD] = M;
                d[HD + 1] = Lc;
            }
        }
    }
}

// The decode attention's merge per (query, q head) -- one workgroup each,
// thread d the output element d: M = max over the query's chunks of m_c,
// e_c = exp(m_c - M), L = sum e_c l_c and O = sum e_c O_c as fmaf chains
// over the chunks ascending; out = O / L * sigmoid(gate).
__global__ __launch_bounds__(256) void attn_prefill_merge_kernel(AttnPrefill a) {
    __shared__ float e[64];
    __shared__ float Ls;
    const uint32_t q = blockIdx.x / a.nq, head = blockIdx.x % a.nq, HD = a.hd, C = a.n_chunks, PS = att_rec(HD);
    const uint32_t NC = att_geom((uint32_t)a.pos0 + q + 1u, C, a.chunk_min).n;
    const float *pb = a.part + ((size_t)q * a.nq + head) * C * PS;
    const uint32_t t = threadIdx.x;
    if (t < 64) {
        const uint32_t ci = min(t, NC - 1);
        const float m = pb[(size_t)ci * PS + HD], l = pb[(size_t)ci * PS + HD + 1];
        float M = t < NC ? m : -INFINITY;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
        const float ev = t < NC ? att_exp(m - M) : 0.0f;
        float L = 0.0f;
        for (uint32_t k = 0; k < NC; k++) {
            const float ek = __shfl(ev, (int)k, 64), lk = __shfl(l, (int)k, 64);
            L = fmaf(ek, lk, L);
        }
        e[t] = ev;
        if (t == 0) Ls = L;
    }
    __syncthreads();
    if (t < HD) {
        float O = 0.0f;
        for (uint32_t k = 0; k < NC; k++) O = fmaf(e[k], pb[(size_t)k * PS + t], O);
        const float gate = a.qg[((size_t)q * a.nq + head) * 2 * HD + HD + t];
        a.out[((size_t)q * a.nq + head) * HD + t] = (O / Ls) * dev_sigmoid(gate);
    }
}

}  // namespace

hipError_t launch_embed_ubatch(const void *embd, int type, uint32_t E, const int32_t *tokens, uint32_t n_tok, float *x,
                               hipStream_t s) {
    const dim3 grid((E / 4 + 255) / 256, n_tok);
    hipLaunchKernelGGL(embed_ubatch_kernel, grid, dim3(256), 0, s, static_cast<const char *>(embd), type, E,
                       (uint64_t)sinter_row_bytes_dev(type, E), tokens, x);
    return hipGetLastError();
}

hipError_t launch_gdn_ubatch(const float *qkv, const float *alpha, const float *beta, const float *dt_bias,
                             const float *ssm_a, float *state, float *o, float *work, uint32_t hk, uint32_t hv,
                             uint32_t d, uint32_t n_tok, float eps, float scale, hipStream_t s) {
    GdnUb a;
    a.qkv = qkv; a.alpha = alpha; a.beta = beta; a.dt_bias = dt_bias; a.ssm_a = ssm_a; a.state = state; a.o = o;
    a.qn = work;
    a.kn = a.qn + (size_t)n_tok * hk * d;
    a.gate = a.kn + (size_t)n_tok * hk * d;
    a.bgate = a.gate + (size_t)n_tok * hv;
    a.hk = hk; a.hv = hv; a.d = d; a.cols = d >= 128 ? 32u : 16u; a.n_tok = n_tok;
    a.c_stride = (2 * hk + hv) * d;
    a.eps = eps; a.scale = scale;
    const uint32_t items = hv * (d / a.cols), rpt = d / (256u / a.cols);
    if (n_tok == 0) return hipSuccess;
    hipLaunchKernelGGL(gdn_prep_ubatch_kernel, dim3(n_tok, hk), dim3(256), 0, s, a);
    switch (rpt) {
    case 4: hipLaunchKernelGGL(gdn_scan_ubatch_kernel<4>, dim3(items), dim3(256), 0, s, a); break;
    case 8: hipLaunchKernelGGL(gdn_scan_ubatch_kernel<8>, dim3(items), dim3(256), 0, s, a); break;
    case 16: hipLaunchKernelGGL(gdn_scan_ubatch_kernel<16>, dim3(items), dim3(256), 0, s, a); break;
    case 32: hipLaunchKernelGGL(gdn_scan_ubatch_kernel<32>, dim3(items), dim3(256), 0, s, a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// floats of launch_gdn_ubatch's work buffer
size_t gdn_ubatch_work(uint32_t hk, uint32_t hv, uint32_t d, uint32_t n_tok) {
    return (size_t)n_tok * (2 * (size_t)hk * d + 2 * (size_t)hv);
}

hipError_t launch_attn_prep_ubatch(const float *qg, const float *k, const float *v, const float *q_norm,
                                   const float *k_norm, void *kc, void *vc, uint32_t kv_type, int32_t pos0,
                                   uint32_t n_tok, uint32_t nq, uint32_t nkv, uint32_t hd, uint32_t rope_dims,
                                   float theta_scale, float eps, float *qr, hipStream_t s) {
    AttnPrepUb a;
    a.qg = qg; a.k = k; a.v = v; a.q_norm = q_norm; a.k_norm = k_norm; a.kc = kc; a.vc = vc; a.qr = qr;
    a.pos0 = pos0; a.n_tok = n_tok; a.nq = nq; a.nkv = nkv; a.hd = hd; a.rope_dims = rope_dims; a.kv_type = kv_type;
    a.theta_scale = theta_scale; a.eps = eps;
    hipLaunchKernelGGL(attn_prep_ubatch_kernel, dim3(n_tok, (nq + nkv + 3) / 4), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_attn_prefill(const float *qr, const float *qg, const void *kc, const void *vc, uint32_t kv_type,
                               int32_t pos0, uint32_t n_tok, uint32_t nq, uint32_t nkv, uint32_t hd,
                               uint32_t n_chunks, uint32_t chunk_min, float scale, float *part, float *out,
                               hipStream_t s) {
    AttnPrefill a;
    a.qr = qr; a.qg = qg; a.kc = kc; a.vc = vc; a.part = part; a.out = out; a.pos0 = pos0; a.n_tok = n_tok;
    a.nq = nq; a.nkv = nkv; a.hd = hd; a.kv_type = kv_type; a.n_chunks = n_chunks; a.chunk_min = chunk_min;
    a.scale = scale;
    if (n_tok == 0) return hipSuccess;
    // chunks of the deepest query (the others have as many or fewer)
    const uint32_t cmax = att_geom((uint32_t)pos0 + n_tok, n_chunks, chunk_min).n;
    const uint32_t items = nkv * cmax * (nq / nkv) * ((n_tok + PF_SLOTS - 1) / PF_SLOTS);
    if (kv_type == SINTER_Q8_0)
        hipLaunchKernelGGL(attn_prefill_split_kernel<true>, dim3(items), dim3(256), 0, s, a, cmax);
    else
        hipLaunchKernelGGL(attn_prefill_split_kernel<false>, dim3(items), dim3(256), 0, s, a, cmax);
    hipLaunchKernelGGL(attn_prefill_merge_kernel, dim3(n_tok * nq), dim3(256), 0, s, a);
    return hipGetLastError();
}

// floats of launch_attn_prefill's partials buffer
size_t attn_prefill_part(uint32_t n_tok, uint32_t nq, uint32_t hd, uint32_t n_chunks) {
    return (size_t)n_tok * nq * n_chunks * att_rec(hd);
}

}  // namespace sinter
