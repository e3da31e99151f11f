// SINTER_OP_ATTN_DECODE: one full-attention layer's decode step after the
// q|gate / k / v projections, fused:
//   per-head RMSNorm * weight + NEOX RoPE on the first rope_dims dims
//                                              (k0/ops/attn.cuh:109-182)
//   KV append at row pos, f16 (attn.cuh:184-211) or Q8_0 blocks (ggml's
//   f32 -> q8_0 block quantiser)
//   split-K online-softmax partials            (attn.cuh:244-401)
//   max/LSE merge by the last-arriving block   (attn.cuh:403-458)
//   sigmoid output gate                        (attn.cuh:460-488)
// Work item = (kv head g, chunk c).  An item serves all NQ/NKV q heads of
// its group from one read of its K/V rows (GQA sharing).  The item whose
// chunk holds `pos` also appends the new K/V row and uses it directly.  Each
// item publishes an fp64 partial {acc[HD], max, sum} per q head; the block
// that arrives last for kv head g merges that head group and applies the
// gate, so the reference's separate FATTN_REDUCE / ATTN_GATE windows (and
// their barriers) disappear.
//
// Declared numerics (oracle/oracle.c or_attn_decode_kv): q/k norms and RoPE
// in fp32 as ggml; scores are fp64 sums of exact products times the fp32
// scale; softmax and the V sum in fp64; the merged output rounded to fp32
// once.  A Q8_0 cache element is dequantised exactly (int8 code times the
// block's f16 scale, exact in fp32) before it enters the same arithmetic.
#pragma once
#include "dev_common.h"

namespace sinter {

constexpr int ATT_TILE = 32;   // KV positions per LDS tile
constexpr int ATT_MAXG = 8;    // max q heads per kv head
constexpr uint32_t ATT_Q8_HEAD = 272;   // one head's 256 elements as eight 34-byte Q8_0 blocks
// Q8_0 tile LDS map (in the f16 tiles' 64 KiB): raw K tiles at 0 and
// ATT_Q8_RAWB, raw V tiles at 2 * ATT_Q8_RAWB (+ ATT_Q8_RAWB), then the
// current tile split into codes [32][256] K and V, and scales [32][8] K and V
constexpr uint32_t ATT_Q8_RAWB = 9600;  // 32 rows x 272 B, plus the third DMA's overrun (56 chunks)
constexpr uint32_t ATT_Q8_KC = 4 * ATT_Q8_RAWB, ATT_Q8_VC = ATT_Q8_KC + 32 * 256;
constexpr uint32_t ATT_Q8_KS = ATT_Q8_VC + 32 * 256, ATT_Q8_VS = ATT_Q8_KS + 32 * 8 * 4;
static_assert(ATT_Q8_VS + 32 * 8 * 4 <= 4 * ATT_TILE * 512, "Q8_0 tiles fit the f16 tile region");
static_assert(ATT_Q8_RAWB % 16 == 0 && 4 * 136 * 16 + 56 * 16 <= ATT_Q8_RAWB, "raw tile plus overrun");

// The 8 elements [8p, 8p+8) of a 256-element head row, as exact doubles.
// f16: the row's 512 bytes (16-aligned).  Q8_0: the row split in LDS into
// its 256 int8 codes (row) and the eight block scales, sc being the scale of
// block p/4; a code times its scale is exact in fp64.
template <bool Q8>
__device__ __forceinline__ void att_row8(const LDS unsigned char *row, uint32_t p, float sc, double out[8]) {
    if constexpr (!Q8) {
        (void)sc;
        const u32x4 u = *reinterpret_cast<const LDS u32x4 *>(row + 16 * p);
        const uint32_t uw[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (uint32_t k = 0; k < 4; k++) {
            out[2 * k] = (double)h2f((uint16_t)(uw[k] & 0xffff));
            out[2 * k + 1] = (double)h2f((uint16_t)(uw[k] >> 16));
        }
    } else {
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        const u32x2 c = *reinterpret_cast<const LDS u32x2 *>(row + 8 * p);
        const double d = (double)sc;
#pragma unroll
        for (uint32_t k = 0; k < 8; k++) {
            const uint32_t w = k < 4 ? c.x : c.y;
            out[k] = (double)(int)(int8_t)((w >> (8 * (k & 3))) & 0xffu) * d;
        }
    }
}

// One Q8_0 block (34 bytes at src, 2-aligned: f16 d, 32 int8 codes) split
// into its codes (32 bytes at dst, 16-aligned) and its scale as f32.
__device__ __forceinline__ void att_q8_split(const LDS unsigned char *src, LDS unsigned char *dst, LDS float *sc) {
    const LDS uint16_t *h = reinterpret_cast<const LDS uint16_t *>(src);
    uint32_t w[8];
#pragma unroll
    for (int i = 0; i < 8; i++) w[i] = (uint32_t)h[1 + 2 * i] | ((uint32_t)h[2 + 2 * i] << 16);
    *sc = h2f(h[0]);
    const u32x4 a = {w[0], w[1], w[2], w[3]}, b = {w[4], w[5], w[6], w[7]};
    *reinterpret_cast<LDS u32x4 *>(dst) = a;
    *reinterpret_cast<LDS u32x4 *>(dst + 16) = b;
}

// ggml's f32 -> Q8_0 block quantiser (quantize_row_q8_0_ref; the KV-cache
// copy kernels do the same): per 32 elements amax = max |x|, d = amax / 127,
// id = d ? 1/d : 0, q = roundf(x * id), d stored as f16.  Thread t holds
// element t of a 256-element head; each 32-lane half-wave is one block; the
// 272-byte row lands in LDS at `row`.
__device__ __forceinline__ void att_quant_q8_0(float x, LDS unsigned char *row) {
    const uint32_t t = tid(), e = t & 31u;
    float am = fabsf(x);
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) am = fmaxf(am, __shfl_xor(am, o, 64));
    const float d = am / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    LDS unsigned char *blk = row + (t >> 5) * 34u;
    blk[2 + e] = (unsigned char)(int8_t)roundf(x * id);
    if (e == 0) *reinterpret_cast<LDS uint16_t *>(blk) = f2h(d);
}

// Per-pass cache (interpreter only): every attention op of one pass reads the
// same position from the same pass cell, so the first one of the pass loads
// it and computes the rope rotation; the others reuse both.  Key: pass
// index, pos, theta_scale bits, rope_dims, pass cell address (lo, hi); the
// interpreter invalidates it (key[0] = ~0) at launch.
__shared__ __attribute__((aligned(16))) float g_att_rot[256];
__shared__ uint32_t g_att_key[6];
constexpr uint32_t ATT_NO_CACHE = 0xffffffffu;

// The q heads of a kv group (and, for the chunk that appends, the new k row)
// normalised and rotated: y = rmsnorm(x) * w per 256-wide head, then NEOX
// RoPE on the first rope_dims dims.  Wave w takes heads w, w + 4, ...; lane l
// holds elements 4l .. 4l+3 of a head, so the head's sum of squares is the
// lane's four fp32 squares added in fp64 in order, then a wave butterfly (no
// workgroup barrier), and rope pair (i, i + rope_dims/2) lies in lanes i/4
// and i/4 + rope_dims/8 at the same component (rope_dims a multiple of 8).
// Rope pair i turns by theta_i = pos * theta_scale^i (repeated fp32
// products, as ggml's rope cache), cos/sin evaluated in double and rounded
// to fp32, into rot (cos | sin) -- only when compute_rot; otherwise rot
// already holds this position's rotation.  Rows j < nq read their raw
// values from src row j and use the q norm weight qw, row nq (if nh > nq)
// the k norm weight kw; results land in dst row j.  Ends with a workgroup
// barrier.
__device__ __forceinline__ void att_prep(uint32_t nq, uint32_t nh, float eps, int pos, float theta_scale,
                                         uint32_t rope_dims, const LDS float *src, const LDS float *qw,
                                         const LDS float *kw, LDS float *dst, LDS float *rot, bool compute_rot) {
    const uint32_t t = tid(), lane = t & 63u, w = t >> 6, half = rope_dims / 2, pl = half / 4;
    if (compute_rot) {
        // cos on wave 0, sin on wave 1 (the two run side by side)
        const uint32_t ri = t < 64 ? t : t - 64;
        if (t < 128 && ri < half) {
            float th = (float)pos;
            for (uint32_t i = 0; i < ri; i++) th *= theta_scale;
            if (t < 64) rot[ri] = (float)cos((double)th);
            else rot[128 + ri] = (float)sin((double)th);
        }
        __syncthreads();
    }
    const uint32_t e0 = 4 * lane, partner = lane < pl ? lane + pl : lane - pl;
    for (uint32_t j = w; j < nh; j += WAVES) {
        const f32x4 x = *reinterpret_cast<const LDS f32x4 *>(src + j * 256 + e0);
        const f32x4 wt = *reinterpret_cast<const LDS f32x4 *>((j < nq ? qw : kw) + e0);
        double ss = (double)(x.x * x.x);
        ss += (double)(x.y * x.y);
        ss += (double)(x.z * x.z);
        ss += (double)(x.w * x.w);
        ss = wave_sum_f64(ss);
        const float hs = 1.0f / sqrtf((float)(ss / 256.0) + eps);
        const float xv[4] = {x.x, x.y, x.z, x.w}, wv[4] = {wt.x, wt.y, wt.z, wt.w};
        float y[4], o[4];
#pragma unroll
        for (uint32_t c = 0; c < 4; c++) {
            const float nrm = xv[c] * hs;
            y[c] = nrm * wv[c];
        }
#pragma unroll
        for (uint32_t c = 0; c < 4; c++) o[c] = __shfl(y[c], (int)partner, 64);
#pragma unroll
        for (uint32_t c = 0; c < 4; c++) {
            const uint32_t i = e0 + c;
            if (i < half) {
                const float a0 = y[c] * rot[i], a1 = o[c] * rot[128 + i];
                y[c] = a0 - a1;
            } else if (i < 2 * half) {
                const float b0 = o[c] * rot[128 + i - half], b1 = y[c] * rot[i - half];
                y[c] = b0 + b1;
            }
        }
        const f32x4 r = {y[0], y[1], y[2], y[3]};
        *reinterpret_cast<LDS f32x4 *>(dst + j * 256 + e0) = r;
    }
    __syncthreads();
}

// Tile-loop thread roles: t = 64 rg + 32 hg + p.  Thread t covers tile rows
// [8 rg, 8 rg + 8), q head slots [4 hg, 4 hg + 4) and dims [8 p, 8 p + 8):
// for the scores it holds the slots' q (fp64) for its dims and forms the
// 8 x 4 partial dot products over them; for V it accumulates the same
// rows x slots x dims.  Every K/V element of a tile is converted by two
// threads (the two slot groups), every product appears once.
constexpr uint32_t ATT_RG = 8, ATT_HG = 4, ATT_DP = 8;

// Reduce-scatter of 32 fp64 partials over the 32 lanes of a half-wave
// without selects: lane p keeps its partials permuted, physical slot k
// holding logical index k ^ att_perm(p), where att_perm is the GF(2)-linear
// map taking the lane bits (1, 2, 4, 8, 16) to (1, 2, 7, 12, 16).  Every step
// then pairs each lane with one whose permutation differs by exactly the
// half being folded -- xor 16 (a shuffle), the row mirror (p ^ 15 within the
// row, whose image differs by 8), the half-row mirror (p ^ 7: by 4), xor 2,
// xor 1 -- so all lanes add the partner's upper half to their lower half:
// v[k] += partner's v[k + N].  Lane p ends with logical index att_perm(p).
__device__ __forceinline__ uint32_t att_perm(uint32_t p) {
    return (p & 16u) | ((p & 1u) ? 1u : 0u) ^ ((p & 2u) ? 2u : 0u) ^ ((p & 4u) ? 7u : 0u) ^ ((p & 8u) ? 12u : 0u);
}
template <int CTRL, int N>
__device__ __forceinline__ void att_rs_step(double v[]) {
#pragma unroll
    for (int k = 0; k < N; k++) v[k] = v[k] + dpp_d<CTRL>(v[k + N]);
}
__device__ __forceinline__ void att_rs_step_x16(double v[]) {
#pragma unroll
    for (int k = 0; k < 16; k++) v[k] = v[k] + __shfl_xor(v[k + 16], 16, 64);
}

// Wave 0: wait until each of the n (<= 64) generation flags at f holds at
// least target (wrap-safe); lane l polls flag l, one round trip per round.
// False on timeout (error raised); the result is wave-uniform.
__device__ __forceinline__ bool att_wait_flags(const uint32_t *f, uint32_t n, uint32_t target, uint64_t spin_limit,
                                               unsigned *err, uint32_t aux) {
    const uint32_t lane = lane_id();
    const __amdgpu_buffer_rsrc_t r = coh_rsrc(f, n * 4);
    const uint64_t t0 = wall_clock64();
    while (true) {
        bool ok = true;
        if (lane < n) ok = (int)(__float_as_uint(ld_coh4b(r, lane * 4)) - target) >= 0;
        if (__builtin_amdgcn_ballot_w64(!ok) == 0) return true;
        __builtin_amdgcn_s_sleep(1);
        const uint32_t el = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(wall_clock64() - t0));
        if (el > spin_limit) {
            if (lane == 0) raise_error(err, SINTER_E_TIMEOUT_BARRIER, aux);
            return false;
        }
    }
}

// ts (thread 0, or null): wall clock stamps [1] after the q prep, [2] after
// the KV tiles.  spin_limit bounds the wait for the other chunks of the kv
// head (wall clock ticks).  pass_id: the interpreter's pass index (the
// per-pass cache above), or ATT_NO_CACHE.
template <bool Q8>
__device__ __forceinline__ void op_attn_decode_t(const sinter_instr &ins, unsigned *err, uint64_t *ts,
                                                 uint64_t spin_limit, uint32_t pass_id) {
    // the payload, read once into registers: the op stores to the KV cache
    // and the partials, which the compiler cannot tell apart from the payload
    // (every field would be reloaded from memory after each such store)
    const sinter_attn_args a = *reinterpret_cast<const sinter_attn_args *>(ins.payload);
    const uint32_t rel = blockIdx.x - ins.block_lo, nblk = ins.block_hi - ins.block_lo;
    const uint32_t NQ = a.nq, NKV = a.nkv, HD = a.hd, C = a.n_chunks;
    const uint32_t pc_lo = (uint32_t)(uintptr_t)a.pass_cell, pc_hi = (uint32_t)((uintptr_t)a.pass_cell >> 32);
    const bool cached = pass_id != ATT_NO_CACHE && g_att_key[0] == pass_id && g_att_key[4] == pc_lo &&
                        g_att_key[5] == pc_hi;
    const int pos = cached ? (int)g_att_key[1] : ld_coh(&reinterpret_cast<const sinter_pass_cell *>(a.pass_cell)->pos);
    const bool rot_cached = cached && g_att_key[2] == __float_as_uint(a.theta_scale) && g_att_key[3] == a.rope_dims;
    const uint32_t gqa = NKV ? NQ / NKV : 0;
    constexpr bool q8 = Q8;
    const bool ok = HD == 256 && NKV && NQ % NKV == 0 && gqa >= 1 && gqa <= ATT_MAXG && C >= 1 && C <= 64 &&
                    NKV * C <= nblk && a.rope_dims <= HD && (a.rope_dims % 8) == 0 && pos >= 0 &&
                    (uint32_t)pos < a.n_ctx && (q8 == (a.kv_type == SINTER_Q8_0));
    if (!ok) {
        if (rel == 0 && threadIdx.x == 0) raise_error(err, SINTER_E_BAD_SHAPE, ins.dbg_node);
        return;
    }
    if (rel >= NKV * C) return;   // one item per workgroup (the merge waits for its kv head's chunks)
    // this chunk's generation flag (written only by this item, once per call)
    const uint32_t gen = ld_coh(a.count + rel);
    const uint32_t t = tid();
    const uint32_t PS = HD + 2;
    // cache row: all kv heads of a position; one head HB bytes
    const uint32_t HB = q8 ? ATT_Q8_HEAD : HD * 2u, RWB = NKV * HB;
    const uint32_t n_kv = (uint32_t)pos + 1;
    const uint32_t clen = (n_kv + C - 1) / C;

    // LDS map (the scratch region): K and V tiles double-buffered by LDS-DMA,
    // q heads (and the new k row), prep scratch, scores -> weights, softmax
    // corrections; after the tiles the K/V area holds the row-group sums,
    // then the merge's weights.
    lds_char *L = (lds_char *)g_big;
    LDS unsigned char *Lu = reinterpret_cast<LDS unsigned char *>(L);
    LDS uint16_t *kb = reinterpret_cast<LDS uint16_t *>(L);                          // [2][32][256]
    LDS uint16_t *vb = reinterpret_cast<LDS uint16_t *>(L + 2 * ATT_TILE * 512);     // [2][32][256]
    LDS float *qf = reinterpret_cast<LDS float *>(L + 4 * ATT_TILE * 512);           // [gqa][256] q, then the new k row
    LDS float *qn = qf + (ATT_MAXG + 1) * 256;    // [ATT_MAXG+4][256] raw q / k / v rows (then prep scratch), q_norm, k_norm
    LDS float *rot = (LDS float *)g_att_rot;                                         // [2][128] rope cos | sin
    LDS double *pred = reinterpret_cast<LDS double *>(qn + (ATT_MAXG + 4) * 256);    // [5][ATT_MAXG+1]
    LDS double *sc = pred + 5 * (ATT_MAXG + 1);                                      // [ATT_MAXG][32] scores -> weights
    LDS double *corr = sc + ATT_MAXG * ATT_TILE;                                     // [ATT_MAXG]
    LDS uint16_t *knew = reinterpret_cast<LDS uint16_t *>(corr + ATT_MAXG);          // [256]
    LDS uint16_t *vnew = knew + 256;                                                 // [256]
    LDS unsigned *flag = reinterpret_cast<LDS unsigned *>(vnew + 256);
    // Q8_0: the appended K / V head rows (16-aligned)
    LDS unsigned char *knew8 = reinterpret_cast<LDS unsigned char *>(
        ((uint32_t)(uintptr_t)(flag + 1) + 15u) & ~15u);
    LDS unsigned char *vnew8 = knew8 + ATT_Q8_HEAD;

    LDS double *comb = reinterpret_cast<LDS double *>(L);       // after the tiles: [4 rg][16][64 lanes]
    LDS double *mw = reinterpret_cast<LDS double *>(L);         // merge: [C][gqa] m, then weights e
    LDS double *mlv = mw + 64 * ATT_MAXG;                       //        [C][gqa] l
    LDS double *mM = mlv + 64 * ATT_MAXG;                       //        [ATT_MAXG + gqa]: L at ATT_MAXG + h
    LDS double *msum = mM + 2 * ATT_MAXG;                       //        [256] per-thread element partials
    const uint32_t w = __builtin_amdgcn_readfirstlane(t >> 6), lane = t & 63u;
    const uint32_t kbase = (uint32_t)(uintptr_t)kb, vbase = (uint32_t)(uintptr_t)vb;

    const uint32_t g = rel / C, c = rel % C;
    const uint32_t kv0 = min(c * clen, n_kv), kv1 = min(kv0 + clen, n_kv);
    const bool owner = kv0 <= (uint32_t)pos && (uint32_t)pos < kv1;
    const uint32_t ntile = (kv1 - kv0 + ATT_TILE - 1) / ATT_TILE;
    // Tile j (32 rows of this kv head: HB bytes of K and of V each) into
    // buffer j % 2 (16 KiB apart), rows back to back.  f16: each wave DMAs
    // rows 2k, 2k+1 for k = w, w+4, w+8, w+12 of K and of V (lane l: row
    // 2k + l/32, bytes 16 (l%32) ..) -- 8 DMAs per wave.  Q8_0: the tile's
    // 32 x 17 16-byte chunks into raw buffer j % 2 (ATT_Q8_RAWB apart),
    // wave w chunks [136w, 136w + 192) in three whole-wave DMAs per matrix --
    // 6 per wave; the last 56 chunks of a wave are the next wave's first (the
    // same bytes written twice), past the tile (wave 3) they land in the
    // buffer's overrun.  Rows past kv1 re-read row kv1-1 (masked in the
    // scores).
    auto issue_tile = [&](uint32_t j) {
        const uint32_t t0 = kv0 + j * ATT_TILE, bo = (j & 1) * ATT_TILE * 512;
        if (!q8) {
#pragma unroll
            for (uint32_t kk = 0; kk < 4; kk++) {
                const uint32_t k = w + 4 * kk, row = min(t0 + 2 * k + (lane >> 5), kv1 - 1);
                const uint32_t voff = row * RWB + g * HB + (lane & 31) * 16;
                lds_dma16<true>((uintptr_t)a.kc, voff, kbase + bo + k * 1024);
                lds_dma16<true>((uintptr_t)a.vc, voff, vbase + bo + k * 1024);
            }
            return;
        }
        const uint32_t rb = (j & 1) * ATT_Q8_RAWB;
#pragma unroll
        for (uint32_t kk = 0; kk < 3; kk++) {
            const uint32_t c0 = 136u * w + 64u * kk, ci = c0 + lane;
            const uint32_t row = min(t0 + ci / 17u, kv1 - 1), voff = row * RWB + g * HB + (ci % 17u) * 16u;
            lds_dma16<true>((uintptr_t)a.kc, voff, kbase + rb + c0 * 16u);
            lds_dma16<true>((uintptr_t)a.vc, voff, kbase + 2 * ATT_Q8_RAWB + rb + c0 * 16u);
        }
    };
    const uint32_t rg = t >> 6, hg = (t >> 5) & 1, p = t & 31, mp = att_perm(p);
    double qd[ATT_HG][ATT_DP];      // q slots 4hg + (j ^ mp%4), dims 8p.. (fp64)
    double acc[ATT_HG][ATT_DP];     // V sums over this thread's rows
    double mrun = -INFINITY, lrun = 0.0;   // softmax state of slot t/32 (every lane of the half-wave)
    {
        // The raw q heads g*gqa .. (and, for the owner, the new k and v
        // rows) by LDS-DMA into qn rows 0..gqa+1, the q and k norm weights
        // into rows ATT_MAXG+2, +3, one 1 KiB row per wave instruction; then
        // the first two tiles.  Every load before the tiles is a DMA, so the
        // explicit wait below is exact (a compiler-visible load here would
        // make the compiler's own wait count the tiles too) and the prep runs
        // while the tiles still stream in.
        const uint32_t nraw = owner ? gqa + 2 : gqa;
        const uint32_t qnbase = (uint32_t)(uintptr_t)qn;
        if (w < 2) {
            const float *src = w == 0 ? a.q_norm : a.k_norm;
            const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)src);
            const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)((uintptr_t)src >> 32));
            lds_dma16<false>(((uintptr_t)hi << 32) | lo, lane * 16, qnbase + (ATT_MAXG + 2 + w) * 1024);
        }
        for (uint32_t j = w; j < nraw; j += WAVES) {
            const float *src = j < gqa ? a.qg + (size_t)(g * gqa + j) * 2 * HD
                             : j == gqa ? a.k + (size_t)g * HD : a.v + (size_t)g * HD;
            const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)src);
            const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)((uintptr_t)src >> 32));
            lds_dma16<true>(((uintptr_t)hi << 32) | lo, lane * 16, qnbase + j * 1024);
        }
        if (ntile > 0) issue_tile(0);
        if (ntile > 1) issue_tile(1);
        const uint32_t per = q8 ? 6u : 8u;   // DMAs per tile per wave
        const uint32_t behind = (ntile > 0 ? per : 0u) + (ntile > 1 ? per : 0u);
        if (behind == 16) asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
        else if (behind == 12) asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
        else if (behind == 8) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
        else if (behind == 6) asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
        else dma_wait();
        __syncthreads();
        const float vraw = owner ? qn[(gqa + 1) * 256 + t] : 0.0f;
        att_prep(gqa, owner ? gqa + 1 : gqa, a.eps, pos, a.theta_scale, a.rope_dims, qn, qn + (ATT_MAXG + 2) * 256,
                 qn + (ATT_MAXG + 3) * 256, qf, rot, !rot_cached);
        if (owner && !q8) vnew[t] = f2h(vraw);
        if (owner && q8) att_quant_q8_0(vraw, vnew8);
        // (att_prep ended with a workgroup barrier: every thread has read the key)
        if (pass_id != ATT_NO_CACHE && t == 0) {
            g_att_key[0] = pass_id; g_att_key[1] = (uint32_t)pos; g_att_key[2] = __float_as_uint(a.theta_scale);
            g_att_key[3] = a.rope_dims; g_att_key[4] = pc_lo; g_att_key[5] = pc_hi;
        }
    }
    if (owner && !q8) {
        const uint16_t kh = f2h(qf[gqa * 256 + t]), vh = vnew[t];
        knew[t] = kh;
        const size_t o = (size_t)pos * RWB + (size_t)g * HB + 2u * t;
        st_coh(reinterpret_cast<uint16_t *>(static_cast<char *>(a.kc) + o), kh);
        st_coh(reinterpret_cast<uint16_t *>(static_cast<char *>(a.vc) + o), vh);
    }
    if (owner && q8) {
        // the head's K row quantised like its V row above, then both rows
        // (272 B each) stored by 17 lanes of 16 bytes
        att_quant_q8_0(qf[gqa * 256 + t], knew8);
        __syncthreads();
        // the new rows split like the tiles: codes at knew / vnew, scales after them
        if (t < 16) {
            LDS unsigned char *nd = reinterpret_cast<LDS unsigned char *>(t < 8 ? knew : vnew);
            att_q8_split((t < 8 ? knew8 : vnew8) + 34u * (t & 7u), nd + 32u * (t & 7u),
                         reinterpret_cast<LDS float *>(nd + 256) + (t & 7u));
        }

        if ((t & 31u) < 17u && t < 64) {
            const uint32_t i = t & 31u;
            const LDS unsigned char *src = (t < 32 ? knew8 : vnew8) + 16u * i;
            const u32x4 u = *reinterpret_cast<const LDS u32x4 *>(src);
            char *dst = static_cast<char *>(t < 32 ? a.kc : a.vc) + (size_t)pos * RWB + (size_t)g * HB + 16u * i;
            st_coh(reinterpret_cast<uint64_t *>(dst), (uint64_t)u.x | ((uint64_t)u.y << 32));
            st_coh(reinterpret_cast<uint64_t *>(dst) + 1, (uint64_t)u.z | ((uint64_t)u.w << 32));
        }
    }
#pragma unroll
    for (uint32_t j = 0; j < ATT_HG; j++) {
        const uint32_t hh = ATT_HG * hg + (j ^ (mp & 3));
        const f32x4 q0 = *reinterpret_cast<const LDS f32x4 *>(qf + hh * 256 + ATT_DP * p);
        const f32x4 q1 = *reinterpret_cast<const LDS f32x4 *>(qf + hh * 256 + ATT_DP * p + 4);
        const float qv[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
        for (uint32_t d = 0; d < ATT_DP; d++) {
            qd[j][d] = hh < gqa ? (double)qv[d] : 0.0;
            acc[j][d] = 0.0;
        }
    }
    if (ts) ts[1] = wall_clock64();

    for (uint32_t j = 0; j < ntile; j++) {
        const uint32_t t0 = kv0 + j * ATT_TILE, bo = (j & 1) * ATT_TILE * 512;
        if (j == 0) {
            dma_wait();   // (also the owner's cache stores)
        } else {
            // tile j landed; tile j+1 (issued last step) may still fly
            if (j + 1 < ntile) {
                if (q8) asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
                else asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
            } else {
                dma_wait();
            }
        }
        __syncthreads();
        if constexpr (Q8) {
            // thread t splits block t % 8 of row t / 8 of the K and the V tile
            const uint32_t rr = t >> 3, bb = t & 7u, rb = (j & 1) * ATT_Q8_RAWB;
            const LDS unsigned char *raw = Lu + rb + rr * ATT_Q8_HEAD + 34u * bb;
            att_q8_split(raw, Lu + ATT_Q8_KC + rr * 256 + 32u * bb, reinterpret_cast<LDS float *>(Lu + ATT_Q8_KS) + t);
            sched_fence();   // one block's words live at a time
            att_q8_split(raw + 2 * ATT_Q8_RAWB, Lu + ATT_Q8_VC + rr * 256 + 32u * bb,
                         reinterpret_cast<LDS float *>(Lu + ATT_Q8_VS) + t);
            __syncthreads();
        }
        // scores: partial dots over dims 8p..8p+7 (ascending) of rows
        // 8rg + (i ^ mp/4) and slots 4hg + (jj ^ mp%4) in slot i*4 + jj (the
        // permuted order above), then the reduce-scatter over the 32 lanes of
        // the half-wave leaves lane p with row 8rg + mp/4, slot 4hg + mp%4
        {
            double part[ATT_RG * ATT_HG];
#pragma unroll
            for (uint32_t i = 0; i < ATT_RG; i++) {
                const uint32_t r = ATT_RG * rg + (i ^ (mp >> 2));
                const bool nr = owner && t0 + r == (uint32_t)pos;
                const LDS unsigned char *kr = nr ? reinterpret_cast<const LDS unsigned char *>(knew)
                                            : q8 ? Lu + ATT_Q8_KC + r * 256
                                                 : reinterpret_cast<const LDS unsigned char *>(kb) + bo + r * 512;
                const float ks = !q8 ? 0.0f
                                : nr ? reinterpret_cast<const LDS float *>(kr + 256)[p >> 2]
                                     : reinterpret_cast<const LDS float *>(Lu + ATT_Q8_KS)[r * 8 + (p >> 2)];
                double kd[ATT_DP];
                att_row8<Q8>(kr, p, ks, kd);
#pragma unroll
                for (uint32_t jj = 0; jj < ATT_HG; jj++) {
                    double d = 0.0;
#pragma unroll
                    for (uint32_t dd = 0; dd < ATT_DP; dd++) d = fma(qd[jj][dd], kd[dd], d);
                    part[i * ATT_HG + jj] = d;
                }
            }
            att_rs_step_x16(part);
            att_rs_step<DPP_MIRROR, 8>(part);
            att_rs_step<DPP_HALF_MIRROR, 4>(part);
            att_rs_step<DPP_XOR2, 2>(part);
            att_rs_step<DPP_XOR1, 1>(part);
            const uint32_t r = ATT_RG * rg + (mp >> 2), hh = ATT_HG * hg + (mp & 3);
            sc[hh * ATT_TILE + r] = (t0 + r < kv1) ? part[0] * (double)a.scale : -INFINITY;
        }
        __syncthreads();
        // online softmax: head slot hh = t/32 over its 32 rows (lane r);
        // max and sum over the 32 lanes with DPP plus one cross-row step
        {
            const uint32_t hh = t / ATT_TILE, r = t % ATT_TILE;
            const double s = sc[hh * ATT_TILE + r];
            double mt = s;
            mt = fmax(mt, dpp_d<DPP_XOR1>(mt));
            mt = fmax(mt, dpp_d<DPP_XOR2>(mt));
            mt = fmax(mt, dpp_d<DPP_HALF_MIRROR>(mt));
            mt = fmax(mt, dpp_d<DPP_MIRROR>(mt));
            mt = fmax(mt, __shfl_xor(mt, 16, 64));
            const double mo = mrun;
            const double mn = fmax(mo, mt);
            const double wgt = (s == -INFINITY || hh >= gqa) ? 0.0 : exp(s - mn);
            double ws = row16_sum_f64(wgt);
            ws += __shfl_xor(ws, 16, 64);
            sc[hh * ATT_TILE + r] = wgt;
            // (an unchanged max: exp(0) = 1 exactly, so the call is skipped)
            const double cf = (mo == -INFINITY) ? 0.0 : (mo == mn ? 1.0 : exp(mo - mn));
            lrun = lrun * cf + ws;
            mrun = mn;
            if (r == 0) corr[hh] = cf;
        }
        __syncthreads();
        // V: rows 8rg+i, slots 4hg+jj, dims 8p.. (the weights are broadcast reads)
        {
#pragma unroll
            for (uint32_t jj = 0; jj < ATT_HG; jj++) {
                const double cf = corr[ATT_HG * hg + jj];
#pragma unroll
                for (uint32_t dd = 0; dd < ATT_DP; dd++) acc[jj][dd] = acc[jj][dd] * cf;
            }
#pragma unroll
            for (uint32_t i = 0; i < ATT_RG; i++) {
                const uint32_t r = ATT_RG * rg + i;
                const bool nr = owner && t0 + r == (uint32_t)pos;
                const LDS unsigned char *vr = nr ? reinterpret_cast<const LDS unsigned char *>(vnew)
                                            : q8 ? Lu + ATT_Q8_VC + r * 256
                                                 : reinterpret_cast<const LDS unsigned char *>(vb) + bo + r * 512;
                const float vs = !q8 ? 0.0f
                                : nr ? reinterpret_cast<const LDS float *>(vr + 256)[p >> 2]
                                     : reinterpret_cast<const LDS float *>(Lu + ATT_Q8_VS)[r * 8 + (p >> 2)];
                double wt[ATT_HG];
#pragma unroll
                for (uint32_t jj = 0; jj < ATT_HG; jj++) wt[jj] = sc[(ATT_HG * hg + jj) * ATT_TILE + r];
                double vd[ATT_DP];
                att_row8<Q8>(vr, p, vs, vd);
#pragma unroll
                for (uint32_t jj = 0; jj < ATT_HG; jj++)
#pragma unroll
                    for (uint32_t dd = 0; dd < ATT_DP; dd++) acc[jj][dd] = fma(wt[jj], vd[dd], acc[jj][dd]);
            }
        }
        __syncthreads();
        // the tile after next into the buffer just freed
        if (j + 2 < ntile) issue_tile(j + 2);
    }
    if (ts) ts[2] = wall_clock64();

    // the chunk's partial: the four row groups' V sums added in order (two
    // rounds of four dims each through LDS), published with m and l
    double *pbase = a.part + ((size_t)g * C + c) * gqa * PS;
    {
        const uint32_t hh = t >> 5, pp = t & 31;   // output: slot hh, dims 8pp + 4k + 0..3
#pragma unroll
        for (uint32_t k = 0; k < 2; k++) {
            // value (jj, dd) of lane l of row group rg at comb[(rg*16 + jj*4 + dd)*64 + l]:
            // every write and read instruction touches 64 consecutive doubles
#pragma unroll
            for (uint32_t jj = 0; jj < ATT_HG; jj++)
#pragma unroll
                for (uint32_t dd = 0; dd < 4; dd++) comb[(rg * 16 + jj * 4 + dd) * 64 + (t & 63)] = acc[jj][4 * k + dd];
            __syncthreads();
            // thread (hh, pp) sums row groups 0..3 of wave lane (hh/4)*32 + pp
            const uint32_t src_lane = (hh / ATT_HG) * 32 + pp, jj = hh % ATT_HG;
            double o[4];
#pragma unroll
            for (uint32_t dd = 0; dd < 4; dd++) {
                double sum = 0.0;
#pragma unroll
                for (uint32_t r4 = 0; r4 < 4; r4++) sum += comb[(r4 * 16 + jj * 4 + dd) * 64 + src_lane];
                o[dd] = sum;
            }
            if (hh < gqa) {
                double *d = pbase + hh * PS + ATT_DP * pp + 4 * k;
                st_coh(d, o[0]); st_coh(d + 1, o[1]); st_coh(d + 2, o[2]); st_coh(d + 3, o[3]);
            }
            __syncthreads();
        }
        if ((t & 31) == 0 && hh < gqa) {
            st_coh(pbase + hh * PS + HD, mrun);
            st_coh(pbase + hh * PS + HD + 1, lrun);
        }
    }

    // the merge's element mapping: this workgroup finalises elements
    // [c*ne, ...) of the head group's gqa*HD outputs, tpe threads per element
    const uint32_t E = gqa * HD, ne = (E + C - 1) / C, e0 = c * ne, e1 = min(e0 + ne, E);
    uint32_t tpe = 1;                           // a power of two <= C
    while (tpe * 2 <= C && tpe * 2 * ne <= BLOCK_THREADS) tpe *= 2;
    const uint32_t cpt = (C + tpe - 1) / tpe;   // chunks per thread
    const uint32_t ept = BLOCK_THREADS / tpe;   // elements per pass

    // wait for the kv head's C chunks: each publishes generation gen + 1 in
    // its own flag (one store, after its partial's stores completed) and
    // waits for all C flags of the head; the merge's gates are loaded while
    // the flags are polled (a load before the settle would be waited for)
    settle_vmem();
    __syncthreads();
    if (t == 0) st_coh(a.count + rel, gen + 1u);
    float gate0 = 0.0f;
    {
        const uint32_t el = min(e0 + t / tpe, E - 1);
        gate0 = ld_coh(a.qg + (size_t)(g * gqa + el / HD) * 2 * HD + HD + el % HD);
    }
    if (t < 64) {
        const bool okw = att_wait_flags(a.count + g * C, C, gen + 1u, spin_limit, err, ins.dbg_node);
        if (t == 0) *flag = okw ? 1u : 0u;
    }
    __syncthreads();
    if (*flag == 0) return;

    // merge: M = max m_i, acc = sum_i e_i acc_i, l = sum_i e_i l_i with
    // e_i = exp(m_i - M), chunks ascending (runs of cpt chunks per thread,
    // the runs then ascending); out = acc/l * sigmoid(gate).  Every load of
    // the first pass is issued at once: m and l of each (chunk, slot) and
    // this thread's first eight chunk values.
    {
        const __amdgpu_buffer_rsrc_t r = coh_rsrc(a.part + (size_t)g * C * gqa * PS, C * gqa * PS * 8);
        double vpre[8];
        {
            const uint32_t el = min(e0 + t / tpe, e1 - 1), hh = el / HD, dd = el % HD, i0 = (t % tpe) * cpt;
#pragma unroll
            for (uint32_t k = 0; k < 8; k++) {
                const uint32_t i = min(i0 + k, C - 1);
                vpre[k] = ld_coh8(r, (((size_t)i * gqa + hh) * PS + dd) * 8);
            }
        }
        {
            // (C*gqa <= 512: two per thread)
            const uint32_t n = C * gqa, i0 = t, i1 = t + BLOCK_THREADS;
            const uint32_t j0 = min(i0, n - 1), j1 = min(i1, n - 1);
            const double m0 = ld_coh8(r, ((size_t)j0 * PS + HD) * 8), l0 = ld_coh8(r, ((size_t)j0 * PS + HD + 1) * 8);
            const double m1 = ld_coh8(r, ((size_t)j1 * PS + HD) * 8), l1 = ld_coh8(r, ((size_t)j1 * PS + HD + 1) * 8);
            if (i0 < n) { mw[i0] = m0; mlv[i0] = l0; }
            if (i1 < n) { mw[i1] = m1; mlv[i1] = l1; }
        }
        __syncthreads();
        // slot h on wave h % 4, chunk i on lane i: M by a wave max, then the
        // weights e_i and L = sum_i e_i l_i (a wave sum)
        for (uint32_t h = w; h < gqa; h += WAVES) {
            const double m = lane < C ? mw[lane * gqa + h] : -INFINITY;
            double M = m;
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) M = fmax(M, __shfl_xor(M, o, 64));
            const double e = (m == -INFINITY) ? 0.0 : exp(m - M);
            const double le = (lane < C && e != 0.0) ? e * mlv[lane * gqa + h] : 0.0;
            const double Ls = wave_sum_f64(le);
            if (lane < C) mw[lane * gqa + h] = e;
            if (lane == 0) mM[ATT_MAXG + h] = Ls;
        }
        __syncthreads();
        for (uint32_t eb = e0; eb < e1; eb += ept) {
            const uint32_t el = eb + t / tpe, sub = t % tpe;
            const uint32_t elc = min(el, e1 - 1), hh = elc / HD, dd = elc % HD;
            const uint32_t i0 = sub * cpt, i1 = min(i0 + cpt, C);
            double O = 0.0;
            // eight chunks' values per batch, all loads issued first (the
            // first batch of the first pass is already in flight)
            for (uint32_t ib = i0; ib < i1; ib += 8) {
                double v[8];
#pragma unroll
                for (uint32_t k = 0; k < 8; k++) {
                    const uint32_t i = min(ib + k, C - 1);
                    v[k] = (eb == e0 && ib == i0) ? vpre[k] : ld_coh8(r, (((size_t)i * gqa + hh) * PS + dd) * 8);
                }
#pragma unroll
                for (uint32_t k = 0; k < 8; k++) {
                    const double e = ib + k < i1 ? mw[(ib + k) * gqa + hh] : 0.0;
                    if (e != 0.0) O = fma(e, v[k], O);
                }
            }
            msum[t] = O;
            __syncthreads();
            if (el < e1 && sub == 0) {
                double tot = 0.0;
                for (uint32_t s2 = 0; s2 < tpe; s2++) tot += msum[t + s2];
                const uint32_t h = g * gqa + hh;
                const float att = (float)(tot / mM[ATT_MAXG + hh]);
                const float gate = eb == e0 ? gate0 : ld_coh(a.qg + (size_t)h * 2 * HD + HD + dd);
                st_coh(a.out + (size_t)h * HD + dd, att * dev_sigmoid(gate));
            }
            __syncthreads();
        }
    }
    settle_vmem();
}

// the attention op of the KV cache types in feature set F
template <uint32_t F>
__device__ __forceinline__ void op_attn_decode(const sinter_instr &ins, unsigned *err, uint64_t *ts,
                                               uint64_t spin_limit, uint32_t pass_id) {
    // (op_attn_decode_t raises BAD_SHAPE itself for a cache of the other type)
    if constexpr ((F & FEAT_KV_Q80) == 0) {
        op_attn_decode_t<false>(ins, err, ts, spin_limit, pass_id);
    } else if constexpr ((F & FEAT_KV_F16) == 0) {
        op_attn_decode_t<true>(ins, err, ts, spin_limit, pass_id);
    } else {
        if (reinterpret_cast<const sinter_attn_args *>(ins.payload)->kv_type == SINTER_Q8_0)
            op_attn_decode_t<true>(ins, err, ts, spin_limit, pass_id);
        else
            op_attn_decode_t<false>(ins, err, ts, spin_limit, pass_id);
    }
}

}  // namespace sinter
