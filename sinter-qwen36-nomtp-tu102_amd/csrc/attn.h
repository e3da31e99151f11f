// SINTER_OP_ATTN_DECODE: one full-attention layer's decode step after the
// q|gate / k / v projections, fused:
//   per-head RMSNorm * weight + NEOX RoPE on the first rope_dims dims
//                                              (k0/ops/attn.cuh:109-182)
//   KV append at row pos, f16 (attn.cuh:184-211) or Q8_0 blocks (ggml's
//   f32 -> q8_0 block quantiser)
//   split-K online-softmax partials            (attn.cuh:244-401)
//   max/LSE merge by the chunks themselves     (attn.cuh:403-458)
//   sigmoid output gate                        (attn.cuh:460-488)
// Work item = (kv head g, chunk c).  An item serves all NQ/NKV q heads of
// its group from one read of its K/V rows (GQA sharing).  The item whose
// chunk holds `pos` also appends the new K/V row and uses it directly.  Each
// item publishes an fp32 partial {acc[HD], max, sum} per q head, then the
// kv head's chunks wait for each other and each merges a slice of the head
// group's outputs and applies the gate, so the reference's separate
// FATTN_REDUCE / ATTN_GATE windows (and their barriers) disappear.
//
// Declared numerics (fp32 folds in the reference's manner, attn.cuh:33-42;
// oracle/oracle.c or_attn_split computes the same values):
//   chunks   whole 32-position tiles: T = ceil(n_kv/32) tiles, tpc =
//            max(ceil(T/C), ceil(chunk_min/32)) tiles per chunk, ceil(T/tpc)
//            chunks (att_geom) -- fewer, longer chunks at shallow depth;
//   scores   q (fp32, normalised and rotated) . k: lane p of 32 holds dims
//            8p..8p+7 and chains fmaf over them in ascending order; the 32
//            lane sums are added by the tree of lane xor-masks 16, 15, 7, 2, 1
//            (level by level); times the fp32 scale; rows past n_kv -> -inf;
//   groups   the rows of a tile split into 8 row groups (row mod 8), each
//            with its own online softmax per q head over its rows of the
//            chunk's tiles (ascending):
//   softmax  per tile: m' = max(m, max of the group's scores in the tile);
//            w = exp(s - m') and the correction exp(m - m') (0 before the
//            group's first row, 1 when m is unchanged) evaluated in fp64 and
//            rounded to fp32; the tile's (<= 4) w of the group added as
//            (w0 + w1) + (w2 + w3); l = l*corr + sum;
//   V sums   per (q head, dim): acc = acc*corr per tile, then fmaf(w, v, acc)
//            over the group's rows of the tile ascending;
//   chunk    the 8 groups merged per q head: M = max m_g, e_g = exp(m_g - M)
//            (0 for a group without rows), L and O fmaf chains over the groups
//            ascending -- the chunk's partial {O, M, L};
//   merge    M = max over chunks of m; e_c = exp(m_c - M) (fp64, rounded);
//            L and O are fmaf chains over the chunks ascending; out = O / L,
//            then times sigmoid(gate).
// A Q8_0 cache element is its int8 code times its block's f16 scale, exact in
// fp32; an f16 element converts exactly.
#pragma once
#include "dev_common.h"

namespace sinter {

constexpr int ATT_TILE = 32;   // KV positions per LDS tile
constexpr int ATT_MAXG = 8;    // max q heads per kv head
constexpr uint32_t ATT_Q8_HEAD = 272;   // one head's 256 elements as eight 34-byte Q8_0 blocks
// Tiles in flight: tile j lands in buffer j % ATT_NBUF of the scratch region
// (g_big); tile j + 2 is issued once every wave is past tile j - 1.
constexpr uint32_t ATT_NBUF = 3;
constexpr uint32_t ATT_F16_BUF = 2 * ATT_TILE * 512;   // f16: K rows [32][512 B], then V rows
static_assert(ATT_NBUF * ATT_F16_BUF <= BIG_BYTES, "f16 tiles fit the scratch region");
// Q8_0 tile LDS map: raw K and V tiles of buffer b at 2 b ATT_Q8_RAWB (+
// ATT_Q8_RAWB), then the current tile split into codes [32][256] K and V,
// and scales [32][8] K and V
constexpr uint32_t ATT_Q8_RAWB = 9600;  // 32 rows x 272 B, plus the third DMA's overrun (56 chunks)
constexpr uint32_t ATT_Q8_KC = 2 * ATT_NBUF * ATT_Q8_RAWB, ATT_Q8_VC = ATT_Q8_KC + 32 * 256;
constexpr uint32_t ATT_Q8_KS = ATT_Q8_VC + 32 * 256, ATT_Q8_VS = ATT_Q8_KS + 32 * 8 * 4;
static_assert(ATT_Q8_VS + 32 * 8 * 4 <= BIG_BYTES, "Q8_0 tiles fit the scratch region");
static_assert(ATT_Q8_RAWB % 16 == 0 && 4 * 136 * 16 + 56 * 16 <= ATT_Q8_RAWB, "raw tile plus overrun");

// The 8 elements [8p, 8p+8) of a 256-element head row as fp32 (exact).
// f16: the row's 512 bytes (16-aligned).  Q8_0: the row split in LDS into
// its 256 int8 codes (row) and the eight block scales, sc being the scale of
// block p/4; a code times its scale is exact in fp32.
template <bool Q8>
__device__ __forceinline__ void att_row8(const LDS unsigned char *row, uint32_t p, float sc, float out[8]) {
    if constexpr (!Q8) {
        (void)sc;
        const u32x4 u = *reinterpret_cast<const LDS u32x4 *>(row + 16 * p);
        const uint32_t uw[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (uint32_t k = 0; k < 4; k++) {
            out[2 * k] = h2f((uint16_t)(uw[k] & 0xffff));
            out[2 * k + 1] = h2f((uint16_t)(uw[k] >> 16));
        }
    } else {
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        const u32x2 c = *reinterpret_cast<const LDS u32x2 *>(row + 8 * p);
#pragma unroll
        for (uint32_t k = 0; k < 8; k++) {
            const uint32_t w = k < 4 ? c.x : c.y;
            out[k] = (float)(int)(int8_t)((w >> (8 * (k & 3))) & 0xffu) * sc;
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

// Tile-loop thread roles: t = 32 rr + p.  For the scores thread t covers the
// tile rows rr + 8i (i < 4), all ATT_MAXG q head slots and dims [8p, 8p+8):
// it holds the slots' q for its dims and forms the 4 x 8 partial dot
// products over them; for the V sums it accumulates the same rows, slots and
// dims.  Every product appears once.
// Reduce-scatter of 32 fp32 partials over the 32 lanes of a half-wave
// without selects: lane p keeps its partials permuted, physical slot k
// holding logical index k ^ att_perm(p), where att_perm is the GF(2)-linear
// map taking the lane bits (1, 2, 4, 8, 16) to (1, 2, 7, 12, 16).  Every step
// then pairs each lane with one whose permutation differs by exactly the
// half being folded -- xor 16 (a shuffle), the row mirror (p ^ 15 within the
// row, whose image differs by 8), the half-row mirror (p ^ 7: by 4), xor 2,
// xor 1 -- so all lanes add the partner's upper half to their lower half:
// v[k] += partner's v[k + N].  Lane p ends with logical index att_perm(p),
// the sum over the lanes by the tree of masks 16, 15, 7, 2, 1.
__device__ __forceinline__ uint32_t att_perm(uint32_t p) {
    return (p & 16u) | ((p & 1u) ? 1u : 0u) ^ ((p & 2u) ? 2u : 0u) ^ ((p & 4u) ? 7u : 0u) ^ ((p & 8u) ? 12u : 0u);
}
template <int CTRL, int N>
__device__ __forceinline__ void att_rs_step(float v[]) {
#pragma unroll
    for (int k = 0; k < N; k++) v[k] = v[k] + dpp_f<CTRL>(v[k + N]);
}
__device__ __forceinline__ void att_rs_step_x16(float v[]) {
#pragma unroll
    for (int k = 0; k < 16; k++) v[k] = v[k] + __shfl_xor(v[k + 16], 16, 64);
}
// Max / sum over the 32 lanes of a half-wave, lane masks 1, 2, 7, 15, 16 in
// this order (every lane gets the result)
__device__ __forceinline__ float att_max32(float v) {
    v = fmaxf(v, dpp_f<DPP_XOR1>(v));
    v = fmaxf(v, dpp_f<DPP_XOR2>(v));
    v = fmaxf(v, dpp_f<DPP_HALF_MIRROR>(v));
    v = fmaxf(v, dpp_f<DPP_MIRROR>(v));
    return fmaxf(v, __shfl_xor(v, 16, 64));
}
__device__ __forceinline__ float att_sum32(float v) {
    v = v + dpp_f<DPP_XOR1>(v);
    v = v + dpp_f<DPP_XOR2>(v);
    v = v + dpp_f<DPP_HALF_MIRROR>(v);
    v = v + dpp_f<DPP_MIRROR>(v);
    return v + __shfl_xor(v, 16, 64);
}
// fp64-evaluated exponential rounded to fp32 (the declared transcendental rule)
__device__ __forceinline__ float att_exp(float x) { return (float)exp((double)x); }

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
    const uint64_t hdr = ins_hdr(ins);
    const uint32_t rel = blockIdx.x - hdr_lo(hdr), nblk = hdr_hi(hdr) - hdr_lo(hdr);
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
    const uint32_t PS = att_rec(HD);
    // cache row: all kv heads of a position; one head HB bytes
    const uint32_t HB = q8 ? ATT_Q8_HEAD : HD * 2u, RWB = NKV * HB;
    const uint32_t n_kv = (uint32_t)pos + 1;
    const AttGeom geo = att_geom(n_kv, C, a.chunk_min);

    // LDS map: K and V tiles (ATT_NBUF buffers by LDS-DMA) in the scratch
    // region; in the GEMV activation buffer (unused by this op): q heads (and
    // the new k row), prep scratch, the tile weights of each half-wave, the
    // new K/V rows, the merge's chunk weights.
    lds_char *L = (lds_char *)g_big;
    LDS unsigned char *Lu = reinterpret_cast<LDS unsigned char *>(L);
    lds_char *Q = (lds_char *)g_qbuf;
    LDS float *qf = reinterpret_cast<LDS float *>(Q);                                // [gqa][256] q, then the new k row
    LDS float *qn = qf + (ATT_MAXG + 1) * 256;    // [ATT_MAXG+4][256] raw q / k / v rows (then prep scratch), q_norm, k_norm
    LDS float *rot = (LDS float *)g_att_rot;                                         // [2][128] rope cos | sin
    LDS float *wl = qn + (ATT_MAXG + 4) * 256;    // [8 row groups][4 rows x 8 slots weights | 8 corr], then m, l [2][8][8]
    LDS float *me = wl + 8 * 5 * ATT_MAXG + 2 * 8 * ATT_MAXG;                        // merge: [64][ATT_MAXG] chunk weights
    LDS float *mL = me + 64 * ATT_MAXG;                                              //        [ATT_MAXG] L per slot
    LDS uint16_t *knew = reinterpret_cast<LDS uint16_t *>(mL + ATT_MAXG);            // [256]
    LDS uint16_t *vnew = knew + 256;                                                 // [256]
    LDS unsigned *flag = reinterpret_cast<LDS unsigned *>(vnew + 256);
    // Q8_0: the appended K / V head rows (16-aligned)
    LDS unsigned char *knew8 = reinterpret_cast<LDS unsigned char *>(
        ((uint32_t)(uintptr_t)(flag + 1) + 15u) & ~15u);
    LDS unsigned char *vnew8 = knew8 + ATT_Q8_HEAD;

    const uint32_t w = __builtin_amdgcn_readfirstlane(t >> 6), lane = t & 63u;
    const uint32_t kbase = (uint32_t)(uintptr_t)L;

    const uint32_t g = rel / C, c = rel % C;
    if (c >= geo.n) {
        // no positions for this chunk at this depth: its generation flag
        // still advances, so every flag of the kv head moves in step
        if (t == 0) st_coh(a.count + rel, gen + 1u);
        return;
    }
    const uint32_t kv0 = c * geo.tpc * ATT_TILE, kv1 = min(kv0 + geo.tpc * ATT_TILE, n_kv);
    const bool owner = kv0 <= (uint32_t)pos && (uint32_t)pos < kv1;
    const uint32_t ntile = (kv1 - kv0 + ATT_TILE - 1) / ATT_TILE;
    // Tile j (32 rows of this kv head: HB bytes of K and of V each) into
    // buffer j % ATT_NBUF, rows back to back.  f16: each wave DMAs
    // rows 2k, 2k+1 for k = w, w+4, w+8, w+12 of K and of V (lane l: row
    // 2k + l/32, bytes 16 (l%32) ..) -- 8 DMAs per wave.  Q8_0: the tile's
    // 32 x 17 16-byte chunks into raw buffer j % ATT_NBUF (K, then V),
    // wave w chunks [136w, 136w + 192) in three whole-wave DMAs per matrix --
    // 6 per wave; the last 56 chunks of a wave are the next wave's first (the
    // same bytes written twice), past the tile (wave 3) they land in the
    // buffer's overrun.  Rows past kv1 re-read row kv1-1 (masked in the
    // scores).
    auto issue_tile = [&](uint32_t j) {
        const uint32_t t0 = kv0 + j * ATT_TILE, bo = (j % ATT_NBUF) * ATT_F16_BUF;
        if (!q8) {
#pragma unroll
            for (uint32_t kk = 0; kk < 4; kk++) {
                const uint32_t k = w + 4 * kk, row = min(t0 + 2 * k + (lane >> 5), kv1 - 1);
                const uint32_t voff = row * RWB + g * HB + (lane & 31) * 16;
                lds_dma16<true>((uintptr_t)a.kc, voff, kbase + bo + k * 1024);
                lds_dma16<true>((uintptr_t)a.vc, voff, kbase + bo + ATT_TILE * 512 + k * 1024);
            }
            return;
        }
        const uint32_t rb = (j % ATT_NBUF) * 2 * ATT_Q8_RAWB;
#pragma unroll
        for (uint32_t kk = 0; kk < 3; kk++) {
            const uint32_t c0 = 136u * w + 64u * kk, ci = c0 + lane;
            const uint32_t row = min(t0 + ci / 17u, kv1 - 1), voff = row * RWB + g * HB + (ci % 17u) * 16u;
            lds_dma16<true>((uintptr_t)a.kc, voff, kbase + rb + c0 * 16u);
            lds_dma16<true>((uintptr_t)a.vc, voff, kbase + rb + ATT_Q8_RAWB + c0 * 16u);
        }
    };    {
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
    // Thread roles in the tile loop: t = 32 rr + p.  Row group rr (one
    // half-wave) takes the tile rows rr + 8i (i < 4); lane p the dims
    // 8p..8p+7.  A lane holds every head slot's q for its dims (register slot
    // s holding head slot s ^ (mp & 7), permuted for the reduce-scatter) and
    // the V sums of every slot for its dims.  Each row group keeps its own
    // online softmax per slot (the group's rows of a slot sit in 4 lanes), so
    // a tile needs one workgroup barrier; the eight groups are merged at the
    // chunk's end.
    const uint32_t rr = t >> 5, p = t & 31, mp = att_perm(p);
    float qv[ATT_MAXG][8], acc[ATT_MAXG][8];
#pragma unroll
    for (uint32_t s = 0; s < ATT_MAXG; s++) {
        const uint32_t hh = s ^ (mp & 7u);
        const f32x4 q0 = *reinterpret_cast<const LDS f32x4 *>(qf + hh * 256 + 8 * p);
        const f32x4 q1 = *reinterpret_cast<const LDS f32x4 *>(qf + hh * 256 + 8 * p + 4);
        const float q8v[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
        for (uint32_t d = 0; d < 8; d++) {
            qv[s][d] = hh < gqa ? q8v[d] : 0.0f;
            acc[s][d] = 0.0f;
        }
    }
    // softmax state of (row group rr, slot mp % 8): the same in the group's 4 lanes of that slot
    float mrun = -INFINITY, lrun = 0.0f;
    const uint32_t my_s = mp & 7u, my_i = mp >> 3;
    LDS float *wgr = wl + rr * (4 * ATT_MAXG + ATT_MAXG);   // this group's weights [4 rows][8 slots], then corr [8]
    if (ts) ts[1] = wall_clock64();

    for (uint32_t j = 0; j < ntile; j++) {
        const uint32_t t0 = kv0 + j * ATT_TILE, b = j % ATT_NBUF;
        if (j == 0 || j + 1 >= ntile) {
            dma_wait();   // (the first: also the owner's cache stores)
        } else {
            // tile j landed; tile j+1 may still fly
            if (q8) asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
            else asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
        }
        __syncthreads();   // tile j landed for every wave; every wave is past tile j - 1
        if (j + 2 < ntile) issue_tile(j + 2);   // into the buffer tile j - 1 used
        const LDS unsigned char *kt = Lu + b * ATT_F16_BUF, *vt = kt + ATT_TILE * 512;
        if constexpr (Q8) {
            // thread t splits block t % 8 of row t / 8 of the K and the V tile
            const uint32_t rq = t >> 3, bb = t & 7u, rb = b * 2 * ATT_Q8_RAWB;
            const LDS unsigned char *raw = Lu + rb + rq * ATT_Q8_HEAD + 34u * bb;
            att_q8_split(raw, Lu + ATT_Q8_KC + rq * 256 + 32u * bb, reinterpret_cast<LDS float *>(Lu + ATT_Q8_KS) + t);
            sched_fence();   // one block's words live at a time
            att_q8_split(raw + ATT_Q8_RAWB, Lu + ATT_Q8_VC + rq * 256 + 32u * bb,
                         reinterpret_cast<LDS float *>(Lu + ATT_Q8_VS) + t);
            __syncthreads();
            kt = Lu + ATT_Q8_KC;
            vt = Lu + ATT_Q8_VC;
        }
        // scores: partial dots over dims 8p..8p+7 (ascending fmaf) of rows
        // rr + 8 (i ^ mp/8) and slots s ^ mp%8 in slot 8i + s; the
        // reduce-scatter over the half-wave leaves lane p with row rr + 8 (mp/8),
        // slot mp%8
        float part[4 * ATT_MAXG];
#pragma unroll
        for (uint32_t i = 0; i < 4; i++) {
            const uint32_t r = rr + 8 * (i ^ (mp >> 3));
            const bool nr = owner && t0 + r == (uint32_t)pos;
            const LDS unsigned char *kr = nr ? reinterpret_cast<const LDS unsigned char *>(knew)
                                             : kt + r * (q8 ? 256u : 512u);
            const float ks = !q8 ? 0.0f
                            : nr ? reinterpret_cast<const LDS float *>(kr + 256)[p >> 2]
                                 : reinterpret_cast<const LDS float *>(Lu + ATT_Q8_KS)[r * 8 + (p >> 2)];
            float kd[8];
            att_row8<Q8>(kr, p, ks, kd);
#pragma unroll
            for (uint32_t s = 0; s < ATT_MAXG; s++) {
                float d = 0.0f;
#pragma unroll
                for (uint32_t dd = 0; dd < 8; dd++) d = fmaf(qv[s][dd], kd[dd], d);
                part[i * ATT_MAXG + s] = d;
            }
        }
        att_rs_step_x16(part);
        att_rs_step<DPP_MIRROR, 8>(part);
        att_rs_step<DPP_HALF_MIRROR, 4>(part);
        att_rs_step<DPP_XOR2, 2>(part);
        att_rs_step<DPP_XOR1, 1>(part);
        // the group's online softmax of slot my_s over its (<= 4) rows of the
        // tile: the lanes of one slot differ by the lane masks 15 (row i ^ 1)
        // and 16 (row i ^ 2)
        {
            const uint32_t r = rr + 8 * my_i;
            const bool valid = my_s < gqa && t0 + r < kv1;
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
            wgr[my_i * ATT_MAXG + my_s] = wgt;
            if (my_i == 0) wgr[4 * ATT_MAXG + my_s] = cf;
        }
        // (read back by this wave only: LDS accesses of a wave complete in order)
        {
            const f32x4 c0 = *reinterpret_cast<const LDS f32x4 *>(wgr + 4 * ATT_MAXG);
            const f32x4 c1 = *reinterpret_cast<const LDS f32x4 *>(wgr + 4 * ATT_MAXG + 4);
            const float cfv[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
#pragma unroll
            for (uint32_t s = 0; s < ATT_MAXG; s++)
#pragma unroll
                for (uint32_t dd = 0; dd < 8; dd++) acc[s][dd] = acc[s][dd] * cfv[s];
        }
        // V: the group's rows ascending, every slot, dims 8p..
#pragma unroll
        for (uint32_t i = 0; i < 4; i++) {
            const uint32_t r = rr + 8 * i;
            if (t0 + r < kv1) {
                const bool nr = owner && t0 + r == (uint32_t)pos;
                const LDS unsigned char *vr = nr ? reinterpret_cast<const LDS unsigned char *>(vnew)
                                                 : vt + r * (q8 ? 256u : 512u);
                const float vs = !q8 ? 0.0f
                                : nr ? reinterpret_cast<const LDS float *>(vr + 256)[p >> 2]
                                     : reinterpret_cast<const LDS float *>(Lu + ATT_Q8_VS)[r * 8 + (p >> 2)];
                float vd[8];
                att_row8<Q8>(vr, p, vs, vd);
                const f32x4 w0 = *reinterpret_cast<const LDS f32x4 *>(wgr + i * ATT_MAXG);
                const f32x4 w1 = *reinterpret_cast<const LDS f32x4 *>(wgr + i * ATT_MAXG + 4);
                const float w8[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
                for (uint32_t s = 0; s < 6; s++)
#pragma unroll
                    for (uint32_t dd = 0; dd < 8; dd++) acc[s][dd] = fmaf(w8[s], vd[dd], acc[s][dd]);
                if (gqa > 6) {
#pragma unroll
                    for (uint32_t s = 6; s < ATT_MAXG; s++)
#pragma unroll
                        for (uint32_t dd = 0; dd < 8; dd++) acc[s][dd] = fmaf(w8[s], vd[dd], acc[s][dd]);
                }
            }
        }
    }
    if (ts) ts[2] = wall_clock64();

    // the chunk's partial: the eight row groups merged per slot (through LDS,
    // in the tile region): M = max m_g, e_g = exp(m_g - M) (0 for a group
    // without rows), L and O fmaf chains over the groups ascending
    float *pbase = a.part + ((size_t)g * C + c) * gqa * PS;
    LDS float *comb = reinterpret_cast<LDS float *>(L);   // [8 rr][ATT_MAXG][256]
    LDS float *gm = wl + 8 * (4 * ATT_MAXG + ATT_MAXG);   // [8 rr][ATT_MAXG] m, then l
    __syncthreads();   // every wave done with the last tile's buffers
#pragma unroll
    for (uint32_t s = 0; s < ATT_MAXG; s++) {
        LDS float *d = comb + (rr * ATT_MAXG + s) * 256 + 8 * p;
        const f32x4 v0 = {acc[s][0], acc[s][1], acc[s][2], acc[s][3]};
        const f32x4 v1 = {acc[s][4], acc[s][5], acc[s][6], acc[s][7]};
        *reinterpret_cast<LDS f32x4 *>(d) = v0;
        *reinterpret_cast<LDS f32x4 *>(d + 4) = v1;
    }
    if (my_i == 0) {
        gm[rr * ATT_MAXG + my_s] = mrun;
        gm[8 * ATT_MAXG + rr * ATT_MAXG + my_s] = lrun;
    }
    __syncthreads();
    // each (row group, slot) weight e_g once: lane 8 g + s of wave 0 (in the
    // merge's weight array, unused until the merge); the slot's M at [64 + s]
    LDS float *ew = me;
    if (t < 64) {
        const uint32_t g2 = t >> 3, s = t & 7u;
        float M = -INFINITY;
#pragma unroll
        for (uint32_t k = 0; k < 8; k++) M = fmaxf(M, gm[k * ATT_MAXG + s]);
        const float mg = gm[g2 * ATT_MAXG + s];
        ew[g2 * ATT_MAXG + s] = (s < gqa && mg != -INFINITY) ? att_exp(mg - M) : 0.0f;
        if (g2 == 0) ew[64 + s] = M;
    }
    __syncthreads();
    {
        const uint32_t s = t >> 5, po = t & 31;
        const float M = ew[64 + s];
        float Lc = 0.0f, o[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (uint32_t g2 = 0; g2 < 8; g2++) {
            const float e = ew[g2 * ATT_MAXG + s];
            Lc = fmaf(e, gm[8 * ATT_MAXG + g2 * ATT_MAXG + s], Lc);
            const f32x4 c0 = *reinterpret_cast<const LDS f32x4 *>(comb + (g2 * ATT_MAXG + s) * 256 + 8 * po);
            const f32x4 c1 = *reinterpret_cast<const LDS f32x4 *>(comb + (g2 * ATT_MAXG + s) * 256 + 8 * po + 4);
            const float cv[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
#pragma unroll
            for (uint32_t dd = 0; dd < 8; dd++) o[dd] = fmaf(e, cv[dd], o[dd]);
        }
        if (s < gqa) {
            float *d = pbase + s * PS + 8 * po;
            st_coh4(d, make_float4(o[0], o[1], o[2], o[3]));
            st_coh4(d + 4, make_float4(o[4], o[5], o[6], o[7]));
            if (po == 0) {
                st_coh(pbase + s * PS + HD, M);
                st_coh(pbase + s * PS + HD + 1, Lc);
            }
        }
    }

    // the merge's element mapping: this workgroup finalises elements
    // [e0, e1) of the head group's gqa*HD outputs (slots s_lo .. s_hi)
    const uint32_t E = gqa * HD, NC = geo.n, ne = (E + NC - 1) / NC, e0 = c * ne, e1 = min(e0 + ne, E);

    // wait for the kv head's NC chunks: each publishes generation gen + 1 in
    // its own flag (one store, after its partial's stores completed) and
    // waits for all NC flags of the head
    settle_vmem();
    __syncthreads();
    if (t == 0) st_coh(a.count + rel, gen + 1u);
    if (t < 64) {
        const bool okw = att_wait_flags(a.count + g * C, NC, gen + 1u, spin_limit, err, ins.dbg_node);
        if (t == 0) *flag = okw ? 1u : 0u;
    }
    __syncthreads();
    if (*flag == 0) return;
    if (e0 >= e1) { settle_vmem(); return; }

    // merge: M = max_c m_c, e_c = exp(m_c - M), L = sum_c e_c l_c and
    // O = sum_c e_c acc_c as fmaf chains over the chunks ascending;
    // out = O / L * sigmoid(gate).  One load round trip: every value of the
    // workgroup's elements in every chunk (pair q = t, t + 256, .. of the
    // chunk-major (chunk, element) pairs), the m / l of every chunk for its
    // slots and the gates are loaded before any is used, then staged in LDS
    // (the tile region).
    const uint32_t nel = e1 - e0, s_lo = e0 / HD, nsl = (e1 - 1) / HD - s_lo + 1, npair = NC * nel;
    LDS float *mv = reinterpret_cast<LDS float *>(L);   // [NC][nel] values
    LDS float *mm = mv + npair;                         // [nsl][NC] m, then [nsl][NC] l
    LDS float *mw = mm + 2 * nsl * NC;                  // [nsl][NC] e_c, then [nsl] L
    const uint32_t pbytes = NC * gqa * PS * 4;   // (an offset of pbytes lies outside: loads 0, no access)
    const __amdgpu_buffer_rsrc_t r = coh_rsrc(a.part + (size_t)g * C * gqa * PS, pbytes);
    constexpr uint32_t MAXV = (ATT_MAXG * 256 + 64 + BLOCK_THREADS - 1) / BLOCK_THREADS;   // pairs per thread
    constexpr uint32_t MAXG = (ATT_MAXG * 256 + BLOCK_THREADS - 1) / BLOCK_THREADS;        // elements per thread
    float v[MAXV], ml[4], gt[MAXG];
#pragma unroll
    for (uint32_t k = 0; k < MAXV; k++) {
        const uint32_t q = t + k * BLOCK_THREADS, cq = q / nel, el = e0 + q % nel;
        const uint32_t off = q < npair ? ((cq * gqa + el / HD) * PS + el % HD) * 4 : pbytes;
        v[k] = ld_coh4b(r, off);
    }
#pragma unroll
    for (uint32_t k = 0; k < 2; k++) {
        const uint32_t q = t + k * BLOCK_THREADS, sl = q / NC, cq = q % NC;
        const uint32_t off = sl < nsl ? ((cq * gqa + s_lo + sl) * PS + HD) * 4 : pbytes;
        ml[2 * k] = ld_coh4b(r, off);
        ml[2 * k + 1] = ld_coh4b(r, off + 4);
    }
#pragma unroll
    for (uint32_t k = 0; k < MAXG; k++) {
        const uint32_t j = t + k * BLOCK_THREADS, el = e0 + min(j, nel - 1), h = g * gqa + el / HD;
        gt[k] = j < nel ? ld_coh(a.qg + (size_t)h * 2 * HD + HD + el % HD) : 0.0f;
    }
#pragma unroll
    for (uint32_t k = 0; k < MAXV; k++) {
        const uint32_t q = t + k * BLOCK_THREADS;
        if (q < npair) mv[q] = v[k];
    }
#pragma unroll
    for (uint32_t k = 0; k < 2; k++) {
        const uint32_t q = t + k * BLOCK_THREADS;
        if (q < nsl * NC) { mm[q] = ml[2 * k]; mm[nsl * NC + q] = ml[2 * k + 1]; }
    }
    __syncthreads();
    // per slot (wave sl % 4), lane k = chunk k: M, e_k, then the L chain
    for (uint32_t sl = w; sl < nsl; sl += WAVES) {
        const float m = lane < NC ? mm[sl * NC + lane] : -INFINITY;
        const float l = lane < NC ? mm[nsl * NC + sl * NC + lane] : 0.0f;
        float M = m;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
        const float e = lane < NC ? att_exp(m - M) : 0.0f;
        float Ls = 0.0f;
        for (uint32_t k = 0; k < NC; k++) {
            const float ek = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, e), (int)k));
            const float lk = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, l), (int)k));
            Ls = fmaf(ek, lk, Ls);
        }
        if (lane < NC) mw[sl * NC + lane] = e;
        if (lane == 0) mw[nsl * NC + sl] = Ls;
    }
    __syncthreads();
#pragma unroll
    for (uint32_t k = 0; k < MAXG; k++) {
        const uint32_t j = t + k * BLOCK_THREADS;
        if (j < nel) {
            const uint32_t el = e0 + j, sl = el / HD - s_lo, h = g * gqa + el / HD;
            const LDS float *ec = mw + sl * NC;
            float O = 0.0f;
            for (uint32_t cq = 0; cq < NC; cq++) O = fmaf(ec[cq], mv[cq * nel + j], O);
            st_coh(a.out + (size_t)h * HD + el % HD, (O / mw[nsl * NC + sl]) * dev_sigmoid(gt[k]));
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
