// The interpreter ISA as seen by the kernels: the public ABI structs plus the
// launch envelope.  The structs themselves live in include/sinter.h because
// they are the contract between the program packer (model.cpp), callers that
// build programs by hand, and the ops (core/isa.cuh:32-88 in the reference).
#pragma once
#include <hip/hip_runtime.h>

#include "../../include/sinter.h"

static_assert(sizeof(sinter_instr) == 256, "instruction size is part of the ABI");
static_assert(sizeof(sinter_gemv_args) <= 240, "gemv payload");
static_assert(sizeof(sinter_gdn_args) <= 240, "gdn payload");
static_assert(sizeof(sinter_attn_args) <= 240, "attn payload");
static_assert(sizeof(sinter_gemv_seg) == 40, "gemv segment");

namespace sinter {

// Launch envelope of the cooperative interpreter: one 256-thread workgroup
// (4 wave64) per CU; all LDS is static (dev_common.h).
constexpr unsigned BLOCK_THREADS = 256;
constexpr unsigned WAVES = BLOCK_THREADS / 64u;

// Interpreter specialisations.  One interpreter kernel is compiled per set of
// GEMV weight types, GEMV activation (vec_dot) types and KV cache types; the
// code of the ops' cases outside the set is left out of it.  At upload the
// host computes the set a program uses and launches the smallest kernel
// that covers it (the persistent kernel's code is fetched anew by every
// phase, and the specialised kernel decodes the 27B Q4_K_M model ~2 %
// faster than the general one).
enum : uint32_t {
    FEAT_W_Q4K = 1u << 0, FEAT_W_Q6K = 1u << 1, FEAT_W_Q80 = 1u << 2, FEAT_W_BF16 = 1u << 3, FEAT_W_F32 = 1u << 4,
    FEAT_X_Q8K = 1u << 5, FEAT_X_Q80 = 1u << 6, FEAT_X_BF16 = 1u << 7, FEAT_X_F32 = 1u << 8,
    FEAT_KV_F16 = 1u << 9, FEAT_KV_Q80 = 1u << 10,
    FEAT_ALL = (1u << 11) - 1u,
    // K-quant weights, Q8_K activations, f16 KV cache (the Q4_K_M decode)
    FEAT_KQUANT = FEAT_W_Q4K | FEAT_W_Q6K | FEAT_X_Q8K | FEAT_KV_F16,
    // the same over a Q8_0 KV cache
    FEAT_KQUANT_Q8KV = FEAT_W_Q4K | FEAT_W_Q6K | FEAT_X_Q8K | FEAT_KV_Q80,
    // bf16 weights and activations, f16 KV cache
    FEAT_BF16SET = FEAT_W_BF16 | FEAT_X_BF16 | FEAT_KV_F16,
};
// the feature bit of a GEMV weight type / activation type (0 for a type no
// op handles) / KV cache type
__host__ __device__ constexpr uint32_t feat_w(uint32_t t) {
    return t == SINTER_Q4_K ? FEAT_W_Q4K : t == SINTER_Q6_K ? FEAT_W_Q6K : t == SINTER_Q8_0 ? FEAT_W_Q80
         : t == SINTER_BF16 ? FEAT_W_BF16 : t == SINTER_F32 ? FEAT_W_F32 : 0u;
}
__host__ __device__ constexpr uint32_t feat_x(uint32_t vt) {
    return vt == SINTER_Q8_K ? FEAT_X_Q8K : vt == SINTER_Q8_0 ? FEAT_X_Q80 : vt == SINTER_BF16 ? FEAT_X_BF16
         : vt == SINTER_F32 ? FEAT_X_F32 : 0u;
}
// (kv_type 0 is the f16 cache, as SINTER_F16)
__host__ __device__ constexpr uint32_t feat_kv(uint32_t t) { return t == SINTER_Q8_0 ? FEAT_KV_Q80 : FEAT_KV_F16; }

// The interpreter's LDS table of instruction headers (interp.hip): entries.
constexpr uint32_t HDR_CAP = 1024;

// LDS: the quantised GEMV activation, and one 96 KiB scratch region shared by
// the ops: the GEMV's activation staging (prologue) and then its per-wave
// item-term rings; attention's tiles; the GDN step's vectors.
constexpr unsigned QBUF_BYTES = 40u * 1024u;   // padded activation: Q8_K K=17408 20944 B; BF16 K=17408 39168 B
constexpr unsigned BIG_BYTES = 96u * 1024u;
constexpr unsigned ATT_REGION = 36u * 1024u;   // attention: three regions at 0, 36 and 72 KiB
// GEMV item-term ring of one wave, in doubles (8 KiB; a SwiGLU pair splits
// it into a gate half and an up half)
constexpr uint32_t RING_CAP = 1024u;
// the deepest weight prefetch of any item type (items in flight per lane):
// the ring must hold the rows one group of that many steps touches
constexpr uint32_t GEMV_DMAX = 4u;
static_assert(WAVES * RING_CAP * 8u <= BIG_BYTES, "rings fit the scratch region");
// A term-ring row holds a row's item terms padded with -0.0 (an exact no-op
// in the fold) to a multiple of RING_PAD, so the fold reads whole 16-byte
// pairs in batches of RING_PAD with no masking -- or, when rows that long
// would not leave the ring room for the rows one 64-item step touches (short
// rows), to a multiple of 2.  cap = ring capacity in terms, tpr = rows one
// step can touch, plus one.
constexpr uint32_t RING_PAD = 8u;
__host__ __device__ inline uint32_t ring_row(uint32_t ipr, uint32_t cap, uint32_t tpr) {
    const uint32_t p8 = (ipr + RING_PAD - 1u) & ~(RING_PAD - 1u);
    return cap / p8 >= tpr ? p8 : ipr + (ipr & 1u);
}

// GEMV activation layout in LDS.  Padded so that lanes working on different
// groups/chunks start on different LDS banks (an unpadded 256-byte group
// stride puts every group on bank 0 and serialises the activation reads):
//   Q8_K: int8 codes, group g at g*ACT_GSTRIDE | d f32[G] | (16-aligned) bsums i16[16G]
//   Q8_0: int8 codes, group g at g*ACT_GSTRIDE | d f32[K/32] (f16-rounded)
//   BF16: 64-element chunk c at c*ACT_BF_CSTRIDE (u16)
//   F32:  64-element chunk c at c*ACT_F_CSTRIDE
constexpr uint32_t ACT_GSTRIDE = 272;
constexpr uint32_t ACT_BF_CSTRIDE = 144;
constexpr uint32_t ACT_F_CSTRIDE = 272;
__host__ __device__ inline uint32_t act_bs_off(uint32_t K) {
    return (K / 256) * ACT_GSTRIDE + (((K / 256) * 4 + 15u) & ~15u);
}
__host__ __device__ inline uint32_t act_bytes(int vt, uint32_t K) {
    if (vt == SINTER_Q8_K) return act_bs_off(K) + (K / 16) * 2;
    if (vt == SINTER_Q8_0) return (K / 256) * ACT_GSTRIDE + (K / 32) * 4;
    if (vt == SINTER_BF16) return (K / 64) * ACT_BF_CSTRIDE;
    return (K / 64) * ACT_F_CSTRIDE;
}

// bytes of one row of k elements of a ggml type
__host__ __device__ inline size_t sinter_row_bytes_dev(int t, int64_t k) {
    switch (t) {
    case SINTER_F32: return (size_t)k * 4;
    case SINTER_F16: case SINTER_BF16: return (size_t)k * 2;
    case SINTER_Q8_0: return (size_t)(k / 32) * 34;
    case SINTER_Q4_K: return (size_t)(k / 256) * 144;
    case SINTER_Q6_K: return (size_t)(k / 256) * 210;
    case SINTER_Q8_K: return (size_t)(k / 256) * 292;
    default: return 0;
    }
}

// Split-K geometry of decode attention over n_kv >= 1 positions and at most
// C >= 1 chunks of whole 32-position tiles, each at least chunk_min
// positions long: T tiles, tpc tiles per chunk, n (1 <= n <= C) non-empty
// chunks; chunk c covers tiles [c*tpc, min((c+1)*tpc, T)).
struct AttGeom { uint32_t tiles, tpc, n; };
__host__ __device__ inline AttGeom att_geom(uint32_t n_kv, uint32_t C, uint32_t chunk_min) {
    AttGeom g;
    g.tiles = (n_kv + 31u) / 32u;
    const uint32_t a = (g.tiles + C - 1u) / C, b = (chunk_min + 31u) / 32u;
    g.tpc = a > b ? a : b;
    if (g.tpc == 0) g.tpc = 1;
    g.n = (g.tiles + g.tpc - 1u) / g.tpc;
    return g;
}
// fp32 elements of one partial record (acc[hd], max, sum; 16-byte aligned)
__host__ __device__ inline uint32_t att_rec(uint32_t hd) { return hd + 4u; }

// GEMV items: one 256-element group for the quantised types (one Q4_K /
// Q6_K block, eight Q8_0 blocks), 64 elements for BF16 / F32.
__host__ __device__ inline uint32_t item_elems(int t) { return (t == SINTER_BF16 || t == SINTER_F32) ? 64u : 256u; }
__host__ __device__ inline uint32_t item_bytes(int t) {
    return t == SINTER_Q4_K ? 144u : t == SINTER_Q6_K ? 210u : t == SINTER_Q8_0 ? 272u : t == SINTER_BF16 ? 128u : 256u;
}
// 16-byte loads that bring one item into registers (Q6_K: a 4-aligned
// 224-byte window around the 2-aligned 210-byte block)
__host__ __device__ inline uint32_t item_loads(int t) {
    return t == SINTER_Q4_K ? 9u : t == SINTER_Q6_K ? 14u : t == SINTER_Q8_0 ? 17u : t == SINTER_BF16 ? 8u : 16u;
}

// A GEMV instruction compiled for the kernel: everything about its work split
// that depends only on the instruction, computed by the host when the program
// is uploaded (or a standalone op is launched), so that starting the op on
// the device is a few scalar loads instead of divisions and table builds.
struct GemvSegPlan {
    uint64_t wa, wb;                    // weights: A (gate rows for SwiGLU), B (up rows) or 0
    uint64_t y, aux, w2;                // the segment's epilogue operands (sinter_gemv_seg)
    uint32_t rows, base;                // rows; global row of segment row 0
    uint32_t type, swig, ib;            // weight type; SwiGLU pair; item bytes
    uint32_t epi, dconv, _pad;          // epilogue mode, conv taps
};
struct GemvPlan {
    uint32_t ok;                        // passed validation (otherwise the op raises BAD_SHAPE)
    uint32_t feat;                      // feature bits of its activation and weight types
    uint32_t n_seg, ipr, vt, any_argmax, total_rows;
    uint32_t mipr;                      // floor((2^32-1) / ipr)
    // the term ring of a wave: R rows of P terms (per matrix); mR = floor((2^32-1) / R)
    uint32_t P, R, mR;
    uint32_t q64, r64;                  // 64 / ipr, 64 % ipr: one 64-item step in rows + items
    uint32_t q32, r32;                  // the same for a 32-item step (SwiGLU pairs)
    GemvSegPlan seg[SINTER_GEMV_MAX_SEG];
};
// a GEMV's loads past the end of its rows read the plan instead: it must
// cover the largest item load (272 B)
static_assert(sizeof(GemvPlan) >= 272, "plan doubles as the dummy load target");
// Wave v of an op (v = 4 * (block - block_lo) + wave) owns global rows
// [cuts[v], cuts[v+1]); each instruction has PLAN_CUTS cut slots.
constexpr uint32_t PLAN_MAX_BLOCKS = 1024;
constexpr uint32_t PLAN_CUTS = PLAN_MAX_BLOCKS * WAVES + 1;

}  // namespace sinter
