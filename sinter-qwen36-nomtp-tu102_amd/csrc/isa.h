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
// (4 wave64) per CU; all LDS is static (lds.h), 152 KiB of the CU's 160 KiB.
constexpr unsigned BLOCK_THREADS = 256;

// GEMV LDS: three 36 KiB weight-tile buffers filled by LDS-DMA, each wave
// issuing TILE_CPW 1 KiB chunks per tile; the quantised activation; the
// buffered row results.
constexpr unsigned TILE_BYTES = 36u * 1024u;
constexpr unsigned TILE_CPW = TILE_BYTES / 1024u / (BLOCK_THREADS / 64u);
constexpr unsigned QBUF_BYTES = 40u * 1024u;   // padded activation: Q8_K K=17408 20944 B; BF16 K=17408 39168 B
constexpr unsigned RES_CAP = 512u;             // rows buffered before the epilogue runs
constexpr unsigned CB_CAP = 776u;              // GEMV term ring (doubles): the rows of two tiles
                                               // of up to 256 item terms, padded (RING_PAD)
static_assert(TILE_CPW * 4u * 1024u == TILE_BYTES, "tile = whole chunks per wave");
// A term-ring row holds a row's item terms padded with -0.0 (an exact no-op
// in the fold) to a multiple of RING_PAD, so the fold reads whole 16-byte
// pairs in batches of RING_PAD with no masking -- or, when rows that long
// would not leave the ring room for the rows one tile touches (short rows,
// many per tile), to a multiple of 2.  cap = ring capacity in terms, tpr =
// rows one tile can touch, less one.
constexpr uint32_t RING_PAD = 8u;
__host__ __device__ inline uint32_t ring_row(uint32_t ipr, uint32_t cap, uint32_t tpr) {
    const uint32_t p8 = (ipr + RING_PAD - 1u) & ~(RING_PAD - 1u);
    return cap / p8 >= tpr + 1u ? p8 : ipr + (ipr & 1u);
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

// GEMV items: one 256-element group for the quantised types (one Q4_K /
// Q6_K block, eight Q8_0 blocks), 64 elements for BF16 / F32.
__host__ __device__ inline uint32_t item_elems(int t) { return (t == SINTER_BF16 || t == SINTER_F32) ? 64u : 256u; }
__host__ __device__ inline uint32_t item_bytes(int t) {
    return t == SINTER_Q4_K ? 144u : t == SINTER_Q6_K ? 210u : t == SINTER_Q8_0 ? 272u : t == SINTER_BF16 ? 128u : 256u;
}
// items of one matrix per tile: every lane busy, at most TILE_BYTES - 16
__host__ __device__ inline uint32_t items_per_tile(int t, bool swiglu) {
    const uint32_t n = (t == SINTER_Q4_K || t == SINTER_BF16) ? 256u : 128u;
    return swiglu ? n / 2 : n;
}

// A GEMV instruction compiled for the kernel: everything about its work split
// that depends only on the instruction, computed by the host when the program
// is uploaded (or a standalone op is launched), so that starting the op on
// the device is a few scalar loads instead of divisions and table builds.
struct GemvSegPlan {
    uint64_t wa, wb;                    // weights: A (gate rows for SwiGLU), B (up rows) or 0
    uint32_t rows, base;                // rows; global row of segment row 0
    uint32_t type, swig, ib, T, qT, rT; // item bytes; items of each matrix per tile; T / ipr; T % ipr
};
struct GemvPlan {
    uint32_t ok;                        // passed validation (otherwise the op raises BAD_SHAPE)
    uint32_t n_seg, ipr, vt, any_argmax, total_rows;
    // the term ring: P = ipr rounded up to RING_PAD, R rows of P terms,
    // mipr / mR = floor((2^32-1) / ipr or R), RP = R * P, defer = fold one tile late
    uint32_t mipr, P, R, mR, RP, defer;
    GemvSegPlan seg[SINTER_GEMV_MAX_SEG];
};
// Workgroup w of an op owns global rows [cuts[w], cuts[w+1]); each
// instruction has PLAN_CUTS cut slots.
constexpr uint32_t PLAN_MAX_BLOCKS = 1024;
constexpr uint32_t PLAN_CUTS = PLAN_MAX_BLOCKS + 1;

}  // namespace sinter
