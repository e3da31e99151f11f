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
constexpr unsigned CB_CAP = 512u;              // item terms of one tile (rows of up to 512 items)
static_assert(TILE_CPW * 4u * 1024u == TILE_BYTES, "tile = whole chunks per wave");

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

}  // namespace sinter
