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
// (4 wave64) per CU, the whole 160 KiB LDS of the CU available to it.
constexpr unsigned BLOCK_THREADS = 256;
constexpr unsigned LDS_BYTES = 152u * 1024u;

// LDS map used by the GEMV op (bytes):
//   [0, 64)              reduction scratch (8 doubles)
//   [64, 64+QBUF)        quantised activation (int8 codes, scales, bsums)
//   then two weight tile buffers of TILE_BYTES each, then per-block terms.
constexpr unsigned RED_BYTES = 128;
constexpr unsigned QBUF_BYTES = 36u * 1024u;   // Q8_K K<=17408: 19856 B; BF16 K<=17408: 34816 B
constexpr unsigned TILE_BYTES = 52u * 1024u;
constexpr unsigned CB_BYTES = 256u * 8u;       // one fp64 term per (row, block) item
constexpr unsigned ROWV_BYTES = 256u * 4u;
static_assert(RED_BYTES + QBUF_BYTES + 2 * TILE_BYTES + CB_BYTES + ROWV_BYTES <= LDS_BYTES, "lds map");

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
