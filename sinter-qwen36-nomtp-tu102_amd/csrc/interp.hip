// The interpreter spine for gfx950 and the standalone op / synthesis kernels.
//
// sinter_interp is one cooperative grid (one 256-thread workgroup per CU)
// that walks the instruction array once per pass, crossing a grid barrier at
// every BOUNDARY and dispatching every other instruction whose
// [block_lo, block_hi) range holds the workgroup (core/interp.cu:39-146).
// A launch runs n_passes passes back to back; the greedy-argmax epilogue of
// the head GEMV advances the pass cell (token, pos) on device, so a greedy
// decode of many tokens needs no host round trip between tokens.
//
// Error protocol (core/interp.cuh:36-56): an unknown kind is seen by every
// workgroup at the same instruction, all return, no barrier is left half
// arrived.  Ops raise into the error cell and return normally; the cell is
// sampled after the pass-end barrier, uniformly.  A barrier wait that exceeds
// the spin limit raises SINTER_E_BAD_KIND+16 (timeout) and returns, so a
// broken program ends the kernel instead of hanging the device.
#include <hip/hip_runtime.h>

#include "internal.h"
#include "gemv.h"
#include "gdn.h"
#include "attn.h"
#include "synth.h"

namespace sinter {

__device__ __forceinline__ bool kind_wired(unsigned k) {
    return k == SINTER_OP_NOP || k == SINTER_OP_BOUNDARY || k == SINTER_OP_GEMV ||
           k == SINTER_OP_GDN_STEP || k == SINTER_OP_ATTN_DECODE;
}


// Grid barrier, two-level, over monotonic counters (zeroed before the
// launch): workgroup w counts into group counter w/16 (its own 128-byte
// line); the group's last arriver counts into the root; every workgroup's
// thread 0 spins on the root until epoch*groups arrivals.  Sixteen arrivals
// per line instead of the whole grid on one line (atomics to one address
// serialise at the memory side).  No cache writeback or invalidate: every
// wave first waits for its own memory operations, and all data that crosses
// workgroups moves through device-coherent loads and stores (dev_common.h).
// Split in two so that work that does not depend on the barrier (the next
// GEMV's first weight tiles) can be issued between arriving and waiting.
__device__ __forceinline__ void grid_arrive(unsigned *bar, unsigned *groups, unsigned &epoch) {
    settle_vmem();
    __syncthreads();
    epoch += 1;
    if (threadIdx.x == 0) {
        const unsigned g = blockIdx.x >> 4;
        const unsigned gsize = min(16u, gridDim.x - g * 16u);
        const unsigned old = __hip_atomic_fetch_add(groups + g * 32u, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old + 1u == epoch * gsize) __hip_atomic_fetch_add(bar, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Returns false on timeout.
__device__ __forceinline__ bool grid_wait(unsigned *bar, unsigned epoch, uint64_t spin_limit_ticks, unsigned *err) {
    __shared__ unsigned timed_out;
    if (threadIdx.x == 0) {
        timed_out = 0;
        const unsigned target = epoch * ((gridDim.x + 15u) >> 4);
        const uint64_t t0 = wall_clock64();
        while ((int)(atomic_load_relaxed_agent(bar) - target) < 0) {
            __builtin_amdgcn_s_sleep(1);
            if (wall_clock64() - t0 > spin_limit_ticks) {
                raise_error(err, SINTER_E_TIMEOUT_BARRIER, epoch);
                timed_out = 1;
                break;
            }
        }
    }
    __syncthreads();
    return timed_out == 0;
}


}  // namespace sinter

using namespace sinter;

extern "C" __global__ void __launch_bounds__(BLOCK_THREADS)
sinter_interp(const sinter_instr *__restrict__ prog, InterpCtl ctl) {
    unsigned epoch = 0;
    GemvState pf;                 // a GEMV begun before the barrier that precedes it
    uint32_t pf_i = 0xffffffffu;  // its instruction index
    const uint32_t n = ctl.n_instr;
    // one copy of each op's code in the kernel: the pass end is handled as a
    // barrier at index n, and every GEMV runs through gemv_begin + gemv_run
    for (uint32_t pass = 0; pass < ctl.n_passes; ++pass) {
        const uint64_t t0 = wall_clock64();
        for (uint32_t i = 0; i <= n; ++i) {
            const unsigned kind = i < n ? prog[i].kind : (unsigned)SINTER_OP_BOUNDARY;
            if (kind == SINTER_OP_BOUNDARY) {
                const uint64_t s = (ctl.op_cycles && blockIdx.x == 0) ? wall_clock64() : 0;
                grid_arrive(ctl.bar, ctl.groups, epoch);
                // begin the next GEMV (the next pass's first one at the pass end)
                const uint32_t nx = i + 1 < n ? i + 1 : (i == n && pass + 1 < ctl.n_passes ? 0u : 0xffffffffu);
                if (nx != 0xffffffffu) {
                    const sinter_instr &ni = prog[nx];
                    if (ni.kind == SINTER_OP_GEMV && blockIdx.x >= ni.block_lo && blockIdx.x < ni.block_hi) {
                        gemv_begin(ni, ctl.plans + nx, ctl.cuts + (size_t)nx * PLAN_CUTS, ctl.err, pf);
                        pf_i = nx;
                    }
                }
                if (!grid_wait(ctl.bar, epoch, ctl.spin_limit, ctl.err)) { settle_vmem(); return; }
                if (ctl.op_cycles && blockIdx.x == 0 && threadIdx.x == 0)
                    ctl.op_cycles[SINTER_OP_BOUNDARY] += (long long)(wall_clock64() - s);
                if (i < n) continue;
                // pass end: a uniform error sample after everyone finished
                __shared__ unsigned e;
                if (threadIdx.x == 0) e = __hip_atomic_load(ctl.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __syncthreads();
                if (blockIdx.x == 0 && threadIdx.x == 0 && ctl.pass_cycles && ctl.pass_cycles_cap)
                    ctl.pass_cycles[(ctl.pass_base + pass) % ctl.pass_cycles_cap] = (long long)(wall_clock64() - t0);
                if (e) { settle_vmem(); return; }
                continue;
            }
            const sinter_instr &ins = prog[i];
            if (kind >= SINTER_OP_KIND_COUNT || !kind_wired(kind)) {
                if (blockIdx.x == 0 && threadIdx.x == 0)
                    raise_error(ctl.err, kind >= SINTER_OP_KIND_COUNT ? SINTER_E_BAD_KIND : SINTER_E_UNWIRED_KIND, i);
                settle_vmem();
                return;
            }
            if (blockIdx.x >= ins.block_lo && blockIdx.x < ins.block_hi) {
                const uint64_t s = (ctl.op_cycles && blockIdx.x == 0) ? wall_clock64() : 0;
                if (kind == SINTER_OP_GEMV) {
                    if (pf_i != i) gemv_begin(ins, ctl.plans + i, ctl.cuts + (size_t)i * PLAN_CUTS, ctl.err, pf);
                    pf_i = 0xffffffffu;
                    gemv_run(ins, ctl.err, pf);
                } else if (kind == SINTER_OP_GDN_STEP) {
                    op_gdn_step(ins, ctl.err);
                } else if (kind == SINTER_OP_ATTN_DECODE) {
                    op_attn_decode(ins, ctl.err);
                }
                if (ctl.op_cycles && blockIdx.x == 0 && threadIdx.x == 0)
                    ctl.op_cycles[kind] += (long long)(wall_clock64() - s);
            }
        }
    }
}

// One instruction over the whole (non-cooperative) grid: the standalone op
// entry points.  The instruction sits in device memory like a program entry,
// so ops index its payload with ordinary loads.  Ops that need cross-block results use last-arriver counters,
// never a grid barrier, so co-residency is not required here.
extern "C" __global__ void __launch_bounds__(BLOCK_THREADS)
sinter_op_kernel(const sinter_instr *__restrict__ ins, const GemvPlan *__restrict__ plan,
                 const uint32_t *__restrict__ cuts, unsigned *err) {
    // the host sets block_lo = 0, block_hi = gridDim.x
    switch (ins->kind) {
    case SINTER_OP_GEMV: op_gemv(*ins, plan, cuts, err); break;
    case SINTER_OP_GDN_STEP: op_gdn_step(*ins, err); break;
    case SINTER_OP_ATTN_DECODE: op_attn_decode(*ins, err); break;
    default: break;
    }
}

// Synthetic tensor fill: one thread per 256-element group (weights) or per
// element (f32 / f16 tensors).
extern "C" __global__ void sinter_synth_kernel(uint8_t *dst, int kind, int type, uint64_t n_units,
                                               uint64_t seed, float a, float b) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_units) return;
    if (kind == SINTER_SYN_WEIGHT || kind == SINTER_SYN_Q8_0_CFG1) {
        const uint32_t gb = sx_group_bytes(type);
        uint8_t tmp[1024];
        sx_weight_group(seed, i, type, kind == SINTER_SYN_Q8_0_CFG1, tmp);
        for (uint32_t k = 0; k < gb; k++) dst[i * gb + k] = tmp[k];
    } else if (kind == SINTER_SYN_NORMAL) {
        reinterpret_cast<float *>(dst)[i] = a + b * sx_normal(seed, i);
    } else if (kind == SINTER_SYN_UNIFORM) {
        reinterpret_cast<float *>(dst)[i] = a + (b - a) * sx_unit(seed, i);
    } else if (kind == SINTER_SYN_NORMAL_F16) {
        reinterpret_cast<uint16_t *>(dst)[i] = sx_f2h(b * sx_normal(seed, i));
    }
}

// ----------------------------------------------------------------- launchers

namespace sinter {

hipError_t launch_op(const sinter_instr *ins_dev, const GemvPlan *plan, const uint32_t *cuts, uint32_t blocks,
                     unsigned *err, hipStream_t s) {
    hipLaunchKernelGGL(sinter_op_kernel, dim3(blocks), dim3(BLOCK_THREADS), 0, s, ins_dev, plan, cuts, err);
    return hipGetLastError();
}

hipError_t launch_interp(const sinter_instr *prog, const InterpCtl &ctl, uint32_t blocks, hipStream_t s) {
    InterpCtl c = ctl;
    const sinter_instr *p = prog;
    void *args[] = {(void *)&p, (void *)&c};
    return hipLaunchCooperativeKernel((const void *)sinter_interp, dim3(blocks), dim3(BLOCK_THREADS), args, 0, s);
}

hipError_t interp_max_blocks(int *blocks_per_cu) {
    return hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, (const void *)sinter_interp,
                                                        BLOCK_THREADS, 0);
}

hipError_t launch_synth(void *dst, int kind, int type, uint64_t n_units, uint64_t seed, float a, float b,
                        hipStream_t s) {
    if (n_units == 0) return hipSuccess;
    const uint32_t tpb = 256;
    const uint64_t nb = (n_units + tpb - 1) / tpb;
    hipLaunchKernelGGL(sinter_synth_kernel, dim3((uint32_t)nb), dim3(tpb), 0, s, (uint8_t *)dst, kind, type,
                       n_units, seed, a, b);
    return hipGetLastError();
}

}  // namespace sinter
