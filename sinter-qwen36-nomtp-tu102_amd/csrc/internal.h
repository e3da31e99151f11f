// Declarations shared by the kernel TU (interp.hip) and the host TUs
// (host.cpp, model.cpp).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "isa.h"

namespace sinter {

// Kernel-side control block of one interpreter launch (core/interp.cuh:60-75)
struct InterpCtl {
    unsigned *flags;          // grid barrier flags, one word per workgroup, zeroed before the launch
    unsigned *err;            // [0] code, [1] aux
    long long *pass_cycles;   // ring of per-pass durations (wall clock ticks), or null
    long long *op_cycles;     // per-kind durations on block 0, or null
    unsigned long long *trace;  // [n_instr + 1][blocks][4] wall clock stamps of the launch's first pass, or null
    uint64_t spin_limit;      // barrier spin limit in wall clock ticks
    const GemvPlan *plans;    // [n_instr], GEMV entries filled
    const uint32_t *cuts;     // [n_instr][PLAN_CUTS]
    uint32_t n_instr;
    uint32_t n_passes;
    uint32_t pass_cycles_cap;
    uint32_t pass_base;
};

hipError_t launch_op(const sinter_instr *ins_dev, const GemvPlan *plan, const uint32_t *cuts, uint32_t blocks,
                     unsigned *err, hipStream_t s, bool cooperative);
// the interpreter kernel whose feature set (isa.h) covers feat: the
// K-quant or bf16 specialisation when one does, else the general one
hipError_t launch_interp(const sinter_instr *prog, const InterpCtl &ctl, uint32_t blocks, hipStream_t s,
                         uint32_t feat);
const char *interp_kernel_name(uint32_t feat);
hipError_t interp_max_blocks(int *blocks_per_cu);
hipError_t launch_synth(void *dst, int kind, int type, uint64_t n_units, uint64_t seed, float a, float b,
                        hipStream_t s);

// host-side helpers (host.cpp)
int set_error(int status, const char *fmt, ...);
bool hip_ok(hipError_t e, const char *what);
unsigned *op_err_cell();  // per-device error cell of the standalone op launches
// the no-allocation attention op (interp.hip): validate sizes, launch on s
int attn_noalloc(const sinter_attn_args &a, uint32_t blocks, hipStream_t s);
// its error cell on the current device (null before its first call there)
unsigned *noalloc_err_cell();
// the grid-barrier litmus (sinter_litmus_barrier)
int litmus_barrier(uint32_t blocks, uint32_t epochs, uint32_t mode, uint64_t counts[3]);
int validate_gemv(const sinter_gemv_args &a, const char **why);
// the plan and the nblk + 1 row cuts of a validated GEMV run by nblk workgroups
// bw: per-block work weights (null: uniform)
void build_gemv_plan(const sinter_gemv_args &a, uint32_t nblk, GemvPlan &p, uint32_t *cuts, const uint32_t *bw);

}  // namespace sinter
