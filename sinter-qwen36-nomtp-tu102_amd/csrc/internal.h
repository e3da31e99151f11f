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
    // launch inputs: every workgroup writes the fields cell_set names into
    // the pass cell before its first barrier (bit 0 token, bit 1 pos, bit 2
    // steps = 0; all write the same values)
    sinter_pass_cell *cell;
    int32_t cell_token, cell_pos;
    uint32_t cell_set;
    unsigned epoch0;          // barrier epoch the flags hold at the launch (0: zeroed flags)
    // launch record in host-visible memory, or null: [1] token, [2] pos, [3]
    // error code of the pass cell after the last pass, then [0] = seq; written
    // only by a launch that ran all its passes
    unsigned *out;
    uint32_t seq;
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
// the pass cell's token after the host's last launch (its launch record)
int32_t host_last_token(const sinter_host *h);
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

namespace sinter {

// the batched prefill's own kernels (prefill.hip), launched on s
hipError_t launch_embed_ubatch(const void *embd, int type, uint32_t E, const int32_t *tokens, uint32_t n_tok, float *x,
                               hipStream_t s);
// the GDN step over n_tok tokens; work: gdn_ubatch_work(...) floats
hipError_t launch_gdn_ubatch(const float *qkv, const float *alpha, const float *beta, const float *dt_bias,
                             const float *ssm_a, float *state, float *o, float *work, uint32_t hk, uint32_t hv,
                             uint32_t d, uint32_t n_tok, float eps, float scale, hipStream_t s);
size_t gdn_ubatch_work(uint32_t hk, uint32_t hv, uint32_t d, uint32_t n_tok);
hipError_t launch_attn_prep_ubatch(const float *qg, const float *k, const float *v, const float *q_norm,
                                   const float *k_norm, void *kc, void *vc, uint32_t kv_type, int32_t pos0,
                                   uint32_t n_tok, uint32_t nq, uint32_t nkv, uint32_t hd, uint32_t rope_dims,
                                   float theta_scale, float eps, float *qr, hipStream_t s);
// causal attention of n_tok queries at positions pos0.. over the cache, split
// per query as the decode splits it; part: attn_prefill_part(...) floats
hipError_t launch_attn_prefill(const float *qr, const float *qg, const void *kc, const void *vc, uint32_t kv_type,
                               int32_t pos0, uint32_t n_tok, uint32_t nq, uint32_t nkv, uint32_t hd,
                               uint32_t n_chunks, uint32_t chunk_min, float scale, float *part, float *out,
                               hipStream_t s);
size_t attn_prefill_part(uint32_t n_tok, uint32_t nq, uint32_t hd, uint32_t n_chunks);

}  // namespace sinter
