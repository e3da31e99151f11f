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
// the spin limit raises SINTER_E_TIMEOUT_BARRIER and returns, so a broken
// program ends the kernel instead of hanging the device.
#include <hip/hip_runtime.h>

#include <cstring>
#include <mutex>

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


}  // namespace sinter

using namespace sinter;

// The program's instruction headers, copied into LDS at launch (the first
// HDR_CAP; a longer program reads the rest with scalar loads): the program
// (256 B per instruction) is far larger than the scalar cache, so a header
// read from memory is an L2 round trip on the way to every op and barrier.
// (HDR_CAP is in isa.h)
__shared__ uint64_t g_hdr[HDR_CAP];

// The interpreter over feature set F (the GEMV weight / activation types and
// KV cache types its ops handle; isa.h): one kernel per set below.
template <uint32_t F>
__device__ __forceinline__ void interp_main(const sinter_instr *__restrict__ prog, const InterpCtl &ctl) {
    unsigned epoch = ctl.epoch0;
    const uint32_t n = ctl.n_instr;
    const bool timed = ctl.op_cycles && blockIdx.x == 0;
    // i in [0, n]: i == n is the pass-end barrier.  A barrier followed by a
    // GEMV this block takes part in runs as one op (gemv_op): the GEMV's
    // first weight slots are loaded between arriving and waiting, so the
    // barrier wait overlaps weight streaming; the pass end's successor is the
    // next pass's first instruction.  One copy of each op's code.
    uint32_t pass = 0, i = 0;
    uint64_t t0 = wall_clock64();
    for (uint32_t k = threadIdx.x; k < min(n, HDR_CAP); k += BLOCK_THREADS)
        g_hdr[k] = *(const GLB uint64_t *)&prog[k];
    auto hdr_at = [&](uint32_t k) -> uint64_t { return k < HDR_CAP ? g_hdr[k] : ins_hdr(prog[k]); };
    if (threadIdx.x == 0) {
        g_att_key[0] = ATT_NO_CACHE;   // no attention cache from an earlier launch
        // the launch's inputs into the pass cell: every workgroup stores the
        // same values and waits for its stores, so its own reads below see
        // them, and each workgroup's stores precede its first arrival
        if (ctl.cell_set & 1u) st_coh(&ctl.cell->token, ctl.cell_token);
        if (ctl.cell_set & 2u) st_coh(&ctl.cell->pos, ctl.cell_pos);
        if (ctl.cell_set & 4u) st_coh(&ctl.cell->steps, 0);
        settle_vmem();
    }
    __syncthreads();
    const bool traced = ctl.trace != nullptr;
    auto stamp = [&](uint32_t ii, uint32_t k, uint64_t v) {
        if (traced && pass == 0 && threadIdx.x == 0) ctl.trace[((size_t)ii * gridDim.x + blockIdx.x) * 4 + k] = v;
    };
    while (pass < ctl.n_passes) {
        const uint64_t hdr = i < n ? hdr_at(i) : 0u;
        const unsigned kind = i < n ? hdr_kind(hdr) : (unsigned)SINTER_OP_BOUNDARY;
        if (kind == SINTER_OP_BOUNDARY) {
            const bool pass_end = i == n;
            const uint32_t nx = pass_end ? 0u : i + 1;
            const bool more = nx < n && (pass + (pass_end ? 1u : 0u)) < ctl.n_passes;
            const uint64_t hnx = more ? hdr_at(nx) : 0u;
            const bool in_nx = more && blockIdx.x >= hdr_lo(hnx) && blockIdx.x < hdr_hi(hnx);
            const bool fused = in_nx && hdr_kind(hnx) == SINTER_OP_GEMV;
            const bool fused_gdn = in_nx && hdr_kind(hnx) == SINTER_OP_GDN_STEP;
            const uint64_t s = timed ? wall_clock64() : 0;
            GridCross gx;
            gx.flags = ctl.flags; gx.err = ctl.err; gx.epoch = &epoch;
            gx.spin_limit = ctl.spin_limit; gx.pass_end = pass_end; gx.t0 = t0; gx.t_wait_end = 0;
            gx.pass_slot = (pass_end && blockIdx.x == 0 && ctl.pass_cycles && ctl.pass_cycles_cap)
                               ? ctl.pass_cycles + (ctl.pass_base + pass) % ctl.pass_cycles_cap
                               : nullptr;
            if (fused) {
                uint64_t *ts = (traced && pass + (pass_end ? 1u : 0u) == 0 && threadIdx.x == 0)
                                   ? (uint64_t *)ctl.trace + ((size_t)nx * gridDim.x + blockIdx.x) * 4 : nullptr;
                if (ts) ts[0] = s ? s : wall_clock64();
                if (!gemv_op<F>(prog[nx], ctl.plans + nx, ctl.cuts + (size_t)nx * PLAN_CUTS, ctl.err, &gx, ts, hnx))
                    return;
                if (ts) ts[3] = wall_clock64();
            } else if (fused_gdn) {
                // the GDN step loads its state slice across the barrier; the
                // boundary's record keeps the arrival and the wait's end
                uint64_t *ts = (traced && pass + (pass_end ? 1u : 0u) == 0 && threadIdx.x == 0)
                                   ? (uint64_t *)ctl.trace + ((size_t)nx * gridDim.x + blockIdx.x) * 4 : nullptr;
                stamp(i, 0, wall_clock64());
                if (!op_gdn_step(prog[nx], ctl.err, ts, &gx)) return;
                stamp(i, 1, gx.t_wait_end);
                if (ts) { ts[0] = gx.t_wait_end; ts[3] = wall_clock64(); }
            } else {
                stamp(i, 0, wall_clock64());
                grid_arrive(ctl.flags, epoch);
                if (!grid_wait(ctl.flags, epoch, ctl.spin_limit, ctl.err)) { settle_vmem(); return; }
                gx.t_wait_end = wall_clock64();
                if (pass_end) {
                    // a uniform error sample after everyone finished the pass
                    __shared__ unsigned e;
                    if (threadIdx.x == 0) {
                        e = __hip_atomic_load(ctl.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        if (gx.pass_slot) *gx.pass_slot = (long long)(gx.t_wait_end - t0);
                    }
                    __syncthreads();
                    if (e) { settle_vmem(); return; }
                }
                stamp(i, 1, gx.t_wait_end);
            }
            if (timed && threadIdx.x == 0) {
                const uint64_t e = wall_clock64();
                ctl.op_cycles[SINTER_OP_BOUNDARY] += (long long)(gx.t_wait_end - s);
                if (fused) ctl.op_cycles[SINTER_OP_GEMV] += (long long)(e - gx.t_wait_end);
                if (fused_gdn) ctl.op_cycles[SINTER_OP_GDN_STEP] += (long long)(e - gx.t_wait_end);
            }
            const bool took_next = fused || fused_gdn;
            if (pass_end) {
                pass += 1;
                t0 = gx.t_wait_end;
                i = took_next ? 1u : 0u;
            } else {
                i += took_next ? 2u : 1u;
            }
            continue;
        }
        const sinter_instr &ins = prog[i];
        if (kind >= SINTER_OP_KIND_COUNT || !kind_wired(kind)) {
            if (blockIdx.x == 0 && threadIdx.x == 0)
                raise_error(ctl.err, kind >= SINTER_OP_KIND_COUNT ? SINTER_E_BAD_KIND : SINTER_E_UNWIRED_KIND, i);
            settle_vmem();
            return;
        }
        if (blockIdx.x >= hdr_lo(hdr) && blockIdx.x < hdr_hi(hdr)) {
            const uint64_t s = timed ? wall_clock64() : 0;
            stamp(i, 0, wall_clock64());
            if (kind == SINTER_OP_GEMV) {
                uint64_t *ts = (traced && pass == 0 && threadIdx.x == 0)
                                   ? (uint64_t *)ctl.trace + ((size_t)i * gridDim.x + blockIdx.x) * 4 : nullptr;
                (void)gemv_op<F>(ins, ctl.plans + i, ctl.cuts + (size_t)i * PLAN_CUTS, ctl.err, nullptr, ts, hdr);
            } else {
                uint64_t *ts = (traced && pass == 0 && threadIdx.x == 0)
                                   ? (uint64_t *)ctl.trace + ((size_t)i * gridDim.x + blockIdx.x) * 4 : nullptr;
                if (kind == SINTER_OP_GDN_STEP) (void)op_gdn_step(ins, ctl.err, ts, nullptr);
                else if (kind == SINTER_OP_ATTN_DECODE) op_attn_decode<F>(ins, ctl.err, ts, ctl.spin_limit, pass);
            }
            if (timed && threadIdx.x == 0) ctl.op_cycles[kind] += (long long)(wall_clock64() - s);
            stamp(i, 3, wall_clock64());
        }
        i += 1;
    }
    // every pass ran: the launch record (the last pass-end barrier put every
    // workgroup's cell and error stores before this)
    if (ctl.out && blockIdx.x == 0 && threadIdx.x == 0) {
        const unsigned e = __hip_atomic_load(ctl.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int tok = ld_coh(&ctl.cell->token), pos = ld_coh(&ctl.cell->pos);
        __hip_atomic_store(ctl.out + 1, (unsigned)tok, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        __hip_atomic_store(ctl.out + 2, (unsigned)pos, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        __hip_atomic_store(ctl.out + 3, e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        __hip_atomic_store(ctl.out, ctl.seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
        settle_vmem();
    }
}

extern "C" __global__ void __launch_bounds__(BLOCK_THREADS)
sinter_interp(const sinter_instr *__restrict__ prog, InterpCtl ctl) {
    interp_main<FEAT_ALL>(prog, ctl);
}
extern "C" __global__ void __launch_bounds__(BLOCK_THREADS)
sinter_interp_kquant(const sinter_instr *__restrict__ prog, InterpCtl ctl) {
    interp_main<FEAT_KQUANT>(prog, ctl);
}
extern "C" __global__ void __launch_bounds__(BLOCK_THREADS)
sinter_interp_kquant_q8kv(const sinter_instr *__restrict__ prog, InterpCtl ctl) {
    interp_main<FEAT_KQUANT_Q8KV>(prog, ctl);
}
extern "C" __global__ void __launch_bounds__(BLOCK_THREADS)
sinter_interp_bf16(const sinter_instr *__restrict__ prog, InterpCtl ctl) {
    interp_main<FEAT_BF16SET>(prog, ctl);
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
    case SINTER_OP_GEMV: (void)gemv_op<FEAT_ALL>(*ins, plan, cuts, err, nullptr, nullptr, ins_hdr(*ins)); break;
    case SINTER_OP_GDN_STEP: (void)op_gdn_step(*ins, err, nullptr, nullptr); break;
    // (attention launches cooperatively: its chunks of one kv head wait for
    // each other, bounded by a 2 s spin limit at 100 MHz)
    case SINTER_OP_ATTN_DECODE: op_attn_decode<FEAT_ALL>(*ins, err, nullptr, 200000000ull, ATT_NO_CACHE); break;
    default: break;
    }
}

// ---------------------------------------------------------------- no-allocation attention
// sinter_op_attn_decode_noalloc: the standalone attention op with its split-K
// partials, per-chunk generation flags and error cell in this file-scope
// device array instead of caller-allocated workspace.  Layout: error cell
// [0, 256) | flags [256, 256 + 4 * NOALLOC_FLAG_WORDS) | partials (fp32).
// Every call on a device shares the array; calls that overlap on one
// device race.
constexpr size_t NOALLOC_FLAG_WORDS = 1024;
constexpr size_t NOALLOC_PART_BYTES = 2u << 20;
constexpr size_t NOALLOC_FLAG_OFF = 256, NOALLOC_PART_OFF = NOALLOC_FLAG_OFF + NOALLOC_FLAG_WORDS * 4;
static __device__ __align__(256) unsigned char scratch[NOALLOC_PART_OFF + NOALLOC_PART_BYTES];

// p[0..n) = 0 (a kernel rather than a memset node, so a caller may capture it)
extern "C" __global__ void sinter_clear_u32(unsigned *p, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}

// The attention op with its instruction passed by value (nothing staged in
// device memory for it).
extern "C" __global__ void __launch_bounds__(BLOCK_THREADS) sinter_op_noalloc_kernel(sinter_instr ins, unsigned *err) {
    op_attn_decode<FEAT_ALL>(ins, err, nullptr, 200000000ull, ATT_NO_CACHE);
}

// ---------------------------------------------------------------- barrier litmus
// The grid barrier (grid_arrive / grid_wait) and the device-coherent data
// path under test (tests/litmus_boundary.cu in the reference).  Per epoch e,
// thread 0 of block b: a pseudo-random delay (so blocks complete in varying
// order), one device-scope atomic increment of the arrival count, then
// payload[b] = e, and (optionally) a read of the next block's payload line
// (that block runs on another XCD: workgroups are dealt to the XCDs in
// turn), which leaves last epoch's value wherever that read caches it.  After the barrier it
// reads block (b+1)%G's payload and the count: a payload older than e is a
// stale observation (a newer one is allowed: that block may already have
// crossed and published e + 1), a count below e*G an early release.
// Modes (sinter.h): COHERENT (sc1 store, sc1 load: the protocol the ops
// use), PLAIN_STORE (plain cached payload store), PLAIN_LOAD (plain cached
// payload load), LATE_PUBLISH (payload stored after arriving); bits 4-5 the
// pre-read (0 none, 1 plain, 2 sc1).  Every wait is the barrier's own bounded
// spin, so the kernel always exits.
constexpr uint32_t LITMUS_PLAIN_ST = SINTER_LITMUS_PLAIN_STORE, LITMUS_PLAIN_LD = SINTER_LITMUS_PLAIN_LOAD,
                   LITMUS_LATE = SINTER_LITMUS_LATE_PUBLISH;
constexpr uint32_t LITMUS_LINE = 64;   // payload stride in words (256 B)

__device__ __forceinline__ uint32_t litmus_hash(uint32_t x) {
    x ^= x >> 16; x *= 0x7feb352du; x ^= x >> 15; x *= 0x846ca68bu; x ^= x >> 16;
    return x;
}

extern "C" __global__ void __launch_bounds__(BLOCK_THREADS)
sinter_litmus_kernel(unsigned *flags, unsigned *err, unsigned *counter, unsigned *payload, unsigned *obs,
                     uint32_t epochs, uint32_t mode, uint64_t spin_limit, uint32_t seed) {
    unsigned epoch = 0;
    const uint32_t warm = (mode >> 4) & 3u;
    mode &= 15u;
    const uint32_t G = gridDim.x, b = blockIdx.x, rd = (b + 1) % G;
    unsigned *mine = payload + (size_t)b * LITMUS_LINE;
    const unsigned *theirs = payload + (size_t)rd * LITMUS_LINE;
    unsigned sink = 0, stale = 0, early = 0;
    for (uint32_t e = 1; e <= epochs; e++) {
        const uint32_t h = litmus_hash(seed ^ (b * 0x9E3779B9u) ^ (e * 0x85EBCA6Bu));
        if (threadIdx.x == 0) {
            const uint64_t until = wall_clock64() + (h & 31u);   // 0..0.31 us
            while (wall_clock64() < until) {}
            __hip_atomic_fetch_add(gp(counter), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (mode == LITMUS_PLAIN_ST) *gp(mine) = e;
            else if (mode != LITMUS_LATE) st_coh(mine, e);
            if (warm == 1) sink += *gp(theirs);   // warm the reader's caches with the old value
            else if (warm == 2) sink += ld_coh(theirs);
        }
        grid_arrive(flags, epoch);
        if (mode == LITMUS_LATE && threadIdx.x == 0) {
            const uint64_t until = wall_clock64() + 100u + ((h >> 8) & 255u);   // 1..3.5 us
            while (wall_clock64() < until) {}
            st_coh(mine, e);
        }
        if (!grid_wait(flags, epoch, spin_limit, err)) { settle_vmem(); return; }
        if (threadIdx.x == 0) {
            asm volatile("" ::: "memory");
            const unsigned v = mode == LITMUS_PLAIN_LD ? *gp(theirs) : ld_coh(theirs);
            const unsigned c = ld_coh(counter);
            // older than e is stale; newer is allowed (the writer may have
            // crossed already and published e + 1 before this read)
            stale += (int)(v - e) < 0 ? 1u : 0u;
            early += c < e * G ? 1u : 0u;
        }
    }
    if (threadIdx.x == 0) {
        __hip_atomic_fetch_add(gp(obs), stale, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_fetch_add(gp(obs + 1), early, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (sink == 0xFFFFFFFFu) st_coh(obs + 2, sink);   // keeps the warming reads
    }
    settle_vmem();
}

// Synthetic tensor fill: one thread per 256-element group (weights) or per
// element (f32 / f16 tensors).
extern "C" __global__ void sinter_synth_kernel(uint8_t *dst, int kind, int type, uint64_t n_units,
                                               uint64_t seed, float a, float b) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_units) return;
    if (kind == SINTER_SYN_WEIGHT || kind == SINTER_SYN_Q8_0_CFG1) {
        // written in place (a private staging array would live in scratch)
        sx_weight_group(seed, i, type, kind == SINTER_SYN_Q8_0_CFG1, dst + i * sx_group_bytes(type));
    } else if (kind == SINTER_SYN_NORMAL) {
        reinterpret_cast<float *>(dst)[i] = a + b * sx_normal(seed, i);
    } else if (kind == SINTER_SYN_UNIFORM) {
        reinterpret_cast<float *>(dst)[i] = a + (b - a) * sx_unit(seed, i);
    } else if (kind == SINTER_SYN_NORMAL_F16) {
        reinterpret_cast<uint16_t *>(dst)[i] = sx_f2h(b * sx_normal(seed, i));
    } else if (kind == SINTER_SYN_NORMAL_Q8_0) {
        sx_q8_0_normal_block(seed, i, b, dst + i * 34);
    }
}

// ----------------------------------------------------------------- launchers

namespace sinter {

hipError_t launch_op(const sinter_instr *ins_dev, const GemvPlan *plan, const uint32_t *cuts, uint32_t blocks,
                     unsigned *err, hipStream_t s, bool cooperative) {
    if (cooperative) {
        const sinter_instr *i = ins_dev;
        const GemvPlan *pl = plan;
        const uint32_t *cu = cuts;
        unsigned *e = err;
        void *args[] = {(void *)&i, (void *)&pl, (void *)&cu, (void *)&e};
        return hipLaunchCooperativeKernel((const void *)sinter_op_kernel, dim3(blocks), dim3(BLOCK_THREADS), args, 0, s);
    }
    hipLaunchKernelGGL(sinter_op_kernel, dim3(blocks), dim3(BLOCK_THREADS), 0, s, ins_dev, plan, cuts, err);
    return hipGetLastError();
}

// the smallest interpreter whose feature set covers `feat`
static const void *interp_kernel(uint32_t feat) {
    if ((feat & ~(uint32_t)FEAT_KQUANT) == 0) return (const void *)sinter_interp_kquant;
    if ((feat & ~(uint32_t)FEAT_KQUANT_Q8KV) == 0) return (const void *)sinter_interp_kquant_q8kv;
    if ((feat & ~(uint32_t)FEAT_BF16SET) == 0) return (const void *)sinter_interp_bf16;
    return (const void *)sinter_interp;
}

const char *interp_kernel_name(uint32_t feat) {
    const void *k = interp_kernel(feat);
    return k == (const void *)sinter_interp_kquant      ? "sinter_interp_kquant"
         : k == (const void *)sinter_interp_kquant_q8kv ? "sinter_interp_kquant_q8kv"
         : k == (const void *)sinter_interp_bf16        ? "sinter_interp_bf16"
                                                        : "sinter_interp";
}

hipError_t launch_interp(const sinter_instr *prog, const InterpCtl &ctl, uint32_t blocks, hipStream_t s,
                         uint32_t feat) {
    InterpCtl c = ctl;
    const sinter_instr *p = prog;
    void *args[] = {(void *)&p, (void *)&c};
    return hipLaunchCooperativeKernel(interp_kernel(feat), dim3(blocks), dim3(BLOCK_THREADS), args, 0, s);
}

// workgroups per CU every interpreter kernel can hold (the least of them)
hipError_t interp_max_blocks(int *blocks_per_cu) {
    int least = 1 << 30;
    for (const void *k : {(const void *)sinter_interp, (const void *)sinter_interp_kquant,
                          (const void *)sinter_interp_kquant_q8kv, (const void *)sinter_interp_bf16}) {
        int n = 0;
        const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k, BLOCK_THREADS, 0);
        if (e != hipSuccess) return e;
        least = n < least ? n : least;
    }
    *blocks_per_cu = least;
    return hipSuccess;
}

// Device address of `scratch` on the current device, looked up once per
// device (hipGetSymbolAddress with that device current) and kept: the
// array's name is not a device address in host code.
static std::mutex g_noalloc_mu;
static unsigned char *g_noalloc_ptr[64];

static unsigned char *noalloc_scratch(int *dev_out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
    if (dev_out) *dev_out = dev;
    std::lock_guard<std::mutex> lk(g_noalloc_mu);
    if (!g_noalloc_ptr[dev]) {
        void *p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return nullptr;
        g_noalloc_ptr[dev] = static_cast<unsigned char *>(p);
    }
    return g_noalloc_ptr[dev];
}

unsigned *noalloc_err_cell() {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
    std::lock_guard<std::mutex> lk(g_noalloc_mu);
    return reinterpret_cast<unsigned *>(g_noalloc_ptr[dev]);
}

int attn_noalloc(const sinter_attn_args &args, uint32_t blocks, hipStream_t s) {
    const size_t part_bytes = sinter_attn_part_len(args.nq, args.nkv, args.hd, args.n_chunks) * 4;
    const uint32_t flags = sinter_attn_count_len(args.nkv, args.n_chunks);
    if (part_bytes > NOALLOC_PART_BYTES || flags > NOALLOC_FLAG_WORDS)
        return set_error(SINTER_ERR_ARG,
                         "attn_noalloc: %zu B of partials and %u flags exceed the scratch maximum (%zu B, %zu flags)",
                         part_bytes, flags, NOALLOC_PART_BYTES, NOALLOC_FLAG_WORDS);
    unsigned char *p = noalloc_scratch(nullptr);
    if (!p) return set_error(SINTER_ERR_HIP, "attn_noalloc: hipGetSymbolAddress(scratch) failed");
    sinter_instr ins;
    std::memset(&ins, 0, sizeof ins);
    ins.kind = SINTER_OP_ATTN_DECODE;
    ins.block_lo = 0;
    ins.block_hi = (uint16_t)blocks;
    sinter_attn_args a = args;
    a.part = reinterpret_cast<float *>(p + NOALLOC_PART_OFF);
    a.count = reinterpret_cast<uint32_t *>(p + NOALLOC_FLAG_OFF);
    std::memcpy(ins.payload, &a, sizeof a);
    // every chunk starts the call at generation 0 (an earlier call may have
    // used another chunk split, leaving mixed generations in one head)
    hipLaunchKernelGGL(sinter_clear_u32, dim3((flags + 255) / 256), dim3(256), 0, s, a.count, flags);
    if (!hip_ok(hipGetLastError(), "attn_noalloc: flag clear")) return SINTER_ERR_HIP;
    unsigned *err = reinterpret_cast<unsigned *>(p);
    void *kargs[] = {(void *)&ins, (void *)&err};
    if (!hip_ok(hipLaunchCooperativeKernel((const void *)sinter_op_noalloc_kernel, dim3(blocks), dim3(BLOCK_THREADS),
                                           kargs, 0, s),
                "attn_noalloc: launch"))
        return SINTER_ERR_HIP;
    return SINTER_OK;
}

int litmus_barrier(uint32_t blocks, uint32_t epochs, uint32_t mode, uint64_t counts[3]) {
    int per_cu = 0, dev = 0, cus = 0;
    if (!hip_ok(hipGetDevice(&dev), "litmus: device") ||
        !hip_ok(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev), "litmus: CUs") ||
        !hip_ok(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, sinter_litmus_kernel, BLOCK_THREADS, 0),
                "litmus: occupancy"))
        return SINTER_ERR_HIP;
    if (blocks < 2 || blocks > 1024 || blocks > (uint32_t)(per_cu * cus) || (mode & 15u) > LITMUS_LATE ||
        ((mode >> 4) & 3u) > 2u || (mode & ~0x3Fu) || epochs == 0)
        return set_error(SINTER_ERR_ARG, "litmus: blocks %u (2..%d co-resident, <= 1024), mode %u, epochs %u", blocks,
                         per_cu * cus, mode, epochs);
    // [err 64 B | counter 64 B | observations 64 B | flags 4 KiB | payload lines]
    const size_t bytes = 192 + 4096 + (size_t)blocks * LITMUS_LINE * 4;
    unsigned char *buf = nullptr;
    if (!hip_ok(hipMalloc(&buf, bytes), "litmus: alloc")) return SINTER_ERR_HIP;
    int rc = SINTER_OK;
    unsigned *err = reinterpret_cast<unsigned *>(buf), *counter = err + 16, *obs = err + 32, *flags = err + 48;
    unsigned *payload = flags + 1024;
    uint64_t spin = 200000000ull;   // 2 s of wall clock ticks per barrier wait
    uint32_t seed = 0x5151u ^ mode;
    void *args[] = {&flags, &err, &counter, &payload, &obs, &epochs, &mode, &spin, &seed};
    unsigned h[34];
    if (!hip_ok(hipMemset(buf, 0, bytes), "litmus: clear") ||
        !hip_ok(hipLaunchCooperativeKernel((const void *)sinter_litmus_kernel, dim3(blocks), dim3(BLOCK_THREADS), args,
                                           0, nullptr),
                "litmus: launch") ||
        !hip_ok(hipDeviceSynchronize(), "litmus: run") ||
        !hip_ok(hipMemcpy(h, buf, sizeof h, hipMemcpyDeviceToHost), "litmus: read"))
        rc = SINTER_ERR_HIP;
    else if (h[0])
        rc = set_error(SINTER_ERR_DEVICE, "litmus: device error %u (aux %u)", h[0], h[1]);
    else {
        counts[0] = h[32];
        counts[1] = h[33];
        counts[2] = h[16];
    }
    (void)hipFree(buf);
    return rc;
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
