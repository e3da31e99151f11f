// Device-side building blocks shared by every op family: wave64 reductions,
// agent-scope (cross-XCD) loads/stores and fences, f16/bf16 conversions and
// the activation-quantiser arithmetic.
//
// Coherence on gfx950: each of the 8 XCDs has its own L2.  Data that one
// workgroup writes and another reads later in the pass moves through
// device-coherent loads and stores (below), ordered by the grid barrier's
// counter.  Weights are immutable and use plain (non-temporal) loads.
#pragma once
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "isa.h"

namespace sinter {

typedef __attribute__((address_space(3))) void lds_void;
// Explicit LDS (address space 3) pointers: a generic pointer into LDS makes
// the compiler emit flat loads, which also count against vmcnt and so wait
// for every in-flight LDS-DMA load.
#define LDS __attribute__((address_space(3)))
// Explicit global (address space 1) pointers for the same reason: flat
// instructions also count against lgkmcnt, so every LDS wait after a flat
// global access would wait for it too.
#define GLB __attribute__((address_space(1)))
template <class T>
__device__ __forceinline__ GLB T *gp(T *p) { return (GLB T *)p; }
template <class T>
__device__ __forceinline__ const GLB T *gp(const T *p) { return (const GLB T *)p; }
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef LDS char lds_char;

// ---------------------------------------------------------------- static LDS
// g_big: scratch shared by the ops (GEMV staging then term rings, attention
// tiles, GDN vectors); g_qbuf: the quantised GEMV activation.
__shared__ __attribute__((aligned(16))) char g_big[BIG_BYTES];
__shared__ __attribute__((aligned(16))) char g_qbuf[QBUF_BYTES];
__shared__ double g_red[16];
__shared__ double g_part[16];
// the running op's payload, copied out of the program once per op so that
// reading it is an LDS access rather than a global one
__shared__ __attribute__((aligned(16))) unsigned char g_args[240];

// ---------------------------------------------------------------- wave64

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
// The thread index behind an empty asm: the interpreter runs every op inside
// one persistent loop, and values an op derives from a plain threadIdx.x
// (LDS addresses, lane permutations) are loop-invariant, so the compiler
// hoists them all to the kernel entry and keeps them live -- in registers,
// or in scratch -- for the whole kernel.  Derived from tid() they are
// recomputed by each op invocation instead.
__device__ __forceinline__ uint32_t tid() {
    uint32_t t = threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }

__device__ __forceinline__ float wave_max_f32(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ int wave_sum_i32(int v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// ---------------------------------------------------------------- DPP rows
// In-VALU lane exchanges within a 16-lane row (no LDS round trip).  Every
// lane of the row must be active.  After the four steps of row16_* every lane
// of the row holds the same value: each step combines a lane with its
// partner in a commutative operation, so partners compute identical results.
enum : int {
    DPP_XOR1 = 0xB1,         // quad_perm [1,0,3,2]
    DPP_XOR2 = 0x4E,         // quad_perm [2,3,0,1]
    DPP_HALF_MIRROR = 0x141, // lane i <- lane 7-i within each half-row
    DPP_MIRROR = 0x140,      // lane i <- lane 15-i within the row
};
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) { return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, false); }
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) { return __int_as_float(dpp_i<CTRL>(__float_as_int(v))); }
template <int CTRL>
__device__ __forceinline__ double dpp_d(double v) {
    const uint64_t u = __double_as_longlong(v);
    const uint32_t lo = (uint32_t)dpp_i<CTRL>((int)(uint32_t)u), hi = (uint32_t)dpp_i<CTRL>((int)(uint32_t)(u >> 32));
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, dpp_f<DPP_XOR1>(v));
    v = fmaxf(v, dpp_f<DPP_XOR2>(v));
    v = fmaxf(v, dpp_f<DPP_HALF_MIRROR>(v));
    return fmaxf(v, dpp_f<DPP_MIRROR>(v));
}
__device__ __forceinline__ float row16_minf(float v) {
    v = fminf(v, dpp_f<DPP_XOR1>(v));
    v = fminf(v, dpp_f<DPP_XOR2>(v));
    v = fminf(v, dpp_f<DPP_HALF_MIRROR>(v));
    return fminf(v, dpp_f<DPP_MIRROR>(v));
}
__device__ __forceinline__ int row16_min(int v) {
    v = min(v, dpp_i<DPP_XOR1>(v));
    v = min(v, dpp_i<DPP_XOR2>(v));
    v = min(v, dpp_i<DPP_HALF_MIRROR>(v));
    return min(v, dpp_i<DPP_MIRROR>(v));
}
__device__ __forceinline__ double row16_sum_f64(double v) {
    v += dpp_d<DPP_XOR1>(v);
    v += dpp_d<DPP_XOR2>(v);
    v += dpp_d<DPP_HALF_MIRROR>(v);
    return v + dpp_d<DPP_MIRROR>(v);
}
__device__ __forceinline__ double readlane_f64(double v, int lane) {
    const uint64_t u = __double_as_longlong(v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, lane);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), lane);
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// Block-wide fp64 sum over a 256-thread workgroup (every thread active;
// the wave count is the constant WAVES, not blockDim.x, whose read is a
// vector load from the dispatch's implicit arguments); every thread gets the
// same total.  `red` is LDS scratch of >= 16
// doubles.  Rows are reduced with DPP, the four row sums of a wave and then
// the wave sums are added in a fixed order; the result is order-dependent
// only at fp64 rounding level (callers round to fp32).
template <class P>
__device__ __forceinline__ double block_sum_f64(double v, P red) {
    v = row16_sum_f64(v);
    const double w = ((readlane_f64(v, 0) + readlane_f64(v, 16)) + readlane_f64(v, 32)) + readlane_f64(v, 48);
    constexpr int nw = (int)WAVES;
    __syncthreads();
    if (lane_id() == 0) red[wave_id()] = w;
    __syncthreads();
    double t = 0.0;
    for (int i = 0; i < nw; i++) t += red[i];
    __syncthreads();
    return t;
}

// Two block sums at once (the same fold as block_sum_f64 for each).
template <class P>
__device__ __forceinline__ void block_sum2_f64(double &a, double &b, P red) {
    a = row16_sum_f64(a);
    b = row16_sum_f64(b);
    const double wa = ((readlane_f64(a, 0) + readlane_f64(a, 16)) + readlane_f64(a, 32)) + readlane_f64(a, 48);
    const double wb = ((readlane_f64(b, 0) + readlane_f64(b, 16)) + readlane_f64(b, 32)) + readlane_f64(b, 48);
    constexpr int nw = (int)WAVES;
    __syncthreads();
    if (lane_id() == 0) { red[2 * wave_id()] = wa; red[2 * wave_id() + 1] = wb; }
    __syncthreads();
    double ta = 0.0, tb = 0.0;
    for (int i = 0; i < nw; i++) { ta += red[2 * i]; tb += red[2 * i + 1]; }
    __syncthreads();
    a = ta;
    b = tb;
}

// Sum over aligned groups of n lanes (n a power of two, 1..64), every lane of
// a group getting the group's sum: the butterfly a[t] += a[t ^ m], m = 1, 2,
// 4, ..., n/2 (after the step at distance m every lane holds the sum of its
// aligned group of 2m lanes; the partner order does not matter, an fp32 add
// commutes exactly).  Within a 16-lane row the steps at distance 4 and 8 use
// the half-row and row mirrors (the partner holds the same partial sum as the
// lane at distance 4 / 8 once the smaller steps are done, so the sums are
// bit-identical); wider steps use cross-lane shuffles.
__device__ __forceinline__ float lanes_sum_f32(float v, uint32_t n) {
    if (n >= 2) v += dpp_f<DPP_XOR1>(v);
    if (n >= 4) v += dpp_f<DPP_XOR2>(v);
    if (n >= 8) v += dpp_f<DPP_HALF_MIRROR>(v);
    if (n >= 16) v += dpp_f<DPP_MIRROR>(v);
    if (n >= 32) v += __shfl_xor(v, 16, 64);
    if (n >= 64) v += __shfl_xor(v, 32, 64);
    return v;
}

// ---------------------------------------------------------------- conversions

__device__ __forceinline__ float h2f(uint16_t h) {
    return __half2float(__ushort_as_half(h));
}
__device__ __forceinline__ uint16_t f2h(float f) {  // round to nearest even
    return __half_as_ushort(__float2half_rn(f));
}
__device__ __forceinline__ float bf2f(uint16_t h) {
    return __uint_as_float((uint32_t)h << 16);
}
// ggml FP32->BF16: quiet NaN, otherwise round half to even
__device__ __forceinline__ uint16_t f2bf(float f) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 64);
    return (uint16_t)((u + (0x7fffu + ((u >> 16) & 1u))) >> 16);
}

// ggml silu/sigmoid/softplus in fp32 with the exponential evaluated in fp64
// and rounded once (the declared transcendental rule).
__device__ __forceinline__ float dev_silu(float x) { return x / (1.0f + (float)exp(-(double)x)); }
__device__ __forceinline__ float dev_sigmoid(float x) { return 1.0f / (1.0f + (float)exp(-(double)x)); }
__device__ __forceinline__ float dev_softplus(float x) {
    if (x > 20.0f) return x;
    const float e = (float)exp((double)x);
    return (float)log((double)(1.0f + e));
}

// ---------------------------------------------------------------- memory scope

__device__ __forceinline__ unsigned atomic_load_relaxed_agent(const unsigned *p) {
    return __hip_atomic_load(gp(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Cross-workgroup data -- every activation, partial and pass-cell word that
// one workgroup writes and another reads later in the pass -- moves through
// device-coherent accesses (agent-scope relaxed atomics: sc1 loads and
// stores, which neither hit nor leave stale lines in an XCD's L2).  A
// workgroup's coherent stores are complete once it has waited vmcnt(0), so
// the grid barrier needs no L2 writeback or invalidate (each costs
// microseconds on gfx950) and orders them by the barrier counter alone.
// Immutable data (weights, norms) and data a workgroup only shares with
// itself across passes (recurrent and conv state) use ordinary cached
// accesses.
// (through global-address-space pointers: a generic pointer would make the
// compiler emit flat instructions, which also count against lgkmcnt and so
// make every LDS wait after them wait for the global access too)
template <class T>
__device__ __forceinline__ T ld_coh(const T *p) {
    return __hip_atomic_load((const __attribute__((address_space(1))) T *)(p), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
}
template <class T>
__device__ __forceinline__ void st_coh(T *p, T v) {
    __hip_atomic_store((__attribute__((address_space(1))) T *)(p), v, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
// 16 bytes (16-aligned) as two coherent 8-byte loads / stores
__device__ __forceinline__ float4 ld_coh4(const float *p) {
    const uint64_t *q = reinterpret_cast<const uint64_t *>(p);
    const uint64_t a = ld_coh(q), b = ld_coh(q + 1);
    return make_float4(__uint_as_float((uint32_t)a), __uint_as_float((uint32_t)(a >> 32)),
                       __uint_as_float((uint32_t)b), __uint_as_float((uint32_t)(b >> 32)));
}
__device__ __forceinline__ void st_coh4(float *p, float4 v) {
    uint64_t *q = reinterpret_cast<uint64_t *>(p);
    st_coh(q, (uint64_t)__float_as_uint(v.x) | ((uint64_t)__float_as_uint(v.y) << 32));
    st_coh(q + 1, (uint64_t)__float_as_uint(v.z) | ((uint64_t)__float_as_uint(v.w) << 32));
}
// Bulk coherent reads: raw buffer loads with the sc1 cache policy (plain,
// non-atomic loads the compiler batches freely; a load past num_records
// returns 0 instead of faulting).  The base must be wave-uniform.
typedef float f32x4_t __attribute__((ext_vector_type(4)));
constexpr int CPOL_SC1 = 16;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t coh_rsrc(const void *base, uint32_t bytes) {
    // readfirstlane returns int: widen through uint32_t (a sign-extended low
    // word with bit 31 set would overwrite the high word)
    const uintptr_t b = reinterpret_cast<uintptr_t>(base);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b);
    const uintptr_t u = ((uintptr_t)hi << 32) | (uintptr_t)lo;
    return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void *>(u), (short)0,
                                             (int)__builtin_amdgcn_readfirstlane(bytes), 0x00020000);
}
__device__ __forceinline__ float4 ld_coh16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const f32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, CPOL_SC1);
    return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ double ld_coh8(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(double, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, CPOL_SC1));
}
__device__ __forceinline__ float ld_coh4b(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, CPOL_SC1));
}

// the compiler's scheduler moves no instruction across this point
__device__ __forceinline__ void sched_fence() { __builtin_amdgcn_sched_barrier(0); }

// wait until this wave's memory operations are complete (a real s_waitcnt
// the compiler's wait-count pass accounts for); gfx9 encoding vmcnt 0,
// expcnt 7, lgkmcnt 15
__device__ __forceinline__ void settle_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Record the first error: err[0] = code (first writer wins), err[1] = aux.
// Ops call this and return normally so every block still reaches the next
// grid barrier (core/interp.cuh error protocol).
__device__ __forceinline__ void raise_error(unsigned *err, unsigned code, unsigned aux) {
    if (!err) return;
    if (atomicCAS(err, 0u, code) == 0u)
        __hip_atomic_store(gp(err + 1), aux, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------- LDS-DMA

// One 1 KiB LDS-DMA chunk per wave: lane l's 16 bytes at base + voff land at
// lds_base + 16*l (gfx950 global_load_lds_dwordx4: no VGPRs involved).
// Issued from inline asm so the compiler does not treat the pending DMA as
// aliasing every later LDS access; callers wait for it explicitly
// (dma_wait).  M0 (the LDS base of the DMA) is restored before the asm ends;
// one wait state separates the M0 write from the DMA that reads it.  COH
// selects the device-coherent cache policy (sc1) for data another workgroup
// wrote earlier in the pass.
template <bool COH>
__device__ __forceinline__ void lds_dma16(uintptr_t base, uint32_t voff, uint32_t lds_base) {
    uint32_t saved;
    if (COH) {
        asm volatile(
            "s_mov_b32 %0, m0\n\t"
            "s_mov_b32 m0, %1\n\t"
            "s_nop 0\n\t"
            "global_load_lds_dwordx4 %2, %3 sc1\n\t"
            "s_mov_b32 m0, %0"
            : "=&s"(saved)
            : "s"(lds_base), "v"(voff), "s"(base)
            : "memory");
    } else {
        asm volatile(
            "s_mov_b32 %0, m0\n\t"
            "s_mov_b32 m0, %1\n\t"
            "s_nop 0\n\t"
            "global_load_lds_dwordx4 %2, %3\n\t"
            "s_mov_b32 m0, %0"
            : "=&s"(saved)
            : "s"(lds_base), "v"(voff), "s"(base)
            : "memory");
    }
}
__device__ __forceinline__ void dma_wait() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// ---------------------------------------------------------------- grid barrier

// Grid barrier over per-workgroup flags (zeroed before the launch, packed 4
// bytes apart after the barrier cells): workgroup w stores its epoch into
// flag w (a plain device-coherent store, no atomic and no reply to wait
// for); wave 0 of every workgroup polls all flags at once -- one 16-byte
// load per lane covers 256 workgroups -- until each holds at least the
// epoch.  The arrival costs one store, the release one load round trip.  No
// cache writeback or invalidate: every wave first waits for its own memory
// operations, and all data that crosses workgroups moves through
// device-coherent loads and stores (dev_common.h).  Split in two so that work
// that does not depend on the barrier (the next GEMV's first weight slots) can
// be issued between arriving and waiting.  `flags` holds gridDim.x words
// (<= 1024).
__device__ __forceinline__ void grid_arrive(unsigned *flags, unsigned &epoch) {
    settle_vmem();
    __syncthreads();
    epoch += 1;
    if (threadIdx.x == 0) __hip_atomic_store(gp(flags + blockIdx.x), epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Returns false on timeout (after spin_limit_ticks < 2^32 wall clock ticks).
__device__ __forceinline__ bool grid_wait(const unsigned *flags, unsigned epoch, uint64_t spin_limit_ticks,
                                          unsigned *err) {
    __shared__ unsigned timed_out;
    if (threadIdx.x < 64) {
        const uint32_t n = gridDim.x, lane = threadIdx.x;
        // (the range a whole number of 16-byte loads: the region past the
        // flags is zeroed too, and those words are skipped below)
        const __amdgpu_buffer_rsrc_t r = coh_rsrc(flags, ((n + 3u) & ~3u) * 4);
        const uint64_t t0 = wall_clock64();
        unsigned to = 0;
        while (true) {
            bool ok = true;
            for (uint32_t base = 0; base < n; base += 256) {
                const uint32_t i = base + lane * 4;
                const float4 f4 = ld_coh16(r, i * 4);
                const unsigned fv[4] = {__float_as_uint(f4.x), __float_as_uint(f4.y), __float_as_uint(f4.z),
                                        __float_as_uint(f4.w)};
#pragma unroll
                for (int k = 0; k < 4; k++) ok = ok && (i + k >= n || (int)(fv[k] - epoch) >= 0);
            }
            if (__builtin_amdgcn_ballot_w64(!ok) == 0) break;
            __builtin_amdgcn_s_sleep(1);
            const uint32_t el = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(wall_clock64() - t0));
            if (el > spin_limit_ticks) {
                if (lane == 0) raise_error(err, SINTER_E_TIMEOUT_BARRIER, epoch);
                to = 1;
                break;
            }
        }
        if (lane == 0) timed_out = to;
    }
    __syncthreads();
    return timed_out == 0;
}

// A grid barrier fused with the op after it (interp.hip): the op's loads that
// do not depend on the barrier are issued between arriving and waiting.
struct GridCross {
    unsigned *flags, *err;
    unsigned *epoch;
    uint64_t spin_limit;
    bool pass_end;              // sample the error cell after the wait
    long long *pass_slot;       // record (wall clock - t0) after the wait (block 0), or null
    uint64_t t0;
    uint64_t t_wait_end;        // out: wall clock after the wait (block 0 timing)
};

// Arrive, run pre() (the op's barrier-independent loads), wait.  False when
// the kernel must stop: a barrier timeout, or an error seen at a pass end.
template <class Pre>
__device__ __forceinline__ bool cross_barrier(GridCross &gx, Pre &&pre) {
    grid_arrive(gx.flags, *gx.epoch);
    pre();
    const bool crossed = grid_wait(gx.flags, *gx.epoch, gx.spin_limit, gx.err);
    gx.t_wait_end = wall_clock64();
    if (!crossed) { settle_vmem(); return false; }
    if (gx.pass_end) {
        __shared__ unsigned e;
        if (threadIdx.x == 0) {
            e = __hip_atomic_load(gx.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (gx.pass_slot) *gx.pass_slot = (long long)(gx.t_wait_end - gx.t0);
        }
        __syncthreads();
        if (e) { settle_vmem(); return false; }
    }
    return true;
}

// ---------------------------------------------------------------- instruction header

// An instruction's header {kind, block_lo, block_hi, flags} as one 64-bit
// scalar load (constant address space: a program does not change while a
// launch runs).  Its 16-bit fields read one by one from global memory are
// vector loads, each waited for with a vmcnt(0) that also waits for every
// vector load and store of the wave still in flight.
typedef const __attribute__((address_space(4))) uint64_t chdr_t;
__device__ __forceinline__ uint64_t ins_hdr(const sinter_instr &ins) { return *(chdr_t *)&ins; }
__device__ __forceinline__ uint32_t hdr_kind(uint64_t h) { return (uint32_t)h & 0xffffu; }
__device__ __forceinline__ uint32_t hdr_lo(uint64_t h) { return (uint32_t)(h >> 16) & 0xffffu; }
__device__ __forceinline__ uint32_t hdr_hi(uint64_t h) { return (uint32_t)(h >> 32) & 0xffffu; }
static_assert(offsetof(sinter_instr, kind) == 0 && offsetof(sinter_instr, block_lo) == 2 &&
                  offsetof(sinter_instr, block_hi) == 4,
              "instruction header layout");

// ---------------------------------------------------------------- block formats

struct blk_q8_0 { uint16_t d; int8_t qs[32]; };                                  // 34 B
struct blk_q4_K { uint16_t d, dmin; uint8_t scales[12]; uint8_t qs[128]; };      // 144 B
struct blk_q6_K { uint8_t ql[128]; uint8_t qh[64]; int8_t scales[16]; uint16_t d; }; // 210 B
static_assert(sizeof(blk_q8_0) == 34, "q8_0");
static_assert(sizeof(blk_q4_K) == 144, "q4_K");
static_assert(sizeof(blk_q6_K) == 210, "q6_K");

}  // namespace sinter
