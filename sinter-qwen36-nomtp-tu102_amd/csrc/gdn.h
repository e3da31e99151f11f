// SINTER_OP_GDN_STEP: one token of the gated-DeltaNet recurrence, fused:
//   q/k l2 norm        (k0/ops/gdn.cuh:174-212)
//   gates g, beta      (k0/ops/gdn.cuh:215-245)
//   delta-rule update  (k0/ops/gdn.cuh:248-337)
// The causal conv + silu has already run in the qkv GEMV epilogue, and the
// gated RMSNorm runs in the prologue of the ssm_out GEMV, so the reference's
// STATE_LOAD / CONV_SHIFT_CONCAT / SSM_CONV_SILU / QK_L2NORM / GDN_GATES /
// GDN_STEP / GATED_RMSNORM / STATE_STORE chain (8 instructions, 6 barriers)
// becomes this one op between two barriers.
//
// Work item = (v-head h, slice of `cols` state columns).  Columns are
// independent in the delta rule, so a head's 128 columns spread over
// D/cols workgroups; each streams its cols*D*4 bytes of state once in and
// once out (in place).  The k-head of v-head h is h % HK (gdn.cuh:257-259).
//
// Declared numerics (oracle/oracle.c or_gdn_step), fp32 folds in the style
// of k0/ops/gdn.cuh:19-28: kv and o are per-thread sequential fp32 sums over
// the thread's RPT rows ascending (acc = acc + s*x, a rounded product then a
// rounded add, never contracted), closed by the butterfly a[t] += a[t ^ m],
// m = 1, 2, 4, ... over the column's tpc = 256 / cols threads
// (lanes_sum_f32); delta = (v - g*kv) * beta and the state update g*S + k*delta
// are the reference's fp32 expressions (mul, mul, add); o is scaled last.
#pragma once
#include <type_traits>

#include "dev_common.h"

namespace sinter {

// ts (thread 0, or null): wall clock stamps [1] after the first item's
// norms and gates, [2] after its state update.  gx (or null): the grid
// barrier before the op, crossed here with the first item's state slice
// loaded between arriving and waiting (the state is this workgroup's own
// from the previous pass); false when the kernel must stop.
__device__ __forceinline__ bool op_gdn_step(const sinter_instr &ins, unsigned *err, uint64_t *ts, GridCross *gx) {
    lds_char *lds = (lds_char *)g_big;
    const sinter_gdn_args &a = *reinterpret_cast<const sinter_gdn_args *>(ins.payload);
    const uint64_t hdr = ins_hdr(ins);
    const uint32_t rel = blockIdx.x - hdr_lo(hdr), nblk = hdr_hi(hdr) - hdr_lo(hdr);
    const uint32_t D = a.d, HK = a.hk, HV = a.hv, cols = a.cols;
    // supported envelope: D in {64,128,256}, cols divides D, 256 threads
    // split evenly over cols columns with >= 4 rows per thread
    const uint32_t tpc = cols ? BLOCK_THREADS / cols : 0;  // threads per column
    const bool ok = (D == 64 || D == 128 || D == 256) && cols && (D % cols) == 0 &&
                    (BLOCK_THREADS % cols) == 0 && tpc && tpc <= 64 && (D % tpc) == 0 && (D / tpc) % 4 == 0 &&
                    (D / tpc) <= 32 && HK && HV % HK == 0;
    if (!ok) {
        if (gx && !cross_barrier(*gx, [] {})) return false;
        if (rel == 0 && threadIdx.x == 0) raise_error(err, SINTER_E_BAD_SHAPE, ins.dbg_node);
        return true;
    }
    const uint32_t rpt = D / tpc;  // rows per thread
    LDS float *qs = reinterpret_cast<LDS float *>(lds);          // [D] normalised q
    LDS float *ks = qs + 256;                                     // [D] normalised k
    LDS double *red = reinterpret_cast<LDS double *>(ks + 256);   // 16 doubles
    const uint32_t slices = D / cols, n_items = HV * slices;

    // the item loop with the rows per thread a compile-time constant, so the
    // state loads are unconditional and the wait counts exact
    auto items = [&](auto rptc) -> bool {
    constexpr uint32_t RPT = decltype(rptc)::value;
    // this thread's state: column c0 + threadIdx.x / tpc of v-head h, rows
    // [i0, i0 + RPT) (unconditional 16-byte loads: the wait counts stay exact)
    auto state_row = [&](uint32_t item) {
        const uint32_t h = item / slices, c0 = (item % slices) * cols;
        return gp(a.state + ((size_t)h * D + c0 + threadIdx.x / tpc) * D + (threadIdx.x % tpc) * RPT);
    };
    float s[RPT];
    auto load_state = [&](uint32_t item) {
        const GLB float *srow = state_row(item);
#pragma unroll
        for (uint32_t r = 0; r < RPT; r += 4) {
            const f32x4 t = *reinterpret_cast<const GLB f32x4 *>(srow + r);
            s[r] = t.x; s[r + 1] = t.y; s[r + 2] = t.z; s[r + 3] = t.w;
        }
    };
    if (gx && !cross_barrier(*gx, [&] { if (rel < n_items) load_state(rel); })) return false;
    for (uint32_t item = rel; item < n_items; item += nblk) {
        const uint32_t h = item / slices, c0 = (item % slices) * cols;
        const uint32_t hk = h % HK;
        const float *qsrc = a.qkv + (size_t)hk * D;
        const float *ksrc = a.qkv + (size_t)HK * D + (size_t)hk * D;
        const float *vsrc = a.qkv + (size_t)2 * HK * D + (size_t)h * D;
        // this thread: column c0 + threadIdx.x / tpc, rows [i0, i0 + rpt)
        const uint32_t col = c0 + threadIdx.x / tpc;
        const uint32_t i0 = (threadIdx.x % tpc) * RPT;
        // every load of the item first (one memory round trip): q, k, v and
        // the raw gates (written by the projection), then the state slice
        // unless it crossed the barrier (unconditional: lanes past D re-read
        // element t % D and drop it, so no divergent branch hides the loads'
        // order from the wait counts)
        const uint32_t tq = threadIdx.x & (D - 1);
        const float qv = ld_coh(qsrc + tq), kv = ld_coh(ksrc + tq);
        const float vcol = ld_coh(vsrc + col);
        const float alpha = ld_coh(a.alpha + h), braw = ld_coh(a.beta + h);
        const float dtb = gp(a.dt_bias)[h], sa = gp(a.ssm_a)[h];
        GLB float *srow = state_row(item);
        if (!gx || item != rel) load_state(item);
        // l2 norm of q and k (ggml: fp32 squares summed in double,
        // scale = 1/fmaxf(sqrtf(sum), eps)); both sums in one reduction
        const bool mine = threadIdx.x < D;
        double sq = mine ? (double)(qv * qv) : 0.0, sk = mine ? (double)(kv * kv) : 0.0;
        block_sum2_f64(sq, sk, red);
        if (threadIdx.x < D) {
            qs[threadIdx.x] = qv * (1.0f / fmaxf(sqrtf((float)sq), a.eps));
            ks[threadIdx.x] = kv * (1.0f / fmaxf(sqrtf((float)sk), a.eps));
        }
        // gates, in every lane (no broadcast needed) while the state lands
        const float sp = dev_softplus(alpha + dtb);
        const float g = (float)exp((double)(sp * sa));
        const float beta = dev_sigmoid(braw);
        __syncthreads();
        if (ts && item == rel) ts[1] = wall_clock64();

        float dkv = 0.0f;
#pragma unroll
        for (uint32_t r = 0; r < RPT; r++) {
            const float pr = s[r] * ks[i0 + r];
            dkv = dkv + pr;
        }
        const float kvf = lanes_sum_f32(dkv, tpc);
        const float t1 = g * kvf;
        const float t2 = vcol - t1;
        const float delta = t2 * beta;
        float dout = 0.0f;
#pragma unroll
        for (uint32_t r = 0; r < RPT; r++) {
            const float u1 = g * s[r];
            const float u2 = ks[i0 + r] * delta;
            s[r] = u1 + u2;
            const float pr = s[r] * qs[i0 + r];
            dout = dout + pr;
        }
        dout = lanes_sum_f32(dout, tpc);
#pragma unroll
        for (uint32_t r = 0; r < RPT; r += 4) {
            const f32x4 v = {s[r], s[r + 1], s[r + 2], s[r + 3]};
            *reinterpret_cast<GLB f32x4 *>(srow + r) = v;
        }
        if ((threadIdx.x % tpc) == 0) st_coh(a.o + (size_t)h * D + col, dout * a.scale);
        if (ts && item == rel) ts[2] = wall_clock64();
        __syncthreads();  // qs/ks reused by the next item
    }
    return true;
    };
    switch (rpt) {
    case 4: return items(std::integral_constant<uint32_t, 4>{});
    case 8: return items(std::integral_constant<uint32_t, 8>{});
    case 16: return items(std::integral_constant<uint32_t, 16>{});
    default: return items(std::integral_constant<uint32_t, 32>{});
    }
}

}  // namespace sinter
