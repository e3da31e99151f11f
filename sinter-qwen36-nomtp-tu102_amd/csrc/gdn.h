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
// Declared numerics (oracle/oracle.c or_gdn_step): kv and o are fp64 sums of
// exact fp32 products rounded to fp32 once; delta and the state update are
// the reference's fp32 expressions (mul, mul, add; no contraction).
#pragma once
#include "dev_common.h"

namespace sinter {

// ts (thread 0, or null): wall clock stamps [1] after the first item's
// norms and gates, [2] after its state update.
__device__ __forceinline__ void op_gdn_step(const sinter_instr &ins, unsigned *err, uint64_t *ts) {
    lds_char *lds = (lds_char *)g_big;
    const sinter_gdn_args &a = *reinterpret_cast<const sinter_gdn_args *>(ins.payload);
    const uint32_t rel = blockIdx.x - ins.block_lo, nblk = ins.block_hi - ins.block_lo;
    const uint32_t D = a.d, HK = a.hk, HV = a.hv, cols = a.cols;
    // supported envelope: D in {64,128,256}, cols divides D, 256 threads
    // split evenly over cols columns with >= 4 rows per thread
    const uint32_t tpc = cols ? BLOCK_THREADS / cols : 0;  // threads per column
    const bool ok = (D == 64 || D == 128 || D == 256) && cols && (D % cols) == 0 &&
                    (BLOCK_THREADS % cols) == 0 && tpc && tpc <= 64 && (D % tpc) == 0 && (D / tpc) % 4 == 0 &&
                    (D / tpc) <= 32 && HK && HV % HK == 0;
    if (!ok) {
        if (rel == 0 && threadIdx.x == 0) raise_error(err, SINTER_E_BAD_SHAPE, ins.dbg_node);
        return;
    }
    const uint32_t rpt = D / tpc;  // rows per thread
    LDS float *qs = reinterpret_cast<LDS float *>(lds);          // [D] normalised q
    LDS float *ks = qs + 256;                                     // [D] normalised k
    LDS double *red = reinterpret_cast<LDS double *>(ks + 256);   // 16 doubles
    LDS float *gb = reinterpret_cast<LDS float *>(red + 16);      // g, beta
    const uint32_t slices = D / cols, n_items = HV * slices;

    for (uint32_t item = rel; item < n_items; item += nblk) {
        const uint32_t h = item / slices, c0 = (item % slices) * cols;
        const uint32_t hk = h % HK;
        const float *qsrc = a.qkv + (size_t)hk * D;
        const float *ksrc = a.qkv + (size_t)HK * D + (size_t)hk * D;
        const float *vsrc = a.qkv + (size_t)2 * HK * D + (size_t)h * D;
        // l2 norm of q and k (ggml: fp32 squares summed in double,
        // scale = 1/fmaxf(sqrtf(sum), eps))
        double sq = 0.0, sk = 0.0;
        float qv = 0.0f, kv = 0.0f;
        if (threadIdx.x < D) {
            qv = ld_coh(qsrc + threadIdx.x);
            kv = ld_coh(ksrc + threadIdx.x);
            sq = (double)(qv * qv);
            sk = (double)(kv * kv);
        }
        sq = block_sum_f64(sq, red);
        sk = block_sum_f64(sk, red);
        if (threadIdx.x < D) {
            qs[threadIdx.x] = qv * (1.0f / fmaxf(sqrtf((float)sq), a.eps));
            ks[threadIdx.x] = kv * (1.0f / fmaxf(sqrtf((float)sk), a.eps));
        }
        if (threadIdx.x == 0) {
            const float sp = dev_softplus(ld_coh(a.alpha + h) + gp(a.dt_bias)[h]);
            gb[0] = (float)exp((double)(sp * gp(a.ssm_a)[h]));
            gb[1] = dev_sigmoid(ld_coh(a.beta + h));
        }
        __syncthreads();
        if (ts && item == rel) ts[1] = wall_clock64();
        const float g = gb[0], beta = gb[1];

        // this thread: column c0 + threadIdx.x / tpc, rows [i0, i0 + rpt)
        const uint32_t col = c0 + threadIdx.x / tpc;
        const uint32_t i0 = (threadIdx.x % tpc) * rpt;
        GLB float *srow = gp(a.state + ((size_t)h * D + col) * D + i0);
        float s[32];
#pragma unroll
        for (uint32_t r = 0; r < 32; r += 4) {
            if (r < rpt) {
                const f32x4 t = *reinterpret_cast<const GLB f32x4 *>(srow + r);
                s[r] = t.x; s[r + 1] = t.y; s[r + 2] = t.z; s[r + 3] = t.w;
            }
        }
        double dkv = 0.0;
#pragma unroll
        for (uint32_t r = 0; r < 32; r++)
            if (r < rpt) dkv += (double)s[r] * (double)ks[i0 + r];
        for (uint32_t o = 1; o < tpc; o <<= 1) dkv += __shfl_xor(dkv, (int)o, 64);
        const float kvf = (float)dkv;
        const float t1 = g * kvf;
        const float t2 = ld_coh(vsrc + col) - t1;
        const float delta = t2 * beta;
        double dout = 0.0;
#pragma unroll
        for (uint32_t r = 0; r < 32; r++) {
            if (r < rpt) {
                const float u1 = g * s[r];
                const float u2 = ks[i0 + r] * delta;
                s[r] = u1 + u2;
                dout += (double)s[r] * (double)qs[i0 + r];
            }
        }
        for (uint32_t o = 1; o < tpc; o <<= 1) dout += __shfl_xor(dout, (int)o, 64);
#pragma unroll
        for (uint32_t r = 0; r < 32; r += 4)
            if (r < rpt) {
                const f32x4 v = {s[r], s[r + 1], s[r + 2], s[r + 3]};
                *reinterpret_cast<GLB f32x4 *>(srow + r) = v;
            }
        if ((threadIdx.x % tpc) == 0) st_coh(a.o + (size_t)h * D + col, (float)dout * a.scale);
        if (ts && item == rel) ts[2] = wall_clock64();
        __syncthreads();  // qs/ks/gb reused by the next item
    }
}

}  // namespace sinter
