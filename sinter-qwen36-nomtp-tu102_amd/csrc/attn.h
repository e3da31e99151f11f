// SINTER_OP_ATTN_DECODE: one full-attention layer's decode step after the
// q|gate / k / v projections, fused:
//   per-head RMSNorm * weight + NEOX RoPE on the first rope_dims dims
//                                              (k0/ops/attn.cuh:109-182)
//   f16 KV append at row pos                   (attn.cuh:184-211)
//   split-K online-softmax partials            (attn.cuh:244-401)
//   max/LSE merge by the last-arriving block   (attn.cuh:403-458)
//   sigmoid output gate                        (attn.cuh:460-488)
// Work item = (kv head g, chunk c).  An item serves all NQ/NKV q heads of
// its group from one read of its K/V rows (GQA sharing).  The item whose
// chunk holds `pos` also appends the new K/V row and uses it directly.  Each
// item publishes an fp64 partial {acc[HD], max, sum} per q head; the block
// that arrives last for kv head g merges that head group and applies the
// gate, so the reference's separate FATTN_REDUCE / ATTN_GATE windows (and
// their barriers) disappear.
//
// Declared numerics (oracle/oracle.c or_attn_decode): q/k norms and RoPE in
// fp32 as ggml; scores are fp64 sums of exact products times the fp32 scale;
// softmax and the V sum in fp64; the merged output rounded to fp32 once.
#pragma once
#include "dev_common.h"

namespace sinter {

constexpr int ATT_TILE = 32;   // KV positions per LDS tile
constexpr int ATT_MAXG = 8;    // max q heads per kv head

// The q heads of a kv group (and, for the chunk that appends, the new k row)
// normalised and rotated together: y = rmsnorm(x) * w per 256-wide head, then
// NEOX RoPE on the first rope_dims dims.  Thread t holds dim t of every head.
// Per-head sums of squares are reduced like block_sum_f64 (DPP rows, the four
// row sums of a wave, then the waves in order), all heads at once, so the
// whole prologue costs three workgroup barriers.  Rope pair i turns by
// theta_i = pos * theta_scale^i (repeated fp32 products, as ggml's rope
// cache), cos/sin evaluated in double and rounded to fp32.
// x[j] for j < nh are the raw values; rows j < nq use qw, row nq (if nh > nq)
// uses kw.  Results land in dst[j*256 + t].  LDS: qn [ATT_MAXG+1][256]
// floats, rot [2][128] floats, red [4][ATT_MAXG+1] doubles.
__device__ __forceinline__ void att_prep(const float x[ATT_MAXG + 1], uint32_t nq, uint32_t nh, const float *qw,
                                         const float *kw, float eps, int pos, float theta_scale, uint32_t rope_dims,
                                         float *dst, float *qn, float *rot, double *red) {
    const uint32_t t = threadIdx.x, half = rope_dims / 2;
    if (t < half) {
        float th = (float)pos;
        for (uint32_t i = 0; i < t; i++) th *= theta_scale;
        rot[t] = (float)cos((double)th);
        rot[128 + t] = (float)sin((double)th);
    }
#pragma unroll
    for (uint32_t j = 0; j < ATT_MAXG + 1; j++) {
        if (j < nh) {
            const double v = row16_sum_f64((double)(x[j] * x[j]));
            const double w = ((readlane_f64(v, 0) + readlane_f64(v, 16)) + readlane_f64(v, 32)) + readlane_f64(v, 48);
            if (lane_id() == 0) red[wave_id() * (ATT_MAXG + 1) + j] = w;
        }
    }
    __syncthreads();
#pragma unroll
    for (uint32_t j = 0; j < ATT_MAXG + 1; j++) {
        if (j < nh) {
            double ss = 0.0;
            for (int wv = 0; wv < (int)(BLOCK_THREADS / 64); wv++) ss += red[wv * (ATT_MAXG + 1) + j];
            const float mean = (float)(ss / 256.0);
            const float sc = 1.0f / sqrtf(mean + eps);
            const float nrm = x[j] * sc;
            qn[j * 256 + t] = nrm * (j < nq ? qw[t] : kw[t]);
        }
    }
    __syncthreads();
    for (uint32_t j = 0; j < nh; j++) {
        const float *r = qn + j * 256;
        float y = r[t];
        if (t < half) {
            const float x0 = r[t], x1 = r[t + half], c = rot[t], s = rot[128 + t];
            const float a0 = x0 * c, a1 = x1 * s;
            y = a0 - a1;
        } else if (t < 2 * half) {
            const uint32_t i = t - half;
            const float x0 = r[i], x1 = r[t], c = rot[i], s = rot[128 + i];
            const float b0 = x0 * s, b1 = x1 * c;
            y = b0 + b1;
        }
        dst[j * 256 + t] = y;
    }
    __syncthreads();
}

constexpr uint32_t ATT_FAN = 8;   // partials merged per step of the merge tree

// Merge n (<= ATT_FAN) consecutive partials {acc[HD], m, l} of each of gqa
// q heads (fp64, coherent reads): M = max m_i, acc = sum_i e_i acc_i,
// l = sum_i e_i l_i with e_i = exp(m_i - M), in ascending i; a partial with
// m = -inf contributes nothing.  Thread t owns dim t.  With dst, the merged
// unnormalised partial goes there; otherwise out = acc/l * sigmoid(gate).
// ew: LDS scratch of ATT_MAXG * (ATT_FAN + 1) doubles.
__device__ __forceinline__ void att_merge(const sinter_attn_args &a, const double *src, uint32_t n, uint32_t gqa, uint32_t g,
                          double *dst, double *ew) {
    const uint32_t t = threadIdx.x, HD = a.hd, PS = HD + 2;
    const __amdgpu_buffer_rsrc_t r = coh_rsrc(src, n * gqa * PS * 8);
    // weights e[hh][i] and the max, one lane per q head
    if (t < gqa) {
        double m[ATT_FAN], M = -INFINITY;
#pragma unroll
        for (uint32_t i = 0; i < ATT_FAN; i++) {
            m[i] = i < n ? ld_coh8(r, ((i * gqa + t) * PS + HD) * 8) : -INFINITY;
            M = fmax(M, m[i]);
        }
#pragma unroll
        for (uint32_t i = 0; i < ATT_FAN; i++)
            ew[t * (ATT_FAN + 1) + i] = (m[i] == -INFINITY) ? 0.0 : exp(m[i] - M);
        ew[t * (ATT_FAN + 1) + ATT_FAN] = M;
    }
    __syncthreads();
    for (uint32_t hh = 0; hh < gqa; hh++) {
        const double *e = ew + hh * (ATT_FAN + 1);
        double pv[ATT_FAN], lv[ATT_FAN];
#pragma unroll
        for (uint32_t i = 0; i < ATT_FAN; i++) {
            const uint32_t o = (i * gqa + hh) * PS;
            pv[i] = i < n ? ld_coh8(r, (o + t) * 8) : 0.0;
            lv[i] = i < n ? ld_coh8(r, (o + HD + 1) * 8) : 0.0;
        }
        double O = 0.0, L = 0.0;
#pragma unroll
        for (uint32_t i = 0; i < ATT_FAN; i++) {
            if (i < n && e[i] != 0.0) {
                O = fma(e[i], pv[i], O);
                L = fma(e[i], lv[i], L);
            }
        }
        if (dst) {
            double *d = dst + hh * PS;
            st_coh(d + t, O);
            if (t == 0) { st_coh(d + HD, e[ATT_FAN]); st_coh(d + HD + 1, L); }
        } else {
            const uint32_t h = g * gqa + hh;
            const float att = (float)(O / L);
            const float gate = ld_coh(a.qg + (size_t)h * 2 * HD + HD + t);
            st_coh(a.out + (size_t)h * HD + t, att * dev_sigmoid(gate));
        }
    }
    settle_vmem();
    __syncthreads();
}

// Count one arrival at *cnt of `total`; true (uniform) for the last arriver,
// which also resets the counter for the next use.
__device__ __forceinline__ bool att_arrive(uint32_t *cnt, uint32_t total, unsigned *flag) {
    settle_vmem();   // every wave's partial stores complete before the count
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const unsigned last = (old == total - 1) ? 1u : 0u;
        if (last) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *flag = last;
    }
    __syncthreads();
    return *flag != 0;
}

__device__ __forceinline__ void op_attn_decode(const sinter_instr &ins, unsigned *err) {
    // the payload, read once into registers: the op stores to the KV cache
    // and the partials, which the compiler cannot tell apart from the payload
    // (every field would be reloaded from memory after each such store)
    const sinter_attn_args a = *reinterpret_cast<const sinter_attn_args *>(ins.payload);
    const uint32_t rel = blockIdx.x - ins.block_lo, nblk = ins.block_hi - ins.block_lo;
    const uint32_t NQ = a.nq, NKV = a.nkv, HD = a.hd, C = a.n_chunks;
    const int pos = ld_coh(&reinterpret_cast<const sinter_pass_cell *>(a.pass_cell)->pos);
    const uint32_t gqa = NKV ? NQ / NKV : 0;
    const bool ok = HD == 256 && NKV && NQ % NKV == 0 && gqa >= 1 && gqa <= ATT_MAXG && C >= 1 &&
                    C <= ATT_FAN * ATT_FAN &&
                    a.rope_dims <= HD && (a.rope_dims % 2) == 0 && pos >= 0 && (uint32_t)pos < a.n_ctx;
    if (!ok) {
        if (rel == 0 && threadIdx.x == 0) raise_error(err, SINTER_E_BAD_SHAPE, ins.dbg_node);
        return;
    }
    const uint32_t t = threadIdx.x;
    const uint32_t RW = NKV * HD;
    const uint32_t n_kv = (uint32_t)pos + 1;
    uint32_t clen = (n_kv + C - 1) / C;
    clen = (clen + ATT_TILE - 1) / ATT_TILE * ATT_TILE;

    // LDS map (the scratch region): q heads, K tile, new K/V row |
    // V tile, scores, softmax state, scratch
    float *qf = reinterpret_cast<float *>(g_big);                      // [gqa][256] q, then the new k row
    uint16_t *kt = reinterpret_cast<uint16_t *>(qf + (ATT_MAXG + 1) * 256);   // [32][256]
    uint16_t *knew = kt + ATT_TILE * 256;                                // [256]
    uint16_t *vnew = knew + 256;                                         // [256]
    uint16_t *vt = reinterpret_cast<uint16_t *>(g_big + ATT_REGION);                // [32][256]
    double *sc = reinterpret_cast<double *>(vt + ATT_TILE * 256);        // [gqa][32] scores -> weights
    double *mrun = sc + ATT_MAXG * ATT_TILE;                             // [gqa]
    double *lrun = mrun + ATT_MAXG;                                      // [gqa]
    double *corr = lrun + ATT_MAXG;                                      // [gqa]
    double *red = corr + ATT_MAXG;                                       // 16
    float *knf = reinterpret_cast<float *>(red + 16);                    // [256] k scratch
    unsigned *flag = reinterpret_cast<unsigned *>(knf + 256);
    double *ew = reinterpret_cast<double *>(g_big + 2 * ATT_REGION);    // [ATT_MAXG][ATT_FAN+1] merge weights
    float *qn = reinterpret_cast<float *>(g_big + 2 * ATT_REGION + 1024);   // [ATT_MAXG+1][256] prep scratch
    float *rot = qn + (ATT_MAXG + 1) * 256;                                  // [2][128] rope cos | sin
    double *pred = reinterpret_cast<double *>(rot + 256);                   // [4][ATT_MAXG+1]

    for (uint32_t item = rel; item < NKV * C; item += nblk) {
        const uint32_t g = item / C, c = item % C;
        const uint32_t kv0 = min(c * clen, n_kv), kv1 = min(kv0 + clen, n_kv);
        const bool owner = kv0 <= (uint32_t)pos && (uint32_t)pos < kv1;

        {
            // q heads g*gqa .. and, for the owner, the new k row (as head gqa)
            float xr[ATT_MAXG + 1];
#pragma unroll
            for (uint32_t hh = 0; hh < ATT_MAXG; hh++)
                xr[hh] = hh < gqa ? ld_coh(a.qg + (size_t)(g * gqa + hh) * 2 * HD + t) : 0.0f;
            xr[ATT_MAXG] = 0.0f;
            if (owner) {
#pragma unroll
                for (uint32_t hh = 0; hh <= ATT_MAXG; hh++)
                    if (hh == gqa) xr[hh] = ld_coh(a.k + (size_t)g * HD + t);
            }
            att_prep(xr, gqa, owner ? gqa + 1 : gqa, a.q_norm, a.k_norm, a.eps, pos, a.theta_scale, a.rope_dims, qf,
                     qn, rot, pred);
        }
        if (owner) {
            const uint16_t kh = f2h(qf[gqa * 256 + t]), vh = f2h(ld_coh(a.v + (size_t)g * HD + t));
            knew[t] = kh;
            vnew[t] = vh;
            st_coh(a.kc + (size_t)pos * RW + (size_t)g * HD + t, kh);
            st_coh(a.vc + (size_t)pos * RW + (size_t)g * HD + t, vh);
        }
        if (t < gqa) { mrun[t] = -INFINITY; lrun[t] = 0.0; }
        double acc[ATT_MAXG];
#pragma unroll
        for (int hh = 0; hh < ATT_MAXG; hh++) acc[hh] = 0.0;
        __syncthreads();

        for (uint32_t t0 = kv0; t0 < kv1; t0 += ATT_TILE) {
            // K and V tiles of this kv head: 32 rows x 512 B each
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint32_t idx = t + k * 256, r = idx >> 5, ch = idx & 31, j = t0 + r;
                uint4 kv4 = make_uint4(0, 0, 0, 0), vv4 = make_uint4(0, 0, 0, 0);
                if (j < kv1) {
                    if (owner && j == (uint32_t)pos) {
                        kv4 = reinterpret_cast<const uint4 *>(knew)[ch];
                        vv4 = reinterpret_cast<const uint4 *>(vnew)[ch];
                    } else {
                        const size_t o = (size_t)j * RW + (size_t)g * HD;
                        kv4 = reinterpret_cast<const uint4 *>(a.kc + o)[ch];
                        vv4 = reinterpret_cast<const uint4 *>(a.vc + o)[ch];
                    }
                }
                reinterpret_cast<uint4 *>(kt)[idx] = kv4;
                reinterpret_cast<uint4 *>(vt)[idx] = vv4;
            }
            __syncthreads();
            // scores: thread (r = t/8, part = t%8) covers dims [32 part, 32 part + 32)
            {
                const uint32_t r = t >> 3, part = t & 7;
                const uint16_t *kr = kt + r * 256 + part * 32;
                for (uint32_t hh = 0; hh < gqa; hh++) {
                    const float *q = qf + hh * 256 + part * 32;
                    double d = 0.0;
#pragma unroll
                    for (int i = 0; i < 32; i++) d = fma((double)q[i], (double)h2f(kr[i]), d);
                    d += __shfl_xor(d, 1, 64);
                    d += __shfl_xor(d, 2, 64);
                    d += __shfl_xor(d, 4, 64);
                    if (part == 0) sc[hh * ATT_TILE + r] = (t0 + r < kv1) ? d * (double)a.scale : -INFINITY;
                }
            }
            __syncthreads();
            // online softmax per head: 32 lanes per head
            if (t < gqa * ATT_TILE) {
                const uint32_t hh = t / ATT_TILE, r = t % ATT_TILE;
                const double s = sc[hh * ATT_TILE + r];
                double mt = s;
#pragma unroll
                for (int o = 16; o > 0; o >>= 1) mt = fmax(mt, __shfl_xor(mt, o, 64));
                const double mo = mrun[hh];
                const double mn = fmax(mo, mt);
                const double w = (s == -INFINITY) ? 0.0 : exp(s - mn);
                double ws = w;
#pragma unroll
                for (int o = 16; o > 0; o >>= 1) ws += __shfl_xor(ws, o, 64);
                sc[hh * ATT_TILE + r] = w;
                if (r == 0) {
                    const double cf = (mo == -INFINITY) ? 0.0 : exp(mo - mn);
                    corr[hh] = cf;
                    lrun[hh] = lrun[hh] * cf + ws;
                    mrun[hh] = mn;
                }
            }
            __syncthreads();
            // V accumulation: thread t owns dim t
            for (uint32_t hh = 0; hh < gqa; hh++) {
                double v = acc[hh] * corr[hh];
                const double *w = sc + hh * ATT_TILE;
#pragma unroll 8
                for (int r = 0; r < ATT_TILE; r++) v = fma(w[r], (double)h2f(vt[r * 256 + t]), v);
                acc[hh] = v;
            }
            __syncthreads();
        }

        // publish the partial; the merge is a tree of fan-in ATT_FAN over
        // the chunks, each node merged by the last arriver of its children
        const uint32_t PS = HD + 2, G1 = (C + ATT_FAN - 1) / ATT_FAN, g1 = c / ATT_FAN;
        double *pbase = a.part + ((size_t)g * C + c) * gqa * PS;
        for (uint32_t hh = 0; hh < gqa; hh++) {
            double *p = pbase + hh * PS;
            st_coh(p + t, acc[hh]);
            if (t == 0) { st_coh(p + HD, mrun[hh]); st_coh(p + HD + 1, lrun[hh]); }
        }
        const uint32_t n1 = min(ATT_FAN, C - g1 * ATT_FAN);
        double *lvl1 = a.part + (size_t)NKV * C * gqa * PS;                 // [NKV][G1][gqa][PS]
        if (att_arrive(a.count + NKV + g * G1 + g1, n1, flag)) {
            double *node = lvl1 + ((size_t)g * G1 + g1) * gqa * PS;
            att_merge(a, a.part + ((size_t)g * C + g1 * ATT_FAN) * gqa * PS, n1, gqa, g, G1 > 1 ? node : nullptr, ew);
            if (G1 > 1 && att_arrive(a.count + g, G1, flag)) {
                // G1 <= ATT_FAN: the root merges the group nodes
                att_merge(a, lvl1 + (size_t)g * G1 * gqa * PS, G1, gqa, g, nullptr, ew);
            }
        }
        __syncthreads();
    }
}

}  // namespace sinter
