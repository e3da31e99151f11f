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
                                         LDS float *dst, LDS float *qn, LDS float *rot, LDS double *red) {
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
            qn[j * 256 + t] = nrm * (j < nq ? gp(qw)[t] : gp(kw)[t]);
        }
    }
    __syncthreads();
    for (uint32_t j = 0; j < nh; j++) {
        const LDS float *r = qn + j * 256;
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
// m = -inf contributes nothing.  Thread t owns dim t; every load is issued
// before the first is used (one memory round trip).  With dst, the merged
// unnormalised partial goes there; otherwise out = acc/l * sigmoid(gate).
// ew: LDS scratch of ATT_MAXG * (ATT_FAN + 2) doubles.
__device__ __forceinline__ void att_merge(const sinter_attn_args &a, const double *src, uint32_t n, uint32_t gqa, uint32_t g,
                          double *dst, LDS double *ew) {
    const uint32_t t = threadIdx.x, HD = a.hd, PS = HD + 2;
    const __amdgpu_buffer_rsrc_t r = coh_rsrc(src, n * gqa * PS * 8);
    double pv[ATT_MAXG][ATT_FAN], m[ATT_FAN], lv[ATT_FAN];
#pragma unroll
    for (uint32_t hh = 0; hh < ATT_MAXG; hh++)
#pragma unroll
        for (uint32_t i = 0; i < ATT_FAN; i++)
            pv[hh][i] = (hh < gqa && i < n) ? ld_coh8(r, ((i * gqa + hh) * PS + t) * 8) : 0.0;
    // weights e[hh][i], the max and l, one lane per q head
    if (t < gqa) {
#pragma unroll
        for (uint32_t i = 0; i < ATT_FAN; i++) {
            m[i] = i < n ? ld_coh8(r, ((i * gqa + t) * PS + HD) * 8) : -INFINITY;
            lv[i] = i < n ? ld_coh8(r, ((i * gqa + t) * PS + HD + 1) * 8) : 0.0;
        }
        double M = -INFINITY;
#pragma unroll
        for (uint32_t i = 0; i < ATT_FAN; i++) M = fmax(M, m[i]);
        double L = 0.0;
#pragma unroll
        for (uint32_t i = 0; i < ATT_FAN; i++) {
            const double e = (m[i] == -INFINITY) ? 0.0 : exp(m[i] - M);
            ew[t * (ATT_FAN + 2) + i] = e;
            if (i < n && e != 0.0) L = fma(e, lv[i], L);
        }
        ew[t * (ATT_FAN + 2) + ATT_FAN] = M;
        ew[t * (ATT_FAN + 2) + ATT_FAN + 1] = L;
    }
    __syncthreads();
#pragma unroll
    for (uint32_t hh = 0; hh < ATT_MAXG; hh++) {
        if (hh >= gqa) break;
        const LDS double *e = ew + hh * (ATT_FAN + 2);
        double O = 0.0;
#pragma unroll
        for (uint32_t i = 0; i < ATT_FAN; i++)
            if (i < n && e[i] != 0.0) O = fma(e[i], pv[hh][i], O);
        const double L = e[ATT_FAN + 1];
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
__device__ __forceinline__ bool att_arrive(uint32_t *cnt, uint32_t total, LDS unsigned *flag) {
    settle_vmem();   // every wave's partial stores complete before the count
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned old = __hip_atomic_fetch_add(gp(cnt), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const unsigned last = (old == total - 1) ? 1u : 0u;
        if (last) __hip_atomic_store(gp(cnt), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *flag = last;
    }
    __syncthreads();
    return *flag != 0;
}

// ts (thread 0, or null): wall clock stamps [1] after the q prep of the
// first item, [2] after its KV tiles.
__device__ __forceinline__ void op_attn_decode(const sinter_instr &ins, unsigned *err, uint64_t *ts) {
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

    // LDS map (the scratch region): K and V tiles double-buffered by LDS-DMA,
    // q heads (and the new k row), prep scratch, scores, softmax state
    lds_char *L = (lds_char *)g_big;
    LDS uint16_t *kb = reinterpret_cast<LDS uint16_t *>(L);                          // [2][32][256]
    LDS uint16_t *vb = reinterpret_cast<LDS uint16_t *>(L + 2 * ATT_TILE * 512);     // [2][32][256]
    LDS float *qf = reinterpret_cast<LDS float *>(L + 4 * ATT_TILE * 512);           // [gqa][256] q, then the new k row
    LDS float *qn = qf + (ATT_MAXG + 1) * 256;    // [ATT_MAXG+2][256] raw q / k / v rows, then prep scratch
    LDS float *rot = qn + (ATT_MAXG + 2) * 256;                                      // [2][128] rope cos | sin
    LDS double *pred = reinterpret_cast<LDS double *>(rot + 256);                    // [4][ATT_MAXG+1]
    LDS double *sc = pred + 4 * (ATT_MAXG + 1);                                      // [32][ATT_MAXG] scores -> weights
    LDS double *mrun = sc + ATT_MAXG * ATT_TILE;                                     // [gqa]
    LDS double *lrun = mrun + ATT_MAXG;                                              // [gqa]
    LDS double *corr = lrun + ATT_MAXG;                                              // [gqa]
    LDS double *ew = corr + ATT_MAXG;                                                // [ATT_MAXG][ATT_FAN+2] merge weights
    LDS uint16_t *knew = reinterpret_cast<LDS uint16_t *>(ew + ATT_MAXG * (ATT_FAN + 2));   // [256]
    LDS uint16_t *vnew = knew + 256;                                                 // [256]
    LDS unsigned *flag = reinterpret_cast<LDS unsigned *>(vnew + 256);
    const uint32_t w = __builtin_amdgcn_readfirstlane(wave_id()), lane = lane_id();
    const uint32_t kbase = (uint32_t)(uintptr_t)kb, vbase = (uint32_t)(uintptr_t)vb;

    for (uint32_t item = rel; item < NKV * C; item += nblk) {
        const uint32_t g = item / C, c = item % C;
        const uint32_t kv0 = min(c * clen, n_kv), kv1 = min(kv0 + clen, n_kv);
        const bool owner = kv0 <= (uint32_t)pos && (uint32_t)pos < kv1;
        const uint32_t ntile = (kv1 - kv0 + ATT_TILE - 1) / ATT_TILE;
        // Tile j (32 rows of this kv head: 512 B of K and of V each) into
        // buffer j % 2: each wave DMAs rows 2k, 2k+1 for k = w, w+4, w+8,
        // w+12 of K and of V (lane l: row 2k + l/32, bytes 16 (l%32) ..);
        // rows past kv1 re-read row kv1-1 (masked in the scores).
        auto issue_tile = [&](uint32_t j) {
            const uint32_t t0 = kv0 + j * ATT_TILE, bo = (j & 1) * ATT_TILE * 512;
#pragma unroll
            for (uint32_t kk = 0; kk < 4; kk++) {
                const uint32_t k = w + 4 * kk, row = min(t0 + 2 * k + (lane >> 5), kv1 - 1);
                const uint32_t voff = (row * RW + g * HD) * 2 + (lane & 31) * 16;
                lds_dma16<true>((uintptr_t)a.kc, voff, kbase + bo + k * 1024);
                lds_dma16<true>((uintptr_t)a.vc, voff, vbase + bo + k * 1024);
            }
        };
        {
            // The raw q heads g*gqa .. (and, for the owner, the new k and v
            // rows) by LDS-DMA into qn rows 0..gqa+1, one 1 KiB row per wave
            // instruction; then the first two tiles.  Every wait is explicit,
            // so the prep below runs while the tiles still stream in.
            const uint32_t nraw = owner ? gqa + 2 : gqa;
            const uint32_t qnbase = (uint32_t)(uintptr_t)qn;
            for (uint32_t j = w; j < nraw; j += WAVES) {
                const float *src = j < gqa ? a.qg + (size_t)(g * gqa + j) * 2 * HD
                                 : j == gqa ? a.k + (size_t)g * HD : a.v + (size_t)g * HD;
                const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)src);
                const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)((uintptr_t)src >> 32));
                lds_dma16<true>(((uintptr_t)hi << 32) | lo, lane * 16, qnbase + j * 1024);
            }
            // this wave's raw-row DMAs, then 8 per tile
            const uint32_t my_raw = nraw > w ? (nraw - w + WAVES - 1) / WAVES : 0u;
            if (ntile > 0) issue_tile(0);
            if (ntile > 1) issue_tile(1);
            const uint32_t behind = (ntile > 0 ? 8u : 0u) + (ntile > 1 ? 8u : 0u);
            (void)my_raw;
            if (behind == 16) asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
            else if (behind == 8) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
            else dma_wait();
            __syncthreads();
            float xr[ATT_MAXG + 1];
#pragma unroll
            for (uint32_t hh = 0; hh <= ATT_MAXG; hh++) xr[hh] = hh < nraw && hh <= gqa ? qn[hh * 256 + t] : 0.0f;
            const float vraw = owner ? qn[(gqa + 1) * 256 + t] : 0.0f;
            __syncthreads();
            att_prep(xr, gqa, owner ? gqa + 1 : gqa, a.q_norm, a.k_norm, a.eps, pos, a.theta_scale, a.rope_dims, qf,
                     qn, rot, pred);
            if (owner) vnew[t] = f2h(vraw);
        }
        if (owner) {
            const uint16_t kh = f2h(qf[gqa * 256 + t]), vh = vnew[t];
            knew[t] = kh;
            st_coh(a.kc + (size_t)pos * RW + (size_t)g * HD + t, kh);
            st_coh(a.vc + (size_t)pos * RW + (size_t)g * HD + t, vh);
        }
        if (ts && item == rel) ts[1] = wall_clock64();
        if (t < gqa) { mrun[t] = -INFINITY; lrun[t] = 0.0; }
        double acc[ATT_MAXG];
#pragma unroll
        for (int hh = 0; hh < ATT_MAXG; hh++) acc[hh] = 0.0;

        for (uint32_t j = 0; j < ntile; j++) {
            const uint32_t t0 = kv0 + j * ATT_TILE, bo = (j & 1) * ATT_TILE * 256;
            if (j == 0) {
                dma_wait();   // (also the owner's cache stores)
            } else {
                // tile j landed; tile j+1 (issued last step) may still fly
                if (j + 1 < ntile) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
                else dma_wait();
            }
            __syncthreads();
            // scores: thread (r = t/8, part = t%8) covers dims [32 part, 32 part + 32)
            // of every q head slot (k converted once); the eight parts are
            // combined with DPP in the butterfly order (d0+d1)+(d2+d3) + ...
            // Slots past gqa compute on stale rows and are weighted 0 below.
            // sc is position-major: sc[r * ATT_MAXG + hh].
            {
                const uint32_t r = t >> 3, part = t & 7;
                const LDS uint16_t *kr = ((owner && t0 + r == (uint32_t)pos) ? knew : kb + bo + r * 256) + part * 32;
                double kd[32];
#pragma unroll
                for (int i = 0; i < 32; i += 8) {
                    const u32x4 u = *reinterpret_cast<const LDS u32x4 *>(kr + i);
                    const uint32_t uw[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                    for (int k = 0; k < 4; k++) {
                        kd[i + 2 * k] = (double)h2f((uint16_t)(uw[k] & 0xffff));
                        kd[i + 2 * k + 1] = (double)h2f((uint16_t)(uw[k] >> 16));
                    }
                }
                // dims ascending per head; the eight head chains interleaved
                double d[ATT_MAXG];
#pragma unroll
                for (uint32_t hh = 0; hh < ATT_MAXG; hh++) d[hh] = 0.0;
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    f32x4 qv[ATT_MAXG];
#pragma unroll
                    for (uint32_t hh = 0; hh < ATT_MAXG; hh++)
                        qv[hh] = reinterpret_cast<const LDS f32x4 *>(qf + hh * 256 + part * 32)[i];
#pragma unroll
                    for (uint32_t hh = 0; hh < ATT_MAXG; hh++) {
                        d[hh] = fma((double)qv[hh].x, kd[4 * i], d[hh]);
                        d[hh] = fma((double)qv[hh].y, kd[4 * i + 1], d[hh]);
                        d[hh] = fma((double)qv[hh].z, kd[4 * i + 2], d[hh]);
                        d[hh] = fma((double)qv[hh].w, kd[4 * i + 3], d[hh]);
                    }
                }
#pragma unroll
                for (uint32_t hh = 0; hh < ATT_MAXG; hh++) d[hh] += dpp_d<DPP_XOR1>(d[hh]);
#pragma unroll
                for (uint32_t hh = 0; hh < ATT_MAXG; hh++) d[hh] += dpp_d<DPP_XOR2>(d[hh]);
#pragma unroll
                for (uint32_t hh = 0; hh < ATT_MAXG; hh++) d[hh] += dpp_d<DPP_HALF_MIRROR>(d[hh]);
                // lane `part` stores head slot `part`
                double mine = d[0];
#pragma unroll
                for (uint32_t hh = 1; hh < ATT_MAXG; hh++) mine = part == hh ? d[hh] : mine;
                sc[r * ATT_MAXG + part] = (t0 + r < kv1) ? mine * (double)a.scale : -INFINITY;
            }
            __syncthreads();
            // online softmax: head slot hh = t/32 over its 32 rows (lane r);
            // max and sum over the 32 lanes with DPP plus one cross-row step
            {
                const uint32_t hh = t / ATT_TILE, r = t % ATT_TILE;
                const double s = sc[r * ATT_MAXG + hh];
                double mt = s;
                mt = fmax(mt, dpp_d<DPP_XOR1>(mt));
                mt = fmax(mt, dpp_d<DPP_XOR2>(mt));
                mt = fmax(mt, dpp_d<DPP_HALF_MIRROR>(mt));
                mt = fmax(mt, dpp_d<DPP_MIRROR>(mt));
                mt = fmax(mt, __shfl_xor(mt, 16, 64));
                const double mo = mrun[hh];
                const double mn = fmax(mo, mt);
                const double wgt = (s == -INFINITY || hh >= gqa) ? 0.0 : exp(s - mn);
                double ws = wgt;
#pragma unroll
                for (int o = 16; o > 0; o >>= 1) ws += __shfl_xor(ws, o, 64);
                sc[r * ATT_MAXG + hh] = wgt;
                if (r == 0 && hh < gqa) {
                    const double cf = (mo == -INFINITY) ? 0.0 : exp(mo - mn);
                    corr[hh] = cf;
                    lrun[hh] = lrun[hh] * cf + ws;
                    mrun[hh] = mn;
                }
            }
            __syncthreads();
            // V accumulation: thread t owns dim t; per row, v converted once
            // and the eight slot weights read as four broadcast 16-byte loads
#pragma unroll
            for (uint32_t hh = 0; hh < ATT_MAXG; hh++)
                if (hh < gqa) acc[hh] = acc[hh] * corr[hh];
#pragma unroll 4
            for (uint32_t r = 0; r < ATT_TILE; r++) {
                const LDS uint16_t *vr = (owner && t0 + r == (uint32_t)pos) ? vnew : vb + bo + r * 256;
                const double v = (double)h2f(vr[t]);
                typedef double f64x2 __attribute__((ext_vector_type(2)));
                const LDS f64x2 *w2 = reinterpret_cast<const LDS f64x2 *>(sc + r * ATT_MAXG);
                f64x2 wv[ATT_MAXG / 2];
#pragma unroll
                for (uint32_t k = 0; k < ATT_MAXG / 2; k++) wv[k] = w2[k];
#pragma unroll
                for (uint32_t hh = 0; hh < ATT_MAXG; hh++) acc[hh] = fma(wv[hh / 2][hh % 2], v, acc[hh]);
            }
            __syncthreads();
            // the tile after next into the buffer just freed
            if (j + 2 < ntile) issue_tile(j + 2);
        }

        if (ts && item == rel) ts[2] = wall_clock64();
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
