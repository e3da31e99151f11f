// C ABI: status/error plumbing, standalone op entry points, synthetic data,
// and the host control plane (core/host.cpp:19-245 in the reference).
//
// Control-plane design on MI355X: the reference keeps one cooperative kernel
// resident and rings a host-mapped doorbell per pass.  Here a pass (or a run
// of greedy passes) is one cooperative launch of the interpreter: a launch
// costs microseconds against a ~2.5 ms pass, needs no PCIe polling from the
// device, and a faulty program ends with its kernel instead of leaving a
// resident grid behind.  The lifecycle and status semantics of host_init /
// upload / launch / run_pass / shutdown / destroy are kept.
#include <hip/hip_runtime.h>

#include <chrono>
#include <cstdarg>
#include <cstddef>
#include <cstdio>
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "internal.h"
#include "synth.h"

namespace sinter {

static thread_local std::string g_last_error;

int set_error(int status, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return status;
}

bool hip_ok(hipError_t e, const char *what) {
    if (e == hipSuccess) return true;
    set_error(SINTER_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
    return false;
}

// Per-device state of the standalone op entry points: the error cell and a
// ring of instruction slots (an op reads its instruction from device memory,
// as the interpreter does).  A slot is reused after OP_RING launches; the
// copy into it is ordered on the caller's stream.
constexpr unsigned OP_RING = 256;
struct OpSlot {
    sinter_instr ins;
    GemvPlan plan;
    uint32_t cuts[PLAN_CUTS];
};
struct OpDev {
    unsigned *err = nullptr;
    OpSlot *ring = nullptr;
    unsigned next = 0;
};

static OpDev *op_dev() {
    static std::mutex mu;
    static std::map<int, OpDev> devs;
    int dev = 0;
    if (!hip_ok(hipGetDevice(&dev), "op state: hipGetDevice")) return nullptr;
    std::lock_guard<std::mutex> lk(mu);
    OpDev &d = devs[dev];
    if (!d.err) {
        char *p = nullptr;
        if (!hip_ok(hipMalloc(&p, 256 + OP_RING * sizeof(OpSlot)), "op state: hipMalloc")) return nullptr;
        if (!hip_ok(hipMemset(p, 0, 256), "op state: hipMemset")) return nullptr;
        d.err = reinterpret_cast<unsigned *>(p);
        d.ring = reinterpret_cast<OpSlot *>(p + 256);
    }
    return &d;
}

unsigned *op_err_cell() {
    OpDev *d = op_dev();
    return d ? d->err : nullptr;
}

static OpSlot *op_slot() {
    OpDev *d = op_dev();
    if (!d) return nullptr;
    static std::mutex mu;
    std::lock_guard<std::mutex> lk(mu);
    return d->ring + (d->next++ % OP_RING);
}

static bool al16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

static int vdot(int t) {
    return (t == SINTER_Q4_K || t == SINTER_Q6_K) ? SINTER_Q8_K
         : (t == SINTER_Q8_0) ? SINTER_Q8_0
         : (t == SINTER_BF16) ? SINTER_BF16
         : (t == SINTER_F32) ? SINTER_F32 : -1;
}

int validate_gemv(const sinter_gemv_args &a, const char **why) {
    auto bad = [&](const char *w) { *why = w; return SINTER_ERR_ARG; };
    if (a.n_seg < 1 || a.n_seg > SINTER_GEMV_MAX_SEG) return bad("n_seg out of range");
    if (a.K == 0 || a.K % 256 || a.K > (1u << 20)) return bad("K must be a positive multiple of 256, at most 2^20");
    const int vt = vdot(a.seg[0].type);
    if (vt < 0) return bad("unsupported weight type");
    const uint64_t need = act_bytes(vt, a.K);
    if (need > QBUF_BYTES) return bad("K too large for the activation buffer");
    switch (a.pro) {
    case SINTER_PRO_PLAIN:
        if (!a.x || !al16(a.x)) return bad("x must be a 16-byte aligned device pointer");
        break;
    case SINTER_PRO_RMSNORM:
        if (!a.x || !al16(a.x) || !a.norm_w || !al16(a.norm_w)) return bad("x / norm_w missing or unaligned");
        break;
    case SINTER_PRO_GATED:
    case SINTER_PRO_GATED_G:
        if (!a.x || !al16(a.x) || !a.norm_w || !a.aux || !al16(a.aux)) return bad("gated: x / norm_w / z");
        if (a.gn_log2d < 2 || a.gn_log2d > 8) return bad("gated: head width must be 4..256");
        break;
    case SINTER_PRO_EMBED:
        if (!a.aux || !a.token || !a.norm_w || !al16(a.norm_w) || a.aux_rows == 0)
            return bad("embed: rows / token / norm_w / aux_rows");
        if (sinter_row_bytes_dev(a.aux_type, a.K) == 0) return bad("embed: type");
        if (a.x_out && !al16(a.x_out)) return bad("embed: x_out unaligned");
        break;
    default: return bad("unknown prologue");
    }
    // the prologue stages x (and the norm weights or z) as f32 in the LDS
    // scratch region; the gated norms also the head-width norm weights, in
    // its last KiB
    const bool gated_pro = a.pro == SINTER_PRO_GATED || a.pro == SINTER_PRO_GATED_G;
    if ((uint64_t)a.K * 4 * (a.pro == SINTER_PRO_PLAIN ? 1u : 2u) + (gated_pro ? 1024u : 0u) > BIG_BYTES)
        return bad("K too large for the prologue's staging area");
    // the term ring (gemv.h): R rows of P terms per wave must hold the rows
    // one 64-item step touches plus one
    {
        const uint32_t ipr = a.K / item_elems(a.seg[0].type);
        bool any_swig = false;
        for (int s = 0; s < a.n_seg; s++) any_swig |= a.seg[s].epi == SINTER_EPI_SWIGLU;
        // one group of GEMV_DMAX 64-item steps (32 for SwiGLU pairs)
        const uint32_t si = any_swig ? 32u : 64u;
        const uint32_t cap = any_swig ? RING_CAP / 2 : RING_CAP, tpr = (si * GEMV_DMAX - 1) / ipr + 2;
        const uint32_t P = ring_row(ipr, cap, tpr), R = cap / P;
        if (R < tpr) return bad("rows too long for the term ring");
    }
    for (int s = 0; s < a.n_seg; s++) {
        const sinter_gemv_seg &g = a.seg[s];
        if (vdot(g.type) != vt) return bad("segments must share one vec_dot type");
        if (!g.w || !al16(g.w) || !g.y) return bad("segment weights must be 16-byte aligned; y required");
        if ((uint64_t)g.rows * sinter_row_bytes_dev(g.type, a.K) >= (1ull << 32))
            return bad("segment larger than 4 GiB");
        switch (g.epi) {
        case SINTER_EPI_STORE: case SINTER_EPI_SILU: break;
        case SINTER_EPI_RESID: if (!g.aux) return bad("resid: aux"); break;
        case SINTER_EPI_SWIGLU: if (!g.w2 || !al16(g.w2)) return bad("swiglu: w2"); break;
        case SINTER_EPI_ARGMAX: if (!a.epi_ws) return bad("argmax: epi_ws"); break;
        case SINTER_EPI_CONV:
            if (!g.w2 || !g.aux || g.dconv < 2 || g.dconv > 4) return bad("conv: w2 / aux / dconv (2..4 taps)");
            break;
        default: return bad("unknown epilogue");
        }
    }
    return SINTER_OK;
}

// Byte-balanced row cut w of n over the concatenated, byte-weighted row
// space of segments [s0, s1) (a SwiGLU row weighs both matrices), as a
// global row.  Any monotone split is correct; this one balances bytes.
static uint32_t row_cut(const sinter_gemv_args &a, int s0, int s1, uint32_t row0, uint64_t w, uint64_t n) {
    uint64_t total = 0;
    for (int s = s0; s < s1; s++)
        total += (uint64_t)a.seg[s].rows * sinter_row_bytes_dev(a.seg[s].type, a.K) *
                 (a.seg[s].epi == SINTER_EPI_SWIGLU ? 2u : 1u);
    uint32_t rows = row0;
    if (w >= n) {
        for (int s = s0; s < s1; s++) rows += a.seg[s].rows;
        return rows;
    }
    const uint64_t target = total * w / n;
    uint64_t acc = 0;
    for (int s = s0; s < s1; s++) {
        const uint64_t rb = sinter_row_bytes_dev(a.seg[s].type, a.K) * (a.seg[s].epi == SINTER_EPI_SWIGLU ? 2u : 1u);
        const uint64_t sb = (uint64_t)a.seg[s].rows * rb;
        if (target < acc + sb) return rows + (uint32_t)((target - acc + rb / 2) / rb);
        acc += sb;
        rows += a.seg[s].rows;
    }
    return rows;
}

void build_gemv_plan(const sinter_gemv_args &a, uint32_t nblk, GemvPlan &p, uint32_t *cuts, const uint32_t *bw) {
    std::memset(&p, 0, sizeof p);
    p.ok = 1;
    p.n_seg = a.n_seg;
    p.ipr = a.K / item_elems(a.seg[0].type);
    p.vt = (uint32_t)vdot(a.seg[0].type);
    p.feat = feat_x(p.vt);
    bool any_swig = false;
    uint32_t base = 0;
    for (int s = 0; s < a.n_seg; s++) {
        const sinter_gemv_seg &g = a.seg[s];
        const bool sw = g.epi == SINTER_EPI_SWIGLU;
        GemvSegPlan &q = p.seg[s];
        q.wa = reinterpret_cast<uint64_t>(g.w);
        q.wb = sw ? reinterpret_cast<uint64_t>(g.w2) : 0;
        q.rows = g.rows;
        q.base = base;
        q.type = g.type;
        p.feat |= feat_w(g.type);
        q.swig = sw ? 1u : 0u;
        q.ib = item_bytes(g.type);
        q.y = reinterpret_cast<uint64_t>(g.y);
        q.aux = reinterpret_cast<uint64_t>(g.aux);
        q.w2 = reinterpret_cast<uint64_t>(g.w2);
        q.epi = g.epi;
        q.dconv = g.dconv;
        any_swig |= sw;
        if (g.epi == SINTER_EPI_ARGMAX) p.any_argmax = 1;
        base += g.rows;
    }
    p.total_rows = base;
    p.mipr = 0xFFFFFFFFu / p.ipr;
    p.q64 = 64 / p.ipr;
    p.r64 = 64 % p.ipr;
    p.q32 = 32 / p.ipr;
    p.r32 = 32 % p.ipr;
    const uint32_t cap = any_swig ? RING_CAP / 2 : RING_CAP;
    p.P = ring_row(p.ipr, cap, ((any_swig ? 32u : 64u) * GEMV_DMAX - 1) / p.ipr + 2);
    p.R = cap / p.P;
    p.mR = 0xFFFFFFFFu / p.R;

    // wave cuts.  Every segment gets whole waves, in proportion to its bytes
    // (at least one), so that a wave's rows are one streaming loop over one
    // matrix; rows are byte-balanced inside a segment.  With fewer waves than
    // segments, the cuts balance bytes over all rows and a wave streams the
    // segments of its range one after another.
    const uint32_t nw = nblk * WAVES;
    int rs[SINTER_GEMV_MAX_SEG + 1], nruns = 0;
    for (int s = 0; s < a.n_seg; s++)
        rs[nruns++] = s;
    rs[nruns] = a.n_seg;
    if ((uint32_t)nruns > nw) {
        for (uint32_t w = 0; w <= nw; w++) cuts[w] = row_cut(a, 0, a.n_seg, 0, w, nw);   // (shares ignored)
        return;
    }
    uint64_t rb[SINTER_GEMV_MAX_SEG], total = 0;
    for (int r = 0; r < nruns; r++) {
        rb[r] = 0;
        for (int s = rs[r]; s < rs[r + 1]; s++)
            rb[r] += (uint64_t)a.seg[s].rows * sinter_row_bytes_dev(a.seg[s].type, a.K) * (p.seg[s].swig ? 2u : 1u);
        total += rb[r];
    }
    // largest remainder, at least one wave per run
    uint32_t nwr[SINTER_GEMV_MAX_SEG], used = 0;
    double frac[SINTER_GEMV_MAX_SEG];
    for (int r = 0; r < nruns; r++) {
        const double qv = total ? (double)nw * (double)rb[r] / (double)total : 0.0;
        nwr[r] = std::max(1u, (uint32_t)qv);
        frac[r] = qv - (double)(uint32_t)qv;
        used += nwr[r];
    }
    while (used > nw) {   // the minimum of one wave pushed the total over
        int big = -1;
        for (int r = 0; r < nruns; r++)
            if (nwr[r] > 1 && (big < 0 || nwr[r] > nwr[big])) big = r;
        nwr[big]--;
        used--;
    }
    while (used < nw) {
        int best = 0;
        for (int r = 1; r < nruns; r++)
            if (frac[r] > frac[best]) best = r;
        nwr[best]++;
        frac[best] = -1.0;
        used++;
    }
    // inside a run, wave w's share of the bytes is proportional to its
    // block's weight bw (uniform without one)
    uint32_t w0 = 0, row0 = 0;
    for (int r = 0; r < nruns; r++) {
        uint64_t tw = 0;
        for (uint32_t w = 0; w < nwr[r]; w++) tw += bw ? bw[(w0 + w) / WAVES] : 1u;
        uint64_t cw = 0;
        for (uint32_t w = 0; w < nwr[r]; w++) {
            cuts[w0 + w] = row_cut(a, rs[r], rs[r + 1], row0, cw, tw);
            cw += bw ? bw[(w0 + w) / WAVES] : 1u;
        }
        w0 += nwr[r];
        for (int s = rs[r]; s < rs[r + 1]; s++) row0 += a.seg[s].rows;
    }
    cuts[nw] = row0;
}

template <class T>
static int run_one(int kind, const T &args, uint32_t blocks, void *stream) {
    if (blocks == 0 || blocks > 65535) return set_error(SINTER_ERR_ARG, "blocks must be 1..65535");
    if (kind == SINTER_OP_GEMV && blocks > PLAN_MAX_BLOCKS)
        return set_error(SINTER_ERR_ARG, "gemv: at most %u blocks", PLAN_MAX_BLOCKS);
    unsigned *err = op_err_cell();
    if (!err) return SINTER_ERR_HIP;
    static thread_local OpSlot host;
    std::memset(&host.ins, 0, sizeof host.ins);
    std::memset(&host.plan, 0, sizeof host.plan);
    host.ins.kind = (uint16_t)kind;
    host.ins.block_lo = 0;
    host.ins.block_hi = (uint16_t)blocks;
    std::memcpy(host.ins.payload, &args, sizeof args);
    size_t bytes = offsetof(OpSlot, cuts);
    if (kind == SINTER_OP_GEMV) {
        sinter_gemv_args g;
        std::memcpy(&g, host.ins.payload, sizeof g);
        build_gemv_plan(g, blocks, host.plan, host.cuts, nullptr);
        bytes += (size_t)(blocks * WAVES + 1) * 4;
    }
    OpSlot *slot = op_slot();
    if (!slot) return SINTER_ERR_HIP;
    // pageable source: the copy is staged before hipMemcpyAsync returns
    if (!hip_ok(hipMemcpyAsync(slot, &host, bytes, hipMemcpyHostToDevice, (hipStream_t)stream), "op upload"))
        return SINTER_ERR_HIP;
    if (!hip_ok(launch_op(&slot->ins, &slot->plan, slot->cuts, blocks, err, (hipStream_t)stream,
                          kind == SINTER_OP_ATTN_DECODE), "op launch"))
        return SINTER_ERR_HIP;
    return SINTER_OK;
}

}  // namespace sinter

using namespace sinter;

extern "C" {

const char *sinter_last_error(void) { return g_last_error.c_str(); }

// Rig precheck (tests/devinfo.cu in the reference): runtime version, device
// name, CU count, LDS, cooperative support, interpreter occupancy.
int sinter_device_info(int device, char *buf, size_t n) {
    if (!buf || n == 0) return set_error(SINTER_ERR_ARG, "device_info: buffer");
    int rt = 0, drv = 0, coop = 0, per_cu = -1;
    hipError_t e1 = hipRuntimeGetVersion(&rt);
    hipError_t e2 = hipDriverGetVersion(&drv);
    hipDeviceProp_t p;
    std::memset(&p, 0, sizeof p);
    hipError_t e3 = hipGetDeviceProperties(&p, device);
    hipError_t e4 = hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, device);
    hipError_t e5 = hipSetDevice(device);
    void *probe = nullptr;
    hipError_t e6 = hipMalloc(&probe, 4096);
    if (e6 == hipSuccess) (void)hipFree(probe);
    hipError_t e7 = interp_max_blocks(&per_cu);
    std::snprintf(buf, n,
                  "runtime %d driver %d | %s (%s) CUs %d LDS/block %zu coop %d | interp blocks/CU %d | "
                  "errors: version %s, props %s, attr %s, setdev %s, malloc %s, occupancy %s",
                  rt, drv, p.name, p.gcnArchName, p.multiProcessorCount, (size_t)p.sharedMemPerBlock, coop, per_cu,
                  hipGetErrorString(e1 ? e1 : e2), hipGetErrorString(e3), hipGetErrorString(e4),
                  hipGetErrorString(e5), hipGetErrorString(e6), hipGetErrorString(e7));
    return (e3 || e5 || e6 || e7) ? set_error(SINTER_ERR_HIP, "%s", buf) : SINTER_OK;
}
int sinter_abi_version(void) { return SINTER_ABI_VERSION; }
size_t sinter_row_bytes(int type, int64_t k) { return sinter_row_bytes_dev(type, k); }

int sinter_op_gemv(const sinter_gemv_args *a, uint32_t blocks, void *stream) {
    if (!a) return set_error(SINTER_ERR_ARG, "null args");
    const char *why = "";
    if (validate_gemv(*a, &why) != SINTER_OK) return set_error(SINTER_ERR_ARG, "gemv: %s", why);
    return run_one(SINTER_OP_GEMV, *a, blocks, stream);
}

int sinter_op_gdn_step(const sinter_gdn_args *a, uint32_t blocks, void *stream) {
    if (!a || !a->qkv || !a->alpha || !a->beta || !a->dt_bias || !a->ssm_a || !a->state || !a->o)
        return set_error(SINTER_ERR_ARG, "gdn: null pointer");
    const uint32_t D = a->d, cols = a->cols;
    const uint32_t tpc = cols ? BLOCK_THREADS / cols : 0;
    if (!(D == 64 || D == 128 || D == 256) || !cols || D % cols || BLOCK_THREADS % cols || !tpc || tpc > 64 ||
        D % tpc || (D / tpc) % 4 || D / tpc > 32 || !a->hk || a->hv % a->hk || !al16(a->state))
        return set_error(SINTER_ERR_ARG, "gdn: unsupported shape (D=%u cols=%u hk=%u hv=%u)", D, cols, a->hk, a->hv);
    return run_one(SINTER_OP_GDN_STEP, *a, blocks, stream);
}

size_t sinter_attn_part_len(uint32_t nq, uint32_t nkv, uint32_t hd, uint32_t n_chunks) {
    if (!nkv || !n_chunks) return 0;
    return (size_t)nkv * n_chunks * (nq / nkv) * att_rec(hd);
}

uint32_t sinter_attn_count_len(uint32_t nkv, uint32_t n_chunks) {
    return nkv * n_chunks;
}

// KV cache element types the attention op reads (0 means f16)
static bool kv_type_ok(uint32_t t) { return t == 0 || t == SINTER_F16 || t == SINTER_Q8_0; }

int sinter_op_attn_decode(const sinter_attn_args *a, uint32_t blocks, void *stream) {
    if (!a || !a->qg || !a->k || !a->v || !a->q_norm || !a->k_norm || !a->kc || !a->vc || !a->part || !a->count ||
        !a->out || !a->pass_cell)
        return set_error(SINTER_ERR_ARG, "attn: null pointer");
    if (a->hd != 256 || !a->nkv || a->nq % a->nkv || a->nq / a->nkv > 8 || !a->n_chunks || a->n_chunks > 64 ||
        a->rope_dims > a->hd ||
        a->rope_dims % 8 || !al16(a->kc) || !al16(a->vc) || !kv_type_ok(a->kv_type))
        return set_error(SINTER_ERR_ARG, "attn: unsupported shape or KV type (hd=%u nq=%u nkv=%u kv_type=%u)", a->hd,
                         a->nq, a->nkv, a->kv_type);
    // one (kv head, chunk) item per workgroup, all of them resident (the
    // chunks of a kv head wait for each other before merging)
    if ((uint64_t)a->nkv * a->n_chunks > blocks)
        return set_error(SINTER_ERR_ARG, "attn: blocks (%u) must be >= nkv * n_chunks (%u)", blocks,
                         a->nkv * a->n_chunks);
    return run_one(SINTER_OP_ATTN_DECODE, *a, blocks, stream);
}

int sinter_op_attn_decode_noalloc(const sinter_attn_args *a, uint32_t blocks, void *stream) {
    if (!a || !a->qg || !a->k || !a->v || !a->q_norm || !a->k_norm || !a->kc || !a->vc || !a->out || !a->pass_cell)
        return set_error(SINTER_ERR_ARG, "attn_noalloc: null pointer");
    if (a->part || a->count)
        return set_error(SINTER_ERR_ARG, "attn_noalloc: part and count must be NULL (the library supplies them)");
    if (a->hd != 256 || !a->nkv || a->nq % a->nkv || a->nq / a->nkv > 8 || !a->n_chunks || a->n_chunks > 64 ||
        a->rope_dims > a->hd || a->rope_dims % 8 || !al16(a->kc) || !al16(a->vc) || !kv_type_ok(a->kv_type))
        return set_error(SINTER_ERR_ARG, "attn_noalloc: unsupported shape or KV type (hd=%u nq=%u nkv=%u kv_type=%u)",
                         a->hd, a->nq, a->nkv, a->kv_type);
    if ((uint64_t)a->nkv * a->n_chunks > blocks || blocks > PLAN_MAX_BLOCKS)
        return set_error(SINTER_ERR_ARG, "attn_noalloc: blocks (%u) must be >= nkv * n_chunks (%u) and <= %u", blocks,
                         a->nkv * a->n_chunks, PLAN_MAX_BLOCKS);
    return attn_noalloc(*a, blocks, (hipStream_t)stream);
}

int sinter_copy_calibration(int device, size_t bytes, int reps) {
    if (bytes == 0 || reps < 1) return set_error(SINTER_ERR_ARG, "copy_calibration: bytes / reps");
    if (!hip_ok(hipSetDevice(device), "copy_calibration: device")) return SINTER_ERR_HIP;
    void *a = nullptr, *b = nullptr;
    int rc = SINTER_OK;
    if (!hip_ok(hipMalloc(&a, bytes), "copy_calibration: alloc") || !hip_ok(hipMalloc(&b, bytes), "copy_calibration: alloc") ||
        !hip_ok(hipMemset(a, 1, bytes), "copy_calibration: fill"))
        rc = SINTER_ERR_HIP;
    for (int i = 0; rc == SINTER_OK && i < reps; i++)
        if (!hip_ok(hipMemcpy(b, a, bytes, hipMemcpyDeviceToDevice), "copy_calibration: copy")) rc = SINTER_ERR_HIP;
    if (rc == SINTER_OK && !hip_ok(hipDeviceSynchronize(), "copy_calibration: sync")) rc = SINTER_ERR_HIP;
    if (a) (void)hipFree(a);
    if (b) (void)hipFree(b);
    return rc;
}

int sinter_litmus_barrier(uint32_t blocks, uint32_t epochs, int mode, uint64_t counts[3]) {
    if (!counts || mode < 0) return set_error(SINTER_ERR_ARG, "litmus: counts / mode");
    return litmus_barrier(blocks, epochs, (uint32_t)mode, counts);
}

int sinter_op_error(uint32_t *code, uint32_t *aux) {
    unsigned *err = op_err_cell();
    if (!err) return set_error(SINTER_ERR_HIP, "no error cell");
    if (!hip_ok(hipDeviceSynchronize(), "synchronize")) return SINTER_ERR_HIP;
    unsigned h[2] = {0, 0};
    if (!hip_ok(hipMemcpy(h, err, 8, hipMemcpyDeviceToHost), "error cell read")) return SINTER_ERR_HIP;
    if (!hip_ok(hipMemset(err, 0, 8), "error cell clear")) return SINTER_ERR_HIP;
    // the no-allocation op's cell on this device, when it has run here
    if (unsigned *e2 = noalloc_err_cell()) {
        unsigned h2[2] = {0, 0};
        const unsigned zero[2] = {0, 0};
        if (!hip_ok(hipMemcpy(h2, e2, 8, hipMemcpyDeviceToHost), "error cell read") ||
            !hip_ok(hipMemcpy(e2, zero, 8, hipMemcpyHostToDevice), "error cell clear"))
            return SINTER_ERR_HIP;
        if (!h[0]) { h[0] = h2[0]; h[1] = h2[1]; }
    }
    if (code) *code = h[0];
    if (aux) *aux = h[1];
    return SINTER_OK;
}

int sinter_argmax_ws_create(uint32_t blocks, int32_t *pass_cell, int32_t *history, uint32_t history_cap,
                            sinter_argmax_ws **out_dev) {
    if (!out_dev || !pass_cell || blocks == 0) return set_error(SINTER_ERR_ARG, "argmax ws: args");
    char *mem = nullptr;
    const size_t bytes = 256 + (size_t)blocks * 8 + 256;
    if (!hip_ok(hipMalloc(&mem, bytes), "argmax ws alloc")) return SINTER_ERR_HIP;
    if (!hip_ok(hipMemset(mem, 0, bytes), "argmax ws clear")) return SINTER_ERR_HIP;
    sinter_argmax_ws h;
    std::memset(&h, 0, sizeof h);
    h.count = reinterpret_cast<uint32_t *>(mem + 128);
    h.part_val = reinterpret_cast<float *>(mem + 256);
    h.part_idx = reinterpret_cast<int32_t *>(mem + 256 + (size_t)blocks * 4);
    h.pass_cell = pass_cell;
    h.history = history;
    h.history_cap = history_cap;
    h.capacity = blocks;
    if (!hip_ok(hipMemcpy(mem, &h, sizeof h, hipMemcpyHostToDevice), "argmax ws upload")) return SINTER_ERR_HIP;
    *out_dev = reinterpret_cast<sinter_argmax_ws *>(mem);
    return SINTER_OK;
}

void sinter_argmax_ws_destroy(sinter_argmax_ws *dev) {
    if (dev) (void)hipFree(dev);
}

uint64_t sinter_seed(uint64_t config_id, const char *name, int64_t layer) {
    uint64_t h = 1469598103934665603ull;  // FNV-1a over the name
    for (const char *p = name ? name : ""; *p; p++) { h ^= (uint8_t)*p; h *= 1099511628211ull; }
    return sx_mix(sx_mix(config_id) ^ h ^ sx_mix((uint64_t)layer + 0x5151));
}

int sinter_synth(int dev, void *dst, int kind, int type, int64_t rows, int64_t k, uint64_t seed, float a, float b,
                 void *stream) {
    if (!dst || rows < 0 || k < 0) return set_error(SINTER_ERR_ARG, "synth: args");
    const bool weight = kind == SINTER_SYN_WEIGHT || kind == SINTER_SYN_Q8_0_CFG1;
    if (weight) {
        if (k % 256) return set_error(SINTER_ERR_ARG, "synth: k must be a multiple of 256");
        if (kind == SINTER_SYN_Q8_0_CFG1 && type != SINTER_Q8_0) return set_error(SINTER_ERR_ARG, "synth: cfg1 is Q8_0");
        if (!(type == SINTER_Q4_K || type == SINTER_Q6_K || type == SINTER_Q8_0 || type == SINTER_BF16 ||
              type == SINTER_F16 || type == SINTER_F32))
            return set_error(SINTER_ERR_ARG, "synth: type");
    } else if (kind == SINTER_SYN_NORMAL_Q8_0) {
        if (k % 32) return set_error(SINTER_ERR_ARG, "synth: q8_0 k must be a multiple of 32");
    } else if (kind != SINTER_SYN_NORMAL && kind != SINTER_SYN_UNIFORM && kind != SINTER_SYN_NORMAL_F16) {
        return set_error(SINTER_ERR_ARG, "synth: kind");
    }
    const uint64_t n_units = weight ? (uint64_t)rows * (uint64_t)(k / 256)
                           : kind == SINTER_SYN_NORMAL_Q8_0 ? (uint64_t)rows * (uint64_t)(k / 32)
                           : (uint64_t)rows * (uint64_t)k;
    if (dev) {
        if (!hip_ok(launch_synth(dst, kind, type, n_units, seed, a, b, (hipStream_t)stream), "synth launch"))
            return SINTER_ERR_HIP;
        return SINTER_OK;
    }
    const unsigned nt = std::max(1u, std::min(64u, std::thread::hardware_concurrency()));
    std::vector<std::thread> th;
    for (unsigned w = 0; w < nt; w++) {
        th.emplace_back([=]() {
            const uint64_t lo = n_units * w / nt, hi = n_units * (w + 1) / nt;
            uint8_t *d = static_cast<uint8_t *>(dst);
            for (uint64_t i = lo; i < hi; i++) {
                if (weight) {
                    const uint32_t gb = sx_group_bytes(type);
                    sx_weight_group(seed, i, type, kind == SINTER_SYN_Q8_0_CFG1, d + i * gb);
                } else if (kind == SINTER_SYN_NORMAL) {
                    reinterpret_cast<float *>(d)[i] = a + b * sx_normal(seed, i);
                } else if (kind == SINTER_SYN_UNIFORM) {
                    reinterpret_cast<float *>(d)[i] = a + (b - a) * sx_unit(seed, i);
                } else if (kind == SINTER_SYN_NORMAL_Q8_0) {
                    sx_q8_0_normal_block(seed, i, b, d + i * 34);
                } else {
                    reinterpret_cast<uint16_t *>(d)[i] = sx_f2h(b * sx_normal(seed, i));
                }
            }
        });
    }
    for (auto &t : th) t.join();
    return SINTER_OK;
}

}  // extern "C"

// ----------------------------------------------------------------- host control plane

// control cells: error cell, pass cell, then the grid barrier's flags (one
// word per workgroup, up to 1024; the region is 8 KiB)
static constexpr size_t CELL_GROUPS = 4096, CELL_GROUP_BYTES = 64 * 128, CELL_BYTES = CELL_GROUPS + CELL_GROUP_BYTES;

struct sinter_host {
    int device = -1;
    hipStream_t stream = nullptr;
    sinter_instr *d_prog = nullptr;
    GemvPlan *d_plans = nullptr;          // [n_instr]
    uint32_t *d_cuts = nullptr;           // [n_instr][PLAN_CUTS]
    uint32_t n_instr = 0, epoch_stride = 0;
    uint32_t feat = FEAT_ALL;             // the uploaded program's feature set (isa.h)
    unsigned *d_cells = nullptr;          // [32] err[2] | byte 1024 pass cell |
                                          // byte CELL_GROUPS: grid barrier flags (4 B per workgroup)
    sinter_pass_cell *d_pass = nullptr;
    int32_t *d_history = nullptr;
    uint32_t history_cap = 0;
    long long *d_pass_cycles = nullptr;
    unsigned pass_cycles_cap = 0;
    uint32_t passes_done = 0;
    long long *d_op_cycles = nullptr;
    unsigned long long *d_trace = nullptr;  // caller-owned, consumed by the next launch
    uint32_t blocks = 0;
    uint64_t spin_limit = 0;
    uint64_t clock_khz = 0;
    bool launched = false;
    bool profile_ops = false;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;  // bracket every interpreter launch
    float last_ms = 0.0f;
    // launch inputs for the next launch (set_pos), the launch record in
    // pinned host memory, and the barrier epoch the flags hold after the last
    // launch (valid only after a launch that ran all its passes)
    int32_t pend_pos = 0;
    bool have_pos = false;
    unsigned *out = nullptr;            // [seq, token, pos, err]
    uint32_t seq = 0;
    unsigned epoch = 0;
    bool epoch_ok = false;
    uint32_t pass_barriers = 0;         // grid barriers per pass: the program's BOUNDARYs + the pass end
    std::vector<sinter_instr> prog;       // host copy of the uploaded program
};

// Wait until the work queued on s has finished, or timeout_ms passed
// (SINTER_ERR_TIMEOUT; SINTER_ERR_HIP on a device error).  A launch runs for
// milliseconds and the caller needs its result at once, so the stream is
// polled without sleeping (yielding the core between queries) for the first
// WAIT_SPIN_MS -- a sleeping poll adds its sleep quantum plus the scheduler's
// wake-up latency to every pass -- and with 100 us sleeps after that.
static constexpr double WAIT_SPIN_MS = 2000.0;
static int wait_stream(hipStream_t s, double timeout_ms, const char *what) {
    const auto t0 = std::chrono::steady_clock::now();
    const auto deadline = t0 + std::chrono::duration<double, std::milli>(timeout_ms);
    const auto spin_end = t0 + std::chrono::duration<double, std::milli>(WAIT_SPIN_MS);
    for (;;) {
        const hipError_t q = hipStreamQuery(s);
        if (q == hipSuccess) return SINTER_OK;
        if (q != hipErrorNotReady) return hip_ok(q, what) ? SINTER_OK : SINTER_ERR_HIP;
        const auto now = std::chrono::steady_clock::now();
        if (now > deadline) return SINTER_ERR_TIMEOUT;
        if (now < spin_end) std::this_thread::yield();
        else std::this_thread::sleep_for(std::chrono::microseconds(100));
    }
}

// One launch of n_passes passes.  cell_set / token: the pass cell fields the
// kernel writes before its first barrier (bit 0 token, bit 1 pos -- the
// pending set_pos --, bit 2 steps = 0).  The barrier flags are zeroed only
// when their epoch is unknown (the first launch, or one that stopped early);
// otherwise the epochs continue from the last launch's.  The result comes
// back through the launch record in pinned host memory; the device error
// cell is read only when the record is missing (a launch that stopped early).
static int run_launch(sinter_host *h, uint32_t n_passes, double timeout_ms, uint32_t cell_set = 0,
                      int32_t token = 0) {
    InterpCtl ctl;
    std::memset(&ctl, 0, sizeof ctl);
    ctl.cell = h->d_pass;
    ctl.cell_token = token;
    ctl.cell_pos = h->pend_pos;
    ctl.cell_set = cell_set | (h->have_pos ? 2u : 0u);
    ctl.out = h->out;
    ctl.seq = ++h->seq;
    if (ctl.seq == 0) ctl.seq = ++h->seq;   // (0 never marks a record)
    ctl.flags = h->d_cells + CELL_GROUPS / 4;
    ctl.err = h->d_cells + 32;
    ctl.pass_cycles = h->d_pass_cycles;
    ctl.pass_cycles_cap = h->pass_cycles_cap;
    ctl.pass_base = h->passes_done;
    ctl.op_cycles = h->profile_ops ? h->d_op_cycles : nullptr;
    ctl.trace = h->d_trace;
    h->d_trace = nullptr;
    ctl.spin_limit = h->spin_limit;
    ctl.plans = h->d_plans;
    ctl.cuts = h->d_cuts;
    ctl.n_instr = h->n_instr;
    ctl.n_passes = n_passes;
    if (!h->epoch_ok) {
        if (!hip_ok(hipMemsetAsync(h->d_cells + CELL_GROUPS / 4, 0, CELL_GROUP_BYTES, h->stream),
                    "barrier flags reset"))
            return SINTER_RUN_ERR;
        h->epoch = 0;
    }
    ctl.epoch0 = h->epoch;
    h->epoch_ok = false;   // until this launch is seen to finish every pass
    h->have_pos = false;
    if (!hip_ok(hipEventRecord(h->ev0, h->stream), "event")) return SINTER_RUN_ERR;
    if (!hip_ok(launch_interp(h->d_prog, ctl, h->blocks, h->stream, h->feat), "cooperative launch"))
        return SINTER_RUN_ERR;
    if (!hip_ok(hipEventRecord(h->ev1, h->stream), "event")) return SINTER_RUN_ERR;
    h->passes_done += n_passes;
    // wait with a watchdog; the kernel's own barrier spin limit bounds it too
    const int ws = wait_stream(h->stream, timeout_ms, "interpreter");
    if (ws == SINTER_ERR_TIMEOUT) {
        set_error(SINTER_ERR_TIMEOUT, "watchdog: pass did not finish in %.1f ms", timeout_ms);
        return SINTER_RUN_TIMEOUT;
    }
    if (ws != SINTER_OK) return SINTER_RUN_ERR;
    (void)hipEventElapsedTime(&h->last_ms, h->ev0, h->ev1);
    const volatile unsigned *rec = h->out;
    if (rec[0] == ctl.seq && rec[3] == 0) {
        h->epoch = ctl.epoch0 + n_passes * h->pass_barriers;
        h->epoch_ok = true;
        return SINTER_RUN_OK;
    }
    // stopped early (or an error in the record): the device's error cell
    unsigned e[2] = {0, 0};
    if (!hip_ok(hipMemcpy(e, h->d_cells + 32, 8, hipMemcpyDeviceToHost), "error cell")) return SINTER_RUN_ERR;
    if (e[0]) {
        set_error(SINTER_ERR_DEVICE, "device error %u (aux %u)", e[0], e[1]);
        return SINTER_RUN_ERR;
    }
    return set_error(SINTER_ERR_DEVICE, "launch ended without its record (seq %u, record %u)", ctl.seq, rec[0]),
           SINTER_RUN_ERR;
}

extern "C" {

int sinter_host_init(sinter_host **out, int device, unsigned pass_cycles_cap) {
    if (!out) return set_error(SINTER_ERR_ARG, "null out");
    *out = nullptr;
    if (!hip_ok(hipSetDevice(device), "hipSetDevice")) return SINTER_ERR_HIP;
    hipDeviceProp_t p;
    if (!hip_ok(hipGetDeviceProperties(&p, device), "device properties")) return SINTER_ERR_HIP;
    int coop = 0;
    (void)hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, device);
    int per_cu = 0;
    if (!hip_ok(interp_max_blocks(&per_cu), "occupancy")) return SINTER_ERR_HIP;
    if (!coop || per_cu < 1)
        return set_error(SINTER_ERR_DEVICE, "device %d cannot run the interpreter envelope (coop %d, blocks/CU %d)",
                         device, coop, per_cu);
    sinter_host *h = new sinter_host();
    h->device = device;
    h->blocks = (uint32_t)p.multiProcessorCount;  // one workgroup per CU
    int khz = 0;
    (void)hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, device);
    h->clock_khz = khz > 0 ? (uint64_t)khz : 100000;
    h->spin_limit = h->clock_khz * 1000ull * 10ull;  // 10 s
    bool ok = hip_ok(hipStreamCreateWithFlags(&h->stream, hipStreamNonBlocking), "stream") &&
              hip_ok(hipEventCreate(&h->ev0), "event") && hip_ok(hipEventCreate(&h->ev1), "event") &&
              hip_ok(hipMalloc(&h->d_cells, CELL_BYTES), "cells") && hip_ok(hipMemset(h->d_cells, 0, CELL_BYTES), "cells clear") &&
              hip_ok(hipHostMalloc(reinterpret_cast<void **>(&h->out), 64, hipHostMallocCoherent), "launch record");
    if (ok) std::memset(h->out, 0, 64);
    if (ok) h->d_pass = reinterpret_cast<sinter_pass_cell *>(reinterpret_cast<char *>(h->d_cells) + 1024);
    h->pass_cycles_cap = pass_cycles_cap;
    if (ok && pass_cycles_cap) {
        ok = hip_ok(hipMalloc(&h->d_pass_cycles, (size_t)pass_cycles_cap * 8), "pass cycles") &&
             hip_ok(hipMemset(h->d_pass_cycles, 0, (size_t)pass_cycles_cap * 8), "pass cycles clear");
    }
    if (ok)
        ok = hip_ok(hipMalloc(&h->d_op_cycles, SINTER_OP_KIND_COUNT * 8), "op cycles") &&
             hip_ok(hipMemset(h->d_op_cycles, 0, SINTER_OP_KIND_COUNT * 8), "op cycles clear");
    if (!ok) {
        sinter_host_destroy(h);
        return SINTER_ERR_HIP;
    }
    // token history of greedy runs (the argmax epilogue appends to it)
    if (!hip_ok(hipMalloc(&h->d_history, 65536 * 4), "history")) { sinter_host_destroy(h); return SINTER_ERR_HIP; }
    h->history_cap = 65536;
    *out = h;
    return SINTER_OK;
}

int sinter_host_upload(sinter_host *h, const sinter_instr *prog, uint32_t n_instr, uint32_t epoch_stride) {
    if (!h || !prog || n_instr == 0) return set_error(SINTER_ERR_ARG, "upload: args");
    if (h->launched) return set_error(SINTER_ERR_STATE, "upload after launch");
    for (uint32_t i = 0; i < n_instr; i++) {
        const sinter_instr &in = prog[i];
        if (in.kind != SINTER_OP_BOUNDARY && in.kind != SINTER_OP_NOP && in.kind < SINTER_OP_KIND_COUNT &&
            (in.block_lo >= in.block_hi || in.block_hi > h->blocks))
            return set_error(SINTER_ERR_ARG, "instruction %u: block range [%u,%u) outside the %u-block grid", i,
                             in.block_lo, in.block_hi, h->blocks);
        if (in.kind == SINTER_OP_GEMV) {
            sinter_gemv_args a;
            std::memcpy(&a, in.payload, sizeof a);
            const char *why = "";
            if (validate_gemv(a, &why) != SINTER_OK)
                return set_error(SINTER_ERR_ARG, "instruction %u (gemv): %s", i, why);
        }
    }
    std::vector<GemvPlan> plans(n_instr);
    std::vector<uint32_t> cuts((size_t)n_instr * PLAN_CUTS, 0u);
    // the feature set the program needs: every GEMV's activation and weight
    // types, every attention op's KV cache type
    uint32_t feat = 0;
    for (uint32_t i = 0; i < n_instr; i++) {
        std::memset(&plans[i], 0, sizeof(GemvPlan));
        if (prog[i].kind == SINTER_OP_ATTN_DECODE) {
            sinter_attn_args a;
            std::memcpy(&a, prog[i].payload, sizeof a);
            feat |= feat_kv(a.kv_type);
        }
        if (prog[i].kind != SINTER_OP_GEMV) continue;
        sinter_gemv_args a;
        std::memcpy(&a, prog[i].payload, sizeof a);
        build_gemv_plan(a, prog[i].block_hi - prog[i].block_lo, plans[i], cuts.data() + (size_t)i * PLAN_CUTS, nullptr);
        feat |= plans[i].feat;
    }
    if (h->d_prog) (void)hipFree(h->d_prog);
    if (h->d_plans) (void)hipFree(h->d_plans);
    if (h->d_cuts) (void)hipFree(h->d_cuts);
    h->d_prog = nullptr;
    h->d_plans = nullptr;
    h->d_cuts = nullptr;
    h->n_instr = 0;
    if (!hip_ok(hipMalloc(&h->d_prog, (size_t)n_instr * sizeof(sinter_instr)), "program alloc") ||
        !hip_ok(hipMalloc(&h->d_plans, (size_t)n_instr * sizeof(GemvPlan)), "plan alloc") ||
        !hip_ok(hipMalloc(&h->d_cuts, cuts.size() * 4), "cuts alloc"))
        return SINTER_ERR_HIP;
    if (!hip_ok(hipMemcpy(h->d_prog, prog, (size_t)n_instr * sizeof(sinter_instr), hipMemcpyHostToDevice),
                "program upload") ||
        !hip_ok(hipMemcpy(h->d_plans, plans.data(), (size_t)n_instr * sizeof(GemvPlan), hipMemcpyHostToDevice),
                "plan upload") ||
        !hip_ok(hipMemcpy(h->d_cuts, cuts.data(), cuts.size() * 4, hipMemcpyHostToDevice), "cuts upload"))
        return SINTER_ERR_HIP;
    h->n_instr = n_instr;
    h->epoch_stride = epoch_stride;
    h->pass_barriers = 1;
    for (uint32_t i = 0; i < n_instr; i++) h->pass_barriers += prog[i].kind == SINTER_OP_BOUNDARY ? 1u : 0u;
    h->epoch_ok = false;
    // SINTER_INTERP=general (a diagnostic): launch the general interpreter
    // whatever the program's types
    const char *force = std::getenv("SINTER_INTERP");
    h->feat = (force && std::strcmp(force, "general") == 0) ? (uint32_t)FEAT_ALL : feat;
    h->prog.assign(prog, prog + n_instr);
    return SINTER_OK;
}

const char *sinter_host_kernel(const sinter_host *h) {
    return h && h->n_instr ? interp_kernel_name(h->feat) : nullptr;
}

int sinter_host_set_gemv_shares(sinter_host *h, uint32_t instr, const float *share, uint32_t n) {
    if (!h || !h->d_cuts || instr >= h->n_instr || !share) return set_error(SINTER_ERR_ARG, "set_gemv_shares: args");
    const sinter_instr &in = h->prog[instr];
    if (in.kind != SINTER_OP_GEMV) return set_error(SINTER_ERR_ARG, "set_gemv_shares: instruction %u is not a GEMV", instr);
    const uint32_t nblk = in.block_hi - in.block_lo;
    if (n != nblk) return set_error(SINTER_ERR_ARG, "set_gemv_shares: %u shares for %u blocks", n, nblk);
    // weights in 1/4096 of the mean share, each in [1/16, 16] of it
    double sum = 0.0;
    for (uint32_t b = 0; b < n; b++) {
        if (!(share[b] > 0.0f) || !std::isfinite(share[b]))
            return set_error(SINTER_ERR_ARG, "set_gemv_shares: share %u not positive and finite", b);
        sum += share[b];
    }
    std::vector<uint32_t> bw(n);
    for (uint32_t b = 0; b < n; b++)
        bw[b] = (uint32_t)std::lround(std::min(16.0, std::max(1.0 / 16.0, share[b] * n / sum)) * 4096.0);
    sinter_gemv_args a;
    std::memcpy(&a, in.payload, sizeof a);
    GemvPlan plan;
    std::vector<uint32_t> cuts(PLAN_CUTS, 0u);
    build_gemv_plan(a, nblk, plan, cuts.data(), bw.data());
    // a monotone split of all rows from row 0 (what the kernel requires)
    bool mono = cuts[0] == 0 && cuts[nblk * WAVES] == plan.total_rows;
    for (uint32_t w = 0; w < nblk * WAVES; w++) mono = mono && cuts[w] <= cuts[w + 1];
    if (!mono) return set_error(SINTER_ERR_ARG, "set_gemv_shares: cuts not monotone");
    // the kernel reads the cuts of a launch from device memory: none may run
    if (!hip_ok(hipStreamSynchronize(h->stream), "set_gemv_shares sync") ||
        !hip_ok(hipMemcpy(h->d_cuts + (size_t)instr * PLAN_CUTS, cuts.data(), (size_t)(nblk * WAVES + 1) * 4,
                          hipMemcpyHostToDevice), "cuts upload"))
        return SINTER_ERR_HIP;
    return SINTER_OK;
}

int sinter_host_launch(sinter_host *h) {
    if (!h || !h->d_prog) return set_error(SINTER_ERR_STATE, "launch before upload");
    h->launched = true;
    return SINTER_OK;
}

int sinter_host_run_pass(sinter_host *h, int32_t token, double timeout_ms) {
    if (!h || !h->launched) return set_error(SINTER_ERR_STATE, "run_pass before launch"), SINTER_RUN_ERR;
    return run_launch(h, 1, timeout_ms, 1u, token);
}

int sinter_host_run_passes(sinter_host *h, int32_t token, uint32_t n_passes, int32_t *tokens_out, double timeout_ms) {
    if (!h || !h->launched) return set_error(SINTER_ERR_STATE, "run_passes before launch"), SINTER_RUN_ERR;
    if (n_passes == 0 || n_passes > h->history_cap) return set_error(SINTER_ERR_ARG, "n_passes"), SINTER_RUN_ERR;
    const int rs = run_launch(h, n_passes, timeout_ms, 1u | 4u, token);
    if (rs != SINTER_RUN_OK) return rs;
    if (tokens_out &&
        !hip_ok(hipMemcpy(tokens_out, h->d_history, (size_t)n_passes * 4, hipMemcpyDeviceToHost), "history read"))
        return SINTER_RUN_ERR;
    return SINTER_RUN_OK;
}

int sinter_host_shutdown(sinter_host *h, double timeout_ms) {
    if (!h) return set_error(SINTER_ERR_ARG, "null host");
    if (!h->launched) return SINTER_OK;
    const int ws = wait_stream(h->stream, timeout_ms, "shutdown");
    if (ws == SINTER_ERR_TIMEOUT) return set_error(SINTER_ERR_TIMEOUT, "shutdown watchdog");
    if (ws != SINTER_OK) return ws;
    h->launched = false;
    return SINTER_OK;
}

void sinter_host_destroy(sinter_host *h) {
    if (!h) return;
    if (h->stream) (void)hipStreamSynchronize(h->stream);
    if (h->d_prog) (void)hipFree(h->d_prog);
    if (h->d_plans) (void)hipFree(h->d_plans);
    if (h->d_cuts) (void)hipFree(h->d_cuts);
    if (h->d_cells) (void)hipFree(h->d_cells);
    if (h->d_pass_cycles) (void)hipFree(h->d_pass_cycles);
    if (h->d_op_cycles) (void)hipFree(h->d_op_cycles);
    if (h->d_history) (void)hipFree(h->d_history);
    if (h->out) (void)hipHostFree(h->out);
    if (h->ev0) (void)hipEventDestroy(h->ev0);
    if (h->ev1) (void)hipEventDestroy(h->ev1);
    if (h->stream) (void)hipStreamDestroy(h->stream);
    delete h;
}

int sinter_host_read_pass_cycles(sinter_host *h, long long *out, unsigned count) {
    if (!h || !out || !h->d_pass_cycles || count > h->pass_cycles_cap) return set_error(SINTER_ERR_ARG, "pass cycles");
    if (!hip_ok(hipMemcpy(out, h->d_pass_cycles, (size_t)count * 8, hipMemcpyDeviceToHost), "pass cycles read"))
        return SINTER_ERR_HIP;
    return SINTER_OK;
}

int sinter_host_trace_next(sinter_host *h, unsigned long long *dev_buf, size_t words) {
    if (!h || !dev_buf) return set_error(SINTER_ERR_ARG, "trace: args");
    if (words < ((size_t)h->n_instr + 1) * h->blocks * 4) return set_error(SINTER_ERR_ARG, "trace: buffer too small");
    h->d_trace = dev_buf;
    return SINTER_OK;
}

int sinter_host_reset_op_cycles(sinter_host *h) {
    if (!h) return set_error(SINTER_ERR_ARG, "null host");
    h->profile_ops = true;
    return hip_ok(hipMemset(h->d_op_cycles, 0, SINTER_OP_KIND_COUNT * 8), "op cycles reset") ? SINTER_OK
                                                                                              : SINTER_ERR_HIP;
}

int sinter_host_read_op_cycles(sinter_host *h, long long *out, unsigned count) {
    if (!h || !out || count > SINTER_OP_KIND_COUNT) return set_error(SINTER_ERR_ARG, "op cycles");
    return hip_ok(hipMemcpy(out, h->d_op_cycles, (size_t)count * 8, hipMemcpyDeviceToHost), "op cycles read")
               ? SINTER_OK
               : SINTER_ERR_HIP;
}

sinter_pass_cell *sinter_host_pass_cell(sinter_host *h) { return h ? h->d_pass : nullptr; }

float sinter_host_last_launch_ms(sinter_host *h) { return h ? h->last_ms : 0.0f; }

int32_t *sinter_host_history(sinter_host *h, uint32_t *cap) {
    if (!h) return nullptr;
    if (cap) *cap = h->history_cap;
    return h->d_history;
}

int sinter_host_error(sinter_host *h, uint32_t *code, uint32_t *aux) {
    if (!h) return set_error(SINTER_ERR_ARG, "null host");
    unsigned e[2] = {0, 0};
    if (!hip_ok(hipMemcpy(e, h->d_cells + 32, 8, hipMemcpyDeviceToHost), "error cell")) return SINTER_ERR_HIP;
    if (code) *code = e[0];
    if (aux) *aux = e[1];
    return SINTER_OK;
}

int sinter_host_grid(sinter_host *h, uint32_t *blocks, uint32_t *threads, uint32_t *lds_bytes) {
    if (!h) return set_error(SINTER_ERR_ARG, "null host");
    if (blocks) *blocks = h->blocks;
    if (threads) *threads = BLOCK_THREADS;
    if (lds_bytes) *lds_bytes = BIG_BYTES + QBUF_BYTES + HDR_CAP * 8 + 512;
    return SINTER_OK;
}

int sinter_host_set_grid(sinter_host *h, uint32_t blocks) {
    if (!h || blocks == 0 || blocks > CELL_GROUP_BYTES / 128 * 16) return set_error(SINTER_ERR_ARG, "set_grid: args");
    if (h->launched) return set_error(SINTER_ERR_STATE, "set_grid after launch");
    hipDeviceProp_t p;
    if (!hip_ok(hipGetDeviceProperties(&p, h->device), "device properties")) return SINTER_ERR_HIP;
    int per_cu = 0;
    if (!hip_ok(interp_max_blocks(&per_cu), "occupancy")) return SINTER_ERR_HIP;
    if (blocks > (uint32_t)(per_cu * p.multiProcessorCount))
        return set_error(SINTER_ERR_ARG, "set_grid: %u blocks exceed the co-resident limit %d", blocks,
                         per_cu * p.multiProcessorCount);
    h->blocks = blocks;
    h->epoch_ok = false;   // flags of workgroups that have not run yet
    return SINTER_OK;
}

int sinter_host_set_pos(sinter_host *h, int32_t pos) {
    if (!h) return set_error(SINTER_ERR_ARG, "null host");
    // the next launch's workgroups write it into the pass cell (no command
    // of its own on the stream)
    h->pend_pos = pos;
    h->have_pos = true;
    return SINTER_OK;
}

}  // extern "C"

namespace sinter {
int32_t host_last_token(const sinter_host *h) {
    return h && h->out ? (int32_t)((const volatile unsigned *)h->out)[1] : -1;
}
}  // namespace sinter
