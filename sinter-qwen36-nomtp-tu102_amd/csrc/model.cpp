// Model residency, state, and the pass program for one MI355X.
//
// Replaces, for this layout, the reference's harness residency/runtime
// (k0/harness.cpp:402-566), its packer (harness.cpp:668-1060) and the offline
// schedule compiler (k0/compile_schedule.py:358-703).  The whole model lives
// on one GPU (15.5 GB Q4_K_M-mix or ~54 GB bf16 of 288 GB HBM3E); the dual-GPU
// split and its exchange are gone.
//
// Pass program (per layer; B = grid barrier):
//   GEMV  pro=RMSNORM(attn_norm) [EMBED on layer 0]
//         GDN : qkv (EPI_CONV: conv+silu, conv state update) | z | alpha | beta
//         ATTN: q|gate | k | v
//   B
//   GDN_STEP (l2norm, gates, delta rule)  |  ATTN_DECODE (norm+rope, KV append,
//                                             split-K, merge, gate)
//   B
//   GEMV  pro=GATED(ssm_norm, z) for GDN / PLAIN for ATTN; ssm_out|attn_output, EPI_RESID -> H
//   B
//   GEMV  pro=RMSNORM(post_attention_norm); ffn_gate,ffn_up EPI_SWIGLU -> F
//   B
//   GEMV  pro=PLAIN; ffn_down EPI_RESID -> X
//   B
// then GEMV pro=RMSNORM(output_norm); output EPI_ARGMAX -> logits, token.
// 5 barriers per layer (the reference schedule has 15) plus the pass-end one.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <array>
#include <cmath>
#include <cstddef>
#include <cstring>
#include <string>
#include <vector>

#include "internal.h"
#include "synth.h"

using namespace sinter;

namespace {

struct Tensor {
    void *d = nullptr;
    size_t bytes = 0;
    int type = 0;
    int64_t rows = 0, k = 0;
};

// slot numbering shared with oracle/oracle.h
enum {
    S_ATTN_NORM = 0, S_POST_NORM, S_FFN_GATE, S_FFN_UP, S_FFN_DOWN,
    S_QKV = 5, S_Z, S_ALPHA, S_BETA, S_SSM_OUT, S_CONV_W, S_DT_BIAS, S_SSM_A, S_SSM_NORM,
    S_WQ = 5, S_WK, S_WV, S_WO, S_Q_NORM, S_K_NORM,
    NSLOT = 16
};

bool is_attn(const sinter_model_config &c, int il) {
    return c.attn_every > 0 && (il % c.attn_every) == c.attn_every - 1;
}

}  // namespace

// split-K chunks per kv head at most: one (kv head, chunk) item per
// workgroup, at most 64 (one merge lane per chunk)
static uint32_t attn_chunks(uint32_t blocks, uint32_t nkv) {
    return std::min(64u, std::max(1u, blocks / nkv));
}

struct sinter_model {
    sinter_model_config cfg{};
    int device = 0;
    uint32_t blocks = 0;
    sinter_host *host = nullptr;
    hipStream_t stream = nullptr;
    std::vector<std::array<Tensor, NSLOT>> W;
    Tensor embd, onorm, output;
    std::vector<std::array<Tensor, 2>> S;
    float *X = nullptr, *H = nullptr, *qkv = nullptr, *z = nullptr, *al = nullptr, *be = nullptr, *o = nullptr;
    float *ffn = nullptr, *qg = nullptr, *kk = nullptr, *vv = nullptr, *att = nullptr, *logits = nullptr;
    float *part = nullptr;
    unsigned *count = nullptr;
    sinter_argmax_ws *ws = nullptr;
    std::vector<sinter_instr> prog;
    uint32_t n_boundaries = 0;
    uint64_t weight_bytes = 0;
    std::vector<void *> allocs;
    uint64_t seed = 0;
    sinter_gguf *gg = nullptr;   // weights come from this file when set (else synthesised)
    const sinter_model_bindings *ext = nullptr;   // caller-owned weights and state (creation only)
    bool embed_outside = false;  // the caller writes the embedded row into X before each pass
    // batched prefill buffers for ubatches of up to pf_cap tokens (allocated
    // at the first batched prefill, kept until the model is destroyed)
    struct Prefill {
        uint32_t cap = 0;
        int32_t *tok = nullptr;
        float *x = nullptr, *qkv = nullptr, *conv = nullptr, *z = nullptr, *al = nullptr, *be = nullptr;
        float *o = nullptr, *work = nullptr, *qg = nullptr, *k = nullptr, *v = nullptr, *qr = nullptr;
        float *att = nullptr, *gate = nullptr, *up = nullptr, *part = nullptr;
        void *xq = nullptr;
    } pf;
};

namespace {

void *dalloc(sinter_model *m, size_t bytes) {
    void *p = nullptr;
    // 256 B of slack: tile loads round the last row up to 16 bytes
    const size_t sz = (bytes + 256 + 255) & ~(size_t)255;
    if (hipMalloc(&p, sz) != hipSuccess) return nullptr;
    if (hipMemsetAsync(p, 0, sz, m->stream) != hipSuccess) return nullptr;
    m->allocs.push_back(p);
    return p;
}

// GGUF tensor name of a weight: blk.<il>.<name>.weight (globals: <name>.weight)
std::string gguf_name(const char *name, int il) {
    std::string n = name;
    n = n == "ssm_dt_bias" ? "ssm_dt.bias" : n == "ssm_a" ? n : n + ".weight";
    return il >= 0 ? "blk." + std::to_string(il) + "." + n : n;
}

// The GGUF tensor for a weight of `rows` rows of k elements: it must exist
// with exactly that shape and a type the kernels read.  Returns its index
// (set_error and -1 otherwise).
int64_t gguf_lookup(sinter_model *m, const char *name, int il, int64_t rows, int64_t k, bool want_f32) {
    const std::string gn = gguf_name(name, il);
    const int64_t i = sinter_gguf_find(m->gg, gn.c_str());
    sinter_gguf_tensor t;
    if (i < 0 || sinter_gguf_get_tensor(m->gg, (uint64_t)i, &t) != SINTER_OK) {
        set_error(SINTER_ERR_ARG, "gguf: tensor %s missing", gn.c_str());
        return -1;
    }
    // weights: rows of k elements; f32 vectors (norms, conv taps [dconv x C]
    // with the taps of a channel contiguous): the element count
    const bool shape_ok = want_f32 ? (int64_t)(t.ne[0] * t.ne[1] * t.ne[2] * t.ne[3]) == rows * k
                                   : (int64_t)t.ne[0] == k && (int64_t)(t.ne[1] * t.ne[2] * t.ne[3]) == rows;
    if (!shape_ok) {
        set_error(SINTER_ERR_ARG, "gguf: tensor %s is %llux%llu, the model needs %lldx%lld", gn.c_str(),
                  (unsigned long long)t.ne[0], (unsigned long long)(t.ne[1] * t.ne[2] * t.ne[3]), (long long)k,
                  (long long)rows);
        return -1;
    }
    const bool ok = want_f32 ? t.type == SINTER_F32
                             : (t.type == SINTER_Q4_K || t.type == SINTER_Q6_K || t.type == SINTER_Q8_0 ||
                                t.type == SINTER_BF16 || t.type == SINTER_F32);
    if (!ok) {
        set_error(SINTER_ERR_ARG, "gguf: tensor %s has type %u, which the kernels do not read here", gn.c_str(), t.type);
        return -1;
    }
    return i;
}

bool upload(sinter_model *m, Tensor &t, int64_t gi) {
    sinter_gguf_tensor g;
    if (sinter_gguf_get_tensor(m->gg, (uint64_t)gi, &g) != SINTER_OK || g.nbytes != t.bytes) return false;
    return hip_ok(hipMemcpyAsync(t.d, g.data, t.bytes, hipMemcpyHostToDevice, m->stream), "gguf upload");
}

// A recurrent-state or KV-cache buffer: allocated (zeroed), or the caller's.
bool state_buffer(sinter_model *m, Tensor &t, int il, int s) {
    if (!m->ext) return (t.d = dalloc(m, t.bytes)) != nullptr;
    t.d = m->ext->states ? m->ext->states[(size_t)il * 2 + s] : nullptr;
    if (!t.d || (reinterpret_cast<uintptr_t>(t.d) & 15u)) {
        set_error(SINTER_ERR_ARG, "bound model: state %d of layer %d null or unaligned", s, il);
        return false;
    }
    return true;
}

// A bound model's pointer and type for tensor t of layer il (-1: the
// globals embd / onorm / output), numbered as sinter_model_tensor_info.
size_t ext_index(const sinter_model *m, const Tensor &t, int il) {
    if (il >= 0) return (size_t)il * NSLOT + (size_t)(&t - m->W[il].data());
    return (size_t)m->cfg.n_layer * NSLOT + (&t == &m->embd ? 0u : &t == &m->onorm ? 1u : 2u);
}

bool bind(sinter_model *m, Tensor &t, int il, int type, int64_t rows, int64_t k) {
    const size_t i = ext_index(m, t, il);
    t.d = m->ext->tensors[i];
    t.type = m->ext->types ? m->ext->types[i] : type;
    t.rows = rows;
    t.k = k;
    t.bytes = sinter_row_bytes_dev(t.type, k) * (size_t)rows;
    if (!t.d || (reinterpret_cast<uintptr_t>(t.d) & 15u) || t.bytes == 0) {
        set_error(SINTER_ERR_ARG, "bound model: tensor %zu (layer %d) null, unaligned or of a type the kernels do "
                  "not read", i, il);
        return false;
    }
    m->weight_bytes += t.bytes;
    return true;
}

bool make_weight(sinter_model *m, Tensor &t, const char *name, int il, int type, int64_t rows, int64_t k) {
    if (m->ext) return bind(m, t, il, type, rows, k);
    int64_t gi = -1;
    if (m->gg) {
        if ((gi = gguf_lookup(m, name, il, rows, k, false)) < 0) return false;
        sinter_gguf_tensor g;
        sinter_gguf_get_tensor(m->gg, (uint64_t)gi, &g);
        type = (int)g.type;
    }
    t.type = type;
    t.rows = rows;
    t.k = k;
    t.bytes = sinter_row_bytes_dev(type, k) * (size_t)rows;
    t.d = dalloc(m, t.bytes);
    if (!t.d) return false;
    m->weight_bytes += t.bytes;
    if (m->gg) return upload(m, t, gi);
    return launch_synth(t.d, SINTER_SYN_WEIGHT, type, (uint64_t)rows * (uint64_t)(k / 256),
                        sinter_seed(m->seed, name, il), 0.f, 0.f, m->stream) == hipSuccess;
}

bool make_vec(sinter_model *m, Tensor &t, const char *name, int il, int64_t n, int kind, float a, float b) {
    if (m->ext) return bind(m, t, il, SINTER_F32, 1, n) && (t.type == SINTER_F32 ||
                                                            (set_error(SINTER_ERR_ARG, "bound model: vector not f32"), false));
    int64_t gi = -1;
    if (m->gg && (gi = gguf_lookup(m, name, il, 1, n, true)) < 0) return false;
    t.type = SINTER_F32;
    t.rows = 1;
    t.k = n;
    t.bytes = (size_t)n * 4;
    t.d = dalloc(m, t.bytes);
    if (!t.d) return false;
    m->weight_bytes += t.bytes;
    if (m->gg) return upload(m, t, gi);
    return launch_synth(t.d, kind, SINTER_F32, (uint64_t)n, sinter_seed(m->seed, name, il), a, b, m->stream) ==
           hipSuccess;
}

sinter_instr mk_instr(uint16_t kind, uint32_t blocks, uint32_t dbg) {
    sinter_instr in;
    std::memset(&in, 0, sizeof in);
    in.kind = kind;
    in.block_lo = 0;
    in.block_hi = (uint16_t)blocks;
    in.dbg_node = dbg;
    return in;
}

template <class T>
void push(sinter_model *m, uint16_t kind, const T &args, uint32_t dbg) {
    sinter_instr in = mk_instr(kind, m->blocks, dbg);
    static_assert(sizeof(T) <= sizeof(in.payload), "payload");
    std::memcpy(in.payload, &args, sizeof args);
    m->prog.push_back(in);
}

void boundary(sinter_model *m) {
    m->prog.push_back(mk_instr(SINTER_OP_BOUNDARY, m->blocks, 0));
    m->n_boundaries++;
}

sinter_gemv_seg seg(const Tensor &w, float *y, int epi, const void *w2 = nullptr, float *aux = nullptr,
                    int dconv = 0) {
    sinter_gemv_seg s;
    std::memset(&s, 0, sizeof s);
    s.w = w.d;
    s.w2 = w2;
    s.y = y;
    s.aux = aux;
    s.rows = (uint32_t)w.rows;
    s.type = (uint8_t)w.type;
    s.epi = (uint8_t)epi;
    s.dconv = (uint8_t)dconv;
    return s;
}

// Steps 1-3 of layer il: mixer input projections (the embedding lookup when
// `embed`), the recurrent / attention core, the output projection with the
// residual H = X + W_out . a.
void push_mixer(sinter_model *m, int il, bool embed) {
    const sinter_model_config &c = m->cfg;
    const int E = c.n_embd, D = c.gdn_d, HD = c.head_dim;
    const sinter_pass_cell *pc = sinter_host_pass_cell(m->host);
    int log2d = 0;
    while ((1 << log2d) < D) log2d++;
    const auto &w = m->W[il];
    const bool at = is_attn(c, il);
    const uint32_t dbg = (uint32_t)il * 8;
    // 1. mixer input projections
    sinter_gemv_args g1;
    std::memset(&g1, 0, sizeof g1);
    g1.K = (uint32_t)E;
    g1.eps = c.eps;
    g1.norm_w = (const float *)w[S_ATTN_NORM].d;
    if (embed) {
        g1.pro = SINTER_PRO_EMBED;
        g1.aux = m->embd.d;
        g1.aux_type = (uint8_t)m->embd.type;
        g1.aux_rows = (uint32_t)m->embd.rows;
        g1.token = &pc->token;
        g1.x_out = m->X;
    } else {
        g1.pro = SINTER_PRO_RMSNORM;
        g1.x = m->X;
    }
    if (at) {
        g1.n_seg = 3;
        g1.seg[0] = seg(w[S_WQ], m->qg, SINTER_EPI_STORE);
        g1.seg[1] = seg(w[S_WK], m->kk, SINTER_EPI_STORE);
        g1.seg[2] = seg(w[S_WV], m->vv, SINTER_EPI_STORE);
    } else {
        g1.n_seg = 4;
        g1.seg[0] = seg(w[S_QKV], m->qkv, SINTER_EPI_CONV, w[S_CONV_W].d, (float *)m->S[il][0].d, c.conv_k);
        g1.seg[1] = seg(w[S_Z], m->z, SINTER_EPI_SILU);   // the gate silu(z), once
        g1.seg[2] = seg(w[S_ALPHA], m->al, SINTER_EPI_STORE);
        g1.seg[3] = seg(w[S_BETA], m->be, SINTER_EPI_STORE);
    }
    push(m, SINTER_OP_GEMV, g1, dbg + 0);
    boundary(m);
    // 2. recurrent / attention core
    if (at) {
        sinter_attn_args a;
        std::memset(&a, 0, sizeof a);
        a.qg = m->qg;
        a.k = m->kk;
        a.v = m->vv;
        a.q_norm = (const float *)w[S_Q_NORM].d;
        a.k_norm = (const float *)w[S_K_NORM].d;
        a.kc = m->S[il][0].d;
        a.vc = m->S[il][1].d;
        a.kv_type = (uint32_t)c.t_kv;
        a.part = m->part;
        a.count = m->count;
        a.out = m->att;
        a.pass_cell = &pc->token;
        a.nq = (uint32_t)c.attn_nq;
        a.nkv = (uint32_t)c.attn_nkv;
        a.hd = (uint32_t)HD;
        a.rope_dims = (uint32_t)c.rope_dims;
        a.n_ctx = (uint32_t)c.n_ctx;
        a.n_chunks = (uint32_t)c.attn_chunks;
        a.chunk_min = (uint32_t)c.attn_chunk_min;
        a.theta_scale = (float)std::pow((double)c.rope_base, -2.0 / (double)c.rope_dims);
        a.eps = c.eps;
        a.scale = 1.0f / std::sqrt((float)HD);
        push(m, SINTER_OP_ATTN_DECODE, a, dbg + 1);
    } else {
        sinter_gdn_args a;
        std::memset(&a, 0, sizeof a);
        a.qkv = m->qkv;
        a.alpha = m->al;
        a.beta = m->be;
        a.dt_bias = (const float *)w[S_DT_BIAS].d;
        a.ssm_a = (const float *)w[S_SSM_A].d;
        a.state = (float *)m->S[il][1].d;
        a.o = m->o;
        a.hk = (uint32_t)c.gdn_hk;
        a.hv = (uint32_t)c.gdn_hv;
        a.d = (uint32_t)D;
        // 32 columns per item: 128 items at 32 heads x 128, so half the
        // grid goes straight on to the next GEMV's first weight loads
        // (measured faster than 256 items of 16 columns)
        a.cols = D >= 128 ? 32u : 16u;
        a.eps = c.eps;
        a.scale = 1.0f / std::sqrt((float)D);
        push(m, SINTER_OP_GDN_STEP, a, dbg + 1);
    }
    boundary(m);
    // 3. mixer output projection + residual: H = X + W_out . a
    sinter_gemv_args g3;
    std::memset(&g3, 0, sizeof g3);
    g3.eps = c.eps;
    g3.n_seg = 1;
    if (at) {
        g3.K = (uint32_t)(c.attn_nq * HD);
        g3.pro = SINTER_PRO_PLAIN;
        g3.x = m->att;
        g3.seg[0] = seg(w[S_WO], m->H, SINTER_EPI_RESID, nullptr, m->X);
    } else {
        g3.K = (uint32_t)(c.gdn_hv * D);
        g3.pro = SINTER_PRO_GATED_G;
        g3.x = m->o;
        g3.norm_w = (const float *)w[S_SSM_NORM].d;
        g3.aux = m->z;
        g3.gn_log2d = (uint8_t)log2d;
        g3.seg[0] = seg(w[S_SSM_OUT], m->H, SINTER_EPI_RESID, nullptr, m->X);
    }
    push(m, SINTER_OP_GEMV, g3, dbg + 2);
    boundary(m);
}

// Steps 4-5 of layer il: FFN gate/up with SwiGLU, down with the residual
// X = H + W_down . f.
void push_ffn(sinter_model *m, int il) {
    const sinter_model_config &c = m->cfg;
    const int E = c.n_embd;
    const auto &w = m->W[il];
    const uint32_t dbg = (uint32_t)il * 8;
    // 4. FFN gate/up with SwiGLU
    sinter_gemv_args g4;
    std::memset(&g4, 0, sizeof g4);
    g4.K = (uint32_t)E;
    g4.eps = c.eps;
    g4.pro = SINTER_PRO_RMSNORM;
    g4.x = m->H;
    g4.norm_w = (const float *)w[S_POST_NORM].d;
    g4.n_seg = 1;
    g4.seg[0] = seg(w[S_FFN_GATE], m->ffn, SINTER_EPI_SWIGLU, w[S_FFN_UP].d);
    push(m, SINTER_OP_GEMV, g4, dbg + 3);
    boundary(m);
    // 5. FFN down + residual: X = H + W_down . f
    sinter_gemv_args g5;
    std::memset(&g5, 0, sizeof g5);
    g5.K = (uint32_t)c.n_ff;
    g5.eps = c.eps;
    g5.pro = SINTER_PRO_PLAIN;
    g5.x = m->ffn;
    g5.n_seg = 1;
    g5.seg[0] = seg(w[S_FFN_DOWN], m->X, SINTER_EPI_RESID, nullptr, m->H);
    push(m, SINTER_OP_GEMV, g5, dbg + 4);
    boundary(m);
}

void build_program(sinter_model *m) {
    const sinter_model_config &c = m->cfg;
    const int E = c.n_embd;
    m->prog.clear();
    m->n_boundaries = 0;
    for (int il = 0; il < c.n_layer; il++) {
        push_mixer(m, il, il == 0 && !m->embed_outside);
        push_ffn(m, il);
    }
    // head: final norm, logits, greedy argmax
    sinter_gemv_args gh;
    std::memset(&gh, 0, sizeof gh);
    gh.K = (uint32_t)E;
    gh.eps = c.eps;
    gh.pro = SINTER_PRO_RMSNORM;
    gh.x = m->X;
    gh.norm_w = (const float *)m->onorm.d;
    gh.epi_ws = m->ws;
    gh.n_seg = 1;
    gh.seg[0] = seg(m->output, m->logits, SINTER_EPI_ARGMAX);
    push(m, SINTER_OP_GEMV, gh, (uint32_t)c.n_layer * 8);
}

int check_config(const sinter_model_config &c) {
    if (c.n_layer < 1 || c.n_embd <= 0 || c.n_embd % 256 || c.n_ff % 256 || c.n_vocab < 1)
        return set_error(SINTER_ERR_ARG, "config: n_layer/n_embd/n_ff/n_vocab");
    if (c.gdn_hk < 1 || c.gdn_hv % c.gdn_hk || !(c.gdn_d == 64 || c.gdn_d == 128 || c.gdn_d == 256) || c.conv_k < 2 ||
        c.conv_k > 8 || ((2 * c.gdn_hk + c.gdn_hv) * c.gdn_d) % 256 || (c.gdn_hv * c.gdn_d) % 256)
        return set_error(SINTER_ERR_ARG, "config: gated-DeltaNet shape");
    if (c.head_dim != 256 || c.attn_nkv < 1 || c.attn_nq % c.attn_nkv || c.attn_nq / c.attn_nkv > 8 ||
        c.rope_dims > c.head_dim || c.rope_dims % 8 || c.n_ctx < 1)
        return set_error(SINTER_ERR_ARG, "config: attention shape");
    if (!(c.t_kv == 0 || c.t_kv == SINTER_F16 || c.t_kv == SINTER_Q8_0))
        return set_error(SINTER_ERR_ARG, "config: KV cache type must be F16 or Q8_0");
    if (c.attn_chunks < 0 || c.attn_chunks > 64 || c.attn_chunk_min < 0)
        return set_error(SINTER_ERR_ARG, "config: attn_chunks must be 0..64, attn_chunk_min >= 0");
    return SINTER_OK;
}

}  // namespace

extern "C" {

void sinter_model_destroy(sinter_model *m) {
    if (!m) return;
    if (m->stream) (void)hipStreamSynchronize(m->stream);
    if (m->host) sinter_host_destroy(m->host);
    for (void *p : m->allocs) (void)hipFree(p);
    if (m->ws) sinter_argmax_ws_destroy(m->ws);
    if (m->stream) (void)hipStreamDestroy(m->stream);
    delete m;
}

}  // extern "C"

// Allocate, fill (synthesise, or upload from gg) and program a model.
static int model_create(const sinter_model_config *cfg, int device, uint64_t seed, uint32_t blocks, sinter_gguf *gg,
                        sinter_model **out, const sinter_model_bindings *ext = nullptr) {
    if (!cfg || !out) return set_error(SINTER_ERR_ARG, "model: null argument");
    *out = nullptr;
    int rc = check_config(*cfg);
    if (rc) return rc;
    sinter_model *m = new sinter_model();
    m->cfg = *cfg;
    if (m->cfg.t_kv == 0) m->cfg.t_kv = SINTER_F16;
    m->device = device;
    m->seed = seed;
    m->gg = gg;
    m->ext = ext;
    m->embed_outside = ext && ext->embed_outside;
    auto fail = [&](int st) { m->gg = nullptr; m->ext = nullptr; sinter_model_destroy(m); return st; };
    if ((rc = sinter_host_init(&m->host, device, 1024)) != SINTER_OK) return fail(rc);
    uint32_t hb = 0;
    sinter_host_grid(m->host, &hb, nullptr, nullptr);
    m->blocks = blocks ? std::min(blocks, hb) : hb;
    if ((rc = sinter_host_set_grid(m->host, m->blocks)) != SINTER_OK) return fail(rc);
    // the split-K attention geometry (at most one chunk per workgroup and kv head)
    {
        const uint32_t cmax = attn_chunks(m->blocks, (uint32_t)m->cfg.attn_nkv);
        m->cfg.attn_chunks = m->cfg.attn_chunks ? (int32_t)std::min((uint32_t)m->cfg.attn_chunks, cmax) : (int32_t)cmax;
        if (m->cfg.attn_chunk_min == 0) m->cfg.attn_chunk_min = SINTER_ATTN_CHUNK_MIN;
    }
    if (!hip_ok(hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking), "model stream")) return fail(SINTER_ERR_HIP);
    const sinter_model_config &c = m->cfg;
    const int E = c.n_embd, F = c.n_ff, D = c.gdn_d, HK = c.gdn_hk, HV = c.gdn_hv;
    const int C = (2 * HK + HV) * D, VD = HV * D;
    const int NQ = c.attn_nq, NKV = c.attn_nkv, HD = c.head_dim, RW = NKV * HD;
    m->W.resize(c.n_layer);
    m->S.resize(c.n_layer);
    bool ok = true;
    for (int il = 0; il < c.n_layer && ok; il++) {
        auto &w = m->W[il];
        ok = ok && make_vec(m, w[S_ATTN_NORM], "attn_norm", il, E, SINTER_SYN_NORMAL, 1.0f, 0.02f);
        ok = ok && make_vec(m, w[S_POST_NORM], "post_attention_norm", il, E, SINTER_SYN_NORMAL, 1.0f, 0.02f);
        ok = ok && make_weight(m, w[S_FFN_GATE], "ffn_gate", il, c.t_default, F, E);
        ok = ok && make_weight(m, w[S_FFN_UP], "ffn_up", il, c.t_default, F, E);
        ok = ok && make_weight(m, w[S_FFN_DOWN], "ffn_down", il, c.t_ffn_down, E, F);
        if (is_attn(c, il)) {
            ok = ok && make_weight(m, w[S_WQ], "attn_q", il, c.t_default, (int64_t)NQ * 2 * HD, E);
            ok = ok && make_weight(m, w[S_WK], "attn_k", il, c.t_default, RW, E);
            ok = ok && make_weight(m, w[S_WV], "attn_v", il, c.t_attn_v, RW, E);
            ok = ok && make_weight(m, w[S_WO], "attn_output", il, c.t_default, E, (int64_t)NQ * HD);
            ok = ok && make_vec(m, w[S_Q_NORM], "attn_q_norm", il, HD, SINTER_SYN_NORMAL, 1.0f, 0.02f);
            ok = ok && make_vec(m, w[S_K_NORM], "attn_k_norm", il, HD, SINTER_SYN_NORMAL, 1.0f, 0.02f);
            Tensor &K = m->S[il][0], &V = m->S[il][1];
            // f16, or Q8_0 blocks of 32 (34 bytes)
            K.bytes = V.bytes = (size_t)c.n_ctx * (c.t_kv == SINTER_Q8_0 ? (size_t)RW / 32 * 34 : (size_t)RW * 2);
            K.type = V.type = c.t_kv;
            ok = ok && state_buffer(m, K, il, 0) && state_buffer(m, V, il, 1);
        } else {
            ok = ok && make_weight(m, w[S_QKV], "attn_qkv", il, c.t_default, C, E);
            ok = ok && make_weight(m, w[S_Z], "attn_gate", il, c.t_default, VD, E);
            ok = ok && make_weight(m, w[S_ALPHA], "ssm_alpha", il, c.t_default, HV, E);
            ok = ok && make_weight(m, w[S_BETA], "ssm_beta", il, c.t_default, HV, E);
            ok = ok && make_weight(m, w[S_SSM_OUT], "ssm_out", il, c.t_default, E, VD);
            ok = ok && make_vec(m, w[S_CONV_W], "ssm_conv1d", il, (int64_t)C * c.conv_k, SINTER_SYN_UNIFORM, -0.5f, 0.5f);
            ok = ok && make_vec(m, w[S_DT_BIAS], "ssm_dt_bias", il, HV, SINTER_SYN_UNIFORM, -6.9f, -2.3f);
            ok = ok && make_vec(m, w[S_SSM_A], "ssm_a", il, HV, SINTER_SYN_UNIFORM, -16.0f, -1.0f);
            ok = ok && make_vec(m, w[S_SSM_NORM], "ssm_norm", il, D, SINTER_SYN_NORMAL, 1.0f, 0.02f);
            Tensor &cs = m->S[il][0], &ss = m->S[il][1];
            cs.bytes = (size_t)C * (c.conv_k - 1) * 4;
            ss.bytes = (size_t)HV * D * D * 4;
            cs.type = ss.type = SINTER_F32;
            ok = ok && state_buffer(m, cs, il, 0) && state_buffer(m, ss, il, 1);
        }
    }
    if (!m->embed_outside) ok = ok && make_weight(m, m->embd, "token_embd", -1, c.t_embd, c.n_vocab, E);
    ok = ok && make_vec(m, m->onorm, "output_norm", -1, E, SINTER_SYN_NORMAL, 1.0f, 0.02f);
    // a GGUF without output.weight ties the head to the embedding
    const bool tied = gg && sinter_gguf_find(gg, "output.weight") < 0;
    ok = ok && make_weight(m, m->output, tied ? "token_embd" : "output", -1, c.t_output, c.n_vocab, E);
    auto fa = [&](size_t n) { return (float *)dalloc(m, n * 4); };
    ok = ok && (m->X = fa(E)) && (m->H = fa(E)) && (m->qkv = fa(C)) && (m->z = fa(VD)) && (m->al = fa(HV)) &&
         (m->be = fa(HV)) && (m->o = fa(VD)) && (m->ffn = fa(F)) && (m->qg = fa((size_t)NQ * 2 * HD)) &&
         (m->kk = fa(RW)) && (m->vv = fa(RW)) && (m->att = fa((size_t)NQ * HD)) &&
         (m->logits = ext && ext->logits ? ext->logits : fa(c.n_vocab));
    const uint32_t chunks = (uint32_t)c.attn_chunks;
    ok = ok && (m->part = (float *)dalloc(m, sinter_attn_part_len(NQ, NKV, HD, chunks) * 4));
    ok = ok && (m->count = (unsigned *)dalloc(m, (size_t)sinter_attn_count_len(NKV, chunks) * 4));
    if (!ok) {
        if (gg && std::strncmp(sinter_last_error(), "gguf", 4) == 0) return fail(SINTER_ERR_ARG);
        if (ext && std::strncmp(sinter_last_error(), "bound model", 11) == 0) return fail(SINTER_ERR_ARG);
        return fail(set_error(SINTER_ERR_NOMEM, "model: device allocation or synthesis failed"));
    }
    if (!hip_ok(hipStreamSynchronize(m->stream), "model synthesis")) return fail(SINTER_ERR_HIP);
    m->gg = nullptr;   // every byte is on the device now; the caller owns the file
    m->ext = nullptr;  // (the bound pointers live on in the tensors)
    uint32_t hcap = 0;
    int32_t *hist = sinter_host_history(m->host, &hcap);
    if ((rc = sinter_argmax_ws_create(m->blocks, &sinter_host_pass_cell(m->host)->token, hist, hcap, &m->ws)))
        return fail(rc);
    build_program(m);
    if ((rc = sinter_host_upload(m->host, m->prog.data(), (uint32_t)m->prog.size(), m->n_boundaries + 1)))
        return fail(rc);
    if ((rc = sinter_host_launch(m->host))) return fail(rc);
    *out = m;
    return SINTER_OK;
}

// The model shape of a GGUF file, from its tensor table (shapes are what the
// weights are) and, for the scalars no tensor carries, its metadata.
static int gguf_config(sinter_gguf *g, int32_t n_ctx, sinter_model_config *c) {
    auto tensor = [&](const std::string &n, sinter_gguf_tensor *t) {
        const int64_t i = sinter_gguf_find(g, n.c_str());
        return i >= 0 && sinter_gguf_get_tensor(g, (uint64_t)i, t) == SINTER_OK;
    };
    std::memset(c, 0, sizeof *c);
    sinter_gguf_tensor t;
    if (!tensor("token_embd.weight", &t)) return set_error(SINTER_ERR_ARG, "gguf: no token_embd.weight");
    c->n_embd = (int32_t)t.ne[0];
    c->n_vocab = (int32_t)t.ne[1];
    c->t_embd = (int32_t)t.type;
    char arch[128] = "";
    (void)sinter_gguf_kv_str(g, "general.architecture", arch, sizeof arch);
    const std::string a = arch;
    int64_t iv = 0;
    double fv = 0.0;
    // decoder blocks: blk.0 .. blk.N-1 with a mixer, less the multi-token
    // prediction blocks the decode graph does not run
    int n = 0;
    while (tensor("blk." + std::to_string(n) + ".attn_norm.weight", &t)) n++;
    if (sinter_gguf_kv_i64(g, (a + ".nextn_predict_layers").c_str(), &iv) == SINTER_OK && iv > 0 && iv < n) n -= (int)iv;
    c->n_layer = n;
    if (n < 1) return set_error(SINTER_ERR_ARG, "gguf: no decoder blocks");
    int first_attn = -1;
    for (int il = 0; il < n && first_attn < 0; il++)
        if (tensor("blk." + std::to_string(il) + ".attn_q.weight", &t)) first_attn = il;
    c->attn_every = first_attn + 1;
    for (int il = 0; il < n; il++) {
        const std::string b = "blk." + std::to_string(il) + ".";
        const bool at = tensor(b + "attn_q.weight", &t), dn = tensor(b + "ssm_a", &t);
        const bool want = first_attn >= 0 && il % c->attn_every == c->attn_every - 1;
        if (at == dn) return set_error(SINTER_ERR_ARG, "gguf: block %d is neither an attention nor a gated-DeltaNet block", il);
        if (at != want) return set_error(SINTER_ERR_ARG, "gguf: attention blocks are not every %d-th block", c->attn_every);
    }
    if (!tensor("blk.0.ffn_gate.weight", &t)) return set_error(SINTER_ERR_ARG, "gguf: no blk.0.ffn_gate.weight");
    c->n_ff = (int32_t)t.ne[1];
    c->t_default = (int32_t)t.type;
    if (tensor("blk.0.ffn_down.weight", &t)) c->t_ffn_down = (int32_t)t.type;
    int gdn = -1;   // the first gated-DeltaNet block
    for (int il = 0; il < n && gdn < 0; il++)
        if (!(c->attn_every > 0 && il % c->attn_every == c->attn_every - 1)) gdn = il;
    if (gdn >= 0) {
        const std::string b = "blk." + std::to_string(gdn) + ".";
        sinter_gguf_tensor qkv, cw;
        if (!tensor(b + "ssm_norm.weight", &t) || !tensor(b + "ssm_a", &cw) || !tensor(b + "attn_qkv.weight", &qkv))
            return set_error(SINTER_ERR_ARG, "gguf: gated-DeltaNet block %d lacks ssm_norm / ssm_a / attn_qkv", gdn);
        c->gdn_d = (int32_t)t.ne[0];
        c->gdn_hv = (int32_t)cw.ne[0];
        c->gdn_hk = (int32_t)(((int64_t)qkv.ne[1] - (int64_t)c->gdn_hv * c->gdn_d) / (2 * c->gdn_d));
        if (!tensor(b + "ssm_conv1d.weight", &t)) return set_error(SINTER_ERR_ARG, "gguf: no %sssm_conv1d.weight", b.c_str());
        c->conv_k = (int32_t)t.ne[0];
    }
    if (first_attn >= 0) {
        const std::string b = "blk." + std::to_string(first_attn) + ".";
        sinter_gguf_tensor q, k, v;
        if (!tensor(b + "attn_q_norm.weight", &t) || !tensor(b + "attn_q.weight", &q) || !tensor(b + "attn_k.weight", &k) ||
            !tensor(b + "attn_v.weight", &v))
            return set_error(SINTER_ERR_ARG, "gguf: attention block %d lacks q_norm / q / k / v", first_attn);
        c->head_dim = (int32_t)t.ne[0];
        c->attn_nq = (int32_t)(q.ne[1] / (2 * (uint64_t)c->head_dim));
        c->attn_nkv = (int32_t)(k.ne[1] / (uint64_t)c->head_dim);
        c->t_attn_v = (int32_t)v.type;
    }
    c->rope_dims = c->head_dim / 4;
    if (sinter_gguf_kv_i64(g, (a + ".rope.dimension_count").c_str(), &iv) == SINTER_OK) c->rope_dims = (int32_t)iv;
    c->rope_base = 10000.0f;
    if (sinter_gguf_kv_f64(g, (a + ".rope.freq_base").c_str(), &fv) == SINTER_OK) c->rope_base = (float)fv;
    c->eps = 1e-6f;
    if (sinter_gguf_kv_f64(g, (a + ".attention.layer_norm_rms_epsilon").c_str(), &fv) == SINTER_OK) c->eps = (float)fv;
    c->n_ctx = n_ctx;
    c->t_output = tensor("output.weight", &t) ? (int32_t)t.type : c->t_embd;
    return SINTER_OK;
}

extern "C" {

int sinter_model_create(const sinter_model_config *cfg, int device, uint64_t seed, uint32_t blocks,
                        sinter_model **out) {
    return model_create(cfg, device, seed, blocks, nullptr, out);
}

int sinter_model_create_bound(const sinter_model_config *cfg, int device, uint32_t blocks,
                              const sinter_model_bindings *b, sinter_model **out) {
    if (!b || !b->tensors) return set_error(SINTER_ERR_ARG, "bound model: no bindings");
    return model_create(cfg, device, 0, blocks, nullptr, out, b);
}

int sinter_model_config_from_gguf(sinter_gguf *g, int32_t n_ctx, sinter_model_config *cfg) {
    if (!g || !cfg || n_ctx < 1) return set_error(SINTER_ERR_ARG, "config_from_gguf: args");
    return gguf_config(g, n_ctx, cfg);
}

int sinter_model_create_from_gguf(sinter_gguf *g, int device, int32_t n_ctx, uint32_t blocks, sinter_model **out) {
    if (!g || !out) return set_error(SINTER_ERR_ARG, "create_from_gguf: null argument");
    sinter_model_config c;
    const int rc = gguf_config(g, n_ctx, &c);
    if (rc != SINTER_OK) return rc;
    return model_create(&c, device, 0, blocks, g, out);
}

int sinter_model_get_config(sinter_model *m, sinter_model_config *cfg) {
    if (!m || !cfg) return set_error(SINTER_ERR_ARG, "get_config: args");
    *cfg = m->cfg;
    return SINTER_OK;
}

int sinter_model_synth_context(sinter_model *m, int32_t n_past, uint64_t seed) {
    if (!m || n_past < 0 || n_past > m->cfg.n_ctx) return set_error(SINTER_ERR_ARG, "synth_context: args");
    const sinter_model_config &c = m->cfg;
    const int RW = c.attn_nkv * c.head_dim;
    for (int il = 0; il < c.n_layer; il++) {
        hipError_t e = hipSuccess;
        if (is_attn(c, il)) {
            // f16 elements, or Q8_0 blocks of the same N(0,1) values
            const bool q8 = c.t_kv == SINTER_Q8_0;
            const int kind = q8 ? SINTER_SYN_NORMAL_Q8_0 : SINTER_SYN_NORMAL_F16;
            const uint64_t units = (uint64_t)n_past * RW / (q8 ? 32u : 1u);
            e = launch_synth(m->S[il][0].d, kind, 0, units, sinter_seed(seed, "cache_k", il), 0.f, 1.0f, m->stream);
            if (e == hipSuccess)
                e = launch_synth(m->S[il][1].d, kind, 0, units, sinter_seed(seed, "cache_v", il), 0.f, 1.0f,
                                 m->stream);
        } else {
            e = launch_synth(m->S[il][0].d, SINTER_SYN_NORMAL, 0, m->S[il][0].bytes / 4,
                             sinter_seed(seed, "conv_state", il), 0.f, 1.0f, m->stream);
            if (e == hipSuccess)
                e = launch_synth(m->S[il][1].d, SINTER_SYN_NORMAL, 0, m->S[il][1].bytes / 4,
                                 sinter_seed(seed, "ssm_state", il), 0.f, 0.1f, m->stream);
        }
        if (!hip_ok(e, "context synthesis")) return SINTER_ERR_HIP;
    }
    return hip_ok(hipStreamSynchronize(m->stream), "context synthesis") ? SINTER_OK : SINTER_ERR_HIP;
}

int sinter_model_bench_program(sinter_model *m, int kind, uint64_t seed) {
    if (!m) return set_error(SINTER_ERR_ARG, "bench_program: null model");
    const sinter_model_config &c = m->cfg;
    if (kind < SINTER_BENCH_GEMV || kind > SINTER_BENCH_ATTN) return set_error(SINTER_ERR_ARG, "bench_program: kind");
    int n = 0;
    for (int il = 0; il < c.n_layer; il++)
        n += kind == SINTER_BENCH_GEMV || (kind == SINTER_BENCH_ATTN) == is_attn(c, il);
    if (n == 0) return set_error(SINTER_ERR_ARG, "bench_program: the model has no layer of that kind");
    int rc = sinter_host_shutdown(m->host, 60000.0);
    if (rc) return rc;
    // x ~ N(0,1): the plain GEMV's input, the mixers' norm input
    if (!hip_ok(launch_synth(m->X, SINTER_SYN_NORMAL, 0, (uint64_t)c.n_embd, sinter_seed(seed, "bench_x", 0), 0.f,
                             1.f, m->stream),
                "bench input"))
        return SINTER_ERR_HIP;
    m->prog.clear();
    m->n_boundaries = 0;
    for (int il = 0; il < c.n_layer; il++) {
        if (kind == SINTER_BENCH_GEMV) {
            // y = W x: the layer's ffn_gate matrix, plain input, stored output
            sinter_gemv_args g;
            std::memset(&g, 0, sizeof g);
            g.K = (uint32_t)c.n_embd;
            g.eps = c.eps;
            g.pro = SINTER_PRO_PLAIN;
            g.x = m->X;
            g.n_seg = 1;
            g.seg[0] = seg(m->W[il][S_FFN_GATE], m->ffn, SINTER_EPI_STORE);
            push(m, SINTER_OP_GEMV, g, (uint32_t)il * 8);
            boundary(m);
        } else if ((kind == SINTER_BENCH_ATTN) == is_attn(c, il)) {
            push_mixer(m, il, false);
        }
    }
    // the pass-end barrier closes the last op
    m->prog.pop_back();
    m->n_boundaries--;
    if (!hip_ok(hipStreamSynchronize(m->stream), "bench input")) return SINTER_ERR_HIP;
    if ((rc = sinter_host_upload(m->host, m->prog.data(), (uint32_t)m->prog.size(), m->n_boundaries + 1))) return rc;
    return sinter_host_launch(m->host);
}

// the argument checks every prefill entry shares
static int prefill_args(sinter_model *m, const int32_t *tokens, uint32_t n, int32_t pos0) {
    if (!m || !tokens || n == 0 || pos0 < 0 || (int64_t)pos0 + n > m->cfg.n_ctx)
        return set_error(SINTER_ERR_ARG, "prefill: tokens / n / pos0 out of range");
    if (m->embed_outside) return set_error(SINTER_ERR_STATE, "prefill: the caller embeds each token");
    for (uint32_t i = 0; i < n; i++)
        if (tokens[i] < 0 || tokens[i] >= m->cfg.n_vocab) return set_error(SINTER_ERR_ARG, "prefill: token %u out of range", i);
    return SINTER_OK;
}

// Whether the batched prefill runs this model: every matrix a type the
// batched GEMV reads (Q4_K, Q6_K); why (if not) names the first that is not.
static bool prefill_batched_ok(const sinter_model *m, std::string &why) {
    const sinter_model_config &c = m->cfg;
    auto kq = [](const Tensor &t) { return t.type == SINTER_Q4_K || t.type == SINTER_Q6_K; };
    for (int il = 0; il < c.n_layer; il++) {
        const auto &w = m->W[il];
        const bool at = is_attn(c, il);
        const int mats_gdn[] = {S_QKV, S_Z, S_ALPHA, S_BETA, S_SSM_OUT, S_FFN_GATE, S_FFN_UP, S_FFN_DOWN};
        const int mats_att[] = {S_WQ, S_WK, S_WV, S_WO, S_FFN_GATE, S_FFN_UP, S_FFN_DOWN};
        const int *ms = at ? mats_att : mats_gdn;
        const int nm = at ? 7 : 8;
        for (int i = 0; i < nm; i++)
            if (!kq(w[ms[i]])) {
                why = "layer " + std::to_string(il) + " matrix slot " + std::to_string(ms[i]) + " has type " +
                      std::to_string(w[ms[i]].type);
                return false;
            }
    }
    if (!kq(m->output)) {
        why = "the output matrix has type " + std::to_string(m->output.type);
        return false;
    }
    if (c.conv_k > 8) {
        why = "conv kernel longer than 8 taps";
        return false;
    }
    return true;
}

// The batched prefill's buffers for ubatches of up to cap tokens.
static int prefill_buffers(sinter_model *m, uint32_t cap) {
    if (m->pf.cap >= cap) return SINTER_OK;
    const sinter_model_config &c = m->cfg;
    const size_t E = (size_t)c.n_embd, F = (size_t)c.n_ff, D = (size_t)c.gdn_d, HD = (size_t)c.head_dim;
    const size_t C = (size_t)(2 * c.gdn_hk + c.gdn_hv) * D, VD = (size_t)c.gdn_hv * D;
    const size_t NQ = (size_t)c.attn_nq, RW = (size_t)c.attn_nkv * HD;
    const size_t kmax = std::max({E, F, VD, NQ * HD});
    // (buffers of an earlier, smaller cap stay in the model's allocation list)
    auto f = [&](size_t n) { return static_cast<float *>(dalloc(m, n * 4)); };
    m->pf.tok = static_cast<int32_t *>(dalloc(m, (size_t)cap * 4));
    m->pf.x = f(cap * E);
    m->pf.qkv = f(cap * C);
    m->pf.conv = f(cap * C);
    m->pf.z = f(cap * VD);
    m->pf.al = f(cap * (size_t)c.gdn_hv);
    m->pf.be = f(cap * (size_t)c.gdn_hv);
    m->pf.o = f(cap * VD);
    m->pf.work = f(gdn_ubatch_work((uint32_t)c.gdn_hk, (uint32_t)c.gdn_hv, (uint32_t)D, cap));
    m->pf.qg = f(cap * NQ * 2 * HD);
    m->pf.k = f(cap * RW);
    m->pf.v = f(cap * RW);
    m->pf.qr = f(cap * NQ * HD);
    m->pf.att = f(cap * NQ * HD);
    m->pf.gate = f(cap * F);
    m->pf.up = f(cap * F);
    m->pf.part = f(attn_prefill_part(cap, (uint32_t)NQ, (uint32_t)HD, (uint32_t)c.attn_chunks));
    m->pf.xq = dalloc(m, (size_t)cap * (kmax / 256) * 292);
    const bool ok = m->pf.tok && m->pf.x && m->pf.qkv && m->pf.conv && m->pf.z && m->pf.al && m->pf.be && m->pf.o &&
                    m->pf.work && m->pf.qg && m->pf.k && m->pf.v && m->pf.qr && m->pf.att && m->pf.gate &&
                    m->pf.up && m->pf.part && m->pf.xq;
    if (!ok) {
        m->pf.cap = 0;
        return set_error(SINTER_ERR_HIP, "prefill: buffers for a ubatch of %u tokens", cap);
    }
    m->pf.cap = cap;
    return SINTER_OK;
}

// One ubatch of T tokens at positions pos.. through every layer (the
// tokens already in pf.tok); on the last ubatch, the head on its last token.
static int prefill_ubatch(sinter_model *m, uint32_t T, int32_t pos, bool last) {
    const sinter_model_config &c = m->cfg;
    const hipStream_t s = m->stream;
    void *sv = (void *)s;
    const uint32_t E = (uint32_t)c.n_embd, F = (uint32_t)c.n_ff, D = (uint32_t)c.gdn_d, HD = (uint32_t)c.head_dim;
    const uint32_t HK = (uint32_t)c.gdn_hk, HV = (uint32_t)c.gdn_hv, C = (2 * HK + HV) * D, VD = HV * D;
    const uint32_t NQ = (uint32_t)c.attn_nq, NKV = (uint32_t)c.attn_nkv, RW = NKV * HD;
    auto &p = m->pf;
    int rc = SINTER_OK;
    auto gemv = [&](const Tensor &w, uint32_t k, float *y, int acc) {
        if (rc == SINTER_OK) rc = sinter_op_gemv_ubatch(w.type, w.d, w.rows, k, p.xq, T, y, acc, sv);
    };
    auto hip = [&](hipError_t e, const char *what) {
        if (rc == SINTER_OK && !hip_ok(e, what)) rc = SINTER_ERR_HIP;
    };
    hip(launch_embed_ubatch(m->embd.d, m->embd.type, E, p.tok, T, p.x, s), "prefill: embed");
    const float theta_scale = (float)std::pow((double)c.rope_base, -2.0 / (double)c.rope_dims);
    for (int il = 0; il < c.n_layer && rc == SINTER_OK; il++) {
        const auto &w = m->W[il];
        rc = sinter_rmsnorm_quant_q8k_ubatch(p.x, (const float *)w[S_ATTN_NORM].d, c.eps, E, T, p.xq, sv);
        if (is_attn(c, il)) {
            gemv(w[S_WQ], E, p.qg, 0);
            gemv(w[S_WK], E, p.k, 0);
            gemv(w[S_WV], E, p.v, 0);
            hip(launch_attn_prep_ubatch(p.qg, p.k, p.v, (const float *)w[S_Q_NORM].d, (const float *)w[S_K_NORM].d,
                                        m->S[il][0].d, m->S[il][1].d, (uint32_t)c.t_kv, pos, T, NQ, NKV, HD,
                                        (uint32_t)c.rope_dims, theta_scale, c.eps, p.qr, s),
                "prefill: attention prep");
            hip(launch_attn_prefill(p.qr, p.qg, m->S[il][0].d, m->S[il][1].d, (uint32_t)c.t_kv, pos, T, NQ, NKV, HD,
                                    (uint32_t)c.attn_chunks, (uint32_t)c.attn_chunk_min,
                                    1.0f / std::sqrt((float)HD), p.part, p.att, s),
                "prefill: attention");
            if (rc == SINTER_OK) rc = sinter_quant_q8k_ubatch(p.att, (int64_t)NQ * HD, T, p.xq, sv);
            gemv(w[S_WO], NQ * HD, p.x, 1);
        } else {
            gemv(w[S_QKV], E, p.qkv, 0);
            gemv(w[S_Z], E, p.z, 0);
            gemv(w[S_ALPHA], E, p.al, 0);
            gemv(w[S_BETA], E, p.be, 0);
            if (rc == SINTER_OK)
                rc = sinter_conv_silu_ubatch(p.qkv, (float *)m->S[il][0].d, (const float *)w[S_CONV_W].d, p.conv, C,
                                             (uint32_t)c.conv_k, T, sv);
            hip(launch_gdn_ubatch(p.conv, p.al, p.be, (const float *)w[S_DT_BIAS].d, (const float *)w[S_SSM_A].d,
                                  (float *)m->S[il][1].d, p.o, p.work, HK, HV, D, T, c.eps,
                                  1.0f / std::sqrt((float)D), s),
                "prefill: gated DeltaNet");
            if (rc == SINTER_OK)
                rc = sinter_gated_rmsnorm_quant_q8k_ubatch(p.o, p.z, (const float *)w[S_SSM_NORM].d, D, c.eps, VD, T,
                                                           p.xq, sv);
            gemv(w[S_SSM_OUT], VD, p.x, 1);
        }
        if (rc == SINTER_OK)
            rc = sinter_rmsnorm_quant_q8k_ubatch(p.x, (const float *)w[S_POST_NORM].d, c.eps, E, T, p.xq, sv);
        gemv(w[S_FFN_GATE], E, p.gate, 0);
        gemv(w[S_FFN_UP], E, p.up, 0);
        if (rc == SINTER_OK) rc = sinter_swiglu_quant_q8k_ubatch(p.gate, p.up, F, T, p.xq, sv);
        gemv(w[S_FFN_DOWN], F, p.x, 1);
    }
    (void)RW;
    if (rc == SINTER_OK && last) {
        // the head on the last token: output norm + Q8_K, logits
        rc = sinter_rmsnorm_quant_q8k_ubatch(p.x + (size_t)(T - 1) * E, (const float *)m->onorm.d, c.eps, E, 1, p.xq,
                                             sv);
        if (rc == SINTER_OK)
            rc = sinter_op_gemv_ubatch(m->output.type, m->output.d, m->output.rows, E, p.xq, 1, m->logits, 0, sv);
    }
    return rc;
}

int sinter_model_prefill_batched(sinter_model *m, const int32_t *tokens, uint32_t n, int32_t pos0, uint32_t ubatch,
                                 int32_t *next_token) {
    if (int rc = prefill_args(m, tokens, n, pos0)) return rc;
    if (ubatch < 1 || ubatch > SINTER_PREFILL_UBATCH_MAX)
        return set_error(SINTER_ERR_ARG, "prefill: ubatch %u (1..%u)", ubatch, (unsigned)SINTER_PREFILL_UBATCH_MAX);
    std::string why;
    if (!prefill_batched_ok(m, why)) return set_error(SINTER_ERR_ARG, "prefill: not batched: %s", why.c_str());
    const uint32_t cap = std::min(ubatch, n);
    if (int rc = prefill_buffers(m, cap)) return rc;
    int rc = SINTER_OK;
    for (uint32_t b = 0; rc == SINTER_OK && b < n; b += cap) {
        const uint32_t T = std::min(cap, n - b);
        if (!hip_ok(hipMemcpyAsync(m->pf.tok, tokens + b, (size_t)T * 4, hipMemcpyHostToDevice, m->stream),
                    "prefill: tokens"))
            return SINTER_ERR_HIP;
        rc = prefill_ubatch(m, T, pos0 + (int32_t)b, b + T == n);
        // (the token copy of the next ubatch reads host memory the caller
        // owns: the stream is drained before it is queued)
        if (rc == SINTER_OK && !hip_ok(hipStreamSynchronize(m->stream), "prefill: ubatch")) rc = SINTER_ERR_HIP;
    }
    if (rc != SINTER_OK) return rc;
    // the greedy continuation: the first maximum of the logits (the decode
    // head's argmax), also left in the pass cell as a decode pass leaves it
    std::vector<float> lg((size_t)m->cfg.n_vocab);
    if (!hip_ok(hipMemcpy(lg.data(), m->logits, lg.size() * 4, hipMemcpyDeviceToHost), "prefill: logits"))
        return SINTER_ERR_HIP;
    int32_t best = 0;
    for (int32_t i = 1; i < m->cfg.n_vocab; i++)
        if (lg[(size_t)i] > lg[(size_t)best]) best = i;
    if (!hip_ok(hipMemcpy(&sinter_host_pass_cell(m->host)->token, &best, 4, hipMemcpyHostToDevice), "prefill: token"))
        return SINTER_ERR_HIP;
    if (next_token) *next_token = best;
    return SINTER_OK;
}

int sinter_model_prefill(sinter_model *m, const int32_t *tokens, uint32_t n, int32_t pos0, int32_t *next_token) {
    if (int rc = prefill_args(m, tokens, n, pos0)) return rc;
    std::string why;
    if (prefill_batched_ok(m, why))
        return sinter_model_prefill_batched(m, tokens, n, pos0, SINTER_PREFILL_UBATCH, next_token);
    return sinter_model_prefill_tokenwise(m, tokens, n, pos0, next_token);
}

int sinter_model_decode(sinter_model *m, int32_t token, int32_t pos, float *logits_host, int32_t *next_token) {
    if (!m || pos < 0 || pos >= m->cfg.n_ctx || token < 0 || token >= m->cfg.n_vocab)
        return set_error(SINTER_ERR_ARG, "decode: token/pos out of range");
    int rc = sinter_host_set_pos(m->host, pos);
    if (rc) return rc;
    const int rs = sinter_host_run_pass(m->host, token, 120000.0);
    if (rs != SINTER_RUN_OK) return rs == SINTER_RUN_TIMEOUT ? SINTER_ERR_TIMEOUT : SINTER_ERR_DEVICE;
    if (logits_host &&
        !hip_ok(hipMemcpy(logits_host, m->logits, (size_t)m->cfg.n_vocab * 4, hipMemcpyDeviceToHost), "logits"))
        return SINTER_ERR_HIP;
    if (next_token) *next_token = host_last_token(m->host);   // (the launch record: no device read)
    return SINTER_OK;
}

int sinter_model_greedy(sinter_model *m, int32_t token, int32_t pos, uint32_t n, int32_t *tokens_out) {
    if (!m || pos < 0 || (int64_t)pos + n > m->cfg.n_ctx || token < 0 || token >= m->cfg.n_vocab)
        return set_error(SINTER_ERR_ARG, "greedy: token/pos/n out of range");
    if (m->embed_outside && n > 1)
        return set_error(SINTER_ERR_STATE, "greedy: the caller embeds each token (one pass per call)");
    int rc = sinter_host_set_pos(m->host, pos);
    if (rc) return rc;
    const int rs = sinter_host_run_passes(m->host, token, n, tokens_out, 600000.0);
    if (rs != SINTER_RUN_OK) return rs == SINTER_RUN_TIMEOUT ? SINTER_ERR_TIMEOUT : SINTER_ERR_DEVICE;
    return SINTER_OK;
}

int sinter_model_prefill_tokenwise(sinter_model *m, const int32_t *tokens, uint32_t n, int32_t pos0,
                                   int32_t *next_token) {
    if (int rc = prefill_args(m, tokens, n, pos0)) return rc;
    uint32_t cap = 0;
    (void)sinter_host_history(m->host, &cap);
    cap = std::max(1u, std::min(cap, 1024u));
    int32_t *d_tok = nullptr;
    if (!hip_ok(hipMalloc(&d_tok, (size_t)n * 4), "prefill: token buffer")) return SINTER_ERR_HIP;
    // forced / n_forced of the argmax workspace (device memory), written
    // between launches only
    auto set_forced = [&](const int32_t *p, uint32_t nf) {
        struct { const int32_t *p; uint32_t n; } f = {p, nf};
        return hip_ok(hipMemcpy(reinterpret_cast<char *>(m->ws) + offsetof(sinter_argmax_ws, forced), &f.p,
                                sizeof f.p, hipMemcpyHostToDevice), "prefill: forced") &&
               hip_ok(hipMemcpy(reinterpret_cast<char *>(m->ws) + offsetof(sinter_argmax_ws, n_forced), &f.n,
                                sizeof f.n, hipMemcpyHostToDevice), "prefill: n_forced");
    };
    int rc = hip_ok(hipMemcpy(d_tok, tokens, (size_t)n * 4, hipMemcpyHostToDevice), "prefill: tokens") ? SINTER_OK
                                                                                                      : SINTER_ERR_HIP;
    for (uint32_t b = 0; rc == SINTER_OK && b < n; b += cap) {
        const uint32_t len = std::min(cap, n - b);
        if (!set_forced(d_tok + b, n - b)) { rc = SINTER_ERR_HIP; break; }
        if ((rc = sinter_host_set_pos(m->host, pos0 + (int32_t)b))) break;
        const int rs = sinter_host_run_passes(m->host, tokens[b], len, nullptr, 600000.0);
        if (rs != SINTER_RUN_OK) rc = rs == SINTER_RUN_TIMEOUT ? SINTER_ERR_TIMEOUT : SINTER_ERR_DEVICE;
    }
    if (!set_forced(nullptr, 0) && rc == SINTER_OK) rc = SINTER_ERR_HIP;
    (void)hipFree(d_tok);
    if (rc == SINTER_OK && next_token) *next_token = host_last_token(m->host);
    return rc;
}

int sinter_model_logits(sinter_model *m, float *logits_host) {
    if (!m || !logits_host) return set_error(SINTER_ERR_ARG, "logits: args");
    return hip_ok(hipMemcpy(logits_host, m->logits, (size_t)m->cfg.n_vocab * 4, hipMemcpyDeviceToHost), "logits")
               ? SINTER_OK
               : SINTER_ERR_HIP;
}

int sinter_model_tensor_info(sinter_model *m, int64_t layer, int slot, void **dev_ptr, size_t *bytes, int *type) {
    if (!m || slot < 0 || slot >= NSLOT || layer < 0 || layer > m->cfg.n_layer) return set_error(SINTER_ERR_ARG, "slot");
    const Tensor *t = nullptr;
    if (layer == m->cfg.n_layer) {
        t = slot == 0 ? &m->embd : slot == 1 ? &m->onorm : slot == 2 ? &m->output : nullptr;
    } else {
        t = &m->W[layer][slot];
    }
    if (!t) return set_error(SINTER_ERR_ARG, "slot");
    if (dev_ptr) *dev_ptr = t->d;
    if (bytes) *bytes = t->d ? t->bytes : 0;
    if (type) *type = t->type;
    return SINTER_OK;
}

int sinter_model_state_info(sinter_model *m, int64_t layer, int slot, void **dev_ptr, size_t *bytes) {
    if (!m || layer < 0 || layer >= m->cfg.n_layer || slot < 0 || slot > 1) return set_error(SINTER_ERR_ARG, "state");
    if (dev_ptr) *dev_ptr = m->S[layer][slot].d;
    if (bytes) *bytes = m->S[layer][slot].bytes;
    return SINTER_OK;
}

int sinter_model_copy(sinter_model *m, void *dst, const void *src, size_t bytes, int dir) {
    if (!m || !dst || !src) return set_error(SINTER_ERR_ARG, "copy");
    const hipMemcpyKind k = dir == 0 ? hipMemcpyDeviceToHost : dir == 1 ? hipMemcpyHostToDevice : hipMemcpyDeviceToDevice;
    return hip_ok(hipMemcpy(dst, src, bytes, k), "copy") ? SINTER_OK : SINTER_ERR_HIP;
}

int sinter_model_info(sinter_model *m, uint64_t *weight_bytes, uint32_t *n_instr, uint32_t *n_boundaries,
                      uint32_t *blocks) {
    if (!m) return set_error(SINTER_ERR_ARG, "null model");
    if (weight_bytes) *weight_bytes = m->weight_bytes;
    if (n_instr) *n_instr = (uint32_t)m->prog.size();
    if (n_boundaries) *n_boundaries = m->n_boundaries + 1;
    if (blocks) *blocks = m->blocks;
    return SINTER_OK;
}

sinter_host *sinter_model_host(sinter_model *m) { return m ? m->host : nullptr; }

int sinter_model_buffer(sinter_model *m, const char *name, void **dev_ptr, size_t *bytes) {
    if (!m || !name) return set_error(SINTER_ERR_ARG, "buffer: args");
    const sinter_model_config &c = m->cfg;
    const size_t E = (size_t)c.n_embd, VD = (size_t)c.gdn_hv * c.gdn_d, NQHD = (size_t)c.attn_nq * c.head_dim;
    const size_t C = (size_t)(2 * c.gdn_hk + c.gdn_hv) * c.gdn_d, RW = (size_t)c.attn_nkv * c.head_dim;
    const uint32_t chunks = (uint32_t)c.attn_chunks;
    struct B { const char *n; void *p; size_t b; } tab[] = {
        {"X", m->X, E * 4}, {"H", m->H, E * 4}, {"qkv", m->qkv, C * 4}, {"z", m->z, VD * 4},
        {"alpha", m->al, (size_t)c.gdn_hv * 4}, {"beta", m->be, (size_t)c.gdn_hv * 4}, {"o", m->o, VD * 4},
        {"ffn", m->ffn, (size_t)c.n_ff * 4}, {"qg", m->qg, NQHD * 2 * 4}, {"k", m->kk, RW * 4}, {"v", m->vv, RW * 4},
        {"att", m->att, NQHD * 4}, {"logits", m->logits, (size_t)c.n_vocab * 4},
        {"attn_part", m->part, sinter_attn_part_len(c.attn_nq, c.attn_nkv, c.head_dim, chunks) * 4},
        {"attn_count", m->count, (size_t)sinter_attn_count_len(c.attn_nkv, chunks) * 4},
        {"argmax_ws", m->ws, sizeof(sinter_argmax_ws)}};
    for (const B &b : tab)
        if (std::strcmp(b.n, name) == 0) {
            if (dev_ptr) *dev_ptr = b.p;
            if (bytes) *bytes = b.b;
            return SINTER_OK;
        }
    return set_error(SINTER_ERR_ARG, "buffer: no buffer named %s", name);
}

int sinter_model_program(sinter_model *m, sinter_instr *out, uint32_t cap, uint32_t *n_instr) {
    if (!m) return set_error(SINTER_ERR_ARG, "program: null model");
    if (n_instr) *n_instr = (uint32_t)m->prog.size();
    if (out) {
        if (cap < m->prog.size()) return set_error(SINTER_ERR_ARG, "program: %u slots for %zu instructions", cap, m->prog.size());
        std::memcpy(out, m->prog.data(), m->prog.size() * sizeof(sinter_instr));
    }
    return SINTER_OK;
}

// Static load balance of the GEMVs: every workgroup of a GEMV streams an equal
// share of its bytes, but some workgroups are released from the barrier, or
// stream, systematically later than others (the spread follows the
// workgroup's XCD and is stable across layers), and the phase ends with the
// last one.  Each round traces `traces` greedy passes; for every workgroup b
// of every GEMV, with d_b its streaming time after the prologue and E_b its
// end minus the mean end, the workgroup's share is scaled by
// (d_b - E_b) / d_b (averaged over the traces and over the GEMVs of the same
// shape, clamped to [0.7, 1.3]), which would end every workgroup together.
// After `rounds` updates a last measurement keeps, per shape, the shares
// with the shortest tail.  Only the row ranges change: every row's value is
// bit-identical.  Decodes (rounds + 1) * traces tokens from (*token, *pos),
// which are advanced.
int sinter_model_balance(sinter_model *m, int32_t *token, int32_t *pos, uint32_t rounds, uint32_t traces) {
    if (!m || !token || !pos || traces == 0 || *pos < 0 ||
        (int64_t)*pos + (int64_t)(rounds + 1) * traces > m->cfg.n_ctx)
        return set_error(SINTER_ERR_ARG, "balance: args");
    const size_t n = m->prog.size(), B = m->blocks, words = (n + 1) * B * 4;
    // GEMVs of one shape share their statistics
    std::vector<int> grp(n, -1);
    std::vector<std::array<uint32_t, 6>> keys;
    for (size_t i = 0; i < n; i++) {
        if (m->prog[i].kind != SINTER_OP_GEMV || m->prog[i].block_lo != 0 || m->prog[i].block_hi != B) continue;
        sinter_gemv_args a;
        std::memcpy(&a, m->prog[i].payload, sizeof a);
        const std::array<uint32_t, 6> k = {a.pro, a.K, a.n_seg, a.seg[0].rows, (uint32_t)a.seg[0].type, a.seg[0].epi};
        size_t g = 0;
        while (g < keys.size() && keys[g] != k) g++;
        if (g == keys.size()) keys.push_back(k);
        grp[i] = (int)g;
    }
    std::vector<float> share(n * B, 1.0f), best(n * B, 1.0f);
    std::vector<double> best_tail(keys.size(), 0.0);
    std::vector<char> frozen(keys.size(), 0);
    unsigned long long *d_trace = nullptr;
    if (!hip_ok(hipMalloc(&d_trace, words * 8), "balance trace alloc")) return SINTER_ERR_HIP;
    std::vector<unsigned long long> t(words);
    int rc = SINTER_OK;
    // rounds + 1 measurements: each after the previous update; a shape whose
    // tail (last end minus mean end) got longer returns to its best shares
    // and is not updated again
    for (uint32_t r = 0; r <= rounds && rc == SINTER_OK; r++) {
        std::vector<double> acc(keys.size() * B, 0.0), tail(keys.size(), 0.0);
        std::vector<uint32_t> cnt(keys.size(), 0);
        for (uint32_t k = 0; k < traces && rc == SINTER_OK; k++) {
            int32_t next = 0;
            rc = sinter_host_trace_next(m->host, d_trace, words);
            if (rc == SINTER_OK) rc = sinter_model_greedy(m, *token, *pos, 1, &next);
            if (rc != SINTER_OK) break;
            if (!hip_ok(hipMemcpy(t.data(), d_trace, words * 8, hipMemcpyDeviceToHost), "balance trace read")) {
                rc = SINTER_ERR_HIP;
                break;
            }
            *token = next;
            *pos += 1;
            for (size_t i = 0; i < n; i++) {
                if (grp[i] < 0) continue;
                const unsigned long long *ti = t.data() + i * B * 4;
                bool ok = true;
                for (size_t b = 0; b < B; b++) ok = ok && ti[b * 4 + 3] > ti[b * 4 + 2] && ti[b * 4 + 2] > 0;
                if (!ok) continue;
                double emean = 0.0, emax = 0.0;
                for (size_t b = 0; b < B; b++) {
                    emean += (double)ti[b * 4 + 3];
                    emax = std::max(emax, (double)ti[b * 4 + 3]);
                }
                emean /= (double)B;
                for (size_t b = 0; b < B; b++) {
                    const double d = (double)(ti[b * 4 + 3] - ti[b * 4 + 2]);
                    const double e = (double)ti[b * 4 + 3] - emean;
                    acc[grp[i] * B + b] += std::min(1.3, std::max(0.7, (d - e) / d));
                }
                tail[grp[i]] += emax - emean;
                cnt[grp[i]]++;
            }
        }
        if (rc != SINTER_OK) break;
        for (size_t g = 0; g < keys.size(); g++) {
            if (cnt[g] == 0) continue;
            const double tg = tail[g] / cnt[g];
            const bool worse = r > 0 && tg > best_tail[g];
            if (!worse) best_tail[g] = tg;
            for (size_t i = 0; i < n; i++) {
                if (grp[i] != (int)g) continue;
                float *sh = share.data() + i * B, *bs = best.data() + i * B;
                if (worse) {
                    frozen[g] = 1;
                    std::copy(bs, bs + B, sh);
                } else {
                    std::copy(sh, sh + B, bs);
                    if (r < rounds && !frozen[g])
                        for (size_t b = 0; b < B; b++) sh[b] *= (float)(acc[g * B + b] / cnt[g]);
                }
                if (worse || (r < rounds && !frozen[g])) {
                    rc = sinter_host_set_gemv_shares(m->host, (uint32_t)i, sh, (uint32_t)B);
                    if (rc != SINTER_OK) break;
                }
            }
            if (rc != SINTER_OK) break;
        }
    }
    (void)hipFree(d_trace);
    return rc;
}

}  // extern "C"
