// A ggml dynamic backend ("SINTER") that runs the batch-1 decode graph of the
// Qwen3.6 hybrid through libsinter's persistent interpreter and hands every
// other graph to the stock ggml HIP backend.
//
// Built only where ggml's headers are present (build.py: SINTER_GGML_INCLUDE
// and SINTER_GGML_LIB); the ggml tree is not part of this repository, so this
// file is NOT compiled or tested here.  Contract it implements
// (docs/INTEGRATION-FINDINGS.md:182-313 of the reference):
//   * ggml_backend_init() returns a registry with api_version ==
//     GGML_BACKEND_API_VERSION holding ONE device of type GPU (never META),
//     loaded through GGML_BACKEND_PATH and selected with --device SINTER;
//   * the device forwards buffer types, memory, supports_op and supports_buft
//     to the stock HIP device (one GPU: no meta buffers, so every tensor's
//     ->data is a plain device pointer in this process);
//   * graph_compute fingerprints the graph it receives (the whole decode
//     stack as one split, the scheduler's copy tensors renamed
//     "<backend>#<name>#<c>"): a batch-1 decode graph of the model is run by a
//     sinter model bound to the graph's own weight, KV-cache and recurrent-state
//     tensors (sinter_model_create_bound) writing the logits into
//     result_output; prefill (GDN node suffix __fgdn_ch__, or ne[2] > 1:
//     docs/PREFILL-SEMANTICS.md:344-377), batch > 1, a KV row other than the
//     position, or any shape the model does not match is delegated unchanged.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "ggml-backend-impl.h"
#include "ggml-backend.h"
#include "ggml.h"
#include "sinter.h"

namespace {

// ------------------------------------------------------------------ names

// A tensor's name without the scheduler's copy decoration "<backend>#<name>#<c>".
std::string base_name(const ggml_tensor *t) {
    std::string n = t->name;
    const size_t a = n.find('#');
    if (a == std::string::npos) return n;
    const size_t b = n.rfind('#');
    return b > a ? n.substr(a + 1, b - a - 1) : n.substr(a + 1);
}

// The tensor a view reads from (the cache tensors appear through views).
const ggml_tensor *view_root(const ggml_tensor *t) {
    while (t && t->view_src) t = t->view_src;
    return t;
}

// ggml type -> sinter_type (the numbering is ggml's; only what the kernels read)
int sinter_type_of(ggml_type t) {
    switch (t) {
    case GGML_TYPE_F32: return SINTER_F32;
    case GGML_TYPE_F16: return SINTER_F16;
    case GGML_TYPE_BF16: return SINTER_BF16;
    case GGML_TYPE_Q8_0: return SINTER_Q8_0;
    case GGML_TYPE_Q4_K: return SINTER_Q4_K;
    case GGML_TYPE_Q6_K: return SINTER_Q6_K;
    default: return -1;
    }
}

// ------------------------------------------------------------------ fingerprint

// What one received graph is, as far as the decode path cares.
struct Shape {
    bool decode = false;              // a batch-1 decode graph of a Qwen3.6-style hybrid
    std::string why;                  // the reason it is not (logged once per reason)
    std::map<std::string, ggml_tensor *> named;   // every node and leaf by base name
    int n_layer = 0, n_gdn = 0, n_attn = 0;
    ggml_tensor *logits = nullptr, *tokens = nullptr, *embd = nullptr, *pos = nullptr;
};

Shape inspect(ggml_cgraph *g) {
    Shape s;
    auto note = [&](ggml_tensor *t) {
        if (t && t->name[0]) s.named.emplace(base_name(t), t);
    };
    const int n = ggml_graph_n_nodes(g);
    for (int i = 0; i < n; i++) {
        ggml_tensor *t = ggml_graph_node(g, i);
        note(t);
        for (int j = 0; j < GGML_MAX_SRC; j++) note(t->src[j]);
        if (t->op == GGML_OP_GATED_DELTA_NET) {
            const std::string nm = t->name;
            if (nm.find("__fgdn_ch__") != std::string::npos) { s.why = "prefill (chunked GDN node)"; return s; }
            if (nm.find("__fgdn_ar__") == std::string::npos) { s.why = "GDN node without the decode suffix"; return s; }
            // ne[2] of q is the token count of the ubatch
            if (t->src[0] && t->src[0]->ne[2] != 1) { s.why = "GDN over more than one token"; return s; }
            s.n_gdn++;
        } else if (t->op == GGML_OP_FLASH_ATTN_EXT) {
            if (t->src[0] && t->src[0]->ne[1] != 1) { s.why = "attention over more than one query"; return s; }
            s.n_attn++;
        }
    }
    s.logits = s.named.count("result_output") ? s.named["result_output"] : nullptr;
    s.tokens = s.named.count("inp_tokens") ? s.named["inp_tokens"] : nullptr;
    s.embd = s.named.count("inp_embd") ? s.named["inp_embd"] : nullptr;
    s.pos = s.named.count("inp_pos") ? s.named["inp_pos"] : nullptr;
    s.n_layer = s.n_gdn + s.n_attn;
    if (!s.logits || s.logits->ne[1] != 1) { s.why = "no single-row result_output"; return s; }
    if (!s.pos || ggml_nelements(s.pos) != 1) { s.why = "no single position"; return s; }
    if (!s.tokens && !s.embd) { s.why = "neither token ids nor an embedded row as input"; return s; }
    if (s.n_gdn == 0 || s.n_attn == 0) { s.why = "not the hybrid decode graph"; return s; }
    s.decode = true;
    return s;
}

// ------------------------------------------------------------------ binding

// Per-layer weight names in the slot numbering of sinter_model_tensor_info
// (the same table as schedule.py's packer).
const char *const kCommon[5] = {"attn_norm.weight", "post_attention_norm.weight", "ffn_gate.weight",
                                "ffn_up.weight", "ffn_down.weight"};
const char *const kGdn[9] = {"attn_qkv.weight", "attn_gate.weight", "ssm_alpha.weight", "ssm_beta.weight",
                             "ssm_out.weight", "ssm_conv1d.weight", "ssm_dt.bias", "ssm_a", "ssm_norm.weight"};
const char *const kAttn[6] = {"attn_q.weight", "attn_k.weight", "attn_v.weight", "attn_output.weight",
                              "attn_q_norm.weight", "attn_k_norm.weight"};

struct Bound {
    sinter_model *m = nullptr;
    std::vector<void *> tensors, states;
    std::vector<int32_t> types;
    const void *key_logits = nullptr;   // the graph instance the model was bound to
    bool embed_outside = false;
    float *x = nullptr;                 // the model's X buffer (embed_outside)
};

// Resolve the decode graph's tensors into bindings and a config; false (with
// the reason) when anything the model needs is missing or mis-shaped.
bool bind_graph(const Shape &s, ggml_backend_t stock, sinter_model_config &c, Bound &b, std::string &why) {
    auto get = [&](const std::string &n) -> ggml_tensor * {
        auto it = s.named.find(n);
        return it == s.named.end() ? nullptr : it->second;
    };
    ggml_tensor *embd_w = get("token_embd.weight"), *out_w = get("output.weight"), *onorm = get("output_norm.weight");
    if (!onorm) { why = "no output_norm.weight"; return false; }
    if (!out_w) out_w = embd_w;                    // tied head
    if (!out_w) { why = "no head weight"; return false; }
    std::memset(&c, 0, sizeof c);
    c.n_layer = s.n_layer;
    c.n_embd = (int32_t)out_w->ne[0];
    c.n_vocab = (int32_t)out_w->ne[1];
    // scalars no weight carries, from the ops that use them: the RMS-norm
    // epsilon (op_params[0]), the rope's rotated dims ([1]) and base ([5])
    c.eps = 1e-6f;
    c.rope_base = 1e7f;
    c.rope_dims = 64;
    for (const auto &kv : s.named) {
        const ggml_tensor *t = kv.second;
        if (t->op == GGML_OP_RMS_NORM) std::memcpy(&c.eps, t->op_params, sizeof(float));
        if (t->op == GGML_OP_ROPE) {
            c.rope_dims = t->op_params[1];
            std::memcpy(&c.rope_base, t->op_params + 5, sizeof(float));
        }
    }
    c.t_kv = SINTER_F16;
    int first_attn = -1;
    for (int il = 0; il < c.n_layer && first_attn < 0; il++)
        if (get("blk." + std::to_string(il) + ".attn_q.weight")) first_attn = il;
    if (first_attn < 0) { why = "no attention layer"; return false; }
    c.attn_every = first_attn + 1;
    const std::string l0 = "blk." + std::to_string(first_attn) + ".";
    ggml_tensor *wq = get(l0 + "attn_q.weight"), *wk = get(l0 + "attn_k.weight"), *qn = get(l0 + "attn_q_norm.weight");
    ggml_tensor *up = get("blk.0.ffn_up.weight"), *qkv = get("blk.0.attn_qkv.weight"), *sa = get("blk.0.ssm_a");
    ggml_tensor *sn = get("blk.0.ssm_norm.weight");
    if (!wq || !wk || !qn || !up || !qkv || !sa || !sn) { why = "layer 0 / first attention layer incomplete"; return false; }
    ggml_tensor *cw = get("blk.0.ssm_conv1d.weight");
    if (!cw) { why = "no ssm_conv1d.weight"; return false; }
    c.conv_k = (int32_t)cw->ne[0];
    c.head_dim = (int32_t)qn->ne[0];
    c.attn_nq = (int32_t)(wq->ne[1] / (2 * c.head_dim));
    c.attn_nkv = (int32_t)(wk->ne[1] / c.head_dim);
    c.n_ff = (int32_t)up->ne[1];
    c.gdn_d = (int32_t)sn->ne[0];
    c.gdn_hv = (int32_t)ggml_nelements(sa);
    c.gdn_hk = (int32_t)((qkv->ne[1] / c.gdn_d - c.gdn_hv) / 2);
    // the KV cache tensors (views of cache_k_l<il> / cache_v_l<il>)
    ggml_tensor *kc0 = get("cache_k_l" + std::to_string(first_attn));
    if (!kc0) { why = "no KV cache tensor"; return false; }
    const ggml_tensor *kr = view_root(kc0);
    c.n_ctx = (int32_t)(ggml_nelements(kr) / ((int64_t)c.attn_nkv * c.head_dim));
    if (kr->type == GGML_TYPE_Q8_0) c.t_kv = SINTER_Q8_0;
    else if (kr->type != GGML_TYPE_F16) { why = "KV cache neither f16 nor q8_0"; return false; }
    c.t_default = sinter_type_of(qkv->type);
    c.t_attn_v = c.t_ffn_down = c.t_output = c.t_embd = c.t_default;

    const size_t nt = (size_t)c.n_layer * 16 + 3;
    b.tensors.assign(nt, nullptr);
    b.types.assign(nt, SINTER_F32);
    b.states.assign((size_t)c.n_layer * 2, nullptr);
    auto put = [&](size_t i, ggml_tensor *t) -> bool {
        if (!t) return false;
        const int st = sinter_type_of(t->type);
        if (st < 0) return false;
        b.tensors[i] = t->data;
        b.types[i] = st;
        return true;
    };
    for (int il = 0; il < c.n_layer; il++) {
        const std::string p = "blk." + std::to_string(il) + ".";
        const bool at = il % c.attn_every == c.attn_every - 1;
        for (int k = 0; k < 5; k++)
            if (!put((size_t)il * 16 + k, get(p + kCommon[k]))) { why = p + kCommon[k]; return false; }
        const int nk = at ? 6 : 9;
        for (int k = 0; k < nk; k++) {
            const char *nm = at ? kAttn[k] : kGdn[k];
            if (!put((size_t)il * 16 + 5 + k, get(p + nm))) { why = p + nm; return false; }
        }
        const std::string sfx = std::to_string(il);
        ggml_tensor *s0 = get((at ? "cache_k_l" : "cache_r_l") + sfx), *s1 = get((at ? "cache_v_l" : "cache_s_l") + sfx);
        if (!s0 || !s1) { why = "state of layer " + sfx; return false; }
        b.states[(size_t)il * 2] = view_root(s0)->data;
        b.states[(size_t)il * 2 + 1] = view_root(s1)->data;
    }
    b.embed_outside = s.tokens == nullptr;
    const size_t g0 = (size_t)c.n_layer * 16;
    if (!b.embed_outside && !put(g0, embd_w)) { why = "token_embd.weight not on the GPU"; return false; }
    if (!put(g0 + 1, onorm) || !put(g0 + 2, out_w)) { why = "head tensors"; return false; }
    (void)stock;
    return true;
}

// ------------------------------------------------------------------ backend

struct Ctx {
    ggml_backend_t stock = nullptr;    // the HIP backend every miss goes to
    Bound bound;
    std::map<std::string, int> misses; // reasons already logged
};

const char *be_name(ggml_backend_t) { return "SINTER"; }

void be_free(ggml_backend_t be) {
    Ctx *c = static_cast<Ctx *>(be->context);
    if (c->bound.m) sinter_model_destroy(c->bound.m);
    if (c->stock) ggml_backend_free(c->stock);
    delete c;
    delete be;
}

void be_synchronize(ggml_backend_t be) { ggml_backend_synchronize(static_cast<Ctx *>(be->context)->stock); }

enum ggml_status delegate(Ctx *c, ggml_cgraph *g, const std::string &why) {
    if (c->misses[why]++ == 0) std::fprintf(stderr, "sinter: graph delegated to the stock backend: %s\n", why.c_str());
    return ggml_backend_graph_compute(c->stock, g);
}

enum ggml_status be_graph_compute(ggml_backend_t be, ggml_cgraph *g) {
    Ctx *c = static_cast<Ctx *>(be->context);
    Shape s = inspect(g);
    if (!s.decode) return delegate(c, g, s.why);
    Bound &b = c->bound;
    // (re)bind when the graph's buffers are not the ones the model holds
    if (!b.m || b.key_logits != s.logits->data) {
        if (b.m) sinter_model_destroy(b.m);
        b = Bound();
        sinter_model_config cfg;
        std::string why;
        if (!bind_graph(s, c->stock, cfg, b, why)) return delegate(c, g, "unbindable decode graph: " + why);
        sinter_model_bindings mb;
        std::memset(&mb, 0, sizeof mb);
        mb.tensors = b.tensors.data();
        mb.types = b.types.data();
        mb.states = b.states.data();
        mb.logits = static_cast<float *>(s.logits->data);
        mb.embed_outside = b.embed_outside ? 1u : 0u;
        if (sinter_model_create_bound(&cfg, 0, 0, &mb, &b.m) != SINTER_OK)
            return delegate(c, g, std::string("bound model refused: ") + sinter_last_error());
        b.key_logits = s.logits->data;
        if (b.embed_outside) {
            void *x = nullptr;
            size_t xb = 0;
            if (sinter_model_buffer(b.m, "X", &x, &xb) != SINTER_OK) return delegate(c, g, "no X buffer");
            b.x = static_cast<float *>(x);
        }
    }
    // this pass's inputs: position, token (or the embedded row)
    int32_t pos = 0, tok = 0;
    ggml_backend_tensor_get(s.pos, &pos, 0, sizeof pos);
    if (s.tokens) ggml_backend_tensor_get(s.tokens, &tok, 0, sizeof tok);
    if (b.embed_outside) {
        // the embedded row, device to device into the model's X
        const size_t bytes = (size_t)ggml_nelements(s.embd) * sizeof(float);
        if (s.embd->type != GGML_TYPE_F32 || sinter_model_copy(b.m, b.x, s.embd->data, bytes, 2) != SINTER_OK)
            return delegate(c, g, "embedded row copy failed");
    }
    // the KV row the stock graph would write must be the position (one
    // sequence, no holes): the kernel attends over rows [0, pos]
    if (s.named.count("k_idxs")) {
        int64_t row = -1;
        ggml_tensor *ki = s.named["k_idxs"];
        if (ki->type == GGML_TYPE_I64) ggml_backend_tensor_get(ki, &row, 0, sizeof row);
        if (row != pos) return delegate(c, g, "KV row is not the position");
    }
    if (sinter_model_decode(b.m, tok, pos, nullptr, nullptr) != SINTER_OK) {
        std::fprintf(stderr, "sinter: decode pass failed: %s\n", sinter_last_error());
        return GGML_STATUS_FAILED;
    }
    return GGML_STATUS_SUCCESS;
}

// ------------------------------------------------------------------ device

struct DevCtx {
    ggml_backend_dev_t hip = nullptr;  // the stock HIP device everything is forwarded to
};

const char *dev_name(ggml_backend_dev_t) { return "SINTER"; }
const char *dev_description(ggml_backend_dev_t) { return "sinter persistent decode on MI355X (gfx950)"; }

void dev_memory(ggml_backend_dev_t d, size_t *free, size_t *total) {
    ggml_backend_dev_memory(static_cast<DevCtx *>(d->context)->hip, free, total);
}

enum ggml_backend_dev_type dev_type(ggml_backend_dev_t) { return GGML_BACKEND_DEVICE_TYPE_GPU; }

void dev_props(ggml_backend_dev_t d, ggml_backend_dev_props *p) {
    ggml_backend_dev_get_props(static_cast<DevCtx *>(d->context)->hip, p);
    p->name = dev_name(d);
    p->description = dev_description(d);
    p->type = GGML_BACKEND_DEVICE_TYPE_GPU;
}

ggml_guid_t be_guid() {
    static ggml_guid guid = {0x73, 0x69, 0x6e, 0x74, 0x65, 0x72, 0x2d, 0x67, 0x66, 0x78, 0x39, 0x35, 0x30, 0x00, 0x00, 0x01};
    return &guid;
}

ggml_backend_t dev_init_backend(ggml_backend_dev_t d, const char *params) {
    DevCtx *dc = static_cast<DevCtx *>(d->context);
    Ctx *c = new Ctx();
    c->stock = ggml_backend_dev_init(dc->hip, params);
    if (!c->stock) {
        delete c;
        return nullptr;
    }
    ggml_backend_i iface;
    std::memset(&iface, 0, sizeof iface);
    iface.get_name = be_name;
    iface.free = be_free;
    iface.synchronize = be_synchronize;
    iface.graph_compute = be_graph_compute;   // no graph_optimize: the received order is the captured one
    return new ggml_backend{be_guid(), iface, d, c};
}

ggml_backend_buffer_type_t dev_buffer_type(ggml_backend_dev_t d) {
    return ggml_backend_dev_buffer_type(static_cast<DevCtx *>(d->context)->hip);
}

ggml_backend_buffer_type_t dev_host_buffer_type(ggml_backend_dev_t d) {
    return ggml_backend_dev_host_buffer_type(static_cast<DevCtx *>(d->context)->hip);
}

bool dev_supports_op(ggml_backend_dev_t d, const ggml_tensor *op) {
    return ggml_backend_dev_supports_op(static_cast<DevCtx *>(d->context)->hip, op);
}

bool dev_supports_buft(ggml_backend_dev_t d, ggml_backend_buffer_type_t buft) {
    return ggml_backend_dev_supports_buft(static_cast<DevCtx *>(d->context)->hip, buft);
}

// ------------------------------------------------------------------ registry

const char *reg_name(ggml_backend_reg_t) { return "SINTER"; }

struct RegCtx {
    DevCtx dctx;
    ggml_backend_device dev;
    bool have = false;
};

RegCtx *reg_ctx() {
    static RegCtx r;
    static bool init = false;
    if (init) return &r;
    init = true;
    // the stock HIP device: loaded before this library (GGML_BACKEND_PATH is
    // read last), the first GPU device whose name is not ours
    for (size_t i = 0; i < ggml_backend_dev_count(); i++) {
        ggml_backend_dev_t d = ggml_backend_dev_get(i);
        if (ggml_backend_dev_type(d) == GGML_BACKEND_DEVICE_TYPE_GPU &&
            std::strcmp(ggml_backend_dev_name(d), "SINTER") != 0) {
            r.dctx.hip = d;
            break;
        }
    }
    if (!r.dctx.hip) return &r;
    ggml_backend_device_i di;
    std::memset(&di, 0, sizeof di);
    di.get_name = dev_name;
    di.get_description = dev_description;
    di.get_memory = dev_memory;
    di.get_type = dev_type;
    di.get_props = dev_props;
    di.init_backend = dev_init_backend;
    di.get_buffer_type = dev_buffer_type;
    di.get_host_buffer_type = dev_host_buffer_type;
    di.supports_op = dev_supports_op;
    di.supports_buft = dev_supports_buft;
    r.dev.iface = di;
    r.dev.context = &r.dctx;
    r.have = true;
    return &r;
}

size_t reg_device_count(ggml_backend_reg_t) { return reg_ctx()->have ? 1 : 0; }

ggml_backend_dev_t reg_device(ggml_backend_reg_t, size_t i) {
    RegCtx *r = reg_ctx();
    return r->have && i == 0 ? &r->dev : nullptr;
}

ggml_backend_reg_t sinter_reg() {
    static ggml_backend_reg reg;
    static bool init = false;
    if (!init) {
        init = true;
        ggml_backend_reg_i ri;
        std::memset(&ri, 0, sizeof ri);
        ri.get_name = reg_name;
        ri.get_device_count = reg_device_count;
        ri.get_device = reg_device;
        reg.api_version = GGML_BACKEND_API_VERSION;
        reg.iface = ri;
        reg.context = nullptr;
        reg_ctx()->dev.reg = &reg;
    }
    return &reg;
}

}  // namespace

// Entry points of a dynamically loaded ggml backend (ggml-backend-impl.h's
// GGML_BACKEND_DL_IMPL / GGML_BACKEND_DL_SCORE_IMPL protocol).
extern "C" {
GGML_BACKEND_API ggml_backend_reg_t ggml_backend_init(void) { return sinter_reg(); }
// 0 = unusable here: no MI355X-class device visible to libsinter
GGML_BACKEND_API int ggml_backend_score(void) {
    char name[128] = "";
    return sinter_device_info(0, name, sizeof name) == SINTER_OK ? 100 : 0;
}
}
