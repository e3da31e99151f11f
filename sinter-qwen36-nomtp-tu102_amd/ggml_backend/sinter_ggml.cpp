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
// The decisions themselves (which graph is a decode graph, what it binds to,
// when to rebind, which pass inputs run) are graph_rules.cpp's, over a
// ggml-free description of the graph, so they are tested without ggml.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "ggml-backend-impl.h"
#include "ggml-backend.h"
#include "ggml.h"
#include "graph_rules.h"
#include "sinter.h"

namespace {

using namespace sinter_ggml;

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

int32_t op_of(ggml_op op) {
    switch (op) {
    case GGML_OP_RMS_NORM: return G_RMS_NORM;
    case GGML_OP_ROPE: return G_ROPE;
    case GGML_OP_GATED_DELTA_NET: return G_GDN;
    case GGML_OP_FLASH_ATTN_EXT: return G_FATTN;
    default: return G_OTHER;
    }
}

// The ggml-free description of a received graph (graph_rules.h): every node,
// its operands and the tensors views read from.
struct Described {
    GraphDesc g;
    std::map<const ggml_tensor *, int32_t> index;
    std::vector<const ggml_tensor *> ptr;
};

int32_t add(Described &d, const ggml_tensor *t) {
    if (!t) return -1;
    auto it = d.index.find(t);
    if (it != d.index.end()) return it->second;
    const int32_t i = (int32_t)d.g.t.size();
    d.index.emplace(t, i);
    d.g.t.emplace_back();
    d.ptr.push_back(t);
    const int32_t root = add(d, t->view_src), src0 = add(d, t->src[0]);
    GTensor &g = d.g.t[(size_t)i];   // (after the recursive adds: the vector may have grown)
    g.name = t->name;
    g.op = op_of(t->op);
    g.type = sinter_type_of(t->type);
    for (int k = 0; k < 4; k++) g.ne[k] = t->ne[k];
    g.data = t->data;
    g.root = root;
    g.src0 = src0;
    std::memcpy(g.op_params, t->op_params, sizeof g.op_params);
    return i;
}

Described describe(ggml_cgraph *graph) {
    Described d;
    const int n = ggml_graph_n_nodes(graph);
    for (int i = 0; i < n; i++) {
        ggml_tensor *t = ggml_graph_node(graph, i);
        add(d, t);
        for (int j = 0; j < GGML_MAX_SRC; j++) add(d, t->src[j]);
    }
    return d;
}

// ------------------------------------------------------------------ backend

struct Ctx {
    ggml_backend_t stock = nullptr;    // the HIP backend every miss goes to
    sinter_model *m = nullptr;         // bound to `bound`
    Binding bound;
    std::vector<void *> tensors, states;   // sinter_model_bindings' arrays of `bound`
    float *x = nullptr;                // the model's X buffer (embed_outside)
    std::map<std::string, int> misses; // reasons already logged
};

const char *be_name(ggml_backend_t) { return "SINTER"; }

void be_free(ggml_backend_t be) {
    Ctx *c = static_cast<Ctx *>(be->context);
    if (c->m) sinter_model_destroy(c->m);
    if (c->stock) ggml_backend_free(c->stock);
    delete c;
    delete be;
}

void be_synchronize(ggml_backend_t be) { ggml_backend_synchronize(static_cast<Ctx *>(be->context)->stock); }

enum ggml_status delegate(Ctx *c, ggml_cgraph *g, const std::string &why) {
    if (c->misses[why]++ == 0) std::fprintf(stderr, "sinter: graph delegated to the stock backend: %s\n", why.c_str());
    return ggml_backend_graph_compute(c->stock, g);
}

// (Re)build the bound model over `now` -- whenever any bound pointer or type
// differs from the model's, not only the logits buffer.
bool rebind(Ctx *c, const Binding &now, std::string &why) {
    if (c->m) sinter_model_destroy(c->m);
    c->m = nullptr;
    c->x = nullptr;
    c->bound = now;
    c->tensors.assign(now.tensors.size(), nullptr);
    c->states.assign(now.states.size(), nullptr);
    for (size_t i = 0; i < now.tensors.size(); i++) c->tensors[i] = const_cast<void *>(now.tensors[i]);
    for (size_t i = 0; i < now.states.size(); i++) c->states[i] = const_cast<void *>(now.states[i]);
    sinter_model_bindings mb;
    std::memset(&mb, 0, sizeof mb);
    mb.tensors = c->tensors.data();
    mb.types = c->bound.types.data();
    mb.states = c->states.data();
    mb.logits = static_cast<float *>(const_cast<void *>(now.logits));
    mb.embed_outside = now.embed_outside ? 1u : 0u;
    if (sinter_model_create_bound(&c->bound.cfg, 0, 0, &mb, &c->m) != SINTER_OK) {
        why = std::string("bound model refused: ") + sinter_last_error();
        c->m = nullptr;
        return false;
    }
    if (now.embed_outside) {
        void *x = nullptr;
        size_t xb = 0;
        if (sinter_model_buffer(c->m, "X", &x, &xb) != SINTER_OK) { why = "no X buffer"; return false; }
        c->x = static_cast<float *>(x);
    }
    return true;
}

enum ggml_status be_graph_compute(ggml_backend_t be, ggml_cgraph *g) {
    Ctx *c = static_cast<Ctx *>(be->context);
    const Described d = describe(g);
    const Classified cl = classify(d.g);
    if (!cl.decode) return delegate(c, g, cl.why);
    Binding now;
    std::string why;
    if (!bind(d.g, cl, now, why)) return delegate(c, g, "unbindable decode graph: " + why);
    // this pass's inputs: position (1 or 4 M-RoPE ids), the KV row the graph
    // writes, the token (or the embedded row)
    const ggml_tensor *pt = d.ptr[(size_t)cl.pos];
    int32_t ids[4] = {0, 0, 0, 0}, pos = 0, tok = 0;
    const int n_ids = (int)ggml_nelements(pt);
    ggml_backend_tensor_get(const_cast<ggml_tensor *>(pt), ids, 0, (size_t)n_ids * sizeof(int32_t));
    int64_t row = -1;
    const bool have_row = cl.k_idxs >= 0;
    if (have_row) {
        const ggml_tensor *ki = d.ptr[(size_t)cl.k_idxs];
        if (ki->type != GGML_TYPE_I64) return delegate(c, g, "k_idxs not i64");
        ggml_backend_tensor_get(const_cast<ggml_tensor *>(ki), &row, 0, sizeof row);
    }
    if (!pass_inputs(ids, n_ids, have_row, row, pos, why)) return delegate(c, g, why);
    if (!c->m || !same_binding(c->bound, now))
        if (!rebind(c, now, why)) return delegate(c, g, why);
    if (cl.tokens >= 0) ggml_backend_tensor_get(const_cast<ggml_tensor *>(d.ptr[(size_t)cl.tokens]), &tok, 0, sizeof tok);
    if (now.embed_outside) {
        // the embedded row, device to device into the model's X
        const ggml_tensor *e = d.ptr[(size_t)cl.embd];
        const size_t bytes = (size_t)ggml_nelements(e) * sizeof(float);
        if (e->type != GGML_TYPE_F32 || sinter_model_copy(c->m, c->x, e->data, bytes, 2) != SINTER_OK)
            return delegate(c, g, "embedded row copy failed");
    }
    if (sinter_model_decode(c->m, tok, pos, nullptr, nullptr) != SINTER_OK) {
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
