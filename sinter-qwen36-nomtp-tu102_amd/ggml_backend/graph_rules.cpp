// The ggml backend shim's decisions on a ggml-free graph description (see
// graph_rules.h), and a C ABI over them for tests (sinter_rules_*).
#include "graph_rules.h"

#include <cstring>

namespace sinter_ggml {

std::string base_name(const std::string &n) {
    const size_t a = n.find('#');
    if (a == std::string::npos) return n;
    const size_t b = n.rfind('#');
    return b > a ? n.substr(a + 1, b - a - 1) : n.substr(a + 1);
}

static int64_t nelem(const GTensor &t) { return t.ne[0] * t.ne[1] * t.ne[2] * t.ne[3]; }

static const GTensor &root_of(const GraphDesc &g, int32_t i) {
    while (g.t[(size_t)i].root >= 0) i = g.t[(size_t)i].root;
    return g.t[(size_t)i];
}

Classified classify(const GraphDesc &g) {
    Classified c;
    const int32_t n = (int32_t)g.t.size();
    for (int32_t i = 0; i < n; i++) {
        const GTensor &t = g.t[(size_t)i];
        if (!t.name.empty()) c.named.emplace(base_name(t.name), i);
    }
    for (int32_t i = 0; i < n; i++) {
        const GTensor &t = g.t[(size_t)i];
        if (t.op == G_GDN) {
            if (t.name.find("__fgdn_ch__") != std::string::npos) { c.why = "prefill (chunked GDN node)"; return c; }
            if (t.name.find("__fgdn_ar__") == std::string::npos) { c.why = "GDN node without the decode suffix"; return c; }
            // ne[2] of q is the token count of the ubatch
            if (t.src0 < 0 || g.t[(size_t)t.src0].ne[2] != 1) { c.why = "GDN over more than one token"; return c; }
            c.n_gdn++;
        } else if (t.op == G_FATTN) {
            // q is [head dim, tokens, heads, ...]
            if (t.src0 < 0 || g.t[(size_t)t.src0].ne[1] != 1) { c.why = "attention over more than one query"; return c; }
            c.n_attn++;
        } else if (t.op == G_ROPE) {
            const int32_t mode = t.op_params[ROPE_P_MODE];
            if (mode != ROPE_MODE_NEOX && mode != ROPE_MODE_IMROPE) { c.why = "rope mode neither NEOX nor IMROPE"; return c; }
        }
    }
    auto find = [&](const char *nm) {
        auto it = c.named.find(nm);
        return it == c.named.end() ? -1 : it->second;
    };
    c.logits = find("result_output");
    c.tokens = find("inp_tokens");
    c.embd = find("inp_embd");
    c.pos = find("inp_pos");
    c.k_idxs = find("k_idxs");
    if (c.logits < 0 || g.t[(size_t)c.logits].ne[1] != 1) { c.why = "no single-row result_output"; return c; }
    // one position id per token, or the 4 M-RoPE ids of one token
    if (c.pos < 0 || !(nelem(g.t[(size_t)c.pos]) == 1 || nelem(g.t[(size_t)c.pos]) == 4)) {
        c.why = "no single token position";
        return c;
    }
    if (c.tokens >= 0 && nelem(g.t[(size_t)c.tokens]) != 1) { c.why = "more than one token id"; return c; }
    if (c.tokens < 0 && c.embd < 0) { c.why = "neither token ids nor an embedded row as input"; return c; }
    if (c.n_gdn == 0 || c.n_attn == 0) { c.why = "not the hybrid decode graph"; return c; }
    c.decode = true;
    return c;
}

// the weight types the GEMV kernels read; vectors must be f32
static bool matrix_type_ok(int32_t t) {
    return t == SINTER_Q4_K || t == SINTER_Q6_K || t == SINTER_Q8_0 || t == SINTER_BF16 || t == SINTER_F32;
}

// Per-layer weight names in the slot numbering of sinter_model_tensor_info.
static const char *const kCommon[5] = {"attn_norm.weight", "post_attention_norm.weight", "ffn_gate.weight",
                                       "ffn_up.weight", "ffn_down.weight"};
static const bool kCommonVec[5] = {true, true, false, false, false};
static const char *const kGdn[9] = {"attn_qkv.weight", "attn_gate.weight", "ssm_alpha.weight", "ssm_beta.weight",
                                    "ssm_out.weight", "ssm_conv1d.weight", "ssm_dt.bias", "ssm_a", "ssm_norm.weight"};
static const bool kGdnVec[9] = {false, false, false, false, false, true, true, true, true};
static const char *const kAttn[6] = {"attn_q.weight", "attn_k.weight", "attn_v.weight", "attn_output.weight",
                                     "attn_q_norm.weight", "attn_k_norm.weight"};
static const bool kAttnVec[6] = {false, false, false, false, true, true};

bool bind(const GraphDesc &g, const Classified &cl, Binding &b, std::string &why) {
    b = Binding();
    auto get = [&](const std::string &n) -> const GTensor * {
        auto it = cl.named.find(n);
        return it == cl.named.end() ? nullptr : &g.t[(size_t)it->second];
    };
    sinter_model_config &c = b.cfg;
    std::memset(&c, 0, sizeof c);
    const GTensor *embd_w = get("token_embd.weight"), *out_w = get("output.weight"), *onorm = get("output_norm.weight");
    if (!onorm) { why = "no output_norm.weight"; return false; }
    if (!out_w) out_w = embd_w;                    // tied head
    if (!out_w) { why = "no head weight"; return false; }
    c.n_layer = cl.n_gdn + cl.n_attn;
    c.n_embd = (int32_t)out_w->ne[0];
    c.n_vocab = (int32_t)out_w->ne[1];
    // scalars no weight carries, from the ops that use them -- required, all
    // equal: the RMS-norm epsilon (op_params[0]), the rope's rotated dims and
    // base
    bool have_eps = false, have_rope = false;
    for (const GTensor &t : g.t) {
        if (t.op == G_RMS_NORM) {
            float e;
            std::memcpy(&e, &t.op_params[0], sizeof e);
            if (have_eps && e != c.eps) { why = "RMS norms with different eps"; return false; }
            c.eps = e;
            have_eps = true;
        } else if (t.op == G_ROPE) {
            float base;
            std::memcpy(&base, &t.op_params[ROPE_P_BASE], sizeof base);
            if (have_rope && (t.op_params[ROPE_P_NDIMS] != c.rope_dims || base != c.rope_base)) {
                why = "ropes with different dims or base";
                return false;
            }
            c.rope_dims = t.op_params[ROPE_P_NDIMS];
            c.rope_base = base;
            have_rope = true;
        }
    }
    if (!have_eps) { why = "no RMS_NORM to read eps from"; return false; }
    if (!have_rope) { why = "no ROPE to read the rotated dims and base from"; return false; }
    // the layer pattern: attention every attn_every layers, the rest GDN
    int first_attn = -1;
    for (int il = 0; il < c.n_layer && first_attn < 0; il++)
        if (get("blk." + std::to_string(il) + ".attn_q.weight")) first_attn = il;
    if (first_attn < 0) { why = "no attention layer"; return false; }
    c.attn_every = first_attn + 1;
    for (int il = 0; il < c.n_layer; il++) {
        const bool at = get("blk." + std::to_string(il) + ".attn_q.weight") != nullptr;
        if (at != (il % c.attn_every == c.attn_every - 1)) { why = "layer pattern is not every " + std::to_string(c.attn_every); return false; }
    }
    const std::string l0 = "blk." + std::to_string(first_attn) + ".";
    const GTensor *wq = get(l0 + "attn_q.weight"), *wk = get(l0 + "attn_k.weight"), *wv = get(l0 + "attn_v.weight");
    const GTensor *qn = get(l0 + "attn_q_norm.weight");
    const GTensor *up = get("blk.0.ffn_up.weight"), *down = get("blk.0.ffn_down.weight"), *qkv = get("blk.0.attn_qkv.weight");
    const GTensor *sa = get("blk.0.ssm_a"), *sn = get("blk.0.ssm_norm.weight"), *cw = get("blk.0.ssm_conv1d.weight");
    if (!wq || !wk || !wv || !qn || !up || !down || !qkv || !sa || !sn || !cw) {
        why = "layer 0 / first attention layer incomplete";
        return false;
    }
    c.conv_k = (int32_t)cw->ne[0];
    c.head_dim = (int32_t)qn->ne[0];
    c.attn_nq = (int32_t)(wq->ne[1] / (2 * c.head_dim));
    c.attn_nkv = (int32_t)(wk->ne[1] / c.head_dim);
    c.n_ff = (int32_t)up->ne[1];
    c.gdn_d = (int32_t)sn->ne[0];
    c.gdn_hv = (int32_t)nelem(*sa);
    c.gdn_hk = (int32_t)((qkv->ne[1] / c.gdn_d - c.gdn_hv) / 2);
    // the configuration's per-kind types are the first layers' own (each
    // binding carries its tensor's type, so mixed-type models bind too)
    c.t_default = qkv->type;
    c.t_attn_v = wv->type;
    c.t_ffn_down = down->type;
    c.t_output = out_w->type;
    c.t_embd = embd_w ? embd_w->type : out_w->type;
    // the KV cache (views of cache_k_l<il> / cache_v_l<il>): f16 or q8_0 rows
    const GTensor *kc0 = get("cache_k_l" + std::to_string(first_attn));
    if (!kc0) { why = "no KV cache tensor"; return false; }
    const int32_t kc0i = cl.named.at("cache_k_l" + std::to_string(first_attn));
    const GTensor &kr = root_of(g, kc0i);
    if (kr.type != SINTER_F16 && kr.type != SINTER_Q8_0) { why = "KV cache neither f16 nor q8_0"; return false; }
    c.t_kv = kr.type;
    c.n_ctx = (int32_t)(nelem(kr) / ((int64_t)c.attn_nkv * c.head_dim));

    const size_t nt = (size_t)c.n_layer * 16 + 3;
    b.tensors.assign(nt, nullptr);
    b.types.assign(nt, SINTER_F32);
    b.states.assign((size_t)c.n_layer * 2, nullptr);
    auto put = [&](size_t i, const GTensor *t, bool vec, const std::string &nm) -> bool {
        if (!t) { why = "missing " + nm; return false; }
        if (vec ? t->type != SINTER_F32 : !matrix_type_ok(t->type)) { why = nm + ": a type the kernels do not read"; return false; }
        b.tensors[i] = t->data;
        b.types[i] = t->type;
        return true;
    };
    const int64_t C = (int64_t)(2 * c.gdn_hk + c.gdn_hv) * c.gdn_d;
    for (int il = 0; il < c.n_layer; il++) {
        const std::string p = "blk." + std::to_string(il) + ".";
        const bool at = il % c.attn_every == c.attn_every - 1;
        for (int k = 0; k < 5; k++)
            if (!put((size_t)il * 16 + k, get(p + kCommon[k]), kCommonVec[k], p + kCommon[k])) return false;
        const int nk = at ? 6 : 9;
        for (int k = 0; k < nk; k++) {
            const char *nm = at ? kAttn[k] : kGdn[k];
            if (!put((size_t)il * 16 + 5 + k, get(p + nm), at ? kAttnVec[k] : kGdnVec[k], p + nm)) return false;
        }
        const std::string sfx = std::to_string(il);
        const std::string n0 = (at ? "cache_k_l" : "cache_r_l") + sfx, n1 = (at ? "cache_v_l" : "cache_s_l") + sfx;
        if (!cl.named.count(n0) || !cl.named.count(n1)) { why = "state of layer " + sfx; return false; }
        const GTensor &s0 = root_of(g, cl.named.at(n0)), &s1 = root_of(g, cl.named.at(n1));
        if (at) {
            if (s0.type != c.t_kv || s1.type != c.t_kv || nelem(s0) != nelem(kr) || nelem(s1) != nelem(kr)) {
                why = "KV cache of layer " + sfx + " unlike layer " + std::to_string(first_attn) + "'s";
                return false;
            }
        } else if (s0.type != SINTER_F32 || s1.type != SINTER_F32 || nelem(s0) < C * (c.conv_k - 1) ||
                   nelem(s1) < (int64_t)c.gdn_hv * c.gdn_d * c.gdn_d) {
            why = "recurrent state of layer " + sfx + " not f32 or too small";
            return false;
        }
        b.states[(size_t)il * 2] = s0.data;
        b.states[(size_t)il * 2 + 1] = s1.data;
    }
    b.embed_outside = cl.tokens < 0;
    const size_t g0 = (size_t)c.n_layer * 16;
    if (!b.embed_outside && !put(g0, embd_w, false, "token_embd.weight")) return false;
    if (!put(g0 + 1, onorm, true, "output_norm.weight") || !put(g0 + 2, out_w, false, "head weight")) return false;
    b.logits = g.t[(size_t)cl.logits].data;
    return true;
}

bool same_binding(const Binding &a, const Binding &b) {
    return a.tensors == b.tensors && a.types == b.types && a.states == b.states && a.logits == b.logits &&
           a.embed_outside == b.embed_outside && std::memcmp(&a.cfg, &b.cfg, sizeof a.cfg) == 0;
}

bool pass_inputs(const int32_t *pos_ids, int n_ids, bool have_row, int64_t row, int32_t &pos, std::string &why) {
    if (!pos_ids || !(n_ids == 1 || n_ids == 4)) { why = "no single token position"; return false; }
    // the M-RoPE ids of a text token are equal; then IMROPE is NEOX rope at that position
    for (int i = 1; i < n_ids; i++)
        if (pos_ids[i] != pos_ids[0]) { why = "M-RoPE position ids differ (not a text token)"; return false; }
    pos = pos_ids[0];
    if (pos < 0) { why = "negative position"; return false; }
    if (have_row && row != pos) { why = "KV row is not the position"; return false; }
    return true;
}

}  // namespace sinter_ggml

// ------------------------------------------------------------------ C ABI for tests

extern "C" {

// one tensor of a flattened description
typedef struct sinter_rules_tensor {
    const char *name;
    int32_t op, type;
    int64_t ne[4];
    uint64_t data;
    int32_t root, src0;
    int32_t op_params[16];
} sinter_rules_tensor;

static sinter_ggml::GraphDesc to_desc(const sinter_rules_tensor *t, int n) {
    sinter_ggml::GraphDesc g;
    g.t.resize((size_t)n);
    for (int i = 0; i < n; i++) {
        sinter_ggml::GTensor &d = g.t[(size_t)i];
        d.name = t[i].name ? t[i].name : "";
        d.op = t[i].op;
        d.type = t[i].type;
        for (int k = 0; k < 4; k++) d.ne[k] = t[i].ne[k];
        d.data = reinterpret_cast<const void *>(t[i].data);
        d.root = t[i].root;
        d.src0 = t[i].src0;
        std::memcpy(d.op_params, t[i].op_params, sizeof d.op_params);
    }
    return g;
}

static void copy_why(const std::string &w, char *why, int cap) {
    if (why && cap > 0) {
        std::strncpy(why, w.c_str(), (size_t)cap - 1);
        why[cap - 1] = 0;
    }
}

// 1: the batch-1 decode graph; 0: delegated (why says which rule)
int sinter_rules_classify(const sinter_rules_tensor *t, int n, char *why, int cap) {
    const sinter_ggml::Classified c = sinter_ggml::classify(to_desc(t, n));
    copy_why(c.why, why, cap);
    return c.decode ? 1 : 0;
}

// 1: bound (cfg, tensors[n_layer*16+3], types, states[n_layer*2], logits,
// embed_outside filled); 0: refused (why).  Capacities are checked.
int sinter_rules_bind(const sinter_rules_tensor *t, int n, sinter_model_config *cfg, uint64_t *tensors,
                      int32_t *types, int tensor_cap, uint64_t *states, int state_cap, uint64_t *logits,
                      int *embed_outside, char *why, int cap) {
    const sinter_ggml::GraphDesc g = to_desc(t, n);
    const sinter_ggml::Classified c = sinter_ggml::classify(g);
    if (!c.decode) { copy_why(c.why, why, cap); return 0; }
    sinter_ggml::Binding b;
    std::string w;
    if (!sinter_ggml::bind(g, c, b, w)) { copy_why(w, why, cap); return 0; }
    if ((int)b.tensors.size() > tensor_cap || (int)b.states.size() > state_cap) { copy_why("capacity", why, cap); return 0; }
    *cfg = b.cfg;
    for (size_t i = 0; i < b.tensors.size(); i++) {
        tensors[i] = reinterpret_cast<uint64_t>(b.tensors[i]);
        types[i] = b.types[i];
    }
    for (size_t i = 0; i < b.states.size(); i++) states[i] = reinterpret_cast<uint64_t>(b.states[i]);
    *logits = reinterpret_cast<uint64_t>(b.logits);
    *embed_outside = b.embed_outside ? 1 : 0;
    copy_why("", why, cap);
    return 1;
}

// 1: both descriptions bind, to the same binding; 0: they bind differently
// (a bound model would be rebuilt); -1: one of them does not bind
int sinter_rules_same_binding(const sinter_rules_tensor *a, int na, const sinter_rules_tensor *b, int nb) {
    const sinter_ggml::GraphDesc ga = to_desc(a, na), gb = to_desc(b, nb);
    const sinter_ggml::Classified ca = sinter_ggml::classify(ga), cb = sinter_ggml::classify(gb);
    sinter_ggml::Binding ba, bb;
    std::string w;
    if (!ca.decode || !cb.decode || !sinter_ggml::bind(ga, ca, ba, w) || !sinter_ggml::bind(gb, cb, bb, w)) return -1;
    return sinter_ggml::same_binding(ba, bb) ? 1 : 0;
}

// 1: this pass runs at *pos; 0: delegated (why)
int sinter_rules_pass_inputs(const int32_t *pos_ids, int n_ids, int have_row, int64_t row, int32_t *pos, char *why,
                             int cap) {
    int32_t p = -1;
    std::string w;
    const bool ok = sinter_ggml::pass_inputs(pos_ids, n_ids, have_row != 0, row, p, w);
    copy_why(w, why, cap);
    if (pos) *pos = p;
    return ok ? 1 : 0;
}

}  // extern "C"
