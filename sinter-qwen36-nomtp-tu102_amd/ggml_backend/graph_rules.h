// The decisions of the ggml backend shim (sinter_ggml.cpp), on a ggml-free
// description of a received graph, so that they can be built and tested
// without a ggml tree:
//   classify   is this graph the batch-1 decode graph of a Qwen3.6-style
//              hybrid?  (docs/INTEGRATION-FINDINGS.md:182-236: one split, the
//              scheduler's copies renamed "<backend>#<name>#<c>"; a prefill
//              misses on the chunked GDN node suffix __fgdn_ch__ or a token
//              count ne[2] > 1, docs/PREFILL-SEMANTICS.md:344-377)
//   bind       resolve its weight, KV-cache, recurrent-state and logits
//              tensors and its scalars into a sinter_model_config and
//              bindings; refuse what the kernels cannot run
//   same       whether a binding still matches the bound model (every
//              pointer and type)
//   pass       this pass's inputs: the position (one id, or the 4 equal
//              M-RoPE ids of a text token) and the KV row the graph writes
#pragma once
#include <cstdint>
#include <map>
#include <string>
#include <vector>

#include "../../include/sinter.h"

namespace sinter_ggml {

// the ops the rules look at (everything else is G_OTHER)
enum GOp : int32_t { G_OTHER = 0, G_RMS_NORM = 1, G_ROPE = 2, G_GDN = 3, G_FATTN = 4 };

// ggml's rope op parameters (ggml.c ggml_rope_impl): op_params[1] rotated
// dims, [2] mode, [5] freq_base (float bits), [11..14] the M-RoPE sections
constexpr int ROPE_P_NDIMS = 1, ROPE_P_MODE = 2, ROPE_P_BASE = 5, ROPE_P_SECTIONS = 11;
constexpr int32_t ROPE_MODE_NEOX = 2, ROPE_MODE_IMROPE = 40;

// One tensor of the graph (node or leaf).
struct GTensor {
    std::string name;          // as in the graph (may carry the scheduler's copy decoration)
    int32_t op = G_OTHER;
    int32_t type = -1;         // sinter_type, -1 for a type libsinter does not know
    int64_t ne[4] = {1, 1, 1, 1};
    const void *data = nullptr;
    int32_t root = -1;         // index of the tensor a view reads from (-1: not a view)
    int32_t src0 = -1;         // index of the op's first operand (-1: none)
    int32_t op_params[16] = {};
};

struct GraphDesc {
    std::vector<GTensor> t;
};

// A tensor's name without the scheduler's copy decoration "<backend>#<name>#<c>".
std::string base_name(const std::string &n);

struct Classified {
    bool decode = false;
    std::string why;                       // why not (empty when decode)
    std::map<std::string, int32_t> named;  // tensor index by base name
    int32_t n_gdn = 0, n_attn = 0;
    int32_t logits = -1, tokens = -1, embd = -1, pos = -1, k_idxs = -1;
};
Classified classify(const GraphDesc &g);

// What a bound model runs over: the config (types from the tensors
// themselves) and sinter_model_bindings' arrays (device pointers as in the
// graph).
struct Binding {
    sinter_model_config cfg{};
    std::vector<const void *> tensors, states;
    std::vector<int32_t> types;
    const void *logits = nullptr;
    bool embed_outside = false;
};
bool bind(const GraphDesc &g, const Classified &c, Binding &b, std::string &why);
bool same_binding(const Binding &a, const Binding &b);

// This pass's position from the graph's position ids (n_ids = 1, or 4 equal
// M-RoPE ids), and the KV row the graph writes (have_row: a k_idxs input
// exists) -- which must be the position: the kernel appends at row pos and
// attends over rows [0, pos].  False (with the reason) otherwise.
bool pass_inputs(const int32_t *pos_ids, int n_ids, bool have_row, int64_t row, int32_t &pos, std::string &why);

}  // namespace sinter_ggml
