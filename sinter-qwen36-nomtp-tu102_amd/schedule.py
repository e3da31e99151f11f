"""This build's schedule compiler (host side).

Input: a ggml decode graph in the extraction format of the reference's
k0/schedule.csv + k0/leaves.csv (one row per node: op, type, ne, sources,
block, macro op; one row per leaf: type, ne, classification; see
k0/compile_schedule.py:75-108 for the reader it replaces).

Output:
  * node accounting -- which nodes a single-sequence decode pass executes and
    which it drops, by category (k0/program.json "coverage" / "drops");
  * per-pass DRAM bytes as a function of the attended positions n_kv
    (k0/program.json "per_pass.dram_bytes", k0/compile_schedule.py:838-851);
  * this build's fused program: every live node assigned to exactly one of
    this build's ops (GEMV with its prologue and epilogue, GDN_STEP,
    ATTN_DECODE), one grid barrier after each op, as a SYMBOLIC program whose
    operands are names -- gguf:<tensor>, buf:<activation>, state:<role>.<layer>,
    cell:<pass cell field> -- that pack() resolves against a sinter Model
    (the symbolic-program contract of k0/compile_schedule.py:946-990 and the
    packer of k0/harness.cpp:589-628, restated for this ISA).

The fusion is this build's own: where the reference emits one instruction
per macro op and merges adjacent independent windows (964 barriers per pass
at its granularity), this ISA fuses each layer into five ops -- mixer input
projections (norm + GEMV + conv), the recurrent step or attention, the mixer
output projection (gated norm + GEMV + residual), the FFN gate/up (norm +
GEMV + SwiGLU) and down (GEMV + residual) -- plus the head, so a 64-layer
pass has 321 barriers.
"""
import csv
import json
from collections import Counter, defaultdict

# bytes per element of the graph's tensor types (logical, unpadded)
BPE = {"f32": 4.0, "f16": 2.0, "bf16": 2.0, "i32": 4.0, "i64": 8.0, "q4_0": 18.0 / 32.0,
       "q4_0_ar16": 10.0 / 16.0, "q8_0": 34.0 / 32.0, "q4_k": 144.0 / 256.0, "q6_k": 210.0 / 256.0}


class Graph:
    def __init__(self, nodes, leaves):
        self.nodes = nodes      # idx -> dict(op, type, ne, params, src, block, mid, mkind)
        self.leaves = leaves    # idx -> dict(type, ne, cls)
        self.users = defaultdict(list)
        for i, n in nodes.items():
            for s in n["src"]:
                self.users[s].append(i)

    def leaf(self, ref):
        return self.leaves[int(ref[1:])]

    def node(self, ref):
        return self.nodes[int(ref[1:])]


def load(schedule_csv, leaves_csv):
    nodes, leaves = {}, {}
    with open(schedule_csv) as f:
        for r in csv.DictReader(f):
            nodes[int(r["node_idx"])] = {
                "op": r["op"], "type": r["type"], "ne": [int(x) for x in r["ne"].split("x")],
                "params": r["decoded_params"], "src": r["src_refs"].split(";") if r["src_refs"] else [],
                "block": r["block_idx"], "mid": int(r["macro_op_id"]), "mkind": r["macro_kind"]}
    with open(leaves_csv) as f:
        for r in csv.DictReader(f):
            leaves[int(r["leaf_idx"])] = {"type": r["type"], "ne": [int(x) for x in r["ne"].split("x")],
                                          "cls": r["classification"]}
    return Graph(nodes, leaves)


def numel(ne):
    n = 1
    for d in ne:
        n *= d
    return n


# ------------------------------------------------------------------ accounting

def _state_leaf(g, i):
    """The recurrent-state leaf class (conv_state / ssm_state) a node reads,
    directly or through other nodes, or None."""
    seen, todo = set(), ["n%d" % i]
    while todo:
        r = todo.pop()
        if r in seen:
            continue
        seen.add(r)
        if r.startswith("l"):
            c = g.leaf(r)["cls"]
            if c.startswith("state:"):
                return c.split(":", 1)[1].split("(")[0]
        else:
            todo += g.node(r)["src"]
    return None


def drops(g):
    """Nodes a single-sequence decode pass does not execute, by category:
    views of the recurrent-state row indices that nothing reads, the
    zero-extent clear chains of the conv and the ssm state (no sequence to
    clear), and the f32 -> f16 mask conversion (the host writes the f16
    mask)."""
    out = {"dead_index_views": [], "zero_extent_conv_state_chain": [], "zero_extent_ssm_state_chain": [],
           "host_mask_conversion": []}
    for i, n in sorted(g.nodes.items()):
        ref = "n%d" % i
        if n["op"] == "VIEW" and not g.users[ref] and all(
                s.startswith("l") and g.leaf(s)["cls"].startswith("other:rs_") for s in n["src"]):
            out["dead_index_views"].append(i)
        elif 0 in n["ne"]:
            kind = _state_leaf(g, i)
            if kind not in ("conv_state", "ssm_state"):
                raise ValueError("zero-extent node %d reads no recurrent state" % i)
            out["zero_extent_%s_chain" % kind].append(i)
        elif n["op"] == "CPY" and n["type"] == "f16" and any(
                s.startswith("l") and g.leaf(s)["cls"] == "mask" for s in n["src"]):
            out["host_mask_conversion"].append(i)
    return out


def accounting(g):
    d = drops(g)
    dropped = sum(len(v) for v in d.values())
    return {"nodes": len(g.nodes), "emitted_nodes": len(g.nodes) - dropped, "dropped_nodes": dropped,
            "drops": {k: len(v) for k, v in d.items()}}


def live_nodes(g):
    dead = set(i for v in drops(g).values() for i in v)
    return [i for i in sorted(g.nodes) if i not in dead]


# ------------------------------------------------------------------ DRAM bytes

def dram(g, logits_copies=3):
    """Per-pass DRAM bytes: fixed + per_n_kv * n_kv.  Weights are read once
    at their logical size (the embedding table contributes one row); the
    recurrent and conv states are read and written once; each attention
    layer appends one K and one V row and reads every K/V row and f16 mask
    element of the attended positions.  logits_copies counts the vocab-sized
    f32 logits traffic (the reference's harness writes them and copies them
    once more: 3; this build writes them once: 1)."""
    weight_stream, embd_row, ssm, conv = 0.0, 0.0, 0, 0
    kv_row, mask_bpe, n_attn = 0, 0.0, 0
    for l in g.leaves.values():
        cls = l["cls"]
        if cls == "weight:token_embd.weight":
            embd_row = l["ne"][0] * BPE[l["type"]]
        elif cls.startswith("weight:"):
            weight_stream += numel(l["ne"]) * BPE[l["type"]]
        elif cls.startswith("state:ssm_state"):
            ssm += numel(l["ne"]) * int(BPE[l["type"]])
        elif cls.startswith("state:conv_state"):
            conv += numel(l["ne"]) * int(BPE[l["type"]])
        elif cls.startswith("cache_k(") or cls.startswith("cache_v("):
            kv_row += l["ne"][0] * int(BPE[l["type"]])
            n_attn += cls.startswith("cache_k(")
    masks = [l for l in g.leaves.values() if l["cls"] == "mask" and l["type"] == "f16"]
    mask_bpe = BPE[masks[0]["type"]] if masks else 0.0
    vocab = max(n["ne"][0] for n in g.nodes.values() if n["mkind"] == "head_gemv")
    state_rw = 2 * (ssm + conv)
    logits = vocab * 4 * logits_copies
    fixed = weight_stream + embd_row + state_rw + kv_row + logits
    per_n_kv = kv_row + n_attn * mask_bpe
    return {"weight_stream": weight_stream, "embd_row": embd_row, "state_rw": state_rw, "kv_append_write": kv_row,
            "logits_rw": logits, "fixed": fixed, "per_n_kv": per_n_kv,
            "formula": "%d + %d * n_kv" % (round(fixed), round(per_n_kv))}


# ------------------------------------------------------------------ fusion

# the five ops of a layer and the head, in program order
P, S, A, O, G, D, H = "proj", "step", "attn", "out", "ffn_gate_up", "ffn_down", "head"
# weight name (without "blk.N." and ".weight") -> the op its GEMV belongs to
GEMV_OP = {"attn_qkv": P, "attn_gate": P, "ssm_alpha": P, "ssm_beta": P, "attn_q": P, "attn_k": P, "attn_v": P,
           "ssm_out": O, "attn_output": O, "ffn_gate": G, "ffn_up": G, "ffn_down": D, "output": H}
# macro kind -> op of its other nodes (rmsnorm and residual_add by ordinal)
KIND_OP = {"embed_lookup": P, "conv_state_shift": P, "conv_concat_store": P, "ssm_conv_silu": P, "qkv_mmvq": P,
           "qk_l2norm": S, "gdn_gates": S, "ssm_state_fetch": S, "deltanet_step": S, "ssm_state_store": S,
           "gated_out_norm": O, "out_proj_ar16": O, "o_gemv": O,
           "q_gemv_norm_rope": A, "k_gemv_norm_rope": A, "v_gemv": A, "kv_append": A, "fattn_prep": A,
           "fattn_decode": A, "attn_gate_out": A, "ffn_fused": G, "logits_row_select": H, "head_gemv": H}
GDN_ORDER, ATTN_ORDER = (P, S, O, G, D), (P, A, O, G, D)


def _weights(g, n):
    return [g.leaf(s)["cls"].split(":", 1)[1] for s in n["src"]
            if s.startswith("l") and g.leaf(s)["cls"].startswith("weight:")]


def _short(name):
    """blk.N.attn_qkv.weight -> attn_qkv; output.weight -> output"""
    parts = name.split(".")
    if parts[0] == "blk":
        parts = parts[2:]
    return ".".join(p for p in parts if p != "weight")


def fuse(g):
    """Assign every live node to one op of this build's program: returns
    (ops, owner) where ops is the program order [(layer, role), ...] and
    owner maps node -> index into ops.  Raises ValueError on a node no op
    can take or on a graph edge that would run backwards across ops."""
    live = live_nodes(g)
    layers = sorted({int(g.nodes[i]["block"]) for i in live if g.nodes[i]["block"].isdigit()})
    kinds = defaultdict(set)
    for i in live:
        kinds[g.nodes[i]["block"]].add(g.nodes[i]["mkind"])
    ltype = {}
    for il in layers:
        k = kinds[str(il)]
        if "deltanet_step" in k and "fattn_decode" not in k:
            ltype[il] = "gdn"
        elif "fattn_decode" in k and "deltanet_step" not in k:
            ltype[il] = "attn"
        else:
            raise ValueError("block %d is neither a GDN nor an attention layer" % il)
    ops = []
    for il in layers:
        ops += [(il, r) for r in (GDN_ORDER if ltype[il] == "gdn" else ATTN_ORDER)]
    ops.append((None, H))
    index = {op: k for k, op in enumerate(ops)}
    # the silu of the z gate is the z segment's epilogue: nodes of
    # gated_out_norm computed from the attn_gate GEMV alone go to the proj op
    owner, seen_norm, seen_add = {}, Counter(), Counter()
    for i in live:
        n = g.nodes[i]
        blk = n["block"]
        il = 0 if blk == "pre" else (None if blk == "post" else int(blk))
        role = None
        ws = _weights(g, n)
        if n["op"] == "MUL_MAT" and ws:
            role = GEMV_OP.get(_short(ws[0]))
        elif n["mkind"] == "rmsnorm":
            role = H if il is None else (P if seen_norm[blk] < 2 else G)
        elif n["mkind"] == "residual_add":
            role = O if seen_add[blk] == 0 else D
            seen_add[blk] += 1
        elif n["mkind"] == "gated_out_norm" and all(
                s.startswith("n") and owner.get(int(s[1:])) == index.get((il, P)) for s in n["src"]):
            role = P
        elif n["mkind"] == "ffn_fused" and n["op"] != "GLU" and any(
                s.startswith("n") and owner.get(int(s[1:])) == index.get((il, D)) for s in n["src"]):
            role = D
        else:
            role = KIND_OP.get(n["mkind"])
        if n["mkind"] == "rmsnorm":
            seen_norm[blk] += 1
        if role is None or (il, role) not in index:
            raise ValueError("node %d (%s, %s) fits no op" % (i, n["op"], n["mkind"]))
        owner[i] = index[(il, role)]
    # every edge runs forward: an op only reads what earlier ops (or itself) produced
    for i in live:
        for s in g.nodes[i]["src"]:
            if s.startswith("n") and int(s[1:]) in owner and owner[int(s[1:])] > owner[i]:
                raise ValueError("node %d reads node %s of a later op" % (i, s))
    return ops, owner


def symbolic_program(g):
    """This build's program for graph g as a list of symbolic instructions:
    {"kind": GEMV | GDN_STEP | ATTN_DECODE | BOUNDARY, "layer": N, "role": ...,
    operands by name}.  One BOUNDARY after every op except the head (the pass
    end closes it)."""
    ops, owner = fuse(g)
    live = live_nodes(g)
    by_op = defaultdict(list)
    for i in live:
        by_op[owner[i]].append(i)

    def gemv_weights(k):
        return [w for i in by_op[k] if g.nodes[i]["op"] == "MUL_MAT" for w in _weights(g, g.nodes[i])]

    def named(k, short):
        for w in gemv_weights(k) + [w for i in by_op[k] for w in _weights(g, g.nodes[i])]:
            if _short(w) == short:
                return "gguf:" + w
        raise ValueError("op %s has no %s weight" % (ops[k], short))

    prog = []
    for k, (il, role) in enumerate(ops):
        pre = "blk.%d." % il if il is not None else ""
        gw = lambda s: "gguf:%s%s.weight" % (pre, s)   # noqa: E731
        kinds = {g.nodes[i]["mkind"] for i in by_op[k]}
        if role == P:
            ins = {"kind": "GEMV", "layer": il, "role": role, "norm_w": gw("attn_norm")}
            if "embed_lookup" in kinds:
                ins.update(pro="EMBED", aux="gguf:token_embd.weight", token="cell:token", x_out="buf:X")
            else:
                ins.update(pro="RMSNORM", x="buf:X")
            if "deltanet_step" in {g.nodes[i]["mkind"] for i in by_op[k + 1]}:
                ins["seg"] = [{"w": named(k, "attn_qkv"), "y": "buf:qkv", "epi": "CONV",
                               "aux": "state:conv.%d" % il, "w2": gw("ssm_conv1d")},
                              {"w": named(k, "attn_gate"), "y": "buf:z", "epi": "SILU"},
                              {"w": named(k, "ssm_alpha"), "y": "buf:alpha", "epi": "STORE"},
                              {"w": named(k, "ssm_beta"), "y": "buf:beta", "epi": "STORE"}]
            else:
                ins["seg"] = [{"w": named(k, "attn_q"), "y": "buf:qg", "epi": "STORE"},
                              {"w": named(k, "attn_k"), "y": "buf:k", "epi": "STORE"},
                              {"w": named(k, "attn_v"), "y": "buf:v", "epi": "STORE"}]
        elif role == S:
            ins = {"kind": "GDN_STEP", "layer": il, "role": role, "qkv": "buf:qkv", "alpha": "buf:alpha",
                   "beta": "buf:beta", "dt_bias": "gguf:%sssm_dt.bias" % pre, "ssm_a": "gguf:%sssm_a" % pre,
                   "state": "state:ssm.%d" % il, "o": "buf:o"}
        elif role == A:
            ins = {"kind": "ATTN_DECODE", "layer": il, "role": role, "qg": "buf:qg", "k": "buf:k", "v": "buf:v",
                   "q_norm": gw("attn_q_norm"), "k_norm": gw("attn_k_norm"), "kc": "state:cache_k.%d" % il,
                   "vc": "state:cache_v.%d" % il, "part": "buf:attn_part", "count": "buf:attn_count",
                   "out": "buf:att", "pass_cell": "cell:token"}
        elif role == O:
            if "gated_out_norm" in kinds:
                ins = {"kind": "GEMV", "layer": il, "role": role, "pro": "GATED_G", "x": "buf:o",
                       "norm_w": gw("ssm_norm"), "aux": "buf:z",
                       "seg": [{"w": named(k, "ssm_out"), "y": "buf:H", "epi": "RESID", "aux": "buf:X"}]}
            else:
                ins = {"kind": "GEMV", "layer": il, "role": role, "pro": "PLAIN", "x": "buf:att",
                       "seg": [{"w": named(k, "attn_output"), "y": "buf:H", "epi": "RESID", "aux": "buf:X"}]}
        elif role == G:
            ins = {"kind": "GEMV", "layer": il, "role": role, "pro": "RMSNORM", "x": "buf:H",
                   "norm_w": gw("post_attention_norm"),
                   "seg": [{"w": named(k, "ffn_gate"), "w2": named(k, "ffn_up"), "y": "buf:ffn", "epi": "SWIGLU"}]}
        elif role == D:
            ins = {"kind": "GEMV", "layer": il, "role": role, "pro": "PLAIN", "x": "buf:ffn",
                   "seg": [{"w": named(k, "ffn_down"), "y": "buf:X", "epi": "RESID", "aux": "buf:H"}]}
        else:
            ins = {"kind": "GEMV", "layer": None, "role": role, "pro": "RMSNORM", "x": "buf:X",
                   "norm_w": "gguf:output_norm.weight", "epi_ws": "buf:argmax_ws",
                   "seg": [{"w": named(k, "output"), "y": "buf:logits", "epi": "ARGMAX"}]}
        ins["nodes"] = len(by_op[k])
        prog.append(ins)
        if role != H:
            prog.append({"kind": "BOUNDARY"})
    return prog


# ------------------------------------------------------------------ packer

# gguf tensor name (without "blk.N.") -> the model's weight slot
_SLOT_COMMON = {"attn_norm.weight": 0, "post_attention_norm.weight": 1, "ffn_gate.weight": 2,
                "ffn_up.weight": 3, "ffn_down.weight": 4}
_SLOT_GDN = {"attn_qkv.weight": 5, "attn_gate.weight": 6, "ssm_alpha.weight": 7, "ssm_beta.weight": 8,
             "ssm_out.weight": 9, "ssm_conv1d.weight": 10, "ssm_dt.bias": 11, "ssm_a": 12, "ssm_norm.weight": 13}
_SLOT_ATTN = {"attn_q.weight": 5, "attn_k.weight": 6, "attn_v.weight": 7, "attn_output.weight": 8,
              "attn_q_norm.weight": 9, "attn_k_norm.weight": 10}
_SLOT_GLOBAL = {"token_embd.weight": 0, "output_norm.weight": 1, "output.weight": 2}


def program_layers(prog):
    return sorted({i["layer"] for i in prog if i.get("layer") is not None})


def truncate(prog, n_layer):
    """The program of the first n_layer layers and the head (a smaller model
    of the same layer pattern)."""
    out = []
    for ins in prog:
        if ins["kind"] != "BOUNDARY" and ins.get("layer") is not None and ins["layer"] >= n_layer:
            continue
        if ins["kind"] == "BOUNDARY" and out and out[-1]["kind"] == "BOUNDARY":
            continue
        out.append(ins)
    return out


def pack(model, prog):
    """Resolve a symbolic program against a sinter Model and pack it into
    sinter_instr records (the in-library packer, model.cpp build_program,
    writes the same bytes for the same model).  Shapes, types and scalars
    come from the model: the program only names operands."""
    import ctypes as C
    import math
    import numpy as np
    import sinter

    cfg, info = model.cfg, model.info()
    blocks = info["blocks"]
    L = sinter.lib()
    pc = L.sinter_host_pass_cell(model.host())
    attn_layers = {i["layer"] for i in prog if i["kind"] == "ATTN_DECODE"}

    def tensor(name):
        n = name.split(":", 1)[1]
        if n.startswith("blk."):
            il = int(n.split(".")[1])
            rest = n.split(".", 2)[2]
            slot = _SLOT_COMMON.get(rest, (_SLOT_ATTN if il in attn_layers else _SLOT_GDN).get(rest))
        else:
            il, slot = cfg.n_layer, _SLOT_GLOBAL.get(n)
        if slot is None:
            raise ValueError("unknown tensor " + name)
        return model.tensor(il, slot)

    def ptr(name):
        if name is None:
            return None
        ns, n = name.split(":", 1)
        if ns == "gguf":
            return tensor(name)[0]
        if ns == "buf":
            p, nb = C.c_void_p(), C.c_size_t()
            sinter.check(L.sinter_model_buffer(model.h, n.encode(), C.byref(p), C.byref(nb)), "buffer " + n)
            return p.value
        if ns == "state":
            role, il = n.split(".")
            return model.state(int(il), 0 if role in ("conv", "cache_k") else 1)[0]
        if ns == "cell" and n == "token":
            return pc
        raise ValueError("cannot resolve " + name)

    PRO = {"PLAIN": sinter.PRO_PLAIN, "RMSNORM": sinter.PRO_RMSNORM, "EMBED": sinter.PRO_EMBED,
           "GATED_G": sinter.PRO_GATED_G}
    EPI = {"STORE": sinter.EPI_STORE, "RESID": sinter.EPI_RESID, "SWIGLU": sinter.EPI_SWIGLU,
           "ARGMAX": sinter.EPI_ARGMAX, "CONV": sinter.EPI_CONV, "SILU": sinter.EPI_SILU}
    ROLE_DBG = {P: 0, S: 1, A: 1, O: 2, G: 3, D: 4}
    K_OF = {P: cfg.n_embd, G: cfg.n_embd, H: cfg.n_embd, D: cfg.n_ff}
    log2d = int(math.log2(cfg.gdn_d))
    out = (sinter.Instr * len(prog))()
    for k, ins in enumerate(prog):
        o = out[k]
        o.block_lo, o.block_hi = 0, blocks
        if ins["kind"] == "BOUNDARY":
            o.kind = sinter.OP_BOUNDARY
            continue
        il = ins["layer"]
        o.dbg_node = cfg.n_layer * 8 if il is None else il * 8 + ROLE_DBG[ins["role"]]
        if ins["kind"] == "GEMV":
            o.kind = sinter.OP_GEMV
            a = sinter.GemvArgs()
            a.eps = cfg.eps
            a.pro = PRO[ins["pro"]]
            a.x, a.norm_w = ptr(ins.get("x")), ptr(ins.get("norm_w"))
            if ins["role"] == O:
                a.K = cfg.attn_nq * cfg.head_dim if il in attn_layers else cfg.gdn_hv * cfg.gdn_d
            else:
                a.K = K_OF[ins["role"]]
            if ins["pro"] == "EMBED":
                ep, nb, et = tensor(ins["aux"])
                a.aux, a.aux_type, a.aux_rows = ep, et, nb // sinter.row_bytes(et, a.K)
                a.token, a.x_out = ptr(ins["token"]), ptr(ins["x_out"])
            elif ins["pro"] == "GATED_G":
                a.aux, a.gn_log2d = ptr(ins["aux"]), log2d
            a.epi_ws = ptr(ins.get("epi_ws"))
            a.n_seg = len(ins["seg"])
            for j, sg in enumerate(ins["seg"]):
                wp, nb, wt = tensor(sg["w"])
                seg = a.seg[j]
                seg.w, seg.y, seg.aux = wp, ptr(sg["y"]), ptr(sg.get("aux"))
                seg.w2 = ptr(sg.get("w2"))
                seg.rows = nb // sinter.row_bytes(wt, a.K)
                seg.type, seg.epi = wt, EPI[sg["epi"]]
                seg.dconv = cfg.conv_k if sg["epi"] == "CONV" else 0
        elif ins["kind"] == "GDN_STEP":
            o.kind = sinter.OP_GDN_STEP
            a = sinter.GdnArgs()
            for f in ("qkv", "alpha", "beta", "dt_bias", "ssm_a", "state", "o"):
                setattr(a, f, ptr(ins[f]))
            a.hk, a.hv, a.d = cfg.gdn_hk, cfg.gdn_hv, cfg.gdn_d
            a.cols = 32 if cfg.gdn_d >= 128 else 16
            a.eps = cfg.eps
            a.scale = float(np.float32(1.0) / np.sqrt(np.float32(cfg.gdn_d)))
        else:
            o.kind = sinter.OP_ATTN_DECODE
            a = sinter.AttnArgs()
            for f in ("qg", "k", "v", "q_norm", "k_norm", "kc", "vc", "part", "count", "out", "pass_cell"):
                setattr(a, f, ptr(ins[f]))
            a.nq, a.nkv, a.hd, a.rope_dims, a.n_ctx = cfg.attn_nq, cfg.attn_nkv, cfg.head_dim, cfg.rope_dims, cfg.n_ctx
            # the split-K geometry the model resolved (its config), else the
            # library default for this grid
            a.n_chunks = cfg.attn_chunks or min(64, max(1, blocks // cfg.attn_nkv))
            a.chunk_min = cfg.attn_chunk_min or sinter.ATTN_CHUNK_MIN
            a.theta_scale = float(np.float32(math.pow(float(np.float32(cfg.rope_base)), -2.0 / cfg.rope_dims)))
            a.eps = cfg.eps
            a.scale = float(np.float32(1.0) / np.sqrt(np.float32(cfg.head_dim)))
            a.kv_type = cfg.t_kv or sinter.F16
        C.memmove(o.payload, C.byref(a), C.sizeof(a))
    return out


def compile_graph(schedule_csv, leaves_csv):
    """Everything the compiler reports for one graph (JSON-serialisable)."""
    g = load(schedule_csv, leaves_csv)
    prog = symbolic_program(g)
    return {"coverage": accounting(g), "dram_bytes": dram(g),
            "program": {"ops": sum(1 for i in prog if i["kind"] != "BOUNDARY"),
                        "boundaries_per_pass": sum(1 for i in prog if i["kind"] == "BOUNDARY") + 1,
                        "instructions": prog}}


if __name__ == "__main__":
    import sys
    out = compile_graph(sys.argv[1], sys.argv[2])
    json.dump(out, sys.stdout, indent=1)
