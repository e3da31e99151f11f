"""The ggml backend shim's decisions (ggml_backend/graph_rules.cpp), on the CPU.

The graph description is built from the reference's own captured decode graph
(tests/golden/k0_schedule.csv nodes and k0_leaves.csv leaves: a batch-1 decode
of the 64-layer Qwen3.6 hybrid, 48 gated-DeltaNet + 16 attention layers),
named the way llama.cpp names the tensors the shim looks up (inp_tokens,
inp_pos with the 4 M-RoPE ids of a token, cache_k_l<i> / cache_v_l<i>,
cache_r_l<i> / cache_s_l<i>, k_idxs, result_output, GDN nodes with the
__fgdn_ar__ decode suffix: docs/INTEGRATION-FINDINGS.md:182-236,
docs/PREFILL-SEMANTICS.md:344-377).  Each rule is checked by a hit and by the
miss that one change to the description causes.
"""
import copy
import csv
import ctypes as C
import os
import struct

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
RULES = os.path.join(ROOT, "sinter-qwen36-nomtp-tu102_amd", "ggml_backend", "libsinter_ggml_rules.so")

F32, F16, Q8_0, Q4_K, Q6_K, BF16 = 0, 1, 8, 12, 14, 30
G_OTHER, G_RMS_NORM, G_ROPE, G_GDN, G_FATTN = 0, 1, 2, 3, 4


class RT(C.Structure):
    _fields_ = [("name", C.c_char_p), ("op", C.c_int32), ("type", C.c_int32), ("ne", C.c_int64 * 4),
                ("data", C.c_uint64), ("root", C.c_int32), ("src0", C.c_int32), ("op_params", C.c_int32 * 16)]


class Cfg(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("n_layer", "attn_every", "n_embd", "n_ff", "n_vocab", "gdn_hk", "gdn_hv",
                                         "gdn_d", "conv_k", "attn_nq", "attn_nkv", "head_dim", "rope_dims")] + \
               [("rope_base", C.c_float), ("eps", C.c_float), ("n_ctx", C.c_int32)] + \
               [(n, C.c_int32) for n in ("t_default", "t_attn_v", "t_ffn_down", "t_output", "t_embd", "t_kv",
                                         "attn_chunks", "attn_chunk_min")]


@pytest.fixture(scope="module")
def rules():
    if not os.path.exists(RULES):
        import sys
        sys.path.insert(0, os.path.join(ROOT, "sinter-qwen36-nomtp-tu102_amd"))
        import build
        build.build_ggml_rules()
    L = C.CDLL(RULES)
    L.sinter_rules_classify.argtypes = [C.POINTER(RT), C.c_int, C.c_char_p, C.c_int]
    L.sinter_rules_bind.argtypes = [C.POINTER(RT), C.c_int, C.POINTER(Cfg), C.POINTER(C.c_uint64),
                                    C.POINTER(C.c_int32), C.c_int, C.POINTER(C.c_uint64), C.c_int,
                                    C.POINTER(C.c_uint64), C.POINTER(C.c_int), C.c_char_p, C.c_int]
    L.sinter_rules_same_binding.argtypes = [C.POINTER(RT), C.c_int, C.POINTER(RT), C.c_int]
    L.sinter_rules_pass_inputs.argtypes = [C.POINTER(C.c_int32), C.c_int, C.c_int, C.c_int64,
                                           C.POINTER(C.c_int32), C.c_char_p, C.c_int]
    return L


def _ne(s):
    return [int(v) for v in s.split("x")]


def _leaf_name(cls):
    if cls.startswith("weight:"):
        return cls[len("weight:"):]
    if cls == "input_tokens":
        return "inp_tokens"
    if cls == "positions":
        return "inp_pos"
    if cls == "mask":
        return "kq_mask"
    for pre, new in (("cache_k(blk.", "cache_k_l"), ("cache_v(blk.", "cache_v_l"),
                     ("state:conv_state(blk.", "cache_r_l"), ("state:ssm_state(blk.", "cache_s_l")):
        if cls.startswith(pre):
            return new + cls[len(pre):-1]
    return cls.split(":", 1)[1] if ":" in cls else cls


def _params(op, text):
    p = [0] * 16
    kv = dict(t.split("=", 1) for t in text.split() if "=" in t)
    if op == G_RMS_NORM:
        p[0] = struct.unpack("<i", struct.pack("<f", float(kv["eps"])))[0]
    elif op == G_ROPE:
        p[1] = int(kv["n_dims"])
        p[2] = int(kv["mode"].split("(")[1].rstrip(")"))
        p[5] = struct.unpack("<i", struct.pack("<f", float(kv["freq_base"])))[0]
    return p


TYPES = {"f32": F32, "f16": F16, "q4_0": -1, "q4_0_ar16": -1, "i32": -1, "i64": -1}


def captured_graph():
    """[dict] tensors of the reference's captured decode graph: leaves, then nodes"""
    leaves, nodes = [], []
    with open(os.path.join(HERE, "golden", "k0_leaves.csv")) as f:
        for r in csv.DictReader(f):
            leaves.append(r)
    with open(os.path.join(HERE, "golden", "k0_schedule.csv")) as f:
        for r in csv.DictReader(f):
            nodes.append(r)
    nl = len(leaves)
    out = []
    for r in leaves:
        i = int(r["leaf_idx"])
        out.append(dict(name=_leaf_name(r["classification"]), op=G_OTHER, type=TYPES[r["type"]], ne=_ne(r["ne"]),
                        data=0x7f0000000000 + 0x100000 * i, root=-1, src0=-1, params=[0] * 16, wtype=r["type"]))
    vocab = max(_ne(r["ne"])[0] for r in nodes if r["op"] == "MUL_MAT")
    for r in nodes:
        i = int(r["node_idx"])
        op = {"RMS_NORM": G_RMS_NORM, "ROPE": G_ROPE, "GATED_DELTA_NET": G_GDN,
              "FLASH_ATTN_EXT": G_FATTN}.get(r["op"], G_OTHER)
        ne = _ne(r["ne"])
        name = ""
        if op == G_GDN:
            name = "__fgdn_ar__-%s" % r["block_idx"]
        elif r["op"] == "MUL_MAT" and ne[0] == vocab and r["block_idx"] == "post":
            name = "result_output"
        refs = [s for s in r["src_refs"].split(";") if s]
        src0 = -1
        if refs:
            src0 = int(refs[0][1:]) + (nl if refs[0][0] == "n" else 0)
        out.append(dict(name=name, op=op, type=TYPES.get(r["type"], -1), ne=ne, data=0x7e0000000000 + 0x1000 * i,
                        root=-1, src0=src0, params=_params(op, r["decoded_params"]), wtype=r["type"]))
    return out


def q4km(desc):
    """The same graph over a Q4_K_M-style model (Q6_K for attn_v, ffn_down and
    the head, Q4_K elsewhere; the f16 embedding as Q4_K)"""
    d = copy.deepcopy(desc)
    for t in d:
        if t["op"] == G_OTHER and t["name"].endswith(".weight") and t["wtype"] in ("q4_0", "q4_0_ar16", "f16") \
                and "cache" not in t["name"]:
            heavy = t["name"].endswith(("attn_v.weight", "ffn_down.weight")) or t["name"] == "output.weight"
            t["type"] = Q6_K if heavy else Q4_K
    return d


def arr(desc):
    a = (RT * len(desc))()
    keep = []
    for i, t in enumerate(desc):
        nm = t["name"].encode()
        keep.append(nm)
        a[i].name = nm
        a[i].op, a[i].type = t["op"], t["type"]
        for k in range(4):
            a[i].ne[k] = t["ne"][k]
        a[i].data, a[i].root, a[i].src0 = t["data"], t["root"], t["src0"]
        for k in range(16):
            a[i].op_params[k] = t["params"][k]
    return a, keep


def classify(L, desc):
    a, keep = arr(desc)
    why = C.create_string_buffer(256)
    return L.sinter_rules_classify(a, len(desc), why, 256), why.value.decode()


def bind(L, desc):
    a, keep = arr(desc)
    cfg = Cfg()
    nt, ns = 64 * 16 + 3, 128
    tens, types, states = (C.c_uint64 * nt)(), (C.c_int32 * nt)(), (C.c_uint64 * ns)()
    logits, eo = C.c_uint64(), C.c_int()
    why = C.create_string_buffer(256)
    ok = L.sinter_rules_bind(a, len(desc), C.byref(cfg), tens, types, nt, states, ns, C.byref(logits), C.byref(eo),
                             why, 256)
    return ok, why.value.decode(), cfg, list(tens), list(types), list(states), logits.value, eo.value


def find(desc, name):
    return next(i for i, t in enumerate(desc) if t["name"] == name)


def test_captured_decode_graph_is_a_decode_hit(rules):
    d = captured_graph()
    assert classify(rules, d) == (1, "")


def test_captured_q4_0_model_does_not_bind(rules):
    """The reference's own model is Q4_0: a decode graph, but weights the
    kernels do not read -- delegated, with the tensor named."""
    ok, why, *_ = bind(rules, captured_graph())
    assert ok == 0 and "a type the kernels do not read" in why


def test_q4km_graph_binds_to_the_model_shape(rules):
    d = q4km(captured_graph())
    ok, why, cfg, tens, types, states, logits, eo = bind(rules, d)
    assert ok == 1, why
    assert (cfg.n_layer, cfg.attn_every, cfg.n_embd, cfg.n_ff, cfg.n_vocab) == (64, 4, 5120, 17408, 248320)
    assert (cfg.gdn_hk, cfg.gdn_hv, cfg.gdn_d, cfg.conv_k) == (16, 48, 128, 4)
    assert (cfg.attn_nq, cfg.attn_nkv, cfg.head_dim, cfg.rope_dims) == (24, 4, 256, 64)
    assert cfg.rope_base == 1e7 and cfg.eps == struct.unpack("<f", struct.pack("<f", 1e-6))[0]
    assert cfg.n_ctx == 262144 and cfg.t_kv == F16
    # the config's types are the tensors' own (not the qkv type for all)
    assert (cfg.t_default, cfg.t_attn_v, cfg.t_ffn_down, cfg.t_output, cfg.t_embd) == (Q4_K, Q6_K, Q6_K, Q6_K, Q4_K)
    # bindings point at the graph's own tensors, in sinter_model_tensor_info order
    assert tens[3 * 16 + 5 + 2] == d[find(d, "blk.3.attn_v.weight")]["data"] and types[3 * 16 + 5 + 2] == Q6_K
    assert tens[0 * 16 + 5 + 0] == d[find(d, "blk.0.attn_qkv.weight")]["data"]
    assert tens[64 * 16 + 0] == d[find(d, "token_embd.weight")]["data"]
    assert tens[64 * 16 + 2] == d[find(d, "output.weight")]["data"]
    assert states[2 * 3] == d[find(d, "cache_k_l3")]["data"] and states[2 * 3 + 1] == d[find(d, "cache_v_l3")]["data"]
    assert states[0] == d[find(d, "cache_r_l0")]["data"] and states[1] == d[find(d, "cache_s_l0")]["data"]
    assert logits == d[find(d, "result_output")]["data"] and eo == 0


@pytest.mark.parametrize("change,expect", [
    ("chunked_gdn", "prefill (chunked GDN node)"),
    ("gdn_no_suffix", "GDN node without the decode suffix"),
    ("gdn_tokens", "GDN over more than one token"),
    ("fa_batch", "attention over more than one query"),
    ("two_logit_rows", "no single-row result_output"),
    ("no_logits", "no single-row result_output"),
    ("two_positions", "no single token position"),
    ("rope_mode", "rope mode neither NEOX nor IMROPE"),
    ("no_input", "neither token ids nor an embedded row as input"),
])
def test_classify_misses(rules, change, expect):
    d = captured_graph()
    gdn = [i for i, t in enumerate(d) if t["op"] == G_GDN]
    fa = [i for i, t in enumerate(d) if t["op"] == G_FATTN]
    if change == "chunked_gdn":
        d[gdn[5]]["name"] = "__fgdn_ch__-5"
    elif change == "gdn_no_suffix":
        d[gdn[0]]["name"] = "gdn-0"
    elif change == "gdn_tokens":        # a prefill ubatch: ne[2] of q is its token count
        d[d[gdn[7]]["src0"]]["ne"][2] = 8
    elif change == "fa_batch":          # batch > 1: q carries more than one query
        d[d[fa[2]]["src0"]]["ne"][1] = 4
    elif change == "two_logit_rows":
        d[find(d, "result_output")]["ne"][1] = 2
    elif change == "no_logits":
        d[find(d, "result_output")]["name"] = "logits"
    elif change == "two_positions":
        d[find(d, "inp_pos")]["ne"][0] = 8
    elif change == "rope_mode":
        next(t for t in d if t["op"] == G_ROPE)["params"][2] = 0
    elif change == "no_input":
        d[find(d, "inp_tokens")]["name"] = "tokens"
    assert classify(rules, d) == (0, expect)


@pytest.mark.parametrize("change,expect", [
    ("no_eps", "no RMS_NORM to read eps from"),
    ("two_eps", "RMS norms with different eps"),
    ("no_rope", "no ROPE to read the rotated dims and base from"),
    ("pattern", "layer pattern is not every 4"),
    ("kv_type", "KV cache neither f16 nor q8_0"),
    ("f16_matrix", "blk.9.ffn_gate.weight: a type the kernels do not read"),
    ("missing", "missing blk.12.ssm_out.weight"),
    ("small_state", "recurrent state of layer 5 not f32 or too small"),
])
def test_bind_refusals(rules, change, expect):
    d = q4km(captured_graph())
    if change == "no_eps":
        for t in d:
            if t["op"] == G_RMS_NORM:
                t["op"] = G_OTHER
    elif change == "two_eps":
        [t for t in d if t["op"] == G_RMS_NORM][3]["params"][0] = struct.unpack("<i", struct.pack("<f", 1e-5))[0]
    elif change == "no_rope":
        for t in d:
            if t["op"] == G_ROPE:
                t["op"] = G_OTHER
    elif change == "pattern":
        d[find(d, "blk.7.attn_q.weight")]["name"] = "blk.7.attn_q_other.weight"
    elif change == "kv_type":
        d[find(d, "cache_k_l3")]["type"] = F32
    elif change == "f16_matrix":
        d[find(d, "blk.9.ffn_gate.weight")]["type"] = F16
    elif change == "missing":
        d[find(d, "blk.12.ssm_out.weight")]["name"] = "blk.12.ssm_out_x.weight"
    elif change == "small_state":
        d[find(d, "cache_s_l5")]["ne"][0] = 1000
    ok, why, *_ = bind(rules, d)
    assert (ok, why) == (0, expect)


def test_tied_head_and_embedded_input(rules):
    d = q4km(captured_graph())
    d[find(d, "output.weight")]["name"] = "output_unused"        # no output.weight: the head is the embedding
    ok, why, cfg, tens, types, states, logits, eo = bind(rules, d)
    assert ok == 1, why
    assert tens[64 * 16 + 2] == d[find(d, "token_embd.weight")]["data"] and cfg.t_output == Q4_K
    d[find(d, "inp_tokens")]["name"] = "inp_embd"                # the caller embeds the token
    ok, why, cfg, tens, types, states, logits, eo = bind(rules, d)
    assert ok == 1 and eo == 1 and tens[64 * 16 + 0] == 0


def test_mixed_type_layers_bind_per_tensor(rules):
    """Q4_K_M files mix Q4_K and Q6_K in one kind of tensor across layers: each
    binding carries its own tensor's type."""
    d = q4km(captured_graph())
    d[find(d, "blk.10.ffn_down.weight")]["type"] = Q4_K
    ok, why, cfg, tens, types, *_ = bind(rules, d)
    assert ok == 1 and types[10 * 16 + 4] == Q4_K and types[11 * 16 + 4] == Q6_K and cfg.t_ffn_down == Q6_K


@pytest.mark.parametrize("what", ["weight", "state", "logits", "type"])
def test_rebinding_is_keyed_on_every_binding(rules, what):
    """A bound model is rebuilt when any bound pointer or type moves, not
    only the logits buffer."""
    a = q4km(captured_graph())
    b = copy.deepcopy(a)
    aa, ka = arr(a)
    ab, kb = arr(b)
    assert rules.sinter_rules_same_binding(aa, len(a), ab, len(b)) == 1
    if what == "weight":
        b[find(b, "blk.5.ffn_down.weight")]["data"] += 0x10000
    elif what == "state":
        b[find(b, "cache_s_l9")]["data"] += 0x10000
    elif what == "logits":
        b[find(b, "result_output")]["data"] += 0x10000
    else:
        b[find(b, "blk.2.ffn_up.weight")]["type"] = Q6_K
    ab, kb = arr(b)
    assert rules.sinter_rules_same_binding(aa, len(a), ab, len(b)) == 0


@pytest.mark.parametrize("ids,row,ok,why", [
    ([4100], 4100, 1, ""), ([4100] * 4, 4100, 1, ""), ([4100] * 4, None, 1, ""),
    ([4100, 4100, 4100, 7], 4100, 0, "M-RoPE position ids differ (not a text token)"),
    ([4100] * 4, 4099, 0, "KV row is not the position"),
    ([4100, 4100], 4100, 0, "no single token position"),
])
def test_pass_inputs(rules, ids, row, ok, why):
    a = (C.c_int32 * len(ids))(*ids)
    pos = C.c_int32()
    w = C.create_string_buffer(128)
    got = rules.sinter_rules_pass_inputs(a, len(ids), row is not None, row if row is not None else -1, C.byref(pos),
                                         w, 128)
    assert (got, w.value.decode()) == (ok, why)
    if ok:
        assert pos.value == ids[0]
