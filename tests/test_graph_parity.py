"""The oracle's decode pass against the reference's captured decode graph.

tests/graph_exec.py evaluates the nodes of k0/schedule.csv -- the prologue,
blocks 0-3 (three gated-DeltaNet blocks and the first attention block) and
the epilogue spliced onto block 3 -- with the leaves bound to one set of
synthetic weights, states and KV caches at the reference model's own layer
shapes (hidden 5120, FFN 17408, 16 k-heads / 48 v-heads of 128, 24 q-heads /
4 kv-heads of 256; a 1024-row vocabulary instead of 248320).  The oracle's
or_decode_step runs a 4-layer model with the same bytes.  Both use the same
pinned arithmetic primitives, so the logits, every block's residual output,
the updated conv/recurrent states and the appended KV rows must be
bit-identical; any difference in how the oracle composes the pass (norm and
residual placement, the q|gate interleave, the qkv split, the gates path, the
conv window shift, the output gate, the KV row) shows up as a mismatch.
"""
import ctypes as C

import numpy as np
import pytest

from graph_exec import GraphExec, QWeight, T, load_graph

E, F, HK, HV, D, DCONV = 5120, 17408, 16, 48, 128, 4
NQ, NKV, HD, VOCAB, NCTX = 24, 4, 256, 1024, 33024
CH = (2 * HK + HV) * D

# GGUF tensor name suffix -> oracle weight slot (oracle/oracle.h)
DN_SLOTS = {"attn_norm.weight": 0, "post_attention_norm.weight": 1, "ffn_gate.weight": 2, "ffn_up.weight": 3,
            "ffn_down.weight": 4, "attn_qkv.weight": 5, "attn_gate.weight": 6, "ssm_alpha.weight": 7,
            "ssm_beta.weight": 8, "ssm_out.weight": 9, "ssm_conv1d.weight": 10, "ssm_dt.bias": 11, "ssm_a": 12,
            "ssm_norm.weight": 13}
AT_SLOTS = {"attn_norm.weight": 0, "post_attention_norm.weight": 1, "ffn_gate.weight": 2, "ffn_up.weight": 3,
            "ffn_down.weight": 4, "attn_q.weight": 5, "attn_k.weight": 6, "attn_v.weight": 7,
            "attn_output.weight": 8, "attn_q_norm.weight": 9, "attn_k_norm.weight": 10}


@pytest.fixture(scope="module")
def graph():
    return load_graph()


def synth(sn, kind, type_, rows, k, seed, a=0.0, b=0.0):
    if kind == sn.SYN_WEIGHT:
        out = np.zeros(sn.row_bytes(type_, k) * rows, np.uint8)
    elif kind == sn.SYN_NORMAL_F16:
        out = np.zeros(rows * k, np.uint16)
    else:
        out = np.zeros(rows * k, np.float32)
    sn.check(sn.lib().sinter_synth(0, out.ctypes.data, kind, type_, rows, k, seed, a, b, None), "synth")
    return out


def test_captured_graph_matches_oracle_decode(sn, orc, graph):
    nodes, leaves = graph
    L = orc.lib()
    cfg = orc.Cfg(n_layer=4, attn_every=4, n_embd=E, n_ff=F, n_vocab=VOCAB, gdn_hk=HK, gdn_hv=HV, gdn_d=D,
                  conv_k=DCONV, attn_nq=NQ, attn_nkv=NKV, head_dim=HD, rope_dims=64, rope_base=1e7, eps=1e-6,
                  n_ctx=NCTX, t_default=orc.Q4_K, t_attn_v=orc.Q6_K, t_ffn_down=orc.Q6_K, t_output=orc.Q6_K,
                  t_embd=orc.Q4_K, attn_chunks=64, attn_chunk_min=128)
    W, Y = sn.SYN_WEIGHT, sn.SYN_NORMAL
    seed = 777
    w = {}   # (layer, slot) -> (type, array, k, rows)
    for il in range(4):
        at = il == 3
        def wt(slot, t, rows, k):
            w[(il, slot)] = (t, synth(sn, W, t, rows, k, seed + 100 * il + slot), k, rows)
        def vec(slot, n, kind, a, b):
            w[(il, slot)] = (orc.F32, synth(sn, kind, orc.F32, 1, n, seed + 100 * il + slot, a, b), n, 1)
        vec(0, E, Y, 1.0, 0.02)
        vec(1, E, Y, 1.0, 0.02)
        wt(2, orc.Q4_K, F, E)
        wt(3, orc.Q4_K, F, E)
        wt(4, orc.Q6_K, E, F)
        if at:
            wt(5, orc.Q4_K, NQ * 2 * HD, E)
            wt(6, orc.Q4_K, NKV * HD, E)
            wt(7, orc.Q6_K, NKV * HD, E)
            wt(8, orc.Q4_K, E, NQ * HD)
            vec(9, HD, Y, 1.0, 0.02)
            vec(10, HD, Y, 1.0, 0.02)
        else:
            wt(5, orc.Q4_K, CH, E)
            wt(6, orc.Q4_K, HV * D, E)
            wt(7, orc.Q4_K, HV, E)
            wt(8, orc.Q4_K, HV, E)
            wt(9, orc.Q4_K, E, HV * D)
            vec(10, CH * DCONV, sn.SYN_UNIFORM, -0.5, 0.5)
            vec(11, HV, sn.SYN_UNIFORM, -6.9, -2.3)
            vec(12, HV, sn.SYN_UNIFORM, -16.0, -1.0)
            vec(13, D, Y, 1.0, 0.02)
    embd = synth(sn, W, orc.Q4_K, VOCAB, E, seed + 1)
    onorm = synth(sn, Y, orc.F32, 1, E, seed + 2, 1.0, 0.02)
    outw = synth(sn, W, orc.Q6_K, VOCAB, E, seed + 3)
    pos, token = 2047, 613
    st0 = {}
    for il in range(3):
        st0[(il, 0)] = synth(sn, Y, orc.F32, 1, CH * (DCONV - 1), seed + 500 + il, 0.0, 1.0)
        st0[(il, 1)] = synth(sn, Y, orc.F32, 1, HV * D * D, seed + 600 + il, 0.0, 0.1)
    for s in range(2):
        c = np.zeros(NCTX * NKV * HD, np.uint16)
        c[:pos * NKV * HD] = synth(sn, sn.SYN_NORMAL_F16, orc.F16, 1, pos * NKV * HD, seed + 700 + s, 0.0, 1.0)
        st0[(3, s)] = c

    # ---------------------------------------------------------- the oracle
    wp = (C.c_void_p * (4 * 16 + 3))()
    for (il, slot), (_, a, _, _) in w.items():
        wp[il * 16 + slot] = a.ctypes.data
    wp[64], wp[65], wp[66] = embd.ctypes.data, onorm.ctypes.data, outw.ctypes.data
    ost = {k: v.copy() for k, v in st0.items()}
    sp = (C.c_void_p * 8)()
    for (il, s), a in ost.items():
        sp[il * 2 + s] = a.ctypes.data
    logits = np.zeros(VOCAB, np.float32)
    resid = np.zeros(4 * E, np.float32)
    otok = L.or_decode_step(C.byref(cfg), wp, sp, token, pos, logits.ctypes.data, resid.ctypes.data)

    # ---------------------------------------------------------- the captured graph
    est = {k: v.copy() for k, v in st0.items()}
    bind = {}
    for li, lf in leaves.items():
        cls = lf["cls"]
        if cls.startswith("weight:blk."):
            blk, name = cls[len("weight:blk."):].split(".", 1)
            il = int(blk)
            if il > 3:
                continue
            slot = (AT_SLOTS if il == 3 else DN_SLOTS)[name]
            t, a, k, rows = w[(il, slot)]
            bind[li] = QWeight(t, a, k, rows) if t != orc.F32 else T(a, lf["ne"])
        elif cls.startswith("state:"):
            il = int(cls.split("blk.")[1].rstrip(")"))
            if il <= 3:
                bind[li] = T(est[(il, 0 if cls.startswith("state:conv") else 1)], lf["ne"])
        elif cls.startswith("cache_"):
            il = int(cls.split("blk.")[1].rstrip(")"))
            if il <= 3:
                bind[li] = T(est[(il, 0 if cls.startswith("cache_k") else 1)].view(np.float16), [NKV * HD, NCTX])
        elif cls == "weight:token_embd.weight":
            bind[li] = QWeight(orc.Q4_K, embd, E, VOCAB)
        elif cls == "weight:output_norm.weight":
            bind[li] = T(onorm, [E])
        elif cls == "weight:output.weight":
            bind[li] = QWeight(orc.Q6_K, outw, E, VOCAB)
        elif cls == "input_tokens":
            bind[li] = T(np.array([token], np.int32), [1])
        elif cls == "positions":
            bind[li] = T(np.array([pos] * 4, np.int32), [4])
        elif cls in ("other:k_idxs", "other:v_idxs"):
            bind[li] = T(np.array([pos], np.int64), [1])
        elif cls in ("other:rs_main_index", "other:out_row_index", "other:rs_copy_indices_buf"):
            bind[li] = T(np.array([0], np.int32), [1])
        elif cls == "other:rs_clear_index":
            bind[li] = T(np.zeros(0, np.int32), [0])
        elif cls == "mask":
            if lf["type"] == "f32":
                m = np.full(lf["ne"][0], -np.inf, np.float32)
                m[:pos + 1] = 0.0
                bind[li] = T(m, lf["ne"])
            else:
                bind[li] = T(np.zeros(lf["ne"][0], np.float16), lf["ne"])
    # l2 is the embedding row re-entering the graph as the trunk root
    trunk_root = [li for li, lf in leaves.items() if lf["cls"] == "other:embd_trunk_input"]
    blocks = {b: sorted(i for i, n in nodes.items() if n["block"] == b) for b in ("pre", "0", "1", "2", "3", "post")}
    last3 = blocks["3"][-1]
    post_src = [r for r in nodes[blocks["post"][0]]["src"] if r.startswith("n")][0]
    ex = GraphExec(nodes, leaves, orc, bind, alias={"l%d" % trunk_root[0]: "n0", post_src: "n%d" % last3},
                   attn_split=(cfg.attn_chunks, cfg.attn_chunk_min))
    order = sorted(blocks["pre"] + blocks["0"] + blocks["1"] + blocks["2"] + blocks["3"]) + blocks["post"]
    vals = ex.run(order)

    glog = vals[blocks["post"][-1]].flat()
    assert glog.shape == logits.shape
    for b in range(4):
        tail = vals[blocks[str(b)][-1]].flat()
        assert nodes[blocks[str(b)][-1]]["op"] == "ADD"
        np.testing.assert_array_equal(tail, resid[b * E:(b + 1) * E], err_msg=f"block {b} residual output")
    np.testing.assert_array_equal(glog, logits)
    assert int(np.argmax(glog)) == otok
    for k in st0:
        np.testing.assert_array_equal(est[k], ost[k], err_msg=f"state/cache {k}")
    # the step changed every state it owns, and exactly one KV row per cache
    for il in range(3):
        assert not np.array_equal(est[(il, 0)], st0[(il, 0)]) and not np.array_equal(est[(il, 1)], st0[(il, 1)])
    for s in range(2):
        changed = np.nonzero((est[(3, s)] != st0[(3, s)]).reshape(NCTX, NKV * HD).any(1))[0]
        assert list(changed) == [pos]
