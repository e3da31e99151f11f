"""This build's schedule compiler (sinter-qwen36-nomtp-tu102_amd/schedule.py) on
the reference's captured decode graph (tests/golden/k0_schedule.csv,
k0_leaves.csv), on the CPU.

Pinned against the reference's compiled program header
(tests/golden/k0_program_meta.json, from k0/program.json): the node
accounting (3704 nodes = 3221 executed + 483 dropped, by the same four
categories: 2 dead index views, 240 + 240 zero-extent state clear-chain
nodes, 1 host-side mask conversion) and the per-pass DRAM formula
16695695360 + 65568 * n_kv.  The fused program must give every executed node
exactly one op, never read a later op's result, and have 5 ops per layer
plus the head: 321 barriers per pass.
"""
import json
import os

import pytest

import schedule

HERE = os.path.dirname(os.path.abspath(__file__))
SCHED = os.path.join(HERE, "golden", "k0_schedule.csv")
LEAVES = os.path.join(HERE, "golden", "k0_leaves.csv")
META = json.load(open(os.path.join(HERE, "golden", "k0_program_meta.json")))


@pytest.fixture(scope="module")
def g():
    return schedule.load(SCHED, LEAVES)


def test_node_accounting_matches_the_reference_program(g):
    acc = schedule.accounting(g)
    cov = META["coverage"]
    assert (acc["nodes"], acc["emitted_nodes"], acc["dropped_nodes"]) == \
        (cov["nodes"], cov["emitted_nodes"], cov["dropped_nodes"]) == (3704, 3221, 483)
    # the same categories and counts as program.json's "drops"
    ref = sorted(d["count"] for d in META["drops"])
    assert sorted(acc["drops"].values()) == ref == [1, 2, 240, 240]
    assert acc["drops"] == {"dead_index_views": 2, "zero_extent_conv_state_chain": 240,
                            "zero_extent_ssm_state_chain": 240, "host_mask_conversion": 1}


def test_dram_formula_matches_the_reference_program(g):
    d = schedule.dram(g)
    ref = META["per_pass"]["dram_bytes"]
    assert d["formula"] == ref["formula"] == "16695695360 + 65568 * n_kv"
    for n_kv in (33024, 262144):
        assert d["fixed"] + d["per_n_kv"] * n_kv == ref["at_n_kv_%d" % n_kv]
    assert (d["state_rw"], d["kv_append_write"], d["logits_rw"]) == \
        (ref["state_rw"], ref["kv_append_write"], ref["logits_rw"])
    # program.json's weight_stream counts the one embedding row with the weights
    assert d["weight_stream"] + d["embd_row"] == ref["weight_stream"]
    # this build writes the logits once
    assert schedule.dram(g, logits_copies=1)["fixed"] == d["fixed"] - 2 * 248320 * 4


def test_fused_program_covers_every_node_once_in_dependency_order(g):
    ops, owner = schedule.fuse(g)          # raises on an uncovered node or a backward edge
    live = schedule.live_nodes(g)
    assert sorted(owner) == live and len(live) == 3221
    assert len(ops) == 64 * 5 + 1
    kinds = [r for _, r in ops[:-1]]
    for il in range(64):
        want = ["proj", "attn" if il % 4 == 3 else "step", "out", "ffn_gate_up", "ffn_down"]
        assert kinds[5 * il:5 * il + 5] == want, il
    # each op is fed only by itself and earlier ops; every op owns nodes
    assert set(owner.values()) == set(range(len(ops)))


def test_symbolic_program_operands(g):
    prog = schedule.symbolic_program(g)
    assert sum(i["kind"] == "BOUNDARY" for i in prog) + 1 == 321        # + the pass end
    assert sum(i["kind"] == "GEMV" for i in prog) == 64 * 4 + 1
    assert sum(i["kind"] == "GDN_STEP" for i in prog) == 48 and sum(i["kind"] == "ATTN_DECODE" for i in prog) == 16
    first = prog[0]
    assert first["pro"] == "EMBED" and first["aux"] == "gguf:token_embd.weight"
    assert [s["w"] for s in first["seg"]] == ["gguf:blk.0.attn_qkv.weight", "gguf:blk.0.attn_gate.weight",
                                             "gguf:blk.0.ssm_alpha.weight", "gguf:blk.0.ssm_beta.weight"]
    attn = [i for i in prog if i["kind"] == "ATTN_DECODE"][0]
    assert attn["layer"] == 3 and attn["kc"] == "state:cache_k.3"
    head = prog[-1]
    assert head["seg"][0]["w"] == "gguf:output.weight" and head["seg"][0]["epi"] == "ARGMAX"
    # every weight the graph reads is named by exactly one operand, except the
    # embedding table (the first op's aux) and the norm vectors (norm_w)
    names = []
    for i in prog:
        for s in i.get("seg", []):
            names += [s["w"]] + ([s["w2"]] if s.get("w2", "").startswith("gguf:") else [])
        names += [i[f] for f in ("norm_w", "aux", "dt_bias", "ssm_a", "q_norm", "k_norm")
                  if isinstance(i.get(f), str) and i[f].startswith("gguf:")]
    graph_weights = {"gguf:" + l["cls"].split(":", 1)[1] for l in g.leaves.values() if l["cls"].startswith("weight:")}
    assert len(names) == len(set(names)) and set(names) == graph_weights


def test_a_graph_with_a_missing_op_is_refused(g):
    # drop layer 5's recurrent step: its block is then neither kind of layer
    import copy
    bad = copy.deepcopy(g)
    for i, n in bad.nodes.items():
        if n["block"] == "5" and n["mkind"] == "deltanet_step":
            n["mkind"] = "unknown_kind"
    with pytest.raises(ValueError):
        schedule.fuse(bad)


def test_truncated_program_for_a_smaller_model(g):
    prog = schedule.truncate(schedule.symbolic_program(g), 8)
    assert sum(i["kind"] != "BOUNDARY" for i in prog) == 8 * 5 + 1
    assert prog[-1]["role"] == "head" and prog[-2]["kind"] == "BOUNDARY"
    assert schedule.program_layers(prog) == list(range(8))
