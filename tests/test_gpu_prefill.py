"""On-GPU prefill: the batched prefill (sinter_model_prefill_batched, each
layer once per ubatch of tokens) and the decode program over the prompt
(sinter_model_prefill_tokenwise, each pass's next token forced to the
prompt's) leave the KV rows, the recurrent and conv states and the logits of
decoding the prompt one token at a time -- checked bit for bit against
single-pass decodes, against each other (ragged ubatches, both KV cache
types, split-K geometries whose chunk length changes inside a block of
queries) and against the CPU oracle."""
import ctypes as C

import numpy as np
import pytest

from test_gpu_model import compare_logits, small_config

pytestmark = pytest.mark.gpu


def device_bytes(m, d, nb):
    a = np.empty(nb, np.uint8)
    m.d2h(a, d, nb)
    return a


def same_state(a, b, cfg):
    for il in range(cfg.n_layer):
        for s in range(2):
            da, na = a.state(il, s)
            db, nb = b.state(il, s)
            assert na == nb
            assert np.array_equal(device_bytes(a, da, na), device_bytes(b, db, nb)), (il, s)


@pytest.mark.parametrize("mode", ["tokenwise", "batched"])
def test_prefill_equals_single_pass_decodes(sn, torch_gpu, mode):
    """1100 tokens: more passes than one decode-program launch runs (1024),
    five ubatches of the batched prefill (the last one ragged)."""
    cfg = small_config(sn, n_layer=8, n_ctx=1280)
    n = 1100
    toks = [int(t) for t in np.random.default_rng(3).integers(0, cfg.n_vocab, n)]
    a, b = sn.Model(cfg, seed=41), sn.Model(cfg, seed=41)
    try:
        print(f"prefill {mode}: {n} tokens", flush=True)
        nxt_a = a.prefill(toks, 0, mode=mode)
        print("prefill: the same tokens one pass per call", flush=True)
        nxt_b = None
        for i, t in enumerate(toks):
            nxt_b = b.decode(t, i)
        assert nxt_a == nxt_b
        assert np.array_equal(a.logits(), b.logits())
        same_state(a, b, cfg)
        assert a.greedy(nxt_a, n, 8) == b.greedy(nxt_b, n, 8)
    finally:
        a.close()
        b.close()


@pytest.mark.parametrize("mode", ["tokenwise", "batched"])
def test_prefill_matches_oracle_from_a_context(sn, orc, torch_gpu, mode):
    cfg = small_config(sn, n_layer=4, n_ctx=256)
    m = sn.Model(cfg, seed=43)
    try:
        m.synth_context(40, seed=44)
        mirror = orc.ModelMirror(m)
        prompt = [17, 2999, 0, 1234, 77, 5]
        print(f"prefill {mode}: {len(prompt)} tokens after a 40-token context", flush=True)
        nxt = m.prefill(prompt, 40, mode=mode)
        rtok, rlog = None, None
        for i, t in enumerate(prompt):
            rtok, rlog = mirror.step(t, 40 + i)
        print(f"prefill next: gpu {nxt} oracle {rtok}", flush=True)
        assert nxt == rtok
        compare_logits(m.logits(), rlog)
        # decoding continues from the prefilled state
        gpu = m.greedy(nxt, 46, 3)
        ref, t = [], nxt
        for p in (46, 47, 48):
            t = mirror.step(t, p)[0]
            ref.append(t)
        assert gpu == ref
    finally:
        m.close()


def test_prefill_refuses_bad_arguments(sn, torch_gpu):
    cfg = small_config(sn, n_layer=4, n_ctx=64)
    m = sn.Model(cfg, seed=45)
    try:
        L = sn.lib()
        arr = (C.c_int32 * 8)(*range(8))
        nxt = C.c_int32()
        assert L.sinter_model_prefill(m.h, arr, 8, 60, C.byref(nxt)) == sn.ERR_ARG      # past n_ctx
        assert L.sinter_model_prefill(m.h, arr, 0, 0, C.byref(nxt)) == sn.ERR_ARG
        bad = (C.c_int32 * 2)(1, cfg.n_vocab)
        assert L.sinter_model_prefill(m.h, bad, 2, 0, C.byref(nxt)) == sn.ERR_ARG      # token out of range
        assert 0 <= m.prefill([1, 2, 3], 0) < cfg.n_vocab      # the refusals left the model usable
    finally:
        m.close()


# (ubatch, KV type, attn_chunks, attn_chunk_min, context, prompt): one-token
# ubatches; a ragged 7; chunks of 2 and 3 per kv head, where a query's chunk
# length (tiles per chunk) changes every few positions, so the 8 queries of a
# block split differently; a Q8_0 cache
BATCH_CASES = [
    (1, "f16", 0, 0, 0, 40),
    (7, "f16", 0, 0, 30, 150),
    (64, "f16", 2, 128, 0, 300),
    (33, "q8_0", 3, 32, 17, 260),
    (256, "q8_0", 0, 0, 100, 380),
]


@pytest.mark.parametrize("ub,kv,chunks,cmin,ctx,n", BATCH_CASES)
def test_batched_prefill_equals_tokenwise(sn, torch_gpu, ub, kv, chunks, cmin, ctx, n):
    cfg = small_config(sn, n_layer=4, n_ctx=512)
    cfg.t_kv = {"f16": sn.F16, "q8_0": sn.Q8_0}[kv]
    cfg.attn_chunks, cfg.attn_chunk_min = chunks, cmin
    rng = np.random.default_rng(ub * 1000 + n)
    toks = [int(t) for t in rng.integers(0, cfg.n_vocab, n)]
    a, b = sn.Model(cfg, seed=47), sn.Model(cfg, seed=47)
    try:
        if ctx:
            a.synth_context(ctx, seed=48)
            b.synth_context(ctx, seed=48)
        print(f"batched prefill ubatch={ub} kv={kv} chunks={chunks} cmin={cmin} ctx={ctx} n={n}", flush=True)
        nxt_a = a.prefill(toks, ctx, mode="batched", ubatch=ub)
        print("tokenwise prefill of the same prompt", flush=True)
        nxt_b = b.prefill(toks, ctx, mode="tokenwise")
        assert nxt_a == nxt_b
        assert np.array_equal(a.logits(), b.logits())
        same_state(a, b, cfg)
        # a second prefill continues from the first (its positions follow)
        more = [int(t) for t in rng.integers(0, cfg.n_vocab, 20)]
        print("a second batched prefill after the first", flush=True)
        assert a.prefill(more, ctx + n, mode="batched", ubatch=ub) == b.prefill(more, ctx + n, mode="tokenwise")
        assert np.array_equal(a.logits(), b.logits())
        same_state(a, b, cfg)
    finally:
        a.close()
        b.close()


def test_batched_prefill_refuses_other_weight_types(sn, torch_gpu):
    """A bf16 model has no batched path: sinter_model_prefill_batched refuses
    it, sinter_model_prefill runs the decode passes instead."""
    cfg = small_config(sn, n_layer=4, n_ctx=64, quant="bf16")
    m = sn.Model(cfg, seed=49)
    try:
        L = sn.lib()
        arr = (C.c_int32 * 4)(5, 6, 7, 8)
        nxt = C.c_int32()
        assert L.sinter_model_prefill_batched(m.h, arr, 4, 0, 16, C.byref(nxt)) == sn.ERR_ARG
        assert L.sinter_model_prefill(m.h, arr, 4, 0, C.byref(nxt)) == sn.OK
    finally:
        m.close()
    cfg = small_config(sn, n_layer=4, n_ctx=64)
    m = sn.Model(cfg, seed=49)
    try:
        L = sn.lib()
        arr = (C.c_int32 * 4)(5, 6, 7, 8)
        nxt = C.c_int32()
        assert L.sinter_model_prefill_batched(m.h, arr, 4, 0, 0, C.byref(nxt)) == sn.ERR_ARG      # ubatch 0
        assert L.sinter_model_prefill_batched(m.h, arr, 4, 0, 4096, C.byref(nxt)) == sn.ERR_ARG   # over the max
        assert L.sinter_model_prefill_batched(m.h, arr, 4, 62, 16, C.byref(nxt)) == sn.ERR_ARG   # past n_ctx
    finally:
        m.close()


@pytest.mark.parametrize("d,hk,hv", [(64, 2, 4), (256, 1, 2)])
def test_batched_prefill_gdn_head_sizes(sn, torch_gpu, d, hk, hv):
    """The GDN scan's other layouts (head size 64: 16 columns per item, 4 rows
    per thread; 256: 32 rows per thread) against the decode program."""
    cfg = small_config(sn, n_layer=4, n_ctx=256)
    cfg.gdn_d, cfg.gdn_hk, cfg.gdn_hv = d, hk, hv
    toks = [int(t) for t in np.random.default_rng(d).integers(0, cfg.n_vocab, 70)]
    a, b = sn.Model(cfg, seed=51), sn.Model(cfg, seed=51)
    try:
        print(f"batched prefill gdn_d={d} hk={hk} hv={hv}", flush=True)
        nxt_a = a.prefill(toks, 0, mode="batched", ubatch=32)
        nxt_b = b.prefill(toks, 0, mode="tokenwise")
        assert nxt_a == nxt_b
        assert np.array_equal(a.logits(), b.logits())
        same_state(a, b, cfg)
    finally:
        a.close()
        b.close()
