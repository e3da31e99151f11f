"""On-GPU prefill (sinter_model_prefill): the prompt's tokens run through
the decode program with each pass's next token forced to the prompt's, so the
KV rows, the recurrent and conv states and the logits it leaves are those of
decoding the prompt one token at a time -- checked bit for bit against
single-pass decodes (over two launches) and against the CPU oracle."""
import ctypes as C

import numpy as np
import pytest

from test_gpu_model import compare_logits, small_config

pytestmark = pytest.mark.gpu


def device_bytes(m, d, nb):
    a = np.empty(nb, np.uint8)
    m.d2h(a, d, nb)
    return a


def test_prefill_equals_single_pass_decodes(sn, torch_gpu):
    cfg = small_config(sn, n_layer=8, n_ctx=1280)
    n = 1100                                   # more passes than one prefill launch runs (1024)
    toks = [int(t) for t in np.random.default_rng(3).integers(0, cfg.n_vocab, n)]
    a, b = sn.Model(cfg, seed=41), sn.Model(cfg, seed=41)
    try:
        print(f"prefill: {n} tokens in launches", flush=True)
        nxt_a = a.prefill(toks, 0)
        print("prefill: the same tokens one pass per call", flush=True)
        nxt_b = None
        for i, t in enumerate(toks):
            nxt_b = b.decode(t, i)
        assert nxt_a == nxt_b
        assert np.array_equal(a.logits(), b.logits())
        for il in range(cfg.n_layer):
            for s in range(2):
                da, na = a.state(il, s)
                db, nb = b.state(il, s)
                assert na == nb
                assert np.array_equal(device_bytes(a, da, na), device_bytes(b, db, nb)), (il, s)
        assert a.greedy(nxt_a, n, 8) == b.greedy(nxt_b, n, 8)
    finally:
        a.close()
        b.close()


def test_prefill_matches_oracle_from_a_context(sn, orc, torch_gpu):
    cfg = small_config(sn, n_layer=4, n_ctx=256)
    m = sn.Model(cfg, seed=43)
    try:
        m.synth_context(40, seed=44)
        mirror = orc.ModelMirror(m)
        prompt = [17, 2999, 0, 1234, 77, 5]
        nxt = m.prefill(prompt, 40)
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
