"""End-to-end decode on the GPU interpreter vs the CPU oracle.

The model is created through the C ABI (weights synthesised on device),
then mirrored to host memory for the oracle, so both sides run the same
pass on the same bytes.  Greedy token ids must be identical; logits are
compared element-wise (bit-exact except for fp64 fold-order effects).
"""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def small_config(sn, n_layer=4, n_ctx=512, quant="q4_k_m"):
    c = sn.qwen36_27b_config(n_ctx=n_ctx, quant=quant, n_layer=n_layer)
    c.n_embd, c.n_ff, c.n_vocab = 1024, 2048, 3000
    c.gdn_hk, c.gdn_hv = 2, 4
    c.attn_nq, c.attn_nkv = 8, 2
    return c


def compare_logits(got, ref):
    ulp = np.abs(np.spacing(ref))
    bad = np.abs(got - ref) > 4 * ulp
    assert bad.mean() < 1e-3, (bad.mean(), np.abs(got - ref).max())
    rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert rel < 1e-5, rel


@pytest.mark.parametrize("quant", ["q4_k_m", "bf16"])
def test_small_model_decode_matches_oracle(sn, orc, torch_gpu, quant):
    cfg = small_config(sn, quant=quant)
    print(f"small model {quant}: create", flush=True)
    m = sn.Model(cfg, seed=11)
    try:
        m.synth_context(40, seed=12)
        mirror = orc.ModelMirror(m)
        info = m.info()
        assert info["n_boundaries"] == 5 * cfg.n_layer + 1
        # the interpreter specialised for the program's types runs it
        assert info["kernel"] == {"q4_k_m": "sinter_interp_kquant", "bf16": "sinter_interp_bf16"}[quant]
        tok, pos = 17, 40
        for step in range(6):
            logits = np.zeros(cfg.n_vocab, np.float32)
            nxt = m.decode(tok, pos, logits)
            rtok, rlog = mirror.step(tok, pos)
            print(f"step {step}: gpu {nxt} oracle {rtok}", flush=True)
            compare_logits(logits, rlog)
            assert nxt == rtok == int(np.argmax(rlog))
            tok, pos = nxt, pos + 1
    finally:
        m.close()


def test_full_shape_decode_matches_oracle(sn, orc, torch_gpu):
    """The benchmark configuration itself (64 layers, Qwen3.6-27B shapes,
    Q4_K_M mix, 4096-token synthetic context), single-pass path: two greedy
    steps on the GPU and on the CPU oracle from the same weights and state;
    identical token ids, logits within rel L2 1e-5 (the pass bar is 1e-2).
    Then a 20-token batched prefill (ubatches of 8, 8 and 4 tokens) against
    the oracle stepping the same tokens: the same next token and logits
    within rel L2 1e-5."""
    cfg = sn.qwen36_27b_config(n_ctx=4096 + 32, quant="q4_k_m")
    print("full shape: create", flush=True)
    m = sn.Model(cfg, seed=2026)
    try:
        m.synth_context(4096, seed=2027)
        print("full shape: mirror to host", flush=True)
        mirror = orc.ModelMirror(m)
        tok, pos = 1, 4096
        for step in range(2):
            logits = np.zeros(cfg.n_vocab, np.float32)
            nxt = m.decode(tok, pos, logits)
            rtok, rlog = mirror.step(tok, pos)
            rel = np.linalg.norm(logits - rlog) / np.linalg.norm(rlog)
            print(f"full shape step {step}: gpu {nxt} oracle {rtok} rel {rel:.2e}", flush=True)
            assert nxt == rtok == int(np.argmax(rlog))
            assert rel < 1e-5, rel
            tok, pos = nxt, pos + 1
        prompt = [int(t) for t in np.random.default_rng(2028).integers(0, cfg.n_vocab, 20)]
        print(f"full shape: batched prefill of {len(prompt)} tokens at {pos}", flush=True)
        nxt = m.prefill(prompt, pos, mode="batched", ubatch=8)
        for i, t in enumerate(prompt):
            rtok, rlog = mirror.step(t, pos + i)
        rel = np.linalg.norm(m.logits() - rlog) / np.linalg.norm(rlog)
        print(f"full shape prefill: gpu {nxt} oracle {rtok} rel {rel:.2e}", flush=True)
        assert nxt == rtok
        assert rel < 1e-5, rel
    finally:
        m.close()


def test_full_shape_balanced_greedy_matches_oracle(sn, orc, torch_gpu):
    """The path the benchmark times, at its configuration: the static GEMV
    load balance (traced single passes), then one launch of 12 greedy passes
    of the cooperative interpreter.  Every token id equals the CPU oracle's
    greedy decode from the same weights and 4096-token state, and the logits
    of the launch's last pass are within rel L2 1e-5 of the oracle's."""
    cfg = sn.qwen36_27b_config(n_ctx=4096 + 32, quant="q4_k_m")
    print("balanced greedy: create", flush=True)
    m = sn.Model(cfg, seed=2026)
    try:
        m.synth_context(4096, seed=2027)
        mirror = orc.ModelMirror(m)
        tok, pos = m.balance(1, 4096, rounds=1, traces=2)     # 4 traced greedy passes
        rtok = 1
        for i in range(4):
            rtok, _ = mirror.step(rtok, 4096 + i)
        print(f"balanced greedy: balance ended at ({tok}, {pos}), oracle token {rtok}", flush=True)
        assert (tok, pos) == (rtok, 4100)
        toks = m.greedy(tok, pos, 12)
        last = m.logits()
        ref = []
        for i in range(12):
            rtok, rlog = mirror.step(rtok, pos + i)
            ref.append(rtok)
        print(f"balanced greedy: gpu {toks} oracle {ref}", flush=True)
        assert toks == ref
        rel = np.linalg.norm(last - rlog) / np.linalg.norm(rlog)
        assert rel < 1e-5, rel
    finally:
        m.close()


@pytest.mark.timeout(400)
def test_config5_bf16_full_context_matches_oracle(sn, orc, torch_gpu):
    """BASELINE config 5 at its full shape: 64 layers (48 gated-DeltaNet + 16
    attention), bf16 weights, 131072 f16 KV positions, 131068 of them filled
    (so every split-K merge runs over 64 chunks of ~2048 positions per KV
    head).  Two greedy passes in one launch equal the oracle's tokens; the
    last logits are within rel L2 1e-5 (the host mirror holds ~63 GB)."""
    cfg = sn.qwen36_27b_config(n_ctx=131072, quant="bf16")
    print("config 5: create", flush=True)
    m = sn.Model(cfg, seed=5005)
    mirror = None
    try:
        ctx = 131068
        m.synth_context(ctx, seed=5006)
        print("config 5: mirror to host", flush=True)
        mirror = orc.ModelMirror(m)
        toks = m.greedy(9, ctx, 2)
        last = m.logits()
        ref, rtok = [], 9
        for i in range(2):
            rtok, rlog = mirror.step(rtok, ctx + i)
            ref.append(rtok)
            print(f"config 5 step {i}: gpu {toks[i]} oracle {rtok}", flush=True)
        assert toks == ref
        rel = np.linalg.norm(last - rlog) / np.linalg.norm(rlog)
        assert rel < 1e-5, rel
    finally:
        del mirror
        m.close()


@pytest.mark.timeout(400)
def test_full_shape_256_greedy_steps_match_oracle(sn, orc, torch_gpu):
    """The benchmark's decode at its configuration for the north star's 256
    greedy steps: 64 layers, Q4_K_M mix, 4096-token synthetic context, the
    static GEMV balance, then 16 launches of 16 greedy passes of the
    cooperative interpreter.  All 256 token ids equal the CPU oracle's greedy
    decode from the same weights and state, and each launch's last logits are
    within rel L2 1e-5 of the oracle's."""
    cfg = sn.qwen36_27b_config(n_ctx=4096 + 300, quant="q4_k_m")
    print("256 steps: create", flush=True)
    m = sn.Model(cfg, seed=2026)
    try:
        m.synth_context(4096, seed=2027)
        mirror = orc.ModelMirror(m)
        tok, pos = m.balance(1, 4096, rounds=1, traces=2)
        rtok = 1
        for i in range(4):
            rtok, _ = mirror.step(rtok, 4096 + i)
        assert (tok, pos) == (rtok, 4100)
        done, worst = 0, 0.0
        while done < 256:
            toks = m.greedy(tok, pos, 16)
            last = m.logits()
            ref = []
            for i in range(16):
                rtok, rlog = mirror.step(rtok, pos + i)
                ref.append(rtok)
            rel = float(np.linalg.norm(last - rlog) / np.linalg.norm(rlog))
            worst = max(worst, rel)
            print(f"256 steps: {done}..{done + 15} gpu {toks} oracle {ref} rel {rel:.1e}", flush=True)
            assert toks == ref, (done, toks, ref)
            tok, pos, done = toks[-1], pos + 16, done + 16
        assert worst < 1e-5, worst
    finally:
        m.close()


def test_greedy_multi_pass_equals_single_passes(sn, orc, torch_gpu):
    cfg = small_config(sn, n_layer=8)
    m = sn.Model(cfg, seed=21)
    try:
        m.synth_context(100, seed=22)
        mirror = orc.ModelMirror(m)
        toks = m.greedy(5, 100, 12)        # one launch, 12 passes
        ref = []
        tok = 5
        for i in range(12):
            tok, _ = mirror.step(tok, 100 + i)
            ref.append(tok)
        assert toks == ref
    finally:
        m.close()


def test_gemv_balance_leaves_results_unchanged(sn, torch_gpu):
    """sinter_model_balance moves GEMV rows between workgroups: the tokens it
    decodes and every later token and logit equal those of a model that was
    never rebalanced (rows are folded by one lane each, wherever they run)."""
    cfg = small_config(sn, n_layer=8)
    a, b = sn.Model(cfg, seed=31), sn.Model(cfg, seed=31)
    try:
        for m in (a, b):
            m.synth_context(100, seed=32)
        ref = a.greedy(5, 100, 16)
        tok, pos = b.balance(5, 100, rounds=3, traces=2)   # 4 measurements of 2 passes
        assert (tok, pos) == (ref[7], 108)
        assert b.greedy(tok, pos, 8) == ref[8:16]
        la, lb = np.zeros(cfg.n_vocab, np.float32), np.zeros(cfg.n_vocab, np.float32)
        assert a.decode(ref[15], 116, la) == b.decode(ref[15], 116, lb)
        assert np.array_equal(la, lb)
        # the low-level entry point refuses what it cannot apply
        h = b.host()
        one = (C.c_float * cfg.n_vocab)(*([1.0] * cfg.n_vocab))
        assert sn.lib().sinter_host_set_gemv_shares(h, 1, one, 3) == sn.ERR_ARG   # wrong count / not a GEMV
        assert sn.lib().sinter_host_set_gemv_shares(h, 10 ** 6, one, 3) == sn.ERR_ARG
    finally:
        a.close()
        b.close()


def test_error_cell_path_bad_kind(sn, torch_gpu):
    """An unknown instruction kind ends the pass with RUN_ERR and the
    instruction index in the error cell (core/interp.cuh error protocol)."""
    L = sn.lib()
    h = C.c_void_p()
    sn.check(L.sinter_host_init(C.byref(h), 0, 0), "init")
    try:
        prog = (sn.Instr * 3)()
        blocks = C.c_uint32()
        L.sinter_host_grid(h, C.byref(blocks), None, None)
        prog[0].kind, prog[0].block_hi = sn.OP_NOP, blocks.value
        prog[1].kind = sn.OP_BOUNDARY
        prog[2].kind, prog[2].block_hi = 77, blocks.value
        sn.check(L.sinter_host_upload(h, prog, 3, 1), "upload")
        sn.check(L.sinter_host_launch(h), "launch")
        assert L.sinter_host_run_pass(h, 0, 20000.0) == sn.RUN_ERR
        code, aux = C.c_uint32(), C.c_uint32()
        L.sinter_host_error(h, C.byref(code), C.byref(aux))
        assert code.value == sn.E_BAD_KIND and aux.value == 2
        assert L.sinter_host_shutdown(h, 1000.0) == 0
    finally:
        L.sinter_host_destroy(h)


@pytest.mark.parametrize("quant,special", [("q4_k_m", "sinter_interp_kquant"), ("bf16", "sinter_interp_bf16")])
def test_specialised_interpreter_equals_general(sn, torch_gpu, monkeypatch, quant, special):
    """A specialised interpreter (the cases of other types compiled out) and
    the general one decode bit-identically: same tokens, same logits."""
    cfg = small_config(sn, n_layer=8, n_ctx=256, quant=quant)
    runs = {}
    for name in (special, "sinter_interp"):
        if name == "sinter_interp":
            monkeypatch.setenv("SINTER_INTERP", "general")
        m = sn.Model(cfg, seed=71)
        try:
            assert m.info()["kernel"] == name
            m.synth_context(50, seed=72)
            toks = m.greedy(11, 50, 12)
            runs[name] = (toks, m.logits().copy())
            print(f"{name}: {toks}", flush=True)
        finally:
            m.close()
    (ta, la), (tb, lb) = runs.values()
    assert ta == tb
    assert np.array_equal(la, lb)
