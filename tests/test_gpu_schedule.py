"""The schedule compiler's program on the GPU: the symbolic program compiled
from the reference's captured decode graph (tests/golden/k0_schedule.csv),
cut to the first 8 layers and packed against a model of the same layer
pattern (schedule.pack), is byte-identical to the program the library's own
packer uploads (model.cpp build_program), and decodes to the same tokens and
logits once uploaded in its place."""
import os

import numpy as np
import pytest

import schedule

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))


def small_config(sn, n_layer=8):
    c = sn.qwen36_27b_config(n_ctx=256, n_layer=n_layer)
    c.n_embd, c.n_ff, c.n_vocab = 1024, 2048, 3000
    c.gdn_hk, c.gdn_hv = 2, 4
    c.attn_nq, c.attn_nkv = 8, 2
    return c


def test_compiled_program_equals_the_library_program_and_decodes(sn, torch_gpu):
    g = schedule.load(os.path.join(HERE, "golden", "k0_schedule.csv"), os.path.join(HERE, "golden", "k0_leaves.csv"))
    prog = schedule.truncate(schedule.symbolic_program(g), 8)
    cfg = small_config(sn)
    a, b = sn.Model(cfg, seed=41), sn.Model(cfg, seed=41)
    try:
        packed = schedule.pack(b, prog)
        own = b.program()
        print(f"schedule: {len(packed)} packed, {len(own)} own instructions", flush=True)
        assert len(packed) == len(own)
        for k in range(len(own)):
            assert bytes(packed[k]) == bytes(own[k]), (k, own[k].kind)
        b.upload_program(packed)
        for m in (a, b):
            m.synth_context(40, seed=42)
        ta, tb = a.greedy(7, 40, 6), b.greedy(7, 40, 6)
        assert ta == tb
        assert np.array_equal(a.logits(), b.logits())
    finally:
        a.close()
        b.close()
