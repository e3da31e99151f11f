"""A model loaded from a GGUF file (sinter_model_create_from_gguf) on the GPU.

The file is written by tests/gguf_model.py; every weight on the device must
equal the file's bytes (the blocks are uploaded as they lie, never repacked),
and greedy decoding must equal the CPU oracle run on those device tensors,
for a Q4_K/Q6_K mix, an all-Q8_0 file and a file with a tied head and a
trailing multi-token-prediction block.
"""
import numpy as np
import pytest

from gguf_model import Q4_K, Q6_K, Q8_0, make_model_gguf, small_cfg

pytestmark = pytest.mark.gpu

GDN_NAMES = {0: "attn_norm.weight", 1: "post_attention_norm.weight", 2: "ffn_gate.weight", 3: "ffn_up.weight",
             4: "ffn_down.weight", 5: "attn_qkv.weight", 6: "attn_gate.weight", 7: "ssm_alpha.weight",
             8: "ssm_beta.weight", 9: "ssm_out.weight", 10: "ssm_conv1d.weight", 11: "ssm_dt.bias", 12: "ssm_a",
             13: "ssm_norm.weight"}
ATT_NAMES = {0: "attn_norm.weight", 1: "post_attention_norm.weight", 2: "ffn_gate.weight", 3: "ffn_up.weight",
             4: "ffn_down.weight", 5: "attn_q.weight", 6: "attn_k.weight", 7: "attn_v.weight",
             8: "attn_output.weight", 9: "attn_q_norm.weight", 10: "attn_k_norm.weight"}


@pytest.mark.parametrize("variant", ["q4_k_m", "q8_0", "tied_mtp"])
def test_gguf_model_uploads_file_bytes_and_decodes(sn, orc, torch_gpu, tmp_path, variant):
    c = small_cfg()
    types = {"default": Q8_0, "ffn_down": Q8_0, "attn_v": Q8_0, "embd": Q8_0, "output": Q8_0} \
        if variant == "q8_0" else None
    path = str(tmp_path / "m.gguf")
    tensors = make_model_gguf(sn, path, c, types=types, tied=variant == "tied_mtp",
                              extra_block=variant == "tied_mtp")
    print(f"gguf {variant}: create from file", flush=True)
    with sn.Gguf(path) as g:
        m = sn.Model(g.config(256), gguf=g)
    try:
        cfg = m.cfg
        assert cfg.n_layer == c["n_layer"] and cfg.n_embd == c["E"]
        for il in range(cfg.n_layer):
            names = ATT_NAMES if il % 4 == 3 else GDN_NAMES
            for slot, nm in names.items():
                d, nb, t = m.tensor(il, slot)
                ft, _, data = tensors["blk.%d.%s" % (il, nm)]
                got = np.empty(nb, np.uint8)
                m.d2h(got, d, nb)
                assert t == ft and np.array_equal(got, data.view(np.uint8).reshape(-1)), (il, nm)
        for slot, nm in ((0, "token_embd.weight"), (1, "output_norm.weight"),
                         (2, "token_embd.weight" if variant == "tied_mtp" else "output.weight")):
            d, nb, t = m.tensor(cfg.n_layer, slot)
            got = np.empty(nb, np.uint8)
            m.d2h(got, d, nb)
            assert np.array_equal(got, tensors[nm][2].view(np.uint8).reshape(-1)), nm
        m.synth_context(30, seed=77)
        mirror = orc.ModelMirror(m)
        toks = m.greedy(11, 30, 4)
        last = m.logits()
        ref, rt = [], 11
        for i in range(4):
            rt, rlog = mirror.step(rt, 30 + i)
            ref.append(rt)
        print(f"gguf {variant}: gpu {toks} oracle {ref}", flush=True)
        assert toks == ref
        assert np.linalg.norm(last - rlog) / np.linalg.norm(rlog) < 1e-5
    finally:
        m.close()


def test_gguf_model_refuses_unsupported_weight_type(sn, torch_gpu, tmp_path):
    """A weight type the kernels do not read (Q5_K here) is refused before
    anything runs, with the tensor named in the message."""
    from gguf_writer import Writer
    c = small_cfg()
    path = str(tmp_path / "m.gguf")
    tensors = make_model_gguf(sn, path, c)
    w = Writer()
    for name, (t, ne, data) in tensors.items():
        if name == "blk.0.ffn_gate.weight":
            t, data = 13, np.zeros(176 * (ne[0] // 256) * ne[1], np.uint8)   # Q5_K blocks
        w.add_tensor(name, ne, t, data)
    w.write(path)
    import ctypes as C
    with sn.Gguf(path) as g:
        h = C.c_void_p()
        rc = sn.lib().sinter_model_create_from_gguf(g.h, 0, 256, 0, C.byref(h))
        assert rc == sn.ERR_ARG and not h.value
        assert b"blk.0.ffn_gate.weight" in sn.lib().sinter_last_error()
