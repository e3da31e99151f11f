"""Write a small hybrid-model GGUF file for the loader tests -- test-only.

Tensor names follow llama.cpp's qwen35 GGUF naming (the names k0/leaves.csv
records): blk.N.{attn_norm, post_attention_norm, ffn_gate, ffn_up, ffn_down}
.weight; gated-DeltaNet blocks blk.N.{attn_qkv, attn_gate, ssm_alpha,
ssm_beta, ssm_out, ssm_conv1d, ssm_norm}.weight, blk.N.ssm_dt.bias,
blk.N.ssm_a; attention blocks blk.N.{attn_q, attn_k, attn_v, attn_output,
attn_q_norm, attn_k_norm}.weight; token_embd.weight, output_norm.weight,
output.weight.  Weight bytes come from sinter_synth on the host.
"""
import numpy as np

from gguf_writer import K_ARRAY, K_F32, K_I32, K_STRING, K_U32, Writer

F32, Q8_0, Q4_K, Q6_K, BF16 = 0, 8, 12, 14, 30


def small_cfg():
    return dict(n_layer=4, attn_every=4, E=1024, F=2048, V=3000, HK=2, HV=4, D=128, K=4, NQ=8, NKV=2, HD=256,
                rope_dims=64, rope_base=1e7, eps=1e-6)


def make_model_gguf(sn, path, c, types=None, tied=False, seed=4242, extra_block=False):
    """Write the model; returns {gguf name: (type, ne, bytes)}."""
    types = types or {}
    td = types.get("default", Q4_K)
    L = sn.lib()
    tensors = {}

    def weight(name, t, rows, k, s):
        out = np.zeros(sn.row_bytes(t, k) * rows, np.uint8)
        sn.check(L.sinter_synth(0, out.ctypes.data, sn.SYN_WEIGHT, t, rows, k, s, 0.0, 0.0, None), "synth")
        tensors[name] = (t, [k, rows], out)

    def vec(name, n, kind, a, b, s, ne=None):
        out = np.zeros(n, np.float32)
        sn.check(L.sinter_synth(0, out.ctypes.data, kind, F32, 1, n, s, a, b, None), "synth")
        tensors[name] = (F32, ne or [n], out)

    E, F, D, HK, HV = c["E"], c["F"], c["D"], c["HK"], c["HV"]
    C = (2 * HK + HV) * D
    s = seed
    n_blocks = c["n_layer"] + (1 if extra_block else 0)
    for il in range(n_blocks):
        b = "blk.%d." % il
        at = c["attn_every"] > 0 and il % c["attn_every"] == c["attn_every"] - 1
        vec(b + "attn_norm.weight", E, sn.SYN_NORMAL, 1.0, 0.02, s + 1)
        vec(b + "post_attention_norm.weight", E, sn.SYN_NORMAL, 1.0, 0.02, s + 2)
        weight(b + "ffn_gate.weight", types.get("ffn_gate", td), F, E, s + 3)
        weight(b + "ffn_up.weight", types.get("ffn_up", td), F, E, s + 4)
        weight(b + "ffn_down.weight", types.get("ffn_down", Q6_K), E, F, s + 5)
        if at:
            weight(b + "attn_q.weight", td, c["NQ"] * 2 * c["HD"], E, s + 6)
            weight(b + "attn_k.weight", td, c["NKV"] * c["HD"], E, s + 7)
            weight(b + "attn_v.weight", types.get("attn_v", Q6_K), c["NKV"] * c["HD"], E, s + 8)
            weight(b + "attn_output.weight", td, E, c["NQ"] * c["HD"], s + 9)
            vec(b + "attn_q_norm.weight", c["HD"], sn.SYN_NORMAL, 1.0, 0.02, s + 10)
            vec(b + "attn_k_norm.weight", c["HD"], sn.SYN_NORMAL, 1.0, 0.02, s + 11)
        else:
            weight(b + "attn_qkv.weight", td, C, E, s + 6)
            weight(b + "attn_gate.weight", td, HV * D, E, s + 7)
            weight(b + "ssm_alpha.weight", td, HV, E, s + 8)
            weight(b + "ssm_beta.weight", td, HV, E, s + 9)
            weight(b + "ssm_out.weight", td, E, HV * D, s + 10)
            vec(b + "ssm_conv1d.weight", C * c["K"], sn.SYN_UNIFORM, -0.5, 0.5, s + 11, ne=[c["K"], C])
            vec(b + "ssm_dt.bias", HV, sn.SYN_UNIFORM, -6.9, -2.3, s + 12)
            vec(b + "ssm_a", HV, sn.SYN_UNIFORM, -16.0, -1.0, s + 13)
            vec(b + "ssm_norm.weight", D, sn.SYN_NORMAL, 1.0, 0.02, s + 14)
        s += 100
    weight("token_embd.weight", types.get("embd", Q4_K), c["V"], E, s + 1)
    vec("output_norm.weight", E, sn.SYN_NORMAL, 1.0, 0.02, s + 2)
    if not tied:
        weight("output.weight", types.get("output", Q6_K), c["V"], E, s + 3)
    w = Writer()
    w.add_kv("general.architecture", K_STRING, "qwen35")
    w.add_kv("general.alignment", K_U32, 32)
    w.add_kv("qwen35.block_count", K_U32, n_blocks)
    w.add_kv("qwen35.rope.dimension_count", K_U32, c["rope_dims"])
    w.add_kv("qwen35.rope.freq_base", K_F32, c["rope_base"])
    w.add_kv("qwen35.attention.layer_norm_rms_epsilon", K_F32, c["eps"])
    w.add_kv("qwen35.rope.dimension_sections", K_ARRAY, [11, 11, 10, 0], K_I32)
    if extra_block:
        w.add_kv("qwen35.nextn_predict_layers", K_U32, 1)
    for name, (t, ne, data) in tensors.items():
        w.add_tensor(name, ne, t, data)
    w.write(path)
    return tensors
