"""The C-ABI library loads and exports every declared entry point; host-side
logic that runs without a GPU (argument validation, synthetic data)."""
import ctypes as C
import os
import re
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "sinter.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = set(re.findall(r"\b(sinter_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def test_every_declared_symbol_is_exported(sn):
    lib = sn.lib()
    names = declared_functions()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    out = subprocess.run(["nm", "-D", "--defined-only", sn.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT (sinter_[a-z0-9_]+)", out))
    assert set(names) <= exported


def test_abi_version_and_struct_layout(sn, tmp_path):
    assert sn.lib().sinter_abi_version() == 1
    src = tmp_path / "sz.c"
    src.write_text('#include "sinter.h"\n#include <stdio.h>\n#include <stddef.h>\nint main(void){printf("%zu %zu %zu %zu %zu %zu %zu\\n",'
                   'sizeof(sinter_instr),sizeof(sinter_gemv_seg),sizeof(sinter_gemv_args),sizeof(sinter_gdn_args),'
                   'sizeof(sinter_attn_args),sizeof(sinter_model_config),offsetof(sinter_gemv_args,seg));return 0;}\n')
    exe = tmp_path / "sz"
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    got = list(map(int, subprocess.run([str(exe)], capture_output=True, text=True).stdout.split()))
    assert got == [C.sizeof(sn.Instr), C.sizeof(sn.GemvSeg), C.sizeof(sn.GemvArgs), C.sizeof(sn.GdnArgs),
                   C.sizeof(sn.AttnArgs), C.sizeof(sn.ModelConfig), sn.GemvArgs.seg.offset]


def test_row_bytes(sn):
    L = sn.lib()
    assert L.sinter_row_bytes(sn.Q4_K, 5120) == 2880
    assert L.sinter_row_bytes(sn.Q6_K, 5120) == 4200
    assert L.sinter_row_bytes(sn.Q6_K, 17408) == 14280
    assert L.sinter_row_bytes(sn.Q8_0, 5120) == 5440
    assert L.sinter_row_bytes(sn.BF16, 5120) == 10240


def test_gemv_argument_validation_rejects_before_launch(sn):
    """Shapes the kernel does not support are refused on the host with
    SINTER_ERR_ARG and a message; no device call is made."""
    L = sn.lib()
    a = sn.GemvArgs()
    a.K = 5000                       # not a multiple of 256
    a.n_seg = 1
    a.pro = sn.PRO_PLAIN
    a.x = 16
    a.seg[0].w = 256
    a.seg[0].y = 512
    a.seg[0].rows = 4
    a.seg[0].type = sn.Q4_K
    assert L.sinter_op_gemv(C.byref(a), 4, None) == sn.ERR_ARG
    assert b"multiple of 256" in L.sinter_last_error()
    a.K = 5120
    a.seg[0].w = 258                 # unaligned weights
    assert L.sinter_op_gemv(C.byref(a), 4, None) == sn.ERR_ARG
    a.seg[0].w = 256
    a.seg[1].type = sn.Q8_0          # mixed vec_dot types
    a.seg[1].w = 256
    a.seg[1].y = 512
    a.n_seg = 2
    assert L.sinter_op_gemv(C.byref(a), 4, None) == sn.ERR_ARG
    assert b"vec_dot" in L.sinter_last_error()
    a.n_seg = 1
    a.K = 65536                      # activation does not fit the LDS buffer
    assert L.sinter_op_gemv(C.byref(a), 4, None) == sn.ERR_ARG
    g = sn.GdnArgs()
    assert L.sinter_op_gdn_step(C.byref(g), 4, None) == sn.ERR_ARG
    t = sn.AttnArgs()
    assert L.sinter_op_attn_decode(C.byref(t), 4, None) == sn.ERR_ARG
    # a valid shape, but fewer workgroups than (kv head, chunk) items: the
    # chunks of a kv head wait for each other, so every item needs its own
    t = sn.AttnArgs(nq=24, nkv=4, hd=256, rope_dims=64, n_ctx=64, n_chunks=16, theta_scale=0.5, eps=1e-6,
                    scale=0.0625)
    t.qg = t.k = t.v = t.q_norm = t.k_norm = t.part = t.count = t.out = t.pass_cell = 256
    t.kc = t.vc = 256
    assert L.sinter_op_attn_decode(C.byref(t), 63, None) == sn.ERR_ARG
    assert b"nkv * n_chunks" in L.sinter_last_error()


def test_gemv_ubatch_argument_validation_rejects_before_launch(sn):
    """The batched GEMV and its Q8_K quantiser refuse unsupported types,
    shapes and alignments on the host (SINTER_ERR_ARG, nothing launched);
    zero tokens is a no-op."""
    L = sn.lib()
    f = L.sinter_op_gemv_ubatch
    W, X, Y = C.c_void_p(4096), C.c_void_p(8192), C.c_void_p(16384)
    assert f(sn.Q8_0, W, 16, 256, X, 4, Y, 0, None) == sn.ERR_ARG
    assert b"Q4_K or Q6_K" in L.sinter_last_error()
    assert f(sn.Q4_K, W, 16, 300, X, 4, Y, 0, None) == sn.ERR_ARG
    assert b"multiple of 256" in L.sinter_last_error()
    assert f(sn.Q4_K, W, 0, 256, X, 4, Y, 0, None) == sn.ERR_ARG
    assert f(sn.Q4_K, W, 16, 256, X, 0, Y, 0, None) == sn.OK
    assert f(sn.Q4_K, None, 16, 256, X, 4, Y, 0, None) == sn.ERR_ARG
    assert f(sn.Q4_K, C.c_void_p(4100), 16, 256, X, 4, Y, 0, None) == sn.ERR_ARG      # Q4_K: 16-byte weights
    assert b"alignment" in L.sinter_last_error()
    assert f(sn.Q6_K, W, 16, 256, C.c_void_p(8194), 4, Y, 0, None) == sn.ERR_ARG      # activations: 4 bytes
    assert f(sn.Q6_K, C.c_void_p(4098), 16, 256, X, 4, Y, 0, None) == sn.ERR_ARG      # Q6_K: 4-byte weights
    q = L.sinter_quant_q8k_ubatch
    assert q(X, 300, 4, Y, None) == sn.ERR_ARG
    assert b"multiple of 256" in L.sinter_last_error()
    assert q(X, 256, 0, Y, None) == sn.OK
    assert q(C.c_void_p(8196), 256, 4, Y, None) == sn.ERR_ARG                        # x: 16 bytes
    assert q(X, 256, 4, C.c_void_p(16386), None) == sn.ERR_ARG                       # xq: 4 bytes
    assert q(None, 256, 4, Y, None) == sn.ERR_ARG
    n = L.sinter_rmsnorm_quant_q8k_ubatch
    assert n(X, None, C.c_float(1e-6), 300, 4, Y, None) == sn.ERR_ARG
    assert n(X, None, C.c_float(1e-6), 256, 0, Y, None) == sn.OK
    assert n(X, C.c_void_p(8196), C.c_float(1e-6), 256, 4, Y, None) == sn.ERR_ARG   # w: 16 bytes
    assert n(X, None, C.c_float(-1.0), 256, 4, Y, None) == sn.ERR_ARG
    g = L.sinter_swiglu_quant_q8k_ubatch
    assert g(X, X, 300, 4, Y, None) == sn.ERR_ARG
    assert g(X, X, 256, 0, Y, None) == sn.OK
    assert g(X, C.c_void_p(8200), 256, 4, Y, None) == sn.ERR_ARG                     # up: 16 bytes
    gn = L.sinter_gated_rmsnorm_quant_q8k_ubatch
    assert gn(X, X, X, 128, C.c_float(1e-6), 300, 4, Y, None) == sn.ERR_ARG
    assert gn(X, X, X, 96, C.c_float(1e-6), 256, 4, Y, None) == sn.ERR_ARG          # head_dim: a power of two
    assert b"head_dim" in L.sinter_last_error()
    assert gn(X, X, X, 512, C.c_float(1e-6), 512, 4, Y, None) == sn.ERR_ARG
    assert gn(X, X, X, 128, C.c_float(1e-6), 256, 0, Y, None) == sn.OK
    cv = L.sinter_conv_silu_ubatch
    assert cv(X, X, X, Y, 64, 9, 4, None) == sn.ERR_ARG                              # dconv 1..8
    assert cv(X, X, X, Y, 0, 4, 4, None) == sn.ERR_ARG
    assert cv(X, X, X, Y, 64, 4, 0, None) == sn.OK
    assert cv(X, None, X, Y, 64, 4, 4, None) == sn.ERR_ARG


def test_model_config_validation(sn):
    L = sn.lib()
    cfg = sn.qwen36_27b_config()
    cfg.head_dim = 128               # attention op supports head_dim 256
    h = C.c_void_p()
    assert L.sinter_model_create(C.byref(cfg), 0, 1, 0, C.byref(h)) == sn.ERR_ARG


def test_host_synth_is_deterministic_and_scaled(sn, orc):
    L = sn.lib()
    for t, std in ((sn.Q4_K, 0.02), (sn.Q6_K, 0.02), (sn.Q8_0, 0.02), (sn.BF16, 0.02)):
        n = sn.row_bytes(t, 5120) * 64
        a = np.zeros(n, np.uint8)
        b = np.zeros(n, np.uint8)
        assert L.sinter_synth(0, a.ctypes.data, sn.SYN_WEIGHT, t, 64, 5120, 77, 0, 0, None) == 0
        assert L.sinter_synth(0, b.ctypes.data, sn.SYN_WEIGHT, t, 64, 5120, 77, 0, 0, None) == 0
        assert np.array_equal(a, b)
        rb = sn.row_bytes(t, 5120)
        vals = np.concatenate([orc.dequant(t, a[r * rb:(r + 1) * rb], 5120) for r in range(64)])
        assert abs(vals.mean()) < 0.15 * std and 0.6 * std < vals.std() < 1.6 * std, (t, vals.mean(), vals.std())
    x = np.zeros(100000, np.float32)
    assert L.sinter_synth(0, x.ctypes.data, sn.SYN_NORMAL, 0, 1, x.size, 5, 1.0, 0.5, None) == 0
    assert abs(x.mean() - 1.0) < 0.01 and abs(x.std() - 0.5) < 0.01
    assert L.sinter_synth(0, x.ctypes.data, sn.SYN_UNIFORM, 0, 1, x.size, 5, -2.0, 3.0, None) == 0
    assert x.min() >= -2.0 and x.max() < 3.0 and abs(x.mean() - 0.5) < 0.05
    s1 = L.sinter_seed(1, b"ffn_up", 3)
    assert s1 != L.sinter_seed(1, b"ffn_up", 4) and s1 != L.sinter_seed(1, b"ffn_gate", 3)
    assert s1 == L.sinter_seed(1, b"ffn_up", 3)


def test_q8_0_cache_synth_is_the_oracle_quantisation_of_the_normal_synth(sn, orc):
    """SYN_NORMAL_Q8_0 (the synthetic Q8_0 KV cache) = ggml's reference q8_0
    quantiser applied to the SYN_NORMAL values of the same seed."""
    L = sn.lib()
    rows, k = 13, 1024
    q = np.zeros(rows * k // 32 * 34, np.uint8)
    assert L.sinter_synth(0, q.ctypes.data, sn.SYN_NORMAL_Q8_0, 0, rows, k, 31, 0.0, 1.0, None) == 0
    x = np.zeros(rows * k, np.float32)
    assert L.sinter_synth(0, x.ctypes.data, sn.SYN_NORMAL, 0, 1, x.size, 31, 0.0, 1.0, None) == 0
    ref = np.zeros_like(q)
    orc.lib().or_quant_q8_0_ref(x.ctypes.data, ref.ctypes.data, x.size)
    assert np.array_equal(q, ref)
    assert L.sinter_synth(0, q.ctypes.data, sn.SYN_NORMAL_Q8_0, 0, 1, 100, 31, 0.0, 1.0, None) == sn.ERR_ARG


def test_cfg1_q8_0_synth_matches_config(sn, orc):
    """config 1: int8 codes uniform in [-127,127], f16 scale |N(0,0.02)|"""
    L = sn.lib()
    rows, k = 64, 5120
    w = np.zeros(sn.row_bytes(sn.Q8_0, k) * rows, np.uint8)
    assert L.sinter_synth(0, w.ctypes.data, sn.SYN_Q8_0_CFG1, sn.Q8_0, rows, k, 9, 0, 0, None) == 0
    blk = w.reshape(-1, 34)
    d = blk[:, :2].copy().view(np.float16)[:, 0].astype(np.float64)
    q = blk[:, 2:].view(np.int8).astype(np.int64)
    assert d.min() >= 0 and abs(d.mean() - 0.02 * np.sqrt(2 / np.pi)) < 0.002
    assert q.min() == -127 and q.max() == 127 and abs(q.mean()) < 0.5


def test_build_gate_enforces_the_spill_budget():
    """The resource gate fails a build whose persistent kernel spills more
    registers than its committed budget, or uses scratch; the committed
    build's own figures pass."""
    import sys
    sys.path.insert(0, os.path.join(ROOT, "sinter-qwen36-nomtp-tu102_amd"))
    import build
    base = {n: {"vgpr_spill": v, "sgpr_spill": s_, "scratch": 0, "lds": 1024, "occupancy": 1}
            for n, (v, s_) in build.SPILL_BUDGET.items()}
    for n in build.PERSISTENT:
        base.setdefault(n, {"vgpr_spill": 0, "sgpr_spill": 0, "scratch": 0, "lds": 1024, "occupancy": 1})
    assert build.gate(base) == []
    over = {n: dict(k) for n, k in base.items()}
    over["sinter_interp_kquant"]["sgpr_spill"] += 1
    assert any("over the budget" in b for b in build.gate(over))
    scratch = {n: dict(k) for n, k in base.items()}
    scratch["sinter_interp_bf16"]["scratch"] = 16
    assert any("scratch" in b for b in build.gate(scratch))
    # the committed build's report is within the budget
    rep = os.path.join(ROOT, "sinter-qwen36-nomtp-tu102_amd", "resource_usage.txt")
    if os.path.exists(rep):
        lines = open(rep).read().split("\n")
        cols = lines[0].split()[1:]
        figs = {}
        for ln in lines[1:]:
            if ln.strip():
                f = ln.split()
                figs[f[0]] = {c: int(v) if v.lstrip("-").isdigit() else v for c, v in zip(cols, f[1:])}
        for n, (vmax, smax) in build.SPILL_BUDGET.items():
            if n in figs:
                assert figs[n]["vgpr_spill"] <= vmax and figs[n]["sgpr_spill"] <= smax, n
