"""ctypes wrapper of the CPU oracle (liboracle.so) -- TEST INFRASTRUCTURE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this
module, and only as the checker or the timed CPU baseline.  The product path
(libsinter.so) never calls it.
"""
import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

F32, F16, Q8_0, Q4_K, Q6_K, Q8_K, BF16 = 0, 1, 8, 12, 14, 15, 30
NSLOT, NST = 16, 2


class Cfg(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("n_layer", "attn_every", "n_embd", "n_ff", "n_vocab", "gdn_hk",
                                         "gdn_hv", "gdn_d", "conv_k", "attn_nq", "attn_nkv", "head_dim",
                                         "rope_dims")] + \
               [("rope_base", C.c_float), ("eps", C.c_float), ("n_ctx", C.c_int32)] + \
               [(n, C.c_int32) for n in ("t_default", "t_attn_v", "t_ffn_down", "t_output", "t_embd", "t_kv",
                                         "attn_chunks", "attn_chunk_min")]


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        p, i, i64, f = C.c_void_p, C.c_int, C.c_int64, C.c_float
        sig = {
            "or_f16_to_f32": (f, [C.c_uint16]), "or_f32_to_f16": (C.c_uint16, [f]),
            "or_bf16_to_f32": (f, [C.c_uint16]), "or_f32_to_bf16": (C.c_uint16, [f]),
            "or_nearest_int": (i, [f]),
            "or_row_bytes": (C.c_size_t, [i, i64]),
            "or_dequant_row": (None, [i, p, p, i64]),
            "or_quant_q8_0": (None, [p, p, i64]), "or_quant_q8_K": (None, [p, p, i64]),
            "or_quant_q8_0_ref": (None, [p, p, i64]),
            "or_quant_bf16": (None, [p, p, i64]),
            "or_block_term": (C.c_double, [i, p, p]),
            "or_gemv": (None, [i, p, i64, i64, p, p]), "or_gemv_q": (None, [i, p, i64, i64, p, p]),
            "or_rmsnorm": (None, [p, p, p, i64, f]), "or_l2norm": (None, [p, p, i64, f]),
            "or_silu": (f, [f]), "or_sigmoid": (f, [f]), "or_softplus": (f, [f]),
            "or_conv_silu": (None, [p, p, p, p, i64, i]),
            "or_gdn_gates": (None, [p, p, p, p, p, p, i]),
            "or_gdn_step": (None, [p, p, p, p, p, p, p, i, i, i, f, i]),
            "or_gdn_cols": (i, [i]),
            "or_gated_rmsnorm": (None, [p, p, p, p, i, i, f]),
            "or_rope_theta_scale": (f, [f, i]), "or_rope_neox": (None, [p, i, i, i, f]),
            "or_attn_decode": (None, [p, p, p, i, i, i, i, i, f, p]),
            "or_attn_decode_kv": (None, [p, p, p, i, i, i, i, i, f, p]),
            "or_attn_split": (None, [p, p, p, i, i, i, i, i, f, i, i, p]),
            "or_attn_geom": (None, [i, i, i, C.POINTER(i), C.POINTER(i), C.POINTER(i)]),
            "or_is_attn_layer": (i, [C.POINTER(Cfg), i]),
            "or_gdn_mixer": (None, [C.POINTER(Cfg), p, p, p, p, p]),
            "or_row_isa": (i, []),
            "or_attn_mixer": (None, [C.POINTER(Cfg), p, p, p, i, p, p]),
            "or_ffn": (None, [C.POINTER(Cfg), p, p, p]),
            "or_decode_step": (i, [C.POINTER(Cfg), p, p, i, i, p, p]),
            "or_argmax_first": (i64, [p, i64]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def P(a):
    return None if a is None else a.ctypes.data


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def row_bytes(t, k):
    return lib().or_row_bytes(t, k)


def vec_dot_type(t):
    return {Q8_0: Q8_0, Q4_K: Q8_K, Q6_K: Q8_K, BF16: BF16, F32: F32}[t]


def quantize(t, x):
    """x (f32, len k) -> the vec_dot activation bytes of weight type t."""
    x = f32(x)
    vt = vec_dot_type(t)
    if vt == F32:
        return x.copy()
    out = np.zeros(row_bytes(vt, x.size) if vt != BF16 else x.size * 2, dtype=np.uint8)
    fn = {Q8_0: lib().or_quant_q8_0, Q8_K: lib().or_quant_q8_K, BF16: lib().or_quant_bf16}[vt]
    fn(P(x), P(out), x.size)
    return out


def gemv(t, w, rows, k, x):
    y = np.zeros(rows, dtype=np.float32)
    x = f32(x)
    lib().or_gemv(t, P(w), rows, k, P(x), P(y))
    return y


def dequant(t, row, k):
    out = np.zeros(k, dtype=np.float32)
    lib().or_dequant_row(t, P(row), P(out), k)
    return out


def rmsnorm(x, w, eps=1e-6):
    x = f32(x)
    y = np.zeros_like(x)
    lib().or_rmsnorm(P(x), P(f32(w)) if w is not None else None, P(y), x.size, eps)
    return y


def cfg_from(mc):
    """oracle Cfg from a sinter.ModelConfig (same field order)."""
    c = Cfg()
    for name, _ in Cfg._fields_:
        setattr(c, name, getattr(mc, name))
    return c


class ModelMirror:
    """Host copies of a sinter model's weights and state, in the oracle's
    slot layout, so or_decode_step can run the same pass on the CPU."""

    def __init__(self, model):
        import sinter  # the product binding, used here only to read device tensors back
        self.cfg = cfg_from(model.cfg)
        c = self.cfg
        self._keep = []
        ptrs = (C.c_void_p * (c.n_layer * NSLOT + 3))()
        for il in range(c.n_layer):
            for s in range(NSLOT):
                d, nb, _ = model.tensor(il, s)
                if d and nb:
                    a = np.empty(nb, dtype=np.uint8)
                    model.d2h(a, d, nb)
                    self._keep.append(a)
                    ptrs[il * NSLOT + s] = a.ctypes.data
        for s in range(3):
            d, nb, _ = model.tensor(c.n_layer, s)
            a = np.empty(nb, dtype=np.uint8)
            model.d2h(a, d, nb)
            self._keep.append(a)
            ptrs[c.n_layer * NSLOT + s] = a.ctypes.data
        self.weights = ptrs
        self.state_arrays = []
        st = (C.c_void_p * (c.n_layer * NST))()
        for il in range(c.n_layer):
            for s in range(NST):
                d, nb = model.state(il, s)
                a = np.empty(nb, dtype=np.uint8)
                model.d2h(a, d, nb)
                self.state_arrays.append(a)
                st[il * NST + s] = a.ctypes.data
        self.state = st
        del sinter

    def step(self, token, pos, resid=None):
        logits = np.zeros(self.cfg.n_vocab, dtype=np.float32)
        nxt = lib().or_decode_step(C.byref(self.cfg), self.weights, self.state, token, pos, P(logits), P(resid))
        return nxt, logits
