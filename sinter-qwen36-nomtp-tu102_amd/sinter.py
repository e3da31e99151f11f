"""ctypes binding of libsinter.so (include/sinter.h).

Host-side mirror of the C ABI for tests, smoke() and bench.py.  The HIP
library is the product: loading fails loudly when libsinter.so is missing,
and nothing here falls back to a CPU path.
"""
import ctypes as C
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libsinter.so")

# sinter_type
F32, F16, Q8_0, Q4_K, Q6_K, Q8_K, BF16 = 0, 1, 8, 12, 14, 15, 30
ATTN_CHUNK_MIN = 128   # SINTER_ATTN_CHUNK_MIN: default positions per split-K attention chunk
PREFILL_UBATCH = 256   # SINTER_PREFILL_UBATCH: tokens per ubatch of the batched prefill
# ops
OP_NOP, OP_BOUNDARY, OP_GEMV, OP_GDN_STEP, OP_ATTN_DECODE, OP_KIND_COUNT = range(6)
BENCH_GEMV, BENCH_GDN, BENCH_ATTN = 1, 2, 3
PRO_PLAIN, PRO_RMSNORM, PRO_GATED, PRO_EMBED, PRO_GATED_G = range(5)
EPI_STORE, EPI_RESID, EPI_SWIGLU, EPI_ARGMAX, EPI_CONV, EPI_SILU = range(6)
SYN_WEIGHT, SYN_Q8_0_CFG1, SYN_NORMAL, SYN_UNIFORM, SYN_NORMAL_F16, SYN_NORMAL_Q8_0 = range(6)
OK, ERR_ARG, ERR_HIP, ERR_DEVICE, ERR_TIMEOUT, ERR_STATE, ERR_NOMEM = 0, -1, -2, -3, -4, -5, -6
RUN_OK, RUN_ERR, RUN_TIMEOUT = 0, 1, 2
E_NONE, E_BAD_KIND, E_UNWIRED_KIND, E_BAD_SHAPE, E_TIMEOUT_BARRIER = 0, 1, 2, 3, 5

BLOCK_BYTES = {F32: 4, F16: 2, BF16: 2, Q8_0: 34, Q4_K: 144, Q6_K: 210, Q8_K: 292}
BLOCK_ELEMS = {F32: 1, F16: 1, BF16: 1, Q8_0: 32, Q4_K: 256, Q6_K: 256, Q8_K: 256}


def row_bytes(t, k):
    return (k // BLOCK_ELEMS[t]) * BLOCK_BYTES[t]


vp = C.c_void_p


class Instr(C.Structure):
    _fields_ = [("kind", C.c_uint16), ("block_lo", C.c_uint16), ("block_hi", C.c_uint16),
                ("flags", C.c_uint16), ("dbg_node", C.c_uint32), ("_pad", C.c_uint32),
                ("payload", C.c_ubyte * 240)]


class GemvSeg(C.Structure):
    _fields_ = [("w", vp), ("w2", vp), ("y", vp), ("aux", vp), ("rows", C.c_uint32),
                ("type", C.c_uint8), ("epi", C.c_uint8), ("dconv", C.c_uint8), ("_pad", C.c_uint8)]


class GemvArgs(C.Structure):
    _fields_ = [("x", vp), ("norm_w", vp), ("aux", vp), ("token", vp), ("x_out", vp), ("epi_ws", vp),
                ("K", C.c_uint32), ("eps", C.c_float), ("pro", C.c_uint8), ("n_seg", C.c_uint8),
                ("aux_type", C.c_uint8), ("gn_log2d", C.c_uint8), ("aux_rows", C.c_uint32),
                ("seg", GemvSeg * 4)]


class GdnArgs(C.Structure):
    _fields_ = [("qkv", vp), ("alpha", vp), ("beta", vp), ("dt_bias", vp), ("ssm_a", vp), ("state", vp),
                ("o", vp), ("hk", C.c_uint32), ("hv", C.c_uint32), ("d", C.c_uint32), ("cols", C.c_uint32),
                ("eps", C.c_float), ("scale", C.c_float)]


class AttnArgs(C.Structure):
    _fields_ = [("qg", vp), ("k", vp), ("v", vp), ("q_norm", vp), ("k_norm", vp), ("kc", vp), ("vc", vp),
                ("part", vp), ("count", vp), ("out", vp), ("pass_cell", vp),
                ("nq", C.c_uint32), ("nkv", C.c_uint32), ("hd", C.c_uint32), ("rope_dims", C.c_uint32),
                ("n_ctx", C.c_uint32), ("n_chunks", C.c_uint32), ("theta_scale", C.c_float),
                ("eps", C.c_float), ("scale", C.c_float), ("kv_type", C.c_uint32), ("chunk_min", C.c_uint32)]


class ModelBindings(C.Structure):
    _fields_ = [("tensors", C.POINTER(vp)), ("types", C.POINTER(C.c_int32)), ("states", C.POINTER(vp)),
                ("logits", vp), ("embed_outside", C.c_uint32), ("_pad", C.c_uint32)]


class GgufTensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("type", C.c_uint32), ("n_dims", C.c_uint32), ("ne", C.c_uint64 * 4),
                ("offset", C.c_uint64), ("nbytes", C.c_uint64), ("data", vp)]


class PassCell(C.Structure):
    _fields_ = [("token", C.c_int32), ("pos", C.c_int32), ("steps", C.c_int32), ("_pad", C.c_int32)]


class ModelConfig(C.Structure):
    _fields_ = [("n_layer", C.c_int32), ("attn_every", C.c_int32), ("n_embd", C.c_int32), ("n_ff", C.c_int32),
                ("n_vocab", C.c_int32), ("gdn_hk", C.c_int32), ("gdn_hv", C.c_int32), ("gdn_d", C.c_int32),
                ("conv_k", C.c_int32), ("attn_nq", C.c_int32), ("attn_nkv", C.c_int32),
                ("head_dim", C.c_int32), ("rope_dims", C.c_int32), ("rope_base", C.c_float),
                ("eps", C.c_float), ("n_ctx", C.c_int32), ("t_default", C.c_int32), ("t_attn_v", C.c_int32),
                ("t_ffn_down", C.c_int32), ("t_output", C.c_int32), ("t_embd", C.c_int32), ("t_kv", C.c_int32),
                ("attn_chunks", C.c_int32), ("attn_chunk_min", C.c_int32)]


assert C.sizeof(Instr) == 256 and C.sizeof(GemvSeg) == 40
assert C.sizeof(GemvArgs) == 224 and C.sizeof(GdnArgs) == 80 and C.sizeof(AttnArgs) == 136


def qwen36_27b_config(n_ctx=4352, quant="q4_k_m", n_layer=64, kv="f16"):
    """The 27B-shaped hybrid: 48 gated-DeltaNet + 16 attention layers; KV
    cache f16 or q8_0."""
    tkv = {"f16": F16, "q8_0": Q8_0}[kv]
    if quant == "q4_k_m":
        td, tv, tdown, tout, temb = Q4_K, Q6_K, Q6_K, Q6_K, Q4_K
    elif quant == "bf16":
        td = tv = tdown = tout = temb = BF16
    else:
        raise ValueError(quant)
    return ModelConfig(n_layer=n_layer, attn_every=4, n_embd=5120, n_ff=17408, n_vocab=151936,
                       gdn_hk=16, gdn_hv=32, gdn_d=128, conv_k=4, attn_nq=24, attn_nkv=4, head_dim=256,
                       rope_dims=64, rope_base=1e7, eps=1e-6, n_ctx=n_ctx, t_default=td, t_attn_v=tv,
                       t_ffn_down=tdown, t_output=tout, t_embd=temb, t_kv=tkv)


_lib = None


_system_runtime = False


def use_system_runtime():
    """Make this process load libsinter on the system ROCm runtime (the one
    the image's tools, rocprofv3 among them, belong to) instead of torch's
    bundled copy.  Call it before the first lib() in a process that will not
    import torch: once the system libamdhip64.so.7 is loaded, torch imported
    later would bind to it and not run."""
    global _system_runtime
    if _lib is not None or "torch" in sys.modules:
        raise RuntimeError("use_system_runtime() must come before lib() and before any torch import")
    _system_runtime = True


def lib():
    """Load libsinter.so; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError("libsinter.so is not built (run __graft_entry__.build()); "
                           "there is no CPU fallback")
    # One HIP runtime per process: torch ships its own libamdhip64.so.7, and
    # whichever copy is loaded first satisfies the other's dependency.  torch
    # does not run on the system copy, while libsinter runs on either, so
    # unless the process chose the system runtime (use_system_runtime), let
    # torch (when installed) load its runtime first.
    if not _system_runtime:
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
    L = C.CDLL(LIB_PATH)
    I, U32, I64, U64 = C.c_int, C.c_uint32, C.c_int64, C.c_uint64
    sig = {
        "sinter_last_error": (C.c_char_p, []),
        "sinter_abi_version": (I, []),
        "sinter_device_info": (I, [I, C.c_char_p, C.c_size_t]),
        "sinter_row_bytes": (C.c_size_t, [I, I64]),
        "sinter_attn_part_len": (C.c_size_t, [U32, U32, U32, U32]),
        "sinter_attn_count_len": (U32, [U32, U32]),
        "sinter_op_gemv": (I, [C.POINTER(GemvArgs), U32, vp]),
        "sinter_op_gdn_step": (I, [C.POINTER(GdnArgs), U32, vp]),
        "sinter_op_attn_decode": (I, [C.POINTER(AttnArgs), U32, vp]),
        "sinter_op_gemv_ubatch": (I, [I, vp, I64, I64, vp, U32, vp, I, vp]),
        "sinter_quant_q8k_ubatch": (I, [vp, I64, U32, vp, vp]),
        "sinter_rmsnorm_quant_q8k_ubatch": (I, [vp, vp, C.c_float, I64, U32, vp, vp]),
        "sinter_swiglu_quant_q8k_ubatch": (I, [vp, vp, I64, U32, vp, vp]),
        "sinter_gated_rmsnorm_quant_q8k_ubatch": (I, [vp, vp, vp, U32, C.c_float, I64, U32, vp, vp]),
        "sinter_conv_silu_ubatch": (I, [vp, vp, vp, vp, I64, U32, U32, vp]),
        "sinter_op_attn_decode_noalloc": (I, [C.POINTER(AttnArgs), U32, vp]),
        "sinter_litmus_barrier": (I, [U32, U32, I, C.POINTER(C.c_uint64)]),
        "sinter_copy_calibration": (I, [I, C.c_size_t, I]),
        "sinter_hbm_peak": (I, [C.c_uint64, U32, C.POINTER(C.c_double), C.POINTER(C.c_double)]),
        "sinter_op_error": (I, [C.POINTER(U32), C.POINTER(U32)]),
        "sinter_argmax_ws_create": (I, [U32, vp, vp, U32, C.POINTER(vp)]),
        "sinter_argmax_ws_destroy": (None, [vp]),
        "sinter_synth": (I, [I, vp, I, I, I64, I64, U64, C.c_float, C.c_float, vp]),
        "sinter_seed": (U64, [U64, C.c_char_p, I64]),
        "sinter_host_init": (I, [C.POINTER(vp), I, C.c_uint]),
        "sinter_host_upload": (I, [vp, C.POINTER(Instr), U32, U32]),
        "sinter_host_launch": (I, [vp]),
        "sinter_host_run_pass": (I, [vp, C.c_int32, C.c_double]),
        "sinter_host_run_passes": (I, [vp, C.c_int32, U32, C.POINTER(C.c_int32), C.c_double]),
        "sinter_host_shutdown": (I, [vp, C.c_double]),
        "sinter_host_destroy": (None, [vp]),
        "sinter_host_read_pass_cycles": (I, [vp, C.POINTER(C.c_longlong), C.c_uint]),
        "sinter_host_reset_op_cycles": (I, [vp]),
        "sinter_host_read_op_cycles": (I, [vp, C.POINTER(C.c_longlong), C.c_uint]),
        "sinter_host_trace_next": (I, [vp, vp, C.c_size_t]),
        "sinter_host_pass_cell": (vp, [vp]),
        "sinter_host_history": (vp, [vp, C.POINTER(U32)]),
        "sinter_host_error": (I, [vp, C.POINTER(U32), C.POINTER(U32)]),
        "sinter_host_grid": (I, [vp, C.POINTER(U32), C.POINTER(U32), C.POINTER(U32)]),
        "sinter_host_kernel": (C.c_char_p, [vp]),
        "sinter_host_set_pos": (I, [vp, C.c_int32]),
        "sinter_host_set_grid": (I, [vp, U32]),
        "sinter_host_set_gemv_shares": (I, [vp, U32, C.POINTER(C.c_float), U32]),
        "sinter_host_last_launch_ms": (C.c_float, [vp]),
        "sinter_model_create": (I, [C.POINTER(ModelConfig), I, U64, U32, C.POINTER(vp)]),
        "sinter_model_destroy": (None, [vp]),
        "sinter_model_decode": (I, [vp, C.c_int32, C.c_int32, vp, C.POINTER(C.c_int32)]),
        "sinter_model_greedy": (I, [vp, C.c_int32, C.c_int32, U32, C.POINTER(C.c_int32)]),
        "sinter_model_prefill": (I, [vp, C.POINTER(C.c_int32), U32, C.c_int32, C.POINTER(C.c_int32)]),
        "sinter_model_prefill_tokenwise": (I, [vp, C.POINTER(C.c_int32), U32, C.c_int32, C.POINTER(C.c_int32)]),
        "sinter_model_prefill_batched": (I, [vp, C.POINTER(C.c_int32), U32, C.c_int32, U32,
                                             C.POINTER(C.c_int32)]),
        "sinter_model_create_bound": (I, [C.POINTER(ModelConfig), I, U32, C.POINTER(ModelBindings), C.POINTER(vp)]),
        "sinter_model_synth_context": (I, [vp, C.c_int32, U64]),
        "sinter_model_logits": (I, [vp, vp]),
        "sinter_model_tensor_info": (I, [vp, I64, I, C.POINTER(vp), C.POINTER(C.c_size_t), C.POINTER(I)]),
        "sinter_model_state_info": (I, [vp, I64, I, C.POINTER(vp), C.POINTER(C.c_size_t)]),
        "sinter_model_copy": (I, [vp, vp, vp, C.c_size_t, I]),
        "sinter_model_info": (I, [vp, C.POINTER(U64), C.POINTER(U32), C.POINTER(U32), C.POINTER(U32)]),
        "sinter_model_host": (vp, [vp]),
        "sinter_model_bench_program": (I, [vp, I, C.c_uint64]),
        "sinter_model_buffer": (I, [vp, C.c_char_p, C.POINTER(vp), C.POINTER(C.c_size_t)]),
        "sinter_model_program": (I, [vp, vp, U32, C.POINTER(U32)]),
        "sinter_model_balance": (I, [vp, C.POINTER(C.c_int32), C.POINTER(C.c_int32), U32, U32]),
        "sinter_model_get_config": (I, [vp, C.POINTER(ModelConfig)]),
        "sinter_gguf_open": (I, [C.c_char_p, C.POINTER(vp)]),
        "sinter_gguf_close": (None, [vp]),
        "sinter_gguf_info": (I, [vp, C.POINTER(U32), C.POINTER(U64), C.POINTER(U64), C.POINTER(U64)]),
        "sinter_gguf_get_tensor": (I, [vp, U64, C.POINTER(GgufTensor)]),
        "sinter_gguf_find": (I64, [vp, C.c_char_p]),
        "sinter_gguf_kv_i64": (I, [vp, C.c_char_p, C.POINTER(I64)]),
        "sinter_gguf_kv_f64": (I, [vp, C.c_char_p, C.POINTER(C.c_double)]),
        "sinter_gguf_kv_str": (I, [vp, C.c_char_p, C.c_char_p, C.c_size_t]),
        "sinter_gguf_kv_arr_i64": (I, [vp, C.c_char_p, C.POINTER(I64), C.c_size_t, C.POINTER(C.c_size_t)]),
        "sinter_model_config_from_gguf": (I, [vp, C.c_int32, C.POINTER(ModelConfig)]),
        "sinter_model_create_from_gguf": (I, [vp, I, C.c_int32, U32, C.POINTER(vp)]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    _lib = L
    return L


class SinterError(RuntimeError):
    pass


def check(rc, what=""):
    if rc != 0:
        msg = lib().sinter_last_error()
        raise SinterError(f"{what}: status {rc}: {msg.decode() if msg else ''}")
    return rc


def device_info(device=0):
    buf = C.create_string_buffer(1024)
    rc = lib().sinter_device_info(device, buf, 1024)
    return rc, buf.value.decode()


def op_error():
    code, aux = C.c_uint32(0), C.c_uint32(0)
    check(lib().sinter_op_error(C.byref(code), C.byref(aux)), "op_error")
    return code.value, aux.value


class Gguf:
    """A read-only GGUF file (sinter_gguf_*)."""

    def __init__(self, path):
        h = vp()
        check(lib().sinter_gguf_open(path.encode(), C.byref(h)), "gguf_open")
        self.h = h

    def close(self):
        if self.h:
            lib().sinter_gguf_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def info(self):
        v, nt, nk, al = C.c_uint32(), C.c_uint64(), C.c_uint64(), C.c_uint64()
        check(lib().sinter_gguf_info(self.h, C.byref(v), C.byref(nt), C.byref(nk), C.byref(al)), "gguf_info")
        return {"version": v.value, "n_tensors": nt.value, "n_kv": nk.value, "alignment": al.value}

    def tensor(self, i):
        t = GgufTensor()
        check(lib().sinter_gguf_get_tensor(self.h, i, C.byref(t)), "gguf_tensor")
        return t

    def find(self, name):
        return lib().sinter_gguf_find(self.h, name.encode())

    def kv_i64(self, key):
        v = C.c_int64()
        check(lib().sinter_gguf_kv_i64(self.h, key.encode(), C.byref(v)), "gguf_kv_i64")
        return v.value

    def kv_f64(self, key):
        v = C.c_double()
        check(lib().sinter_gguf_kv_f64(self.h, key.encode(), C.byref(v)), "gguf_kv_f64")
        return v.value

    def kv_str(self, key):
        buf = C.create_string_buffer(4096)
        check(lib().sinter_gguf_kv_str(self.h, key.encode(), buf, 4096), "gguf_kv_str")
        return buf.value.decode()

    def kv_arr_i64(self, key):
        n = C.c_size_t()
        check(lib().sinter_gguf_kv_arr_i64(self.h, key.encode(), None, 0, C.byref(n)), "gguf_kv_arr")
        out = (C.c_int64 * max(1, n.value))()
        check(lib().sinter_gguf_kv_arr_i64(self.h, key.encode(), out, n.value, C.byref(n)), "gguf_kv_arr")
        return list(out)[:n.value]

    def config(self, n_ctx):
        c = ModelConfig()
        check(lib().sinter_model_config_from_gguf(self.h, n_ctx, C.byref(c)), "config_from_gguf")
        return c


class Model:
    """Owner of a sinter_model handle."""

    def __init__(self, cfg, seed=1, device=0, blocks=0, gguf=None, bindings=None):
        """bindings: (tensors, types, states, logits, embed_outside) -- device
        pointers the model runs over without owning them (sinter_model_bindings)."""
        h = vp()
        if bindings is not None:
            tensors, types, states, logits, embed_outside = bindings
            self._bind = (
                (vp * len(tensors))(*tensors), (C.c_int32 * len(types))(*types), (vp * len(states))(*states))
            b = ModelBindings(tensors=self._bind[0], types=self._bind[1], states=self._bind[2], logits=logits,
                              embed_outside=1 if embed_outside else 0)
            check(lib().sinter_model_create_bound(C.byref(cfg), device, blocks, C.byref(b), C.byref(h)),
                  "model_create_bound")
        elif gguf is not None:
            check(lib().sinter_model_create_from_gguf(gguf.h, device, cfg.n_ctx, blocks, C.byref(h)),
                  "model_create_from_gguf")
            cfg = ModelConfig()
            check(lib().sinter_model_get_config(h, C.byref(cfg)), "get_config")
        else:
            check(lib().sinter_model_create(C.byref(cfg), device, seed, blocks, C.byref(h)), "model_create")
        # the configuration as the model resolved it (defaults filled in)
        cfg = ModelConfig()
        check(lib().sinter_model_get_config(h, C.byref(cfg)), "get_config")
        self.cfg = cfg
        self.h = h

    def close(self):
        if self.h:
            lib().sinter_model_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def info(self):
        wb, ni, nb, bl = C.c_uint64(), C.c_uint32(), C.c_uint32(), C.c_uint32()
        check(lib().sinter_model_info(self.h, C.byref(wb), C.byref(ni), C.byref(nb), C.byref(bl)), "info")
        k = lib().sinter_host_kernel(self.host())
        return {"weight_bytes": wb.value, "n_instr": ni.value, "n_boundaries": nb.value, "blocks": bl.value,
                "kernel": k.decode() if k else None}

    def synth_context(self, n_past, seed):
        check(lib().sinter_model_synth_context(self.h, n_past, seed), "synth_context")

    def decode(self, token, pos, logits=None):
        nt = C.c_int32()
        ptr = logits.ctypes.data if logits is not None else None
        check(lib().sinter_model_decode(self.h, token, pos, ptr, C.byref(nt)), "decode")
        return nt.value

    def greedy(self, token, pos, n):
        out = (C.c_int32 * n)()
        check(lib().sinter_model_greedy(self.h, token, pos, n, out), "greedy")
        return list(out)

    def prefill(self, tokens, pos0=0, mode="auto", ubatch=PREFILL_UBATCH):
        """Prefill tokens at positions pos0.. on the GPU; returns the greedy
        next token.  mode "auto": batched when the model's matrices allow it,
        else the decode passes; "batched" (ubatches of `ubatch` tokens) or
        "tokenwise" (the decode passes with the prompt's tokens forced)."""
        arr = (C.c_int32 * len(tokens))(*tokens)
        nxt = C.c_int32()
        if mode == "auto":
            rc = lib().sinter_model_prefill(self.h, arr, len(tokens), pos0, C.byref(nxt))
        elif mode == "batched":
            rc = lib().sinter_model_prefill_batched(self.h, arr, len(tokens), pos0, ubatch, C.byref(nxt))
        elif mode == "tokenwise":
            rc = lib().sinter_model_prefill_tokenwise(self.h, arr, len(tokens), pos0, C.byref(nxt))
        else:
            raise ValueError(f"prefill mode {mode!r}")
        check(rc, "prefill")
        return nxt.value

    def logits(self, out=None):
        """Logits of the last decoded pass (float32[n_vocab])."""
        import numpy as np
        if out is None:
            out = np.zeros(self.cfg.n_vocab, np.float32)
        check(lib().sinter_model_logits(self.h, out.ctypes.data), "logits")
        return out

    def tensor(self, layer, slot):
        p, nb, t = vp(), C.c_size_t(), C.c_int()
        check(lib().sinter_model_tensor_info(self.h, layer, slot, C.byref(p), C.byref(nb), C.byref(t)), "tensor")
        return p.value, nb.value, t.value

    def state(self, layer, slot):
        p, nb = vp(), C.c_size_t()
        check(lib().sinter_model_state_info(self.h, layer, slot, C.byref(p), C.byref(nb)), "state")
        return p.value, nb.value

    def d2h(self, dst_np, src_dev, nbytes):
        check(lib().sinter_model_copy(self.h, dst_np.ctypes.data, src_dev, nbytes, 0), "copy d2h")

    def h2d(self, dst_dev, src_np, nbytes):
        check(lib().sinter_model_copy(self.h, dst_dev, src_np.ctypes.data, nbytes, 1), "copy h2d")

    def host(self):
        return lib().sinter_model_host(self.h)

    def buffer(self, name):
        """(device pointer, bytes) of one of the model's own buffers (X, H, logits, ...)."""
        p, nb = vp(), C.c_size_t()
        check(lib().sinter_model_buffer(self.h, name.encode(), C.byref(p), C.byref(nb)), "buffer " + name)
        return p.value, nb.value

    def program(self):
        """A copy of the model's uploaded program (sinter_instr records)."""
        n = C.c_uint32()
        check(lib().sinter_model_program(self.h, None, 0, C.byref(n)), "program")
        out = (Instr * n.value)()
        check(lib().sinter_model_program(self.h, out, n.value, C.byref(n)), "program")
        return out

    def upload_program(self, instrs):
        """Replace the model's program with packed instructions (e.g. from
        schedule.pack): the host is stopped, the program uploaded (one barrier
        epoch per BOUNDARY plus the pass end) and launched again."""
        h, L = self.host(), lib()
        nb = sum(1 for i in instrs if i.kind == OP_BOUNDARY) + 1
        check(L.sinter_host_shutdown(h, 60000.0), "shutdown")
        check(L.sinter_host_upload(h, instrs, len(instrs), nb), "upload")
        check(L.sinter_host_launch(h), "launch")

    def bench_program(self, kind, seed=1):
        """Replace the decode program with a single-op benchmark program
        (BENCH_GEMV / BENCH_GDN / BENCH_ATTN; sinter_model_bench_program)."""
        check(lib().sinter_model_bench_program(self.h, kind, seed), "bench_program")

    def time_passes(self, pos, n):
        """Run n passes of the uploaded program in one launch at position
        pos; returns the interpreter kernel's time in ms (HIP events)."""
        h, L = self.host(), lib()
        check(L.sinter_host_set_pos(h, pos), "set_pos")
        out = (C.c_int32 * n)()
        rs = L.sinter_host_run_passes(h, 0, n, out, 600000.0)
        if rs != RUN_OK:
            raise SinterError(f"run_passes: status {rs}: {L.sinter_last_error().decode()}")
        return float(L.sinter_host_last_launch_ms(h))

    def balance(self, token, pos, rounds=2, traces=4):
        """Static GEMV load balance (sinter_model_balance): decodes
        rounds*traces greedy tokens from (token, pos); returns the next
        (token, pos)."""
        t, p = C.c_int32(token), C.c_int32(pos)
        check(lib().sinter_model_balance(self.h, C.byref(t), C.byref(p), rounds, traces), "balance")
        return t.value, p.value
