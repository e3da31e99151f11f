"""A model over caller-owned device memory (sinter_model_create_bound) -- the
path a host framework takes with its own weight, KV-cache and recurrent-state
tensors: bound to byte copies of a model's weights and state it decodes
exactly like that model, with the embedding done inside the pass or by the
caller; bad bindings are refused before anything runs."""
import ctypes as C

import numpy as np
import pytest

from test_gpu_model import small_config

pytestmark = pytest.mark.gpu


def clone(sn, torch, m, keep):
    """device copies of m's weights and states: (tensor ptrs, types, state ptrs)"""
    cfg = m.cfg
    n = cfg.n_layer * 16 + 3
    ptrs, types = [None] * n, [0] * n
    for i in range(n):
        il, s = (i // 16, i % 16) if i < cfg.n_layer * 16 else (cfg.n_layer, i - cfg.n_layer * 16)
        d, nb, t = m.tensor(il, s)
        types[i] = t
        if d and nb:
            buf = torch.empty(nb + 256, dtype=torch.uint8, device="cuda")
            sn.check(sn.lib().sinter_model_copy(m.h, C.c_void_p(buf.data_ptr()), C.c_void_p(d), nb, 2), "copy")
            keep.append(buf)
            ptrs[i] = buf.data_ptr()
    states = []
    for il in range(cfg.n_layer):
        for s in range(2):
            d, nb = m.state(il, s)
            buf = torch.empty(nb + 256, dtype=torch.uint8, device="cuda")
            sn.check(sn.lib().sinter_model_copy(m.h, C.c_void_p(buf.data_ptr()), C.c_void_p(d), nb, 2), "copy")
            keep.append(buf)
            states.append(buf.data_ptr())
    torch.cuda.synchronize()
    return ptrs, types, states


def test_bound_model_decodes_like_its_source(sn, torch_gpu):
    torch = torch_gpu
    cfg = small_config(sn, n_layer=8, n_ctx=256)
    a = sn.Model(cfg, seed=81)
    keep = []
    try:
        a.synth_context(50, seed=82)
        ptrs, types, states = clone(sn, torch, a, keep)
        logits = torch.zeros(cfg.n_vocab, dtype=torch.float32, device="cuda")
        print("bound model: create over cloned weights and state", flush=True)
        b = sn.Model(cfg, bindings=(ptrs, types, states, logits.data_ptr(), False))
        try:
            assert b.info()["weight_bytes"] == a.info()["weight_bytes"]
            ta, tb = a.greedy(7, 50, 12), b.greedy(7, 50, 12)
            assert ta == tb
            la, lb = np.zeros(cfg.n_vocab, np.float32), np.zeros(cfg.n_vocab, np.float32)
            assert a.decode(ta[-1], 62, la) == b.decode(tb[-1], 62, lb)
            assert np.array_equal(la, lb)
            assert np.array_equal(logits.cpu().numpy(), lb)     # the head wrote the caller's buffer
            # the KV and recurrent state live in the caller's buffers
            for il in range(cfg.n_layer):
                for s in range(2):
                    d, nb = a.state(il, s)
                    ga = np.empty(nb, np.uint8)
                    a.d2h(ga, d, nb)
                    hb = np.empty(nb, np.uint8)
                    b.d2h(hb, states[il * 2 + s], nb)
                    assert np.array_equal(ga, hb), (il, s)
        finally:
            b.close()
    finally:
        a.close()


def test_bound_model_with_the_embedding_outside(sn, orc, torch_gpu):
    torch = torch_gpu
    cfg = small_config(sn, n_layer=4, n_ctx=128)
    a = sn.Model(cfg, seed=83)
    keep = []
    try:
        a.synth_context(20, seed=84)
        ptrs, types, states = clone(sn, torch, a, keep)
        d, nb, et = a.tensor(cfg.n_layer, 0)
        emb = np.empty(nb, np.uint8)
        a.d2h(emb, d, nb)
        rb = nb // cfg.n_vocab
        ptrs[cfg.n_layer * 16] = None                  # no embedding table on the bound side
        b = sn.Model(cfg, bindings=(ptrs, types, states, None, True))
        try:
            x_ptr, x_bytes = b.buffer("X")
            assert x_bytes >= cfg.n_embd * 4
            tok = 11
            for pos in range(20, 24):
                la, lb = np.zeros(cfg.n_vocab, np.float32), np.zeros(cfg.n_vocab, np.float32)
                row = orc.dequant(et, emb[tok * rb:(tok + 1) * rb], cfg.n_embd)
                b.h2d(x_ptr, row, cfg.n_embd * 4)
                nb_ = b.decode(tok, pos, lb)
                na_ = a.decode(tok, pos, la)
                assert na_ == nb_ and np.array_equal(la, lb), pos
                tok = na_
            # several passes per call need the embedding inside the pass
            assert sn.lib().sinter_model_greedy(b.h, tok, 24, 2, None) == sn.ERR_STATE
        finally:
            b.close()
    finally:
        a.close()


def test_bound_model_refuses_bad_bindings(sn, torch_gpu):
    torch = torch_gpu
    cfg = small_config(sn, n_layer=4, n_ctx=64)
    a = sn.Model(cfg, seed=85)
    keep = []
    try:
        ptrs, types, states = clone(sn, torch, a, keep)
        L = sn.lib()
        for bad in ("null weight", "unaligned", "bad type", "null state"):
            p, t, st = list(ptrs), list(types), list(states)
            if bad == "null weight":
                p[2] = None
            elif bad == "unaligned":
                p[2] = p[2] + 4
            elif bad == "bad type":
                t[2] = 99
            else:
                st[3] = None
            arr = ((C.c_void_p * len(p))(*p), (C.c_int32 * len(t))(*t), (C.c_void_p * len(st))(*st))
            bnd = sn.ModelBindings(tensors=arr[0], types=arr[1], states=arr[2], logits=None, embed_outside=0)
            h = C.c_void_p()
            assert L.sinter_model_create_bound(C.byref(cfg), 0, 0, C.byref(bnd), C.byref(h)) == sn.ERR_ARG, bad
            assert not h.value
    finally:
        a.close()
