"""Q8_0 KV cache on the GPU: the attention op appends the new K / V rows as
ggml Q8_0 blocks (its f32 -> q8_0 block quantiser, restated by the oracle's
or_quant_q8_0_ref) and attends over the dequantised cache with the same fp64
arithmetic as the f16 cache; a model with a Q8_0 cache decodes like the CPU
oracle; and the Q8_0 cache's effect on the logits against the f16 cache is
measured and bounded (the same weights and prompt, prefilled on the GPU)."""
import ctypes as C

import numpy as np
import pytest

from test_gpu_model import compare_logits, small_config
from test_gpu_ops import dev, empty_f32, host, stream

pytestmark = pytest.mark.gpu

Q8_0, F16 = 8, 1


def q8_rows(orc, x):
    """rows of f32 -> rows of Q8_0 blocks (uint8), the oracle's quantiser"""
    rows, n = x.shape
    out = np.zeros((rows, n // 32 * 34), np.uint8)
    for r in range(rows):
        xr = np.ascontiguousarray(x[r], np.float32)
        orc.lib().or_quant_q8_0_ref(xr.ctypes.data, out[r].ctypes.data, n)
    return out


@pytest.mark.parametrize("pos,n_ctx,chunks,cmin", [(0, 64, 64, 0), (5, 4096, 64, 0), (1000, 4096, 64, 128),
                                                   (4095, 4096, 7, 0), (300, 4096, 1, 0), (2000, 4096, 9, 256),
                                                   (3000, 4096, 17, 0), (32767, 32768, 64, 128)])
def test_attn_decode_q8_cache_matches_oracle(sn, orc, torch_gpu, pos, n_ctx, chunks, cmin):
    torch = torch_gpu
    NQ, NKV, HD = 24, 4, 256
    RW = NKV * HD
    rng = np.random.default_rng(70 + pos)
    qg = (rng.standard_normal(NQ * 2 * HD) * 2).astype(np.float32)
    k = rng.standard_normal(RW).astype(np.float32)
    v = rng.standard_normal(RW).astype(np.float32)
    qn = (1 + 0.02 * rng.standard_normal(HD)).astype(np.float32)
    kn = (1 + 0.02 * rng.standard_normal(HD)).astype(np.float32)
    K = np.zeros((n_ctx, RW // 32 * 34), np.uint8)
    V = np.zeros_like(K)
    if pos:
        K[:pos] = q8_rows(orc, rng.standard_normal((pos, RW)).astype(np.float32))
        V[:pos] = q8_rows(orc, rng.standard_normal((pos, RW)).astype(np.float32))
    ts = orc.lib().or_rope_theta_scale(1e7, 64)
    dK, dV = dev(torch, K), dev(torch, V)
    dqg, dk, dv_, dqn, dkn = dev(torch, qg), dev(torch, k), dev(torch, v), dev(torch, qn), dev(torch, kn)
    part = torch.zeros(sn.lib().sinter_attn_part_len(NQ, NKV, HD, chunks), dtype=torch.float32, device="cuda")
    cnt = torch.zeros(sn.lib().sinter_attn_count_len(NKV, chunks), dtype=torch.int32, device="cuda")
    out = empty_f32(torch, NQ * HD)
    cell = dev(torch, np.array([0, pos, 0, 0], np.int32))
    a = sn.AttnArgs(nq=NQ, nkv=NKV, hd=HD, rope_dims=64, n_ctx=n_ctx, n_chunks=chunks, theta_scale=ts, eps=1e-6,
                    scale=0.0625, kv_type=Q8_0, chunk_min=cmin)
    a.qg, a.k, a.v, a.q_norm, a.k_norm = dqg.data_ptr(), dk.data_ptr(), dv_.data_ptr(), dqn.data_ptr(), dkn.data_ptr()
    a.kc, a.vc, a.part, a.count, a.out, a.pass_cell = (dK.data_ptr(), dV.data_ptr(), part.data_ptr(),
                                                       cnt.data_ptr(), out.data_ptr(), cell.data_ptr())
    print(f"attn_decode q8 cache pos={pos} n_ctx={n_ctx} chunks={chunks}", flush=True)
    sn.check(sn.lib().sinter_op_attn_decode(C.byref(a), 256, C.c_void_p(stream(torch))), "attn")
    torch.cuda.synchronize()
    assert sn.op_error()[0] == 0
    L = orc.lib()
    qr = np.zeros((NQ, HD), np.float32)
    for h in range(NQ):
        L.or_rmsnorm(qg[h * 2 * HD:].ctypes.data, qn.ctypes.data, qr[h].ctypes.data, HD, 1e-6)
        L.or_rope_neox(qr[h].ctypes.data, HD, 64, pos, ts)
    kr = np.zeros((NKV, HD), np.float32)
    for g in range(NKV):
        L.or_rmsnorm(k[g * HD:].ctypes.data, kn.ctypes.data, kr[g].ctypes.data, HD, 1e-6)
        L.or_rope_neox(kr[g].ctypes.data, HD, 64, pos, ts)
    # the appended rows are the oracle's quantisation of the roped k and raw v, byte for byte
    K[pos] = q8_rows(orc, kr.reshape(1, -1))[0]
    V[pos] = q8_rows(orc, v.reshape(1, -1))[0]
    assert np.array_equal(host(dK)[pos], K[pos])
    assert np.array_equal(host(dV)[pos], V[pos])
    att = np.zeros((NQ, HD), np.float32)
    L.or_attn_split(qr.ctypes.data, K.ctypes.data, V.ctypes.data, Q8_0, pos + 1, NQ, NKV, HD, 0.0625, chunks, cmin,
                    att.ctypes.data)
    gate = qg.reshape(NQ, 2, HD)[:, 1]
    sig = np.array([[L.or_sigmoid(float(gate[h, i])) for i in range(HD)] for h in range(NQ)], np.float32)
    ref = (att * sig).astype(np.float32)
    got = host(out).reshape(NQ, HD)
    assert np.array_equal(got, ref), (np.abs(got - ref).max(), np.mean(got == ref))
    # the pin: exact fp64 attention over the dequantised cache within rel L2 1e-5
    ex = np.zeros((NQ, HD), np.float32)
    L.or_attn_decode_kv(qr.ctypes.data, K.ctypes.data, V.ctypes.data, Q8_0, pos + 1, NQ, NKV, HD, 0.0625,
                        ex.ctypes.data)
    assert np.linalg.norm(got - ex * sig) <= 1e-5 * np.linalg.norm(ex * sig)


def test_device_q8_0_synth_equals_host(sn, torch_gpu):
    torch = torch_gpu
    rows, k = 37, 1024
    h = np.zeros(rows * k // 32 * 34, np.uint8)
    sn.check(sn.lib().sinter_synth(0, h.ctypes.data, sn.SYN_NORMAL_Q8_0, 0, rows, k, 99, 0.0, 1.0, None), "synth")
    d = torch.zeros(h.size, dtype=torch.uint8, device="cuda")
    sn.check(sn.lib().sinter_synth(1, C.c_void_p(d.data_ptr()), sn.SYN_NORMAL_Q8_0, 0, rows, k, 99, 0.0, 1.0,
                                   C.c_void_p(stream(torch))), "synth dev")
    torch.cuda.synchronize()
    assert np.array_equal(host(d), h)


def test_small_model_q8_cache_decode_matches_oracle(sn, orc, torch_gpu):
    cfg = small_config(sn, n_layer=4, n_ctx=512)
    cfg.t_kv = Q8_0
    m = sn.Model(cfg, seed=51)
    try:
        m.synth_context(60, seed=52)
        mirror = orc.ModelMirror(m)
        assert m.info()["kernel"] == "sinter_interp_kquant_q8kv"
        tok, pos = 9, 60
        for step in range(5):
            logits = np.zeros(cfg.n_vocab, np.float32)
            nxt = m.decode(tok, pos, logits)
            rtok, rlog = mirror.step(tok, pos)
            print(f"q8 cache step {step}: gpu {nxt} oracle {rtok}", flush=True)
            compare_logits(logits, rlog)
            assert nxt == rtok
            tok, pos = nxt, pos + 1
        # the caches the GPU wrote equal the oracle's, byte for byte
        for il in range(cfg.n_layer):
            if il % cfg.attn_every == cfg.attn_every - 1:
                for s in range(2):
                    d, nb = m.state(il, s)
                    got = np.empty(nb, np.uint8)
                    m.d2h(got, d, nb)
                    assert np.array_equal(got, mirror.state_arrays[il * 2 + s]), (il, s)
    finally:
        m.close()


def test_q8_cache_against_f16_cache(sn, torch_gpu):
    """The accuracy cost of the Q8_0 cache: the same weights and prompt, one
    model per cache type, prefilled on the GPU; the logits after the prompt
    and along 16 greedy steps of the f16 model (both fed the f16 model's
    tokens) are compared: relative L2, KL(f16 || q8) and top-1 agreement."""
    cfg = small_config(sn, n_layer=8, n_ctx=1024)
    prompt = [int(t) for t in np.random.default_rng(5).integers(0, cfg.n_vocab, 700)]
    models = {}
    try:
        for name, t in (("f16", F16), ("q8", Q8_0)):
            cfg.t_kv = t
            models[name] = sn.Model(cfg, seed=61)
        nxt = {n: m.prefill(prompt, 0) for n, m in models.items()}
        rels, kls, agree = [], [], 0
        t = nxt["f16"]
        for i in range(17):
            if i:   # both models take the f16 model's greedy token
                outs = {n: m.decode(t, len(prompt) + i - 1) for n, m in models.items()}
                t = outs["f16"]
            a, b = (models[n].logits().astype(np.float64) for n in ("f16", "q8"))
            rels.append(np.linalg.norm(a - b) / np.linalg.norm(a))
            pa, pb = np.exp(a - a.max()), np.exp(b - b.max())
            pa, pb = pa / pa.sum(), pb / pb.sum()
            kls.append(float(np.sum(pa * (np.log(pa + 1e-300) - np.log(pb + 1e-300)))))
            agree += int(np.argmax(a) == np.argmax(b))
        print(f"q8 vs f16 cache over {len(rels)} positions: rel L2 max {max(rels):.3e} mean {np.mean(rels):.3e}; "
              f"KL max {max(kls):.3e} mean {np.mean(kls):.3e}; top-1 agreement {agree}/{len(rels)}", flush=True)
        assert max(rels) < 0.05 and max(kls) < 0.01 and agree >= len(rels) - 1
    finally:
        for m in models.values():
            m.close()
