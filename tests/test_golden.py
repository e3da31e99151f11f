"""The committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_golden.py from the CPU oracle) against the oracle today and
against independent float64 restatements (tests/refimpl.py), CPU only.

A change to oracle/oracle.c that moves any result fails the recompute; the
refimpl checks tie the fixtures to the published block layouts rather than
to the oracle's own code.
"""
import os

import numpy as np
import pytest

import refimpl as R

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
Q8_0, Q4_K, Q6_K, Q8_K = 8, 12, 14, 15


def load(name):
    return dict(np.load(os.path.join(GOLD, name), allow_pickle=False))


@pytest.mark.parametrize("name", ["q4k_rows.npz", "q6k_rows.npz", "q80_rows.npz"])
def test_gemv_fixture_recomputes_and_matches_float64(orc, name):
    f = load(name)
    t, k, rows = int(f["type"]), int(f["k"]), int(f["rows"])
    L = orc.lib()
    rb = L.or_row_bytes(t, k)
    deq = np.zeros((rows, k), np.float32)
    for r in range(rows):
        row = np.ascontiguousarray(f["w"][r * rb:(r + 1) * rb])
        L.or_dequant_row(t, row.ctypes.data, deq[r].ctypes.data, k)
    assert np.array_equal(deq, f["dequant"])
    y = np.zeros(rows, np.float32)
    L.or_gemv(t, f["w"].ctypes.data, rows, k, f["x"].ctypes.data, y.ctypes.data)
    assert np.array_equal(y, f["y"])
    # the dequantised values from the published layout, in float64: exact
    # for the Q8_0 / Q6_K products, and for Q4_K equal to ggml's fp32
    # expression d*sc*q - dmin*m within fp32 rounding
    ref = R.unpack(t, f["w"], k).reshape(rows, k)
    assert np.allclose(f["dequant"], ref, rtol=2e-7, atol=1e-9)
    # y against an fp64 dot of the dequantised rows with the dequantised Q8_K /
    # Q8_0 activation: the GEMV's activation quantisation error only
    xq = np.zeros(L.or_row_bytes(Q8_K if t != Q8_0 else Q8_0, k), np.uint8)
    if t == Q8_0:
        L.or_quant_q8_0(f["x"].ctypes.data, xq.ctypes.data, k)
        xd = R.unpack_q80(xq, k).reshape(-1)
    else:
        L.or_quant_q8_K(f["x"].ctypes.data, xq.ctypes.data, k)
        xd = R.unpack_q8k(xq, k)
    y64 = ref @ xd
    assert np.allclose(f["y"], y64, rtol=1e-6, atol=1e-6 * np.abs(y64).max())


def test_q4k_fixture_has_distinct_scales(orc):
    f = load("q4k_rows.npz")
    raw = f["w"].reshape(-1, 144)
    s = raw[:, 4:16].astype(np.int64)
    sc = np.concatenate([s[:, 0:4] & 63, (s[:, 8:12] & 15) | ((s[:, 0:4] >> 6) << 4)], 1)
    mn = np.concatenate([s[:, 4:8] & 63, (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)], 1)
    for b in range(raw.shape[0]):
        assert len(set(sc[b])) == 8 and len(set(mn[b])) == 8


def test_q8k_fixture_and_edge_chunks(orc):
    f = load("q8k_quant.npz")
    x, q = f["x"], f["q8k"]
    L = orc.lib()
    got = np.zeros_like(q)
    L.or_quant_q8_K(x.ctypes.data, got.ctypes.data, x.size)
    assert np.array_equal(got, q)
    blk = q.reshape(-1, 292)
    d = blk[:, 0:4].copy().view(np.float32)[:, 0]
    codes = blk[:, 4:260].view(np.int8)
    bs = blk[:, 260:292].copy().view(np.int16)
    assert d[1] == 0 and not codes[1].any()                       # the all-zero chunk
    assert codes[2][10] == -127 and codes[2][200] == 127          # first index of a |max| tie wins
    assert np.array_equal(bs, codes.reshape(-1, 16, 16).astype(np.int64).sum(-1))
    assert np.all(np.abs(codes.astype(np.int64)) <= 127)


def test_gdn_fixture_recomputes(orc):
    f = load("gdn_step.npz")
    L = orc.lib()
    HK, HV, D = int(f["hk"]), int(f["hv"]), int(f["d"])
    qkv = f["qkv"]
    q, k, v = qkv[:HK * D].copy(), qkv[HK * D:2 * HK * D].copy(), qkv[2 * HK * D:].copy()
    for h in range(HK):
        L.or_l2norm(q[h * D:].ctypes.data, q[h * D:].ctypes.data, D, 1e-6)
        L.or_l2norm(k[h * D:].ctypes.data, k[h * D:].ctypes.data, D, 1e-6)
    g, bt = np.zeros(HV, np.float32), np.zeros(HV, np.float32)
    L.or_gdn_gates(f["alpha"].ctypes.data, f["beta_raw"].ctypes.data, f["dt_bias"].ctypes.data,
                   f["ssm_a"].ctypes.data, g.ctypes.data, bt.ctypes.data, HV)
    st, o = f["state_in"].copy(), np.zeros(HV * D, np.float32)
    L.or_gdn_step(q.ctypes.data, k.ctypes.data, v.ctypes.data, g.ctypes.data, bt.ctypes.data, st.ctypes.data,
                  o.ctypes.data, HV, HK, D, float(f["scale"]), int(f["cols"]))
    assert np.array_equal(st, f["state_out"]) and np.array_equal(o, f["o"])
    # float64 restatement of the delta rule on the same normalised inputs
    o64, M64 = R.gdn_step64(q.reshape(HK, D), k.reshape(HK, D), v.reshape(HV, D), g, bt, f["state_in"], HK)
    assert np.allclose(st, M64, rtol=1e-5, atol=1e-6)
    assert np.allclose(o.reshape(HV, D), o64, rtol=1e-4, atol=1e-6)


def test_attn_fixture_recomputes(orc):
    f = load("attn.npz")
    L = orc.lib()
    NQ, NKV, HD, pos = int(f["nq"]), int(f["nkv"]), int(f["hd"]), int(f["pos"])
    ts = float(f["theta_scale"])
    qr = np.zeros((NQ, HD), np.float32)
    for h in range(NQ):
        L.or_rmsnorm(f["qg"][h * 2 * HD:].ctypes.data, f["q_norm"].ctypes.data, qr[h].ctypes.data, HD, 1e-6)
        L.or_rope_neox(qr[h].ctypes.data, HD, 64, pos, ts)
    Kc, Vc = f["kc_in"].copy(), f["vc_in"].copy()
    Kc[pos], Vc[pos] = f["k_row"], f["v_row"]
    att = np.zeros((NQ, HD), np.float32)
    L.or_attn_decode(qr.ctypes.data, Kc.ctypes.data, Vc.ctypes.data, pos + 1, NQ, NKV, HD, NKV * HD, 0.0625,
                     att.ctypes.data)
    gate = f["qg"].reshape(NQ, 2, HD)[:, 1]
    out = np.array([[np.float32(att[h, i]) * np.float32(L.or_sigmoid(float(gate[h, i]))) for i in range(HD)]
                    for h in range(NQ)], np.float32)
    assert np.array_equal(out, f["out"])
    # float64 softmax restatement
    ref = R.attn64(qr.astype(np.float64), Kc.view(np.float16).astype(np.float64)[:pos + 1],
                   Vc.view(np.float16).astype(np.float64)[:pos + 1], NQ, NKV, HD, 0.0625)
    sig = 1.0 / (1.0 + np.exp(-gate.astype(np.float64)))
    assert np.allclose(out, ref.reshape(NQ, HD) * sig, rtol=1e-5, atol=1e-6)
