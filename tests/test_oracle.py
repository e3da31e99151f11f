"""Pins the CPU oracle (CPU only, no GPU).

Each check is chosen so that a plausible mistake in oracle/oracle.c (a
swapped scale/min, a wrong nibble or bit-pair order, a dropped term, a wrong
sign, a transposed state) fails it: closed forms, independent float64
restatements (tests/refimpl.py), brute force over code spaces, and the
committed golden vectors.
"""
import ctypes as C

import numpy as np
import pytest

import refimpl as R

Q8_0, Q4_K, Q6_K, Q8_K, BF16, F32 = 8, 12, 14, 15, 30, 0


def P(a):
    return a.ctypes.data


# ----------------------------------------------------------------- scalar conversions

def test_f16_roundtrip_all_codes(orc):
    L = orc.lib()
    codes = np.arange(65536, dtype=np.uint16)
    ref = codes.view(np.float16).astype(np.float32)
    got = np.array([L.or_f16_to_f32(int(c)) for c in codes[::7]], np.float32)
    r = ref[::7]
    fin = np.isfinite(r)
    assert np.array_equal(got[fin], r[fin])
    assert np.all(np.isnan(got[~np.isfinite(r) & np.isnan(r)]))


def test_f32_to_f16_matches_ieee_rne(orc):
    L = orc.lib()
    rng = np.random.default_rng(0)
    xs = np.concatenate([
        rng.standard_normal(4000).astype(np.float32) * np.float32(10) ** rng.integers(-9, 5, 4000).astype(np.float32),
        np.array([0.0, -0.0, 65504, 65519.99, 65520, 1e9, 2 ** -24, 2 ** -25, 3 * 2 ** -26, 2 ** -14,
                  2 ** -14 - 2 ** -26, 1 + 2 ** -11, 1 + 3 * 2 ** -11, -(1 + 2 ** -11)], np.float32)])
    got = np.array([L.or_f32_to_f16(float(x)) for x in xs], np.uint16)
    ref = xs.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


def test_bf16_matches_torch_rne(orc):
    import torch
    L = orc.lib()
    rng = np.random.default_rng(1)
    xs = (rng.standard_normal(3000) * 100).astype(np.float32)
    # exact halfway cases: low 16 bits 0x8000 with even and odd bit 16
    hw = (np.array([0x3f808000, 0x3f818000, 0xbf808000, 0x40490000], np.uint32)).view(np.float32)
    xs = np.concatenate([xs, hw])
    got = np.array([L.or_f32_to_bf16(float(x)) for x in xs], np.uint16)
    ref = torch.from_numpy(xs).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, ref)


def test_nearest_int_is_round_half_even(orc):
    L = orc.lib()
    xs = np.concatenate([np.arange(-300, 300) * 0.5, np.random.default_rng(2).uniform(-4e5, 4e5, 2000)])
    xs = xs.astype(np.float32)
    got = np.array([L.or_nearest_int(float(x)) for x in xs])
    assert np.array_equal(got, np.rint(xs).astype(np.int64))


# ----------------------------------------------------------------- block formats

def test_q4k_dequant_closed_form_all_scale_codes(orc):
    """Every 6-bit scale and min value appears; dequant must equal
    d*sc*q - dmin*m with the layout's scale packing and nibble order."""
    rng = np.random.default_rng(3)
    for blk in range(8):
        sc = np.arange(8) + 8 * blk          # 0..63 across the 8 blocks
        mn = 63 - (np.arange(8) * 8 + blk)    # 63..0, distinct pattern
        q = rng.integers(0, 16, 256)
        d = np.float16(0.0123).view(np.uint16)
        dm = np.float16(0.0071).view(np.uint16)
        b = R.pack_q4k(d, dm, sc, mn, q)
        got = orc.dequant(Q4_K, b, 256)
        df, dmf = np.float32(np.float16(0.0123)), np.float32(np.float16(0.0071))
        sub = np.arange(256) // 32
        ref = (df * sc[sub].astype(np.float32)) * q.astype(np.float32) - dmf * mn[sub].astype(np.float32)
        assert np.array_equal(got, ref.astype(np.float32))


def test_q6k_dequant_closed_form(orc):
    rng = np.random.default_rng(4)
    for _ in range(4):
        sc = rng.integers(-128, 128, 16)
        q = rng.integers(-32, 32, 256)
        d = np.float16(0.00037).view(np.uint16)
        b = R.pack_q6k(d, sc, q)
        got = orc.dequant(Q6_K, b, 256)
        ref = (np.float32(np.float16(0.00037)) * sc[np.arange(256) // 16].astype(np.float32)) * q.astype(np.float32)
        assert np.array_equal(got, ref)


def test_q8k_quantizer_invariants(orc):
    rng = np.random.default_rng(5)
    x = (rng.standard_normal(1024) * rng.uniform(0.01, 30, 1024)).astype(np.float32)
    x[256:512] = 0.0                      # an all-zero block
    x[515] = 7.0                          # tie on |max|: first (positive) wins
    x[519] = -7.0
    x[512:515] = 0.1
    x[516:519] = 0.1
    x[520:768] = 0.1
    q = orc.quantize(Q6_K, x)
    blk = q.reshape(-1, 292)
    d = blk[:, 0:4].copy().view(np.float32)[:, 0]
    qs = blk[:, 4:260].view(np.int8).astype(np.int64)
    bs = blk[:, 260:292].copy().view(np.int16).astype(np.int64)
    assert d[1] == 0 and np.all(qs[1] == 0) and np.all(bs[1] == 0)
    assert qs[2][515 - 512] == -127 and qs[2][519 - 512] == 127 and d[2] < 0
    for i in (0, 2, 3):
        xb = x[256 * i:256 * i + 256].astype(np.float64)
        assert np.all(np.abs(xb - d[i] * qs[i]) <= abs(d[i]) * 0.5 * (1 + 1e-6))
        assert np.array_equal(bs[i], qs[i].reshape(16, 16).sum(1))
        assert qs[i].max() <= 127 and qs[i].min() >= -127


def test_q8_0_quantizer_invariants(orc):
    rng = np.random.default_rng(6)
    x = (rng.standard_normal(512) * 3).astype(np.float32)
    x[32:64] = 0
    q = orc.quantize(Q8_0, x).reshape(-1, 34)
    d = q[:, 0:2].copy().view(np.float16)[:, 0].astype(np.float64)
    qs = q[:, 2:].view(np.int8).astype(np.int64)
    assert d[1] == 0 and np.all(qs[1] == 0)
    for i in range(16):
        xb = x[32 * i:32 * i + 32]
        amax = np.abs(xb).max()
        assert d[i] == float(np.float16(np.float32(amax) / np.float32(127)))
        if amax > 0:
            assert np.array_equal(qs[i], np.rint(xb * (np.float32(127) / np.float32(amax))).astype(np.int64))


def test_q8_0_ref_quantizer_known_answers(orc):
    """ggml's reference Q8_0 form (the KV cache's): id = 1/d, codes rounded
    half away from zero -- where the x86 form (id = 127/amax, half to even)
    differs, this one must be taken."""
    x = np.zeros(96, np.float32)
    x[0], x[1], x[2], x[3] = 127.0, 62.5, -62.5, -127.0      # d = 1: ties at +-62.5
    x[64:96] = (np.random.default_rng(8).standard_normal(32) * 0.37).astype(np.float32)
    y = np.zeros(3 * 34, np.uint8)
    orc.lib().or_quant_q8_0_ref(P(x), P(y), 96)
    b = y.reshape(3, 34)
    d = b[:, :2].copy().view(np.float16)[:, 0]
    qs = b[:, 2:].view(np.int8).astype(np.int64)
    assert d[0] == 1.0 and list(qs[0, :4]) == [127, 63, -63, -127] and not qs[0, 4:].any()
    assert d[1] == 0 and not qs[1].any()                      # an all-zero block
    xb = x[64:96].astype(np.float64)
    amax = np.abs(xb).max()
    df = np.float32(np.float32(amax) / np.float32(127))
    assert d[2] == np.float16(df)
    assert np.abs(qs[2]).max() == 127 and qs[2][np.argmax(np.abs(xb))] * np.sign(xb[np.argmax(np.abs(xb))]) == 127
    # each code is the nearest integer to x / d (d before its f16 rounding)
    assert np.all(np.abs(qs[2] - xb / float(df)) <= 0.5 + 1e-6)
    # where 1/d and 127/amax give different codes, the 1/d one is taken
    rng = np.random.default_rng(9)
    found = 0
    for _ in range(2000):
        xs = (rng.standard_normal(32) * rng.uniform(0.01, 10)).astype(np.float32)
        am = np.float32(np.abs(xs).max())
        dd = np.float32(am / np.float32(127))
        a_ = np.trunc(xs * (np.float32(1) / dd) + np.copysign(np.float32(0.5), xs))      # roundf(x / d form)
        b_ = np.rint(xs * (np.float32(127) / am))
        if np.array_equal(a_, b_):
            continue
        found += 1
        yy = np.zeros(34, np.uint8)
        orc.lib().or_quant_q8_0_ref(P(xs), P(yy), 32)
        assert np.array_equal(yy[2:].view(np.int8).astype(np.float32), a_.astype(np.float32))
    assert found > 0


def test_attention_over_q8_0_cache_equals_dequantised_f32(orc):
    """or_attn_decode_kv over a Q8_0 cache equals the float64 reference over
    the dequantised cache (codes times block scales)."""
    rng = np.random.default_rng(19)
    nq, nkv, hd, n = 6, 2, 256, 130
    q = rng.standard_normal((nq, hd)).astype(np.float32)
    kf = rng.standard_normal((n, nkv * hd)).astype(np.float32)
    vf = rng.standard_normal((n, nkv * hd)).astype(np.float32)
    K = np.zeros((n, nkv * hd // 32 * 34), np.uint8)
    V = np.zeros_like(K)
    for j in range(n):
        orc.lib().or_quant_q8_0_ref(P(kf[j]), P(K[j]), nkv * hd)
        orc.lib().or_quant_q8_0_ref(P(vf[j]), P(V[j]), nkv * hd)

    def deq(c):
        b = c.reshape(n, -1, 34)
        d = b[:, :, :2].copy().view(np.float16)[..., 0].astype(np.float64)
        return (b[:, :, 2:].view(np.int8).astype(np.float64) * d[..., None]).reshape(n, -1)
    out = np.zeros((nq, hd), np.float32)
    orc.lib().or_attn_decode_kv(P(q), P(K), P(V), Q8_0, n, nq, nkv, hd, 0.0625, P(out))
    ref = R.attn64(q.astype(np.float64), deq(K), deq(V), nq, nkv, hd, 0.0625)
    assert np.allclose(out, ref, rtol=1e-6, atol=1e-7)
    # and over an f16 cache it is or_attn_decode exactly
    Kh, Vh = kf.astype(np.float16), vf.astype(np.float16)
    o1, o2 = np.zeros((nq, hd), np.float32), np.zeros((nq, hd), np.float32)
    orc.lib().or_attn_decode_kv(P(q), P(Kh), P(Vh), 1, n, nq, nkv, hd, 0.0625, P(o1))
    orc.lib().or_attn_decode(P(q), P(Kh), P(Vh), n, nq, nkv, hd, nkv * hd, 0.0625, P(o2))
    assert np.array_equal(o1, o2)


@pytest.mark.parametrize("t", [Q4_K, Q6_K, Q8_0])
def test_block_term_equals_float64_dequant_dot(orc, sn, t):
    """integer-sum block term == float64 dequantise-then-dot (different
    formulation; exact up to fp64 rounding)."""
    rng = np.random.default_rng(7 + t)
    k = 256
    w = np.zeros(orc.row_bytes(t, k), np.uint8)
    sn.lib().sinter_synth(0, w.ctypes.data, 0, t, 1, k, 99 + t, 0.0, 0.0, None)
    x = rng.standard_normal(k).astype(np.float32)
    xq = orc.quantize(t, x)
    wd = R.unpack(t, w, k)[0]
    xd = R.unpack_q8k(xq, k) if t != Q8_0 else R.unpack_q80(xq, k)[0]
    ref = float(wd @ xd)
    if t == Q8_0:
        got = sum(orc.lib().or_block_term(t, P(w) + 34 * i, P(xq) + 34 * i) for i in range(8))
    else:
        got = orc.lib().or_block_term(t, P(w), P(xq))
    assert abs(got - ref) <= 1e-12 * max(1.0, abs(ref))


@pytest.mark.parametrize("t,k", [(Q4_K, 5120), (Q6_K, 5120), (Q6_K, 17408), (Q8_0, 5120), (BF16, 4096)])
def test_gemv_matches_float64_reference(orc, sn, t, k):
    rng = np.random.default_rng(11)
    rows = 37
    w = np.zeros(orc.row_bytes(t, k) * rows, np.uint8)
    sn.lib().sinter_synth(0, w.ctypes.data, 0, t, rows, k, 1234 + t, 0.0, 0.0, None)
    x = rng.standard_normal(k).astype(np.float32)
    y = orc.gemv(t, w, rows, k, x)
    xq = orc.quantize(t, x)
    xd = {Q8_0: lambda: R.unpack_q80(xq, k)[0], BF16: lambda: R.unpack_bf16(xq, k)[0]}.get(
        t, lambda: R.unpack_q8k(xq, k))()
    ref = R.unpack(t, w, k) @ xd
    assert np.allclose(y, ref, rtol=2e-7, atol=1e-9)
    # and against the unquantised activation: the quantisation error scale
    ref_fp = R.unpack(t, w, k) @ x.astype(np.float64)
    rel = np.linalg.norm(y - ref_fp) / np.linalg.norm(ref_fp)
    assert rel < (5e-3 if t == BF16 else 2e-2)  # bf16 activation rounding ~2e-3


# ----------------------------------------------------------------- norms and unary ops

def test_rmsnorm_closed_form_and_reference(orc):
    x = np.full(512, -3.0, np.float32)
    w = np.linspace(0.5, 1.5, 512).astype(np.float32)
    y = orc.rmsnorm(x, w, 1e-6)
    assert np.allclose(y, -w / np.sqrt(1 + 1e-6 / 9), rtol=1e-6)
    x = np.random.default_rng(12).standard_normal(5120).astype(np.float32) * 7
    y = orc.rmsnorm(x, w.repeat(10), 1e-6)
    assert np.allclose(y, R.rmsnorm64(x, w.repeat(10)), rtol=3e-7, atol=1e-7)


def test_unary_ops(orc):
    L = orc.lib()
    xs = np.linspace(-30, 30, 601).astype(np.float32)
    # softplus follows ggml's fp32 form logf(1 + expf(x)): for x << 0 the sum
    # rounds to 1 and the result to 0, an absolute error below 1e-7
    for fn, ref, atol in ((L.or_silu, R.silu64, 1e-30), (L.or_sigmoid, R.sigmoid64, 1e-30),
                          (L.or_softplus, R.softplus64, 1e-7)):
        got = np.array([fn(float(v)) for v in xs], np.float64)
        assert np.allclose(got, ref(xs.astype(np.float64)), rtol=3e-7, atol=atol)
    assert L.or_softplus(25.0) == 25.0          # linear branch above 20
    assert abs(L.or_sigmoid(0.0) - 0.5) == 0.0


def test_l2norm(orc):
    L = orc.lib()
    x = np.random.default_rng(13).standard_normal(128).astype(np.float32)
    y = np.zeros_like(x)
    L.or_l2norm(P(x), P(y), 128, 1e-6)
    assert np.allclose(y, x / np.linalg.norm(x.astype(np.float64)), rtol=3e-7)
    z = np.full(128, 1e-9, np.float32)           # eps floor: scale = 1/eps
    L.or_l2norm(P(z), P(y), 128, 1e-6)
    assert np.allclose(y, z / np.float32(1e-6), rtol=1e-6)


# ----------------------------------------------------------------- gated DeltaNet

def _gdn_inputs(seed, HK=2, HV=4, D=128):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((HK, D)).astype(np.float32)
    k = rng.standard_normal((HK, D)).astype(np.float32)
    q /= np.linalg.norm(q, axis=1, keepdims=True)
    k /= np.linalg.norm(k, axis=1, keepdims=True)
    v = rng.standard_normal((HV, D)).astype(np.float32)
    g = rng.uniform(0.5, 0.99, HV).astype(np.float32)
    beta = rng.uniform(0.1, 0.9, HV).astype(np.float32)
    M = (rng.standard_normal((HV, D, D)) * 0.1).astype(np.float32)
    return q, k, v, g, beta, M


def _or_gdn(orc, q, k, v, g, beta, M, cols=32):
    HV, D, _ = M.shape
    o = np.zeros((HV, D), np.float32)
    st = M.copy()
    orc.lib().or_gdn_step(P(q), P(k), P(v), P(g), P(beta), P(st), P(o), HV, q.shape[0], D,
                          np.float32(1) / np.sqrt(np.float32(D)), cols)
    return o, st


def test_gdn_step_reference(orc):
    q, k, v, g, beta, M = _gdn_inputs(14)
    o, st = _or_gdn(orc, q, k, v, g, beta, M)
    o64, M64 = R.gdn_step64(q, k, v, g, beta, M, q.shape[0])
    assert np.allclose(st, M64, rtol=1e-5, atol=1e-6)
    assert np.allclose(o, o64, rtol=1e-4, atol=1e-6)


@pytest.mark.parametrize("cols", [16, 32])
def test_gdn_step_exact_dyadic(orc, cols):
    """Inputs on dyadic grids, so that kv, delta and the updated state are
    exact in fp32 whatever the fold order: the oracle's S' must equal the
    exact fp64 delta rule bit for bit -- a dropped or misindexed term, a
    transposed state or a wrong head map fails it -- and o must be within
    fp32 rounding of it."""
    rng = np.random.default_rng(31 + cols)
    HK, HV, D = 2, 4, 128
    q = (rng.integers(-8, 9, (HK, D)) / 64).astype(np.float32)
    k = (rng.integers(-8, 9, (HK, D)) / 64).astype(np.float32)
    v = (rng.integers(-8, 9, (HV, D)) / 8).astype(np.float32)
    g = np.array([0.5, 1.0, 0.25, 0.75], np.float32)
    beta = np.array([0.5, 0.25, 1.0, 0.125], np.float32)
    M = (rng.integers(-8, 9, (HV, D, D)) / 16).astype(np.float32)
    o, st = _or_gdn(orc, q, k, v, g, beta, M, cols)
    o64, M64 = R.gdn_step64(q, k, v, g, beta, M, HK)
    # kv, delta and S' stay on a 2^-21 grid below 2: exact in fp32
    assert np.array_equal(st.astype(np.float64), M64)
    # the o sums need more than 24 bits: within fp32 rounding of the exact value
    assert np.allclose(o, o64, rtol=2e-6, atol=1e-7)


def test_gdn_step_closed_forms(orc):
    q, k, v, g, beta, M = _gdn_inputs(15)
    # k = 0: the state only decays, S' = g*S exactly (fp32 product)
    o, st = _or_gdn(orc, q, np.zeros_like(k), v, g, beta, M)
    assert np.array_equal(st, (g[:, None, None] * M).astype(np.float32))
    # g = 1, beta = 0: the state is unchanged, o = S^T q / sqrt(D)
    o, st = _or_gdn(orc, q, k, v, np.ones_like(g), np.zeros_like(beta), M)
    assert np.array_equal(st, M)
    D = M.shape[1]
    ref = np.stack([M[h].astype(np.float64) @ q[h % 2] for h in range(4)]) / np.sqrt(D)
    assert np.allclose(o, ref, rtol=1e-6, atol=1e-7)


def test_conv_silu(orc):
    rng = np.random.default_rng(16)
    C_, dc = 512, 4
    st = rng.standard_normal(C_ * 3).astype(np.float32)
    w = rng.uniform(-0.5, 0.5, C_ * 4).astype(np.float32)
    x = rng.standard_normal(C_).astype(np.float32)
    out = np.zeros(C_, np.float32)
    st2 = st.copy()
    orc.lib().or_conv_silu(P(x), P(st2), P(w), P(out), C_, dc)
    win = np.concatenate([st.reshape(C_, 3), x[:, None]], 1).astype(np.float64)
    ref = R.silu64((win * w.reshape(C_, 4)).sum(1))
    assert np.allclose(out, ref, rtol=3e-7, atol=1e-8)
    assert np.array_equal(st2.reshape(C_, 3), win[:, 1:].astype(np.float32))


def test_gdn_gates(orc):
    a = np.array([-3.0, 0.5, 25.0, 1.0], np.float32)
    b = np.array([0.0, -2.0, 3.0, 30.0], np.float32)
    dt = np.array([-4.0, -2.5, -6.0, 0.0], np.float32)
    A = np.array([-1.0, -8.0, -16.0, -0.5], np.float32)
    g = np.zeros(4, np.float32)
    be = np.zeros(4, np.float32)
    orc.lib().or_gdn_gates(P(a), P(b), P(dt), P(A), P(g), P(be), 4)
    ab = a.astype(np.float64) + dt
    assert np.allclose(g, np.exp(R.softplus64(ab) * A), rtol=1e-6)
    assert np.allclose(be, R.sigmoid64(b.astype(np.float64)), rtol=1e-6)


# ----------------------------------------------------------------- attention

def test_rope_theta_scale_constant(orc):
    ts = orc.lib().or_rope_theta_scale(1e7, 64)
    assert np.float32(ts) == np.float32.fromhex("0x1.356656p-1") if hasattr(np.float32, "fromhex") else \
        np.float32(ts) == np.float32(float.fromhex("0x1.356656p-1"))


def test_rope_identity_at_pos0_and_reference(orc):
    x = np.random.default_rng(17).standard_normal(256).astype(np.float32)
    y = x.copy()
    ts = orc.lib().or_rope_theta_scale(1e7, 64)
    orc.lib().or_rope_neox(P(y), 256, 64, 0, ts)
    assert np.array_equal(y, x)
    for pos in (1, 7, 4095, 131071):
        y = x.copy()
        orc.lib().or_rope_neox(P(y), 256, 64, pos, ts)
        assert np.array_equal(y[64:], x[64:])
        # ggml's rope cache forms theta_i by repeated fp32 products theta_{i+1} =
        # theta_i * theta_scale; restate that and compare tightly ...
        th = np.zeros(32, np.float32)
        t = np.float32(pos)
        for i in range(32):
            th[i] = t
            t = np.float32(t * np.float32(ts))
        c, s_ = np.cos(th.astype(np.float64)), np.sin(th.astype(np.float64))
        x0, x1 = x[:32].astype(np.float64), x[32:64].astype(np.float64)
        assert np.allclose(y[:32], x0 * c - x1 * s_, atol=2e-6)
        assert np.allclose(y[32:64], x0 * s_ + x1 * c, atol=2e-6)
        # ... and loosely against the exact-power rotation (the fp32 product
        # chain drifts by ~i*2^-24 relative in theta)
        ref = R.rope64(x, pos, 64, np.float32(ts))
        assert np.allclose(y, ref, atol=max(1e-5, pos * 4e-7))
        # rotation preserves every pair's norm
        n0 = x[:32].astype(np.float64) ** 2 + x[32:64].astype(np.float64) ** 2
        n1 = y[:32].astype(np.float64) ** 2 + y[32:64].astype(np.float64) ** 2
        assert np.allclose(n0, n1, rtol=1e-5)


def test_attention_reference_and_single_position(orc):
    rng = np.random.default_rng(18)
    nq, nkv, hd, n = 6, 2, 256, 300
    q = rng.standard_normal((nq, hd)).astype(np.float32)
    K = rng.standard_normal((n, nkv * hd)).astype(np.float16)
    V = rng.standard_normal((n, nkv * hd)).astype(np.float16)
    out = np.zeros((nq, hd), np.float32)
    orc.lib().or_attn_decode(P(q), P(K), P(V), n, nq, nkv, hd, nkv * hd, 0.0625, P(out))
    ref = R.attn64(q.astype(np.float64), K.astype(np.float64), V.astype(np.float64), nq, nkv, hd, 0.0625)
    assert np.allclose(out, ref, rtol=1e-6, atol=1e-7)
    orc.lib().or_attn_decode(P(q), P(K), P(V), 1, nq, nkv, hd, nkv * hd, 0.0625, P(out))
    for h in range(nq):
        g = h // (nq // nkv)
        assert np.array_equal(out[h], V[0, g * hd:(g + 1) * hd].astype(np.float32))


def test_argmax_first_max_wins(orc):
    x = np.array([1, 5, 3, 5, 5, -1], np.float32)
    assert orc.lib().or_argmax_first(P(x), 6) == 1
    x = np.array([-np.inf, -2, -2], np.float32)
    assert orc.lib().or_argmax_first(P(x), 3) == 1


# ---------------------------------------------------------------- split-K attention (fp32 declared folds)

def _attn_case(rng, n, nq, nkv, hd=256):
    q = rng.standard_normal((nq, hd)).astype(np.float32)
    K = rng.standard_normal((n, nkv * hd)).astype(np.float16)
    V = rng.standard_normal((n, nkv * hd)).astype(np.float16)
    return q, K, V


@pytest.mark.parametrize("n,nq,nkv,chunks,cmin", [(1, 24, 4, 64, 0), (33, 24, 4, 64, 0), (100, 8, 2, 3, 0),
                                                  (4097, 24, 4, 64, 128), (4097, 24, 4, 64, 256),
                                                  (777, 16, 2, 32, 1000), (64, 4, 4, 1, 0), (300, 12, 4, 9, 64)])
def test_attn_split_near_exact_attention(orc, n, nq, nkv, chunks, cmin):
    """or_attn_split (fp32 folds) within rel L2 1e-5 of the exact fp64
    attention, and its geometry covers [0, n) with at most `chunks`
    non-empty chunks of whole tiles, each at least chunk_min long (but the
    last)."""
    rng = np.random.default_rng(n + nq)
    q, K, V = _attn_case(rng, n, nq, nkv)
    out = np.zeros((nq, 256), np.float32)
    ex = np.zeros((nq, 256), np.float32)
    L = orc.lib()
    L.or_attn_split(P(q), P(K), P(V), 1, n, nq, nkv, 256, 0.0625, chunks, cmin, P(out))
    L.or_attn_decode(P(q), P(K.view(np.uint16)), P(V.view(np.uint16)), n, nq, nkv, 256, nkv * 256, 0.0625, P(ex))
    assert np.linalg.norm(out - ex) <= 1e-5 * np.linalg.norm(ex)
    T, tpc, nch = C.c_int(), C.c_int(), C.c_int()
    L.or_attn_geom(n, chunks, cmin, C.byref(T), C.byref(tpc), C.byref(nch))
    assert T.value == -(-n // 32) and 1 <= nch.value <= chunks
    assert (nch.value - 1) * tpc.value < T.value <= nch.value * tpc.value      # every chunk non-empty, all covered
    assert tpc.value * 32 >= cmin and tpc.value >= -(-T.value // chunks)


def test_attn_split_closed_forms(orc):
    """One position: the output is the V row exactly (weight exp(0) = 1, one
    chunk).  Identical keys: every weight is 1, so the output is the mean of
    the V rows (to fp32 rounding).  A shifted score (q scaled so all scores
    move together) leaves the softmax unchanged."""
    rng = np.random.default_rng(5)
    L = orc.lib()
    q, K, V = _attn_case(rng, 1, 8, 2)
    out = np.zeros((8, 256), np.float32)
    L.or_attn_split(P(q), P(K), P(V), 1, 1, 8, 2, 256, 0.0625, 64, 0, P(out))
    assert np.array_equal(out, np.repeat(V.astype(np.float32).reshape(2, 256), 4, axis=0))
    n = 200
    q, K, V = _attn_case(rng, n, 8, 2)
    K[:] = K[0]
    L.or_attn_split(P(q), P(K), P(V), 1, n, 8, 2, 256, 0.0625, 7, 0, P(out))
    mean = V.astype(np.float64).reshape(n, 2, 256).mean(axis=0)
    assert np.allclose(out.reshape(2, 4, 256), mean[:, None, :], rtol=2e-6, atol=2e-6)


def test_attn_split_planted_mistakes_are_caught(orc):
    """The fp64 pin separates the fold from plausible mistakes: attention with
    the wrong scale, or with the last position dropped, is far outside the
    1e-5 band the correct fold meets."""
    rng = np.random.default_rng(9)
    L = orc.lib()
    n, nq, nkv = 300, 8, 2
    q, K, V = _attn_case(rng, n, nq, nkv)
    q *= 8
    ex = np.zeros((nq, 256), np.float32)
    L.or_attn_decode(P(q), P(K.view(np.uint16)), P(V.view(np.uint16)), n, nq, nkv, 256, nkv * 256, 0.0625, P(ex))
    good = np.zeros((nq, 256), np.float32)
    L.or_attn_split(P(q), P(K), P(V), 1, n, nq, nkv, 256, 0.0625, 9, 0, P(good))
    assert np.linalg.norm(good - ex) <= 1e-6 * np.linalg.norm(ex)
    for args in ((n, 0.125), (n - 1, 0.0625)):
        bad = np.zeros((nq, 256), np.float32)
        L.or_attn_split(P(q), P(K), P(V), 1, args[0], nq, nkv, 256, args[1], 9, 0, P(bad))
        assert np.linalg.norm(bad - ex) > 1e-5 * np.linalg.norm(ex)
