"""Independent numpy (float64) restatements used to pin the C oracle.

These are written from the published ggml block layouts and the model
equations, in a different form from oracle/oracle.c (vectorised unpacking,
dequantise-then-dot in float64 instead of integer block sums), so that a
mistake in either shows up as a mismatch.  Test-only code.
"""
import numpy as np

# ----------------------------------------------------------------- packers


def pack_q4k(d, dmin, sc, mn, q):
    """One Q4_K block from d, dmin (f16 bit patterns), 8 scales, 8 mins
    (6-bit) and 256 codes (0..15)."""
    sc = np.asarray(sc, np.int64)
    mn = np.asarray(mn, np.int64)
    q = np.asarray(q, np.int64)
    b = np.zeros(144, np.uint8)
    b[0:2] = np.frombuffer(np.uint16(d).tobytes(), np.uint8)
    b[2:4] = np.frombuffer(np.uint16(dmin).tobytes(), np.uint8)
    s = np.zeros(12, np.int64)
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    b[4:16] = s.astype(np.uint8)
    # element e = 64*p + l (low nibble of byte 32p+l) or 64*p + 32 + l (high)
    qs = np.zeros(128, np.int64)
    for p in range(4):
        qs[32 * p:32 * p + 32] = q[64 * p:64 * p + 32] | (q[64 * p + 32:64 * p + 64] << 4)
    b[16:] = qs.astype(np.uint8)
    return b


def pack_q6k(d, sc, q):
    """One Q6_K block: d (f16 bits), 16 int8 scales, 256 codes in -32..31."""
    u = np.asarray(q, np.int64) + 32
    ql = np.zeros(128, np.int64)
    qh = np.zeros(64, np.int64)
    for n in range(2):
        for l in range(32):
            e = 128 * n + l
            ql[64 * n + l] = (u[e] & 15) | ((u[e + 64] & 15) << 4)
            ql[64 * n + l + 32] = (u[e + 32] & 15) | ((u[e + 96] & 15) << 4)
            qh[32 * n + l] = (u[e] >> 4) | ((u[e + 32] >> 4) << 2) | ((u[e + 64] >> 4) << 4) | ((u[e + 96] >> 4) << 6)
    b = np.zeros(210, np.uint8)
    b[0:128] = ql.astype(np.uint8)
    b[128:192] = qh.astype(np.uint8)
    b[192:208] = np.asarray(sc, np.int64).astype(np.int8).view(np.uint8)
    b[208:210] = np.frombuffer(np.uint16(d).tobytes(), np.uint8)
    return b


# ----------------------------------------------------------------- unpackers (vectorised)


def f16(bits):
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float64)


def unpack_q4k(raw, k):
    """rows of Q4_K bytes -> float64 [rows, k]"""
    raw = np.asarray(raw, np.uint8).reshape(-1, 144)
    d = f16(raw[:, 0:2].copy().view(np.uint16)[:, 0])
    dm = f16(raw[:, 2:4].copy().view(np.uint16)[:, 0])
    s = raw[:, 4:16].astype(np.int64)
    sc = np.zeros((raw.shape[0], 8), np.int64)
    mn = np.zeros((raw.shape[0], 8), np.int64)
    sc[:, :4] = s[:, 0:4] & 63
    mn[:, :4] = s[:, 4:8] & 63
    sc[:, 4:] = (s[:, 8:12] & 15) | ((s[:, 0:4] >> 6) << 4)
    mn[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    qs = raw[:, 16:].astype(np.int64).reshape(-1, 4, 32)
    q = np.concatenate([np.stack([qs[:, p] & 15, qs[:, p] >> 4], 1).reshape(-1, 64) for p in range(4)], 1)
    sub = np.repeat(np.arange(8), 32)
    vals = d[:, None] * sc[:, sub] * q - dm[:, None] * mn[:, sub]
    return vals.reshape(-1, k)


def unpack_q6k(raw, k):
    raw = np.asarray(raw, np.uint8).reshape(-1, 210)
    ql = raw[:, :128].astype(np.int64)
    qh = raw[:, 128:192].astype(np.int64)
    sc = raw[:, 192:208].view(np.int8).astype(np.int64)
    d = f16(raw[:, 208:210].copy().view(np.uint16)[:, 0])
    q = np.zeros((raw.shape[0], 256), np.int64)
    for n in range(2):
        l = np.arange(32)
        a, b, h = ql[:, 64 * n + l], ql[:, 64 * n + 32 + l], qh[:, 32 * n + l]
        q[:, 128 * n + l] = (a & 15) | ((h & 3) << 4)
        q[:, 128 * n + 32 + l] = (b & 15) | (((h >> 2) & 3) << 4)
        q[:, 128 * n + 64 + l] = (a >> 4) | (((h >> 4) & 3) << 4)
        q[:, 128 * n + 96 + l] = (b >> 4) | (((h >> 6) & 3) << 4)
    q -= 32
    vals = d[:, None] * sc[:, np.arange(256) // 16] * q
    return vals.reshape(-1, k)


def unpack_q80(raw, k):
    raw = np.asarray(raw, np.uint8).reshape(-1, 34)
    d = f16(raw[:, 0:2].copy().view(np.uint16)[:, 0])
    q = raw[:, 2:].view(np.int8).astype(np.float64)
    return (d[:, None] * q).reshape(-1, k)


def unpack_bf16(raw, k):
    u = np.asarray(raw, np.uint8).view(np.uint16).astype(np.uint32) << 16
    return u.view(np.float32).astype(np.float64).reshape(-1, k)


def unpack_q8k(raw, k):
    raw = np.asarray(raw, np.uint8).reshape(-1, 292)
    d = raw[:, 0:4].copy().view(np.float32)[:, 0].astype(np.float64)
    q = raw[:, 4:260].view(np.int8).astype(np.float64)
    return (d[:, None] * q).reshape(-1)


def unpack(t, raw, k):
    return {12: unpack_q4k, 14: unpack_q6k, 8: unpack_q80, 30: unpack_bf16}[t](raw, k)


# ----------------------------------------------------------------- float64 model pieces


def rmsnorm64(x, w, eps=1e-6):
    x = np.asarray(x, np.float64)
    y = x / np.sqrt(np.mean(x * x) + eps)
    return y * w if w is not None else y


def silu64(x):
    return x / (1.0 + np.exp(-x))


def sigmoid64(x):
    return 1.0 / (1.0 + np.exp(-x))


def softplus64(x):
    return np.where(x > 20, x, np.log1p(np.exp(np.minimum(x, 20))))


def rope64(x, pos, n_dims, theta_scale):
    x = np.array(x, np.float64)
    half = n_dims // 2
    th = pos * np.asarray(theta_scale, np.float64) ** np.arange(half)
    c, s = np.cos(th), np.sin(th)
    x0, x1 = x[:half].copy(), x[half:n_dims].copy()
    x[:half] = x0 * c - x1 * s
    x[half:n_dims] = x0 * s + x1 * c
    return x


def gdn_step64(q, k, v, g, beta, M, hk):
    """M[h][col][i] = S[i][col]; returns (o, M')"""
    HV, D, _ = M.shape
    M = M.astype(np.float64).copy()
    o = np.zeros((HV, D))
    for h in range(HV):
        kh, qh = k[h % hk], q[h % hk]
        S = M[h].T  # S[i][col]
        kv = S.T @ kh
        delta = (v[h] - g[h] * kv) * beta[h]
        S = g[h] * S + np.outer(kh, delta)
        M[h] = S.T
        o[h] = S.T @ qh / np.sqrt(D)
    return o, M


def attn64(q, K, V, nq, nkv, hd, scale):
    """q [nq, hd]; K, V [n_kv, nkv*hd] float64 -> [nq, hd]"""
    gqa = nq // nkv
    out = np.zeros((nq, hd))
    for h in range(nq):
        g = h // gqa
        k = K[:, g * hd:(g + 1) * hd]
        v = V[:, g * hd:(g + 1) * hd]
        s = (k @ q[h]) * scale
        p = np.exp(s - s.max())
        out[h] = (p @ v) / p.sum()
    return out
