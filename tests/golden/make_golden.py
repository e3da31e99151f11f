"""Write the small golden fixtures under tests/golden/ from the CPU oracle.

Run: python tests/golden/make_golden.py   (needs oracle/liboracle.so: make -C oracle)

Each fixture is an .npz (no pickles) of inputs and the oracle's outputs:
  q4k_rows.npz   3 rows x K=512 Q4_K, every sub-block scale and min distinct;
                 dequantised rows; a GEMV against x (Q8_K activation) -> y
  q6k_rows.npz   3 rows x K=512 Q6_K, all 16 int8 scales distinct; same
  q80_rows.npz   3 rows x K=512 Q8_0, per-block distinct f16 scales; same
  q8k_quant.npz  Q8_K quantisation of x with edge chunks (all zero; +/-max
                 tie, first index wins; half-way codes)
  gdn_step.npz   one GDN step, HK=2 HV=4 D=64 (16 state columns per item):
                 raw qkv / gates / state in, output and updated state out
  attn.npz       one attention decode step, NQ=4 NKV=2 HD=256 at pos 37
The tests recompute every output with the oracle (tests/test_golden.py) and
run the GPU ops on the same inputs (tests/test_gpu_golden.py).
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
import oracle as orc  # noqa: E402

Q8_0, Q4_K, Q6_K, Q8_K = 8, 12, 14, 15
K, ROWS = 512, 3


def f16(v):
    return np.float16(v).view(np.uint16)


def pack_q4k_scales(sc, mn):
    """ggml get_scale_min_k4 layout: 8 six-bit scales and mins in 12 bytes."""
    s = np.zeros(12, np.uint8)
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 0xF) | ((mn[j + 4] & 0xF) << 4)
    return s


def q4k_rows(rng):
    blocks = []
    for r in range(ROWS):
        for b in range(K // 256):
            i = r * (K // 256) + b
            sc = [(1 + 7 * j + 3 * i) % 64 for j in range(8)]
            mn = [(2 + 5 * j + 11 * i) % 64 for j in range(8)]
            assert len(set(sc)) == 8 and len(set(mn)) == 8
            d = f16(0.0123 + 0.001 * i)
            dmin = f16(0.0045 + 0.0007 * i)
            blk = np.concatenate([np.array([d, dmin], np.uint16).view(np.uint8), pack_q4k_scales(sc, mn),
                                  rng.integers(0, 256, 128, dtype=np.uint8)])
            blocks.append(blk)
    return np.concatenate(blocks)


def q6k_rows(rng):
    blocks = []
    for r in range(ROWS):
        for b in range(K // 256):
            i = r * (K // 256) + b
            sc = np.array([(-20 + 3 * j + i) for j in range(16)], np.int8)
            blk = np.concatenate([rng.integers(0, 256, 128, dtype=np.uint8), rng.integers(0, 256, 64, dtype=np.uint8),
                                  sc.view(np.uint8), np.array([f16(0.0031 + 0.0002 * i)], np.uint16).view(np.uint8)])
            blocks.append(blk)
    return np.concatenate(blocks)


def q80_rows(rng):
    blocks = []
    for r in range(ROWS):
        for b in range(K // 32):
            i = r * (K // 32) + b
            blk = np.concatenate([np.array([f16(0.001 + 0.00037 * i)], np.uint16).view(np.uint8),
                                  rng.integers(-127, 128, 32, dtype=np.int8).view(np.uint8)])
            blocks.append(blk)
    return np.concatenate(blocks)


def dequant(t, w):
    L = orc.lib()
    rb = L.or_row_bytes(t, K)
    out = np.zeros((ROWS, K), np.float32)
    for r in range(ROWS):
        row = np.ascontiguousarray(w[r * rb:(r + 1) * rb])
        L.or_dequant_row(t, row.ctypes.data, out[r].ctypes.data, K)
    return out


def gemv(t, w, x):
    y = np.zeros(ROWS, np.float32)
    orc.lib().or_gemv(t, w.ctypes.data, ROWS, K, x.ctypes.data, y.ctypes.data)
    return y


def edge_x(rng, k):
    x = rng.standard_normal(k).astype(np.float32)
    x[256:512] = 0.0                                  # all-zero chunk: d = 0, codes 0
    if k >= 1024:
        c = x[512:768]
        c[:] = rng.uniform(-1, 1, 256).astype(np.float32)
        c[10], c[200] = -3.0, 3.0                     # |max| tie: first index (negative) wins
        c[50] = 3.0 * 0.5 / 127.0                     # lands near a half-way code
    return x


def q8k(x):
    n = x.size
    rb = orc.lib().or_row_bytes(Q8_K, n)
    y = np.zeros(rb, np.uint8)
    orc.lib().or_quant_q8_K(x.ctypes.data, y.ctypes.data, n)
    return y


def gdn(rng):
    L = orc.lib()
    HK, HV, D = 2, 4, 64
    qkv = rng.standard_normal((2 * HK + HV) * D).astype(np.float32)
    al = (rng.standard_normal(HV) * 1.4).astype(np.float32)
    be = rng.standard_normal(HV).astype(np.float32)
    al[1] = 40.0                                      # softplus linear branch
    dt = rng.uniform(-6.9, -2.3, HV).astype(np.float32)
    A = rng.uniform(-16, -1, HV).astype(np.float32)
    M = (rng.standard_normal((HV, D, D)) * 0.1).astype(np.float32)
    scale = np.float32(1) / np.sqrt(np.float32(D))
    q = qkv[:HK * D].copy()
    k = qkv[HK * D:2 * HK * D].copy()
    for h in range(HK):
        L.or_l2norm(q[h * D:].ctypes.data, q[h * D:].ctypes.data, D, 1e-6)
        L.or_l2norm(k[h * D:].ctypes.data, k[h * D:].ctypes.data, D, 1e-6)
    g = np.zeros(HV, np.float32)
    bt = np.zeros(HV, np.float32)
    L.or_gdn_gates(al.ctypes.data, be.ctypes.data, dt.ctypes.data, A.ctypes.data, g.ctypes.data, bt.ctypes.data, HV)
    o = np.zeros(HV * D, np.float32)
    st = M.copy()
    v = qkv[2 * HK * D:].copy()
    cols = 16
    L.or_gdn_step(q.ctypes.data, k.ctypes.data, v.ctypes.data, g.ctypes.data, bt.ctypes.data, st.ctypes.data,
                  o.ctypes.data, HV, HK, D, scale, cols)
    return dict(hk=HK, hv=HV, d=D, cols=cols, scale=scale, qkv=qkv, alpha=al, beta_raw=be, dt_bias=dt, ssm_a=A, state_in=M,
                o=o, state_out=st)


def attn(rng):
    L = orc.lib()
    NQ, NKV, HD, pos, n_ctx = 4, 2, 256, 37, 64
    RW = NKV * HD
    qg = (rng.standard_normal(NQ * 2 * HD) * 2).astype(np.float32)
    k = rng.standard_normal(RW).astype(np.float32)
    v = rng.standard_normal(RW).astype(np.float32)
    qn = (1 + 0.02 * rng.standard_normal(HD)).astype(np.float32)
    kn = (1 + 0.02 * rng.standard_normal(HD)).astype(np.float32)
    Kc = np.zeros((n_ctx, RW), np.float16)
    Vc = np.zeros((n_ctx, RW), np.float16)
    Kc[:pos] = rng.standard_normal((pos, RW))
    Vc[:pos] = rng.standard_normal((pos, RW))
    ts = np.float32(L.or_rope_theta_scale(1e7, 64))
    qr = np.zeros((NQ, HD), np.float32)
    for h in range(NQ):
        L.or_rmsnorm(qg[h * 2 * HD:].ctypes.data, qn.ctypes.data, qr[h].ctypes.data, HD, 1e-6)
        L.or_rope_neox(qr[h].ctypes.data, HD, 64, pos, ts)
    kr = np.zeros((NKV, HD), np.float32)
    for g in range(NKV):
        L.or_rmsnorm(k[g * HD:].ctypes.data, kn.ctypes.data, kr[g].ctypes.data, HD, 1e-6)
        L.or_rope_neox(kr[g].ctypes.data, HD, 64, pos, ts)
    K1, V1 = Kc.copy(), Vc.copy()
    K1[pos] = kr.reshape(-1).astype(np.float16)
    V1[pos] = v.astype(np.float16)
    att = np.zeros((NQ, HD), np.float32)
    L.or_attn_decode(qr.ctypes.data, K1.ctypes.data, V1.ctypes.data, pos + 1, NQ, NKV, HD, RW, 0.0625,
                     att.ctypes.data)
    gate = qg.reshape(NQ, 2, HD)[:, 1]
    out = np.array([[np.float32(att[h, i]) * np.float32(L.or_sigmoid(float(gate[h, i]))) for i in range(HD)]
                    for h in range(NQ)], np.float32)
    return dict(nq=NQ, nkv=NKV, hd=HD, pos=pos, n_ctx=n_ctx, theta_scale=ts, qg=qg, k=k, v=v, q_norm=qn, k_norm=kn,
                kc_in=Kc.view(np.uint16), vc_in=Vc.view(np.uint16), k_row=K1[pos].view(np.uint16),
                v_row=V1[pos].view(np.uint16), out=out)


def main():
    rng = np.random.default_rng(20261201)
    x = edge_x(rng, K)
    for name, t, make in (("q4k_rows", Q4_K, q4k_rows), ("q6k_rows", Q6_K, q6k_rows), ("q80_rows", Q8_0, q80_rows)):
        w = make(rng)
        assert w.size == orc.lib().or_row_bytes(t, K) * ROWS
        np.savez_compressed(os.path.join(HERE, name + ".npz"), type=t, k=K, rows=ROWS, w=w, x=x,
                            dequant=dequant(t, w), y=gemv(t, w, x))
    xq = edge_x(rng, 1024)
    np.savez_compressed(os.path.join(HERE, "q8k_quant.npz"), x=xq, q8k=q8k(xq))
    np.savez_compressed(os.path.join(HERE, "gdn_step.npz"), **gdn(rng))
    np.savez_compressed(os.path.join(HERE, "attn.npz"), **attn(rng))
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))


if __name__ == "__main__":
    main()
