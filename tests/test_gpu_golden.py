"""The golden fixtures (tests/golden/*.npz) through the GPU ops, via the C
ABI: the kernels must reproduce the committed oracle outputs -- GEMV rows and
the GDN step bit for bit, attention within the split-K merge's 1-ulp rule,
the appended K/V rows bit for bit."""
import ctypes as C
import os

import numpy as np
import pytest

from test_gpu_ops import assert_ulp, dev, empty_f32, host, run_gemv, stream

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return dict(np.load(os.path.join(GOLD, name), allow_pickle=False))


@pytest.mark.parametrize("name,blocks", [("q4k_rows.npz", 1), ("q4k_rows.npz", 3), ("q6k_rows.npz", 2),
                                         ("q80_rows.npz", 3)])
def test_gemv_golden(sn, torch_gpu, name, blocks):
    torch = torch_gpu
    f = load(name)
    t, k, rows = int(f["type"]), int(f["k"]), int(f["rows"])
    dw, dx, dy = dev(torch, f["w"]), dev(torch, f["x"]), empty_f32(torch, rows)
    a = sn.GemvArgs(K=k, pro=sn.PRO_PLAIN, n_seg=1, eps=1e-6)
    a.x = dx.data_ptr()
    a.seg[0] = sn.GemvSeg(w=dw.data_ptr(), y=dy.data_ptr(), rows=rows, type=t, epi=sn.EPI_STORE)
    print(f"golden {name} blocks={blocks}", flush=True)
    run_gemv(sn, torch, a, blocks)
    assert np.array_equal(host(dy), f["y"])


def test_gdn_golden(sn, torch_gpu):
    torch = torch_gpu
    f = load("gdn_step.npz")
    HK, HV, D = int(f["hk"]), int(f["hv"]), int(f["d"])
    d = {n: dev(torch, f[n]) for n in ("qkv", "alpha", "beta_raw", "dt_bias", "ssm_a", "state_in")}
    do = empty_f32(torch, HV * D)
    a = sn.GdnArgs(hk=HK, hv=HV, d=D, cols=16, eps=1e-6, scale=float(f["scale"]))
    a.qkv, a.alpha, a.beta, a.dt_bias, a.ssm_a = (d["qkv"].data_ptr(), d["alpha"].data_ptr(), d["beta_raw"].data_ptr(),
                                                  d["dt_bias"].data_ptr(), d["ssm_a"].data_ptr())
    a.state, a.o = d["state_in"].data_ptr(), do.data_ptr()
    print(f"golden gdn_step HK={HK} HV={HV} D={D} cols=16 blocks=16", flush=True)
    sn.check(sn.lib().sinter_op_gdn_step(C.byref(a), 16, C.c_void_p(stream(torch))), "gdn")
    torch.cuda.synchronize()
    assert sn.op_error()[0] == 0
    assert np.array_equal(host(d["state_in"]), f["state_out"])
    assert np.array_equal(host(do), f["o"])


@pytest.mark.parametrize("chunks,blocks,cmin", [(1, 2, 0), (4, 8, 0), (9, 18, 0), (9, 23, 0), (4, 8, 64)])
def test_attn_golden(sn, orc, torch_gpu, chunks, blocks, cmin):
    """The attention fixture (exact fp64 attention of a decode step): the GPU
    output equals the oracle's restatement of the op's fp32 folds
    (or_attn_split) bit for bit and the fixture within rel L2 1e-5; the
    appended rows are the fixture's."""
    torch = torch_gpu
    f = load("attn.npz")
    NQ, NKV, HD, pos, n_ctx = (int(f[n]) for n in ("nq", "nkv", "hd", "pos", "n_ctx"))
    dK, dV = dev(torch, f["kc_in"]), dev(torch, f["vc_in"])
    dqg, dk, dv_, dqn, dkn = (dev(torch, f[n]) for n in ("qg", "k", "v", "q_norm", "k_norm"))
    part = torch.zeros(sn.lib().sinter_attn_part_len(NQ, NKV, HD, chunks), dtype=torch.float32, device="cuda")
    cnt = torch.zeros(sn.lib().sinter_attn_count_len(NKV, chunks), dtype=torch.int32, device="cuda")
    out = empty_f32(torch, NQ * HD)
    cell = dev(torch, np.array([0, pos, 0, 0], np.int32))
    a = sn.AttnArgs(nq=NQ, nkv=NKV, hd=HD, rope_dims=64, n_ctx=n_ctx, n_chunks=chunks,
                    theta_scale=float(f["theta_scale"]), eps=1e-6, scale=0.0625, chunk_min=cmin)
    a.qg, a.k, a.v, a.q_norm, a.k_norm = dqg.data_ptr(), dk.data_ptr(), dv_.data_ptr(), dqn.data_ptr(), dkn.data_ptr()
    a.kc, a.vc, a.part, a.count, a.out, a.pass_cell = (dK.data_ptr(), dV.data_ptr(), part.data_ptr(),
                                                       cnt.data_ptr(), out.data_ptr(), cell.data_ptr())
    print(f"golden attn pos={pos} chunks={chunks} blocks={blocks} chunk_min={cmin}", flush=True)
    sn.check(sn.lib().sinter_op_attn_decode(C.byref(a), blocks, C.c_void_p(stream(torch))), "attn")
    torch.cuda.synchronize()
    assert sn.op_error()[0] == 0
    assert np.all(host(cnt) == 1)            # every (kv head, chunk) flag at generation 1
    assert np.array_equal(host(dK)[pos], f["k_row"]) and np.array_equal(host(dV)[pos], f["v_row"])
    got = host(out).reshape(NQ, HD)
    # the oracle's fp32 split over the same rows
    L = orc.lib()
    qr = np.zeros((NQ, HD), np.float32)
    for h in range(NQ):
        L.or_rmsnorm(f["qg"][h * 2 * HD:].ctypes.data, f["q_norm"].ctypes.data, qr[h].ctypes.data, HD, 1e-6)
        L.or_rope_neox(qr[h].ctypes.data, HD, 64, pos, float(f["theta_scale"]))
    Kc, Vc = f["kc_in"].copy(), f["vc_in"].copy()
    Kc[pos], Vc[pos] = f["k_row"], f["v_row"]
    att = np.zeros((NQ, HD), np.float32)
    L.or_attn_split(qr.ctypes.data, Kc.ctypes.data, Vc.ctypes.data, orc.F16, pos + 1, NQ, NKV, HD, 0.0625, chunks,
                    cmin, att.ctypes.data)
    gate = f["qg"].reshape(NQ, 2, HD)[:, 1]
    sig = np.array([[L.or_sigmoid(float(gate[h, i])) for i in range(HD)] for h in range(NQ)], np.float32)
    assert np.array_equal(got, (att * sig).astype(np.float32))
    assert np.linalg.norm(got - f["out"]) <= 1e-5 * np.linalg.norm(f["out"])
