"""GPU parity of the batched GEMV over a ubatch of tokens
(sinter_op_gemv_ubatch, the trunk GEMM of a batched prefill) against the CPU
oracle.  Each token's outputs must equal the oracle's single-token GEMV of
that token bit for bit: the kernel computes the integer dot products on
int8 MFMA, but the fp64 item terms and their fold in item order are the
oracle's (oracle/oracle.c or_block_term / or_gemv_q), and the single-token
device GEMV is bit-exact against the same oracle (test_gpu_ops.py).

Shapes cover one token, token counts that are not a multiple of the 16-token
tile or of the 64-token weight pass, row counts that are not a multiple of
the 16-row tile, odd block counts per row (Q6_K's 210-byte blocks then start
on both 4-byte phases), K up to 17408, zero activations and activations over
six decades of scale.  A second test fills the weight blocks with random
bytes (every scale, min and code pattern, Q6_K's -128 scale included) with
finite f16 block scales.

The ubatch Q8_K quantiser (sinter_quant_q8k_ubatch) is compared byte for
byte with the oracle's (or_quant_q8_K: ggml quantize_row_q8_K_ref), over an
all-zero block, a block of tied |x| whose first largest element sets the
sign, and magnitudes from 1e-4 to 1e4; chained with the batched GEMV it must
reproduce the oracle's f32 GEMV of every token.
"""
import ctypes as C

import numpy as np
import pytest

from test_gpu_ops import dev, empty_f32, host, stream, synth_w, xvec

pytestmark = pytest.mark.gpu

Q4_K, Q6_K = 12, 14


def activations(k, n_tok, seed):
    xs = []
    for j in range(n_tok):
        if j % 11 == 5:
            xs.append(np.zeros(k, np.float32))          # d = 0: every term is 0
        else:
            x = xvec(k, seed + j, zero_block=(j % 3 == 0))
            xs.append((x * np.float32(10.0 ** ((j % 7) - 3))).astype(np.float32))
    return xs


def run_ubatch(sn, orc, torch, t, w, rows, k, xs):
    n_tok = len(xs)
    xq = np.concatenate([orc.quantize(t, x) for x in xs])
    dw, dxq, dy = dev(torch, w), dev(torch, xq), empty_f32(torch, n_tok * rows)
    print(f"gemv_ubatch type={t} rows={rows} k={k} tokens={n_tok}", flush=True)
    rc = sn.lib().sinter_op_gemv_ubatch(t, C.c_void_p(dw.data_ptr()), rows, k, C.c_void_p(dxq.data_ptr()),
                                        n_tok, C.c_void_p(dy.data_ptr()), 0, C.c_void_p(stream(torch)))
    sn.check(rc, "gemv_ubatch")
    torch.cuda.synchronize()
    return host(dy).reshape(n_tok, rows)


@pytest.mark.parametrize("t,rows,k,n_tok", [
    (Q4_K, 48, 256, 1), (Q4_K, 100, 5120, 5), (Q4_K, 1024, 5120, 64), (Q4_K, 300, 6144, 70),
    (Q4_K, 33, 17408, 17),
    (Q6_K, 48, 5120, 1), (Q6_K, 37, 768, 33), (Q6_K, 256, 17408, 16), (Q6_K, 130, 1280, 129)])
def test_gemv_ubatch_matches_per_token_gemv(sn, orc, torch_gpu, t, rows, k, n_tok):
    w = synth_w(sn, t, rows, k, 500 + t + k + rows)
    xs = activations(k, n_tok, 1000 + rows)
    got = run_ubatch(sn, orc, torch_gpu, t, w, rows, k, xs)
    for j, x in enumerate(xs):
        assert np.array_equal(got[j], orc.gemv(t, w, rows, k, x)), j


@pytest.mark.parametrize("t,rows,k,n_tok", [
    (Q4_K, 16384, 512, 100),    # 256 row tiles: four token tiles per workgroup, the last group three
    (Q4_K, 8192, 512, 64),      # 128 row tiles: two token tiles per workgroup
    (Q6_K, 16384, 512, 100),
    (Q6_K, 8192, 768, 40)])     # two token tiles per workgroup, the last group one
def test_gemv_ubatch_multi_tile_workgroups(sn, orc, torch_gpu, t, rows, k, n_tok):
    """Shapes with enough row tiles that a workgroup takes several 16-token
    tiles (its waves staging tiles 1-3, a partial last token group): the
    production shapes of a batched prefill run this path."""
    w = synth_w(sn, t, rows, k, 700 + t + k + rows)
    xs = activations(k, n_tok, 2000 + rows)
    got = run_ubatch(sn, orc, torch_gpu, t, w, rows, k, xs)
    for j, x in enumerate(xs):
        assert np.array_equal(got[j], orc.gemv(t, w, rows, k, x)), j


@pytest.mark.parametrize("t", [Q4_K, Q6_K])
def test_gemv_ubatch_random_block_bytes(sn, orc, torch_gpu, t):
    rows, k, n_tok = 80, 2304, 23           # 9 blocks per row
    rng = np.random.default_rng(77 + t)
    w = rng.integers(0, 256, sn.row_bytes(t, k) * rows, dtype=np.uint8)
    blocks = w.reshape(rows * (k // 256), sn.BLOCK_BYTES[t])
    d = rng.standard_normal((blocks.shape[0], 2)).astype(np.float16)
    if t == Q4_K:
        blocks[:, 0:4] = d.view(np.uint8)            # d, dmin
    else:
        blocks[:, 208:210] = d[:, :1].view(np.uint8)  # d
    xs = activations(k, n_tok, 3000 + t)
    got = run_ubatch(sn, orc, torch_gpu, t, w, rows, k, xs)
    for j, x in enumerate(xs):
        assert np.array_equal(got[j], orc.gemv(t, w, rows, k, x)), j


def quant_inputs(k, n_tok, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n_tok, k)).astype(np.float32)
    x[0, :256] = 0.0                                    # an all-zero block
    if k >= 512:
        x[0, 256:512] = 0.5 * np.sign(x[0, 256:512])       # every |x| tied: the first element sets the sign
        x[0, 300] = -3.0                                 # a tie between the first and a later larger |x|
        x[0, 400] = 3.0
    for t in range(1, n_tok):
        x[t] *= np.float32(10.0 ** ((t % 9) - 4))         # 1e-4 .. 1e4
    return x


@pytest.mark.parametrize("k,n_tok", [(256, 1), (5120, 7), (17408, 33)])
def test_quant_q8k_ubatch_matches_oracle(sn, orc, torch_gpu, k, n_tok):
    torch = torch_gpu
    x = quant_inputs(k, n_tok, 40 + k)
    dx = dev(torch, x.reshape(-1))
    dq = torch.zeros(n_tok * sn.row_bytes(sn.Q8_K, k), dtype=torch.uint8, device="cuda")
    print(f"quant_q8k_ubatch k={k} tokens={n_tok}", flush=True)
    sn.check(sn.lib().sinter_quant_q8k_ubatch(C.c_void_p(dx.data_ptr()), k, n_tok, C.c_void_p(dq.data_ptr()),
                                              C.c_void_p(stream(torch))), "quant_q8k_ubatch")
    torch.cuda.synchronize()
    got = host(dq).reshape(n_tok, -1)
    for t in range(n_tok):
        assert np.array_equal(got[t], orc.quantize(Q4_K, x[t])), t


@pytest.mark.parametrize("t,rows,k,n_tok", [(Q4_K, 200, 5120, 40), (Q6_K, 96, 17408, 20)])
def test_device_quantised_ubatch_equals_oracle_gemv(sn, orc, torch_gpu, t, rows, k, n_tok):
    """f32 activations quantised on the device, then the batched GEMV: each
    token's outputs equal the oracle's GEMV of that f32 vector."""
    torch = torch_gpu
    w = synth_w(sn, t, rows, k, 900 + t)
    x = quant_inputs(k, n_tok, 60 + t)
    dw, dx, dy = dev(torch, w), dev(torch, x.reshape(-1)), empty_f32(torch, n_tok * rows)
    dq = torch.zeros(n_tok * sn.row_bytes(sn.Q8_K, k), dtype=torch.uint8, device="cuda")
    s = C.c_void_p(stream(torch))
    print(f"quant + gemv_ubatch type={t} rows={rows} k={k} tokens={n_tok}", flush=True)
    sn.check(sn.lib().sinter_quant_q8k_ubatch(C.c_void_p(dx.data_ptr()), k, n_tok, C.c_void_p(dq.data_ptr()), s),
             "quant")
    sn.check(sn.lib().sinter_op_gemv_ubatch(t, C.c_void_p(dw.data_ptr()), rows, k, C.c_void_p(dq.data_ptr()), n_tok,
                                            C.c_void_p(dy.data_ptr()), 0, s), "gemv_ubatch")
    torch.cuda.synchronize()
    got = host(dy).reshape(n_tok, rows)
    for j in range(n_tok):
        assert np.array_equal(got[j], orc.gemv(t, w, rows, k, x[j])), j


@pytest.mark.parametrize("k,n_tok,weighted", [(5120, 9, True), (17408, 5, False), (6144, 3, True)])
def test_rmsnorm_quant_q8k_ubatch_matches_oracle(sn, orc, torch_gpu, k, n_tok, weighted):
    """RMSNorm (the single-token GEMV's RMSNORM prologue) then Q8_K over a
    ubatch: byte for byte the oracle's or_rmsnorm then or_quant_q8_K."""
    torch = torch_gpu
    x = quant_inputs(k, n_tok, 80 + k)
    x[0, :256] = 0.0
    w = (1.0 + 0.1 * np.random.default_rng(k).standard_normal(k)).astype(np.float32) if weighted else None
    eps = 1e-6
    dx = dev(torch, x.reshape(-1))
    dwt = dev(torch, w) if weighted else None
    dq = torch.zeros(n_tok * sn.row_bytes(sn.Q8_K, k), dtype=torch.uint8, device="cuda")
    print(f"rmsnorm_quant_q8k_ubatch k={k} tokens={n_tok} weighted={weighted}", flush=True)
    sn.check(sn.lib().sinter_rmsnorm_quant_q8k_ubatch(C.c_void_p(dx.data_ptr()),
                                                      C.c_void_p(dwt.data_ptr()) if weighted else None, eps, k, n_tok,
                                                      C.c_void_p(dq.data_ptr()), C.c_void_p(stream(torch))),
             "rmsnorm_quant")
    torch.cuda.synchronize()
    got = host(dq).reshape(n_tok, -1)
    for t in range(n_tok):
        assert np.array_equal(got[t], orc.quantize(Q4_K, orc.rmsnorm(x[t], w, eps))), t


@pytest.mark.parametrize("k", [5120, 2048])
def test_rmsnorm_ubatch_equals_single_token_prologue_wide_range(sn, orc, torch_gpu, k):
    """RMSNorm + Q8_K over a ubatch then the batched GEMV gives, token by
    token, the single-token GEMV with the RMSNORM prologue bit for bit, also
    on rows whose values span 1e-6 .. 1e3 (where an fp64 sum of squares in
    another order can round differently): both sum in the same fixed tree."""
    from test_gpu_ops import run_gemv
    torch = torch_gpu
    rows, T, eps = 700, 6, 1e-6
    rng = np.random.default_rng(k + 3)
    x = rng.standard_normal((T, k)).astype(np.float32)
    x *= (10.0 ** rng.uniform(-6, 3, (T, k))).astype(np.float32)     # nine decades in one row
    wn = (1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    w = synth_w(sn, Q4_K, rows, k, 909 + k)
    dx, dwn, dw = dev(torch, x.reshape(-1)), dev(torch, wn), dev(torch, w)
    dq = torch.zeros(T * sn.row_bytes(sn.Q8_K, k), dtype=torch.uint8, device="cuda")
    dy = empty_f32(torch, T * rows)
    s = C.c_void_p(stream(torch))
    print(f"rmsnorm ubatch vs prologue k={k} tokens={T}", flush=True)
    sn.check(sn.lib().sinter_rmsnorm_quant_q8k_ubatch(C.c_void_p(dx.data_ptr()), C.c_void_p(dwn.data_ptr()), eps, k, T,
                                                      C.c_void_p(dq.data_ptr()), s), "rmsnorm_quant")
    sn.check(sn.lib().sinter_op_gemv_ubatch(Q4_K, C.c_void_p(dw.data_ptr()), rows, k, C.c_void_p(dq.data_ptr()), T,
                                            C.c_void_p(dy.data_ptr()), 0, s), "gemv_ubatch")
    torch.cuda.synchronize()
    got = host(dy).reshape(T, rows)
    for t in range(T):
        dxt, dyt = dev(torch, x[t]), empty_f32(torch, rows)
        a = sn.GemvArgs(K=k, pro=sn.PRO_RMSNORM, n_seg=1, eps=eps)
        a.x, a.norm_w = dxt.data_ptr(), dwn.data_ptr()
        a.seg[0] = sn.GemvSeg(w=dw.data_ptr(), y=dyt.data_ptr(), rows=rows, type=Q4_K, epi=sn.EPI_STORE)
        run_gemv(sn, torch, a, 256)
        assert np.array_equal(got[t], host(dyt)), t


def test_batched_ffn_block_matches_oracle(sn, orc, torch_gpu):
    """The FFN sub-layer over a ubatch from the batched pieces -- RMSNorm +
    Q8_K, the gate and up GEMVs, SwiGLU + Q8_K, the down GEMV accumulated
    into the residual -- equals, token by token, the oracle's
    x + or_ffn(or_rmsnorm(x, post_norm)) (oracle/oracle.c or_ffn)."""
    torch = torch_gpu
    E, F, T, eps = 1024, 2048, 21, 1e-6
    rng = np.random.default_rng(5)
    x = rng.standard_normal((T, E)).astype(np.float32)
    wn = (1.0 + 0.1 * rng.standard_normal(E)).astype(np.float32)
    wg, wu = synth_w(sn, Q4_K, F, E, 1201), synth_w(sn, Q4_K, F, E, 1202)
    wd = synth_w(sn, Q6_K, E, F, 1203)
    d = {n: dev(torch, a) for n, a in (("x", x.reshape(-1)), ("wn", wn), ("wg", wg), ("wu", wu), ("wd", wd))}
    g, u = empty_f32(torch, T * F), empty_f32(torch, T * F)
    xq = torch.zeros(T * sn.row_bytes(sn.Q8_K, E), dtype=torch.uint8, device="cuda")
    fq = torch.zeros(T * sn.row_bytes(sn.Q8_K, F), dtype=torch.uint8, device="cuda")
    L, s = sn.lib(), C.c_void_p(stream(torch))
    ptr = lambda t: C.c_void_p(t.data_ptr())  # noqa: E731
    print(f"batched ffn E={E} F={F} tokens={T}", flush=True)
    sn.check(L.sinter_rmsnorm_quant_q8k_ubatch(ptr(d["x"]), ptr(d["wn"]), eps, E, T, ptr(xq), s), "norm")
    sn.check(L.sinter_op_gemv_ubatch(Q4_K, ptr(d["wg"]), F, E, ptr(xq), T, ptr(g), 0, s), "gate")
    sn.check(L.sinter_op_gemv_ubatch(Q4_K, ptr(d["wu"]), F, E, ptr(xq), T, ptr(u), 0, s), "up")
    sn.check(L.sinter_swiglu_quant_q8k_ubatch(ptr(g), ptr(u), F, T, ptr(fq), s), "swiglu")
    sn.check(L.sinter_op_gemv_ubatch(Q6_K, ptr(d["wd"]), E, F, ptr(fq), T, ptr(d["x"]), 1, s), "down + residual")
    torch.cuda.synchronize()
    got = host(d["x"]).reshape(T, E)

    cfg = orc.Cfg()
    cfg.n_embd, cfg.n_ff, cfg.t_default, cfg.t_ffn_down = E, F, Q4_K, Q6_K
    slots = (C.c_void_p * orc.NSLOT)()
    slots[2], slots[3], slots[4] = wg.ctypes.data, wu.ctypes.data, wd.ctypes.data   # FFN gate, up, down
    for t in range(T):
        xn = orc.rmsnorm(x[t], wn, eps)
        a = np.zeros(E, np.float32)
        orc.lib().or_ffn(C.byref(cfg), slots, orc.P(xn), orc.P(a))
        assert np.array_equal(got[t], x[t] + a), t


@pytest.mark.parametrize("d,k,n_tok", [(128, 4096, 6), (64, 768, 3), (256, 1024, 2)])
def test_gated_rmsnorm_quant_q8k_ubatch_matches_oracle(sn, orc, torch_gpu, d, k, n_tok):
    """Per-head gated RMSNorm then Q8_K over a ubatch: byte for byte the
    oracle's or_gated_rmsnorm then or_quant_q8_K."""
    torch = torch_gpu
    rng = np.random.default_rng(d + k)
    x = quant_inputs(k, n_tok, 90 + d)
    x[0, :d] = 0.0                                       # an all-zero head
    z = (2.0 * rng.standard_normal((n_tok, k))).astype(np.float32)
    w = (1.0 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    eps = 1e-6
    dx, dz, dw = dev(torch, x.reshape(-1)), dev(torch, z.reshape(-1)), dev(torch, w)
    dq = torch.zeros(n_tok * sn.row_bytes(sn.Q8_K, k), dtype=torch.uint8, device="cuda")
    print(f"gated_rmsnorm_quant_q8k_ubatch d={d} k={k} tokens={n_tok}", flush=True)
    sn.check(sn.lib().sinter_gated_rmsnorm_quant_q8k_ubatch(C.c_void_p(dx.data_ptr()), C.c_void_p(dz.data_ptr()),
                                                            C.c_void_p(dw.data_ptr()), d, eps, k, n_tok,
                                                            C.c_void_p(dq.data_ptr()), C.c_void_p(stream(torch))),
             "gated_rmsnorm_quant")
    torch.cuda.synchronize()
    got = host(dq).reshape(n_tok, -1)
    for t in range(n_tok):
        y = np.zeros(k, np.float32)
        orc.lib().or_gated_rmsnorm(orc.P(x[t]), orc.P(z[t]), orc.P(w), orc.P(y), k // d, d, eps)
        assert np.array_equal(got[t], orc.quantize(Q4_K, y)), t


@pytest.mark.parametrize("channels,dconv,n_tok", [(8192, 4, 37), (300, 2, 5), (64, 1, 3)])
def test_conv_silu_ubatch_matches_oracle_token_loop(sn, orc, torch_gpu, channels, dconv, n_tok):
    """The causal conv + silu over a ubatch equals the oracle's or_conv_silu
    applied token after token: every output row and the final state, bit for
    bit."""
    torch = torch_gpu
    rng = np.random.default_rng(channels + dconv)
    x = rng.standard_normal((n_tok, channels)).astype(np.float32)
    st = (0.5 * rng.standard_normal(channels * max(dconv - 1, 1))).astype(np.float32)[:channels * (dconv - 1)]
    cw = (0.3 * rng.standard_normal(channels * dconv)).astype(np.float32)
    dx, dcw, dy = dev(torch, x.reshape(-1)), dev(torch, cw), empty_f32(torch, n_tok * channels)
    dst = dev(torch, st) if dconv > 1 else None
    print(f"conv_silu_ubatch channels={channels} dconv={dconv} tokens={n_tok}", flush=True)
    sn.check(sn.lib().sinter_conv_silu_ubatch(C.c_void_p(dx.data_ptr()), C.c_void_p(dst.data_ptr()) if dst is not None
                                              else None, C.c_void_p(dcw.data_ptr()), C.c_void_p(dy.data_ptr()),
                                              channels, dconv, n_tok, C.c_void_p(stream(torch))), "conv_silu")
    torch.cuda.synchronize()
    got = host(dy).reshape(n_tok, channels)
    ref_st = st.copy()
    for t in range(n_tok):
        out = np.zeros(channels, np.float32)
        orc.lib().or_conv_silu(orc.P(x[t]), orc.P(ref_st) if dconv > 1 else None, orc.P(cw), orc.P(out), channels,
                               dconv)
        assert np.array_equal(got[t], out), t
    if dconv > 1:
        assert np.array_equal(host(dst), ref_st)
