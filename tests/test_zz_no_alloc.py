"""sinter_op_attn_decode_noalloc against sinter_op_attn_decode (GPU).

The no-allocation entry point keeps its split-K partials and generation
flags in the library's fixed device array; its outputs (the gated attention
output and the appended K/V rows) must equal, bit for bit, those of the
existing entry point run on caller-allocated workspace from the same inputs.
Two calls in a row, the second smaller (fewer positions, fewer chunks, a
different GQA shape), then the first shape again; sizes past the array's
maximum are refused before anything runs.
"""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def make_case(sn, orc, torch, nq, nkv, pos, n_ctx, chunks, seed):
    HD = 256
    RW = nkv * HD
    rng = np.random.default_rng(seed)
    qg = (rng.standard_normal(nq * 2 * HD) * 2).astype(np.float32)
    k = rng.standard_normal(RW).astype(np.float32)
    v = rng.standard_normal(RW).astype(np.float32)
    qn = (1 + 0.02 * rng.standard_normal(HD)).astype(np.float32)
    kn = (1 + 0.02 * rng.standard_normal(HD)).astype(np.float32)
    K = np.zeros((n_ctx, RW), np.float16)
    V = np.zeros((n_ctx, RW), np.float16)
    K[:pos] = rng.standard_normal((pos, RW))
    V[:pos] = rng.standard_normal((pos, RW))
    ts = orc.lib().or_rope_theta_scale(1e7, 64)

    def d(a):
        return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")
    keep = dict(qg=d(qg), k=d(k), v=d(v), qn=d(qn), kn=d(kn), cell=d(np.array([0, pos, 0, 0], np.int32)))
    bufs = []
    for _ in range(2):   # one set of caches/outputs per entry point
        bufs.append(dict(K=d(K.view(np.uint16)), V=d(V.view(np.uint16)),
                         out=torch.zeros(nq * HD, dtype=torch.float32, device="cuda")))
    a = sn.AttnArgs(nq=nq, nkv=nkv, hd=HD, rope_dims=64, n_ctx=n_ctx, n_chunks=chunks, theta_scale=ts, eps=1e-6,
                    scale=0.0625)
    a.qg, a.k, a.v = keep["qg"].data_ptr(), keep["k"].data_ptr(), keep["v"].data_ptr()
    a.q_norm, a.k_norm, a.pass_cell = keep["qn"].data_ptr(), keep["kn"].data_ptr(), keep["cell"].data_ptr()
    return a, keep, bufs


def run_pair(sn, orc, torch, nq, nkv, pos, n_ctx, chunks, seed):
    a, keep, bufs = make_case(sn, orc, torch, nq, nkv, pos, n_ctx, chunks, seed)
    st = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    L = sn.lib()
    # the existing entry point on caller workspace
    part = torch.zeros(L.sinter_attn_part_len(nq, nkv, 256, chunks), dtype=torch.float32, device="cuda")
    cnt = torch.zeros(L.sinter_attn_count_len(nkv, chunks), dtype=torch.int32, device="cuda")
    a.kc, a.vc, a.out = bufs[0]["K"].data_ptr(), bufs[0]["V"].data_ptr(), bufs[0]["out"].data_ptr()
    a.part, a.count = part.data_ptr(), cnt.data_ptr()
    print(f"attn workspace nq={nq} nkv={nkv} pos={pos} chunks={chunks}", flush=True)
    sn.check(L.sinter_op_attn_decode(C.byref(a), 256, st), "attn")
    torch.cuda.synchronize()
    assert sn.op_error()[0] == 0
    # the no-allocation entry point
    a.kc, a.vc, a.out = bufs[1]["K"].data_ptr(), bufs[1]["V"].data_ptr(), bufs[1]["out"].data_ptr()
    a.part, a.count = None, None
    print(f"attn noalloc nq={nq} nkv={nkv} pos={pos} chunks={chunks}", flush=True)
    sn.check(L.sinter_op_attn_decode_noalloc(C.byref(a), 256, st), "attn_noalloc")
    torch.cuda.synchronize()
    assert sn.op_error()[0] == 0
    for key in ("out", "K", "V"):
        assert torch.equal(bufs[0][key], bufs[1][key]), key
    return bufs[1]["out"].cpu().numpy()


def test_noalloc_attention_equals_workspace_entry_point(sn, orc, torch_gpu):
    torch = torch_gpu
    first = run_pair(sn, orc, torch, 24, 4, 4095, 4096, 64, 1)      # 256 items, the model's shape
    second = run_pair(sn, orc, torch, 8, 2, 700, 1024, 9, 2)        # smaller: 18 items, gqa 4
    assert first.size == 24 * 256 and second.size == 8 * 256
    again = run_pair(sn, orc, torch, 24, 4, 4095, 4096, 64, 1)      # the first shape after the smaller one
    assert np.array_equal(first, again)


def test_noalloc_attention_refuses_what_it_cannot_hold(sn, orc, torch_gpu):
    torch = torch_gpu
    L = sn.lib()
    a, keep, bufs = make_case(sn, orc, torch, 64, 8, 100, 256, 32, 3)   # 8*32*8*260*4 B > 2 MiB of partials
    a.kc, a.vc, a.out = bufs[0]["K"].data_ptr(), bufs[0]["V"].data_ptr(), bufs[0]["out"].data_ptr()
    st = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert L.sinter_op_attn_decode_noalloc(C.byref(a), 256, st) == sn.ERR_ARG
    assert b"scratch maximum" in L.sinter_last_error()
    a.n_chunks = 8
    dummy = torch.zeros(16, dtype=torch.float32, device="cuda")
    a.part = dummy.data_ptr()                  # workspace is the library's: refused
    assert L.sinter_op_attn_decode_noalloc(C.byref(a), 256, st) == sn.ERR_ARG
    torch.cuda.synchronize()
