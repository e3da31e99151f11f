"""Batch-1 greedy decode benchmark of the Qwen3.6-27B-shaped hybrid model on
one MI355X (64 layers = 48 gated-DeltaNet + 16
attention, Q4_K_M-style mix, 4096-token context).

A step is one decode pass (one token).  Weights are synthetic random-init
(generated on the device); the 4096-token context is a seeded synthetic KV
cache / recurrent state.  W warmup tokens (one launch), then K tokens timed
as launches of --passes-per-launch greedy passes of the cooperative
interpreter (each call returns once its launch has finished).  Prints one
JSON line.  --config selects the other BASELINE configs (1-3: single op
groups; 5: bf16 at 131072 positions).

The roofline object prices the algorithmic bytes per token (weights read
once, KV rows read once, recurrent state read+written, logits written)
against 8 TB/s, using the interpreter kernel's own duration measured with HIP
events recorded on its launch stream.  cpu_baseline times the CPU oracle
(the repository's restatement of ggml's CPU semantics, OpenMP over rows) on
a bounded sample of the same decode.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "sinter-qwen36-nomtp-tu102_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

METRIC = "batch-1 decode tok/s, 27B-shaped Q4_K @4k ctx; achieved HBM GB/s vs peak"
PEAK_GBS = 8000.0


def bytes_per_token(cfg, m, n_attended):
    """Algorithmic HBM bytes of one decode pass at n_attended KV positions."""
    import sinter
    n_attn = sum(1 for il in range(cfg.n_layer) if il % cfg.attn_every == cfg.attn_every - 1)
    n_gdn = cfg.n_layer - n_attn
    wb = m.info()["weight_bytes"]
    _, emb_bytes, emb_type = m.tensor(cfg.n_layer, 0)
    weights = wb - emb_bytes + sinter.row_bytes(emb_type, cfg.n_embd)      # one embedding row
    D = cfg.gdn_d
    C = (2 * cfg.gdn_hk + cfg.gdn_hv) * D
    gdn_state = n_gdn * cfg.gdn_hv * D * D * 4 * 2                         # read + write
    conv_state = n_gdn * C * (cfg.conv_k - 1) * 4 * 2
    rw = cfg.attn_nkv * cfg.head_dim
    kv_row = n_attn * 2 * rw * 2                                             # K and V, f16
    logits = cfg.n_vocab * 4
    return {"weights": weights, "gdn_state": gdn_state, "conv_state": conv_state,
            "kv_read": kv_row * n_attended, "kv_append": kv_row, "logits": logits,
            "total": weights + gdn_state + conv_state + kv_row * n_attended + kv_row + logits}


TRAFFIC_SUMMARY = os.path.join(ROOT, "profiles", "traffic_sinter_interp_kquant_e2e_q4km_ctx4096.md")


HBM_PEAK_BYTES, HBM_PEAK_REPS = 2 << 30, 5


def measured_peak():
    """The box's measured HBM bandwidth (sinter_hbm_peak: a library read
    stream and a copy over a 2 GiB buffer, far past the 256 MB memory-side
    cache, 5 timed passes each): {"read": GB/s, "copy": GB/s}."""
    import ctypes as C
    import sinter
    r, c = C.c_double(), C.c_double()
    sinter.check(sinter.lib().sinter_hbm_peak(HBM_PEAK_BYTES, HBM_PEAK_REPS, C.byref(r), C.byref(c)), "hbm_peak")
    return {"read": round(r.value, 1), "copy": round(c.value, 1)}


def roofline_peaks(achieved):
    """roofline fields for the measured peak (the decode reads ~97 % of its
    bytes, so the read stream is its practical ceiling)"""
    pk = measured_peak()
    return {"peak_measured": pk["read"], "frac_measured": round(achieved / pk["read"], 4),
            "peak_measured_how": f"sinter_hbm_peak read stream, {HBM_PEAK_BYTES >> 30} GiB x {HBM_PEAK_REPS} "
                                 f"(copy: {pk['copy']} GB/s read+written)"}


def kernel_source_digest():
    """sha256 of the interpreter's sources (interp.hip and the csrc/*.h
    headers, sorted by name) and of the compiler flags it is built with
    (build.py FLAGS): the traffic summary records the digest of the build it
    was measured on.  Other translation units of the library (the batched
    GEMV) do not enter it: they are separate code objects."""
    import hashlib
    import importlib.util
    pkg = os.path.join(ROOT, "sinter-qwen36-nomtp-tu102_amd")
    d = os.path.join(pkg, "csrc")
    h = hashlib.sha256()
    files = [os.path.join(d, fn) for fn in sorted(os.listdir(d)) if fn.endswith(".h") or fn == "interp.hip"]
    for path in files:
        h.update(os.path.basename(path).encode())
        with open(path, "rb") as f:
            h.update(f.read())
    spec = importlib.util.spec_from_file_location("sinter_build_flags", os.path.join(pkg, "build.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    h.update(("FLAGS:" + "\x00".join(mod.FLAGS)).encode())
    return h.hexdigest()


def measured_traffic(passes_per_launch, quant, ctx):
    """(HBM bytes per launch of the interpreter, the commit it was measured
    at) from the committed counter summary (FETCH_SIZE + WRITE_SIZE per pass,
    scaled against a copy kernel of known size); (None, None) when no summary
    exists, when it was measured on other kernel sources than these (a stale
    figure), or when the run is not the summarised workload (q4_k_m weights,
    4096-token context)."""
    if quant != "q4_k_m" or ctx != 4096:
        return None, None
    fields = {}
    try:
        with open(TRAFFIC_SUMMARY) as f:
            for line in f:
                for key in ("traffic_bytes_per_pass", "kernel_sources_sha256", "measured_at_commit"):
                    if line.startswith(key + ":"):
                        fields[key] = line.split(":", 1)[1].strip()
    except OSError:
        return None, None
    if "traffic_bytes_per_pass" not in fields or fields.get("kernel_sources_sha256") != kernel_source_digest():
        return None, None
    return round(float(fields["traffic_bytes_per_pass"]) * passes_per_launch), fields.get("measured_at_commit")


CPU_LABEL = "ggml-semantics CPU restatement (oracle/oracle.c: ggml's quantisers and block dots, OpenMP over rows"


def cpu_threads():
    return int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))


def cpu_isa():
    import oracle
    return "AVX-512 row kernels" if oracle.lib().or_row_isa() == 512 else "baseline-ISA row kernels"


def median_timed(fn, runs=5, warmup=1):
    """Median wall time (s) of fn over `runs` calls after `warmup` calls."""
    import numpy as np
    for _ in range(warmup):
        fn()
    ts = []
    for _ in range(runs):
        s = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - s)
    return float(np.median(ts)), ts


def cpu_baseline(m, ctx, seconds):
    """Time the CPU oracle decoding from the same synthetic context: one
    warmup step, then at least 5 timed steps (more while `seconds` lasts);
    the rate is 1 / the median step time."""
    import numpy as np
    import oracle
    t0 = time.perf_counter()
    mirror = oracle.ModelMirror(m)
    copy_s = time.perf_counter() - t0
    state = {"tok": 1, "pos": ctx}

    def step():
        state["tok"], _ = mirror.step(state["tok"], state["pos"])
        state["pos"] += 1
    step()   # warmup
    ts, spent = [], 0.0
    while len(ts) < 5 or spent < seconds:
        s = time.perf_counter()
        step()
        ts.append(time.perf_counter() - s)
        spent += ts[-1]
    med = float(np.median(ts))
    threads = cpu_threads()
    return {"value": round(1.0 / med, 4), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"{CPU_LABEL}, {cpu_isa()}, {threads} threads): greedy decode steps of the same model "
                      f"from position {ctx}, 1 warmup + {len(ts)} timed, median {med * 1e3:.1f} ms/step "
                      f"(weights copied to host in {copy_s:.1f} s)"}


OP_CONFIGS = {
    1: ("Q8_0 GEMV y = W x, W 17408x5120 (ffn_gate shape), x fp32[5120], y fp32[17408]", 4),
    2: ("gated-DeltaNet layer mixer: RMSNorm, Q4_K qkv 8192 / z 4096 / alpha, beta 32 x 5120, causal conv 4, "
        "l2 norms, gates, delta-rule step on 32 x 128x128 fp32 state, gated RMSNorm, Q4_K out 5120x4096, residual", 6),
    3: ("attention layer mixer: RMSNorm, Q4_K q|gate 12288 / k 1024 and Q6_K v 1024 x 5120, q/k RMSNorm, "
        "NEOX RoPE 64/256, f16 KV append, split-K GQA decode 24q/4kv over the cache, sigmoid gate, "
        "Q4_K out 5120x6144, residual", 4),
}
GDN_SLOTS, ATTN_SLOTS = (0, 5, 6, 7, 8, 9, 10, 11, 12, 13), (0, 5, 6, 7, 8, 9, 10)


def op_bench(args):
    """one op group (a GEMV, a GDN mixer, an attention
    mixer) per layer of a synthetic model, consecutive groups on different
    weight copies (>= 4, past the 256 MB MALL), each group after a grid
    barrier as in the decode (sinter_model_bench_program).  Reports the
    median per-group time over timed launches."""
    import ctypes as C
    import numpy as np
    import sinter
    c = args.config
    desc, n_inst = OP_CONFIGS[c]
    ctx = args.ctx if c == 3 else 0
    cfg = sinter.qwen36_27b_config(n_ctx=max(ctx, 64), quant="q4_k_m", n_layer=n_inst)
    cfg.n_vocab = 512
    cfg.attn_every = 1 if c == 3 else 0
    cfg.attn_chunk_min = args.attn_chunk_min
    if c == 1:
        cfg.t_default = sinter.Q8_0
    t0 = time.perf_counter()
    m = sinter.Model(cfg, seed=args.seed)
    m.synth_context(max(ctx - 1, 0), seed=args.seed + 1)
    m.bench_program(c, seed=args.seed + 2)
    print(f"# config {c}: model ready in {time.perf_counter() - t0:.1f} s", file=sys.stderr, flush=True)
    pos = max(ctx - 1, 0)
    ppl = max(1, args.passes_per_launch)
    for _ in range(2):
        m.time_passes(pos, ppl)
    launches = max(5, args.steps // ppl)
    ms = [m.time_passes(pos, ppl) for _ in range(launches)]
    us = float(np.median(ms)) * 1e3 / (ppl * n_inst)
    # algorithmic bytes of one group
    E = cfg.n_embd
    if c == 1:
        _, wbytes, _ = m.tensor(0, 2)
        nbytes = wbytes + E * 4 + cfg.n_ff * 4
        parts = {"weights": wbytes, "x": E * 4, "y": cfg.n_ff * 4}
    elif c == 2:
        wbytes = sum(m.tensor(0, s)[1] for s in GDN_SLOTS)
        D, C_ = cfg.gdn_d, (2 * cfg.gdn_hk + cfg.gdn_hv) * cfg.gdn_d
        state = cfg.gdn_hv * D * D * 4 * 2
        conv = C_ * (cfg.conv_k - 1) * 4 * 2
        nbytes = wbytes + state + conv + 2 * E * 4
        parts = {"weights": wbytes, "ssm_state_rw": state, "conv_state_rw": conv, "x_and_out": 2 * E * 4}
    else:
        wbytes = sum(m.tensor(0, s)[1] for s in ATTN_SLOTS)
        kv_row = cfg.attn_nkv * cfg.head_dim * 2 * 2
        nbytes = wbytes + kv_row * (pos + 1) + kv_row + 2 * E * 4
        parts = {"weights": wbytes, "kv_read": kv_row * (pos + 1), "kv_append": kv_row, "x_and_out": 2 * E * 4}
    achieved = nbytes / (us * 1e-6) / 1e9
    line = {
        "metric": f"config {c}: {desc}; time per op group (after its grid barrier) and achieved HBM GB/s vs peak",
        "value": round(us, 3), "unit": "us", "n_gpus": 1, "steps": launches * ppl * n_inst, "warmup": 2 * ppl * n_inst,
        "ms_per_step": round(us / 1e3, 6), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8" if c == 1 else "int8/f32", "data": "synthetic (seeded random-init weights, x ~ N(0,1), "
        "states N(0,0.1), f16 KV N(0,1))",
        "config": {"workload": f"BASELINE config {c}", "instances_rotated": n_inst, "context": ctx if c == 3 else None,
                   "passes_per_launch": ppl, "launches": launches, "bytes_per_op": nbytes, "bytes_breakdown": parts},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_GBS, 4), "traffic": None, "kernel": m.info()["kernel"],
                     "roofline_us": round(nbytes / (PEAK_GBS * 1e9) * 1e6, 3)},
    }
    line["roofline"].update(roofline_peaks(achieved))
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = op_cpu_baseline(m, c, pos)
    m.close()
    print(json.dumps(line), flush=True)


UBATCH_MATS = (  # one gated-DeltaNet layer's trunk matrices in the Q4_K_M mix: (name, type, rows, k)
    ("ssm_qkv", 12, 8192, 5120), ("ssm_z", 12, 4096, 5120), ("ssm_beta", 12, 32, 5120),
    ("ssm_alpha", 12, 32, 5120), ("ssm_out", 12, 5120, 4096), ("ffn_gate", 12, 17408, 5120),
    ("ffn_up", 12, 17408, 5120), ("ffn_down", 14, 5120, 17408))
MFMA_INT8_PEAK_TOPS = 5000.0


def ubatch_bench(args):
    """The batched GEMV of a batched prefill (sinter_op_gemv_ubatch) over one
    gated-DeltaNet layer's trunk matrices (qkv, z, beta, alpha, out, gate,
    up, down: 220.8 MB at Q4_K / Q6_K) for a ubatch of --ubatch tokens.  A
    step is the eight launches over one of >= 4 rotated weight copies (past
    the 256 MB memory-side cache).  Weights are synthetic (seeded, on the
    device), activations seeded Q8_K blocks; results are bit-identical per
    token to the single-token GEMV (tests/test_gpu_ubatch.py).  The roofline
    is int8 MFMA: the integer multiply-adds of the step over its time."""
    import ctypes as C
    import numpy as np
    import torch
    import sinter
    L = sinter.lib()
    T = args.ubatch
    s = torch.cuda.current_stream()
    sp = C.c_void_p(s.cuda_stream)
    layer_bytes = sum(sinter.row_bytes(t, k) * r for _, t, r, k in UBATCH_MATS)
    n_copy = max(4, int(np.ceil(1.0e9 / layer_bytes)))
    copies = []
    for c in range(n_copy):
        mats = []
        for j, (_, t, r, k) in enumerate(UBATCH_MATS):
            w = torch.empty(sinter.row_bytes(t, k) * r, dtype=torch.uint8, device="cuda")
            sinter.check(L.sinter_synth(1, C.c_void_p(w.data_ptr()), 0, t, r, k, args.seed + 97 * c + j, 0, 0, sp),
                         "synth")
            mats.append(w)
        copies.append(mats)
    rng = np.random.default_rng(args.seed)
    xq = {}
    for k in sorted({k for _, _, _, k in UBATCH_MATS}):
        nb = k // 256
        blk = np.zeros((T * nb, 292), np.uint8)
        blk[:, 0:4] = (np.abs(rng.standard_normal((T * nb, 1))) * 0.01 + 1e-3).astype(np.float32).view(np.uint8)
        blk[:, 4:260] = rng.integers(-127, 128, (T * nb, 256)).astype(np.int8).view(np.uint8)
        xq[k] = torch.from_numpy(blk.reshape(-1)).cuda()
    ys = [torch.empty(T * r, dtype=torch.float32, device="cuda") for _, _, r, _ in UBATCH_MATS]

    def launch(c, j):
        _, t, r, k = UBATCH_MATS[j]
        sinter.check(L.sinter_op_gemv_ubatch(t, C.c_void_p(copies[c][j].data_ptr()), r, k,
                                             C.c_void_p(xq[k].data_ptr()), T, C.c_void_p(ys[j].data_ptr()), 0, sp),
                     "gemv_ubatch")

    for i in range(args.warmup):
        for j in range(len(UBATCH_MATS)):
            launch(i % n_copy, j)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    for i in range(args.steps):
        for j in range(len(UBATCH_MATS)):
            launch(i % n_copy, j)
    e1.record(s)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    # per-matrix launch time (events around each launch, a second timed run)
    per = []
    for j, (name, t, r, k) in enumerate(UBATCH_MATS):
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        ev[0].record(s)
        for i in range(args.steps):
            launch(i % n_copy, j)
        ev[1].record(s)
        torch.cuda.synchronize()
        us = ev[0].elapsed_time(ev[1]) / args.steps * 1e3
        per.append({"matrix": name, "type": "Q4_K" if t == 12 else "Q6_K", "rows": r, "k": k, "us": round(us, 2),
                    "tops": round(2.0 * r * k * T / (us * 1e-6) / 1e12, 1)})
    # spot check: ssm_out's outputs of token 0 against the oracle's GEMV over
    # the same quantised activation
    check = None
    try:
        import oracle
        j = 4
        _, t, r, k = UBATCH_MATS[j]
        launch(0, j)
        torch.cuda.synchronize()
        wh = copies[0][j].cpu().numpy()
        xh = xq[k].cpu().numpy()[:sinter.row_bytes(sinter.Q8_K, k)]
        ref = np.zeros(r, np.float32)
        oracle.lib().or_gemv_q(t, oracle.P(wh), r, k, oracle.P(xh), oracle.P(ref))
        check = {"matrix": UBATCH_MATS[j][0], "token": 0, "bit_exact": bool(np.array_equal(ys[j].cpu().numpy()[:r], ref))}
    except ImportError:
        pass
    macs = sum(r * k for _, _, r, k in UBATCH_MATS)
    tops = 2.0 * macs * T / (ms * 1e-3) / 1e12
    line = {
        "metric": "prefill trunk GEMM: tokens/s through one gated-DeltaNet layer's matrices (batched GEMV, "
                  "sinter_op_gemv_ubatch)",
        "value": round(T / (ms * 1e-3), 1), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8 (fp64 item terms)",
        "data": "synthetic (seeded random-init Q4_K / Q6_K weights, seeded Q8_K activations)",
        "config": {"workload": f"ubatch of {T} tokens x one GDN layer's trunk (Qwen3.6-27B shapes, Q4_K_M mix)",
                   "ubatch": T, "weight_bytes_per_step": layer_bytes, "weight_copies_rotated": n_copy,
                   "per_matrix": per, "oracle_spot_check": check},
        "roofline": {"bound": "mfma", "achieved": round(tops, 1), "peak": MFMA_INT8_PEAK_TOPS, "unit": "TOP/s",
                     "frac": round(tops / MFMA_INT8_PEAK_TOPS, 4), "traffic": None,
                     "kernel": "ubatch_gemv_kernel",
                     "weights_gbs": round(layer_bytes / (ms * 1e-3) / 1e9, 1)},
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = ubatch_cpu_baseline(args)
    print(json.dumps(line), flush=True)


def ubatch_cpu_baseline(args):
    """The same layer trunk on the CPU oracle (or_gemv, one token at a time):
    tokens/s over 2 tokens after a warmup token."""
    import numpy as np
    import oracle
    import sinter
    mats = []
    for j, (_, t, r, k) in enumerate(UBATCH_MATS):
        w = np.zeros(sinter.row_bytes(t, k) * r, np.uint8)
        sinter.check(sinter.lib().sinter_synth(0, w.ctypes.data, 0, t, r, k, args.seed + j, 0, 0, None), "synth")
        mats.append(w)
    xs = {k: np.random.default_rng(args.seed + k).standard_normal(k).astype(np.float32)
          for k in {k for _, _, _, k in UBATCH_MATS}}

    def one():
        for j, (_, t, r, k) in enumerate(UBATCH_MATS):
            oracle.gemv(t, mats[j], r, k, xs[k])

    one()
    t0 = time.perf_counter()
    for _ in range(2):
        one()
    sec = (time.perf_counter() - t0) / 2
    threads = cpu_threads()
    return {"value": round(1.0 / sec, 2), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"{CPU_LABEL}, {cpu_isa()}, {threads} threads): or_gemv over the eight matrices per token "
                      f"(Q8_K quantise + rows), 1 warmup + 2 timed tokens, mean {sec * 1e3:.1f} ms/token"}


def op_cpu_baseline(m, c, pos):
    """The same op group on the CPU oracle (layer 0's weights and state),
    median of 5 after a warmup."""
    import ctypes as C
    import numpy as np
    import oracle
    L = oracle.lib()
    rng = np.random.default_rng(7)
    E = m.cfg.n_embd
    x = rng.standard_normal(E).astype(np.float32)
    threads = cpu_threads()
    if c == 1:
        d, nb, t = m.tensor(0, 2)
        w = np.empty(nb, np.uint8)
        m.d2h(w, d, nb)
        med, _ = median_timed(lambda: oracle.gemv(t, w, m.cfg.n_ff, E, x))
        what = "or_gemv (Q8_0 quantise of x + 17408 rows)"
    else:
        mirror = oracle.ModelMirror(m)
        wl = C.c_void_p(C.addressof(mirror.weights))
        st = C.c_void_p(C.addressof(mirror.state))
        out = np.zeros(E, np.float32)
        if c == 2:
            med, _ = median_timed(lambda: L.or_gdn_mixer(C.byref(mirror.cfg), wl, st, oracle.P(x), oracle.P(out), None))
            what = "or_gdn_mixer (projections, conv, step, gated norm, out)"
        else:
            med, _ = median_timed(lambda: L.or_attn_mixer(C.byref(mirror.cfg), wl, st, oracle.P(x), pos,
                                                          oracle.P(out), None))
            what = f"or_attn_mixer (projections, norms, rope, attention over {pos + 1} positions, gate, out)"
    return {"value": round(med * 1e6, 1), "unit": "us", "cores": threads, "kind": "port",
            "sample": f"{CPU_LABEL}, {cpu_isa()}, {threads} threads): {what}, layer 0, 1 warmup + 5 timed, median"}


def single_pass_latency(m, tok, pos, n=8):
    """Per-token latency of one pass per launch (sinter_model_decode: pos and
    token set, one cooperative launch, the next token read back): median wall
    time of n calls, and the median of those launches' own kernel time (HIP
    events on the interpreter's stream)."""
    import numpy as np
    import sinter
    L = sinter.lib()
    ts, ks = [], []
    for i in range(n):
        s = time.perf_counter()
        tok = m.decode(tok, pos + i)
        ts.append(time.perf_counter() - s)
        ks.append(float(L.sinter_host_last_launch_ms(m.host())))
    return float(np.median(ts)) * 1e3, tok, float(np.median(ks))


def parity(m, cfg, args):
    """Greedy decode through the path the benchmark times -- the static GEMV
    load balance, then launches of --passes-per-launch greedy passes of the
    cooperative interpreter -- and through the CPU oracle from the same weights
    and state, step by step.  Every token id must be identical; the logits of
    each launch's last pass must be within rel L2 1e-2 (reported exactly).
    A mismatch ends the check (the two decodes would then follow different
    tokens)."""
    import numpy as np
    import oracle
    t0 = time.perf_counter()
    mirror = oracle.ModelMirror(m)
    copy_s = time.perf_counter() - t0
    tok, pos = 1, args.ctx
    rtok, t_cpu, worst_rel, mism, toks = 1, 0.0, 0.0, 0, []
    n_bal = (args.balance[0] + 1) * args.balance[1] if args.balance[1] else 0
    if n_bal:
        tok, pos = m.balance(tok, pos, args.balance[0], args.balance[1])
        s = time.perf_counter()
        for i in range(n_bal):
            rtok, _ = mirror.step(rtok, args.ctx + i)
        t_cpu += time.perf_counter() - s
        mism += int(tok != rtok)
        print(f"# balance: {n_bal} traced passes, gpu token {tok}, cpu token {rtok}", file=sys.stderr, flush=True)
    ppl = max(1, args.passes_per_launch)
    done = 0
    while done < args.parity_steps and mism == 0:
        n = min(ppl, args.parity_steps - done)
        out = m.greedy(tok, pos, n)
        last = m.logits()
        s = time.perf_counter()
        ref = []
        for i in range(n):
            rtok, rlog = mirror.step(rtok, pos + i)
            ref.append(rtok)
        t_cpu += time.perf_counter() - s
        rel = float(np.linalg.norm(last - rlog) / np.linalg.norm(rlog))
        worst_rel = max(worst_rel, rel)
        mism += sum(int(a != b) for a, b in zip(out, ref))
        print(f"# steps {done}..{done + n - 1}: gpu {out} cpu {ref} last-pass logits rel L2 {rel:.3e}",
              file=sys.stderr, flush=True)
        toks += out
        tok, pos, done = out[-1], pos + n, done + n
    print(json.dumps({"parity_steps": done, "requested": args.parity_steps, "quant": args.quant,
                      "context": args.ctx, "path": f"balance {args.balance[0]}x{args.balance[1]}, "
                      f"greedy launches of {ppl} passes", "token_mismatches": mism,
                      "worst_last_pass_logits_rel_l2": worst_rel, "tokens": toks,
                      "cpu_seconds": round(t_cpu, 1), "mirror_copy_seconds": round(copy_s, 1),
                      "pass": mism == 0 and done == args.parity_steps and worst_rel <= 1e-2}), flush=True)


def prefill_only(m, cfg, args):
    """--prefill-check / --prefill-reps: the batched prefill of a --ctx-token
    prompt alone, optionally checked bit for bit against the decode program
    over the same prompt on a second model of the same weights."""
    import random

    import numpy as np
    import sinter
    rng = random.Random(args.seed + 1)
    prompt = [rng.randrange(cfg.n_vocab) for _ in range(args.ctx)]
    times = []
    tok = None
    for r in range(max(1, args.prefill_reps)):
        t1 = time.perf_counter()
        tok = m.prefill(prompt, 0, mode="batched")
        times.append(time.perf_counter() - t1)
        print(f"# batched prefill {r}: {args.ctx} tokens in {times[-1]:.3f} s; next token {tok}",
              file=sys.stderr, flush=True)
    best = min(times)
    line = {"metric": "prefill tok/s, 27B-shaped Q4_K (batched prefill, ubatch 256)", "value": round(args.ctx / best, 2),
            "unit": "tok/s", "n_gpus": 1, "higher_is_better": True, "tokens": args.ctx,
            "seconds": [round(t, 4) for t in times], "next_token": tok,
            "config": {"workload": f"{args.ctx}-token prompt from position 0, Qwen3.6-27B-shaped hybrid, "
                                   f"{args.quant} weights", "ubatch": sinter.PREFILL_UBATCH},
            "data": f"synthetic (seeded random-init weights; random.Random({args.seed + 1}) token ids)"}
    if args.prefill_check:
        ref = sinter.Model(cfg, seed=args.seed)
        try:
            t1 = time.perf_counter()
            rtok = ref.prefill(prompt, 0, mode="tokenwise")
            ts = time.perf_counter() - t1
            print(f"# tokenwise prefill: {args.ctx} tokens in {ts:.1f} s; next token {rtok}", file=sys.stderr,
                  flush=True)
            same = {"next_token": tok == rtok, "logits": bool(np.array_equal(m.logits(), ref.logits()))}
            n_diff = 0
            for il in range(cfg.n_layer):
                for sl in range(2):
                    da, na = m.state(il, sl)
                    db, nb = ref.state(il, sl)
                    a = np.empty(na, np.uint8)
                    b = np.empty(nb, np.uint8)
                    m.d2h(a, da, na)
                    ref.d2h(b, db, nb)
                    if na != nb or not np.array_equal(a, b):
                        n_diff += 1
            same["states"] = n_diff == 0
            line["check"] = {"against": "sinter_model_prefill_tokenwise (the decode program over the prompt), "
                                        "a second model of the same weights",
                             "tokenwise_seconds": round(ts, 3), "tokenwise_tok_s": round(args.ctx / ts, 2),
                             "bit_identical": same, "state_buffers_differing": n_diff,
                             "compared": "next token, logits, K and V caches of every attention layer, conv and "
                                         "recurrent state of every GDN layer (whole buffers, byte for byte)"}
        finally:
            ref.close()
    print(json.dumps(line), flush=True)
    if args.prefill_check and not all(line["check"]["bit_identical"].values()):
        sys.exit(1)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--config", type=int, default=4, choices=[1, 2, 3, 4, 5],
                    help="BASELINE config: 4 (default) the e2e Q4_K_M decode at 4096 context; 5 the e2e bf16 "
                         "decode at 131072 KV positions; 1-3 single-op timings (Q8_0 GEMV, GDN mixer, attention "
                         "mixer at --ctx positions) over rotated weight copies")
    ap.add_argument("--steps", type=int, default=None, help="timed tokens (default 256; config 5: 128)")
    ap.add_argument("--warmup", type=int, default=None, help="untimed warmup tokens (default 16; config 5: 4)")
    ap.add_argument("--balance", type=int, nargs=2, default=(2, 4), metavar=("ROUNDS", "TRACES"),
                    help="static GEMV load balance before the warmup: ROUNDS updates, each measured on TRACES "
                         "traced greedy passes (sinter_model_balance; TRACES = 0: off)")
    ap.add_argument("--ctx", type=int, default=None,
                    help="context positions (default 4096; config 5: 131072 less the decoded tokens)")
    ap.add_argument("--quant", default="q4_k_m", choices=["q4_k_m", "bf16"])
    ap.add_argument("--context", choices=["prefill", "synth"], default=None,
                    help="how the context is made: prefill (default for config 4, as BASELINE specifies it): "
                         "seeded random prompt tokens through sinter_model_prefill on the GPU (the batched "
                         "prefill); synth (default for config 5, whose 131072-token prefill "
                         "would take ~35 min, and for --parity-steps): seeded synthetic KV and recurrent state")
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--seed", type=int, default=2026)
    ap.add_argument("--attn-chunk-min", type=int, default=0, metavar="N",
                    help="split-K attention: positions per chunk at least (0: the library default)")
    ap.add_argument("--passes-per-launch", type=int, default=16,
                    help="greedy passes per cooperative launch (the warmup is one launch)")
    ap.add_argument("--profile-ops", type=int, default=0,
                    help="after the timed run, N more tokens with block-0 per-kind timers (stderr)")
    ap.add_argument("--parity-steps", type=int, default=0, metavar="N",
                    help="only check parity: from a fresh synthetic context, N greedy decode steps on the GPU "
                         "and on the CPU oracle (same weights and state); token ids must be identical, logits "
                         "within rel L2 1e-2; prints one JSON line and exits")
    ap.add_argument("--ubatch", type=int, default=0, metavar="T",
                    help="measure the batched GEMV of a batched prefill: T tokens through one GDN layer's "
                         "trunk matrices (sinter_op_gemv_ubatch) instead of the decode")
    ap.add_argument("--prefill-check", action="store_true",
                    help="only the prefill: the --ctx-token prompt through the batched prefill (timed), then a "
                         "second model of the same weights through the decode program over the prompt (timed); "
                         "the next token, logits, KV caches and recurrent / conv states must be bit-identical; "
                         "prints one JSON line and exits")
    ap.add_argument("--prefill-reps", type=int, default=0, metavar="N",
                    help="only the batched prefill: N timed prefills of the --ctx-token prompt at position 0 "
                         "(each from the state the last left: the same work); prints one JSON line and exits")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only copy MIB MiB device-to-device 3 times (the HIP runtime's copy kernel) and exit: the "
                         "known-size reference the FETCH_SIZE / WRITE_SIZE counters are scaled by")
    args = ap.parse_args()
    if args.config == 5:
        args.quant = "bf16"
    if args.context is None:
        args.context = "synth" if args.config == 5 or args.parity_steps else "prefill"
    if args.steps is None:
        args.steps = 128 if args.config == 5 else 256
    if args.warmup is None:
        args.warmup = 4 if args.config == 5 else 16
    if args.ctx is None:
        # config 5: the KV cache holds 131072 positions, the decoded tokens included
        n_bal = (args.balance[0] + 1) * args.balance[1] if args.balance[1] else 0
        args.ctx = 131072 - (n_bal + args.warmup + max(args.steps, args.parity_steps) + args.profile_ops + 24) \
            if args.config == 5 else 4096
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} is not supported: this build runs the decode path on one GPU "
              "(the 27B model fits one MI355X; no multi-GPU path is built)", file=sys.stderr)
        sys.exit(2)

    # The decode, op and calibration runs need no torch: they load libsinter on
    # the system ROCm runtime, the one rocprofv3 belongs to (torch would bring
    # its own bundled HIP/HSA runtime into the process).  Every model call
    # below returns after its device work has finished.  The batched-GEMV run
    # uses torch for its buffers, so torch's runtime is loaded there.
    import sinter
    if not args.ubatch:
        sinter.use_system_runtime()

    if args.copy_calibration:
        n = args.copy_calibration << 20
        sinter.check(sinter.lib().sinter_copy_calibration(0, n, 3), "copy calibration")
        print(json.dumps({"copy_calibration_bytes": n, "copies": 3}), flush=True)
        return

    if args.ubatch:
        ubatch_bench(args)
        return
    if args.config in (1, 2, 3):
        op_bench(args)
        return
    n_bal = (args.balance[0] + 1) * args.balance[1] if args.balance[1] else 0
    n_ctx = args.ctx + n_bal + args.warmup + max(args.steps, args.parity_steps) + args.profile_ops + 24
    cfg = sinter.qwen36_27b_config(n_ctx=n_ctx, quant=args.quant)
    cfg.attn_chunk_min = args.attn_chunk_min
    t0 = time.perf_counter()
    m = sinter.Model(cfg, seed=args.seed)
    setup_s = time.perf_counter() - t0
    print(f"# model ready in {setup_s:.1f} s: {m.info()}", file=sys.stderr, flush=True)
    tok, prefill_info = 1, None
    if args.prefill_check or args.prefill_reps:
        prefill_only(m, cfg, args)
        m.close()
        return
    if args.context == "prefill" and args.ctx > 0:
        import random
        rng = random.Random(args.seed + 1)
        prompt = [rng.randrange(cfg.n_vocab) for _ in range(args.ctx)]
        t1 = time.perf_counter()
        tok = m.prefill(prompt, 0)
        ps = time.perf_counter() - t1
        prefill_info = {"tokens": args.ctx, "seconds": round(ps, 3), "tok_s": round(args.ctx / ps, 2),
                        "path": "sinter_model_prefill: batched (ubatches of 256 tokens, each layer once per ubatch)",
                        "prompt": f"random.Random({args.seed + 1}) token ids"}
        print(f"# prefilled {args.ctx} tokens on the GPU in {ps:.1f} s; next token {tok}", file=sys.stderr, flush=True)
    else:
        m.synth_context(args.ctx, seed=args.seed + 1)

    if args.parity_steps:
        parity(m, cfg, args)
        m.close()
        return

    L = sinter.lib()
    ppl = max(1, min(args.passes_per_launch, args.steps))
    pos = args.ctx
    if n_bal:
        # untimed: rebalances the GEMV row ranges (results are unchanged)
        tok, pos = m.balance(tok, pos, args.balance[0], args.balance[1])
    if args.warmup:
        toks = m.greedy(tok, pos, args.warmup)
        tok = toks[-1]
    pos0 = pos + args.warmup
    # K timed tokens as launches of `ppl` greedy passes each (the last launch
    # takes the remainder); every launch's kernel time comes from HIP events
    # recorded on the interpreter's own stream
    toks, launch_ms = [], []
    t0 = time.perf_counter()
    done = 0
    while done < args.steps:
        n = min(ppl, args.steps - done)
        out = m.greedy(tok, pos0 + done, n)
        launch_ms.append(L.sinter_host_last_launch_ms(m.host()))
        toks += out
        tok = out[-1]
        done += n
    wall = time.perf_counter() - t0
    kernel_ms = sum(launch_ms)
    print(f"# timed {args.steps} tokens in {len(launch_ms)} launches of <= {ppl} passes: wall {wall * 1e3:.2f} ms, "
          f"interpreter kernel {kernel_ms:.2f} ms (per launch: mean {kernel_ms / len(launch_ms):.3f} ms, "
          f"min {min(launch_ms):.3f}, max {max(launch_ms):.3f}); tokens[:8] {toks[:8]}", file=sys.stderr, flush=True)

    if args.profile_ops:
        import ctypes as C
        h = m.host()
        L.sinter_host_reset_op_cycles(h)
        m.greedy(toks[-1], pos0 + args.steps, args.profile_ops)
        cyc = (C.c_longlong * 5)()
        L.sinter_host_read_op_cycles(h, cyc, 5)
        names = ["nop", "boundary", "gemv", "gdn_step", "attn_decode"]
        # wall clock ticks: 100 MHz on MI355X
        rep = {n: round(c / 1e5 / args.profile_ops, 4) for n, c in zip(names, cyc)}
        print(f"# block-0 ms per token by kind: {rep}", file=sys.stderr, flush=True)
    # one pass per launch (the reference's doorbell rhythm): per-token latency
    sp_ms, _, sp_kernel_ms = single_pass_latency(m, toks[-1], pos0 + args.steps + args.profile_ops)
    mean_attended = pos0 + (args.steps + 1) / 2.0
    bpt = bytes_per_token(cfg, m, mean_attended)
    traffic, traffic_commit = measured_traffic(ppl, args.quant, args.ctx)
    tok_s = args.steps / wall
    achieved = bpt["total"] * args.steps / (kernel_ms * 1e-3) / 1e9
    line = {
        "metric": METRIC, "value": round(tok_s, 3), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(wall * 1e3 / args.steps, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8" if args.quant == "q4_k_m" else "bf16",
        "data": (f"synthetic (seeded random-init weights; {args.ctx}-token context prefilled on the GPU from seeded "
                 f"random token ids)" if prefill_info else
                 f"synthetic (seeded random-init weights and {args.ctx}-token synthetic KV/recurrent state)"),
        "config": {"workload": f"BASELINE config {args.config}: e2e greedy decode, Qwen3.6-27B-shaped hybrid "
                               f"(48 GDN + 16 attention), {args.quant} weights, {args.ctx}-token context",
                   "context": args.ctx, "n_ctx": n_ctx, "global_batch": 1, "parallelism": "none (1 GPU)",
                   "gemv_balance": f"{args.balance[0]} updates, {n_bal} traced passes (untimed)",
                   "bytes_per_token": bpt["total"], "bytes_breakdown": bpt},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_GBS, 4), "traffic": traffic,
                     "traffic_measured_at": traffic_commit,
                     "kernel": m.info()["kernel"], "passes_per_launch": ppl,
                     "kernel_ms_per_launch": round(kernel_ms / len(launch_ms), 4),
                     "kernel_ms_per_token": round(kernel_ms / args.steps, 4)},
        "prefill": prefill_info,
        "single_pass": {"ms_per_token": round(sp_ms, 4), "calls": 8, "kernel_ms": round(sp_kernel_ms, 4),
                        "path": "sinter_model_decode: one cooperative launch per token, token read back"},
    }
    line["roofline"].update(roofline_peaks(achieved))
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(m, args.ctx, args.cpu_seconds)
    m.close()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
