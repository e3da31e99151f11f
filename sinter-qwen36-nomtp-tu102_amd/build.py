"""Build libsinter.so (HIP for gfx950) in-tree, behind a resource gate.

Run as `python sinter-qwen36-nomtp-tu102_amd/build.py`; __graft_entry__.build()
calls build().  Every translation unit gets the same numerics flags: no
floating-point contraction (the declared fp32 expressions are evaluated
exactly as written, matching the CPU oracle) and no packed-fp32 instructions.

Resource gate: the compiler's kernel-resource-usage remarks are parsed for
every kernel.  The build fails if any kernel uses scratch (private memory:
register spills to memory or stack arrays), has a dynamic stack, if a
persistent-grid kernel cannot keep one 256-thread workgroup per CU (LDS over
160 KiB or occupancy below one wave per SIMD), or if a persistent kernel
spills more registers (VGPRs into AGPRs, SGPRs into VGPR lanes) than its
committed budget (SPILL_BUDGET).  The figures are written to
resource_usage.txt beside the library.
"""
import os
import re
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libsinter.so")
REPORT = os.path.join(HERE, "resource_usage.txt")
SOURCES = ["interp.hip", "ubatch.hip", "prefill.hip", "hbm.hip", "host.cpp", "model.cpp", "gguf.cpp"]
# -Os: the 27B Q4_K_M decode per token (alternating runs on one box) is
# 6.07 ms at -O3, 6.00 at -O2, 5.94 at -Os (fewer spilled registers in the
# K-quant interpreter), 6.08 at -Oz; -O1 6.07; the max-ILP scheduler and
# -fno-slp-vectorize on top of -Os are slower.  No floating-point effect:
# contraction is off and no fast-math flag is set at any level.
FLAGS = [
    "--offload-arch=gfx950", "-Os", "-std=c++17", "-fPIC", "-shared",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
    "-Rpass-analysis=kernel-resource-usage",
]
# kernels that run as one resident workgroup per CU (cooperative grids)
PERSISTENT = {"sinter_interp", "sinter_interp_kquant", "sinter_interp_kquant_q8kv", "sinter_interp_bf16", "sinter_op_kernel", "sinter_op_noalloc_kernel", "sinter_litmus_kernel"}
LDS_LIMIT = 160 * 1024
# Register budget of the persistent kernels: the most VGPRs spilled into
# AGPRs and SGPRs spilled into VGPR lanes the build accepts (the figures of
# the committed build; a change that spills more fails until it is measured
# and the budget raised on purpose).  Spills to memory (scratch) are never
# accepted.
# Raised once on purpose: the fp32 GDN-step folds moved the K-quant kernels
# from (12, 406) / (18, 405) to (22, 475) / (22, 492) spills, with the
# 27B-shaped decode unchanged (A/B, three alternating runs each: 5.924 vs
# 5.932 ms per token).  The single-round-trip attention merge then brought
# every kernel's SGPR spills down (K-quant 475 -> 335) and gave the
# standalone op kernel one VGPR kept in an AGPR; reading instruction headers
# with one scalar load brought them to 278 and moved 2 VGPRs of the Q8_0-cache
# kernel into AGPRs; the header table in LDS moved them by a few either way,
# the GEMV's setup after the barrier's arrival by a few more.  Three Q4_K
# slots in the GEMV body instead of four (0.4 % faster) moved 2 more VGPRs of
# the K-quant kernels into AGPRs; one copy of the final row fold for both
# weight types of the K-quant kernels (1 % faster) took them from 24 to 12.
SPILL_BUDGET = {
    "sinter_interp": (20, 337),
    "sinter_interp_kquant": (12, 288),
    "sinter_interp_kquant_q8kv": (12, 307),
    "sinter_interp_bf16": (12, 289),
    "sinter_op_kernel": (1, 18),
    "sinter_op_noalloc_kernel": (0, 0),
}

_FIELDS = {
    "TotalSGPRs": "sgprs", "VGPRs": "vgprs", "AGPRs": "agprs",
    "ScratchSize [bytes/lane]": "scratch", "Dynamic Stack": "dyn_stack",
    "Occupancy [waves/SIMD]": "occupancy", "SGPRs Spill": "sgpr_spill",
    "VGPRs Spill": "vgpr_spill", "LDS Size [bytes/block]": "lds",
}


def hipcc():
    for c in ("/opt/rocm/bin/hipcc", "hipcc"):
        if os.path.exists(c) or c == "hipcc":
            return c
    return "hipcc"


def parse_resource_usage(text):
    """{kernel: {field: value}} from -Rpass-analysis=kernel-resource-usage
    remarks (the device pass prints one block of remarks per kernel)."""
    kernels, cur = {}, None
    for line in text.splitlines():
        m = re.search(r"remark:\s+Function Name: (\S+)", line)
        if m:
            cur = kernels.setdefault(m.group(1), {})
            continue
        m = re.search(r"remark:\s+([A-Za-z][A-Za-z /\[\]]*?): (\S+) \[-Rpass-analysis", line)
        if m and cur is not None and m.group(1) in _FIELDS:
            v = m.group(2)
            cur[_FIELDS[m.group(1)]] = v if v in ("True", "False") else int(v)
    return kernels


def gate(kernels):
    """Reasons the build must fail (empty: pass)."""
    bad = []
    if not kernels:
        bad.append("no kernel-resource-usage remarks found")
    for name, k in kernels.items():
        if k.get("scratch", 0) != 0:
            bad.append(f"{name}: {k['scratch']} bytes/lane of scratch")
        if k.get("dyn_stack") == "True":
            bad.append(f"{name}: dynamic stack")
        if name in PERSISTENT:
            if k.get("lds", 0) > LDS_LIMIT:
                bad.append(f"{name}: {k['lds']} B of LDS per workgroup (> {LDS_LIMIT})")
            if k.get("occupancy", 0) < 1:
                bad.append(f"{name}: occupancy {k.get('occupancy')} waves/SIMD")
    for name in PERSISTENT:
        if kernels and name not in kernels:
            bad.append(f"{name}: no resource remarks")
    for name, (vmax, smax) in SPILL_BUDGET.items():
        k = kernels.get(name)
        if k is None:
            continue
        if k.get("vgpr_spill", 0) > vmax or k.get("sgpr_spill", 0) > smax:
            bad.append(f"{name}: {k.get('vgpr_spill')} VGPR / {k.get('sgpr_spill')} SGPR spills over the budget "
                       f"({vmax} / {smax})")
    return bad


def report_text(kernels):
    cols = ["vgprs", "agprs", "sgprs", "vgpr_spill", "sgpr_spill", "scratch", "lds", "occupancy"]
    lines = ["kernel " + " ".join(cols)]
    for name in sorted(kernels):
        lines.append(name + " " + " ".join(str(kernels[name].get(c, "?")) for c in cols))
    return "\n".join(lines) + "\n"


def build(verbose=False):
    srcs = [os.path.join(CSRC, s) for s in SOURCES]
    tmp = LIB + ".tmp"
    cmd = [hipcc()] + FLAGS + srcs + ["-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    text = r.stdout + r.stderr
    out = "\n".join(l for l in text.splitlines()
                    if "packed-fp32-ops" not in l and "remark:" not in l and "-Rpass-analysis" not in l
                    and not re.match(r"^\s*\d+ \|", l) and not re.match(r"^\s*\|\s*\^", l))
    if r.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + out)
    kernels = parse_resource_usage(text)
    bad = gate(kernels)
    if bad:
        if os.path.exists(tmp):
            os.remove(tmp)
        raise RuntimeError("resource gate failed:\n  " + "\n  ".join(bad) + "\n" + report_text(kernels))
    with open(REPORT, "w") as f:
        f.write(report_text(kernels))
    os.replace(tmp, LIB)
    if verbose:
        print(report_text(kernels), end="", flush=True)
    return LIB


GGML_SHIM_SRC = os.path.join(HERE, "ggml_backend", "sinter_ggml.cpp")
GGML_SHIM_LIB = os.path.join(HERE, "ggml_backend", "libsinter_ggml.so")
GGML_RULES_SRC = os.path.join(HERE, "ggml_backend", "graph_rules.cpp")
GGML_RULES_LIB = os.path.join(HERE, "ggml_backend", "libsinter_ggml_rules.so")


def build_ggml_rules(verbose=False):
    """The ggml shim's decision rules (ggml_backend/graph_rules.cpp: which
    graph is a decode graph, what it binds to, when to rebind), built on
    their own with g++ -- no ggml tree and no GPU needed -- so that the CPU
    tests exercise them (tests/test_shim_rules.py)."""
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", GGML_RULES_SRC, "-o", GGML_RULES_LIB + ".tmp"]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("ggml rules build failed:\n" + r.stdout + r.stderr)
    os.replace(GGML_RULES_LIB + ".tmp", GGML_RULES_LIB)
    return GGML_RULES_LIB


def build_ggml_shim(verbose=False):
    """The ggml dynamic backend (ggml_backend/sinter_ggml.cpp), only when a
    ggml tree is named: SINTER_GGML_INCLUDE (the directory holding
    ggml-backend-impl.h and ggml.h) and SINTER_GGML_LIB (holding
    libggml-base.so).  Returns the library path, or None when not asked for
    -- no ggml tree ships with this repository, so by default it is skipped."""
    inc, libdir = os.environ.get("SINTER_GGML_INCLUDE"), os.environ.get("SINTER_GGML_LIB")
    if not inc:
        return None
    if not os.path.exists(os.path.join(inc, "ggml-backend-impl.h")):
        raise RuntimeError(f"SINTER_GGML_INCLUDE={inc} has no ggml-backend-impl.h")
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-I", inc,
           "-I", os.path.join(os.path.dirname(HERE), "include"), GGML_SHIM_SRC, GGML_RULES_SRC, "-o", GGML_SHIM_LIB,
           "-L", HERE, "-lsinter", "-Wl,-rpath," + HERE]
    if libdir:
        cmd += ["-L", libdir, "-lggml-base", "-Wl,-rpath," + libdir]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("ggml shim build failed:\n" + r.stdout + r.stderr)
    return GGML_SHIM_LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
    print(build_ggml_rules(verbose="-v" in sys.argv))
    print(build_ggml_shim(verbose="-v" in sys.argv) or "ggml shim: skipped (SINTER_GGML_INCLUDE not set)")
