"""Execute the reference's captured decode graph on the CPU -- test-only.

The reference records the llama.cpp decode graph of the Qwen3.6-27B hybrid
as two CSV files (k0/schedule.csv: one row per ggml node with op, output
shape, decoded op params, source references, block and macro tags;
k0/leaves.csv: one row per leaf tensor with its classification, e.g.
`weight:blk.3.attn_q.weight`, `state:conv_state(blk.0)`, `positions`).
Committed copies live in tests/golden/.

GraphExec walks those nodes in order and evaluates each with ggml's op
semantics on numpy tensors (views carry element offsets and strides, as
ggml tensors do), binding leaves to caller-supplied arrays.  Arithmetic
primitives with a declared numeric rule (quantised matmul, RMS/L2 norms,
silu/sigmoid/softplus, the delta-rule step, RoPE, attention) call the CPU
oracle's primitives, which other tests pin; everything else -- which node
feeds which, views and their offsets, residual adds, gating, state
write-back, KV append rows -- comes from the capture.  Comparing its output
with oracle.or_decode_step therefore checks the oracle's composition of the
decode pass against the reference's graph, independently of how the oracle
was written.

The capture stores view offsets but not view strides.  A VIEW is taken
contiguous from its offset, except (a) a slice of every row of a 2-D source
(same row count, fewer columns: the conv window shift, VIEW 3x10240 of the
4x10240 window at offset 4 bytes), which keeps the source's row stride, and
(b) the two q|gate slices of the attention q projection, whose per-head
stride of 2*head_dim floats comes from the model builder (docs/BLOCKS.md:104:
"per-head stride 512 f32, from builder"); their offsets (0 and 1024 bytes)
are the capture's.
"""
import csv
import ctypes as C
import math
import os
import re

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
SCHEDULE = os.path.join(GOLDEN, "k0_schedule.csv")
LEAVES = os.path.join(GOLDEN, "k0_leaves.csv")


def load_graph(schedule=SCHEDULE, leaves=LEAVES):
    nodes, lvs = {}, {}
    with open(schedule) as f:
        for r in csv.DictReader(f):
            nodes[int(r["node_idx"])] = {
                "op": r["op"], "type": r["type"], "ne": [int(x) for x in r["ne"].split("x")],
                "params": r["decoded_params"], "src": r["src_refs"].split(";") if r["src_refs"] else [],
                "block": r["block_idx"], "mid": int(r["macro_op_id"]), "mkind": r["macro_kind"]}
    with open(leaves) as f:
        for r in csv.DictReader(f):
            lvs[int(r["leaf_idx"])] = {"type": r["type"], "ne": [int(x) for x in r["ne"].split("x")],
                                       "cls": r["classification"]}
    return nodes, lvs


def param(node, name):
    m = re.search(r"\b%s=([^ ]+)" % re.escape(name), node["params"])
    return m.group(1) if m else None


class T:
    """A ggml-style tensor: a flat numpy buffer, an element offset, ne[4]
    (ne0 fastest) and element strides nb[4]."""
    __slots__ = ("buf", "off", "ne", "nb")

    def __init__(self, buf, ne, nb=None, off=0):
        ne = list(ne) + [1] * (4 - len(ne))
        if nb is None:
            nb = [1, ne[0], ne[0] * ne[1], ne[0] * ne[1] * ne[2]]
        self.buf, self.off, self.ne, self.nb = buf, off, ne, list(nb)

    @property
    def n(self):
        return self.ne[0] * self.ne[1] * self.ne[2] * self.ne[3]

    def contiguous(self):
        return self.nb == [1, self.ne[0], self.ne[0] * self.ne[1], self.ne[0] * self.ne[1] * self.ne[2]]

    def view4(self):
        """numpy view indexed [i3, i2, i1, i0] (writeable when buf is)."""
        it = self.buf.itemsize
        if self.n == 0:
            return np.zeros((self.ne[3], self.ne[2], self.ne[1], self.ne[0]), self.buf.dtype)
        return np.lib.stride_tricks.as_strided(
            self.buf[self.off:], shape=(self.ne[3], self.ne[2], self.ne[1], self.ne[0]),
            strides=(self.nb[3] * it, self.nb[2] * it, self.nb[1] * it, self.nb[0] * it))

    def flat(self):
        """the elements in ggml order (ne0 fastest), as a new array"""
        return self.view4().reshape(-1).copy()

    def rows(self):
        """[n_rows, ne0] copy"""
        return self.flat().reshape(-1, self.ne[0])


class QWeight:
    """A quantised (or f32/bf16) weight bound to a leaf: raw bytes of `rows`
    rows of k elements of ggml type `type`."""

    def __init__(self, type_, data, k, rows):
        self.type, self.data, self.k, self.rows = type_, data, k, rows


class GraphExec:
    """Evaluates nodes of a captured graph.  `bind` maps leaf index -> T or
    QWeight; `alias` maps a node/leaf reference to another one (to splice
    sections of the graph together)."""

    def __init__(self, nodes, leaves, orc, bind, alias=None, attn_split=(64, 128)):
        """attn_split: (chunks, chunk_min) of the split-K attention whose
        declared fp32 folds FLASH_ATTN_EXT is evaluated with (or_attn_split,
        the attention the product runs)."""
        self.nodes, self.leaves, self.orc = nodes, leaves, orc
        self.attn_split = attn_split
        self.vals = {}
        self.bind = bind
        self.alias = alias or {}
        self.L = orc.lib()

    # -------------------------------------------------------------- refs
    def get(self, ref):
        ref = self.alias.get(ref, ref)
        if ref.startswith("n"):
            return self.vals[int(ref[1:])]
        i = int(ref[1:])
        if i not in self.bind:
            raise KeyError("leaf l%d (%s) is not bound" % (i, self.leaves[i]["cls"]))
        return self.bind[i]

    def run(self, node_ids):
        for i in node_ids:
            self.vals[i] = self.eval(i, self.nodes[i])
        return self.vals

    # -------------------------------------------------------------- ops
    def f32(self, t):
        return t.flat().astype(np.float32)

    def unary(self, name, x):
        fn = {"silu": self.L.or_silu, "sigmoid": self.L.or_sigmoid, "softplus": self.L.or_softplus}[name]
        return np.array([fn(float(v)) for v in x], np.float32)

    def broadcast(self, a, b, op):
        """ggml binary op: b repeats over a's shape (ne of b divides ne of a)."""
        av = a.view4().astype(np.float32)
        bv = b.view4().astype(np.float32)
        reps = [av.shape[d] // bv.shape[d] for d in range(4)]
        bb = np.tile(bv, reps)
        out = (av * bb) if op == "mul" else (av + bb)
        return T(out.astype(np.float32).reshape(-1), a.ne)

    def eval(self, i, nd):
        op, ne, src = nd["op"], nd["ne"], nd["src"]
        s = [self.get(r) for r in src]
        if op in ("RESHAPE",):
            x = s[0]
            if not x.contiguous():
                raise ValueError("n%d: reshape of a non-contiguous tensor" % i)
            return T(x.buf, ne, off=x.off)
        if op == "VIEW":
            x = s[0]
            off_b = int(param(nd, "offset"))
            es = x.buf.itemsize
            assert off_b % es == 0
            parent = self.nodes.get(int(src[0][1:])) if src[0].startswith("n") else None
            if nd["mkind"] in ("q_gemv_norm_rope", "attn_gate_out") and parent and parent["op"] == "MUL_MAT":
                # the q|gate slices: one head of q then one head of gate, per
                # head (the builder's stride, not recorded by the capture)
                nb = [1, 2 * ne[0], 2 * ne[0] * ne[1], 2 * ne[0] * ne[1] * ne[2]]
            elif ne[0] < x.ne[0] and ne[1] == x.ne[1] and ne[1] > 1:
                # a slice of every row of a 2-D source (the conv window
                # shift) keeps the source's row stride
                nb = [1, x.nb[1], x.nb[2], x.nb[3]]
            else:
                nb = [1, ne[0], ne[0] * ne[1], ne[0] * ne[1] * ne[2]]
            return T(x.buf, ne, nb, x.off + off_b // es)
        if op == "PERMUTE":
            ax = [int(v) for v in re.search(r"axes=\[([^\]]*)\]", nd["params"]).group(1).split()]
            x = s[0]
            # ggml_permute: source dim d goes to position ax[d]
            nne, nnb = [0] * 4, [0] * 4
            for d in range(4):
                nne[ax[d]], nnb[ax[d]] = x.ne[d], x.nb[d]
            assert nne == ne, (i, nne, ne)
            return T(x.buf, nne, nnb, x.off)
        if op == "TRANSPOSE":
            x = s[0]
            return T(x.buf, [x.ne[1], x.ne[0], x.ne[2], x.ne[3]], [x.nb[1], x.nb[0], x.nb[2], x.nb[3]], x.off)
        if op == "CONT":
            return T(s[0].flat(), ne)
        if op == "SCALE":
            if math.prod(ne) != 0:
                raise NotImplementedError("SCALE with elements")
            return T(np.zeros(0, np.float32), ne)
        if op == "GET_ROWS":
            w, idx = s
            ids = idx.flat().astype(np.int64)
            if len(ids) == 0:
                return T(np.zeros(0, np.float32), ne)
            if isinstance(w, QWeight):
                out = np.concatenate([self.orc.dequant(w.type, w.data[r * self.orc.row_bytes(w.type, w.k):
                                                                     (r + 1) * self.orc.row_bytes(w.type, w.k)], w.k)
                                      for r in ids])
            else:
                rows = w.rows()
                out = np.concatenate([rows[r] for r in ids]).astype(np.float32)
            return T(out, ne)
        if op == "CPY":
            x, dst = s
            if x.n != dst.n:
                raise ValueError("n%d: CPY of %d into %d elements" % (i, x.n, dst.n))
            if x.n:
                v = dst.view4()
                v[...] = x.flat().reshape(v.shape).astype(dst.buf.dtype)
            return dst
        if op == "CONCAT":
            a, b = s
            assert int(param(nd, "dim")) == 0
            av, bv = a.view4(), b.view4()
            out = np.concatenate([av, bv], axis=3).astype(np.float32)
            return T(out.reshape(-1), ne)
        if op == "RMS_NORM":
            eps = float(np.float32(param(nd, "eps")))
            x = s[0].rows().astype(np.float32)
            y = np.zeros_like(x)
            for r in range(x.shape[0]):
                xr, yr = np.ascontiguousarray(x[r]), np.zeros(x.shape[1], np.float32)
                self.L.or_rmsnorm(xr.ctypes.data, None, yr.ctypes.data, x.shape[1], eps)
                y[r] = yr
            return T(y.reshape(-1), ne)
        if op == "L2_NORM":
            eps = float(np.float32(param(nd, "eps")))
            x = s[0].rows().astype(np.float32)
            y = np.zeros_like(x)
            for r in range(x.shape[0]):
                xr, yr = np.ascontiguousarray(x[r]), np.zeros(x.shape[1], np.float32)
                self.L.or_l2norm(xr.ctypes.data, yr.ctypes.data, x.shape[1], eps)
                y[r] = yr
            return T(y.reshape(-1), ne)
        if op == "MUL":
            return self.broadcast(s[0], s[1], "mul")
        if op == "ADD":
            return self.broadcast(s[0], s[1], "add")
        if op == "UNARY":
            name = re.match(r"(\w+)\(", param(nd, "unary")).group(1)
            return T(self.unary(name, self.f32(s[0])), ne)
        if op == "GLU":
            assert param(nd, "glu").startswith("swiglu") and param(nd, "swapped") == "0"
            g, u = self.f32(s[0]), self.f32(s[1])
            return T(self.unary("silu", g) * u, ne)
        if op == "MUL_MAT":
            w, x = s
            if not isinstance(w, QWeight):
                raise TypeError("n%d: MUL_MAT weight must be bound to a QWeight" % i)
            xv = self.f32(x)
            assert xv.size == w.k, (i, xv.size, w.k)
            y = self.orc.gemv(w.type, w.data, w.rows, w.k, xv)
            return T(y, [w.rows, 1, 1, 1])
        if op == "SSM_CONV":
            win, kern = s          # win [d_conv, C] (ne0 = d_conv), kernel [d_conv, C]
            dc, ch = win.ne[0], win.ne[1]
            wv = win.rows().astype(np.float64)    # [C, dc]
            kv = kern.rows().astype(np.float64)
            acc = np.zeros(ch, np.float64)
            for j in range(dc):                   # taps in order, exact products, one rounding
                acc = acc + wv[:, j] * kv[:, j]
            return T(acc.astype(np.float32), ne)
        if op == "GATED_DELTA_NET":
            q, k, v, g, beta, st = s
            D, HK = q.ne[0], q.ne[1]
            HV = v.ne[1]
            qf, kf, vf = self.f32(q), self.f32(k), self.f32(v)
            # g is the log decay (softplus(a + dt_bias) * ssm_a); the op decays by exp(g)
            ge = np.array([np.float32(math.exp(float(x))) for x in self.f32(g)], np.float32)
            bf = self.f32(beta)
            state = self.f32(st).copy()
            o = np.zeros(HV * D, np.float32)
            scale = np.float32(1.0) / np.sqrt(np.float32(D))
            self.L.or_gdn_step(qf.ctypes.data, kf.ctypes.data, vf.ctypes.data, ge.ctypes.data, bf.ctypes.data,
                               state.ctypes.data, o.ctypes.data, HV, HK, D, float(scale), self.L.or_gdn_cols(D))
            out = np.concatenate([o, state])
            assert out.size == math.prod(ne)
            return T(out, ne)
        if op == "ROPE":
            x, pos = s
            mode = param(nd, "mode")
            nd_ = int(param(nd, "n_dims"))
            base = float(param(nd, "freq_base"))
            ids = pos.flat()
            if mode.startswith("IMROPE") and not np.all(ids == ids[0]):
                raise NotImplementedError("IMROPE with distinct position ids")
            for p_ in ("freq_scale", "attn_factor"):
                assert float(param(nd, p_)) == 1.0
            assert float(param(nd, "ext_factor")) == 0.0
            ts = self.L.or_rope_theta_scale(base, nd_)
            rows = s[0].rows().astype(np.float32)
            for r in range(rows.shape[0]):
                xr = np.ascontiguousarray(rows[r])
                self.L.or_rope_neox(xr.ctypes.data, rows.shape[1], nd_, int(ids[0]), ts)
                rows[r] = xr
            return T(rows.reshape(-1), ne)
        if op == "SET_ROWS":
            val, idx, dst = s
            r = int(idx.flat()[0])
            row = self.f32(val)
            v = dst.view4()
            assert v.shape[0] == 1 and v.shape[1] == 1 and 0 <= r < v.shape[2] and v.shape[3] == row.size
            v[0, 0, r, :] = row.astype(np.float16)
            return dst
        if op == "FLASH_ATTN_EXT":
            q, k, v, mask = s
            scale = float(np.float32(param(nd, "scale")))
            assert float(param(nd, "max_bias")) == 0.0 and float(param(nd, "logit_softcap")) == 0.0
            HD, NQ = q.ne[0], q.ne[2]
            n_kv, NKV = k.ne[1], k.ne[2]
            mk = mask.flat().astype(np.float32)[:n_kv]
            open_ = np.nonzero(mk == 0.0)[0]
            n_att = len(open_)
            if not (np.all(open_ == np.arange(n_att)) and np.all(np.isneginf(mk[n_att:]))):
                raise NotImplementedError("mask is not a causal prefix")
            # K/V views are cache rows of NKV*HD f16, heads contiguous
            kb = k.buf
            assert k.nb[0] == 1 and k.nb[1] == NKV * HD and k.nb[2] == HD
            assert v.nb[0] == 1 and v.nb[1] == NKV * HD and v.nb[2] == HD
            qf = np.ascontiguousarray(q.flat().astype(np.float32))
            kc = np.ascontiguousarray(k.buf[k.off:k.off + n_kv * NKV * HD])
            vc = np.ascontiguousarray(v.buf[v.off:v.off + n_kv * NKV * HD])
            out = np.zeros(NQ * HD, np.float32)
            self.L.or_attn_split(qf.ctypes.data, kc.ctypes.data, vc.ctypes.data, self.orc.F16, n_att, NQ, NKV, HD,
                                 scale, self.attn_split[0], self.attn_split[1], out.ctypes.data)
            del kb
            return T(out, ne)
        raise NotImplementedError("op %s (n%d)" % (op, i))
