"""GGUF v3 loader (sinter_gguf_*, sinter_model_config_from_gguf) on the CPU.

A file written by tests/gguf_writer.py from the published v3 layout is read
back through the C ABI: the tensor table (names, types, shapes, offsets,
sizes, data bytes), metadata of every kind used, the derived model shape,
and refusal of malformed files with SINTER_ERR_ARG (bad magic, version,
truncation at every header boundary, unknown tensor type, partial block rows,
misaligned or out-of-file data, nested arrays) -- never a crash.
"""
import ctypes as C
import struct

import numpy as np
import pytest

from gguf_model import Q4_K, Q6_K, make_model_gguf, small_cfg
from gguf_writer import K_ARRAY, K_I32, K_STRING, K_U32, Writer


@pytest.fixture(scope="module")
def model_file(sn, tmp_path_factory):
    p = tmp_path_factory.mktemp("gguf") / "small.gguf"
    c = small_cfg()
    tensors = make_model_gguf(sn, str(p), c)
    return str(p), c, tensors


def test_tensor_table_and_bytes(sn, model_file):
    path, c, tensors = model_file
    with sn.Gguf(path) as g:
        info = g.info()
        assert info["version"] == 3 and info["alignment"] == 32 and info["n_tensors"] == len(tensors)
        for i in range(info["n_tensors"]):
            t = g.tensor(i)
            name = t.name.decode()
            typ, ne, data = tensors[name]
            assert t.type == typ and list(t.ne)[:len(ne)] == ne and t.n_dims == len(ne)
            assert t.nbytes == data.nbytes and t.offset % 32 == 0
            got = np.ctypeslib.as_array((C.c_uint8 * t.nbytes).from_address(t.data))
            assert np.array_equal(got, data.view(np.uint8).reshape(-1)), name
            assert g.find(name) == i
        assert g.find("no.such.tensor") == -1


def test_metadata_kinds(sn, model_file):
    path, c, _ = model_file
    with sn.Gguf(path) as g:
        assert g.kv_str("general.architecture") == "qwen35"
        assert g.kv_i64("qwen35.block_count") == c["n_layer"]
        assert g.kv_f64("qwen35.rope.freq_base") == np.float32(c["rope_base"])
        assert g.kv_f64("qwen35.rope.dimension_count") == c["rope_dims"]   # integers read as numbers too
        assert g.kv_arr_i64("qwen35.rope.dimension_sections") == [11, 11, 10, 0]
        L = sn.lib()
        v = C.c_int64()
        assert L.sinter_gguf_kv_i64(g.h, b"general.architecture", C.byref(v)) == sn.ERR_ARG   # a string
        assert L.sinter_gguf_kv_i64(g.h, b"missing.key", C.byref(v)) == sn.ERR_ARG
        small = C.create_string_buffer(3)
        assert L.sinter_gguf_kv_str(g.h, b"general.architecture", small, 3) == sn.ERR_ARG


def test_model_config_from_tensor_shapes(sn, model_file):
    path, c, _ = model_file
    with sn.Gguf(path) as g:
        cfg = g.config(512)
    want = dict(n_layer=c["n_layer"], attn_every=c["attn_every"], n_embd=c["E"], n_ff=c["F"], n_vocab=c["V"],
                gdn_hk=c["HK"], gdn_hv=c["HV"], gdn_d=c["D"], conv_k=c["K"], attn_nq=c["NQ"], attn_nkv=c["NKV"],
                head_dim=c["HD"], rope_dims=c["rope_dims"], n_ctx=512, t_default=Q4_K, t_attn_v=Q6_K,
                t_ffn_down=Q6_K, t_output=Q6_K, t_embd=Q4_K)
    for k, v in want.items():
        assert getattr(cfg, k) == v, k
    assert cfg.rope_base == np.float32(1e7) and cfg.eps == np.float32(1e-6)


def test_multi_token_prediction_block_and_tied_head(sn, tmp_path):
    """A trailing nextn (multi-token prediction) block is not a decoder block;
    a file without output.weight ties the head to token_embd."""
    c = small_cfg()
    p = tmp_path / "mtp.gguf"
    make_model_gguf(sn, str(p), c, tied=True, extra_block=True)
    with sn.Gguf(str(p)) as g:
        cfg = g.config(256)
        assert g.find("output.weight") == -1 and g.find("blk.4.attn_norm.weight") >= 0
    assert cfg.n_layer == c["n_layer"] and cfg.t_output == cfg.t_embd


def _write(tmp_path, name, w):
    p = tmp_path / name
    w.write(str(p))
    return p


def _expect_refused(sn, path, what):
    h = C.c_void_p()
    rc = sn.lib().sinter_gguf_open(str(path).encode(), C.byref(h))
    msg = sn.lib().sinter_last_error().decode()
    assert rc == sn.ERR_ARG and not h.value, (what, rc)
    return msg


def test_malformed_files_are_refused(sn, tmp_path):
    data = np.arange(512, dtype=np.float32)
    good = Writer()
    good.add_kv("general.architecture", K_STRING, "qwen35")
    good.add_kv("some.array", K_ARRAY, [1, 2, 3], K_I32)
    good.add_tensor("a", [256, 2], 0, data)
    gp = _write(tmp_path, "good.gguf", good)
    with sn.Gguf(str(gp)) as g:
        assert g.info()["n_tensors"] == 1
    raw = gp.read_bytes()
    header_len = len(good.header(good.offsets()))

    bad = tmp_path / "magic.gguf"
    bad.write_bytes(b"GGUG" + raw[4:])
    assert "magic" in _expect_refused(sn, bad, "magic")
    bad.write_bytes(raw[:4] + struct.pack("<I", 2) + raw[8:])
    assert "version" in _expect_refused(sn, bad, "version")
    # truncated anywhere inside the header, or inside the tensor data
    for cut in list(range(0, header_len, 3)) + [header_len + 100, len(raw) - 1]:
        bad.write_bytes(raw[:cut])
        _expect_refused(sn, bad, "truncated at %d" % cut)
    bad.write_bytes(b"")
    _expect_refused(sn, bad, "empty")

    w = Writer()
    w.add_tensor("q", [256, 1], 99, np.zeros(64, np.uint8))
    assert "unknown type" in _expect_refused(sn, _write(tmp_path, "type.gguf", w), "type")
    w = Writer()
    w.add_tensor("q", [100, 1], Q4_K, np.zeros(144, np.uint8))    # 100 is not a whole Q4_K block
    assert "block" in _expect_refused(sn, _write(tmp_path, "block.gguf", w), "partial block")
    w = Writer()
    w.add_kv("nested", K_ARRAY, [], K_ARRAY)
    assert "nested" in _expect_refused(sn, _write(tmp_path, "nested.gguf", w), "nested")
    w = Writer()
    w.add_kv("general.alignment", K_U32, 24)
    w.add_tensor("a", [8], 0, np.zeros(8, np.float32))
    assert "alignment" in _expect_refused(sn, _write(tmp_path, "align.gguf", w), "alignment")

    # a tensor whose offset is misaligned, or whose data runs past the end
    class Off(Writer):
        def __init__(self, delta):
            super().__init__()
            self.delta = delta

        def offsets(self):
            return [o + self.delta for o in super().offsets()]
    w = Off(4)
    w.add_tensor("a", [8], 0, np.zeros(8, np.float32))
    assert "aligned" in _expect_refused(sn, _write(tmp_path, "mis.gguf", w), "misaligned")
    w = Off(1 << 20)
    w.add_tensor("a", [8], 0, np.zeros(8, np.float32))
    assert "past the end" in _expect_refused(sn, _write(tmp_path, "past.gguf", w), "past end")
    w = Writer()
    w.add_tensor("a", [8], 0, np.zeros(8, np.float32))
    w.add_tensor("a", [8], 0, np.zeros(8, np.float32))
    assert "duplicate" in _expect_refused(sn, _write(tmp_path, "dup.gguf", w), "duplicate")
    # dimensions whose byte count wraps 128 bits (2^62 * 2^62 * 4 * 4 B = 2^128),
    # a zero dimension, and one past INT64_MAX
    for ne, what in (([1 << 62, 1 << 62, 4], "larger than the file"), ([8, 0], "is 0"),
                     ([8, (1 << 63) + 8], "INT64_MAX")):
        w = Writer()
        w.add_tensor("a", ne, 0, np.zeros(8, np.float32))
        assert what in _expect_refused(sn, _write(tmp_path, "dims.gguf", w), str(ne))
    assert sn.lib().sinter_gguf_open(str(tmp_path / "missing.gguf").encode(), C.byref(C.c_void_p())) == sn.ERR_ARG


def test_config_refuses_irregular_attention_pattern(sn, tmp_path):
    c = small_cfg()
    p = tmp_path / "m.gguf"
    tensors = make_model_gguf(sn, str(p), c)
    # drop the attention block's q projection: blocks are no longer periodic
    w = Writer()
    for name, (t, ne, data) in tensors.items():
        if name != "blk.3.attn_q.weight":
            w.add_tensor(name, ne, t, data)
    q = tmp_path / "irregular.gguf"
    w.write(str(q))
    with sn.Gguf(str(q)) as g:
        cfg = sn.ModelConfig()
        assert sn.lib().sinter_model_config_from_gguf(g.h, 256, C.byref(cfg)) == sn.ERR_ARG


def test_mutated_files_open_or_are_refused(sn, tmp_path):
    """Seeded byte mutations of a valid file (header, metadata, tensor table
    and data regions; single-byte flips, 4-byte overwrites with extreme
    values, truncations): every file either opens with a self-consistent
    table -- each tensor's data inside the file -- or is refused with
    SINTER_ERR_ARG; the parser never reads outside the file."""
    data = np.arange(1024, dtype=np.float32)
    w = Writer()
    w.add_kv("general.architecture", K_STRING, "qwen35")
    w.add_kv("qwen35.block_count", K_U32, 4)
    w.add_kv("some.array", K_ARRAY, [1, 2, 3, 4], K_I32)
    w.add_tensor("a", [256, 2], 0, data[:512])
    w.add_tensor("b.weight", [256, 2], 0, data[512:])
    raw = bytearray(_write(tmp_path, "base.gguf", w).read_bytes())
    header_len = len(w.header(w.offsets()))
    rng = np.random.default_rng(2027)
    path = tmp_path / "mut.gguf"
    opened = refused = 0
    for it in range(300):
        b = bytearray(raw)
        kind = it % 3
        if kind == 0:
            pos = int(rng.integers(0, header_len))
            b[pos] ^= 1 << int(rng.integers(0, 8))
        elif kind == 1:
            pos = int(rng.integers(0, header_len - 4))
            b[pos:pos + 4] = struct.pack("<I", int(rng.choice([0, 1, 0x7fffffff, 0xffffffff, 255, 65536])))
        else:
            b = b[:int(rng.integers(0, len(b)))]
        path.write_bytes(bytes(b))
        h = C.c_void_p()
        rc = sn.lib().sinter_gguf_open(str(path).encode(), C.byref(h))
        if rc != sn.OK:
            assert rc == sn.ERR_ARG, (it, rc)
            refused += 1
            continue
        opened += 1
        g = sn.Gguf.__new__(sn.Gguf)      # (the handle just opened)
        g.h = h
        try:
            info = g.info()
            for i in range(info["n_tensors"]):
                t = g.tensor(i)
                assert t.nbytes <= len(b)
        finally:
            g.close()
    assert opened and refused
