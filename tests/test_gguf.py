"""GGUF reader (CPU, no GPU calls): libqmsg's parser against the reference's own qms_gguf_open
(oracle/_ref, compiled from src/gguf.c) on files written by tests/gguf_file.py, plus the
files' MoE layers through the reference's qms_model_load + moe() against the oracle."""
import ctypes
import functools
import os
import struct

import numpy as np
import pytest

import gguf_file as gf
import oracle as orc

# the reference build is loaded on first use, not at import: collecting this module under
# -m gpu must not map it into the GPU test process
need_ref = pytest.mark.skipif(orc.ref_library_path() is None, reason="oracle/_ref (the reference build) is not built here")


@functools.lru_cache(maxsize=None)
def ref_lib():
    return orc.load_ref()


@pytest.fixture(scope="module")
def q():
    from large_model_amd import qmsg
    return qmsg


def small_layers(down_types=(orc.T_Q4_0, orc.T_Q4_1), E=256, X=16, K=4, F=256, seed=40):
    return [orc.Layer(E, X, K, F, seed + l, layer=l, down_type=dt) for l, dt in enumerate(down_types)]


def ref_table(path, cap=256):
    names = ctypes.create_string_buffer(96 * cap)
    a = {k: np.zeros(cap, np.int32) for k in ("type", "n_dims", "shard")}
    ne = np.zeros(4 * cap, np.int64)
    off = np.zeros(cap, np.uint64)
    nb = np.zeros(cap, np.uint64)
    n = ref_lib().qref_gguf_table(os.fsencode(path), cap, names, a["type"].ctypes.data, a["n_dims"].ctypes.data,
                          ne.ctypes.data, a["shard"].ctypes.data, off.ctypes.data, nb.ctypes.data)
    if n < 0:
        return None
    raw = names.raw
    return [{"name": raw[96 * i:96 * i + 96].split(b"\0")[0].decode(), "type": int(a["type"][i]),
             "n_dims": int(a["n_dims"][i]), "ne": [int(v) for v in ne[4 * i:4 * i + 4]], "shard": int(a["shard"][i]),
             "off": int(off[i]), "nbytes": int(nb[i])} for i in range(n)]


def test_table_against_writer(q, tmp_path):
    """Independent of the reference: names, shapes, types and absolute offsets as written."""
    lays = small_layers()
    path = str(tmp_path / "m.gguf")
    kvs = [("general.architecture", gf.STR, "qwen3moe"), ("x.u8", gf.U8, 7)]
    ts = [("a", gf.T_F32, [8], np.arange(8, dtype=np.float32).tobytes()),
          ("b", gf.T_Q4_0, [64, 3], bytes(range(108))),
          ("c", gf.T_Q6_K, [256, 2], bytes(420))]
    offs = gf.write_gguf(path, kvs, ts, alignment=64)
    with q.Gguf(path) as g:
        tab = g.tensors()
        assert [t["name"] for t in tab] == ["a", "b", "c"]
        assert [t["off"] for t in tab] == [offs["a"], offs["b"], offs["c"]]
        assert [t["nbytes"] for t in tab] == [32, 108, 420]
        assert tab[1]["ne"] == [64, 3, 1, 1] and tab[1]["n_dims"] == 2 and tab[2]["type"] == gf.T_Q6_K
        assert all(t["off"] % 64 == 0 for t in tab)
        assert g.find("b") == 1 and g.find("zz") == -1
        assert g.get_int("x.u8") == 7 and g.get_str("general.architecture") == "qwen3moe"
    del lays


@need_ref
@pytest.mark.parametrize("shards", [1, 3])
def test_table_and_values_match_reference(q, tmp_path, shards):
    lays = small_layers((orc.T_Q4_0, orc.T_Q4_1, orc.T_Q6_K))
    path, _ = gf.moe_model(str(tmp_path / "m.gguf"), lays, n_shards=shards)
    ref = ref_table(path)
    with q.Gguf(path) as g:
        mine = g.tensors()
        assert mine == ref
        assert len({t["shard"] for t in mine}) == shards
        for key in ("qwen3moe.block_count", "qwen3moe.embedding_length", "qwen3moe.expert_count",
                    "qwen3moe.attention.layer_norm_rms_epsilon", "qwen3moe.rope.freq_base", "general.alignment",
                    "general.architecture", "tokenizer.ggml.tokens", "no.such.key"):
            ri, rf = ctypes.c_int64(), ctypes.c_double()
            rc = ref_lib().qref_gguf_value(os.fsencode(path), key.encode(), ctypes.byref(ri), ctypes.byref(rf))
            for bit, get, rv in ((1, g.get_int, ri), (2, g.get_float, rf)):
                if rc & bit:
                    with pytest.raises(q.QmsgError):
                        get(key)
                else:
                    assert get(key) == rv.value, key


@need_ref
def test_scalar_conversions_match_reference(q, tmp_path):
    """Every scalar value type through get_int / get_float, as qms_gguf_get_* convert them."""
    path = str(tmp_path / "kv.gguf")
    kvs = [("u8", gf.U8, 250), ("i8", gf.I8, -5), ("u16", gf.U16, 65000), ("i16", gf.I16, -300),
           ("u32", gf.U32, 4000000000), ("i32", gf.I32, -7), ("f32", gf.F32, -2.75), ("bool", gf.BOOL, 1),
           ("u64", gf.U64, 2 ** 63 + 5), ("i64", gf.I64, -(2 ** 40)), ("f64", gf.F64, 1e-6), ("s", gf.STR, "x"),
           ("arr", gf.ARR, (gf.U32, [1, 2, 3])), ("nested", gf.ARR, (gf.ARR, [(gf.I8, [1]), (gf.STR, ["a"])]))]
    gf.write_gguf(path, kvs, [("t", gf.T_F32, [4], bytes(16))])
    with q.Gguf(path) as g:
        for key, _, _ in kvs:
            ri, rf = ctypes.c_int64(), ctypes.c_double()
            rc = ref_lib().qref_gguf_value(os.fsencode(path), key.encode(), ctypes.byref(ri), ctypes.byref(rf))
            assert rc >= 0
            for bit, get, rv in ((1, g.get_int, ri), (2, g.get_float, rf)):
                if rc & bit:
                    with pytest.raises(q.QmsgError):
                        get(key)
                else:
                    got = get(key)
                    assert got == rv.value or (np.isnan(got) and np.isnan(rv.value)), key
        assert g.tensors()[0]["nbytes"] == 16


def bad_files(tmp_path):
    """(name, path) of files both readers must refuse."""
    ts = [("t", gf.T_F32, [64], bytes(256))]
    out = []
    p = str(tmp_path / "notgguf.gguf")
    open(p, "wb").write(b"GGML" + bytes(60))
    out.append(("magic", p))
    p = str(tmp_path / "v2.gguf")
    gf.write_gguf(p, [], ts, version=2)
    out.append(("version", p))
    p = str(tmp_path / "short_header.gguf")
    gf.write_gguf(p, [("k", gf.STR, "abcdef")], ts, truncate=30)
    out.append(("truncated metadata", p))
    p = str(tmp_path / "short_data.gguf")
    full = gf.write_gguf(p, [], ts)["t"] + 256
    gf.write_gguf(p, [], ts, truncate=full - 1)
    out.append(("tensor past end", p))
    p = str(tmp_path / "dims.gguf")
    gf.write_gguf(p, [], [("t", gf.T_F32, [1, 1, 1, 1, 64], bytes(256))])
    out.append(("five dims", p))
    p = str(tmp_path / "badtype.gguf")
    with open(p, "wb") as f:     # one metadata entry "k" of value type 13 (no such type)
        f.write(b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 1) + b"k" + struct.pack("<I", 13) +
                bytes(16))
    out.append(("unknown value type", p))
    out.append(("missing shard", str(tmp_path / "gone-00001-of-00002.gguf")))
    out.append(("missing file", str(tmp_path / "nothing.gguf")))
    return out


def test_bad_files_are_refused(q, tmp_path):
    for name, path in bad_files(tmp_path):
        with pytest.raises(q.QmsgError) as ei:
            q.Gguf(path)
        assert ei.value.status == -1, name
        if ref_lib() is not None:
            assert ref_table(path) is None, name


def _nested(depth):
    """An array value nested `depth` levels deep around one i8 array."""
    v = (gf.I8, [1, 2])
    for _ in range(depth - 1):
        v = (gf.ARR, [v])
    return v


def test_hostile_sizes_are_refused(q, tmp_path):
    """Sizes from the file that wrap 64-bit arithmetic or recurse without end are refused (the
    reader's own checks: the reference multiplies the tensor extent unchecked)."""
    cases = {
        "extent wraps": [("t", gf.T_F32, [2 ** 33, 2 ** 33], bytes(16))],
        "negative dim": [("t", gf.T_F32, [4, 2 ** 63 + 1], bytes(16))],
        "rows wrap": [("t", gf.T_Q4_0, [32, 2 ** 62, 4, 2], bytes(18))],
    }
    for name, ts in cases.items():
        p = str(tmp_path / (name.replace(" ", "_") + ".gguf"))
        gf.write_gguf(p, [], ts)
        with pytest.raises(q.QmsgError, match="does not fit") as ei:
            q.Gguf(p)
        assert ei.value.status == -1, name
    p = str(tmp_path / "deep.gguf")
    gf.write_gguf(p, [("deep", gf.ARR, _nested(20))], [("t", gf.T_F32, [4], bytes(16))])
    with pytest.raises(q.QmsgError, match="metadata"):
        q.Gguf(p)
    p = str(tmp_path / "shallow.gguf")
    gf.write_gguf(p, [("deep", gf.ARR, _nested(8)), ("k", gf.U8, 3)], [("t", gf.T_F32, [4], bytes(16))])
    with q.Gguf(p) as g:
        assert g.get_int("k") == 3
    p = str(tmp_path / "count_wraps.gguf")
    with open(p, "wb") as f:     # one metadata entry "a": an u32 array of 2^62 + 1 elements
        f.write(b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 1) + b"a" +
                struct.pack("<IIQ", gf.ARR, gf.U32, 2 ** 62 + 1) + bytes(16))
    with pytest.raises(q.QmsgError, match="metadata"):
        q.Gguf(p)


def test_moe_cfg(q, tmp_path):
    lays = small_layers()
    path, _ = gf.moe_model(str(tmp_path / "m.gguf"), lays, eps=1e-5)
    with q.Gguf(path) as g:
        c = g.moe_cfg()
    assert c == {"n_embd": 256, "n_expert": 16, "n_used": 4, "n_ff_exp": 256, "n_layer": 2,
                 "eps": float(np.float32(1e-5))}
    p = str(tmp_path / "llama.gguf")
    gf.write_gguf(p, [("general.architecture", gf.STR, "llama")], [("t", gf.T_F32, [4], bytes(16))])
    with q.Gguf(p) as g, pytest.raises(q.QmsgError, match="not qwen3moe"):
        g.moe_cfg()
    p = str(tmp_path / "nokey.gguf")
    gf.write_gguf(p, [("general.architecture", gf.STR, "qwen3moe"), ("qwen3moe.block_count", gf.U32, 2)],
                  [("t", gf.T_F32, [4], bytes(16))])
    with q.Gguf(p) as g, pytest.raises(q.QmsgError, match="no numeric scalar"):
        g.moe_cfg()


@need_ref
def test_reference_loader_moe_equals_oracle(tmp_path):
    """The written file as the reference reads it (qms_model_load, then moe() of each layer)
    gives the oracle's output bit for bit: the file holds exactly the oracle's layers."""
    lays = small_layers((orc.T_Q4_0, orc.T_Q4_1, orc.T_Q6_K))
    path, _ = gf.moe_model(str(tmp_path / "m.gguf"), lays, n_shards=2)
    x = orc.make_input(256, 3, 5)
    for l, lay in enumerate(lays):
        out = np.empty_like(x)
        assert ref_lib().qref_gguf_moe(os.fsencode(path), l, x.ctypes.data, 3, out.ctypes.data) == 0
        assert np.array_equal(out.view(np.uint32), lay.moe(x).view(np.uint32)), l


@need_ref
def test_reference_loader_typed_experts_off_grid(tmp_path):
    """The same for Q8_0, F16 and F32 expert tensors at an n_embd off the integer kernels' grid
    (the layers the slot kernels run)."""
    import expert_types as et
    E, X, K, F, T = 288, 12, 3, 160, 4
    lays = [et.typed_layer(E, X, K, F, types, 70 + 10 * l)
            for l, types in enumerate(((orc.T_Q8_0, orc.T_Q8_0, orc.T_Q8_0),
                                       (orc.T_F16, orc.T_Q8_0, orc.T_F32)))]
    path, _ = gf.moe_model(str(tmp_path / "q8.gguf"), lays)
    x = orc.make_input(E, T, 5, rmsnorm=True)
    for l, lay in enumerate(lays):
        out = np.empty_like(x)
        assert ref_lib().qref_gguf_moe(os.fsencode(path), l, x.ctypes.data, T, out.ctypes.data) == 0
        assert np.array_equal(out.view(np.uint32), lay.moe(x).view(np.uint32)), l


def test_mutated_files_under_sanitizers(tmp_path):
    """The reader on 2,000 mutations of a valid model file (bit flips, bytes set to boundary
    integers, truncations; mostly in the header and tables), built from its own source with
    AddressSanitizer and UBSan as host code: every open either fails cleanly or gives a table
    and keys that can all be queried, with no sanitizer report."""
    import shutil
    import subprocess
    if shutil.which("g++") is None:
        pytest.skip("no g++")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    exe = str(tmp_path / "gguf_fuzz")
    cmd = ["g++", "-std=c++17", "-g", "-O1", "-fsanitize=address,undefined", "-fno-sanitize-recover=undefined",
           "-I", os.path.join(root, "include"), os.path.join(root, "large_model_amd", "csrc", "qmsg_gguf.cpp"),
           os.path.join(root, "tests", "gguf_fuzz.cpp"), "-o", exe]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        pytest.skip("sanitizer build unavailable: " + r.stderr[-200:])
    lays = [orc.Layer(256, 4, 2, 64, 40 + l, layer=l, down_type=dt)
            for l, dt in enumerate((orc.T_Q4_0, orc.T_Q4_1))]
    seed_path, _ = gf.moe_model(str(tmp_path / "seed.gguf"), lays, eps=1e-5)
    r = subprocess.run([exe, seed_path, "2000", "7"], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-2000:]
    assert "opened" in r.stdout and "ERROR" not in r.stderr, r.stderr[-2000:]
