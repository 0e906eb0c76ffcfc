""".lancius model files on the host (liblancius_graph: lancius_graph_load /
_save / _save_v2 / _load_mapped, lancius_crc32), checked against:

  * the reference's own files: stable/v9S/*.lancius (v9 records, which the
    reference's v10+ loader cannot read) and v10 files written by the
    reference's compiled lancius_graph_save (tests/golden/models/ref_*.lancius);
  * oracle/model_file.py, the Python restatement of the record layout, itself
    pinned here by re-serialising the shipped files byte for byte;
  * zlib.crc32 for the v2 checksum.
"""
import ctypes as C
import struct
import zlib
from pathlib import Path

import numpy as np
import pytest

import oracle
from lancius_amd import abi, graph_lib, graphs
from oracle import model_file as mf

MODELS = Path(__file__).resolve().parent / "golden" / "models"
V9_FILES = ["pytorch_lenet", "test_model", "cifar10_lenet"]
REF_V10 = [f"ref_{n}" for n in graphs.IO_GRAPHS]


def data_of(name: str) -> bytes:
    return (MODELS / f"{name}.lancius").read_bytes()


def load(path, mapped=False):
    lib = graph_lib()
    lib.lancius_clear_error()
    if mapped:
        wm = abi.WeightMap()
        g = lib.lancius_graph_load_mapped(str(path).encode(), C.byref(wm))
        return g, wm
    return lib.lancius_graph_load(str(path).encode())


def nodes_of(g):
    return [g.contents.nodes[i] for i in range(g.contents.node_count)]


def check_against_records(g, recs, weights_loaded=True):
    """Every non-NOP record rebuilt in order with its attributes, inputs and
    weights (lancius_serialize.c:137-240)."""
    kept = [r for r in recs if r["op"] != abi.OP["NOP"]]
    nodes = nodes_of(g)
    assert len(nodes) == len(kept)
    by_file_id = {}
    for r, n in zip(kept, nodes):
        c = n.contents
        assert c.op == r["op"]
        assert (c.kernel_h, c.kernel_w, c.stride, c.pad) == r["meta"]
        assert tuple(c.axes) == r["axes"]
        assert c.attr_val == r["attr"]
        assert c.is_view == r["is_view"]
        if r["is_view"]:
            assert tuple(c.strides) == r["strides"]
            assert c.view_source.contents.id == by_file_id[r["view_source"]].contents.id
        assert [c.inputs[j].contents.id for j in range(c.input_count)] == [
            by_file_id[i].contents.id for i in r["inputs"]]
        if r["op"] in (abi.OP["INPUT"], abi.OP["RESHAPE"], abi.OP["CONST"]):
            nd = 4 if r["ndim"] == 4 else (r["ndim"] if r["op"] == abi.OP["RESHAPE"] else 2)
            assert abi.node_shape(n) == tuple(r["shape"][:nd])
        by_file_id[r["id"]] = n
        w = r["weights"]
        if w is None:
            assert not c.runtime_data and not c.runtime_data_int8
            continue
        assert c.dtype == r["dtype"] and c.scale == r["scale"]
        if not weights_loaded:
            assert not c.runtime_data and not c.runtime_data_int8
        elif r["dtype"] == abi.DTYPE_INT8:
            got = np.ctypeslib.as_array(c.runtime_data_int8, shape=(w.size,))
            np.testing.assert_array_equal(got, w)
        else:
            got = np.ctypeslib.as_array(c.runtime_data, shape=(w.size,))
            np.testing.assert_array_equal(got, w)  # bit for bit
    return by_file_id


# ---- CRC-32 ---------------------------------------------------------------------------


@pytest.mark.parametrize("n", [0, 1, 7, 8, 9, 63, 1000, 1 << 20, (40 << 20) + 7])
def test_crc32_matches_zlib(n):
    """Serial below 8 MiB; above, chunk CRCs on threads joined by the
    x^(8 len) mod P combination."""
    lib = graph_lib()
    buf = np.random.default_rng(n).integers(0, 256, n, dtype=np.uint8).tobytes()
    assert lib.lancius_crc32(0, buf, n) == zlib.crc32(buf)
    assert lib.lancius_crc32(0xDEADBEEF, buf, n) == zlib.crc32(buf, 0xDEADBEEF)
    # chained: crc(a + b) == crc(crc(a), b)
    h = n // 3
    assert lib.lancius_crc32(lib.lancius_crc32(0, buf[:h], h), buf[h:], n - h) == zlib.crc32(buf)


def test_crc32_check_value():
    # the standard check value of CRC-32/ISO-HDLC
    assert graph_lib().lancius_crc32(0, b"123456789", 9) == 0xCBF43926


# ---- the restatement is pinned by the reference's files --------------------------------


@pytest.mark.parametrize("name", V9_FILES)
def test_restatement_reproduces_v9_files(name):
    data = data_of(name)
    recs = mf.read_records(data, 9)
    assert mf.write_records(recs, 9) == data
    with pytest.raises(ValueError):
        mf.read_records(data, 10)


@pytest.mark.parametrize("name", REF_V10)
def test_restatement_reproduces_reference_v10_files(name):
    data = data_of(name)
    recs = mf.read_records(data, 10)
    assert mf.write_records(recs, 10) == data


def test_lenet_records_match_the_reference_logits():
    """The reference's loader and executor on the LeNet records (re-laid as
    v10 by the restatement) reproduce the logits the reference shipped."""
    K = np.load(Path(__file__).resolve().parent / "golden" / "model_io.npz")
    shipped = np.fromfile(MODELS / "lancius_out.bin", dtype="<f4")
    onnx = np.fromfile(MODELS / "baseline_out.bin", dtype="<f4")
    assert oracle.normwise_error(shipped, K["lenet_logits"]) < 1e-7
    assert oracle.normwise_error(onnx, K["lenet_logits"]) < 2e-6
    assert int(np.argmax(K["lenet_logits"])) == int(np.argmax(onnx)) == 7


# ---- the C loader ------------------------------------------------------------------------


@pytest.mark.parametrize("name", V9_FILES + REF_V10)
def test_load_matches_records(name):
    layout = 9 if name in V9_FILES else 10
    recs = mf.read_records(data_of(name), layout)
    g = load(MODELS / f"{name}.lancius")
    assert g, f"load failed: {graph_lib().lancius_get_error()}"
    check_against_records(g, recs)
    graph_lib().lancius_graph_destroy(g)  # frees the loaded weights


@pytest.mark.parametrize("name", V9_FILES + REF_V10)
def test_load_mapped_offsets(name):
    layout = 9 if name in V9_FILES else 10
    data = data_of(name)
    recs = mf.read_records(data, layout)
    g, wm = load(MODELS / f"{name}.lancius", mapped=True)
    assert g
    assert wm.format == layout and wm.file_bytes == len(data) and wm.crc32 == 0
    by_id = check_against_records(g, recs, weights_loaded=False)
    weighted = [r for r in recs if r["weights"] is not None]
    assert wm.count == len(weighted)
    for k, r in enumerate(weighted):
        ref = wm.refs[k]
        assert ref.node.contents.id == by_id[r["id"]].contents.id
        w = r["weights"]
        assert ref.elements == w.size and ref.scale == r["scale"]
        assert ref.file_dtype == (abi.DTYPE_INT8 if r["dtype"] == abi.DTYPE_INT8 else abi.DTYPE_FP64)
        raw = data[ref.file_offset:ref.file_offset + w.nbytes]
        assert raw == np.ascontiguousarray(w).tobytes()
    graph_lib().lancius_weight_map_free(C.byref(wm))
    graph_lib().lancius_graph_destroy(g)


def test_mapped_int8_weights_keep_dtype_through_set_dtype():
    g, wm = load(MODELS / "cifar10_lenet.lancius", mapped=True)
    lib = graph_lib()
    lib.lancius_graph_set_dtype(g, abi.DTYPE_FP32)
    i8 = [n for n in nodes_of(g) if n.contents.op == abi.OP["INPUT"] and n.contents.dtype == abi.DTYPE_INT8]
    assert len(i8) == 3  # image and both filters
    lib.lancius_weight_map_free(C.byref(wm))
    lib.lancius_graph_destroy(g)


# ---- the C writer -------------------------------------------------------------------------


@pytest.mark.parametrize("name", graphs.IO_GRAPHS)
def test_save_is_byte_identical_to_the_reference(tmp_path, name):
    lib = graph_lib()
    bg = graphs.build_io_graph(lib, name)
    path = tmp_path / "mine.lancius"
    lib.lancius_graph_save(bg.g, str(path).encode())
    assert path.read_bytes() == data_of(f"ref_{name}")
    bg.destroy()


@pytest.mark.parametrize("name", V9_FILES)
def test_v9_resaved_as_v10(tmp_path, name):
    """load (v9) -> save writes exactly the restatement's v10 layout of the
    same records (NOP records dropped and ids renumbered, as a reference
    load + save would)."""
    g = load(MODELS / f"{name}.lancius")
    path = tmp_path / "v10.lancius"
    graph_lib().lancius_graph_save(g, str(path).encode())
    recs10 = mf.read_records(path.read_bytes(), 10)
    recs9 = [r for r in mf.read_records(data_of(name), 9) if r["op"] != abi.OP["NOP"]]
    assert len(recs10) == len(recs9)
    for a, b in zip(recs10, recs9):
        assert a["op"] == b["op"] and a["meta"] == b["meta"]
        if b["weights"] is not None:
            np.testing.assert_array_equal(a["weights"], b["weights"])
    g2 = load(path)
    check_against_records(g2, recs10)
    graph_lib().lancius_graph_destroy(g2)
    graph_lib().lancius_graph_destroy(g)


def test_reference_loader_reads_our_files(tmp_path):
    """The reference's lancius_graph_load on files our lancius_graph_save
    wrote, for graphs whose ops are all in that loader's subset (it skips
    BROADCAST and GELU, lancius_serialize.c:175-176, which then breaks every
    node after them)."""
    ref = oracle.ref_lib()
    if ref is None:
        pytest.skip("reference library not built")
    lib = graph_lib()
    bg = graphs.build_io_graph(lib, "io_conv_i8")
    sources = [("io_conv_i8", bg.g)] + [(n, load(MODELS / f"{n}.lancius")) for n in ("pytorch_lenet", "test_model")]
    for name, g in sources:
        path = tmp_path / f"{name}.lancius"
        lib.lancius_graph_save(g, str(path).encode())
        rg = ref.lancius_graph_load(str(path).encode())
        assert rg, name
        check_against_records(rg, mf.read_records(path.read_bytes(), 10))
    for _, g in sources[1:]:
        lib.lancius_graph_destroy(g)
    bg.destroy()


# ---- v2 container ----------------------------------------------------------------------------


def _v2_header(data: bytes) -> dict:
    f = struct.unpack_from("<7IIQII", data, 0)
    keys = ["magic", "version", "flags", "node_count", "tensor_count", "attribute_count", "header_size",
            "reserved0", "weight_block_offset", "checksum_crc32", "reserved1"]
    return dict(zip(keys, f))


@pytest.mark.parametrize("src", ["pytorch_lenet", "ref_io_conv_i8", "ref_io_mlp"])
@pytest.mark.parametrize("wdtype", [abi.DTYPE_FP64, abi.DTYPE_FP32])
def test_v2_roundtrip(tmp_path, src, wdtype):
    lib = graph_lib()
    layout = 9 if src in V9_FILES else 10
    recs = [r for r in mf.read_records(data_of(src), layout) if r["op"] != abi.OP["NOP"]]
    g = load(MODELS / f"{src}.lancius")
    path = tmp_path / "m.lancius2"
    assert lib.lancius_graph_save_v2(g, str(path).encode(), wdtype) == 0
    data = path.read_bytes()
    h = _v2_header(data)
    assert h["magic"] == 0x32434E41 and h["version"] == 2 and h["header_size"] == 48
    assert h["flags"] == 3 and h["reserved0"] == 0 and h["reserved1"] == 0
    assert h["node_count"] == len(recs) == h["attribute_count"]
    assert h["tensor_count"] == sum(r["weights"] is not None for r in recs)
    assert h["weight_block_offset"] % 4096 == 0
    assert h["checksum_crc32"] == zlib.crc32(data[48:])
    g2, wm = load(path, mapped=True)
    assert g2 and wm.format == 2 and wm.crc32 == h["checksum_crc32"]
    for k in range(wm.count):
        assert (wm.refs[k].file_offset - h["weight_block_offset"]) % 256 == 0
    g3 = load(path)
    if wdtype == abi.DTYPE_FP32:
        for r in recs:  # fp64 weights come back rounded to fp32
            if r["weights"] is not None and r["dtype"] != abi.DTYPE_INT8:
                r["weights"] = r["weights"].astype(np.float32).astype(np.float64)
    check_against_records(g3, recs)
    for k in range(wm.count):
        r = wm.refs[k]
        want = abi.DTYPE_INT8 if r.node.contents.dtype == abi.DTYPE_INT8 else wdtype
        assert r.file_dtype == want
    lib.lancius_weight_map_free(C.byref(wm))
    for x in (g, g2, g3):
        lib.lancius_graph_destroy(x)


def test_v2_rejects_corruption(tmp_path):
    lib = graph_lib()
    g = load(MODELS / "ref_io_mlp.lancius")
    path = tmp_path / "m.lancius2"
    assert lib.lancius_graph_save_v2(g, str(path).encode(), abi.DTYPE_FP64) == 0
    lib.lancius_graph_destroy(g)
    data = bytearray(path.read_bytes())
    h = _v2_header(bytes(data))
    for at in (60, 200, h["weight_block_offset"] + 5, len(data) - 1):  # records and weights
        bad = bytearray(data)
        bad[at] ^= 0x40
        p = tmp_path / f"bad{at}"
        p.write_bytes(bytes(bad))
        assert not load(p)
        assert lib.lancius_get_error() == -6  # LANCIUS_ERROR_INVALID_MODEL
    for field, off, val in (("version", 4, 3), ("header_size", 24, 64), ("flags", 8, 0)):
        bad = bytearray(data)
        struct.pack_into("<I", bad, off, val)
        p = tmp_path / f"hdr_{field}"
        p.write_bytes(bytes(bad))
        assert not load(p), field
    p = tmp_path / "short"
    p.write_bytes(bytes(data[:h["weight_block_offset"] + 3]))
    assert not load(p)


# ---- malformed input ----------------------------------------------------------------------------


def test_truncated_files_fail_cleanly(tmp_path):
    lib = graph_lib()
    data = data_of("ref_io_mlp")
    cuts = sorted(set(list(range(0, 64)) + list(range(64, len(data), 37)) + [len(data) - 1]))
    for cut in cuts:
        p = tmp_path / "t.lancius"
        p.write_bytes(data[:cut])
        g = load(p)
        if g:  # a prefix can never be a complete file of these records
            lib.lancius_graph_destroy(g)
            raise AssertionError(f"truncated at {cut} loaded")
        assert lib.lancius_get_error() in (-6, -8)


def test_malformed_headers_and_records(tmp_path):
    lib = graph_lib()
    data = bytearray(data_of("test_model"))

    def fails(buf: bytes) -> bool:
        p = tmp_path / "m.lancius"
        p.write_bytes(buf)
        g = load(p)
        if g:
            lib.lancius_graph_destroy(g)
        return not g

    bad = bytearray(data)
    bad[0] ^= 1
    assert fails(bytes(bad))  # magic
    bad = bytearray(data)
    struct.pack_into("<I", bad, 4, 2_000_000)
    assert fails(bytes(bad))  # node count over the sanity limit
    # record 0: id at 8, op 12, ndim 16, shape 17..48, input_count 49
    bad = bytearray(data)
    struct.pack_into("<I", bad, 8, 4 + 1000)
    assert fails(bytes(bad))  # id beyond node_count + 1000
    bad = bytearray(data)
    struct.pack_into("<I", bad, 49, 17)
    assert fails(bytes(bad))  # more than 16 inputs
    bad = bytearray(data)
    bad[16] = 5
    assert fails(bytes(bad))  # rank 5
    assert fails(b"")
    assert not load(tmp_path / "does_not_exist.lancius")
    assert lib.lancius_get_error() == -8  # LANCIUS_ERROR_IO


def test_overflowing_shapes_fail(tmp_path):
    """Element counts are formed with overflow checks: a record of shape
    [2^32, 2^32] (whose product wraps to 0 in 64 bits) and a MATMUL whose
    derived shape overflows both fail the load, with or without a payload."""
    lib = graph_lib()
    recs = mf.read_records(data_of("test_model"), 9)
    # test_model: x, W (weights), MATMUL(x, W), RELU(MATMUL)

    def fails(r) -> bool:
        """The loader refuses the v10 file, or (the layout is found by
        parsing) reads it as some other v9 record stream in which every node
        has a representable element count and none has the crafted dims."""
        p = tmp_path / "o.lancius"
        p.write_bytes(mf.write_records(r, 10))
        g = load(p)
        if not g:
            return True
        ok = True
        for i in range(g.contents.node_count):
            n = g.contents.nodes[i].contents
            dims = [int(d) for d in n.shape[:n.ndim]]
            ok = ok and float(np.prod([float(d) for d in dims])) <= 2.0 ** 40 and max(dims, default=0) < 1 << 32
        lib.lancius_graph_destroy(g)
        return ok

    r = [dict(x) for x in recs]
    r[0]["shape"] = (1 << 32, 1 << 32, 0, 0)  # x, no payload
    assert fails(r)
    r = [dict(x) for x in recs]
    r[1].update(shape=(1 << 32, 1 << 32, 0, 0), weights=np.zeros(0))  # W: wrapped count 0 would match 0 bytes
    assert fails(r)
    r = [dict(x) for x in recs]
    r[0]["shape"] = (1 << 33, 20, 0, 0)  # x [2^33, 20] and W [20, 2^33] are representable ...
    r[1].update(shape=(20, 1 << 33, 0, 0), weights=None)
    assert fails(r)  # ... the MATMUL the builder derives, [2^33, 2^33], is not
    p = tmp_path / "ok.lancius"
    p.write_bytes(mf.write_records([dict(x) for x in recs], 10))
    g = load(p)
    assert g and g.contents.node_count == len(recs)
    lib.lancius_graph_destroy(g)


def test_unknown_op_is_skipped_and_its_readers_fail(tmp_path):
    recs = mf.read_records(data_of("test_model"), 9)
    # test_model: x, W (weights), MATMUL(x, W), RELU(MATMUL)
    r = [dict(x) for x in recs]
    r[3]["op"] = 99  # RELU -> unknown: skipped, nothing reads it
    p = tmp_path / "a.lancius"
    p.write_bytes(mf.write_records(r, 10))
    g = load(p)
    assert g and g.contents.node_count == 3
    graph_lib().lancius_graph_destroy(g)
    r = [dict(x) for x in recs]
    r[2]["op"] = 99  # MATMUL -> unknown: the RELU reading it cannot be built
    p.write_bytes(mf.write_records(r, 10))
    assert not load(p)
