"""TEST INFRASTRUCTURE ONLY: a Python restatement of the .lancius model-file
records, used by tests/ and tests/golden/make_golden.py to check the C loader
and writer of liblancius_graph (lancius_amd/csrc/host/graph_io.c).  Nothing in
the product imports it.

Record layout (bleeding/v11A1/src/core/lancius_serialize.c:13-63 writes it,
:65-259 reads it):
    magic u32 = 0x21434E41, node_count u32, then per node
    id u32, op u32 (sizeof(lancius_opcode) == 4), ndim u8, shape 4 x u64,
    input_count u32, input ids u32[input_count], attr_val f64,
    (kernel_h, kernel_w, stride, pad) u32[4], axes u32[4],
    is_view u8 [+ strides 4 x u64, view source id u32]      (v10+ only, :35-42)
    has_weights u8 [+ dtype u8, scale f64,
                    elements x i8 (dtype INT8) or x f64 (any other dtype)]
The v9 layout (stable/v9S/src/core/lancius_serialize.c) has no is_view byte.
Weights are written for INPUT nodes only (:44); their element count is that of
the rebuilt INPUT node, whose rank is 4 when ndim == 4 and 2 otherwise
(lancius_input / lancius_input_4d, bleeding/v11A1/src/ir/lancius_ir.c:145-153).

Pinned by: the reference's own shipped files (stable/v9S/*.lancius parse to
their exact length), files written by the reference's compiled
lancius_graph_save (tests/golden/models/ref_*.lancius), and the reference's
shipped LeNet logits (stable/v9S/lancius_out.bin) reproduced by running the
parsed graph through the compiled reference executor.
"""
from __future__ import annotations

import struct

import numpy as np

MAGIC_V1 = 0x21434E41
DTYPE_FP64, DTYPE_INT8 = 0, 1
OP_INPUT = 1


def input_elements(ndim: int, shape) -> int:
    if ndim == 4:
        return int(shape[0] * shape[1] * shape[2] * shape[3])
    return int(shape[0] * shape[1])


def read_records(data: bytes, layout: int) -> list[dict]:
    """Every record of a v9 (layout=9) or v10 (layout=10) file.  Raises
    ValueError unless the records end exactly at the end of the data."""
    off = 0

    def take(fmt: str):
        nonlocal off
        size = struct.calcsize(fmt)
        if off + size > len(data):
            raise ValueError("truncated")
        vals = struct.unpack_from(fmt, data, off)
        off += size
        return vals

    magic, count = take("<II")
    if magic != MAGIC_V1:
        raise ValueError("bad magic")
    recs = []
    for _ in range(count):
        nid, op, ndim = take("<IIB")
        shape = take("<4Q")
        (ic,) = take("<I")
        if ic > 16:
            raise ValueError("input count")
        ins = take(f"<{ic}I") if ic else ()
        (attr,) = take("<d")
        meta = take("<4I")
        axes = take("<4I")
        rec = {"id": nid, "op": op, "ndim": ndim, "shape": shape, "inputs": ins, "attr": attr, "meta": meta,
               "axes": axes, "is_view": 0, "strides": (0, 0, 0, 0), "view_source": 0xFFFFFFFF, "weights": None}
        if layout == 10:
            (rec["is_view"],) = take("<B")
            if rec["is_view"] > 1:
                raise ValueError("is_view")
            if rec["is_view"]:
                rec["strides"] = take("<4Q")
                (rec["view_source"],) = take("<I")
        (has_w,) = take("<B")
        if has_w > 1:
            raise ValueError("has_weights")
        if has_w:
            if op != OP_INPUT:
                raise ValueError("weights on a non-INPUT record")
            dtype, scale = take("<Bd")
            e = input_elements(ndim, shape)
            if dtype == DTYPE_INT8:
                w = np.frombuffer(data, dtype=np.int8, count=e, offset=off).copy()
                off += e
            else:
                w = np.frombuffer(data, dtype="<f8", count=e, offset=off).copy()
                off += 8 * e
            if off > len(data):
                raise ValueError("truncated weights")
            rec.update(dtype=dtype, scale=scale, weights=w)
        recs.append(rec)
    if off != len(data):
        raise ValueError(f"{len(data) - off} trailing bytes")
    return recs


def write_records(recs: list[dict], layout: int = 10) -> bytes:
    """Bytes of the records as lancius_graph_save writes them (layout 10) or
    the v9 layout."""
    out = [struct.pack("<II", MAGIC_V1, len(recs))]
    for r in recs:
        out.append(struct.pack("<IIB", r["id"], r["op"], r["ndim"]))
        out.append(struct.pack("<4Q", *r["shape"]))
        out.append(struct.pack("<I", len(r["inputs"])))
        if r["inputs"]:
            out.append(struct.pack(f"<{len(r['inputs'])}I", *r["inputs"]))
        out.append(struct.pack("<d", r["attr"]))
        out.append(struct.pack("<4I", *r["meta"]))
        out.append(struct.pack("<4I", *r["axes"]))
        if layout == 10:
            out.append(struct.pack("<B", r["is_view"]))
            if r["is_view"]:
                out.append(struct.pack("<4Q", *r["strides"]))
                out.append(struct.pack("<I", r["view_source"]))
        w = r["weights"]
        out.append(struct.pack("<B", 0 if w is None else 1))
        if w is not None:
            out.append(struct.pack("<Bd", r["dtype"], r["scale"]))
            out.append(np.ascontiguousarray(w, dtype=np.int8 if r["dtype"] == DTYPE_INT8 else "<f8").tobytes())
    return b"".join(out)
