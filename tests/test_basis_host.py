"""The BASIS static graph builders of liblancius_graph.so against the
reference's own src/basis/stage6_ir/graph.c (compiled from its source into
oracle/_ref/libbasis_ref.so by oracle/Makefile): the same node arrays, shape
rules and print-out for the same build sequence."""
import ctypes as C
import os
import tempfile
from pathlib import Path

import pytest

from lancius_amd import graph_lib
from lancius_amd.basis import OP, Graph

REF_BASIS = Path(__file__).resolve().parents[1] / "oracle" / "_ref" / "libbasis_ref.so"
needs_ref = pytest.mark.skipif(not REF_BASIS.exists(), reason="reference build (oracle/_ref) not present")


def _ref_lib():
    return C.CDLL(str(REF_BASIS))


def _mlp_sequence(g: Graph) -> dict:
    """x . W1 + b1 -> tanh -> . W2 + b2 -> relu, a residual add and enough
    extra nodes to make the node array grow past 16 and 32 entries."""
    ids = {}
    ids["x"] = g.input("x", 64, 32)
    ids["W1"] = g.input("W1", 32, 48)
    ids["b1"] = g.input("b1", 1, 48)
    ids["h"] = g.matmul(ids["x"], ids["W1"])
    ids["hb"] = g.broadcast_add(ids["h"], ids["b1"])
    ids["ht"] = g.tanh(ids["hb"])
    ids["W2"] = g.input("W2", 48, 48)
    ids["b2"] = g.input("b2", 1, 48)
    ids["y"] = g.matmul(ids["ht"], ids["W2"])
    ids["yb"] = g.broadcast_add(ids["y"], ids["b2"])
    ids["yr"] = g.relu(ids["yb"])
    ids["res"] = g.add(ids["yr"], ids["ht"])
    prev = ids["res"]
    for i in range(30):
        prev = g.tanh(prev) if i % 2 else g.relu(prev)
    ids["last"] = prev
    return ids


def _nodes(g: Graph):
    out = []
    for i in range(g.count):
        n = g.node(i)
        out.append((n.id, n.op, tuple(n.input_ids), n.rows, n.cols, n.name.decode() if n.name else None))
    return out


def test_builders_shapes_and_ids():
    g = Graph(graph_lib())
    ids = _mlp_sequence(g)
    nodes = _nodes(g)
    assert g.count == 42 and g.g.contents.node_cap == 64  # 16 -> 32 -> 64
    assert nodes[ids["h"]] == (ids["h"], OP["MATMUL"], (ids["x"], ids["W1"]), 64, 48, None)
    assert nodes[ids["hb"]][1:5] == (OP["BROADCAST_ADD"], (ids["h"], ids["b1"]), 64, 48)
    assert nodes[ids["ht"]][1:3] == (OP["TANH"], (ids["hb"], -1))
    assert nodes[ids["res"]][1:5] == (OP["ADD"], (ids["yr"], ids["ht"]), 64, 48)
    assert nodes[ids["x"]] == (0, OP["INPUT"], (-1, -1), 64, 32, "x")
    assert [n[0] for n in nodes] == list(range(g.count))
    g.close()


def test_shape_errors_return_null_and_add_nothing(capfd):
    g = Graph(graph_lib())
    a, b = g.input("a", 4, 5), g.input("b", 6, 7)
    row = g.input("row", 2, 5)
    assert g.matmul(a, b) is None
    assert g.add(a, b) is None
    assert g.broadcast_add(a, row) is None
    assert g.count == 3
    err = capfd.readouterr().err
    assert err.count("[BASIS IR]") == 3
    g.close()


def test_null_operands_are_rejected():
    lib = graph_lib()
    g = Graph(lib)
    x = g.input("x", 2, 2)
    assert not lib.basis_graph_matmul(g.g, None, C.byref(g.node(x)))
    assert not lib.basis_graph_relu(g.g, None)
    assert not lib.basis_graph_input(None, b"x", 1, 1)
    lib.basis_graph_free(None)
    g.close()


def _printed(g: Graph) -> str:
    libc = C.CDLL(None)
    with tempfile.TemporaryFile(mode="w+b") as f:
        saved = os.dup(1)
        os.dup2(f.fileno(), 1)
        try:
            g.lib.basis_graph_print(g.g)
            libc.fflush(None)
        finally:
            os.dup2(saved, 1)
            os.close(saved)
        f.seek(0)
        return f.read().decode()


@needs_ref
def test_same_nodes_as_reference_builders():
    ours, ref = Graph(graph_lib()), Graph(_ref_lib())
    ids_o, ids_r = _mlp_sequence(ours), _mlp_sequence(ref)
    assert ids_o == ids_r
    assert _nodes(ours) == _nodes(ref)
    assert (ours.g.contents.node_count, ours.g.contents.node_cap) == (ref.g.contents.node_count,
                                                                      ref.g.contents.node_cap)
    ours.close()
    ref.close()


@needs_ref
def test_shape_rules_match_reference():
    for build in (lambda g, a, b, r: g.matmul(a, b), lambda g, a, b, r: g.add(a, b),
                  lambda g, a, b, r: g.broadcast_add(a, r), lambda g, a, b, r: g.matmul(a, r),
                  lambda g, a, b, r: g.add(a, a), lambda g, a, b, r: g.broadcast_add(b, r)):
        results = []
        for lib in (graph_lib(), _ref_lib()):
            g = Graph(lib)
            a, b, r = g.input("a", 3, 5), g.input("b", 5, 3), g.input("r", 1, 3)
            got = build(g, a, b, r)
            results.append((got, _nodes(g)))
            g.close()
        assert results[0] == results[1]


@needs_ref
def test_print_matches_reference():
    ours, ref = Graph(graph_lib()), Graph(_ref_lib())
    _mlp_sequence(ours)
    _mlp_sequence(ref)
    text = _printed(ours)
    assert text == _printed(ref)
    assert text.startswith("=== BASIS Static Graph IR ===\n") and 'None (Name: "W1")' in text
    ours.close()
    ref.close()
