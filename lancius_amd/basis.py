"""ctypes side of include/lancius_basis.h: the BASIS graph builders
(liblancius_graph.so, or any library with the reference's graph.c names),
the BASIS memory API on HBM and the device executor for BASIS graphs
(liblancius_hip.so)."""
from __future__ import annotations

import ctypes as C

import numpy as np

from .runtime import Device, HipError, _check

OP = {"INPUT": 0, "MATMUL": 1, "ADD": 2, "RELU": 3, "TANH": 4, "BROADCAST_ADD": 5}
KEEP_ALL = 0x1


class BasisNode(C.Structure):
    """basis_node (include/basis/stage6_ir/graph.h:16-23)."""
    _fields_ = [("id", C.c_int), ("op", C.c_int), ("input_ids", C.c_int * 2), ("rows", C.c_size_t),
                ("cols", C.c_size_t), ("name", C.c_char_p)]


class BasisGraph(C.Structure):
    """basis_graph (include/basis/stage6_ir/graph.h:25-29)."""
    _fields_ = [("nodes", C.POINTER(BasisNode)), ("node_count", C.c_size_t), ("node_cap", C.c_size_t)]


NodeP, GraphP = C.POINTER(BasisNode), C.POINTER(BasisGraph)


def declare_builders(lib: C.CDLL) -> C.CDLL:
    lib.basis_graph_new.restype = GraphP
    lib.basis_graph_input.argtypes = [GraphP, C.c_char_p, C.c_size_t, C.c_size_t]
    for name in ("basis_graph_input", "basis_graph_matmul", "basis_graph_add", "basis_graph_broadcast_add",
                 "basis_graph_relu", "basis_graph_tanh"):
        getattr(lib, name).restype = NodeP
    for name in ("basis_graph_matmul", "basis_graph_add", "basis_graph_broadcast_add"):
        getattr(lib, name).argtypes = [GraphP, NodeP, NodeP]
    lib.basis_graph_relu.argtypes = [GraphP, NodeP]
    lib.basis_graph_tanh.argtypes = [GraphP, NodeP]
    lib.basis_graph_print.argtypes = [GraphP]
    lib.basis_graph_print.restype = None
    lib.basis_graph_free.argtypes = [GraphP]
    lib.basis_graph_free.restype = None
    return lib


def declare_device(lib: C.CDLL) -> C.CDLL:
    vp, sz, i32 = C.c_void_p, C.c_size_t, C.c_int
    lib.basis_arena_create.argtypes = [sz]
    lib.basis_arena_create.restype = vp
    lib.basis_arena_alloc.argtypes = [vp, sz, sz]
    lib.basis_arena_alloc.restype = vp
    lib.basis_arena_reset.argtypes = [vp]
    lib.basis_arena_reset.restype = None
    lib.basis_arena_destroy.argtypes = [vp]
    lib.basis_arena_destroy.restype = None
    lib.basis_pool_create.argtypes = [sz, sz]
    lib.basis_pool_create.restype = vp
    lib.basis_pool_alloc.argtypes = [vp]
    lib.basis_pool_alloc.restype = vp
    lib.basis_pool_free.argtypes = [vp, vp]
    lib.basis_pool_free.restype = None
    lib.basis_pool_destroy.argtypes = [vp]
    lib.basis_pool_destroy.restype = None
    lib.lancius_basis_arena_capacity.argtypes = [vp]
    lib.lancius_basis_arena_capacity.restype = sz
    lib.lancius_basis_pool_capacity.argtypes = [vp]
    lib.lancius_basis_pool_capacity.restype = sz
    lib.lancius_basis_program_create.argtypes = [vp, GraphP, C.c_uint, C.POINTER(vp)]
    lib.lancius_basis_program_upload.argtypes = [vp, i32, vp, sz]
    lib.lancius_basis_program_run.argtypes = [vp]
    lib.lancius_basis_program_download.argtypes = [vp, i32, vp, sz]
    lib.lancius_basis_program_buffer.argtypes = [vp, i32]
    lib.lancius_basis_program_buffer.restype = vp
    lib.lancius_basis_program_info.argtypes = [vp, C.POINTER(sz), C.POINTER(sz)]
    lib.lancius_basis_program_destroy.argtypes = [vp]
    lib.lancius_basis_program_destroy.restype = None
    return lib


class Graph:
    """A basis_graph built through `lib`'s builders.  Operands are passed as
    copies of their nodes (the builders read only id and shape), so no
    pointer into the growing node array is ever held across a call."""

    def __init__(self, lib: C.CDLL):
        self.lib = declare_builders(lib)
        self.g = lib.basis_graph_new()
        if not self.g:
            raise MemoryError("basis_graph_new")

    def node(self, i: int) -> BasisNode:
        n = self.g.contents.nodes[i]
        c = BasisNode()
        C.memmove(C.byref(c), C.byref(n), C.sizeof(BasisNode))
        return c

    @property
    def count(self) -> int:
        return int(self.g.contents.node_count)

    def _id(self, p) -> int | None:
        return int(p.contents.id) if p else None

    def input(self, name: str, rows: int, cols: int) -> int | None:
        return self._id(self.lib.basis_graph_input(self.g, name.encode(), rows, cols))

    def matmul(self, a: int, b: int) -> int | None:
        return self._id(self.lib.basis_graph_matmul(self.g, C.byref(self.node(a)), C.byref(self.node(b))))

    def add(self, a: int, b: int) -> int | None:
        return self._id(self.lib.basis_graph_add(self.g, C.byref(self.node(a)), C.byref(self.node(b))))

    def broadcast_add(self, a: int, bias: int) -> int | None:
        return self._id(self.lib.basis_graph_broadcast_add(self.g, C.byref(self.node(a)), C.byref(self.node(bias))))

    def relu(self, a: int) -> int | None:
        return self._id(self.lib.basis_graph_relu(self.g, C.byref(self.node(a))))

    def tanh(self, a: int) -> int | None:
        return self._id(self.lib.basis_graph_tanh(self.g, C.byref(self.node(a))))

    def close(self) -> None:
        if self.g:
            self.lib.basis_graph_free(self.g)
            self.g = None


class Program:
    """lancius_basis_program_*: a BASIS graph compiled for the device."""

    def __init__(self, dev: Device, graph: Graph, flags: int = 0):
        self.dev = dev
        self.lib = declare_device(dev.lib)
        self.graph = graph
        self.p = C.c_void_p()
        _check(self.lib.lancius_basis_program_create(dev.ctx, graph.g, flags, C.byref(self.p)))

    def upload(self, node_id: int, arr) -> None:
        a = np.ascontiguousarray(arr, dtype=np.float32)
        _check(self.lib.lancius_basis_program_upload(self.p, node_id, a.ctypes.data_as(C.c_void_p), a.size))

    def run(self) -> None:
        _check(self.lib.lancius_basis_program_run(self.p))

    def download(self, node_id: int) -> np.ndarray:
        n = self.graph.node(node_id)
        out = np.empty((n.rows, n.cols), np.float32)
        _check(self.lib.lancius_basis_program_download(self.p, node_id, out.ctypes.data_as(C.c_void_p), out.size))
        return out

    def buffer(self, node_id: int) -> int | None:
        return self.lib.lancius_basis_program_buffer(self.p, node_id)

    def info(self) -> dict:
        launches, arena = C.c_size_t(), C.c_size_t()
        _check(self.lib.lancius_basis_program_info(self.p, C.byref(launches), C.byref(arena)))
        return {"launches": int(launches.value), "arena_bytes": int(arena.value)}

    def close(self) -> None:
        if self.p:
            self.lib.lancius_basis_program_destroy(self.p)
            self.p = C.c_void_p()


__all__ = ["OP", "KEEP_ALL", "BasisNode", "BasisGraph", "Graph", "Program", "declare_builders", "declare_device",
           "HipError"]
