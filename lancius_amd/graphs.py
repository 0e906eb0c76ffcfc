"""The BASELINE.json config graphs, built through any library that exports
the Lancius graph API (liblancius_graph.so here, or the reference library).

Recipes (node creation order matters: it fixes ids, wave order and plan
offsets):
  mlp    INPUT x[64,784], W1[784,256], b1[1,256], W2[256,10], b2[1,10];
         MATMUL -> BROADCAST -> ADD -> RELU -> MATMUL -> BROADCAST -> ADD
         -> SOFTMAX  (13 nodes, 7 waves)
  conv   INPUT_4D in[N,C_in,H,W], w[C_out,C_in,3,3]; CONV2D(stride 1, pad 1)
         -> RELU, then lancius_optimize_fusion -> CONV2D_RELU_FUSED + NOP
         (4 nodes, 2 waves)
  block  pre-norm transformer encoder block, one branch per sequence sharing
         the 16 weight INPUTs:
           x[S,d] -> LAYERNORM -> 3 x (MATMUL + BROADCAST + ADD) -> RESHAPE
           [S,H,D] -> ATTENTION (causal) -> RESHAPE [S,d] -> MATMUL + BROADCAST
           + ADD -> ADD x -> LAYERNORM -> MATMUL + BROADCAST + ADD -> GELU
           -> MATMUL + BROADCAST + ADD -> ADD residual
         (16 + 29 per sequence = 132 nodes, 17 waves at batch 4)
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

from . import abi


@dataclass
class BuiltGraph:
    lib: C.CDLL
    g: abi.GraphP
    nodes: dict = field(default_factory=dict)   # name -> NodeP
    inputs: list = field(default_factory=list)  # INPUT node names in creation order
    outputs: list = field(default_factory=list) # sink node names

    def node(self, name: str) -> abi.NodeP:
        return self.nodes[name]

    def destroy(self) -> None:
        if self.g:
            self.lib.lancius_graph_destroy(self.g)
            self.g = None


def _inp(bg: BuiltGraph, name: str, *shape: int) -> abi.NodeP:
    lib, g = bg.lib, bg.g
    n = lib.lancius_input(g, *shape) if len(shape) == 2 else lib.lancius_input_4d(g, *shape)
    if not n:
        raise RuntimeError(f"lancius_input failed for {name}")
    bg.nodes[name] = n
    bg.inputs.append(name)
    return n


def _ok(n, what: str):
    if not n:
        raise RuntimeError(f"graph builder failed: {what}")
    return n


def build_mlp(lib: C.CDLL, batch: int = 64, d_in: int = 784, hidden: int = 256, classes: int = 10) -> BuiltGraph:
    bg = BuiltGraph(lib, _ok(lib.lancius_graph_create(), "graph_create"))
    x = _inp(bg, "x", batch, d_in)
    w1 = _inp(bg, "W1", d_in, hidden)
    b1 = _inp(bg, "b1", 1, hidden)
    w2 = _inp(bg, "W2", hidden, classes)
    b2 = _inp(bg, "b2", 1, classes)
    mm1 = _ok(lib.lancius_matmul(bg.g, x, w1), "mm1")
    bc1 = _ok(lib.lancius_broadcast(bg.g, b1, batch, hidden), "bc1")
    a1 = _ok(lib.lancius_add(bg.g, mm1, bc1), "add1")
    r1 = _ok(lib.lancius_relu(bg.g, a1), "relu")
    mm2 = _ok(lib.lancius_matmul(bg.g, r1, w2), "mm2")
    bc2 = _ok(lib.lancius_broadcast(bg.g, b2, batch, classes), "bc2")
    a2 = _ok(lib.lancius_add(bg.g, mm2, bc2), "add2")
    sm = _ok(lib.lancius_softmax(bg.g, a2), "softmax")
    bg.nodes.update(mm1=mm1, bc1=bc1, add1=a1, relu=r1, mm2=mm2, bc2=bc2, add2=a2, softmax=sm)
    bg.outputs = ["softmax"]
    return bg


def build_conv(lib: C.CDLL, N: int = 32, C_in: int = 64, H: int = 56, W: int = 56, C_out: int = 128,
               fuse: bool = True) -> BuiltGraph:
    bg = BuiltGraph(lib, _ok(lib.lancius_graph_create(), "graph_create"))
    x = _inp(bg, "x", N, C_in, H, W)
    w = _inp(bg, "w", C_out, C_in, 3, 3)
    conv = _ok(lib.lancius_conv2d(bg.g, x, w, 1, 1), "conv2d")
    relu = _ok(lib.lancius_relu(bg.g, conv), "relu")
    bg.nodes.update(conv=conv, relu=relu)
    if fuse:
        lib.lancius_optimize_fusion(bg.g)
    bg.outputs = ["relu"]
    return bg


BLOCK_WEIGHTS = ("g1", "be1", "Wq", "bq", "Wk", "bk", "Wv", "bv", "Wo", "bo", "g2", "be2", "W1", "bf1", "W2", "bf2")


def build_block(lib: C.CDLL, batch: int = 4, S: int = 1024, d: int = 1024, H: int = 16, F: int = 4096,
                noncausal: bool = False) -> BuiltGraph:
    D = d // H
    bg = BuiltGraph(lib, _ok(lib.lancius_graph_create(), "graph_create"))
    shapes = {"g1": (1, d), "be1": (1, d), "Wq": (d, d), "bq": (1, d), "Wk": (d, d), "bk": (1, d), "Wv": (d, d),
              "bv": (1, d), "Wo": (d, d), "bo": (1, d), "g2": (1, d), "be2": (1, d), "W1": (d, F), "bf1": (1, F),
              "W2": (F, d), "bf2": (1, d)}
    w = {k: _inp(bg, k, *shapes[k]) for k in BLOCK_WEIGHTS}
    g = bg.g

    def linear(x, W, b, rows, cols, tag):
        mm = _ok(lib.lancius_matmul(g, x, W), f"{tag} matmul")
        bc = _ok(lib.lancius_broadcast(g, b, rows, cols), f"{tag} broadcast")
        return _ok(lib.lancius_add(g, mm, bc), f"{tag} add")

    for s in range(batch):
        x = _inp(bg, f"x{s}", S, d)
        ln1 = _ok(lib.lancius_layernorm(g, x, w["g1"], w["be1"]), "ln1")
        q = linear(ln1, w["Wq"], w["bq"], S, d, "q")
        k = linear(ln1, w["Wk"], w["bk"], S, d, "k")
        v = linear(ln1, w["Wv"], w["bv"], S, d, "v")
        q3 = _ok(lib.lancius_reshape(g, q, 3, S, H, D, 0), "reshape q")
        k3 = _ok(lib.lancius_reshape(g, k, 3, S, H, D, 0), "reshape k")
        v3 = _ok(lib.lancius_reshape(g, v, 3, S, H, D, 0), "reshape v")
        att = _ok(lib.lancius_attention(g, q3, k3, v3), "attention")
        if noncausal:
            att.contents.axes[0] = 1
        att2 = _ok(lib.lancius_reshape(g, att, 2, S, d, 0, 0), "reshape att")
        o = linear(att2, w["Wo"], w["bo"], S, d, "o")
        x1 = _ok(lib.lancius_add(g, o, x), "residual 1")
        ln2 = _ok(lib.lancius_layernorm(g, x1, w["g2"], w["be2"]), "ln2")
        f1 = _ok(lib.lancius_gelu(g, linear(ln2, w["W1"], w["bf1"], S, F, "ffn1")), "gelu")
        f2 = linear(f1, w["W2"], w["bf2"], S, d, "ffn2")
        y = _ok(lib.lancius_add(g, f2, x1), "residual 2")
        bg.nodes.update({f"ln1_{s}": ln1, f"att{s}": att, f"x1_{s}": x1, f"y{s}": y})
        bg.outputs.append(f"y{s}")
    return bg


def build_relu_chain(lib: C.CDLL, depth: int = 20, rows: int = 1024, cols: int = 1024) -> BuiltGraph:
    """S9/examples/audit_memory_pool.c:13-69: INPUT -> 20 x RELU."""
    bg = BuiltGraph(lib, _ok(lib.lancius_graph_create(), "graph_create"))
    cur = _inp(bg, "x", rows, cols)
    for i in range(depth):
        cur = _ok(lib.lancius_relu(bg.g, cur), "relu")
        bg.nodes[f"relu{i}"] = cur
    bg.outputs = [f"relu{depth - 1}"]
    return bg
