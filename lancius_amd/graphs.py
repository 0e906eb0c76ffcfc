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
    keep: list = field(default_factory=list)    # host arrays bound as runtime_data

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


# ---- training graphs (forward + lancius_ir_autodiff) --------------------------


def build_mlp_ce(lib: C.CDLL, batch: int = 64, d_in: int = 784, hidden: int = 128, classes: int = 10) -> BuiltGraph:
    """Forward graph of B/examples/train_mnist.c:87-96 (creation order kept):
    INPUT X, W1, b1, W2, b2, Y; MATMUL -> ADD(BROADCAST b1) -> RELU -> MATMUL
    -> ADD(BROADCAST b2) -> CROSS_ENTROPY against Y."""
    bg = BuiltGraph(lib, _ok(lib.lancius_graph_create(), "graph_create"))
    g = bg.g
    x = _inp(bg, "X", batch, d_in)
    w1 = _inp(bg, "W1", d_in, hidden)
    b1 = _inp(bg, "b1", 1, hidden)
    w2 = _inp(bg, "W2", hidden, classes)
    b2 = _inp(bg, "b2", 1, classes)
    y = _inp(bg, "Y", batch, classes)
    z1 = _ok(lib.lancius_matmul(g, x, w1), "Z1")
    a1 = _ok(lib.lancius_add(g, z1, _ok(lib.lancius_broadcast(g, b1, batch, hidden), "bc1")), "A1")
    h1 = _ok(lib.lancius_relu(g, a1), "H1")
    z2 = _ok(lib.lancius_matmul(g, h1, w2), "Z2")
    a2 = _ok(lib.lancius_add(g, z2, _ok(lib.lancius_broadcast(g, b2, batch, classes), "bc2")), "A2")
    loss = _ok(lib.lancius_cross_entropy(g, a2, y), "loss")
    bg.nodes.update(Z1=z1, A1=a1, H1=h1, Z2=z2, A2=a2, loss=loss)
    bg.outputs = ["loss"]
    return bg


def build_cnn_ce(lib: C.CDLL, batch: int = 8, fuse: bool = False) -> BuiltGraph:
    """Forward graph of B/examples/train_cifar10.c:89-119 (creation order kept):
    conv 5x5 pad 2 (3->16) -> RELU -> MAXPOOL 2/2 -> conv 5x5 pad 2 (16->32) ->
    RELU -> MAXPOOL 2/2 -> FLATTEN -> FC 2048->120 + bias -> RELU -> FC 120->10
    + bias -> CROSS_ENTROPY.  fuse=True runs lancius_optimize_fusion first
    (Conv+ReLU pairs become CONV2D_RELU_FUSED + NOP)."""
    bg = BuiltGraph(lib, _ok(lib.lancius_graph_create(), "graph_create"))
    g = bg.g
    x = _inp(bg, "X", batch, 3, 32, 32)
    w1 = _inp(bg, "W1", 16, 3, 5, 5)
    c1 = _ok(lib.lancius_conv2d(g, x, w1, 1, 2), "C1")
    r1 = _ok(lib.lancius_relu(g, c1), "R1")
    p1 = _ok(lib.lancius_maxpool2d(g, r1, 2, 2), "P1")
    w2 = _inp(bg, "W2", 32, 16, 5, 5)
    c2 = _ok(lib.lancius_conv2d(g, p1, w2, 1, 2), "C2")
    r2 = _ok(lib.lancius_relu(g, c2), "R2")
    p2 = _ok(lib.lancius_maxpool2d(g, r2, 2, 2), "P2")
    f = _ok(lib.lancius_flatten(g, p2), "F")
    w3 = _inp(bg, "W3", 2048, 120)
    b1 = _inp(bg, "b1", 1, 120)
    z1 = _ok(lib.lancius_matmul(g, f, w3), "Z1")
    a1 = _ok(lib.lancius_add(g, z1, _ok(lib.lancius_broadcast(g, b1, batch, 120), "bc1")), "A1")
    h1 = _ok(lib.lancius_relu(g, a1), "H1")
    w4 = _inp(bg, "W4", 120, 10)
    b2 = _inp(bg, "b2", 1, 10)
    z2 = _ok(lib.lancius_matmul(g, h1, w4), "Z2")
    a2 = _ok(lib.lancius_add(g, z2, _ok(lib.lancius_broadcast(g, b2, batch, 10), "bc2")), "A2")
    y = _inp(bg, "Y", batch, 10)
    loss = _ok(lib.lancius_cross_entropy(g, a2, y), "loss")
    bg.nodes.update(C1=c1, R1=r1, P1=p1, C2=c2, R2=r2, P2=p2, F=f, Z1=z1, A1=a1, H1=h1, Z2=z2, A2=a2, loss=loss)
    if fuse:
        lib.lancius_optimize_fusion(g)
    bg.outputs = ["loss"]
    return bg


def build_gradcheck(lib: C.CDLL) -> BuiltGraph:
    """Forward graph of S9/examples/test_grad_check.c:28-37: conv 3x3 (3->4,
    stride 1, pad 0) on [2,3,8,8] -> RELU -> FLATTEN -> MATMUL [144,5] ->
    CROSS_ENTROPY."""
    bg = BuiltGraph(lib, _ok(lib.lancius_graph_create(), "graph_create"))
    g = bg.g
    x = _inp(bg, "X", 2, 3, 8, 8)
    w1 = _inp(bg, "W1", 4, 3, 3, 3)
    c1 = _ok(lib.lancius_conv2d(g, x, w1, 1, 0), "C1")
    r1 = _ok(lib.lancius_relu(g, c1), "R1")
    f1 = _ok(lib.lancius_flatten(g, r1), "F1")
    w2 = _inp(bg, "W2", 144, 5)
    z1 = _ok(lib.lancius_matmul(g, f1, w2), "Z1")
    y = _inp(bg, "Y", 2, 5)
    loss = _ok(lib.lancius_cross_entropy(g, z1, y), "loss")
    bg.nodes.update(C1=c1, R1=r1, F1=f1, Z1=z1, loss=loss)
    bg.outputs = ["loss"]
    return bg


def build_ops_loss(lib: C.CDLL, R: int = 8, Cc: int = 5) -> BuiltGraph:
    """A scalar loss whose gradient graph holds the remaining dispatch ops
    (R >= Cc: the BROADCAST of the [R,1] vector v reads v[c] for c < Cc,
    lancius_scheduler.c:275-276):
      A = X - Y;  B = A * X;  S = SOFTMAX(B);  S2 = S + BROADCAST(v);
      M = TRANSPOSE(S2) . Z;  loss = SUM(M * Wm)
    (the product with Wm keeps the softmax gradient from being constant along
    rows, which SOFTMAX_BWD would map to exactly zero; v joins after the
    softmax because row sums of a softmax gradient are zero).
    Backward: BROADCAST of the seed, MUL, MATMUL/TRANSPOSE, SOFTMAX_BWD,
    SUM_AXIS1 (v's gradient), SUB's -1 CONST and ADD accumulation into X."""
    bg = BuiltGraph(lib, _ok(lib.lancius_graph_create(), "graph_create"))
    g = bg.g
    x = _inp(bg, "X", R, Cc)
    y = _inp(bg, "Y", R, Cc)
    v = _inp(bg, "v", R, 1)
    z = _inp(bg, "Z", R, Cc)
    wm = _inp(bg, "Wm", Cc, Cc)
    a = _ok(lib.lancius_sub(g, x, y), "A")
    b = _ok(lib.lancius_mul(g, a, x), "B")
    s = _ok(lib.lancius_softmax(g, b), "S")
    s2 = _ok(lib.lancius_add(g, s, _ok(lib.lancius_broadcast(g, v, R, Cc), "bcv")), "S2")
    t = _ok(lib.lancius_transpose(g, s2), "T")
    m = _ok(lib.lancius_matmul(g, t, z), "M")
    m2 = _ok(lib.lancius_mul(g, m, wm), "M2")
    loss = _ok(lib.lancius_sum(g, m2), "loss")
    bg.nodes.update(A=a, B=b, S=s, S2=s2, T=t, M=m, M2=m2, loss=loss)
    bg.outputs = ["loss"]
    return bg


@dataclass
class TrainGraph(BuiltGraph):
    """The training graph of lancius_ir_autodiff over a forward BuiltGraph.
    `nodes`/`inputs` name the training graph's INPUT copies after the forward
    inputs; `grads[name]` is the gradient node of forward input `name` (absent
    when the loss does not depend on it); outputs = loss + every gradient."""
    tg: abi.TrainingGraphP = None
    fwd: BuiltGraph = None
    grads: dict = field(default_factory=dict)

    def destroy(self) -> None:
        if self.tg:
            self.lib.lancius_training_graph_destroy(self.tg)
            self.tg = None
            self.g = None
        if self.fwd:
            self.fwd.destroy()
            self.fwd = None


def build_training(lib: C.CDLL, fwd: BuiltGraph, loss: str = "loss") -> TrainGraph:
    tg = lib.lancius_ir_autodiff(fwd.g, fwd.node(loss))
    if not tg:
        raise RuntimeError("lancius_ir_autodiff failed")
    t = TrainGraph(lib, tg.contents.graph, tg=tg, fwd=fwd)
    g = tg.contents.graph.contents
    ins = [g.nodes[i] for i in range(g.node_count) if g.nodes[i].contents.op == abi.OP["INPUT"]]
    if len(ins) != len(fwd.inputs):
        raise RuntimeError("training graph inputs do not match the forward graph")
    for name, n in zip(fwd.inputs, ins):
        t.nodes[name] = n
        t.inputs.append(name)
    t.nodes["loss"] = tg.contents.loss_node
    t.outputs = ["loss"]
    for name in fwd.inputs:
        gn = tg.contents.grad_nodes[fwd.node(name).contents.id]
        if gn:
            t.grads[name] = gn
            t.nodes[f"d{name}"] = gn
            t.outputs.append(f"d{name}")
    return t


IO_GRAPHS = ("io_mlp", "io_conv_i8")


def _bind(bg: BuiltGraph, name: str, arr) -> None:
    """Bind fp64 host data to an INPUT node (kept alive by the BuiltGraph)."""
    import numpy as np

    a = np.ascontiguousarray(arr, dtype=np.float64)
    bg.keep.append(a)
    bg.node(name).contents.runtime_data = a.ctypes.data_as(C.POINTER(C.c_double))


def build_io_graph(lib: C.CDLL, name: str) -> BuiltGraph:
    """Graphs with stored weights for the model-file tests: the same builder
    calls give the same node ids and bytes with either library.

    io_mlp: MATMUL, BROADCAST + ADD, RELU marked as a view of the MATMUL
    (is_view, strides, view_source), CONST, GELU, LAYERNORM, SOFTMAX, and a
    RESHAPE feeding a non-causal ATTENTION (axes[0] = 1).
    io_conv_i8: conv + ReLU fused (the fusion pass leaves a NOP), MAXPOOL2D,
    FLATTEN, MATMUL, after lancius_quantize_graph (int8 image and filter)."""
    from . import prng

    bg = BuiltGraph(lib, _ok(lib.lancius_graph_create(), "graph_create"))
    g = bg.g
    if name == "io_mlp":
        x = _inp(bg, "x", 4, 8)
        w1 = _inp(bg, "W1", 8, 16)
        b1 = _inp(bg, "b1", 1, 16)
        mm = _ok(lib.lancius_matmul(g, x, w1), "mm")
        a = _ok(lib.lancius_add(g, mm, _ok(lib.lancius_broadcast(g, b1, 4, 16), "bc")), "add")
        r = _ok(lib.lancius_relu(g, a), "relu")
        r.contents.is_view = 1
        r.contents.strides[0], r.contents.strides[1] = 16, 1
        r.contents.view_source = mm
        s = _ok(lib.lancius_add(g, r, _ok(lib.lancius_const(g, 0.5, 4, 16), "const")), "add2")
        gl = _ok(lib.lancius_gelu(g, s), "gelu")
        gam = _inp(bg, "gamma", 1, 16)
        bet = _inp(bg, "beta", 1, 16)
        ln = _ok(lib.lancius_layernorm(g, gl, gam, bet), "ln")
        w2 = _inp(bg, "W2", 16, 10)
        bg.nodes["probs"] = _ok(lib.lancius_softmax(g, _ok(lib.lancius_matmul(g, ln, w2), "mm2")), "softmax")
        q = _inp(bg, "q", 4, 16)
        q3 = _ok(lib.lancius_reshape(g, q, 3, 4, 2, 8, 1), "reshape")
        att = _ok(lib.lancius_attention(g, q3, q3, q3), "attention")
        att.contents.axes[0] = 1
        bg.nodes["att"] = att
        bg.outputs = ["probs", "att"]
        _bind(bg, "W1", prng.normal(90, (8, 16)))
        _bind(bg, "b1", prng.normal(91, (1, 16)))
        _bind(bg, "gamma", prng.normal(92, (1, 16), mean=1.0, std=0.1))
        _bind(bg, "beta", prng.normal(93, (1, 16), std=0.1))
        _bind(bg, "W2", prng.normal(94, (16, 10)))
    elif name == "io_conv_i8":
        img = _inp(bg, "img", 2, 3, 8, 8)
        w = _inp(bg, "w", 4, 3, 3, 3)
        cv = _ok(lib.lancius_conv2d(g, img, w, 1, 1), "conv")
        r = _ok(lib.lancius_relu(g, cv), "relu")
        mp = _ok(lib.lancius_maxpool2d(g, r, 2, 2), "pool")
        fl = _ok(lib.lancius_flatten(g, mp), "flatten")
        wf = _inp(bg, "Wf", 64, 5)
        bg.nodes["logits"] = _ok(lib.lancius_matmul(g, fl, wf), "mm")
        bg.outputs = ["logits"]
        lib.lancius_optimize_fusion(g)
        _bind(bg, "img", prng.normal(95, (2, 3, 8, 8)))
        _bind(bg, "w", prng.normal(96, (4, 3, 3, 3), std=0.4))
        _bind(bg, "Wf", prng.normal(97, (64, 5)))
        lib.lancius_quantize_graph(g)
    else:
        raise ValueError(name)
    return bg
