"""The oracle's restatement of the training and reduction ops (SUB, MUL,
RELU_BWD, TRANSPOSE, SUM*, SOFTMAX_BWD, CROSS_ENTROPY(_BWD), MAXPOOL2D(_BWD),
conv backward) and of the autodiff training graphs, pinned by the reference's
own outputs (tests/golden, written by the compiled reference) and by what the
mathematics fixes: numpy closed forms, the softmax Jacobian, adjoint
identities of the convolution, and finite differences
(S9/examples/test_grad_check.c:60-120)."""
import ctypes as C
from pathlib import Path

import numpy as np
import pytest

import oracle
from lancius_amd import abi, graph_lib, graphs, prng
from tests.golden.make_golden import TRAIN_GRAPHS, TRAIN_SEEDS, train_feeds

GOLD = Path(__file__).resolve().parent / "golden"
K = np.load(GOLD / "kernels.npz")
T = np.load(GOLD / "train_outputs.npz")


def close(got, ref, tol=1e-12):
    assert oracle.normwise_error(got, ref) <= tol


# ---- reference golden vectors ------------------------------------------------------


def test_elementwise_golden():
    a, b = K["ew_a"], K["ew_b"]
    close(oracle.sub(a, b), K["sub_out"], 0)
    close(oracle.mul(a, b), K["mul_out"], 0)
    np.testing.assert_array_equal(oracle.relu_bwd(b, a), K["relu_bwd_out"])


def test_reductions_golden():
    a = K["ew_a"]
    np.testing.assert_array_equal(oracle.transpose(a), K["transpose_out"])
    close(oracle.sum_all(a), K["sum_out"].ravel()[0])
    close(oracle.sum_axis0(a), K["sum_axis0_out"])
    close(oracle.sum_axis1(a), K["sum_axis1_out"])


def test_softmax_bwd_golden():
    close(oracle.softmax_bwd(K["ew_b"], K["softmax_bwd_y"]), K["softmax_bwd_out"])


def test_cross_entropy_golden():
    close(oracle.cross_entropy(K["ce_x"], K["ce_y"]), K["ce_out"].ravel()[0])
    close(oracle.cross_entropy_bwd(K["ce_x"], K["ce_y"], float(K["ce_g"].ravel()[0])), K["ce_bwd_out"])


@pytest.mark.parametrize("tag,stride,pad", [("s1p1", 1, 1), ("s2p2", 2, 2)])
def test_conv_backward_golden(tag, stride, pad):
    x, w, g = K[f"cbwd_{tag}_x"], K[f"cbwd_{tag}_w"], K[f"cbwd_{tag}_g"]
    close(oracle.conv2d_bwd_input(g, w, x.shape, stride, pad), K[f"cbwd_{tag}_dx"])
    close(oracle.conv2d_bwd_weight(g, x, w.shape, stride, pad), K[f"cbwd_{tag}_dw"])


@pytest.mark.parametrize("tag,k,s", [("k3s2", 3, 2), ("k2s2", 2, 2)])
def test_maxpool_golden(tag, k, s):
    x = K["pool_x"]
    np.testing.assert_array_equal(oracle.maxpool2d(x, k, s), K[f"pool_{tag}_out"])
    close(oracle.maxpool2d_bwd(K[f"pool_{tag}_g"], x, k, s), K[f"pool_{tag}_dx"])


# ---- closed forms ----------------------------------------------------------------------


def test_transpose_and_sums_closed_forms():
    a = prng.normal(30, (37, 23)).astype(np.float64)
    np.testing.assert_array_equal(oracle.transpose(a), a.T)
    np.testing.assert_array_equal(oracle.transpose(oracle.transpose(a)), a)
    assert abs(oracle.sum_all(a) - a.sum()) <= 1e-12 * np.abs(a).sum()
    np.testing.assert_allclose(oracle.sum_axis0(a), a.sum(0, keepdims=True), rtol=0, atol=1e-12)
    np.testing.assert_allclose(oracle.sum_axis1(a), a.sum(1, keepdims=True), rtol=0, atol=1e-12)
    assert oracle.sum_all(np.zeros((0,))) == 0.0


def test_softmax_bwd_is_jacobian_product():
    x = prng.normal(31, (5, 7)).astype(np.float64)
    dy = prng.normal(32, (5, 7)).astype(np.float64)
    y = oracle.softmax(x)
    got = oracle.softmax_bwd(dy, y)
    for r in range(5):
        J = np.diag(y[r]) - np.outer(y[r], y[r])  # d softmax / d x
        np.testing.assert_allclose(got[r], J @ dy[r], rtol=1e-12, atol=1e-14)


def test_cross_entropy_closed_form_and_finite_difference():
    x = prng.normal(33, (4, 6), std=2.0).astype(np.float64)
    lab = np.array([1, 5, 0, 3])
    y = np.zeros((4, 6))
    y[np.arange(4), lab] = 1.0
    lse = np.log(np.exp(x - x.max(1, keepdims=True)).sum(1)) + x.max(1)
    want = np.mean(lse - x[np.arange(4), lab])
    assert abs(oracle.cross_entropy(x, y) - want) <= 1e-12
    # d loss / d x = (softmax(x) - y) / rows, the CE_BWD formula with g = 1
    g = oracle.cross_entropy_bwd(x, y, 1.0)
    h = 1e-6
    for r, c in [(0, 0), (1, 5), (2, 3), (3, 3)]:
        xp, xm = x.copy(), x.copy()
        xp[r, c] += h
        xm[r, c] -= h
        fd = (oracle.cross_entropy(xp, y) - oracle.cross_entropy(xm, y)) / (2 * h)
        assert abs(fd - g[r, c]) <= 1e-7
    # the scale g multiplies linearly
    np.testing.assert_allclose(oracle.cross_entropy_bwd(x, y, 0.25), 0.25 * g, rtol=1e-14)


def test_cross_entropy_target_selection():
    # only entries exactly equal to 1.0 select a class (lancius_scheduler.c:80):
    # a row of 0.9999 contributes nothing, a row with two 1.0 entries both
    x = np.array([[2.0, -1.0, 0.5], [0.3, 0.2, 0.1]])
    y = np.array([[0.9999, 0.0, 0.0], [1.0, 0.0, 1.0]])
    lse = np.log(np.exp(x[1] - x[1].max()).sum()) + x[1].max()
    want = ((lse - x[1, 0]) + (lse - x[1, 2])) / 2
    assert oracle.cross_entropy(x, y) == pytest.approx(want, rel=1e-14)
    assert oracle.cross_entropy(x, np.zeros_like(x)) == 0.0


@pytest.mark.parametrize("stride,pad,k", [(1, 0, 3), (1, 1, 3), (1, 2, 5), (2, 1, 3), (2, 0, 2), (3, 2, 5)])
def test_conv_backward_adjoint_identities(stride, pad, k):
    """<conv(x,w), g> = <x, bwd_in(g,w)> = <w, bwd_w(g,x)>."""
    x = prng.normal(40 + k, (2, 3, 9, 8)).astype(np.float64)
    w = prng.normal(41 + k, (4, 3, k, k)).astype(np.float64)
    y = oracle.conv2d(x, w, stride, pad)
    g = prng.normal(42 + k, y.shape).astype(np.float64)
    lhs = np.sum(y * g)
    assert np.sum(x * oracle.conv2d_bwd_input(g, w, x.shape, stride, pad)) == pytest.approx(lhs, rel=1e-12)
    assert np.sum(w * oracle.conv2d_bwd_weight(g, x, w.shape, stride, pad)) == pytest.approx(lhs, rel=1e-12)


def test_maxpool_closed_forms():
    x = prng.normal(50, (2, 2, 6, 8)).astype(np.float64)
    ref = x.reshape(2, 2, 3, 2, 4, 2).max(axis=(3, 5))
    np.testing.assert_array_equal(oracle.maxpool2d(x, 2, 2), ref)
    g = prng.normal(51, (2, 2, 3, 4)).astype(np.float64)
    dx = oracle.maxpool2d_bwd(g, x, 2, 2)
    assert np.sum(dx) == pytest.approx(np.sum(g), rel=1e-12)
    assert np.count_nonzero(dx) == g.size  # one winner per window, no ties in random data
    # a window with nothing above -1e9 sends its gradient to (0,0) of the plane
    x2 = np.full((1, 1, 4, 4), -5e9)
    x2[0, 0, 0, 0] = -4e9
    dx2 = oracle.maxpool2d_bwd(np.ones((1, 1, 2, 2)), x2, 2, 2)
    assert dx2[0, 0, 0, 0] == 4.0 and np.count_nonzero(dx2) == 1
    np.testing.assert_array_equal(oracle.maxpool2d(x2, 2, 2), np.full((1, 1, 2, 2), -1e9))


# ---- training graphs -----------------------------------------------------------------


def _run_oracle(t, feeds):
    keep = []
    for name in t.inputs:
        arr = np.ascontiguousarray(feeds[name], dtype=np.float64)
        keep.append(arr)
        t.node(name).contents.runtime_data = arr.ctypes.data_as(C.POINTER(C.c_double))
    sched = graph_lib().lancius_ir_schedule(t.g)
    oracle.schedule_execute(sched)
    out = {}
    for name in t.outputs:
        n = t.node(name)
        out[name] = np.ctypeslib.as_array(n.contents.runtime_data, shape=(abi.node_elems(n),)).copy().reshape(
            abi.node_shape(n))
    oracle.release(t.g)
    for name in t.inputs:
        t.node(name).contents.runtime_data = None
    graph_lib().lancius_schedule_destroy(sched)
    return out


@pytest.mark.parametrize("name", sorted(TRAIN_GRAPHS))
def test_training_graph_matches_reference_run(name):
    """liblancius_graph's autodiff graph, executed by the oracle, gives the
    reference's loss and gradients (reference graph, reference executor)."""
    lib = graph_lib()
    t = graphs.build_training(lib, TRAIN_GRAPHS[name](lib))
    stored = "cnn" if name == "cnn_fused" else name
    got = _run_oracle(t, train_feeds(t, TRAIN_SEEDS[name]))
    for out in t.outputs:
        close(got[out], T[f"{stored}_out_{out}"], 1e-10)
    t.destroy()


def test_gradcheck_finite_differences():
    """S9/examples/test_grad_check.c:60-120: autodiff gradients of W1 (conv)
    and W2 (matmul) against central differences of the forward loss,
    h = 1e-5, relative error < 1e-4."""
    lib = graph_lib()
    t = graphs.build_training(lib, graphs.build_gradcheck(lib))
    feeds = train_feeds(t, 9100)
    grads = _run_oracle(t, feeds)
    fwd = graphs.build_gradcheck(lib)
    sched = lib.lancius_ir_schedule(fwd.g)

    def loss(fd):
        keep = []
        for name in fwd.inputs:
            arr = np.ascontiguousarray(fd[name], dtype=np.float64)
            keep.append(arr)
            fwd.node(name).contents.runtime_data = arr.ctypes.data_as(C.POINTER(C.c_double))
        oracle.schedule_execute(sched)
        v = fwd.node("loss").contents.runtime_data[0]
        oracle.release(fwd.g)
        return v

    h = 1e-5
    for wname in ("W1", "W2"):
        w = feeds[wname].astype(np.float64)
        fd = np.zeros(w.size)
        for i in range(w.size):
            wp, wm = w.copy().ravel(), w.copy().ravel()
            wp[i] += h
            wm[i] -= h
            fd[i] = (loss({**feeds, wname: wp.reshape(w.shape)}) - loss({**feeds, wname: wm.reshape(w.shape)})) / (2 * h)
        ag = grads[f"d{wname}"].ravel()
        err = np.abs(ag - fd) / (np.abs(ag) + np.abs(fd) + 1e-8)
        assert err.max() < 1e-4, (wname, err.max())
    lib.lancius_schedule_destroy(sched)
    fwd.destroy()
    t.destroy()
