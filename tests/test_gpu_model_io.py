"""Model files straight into the device arena: lancius_graph_load_mapped +
lancius_device_upload_weights (lancius_hip_upload_file), and the drop-in
lancius_graph_load + lancius_schedule_execute_device, on the reference's own
models:

  * stable/v9S/pytorch_lenet.lancius on parity_input.bin against the ONNX
    Runtime logits the reference ships (baseline_out.bin) and the reference
    executor's logits (model_io.npz; the shipped lancius_out.bin is them in
    fp32): fp32 device arithmetic against fp64, normwise error within
    1e-4 * max(1, sqrt(K)/32) for the longest reduction K = 2048, argmax
    bit-exact;
  * stable/v9S/cifar10_lenet.lancius (int8 image and filters, BROADCAST,
    CROSS_ENTROPY on its stored batch) against the reference executor's
    logits;
  * a v2 file with fp32 weights gives bit-identical outputs.
"""
import ctypes as C
from pathlib import Path

import numpy as np
import pytest

import oracle
from lancius_amd import DEVICE_KEEP_ALL, DeviceProgram, HipError, abi, graph_lib, prng
from lancius_amd.runtime import FileTensor
from tests.conftest import case, record_parity, top2_margin

pytestmark = pytest.mark.gpu

GOLD = Path(__file__).resolve().parent / "golden"
MODELS = GOLD / "models"
K = np.load(GOLD / "model_io.npz")
X = np.fromfile(MODELS / "parity_input.bin", dtype="<f4")
ONNX = np.fromfile(MODELS / "baseline_out.bin", dtype="<f4")
TOL = oracle.tolerance(2048)


def nodes_of(g):
    return [g.contents.nodes[i] for i in range(g.contents.node_count)]


def lenet_io(g, wm=None):
    """Input and logits nodes as examples/parity_runner.c:14-18 finds them
    (the 4-D INPUT without stored data: not in the weight map when mapped)."""
    ns = nodes_of(g)
    stored = {wm.refs[k].node.contents.id for k in range(wm.count)} if wm is not None else set()
    x = [n for n in ns if n.contents.op == abi.OP["INPUT"] and n.contents.ndim == 4 and not n.contents.runtime_data
         and n.contents.id not in stored]
    y = [n for n in ns if n.contents.ndim == 2 and n.contents.shape[1] == 10 and n.contents.op != abi.OP["INPUT"]]
    return x[0], y[-1]


def run_mapped(dev, path, flags=0, feed=None):
    """load_mapped -> fp32 -> schedule/plan -> program -> weights from the
    file -> feed -> run.  Returns (program, graph, map, sched, plan)."""
    lib = graph_lib()
    wm = abi.WeightMap()
    g = lib.lancius_graph_load_mapped(str(path).encode(), C.byref(wm))
    assert g, lib.lancius_get_error()
    lib.lancius_graph_set_dtype(g, abi.DTYPE_FP32)
    sched = lib.lancius_ir_schedule(g)
    plan = lib.lancius_build_memory_plan(sched, g)
    prog = DeviceProgram(dev, g, sched, plan, flags)
    case(f"upload_weights {Path(path).name} ({wm.count} tensors, layout v{wm.format})")
    prog.upload_weights(path, wm)
    if feed:
        feed(prog, g, wm)
    prog.run()
    return prog, g, wm, sched, plan


def release(prog, g, wm, sched, plan):
    lib = graph_lib()
    prog.close()
    lib.lancius_memory_plan_destroy(plan)
    lib.lancius_schedule_destroy(sched)
    lib.lancius_weight_map_free(C.byref(wm))
    lib.lancius_graph_destroy(g)


def feed_lenet(prog, g, wm):
    x, _ = lenet_io(g, wm)
    prog.upload(x, X)


def test_lenet_from_file_matches_onnx_and_reference(dev):
    res = run_mapped(dev, MODELS / "pytorch_lenet.lancius", feed=feed_lenet)
    prog, g = res[0], res[1]
    got = prog.download(lenet_io(g, res[2])[1]).ravel()
    record_parity("LeNet (pytorch_lenet.lancius) logits vs ONNX Runtime", oracle.normwise_error(got, ONNX), TOL,
                  argmax_exact=True, top2_margin_ref=top2_margin(ONNX), top2_margin_dev=top2_margin(got))
    record_parity("LeNet (pytorch_lenet.lancius) logits vs the reference executor",
                  oracle.normwise_error(got, K["lenet_logits"]), TOL, top2_margin_ref=top2_margin(K["lenet_logits"]))
    assert oracle.normwise_error(got, ONNX) <= TOL
    assert oracle.normwise_error(got, K["lenet_logits"]) <= TOL
    assert int(np.argmax(got)) == int(np.argmax(ONNX)) == 7
    release(*res)


def test_lenet_drop_in_executor(dev):
    """lancius_graph_load (host fp64 weights) + lancius_schedule_execute_device,
    as examples/parity_runner.c drives the reference."""
    lib = graph_lib()
    g = lib.lancius_graph_load(str(MODELS / "pytorch_lenet.lancius").encode())
    x, y = lenet_io(g)
    xin = X.astype(np.float64)
    x.contents.runtime_data = xin.ctypes.data_as(C.POINTER(C.c_double))
    sched = lib.lancius_ir_schedule(g)
    case("lenet drop-in")
    rc = dev.lib.lancius_schedule_execute_device(sched, g, dev.ctx)
    assert rc == 0, dev.lib.lancius_hip_last_error()
    got = np.ctypeslib.as_array(y.contents.runtime_data, shape=(10,)).copy()
    assert oracle.normwise_error(got, K["lenet_logits"]) <= TOL
    assert int(np.argmax(got)) == 7
    x.contents.runtime_data = None
    lib.lancius_schedule_destroy(sched)
    lib.lancius_graph_destroy(g)  # frees the loaded weights (the sink's buffer is the caller's)


def test_cifar_int8_model_from_file(dev):
    res = run_mapped(dev, MODELS / "cifar10_lenet.lancius", flags=DEVICE_KEEP_ALL)
    prog, g = res[0], res[1]
    ns = nodes_of(g)
    logits = [n for n in ns if n.contents.op == abi.OP["ADD"] and abi.node_shape(n) == (32, 10)][-1]
    loss = [n for n in ns if n.contents.op == abi.OP["CROSS_ENTROPY"]][0]
    got = prog.download(logits)
    assert oracle.normwise_error(got, K["cifar_logits"]) <= TOL
    # the stored label buffer is all zeros, so the loss is exactly 0
    assert float(prog.download(loss).ravel()[0]) == float(K["cifar_loss"][0]) == 0.0
    assert np.array_equal(np.argmax(got, axis=1), np.argmax(K["cifar_logits"], axis=1))
    # the filters stayed int8 on the device, the image became fp32
    info = prog.info()
    assert info["launches"] >= 1
    release(*res)


def test_v2_fp32_file_gives_identical_bits(dev, tmp_path):
    lib = graph_lib()
    g = lib.lancius_graph_load(str(MODELS / "pytorch_lenet.lancius").encode())
    path = tmp_path / "lenet_fp32.lancius2"
    assert lib.lancius_graph_save_v2(g, str(path).encode(), abi.DTYPE_FP32) == 0
    lib.lancius_graph_destroy(g)
    outs = []
    for p in (MODELS / "pytorch_lenet.lancius", path):
        res = run_mapped(dev, p, feed=feed_lenet)
        outs.append(res[0].download(lenet_io(res[1], res[2])[1]).ravel())
        assert res[2].format in (9, 2)
        release(*res)
    assert np.array_equal(outs[0], outs[1])


def test_upload_file_conversions(dev, tmp_path):
    """Tensors spanning several 16 MiB staging pieces: fp64 -> fp32 (round
    to nearest), fp32 copy, int8 copy, int8 -> fp32 dequantized in fp64."""
    a64 = prng.normal(700, (5_000_003,)).astype(np.float64) * np.pi  # 40 MB, 3 pieces
    a32 = prng.normal(701, (4_500_001,))                             # 18 MB, 2 pieces
    q = np.round(prng.uniform(702, (17_000_001,), -127.4, 127.4)).astype(np.int8)
    path = tmp_path / "blob.bin"
    blob = b"PAD" + a64.tobytes() + a32.tobytes() + q.tobytes()
    path.write_bytes(blob)
    offs = [3, 3 + a64.nbytes, 3 + a64.nbytes + a32.nbytes]
    bufs = [dev.alloc(a64.size * 4), dev.alloc(a32.size * 4), dev.alloc(q.size), dev.alloc(q.size * 4)]
    scale = 0.0123
    T = FileTensor * 4
    ts = T((bufs[0].ptr, 2, 0, offs[0], a64.size, 0.0), (bufs[1].ptr, 2, 2, offs[1], a32.size, 0.0),
           (bufs[2].ptr, 1, 1, offs[2], q.size, 0.0), (bufs[3].ptr, 2, 1, offs[2], q.size, scale))
    case("upload_file conversions")
    rc = dev.lib.lancius_hip_upload_file(dev.ctx, str(path).encode(), 4, ts)
    assert rc == 0, dev.lib.lancius_hip_last_error()
    assert np.array_equal(dev.download(bufs[0], (a64.size,)), a64.astype(np.float32))
    assert np.array_equal(dev.download(bufs[1], (a32.size,)), a32)
    assert np.array_equal(dev.download(bufs[2], (q.size,), np.int8), q)
    assert np.array_equal(dev.download(bufs[3], (q.size,)), (q.astype(np.float64) * scale).astype(np.float32))
    for b in bufs:
        b.free()


def test_upload_file_rejects_bad_requests(dev, tmp_path):
    path = tmp_path / "small.bin"
    path.write_bytes(b"\0" * 1000)
    buf = dev.alloc(4096)
    case("upload_file refusals")
    for t, code in (((buf.ptr, 2, 0, 0, 126, 0.0), -3),   # 1008 bytes > 1000
                    ((buf.ptr, 2, 0, 1001, 0, 0.0), -3),  # offset past the end
                    ((buf.ptr, 1, 0, 0, 8, 0.0), -5),     # fp64 into int8
                    ((None, 2, 2, 0, 4, 0.0), -2)):
        ts = (FileTensor * 1)(t)
        assert dev.lib.lancius_hip_upload_file(dev.ctx, str(path).encode(), 1, ts) == code
    ts = (FileTensor * 1)((buf.ptr, 2, 2, 0, 4, 0.0))
    assert dev.lib.lancius_hip_upload_file(dev.ctx, str(tmp_path / "missing").encode(), 1, ts) == -4
    buf.free()


def test_upload_weights_rejects_a_foreign_map(dev):
    """A map whose nodes are not this program's INPUTs is refused before any
    copy."""
    lib = graph_lib()
    wm = abi.WeightMap()
    g = lib.lancius_graph_load_mapped(str(MODELS / "test_model.lancius").encode(), C.byref(wm))
    g2 = lib.lancius_graph_create()
    a = lib.lancius_input(g2, 2, 2)
    lib.lancius_relu(g2, a)
    sched = lib.lancius_ir_schedule(g2)
    prog = DeviceProgram(dev, g2, sched)
    case("upload_weights foreign map")
    with pytest.raises(HipError):
        prog.upload_weights(MODELS / "test_model.lancius", wm)
    prog.close()
    lib.lancius_schedule_destroy(sched)
    lib.lancius_graph_destroy(g2)
    lib.lancius_weight_map_free(C.byref(wm))
    lib.lancius_graph_destroy(g)
