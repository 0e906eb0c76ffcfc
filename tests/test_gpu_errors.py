"""Error paths of the C ABI on the device: an allocation HBM cannot satisfy
comes back as the reference's out-of-memory status (LANCIUS_ERROR_OOM = -1,
bleeding/v11A1/include/lancius/lancius_error.h:6-18) with a message, nothing
aborts, and the same context keeps working afterwards."""
import numpy as np
import pytest

import oracle
from lancius_amd import DeviceProgram, HipError, graph_lib, prng
from tests.conftest import case

pytestmark = pytest.mark.gpu


def _gemm_still_right(dev):
    M, K, N = 96, 200, 160
    A, B = prng.normal(5, (M, K)), prng.normal(6, (K, N))
    dA, dB, dC = dev.upload(A), dev.upload(B), dev.alloc(M * N * 4)
    dev.gemm(dC, dA, dB, M, K, N)
    got = dev.download(dC, (M, N))
    for b in (dA, dB, dC):
        b.free()
    assert oracle.normwise_error(got, oracle.matmul(A, B)) <= oracle.tolerance(K)


def test_malloc_beyond_hbm_is_oom(dev):
    case("lancius_hip_malloc of 1 TiB")
    with pytest.raises(HipError) as e:
        dev.alloc(1 << 40)
    assert e.value.code == -1, e.value
    assert "hipMalloc" in dev.lib.lancius_hip_last_error().decode()
    _gemm_still_right(dev)


def test_program_beyond_hbm_is_oom(dev):
    """A graph whose arena (a 256 GiB INPUT and its 256 GiB RELU) cannot fit
    in 288 GB of HBM: lancius_device_program_create returns -1 and frees what it
    built; the context then runs a GEMM correctly."""
    lib = graph_lib()
    g = lib.lancius_graph_create()
    x = lib.lancius_input(g, 1 << 18, 1 << 18)
    lib.lancius_relu(g, x)
    sched = lib.lancius_ir_schedule(g)
    case("device program of a 512 GiB graph")
    with pytest.raises(HipError) as e:
        DeviceProgram(dev, g, sched, None, 0)
    assert e.value.code == -1, e.value
    lib.lancius_schedule_destroy(sched)
    lib.lancius_graph_destroy(g)
    _gemm_still_right(dev)
    # the failed call left no half-built state behind: a normal program works
    g = lib.lancius_graph_create()
    x = lib.lancius_input(g, 64, 64)
    r = lib.lancius_relu(g, x)
    sched = lib.lancius_ir_schedule(g)
    prog = DeviceProgram(dev, g, sched, None, 0)
    xv = prng.normal(9, (64, 64))
    prog.upload(x, xv)
    prog.run()
    np.testing.assert_array_equal(prog.download(r).reshape(64, 64), np.maximum(xv, 0))
    prog.close()
    lib.lancius_schedule_destroy(sched)
    lib.lancius_graph_destroy(g)
