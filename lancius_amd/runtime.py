"""Python host side of the MI355X backend: loads the C-ABI libraries and wraps
them for numpy users (tests, bench, smoke).

Nothing here computes: every kernel call goes to liblancius_hip.so, and a
missing library raises immediately (there is no CPU fallback).
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

from . import abi

PKG = Path(__file__).resolve().parent
HIP_LIB = PKG / "liblancius_hip.so"
GRAPH_LIB = PKG / "liblancius_graph.so"

ACT_NONE, ACT_RELU, ACT_GELU, ACT_TANH = 0, 1, 2, 3
MAX_GROUP = 16

# LANCIUS_DEVICE_* flags (include/lancius_hip_graph.h)
DEVICE_NO_FUSION, DEVICE_KEEP_ALL, DEVICE_NO_GROUP, DEVICE_GRAPH, DEVICE_NO_CHAIN = 0x1, 0x2, 0x4, 0x8, 0x10


class HipError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"lancius_hip error {code}: {message}")
        self.code = code


class FileTensor(C.Structure):
    """lancius_hip_file_tensor (include/lancius_hip.h)."""
    _fields_ = [("dst", C.c_void_p), ("dst_dtype", C.c_int), ("file_dtype", C.c_int), ("file_offset", C.c_uint64),
                ("elements", C.c_uint64), ("scale", C.c_double)]


class ProgramInfo(C.Structure):
    _fields_ = [
        ("arena_bytes", C.c_size_t),
        ("plan_bytes", C.c_size_t),
        ("input_bytes", C.c_size_t),
        ("launches", C.c_uint32),
        ("fused_nodes", C.c_uint32),
        ("aliased_nodes", C.c_uint32),
        ("replanned", C.c_uint32),
        ("used_caller_plan", C.c_uint32),
    ]


_hip: C.CDLL | None = None
_graph: C.CDLL | None = None


def _declare_hip(lib: C.CDLL) -> C.CDLL:
    vp, sz, i32, f32 = C.c_void_p, C.c_size_t, C.c_int, C.c_float
    vpp = C.POINTER(C.c_void_p)
    lib.lancius_hip_ctx_create.argtypes = [i32, vp, C.POINTER(vp)]
    lib.lancius_hip_ctx_destroy.argtypes = [vp]
    lib.lancius_hip_ctx_destroy.restype = None
    lib.lancius_hip_last_error.restype = C.c_char_p
    lib.lancius_hip_last_status.restype = i32
    lib.lancius_hip_device_count.restype = i32
    lib.lancius_hip_malloc.argtypes = [vp, C.POINTER(vp), sz]
    lib.lancius_hip_free.argtypes = [vp, vp]
    lib.lancius_hip_upload.argtypes = [vp, vp, vp, sz]
    lib.lancius_hip_download.argtypes = [vp, vp, vp, sz]
    lib.lancius_hip_synchronize.argtypes = [vp]
    lib.lancius_hip_timer_start.argtypes = [vp]
    lib.lancius_hip_timer_stop.argtypes = [vp, C.POINTER(f32)]
    lib.lancius_hip_gemm_f32.argtypes = [vp, vp, vp, vp, sz, sz, sz, vp, i32, vp]
    lib.lancius_hip_gemm_grouped_f32.argtypes = [vp, sz, vpp, vpp, vpp, sz, sz, sz, vpp, i32, vpp]
    lib.lancius_hip_gemm_f32_noalloc.argtypes = [vp, vp, vp, vp, sz, sz, sz, vp, i32, vp]
    lib.lancius_hip_conv2d_f32.argtypes = [vp, vp, vp, vp, vp, sz, sz, sz, sz, sz, sz, sz, sz, sz, i32]
    lib.lancius_hip_conv2d_packed_f32.argtypes = [vp, vp, vp, vp, vp, sz, sz, sz, sz, sz, sz, sz, sz, sz, i32]
    lib.lancius_hip_conv2d_pack_weight.argtypes = [vp, vp, vp, sz, sz, sz, sz]
    lib.lancius_hip_conv2d_packed_bytes.argtypes = [sz, sz, sz, sz]
    lib.lancius_hip_conv2d_packed_bytes.restype = sz
    lib.lancius_hip_attention_f32.argtypes = [vp, vp, vp, vp, vp, sz, sz, sz, sz, i32, f32]
    lib.lancius_hip_attention_grouped_f32.argtypes = [vp, sz, vpp, vpp, vpp, vpp, sz, sz, sz, i32, f32]
    lib.lancius_hip_layernorm_f32.argtypes = [vp, vp, vp, vp, vp, sz, sz, f32]
    lib.lancius_hip_layernorm_grouped_f32.argtypes = [vp, sz, C.POINTER(vp), C.POINTER(vp), C.POINTER(vp),
                                                      C.POINTER(vp), sz, sz, f32]
    lib.lancius_hip_softmax_f32.argtypes = [vp, vp, vp, vp, sz, sz]
    lib.lancius_hip_mlp2_f32.argtypes = [vp, vp, vp, vp, vp, vp, i32, vp, vp, sz, sz, sz, sz, i32]
    lib.lancius_hip_mlp2_ex_f32.argtypes = [vp, vp, vp, vp, vp, vp, i32, vp, vp, i32, sz, sz, sz, sz, i32]
    lib.lancius_hip_add_f32.argtypes = [vp, vp, vp, vp, sz]
    lib.lancius_hip_tanh_f32.argtypes = [vp, vp, vp, sz]
    lib.lancius_hip_bias_act_f32.argtypes = [vp, vp, vp, vp, sz, sz, i32]
    lib.lancius_hip_relu_f32.argtypes = [vp, vp, vp, sz]
    lib.lancius_hip_gelu_f32.argtypes = [vp, vp, vp, sz]
    lib.lancius_hip_copy_f32.argtypes = [vp, vp, vp, sz]
    lib.lancius_hip_broadcast_f32.argtypes = [vp, vp, vp, sz, sz, sz]
    lib.lancius_hip_fill_f32.argtypes = [vp, vp, f32, sz]
    lib.lancius_hip_attention_gqa_f32.argtypes = [vp, vp, vp, vp, vp] + [sz] * 6 + [i32, f32]
    lib.lancius_hip_attention_decode_f32.argtypes = [vp, vp, vp, vp, vp, vp] + [sz] * 5 + [f32]
    lib.lancius_hip_rmsnorm_f32.argtypes = [vp, vp, vp, vp, sz, sz, f32]
    lib.lancius_hip_swiglu_f32.argtypes = [vp, vp, vp, vp, sz]
    lib.lancius_hip_rope_f32.argtypes = [vp, vp, vp] + [sz] * 5 + [i32]
    lib.lancius_hip_quantize_i8.argtypes = [vp, vp, vp, vp, sz]
    lib.lancius_hip_gemm_i8_f32.argtypes = [vp, vp, vp, vp, C.c_double, sz, sz, sz, vp, i32, vp]
    lib.lancius_hip_gemm_i8p_f32.argtypes = [vp, vp, vp, vp, C.c_double, sz, sz, sz, vp, i32, vp]
    lib.lancius_hip_i8_pack_weight.argtypes = [vp, vp, vp, sz, sz]
    lib.lancius_hip_i8_packed_bytes.argtypes = [sz, sz]
    lib.lancius_hip_i8_packed_bytes.restype = sz
    lib.lancius_hip_conv2d_i8_f32.argtypes = [vp, vp, vp, vp, C.c_double, vp] + [sz] * 9 + [i32]
    lib.lancius_hip_gemm_ex_f32.argtypes = [vp, vp, vp, vp, sz, sz, sz, i32, i32, vp, i32, vp]
    lib.lancius_hip_gemm_grouped_ex_f32.argtypes = [vp, sz, C.POINTER(vp), C.POINTER(vp), C.POINTER(vp), sz, sz, sz,
                                                    i32, i32, C.POINTER(vp), i32, C.POINTER(vp)]
    for name in ("lancius_hip_sub_f32", "lancius_hip_mul_f32", "lancius_hip_relu_bwd_f32"):
        getattr(lib, name).argtypes = [vp, vp, vp, vp, sz]
    lib.lancius_hip_transpose_f32.argtypes = [vp, vp, vp, sz, sz]
    lib.lancius_hip_sum_f32.argtypes = [vp, vp, vp, sz]
    lib.lancius_hip_sum_axis0_f32.argtypes = [vp, vp, vp, sz, sz]
    lib.lancius_hip_sum_axis1_f32.argtypes = [vp, vp, vp, sz, sz]
    lib.lancius_hip_softmax_bwd_f32.argtypes = [vp, vp, vp, vp, sz, sz]
    lib.lancius_hip_cross_entropy_f32.argtypes = [vp, vp, vp, vp, sz, sz]
    lib.lancius_hip_cross_entropy_bwd_f32.argtypes = [vp, vp, vp, vp, vp, sz, sz]
    lib.lancius_hip_conv2d_bwd_input_f32.argtypes = [vp, vp, vp, vp] + [sz] * 11
    lib.lancius_hip_conv2d_bwd_weight_f32.argtypes = [vp, vp, vp, vp] + [sz] * 11
    lib.lancius_hip_maxpool2d_f32.argtypes = [vp, vp, vp] + [sz] * 6
    lib.lancius_hip_maxpool2d_bwd_f32.argtypes = [vp, vp, vp, vp] + [sz] * 8
    lib.lancius_hip_ctx_create_own_stream.argtypes = [i32, C.POINTER(vp)]
    lib.lancius_hip_ctx_device.argtypes = [vp]
    lib.lancius_hip_ctx_stream.argtypes = [vp]
    lib.lancius_hip_ctx_stream.restype = vp
    lib.lancius_hip_stream_wait.argtypes = [vp, vp]
    lib.lancius_hip_capture_begin.argtypes = [vp]
    lib.lancius_hip_capture_end.argtypes = [vp, C.POINTER(vp)]
    lib.lancius_hip_graph_launch.argtypes = [vp, vp]
    lib.lancius_hip_graph_destroy.argtypes = [vp]
    lib.lancius_hip_graph_destroy.restype = None
    lib.lancius_hip_peak_probe.argtypes = [vp, i32, C.POINTER(C.c_double)]
    lib.kernel_matmul_f32.argtypes = [vp, vp, vp, sz, sz, sz]
    lib.kernel_matmul_f32.restype = None
    # device executor
    lib.lancius_device_program_create.argtypes = [vp, abi.GraphP, abi.ScheduleP, abi.PlanP, C.c_uint32,
                                                  C.POINTER(vp)]
    lib.lancius_device_program_destroy.argtypes = [vp]
    lib.lancius_device_program_destroy.restype = None
    lib.lancius_device_program_info_get.argtypes = [vp, C.POINTER(ProgramInfo)]
    lib.lancius_device_upload.argtypes = [vp, abi.NodeP, vp, i32]
    lib.lancius_device_download.argtypes = [vp, abi.NodeP, vp, i32]
    lib.lancius_device_download_argmax.argtypes = [vp, abi.NodeP, vp]
    lib.lancius_device_buffer.argtypes = [vp, abi.NodeP]
    lib.lancius_device_buffer.restype = vp
    lib.lancius_device_run.argtypes = [vp]
    lib.lancius_schedule_execute_device.argtypes = [abi.ScheduleP, abi.GraphP, vp]
    lib.lancius_device_upload_weights.argtypes = [vp, C.c_char_p, abi.WeightMapP]
    lib.lancius_hip_upload_file.argtypes = [vp, C.c_char_p, sz, C.POINTER(FileTensor)]
    return lib


def hip_lib() -> C.CDLL:
    """liblancius_hip.so; raises if it has not been built."""
    global _hip
    if _hip is None:
        if not HIP_LIB.exists():
            raise RuntimeError(f"{HIP_LIB} is missing: build it with `python -m lancius_amd.build`")
        _hip = _declare_hip(C.CDLL(str(HIP_LIB)))
    return _hip


def graph_lib() -> C.CDLL:
    global _graph
    if _graph is None:
        if not GRAPH_LIB.exists():
            raise RuntimeError(f"{GRAPH_LIB} is missing: build it with `python -m lancius_amd.build`")
        lib = abi.declare_model_io(abi.declare_graph_api(C.CDLL(str(GRAPH_LIB))))
        lib.lancius_graph_set_dtype.argtypes = [abi.GraphP, C.c_int]
        lib.lancius_graph_set_dtype.restype = None
        _graph = lib
    return _graph


def device_count() -> int:
    return int(hip_lib().lancius_hip_device_count())


def _check(rc: int) -> None:
    if rc != 0:
        raise HipError(rc, hip_lib().lancius_hip_last_error().decode(errors="replace"))


def _ptrs(items) -> C.Array:
    arr = (C.c_void_p * max(1, len(items)))()
    for i, x in enumerate(items):
        arr[i] = None if x is None else int(x)
    return arr


class Buffer:
    """A device allocation owned by a Device."""

    def __init__(self, dev: "Device", ptr: int, nbytes: int):
        self.dev, self.ptr, self.nbytes = dev, ptr, nbytes

    def __int__(self) -> int:
        return self.ptr

    def offset(self, nbytes: int) -> int:
        return self.ptr + nbytes

    def free(self) -> None:
        if self.ptr:
            _check(self.dev.lib.lancius_hip_free(self.dev.ctx, C.c_void_p(self.ptr)))
            self.ptr = 0


class Device:
    """A lancius_hip context on one GPU: the null stream by default, a
    caller's hipStream_t (`stream`), or a stream of its own (`own_stream`)."""

    def __init__(self, device: int = 0, stream: int | None = None, own_stream: bool = False):
        self.lib = hip_lib()
        ctx = C.c_void_p()
        if own_stream:
            _check(self.lib.lancius_hip_ctx_create_own_stream(device, C.byref(ctx)))
        else:
            _check(self.lib.lancius_hip_ctx_create(device, C.c_void_p(stream) if stream else None, C.byref(ctx)))
        self.ctx = ctx
        self._buffers: list[Buffer] = []

    # -- memory --------------------------------------------------------------
    def alloc(self, nbytes: int) -> Buffer:
        p = C.c_void_p()
        _check(self.lib.lancius_hip_malloc(self.ctx, C.byref(p), max(1, int(nbytes))))
        b = Buffer(self, p.value, int(nbytes))
        self._buffers.append(b)
        return b

    def upload(self, arr: np.ndarray) -> Buffer:
        arr = np.ascontiguousarray(arr)
        b = self.alloc(arr.nbytes)
        _check(self.lib.lancius_hip_upload(self.ctx, C.c_void_p(b.ptr), arr.ctypes.data_as(C.c_void_p), arr.nbytes))
        return b

    def write(self, dst: int, arr: np.ndarray) -> None:
        arr = np.ascontiguousarray(arr)
        _check(self.lib.lancius_hip_upload(self.ctx, C.c_void_p(int(dst)), arr.ctypes.data_as(C.c_void_p), arr.nbytes))

    def download(self, src: int, shape, dtype=np.float32) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        _check(self.lib.lancius_hip_download(self.ctx, out.ctypes.data_as(C.c_void_p), C.c_void_p(int(src)),
                                             out.nbytes))
        return out

    def synchronize(self) -> None:
        _check(self.lib.lancius_hip_synchronize(self.ctx))

    def timer_start(self) -> None:
        _check(self.lib.lancius_hip_timer_start(self.ctx))

    def timer_stop(self) -> float:
        ms = C.c_float()
        _check(self.lib.lancius_hip_timer_stop(self.ctx, C.byref(ms)))
        return float(ms.value)

    def peak_probe(self, which: str) -> float:
        """Measured fp32 MFMA TFLOP/s ("mfma"), HBM copy GB/s ("hbm") or HBM read GB/s ("hbm_read")."""
        out = C.c_double()
        _check(self.lib.lancius_hip_peak_probe(self.ctx, {"mfma": 0, "hbm": 1, "hbm_read": 2}[which], C.byref(out)))
        return float(out.value)

    def close(self) -> None:
        for b in self._buffers:
            b.free()
        self._buffers.clear()
        if self.ctx:
            self.lib.lancius_hip_ctx_destroy(self.ctx)
            self.ctx = None

    # -- kernels (device addresses as ints / Buffers) --------------------------
    def gemm(self, C_, A, B, M, K, N, bias=None, act=ACT_NONE, residual=None) -> None:
        _check(self.lib.lancius_hip_gemm_f32(self.ctx, _vp(C_), _vp(A), _vp(B), M, K, N, _vp(bias), act,
                                             _vp(residual)))

    def gemm_ex(self, C_, A, B, M, K, N, trans_a=False, trans_b=False, bias=None, act=ACT_NONE,
                residual=None) -> None:
        _check(self.lib.lancius_hip_gemm_ex_f32(self.ctx, _vp(C_), _vp(A), _vp(B), M, K, N, int(trans_a),
                                                int(trans_b), _vp(bias), act, _vp(residual)))

    def gemm_grouped(self, Cs, As, Bs, M, K, N, biases=None, act=ACT_NONE, residuals=None) -> None:
        n = len(Cs)
        _check(self.lib.lancius_hip_gemm_grouped_f32(
            self.ctx, n, _ptrs(Cs), _ptrs(As), _ptrs(Bs), M, K, N,
            _ptrs(biases) if biases is not None else None, act,
            _ptrs(residuals) if residuals is not None else None))

    def conv2d(self, out, x, w, bias, N, C_in, H, W, C_out, K_h, K_w, stride, pad, act=ACT_NONE) -> None:
        _check(self.lib.lancius_hip_conv2d_f32(self.ctx, _vp(out), _vp(x), _vp(w), _vp(bias), N, C_in, H, W, C_out,
                                               K_h, K_w, stride, pad, act))

    def attention(self, out, q, k, v, batch, S, H, D, causal=True, scale=None) -> None:
        scale = 1.0 / np.sqrt(D) if scale is None else scale
        _check(self.lib.lancius_hip_attention_f32(self.ctx, _vp(out), _vp(q), _vp(k), _vp(v), batch, S, H, D,
                                                  int(bool(causal)), float(scale)))

    def attention_grouped(self, outs, qs, ks, vs, S, H, D, causal=True, scale=None) -> None:
        scale = 1.0 / np.sqrt(D) if scale is None else scale
        _check(self.lib.lancius_hip_attention_grouped_f32(self.ctx, len(outs), _ptrs(outs), _ptrs(qs), _ptrs(ks),
                                                          _ptrs(vs), S, H, D, int(bool(causal)), float(scale)))

    def layernorm(self, out, x, gamma, beta, rows, hidden, eps=1e-5) -> None:
        _check(self.lib.lancius_hip_layernorm_f32(self.ctx, _vp(out), _vp(x), _vp(gamma), _vp(beta), rows, hidden,
                                                  float(eps)))

    def layernorm_grouped(self, outs, xs, gammas, betas, rows, hidden, eps=1e-5) -> None:
        _check(self.lib.lancius_hip_layernorm_grouped_f32(self.ctx, len(outs), _ptrs(outs), _ptrs(xs), _ptrs(gammas),
                                                          _ptrs(betas), rows, hidden, float(eps)))

    def softmax(self, probs, argmax, x, rows, cols) -> None:
        _check(self.lib.lancius_hip_softmax_f32(self.ctx, _vp(probs), _vp(argmax), _vp(x), rows, cols))

    def mlp2(self, out, argmax, x, w1, b1, act1, w2, b2, M, K1, N1, N2, softmax=True, act2=None) -> None:
        if act2 is None:
            _check(self.lib.lancius_hip_mlp2_f32(self.ctx, _vp(out), _vp(argmax), _vp(x), _vp(w1), _vp(b1), act1,
                                                 _vp(w2), _vp(b2), M, K1, N1, N2, int(bool(softmax))))
        else:
            _check(self.lib.lancius_hip_mlp2_ex_f32(self.ctx, _vp(out), _vp(argmax), _vp(x), _vp(w1), _vp(b1), act1,
                                                    _vp(w2), _vp(b2), act2, M, K1, N1, N2, int(bool(softmax))))

    def add(self, out, a, b, n) -> None:
        _check(self.lib.lancius_hip_add_f32(self.ctx, _vp(out), _vp(a), _vp(b), n))

    def relu(self, out, a, n) -> None:
        _check(self.lib.lancius_hip_relu_f32(self.ctx, _vp(out), _vp(a), n))

    def tanh(self, out, a, n) -> None:
        _check(self.lib.lancius_hip_tanh_f32(self.ctx, _vp(out), _vp(a), n))

    def bias_act(self, out, a, bias, rows, cols, act=ACT_NONE) -> None:
        _check(self.lib.lancius_hip_bias_act_f32(self.ctx, _vp(out), _vp(a), _vp(bias), rows, cols, act))

    def gelu(self, out, a, n) -> None:
        _check(self.lib.lancius_hip_gelu_f32(self.ctx, _vp(out), _vp(a), n))

    def copy(self, out, a, n) -> None:
        _check(self.lib.lancius_hip_copy_f32(self.ctx, _vp(out), _vp(a), n))

    def broadcast(self, out, row, rows, cols, cols_in) -> None:
        _check(self.lib.lancius_hip_broadcast_f32(self.ctx, _vp(out), _vp(row), rows, cols, cols_in))

    def fill(self, out, value, n) -> None:
        _check(self.lib.lancius_hip_fill_f32(self.ctx, _vp(out), float(value), n))

    # -- decode-side attention family ------------------------------------------
    def attention_gqa(self, out, q, k, v, batch, S_q, S_kv, H_q, H_kv, D, causal=True, scale=None) -> None:
        scale = 1.0 / np.sqrt(D) if scale is None else scale
        _check(self.lib.lancius_hip_attention_gqa_f32(self.ctx, _vp(out), _vp(q), _vp(k), _vp(v), batch, S_q, S_kv,
                                                      H_q, H_kv, D, int(bool(causal)), float(scale)))

    def attention_decode(self, out, q, k_cache, v_cache, kv_lens, batch, S_kv, H_q, H_kv, D, scale=None) -> None:
        scale = 1.0 / np.sqrt(D) if scale is None else scale
        _check(self.lib.lancius_hip_attention_decode_f32(self.ctx, _vp(out), _vp(q), _vp(k_cache), _vp(v_cache),
                                                         _vp(kv_lens), batch, S_kv, H_q, H_kv, D, float(scale)))

    def rmsnorm(self, out, x, gamma, rows, hidden, eps=1e-5) -> None:
        _check(self.lib.lancius_hip_rmsnorm_f32(self.ctx, _vp(out), _vp(x), _vp(gamma), rows, hidden, float(eps)))

    def swiglu(self, out, gate, up, n) -> None:
        _check(self.lib.lancius_hip_swiglu_f32(self.ctx, _vp(out), _vp(gate), _vp(up), n))

    def rope(self, out, x, count, batch, S, H, head_dim, pos_offset=0) -> None:
        _check(self.lib.lancius_hip_rope_f32(self.ctx, _vp(out), _vp(x), count, batch, S, H, head_dim,
                                             int(pos_offset)))

    # -- int8 path -------------------------------------------------------------
    def quantize_i8(self, q, scale, x, n) -> None:
        """q (int8 device buffer), scale (device buffer of one double)."""
        _check(self.lib.lancius_hip_quantize_i8(self.ctx, _vp(q), _vp(scale), _vp(x), n))

    def gemm_i8(self, C_, A, B_i8, scale_b, M, K, N, bias=None, act=ACT_NONE, residual=None) -> None:
        _check(self.lib.lancius_hip_gemm_i8_f32(self.ctx, _vp(C_), _vp(A), _vp(B_i8), float(scale_b), M, K, N,
                                                _vp(bias), act, _vp(residual)))

    def conv2d_packed_bytes(self, C_out, C_in, K_h, K_w) -> int:
        return int(self.lib.lancius_hip_conv2d_packed_bytes(C_out, C_in, K_h, K_w))

    def conv2d_pack_weight(self, packed, w, C_out, C_in, K_h, K_w) -> None:
        _check(self.lib.lancius_hip_conv2d_pack_weight(self.ctx, _vp(packed), _vp(w), C_out, C_in, K_h, K_w))

    def conv2d_packed(self, out, x, packed, bias, N, C_in, H, W, C_out, K_h, K_w, stride, pad, act=ACT_NONE) -> None:
        _check(self.lib.lancius_hip_conv2d_packed_f32(self.ctx, _vp(out), _vp(x), _vp(packed), _vp(bias), N, C_in, H,
                                                      W, C_out, K_h, K_w, stride, pad, act))

    def i8_packed_bytes(self, K, N) -> int:
        return int(self.lib.lancius_hip_i8_packed_bytes(K, N))

    def i8_pack_weight(self, packed, B_i8, K, N) -> None:
        _check(self.lib.lancius_hip_i8_pack_weight(self.ctx, _vp(packed), _vp(B_i8), K, N))

    def gemm_i8p(self, C_, A, packed, scale_b, M, K, N, bias=None, act=ACT_NONE, residual=None) -> None:
        _check(self.lib.lancius_hip_gemm_i8p_f32(self.ctx, _vp(C_), _vp(A), _vp(packed), float(scale_b), M, K, N,
                                                 _vp(bias), act, _vp(residual)))

    def conv2d_i8(self, out, x, w_i8, scale_w, bias, N, C_in, H, W, C_out, K_h, K_w, stride, pad,
                  act=ACT_NONE) -> None:
        _check(self.lib.lancius_hip_conv2d_i8_f32(self.ctx, _vp(out), _vp(x), _vp(w_i8), float(scale_w), _vp(bias),
                                                  N, C_in, H, W, C_out, K_h, K_w, stride, pad, act))

    # -- training / reduction ops ----------------------------------------------
    def sub(self, out, a, b, n) -> None:
        _check(self.lib.lancius_hip_sub_f32(self.ctx, _vp(out), _vp(a), _vp(b), n))

    def mul(self, out, a, b, n) -> None:
        _check(self.lib.lancius_hip_mul_f32(self.ctx, _vp(out), _vp(a), _vp(b), n))

    def relu_bwd(self, out, grad, fwd, n) -> None:
        _check(self.lib.lancius_hip_relu_bwd_f32(self.ctx, _vp(out), _vp(grad), _vp(fwd), n))

    def transpose(self, out, a, rows, cols) -> None:
        _check(self.lib.lancius_hip_transpose_f32(self.ctx, _vp(out), _vp(a), rows, cols))

    def sum(self, out, a, n) -> None:
        _check(self.lib.lancius_hip_sum_f32(self.ctx, _vp(out), _vp(a), n))

    def sum_axis0(self, out, a, rows, cols) -> None:
        _check(self.lib.lancius_hip_sum_axis0_f32(self.ctx, _vp(out), _vp(a), rows, cols))

    def sum_axis1(self, out, a, rows, cols) -> None:
        _check(self.lib.lancius_hip_sum_axis1_f32(self.ctx, _vp(out), _vp(a), rows, cols))

    def softmax_bwd(self, out, dy, y, rows, cols) -> None:
        _check(self.lib.lancius_hip_softmax_bwd_f32(self.ctx, _vp(out), _vp(dy), _vp(y), rows, cols))

    def cross_entropy(self, out, x, y, rows, cols) -> None:
        _check(self.lib.lancius_hip_cross_entropy_f32(self.ctx, _vp(out), _vp(x), _vp(y), rows, cols))

    def cross_entropy_bwd(self, out, x, y, g, rows, cols) -> None:
        _check(self.lib.lancius_hip_cross_entropy_bwd_f32(self.ctx, _vp(out), _vp(x), _vp(y), _vp(g), rows, cols))

    def conv2d_bwd_input(self, dx, dy, w, N, C_in, H, W, C_out, H_out, W_out, K_h, K_w, stride, pad) -> None:
        _check(self.lib.lancius_hip_conv2d_bwd_input_f32(self.ctx, _vp(dx), _vp(dy), _vp(w), N, C_in, H, W, C_out,
                                                         H_out, W_out, K_h, K_w, stride, pad))

    def conv2d_bwd_weight(self, dw, dy, x, N, C_in, H, W, C_out, H_out, W_out, K_h, K_w, stride, pad) -> None:
        _check(self.lib.lancius_hip_conv2d_bwd_weight_f32(self.ctx, _vp(dw), _vp(dy), _vp(x), N, C_in, H, W, C_out,
                                                          H_out, W_out, K_h, K_w, stride, pad))

    def maxpool2d(self, out, x, N, C, H, W, K, stride) -> None:
        _check(self.lib.lancius_hip_maxpool2d_f32(self.ctx, _vp(out), _vp(x), N, C, H, W, K, stride))

    def maxpool2d_bwd(self, dx, dy, x, N, C, H, W, H_out, W_out, K, stride) -> None:
        _check(self.lib.lancius_hip_maxpool2d_bwd_f32(self.ctx, _vp(dx), _vp(dy), _vp(x), N, C, H, W, H_out, W_out,
                                                      K, stride))


def _vp(x) -> C.c_void_p | None:
    if x is None:
        return None
    return C.c_void_p(int(x))


class DeviceProgram:
    """A compiled graph (lancius_device_program) on a Device."""

    def __init__(self, dev: Device, g: abi.GraphP, sched: abi.ScheduleP, plan: abi.PlanP | None = None,
                 flags: int = 0):
        self.dev = dev
        self.lib = dev.lib
        p = C.c_void_p()
        _check(self.lib.lancius_device_program_create(dev.ctx, g, sched, plan, flags, C.byref(p)))
        self.prog = p

    def info(self) -> dict:
        inf = ProgramInfo()
        _check(self.lib.lancius_device_program_info_get(self.prog, C.byref(inf)))
        return {f: getattr(inf, f) for f, _ in ProgramInfo._fields_}

    def upload(self, node: abi.NodeP, arr: np.ndarray) -> None:
        arr = np.ascontiguousarray(arr)
        dt = {np.dtype(np.float32): abi.DTYPE_FP32, np.dtype(np.float64): abi.DTYPE_FP64,
              np.dtype(np.int8): abi.DTYPE_INT8}.get(arr.dtype)
        if dt is None:
            raise TypeError("upload takes float32, float64 or int8 (quantized weights)")
        if arr.size != abi.node_elems(node):
            raise ValueError(f"node has {abi.node_elems(node)} elements, array {arr.size}")
        _check(self.lib.lancius_device_upload(self.prog, node, arr.ctypes.data_as(C.c_void_p), dt))

    def download(self, node: abi.NodeP, dtype=np.float32) -> np.ndarray:
        out = np.empty(abi.node_shape(node), dtype=dtype)
        dt = abi.DTYPE_FP32 if out.dtype == np.float32 else abi.DTYPE_FP64
        _check(self.lib.lancius_device_download(self.prog, node, out.ctypes.data_as(C.c_void_p), dt))
        return out

    def argmax(self, node: abi.NodeP) -> np.ndarray:
        out = np.empty(node.contents.shape[0], dtype=np.int32)
        _check(self.lib.lancius_device_download_argmax(self.prog, node, out.ctypes.data_as(C.c_void_p)))
        return out

    def buffer(self, node: abi.NodeP) -> int:
        return int(self.lib.lancius_device_buffer(self.prog, node) or 0)

    def upload_weights(self, path, wmap: abi.WeightMap) -> None:
        """Stream every tensor of a lancius_graph_load_mapped map from the
        model file into the program's INPUT buffers."""
        _check(self.lib.lancius_device_upload_weights(self.prog, str(path).encode(), C.byref(wmap)))

    def run(self) -> None:
        _check(self.lib.lancius_device_run(self.prog))

    def close(self) -> None:
        if self.prog:
            self.lib.lancius_device_program_destroy(self.prog)
            self.prog = None
