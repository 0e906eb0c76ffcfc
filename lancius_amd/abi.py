"""ctypes mirror of the Lancius graph structs (include/lancius_abi.h).

Field order and types follow bleeding/v11A1/include/lancius/lancius_ir.h:31-62,
lancius_types.h:9-60, lancius_scheduler.h:10-12 and
lancius_memory_planner.h:13-17.  Used by the tests and the bench to inspect
nodes built by liblancius_graph (or the reference library).
"""
from __future__ import annotations

import ctypes as C

DTYPE_FP64, DTYPE_INT8, DTYPE_FP32, DTYPE_INT32 = 0, 1, 2, 3

OP = {
    "NOP": 0, "INPUT": 1, "CONST": 2, "ADD": 3, "SUB": 4, "MUL": 5, "MATMUL": 6, "RELU": 7,
    "SOFTMAX": 8, "SUM": 9, "BROADCAST": 10, "TRANSPOSE": 11, "RELU_BWD": 12, "SOFTMAX_BWD": 13,
    "SUM_AXIS0": 14, "SUM_AXIS1": 15, "CONV2D": 16, "MAXPOOL2D": 17, "FLATTEN": 18,
    "CONV2D_RELU_FUSED": 19, "CROSS_ENTROPY": 20, "CROSS_ENTROPY_BWD": 21, "PERMUTE": 22,
    "MATMUL_BATCHED": 23, "CONV2D_BWD": 24, "CONV2D_BWD_W": 25, "MAXPOOL2D_BWD": 26, "RESHAPE": 27,
    "EMBEDDING": 28, "LAYERNORM": 29, "GELU": 30, "ROPE": 31, "ATTENTION": 32, "KV_CACHE_READ": 33,
    "KV_CACHE_WRITE": 34, "RMSNORM": 35, "SWIGLU": 36, "GQA": 37,
}
OP_NAME = {v: k for k, v in OP.items()}


class RuntimeState(C.Structure):
    _fields_ = [
        ("buffer", C.c_void_p),
        ("buffer_int8", C.c_void_p),
        ("dtype", C.c_int),
        ("scale", C.c_double),
        ("owner", C.c_int),
        ("buffer_owner", C.c_int),
        ("int8_owner", C.c_int),
        ("offset", C.c_size_t),
        ("flags", C.c_uint32),
    ]


class Node(C.Structure):
    pass


Node._fields_ = [
    ("id", C.c_uint32),
    ("op", C.c_int),
    ("shape", C.c_size_t * 4),
    ("ndim", C.c_uint8),
    ("kernel_h", C.c_uint32),
    ("kernel_w", C.c_uint32),
    ("stride", C.c_uint32),
    ("pad", C.c_uint32),
    ("axes", C.c_uint32 * 4),
    ("inputs", C.POINTER(C.POINTER(Node))),
    ("input_count", C.c_uint32),
    ("attr_val", C.c_double),
    ("runtime_data", C.POINTER(C.c_double)),
    ("dtype", C.c_int),
    ("scale", C.c_double),
    ("runtime_data_int8", C.POINTER(C.c_int8)),
    ("rt", C.POINTER(RuntimeState)),
    ("is_view", C.c_uint8),
    ("strides", C.c_size_t * 4),
    ("view_source", C.POINTER(Node)),
]


class Graph(C.Structure):
    _fields_ = [
        ("arena", C.c_void_p),
        ("nodes", C.POINTER(C.POINTER(Node))),
        ("node_count", C.c_uint32),
        ("node_cap", C.c_uint32),
        ("next_id", C.c_uint32),
        ("rt_states", C.POINTER(RuntimeState)),
        ("rt_cap", C.c_size_t),
    ]


class Wave(C.Structure):
    _fields_ = [("nodes", C.POINTER(C.POINTER(Node))), ("node_count", C.c_uint32)]


class MemoryPlan(C.Structure):
    _fields_ = [
        ("peak_memory", C.c_size_t),
        ("offsets", C.POINTER(C.c_size_t)),
        ("is_pooled", C.POINTER(C.c_uint8)),
    ]


class Schedule(C.Structure):
    _fields_ = [
        ("waves", C.POINTER(Wave)),
        ("wave_count", C.c_uint32),
        ("plan", C.POINTER(MemoryPlan)),
        ("static_pool", C.c_void_p),
    ]


NodeP = C.POINTER(Node)
GraphP = C.POINTER(Graph)
ScheduleP = C.POINTER(Schedule)
PlanP = C.POINTER(MemoryPlan)


def node_elems(n: NodeP) -> int:
    e = 1
    for d in range(n.contents.ndim):
        e *= n.contents.shape[d]
    return e


def node_shape(n: NodeP) -> tuple[int, ...]:
    return tuple(n.contents.shape[d] for d in range(n.contents.ndim))


class TrainingGraph(C.Structure):
    """lancius_training_graph (B/include/lancius/lancius_autodiff.h:8-13)."""
    _fields_ = [("graph", GraphP), ("loss_node", NodeP), ("grad_nodes", C.POINTER(NodeP)), ("max_id", C.c_uint32)]


TrainingGraphP = C.POINTER(TrainingGraph)


class WeightRef(C.Structure):
    """lancius_weight_ref (include/lancius_abi.h)."""
    _fields_ = [("node", NodeP), ("file_offset", C.c_uint64), ("elements", C.c_uint64), ("file_dtype", C.c_int),
                ("scale", C.c_double)]


class WeightMap(C.Structure):
    """lancius_weight_map (include/lancius_abi.h)."""
    _fields_ = [("format", C.c_uint32), ("count", C.c_uint32), ("refs", C.POINTER(WeightRef)),
                ("file_bytes", C.c_uint64), ("crc32", C.c_uint32)]


WeightMapP = C.POINTER(WeightMap)


def declare_graph_api(lib: C.CDLL) -> C.CDLL:
    """Prototypes of the graph-path functions shared by liblancius_graph and
    the reference library (same names and signatures)."""
    sz = C.c_size_t
    lib.lancius_graph_create.restype = GraphP
    lib.lancius_graph_destroy.argtypes = [GraphP]
    lib.lancius_graph_destroy.restype = None
    lib.lancius_input.argtypes = [GraphP, sz, sz]
    lib.lancius_input.restype = NodeP
    lib.lancius_input_4d.argtypes = [GraphP, sz, sz, sz, sz]
    lib.lancius_input_4d.restype = NodeP
    lib.lancius_const.argtypes = [GraphP, C.c_double, sz, sz]
    lib.lancius_const.restype = NodeP
    for name in ("lancius_add", "lancius_matmul"):
        getattr(lib, name).argtypes = [GraphP, NodeP, NodeP]
        getattr(lib, name).restype = NodeP
    for name in ("lancius_relu", "lancius_softmax", "lancius_gelu", "lancius_flatten"):
        getattr(lib, name).argtypes = [GraphP, NodeP]
        getattr(lib, name).restype = NodeP
    lib.lancius_broadcast.argtypes = [GraphP, NodeP, sz, sz]
    lib.lancius_broadcast.restype = NodeP
    lib.lancius_conv2d.argtypes = [GraphP, NodeP, NodeP, C.c_uint32, C.c_uint32]
    lib.lancius_conv2d.restype = NodeP
    lib.lancius_reshape.argtypes = [GraphP, NodeP, C.c_uint8, sz, sz, sz, sz]
    lib.lancius_reshape.restype = NodeP
    lib.lancius_attention.argtypes = [GraphP, NodeP, NodeP, NodeP]
    lib.lancius_attention.restype = NodeP
    lib.lancius_layernorm.argtypes = [GraphP, NodeP, NodeP, NodeP]
    lib.lancius_layernorm.restype = NodeP
    for name in ("lancius_sub", "lancius_mul", "lancius_relu_bwd", "lancius_softmax_bwd", "lancius_cross_entropy"):
        getattr(lib, name).argtypes = [GraphP, NodeP, NodeP]
        getattr(lib, name).restype = NodeP
    for name in ("lancius_sum", "lancius_transpose", "lancius_sum_axis0", "lancius_sum_axis1"):
        getattr(lib, name).argtypes = [GraphP, NodeP]
        getattr(lib, name).restype = NodeP
    lib.lancius_broadcast_4d.argtypes = [GraphP, NodeP, sz, sz, sz, sz]
    lib.lancius_broadcast_4d.restype = NodeP
    lib.lancius_maxpool2d.argtypes = [GraphP, NodeP, C.c_uint32, C.c_uint32]
    lib.lancius_maxpool2d.restype = NodeP
    lib.lancius_cross_entropy_bwd.argtypes = [GraphP, NodeP, NodeP, NodeP]
    lib.lancius_cross_entropy_bwd.restype = NodeP
    lib.lancius_conv2d_bwd.argtypes = [GraphP, NodeP, NodeP, NodeP, C.c_uint32, C.c_uint32]
    lib.lancius_conv2d_bwd.restype = NodeP
    lib.lancius_conv2d_bwd_w.argtypes = [GraphP, NodeP, NodeP, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32]
    lib.lancius_conv2d_bwd_w.restype = NodeP
    lib.lancius_maxpool2d_bwd.argtypes = [GraphP, NodeP, NodeP, C.c_uint32, C.c_uint32]
    lib.lancius_maxpool2d_bwd.restype = NodeP
    lib.lancius_ir_autodiff.argtypes = [GraphP, NodeP]
    lib.lancius_ir_autodiff.restype = TrainingGraphP
    lib.lancius_training_graph_destroy.argtypes = [TrainingGraphP]
    lib.lancius_training_graph_destroy.restype = None
    for name in ("lancius_rmsnorm", "lancius_swiglu"):
        getattr(lib, name).argtypes = [GraphP, NodeP, NodeP]
        getattr(lib, name).restype = NodeP
    lib.lancius_gqa.argtypes = [GraphP, NodeP, NodeP, NodeP, C.c_uint32, C.c_uint32]
    lib.lancius_gqa.restype = NodeP
    lib.lancius_quantize_graph.argtypes = [GraphP]
    lib.lancius_quantize_graph.restype = None
    lib.lancius_optimize_fusion.argtypes = [GraphP]
    lib.lancius_optimize_fusion.restype = None
    lib.lancius_ir_schedule.argtypes = [GraphP]
    lib.lancius_ir_schedule.restype = ScheduleP
    lib.lancius_schedule_destroy.argtypes = [ScheduleP]
    lib.lancius_schedule_destroy.restype = None
    lib.lancius_schedule_attach_pool.argtypes = [ScheduleP, C.c_void_p, PlanP]
    lib.lancius_schedule_attach_pool.restype = None
    lib.lancius_schedule_peak_memory.argtypes = [ScheduleP]
    lib.lancius_schedule_peak_memory.restype = sz
    lib.lancius_build_memory_plan.argtypes = [ScheduleP, GraphP]
    lib.lancius_build_memory_plan.restype = PlanP
    lib.lancius_memory_plan_destroy.argtypes = [PlanP]
    lib.lancius_memory_plan_destroy.restype = None
    lib.lancius_get_error.restype = C.c_int
    lib.lancius_clear_error.restype = None
    lib.lancius_graph_load.argtypes = [C.c_char_p]
    lib.lancius_graph_load.restype = GraphP
    lib.lancius_graph_save.argtypes = [GraphP, C.c_char_p]
    lib.lancius_graph_save.restype = None
    lib.lancius_permute.argtypes = [GraphP, NodeP, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32]
    lib.lancius_permute.restype = NodeP
    lib.lancius_matmul_batched.argtypes = [GraphP, NodeP, NodeP]
    lib.lancius_matmul_batched.restype = NodeP
    return lib


def declare_model_io(lib: C.CDLL) -> C.CDLL:
    """Model-file functions of liblancius_graph with no reference
    counterpart (v2 container, mapped loading, CRC-32)."""
    lib.lancius_graph_save_v2.argtypes = [GraphP, C.c_char_p, C.c_int]
    lib.lancius_graph_save_v2.restype = C.c_int
    lib.lancius_graph_load_mapped.argtypes = [C.c_char_p, WeightMapP]
    lib.lancius_graph_load_mapped.restype = GraphP
    lib.lancius_weight_map_free.argtypes = [WeightMapP]
    lib.lancius_weight_map_free.restype = None
    lib.lancius_crc32.argtypes = [C.c_uint32, C.c_void_p, C.c_size_t]
    lib.lancius_crc32.restype = C.c_uint32
    return lib


def set_graph_dtype(g: GraphP, dtype: int) -> None:
    """Mark every node with `dtype` (the planner sizes blocks by dtype)."""
    for i in range(g.contents.node_count):
        n = g.contents.nodes[i]
        n.contents.dtype = dtype
        if n.contents.rt:
            n.contents.rt.contents.dtype = dtype


def schedule_waves(s: ScheduleP) -> list[list[int]]:
    return [[s.contents.waves[w].nodes[i].contents.id for i in range(s.contents.waves[w].node_count)]
            for w in range(s.contents.wave_count)]


def plan_offsets(plan: PlanP, ids: int) -> tuple[int, list[int], list[int]]:
    p = plan.contents
    return p.peak_memory, [p.offsets[i] for i in range(ids)], [p.is_pooled[i] for i in range(ids)]
