"""The C-ABI boundary without a GPU: the libraries load, export every symbol
their headers declare, keep C++ out of the public headers, and the struct
layout of include/lancius_abi.h is the reference's."""
import ctypes as C
import re
import subprocess
from pathlib import Path

import pytest

from lancius_amd import runtime

ROOT = Path(__file__).resolve().parents[1]
INCLUDE = ROOT / "include"
REF_INCLUDE = Path("/root/reference/bleeding/v11A1/include")


def _declared(header: Path, marker: str | None = None) -> set[str]:
    text = header.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = set()
    for m in re.finditer(r"(?:^|\n)\s*(?:LANCIUS_(?:HIP|BASIS)_EXPORT\s+)?[A-Za-z_][\w\s\*]*?\b([a-z_][a-z0-9_]*)\s*\(",
                         text):
        line = m.group(0)
        if "typedef" in line or "#define" in line or "static inline" in line:
            continue
        if marker and marker not in line:
            continue
        names.add(m.group(1))
    return names


def _hip_declared() -> set[str]:
    return (_declared(INCLUDE / "lancius_hip.h", "LANCIUS_HIP_EXPORT")
            | _declared(INCLUDE / "lancius_hip_graph.h", "LANCIUS_HIP_EXPORT")
            | _declared(INCLUDE / "lancius_basis.h", "LANCIUS_BASIS_EXPORT"))


def test_hip_library_exports_every_declared_symbol():
    lib = C.CDLL(str(runtime.HIP_LIB))
    names = _hip_declared()
    assert {"lancius_hip_gemm_f32", "lancius_hip_attention_f32", "lancius_hip_conv2d_f32", "kernel_matmul_f32",
            "lancius_device_program_create", "lancius_schedule_execute_device", "basis_arena_create",
            "basis_pool_free", "lancius_basis_program_run"} <= names
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert missing == []


def test_hip_library_exports_nothing_else():
    out = subprocess.run(["nm", "-D", "--defined-only", str(runtime.HIP_LIB)], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert sorted(n for n in exported if n not in _hip_declared() and not n.startswith("_")) == []


def test_graph_library_exports_every_declared_symbol():
    lib = C.CDLL(str(runtime.GRAPH_LIB))
    names = _declared(INCLUDE / "lancius_graph.h")
    assert "lancius_build_memory_plan" in names and "lancius_ir_schedule" in names
    assert [n for n in sorted(names) if not hasattr(lib, n)] == []
    # the BASIS builders (the lancius_basis.h declarations without the export marker)
    basis = _declared(INCLUDE / "lancius_basis.h") - _declared(INCLUDE / "lancius_basis.h", "LANCIUS_BASIS_EXPORT")
    assert {"basis_graph_new", "basis_graph_matmul", "basis_graph_print", "basis_graph_free"} <= basis
    assert [n for n in sorted(basis) if not hasattr(lib, n)] == []


def test_no_gpu_call_needed_to_load():
    lib = runtime.hip_lib()
    assert isinstance(lib.lancius_hip_device_count(), int)


@pytest.mark.parametrize("header", ["lancius_hip.h", "lancius_hip_graph.h", "lancius_graph.h", "lancius_abi.h",
                                    "lancius_basis.h"])
def test_public_headers_are_c(tmp_path, header):
    src = tmp_path / "t.c"
    src.write_text(f'#include "{header}"\nint main(void) {{ return 0; }}\n')
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", "-pedantic", f"-I{INCLUDE}", "-c", str(src), "-o",
                    str(tmp_path / "t.o")], check=True)


LAYOUT_PROBE = r"""
#include <stdio.h>
#include <stddef.h>
%(includes)s
#define F(T, f) printf(#T "." #f " %%zu %%zu\n", offsetof(T, f), sizeof(((T*)0)->f))
int main(void) {
    F(lancius_node, id); F(lancius_node, op); F(lancius_node, shape); F(lancius_node, ndim);
    F(lancius_node, kernel_h); F(lancius_node, kernel_w); F(lancius_node, stride); F(lancius_node, pad);
    F(lancius_node, axes); F(lancius_node, inputs); F(lancius_node, input_count); F(lancius_node, attr_val);
    F(lancius_node, runtime_data); F(lancius_node, dtype); F(lancius_node, scale);
    F(lancius_node, runtime_data_int8); F(lancius_node, rt); F(lancius_node, is_view); F(lancius_node, strides);
    F(lancius_node, view_source);
    F(lancius_graph, arena); F(lancius_graph, nodes); F(lancius_graph, node_count); F(lancius_graph, node_cap);
    F(lancius_graph, next_id); F(lancius_graph, rt_states); F(lancius_graph, rt_cap);
    F(lancius_runtime_state, buffer); F(lancius_runtime_state, buffer_int8); F(lancius_runtime_state, dtype);
    F(lancius_runtime_state, scale); F(lancius_runtime_state, owner); F(lancius_runtime_state, buffer_owner);
    F(lancius_runtime_state, int8_owner); F(lancius_runtime_state, offset); F(lancius_runtime_state, flags);
    F(lancius_wave, nodes); F(lancius_wave, node_count);
    F(lancius_schedule, waves); F(lancius_schedule, wave_count); F(lancius_schedule, plan);
    F(lancius_schedule, static_pool);
    F(lancius_memory_plan, peak_memory); F(lancius_memory_plan, offsets); F(lancius_memory_plan, is_pooled);
    printf("sizes %%zu %%zu %%zu %%zu %%zu\n", sizeof(lancius_node), sizeof(lancius_graph),
           sizeof(lancius_runtime_state), sizeof(lancius_schedule), sizeof(lancius_memory_plan));
    printf("ops %%d %%d %%d %%d %%d %%d %%d\n", LANCIUS_OP_MATMUL, LANCIUS_OP_CONV2D_RELU_FUSED, LANCIUS_OP_RESHAPE,
           LANCIUS_OP_LAYERNORM, LANCIUS_OP_GELU, LANCIUS_OP_ATTENTION, LANCIUS_OP_GQA);
    printf("dtype %%d %%d\n", LANCIUS_DTYPE_FP32, LANCIUS_DTYPE_INT32);
    return 0;
}
"""


def _layout(tmp_path, includes: str, incdir: Path, tag: str) -> str:
    src = tmp_path / f"{tag}.c"
    src.write_text(LAYOUT_PROBE % {"includes": includes})
    exe = tmp_path / tag
    subprocess.run(["gcc", "-std=gnu11", f"-I{incdir}", str(src), "-o", str(exe)], check=True)
    return subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout


@pytest.mark.skipif(not REF_INCLUDE.is_dir(), reason="reference headers are only present in the build container")
def test_struct_layout_matches_reference_headers(tmp_path):
    ref = _layout(tmp_path, '#include "lancius/lancius_ir.h"\n#include "lancius/lancius_scheduler.h"\n'
                            '#include "lancius/lancius_memory_planner.h"', REF_INCLUDE, "ref")
    ours = _layout(tmp_path, '#include "lancius_abi.h"', INCLUDE, "ours")
    assert ours == ref


@pytest.mark.skipif(not REF_INCLUDE.is_dir(), reason="reference headers are only present in the build container")
def test_abi_header_coexists_with_reference_headers(tmp_path):
    src = tmp_path / "both.c"
    src.write_text('#include "lancius/lancius_ir.h"\n#include "lancius/lancius_scheduler.h"\n'
                   '#include "lancius/lancius_memory_planner.h"\n#include "lancius_hip_graph.h"\n'
                   'int main(void) { return 0; }\n')
    subprocess.run(["gcc", "-std=gnu11", f"-I{REF_INCLUDE}", f"-I{INCLUDE}", "-c", str(src), "-o",
                    str(tmp_path / "both.o")], check=True)


def test_python_mirror_matches_c_layout(tmp_path):
    from lancius_amd import abi

    text = _layout(tmp_path, '#include "lancius_abi.h"', INCLUDE, "mirror")
    off = {}
    for line in text.splitlines():
        parts = line.split()
        if "." in parts[0]:
            off[parts[0]] = int(parts[1])
    for cname, py in (("lancius_node", abi.Node), ("lancius_graph", abi.Graph),
                      ("lancius_runtime_state", abi.RuntimeState), ("lancius_schedule", abi.Schedule),
                      ("lancius_memory_plan", abi.MemoryPlan)):
        for field, _ in py._fields_:
            assert getattr(py, field).offset == off[f"{cname}.{field}"], (cname, field)
    sizes = [int(x) for x in text.split("sizes")[1].split()[:5]]
    assert sizes == [C.sizeof(abi.Node), C.sizeof(abi.Graph), C.sizeof(abi.RuntimeState), C.sizeof(abi.Schedule),
                     C.sizeof(abi.MemoryPlan)]


BASIS_INCLUDE = Path("/root/reference/include")

BASIS_PROBE = r"""
#include <stdio.h>
#include <stddef.h>
%(includes)s
#define F(T, f) printf(#T "." #f " %%zu %%zu\n", offsetof(T, f), sizeof(((T*)0)->f))
int main(void) {
    F(basis_node, id); F(basis_node, op); F(basis_node, input_ids); F(basis_node, rows); F(basis_node, cols);
    F(basis_node, name); F(basis_graph, nodes); F(basis_graph, node_count); F(basis_graph, node_cap);
    printf("sizes %%zu %%zu\n", sizeof(basis_node), sizeof(basis_graph));
    printf("ops %%d %%d %%d %%d %%d %%d\n", BASIS_OP_INPUT, BASIS_OP_MATMUL, BASIS_OP_ADD, BASIS_OP_RELU, BASIS_OP_TANH,
           BASIS_OP_BROADCAST_ADD);
    return 0;
}
"""


def _basis_layout(tmp_path, includes: str, incdirs: list[Path], tag: str) -> str:
    src = tmp_path / f"{tag}.c"
    src.write_text(BASIS_PROBE % {"includes": includes})
    exe = tmp_path / tag
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", *[f"-I{d}" for d in incdirs], str(src), "-o", str(exe)],
                   check=True)
    return subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout


@pytest.mark.skipif(not BASIS_INCLUDE.is_dir(), reason="reference headers are only present in the build container")
def test_basis_layout_matches_reference_headers(tmp_path):
    """include/basis/stage6_ir/graph.h:7-39 and include/basis/core/memory.h:
    same layouts and enum values, and either header order compiles."""
    ref = _basis_layout(tmp_path, '#include "basis/stage6_ir/graph.h"\n#include "basis/core/memory.h"',
                        [BASIS_INCLUDE], "ref")
    ours = _basis_layout(tmp_path, '#include "lancius_basis.h"', [INCLUDE], "ours")
    assert ours == ref
    for order, tag in ((('"lancius_basis.h"', '"basis/stage6_ir/graph.h"', '"basis/core/memory.h"'), "a"),
                       (('"basis/stage6_ir/graph.h"', '"basis/core/memory.h"', '"lancius_basis.h"'), "b")):
        both = _basis_layout(tmp_path, "\n".join(f"#include {h}" for h in order), [INCLUDE, BASIS_INCLUDE], tag)
        assert both == ref
