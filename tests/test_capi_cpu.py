"""The C ABI without a GPU: libadi_hip.so loads, exports every entry point
include/adi_hip.h declares, its struct layouts match the ctypes mirror, and a
context cannot be created where there is no gfx950 device (the error path
returns a status and a message rather than crashing)."""
import ctypes as C
import os
import re
import subprocess

import pytest

from adi_amd import hip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "adi_hip.h")
HEADERS = [HEADER, os.path.join(ROOT, "include", "adi_hip_gguf.h")]

STRUCTS = {
    "adi_hip_expert_matrix": hip.ExpertMatrix,
    "adi_hip_ne_matrix": hip.NeMatrix,
    "adi_hip_head_chunk": hip.HeadChunk,
    "adi_hip_bf16_matrix": hip.Bf16Matrix,
    "adi_hip_expert_stack": hip.ExpertStack,
    "adi_hip_moe_layer": hip.MoeLayer,
    "adi_hip_kernel_profile": hip.KernelProfile,
    "adi_hip_embedding": hip.Embedding,
    "adi_hip_gguf_tensor": hip.GgufTensor,
    "adi_hip_moe_geometry": hip.MoeGeometry,
    "adi_hip_full_attention": hip.FullAttentionStruct,
    "adi_hip_linear_attention": hip.LinearAttentionStruct,
    "adi_hip_decoder_layer": hip.DecoderLayerStruct,
    "adi_hip_layer_state": hip.LayerState,
    "adi_hip_model": hip.ModelStruct,
    "adi_hip_decoder_state": hip.DecoderStateStruct,
}


def declared_functions():
    text = "".join(open(h).read() for h in HEADERS)
    return sorted(set(re.findall(r"^\s*(?:int|void|uint32_t|uint64_t|const char \*)\s*(adi_hip_\w+)\s*\(",
                                 text, re.M)))


def test_library_exports_every_declared_symbol():
    lib = hip.load()
    names = declared_functions()
    assert len(names) >= 25
    for name in names:
        assert hasattr(lib, name), f"{name} is declared but not exported"
    bound = {n for n, _, _ in hip.SIGNATURES}
    assert bound == set(names), "ctypes bindings and header disagree"
    nm = subprocess.run(["nm", "-D", "--defined-only", hip.LIBRARY], capture_output=True, text=True,
                        check=True).stdout
    exported = set(re.findall(r"\s[TW]\s(adi_hip_\w+)$", nm, re.M))
    assert exported == set(names), "library exports undeclared adi_hip_* symbols"


def test_struct_layouts_match_header(tmp_path):
    lines = ["#include <stdio.h>", "#include <stddef.h>", '#include "adi_hip_gguf.h"', "int main(void) {"]
    for cname, ctype in STRUCTS.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for field, _ in ctype._fields_:
            lines.append(f'printf("{cname} {field} %zu\\n", offsetof({cname}, {field}));')
    lines += ["return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", "-I", os.path.dirname(HEADER), str(src),
                    "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split("\n")
    want = {}
    for line in filter(None, out):
        cname, field, value = line.split()
        want[(cname, field)] = int(value)
    for cname, ctype in STRUCTS.items():
        assert want[(cname, "size")] == C.sizeof(ctype), cname
        for field, _ in ctype._fields_:
            assert want[(cname, field)] == getattr(ctype, field).offset, (cname, field)


def test_header_compiles_as_cpp(tmp_path):
    src = tmp_path / "use.cpp"
    src.write_text('#include "adi_hip_gguf.h"\nint main() { adi_hip_context *c = nullptr; '
                   'return adi_hip_set_reduction_isa(c, 16) == ADI_HIP_INVALID_ARGUMENT ? 0 : 1; }\n')
    subprocess.run(["g++", "-std=c++17", "-fsyntax-only", "-Wall", "-Werror", "-I",
                    os.path.dirname(HEADER), str(src)], check=True)


def test_no_device_is_an_error_not_a_crash():
    torch = pytest.importorskip("torch")
    if torch.cuda.is_available():
        pytest.skip("a GPU is present; the GPU suite covers context creation")
    lib = hip.load()
    handle = C.c_void_p()
    status = lib.adi_hip_context_create(0, C.byref(handle))
    assert status == hip.INVALID_ARGUMENT
    assert handle.value is None
    assert b"device" in lib.adi_hip_last_error(None)
    # every entry point rejects a null context without touching a device
    assert lib.adi_hip_set_reduction_isa(None, 16) == hip.INVALID_ARGUMENT
    assert lib.adi_hip_expert_matmul(None, None, None, 1, None) == hip.INVALID_ARGUMENT


def test_backend_library_exports_the_driver():
    """Where the reference is present, its runtime linked with hip_backend()
    loads on a host without a GPU (the table is created on first use)."""
    import backend_binding as bb
    if not bb.available():
        pytest.skip("oracle/_ref/libadi_backend.so is not built here")
    lib = bb.load()
    for name in ("bd_backend_name", "bd_expert_matmul", "bd_ne_matmul", "bd_head_matmul",
                 "bd_bf16_matmul", "bd_rms_norm"):
        assert hasattr(lib, name)
    assert bb.name(bb.CPU) in ("scalar", "avx2", "avx512")


def test_status_codes_are_distinct_and_mirrored():
    """Every ADI_HIP_* status a call can return has its own value, and the
    ctypes mirror carries the same numbers, so a caller can tell them apart."""
    text = "".join(open(h).read() for h in HEADERS)
    codes = dict(re.findall(r"^#define ADI_HIP_(OK|[A-Z_]+_(?:ARGUMENT|MEMORY|ERROR|RANGE|FOUND))\s+\(?(-?\d+)\)?",
                            text, re.M))
    assert set(codes) == {"OK", "INVALID_ARGUMENT", "OUT_OF_MEMORY", "DEVICE_ERROR", "OUT_OF_RANGE", "NOT_FOUND"}
    values = {int(v) for v in codes.values()}
    assert len(values) == len(codes), f"status codes collide: {codes}"
    for name, value in codes.items():
        assert getattr(hip, name) == int(value), name
