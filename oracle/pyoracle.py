"""ctypes bindings for the CPU checkers (TEST INFRASTRUCTURE ONLY).

`liboracle.so` is the C restatement in adi_oracle.c; `_ref/libadi_ref.so` is
the reference's own CPU path compiled from its sources (optional: present only
where it was built). Only tests, the smoke check and the benchmark's
CPU-baseline leg use this module; the product path never does.
"""
from __future__ import annotations

import ctypes as C
import os
from typing import Optional

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# ADI_ORACLE_LIBRARY names another build of the oracle (the sanitizer build
# of tests/sanitize.sh); by default the in-tree one.
ORACLE_PATH = os.environ.get("ADI_ORACLE_LIBRARY") or os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libadi_ref.so")

u16p = C.POINTER(C.c_uint16)
u32p = C.POINTER(C.c_uint32)
f32p = C.POINTER(C.c_float)
i8p = C.POINTER(C.c_int8)
u8p = C.POINTER(C.c_uint8)


class ExpertMatrix(C.Structure):
    _fields_ = [
        ("rows", C.c_uint32), ("columns", C.c_uint32),
        ("trellis", u16p), ("su_f16", u16p), ("sv_f16", u16p),
        ("wave_gamma_f16", u16p), ("tlut", f32p), ("state_values", f32p),
    ]


class NeMatrix(C.Structure):
    _fields_ = [
        ("rows", C.c_uint32), ("columns", C.c_uint32),
        ("trellis", u16p), ("su", i8p), ("sv", i8p),
        ("weight_scale", C.c_float), ("tlut", f32p), ("state_values", f32p),
    ]


class HeadChunk(C.Structure):
    _fields_ = [
        ("rows", C.c_uint32), ("columns", C.c_uint32),
        ("packed", u8p), ("group_scale_f16", u16p),
        ("protected_rows", u32p), ("protected_bf16", u16p),
        ("protected_count", C.c_uint32),
    ]


class Bf16Matrix(C.Structure):
    _fields_ = [("rows", C.c_uint32), ("columns", C.c_uint32), ("values", u16p)]


class Embedding(C.Structure):
    _fields_ = [
        ("rows", C.c_uint32), ("columns", C.c_uint32), ("packed", u8p),
        ("minimum_f16", u16p), ("maximum_f16", u16p), ("exception_indexes", u32p),
        ("exception_bf16", u16p), ("exception_count", C.c_uint32),
    ]


class MoeLayer(C.Structure):
    _fields_ = [
        ("hidden", C.c_uint32), ("expert_hidden", C.c_uint32), ("experts", C.c_uint32),
        ("router", Bf16Matrix), ("shared_expert_gate", Bf16Matrix),
        ("expert_matrices", C.POINTER(ExpertMatrix)),
        ("shared_gate", NeMatrix), ("shared_up", NeMatrix), ("shared_down", NeMatrix),
    ]


class FullAttention(C.Structure):
    _fields_ = [("query", NeMatrix), ("key", NeMatrix), ("value", NeMatrix), ("output", NeMatrix),
                ("query_norm", C.POINTER(C.c_uint16)), ("key_norm", C.POINTER(C.c_uint16))]


class LinearAttention(C.Structure):
    _fields_ = [("qkv", NeMatrix), ("gate", NeMatrix), ("output", NeMatrix),
                ("alpha", Bf16Matrix), ("beta", Bf16Matrix),
                ("convolution", C.POINTER(C.c_uint16)), ("alpha_bias", C.POINTER(C.c_uint16)),
                ("a_log", C.POINTER(C.c_uint16)), ("norm", C.POINTER(C.c_uint16))]


class DecoderLayer(C.Structure):
    _fields_ = [("input_norm", C.POINTER(C.c_uint16)), ("post_attention_norm", C.POINTER(C.c_uint16)),
                ("full_attention", C.c_int), ("full", FullAttention), ("linear", LinearAttention),
                ("moe", MoeLayer)]


def ptr(array: Optional[np.ndarray], ctype):
    if array is None:
        return C.cast(None, C.POINTER(ctype))
    assert array.flags["C_CONTIGUOUS"], "oracle arrays must be contiguous"
    return array.ctypes.data_as(C.POINTER(ctype))


def _declare(lib, name, restype, *argtypes):
    fn = getattr(lib, name)
    fn.restype = restype
    fn.argtypes = list(argtypes)
    return fn


class _Common:
    """Signatures shared by the oracle (ao_*) and the reference shim (ref_*)."""


def load_oracle() -> C.CDLL:
    if not os.path.exists(ORACLE_PATH):
        raise RuntimeError(f"{ORACLE_PATH} is not built; run `make -C oracle`")
    lib = C.CDLL(ORACLE_PATH)
    _declare(lib, "ao_f16_to_f32", C.c_float, C.c_uint16)
    _declare(lib, "ao_f32_to_f16", C.c_uint16, C.c_float)
    _declare(lib, "ao_bf16_to_f32", C.c_float, C.c_uint16)
    _declare(lib, "ao_expert_tile_states", None, u16p, u16p)
    _declare(lib, "ao_ne_tile_states", None, u16p, u16p)
    _declare(lib, "ao_build_expert_state_values", None, f32p, f32p)
    _declare(lib, "ao_build_ne_state_values", None, f32p, f32p)
    _declare(lib, "ao_build_ne_signed_tlut", None, f32p, f32p)
    _declare(lib, "ao_build_wave_indexes", C.c_int, C.c_uint32, C.c_uint32, u16p)
    _declare(lib, "ao_hadamard", C.c_int, f32p, C.c_uint32)
    _declare(lib, "ao_expert_decode_tiles", C.c_int, C.POINTER(ExpertMatrix), f32p)
    _declare(lib, "ao_ne_decode_tiles", C.c_int, C.POINTER(NeMatrix), f32p)
    _declare(lib, "ao_expert_matmul", C.c_int, C.POINTER(ExpertMatrix), f32p, C.c_uint32, f32p)
    _declare(lib, "ao_ne_matmul", C.c_int, C.POINTER(NeMatrix), f32p, C.c_uint32, f32p)
    _declare(lib, "ao_expert_accumulate", C.c_int, C.POINTER(ExpertMatrix), f32p, C.c_uint32, f32p)
    _declare(lib, "ao_ne_accumulate", C.c_int, C.POINTER(NeMatrix), f32p, C.c_uint32, f32p)
    _declare(lib, "ao_head_matmul", C.c_int, C.POINTER(HeadChunk), f32p, C.c_uint32, f32p, C.c_uint32)
    _declare(lib, "ao_bf16_dot", C.c_float, u16p, f32p, C.c_uint32, C.c_uint32)
    _declare(lib, "ao_bf16_matmul", C.c_int, C.POINTER(Bf16Matrix), f32p, C.c_uint32, f32p, C.c_uint32)
    _declare(lib, "ao_rms_norm", C.c_int, f32p, u16p, C.c_uint32, C.c_float, C.c_float, f32p)
    _declare(lib, "ao_silu", C.c_float, C.c_float)
    _declare(lib, "ao_sigmoid", C.c_float, C.c_float)
    _declare(lib, "ao_top_experts", C.c_int, f32p, C.c_uint32, u32p, f32p)
    _declare(lib, "ao_moe_route", C.c_int, f32p, C.c_uint32, C.c_uint32, u32p, f32p,
             u32p, u32p, u32p, u32p)
    _declare(lib, "ao_moe_forward", C.c_int, C.POINTER(MoeLayer), f32p, C.c_uint32, f32p,
             C.c_uint32, f32p, u32p, f32p, C.c_int)
    _declare(lib, "ao_embedding_row", C.c_int, C.POINTER(Embedding), C.c_uint32, f32p)
    _declare(lib, "ao_argmax", C.c_uint32, f32p, C.c_uint32)
    _declare(lib, "ao_fnv1a64", C.c_uint64, C.c_uint64, C.c_void_p, C.c_size_t)
    _declare(lib, "ao_sample_token", C.c_int, f32p, C.c_uint32, C.c_float, C.c_float, C.c_uint64, u32p)
    _declare(lib, "ao_mt19937_64", None, C.c_uint64, C.c_uint32, C.POINTER(C.c_uint64))
    _declare(lib, "ao_normalize_head", C.c_int, f32p, u16p, C.c_uint32, C.c_float)
    _declare(lib, "ao_rope_table", None, C.c_uint32, f32p, f32p)
    _declare(lib, "ao_apply_rope", None, f32p, f32p, f32p)
    _declare(lib, "ao_grouped_attention", C.c_int, f32p, f32p, f32p, C.c_uint32, C.c_uint32,
             C.c_uint32, C.c_uint32, C.c_uint32, f32p)
    _declare(lib, "ao_l2_normalize", C.c_int, f32p, C.c_uint32, C.c_float)
    _declare(lib, "ao_gated_delta_update", C.c_float, f32p, f32p, f32p, C.c_float, C.c_float,
             C.c_float, C.c_uint32)
    _declare(lib, "ao_full_attention_forward", C.c_int, C.POINTER(FullAttention), C.c_uint32,
             f32p, f32p, f32p, f32p)
    _declare(lib, "ao_gated_delta_key_head", C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32)
    _declare(lib, "ao_linear_attention_forward", C.c_int, C.POINTER(LinearAttention), f32p, f32p,
             f32p, f32p, C.c_uint32)
    _declare(lib, "ao_decode_layer", C.c_int, C.POINTER(DecoderLayer), C.c_uint32, f32p, f32p,
             f32p, f32p, f32p, C.c_uint32)
    return lib


def ref_available() -> bool:
    return os.path.exists(REF_PATH)


def load_ref() -> C.CDLL:
    if not ref_available():
        raise RuntimeError(f"{REF_PATH} is not built; run `make -C oracle ref`")
    lib = C.CDLL(REF_PATH)
    _declare(lib, "ref_selected_isa_lanes", C.c_int)
    _declare(lib, "ref_force_isa_lanes", None, C.c_int)
    _declare(lib, "ref_avx512_vbmi", C.c_int)
    _declare(lib, "ref_worker_threads", C.c_uint32)
    _declare(lib, "ref_kernel_profiling", None, C.c_int)
    _declare(lib, "ref_kernel_profile", C.c_uint32, C.c_uint32, C.c_char_p, C.c_uint32,
             C.POINTER(C.c_uint64), C.POINTER(C.c_uint64), C.POINTER(C.c_uint64))
    _declare(lib, "ref_f16_to_f32", C.c_float, C.c_uint16)
    _declare(lib, "ref_f32_to_f16", C.c_uint16, C.c_float)
    _declare(lib, "ref_silu", C.c_float, C.c_float)
    _declare(lib, "ref_sigmoid", C.c_float, C.c_float)
    _declare(lib, "ref_expert_tile_states", None, u16p, u16p)
    _declare(lib, "ref_expert_row_states", None, u16p, u16p)
    _declare(lib, "ref_ne_tile_states", None, u16p, u16p)
    _declare(lib, "ref_ne_row_states", None, u16p, u16p)
    _declare(lib, "ref_build_expert_state_values", None, f32p, f32p)
    _declare(lib, "ref_build_ne_state_values", None, f32p, f32p)
    _declare(lib, "ref_build_ne_signed_tlut", None, f32p, f32p)
    _declare(lib, "ref_build_wave_indexes", C.c_int, C.c_uint32, C.c_uint32, u16p)
    _declare(lib, "ref_hadamard", None, f32p, C.c_uint32)
    _declare(lib, "ref_expert_matmul", C.c_int, C.POINTER(ExpertMatrix), f32p, C.c_uint32, f32p)
    _declare(lib, "ref_ne_matmul", C.c_int, C.POINTER(NeMatrix), f32p, C.c_uint32, f32p)
    _declare(lib, "ref_head_matmul", C.c_int, C.POINTER(HeadChunk), f32p, C.c_uint32, f32p)
    _declare(lib, "ref_bf16_matmul", C.c_int, C.POINTER(Bf16Matrix), f32p, C.c_uint32, f32p)
    _declare(lib, "ref_rms_norm", C.c_int, f32p, u16p, C.c_uint32, C.c_float, C.c_float, f32p)
    _declare(lib, "ref_top_experts", C.c_int, f32p, C.c_uint32, u32p, f32p)
    _declare(lib, "ref_moe_layer_create", C.c_void_p, C.POINTER(MoeLayer))
    _declare(lib, "ref_moe_layer_destroy", None, C.c_void_p)
    _declare(lib, "ref_moe_forward", C.c_int, C.c_void_p, f32p, C.c_uint32, f32p, f32p, u32p, f32p)
    _declare(lib, "ref_embedding_row", C.c_int, C.POINTER(Embedding), C.c_uint32, f32p)
    _declare(lib, "ref_sample_token", C.c_int, f32p, C.c_uint32, C.c_float, C.c_float, C.c_uint64,
             C.POINTER(C.c_uint64), u32p)
    _declare(lib, "ref_gguf_summary", C.c_int, C.c_char_p, C.POINTER(C.c_uint64),
             C.POINTER(C.c_uint64), C.POINTER(C.c_uint64))
    _declare(lib, "ref_grouped_attention", C.c_int, f32p, f32p, f32p, C.c_uint32, C.c_uint32,
             C.c_uint32, C.c_uint32, C.c_uint32, f32p)
    _declare(lib, "ref_gated_delta_update", C.c_float, f32p, f32p, f32p, C.c_float, C.c_float,
             C.c_float, C.c_uint32)
    _declare(lib, "ref_l2_normalize", C.c_int, f32p, C.c_uint32, C.c_float)
    return lib


def ref_kernel_profiles(lib) -> dict:
    """The reference's per-kind profile since ref_kernel_profiling(1):
    {kind name: (calls, milliseconds, work items)} for kinds that ran."""
    out = {}
    calls, ns, work = C.c_uint64(), C.c_uint64(), C.c_uint64()
    name = C.create_string_buffer(32)
    count = lib.ref_kernel_profile(0, name, 32, C.byref(calls), C.byref(ns), C.byref(work))
    for kind in range(count):
        lib.ref_kernel_profile(kind, name, 32, C.byref(calls), C.byref(ns), C.byref(work))
        if calls.value:
            out[name.value.decode()] = (int(calls.value), ns.value / 1e6, int(work.value))
    return out


# ---- struct builders over numpy arrays (the caller keeps the arrays alive) --

def expert_struct(m, state_values: Optional[np.ndarray] = None) -> ExpertMatrix:
    return ExpertMatrix(
        m.rows, m.columns, ptr(m.trellis, C.c_uint16), ptr(m.su_f16, C.c_uint16),
        ptr(m.sv_f16, C.c_uint16), ptr(m.wave_gamma_f16, C.c_uint16),
        ptr(m.tlut, C.c_float), ptr(state_values, C.c_float))


def ne_struct(m, state_values: Optional[np.ndarray] = None) -> NeMatrix:
    return NeMatrix(
        m.rows, m.columns, ptr(m.trellis, C.c_uint16), ptr(m.su, C.c_int8),
        ptr(m.sv, C.c_int8), C.c_float(m.weight_scale), ptr(m.tlut, C.c_float),
        ptr(state_values, C.c_float))


def head_struct(h) -> HeadChunk:
    count = 0 if h.protected_rows is None else int(h.protected_rows.size)
    return HeadChunk(
        h.rows, h.columns, ptr(h.packed, C.c_uint8), ptr(h.group_scale_f16, C.c_uint16),
        ptr(h.protected_rows, C.c_uint32), ptr(h.protected_bf16, C.c_uint16), count)


def bf16_struct(values: np.ndarray) -> Bf16Matrix:
    rows, columns = values.shape
    return Bf16Matrix(rows, columns, ptr(values, C.c_uint16))


class MoeLayerStruct:
    """Holds a MoeLayer struct and the arrays/structs it points into."""

    def __init__(self, layer):
        self.layer = layer
        experts = layer.experts
        self._experts = (ExpertMatrix * (experts * 3))()
        for e in range(experts):
            for p, m in enumerate((layer.gate[e], layer.up[e], layer.down[e])):
                self._experts[e * 3 + p] = expert_struct(m)
        self.struct = MoeLayer(
            layer.hidden, layer.expert_hidden, experts,
            bf16_struct(layer.router_bf16), bf16_struct(layer.shared_expert_gate_bf16),
            C.cast(self._experts, C.POINTER(ExpertMatrix)),
            ne_struct(layer.shared_gate), ne_struct(layer.shared_up), ne_struct(layer.shared_down))


# ---- numpy-level helpers ----------------------------------------------------

def check(status: int, what: str) -> None:
    if status != 0:
        raise ValueError(f"{what} failed with status {status}")


def expert_matmul(lib, m, inputs: np.ndarray, prefix="ao") -> np.ndarray:
    inputs = np.ascontiguousarray(inputs, dtype=np.float32).reshape(-1, m.columns)
    out = np.zeros((inputs.shape[0], m.rows), np.float32)
    s = expert_struct(m)
    check(getattr(lib, f"{prefix}_expert_matmul")(C.byref(s), ptr(inputs, C.c_float),
                                                  inputs.shape[0], ptr(out, C.c_float)),
          "expert_matmul")
    return out


def ne_matmul(lib, m, inputs: np.ndarray, prefix="ao") -> np.ndarray:
    inputs = np.ascontiguousarray(inputs, dtype=np.float32).reshape(-1, m.columns)
    out = np.zeros((inputs.shape[0], m.rows), np.float32)
    s = ne_struct(m)
    check(getattr(lib, f"{prefix}_ne_matmul")(C.byref(s), ptr(inputs, C.c_float),
                                              inputs.shape[0], ptr(out, C.c_float)),
          "ne_matmul")
    return out


def head_matmul(lib, h, inputs: np.ndarray, isa: int = 16, prefix="ao") -> np.ndarray:
    inputs = np.ascontiguousarray(inputs, dtype=np.float32).reshape(-1, h.columns)
    out = np.zeros((inputs.shape[0], h.rows), np.float32)
    s = head_struct(h)
    if prefix == "ao":
        status = lib.ao_head_matmul(C.byref(s), ptr(inputs, C.c_float), inputs.shape[0],
                                    ptr(out, C.c_float), isa)
    else:
        status = lib.ref_head_matmul(C.byref(s), ptr(inputs, C.c_float), inputs.shape[0],
                                     ptr(out, C.c_float))
    check(status, "head_matmul")
    return out


def bf16_matmul(lib, values: np.ndarray, inputs: np.ndarray, isa: int = 16,
                prefix="ao") -> np.ndarray:
    rows, columns = values.shape
    inputs = np.ascontiguousarray(inputs, dtype=np.float32).reshape(-1, columns)
    out = np.zeros((inputs.shape[0], rows), np.float32)
    s = bf16_struct(np.ascontiguousarray(values))
    if prefix == "ao":
        status = lib.ao_bf16_matmul(C.byref(s), ptr(inputs, C.c_float), inputs.shape[0],
                                    ptr(out, C.c_float), isa)
    else:
        status = lib.ref_bf16_matmul(C.byref(s), ptr(inputs, C.c_float), inputs.shape[0],
                                     ptr(out, C.c_float))
    check(status, "bf16_matmul")
    return out


def embedding_struct(e) -> Embedding:
    """e: adi_amd.synthetic.Embedding (arrays kept alive by the caller)."""
    return Embedding(e.rows, e.columns, ptr(e.packed, C.c_uint8), ptr(e.minimum_f16, C.c_uint16),
                     ptr(e.maximum_f16, C.c_uint16), ptr(e.exception_indexes, C.c_uint32),
                     ptr(e.exception_bf16, C.c_uint16), int(e.exception_indexes.size))


def embedding_rows(lib, e, tokens, prefix="ao") -> np.ndarray:
    out = np.zeros((len(tokens), e.columns), np.float32)
    s = embedding_struct(e)
    fn = getattr(lib, f"{prefix}_embedding_row")
    for i, t in enumerate(tokens):
        row = np.zeros(e.columns, np.float32)
        check(fn(C.byref(s), int(t), ptr(row, C.c_float)), "embedding_row")
        out[i] = row
    return out


def ref_sample_token(lib, logits: np.ndarray, temperature: float, top_p: float, seed: int):
    """(token, the engine's first 64-bit word) of the compiled sample_token."""
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    word = C.c_uint64()
    token = np.zeros(1, np.uint32)
    check(lib.ref_sample_token(ptr(logits, C.c_float), logits.size, temperature, top_p, seed,
                               C.byref(word), ptr(token, C.c_uint32)), "sample_token")
    return int(token[0]), word.value


def sample_token(lib, logits: np.ndarray, temperature: float, top_p: float, word: int) -> int:
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    token = np.zeros(1, np.uint32)
    check(lib.ao_sample_token(ptr(logits, C.c_float), logits.size, temperature, top_p, word,
                              ptr(token, C.c_uint32)), "sample_token")
    return int(token[0])


def mt19937_64(lib, seed: int, count: int) -> list:
    """The first `count` outputs of std::mt19937_64(seed)."""
    out = (C.c_uint64 * max(count, 1))()
    lib.ao_mt19937_64(seed, count, out)
    return [int(v) for v in out[:count]]


def ref_gguf_summary(lib, path: str):
    """(tensors, metadata, alignment) as the reference's GgufFile reads the
    file, or None when it rejects it."""
    t, m, a = C.c_uint64(), C.c_uint64(), C.c_uint64()
    if lib.ref_gguf_summary(os.fsencode(path), C.byref(t), C.byref(m), C.byref(a)) != 0:
        return None
    return t.value, m.value, a.value


def top_experts(lib, logits: np.ndarray, prefix="ao"):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    experts = np.zeros(8, np.uint32)
    weights = np.zeros(8, np.float32)
    check(getattr(lib, f"{prefix}_top_experts")(ptr(logits, C.c_float), logits.size,
                                                ptr(experts, C.c_uint32),
                                                ptr(weights, C.c_float)), "top_experts")
    return experts, weights


def moe_route(lib, logits: np.ndarray):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    batch, experts = logits.shape
    out = dict(
        route_expert=np.zeros(batch * 8, np.uint32),
        route_weight=np.zeros(batch * 8, np.float32),
        counts=np.zeros(experts, np.uint32),
        offsets=np.zeros(experts + 1, np.uint32),
        grouped_batch=np.zeros(batch * 8, np.uint32),
        route_to_grouped=np.zeros(batch * 8, np.uint32),
    )
    check(lib.ao_moe_route(ptr(logits, C.c_float), batch, experts,
                           ptr(out["route_expert"], C.c_uint32), ptr(out["route_weight"], C.c_float),
                           ptr(out["counts"], C.c_uint32), ptr(out["offsets"], C.c_uint32),
                           ptr(out["grouped_batch"], C.c_uint32),
                           ptr(out["route_to_grouped"], C.c_uint32)), "moe_route")
    return out


def moe_forward(lib, layer, inputs: np.ndarray, isa: int = 16,
                logit_bias: Optional[np.ndarray] = None, threads: int = 0):
    inputs = np.ascontiguousarray(inputs, dtype=np.float32).reshape(-1, layer.hidden)
    batch = inputs.shape[0]
    out = np.zeros((batch, layer.hidden), np.float32)
    route_expert = np.zeros(batch * 8, np.uint32)
    route_weight = np.zeros(batch * 8, np.float32)
    holder = MoeLayerStruct(layer)
    bias = None if logit_bias is None else np.ascontiguousarray(logit_bias, np.float32)
    check(lib.ao_moe_forward(C.byref(holder.struct), ptr(inputs, C.c_float), batch,
                             ptr(bias, C.c_float), isa, ptr(out, C.c_float),
                             ptr(route_expert, C.c_uint32), ptr(route_weight, C.c_float),
                             threads), "moe_forward")
    return out, route_expert.reshape(batch, 8), route_weight.reshape(batch, 8)


class RefMoeLayer:
    """A layer prepared inside the reference library (its codec caches built
    once, as the model does at load)."""

    def __init__(self, ref_lib, layer):
        self.lib = ref_lib
        self.layer = layer
        self.holder = MoeLayerStruct(layer)
        self.handle = ref_lib.ref_moe_layer_create(C.byref(self.holder.struct))
        if not self.handle:
            raise RuntimeError("reference MoE layer preparation failed")

    def forward(self, inputs: np.ndarray, logit_bias: Optional[np.ndarray] = None,
                out: Optional[np.ndarray] = None):
        inputs = np.ascontiguousarray(inputs, dtype=np.float32).reshape(-1, self.layer.hidden)
        batch = inputs.shape[0]
        if out is None:
            out = np.zeros((batch, self.layer.hidden), np.float32)
        route_expert = np.zeros(batch * 8, np.uint32)
        route_weight = np.zeros(batch * 8, np.float32)
        bias = None if logit_bias is None else np.ascontiguousarray(logit_bias, np.float32)
        check(self.lib.ref_moe_forward(self.handle, ptr(inputs, C.c_float), batch,
                                       ptr(bias, C.c_float), ptr(out, C.c_float),
                                       ptr(route_expert, C.c_uint32),
                                       ptr(route_weight, C.c_float)), "ref_moe_forward")
        return out, route_expert.reshape(batch, 8), route_weight.reshape(batch, 8)

    def close(self):
        if self.handle:
            self.lib.ref_moe_layer_destroy(self.handle)
            self.handle = None

    def __del__(self):
        self.close()


# ---- attention of one decode token -----------------------------------------

class FullAttentionStruct:
    """Holds an ao_full_attention over a synthetic.FullAttention."""

    def __init__(self, layer):
        self.layer = layer
        self.struct = FullAttention(ne_struct(layer.query), ne_struct(layer.key),
                                    ne_struct(layer.value), ne_struct(layer.output),
                                    ptr(layer.query_norm, C.c_uint16), ptr(layer.key_norm, C.c_uint16))


class LinearAttentionStruct:
    """Holds an ao_linear_attention over a synthetic.LinearAttention."""

    def __init__(self, layer):
        self.layer = layer
        self.struct = LinearAttention(
            ne_struct(layer.qkv), ne_struct(layer.gate), ne_struct(layer.output),
            bf16_struct(layer.alpha), bf16_struct(layer.beta),
            ptr(layer.convolution, C.c_uint16), ptr(layer.alpha_bias, C.c_uint16),
            ptr(layer.a_log, C.c_uint16), ptr(layer.norm, C.c_uint16))


def full_attention_forward(lib, held: FullAttentionStruct, position: int, x: np.ndarray,
                           keys: np.ndarray, values: np.ndarray) -> np.ndarray:
    """keys/values: float32 [capacity, 2, 256], entry `position` is written."""
    out = np.zeros(held.layer.hidden, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    check(lib.ao_full_attention_forward(C.byref(held.struct), position, ptr(x, C.c_float),
                                        ptr(out, C.c_float), ptr(keys, C.c_float),
                                        ptr(values, C.c_float)), "ao_full_attention_forward")
    return out


def linear_attention_forward(lib, held: LinearAttentionStruct, x: np.ndarray,
                             convolution: np.ndarray, recurrent: np.ndarray,
                             isa: int = 16) -> np.ndarray:
    """convolution float32 [8192 * 3], recurrent float32 [32 * 128 * 128],
    updated in place."""
    out = np.zeros(held.layer.hidden, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    check(lib.ao_linear_attention_forward(C.byref(held.struct), ptr(x, C.c_float),
                                          ptr(out, C.c_float), ptr(convolution, C.c_float),
                                          ptr(recurrent, C.c_float), isa),
          "ao_linear_attention_forward")
    return out


def grouped_attention(lib, queries, keys, values, tokens, query_heads, kv_heads, head_size,
                      query_stride, prefix="ao") -> np.ndarray:
    out = np.zeros(query_heads * head_size, np.float32)
    q, k, v = (np.ascontiguousarray(a, np.float32) for a in (queries, keys, values))
    check(getattr(lib, f"{prefix}_grouped_attention")(
        ptr(q, C.c_float), ptr(k, C.c_float), ptr(v, C.c_float), tokens, query_heads, kv_heads,
        head_size, query_stride, ptr(out, C.c_float)), f"{prefix}_grouped_attention")
    return out


class DecoderLayerStruct:
    """Holds an ao_decoder_layer over a synthetic.DecoderLayer and its state
    (keys/values for full attention, convolution/recurrent for linear)."""

    def __init__(self, layer, capacity: int = 0):
        self.layer = layer
        self.moe = MoeLayerStruct(layer.moe)
        self.full = FullAttentionStruct(layer.full) if layer.full is not None else None
        self.linear = LinearAttentionStruct(layer.linear) if layer.linear is not None else None
        self.struct = DecoderLayer(
            ptr(layer.input_norm, C.c_uint16), ptr(layer.post_attention_norm, C.c_uint16),
            int(self.full is not None), self.full.struct if self.full else FullAttention(),
            self.linear.struct if self.linear else LinearAttention(), self.moe.struct)
        self.keys = np.zeros((max(capacity, 1), 2, 256), np.float32)
        self.values = np.zeros_like(self.keys)
        self.convolution = np.zeros(8192 * 3, np.float32)
        self.recurrent = np.zeros(32 * 128 * 128, np.float32)

    def decode(self, lib, position: int, hidden: np.ndarray, isa: int = 16) -> None:
        """hidden: float32 row, updated in place."""
        check(lib.ao_decode_layer(C.byref(self.struct), position, ptr(hidden, C.c_float),
                                  ptr(self.keys, C.c_float), ptr(self.values, C.c_float),
                                  ptr(self.convolution, C.c_float),
                                  ptr(self.recurrent, C.c_float), isa), "ao_decode_layer")
