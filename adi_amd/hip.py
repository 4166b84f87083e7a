"""ctypes binding of libadi_hip.so, the C ABI in include/adi_hip.h and
include/adi_hip_gguf.h.

torch is used only to own device memory and to hand its current stream to the
library; every computation runs in the library's HIP kernels. Loading fails
loudly when the library is not built: there is no fallback path.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass
from typing import Optional

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# ADI_HIP_LIBRARY names another build of the same library (the host-side
# sanitizer build of tests/sanitize.sh); by default the in-tree one.
LIBRARY = os.environ.get("ADI_HIP_LIBRARY") or os.path.join(HERE, "libadi_hip.so")

OK = 0
INVALID_ARGUMENT = -1
OUT_OF_MEMORY = -2
DEVICE_ERROR = -3
OUT_OF_RANGE = -4
NOT_FOUND = -5

GGML_F32, GGML_F16, GGML_I8, GGML_I16, GGML_I32, GGML_I64, GGML_F64, GGML_BF16 = 0, 1, 24, 25, 26, 27, 28, 30

vp = C.c_void_p
u32 = C.c_uint32
u64 = C.c_uint64
f32 = C.c_float


class ExpertMatrix(C.Structure):
    _fields_ = [("rows", u32), ("columns", u32), ("trellis", vp), ("su_f16", vp),
                ("sv_f16", vp), ("wave_gamma_f16", vp), ("codebook", vp)]


class NeMatrix(C.Structure):
    _fields_ = [("rows", u32), ("columns", u32), ("trellis", vp), ("su", vp), ("sv", vp),
                ("weight_scale", f32), ("codebook", vp)]


class HeadChunk(C.Structure):
    _fields_ = [("rows", u32), ("columns", u32), ("packed", vp), ("group_scale_f16", vp),
                ("protected_rows", vp), ("protected_bf16", vp), ("protected_count", u32)]


class Bf16Matrix(C.Structure):
    _fields_ = [("rows", u32), ("columns", u32), ("values", vp)]


class Embedding(C.Structure):
    _fields_ = [("rows", u32), ("columns", u32), ("packed", vp), ("minimum_f16", vp),
                ("maximum_f16", vp), ("exception_indexes", vp), ("exception_bf16", vp),
                ("exception_count", u32)]


class ExpertStack(C.Structure):
    _fields_ = [("trellis", vp), ("su_f16", vp), ("sv_f16", vp), ("wave_gamma_f16", vp)]


class MoeLayer(C.Structure):
    _fields_ = [("hidden", u32), ("expert_hidden", u32), ("experts", u32),
                ("router", Bf16Matrix), ("shared_expert_gate", Bf16Matrix),
                ("gate", ExpertStack), ("up", ExpertStack), ("down", ExpertStack),
                ("expert_codebook", vp),
                ("shared_gate", NeMatrix), ("shared_up", NeMatrix), ("shared_down", NeMatrix)]


class FullAttentionStruct(C.Structure):
    _fields_ = [("query", NeMatrix), ("key", NeMatrix), ("value", NeMatrix), ("output", NeMatrix),
                ("query_norm", C.c_void_p), ("key_norm", C.c_void_p)]


class LinearAttentionStruct(C.Structure):
    _fields_ = [("qkv", NeMatrix), ("gate", NeMatrix), ("output", NeMatrix),
                ("alpha", Bf16Matrix), ("beta", Bf16Matrix), ("convolution", C.c_void_p),
                ("alpha_bias", C.c_void_p), ("a_log", C.c_void_p), ("norm", C.c_void_p)]


class DecoderLayerStruct(C.Structure):
    _fields_ = [("input_norm", C.c_void_p), ("post_attention_norm", C.c_void_p),
                ("full_attention", C.c_int), ("full", FullAttentionStruct),
                ("linear", LinearAttentionStruct), ("moe", MoeLayer)]


class LayerState(C.Structure):
    _fields_ = [("keys", C.c_void_p), ("values", C.c_void_p), ("capacity", C.c_uint32),
                ("convolution", C.c_void_p), ("recurrent", C.c_void_p)]


class ModelStruct(C.Structure):
    _fields_ = [("layers", u32), ("layer", C.POINTER(DecoderLayerStruct)),
                ("embedding", C.POINTER(Embedding)), ("final_norm", vp), ("head_chunks", u32),
                ("head", C.POINTER(HeadChunk)), ("context", u32)]


class DecoderStateStruct(C.Structure):
    _fields_ = [("position", u32), ("layers", C.POINTER(LayerState))]


class BatcherOptions(C.Structure):
    _fields_ = [("max_batch", u32), ("capacity", u32), ("prefill_ubatch", u32),
                ("stop_tokens", C.POINTER(u32)), ("stop_count", u32),
                ("masked_tokens", C.POINTER(u32)), ("masked_count", u32), ("direct_steps", u32)]


class GenerationOptions(C.Structure):
    _fields_ = [("max_output_tokens", u32), ("temperature", f32), ("top_p", f32), ("seed", u64)]


class RequestStatus(C.Structure):
    _fields_ = [("state", u32), ("input_tokens", u32), ("output_tokens", u32),
                ("prefill_seconds", C.c_double), ("decode_seconds", C.c_double)]


class KernelProfile(C.Structure):
    _fields_ = [("name", C.c_char * 48), ("launches", C.c_uint64), ("total_ms", C.c_double)]


class GgufTensor(C.Structure):
    _fields_ = [("type", u32), ("dimension_count", u32), ("dimensions", C.c_uint64 * 4),
                ("elements", C.c_uint64), ("bytes", C.c_uint64), ("data", vp)]


class MoeGeometry(C.Structure):
    _fields_ = [("layers", u32), ("hidden", u32), ("experts", u32), ("active_experts", u32),
                ("expert_hidden", u32), ("shared_hidden", u32)]


u64 = C.c_uint64
cs = C.c_char_p


# (name, restype, argtypes) of every exported entry point.
SIGNATURES = [
    ("adi_hip_context_create", C.c_int, [C.c_int, C.POINTER(vp)]),
    ("adi_hip_context_destroy", None, [vp]),
    ("adi_hip_last_error", C.c_char_p, [vp]),
    ("adi_hip_set_stream", C.c_int, [vp, vp]),
    ("adi_hip_synchronize", C.c_int, [vp]),
    ("adi_hip_set_fused_decode", C.c_int, [vp, C.c_int]),
    ("adi_hip_set_workspace_limit", C.c_int, [vp, C.c_size_t]),
    ("adi_hip_set_reduction_isa", C.c_int, [vp, u32]),
    ("adi_hip_device_alloc", C.c_int, [vp, C.c_size_t, C.POINTER(vp)]),
    ("adi_hip_device_free", None, [vp, vp]),
    ("adi_hip_copy_to_device", C.c_int, [vp, vp, vp, C.c_size_t]),
    ("adi_hip_copy_to_host", C.c_int, [vp, vp, vp, C.c_size_t]),
    ("adi_hip_codebook_create_expert", C.c_int, [vp, vp, C.POINTER(vp)]),
    ("adi_hip_codebook_create_ne", C.c_int, [vp, vp, C.POINTER(vp)]),
    ("adi_hip_codebook_destroy", None, [vp]),
    ("adi_hip_expert_matmul", C.c_int, [vp, C.POINTER(ExpertMatrix), vp, u32, vp]),
    ("adi_hip_expert_matvec", C.c_int, [vp, C.POINTER(ExpertMatrix), vp, vp]),
    ("adi_hip_ne_matmul", C.c_int, [vp, C.POINTER(NeMatrix), vp, u32, vp]),
    ("adi_hip_ne_matvec", C.c_int, [vp, C.POINTER(NeMatrix), vp, vp]),
    ("adi_hip_hadamard", C.c_int, [vp, vp, u32, u32]),
    ("adi_hip_expert_decode", C.c_int, [vp, C.POINTER(ExpertMatrix), vp]),
    ("adi_hip_ne_decode", C.c_int, [vp, C.POINTER(NeMatrix), vp]),
    ("adi_hip_head_matmul", C.c_int, [vp, C.POINTER(HeadChunk), vp, u32, vp]),
    ("adi_hip_head_matvec", C.c_int, [vp, C.POINTER(HeadChunk), vp, vp]),
    ("adi_hip_head_argmax", C.c_int, [vp, C.POINTER(HeadChunk), vp, u32, vp, vp]),
    ("adi_hip_bf16_matmul", C.c_int, [vp, C.POINTER(Bf16Matrix), vp, u32, vp]),
    ("adi_hip_bf16_matvec", C.c_int, [vp, C.POINTER(Bf16Matrix), vp, vp]),
    ("adi_hip_rms_norm", C.c_int, [vp, vp, vp, u32, u32, f32, f32, vp]),
    ("adi_hip_top_experts", C.c_int, [vp, vp, u32, u32, vp, vp]),
    ("adi_hip_moe_route", C.c_int, [vp, vp, vp, u32, u32, vp, vp, vp, vp, vp, vp]),
    ("adi_hip_moe_forward", C.c_int, [vp, C.POINTER(MoeLayer), vp, u32, vp, vp, vp, vp]),
    ("adi_hip_moe_forward_static", C.c_int, [vp, C.POINTER(MoeLayer), vp, u32, vp, vp, vp, vp]),
    ("adi_hip_embedding_rows", C.c_int, [vp, C.POINTER(Embedding), vp, u32, vp]),
    ("adi_hip_argmax_rows", C.c_int, [vp, vp, u32, u32, vp]),
    ("adi_hip_sample_rows", C.c_int, [vp, vp, u32, u32, f32, f32, vp, vp]),
    ("adi_hip_full_attention_forward", C.c_int,
     [vp, C.POINTER(FullAttentionStruct), u32, vp, vp, vp, vp, u32]),
    ("adi_hip_linear_attention_forward", C.c_int,
     [vp, C.POINTER(LinearAttentionStruct), vp, vp, vp, vp]),
    ("adi_hip_decode_layer", C.c_int,
     [vp, C.POINTER(DecoderLayerStruct), u32, vp, C.POINTER(LayerState)]),
    ("adi_hip_full_attention_prefill", C.c_int,
     [vp, C.POINTER(FullAttentionStruct), u32, u32, vp, vp, vp, vp, u32]),
    ("adi_hip_linear_attention_prefill", C.c_int,
     [vp, C.POINTER(LinearAttentionStruct), u32, vp, vp, vp, vp]),
    ("adi_hip_prefill_layer", C.c_int,
     [vp, C.POINTER(DecoderLayerStruct), u32, u32, vp, C.POINTER(LayerState)]),
    ("adi_hip_decode_batch", C.c_int,
     [vp, C.POINTER(ModelStruct), C.POINTER(u32), u32, C.POINTER(DecoderStateStruct), vp]),
    ("adi_hip_prefill", C.c_int,
     [vp, C.POINTER(ModelStruct), C.POINTER(u32), u32, u32, C.POINTER(DecoderStateStruct), vp]),
    ("adi_hip_decode_graph_create", C.c_int,
     [vp, C.POINTER(ModelStruct), u32, C.POINTER(DecoderStateStruct), vp, vp, C.POINTER(vp)]),
    ("adi_hip_decode_graph_launch", C.c_int, [vp, C.POINTER(DecoderStateStruct)]),
    ("adi_hip_decode_graph_captures", u32, [vp]),
    ("adi_hip_decode_graph_destroy", None, [vp]),
    ("adi_hip_batcher_create", C.c_int,
     [vp, C.POINTER(ModelStruct), C.POINTER(BatcherOptions), C.POINTER(vp)]),
    ("adi_hip_batcher_destroy", None, [vp]),
    ("adi_hip_batcher_submit", C.c_int,
     [vp, C.POINTER(u32), u32, C.POINTER(GenerationOptions), C.POINTER(u64)]),
    ("adi_hip_batcher_cancel", C.c_int, [vp, u64]),
    ("adi_hip_batcher_step", C.c_int, [vp, C.POINTER(u32)]),
    ("adi_hip_batcher_status", C.c_int, [vp, u64, C.POINTER(RequestStatus), C.POINTER(u32), u32]),
    ("adi_hip_batcher_request_error", C.c_char_p, [vp, u64]),
    ("adi_hip_batcher_release", C.c_int, [vp, u64]),
    ("adi_hip_batcher_force_failure", C.c_int, [vp, C.c_int]),
    ("adi_hip_profiling_enable", C.c_int, [vp, C.c_int]),
    ("adi_hip_profiling_read", C.c_int, [vp, C.POINTER(KernelProfile), u32, C.POINTER(u32)]),
    # include/adi_hip_gguf.h
    ("adi_hip_gguf_open", C.c_int, [cs, C.POINTER(vp)]),
    ("adi_hip_gguf_close", None, [vp]),
    ("adi_hip_gguf_error", C.c_char_p, []),
    ("adi_hip_gguf_version", u32, [vp]),
    ("adi_hip_gguf_alignment", u64, [vp]),
    ("adi_hip_gguf_metadata_count", u64, [vp]),
    ("adi_hip_gguf_tensor_count", u64, [vp]),
    ("adi_hip_gguf_find_tensor", C.c_int, [vp, cs, C.POINTER(GgufTensor)]),
    ("adi_hip_gguf_integer", C.c_int, [vp, cs, C.POINTER(u64)]),
    ("adi_hip_gguf_number", C.c_int, [vp, cs, C.POINTER(C.c_double)]),
    ("adi_hip_gguf_boolean", C.c_int, [vp, cs, C.POINTER(C.c_int)]),
    ("adi_hip_gguf_string", C.c_int, [vp, cs, C.POINTER(vp), C.POINTER(u64)]),
    ("adi_hip_gguf_string_array", C.c_int, [vp, cs, u64, C.POINTER(u64), C.POINTER(vp), C.POINTER(u64)]),
    ("adi_hip_gguf_integer_array", C.c_int, [vp, cs, u64, C.POINTER(u64), C.POINTER(u64)]),
    ("adi_hip_gguf_moe_geometry", C.c_int, [vp, C.POINTER(MoeGeometry)]),
    ("adi_hip_gguf_check_moe_layer", C.c_int, [vp, u32]),
    ("adi_hip_gguf_upload_codebooks", C.c_int, [vp, vp, C.POINTER(vp), C.POINTER(vp)]),
    ("adi_hip_gguf_upload_moe_layer", C.c_int, [vp, vp, u32, vp, vp, C.POINTER(vp), C.POINTER(MoeLayer)]),
    ("adi_hip_weights_destroy", None, [vp]),
    ("adi_hip_gguf_upload_embedding", C.c_int, [vp, vp, C.POINTER(vp), C.POINTER(Embedding)]),
    ("adi_hip_gguf_check_decoder_layer", C.c_int, [vp, u32]),
    ("adi_hip_gguf_upload_decoder_layer", C.c_int, [vp, vp, u32, vp, vp, C.POINTER(vp),
                                                    C.POINTER(DecoderLayerStruct)]),
    ("adi_hip_gguf_check_head", C.c_int, [vp]),
    ("adi_hip_gguf_upload_head", C.c_int, [vp, vp, C.POINTER(vp), C.POINTER(HeadChunk),
                                           C.POINTER(vp)]),
    ("adi_hip_gguf_check_embedding", C.c_int, [vp]),
]

_lib: Optional[C.CDLL] = None


def load() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIBRARY):
            raise RuntimeError(
                f"{LIBRARY} is not built: run `python -m adi_amd.build` (the HIP path has no fallback)")
        lib = C.CDLL(LIBRARY)
        for name, restype, argtypes in SIGNATURES:
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
    return _lib


class HipError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"status {status}: {message}")
        self.status = status


def _addr(t) -> Optional[int]:
    if t is None:
        return None
    return t.data_ptr()


class Context:
    """One adi_hip_context bound to torch's current stream on `device`."""

    def __init__(self, device: int = 0, isa_lanes: int = 16):
        import torch
        self.torch = torch
        self.lib = load()
        handle = vp()
        status = self.lib.adi_hip_context_create(device, C.byref(handle))
        if status != OK:
            raise HipError(status, self.lib.adi_hip_last_error(None).decode())
        self.handle = handle
        self.device = device
        self._books = []
        self.check(self.lib.adi_hip_set_stream(self.handle, vp(torch.cuda.current_stream(device).cuda_stream)))
        self.set_isa(isa_lanes)

    def use_stream(self, stream) -> None:
        """Launch on `stream` (a torch stream) from now on."""
        self.check(self.lib.adi_hip_set_stream(self.handle, vp(stream.cuda_stream)))

    # -- plumbing --
    def check(self, status: int) -> None:
        if status != OK:
            raise HipError(status, self.lib.adi_hip_last_error(self.handle).decode())

    def set_isa(self, lanes: int) -> None:
        self.check(self.lib.adi_hip_set_reduction_isa(self.handle, lanes))
        self.isa_lanes = lanes

    def synchronize(self) -> None:
        self.check(self.lib.adi_hip_synchronize(self.handle))

    def set_fused_decode(self, enabled) -> None:
        """One persistent launch for a MoE block of 1-12 rows and for NE
        projections of up to 4 rows (True, the default), or the separate
        launches (False); "gemv" is the separate launches with the
        decode-GEMV path up to 16 rows (the one-launch block's arithmetic)."""
        mode = 2 if enabled == "gemv" else (1 if enabled else 0)
        self.check(self.lib.adi_hip_set_fused_decode(self.handle, mode))

    def set_workspace_limit(self, limit: int | None) -> None:
        """Cap each scratch arena at `limit` bytes (None: no cap); a call that
        would grow one beyond it fails with OUT_OF_MEMORY."""
        self.check(self.lib.adi_hip_set_workspace_limit(self.handle, (1 << 64) - 1 if limit is None else limit))

    def close(self) -> None:
        if getattr(self, "handle", None):
            for book in self._books:
                self.lib.adi_hip_codebook_destroy(book)
            self._books = []
            self.lib.adi_hip_context_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- codebooks --
    def expert_codebook(self, tlut: np.ndarray) -> int:
        tlut = np.ascontiguousarray(tlut, np.float32)
        out = vp()
        self.check(self.lib.adi_hip_codebook_create_expert(self.handle, tlut.ctypes.data, C.byref(out)))
        self._books.append(out)
        return out.value

    def ne_codebook(self, tlut: np.ndarray) -> int:
        tlut = np.ascontiguousarray(tlut, np.float32)
        out = vp()
        self.check(self.lib.adi_hip_codebook_create_ne(self.handle, tlut.ctypes.data, C.byref(out)))
        self._books.append(out)
        return out.value

    # -- device upload helpers --
    def to_device(self, array: np.ndarray):
        torch = self.torch
        array = np.ascontiguousarray(array)
        dtype = {np.dtype(np.uint16): torch.int16, np.dtype(np.int8): torch.int8,
                 np.dtype(np.uint8): torch.uint8, np.dtype(np.uint32): torch.int32,
                 np.dtype(np.float32): torch.float32}[array.dtype]
        view = array.view({torch.int16: np.int16, torch.int8: np.int8, torch.uint8: np.uint8,
                           torch.int32: np.int32, torch.float32: np.float32}[dtype])
        return torch.from_numpy(view).to(f"cuda:{self.device}")

    # -- profiling --
    def profiling(self, enabled: bool) -> None:
        self.check(self.lib.adi_hip_profiling_enable(self.handle, 1 if enabled else 0))

    def profile(self) -> dict:
        count = u32()
        buf = (KernelProfile * 64)()
        self.check(self.lib.adi_hip_profiling_read(self.handle, buf, 64, C.byref(count)))
        return {buf[i].name.decode(): (buf[i].launches, buf[i].total_ms)
                for i in range(min(count.value, 64))}


@dataclass
class DeviceExpert:
    struct: ExpertMatrix
    tensors: tuple


@dataclass
class DeviceNe:
    struct: NeMatrix
    tensors: tuple


@dataclass
class DeviceHead:
    struct: HeadChunk
    tensors: tuple


def upload_expert(ctx: Context, m, codebook: int) -> DeviceExpert:
    t = tuple(ctx.to_device(a) for a in (m.trellis, m.su_f16, m.sv_f16, m.wave_gamma_f16))
    s = ExpertMatrix(m.rows, m.columns, *(x.data_ptr() for x in t), codebook)
    return DeviceExpert(s, t)


def upload_ne(ctx: Context, m, codebook: int) -> DeviceNe:
    t = tuple(ctx.to_device(a) for a in (m.trellis, m.su, m.sv))
    s = NeMatrix(m.rows, m.columns, t[0].data_ptr(), t[1].data_ptr(), t[2].data_ptr(),
                 float(m.weight_scale), codebook)
    return DeviceNe(s, t)


def upload_head(ctx: Context, h) -> DeviceHead:
    packed = ctx.to_device(h.packed)
    scales = ctx.to_device(h.group_scale_f16)
    tensors = [packed, scales]
    prot_rows = prot_vals = None
    count = 0
    if h.protected_rows is not None and h.protected_rows.size:
        prot_rows = ctx.to_device(h.protected_rows)
        prot_vals = ctx.to_device(h.protected_bf16)
        tensors += [prot_rows, prot_vals]
        count = int(h.protected_rows.size)
    s = HeadChunk(h.rows, h.columns, packed.data_ptr(), scales.data_ptr(),
                  _addr(prot_rows), _addr(prot_vals), count)
    return DeviceHead(s, tuple(tensors))


@dataclass
class DeviceMoeLayer:
    struct: MoeLayer
    tensors: tuple
    experts: int
    hidden: int


def stack_experts(mats):
    return (np.concatenate([m.trellis for m in mats]), np.concatenate([m.su_f16 for m in mats]),
            np.concatenate([m.sv_f16 for m in mats]), np.concatenate([m.wave_gamma_f16 for m in mats]))


def upload_moe_layer(ctx: Context, layer, expert_book: int, ne_book: int) -> DeviceMoeLayer:
    keep = []

    def dev(a):
        t = ctx.to_device(a)
        keep.append(t)
        return t.data_ptr()

    stacks = []
    for kind in ("gate", "up", "down"):
        held = getattr(layer, "stacks", None)
        arrays = held[kind] if held else stack_experts(getattr(layer, kind))
        stacks.append(ExpertStack(*(dev(a) for a in arrays)))
    shared = []
    for m in (layer.shared_gate, layer.shared_up, layer.shared_down):
        d = upload_ne(ctx, m, ne_book)
        keep.extend(d.tensors)
        shared.append(d.struct)
    router = Bf16Matrix(layer.experts, layer.hidden, dev(layer.router_bf16))
    gate = Bf16Matrix(1, layer.hidden, dev(layer.shared_expert_gate_bf16))
    s = MoeLayer(layer.hidden, layer.expert_hidden, layer.experts, router, gate,
                 stacks[0], stacks[1], stacks[2], expert_book, shared[0], shared[1], shared[2])
    return DeviceMoeLayer(s, tuple(keep), layer.experts, layer.hidden)


# ---- checkpoints (GGUF v3) ---------------------------------------------------

_GGML_NUMPY = {GGML_F32: np.float32, GGML_F16: np.uint16, GGML_I8: np.int8, GGML_I16: np.uint16,
               GGML_I32: np.int32, GGML_I64: np.int64, GGML_F64: np.float64, GGML_BF16: np.uint16}


class Gguf:
    """An open GGUF v3 file (adi_hip_gguf); host-side, needs no GPU."""

    def __init__(self, path: str):
        self.lib = load()
        handle = vp()
        status = self.lib.adi_hip_gguf_open(os.fsencode(path), C.byref(handle))
        if status != OK:
            raise HipError(status, self.lib.adi_hip_gguf_error().decode())
        self.handle = handle

    def _fail(self, status: int):
        raise HipError(status, self.lib.adi_hip_gguf_error().decode())

    def close(self) -> None:
        if getattr(self, "handle", None):
            self.lib.adi_hip_gguf_close(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def version(self) -> int:
        return self.lib.adi_hip_gguf_version(self.handle)

    @property
    def alignment(self) -> int:
        return self.lib.adi_hip_gguf_alignment(self.handle)

    @property
    def metadata_count(self) -> int:
        return self.lib.adi_hip_gguf_metadata_count(self.handle)

    @property
    def tensor_count(self) -> int:
        return self.lib.adi_hip_gguf_tensor_count(self.handle)

    def tensor(self, name: str):
        """(GgufTensor, numpy view of its data) or None when absent."""
        t = GgufTensor()
        status = self.lib.adi_hip_gguf_find_tensor(self.handle, name.encode(), C.byref(t))
        if status == NOT_FOUND:
            return None
        if status != OK:
            self._fail(status)
        dtype = _GGML_NUMPY[t.type]
        buf = (C.c_uint8 * t.bytes).from_address(t.data)
        return t, np.frombuffer(buf, dtype=dtype, count=t.elements)

    def _scalar(self, fn, key, ctype):
        out = ctype()
        status = fn(self.handle, key.encode(), C.byref(out))
        if status == NOT_FOUND:
            return None
        if status != OK:
            self._fail(status)
        return out.value

    def integer(self, key: str):
        return self._scalar(self.lib.adi_hip_gguf_integer, key, u64)

    def number(self, key: str):
        return self._scalar(self.lib.adi_hip_gguf_number, key, C.c_double)

    def boolean(self, key: str):
        v = self._scalar(self.lib.adi_hip_gguf_boolean, key, C.c_int)
        return None if v is None else bool(v)

    def string(self, key: str):
        data, length = vp(), u64()
        status = self.lib.adi_hip_gguf_string(self.handle, key.encode(), C.byref(data), C.byref(length))
        if status == NOT_FOUND:
            return None
        if status != OK:
            self._fail(status)
        return C.string_at(data.value, length.value).decode()

    def string_array(self, key: str):
        count, data, length = u64(), vp(), u64()
        status = self.lib.adi_hip_gguf_string_array(self.handle, key.encode(), 0, C.byref(count), None, None)
        if status == NOT_FOUND:
            return []
        if status != OK:
            self._fail(status)
        out = []
        for i in range(count.value):
            self.lib.adi_hip_gguf_string_array(self.handle, key.encode(), i, C.byref(count),
                                               C.byref(data), C.byref(length))
            out.append(C.string_at(data.value, length.value).decode())
        return out

    def integer_array(self, key: str):
        count, value = u64(), u64()
        status = self.lib.adi_hip_gguf_integer_array(self.handle, key.encode(), 0, C.byref(count), None)
        if status == NOT_FOUND:
            return []
        if status != OK:
            self._fail(status)
        out = []
        for i in range(count.value):
            self.lib.adi_hip_gguf_integer_array(self.handle, key.encode(), i, C.byref(count), C.byref(value))
            out.append(value.value)
        return out

    def moe_geometry(self) -> MoeGeometry:
        g = MoeGeometry()
        status = self.lib.adi_hip_gguf_moe_geometry(self.handle, C.byref(g))
        if status != OK:
            self._fail(status)
        return g

    def check_moe_layer(self, layer: int) -> None:
        status = self.lib.adi_hip_gguf_check_moe_layer(self.handle, layer)
        if status != OK:
            self._fail(status)

    def check_embedding(self) -> None:
        status = self.lib.adi_hip_gguf_check_embedding(self.handle)
        if status != OK:
            self._fail(status)

    def check_decoder_layer(self, layer: int) -> None:
        status = self.lib.adi_hip_gguf_check_decoder_layer(self.handle, layer)
        if status != OK:
            self._fail(status)

    def check_head(self) -> None:
        status = self.lib.adi_hip_gguf_check_head(self.handle)
        if status != OK:
            self._fail(status)


@dataclass
class GgufMoeLayer:
    """A layer uploaded from a checkpoint; owns its adi_hip_weights."""
    struct: MoeLayer
    weights: int
    experts: int
    hidden: int
    lib: object = None

    def close(self) -> None:
        if self.weights:
            self.lib.adi_hip_weights_destroy(vp(self.weights))
            self.weights = 0

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def upload_codebooks_gguf(ctx: Context, file: Gguf):
    expert, ne = vp(), vp()
    ctx.check(ctx.lib.adi_hip_gguf_upload_codebooks(ctx.handle, file.handle, C.byref(expert), C.byref(ne)))
    ctx._books.extend([expert, ne])
    return expert.value, ne.value


def upload_moe_layer_gguf(ctx: Context, file: Gguf, layer: int, expert_book: int,
                          ne_book: int) -> GgufMoeLayer:
    weights = vp()
    s = MoeLayer()
    ctx.check(ctx.lib.adi_hip_gguf_upload_moe_layer(ctx.handle, file.handle, layer, vp(expert_book),
                                                    vp(ne_book), C.byref(weights), C.byref(s)))
    return GgufMoeLayer(s, weights.value, s.experts, s.hidden, ctx.lib)


@dataclass
class GgufEmbedding:
    """An embedding table uploaded from a checkpoint; owns its adi_hip_weights."""
    struct: Embedding
    weights: int
    lib: object = None

    def close(self) -> None:
        if self.weights:
            self.lib.adi_hip_weights_destroy(vp(self.weights))
            self.weights = 0

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


@dataclass
class GgufDecoderLayer:
    """A whole decoder layer uploaded from a checkpoint (norms, attention,
    MoE block); owns its adi_hip_weights."""
    struct: DecoderLayerStruct
    weights: int
    lib: object = None

    def close(self) -> None:
        if self.weights:
            self.lib.adi_hip_weights_destroy(vp(self.weights))
            self.weights = 0

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def upload_decoder_layer_gguf(ctx: Context, file: Gguf, layer: int, expert_book: int,
                              ne_book: int) -> GgufDecoderLayer:
    weights = vp()
    s = DecoderLayerStruct()
    ctx.check(ctx.lib.adi_hip_gguf_upload_decoder_layer(ctx.handle, file.handle, layer, vp(expert_book),
                                                        vp(ne_book), C.byref(weights), C.byref(s)))
    return GgufDecoderLayer(s, weights.value, ctx.lib)


@dataclass
class GgufHead:
    """The output head (eight chunks end to end) and the final norm uploaded
    from a checkpoint; owns its adi_hip_weights."""
    struct: HeadChunk
    final_norm: int
    weights: int
    lib: object = None

    def close(self) -> None:
        if self.weights:
            self.lib.adi_hip_weights_destroy(vp(self.weights))
            self.weights = 0

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def upload_head_gguf(ctx: Context, file: Gguf) -> GgufHead:
    weights, norm = vp(), vp()
    s = HeadChunk()
    ctx.check(ctx.lib.adi_hip_gguf_upload_head(ctx.handle, file.handle, C.byref(weights), C.byref(s),
                                               C.byref(norm)))
    return GgufHead(s, norm.value, weights.value, ctx.lib)


def upload_embedding_gguf(ctx: Context, file: Gguf) -> GgufEmbedding:
    weights = vp()
    s = Embedding()
    ctx.check(ctx.lib.adi_hip_gguf_upload_embedding(ctx.handle, file.handle, C.byref(weights),
                                                    C.byref(s)))
    return GgufEmbedding(s, weights.value, ctx.lib)


@dataclass
class DeviceEmbedding:
    struct: Embedding
    tensors: tuple


def upload_embedding(ctx: Context, e) -> DeviceEmbedding:
    """e: adi_amd.synthetic.Embedding."""
    keep = [ctx.to_device(a) for a in (e.packed, e.minimum_f16, e.maximum_f16)]
    count = int(e.exception_indexes.size)
    if count:
        keep += [ctx.to_device(e.exception_indexes), ctx.to_device(e.exception_bf16)]
    ptrs = [t.data_ptr() for t in keep] + [None, None][:5 - len(keep)]
    s = Embedding(e.rows, e.columns, *ptrs, count)
    return DeviceEmbedding(s, tuple(keep))


def embedding_rows(ctx: Context, emb, tokens, count: int, out) -> None:
    ctx.check(ctx.lib.adi_hip_embedding_rows(ctx.handle, C.byref(emb.struct), tokens.data_ptr(),
                                             count, out.data_ptr()))


def argmax_rows(ctx: Context, logits, rows: int, count: int, tokens) -> None:
    ctx.check(ctx.lib.adi_hip_argmax_rows(ctx.handle, logits.data_ptr(), rows, count,
                                          tokens.data_ptr()))


def sample_rows(ctx: Context, logits, rows: int, count: int, temperature: float, top_p: float,
                words, tokens) -> None:
    ctx.check(ctx.lib.adi_hip_sample_rows(ctx.handle, logits.data_ptr(), rows, count, temperature,
                                          top_p, _addr(words), tokens.data_ptr()))


# ---- calls on device tensors ------------------------------------------------

def expert_matmul(ctx: Context, m: DeviceExpert, x, batch: int, out) -> None:
    ctx.check(ctx.lib.adi_hip_expert_matmul(ctx.handle, C.byref(m.struct), x.data_ptr(), batch,
                                            out.data_ptr()))


def hadamard(ctx: Context, values, n: int, count: int) -> None:
    ctx.check(ctx.lib.adi_hip_hadamard(ctx.handle, values.data_ptr(), n, count))


def expert_decode(ctx: Context, m: DeviceExpert, out) -> None:
    ctx.check(ctx.lib.adi_hip_expert_decode(ctx.handle, C.byref(m.struct), out.data_ptr()))


def ne_decode(ctx: Context, m: DeviceNe, out) -> None:
    ctx.check(ctx.lib.adi_hip_ne_decode(ctx.handle, C.byref(m.struct), out.data_ptr()))


def ne_matmul(ctx: Context, m: DeviceNe, x, batch: int, out) -> None:
    ctx.check(ctx.lib.adi_hip_ne_matmul(ctx.handle, C.byref(m.struct), x.data_ptr(), batch,
                                        out.data_ptr()))


def head_matmul(ctx: Context, h: DeviceHead, x, batch: int, out) -> None:
    ctx.check(ctx.lib.adi_hip_head_matmul(ctx.handle, C.byref(h.struct), x.data_ptr(), batch,
                                          out.data_ptr()))


def head_argmax(ctx: Context, h: DeviceHead, x, batch: int, logits, argmax) -> None:
    ctx.check(ctx.lib.adi_hip_head_argmax(ctx.handle, C.byref(h.struct), x.data_ptr(), batch,
                                          _addr(logits), argmax.data_ptr()))


def bf16_matmul(ctx: Context, values, rows: int, columns: int, x, batch: int, out) -> None:
    s = Bf16Matrix(rows, columns, values.data_ptr())
    ctx.check(ctx.lib.adi_hip_bf16_matmul(ctx.handle, C.byref(s), x.data_ptr(), batch,
                                          out.data_ptr()))


def rms_norm(ctx: Context, x, weight, count: int, rows: int, offset: float, eps: float, out) -> None:
    ctx.check(ctx.lib.adi_hip_rms_norm(ctx.handle, x.data_ptr(), weight.data_ptr(), count, rows,
                                       offset, eps, out.data_ptr()))


def top_experts(ctx: Context, logits, batch: int, experts: int, route_expert, route_weight) -> None:
    ctx.check(ctx.lib.adi_hip_top_experts(ctx.handle, logits.data_ptr(), batch, experts,
                                          route_expert.data_ptr(), route_weight.data_ptr()))


def moe_route(ctx: Context, logits, bias, batch: int, experts: int, out: dict) -> None:
    ctx.check(ctx.lib.adi_hip_moe_route(
        ctx.handle, logits.data_ptr(), _addr(bias), batch, experts,
        out["route_expert"].data_ptr(), out["route_weight"].data_ptr(), out["counts"].data_ptr(),
        out["offsets"].data_ptr(), out["grouped_batch"].data_ptr(),
        out["route_to_grouped"].data_ptr()))


def moe_forward(ctx: Context, layer: DeviceMoeLayer, x, batch: int, bias, out,
                route_expert=None, route_weight=None) -> None:
    ctx.check(ctx.lib.adi_hip_moe_forward(ctx.handle, C.byref(layer.struct), x.data_ptr(), batch,
                                          _addr(bias), out.data_ptr(), _addr(route_expert),
                                          _addr(route_weight)))


# ---- layers generated directly in device memory (benchmark rotation) --------

def random_device_moe_layer(ctx: Context, seed: int, hidden: int, expert_hidden: int,
                            experts: int, expert_book: int, ne_book: int) -> DeviceMoeLayer:
    """A layer with the synthetic distributions of adi_amd.synthetic, drawn
    with torch's device generator (no host round trip)."""
    torch = ctx.torch
    dev = f"cuda:{ctx.device}"
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    keep = []

    def words(n):
        t = torch.randint(-32768, 32768, (n,), dtype=torch.int16, device=dev, generator=g)
        keep.append(t)
        return t.data_ptr()

    def lognormal_f16(n):
        t = torch.empty(n, device=dev).log_normal_(0.0, 0.5, generator=g).half().view(torch.int16)
        keep.append(t)
        return t.data_ptr()

    def bf16(shape):
        t = (torch.randn(shape, device=dev, generator=g) * 0.02).to(torch.bfloat16).view(torch.int16)
        keep.append(t)
        return t.data_ptr()

    def signs(n):
        t = (torch.randint(0, 2, (n,), device=dev, generator=g) * 2 - 1).to(torch.int8)
        keep.append(t)
        return t.data_ptr()

    def stack(rows, columns):
        tiles = (rows // 16) * (columns // 16)
        return ExpertStack(words(experts * tiles * 24), lognormal_f16(experts * columns),
                           lognormal_f16(experts * rows),
                           lognormal_f16(experts * (rows // 16 + columns // 16)))

    def ne(rows, columns):
        tiles = (rows // 16) * (columns // 16)
        scale = float(torch.empty(1).log_normal_(0.0, 0.5, generator=torch.Generator().manual_seed(seed)).item())
        return NeMatrix(rows, columns, words(tiles * 64), signs(columns), signs(rows), scale, ne_book)

    s = MoeLayer(hidden, expert_hidden, experts,
                 Bf16Matrix(experts, hidden, bf16((experts, hidden))),
                 Bf16Matrix(1, hidden, bf16((1, hidden))),
                 stack(expert_hidden, hidden), stack(expert_hidden, hidden),
                 stack(hidden, expert_hidden), expert_book,
                 ne(expert_hidden, hidden), ne(expert_hidden, hidden), ne(hidden, expert_hidden))
    return DeviceMoeLayer(s, tuple(keep), experts, hidden)


@dataclass
class DeviceFullAttention:
    struct: FullAttentionStruct
    tensors: tuple


@dataclass
class DeviceLinearAttention:
    struct: LinearAttentionStruct
    tensors: tuple


def upload_full_attention(ctx: Context, layer, ne_book: int) -> DeviceFullAttention:
    """layer: adi_amd.synthetic.FullAttention."""
    mats = [upload_ne(ctx, m, ne_book) for m in (layer.query, layer.key, layer.value, layer.output)]
    norms = [ctx.to_device(a) for a in (layer.query_norm, layer.key_norm)]
    s = FullAttentionStruct(*(m.struct for m in mats), *(t.data_ptr() for t in norms))
    return DeviceFullAttention(s, (mats, norms))


def upload_linear_attention(ctx: Context, layer, ne_book: int) -> DeviceLinearAttention:
    """layer: adi_amd.synthetic.LinearAttention."""
    mats = [upload_ne(ctx, m, ne_book) for m in (layer.qkv, layer.gate, layer.output)]
    alpha = ctx.to_device(layer.alpha)
    beta = ctx.to_device(layer.beta)
    rest = [ctx.to_device(a) for a in (layer.convolution, layer.alpha_bias, layer.a_log, layer.norm)]
    s = LinearAttentionStruct(
        *(m.struct for m in mats),
        Bf16Matrix(32, layer.hidden, alpha.data_ptr()), Bf16Matrix(32, layer.hidden, beta.data_ptr()),
        *(t.data_ptr() for t in rest))
    return DeviceLinearAttention(s, (mats, alpha, beta, rest))


def full_attention_forward(ctx: Context, layer: DeviceFullAttention, position: int, x, out,
                           keys, values, capacity: int) -> None:
    ctx.check(load().adi_hip_full_attention_forward(
        ctx.handle, C.byref(layer.struct), position, _addr(x), _addr(out), _addr(keys),
        _addr(values), capacity))


def linear_attention_forward(ctx: Context, layer: DeviceLinearAttention, x, out, convolution,
                             recurrent) -> None:
    ctx.check(load().adi_hip_linear_attention_forward(
        ctx.handle, C.byref(layer.struct), _addr(x), _addr(out), _addr(convolution),
        _addr(recurrent)))


@dataclass
class DeviceDecoderLayer:
    struct: DecoderLayerStruct
    tensors: tuple


def upload_decoder_layer(ctx: Context, layer, expert_book: int, ne_book: int) -> DeviceDecoderLayer:
    """layer: adi_amd.synthetic.DecoderLayer."""
    norms = [ctx.to_device(a) for a in (layer.input_norm, layer.post_attention_norm)]
    moe = upload_moe_layer(ctx, layer.moe, expert_book, ne_book)
    full = upload_full_attention(ctx, layer.full, ne_book) if layer.full is not None else None
    linear = (upload_linear_attention(ctx, layer.linear, ne_book)
              if layer.linear is not None else None)
    s = DecoderLayerStruct(norms[0].data_ptr(), norms[1].data_ptr(), int(full is not None),
                           full.struct if full else FullAttentionStruct(),
                           linear.struct if linear else LinearAttentionStruct(), moe.struct)
    return DeviceDecoderLayer(s, (norms, moe, full, linear))


def layer_state(full: bool, capacity: int = 0):
    """Zeroed device state of one layer for a new sequence: the KV cache of
    a full-attention layer, else the convolution and recurrent state."""
    import torch
    if full:
        keys = torch.zeros((capacity, 2, 256), dtype=torch.float32, device="cuda")
        values = torch.zeros_like(keys)
        return LayerState(keys.data_ptr(), values.data_ptr(), capacity, None, None), (keys, values)
    conv = torch.zeros(8192 * 3, dtype=torch.float32, device="cuda")
    rec = torch.zeros(32 * 128 * 128, dtype=torch.float32, device="cuda")
    return LayerState(None, None, 0, conv.data_ptr(), rec.data_ptr()), (conv, rec)


def decode_layer(ctx: Context, layer: DeviceDecoderLayer, position: int, hidden, state) -> None:
    ctx.check(load().adi_hip_decode_layer(ctx.handle, C.byref(layer.struct), position,
                                          _addr(hidden), C.byref(state)))


def full_attention_prefill(ctx: Context, layer: DeviceFullAttention, position: int, count: int, x,
                           out, keys, values, capacity: int) -> None:
    ctx.check(load().adi_hip_full_attention_prefill(
        ctx.handle, C.byref(layer.struct), position, count, _addr(x), _addr(out), _addr(keys),
        _addr(values), capacity))


def linear_attention_prefill(ctx: Context, layer: DeviceLinearAttention, count: int, x, out,
                             convolution, recurrent) -> None:
    ctx.check(load().adi_hip_linear_attention_prefill(
        ctx.handle, C.byref(layer.struct), count, _addr(x), _addr(out), _addr(convolution),
        _addr(recurrent)))


def prefill_layer(ctx: Context, layer: DeviceDecoderLayer, position: int, count: int, hidden,
                  state) -> None:
    ctx.check(load().adi_hip_prefill_layer(ctx.handle, C.byref(layer.struct), position, count,
                                           _addr(hidden), C.byref(state)))


# ---- the whole model: decode steps over sequences, prompt prefill -----------

CONTEXT = 262144  # ModelConfig::context of the checkpoint


class Model:
    """adi_hip_model over uploaded parts: decoder layers (DeviceDecoderLayer or
    GgufDecoderLayer), an embedding, the final norm (device bf16 tensor) and
    head chunks (DeviceHead or GgufHead), whose rows in order cover the
    vocabulary."""

    def __init__(self, layers, embedding, final_norm, heads, context: int = CONTEXT):
        self.layers = list(layers)
        self.embedding, self.final_norm, self.heads = embedding, final_norm, list(heads)
        self._layer_array = (DecoderLayerStruct * len(self.layers))(*(L.struct for L in self.layers))
        self._head_array = (HeadChunk * len(self.heads))(*(h.struct for h in self.heads))
        self.struct = ModelStruct(len(self.layers), self._layer_array, C.pointer(embedding.struct),
                                  _addr(final_norm), len(self.heads), self._head_array, context)
        self.vocabulary = int(embedding.struct.rows)
        self.hidden = int(embedding.struct.columns)

    def full_attention(self, layer: int) -> bool:
        return bool(self.layers[layer].struct.full_attention)


class Sequence:
    """A sequence's decoder state on the device: position and one
    LayerState per layer of `model`, zeroed (a new sequence); full-attention
    caches hold `capacity` positions."""

    def __init__(self, model: Model, capacity: int):
        made = [layer_state(model.full_attention(i), capacity) for i in range(len(model.layers))]
        self.tensors = [keep for _, keep in made]
        self._layers = (LayerState * len(made))(*(state for state, _ in made))
        self.struct = DecoderStateStruct(0, self._layers)
        self.capacity = capacity

    @property
    def position(self) -> int:
        return int(self.struct.position)

    def reset(self) -> None:
        for keep in self.tensors:
            for t in keep:
                t.zero_()
        self.struct.position = 0


def decode_batch(ctx: Context, model: Model, tokens, sequences, logits=None) -> None:
    """One decode step of each sequence with its token (host ints): logits
    [len(sequences), vocabulary] (device tensor or None); positions advance."""
    n = len(sequences)
    toks = (u32 * max(n, 1))(*[int(t) for t in tokens])
    states = (DecoderStateStruct * max(n, 1))(*(s.struct for s in sequences))
    status = ctx.lib.adi_hip_decode_batch(ctx.handle, C.byref(model.struct), toks, n, states,
                                          _addr(logits))
    for s, st in zip(sequences, states):
        s.struct.position = st.position
    ctx.check(status)


class DecodeGraph:
    """adi_hip_decode_graph: one decode step of `sequences` captured as a HIP
    graph. Each launch() replays it: the step's tokens are read from
    `tokens` (device int32/uint32 [len(sequences)]), logits go to `logits`
    (device [len(sequences)][vocabulary] or None), and every sequence's
    position advances by one."""

    def __init__(self, ctx: Context, model: Model, sequences, tokens, logits=None):
        self.ctx, self.model, self.sequences = ctx, model, list(sequences)
        self._keep = (tokens, logits)
        n = len(self.sequences)
        self._states = (DecoderStateStruct * max(n, 1))(*(s.struct for s in self.sequences))
        handle = vp()
        ctx.check(ctx.lib.adi_hip_decode_graph_create(ctx.handle, C.byref(model.struct), n,
                                                      self._states, _addr(tokens), _addr(logits),
                                                      C.byref(handle)))
        self.handle = handle

    def launch(self) -> None:
        for st, s in zip(self._states, self.sequences):
            st.position = s.struct.position
        status = self.ctx.lib.adi_hip_decode_graph_launch(self.handle, self._states)
        for st, s in zip(self._states, self.sequences):
            s.struct.position = st.position
        self.ctx.check(status)

    @property
    def captures(self) -> int:
        return int(self.ctx.lib.adi_hip_decode_graph_captures(self.handle))

    def close(self) -> None:
        if self.handle:
            self.ctx.lib.adi_hip_decode_graph_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def prefill(ctx: Context, model: Model, tokens, sequence: Sequence, logits=None,
            ubatch: int = 0) -> None:
    """prefill_prompt of `tokens` (host ints) into the sequence, chunks of
    `ubatch` (0: 128); logits [vocabulary] of the last token (device) or None."""
    toks = (u32 * max(len(tokens), 1))(*[int(t) for t in tokens])
    ctx.check(ctx.lib.adi_hip_prefill(ctx.handle, C.byref(model.struct), toks, len(tokens), ubatch,
                                      C.byref(sequence.struct), _addr(logits)))
