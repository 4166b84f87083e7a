"""GGUF v3 files for the tests: a general writer and synthetic MoE
checkpoints in the reference's tensor naming and layout (docs/gguf.md,
src/model.cpp:267-314, 431-533).

GGUF order puts the contiguous dimension first, so a 32-expert chunk tensor
with dims {24, tiles, 32} holds the 32 experts' trellis end to end, and a
bf16 matrix with dims {columns, rows} is row-major.
"""
from __future__ import annotations

import struct
from typing import List, Sequence, Tuple

import numpy as np

# metadata value types (include/adi/gguf.hpp:13-27)
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
# tensor types (include/adi/gguf.hpp:30-39)
T_F32, T_F16, T_I8, T_I16, T_I32, T_I64, T_F64, T_BF16 = 0, 1, 24, 25, 26, 27, 28, 30

_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f",
           BOOL: "<B", U64: "<Q", I64: "<q", F64: "<d"}


def _string(s) -> bytes:
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _value(kind: int, value) -> bytes:
    if kind in _SCALAR:
        return struct.pack(_SCALAR[kind], value)
    if kind == STRING:
        return _string(value)
    if kind == ARRAY:
        element, items = value
        out = struct.pack("<IQ", element, len(items))
        for item in items:
            out += _value(element, item)
        return out
    raise ValueError(kind)


def gguf_bytes(metadata: Sequence[Tuple[str, int, object]],
               tensors: Sequence[Tuple[str, int, Sequence[int], bytes]],
               alignment: int = 32, version: int = 3, magic: int = 0x46554747) -> bytes:
    """metadata: (key, type, value); tensors: (name, ggml type, GGUF dims, data)."""
    head = struct.pack("<IIQQ", magic, version, len(tensors), len(metadata))
    for key, kind, value in metadata:
        head += _string(key) + struct.pack("<I", kind) + _value(kind, value)
    offsets, at, end = [], 0, 0
    for _, _, _, data in tensors:
        offsets.append(at)
        end = at + len(data)  # the file ends with the last tensor's bytes
        at = (end + alignment - 1) // alignment * alignment
    for (name, kind, dims, _), offset in zip(tensors, offsets):
        head += _string(name) + struct.pack("<I", len(dims))
        head += b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", kind, offset)
    head += b"\0" * ((-len(head)) % alignment)
    body = bytearray(end)
    for (_, _, _, data), offset in zip(tensors, offsets):
        body[offset:offset + len(data)] = data
    return head + bytes(body)


def reference_fixture() -> bytes:
    """The container of the reference's own GGUF test (tests/gguf_test.cpp:
    36-79): five metadata entries and one 2x2 f32 tensor [1, 2, 3, 4]."""
    metadata = [
        ("general.alignment", U32, 32),
        ("general.architecture", STRING, "adi"),
        ("adi.additive", BOOL, 1),
        ("tokenizer.ggml.tokens", ARRAY, (STRING, ["hello", "world"])),
        ("tokenizer.ggml.token_type", ARRAY, (U32, [1, 3])),
    ]
    data = np.array([1, 2, 3, 4], np.float32).tobytes()
    return gguf_bytes(metadata, [("test.weight", T_F32, [2, 2], data)])


def moe_metadata(layers: int, hidden: int, expert_hidden: int, experts: int,
                 **overrides) -> List[Tuple[str, int, object]]:
    """The metadata the packed MoE path reads (src/model.cpp:180-224)."""
    entries = {
        "general.architecture": (STRING, "qwen35moe"),
        "general.name": (STRING, "synthetic-moe"),
        "adi.format_version": (U32, 1),
        "adi.additive": (BOOL, 1),
        "adi.model_family": (STRING, "mach1"),
        "adi.expert_codec": (STRING, "trained_susv_wave_gamma_chunked_v1"),
        "adi.ne_codec": (STRING, "canon_rht_bitshift_trellis_intlattice"),
        "adi.expert.k_num": (U32, 3),
        "adi.expert.k_den": (U32, 2),
        "adi.expert.l": (U32, 16),
        "adi.expert.v": (U32, 8),
        "adi.expert.tlut_bits": (U32, 15),
        "adi.expert.tile_x": (U32, 16),
        "adi.expert.tile_y": (U32, 16),
        "qwen35moe.block_count": (U32, layers),
        "qwen35moe.embedding_length": (U32, hidden),
        "qwen35moe.expert_count": (U32, experts),
        "qwen35moe.expert_used_count": (U32, 8),
        "qwen35moe.expert_feed_forward_length": (U32, expert_hidden),
        "qwen35moe.expert_shared_feed_forward_length": (U32, expert_hidden),
    }
    for key, value in overrides.items():
        key = key.replace("__", ".")
        if value is None:
            entries.pop(key, None)
        else:
            entries[key] = value
    return [(k, t, v) for k, (t, v) in entries.items()]


def ne_tensors(layer_index: int, source: str, m) -> List[Tuple[str, int, List[int], bytes]]:
    """One NE matrix (adi_amd.synthetic.NeMatrix) as
    mach.ne.{layer}.{source}|{trellis|SU|SV|Wscale} (src/model.cpp:267-314)."""
    base = f"mach.ne.{layer_index}.{source}|"
    tiles = (m.rows // 16) * (m.columns // 16)
    return [(base + "trellis", T_I16, [64, tiles], np.asarray(m.trellis, np.uint16).tobytes()),
            (base + "SU", T_I8, [m.columns], np.asarray(m.su, np.int8).tobytes()),
            (base + "SV", T_I8, [m.rows], np.asarray(m.sv, np.int8).tobytes()),
            (base + "Wscale", T_F32, [1], np.array([m.weight_scale], np.float32).tobytes())]


def moe_tensors(layers, indices=None) -> List[Tuple[str, int, List[int], bytes]]:
    """The mach.*, hf.* and TLUT tensors of synthetic MoE layers
    (adi_amd.synthetic.MoeLayer), all sharing the first layer's TLUTs; layer
    i is written as checkpoint layer indices[i] (default i)."""
    first = layers[0]
    out = [
        ("mach.tlut.expert.tlut", T_F32, [8, 32768], np.asarray(first.expert_tlut, np.float32).tobytes()),
        ("mach.tlut.ne.tlut", T_F32, [2, 512], np.asarray(first.ne_tlut, np.float32).tobytes()),
    ]
    indices = list(range(len(layers))) if indices is None else indices
    for li, layer in zip(indices, layers):
        H, I, E = layer.hidden, layer.expert_hidden, layer.experts
        p = f"model.language_model.layers.{li}."
        out.append((f"hf.{p}mlp.gate.weight", T_BF16, [H, E], np.asarray(layer.router_bf16, np.uint16).tobytes()))
        out.append((f"hf.{p}mlp.shared_expert_gate.weight", T_BF16, [H, 1],
                    np.asarray(layer.shared_expert_gate_bf16, np.uint16).tobytes()))
        for name, mats, rows, columns in (("gate", layer.gate, I, H), ("up", layer.up, I, H),
                                          ("down", layer.down, H, I)):
            tiles = (rows // 16) * (columns // 16)
            gammas = rows // 16 + columns // 16
            for chunk in range(0, E, 32):
                part = mats[chunk:chunk + 32]
                base = f"mach.expert.{li}.e{chunk}.{name}."
                out.append((base + "trellis", T_I16, [24, tiles, 32],
                            np.concatenate([m.trellis for m in part]).astype(np.uint16).tobytes()))
                out.append((base + "su", T_F16, [columns, 32],
                            np.concatenate([m.su_f16 for m in part]).astype(np.uint16).tobytes()))
                out.append((base + "sv", T_F16, [rows, 32],
                            np.concatenate([m.sv_f16 for m in part]).astype(np.uint16).tobytes()))
                out.append((base + "wave_gamma", T_F16, [gammas, 32],
                            np.concatenate([m.wave_gamma_f16 for m in part]).astype(np.uint16).tobytes()))
        for name, m in (("gate", layer.shared_gate), ("up", layer.shared_up), ("down", layer.shared_down)):
            out += ne_tensors(li, f"{p}mlp.shared_expert.{name}_proj.weight", m)
    return out


def attention_tensors(layer_index: int, d) -> List[Tuple[str, int, List[int], bytes]]:
    """The norms and attention tensors of a synthetic decoder layer
    (adi_amd.synthetic.DecoderLayer) at checkpoint layer `layer_index`, named
    as MachModel::cache_descriptors reads them (src/model.cpp:619-683)."""
    p = f"model.language_model.layers.{layer_index}."
    bf = lambda name, dims, a: ("hf." + name, T_BF16, dims, np.asarray(a, np.uint16).tobytes())
    H = d.moe.hidden
    out = [bf(p + "input_layernorm.weight", [H], d.input_norm),
           bf(p + "post_attention_layernorm.weight", [H], d.post_attention_norm)]
    if d.full is not None:
        a = p + "self_attn."
        for name, m in (("q_proj", d.full.query), ("k_proj", d.full.key), ("v_proj", d.full.value),
                        ("o_proj", d.full.output)):
            out += ne_tensors(layer_index, a + name + ".weight", m)
        out += [bf(a + "q_norm.weight", [256], d.full.query_norm),
                bf(a + "k_norm.weight", [256], d.full.key_norm)]
    else:
        a = p + "linear_attn."
        L = d.linear
        for name, m in (("in_proj_qkv", L.qkv), ("in_proj_z", L.gate), ("out_proj", L.output)):
            out += ne_tensors(layer_index, a + name + ".weight", m)
        out += [bf(a + "in_proj_a.weight", [H, 32], L.alpha), bf(a + "in_proj_b.weight", [H, 32], L.beta),
                bf(a + "conv1d.weight", [4, 1, 8192], L.convolution), bf(a + "dt_bias", [32], L.alpha_bias),
                bf(a + "A_log", [32], L.a_log), bf(a + "norm.weight", [128], L.norm)]
    return out


def head_tensors(chunks, final_norm) -> List[Tuple[str, int, List[int], bytes]]:
    """Eight output-head chunks (adi_amd.synthetic.HeadChunk, chunk-local
    protected rows) and the final norm, as MachModel::head_chunk and
    final_norm_ read them (src/model.cpp:367-420, 604)."""
    out = []
    rows = chunks[0].rows
    for c, h in enumerate(chunks):
        p = f"mach.output.{c}.LMHEADCHUNK:{c * rows}:{(c + 1) * rows}|"
        out.append((p + "qp", T_I8, [h.columns // 8 * 5, h.rows], np.asarray(h.packed, np.uint8).tobytes()))
        out.append((p + "gscale", T_F16, [h.columns // 64, h.rows],
                    np.asarray(h.group_scale_f16, np.uint16).tobytes()))
        if h.protected_rows is not None and h.protected_rows.size:
            n = int(h.protected_rows.size)
            out.append((p + "prot_rows", T_I32, [n], np.asarray(h.protected_rows, np.uint32).tobytes()))
            out.append((p + "prot_dense", T_BF16, [h.columns, n], np.asarray(h.protected_bf16, np.uint16).tobytes()))
    out.append(("hf.model.language_model.norm.weight", T_BF16, [chunks[0].columns],
                np.asarray(final_norm, np.uint16).tobytes()))
    return out


def embedding_tensors(e) -> List[Tuple[str, int, List[int], bytes]]:
    """mach.embedding.* of a synthetic table (adi_amd.synthetic.Embedding),
    as MachModel::embedding reads them (src/model.cpp:316-363)."""
    n = int(e.exception_indexes.size)
    return [
        ("mach.embedding.q_packed", T_I8, [e.columns // 2, e.rows], np.asarray(e.packed, np.uint8).tobytes()),
        ("mach.embedding.mn", T_F16, [e.columns // 64, e.rows], np.asarray(e.minimum_f16, np.uint16).tobytes()),
        ("mach.embedding.mx", T_F16, [e.columns // 64, e.rows], np.asarray(e.maximum_f16, np.uint16).tobytes()),
        ("mach.embedding.exc_idx", T_I32, [n], np.asarray(e.exception_indexes, np.uint32).tobytes()),
        ("mach.embedding.exc_bits", T_I16, [n], np.asarray(e.exception_bf16, np.uint16).tobytes()),
    ]


def write_moe_checkpoint(path, layers, metadata=None, tensors=None) -> None:
    first = layers[0]
    md = metadata if metadata is not None else moe_metadata(len(layers), first.hidden,
                                                            first.expert_hidden, first.experts)
    ts = tensors if tensors is not None else moe_tensors(layers)
    with open(path, "wb") as f:
        f.write(gguf_bytes(md, ts))
