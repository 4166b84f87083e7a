"""The GGUF reader and the MoE tensor checks without a GPU (host code of
libadi_hip.so): the reference's own container test (tests/gguf_test.cpp),
every rejection rule of GgufFile::GgufFile (src/gguf.cpp:232-330), and the
packed-tensor mapping and validation of MachModel (src/model.cpp:180-224,
267-314, 431-533, 808-880) on synthetic checkpoints."""
import struct

import numpy as np
import pytest

from adi_amd import hip
from adi_amd import synthetic as syn

import gguf_fixture as gf


def write(path, data: bytes):
    path.write_bytes(data)
    return str(path)


def open_fails(path, match):
    with pytest.raises(hip.HipError) as info:
        hip.Gguf(path)
    assert info.value.status == hip.INVALID_ARGUMENT
    assert match in str(info.value), str(info.value)


def test_reference_fixture(tmp_path):
    # tests/gguf_test.cpp:133-168
    with hip.Gguf(write(tmp_path / "fixture.gguf", gf.reference_fixture())) as f:
        assert f.version == 3
        assert f.alignment == 32
        assert f.metadata_count == 5
        assert f.tensor_count == 1
        assert f.integer("general.alignment") == 32
        assert f.string("general.architecture") == "adi"
        assert f.boolean("adi.additive") is True
        assert f.string_array("tokenizer.ggml.tokens") == ["hello", "world"]
        assert f.integer_array("tokenizer.ggml.token_type") == [1, 3]
        info, data = f.tensor("test.weight")
        assert list(info.dimensions[:info.dimension_count]) == [2, 2]
        assert info.type == hip.GGML_F32
        assert info.elements == 4 and info.bytes == 16
        assert data.tolist() == [1.0, 2.0, 3.0, 4.0]
        assert f.tensor("missing.weight") is None
        assert f.integer("missing.key") is None


def test_unicode_path(tmp_path):
    path = tmp_path / "adi-gguf-模型-test.gguf"
    with hip.Gguf(write(path, gf.reference_fixture())) as f:
        assert f.tensor("test.weight") is not None


def test_truncated_file_is_rejected(tmp_path):
    data = gf.reference_fixture()
    open_fails(write(tmp_path / "bad.gguf", data[:-1]), "outside file")
    open_fails(write(tmp_path / "tiny.gguf", data[:20]), "too small")
    open_fails(write(tmp_path / "head.gguf", data[:40]), "truncated")


def test_missing_file(tmp_path):
    open_fails(str(tmp_path / "absent.gguf"), "cannot open")


@pytest.mark.parametrize("case, match", [
    ("magic", "bad magic"),
    ("version", "only version 3"),
    ("duplicate_key", "duplicate metadata key"),
    ("duplicate_tensor", "duplicate tensor name"),
    ("no_dims", "unsupported dimension count"),
    ("five_dims", "unsupported dimension count"),
    ("zero_extent", "invalid tensor dimensions"),
    ("tensor_type", "unsupported tensor type"),
    ("alignment", "power of two"),
    ("value_type", "unknown metadata value type"),
    ("nested", "nested too deeply"),
    ("offset", "outside file"),
])
def test_malformed_files_are_rejected(tmp_path, case, match):
    md = [("general.alignment", gf.U32, 32), ("general.architecture", gf.STRING, "adi")]
    data4 = np.arange(4, dtype=np.float32).tobytes()
    ts = [("a.weight", gf.T_F32, [2, 2], data4)]
    kw = {}
    if case == "magic":
        kw["magic"] = 0x46554746
    elif case == "version":
        kw["version"] = 2
    elif case == "duplicate_key":
        md.append(("general.architecture", gf.STRING, "again"))
    elif case == "duplicate_tensor":
        ts.append(("a.weight", gf.T_F32, [4], data4))
    elif case == "no_dims":
        ts = [("a.weight", gf.T_F32, [], data4)]
    elif case == "five_dims":
        ts = [("a.weight", gf.T_F32, [1, 1, 1, 2, 2], data4)]
    elif case == "zero_extent":
        ts = [("a.weight", gf.T_F32, [0, 4], data4)]
    elif case == "tensor_type":
        ts = [("a.weight", 2, [2, 2], data4)]  # a GGML block-quant type
    elif case == "alignment":
        md[0] = ("general.alignment", gf.U32, 24)
    elif case == "value_type":
        md.append(("bad.type", 13, 0))
    elif case == "nested":
        value = (gf.U8, [1])
        for _ in range(10):
            value = (gf.ARRAY, [value])
        md.append(("deep", gf.ARRAY, value))
    data = None
    if case == "value_type":
        # a value type the writer cannot encode: patch it in after the fact
        data = gf.gguf_bytes(md[:2] + [("bad.type", gf.U8, 0)], ts)
        key = gf._string("bad.type")
        at = data.index(key) + len(key)
        data = data[:at] + struct.pack("<I", 13) + data[at + 4:]
    elif case == "offset":
        data = gf.gguf_bytes(md, ts)
        data = data[:-8]  # the tensor's bytes end past the file
    else:
        data = gf.gguf_bytes(md, ts, **kw)
    open_fails(write(tmp_path / f"{case}.gguf", data), match)


def test_metadata_conversions(tmp_path):
    md = [("neg", gf.I32, -5), ("pos", gf.I16, 7), ("f", gf.F32, 1.5), ("d", gf.F64, 1e-6),
          ("flag", gf.BOOL, 0), ("u8", gf.U8, 200), ("big", gf.U64, 1 << 40),
          ("strs", gf.ARRAY, (gf.STRING, ["a", "bc", ""])), ("ints", gf.ARRAY, (gf.I32, [1, 2]))]
    with hip.Gguf(write(tmp_path / "m.gguf", gf.gguf_bytes(md, []))) as f:
        assert f.integer("neg") is None          # negative signed: no integer (src/gguf.cpp:444-459)
        assert f.integer("pos") == 7
        assert f.integer("f") is None
        assert f.number("f") == 1.5 and f.number("d") == 1e-6 and f.number("pos") == 7.0
        assert f.boolean("flag") is False and f.boolean("pos") is None
        assert f.integer("u8") == 200 and f.integer("big") == 1 << 40
        assert f.string("pos") is None
        assert f.string_array("strs") == ["a", "bc", ""]
        assert f.string_array("ints") == []      # not an array of strings
        assert f.integer_array("ints") == []     # signed elements are not read (src/gguf.cpp:533-566)
        assert f.tensor_count == 0


# ---- the packed MoE tensors ---------------------------------------------------

def small_layer(seed=0, hidden=256, expert_hidden=64, experts=32):
    return syn.moe_layer(syn.rng_for(9, seed), hidden=hidden, expert_hidden=expert_hidden,
                         experts=experts)


@pytest.fixture(scope="module")
def layers():
    first = small_layer(0, experts=64)
    second = small_layer(1, experts=64)
    return [first, second]


@pytest.fixture()
def checkpoint(tmp_path, layers):
    path = str(tmp_path / "moe.gguf")
    gf.write_moe_checkpoint(path, layers)
    return path


def test_moe_geometry_and_layer_checks(checkpoint, layers):
    with hip.Gguf(checkpoint) as f:
        g = f.moe_geometry()
        assert (g.layers, g.hidden, g.experts, g.active_experts, g.expert_hidden, g.shared_hidden) == \
            (2, 256, 64, 8, 64, 64)
        f.check_moe_layer(0)
        f.check_moe_layer(1)
        with pytest.raises(hip.HipError, match="layer index is out of range"):
            f.check_moe_layer(2)


def test_chunk_tensors_hold_the_experts_end_to_end(checkpoint, layers):
    # expert e's slice of its 32-expert chunk (src/model.cpp:472-533)
    L = layers[1]
    with hip.Gguf(checkpoint) as f:
        for e in (0, 31, 32, 63):
            chunk, offset = e // 32 * 32, e % 32
            for name, mats in (("gate", L.gate), ("down", L.down)):
                m = mats[e]
                info, words = f.tensor(f"mach.expert.1.e{chunk}.{name}.trellis")
                n = m.trellis.size
                assert np.array_equal(words[offset * n:(offset + 1) * n], m.trellis)
                info, su = f.tensor(f"mach.expert.1.e{chunk}.{name}.su")
                assert np.array_equal(su[offset * m.columns:(offset + 1) * m.columns], m.su_f16)
        info, router = f.tensor("hf.model.language_model.layers.1.mlp.gate.weight")
        assert list(info.dimensions[:2]) == [256, 64]
        assert np.array_equal(router.reshape(64, 256), L.router_bf16)


def mutate(layers, name=None, metadata=None, drop=None, data=None, dims=None):
    md = gf.moe_metadata(len(layers), layers[0].hidden, layers[0].expert_hidden, layers[0].experts,
                         **(metadata or {}))
    ts = []
    for t in gf.moe_tensors(layers):
        if t[0] == drop:
            continue
        if t[0] == name:
            t = (t[0], t[1], dims if dims is not None else t[2], data if data is not None else t[3])
        ts.append(t)
    return md, ts


TRELLIS = "mach.expert.0.e32.up.trellis"
SU = "mach.expert.0.e0.down.su"
NE_SU = "mach.ne.0.model.language_model.layers.0.mlp.shared_expert.up_proj.weight|SU"
NE_SCALE = "mach.ne.0.model.language_model.layers.0.mlp.shared_expert.down_proj.weight|Wscale"
ROUTER = "hf.model.language_model.layers.0.mlp.gate.weight"


def bad_su(layers):
    m = layers[0].down[0]
    v = np.concatenate([x.su_f16 for x in layers[0].down[:32]]).astype(np.uint16)
    v[5] = 0x7C00  # +inf
    return v.tobytes()


def bad_signs(layers):
    v = np.asarray(layers[0].shared_up.su, np.int8).copy()
    v[3] = 0
    return v.tobytes()


def bad_router(layers):
    v = np.asarray(layers[0].router_bf16, np.uint16).copy().reshape(-1)
    v[100] = 0x7FC0  # NaN
    return v.tobytes()


@pytest.mark.parametrize("change, match", [
    (dict(drop=TRELLIS), "missing or invalid tensor 'mach.expert.0.e32.up.trellis'"),
    (dict(name=TRELLIS, dims=[24, 64, 16]), "unexpected tensor shape"),
    (dict(name=SU, data="bad_su"), "nonfinite tensor 'mach.expert.0.e0.down.su'"),
    (dict(name=NE_SU, data="bad_signs"), "invalid non-expert sign tensor"),
    (dict(name=NE_SCALE, data=np.array([-1.0], np.float32).tobytes()), "unexpected non-expert shape"),
    (dict(name=ROUTER, data="bad_router"), "nonfinite tensor"),
    (dict(metadata={"adi__expert_codec": (gf.STRING, "other")}), "unsupported metadata 'adi.expert_codec'"),
    (dict(metadata={"qwen35moe__expert_used_count": (gf.U32, 4)}), "unsupported MoE geometry"),
    (dict(metadata={"adi__format_version": (gf.U32, 2)}), "unsupported additive format"),
    (dict(metadata={"qwen35moe__expert_count": None}), "qwen35moe.expert_count"),
    (dict(drop="mach.tlut.ne.tlut"), "mach.tlut.ne.tlut"),
])
def test_malformed_layers_are_rejected(tmp_path, layers, change, match):
    change = dict(change)
    if isinstance(change.get("data"), str):
        change["data"] = globals()[change["data"]](layers)
    md, ts = mutate(layers, **change)
    path = str(tmp_path / "bad.gguf")
    gf.write_moe_checkpoint(path, layers, md, ts)
    with hip.Gguf(path) as f:
        with pytest.raises(hip.HipError) as info:
            f.moe_geometry()
            f.check_moe_layer(0)
        assert info.value.status == hip.INVALID_ARGUMENT
        assert match in str(info.value), str(info.value)


# ---- the embedding table --------------------------------------------------------

def embedding_checkpoint(tmp_path, layers, e, change=None):
    ts = gf.moe_tensors(layers) + gf.embedding_tensors(e)
    if change:
        name, data = change
        ts = [(t[0], t[1], t[2], data) if t[0] == name else t for t in ts]
    md = gf.moe_metadata(len(layers), layers[0].hidden, layers[0].expert_hidden, layers[0].experts)
    path = str(tmp_path / "emb.gguf")
    gf.write_moe_checkpoint(path, layers, md, ts)
    return path


def test_embedding_tensors_round_trip(tmp_path, layers):
    e = syn.embedding(syn.rng_for(9, 7), 300, 256, exceptions=50)
    with hip.Gguf(embedding_checkpoint(tmp_path, layers, e)) as f:
        info, packed = f.tensor("mach.embedding.q_packed")
        assert list(info.dimensions[:2]) == [128, 300]
        assert np.array_equal(packed.view(np.uint8), e.packed)
        info, idx = f.tensor("mach.embedding.exc_idx")
        assert np.array_equal(idx.view(np.uint32), e.exception_indexes)


def test_reference_reader_agrees(tmp_path, layers):
    """The compiled GgufFile accepts and rejects the same files as this
    reader (where the reference is built here)."""
    import pyoracle as po
    if not po.ref_available():
        pytest.skip("oracle/_ref is not built here")
    ref = po.load_ref()
    good = embedding_checkpoint(tmp_path, layers, syn.embedding(syn.rng_for(9, 8), 64, 256, 8))
    with hip.Gguf(good) as f:
        assert po.ref_gguf_summary(ref, good) == (f.tensor_count, f.metadata_count, f.alignment)
    data = gf.reference_fixture()
    for i, bad in enumerate([data[:-1], data[:20], data[:40], b"GGUX" + data[4:],
                             data[:4] + struct.pack("<I", 2) + data[8:]]):
        path = write(tmp_path / f"bad{i}.gguf", bad)
        assert po.ref_gguf_summary(ref, path) is None
        with pytest.raises(hip.HipError):
            hip.Gguf(path)


def bad_exception_order(e):
    v = e.exception_indexes.copy()
    v[3], v[4] = v[4], v[3]
    return v.astype(np.uint32).tobytes()


def bad_minimum(e):
    v = e.minimum_f16.copy()
    v[10] = syn.f16_bits(np.array([1.0], np.float32))[0]  # above its maximum
    return v.astype(np.uint16).tobytes()


def bad_exception_value(e):
    v = e.exception_bf16.copy()
    v[2] = 0x7F80  # +inf
    return v.astype(np.uint16).tobytes()


@pytest.mark.parametrize("name, make, match", [
    ("mach.embedding.exc_idx", bad_exception_order, "malformed embedding tensors"),
    ("mach.embedding.mn", bad_minimum, "minimum exceeds maximum"),
    ("mach.embedding.exc_bits", bad_exception_value, "nonfinite tensor 'mach.embedding.exc_bits'"),
])
def test_malformed_embedding_is_rejected(tmp_path, layers, name, make, match):
    # src/model.cpp:342-363, 836-849
    e = syn.embedding(syn.rng_for(9, 9), 64, 256, exceptions=20)
    with hip.Gguf(embedding_checkpoint(tmp_path, layers, e)) as f:
        f.check_embedding()
    path = embedding_checkpoint(tmp_path, layers, e, (name, make(e)))
    with hip.Gguf(path) as f:
        with pytest.raises(hip.HipError) as info:
            f.check_embedding()
        assert info.value.status == hip.INVALID_ARGUMENT
        assert match in str(info.value), str(info.value)


# ---- decoder layers and the output head ----------------------------------------

def decoder_checkpoint_tensors(hidden=256, vocabulary=1024):
    """Checkpoint layers 0 (Gated DeltaNet) and 3 (full attention) of a
    four-layer model, with the embedding, the eight head chunks (protected
    rows in two of them) and the final norm."""
    rng = syn.rng_for(9, 40)
    etlut, ntlut = syn.expert_tlut(rng), syn.ne_tlut(rng)
    layers = {i: syn.decoder_layer(syn.rng_for(9, 41 + i), (i + 1) % 4 == 0, hidden, 64, 32, etlut, ntlut)
              for i in (0, 3)}
    chunks = [syn.head_chunk(syn.rng_for(9, 50 + c), vocabulary // 8, hidden, protected=3 if c in (2, 7) else 0)
              for c in range(8)]
    norm = syn.bf16_bits_rne(rng.normal(0.0, 0.1, hidden).astype(np.float32))
    md = gf.moe_metadata(4, hidden, 64, 32)
    ts = gf.moe_tensors([layers[0].moe, layers[3].moe], indices=[0, 3])
    for i in (0, 3):
        ts += gf.attention_tensors(i, layers[i])
    ts += gf.embedding_tensors(syn.embedding(syn.rng_for(9, 60), vocabulary, hidden, exceptions=4))
    ts += gf.head_tensors(chunks, norm)
    return md, ts, layers, chunks, norm


@pytest.fixture(scope="module")
def decoder_parts():
    return decoder_checkpoint_tensors()[:2]


def decoder_file(tmp_path, parts, drop=None, replace=None):
    md, ts = parts
    out = []
    for t in ts:
        if t[0] == drop:
            continue
        if replace is not None and t[0] in replace:
            name, kind, dims, data = t
            new = replace[t[0]]
            out.append((name, new.get("type", kind), new.get("dims", dims), new.get("data", data)))
            continue
        out.append(t)
    return write(tmp_path / "decoder.gguf", gf.gguf_bytes(md, out))


def test_decoder_layer_and_head_checks(tmp_path, decoder_parts):
    with hip.Gguf(decoder_file(tmp_path, decoder_parts)) as f:
        f.check_decoder_layer(0)
        f.check_decoder_layer(3)
        with pytest.raises(hip.HipError, match="missing or invalid tensor"):
            f.check_decoder_layer(1)  # not in this file
        with pytest.raises(hip.HipError, match="layer index is out of range"):
            f.check_decoder_layer(4)
        f.check_head()


def tensor_bytes(parts, name):
    return next(t for t in parts[1] if t[0] == name)


Q = "mach.ne.3.model.language_model.layers.3.self_attn.q_proj.weight|"
QKV = "mach.ne.0.model.language_model.layers.0.linear_attn.in_proj_qkv.weight|"
LIN = "hf.model.language_model.layers.0.linear_attn."


@pytest.mark.parametrize("layer, change, match", [
    (3, {"drop": Q + "SV"}, "missing or invalid tensor"),
    (3, {"replace": {Q + "SV": {"dims": [4096], "data": b"\x01" * 4096}}}, "unexpected tensor shape"),
    (0, {"replace": {QKV + "SU": {"data": b"\x01" * 255 + b"\x00"}}}, "invalid non-expert sign tensor"),
    (0, {"replace": {QKV + "Wscale": {"data": np.array([-1.0], np.float32).tobytes()}}},
     "unexpected non-expert shape"),
    (0, {"drop": LIN + "conv1d.weight"}, "missing or invalid tensor"),
    (0, {"replace": {LIN + "conv1d.weight": {"dims": [4, 8192]}}}, "unexpected tensor shape"),
    (0, {"replace": {LIN + "A_log": {"data": np.full(32, 0x7F80, np.uint16).tobytes()}}}, "nonfinite tensor"),
    (3, {"replace": {"hf.model.language_model.layers.3.self_attn.k_norm.weight":
                     {"type": gf.T_F16}}}, "missing or invalid tensor"),
    (3, {"drop": "hf.model.language_model.layers.3.post_attention_layernorm.weight"}, "missing or invalid tensor"),
])
def test_decoder_layer_rejections(tmp_path, decoder_parts, layer, change, match):
    with hip.Gguf(decoder_file(tmp_path, decoder_parts, **change)) as f:
        with pytest.raises(hip.HipError, match=match):
            f.check_decoder_layer(layer)


H2 = "mach.output.2.LMHEADCHUNK:256:384|"
H5 = "mach.output.5.LMHEADCHUNK:640:768|"


@pytest.mark.parametrize("change, match", [
    ({"drop": H2 + "prot_dense"}, "incomplete protected output rows"),
    ({"replace": {H2 + "prot_rows": {"data": np.array([0, 5, 128], np.uint32).tobytes()}}},
     "protected output row is out of range"),
    ({"replace": {H5 + "gscale": {"data": np.full(4 * 128, 0x7C00, np.uint16).tobytes()}}},
     "nonfinite tensor 'output head scale'"),
    ({"drop": H5 + "qp"}, "missing or invalid tensor"),
    ({"drop": "hf.model.language_model.norm.weight"}, "missing or invalid tensor"),
    ({"replace": {H5 + "qp": {"dims": [160, 64]}}}, "unexpected tensor shape"),
])
def test_head_rejections(tmp_path, decoder_parts, change, match):
    with hip.Gguf(decoder_file(tmp_path, decoder_parts, **change)) as f:
        with pytest.raises(hip.HipError, match=match):
            f.check_head()
