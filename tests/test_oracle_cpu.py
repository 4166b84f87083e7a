"""Pins the oracle (oracle/adi_oracle.c) before the GPU tests compare against it:

* against the golden vectors the compiled reference produced
  (tests/golden/golden.npz, written by tests/golden/make_golden.py);
* against the compiled reference itself where oracle/_ref is built;
* against what the mathematics fixes independently of the oracle's loops:
  bit-by-bit trellis windows, the closed-form state hash, brute-force
  dense reconstructions in float64, Sylvester Hadamard matrices, the
  renormalised softmax identity, permutation invariants, and the
  reference's own known answers (tests/kernels_test.cpp, tests/executor_test.cpp).
"""
import ctypes as C
import hashlib
import os

import numpy as np
import pytest
import scipy.linalg

import pyoracle as po
from adi_amd import synthetic as syn

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "golden.npz")


@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN, allow_pickle=False)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def f32p(a):
    return po.ptr(a, C.c_float)


def u16p(a):
    return po.ptr(a, C.c_uint16)


# ---- trellis walks ----------------------------------------------------------

def window_state(words, index, fresh, total_bits):
    """16-bit window read bit by bit, most significant bit of each u16 word
    first (tests/expert_trellis_test.cpp:17-33): shares no arithmetic with the
    oracle's shift-and-or walk."""
    value = 0
    for bit in range(16):
        pos = (index * fresh + bit) % total_bits
        value = (value << 1) | ((int(words[pos // 16]) >> (15 - pos % 16)) & 1)
    return value


def test_expert_walk_matches_golden_and_bitwise(oracle, golden):
    for words, want in zip(golden["expert_tiles"], golden["expert_states"]):
        got = np.zeros(32, np.uint16)
        w = np.ascontiguousarray(words)
        oracle.ao_expert_tile_states(u16p(w), u16p(got))
        assert np.array_equal(got, want)
        assert [window_state(w, i, 12, 384) for i in range(32)] == got.tolist()


def test_ne_walk_matches_golden_and_bitwise(oracle, golden):
    for words, want in zip(golden["ne_tiles"], golden["ne_states"]):
        got = np.zeros(128, np.uint16)
        w = np.ascontiguousarray(words)
        oracle.ao_ne_tile_states(u16p(w), u16p(got))
        assert np.array_equal(got, want)
        assert [window_state(w, i, 8, 1024) for i in range(128)] == got.tolist()


def test_walks_against_reference_random(oracle, ref):
    rng = np.random.default_rng(5)
    for _ in range(500):
        w = rng.integers(0, 65536, 24).astype(np.uint16)
        a, b, c = (np.zeros(32, np.uint16) for _ in range(3))
        oracle.ao_expert_tile_states(u16p(w), u16p(a))
        ref.ref_expert_tile_states(u16p(w), u16p(b))
        ref.ref_expert_row_states(u16p(w), u16p(c))
        assert np.array_equal(a, b) and np.array_equal(a, c)
        n = rng.integers(0, 65536, 64).astype(np.uint16)
        a, b, c = (np.zeros(128, np.uint16) for _ in range(3))
        oracle.ao_ne_tile_states(u16p(n), u16p(a))
        ref.ref_ne_tile_states(u16p(n), u16p(b))
        ref.ref_ne_row_states(u16p(n), u16p(c))
        assert np.array_equal(a, b) and np.array_equal(a, c)


# ---- codec tables -------------------------------------------------------------

def test_state_tables_match_golden(oracle, golden):
    et, nt = golden["expert_tlut"], golden["ne_tlut"]
    ev = np.zeros(65536 * 8, np.float32)
    nv = np.zeros(65536 * 2, np.float32)
    sv = np.zeros(2048, np.float32)
    oracle.ao_build_expert_state_values(f32p(et), f32p(ev))
    oracle.ao_build_ne_state_values(f32p(nt), f32p(nv))
    oracle.ao_build_ne_signed_tlut(f32p(nt), f32p(sv))
    assert hashlib.sha256(ev.tobytes()).hexdigest() == str(golden["expert_state_values_sha256"])
    assert hashlib.sha256(nv.tobytes()).hexdigest() == str(golden["ne_state_values_sha256"])
    s = golden["table_sample_states"]
    assert np.array_equal(bits(ev.reshape(-1, 8)[s]), bits(golden["expert_state_values_sample"]))
    assert np.array_equal(bits(nv.reshape(-1, 2)[s]), bits(golden["ne_state_values_sample"]))
    assert np.array_equal(bits(sv), bits(golden["ne_signed_tlut"]))


def test_state_hash_closed_form(oracle):
    """Every state's values are its TLUT row (s(s+1) mod 2^15, expert;
    bits 6..14, NE) rounded through f16, component 0 negated by bit 15
    (src/codec_cache.cpp:17-115), computed here in numpy."""
    rng = np.random.default_rng(11)
    et = rng.uniform(-1, 1, 32768 * 8).astype(np.float32)
    nt = rng.uniform(-1, 1, 1024).astype(np.float32)
    ev = np.zeros(65536 * 8, np.float32)
    nv = np.zeros(65536 * 2, np.float32)
    sv = np.zeros(2048, np.float32)
    oracle.ao_build_expert_state_values(f32p(et), f32p(ev))
    oracle.ao_build_ne_state_values(f32p(nt), f32p(nv))
    oracle.ao_build_ne_signed_tlut(f32p(nt), f32p(sv))
    s = np.arange(65536, dtype=np.uint64)
    p = (s * (s + 1)) & 0xFFFF
    neg = ((p >> 15) & 1).astype(bool)
    want = et.reshape(-1, 8)[(p & 0x7FFF).astype(np.int64)].astype(np.float16).astype(np.float32)
    want[neg, 0] = -want[neg, 0]
    assert np.array_equal(bits(ev.reshape(-1, 8)), bits(want))
    nw = nt.reshape(-1, 2)[((p >> 6) & 0x1FF).astype(np.int64)].astype(np.float16).astype(np.float32)
    nw[neg, 0] = -nw[neg, 0]
    assert np.array_equal(bits(nv.reshape(-1, 2)), bits(nw))
    # the signed table reproduces every state (tests/codec_cache_test.cpp:134-141)
    signed = sv.reshape(-1, 2)[((p >> 6) & 0x3FF).astype(np.int64)]
    assert np.array_equal(bits(signed), bits(nv.reshape(-1, 2)))
    # only even rows are reachable: 16384 of the 32768 expert rows
    rows = np.unique(p & 0x7FFF)
    assert rows.size == 16384 and np.all(rows % 2 == 0)


def test_wave_indexes_closed_form(oracle, golden):
    for key in golden.files:
        if not key.startswith("waves_"):
            continue
        r, c = (int(v) for v in key[6:].split("x"))
        got = np.zeros(r * c, np.uint16)
        assert oracle.ao_build_wave_indexes(r, c, u16p(got)) == 0
        assert np.array_equal(got, golden[key])
    for r in (1, 2, 3, 8, 32, 128):
        for c in (1, 2, 5, 32, 128):
            got = np.zeros(r * c, np.uint16)
            oracle.ao_build_wave_indexes(r, c, u16p(got))
            tr, tc = np.divmod(np.arange(r * c), c)
            d = tr + tc
            closed = np.where(d <= c - 1, r + c - 1 - d, r + c - 2 - d)
            assert np.array_equal(got, closed)
            assert (r - 1) not in set(got.tolist())  # slot R_t - 1 is never used


# ---- conversions ----------------------------------------------------------

def test_f16_conversions(oracle, golden):
    values = golden["f32_values"]
    got = np.array([oracle.ao_f32_to_f16(float(v)) for v in values], np.uint16)
    assert np.array_equal(got, golden["f32_to_f16"])
    finite = np.isfinite(values)
    with np.errstate(over="ignore"):
        assert np.array_equal(got[finite], values[finite].astype(np.float16).view(np.uint16))
    back = np.array([oracle.ao_f16_to_f32(h) for h in range(65536)], np.float32)
    assert hashlib.sha256(back.tobytes()).hexdigest() == str(golden["f16_to_f32_all_sha256"])
    ok = np.isfinite(back)
    assert np.array_equal(bits(back[ok]),
                          bits(np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
                               .astype(np.float32)[ok]))
    for v in (0.0, -0.0, 1.0, -2.0, 0.333251953125, 65504.0):  # tests/kernels_test.cpp:111-115
        assert oracle.ao_f16_to_f32(oracle.ao_f32_to_f16(v)) == v


# ---- Hadamard -------------------------------------------------------------

@pytest.mark.parametrize("n", [1, 2, 16, 512, 2048])
def test_hadamard_matches_sylvester(oracle, n):
    rng = np.random.default_rng(n)
    x = rng.standard_normal(n).astype(np.float32)
    y = x.copy()
    assert oracle.ao_hadamard(f32p(y), n) == 0
    want = scipy.linalg.hadamard(n) @ x.astype(np.float64) / np.sqrt(n)
    np.testing.assert_allclose(y, want, rtol=0, atol=1e-5 * max(1.0, np.abs(want).max()))
    z = y.copy()
    oracle.ao_hadamard(f32p(z), n)
    np.testing.assert_allclose(z, x, atol=1e-5)
    assert oracle.ao_hadamard(f32p(y), 3) != 0


# ---- projections -------------------------------------------------------------

def dense_expert(oracle, m):
    """W[r][c] = gamma(tile) * V(state)[component], assembled from the tile
    walk, then y = sv * H_R(W @ H_C(su * x)) in float64."""
    values = np.zeros((m.rows, m.columns), np.float32)
    s = po.expert_struct(m)
    assert oracle.ao_expert_decode_tiles(C.byref(s), f32p(values)) == 0
    waves = np.zeros((m.rows // 16) * (m.columns // 16), np.uint16)
    oracle.ao_build_wave_indexes(m.rows // 16, m.columns // 16, u16p(waves))
    gamma = syn.f16_to_f32(m.wave_gamma_f16)[waves.astype(np.int64)].reshape(m.rows // 16, m.columns // 16)
    return values.astype(np.float64) * np.kron(gamma, np.ones((16, 16)))


def reference_projection(W, x, su, sv):
    n_in, n_out = W.shape[1], W.shape[0]
    xh = scipy.linalg.hadamard(n_in) @ (x.astype(np.float64) * su).T / np.sqrt(n_in)
    z = W @ xh
    return ((scipy.linalg.hadamard(n_out) @ z / np.sqrt(n_out)).T * sv)


@pytest.mark.parametrize("rows,columns", [(16, 16), (64, 32), (32, 128)])
def test_expert_projection_brute_force_and_golden(oracle, golden, rows, columns):
    tag = f"expert_{rows}x{columns}"
    m = syn.ExpertMatrix(rows, columns, golden[f"{tag}_trellis"], golden[f"{tag}_su"],
                         golden[f"{tag}_sv"], golden[f"{tag}_gamma"], golden["expert_tlut"])
    x = golden[f"{tag}_x"]
    for b in (1, 2, 4):
        got = po.expert_matmul(oracle, m, x[:b])
        assert np.array_equal(bits(got), bits(golden[f"{tag}_y{b}"]))
    W = dense_expert(oracle, m)
    want = reference_projection(W, x, syn.f16_to_f32(m.su_f16), syn.f16_to_f32(m.sv_f16))
    got = po.expert_matmul(oracle, m, x)
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-5 * np.abs(want).max())


@pytest.mark.parametrize("rows,columns", [(16, 16), (64, 32), (32, 128)])
def test_ne_projection_brute_force_and_golden(oracle, golden, rows, columns):
    tag = f"ne_{rows}x{columns}"
    m = syn.NeMatrix(rows, columns, golden[f"{tag}_trellis"], golden[f"{tag}_su"], golden[f"{tag}_sv"],
                     float(golden[f"{tag}_scale"][0]), golden["ne_tlut"])
    x = golden[f"{tag}_x"]
    for b in (1, 3):
        got = po.ne_matmul(oracle, m, x[:b])
        assert np.array_equal(bits(got), bits(golden[f"{tag}_y{b}"]))
    W = np.zeros((rows, columns), np.float32)
    s = po.ne_struct(m)
    assert oracle.ao_ne_decode_tiles(C.byref(s), f32p(W)) == 0
    want = reference_projection(W.astype(np.float64), x, m.su.astype(np.float64), m.sv.astype(np.float64))
    got = po.ne_matmul(oracle, m, x)
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-5 * np.abs(want).max())


def test_projection_known_answers(oracle):
    """tests/kernels_test.cpp:32-137."""
    tlut = np.tile(np.arange(1, 9, dtype=np.float32), 32768)
    one = syn.f16_bits(np.ones(16, np.float32))
    m = syn.ExpertMatrix(16, 16, np.zeros(24, np.uint16), one, one,
                         syn.f16_bits(np.array([1.0, 2.0], np.float32)), tlut)
    y = po.expert_matmul(oracle, m, np.ones((1, 16), np.float32))[0]
    assert abs(y[0] - 32.0) < 1e-5 and np.all(np.abs(y[1:]) < 1e-5)
    ntlut = np.tile(np.array([1.0, 2.0], np.float32), 512)
    signs = np.ones(16, np.int8)
    n = syn.NeMatrix(16, 16, np.zeros(64, np.uint16), signs, signs, 0.5, ntlut)
    y = po.ne_matmul(oracle, n, np.ones((1, 16), np.float32))[0]
    assert abs(y[0] - 8.0) < 1e-5 and np.all(np.abs(y[1:]) < 1e-5)
    # batch == repeated matvec, bit for bit (tests/kernels_test.cpp:78-105)
    x = np.stack([np.ones(16, np.float32), -0.5 * np.ones(16, np.float32)])
    both = po.expert_matmul(oracle, m, x)
    assert np.array_equal(bits(both[1]), bits(po.expert_matmul(oracle, m, x[1:])[0]))


def test_projections_against_reference_full_size(oracle, ref):
    rng = syn.rng_for(0, 31)
    et, nt = syn.expert_tlut(rng), syn.ne_tlut(rng)
    for r, c in ((512, 2048), (2048, 512)):
        m = syn.expert_matrix(rng, r, c, et)
        x = syn.hidden_states(rng, 4, c)
        assert np.array_equal(bits(po.expert_matmul(oracle, m, x)),
                              bits(po.expert_matmul(ref, m, x, prefix="ref")))
    n = syn.ne_matrix(rng, 2048, 2048, nt)
    x = syn.hidden_states(rng, 4, 2048)
    for b in (1, 4):
        assert np.array_equal(bits(po.ne_matmul(oracle, n, x[:b])),
                              bits(po.ne_matmul(ref, n, x[:b], prefix="ref")))


# ---- ISA-ordered dots --------------------------------------------------------

def lane_model(w, x, lanes, fused):
    """The CPU lane order written out in numpy float32: lanes accumulate
    columns j, j+L, ..., then lanes are summed 0..L-1, then the tail
    (tests/simd_dispatch_test.cpp:83-108 states it for AVX2). Fused lanes
    round once per multiply-add (computed exactly in float64, then rounded:
    exact because a float32 product fits in float64)."""
    w = w.astype(np.float32)
    x = x.astype(np.float32)
    acc = np.zeros(lanes, np.float32)
    full = len(w) // lanes * lanes
    for k in range(0, full, lanes):
        if fused:
            acc = (acc.astype(np.float64) + w[k:k + lanes].astype(np.float64) * x[k:k + lanes]).astype(np.float32)
        else:
            acc = (acc + (w[k:k + lanes] * x[k:k + lanes])).astype(np.float32)
    s = np.float32(0.0)
    for v in acc:
        s = np.float32(s + v)
    for k in range(full, len(w)):
        if fused:
            s = np.float32(np.float64(s) + np.float64(w[k]) * np.float64(x[k]))
        else:
            s = np.float32(s + np.float32(w[k] * x[k]))
    return s


@pytest.mark.parametrize("isa", [1, 8, 16])
def test_bf16_dot_orders(oracle, golden, isa):
    w, x = golden["bf16_w"], golden["bf16_x"]
    got = po.bf16_matmul(oracle, w, x, isa=isa)
    assert np.array_equal(bits(got), bits(golden[f"bf16_y_isa{isa}"]))
    wf = syn.bf16_to_f32(w)
    for b in range(x.shape[0]):
        for r in range(w.shape[0]):
            assert bits(got[b, r]) == bits(lane_model(wf[r], x[b], isa, isa == 16))
    # tests/kernels_test.cpp:245-253
    kw = np.array([[0x3F80, 0x4000, 0x4040], [0x4080, 0x40A0, 0x40C0]], np.uint16)
    assert po.bf16_matmul(oracle, kw, np.array([[1, 2, 3]], np.float32), isa=isa).tolist() == [[14.0, 32.0]]


@pytest.mark.parametrize("isa", [1, 8, 16])
def test_head_orders(oracle, golden, isa):
    h = syn.HeadChunk(37, 128, golden["head_packed"], golden["head_scales"],
                      golden["head_protected_rows"], golden["head_protected_bf16"])
    got = po.head_matmul(oracle, h, golden["head_x"], isa=isa)
    assert np.array_equal(bits(got), bits(golden[f"head_y_isa{isa}"]))
    # every order is within fp32 rounding of the float64 dense product
    codes = np.zeros((37, 128))
    packed = h.packed.reshape(37, -1)
    for r in range(37):
        for blk in range(16):
            word = int.from_bytes(packed[r, blk * 5:blk * 5 + 5].tobytes(), "little")
            for i in range(8):
                codes[r, blk * 8 + i] = ((word >> (5 * i)) & 31) - 16
    W = codes * np.repeat(syn.f16_to_f32(h.group_scale_f16).reshape(37, 2), 64, axis=1)
    want = golden["head_x"].astype(np.float64) @ W.T
    mask = np.ones(37, bool)
    mask[h.protected_rows] = False
    np.testing.assert_allclose(got[:, mask], want[:, mask], rtol=0, atol=1e-4 * np.abs(want).max())


def test_head_known_answer(oracle):
    """tests/kernels_test.cpp:193-201."""
    h = syn.HeadChunk(1, 64, np.zeros(40, np.uint8), syn.f16_bits(np.array([0.5], np.float32)))
    for isa in (1, 8, 16):
        assert po.head_matmul(oracle, h, np.ones((1, 64), np.float32), isa=isa)[0, 0] == -512.0


def test_dots_against_reference(oracle, ref):
    rng = syn.rng_for(0, 77)
    h = syn.head_chunk(rng, 300, 2048, protected=2)
    x = syn.rms_normalized(syn.hidden_states(rng, 3, 2048))
    w = syn.bf16_bits_rne(rng.normal(0, 0.02, (256, 2048)).astype(np.float32))
    try:
        for isa in (1, 8, 16):
            ref.ref_force_isa_lanes(isa)
            assert np.array_equal(bits(po.head_matmul(oracle, h, x, isa=isa)),
                                  bits(po.head_matmul(ref, h, x, prefix="ref")))
            assert np.array_equal(bits(po.bf16_matmul(oracle, w, x, isa=isa)),
                                  bits(po.bf16_matmul(ref, w, x, prefix="ref")))
    finally:
        ref.ref_force_isa_lanes(0)


# ---- routing -----------------------------------------------------------------

def test_top_experts_golden_and_identity(oracle, golden):
    for row, we, ww in zip(golden["topk_logits"], golden["topk_experts"], golden["topk_weights"]):
        e, w = po.top_experts(oracle, row)
        assert np.array_equal(e, we) and np.array_equal(bits(w), bits(ww))
    # tests/executor_test.cpp:29-59
    logits = np.arange(16, dtype=np.float32)
    e, w = po.top_experts(oracle, logits)
    assert e.tolist() == list(range(15, 7, -1))
    p = np.exp(logits.astype(np.float64) - 15)
    p /= p.sum()
    np.testing.assert_allclose(w, p[e] / p[e].sum(), atol=2e-7)
    assert oracle.ao_top_experts(f32p(logits[:7].copy()), 7,
                                 po.ptr(np.zeros(8, np.uint32), C.c_uint32), f32p(np.zeros(8, np.float32))) != 0


def test_route_permutation_invariants(oracle):
    rng = np.random.default_rng(3)
    for batch, experts in ((1, 16), (7, 256), (128, 256), (512, 256)):
        logits = rng.normal(0, 1, (batch, experts)).astype(np.float32)
        r = po.moe_route(oracle, logits)
        e = r["route_expert"].reshape(batch, 8)
        assert np.array_equal(r["counts"], np.bincount(e.ravel(), minlength=experts))
        assert np.array_equal(r["offsets"], np.concatenate([[0], np.cumsum(r["counts"])]))
        # grouped order = slots sorted stably by expert
        order = np.argsort(e.ravel(), kind="stable")
        assert np.array_equal(r["grouped_batch"], (order // 8).astype(np.uint32))
        inverse = np.empty_like(order)
        inverse[order] = np.arange(order.size)
        assert np.array_equal(r["route_to_grouped"], inverse.astype(np.uint32))
        for b in range(batch):
            assert np.array_equal(e[b], po.top_experts(oracle, logits[b])[0])


# ---- MoE block ----------------------------------------------------------------

def golden_layer(golden):
    L = syn.MoeLayer(256, 64, 16, golden["moe_router"], golden["moe_shared_gate_w"],
                     expert_tlut=golden["expert_tlut"], ne_tlut=golden["ne_tlut"])
    for name, lst, (r, c) in (("gate", L.gate, (64, 256)), ("up", L.up, (64, 256)), ("down", L.down, (256, 64))):
        for e in range(16):
            lst.append(syn.ExpertMatrix(r, c, golden[f"moe_{name}_trellis"][e], golden[f"moe_{name}_su"][e],
                                        golden[f"moe_{name}_sv"][e], golden[f"moe_{name}_gamma"][e],
                                        golden["expert_tlut"]))
    for name, attr, (r, c) in (("sgate", "shared_gate", (64, 256)), ("sup", "shared_up", (64, 256)),
                               ("sdown", "shared_down", (256, 64))):
        setattr(L, attr, syn.NeMatrix(r, c, golden[f"moe_{name}_trellis"], golden[f"moe_{name}_su"],
                                      golden[f"moe_{name}_sv"], float(golden[f"moe_{name}_scale"][0]),
                                      golden["ne_tlut"]))
    return L


def test_moe_block_golden(oracle, golden):
    L = golden_layer(golden)
    x = golden["moe_x"]
    for b, use_bias in ((1, False), (5, False), (5, True)):
        tag = f"b{b}{'_bias' if use_bias else ''}"
        y, e, w = po.moe_forward(oracle, L, x[:b], isa=16,
                                 logit_bias=golden["moe_bias"] if use_bias else None)
        assert np.array_equal(bits(y), bits(golden[f"moe_y_{tag}"]))
        assert np.array_equal(e, golden[f"moe_experts_{tag}"])
        assert np.array_equal(bits(w), bits(golden[f"moe_weights_{tag}"]))


def test_moe_batch_equals_per_token(oracle, golden):
    """tests/moe_batch_test.cpp:138-149: each row of a batch gets exactly the
    routes, weights and output of the single-row call."""
    L = golden_layer(golden)
    x = golden["moe_x"]
    y, e, w = po.moe_forward(oracle, L, x, isa=16)
    for b in range(x.shape[0]):
        y1, e1, w1 = po.moe_forward(oracle, L, x[b:b + 1], isa=16)
        assert np.array_equal(bits(y[b]), bits(y1[0])) and np.array_equal(e[b], e1[0])


def test_moe_block_against_reference(oracle, ref):
    rng = syn.rng_for(2, 9)
    L = syn.moe_layer(rng, hidden=512, expert_hidden=128, experts=32)
    rl = po.RefMoeLayer(ref, L)
    lanes = ref.ref_selected_isa_lanes()
    for batch in (1, 3, 40):
        x = syn.hidden_states(rng, batch, 512)
        bias = syn.zipf_bias(rng, 32)
        a = po.moe_forward(oracle, L, x, isa=lanes, logit_bias=bias)
        b = rl.forward(x, bias)
        assert np.array_equal(bits(a[0]), bits(b[0]))
        assert np.array_equal(a[1], b[1]) and np.array_equal(bits(a[2]), bits(b[2]))
    rl.close()


def test_rms_norm_known_answer(oracle):
    """tests/kernels_test.cpp:310-321."""
    out = np.zeros(2, np.float32)
    x = np.array([3.0, 4.0], np.float32)
    assert oracle.ao_rms_norm(f32p(x), u16p(np.full(2, 0x3F80, np.uint16)), 2, 0.0, 0.0, f32p(out)) == 0
    np.testing.assert_allclose(out, [3 / np.sqrt(12.5), 4 / np.sqrt(12.5)], atol=1e-6)
    oracle.ao_rms_norm(f32p(x), u16p(np.zeros(2, np.uint16)), 2, 1.0, 0.0, f32p(out))
    np.testing.assert_allclose(out, [3 / np.sqrt(12.5), 4 / np.sqrt(12.5)], atol=1e-6)
