"""The attention half of a decode step on the GPU against the oracle
(pinned in test_attention_cpu.py): full GQA attention with its KV cache and
Gated DeltaNet with its convolution and recurrent state, token after token,
at hidden 256 and at the model's 2048. Outputs and states agree to float
rounding (the reductions run in another order): outputs within 1e-4 of the
largest output, caches and states elementwise within 1e-4 of their largest
value."""
import numpy as np
import pytest
import torch

import pyoracle as po
from adi_amd import hip
from adi_amd import synthetic as syn
from conftest import max_rel_error

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.fixture(scope="module", params=[256, 2048])
def full_layer(request, gpu):
    rng = syn.rng_for(40, request.param)
    tlut = syn.ne_tlut(rng)
    layer = syn.full_attention(rng, request.param, tlut)
    return layer, hip.upload_full_attention(gpu, layer, gpu.ne_codebook(tlut))


def test_full_attention_tokens(gpu, oracle, full_layer):
    layer, d = full_layer
    hidden, capacity = layer.hidden, 6
    held = po.FullAttentionStruct(layer)
    keys = np.zeros((capacity, 2, 256), np.float32)
    values = np.zeros_like(keys)
    dk = torch.zeros((capacity, 2, 256), dtype=torch.float32, device="cuda")
    dv = torch.zeros_like(dk)
    out = torch.empty(hidden, dtype=torch.float32, device="cuda")
    rng = syn.rng_for(41, hidden)
    for position in range(capacity):
        x = syn.rms_normalized(syn.hidden_states(rng, 1, hidden))[0]
        want = po.full_attention_forward(oracle, held, position, x, keys, values)
        hip.full_attention_forward(gpu, d, position, dev(x), out, dk, dv, capacity)
        got = out.cpu().numpy()
        assert max_rel_error(got, want) <= 1e-4, position
        for cache, ref in ((dk, keys), (dv, values)):
            c = cache.cpu().numpy()[:position + 1]
            assert np.max(np.abs(c - ref[:position + 1])) <= 1e-4 * np.max(np.abs(ref)), position


@pytest.mark.parametrize("position", [31, 300, 2500])
def test_full_attention_long_history(gpu, oracle, full_layer, position):
    """A history written straight into both caches, then one token: the
    history splits over 1, 10 and 64 blocks per head."""
    layer, d = full_layer
    hidden, capacity = layer.hidden, position + 1
    rng = syn.rng_for(42, position)
    keys = rng.normal(0.0, 1.0, (capacity, 2, 256)).astype(np.float32)
    values = rng.normal(0.0, 1.0, (capacity, 2, 256)).astype(np.float32)
    keys[position] = 0.0
    values[position] = 0.0
    dk, dv = dev(keys), dev(values)
    x = syn.rms_normalized(syn.hidden_states(rng, 1, hidden))[0]
    held = po.FullAttentionStruct(layer)
    want = po.full_attention_forward(oracle, held, position, x, keys, values)
    out = torch.empty(hidden, dtype=torch.float32, device="cuda")
    hip.full_attention_forward(gpu, d, position, dev(x), out, dk, dv, capacity)
    assert max_rel_error(out.cpu().numpy(), want) <= 1e-4
    assert np.max(np.abs(dk.cpu().numpy()[position] - keys[position])) <= 1e-4 * np.abs(keys[position]).max()


def test_full_attention_rejections(gpu, full_layer):
    layer, d = full_layer
    hidden = layer.hidden
    x = torch.zeros(hidden, dtype=torch.float32, device="cuda")
    out = torch.empty_like(x)
    cache = torch.zeros((2, 2, 256), dtype=torch.float32, device="cuda")
    with pytest.raises(hip.HipError, match="full attention state or input shape mismatch") as info:
        hip.full_attention_forward(gpu, d, 2, x, out, cache, cache.clone(), 2)
    assert info.value.status == hip.INVALID_ARGUMENT
    bad = hip.FullAttentionStruct.from_buffer_copy(d.struct)
    bad.key.rows = 256
    with pytest.raises(hip.HipError, match="full attention state or input shape mismatch"):
        hip.full_attention_forward(gpu, hip.DeviceFullAttention(bad, d.tensors), 0, x, out, cache,
                                   cache.clone(), 2)
    torch.cuda.synchronize()


@pytest.fixture(scope="module", params=[256, 2048])
def linear_layer(request, gpu):
    rng = syn.rng_for(43, request.param)
    tlut = syn.ne_tlut(rng)
    layer = syn.linear_attention(rng, request.param, tlut)
    return layer, hip.upload_linear_attention(gpu, layer, gpu.ne_codebook(tlut))


@pytest.mark.parametrize("isa", [1, 16])
def test_linear_attention_tokens(gpu, oracle, linear_layer, isa):
    layer, d = linear_layer
    hidden = layer.hidden
    held = po.LinearAttentionStruct(layer)
    conv = np.zeros(8192 * 3, np.float32)
    rec = np.zeros(32 * 128 * 128, np.float32)
    dconv = torch.zeros(8192 * 3, dtype=torch.float32, device="cuda")
    drec = torch.zeros(32 * 128 * 128, dtype=torch.float32, device="cuda")
    out = torch.empty(hidden, dtype=torch.float32, device="cuda")
    rng = syn.rng_for(44, hidden + isa)
    gpu.set_isa(isa)
    try:
        for step in range(5):
            x = syn.rms_normalized(syn.hidden_states(rng, 1, hidden))[0]
            want = po.linear_attention_forward(oracle, held, x, conv, rec, isa=isa)
            hip.linear_attention_forward(gpu, d, dev(x), out, dconv, drec)
            assert max_rel_error(out.cpu().numpy(), want) <= 1e-4, step
            # the convolution history holds the qkv projections
            c = dconv.cpu().numpy()
            assert np.max(np.abs(c - conv)) <= 1e-4 * np.max(np.abs(conv)), step
            r = drec.cpu().numpy()
            assert np.max(np.abs(r - rec)) <= 1e-4 * np.max(np.abs(rec)), step
    finally:
        gpu.set_isa(16)


def test_linear_attention_rejections(gpu, linear_layer):
    layer, d = linear_layer
    x = torch.zeros(layer.hidden, dtype=torch.float32, device="cuda")
    out = torch.empty_like(x)
    conv = torch.zeros(8192 * 3, dtype=torch.float32, device="cuda")
    rec = torch.zeros(32 * 128 * 128, dtype=torch.float32, device="cuda")
    bad = hip.LinearAttentionStruct.from_buffer_copy(d.struct)
    bad.gate.rows = 2048
    with pytest.raises(hip.HipError, match="linear attention input shape mismatch") as info:
        hip.linear_attention_forward(gpu, hip.DeviceLinearAttention(bad, d.tensors), x, out, conv, rec)
    assert info.value.status == hip.INVALID_ARGUMENT
    bad = hip.LinearAttentionStruct.from_buffer_copy(d.struct)
    bad.alpha.rows = 16
    with pytest.raises(hip.HipError, match="linear attention decay shape mismatch"):
        hip.linear_attention_forward(gpu, hip.DeviceLinearAttention(bad, d.tensors), x, out, conv, rec)
    torch.cuda.synchronize()


@pytest.mark.parametrize("count", [1, 2, 4, 40])
def test_projection_group_equals_separate_launches(gpu, count):
    """At hidden 2048 the query, key and value projections (Gated DeltaNet:
    qkv and gate) of 1-4 tokens run as one NE launch, and from 8 tokens they
    share one prologue launch (key and value one MFMA launch too); with the
    one-launch paths switched off they run one projection at a time. Outputs,
    caches and states are bit-identical, on two calls in a row (the tickets
    the first call cleared are reused)."""
    hidden = 2048
    rng = syn.rng_for(45, count)
    tlut = syn.ne_tlut(rng)
    full = hip.upload_full_attention(gpu, syn.full_attention(rng, hidden, tlut), gpu.ne_codebook(tlut))
    linear = hip.upload_linear_attention(gpu, syn.linear_attention(rng, hidden, tlut),
                                         gpu.ne_codebook(tlut))
    xs = [dev(syn.rms_normalized(syn.hidden_states(rng, count, hidden))) for _ in range(2)]
    capacity = 2 * count

    def run(fused):
        gpu.set_fused_decode(fused)
        try:
            keys = torch.zeros((capacity, 2, 256), dtype=torch.float32, device="cuda")
            values = torch.zeros_like(keys)
            conv = torch.zeros(8192 * 3, dtype=torch.float32, device="cuda")
            rec = torch.zeros(32 * 128 * 128, dtype=torch.float32, device="cuda")
            outs = []
            for step, x in enumerate(xs):
                fo = torch.full((count, hidden), float("nan"), dtype=torch.float32, device="cuda")
                lo = torch.full_like(fo, float("nan"))
                hip.full_attention_prefill(gpu, full, step * count, count, x, fo, keys, values,
                                           capacity)
                hip.linear_attention_prefill(gpu, linear, count, x, lo, conv, rec)
                outs += [fo, lo]
            gpu.synchronize()
            return [t.cpu().numpy() for t in outs + [keys, values, conv, rec]]
        finally:
            gpu.set_fused_decode(True)

    one, separate = run(True), run(False)
    for i, (a, b) in enumerate(zip(one, separate)):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), i
