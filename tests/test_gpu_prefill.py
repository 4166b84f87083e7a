"""Prefill chunks through attention and the decoder layer on the GPU against
the oracle's one-token path run over the same tokens in order (a chunk must
give what decoding its tokens one after another gives): full attention with
its KV cache, Gated DeltaNet with its convolution and recurrent state, and a
whole decoder layer, over two consecutive chunks; chunks of 64 tokens and
more take the MFMA projections. Outputs within 1e-3 of their largest value,
caches and states elementwise within 1e-3 of their largest value."""
import numpy as np
import pytest
import torch

import pyoracle as po
from adi_amd import hip
from adi_amd import synthetic as syn
from conftest import max_rel_error

pytestmark = pytest.mark.gpu

HIDDEN = 256
CHUNKS = [(0, 7), (7, 70)]  # (position, count): a short chunk, then one on the MFMA path


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def close(got, want, what):
    assert np.max(np.abs(got - want)) <= 1e-3 * np.max(np.abs(want)), what


@pytest.fixture(scope="module")
def tluts():
    rng = syn.rng_for(60, 0)
    return syn.expert_tlut(rng), syn.ne_tlut(rng)


def test_full_attention_prefill(gpu, oracle, tluts):
    rng = syn.rng_for(61, 0)
    layer = syn.full_attention(rng, HIDDEN, tluts[1])
    d = hip.upload_full_attention(gpu, layer, gpu.ne_codebook(tluts[1]))
    held = po.FullAttentionStruct(layer)
    capacity = sum(c for _, c in CHUNKS)
    keys = np.zeros((capacity, 2, 256), np.float32)
    values = np.zeros_like(keys)
    dk = torch.zeros((capacity, 2, 256), dtype=torch.float32, device="cuda")
    dv = torch.zeros_like(dk)
    for position, count in CHUNKS:
        x = syn.rms_normalized(syn.hidden_states(rng, count, HIDDEN))
        want = np.stack([po.full_attention_forward(oracle, held, position + b, x[b], keys, values)
                         for b in range(count)])
        out = torch.empty((count, HIDDEN), dtype=torch.float32, device="cuda")
        hip.full_attention_prefill(gpu, d, position, count, dev(x), out, dk, dv, capacity)
        assert max_rel_error(out.cpu().numpy(), want) <= 1e-3, (position, count)
        end = position + count
        close(dk.cpu().numpy()[:end], keys[:end], "keys")
        close(dv.cpu().numpy()[:end], values[:end], "values")


def test_linear_attention_prefill(gpu, oracle, tluts):
    rng = syn.rng_for(62, 0)
    layer = syn.linear_attention(rng, HIDDEN, tluts[1])
    d = hip.upload_linear_attention(gpu, layer, gpu.ne_codebook(tluts[1]))
    held = po.LinearAttentionStruct(layer)
    conv = np.zeros(8192 * 3, np.float32)
    rec = np.zeros(32 * 128 * 128, np.float32)
    dconv = torch.zeros(8192 * 3, dtype=torch.float32, device="cuda")
    drec = torch.zeros(32 * 128 * 128, dtype=torch.float32, device="cuda")
    for position, count in CHUNKS + [(77, 2)]:
        x = syn.rms_normalized(syn.hidden_states(rng, count, HIDDEN))
        want = np.stack([po.linear_attention_forward(oracle, held, x[b], conv, rec, isa=16)
                         for b in range(count)])
        out = torch.empty((count, HIDDEN), dtype=torch.float32, device="cuda")
        hip.linear_attention_prefill(gpu, d, count, dev(x), out, dconv, drec)
        assert max_rel_error(out.cpu().numpy(), want) <= 1e-3, (position, count)
        close(dconv.cpu().numpy(), conv, "convolution state")
        close(drec.cpu().numpy(), rec, "recurrent state")


@pytest.mark.parametrize("full", [False, True])
def test_prefill_layer(gpu, oracle, tluts, full):
    rng = syn.rng_for(63, int(full))
    etlut, ntlut = tluts
    layer = syn.decoder_layer(rng, full, HIDDEN, 64, 16, etlut, ntlut)
    d = hip.upload_decoder_layer(gpu, layer, gpu.expert_codebook(etlut), gpu.ne_codebook(ntlut))
    capacity = sum(c for _, c in CHUNKS)
    held = po.DecoderLayerStruct(layer, capacity=capacity)
    state, keep = hip.layer_state(full, capacity)
    for position, count in CHUNKS:
        h = syn.hidden_states(rng, count, HIDDEN)
        want = h.copy()
        for b in range(count):
            held.decode(oracle, position + b, want[b], isa=16)
        hidden = dev(h)
        hip.prefill_layer(gpu, d, position, count, hidden, state)
        assert max_rel_error(hidden.cpu().numpy(), want) <= 1e-3, (position, count)


def test_prefill_rejections(gpu, oracle, tluts):
    rng = syn.rng_for(64, 0)
    layer = syn.full_attention(rng, HIDDEN, tluts[1])
    d = hip.upload_full_attention(gpu, layer, gpu.ne_codebook(tluts[1]))
    x = torch.zeros((4, HIDDEN), dtype=torch.float32, device="cuda")
    out = torch.empty_like(x)
    cache = torch.zeros((5, 2, 256), dtype=torch.float32, device="cuda")
    with pytest.raises(hip.HipError, match="full attention state or input shape mismatch"):
        hip.full_attention_prefill(gpu, d, 2, 4, x, out, cache, cache.clone(), 5)  # 2 + 4 > 5
    with pytest.raises(hip.HipError, match="full attention state or input shape mismatch"):
        hip.full_attention_prefill(gpu, d, 0, 0, x, out, cache, cache.clone(), 5)
    torch.cuda.synchronize()


def test_chunk_rope_equals_single_tokens(gpu, tluts):
    """A chunk's keys are bit-identical with the keys of its tokens projected
    one at a time: the key projection runs each row in the same order at any
    batch below the MFMA path (8 rows), so the only difference could be the RoPE table,
    and the chunk's must be rope_table(position + b) itself (the reference
    builds its prefill table on the host, src/executor.cpp:1853-1866)."""
    rng = syn.rng_for(64, 0)
    layer = syn.full_attention(rng, HIDDEN, tluts[1])
    d = hip.upload_full_attention(gpu, layer, gpu.ne_codebook(tluts[1]))
    for position, count in ((0, 5), (1000, 7), (5000, 3)):
        capacity = position + count
        x = dev(syn.rms_normalized(syn.hidden_states(rng, count, HIDDEN)))
        chunk_keys = torch.zeros((capacity, 2, 256), dtype=torch.float32, device="cuda")
        chunk_values = torch.zeros_like(chunk_keys)
        out = torch.empty((count, HIDDEN), dtype=torch.float32, device="cuda")
        hip.full_attention_prefill(gpu, d, position, count, x, out, chunk_keys, chunk_values,
                                   capacity)
        one_keys = torch.zeros_like(chunk_keys)
        one_values = torch.zeros_like(chunk_keys)
        row = torch.empty(HIDDEN, dtype=torch.float32, device="cuda")
        for b in range(count):
            hip.full_attention_forward(gpu, d, position + b, x[b].contiguous(), row, one_keys,
                                       one_values, capacity)
        got = chunk_keys.cpu().numpy()[position:].view(np.uint32)
        want = one_keys.cpu().numpy()[position:].view(np.uint32)
        assert np.array_equal(got, want), (position, count)
