"""A hybrid stack decoding token by token on the GPU against the oracle:
the embedding row, four decoder layers (three Gated DeltaNet layers then a
full-attention layer, the reference's 3:1 pattern, src/executor.cpp:
1473-1529), the final RMS norm, the int5 head and the greedy choice, all on
device memory with one row of state per layer. The next token is the
oracle's (teacher forcing), so a near tie cannot fork the two sequences;
where the oracle's top two logits are clearly apart the GPU picks the same
token. Hidden rows and logits agree within 1e-3 of their largest value."""
import numpy as np
import pytest
import torch

import pyoracle as po
from adi_amd import hip
from adi_amd import synthetic as syn
from conftest import max_rel_error

pytestmark = pytest.mark.gpu

HIDDEN, EXPERT_HIDDEN, EXPERTS, VOCAB, STEPS = 256, 64, 16, 512, 8


@pytest.fixture(scope="module")
def stack(gpu):
    rng = syn.rng_for(50, 0)
    etlut, ntlut = syn.expert_tlut(rng), syn.ne_tlut(rng)
    layers = [syn.decoder_layer(rng, i % 4 == 3, HIDDEN, EXPERT_HIDDEN, EXPERTS, etlut, ntlut)
              for i in range(4)]
    emb = syn.embedding(rng, VOCAB, HIDDEN, exceptions=20)
    head = syn.head_chunk(rng, VOCAB, HIDDEN)
    final_norm = syn.bf16_bits_rne(rng.normal(0.0, 0.1, HIDDEN).astype(np.float32))
    ebook, nbook = gpu.expert_codebook(etlut), gpu.ne_codebook(ntlut)
    device = dict(
        layers=[hip.upload_decoder_layer(gpu, L, ebook, nbook) for L in layers],
        emb=hip.upload_embedding(gpu, emb), head=hip.upload_head(gpu, head),
        final_norm=gpu.to_device(final_norm))
    return layers, emb, head, final_norm, device


def test_stack_decode_matches_oracle(gpu, oracle, stack):
    layers, emb, head, final_norm, d = stack
    held = [po.DecoderLayerStruct(L, capacity=STEPS) for L in layers]
    states = [hip.layer_state(L.full is not None, STEPS) for L in layers]
    hidden = torch.empty((1, HIDDEN), dtype=torch.float32, device="cuda")
    normed = torch.empty_like(hidden)
    logits = torch.empty((1, VOCAB), dtype=torch.float32, device="cuda")
    token = 7
    agreed = 0
    for step in range(STEPS):
        h = po.embedding_rows(oracle, emb, [token])[0]
        hip.embedding_rows(gpu, d["emb"], torch.tensor([token], dtype=torch.int32, device="cuda"), 1,
                           hidden)
        for i, (L, held_layer, (state, _)) in enumerate(zip(d["layers"], held, states)):
            held_layer.decode(oracle, step, h, isa=16)
            hip.decode_layer(gpu, L, step, hidden, state)
            assert max_rel_error(hidden.cpu().numpy()[0], h) <= 1e-3, (step, i)
        n = np.zeros(HIDDEN, np.float32)
        assert oracle.ao_rms_norm(po.ptr(h, po.C.c_float), po.ptr(final_norm, po.C.c_uint16), HIDDEN,
                                  1.0, 1e-6, po.ptr(n, po.C.c_float)) == 0
        want = po.head_matmul(oracle, head, n[None, :], isa=16)[0]
        gpu.check(gpu.lib.adi_hip_rms_norm(gpu.handle, hidden.data_ptr(), d["final_norm"].data_ptr(),
                                           HIDDEN, 1, 1.0, 1e-6, normed.data_ptr()))
        hip.head_matmul(gpu, d["head"], normed, 1, logits)
        got = logits.cpu().numpy()[0]
        assert max_rel_error(got, want) <= 1e-3, step
        top2 = np.sort(want)[-2:]
        if top2[1] - top2[0] > 2e-3 * np.max(np.abs(want)):
            assert int(np.argmax(got)) == int(np.argmax(want)), step
            agreed += 1
        token = int(np.argmax(want))
    assert agreed >= STEPS // 2


def test_decode_layer_rejections(gpu, stack):
    _, _, _, _, d = stack
    hidden = torch.zeros((1, HIDDEN), dtype=torch.float32, device="cuda")
    state, _ = hip.layer_state(True, 2)
    full = [L for L in d["layers"] if L.struct.full_attention][0]
    with pytest.raises(hip.HipError, match="full attention state or input shape mismatch"):
        hip.decode_layer(gpu, full, 2, hidden, state)  # position past the cache
    torch.cuda.synchronize()


@pytest.fixture(scope="module")
def wide_layers(gpu):
    """A Gated DeltaNet and a full-attention layer of the 40-layer stack's
    geometry (hidden 2048, 256 experts)."""
    g = syn.StackGeometry()
    etlut, ntlut = syn.stack_codebooks()
    ebook, nbook = gpu.expert_codebook(etlut), gpu.ne_codebook(ntlut)
    return [hip.upload_decoder_layer(gpu, syn.stack_layer(g, i, etlut, ntlut), ebook, nbook)
            for i in (0, 3)]


@pytest.mark.parametrize("count", [1, 2, 4, 40])
def test_layer_norms_folded_equal_separate_launches(gpu, wide_layers, count):
    """At hidden 2048 a layer of 1-4 tokens runs its input RMS norm (with the
    residual add) inside its first attention projection launch and the
    post-attention norm inside its output projection launch; at any token
    count the Gated DeltaNet's alpha and beta matmuls are one launch (the
    small-batch kernel below 32 tokens, the register-tiled one from 32). With
    the one-launch paths off they are launches of their own. Hidden rows and
    every state are bit-identical over three steps of both layers."""
    rng = syn.rng_for(51, count)
    x0 = syn.hidden_states(rng, count, 2048)

    def run(fused):
        gpu.set_fused_decode(fused)
        try:
            hidden = gpu.to_device(x0.copy())
            states = [hip.layer_state(i == 1, 3 * count) for i in range(2)]
            for step in range(3):
                for layer, (state, _) in zip(wide_layers, states):
                    if count == 1:
                        hip.decode_layer(gpu, layer, step, hidden, state)
                    else:
                        hip.prefill_layer(gpu, layer, step * count, count, hidden, state)
            gpu.synchronize()
            return [hidden.cpu().numpy()] + [t.cpu().numpy() for _, keep in states for t in keep]
        finally:
            gpu.set_fused_decode(True)

    one, separate = run(True), run(False)
    for i, (a, b) in enumerate(zip(one, separate)):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), i
