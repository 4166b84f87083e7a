"""The full hybrid stack on the GPU against the oracle's token-by-token run
(tests/golden/stack40.npz, written by tests/golden/make_stack40.py): 40
layers at hidden 2048, every fourth full GQA attention and the others Gated
DeltaNet, each with the 256-expert top-8 MoE block and a shared expert, the
151,936-token embedding and int5 head (adi_amd.synthetic.StackGeometry).

The device prefills the 256-token prompt in two chunks of 128
(adi_hip_prefill_layer per layer: batched norms, projections on the MFMA
path, the expert-sorted grouped MoE GEMMs; src/executor.cpp:1827-2101), then
runs 64 decode steps (adi_hip_decode_layer, src/executor.cpp:1473-1529),
fed the oracle's greedy tokens (teacher forcing, so a near tie cannot fork
the two runs). Checked, each within 1e-3 of the largest value:
  * the last prompt token's row after every layer;
  * the logits after the prompt and after the last decode step;
  * every layer's two state tensors (KV cache, or convolution and recurrent
    state) at 2,048 seeded elements each, against their largest value;
and the device's greedy token equals the oracle's at every step whose top-two
logit margin exceeds twice that tolerance (there the 1e-3 agreement of the
logits fixes the order). decoder_state_checksum (src/main.cpp:105-117) is
printed for both runs; the two differ in the last bits of the floats, so the
digests are reported, not compared."""
import os
import sys

import numpy as np
import pytest
import torch

import pyoracle as po
from adi_amd import hip
from adi_amd import synthetic as syn
from conftest import error_report, max_rel_error

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_stack40 as fixture  # noqa: E402

pytestmark = pytest.mark.gpu
FIXTURE = os.path.join(HERE, "golden", "stack40.npz")
TOL = 1e-3


@pytest.mark.timeout(900)
@pytest.mark.skipif(not os.path.exists(FIXTURE), reason="tests/golden/stack40.npz not generated")
def test_stack40_matches_oracle(gpu, oracle):
    want = np.load(FIXTURE)
    g = syn.StackGeometry()
    etlut, ntlut = syn.stack_codebooks()
    ebook, nbook = gpu.expert_codebook(etlut), gpu.ne_codebook(ntlut)
    layers = []
    for i in range(g.layers):
        layers.append(hip.upload_decoder_layer(gpu, syn.stack_layer(g, i, etlut, ntlut), ebook,
                                               nbook))
        if i % 10 == 9:
            print(f"stack40: {i + 1} layers uploaded", flush=True)
    emb_host, head_host, norm_host, prompt = syn.stack_token_side(g)
    assert np.array_equal(prompt, want["prompt"]), "the synthetic model differs from the fixture's"
    emb, head = hip.upload_embedding(gpu, emb_host), hip.upload_head(gpu, head_host)
    final_norm = gpu.to_device(norm_host)
    del emb_host, head_host
    capacity = g.prompt + g.greedy_steps
    states = [hip.layer_state(g.full_attention(i), capacity) for i in range(g.layers)]
    tokens = torch.tensor(prompt.astype(np.int32), device="cuda")
    hidden = torch.empty((g.ubatch, g.hidden), dtype=torch.float32, device="cuda")
    normed = torch.empty((1, g.hidden), dtype=torch.float32, device="cuda")
    logits = torch.empty((1, g.vocab), dtype=torch.float32, device="cuda")
    picked = torch.empty(1, dtype=torch.int32, device="cuda")

    def head_logits(row):
        gpu.check(gpu.lib.adi_hip_rms_norm(gpu.handle, row.data_ptr(), final_norm.data_ptr(),
                                           g.hidden, 1, 1.0, 1e-6, normed.data_ptr()))
        hip.head_matmul(gpu, head, normed, 1, logits)
        hip.argmax_rows(gpu, logits, 1, g.vocab, picked)
        return logits.cpu().numpy()[0], int(picked.cpu().numpy()[0])

    # prompt: chunks of 128 through every layer
    rows_after = np.zeros((g.layers, g.hidden), np.float32)
    for c in range(0, g.prompt, g.ubatch):
        hip.embedding_rows(gpu, emb, tokens[c:c + g.ubatch], g.ubatch, hidden)
        for i, (layer, (state, _)) in enumerate(zip(layers, states)):
            hip.prefill_layer(gpu, layer, c, g.ubatch, hidden, state)
            if c + g.ubatch == g.prompt:
                rows_after[i] = hidden[g.ubatch - 1].cpu().numpy()
    for i in range(g.layers):
        assert max_rel_error(rows_after[i], want["hidden_prefill"][i]) <= TOL, ("layer", i)
    got, choice = head_logits(hidden[g.ubatch - 1:g.ubatch])
    report = error_report(got, want["logits_prefill"])
    print(f"stack40 prefill logits: {report}", flush=True)
    assert report["max_rel"] <= TOL
    agreed = checked = 0

    def agree(step, choice):
        nonlocal agreed, checked
        if want["margin"][step] > 2 * TOL * want["logit_max"][step]:
            checked += 1
            assert choice == int(want["tokens"][step]), ("greedy token", step)
            agreed += 1

    agree(0, choice)
    # decode steps, fed the oracle's tokens
    token = torch.empty(1, dtype=torch.int32, device="cuda")
    for step in range(g.greedy_steps):
        token.fill_(int(want["tokens"][step]))
        row = hidden[0:1]
        hip.embedding_rows(gpu, emb, token, 1, row)
        for layer, (state, _) in zip(layers, states):
            hip.decode_layer(gpu, layer, g.prompt + step, row, state)
        got, choice = head_logits(row)
        agree(step + 1, choice)
    report = error_report(got, want["logits_final"])
    print(f"stack40 final logits: {report}; greedy tokens equal at {agreed} of {checked} "
          f"clear steps (of {g.greedy_steps + 1})", flush=True)
    assert report["max_rel"] <= TOL
    assert checked >= (g.greedy_steps + 1) // 2

    # states at the end
    end = g.prompt + g.greedy_steps
    tensors = []
    for i, (state, keep) in enumerate(states):
        a, b = (t.cpu().numpy() for t in keep)
        pair = (a[:end].ravel(), b[:end].ravel()) if g.full_attention(i) else (a.ravel(), b.ravel())
        tensors.append(pair)
        for j, t in enumerate(pair):
            idx = fixture.state_sample_indexes(i, j, t.size)
            err = np.abs(t[idx] - want["state_sample"][i, j]).max() / want["state_max"][i, j]
            assert err <= TOL, ("state", i, j, float(err))
            assert abs(np.abs(t).max() - want["state_max"][i, j]) <= TOL * want["state_max"][i, j]
    gpu_checksum = fixture.decoder_state_checksum(oracle, end, tensors)
    print(f"stack40 decoder_state_checksum: device {gpu_checksum:#018x}, oracle "
          f"{int(want['checksum'][0]):#018x}", flush=True)
