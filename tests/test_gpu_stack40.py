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
digests are reported, not compared.

A second run drives the same weights through the model-level entries that
the benchmark times: adi_hip_prefill of the prompt at ubatch 128 (the final
norm and head on its last token inside the call), then 64 adi_hip_decode_batch
steps of the one sequence, teacher-forced, each writing its logits row
(src/executor.cpp:1592-1825, 1827-2101; the residual adds fused into the next
layer's norm). Its logits, greedy tokens and states are held to the same
checks."""
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


@pytest.fixture(scope="module")
def stack(gpu):
    if not os.path.exists(FIXTURE):
        pytest.skip("tests/golden/stack40.npz not generated")
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
    model = hip.Model(layers, emb, final_norm, [head])
    yield dict(want=want, g=g, layers=layers, emb=emb, head=head, final_norm=final_norm,
               prompt=prompt, model=model)
    del layers, model
    torch.cuda.empty_cache()


class Greedy:
    """Counts the steps whose greedy token is checked (top-two margin above
    twice the tolerance) and asserts the device's choice there."""

    def __init__(self, want):
        self.want, self.agreed, self.checked = want, 0, 0

    def __call__(self, step, choice):
        if self.want["margin"][step] > 2 * TOL * self.want["logit_max"][step]:
            self.checked += 1
            assert choice == int(self.want["tokens"][step]), ("greedy token", step)
            self.agreed += 1


def check_states(oracle, g, want, keeps, label):
    """Every layer's two state tensors at the fixture's sampled indexes and
    their largest value; returns decoder_state_checksum of the device's."""
    end = g.prompt + g.greedy_steps
    tensors = []
    for i, keep in enumerate(keeps):
        a, b = (t.cpu().numpy() for t in keep)
        pair = (a[:end].ravel(), b[:end].ravel()) if g.full_attention(i) else (a.ravel(), b.ravel())
        tensors.append(pair)
        for j, t in enumerate(pair):
            idx = fixture.state_sample_indexes(i, j, t.size)
            err = np.abs(t[idx] - want["state_sample"][i, j]).max() / want["state_max"][i, j]
            assert err <= TOL, (label, "state", i, j, float(err))
            assert abs(np.abs(t).max() - want["state_max"][i, j]) <= TOL * want["state_max"][i, j]
    return fixture.decoder_state_checksum(oracle, end, tensors)


@pytest.mark.timeout(900)
def test_stack40_matches_oracle(gpu, oracle, stack):
    want, g, layers, emb, head = (stack[k] for k in ("want", "g", "layers", "emb", "head"))
    final_norm, prompt = stack["final_norm"], stack["prompt"]
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
    agree = Greedy(want)
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
    print(f"stack40 final logits: {report}; greedy tokens equal at {agree.agreed} of "
          f"{agree.checked} clear steps (of {g.greedy_steps + 1})", flush=True)
    assert report["max_rel"] <= TOL
    assert agree.checked >= (g.greedy_steps + 1) // 2
    gpu_checksum = check_states(oracle, g, want, [keep for _, keep in states], "layer entries")
    print(f"stack40 decoder_state_checksum: device {gpu_checksum:#018x}, oracle "
          f"{int(want['checksum'][0]):#018x}", flush=True)


@pytest.mark.timeout(900)
def test_stack40_model_entries_match_oracle(gpu, oracle, stack):
    """The benchmark's entries: adi_hip_prefill (two 128-token chunks, logits
    of the last prompt token) and 64 teacher-forced adi_hip_decode_batch
    steps of one sequence."""
    want, g, model = stack["want"], stack["g"], stack["model"]
    seq = hip.Sequence(model, g.prompt + g.greedy_steps)
    logits = torch.empty((1, g.vocab), dtype=torch.float32, device="cuda")
    picked = torch.empty(1, dtype=torch.int32, device="cuda")

    def choice():
        hip.argmax_rows(gpu, logits, 1, g.vocab, picked)
        return int(picked.cpu().numpy()[0])

    print("stack40 model entries: prefill", flush=True)
    hip.prefill(gpu, model, [int(t) for t in stack["prompt"]], seq, logits[0], ubatch=g.ubatch)
    assert seq.position == g.prompt
    report = error_report(logits.cpu().numpy()[0], want["logits_prefill"])
    print(f"stack40 model entries, prefill logits: {report}", flush=True)
    assert report["max_rel"] <= TOL
    agree = Greedy(want)
    agree(0, choice())
    for step in range(g.greedy_steps):
        hip.decode_batch(gpu, model, [int(want["tokens"][step])], [seq], logits)
        agree(step + 1, choice())
    assert seq.position == g.prompt + g.greedy_steps
    report = error_report(logits.cpu().numpy()[0], want["logits_final"])
    print(f"stack40 model entries, final logits: {report}; greedy tokens equal at "
          f"{agree.agreed} of {agree.checked} clear steps", flush=True)
    assert report["max_rel"] <= TOL
    assert agree.checked >= (g.greedy_steps + 1) // 2
    gpu_checksum = check_states(oracle, g, want, seq.tensors, "model entries")
    print(f"stack40 model entries decoder_state_checksum: device {gpu_checksum:#018x}, oracle "
          f"{int(want['checksum'][0]):#018x}", flush=True)


@pytest.mark.timeout(600)
@pytest.mark.parametrize("count", [1, 4, 16])
def test_stack40_graph_replay_equals_direct(gpu, stack, count):
    """The benchmark's replayed decode step at the full geometry: `count`
    sequences prefilled with the prompt, then 8 greedy steps replayed from one
    captured step (adi_hip_decode_graph) give the logits of 8 direct
    adi_hip_decode_batch steps bit for bit (one sequence runs the one-launch
    MoE block and the one-launch NE projections inside the graph)."""
    g, model = stack["g"], stack["model"]
    prompt = [int(t) for t in stack["prompt"]]
    capacity = g.prompt + 16
    sets = []
    for _ in range(2):
        seqs = [hip.Sequence(model, capacity) for _ in range(count)]
        for s in seqs:
            hip.prefill(gpu, model, prompt, s, None, ubatch=g.ubatch)
        sets.append(seqs)
    direct, replayed = sets
    tokens = torch.tensor([int(stack["want"]["tokens"][0])] * count, dtype=torch.int32, device="cuda")
    want = torch.empty((count, g.vocab), dtype=torch.float32, device="cuda")
    got = torch.empty_like(want)
    graph = hip.DecodeGraph(gpu, model, replayed, tokens, got)
    try:
        for step in range(8):
            print(f"stack40 graph replay, {count} sequences, step {step}", flush=True)
            hip.decode_batch(gpu, model, [int(t) for t in tokens.cpu().numpy()], direct, want)
            graph.launch()
            assert np.array_equal(got.cpu().numpy().view(np.uint32),
                                  want.cpu().numpy().view(np.uint32)), step
            hip.argmax_rows(gpu, want, count, g.vocab, tokens)
        gpu.synchronize()  # also reports a one-launch MoE wait that ran out
        assert graph.captures == 1
    finally:
        graph.close()
    del sets, direct, replayed
    torch.cuda.empty_cache()
