"""Decode steps over several sequences at once (decode_batch,
src/executor.cpp:1592-1825) and prompt prefill (prefill_prompt,
src/generation.cpp:131-159) through the model-level entry points, against
the oracle running each sequence alone token by token: a hybrid stack of
three Gated DeltaNet layers and one full-attention layer at hidden 256, a
512-token vocabulary (one head chunk, or two chunks whose rows the logits
interleave), sequences of different lengths in one batch. Logits within 1e-3
of their largest value, caches and states elementwise within 1e-3 of their
largest value; the next tokens are the oracle's (teacher forcing). The
reference's own batch test (tests/model_batch_test.cpp) asks the same:
batched logits equal serial ones, every position advances by one, and a
batch holding an exhausted sequence is rejected with no state changed."""
import numpy as np
import pytest
import torch

from adi_amd import hip
from conftest import max_rel_error
import small_model
from small_model import VOCAB

pytestmark = pytest.mark.gpu

CAPACITY = 16


@pytest.fixture(scope="module")
def parts(gpu):
    return small_model.build(gpu)


def close(got, want, what):
    assert np.max(np.abs(got - want)) <= 1e-3 * np.max(np.abs(want)), what


@pytest.mark.parametrize("chunks", ["one", "two"])
def test_decode_batch_matches_each_sequence_alone(gpu, oracle, parts, chunks):
    model = parts[chunks]
    prompts = [[], [3, 9], [5, 1, 4, 1, 5]]
    seqs = [hip.Sequence(model, CAPACITY) for _ in prompts]
    orc = [small_model.OracleSequence(parts, CAPACITY) for _ in prompts]
    tokens = []
    for prompt, s, o in zip(prompts, seqs, orc):
        if not prompt:
            tokens.append(7)
            continue
        print("prefill", chunks, len(prompt), flush=True)
        logits = torch.empty(VOCAB, dtype=torch.float32, device="cuda")
        hip.prefill(gpu, model, prompt, s, logits, ubatch=2)
        for t in prompt:
            want = o.step(oracle, t)
        assert max_rel_error(logits.cpu().numpy(), want) <= 1e-3
        assert s.position == len(prompt)
        tokens.append(int(np.argmax(want)))
    for step in range(4):
        print("decode_batch", chunks, step, tokens, flush=True)
        out = torch.empty((len(seqs), VOCAB), dtype=torch.float32, device="cuda")
        hip.decode_batch(gpu, model, tokens, seqs, out)
        got = out.cpu().numpy()
        nxt = []
        for b, o in enumerate(orc):
            want = o.step(oracle, tokens[b])
            assert max_rel_error(got[b], want) <= 1e-3, (step, b)
            nxt.append(int(np.argmax(want)))
        tokens = nxt
    for prompt, s, o in zip(prompts, seqs, orc):
        assert s.position == len(prompt) + 4 == o.position
        for i, held in enumerate(o.held):
            keep = s.tensors[i]
            if parts["layers"][i].full is not None:
                close(keep[0].cpu().numpy()[:s.position], held.keys[:s.position], ("keys", i))
                close(keep[1].cpu().numpy()[:s.position], held.values[:s.position], ("values", i))
            else:
                close(keep[0].cpu().numpy(), held.convolution, ("convolution", i))
                close(keep[1].cpu().numpy(), held.recurrent, ("recurrent", i))


@pytest.mark.parametrize("count", [9, 17, 40])
def test_decode_batch_many_sequences_mixed_positions(gpu, oracle, parts, count):
    """Batches on both sides of the kernels' row thresholds, through the model
    entry: from 8 rows the NE projections run on the MFMA GEMM, from 16 the
    expert projections too, and above 32 rows the per-sequence attention
    kernels take a second group of row pointers. Each sequence starts at its
    own position (prompts of 0-5 tokens) and every row is compared with the
    oracle decoding that sequence alone, for two steps."""
    model = parts["one"]
    rng = np.random.default_rng(1000 + count)
    prompts = [[int(t) for t in rng.integers(3, VOCAB, size=i % 6)] for i in range(count)]
    seqs = [hip.Sequence(model, CAPACITY) for _ in prompts]
    orc = [small_model.OracleSequence(parts, CAPACITY) for _ in prompts]
    tokens = []
    print("prefill", count, flush=True)
    for prompt, s, o in zip(prompts, seqs, orc):
        if not prompt:
            tokens.append(int(rng.integers(3, VOCAB)))
            continue
        hip.prefill(gpu, model, prompt, s, None, ubatch=4)
        for t in prompt:
            want = o.step(oracle, t)
        tokens.append(int(np.argmax(want)))
    for step in range(2):
        print("decode_batch", count, step, flush=True)
        out = torch.empty((count, VOCAB), dtype=torch.float32, device="cuda")
        hip.decode_batch(gpu, model, tokens, seqs, out)
        got = out.cpu().numpy()
        nxt = []
        for b, o in enumerate(orc):
            want = o.step(oracle, tokens[b])
            assert max_rel_error(got[b], want) <= 1e-3, (count, step, b, len(prompts[b]))
            nxt.append(int(np.argmax(want)))
        tokens = nxt
    for prompt, s in zip(prompts, seqs):
        assert s.position == len(prompt) + 2


def test_fresh_sequences_batched_equal_decoded_alone(gpu, parts):
    """tests/model_batch_test.cpp:24-51: two new sequences decoded as one
    batch give the logits of each decoded alone, and both reach position 1.
    Here 'equal' is within 1e-3: the batched projections take other kernels."""
    model = parts["one"]
    tokens = [11, 300]
    alone = []
    for t in tokens:
        s = hip.Sequence(model, CAPACITY)
        out = torch.empty((1, VOCAB), dtype=torch.float32, device="cuda")
        hip.decode_batch(gpu, model, [t], [s], out)
        alone.append(out.cpu().numpy()[0])
    seqs = [hip.Sequence(model, CAPACITY) for _ in tokens]
    out = torch.empty((2, VOCAB), dtype=torch.float32, device="cuda")
    hip.decode_batch(gpu, model, tokens, seqs, out)
    got = out.cpu().numpy()
    for b in range(2):
        assert max_rel_error(got[b], alone[b]) <= 1e-3
        assert seqs[b].position == 1


def test_rejections_leave_states_untouched(gpu, parts):
    model = parts["one"]
    seqs = [hip.Sequence(model, 4) for _ in range(2)]
    hip.decode_batch(gpu, model, [1, 2], seqs, None)
    gpu.synchronize()
    full = [i for i in range(4) if model.full_attention(i)][0]
    before = [s.tensors[full][0].clone() for s in seqs]
    out = torch.full((2, VOCAB), 7.0, device="cuda")
    with pytest.raises(hip.HipError, match="decoder batch token is out of range") as e:
        hip.decode_batch(gpu, model, [1, VOCAB], seqs, out)
    assert e.value.status == hip.INVALID_ARGUMENT
    short = hip.Model(model.layers, model.embedding, model.final_norm, model.heads, context=2)
    seqs[1].struct.position = 2
    with pytest.raises(hip.HipError, match="decoder context is exhausted") as e:
        hip.decode_batch(gpu, short, [1, 2], seqs, out)
    assert e.value.status == hip.OUT_OF_RANGE
    seqs[1].struct.position = 4  # the caches hold 4 positions
    with pytest.raises(hip.HipError, match="decoder batch state mismatch"):
        hip.decode_batch(gpu, model, [1, 2], seqs, out)
    seqs[1].struct.position = 1
    assert [s.position for s in seqs] == [1, 1]
    gpu.synchronize()
    assert torch.all(out == 7.0)
    for s, b in zip(seqs, before):
        assert torch.equal(s.tensors[full][0], b)
    with pytest.raises(hip.HipError, match="decoder batch shape mismatch"):
        hip.decode_batch(gpu, model, [], [], out)
    s = hip.Sequence(model, 4)
    with pytest.raises(hip.HipError, match="prefill shape or context is invalid"):
        hip.prefill(gpu, model, [], s)
    with pytest.raises(hip.HipError, match="prefill token is out of range"):
        hip.prefill(gpu, model, [1, VOCAB], s)
    with pytest.raises(hip.HipError, match="prefill_ubatch"):
        hip.prefill(gpu, model, [1, 2], s, ubatch=5000)
    with pytest.raises(hip.HipError, match="prefill state mismatch"):
        hip.prefill(gpu, model, [1, 2, 3, 4, 5], s)  # more than the caches hold
    assert s.position == 0
