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


@pytest.mark.parametrize("count", [3, 40])
def test_decode_batch_one_launch_paths_equal_separate_launches(gpu, parts, count):
    """A decode step's Gated DeltaNet core (convolution, delta rule, gated
    norm) runs as one launch per 32 sequences, and up to 12 rows the MoE
    block and up to 4 the NE projections are single launches too; with the
    one-launch paths off every part is a launch of its own. Logits, caches
    and states are bit-identical over three steps of sequences at different
    positions (40 sequences: two groups of row pointers)."""
    model = parts["one"]

    def run(fused):
        gpu.set_fused_decode(fused)
        try:
            seqs = [hip.Sequence(model, CAPACITY) for _ in range(count)]
            for i, s in enumerate(seqs):
                if i % 4:
                    hip.prefill(gpu, model, [(3 * i + j) % VOCAB for j in range(i % 4)], s, None, ubatch=2)
            tokens = [(5 * i + 1) % VOCAB for i in range(count)]
            outs = []
            for step in range(3):
                print("decode_batch", count, fused, step, flush=True)
                out = torch.empty((count, VOCAB), dtype=torch.float32, device="cuda")
                hip.decode_batch(gpu, model, tokens, seqs, out)
                outs.append(out.cpu().numpy())
                tokens = [int(t) for t in np.argmax(outs[-1], axis=1)]
            gpu.synchronize()
            return outs + [t.cpu().numpy() for s in seqs for keep in s.tensors for t in keep]
        finally:
            gpu.set_fused_decode(True)

    one, separate = run(True), run(False)
    for i, (a, b) in enumerate(zip(one, separate)):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), i


def test_decode_batch_long_histories(gpu, parts):
    """Two sequences past 1,000 entries decoded in one step: each row's
    history then splits into 32 parts, where the flash-decoding blocks of
    the eight query heads of a KV head share an XCD. The logits are
    bit-identical with the one-launch paths off (norm/rotation, partial and
    merge launches), and within 1e-3 of the same tokens taken through the
    single-sequence chunk kernels (a one-token prefill each: 33-34 splits,
    the kernels the attention tests hold to the oracle at histories up to
    2,500 entries)."""
    model = parts["one"]
    capacity = 1100
    rng = np.random.default_rng(2024)
    prompts = [[int(t) for t in rng.integers(3, VOCAB, size=n)] for n in (1030, 1057)]

    def prefilled():
        seqs = [hip.Sequence(model, capacity) for _ in prompts]
        for prompt, s in zip(prompts, seqs):
            hip.prefill(gpu, model, prompt, s, None, ubatch=128)
        return seqs

    def run(fused):
        gpu.set_fused_decode(fused)
        try:
            seqs = prefilled()
            print("decode_batch long", fused, flush=True)
            out = torch.empty((2, VOCAB), dtype=torch.float32, device="cuda")
            hip.decode_batch(gpu, model, [5, 9], seqs, out)
            gpu.synchronize()
            return out.cpu().numpy()
        finally:
            gpu.set_fused_decode(True)

    one, separate = run(True), run(False)
    assert np.array_equal(one.view(np.uint32), separate.view(np.uint32))
    seqs = prefilled()
    for b, (s, token) in enumerate(zip(seqs, [5, 9])):
        logits = torch.empty(VOCAB, dtype=torch.float32, device="cuda")
        hip.prefill(gpu, model, [token], s, logits, ubatch=128)
        assert max_rel_error(one[b], logits.cpu().numpy()) <= 1e-3, b


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


def bits(t):
    return t.cpu().numpy().view(np.uint32)


def twin_sequences(gpu, model, prompts, capacity):
    """Two identical sets of sequences, each prefilled with the prompts."""
    sets = []
    for _ in range(2):
        seqs = [hip.Sequence(model, capacity) for _ in prompts]
        for p, s in zip(prompts, seqs):
            if p:
                hip.prefill(gpu, model, p, s, None, ubatch=128)
        sets.append(seqs)
    return sets


@pytest.mark.parametrize("count", [1, 3, 20])
def test_decode_graph_replays_equal_direct_steps(gpu, parts, count):
    """A captured decode step replayed 8 times gives, bit for bit, the logits
    and states of 8 directly launched adi_hip_decode_batch steps at the same
    positions, fed the same (greedy) tokens from a device array; then the
    positions are reset by the caller (the graph takes them over) and the
    replays still match."""
    model = parts["two"]
    prompts = [[3 + (7 * i) % 500] * (i % 4) for i in range(count)]
    direct, replayed = twin_sequences(gpu, model, prompts, CAPACITY)
    tokens = torch.tensor([11 + i for i in range(count)], dtype=torch.int32, device="cuda")
    want = torch.empty((count, VOCAB), dtype=torch.float32, device="cuda")
    got = torch.empty_like(want)
    graph = hip.DecodeGraph(gpu, model, replayed, tokens, got)
    try:
        for round_ in range(2):
            for step in range(8 if round_ == 0 else 3):
                print("decode graph", count, round_, step, flush=True)
                host = [int(t) for t in tokens.cpu().numpy()]
                hip.decode_batch(gpu, model, host, direct, want)
                graph.launch()
                assert np.array_equal(bits(got), bits(want)), (count, round_, step)
                assert [s.position for s in replayed] == [s.position for s in direct]
                picked = torch.empty(count, dtype=torch.int32, device="cuda")
                hip.argmax_rows(gpu, want, count, VOCAB, picked)
                tokens.copy_(picked)
            for a, b in zip(direct, replayed):
                for ta, tb in zip(a.tensors, b.tensors):
                    for x, y in zip(ta, tb):
                        assert torch.equal(x, y)
            for s in direct + replayed:  # the caller resets every sequence
                s.reset()
        assert graph.captures == 1
    finally:
        graph.close()


def test_decode_graph_recaptures_when_needed(gpu, parts):
    """The graph re-records itself when the positions pass the span it
    covers (512) and when a call in between has grown a scratch arena; the
    replays stay equal to direct steps. A launch with other sequences is
    rejected."""
    model = parts["one"]
    capacity = 520
    prompt = [5 + (i * 13) % 400 for i in range(509)]
    direct, replayed = twin_sequences(gpu, model, [prompt, prompt[:3]], capacity)
    tokens = torch.tensor([17, 29], dtype=torch.int32, device="cuda")
    want = torch.empty((2, VOCAB), dtype=torch.float32, device="cuda")
    got = torch.empty_like(want)
    graph = hip.DecodeGraph(gpu, model, replayed, tokens, got)
    try:
        for step in range(6):  # positions 509..514 of the first sequence
            print("decode graph span", step, flush=True)
            hip.decode_batch(gpu, model, [17, 29], direct, want)
            graph.launch()
            assert np.array_equal(bits(got), bits(want)), step
        assert graph.captures == 2  # at position 512
        # a larger call grows the shared scratch arenas
        big = hip.Sequence(model, 300)
        hip.prefill(gpu, model, list(range(3, 259)), big, None, ubatch=256)
        hip.decode_batch(gpu, model, [17, 29], direct, want)
        graph.launch()
        assert np.array_equal(bits(got), bits(want))
        assert graph.captures == 3
        other = [hip.Sequence(model, capacity) for _ in range(2)]
        states = (hip.DecoderStateStruct * 2)(*(s.struct for s in other))
        status = gpu.lib.adi_hip_decode_graph_launch(graph.handle, states)
        assert status == hip.INVALID_ARGUMENT
        assert "differ from the captured" in gpu.lib.adi_hip_last_error(gpu.handle).decode()
        assert [s.position for s in other] == [0, 0]
    finally:
        graph.close()
