"""Continuous batching on the GPU (ContinuousBatcher, src/generation.cpp:
343-660) over the small hybrid model, against the oracle decoding each
request alone. The loop is driven one iteration at a time, so the admission
order is observable: one pending request is admitted per iteration, every
active request gets one token per iteration, and a request leaves on a stop
token (not kept), at its output limit, or when cancelled. Each request's
tokens are checked along its own path: the oracle recomputes the logits for
the tokens the GPU chose, and the GPU's choice must be the oracle's greedy
token (where the top two logits are clearly apart) or, when sampling, the
oracle's sample_token with the request's next std::mt19937_64 word."""
import threading

import numpy as np
import pytest

import pyoracle as po
import small_model
from adi_amd import hip
from adi_amd import serving

pytestmark = pytest.mark.gpu

CAPACITY = 12
MASKED = [0, 1, 2, 510]


@pytest.fixture(scope="module")
def ctx():
    c = hip.Context(0)  # the batcher's own: its worker thread owns it while it runs
    yield c
    c.synchronize()
    c.close()


@pytest.fixture(scope="module")
def parts(ctx):
    return small_model.build(ctx, seed=71)


def masked(logits):
    out = logits.copy()
    out[MASKED] = np.finfo(np.float32).min
    return out


def check_path(oracle, parts, prompt, tokens, temperature, top_p, seed, stop=()):
    """Replays the request on the oracle along the GPU's tokens; returns how
    many choices were compared."""
    o = small_model.OracleSequence(parts, CAPACITY)
    for t in prompt:
        raw = o.step(oracle, t)
    logits = masked(raw)
    words = iter(po.mt19937_64(oracle, seed, 64))
    compared = 0
    for i, got in enumerate(list(tokens) + [None]):
        if temperature == 0.0:
            want = int(np.argmax(logits))
            top2 = np.sort(logits)[-2:]
            clear = top2[1] - top2[0] > 2e-3 * np.max(np.abs(raw))
        else:
            want = po.sample_token(oracle, logits, temperature, top_p, next(words))
            clear = True
        if got is None:  # the choice that ended the request
            return compared, want
        if clear:
            assert got == want, (i, got, want)
            compared += 1
        assert got not in stop and got not in MASKED
        raw = o.step(oracle, got)
        logits = masked(raw)


def test_admission_order_and_oracle_paths(ctx, oracle, parts):
    b = serving.ContinuousBatcher(ctx, parts["one"], max_batch=4, capacity=CAPACITY,
                                  prefill_ubatch=2, masked_tokens=MASKED, start=False)
    try:
        reqs = [
            ([3, 9, 4], dict(max_output_tokens=5, temperature=0.0)),
            ([5, 1], dict(max_output_tokens=6, temperature=0.8, top_p=0.9, seed=1234)),
            ([7], dict(max_output_tokens=4, temperature=0.0)),
        ]
        ids = [b.submit(p, **o) for p, o in reqs]
        print("batcher step 1", flush=True)
        assert b.step() == 3
        counts = [b.status(i)[2].output_tokens for i in ids]
        states = [b.status(i)[0] for i in ids]
        assert counts == [1, 0, 0] and states == [serving.RUNNING, serving.PENDING, serving.PENDING]
        print("batcher step 2", flush=True)
        b.step()
        assert [b.status(i)[2].output_tokens for i in ids] == [2, 1, 0]
        steps = 2
        while b.step() > 0:
            steps += 1
            assert steps < 20
        for (prompt, o), i in zip(reqs, ids):
            r = b.result(i)
            assert r.finish_reason == "length" and r.output_tokens == o["max_output_tokens"]
            assert r.input_tokens == len(prompt) and len(r.tokens) == r.output_tokens
            assert r.prefill_seconds > 0.0 and r.decode_seconds >= 0.0
            compared, _ = check_path(oracle, parts, prompt, r.tokens, o["temperature"],
                                     o.get("top_p", 0.9), o.get("seed", 0))
            assert compared >= len(r.tokens) - 1, (prompt, compared)
    finally:
        b.close()


def test_stop_token_cancel_and_failures(ctx, oracle, parts):
    # the oracle's first greedy token for the prompt is made a stop token
    o = small_model.OracleSequence(parts, CAPACITY)
    for t in [8, 8]:
        logits = masked(o.step(oracle, t))
    first = int(np.argmax(logits))
    b = serving.ContinuousBatcher(ctx, parts["two"], max_batch=2, capacity=CAPACITY,
                                  masked_tokens=MASKED, stop_tokens=[first], start=False)
    try:
        stopped = b.submit([8, 8], max_output_tokens=5, temperature=0.0)
        running = b.submit([4], max_output_tokens=8, temperature=0.0)
        empty = b.submit([], max_output_tokens=2, temperature=0.0)
        long = b.submit(list(range(3, 3 + CAPACITY)), temperature=0.0)  # no room to generate
        b.step()
        r = b.result(stopped)
        assert r.finish_reason == "stop_token" and r.tokens == [] and r.output_tokens == 0
        b.step()  # `running` admitted
        b.cancel(running)
        b.step()  # fails `running`, admits `empty`, which fails
        with pytest.raises(serving.GenerationError, match="generation cancelled"):
            b.result(running)
        with pytest.raises(serving.GenerationError, match="prompt exceeds model context"):
            b.result(empty)
        b.step()
        with pytest.raises(serving.GenerationError, match="prompt exceeds model context"):
            b.result(long)
        assert b.step() == 0
        with pytest.raises(hip.HipError, match="invalid generation options"):
            b.submit([1], temperature=3.0)
        with pytest.raises(hip.HipError, match="max_output_tokens exceeds model context"):
            b.submit([1], max_output_tokens=hip.CONTEXT + 1)
        with pytest.raises(serving.GenerationError, match="max_output_tokens must be positive"):
            b.submit([1], max_output_tokens=0)
    finally:
        b.close()


def test_forced_failures_leave_the_loop_consistent(ctx, oracle, parts):
    """Failures forced from the host (no kernel faults): a failed admission
    fails that request alone and leaves its slot free; a failed step (as a
    one-launch MoE wait that ran out would report at the step's synchronize)
    fails every active request, returns the error, and frees every slot, so
    the next request is admitted and decodes along the oracle's path."""
    b = serving.ContinuousBatcher(ctx, parts["two"], max_batch=2, capacity=CAPACITY,
                                  masked_tokens=MASKED, start=False)
    try:
        lib = ctx.lib
        assert lib.adi_hip_batcher_force_failure(b.handle, 3) == hip.INVALID_ARGUMENT
        ctx.check(lib.adi_hip_batcher_force_failure(b.handle, 1))
        a = b.submit([5, 6], max_output_tokens=3, temperature=0.0)
        assert b.step() == 0
        with pytest.raises(serving.GenerationError, match="admission failure forced by the host"):
            b.result(a)
        first = b.submit([7], max_output_tokens=6, temperature=0.0)
        second = b.submit([8, 9], max_output_tokens=6, temperature=0.0)
        b.step()
        b.step()  # both admitted, one token each so far
        assert b.status(first)[0] == serving.RUNNING and b.status(second)[0] == serving.RUNNING
        ctx.check(lib.adi_hip_batcher_force_failure(b.handle, 2))
        with pytest.raises(hip.HipError, match="decode step failure forced by the host"):
            b.step()
        for r in (first, second):
            assert b.status(r)[0] == serving.FAILED
            with pytest.raises(serving.GenerationError, match="decode step failure forced"):
                b.result(r)
        after = b.submit([7], max_output_tokens=4, temperature=0.0)
        while b.step() != 0:
            pass
        r = b.result(after)
        assert r.output_tokens == 4
        compared, _ = check_path(oracle, parts, [7], r.tokens, 0.0, 0.9, 0)
        assert compared >= len(r.tokens) - 1
    finally:
        b.close()


def test_replayed_steps_give_the_direct_tokens(ctx, oracle, parts):
    """Three sampled and greedy requests with the recorded-step replay on and
    off: the same tokens (the replayed step gives the direct step's bits), and
    both along the oracle's path."""
    results = []
    for replay in (True, False):
        b = serving.ContinuousBatcher(ctx, parts["two"], max_batch=3, capacity=CAPACITY,
                                      masked_tokens=MASKED, start=False, replay_steps=replay)
        try:
            ids = [b.submit([9, 4], max_output_tokens=7, temperature=0.0),
                   b.submit([6], max_output_tokens=8, temperature=0.8, top_p=0.9, seed=5),
                   b.submit([3, 3, 8], max_output_tokens=6, temperature=0.0)]
            while b.step() != 0:
                pass
            results.append([b.result(i).tokens for i in ids])
        finally:
            b.close()
    assert results[0] == results[1]
    for prompt, toks, (t, p, seed) in zip([[9, 4], [6], [3, 3, 8]], results[0],
                                          [(0.0, 0.9, 0), (0.8, 0.9, 5), (0.0, 0.9, 0)]):
        compared, _ = check_path(oracle, parts, prompt, toks, t, p, seed)
        assert compared >= len(toks) - 1


def test_error_messages_are_per_thread(ctx):
    """A failed call on one thread leaves the context's message on other
    threads alone: a batcher's submit may fail on a client thread while the
    stepping thread's own calls succeed (adi_hip_last_error reads back the
    calling thread's last call)."""
    ctx.synchronize()
    seen = {}

    def failing():
        status = ctx.lib.adi_hip_set_reduction_isa(ctx.handle, 3)
        seen["status"] = status
        seen["message"] = ctx.lib.adi_hip_last_error(ctx.handle).decode()

    t = threading.Thread(target=failing)
    t.start()
    t.join()
    assert seen["status"] == hip.INVALID_ARGUMENT and seen["message"] != ""
    assert ctx.lib.adi_hip_last_error(ctx.handle).decode() == ""
    ctx.check(ctx.lib.adi_hip_synchronize(ctx.handle))
    assert ctx.lib.adi_hip_last_error(ctx.handle).decode() == ""


def test_more_requests_than_slots_and_the_worker_thread(ctx, oracle, parts):
    """Five requests from five threads through two slots with the worker
    thread: each result is the one the same request gives when it runs
    alone in the batcher, and the streamed tokens are the result's."""
    prompts = [[3], [4, 5], [6], [7, 8, 9], [10]]
    alone = []
    b = serving.ContinuousBatcher(ctx, parts["one"], max_batch=1, capacity=CAPACITY,
                                  masked_tokens=MASKED, start=False)
    try:
        for p in prompts:
            i = b.submit(p, max_output_tokens=4, temperature=0.0)
            while b.step() > 0:
                pass
            alone.append(b.result(i).tokens)
    finally:
        b.close()
    b = serving.ContinuousBatcher(ctx, parts["one"], max_batch=2, capacity=CAPACITY,
                                  masked_tokens=MASKED)
    results, streamed = [None] * len(prompts), [[] for _ in prompts]

    def run(k):
        results[k] = b.generate(prompts[k], max_output_tokens=4, temperature=0.0,
                                token_callback=streamed[k].append)

    try:
        threads = [threading.Thread(target=run, args=(k,)) for k in range(len(prompts))]
        for t in threads:
            t.start()
        for t in threads:
            t.join(timeout=120)
            assert not t.is_alive()
    finally:
        b.close()
    for k, r in enumerate(results):
        assert r is not None and r.finish_reason == "length"
        assert streamed[k] == r.tokens
        # batched against alone: equal where the greedy choice is clear
        compared, _ = check_path(oracle, parts, prompts[k], r.tokens, 0.0, 0.9, 0)
        assert compared >= 3
        assert r.tokens[:1] == alone[k][:1]
