"""The oracle's token-side functions pinned without a GPU: embedding rows
(mach_embedding_row, src/kernels.cpp:802-845) by a closed form and by the
compiled reference, and the greedy choice of sample_token
(src/generation.cpp:180-183) by the compiled reference with ties and signed
zeros."""
import ctypes as C

import numpy as np
import pytest

import pyoracle as po
from adi_amd import synthetic as syn


@pytest.fixture(scope="module")
def oracle():
    return po.load_oracle()


@pytest.fixture(scope="module")
def ref():
    if not po.ref_available():
        pytest.skip("oracle/_ref is not built here")
    return po.load_ref()


def test_embedding_closed_form(oracle):
    # group 0: min 0, max 15 -> step 1, value = code; group 1: min == max = 1
    # -> step 1e-8/15, value rounds back to 1.0; then exceptions overwrite
    rows, columns = 3, 128
    codes = np.arange(rows * columns, dtype=np.uint32) % 16
    packed = ((codes[0::2] << 4) | codes[1::2]).astype(np.uint8)
    f16 = lambda v: syn.f16_bits(np.array([v], np.float32))[0]
    mn = np.array([f16(0.0), f16(1.0)] * rows, np.uint16)
    mx = np.array([f16(15.0), f16(1.0)] * rows, np.uint16)
    ex = np.array([columns + 5, 2 * columns + 127], np.uint32)
    bits = syn.bf16_bits_rne(np.array([-2.5, 7.0], np.float32)).astype(np.uint16)
    e = syn.Embedding(rows, columns, packed, mn, mx, ex, bits)
    got = po.embedding_rows(oracle, e, [0, 1, 2])
    want = np.where(np.arange(columns) < 64, codes[:columns] % 16, 1.0).astype(np.float32)
    want = np.tile(want, (3, 1))
    want[1, 5] = -2.5
    want[2, 127] = 7.0
    assert np.array_equal(got, want)
    s = po.embedding_struct(e)
    row = np.zeros(columns, np.float32)
    assert oracle.ao_embedding_row(C.byref(s), 3, po.ptr(row, C.c_float)) == -1  # token >= rows


@pytest.mark.parametrize("rows,columns,exceptions", [(50, 64, 0), (300, 256, 200), (17, 2048, 600)])
def test_embedding_matches_reference(oracle, ref, rows, columns, exceptions):
    e = syn.embedding(syn.rng_for(21, rows), rows, columns, exceptions=exceptions)
    tokens = sorted({0, 1, rows // 2, rows - 1})
    a = po.embedding_rows(oracle, e, tokens)
    b = po.embedding_rows(ref, e, tokens, prefix="ref")
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def argmax(oracle, logits):
    logits = np.ascontiguousarray(logits, np.float32)
    return oracle.ao_argmax(po.ptr(logits, C.c_float), logits.size)


def test_argmax_matches_reference_greedy(oracle, ref):
    rng = np.random.default_rng(5)
    cases = [rng.normal(0, 3, 1000).astype(np.float32) for _ in range(5)]
    tie = rng.normal(0, 1, 500).astype(np.float32)
    tie[[17, 300, 499]] = 9.0  # equal maxima: the first wins
    zeros = np.full(64, -1.0, np.float32)
    zeros[[10, 20]] = [-0.0, 0.0]  # -0 == +0: the first wins
    cases += [tie, zeros, np.array([1.0], np.float32)]
    for logits in cases:
        want, _ = po.ref_sample_token(ref, logits, 0.0, 1.0, 0)
        assert argmax(oracle, logits) == want
    assert argmax(oracle, tie) == 17 and argmax(oracle, zeros) == 10


@pytest.mark.parametrize("count", [1, 7, 1000, 151936])
def test_sample_token_matches_reference(oracle, ref, count):
    """The oracle's sample_token given the engine's first word draws the
    same token as the compiled sample_token with its std::mt19937_64."""
    rng = np.random.default_rng(count)
    for trial in range(40 if count < 100000 else 6):
        kind = trial % 4
        if kind == 0:
            logits = rng.normal(0, 3, count).astype(np.float32)
        elif kind == 1:
            logits = rng.integers(-3, 3, count).astype(np.float32)   # ties
        elif kind == 2:
            logits = rng.normal(0, 0.01, count).astype(np.float32)  # flat
        else:
            logits = rng.normal(0, 1, count).astype(np.float32)
            logits[0] = -0.0
        temperature = float(rng.choice([0.0, 1e-4, 0.1, 0.7, 2.0]))
        top_p = float(rng.choice([0.05, 0.5, 0.9, 1.0]))
        want, word = po.ref_sample_token(ref, logits, temperature, top_p, int(rng.integers(0, 2**63)))
        assert po.sample_token(oracle, logits, temperature, top_p, word) == want


def test_sample_token_closed_form(oracle):
    # two tokens, logits 0 and ln 3 at temperature 1: p = 1/3 and 1 in sorted
    # order (token 1 first); kept sum 4/3 at top_p 1; target = u * 4/3
    logits = np.array([0.0, np.log(3.0)], np.float32)
    t1 = po.sample_token(oracle, logits, 1.0, 1.0, 0)              # u = 0 -> first sorted
    t2 = po.sample_token(oracle, logits, 1.0, 1.0, (1 << 64) - 1)  # u -> 1 -> last
    t3 = po.sample_token(oracle, logits, 1.0, 0.5, (1 << 64) - 1)  # top_p 0.5 keeps one
    assert (t1, t2, t3) == (1, 0, 1)


@pytest.mark.parametrize("temperature,top_p", [(-1.0, 0.9), (5e-5, 0.9), (2.5, 0.9), (1.0, 0.0),
                                               (1.0, 1.5), (float("nan"), 0.9)])
def test_sample_token_rejects_parameters(oracle, temperature, top_p):
    logits = np.zeros(4, np.float32)
    with pytest.raises(ValueError):
        po.sample_token(oracle, logits, temperature, top_p, 1)


def _device_order_sum(p: np.ndarray, threads: int) -> float:
    """sum(p) in the order one block of `threads` threads adds a span on the
    device: thread t adds the float4 groups t, t + threads, ... in index
    order, each lane pair of a wave is then added in a butterfly (offsets 32
    down to 1), and the waves' sums are added in wave order from 0."""
    assert p.size % 4 == 0
    groups = p.reshape(-1, 4)
    acc = np.zeros(threads, np.float64)
    for start in range(0, groups.shape[0], threads):
        block = groups[start:start + threads]
        for c in range(4):
            acc[:block.shape[0]] = acc[:block.shape[0]] + block[:, c]
    lanes = acc.reshape(-1, 64)
    for offset in (32, 16, 8, 4, 2, 1):
        lanes = lanes + lanes[:, np.arange(64) ^ offset]
    total = 0.0
    for w in range(lanes.shape[0]):
        total = total + lanes[w, 0]
    return total


def _device_denominator(p: np.ndarray) -> float:
    """adi_hip_sample_rows' sum of p: one 1024-thread block below 32,768
    logits; above, spans of up to 64 blocks of 256 threads, added in span
    order (k_expsum_parts, k_sample_rows)."""
    n = p.size
    if n < 32768:
        return _device_order_sum(p, 1024)
    wanted = min(64, -(-n // 4096))
    span = (-(-n // wanted) + 3) & ~3
    total = 0.0
    for begin in range(0, n, span):
        total = total + _device_order_sum(p[begin:begin + span], 256)
    return total


@pytest.mark.parametrize("count", [4096, 151936, 248320])
def test_top_p_denominator_order_bound(count):
    """The sampler's one known departure from sample_token: the reference adds
    sum(p) in descending-logit order (src/generation.cpp:185-194), the device
    in its thread/tree order. Both are double sums of positive terms, so they
    differ by less than the recursive-summation bound (count - 1) * 2^-53
    relative (measured: 3.5e-15 at 4,096 logits, 2.5e-14 at 151,936, 4.4e-14 at
    248,320). A draw picks another token only if its threshold lies within that
    relative distance of a running sum."""
    rng = np.random.default_rng([syn.SEED_BASE, 91, count])
    worst = 0.0
    for _ in range(4):
        logits = rng.normal(0.0, 2.0, count).astype(np.float32)
        logits[rng.integers(0, count, 16)] += 12.0
        m = np.float64(logits.max())
        p = np.exp((logits.astype(np.float64) - m) / np.float64(np.float32(0.7)))
        order = np.lexsort((np.arange(count), -logits.astype(np.float64)))
        reference = np.cumsum(p[order])[-1]  # sequential adds in sorted order
        device = _device_denominator(p)
        worst = max(worst, abs(device - reference) / reference)
    print(f"count {count}: largest relative denominator difference {worst:.3g}")
    assert worst <= (count - 1) * 2.0 ** -53


def test_mt19937_64_known_answer_and_reference(oracle, ref):
    """The oracle's std::mt19937_64: C++11 [rand.predef] requires the 10000th
    output of a default-constructed engine (seed 5489) to be
    9981545732273789042; and the first word of each seeded engine is the one
    the compiled sample_token's engine draws first."""
    assert po.mt19937_64(oracle, 5489, 10000)[-1] == 9981545732273789042
    logits = np.linspace(-1.0, 1.0, 64).astype(np.float32)
    for seed in (0, 1, 1234, 2**63 + 5):
        _, word = po.ref_sample_token(ref, logits, 0.7, 0.9, seed)
        assert po.mt19937_64(oracle, seed, 1)[0] == word, seed
    # and the stream continues past the first twist (312 words)
    words = po.mt19937_64(oracle, 42, 700)
    assert len(set(words)) == 700
