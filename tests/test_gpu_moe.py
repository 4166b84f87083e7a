"""One MoE block on the GPU against the oracle: routes bit-exact, outputs
within max relative error 1e-3."""
import numpy as np
import pytest
import torch

import pyoracle as po
from adi_amd import hip
from adi_amd import synthetic as syn
from conftest import max_rel_error

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def small_layer(gpu):
    rng = syn.rng_for(2, 5)
    layer = syn.moe_layer(rng, hidden=256, expert_hidden=64, experts=16)
    dl = hip.upload_moe_layer(gpu, layer, gpu.expert_codebook(layer.expert_tlut),
                              gpu.ne_codebook(layer.ne_tlut))
    return layer, dl


@pytest.fixture(scope="module")
def full_layer(gpu):
    rng = syn.rng_for(2, 0)
    layer = syn.moe_layer(rng)  # hidden 2048, expert 512, 256 experts
    dl = hip.upload_moe_layer(gpu, layer, gpu.expert_codebook(layer.expert_tlut),
                              gpu.ne_codebook(layer.ne_tlut))
    return layer, dl


def run_moe(gpu, dl, x, bias):
    batch = x.shape[0]
    out = torch.empty((batch, dl.hidden), dtype=torch.float32, device="cuda")
    re = torch.empty(batch * 8, dtype=torch.int32, device="cuda")
    rw = torch.empty(batch * 8, dtype=torch.float32, device="cuda")
    hip.moe_forward(gpu, dl, gpu.to_device(x), batch, None if bias is None else gpu.to_device(bias),
                    out, re, rw)
    return (out.cpu().numpy(), re.cpu().numpy().astype(np.uint32).reshape(batch, 8),
            rw.cpu().numpy().reshape(batch, 8))


def check(oracle, layer, got, x, bias):
    want, we, ww = po.moe_forward(oracle, layer, x, isa=16, logit_bias=bias)
    out, ge, gw = got
    assert np.array_equal(ge, we), "routes differ"
    np.testing.assert_allclose(gw, ww, rtol=4e-7)
    assert max_rel_error(out, want) <= 1e-3


@pytest.mark.parametrize("batch", [1, 2, 4, 16, 33, 64, 97])
@pytest.mark.parametrize("bias", [False, True])
def test_moe_small(gpu, oracle, small_layer, batch, bias):
    layer, dl = small_layer
    rng = syn.rng_for(2, 100 + batch)
    x = syn.hidden_states(rng, batch, layer.hidden)
    b = syn.zipf_bias(rng, layer.experts) if bias else None
    check(oracle, layer, run_moe(gpu, dl, x, b), x, b)


@pytest.mark.parametrize("batch,bias", [(1, False), (4, False), (16, False), (128, True),
                                        (512, True)])
def test_moe_full(gpu, oracle, full_layer, batch, bias):
    layer, dl = full_layer
    rng = syn.rng_for(3 if bias else 2, 200 + batch)
    x = syn.hidden_states(rng, batch, layer.hidden)
    b = syn.zipf_bias(rng, layer.experts) if bias else None
    check(oracle, layer, run_moe(gpu, dl, x, b), x, b)


def test_moe_repeated_calls_are_deterministic(gpu, full_layer):
    layer, dl = full_layer
    rng = syn.rng_for(2, 77)
    x = syn.hidden_states(rng, 16, layer.hidden)
    first = run_moe(gpu, dl, x, None)
    for _ in range(3):
        again = run_moe(gpu, dl, x, None)
        assert np.array_equal(first[0].view(np.uint32), again[0].view(np.uint32))
        assert np.array_equal(first[1], again[1])


def run_both(gpu, dl, x, bias):
    """The layer with the one-launch batch-1 path and with the separate
    launches (the same arithmetic); adi_hip_synchronize reports a cross-block
    wait of the one launch that ran out."""
    try:
        gpu.set_fused_decode(True)
        fused = run_moe(gpu, dl, x, bias)
        gpu.synchronize()
        gpu.set_fused_decode(False)
        separate = run_moe(gpu, dl, x, bias)
    finally:
        gpu.set_fused_decode(True)
    return fused, separate


@pytest.mark.parametrize("seed", [0, 1, 2, 3])
@pytest.mark.parametrize("bias", [False, True])
def test_moe_one_launch_equals_separate_launches(gpu, oracle, full_layer, seed, bias):
    layer, dl = full_layer
    rng = syn.rng_for(2, 300 + seed)
    x = syn.hidden_states(rng, 1, layer.hidden)
    b = syn.zipf_bias(rng, layer.experts) if bias else None
    fused, separate = run_both(gpu, dl, x, b)
    assert np.array_equal(fused[1], separate[1]), "routes differ"
    assert np.array_equal(fused[2].view(np.uint32), separate[2].view(np.uint32)), "weights differ"
    assert np.array_equal(fused[0].view(np.uint32), separate[0].view(np.uint32)), "outputs differ"
    check(oracle, layer, fused, x, b)


def test_moe_one_launch_repeated_calls(gpu, full_layer):
    """Back-to-back one-row calls on new inputs: each call's counters start
    from zero (the last block of a call clears them), so every call equals the
    separate launches on its own input."""
    layer, dl = full_layer
    rng = syn.rng_for(2, 400)
    xs = [syn.hidden_states(rng, 1, layer.hidden) for _ in range(6)]
    outs = [run_moe(gpu, dl, x, None) for x in xs]
    gpu.synchronize()
    gpu.set_fused_decode(False)
    try:
        for x, got in zip(xs, outs):
            want = run_moe(gpu, dl, x, None)
            assert np.array_equal(got[0].view(np.uint32), want[0].view(np.uint32))
            assert np.array_equal(got[1], want[1])
    finally:
        gpu.set_fused_decode(True)


def run_few_both(gpu, dl, x, bias):
    """The layer as the one-launch block of 2-12 rows and as the separate
    launches on the decode-GEMV path (the same arithmetic)."""
    try:
        gpu.set_fused_decode(True)
        fused = run_moe(gpu, dl, x, bias)
        gpu.synchronize()
        gpu.set_fused_decode("gemv")
        separate = run_moe(gpu, dl, x, bias)
    finally:
        gpu.set_fused_decode(True)
    return fused, separate


@pytest.mark.parametrize("batch", [2, 3, 4, 8, 12])
@pytest.mark.parametrize("bias", [False, True])
def test_moe_few_rows_one_launch_equals_separate_launches(gpu, oracle, full_layer, batch, bias):
    """2-12 rows in one launch (k_moe_decode_few) against the separate
    decode-GEMV launches: routes, weights and outputs bit-identical, and within
    the tolerance of the oracle."""
    layer, dl = full_layer
    rng = syn.rng_for(2, 500 + 7 * batch + (1 if bias else 0))
    x = syn.hidden_states(rng, batch, layer.hidden)
    b = syn.zipf_bias(rng, layer.experts) if bias else None
    print(f"moe few rows: batch {batch}, bias {bias}", flush=True)
    fused, separate = run_few_both(gpu, dl, x, b)
    assert np.array_equal(fused[1], separate[1]), "routes differ"
    assert np.array_equal(fused[2].view(np.uint32), separate[2].view(np.uint32)), "weights differ"
    assert np.array_equal(fused[0].view(np.uint32), separate[0].view(np.uint32)), "outputs differ"
    check(oracle, layer, fused, x, b)


def test_moe_few_rows_shared_slots(gpu, oracle, full_layer):
    """Every row the same input: all rows choose the same eight experts, so
    each slot holds all 12 rows (the widest slots)."""
    layer, dl = full_layer
    rng = syn.rng_for(2, 600)
    x = np.repeat(syn.hidden_states(rng, 1, layer.hidden), 12, axis=0)
    fused, separate = run_few_both(gpu, dl, x, None)
    assert np.array_equal(fused[1], separate[1])
    assert np.array_equal(fused[0].view(np.uint32), separate[0].view(np.uint32))
    assert np.array_equal(fused[0][0].view(np.uint32), fused[0][11].view(np.uint32))
    check(oracle, layer, fused, x, None)


def test_moe_few_rows_repeated_calls(gpu, full_layer):
    """Back-to-back calls of 12, 1, 5, 2, 1 and 12 rows on new inputs: every
    call's counters start from zero (the last block through clears them), and
    the one-row block's leftover combine rows sit outside the few-row block's
    counters."""
    layer, dl = full_layer
    rng = syn.rng_for(2, 700)
    xs = [syn.hidden_states(rng, n, layer.hidden) for n in (12, 1, 5, 2, 1, 12)]
    outs = [run_moe(gpu, dl, x, None) for x in xs]
    gpu.synchronize()
    gpu.set_fused_decode("gemv")
    try:
        for x, got in zip(xs, outs):
            want = run_moe(gpu, dl, x, None)
            assert np.array_equal(got[0].view(np.uint32), want[0].view(np.uint32))
            assert np.array_equal(got[1], want[1])
    finally:
        gpu.set_fused_decode(True)
