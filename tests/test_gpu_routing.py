"""Router, top_experts and the stable counting sort on the GPU: bit-exact
against the oracle for every CPU reduction order (scalar, AVX2, AVX-512)."""
import numpy as np
import pytest
import torch

import pyoracle as po
from adi_amd import hip
from adi_amd import synthetic as syn

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("isa", [1, 8, 16])
@pytest.mark.parametrize("rows,columns,batch", [(256, 2048, 1), (256, 2048, 5), (1, 2048, 3),
                                                (4, 67, 2), (37, 13, 9), (256, 2048, 128),
                                                # register-tiled path: partial row and token
                                                # blocks, several K chunks; 8 x 8 tiles dealt
                                                # by row tiles (under 8 token tiles) and by
                                                # token tiles, then 16 x 16 tiles past 256
                                                (37, 512, 45), (256, 4096, 33), (20, 256, 64),
                                                (37, 512, 70), (37, 512, 300),
                                                # either side of the tile-shape switch
                                                (20, 256, 256), (20, 256, 257)])
def test_bf16_matmul_bit_exact(gpu, oracle, isa, rows, columns, batch):
    rng = syn.rng_for(2, rows * 31 + columns + batch)
    w = syn.bf16_bits_rne(rng.normal(0, 0.02, (rows, columns)).astype(np.float32))
    x = syn.hidden_states(rng, batch, columns)
    want = po.bf16_matmul(oracle, w, x, isa=isa)
    gpu.set_isa(isa)
    try:
        out = torch.empty((batch, rows), dtype=torch.float32, device="cuda")
        hip.bf16_matmul(gpu, gpu.to_device(w), rows, columns, gpu.to_device(x), batch, out)
        assert np.array_equal(bits(out.cpu().numpy()), bits(want))
    finally:
        gpu.set_isa(16)


def test_bf16_known_answer(gpu):
    """tests/kernels_test.cpp:245-253: rows (1,2,3) and (4,5,6) times (1,2,3)."""
    w = np.array([[0x3F80, 0x4000, 0x4040], [0x4080, 0x40A0, 0x40C0]], np.uint16)
    out = torch.empty((1, 2), dtype=torch.float32, device="cuda")
    for isa in (1, 8, 16):
        gpu.set_isa(isa)
        hip.bf16_matmul(gpu, gpu.to_device(w), 2, 3, torch.tensor([[1.0, 2.0, 3.0]], device="cuda"),
                        1, out)
        assert out.cpu().numpy().tolist() == [[14.0, 32.0]]
    gpu.set_isa(16)


def make_logits(rng, batch, experts, ties):
    logits = rng.normal(0, 1, (batch, experts)).astype(np.float32)
    if ties:
        logits = np.round(logits * 2).astype(np.float32)
    return logits


@pytest.mark.parametrize("batch,experts,ties", [(1, 256, False), (7, 256, True), (64, 16, True),
                                                (512, 256, False), (3, 8, True), (5, 1024, True)])
def test_top_experts(gpu, oracle, batch, experts, ties):
    rng = syn.rng_for(3, batch * experts + ties)
    logits = make_logits(rng, batch, experts, ties)
    if ties:
        logits[0, :] = 0.0  # all equal: lowest indices win
    out_e = torch.empty(batch * 8, dtype=torch.int32, device="cuda")
    out_w = torch.empty(batch * 8, dtype=torch.float32, device="cuda")
    hip.top_experts(gpu, gpu.to_device(logits), batch, experts, out_e, out_w)
    got_e = out_e.cpu().numpy().astype(np.uint32).reshape(batch, 8)
    got_w = out_w.cpu().numpy().reshape(batch, 8)
    for b in range(batch):
        e, w = po.top_experts(oracle, logits[b])
        assert np.array_equal(got_e[b], e)
        np.testing.assert_allclose(got_w[b], w, rtol=4e-7, atol=0)
    if ties:
        assert got_e[0].tolist() == list(range(8))


def test_top_experts_reference_order(gpu):
    """tests/executor_test.cpp:29-59: logits 0..15 route to experts 15..8 with
    weights equal to the renormalised full softmax."""
    logits = np.arange(16, dtype=np.float32)[None, :]
    out_e = torch.empty(8, dtype=torch.int32, device="cuda")
    out_w = torch.empty(8, dtype=torch.float32, device="cuda")
    hip.top_experts(gpu, gpu.to_device(logits), 1, 16, out_e, out_w)
    assert out_e.cpu().tolist() == list(range(15, 7, -1))
    p = np.exp(logits[0] - logits[0].max())
    p /= p.sum()
    sel = p[15:7:-1]
    np.testing.assert_allclose(out_w.cpu().numpy(), sel / sel.sum(), atol=2e-7)


@pytest.mark.parametrize("batch,experts,bias", [(1, 256, False), (4, 256, False), (16, 256, True),
                                                (128, 256, True), (512, 256, True), (9, 16, False)])
def test_moe_route_permutation_bit_exact(gpu, oracle, batch, experts, bias):
    rng = syn.rng_for(3, 1000 + batch)
    logits = make_logits(rng, batch, experts, False)
    b = syn.zipf_bias(rng, experts) if bias else None
    want = po.moe_route(oracle, logits + (b if bias else 0))
    dev = {k: torch.empty(v.shape, dtype=torch.int32 if v.dtype == np.uint32 else torch.float32,
                          device="cuda") for k, v in want.items()}
    hip.moe_route(gpu, gpu.to_device(logits), gpu.to_device(b) if bias else None, batch, experts, dev)
    for key in ("route_expert", "counts", "offsets", "grouped_batch", "route_to_grouped"):
        got = dev[key].cpu().numpy().astype(np.uint32)
        assert np.array_equal(got, want[key]), key
    np.testing.assert_allclose(dev["route_weight"].cpu().numpy(), want["route_weight"], rtol=4e-7)
