"""Checkpoint to HBM: a synthetic GGUF checkpoint in the reference's tensor
layout is uploaded with adi_hip_gguf_upload_moe_layer and its codebooks with
adi_hip_gguf_upload_codebooks; the MoE block computed from it is bit-identical
to the block computed from the same layer uploaded array by array, and
matches the oracle (routes exact, outputs within 1e-3)."""
import numpy as np
import pytest
import torch

import gguf_fixture as gf
from adi_amd import hip
from adi_amd import synthetic as syn
from test_gpu_moe import check, run_moe

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def checkpoint(gpu, tmp_path_factory):
    # two layers with 64 experts (two 32-expert chunks) at the full widths
    # (a checkpoint has one expert and one NE table for all layers)
    first = syn.moe_layer(syn.rng_for(11, 0), experts=64)
    layers = [first, syn.moe_layer(syn.rng_for(11, 1), experts=64, etlut=first.expert_tlut,
                                   ntlut=first.ne_tlut)]
    path = str(tmp_path_factory.mktemp("gguf") / "moe.gguf")
    gf.write_moe_checkpoint(path, layers)
    with hip.Gguf(path) as f:
        ebook, nbook = hip.upload_codebooks_gguf(gpu, f)
        uploaded = [hip.upload_moe_layer_gguf(gpu, f, i, ebook, nbook) for i in range(2)]
    # the file is closed: the device copies must not depend on the mapping
    direct = [hip.upload_moe_layer(gpu, L, gpu.expert_codebook(L.expert_tlut),
                                   gpu.ne_codebook(L.ne_tlut)) for L in layers]
    yield layers, uploaded, direct
    for u in uploaded:
        u.close()


@pytest.mark.parametrize("batch,bias", [(1, False), (5, False), (64, True), (200, True)])
@pytest.mark.parametrize("index", [0, 1])
def test_gguf_layer_matches_direct_upload_and_oracle(gpu, oracle, checkpoint, index, batch, bias):
    layers, uploaded, direct = checkpoint
    layer = layers[index]
    rng = syn.rng_for(12, 10 * batch + index)
    x = syn.hidden_states(rng, batch, layer.hidden)
    b = syn.zipf_bias(rng, layer.experts) if bias else None
    got = run_moe(gpu, uploaded[index], x, b)
    ref = run_moe(gpu, direct[index], x, b)
    assert np.array_equal(got[0].view(np.uint32), ref[0].view(np.uint32))
    assert np.array_equal(got[1], ref[1]) and np.array_equal(got[2].view(np.uint32), ref[2].view(np.uint32))
    check(oracle, layer, got, x, b)


def test_gguf_descriptor_geometry(checkpoint):
    layers, uploaded, _ = checkpoint
    s = uploaded[0].struct
    assert (s.hidden, s.expert_hidden, s.experts) == (2048, 512, 64)
    assert (s.router.rows, s.router.columns) == (64, 2048)
    assert (s.shared_down.rows, s.shared_down.columns) == (2048, 512)
    assert s.shared_up.weight_scale == np.float32(layers[0].shared_up.weight_scale)


def test_gguf_upload_errors(gpu, checkpoint, tmp_path):
    layers, _, _ = checkpoint
    path = str(tmp_path / "one.gguf")
    gf.write_moe_checkpoint(path, layers[:1])
    with hip.Gguf(path) as f:
        ebook, nbook = hip.upload_codebooks_gguf(gpu, f)
        with pytest.raises(hip.HipError, match="layer index is out of range") as info:
            hip.upload_moe_layer_gguf(gpu, f, 1, ebook, nbook)
        assert info.value.status == hip.INVALID_ARGUMENT
        with pytest.raises(hip.HipError, match="codebooks required"):
            hip.upload_moe_layer_gguf(gpu, f, 0, nbook, ebook)
    # the context still works after a rejected upload
    torch.cuda.synchronize()
