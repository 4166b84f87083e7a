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


# ---- decoder layers and the output head from a checkpoint ---------------------

@pytest.fixture(scope="module")
def decoder_checkpoint(gpu, tmp_path_factory):
    from test_gguf_cpu import decoder_checkpoint_tensors
    md, ts, layers, chunks, norm = decoder_checkpoint_tensors()
    path = str(tmp_path_factory.mktemp("gguf") / "decoder.gguf")
    with open(path, "wb") as out:
        out.write(gf.gguf_bytes(md, ts))
    etlut, ntlut = layers[0].moe.expert_tlut, layers[0].moe.ne_tlut
    with hip.Gguf(path) as f:
        ebook, nbook = hip.upload_codebooks_gguf(gpu, f)
        uploaded = {i: hip.upload_decoder_layer_gguf(gpu, f, i, ebook, nbook) for i in (0, 3)}
        head = hip.upload_head_gguf(gpu, f)
    direct_books = gpu.expert_codebook(etlut), gpu.ne_codebook(ntlut)
    direct = {i: hip.upload_decoder_layer(gpu, layers[i], *direct_books) for i in (0, 3)}
    yield layers, chunks, norm, uploaded, direct, head
    for u in uploaded.values():
        u.close()
    head.close()


@pytest.mark.parametrize("index", [0, 3])
def test_gguf_decoder_layer_matches_direct_upload(gpu, decoder_checkpoint, index):
    """Three decode steps of a Gated DeltaNet layer (0) and a full-attention
    layer (3) from the checkpoint against the same layer uploaded array by
    array: hidden rows and the layer state bit for bit."""
    layers, _, _, uploaded, direct, _ = decoder_checkpoint
    full = layers[index].full is not None
    hidden_width = layers[index].moe.hidden
    rng = syn.rng_for(13, index)
    rows = [torch.tensor(syn.hidden_states(rng, 1, hidden_width), device="cuda") for _ in range(3)]
    results = []
    for layer in (uploaded[index], direct[index]):
        state, keep = hip.layer_state(full, 3)
        outs = []
        for step, x in enumerate(rows):
            h = x.clone()
            hip.decode_layer(gpu, layer, step, h, state)
            outs.append(h.cpu().numpy())
        gpu.synchronize()
        results.append((outs, [t.cpu().numpy() for t in keep]))
    (a, sa), (b, sb) = results
    for x, y in zip(a, b):
        assert np.array_equal(x.view(np.uint32), y.view(np.uint32))
    for x, y in zip(sa, sb):
        assert np.array_equal(x.view(np.uint32), y.view(np.uint32))


def test_gguf_head_matches_direct_upload(gpu, decoder_checkpoint):
    """The eight chunks uploaded end to end as one head: logits bit for bit
    against the same rows uploaded as one array (protected rows renumbered),
    and the final norm copied as it is."""
    _, chunks, norm, _, _, head = decoder_checkpoint
    rows = chunks[0].rows
    columns = chunks[0].columns
    whole = syn.HeadChunk(rows * 8, columns, np.concatenate([c.packed for c in chunks]),
                          np.concatenate([c.group_scale_f16 for c in chunks]))
    prot = [(c * rows + h.protected_rows, h.protected_bf16) for c, h in enumerate(chunks)
            if h.protected_rows is not None and h.protected_rows.size]
    whole.protected_rows = np.concatenate([r for r, _ in prot]).astype(np.uint32)
    whole.protected_bf16 = np.concatenate([v for _, v in prot])
    assert head.struct.rows == rows * 8 and head.struct.protected_count == whole.protected_rows.size
    direct = hip.upload_head(gpu, whole)
    x = torch.tensor(syn.hidden_states(syn.rng_for(13, 9), 4, columns), device="cuda")
    got = torch.empty((4, rows * 8), dtype=torch.float32, device="cuda")
    want = torch.empty_like(got)
    hip.head_matmul(gpu, head, x, 4, got)
    hip.head_matmul(gpu, direct, x, 4, want)
    gpu.synchronize()
    assert np.array_equal(got.cpu().numpy().view(np.uint32), want.cpu().numpy().view(np.uint32))
    back = np.zeros(columns, np.uint16)
    gpu.check(gpu.lib.adi_hip_copy_to_host(gpu.handle, back.ctypes.data, head.final_norm, back.nbytes))
    assert np.array_equal(back, norm)
