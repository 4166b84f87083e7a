"""The token side of decoding on the GPU against the oracle: embedding rows
bit-exact (tokens read from device memory, a token past the table gives a NaN
row), the greedy choice bit-exact (ties to the first index, a non-finite row
gives 0xFFFFFFFF), and the embedding table uploaded from a checkpoint."""
import numpy as np
import pytest
import torch

import gguf_fixture as gf
import pyoracle as po
from adi_amd import hip
from adi_amd import synthetic as syn

pytestmark = pytest.mark.gpu


def device_rows(gpu, emb, tokens, columns):
    t = torch.tensor(np.asarray(tokens, np.uint32).view(np.int32), device="cuda")
    out = torch.empty((len(tokens), columns), dtype=torch.float32, device="cuda")
    hip.embedding_rows(gpu, emb, t, len(tokens), out)
    return out.cpu().numpy()


@pytest.mark.parametrize("rows,columns,exceptions", [(50, 64, 0), (300, 256, 200), (1000, 2048, 4000)])
def test_embedding_rows_bit_exact(gpu, oracle, rows, columns, exceptions):
    e = syn.embedding(syn.rng_for(22, rows), rows, columns, exceptions=exceptions)
    emb = hip.upload_embedding(gpu, e)
    rng = np.random.default_rng(rows)
    tokens = [0, rows - 1] + rng.integers(0, rows, 30).tolist() + [rows - 1, 0]
    got = device_rows(gpu, emb, tokens, columns)
    want = po.embedding_rows(oracle, e, tokens)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_embedding_token_out_of_range(gpu, oracle):
    e = syn.embedding(syn.rng_for(22, 1), 40, 128, exceptions=10)
    emb = hip.upload_embedding(gpu, e)
    got = device_rows(gpu, emb, [3, 40, 39, 0xFFFFFFFF], 128)
    assert np.isnan(got[1]).all() and np.isnan(got[3]).all()
    want = po.embedding_rows(oracle, e, [3, 39])
    assert np.array_equal(got[[0, 2]].view(np.uint32), want.view(np.uint32))


def test_embedding_rejects_bad_shapes(gpu):
    e = syn.embedding(syn.rng_for(22, 2), 8, 128)
    emb = hip.upload_embedding(gpu, e)
    emb.struct.columns = 96
    t = torch.zeros(1, dtype=torch.int32, device="cuda")
    out = torch.empty((1, 128), dtype=torch.float32, device="cuda")
    with pytest.raises(hip.HipError, match="Mach embedding shape mismatch"):
        hip.embedding_rows(gpu, emb, t, 1, out)


def test_argmax_rows(gpu, oracle):
    rng = np.random.default_rng(3)
    rows, count = 6, 151936
    logits = rng.normal(0, 4, (rows, count)).astype(np.float32)
    logits[1, [5, 77777, 151935]] = 40.0                   # ties: the first index
    logits[2, :] = -1.0
    logits[2, [100, 200]] = [-0.0, 0.0]                    # -0 == +0: the first
    logits[3, 123] = np.inf                                # non-finite row
    logits[4, 9] = np.nan
    logits[5, count - 1] = 50.0                            # the last element
    t = torch.empty(rows, dtype=torch.int32, device="cuda")
    hip.argmax_rows(gpu, torch.from_numpy(logits).cuda(), rows, count, t)
    got = t.cpu().numpy().view(np.uint32)
    for r in range(rows):
        if r in (3, 4):
            assert got[r] == 0xFFFFFFFF
        else:
            row = np.ascontiguousarray(logits[r])
            assert got[r] == oracle.ao_argmax(po.ptr(row, po.C.c_float), count)
    assert got[1] == 5 and got[2] == 100 and got[5] == count - 1


def test_embedding_from_checkpoint(gpu, oracle, tmp_path):
    layer = syn.moe_layer(syn.rng_for(22, 3), hidden=256, expert_hidden=64, experts=32)
    e = syn.embedding(syn.rng_for(22, 4), 500, 256, exceptions=300)
    path = str(tmp_path / "emb.gguf")
    md = gf.moe_metadata(1, 256, 64, 32)
    gf.write_moe_checkpoint(path, [layer], md, gf.moe_tensors([layer]) + gf.embedding_tensors(e))
    with hip.Gguf(path) as f:
        emb = hip.upload_embedding_gguf(gpu, f)
    assert (emb.struct.rows, emb.struct.columns, emb.struct.exception_count) == (500, 256, 300)
    tokens = [0, 7, 499, 250]
    got = device_rows(gpu, emb, tokens, 256)
    want = po.embedding_rows(oracle, e, tokens)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    emb.close()
