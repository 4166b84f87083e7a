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


@pytest.mark.parametrize("count", [1, 5, 4097, 32767, 32768, 32771, 248320, 262147])
def test_argmax_rows_split_and_unaligned(gpu, oracle, count):
    """Rows of 32,768 logits and more split over up to 64 blocks; odd counts
    leave every other row unaligned. Ties across spans keep the first index
    and a non-finite logit in any span marks its row."""
    rng = np.random.default_rng(count)
    rows = 5
    logits = rng.normal(0, 3, (rows, count)).astype(np.float32)
    logits[1, [count - 1, count // 2, 0]] = 30.0                 # first of three ties
    logits[2, count - 1] = 31.0
    logits[3, count // 3] = np.nan
    logits[4, count - 1] = -np.inf
    t = torch.empty(rows, dtype=torch.int32, device="cuda")
    hip.argmax_rows(gpu, torch.from_numpy(logits).cuda(), rows, count, t)
    got = t.cpu().numpy().view(np.uint32)
    for r in range(rows):
        row = np.ascontiguousarray(logits[r])
        finite = np.isfinite(row).all()
        want = oracle.ao_argmax(po.ptr(row, po.C.c_float), count) if finite else 0xFFFFFFFF
        assert got[r] == want, (count, r)
    assert got[1] == 0 and got[2] == count - 1


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


def sample_device(gpu, logits, temperature, top_p, words):
    rows, count = logits.shape
    t = torch.empty(rows, dtype=torch.int32, device="cuda")
    w = torch.tensor(np.asarray(words, np.uint64).view(np.int64), device="cuda")
    hip.sample_rows(gpu, torch.from_numpy(np.ascontiguousarray(logits)).cuda(), rows, count,
                    temperature, top_p, w, t)
    return t.cpu().numpy().view(np.uint32)


def logit_rows(rng, rows, count):
    out = np.empty((rows, count), np.float32)
    for r in range(rows):
        kind = r % 4
        if kind == 0:
            out[r] = rng.normal(0, 3, count)
        elif kind == 1:
            out[r] = rng.integers(-4, 4, count)            # many ties
        elif kind == 2:
            out[r] = rng.normal(0, 0.05, count)            # flat: top-p keeps many
        else:
            out[r] = rng.normal(0, 1.5, count)
            out[r, rng.integers(0, count, 5)] = 0.0
            out[r, min(1, count - 1)] = -0.0
    return out


@pytest.mark.parametrize("temperature,top_p", [(0.0, 0.9), (1e-4, 0.9), (0.7, 0.9), (1.0, 1.0),
                                               (2.0, 0.5), (0.3, 0.05)])
def test_sample_rows_match_oracle(gpu, oracle, temperature, top_p):
    rng = np.random.default_rng(int(temperature * 1000 + top_p * 100))
    rows, count = 12, 151936
    logits = logit_rows(rng, rows, count)
    words = rng.integers(0, 2**63, rows, dtype=np.uint64) * 2 + rng.integers(0, 2, rows, dtype=np.uint64)
    got = sample_device(gpu, logits, temperature, top_p, words)
    want = [po.sample_token(oracle, logits[r], temperature, top_p, int(words[r])) for r in range(rows)]
    assert got.tolist() == want


def test_sample_rows_small_vocabularies_and_edges(gpu, oracle):
    rng = np.random.default_rng(77)
    for count in (1, 2, 63, 4096, 4097, 12289):
        logits = logit_rows(rng, 8, count)
        words = np.array([0, (1 << 64) - 1] + rng.integers(0, 2**63, 6).tolist(), np.uint64)
        for temperature, top_p in ((0.8, 0.95), (1.5, 1.0)):
            got = sample_device(gpu, logits, temperature, top_p, words)
            want = [po.sample_token(oracle, logits[r], temperature, top_p, int(words[r]))
                    for r in range(8)]
            assert got.tolist() == want, (count, temperature, top_p)


def test_sample_rows_non_finite_and_parameters(gpu):
    logits = np.random.default_rng(5).normal(0, 1, (3, 1000)).astype(np.float32)
    logits[1, 10] = np.nan
    logits[2, 999] = -np.inf
    got = sample_device(gpu, logits, 0.7, 0.9, [1, 2, 3])
    assert got[1] == 0xFFFFFFFF and got[2] == 0xFFFFFFFF and got[0] < 1000
    # rows long enough to split over blocks: the flag of any span marks the row
    long_rows = np.random.default_rng(6).normal(0, 1, (3, 40000)).astype(np.float32)
    long_rows[1, 39999] = np.nan
    long_rows[2, 20000] = np.inf
    got = sample_device(gpu, long_rows, 0.7, 0.9, [4, 5, 6])
    assert got[1] == 0xFFFFFFFF and got[2] == 0xFFFFFFFF and got[0] < 40000
    t = torch.empty(3, dtype=torch.int32, device="cuda")
    x = torch.from_numpy(logits).cuda()
    for temperature, top_p in ((5e-5, 0.9), (2.5, 0.9), (0.7, 0.0), (0.7, 1.01)):
        with pytest.raises(hip.HipError, match="invalid sampling parameters"):
            hip.sample_rows(gpu, x, 3, 1000, temperature, top_p, None, t)
    with pytest.raises(hip.HipError, match="one random word per row"):
        hip.sample_rows(gpu, x, 3, 1000, 0.7, 0.9, None, t)
