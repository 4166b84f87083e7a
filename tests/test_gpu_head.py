"""int5_g64 output head on the GPU: logits within max relative error 1e-3 of
the CPU path, protected rows bit-exact, greedy arg-max bit-exact."""
import numpy as np
import pytest
import torch

import pyoracle as po
from adi_amd import hip
from adi_amd import synthetic as syn
from conftest import max_rel_error

pytestmark = pytest.mark.gpu


def run_head(gpu, h, x):
    batch = x.shape[0]
    dh = hip.upload_head(gpu, h)
    logits = torch.empty((batch, h.rows), dtype=torch.float32, device="cuda")
    arg = torch.empty(batch, dtype=torch.int32, device="cuda")
    hip.head_argmax(gpu, dh, gpu.to_device(x), batch, logits, arg)
    plain = torch.empty((batch, h.rows), dtype=torch.float32, device="cuda")
    hip.head_matmul(gpu, dh, gpu.to_device(x), batch, plain)
    return logits.cpu().numpy(), arg.cpu().numpy().astype(np.uint32), plain.cpu().numpy()


@pytest.mark.parametrize("isa", [1, 8, 16])
@pytest.mark.parametrize("rows,columns,protected,batch", [
    (1, 64, 0, 1), (37, 128, 0, 3), (1000, 2048, 3, 4), (3000, 192, 2, 2), (151936, 2048, 0, 1),
    (151936, 2048, 0, 4)])
def test_head_logits_and_argmax(gpu, oracle, isa, rows, columns, protected, batch):
    rng = syn.rng_for(1, rows + columns + protected)
    h = syn.head_chunk(rng, rows, columns, protected)
    x = syn.rms_normalized(syn.hidden_states(rng, batch, columns))
    want = po.head_matmul(oracle, h, x, isa=isa)
    gpu.set_isa(isa)
    try:
        logits, arg, plain = run_head(gpu, h, x)
    finally:
        gpu.set_isa(16)
    assert max_rel_error(logits, want) <= 1e-3
    assert np.array_equal(logits.view(np.uint32), plain.view(np.uint32))
    assert np.array_equal(arg, np.argmax(want, axis=1).astype(np.uint32))
    if protected:
        rows_p = h.protected_rows.astype(np.int64)
        assert np.array_equal(logits[:, rows_p].view(np.uint32), want[:, rows_p].view(np.uint32))


@pytest.mark.parametrize("batch", [1, 2, 3, 4, 5, 9])
def test_head_2048_columns_by_batch(gpu, oracle, batch):
    """The 2048-column head (MFMA tiles of 16 rows, four tokens per pass) on
    rows that do not fill the last tile, one to three passes."""
    rng = syn.rng_for(1, 5000 + batch)
    h = syn.head_chunk(rng, 1000, 2048, 0)
    x = syn.rms_normalized(syn.hidden_states(rng, batch, 2048))
    want = po.head_matmul(oracle, h, x, isa=16)
    logits, arg, plain = run_head(gpu, h, x)
    assert max_rel_error(logits, want) <= 1e-3
    assert np.array_equal(logits.view(np.uint32), plain.view(np.uint32))
    assert np.array_equal(arg, np.argmax(want, axis=1).astype(np.uint32))


def test_head_argmax_near_ties(gpu, oracle):
    """Rows built to tie or nearly tie with the maximum: the certified
    arg-max must still return the CPU path's first maximum."""
    rng = syn.rng_for(1, 4242)
    rows, columns = 2000, 2048
    h = syn.head_chunk(rng, rows, columns, 0)
    per_row = columns // 8 * 5
    # duplicate one row several times, and a copy with one code changed
    h.packed.reshape(rows, per_row)[[10, 500, 1500]] = h.packed.reshape(rows, per_row)[1999]
    h.group_scale_f16.reshape(rows, -1)[[10, 500, 1500]] = h.group_scale_f16.reshape(rows, -1)[1999]
    x = syn.rms_normalized(syn.hidden_states(rng, 2, columns))
    # make row 1999 the maximum for token 0 by aligning x with it
    want = po.head_matmul(oracle, h, x, isa=16)
    logits, arg, _ = run_head(gpu, h, x)
    assert np.array_equal(arg, np.argmax(want, axis=1).astype(np.uint32))


def test_head_known_answer(gpu):
    """tests/kernels_test.cpp:193-201: zero codes (weight -16), scale 0.5,
    x = 1 over 64 columns gives -512."""
    h = syn.HeadChunk(1, 64, np.zeros(40, np.uint8), syn.f16_bits(np.array([0.5], np.float32)))
    logits, arg, _ = run_head(gpu, h, np.ones((1, 64), np.float32))
    assert logits[0, 0] == -512.0 and arg[0] == 0
