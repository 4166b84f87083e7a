"""Packed projections on the GPU against the oracle (C restatement of the
reference CPU path): decoded weights bit-exact, outputs within max relative
error 1e-3 (max |g - c| / max |c| per output vector, fp32 accumulation)."""
import numpy as np
import pytest
import torch

import pyoracle as po
from adi_amd import hip
from adi_amd import synthetic as syn
from conftest import max_rel_error

pytestmark = pytest.mark.gpu
TOL = 1e-3

EXPERT_SHAPES = [(16, 16), (64, 32), (32, 128), (512, 2048), (2048, 512), (16, 4096)]
NE_SHAPES = [(16, 16), (64, 32), (128, 2048), (2048, 2048), (512, 2048), (2048, 512)]


@pytest.fixture(scope="module")
def books(gpu):
    rng = syn.rng_for(0, 7)
    et, nt = syn.expert_tlut(rng), syn.ne_tlut(rng)
    return et, nt, gpu.expert_codebook(et), gpu.ne_codebook(nt)


@pytest.mark.parametrize("rows,columns", EXPERT_SHAPES)
def test_expert_decode_bit_exact(gpu, books, oracle, rows, columns):
    et, _, eb, _ = books
    m = syn.expert_matrix(syn.rng_for(0, rows * 7 + columns), rows, columns, et)
    want = np.zeros((rows, columns), np.float32)
    s = po.expert_struct(m)
    po.check(oracle.ao_expert_decode_tiles(po.C.byref(s), po.ptr(want, po.C.c_float)), "decode")
    dm = hip.upload_expert(gpu, m, eb)
    out = torch.empty((rows, columns), dtype=torch.float32, device="cuda")
    hip.expert_decode(gpu, dm, out)
    got = out.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("rows,columns", NE_SHAPES)
def test_ne_decode_bit_exact(gpu, books, oracle, rows, columns):
    _, nt, _, nb = books
    m = syn.ne_matrix(syn.rng_for(0, rows * 11 + columns), rows, columns, nt)
    want = np.zeros((rows, columns), np.float32)
    s = po.ne_struct(m)
    po.check(oracle.ao_ne_decode_tiles(po.C.byref(s), po.ptr(want, po.C.c_float)), "decode")
    dm = hip.upload_ne(gpu, m, nb)
    out = torch.empty((rows, columns), dtype=torch.float32, device="cuda")
    hip.ne_decode(gpu, dm, out)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("rows,columns", EXPERT_SHAPES)
@pytest.mark.parametrize("batch", [1, 2, 4, 5, 15, 16, 33])
def test_expert_matmul(gpu, books, oracle, rows, columns, batch):
    et, _, eb, _ = books
    rng = syn.rng_for(0, rows + columns + batch)
    m = syn.expert_matrix(rng, rows, columns, et)
    x = syn.hidden_states(rng, batch, columns)
    want = po.expert_matmul(oracle, m, x)
    dm = hip.upload_expert(gpu, m, eb)
    out = torch.empty((batch, rows), dtype=torch.float32, device="cuda")
    hip.expert_matmul(gpu, dm, gpu.to_device(x), batch, out)
    assert max_rel_error(out.cpu().numpy(), want) <= TOL


# from 16 rows (expert) and 8 rows (NE) a single projection runs as an MFMA
# GEMM (f16 hi/lo operands, fp32 accumulation): the error stays near fp32
# rounding, well inside 1e-3
MFMA_TOL = 1e-4


@pytest.mark.parametrize("rows,columns", [(16, 64), (64, 128), (512, 2048), (2048, 512)])
@pytest.mark.parametrize("batch", [16, 33, 64, 100, 300])
def test_expert_matmul_mfma(gpu, books, oracle, rows, columns, batch):
    et, _, eb, _ = books
    rng = syn.rng_for(0, 5 * rows + columns + batch)
    m = syn.expert_matrix(rng, rows, columns, et)
    x = syn.hidden_states(rng, batch, columns)
    want = po.expert_matmul(oracle, m, x)
    dm = hip.upload_expert(gpu, m, eb)
    out = torch.empty((batch, rows), dtype=torch.float32, device="cuda")
    hip.expert_matmul(gpu, dm, gpu.to_device(x), batch, out)
    assert max_rel_error(out.cpu().numpy(), want) <= MFMA_TOL


@pytest.mark.parametrize("rows,columns", [(16, 32), (128, 2048), (512, 2048), (2048, 512)])
@pytest.mark.parametrize("batch", [8, 9, 31, 64, 100, 300])
def test_ne_matmul_mfma(gpu, books, oracle, rows, columns, batch):
    _, nt, _, nb = books
    rng = syn.rng_for(0, 11 * rows + columns + batch)
    m = syn.ne_matrix(rng, rows, columns, nt)
    x = syn.hidden_states(rng, batch, columns)
    want = po.ne_matmul(oracle, m, x)
    dm = hip.upload_ne(gpu, m, nb)
    out = torch.empty((batch, rows), dtype=torch.float32, device="cuda")
    hip.ne_matmul(gpu, dm, gpu.to_device(x), batch, out)
    assert max_rel_error(out.cpu().numpy(), want) <= MFMA_TOL


@pytest.mark.parametrize("rows,columns", NE_SHAPES)
@pytest.mark.parametrize("batch", [1, 3, 4, 7, 8, 16])
def test_ne_matmul(gpu, books, oracle, rows, columns, batch):
    _, nt, _, nb = books
    rng = syn.rng_for(0, rows * 3 + columns + batch)
    m = syn.ne_matrix(rng, rows, columns, nt)
    x = syn.hidden_states(rng, batch, columns)
    want = po.ne_matmul(oracle, m, x)
    dm = hip.upload_ne(gpu, m, nb)
    out = torch.empty((batch, rows), dtype=torch.float32, device="cuda")
    hip.ne_matmul(gpu, dm, gpu.to_device(x), batch, out)
    assert max_rel_error(out.cpu().numpy(), want) <= TOL


@pytest.mark.parametrize("rows,columns", [(2048, 2048), (512, 2048), (8192, 2048), (4096, 2048),
                                          (2048, 4096), (512, 4096)])
@pytest.mark.parametrize("batch", [1, 2, 4])
def test_ne_one_launch_equals_separate_launches(gpu, books, oracle, rows, columns, batch):
    """The one-launch NE projection (rows of up to four inputs) against the
    prologue + GEMV + epilogue launches: bit-identical, and within the
    tolerance of the oracle."""
    _, nt, _, nb = books
    rng = syn.rng_for(0, 7 * rows + columns + 13 * batch)
    m = syn.ne_matrix(rng, rows, columns, nt)
    x = syn.hidden_states(rng, batch, columns)
    dm = hip.upload_ne(gpu, m, nb)
    xd = gpu.to_device(x)
    one = torch.full((batch, rows), float("nan"), dtype=torch.float32, device="cuda")
    sep = torch.full((batch, rows), float("nan"), dtype=torch.float32, device="cuda")
    hip.ne_matmul(gpu, dm, xd, batch, one)
    gpu.set_fused_decode(False)
    try:
        hip.ne_matmul(gpu, dm, xd, batch, sep)
    finally:
        gpu.set_fused_decode(True)
    gpu.synchronize()
    a, b = one.cpu().numpy(), sep.cpu().numpy()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), "one launch differs from separate launches"
    assert max_rel_error(a, po.ne_matmul(oracle, m, x)) <= TOL
    # a second call reuses the ticket the first one cleared
    hip.ne_matmul(gpu, dm, xd, batch, one)
    gpu.synchronize()
    assert np.array_equal(one.cpu().numpy().view(np.uint32), b.view(np.uint32))


def test_known_answers(gpu):
    """tests/kernels_test.cpp:32-137: a zero expert tile with TLUT rows
    1..8 and gamma slot 1 = 2 gives out[0] = 32; the NE tile with TLUT (1, 2)
    and Wscale 0.5 gives out[0] = 8; every other output is 0."""
    tlut = np.tile(np.arange(1, 9, dtype=np.float32), 32768)
    one = syn.f16_bits(np.ones(16, np.float32))
    m = syn.ExpertMatrix(16, 16, np.zeros(24, np.uint16), one, one,
                         syn.f16_bits(np.array([1.0, 2.0], np.float32)), tlut)
    dm = hip.upload_expert(gpu, m, gpu.expert_codebook(tlut))
    out = torch.empty((1, 16), dtype=torch.float32, device="cuda")
    hip.expert_matmul(gpu, dm, torch.ones((1, 16), device="cuda"), 1, out)
    got = out.cpu().numpy()[0]
    assert abs(got[0] - 32.0) < 1e-5 and np.all(np.abs(got[1:]) < 1e-5)

    ntlut = np.tile(np.array([1.0, 2.0], np.float32), 512)
    signs = np.ones(16, np.int8)
    n = syn.NeMatrix(16, 16, np.zeros(64, np.uint16), signs, signs, 0.5, ntlut)
    dn = hip.upload_ne(gpu, n, gpu.ne_codebook(ntlut))
    hip.ne_matmul(gpu, dn, torch.ones((1, 16), device="cuda"), 1, out)
    got = out.cpu().numpy()[0]
    assert abs(got[0] - 8.0) < 1e-5 and np.all(np.abs(got[1:]) < 1e-5)


def test_shape_errors_leave_outputs_untouched(gpu, books):
    et, _, eb, _ = books
    m = syn.expert_matrix(syn.rng_for(0, 99), 48, 16, et)  # 48 rows: not a power of two
    dm = hip.upload_expert(gpu, m, eb)
    out = torch.full((1, 48), 7.0, device="cuda")
    with pytest.raises(hip.HipError) as err:
        hip.expert_matmul(gpu, dm, torch.ones((1, 16), device="cuda"), 1, out)
    assert err.value.status == hip.INVALID_ARGUMENT
    assert "powers of two" in str(err.value)
    assert torch.all(out == 7.0)
    m2 = syn.expert_matrix(syn.rng_for(0, 98), 16, 16, et)
    dm2 = hip.upload_expert(gpu, m2, eb)
    with pytest.raises(hip.HipError):
        hip.expert_matmul(gpu, dm2, torch.ones((1, 16), device="cuda"), 0, out)


@pytest.mark.parametrize("n", [16, 64, 128, 512, 2048, 4096, 8192])
def test_hadamard_bit_exact(gpu, oracle, n):
    rng = np.random.default_rng(n)
    x = rng.standard_normal((5, n)).astype(np.float32)
    want = x.copy()
    for row in want:
        assert oracle.ao_hadamard(po.ptr(row, po.C.c_float), n) == 0
    dev = gpu.to_device(x)
    hip.hadamard(gpu, dev, n, 5)
    assert np.array_equal(dev.cpu().numpy().view(np.uint32), want.view(np.uint32))
