"""The drop-in seam: adi_amd/backend/hip_backend.cpp is an adi::Backend table
(include/adi/backend.hpp:10-23) over the C ABI. These tests call it and the
reference's own cpu_backend() (src/backend.cpp:11-26) through the same
dispatch table, compiled from the reference sources (oracle/Makefile
`make backend`), on identical host arrays."""
import numpy as np
import pytest

from adi_amd import synthetic as syn

import backend_binding as bb
from conftest import max_rel_error

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not bb.available(),
                                 reason="oracle/_ref/libadi_backend.so is built only where the "
                                        "reference sources are present")]


def test_backend_names():
    cpu = bb.name(bb.CPU)
    assert bb.name(bb.HIP) == "hip:" + cpu


@pytest.mark.parametrize("rows,columns", [(512, 2048), (2048, 512), (64, 32), (16, 16)])
@pytest.mark.parametrize("batch", [1, 4, 16])
def test_backend_expert(rows, columns, batch):
    rng = syn.rng_for(1, rows + columns + batch)
    m = syn.expert_matrix(rng, rows, columns, syn.expert_tlut(rng))
    x = syn.hidden_states(rng, batch, columns)
    want = bb.expert_matmul(bb.CPU, m, x, batch)
    got = bb.expert_matmul(bb.HIP, m, x, batch)
    assert max_rel_error(got, want) <= 1e-3


@pytest.mark.parametrize("rows,columns", [(2048, 2048), (512, 2048), (2048, 512), (32, 64)])
@pytest.mark.parametrize("batch", [1, 4])
def test_backend_ne(rows, columns, batch):
    rng = syn.rng_for(1, 7 * rows + columns + batch)
    m = syn.ne_matrix(rng, rows, columns, syn.ne_tlut(rng))
    x = syn.hidden_states(rng, batch, columns)
    want = bb.ne_matmul(bb.CPU, m, x, batch)
    got = bb.ne_matmul(bb.HIP, m, x, batch)
    assert max_rel_error(got, want) <= 1e-3


@pytest.mark.parametrize("batch", [1, 4])
@pytest.mark.parametrize("protected", [0, 3])
def test_backend_head(batch, protected):
    rng = syn.rng_for(2, 31 + batch + protected)
    h = syn.head_chunk(rng, 4096, 2048, protected=protected)
    x = syn.rms_normalized(syn.hidden_states(rng, batch, 2048))
    want = bb.head_matmul(bb.CPU, h, x, batch)
    got = bb.head_matmul(bb.HIP, h, x, batch)
    assert max_rel_error(got, want) <= 1e-3
    if protected:
        # protected rows are the ISA-ordered bf16 dot on both sides
        rows = h.protected_rows.astype(np.int64)
        assert np.array_equal(got[:, rows].view(np.uint32), want[:, rows].view(np.uint32))


@pytest.mark.parametrize("rows,columns,batch", [(256, 2048, 1), (256, 2048, 5), (1, 2048, 3),
                                                 (7, 40, 2)])
def test_backend_bf16_bit_exact(rows, columns, batch):
    """hip_backend() follows the host's cpu_backend() reduction order, so the
    router dot is bit-identical with it."""
    rng = syn.rng_for(1, rows * 3 + columns + batch)
    values = syn.bf16_bits_rne(rng.normal(0.0, 0.02, rows * columns).astype(np.float32))
    x = syn.hidden_states(rng, batch, columns)
    want = bb.bf16_matmul(bb.CPU, values, rows, columns, x, batch)
    got = bb.bf16_matmul(bb.HIP, values, rows, columns, x, batch)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_backend_rms_norm():
    rng = syn.rng_for(1, 99)
    x = syn.hidden_states(rng, 1, 2048)[0]
    weight = syn.bf16_bits_rne(rng.normal(0.0, 0.1, 2048).astype(np.float32))
    want = bb.rms_norm(bb.CPU, x, weight, 1.0, 1e-6)
    got = bb.rms_norm(bb.HIP, x, weight, 1.0, 1e-6)
    assert max_rel_error(got, want) <= 1e-6


def test_backend_embedding_row_bit_exact():
    e = syn.embedding(syn.rng_for(1, 321), 400, 2048, exceptions=500)
    for token in (0, 17, 399):
        want = bb.embedding_row(bb.CPU, e, token)
        got = bb.embedding_row(bb.HIP, e, token)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    errors = []
    for which in (bb.CPU, bb.HIP):
        for token, size in ((400, 2048), (3, 2047)):
            with pytest.raises(bb.BackendError) as info:
                bb.embedding_row(which, e, token, out_size=size)
            errors.append((which, info.value.status, info.value.message))
    assert [x[1:] for x in errors[:2]] == [x[1:] for x in errors[2:]]
    assert errors[0][1:] == (1, "Mach embedding shape mismatch")


def test_backend_repeated_calls_reuse_device_weights():
    rng = syn.rng_for(1, 1234)
    m = syn.expert_matrix(rng, 512, 2048, syn.expert_tlut(rng))
    x = syn.hidden_states(rng, 2, 2048)
    first = bb.expert_matmul(bb.HIP, m, x, 2)
    for _ in range(3):
        assert np.array_equal(bb.expert_matmul(bb.HIP, m, x, 2).view(np.uint32),
                              first.view(np.uint32))


@pytest.mark.parametrize("batch,x_extra,out_extra", [(1, 1, 0), (1, 0, 1), (3, 0, -1), (0, 0, 0)])
def test_backend_shape_errors_match_the_reference(batch, x_extra, out_extra):
    """Mismatched spans raise std::invalid_argument with the reference's own
    message, from both tables."""
    rng = syn.rng_for(1, 555)
    m = syn.expert_matrix(rng, 64, 32, syn.expert_tlut(rng))
    x = syn.hidden_states(rng, max(batch, 1), 32)
    x_size = batch * 32 + x_extra
    out_size = max(batch * 64 + out_extra, 0)
    errors = []
    for which in (bb.CPU, bb.HIP):
        with pytest.raises(bb.BackendError) as info:
            bb.expert_matmul(which, m, np.resize(x, max(x_size, 1)), batch, out_size=out_size,
                             x_size=x_size)
        errors.append((info.value.status, info.value.message))
    assert errors[0] == errors[1]
    assert errors[0][0] == 1


def test_backend_weight_cache_follows_contents():
    """The HIP table caches device copies of weights by host address. New
    contents at the same address replace the copy (results follow the new
    weights, as the CPU table's do), also when a single word changes, and
    hip_backend_release_weights() drops every copy; calls after it upload
    again."""
    rng = syn.rng_for(1, 977)
    m = syn.ne_matrix(rng, 512, 2048, syn.ne_tlut(rng))
    x = syn.hidden_states(rng, 1, 2048)
    first = bb.ne_matmul(bb.HIP, m, x, 1)
    assert max_rel_error(first, bb.ne_matmul(bb.CPU, m, x, 1)) <= 1e-3
    m.trellis[:] = syn.uniform_words(rng, m.trellis.size)  # same buffer, new weights
    second = bb.ne_matmul(bb.HIP, m, x, 1)
    assert max_rel_error(second, bb.ne_matmul(bb.CPU, m, x, 1)) <= 1e-3
    assert not np.array_equal(first, second)
    # one word changed between the points a sampled fingerprint would read:
    # the copy is keyed on the full contents, so the change is seen
    spacing = (m.trellis.nbytes - 8) // 63
    word = (spacing + spacing // 2) // 2
    m.trellis[word] ^= 0x5A5A
    changed = bb.ne_matmul(bb.HIP, m, x, 1)
    assert max_rel_error(changed, bb.ne_matmul(bb.CPU, m, x, 1)) <= 1e-3
    assert not np.array_equal(changed, second)
    m.trellis[word] ^= 0x5A5A
    second = bb.ne_matmul(bb.HIP, m, x, 1)
    bb.release_weights()
    third = bb.ne_matmul(bb.HIP, m, x, 1)
    assert np.array_equal(third.view(np.uint32), second.view(np.uint32))
