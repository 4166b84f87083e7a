"""adi_hip_moe_forward_static, the MoE entry that allocates nothing (its
intermediates live in the library's fixed per-GPU scratch array), against
adi_hip_moe_forward on the same layer and inputs, both through the C ABI:
routes and outputs bit-identical (the two run the same kernels on the same
data), on two calls in a row, the second with a smaller batch, so the second
call runs over the first call's leftover scratch contents. A batch above 16
is rejected with the outputs untouched."""
import ctypes as C

import numpy as np
import pytest
import torch

from adi_amd import hip
from adi_amd import synthetic as syn

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def layer(gpu):
    rng = syn.rng_for(70, 0)
    host = syn.stacked_moe_layer(rng)
    dev = hip.upload_moe_layer(gpu, host, gpu.expert_codebook(host.expert_tlut),
                               gpu.ne_codebook(host.ne_tlut))
    return dev


def run(gpu, entry, layer, x, batch, bias):
    out = torch.full((batch, layer.hidden), float("nan"), dtype=torch.float32, device="cuda")
    routes = torch.zeros(batch * 8, dtype=torch.int32, device="cuda")
    weights = torch.zeros(batch * 8, dtype=torch.float32, device="cuda")
    status = entry(gpu.handle, C.byref(layer.struct), x.data_ptr(), batch,
                   None if bias is None else bias.data_ptr(), out.data_ptr(), routes.data_ptr(),
                   weights.data_ptr())
    return status, out, routes, weights


def test_static_entry_equals_allocating_entry(gpu, layer):
    rng = syn.rng_for(70, 1)
    lib = hip.load()
    for batch in (16, 4, 1):  # each call smaller than the one before
        x = gpu.to_device(syn.hidden_states(rng, batch, layer.hidden))
        status, want, want_routes, want_weights = run(gpu, lib.adi_hip_moe_forward, layer, x,
                                                      batch, None)
        assert status == hip.OK, gpu.lib.adi_hip_last_error(gpu.handle)
        status, got, got_routes, got_weights = run(gpu, lib.adi_hip_moe_forward_static, layer, x,
                                                   batch, None)
        assert status == hip.OK, gpu.lib.adi_hip_last_error(gpu.handle)
        torch.cuda.synchronize()
        assert torch.equal(got_routes, want_routes), batch
        assert torch.equal(got_weights.view(torch.int32), want_weights.view(torch.int32)), batch
        assert torch.equal(got.view(torch.int32), want.view(torch.int32)), batch


def test_static_entry_rejects_large_batches(gpu, layer):
    rng = syn.rng_for(70, 2)
    lib = hip.load()
    x = gpu.to_device(syn.hidden_states(rng, 17, layer.hidden))
    status, out, routes, _ = run(gpu, lib.adi_hip_moe_forward_static, layer, x, 17, None)
    assert status == hip.INVALID_ARGUMENT
    assert b"1..16" in lib.adi_hip_last_error(gpu.handle)
    torch.cuda.synchronize()
    assert torch.isnan(out).all() and not routes.any()
