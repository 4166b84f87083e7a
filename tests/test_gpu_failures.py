"""Failure paths forced from the host: a device allocation the GPU cannot
satisfy and a workspace growth beyond the context's limit. Each fails with
OUT_OF_MEMORY and a message, leaves the outputs untouched, and leaves the
context usable: the same calls then give the bit-identical results of a
context that never failed. The reference's counterpart is the exception a
setup or request-time step throws (src/kernels.cpp:393-408), which leaves the
caller's buffers as they were."""
import ctypes as C

import numpy as np
import pytest
import torch

from adi_amd import hip
from adi_amd import synthetic as syn

pytestmark = pytest.mark.gpu

SENTINEL = 7.0


def make_calls(ctx):
    """Upload one NE matrix, one expert matrix and a small MoE layer on `ctx`,
    and return the calls (name, run(out), output shape) that need a workspace:
    batch 64 projections (the MFMA paths) and a 128-row MoE block."""
    rng = syn.rng_for(41, 0)
    et, nt = syn.expert_tlut(rng), syn.ne_tlut(rng)
    ne = hip.upload_ne(ctx, syn.ne_matrix(rng, 512, 2048, nt), ctx.ne_codebook(nt))
    ex = hip.upload_expert(ctx, syn.expert_matrix(rng, 512, 2048, et), ctx.expert_codebook(et))
    layer = syn.moe_layer(rng, hidden=256, expert_hidden=64, experts=16)
    moe = hip.upload_moe_layer(ctx, layer, ctx.expert_codebook(layer.expert_tlut),
                               ctx.ne_codebook(layer.ne_tlut))
    x = ctx.to_device(syn.hidden_states(rng, 64, 2048))
    xm = ctx.to_device(syn.hidden_states(rng, 128, 256))
    keep = (ne, ex, moe, layer)
    return keep, [
        ("ne_matmul", lambda out: hip.ne_matmul(ctx, ne, x, 64, out), (64, 512)),
        ("expert_matmul", lambda out: hip.expert_matmul(ctx, ex, x, 64, out), (64, 512)),
        ("moe_forward", lambda out: hip.moe_forward(ctx, moe, xm, 128, None, out, None, None),
         (128, 256)),
    ]


def run_all(ctx, calls):
    outs = []
    for name, run, shape in calls:
        print("case", name, shape, flush=True)
        out = torch.full(shape, SENTINEL, dtype=torch.float32, device="cuda")
        run(out)
        outs.append(out)
    ctx.synchronize()
    return [o.cpu().numpy() for o in outs]


@pytest.fixture(scope="module")
def reference_outputs():
    ctx = hip.Context(0)
    keep, calls = make_calls(ctx)
    outs = run_all(ctx, calls)
    del keep
    ctx.close()
    return outs


def test_workspace_limit_fails_before_launch(reference_outputs):
    ctx = hip.Context(0)  # fresh: its arenas are empty
    try:
        keep, calls = make_calls(ctx)
        ctx.set_workspace_limit(4096)
        for name, run, shape in calls:
            print("case", name, shape, "limit 4096", flush=True)
            out = torch.full(shape, SENTINEL, dtype=torch.float32, device="cuda")
            with pytest.raises(hip.HipError) as err:
                run(out)
            assert err.value.status == hip.OUT_OF_MEMORY, name
            assert "workspace limit of 4096 bytes" in str(err.value), name
            ctx.synchronize()
            assert torch.all(out == SENTINEL), name
        ctx.set_workspace_limit(None)
        for got, want in zip(run_all(ctx, calls), reference_outputs):
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        # arenas already grown are kept: a limit below them fails nothing
        ctx.set_workspace_limit(4096)
        for got, want in zip(run_all(ctx, calls), reference_outputs):
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        del keep
    finally:
        ctx.close()


def test_failed_device_allocation_leaves_the_context_usable(reference_outputs):
    ctx = hip.Context(0)
    try:
        keep, calls = make_calls(ctx)
        pointer = C.c_void_p()
        print("case device_alloc 2**50 bytes", flush=True)
        status = ctx.lib.adi_hip_device_alloc(ctx.handle, C.c_size_t(1 << 50), C.byref(pointer))
        assert status == hip.OUT_OF_MEMORY
        assert pointer.value is None
        # the failed hipMalloc must not fail the launches that follow
        for got, want in zip(run_all(ctx, calls), reference_outputs):
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        del keep
    finally:
        ctx.close()
