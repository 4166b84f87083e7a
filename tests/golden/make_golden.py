"""Writes the golden vectors in tests/golden/golden.npz from the reference's
own CPU path (oracle/_ref/libadi_ref.so, compiled from the reference sources
by `make -C oracle ref`).

Every array is data: seeded inputs and the outputs the compiled reference
returned for them. Run in the container that has the reference sources:

    python tests/golden/make_golden.py

Cases (the reference functions they come from):
  expert/NE tile walks ........ for_each_expert_state / for_each_ne_state
                                (src/expert_trellis.hpp:44-59, src/ne_trellis.hpp:27-41)
  state tables ................ build_expert_state_values / build_ne_state_values /
                                build_ne_signed_tlut (src/codec_cache.cpp:33-115):
                                sampled rows + SHA-256 of the full tables
  wave indexes ................ build_wave_indexes (src/codec_cache.cpp:117-147)
  f16 conversions ............. f32_to_f16 / f16_to_f32 (src/kernels.cpp:309-379)
  expert / NE projections ..... mach_expert_matmul / mach_ne_matmul
  int5 head ................... mach_head_matmul under scalar, AVX2 and AVX-512
  bf16 dense .................. bf16_matmul under scalar, AVX2 and AVX-512
  top_experts ................. src/executor.cpp:193-229, with forced ties
  MoE block ................... the reference entry points composed in
                                moe_forward / moe_forward_batch order
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "oracle"))

import pyoracle as po  # noqa: E402
from adi_amd import synthetic as syn  # noqa: E402


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def main():
    ref = po.load_ref()
    out = {}
    rng = syn.rng_for(9, 0)

    # tile walks: degenerate streams then random ones
    tiles = [np.zeros(24, np.uint16), np.full(24, 0xFFFF, np.uint16)]
    for word in range(24):
        for bit in (0, 7, 15):
            t = np.zeros(24, np.uint16)
            t[word] = 1 << bit
            tiles.append(t)
    tiles += [syn.uniform_words(rng, 24) for _ in range(64)]
    et = np.stack(tiles)
    es = np.zeros((len(et), 32), np.uint16)
    for i, t in enumerate(et):
        ref.ref_expert_tile_states(po.ptr(t, po.C.c_uint16), po.ptr(es[i], po.C.c_uint16))
    out["expert_tiles"], out["expert_states"] = et, es
    ntiles = [np.zeros(64, np.uint16), np.full(64, 0xFFFF, np.uint16)]
    for word in (0, 1, 31, 62, 63):
        t = np.zeros(64, np.uint16)
        t[word] = 0x8001
        ntiles.append(t)
    ntiles += [syn.uniform_words(rng, 64) for _ in range(32)]
    nt = np.stack(ntiles)
    ns = np.zeros((len(nt), 128), np.uint16)
    for i, t in enumerate(nt):
        ref.ref_ne_tile_states(po.ptr(t, po.C.c_uint16), po.ptr(ns[i], po.C.c_uint16))
    out["ne_tiles"], out["ne_states"] = nt, ns

    # state tables for a seeded TLUT
    etlut = syn.expert_tlut(rng)
    ntlut = syn.ne_tlut(rng)
    ev = np.zeros(65536 * 8, np.float32)
    nv = np.zeros(65536 * 2, np.float32)
    sv = np.zeros(1024 * 2, np.float32)
    ref.ref_build_expert_state_values(po.ptr(etlut, po.C.c_float), po.ptr(ev, po.C.c_float))
    ref.ref_build_ne_state_values(po.ptr(ntlut, po.C.c_float), po.ptr(nv, po.C.c_float))
    ref.ref_build_ne_signed_tlut(po.ptr(ntlut, po.C.c_float), po.ptr(sv, po.C.c_float))
    sample = np.sort(rng.choice(65536, 512, replace=False)).astype(np.uint32)
    out["expert_tlut"], out["ne_tlut"] = etlut, ntlut
    out["table_sample_states"] = sample
    out["expert_state_values_sample"] = ev.reshape(65536, 8)[sample]
    out["ne_state_values_sample"] = nv.reshape(65536, 2)[sample]
    out["ne_signed_tlut"] = sv
    out["expert_state_values_sha256"] = np.array(sha(ev))
    out["ne_state_values_sha256"] = np.array(sha(nv))

    # wave indexes
    shapes = [(1, 1), (1, 4), (4, 1), (2, 3), (32, 128), (128, 32), (5, 7), (16, 16)]
    for r, c in shapes:
        w = np.zeros(r * c, np.uint16)
        po.check(ref.ref_build_wave_indexes(r, c, po.ptr(w, po.C.c_uint16)), "waves")
        out[f"waves_{r}x{c}"] = w

    # f16 conversions
    special = np.array([0.0, -0.0, 1.0, -2.0, 0.333251953125, 65504.0, 65520.0, 1e-8, 2.0 ** -24,
                        2.0 ** -25, 3 * 2.0 ** -26, 2.0 ** -14, 6.1e-5, np.inf, -np.inf, np.nan,
                        1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 1e5], np.float32)
    values = np.concatenate([special, rng.normal(0, 1, 2000).astype(np.float32),
                             rng.lognormal(0, 4, 2000).astype(np.float32),
                             (rng.uniform(-1, 1, 1000) * 2.0 ** -14).astype(np.float32)])
    out["f32_values"] = values
    out["f32_to_f16"] = np.array([ref.ref_f32_to_f16(float(v)) for v in values], np.uint16)
    all_half = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    out["f16_to_f32_all_sha256"] = np.array(sha(np.array([ref.ref_f16_to_f32(int(h)) for h in all_half],
                                                         np.float32)))

    # projections
    for (r, c) in [(16, 16), (64, 32), (32, 128)]:
        m = syn.expert_matrix(rng, r, c, etlut)
        x = syn.hidden_states(rng, 4, c)
        for key, val in (("trellis", m.trellis), ("su", m.su_f16), ("sv", m.sv_f16),
                         ("gamma", m.wave_gamma_f16), ("x", x)):
            out[f"expert_{r}x{c}_{key}"] = val
        for b in (1, 2, 4):
            out[f"expert_{r}x{c}_y{b}"] = po.expert_matmul(ref, m, x[:b], prefix="ref")
        n = syn.ne_matrix(rng, r, c, ntlut)
        xn = syn.hidden_states(rng, 4, c)
        for key, val in (("trellis", n.trellis), ("su", n.su), ("sv", n.sv), ("x", xn),
                         ("scale", np.array([n.weight_scale], np.float32))):
            out[f"ne_{r}x{c}_{key}"] = val
        for b in (1, 3):
            out[f"ne_{r}x{c}_y{b}"] = po.ne_matmul(ref, n, xn[:b], prefix="ref")

    # int5 head and bf16 dense under the three ISA orders
    h = syn.head_chunk(rng, 37, 128, protected=2)
    xh = syn.rms_normalized(syn.hidden_states(rng, 3, 128))
    out.update(head_packed=h.packed, head_scales=h.group_scale_f16, head_protected_rows=h.protected_rows,
               head_protected_bf16=h.protected_bf16, head_x=xh)
    w = syn.bf16_bits_rne(rng.normal(0, 0.02, (5, 67)).astype(np.float32))
    xb = syn.hidden_states(rng, 2, 67)
    out.update(bf16_w=w, bf16_x=xb)
    for lanes in (1, 8, 16):
        ref.ref_force_isa_lanes(lanes)
        out[f"head_y_isa{lanes}"] = po.head_matmul(ref, h, xh, prefix="ref")
        out[f"bf16_y_isa{lanes}"] = po.bf16_matmul(ref, w, xb, prefix="ref")
    ref.ref_force_isa_lanes(0)

    # top_experts with forced ties
    logits = rng.normal(0, 1, (40, 256)).astype(np.float32)
    logits[::3] = np.round(logits[::3] * 2)
    logits[1] = 0.0
    out["topk_logits"] = logits
    res = [po.top_experts(ref, row, prefix="ref") for row in logits]
    out["topk_experts"] = np.stack([r[0] for r in res])
    out["topk_weights"] = np.stack([r[1] for r in res])

    # a small MoE block
    layer = syn.moe_layer(rng, hidden=256, expert_hidden=64, experts=16, etlut=etlut, ntlut=ntlut)
    out["moe_router"] = layer.router_bf16
    out["moe_shared_gate_w"] = layer.shared_expert_gate_bf16
    for name, mats in (("gate", layer.gate), ("up", layer.up), ("down", layer.down)):
        t, su, sv_, g = (np.stack(a) for a in zip(*[(m.trellis, m.su_f16, m.sv_f16, m.wave_gamma_f16)
                                                      for m in mats]))
        out.update({f"moe_{name}_trellis": t, f"moe_{name}_su": su, f"moe_{name}_sv": sv_,
                    f"moe_{name}_gamma": g})
    for name, m in (("sgate", layer.shared_gate), ("sup", layer.shared_up), ("sdown", layer.shared_down)):
        out.update({f"moe_{name}_trellis": m.trellis, f"moe_{name}_su": m.su, f"moe_{name}_sv": m.sv,
                    f"moe_{name}_scale": np.array([m.weight_scale], np.float32)})
    bias = syn.zipf_bias(rng, 16)
    xm = syn.hidden_states(rng, 5, 256)
    out.update(moe_bias=bias, moe_x=xm)
    ref.ref_force_isa_lanes(16)
    rl = po.RefMoeLayer(ref, layer)
    for b, use_bias in ((1, False), (5, False), (5, True)):
        y, e, wt = rl.forward(xm[:b], bias if use_bias else None)
        tag = f"b{b}{'_bias' if use_bias else ''}"
        out.update({f"moe_y_{tag}": y, f"moe_experts_{tag}": e, f"moe_weights_{tag}": wt})
    rl.close()
    ref.ref_force_isa_lanes(0)

    path = os.path.join(HERE, "golden.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main()
