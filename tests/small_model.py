"""A small hybrid model for the model-level GPU tests: three Gated DeltaNet
layers then one full-attention layer at hidden 256 (16 experts of 64), a
512-token vocabulary, uploaded once per module, and its oracle twin that
decodes one sequence token by token."""
import numpy as np

import pyoracle as po
from adi_amd import hip
from adi_amd import synthetic as syn

HIDDEN, EXPERT_HIDDEN, EXPERTS, VOCAB = 256, 64, 16, 512


def head_rows(h, first, end):
    per_row = h.columns // 8 * 5
    groups = h.columns // 64
    return syn.HeadChunk(end - first, h.columns,
                         h.packed.reshape(h.rows, per_row)[first:end].reshape(-1).copy(),
                         h.group_scale_f16.reshape(h.rows, groups)[first:end].reshape(-1).copy())


def build(gpu, seed: int = 70):
    """Host parts and two device models over the same layers: `one` with a
    single head chunk, `two` with the head split at row 200."""
    rng = syn.rng_for(seed, 0)
    etlut, ntlut = syn.expert_tlut(rng), syn.ne_tlut(rng)
    layers = [syn.decoder_layer(rng, i % 4 == 3, HIDDEN, EXPERT_HIDDEN, EXPERTS, etlut, ntlut)
              for i in range(4)]
    emb = syn.embedding(rng, VOCAB, HIDDEN, exceptions=20)
    head = syn.head_chunk(rng, VOCAB, HIDDEN)
    final_norm = syn.bf16_bits_rne(rng.normal(0.0, 0.1, HIDDEN).astype(np.float32))
    ebook, nbook = gpu.expert_codebook(etlut), gpu.ne_codebook(ntlut)
    dlayers = [hip.upload_decoder_layer(gpu, L, ebook, nbook) for L in layers]
    demb, dnorm = hip.upload_embedding(gpu, emb), gpu.to_device(final_norm)
    one = hip.Model(dlayers, demb, dnorm, [hip.upload_head(gpu, head)])
    two = hip.Model(dlayers, demb, dnorm, [hip.upload_head(gpu, head_rows(head, 0, 200)),
                                           hip.upload_head(gpu, head_rows(head, 200, VOCAB))])
    return dict(layers=layers, emb=emb, head=head, final_norm=final_norm, one=one, two=two)


class OracleSequence:
    """One sequence decoded by the oracle; step() returns the logits."""

    def __init__(self, parts, capacity: int):
        self.parts = parts
        self.held = [po.DecoderLayerStruct(L, capacity=capacity) for L in parts["layers"]]
        self.position = 0

    def step(self, oracle, token: int) -> np.ndarray:
        p = self.parts
        h = po.embedding_rows(oracle, p["emb"], [token])[0].copy()
        for held in self.held:
            held.decode(oracle, self.position, h, isa=16)
        self.position += 1
        n = np.zeros(HIDDEN, np.float32)
        assert oracle.ao_rms_norm(po.ptr(h, po.C.c_float), po.ptr(p["final_norm"], po.C.c_uint16),
                                  HIDDEN, 1.0, 1e-6, po.ptr(n, po.C.c_float)) == 0
        return po.head_matmul(oracle, p["head"], n[None, :], isa=16)[0]
