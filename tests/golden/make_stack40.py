"""Writes tests/golden/stack40.npz: the oracle's run of the full hybrid
decoder stack, the fixture tests/test_gpu_stack40.py compares the device run
with.

The stack (adi_amd.synthetic.StackGeometry): 40 layers at hidden 2048, every
fourth full GQA attention (16 query / 2 KV heads of 256) and the others Gated
DeltaNet, each with the 256-expert top-8 MoE block and a shared expert; a
151,936-token int4 embedding and int5 head; random-init packed weights from
seeds. The oracle runs it the way decode_layer does, token by token
(src/executor.cpp:1473-1529): the 256 prompt tokens, then the final norm and
head on the last one, then 64 greedy decode steps (temperature 0, the first
maximum, src/generation.cpp:177-183), each feeding back the token it chose.
The reference's prefill (src/executor.cpp:1827-2101) computes the same
quantities for a chunk at once; the device's prefill is compared with this
token-by-token run.

Recorded:
  prompt, tokens         the prompt and the 65 greedy tokens (after the
                         prompt, then after each decode step)
  margin, logit_max      per head evaluation: top-1 minus top-2 logit, and
                         the largest |logit|
  logits_prefill         all logits after the prompt
  logits_final           all logits after the last decode step
  hidden_prefill         [40, 2048] the last prompt token's row after each layer
  state_max              [40, 2] the largest |value| of each layer's two state
                         tensors (keys and values, or convolution and
                         recurrent) at the end
  state_sample           [40, 2, SAMPLES] those tensors at seeded indexes
                         (state_sample_indexes)
  state_fnv              [40, 2] FNV-1a of each tensor's float bits
  checksum               decoder_state_checksum over every layer
                         (src/main.cpp:105-117)

    python tests/golden/make_stack40.py      # about ten minutes on 8 cores

The prompt runs through the layers as a pipeline of 8 host threads (thread k
owns five consecutive layers; each layer still sees its tokens in order), so
the result is the plain token-by-token one.
"""
from __future__ import annotations

import ctypes
import os
import queue
import sys
import threading
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "oracle"))

import pyoracle as po  # noqa: E402
from adi_amd import synthetic as syn  # noqa: E402

OUT = os.path.join(HERE, "stack40.npz")
SAMPLES = 2048
FNV_OFFSET = 0xCBF29CE484222325


def state_sample_indexes(layer: int, tensor: int, size: int) -> np.ndarray:
    """Seeded flat indexes into tensor `tensor` (0: keys or convolution, 1:
    values or recurrent) of layer `layer`."""
    rng = np.random.default_rng([syn.SEED_BASE + syn.STACK_CONFIG, 7, layer, tensor])
    return np.sort(rng.choice(size, SAMPLES, replace=False))


def layer_tensors(held, position: int):
    """The layer's two state tensors as the reference holds them: the keys and
    values of positions 0..position-1, or the convolution and recurrent state."""
    if held.full is not None:
        return held.keys[:position].ravel(), held.values[:position].ravel()
    return held.convolution, held.recurrent


def decoder_state_checksum(lib, position: int, tensors) -> int:
    """FNV-1a over the position, then each layer's keys, values, convolution
    and recurrent floats (the empty ones add nothing), src/main.cpp:105-117."""
    h = FNV_OFFSET
    pos = np.array([position], np.uint32)
    h = lib.ao_fnv1a64(h, pos.ctypes.data, 4)
    for a, b in tensors:
        for t in (a, b):
            t = np.ascontiguousarray(t, np.float32)
            h = lib.ao_fnv1a64(h, t.ctypes.data, t.nbytes)
    return h


def top2_margin(logits: np.ndarray):
    top = np.partition(logits, -2)[-2:]
    return float(top.max() - top.min()), float(np.abs(logits).max())


def main(argv=None) -> None:
    import argparse
    p = argparse.ArgumentParser()
    p.add_argument("--layers", type=int, default=40)
    p.add_argument("--prompt", type=int, default=256)
    p.add_argument("--steps", type=int, default=64)
    p.add_argument("--out", default=OUT, help="a shortened run (to try the script) writes elsewhere")
    args = p.parse_args(argv)
    g = syn.StackGeometry(layers=args.layers, prompt=args.prompt, greedy_steps=args.steps)
    lib = po.load_oracle()
    t0 = time.time()
    etlut, ntlut = syn.stack_codebooks()
    layers = [syn.stack_layer(g, i, etlut, ntlut) for i in range(g.layers)]
    emb, head, final_norm, prompt = syn.stack_token_side(g)
    capacity = g.prompt + g.greedy_steps
    held = [po.DecoderLayerStruct(L, capacity=capacity) for L in layers]
    print(f"model drawn in {time.time() - t0:.0f} s", flush=True)

    def head_logits(h):
        n = np.zeros(g.hidden, np.float32)
        po.check(lib.ao_rms_norm(po.ptr(h, po.C.c_float), po.ptr(final_norm, po.C.c_uint16),
                                 g.hidden, 1.0, 1e-6, po.ptr(n, po.C.c_float)), "rms_norm")
        return po.head_matmul(lib, head, n[None, :], isa=16)[0]

    # prompt: a pipeline over the layers, each thread single-threaded inside
    rows = po.embedding_rows(lib, emb, prompt)
    stages = 8
    per = (g.layers + stages - 1) // stages
    groups = [list(range(i, min(i + per, g.layers))) for i in range(0, g.layers, per)]
    queues = [queue.Queue() for _ in range(len(groups) + 1)]
    hidden_prefill = np.zeros((g.layers, g.hidden), np.float32)
    failures = []
    gomp = ctypes.CDLL("libgomp.so.1")

    def worker(k):
        try:
            gomp.omp_set_num_threads(1)
            for _ in range(g.prompt):
                t, h = queues[k].get()
                if h is None:
                    queues[k + 1].put((t, None))
                    return
                for i in groups[k]:
                    held[i].decode(lib, t, h, isa=16)
                    if t == g.prompt - 1:
                        hidden_prefill[i] = h
                queues[k + 1].put((t, h))
        except Exception as exc:  # noqa: BLE001 -- reported after the join
            failures.append(exc)
            queues[k + 1].put((0, None))

    threads = [threading.Thread(target=worker, args=(k,)) for k in range(len(groups))]
    for th in threads:
        th.start()
    t0 = time.time()
    for t in range(g.prompt):
        queues[0].put((t, rows[t].copy()))
    last = None
    for n in range(g.prompt):
        t, h = queues[-1].get()
        if h is None:
            break
        last = h
        if n % 32 == 31:
            print(f"prompt token {n + 1}/{g.prompt} ({time.time() - t0:.0f} s)", flush=True)
    for th in threads:
        th.join()
    if failures:
        raise failures[0]

    logits = head_logits(last)
    logits_prefill = logits.copy()
    tokens = [int(lib.ao_argmax(po.ptr(logits, po.C.c_float), g.vocab))]
    margins, maxima = [top2_margin(logits)[0]], [top2_margin(logits)[1]]
    for step in range(g.greedy_steps):
        position = g.prompt + step
        h = po.embedding_rows(lib, emb, [tokens[-1]])[0].copy()
        for L in held:
            L.decode(lib, position, h, isa=16)
        logits = head_logits(h)
        tokens.append(int(lib.ao_argmax(po.ptr(logits, po.C.c_float), g.vocab)))
        m, mx = top2_margin(logits)
        margins.append(m)
        maxima.append(mx)
        if step % 8 == 7:
            print(f"decode step {step + 1}/{g.greedy_steps} ({time.time() - t0:.0f} s)", flush=True)

    end = g.prompt + g.greedy_steps
    tensors = [layer_tensors(L, end) for L in held]
    state_max = np.zeros((g.layers, 2), np.float32)
    state_sample = np.zeros((g.layers, 2, SAMPLES), np.float32)
    state_fnv = np.zeros((g.layers, 2), np.uint64)
    for i, pair in enumerate(tensors):
        for j, t in enumerate(pair):
            t = np.ascontiguousarray(t, np.float32)
            state_max[i, j] = np.abs(t).max()
            state_sample[i, j] = t[state_sample_indexes(i, j, t.size)]
            state_fnv[i, j] = lib.ao_fnv1a64(FNV_OFFSET, t.ctypes.data, t.nbytes)
    checksum = decoder_state_checksum(lib, end, tensors)
    np.savez_compressed(
        args.out, prompt=prompt, tokens=np.array(tokens, np.uint32),
        margin=np.array(margins, np.float32), logit_max=np.array(maxima, np.float32),
        logits_prefill=logits_prefill, logits_final=logits, hidden_prefill=hidden_prefill,
        state_max=state_max, state_sample=state_sample, state_fnv=state_fnv,
        checksum=np.array([checksum], np.uint64))
    print(f"wrote {args.out}: tokens {tokens[:8]}..., checksum {checksum:#018x}, "
          f"{time.time() - t0:.0f} s", flush=True)


if __name__ == "__main__":
    main()
