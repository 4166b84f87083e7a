"""Continuous batching on the device: the reference's ContinuousBatcher
(src/generation.cpp:343-660, include/adi/generation.hpp:75-95) over the
library's adi_hip_batcher, with token ids in place of text (the tokenizer
and chat template stay with the caller).

A worker thread runs the loop: while requests are pending or active it calls
adi_hip_batcher_step, one iteration of the reference's loop (admit the oldest
pending request by prefilling its prompt, sample every active sequence,
finish on a stop token or the output limit, decode the rest in one batched
step). While the same sequences keep stepping, their decode step is
recorded once as a HIP graph and replayed (replay_steps=False launches every
step directly; both give the same bits). generate() submits a request and blocks until it finishes, passing
each new token to `token_callback` as it appears and cancelling the request
when `cancelled()` turns true, as generate_from_prompt does. The worker owns
the context while the batcher runs: other work must not use it meanwhile."""
from __future__ import annotations

import ctypes as C
import threading
import time
from dataclasses import dataclass
from typing import Callable, Optional, Sequence

from . import hip

PENDING, RUNNING, STOP_TOKEN, LENGTH, FAILED = 0, 1, 2, 3, 4


@dataclass
class GenerationResult:
    """adi::GenerationResult (include/adi/generation.hpp:29-38) with token
    ids in place of text."""
    tokens: list
    input_tokens: int
    output_tokens: int
    finish_reason: str  # "stop_token" or "length"
    prefill_seconds: float
    decode_seconds: float


class GenerationError(RuntimeError):
    pass


class ContinuousBatcher:
    def __init__(self, ctx: hip.Context, model: hip.Model, max_batch: int = 16,
                 capacity: int = 4096, prefill_ubatch: int = 128,
                 stop_tokens: Sequence[int] = (), masked_tokens: Sequence[int] = (),
                 start: bool = True, replay_steps: bool = True):
        self.ctx, self.model = ctx, model
        stop = (hip.u32 * max(len(stop_tokens), 1))(*stop_tokens)
        masked = (hip.u32 * max(len(masked_tokens), 1))(*masked_tokens)
        options = hip.BatcherOptions(max_batch, capacity, prefill_ubatch, stop, len(stop_tokens),
                                     masked, len(masked_tokens), 0 if replay_steps else 1)
        handle = hip.vp()
        ctx.check(ctx.lib.adi_hip_batcher_create(ctx.handle, C.byref(model.struct),
                                                 C.byref(options), C.byref(handle)))
        self.handle = handle
        self._cond = threading.Condition()
        self._stop = False
        self._work = 0          # requests pending or active, as of the last step
        self._submitted = 0     # submissions so far
        self._steps = 0
        self._failure: Optional[hip.HipError] = None
        self._thread = None
        if start:
            self._thread = threading.Thread(target=self._run, name="adi-batcher", daemon=True)
            self._thread.start()

    # -- the worker loop (Impl::run, src/generation.cpp:540-660) --
    def _run(self):
        while True:
            with self._cond:
                idle = self._work == 0
                while not self._stop and self._work == 0:
                    self._cond.wait()
                if self._stop:
                    return
            if idle:
                # a short window makes simultaneous arrivals deterministic
                # without imposing meaningful latency on a lone request
                time.sleep(0.002)
            try:
                self.step()
            except hip.HipError as error:  # the decode step failed its requests
                self._failure = error
            with self._cond:
                self._cond.notify_all()

    def step(self) -> int:
        """One loop iteration; returns the requests still pending or active."""
        remaining = hip.u32()
        with self._cond:
            seen = self._submitted
        status = self.ctx.lib.adi_hip_batcher_step(self.handle, C.byref(remaining))
        with self._cond:
            # a request submitted during the step may be missing from its count
            self._work = remaining.value if self._submitted == seen else max(remaining.value, 1)
            self._steps += 1
            self._cond.notify_all()
        self.ctx.check(status)
        return remaining.value

    # -- requests --
    def submit(self, prompt: Sequence[int], max_output_tokens: Optional[int] = None,
               temperature: float = 0.7, top_p: float = 0.9, seed: int = 0) -> int:
        if max_output_tokens is not None and max_output_tokens <= 0:
            raise GenerationError("max_output_tokens must be positive")
        toks = (hip.u32 * max(len(prompt), 1))(*[int(t) for t in prompt])
        opts = hip.GenerationOptions(0 if max_output_tokens is None else max_output_tokens,
                                     temperature, top_p, seed)
        request = hip.u64()
        self.ctx.check(self.ctx.lib.adi_hip_batcher_submit(self.handle, toks, len(prompt),
                                                           C.byref(opts), C.byref(request)))
        with self._cond:
            self._submitted += 1
            self._work += 1
            self._cond.notify_all()
        return request.value

    def cancel(self, request: int) -> None:
        self.ctx.check(self.ctx.lib.adi_hip_batcher_cancel(self.handle, request))

    def status(self, request: int):
        """(state, tokens so far, RequestStatus)."""
        st = hip.RequestStatus()
        cap = 1 << 16
        buf = (hip.u32 * cap)()
        self.ctx.check(self.ctx.lib.adi_hip_batcher_status(self.handle, request, C.byref(st), buf,
                                                           cap))
        return st.state, list(buf[:min(st.output_tokens, cap)]), st

    def result(self, request: int) -> GenerationResult:
        """The finished request's result (its error raised if it failed);
        the request is released."""
        state, tokens, st = self.status(request)
        if state in (PENDING, RUNNING):
            raise GenerationError("request has not finished")
        error = self.ctx.lib.adi_hip_batcher_request_error(self.handle, request).decode()
        self.ctx.lib.adi_hip_batcher_release(self.handle, request)
        if state == FAILED:
            raise GenerationError(error)
        return GenerationResult(tokens, st.input_tokens, st.output_tokens,
                                "stop_token" if state == STOP_TOKEN else "length",
                                st.prefill_seconds, st.decode_seconds)

    def generate(self, prompt: Sequence[int], max_output_tokens: Optional[int] = None,
                 temperature: float = 0.7, top_p: float = 0.9, seed: int = 0,
                 token_callback: Optional[Callable[[int], None]] = None,
                 cancelled: Optional[Callable[[], bool]] = None) -> GenerationResult:
        """generate_from_prompt (src/generation.cpp:662-676) on token ids."""
        if self._thread is None:
            raise GenerationError("the batcher was created without its worker thread")
        request = self.submit(prompt, max_output_tokens, temperature, top_p, seed)
        sent = 0
        while True:
            with self._cond:
                self._cond.wait(timeout=0.05)
            state, tokens, _ = self.status(request)
            if token_callback is not None:
                try:
                    for t in tokens[sent:]:
                        token_callback(t)
                except BaseException:
                    self.cancel(request)  # Request::callback_failed
                    raise
                sent = len(tokens)
            if cancelled is not None and state in (PENDING, RUNNING) and cancelled():
                self.cancel(request)
            if state not in (PENDING, RUNNING):
                return self.result(request)
            if self._thread is not None and not self._thread.is_alive():
                raise GenerationError("continuous batcher stopped")

    def close(self) -> None:
        if self._thread is not None:
            with self._cond:
                self._stop = True
                self._cond.notify_all()
            self._thread.join()
            self._thread = None
        if self.handle:
            self.ctx.lib.adi_hip_batcher_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
