"""Continuous-batching request scheduler over the C ABI (``mla_scheduler_*``).

The reference's server (src/serve/server.cpp) runs one request at a time on each of its
worker threads' private sessions; ``Scheduler`` serves all requests from one stepping
thread in the library that batches their decode tokens and prompt chunks into
``mla_engine_step`` calls, with the server's bounded queue, deadlines, cancellation,
request limits and metrics.  The HTTP layer is the caller's.
"""
from __future__ import annotations

import codecs
import contextlib
import ctypes as C
import threading
import time

import numpy as np

from . import MlaError, check, lib
from .generation import GenerationConfig, c_config


class _SchedulerConfig(C.Structure):
    _fields_ = [("max_context", C.c_int), ("max_new_tokens", C.c_int), ("max_queue", C.c_int),
                ("request_timeout_seconds", C.c_int)]


class _Status(C.Structure):
    _fields_ = [("done", C.c_int), ("error", C.c_int), ("error_message", C.c_char * 240),
                ("finish_reason", C.c_char * 16), ("prompt_tokens", C.c_uint64),
                ("completion_tokens", C.c_uint64), ("queue_seconds", C.c_double),
                ("prefill_seconds", C.c_double), ("decode_seconds", C.c_double),
                ("first_token_seconds", C.c_double)]


class _Metrics(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in ("requests", "completed", "rejected", "errors",
                                          "generated_tokens")] + \
               [(n, C.c_double) for n in ("queue_seconds", "prefill_seconds", "decode_seconds",
                                          "first_token_seconds")] + \
               [(n, C.c_uint64) for n in ("queue_depth", "running", "steps")]


class Scheduler:
    """ServerConfig's limits (include/mini_mla/server.hpp:5-10): max_context,
    max_new_tokens, max_queue, request_timeout_seconds."""

    def __init__(self, engine, tokenizer, max_context: int = 2048, max_new_tokens: int = 128,
                 max_queue: int = 16, request_timeout_seconds: int = 60):
        c = _SchedulerConfig(max_context, max_new_tokens, max_queue, request_timeout_seconds)
        h = C.c_void_p()
        # Calls in progress on other threads, so close() never frees the scheduler under
        # one of them (a server's handler threads poll while it shuts down).
        self._cv = threading.Condition()
        self._active, self._closing = 0, False
        check(lib().mla_scheduler_create(engine.handle, tokenizer._h, C.byref(c), C.byref(h)))
        self._lib = lib()  # used by close(), which may run at interpreter exit
        self._h, self.engine, self.tokenizer = h, engine, tokenizer
        self.max_new_tokens = max_new_tokens
        engine._attach(self)  # closing the engine stops this scheduler first

    @contextlib.contextmanager
    def _use(self):
        with self._cv:
            if not getattr(self, "_h", None) or self._closing:
                raise MlaError(7, "Scheduler is closed")
            self._active += 1
            h = self._h
        try:
            yield h
        finally:
            with self._cv:
                self._active -= 1
                self._cv.notify_all()

    def close(self):
        """Stops the scheduler (queued requests never start, running ones end as
        cancelled, waiting polls return), waits for calls in progress on other threads,
        then frees it."""
        cv = getattr(self, "_cv", None)
        if cv is None:
            return
        with cv:
            h = getattr(self, "_h", None)
            if not h or self._closing:
                return
            self._closing = True
        self._lib.mla_scheduler_stop(h)
        with cv:
            cv.wait_for(lambda: self._active == 0)
            self._h = None
        self._lib.mla_scheduler_destroy(h)

    def __del__(self):
        self.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def submit(self, prompt_ids, config: GenerationConfig | None = None, stream: bool = False,
               max_tokens_given: bool = True) -> int:
        """Queues prompt_ids (<|bos|> included).  max_tokens_given=False: the server's
        default token budget min(max_new_tokens, max_context - len(prompt))."""
        ids = np.ascontiguousarray(prompt_ids, dtype=np.uint16).ravel()
        c, keep = c_config(config, max_new_tokens_default=not max_tokens_given)
        rid = C.c_uint64()
        with self._use() as h:
            check(lib().mla_scheduler_submit(h, ids.ctypes.data, ids.size, C.byref(c),
                                             int(stream), C.byref(rid)))
        del keep
        return rid.value

    def submit_text(self, prompt: str, config: GenerationConfig | None = None,
                    stream: bool = False, max_tokens_given: bool = True) -> int:
        """A completion request: <|bos|> + encode(prompt) (server.cpp:297-299)."""
        ids = [self.tokenizer.special("<|bos|>")] + self.tokenizer.encode(prompt).tolist()
        return self.submit(ids, config, stream, max_tokens_given)

    def cancel(self, rid: int) -> None:
        with self._use() as h:
            check(lib().mla_scheduler_cancel(h, rid))

    def poll(self, rid: int, timeout: float = 0.0):
        """(new text bytes, status dict); status["done"] once the request has ended (it is
        then forgotten), with "tokens" holding the generated ids."""
        buf = C.create_string_buffer(1 << 16)
        n = C.c_size_t()
        tokens = np.empty(65536, np.uint16)
        st = _Status()
        with self._use() as h:
            check(lib().mla_scheduler_poll(h, rid, int(timeout * 1000), buf, len(buf),
                                           C.byref(n), tokens.ctypes.data, tokens.size,
                                           C.byref(st)))
        status = {k: getattr(st, k) for k, _ in _Status._fields_}
        status["error_message"] = st.error_message.decode(errors="replace")
        status["finish_reason"] = st.finish_reason.decode()
        if st.done:
            status["tokens"] = tokens[:st.completion_tokens].tolist()
        return buf.raw[:n.value], status

    def stream(self, rid: int, timeout: float = 120.0):
        """Yields text chunks as they come; returns the final status (StopIteration.value)."""
        end = time.monotonic() + timeout
        utf8 = codecs.getincrementaldecoder("utf-8")()  # a poll may end inside a character
        while True:
            text, status = self.poll(rid, 0.05)
            chunk = utf8.decode(text, final=bool(status["done"]))
            if chunk:
                yield chunk
            if status["done"]:
                return status
            if time.monotonic() > end:
                raise TimeoutError(f"request {rid} still running after {timeout} s")

    def result(self, rid: int, timeout: float = 120.0) -> dict:
        """Waits for the end: text (all of it), tokens, finish_reason, error, timings.
        Raises MlaError when the request failed."""
        chunks, gen = [], self.stream(rid, timeout)
        while True:
            try:
                chunks.append(next(gen))
            except StopIteration as stop:
                status = stop.value
                break
        if status["error"]:
            raise MlaError(status["error"], status["error_message"])
        status["text"] = "".join(chunks)
        return status

    def metrics(self) -> dict:
        m = _Metrics()
        with self._use() as h:
            check(lib().mla_scheduler_metrics_get(h, C.byref(m)))
        return {k: getattr(m, k) for k, _ in _Metrics._fields_}

    def metrics_text(self) -> str:
        n = C.c_size_t()
        with self._use() as h:
            check(lib().mla_scheduler_metrics_text(h, None, 0, C.byref(n)))
            buf = C.create_string_buffer(n.value + 1)
            check(lib().mla_scheduler_metrics_text(h, buf, len(buf), C.byref(n)))
        return buf.raw[:n.value].decode()


__all__ = ["Scheduler"]
