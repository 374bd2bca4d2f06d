"""Python harness over the engine_* entry points of libsardyne.so.

A ``LoadedModel`` owns one engine_model (weights in GPU memory); ``LoadedModel.session`` opens an
engine_ctx (KV cache and working memory in GPU memory) wrapped as a ``Session``. A session is fed
token ids and returns the logits the engine left in its host buffer, copied out. Engine errors
surface as ``ValueError`` carrying the engine's own message (the messages callers match on, e.g.
"contesto pieno" or "vocabolario").

This is the build's test and benchmark harness, not a copy of the reference's Python runtime: the
reference's own ``sardyne/runtime.py`` binds this library unchanged through ``SARDYNE_LIB``.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

from sardyne_amd import capi

_I32 = np.iinfo(np.int32)


def _message(raw: bytes | None) -> str:
    return (raw or b"").decode("utf-8", errors="replace")


class LoadedModel:
    """A GGUF file (llama / qwen2 / qwen3 / qwen3moe) uploaded to the GPU."""

    def __init__(self, path):
        self.path = Path(path)
        self._lib = capi.lib()
        err = ctypes.create_string_buffer(512)
        self._h = self._lib.engine_model_load(str(self.path).encode(), err, len(err))
        if not self._h:
            raise ValueError(_message(err.value))
        self.info = capi.EngineModelInfo()
        self._lib.engine_model_get_info(self._h, ctypes.byref(self.info))

    @property
    def n_vocab(self) -> int:
        return self.info.n_vocab

    def memory(self) -> dict:
        """Memory the model holds (sdy_model_memory, sdy_model_host_weights): weight bytes in device
        memory, the prefill GEMM's tiled copies and how many matrices got a copy / were left without
        one, and the expert stacks kept in pinned host memory (bytes, layers)."""
        w, g, nc, ns = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_int(), ctypes.c_int()
        capi.check(self._lib.sdy_model_memory(self._h, ctypes.byref(w), ctypes.byref(g), ctypes.byref(nc),
                                              ctypes.byref(ns)))
        hb, hl = ctypes.c_size_t(), ctypes.c_int()
        capi.check(self._lib.sdy_model_host_weights(self._h, ctypes.byref(hb), ctypes.byref(hl)))
        return {"weight_bytes": w.value, "gemm_copy_bytes": g.value, "gemm_copies": nc.value,
                "gemm_copies_skipped": ns.value, "host_expert_bytes": hb.value, "host_expert_layers": hl.value}

    def session(self, max_seq: int = 2048, n_batch: int = 64, logits_all: bool = False,
                n_threads: int = 0) -> "Session":
        return Session(self, max_seq, n_batch, logits_all, n_threads)

    def close(self):
        h, self._h = getattr(self, "_h", None), None
        if h:
            self._lib.engine_model_free(h)

    __del__ = close

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


class Session:
    """One engine context: a KV cache of ``max_seq`` positions, evaluated ``n_batch`` tokens per
    forward. With ``logits_all`` every fed token's logits are returned, else the last one's."""

    def __init__(self, model: LoadedModel, max_seq: int, n_batch: int, logits_all: bool, n_threads: int):
        self.model = model  # the context reads the model's weights: keep it alive
        self._lib = model._lib
        self._h = None
        self.max_seq = min(int(max_seq), model.info.max_pos)
        self.n_batch = int(n_batch)
        self.logits_all = bool(logits_all)
        err = ctypes.create_string_buffer(512)
        self._h = self._lib.engine_ctx_new(model._h, self.max_seq, self.n_batch, int(self.logits_all), int(n_threads),
                                           err, len(err))
        if not self._h:
            raise ValueError(_message(err.value))
        self.n_threads = self._lib.engine_ctx_n_threads(self._h)

    @property
    def position(self) -> int:
        """Tokens held in the KV cache (engine_n_past)."""
        return self._lib.engine_n_past(self._h)

    def _raise(self):
        raise ValueError(_message(self._lib.engine_last_error(self._h)))

    def _eval(self, ids: np.ndarray) -> np.ndarray:
        ptr = ids.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))
        if self._lib.engine_eval(self._h, ptr, int(ids.size)) != 0:
            self._raise()
        rows = self._lib.engine_n_logits(self._h)
        buf = self._lib.engine_logits(self._h)
        return np.ctypeslib.as_array(buf, shape=(rows, self.model.n_vocab)).copy()

    def feed(self, tokens) -> np.ndarray:
        """Evaluates the tokens after the cached ones. Returns [n, vocab] logits with logits_all
        (fed in n_batch pieces, the engine's limit for that mode), else the last token's [vocab]."""
        ids = np.asarray(tokens, dtype=np.int64).reshape(-1)
        if ids.size and (ids.min() < _I32.min or ids.max() > _I32.max):
            raise ValueError("id di token fuori dall'intervallo int32")
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        if not self.logits_all:
            return self._eval(ids)[-1]
        if ids.size == 0:
            return self._eval(ids)  # the engine's own "nessun token" error
        return np.concatenate([self._eval(ids[i:i + self.n_batch]) for i in range(0, ids.size, self.n_batch)])

    def step(self, token: int) -> np.ndarray:
        """One token: the decode step."""
        out = self.feed([int(token)])
        return out[-1] if self.logits_all else out

    def rewind(self, n: int):
        """Keeps the first n cached positions (engine_truncate)."""
        if self._lib.engine_truncate(self._h, int(n)) != 0:
            self._raise()

    def clear(self):
        self._lib.engine_reset(self._h)

    def close(self):
        h, self._h = getattr(self, "_h", None), None
        if h:
            self._lib.engine_ctx_free(h)

    __del__ = close


def greedy(session: Session, prompt, n_new: int, stop=()) -> list[int]:
    """Clears the session, feeds the prompt, then appends argmax tokens one step at a time until
    n_new tokens, a stop id, or a full context. Returns the new tokens."""
    stop = {stop} if isinstance(stop, int) else set(stop)
    out: list[int] = []
    if n_new <= 0:
        return out
    session.clear()
    logits = session.feed(prompt)
    while True:
        if logits.ndim == 2:
            logits = logits[-1]
        nxt = int(np.argmax(logits))
        out.append(nxt)
        if len(out) == n_new or nxt in stop or session.position >= session.max_seq:
            return out
        logits = session.step(nxt)
