"""Micro-batching embedding engine (src/webgpu/embedding-engine.ts:1-95).

Same contract as the reference: ``embed(text)`` tokenizes, prepends BOS,
queues the request and resolves with that request's embedding; a flush takes
up to ``max_batch_size`` queued requests (capped by the runtime's storage
limit and to 8 for sequences of 1500+ tokens), pads each after its tokens
with ``pad_token``, runs one plan per ``batch:sequence`` key, and resolves
(or rejects) every request of the batch. asyncio stands in for the JS event
loop: ``call_later(batch_window_ms)`` for ``setTimeout``, futures for
promises.
"""
from __future__ import annotations

import asyncio
import math
from dataclasses import dataclass
from typing import Any, Callable, Protocol

import numpy as np


class TokenizerResult(Protocol):
    input_ids: Any  # has .tolist() -> list[list[int]]


TokenizerLike = Callable[[str], TokenizerResult]


class EmbeddingPlan(Protocol):
    async def run(self, ids: np.ndarray, lengths: np.ndarray) -> list: ...


class EmbeddingRuntime(Protocol):
    maxStorageBufferBindingSize: int | None

    def createPlan(self, batch: int, sequence: int) -> EmbeddingPlan: ...  # noqa: N802


@dataclass
class _Pending:
    tokens: list[int]
    future: asyncio.Future


class NemotronEmbeddingEngine:
    """Micro-batches simultaneous embedding calls onto one execution plan."""

    def __init__(self, runtime: EmbeddingRuntime, tokenizer: TokenizerLike, max_batch_size: int = 16,
                 batch_window_ms: float = 0, bos_token: int = 1, pad_token: int = 11):
        if max_batch_size < 1 or max_batch_size > 16:
            raise ValueError("maxBatchSize must be between 1 and 16")
        self.runtime = runtime
        self.tokenizer = tokenizer
        self.max_batch_size = max_batch_size
        self.batch_window_ms = batch_window_ms
        self.bos_token = bos_token
        self.pad_token = pad_token
        self._pending: list[_Pending] = []
        self._plans: dict[str, EmbeddingPlan] = {}
        self._scheduled = False
        self._flushing = False

    def embed(self, text: str) -> asyncio.Future:
        """src/webgpu/embedding-engine.ts:40-47."""
        tokens = [int(t) for t in self.tokenizer(text).input_ids.tolist()[0]]
        if not tokens or tokens[0] != self.bos_token:
            tokens.insert(0, self.bos_token)
        future = asyncio.get_running_loop().create_future()
        self._pending.append(_Pending(tokens, future))
        self._schedule()
        return future

    def _schedule(self) -> None:
        if self._scheduled or self._flushing:
            return
        self._scheduled = True

        def fire():
            self._scheduled = False
            asyncio.ensure_future(self._flush())

        asyncio.get_running_loop().call_later(self.batch_window_ms / 1000.0, fire)

    async def _flush(self) -> None:
        """src/webgpu/embedding-engine.ts:58-95."""
        if self._flushing:
            return
        self._flushing = True
        try:
            while self._pending:
                candidates = self._pending[: self.max_batch_size]
                candidate_sequence = max(len(r.tokens) for r in candidates)
                storage_limit = getattr(self.runtime, "maxStorageBufferBindingSize", None)
                if storage_limit is None:
                    storage_limit = math.inf
                bytes_per_request = candidate_sequence * 6144 * 2 * 2
                storage_cap = max(1, math.floor(storage_limit / bytes_per_request)) if storage_limit != math.inf else math.inf
                long_cap = 8 if candidate_sequence >= 1500 else self.max_batch_size
                take = int(min(self.max_batch_size, storage_cap, long_cap))
                requests, self._pending = self._pending[:take], self._pending[take:]
                sequence = max(len(r.tokens) for r in requests)
                ids = np.full(len(requests) * sequence, self.pad_token, dtype=np.uint32)
                lengths = np.zeros(len(requests), dtype=np.uint32)
                for i, r in enumerate(requests):
                    ids[i * sequence:i * sequence + len(r.tokens)] = r.tokens
                    lengths[i] = len(r.tokens)
                key = f"{len(requests)}:{sequence}"
                plan = self._plans.get(key)
                if plan is None:
                    plan = self.runtime.createPlan(len(requests), sequence)
                    self._plans[key] = plan
                try:
                    embeddings = await plan.run(ids, lengths)
                    for i, r in enumerate(requests):
                        if not r.future.done():
                            r.future.set_result(embeddings[i])
                except Exception as error:  # every request of the batch rejects (:87-88)
                    for r in requests:
                        if not r.future.done():
                            r.future.set_exception(error)
        finally:
            self._flushing = False
            if self._pending:
                self._schedule()
