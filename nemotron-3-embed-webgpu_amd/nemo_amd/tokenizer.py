"""Offline tokenizer for the engine.

The reference loads the model's tokenizer with transformers.js
(``AutoTokenizer.from_pretrained('nvidia/Nemotron-3-Embed-1B-BF16')``,
src/main.ts:163-165) and calls it as ``tokenizer(text).input_ids.tolist()``
(src/webgpu/embedding-engine.ts:41). ``load_tokenizer`` reads the same
``tokenizer.json`` from a local file or directory with the ``tokenizers``
library (no network) and returns a callable with that contract, so
``NemotronEmbeddingEngine`` takes it unchanged. Special tokens are added as
the file's post-processor specifies (the Nemotron tokenizer prepends BOS; the
engine prepends it when a tokenizer does not).
"""
from __future__ import annotations

import os

import numpy as np


class _Encoded:
    """The slice of transformers.js's encoding the engine reads."""

    def __init__(self, ids):
        self.input_ids = np.asarray([ids], dtype=np.int64)


class LocalTokenizer:
    def __init__(self, path: str):
        try:
            from tokenizers import Tokenizer
        except ImportError as error:  # pragma: no cover - depends on the environment
            raise ImportError("load_tokenizer needs the 'tokenizers' package") from error
        file = os.path.join(path, "tokenizer.json") if os.path.isdir(path) else path
        if not os.path.exists(file):
            raise FileNotFoundError(f"no tokenizer.json at {path}")
        self._tokenizer = Tokenizer.from_file(file)

    def __call__(self, text: str) -> _Encoded:
        return _Encoded(self._tokenizer.encode(text).ids)

    def count(self, text: str) -> int:
        """Token count of `text` with special tokens (the exact-length check
        of the comparison workloads, src/main.ts:253-256)."""
        return len(self._tokenizer.encode(text).ids)


def load_tokenizer(path: str) -> LocalTokenizer:
    """tokenizer.json (or a directory holding it) -> engine TokenizerLike."""
    return LocalTokenizer(path)


__all__ = ["LocalTokenizer", "load_tokenizer"]
