"""Offline tokenizer loading (nemo_amd/tokenizer.py): a tokenizer.json on disk
drives the engine as transformers.js's tokenizer drives the reference's
(src/webgpu/embedding-engine.ts:41, src/main.ts:163-167). The file here is a
small word-level tokenizer with a BOS post-processor, written by the
tokenizers library itself."""
import asyncio
import os

import numpy as np
import pytest

tokenizers = pytest.importorskip("tokenizers")

from nemo_amd.engine import NemotronEmbeddingEngine  # noqa: E402
from nemo_amd.tokenizer import load_tokenizer  # noqa: E402


def _write_tokenizer(directory):
    from tokenizers import Tokenizer, models, pre_tokenizers, processors
    vocab = {"<unk>": 0, "<s>": 1, "</s>": 2, "vector": 3, "search": 4, "maps": 5}
    tok = Tokenizer(models.WordLevel(vocab, unk_token="<unk>"))
    tok.pre_tokenizer = pre_tokenizers.Whitespace()
    tok.post_processor = processors.TemplateProcessing(single="<s> $A", special_tokens=[("<s>", 1)])
    path = os.path.join(directory, "tokenizer.json")
    tok.save(path)
    return path


def test_loads_file_or_directory_and_adds_bos(tmp_path):
    path = _write_tokenizer(str(tmp_path))
    for source in (path, str(tmp_path)):
        tok = load_tokenizer(source)
        assert tok("vector search maps").input_ids.tolist() == [[1, 3, 4, 5]]
        assert tok("vector unknownword").input_ids.tolist() == [[1, 3, 0]]
        # the comparison workloads' exact-length property (scripts/workloads.ts:28-29)
        assert tok.count(" ".join(["vector"] * 149)) == 150
    with pytest.raises(FileNotFoundError):
        load_tokenizer(str(tmp_path / "missing"))


def test_engine_runs_on_the_loaded_tokenizer(tmp_path):
    tok = load_tokenizer(_write_tokenizer(str(tmp_path)))
    seen = []

    class Plan:
        def __init__(self, batch, sequence):
            self.batch, self.sequence = batch, sequence

        async def run(self, ids, lengths):
            seen.append((ids.tolist(), lengths.tolist()))
            return [np.full(2, float(i)) for i in range(self.batch)]

    class Runtime:
        maxStorageBufferBindingSize = None

        def createPlan(self, batch, sequence):  # noqa: N802
            return Plan(batch, sequence)

    async def go():
        engine = NemotronEmbeddingEngine(Runtime(), tok)
        return await asyncio.gather(engine.embed("vector search"), engine.embed("maps"))

    out = asyncio.new_event_loop().run_until_complete(go())
    assert [o.tolist() for o in out] == [[0.0, 0.0], [1.0, 1.0]]
    # BOS from the tokenizer is not doubled; the shorter request is padded with 11
    assert seen == [([1, 3, 4, 1, 5, 11], [3, 2])]
