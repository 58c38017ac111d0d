"""The committed golden fixtures (tests/golden/*.json, written by
tests/golden/make_golden.py) against the oracle: the oracle still reproduces
every vector bit for bit, and the fixtures hold the reference's own
known-answer data."""
import json
import os

import numpy as np
import pytest

import oracle
import synth

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


@pytest.mark.parametrize("name", ["q4_k", "q6_k", "q4_0"])
def test_codec_vectors_reproduce(name):
    v = _load("codec_vectors.json")[name]
    raw = np.frombuffer(bytes.fromhex(v["blocks"]), dtype=np.uint8)
    assert np.array_equal(oracle.dequantize(v["type"], raw).view(np.uint32), np.array(v["f32_bits"], np.uint32))


def test_f16_vectors_reproduce():
    v = _load("codec_vectors.json")["f32_to_f16"]
    f = np.array(v["f32_bits"], np.uint32).view(np.float32)
    assert np.array_equal(oracle.float_to_half(f), np.array(v["f16_bits"], np.uint16))


def test_reference_kats_in_fixture():
    k = _load("codec_vectors.json")["reference_kats"]
    for bits, value in k["half_to_float"]:
        assert oracle.half_to_float(bits) == value
    for s, t in k["contextual_merged_length"]:
        assert oracle.contextual_merged_length(s) == t


def test_tiny_forward_reproduces():
    g = _load("tiny_forward.json")
    dims = oracle.Dims(**g["dims"])
    model = synth.oracle_model(dims, synth.model_tensors(dims, seed=g["seed"]))
    for req, bits in zip(g["requests"], g["embeddings_f32_bits"]):
        e = oracle.forward_request(model, np.array(req))
        assert np.array_equal(e.view(np.uint32), np.array(bits, np.uint32))
