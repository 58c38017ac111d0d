"""The self-contained model pack (src/prepacked/format.ts): the reference's
format test (tests/prepacked-format.test.ts:13-33) re-expressed, the parser's
error messages, and agreement of the host packer with the oracle's."""
import json
import struct

import numpy as np
import pytest

import oracle
import synth
from nemo_amd import prepacked as pp


def _q40_block(scale_bits, quants):
    b = bytearray(18)
    b[0:2] = bytes(scale_bits)
    for i in range(16):
        b[2 + i] = quants[i] | (quants[i + 16] << 4)
    return bytes(b)


def test_reference_pack_round_trip():
    first = _q40_block([0x00, 0x3C], [i & 15 for i in range(32)])
    second = _q40_block([0x00, 0x40], [15 - (i & 15) for i in range(32)])
    packed = pp.pack_q40_tile32("fused", [{"name": "first", "k": 32, "n": 1, "bytes": first},
                                          {"name": "second", "k": 32, "n": 1, "bytes": second}])
    assert packed.dimensions == [32, 2]
    assert len(packed.bytes) == 32 * 20
    assert list(packed.bytes[0:8]) == [0x00, 0x3C, 0x00, 0x00, 0x00, 0x11, 0x22, 0x33]
    assert list(packed.bytes[20:28]) == [0x00, 0x40, 0x00, 0x00, 0xFF, 0xEE, 0xDD, 0xCC]
    raw = pp.raw_tensor("norm", [1], 0, bytes([1, 2, 3, 4]))
    data = pp.build_prepacked_file("abc123", 42, {"general.name": "test"}, [raw, packed])
    parsed = pp.parse_prepacked_model(data)
    assert parsed.header["sourceSha256"] == "abc123"
    assert parsed.header["sourceBytes"] == 42
    assert parsed.header["metadata"]["general.name"] == "test"
    norm = parsed.tensors["norm"]
    assert (norm["dimensions"], norm["type"], norm["storage"], norm["byteLength"]) == ([1], 0, "raw", 4)
    fused = parsed.tensors["fused"]
    assert (fused["dimensions"], fused["type"], fused["storage"], fused["byteLength"]) == (
        [32, 2], 2, "q4_0-tile32-compact", 640)
    # payloads at 256-byte aligned offsets from a 256-byte aligned data start
    assert parsed.dataOffset % 256 == 0 and all(t["byteOffset"] % 256 == 0 for t in parsed.tensors.values())
    assert data[fused["byteOffset"]:fused["byteOffset"] + 640] == packed.bytes
    assert data[:8] == b"WGPACK02"


def test_host_packer_matches_oracle_packer():
    n, k = 70, 128
    raw = synth.random_q40(8, n * k // 32).tobytes()
    host = pp.pack_q40_tile32("m", [{"name": "a", "k": k, "n": 30, "bytes": raw[:30 * 4 * 18]},
                                    {"name": "b", "k": k, "n": 40, "bytes": raw[30 * 4 * 18:]}])
    assert host.bytes == oracle.pack_q40_tile32(raw, k, n)


def _file(header_patch=None, tensors=None, truncate=0, magic=b"WGPACK02"):
    data = bytearray(pp.build_prepacked_file("s", 1, {}, tensors or [pp.raw_tensor("t", [4], 0, bytes(16))]))
    data[0:8] = magic
    if header_patch is not None:
        (n,) = struct.unpack_from("<I", data, 8)
        header = json.loads(bytes(data[12:12 + n]))
        header_patch(header)
        hb = json.dumps(header, separators=(",", ":")).encode()
        off = (12 + len(hb) + 255) // 256 * 256
        old_off = (12 + n + 255) // 256 * 256
        data = bytearray(data[:8]) + struct.pack("<I", len(hb)) + hb + bytes(off - 12 - len(hb)) + data[old_off:]
    return bytes(data[:len(data) - truncate])


@pytest.mark.parametrize("make,message", [
    (lambda: b"WGPACK0", "shorter than its prelude"),
    (lambda: _file(magic=b"WGPACK01"), 'invalid prepacked model magic "WGPACK01"'),
    (lambda: b"WGPACK02" + struct.pack("<I", 1000) + b"{}", "header extends past end of file"),
    (lambda: _file(lambda h: h.update(layout="other")), "unsupported prepacked layout other"),
    (lambda: _file(truncate=1), "t extends past end of prepacked file"),
    (lambda: _file(lambda h: h["tensors"].append(dict(h["tensors"][0]))), "duplicate prepacked tensor t"),
    (lambda: _file(lambda h: h["tensors"][0].update(storage="q4_0-tile32-compact")),
     "t has invalid compact Q4_0 metadata"),
    (lambda: _file(lambda h: h["tensors"][0].update(storage="zip")), "t has unsupported storage zip"),
])
def test_parser_errors_match_reference(make, message):
    # src/prepacked/format.ts:147-165
    with pytest.raises(ValueError, match=message.replace("(", r"\(")):
        pp.parse_prepacked_model(make())
