"""Pins of the oracle's codec (oracle/nemo_oracle.c) against the reference's
own known-answer tests and against what the arithmetic fixes.

Each check is chosen so that a plausible mistake in the oracle (a wrong
nibble or scale index, a dropped dmin term, round-to-even instead of the
reference's ties-away f16 encoding) fails it; none retypes the oracle's
formula.
"""
from fractions import Fraction

import numpy as np
import pytest

import oracle
import synth


# --------------------------------------------------------------------------
# binary16 decode: src/gguf/quantization.ts:2-9
# --------------------------------------------------------------------------

def test_half_to_float_reference_kats():
    # tests/quantization.test.ts:5-9
    assert oracle.half_to_float(0x3C00) == 1
    assert oracle.half_to_float(0xC000) == -2
    assert oracle.half_to_float(0x0000) == 0


def test_half_to_float_every_pattern_matches_ieee():
    """All 65,536 patterns against numpy's IEEE binary16 (NaN as NaN)."""
    bits = np.arange(65536, dtype=np.uint32)
    got = np.array([oracle.half_to_float(int(b)) for b in bits])
    want = bits.astype(np.uint16).view(np.float16).astype(np.float64)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan], want[~nan])
    # signed zero survives (sign * 2^-14 * 0)
    assert np.signbit(oracle.half_to_float(0x8000))


# --------------------------------------------------------------------------
# binary16 encode: src/math/f16.ts:4-25 rounds to nearest, ties AWAY from zero
# --------------------------------------------------------------------------

_F16_MAX_FINITE = Fraction(65504)
_F16_OVERFLOW = Fraction(65520)  # midpoint of 65504 and 2^16: ties away -> inf


def _exact_ties_away(v: float) -> int:
    """binary16 bits of the float32 value v by exact rational arithmetic:
    nearest f16, ties away from zero, |v| >= 65520 -> inf."""
    sign = 0x8000 if np.signbit(np.float32(v)) else 0
    a = abs(Fraction(float(v)))
    if a >= _F16_OVERFLOW:
        return sign | 0x7C00
    # candidate magnitudes: the f16 values bracketing a
    lo_bits = int(np.float16(float(a)).view(np.uint16))
    lo = Fraction(float(np.uint16(lo_bits).view(np.float16)))
    if lo > a:
        lo_bits -= 1
        lo = Fraction(float(np.uint16(lo_bits).view(np.float16)))
    hi_bits = lo_bits + 1
    hi = Fraction(float(np.uint16(hi_bits).view(np.float16))) if hi_bits < 0x7C00 else Fraction(65536)
    if a == lo:
        return sign | lo_bits
    return sign | (hi_bits if a - lo >= hi - a else lo_bits)


def _midpoints() -> np.ndarray:
    """Every midpoint between adjacent finite f16 magnitudes (exact in
    float32), with its float32 neighbours on both sides."""
    mags = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float64)
    mids = ((mags[:-1] + mags[1:]) / 2).astype(np.float32)
    below = np.nextafter(mids, np.float32(0))
    above = np.nextafter(mids, np.float32(np.inf))
    return np.concatenate([mids, below, above])


def test_float_to_half_ties_away_on_every_midpoint():
    vals = _midpoints()
    vals = np.concatenate([vals, -vals])
    got = oracle.float_to_half(vals)
    want = np.array([_exact_ties_away(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, want)
    # exact midpoints differ from round-to-nearest-even exactly where the
    # lower neighbour is even: the rule is not RNE
    mids = _midpoints()[:0x7BFF]
    rne = mids.astype(np.float16).view(np.uint16)
    assert np.any(rne != oracle.float_to_half(mids))


def test_float_to_half_dense_sample_and_specials():
    rng = np.random.default_rng(7)
    v = (rng.standard_normal(20000) * np.exp2(rng.integers(-30, 18, 20000))).astype(np.float32)
    got = oracle.float_to_half(v)
    want = np.array([_exact_ties_away(float(x)) for x in v], dtype=np.uint16)
    assert np.array_equal(got, want)
    # off ties the rule agrees with numpy's round-to-nearest-even
    with np.errstate(over="ignore"):
        rne = v.astype(np.float16).view(np.uint16)
    mid = np.isin(v, _midpoints()[:0x7BFF]) | np.isin(-v, _midpoints()[:0x7BFF])
    assert np.array_equal(got[~mid], rne[~mid])
    specials = np.array([np.inf, -np.inf, np.nan, 65504, 65519.99, 65520, 2.0 ** -25, 2.0 ** -26, 0.0, -0.0],
                        dtype=np.float32)
    assert list(oracle.float_to_half(specials)) == [0x7C00, 0xFC00, 0x7C00, 0x7BFF, 0x7BFF, 0x7C00, 0x0001,
                                                   0x0000, 0x0000, 0x8000]


# --------------------------------------------------------------------------
# Q4_K: src/gguf/quantization.ts:11-38
# --------------------------------------------------------------------------

def test_q4k_reference_kat():
    # tests/quantization.test.ts:11-22
    block = np.zeros(144, dtype=np.uint8)
    block[0:2] = [0x00, 0x3C]
    block[4:12] = 1
    block[12:16] = 0x11
    block[16:] = 0x72
    v = oracle.dequantize(12, block)
    assert v[0] == 2 and v[31] == 2 and v[32] == 7 and v[255] == 7
    # the same KAT, every value: low nibble 2 in the first 32 of each 64,
    # high nibble 7 in the second 32 (all scales 1, no minimum)
    assert np.array_equal(v, np.tile(np.repeat([2.0, 7.0], 32), 4).astype(np.float32))


def test_q4k_scale_min_brute_force():
    """Every (scale, min) pair 0..63 x 0..63 in every one of the 8 slots,
    packed by the GGML encoder layout (synth.pack_q4k_scales), decodes back
    through the oracle's scaleAndMin."""
    vals = np.arange(64)
    sc_all, m_all = np.meshgrid(vals, vals, indexing="ij")
    sc_all, m_all = sc_all.reshape(-1), m_all.reshape(-1)
    rng = np.random.default_rng(3)
    for slot in range(8):
        sc = rng.integers(0, 64, (4096, 8))
        m = rng.integers(0, 64, (4096, 8))
        sc[:, slot], m[:, slot] = sc_all, m_all
        packed = synth.pack_q4k_scales(sc, m)
        for i in range(0, 4096, 37):  # a spread of rows (the ctypes call is per row)
            assert oracle.q4k_scale_min(packed[i].tobytes(), slot) == (sc_all[i], m_all[i])
        # every row through the block decoder: d = 1, dmin = 1, q = 1 in
        # sub-block `slot` only -> value = scale - min there
        nb = 4096
        q = np.zeros((nb, 256), dtype=np.int64)
        q[:, 32 * slot:32 * slot + 32] = 1
        blocks = synth.q4k_blocks(np.full(nb, 0x3C00), np.full(nb, 0x3C00), sc, m, q)
        out = oracle.dequantize(12, blocks).reshape(nb, 8, 32)
        assert np.array_equal(out[:, slot, 0], (sc_all - m_all).astype(np.float32))
        others = [j for j in range(8) if j != slot]
        assert np.array_equal(out[:, others, 0], -m[:, others].astype(np.float32))


def _wgsl_q4k(block: np.ndarray) -> np.ndarray:
    """The per-element Q4_K decoder of src/webgpu/quant-matmul.ts:38-60
    (byte offsets, scale index, nibble select), evaluated in float64 and
    stored to float32 as the reference's JavaScript does."""
    b = block.astype(np.int64)
    d = float(np.uint16(b[0] | (b[1] << 8)).view(np.float16))
    dmin = float(np.uint16(b[2] | (b[3] << 8)).view(np.float16))
    out = np.empty(256, dtype=np.float32)
    for column in range(256):
        group, in_group = column // 64, column & 63
        si = group * 2 + (1 if in_group >= 32 else 0)
        if si < 4:
            scale, minimum = b[4 + si] & 63, b[4 + si + 4] & 63
        else:
            scale = (b[4 + si + 4] & 15) | ((b[4 + si - 4] >> 6) << 4)
            minimum = (b[4 + si + 4] >> 4) | ((b[4 + si] >> 6) << 4)
        packed = b[16 + group * 32 + (in_group & 31)]
        quant = (packed >> 4) if in_group >= 32 else (packed & 15)
        out[column] = np.float32(d * scale * quant - dmin * minimum)
    return out


def test_q4k_matches_wgsl_decoder_on_random_blocks():
    raw = synth.random_q4k(11, 24).reshape(24, 144)
    got = oracle.dequantize(12, raw).reshape(24, 256)
    for i in range(24):
        assert np.array_equal(got[i], _wgsl_q4k(raw[i])), f"block {i}"


def test_q4k_subnormal_scales_exact():
    """d and dmin subnormal or at the f16 extremes: the fp32 result equals the
    exact rational value rounded once (the JS double expression)."""
    d = np.array([0x0001, 0x03FF, 0x7BFF, 0x3C00])
    dmin = np.array([0x03FF, 0x0001, 0x3C00, 0x7BFF])
    sc = np.full((4, 8), 63)
    m = np.full((4, 8), 63)
    q = synth.randint(5, 4 * 256, 0, 16).reshape(4, 256)
    raw = synth.q4k_blocks(d, dmin, sc, m, q)
    got = oracle.dequantize(12, raw).reshape(4, 256)
    for i in range(4):
        df = Fraction(float(np.uint16(d[i]).view(np.float16)))
        dmf = Fraction(float(np.uint16(dmin[i]).view(np.float16)))
        for c in range(0, 256, 7):
            exact = df * 63 * int(q[i, c]) - dmf * 63
            assert got[i, c] == np.float32(float(exact)), (i, c)


# --------------------------------------------------------------------------
# Q6_K: src/gguf/quantization.ts:46-74
# --------------------------------------------------------------------------

def test_q6k_reference_kat():
    # tests/quantization.test.ts:35-42
    block = np.zeros(210, dtype=np.uint8)
    block[192:208] = 1
    block[208:210] = [0x00, 0x3C]
    assert np.all(oracle.dequantize(14, block) == -32)


def _wgsl_q6k(block: np.ndarray) -> np.ndarray:
    """The per-element Q6_K decoder of src/webgpu/quant-matmul.ts:111-127."""
    b = block.astype(np.int64)
    d = float(np.uint16(b[208] | (b[209] << 8)).view(np.float16))
    out = np.empty(256, dtype=np.float32)
    for column in range(256):
        half, position = column // 128, column & 127
        quadrant, lane = position // 32, position & 31
        low_byte = b[half * 64 + lane + (quadrant & 1) * 32]
        low = (low_byte >> 4) if quadrant >= 2 else (low_byte & 15)
        high = (b[128 + half * 32 + lane] >> (quadrant * 2)) & 3
        quant = (low | (high << 4)) - 32
        sb = b[192 + half * 8 + lane // 16 + quadrant * 2]
        scale = sb - 256 if sb >= 128 else sb
        out[column] = np.float32(d * scale * quant)
    return out


def test_q6k_matches_wgsl_decoder_on_random_blocks():
    raw = synth.random_q6k(12, 24).reshape(24, 210)
    got = oracle.dequantize(14, raw).reshape(24, 256)
    for i in range(24):
        assert np.array_equal(got[i], _wgsl_q6k(raw[i])), f"block {i}"


def test_q6k_scatter_encoder_round_trip():
    """Blocks built from known (d, int8 scales, 6-bit q) by the GGML scatter
    layout decode to d * scale[e / 16] * (q[e] - 32) for every value e."""
    nb = 16
    d_bits = synth.f16_bits(0.001 + 0.01 * synth.uniform(21, nb))
    scales = synth.randint(22, nb * 16, -128, 128).reshape(nb, 16)
    q = synth.randint(23, nb * 256, 0, 64).reshape(nb, 256)
    got = oracle.dequantize(14, synth.q6k_blocks(d_bits, scales, q)).reshape(nb, 256)
    d = d_bits.view(np.float16).astype(np.float64)[:, None]
    want = (d * np.repeat(scales, 16, axis=1) * (q - 32)).astype(np.float32)
    assert np.array_equal(got, want)


# --------------------------------------------------------------------------
# Q4_0: src/gguf/quantization.ts:40-44, 77-131
# --------------------------------------------------------------------------

def test_q40_reference_kat():
    # tests/quantization.test.ts:24-33
    block = np.zeros(18, dtype=np.uint8)
    block[0:2] = [0x00, 0x3C]
    block[2:] = 0xF0
    v = oracle.dequantize(2, block)
    assert np.all(v[:16] == -8) and np.all(v[16:] == 7)


def test_q40_round_trip_reference_bound():
    # tests/quantization.test.ts:44-49
    values = (np.arange(32, dtype=np.float32) - 16) / 4
    decoded = oracle.dequantize(2, oracle.quantize_q40_block(values))
    assert np.max(np.abs(decoded - values)) < 0.55


def test_q40_quantizer_closed_form():
    """Scale = signed max / -8 stored by the ties-away f16 encoder; the
    signed-max element maps to quant 0 (-8 * scale reproduces it)."""
    rng = np.random.default_rng(5)
    for _ in range(50):
        v = rng.standard_normal(32).astype(np.float32)
        enc = np.frombuffer(oracle.quantize_q40_block(v), dtype=np.uint8)
        i = int(np.argmax(np.abs(v)))
        scale_bits = int(enc[0]) | (int(enc[1]) << 8)
        assert scale_bits == int(oracle.float_to_half(np.float32(v[i] / np.float32(-8)))[0])
        nib = (enc[2 + (i % 16)] >> (4 * (i // 16))) & 15
        assert nib == 0
    assert oracle.quantize_q40_block(np.zeros(32, np.float32)) == bytes([0, 0] + [0x88] * 16)


def test_requantize_q6k_reference_kat():
    # tests/quantization.test.ts:51-59
    source = np.zeros(210, dtype=np.uint8)
    source[192:208] = 1
    source[208:210] = [0x00, 0x3C]
    converted = oracle.requantize_to_q40(source.tobytes(), 14, 256, 1)
    assert len(converted) == 8 * 18
    assert np.all(oracle.dequantize(2, converted) == -32)


def test_requantize_q4k_matches_blockwise_quantizer():
    raw = synth.random_q4k(31, 4)
    out = oracle.requantize_to_q40(raw.tobytes(), 12, 512, 2)
    dec = oracle.dequantize(12, raw)
    want = b"".join(oracle.quantize_q40_block(dec[i:i + 32]) for i in range(0, dec.size, 32))
    assert out == want
    with pytest.raises(ValueError, match="not divisible"):
        oracle.requantize_to_q40(raw.tobytes(), 12, 300, 2)
    with pytest.raises(ValueError, match="expected"):
        oracle.requantize_to_q40(raw.tobytes()[:-1], 12, 512, 2)


# --------------------------------------------------------------------------
# tile32-compact packing: src/prepacked/format.ts:65-99
# --------------------------------------------------------------------------

def _q40_block(scale_bits, quants):
    b = bytearray(18)
    b[0:2] = bytes(scale_bits)
    for i in range(16):
        b[2 + i] = quants[i] | (quants[i + 16] << 4)
    return bytes(b)


def test_pack_tile32_reference_kat():
    # tests/prepacked-format.test.ts:13-27
    first = _q40_block([0x00, 0x3C], [i & 15 for i in range(32)])
    second = _q40_block([0x00, 0x40], [15 - (i & 15) for i in range(32)])
    packed = oracle.pack_q40_tile32(first + second, 32, 2)
    assert len(packed) == 32 * 20
    assert list(packed[0:8]) == [0x00, 0x3C, 0x00, 0x00, 0x00, 0x11, 0x22, 0x33]
    assert list(packed[20:28]) == [0x00, 0x40, 0x00, 0x00, 0xFF, 0xEE, 0xDD, 0xCC]
    assert packed[40:] == bytes(len(packed) - 40)


def test_pack_tile32_layout_tile_kblock_row():
    """Record of (row r, k-block kb) sits at ((r/32 * kBlocks + kb) * 32 + r%32) * 20."""
    n, k = 40, 96
    raw = synth.random_q40(41, n * k // 32).reshape(n, k // 32, 18)
    packed = np.frombuffer(oracle.pack_q40_tile32(raw.tobytes(), k, n), dtype=np.uint8)
    kb_count = k // 32
    assert packed.size == 2 * kb_count * 32 * 20
    for r in range(n):
        for kb in range(kb_count):
            rec = packed[((r // 32 * kb_count + kb) * 32 + r % 32) * 20:][:20]
            assert bytes(rec[0:2]) == raw[r, kb, 0:2].tobytes()
            assert bytes(rec[2:4]) == b"\0\0"
            assert bytes(rec[4:20]) == raw[r, kb, 2:18].tobytes()


# --------------------------------------------------------------------------
# contextualMergedLength: src/webgpu/model.ts:30-32
# --------------------------------------------------------------------------

@pytest.mark.parametrize("source,expected", [(1, 1), (15, 10), (50, 32), (150, 96), (500, 320), (1500, 960),
                                             (5000, 3200)])
def test_contextual_merged_length_reference_kat(source, expected):
    # tests/model-config.test.ts:5-15
    assert oracle.contextual_merged_length(source) == expected


def test_q4k_cpu_matmul_is_the_dequantized_dot():
    """The timed CPU baseline computes the reference's check (src/main.ts:97-104)
    for every element: integer-valued X and W make float64 exact."""
    n, k, m = 8, 512, 3
    d = np.full(n * 2, 0x3C00)  # d = dmin = 1
    sc = synth.randint(51, n * 2 * 8, 0, 4).reshape(n * 2, 8)
    mn = synth.randint(52, n * 2 * 8, 0, 4).reshape(n * 2, 8)
    q = synth.randint(53, n * 2 * 256, 0, 16).reshape(n * 2, 256)
    raw = synth.q4k_blocks(d, d, sc, mn, q).reshape(-1)
    x = synth.randint(54, m * k, -3, 4).astype(np.float32).reshape(m, k)
    got = oracle.q4k_matmul_cpu(raw, x, m, n, k)
    w = oracle.dequantize(12, raw).reshape(n, k).astype(np.int64)
    assert np.array_equal(got, (x.astype(np.int64) @ w.T).astype(np.float64))
