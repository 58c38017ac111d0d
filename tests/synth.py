"""Seeded synthetic inputs for the tests (input generation, not a checker).

PRNG: splitmix64 (state += 0x9E3779B97F4A7C15, then the splitmix64 mix);
normals by Box-Muller on two 53-bit uniforms. Float-to-f16 conversions are
round-to-nearest-even (numpy).

Q4_K / Q6_K encoders for N(0, sigma) weights use the same simple quantizer as
the library's device synthesizer (per-sub-block min/step, 6-bit scales/mins
packed by the inverse of scaleAndMin; Q6_K per-16 amax with int8 scales).
Config-1 style random blocks draw d, dmin ~ f16(U(0.001, 0.02)), 6-bit scales
and mins uniform over 0..63 and nibbles uniform over 0..15.
"""
from __future__ import annotations

import numpy as np

GAMMA = np.uint64(0x9E3779B97F4A7C15)
M1 = np.uint64(0xBF58476D1CE4E5B9)
M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, n: int, offset: int = 0) -> np.ndarray:
    """Outputs offset..offset+n-1 of splitmix64 seeded with `seed`."""
    with np.errstate(over="ignore"):
        i = np.arange(offset + 1, offset + n + 1, dtype=np.uint64)
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + i * GAMMA
        z = (z ^ (z >> np.uint64(30))) * M1
        z = (z ^ (z >> np.uint64(27))) * M2
        return z ^ (z >> np.uint64(31))


def uniform(seed: int, n: int, offset: int = 0) -> np.ndarray:
    """U[0, 1) float64 from the top 53 bits."""
    return (splitmix64(seed, n, offset) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)


def normal(seed: int, n: int) -> np.ndarray:
    u = uniform(seed, 2 * n).reshape(n, 2)
    u1 = 1.0 - u[:, 0]
    return np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u[:, 1])


def randint(seed: int, n: int, lo: int, hi: int) -> np.ndarray:
    """Uniform integers in [lo, hi)."""
    return (splitmix64(seed, n) % np.uint64(hi - lo)).astype(np.int64) + lo


def f16_bits(values) -> np.ndarray:
    return np.asarray(values, dtype=np.float64).astype(np.float16).view(np.uint16)


# --------------------------------------------------------------------------
# Q4_K
# --------------------------------------------------------------------------

def pack_q4k_scales(sc: np.ndarray, m: np.ndarray) -> np.ndarray:
    """[nb, 8] 6-bit scales/mins -> [nb, 12] bytes (inverse of scaleAndMin,
    src/gguf/quantization.ts:11-17)."""
    sc = sc.astype(np.uint32)
    m = m.astype(np.uint32)
    out = np.zeros((sc.shape[0], 12), dtype=np.uint32)
    for j in range(4):
        out[:, j] = (sc[:, j] & 63) | ((sc[:, j + 4] >> 4) << 6)
        out[:, j + 4] = (m[:, j] & 63) | ((m[:, j + 4] >> 4) << 6)
        out[:, j + 8] = (sc[:, j + 4] & 15) | ((m[:, j + 4] & 15) << 4)
    return out.astype(np.uint8)


def q4k_blocks(d_bits, dmin_bits, sc, m, q) -> np.ndarray:
    """Assemble [nb, 144] Q4_K blocks from fields; q is [nb, 256] in 0..15."""
    nb = q.shape[0]
    out = np.zeros((nb, 144), dtype=np.uint8)
    out[:, 0:2] = np.asarray(d_bits, dtype=np.uint16).reshape(nb, 1).view(np.uint8).reshape(nb, 2)
    out[:, 2:4] = np.asarray(dmin_bits, dtype=np.uint16).reshape(nb, 1).view(np.uint8).reshape(nb, 2)
    out[:, 4:16] = pack_q4k_scales(sc, m)
    qq = q.reshape(nb, 4, 2, 32).astype(np.uint8)
    out[:, 16:] = (qq[:, :, 0, :] | (qq[:, :, 1, :] << 4)).reshape(nb, 128)
    return out


def random_q4k(seed: int, n_blocks: int) -> np.ndarray:
    """Config-1 blocks: d, dmin ~ f16(U(0.001, 0.02)), scales/mins U{0..63},
    nibbles U{0..15}."""
    u = uniform(seed, 2 * n_blocks).reshape(n_blocks, 2)
    d = f16_bits(0.001 + 0.019 * u[:, 0])
    dmin = f16_bits(0.001 + 0.019 * u[:, 1])
    sc = randint(seed + 1, n_blocks * 8, 0, 64).reshape(n_blocks, 8)
    m = randint(seed + 2, n_blocks * 8, 0, 64).reshape(n_blocks, 8)
    q = randint(seed + 3, n_blocks * 256, 0, 16).reshape(n_blocks, 256)
    return q4k_blocks(d, dmin, sc, m, q).reshape(-1)


def quantize_q4k(w: np.ndarray) -> np.ndarray:
    """float [rows, k] -> Q4_K bytes [rows * k / 256 * 144]."""
    x = np.asarray(w, dtype=np.float64).reshape(-1, 8, 32)
    nb = x.shape[0]
    offset = -np.minimum(0.0, x.min(axis=2))
    step = (x.max(axis=2) + offset) / 15.0
    d = np.asarray(step.max(axis=1) / 63.0).astype(np.float16)
    dmin = np.asarray(offset.max(axis=1) / 63.0).astype(np.float16)
    df, dmf = d.astype(np.float64)[:, None], dmin.astype(np.float64)[:, None]
    with np.errstate(divide="ignore", invalid="ignore"):
        sc = np.where(df > 0, np.clip(np.rint(step / df), 0, 63), 0)
        m = np.where(dmf > 0, np.clip(np.rint(offset / dmf), 0, 63), 0)
        s = (df * sc)[:, :, None]
        o = (dmf * m)[:, :, None]
        q = np.where(s > 0, np.clip(np.rint((x + o) / s), 0, 15), 0)
    return q4k_blocks(d.view(np.uint16), dmin.view(np.uint16), sc, m, q.reshape(nb, 256)).reshape(-1)


# --------------------------------------------------------------------------
# Q6_K
# --------------------------------------------------------------------------

def q6k_blocks(d_bits, scales, q) -> np.ndarray:
    """Assemble [nb, 210] Q6_K blocks; scales int8 [nb, 16]; q [nb, 256] in
    0..63 (value e = 128h + 32Q + l sits in ql[64h + l + 32 (Q & 1)], high
    nibble for Q >= 2, and qh[32h + l] bits 2Q..2Q+1)."""
    nb = q.shape[0]
    out = np.zeros((nb, 210), dtype=np.uint8)
    qq = q.reshape(nb, 2, 4, 32).astype(np.uint32)
    for h in range(2):
        out[:, 64 * h:64 * h + 32] = ((qq[:, h, 0] & 15) | ((qq[:, h, 2] & 15) << 4)).astype(np.uint8)
        out[:, 64 * h + 32:64 * h + 64] = ((qq[:, h, 1] & 15) | ((qq[:, h, 3] & 15) << 4)).astype(np.uint8)
        out[:, 128 + 32 * h:128 + 32 * h + 32] = ((qq[:, h, 0] >> 4) | ((qq[:, h, 1] >> 4) << 2)
                                                  | ((qq[:, h, 2] >> 4) << 4) | ((qq[:, h, 3] >> 4) << 6)).astype(np.uint8)
    out[:, 192:208] = np.asarray(scales, dtype=np.int8).view(np.uint8)
    out[:, 208:210] = np.asarray(d_bits, dtype=np.uint16).reshape(nb, 1).view(np.uint8).reshape(nb, 2)
    return out


def random_q6k(seed: int, n_blocks: int) -> np.ndarray:
    """d ~ f16(U(0.0005, 0.005)), int8 scales uniform over -128..127, q uniform 0..63."""
    d = f16_bits(0.0005 + 0.0045 * uniform(seed, n_blocks))
    scales = randint(seed + 1, n_blocks * 16, -128, 128).reshape(n_blocks, 16)
    q = randint(seed + 2, n_blocks * 256, 0, 64).reshape(n_blocks, 256)
    return q6k_blocks(d, scales, q).reshape(-1)


def quantize_q6k(w: np.ndarray) -> np.ndarray:
    x = np.asarray(w, dtype=np.float64).reshape(-1, 16, 16)
    nb = x.shape[0]
    step = np.abs(x).max(axis=2) / 31.0
    d = np.asarray(step.max(axis=1) / 127.0).astype(np.float16)
    df = d.astype(np.float64)[:, None]
    with np.errstate(divide="ignore", invalid="ignore"):
        sc = np.where(df > 0, np.clip(np.rint(step / df), 1, 127), 1)
        s = (df * sc)[:, :, None]
        q = np.where(s > 0, np.clip(np.rint(x / s) + 32, 0, 63), 32)
    return q6k_blocks(d.view(np.uint16), sc.astype(np.int8), q.reshape(nb, 256)).reshape(-1)


def random_q40(seed: int, n_blocks: int) -> np.ndarray:
    out = np.zeros((n_blocks, 18), dtype=np.uint8)
    out[:, 0:2] = f16_bits(0.001 + 0.02 * uniform(seed, n_blocks)).reshape(n_blocks, 1).view(np.uint8).reshape(n_blocks, 2)
    out[:, 2:] = randint(seed + 1, n_blocks * 16, 0, 256).reshape(n_blocks, 16).astype(np.uint8)
    return out.reshape(-1)


# --------------------------------------------------------------------------
# Small models
# --------------------------------------------------------------------------

def model_tensors(dims, seed: int, embedding_type: int = 1, sigma: float = 0.02, fused: bool = True) -> dict:
    """name -> (ggml_type, gguf dims, bytes) for a model of `dims`
    (attributes hidden, q_heads, kv_heads, head_dim, intermediate, layers,
    vocab). Matrices Q4_K except ffn_down (Q6_K); norms ~ 1 + N(0, 0.1)."""
    H, F = dims.hidden, dims.intermediate
    QW, KW = dims.q_heads * dims.head_dim, dims.kv_heads * dims.head_dim
    t = {}
    s = seed
    def mat(rows, k, q6=False):
        nonlocal s
        s += 101
        w = sigma * normal(s, rows * k).reshape(rows, k)
        return (14 if q6 else 12, [k, rows], (quantize_q6k(w) if q6 else quantize_q4k(w)).tobytes())
    def norm(n):
        nonlocal s
        s += 101
        return (0, [n], (1.0 + 0.1 * normal(s, n)).astype(np.float32).tobytes())
    for l in range(dims.layers):
        p = f"blk.{l}."
        if fused:
            t[p + "attn_qkv.weight"] = mat(QW + 2 * KW, H)
            t[p + "ffn_gate_up.weight"] = mat(2 * F, H)
        else:
            t[p + "attn_q.weight"] = mat(QW, H)
            t[p + "attn_k.weight"] = mat(KW, H)
            t[p + "attn_v.weight"] = mat(KW, H)
            t[p + "ffn_gate.weight"] = mat(F, H)
            t[p + "ffn_up.weight"] = mat(F, H)
        t[p + "attn_output.weight"] = mat(H, QW)
        t[p + "ffn_down.weight"] = mat(H, F, q6=True)
        t[p + "attn_norm.weight"] = norm(H)
        t[p + "ffn_norm.weight"] = norm(H)
    t["output_norm.weight"] = norm(H)
    s += 101
    emb = sigma * normal(s, dims.vocab * H).reshape(dims.vocab, H)
    if embedding_type == 1:
        t["token_embd.weight"] = (1, [H, dims.vocab], emb.astype(np.float16).tobytes())
    else:
        t["token_embd.weight"] = (14, [H, dims.vocab], quantize_q6k(emb).tobytes())
    return t


def oracle_model(dims, tensors: dict):
    """Dequantize `tensors` into an oracle.Model (fusing parts by rows)."""
    import oracle
    def deq(name):
        typ, dd, data = tensors[name]
        return oracle.dequantize(typ, np.frombuffer(data, np.uint8)).reshape(dd[1], dd[0])
    def cat(name, parts):
        return deq(name) if name in tensors else np.concatenate([deq(p) for p in parts], axis=0)
    od = oracle.Dims(hidden=dims.hidden, q_heads=dims.q_heads, kv_heads=dims.kv_heads, head_dim=dims.head_dim,
                     intermediate=dims.intermediate, layers=dims.layers, vocab=dims.vocab,
                     merge_after_layer=dims.merge_after_layer, rms_epsilon=float(np.float32(dims.rms_epsilon)),
                     rope_theta=float(np.float32(dims.rope_theta)), kv_stride_threshold=dims.kv_stride_threshold,
                     kv_stride=dims.kv_stride, kv_dense_before_merge=dims.kv_dense_before_merge)
    vec = lambda name: np.frombuffer(tensors[name][2], np.float32)
    et, _, eb = tensors["token_embd.weight"]
    m = oracle.Model(od, et, np.frombuffer(eb, np.uint8) if et == 14 else np.frombuffer(eb, np.float16),
                     [vec(f"blk.{l}.attn_norm.weight") for l in range(dims.layers)],
                     [vec(f"blk.{l}.ffn_norm.weight") for l in range(dims.layers)], vec("output_norm.weight"))
    for l in range(dims.layers):
        p = f"blk.{l}."
        m.qkv.append(cat(p + "attn_qkv.weight", [p + "attn_q.weight", p + "attn_k.weight", p + "attn_v.weight"]))
        m.attn_output.append(deq(p + "attn_output.weight"))
        m.gate_up.append(cat(p + "ffn_gate_up.weight", [p + "ffn_gate.weight", p + "ffn_up.weight"]))
        m.down.append(deq(p + "ffn_down.weight"))
    return m
