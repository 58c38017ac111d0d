"""Pins of the oracle's float forward pass (oracle/oracle.py) by closed forms,
invariants and brute force. The reference holds no test of these kernels
(src/webgpu/ops.ts, src/webgpu/model.ts), so each is pinned by what the
mathematics fixes, chosen so that a plausible mistake (a transposed operand,
a wrong head mapping, a missing scale, an off-by-one bin) fails.
"""
import math

import numpy as np
import pytest

import oracle
import synth


def _f16(a):
    return np.asarray(a, dtype=np.float64).astype(np.float16)


# --------------------------------------------------------------------------
# RoPE / YaRN: src/webgpu/model.ts:95-106, src/webgpu/ops.ts:168-193
# --------------------------------------------------------------------------

def test_yarn_correction_dims_reference_head_dim():
    # the reference's literal constants at head_dim 128, theta 1e6: ramp
    # over pair dimensions 20..37
    assert oracle.yarn_correction_range(128, 1e6) == (20, 37)


def test_rope_table_frequency_ends_and_unit_norm():
    t = oracle.rope_table(64, 128, 1e6).astype(np.float64)
    assert np.allclose(np.hypot(t[..., 0], t[..., 1]), 1.0, atol=1e-6)
    assert np.all(t[0, :, 0] == 1) and np.all(t[0, :, 1] == 0)
    # position 1: angle = theta^(-i/64) * f_i, f = 1 below the ramp, 1/16 above
    ang = np.arctan2(t[1, :, 1], t[1, :, 0])
    base = np.array([1e6 ** (-i / 64) for i in range(64)])
    assert np.allclose(ang[:21], base[:21], rtol=1e-6)
    assert np.allclose(ang[37:], base[37:] / 16, rtol=1e-5)
    # inside the ramp the factor lies strictly between
    f = ang[21:37] / base[21:37]
    assert np.all((f < 1) & (f > 1 / 16)) and np.all(np.diff(f) < 0)


def test_rope_identity_norms_and_composition():
    d = oracle.Dims(hidden=128, q_heads=2, kv_heads=1, head_dim=64)
    n = 5
    qkv = _f16(synth.normal(3, n * d.qkv_width).reshape(n, d.qkv_width))
    table = oracle.rope_table(16, d.head_dim, d.rope_theta)
    q, k = oracle.rope(qkv, np.zeros(n, dtype=np.int64), table, d)
    assert np.array_equal(q.reshape(n, -1), qkv[:, :128]) and np.array_equal(k.reshape(n, -1), qkv[:, 128:192])
    q7, _ = oracle.rope(qkv, np.full(n, 7), table, d)
    pairs_in = qkv[:, :128].astype(np.float64).reshape(n, 2, 32, 2)
    pairs_out = q7.astype(np.float64).reshape(n, 2, 32, 2)
    assert np.allclose(np.hypot(*np.moveaxis(pairs_out, -1, 0)), np.hypot(*np.moveaxis(pairs_in, -1, 0)),
                       rtol=2e-3, atol=2e-3)
    # adjacent pairs (2i, 2i+1) rotate by position's angle: rotating by 3
    # then 4 equals rotating by 7 (angle addition on the unrounded values)
    c = table.astype(np.float64)
    e, o = pairs_in[..., 0], pairs_in[..., 1]
    def rot(e, o, p):
        cs, sn = c[p, :, 0], c[p, :, 1]
        return e * cs - o * sn, e * sn + o * cs
    e3, o3 = rot(e, o, 3)
    e7, o7 = rot(e3, o3, 4)
    assert np.allclose(e7, pairs_out[..., 0], atol=4e-3) and np.allclose(o7, pairs_out[..., 1], atol=4e-3)


# --------------------------------------------------------------------------
# attention: src/webgpu/ops.ts:213-362
# --------------------------------------------------------------------------

def _qkv(n, d, seed):
    q = _f16(synth.normal(seed, n * d.q_heads * d.head_dim).reshape(n, d.q_heads, d.head_dim))
    k = _f16(synth.normal(seed + 1, n * d.kv_heads * d.head_dim).reshape(n, d.kv_heads, d.head_dim))
    v = _f16(synth.normal(seed + 2, n * d.kv_heads * d.head_dim).reshape(n, d.kv_heads, d.head_dim))
    return q, k, v


D_ATT = oracle.Dims(hidden=256, q_heads=4, kv_heads=2, head_dim=64)


def test_attention_single_key_returns_value():
    q, k, v = _qkv(1, D_ATT, 10)
    out = oracle.attention(q, k, v, D_ATT)
    for h in range(4):
        assert np.array_equal(out[0, h], v[0, h // 2])


def test_attention_equal_keys_average_values_per_group():
    n = 9
    q, k, v = _qkv(n, D_ATT, 20)
    k[:] = k[0]
    out = oracle.attention(q, k, v, D_ATT).astype(np.float64)
    for h in range(4):
        assert np.allclose(out[:, h], v[:, h // 2].astype(np.float64).mean(axis=0), atol=1e-3)


def test_attention_dominant_key_selects_its_value():
    n = 6
    q, k, v = _qkv(n, D_ATT, 30)
    q[:] = 0
    q[:, :, 0] = 60.0
    k[:] = 0
    k[4, :, 0] = 60.0  # score 3600 / 8 = 450 above every other key
    out = oracle.attention(q, k, v, D_ATT)
    for h in range(4):
        assert np.array_equal(out[:, h], np.broadcast_to(v[4, h // 2], (n, 64)))


def test_attention_brute_force_and_permutation():
    n = 13
    q, k, v = _qkv(n, D_ATT, 40)
    out = oracle.attention(q, k, v, D_ATT).astype(np.float64)
    for h in range(4):
        g = h // 2
        s = np.einsum("id,jd->ij", q[:, h].astype(np.float64), k[:, g].astype(np.float64)) / 8.0
        p = np.exp(s - s.max(axis=1, keepdims=True))
        want = (p / p.sum(axis=1, keepdims=True)) @ v[:, g].astype(np.float64)
        assert np.allclose(out[:, h], want, atol=2e-3, rtol=2e-3)
    perm = np.random.default_rng(1).permutation(n)
    out_p = oracle.attention(q, k[perm], v[perm], D_ATT).astype(np.float64)
    assert np.allclose(out_p, out, atol=2e-3)


def test_attention_stride_three_equals_dense_over_sampled_keys():
    n = 31
    q, k, v = _qkv(n, D_ATT, 50)
    strided = oracle.attention(q, k, v, D_ATT, stride_threshold=20)
    keys = np.arange(0, n, 3)
    # dense attention of every query over only keys 0, 3, 6, ...
    for h in range(4):
        g = h // 2
        s = q[:, h].astype(np.float64) @ k[keys, g].astype(np.float64).T / 8.0
        p = np.exp(s - s.max(axis=1, keepdims=True))
        want = (p / p.sum(axis=1, keepdims=True)) @ v[keys, g].astype(np.float64)
        assert np.allclose(strided[:, h].astype(np.float64), want, atol=2e-3)
    # at or below the threshold every key is used
    assert np.array_equal(oracle.attention(q, k, v, D_ATT, stride_threshold=31),
                          oracle.attention(q, k, v, D_ATT))


# --------------------------------------------------------------------------
# RMSNorm: src/webgpu/ops.ts:21-56
# --------------------------------------------------------------------------

def test_rms_norm_constant_row_and_residual():
    w = np.linspace(0.5, 1.5, 64).astype(np.float32)
    x = _f16(np.full((2, 64), 0.75))
    x_new, norm = oracle.rms_norm(x, w, 1e-5)
    assert np.array_equal(x_new, x)
    # constant c: mean(v^2) = c^2, normalized = c / sqrt(c^2 + eps) * w
    want = _f16(0.75 / math.sqrt(0.75 ** 2 + 1e-5) * w.astype(np.float64))
    assert np.array_equal(norm[0], want) and np.array_equal(norm[1], want)
    # residual: x + delta is stored f16; the sum of squares uses the
    # unrounded sum (delta chosen so x + delta is not an f16 value)
    delta = _f16(np.full((1, 64), 2.0 ** -12))
    xr, nr = oracle.rms_norm(x[:1], w, 1e-5, delta)
    v = 0.75 + 2.0 ** -12
    assert np.array_equal(xr, _f16(np.full((1, 64), v)))
    assert np.array_equal(nr[0], _f16(xr[0].astype(np.float64) / math.sqrt(v * v + 1e-5) * w))


def test_rms_norm_scale_invariance():
    x = _f16(synth.normal(60, 4 * 256).reshape(4, 256))
    w = np.ones(256, np.float32)
    _, a = oracle.rms_norm(x, w, 0.0)
    _, b = oracle.rms_norm(_f16(x.astype(np.float64) * 4), w, 0.0)  # exact power-of-two scale
    assert np.array_equal(a, b)
    assert np.allclose(np.sqrt((a.astype(np.float64) ** 2).mean(axis=1)), 1.0, atol=2e-3)


# --------------------------------------------------------------------------
# SwiGLU: src/webgpu/ops.ts:74-88
# --------------------------------------------------------------------------

def test_swiglu_closed_forms():
    F = 4
    ln3 = math.log(3)
    g = np.array([[0.0, ln3, 30.0, -30.0]])
    u = np.array([[5.0, 2.0, 1.5, 7.0]])
    out = oracle.swiglu(_f16(np.concatenate([g, u], axis=1)), F).astype(np.float64)
    g16 = _f16(g).astype(np.float64)
    assert out[0, 0] == 0
    assert out[0, 1] == _f16(g16[0, 1] * 0.75 * 2.0)  # silu(ln 3) = ln 3 * 3/4 ... of the f16 input
    assert out[0, 2] == _f16(30.0 * 1.5)
    assert abs(out[0, 3]) < 1e-9
    # gate columns are the first F, up the second F
    swapped = oracle.swiglu(_f16(np.concatenate([u, g], axis=1)), F)
    assert not np.array_equal(swapped, out.astype(np.float16))


# --------------------------------------------------------------------------
# token merge: src/webgpu/ops.ts:629-660, src/webgpu/model.ts:226-233
# --------------------------------------------------------------------------

@pytest.mark.parametrize("S", [1, 2, 3, 15, 50, 150, 151])
def test_merge_bins_partition_and_bos(S):
    T = oracle.contextual_merged_length(S)
    bins = oracle.merge_bins(S, T)
    assert bins[0] == (0, 1)
    covered = []
    for a, b in bins[1:]:
        assert 1 <= a < b <= S
        covered.extend(range(a, b))
    if S > 1:
        # T - 1 bins over positions 1..S-1: every position in exactly one bin
        # when T <= S (bins never overlap, never skip)
        assert covered == list(range(1, S))


def test_merge_constant_rows_and_values():
    S = 50
    T = oracle.contextual_merged_length(S)
    x = _f16(np.tile(synth.normal(70, 32), (S, 1)))
    x[0] = 9.0  # BOS row differs
    out = oracle.merge(x, S, T)
    assert np.array_equal(out[0], x[0])
    assert np.array_equal(out[1:], np.broadcast_to(x[1], (T - 1, 32)))
    ramp = _f16(np.arange(S, dtype=np.float64)[:, None] * np.ones((1, 4)))
    out = oracle.merge(ramp, S, T).astype(np.float64)[:, 0]
    for p, (a, b) in enumerate(oracle.merge_bins(S, T)):
        assert out[p] == _f16((a + b - 1) / 2)


# --------------------------------------------------------------------------
# mean pool + L2: src/webgpu/ops.ts:596-615
# --------------------------------------------------------------------------

def test_mean_pool_unit_norm_and_direction():
    row = synth.normal(80, 64)
    x = _f16(np.tile(row, (7, 1)))
    e = oracle.mean_pool(x, 7).astype(np.float64)
    r = x[0].astype(np.float64)
    assert np.allclose(e, r / np.linalg.norm(r), atol=1e-7)
    y = _f16(synth.normal(81, 9 * 64).reshape(9, 64))
    e2 = oracle.mean_pool(y, 5).astype(np.float64)
    assert abs(np.linalg.norm(e2) - 1) < 1e-6
    # rows at or past the length do not contribute
    y2 = y.copy()
    y2[5:] = 100
    assert np.array_equal(oracle.mean_pool(y2, 5), oracle.mean_pool(y, 5))


# --------------------------------------------------------------------------
# matmul (src/main.ts:97-109): integer-valued operands make float64 exact
# --------------------------------------------------------------------------

def test_matmul_orientation_exact():
    x = synth.randint(90, 3 * 8, -4, 5).reshape(3, 8).astype(np.float16)
    w = synth.randint(91, 5 * 8, -4, 5).reshape(5, 8).astype(np.float32)
    y = oracle.matmul(x, w)
    assert y.shape == (3, 5)
    assert np.array_equal(y.astype(np.int64), x.astype(np.int64) @ w.astype(np.int64).T)


# --------------------------------------------------------------------------
# forward: src/webgpu/model.ts:146-176
# --------------------------------------------------------------------------

def _tiny_model(seed=5, layers=2, merge_after=1):
    dims = oracle.Dims(hidden=256, q_heads=4, kv_heads=2, head_dim=64, intermediate=256, layers=layers, vocab=40,
                       merge_after_layer=merge_after)
    return synth.oracle_model(dims, synth.model_tensors(dims, seed=seed))


def test_forward_batch_composition_and_padding():
    m = _tiny_model()
    seqs = [[1, 5, 9, 3], [1, 7], [1, 2, 3, 4, 5, 6]]
    S = 6
    ids = np.full(3 * S, 11, dtype=np.int64)
    for i, s in enumerate(seqs):
        ids[i * S:i * S + len(s)] = s
    batch = oracle.forward(m, ids, [len(s) for s in seqs])
    for i, s in enumerate(seqs):
        single = oracle.forward_request(m, np.array(s))
        assert np.array_equal(batch[i], single)
        assert abs(np.linalg.norm(batch[i]) - 1) < 1e-5
    # padding content is never read
    ids2 = ids.copy()
    ids2[4:6] = 3
    assert np.array_equal(oracle.forward(m, ids2, [len(s) for s in seqs]), batch)


def test_forward_trace_shapes_follow_merge():
    m = _tiny_model(layers=3, merge_after=1)
    trace = {}
    oracle.forward_request(m, np.arange(1, 11), trace)
    assert trace["qkv"][0].shape[0] == 10
    assert trace["qkv"][1].shape[0] == oracle.contextual_merged_length(10)
    assert trace["ffn"][2].shape == (7, 256)
