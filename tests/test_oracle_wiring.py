"""Pins of the oracle's graph wiring (oracle/oracle.py forward_request)
against the reference's execution plan, src/webgpu/model.ts:113-138 (graph)
and :154-168 (order of runs):

* the initial norm uses blk.0.attn_norm; after each attention output the
  residual add is normalized with blk.L.ffn_norm; after each down projection
  with blk.(L+1).attn_norm, or output_norm after the last layer;
* after layer MERGE_AFTER_LAYER - 1 both the residual and the normalized
  stream are merged (model.ts:159), and the merged normalized stream feeds
  the next QKV projection as it is, without a second normalization;
* RoPE positions restart at 0 within the merged request (ops.ts:188,
  token % layerSequence with layerSequence the merged sequence);
* the pool reads the merged normalized stream (model.ts:138).

Each test builds a model whose weights make the expected output a closed
form computed here from first principles (zero or identity projections,
power-of-two norm weights, equal rows), and checks that a plausible wiring
mistake would give a different answer ("mutant" checks), so the test can
fail. The oracle's building blocks (rms_norm, merge, rope, attention, ...)
are pinned separately in test_oracle_forward.py.
"""
import math

import numpy as np
import pytest

import oracle
import synth

D = oracle.Dims(hidden=256, q_heads=4, kv_heads=2, head_dim=64, intermediate=256, layers=6, vocab=32,
                merge_after_layer=4)
H = D.hidden
QKV = D.qkv_width  # 512
EPS = D.rms_epsilon


def f16(a):
    """A stored activation: the shaders compute in float32 and store f16
    (src/webgpu/ops.ts), so a float64 value is rounded to float32, then to
    binary16, both to nearest even."""
    return np.asarray(a, dtype=np.float64).astype(np.float32).astype(np.float16)


def embedding_table(seed=7):
    """f16 [vocab, hidden]; row r scaled by 0.25 * 2^(r % 5) so rows differ
    in magnitude (normalizing before or after averaging then differs)."""
    base = synth.normal(seed, D.vocab * H).reshape(D.vocab, H)
    scale = 0.25 * 2.0 ** (np.arange(D.vocab) % 5)
    return f16(base * scale[:, None])


def make_model(emb, attn_norm, ffn_norm, out_norm, qkv=None, o=None, gu=None, down=None):
    z = lambda r, c: np.zeros((r, c), dtype=np.float32)
    m = oracle.Model(D, oracle.GGML_F16, emb, [np.asarray(w, np.float32) for w in attn_norm],
                     [np.asarray(w, np.float32) for w in ffn_norm], np.asarray(out_norm, np.float32))
    for l in range(D.layers):
        m.qkv.append(qkv[l] if qkv else z(QKV, H))
        m.attn_output.append(o[l] if o else z(H, D.q_heads * D.head_dim))
        m.gate_up.append(gu[l] if gu else z(2 * D.intermediate, H))
        m.down.append(down[l] if down else z(H, D.intermediate))
    return m


def rms_rows(x16, w):
    """Closed form of one RMSNorm with a zero residual delta: f16(x * (1 /
    sqrt(mean(x^2) + eps)) * w) per row (src/webgpu/ops.ts:21-56)."""
    x = x16.astype(np.float64)
    inv = 1.0 / np.sqrt((x * x).mean(axis=1, keepdims=True) + EPS)
    return f16(x * inv * np.asarray(w, np.float64)[None, :])


def l2(v):
    v = np.asarray(v, np.float64)
    return v / np.linalg.norm(v)


def cos(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


# merge bins worked out by hand from src/webgpu/ops.ts:648-654
# (start = 1 + ((p-1)(S-1)) // (T-1), end = 1 + (p(S-1)) // (T-1)):
# S = 3 -> T = 2: [0,1) [1,3); S = 7 -> T = 5: [0,1) [1,2) [2,4) [4,5) [5,7);
# S = 5 -> T = 4 (S-1 = 4, T-1 = 3): [0,1) [1,2) [2,3) [3,5);
# S = 6 -> T = 4 (S-1 = 5, T-1 = 3): [0,1) [1,2) [2,4) [4,6)
BINS = {2: [(0, 1), (1, 2)], 3: [(0, 1), (1, 3)], 5: [(0, 1), (1, 2), (2, 3), (3, 5)],
        6: [(0, 1), (1, 2), (2, 4), (4, 6)], 7: [(0, 1), (1, 2), (2, 4), (4, 5), (5, 7)]}


def merged(rows16, S):
    return np.stack([f16(rows16[a:b].astype(np.float64).mean(axis=0)) for a, b in BINS[S]])


def random_norms(seed, n):
    """float32 norm weights (GGUF F32 tensors), as the model holds them."""
    return [(1.0 + 0.3 * synth.normal(seed + i, H)).astype(np.float32) for i in range(n)]


# --------------------------------------------------------------------------
# zero projections: the embedding is a closed form of the token rows
# --------------------------------------------------------------------------

@pytest.mark.parametrize("ids", [[5] * 7, [3, 9], [3, 9, 17]])
def test_zero_projections_pool_the_output_normalized_merged_rows(ids):
    """All projections zero: attention and FFN add nothing, so x stays the
    token rows, merged after layer 4; the last norm applies output_norm to
    the merged rows and the pool averages those normalized rows."""
    emb = embedding_table()
    w_out = (1.0 + 0.5 * synth.normal(40, H)).astype(np.float32)
    m = make_model(emb, random_norms(41, D.layers), random_norms(60, D.layers), w_out)
    S = len(ids)
    assert oracle.contextual_merged_length(S) == len(BINS[S])
    x = emb[np.array(ids)]
    xm = merged(x, S)
    want = l2(rms_rows(xm, w_out).astype(np.float64).mean(axis=0))
    got = oracle.forward_request(m, np.array(ids))
    assert np.allclose(got, want, atol=1e-7, rtol=0)
    # mutants: each of these wirings gives another embedding
    if len(set(ids)) > 1 and len(BINS[S]) < S:
        unmerged = l2(rms_rows(x, w_out).astype(np.float64).mean(axis=0))  # pool before the merge
        assert cos(unmerged, want) < 1 - 1e-4
    pooled_x = l2(xm.astype(np.float64).mean(axis=0))  # pool of the residual stream
    assert cos(pooled_x, want) < 1 - 1e-3
    wrong_norm = l2(rms_rows(xm, m.attn_norm[-1]).astype(np.float64).mean(axis=0))  # last attn_norm
    assert cos(wrong_norm, want) < 1 - 1e-3


# --------------------------------------------------------------------------
# norm placement: power-of-two constant norm weights scale each normalized
# stream exactly, so every projection input carries its norm's exponent
# --------------------------------------------------------------------------

A_EXP = [1, -1, 2, 0, -2, 3]    # blk.L.attn_norm = 2^A_EXP[L]
B_EXP = [-3, 2, 1, -1, 3, 0]    # blk.L.ffn_norm = 2^B_EXP[L]
C_EXP = -2                      # output_norm


def test_norm_placement_by_power_of_two_weights():
    """Zero O and down projections keep x equal to the token rows; QKV and
    gate/up share one matrix W. Then QKV of layer L sees f16(x inv) * 2^a_L
    (blk.0.attn_norm first, then the post-FFN norm of layer L-1 with
    blk.L.attn_norm) and gate/up of layer L sees f16(x inv) * 2^b_L (the
    post-attention norm with blk.L.ffn_norm); scaling by a power of two is
    exact through f16 rounding and the float64 product, so both projections
    are exactly 2^e * f16(f16(x inv) W^T). Two tokens merge to themselves,
    so the identity also holds after the merge."""
    emb = embedding_table()
    W = (0.05 * synth.normal(70, QKV * H)).reshape(QKV, H).astype(np.float32)
    ones = np.ones(H)
    m = make_model(emb, [2.0 ** a * ones for a in A_EXP], [2.0 ** b * ones for b in B_EXP], 2.0 ** C_EXP * ones,
                   qkv=[W] * D.layers, gu=[W] * D.layers)
    ids = np.array([3, 9])
    trace = {}
    oracle.forward_request(m, ids, trace)
    n0 = rms_rows(emb[ids], ones)
    q0 = f16(n0.astype(np.float64) @ W.astype(np.float64).T)
    for layer in range(D.layers):
        assert np.array_equal(trace["qkv"][layer], f16(2.0 ** A_EXP[layer] * q0.astype(np.float64))), layer
        assert np.array_equal(trace["gate_up"][layer], f16(2.0 ** B_EXP[layer] * q0.astype(np.float64))), layer
        assert np.array_equal(trace["x"][layer], emb[ids])
    assert np.array_equal(trace["norm"][-1], f16(2.0 ** C_EXP * n0.astype(np.float64)))
    # mutants: the same layer's attn_norm after the down projection, or the
    # two norms of a layer swapped, would break the exponent pattern
    for layer in range(1, D.layers):
        assert A_EXP[layer] != A_EXP[layer - 1]
    assert all(a != b for a, b in zip(A_EXP, B_EXP))


# --------------------------------------------------------------------------
# the merged normalized stream feeds layer 5 as it is
# --------------------------------------------------------------------------

def value_passthrough_model(emb, norms, w_out):
    """Layer 4 (the first after the merge) with Wq = Wk = 0, Wv selecting
    hidden columns 0..Hkv*hd-1 and O the identity; every other projection
    zero. The attention then averages the values uniformly over the merged
    positions, so the layer adds the mean of the merged normalized rows'
    first 128 columns (per KV head, shared by its query heads)."""
    qkv = [np.zeros((QKV, H), np.float32) for _ in range(D.layers)]
    o = [np.zeros((H, D.q_heads * D.head_dim), np.float32) for _ in range(D.layers)]
    kv_cols = D.kv_heads * D.head_dim
    v0 = (D.q_heads + D.kv_heads) * D.head_dim
    qkv[4][v0 + np.arange(kv_cols), np.arange(kv_cols)] = 1.0
    o[4][:] = np.eye(H, dtype=np.float32)
    return make_model(emb, norms, random_norms(90, D.layers), w_out, qkv=qkv, o=o)


def passthrough_closed_form(emb, ids, norms, w_out, renormalize=False):
    S = len(ids)
    x = emb[np.array(ids)]
    xm = merged(x, S)
    # stream entering layer 4: the post-FFN norm of layer 3 (blk.4.attn_norm)
    # merged as it is, or (mutant) normalized again after the merge
    nm = rms_rows(xm, norms[4]) if renormalize else merged(rms_rows(x, norms[4]), S)
    v = nm[:, :D.kv_heads * D.head_dim].astype(np.float64)
    per_kv = [f16(v[:, g * D.head_dim:(g + 1) * D.head_dim].mean(axis=0)) for g in range(D.kv_heads)]
    att = np.concatenate([per_kv[h // (D.q_heads // D.kv_heads)] for h in range(D.q_heads)]).astype(np.float64)
    x5 = f16(xm.astype(np.float64) + att[None, :])
    return l2(rms_rows(x5, w_out).astype(np.float64).mean(axis=0))


@pytest.mark.parametrize("ids", [[3, 9, 17], [2, 7, 11, 19, 23, 29, 31]])
def test_merge_keeps_the_normalized_stream_as_it_is(ids):
    emb = embedding_table()
    norms = random_norms(80, D.layers)
    w_out = (1.0 + 0.4 * synth.normal(88, H)).astype(np.float32)
    m = value_passthrough_model(emb, norms, w_out)
    want = passthrough_closed_form(emb, ids, norms, w_out)
    got = oracle.forward_request(m, np.array(ids))
    assert np.allclose(got, want, atol=1e-7, rtol=0)
    mutant = passthrough_closed_form(emb, ids, norms, w_out, renormalize=True)
    assert cos(mutant, want) < 1 - 1e-4


# --------------------------------------------------------------------------
# RoPE positions after the merge
# --------------------------------------------------------------------------

def test_rope_positions_restart_in_the_merged_sequence():
    """Layers after the merge rotate queries and keys by their merged
    positions 0..T-1; the bins of a 7-token request start at 0, 1, 2, 4, 5,
    whose differences differ from the renumbered ones, so the attention
    (relative positions) tells the two apart."""
    emb = embedding_table()
    rng = np.random.default_rng(5)
    qkv = [(0.08 * rng.standard_normal((QKV, H))).astype(np.float32) for _ in range(D.layers)]
    m = make_model(emb, random_norms(100, D.layers), random_norms(110, D.layers), np.ones(H), qkv=qkv)
    ids = np.array([2, 7, 11, 19, 23, 29, 31])
    trace = {}
    oracle.forward_request(m, ids, trace)
    S, T = 7, 5
    table = oracle.rope_table(S, D.head_dim, D.rope_theta)
    for layer, n, pos_ok, pos_bad in ((0, S, np.arange(S), None), (4, T, np.arange(T), np.array([0, 1, 2, 4, 5]))):
        raw = trace["qkv"][layer]
        q, k = oracle.rope(raw, pos_ok, table, D)
        assert np.array_equal(trace["q"][layer], q) and np.array_equal(trace["k"][layer], k)
        v = raw[:, (D.q_heads + D.kv_heads) * D.head_dim:].reshape(n, D.kv_heads, D.head_dim)
        att = oracle.attention(q, k, v, D).reshape(n, -1)
        assert np.array_equal(trace["attention"][layer], att)
        if pos_bad is not None:
            qb, kb = oracle.rope(raw, pos_bad, table, D)
            bad = oracle.attention(qb, kb, v, D).reshape(n, -1)
            assert np.abs(bad.astype(np.float64) - att.astype(np.float64)).max() > 1e-3


# --------------------------------------------------------------------------
# which keys each layer attends: the code's rule and README.md:26's
# --------------------------------------------------------------------------

def uniform_passthrough_model(emb, norms, w_out, layer, dims=D):
    """Layer `layer` with Wq = Wk = 0 (every score 0, so the attention
    weights are uniform over the keys it attends), Wv selecting hidden
    columns 0..Hkv*hd-1 and O the identity; every other projection zero."""
    qkv = [np.zeros((QKV, H), np.float32) for _ in range(dims.layers)]
    o = [np.zeros((H, dims.q_heads * dims.head_dim), np.float32) for _ in range(dims.layers)]
    kv_cols = dims.kv_heads * dims.head_dim
    v0 = (dims.q_heads + dims.kv_heads) * dims.head_dim
    qkv[layer][v0 + np.arange(kv_cols), np.arange(kv_cols)] = 1.0
    o[layer][:] = np.eye(H, dtype=np.float32)
    m = make_model(emb, norms, random_norms(90, dims.layers), w_out, qkv=qkv, o=o)
    m.dims = dims
    return m


def uniform_closed_form(emb, ids, norms, w_out, layer, keys):
    """The embedding of `uniform_passthrough_model` when the pass-through
    layer attends key positions `keys` of its sequence: that layer adds,
    for every query, the mean over those keys of its input's normalized
    rows' first Hkv*hd columns (per KV head); layers before the merge see
    the token rows, layers after it the merged rows."""
    S = len(ids)
    x = emb[np.array(ids)]
    if layer >= D.merge_after_layer:
        x = merged(x, S)
        nm = merged(rms_rows(emb[np.array(ids)], norms[layer]), S)
    else:
        nm = rms_rows(x, norms[layer])
    v = nm[np.array(keys), :D.kv_heads * D.head_dim].astype(np.float64)
    per_kv = [f16(v[:, g * D.head_dim:(g + 1) * D.head_dim].mean(axis=0)) for g in range(D.kv_heads)]
    att = np.concatenate([per_kv[h // (D.q_heads // D.kv_heads)] for h in range(D.q_heads)]).astype(np.float64)
    x = f16(x.astype(np.float64) + att[None, :])
    if layer < D.merge_after_layer:
        x = merged(x, S)
    return l2(rms_rows(x, w_out).astype(np.float64).mean(axis=0))


@pytest.mark.parametrize("dense_before_merge", [0, 1])
def test_key_sampling_rule_before_and_after_the_merge(dense_before_merge):
    """With threshold 4, a 7-token request (5 states after the merge) is
    longer than the threshold in every layer. The code's rule (ops.ts:258,
    kv_dense_before_merge 0) attends keys 0, 3, 6 in the first four layers
    and 0, 3 after the merge; README.md:26's rule (1) attends all 7 keys
    before the merge and the same 0, 3 after it."""
    from dataclasses import replace
    d = replace(D, kv_stride_threshold=4, kv_dense_before_merge=dense_before_merge)
    emb = embedding_table()
    norms = random_norms(120, D.layers)
    w_out = (1.0 + 0.4 * synth.normal(121, H)).astype(np.float32)
    ids = [2, 7, 11, 19, 23, 29, 31]
    for layer, keys, other in ((0, range(7) if dense_before_merge else [0, 3, 6],
                                [0, 3, 6] if dense_before_merge else range(7)),
                               (4, [0, 3], range(5))):
        m = uniform_passthrough_model(emb, norms, w_out, layer, d)
        want = uniform_closed_form(emb, ids, norms, w_out, layer, list(keys))
        got = oracle.forward_request(m, np.array(ids))
        assert np.allclose(got, want, atol=1e-7, rtol=0), f"layer {layer}"
        mutant = uniform_closed_form(emb, ids, norms, w_out, layer, list(other))
        assert cos(mutant, want) < 1 - 1e-4, f"layer {layer}: the other key set gives the same embedding"


# Threshold, request ids, keys attended in layer 0 (before the merge) and in
# layer 4 (after it, ceil(0.64 n) states) under the code's rule: a request
# exactly as long as the threshold attends every key (ops.ts:258 compares
# valid_length > threshold), one state longer attends every third.
KEY_RULE_BOUNDARY = [
    (5, [2, 7, 11, 19, 23], range(5), range(4)),           # 5 states = threshold: dense; 4 after the merge
    (5, [2, 7, 11, 19, 23, 29], [0, 3], range(4)),         # 6 > 5: every third; 4 after the merge: dense
    (4, [2, 7, 11, 19, 23, 29], [0, 3], range(4)),         # 6 > 4 before; 4 = threshold after the merge: dense
    (3, [2, 7, 11, 19, 23, 29], [0, 3], [0, 3]),           # 4 > 3 after the merge too: every third
]


@pytest.mark.parametrize("thr, ids, keys0, keys4", KEY_RULE_BOUNDARY)
def test_key_sampling_rule_at_the_threshold(thr, ids, keys0, keys4):
    """The threshold itself: a layer whose request holds exactly `threshold`
    states attends all of them, one more state switches to every third key.
    A rule with >= instead of > fails the first and third cases, one that
    counts tokens before the merge in later layers fails the third."""
    from dataclasses import replace
    d = replace(D, kv_stride_threshold=thr, kv_dense_before_merge=0)
    emb = embedding_table()
    norms = random_norms(130, D.layers)
    w_out = (1.0 + 0.4 * synth.normal(131, H)).astype(np.float32)
    n, n4 = len(ids), -(-len(ids) * 16 // 25)
    for layer, keys, states in ((0, keys0, n), (4, keys4, n4)):
        m = uniform_passthrough_model(emb, norms, w_out, layer, d)
        want = uniform_closed_form(emb, ids, norms, w_out, layer, list(keys))
        got = oracle.forward_request(m, np.array(ids))
        assert np.allclose(got, want, atol=1e-7, rtol=0), f"layer {layer}"
        other = range(states) if list(keys) != list(range(states)) else range(0, states, 3)
        mutant = uniform_closed_form(emb, ids, norms, w_out, layer, list(other))
        assert cos(mutant, want) < 1 - 1e-4, f"layer {layer}: the other key set gives the same embedding"

