"""The HIP path against closed forms of the reference's graph wiring
(src/webgpu/model.ts:113-138, 154-168), with no oracle forward in between:
models whose projections are zero, unit selections or the identity (values
Q4_K holds exactly: d = 1, a sub-block scale of 1, nibbles 0 or 1), so the
embedding is a closed form of the token rows (tests/test_oracle_wiring.py
states and pins each form). Also the fused RoPE of the attention, checked
from the GPU's own QKV projection after the merge: the attention output the
kernel wrote must be the attention of that projection rotated by the merged
positions 0..T-1 (src/webgpu/ops.ts:168-193, 188).

Bars: closed forms cosine >= 0.99999 per request (the HIP path accumulates
in fp32, the closed forms in float64), and the request that a plausible
wiring mistake would give is further away; attention relative error <= 1e-2.
"""
import numpy as np
import pytest

import oracle
import synth
import test_oracle_wiring as W
from nemo_amd import runtime as rt

pytestmark = pytest.mark.gpu

D = W.D
H, QKV = W.H, W.QKV


def dims():
    return rt.make_dims(hidden=D.hidden, q_heads=D.q_heads, kv_heads=D.kv_heads, head_dim=D.head_dim,
                        intermediate=D.intermediate, layers=D.layers, vocab=D.vocab,
                        merge_after_layer=D.merge_after_layer)


def q4k_exact(w):
    """A matrix of zeros and ones as Q4_K blocks that decode to it exactly
    (d = 1.0, dmin = 0, scale 1 for sub-blocks holding a one, nibble = value)."""
    w = np.asarray(w)
    assert set(np.unique(w)) <= {0.0, 1.0}
    q = w.reshape(-1, 256).astype(np.int64)
    nb = q.shape[0]
    sc = (q.reshape(nb, 8, 32).max(axis=2) > 0).astype(np.int64)
    one = np.full(nb, 0x3C00, dtype=np.uint16)
    return synth.q4k_blocks(one, np.zeros(nb, np.uint16), sc, np.zeros((nb, 8), np.int64), q).tobytes()


def tensors_for(model):
    """name -> (type, gguf dims, bytes) for an oracle.Model of D whose
    matrices hold only zeros and ones."""
    t = {}
    for l in range(D.layers):
        p = f"blk.{l}."
        t[p + "attn_qkv.weight"] = (rt.TYPE_Q4_K, [H, QKV], q4k_exact(model.qkv[l]))
        t[p + "attn_output.weight"] = (rt.TYPE_Q4_K, [D.q_heads * D.head_dim, H], q4k_exact(model.attn_output[l]))
        t[p + "ffn_gate_up.weight"] = (rt.TYPE_Q4_K, [H, 2 * D.intermediate], q4k_exact(model.gate_up[l]))
        assert not model.down[l].any()
        t[p + "ffn_down.weight"] = (rt.TYPE_Q6_K, [D.intermediate, H], bytes(H * D.intermediate // 256 * 210))
        t[p + "attn_norm.weight"] = (rt.TYPE_F32, [H], np.asarray(model.attn_norm[l], np.float32).tobytes())
        t[p + "ffn_norm.weight"] = (rt.TYPE_F32, [H], np.asarray(model.ffn_norm[l], np.float32).tobytes())
    t["output_norm.weight"] = (rt.TYPE_F32, [H], np.asarray(model.output_norm, np.float32).tobytes())
    t["token_embd.weight"] = (rt.TYPE_F16, [H, D.vocab], np.asarray(model.embedding, np.float16).tobytes())
    return t


def run(model_tensors, requests, model_dims=None):
    model = rt.NemotronHipModel(model_tensors, dims=model_dims or dims())
    S = max(len(r) for r in requests)
    ids = np.full(len(requests) * S, 11, dtype=np.uint32)
    for i, r in enumerate(requests):
        ids[i * S:i * S + len(r)] = r
    plan = model.createPlan(len(requests), S)
    return plan.run_sync(ids, [len(r) for r in requests]), plan


REQUESTS = [[3, 9, 17], [2, 7, 11, 19, 23, 29, 31], [5] * 7]


def test_zero_projections_closed_form(torch_cuda):
    emb = W.embedding_table()
    w_out = (1.0 + 0.5 * synth.normal(40, H)).astype(np.float32)
    m = W.make_model(emb, W.random_norms(41, D.layers), W.random_norms(60, D.layers), w_out)
    got, _ = run(tensors_for(m), REQUESTS)
    for i, ids in enumerate(REQUESTS):
        S = len(ids)
        xm = W.merged(emb[np.array(ids)], S)
        want = W.l2(W.rms_rows(xm, w_out).astype(np.float64).mean(axis=0))
        c = W.cos(got[i], want)
        assert c >= 0.99999, f"request {i}: cosine {c}"
        pooled_x = W.l2(xm.astype(np.float64).mean(axis=0))  # a pool of the residual stream
        assert W.cos(got[i], pooled_x) < c


def test_merged_normalized_stream_feeds_the_next_layer(torch_cuda):
    emb = W.embedding_table()
    norms = W.random_norms(80, D.layers)
    w_out = (1.0 + 0.4 * synth.normal(88, H)).astype(np.float32)
    m = W.value_passthrough_model(emb, norms, w_out)
    requests = REQUESTS[:2]
    got, _ = run(tensors_for(m), requests)
    for i, ids in enumerate(requests):
        want = W.passthrough_closed_form(emb, ids, norms, w_out)
        mutant = W.passthrough_closed_form(emb, ids, norms, w_out, renormalize=True)
        c = W.cos(got[i], want)
        assert c >= 0.99999, f"request {i}: cosine {c}"
        assert W.cos(got[i], mutant) < c - 1e-5


def test_fused_rope_uses_merged_positions(torch_cuda):
    """A 7-token request (merged to 5 states, bins starting at 0, 1, 2, 4,
    5) through random Q4_K projections of N(0, 0.15) weights (large enough
    that the scores, and so the attention, depend on relative position: at
    N(0, 0.02) the two position sets differ by 6e-4 only): the last layer's
    attention output, as the kernel wrote it while rotating queries and keys
    on load, against
    the oracle's attention of the GPU's own QKV projection rotated by
    positions 0..4 (and, as the mutant, by the bins' first positions)."""
    d = dims()
    tensors = synth.model_tensors(d, seed=900, sigma=0.15)
    model = rt.NemotronHipModel(tensors, dims=d)
    ids = np.array([1, 7, 11, 19, 23, 29, 31], dtype=np.uint32)
    plan = model.createPlan(1, 7)
    plan.run_sync(ids, [7])
    T = 5
    qkv = plan.read_buffer("qkv")[:T * QKV].reshape(T, QKV)
    att = plan.read_buffer("attention")[:T * D.q_heads * D.head_dim].reshape(T, -1)
    table = oracle.rope_table(7, D.head_dim, D.rope_theta)
    v = qkv[:, (D.q_heads + D.kv_heads) * D.head_dim:].reshape(T, D.kv_heads, D.head_dim)

    def expected(positions):
        q, k = oracle.rope(qkv, positions, table, D)
        return oracle.attention(q, k, v, D).reshape(T, -1).astype(np.float64)

    good, bad = expected(np.arange(T)), expected(np.array([0, 1, 2, 4, 5]))
    a = att.astype(np.float64)
    err = np.linalg.norm(a - good) / np.linalg.norm(good)
    err_bad = np.linalg.norm(a - bad) / np.linalg.norm(bad)
    assert err <= 1e-2, f"attention relative error {err}"
    assert err_bad > 0.05 and err_bad > 20 * err, (err, err_bad)


@pytest.mark.parametrize("dense_before_merge", [0, 1])
def test_key_sampling_rule_before_and_after_the_merge(torch_cuda, dense_before_merge):
    """The attention's key set per layer under both rules (threshold 4, a
    7-token request, 5 states after the merge): uniform attention over the
    keys a layer attends makes the embedding a closed form of that key set
    (tests/test_oracle_wiring.py). The code's rule (src/webgpu/ops.ts:258)
    attends keys 0, 3, 6 before the merge; README.md:26's attends all 7;
    both attend 0, 3 after it."""
    from dataclasses import replace
    d = replace(D, kv_stride_threshold=4, kv_dense_before_merge=dense_before_merge)
    rd = dims()
    rd.kv_stride_threshold, rd.kv_dense_before_merge = 4, dense_before_merge
    emb = W.embedding_table()
    norms = W.random_norms(120, D.layers)
    w_out = (1.0 + 0.4 * synth.normal(121, H)).astype(np.float32)
    ids = [2, 7, 11, 19, 23, 29, 31]
    for layer, keys, other in ((0, range(7) if dense_before_merge else [0, 3, 6],
                                [0, 3, 6] if dense_before_merge else range(7)),
                               (4, [0, 3], range(5))):
        m = W.uniform_passthrough_model(emb, norms, w_out, layer, d)
        got, _ = run(tensors_for(m), [ids], rd)
        want = W.uniform_closed_form(emb, ids, norms, w_out, layer, list(keys))
        mutant = W.uniform_closed_form(emb, ids, norms, w_out, layer, list(other))
        c = W.cos(got[0], want)
        assert c >= 0.99999, f"layer {layer}: cosine {c}"
        assert W.cos(got[0], mutant) < c - 1e-5, f"layer {layer}"


@pytest.mark.parametrize("thr, ids, keys0, keys4", W.KEY_RULE_BOUNDARY)
def test_key_sampling_rule_at_the_threshold(torch_cuda, thr, ids, keys0, keys4):
    """The attention kernel's key rule at the threshold itself, against the
    same closed forms as the oracle (tests/test_oracle_wiring.py): exactly
    `threshold` states attend every key, one more every third, judged on the
    layer's own state count after the merge."""
    from dataclasses import replace
    d = replace(D, kv_stride_threshold=thr, kv_dense_before_merge=0)
    rd = dims()
    rd.kv_stride_threshold = thr
    emb = W.embedding_table()
    norms = W.random_norms(130, D.layers)
    w_out = (1.0 + 0.4 * synth.normal(131, H)).astype(np.float32)
    n, n4 = len(ids), -(-len(ids) * 16 // 25)
    for layer, keys, states in ((0, keys0, n), (4, keys4, n4)):
        m = W.uniform_passthrough_model(emb, norms, w_out, layer, d)
        got, _ = run(tensors_for(m), [ids], rd)
        want = W.uniform_closed_form(emb, ids, norms, w_out, layer, list(keys))
        other = range(states) if list(keys) != list(range(states)) else range(0, states, 3)
        mutant = W.uniform_closed_form(emb, ids, norms, w_out, layer, list(other))
        c = W.cos(got[0], want)
        assert c >= 0.99999, f"layer {layer}: cosine {c}"
        assert W.cos(got[0], mutant) < c - 1e-5, f"layer {layer}"

