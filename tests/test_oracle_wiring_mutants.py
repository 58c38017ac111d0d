"""The wiring pins of test_oracle_wiring.py must fail on a mis-wired forward
pass. Each case plants one plausible mistake in a copy of the oracle's
forward_request (on the CPU, in this process only) and checks that at least
the named pin then fails:

* normalizing again after the merge (src/webgpu/model.ts:159 merges the
  normalized stream as it is);
* the same layer's attn_norm after the down projection (model.ts:133 takes
  the next layer's);
* attn_norm and ffn_norm exchanged after the attention output (model.ts:130);
* pre-merge positions for RoPE after the merge (src/webgpu/ops.ts:188);
* pooling the residual stream (model.ts:138 pools the normalized one);
* merging only the residual stream (model.ts:159 merges both);
* every third key from `threshold` states on instead of above it
  (src/webgpu/ops.ts:258 compares valid_length > threshold);
* the key rule judged on the request's tokens before the merge in the
  layers after it.
"""
import inspect
import textwrap

import pytest

import oracle
import test_oracle_wiring as pins

MUTANTS = {
    "renormalize after merge": (
        "            norm = merge(norm, S, T)\n",
        "            norm = merge(norm, S, T)\n            _, norm = rms_norm(x, model.attn_norm[layer], d.rms_epsilon)\n",
        "test_merge_keeps_the_normalized_stream_as_it_is"),
    "same-layer attn_norm after down": (
        "nxt = model.attn_norm[layer + 1] if layer + 1 < d.layers else model.output_norm",
        "nxt = model.attn_norm[layer] if layer + 1 < d.layers else model.output_norm",
        "test_norm_placement_by_power_of_two_weights"),
    "ffn and attn norms exchanged": (
        "x, norm = rms_norm(x, model.ffn_norm[layer], d.rms_epsilon, delta_o)",
        "x, norm = rms_norm(x, model.attn_norm[layer], d.rms_epsilon, delta_o)",
        "test_norm_placement_by_power_of_two_weights"),
    "pre-merge positions after the merge": (
        "q, k = rope(qkv, np.arange(n), table, d)",
        "q, k = rope(qkv, np.array([b[0] for b in merge_bins(S, T)]) if n != S else np.arange(n), table, d)",
        "test_rope_positions_restart_in_the_merged_sequence"),
    "pool the residual stream": (
        "    return mean_pool(norm, T)",
        "    return mean_pool(x, T)",
        "test_zero_projections_pool_the_output_normalized_merged_rows"),
    "threshold compared with >=": (
        "att = attention(q, k, v, d, n if dense else d.kv_stride_threshold, d.kv_stride)",
        "att = attention(q, k, v, d, n if dense else d.kv_stride_threshold - 1, d.kv_stride)",
        "test_key_sampling_rule_at_the_threshold"),
    "key rule on the tokens before the merge": (
        "att = attention(q, k, v, d, n if dense else d.kv_stride_threshold, d.kv_stride)",
        "att = attention(q, k, v, d, n if dense else d.kv_stride_threshold - (S - n), d.kv_stride)",
        "test_key_sampling_rule_at_the_threshold"),
    "merge only the residual stream": (
        "            norm = merge(norm, S, T)\n",
        "            norm = norm[[b[0] for b in merge_bins(S, T)]]\n",
        "test_merge_keeps_the_normalized_stream_as_it_is"),
}


def _cases(test):
    for mark in getattr(test, "pytestmark", []):
        if mark.name == "parametrize":
            names = mark.args[0]
            multi = "," in names if isinstance(names, str) else len(names) > 1
            return [tuple(v) if multi else (v,) for v in mark.args[1]]
    return [()]


@pytest.mark.parametrize("name", sorted(MUTANTS))
def test_pin_fails_on_mutant(name, monkeypatch):
    original, planted, pin = MUTANTS[name]
    src = inspect.getsource(oracle.forward_request)
    assert original in src, "the oracle changed; update the mutant"
    namespace = dict(vars(oracle))
    exec(textwrap.dedent(src.replace(original, planted)), namespace)
    monkeypatch.setattr(oracle, "forward_request", namespace["forward_request"])
    test = getattr(pins, pin)
    failures = 0
    for case in _cases(test):
        try:
            test(*case)
        except AssertionError:
            failures += 1
    assert failures > 0, f"{pin} passes on the mutant '{name}'"
