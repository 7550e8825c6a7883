"""The dense path around the block (cpu_runner.rs), host side: the oracle's
restatement and the library's host functions (gossmx_attention,
gossmx_yarn_rope, gossmx_greedy_token) against the reference's known-answer
tests, against each other on random inputs, and the oracle's model step
against invariants of the reference's transactional KV design. No device
access: the library's host functions do not touch the GPU."""
import numpy as np
import pytest

import gossmx as G
import oracle as O
import synth

ROPE_20B = dict(rope_theta=150000.0, rope_yarn=1, rope_factor=32.0, rope_original_max_positions=4096)


def bits(a):
    return synth.bf16_bits(np.asarray(a, np.float32))


def bf16v(a):
    return synth.bf16_to_f32(bits(a))


def both_attention(q, keys, values, window, sinks, heads, kv_heads, head_dim):
    want, n, start = O.attention(q, bits(keys), bits(values), window, sinks, heads, kv_heads, head_dim)
    got = G.attention(q, bits(keys), bits(values), window, sinks, heads, kv_heads, head_dim)
    return want, got, n, start


# -- known-answer tests of cpu_runner.rs ------------------------------------------------

def test_attention_kat_bits():
    # attention_preserves_official_bf16_operator_boundaries, cpu_runner.rs:4301-4325
    keys = [[0.5, -0.25], [-0.75, 0.125], [0.375, 0.625]]
    values = [[1.25, -0.5], [-0.75, 2.0], [0.375, -1.5]]
    want, got, _, _ = both_attention([0.3125, -0.6875], keys, values, 3, [0.2], 1, 1, 2)
    assert list(bits(want)) == [16032, 48494]
    assert list(bits(got)) == [16032, 48494]


def test_learned_sink_only_changes_denominator():
    # learned_sink_only_changes_softmax_denominator, cpu_runner.rs:4286-4299
    for attend in (O.attention, None):
        outs = []
        for sink in (-100.0, 10.0):
            if attend:
                outs.append(attend([1.0, 0.0], bits([[1.0, 0.0]]), bits([[4.0, 0.0]]), 4, [sink], 1, 1, 2)[0])
            else:
                outs.append(G.attention([1.0, 0.0], bits([[1.0, 0.0]]), bits([[4.0, 0.0]]), 4, [sink], 1, 1, 2))
        assert abs(outs[0][0] - 4.0) < 1e-4
        assert outs[1][0] < 0.001


def test_full_and_sliding_share_current_token_semantics():
    # full_and_sliding_attention_share_current_token_semantics, cpu_runner.rs:4327-4342
    keys = [[p, 1.0] for p in range(2)]
    values = [[p + 1.0, 0.0] for p in range(2)]
    full = both_attention([0.25, 0.5], keys, values, 8, [0.0], 1, 1, 2)
    sliding = both_attention([0.25, 0.5], keys, values, 2, [0.0], 1, 1, 2)
    for a in full[:2] + sliding[:2]:
        assert (bits(a) == bits(full[0])).all()


@pytest.mark.parametrize("capacity,appends", [(3, 5), (128, 130)])
def test_sliding_cache_retains_exact_window(capacity, appends):
    # sliding_cache_retains_exact_window / gpt_oss_sliding_cache_retains_128_tokens,
    # cpu_runner.rs:4261-4284: len and start_position after the appends, and the
    # window holds exactly the last `capacity` rows: attention over the full
    # history with that window equals attention over those rows alone.
    rng = np.random.default_rng(capacity)
    keys = rng.standard_normal((appends, 2)).astype(np.float32)
    values = np.stack([np.arange(appends, dtype=np.float32), np.ones(appends, np.float32)], 1)
    q = bf16v(rng.standard_normal(2))
    out, n, start = O.attention(q, bits(keys), bits(values), capacity, [0.5], 1, 1, 2)
    assert (n, start) == (capacity, appends - capacity)
    alone, _, _ = O.attention(q, bits(keys[-capacity:]), bits(values[-capacity:]), 10 ** 6, [0.5], 1, 1, 2)
    assert (bits(out) == bits(alone)).all()
    assert (bits(G.attention(q, bits(keys), bits(values), capacity, [0.5], 1, 1, 2)) == bits(out)).all()


def test_yarn_position_zero_applies_attention_scale():
    # yarn_position_zero_applies_attention_scale, cpu_runner.rs:4344-4369
    scale = np.float32(np.float32(0.1) * np.log(np.float32(32.0)) + np.float32(1.0))
    cfg = G.model_config(head_dim=4, **ROPE_20B)
    for got in (O.yarn_rope(O.rope_struct(4), [1, 2, 3, 4], 1, 0), G.yarn_rope(cfg, [1, 2, 3, 4], 1, 0)):
        assert got[0] == bf16v(scale)
        assert got[3] == bf16v(4.0 * scale)


YARN_121_BITS = [
    15750, 15856, 48986, 16004, 16128, 49040, 49038, 16200, 49012, 16252, 16047, 48923,
    49010, 49014, 48994, 48970, 48950, 48932, 48919, 48909, 48897, 48877, 48855, 48834,
    48812, 48790, 48769, 48727, 48684, 48641, 48556, 48428, 49068, 49063, 49008, 49050,
    49035, 16012, 48692, 48964, 16112, 16042, 49013, 48971, 48780, 15876, 16066, 16137,
    16162, 16180, 16193, 16204, 16215, 16226, 16236, 16247, 16257, 16262, 16268, 16273,
    16278, 16284, 16289, 16295,
]


def test_yarn_head_dim_64_position_121_bits():
    # the head_dim 64 half of yarn_position_zero_applies_attention_scale, cpu_runner.rs:4371-4403
    values = (np.arange(64, dtype=np.float32) - 32.0) * 0.03125
    cfg = G.model_config(head_dim=64, **ROPE_20B)
    assert list(bits(O.yarn_rope(O.rope_struct(64), values, 1, 121))) == YARN_121_BITS
    assert list(bits(G.yarn_rope(cfg, values, 1, 121))) == YARN_121_BITS


def test_greedy_token_lowest_index_among_finite_maxima():
    # greedy_token, gpt-oss-bench/src/bin/cpu_parity.rs:750-762
    cases = [([1.0, 3.0, 3.0, 2.0], 1), ([np.nan, -np.inf, 2.0, np.inf], 2), ([-1.0], 0), ([0.0, -0.0], 0)]
    for logits, want in cases:
        assert O.greedy_token(logits) == want
        assert G.greedy_token(logits) == want
    assert O.greedy_token([np.nan, np.inf]) is None
    with pytest.raises(G.GossmxError) as e:
        G.greedy_token([np.nan, np.inf])
    assert e.value.status == G.ERR_NON_FINITE_LOGITS
    rng = np.random.default_rng(3)
    for _ in range(200):
        v = bf16v(rng.standard_normal(rng.integers(1, 50)) * 0.1)  # bf16 values: many ties
        assert O.greedy_token(v) == G.greedy_token(v) == int(np.flatnonzero(v == v.max())[0])


# -- the library's host functions against the oracle on random inputs -------------------

@pytest.mark.parametrize("heads,kv_heads,head_dim", [(1, 1, 2), (4, 2, 16), (8, 8, 8), (64, 8, 64)])
def test_attention_matches_oracle(heads, kv_heads, head_dim):
    rng = np.random.default_rng(heads * 100 + head_dim)
    for tokens in (1, 2, 7, 40):
        for window in (1, 3, 128):
            q = bf16v(rng.standard_normal(heads * head_dim) * 2.0)
            keys = rng.standard_normal((tokens, kv_heads * head_dim)).astype(np.float32)
            values = rng.standard_normal((tokens, kv_heads * head_dim)).astype(np.float32)
            sinks = bf16v(rng.standard_normal(heads))
            want, got, _, _ = both_attention(q, keys, values, window, sinks, heads, kv_heads, head_dim)
            assert (bits(got) == bits(want)).all(), (tokens, window)


@pytest.mark.parametrize("yarn", [1, 0])
def test_yarn_rope_matches_oracle(yarn):
    rng = np.random.default_rng(7 + yarn)
    rope = dict(ROPE_20B, rope_yarn=yarn)
    cfg = G.model_config(head_dim=64, **rope)
    o = O.rope_struct(64, yarn=bool(yarn))
    for position in (0, 1, 2, 121, 4095, 4096, 131071):
        v = bf16v(rng.standard_normal(3 * 64) * 4.0)
        assert (bits(G.yarn_rope(cfg, v, 3, position)) == bits(O.yarn_rope(o, v, 3, position))).all(), position


def test_host_entry_points_reject_bad_arguments():
    with pytest.raises(G.GossmxError) as e:
        G.attention([1.0, 0.0, 0.0], bits([[1.0, 0.0, 0.0]]), bits([[1.0, 0.0, 0.0]]), 4, [0.0, 0.0, 0.0], 3, 2, 1)
    assert e.value.status == G.ERR_INVALID_DIMENSIONS
    with pytest.raises(G.GossmxError) as e:
        G.yarn_rope(G.model_config(head_dim=3, **ROPE_20B), [1, 2, 3], 1, 0)
    assert e.value.status == G.ERR_INVALID_DIMENSIONS
    cfg = G.model_config(vocab=8, hidden=64, layers=1, heads=1, kv_heads=1, head_dim=2, sliding_window=2, **ROPE_20B)
    h = G.C.c_void_p()  # no context: INVALID_ARGUMENT before any device call
    st = G.load().gossmx_model_create(None, G.C.byref(cfg), None, None, None, None, G.C.byref(h))
    assert st == G.ERR_INVALID_ARGUMENT and not h.value


# -- the oracle's model step: invariants of the transactional KV design ---------------

TINY = dict(vocab=300, hidden=64, layers=2, heads=4, kv_heads=2, head_dim=16, sliding_window=4, context_cap=64,
            rms_norm_eps=1e-5, **ROPE_20B)


def tiny_model(seed=5, **over):
    cfg = dict(TINY, **over)
    w = synth.model_weights(cfg, synth.numpy_normal(np.random.default_rng(seed)))
    for i, L in enumerate(w["layers"]):
        L["moe_host"] = O.synthetic_layer(seed, i, experts=4, hidden=cfg["hidden"], intermediate=32, top_k=2)
    return cfg, w


def host_model(cfg, w):
    return O.ModelHost(cfg, w["embedding"], w["final_norm"], w["lm_head"], w["layers"])


PROMPT = np.array([3, 141, 59, 26, 53, 58, 97, 93, 238, 46, 264, 33], np.uint32)


def test_oracle_chunked_prefill_matches_one_step():
    # A prompt run as one layer-major step (prefill_layer_major) and as several
    # committed steps (prepare_step + commit per chunk) sees the same keys and
    # values: the staged rows of a step and the committed cache form one history.
    cfg, w = tiny_model()
    m = host_model(cfg, w)
    st, tokens, logits = O.model_generate(m, PROMPT, 5, prefill_chunk=0, threads=2)
    assert st == O.OK
    for chunk in (1, 5, 11):
        st, t2, l2 = O.model_generate(m, PROMPT, 5, prefill_chunk=chunk, threads=2)
        assert st == O.OK and (t2 == tokens).all()
        assert (l2.view(np.uint32) == logits.view(np.uint32)).all(), chunk


def test_oracle_window_covering_the_sequence_equals_full_attention():
    cfg, w = tiny_model()
    full = [dict(L, sliding=False) for L in w["layers"]]
    wide = host_model(dict(cfg, sliding_window=64), w)
    st, t1, l1 = O.model_generate(wide, PROMPT, 5, threads=2)
    st2, t2, l2 = O.model_generate(host_model(cfg, dict(w, layers=full)), PROMPT, 5, threads=2)
    assert st == st2 == O.OK
    assert (l1.view(np.uint32) == l2.view(np.uint32)).all()
    # ... while the 4-token window of the sliding layer changes the result.
    st3, t3, l3 = O.model_generate(host_model(cfg, w), PROMPT, 5, threads=2)
    assert st3 == O.OK and not (l3.view(np.uint32) == l1.view(np.uint32)).all()


def test_oracle_generate_threads_do_not_change_bits():
    cfg, w = tiny_model(seed=9)
    m = host_model(cfg, w)
    _, t1, l1 = O.model_generate(m, PROMPT, 3, threads=1)
    _, t2, l2 = O.model_generate(m, PROMPT, 3, threads=5)
    assert (l1.view(np.uint32) == l2.view(np.uint32)).all() and (t1 == t2).all()
