"""A GPT-OSS model with its attention on the host and its projections and MoE blocks on the GPU
(gossmx_model_*) against the oracle's whole-model restatement
(oracle_model_generate): greedy tokens and every logits bit, for a small model
and for configs[3], the random-init GPT-OSS-20B forward (63-token prefill,
8 greedy decode steps)."""
import numpy as np
import pytest

import gossmx as G
import oracle as O
import synth

pytestmark = pytest.mark.gpu

ROPE_20B = dict(rope_theta=150000.0, rope_yarn=1, rope_factor=32.0, rope_original_max_positions=4096)
TINY = dict(vocab=300, hidden=64, layers=2, heads=4, kv_heads=2, head_dim=16, sliding_window=4, context_cap=64,
            rms_norm_eps=1e-5, **ROPE_20B)
PROMPT = np.array([3, 141, 59, 26, 53, 58, 97, 93, 238, 46, 264, 33], np.uint32)


@pytest.fixture(scope="module")
def ctx():
    c = G.Context(0)
    yield c
    c.close()


def build(ctx, cfg, w, moe_hosts):
    """Device MoE layers from the hosts' canonical tensors, and the product model."""
    layers, keep = [], []
    for L, host in zip(w["layers"], moe_hosts):
        E, H, I = host.experts, host.hidden, host.intermediate
        gu = G.Weights.upload(ctx, host.gate_up, E, 2 * I, H // 32)
        dn = G.Weights.upload(ctx, host.down, E, H, I // 32)
        moe = G.MoeLayer(ctx, E, H, I, host.top_k, host.router_weight, host.router_bias, gu, host.gate_up_bias, dn,
                         host.down_bias)
        keep += [gu, dn, moe]
        layers.append(dict(L, moe=moe))
    conf = G.model_config(threads=4, **cfg)
    return G.Model(ctx, conf, w["embedding"], w["final_norm"], w["lm_head"], layers), keep


def release(model, keep):
    model.close()
    for k in reversed(keep):
        k.close()


@pytest.fixture(scope="module")
def tiny(ctx):
    cfg = dict(TINY)
    w = synth.model_weights(cfg, synth.numpy_normal(np.random.default_rng(5)))
    hosts = [O.synthetic_layer(5, i, experts=4, hidden=64, intermediate=32, top_k=2) for i in range(cfg["layers"])]
    for L, h in zip(w["layers"], hosts):
        L["moe_host"] = h
    model, keep = build(ctx, cfg, w, hosts)
    oracle = O.ModelHost(cfg, w["embedding"], w["final_norm"], w["lm_head"], w["layers"])
    yield cfg, model, oracle
    release(model, keep)


def assert_bits(got, want):
    assert (np.asarray(got, np.float32).view(np.uint32) == np.asarray(want, np.float32).view(np.uint32)).all()


def test_small_model_matches_oracle(tiny):
    cfg, model, oracle = tiny
    st, want_tokens, want_logits = O.model_generate(oracle, PROMPT, 6, threads=4)
    assert st == O.OK
    tokens, logits = model.generate(PROMPT, 6)
    assert (tokens == want_tokens).all()
    assert_bits(logits, want_logits)
    assert model.position == PROMPT.size + 6
    # CpuKvCache after 18 positions: the sliding layer keeps 4, the full layer all.
    assert model.cache(0) == (4, 14) and model.cache(1) == (18, 0)
    dense, moe = model.times()
    assert dense > 0 and moe > 0


# Projection shapes off the fast paths: Q width 18 (O's input is not a
# multiple of 8 values, so the K-chunked kernel's element-wise loads run), Q/K/V
# and vocab row counts that are not multiples of the 16-row work-group, and a
# 20-token prompt (a full and a partial 16-row input group).
RAGGED = dict(vocab=301, hidden=64, layers=2, heads=3, kv_heads=1, head_dim=6, sliding_window=5, context_cap=64,
              rms_norm_eps=1e-5, **ROPE_20B)


def test_ragged_projection_shapes_match_oracle(ctx):
    cfg = dict(RAGGED)
    w = synth.model_weights(cfg, synth.numpy_normal(np.random.default_rng(7)))
    hosts = [O.synthetic_layer(7, i, experts=4, hidden=64, intermediate=32, top_k=2) for i in range(cfg["layers"])]
    for L, h in zip(w["layers"], hosts):
        L["moe_host"] = h
    model, keep = build(ctx, cfg, w, hosts)
    try:
        oracle = O.ModelHost(cfg, w["embedding"], w["final_norm"], w["lm_head"], w["layers"])
        prompt = (np.arange(20, dtype=np.uint32) * 13) % 301
        st, want_tokens, want_logits = O.model_generate(oracle, prompt, 4, threads=4)
        assert st == O.OK
        tokens, logits = model.generate(prompt, 4)
        assert (tokens == want_tokens).all()
        assert_bits(logits, want_logits)
    finally:
        release(model, keep)


def test_small_model_chunked_prefill(tiny):
    cfg, model, oracle = tiny
    _, _, want = O.model_generate(oracle, PROMPT, 0, threads=4)
    model.reset()
    assert model.position == 0
    for lo in range(0, PROMPT.size, 5):
        logits = model.append(PROMPT[lo:lo + 5])
    assert_bits(logits, want[0])


def test_small_model_failed_step_changes_nothing(tiny):
    cfg, model, oracle = tiny
    _, want_tokens, want_logits = O.model_generate(oracle, PROMPT, 2, threads=4)
    model.prefill(PROMPT)
    with pytest.raises(G.GossmxError) as e:
        model.decode(cfg["vocab"])  # token id out of range
    assert e.value.status == G.ERR_INVALID_ARGUMENT
    with pytest.raises(G.GossmxError):
        model.append(np.zeros(cfg["context_cap"], np.uint32))  # passes the context cap
    assert model.position == PROMPT.size and model.cache(0) == (4, 8)
    assert_bits(model.decode(want_tokens[0]), want_logits[1])
    assert_bits(model.decode(want_tokens[1]), want_logits[2])
    with pytest.raises(G.GossmxError):
        model.reset()
        model.decode(1)  # decode needs a prefill


def test_small_model_moe_failure_mid_step_changes_nothing(ctx, tiny):
    # The first MoE call of the step fails (the library's one-shot injected
    # fault, raised before any launch): the step reports it and commits nothing.
    cfg, model, oracle = tiny
    _, want_tokens, want_logits = O.model_generate(oracle, PROMPT, 1, threads=4)
    model.prefill(PROMPT)
    before = [model.cache(i) for i in range(cfg["layers"])]
    ctx.inject_fault(True)
    with pytest.raises(G.GossmxError) as e:
        model.decode(want_tokens[0])
    assert e.value.status == G.ERR_INJECTED_FAULT
    assert model.position == PROMPT.size and [model.cache(i) for i in range(cfg["layers"])] == before
    assert_bits(model.decode(want_tokens[0]), want_logits[1])


def test_small_model_device_flag_failure_opens_the_breaker(ctx, tiny):
    # The first MoE call of the step runs with its device error flag raised
    # (FAULT_FLAG, a host-sourced write, no kernel faults); the step finds it
    # when it synchronizes, fails with GOSSMX_ERR_DEVICE, opens the circuit
    # breaker and commits nothing. While the breaker is open the next step
    # fails fast; after the reset it matches the oracle.
    cfg, model, oracle = tiny
    _, want_tokens, want_logits = O.model_generate(oracle, PROMPT, 1, threads=4)
    model.prefill(PROMPT)
    before = [model.cache(i) for i in range(cfg["layers"])]
    try:
        ctx.inject_fault(G.FAULT_FLAG)
        with pytest.raises(G.GossmxError) as e:
            model.decode(want_tokens[0])
        assert e.value.status == G.ERR_DEVICE
        assert G.circuit_is_open()
        with pytest.raises(G.GossmxError) as e:
            model.decode(want_tokens[0])
        assert e.value.status == G.ERR_CIRCUIT_OPEN
        assert model.position == PROMPT.size and [model.cache(i) for i in range(cfg["layers"])] == before
    finally:
        G.circuit_reset()
    assert_bits(model.decode(want_tokens[0]), want_logits[1])


def test_small_model_profile_records_carry_layer_and_phase(ctx, tiny):
    # The model step tags its MoE calls with the layer index and the phase
    # (CpuExecutionProfileRecord's layer and phase, cpu_profile.rs:121-150);
    # its round trips count as activation and output transfers.
    cfg, model, _ = tiny
    model.reset()
    ctx.profile(True)
    ctx.profile_reset()
    try:
        s0 = G.stats()
        logits = model.prefill(PROMPT)
        prefill, _ = ctx.profile_events()
        ctx.profile_reset()
        model.decode(G.greedy_token(logits))
        decode, dropped = ctx.profile_events()
        s1 = G.stats()
    finally:
        ctx.profile(False)
        ctx.profile_reset()
        ctx.profile_tag()
        model.reset()
    assert dropped == 0
    for events, phase, m in ((prefill, "prefill", len(PROMPT)), (decode, "decode", 1)):
        assert {e["layer"] for e in events} == set(range(cfg["layers"]))
        assert {e["phase"] for e in events} == {phase}
        assert {e["m"] for e in events} == {m} and {e["memory"] for e in events} == {"device"}
        assert {e["op"] for e in events} >= {"gate_up", "down"}
    assert s1["projections_ok"] - s0["projections_ok"] == 2 * cfg["layers"]
    assert s1["activation_bytes"] > s0["activation_bytes"] and s1["output_bytes"] > s0["output_bytes"]


def test_small_model_follows_a_replaced_stream():
    # gossmx_ctx_set_stream between generations (the context's own stream is
    # destroyed): the model's copies, launches and MoE calls run on the new
    # stream (a plain HIP stream at the default priority), and tokens and
    # logits bits still equal the oracle's.
    import ctypes as C
    hip = C.CDLL("libamdhip64.so")
    c = G.Context(0)
    cfg = dict(TINY)
    w = synth.model_weights(cfg, synth.numpy_normal(np.random.default_rng(6)))
    hosts = [O.synthetic_layer(6, i, experts=4, hidden=64, intermediate=32, top_k=2) for i in range(cfg["layers"])]
    for L, h in zip(w["layers"], hosts):
        L["moe_host"] = h
    model, keep = build(c, cfg, w, hosts)
    stream = C.c_void_p()
    assert hip.hipStreamCreate(C.byref(stream)) == 0
    try:
        oracle = O.ModelHost(cfg, w["embedding"], w["final_norm"], w["lm_head"], w["layers"])
        st, want_tokens, want_logits = O.model_generate(oracle, PROMPT, 4, threads=4)
        assert st == O.OK
        tokens, logits = model.generate(PROMPT, 4)
        assert (tokens == want_tokens).all()
        assert_bits(logits, want_logits)
        c.set_stream(stream.value)
        assert c.stream == stream.value
        model.reset()
        tokens, logits = model.generate(PROMPT, 4)
        assert (tokens == want_tokens).all()
        assert_bits(logits, want_logits)
    finally:
        release(model, keep)
        c.close()
        assert hip.hipStreamDestroy(stream) == 0


def hash_normal(seed):
    """normal(n, std) for model_weights: the oracle's counter-hash Gaussian,
    one stream per tensor, generated on 16 host threads."""
    stream = [1000]

    def normal(n, std):
        stream[0] += 1
        return O.gen_bf16_normal_mt(seed, stream[0], n, 0.0, std, threads=16)

    return normal


def gpt_oss_20b(ctx, layers, seed):
    """random-init GPT-OSS-20B dense weights, device-generated MXFP4
    experts (the bench's synthetic distribution) and their canonical host copies."""
    cfg = dict(G.GPT_OSS_20B, layers=layers, context_cap=4096)
    w = synth.model_weights(cfg, hash_normal(seed))
    layers_out, keep = [], []
    rng = np.random.default_rng(seed)
    for i, L in enumerate(w["layers"]):
        E, H, I, B = 32, 2880, 2880, 90
        gu = G.Weights.generate(ctx, seed, 16 * i + 4, E, 2 * I, B)
        dn = G.Weights.generate(ctx, seed, 16 * i + 5, E, H, B)
        p = synth.dense_layer_params(rng, E)
        moe = G.MoeLayer(ctx, E, H, I, 4, p["router_weight"], p["router_bias"], gu, p["gate_up_bias"], dn,
                         p["down_bias"])
        L["moe_host"] = O.MoeLayerHost(p["router_weight"], p["router_bias"], gu.export_canonical(), p["gate_up_bias"],
                                       dn.export_canonical(), p["down_bias"], E, H, I, 4)
        keep += [gu, dn, moe]
        layers_out.append(dict(L, moe=moe))
    conf = G.model_config(threads=16, **cfg)
    model = G.Model(ctx, conf, w["embedding"], w["final_norm"], w["lm_head"], layers_out)
    oracle = O.ModelHost(cfg, w["embedding"], w["final_norm"], w["lm_head"], w["layers"])
    return model, keep, oracle


@pytest.mark.parametrize("layers", [2, 24])
def test_gpt_oss_20b_greedy_tokens_match_oracle(ctx, layers):
    """configs[3] (24 layers) and a 2-layer cut of it: 63-token prefill, 8 greedy
    decode steps; every token and every logits bit as the oracle's."""
    model, keep, oracle = gpt_oss_20b(ctx, layers, seed=2026)
    prompt = np.random.default_rng(63).integers(0, G.GPT_OSS_20B["vocab"], 63).astype(np.uint32)
    try:
        tokens, logits = model.generate(prompt, 8)
        dense, moe = model.times()
        st, want_tokens, want_logits = O.model_generate(oracle, prompt, 8, threads=16)
        assert st == O.OK
        print(f"layers={layers} tokens={tokens.tolist()} dense={dense:.2f}s moe={moe:.3f}s", flush=True)
        assert (tokens == want_tokens).all()
        assert_bits(logits, want_logits)
    finally:
        release(model, keep)
