"""Process-wide accounting and per-stage profile records on the GPU: the
counters the Xe engine exports as metrics (crates/gpt-oss-xe/src/lib.rs:44-49,
785-825; XeResidencyStats :358-370; the resident cap of AttachConfig
:239-250) and the per-stage records of CpuExecutionProfiler
(crates/gpt-oss-model-runner/src/cpu_profile.rs:121-150). Counters are
process-wide, so every check is on the difference across the calls it makes."""
import numpy as np
import pytest

import gossmx as G
import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = G.Context(0)
    yield c
    c.close()


def gpu_layer(ctx, host):
    E, H, I = host.experts, host.hidden, host.intermediate
    gu = G.Weights.upload(ctx, host.gate_up, E, 2 * I, H // 32)
    dn = G.Weights.upload(ctx, host.down, E, H, I // 32)
    return G.MoeLayer(ctx, E, H, I, host.top_k, host.router_weight, host.router_bias, gu, host.gate_up_bias, dn,
                      host.down_bias, host.alpha, host.limit)


def close(layer):
    layer.close()
    layer.gate_up.close()
    layer.down.close()


def delta(before, after):
    return {k: after[k] - before[k] for k in before}


def test_resident_bytes_follow_weights_and_layers(ctx):
    E, H, I, K = 4, 64, 32, 2
    host = O.synthetic_layer(21, 0, experts=E, hidden=H, intermediate=I, top_k=K)
    s0 = G.stats()
    gu = G.Weights.upload(ctx, host.gate_up, E, 2 * I, H // 32)
    s1 = G.stats()
    d = delta(s0, s1)
    # the planes with their padding and the per-tile flags: above the planes alone
    assert d["resident_bytes"] > gu.device_bytes()
    assert d["weights_bias_uploaded_bytes"] == host.gate_up.nbytes
    assert s1["resident_high_water_bytes"] >= s1["resident_bytes"]
    dn = G.Weights.upload(ctx, host.down, E, H, I // 32)
    s2 = G.stats()
    layer = G.MoeLayer(ctx, E, H, I, K, host.router_weight, host.router_bias, gu, host.gate_up_bias, dn,
                       host.down_bias, host.alpha, host.limit)
    s3 = G.stats()
    layer_bytes = E * H * 2 + E * 4 + E * 2 * I * 4 + E * H * 4
    assert s3["resident_bytes"] - s2["resident_bytes"] == layer_bytes
    assert s3["weights_bias_uploaded_bytes"] - s2["weights_bias_uploaded_bytes"] == layer_bytes
    close(layer)
    assert G.stats()["resident_bytes"] == s0["resident_bytes"]


def test_resident_cap_refuses_creation_before_allocating(ctx):
    E, H, I = 4, 64, 32
    host = O.synthetic_layer(22, 0, experts=E, hidden=H, intermediate=I, top_k=2)
    s0 = G.stats()
    try:
        G.set_resident_cap(s0["resident_bytes"] + 1024)
        assert G.stats()["resident_cap_bytes"] == s0["resident_bytes"] + 1024
        with pytest.raises(G.GossmxError) as e:
            G.Weights.upload(ctx, host.gate_up, E, 2 * I, H // 32)
        assert e.value.status == G.ERR_OUT_OF_MEMORY
        assert "resident cap" in str(e.value)
        with pytest.raises(G.GossmxError) as e:
            G.Weights.generate(ctx, 1, 2, E, H, I // 32)
        assert e.value.status == G.ERR_OUT_OF_MEMORY
        s1 = G.stats()
        assert s1["capacity_refusals"] - s0["capacity_refusals"] == 2
        assert s1["resident_bytes"] == s0["resident_bytes"]
        # nothing was uploaded for the refused creations
        assert s1["weights_bias_uploaded_bytes"] == s0["weights_bias_uploaded_bytes"]
        assert not G.circuit_is_open()  # a capacity refusal is not a device fault
    finally:
        G.set_resident_cap(0)
    w = G.Weights.upload(ctx, host.gate_up, E, 2 * I, H // 32)
    # a layer that does not fit: its weights stay, the layer is refused
    dn = G.Weights.upload(ctx, host.down, E, H, I // 32)
    try:
        G.set_resident_cap(G.stats()["resident_bytes"] + 16)
        with pytest.raises(G.GossmxError) as e:
            G.MoeLayer(ctx, E, H, I, 2, host.router_weight, host.router_bias, w, host.gate_up_bias, dn,
                       host.down_bias, host.alpha, host.limit)
        assert e.value.status == G.ERR_OUT_OF_MEMORY
    finally:
        G.set_resident_cap(0)
    w.close()
    dn.close()
    assert G.stats()["resident_bytes"] == s0["resident_bytes"]


def test_projection_results_and_transfer_bytes(ctx):
    E, H, I, K, m = 4, 64, 32, 2, 3
    host = O.synthetic_layer(23, 0, experts=E, hidden=H, intermediate=I, top_k=K)
    layer = gpu_layer(ctx, host)
    x = O.gen_hidden(23, 1, m, H)
    s0 = G.stats()
    layer.forward(x)
    d = delta(s0, G.stats())
    assert d["projections_ok"] == 1 and d["projections_failed"] == 0 and d["projections_rejected"] == 0
    assert d["activation_bytes"] == m * H * 2
    # logits, selected, routing weights, route order, and the output rows
    # (bf16 values: they cross as bf16 bits and are widened on the host)
    assert d["output_bytes"] == m * E * 4 + 3 * m * K * 4 + m * H * 2
    # device memory: no transfers
    dx, dout = ctx.malloc(x.nbytes), ctx.malloc(m * H * 4)
    ctx.h2d(dx, x)
    s1 = G.stats()
    layer.forward_device(dx, m, dout)
    ctx.synchronize()
    d = delta(s1, G.stats())
    assert d["projections_ok"] == 1 and d["activation_bytes"] == 0 and d["output_bytes"] == 0
    # rejected (shape), failed (injected model error, device fault), refused (breaker open)
    s2 = G.stats()
    with pytest.raises(G.GossmxError):
        layer.forward(x[:0])
    ctx.inject_fault(G.FAULT_INJECTED)
    with pytest.raises(G.GossmxError):
        layer.forward(x)
    try:
        ctx.inject_fault(G.FAULT_DEVICE)
        with pytest.raises(G.GossmxError):
            layer.forward(x)
        assert G.stats()["circuit_open"] == 1
        with pytest.raises(G.GossmxError) as e:
            layer.forward_device(dx, m, dout)
        assert e.value.status == G.ERR_CIRCUIT_OPEN
    finally:
        G.circuit_reset()
    bad = x.copy()
    bad[0, 3] = 0x7F80
    with pytest.raises(G.GossmxError):
        layer.forward(bad, injected_logits=np.zeros((m, E), np.float32))
    d = delta(s2, G.stats())
    assert (d["projections_rejected"], d["projections_failed"], d["projections_refused"], d["projections_ok"]) == \
        (2, 2, 1, 0), d
    assert G.stats()["circuit_open"] == 0
    ctx.free(dx)
    ctx.free(dout)
    close(layer)


def test_stats_reset_keeps_residency(ctx):
    host = O.synthetic_layer(24, 0, experts=2, hidden=64, intermediate=32, top_k=1)
    w = G.Weights.upload(ctx, host.gate_up, 2, 64, 2)
    held = G.stats()["resident_bytes"]
    G.stats_reset()
    s = G.stats()
    assert s["resident_bytes"] == held and s["resident_high_water_bytes"] == held
    assert s["projections_ok"] == 0 and s["weights_bias_uploaded_bytes"] == 0
    w.close()
    assert G.stats()["resident_high_water_bytes"] == held


@pytest.mark.parametrize("m", [1, 4, 40, 200])
def test_profile_events_per_stage(ctx, m):
    """One record per timed stage, with the call's shape, the stage's role and
    kernel family and the caller's tag; the records' durations add up to the
    per-operation totals."""
    E, H, I, K = 8, 128, 96, 4
    host = O.synthetic_layer(25, 0, experts=E, hidden=H, intermediate=I, top_k=K)
    layer = gpu_layer(ctx, host)
    x = O.gen_hidden(25, 1, m, H)
    ctx.profile(True)
    ctx.profile_reset()
    ctx.profile_tag(7, G.PHASE_PREFILL)
    try:
        for _ in range(2):
            layer.forward(x)
        ctx.profile_tag()
        layer.forward(x)
        events, dropped = ctx.profile_events()
        totals = ctx.profile_read()
    finally:
        ctx.profile(False)
    assert dropped == 0
    assert [e["sequence"] for e in events] == list(range(len(events)))
    per_call = len(events) // 3
    assert len(events) == 3 * per_call and per_call >= 3
    starts = [e["start_ns"] for e in events]
    assert starts[0] == 0 and all(a <= b for a, b in zip(starts, starts[1:]))
    for i, e in enumerate(events):
        assert e["m"] == m and e["routes"] == m * K and e["memory"] == "host"
        assert (e["layer"], e["phase"]) == ((7, "prefill") if i < 2 * per_call else (-1, "unknown"))
        assert e["resident_bytes"] > 0 and e["scratch_bytes"] > 0
        if e["op"] == "gate_up":
            assert (e["role"], e["n"], e["k"]) == ("gate_up", 2 * I, H)
        elif e["op"] == "down":
            assert (e["role"], e["n"], e["k"]) == ("down", H, I)
        elif e["op"] == "router_routing":
            assert (e["role"], e["kernel"], e["n"], e["k"]) == ("router", "route", E, H)
        elif e["op"] == "weighting":
            assert (e["kernel"], e["n"]) == ("combine", H)
        if e["kernel"] == "gemm":
            assert e["rows_per_item"] in (8, 16, 32)
        else:
            assert e["rows_per_item"] == 0
    kernels = {e["op"]: e["kernel"] for e in events}
    assert kernels["gate_up"] == ("gemv" if m <= 4 else "gemm")
    for op, tot in totals.items():
        mine = [e for e in events if e["op"] == op]
        assert len(mine) == tot["launches"], op
        if mine:
            assert sum(e["duration_ns"] for e in mine) == pytest.approx(tot["total_ms"] * 1e6, rel=1e-3, abs=64)
    # reading does not consume; a reset clears
    again, _ = ctx.profile_events()
    assert again == events
    ctx.profile_reset()
    assert ctx.profile_events() == ([], 0)
    close(layer)


def test_profile_events_drop_past_the_capacity(ctx):
    """One-row device calls make 3 records each; past GOSSMX_PROFILE_CAPACITY
    records the totals still count, the extra stages are dropped."""
    E, H, I, K = 4, 64, 32, 2
    host = O.synthetic_layer(26, 0, experts=E, hidden=H, intermediate=I, top_k=K)
    layer = gpu_layer(ctx, host)
    x = O.gen_hidden(26, 1, 1, H)
    dx, dout = ctx.malloc(x.nbytes), ctx.malloc(H * 4)
    ctx.h2d(dx, x)
    calls = G.PROFILE_CAPACITY // 3 + 10
    ctx.profile(True)
    ctx.profile_reset()
    try:
        for i in range(calls):
            layer.forward_device(dx, 1, dout)
            if i % 4096 == 4095:
                ctx.profile_events(0)  # folds the pending events
        ctx.synchronize()
        totals = ctx.profile_read()
        events, dropped = ctx.profile_events(capacity=4)
        _, avail_dropped = ctx.profile_events(capacity=0)
    finally:
        ctx.profile(False)
        ctx.profile_reset()
    launches = sum(t["launches"] for t in totals.values())
    assert launches == 3 * calls
    assert dropped == launches - G.PROFILE_CAPACITY == avail_dropped
    assert len(events) == 4 and events[0]["sequence"] == 0
    ctx.free(dx)
    ctx.free(dout)
    close(layer)
