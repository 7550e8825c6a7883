"""GPU parity of the MoE block (gossmx_moe_forward) against the oracle's
moe_batch (cpu_runner.rs:2794-3013): router logits, expert indices, routing
order, routing weights and output, all bit-exact; plus error paths and the
full-size properties (row independence) at the benchmark shapes."""
import os

import numpy as np
import pytest

import gossmx as G
import oracle as O
import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = G.Context(0)
    yield c
    c.close()


def gpu_layer(ctx, host: O.MoeLayerHost, projection: int = G.PROJECTION_RESIDUAL_Q8):
    E, H, I = host.experts, host.hidden, host.intermediate
    gu = G.Weights.upload(ctx, host.gate_up, E, 2 * I, H // 32)
    dn = G.Weights.upload(ctx, host.down, E, H, I // 32)
    return G.MoeLayer(ctx, E, H, I, host.top_k, host.router_weight, host.router_bias, gu, host.gate_up_bias, dn,
                      host.down_bias, host.alpha, host.limit, projection)


def assert_traces_equal(got, want):
    """CpuExpertTrace vectors of every (row, rank): gate_up, SwiGLU, down."""
    for gk, wk in (("trace_gate_up", "gate_up"), ("trace_swiglu", "swiglu"), ("trace_down", "down")):
        g, w = got[gk].view(np.uint32), want[wk].view(np.uint32)
        assert (g == w).all(), f"{gk}: {int((g != w).sum())} mismatches, first {np.argwhere(g != w)[:3].tolist()}"


def close(layer):
    layer.close()
    layer.gate_up.close()
    layer.down.close()


def assert_moe_equal(got, want):
    for key in ("router_logits", "routing_weights", "output"):
        g = np.ascontiguousarray(got[key], np.float32).view(np.uint32)
        w = np.ascontiguousarray(want[key], np.float32).view(np.uint32)
        bad = np.argwhere(g != w)
        assert bad.size == 0, f"{key}: {len(bad)} mismatches, first {bad[:3].tolist()}"
    assert (got["selected"] == want["selected"]).all(), "expert indices differ"
    assert (got["route_order"] == want["route_order"]).all(), "routing order differs"


@pytest.mark.parametrize("experts,hidden,inter,top_k,m", [(3, 64, 32, 2, 2), (4, 96, 64, 2, 5), (8, 128, 96, 4, 17),
                                                           (32, 256, 128, 4, 70), (3, 64, 32, 2, 1),
                                                           (8, 160, 96, 4, 1), (6, 96, 320, 3, 1)])
def test_small_layers_bit_exact(ctx, experts, hidden, inter, top_k, m):
    host = O.synthetic_layer(11, 0, experts=experts, hidden=hidden, intermediate=inter, top_k=top_k)
    x = O.gen_hidden(11, 100, m, hidden)
    want = O.moe_batch(host, x, trace=True)
    assert want["status"] == O.OK
    layer = gpu_layer(ctx, host)
    got = layer.forward(x, trace=True)
    assert_moe_equal(got, want)
    assert (got["trace_down"].view(np.uint32) == want["down"].view(np.uint32)).all()
    close(layer)


PROJECTIONS = [G.PROJECTION_RESIDUAL_Q8, G.PROJECTION_Q8, G.PROJECTION_EXACT_BF16]


@pytest.mark.parametrize("projection", PROJECTIONS, ids=["residual-q8", "q8", "exact-bf16"])
@pytest.mark.parametrize("experts,hidden,inter,top_k,m,inject", [(4, 96, 64, 2, 5, False), (8, 128, 96, 4, 17, True),
                                                                  (32, 256, 128, 4, 70, False),
                                                                  (32, 64, 64, 4, 600, True),
                                                                  (8, 128, 96, 4, 1, False), (5, 96, 64, 3, 1, True)])
def test_projection_modes_bit_exact_with_traces(ctx, projection, experts, hidden, inter, top_k, m, inject):
    """Every CpuExpertProjection (cpu_runner.rs:49-90) against the oracle's
    moe_batch in the same mode: outputs, routing and the gate_up / SwiGLU /
    down traces bit for bit. m = 600 takes the 32-row work items."""
    host = O.synthetic_layer(17, 0, experts=experts, hidden=hidden, intermediate=inter, top_k=top_k)
    x = O.gen_hidden(17, 100 + m, m, hidden)
    logits = None
    if inject:
        logits = O.bf16_round_array(np.random.default_rng(m).standard_normal((m, experts)).astype(np.float32))
    want = O.moe_batch(host, x, injected_logits=logits, trace=True, projection=projection)
    assert want["status"] == O.OK
    layer = gpu_layer(ctx, host, projection)
    got = layer.forward(x, injected_logits=logits, trace=True)
    assert_moe_equal(got, want)
    assert_traces_equal(got, want)
    close(layer)


@pytest.mark.parametrize("projection", [G.PROJECTION_Q8, G.PROJECTION_EXACT_BF16], ids=["q8", "exact-bf16"])
def test_projection_modes_20b_shape(ctx, projection):
    host = O.synthetic_layer(2026, 0)
    x = O.gen_hidden(2026, 5, 3, 2880)
    want = O.moe_batch(host, x, trace=True, projection=projection)
    assert want["status"] == O.OK
    layer = gpu_layer(ctx, host, projection)
    got = layer.forward(x, trace=True)
    assert_moe_equal(got, want)
    assert_traces_equal(got, want)
    close(layer)


def test_exact_bf16_sums_in_sixteen_ordered_lanes(ctx):
    """The oracle's exact-BF16 lane pin (test_oracle.exact_pin_layer): gate_up
    row 0 of expert 0 is 15 in the 16-lane order, where a sequential sum
    gives 0; the GPU's trace and outputs equal the oracle's bits."""
    from test_oracle import exact_pin_layer
    host, x, logits = exact_pin_layer()
    want = O.moe_batch(host, x, injected_logits=logits, trace=True, projection=O.PROJECTION_EXACT_BF16)
    assert want["status"] == O.OK and want["gate_up"][0, 0, 0] == 15.0
    layer = gpu_layer(ctx, host, G.PROJECTION_EXACT_BF16)
    got = layer.forward(x, injected_logits=logits, trace=True)
    assert got["trace_gate_up"][0, 0, 0] == 15.0
    assert_moe_equal(got, want)
    assert_traces_equal(got, want)
    close(layer)


def test_unknown_projection_is_rejected(ctx):
    host = O.synthetic_layer(3, 0, experts=2, hidden=64, intermediate=32, top_k=1)
    with pytest.raises(G.GossmxError) as e:
        gpu_layer(ctx, host, 3)
    assert e.value.status == G.ERR_INVALID_ARGUMENT


@pytest.fixture(scope="module")
def layer20b(ctx):
    host = O.synthetic_layer(2024, 0)
    layer = gpu_layer(ctx, host)
    yield host, layer
    close(layer)


@pytest.mark.parametrize("m", [1, 3])
def test_20b_shape_decode_bit_exact(layer20b, m):
    host, layer = layer20b
    x = O.gen_hidden(2024, 200 + m, m, 2880)
    want = O.moe_batch(host, x)
    assert want["status"] == O.OK
    assert_moe_equal(layer.forward(x), want)


@pytest.mark.parametrize("trace", [False, True], ids=["select-in-gate_up", "one-launch"])
@pytest.mark.parametrize("experts,m", [(32, 1), (128, 1), (128, 4), (5, 4), (17, 3)])
def test_small_batch_routing_bit_exact_and_repeatable(ctx, experts, m, trace):
    """Batches of at most 4 rows with a computed router. One row without
    traces: a logits launch, then every gate_up work-group selects for
    itself. Two to four rows, or the gate_up / SwiGLU traces requested: one
    launch for the router, selection and dispatch (one work-group per expert,
    the last to arrive selects). Three calls in a row, alternating with a
    9-row batch (two-launch path), all equal the oracle: the arrival counter
    resets."""
    host = O.synthetic_layer(31, experts, experts=experts, hidden=256, intermediate=64, top_k=4)
    layer = gpu_layer(ctx, host)
    x = O.gen_hidden(31, m, m, 256)
    x9 = O.gen_hidden(31, 9, 9, 256)
    want, want9 = O.moe_batch(host, x, trace=trace), O.moe_batch(host, x9)
    for _ in range(3):
        got = layer.forward(x, trace=trace)
        assert_moe_equal(got, want)
        if trace:
            assert_traces_equal(got, want)
        assert_moe_equal(layer.forward(x9), want9)
    close(layer)


@pytest.mark.parametrize("trace", [False, True], ids=["select-in-gate_up", "one-launch"])
@pytest.mark.parametrize("experts,top_k", [(40, 4), (7, 3), (100, 1), (128, 2)])
def test_small_batch_routing_ties_and_signed_zeros(ctx, experts, top_k, trace):
    """Router weights of zero make every logit its bias: tied biases and
    -0.0 / +0.0 force the ranked selection's tie rule (lower index first,
    -0.0 equal to +0.0) for batches of 1..4 rows, on both small-batch routing
    paths, against the oracle."""
    host = O.synthetic_layer(33, experts, experts=experts, hidden=128, intermediate=64, top_k=top_k)
    host.router_weight[:] = 0
    rng = np.random.default_rng(experts)
    bias = rng.choice(np.array([0.5, 0.25, -0.0, 0.0, -0.25], np.float32), experts)
    bias[[1, experts - 2]] = 0.5  # ties at the top
    host.router_bias[:] = bias
    layer = gpu_layer(ctx, host)
    for m in (1, 2, 3, 4):
        x = O.gen_hidden(33, m, m, 128)
        want = O.moe_batch(host, x, trace=trace)
        assert want["status"] == O.OK
        got = layer.forward(x, trace=trace)
        assert_moe_equal(got, want)
        if trace:
            assert_traces_equal(got, want)
    close(layer)


@pytest.mark.parametrize("experts,hidden,top_k", [(32, 2880, 4), (5, 96, 2), (64, 352, 4), (65, 3072, 4),
                                                   (128, 160, 3)])
def test_one_row_selects_inside_the_gate_up_launch(ctx, experts, hidden, top_k):
    """One-row batches with a computed router (no gate_up traces) take a
    logits and quantization launch, then every gate_up work-group selects for
    itself, and work-group (0, 0) writes the routing outputs. Bit-exact
    against the oracle, repeated and alternating with a 2-row batch, with the
    RMSNorm in front, and with a non-finite input."""
    host = O.synthetic_layer(41, experts, experts=experts, hidden=hidden, intermediate=64, top_k=top_k)
    layer = gpu_layer(ctx, host)
    x = O.gen_hidden(41, hidden, 1, hidden)
    x2 = O.gen_hidden(41, hidden + 1, 2, hidden)
    want, want2 = O.moe_batch(host, x), O.moe_batch(host, x2)
    assert want["status"] == O.OK and want2["status"] == O.OK
    for _ in range(2):
        assert_moe_equal(layer.forward(x), want)
        assert_moe_equal(layer.forward(x2), want2)
    res = residual_stream(41, 1, hidden)
    w = norm_weights(41, hidden)
    want_r = O.moe_residual(host, res, w, 1e-5)
    assert want_r["status"] == O.OK
    assert_residual_equal(layer.forward_residual(res, w, 1e-5), want_r)
    bad = x.copy()
    bad[0, hidden - 1] = 0x7F80  # +inf bf16
    with pytest.raises(G.GossmxError) as e:
        layer.forward(bad)
    assert e.value.status == G.ERR_NON_FINITE_LOGITS
    assert O.moe_batch(host, bad)["status"] == O.NON_FINITE_LOGITS
    assert_moe_equal(layer.forward(x), want)
    close(layer)


CHECK_THREADS = min(16, os.cpu_count() or 1)


def assert_full_batch_equal(host, x, got, logits=None):
    """Every row of a full-size batch against the oracle, run on its fastest
    forced panel lane (bit-identical to the scalar matmul: the golden hashes
    pin every lane) over the host's cores."""
    want = O.moe_batch(host, x, injected_logits=logits, lane=O.fastest_lane(), threads=CHECK_THREADS)
    assert want["status"] == O.OK
    assert_moe_equal(got, want)


def test_20b_shape_zipf_batch64_all_rows(layer20b):
    """batch 64 with injected Zipf(1.1) logits, every row and the
    grouped order against the oracle."""
    host, layer = layer20b
    rng = np.random.default_rng(64)
    x = synth.hidden_rows(rng, 64)
    logits = synth.zipf_logits(rng, 64, 32)
    got = layer.forward(x, injected_logits=logits)
    assert_full_batch_equal(host, x, got, logits)


def test_prefill_2048_all_rows(layer20b):
    """2048 tokens, router computed, several 32-row work items
    per expert (GemmHuge, two-launch selection): every row."""
    host, layer = layer20b
    rng = np.random.default_rng(2048)
    x = synth.hidden_rows(rng, 2048)
    got = layer.forward(x)
    counts = np.bincount(got["selected"].ravel(), minlength=32)
    assert counts.sum() == 2048 * 4 and counts.max() > 64
    assert_full_batch_equal(host, x, got)


@pytest.mark.parametrize("experts,top_k,m,inject", [
    (8, 6, 5, False),     # top_k > 4: per-row route kernel + dispatch kernel
    (8, 6, 5, True),
    (128, 4, 3, False),   # 128 experts, fused selection + dispatch
    (128, 4, 3, True),
    (128, 4, 80, True),   # m * (experts + 1) > 8448: route + dispatch kernels
    (32, 4, 256, True),   # largest fused batch at 32 experts (256 * 33 = 8448)
    (32, 4, 257, True),   # first batch past it
    (32, 4, 257, False),
])
def test_routing_paths_bit_exact(ctx, experts, top_k, m, inject):
    """Both routing implementations (one work-group selecting and grouping
    every row, or a work-group per row then a grouping kernel) against the
    oracle, with coarse injected logits so that ties occur."""
    host = O.synthetic_layer(31, 0, experts=experts, hidden=64, intermediate=64, top_k=top_k)
    x = O.gen_hidden(31, 300 + m, m, 64)
    logits = None
    if inject:
        rng = np.random.default_rng(m)
        logits = (np.round(rng.standard_normal((m, experts)) * 4.0) / 4.0).astype(np.float32)
    want = O.moe_batch(host, x, injected_logits=logits)
    assert want["status"] == O.OK
    layer = gpu_layer(ctx, host)
    assert_moe_equal(layer.forward(x, injected_logits=logits), want)
    close(layer)


@pytest.fixture(scope="module")
def layer120b(ctx):
    host = O.synthetic_layer(120, 0, experts=128)
    layer = gpu_layer(ctx, host)
    yield host, layer
    close(layer)


def test_120b_shape_decode_bit_exact(layer120b):
    """configs[4] layer shape (128 experts, H = I = 2880), router computed."""
    host, layer = layer120b
    x = O.gen_hidden(120, 7, 2, 2880)
    want = O.moe_batch(host, x)
    assert want["status"] == O.OK
    assert_moe_equal(layer.forward(x), want)


def test_120b_shape_zipf_batch256_all_rows(layer120b):
    """configs[4] decode: batch 256 with injected Zipf(1.2) logits over 128
    experts, every row."""
    host, layer = layer120b
    rng = np.random.default_rng(256)
    x = synth.hidden_rows(rng, 256)
    logits = synth.zipf_logits(rng, 256, 128, 4, 1.2)
    got = layer.forward(x, injected_logits=logits)
    assert_full_batch_equal(host, x, got, logits)


def test_120b_shape_prefill_4096_uniform_all_rows(layer120b):
    """configs[4] prefill: 4096 tokens, near-uniform injected routing over
    128 experts (16,384 routes, about 128 per expert: GemmHuge and the
    two-launch selection with 64 selection work-groups), every row."""
    host, layer = layer120b
    rng = np.random.default_rng(4096)
    x = synth.hidden_rows(rng, 4096)
    logits = synth.uniform_logits(rng, 4096, 128)
    got = layer.forward(x, injected_logits=logits)
    counts = np.bincount(got["selected"].ravel(), minlength=128)
    assert counts.sum() == 4096 * 4 and counts.min() > 64
    assert_full_batch_equal(host, x, got, logits)


# --- order pins: inputs on which the plausible other float orders give other
# bits (test_oracle derives each expected value by hand and checks that the
# alternatives differ); each router and selection path is run by row count:
# one row (selection inside the gate_up launch), 2-4 rows (route_select_kernel
# with its arrival counter), more rows (route_kernel, then the selection
# kernels) and, with injected logits, the one-work-group and two-launch
# selections ---

@pytest.mark.parametrize("m", [1, 3, 8])
@pytest.mark.parametrize("hidden,offset", [(64, 0), (2880, 1424)])
def test_router_dot_order_pins(ctx, hidden, offset, m):
    """test_oracle's 16-lane router pin (scalar_bf16_dot, lib.rs:1007-1029):
    logits 15 and 0 on the pinned rows, where sequential, pairwise, tree-folded,
    reversed and other lane counts give 0, 14 or 16. At hidden 2880 the
    construction straddles the router kernels' staging chunks."""
    from test_oracle import router_pin_case
    w, bias, x = router_pin_case(hidden, offset)
    host = O.MoeLayerHost(w, bias, O.gen_mxfp4(1, 1, 4, 64, hidden // 32), np.zeros(4 * 64, np.float32),
                          O.gen_mxfp4(1, 2, 4, hidden, 1), np.zeros(4 * hidden, np.float32), 4, hidden, 32, 2)
    xs = np.repeat(x[None, :], m, axis=0)
    want = O.moe_batch(host, xs)
    assert want["status"] == O.OK
    layer = gpu_layer(ctx, host)
    got = layer.forward(xs)
    assert (got["router_logits"][:, :2] == [15.0, 0.0]).all()
    assert_moe_equal(got, want)
    close(layer)


def _softmax_pin_layer(router_bias=None):
    host = O.synthetic_layer(41, 0, experts=8, hidden=64, intermediate=32, top_k=4)
    if router_bias is not None:  # computed router: zero weights, so the logits are the bias
        host = O.MoeLayerHost(np.zeros_like(host.router_weight), router_bias, host.gate_up, host.gate_up_bias,
                              host.down, host.down_bias, 8, 64, 32, 4)
    return host


@pytest.mark.parametrize("repeat", [1, 300], ids=["one-work-group", "two-launch"])
def test_softmax_order_pins_injected(ctx, repeat):
    """Injected rows whose bf16 routing weights depend on the softmax
    denominator's rank order (test_oracle.SOFTMAX_PIN_ROWS,
    cpu_runner.rs:3784-3795): reversed, pairwise and float64 sums give other
    weights."""
    from test_oracle import SOFTMAX_PIN_ROWS
    rows = len(SOFTMAX_PIN_ROWS) * repeat
    logits = np.full((rows, 8), -20.0, np.float32)
    for r in range(rows):
        logits[r, [5, 1, 6, 2]] = SOFTMAX_PIN_ROWS[r % len(SOFTMAX_PIN_ROWS)]
    host = _softmax_pin_layer()
    x = O.gen_hidden(41, 1, rows, 64)
    want = O.moe_batch(host, x, injected_logits=logits)
    assert want["status"] == O.OK
    for r, row in enumerate(SOFTMAX_PIN_ROWS):
        assert (want["routing_weights"][r] == O.bf16_round_array(O.softmax(np.array(row, np.float32)))).all()
    layer = gpu_layer(ctx, host)
    got = layer.forward(x, injected_logits=logits)
    assert (got["selected"] == [[5, 1, 6, 2]] * rows).all()
    assert_moe_equal(got, want)
    close(layer)


@pytest.mark.parametrize("m", [1, 3, 8])
@pytest.mark.parametrize("pin", [0, 1])
def test_softmax_order_pins_computed_router(ctx, pin, m):
    """The same pin through a computed router (zero router weights, the pin
    row as the bias), on each router/selection path."""
    from test_oracle import SOFTMAX_PIN_ROWS
    bias = np.full(8, -20.0, np.float32)
    bias[[5, 1, 6, 2]] = SOFTMAX_PIN_ROWS[pin]
    host = _softmax_pin_layer(bias)
    x = O.gen_hidden(41, 2, m, 64)
    want = O.moe_batch(host, x)
    assert want["status"] == O.OK
    assert (want["routing_weights"] == O.bf16_round_array(O.softmax(np.array(SOFTMAX_PIN_ROWS[pin], np.float32)))).all()
    layer = gpu_layer(ctx, host)
    got = layer.forward(x)
    assert (got["selected"] == [[5, 1, 6, 2]] * m).all()
    assert_moe_equal(got, want)
    close(layer)


# Combine pin (cpu_runner.rs:2959-2999: weighted = y * w, the ranks added in
# rank order from 0.0, then bf16). Four equal logits give every rank the weight
# 0.25 (expf(0) = 1, 1/4) and rank k = expert k; all-zero down codes make each
# expert's down output its bias. Column 0 takes 4 * [1, 2^24, 1, -2^24]:
# weighted [1, 2^24, 1, -2^24], in rank order 1 + 2^24 ties to 2^24, + 1 ties
# to 2^24 again, - 2^24 = 0. Column 1 takes 4 * [2^24, 1, -2^24, 1]: 2^24 + 1
# ties to 2^24, - 2^24 = 0, + 1 = 1. Reversed order gives 2 on both columns,
# pairwise 1 on both (2^24 + 1 ties down, 1 - 2^24 is exact), float64 2 on
# both: every alternative differs on column 0.
B24 = float(2 ** 24)
COMBINE_PIN = {0: ([1.0, B24, 1.0, -B24], 0.0), 1: ([B24, 1.0, -B24, 1.0], 1.0)}


def _combine_pin_layer():
    host = O.synthetic_layer(43, 0, experts=4, hidden=64, intermediate=32, top_k=4)
    down = np.zeros((4, 64, 1, 17), np.uint8)
    down[..., 0] = 127  # E8M0 scale 1.0, every code 0 (value 0.0)
    down_bias = host.down_bias.copy().reshape(4, 64)
    for col, (weighted, _) in COMBINE_PIN.items():
        down_bias[:, col] = [4.0 * v for v in weighted]
    return O.MoeLayerHost(np.zeros_like(host.router_weight), np.zeros(4, np.float32), host.gate_up,
                          host.gate_up_bias, down.ravel(), down_bias.ravel(), 4, 64, 32, 4)


@pytest.mark.parametrize("inject", [False, True], ids=["computed", "injected"])
@pytest.mark.parametrize("m", [1, 3, 70])
def test_combine_order_pins(ctx, m, inject):
    from test_oracle import _fold
    F = np.float32
    alternatives = {"reversed": lambda p: _fold(p[::-1], 0.0),
                    "pairwise": lambda p: F(F(p[0] + p[1]) + F(p[2] + p[3])),
                    "float64": lambda p: F(np.sum(np.asarray(p, np.float64)))}
    for col, (weighted, expected) in COMBINE_PIN.items():
        assert _fold(weighted, 0.0) == expected
    for name, fn in alternatives.items():
        assert any(fn(w) != e for w, e in COMBINE_PIN.values()), name
    host = _combine_pin_layer()
    x = O.gen_hidden(43, 1, m, 64)
    logits = np.zeros((m, 4), np.float32) if inject else None
    want = O.moe_batch(host, x, injected_logits=logits)
    assert want["status"] == O.OK
    layer = gpu_layer(ctx, host)
    got = layer.forward(x, injected_logits=logits)
    assert (got["selected"] == [[0, 1, 2, 3]] * m).all() and (got["routing_weights"] == 0.25).all()
    for col, (_, expected) in COMBINE_PIN.items():
        assert (got["output"][:, col] == expected).all(), col
    assert_moe_equal(got, want)
    close(layer)


@pytest.mark.parametrize("experts,hidden,inter,top_k,m,projection", [
    (8, 128, 96, 4, 1, G.PROJECTION_RESIDUAL_Q8),    # one row: the combine inside the down launch
    (8, 128, 96, 4, 5, G.PROJECTION_RESIDUAL_Q8),    # combine8_kernel
    (32, 256, 128, 4, 70, G.PROJECTION_RESIDUAL_Q8),
    (4, 96, 64, 2, 3, G.PROJECTION_EXACT_BF16)])
def test_output_unrounded_matches_oracle(ctx, experts, hidden, inter, top_k, m, projection):
    """output_unrounded: the rank-order weighted sum before its bf16 round trip
    (cpu_runner.rs:2991) equals the oracle's on every path, and rounds to
    the output."""
    host = O.synthetic_layer(47, 0, experts=experts, hidden=hidden, intermediate=inter, top_k=top_k)
    x = O.gen_hidden(47, m, m, hidden)
    want = O.moe_batch(host, x, projection=projection)
    assert want["status"] == O.OK
    layer = gpu_layer(ctx, host, projection)
    got = layer.forward(x, unrounded=True)
    assert_moe_equal(got, want)
    assert (got["output_unrounded"].view(np.uint32) == want["output_unrounded"].view(np.uint32)).all()
    assert (O.bf16_round_array(got["output_unrounded"]).view(np.uint32) == got["output"].view(np.uint32)).all()
    # device memory, the pre-round output at a 4-byte offset: the scalar combine_kernel
    if m > 1:
        dx, dout, dunr = ctx.malloc(x.nbytes), ctx.malloc(m * hidden * 4), ctx.malloc(m * hidden * 4 + 16)
        ctx.h2d(dx, x)
        layer.forward_device(dx, m, dout, output_unrounded=dunr + 4)
        ctx.synchronize()
        unr = np.empty((m, hidden), np.float32)
        out = np.empty((m, hidden), np.float32)
        ctx.d2h(unr, dunr + 4)
        ctx.d2h(out, dout)
        assert (unr.view(np.uint32) == want["output_unrounded"].view(np.uint32)).all()
        assert (out.view(np.uint32) == want["output"].view(np.uint32)).all()
        for p in (dx, dout, dunr):
            ctx.free(p)
    close(layer)


@pytest.mark.parametrize("experts,hidden,inter,top_k,m,projection", [
    (8, 128, 96, 4, 1, G.PROJECTION_RESIDUAL_Q8),
    (8, 128, 96, 4, 5, G.PROJECTION_RESIDUAL_Q8),
    (32, 256, 128, 4, 40, G.PROJECTION_RESIDUAL_Q8),
    (4, 96, 64, 2, 3, G.PROJECTION_EXACT_BF16)])
def test_host_memory_every_output_in_one_call(ctx, experts, hidden, inter, top_k, m, projection):
    """A host-memory call that asks for every output at once (routing, the
    rows, the three traces and the pre-round output: nine pieces of the
    pinned output pack, some of them not multiples of 16 bytes) returns each
    bit for bit as the oracle's, and leaves the bytes around the caller's
    buffers untouched."""
    host = O.synthetic_layer(53, 0, experts=experts, hidden=hidden, intermediate=inter, top_k=top_k)
    x = O.gen_hidden(53, m, m, hidden)
    want = O.moe_batch(host, x, trace=True, projection=projection)
    assert want["status"] == O.OK
    layer = gpu_layer(ctx, host, projection)
    got = layer.forward(x, trace=True, unrounded=True)
    assert_moe_equal(got, want)
    assert_traces_equal(got, want)
    assert (got["output_unrounded"].view(np.uint32) == want["output_unrounded"].view(np.uint32)).all()
    # the same call through the C ABI into canaried buffers
    E, K, H, I = experts, top_k, hidden, inter
    lib = G.load()
    shapes = {"router_logits": (m * E, np.float32), "selected": (m * K, np.uint32),
              "routing_weights": (m * K, np.float32), "output": (m * H, np.float32),
              "route_order": (m * K, np.uint32), "trace_down": (m * K * H, np.float32),
              "trace_gate_up": (m * K * 2 * I, np.float32), "trace_swiglu": (m * K * I, np.float32),
              "output_unrounded": (m * H, np.float32)}
    canary = 0x5A5A5A5A
    bufs = {k: np.full(n + 2, canary, np.uint32).view(dt) for k, (n, dt) in shapes.items()}
    inner = {k: b[1:-1] for k, b in bufs.items()}
    io = G.MoeIo(G._ptr(x), m, None, G._ptr(inner["router_logits"]), G._ptr(inner["selected"]),
                 G._ptr(inner["routing_weights"]), G._ptr(inner["output"]), G._ptr(inner["route_order"]),
                 G._ptr(inner["trace_down"]), G.MEM_HOST, G._ptr(inner["trace_gate_up"]),
                 G._ptr(inner["trace_swiglu"]), G._ptr(inner["output_unrounded"]))
    assert lib.gossmx_moe_forward(ctx.handle, layer._h, G.C.byref(io)) == G.OK
    for k, b in bufs.items():
        raw = b.view(np.uint32)
        assert raw[0] == canary and raw[-1] == canary, k
        assert (inner[k].view(np.uint32) == got[k].reshape(-1).view(np.uint32)).all(), k
    close(layer)


def forced_route_logits(counts, m, top_k):
    """Injected logits whose top-k gives expert e exactly counts[e] routes:
    each row takes the top_k experts with the most routes still to place
    (ties by index; a valid assignment while no count exceeds the rows left),
    ranked by descending logits 4, 3, 2, ... (bf16-exact); the other experts
    get -4."""
    E = len(counts)
    need = np.array(counts, np.int64)
    assert need.sum() == m * top_k and need.max() <= m
    logits = np.full((m, E), -4.0, np.float32)
    for r in range(m):
        order = sorted(range(E), key=lambda e: (-need[e], e))[:top_k]
        assert all(need[e] > 0 for e in order), "counts cannot be placed"
        for rank, e in enumerate(order):
            logits[r, e] = float(4 - rank)
            need[e] -= 1
    return logits


@pytest.mark.parametrize("m,counts", [
    (8, [8, 7, 1, 4, 4, 4, 3, 1]),                                      # 8-row items: a full bucket of 8
    (9, [9, 9, 8, 6, 2, 1, 1, 0]),                                      # first 16-row-item batch: 8, 9 rows
    (48, [16, 17, 8, 9, 15, 1, 7, 32, 33, 24, 0, 2, 3, 4, 5, 16]),      # 16-row items: 16, 17, 32, 33 rows
    (512, [32, 33, 31, 64, 65, 63, 96, 97, 1, 8, 9, 16, 17, 24, 25, 40] + [89] * 15 + [92])])      # 32-row items
def test_bucket_sizes_at_item_and_token_group_boundaries(ctx, m, counts):
    """Expert buckets of exactly 8k and 8k + 1 rows and of exactly one chunk
    and one chunk + 1 (every geometry's item size: 8, 16 and 32 rows), so
    that full items, one-row partial items and single-token-group tails all
    occur; bit for bit against the oracle."""
    E = len(counts)
    host = O.synthetic_layer(59, 0, experts=E, hidden=128, intermediate=96, top_k=4)
    x = O.gen_hidden(59, m, m, 128)
    logits = forced_route_logits(counts, m, 4)
    want = O.moe_batch(host, x, injected_logits=logits)
    assert want["status"] == O.OK
    assert (np.bincount(want["selected"].reshape(-1), minlength=E) == np.array(counts)).all()
    layer = gpu_layer(ctx, host)
    got = layer.forward(x, injected_logits=logits)
    assert_moe_equal(got, want)
    close(layer)


def test_all_experts_selected(ctx):
    host = O.synthetic_layer(5, 0, experts=4, hidden=64, intermediate=64, top_k=4)
    x = O.gen_hidden(5, 1, 9, 64)
    want = O.moe_batch(host, x)
    layer = gpu_layer(ctx, host)
    assert_moe_equal(layer.forward(x), want)
    close(layer)


def test_tied_logits_route_to_lower_index(ctx):
    host = O.synthetic_layer(6, 0, experts=8, hidden=64, intermediate=32, top_k=4)
    x = O.gen_hidden(6, 1, 3, 64)
    logits = np.zeros((3, 8), np.float32)
    logits[0, [1, 5, 6]] = 1.0
    logits[1] = -0.0
    logits[2, 7] = 2.0
    logits[2, 3] = 2.0
    want = O.moe_batch(host, x, injected_logits=logits)
    layer = gpu_layer(ctx, host)
    got = layer.forward(x, injected_logits=logits)
    assert_moe_equal(got, want)
    assert got["selected"][0].tolist() == [1, 5, 6, 0]
    assert got["selected"][1].tolist() == [0, 1, 2, 3]
    close(layer)


def test_non_finite_logits_and_inputs_fail(ctx):
    host = O.synthetic_layer(7, 0, experts=4, hidden=64, intermediate=32, top_k=2)
    layer = gpu_layer(ctx, host)
    x = O.gen_hidden(7, 1, 2, 64)
    logits = np.zeros((2, 4), np.float32)
    logits[1, 2] = np.inf
    with pytest.raises(G.GossmxError) as e:
        layer.forward(x, injected_logits=logits)
    assert e.value.status == G.ERR_NON_FINITE_LOGITS
    assert O.moe_batch(host, x, injected_logits=logits)["status"] == O.NON_FINITE_LOGITS
    bad = x.copy()
    bad[0, 5] = 0x7F80  # +inf bf16: the router logits become non-finite first
    with pytest.raises(G.GossmxError) as e:
        layer.forward(bad)
    assert e.value.status == G.ERR_NON_FINITE_LOGITS
    with pytest.raises(G.GossmxError) as e:  # injected finite logits: the quantizer rejects the input
        layer.forward(bad, injected_logits=np.zeros((2, 4), np.float32))
    assert e.value.status == G.ERR_NON_FINITE_INPUT
    # the context recovers
    want = O.moe_batch(host, x)
    assert_moe_equal(layer.forward(x), want)
    close(layer)


def test_injected_fault_leaves_outputs_untouched(ctx):
    host = O.synthetic_layer(8, 0, experts=4, hidden=64, intermediate=32, top_k=2)
    layer = gpu_layer(ctx, host)
    x = O.gen_hidden(8, 1, 2, 64)
    ctx.inject_fault(True)
    with pytest.raises(G.GossmxError) as e:
        layer.forward(x)
    assert e.value.status == G.ERR_INJECTED_FAULT
    assert_moe_equal(layer.forward(x), O.moe_batch(host, x))
    close(layer)


def test_device_fault_opens_the_circuit_breaker(ctx):
    """A run-time fault (the injected device fault) fails the call with
    GOSSMX_ERR_DEVICE and opens the process-wide breaker; while it is open
    projection calls still validate their arguments, then return
    GOSSMX_ERR_CIRCUIT_OPEN; after the reset the block runs again and matches
    the oracle (XeProjectionEngine::execute_projection,
    crates/gpt-oss-xe/src/lib.rs:680-724)."""
    host = O.synthetic_layer(8, 1, experts=4, hidden=64, intermediate=32, top_k=2)
    layer = gpu_layer(ctx, host)
    x = O.gen_hidden(8, 2, 2, 64)
    want = O.moe_batch(host, x)
    try:
        assert not G.circuit_is_open()
        ctx.inject_fault(G.FAULT_DEVICE)
        with pytest.raises(G.GossmxError) as e:
            layer.forward(x)
        assert e.value.status == G.ERR_DEVICE
        assert G.circuit_is_open()
        with pytest.raises(G.GossmxError) as e:
            layer.forward(x)
        assert e.value.status == G.ERR_CIRCUIT_OPEN
        with pytest.raises(G.GossmxError) as e:  # argument checks come first
            layer.forward(x[:0])
        assert e.value.status == G.ERR_INVALID_DIMENSIONS
        rec = np.zeros(2 * 2, G.RQ8_DTYPE)
        with pytest.raises(G.GossmxError) as e:
            G.mxfp4_matmul(ctx, layer.down, 0, rec, 2, None, np.zeros((2, 64), np.float32))
        assert e.value.status == G.ERR_CIRCUIT_OPEN
        assert G.circuit_is_open()
    finally:
        G.circuit_reset()
    assert not G.circuit_is_open()
    assert_moe_equal(layer.forward(x), want)
    # a model-error fault (mode 1) leaves the breaker closed
    ctx.inject_fault(G.FAULT_INJECTED)
    with pytest.raises(G.GossmxError) as e:
        layer.forward(x)
    assert e.value.status == G.ERR_INJECTED_FAULT
    assert not G.circuit_is_open()
    # a device error flag raised during the call (mode 3): a host-memory call
    # reports it itself, a device-memory call at gossmx_synchronize; both open
    # the breaker, and the flag is cleared once reported
    dx, dout = ctx.malloc(x.nbytes), ctx.malloc(2 * 64 * 4)
    ctx.h2d(dx, x)
    try:
        ctx.inject_fault(G.FAULT_FLAG)
        with pytest.raises(G.GossmxError) as e:
            layer.forward(x)
        assert e.value.status == G.ERR_DEVICE
        assert G.circuit_is_open()
        G.circuit_reset()
        ctx.inject_fault(G.FAULT_FLAG)
        layer.forward_device(dx, 2, dout)
        with pytest.raises(G.GossmxError) as e:
            ctx.synchronize()
        assert e.value.status == G.ERR_DEVICE
        assert G.circuit_is_open()
    finally:
        G.circuit_reset()
    layer.forward_device(dx, 2, dout)
    ctx.synchronize()
    got = np.empty((2, 64), np.float32)
    ctx.d2h(got, dout)
    assert (got.view(np.uint32) == want["output"].view(np.uint32)).all()
    ctx.free(dx)
    ctx.free(dout)
    assert_moe_equal(layer.forward(x), want)
    close(layer)


def test_scratch_requirement_is_none_and_selftest_passes(ctx):
    host = O.synthetic_layer(8, 2, experts=2, hidden=64, intermediate=32, top_k=1)
    layer = gpu_layer(ctx, host)
    assert G.scratch_requirement(layer.gate_up, 5) == (0, 1)
    assert G.scratch_requirement(layer.down, 1, G.ACT_Q8) == (0, 1)
    with pytest.raises(G.GossmxError) as e:
        G.scratch_requirement(layer.down, 0)
    assert e.value.status == G.ERR_INVALID_DIMENSIONS
    ctx.selftest()  # lane layouts, dirty scale operands, sigmoid table
    assert ctx.fast_path()
    close(layer)


def test_bf16_rounding_matches_half_on_every_f32(ctx):
    # The kernels' f32 -> bf16 rounding (gfx950's conversion instruction)
    # against half 2.7.1's from_f32 restated in integer operations, on all
    # 2^32 f32 bit patterns: nearest even, NaN quieted with sign and payload.
    assert ctx.bf16_exhaustive_mismatches() == 0


def test_profiler_counts_every_stage(ctx):
    """Every stage is timed once per call. Batches of at most 4 rows with a
    computed router run the router, selection and dispatch as one launch,
    counted under router_routing (dispatch then has no launch of its own);
    one-row batches launch the router for the logits only, select inside the
    gate_up launch and run the combine inside the down launch (weighting has
    none)."""
    host = O.synthetic_layer(9, 0, experts=4, hidden=64, intermediate=32, top_k=2)
    layer = gpu_layer(ctx, host)
    for m, fused in ((12, False), (4, True), (1, True)):
        x = O.gen_hidden(9, 1, m, 64)
        ctx.profile(True)
        ctx.profile_reset()
        for _ in range(3):
            layer.forward(x)
        rec = ctx.profile_read()
        ctx.profile(False)
        for op in ("router_routing", "dispatch", "gate_up", "down", "weighting"):
            if (fused and op == "dispatch") or (m == 1 and op == "weighting"):
                assert rec[op]["launches"] == 0, (m, op)
            else:
                assert rec[op]["launches"] == 3 and rec[op]["total_ms"] > 0.0, (m, op)
    close(layer)


def residual_stream(seed: int, m: int, hidden: int) -> np.ndarray:
    """A post-attention residual stream: bf16 rows of N(0, 6^2), not normalized."""
    return O.gen_bf16_normal(seed, 500 + m, m * hidden, 0.0, 6.0).reshape(m, hidden)


def norm_weights(seed: int, hidden: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return (1.0 + 0.25 * rng.standard_normal(hidden)).astype(np.float32)


def assert_residual_equal(got, want, rows=None):
    sel = slice(None) if rows is None else rows
    for key in ("router_logits", "routing_weights", "output"):
        if key not in got:
            continue
        g = np.ascontiguousarray(got[key][sel], np.float32).view(np.uint32)
        w = np.ascontiguousarray(want[key], np.float32).view(np.uint32)
        assert (g == w).all(), f"{key}: {int((g != w).sum())} mismatches"
    assert (got["selected"][sel] == want["selected"]).all()
    g = got["next_residual"][sel]
    w = want["next_residual"]
    assert (g == w).all(), f"next_residual: {int((g != w).sum())} mismatches, first {np.argwhere(g != w)[:3].tolist()}"


@pytest.mark.parametrize("inject", [False, True])
@pytest.mark.parametrize("experts,hidden,inter,top_k,m", [(4, 96, 64, 2, 5), (8, 128, 96, 4, 17),
                                                           (32, 256, 128, 4, 70), (32, 64, 64, 4, 300)])
def test_residual_small_layers_bit_exact(ctx, experts, hidden, inter, top_k, m, inject):
    _residual_case(ctx, experts, hidden, inter, top_k, m, inject, G.PROJECTION_RESIDUAL_Q8)


@pytest.mark.parametrize("projection", [G.PROJECTION_Q8, G.PROJECTION_EXACT_BF16], ids=["q8", "exact-bf16"])
@pytest.mark.parametrize("inject", [False, True])
def test_residual_projection_modes(ctx, projection, inject):
    """The MoE half of the decoder layer in the Q8 and exact-BF16 modes (the
    exact mode reads the normalized rows the quantization work-groups store)."""
    _residual_case(ctx, 8, 128, 96, 4, 17, inject, projection)
    _residual_case(ctx, 32, 64, 64, 4, 300, inject, projection)


def _residual_case(ctx, experts, hidden, inter, top_k, m, inject, projection):
    """gossmx_moe_forward_residual = norm_boundary -> moe_batch -> add_residual
    (cpu_runner.rs:2519-2553) against the oracle, every output bit-exact. With
    injected logits the norm runs in the selection kernels' quantization
    work-groups, which at these hidden sizes span several rows each; m = 300
    with 32 experts takes the two-launch selection path."""
    host = O.synthetic_layer(13, 0, experts=experts, hidden=hidden, intermediate=inter, top_k=top_k)
    x = residual_stream(13, m, hidden)
    w = norm_weights(13, hidden)
    logits = None
    if inject:
        logits = O.bf16_round_array(np.random.default_rng(m).standard_normal((m, experts)).astype(np.float32))
    want = O.moe_residual(host, x, w, 1e-5, injected_logits=logits, projection=projection)
    assert want["status"] == O.OK
    layer = gpu_layer(ctx, host, projection)
    got = layer.forward_residual(x, w, 1e-5, injected_logits=logits)
    assert_residual_equal(got, want)
    assert (got["route_order"] == want["route_order"]).all()
    close(layer)


@pytest.mark.parametrize("m", [1, 3])
def test_residual_20b_shape_bit_exact(layer20b, m):
    host, layer = layer20b
    x = residual_stream(2024, m, 2880)
    w = norm_weights(2024, 2880)
    want = O.moe_residual(host, x, w, 1e-5)
    assert want["status"] == O.OK
    assert_residual_equal(layer.forward_residual(x, w, 1e-5), want)


def test_residual_20b_shape_batch64_rows_match(layer20b):
    """configs[1] shape with injected Zipf(1.1) logits; only next_residual
    requested (no f32 output); the oracle checks a sample of rows."""
    host, layer = layer20b
    rng = np.random.default_rng(65)
    x = residual_stream(65, 64, 2880)
    w = norm_weights(65, 2880)
    logits = synth.zipf_logits(rng, 64, 32)
    got = layer.forward_residual(x, w, 1e-5, injected_logits=logits, want_output=False)
    assert "output" not in got
    rows = [0, 31, 63]
    want = O.moe_residual(host, x[rows], w, 1e-5, injected_logits=logits[rows])
    assert_residual_equal(got, want, rows)


def test_residual_zero_row_and_plain_forward_agree(layer20b):
    """A zero residual row normalizes to zeros (sum 0: inverse 1/sqrt(eps));
    and gossmx_moe_forward on the oracle's normalized rows gives the same
    block outputs as the fused call."""
    host, layer = layer20b
    x = residual_stream(77, 3, 2880)
    x[1] = 0
    w = norm_weights(77, 2880)
    fused = layer.forward_residual(x, w, 1e-5)
    want = O.moe_residual(host, x, w, 1e-5)
    assert_residual_equal(fused, want)
    plain = layer.forward(want["normalized"])
    for key in ("router_logits", "routing_weights", "output"):
        assert (plain[key].view(np.uint32) == fused[key].view(np.uint32)).all(), key
