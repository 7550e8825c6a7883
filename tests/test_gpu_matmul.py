"""GPU parity of the kernel boundary (gossmx_mxfp4_matmul) and the resident
weight layout against the CPU oracle: bit-exact output, golden hashes,
tails, special values, canaries and validation (matmul.rs:1049-1893 test
strategy)."""
import hashlib
import json
import os

import numpy as np
import pytest

import gossmx as G
import oracle as O

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "mxfp4_matrix_hashes.json")


@pytest.fixture(scope="module")
def ctx():
    c = G.Context(0)
    yield c
    c.close()


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def assert_same_bits(got, want):
    g, w = bits(got), bits(want)
    nan = np.isnan(np.asarray(want, np.float32))
    assert (np.isnan(np.asarray(got, np.float32)) == nan).all(), "NaN positions differ"
    bad = np.nonzero((g != w) & ~nan)[0]
    assert bad.size == 0, f"{bad.size} mismatches, first at {bad[:5]}: got {np.asarray(got).ravel()[bad[:5]]} " \
                          f"want {np.asarray(want).ravel()[bad[:5]]}"


def test_selftest_lane_layouts(ctx):
    ctx.selftest()


@pytest.mark.parametrize("layout", [G.LAYOUT_CANONICAL_V1, G.LAYOUT_X8_SPLIT_V2])
@pytest.mark.parametrize("rows,blocks", [(16, 1), (21, 5), (40, 3), (5760, 90)])
def test_upload_round_trips(ctx, layout, rows, blocks):
    experts = 2
    canonical = O.gen_mxfp4(5, 7, experts, rows, blocks)
    data = canonical
    if layout == G.LAYOUT_X8_SPLIT_V2:
        per = rows * blocks * 17
        data = np.concatenate([O.pack_x8(canonical[e * per:(e + 1) * per], rows, blocks) for e in range(experts)])
    w = G.Weights.upload(ctx, data, experts, rows, blocks, layout)
    assert (w.export_canonical() == canonical).all()
    w.close()


def test_device_generator_matches_host_generator(ctx):
    w = G.Weights.generate(ctx, 1234, 4, 3, 48, 7)
    assert (w.export_canonical() == O.gen_mxfp4(1234, 4, 3, 48, 7)).all()
    w.close()


def golden_cases():
    with open(GOLDEN) as fh:
        return json.load(fh)["cases"]


@pytest.mark.parametrize("case", golden_cases(), ids=lambda c: f"{c['role']}-m{c['m']}")
def test_golden_hashes_on_gpu(ctx, case):
    n, m = case["n"], case["m"]
    canonical, x8, res, bias = O.bench_fixtures(n, 90, m)
    w = G.Weights.upload(ctx, x8, 1, n, 90, G.LAYOUT_X8_SPLIT_V2)
    out = np.full(m * n, np.nan, np.float32)
    G.mxfp4_matmul(ctx, w, 0, res, m, bias, out)
    assert hashlib.sha256(out.tobytes()).hexdigest() == case["sha256"]
    w.close()


def random_records(rng, m, blocks, kind):
    if kind == G.ACT_Q8:
        a = np.zeros(m * blocks, O.Q8_DTYPE)
        a["scale"] = rng.uniform(0.0, 0.05, m * blocks).astype(np.float32)
        a["values"] = rng.integers(-127, 128, (m * blocks, 32))
        return a
    a = np.zeros(m * blocks, O.RQ8_DTYPE)
    for part, hi in (("primary", 0.05), ("residual", 0.0004)):
        a[part]["scale"] = rng.uniform(0.0, hi, m * blocks).astype(np.float32)
        a[part]["values"] = rng.integers(-127, 128, (m * blocks, 32))
    return a


@pytest.mark.parametrize("kind", [G.ACT_RESIDUAL_Q8, G.ACT_Q8])
# m <= 8, 8 < m < 512 and m >= 512 take the three GEMM geometries (8-, 16- and
# 32-row work items); 600 = 18 x 32 + 24 leaves a ragged last item.
@pytest.mark.parametrize("rows,blocks,m", [(1, 1, 1), (9, 5, 3), (17, 2, 9), (33, 7, 64), (70, 3, 65), (130, 4, 130),
                                            (5760, 90, 2), (2880, 90, 11), (48, 6, 600), (130, 5, 512)])
def test_matmul_bit_exact_tails(ctx, kind, rows, blocks, m):
    rng = np.random.default_rng(rows * 1000 + blocks * 10 + m)
    canonical = O.gen_mxfp4(rows, blocks, 1, rows, blocks)
    act = random_records(rng, m, blocks, kind)
    bias = (rng.standard_normal(rows) * 0.1).astype(np.float32)
    st, want = O.mxfp4_matmul(canonical, rows, blocks, 1, act, m, bias, kind=kind)
    assert st == O.OK
    w = G.Weights.upload(ctx, canonical, 1, rows, blocks)
    got = np.full(m * rows, np.nan, np.float32)
    G.mxfp4_matmul(ctx, w, 0, act, m, bias, got, kind=kind)
    assert_same_bits(got, want)
    w.close()


def test_matmul_special_values_and_no_bias(ctx):
    rows, blocks, m = 24, 4, 3
    canonical = O.gen_mxfp4(9, 9, 1, rows, blocks).reshape(rows, blocks, 17)
    canonical[0, :, 0] = 0x00      # e8m0 2^-127
    canonical[1, 1, 0] = 0xFF      # NaN scale
    canonical[2, :, 1:] = 0x00     # zero codes
    canonical[3, :, 1:] = 0x88     # -0 codes
    canonical[4, :, 1:] = 0x77     # +6 everywhere
    canonical[5, :, 0] = 254       # 2^127: overflows to inf
    canonical[6, :, 0] = 1         # 2^-126: denormal products
    canonical = canonical.ravel()
    rng = np.random.default_rng(3)
    act = random_records(rng, m, blocks, G.ACT_RESIDUAL_Q8)
    act["primary"]["values"][0] = 127
    act["residual"]["values"][0] = -127
    act["primary"]["scale"][1] = 0.0
    st, want = O.mxfp4_matmul(canonical, rows, blocks, 1, act, m, None)
    w = G.Weights.upload(ctx, canonical, 1, rows, blocks)
    got = np.full(m * rows, np.nan, np.float32)
    G.mxfp4_matmul(ctx, w, 0, act, m, None, got)
    assert_same_bits(got, want)
    assert np.isnan(got.reshape(m, rows)[:, 1]).all()
    w.close()


def test_padded_output_columns_are_never_written(ctx):
    # matmul.rs:1121-1165: 1234.0 canaries in the stride padding survive.
    rows, blocks, m, stride = 20, 3, 5, 27
    canonical = O.gen_mxfp4(4, 4, 2, rows, blocks)
    rng = np.random.default_rng(4)
    act = random_records(rng, m, blocks, G.ACT_RESIDUAL_Q8)
    bias = rng.standard_normal(rows).astype(np.float32)
    out = np.full((m - 1) * stride + rows, 1234.0, np.float32)
    want = out.copy()
    st = O.mxfp4_matmul(canonical[rows * blocks * 17:], rows, blocks, 1, act, m, bias, out_stride=stride, out=want)[0]
    assert st == O.OK
    w = G.Weights.upload(ctx, canonical, 2, rows, blocks)
    G.mxfp4_matmul(ctx, w, 1, act, m, bias, out, output_stride=stride)
    assert_same_bits(out, want)
    for r in range(m - 1):
        assert (out[r * stride + rows:(r + 1) * stride] == 1234.0).all()
    w.close()


def test_strided_activation_rows(ctx):
    rows, blocks, m, astride = 32, 3, 4, 5
    canonical = O.gen_mxfp4(6, 6, 1, rows, blocks)
    rng = np.random.default_rng(6)
    act = random_records(rng, m * astride, 1, G.ACT_RESIDUAL_Q8)[: (m - 1) * astride + blocks]
    st, want = O.mxfp4_matmul(canonical, rows, blocks, 1, act, m, None, act_stride=astride)
    assert st == O.OK
    w = G.Weights.upload(ctx, canonical, 1, rows, blocks)
    got = np.full(m * rows, np.nan, np.float32)
    G.mxfp4_matmul(ctx, w, 0, act, m, None, got, row_stride=astride)
    assert_same_bits(got, want)
    w.close()


def test_invalid_problems_fail_before_any_write(ctx):
    rows, blocks, m = 16, 2, 2
    w = G.Weights.upload(ctx, O.gen_mxfp4(1, 1, 1, rows, blocks), 1, rows, blocks)
    act = np.zeros(m * blocks, O.RQ8_DTYPE)
    out = np.full(m * rows, 1234.0, np.float32)
    with pytest.raises(G.GossmxError) as e:
        G.mxfp4_matmul(ctx, w, 0, act, m, np.zeros(rows - 1, np.float32), out)
    assert e.value.status == G.ERR_INVALID_DIMENSIONS
    with pytest.raises(G.GossmxError) as e:
        G.mxfp4_matmul(ctx, w, 0, act[:-1], m, None, out)
    assert e.value.status == G.ERR_INVALID_DIMENSIONS
    with pytest.raises(G.GossmxError) as e:
        G.mxfp4_matmul(ctx, w, 1, act, m, None, out)
    assert e.value.status == G.ERR_INVALID_DIMENSIONS
    assert (out == 1234.0).all()
    ctx.inject_fault(True)
    with pytest.raises(G.GossmxError) as e:
        G.mxfp4_matmul(ctx, w, 0, act, m, None, out)
    assert e.value.status == G.ERR_INJECTED_FAULT
    assert (out == 1234.0).all()
    G.mxfp4_matmul(ctx, w, 0, act, m, None, out)  # the hook fires once
    w.close()


def test_integer_dots_are_exact_at_extremes(ctx):
    # 127 * 12 * 32 = 48,768 per block (matmul.rs:1860-1866); with power-of-two
    # scales every float step is exact, so the output is the integer sum.
    rows, blocks = 16, 90
    canonical = np.tile(np.array([127] + [0x77] * 16, np.uint8), rows * blocks)
    act = np.zeros(blocks, O.RQ8_DTYPE)
    act["primary"]["scale"] = 1.0
    act["primary"]["values"] = 127
    act["residual"]["scale"] = 2.0 ** -7
    act["residual"]["values"] = -127
    w = G.Weights.upload(ctx, canonical, 1, rows, blocks)
    got = np.zeros(rows, np.float32)
    G.mxfp4_matmul(ctx, w, 0, act, 1, None, got)
    expect = blocks * (48768 * 0.5 - 48768 * 0.5 * 2.0 ** -7)
    assert (got == np.float32(expect)).all()
    w.close()
