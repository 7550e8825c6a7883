"""Pins the CPU oracle (oracle/gossmx_oracle.cpp) before anything is checked
against it: the reference's golden SHA-256 vectors, its known-answer tests,
closed forms, and brute force on tiny inputs. CPU only."""
import ctypes as C
import hashlib
import json
import math
import os

import numpy as np
import pytest

import oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "mxfp4_matrix_hashes.json")
LIBM = C.CDLL("libm.so.6")
LIBM.sinf.restype = C.c_float
LIBM.sinf.argtypes = [C.c_float]


def f32(x):
    return np.float32(x)


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a, dtype=np.float32).tobytes()).hexdigest()


def golden_cases():
    with open(GOLDEN) as fh:
        return json.load(fh)["cases"]


# --- golden vectors: mxfp4_matrix_bench.rs:166-372, evidence correctness[] ---

@pytest.mark.parametrize("case", golden_cases(), ids=lambda c: f"{c['role']}-m{c['m']}")
def test_matmul_golden_hash_canonical_and_x8(case):
    n, m = case["n"], case["m"]
    canonical, x8, res, bias = O.bench_fixtures(n, 90, m)
    for data, layout in ((canonical, 1), (x8, 2)):
        st, out = O.mxfp4_matmul(data, n, 90, layout, res, m, bias)
        assert st == O.OK
        assert sha(out) == case["sha256"]


@pytest.mark.parametrize("case", golden_cases(), ids=lambda c: f"{c['role']}-m{c['m']}")
def test_cpu_baseline_lanes_reproduce_golden_hash(case):
    """The Auto lane (x8 AVX2 GEMV at M=1, scalar otherwise) and its all-cores
    variant must be bit-identical to scalar before they are timed
    (mxfp4_matrix_bench.rs:215-246)."""
    n, m = case["n"], case["m"]
    _, x8, res, bias = O.bench_fixtures(n, 90, m)
    for threads in (1, 4):
        out = O.mxfp4_matmul_auto(x8, n, 90, res, m, bias, threads=threads)
        assert sha(out) == case["sha256"]
    # The forced panel lanes (Mxfp4MatmulBackend::Avx2 4x8, ::Avx512Vnni 8x8;
    # matmul.rs:829-961), one thread as the reference runs them and spread.
    lanes = [lane for lane, ok in ((O.LANE_AVX2_4X8, O.lib().oracle_has_avx2()),
                                   (O.LANE_AVX512_8X8, O.lib().oracle_has_avx512_vnni())) if ok]
    assert lanes, "this host runs neither panel lane"
    for lane in lanes:
        for threads in (1, 3):
            out = O.mxfp4_matmul_lane(x8, n, 90, res, m, bias, lane, threads)
            assert sha(out) == case["sha256"], (lane, threads)


# --- known-answer tests of crates/gpt-oss-cpu-kernels/src/lib.rs ---

def test_e8m0_edges_kat():
    # lib.rs:1716-1722
    assert np.float32(O.lib().oracle_e8m0_scale(0)).view(np.uint32) == 0x00400000
    for s in (1, 2, 126, 127, 128, 254):
        assert np.float32(O.lib().oracle_e8m0_scale(s)).view(np.uint32) == s << 23
    assert math.isnan(O.lib().oracle_e8m0_scale(0xFF))


def test_all_codes_decode_and_doubled_integers():
    # lib.rs:1561-1568 (MXFP4_VALUES, lib.rs:37-39) and mxfp4_integer (lib.rs:1067-1074)
    values = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]
    for code, v in enumerate(values):
        got = O.lib().oracle_decode_mxfp4(code)
        assert np.float32(got).view(np.uint32) == np.float32(v).view(np.uint32)
        assert O.lib().oracle_mxfp4_integer(code) == int(2 * v)


def test_adjacent_split_round_trip_kat():
    # lib.rs:1571-1583
    adjacent = np.array([((2 * i) & 15) | (((2 * i + 1) & 15) << 4) for i in range(16)], np.uint8)
    split = np.zeros(16, np.uint8)
    O.lib().oracle_adjacent_to_split(O._p(adjacent), O._p(split))
    for i, b in enumerate(split):
        assert b & 15 == i and b >> 4 == i
    back = np.zeros(16, np.uint8)
    O.lib().oracle_split_to_adjacent(O._p(split), O._p(back))
    assert (back == adjacent).all()


def _q8(scale, values):
    a = np.zeros(1, O.Q8_DTYPE)
    a["scale"] = scale
    a["values"][0] = values
    return a


def test_block_dot_official_scale_kat():
    # lib.rs:1790-1806: scale 127, packed 0x11, q = 1 -> integer 32, float 16.0
    rec = np.array([127] + [0x11] * 16, np.uint8)
    act = _q8(1.0, [1] * 32)
    st, out = O.mxfp4_matmul(rec, 1, 1, 1, act, 1, None, kind=1)
    assert st == O.OK and out[0] == 16.0
    ract = np.zeros(1, O.RQ8_DTYPE)
    ract["primary"] = act[0]
    dots = O.block_dots(rec, 1, 1, ract)
    assert dots[0, 0, 0] == 32 and dots[0, 0, 1] == 0


def test_fused_residual_dot_equals_two_dots_kat():
    # lib.rs:1808-1832
    rec = np.array([129] + [(i | ((15 - i) << 4)) for i in range(16)], np.uint8)
    ract = np.zeros(1, O.RQ8_DTYPE)
    ract["primary"]["scale"] = 0.125
    ract["primary"]["values"][0] = [i - 16 for i in range(32)]
    ract["residual"]["scale"] = 0.001
    ract["residual"]["values"][0] = [31 - i for i in range(32)]
    dots = O.block_dots(rec, 1, 1, ract)[0, 0]
    w = [O.lib().oracle_mxfp4_integer(c) for i in range(16) for c in (rec[1 + i] & 15, rec[1 + i] >> 4)]
    assert dots[0] == sum(int(a) * int(b) for a, b in zip(w, ract["primary"]["values"][0]))
    assert dots[1] == sum(int(a) * int(b) for a, b in zip(w, ract["residual"]["values"][0]))


def test_extreme_block_dot_closed_form():
    # matmul.rs:1860-1866: 127 * 12 * 32 = 48,768 at the extremes.
    rec = np.array([127] + [0x77] * 16, np.uint8)  # every code 7 -> 12
    ract = np.zeros(1, O.RQ8_DTYPE)
    ract["primary"]["values"][0] = [127] * 32
    ract["residual"]["values"][0] = [-127] * 32
    d = O.block_dots(rec, 1, 1, ract)[0, 0]
    assert d[0] == 48768 and d[1] == -48768


def test_invalid_scale_propagates_nan():
    # lib.rs:1598-1635
    rec = np.tile(np.array([0xFF] + [0x11] * 16, np.uint8), 8)
    act = _q8(1.0, [1] * 32)
    st, out = O.mxfp4_matmul(rec, 8, 1, 1, act, 1, np.zeros(8, np.float32), kind=1)
    assert st == O.OK and np.isnan(out).all()
    x8 = O.pack_x8(rec, 8, 1)
    st, out = O.mxfp4_matmul(x8, 8, 1, 2, act, 1, np.zeros(8, np.float32), kind=1)
    assert st == O.OK and np.isnan(out).all()


def test_zero_block_quantization_is_stable():
    # lib.rs:1724-1732, 1764-1775
    st, q = O.quantize_q8(np.zeros(32, np.float32))
    assert st == O.OK and q["scale"][0] == 0.0 and (q["values"][0] == 0).all()
    st, r = O.quantize_residual_q8(np.zeros(32, np.float32))
    assert st == O.OK
    for part in ("primary", "residual"):
        assert r[part]["scale"][0] == 0.0 and (r[part]["values"][0] == 0).all()


def test_residual_q8_reconstructs_better_than_one_pass():
    # lib.rs:1734-1762 (f32 arithmetic as in the Rust test; sinf from libm)
    x = np.array([f32(LIBM.sinf(f32(i) * f32(0.731))) * f32(9.0) + f32(i) * f32(0.013) for i in range(32)],
                 np.float32)
    _, q = O.quantize_q8(x)
    _, r = O.quantize_residual_q8(x)
    e1 = np.abs(x - q["values"][0].astype(np.float32) * q["scale"][0]).sum()
    e2 = np.abs(x - r["primary"]["values"][0].astype(np.float32) * r["primary"]["scale"][0]
                - r["residual"]["values"][0].astype(np.float32) * r["residual"]["scale"][0]).sum()
    assert e2 < e1 * 0.02


@pytest.mark.parametrize("bad", [float("nan"), float("inf"), float("-inf")])
def test_residual_q8_rejects_non_finite(bad):
    # lib.rs:1777-1788
    x = np.zeros(32, np.float32)
    x[7] = bad
    assert O.quantize_residual_q8(x)[0] == O.NON_FINITE_INPUT
    assert O.quantize_q8(x)[0] == O.NON_FINITE_INPUT


def test_quantize_closed_forms():
    # quantize_q8_block (lib.rs:1051-1065): max 127 gives scale 1 and inverse 1,
    # so values are rounded half away from zero (f32::round) and clamped.
    x = np.zeros(32, np.float32)
    x[0] = 127.0
    x[1], x[2], x[3], x[4] = 2.5, -2.5, 0.5, -0.49
    _, q = O.quantize_q8(x)
    assert q["scale"][0] == 1.0
    assert list(q["values"][0][:5]) == [127, 3, -3, 1, 0]
    # Exact multiples of a power-of-two scale reconstruct exactly and leave a
    # zero residual.
    k = np.arange(-16, 16, dtype=np.float32)
    x = k * np.float32(127.0 / 16.0 / 127.0 * 4.0)
    x[0] = -127 * np.float32(0.25)
    _, r = O.quantize_residual_q8(x)
    s = r["primary"]["scale"][0]
    assert s == np.float32(0.25)
    assert (r["primary"]["values"][0].astype(np.float32) * s == x).all()
    assert r["residual"]["scale"][0] == 0.0


def test_exact_bf16_lane_bits_kat():
    # lib.rs:1834-1856: pins bf16 round-to-nearest-even (half 2.7.1).
    rec = np.array([124, 0x75, 0x31, 0xED, 0xA6, 0x42, 0xF9, 0x8B, 0xC4, 0x17, 0x5E, 0x20, 0xDA, 0x63, 0xBF,
                    0x94, 0x28], np.uint8)
    act = np.array([O.bf16_bits(f32(LIBM.sinf((f32(i) - f32(15.5)) * f32(0.137))) * f32(2.25))
                    for i in range(32)], np.uint16)
    lanes = np.zeros(16, np.float32)
    O.lib().oracle_accumulate_mxfp4_bf16_block(O._p(rec), O._p(act), O._p(lanes))
    assert list(lanes.view(np.uint32)) == [
        3206160384, 3217183744, 3204644864, 3169845248, 1062731776, 1067950080, 3215392768,
        3203301376, 1041563648, 1059454976, 3217698816, 1057914880, 1061216256, 3188326400,
        3186294784, 1049509888]


def test_bf16_rounding_ties_and_nan():
    # half 2.7.1 from_f32: round to nearest, ties to even; NaN stays NaN.
    assert O.bf16_bits(np.uint32(0x3F808000).view(np.float32)) == 0x3F80  # tie, even stays
    assert O.bf16_bits(np.uint32(0x3F818000).view(np.float32)) == 0x3F82  # tie, odd rounds up
    assert O.bf16_bits(np.uint32(0x3F808001).view(np.float32)) == 0x3F81
    assert O.bf16_bits(np.uint32(0x7F7FFFFF).view(np.float32)) == 0x7F80  # rounds to +inf
    assert (O.bf16_bits(float("nan")) & 0x7FC0) == 0x7FC0
    v = np.random.default_rng(1).standard_normal(4096).astype(np.float32)
    assert (O.bf16_round_array(v).view(np.uint32) >> 16 == np.array([O.bf16_bits(x) for x in v])).all()


# --- cpu_runner.rs and gpt-oss-moe-semantics KATs ---

def test_swiglu_kat():
    # cpu_runner.rs:4406-4409
    out = O.swiglu(np.array([2.0, 3.0, -1.0, 8.0], np.float32), 2)
    assert list(out) == [7.75, -1.234375]


def test_stable_top_k_kats():
    # cpu_runner.rs:4412-4414 and moe-semantics/src/lib.rs:196-199
    assert list(O.stable_top_k(np.array([1, 2, 2, 0], np.float32), 2)) == [1, 2]
    assert list(O.stable_top_k(np.array([1, 1, 0.5, 1], np.float32), 2)) == [0, 1]


def test_route_top_k_kats():
    # gpu_layer.rs:3284-3291 and moe-semantics/src/lib.rs:229-240
    v = np.array([1, 1, 0.5, 1], np.float32)
    sel = O.stable_top_k(v, 2)
    w = O.softmax(v[sel])
    assert list(sel) == [0, 1] and list(w) == [0.5, 0.5]
    v = np.array([0.0, 2.0, 1.0], np.float32)
    sel = O.stable_top_k(v, 2)
    w = O.softmax(v[sel])
    assert list(sel) == [1, 2] and abs(float(w.sum()) - 1.0) < 1e-6
    w = O.softmax(np.array([1.0, 2.0, 3.0], np.float32))
    assert abs(float(w.sum()) - 1.0) < 1e-6


def tiny_layer(seed=7, experts=3, hidden=64, intermediate=32, top_k=2):
    return O.synthetic_layer(seed, 0, experts=experts, hidden=hidden, intermediate=intermediate, top_k=top_k)


def test_route_grouping_order_kat():
    # cpu_runner.rs:4417-4452: routes (2,0,0),(1,0,1),(2,1,0),(1,1,1) group to
    # (1,0,1),(1,1,1),(2,0,0),(2,1,0). Injected logits rank expert 2 then 1.
    layer = tiny_layer()
    logits = np.array([[0.0, 1.0, 2.0], [0.0, 1.0, 2.0]], np.float32)
    x = O.gen_hidden(3, 9, 2, 64)
    r = O.moe_batch(layer, x, injected_logits=logits)
    assert r["status"] == O.OK
    assert [(int(o) // 2, int(o) % 2) for o in r["route_order"]] == [(0, 1), (1, 1), (0, 0), (1, 0)]
    assert r["selected"].tolist() == [[2, 1], [2, 1]]


# --- glibc expf restatement (the device expf follows the same algorithm) ---

def test_expf_restatement_matches_glibc_on_every_float():
    first = C.c_uint32()
    bad = O.lib().oracle_expf_check(0, 0xFFFFFFFF, 8, C.byref(first))
    assert bad == 0, f"first mismatch at bits {first.value:#010x}"


# --- composition of moe_batch, checked piece by piece (cpu_runner.rs:2794-3013) ---

def _moe_by_pieces(layer, x):
    """moe_batch recomposed from separately pinned oracle pieces."""
    E, H, I, K = layer.experts, layer.hidden, layer.intermediate, layer.top_k
    m = x.shape[0]
    lg = np.zeros((m, E), np.float32)
    O.lib().oracle_bf16_matvec(O._p(layer.router_weight), E, H, O._p(np.ascontiguousarray(x[0])), O._p(lg[0]))
    for r in range(m):
        O.lib().oracle_bf16_matvec(O._p(layer.router_weight), E, H, O._p(np.ascontiguousarray(x[r])), O._p(lg[r]))
    lg = O.bf16_round_array(lg + layer.router_bias[None, :])
    out = np.zeros((m, H), np.float32)
    sel_all, w_all = [], []
    for r in range(m):
        sel = O.stable_top_k(lg[r], K)
        w = O.bf16_round_array(O.softmax(lg[r][sel]))
        sel_all.append(sel)
        w_all.append(w)
        acc = np.zeros(H, np.float32)
        for rank, e in enumerate(sel):
            _, q = O.quantize_residual_q8(O.bf16_to_f32(x[r]))
            gu_w = layer.gate_up[e * 2 * I * (H // 32) * 17:(e + 1) * 2 * I * (H // 32) * 17]
            _, gu = O.mxfp4_matmul(gu_w, 2 * I, H // 32, 1, q, 1, layer.gate_up_bias[e * 2 * I:(e + 1) * 2 * I])
            a = O.bf16_round_array(O.swiglu(O.bf16_round_array(gu), I))
            _, q2 = O.quantize_residual_q8(a)
            dn_w = layer.down[e * H * (I // 32) * 17:(e + 1) * H * (I // 32) * 17]
            _, y = O.mxfp4_matmul(dn_w, H, I // 32, 1, q2, 1, layer.down_bias[e * H:(e + 1) * H])
            acc = acc + O.bf16_round_array(y) * w[rank]
        out[r] = O.bf16_round_array(acc)
    return lg, np.array(sel_all), np.array(w_all), out


def test_moe_batch_equals_composition_of_pieces():
    layer = tiny_layer(experts=4, hidden=96, intermediate=64, top_k=2)
    x = O.gen_hidden(11, 1, 5, 96)
    r = O.moe_batch(layer, x)
    assert r["status"] == O.OK
    lg, sel, w, out = _moe_by_pieces(layer, x)
    assert (r["router_logits"].view(np.uint32) == lg.view(np.uint32)).all()
    assert (r["selected"] == sel).all()
    assert (r["routing_weights"].view(np.uint32) == w.view(np.uint32)).all()
    assert (r["output"].view(np.uint32) == out.view(np.uint32)).all()


def test_router_dot_is_exact_on_exact_inputs():
    # With small-integer bf16 operands every product and partial sum is exact,
    # so any summation order gives the integer dot (scalar_bf16_dot,
    # lib.rs:1007-1029).
    rng = np.random.default_rng(5)
    w = rng.integers(-8, 9, size=(3, 2880)).astype(np.float32)
    x = rng.integers(-8, 9, size=2880).astype(np.float32)
    wb = (w.view(np.uint32) >> 16).astype(np.uint16)
    xb = (x.view(np.uint32) >> 16).astype(np.uint16)
    out = np.zeros(3, np.float32)
    O.lib().oracle_bf16_matvec(O._p(wb), 3, 2880, O._p(xb), O._p(out))
    assert (out == (w.astype(np.int64) @ x.astype(np.int64)).astype(np.float32)).all()
    # General inputs stay within a float64 error bound of the true dot.
    wg = O.gen_bf16_normal(1, 2, 2880, 0.0, 0.02)
    xg = O.gen_bf16_normal(1, 3, 2880)
    O.lib().oracle_bf16_matvec(O._p(wg), 1, 2880, O._p(xg), O._p(out))
    exact = float(O.bf16_to_f32(wg).astype(np.float64) @ O.bf16_to_f32(xg).astype(np.float64))
    assert abs(out[0] - exact) < 1e-4


def test_rms_norm_closed_form():
    # lib.rs:699-730: a constant vector c normalises to c / sqrt(c^2 + eps).
    x = np.full(2880, 2.0, np.float32)
    out = np.zeros_like(x)
    O.lib().oracle_rms_norm(O._p(x), O._p(np.ones_like(x)), 2880, np.float32(1e-5), O._p(out))
    assert np.allclose(out, 2.0 / math.sqrt(4.0 + 1e-5), rtol=1e-6)


def _rms(x, w, eps):
    x = np.asarray(x, np.float32)
    return O.rms_norm(x, np.asarray(w, np.float32), eps)


def test_rms_norm_sums_in_sixteen_lanes():
    # scalar_sum_squares (lib.rs:1031-1043) keeps 16 lane sums. With x =
    # [4096, 1 x 31]: lane 0 = 2^24 + 1 -> 2^24 (RNE), lanes 1..15 = 2, total
    # 2^24 + 30. A sequential sum would stay at 2^24 (every + 1 rounds back).
    x = np.ones(32, np.float32)
    x[0] = 4096.0
    out = _rms(x, np.ones(32), 0.0)
    f = np.float32
    lanes = f(1) / np.sqrt(f(16777246.0) / f(32))
    sequential = f(1) / np.sqrt(f(16777216.0) / f(32))
    assert lanes != sequential
    assert out[1] == lanes  # x[1] = 1 and w[1] = 1: the output is the inverse itself


def test_rms_norm_exact_rows_return_the_weights():
    # Rows whose sum of squares, mean, root and inverse are exact: the output
    # is 1 * w, bit for bit, for any weights (n = 16 and the 2880 of GPT-OSS).
    rng = np.random.default_rng(7)
    for n, v in ((16, 4.0), (2880, 2.0), (2880, 0.25)):
        w = rng.standard_normal(n).astype(np.float32)
        out = _rms(np.full(n, v), w, 0.0)
        assert (out.view(np.uint32) == w.view(np.uint32)).all()


def test_rms_norm_reference_weights_example():
    # The reference's rms_norm_with_weights case (layers/norm.rs:217-228):
    # [2, 2] with weights [0.5, 2] -> [0.5, 2.0] within 0.01; after the bf16
    # boundary exactly.
    out = _rms([2.0, 2.0], [0.5, 2.0], 1e-6)
    assert abs(out[0] - 0.5) < 0.01 and abs(out[1] - 2.0) < 0.01
    x = np.array([[O.bf16_bits(2.0), O.bf16_bits(2.0)]], np.uint16)
    b = O.norm_boundary(x, np.array([0.5, 2.0], np.float32), 1e-6)
    assert b.tolist() == [[0x3F00, 0x4000]]


def test_rms_norm_multiplies_left_to_right():
    # output = (x * inverse) * w (lib.rs:726-728), not x * (inverse * w): with
    # x[0] = w[0] = 1 the first output is the inverse, and rows where the two
    # orders differ show which one the oracle takes.
    rng = np.random.default_rng(11)
    f = np.float32
    differ = 0
    for _ in range(20):
        x = rng.standard_normal(64).astype(np.float32) * f(3)
        w = (rng.standard_normal(64).astype(np.float32) * f(0.7) + f(1)).astype(np.float32)
        x[0], w[0] = 1.0, 1.0
        out = _rms(x, w, 1e-5)
        inv = out[0]
        left = ((x * inv).astype(np.float32) * w).astype(np.float32)
        right = (x * (inv * w).astype(np.float32)).astype(np.float32)
        assert (out.view(np.uint32) == left.view(np.uint32)).all()
        differ += int((left != right).sum())
    assert differ > 0


def test_add_residual_rounds_to_nearest_even():
    # add_residual (cpu_runner.rs:3732-3738) = bf16(residual + update): ties
    # of the bf16 grid (spacing 2^-7 at 1.0) go to the even mantissa.
    res = np.array([0x3F80, 0x3F80, 0x3F80, 0xBF80], np.uint16)  # 1, 1, 1, -1
    upd = np.array([2.0 ** -8, 3 * 2.0 ** -8, -2.0 ** -9, 1.0], np.float32)
    assert O.add_residual(res, upd).tolist() == [0x3F80, 0x3F82, 0x3F80, 0x0000]


def test_moe_one_hot_and_all_experts_invariants():
    # top_k == experts: every expert is used once per row, weights sum ~ 1.
    layer = tiny_layer(experts=3, hidden=64, intermediate=32, top_k=3)
    x = O.gen_hidden(2, 4, 3, 64)
    r = O.moe_batch(layer, x)
    assert r["status"] == O.OK
    for row in r["selected"]:
        assert sorted(row.tolist()) == [0, 1, 2]
    assert np.allclose(r["routing_weights"].sum(1), 1.0, atol=1e-2)
    # Routing in rank order: logits of the selected experts are non-increasing.
    for lg, sel in zip(r["router_logits"], r["selected"]):
        assert (np.diff(lg[sel]) <= 0).all()


def test_moe_rejects_non_finite_logits():
    layer = tiny_layer()
    x = O.gen_hidden(3, 9, 1, 64)
    logits = np.array([[0.0, float("inf"), 1.0]], np.float32)
    assert O.moe_batch(layer, x, injected_logits=logits)["status"] == O.NON_FINITE_LOGITS


# --- order-defined float chains: inputs where the plausible other orders give
# other bits (each alternative is computed here in float32 and must differ) ---

F = np.float32
B24 = float(2 ** 24)  # ulp(2^24) = 2: adding 1 ties back to 2^24


def _bits(v):
    return np.float32(v).view(np.uint32)


def _tree(v):
    v = [F(t) for t in v]
    while len(v) > 1:
        if len(v) % 2:
            v.append(F(0))
        v = [F(v[2 * i] + v[2 * i + 1]) for i in range(len(v) // 2)]
    return v[0]


def _lane_sums(p, lanes):
    acc = [F(0)] * lanes
    for i, t in enumerate(p):
        acc[i % lanes] = F(acc[i % lanes] + F(t))
    return acc


def _fold(v, start=-0.0):
    s = F(start)
    for t in v:
        s = F(s + F(t))
    return s


def dot_alternatives(p):
    """Other summation orders of the products p a bf16 dot might use."""
    return {
        "sequential": _fold(p, 0.0),
        "pairwise tree": _tree(p),
        "16 lanes folded as a tree": _tree(_lane_sums(p, 16)),
        "16 lanes folded 15..0": _fold(_lane_sums(p, 16)[::-1]),
        "8 lanes": _fold(_lane_sums(p, 8)),
        "32 lanes": _fold(_lane_sums(p, 32)),
        "16 blocked lanes": _fold([_fold(p[j * len(p) // 16:(j + 1) * len(p) // 16], 0.0) for j in range(16)]),
        "float64": F(np.sum(np.asarray(p, np.float64))),
    }


def router_pin_case(hidden=64, offset=0):
    """Router rows whose bf16 logits depend on scalar_bf16_dot's order
    (lib.rs:1007-1029): 16 lanes, lane j sums products i = j mod 16 in order,
    lanes folded 0..15. The products are exact (bf16 x bf16); with x[offset] =
    x[offset + 16] = 2^12:
      row 0: products 2^24 at offset (lane 0), -2^24 at offset + 16 (lane 0
        again), 1 at offset + 1..15. Lane 0 cancels before the small lanes
        join: logit 15. A sequential sum absorbs the 1s into 2^24 first
        (logit 0), pairwise trees and other lane counts keep some (14, 0).
      row 1: 2^24 at offset, 1 at offset + 1..15, bias -2^24. Folding the
        lanes 0..15 absorbs every 1 (logit 0); a tree fold keeps 14, a
        reversed fold 16 (the 15 ones sum to 15, then tie to even).
      rows 2, 3: N(0, 0.02) weights, bias 0.
    offset places the construction (a multiple of 16; with hidden 2880 and
    offset 1424 it straddles the router kernel's 1440-element staging)."""
    rng = np.random.default_rng(3)
    x = O.bf16_round_array(rng.standard_normal(hidden).astype(np.float32))
    x[offset:offset + 32] = 1.0
    x[offset] = x[offset + 16] = 4096.0
    w = np.zeros((4, hidden), np.float32)
    w[0, offset], w[0, offset + 16] = 4096.0, -4096.0
    w[0, offset + 1:offset + 16] = 1.0
    w[1, offset] = 4096.0
    w[1, offset + 1:offset + 16] = 1.0
    w[2:] = O.bf16_round_array(rng.standard_normal((2, hidden)).astype(np.float32) * F(0.02))
    bias = np.array([0.0, -B24, 0.0, 0.0], np.float32)
    to_bits = lambda a: (np.ascontiguousarray(a, np.float32).view(np.uint32) >> 16).astype(np.uint16)
    return to_bits(w), bias, to_bits(x)


@pytest.mark.parametrize("hidden,offset", [(64, 0), (2880, 1424)])
def test_bf16_dot_sums_in_sixteen_ordered_lanes(hidden, offset):
    w, bias, x = router_pin_case(hidden, offset)
    got = O.bf16_matvec(w, x)
    wf, xf = O.bf16_to_f32(w), O.bf16_to_f32(x)
    expected = {0: 15.0, 1: B24}
    for row, want in expected.items():
        assert got[row] == want
        p = (wf[row] * xf).astype(np.float32)  # exact products
        ref_logit = O.bf16_round_array(np.array([F(got[row] + bias[row])]))[0]
        for name, alt in dot_alternatives(p).items():
            if alt == got[row]:
                continue
            alt_logit = O.bf16_round_array(np.array([F(alt + bias[row])]))[0]
            assert alt_logit != ref_logit, f"row {row}: {name} would give the same logit"
    # every alternative order differs from the reference on one of the rows
    # (at offset 1424 the 32-lane split lands like the 16-lane one)
    for name in dot_alternatives([0.0]):
        if offset % 32 == 0 or name != "32 lanes":
            assert any(dot_alternatives((wf[r] * xf).astype(np.float32))[name] != got[r] for r in (0, 1)), name
    # the router logits through moe_batch: bf16(dot + bias)
    layer = O.MoeLayerHost(w, bias, O.gen_mxfp4(1, 1, 4, 64, hidden // 32), np.zeros(4 * 64, np.float32),
                           O.gen_mxfp4(1, 2, 4, hidden, 1), np.zeros(4 * hidden, np.float32), 4, hidden, 32, 2)
    r = O.moe_batch(layer, x[None, :])
    assert r["status"] == O.OK
    assert r["router_logits"][0, 0] == 15.0 and r["router_logits"][0, 1] == 0.0


# Rank-ordered bf16 logits whose routing weights depend on the softmax
# denominator's order (cpu_runner.rs:3784-3795: sum of expf(v - max) folded in
# rank order): found by search over random bf16 quadruples, each weight
# checked against the other orders below.
SOFTMAX_PIN_ROWS = [
    [3.859375, -0.8046875, -0.93359375, -4.78125],    # reversed and float64 sums round a weight differently
    [3.375, 0.80078125, 0.71484375, -1.515625],      # the pairwise sum does
]


def _expf(v):
    return np.float32(LIBM_EXPF(float(v)))


LIBM_EXPF = C.CDLL("libm.so.6").expf
LIBM_EXPF.restype = C.c_float
LIBM_EXPF.argtypes = [C.c_float]


def test_softmax_denominator_folds_in_rank_order():
    differs = set()
    for row in SOFTMAX_PIN_ROWS:
        v = np.array(row, np.float32)
        e = [_expf(F(t - v[0])) for t in v]
        seq = _fold(e)
        want = np.array([F(t / seq) for t in e], np.float32)
        got = O.softmax(v)
        assert (got.view(np.uint32) == want.view(np.uint32)).all()
        alts = {"reversed": _fold(e[::-1], 0.0), "pairwise": F(F(e[0] + e[1]) + F(e[2] + e[3])),
                "float64": F(np.sum(np.asarray(e, np.float64)))}
        for name, d in alts.items():
            w_alt = O.bf16_round_array(np.array([F(t / d) for t in e], np.float32))
            if (w_alt.view(np.uint32) != O.bf16_round_array(want).view(np.uint32)).any():
                differs.add(name)
    assert differs == {"reversed", "pairwise", "float64"}


def test_combine_adds_weighted_ranks_in_rank_order():
    # weighted = y * w (exact here: bf16 x bf16), output += weighted in rank
    # order from 0.0, then bf16 (cpu_runner.rs:2959-2999).
    y = np.array([[[B24], [1.0], [-B24], [1.0]],     # in order: 2^24 absorbs the first 1 -> 1
                  [[1.0], [B24], [1.0], [-B24]],     # in order: both 1s absorbed -> 0
                  [[3.0], [-2.0], [0.5], [0.25]]], np.float32)
    w = np.array([[1.0, 1.0, 1.0, 1.0], [1.0, 1.0, 1.0, 1.0], [0.5, 0.25, 1.0, 2.0]], np.float32)
    got = O.combine(y, w)[:, 0]
    assert got.tolist() == [1.0, 0.0, 2.0]
    alts = {"reversed": lambda p: _fold(p[::-1], 0.0), "pairwise": lambda p: F(F(p[0] + p[1]) + F(p[2] + p[3])),
            "float64": lambda p: F(np.sum(np.asarray(p, np.float64)))}
    for name, fn in alts.items():
        outs = [fn([F(y[r, k, 0] * w[r, k]) for k in range(4)]) for r in range(2)]
        assert outs != got[:2].tolist(), name


def _record(scale, codes):
    """A canonical MXFP4 record: scale byte, then code(2j) | code(2j+1) << 4."""
    return np.array([scale] + [codes[2 * j] | (codes[2 * j + 1] << 4) for j in range(16)], np.uint8)


def exact_pin_layer():
    """A one-block layer (hidden = intermediate = 32, 2 experts, top-1,
    routing injected to expert 0) whose exact-BF16 gate_up row 0 depends on
    the 16-lane order of accumulate_mxfp4_bf16_block (lib.rs:932-945): with
    scale 2^10, codes 6 (4.0) and 14 (-4.0) at k = 0 and 16 against x = 2^12
    give products 2^24 and -2^24, both in lane 0, and code 2 (1.0) at k =
    1..15 against x = 2^-10 gives 1 in lanes 1..15. Lane 0 cancels first:
    the row is 15; a sequential sum over k absorbs the 1s into 2^24 (0)."""
    host = O.synthetic_layer(19, 0, experts=2, hidden=32, intermediate=32, top_k=1)
    codes = [6] + [2] * 15 + [14] + [0] * 15
    gate_up = host.gate_up.copy().reshape(2, 64, 17)
    gate_up[0, 0] = _record(137, codes)
    bias = host.gate_up_bias.copy()
    bias[0] = 0.0
    layer = O.MoeLayerHost(host.router_weight, host.router_bias, gate_up.ravel(), bias, host.down,
                           host.down_bias, 2, 32, 32, 1)
    x = np.zeros(32, np.float32)
    x[0] = x[16] = 4096.0
    x[1:16] = 2.0 ** -10
    xb = (x.view(np.uint32) >> 16).astype(np.uint16)[None, :]
    return layer, xb, np.array([[1.0, 0.0]], np.float32)


def test_exact_bf16_projection_sums_in_sixteen_ordered_lanes():
    layer, x, logits = exact_pin_layer()
    r = O.moe_batch(layer, x, injected_logits=logits, trace=True, projection=O.PROJECTION_EXACT_BF16)
    assert r["status"] == O.OK
    assert r["gate_up"][0, 0, 0] == 15.0
    codes = [6] + [2] * 15 + [14] + [0] * 15
    w = np.array([[0.0, 0.5, 1, 1.5, 2, 3, 4, 6, -0.0, -0.5, -1, -1.5, -2, -3, -4, -6][c] * 1024.0 for c in codes],
                 np.float32)
    p = (w * O.bf16_to_f32(x[0])).astype(np.float32)
    for name, alt in dot_alternatives(p).items():
        if name not in ("16 lanes folded as a tree", "16 lanes folded 15..0", "float64"):
            assert alt != 15.0, name
    # The exact path's lane KAT and the residual/Q8 modes agree on routing.
    for proj in (O.PROJECTION_RESIDUAL_Q8, O.PROJECTION_Q8):
        q = O.moe_batch(layer, x, injected_logits=logits, projection=proj)
        assert q["status"] == O.OK and (q["selected"] == r["selected"]).all()


def test_moe_lanes_and_modes_agree_with_the_scalar_matmul():
    """moe_batch on every expert-matmul lane (scalar, Auto, forced panels,
    threaded) gives the scalar lane's bits, for the residual-Q8 and Q8 modes
    (the panel lanes also serve the Q8 kind)."""
    layer = O.synthetic_layer(33, 0, experts=4, hidden=96, intermediate=64, top_k=2)
    x = O.gen_hidden(33, 1, 13, 96)
    for projection in (O.PROJECTION_RESIDUAL_Q8, O.PROJECTION_Q8):
        want = O.moe_batch(layer, x, trace=True, projection=projection)
        assert want["status"] == O.OK
        for lane in (O.LANE_AUTO, O.LANE_AVX2_4X8, O.LANE_AVX512_8X8):
            for threads in (1, 4):
                got = O.moe_batch(layer, x, trace=True, projection=projection, lane=lane, threads=threads)
                if got["status"] == O.UNAVAILABLE_BACKEND:
                    continue
                for key in ("output", "gate_up", "down"):
                    assert (got[key].view(np.uint32) == want[key].view(np.uint32)).all(), (projection, lane, key)


def test_panel_lanes_finish_output_tails_with_scalar_rows():
    """rows % 8 != 0: the complete x8 groups on the panel lane, the tail rows
    on the scalar chain (avx2_matmul, matmul.rs:876-884), for 1..9 input
    rows (partial and full panels) and both activation kinds."""
    rows, blocks = 20, 3
    canonical, _, _, bias = O.bench_fixtures(rows, blocks, 1)
    x8 = O.pack_x8(canonical, rows, blocks)
    for m in (1, 4, 5, 8, 9):
        _, _, res, _ = O.bench_fixtures(rows, blocks, m)
        q8 = np.ascontiguousarray(res["primary"])
        for kind, act in ((2, res), (1, q8)):
            st, want = O.mxfp4_matmul(canonical, rows, blocks, 1, act, m, bias, kind=kind)
            assert st == O.OK
            for lane in (O.LANE_AVX2_4X8, O.LANE_AVX512_8X8):
                if not (O.lib().oracle_has_avx512_vnni() if lane == 8 else O.lib().oracle_has_avx2()):
                    continue
                got = O.mxfp4_matmul_lane(x8, rows, blocks, act, m, bias, lane, 2, kind=kind)
                assert (got.view(np.uint32) == want.view(np.uint32)).all(), (m, kind, lane)


def test_output_unrounded_is_the_combine_sum_before_the_round_trip():
    """moe_batch's output_unrounded: per row and column, the rank-order sum
    from 0.0 of down output (the trace, pinned above) times routing weight,
    before fp32_to_bf16_roundtrip (cpu_runner.rs:2959-2991); its bf16 round
    is the output, and it differs from the output wherever the sum is not a
    bf16 value."""
    layer = O.synthetic_layer(51, 0, experts=6, hidden=64, intermediate=64, top_k=3)
    x = O.gen_hidden(51, 1, 7, 64)
    r = O.moe_batch(layer, x, trace=True)
    assert r["status"] == O.OK
    m, K, H = 7, 3, 64
    want = np.zeros((m, H), np.float32)
    for k in range(K):  # rank order, each product and each sum rounded to f32
        want = (want + (r["down"][:, k, :] * r["routing_weights"][:, k:k + 1]).astype(np.float32)).astype(np.float32)
    assert (r["output_unrounded"].view(np.uint32) == want.view(np.uint32)).all()
    assert (O.bf16_round_array(r["output_unrounded"]).view(np.uint32) == r["output"].view(np.uint32)).all()
    assert (r["output_unrounded"] != r["output"]).mean() > 0.9
