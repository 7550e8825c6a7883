"""ctypes wrapper over the CPU oracle (oracle/gossmx_oracle.cpp).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, always as the checker. The product package never
imports this module.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# ORACLE_LIB names another build (the sanitized test build); by default the
# in-tree library.
LIB_PATH = os.environ.get("ORACLE_LIB") or os.path.join(HERE, "libgossmx_oracle.so")

# numpy views of the reference's Q8Block / ResidualQ8Block (lib.rs:732-742):
# f32 scale + 32 x i8 values, 36 bytes, no padding.
Q8_DTYPE = np.dtype([("scale", "<f4"), ("values", "i1", (32,))])
RQ8_DTYPE = np.dtype([("primary", Q8_DTYPE), ("residual", Q8_DTYPE)])
assert Q8_DTYPE.itemsize == 36 and RQ8_DTYPE.itemsize == 72

OK = 0
INVALID_DIMENSIONS = 3
NON_FINITE_INPUT = 4
NON_FINITE_LOGITS = 8


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = C.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


class OracleLayer(C.Structure):
    _fields_ = [
        ("router_weight", C.c_void_p), ("router_bias", C.c_void_p),
        ("gate_up", C.c_void_p), ("gate_up_bias", C.c_void_p),
        ("down", C.c_void_p), ("down_bias", C.c_void_p),
        ("experts", C.c_size_t), ("hidden", C.c_size_t), ("intermediate", C.c_size_t), ("top_k", C.c_size_t),
        ("alpha", C.c_float), ("limit", C.c_float),
    ]


class OracleRope(C.Structure):
    _fields_ = [("head_dim", C.c_size_t), ("theta", C.c_double), ("yarn", C.c_int32), ("factor", C.c_double),
                ("original_max", C.c_size_t), ("beta_fast", C.c_double), ("beta_slow", C.c_double),
                ("truncate", C.c_int32)]


class OracleDenseLayer(C.Structure):
    _fields_ = [("input_norm", C.c_void_p), ("q_weight", C.c_void_p), ("q_bias", C.c_void_p),
                ("k_weight", C.c_void_p), ("k_bias", C.c_void_p), ("v_weight", C.c_void_p), ("v_bias", C.c_void_p),
                ("o_weight", C.c_void_p), ("o_bias", C.c_void_p), ("sinks", C.c_void_p),
                ("post_attention_norm", C.c_void_p), ("sliding", C.c_int32), ("moe", OracleLayer)]


class OracleModel(C.Structure):
    _fields_ = [("vocab", C.c_size_t), ("hidden", C.c_size_t), ("layers", C.c_size_t), ("heads", C.c_size_t),
                ("kv_heads", C.c_size_t), ("head_dim", C.c_size_t), ("sliding_window", C.c_size_t),
                ("context_cap", C.c_size_t), ("rms_norm_eps", C.c_float), ("rope", OracleRope),
                ("embedding", C.c_void_p), ("final_norm", C.c_void_p), ("lm_head", C.c_void_p),
                ("layer", C.POINTER(OracleDenseLayer))]


def _declare(L):
    vp, sz, i32, u32, f32, u64 = C.c_void_p, C.c_size_t, C.c_int, C.c_uint32, C.c_float, C.c_uint64
    sig = {
        "oracle_bf16_bits": (C.c_uint16, [f32]),
        "oracle_e8m0_scale": (f32, [C.c_uint8]),
        "oracle_decode_mxfp4": (f32, [C.c_uint8]),
        "oracle_mxfp4_integer": (C.c_int32, [C.c_uint8]),
        "oracle_expf_glibc": (f32, [f32]),
        "oracle_expf_restated": (f32, [f32]),
        "oracle_adjacent_to_split": (None, [vp, vp]),
        "oracle_split_to_adjacent": (None, [vp, vp]),
        "oracle_expf_check": (u64, [u32, u32, i32, C.POINTER(u32)]),
        "oracle_quantize_residual_q8": (i32, [vp, sz, vp]),
        "oracle_quantize_q8": (i32, [vp, sz, vp]),
        "oracle_block_dots": (None, [vp, sz, sz, vp, vp]),
        "oracle_mxfp4_matmul": (i32, [vp, sz, sz, sz, i32, i32, vp, sz, sz, sz, sz, vp, sz, vp, sz, sz]),
        "oracle_mxfp4_matmul_auto": (i32, [vp, sz, sz, i32, vp, sz, vp, vp, sz, i32]),
        "oracle_has_avx2": (i32, []),
        "oracle_has_avx512_vnni": (i32, []),
        "oracle_mxfp4_matmul_lane": (i32, [vp, sz, sz, i32, vp, sz, vp, vp, sz, i32, i32]),
        "oracle_bench_weights": (None, [sz, sz, vp]),
        "oracle_bench_residual": (None, [sz, sz, vp]),
        "oracle_bench_bias": (None, [sz, vp]),
        "oracle_pack_x8": (None, [vp, sz, sz, vp]),
        "oracle_bf16_matvec": (None, [vp, sz, sz, vp, vp]),
        "oracle_accumulate_mxfp4_bf16_block": (None, [vp, vp, vp]),
        "oracle_rms_norm": (None, [vp, vp, sz, f32, vp]),
        "oracle_norm_boundary": (None, [vp, vp, sz, f32, vp]),
        "oracle_add_residual": (None, [vp, vp, sz, vp]),
        "oracle_swiglu": (i32, [vp, sz, f32, f32, vp]),
        "oracle_stable_top_k": (None, [vp, sz, sz, vp]),
        "oracle_softmax": (None, [vp, sz, vp]),
        "oracle_combine": (None, [vp, vp, sz, sz, sz, vp]),
        "oracle_moe_batch": (i32, [C.POINTER(OracleLayer), vp, sz, vp, vp, vp, vp, vp, vp, vp, vp, vp, i32, i32]),
        "oracle_moe_batch_ex": (i32, [C.POINTER(OracleLayer), vp, sz, vp, vp, vp, vp, vp, vp, vp, vp, vp, i32, i32, i32]),
        "oracle_moe_batch_full": (i32, [C.POINTER(OracleLayer), vp, sz, vp, vp, vp, vp, vp, vp, vp, vp, vp, i32, i32,
                                        i32, vp]),
        "oracle_stream_hash": (u64, [u64, u64, u64]),
        "oracle_gen_mxfp4": (None, [u64, u64, sz, sz, sz, vp]),
        "oracle_gen_bf16_normal": (None, [u64, u64, sz, f32, f32, vp]),
        "oracle_gen_hidden": (None, [u64, u64, sz, sz, i32, vp]),
        "oracle_gen_bf16_normal_mt": (None, [u64, u64, sz, f32, f32, vp, i32]),
        "oracle_yarn_rope": (i32, [C.POINTER(OracleRope), vp, sz, sz]),
        "oracle_attention": (i32, [vp, vp, vp, sz, sz, vp, sz, sz, sz, vp, C.POINTER(sz), C.POINTER(sz)]),
        "oracle_greedy_token": (i32, [vp, sz, C.POINTER(u32)]),
        "oracle_model_generate": (i32, [C.POINTER(OracleModel), vp, sz, sz, sz, i32, vp, vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


# ---------------------------------------------------------------------------
# Thin numpy helpers.

def bf16_bits(x: float) -> int:
    return lib().oracle_bf16_bits(float(x))


def bf16_round_array(a: np.ndarray) -> np.ndarray:
    """Vectorised half-2.7.1 bf16 round trip (RNE, NaN quieted)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    rb = 0x8000
    up = ((u & rb) != 0) & ((u & (3 * rb - 1)) != 0)
    hi = (u >> 16) + up.astype(np.uint64)
    hi = np.where(nan, (u >> 16) | 0x40, hi)
    return ((hi & 0xFFFF) << 16).astype(np.uint32).view(np.float32)


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def quantize_residual_q8(x: np.ndarray):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(x.size // 32, dtype=RQ8_DTYPE)
    st = lib().oracle_quantize_residual_q8(_p(x), x.size, _p(out))
    return st, out


def quantize_q8(x: np.ndarray):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(x.size // 32, dtype=Q8_DTYPE)
    st = lib().oracle_quantize_q8(_p(x), x.size, _p(out))
    return st, out


def bench_fixtures(n: int, blocks: int, m: int):
    """mxfp4_matrix_bench.rs:524-597 fixtures: canonical, x8, residual, bias."""
    L = lib()
    canonical = np.zeros(n * blocks * 17, dtype=np.uint8)
    L.oracle_bench_weights(n, blocks, _p(canonical))
    x8 = np.zeros_like(canonical)
    L.oracle_pack_x8(_p(canonical), n, blocks, _p(x8))
    residual = np.zeros(m * blocks, dtype=RQ8_DTYPE)
    L.oracle_bench_residual(m, blocks, _p(residual))
    bias = np.zeros(n, dtype=np.float32)
    L.oracle_bench_bias(n, _p(bias))
    return canonical, x8, residual, bias


def pack_x8(canonical: np.ndarray, rows: int, blocks: int) -> np.ndarray:
    out = np.zeros_like(canonical)
    lib().oracle_pack_x8(_p(canonical), rows, blocks, _p(out))
    return out


def mxfp4_matmul(data, rows, blocks, layout, act, m, bias, out_stride=None, kind=2, act_stride=None, out=None,
                 act_bpr=None):
    """Scalar Kernels::mxfp4_matmul; returns (status, output)."""
    out_stride = rows if out_stride is None else out_stride
    act_stride = blocks if act_stride is None else act_stride
    act_bpr = blocks if act_bpr is None else act_bpr
    if out is None:
        out = np.full((m - 1) * out_stride + rows, np.nan, dtype=np.float32)
    st = lib().oracle_mxfp4_matmul(_p(data), data.size, rows, blocks, layout, kind, _p(act), act.size, m, act_bpr,
                                   act_stride, _p(bias), 0 if bias is None else bias.size, _p(out), out.size,
                                   out_stride)
    return st, out


def mxfp4_matmul_auto(data_x8, rows, blocks, act, m, bias, threads=1):
    out = np.full(m * rows, np.nan, dtype=np.float32)
    lib().oracle_mxfp4_matmul_auto(_p(data_x8), rows, blocks, 2, _p(act), m, _p(bias), _p(out), rows, threads)
    return out


def block_dots(canonical, rows, blocks, act):
    out = np.zeros(rows * blocks * 2, dtype=np.int32)
    lib().oracle_block_dots(_p(canonical), rows, blocks, _p(act), _p(out))
    return out.reshape(rows, blocks, 2)


def gen_mxfp4(seed, stream, experts, rows, blocks):
    out = np.zeros(experts * rows * blocks * 17, dtype=np.uint8)
    lib().oracle_gen_mxfp4(seed, stream, experts, rows, blocks, _p(out))
    return out


def gen_bf16_normal(seed, stream, n, mean=0.0, std=1.0):
    out = np.zeros(n, dtype=np.uint16)
    lib().oracle_gen_bf16_normal(seed, stream, n, mean, std, _p(out))
    return out


def gen_hidden(seed, stream, m, h, normalise=True):
    out = np.zeros(m * h, dtype=np.uint16)
    lib().oracle_gen_hidden(seed, stream, m, h, 1 if normalise else 0, _p(out))
    return out.reshape(m, h)


def swiglu(gate_up, intermediate, alpha=1.702, limit=7.0):
    g = np.ascontiguousarray(gate_up, dtype=np.float32)
    out = np.zeros(intermediate, dtype=np.float32)
    lib().oracle_swiglu(_p(g), intermediate, alpha, limit, _p(out))
    return out


def stable_top_k(v, k):
    v = np.ascontiguousarray(v, dtype=np.float32)
    out = np.zeros(min(k, v.size), dtype=np.uint32)
    lib().oracle_stable_top_k(_p(v), v.size, k, _p(out))
    return out


def softmax(v):
    v = np.ascontiguousarray(v, dtype=np.float32)
    out = np.zeros_like(v)
    lib().oracle_softmax(_p(v), v.size, _p(out))
    return out


def combine(y, w):
    """The weighted combine of moe_batch (cpu_runner.rs:2959-2999): y [m][k][h]
    f32, w [m][k] f32 -> [m][h] bf16 values."""
    y = np.ascontiguousarray(y, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    m, k, h = y.shape
    out = np.zeros((m, h), np.float32)
    lib().oracle_combine(_p(y), _p(w), m, k, h, _p(out))
    return out


def bf16_matvec(w_bits, x_bits):
    """Kernels::bf16_matvec rows of w [rows][cols] against x [cols], bf16 bits."""
    w = np.ascontiguousarray(w_bits, dtype=np.uint16)
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    out = np.zeros(w.shape[0], np.float32)
    lib().oracle_bf16_matvec(_p(w), w.shape[0], w.shape[1], _p(x), _p(out))
    return out


class MoeLayerHost:
    """Host copies of one MoE layer in the reference's tensor formats."""

    def __init__(self, router_weight, router_bias, gate_up, gate_up_bias, down, down_bias, experts, hidden,
                 intermediate, top_k=4, alpha=1.702, limit=7.0):
        self.router_weight = np.ascontiguousarray(router_weight, dtype=np.uint16)
        self.router_bias = np.ascontiguousarray(router_bias, dtype=np.float32)
        self.gate_up = np.ascontiguousarray(gate_up, dtype=np.uint8)
        self.gate_up_bias = np.ascontiguousarray(gate_up_bias, dtype=np.float32)
        self.down = np.ascontiguousarray(down, dtype=np.uint8)
        self.down_bias = np.ascontiguousarray(down_bias, dtype=np.float32)
        self.experts, self.hidden, self.intermediate, self.top_k = experts, hidden, intermediate, top_k
        self.alpha, self.limit = alpha, limit

    def struct(self):
        s = OracleLayer()
        s.router_weight = self.router_weight.ctypes.data
        s.router_bias = self.router_bias.ctypes.data
        s.gate_up = self.gate_up.ctypes.data
        s.gate_up_bias = self.gate_up_bias.ctypes.data
        s.down = self.down.ctypes.data
        s.down_bias = self.down_bias.ctypes.data
        s.experts, s.hidden, s.intermediate, s.top_k = self.experts, self.hidden, self.intermediate, self.top_k
        s.alpha, s.limit = self.alpha, self.limit
        return s


PROJECTION_RESIDUAL_Q8, PROJECTION_Q8, PROJECTION_EXACT_BF16 = 0, 1, 2
UNAVAILABLE_BACKEND = 5

# Expert-matmul lanes of moe_batch: the scalar matmul, the faithful Auto lane,
# and the reference's forced AVX2 4x8 / AVX-512 8x8 panel lanes.
LANE_SCALAR, LANE_AUTO, LANE_AVX2_4X8, LANE_AVX512_8X8 = 0, 1, 4, 8


def fastest_lane() -> int:
    """The forced panel lane this host runs (every lane is bit-identical)."""
    if lib().oracle_has_avx512_vnni():
        return LANE_AVX512_8X8
    return LANE_AVX2_4X8 if lib().oracle_has_avx2() else LANE_SCALAR


def mxfp4_matmul_lane(data_x8, rows, blocks, act, m, bias, lane, threads=1, kind=2):
    """A forced panel lane (Mxfp4MatmulBackend::Avx2 / Avx512Vnni) on x8 weights."""
    out = np.full(m * rows, np.nan, dtype=np.float32)
    st = lib().oracle_mxfp4_matmul_lane(_p(data_x8), rows, blocks, kind, _p(act), m, _p(bias), _p(out), rows, lane,
                                        threads)
    if st != OK:
        raise RuntimeError(f"oracle lane {lane}: status {st}")
    return out


def moe_batch(layer: MoeLayerHost, x_bf16: np.ndarray, injected_logits=None, trace=False, auto_lane=False,
              threads=1, projection=PROJECTION_RESIDUAL_Q8, lane=None):
    """CpuModel::moe_batch restated; returns a dict of outputs (or raises).
    projection selects CpuExpertProjection (residual-Q8, Q8, exact-BF16);
    lane the expert-matmul lane (LANE_*; auto_lane=True is LANE_AUTO)."""
    if lane is None:
        lane = LANE_AUTO if auto_lane else LANE_SCALAR
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    m = x.shape[0]
    E, H, I, K = layer.experts, layer.hidden, layer.intermediate, layer.top_k
    res = {
        "router_logits": np.zeros((m, E), np.float32),
        "selected": np.zeros((m, K), np.uint32),
        "routing_weights": np.zeros((m, K), np.float32),
        "output": np.zeros((m, H), np.float32),
        "route_order": np.zeros(m * K, np.uint32),
        "output_unrounded": np.zeros((m, H), np.float32),  # the combine's sum before its bf16 round trip
    }
    if trace:
        res["gate_up"] = np.zeros((m, K, 2 * I), np.float32)
        res["swiglu"] = np.zeros((m, K, I), np.float32)
        res["down"] = np.zeros((m, K, H), np.float32)
    inj = None if injected_logits is None else np.ascontiguousarray(injected_logits, dtype=np.float32)
    s = layer.struct()
    st = lib().oracle_moe_batch_full(C.byref(s), _p(x), m, _p(inj), _p(res["router_logits"]), _p(res["selected"]),
                                     _p(res["routing_weights"]), _p(res["output"]), _p(res["route_order"]),
                                     _p(res.get("gate_up")), _p(res.get("swiglu")), _p(res.get("down")),
                                     lane, threads, projection, _p(res["output_unrounded"]))
    res["status"] = st
    return res


def synthetic_layer(seed: int, layer: int, experts=32, hidden=2880, intermediate=2880, top_k=4,
                    with_experts=True) -> MoeLayerHost:
    """The config-0 layer distribution: router bf16 N(0, 0.02) plus bf16 bias,
    MXFP4 codes uniform over 16 codes, E8M0 exponent uniform in [-8, -4],
    expert biases bf16 N(0, 0.02). Streams are keyed by layer so any layer can
    be regenerated independently (the GPU library uses the same MXFP4 streams).
    """
    base = 16 * layer
    rw = gen_bf16_normal(seed, base + 0, experts * hidden, 0.0, 0.02)
    rb = bf16_to_f32(gen_bf16_normal(seed, base + 1, experts, 0.0, 0.02))
    gub = bf16_to_f32(gen_bf16_normal(seed, base + 2, experts * 2 * intermediate, 0.0, 0.02))
    db = bf16_to_f32(gen_bf16_normal(seed, base + 3, experts * hidden, 0.0, 0.02))
    if with_experts:
        gu = gen_mxfp4(seed, base + 4, experts, 2 * intermediate, hidden // 32)
        dn = gen_mxfp4(seed, base + 5, experts, hidden, intermediate // 32)
    else:
        gu = np.zeros(0, np.uint8)
        dn = np.zeros(0, np.uint8)
    return MoeLayerHost(rw, rb, gu, gub, dn, db, experts, hidden, intermediate, top_k)


MXFP4_STREAM_GATE_UP = 4
MXFP4_STREAM_DOWN = 5


# ---------------------------------------------------------------------------
# The MoE half of a decoder layer around moe_batch (forward_layer_batch,
# cpu_runner.rs:2519-2553).

def rms_norm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """Kernels::rms_norm of one f32 row (lib.rs:699-730)."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.zeros_like(x)
    lib().oracle_rms_norm(_p(x), _p(w), x.size, np.float32(eps), _p(out))
    return out


def norm_boundary(x_bf16: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """norm_boundary (cpu_runner.rs:2680-2687) of every row: bf16 bits out."""
    x = np.ascontiguousarray(x_bf16, np.uint16)
    w = np.ascontiguousarray(w, np.float32)
    out = np.zeros_like(x)
    for r in range(x.shape[0]):
        lib().oracle_norm_boundary(_p(x[r]), _p(w), x.shape[1], np.float32(eps), _p(out[r]))
    return out


def add_residual(residual_bf16: np.ndarray, update: np.ndarray) -> np.ndarray:
    """add_residual (cpu_runner.rs:3732-3738): bf16 bits of residual + update."""
    r = np.ascontiguousarray(residual_bf16, np.uint16)
    u = np.ascontiguousarray(update, np.float32)
    out = np.zeros_like(r)
    lib().oracle_add_residual(_p(r), _p(u), r.size, _p(out))
    return out


def moe_residual(layer: "MoeLayerHost", residual_bf16: np.ndarray, norm_weight: np.ndarray, eps: float,
                 injected_logits=None, projection=PROJECTION_RESIDUAL_Q8) -> dict:
    """norm_boundary -> moe_batch -> add_residual, as forward_layer_batch
    runs them; moe_batch's outputs plus normalized and next_residual."""
    normalized = norm_boundary(residual_bf16, norm_weight, eps)
    res = moe_batch(layer, normalized, injected_logits=injected_logits, projection=projection)
    res["normalized"] = normalized
    if res["status"] == OK:
        res["next_residual"] = add_residual(residual_bf16, res["output"])
    return res


# ---------------------------------------------------------------------------
# The dense path around the block (cpu_runner.rs), test infrastructure only.

def rope_struct(head_dim, theta=150000.0, yarn=True, factor=32.0, original_max=4096, beta_fast=32.0,
                beta_slow=1.0, truncate=False) -> OracleRope:
    return OracleRope(head_dim, theta, 1 if yarn else 0, factor, original_max, beta_fast, beta_slow,
                      1 if truncate else 0)


def yarn_rope(rope: OracleRope, values, heads: int, position: int) -> np.ndarray:
    v = np.array(values, dtype=np.float32)
    lib().oracle_yarn_rope(C.byref(rope), _p(v), heads, position)
    return v


def attention(query, keys, values, window, sinks, heads, kv_heads, head_dim):
    """attention_one over a cache of capacity `window` after appending every
    key/value row; returns (output, cache len, cache start_position)."""
    q = np.ascontiguousarray(query, dtype=np.float32)
    k = np.ascontiguousarray(keys, dtype=np.uint16)
    v = np.ascontiguousarray(values, dtype=np.uint16)
    s = np.ascontiguousarray(sinks, dtype=np.float32)
    out = np.zeros(heads * head_dim, np.float32)
    n, start = C.c_size_t(), C.c_size_t()
    tokens = k.size // (kv_heads * head_dim)
    lib().oracle_attention(_p(q), _p(k), _p(v), tokens, window, _p(s), heads, kv_heads, head_dim, _p(out),
                           C.byref(n), C.byref(start))
    return out, n.value, start.value


def greedy_token(logits):
    v = np.ascontiguousarray(logits, dtype=np.float32)
    t = C.c_uint32()
    st = lib().oracle_greedy_token(_p(v), v.size, C.byref(t))
    return None if st else t.value


def gen_bf16_normal_mt(seed, stream, n, mean=0.0, std=1.0, threads=8):
    out = np.zeros(n, dtype=np.uint16)
    lib().oracle_gen_bf16_normal_mt(seed, stream, n, mean, std, _p(out), threads)
    return out


class ModelHost:
    """A GPT-OSS model in the reference's host formats: config dict (the
    gossmx_model_config fields), embedding/lm_head bf16 [vocab][hidden], final
    norm f32, and per layer the dense tensors plus a MoeLayerHost."""

    def __init__(self, config: dict, embedding, final_norm, lm_head, layers):
        self.config = dict(config)
        self.embedding = np.ascontiguousarray(embedding, dtype=np.uint16)
        self.final_norm = np.ascontiguousarray(final_norm, dtype=np.float32)
        self.lm_head = np.ascontiguousarray(lm_head, dtype=np.uint16)
        self.layers = layers

    def struct(self):
        c = self.config
        m = OracleModel()
        for k in ("vocab", "hidden", "layers", "heads", "kv_heads", "head_dim", "sliding_window", "context_cap"):
            setattr(m, k, c[k])
        m.rms_norm_eps = c["rms_norm_eps"]
        m.rope = rope_struct(c["head_dim"], c["rope_theta"], bool(c["rope_yarn"]), c["rope_factor"],
                             c["rope_original_max_positions"], c.get("rope_beta_fast", 32.0),
                             c.get("rope_beta_slow", 1.0), bool(c.get("rope_truncate", 0)))
        m.embedding, m.final_norm, m.lm_head = (self.embedding.ctypes.data, self.final_norm.ctypes.data,
                                                self.lm_head.ctypes.data)
        table = (OracleDenseLayer * len(self.layers))()
        keep = []
        for i, L in enumerate(self.layers):
            d = table[i]
            for name in ("input_norm", "q_bias", "k_bias", "v_bias", "o_bias", "sinks", "post_attention_norm"):
                a = np.ascontiguousarray(L[name], dtype=np.float32)
                keep.append(a)
                setattr(d, name, a.ctypes.data)
            for name in ("q_weight", "k_weight", "v_weight", "o_weight"):
                a = np.ascontiguousarray(L[name], dtype=np.uint16)
                keep.append(a)
                setattr(d, name, a.ctypes.data)
            d.sliding = 1 if L["sliding"] else 0
            d.moe = L["moe_host"].struct()
        m.layer = table
        return m, (table, keep)


def model_generate(model: ModelHost, prompt, decode_steps, prefill_chunk=0, threads=8):
    """prefill_layer_major then greedy decodes; returns (status, tokens, logits)."""
    p = np.ascontiguousarray(prompt, dtype=np.uint32)
    tokens = np.zeros(decode_steps + 1, np.uint32)
    logits = np.zeros((decode_steps + 1, model.config["vocab"]), np.float32)
    s, keep = model.struct()
    st = lib().oracle_model_generate(C.byref(s), _p(p), p.size, prefill_chunk, decode_steps, threads, _p(tokens),
                                     _p(logits))
    return st, tokens, logits
