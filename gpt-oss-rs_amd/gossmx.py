"""Host-side mirror of gpt-oss-rs's MXFP4 MoE interfaces over libgossmx.so.

`mxfp4_matmul` mirrors `Kernels::mxfp4_matmul` with a residual-Q8 or Q8
`Mxfp4MatmulProblem` (crates/gpt-oss-cpu-kernels/src/matmul.rs:297-414), and
`MoeLayer.moe_batch` mirrors `CpuModel::moe_batch`
(crates/gpt-oss-model-runner/src/cpu_runner.rs:2794-3013), returning one
`MoeStep` per input row like `CpuMoeStep` (:569-575). Errors raise
`GossmxError` carrying the `KernelError`-like status code.

The HIP library is required: importing works anywhere, but every call that
needs the library raises if libgossmx.so is missing; there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import os
import re
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# GOSSMX_LIB names another build of the library (the host-sanitized test
# build, for instance); by default the in-tree libgossmx.so.
LIB_PATH = os.environ.get("GOSSMX_LIB") or os.path.join(HERE, "libgossmx.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "gossmx.h")

OK = 0
ERR_INVALID_ARGUMENT = 1
ERR_UNSUPPORTED = 2
ERR_INVALID_DIMENSIONS = 3
ERR_NON_FINITE_INPUT = 4
ERR_UNAVAILABLE_BACKEND = 5
ERR_DEVICE = 6
ERR_OUT_OF_MEMORY = 7
ERR_NON_FINITE_LOGITS = 8
ERR_INJECTED_FAULT = 9
ERR_BAD_FILE = 10
ERR_CIRCUIT_OPEN = 11

FAULT_NONE = 0
FAULT_INJECTED = 1   # GOSSMX_ERR_INJECTED_FAULT, the breaker stays closed
FAULT_DEVICE = 2     # GOSSMX_ERR_DEVICE, opens the breaker
FAULT_FLAG = 3       # the call runs; its device error flag is raised, reported where the flags are read

LAYOUT_CANONICAL_V1 = 1
LAYOUT_X8_SPLIT_V2 = 2
ACT_Q8 = 1
ACT_RESIDUAL_Q8 = 2
MEM_HOST = 0
MEM_DEVICE = 1

OPS = ("router_routing", "dispatch", "gate_up", "down", "weighting", "matmul", "post_attention_norm")
ROLES = ("none", "router", "gate_up", "down")
KERNELS = ("route", "gemv", "gemm", "exact", "combine")
PHASE_UNKNOWN, PHASE_PREFILL, PHASE_DECODE = 0, 1, 2
PHASES = ("unknown", "prefill", "decode")
PROFILE_CAPACITY = 65536

# The reference's activation records (lib.rs:732-742), 36 and 72 bytes.
Q8_DTYPE = np.dtype([("scale", "<f4"), ("values", "i1", (32,))])
RQ8_DTYPE = np.dtype([("primary", Q8_DTYPE), ("residual", Q8_DTYPE)])


class GossmxError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"gossmx status {status}: {message}")
        self.status = status
        self.message = message


class MatmulProblem(C.Structure):
    _fields_ = [
        ("weights", C.c_void_p), ("expert", C.c_size_t), ("activation_kind", C.c_int),
        ("activations", C.c_void_p), ("activations_len", C.c_size_t), ("m", C.c_size_t),
        ("blocks_per_row", C.c_size_t), ("row_stride", C.c_size_t), ("bias", C.c_void_p),
        ("bias_len", C.c_size_t), ("output", C.c_void_p), ("output_len", C.c_size_t),
        ("output_stride", C.c_size_t), ("memory", C.c_int),
    ]


PROJECTION_RESIDUAL_Q8 = 0   # CpuExpertProjection::ResidualQ8 (the default)
PROJECTION_Q8 = 1            # CpuExpertProjection::Q8
PROJECTION_EXACT_BF16 = 2    # CpuExpertProjection::ExactBf16


class MoeConfig(C.Structure):
    _fields_ = [("experts", C.c_size_t), ("hidden", C.c_size_t), ("intermediate", C.c_size_t),
                ("top_k", C.c_size_t), ("alpha", C.c_float), ("limit", C.c_float), ("projection", C.c_int)]


class RepackInfo(C.Structure):
    _fields_ = [("format_version", C.c_uint32), ("layout_version", C.c_uint32), ("experts", C.c_size_t),
                ("rows", C.c_size_t), ("blocks", C.c_size_t), ("records", C.c_size_t),
                ("payload_offset", C.c_size_t), ("payload_bytes", C.c_size_t)]


class TensorInfo(C.Structure):
    _fields_ = [("dtype", C.c_char * 16), ("rank", C.c_size_t), ("shape", C.c_size_t * 8), ("offset", C.c_size_t),
                ("bytes", C.c_size_t)]


class MoeIo(C.Structure):
    _fields_ = [("x", C.c_void_p), ("m", C.c_size_t), ("injected_logits", C.c_void_p),
                ("router_logits", C.c_void_p), ("selected", C.c_void_p), ("routing_weights", C.c_void_p),
                ("output", C.c_void_p), ("route_order", C.c_void_p), ("trace_down", C.c_void_p),
                ("memory", C.c_int), ("trace_gate_up", C.c_void_p), ("trace_swiglu", C.c_void_p),
                ("output_unrounded", C.c_void_p)]


class ProfileRecord(C.Structure):
    _fields_ = [("op", C.c_int), ("launches", C.c_uint64), ("total_ms", C.c_double)]


class ProfileEvent(C.Structure):
    """gossmx_profile_event: one profiled stage (CpuExecutionProfileRecord)."""
    _fields_ = [("sequence", C.c_uint64), ("op", C.c_int32), ("role", C.c_int32), ("kernel", C.c_int32),
                ("layer", C.c_int32), ("phase", C.c_int32), ("memory", C.c_int32), ("m", C.c_uint32),
                ("n", C.c_uint32), ("k", C.c_uint32), ("routes", C.c_uint32), ("rows_per_item", C.c_uint32),
                ("reserved", C.c_uint32), ("start_ns", C.c_uint64), ("duration_ns", C.c_uint64),
                ("scratch_bytes", C.c_uint64), ("resident_bytes", C.c_uint64)]


class Stats(C.Structure):
    """gossmx_stats: the process-wide projection, transfer and residency counters."""
    _fields_ = [(name, C.c_uint64) for name in (
        "projections_ok", "projections_failed", "projections_refused", "projections_rejected",
        "weights_bias_uploaded_bytes", "activation_bytes", "output_bytes", "resident_bytes",
        "resident_high_water_bytes", "resident_cap_bytes", "capacity_refusals", "repack_cache_hits",
        "repack_cache_misses")] + [("circuit_open", C.c_int32), ("reserved", C.c_int32)]


_lib = None


class ModelConfig(C.Structure):
    """gossmx_model_config (CpuGptOssConfig plus the sequence's context cap)."""
    _fields_ = [("vocab", C.c_size_t), ("hidden", C.c_size_t), ("layers", C.c_size_t), ("heads", C.c_size_t),
                ("kv_heads", C.c_size_t), ("head_dim", C.c_size_t), ("sliding_window", C.c_size_t),
                ("context_cap", C.c_size_t), ("rms_norm_eps", C.c_float), ("rope_theta", C.c_double),
                ("rope_yarn", C.c_int), ("rope_factor", C.c_double), ("rope_original_max_positions", C.c_size_t),
                ("rope_beta_fast", C.c_double), ("rope_beta_slow", C.c_double), ("rope_truncate", C.c_int),
                ("threads", C.c_size_t)]


class DenseLayer(C.Structure):
    """gossmx_dense_layer: one decoder layer's dense tensors and its MoE block."""
    _fields_ = [("input_norm", C.c_void_p), ("q_weight", C.c_void_p), ("q_bias", C.c_void_p),
                ("k_weight", C.c_void_p), ("k_bias", C.c_void_p), ("v_weight", C.c_void_p), ("v_bias", C.c_void_p),
                ("o_weight", C.c_void_p), ("o_bias", C.c_void_p), ("sinks", C.c_void_p),
                ("post_attention_norm", C.c_void_p), ("sliding", C.c_int), ("moe", C.c_void_p)]


# GPT-OSS-20B's attention and RoPE configuration (config.json of the checkpoint).
GPT_OSS_20B = dict(vocab=201088, hidden=2880, layers=24, heads=64, kv_heads=8, head_dim=64, sliding_window=128,
                   rms_norm_eps=1e-5, rope_theta=150000.0, rope_yarn=1, rope_factor=32.0,
                   rope_original_max_positions=4096, rope_beta_fast=32.0, rope_beta_slow=1.0, rope_truncate=0)


def model_config(context_cap: int = 4096, threads: int = 0, **fields) -> ModelConfig:
    """A ModelConfig from keyword fields (rope defaults as CpuRopeScaling's serde defaults)."""
    c = ModelConfig()
    c.rope_beta_fast, c.rope_beta_slow, c.context_cap, c.threads = 32.0, 1.0, context_cap, threads
    for k, v in fields.items():
        setattr(c, k, v)
    return c


def header_symbols() -> list[str]:
    """Every function the public header declares."""
    with open(HEADER) as fh:
        text = fh.read()
    return sorted(set(re.findall(r"\b(gossmx_[a-z0-9_]+)\s*\(", text)))


def load():
    """Loads libgossmx.so; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise GossmxError(ERR_UNAVAILABLE_BACKEND, f"{LIB_PATH} is not built (run gpt-oss-rs_amd/build.py)")
    L = C.CDLL(LIB_PATH)
    vp, sz, i32, u64 = C.c_void_p, C.c_size_t, C.c_int, C.c_uint64
    pp = C.POINTER(C.c_void_p)
    sig = {
        "gossmx_last_error": (C.c_char_p, []),
        "gossmx_version": (i32, []),
        "gossmx_device_count": (i32, [C.POINTER(C.c_int)]),
        "gossmx_ctx_create": (i32, [i32, vp, pp]),
        "gossmx_ctx_destroy": (None, [vp]),
        "gossmx_ctx_set_stream": (i32, [vp, vp]),
        "gossmx_ctx_stream": (vp, [vp]),
        "gossmx_synchronize": (i32, [vp]),
        "gossmx_malloc": (i32, [vp, sz, pp]),
        "gossmx_free": (i32, [vp, vp]),
        "gossmx_memcpy_h2d": (i32, [vp, vp, vp, sz]),
        "gossmx_memcpy_d2h": (i32, [vp, vp, vp, sz]),
        "gossmx_weights_upload": (i32, [vp, vp, sz, sz, sz, sz, i32, pp]),
        "gossmx_weights_generate": (i32, [vp, u64, u64, sz, sz, sz, pp]),
        "gossmx_weights_export": (i32, [vp, vp, vp, sz]),
        "gossmx_weights_shape": (i32, [vp, C.POINTER(sz), C.POINTER(sz), C.POINTER(sz)]),
        "gossmx_weights_device_bytes": (sz, [vp]),
        "gossmx_weights_destroy": (None, [vp]),
        "gossmx_mxfp4_matmul": (i32, [vp, C.POINTER(MatmulProblem)]),
        "gossmx_mxfp4_matmul_check": (i32, [C.POINTER(MatmulProblem), sz, sz, sz]),
        "gossmx_mxfp4_scratch_requirement": (i32, [C.POINTER(MatmulProblem), C.POINTER(sz), C.POINTER(sz)]),
        "gossmx_circuit_is_open": (i32, []),
        "gossmx_circuit_reset": (None, []),
        "gossmx_ctx_fast_path": (i32, [vp, C.POINTER(C.c_int)]),
        "gossmx_layer_create": (i32, [vp, C.POINTER(MoeConfig), vp, vp, vp, vp, vp, vp, pp]),
        "gossmx_layer_destroy": (None, [vp]),
        "gossmx_moe_forward": (i32, [vp, vp, C.POINTER(MoeIo)]),
        "gossmx_moe_forward_noalloc": (i32, [vp, vp, C.POINTER(MoeIo)]),
        "gossmx_repack_inspect": (i32, [C.c_char_p, C.POINTER(RepackInfo), C.c_char_p, sz]),
        "gossmx_weights_load_repack": (i32, [vp, C.c_char_p, C.POINTER(vp)]),
        "gossmx_weights_save_repack": (i32, [vp, vp, C.c_char_p, C.c_char_p, C.c_char_p, C.POINTER(C.c_char_p), sz]),
        "gossmx_repack_cache_key": (i32, [C.c_char_p, C.POINTER(sz), i32, C.c_char_p, C.POINTER(C.c_char_p), sz,
                                          C.c_char_p]),
        "gossmx_safetensors_find": (i32, [C.c_char_p, C.c_char_p, C.POINTER(TensorInfo)]),
        "gossmx_weights_from_safetensors": (i32, [vp, C.POINTER(C.c_char_p), sz, C.c_char_p, C.c_char_p,
                                                  C.POINTER(vp)]),
        "gossmx_weights_open_or_create": (i32, [vp, C.c_char_p, C.c_char_p, C.POINTER(C.c_char_p), sz,
                                                C.POINTER(C.c_char_p), sz, C.c_char_p, C.c_char_p, C.POINTER(vp)]),
        "gossmx_moe_forward_residual": (i32, [vp, vp, C.POINTER(MoeIo), vp, C.c_float, vp]),
        "gossmx_profile_enable": (i32, [vp, i32]),
        "gossmx_profile_read": (i32, [vp, C.POINTER(ProfileRecord), sz, C.POINTER(sz)]),
        "gossmx_profile_reset": (i32, [vp]),
        "gossmx_profile_tag": (i32, [vp, i32, i32]),
        "gossmx_profile_events": (i32, [vp, C.POINTER(ProfileEvent), sz, C.POINTER(sz), C.POINTER(sz),
                                        C.POINTER(u64)]),
        "gossmx_stats_read": (i32, [C.POINTER(Stats)]),
        "gossmx_stats_reset": (None, []),
        "gossmx_set_resident_cap": (i32, [u64]),
        "gossmx_inject_fault": (i32, [vp, i32]),
        "gossmx_capture_begin": (i32, [vp]),
        "gossmx_capture_end": (i32, [vp, pp]),
        "gossmx_graph_launch": (i32, [vp, vp]),
        "gossmx_graph_destroy": (None, [vp]),
        "gossmx_selftest": (i32, [vp]),
        "gossmx_selftest_bf16_exhaustive": (i32, [vp, C.POINTER(u64)]),
        "gossmx_model_create": (i32, [vp, C.POINTER(ModelConfig), vp, vp, vp, C.POINTER(DenseLayer), pp]),
        "gossmx_model_destroy": (None, [vp]),
        "gossmx_model_reset": (i32, [vp]),
        "gossmx_model_prefill": (i32, [vp, vp, sz, vp]),
        "gossmx_model_append": (i32, [vp, vp, sz, vp]),
        "gossmx_model_decode": (i32, [vp, C.c_uint32, vp]),
        "gossmx_model_position": (i32, [vp, C.POINTER(sz)]),
        "gossmx_model_cache": (i32, [vp, sz, C.POINTER(sz), C.POINTER(sz)]),
        "gossmx_model_times": (i32, [vp, C.POINTER(C.c_double), C.POINTER(C.c_double)]),
        "gossmx_greedy_token": (i32, [vp, sz, C.POINTER(C.c_uint32)]),
        "gossmx_yarn_rope": (i32, [C.POINTER(ModelConfig), vp, sz, sz]),
        "gossmx_attention": (i32, [vp, vp, vp, sz, sz, vp, sz, sz, sz, vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def _check(status: int):
    if status != OK:
        raise GossmxError(status, load().gossmx_last_error().decode(errors="replace"))


def _ptr(a):
    if a is None:
        return None
    if isinstance(a, int):
        return a
    if hasattr(a, "data_ptr"):  # torch tensor on the device
        return a.data_ptr()
    return a.ctypes.data_as(C.c_void_p).value


def circuit_is_open() -> bool:
    """The process-wide circuit breaker (XeProjectionEngine::circuit_is_open)."""
    return bool(load().gossmx_circuit_is_open())


def circuit_reset():
    load().gossmx_circuit_reset()


def stats() -> dict:
    """The process-wide counters (gossmx_stats_read): projections by result,
    transfer bytes by direction, resident bytes and the cap."""
    st = Stats()
    _check(load().gossmx_stats_read(C.byref(st)))
    return {name: int(getattr(st, name)) for name, _ in Stats._fields_ if name != "reserved"}


def stats_reset():
    load().gossmx_stats_reset()


def set_resident_cap(nbytes: int):
    """Caps the device bytes of live weights and layers (0: no cap)."""
    _check(load().gossmx_set_resident_cap(int(nbytes)))


def device_count() -> int:
    n = C.c_int(0)
    _check(load().gossmx_device_count(C.byref(n)))
    return n.value


class Context:
    """One device and one in-order stream (CpuExecutionContext analogue)."""

    def __init__(self, device: int = 0, stream: int | None = None):
        self._h = C.c_void_p()
        _check(load().gossmx_ctx_create(device, stream, C.byref(self._h)))
        self.device = device

    @property
    def handle(self):
        return self._h

    @property
    def stream(self) -> int:
        return load().gossmx_ctx_stream(self._h)

    def set_stream(self, stream: int):
        _check(load().gossmx_ctx_set_stream(self._h, stream))

    def synchronize(self):
        _check(load().gossmx_synchronize(self._h))

    def selftest(self):
        _check(load().gossmx_selftest(self._h))

    def inject_fault(self, armed: bool | int = True):
        """Arms the fault hook of the next projection call: True or
        FAULT_INJECTED (a model error), FAULT_DEVICE (a device fault that
        opens the circuit breaker), FAULT_FLAG (the call runs with its device
        error flag raised: GOSSMX_ERR_DEVICE where the flags are next read),
        False or FAULT_NONE (disarm)."""
        mode = int(armed) if not isinstance(armed, bool) else (FAULT_INJECTED if armed else FAULT_NONE)
        _check(load().gossmx_inject_fault(self._h, mode))

    def bf16_exhaustive_mismatches(self) -> int:
        """bf16 rounding on all 2^32 f32 patterns against half's rounding."""
        n = C.c_uint64(0)
        _check(load().gossmx_selftest_bf16_exhaustive(self._h, C.byref(n)))
        return int(n.value)

    def fast_path(self) -> bool:
        """Whether the GEMMs may take the scaled-conversion fast path (the
        self-test at creation found the dirty-operand conversion exact)."""
        v = C.c_int(0)
        _check(load().gossmx_ctx_fast_path(self._h, C.byref(v)))
        return bool(v.value)

    def profile(self, enabled: bool = True):
        _check(load().gossmx_profile_enable(self._h, 1 if enabled else 0))

    def profile_reset(self):
        _check(load().gossmx_profile_reset(self._h))

    def profile_read(self) -> dict:
        recs = (ProfileRecord * len(OPS))()
        n = C.c_size_t(0)
        _check(load().gossmx_profile_read(self._h, recs, len(OPS), C.byref(n)))
        return {OPS[r.op]: {"launches": int(r.launches), "total_ms": float(r.total_ms)} for r in recs[:n.value]}

    def profile_tag(self, layer: int = -1, phase: int = PHASE_UNKNOWN):
        _check(load().gossmx_profile_tag(self._h, layer, phase))

    def profile_events(self, capacity: int | None = None) -> tuple[list[dict], int]:
        """The per-stage records kept since the last reset, oldest first, and
        the number dropped past the context's capacity."""
        avail, written, dropped = C.c_size_t(0), C.c_size_t(0), C.c_uint64(0)
        _check(load().gossmx_profile_events(self._h, None, 0, C.byref(written), C.byref(avail), C.byref(dropped)))
        cap = avail.value if capacity is None else min(capacity, avail.value)
        recs = (ProfileEvent * max(cap, 1))()
        _check(load().gossmx_profile_events(self._h, recs, cap, C.byref(written), C.byref(avail), C.byref(dropped)))
        out = []
        for r in recs[:written.value]:
            ev = {name: int(getattr(r, name)) for name, _ in ProfileEvent._fields_ if name != "reserved"}
            ev["op"] = OPS[r.op]
            ev["role"] = ROLES[r.role]
            ev["kernel"] = KERNELS[r.kernel]
            ev["phase"] = PHASES[r.phase]
            ev["memory"] = "device" if r.memory == MEM_DEVICE else "host"
            out.append(ev)
        return out, int(dropped.value)

    def capture_begin(self):
        _check(load().gossmx_capture_begin(self._h))

    def capture_end(self) -> "Graph":
        h = C.c_void_p()
        _check(load().gossmx_capture_end(self._h, C.byref(h)))
        return Graph(self, h)

    def malloc(self, nbytes: int) -> int:
        p = C.c_void_p()
        _check(load().gossmx_malloc(self._h, nbytes, C.byref(p)))
        return p.value

    def free(self, ptr: int):
        _check(load().gossmx_free(self._h, ptr))

    def h2d(self, dst: int, src: np.ndarray):
        src = np.ascontiguousarray(src)
        _check(load().gossmx_memcpy_h2d(self._h, dst, _ptr(src), src.nbytes))

    def d2h(self, dst: np.ndarray, src: int):
        _check(load().gossmx_memcpy_d2h(self._h, _ptr(dst), src, dst.nbytes))

    def close(self):
        if self._h:
            load().gossmx_ctx_destroy(self._h)
            self._h = C.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


class Graph:
    """A recorded sequence of device-memory calls (gossmx_capture_*)."""

    def __init__(self, ctx: Context, handle: C.c_void_p):
        self.ctx = ctx
        self._h = handle

    def launch(self):
        _check(load().gossmx_graph_launch(self.ctx.handle, self._h))

    def close(self):
        if self._h:
            load().gossmx_graph_destroy(self._h)
            self._h = C.c_void_p()


class Weights:
    """Resident MXFP4 tensor [experts][rows][blocks] in the GPU layout."""

    def __init__(self, ctx: Context, handle: C.c_void_p):
        self.ctx = ctx
        self._h = handle
        e, r, b = C.c_size_t(), C.c_size_t(), C.c_size_t()
        _check(load().gossmx_weights_shape(handle, C.byref(e), C.byref(r), C.byref(b)))
        self.experts, self.rows, self.blocks = e.value, r.value, b.value

    @classmethod
    def upload(cls, ctx: Context, data: np.ndarray, experts: int, rows: int, blocks: int,
               layout: int = LAYOUT_CANONICAL_V1) -> "Weights":
        data = np.ascontiguousarray(data, dtype=np.uint8)
        h = C.c_void_p()
        _check(load().gossmx_weights_upload(ctx.handle, _ptr(data), data.size, experts, rows, blocks, layout,
                                            C.byref(h)))
        return cls(ctx, h)

    @classmethod
    def generate(cls, ctx: Context, seed: int, stream: int, experts: int, rows: int, blocks: int) -> "Weights":
        h = C.c_void_p()
        _check(load().gossmx_weights_generate(ctx.handle, seed, stream, experts, rows, blocks, C.byref(h)))
        return cls(ctx, h)

    @property
    def handle(self):
        return self._h

    def device_bytes(self) -> int:
        return load().gossmx_weights_device_bytes(self._h)

    def export_canonical(self) -> np.ndarray:
        out = np.zeros(self.experts * self.rows * self.blocks * 17, np.uint8)
        _check(load().gossmx_weights_export(self.ctx.handle, self._h, _ptr(out), out.size))
        return out

    def close(self):
        if self._h:
            load().gossmx_weights_destroy(self._h)
            self._h = C.c_void_p()

    # --- on disk (CpuRepackCache) and from SafeTensors (CpuTensorStore) ---

    @classmethod
    def load_repack(cls, ctx: Context, path: str) -> "Weights":
        """A GOSSMX4 container of layout 1, 2 or 3 (RepackedMxfp4::open)."""
        h = C.c_void_p()
        _check(load().gossmx_weights_load_repack(ctx.handle, os.fsencode(path), C.byref(h)))
        return cls(ctx, h)

    def save_repack(self, path: str, tensor_name: str, model_revision: str, source_hashes=()):
        """This tensor as a layout-3 container, published atomically."""
        hs = _cstrings(source_hashes)
        _check(load().gossmx_weights_save_repack(self.ctx.handle, self._h, os.fsencode(path), tensor_name.encode(),
                                                 model_revision.encode(), hs, len(source_hashes)))

    @classmethod
    def from_safetensors(cls, ctx: Context, shards, blocks_name: str, scales_name: str) -> "Weights":
        sh = _cstrings([os.fsdecode(p) for p in shards])
        h = C.c_void_p()
        _check(load().gossmx_weights_from_safetensors(ctx.handle, sh, len(shards), blocks_name.encode(),
                                                      scales_name.encode(), C.byref(h)))
        return cls(ctx, h)

    @classmethod
    def open_or_create(cls, ctx: Context, cache_root: str, model_revision: str, source_hashes, shards,
                       blocks_name: str, scales_name: str) -> "Weights":
        """CpuRepackCache::open_or_create with the resident layout 3."""
        hs = _cstrings(source_hashes)
        sh = _cstrings([os.fsdecode(p) for p in shards])
        h = C.c_void_p()
        _check(load().gossmx_weights_open_or_create(ctx.handle, os.fsencode(cache_root), model_revision.encode(), hs,
                                                    len(source_hashes), sh, len(shards), blocks_name.encode(),
                                                    scales_name.encode(), C.byref(h)))
        return cls(ctx, h)


def _cstrings(values):
    arr = (C.c_char_p * max(1, len(values)))()
    for i, v in enumerate(values):
        arr[i] = v.encode() if isinstance(v, str) else bytes(v)
    return arr


def repack_cache_key(tensor_name: str, shape, layout: int, model_revision: str, source_hashes=()) -> str:
    """SourceIdentity::cache_key (cpu_repack.rs:92-107)."""
    shp = (C.c_size_t * 3)(*shape)
    key = C.create_string_buffer(65)
    _check(load().gossmx_repack_cache_key(tensor_name.encode(), shp, layout, model_revision.encode(),
                                          _cstrings(source_hashes), len(source_hashes), key))
    return key.value.decode()


def repack_inspect(path: str) -> dict:
    """The validated header of a GOSSMX4 container (no device access)."""
    info = RepackInfo()
    name = C.create_string_buffer(1024)
    _check(load().gossmx_repack_inspect(os.fsencode(path), C.byref(info), name, len(name)))
    d = {k: getattr(info, k) for k, _ in RepackInfo._fields_}
    d["tensor_name"] = name.value.decode()
    return d


def safetensors_find(path: str, name: str) -> dict:
    """One tensor of a SafeTensors shard: dtype, shape, absolute byte range."""
    info = TensorInfo()
    _check(load().gossmx_safetensors_find(os.fsencode(path), name.encode(), C.byref(info)))
    return {"dtype": info.dtype.decode(), "shape": tuple(info.shape[:info.rank]), "offset": info.offset,
            "bytes": info.bytes}


def _problem(weights, expert, activations, m, bias, output, output_stride, kind, row_stride, memory,
             activations_len=None, output_len=None, blocks_per_row=None):
    p = MatmulProblem()
    p.weights = weights.handle.value if isinstance(weights, Weights) else None
    p.expert = expert
    p.activation_kind = kind
    p.activations = _ptr(activations)
    p.activations_len = activations_len if activations_len is not None else int(np.asarray(activations).size)
    p.m = m
    p.blocks_per_row = weights.blocks if blocks_per_row is None else blocks_per_row
    p.row_stride = row_stride
    p.bias = _ptr(bias)
    p.bias_len = 0 if bias is None else (bias.numel() if hasattr(bias, "numel") else int(np.asarray(bias).size))
    p.output = _ptr(output)
    p.output_len = output_len if output_len is not None else (output.numel() if hasattr(output, "numel")
                                                             else int(np.asarray(output).size))
    p.output_stride = output_stride
    p.memory = memory
    return p


def mxfp4_matmul(ctx: Context, weights: Weights, expert: int, activations: np.ndarray, m: int,
                 bias: np.ndarray | None, output: np.ndarray, output_stride: int | None = None,
                 kind: int = ACT_RESIDUAL_Q8, row_stride: int | None = None, blocks_per_row: int | None = None):
    """Kernels::mxfp4_matmul on host arrays (matmul.rs:398-414). `activations`
    are Q8_DTYPE or RQ8_DTYPE records; columns output_stride > rows of each
    output row are left untouched."""
    output_stride = weights.rows if output_stride is None else output_stride
    row_stride = weights.blocks if row_stride is None else row_stride
    p = _problem(weights, expert, activations, m, bias, output, output_stride, kind, row_stride, MEM_HOST,
                 blocks_per_row=blocks_per_row)
    _check(load().gossmx_mxfp4_matmul(ctx.handle, C.byref(p)))
    return output


def mxfp4_matmul_device(ctx: Context, weights: Weights, expert: int, activations, activations_len: int, m: int,
                        bias, output, output_len: int, output_stride: int, kind: int = ACT_RESIDUAL_Q8,
                        row_stride: int | None = None):
    """Same on device pointers (ints or torch tensors); asynchronous."""
    row_stride = weights.blocks if row_stride is None else row_stride
    p = _problem(weights, expert, activations, m, bias, output, output_stride, kind, row_stride, MEM_DEVICE,
                 activations_len=activations_len, output_len=output_len)
    _check(load().gossmx_mxfp4_matmul(ctx.handle, C.byref(p)))


def matmul_check(rows: int, blocks: int, experts: int, activations_len: int, m: int, blocks_per_row: int,
                 row_stride: int, bias_len: int | None, output_len: int, output_stride: int,
                 kind: int = ACT_RESIDUAL_Q8, expert: int = 0) -> int:
    """Status of the problem validation alone (no device needed)."""
    p = MatmulProblem()
    p.weights = None
    p.expert = expert
    p.activation_kind = kind
    p.activations = 1  # non-null placeholder, never dereferenced
    p.activations_len = activations_len
    p.m = m
    p.blocks_per_row = blocks_per_row
    p.row_stride = row_stride
    p.bias = None if bias_len is None else 1
    p.bias_len = 0 if bias_len is None else bias_len
    p.output = 1
    p.output_len = output_len
    p.output_stride = output_stride
    p.memory = MEM_HOST
    return load().gossmx_mxfp4_matmul_check(C.byref(p), rows, blocks, experts)


def scratch_requirement(weights: "Weights", m: int, kind: int = ACT_RESIDUAL_Q8) -> tuple[int, int]:
    """Mxfp4MatmulBackend::scratch_requirement of the GPU backend for a dense
    m-row problem on `weights`: (size, alignment)."""
    p = MatmulProblem()
    p.weights = weights.handle.value
    p.expert = 0
    p.activation_kind = kind
    p.activations = 1
    p.activations_len = m * weights.blocks
    p.m = m
    p.blocks_per_row = weights.blocks
    p.row_stride = weights.blocks
    p.bias = None
    p.bias_len = 0
    p.output = 1
    p.output_len = m * weights.rows
    p.output_stride = weights.rows
    p.memory = MEM_HOST
    size, align = C.c_size_t(), C.c_size_t()
    _check(load().gossmx_mxfp4_scratch_requirement(C.byref(p), C.byref(size), C.byref(align)))
    return size.value, align.value


@dataclass
class MoeStep:
    """CpuMoeStep (cpu_runner.rs:569-575)."""
    router_logits: np.ndarray
    selected_experts: np.ndarray
    routing_weights: np.ndarray
    output: np.ndarray


class MoeLayer:
    """One GPT-OSS MoE layer resident on the device."""

    def __init__(self, ctx: Context, experts: int, hidden: int, intermediate: int, top_k: int,
                 router_weight: np.ndarray, router_bias: np.ndarray, gate_up: Weights, gate_up_bias: np.ndarray,
                 down: Weights, down_bias: np.ndarray, alpha: float = 1.702, limit: float = 7.0,
                 projection: int = PROJECTION_RESIDUAL_Q8):
        self.ctx = ctx
        self.experts, self.hidden, self.intermediate, self.top_k = experts, hidden, intermediate, top_k
        self.projection = projection
        cfg = MoeConfig(experts, hidden, intermediate, top_k, alpha, limit, projection)
        rw = np.ascontiguousarray(router_weight, dtype=np.uint16)
        rb = np.ascontiguousarray(router_bias, dtype=np.float32)
        gb = np.ascontiguousarray(gate_up_bias, dtype=np.float32)
        db = np.ascontiguousarray(down_bias, dtype=np.float32)
        self._h = C.c_void_p()
        _check(load().gossmx_layer_create(ctx.handle, C.byref(cfg), _ptr(rw), _ptr(rb), gate_up.handle, _ptr(gb),
                                          down.handle, _ptr(db), C.byref(self._h)))
        self.gate_up, self.down = gate_up, down

    def forward(self, x_bf16: np.ndarray, injected_logits: np.ndarray | None = None, trace: bool = False,
                unrounded: bool = False) -> dict:
        """All outputs as arrays: router_logits, selected, routing_weights,
        output, route_order (+ trace_down, trace_gate_up, trace_swiglu: the
        CpuExpertTrace vectors of every (row, rank); + output_unrounded: the
        combine's sum before its bf16 round trip). The arrays are allocated
        uninitialized: a successful call writes every element."""
        x = np.ascontiguousarray(x_bf16, dtype=np.uint16)
        m = x.shape[0]
        E, K, H = self.experts, self.top_k, self.hidden
        res = {
            "router_logits": np.empty((m, E), np.float32),
            "selected": np.empty((m, K), np.uint32),
            "routing_weights": np.empty((m, K), np.float32),
            "output": np.empty((m, H), np.float32),
            "route_order": np.empty(m * K, np.uint32),
        }
        if trace:
            res["trace_down"] = np.empty((m, K, H), np.float32)
            res["trace_gate_up"] = np.empty((m, K, 2 * self.intermediate), np.float32)
            res["trace_swiglu"] = np.empty((m, K, self.intermediate), np.float32)
        if unrounded:
            res["output_unrounded"] = np.empty((m, H), np.float32)
        inj = None if injected_logits is None else np.ascontiguousarray(injected_logits, dtype=np.float32)
        io = MoeIo(_ptr(x), m, _ptr(inj), _ptr(res["router_logits"]), _ptr(res["selected"]),
                   _ptr(res["routing_weights"]), _ptr(res["output"]), _ptr(res["route_order"]),
                   _ptr(res.get("trace_down")), MEM_HOST, _ptr(res.get("trace_gate_up")),
                   _ptr(res.get("trace_swiglu")), _ptr(res.get("output_unrounded")))
        _check(load().gossmx_moe_forward(self.ctx.handle, self._h, C.byref(io)))
        return res

    def forward_residual(self, residual_bf16: np.ndarray, norm_weight: np.ndarray, epsilon: float = 1e-5,
                         injected_logits: np.ndarray | None = None, want_output: bool = True) -> dict:
        """The MoE half of a decoder layer (forward_layer_batch,
        cpu_runner.rs:2519-2553) on the post-attention residual stream: the
        block runs on norm_boundary(residual, norm_weight) and next_residual
        [m][hidden] bf16 bits is add_residual(residual, output). The other
        outputs are forward()'s; output is omitted with want_output=False."""
        x = np.ascontiguousarray(residual_bf16, dtype=np.uint16)
        w = np.ascontiguousarray(norm_weight, dtype=np.float32)
        m = x.shape[0]
        E, K, H = self.experts, self.top_k, self.hidden
        res = {
            "router_logits": np.empty((m, E), np.float32),
            "selected": np.empty((m, K), np.uint32),
            "routing_weights": np.empty((m, K), np.float32),
            "route_order": np.empty(m * K, np.uint32),
            "next_residual": np.empty((m, H), np.uint16),
        }
        if want_output:
            res["output"] = np.empty((m, H), np.float32)
        inj = None if injected_logits is None else np.ascontiguousarray(injected_logits, dtype=np.float32)
        io = MoeIo(_ptr(x), m, _ptr(inj), _ptr(res["router_logits"]), _ptr(res["selected"]),
                   _ptr(res["routing_weights"]), _ptr(res.get("output")), _ptr(res["route_order"]), None, MEM_HOST)
        _check(load().gossmx_moe_forward_residual(self.ctx.handle, self._h, C.byref(io), _ptr(w), float(epsilon),
                                                  _ptr(res["next_residual"])))
        return res

    def forward_residual_device(self, residual, m: int, norm_weight, epsilon: float, next_residual, output=None,
                                injected_logits=None, selected=None):
        """forward_residual on device pointers (ints or torch tensors), asynchronous."""
        io = MoeIo(_ptr(residual), m, _ptr(injected_logits), None, _ptr(selected), None, _ptr(output), None, None,
                   MEM_DEVICE)
        _check(load().gossmx_moe_forward_residual(self.ctx.handle, self._h, C.byref(io), _ptr(norm_weight),
                                                  float(epsilon), _ptr(next_residual)))

    def forward_device(self, x, m: int, output, injected_logits=None, router_logits=None, selected=None,
                       routing_weights=None, route_order=None, output_unrounded=None):
        """Asynchronous forward on device pointers (ints or torch tensors);
        device-side errors surface at the next Context.synchronize()."""
        io = MoeIo(_ptr(x), m, _ptr(injected_logits), _ptr(router_logits), _ptr(selected), _ptr(routing_weights),
                   _ptr(output), _ptr(route_order), None, MEM_DEVICE, None, None, _ptr(output_unrounded))
        _check(load().gossmx_moe_forward(self.ctx.handle, self._h, C.byref(io)))

    def moe_batch(self, inputs: np.ndarray, injected_logits: np.ndarray | None = None) -> list[MoeStep]:
        """CpuModel::moe_batch: one MoeStep per input row."""
        r = self.forward(inputs, injected_logits)
        return [MoeStep(r["router_logits"][i], r["selected"][i].astype(np.int64), r["routing_weights"][i],
                        r["output"][i]) for i in range(r["output"].shape[0])]

    def close(self):
        if self._h:
            load().gossmx_layer_destroy(self._h)
            self._h = C.c_void_p()


class Model:
    """A GPT-OSS model (gossmx_model_*): attention on host threads, projections, lm_head and MoE layers on the GPU.

    `layers` is a list of dicts with the gossmx_dense_layer tensors (numpy
    arrays: norms, biases and sinks f32, matrices bf16 bits as uint16), the
    `sliding` flag and the `moe` MoeLayer. The arrays are kept alive here."""

    def __init__(self, ctx: Context, config: ModelConfig, embedding, final_norm, lm_head, layers):
        self.ctx, self.config = ctx, config
        keep = []

        def arr(a, dtype):
            a = np.ascontiguousarray(a, dtype=dtype)
            keep.append(a)
            return a.ctypes.data

        table = (DenseLayer * len(layers))()
        for i, L in enumerate(layers):
            d = table[i]
            for name in ("input_norm", "q_bias", "k_bias", "v_bias", "o_bias", "sinks", "post_attention_norm"):
                setattr(d, name, arr(L[name], np.float32))
            for name in ("q_weight", "k_weight", "v_weight", "o_weight"):
                setattr(d, name, arr(L[name], np.uint16))
            d.sliding = 1 if L["sliding"] else 0
            d.moe = L["moe"].handle if hasattr(L["moe"], "handle") else L["moe"]._h.value
        emb, fin, head = arr(embedding, np.uint16), arr(final_norm, np.float32), arr(lm_head, np.uint16)
        self._keep, self._table = keep, table
        self._h = C.c_void_p()
        _check(load().gossmx_model_create(ctx.handle, C.byref(config), emb, fin, head, table, C.byref(self._h)))

    def _logits(self):
        return np.zeros(self.config.vocab, np.float32)

    def prefill(self, tokens) -> np.ndarray:
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        out = self._logits()
        _check(load().gossmx_model_prefill(self._h, _ptr(t), t.size, _ptr(out)))
        return out

    def append(self, tokens) -> np.ndarray:
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        out = self._logits()
        _check(load().gossmx_model_append(self._h, _ptr(t), t.size, _ptr(out)))
        return out

    def decode(self, token: int) -> np.ndarray:
        out = self._logits()
        _check(load().gossmx_model_decode(self._h, int(token), _ptr(out)))
        return out

    def reset(self):
        _check(load().gossmx_model_reset(self._h))

    @property
    def position(self) -> int:
        p = C.c_size_t()
        _check(load().gossmx_model_position(self._h, C.byref(p)))
        return p.value

    def cache(self, layer: int) -> tuple[int, int]:
        n, start = C.c_size_t(), C.c_size_t()
        _check(load().gossmx_model_cache(self._h, layer, C.byref(n), C.byref(start)))
        return n.value, start.value

    def times(self) -> tuple[float, float]:
        """(dense seconds, MoE seconds) accumulated over the model's steps."""
        d, m = C.c_double(), C.c_double()
        _check(load().gossmx_model_times(self._h, C.byref(d), C.byref(m)))
        return d.value, m.value

    def generate(self, prompt, decode_steps: int) -> tuple[np.ndarray, np.ndarray]:
        """prefill then decode_steps greedy decodes: (tokens [decode_steps + 1], logits rows)."""
        logits = [self.prefill(prompt)]
        tokens = [greedy_token(logits[0])]
        for _ in range(decode_steps):
            logits.append(self.decode(tokens[-1]))
            tokens.append(greedy_token(logits[-1]))
        return np.array(tokens, np.uint32), np.stack(logits)

    def close(self):
        if self._h:
            load().gossmx_model_destroy(self._h)
            self._h = C.c_void_p()


def greedy_token(logits) -> int:
    v = np.ascontiguousarray(logits, dtype=np.float32)
    t = C.c_uint32()
    _check(load().gossmx_greedy_token(_ptr(v), v.size, C.byref(t)))
    return t.value


def yarn_rope(config: ModelConfig, values, heads: int, position: int) -> np.ndarray:
    v = np.array(values, dtype=np.float32)
    _check(load().gossmx_yarn_rope(C.byref(config), _ptr(v), heads, position))
    return v


def attention(query, keys, values, window: int, sinks, heads: int, kv_heads: int, head_dim: int) -> np.ndarray:
    q = np.ascontiguousarray(query, dtype=np.float32)
    k = np.ascontiguousarray(keys, dtype=np.uint16)
    v = np.ascontiguousarray(values, dtype=np.uint16)
    s = np.ascontiguousarray(sinks, dtype=np.float32)
    out = np.zeros(heads * head_dim, np.float32)
    tokens = k.size // (kv_heads * head_dim)
    _check(load().gossmx_attention(_ptr(q), _ptr(k), _ptr(v), tokens, window, _ptr(s), heads, kv_heads, head_dim,
                                   _ptr(out)))
    return out
