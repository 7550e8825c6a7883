"""The C-ABI library on a host without a GPU: it loads, exports every
function include/gossmx.h declares, refuses to run without a gfx950 device,
and validates problems exactly like Mxfp4MatmulProblem::new
(crates/gpt-oss-cpu-kernels/src/matmul.rs:245-267, 339-369)."""
import ctypes as C
import os
import subprocess

import numpy as np
import pytest

import gossmx as G

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_library_exports_every_header_symbol():
    L = G.load()
    declared = G.header_symbols()
    assert len(declared) >= 25
    missing = [s for s in declared if not hasattr(L, s)]
    assert not missing, missing
    out = subprocess.run(["nm", "-D", "--defined-only", G.LIB_PATH], capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert set(declared) <= exported


def test_version_and_errors_without_device():
    L = G.load()
    assert L.gossmx_version() == 100
    if G.device_count() > 0:
        pytest.skip("a gfx950 device is visible")
    h = C.c_void_p()
    st = L.gossmx_ctx_create(0, None, C.byref(h))
    assert st == G.ERR_UNAVAILABLE_BACKEND
    assert b"device" in L.gossmx_last_error()
    with pytest.raises(G.GossmxError) as err:
        G.Context(0)
    assert err.value.status == G.ERR_UNAVAILABLE_BACKEND


def test_null_arguments_are_rejected():
    L = G.load()
    assert L.gossmx_synchronize(None) == G.ERR_INVALID_ARGUMENT
    assert L.gossmx_moe_forward(None, None, None) == G.ERR_INVALID_ARGUMENT
    assert L.gossmx_moe_forward_residual(None, None, None, None, 1e-5, None) == G.ERR_INVALID_ARGUMENT
    assert L.gossmx_mxfp4_matmul(None, None) == G.ERR_INVALID_ARGUMENT
    assert L.gossmx_inject_fault(None, 1) == G.ERR_INVALID_ARGUMENT


def test_circuit_breaker_without_device():
    assert not G.circuit_is_open()
    G.circuit_reset()
    assert not G.circuit_is_open()
    L = G.load()
    size, align = C.c_size_t(7), C.c_size_t(7)
    assert L.gossmx_mxfp4_scratch_requirement(None, C.byref(size), C.byref(align)) == G.ERR_INVALID_ARGUMENT
    assert L.gossmx_ctx_fast_path(None, C.byref(C.c_int())) == G.ERR_INVALID_ARGUMENT
    assert L.gossmx_inject_fault(None, 2) == G.ERR_INVALID_ARGUMENT


ROWS, BLOCKS = 40, 3


def check(**kw):
    args = dict(rows=ROWS, blocks=BLOCKS, experts=2, activations_len=2 * BLOCKS, m=2, blocks_per_row=BLOCKS,
                row_stride=BLOCKS, bias_len=ROWS, output_len=2 * ROWS, output_stride=ROWS)
    args.update(kw)
    return G.matmul_check(**args)


def test_validation_accepts_exact_extents():
    assert check() == G.OK
    assert check(bias_len=None) == G.OK
    # strided activations and padded outputs: the last row needs only its own extent
    assert check(row_stride=5, activations_len=5 + BLOCKS) == G.OK
    assert check(output_stride=48, output_len=48 + ROWS) == G.OK
    assert check(kind=G.ACT_Q8) == G.OK


@pytest.mark.parametrize("kw", [
    dict(m=0),
    dict(blocks_per_row=0),
    dict(row_stride=BLOCKS - 1),
    dict(activations_len=2 * BLOCKS - 1),
    dict(blocks_per_row=BLOCKS + 1, row_stride=BLOCKS + 1, activations_len=2 * BLOCKS + 2),
    dict(output_stride=ROWS - 1),
    dict(output_len=2 * ROWS - 1),
    dict(bias_len=ROWS - 1),
    dict(expert=2),
    dict(m=3, row_stride=2**63, activations_len=2**64 - 1, output_len=3 * ROWS),  # checked_mul overflow
])
def test_validation_rejects_like_the_reference(kw):
    assert check(**kw) == G.ERR_INVALID_DIMENSIONS


def test_validation_rejects_unknown_kinds():
    assert check(kind=3) == G.ERR_INVALID_ARGUMENT


def test_header_cites_reference_interfaces():
    with open(os.path.join(ROOT, "include", "gossmx.h")) as fh:
        text = fh.read()
    for cite in ("matmul.rs:398-414", "cpu_runner.rs:2794-3013", "cpu_repack.rs:149-216", "lib.rs:138-157"):
        assert cite in text
