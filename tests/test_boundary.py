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


def test_accounting_without_device():
    # Projection calls count by result: argument failures are "rejected".
    L = G.load()
    before = G.stats()
    assert L.gossmx_moe_forward(None, None, None) == G.ERR_INVALID_ARGUMENT
    assert L.gossmx_moe_forward_noalloc(None, None, None) == G.ERR_INVALID_ARGUMENT
    assert L.gossmx_mxfp4_matmul(None, None) == G.ERR_INVALID_ARGUMENT
    after = G.stats()
    assert after["projections_rejected"] - before["projections_rejected"] == 3
    assert after["projections_ok"] == before["projections_ok"]
    assert L.gossmx_stats_read(None) == G.ERR_INVALID_ARGUMENT
    try:
        G.set_resident_cap(1 << 30)
        assert G.stats()["resident_cap_bytes"] == 1 << 30
    finally:
        G.set_resident_cap(0)
    assert G.stats()["resident_cap_bytes"] == 0
    G.stats_reset()
    s = G.stats()
    assert s["projections_rejected"] == 0 and s["resident_high_water_bytes"] == s["resident_bytes"]
    assert L.gossmx_profile_tag(None, 0, G.PHASE_DECODE) == G.ERR_INVALID_ARGUMENT
    assert L.gossmx_profile_events(None, None, 0, None, None, None) == G.ERR_INVALID_ARGUMENT


def test_profile_event_layout_matches_the_header():
    # Field offsets of gossmx_profile_event and gossmx_stats as the C compiler
    # lays them out (gcc on the header).
    import tempfile
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    src = '''#include <stddef.h>
#include <stdio.h>
#include "gossmx.h"
#define F(T, f) printf("%s %s %zu\\n", #T, #f, offsetof(T, f));
int main(void) {
F(gossmx_profile_event, op) F(gossmx_profile_event, layer) F(gossmx_profile_event, m)
F(gossmx_profile_event, rows_per_item) F(gossmx_profile_event, start_ns) F(gossmx_profile_event, resident_bytes)
F(gossmx_stats, resident_bytes) F(gossmx_stats, repack_cache_misses) F(gossmx_stats, circuit_open)
printf("sizes %zu %zu\\n", sizeof(gossmx_profile_event), sizeof(gossmx_stats));
return 0; }
'''
    with tempfile.TemporaryDirectory() as d:
        c = os.path.join(d, "layout.c")
        exe = os.path.join(d, "layout")
        with open(c, "w") as fh:
            fh.write(src)
        subprocess.run(["gcc", "-std=c99", "-I", os.path.join(root, "include"), c, "-o", exe], check=True)
        out = subprocess.run([exe], capture_output=True, text=True, check=True).stdout.split("\n")
    want = {}
    for line in out:
        parts = line.split()
        if len(parts) == 3 and parts[0] != "sizes":
            want[(parts[0], parts[1])] = int(parts[2])
        elif parts and parts[0] == "sizes":
            sizes = (int(parts[1]), int(parts[2]))
    py = {"gossmx_profile_event": G.ProfileEvent, "gossmx_stats": G.Stats}
    for (t, f), off in want.items():
        assert getattr(py[t], f).offset == off, (t, f)
    assert (C.sizeof(G.ProfileEvent), C.sizeof(G.Stats)) == sizes


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
