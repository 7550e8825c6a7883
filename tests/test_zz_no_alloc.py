"""gossmx_moe_forward_noalloc: the MoE block without allocating, its scratch
carved from a fixed per-device array. Called through the C ABI on device
memory and compared with gossmx_moe_forward bit for bit, two calls in a row
(the second smaller), the first on a fresh context with the device's free
memory unchanged around it; a call past the fixed size fails before
launching and leaves its outputs untouched."""
import ctypes as C

import numpy as np
import pytest

import gossmx as G
import oracle as O
import synth

pytestmark = pytest.mark.gpu

KEYS = (("router_logits", np.float32, "E"), ("selected", np.uint32, "K"), ("routing_weights", np.float32, "K"),
        ("output", np.float32, "H"), ("route_order", np.uint32, "K"))


def device_free_bytes() -> int:
    hip = C.CDLL("libamdhip64.so")
    free, total = C.c_size_t(), C.c_size_t()
    assert hip.hipMemGetInfo(C.byref(free), C.byref(total)) == 0
    return free.value


def run(ctx, layer, fn, x, logits, m, free_bytes=None):
    """One call of `fn` (gossmx_moe_forward or _noalloc) on device buffers;
    returns the status and the host copies of every output (read back also
    after a refused call). With free_bytes (a list), appends the device's free
    memory just before and just after the call (synchronized)."""
    E, K, H = layer.experts, layer.top_k, layer.hidden
    width = {"E": E, "K": K, "H": H}
    bufs = {k: ctx.malloc(m * width[w] * 4) for k, _, w in KEYS}
    for k, _, w in KEYS:  # NaN-filled so that unwritten outputs show
        ctx.h2d(bufs[k], np.full(m * width[w], 0xFFFFFFFF, np.uint32))
    dx = ctx.malloc(x.nbytes)
    ctx.h2d(dx, x)
    dl = None
    if logits is not None:
        dl = ctx.malloc(logits.nbytes)
        ctx.h2d(dl, logits)
    io = G.MoeIo(dx, m, dl, bufs["router_logits"], bufs["selected"], bufs["routing_weights"], bufs["output"],
                 bufs["route_order"], None, G.MEM_DEVICE)
    ctx.synchronize()
    if free_bytes is not None:
        free_bytes.append(device_free_bytes())
    st = fn(ctx.handle, layer._h, C.byref(io))
    ctx.synchronize()
    if free_bytes is not None:
        free_bytes.append(device_free_bytes())
    out = {}
    for k, dt, w in KEYS:
        a = np.empty(m * width[w], dt)
        ctx.d2h(a, bufs[k])
        out[k] = a
    for p in list(bufs.values()) + [dx] + ([dl] if dl else []):
        ctx.free(p)
    return st, out


def test_noalloc_matches_forward_on_two_calls_then_refuses_past_its_size():
    L = G.load()
    with G.Context(0) as ctx:
        host = O.synthetic_layer(2025, 0)
        gu = G.Weights.upload(ctx, host.gate_up, 32, 5760, 90)
        dn = G.Weights.upload(ctx, host.down, 32, 2880, 90)
        layer = G.MoeLayer(ctx, 32, 2880, 2880, 4, host.router_weight, host.router_bias, gu, host.gate_up_bias, dn,
                           host.down_bias)
        rng = np.random.default_rng(7)
        cases = [(64, True), (5, False)]  # Zipf-routed decode batch, then a smaller one with the router computed
        inputs = []
        for m, inject in cases:
            x = synth.hidden_rows(rng, m)
            logits = synth.zipf_logits(rng, m, 32) if inject else None
            st, want = run(ctx, layer, L.gossmx_moe_forward, x, logits, m)  # also loads every kernel once
            assert st == G.OK, L.gossmx_last_error()
            inputs.append((m, x, logits, want))
        # A fresh context (weights and layers do not belong to one): its first
        # call is the no-allocation one, at a shape it has never seen, so no
        # grow-only buffer of the context could serve it; the device's free
        # memory is the same before and after.
        with G.Context(0) as fresh:
            for i, (m, x, logits, want) in enumerate(inputs):
                free = []
                st, got = run(fresh, layer, L.gossmx_moe_forward_noalloc, x, logits, m, free)
                assert st == G.OK, L.gossmx_last_error()
                assert free[0] == free[1], f"call {i} (m={m}) changed free device memory by {free[0] - free[1]} B"
                for k, _, _ in KEYS:
                    assert (got[k].view(np.uint32) == want[k].view(np.uint32)).all(), f"m={m}: {k} differs"
            # two rows against the oracle as well
            x = synth.hidden_rows(rng, 2)
            st, got = run(fresh, layer, L.gossmx_moe_forward_noalloc, x, None, 2)
            assert st == G.OK
            ref = O.moe_batch(host, x)
            assert (got["output"].view(np.uint32) == ref["output"].ravel().view(np.uint32)).all()
            # past the fixed size: refused before any launch, outputs untouched (still NaN)
            big = 1024
            x = synth.hidden_rows(rng, big)
            st, got = run(fresh, layer, L.gossmx_moe_forward_noalloc, x, synth.uniform_logits(rng, big, 32), big)
            assert st == G.ERR_UNSUPPORTED and b"fixed scratch" in L.gossmx_last_error()
            for k, _, _ in KEYS:
                assert (got[k].view(np.uint32) == 0xFFFFFFFF).all(), f"{k} written by a refused call"
            # host memory is refused
            io = G.MoeIo(G._ptr(x[:1]), 1, None, None, None, None, G._ptr(np.zeros((1, 2880), np.float32)), None,
                         None, G.MEM_HOST)
            assert L.gossmx_moe_forward_noalloc(fresh.handle, layer._h, C.byref(io)) == G.ERR_INVALID_ARGUMENT
        layer.close()
        gu.close()
        dn.close()
