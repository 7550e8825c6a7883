"""Two worker threads, each with its own context (stream, scratch, staging) and
layer, calling the MoE block at the same time: the C ABI's threading
contract (one gossmx_ctx per worker, as one CpuExecutionContext per worker in
the reference's runner, cpu_runner.rs:569-575) with process-wide accounting.
Every result is bit-identical to the oracle's moe_batch (cpu_runner.rs:
2794-3013) and the process-wide success count equals the calls made."""
import threading

import numpy as np
import pytest

import gossmx as G
import oracle as O

pytestmark = pytest.mark.gpu


def worker(seed, calls, errors, done):
    try:
        host = O.synthetic_layer(seed, 0, experts=16, hidden=256, intermediate=128, top_k=4)
        cases = []
        for m in (1, 40):
            x = O.gen_hidden(seed, m, m, 256)
            want = O.moe_batch(host, x)
            assert want["status"] == O.OK
            cases.append((x, want))
        with G.Context(0) as ctx:
            gu = G.Weights.upload(ctx, host.gate_up, 16, 256, 256 // 32)
            dn = G.Weights.upload(ctx, host.down, 16, 256, 128 // 32)
            layer = G.MoeLayer(ctx, 16, 256, 128, 4, host.router_weight, host.router_bias, gu, host.gate_up_bias,
                               dn, host.down_bias, host.alpha, host.limit)
            for i in range(calls):
                x, want = cases[i % 2]
                got = layer.forward(x)
                for key in ("router_logits", "routing_weights", "output"):
                    assert (got[key].view(np.uint32) == want[key].view(np.uint32)).all(), (seed, i, key)
                assert (got["selected"] == want["selected"]).all(), (seed, i)
                assert (got["route_order"] == want["route_order"]).all(), (seed, i)
                done[seed] = done.get(seed, 0) + 1
            layer.close()
            gu.close()
            dn.close()
    except BaseException as e:  # reported by the main thread
        errors.append((seed, repr(e)))


def test_two_contexts_on_two_threads_stay_bit_exact():
    calls = 24
    errors, done = [], {}
    s0 = G.stats()
    threads = [threading.Thread(target=worker, args=(seed, calls, errors, done)) for seed in (61, 62)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=240)
    assert not any(t.is_alive() for t in threads), "a worker did not finish"
    assert not errors, errors
    assert done == {61: calls, 62: calls}
    s1 = G.stats()
    assert s1["projections_ok"] - s0["projections_ok"] == 2 * calls
    assert s1["projections_failed"] == s0["projections_failed"]
