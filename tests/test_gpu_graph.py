"""HIP-graph capture of the MoE block (gossmx_capture_*): every replay, with
eager work and synchronizations in between, equals the eager result and the
oracle bit for bit."""
import numpy as np
import pytest

import gossmx as G
import oracle as O

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("m", [1, 3, 12])
def test_captured_forward_replays_match_eager_and_oracle(m):
    """m = 1 and 3 take the one-launch router/selection kernel, whose arrival
    counter must be back at zero after every launch, eager or replayed; m = 1
    also the down projection with the combine in the same launch."""
    with G.Context(0) as ctx:
        E, H, I, K = 8, 128, 64, 4
        host = O.synthetic_layer(21, 0, experts=E, hidden=H, intermediate=I, top_k=K)
        gu = G.Weights.upload(ctx, host.gate_up, E, 2 * I, H // 32)
        dn = G.Weights.upload(ctx, host.down, E, H, I // 32)
        layer = G.MoeLayer(ctx, E, H, I, K, host.router_weight, host.router_bias, gu, host.gate_up_bias, dn,
                           host.down_bias)
        x1 = O.gen_hidden(21, 1, m, H)
        x2 = O.gen_hidden(21, 2, m, H)
        want1 = O.moe_batch(host, x1)["output"]
        want2 = O.moe_batch(host, x2)["output"]
        dx1, dx2 = ctx.malloc(x1.nbytes), ctx.malloc(x2.nbytes)
        dout1, dout2 = ctx.malloc(m * H * 4), ctx.malloc(m * H * 4)
        ctx.h2d(dx1, x1)
        ctx.h2d(dx2, x2)
        layer.forward_device(dx1, m, dout1)  # eager: sizes the scratch buffers
        ctx.synchronize()
        ctx.capture_begin()
        layer.forward_device(dx1, m, dout1)
        graph = ctx.capture_end()
        for _ in range(3):
            layer.forward_device(dx2, m, dout2)  # eager work between replays
            ctx.synchronize()
            got2 = np.empty((m, H), np.float32)
            ctx.d2h(got2, dout2)
            assert (got2.view(np.uint32) == want2.view(np.uint32)).all()
            ctx.h2d(dout1, np.full((m, H), np.nan, np.float32))
            graph.launch()
            ctx.synchronize()
            got1 = np.empty((m, H), np.float32)
            ctx.d2h(got1, dout1)
            assert (got1.view(np.uint32) == want1.view(np.uint32)).all()
        graph.close()
        # host-memory calls are refused while capturing
        ctx.capture_begin()
        with pytest.raises(G.GossmxError) as e:
            layer.forward(x1)
        assert e.value.status == G.ERR_UNSUPPORTED
        ctx.capture_end().close()
        for p in (dx1, dx2, dout1, dout2):
            ctx.free(p)
        layer.close()
        gu.close()
        dn.close()


def test_graph_survives_eager_calls_that_grow_the_scratch():
    """A graph captured at a small batch keeps the scratch addresses it was
    recorded with: an eager call at a much larger batch (which needs larger
    scratch buffers) runs in between, and the replay still equals the
    oracle bit for bit. The buffers the graph holds are freed only when the
    graph is destroyed."""
    with G.Context(0) as ctx:
        E, H, I, K = 8, 128, 64, 4
        host = O.synthetic_layer(23, 0, experts=E, hidden=H, intermediate=I, top_k=K)
        gu = G.Weights.upload(ctx, host.gate_up, E, 2 * I, H // 32)
        dn = G.Weights.upload(ctx, host.down, E, H, I // 32)
        layer = G.MoeLayer(ctx, E, H, I, K, host.router_weight, host.router_bias, gu, host.gate_up_bias, dn,
                           host.down_bias)
        small, big = 12, 700
        xs = O.gen_hidden(23, 1, small, H)
        xb = O.gen_hidden(23, 2, big, H)
        want_s = O.moe_batch(host, xs)["output"]
        dxs, douts = ctx.malloc(xs.nbytes), ctx.malloc(small * H * 4)
        ctx.h2d(dxs, xs)
        layer.forward_device(dxs, small, douts)
        ctx.synchronize()
        ctx.capture_begin()
        layer.forward_device(dxs, small, douts)
        graph = ctx.capture_end()
        for rep in range(2):
            got_b = layer.forward(xb)  # grows every scratch buffer while the graph lives
            rows = [0, 350, big - 1]
            want_b = O.moe_batch(host, xb[rows])
            assert (got_b["output"][rows].view(np.uint32) == want_b["output"].view(np.uint32)).all()
            ctx.h2d(douts, np.full((small, H), np.nan, np.float32))
            graph.launch()
            ctx.synchronize()
            got = np.empty((small, H), np.float32)
            ctx.d2h(got, douts)
            assert (got.view(np.uint32) == want_s.view(np.uint32)).all(), f"replay {rep}"
        graph.close()
        # after the graph is gone the context keeps working at both sizes
        assert (layer.forward(xs)["output"].view(np.uint32) == want_s.view(np.uint32)).all()
        ctx.free(dxs)
        ctx.free(douts)
        layer.close()
        gu.close()
        dn.close()
