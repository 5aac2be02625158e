"""The ops inside a captured HIP graph: every replay matches the eager result bit for bit.

A graph is captured once per op; between replays the test runs eager work of its own (other
launches, synchronisations, fresh allocations), then checks each replay's outputs against the
eager call on the same inputs.  The kernels clear nothing with memset and allocate nothing while
they run, so replays after the first must not drift.
"""

import pytest
import torch

from helpers import dev

pytestmark = pytest.mark.gpu

REPLAYS = 4


def _capture(fn):
    """Capture fn() (returning a tuple of tensors) in a graph after a side-stream warm-up."""
    side = torch.cuda.Stream(dev())
    side.wait_stream(torch.cuda.current_stream(dev()))
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream(dev()).wait_stream(side)
    torch.cuda.synchronize(dev())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = fn()
    return graph, outs


def _check_replays(fn):
    want = [t.clone() for t in fn()]
    graph, outs = _capture(fn)
    scratch = torch.randn(1 << 20, device=dev())
    for r in range(REPLAYS):
        scratch.mul_(1.0001).add_(r)  # eager work between replays
        torch.cuda.synchronize(dev())
        graph.replay()
        torch.cuda.synchronize(dev())
        for got, ref in zip(outs, want):
            assert torch.equal(got, ref), f"replay {r}: max diff {(got.float() - ref.float()).abs().max().item()}"


def _chunkwise_inputs(B, NH, S, DQK, DV, seed):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(B, NH, S, DQK, generator=g) / DQK ** 0.5).to(torch.bfloat16).to(dev())
    k = torch.randn(B, NH, S, DQK, generator=g).to(torch.bfloat16).to(dev())
    v = torch.randn(B, NH, S, DV, generator=g).to(torch.bfloat16).to(dev())
    i = torch.randn(B, NH, S, generator=g).to(torch.bfloat16).to(dev())
    f = (torch.randn(B, NH, S, generator=g) + 3).to(torch.bfloat16).to(dev())
    return q, k, v, i, f


@pytest.mark.parametrize("S,algo", [(256, "auto"), (200, "fused")])
def test_chunkwise_graph_replays(gpu_case, S, algo):
    import xlstm_hip
    q, k, v, i, f = _chunkwise_inputs(1, 2, S, 256, 128, seed=S)

    def fn():
        h, (C, n, m) = xlstm_hip.mlstm_chunkwise(q, k, v, i, f, return_last_states=True, algo=algo)
        return h, C, n, m

    _check_replays(fn)


def test_decode_step_graph_replays(gpu_case):
    import xlstm_hip
    g = torch.Generator().manual_seed(3)
    B, NH, DQK, DV = 2, 4, 256, 512
    q, k = (torch.randn(B, NH, DQK, generator=g).to(torch.bfloat16).to(dev()) for _ in range(2))
    v = torch.randn(B, NH, DV, generator=g).to(torch.bfloat16).to(dev())
    i = torch.randn(B, NH, 1, generator=g).to(dev())
    f = (torch.randn(B, NH, 1, generator=g) + 3).to(dev())
    C = (0.1 * torch.randn(B, NH, DQK, DV, generator=g)).to(dev())
    n = torch.randn(B, NH, DQK, generator=g).abs().to(dev())
    m = torch.randn(B, NH, 1, generator=g).to(dev())

    def fn():
        h, (C1, n1, m1) = xlstm_hip.mlstm_recurrent_step__native(q, k, v, i, f, C, n, m)
        return h, C1, n1, m1

    _check_replays(fn)


def test_slstm_sequence_graph_replays(gpu_case):
    import xlstm_hip
    g = torch.Generator().manual_seed(4)
    B, S, NH, H = 2, 300, 2, 128
    z = torch.randn(B, S, NH, H, generator=g).to(torch.bfloat16).to(dev())
    i, f, o = (torch.randn(B, S, NH, generator=g).to(torch.bfloat16).to(dev()) for _ in range(3))

    def fn():
        h, (c, n, m) = xlstm_hip.slstm_sequence(z, i, f, o)
        return h, c, n, m

    _check_replays(fn)


def test_soft_cap_graph_replays(gpu_case):
    import xlstm_hip
    x = (30 * torch.randn(3, 1000, 777, generator=torch.Generator().manual_seed(5))).to(torch.bfloat16).to(dev())
    _check_replays(lambda: (xlstm_hip.soft_cap(x, 30.0),))


def test_slstm_layer_stages_graph_replays(gpu_case):
    import xlstm_hip
    g = torch.Generator().manual_seed(6)
    x = torch.randn(2, 300, 256, generator=g).to(torch.bfloat16).to(dev())
    w = (0.5 * torch.randn(256, 1, 4, generator=g)).to(torch.bfloat16).to(dev())
    b = torch.randn(256, generator=g).to(torch.bfloat16).to(dev())
    gw = torch.randn(256, generator=g).to(torch.bfloat16).to(dev())

    def fn():
        y = xlstm_hip.causal_conv1d(x, w, b, activation="silu")
        return y, xlstm_hip.group_norm(y.view(600, 256), 4, gw, b, 1e-6)

    _check_replays(fn)


def test_mh_rmsnorm_gate_graph_replays(gpu_case):
    import xlstm_hip
    g = torch.Generator().manual_seed(8)
    h = torch.randn(2, 4, 100, 512, generator=g).to(torch.bfloat16).to(dev())
    w = torch.randn(2048, generator=g).to(torch.bfloat16).to(dev())
    o = torch.randn(2, 100, 2048, generator=g).to(torch.bfloat16).to(dev())
    _check_replays(lambda: (xlstm_hip.mh_rmsnorm_gate(h, w, o, 1e-6),))


def test_gate_proj_graph_replays(gpu_case):
    import xlstm_hip
    g = torch.Generator().manual_seed(9)
    x = torch.randn(300, 2048, generator=g).to(torch.bfloat16).to(dev())
    w = (0.1 * torch.randn(8, 2048, generator=g)).to(torch.bfloat16).to(dev())
    b = torch.randn(8, generator=g).to(torch.bfloat16).to(dev())
    _check_replays(lambda: (xlstm_hip.gate_proj_softcap(x, w, b, 15.0),))
