"""xl_mlstm_chunkwise_fwd_noalloc: the chunkwise forward whose gate-prep scratch is a static
device array (for callers that cannot allocate).

* CPU: the entry point is exported, states its maximum, and rejects requests beyond it (and
  shapes the fused algorithm does not take) before any GPU work;
* GPU: through the C-ABI, two calls in a row (the second on a smaller input, so the array
  holds the first call's larger contents) each equal xl_mlstm_chunkwise_fwd with the fused
  algorithm and a caller workspace, on h and on the last C, n, m: bit for bit where that call
  runs the same unsplit kernels, within the bf16 parity bar where it splits the sequence into
  segments (few heads); and both also meet the bf16 parity bar against the CPU oracle;
* GPU: a long call on one stream and a short one right behind it on a second stream (no host
  sync) both equal the workspace entry point bit for bit (the calls are ordered on the shared
  array); and the call captured in a HIP graph, replayed on fresh inputs copied into its static
  buffers, equals the eager call on every replay.
"""

import ctypes

import pytest
import torch

from helpers import assert_parity, gpu_available

FUSED = 2
BF16, F32 = 1, 0


@pytest.fixture(scope="module")
def lib():
    from xlstm_hip import _lib
    return _lib.load()


def test_noalloc_max_and_rejections(lib):
    from xlstm_hip import _lib
    mx = lib.xl_mlstm_chunkwise_noalloc_max_bytes()
    assert mx == 16 * 1024 * 1024
    per_chunk = lib.xl_mlstm_chunkwise_workspace_size(1, 1, 64, 256, 512, 64, BF16, FUSED)
    assert per_chunk == 1280
    f = lib.xl_mlstm_chunkwise_fwd_noalloc
    p = ctypes.c_void_p(256)  # never dereferenced: the checks fail before any GPU call
    # 4 * 8 * ceil(32768 / 64) = 16384 head-chunks > 13107
    rc = f(p, p, p, p, p, None, None, None, p, None, None, None, 4, 8, 32768, 256, 512, 64, 0.0625, 1e-6,
           BF16, BF16, None)
    assert rc == -2
    msg = lib.xl_last_error()
    assert b"scratch" in msg and b"13107" in msg
    # float32 q/k/v: the fused algorithm (the only one without a workspace) does not take them
    rc = f(p, p, p, p, p, None, None, None, p, None, None, None, 1, 2, 128, 256, 512, 64, 0.0625, 1e-6,
           F32, F32, None)
    assert rc == -2 and b"fused" in lib.xl_last_error()
    # the usual argument checks still apply
    rc = f(p, p, p, p, None, None, None, None, p, None, None, None, 1, 2, 128, 256, 512, 64, 0.0625, 1e-6,
           BF16, BF16, None)
    assert rc == -1 and b"null" in lib.xl_last_error()
    with pytest.raises(ValueError):
        _lib.check(-1, "noalloc")


def _inputs(B, NH, S, DQK, DV, seed, dev):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(B, NH, S, DQK, generator=g) / DQK ** 0.5).to(torch.bfloat16)
    k = torch.randn(B, NH, S, DQK, generator=g).to(torch.bfloat16)
    v = torch.randn(B, NH, S, DV, generator=g).to(torch.bfloat16)
    i = torch.randn(B, NH, S, generator=g).to(torch.bfloat16)
    f = (torch.randn(B, NH, S, generator=g) + 3).to(torch.bfloat16)
    c0 = 0.1 * torch.randn(B, NH, DQK, DV, generator=g)
    n0 = torch.randn(B, NH, DQK, generator=g).abs()
    m0 = torch.randn(B, NH, generator=g)
    return [t.to(dev) for t in (q, k, v, i, f, c0, n0, m0)]


def _run(lib, fn, x, B, NH, S, DQK, DV, workspace=None):
    q, k, v, i, f, c0, n0, m0 = x
    dev = q.device
    h = torch.full((B, NH, S, DV), float("nan"), dtype=torch.bfloat16, device=dev)
    cl = torch.full((B, NH, DQK, DV), float("nan"), device=dev)
    nl = torch.full((B, NH, DQK), float("nan"), device=dev)
    ml = torch.full((B, NH), float("nan"), device=dev)
    st = torch.cuda.current_stream(dev).cuda_stream
    common = [q.data_ptr(), k.data_ptr(), v.data_ptr(), i.data_ptr(), f.data_ptr(), c0.data_ptr(), n0.data_ptr(),
              m0.data_ptr(), h.data_ptr(), cl.data_ptr(), nl.data_ptr(), ml.data_ptr(), B, NH, S, DQK, DV, 64,
              DQK ** -0.5, 1e-6, BF16, BF16]
    if workspace is None:
        rc = fn(*common, st)
    else:
        rc = fn(*common, FUSED, workspace.data_ptr(), workspace.numel(), st)
    assert rc == 0, lib.xl_last_error()
    torch.cuda.synchronize(dev)
    return h, cl, nl, ml


@pytest.mark.gpu
@pytest.mark.skipif(not gpu_available(), reason="needs a GPU")
def test_noalloc_matches_workspace_entry_point(lib, gpu_case):
    from oracle import mlstm as om
    dev = torch.device("cuda:0")
    # second call smaller than the first: the array still holds the first call's gate prep;
    # the first shape also makes the workspace entry point split the sequence, the second not
    for (B, NH, S, DQK, DV, seed) in ((2, 4, 1000, 256, 128, 11), (1, 2, 300, 128, 64, 12)):
        print(f"[noalloc] B{B} NH{NH} S{S} DQK{DQK} DV{DV} seed {seed}", flush=True)
        x = _inputs(B, NH, S, DQK, DV, seed, dev)
        ws_bytes = lib.xl_mlstm_chunkwise_workspace_size(B, NH, S, DQK, DV, 64, BF16, FUSED)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        want = _run(lib, lib.xl_mlstm_chunkwise_fwd, x, B, NH, S, DQK, DV, workspace=ws)
        got = _run(lib, lib.xl_mlstm_chunkwise_fwd_noalloc, x, B, NH, S, DQK, DV)
        # with few heads the workspace entry point splits the sequence into segments (its
        # workspace then holds per-segment states besides the gate prep); the static scratch
        # holds the gate prep only, so the no-allocation call runs unsplit: the same kernels
        # bit for bit when the other call does not split, the parity bar when it does
        prep_only = ((B * NH * ((S + 63) // 64) * 1280 + 255) // 256) * 256
        for a, b, name in zip(got, want, ("h", "C", "n", "m")):
            if ws_bytes == prep_only:
                assert torch.equal(a, b), f"noalloc {name} differs from the workspace entry point"
            else:
                assert_parity(a.cpu(), b.cpu().float(), torch.bfloat16, f"noalloc vs split {name}")
        # and both meet the parity bar against the oracle
        q, k, v, i, f, c0, n0, m0 = (t.cpu().float() for t in x)
        hr, (Cr, nr, mr) = om.arbitrary_length(q, k, v, f, i, c0, n0, m0[..., None], chunk_size=64)
        assert_parity(got[0], hr, torch.bfloat16, "noalloc h")
        assert_parity(got[1], Cr, torch.bfloat16, "noalloc C")
        assert_parity(got[2], nr, torch.bfloat16, "noalloc n")
        assert_parity(got[3], mr.reshape(B, NH), torch.bfloat16, "noalloc m")


def _launch(lib, x, out, B, NH, S, DQK, DV, stream):
    q, k, v, i, f, c0, n0, m0 = x
    h, cl, nl, ml = out
    rc = lib.xl_mlstm_chunkwise_fwd_noalloc(q.data_ptr(), k.data_ptr(), v.data_ptr(), i.data_ptr(), f.data_ptr(),
                                            c0.data_ptr(), n0.data_ptr(), m0.data_ptr(), h.data_ptr(), cl.data_ptr(),
                                            nl.data_ptr(), ml.data_ptr(), B, NH, S, DQK, DV, 64, DQK ** -0.5, 1e-6,
                                            BF16, BF16, stream)
    assert rc == 0, lib.xl_last_error()


def _outs(B, NH, S, DQK, DV, dev):
    return (torch.full((B, NH, S, DV), float("nan"), dtype=torch.bfloat16, device=dev),
            torch.full((B, NH, DQK, DV), float("nan"), device=dev), torch.full((B, NH, DQK), float("nan"), device=dev),
            torch.full((B, NH), float("nan"), device=dev))


@pytest.mark.gpu
@pytest.mark.skipif(not gpu_available(), reason="needs a GPU")
def test_noalloc_two_streams_are_ordered(lib, gpu_case):
    """A long call on one stream and, right behind it with no host sync, a shorter call on a second
    stream: the second waits for the first (they share the static scratch), so both equal the
    workspace entry point's results bit for bit (neither splits the sequence)."""
    dev = torch.device("cuda:0")
    shapes = ((4, 8, 2048, 256, 512, 21), (1, 8, 448, 128, 128, 22))
    xs, wants = [], []
    for (B, NH, S, DQK, DV, seed) in shapes:
        x = _inputs(B, NH, S, DQK, DV, seed, dev)
        ws = torch.empty(lib.xl_mlstm_chunkwise_workspace_size(B, NH, S, DQK, DV, 64, BF16, FUSED), dtype=torch.uint8,
                         device=dev)
        xs.append(x)
        wants.append(_run(lib, lib.xl_mlstm_chunkwise_fwd, x, B, NH, S, DQK, DV, workspace=ws))
    outs = [_outs(*sh[:5], dev) for sh in shapes]
    sa, sb = torch.cuda.Stream(dev), torch.cuda.Stream(dev)
    for s in (sa, sb):
        s.wait_stream(torch.cuda.current_stream(dev))
    for rep in range(3):
        print(f"[noalloc] two streams, rep {rep}", flush=True)
        for o in outs:
            for t in o:
                t.fill_(float("nan"))
        sa.wait_stream(torch.cuda.current_stream(dev))
        sb.wait_stream(torch.cuda.current_stream(dev))
        _launch(lib, xs[0], outs[0], *shapes[0][:5], sa.cuda_stream)
        _launch(lib, xs[1], outs[1], *shapes[1][:5], sb.cuda_stream)
        torch.cuda.synchronize(dev)
        for got, want in zip(outs, wants):
            for a, b, name in zip(got, want, ("h", "C", "n", "m")):
                assert torch.equal(a, b), f"two streams rep {rep}: {name} differs from the workspace entry point"


@pytest.mark.gpu
@pytest.mark.skipif(not gpu_available(), reason="needs a GPU")
def test_noalloc_graph_capture(lib, gpu_case):
    """The entry point captured in a HIP graph (torch.cuda.graph) on static buffers: every replay, on
    new inputs copied into those buffers with eager work and host syncs between replays, equals the
    eager call on the same inputs bit for bit."""
    dev = torch.device("cuda:0")
    B, NH, S, DQK, DV = 1, 4, 512, 256, 128
    static_x = _inputs(B, NH, S, DQK, DV, 30, dev)
    static_out = _outs(B, NH, S, DQK, DV, dev)
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):  # warm-up on a side stream, as torch.cuda.graph expects
        _launch(lib, static_x, static_out, B, NH, S, DQK, DV, side.cuda_stream)
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize(dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _launch(lib, static_x, static_out, B, NH, S, DQK, DV, torch.cuda.current_stream(dev).cuda_stream)
    for rep in range(4):
        print(f"[noalloc] graph replay {rep}", flush=True)
        fresh = _inputs(B, NH, S, DQK, DV, 31 + rep, dev)
        for dst, src in zip(static_x, fresh):
            dst.copy_(src)
        for t in static_out:
            t.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize(dev)
        want = _outs(B, NH, S, DQK, DV, dev)
        _launch(lib, fresh, want, B, NH, S, DQK, DV, torch.cuda.current_stream(dev).cuda_stream)
        torch.cuda.synchronize(dev)
        for a, b, name in zip(static_out, want, ("h", "C", "n", "m")):
            assert torch.equal(a, b), f"graph replay {rep}: {name} differs from the eager call"
