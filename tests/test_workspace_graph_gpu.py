"""The per-stream split-K workspace and HIP graphs: a graph captured on a stream keeps the
workspace addresses it was captured with, so a later eager linear on the same stream that
grows the workspace must leave the old one alive.  The graph (an M = 6 linear whose K is
split on the small-row MFMA kernel) is replayed after the growth, with eager split-K work on
the same stream between the replays, and every replay must equal the eager result bit for
bit (same kernel, same split, same summation order)."""
import numpy as np
import pytest
import torch

import mingtts as mt
import oracle as O
from _gpu_util import dev16, say

pytestmark = pytest.mark.gpu


def _weights(rng, n, k, gpu):
    wb, wr = O.round16(rng.standard_normal((n, k)).astype(np.float32) * np.float32(0.05), O.F16)
    return dev16(wb, O.F16, gpu), wr


def test_graph_keeps_its_split_workspace_after_the_stream_grows_it(gpu):
    rng = np.random.default_rng(11)
    M, N, K = 6, 1024, 4096
    assert mt.linear_kernel(M, N, K, xt=mt.F32, wt=mt.F16) == mt.KERNEL_GEMV_MFMA
    w, _ = _weights(rng, N, K, gpu)
    bias_b, _ = O.round16(rng.standard_normal(N).astype(np.float32) * np.float32(0.1), O.F16)
    bias = dev16(bias_b, O.F16, gpu)
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).to(gpu)
    y_ref = torch.zeros(M, N, device=gpu)
    y_g = torch.zeros(M, N, device=gpu)

    # The growing linear: 512 rows, K forced into 8 splits, so its partial sums need far more
    # than the M = 6 linear's.
    BM, BN, BK = 512, 896, 4864
    bw, bwr = _weights(rng, BN, BK, gpu)
    bxb, bxr = O.round16(rng.standard_normal((BM, BK)).astype(np.float32), O.F16)
    bx = dev16(bxb, O.F16, gpu)
    by = torch.zeros(BM, BN, device=gpu)
    want_big = bxr.astype(np.float64) @ bwr.astype(np.float64).T

    cs = torch.cuda.Stream(device=gpu)

    def small(y):
        rc = mt.linear_raw(x, mt.F32, w, None, mt.F16, bias, y, M, N, K, K, N, mt.GemvFlags.bias, cs)
        assert rc == 0, mt.last_error()

    def big():
        old = mt.set_tuning(mt.TUNE_GEMM_SPLITK, 8)
        try:
            rc = mt.linear_raw(bx, mt.F16, bw, None, mt.F16, None, by, BM, BN, BK, BK, BN, 0, cs)
        finally:
            mt.set_tuning(mt.TUNE_GEMM_SPLITK, old)
        assert rc == 0, mt.last_error()

    say("workspace graph: eager M=6, capture")
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(cs):
        small(y_ref)  # eager first: the workspace may not grow under capture
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=cs):
            small(y_g)
    torch.cuda.synchronize()
    ref = y_ref.cpu().numpy()

    for r in range(3):
        say(f"workspace graph: eager M=512 split 8, replay {r}")
        with torch.cuda.stream(cs):
            big()
        torch.cuda.synchronize()
        got_big = by.cpu().numpy()
        assert O.normwise_rel_err(got_big, want_big) <= 1e-5
        y_g.fill_(np.float32(7.0))
        torch.cuda.synchronize()
        with torch.cuda.stream(cs):
            graph.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(y_g.cpu().numpy(), ref)
    del graph
