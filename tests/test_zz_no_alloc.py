"""vkwr_gemm_f16_noalloc (the allocation-free GEMM entry point) against vkwr_gemm_f16 with a
caller workspace, through the C ABI: same plan and kernels, so the outputs must be equal bit
for bit.  Two calls in a row share the device's scratch; the second is smaller, so stale
partials of the first would show.  Both batches are sized so that their K is split (the
partials go through the scratch)."""
import ctypes

import pytest
import torch

from vkwr_amd import capi

pytestmark = pytest.mark.gpu

_noalloc = capi._sig("vkwr_gemm_f16_noalloc", [ctypes.c_int, ctypes.POINTER(capi.GemmProblem), ctypes.c_void_p])
_max = capi._sig("vkwr_gemm_f16_noalloc_max_bytes", [], ctypes.c_int64)


def _batch(gpu, m, n, k, seed, epilogue=capi.EPI_NONE, nprob=1, kn=False):
    g = torch.Generator(device=gpu).manual_seed(seed)
    probs, outs, keep = [], [], []
    for i in range(nprob):
        a = torch.randn(m, k, device=gpu, generator=g).half()
        b = (torch.randn(*((k, n) if kn else (n, k)), device=gpu, generator=g) * 0.05).half()
        c = torch.full((m, n), float("nan"), device=gpu).half()
        v0 = torch.randn(n, device=gpu, generator=g).half()
        probs.append(capi.gemm_problem(a, b, c, b_layout=capi.GEMM_B_KN if kn else capi.GEMM_B_NK,
                                       epilogue=epilogue, v0=v0 if epilogue == capi.EPI_BIAS else None))
        outs.append(c)
        keep += [a, b, v0]
    return probs, outs, keep


def _run_noalloc(probs):
    arr = capi._arr(probs)
    st = _noalloc(len(probs), arr, capi._stream())
    if st != 0:
        raise RuntimeError(capi._LIB.vkwr_last_error().decode())


def _run_ws(probs, gpu):
    ws = torch.empty(max(capi.gemm_workspace_bytes(probs), 1), dtype=torch.uint8, device=gpu)
    capi.gemm(probs, ws)


@pytest.mark.parametrize("shapes", [
    # (m, n, k, epilogue, problems, [K,N] weights): a K-split batch, then a smaller one
    [(128, 1024, 8192, capi.EPI_NONE, 1, False), (40, 1024, 2048, capi.EPI_BIAS, 3, False)],
    # the large-M kernel's split last round (stream-K partials), then a smaller split batch
    [(500, 4096, 2048, capi.EPI_RELU_SQUARE, 1, False), (64, 1024, 4096, capi.EPI_NONE, 2, False)],
    # the GEMV kernel's K parts ([K,N] weights, M <= 4), then a smaller one
    [(3, 4096, 4096, capi.EPI_NONE, 1, True), (1, 2048, 2048, capi.EPI_BIAS, 2, True)],
])
def test_noalloc_equals_workspace_entry_point(gpu, shapes):
    assert _max() == 32 << 20
    for i, (m, n, k, epi, npb, kn) in enumerate(shapes):
        probs, outs, keep = _batch(gpu, m, n, k, seed=10 + i, epilogue=epi, nprob=npb, kn=kn)
        need = capi.gemm_workspace_bytes(probs)
        assert 0 < need <= _max(), need  # the scratch is really used
        _run_noalloc(probs)
        got = [o.clone() for o in outs]
        for o in outs:
            o.fill_(float("nan"))
        _run_ws(probs, gpu)
        torch.cuda.synchronize()
        for g_, w_ in zip(got, outs):
            assert not torch.isnan(w_).any()
            assert torch.equal(g_, w_), (m, n, k)


def test_noalloc_rejects_batches_beyond_its_scratch(gpu):
    """A batch whose plan needs more than the scratch holds fails on the host with a clear
    message and enqueues nothing."""
    probs, outs, keep = _batch(gpu, 512, 4096, 4096, seed=3)
    need = capi.gemm_workspace_bytes(probs)
    assert need > _max()
    with pytest.raises(RuntimeError, match="at most"):
        _run_noalloc(probs)
    torch.cuda.synchronize()
    assert torch.isnan(outs[0]).all()


def test_noalloc_under_graph_capture(gpu):
    """The use the header names: one uncaptured call first (a batch of one empty problem,
    which performs the per-device address lookup), then a K-split batch captured into a
    HIP graph and replayed three times, with eager work and synchronisation between the
    replays; every replay must equal vkwr_gemm_f16 with a workspace bit for bit."""
    empty = capi.gemm_problem(torch.empty(0, 64, dtype=torch.float16, device=gpu),
                              torch.empty(64, 64, dtype=torch.float16, device=gpu),
                              torch.empty(0, 64, dtype=torch.float16, device=gpu))
    _run_noalloc([empty])
    probs, outs, keep = _batch(gpu, 128, 1024, 8192, seed=21)
    assert 0 < capi.gemm_workspace_bytes(probs) <= _max()
    _run_ws(probs, gpu)
    torch.cuda.synchronize()
    want = [o.clone() for o in outs]
    for o in outs:
        o.fill_(float("nan"))
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            _run_noalloc(probs)
    torch.cuda.synchronize()
    other, other_outs, keep2 = _batch(gpu, 64, 1024, 4096, seed=22)
    for rep in range(3):
        for o in outs:
            o.fill_(float("nan"))
        _run_ws(other, gpu)  # eager work on the same device between the replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for g_, w_ in zip(outs, want):
            assert torch.equal(g_, w_), rep
    del graph
