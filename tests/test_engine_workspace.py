"""GEMM workspace sizing of the engines and the planner's empty-problem cases (host only).

vkwr_gemm_f16's plan -- tile shape, K splits, the large-M kernel's split last
round -- depends on the row count in a way that is not monotone, so an engine
must size its workspace for every row count a step can have.  These tests run the
engines' own sizing on the BASELINE config-3/4 shapes with host tensors (the
planner reads only sizes and pointer alignment; no kernel runs) and check every
reachable row count against the planner.
"""
import ctypes
import types

import pytest
import torch

from vkwr_amd import capi
from vkwr.model_executor import DecodeEngine, MixedEngine, RWKV7Config
from vkwr.model_executor.rwkv7 import LAYER_VECS


def _host_model(cfg, n_layer=2):
    """A model of cfg's shapes whose weights are uninitialised host tensors (sizing only)."""
    C, F = cfg.n_embd, cfg.dim_ffn
    e = lambda *s: torch.empty(*s, dtype=torch.float16)  # noqa: E731
    layers = []
    for l in range(n_layer):
        L = {k: e(C) for k in LAYER_VECS}
        L.update(Wr=e(C, C), Wk=e(C, C), Wv=e(C, C), Wo=e(C, C), w1=e(cfg.rank_w, C), w2=e(C, cfg.rank_w),
                 a1=e(cfg.rank_a, C), a2=e(C, cfg.rank_a), g1=e(cfg.rank_g, C), g2=e(C, cfg.rank_g),
                 key=e(F, C), value=e(C, F))
        if l > 0:
            L.update(v1=e(cfg.rank_v, C), v2=e(C, cfg.rank_v))
        layers.append(L)
    return types.SimpleNamespace(cfg=cfg, layers=layers, head=e(cfg.vocab, C), emb=e(cfg.vocab, C),
                                 ln_out_w=e(C), ln_out_b=e(C))


def test_mixed_engine_workspace_covers_every_row_count_7b():
    """Config 4 (7B shape, 256 decode rows + 4 x 512 chunks = 2304 rows): every GEMM launch the
    step can issue, at every row count 1..2304 (and the head at 1..260 sequences), fits the
    engine's workspace (the split of a GEMM's last round into k-parts, and so its workspace,
    is not monotone in the row count, so every count is checked)."""
    cfg = RWKV7Config.preset("7b")
    eng = MixedEngine(_host_model(cfg), 2304, max_seqs=260)
    have = eng.ws.numel()
    worst = 0
    for R in range(1, 2305):
        for ps in eng._gemm_batches(R, 2):
            need = capi.gemm_workspace_bytes(ps)
            assert need <= have, (R, need, have)
            worst = max(worst, need)
    for S in range(1, 261):
        assert capi.gemm_workspace_bytes(eng._head_problem(S)) <= have
    assert worst == have or capi.gemm_workspace_bytes_upto(eng._head_problem(260)) == have


def test_decode_engine_rowmajor_workspace_covers_every_batch_1p5b():
    """Config 3 shape on the row-major GEMM path (frag=False) with up to 300 rows."""
    cfg = RWKV7Config.preset("1.5b")
    eng = DecodeEngine(_host_model(cfg), 300, frag=False)
    have = eng.ws.numel()
    for B in range(1, 301):
        for ps in eng._all_gemms(B):
            assert capi.gemm_workspace_bytes(ps) <= have, B


def _problem(m, n, k):
    p = ctypes.c_void_p(0x100000)  # never dereferenced: planning only
    return capi.GemmProblem(p, p, p, m, n, k, capi.GEMM_B_NK, capi.ACT_NONE, capi.EPI_NONE, None, None, None)


@pytest.mark.parametrize("m,n,k", [(1, 64, 0), (0, 64, 64), (64, 0, 64), (0, 0, 0), (300, 4096, 0)])
def test_planner_empty_problems(m, n, k):
    """K == 0 (every output is epilogue(0)) and empty problems plan without a K split and
    need no workspace (they used to divide by zero in the planner)."""
    assert capi.gemm_workspace_bytes([_problem(m, n, k)]) == 0
    assert capi.gemm_workspace_bytes([_problem(m, n, k), _problem(0, 8, 8)]) == 0


def test_planner_batch_with_one_empty_problem():
    """A batch mixing an empty problem with a real one plans the real one as alone."""
    alone = capi.gemm_workspace_bytes([_problem(8, 2048, 2048)])
    assert capi.gemm_workspace_bytes([_problem(0, 2048, 2048), _problem(8, 2048, 2048)]) == alone
    assert alone > 0  # 8 rows x 16 tiles leave the CUs idle: K is split
