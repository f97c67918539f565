"""vkwr_v1_rank wrappers (reference vkwr/_ops/v1/v1_rank_ops.py:1-57): the
RWKV-7 w/a/g(/v) low-rank adapters.  Names, signatures and fakes match the
reference."""
import torch
import torch.library

from vkwr import _v1_rank_C  # noqa: F401  (registers the ops)


@torch.library.register_fake("vkwr_v1_rank::linear_wag_rank_in_f16")
def _(M, K, Rw, Ra, Rg, xw, xa, xg, w1_t, a1_t, g1_t):
    return [torch.empty(M, R, dtype=xw.dtype, device=xw.device) for R in (Rw, Ra, Rg)]


def linear_wag_rank_in_f16(M, K, Rw, Ra, Rg, xw, xa, xg, w1_t, a1_t, g1_t):
    return torch.ops.vkwr_v1_rank.linear_wag_rank_in_f16(M, K, Rw, Ra, Rg, xw, xa, xg, w1_t, a1_t, g1_t)


@torch.library.register_fake("vkwr_v1_rank::linear_wagv_rank_in_f16")
def _(M, K, Rw, Ra, Rg, Rv, xw, xa, xg, xv, w1_t, a1_t, g1_t, v1_t):
    return [torch.empty(M, R, dtype=xw.dtype, device=xw.device) for R in (Rw, Ra, Rg, Rv)]


def linear_wagv_rank_in_f16(M, K, Rw, Ra, Rg, Rv, xw, xa, xg, xv, w1_t, a1_t, g1_t, v1_t):
    return torch.ops.vkwr_v1_rank.linear_wagv_rank_in_f16(M, K, Rw, Ra, Rg, Rv, xw, xa, xg, xv, w1_t, a1_t, g1_t,
                                                          v1_t)


@torch.library.register_fake("vkwr_v1_rank::linear_wag_rank_out_f16")
def _(M, C, Kw, Ka, Kg, w1, a1, g1, w2_t, a2_t, g2_t):
    return [torch.empty(M, C, dtype=w1.dtype, device=w1.device) for _ in range(3)]


def linear_wag_rank_out_f16(M, C, Kw, Ka, Kg, w1, a1, g1, w2_t, a2_t, g2_t):
    return torch.ops.vkwr_v1_rank.linear_wag_rank_out_f16(M, C, Kw, Ka, Kg, w1, a1, g1, w2_t, a2_t, g2_t)


@torch.library.register_fake("vkwr_v1_rank::linear_wagv_rank_out_f16")
def _(M, C, Kw, Ka, Kg, Kv, w1, a1, g1, v1, w2_t, a2_t, g2_t, v2_t, v, v_first, v0):
    return [torch.empty(M, C, dtype=w1.dtype, device=w1.device) for _ in range(4)]


def linear_wagv_rank_out_f16(M, C, Kw, Ka, Kg, Kv, w1, a1, g1, v1, w2_t, a2_t, g2_t, v2_t, v, v_first, v0):
    return torch.ops.vkwr_v1_rank.linear_wagv_rank_out_f16(M, C, Kw, Ka, Kg, Kv, w1, a1, g1, v1, w2_t, a2_t, g2_t,
                                                           v2_t, v, v_first, v0)
