"""vkwr_v1_linear wrappers (reference vkwr/_ops/v1/v1_linear_ops.py:1-184).

Names and signatures match the reference.  Fake (meta) registrations return
x.shape[:-1] + [N] for every op -- including the m1_splitk family, whose
reference fakes returned [N] while the real ops return x.shape[:-1] + [N]
(reference v1_linear_ops.py:105-142 vs csrc/v1/linear/linear_ops.cu:1403-1405).
"""
import torch
import torch.library

from vkwr import _v1_linear_C  # noqa: F401  (registers the ops)


def _out(x, n):
    return torch.empty(list(x.shape[:-1]) + [n], dtype=x.dtype, device=x.device)


@torch.library.register_fake("vkwr_v1_linear::linear_f16")
def _(x, weight):
    return _out(x, weight.shape[1])


def linear_f16(x, weight):
    return torch.ops.vkwr_v1_linear.linear_f16(x, weight)

@torch.library.register_fake("vkwr_v1_linear::linear_f16_orig")
def _(x, weight_orig):
    return _out(x, weight_orig.shape[0])


def linear_f16_orig(x, weight_orig):
    return torch.ops.vkwr_v1_linear.linear_f16_orig(x, weight_orig)

@torch.library.register_fake("vkwr_v1_linear::linear_orig_rows_f16")
def _(x, weight_orig, row_tile, out_tile):
    return _out(x, weight_orig.shape[0])


def linear_orig_rows_f16(x, weight_orig, row_tile, out_tile):
    return torch.ops.vkwr_v1_linear.linear_orig_rows_f16(x, weight_orig, row_tile, out_tile)

@torch.library.register_fake("vkwr_v1_linear::linear_orig_rows_cfg_f16")
def _(x, weight_orig, threads, row_tile, out_tile):
    return _out(x, weight_orig.shape[0])


def linear_orig_rows_cfg_f16(x, weight_orig, threads, row_tile, out_tile):
    return torch.ops.vkwr_v1_linear.linear_orig_rows_cfg_f16(x, weight_orig, threads, row_tile, out_tile)

@torch.library.register_fake("vkwr_v1_linear::linear_orig_rows_exact_f16")
def _(x, weight_orig, threads, out_tile, use4):
    return _out(x, weight_orig.shape[0])


def linear_orig_rows_exact_f16(x, weight_orig, threads, out_tile, use4):
    return torch.ops.vkwr_v1_linear.linear_orig_rows_exact_f16(x, weight_orig, threads, out_tile, use4)

@torch.library.register_fake("vkwr_v1_linear::linear_orig_wmma16_f16")
def _(x, weight_orig):
    return _out(x, weight_orig.shape[0])


def linear_orig_wmma16_f16(x, weight_orig):
    return torch.ops.vkwr_v1_linear.linear_orig_wmma16_f16(x, weight_orig)

@torch.library.register_fake("vkwr_v1_linear::linear_f16_orig_lt")
def _(x, weight_orig):
    return _out(x, weight_orig.shape[0])


def linear_f16_orig_lt(x, weight_orig):
    return torch.ops.vkwr_v1_linear.linear_f16_orig_lt(x, weight_orig)

@torch.library.register_fake("vkwr_v1_linear::linear_f16_orig_lt_cfg")
def _(x, weight_orig, workspace_mb, algo_index):
    return _out(x, weight_orig.shape[0])


def linear_f16_orig_lt_cfg(x, weight_orig, workspace_mb, algo_index):
    return torch.ops.vkwr_v1_linear.linear_f16_orig_lt_cfg(x, weight_orig, workspace_mb, algo_index)

@torch.library.register_fake("vkwr_v1_linear::linear_f16_lt")
def _(x, weight):
    return _out(x, weight.shape[1])


def linear_f16_lt(x, weight):
    return torch.ops.vkwr_v1_linear.linear_f16_lt(x, weight)

@torch.library.register_fake("vkwr_v1_linear::linear_f16_m1_splitk")
def _(x, weight):
    return _out(x, weight.shape[1])


def linear_f16_m1_splitk(x, weight):
    return torch.ops.vkwr_v1_linear.linear_f16_m1_splitk(x, weight)

@torch.library.register_fake("vkwr_v1_linear::linear_f16_m1_splitk_cfg")
def _(x, weight, chunk_k):
    return _out(x, weight.shape[1])


def linear_f16_m1_splitk_cfg(x, weight, chunk_k):
    return torch.ops.vkwr_v1_linear.linear_f16_m1_splitk_cfg(x, weight, chunk_k)

@torch.library.register_fake("vkwr_v1_linear::linear_f16_m1_splitk_tile")
def _(x, weight, chunk_k, tile_cols):
    return _out(x, weight.shape[1])


def linear_f16_m1_splitk_tile(x, weight, chunk_k, tile_cols):
    return torch.ops.vkwr_v1_linear.linear_f16_m1_splitk_tile(x, weight, chunk_k, tile_cols)

@torch.library.register_fake("vkwr_v1_linear::linear_f16_m1_splitk_warpred_tile")
def _(x, weight, chunk_k, tile_cols):
    return _out(x, weight.shape[1])


def linear_f16_m1_splitk_warpred_tile(x, weight, chunk_k, tile_cols):
    return torch.ops.vkwr_v1_linear.linear_f16_m1_splitk_warpred_tile(x, weight, chunk_k, tile_cols)

@torch.library.register_fake("vkwr_v1_linear::linear_f16_rows_splitk")
def _(x, weight, chunk_k):
    return _out(x, weight.shape[1])


def linear_f16_rows_splitk(x, weight, chunk_k):
    return torch.ops.vkwr_v1_linear.linear_f16_rows_splitk(x, weight, chunk_k)

@torch.library.register_fake("vkwr_v1_linear::linear_t_f16")
def _(x, weight_t):
    return _out(x, weight_t.shape[0])


def linear_t_f16(x, weight_t):
    return torch.ops.vkwr_v1_linear.linear_t_f16(x, weight_t)

@torch.library.register_fake("vkwr_v1_linear::linear_t_act_f16")
def _(x, weight_t, act):
    return _out(x, weight_t.shape[0])


def linear_t_act_f16(x, weight_t, act):
    return torch.ops.vkwr_v1_linear.linear_t_act_f16(x, weight_t, act)

@torch.library.register_fake("vkwr_v1_linear::linear_t_vres_f16")
def _(x, weight_t, v, v_first, v0):
    return torch.empty_like(v)


def linear_t_vres_f16(x, weight_t, v, v_first, v0):
    return torch.ops.vkwr_v1_linear.linear_t_vres_f16(x, weight_t, v, v_first, v0)
