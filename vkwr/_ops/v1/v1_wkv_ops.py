"""vkwr_v1_wkv wrappers (reference vkwr/_ops/v1/v1_wkv_ops.py:1-109).

Names, signatures and output allocation match the reference.  Fake (meta)
registrations return None for the ``-> ()`` schemas (the reference returned
lists, which disagrees with its own schemas).  The slot-pool wrappers at the
end are additions: they have no reference counterpart.
"""
import torch
import torch.library

from vkwr import _v1_wkv_C  # noqa: F401  (registers the ops)

HEAD_SIZE = 64


@torch.library.register_fake("vkwr_v1_wkv::wkv_seq_fp16")
def _(B, T, C, H, state, r, w, k, v, a, b, y, elapsed_t):
    return None


@torch.library.register_fake("vkwr_v1_wkv::wkv_seq_w0_fp16")
def _(B, T, C, H, state, r, w, w0, k, v, a, b, y, elapsed_t):
    return None


@torch.library.register_fake("vkwr_v1_wkv::wkv_one_fp16")
def _(B, C, H, state, r, w, k, v, a, b, y, elapsed_t):
    return None


@torch.library.register_fake("vkwr_v1_wkv::wkv_one_w0_fp16")
def _(B, C, H, state, r, w, w0, k, v, a, b, y, elapsed_t):
    return None


for _name in ("wkv_forward_fp32", "wkv_forward_seq_fp32", "wkv_forward_small_fp32", "wkv_forward_block_fp32"):
    torch.library.register_fake(f"vkwr_v1_wkv::{_name}")(
        lambda B, T, C, H, state, r, w, k, v, a, b, y: None)


@torch.library.register_fake("vkwr_v1_wkv::advance_i32")
def _(x, amount):
    return None


@torch.library.register_fake("vkwr_v1_wkv::wkv_forward_slots_fp32")
def _(B, T, C, H, state_pool, slots, r, w, k, v, a, b, y):
    return None


# ===== fp16-state wrappers: output buffer + zero elapsed_t =====
def wkv_seq_fp16(B, T, C, H, state, r, w, k, v, a, b):
    y = torch.empty(B, T, C, dtype=r.dtype, device=r.device)
    elapsed_t = torch.zeros(B, dtype=torch.int32, device=r.device)
    torch.ops.vkwr_v1_wkv.wkv_seq_fp16(B, T, C, H, state, r, w, k, v, a, b, y, elapsed_t)
    return y, elapsed_t


def wkv_seq_w0_fp16(B, T, C, H, state, r, w, w0, k, v, a, b):
    y = torch.empty(B, T, C, dtype=r.dtype, device=r.device)
    elapsed_t = torch.zeros(B, dtype=torch.int32, device=r.device)
    torch.ops.vkwr_v1_wkv.wkv_seq_w0_fp16(B, T, C, H, state, r, w, w0, k, v, a, b, y, elapsed_t)
    return y, elapsed_t


def wkv_one_fp16(B, C, H, state, r, w, k, v, a, b):
    y = torch.empty(B, C, dtype=r.dtype, device=r.device)
    elapsed_t = torch.zeros(B, dtype=torch.int32, device=r.device)
    torch.ops.vkwr_v1_wkv.wkv_one_fp16(B, C, H, state, r, w, k, v, a, b, y, elapsed_t)
    return y, elapsed_t


def wkv_one_w0_fp16(B, C, H, state, r, w, w0, k, v, a, b):
    y = torch.empty(B, C, dtype=r.dtype, device=r.device)
    elapsed_t = torch.zeros(B, dtype=torch.int32, device=r.device)
    torch.ops.vkwr_v1_wkv.wkv_one_w0_fp16(B, C, H, state, r, w, w0, k, v, a, b, y, elapsed_t)
    return y, elapsed_t


# ===== fp32-state wrappers: output buffer, no elapsed_t =====
def wkv_forward_fp32(B, T, C, H, state, r, w, k, v, a, b):
    y = torch.empty(B, T, C, dtype=r.dtype, device=r.device)
    torch.ops.vkwr_v1_wkv.wkv_forward_fp32(B, T, C, H, state, r, w, k, v, a, b, y)
    return y


def wkv_forward_seq_fp32(B, T, C, H, state, r, w, k, v, a, b):
    y = torch.empty(B, T, C, dtype=r.dtype, device=r.device)
    torch.ops.vkwr_v1_wkv.wkv_forward_seq_fp32(B, T, C, H, state, r, w, k, v, a, b, y)
    return y


def wkv_forward_small_fp32(B, T, C, H, state, r, w, k, v, a, b):
    y = torch.empty(B, T, C, dtype=r.dtype, device=r.device)
    torch.ops.vkwr_v1_wkv.wkv_forward_small_fp32(B, T, C, H, state, r, w, k, v, a, b, y)
    return y


def wkv_forward_block_fp32(B, T, C, H, state, r, w, k, v, a, b):
    y = torch.empty(B, T, C, dtype=r.dtype, device=r.device)
    torch.ops.vkwr_v1_wkv.wkv_forward_block_fp32(B, T, C, H, state, r, w, k, v, a, b, y)
    return y


# ===== advance_i32: in place, returns None =====
def advance_i32(x, amount):
    torch.ops.vkwr_v1_wkv.advance_i32(x, amount)


# ===== slot-pool state (additions; no reference counterpart) =====
def validate_slots(slots, pool_size):
    """Host-side check that `slots` is a set of distinct indices in [0, pool_size).

    Costs a device->host copy; meant for admission-time checks, not the step loop.
    """
    s = slots.detach().to("cpu", torch.int64)
    if s.dim() != 1:
        raise RuntimeError("slots must have shape [B]")
    if s.numel() and (int(s.min()) < 0 or int(s.max()) >= pool_size):
        raise RuntimeError(f"slot index out of range [0, {pool_size})")
    if torch.unique(s).numel() != s.numel():
        raise RuntimeError("slots must be distinct")


def wkv_forward_slots_fp32(B, T, C, H, state_pool, slots, r, w, k, v, a, b, validate=True):
    """WKV-7 over T tokens with sequence i's fp32 state read from and written back to
    state_pool[slots[i]] in the same pass (replaces index_select -> wkv_forward_fp32 ->
    index_copy_).  Entries of state_pool not named by slots are left bitwise unchanged.

    Out-of-range or duplicate slots raise RuntimeError before the launch (a host check:
    the slots are copied to the host).  validate=False skips it, for callers whose slot
    table is checked on the host already (the continuous batcher's allocator); the kernel
    then still bounds-checks every slot (an out-of-range slot's y rows are NaN and the pool
    is untouched), but duplicate slots race."""
    if validate:
        validate_slots(slots, state_pool.size(0))
    y = torch.empty(B, T, C, dtype=r.dtype, device=r.device)
    torch.ops.vkwr_v1_wkv.wkv_forward_slots_fp32(B, T, C, H, state_pool, slots, r, w, k, v, a, b, y)
    return y


def wkv_one_slots_fp32(B, C, H, state_pool, slots, r, w, k, v, a, b, validate=True):
    """Decode step (T=1) of wkv_forward_slots_fp32; r..b are [B,C], y is [B,C]."""
    y = wkv_forward_slots_fp32(B, 1, C, H, state_pool, slots,
                               *(x.view(B, 1, C) for x in (r, w, k, v, a, b)), validate=validate)
    return y.view(B, C)
