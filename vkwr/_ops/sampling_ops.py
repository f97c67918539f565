"""Sampling op wrappers (the module reference vkwr/_ops/__init__.py:2 imports).

The reference registers the ops vkwr_sampling::{setup_rand,
temperature_topk_topp, repetition_topk_topp} (csrc/sampling/torch_bindings.cpp:36-48)
but does not ship this Python module; these wrappers keep the op names and
argument meaning and add fake (meta) kernels so the ops trace.

    states = setup_rand(seed, B)                 # int8 [B * 32] on the current device
    tok = temperature_topk_topp(logits, states, temperature, top_k, top_p)
    tok = repetition_topk_topp(logits, penalties, states, presence, repetition,
                               decay, temperature, top_k, top_p)   # updates penalties

logits: fp32 [B, V] or [B, T, V] (row b samples from its last token); tok: int32 [B].
"""
import torch
import torch.library

from vkwr import _sampling_C  # noqa: F401  (registers the ops)

STATE_BYTES = 32  # VKWR_SAMPLING_STATE_BYTES


@torch.library.register_fake("vkwr_sampling::temperature_topk_topp")
def _(logits, states, temperature, top_k, top_p):
    B = logits.size(0) if logits.dim() >= 2 else 1
    return logits.new_empty((B,), dtype=torch.int32)


@torch.library.register_fake("vkwr_sampling::repetition_topk_topp")
def _(logits, penalties, states, presence_penalty, repetition_penalty, penalty_decay, temperature, top_k, top_p):
    B = penalties.size(0) if penalties.dim() == 2 else 1
    return logits.new_empty((B,), dtype=torch.int32)


def setup_rand(seed, B):
    """Per-row Philox states for B rows: row b draws from counter subsequence b of `seed`."""
    return torch.ops.vkwr_sampling.setup_rand(seed, B)


def temperature_topk_topp(logits, states, temperature=1.0, top_k=-1, top_p=1.0):
    """One token per row from softmax(logits / temperature) truncated to top_k / top_p.
    top_k <= 0 or > V: no top-k limit; top_p outside [0, 1]: 1; top_p == 0: greedy."""
    return torch.ops.vkwr_sampling.temperature_topk_topp(logits, states, temperature, top_k, top_p)


def repetition_topk_topp(logits, penalties, states, presence_penalty=0.0, repetition_penalty=0.0,
                         penalty_decay=1.0, temperature=1.0, top_k=-1, top_p=1.0):
    """As temperature_topk_topp on logits - penalties; then, in place,
    penalties = penalties * decay + (presence if the drawn token had penalty 0 else repetition)
    on the drawn token of each row."""
    return torch.ops.vkwr_sampling.repetition_topk_topp(logits, penalties, states, presence_penalty,
                                                        repetition_penalty, penalty_decay, temperature,
                                                        top_k, top_p)


__all__ = ["setup_rand", "temperature_topk_topp", "repetition_topk_topp", "STATE_BYTES"]
