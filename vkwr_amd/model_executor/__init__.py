"""RWKV-7 model executor: weights, per-sequence slot state and the batched
decode step, composed from the vkwr_amd kernels (the reference's
vkwr/model_executor package is empty)."""
from vkwr_amd.model_executor.rwkv7 import RWKV7Config, RWKV7Model, RWKV7State, DecodeEngine  # noqa: F401
