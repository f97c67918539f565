"""RWKV-7 model executor: weights, per-sequence slot state, the batched decode
step (on the driver's fused entry points, or composed only of the reference's op
surface), the mixed prefill + decode step, a continuous-batching scheduler and a
GPU token sampler,
composed from the vkwr_amd kernels (the reference's vkwr/model_executor package
is empty)."""
from vkwr.model_executor.rwkv7 import RWKV7Config, RWKV7Model, RWKV7State, DecodeEngine  # noqa: F401
from vkwr.model_executor.mixed import MixedEngine  # noqa: F401
from vkwr.model_executor.op_engine import OpDecodeEngine  # noqa: F401
from vkwr.model_executor.scheduler import ContinuousBatcher, Request, SlotAllocator  # noqa: F401
from vkwr.model_executor.sampling import GpuSampler  # noqa: F401
