"""vkwr_amd: MI355X-native (gfx950) implementation of VKWR's RWKV-7 hot path.

Importing the package loads the HIP extension modules, which register the
reference's torch-op namespaces (``torch.ops.vkwr_v1_wkv``, ``vkwr_rwkv7``, ...)
with the same schemas, and the Python wrappers of ``vkwr_amd._ops`` mirror
``vkwr._ops`` (reference vkwr/__init__.py:1-3, vkwr/_ops/__init__.py:1-5).

torch is imported first on purpose: the kernels link libamdhip64.so.7 and must
bind to the HIP runtime torch already loaded.
"""
import torch  # noqa: F401  (must precede the extension modules)

from vkwr_amd._ops import import_all_ops

import_all_ops()
