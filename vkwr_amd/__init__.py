"""vkwr_amd: the MI355X-native (gfx950) kernels of VKWR's RWKV-7 hot path.

``libvkwr_amd.so`` holds the hand-written HIP kernels behind the C ABI of
include/vkwr_amd.h; ``vkwr_amd.capi`` binds that ABI with ctypes for the model
executor.  The reference-facing package is ``vkwr``: its extension modules
(``vkwr._v1_wkv_C`` ...) register the reference's torch ops on these kernels.

torch is imported first on purpose: the kernels link libamdhip64.so.7 and must
bind to the HIP runtime torch already loaded.
"""
import torch  # noqa: F401  (must precede the kernel library)
