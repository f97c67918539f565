"""vkwr: the reference's Python package, MI355X-native.

``import vkwr`` registers the reference's torch-op namespaces
(``torch.ops.vkwr_v1_wkv``, ``vkwr_v1_linear``, ``vkwr_v1_rank``, ``vkwr_v1_mix``,
``vkwr_v1_norm``, ``vkwr_rwkv7``, ``vkwr_sampling``) with the reference's schemas,
through the extension modules ``vkwr._v1_wkv_C`` ... ``vkwr._sampling_C`` built
next to this file; their kernels are the gfx950 HIP kernels of ``vkwr_amd``
(``libvkwr_amd.so``, C ABI ``include/vkwr_amd.h``).  The import lines are the
reference's own (vkwr/__init__.py:1-3, vkwr/_ops/__init__.py:1-5,
vkwr/_ops/v1/v1_wkv_ops.py:3).  There is no CPU fallback: a missing build
raises ImportError here.
"""
import os as _os

import torch as _torch  # noqa: F401  (first: the kernels bind to the HIP runtime torch loads)

_HERE = _os.path.dirname(_os.path.abspath(__file__))
_EXTS = ("_v1_wkv_C", "_v1_linear_C", "_v1_rank_C", "_v1_mix_C", "_v1_norm_C", "_rwkv7_C", "_sampling_C")
_missing = [n for n in _EXTS if not _os.path.exists(_os.path.join(_HERE, n + ".so"))]
if _missing:
    raise ImportError(f"vkwr: native extension modules not built: {', '.join(_missing)}. Build them with "
                      "`python -c 'import __graft_entry__ as g; g.build()'` (gfx950 HIP kernels); "
                      "there is no CPU fallback.")

from vkwr._ops import import_all_ops  # noqa: E402

import_all_ops()
