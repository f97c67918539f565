"""Op loader (reference vkwr/_ops/__init__.py:1-5).

The reference also imports ``sampling_ops``, a module it does not ship (so
``import vkwr`` fails there); here it wraps the vkwr_sampling ops.
"""


def import_all_ops():
    from vkwr._ops import rwkv7_ops, sampling_ops  # noqa: F401
    from vkwr._ops.v1 import import_all_v1_ops

    import_all_v1_ops()
