def import_all_v1_ops():
    from vkwr._ops.v1 import v1_linear_ops, v1_mix_ops, v1_norm_ops, v1_rank_ops, v1_wkv_ops  # noqa: F401
