"""CPU oracle for the RWKV-7 hot path -- test infrastructure only.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg
may import this package.  The product (``vkwr``, ``vkwr_amd``) never does.
"""
