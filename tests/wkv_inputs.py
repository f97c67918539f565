"""Seeded WKV-7 input generators shared by the tests and bench.py.

``baseline`` follows BASELINE config 0: r,k,v ~ N(0,1); w = exp(-0.6065*sigmoid(N(0,1)))
passed verbatim as the op's raw w; kk = k / ||k|| per head; a = -kk; b = kk*sigmoid(N(0,1)).
``realistic`` follows the reference test helper _make_wkv_realistic_inputs
(reference tests/ops/test_v1_wkv_ops.py:67-132): r,k,v ~ 0.2 N(0,1), w = tanh(N(0,1)),
a = -unit(kk), b = unit(kk)*sigmoid(N(0,1)).
All draws use a CPU torch.Generator so the values do not depend on the device.
"""
import numpy as np
import torch


def make_wkv_inputs(B, T, H, seed=0, dist="baseline"):
    g = torch.Generator().manual_seed(seed)
    C = H * 64
    f32 = torch.float32

    def n(*shape):
        return torch.randn(*shape, generator=g, dtype=f32)

    if dist == "baseline":
        r = n(B, T, C).half()
        k = n(B, T, C).half()
        v = n(B, T, C).half()
        w = torch.exp(-0.6065 * torch.sigmoid(n(B, T, C))).half()
        kk = k.float().view(B, T, H, 64)
        kk = kk / kk.norm(dim=-1, keepdim=True).clamp_min(1e-12)
        a_vec = torch.sigmoid(n(B, T, H, 64))
        a = (-kk).reshape(B, T, C).half()
        b = (kk * a_vec).reshape(B, T, C).half()
    elif dist == "realistic":
        r = (n(B, T, C) * 0.2).half()
        k = (n(B, T, C) * 0.2).half()
        v = (n(B, T, C) * 0.2).half()
        w = torch.tanh(n(B, T, C)).half()
        kk = n(B, T, H, 64)
        kk = kk / (kk.norm(dim=-1, keepdim=True) + 1e-8)
        gate = torch.sigmoid(n(B, T, H, 64))
        a = (-kk).reshape(B, T, C).half()
        b = (kk * gate).reshape(B, T, C).half()
    elif dist == "randn":  # unbounded, shape/dtype tests only
        r, w, k, v, a, b = (n(B, T, C).half() for _ in range(6))
    else:
        raise ValueError(dist)
    return [x.numpy() for x in (r, w, k, v, a, b)]


def make_state(B, H, seed=0, std=0.1, dtype=np.float32):
    if std == 0:
        return np.zeros((B, H, 64, 64), dtype=dtype)
    g = torch.Generator().manual_seed(seed + 1000003)
    s = torch.randn(B, H, 64, 64, generator=g, dtype=torch.float32) * std
    return s.numpy().astype(dtype)
