"""Helpers to read the golden .npz fixtures and to draw seeded op inputs."""

import os

import numpy as np
import torch

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load_npz(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


def bf16_from_bits(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)


def gdn_inputs(B, W, T, H, HV, K, V, *, dtype=torch.bfloat16, seed=0, state_std=0.02,
               state_dtype=torch.float32):
    """Config-2 distributions: q,k,v ~ N(0,1); g = -softplus(N(0,1)) fp32;
    beta = sigmoid(N(0,1)) in the activation dtype; S ~ N(0, state_std^2)."""
    g = torch.Generator().manual_seed(seed)
    BW = B * W
    q = torch.randn(BW, T, H, K, generator=g).to(dtype)
    k = torch.randn(BW, T, H, K, generator=g).to(dtype)
    v = torch.randn(BW, T, HV, V, generator=g).to(dtype)
    gate = -torch.nn.functional.softplus(torch.randn(BW, T, HV, generator=g))
    beta = torch.sigmoid(torch.randn(BW, T, HV, generator=g)).to(dtype)
    S = (torch.randn(B, HV, K, V, generator=g) * state_std).to(state_dtype)
    return q, k, v, gate, beta, S


def conv_inputs(B, W, C, T, *, dtype=torch.bfloat16, seed=0, history=3):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B * W, C, T, generator=g).to(dtype)
    st = torch.randn(B, C, history, generator=g).to(dtype)
    w = (torch.rand(C, 4, generator=g) - 0.5).to(dtype)
    return x, st, w
