"""Helpers for the GPU parity tests: numpy <-> device tensors, direct C-ABI calls."""
import ctypes

import numpy as np
import torch

DEV = "cuda:0"


def dev(a):
    """numpy -> device tensor with the same bits (uint16 arrays become bf16)."""
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16).to(DEV)
    return torch.from_numpy(a.copy()).to(DEV)


def host(t):
    """device tensor -> numpy (bf16 as uint16 bits)."""
    t = t.detach()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    return t.cpu().numpy()


def bits_of(t):
    return host(t)


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def rand_state(rng, N, K, sf=(-3000, 3000), exp=(-3, 3), col=(-1, 1), big_frac=0.02):
    sfv = rng.integers(sf[0], sf[1], (N, K))
    m = rng.random((N, K)) < big_frac
    sfv[m] = rng.integers(-32768, 32768, int(m.sum()))
    ss = rng.integers(-128, 128, (N, K))
    vs = rng.integers(-128, 128, (N, K))
    from oracle import oracle as O
    packed = O.pack(sfv, ss, vs)
    re = rng.integers(exp[0], exp[1] + 1, N).astype(np.int8)
    ce = rng.integers(col[0], col[1] + 1, K).astype(np.int8)
    return packed, re, ce


def rand_grad_bits(rng, N, K, lo=-5, hi=-1):
    from oracle import oracle as O
    mag = 10.0 ** rng.uniform(lo, hi, (N, 1))
    g = (rng.standard_normal((N, K)) * mag).astype(np.float32)
    g[rng.random((N, K)) < 0.05] = 0.0
    return O.f32_to_bf16_bits_array(g)


def sync():
    torch.cuda.synchronize()
