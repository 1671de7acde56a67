"""Helpers for the GPU parity tests: host<->device copies through torch
(device memory plumbing only) and the seeded BASELINE input distributions."""
import sys

import numpy as np
import torch


def dev_t(a):
    """numpy -> contiguous torch tensor on cuda:0 (same bits)."""
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def host(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def note(msg):
    """Flushed progress line naming the case, before each GPU step."""
    print(msg, flush=True)
    sys.stdout.flush()


def ln_inputs(rows, cols, seed):
    """BASELINE config 0 distributions: x~N(0,1), gamma=1+N(0,0.02),
    beta~N(0,0.02), dout~N(0,1)."""
    r = np.random.default_rng(seed)
    x = r.standard_normal((rows, cols), dtype=np.float32)
    gamma = (1 + 0.02 * r.standard_normal(cols)).astype(np.float32)
    beta = (0.02 * r.standard_normal(cols)).astype(np.float32)
    g = r.standard_normal((rows, cols), dtype=np.float32)
    return x, gamma, beta, g


def gelu_inputs(rows, cols, seed):
    """BASELINE config 1 distributions: pre-activation~N(0,1.5) (sigma),
    bias~N(0,0.02), dout~N(0,1)."""
    r = np.random.default_rng(seed)
    x = (1.5 * r.standard_normal((rows, cols), dtype=np.float32)).astype(np.float32)
    b = (0.02 * r.standard_normal(cols)).astype(np.float32)
    g = r.standard_normal((rows, cols), dtype=np.float32)
    return x, b, g
