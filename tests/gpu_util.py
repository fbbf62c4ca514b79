"""Helpers for the GPU parity tests: torch only provides device memory and the stream; every
computation under test goes through the C-ABI of libaic_hip.so."""
import numpy as np
import torch

from autonomousaicore_amd import _lib


def dev(a, dtype=None):
    """numpy -> contiguous cuda tensor (float32 / int64 / bf16 when dtype=torch.bfloat16)."""
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.to("cuda").contiguous()


def host(t):
    torch.cuda.synchronize()
    if t.dtype == torch.bfloat16:
        t = t.float()
    return t.detach().cpu().numpy()


def bf16_round(a):
    """Round a float32 numpy array to bf16 and back (round to nearest even)."""
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16).float().numpy()


def ptr(t):
    return t.data_ptr() if t is not None else None


def stream():
    return torch.cuda.current_stream().cuda_stream


def call(name, *args):
    _lib.call(name, *args)


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    nb = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (nb if nb > 0 else 1.0))
