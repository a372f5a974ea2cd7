"""Shared helpers of the GPU parity tests (numpy fp16 <-> torch device tensors)."""
import sys

import numpy as np


def dev(x, device):
    import torch

    return torch.from_numpy(np.ascontiguousarray(x)).to(device)


def host(t):
    return t.detach().cpu().numpy()


def poisoned(shape, device):
    """fp16 output buffer filled with the 0x7f7f poison (reference harness.cu:50-57)."""
    import torch

    t = torch.empty(shape, dtype=torch.int16, device=device)
    t.fill_(0x7f7f)
    return t.view(torch.float16)


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()
