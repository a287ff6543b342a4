"""Bit-pattern helpers shared by the tests."""
import numpy as np


def bits_u16(t):
    """bf16 torch tensor -> numpy uint16 bit patterns."""
    import torch
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def bits_u8(t):
    import torch
    return t.detach().cpu().contiguous().view(torch.uint8).numpy()


def from_u16(a, device=None):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint16).view(np.int16)).view(torch.bfloat16)
    return t.to(device) if device is not None else t
