"""NumPy storage arrays <-> torch tensors (bit-preserving)."""

from __future__ import annotations

import numpy as np
import torch

TORCH_DTYPE = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}
NAME_OF = {v: k for k, v in TORCH_DTYPE.items()}


def to_torch(arr: np.ndarray, dtype: str, device="cuda") -> torch.Tensor:
    if dtype == "fp8_e4m3":  # uint8 codes
        return torch.from_numpy(np.ascontiguousarray(arr, dtype=np.uint8)).to(device)
    if dtype == "float32":
        t = torch.from_numpy(np.ascontiguousarray(arr, dtype=np.float32))
    else:
        t = torch.from_numpy(np.ascontiguousarray(arr, dtype=np.uint16).view(np.int16)).view(TORCH_DTYPE[dtype])
    return t.to(device)


def to_index(arr: np.ndarray, device="cuda", dtype=torch.int32) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(arr)).to(dtype).to(device)


def to_numpy(t: torch.Tensor) -> np.ndarray:
    """Storage array of a tensor (uint16 bits for 16-bit floats)."""
    t = t.detach().cpu().contiguous()
    if t.dtype in (torch.float32, torch.uint8):
        return t.numpy()
    return t.view(torch.int16).numpy().view(np.uint16)


def to_f64(t: torch.Tensor) -> np.ndarray:
    return t.detach().to(torch.float64).cpu().numpy()
