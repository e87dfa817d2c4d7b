"""Shared helpers for the parity tests: tensors <-> oracle arrays."""
from __future__ import annotations

import hashlib

import numpy as np
import torch

from oracle import paged_oracle as O

TAG = {torch.float16: "f16", torch.bfloat16: "bf16"}
# max-abs tolerance of attention outputs vs the float64 oracle, per storage type
ATOL = {torch.float16: 2e-3, torch.bfloat16: 1e-2}


def bits(t: torch.Tensor) -> np.ndarray:
    """2-byte tensor -> uint16 numpy bit patterns (host copy)."""
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def f32(t: torch.Tensor) -> np.ndarray:
    return O.bits_to_f32(bits(t), TAG[t.dtype])


def sha(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def oracle_decode(q: torch.Tensor, kc: torch.Tensor, vc: torch.Tensor, bt: torch.Tensor,
                  sl: torch.Tensor, scale: float) -> np.ndarray:
    return O.decode_attention(f32(q), f32(kc), f32(vc), bt.cpu().numpy(), sl.cpu().numpy(), scale)


def max_abs(got: torch.Tensor, want: np.ndarray) -> float:
    g = f32(got).astype(np.float64)
    return float(np.max(np.abs(g - want))) if g.size else 0.0
