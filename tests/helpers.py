"""Shared input builders for the parity tests (numpy, seeded)."""

from __future__ import annotations

import numpy as np
import torch

from oracle.fp8 import bf16_bits, bf16_from_bits, bf16_round

PAGE = 64


def bf16_tensor(x: np.ndarray, device) -> torch.Tensor:
    """float32 numpy (rounded to bf16) -> bf16 torch tensor with the same bits."""
    bits = bf16_bits(np.asarray(x, np.float32))
    return torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16).to(device)


def bf16_values(t: torch.Tensor) -> np.ndarray:
    return bf16_from_bits(t.detach().cpu().view(torch.int16).numpy().view(np.uint16))


def randn_bf16(rng: np.random.Generator, shape, scale: float = 1.0) -> np.ndarray:
    return bf16_round((rng.standard_normal(shape) * scale).astype(np.float32))


def permuted_block_table(rng: np.random.Generator, num_seqs: int, pages_per_seq: int) -> np.ndarray:
    perm = rng.permutation(num_seqs * pages_per_seq).astype(np.int32)
    return perm.reshape(num_seqs, pages_per_seq)


def to_dev(a: np.ndarray, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)
