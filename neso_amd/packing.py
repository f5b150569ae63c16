"""Weight layout helpers for the W4A16 kernel (host-side data preparation).

Format: codes ``c[n, k]`` in [0, 15] are packed 8 per int32 along K; column
k is nibble ``k % 8`` (bits 4*(k%8) .. 4*(k%8)+3) of word ``k // 8``, low
nibble first.  These run on whatever device the tensor lives on; they
prepare weights and are not part of the matmul itself.
"""
from __future__ import annotations

import torch


def pack_int4(codes: torch.Tensor) -> torch.Tensor:
    """[N, K] integer codes in [0, 15] -> int32 [N, K/8]."""
    if codes.dim() != 2 or codes.shape[1] % 8:
        raise ValueError("codes must be [N, K] with K a multiple of 8")
    c = codes.to(torch.int64)
    if c.numel() and (int(c.min()) < 0 or int(c.max()) > 15):
        raise ValueError("int4 codes must lie in [0, 15]")
    n, k = c.shape
    c = c.reshape(n, k // 8, 8)
    shifts = torch.arange(0, 32, 4, device=c.device, dtype=torch.int64)
    words = (c << shifts).sum(dim=-1)
    # Reinterpret the unsigned 32-bit value as int32.
    words = torch.where(words >= 2**31, words - 2**32, words)
    return words.to(torch.int32).contiguous()


def unpack_int4(words: torch.Tensor) -> torch.Tensor:
    """int32 [N, K/8] -> uint8 codes [N, K]."""
    if words.dim() != 2:
        raise ValueError("words must be [N, K/8]")
    w = words.to(torch.int64) & 0xFFFFFFFF
    shifts = torch.arange(0, 32, 4, device=w.device, dtype=torch.int64)
    codes = (w.unsqueeze(-1) >> shifts) & 0xF
    return codes.reshape(words.shape[0], -1).to(torch.uint8)
