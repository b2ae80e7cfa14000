"""PyTorch-CPU restatements (test infrastructure, and the second leg of the
CPU baseline in bench.py): tensor programs of

* the FP4 E2M1 G16 decode, mamba2_recall/fp4.py:151-154 with the nibble
  order of :125-130 and the level table of :100-103;
* the packed-row dequantization of decode_state, mamba2_recall/state_codec.py:
  269-289 (packed lane order; INT8 and INT4 tiers, zero tier 0),

running on host cores under torch.set_num_threads.  They are pinned in
tests/test_oracle_pins.py against the C oracle and against vectors the
reference's own decode_state produced (tests/golden/decode_state_vectors.npz).
Only tests/ and bench.py's cpu_baseline use this module.
"""
from __future__ import annotations

import torch

# |level| of the three magnitude bits of an E2M1 code (fp4.py:100-103)
_LEVELS = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], dtype=torch.float32)


def _nibbles(packed: torch.Tensor) -> torch.Tensor:
    """u8 [..., n/2] -> int [..., n]: low nibble first (even position)."""
    low = packed & 15
    high = packed >> 4
    return torch.stack((low, high), dim=-1).reshape(*packed.shape[:-1], packed.shape[-1] * 2)


# signed level of every code byte's two nibbles, low nibble first: [256, 2]
_SIGNED = torch.where(torch.arange(16) >= 8, -_LEVELS.repeat(2), _LEVELS.repeat(2))
_BYTE_PAIRS = torch.stack((_SIGNED[torch.arange(256) & 15], _SIGNED[torch.arange(256) >> 4]), dim=-1)


def fp4_g16_decode(codes: torch.Tensor, block_bytes: torch.Tensor, global_scale: float) -> torch.Tensor:
    """FP16 [rows, cols] of G16 codes u8 [rows, cols/2], E4M3 block bytes u8
    [rows, cols/16] and a binary32 global scale: half(((lev * sign) * block) *
    global), each product rounded in binary32 in that order (the first two
    are exact: at most six significant bits)."""
    rows, half_cols = codes.shape
    signed = _BYTE_PAIRS.index_select(0, codes.reshape(-1).to(torch.int64)).reshape(rows, half_cols * 2)
    block = block_bytes.view(torch.float8_e4m3fn).to(torch.float32)
    product = (signed.reshape(rows, -1, 16) * block[..., None]).reshape(rows, half_cols * 2)
    return (product * torch.tensor(global_scale, dtype=torch.float32)).to(torch.float16)


def decode_rows(lo: torch.Tensor, hi: torch.Tensor, q4: torch.Tensor, s8: torch.Tensor, s4: torch.Tensor,
                n8: int, n4: int) -> torch.Tensor:
    """FP32 [..., 128] of packed rows in packed lane order: the INT8 tier's
    code is the signed byte with low nibble from `lo` and high nibble from
    `hi`, the INT4 tier's the signed nibble of `q4`; each times its row's
    binary16 scale in binary32 (exact); the zero tier decodes to 0."""
    low = _nibbles(lo).to(torch.int16)
    high = _nibbles(hi).to(torch.int16)
    byte = (high << 4) | low
    code8 = torch.where(byte > 127, byte - 256, byte).to(torch.float32)
    nib4 = _nibbles(q4).to(torch.int16)
    code4 = torch.where(nib4 > 7, nib4 - 16, nib4).to(torch.float32)
    scale8 = s8.view(torch.float16).to(torch.float32)[..., None]
    scale4 = s4.view(torch.float16).to(torch.float32)[..., None]
    zero = torch.zeros(*code8.shape[:-1], 128 - n8 - n4, dtype=torch.float32)
    return torch.cat((code8 * scale8, code4 * scale4, zero), dim=-1)
