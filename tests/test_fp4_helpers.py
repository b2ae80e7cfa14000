"""The FP4 format helpers of the drop-in surface, on the CPU: decode_e2m1,
pack_nibbles and unpack_nibbles (reference mamba2_recall/fp4.py:100-130).

decode_e2m1 is checked for all 16 codes against the E2M1 closed form of
docs/FP4_WEIGHT_V1_PROTOCOL.md (magnitudes 0, .5, 1, 1.5, 2, 3, 4, 6 for
bits 0-2, bit 3 the sign; code 8 is -0.0), bit for bit including the sign of
zero.  The nibble packing is checked against an independent numpy packing
(low nibble = even column), over even and odd widths, with the reference's
error messages for out-of-range codes, a wrong packed width and nonzero
padding."""
import numpy as np
import pytest
import torch

from mamba2_recall import fp4

CLOSED_FORM = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]


def test_decode_e2m1_all_codes_closed_form():
    codes = torch.arange(16, dtype=torch.uint8)
    got = fp4.decode_e2m1(codes)
    assert got.dtype == torch.float32
    want = np.array([(-1.0 if c & 8 else 1.0) * CLOSED_FORM[c & 7] for c in range(16)], dtype=np.float32)
    assert np.array_equal(got.numpy().view(np.uint32), want.view(np.uint32))
    assert got.numpy().view(np.uint32)[8] == 0x80000000   # code 8: negative zero
    # shape preserved for a matrix of codes
    m = torch.tensor([[0, 15], [7, 9]], dtype=torch.uint8)
    assert fp4.decode_e2m1(m).tolist() == [[0.0, -6.0], [6.0, -0.5]]


def test_decode_e2m1_rejects_bad_codes():
    with pytest.raises(ValueError, match="E2M1 codes must be uint8"):
        fp4.decode_e2m1(torch.zeros(4, dtype=torch.int32))
    with pytest.raises(ValueError, match="E2M1 nibble outside"):
        fp4.decode_e2m1(torch.tensor([3, 16], dtype=torch.uint8))


def _np_pack(codes):
    rows, cols = codes.shape
    out = np.zeros((rows, (cols + 1) // 2), dtype=np.uint8)
    for c in range(cols):
        out[:, c // 2] |= (codes[:, c] << (4 * (c % 2))).astype(np.uint8)
    return out


@pytest.mark.parametrize("cols", [1, 2, 7, 16, 33])
def test_pack_unpack_round_trip_even_and_odd_widths(cols):
    rng = np.random.default_rng(cols)
    codes = rng.integers(0, 16, (5, cols), dtype=np.uint8)
    packed = fp4.pack_nibbles(torch.from_numpy(codes))
    assert packed.dtype == torch.uint8 and packed.is_contiguous()
    assert np.array_equal(packed.numpy(), _np_pack(codes))
    if cols % 2:   # the padding nibble is zero
        assert not (packed.numpy()[:, -1] & 0xF0).any()
    back = fp4.unpack_nibbles(packed, cols)
    assert back.is_contiguous() and np.array_equal(back.numpy(), codes)


def test_pack_rejects_bad_codes():
    with pytest.raises(ValueError, match="Codes must be uint8 matrix"):
        fp4.pack_nibbles(torch.zeros(4, dtype=torch.uint8))
    with pytest.raises(ValueError, match="Code outside nibble range"):
        fp4.pack_nibbles(torch.tensor([[1, 16]], dtype=torch.uint8))


def test_unpack_rejects_bad_width_and_padding():
    packed = torch.tensor([[0x21, 0x03]], dtype=torch.uint8)
    assert fp4.unpack_nibbles(packed, 3).tolist() == [[1, 2, 3]]
    assert fp4.unpack_nibbles(packed, 4).tolist() == [[1, 2, 3, 0]]
    with pytest.raises(ValueError, match="Nonzero high-nibble padding"):
        fp4.unpack_nibbles(torch.tensor([[0x21, 0x43]], dtype=torch.uint8), 3)
    with pytest.raises(ValueError, match="Packed width differs"):
        fp4.unpack_nibbles(packed, 5)
    with pytest.raises(ValueError, match="Packed width differs"):
        fp4.unpack_nibbles(packed, 3.0)
    with pytest.raises(ValueError, match="Packed values must be uint8 matrix"):
        fp4.unpack_nibbles(packed.view(-1), 4)
