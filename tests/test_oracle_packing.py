"""Pin the packed-format definition (oracle/packing.py) on the CPU."""
import numpy as np
import pytest

from oracle.packing import dequantize, pack_rows, unpack_rows, words_per_row
from tests._util import rng


def _pack_loop(codes, nbits):
    """Bit-by-bit statement of the format, for small inputs."""
    R, C = codes.shape
    W = words_per_row(C, nbits)
    out = np.zeros((R, W), dtype=np.uint64)
    for r in range(R):
        for c in range(C):
            f = int(codes[r, c]) + (1 << (nbits - 1))
            for b in range(nbits):
                pos = c * nbits + b
                out[r, pos >> 5] |= ((f >> b) & 1) << (pos & 31)
    return out.astype(np.uint32)


@pytest.mark.parametrize("nbits", [2, 3, 4, 5, 6, 7, 8])
@pytest.mark.parametrize("C", [1, 7, 32, 33, 100])
def test_pack_matches_bit_loop_and_round_trips(nbits, C):
    r = rng(nbits * 100 + C)
    half = 1 << (nbits - 1)
    codes = r.integers(-half, half, size=(3, C))
    codes[0, 0] = -half
    codes[-1, -1] = half - 1
    p = pack_rows(codes, nbits)
    assert p.shape == (3, words_per_row(C, nbits))
    assert np.array_equal(p, _pack_loop(codes, nbits))
    assert np.array_equal(unpack_rows(p, C, nbits), codes)


def test_known_words():
    codes = np.arange(-8, 8).reshape(1, 16)               # fields 0..15 at 4 bits
    assert pack_rows(codes, 4).tolist() == [[0x76543210, 0xFEDCBA98]]
    # 3-bit fields straddle words: 11 fields of 0b111 = 33 ones
    ones = np.full((1, 11), 3)
    assert pack_rows(ones, 3).tolist() == [[0xFFFFFFFF, 0x1]]


def test_range_and_dequant():
    with pytest.raises(ValueError):
        pack_rows(np.array([[8]]), 4)
    codes = np.array([[-2, 1, 3], [0, -1, 2]])
    scales = np.array([[0.5, 2.0], [0.25, 4.0]], dtype=np.float32)      # [ngroups, R]
    g_idx = np.array([0, 1, 1])
    q = dequantize(codes, scales, g_idx)
    assert q.tolist() == [[-1.0, 0.25, 0.75], [0.0, -4.0, 8.0]]
