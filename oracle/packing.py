"""CPU definition of the packed export format (TEST INFRASTRUCTURE ONLY).

Only ``tests/`` may import this module, as the checker of ``rq_pack_codes`` /
``rq_unpack_dequant``.  The reference has no packed format -- its export keeps full fp32
``int_weight`` / ``scale`` tensors (gptq_utils/gptq_plus_utils.py:1866-1871) -- so this file
states the format itself: row r is a little-endian bitstream, code c occupies bits
[c*nbits, (c+1)*nbits) and is stored as code + 2^(nbits-1); bit b of the row is bit (b & 31)
of 32-bit word (b >> 5); trailing bits are zero.  Dequantisation is
fl32(scales[g_idx[c], r] * code) cast to the layer dtype, as in the reference's
``(scale * q).to(x.dtype)`` (quant_utils.py:478).

Pinned in ``tests/test_oracle_packing.py`` by a bit-by-bit loop on small inputs, known words
and the pack -> unpack identity.
"""
from __future__ import annotations

import numpy as np


def words_per_row(C: int, nbits: int) -> int:
    return (C * nbits + 31) // 32


def pack_rows(codes: np.ndarray, nbits: int) -> np.ndarray:
    """int codes [R, C] -> uint32 [R, words_per_row]."""
    codes = np.asarray(codes, dtype=np.int64)
    R, C = codes.shape
    half = 1 << (nbits - 1)
    fields = codes + half
    if fields.min(initial=0) < 0 or fields.max(initial=0) >= (1 << nbits):
        raise ValueError("code out of range for nbits")
    # bit matrix [R, C, nbits], least significant bit first, flattened to the row bitstream
    bits = ((fields[:, :, None] >> np.arange(nbits)) & 1).astype(np.uint8).reshape(R, C * nbits)
    W = words_per_row(C, nbits)
    pad = np.zeros((R, W * 32 - C * nbits), dtype=np.uint8)
    stream = np.concatenate([bits, pad], axis=1)
    packed = np.packbits(stream, axis=1, bitorder="little")          # bytes, little-endian bits
    return packed.view("<u4").reshape(R, W).astype(np.uint32)


def unpack_rows(packed: np.ndarray, C: int, nbits: int) -> np.ndarray:
    """uint32 [R, words] -> int64 codes [R, C]."""
    packed = np.ascontiguousarray(np.asarray(packed).astype(np.uint32))
    R = packed.shape[0]
    stream = np.unpackbits(packed.view(np.uint8).reshape(R, -1), axis=1, bitorder="little")
    bits = stream[:, :C * nbits].reshape(R, C, nbits).astype(np.int64)
    fields = (bits << np.arange(nbits)).sum(axis=2)
    return fields - (1 << (nbits - 1))


def dequantize(codes: np.ndarray, scales: np.ndarray, g_idx: np.ndarray) -> np.ndarray:
    """fp32 Q[r, c] = scales[g_idx[c], r] * code[r, c] (cast to the layer dtype by the caller)."""
    s = np.asarray(scales, dtype=np.float32)[np.asarray(g_idx), :].T      # [R, C]
    return (s * np.asarray(codes, dtype=np.float32)).astype(np.float32)
