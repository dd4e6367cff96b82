"""GGUF half-block (46-byte) BF16X codec oracle (numpy) -- test infrastructure only.

Restates bf16x_gguf_block.py:29-93:

* block = 32 consecutive row-major weights, 46 bytes:
  [0:2] emax per 16-weight half, floored at 7 (:64); [2:6] sign bits;
  [6:34] 7-bit mantissas; [34:46] 3-bit codes min(emax - e, 7) (:65);
  every field LSB-first (np.packbits bitorder='little', :33);
* decode: exponent = 0 if code == 7 else emax - code (:84), a zero marker.
* fp32 -> bf16 rounding: round to nearest even with NaN quieting (:44-49).

Pinning (tests/test_oracle_gguf.py): ``fp32_to_bf16_bits`` against torch's
bf16 conversion for finite inputs and against golden vectors written by the
reference for NaN/inf inputs; the block layout against hand-built
known-answer blocks; the decode against the reference self-test invariants
(bf16x_gguf_block.py:219-228) and golden vectors from the reference.

Lossless side table (bf16x_gguf_block.py:96-185): ``ovf_mask_bits``,
``pack_ovf_bits``, ``unpack_ovf``, ``apply_ovf_bits``,
``dequantize_lossless_bits``.  Pinning (tests/test_gguf_ovf_host.py): the mask
against an element-by-element brute force and hand-built blocks (delta 6 / 7,
+-0, denormals, the emax floor at 7); the blob against its header and offset
invariants; the whole table by the lossless round trip (every element of
the reference's self-test weights, :203-207, decodes to its original bits)
together with minimality (no entry on an element the plain decode already
returns exactly).
"""
from __future__ import annotations

import numpy as np

QK = 32
BLOCK_BYTES = 46


def fp32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits; NaNs get the quiet bit (bit 22) set before the
    round-to-nearest-even add (bf16x_gguf_block.py:44-49)."""
    n = np.asarray(x, dtype=np.float32).view(np.uint32)
    isnan = (n & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    n = np.where(isnan, (n & np.uint32(0xFFFF0000)) | np.uint32(0x00400000), n)
    n64 = n.astype(np.uint64)
    return ((n64 + np.uint64(0x7FFF) + ((n64 >> np.uint64(16)) & np.uint64(1)))
            >> np.uint64(16)).astype(np.uint16)


def bf16_bits_to_fp32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def _pack_lsb(vals: np.ndarray, nbits: int) -> np.ndarray:
    """(nb, 32) small ints -> (nb, 32*nbits/8) bytes, LSB-first bit order."""
    nb = vals.shape[0]
    bits = ((vals.astype(np.uint32)[:, :, None] >> np.arange(nbits, dtype=np.uint32)) & 1)
    return np.packbits(bits.astype(np.uint8).reshape(nb, 32 * nbits), axis=1, bitorder="little")


def _unpack_lsb(data: np.ndarray, nbits: int) -> np.ndarray:
    nb = data.shape[0]
    bits = np.unpackbits(data, axis=1, bitorder="little")[:, :32 * nbits]
    bits = bits.reshape(nb, 32, nbits).astype(np.uint32)
    return (bits << np.arange(nbits, dtype=np.uint32)).sum(axis=-1)


def quantize_blocks_bits(bits: np.ndarray) -> np.ndarray:
    """bf16 bit patterns (..., 32k) -> uint8 blocks (..., k, 46)."""
    b = np.asarray(bits, dtype=np.uint16)
    n = b.reshape(-1, QK).astype(np.int32)
    nb = n.shape[0]
    sign = (n >> 15) & 1
    expo = (n >> 7) & 0xFF
    mant = n & 0x7F
    emax = np.maximum(expo.reshape(nb, 2, 16).max(axis=-1), 7)
    code = np.minimum(np.repeat(emax, 16, axis=1) - expo, 7)
    out = np.concatenate([emax.astype(np.uint8), _pack_lsb(sign, 1), _pack_lsb(mant, 7),
                          _pack_lsb(code, 3)], axis=1)
    assert out.shape[1] == BLOCK_BYTES
    return out.reshape(*b.shape[:-1], b.shape[-1] // QK, BLOCK_BYTES)


def quantize_blocks(x: np.ndarray) -> np.ndarray:
    """float32 (..., 32k) -> uint8 (..., k, 46) (bf16x_gguf_block.py:57-73)."""
    return quantize_blocks_bits(fp32_to_bf16_bits(x))


def dequantize_blocks_bits(packed: np.ndarray) -> np.ndarray:
    """uint8 blocks (..., k, 46) -> bf16 bits (..., 32k) (bf16x_gguf_block.py:76-87).

    The reference forms (sign<<15)|(expo<<7)|mant in wide unsigned integers
    and keeps the low 16 bits when it converts to float32; for well-formed
    blocks (emax >= 7) no wrap occurs.  Here expo = emax - code is taken mod
    2**16 the same way, so malformed blocks give the same low 16 bits."""
    p = np.asarray(packed, dtype=np.uint8).reshape(-1, BLOCK_BYTES)
    nb = p.shape[0]
    emax = np.repeat(p[:, 0:2].astype(np.int64), 16, axis=1)
    sign = _unpack_lsb(p[:, 2:6], 1).astype(np.int64)
    mant = _unpack_lsb(p[:, 6:34], 7).astype(np.int64)
    code = _unpack_lsb(p[:, 34:46], 3).astype(np.int64)
    expo = np.where(code == 7, 0, emax - code)
    out = ((sign << 15) | ((expo << 7) & 0xFFFF) | mant) & 0xFFFF
    shp = packed.shape
    return out.astype(np.uint16).reshape(*shp[:-2], shp[-2] * QK)


def dequantize_blocks(packed: np.ndarray) -> np.ndarray:
    return bf16_bits_to_fp32(dequantize_blocks_bits(packed))


def student_t_weights(rows: int, cols: int, seed: int = 0) -> np.ndarray:
    """Configuration weights: Student-t(df=3) x 0.015, float32."""
    rng = np.random.default_rng(seed)
    return (rng.standard_t(3, size=(rows, cols)) * 0.015).astype(np.float32)


# --------------------------------------------------------------------------
# lossless side table (bf16x_gguf_block.py:96-185)
# --------------------------------------------------------------------------
OVF_HDR_BYTES = 8


def ovf_mask_bits(bits: np.ndarray) -> np.ndarray:
    """bf16 bits [rows, cols] -> bool mask of the elements the quantizer
    clamps to the zero marker although they are not +-0: exponent delta >= 7
    below the half-block max floored at 7 (bf16x_gguf_block.py:121-128)."""
    b = np.asarray(bits, dtype=np.uint16)
    rows, cols = b.shape
    expo = ((b >> 7) & 0xFF).astype(np.int32).reshape(rows, cols // QK, 2, 16)
    emax = np.maximum(expo.max(axis=-1, keepdims=True), 7)
    delta = (emax - expo).reshape(rows, cols)
    return (delta >= 7) & ((b & 0x7FFF) != 0)


def ovf_mask_bruteforce(bits: np.ndarray) -> np.ndarray:
    """The same mask element by element with Python loops (tiny inputs)."""
    b = np.asarray(bits, dtype=np.uint16)
    rows, cols = b.shape
    out = np.zeros((rows, cols), dtype=bool)
    for r in range(rows):
        for c in range(cols):
            h0 = (c // 16) * 16
            emax = max(7, max(int((int(b[r, k]) >> 7) & 0xFF) for k in range(h0, h0 + 16)))
            e = (int(b[r, c]) >> 7) & 0xFF
            out[r, c] = (emax - e >= 7) and (int(b[r, c]) & 0x7FFF) != 0
    return out


def pack_ovf_bits(bits: np.ndarray) -> bytes:
    """bf16 bits [rows, cols] -> the serialized table: u32 n_rows, u32
    n_entries, u32 row_off[n_rows + 1], {u16 col, u16 bits}[n] in row-major
    order of the mask (bf16x_gguf_block.py:131-148)."""
    b = np.asarray(bits, dtype=np.uint16)
    rows = b.shape[0]
    r, c = np.nonzero(ovf_mask_bits(b))
    row_off = np.zeros(rows + 1, dtype=np.uint32)
    np.cumsum(np.bincount(r, minlength=rows), out=row_off[1:])
    ent = np.empty((r.size, 2), dtype=np.uint16)
    ent[:, 0] = c.astype(np.uint16)
    ent[:, 1] = b[r, c]
    return np.array([rows, r.size], dtype=np.uint32).tobytes() + row_off.tobytes() + ent.tobytes()


def unpack_ovf(blob: bytes):
    """-> (n_rows, row_off, cols, bits) (bf16x_gguf_block.py:151-160)."""
    rows, n = (int(v) for v in np.frombuffer(blob[:OVF_HDR_BYTES], dtype=np.uint32))
    off = OVF_HDR_BYTES
    row_off = np.frombuffer(blob[off:off + 4 * (rows + 1)], dtype=np.uint32)
    off += 4 * (rows + 1)
    ent = np.frombuffer(blob[off:off + 4 * n], dtype=np.uint16).reshape(-1, 2)
    return rows, row_off, ent[:, 0], ent[:, 1]


def apply_ovf_bits(decoded_bits: np.ndarray, blob: bytes) -> np.ndarray:
    """Overwrite the table's elements of decoded bits [rows, cols]
    (bf16x_gguf_block.py:163-171)."""
    rows, row_off, cols, bits = unpack_ovf(blob)
    out = np.array(decoded_bits, dtype=np.uint16, copy=True)
    r = np.repeat(np.arange(rows, dtype=np.int64), np.diff(row_off).astype(np.int64))
    out[r, cols.astype(np.int64)] = bits
    return out


def dequantize_lossless_bits(packed: np.ndarray, blob: bytes) -> np.ndarray:
    """blocks + table -> bf16 bits [rows, cols] (bf16x_gguf_block.py:174-178)."""
    rows = unpack_ovf(blob)[0]
    dec = dequantize_blocks_bits(packed).reshape(rows, -1)
    return apply_ovf_bits(dec, blob)
