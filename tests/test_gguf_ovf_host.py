"""CPU tests of the GGUF lossless side table (bf16x_gguf_block.py:96-185):
the oracle pinned (brute force, hand-built blocks, lossless round trip and
minimality on the reference's self-test weights), then the C++ packer and
the Python API against it byte for byte, and the host validator."""
import ctypes

import numpy as np
import pytest

from oracle import gguf_codec as go

from bfloat16x_amd import _lib, gguf


def selftest_weights(shape, seed=0):
    """The reference self-test distribution (bf16x_gguf_block.py:203-207)."""
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal(shape) * 0.13).astype(np.float32)
    idx = rng.choice(w.size, w.size // 200, replace=False)
    w.reshape(-1)[idx] *= rng.standard_normal(len(idx)) * 8
    return w


def bf(sign, expo, mant):
    return np.uint16((sign << 15) | (expo << 7) | mant)


def test_mask_known_answers():
    row = np.zeros(64, dtype=np.uint16)
    # half 0: max exponent 130
    row[0] = bf(0, 130, 5)      # the max                       -> exact
    row[1] = bf(1, 124, 9)      # delta 6                        -> exact
    row[2] = bf(0, 123, 1)      # delta 7: clamped              -> entry
    row[3] = bf(1, 0, 0)        # -0.0                           -> no entry
    row[4] = bf(0, 0, 0)        # +0.0                           -> no entry
    row[5] = bf(0, 0, 3)        # denormal, delta 130            -> entry
    row[6] = bf(1, 1, 0)        # delta 129                      -> entry
    # half 1: max exponent 3 < 7: emax floored at 7
    row[16] = bf(0, 3, 2)       # delta 4                        -> exact
    row[17] = bf(0, 1, 0)       # delta 6                        -> exact
    row[18] = bf(1, 0, 1)       # denormal, delta 7              -> entry
    row[19] = bf(1, 0, 0)       # -0.0                           -> no entry
    bits = np.stack([row, np.roll(row, 32)])
    m = go.ovf_mask_bits(bits)
    want = np.zeros(64, dtype=bool)
    want[[2, 5, 6, 18]] = True
    assert np.array_equal(m[0], want) and np.array_equal(m[1], np.roll(want, 32))
    assert np.array_equal(go.ovf_mask_bruteforce(bits), m)


@pytest.mark.parametrize("seed", range(4))
def test_mask_matches_bruteforce(seed):
    rng = np.random.default_rng(seed)
    e = rng.integers(0, 256, size=(3, 64))
    e[:, ::5] = rng.integers(100, 140, size=e[:, ::5].shape)
    bits = ((rng.integers(0, 2, size=e.shape) << 15) | (e << 7) | rng.integers(0, 128, size=e.shape)).astype(np.uint16)
    bits[0, :7] = 0
    bits[1, 3] = 0x8000
    assert np.array_equal(go.ovf_mask_bits(bits), go.ovf_mask_bruteforce(bits))


@pytest.mark.parametrize("shape", [(256, 512), (300, 576), (1024, 2048)])
def test_oracle_table_is_lossless_and_minimal(shape):
    bits = go.fp32_to_bf16_bits(selftest_weights(shape))
    packed = go.quantize_blocks_bits(bits)
    blob = go.pack_ovf_bits(bits)
    rows, row_off, cols, ebits = go.unpack_ovf(blob)
    assert rows == shape[0] and row_off[0] == 0 and row_off[-1] == cols.size
    assert len(blob) == 8 + 4 * (rows + 1) + 4 * cols.size
    assert np.array_equal(go.dequantize_lossless_bits(packed, blob), bits)      # lossless
    plain = go.dequantize_blocks_bits(packed).reshape(shape)
    r = np.repeat(np.arange(rows), np.diff(row_off).astype(np.int64))
    assert not np.any(plain[r, cols.astype(np.int64)] == ebits)                   # minimal
    assert np.array_equal(plain != bits, go.ovf_mask_bits(bits))
    assert 0.001 < cols.size / bits.size < 0.05


@pytest.mark.parametrize("shape", [(256, 512), (300, 576), (1024, 2048), (7, 65536)])
def test_pack_ovf_byte_identical(shape):
    w = selftest_weights(shape, seed=1)
    bits = go.fp32_to_bf16_bits(w)
    assert gguf.pack_ovf(w) == go.pack_ovf_bits(bits)
    assert np.array_equal(gguf.ovf_overflow_mask(w), go.ovf_mask_bits(bits))
    assert gguf.ovf_stats(w) == (int(go.ovf_mask_bits(bits).sum()), w.size)
    # bf16_exact: truncation, the same table for values already bf16
    wb = go.bf16_bits_to_fp32(bits).reshape(shape)
    assert gguf.pack_ovf(wb, bf16_exact=True) == go.pack_ovf_bits(bits)
    rows, ro, cols, eb = gguf.unpack_ovf(gguf.pack_ovf(w))
    r2, ro2, c2, eb2 = go.unpack_ovf(go.pack_ovf_bits(bits))
    assert rows == r2 and np.array_equal(ro, ro2) and np.array_equal(cols, c2) and np.array_equal(eb, eb2)


def test_apply_ovf_matches_oracle():
    w = selftest_weights((64, 256), seed=2)
    bits = go.fp32_to_bf16_bits(w)
    blob = gguf.pack_ovf(w)
    dec = go.dequantize_blocks(go.quantize_blocks_bits(bits)).reshape(64, 256)
    got = gguf.apply_ovf(dec, blob)
    assert np.array_equal(go.fp32_to_bf16_bits(got), go.apply_ovf_bits(go.fp32_to_bf16_bits(dec), blob))
    assert np.array_equal(go.fp32_to_bf16_bits(got), bits)


def test_empty_and_zero_tables():
    z = np.zeros((4, 64), dtype=np.float32)
    blob = gguf.pack_ovf(z)
    assert blob == go.pack_ovf_bits(np.zeros((4, 64), np.uint16)) and len(blob) == 8 + 4 * 5
    assert gguf.ovf_stats(z) == (0, 256)


def _check(packed, blob, **tamper):
    rows, ro, cols, eb = go.unpack_ovf(blob)
    ro = np.array(ro, dtype=np.uint32)
    ent = (cols.astype(np.uint32) | (eb.astype(np.uint32) << 16))
    for k, f in tamper.items():
        ro, ent = f(ro, ent)
    p = np.ascontiguousarray(packed).reshape(-1)
    ent1 = ent if ent.size else np.zeros(1, np.uint32)
    cols_total = (p.size // 46 // rows) * 32
    return _lib.lib().bf16x_gguf_ovf_check_host(p.ctypes.data, p.size, rows, cols_total, ro.ctypes.data,
                                                ent1.ctypes.data, ent.size)


def test_host_check_accepts_good_and_rejects_tampered():
    w = selftest_weights((16, 256), seed=3)
    bits = go.fp32_to_bf16_bits(w)
    packed = go.quantize_blocks_bits(bits)
    blob = go.pack_ovf_bits(bits)
    assert _check(packed, blob) == _lib.OK

    def swap(ro, ent):
        e = ent.copy(); e[[0, 1]] = e[[1, 0]]; return ro, e

    def offcol(ro, ent):                     # move an entry to an element the plain decode gets right
        e = ent.copy()
        plain_ok = np.nonzero(~go.ovf_mask_bits(bits)[0])[0]
        e[0] = (e[0] & 0xFFFF0000) | int(plain_ok[0]); return ro, e

    def flip_sign(ro, ent):
        e = ent.copy(); e[0] ^= 0x80000000; return ro, e

    def bad_off(ro, ent):
        r = ro.copy(); r[-1] += 1; return r, ent

    def col_range(ro, ent):
        e = ent.copy(); e[-1] = (e[-1] & 0xFFFF0000) | 256; return ro, e

    for f in (swap, offcol, flip_sign, bad_off, col_range):
        assert _check(packed, blob, t=f) == _lib.ETABLE, f.__name__


@pytest.mark.parametrize("case,exact", [("selftest", False), ("dense", True), ("empty", False)])
def test_pack_ovf_bytes_match_reference(golden, case, exact):
    """The serialized side table, byte for byte, against blobs the reference's
    pack_ovf wrote (tests/golden/make_golden.py): header, row offsets and the
    {u16 col, u16 bits} entries in row-then-column order, from the oracle and
    from the C++ packer behind gguf.pack_ovf."""
    x = golden[f"gguf_ovf_{case}_x"]
    want = golden[f"gguf_ovf_{case}_blob"].tobytes()
    bits = go.fp32_to_bf16_bits(x) if not exact else (x.view(np.uint32) >> 16).astype(np.uint16)
    assert go.pack_ovf_bits(bits) == want
    assert gguf.pack_ovf(x, bf16_exact=exact) == want
    if case == "dense":
        assert int(np.frombuffer(want[4:8], dtype=np.uint32)[0]) > x.shape[0] * 8   # many entries per row
