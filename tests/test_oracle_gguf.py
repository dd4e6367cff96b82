"""Pins the GGUF half-block oracle (oracle/gguf_codec.py): torch's bf16
rounding for finite values, golden vectors written by the reference for the
NaN path, blocks and decodes, hand-built known-answer blocks, and the
reference self-test invariants (bf16x_gguf_block.py:219-228)."""
import numpy as np
import torch

from oracle import gguf_codec as gc


def test_rounding_matches_torch_finite():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(8192) * 10).astype(np.float32)
    u = x.view(np.uint32)
    u[:100] = (u[:100] & 0xFFFF0000) | 0x8000        # ties to even
    u[100:120] = 0x7F7FFFFF                           # rounds up to inf
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(gc.fp32_to_bf16_bits(x), ref)


def test_rounding_matches_reference_golden(golden):
    assert np.array_equal(gc.fp32_to_bf16_bits(golden["gguf_x"]), golden["gguf_bf16_bits"])
    b = golden["gguf_bf16_bits"].reshape(-1)
    # NaN inputs stay NaN with the quiet bit and their sign
    assert np.all((b[:4] & 0x7F80) == 0x7F80) and np.all(b[:4] & 0x0040)
    assert (b[2] >> 15) == 1


def test_blocks_match_reference_golden(golden):
    blocks = gc.quantize_blocks(golden["gguf_x"])
    assert blocks.shape == golden["gguf_blocks"].shape
    assert np.array_equal(blocks, golden["gguf_blocks"])
    deq = gc.dequantize_blocks(blocks)
    assert np.array_equal(deq.view(np.uint32), golden["gguf_dequant"].view(np.uint32))
    junk = gc.dequantize_blocks(golden["gguf_junk_blocks"][None])
    assert np.array_equal(junk.reshape(-1).view(np.uint32),
                          golden["gguf_junk_dequant"].reshape(-1).view(np.uint32))


def test_selftest_recipe_matches_reference_golden(golden):
    rng0 = np.random.default_rng(0)
    w = (rng0.standard_normal((256, 512)) * 0.13).astype(np.float32)
    idx = rng0.choice(w.size, w.size // 200, replace=False)
    w.reshape(-1)[idx] *= rng0.standard_normal(len(idx)) * 8
    blocks = gc.quantize_blocks(w)
    assert np.array_equal(blocks[:32], golden["gguf_selftest_blocks"])
    back = gc.dequantize_blocks(blocks)
    assert np.array_equal(back[:32].view(np.uint32), golden["gguf_selftest_dequant"].view(np.uint32))
    # reference self-test invariants (bf16x_gguf_block.py:219-228)
    orig = gc.fp32_to_bf16_bits(w).reshape(-1)
    got = gc.fp32_to_bf16_bits(back).reshape(-1)
    mism = orig != got
    assert mism.mean() < 0.05
    emax = blocks.reshape(-1, 46)[:, 0:2].astype(int).repeat(16, axis=1).reshape(-1)[mism]
    ge = (got[mism] >> 7) & 0xFF
    assert np.all((orig[mism] & 0x807F) == (got[mism] & 0x807F))
    assert np.all((ge == np.maximum(emax - 7, 0)) | (ge == 0))


def test_known_answer_block():
    bits = np.full(32, 0x3F80, np.uint16)            # 1.0 everywhere
    bits[0] = 0xBF80 | 0x55                          # -1.664..., sign + mant
    bits[17] = 0x3C00                                # e = 120: code 7 -> zero marker
    bits[18] = 0x3C80                                # e = 121: code 6 -> exact
    blk = gc.quantize_blocks_bits(bits)[0]
    assert blk[0] == 127 and blk[1] == 127
    assert blk[2] == 0x01 and blk[3:6].tolist() == [0, 0, 0]    # sign bit 0
    assert blk[6] == 0x55                                       # mant of element 0
    # element 17's code 7 occupies code-stream bits 51..53 -> byte 34+6, bits 3..5
    assert (int(blk[34 + 6]) >> 3) & 7 == 7
    # element 18's code 6 occupies bits 54..56 -> byte 40 bits 6,7 and byte 41 bit 0
    assert ((int(blk[40]) >> 6) | ((int(blk[41]) & 1) << 2)) == 6
    dec = gc.dequantize_blocks_bits(blk[None])
    assert dec[17] == 0x0000 and dec[18] == 0x3C80 and dec[0] == bits[0]
    # emax is floored at 7 for tiny halves
    small = np.zeros(32, np.uint16)
    small[3] = 0x0001
    b2 = gc.quantize_blocks_bits(small)[0]
    assert b2[0] == 7 and b2[1] == 7
    assert np.array_equal(gc.dequantize_blocks_bits(b2[None]), small)
