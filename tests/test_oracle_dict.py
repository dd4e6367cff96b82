"""Pins the packed-dict oracle (oracle/dict_codec.py) against independent checks:
a bit-at-a-time packer, hand-made known answers, the reference's own golden
vectors (tests/golden/golden_ref.npz), round trips to the original bits, and
invariants between the exact and saturated decodes."""
import numpy as np
import pytest

from oracle import dict_codec as dc
from tests.conftest import golden_dict_cases

FIELDS = ("emax", "sign_packed", "mant_packed", "delta_packed", "delta_ovf_idx", "delta_ovf_val")


@pytest.mark.parametrize("b", [1, 3, 7])
@pytest.mark.parametrize("n", [1, 2, 5, 13, 31, 32, 33, 64, 95, 160])
def test_pack_matches_bruteforce(b, n):
    rng = np.random.default_rng(n * 10 + b)
    v = rng.integers(0, 1 << b, size=n)
    got = dc.pack_bits_stream(v, b)
    assert got.dtype == np.int32
    assert got.tolist() == dc.pack_bits_bruteforce(v, b)
    assert got.size == dc.stream_words(n, b)


def test_pack_known_answers():
    # b=1: element i -> bit i of word 0 (LSB first)
    assert dc.pack_bits_stream(np.array([1, 0, 1] + [0] * 29), 1).tolist() == [0b101]
    # b=7: two fields fill the low 14 bits; N=2 pads 18 elements -> 140 bits -> 5 words
    assert dc.pack_bits_stream(np.array([0x7F, 0x01]), 7).tolist() == [0xFF, 0, 0, 0, 0]
    # b=7: element 4 occupies bits 28..34, straddling words 0 and 1
    v = np.zeros(32, np.int64)
    v[4] = 0x7F
    w = dc.pack_bits_stream(v, 7).view(np.uint32)
    assert w[0] == 0xF0000000 and w[1] == 0x7 and w.size == 7
    # b=3: element 10 occupies bits 30..32
    v = np.zeros(32, np.int64)
    v[10] = 0b101
    w = dc.pack_bits_stream(v, 3).view(np.uint32)
    assert w[0] == 0x40000000 and w[1] == 0x1 and w.size == 3
    # the top bit of a word is stored as a negative int32 (wrap of the int64 cast)
    v = np.zeros(32, np.int64)
    v[31] = 1
    assert dc.pack_bits_stream(v, 1).tolist() == [-(1 << 31)]


def test_stream_length_formula_vs_reference(golden):
    for key, bits, sub in golden_dict_cases(golden):
        n = bits.size
        assert golden[key + "_sign_packed"].size == dc.stream_words(n, 1), key
        assert golden[key + "_mant_packed"].size == dc.stream_words(n, 7), key
        assert golden[key + "_delta_packed"].size == dc.stream_words(n, 3), key


def test_quantize_matches_reference_golden(golden):
    for key, bits, sub in golden_dict_cases(golden):
        d = dc.quantize(bits, sub=sub)
        for f in FIELDS:
            ref = golden[key + "_" + f]
            assert d[f].dtype == ref.dtype, (key, f, d[f].dtype, ref.dtype)
            assert np.array_equal(d[f], ref), (key, f)


def test_decode_exact_matches_reference_golden(golden):
    for key, bits, sub in golden_dict_cases(golden):
        d = {f: golden[key + "_" + f] for f in FIELDS}
        d.update(out_f=bits.shape[0], in_f=bits.shape[1], sub=sub)
        dec = dc.decode_exact(d)
        assert np.array_equal(dec, golden[key + "_decoded"]), key
        assert np.array_equal(dec, bits), key          # the format is lossless


@pytest.mark.parametrize("shape", [(64, 128), (33, 96), (8, 2048)])
def test_roundtrip_bench_weights(shape):
    bits = dc.bench_weight_bits(*shape, seed=3)
    d = dc.quantize(bits)
    assert np.array_equal(dc.decode_exact(d), bits)
    assert np.array_equal(dc.decode_two_segment(d), bits)
    # structural invariants of the table
    idx = d["delta_ovf_idx"]
    assert np.all(np.diff(idx.astype(np.int64)) > 0)
    assert np.all(d["delta_ovf_val"] >= 7)


def test_saturated_decode_closed_form():
    # one 16-element run: emax 127 (1.0), one element 9 exponents below,
    # one exactly 7 below, one zero
    bits = np.full((1, 32), 0x3F80, np.uint16)
    bits[0, 3] = 0x3B00 | 0x15          # e = 118 -> delta 9, mant 0x15
    bits[0, 5] = 0xBC00                 # e = 120 -> delta 7 exactly, negative
    bits[0, 7] = 0x0000                 # zero -> delta 127
    d = dc.quantize(bits)
    assert d["delta_ovf_idx"].tolist() == [3, 5, 7]
    assert d["delta_ovf_val"].tolist() == [9, 7, 127]
    sat = dc.decode_saturated(d)[0]
    assert sat[3] == (0 << 15) | (120 << 7) | 0x15     # exponent emax - 7
    assert sat[5] == 0xBC00                            # delta 7 decodes exactly
    assert sat[7] == (120 << 7)                        # zero becomes 2^-7
    ex = dc.decode_exact(d)[0]
    assert np.array_equal(ex, bits[0])
    assert dc.fix_table(d)[0].tolist() == [3, 7]


def test_saturated_vs_exact_invariant():
    bits = dc.bench_weight_bits(16, 512, seed=5)
    d = dc.quantize(bits)
    sat = dc.decode_saturated(d).reshape(-1)
    ex = dc.decode_exact(d).reshape(-1)
    pos, val = dc.fix_table(d)
    diff = np.nonzero(sat != ex)[0]
    assert np.array_equal(diff, pos)
    em = d["emax"].astype(np.int64)[pos // 16]
    assert np.all((sat[pos] >> 7 & 0xFF) == em - 7)
    assert np.all((sat[pos] & 0x807F) == (ex[pos] & 0x807F))


def test_gemv_gemm_refs_use_decoded_weight():
    bits = dc.bench_weight_bits(8, 64, seed=7)
    d = dc.quantize(bits)
    x = np.random.default_rng(0).standard_normal(64)
    w = dc.bits_to_f32(bits).astype(np.float64)
    assert np.allclose(dc.gemv_ref(d, x), w @ x, rtol=0, atol=0)
    xm = np.random.default_rng(1).standard_normal((3, 64))
    assert np.allclose(dc.gemm_ref(d, xm, saturated=False), xm @ w.T, rtol=0, atol=0)
    ws = dc.bits_to_f32(dc.decode_saturated(d)).astype(np.float64)
    assert np.allclose(dc.gemm_ref(d, xm, saturated=True), xm @ ws.T, rtol=0, atol=0)


def test_rne_matches_torch():
    import torch
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(4096) * 3).astype(np.float32)
    u = x.view(np.uint32)
    u[:64] = (u[:64] & 0xFFFF0000) | 0x8000        # exact ties
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(dc.f32_to_bf16_rne(x), ref)


def test_cpu_path_restatement():
    import torch
    from oracle.cpu_path import CpuBf16xLinear
    bits = dc.bench_weight_bits(40, 96, seed=2)
    d = dc.quantize(bits)
    lin = CpuBf16xLinear(d, tile=16)
    dec = lin.decode_to_bf16().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(dec, bits)
    x = torch.randn(3, 96, dtype=torch.float32).to(torch.bfloat16)
    w = torch.from_numpy(dc.bits_to_f32(bits))
    y = lin.forward(x)                       # bf16 matmul, as the reference
    assert y.dtype == torch.bfloat16
    assert torch.allclose(y.float(), x.float() @ w.t(), rtol=2e-2, atol=2e-2)
