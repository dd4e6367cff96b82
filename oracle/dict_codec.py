"""BF16X packed-dict oracle (numpy) -- test infrastructure only.

Restates, on the CPU, the reference's packed-dict format and its consumers:

* ``pack_bits_stream`` / ``unpack_bits_stream``  -> opqk_linear.py:53-77
* ``quantize``                                   -> opqk_linear.py:291-324
* ``decode_exact``  (CPU BF16XLinear tile decode) -> opqk_linear.py:360-377
* ``decode_saturated`` (Triton base decode)       -> bf16x_triton_test.py:11-52
* ``decode_two_segment`` (base decode + fix)      -> bf16x_triton_test.py:55-108
* ``fix_table`` (entries with true delta > 7)     -> bf16x_triton_test.py:96,
                                                     bf16x_fused.py:166-169
* ``gemv_ref`` / ``gemm_ref``                     -> bf16x_fused.py:32-127,
                                                     bf16x_gemm_fused.py:31-114

All bit patterns are handled as numpy ``uint16`` (bf16) and the packed words
as ``int32`` holding the uint32 bit pattern, as the reference stores them.

Pinning (see tests/test_oracle_dict.py):
* the bit packer against a bit-at-a-time brute-force packer and hand-made
  known-answer vectors (LSB-first order, word order);
* the stream length formula against golden vectors written by the reference
  itself for element counts that are not multiples of 32;
* ``quantize`` + ``decode_exact`` by the round trip to the original bf16 bits
  (self-verifying) and by golden vectors from the reference encoder;
* ``decode_saturated`` by its closed form on hand-made cases (exponent
  emax-7 where the 3-bit code saturates) and by the invariant that it agrees
  with the exact decode everywhere except at table entries with delta > 7;
* ``gemv_ref`` / ``gemm_ref`` by float64 matmul of the decoded weight.
"""
from __future__ import annotations

import numpy as np

SUB = 16


# --------------------------------------------------------------------------
# bit streams (opqk_linear.py:53-77)
# --------------------------------------------------------------------------
def stream_words(n: int, b: int) -> int:
    """Length in int32 words of ``pack_bits_stream`` of ``n`` b-bit values.

    The reference pads ``(-n*b) % 32`` *elements* (not bits) before packing
    (opqk_linear.py:55-58) and then rounds the bit count up to whole words
    (:60-62).
    """
    pad = (-n * b) % 32
    nbits = (n + pad) * b
    return (nbits + 31) // 32


def pack_bits_stream(vals: np.ndarray, b: int) -> np.ndarray:
    """b-bit values -> global LSB-first bit stream of int32 words.

    Stream bit k is bit (k mod b) of value k//b and lands in bit (k mod 32)
    of word k//32 (opqk_linear.py:59,63).
    """
    v = np.asarray(vals).astype(np.uint32).reshape(-1)
    n = v.size
    pad = (-n * b) % 32
    if pad:
        v = np.concatenate([v, np.zeros(pad, np.uint32)])
    bits = ((v[:, None] >> np.arange(b, dtype=np.uint32)) & 1).astype(np.uint8).reshape(-1)
    nw = stream_words(n, b)
    if nw * 32 > bits.size:
        bits = np.concatenate([bits, np.zeros(nw * 32 - bits.size, np.uint8)])
    packed = np.packbits(bits, bitorder="little")          # bytes, LSB-first
    return packed.view("<u4").astype(np.uint32).view(np.int32).copy()


def unpack_bits_stream(words: np.ndarray, bit_start: int, nbits: int, b: int) -> np.ndarray:
    """Values of the bit range [bit_start, bit_start+nbits) (opqk_linear.py:67-77)."""
    w = np.asarray(words).view(np.uint32).astype("<u4")
    ws = bit_start // 32
    sk = bit_start % 32
    we = (bit_start + nbits + 31) // 32
    bits = np.unpackbits(w[ws:we].view(np.uint8), bitorder="little")[sk:sk + nbits]
    bits = bits.reshape(-1, b).astype(np.uint32)
    return (bits << np.arange(b, dtype=np.uint32)).sum(axis=1).astype(np.int64)


def pack_bits_bruteforce(vals, b: int) -> list:
    """Bit-at-a-time packer for tiny inputs (an independent statement of the
    stream layout used to pin ``pack_bits_stream``)."""
    vals = [int(v) for v in vals]
    n = len(vals)
    pad = (-n * b) % 32
    vals = vals + [0] * pad
    nw = stream_words(n, b)
    words = [0] * nw
    k = 0
    for v in vals:
        for j in range(b):
            if (v >> j) & 1:
                words[k // 32] |= 1 << (k % 32)
            k += 1
    return [w - (1 << 32) if w >= (1 << 31) else w for w in words]


# --------------------------------------------------------------------------
# encoder (opqk_linear.py:291-324)
# --------------------------------------------------------------------------
def quantize(bits: np.ndarray, sub: int = SUB) -> dict:
    """bf16 bit patterns [out_f, in_f] (uint16) -> packed dict (numpy arrays).

    Fields s=(b>>15)&1, e=(b>>7)&0xFF, m=b&0x7F (:300-303); emax = max of e
    over runs of ``sub`` consecutive flat elements, tail padded with e=0
    (:305-308); delta = emax - e (:309); table = positions with delta >= 7
    in ascending order with their true delta (:311-313); 3-bit code
    min(delta, 7) (:314).
    """
    bits = np.asarray(bits, dtype=np.uint16)
    out_f, in_f = bits.shape
    flat = bits.reshape(-1).astype(np.int32)
    n = flat.size
    sign = (flat >> 15) & 1
    expo = (flat >> 7) & 0xFF
    mant = flat & 0x7F
    pad = (-n) % sub
    e1 = np.concatenate([expo, np.zeros(pad, np.int32)]) if pad else expo
    emax = e1.reshape(-1, sub).max(axis=1)
    delta = (emax[:, None] - e1.reshape(-1, sub)).reshape(-1)[:n]
    ovf = delta >= 7
    return dict(
        emax=emax.astype(np.uint8),
        sign_packed=pack_bits_stream(sign, 1),
        mant_packed=pack_bits_stream(mant, 7),
        delta_packed=pack_bits_stream(np.minimum(delta, 7), 3),
        delta_ovf_idx=np.nonzero(ovf)[0].astype(np.int32),
        delta_ovf_val=delta[ovf].astype(np.uint8),
        out_f=int(out_f), in_f=int(in_f), sub=int(sub),
    )


def fields(d: dict):
    """Unpacked per-element (sign, mant, d3, emax_of_element) as int64 arrays."""
    n = d["out_f"] * d["in_f"]
    sgn = unpack_bits_stream(d["sign_packed"], 0, n, 1)
    mant = unpack_bits_stream(d["mant_packed"], 0, n * 7, 7)
    d3 = unpack_bits_stream(d["delta_packed"], 0, n * 3, 3)
    em = np.asarray(d["emax"]).astype(np.int64)[np.arange(n) // d["sub"]]
    return sgn, mant, d3, em


# --------------------------------------------------------------------------
# decoders
# --------------------------------------------------------------------------
def decode_exact(d: dict) -> np.ndarray:
    """Exact decode as the CPU ``BF16XLinear._decode_tile`` (opqk_linear.py:360-377).

    Where the 3-bit code is 7 the true delta is looked up by ``searchsorted``
    of the flat position in ``delta_ovf_idx`` (clamped to the last entry,
    :368-372); exponent = (emax - delta) & 0xFF (:375).
    Returns uint16 bits [out_f, in_f].
    """
    sgn, mant, dd, em = fields(d)
    n = sgn.size
    idx = np.asarray(d["delta_ovf_idx"]).astype(np.int64)
    val = np.asarray(d["delta_ovf_val"]).astype(np.int64)
    ovf = dd == 7
    if ovf.any() and idx.size > 0:
        loc = np.searchsorted(idx, np.arange(n), side="left")
        loc = np.minimum(loc, idx.size - 1)
        dd = np.where(ovf, val[loc], dd)
    expo = (em - dd) & 0xFF
    out = (sgn << 15) | (expo << 7) | (mant & 0x7F)
    return out.astype(np.uint16).reshape(d["out_f"], d["in_f"])


def decode_saturated(d: dict) -> np.ndarray:
    """Saturated decode as ``_bf16x_decode_kernel`` (bf16x_triton_test.py:11-52):
    the 3-bit code is used as-is, exponent = clamp(emax - d3, 0, 255) (:50).
    Emax is always read at flat index //16 (:46), whatever ``sub`` says."""
    n = d["out_f"] * d["in_f"]
    sgn = unpack_bits_stream(d["sign_packed"], 0, n, 1)
    mant = unpack_bits_stream(d["mant_packed"], 0, n * 7, 7)
    d3 = unpack_bits_stream(d["delta_packed"], 0, n * 3, 3)
    em = np.asarray(d["emax"]).astype(np.int64)[np.arange(n) // 16]
    expo = np.clip(em - d3, 0, 255)
    out = (sgn << 15) | (expo << 7) | mant
    return out.astype(np.uint16).reshape(d["out_f"], d["in_f"])


def fix_table(d: dict):
    """Table entries a GPU consumer must patch: true delta > 7
    (bf16x_triton_test.py:96; bf16x_fused.py:166-169).  Returns (idx, val)."""
    idx = np.asarray(d["delta_ovf_idx"]).astype(np.int64)
    val = np.asarray(d["delta_ovf_val"]).astype(np.int64)
    keep = val > 7
    return idx[keep], val[keep]


def decode_two_segment(d: dict) -> np.ndarray:
    """``bf16x_decode_triton`` (bf16x_triton_test.py:80-108): saturated decode,
    then for entries with val > 7 rewrite the exponent with
    clamp(emax[pos // sub] - val, 0, 255), keeping sign and mantissa (:65-75)."""
    out = decode_saturated(d).reshape(-1).astype(np.int64)
    pos, val = fix_table(d)
    if pos.size:
        em = np.asarray(d["emax"]).astype(np.int64)[pos // d["sub"]]
        cur = out[pos]
        expo = np.clip(em - val, 0, 255)
        out[pos] = (cur & 0x8000) | (expo << 7) | (cur & 0x7F)
    return out.astype(np.uint16).reshape(d["out_f"], d["in_f"])


# --------------------------------------------------------------------------
# reference products
# --------------------------------------------------------------------------
def bits_to_f32(bits: np.ndarray) -> np.ndarray:
    """uint16 bf16 patterns -> exact float32."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_rne(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits, round to nearest even (finite values)."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return r.astype(np.uint16)


def gemv_ref(d: dict, x: np.ndarray) -> np.ndarray:
    """y = W_exact . x (bf16x_fused.py:32-111: the saturated main loop plus the
    correction overlay equals the exact weight).  float64 accumulation;
    returns float64 [out_f] before the bf16 rounding of the kernel's store."""
    w = bits_to_f32(decode_exact(d)).astype(np.float64)
    return w @ np.asarray(x, dtype=np.float64).reshape(-1)


def gemm_ref(d: dict, x: np.ndarray, saturated: bool = True) -> np.ndarray:
    """y[M, out_f] = x[M, in_f] . W^T; ``saturated`` selects the reference
    GEMM's numerics (no overflow correction, bf16x_gemm_fused.py:84-87),
    otherwise the exact weight.  float64 accumulation."""
    wb = decode_saturated(d) if saturated else decode_exact(d)
    w = bits_to_f32(wb).astype(np.float64)
    return np.asarray(x, dtype=np.float64).reshape(-1, d["in_f"]) @ w.T


def rel_err(y: np.ndarray, y_ref: np.ndarray, floor_frac: float = 1e-3):
    """Elementwise |y - y_ref| / max(|y_ref|, floor_frac * rms(y_ref)).
    Returns (max, median)."""
    y = np.asarray(y, dtype=np.float64).reshape(-1)
    r = np.asarray(y_ref, dtype=np.float64).reshape(-1)
    rms = float(np.sqrt(np.mean(r * r))) if r.size else 0.0
    den = np.maximum(np.abs(r), floor_frac * rms + 1e-30)
    e = np.abs(y - r) / den
    return float(e.max()) if e.size else 0.0, float(np.median(e)) if e.size else 0.0


# --------------------------------------------------------------------------
# seeded synthetic weights of the benchmark configurations
# --------------------------------------------------------------------------
def bench_weight_bits(out_f: int, in_f: int, seed: int = 0) -> np.ndarray:
    """N(0, 0.02) with 1 % of entries scaled x30, rounded to bf16 (RNE).

    numpy restatement of the configuration's weight distribution, drawn
    with numpy's default_rng: the same distribution as the benchmark's
    weights (bench.bench_weight, torch's CPU generator) but not the same
    values.  The full-size GPU tests use bench.bench_weight itself."""
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((out_f, in_f), dtype=np.float32) * np.float32(0.02))
    n = w.size
    idx = rng.choice(n, n // 100, replace=False)
    w.reshape(-1)[idx] *= np.float32(30.0)
    return f32_to_bf16_rne(w)
