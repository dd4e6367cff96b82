// Device-side building blocks of the BF16X engine (gfx950 / CDNA4).
//
// The packed-dict format (opqk_linear.py:291-324) stores, for 32 consecutive
// flat elements starting at element 32*a (an "atom"):
//   sign  word a              (bit j = sign of element j)
//   mant  words 7a .. 7a+6    (element j's 7 bits at stream bits 7j..7j+6)
//   delta words 3a .. 3a+2    (element j's 3-bit code at bits 3j..3j+2)
//   emax  bytes 2a, 2a+1      (shared exponent of elements 0-15 / 16-31)
// because every stream is LSB-first and 32 | (element offset) at atom starts.
// A lane that owns an atom therefore loads 1 + 7 + 3 dwords and one u16 with
// no cross-lane dependence, and consecutive lanes read consecutive bytes of
// every stream (dwordx4 + dwordx3 for the 28-byte mantissa run, dwordx3 for
// the 12-byte code run): the loads coalesce without an LDS round trip.
//
// Decoding works on "pairs" (element j, element j+16) packed as two bf16 in
// one 32-bit register (j in the low half).  The two halves of an atom sit
// 112 bits (mantissa) / 48 bits (codes) / 16 bits (sign) apart, so one
// 16-bit-lane transposition of the mantissa and code words puts both fields
// of a pair at the same offset of the two 16-bit lanes: every field is then
// extracted for two elements with one 32-bit shift, and the sign of both
// with one shift of the sign word.  The consumer (v_dot2_f32_bf16, an MFMA
// operand, or a store) uses the same (j, j+16) pairing on its other operand.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bf16x {

typedef uint32_t u32x4a __attribute__((ext_vector_type(4))) __attribute__((aligned(4)));
typedef uint32_t u32x3a __attribute__((ext_vector_type(3))) __attribute__((aligned(4)));
typedef uint32_t u32x2a __attribute__((ext_vector_type(2))) __attribute__((aligned(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// NOTE: never __builtin_bit_cast an ext-vector *element* (v.y, v[1]) with
// this toolchain: it reads element 0.  Copy the element to a scalar first.

struct Atom {
  uint32_t s;       // sign word
  uint32_t m[7];    // mantissa words
  uint32_t d[3];    // 3-bit code words
  uint16_t e;       // emax byte of half 0 | emax byte of half 1 << 8 (kept 16-bit:
                    // a widened copy would be made where the load lands)
};

__device__ __forceinline__ uint32_t alignbit(uint32_t hi, uint32_t lo, uint32_t sh) {
  return __builtin_amdgcn_alignbit(hi, lo, sh);
}
__device__ __forceinline__ uint32_t perm(uint32_t s0, uint32_t s1, uint32_t sel) {
  return __builtin_amdgcn_perm(s0, s1, sel);
}
// (a & 0xFFFF) | (b & 0xFFFF0000): one v_bfi_b32
__device__ __forceinline__ uint32_t lo_hi(uint32_t a, uint32_t b) {
  return (a & 0xFFFFu) | (b & 0xFFFF0000u);
}
// per-16-bit-lane saturating a - b (v_pk_sub_u16 ... clamp)
__device__ __forceinline__ uint32_t pk_sub_sat(uint32_t a, uint32_t b) {
  u16x2 x, y;
  __builtin_memcpy(&x, &a, 4);
  __builtin_memcpy(&y, &b, 4);
  u16x2 r = __builtin_elementwise_sub_sat(x, y);
  uint32_t o;
  __builtin_memcpy(&o, &r, 4);
  return o;
}

// Load the atom with flat atom index `ga` (all streams dword-aligned).
__device__ __forceinline__ Atom load_atom(const uint32_t* __restrict__ sign,
                                          const uint32_t* __restrict__ mant,
                                          const uint32_t* __restrict__ delta,
                                          const uint16_t* __restrict__ emax2,
                                          uint64_t ga) {
  Atom t;
  const uint32_t* mp = mant + 7 * ga;
  const uint32_t* dp = delta + 3 * ga;
  u32x4a m03 = *(const u32x4a*)mp;
  u32x3a m46 = *(const u32x3a*)(mp + 4);
  u32x3a d02 = *(const u32x3a*)dp;
  t.s = sign[ga];
  t.e = emax2[ga];
  uint32_t a0 = m03.x, a1 = m03.y, a2 = m03.z, a3 = m03.w;
  uint32_t a4 = m46.x, a5 = m46.y, a6 = m46.z;
  t.m[0] = a0; t.m[1] = a1; t.m[2] = a2; t.m[3] = a3;
  t.m[4] = a4; t.m[5] = a5; t.m[6] = a6;
  uint32_t b0 = d02.x, b1 = d02.y, b2 = d02.z;
  t.d[0] = b0; t.d[1] = b1; t.d[2] = b2;
  return t;
}

// per-16-bit-lane a - b modulo 2^16 (v_pk_sub_u16)
__device__ __forceinline__ uint32_t pk_sub_wrap(uint32_t a, uint32_t b) {
  u16x2 x, y;
  __builtin_memcpy(&x, &a, 4);
  __builtin_memcpy(&y, &b, 4);
  u16x2 r = x - y;
  uint32_t o;
  __builtin_memcpy(&o, &r, 4);
  return o;
}
// per-16-bit-lane arithmetic shift right by 15: 0xFFFF where bit 15 is set
__device__ __forceinline__ uint32_t pk_ashr15(uint32_t a) {
  typedef short s16x2 __attribute__((ext_vector_type(2)));
  s16x2 x;
  __builtin_memcpy(&x, &a, 4);
  s16x2 r = x >> (short)15;
  uint32_t o;
  __builtin_memcpy(&o, &r, 4);
  return o;
}
// (m & a) | (~m & b): v_bfi_b32
__device__ __forceinline__ uint32_t bfi(uint32_t m, uint32_t a, uint32_t b) { return (m & a) | (~m & b); }

// An atom's fields after the 16-bit-lane transposition (lane lo = elements
// 0..15, lane hi = 16..31), ready for decode_pair.
struct PairState {
  uint32_t pm[7];   // mantissa words
  uint32_t pd[3];   // code words
  uint32_t E;       // emax of each half at bits 7..14 of its 16-bit lane
  uint32_t s;       // sign word
};

__device__ __forceinline__ PairState prep_pairs(const Atom& t) {
  PairState q;
  q.pm[0] = lo_hi(t.m[0], t.m[3]);
  q.pm[1] = alignbit(t.m[4], t.m[0], 16);
  q.pm[2] = lo_hi(t.m[1], t.m[4]);
  q.pm[3] = alignbit(t.m[5], t.m[1], 16);
  q.pm[4] = lo_hi(t.m[2], t.m[5]);
  q.pm[5] = alignbit(t.m[6], t.m[2], 16);
  q.pm[6] = lo_hi(t.m[3], t.m[6]);
  q.pd[0] = lo_hi(t.d[0], t.d[1]);
  q.pd[1] = alignbit(t.d[2], t.d[0], 16);
  q.pd[2] = lo_hi(t.d[1], t.d[2]);
  const uint32_t e16 = t.e;
  q.E = ((e16 & 0xFFu) << 7) | ((e16 & 0xFF00u) << 15);
  q.s = t.s;
  return q;
}

// Pair j (0..15, a compile-time constant after unrolling): bf16(elem j) |
// bf16(elem j+16) << 16.
template <bool ZERO7 = false>
__device__ __forceinline__ uint32_t decode_pair(const PairState& q, int j) {
  // mantissa field at lane bit 7j
  const int mk = (7 * j) >> 4, mo = (7 * j) & 15;
  uint32_t mraw;
  if (mo <= 9) {
    mraw = q.pm[mk] >> mo;
  } else {
    // field straddles two 16-bit chunks: splice byte 1 of chunk k with
    // byte 0 of chunk k+1 in each lane, then the field sits at mo-8
    mraw = perm(q.pm[mk + 1], q.pm[mk], 0x06030401u) >> (mo - 8);
  }
  // code field at lane bit 3j, moved to bits 7..9 of each lane
  const int dk = (3 * j) >> 4, dof = (3 * j) & 15;
  uint32_t dsh;
  if (dof <= 13) {
    dsh = (dof <= 7) ? (q.pd[dk] << (7 - dof)) : (q.pd[dk] >> (dof - 7));
  } else {
    dsh = perm(q.pd[dk + 1], q.pd[dk], 0x06030401u) << (15 - dof);
  }
  dsh &= 0x03800380u;
  uint32_t ex;
  if constexpr (ZERO7) {
    const uint32_t t15 = (dsh << 5) + 0x10001000u;         // bit 15 of a lane set iff code == 7
    ex = bfi(pk_ashr15(t15), 0u, pk_sub_wrap(q.E, dsh));    // (emax - d) << 7 mod 2^16, 0 for code 7
  } else {
    ex = pk_sub_sat(q.E, dsh);                             // (emax - d) << 7 per lane, clamped at 0
  }
  const uint32_t ssh = (j == 15) ? q.s : (q.s << (15 - j));
  // v_bitop3 0xEA = (S0 & S1) | S2: mantissa bits into the exponent word,
  // then the two sign bits (ex has zeros at both masks' positions)
  uint32_t w = __builtin_amdgcn_bitop3_b32(mraw, 0x007F007Fu, ex, 0xEA);
  return __builtin_amdgcn_bitop3_b32(ssh, 0x80008000u, w, 0xEA);
}

// Decode an atom into 16 packed pairs: out[j] = bf16(elem j) | bf16(elem j+16) << 16.
// ZERO7 = false (packed dict): the 3-bit code is the exponent delta, code 7
// saturating at emax-7; the exponent is clamped at 0 like the reference
// kernels (bf16x_triton_test.py:50).
// ZERO7 = true (GGUF half-block, bf16x_gguf_block.py:76-87): code 7 is a zero
// marker (exponent 0), and emax - code is formed in uint16 as there, so a
// malformed block with emax < code wraps instead of clamping.  Per lane,
// (code << 12) + 0x1000 reaches bit 15 exactly for code 7; an arithmetic
// shift by 15 widens that bit to a lane mask which clears the exponent.
template <bool ZERO7 = false>
__device__ __forceinline__ void decode_pairs(const Atom& t, uint32_t out[16]) {
  const PairState q = prep_pairs(t);
#pragma unroll
  for (int j = 0; j < 16; ++j) out[j] = decode_pair<ZERO7>(q, j);
}

// bf16 bits of a finite-or-not float, round to nearest even, NaN kept NaN.
__device__ __forceinline__ uint32_t f32_to_bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return ((u >> 16) | 0x0040u) & 0xFFFFu;
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// GGUF half-block (bf16x_gguf_block.py:6-17): block b is 46 bytes at 46*b,
// [emax lo, emax hi | sign 4 | mant 28 | delta 12], the dict atom's fields in
// AoS order.  Blocks are 2-byte aligned: the 48 bytes from the dword at or
// below the block are loaded (three 16-byte loads, dword aligned) and
// shifted by 0 or 16 bits.  The shift is done where the block is decoded, not
// where it is loaded (values computed from a load at the load site make the
// compiler wait for it there).  `rs` must cover the buffer rounded up to a
// multiple of 4 bytes.
struct GgufRaw {
  u32x4 q0, q1, q2;
  uint32_t sh;                     // 0 or 16
};

__device__ __forceinline__ void load_gguf_raw(__amdgpu_buffer_rsrc_t rs, uint32_t boff, GgufRaw& r) {
  const uint32_t base = boff & ~3u;
  r.sh = (boff & 2u) * 8u;
  r.q0 = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)base, 0, 0);
  r.q1 = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)(base + 16), 0, 0);
  r.q2 = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)(base + 32), 0, 0);
}

__device__ __forceinline__ Atom gguf_atom(const GgufRaw& r) {
  const uint32_t sh = r.sh;
  const uint32_t w0 = r.q0.x, w1 = r.q0.y, w2 = r.q0.z, w3 = r.q0.w, w4 = r.q1.x, w5 = r.q1.y, w6 = r.q1.z;
  const uint32_t w7 = r.q1.w, w8 = r.q2.x, w9 = r.q2.y, w10 = r.q2.z, w11 = r.q2.w;
  // block word k (bytes 4k..4k+3 of the block) = alignbit(w[k+1], w[k], sh);
  // word 11 only needs its low half (block bytes 44-45)
  const uint32_t b0 = alignbit(w1, w0, sh), b1 = alignbit(w2, w1, sh), b2 = alignbit(w3, w2, sh);
  const uint32_t b3 = alignbit(w4, w3, sh), b4 = alignbit(w5, w4, sh), b5 = alignbit(w6, w5, sh);
  const uint32_t b6 = alignbit(w7, w6, sh), b7 = alignbit(w8, w7, sh), b8 = alignbit(w9, w8, sh);
  const uint32_t b9 = alignbit(w10, w9, sh), b10 = alignbit(w11, w10, sh), b11 = alignbit(w11, w11, sh);
  Atom t;
  t.e = (uint16_t)b0;                                         // bytes 0-1
  t.s = alignbit(b1, b0, 16);                                 // bytes 2-5
  t.m[0] = alignbit(b2, b1, 16); t.m[1] = alignbit(b3, b2, 16); t.m[2] = alignbit(b4, b3, 16);
  t.m[3] = alignbit(b5, b4, 16); t.m[4] = alignbit(b6, b5, 16); t.m[5] = alignbit(b7, b6, 16);
  t.m[6] = alignbit(b8, b7, 16);                              // bytes 6-33
  t.d[0] = alignbit(b9, b8, 16); t.d[1] = alignbit(b10, b9, 16); t.d[2] = alignbit(b11, b10, 16);  // 34-45
  return t;
}

__device__ __forceinline__ float bf16lo_to_f32(uint32_t p) { return __uint_as_float(p << 16); }

// bf16(lo) | bf16(hi) << 16 rounded to nearest even (the default rounding
// mode): one v_cvt_pk_bf16_f32 on gfx950.  Used where the inputs are finite
// products of finite bf16 values, for which it gives f32_to_bf16_rne's bits.
__device__ __forceinline__ uint32_t pk_bf16(float lo, float hi) {
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{lo, hi}), bf16x2_t));
}
__device__ __forceinline__ float bf16hi_to_f32(uint32_t p) { return __uint_as_float(p & 0xFFFF0000u); }

__device__ __forceinline__ float dot2_bf16(uint32_t w, uint32_t x, float acc) {
  bf16x2_t a, b;
  __builtin_memcpy(&a, &w, 4);
  __builtin_memcpy(&b, &x, 4);
  return __builtin_amdgcn_fdot2_f32_bf16(a, b, acc, false);
}

// Sum over the 64 lanes of a wave with DPP: row scans (shr 1, 2, 4, 8) leave
// each 16-lane row's sum in its lane 15, row_bcast 15/31 fold the rows; the
// total ends in lane 63.
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += __builtin_amdgcn_update_dpp(0.f, v, 0x111, 0xF, 0xF, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0.f, v, 0x112, 0xF, 0xF, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0.f, v, 0x114, 0xF, 0xF, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0.f, v, 0x118, 0xF, 0xF, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0.f, v, 0x142, 0xA, 0xF, false);  // row_bcast:15
  v += __builtin_amdgcn_update_dpp(0.f, v, 0x143, 0xC, 0xF, false);  // row_bcast:31
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

}  // namespace bf16x
