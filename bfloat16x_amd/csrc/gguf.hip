// GGUF half-block BF16X (bf16x_gguf_block.py:6-17, 25-93) on gfx950: decode
// and decode+GEMV.
//
// A weight [out_f, in_f] (in_f % 32 == 0) is out_f * in_f / 32 blocks of 46
// bytes in row-major order; block b holds the 32 elements 32b .. 32b+31.
// Decoding follows bf16x_gguf_block.py:76-87: exponent = 0 if code == 7
// (zero marker) else emax - code, sign and mantissa kept.  Each block is the
// packed dict's atom in AoS order, so the atom decoder of bf16x_device.h
// serves both formats (decode_pairs<true>).
#include <hip/hip_runtime.h>

#include <mutex>
#include <stdint.h>
#include <stdlib.h>

#include <algorithm>
#include <type_traits>

#include "../../include/bf16x_hip.h"
#include "bf16x_device.h"
#include "launch_common.h"

namespace bf16x {
namespace gguf {

constexpr int kBlockBytes = 46;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, uint64_t bytes) {
  const uint32_t n = bytes > 0xFFFFFFFFull ? 0xFFFFFFFFu : (uint32_t)bytes;
  return __builtin_amdgcn_make_buffer_rsrc((void*)p, (short)0, (int)n, 0x00020000);
}

// 16-byte chunk q of block a of a pass: slot rotated by a/4 (conflict free for
// per-block writes and contiguous reads)
__device__ __forceinline__ int chunk_slot(int a, int q) { return a * 64 + (((q + (a >> 2)) & 3) << 4); }

// ---------------------------------------------------------------------------
// decode: one wave per row, 64 blocks per pass, staged through LDS so that
// each store instruction writes contiguous bytes (1 KB bf16, 2 KB fp32)
// ---------------------------------------------------------------------------
// With OVF, the lossless side table (bf16x_gguf_block.py:96-113) is applied
// in LDS before each pass is stored: row_off [out_f + 1] and entries
// (column | bf16 bits << 16, sorted by row then column) as in the reference's
// blob.  Entries are taken in column order with a per-row cursor: a pass reads
// the next 64 entries of its row, writes those whose column falls in the
// pass, and advances by their count (ballot).
template <bool F32, bool OVF>
__global__ __launch_bounds__(256) void gguf_decode_kernel(const uint8_t* __restrict__ blocks, int64_t out_f,
                                                          int64_t in_f, const uint32_t* __restrict__ ovf_off,
                                                          const uint32_t* __restrict__ ovf_ent,
                                                          void* __restrict__ out) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[4 * 4096];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t row = (int64_t)blockIdx.x * 4 + wave;
  if (row >= out_f) return;
  uint8_t* buf = lds + wave * 4096;
  const int64_t P = in_f >> 5;
  const int passes = (int)((P + 63) >> 6);
  // descriptor based at the row (offsets < 4 GiB); it covers the rest of the
  // blocks rounded up to 4 bytes, which the caller guarantees readable
  const uint64_t row_off = (uint64_t)row * P * kBlockBytes;
  const uint64_t total = ((uint64_t)out_f * P * kBlockBytes + 3) & ~3ull;
  const __amdgpu_buffer_rsrc_t rs = rsrc(blocks + (row_off & ~3ull), total - (row_off & ~3ull));
  const uint32_t skew = (uint32_t)(row_off & 3u);
  auto load = [&](int c, GgufRaw& r) {
    const uint32_t a = (uint32_t)min((int64_t)c * 64 + lane, P - 1);
    load_gguf_raw(rs, skew + a * kBlockBytes, r);
  };
  uint32_t ecur = 0, eend = 0;
  if constexpr (OVF) {
    ecur = ovf_off[row];
    eend = ovf_off[row + 1];
  }
  GgufRaw cur, nxt;
  load(0, cur);
  for (int c = 0; c < passes; ++c) {
    if (c + 1 < passes) load(c + 1, nxt);
    uint32_t p[16];
    decode_pairs<true>(gguf_atom(cur), p);
    uint32_t lo[8], hi[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      lo[i] = perm(p[2 * i + 1], p[2 * i], 0x05040100u);  // elements 2i, 2i+1
      hi[i] = perm(p[2 * i + 1], p[2 * i], 0x07060302u);  // elements 16+2i, 17+2i
    }
    *(u32x4*)(buf + chunk_slot(lane, 0)) = u32x4{lo[0], lo[1], lo[2], lo[3]};
    *(u32x4*)(buf + chunk_slot(lane, 1)) = u32x4{lo[4], lo[5], lo[6], lo[7]};
    *(u32x4*)(buf + chunk_slot(lane, 2)) = u32x4{hi[0], hi[1], hi[2], hi[3]};
    *(u32x4*)(buf + chunk_slot(lane, 3)) = u32x4{hi[4], hi[5], hi[6], hi[7]};
    const int64_t col0 = (int64_t)c * 2048;
    const int64_t nvalid = min((int64_t)2048, in_f - col0);
    if constexpr (OVF) {
      // same wave: these LDS writes land after the decoded values above
      while (ecur < eend) {
        const uint32_t e = ecur + (uint32_t)lane;
        const uint32_t en = e < eend ? ovf_ent[e] : 0xFFFFFFFFu;
        const uint32_t col = en & 0xFFFFu;
        const bool here = e < eend && (int64_t)col >= col0 && (int64_t)col < col0 + nvalid;
        if (here) {
          const uint32_t k = col - (uint32_t)col0;
          *(uint16_t*)(buf + chunk_slot((int)(k >> 5), (int)((k >> 3) & 3)) + (k & 7) * 2) = (uint16_t)(en >> 16);
        }
        // entries are sorted: those before the pass end are a prefix of the 64
        const uint32_t taken = (uint32_t)__builtin_popcountll(__ballot(e < eend && (int64_t)col < col0 + nvalid));
        ecur += taken;
        if (taken < 64) break;
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = 8 * lane + 512 * i;
      const u32x4 v = *(const u32x4*)(buf + chunk_slot(e >> 5, (e & 31) >> 3));
      if (e < nvalid) {
        if constexpr (F32) {
          float* o = (float*)out + row * in_f + col0 + e;
          const uint32_t v0 = v.x, v1 = v.y, v2 = v.z, v3 = v.w;
          *(float4*)o = float4{bf16lo_to_f32(v0), bf16hi_to_f32(v0), bf16lo_to_f32(v1), bf16hi_to_f32(v1)};
          *(float4*)(o + 4) = float4{bf16lo_to_f32(v2), bf16hi_to_f32(v2), bf16lo_to_f32(v3), bf16hi_to_f32(v3)};
        } else {
          *(u32x4a*)((uint16_t*)out + row * in_f + col0 + e) = v;
        }
      }
    }
    cur = nxt;
  }
}

// ---------------------------------------------------------------------------
// x (bf16, in_f) -> pair order per 32-element atom: word i of atom a =
// x[32a + i] | x[32a + 16 + i] << 16, the order decode_pairs produces
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void x_pairs_kernel(const uint16_t* __restrict__ x, int64_t in_f,
                                                      uint32_t* __restrict__ xp) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;   // word index
  if (i >= in_f / 2) return;
  const int64_t a = i >> 4, j = i & 15;
  xp[i] = (uint32_t)x[32 * a + j] | ((uint32_t)x[32 * a + 16 + j] << 16);
}

// ---------------------------------------------------------------------------
// GEMV: one wave per row; lane l takes blocks l, l+64, ... of the row (loads
// of consecutive lanes are contiguous) and the matching 64 bytes of paired x;
// 16 v_dot2_f32_bf16 per block, wave sum by shuffles, y in bf16 or fp32.
// Loads of the next pass are issued before the current one is used; lanes
// past the row's end load its last block again and add nothing.
// ---------------------------------------------------------------------------
// With OVF, each row adds the side table's correction: an entry's element
// decodes as the zero marker (exponent 0, the entry's sign and mantissa;
// checked on the host when the table is attached), so it contributes
// (exact - marker) * x[col].  The row's first 128 entries are loaded before
// the main loop.
template <bool YF32, bool OVF>
__global__ __launch_bounds__(256) void gguf_gemv_kernel(const uint8_t* __restrict__ blocks,
                                                        const uint32_t* __restrict__ xp, int64_t out_f,
                                                        int64_t in_f, const uint32_t* __restrict__ ovf_off,
                                                        const uint32_t* __restrict__ ovf_ent,
                                                        void* __restrict__ y) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // XCD-aware row order: consecutive rows on one XCD
  const int nb = (int)gridDim.x, b = (int)blockIdx.x;
  const int per = nb / 8, extra = nb - per * 8;
  const int lb = nb >= 8 ? ((b & 7) * per + min(b & 7, extra) + (b >> 3)) : b;
  const int64_t row = (int64_t)lb * 4 + wave;
  if (row >= out_f) return;
  const int64_t P = in_f >> 5;
  const int passes = (int)((P + 63) >> 6);
  const uint64_t row_off = (uint64_t)row * P * kBlockBytes;
  const uint64_t total = ((uint64_t)out_f * P * kBlockBytes + 3) & ~3ull;
  const __amdgpu_buffer_rsrc_t rs = rsrc(blocks + (row_off & ~3ull), total - (row_off & ~3ull));
  const uint32_t skew = (uint32_t)(row_off & 3u);
  const __amdgpu_buffer_rsrc_t rx = rsrc(xp, (uint64_t)in_f * 2);
  struct Ld { GgufRaw t; u32x4 x[4]; };
  auto load = [&](int c, Ld& l) {
    const int64_t ai = (int64_t)c * 64 + lane;
    const uint32_t a = (uint32_t)min(ai, P - 1);
    load_gguf_raw(rs, skew + a * kBlockBytes, l.t);
#pragma unroll
    for (int q = 0; q < 4; ++q) l.x[q] = __builtin_amdgcn_raw_buffer_load_b128(rx, (int)(a * 64 + 16 * q), 0, 0);
  };
  float acc = 0.f;
  uint32_t eb = 0, ee = 0, en0 = 0, en1 = 0;
  if constexpr (OVF) {
    eb = ovf_off[row];
    ee = ovf_off[row + 1];
    const uint32_t last = ee > 0 ? ee - 1 : 0;
    en0 = ovf_ent[min(eb + (uint32_t)lane, last)];
    en1 = ovf_ent[min(eb + 64u + (uint32_t)lane, last)];
  }
  Ld cur, nxt;
  load(0, cur);
  for (int c = 0; c < passes; ++c) {
    if (c + 1 < passes) load(c + 1, nxt);
    const bool live = (int64_t)c * 64 + lane < P;
    uint32_t w[16];
    decode_pairs<true>(gguf_atom(cur.t), w);
    float s = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const u32x4 xv = cur.x[q];
      const uint32_t x0 = xv.x, x1 = xv.y, x2 = xv.z, x3 = xv.w;
      s = dot2_bf16(w[4 * q + 0], x0, s);
      s = dot2_bf16(w[4 * q + 1], x1, s);
      s = dot2_bf16(w[4 * q + 2], x2, s);
      s = dot2_bf16(w[4 * q + 3], x3, s);
    }
    acc += live ? s : 0.f;
    cur = nxt;
  }
  if constexpr (OVF) {
    auto corr = [&](uint32_t en) -> float {
      const uint32_t col = min(en & 0xFFFFu, (uint32_t)in_f - 1);
      const uint32_t xw = xp[(col >> 5) * 16 + (col & 15)];
      const float xv = (col & 16) ? bf16hi_to_f32(xw) : bf16lo_to_f32(xw);
      const uint32_t b = en >> 16;
      return (bf16lo_to_f32(b) - bf16lo_to_f32(b & 0x807Fu)) * xv;
    };
    float cs = 0.f;
    const float c0 = corr(en0), c1 = corr(en1);
    cs += (eb + (uint32_t)lane < ee) ? c0 : 0.f;
    cs += (eb + 64u + (uint32_t)lane < ee) ? c1 : 0.f;
    for (uint32_t e = eb + 128u + (uint32_t)lane; e < ee; e += 64) cs += corr(ovf_ent[e]);
    acc += cs;
  }
  acc = wave_sum(acc);
  if (lane == 0) {
    if constexpr (YF32) ((float*)y)[row] = acc;
    else ((uint16_t*)y)[row] = (uint16_t)f32_to_bf16_rne(acc);
  }
}

// ---------------------------------------------------------------------------
// GEMV for rows of 64k columns (k >= 3, in_f <= 32768): the dict GEMV's
// long-row structure (gemv.hip, gemv_long_kernel).  One wave per row, the
// row streamed in NP passes of 64 blocks through a two-slot register ring
// that runs on across the wave's rows; x (bf16, 4-byte aligned) is read once
// per workgroup, rearranged into the decoder's pair order in registers and
// staged in LDS (lane-major: chunk (4 pass + q) * 64 + lane holds pair words
// 4q .. 4q+3 of block 64 pass + lane), so no separate x launch is needed;
// workgroup rows base + 4 i + wave, i < iters.  The
// row's base byte offset is a multiple of 4 (P even), so it enters the loads
// as a scalar offset and the 2-byte skew of a block is its lane's.  OVF: the
// side-table entries of a row (first 64 NP read one row ahead, the rest after
// the wave's last row), each adding (exact - marker) * x[col].
constexpr int kLongMaxIters = 16;

template <int NP, int XS, bool YF32, bool OVF>
__global__ __launch_bounds__(256) void gguf_gemv_long_kernel(const uint8_t* __restrict__ blocks,
                                                             const uint16_t* __restrict__ x, int64_t out_f,
                                                             int64_t in_f, const uint32_t* __restrict__ ovf_off,
                                                             const uint32_t* __restrict__ ovf_ent, int iters,
                                                             void* __restrict__ y) {
  static_assert(NP >= 2, "at least two passes per row");
  constexpr int NB = NP;
  extern __shared__ uint32_t lds[];
  __shared__ float dpart[4][kLongMaxIters];
  __shared__ int drow[4][kLongMaxIters];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int64_t P = in_f >> 5;
  const uint64_t total = ((uint64_t)out_f * P * kBlockBytes + 3) & ~3ull;
  const __amdgpu_buffer_rsrc_t rs = rsrc(blocks, total);
  const __amdgpu_buffer_rsrc_t roff = rsrc(ovf_off, OVF ? (uint64_t)(out_f + 1) * 4 : 0);

  const int nb = (int)gridDim.x, b = (int)blockIdx.x;
  const int per = nb / 8, extra = nb - per * 8;
  const int lb = nb >= 8 ? ((b & 7) * per + min(b & 7, extra) + (b >> 3)) : b;
  const int64_t base = (int64_t)lb * iters * 4 + wave;
  auto row_of = [&](int i) { return min(base + 4 * (int64_t)min(i, iters - 1), out_f - 1); };
  auto load_pass = [&](int i, int c, GgufRaw& t) {
    const uint32_t so = (uint32_t)(row_of(i) * P * kBlockBytes);   // multiple of 4
    const uint32_t boff = (uint32_t)min((int64_t)(64 * c + lane), P - 1) * kBlockBytes;
    const uint32_t vb = boff & ~3u;
    t.sh = (boff & 2u) * 8u;
    t.q0 = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)vb, (int)so, 0);
    t.q1 = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)(vb + 16), (int)so, 0);
    t.q2 = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)(vb + 32), (int)so, 0);
  };
  auto load_off = [&](int i, uint32_t& b0, uint32_t& b1) {
    const int rc = (int)row_of(i);
    b0 = __builtin_amdgcn_raw_buffer_load_b32(roff, rc * 4, 0, 0);
    b1 = __builtin_amdgcn_raw_buffer_load_b32(roff, rc * 4 + 4, 0, 0);
  };
  auto load_ents = [&](uint32_t b0, uint32_t b1, uint32_t* ent) {
    const uint32_t last = b1 > 0 ? b1 - 1 : 0;
#pragma unroll
    for (int k = 0; k < NB; ++k) ent[k] = ovf_ent[min(b0 + (uint32_t)(lane + 64 * k), last)];
  };
  auto x_at = [&](uint32_t k) -> float {
    const uint32_t a = k >> 5, j = k & 15, hi = (k >> 4) & 1;
    const uint32_t wd = lds[((((a >> 6) * 4) + (j >> 2)) * 64 + (a & 63)) * 4 + (j & 3)];
    return hi ? bf16hi_to_f32(wd) : bf16lo_to_f32(wd);
  };
  auto corr = [&](uint32_t en) -> float {   // (exact - marker) * x[col]
    const uint32_t col = min(en & 0xFFFFu, (uint32_t)in_f - 1);
    const uint32_t bits = en >> 16;
    return (bf16lo_to_f32(bits) - bf16lo_to_f32(bits & 0x807Fu)) * x_at(col);
  };

  // prologue: offsets of rows 0 and 1, x (registers, natural order, by the
  // threads that store it: loads under the store's condition stay ahead of
  // the passes instead of being moved behind them), the first two passes,
  // the entries of row 0 (their addresses wait for the offsets); x to LDS in
  // pair order, waiting for x alone
  uint32_t ob0 = 0, ob1 = 0, on0 = 0, on1 = 0;
  if constexpr (OVF) {
    load_off(0, ob0, ob1);
    load_off(1, on0, on1);
  }
  const __amdgpu_buffer_rsrc_t rx = rsrc(x, (uint64_t)in_f * 2);
  u32x4 xs[XS][4];                              // block a's 32 x values, natural order
#pragma unroll
  for (int i = 0; i < XS; ++i) {
    if (threadIdx.x + 256 * i < NP * 64) {
      const uint32_t a = (uint32_t)min((int64_t)(threadIdx.x + 256 * i), P - 1);
#pragma unroll
      for (int q = 0; q < 4; ++q) xs[i][q] = __builtin_amdgcn_raw_buffer_load_b128(rx, (int)(a * 64 + 16 * q), 0, 0);
    }
  }
  GgufRaw R[2];
  load_pass(0, 0, R[0]);
  load_pass(0, 1, R[1]);
  __builtin_amdgcn_sched_barrier(0);
  uint32_t ent[NB] = {};
  if constexpr (OVF) load_ents(ob0, ob1, ent);
#pragma unroll
  for (int i = 0; i < XS; ++i) {
    const int a = threadIdx.x + 256 * i;
    if (a < NP * 64) {
      // natural -> pair order: word j = x[32a + j] | x[32a + 16 + j] << 16
      const uint32_t lo[8] = {xs[i][0].x, xs[i][0].y, xs[i][0].z, xs[i][0].w,
                              xs[i][1].x, xs[i][1].y, xs[i][1].z, xs[i][1].w};
      const uint32_t hi[8] = {xs[i][2].x, xs[i][2].y, xs[i][2].z, xs[i][2].w,
                              xs[i][3].x, xs[i][3].y, xs[i][3].z, xs[i][3].w};
      uint32_t pw[16];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        pw[2 * k] = perm(hi[k], lo[k], 0x05040100u);
        pw[2 * k + 1] = perm(hi[k], lo[k], 0x07060302u);
      }
      u32x4* dst = (u32x4*)lds + (a >> 6) * 4 * 64 + (a & 63);
#pragma unroll
      for (int q = 0; q < 4; ++q) dst[q * 64] = u32x4{pw[4 * q], pw[4 * q + 1], pw[4 * q + 2], pw[4 * q + 3]};
    }
  }
  __syncthreads();

  const u32x4* xl = (const u32x4*)lds + lane;
  float acc0 = 0.f, acc1 = 0.f;
  bool more = false;
  int nparked = 0;
  auto do_row = [&](int i, auto par) {
    constexpr int PAR = decltype(par)::value;
#pragma unroll
    for (int c = 0; c < NP; ++c) {
      GgufRaw& cur = R[(PAR + c) & 1];
      uint32_t w[16];
      decode_pairs<true>(gguf_atom(cur), w);
      float t0 = 0.f, t1 = 0.f;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const u32x4 v = xl[(c * 4 + q) * 64];
        t0 = dot2_bf16(w[4 * q + 0], v.x, t0);
        t1 = dot2_bf16(w[4 * q + 1], v.y, t1);
        t0 = dot2_bf16(w[4 * q + 2], v.z, t0);
        t1 = dot2_bf16(w[4 * q + 3], v.w, t1);
      }
      if (c < NP - 1 || (int64_t)(64 * c + lane) < P) {
        acc0 += t0;
        acc1 += t1;
      }
      if (c + 2 < NP) load_pass(i, c + 2, cur);
      else load_pass(i + 1, c + 2 - NP, cur);
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (OVF) {
#pragma unroll
      for (int k = 0; k < NB; ++k) {
        const float cc = corr(ent[k]);
        acc0 += (ob0 + (uint32_t)(lane + 64 * k) < ob1) ? cc : 0.f;
      }
      more = __builtin_amdgcn_readfirstlane(ob1) > __builtin_amdgcn_readfirstlane(ob0) + 64u * NB;
      uint32_t nn0, nn1;
      load_off(i + 2, nn0, nn1);
      load_ents(on0, on1, ent);
      ob0 = on0; ob1 = on1; on0 = nn0; on1 = nn1;
    }
    const float tot = wave_sum_dpp(acc0 + acc1);
    const int64_t r = base + 4 * (int64_t)i;
    if (OVF && more) {
      if (lane == 63) {
        dpart[wave][nparked] = tot;
        drow[wave][nparked] = i;
      }
      ++nparked;
    } else if (lane == 63 && r < out_f) {
      if constexpr (YF32) ((float*)y)[r] = tot;
      else ((uint16_t*)y)[r] = (uint16_t)f32_to_bf16_rne(tot);
    }
    acc0 = 0.f;
    acc1 = 0.f;
  };
  if constexpr (NP % 2 == 0) {
    for (int i = 0; i < iters; ++i) do_row(i, std::integral_constant<int, 0>{});
  } else {
    int i = 0;
    for (; i + 1 < iters; i += 2) {
      do_row(i, std::integral_constant<int, 0>{});
      do_row(i + 1, std::integral_constant<int, 1>{});
    }
    if (i < iters) do_row(i, std::integral_constant<int, 0>{});
  }
  for (int d = 0; d < nparked; ++d) {            // rows with more entries than the read-ahead
    const int i = __builtin_amdgcn_readfirstlane(drow[wave][d]);
    const int64_t r = base + 4 * (int64_t)i;
    const uint32_t b0 = ovf_off[row_of(i)], b1 = ovf_off[row_of(i) + 1];
    float a = 0.f;
    for (uint32_t e = b0 + 64u * NB + (uint32_t)lane; e < b1; e += 64) a += corr(ovf_ent[e]);
    const float tot = wave_sum_dpp(a) + dpart[wave][d];
    if (lane == 63 && r < out_f) {
      if constexpr (YF32) ((float*)y)[r] = tot;
      else ((uint16_t*)y)[r] = (uint16_t)f32_to_bf16_rne(tot);
    }
  }
}

}  // namespace gguf
}  // namespace bf16x

using namespace bf16x::gguf;

namespace {

int check_gguf(const void* blocks, int64_t n_bytes, int64_t out_f, int64_t in_f) {
  if (!blocks) return BF16X_EARG;
  if (out_f <= 0 || in_f <= 0 || (in_f % 32) != 0) return BF16X_ESHAPE;
  const int64_t nb = out_f * (in_f / 32);
  if (nb > ((int64_t)1 << 31)) return BF16X_ESHAPE;
  if (n_bytes < ((nb * kBlockBytes + 3) & ~(int64_t)3)) return BF16X_ESTREAM_LEN;
  if ((in_f / 32) * kBlockBytes >= (int64_t)0xFFFFFFF0) return BF16X_ESHAPE;   // one row's offsets in 32 bits
  return BF16X_OK;
}

}  // namespace

namespace {

int check_ovf(const uint32_t* row_off, const uint32_t* entries, int64_t n_entries) {
  if (!row_off || !entries || n_entries < 0 || n_entries > 0xFFFFFFFFll) return BF16X_EARG;
  if (!aligned4(row_off) || !aligned4(entries)) return BF16X_EARG;
  return BF16X_OK;
}

int gguf_decode_launch(const uint8_t* blocks, int64_t n_bytes, int64_t out_f, int64_t in_f, const uint32_t* ovf_off,
                       const uint32_t* ovf_ent, void* out, int32_t out_dtype, hipStream_t st) {
  int rc = check_gguf(blocks, n_bytes, out_f, in_f);
  if (rc) return rc;
  if (!out) return BF16X_EARG;
  if (out_dtype != BF16X_BF16 && out_dtype != BF16X_F32) return BF16X_EDTYPE;
  if (!aligned16(out) || !aligned4(blocks)) return BF16X_EARG;
  const int64_t grid = (out_f + 3) / 4;
  if (grid > INT32_MAX) return BF16X_ESHAPE;
  const dim3 g((unsigned)grid), b(256);
  if (ovf_off) {
    if (out_dtype == BF16X_F32)
      hipLaunchKernelGGL((gguf_decode_kernel<true, true>), g, b, 0, st, blocks, out_f, in_f, ovf_off, ovf_ent, out);
    else
      hipLaunchKernelGGL((gguf_decode_kernel<false, true>), g, b, 0, st, blocks, out_f, in_f, ovf_off, ovf_ent, out);
  } else {
    if (out_dtype == BF16X_F32)
      hipLaunchKernelGGL((gguf_decode_kernel<true, false>), g, b, 0, st, blocks, out_f, in_f, nullptr, nullptr, out);
    else
      hipLaunchKernelGGL((gguf_decode_kernel<false, false>), g, b, 0, st, blocks, out_f, in_f, nullptr, nullptr, out);
  }
  return launch_status();
}

// BF16X_TUNE_GGUF_LONG = 0 keeps every shape on the one-pass-ahead kernel.
bool long_enabled() { return tuning(BF16X_TUNE_GGUF_LONG) != 0; }

int gguf_gemv_launch(const void* x, int32_t x_dtype, const uint8_t* blocks, int64_t n_bytes, int64_t out_f,
                     int64_t in_f, const uint32_t* ovf_off, const uint32_t* ovf_ent, void* y, int32_t y_dtype,
                     void* workspace, int64_t workspace_bytes, hipStream_t st) {
  int rc = check_gguf(blocks, n_bytes, out_f, in_f);
  if (rc) return rc;
  if (!x || !y || !workspace) return BF16X_EARG;
  if (x_dtype != BF16X_BF16 || (y_dtype != BF16X_BF16 && y_dtype != BF16X_F32)) return BF16X_EDTYPE;
  if (workspace_bytes < in_f * 2) return BF16X_ECAPACITY;
  if (!aligned2(x) || !aligned16(workspace) || !aligned4(blocks) || !aligned4(y)) return BF16X_EARG;
  const int64_t grid = (out_f + 3) / 4;
  if (grid > INT32_MAX) return BF16X_ESHAPE;
  uint32_t* xp = (uint32_t*)workspace;
  const int64_t P = in_f / 32;
  const int np = (int)((P + 63) / 64);
  if (long_enabled() && P % 2 == 0 && np >= 3 && np <= 16 && aligned4(x)) {
    // rows per wave (as the dict GEMV): 4 from 2048 groups of 4 rows, 2 from 1024
    const int64_t groups = (out_f + 3) / 4;
    int iters = groups >= 2048 ? 4 : (groups >= 1024 ? 2 : 1);
    if (const int64_t t = tuning(BF16X_TUNE_GGUF_ITERS); t > 0) iters = (int)std::min<int64_t>(t, kLongMaxIters);
    const int64_t lgrid = (groups + iters - 1) / iters;
    const size_t lds = (size_t)np * 4 * 64 * 16;
    const int xs = (np * 64 + 255) / 256;
#define BF16X_GL1(NP_, XS_, YF_, OV_)                                                                           \
  hipLaunchKernelGGL((gguf_gemv_long_kernel<NP_, XS_, YF_, OV_>), dim3((unsigned)lgrid), dim3(256), lds, st, blocks, \
                     (const uint16_t*)x, out_f, in_f, ovf_off, ovf_ent, iters, y)
#define BF16X_GL(NP_)                                                                                           \
  case NP_:                                                                                                     \
    if (ovf_off) { if (y_dtype == BF16X_F32) BF16X_GL1(NP_, (NP_ * 64 + 255) / 256, true, true);               \
                   else BF16X_GL1(NP_, (NP_ * 64 + 255) / 256, false, true); }                                  \
    else { if (y_dtype == BF16X_F32) BF16X_GL1(NP_, (NP_ * 64 + 255) / 256, true, false);                      \
           else BF16X_GL1(NP_, (NP_ * 64 + 255) / 256, false, false); }                                         \
    break;
    (void)xs;
    switch (np) {
      BF16X_GL(3) BF16X_GL(4) BF16X_GL(5) BF16X_GL(6) BF16X_GL(7) BF16X_GL(8) BF16X_GL(9) BF16X_GL(10)
      BF16X_GL(11) BF16X_GL(12) BF16X_GL(13) BF16X_GL(14) BF16X_GL(15) BF16X_GL(16)
      default: break;
    }
#undef BF16X_GL
#undef BF16X_GL1
    return launch_status();
  }
  hipLaunchKernelGGL(x_pairs_kernel, dim3((unsigned)((in_f / 2 + 255) / 256)), dim3(256), 0, st, (const uint16_t*)x,
                     in_f, xp);
  const dim3 g((unsigned)grid), b(256);
  if (ovf_off) {
    if (y_dtype == BF16X_F32)
      hipLaunchKernelGGL((gguf_gemv_kernel<true, true>), g, b, 0, st, blocks, xp, out_f, in_f, ovf_off, ovf_ent, y);
    else
      hipLaunchKernelGGL((gguf_gemv_kernel<false, true>), g, b, 0, st, blocks, xp, out_f, in_f, ovf_off, ovf_ent, y);
  } else {
    if (y_dtype == BF16X_F32)
      hipLaunchKernelGGL((gguf_gemv_kernel<true, false>), g, b, 0, st, blocks, xp, out_f, in_f, nullptr, nullptr, y);
    else
      hipLaunchKernelGGL((gguf_gemv_kernel<false, false>), g, b, 0, st, blocks, xp, out_f, in_f, nullptr, nullptr, y);
  }
  return launch_status();
}

}  // namespace

extern "C" int bf16x_gguf_decode(const uint8_t* blocks, int64_t n_bytes, int64_t out_f, int64_t in_f, void* out,
                                 int32_t out_dtype, bf16x_stream_t stream) {
  return gguf_decode_launch(blocks, n_bytes, out_f, in_f, nullptr, nullptr, out, out_dtype, (hipStream_t)stream);
}

extern "C" int bf16x_gguf_decode_lossless(const uint8_t* blocks, int64_t n_bytes, int64_t out_f, int64_t in_f,
                                          const uint32_t* row_off, const uint32_t* entries, int64_t n_entries,
                                          void* out, int32_t out_dtype, bf16x_stream_t stream) {
  const int rc = check_ovf(row_off, entries, n_entries);
  if (rc) return rc;
  return gguf_decode_launch(blocks, n_bytes, out_f, in_f, row_off, entries, out, out_dtype, (hipStream_t)stream);
}

extern "C" int64_t bf16x_gguf_gemv_workspace(int64_t in_f) { return in_f > 0 ? in_f * 2 : 0; }

// ---------------------------------------------------------------------------
// Allocation-free GEMV (bf16x_gguf_gemv_noalloc): the workspace of
// bf16x_gguf_gemv (x rearranged in decode order, in_f * 2 bytes) lives in a
// fixed device array instead, so callers that cannot allocate (graph
// capture, serving loops) pass only inputs and outputs.  Each GPU the library
// runs on holds its own copy of the array for the life of the process; every
// call on that GPU reuses it, so calls that overlap on one GPU race.  The
// array is written in full before it is read, so it needs no clearing.
// ---------------------------------------------------------------------------
namespace {
constexpr int64_t kNoAllocScratchBytes = (int64_t)1 << 17;   // in_f <= 65536
}  // namespace

static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];   // this GPU's address of `scratch`, looked up once

// Device address of the current GPU's copy of `scratch`.  The host-side name
// of a __device__ array is only a stand-in; the address is looked up with
// the device current and kept per device.
int scratch_ptr(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return BF16X_EARG;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return BF16X_OK;
}
}  // namespace

extern "C" int bf16x_gguf_gemv_noalloc(const void* x, int32_t x_dtype, const uint8_t* blocks, int64_t n_bytes,
                                       int64_t out_f, int64_t in_f, void* y, int32_t y_dtype,
                                       bf16x_stream_t stream) {
  if (!x || !y || !blocks) return BF16X_EARG;
  if (in_f * 2 > kNoAllocScratchBytes) return BF16X_ECAPACITY;
  void* ws = nullptr;
  const int rc = scratch_ptr(&ws);
  if (rc) return rc;
  return gguf_gemv_launch(x, x_dtype, blocks, n_bytes, out_f, in_f, nullptr, nullptr, y, y_dtype, ws,
                          kNoAllocScratchBytes, (hipStream_t)stream);
}

extern "C" int bf16x_gguf_gemv(const void* x, int32_t x_dtype, const uint8_t* blocks, int64_t n_bytes, int64_t out_f,
                               int64_t in_f, void* y, int32_t y_dtype, void* workspace, int64_t workspace_bytes,
                               bf16x_stream_t stream) {
  return gguf_gemv_launch(x, x_dtype, blocks, n_bytes, out_f, in_f, nullptr, nullptr, y, y_dtype, workspace,
                          workspace_bytes, (hipStream_t)stream);
}

extern "C" int bf16x_gguf_gemv_lossless(const void* x, int32_t x_dtype, const uint8_t* blocks, int64_t n_bytes,
                                        int64_t out_f, int64_t in_f, const uint32_t* row_off,
                                        const uint32_t* entries, int64_t n_entries, void* y, int32_t y_dtype,
                                        void* workspace, int64_t workspace_bytes, bf16x_stream_t stream) {
  const int rc = check_ovf(row_off, entries, n_entries);
  if (rc) return rc;
  return gguf_gemv_launch(x, x_dtype, blocks, n_bytes, out_f, in_f, row_off, entries, y, y_dtype, workspace,
                          workspace_bytes, (hipStream_t)stream);
}

// ---------------------------------------------------------------------------
// Fused decode + GEMM over GGUF blocks: the wave-specialised kernel of
// gemm_ws.hip with its block loader (46-byte blocks, zero-marker decode).
// The lossless table enters as the step-major plan of bf16x_gguf_kplan_build.
// ---------------------------------------------------------------------------
int64_t bf16x_gemm_ws_workspace(int64_t M, int64_t out_f, int64_t in_f);
int bf16x_gemm_ws_launch(const uint16_t* x, int64_t M, const uint32_t* s, const uint32_t* m, const uint32_t* d,
                         const uint16_t* e, const uint8_t* blocks, const uint32_t* kp_off, const uint32_t* kp_ent,
                         int64_t out_f, int64_t in_f, bool exact, bool yf32, void* y, void* workspace,
                         int64_t workspace_bytes, hipStream_t st);

extern "C" int64_t bf16x_gguf_gemm_workspace(int64_t M, int64_t out_f, int64_t in_f) {
  if (M <= 0 || out_f <= 0 || in_f < 64 || (in_f % 64) != 0) return 0;
  return bf16x_gemm_ws_workspace(M, out_f, in_f);
}

extern "C" int bf16x_gguf_gemm(const void* x, int32_t x_dtype, int64_t M, const uint8_t* blocks, int64_t n_bytes,
                               const uint32_t* kp_off, const uint32_t* kp_ent, int64_t out_f, int64_t in_f, void* y,
                               int32_t y_dtype, void* workspace, int64_t workspace_bytes, bf16x_stream_t stream) {
  int rc = check_gguf(blocks, n_bytes, out_f, in_f);
  if (rc) return rc;
  if (!x || !y || (kp_off == nullptr) != (kp_ent == nullptr)) return BF16X_EARG;
  if (x_dtype != BF16X_BF16 || (y_dtype != BF16X_BF16 && y_dtype != BF16X_F32)) return BF16X_EDTYPE;
  if (M <= 0 || (in_f % 64) != 0) return BF16X_ESHAPE;
  if (kp_off && in_f > 65536) return BF16X_ESHAPE;   // the plan's 16-bit columns
  // 32-bit buffer offsets: x in operand order, and one 128-row tile of blocks
  if (M * in_f * 2 >= (int64_t)0xFFFFFFFF || 128 * (in_f / 32) * kBlockBytes >= (int64_t)0xFFFFFFF0)
    return BF16X_ESHAPE;
  if (!aligned16(x) || !aligned4(blocks) || !aligned4(y)) return BF16X_EARG;
  if (kp_off && (!aligned4(kp_off) || !aligned4(kp_ent))) return BF16X_EARG;
  rc = bf16x_gemm_ws_launch((const uint16_t*)x, M, nullptr, nullptr, nullptr, nullptr, blocks, kp_off, kp_ent, out_f,
                            in_f, kp_off != nullptr, y_dtype == BF16X_F32, y, workspace, workspace_bytes,
                            (hipStream_t)stream);
  return rc ? rc : launch_status();
}
