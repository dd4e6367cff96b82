// Fused decode + GEMM for up to 16 activation rows over weights of 2048 or
// 4096 columns, with the GEMV's memory pattern.
//
// y[M, N] = x[M, K] . W[N, K]^T, fp32 accumulation, M <= 16
// (bf16x_gemm_fused.py:97-114 at its smallest block, BM = 16; EXACT applies
// the row plan, the GEMV's overflow table).
//
// Why: the few-row kernel of gemm_skinny2.hip reads W as 16 rows x 4 atoms
// per load instruction and restages x through LDS at every step; its memory
// skeleton alone (loads, x tile, barriers, no decode) takes longer than the
// whole batch-1 GEMV at 14336x4096.  Here every wave streams whole rows
// exactly as the GEMV does (lane l loads atoms l and 64 + l of its row, the
// row's four streams contiguous), and x is loaded once per workgroup into
// registers in MFMA operand order.
//
// Layout.  One workgroup of 8 waves per CU takes a contiguous run of rows
// (at most 120, a multiple of 8) and walks it in groups of 16 rows.  For each
// group, wave w loads, decodes and writes rows w and w + 8 of the group into
// an LDS tile (the EXACT plan entries of a row written over it by the same
// wave), and requests the next group's atoms and entries as it goes; after a
// barrier every wave multiplies its own K range of the tile:
// v_mfma_f32_16x16x32_bf16 with A = W (the group's 16 rows), B = x (16
// tokens, zero past M).  The 8 partial products of a group are added in wave
// order through LDS and stored.
//
// MFMA k order (as in gemm_skinny2.hip): MFMA i of k-step s takes pair words
// 4i .. 4i+3 of atom 4s + q of row r as lane l = r + 16 q's A operand (words
// hold elements j and j + 16 of an atom); B holds x at the same elements.
// Result register v of lane l = D[4 (l / 16) + v][l % 16]: W row 4 (l / 16)
// + v, token l % 16.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "../../include/bf16x_hip.h"
#include "bf16x_device.h"
#include "gemv_pipe.h"
#include "launch_common.h"

namespace bf16x {
namespace rows16 {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kGroupRows = 16;                // rows per group = MFMA rows
constexpr int kRPW = 2;                       // rows of a group per wave
constexpr int kWaves = kGroupRows / kRPW;     // waves per workgroup
constexpr int kThreads = 64 * kWaves;
constexpr int kMaxTokens = 16;
constexpr int kRedBytes = kWaves * 64 * 16;   // partial sums: per wave 64 lanes x 4 floats
constexpr int kEntBatches = 2;                // plan entries prefetched per lane per row (64 per batch)
constexpr int kMaxRowsWG = 120;               // rows per workgroup at most (its plan offsets in 2 registers)

// 16-byte chunk k (0..3) of atom a in an LDS tile row, swizzled by a / 4,
// rows skewed by 16 bytes, so that the lanes of a decode write (consecutive
// atoms, same k) and of an MFMA read (16 rows x 4 atoms, same chunk) spread
// over the banks.  The counters still report about two conflict cycles per
// LDS instruction cycle; other swizzles (by a / 2) and skews (32 bytes)
// measured within 1 % of this one.
__device__ __forceinline__ int chunk_off(int a, int k) { return a * 64 + ((k ^ (a >> 2)) & 3) * 16; }

// Workgroup b takes rows [b R, min((b + 1) R, out_f)), R = rows_per_wg (a
// multiple of 8), as groups of 16 rows (the last one possibly 8).
template <int NA, bool EXACT, bool YF32>
__global__ __launch_bounds__(kThreads) void gemm_rows_kernel(const uint16_t* __restrict__ x, int M,
                                                         const uint32_t* __restrict__ sign,
                                                         const uint32_t* __restrict__ mant,
                                                         const uint32_t* __restrict__ delta,
                                                         const uint16_t* __restrict__ emax2,
                                                         const uint32_t* __restrict__ tile_off,
                                                         const uint32_t* __restrict__ tile_ent, int out_f, int in_f,
                                                         int rows_per_wg, void* __restrict__ y) {
  constexpr int P = 64 * NA;                  // atoms per row
  constexpr int kRowBytes = P * 64 + 16;      // LDS tile row: P atoms x 64 bytes + 16 (bank skew)
  constexpr int kTileBytes = kGroupRows * kRowBytes;
  constexpr int S = P / 4;                    // MFMA k-steps per row (128 columns each)
  constexpr int SW = S / kWaves;              // k-steps per wave
  static_assert(SW >= 1 && S % kWaves == 0, "whole k-steps per wave");
  // decoded tile, partial sums, a slot per lane for masked plan writes
  // (139,776 bytes at 4096 columns, 74,240 at 2048)
  __shared__ __attribute__((aligned(16))) uint8_t lds[kTileBytes + kRedBytes + 256];
  uint8_t* const tile = lds;
  float* const red = (float*)(lds + kTileBytes);
  uint8_t* const trash = lds + kTileBytes + kRedBytes;     // 64 lanes x 4 bytes

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, q = lane >> 4;      // MFMA role: row r, atom q of a k-step
  const int rbeg = blockIdx.x * rows_per_wg;
  const int rend = min(rbeg + rows_per_wg, out_f);
  if (rbeg >= rend) return;
  const int n = (rend - rbeg + kGroupRows - 1) / kGroupRows;   // groups of this workgroup

  // ---- x in MFMA operand order, once: k-step s = wave * SW + j, MFMA i,
  // token r: elements 32 a + 4 i + {0..3} and 32 a + 16 + 4 i + {0..3} of
  // atom a = 4 s + q, interleaved (e0, e16, e1, e17, ...)
  bf16x8_t xb[SW][4];
  auto stage_x = [&]() {
    const bool live = r < M;
    const __amdgpu_buffer_rsrc_t rx = buf_rsrc(x, (uint64_t)M * in_f * 2);
    const uint32_t xrow = (uint32_t)(live ? r : 0) * (uint32_t)in_f * 2;
#pragma unroll
    for (int j = 0; j < SW; ++j) {
      const int a = 4 * (wave * SW + j) + q;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t off = xrow + (uint32_t)(32 * a + 4 * i) * 2;
        const u32x2 lo = __builtin_amdgcn_raw_buffer_load_b64(rx, (int)off, 0, 0);
        const u32x2 hi = __builtin_amdgcn_raw_buffer_load_b64(rx, (int)off + 32, 0, 0);
        const uint32_t l0 = live ? lo.x : 0u, l1 = live ? lo.y : 0u, h0 = live ? hi.x : 0u, h1 = live ? hi.y : 0u;
        const uint32_t w[4] = {perm(h0, l0, 0x05040100u), perm(h0, l0, 0x07060302u), perm(h1, l1, 0x05040100u),
                               perm(h1, l1, 0x07060302u)};
        __builtin_memcpy(&xb[j][i], w, 16);
      }
    }
  };

  // ---- this wave's rows of group k (rows wave + kWaves j of the group):
  // atoms l, 64 + l through raw buffer loads.  Rows past the workgroup's end
  // (a last group of 8) re-read its last row.
  const uint64_t Pl = (uint64_t)(in_f >> 5);
  const __amdgpu_buffer_rsrc_t rs_ = buf_rsrc(sign, (uint64_t)out_f * Pl * 4);
  const __amdgpu_buffer_rsrc_t rm_ = buf_rsrc(mant, (uint64_t)out_f * Pl * 28);
  const __amdgpu_buffer_rsrc_t rd_ = buf_rsrc(delta, (uint64_t)out_f * Pl * 12);
  const __amdgpu_buffer_rsrc_t re_ = buf_rsrc(emax2, (uint64_t)out_f * Pl * 2);
  auto row_of = [&](int k, int j) { return rbeg + kGroupRows * k + kWaves * j + wave; };
  auto load_row = [&](int rr, Atom (&t)[NA]) {
    const uint32_t sa = (uint32_t)(min(rr, rend - 1) * P);
#pragma unroll
    for (int s = 0; s < NA; ++s) t[s] = load_atom_buf(rs_, rm_, rd_, re_, (uint32_t)(64 * s + lane), sa);
  };
  // plan entries of the row: the first kEntBatches x 64, through a buffer
  // descriptor that spans exactly the row's entries (reads past the row end
  // return 0 and are masked where they are patched; the rest of a long row,
  // rare, is read where it is patched).  The row offsets of the whole
  // workgroup (at most kMaxRowsWG + 1) are loaded once, lane i of vo[h]
  // holding tile_off[rbeg + 64 h + i], and read back with v_readlane: no
  // memory wait inside the loop.
  struct Ent {
    uint32_t b0, b1;
    uint32_t e[kEntBatches];
  };
  uint32_t vo[2] = {0u, 0u};
  if constexpr (EXACT) {
    const __amdgpu_buffer_rsrc_t roff = buf_rsrc(tile_off, (uint64_t)(out_f + 1) * 4);
#pragma unroll
    for (int h = 0; h < 2; ++h)
      vo[h] = __builtin_amdgcn_raw_buffer_load_b32(roff, min(rbeg + 64 * h + lane, out_f) * 4, 0, 0);
  }
  auto off_at = [&](int rl) {                // tile_off[rbeg + rl], rl < 128 (wave-uniform)
    return (uint32_t)__builtin_amdgcn_readlane((int)(rl < 64 ? vo[0] : vo[1]), rl & 63);
  };
  auto load_ent = [&](int rr, Ent& en) {
    const int rl = min(rr, rend - 1) - rbeg;
    const uint32_t o0 = off_at(rl), o1 = off_at(rl + 1);
    en.b0 = o0;
    en.b1 = rr < rend ? o1 : o0;                             // row past the end: no entries
    const __amdgpu_buffer_rsrc_t re_row =
        __builtin_amdgcn_make_buffer_rsrc((void*)(tile_ent + o0), (short)0, (int)((en.b1 - o0) * 4u), 0x00020000);
#pragma unroll
    for (int b = 0; b < kEntBatches; ++b)
      en.e[b] = __builtin_amdgcn_raw_buffer_load_b32(re_row, (lane + 64 * b) * 4, 0, 0);
  };
  auto fetch = [&](int k, Atom (&t)[kRPW][NA], Ent (&en)[kRPW]) {
#pragma unroll
    for (int j = 0; j < kRPW; ++j) {
      const int rr = row_of(min(k, n - 1), j);
      load_row(rr, t[j]);
      if constexpr (EXACT) load_ent(rr, en[j]);
    }
  };
  auto load_atom_of = [&](int k, int j, int s_) {
    const uint32_t sa = (uint32_t)(min(row_of(min(k, n - 1), j), rend - 1) * P);
    return load_atom_buf(rs_, rm_, rd_, re_, (uint32_t)(64 * s_ + lane), sa);
  };
  auto patch_one = [&](uint8_t* myrow, uint32_t e, bool live) {
    const int c = (int)(e >> 16);                           // column (< 4096)
    const int a = c >> 5, j = c & 15, h = (c >> 4) & 1;
    uint8_t* dst = live ? myrow + chunk_off(a, j >> 2) + (j & 3) * 4 + h * 2 : trash + lane * 4;
    *(uint16_t*)dst = (uint16_t)(e & 0xFFFFu);
  };

  // one group: decode this wave's rows (atoms in `cur`) into the tile,
  // patch, barrier, MFMAs over this wave's K range (two independent
  // accumulator chains), partials to LDS, barrier, sum of the partials.
  // The next group's atoms and entries (into `nxt`, `en`) are requested one
  // by one as the current ones are decoded: the waves of a workgroup run in
  // step, and requesting a whole group at once stalls their issue until the
  // CU's load path has taken every request.
  auto group = [&](int k, Atom (&cur)[kRPW][NA], const Ent (&ec)[kRPW], Atom (&nxt)[kRPW][NA],
                   Ent (&en)[kRPW]) {
#pragma unroll
    for (int jr = 0; jr < kRPW; ++jr) {
      uint8_t* const myrow = tile + (kWaves * jr + wave) * kRowBytes;
#pragma unroll
      for (int s = 0; s < NA; ++s) {
        uint32_t w[16];
        decode_pairs(cur[jr][s], w);
        const int a = 64 * s + lane;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
          *(u32x4*)(myrow + chunk_off(a, kk)) = u32x4{w[4 * kk], w[4 * kk + 1], w[4 * kk + 2], w[4 * kk + 3]};
        __builtin_amdgcn_sched_barrier(0);
        nxt[jr][s] = load_atom_of(k + 1, jr, s);
        __builtin_amdgcn_sched_barrier(0);
      }
      if constexpr (EXACT) {
        const uint32_t b0 = ec[jr].b0, b1 = ec[jr].b1;
#pragma unroll
        for (int b = 0; b < kEntBatches; ++b) patch_one(myrow, ec[jr].e[b], b0 + (uint32_t)(lane + 64 * b) < b1);
        for (uint32_t e = b0 + (uint32_t)(lane + 64 * kEntBatches); e < b1; e += 64)
          patch_one(myrow, tile_ent[e], true);
        __builtin_amdgcn_sched_barrier(0);
        load_ent(row_of(min(k + 1, n - 1), jr), en[jr]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    __syncthreads();
    f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
    const uint8_t* arow = tile + r * kRowBytes;
#pragma unroll
    for (int jj = 0; jj < SW; ++jj) {
      const int a = 4 * (wave * SW + jj) + q;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bf16x8_t av = *(const bf16x8_t*)(arow + chunk_off(a, i));
        acc[i & 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, xb[jj][i], acc[i & 1], 0, 0, 0);
      }
    }
    {
      const f32x4 sum = acc[0] + acc[1];
      const float v0 = sum.x, v1 = sum.y, v2 = sum.z, v3 = sum.w;
      *(f32x4*)(red + (wave * 64 + lane) * 4) = f32x4{v0, v1, v2, v3};
    }
    __syncthreads();
    if (tid < kGroupRows * kMaxTokens) {
      const int row = tid & 15, t = tid >> 4;               // output (row of the group, token)
      const int ln = 16 * (row >> 2) + t, v = row & 3;
      float sum = red[ln * 4 + v];
#pragma unroll
      for (int w = 1; w < kWaves; ++w) sum += red[(w * 64 + ln) * 4 + v];
      const int orow = rbeg + kGroupRows * k + row;
      if (t < M && orow < rend) {
        if constexpr (YF32) ((float*)y)[(int64_t)t * out_f + orow] = sum;
        else ((uint16_t*)y)[(int64_t)t * out_f + orow] = (uint16_t)f32_to_bf16_rne(sum);
      }
    }
  };

  // The next group's rows and entries are requested while the current one
  // is decoded; past the last group the request re-reads it (from L2), so
  // every path through the loop has the same loads in flight and the waits
  // for a group's rows count only theirs.  The loop has one exit (whole pairs
  // of groups, the last one after): with an exit after every group the
  // compiler's wait counting also follows paths that never run.  x is
  // requested after the first rows, so its latency (every workgroup reads
  // all of x from L2) and theirs overlap.
  Atom A0[kRPW][NA], A1[kRPW][NA];
  Ent E0[kRPW], E1[kRPW];
  int k = 0;
  __builtin_amdgcn_sched_barrier(0);
  fetch(0, A0, E0);
  __builtin_amdgcn_sched_barrier(0);
  stage_x();
  for (; k + 2 <= n; k += 2) {
    group(k, A0, E0, A1, E1);
    group(k + 1, A1, E1, A0, E0);
  }
  if (k < n) group(k, A0, E0, A1, E1);
}

// Rows per workgroup: the weight's rows spread evenly over one workgroup per
// CU (the LDS tile fills a CU), in multiples of 8, at most kMaxRowsWG.
int rows_per_wg(int64_t out_f) {
  const int cus = device_cus() > 0 ? device_cus() : 256;
  const int64_t per = (out_f + cus - 1) / cus;
  return (int)std::min<int64_t>(kMaxRowsWG, std::max<int64_t>(8, (per + 7) / 8 * 8));
}

}  // namespace rows16
}  // namespace bf16x

using namespace bf16x;

extern "C" int bf16x_gemm_rows(const void* x, int32_t x_dtype, int64_t M, const int32_t* sign, int64_t n_sign,
                               const int32_t* mant, int64_t n_mant, const int32_t* delta, int64_t n_delta,
                               const uint8_t* emax, int64_t n_emax, const uint32_t* tile_off,
                               const uint32_t* tile_ent, int64_t out_f, int64_t in_f, int32_t sub, int32_t mode,
                               void* y, int32_t y_dtype, bf16x_stream_t stream) {
  using namespace bf16x::rows16;
  if (!x || !sign || !mant || !delta || !emax || !y) return BF16X_EARG;
  if (mode != BF16X_EXACT && mode != BF16X_SATURATED) return BF16X_EARG;
  const bool ex = mode == BF16X_EXACT;
  if (ex && (!tile_off || !tile_ent)) return BF16X_EARG;
  if (x_dtype != BF16X_BF16 || (y_dtype != BF16X_BF16 && y_dtype != BF16X_F32)) return BF16X_EDTYPE;
  const int rc = check_dict(out_f, in_f, sub, n_sign, n_mant, n_delta, n_emax);
  if (rc) return rc;
  if (M <= 0 || M > kMaxTokens || (in_f != 2048 && in_f != 4096)) return BF16X_ESHAPE;
  if (out_f * (in_f >> 5) * 28 >= (int64_t)0xFFFFFFFF) return BF16X_ESHAPE;
  if (!aligned4(sign) || !aligned4(mant) || !aligned4(delta) || !aligned2(emax) || !aligned4(x) || !aligned4(y))
    return BF16X_EARG;
  const int rpw = rows_per_wg(out_f);
  const int64_t grid = (out_f + rpw - 1) / rpw;
  const uint32_t *to = ex ? tile_off : nullptr, *te = ex ? tile_ent : nullptr;
  hipStream_t st = (hipStream_t)stream;
#define BF16X_ROWS(NA_, EX_, YF_)                                                                           \
  hipLaunchKernelGGL((gemm_rows_kernel<NA_, EX_, YF_>), dim3((unsigned)grid), dim3(kThreads), 0, st,             \
                     (const uint16_t*)x, (int)M, (const uint32_t*)sign, (const uint32_t*)mant,                 \
                     (const uint32_t*)delta, (const uint16_t*)emax, to, te, (int)out_f, (int)in_f, rpw, y)
#define BF16X_ROWS_NA(NA_)                                                                                  \
  do {                                                                                                      \
    if (ex) { if (y_dtype == BF16X_F32) BF16X_ROWS(NA_, true, true); else BF16X_ROWS(NA_, true, false); }  \
    else { if (y_dtype == BF16X_F32) BF16X_ROWS(NA_, false, true); else BF16X_ROWS(NA_, false, false); }   \
  } while (0)
  if (in_f == 4096) BF16X_ROWS_NA(2);
  else BF16X_ROWS_NA(1);
#undef BF16X_ROWS_NA
#undef BF16X_ROWS
  return launch_status();
}
