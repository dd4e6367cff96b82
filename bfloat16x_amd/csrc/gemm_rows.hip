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
// Layout.  A workgroup is 8 waves; it walks row groups g = blockIdx.x,
// blockIdx.x + gridDim.x, ... of 8 rows.  For each group, wave w loads,
// decodes and writes row 8g + w into an LDS tile (the EXACT plan entries of
// the row written over it by the same wave), then after a barrier every wave
// multiplies its own K range of the tile: v_mfma_f32_16x16x32_bf16 with
// A = W (MFMA rows 0-7 the group's rows, 8-15 repeat them and are dropped),
// B = x (16 tokens, zero past M).  The 8 partial products of a row group are
// added in wave order through LDS and stored.
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

constexpr int kWaves = 8;                     // rows per group, waves per workgroup
constexpr int kMaxTokens = 16;
constexpr int kRowBytes = 128 * 64 + 16;      // LDS tile row: 128 atoms x 64 bytes + 16 (bank skew)
constexpr int kTileBytes = kWaves * kRowBytes;
constexpr int kRedBytes = kWaves * 32 * 16;   // partial sums: 8 waves x 32 lanes x 4 floats
constexpr int kEntBatches = 2;                // plan entries prefetched per lane per row (64 per batch)

// 16-byte chunk k (0..3) of atom a in an LDS tile row, swizzled by a / 4:
// the 16 lanes of a decode write (16 consecutive atoms, same k) then cover
// all 64 banks.  An MFMA read (8 rows x 4 atoms, same chunk) starts row r,
// atom q at bank 4 (r + 4 q) mod 64 with the 16-byte row skew: every 4-bank
// group is hit exactly twice, the minimum for 32 distinct 16-byte reads.
__device__ __forceinline__ int chunk_off(int a, int k) { return a * 64 + ((k ^ (a >> 2)) & 3) * 16; }

template <int NA, bool EXACT, bool YF32>
__global__ __launch_bounds__(512) void gemm_rows_kernel(const uint16_t* __restrict__ x, int M,
                                                        const uint32_t* __restrict__ sign,
                                                        const uint32_t* __restrict__ mant,
                                                        const uint32_t* __restrict__ delta,
                                                        const uint16_t* __restrict__ emax2,
                                                        const uint32_t* __restrict__ tile_off,
                                                        const uint32_t* __restrict__ tile_ent, int out_f, int in_f,
                                                        void* __restrict__ y) {
  constexpr int P = 64 * NA;                  // atoms per row
  constexpr int S = P / 4;                    // MFMA k-steps per row (128 columns each)
  constexpr int SW = S / kWaves;              // k-steps per wave
  static_assert(SW >= 1 && S % kWaves == 0, "whole k-steps per wave");
  // two decoded tiles, two partial-sum buffers, a slot per lane for masked
  // plan writes: 139,776 bytes
  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * kTileBytes + 2 * kRedBytes + 256];
  uint8_t* const tile = lds;
  float* const red = (float*)(lds + 2 * kTileBytes);
  uint8_t* const trash = lds + 2 * kTileBytes + 2 * kRedBytes;     // 64 lanes x 4 bytes

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, q = lane >> 4;      // MFMA role: row r (mod 8), atom q of a k-step
  const int groups = (out_f + kWaves - 1) / kWaves;

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

  // ---- this wave's row of group g: atoms l, 64 + l through raw buffer loads
  const uint64_t Pl = (uint64_t)(in_f >> 5);
  const __amdgpu_buffer_rsrc_t rs_ = buf_rsrc(sign, (uint64_t)out_f * Pl * 4);
  const __amdgpu_buffer_rsrc_t rm_ = buf_rsrc(mant, (uint64_t)out_f * Pl * 28);
  const __amdgpu_buffer_rsrc_t rd_ = buf_rsrc(delta, (uint64_t)out_f * Pl * 12);
  const __amdgpu_buffer_rsrc_t re_ = buf_rsrc(emax2, (uint64_t)out_f * Pl * 2);
  auto row_of = [&](int g) { return min(g * kWaves + wave, out_f - 1); };
  auto load_row = [&](int g, Atom (&t)[NA]) {
    const uint32_t sa = (uint32_t)(row_of(g) * P);
#pragma unroll
    for (int s = 0; s < NA; ++s) t[s] = load_atom_buf(rs_, rm_, rd_, re_, (uint32_t)(64 * s + lane), sa);
  };
  // plan entries of the row: the first kEntBatches x 64, through a buffer
  // descriptor that spans exactly the row's entries (reads past the row end
  // return 0 and are masked where they are patched; the rest of a long row,
  // rare, is read where it is patched).  The row offsets are wave-uniform
  // scalar loads: waiting for them does not wait for the vector loads of the
  // rows in flight, and the entry reads need no per-row address registers.
  struct Ent {
    uint32_t b0, b1;
    uint32_t e[kEntBatches];
  };
  auto load_ent = [&](int g, Ent& en) {
    const int rr = g * kWaves + wave;
    const int rc = row_of(g);
    const uint32_t o0 = tile_off[rc], o1 = tile_off[rc + 1];
    en.b0 = o0;
    en.b1 = rr < out_f ? o1 : o0;                            // padding row: no entries
    const __amdgpu_buffer_rsrc_t re_row =
        __builtin_amdgcn_make_buffer_rsrc((void*)(tile_ent + o0), (short)0, (int)((en.b1 - o0) * 4u), 0x00020000);
#pragma unroll
    for (int b = 0; b < kEntBatches; ++b)
      en.e[b] = __builtin_amdgcn_raw_buffer_load_b32(re_row, (lane + 64 * b) * 4, 0, 0);
  };
  auto patch_one = [&](uint8_t* myrow, uint32_t e, bool live) {
    const int c = (int)(e >> 16);                           // column (< 4096)
    const int a = c >> 5, j = c & 15, h = (c >> 4) & 1;
    uint8_t* dst = live ? myrow + chunk_off(a, j >> 2) + (j & 3) * 4 + h * 2 : trash + lane * 4;
    *(uint16_t*)dst = (uint16_t)(e & 0xFFFFu);
  };
  // this wave's row of a group (atoms in `cur`) decoded into its tile row,
  // the plan's exact values written over it
  auto decode_into = [&](uint8_t* t, Atom (&cur)[NA], const Ent& ec) {
    uint8_t* const myrow = t + wave * kRowBytes;
#pragma unroll
    for (int s = 0; s < NA; ++s) {
      uint32_t w[16];
      decode_pairs(cur[s], w);
      const int a = 64 * s + lane;
#pragma unroll
      for (int k = 0; k < 4; ++k)
        *(u32x4*)(myrow + chunk_off(a, k)) = u32x4{w[4 * k], w[4 * k + 1], w[4 * k + 2], w[4 * k + 3]};
    }
    if constexpr (EXACT) {
      const uint32_t b0 = ec.b0, b1 = ec.b1;
#pragma unroll
      for (int b = 0; b < kEntBatches; ++b) patch_one(myrow, ec.e[b], b0 + (uint32_t)(lane + 64 * b) < b1);
      for (uint32_t e = b0 + (uint32_t)(lane + 64 * kEntBatches); e < b1; e += 64) patch_one(myrow, tile_ent[e], true);
    }
  };
  // this wave's K range of a decoded tile times x: four independent
  // accumulators (one per MFMA of a k-step), then rows 0-7 of the result
  // (lanes 0-31) to the partial-sum buffer
  auto mma = [&](const uint8_t* t, float* rd) {
    f32x4 acc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    const uint8_t* arow = t + (r & 7) * kRowBytes;
#pragma unroll
    for (int jj = 0; jj < SW; ++jj) {
      const int a = 4 * (wave * SW + jj) + q;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bf16x8_t av = *(const bf16x8_t*)(arow + chunk_off(a, i));
        acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, xb[jj][i], acc[i], 0, 0, 0);
      }
    }
    const f32x4 sum = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    if (lane < 32) {
      const float v0 = sum.x, v1 = sum.y, v2 = sum.z, v3 = sum.w;
      *(f32x4*)(rd + (wave * 32 + lane) * 4) = f32x4{v0, v1, v2, v3};
    }
  };
  // the 8 waves' partials of group g added in wave order and stored
  auto reduce = [&](int g, const float* rd) {
    if (tid < kWaves * kMaxTokens) {
      const int row = tid & 7, t = tid >> 3;                // output (row of the group, token)
      const int ln = 16 * (row >> 2) + t, v = row & 3;
      float sum = rd[ln * 4 + v];
#pragma unroll
      for (int w = 1; w < kWaves; ++w) sum += rd[(w * 32 + ln) * 4 + v];
      const int orow = g * kWaves + row;
      if (t < M && orow < out_f) {
        if constexpr (YF32) ((float*)y)[(int64_t)t * out_f + orow] = sum;
        else ((uint16_t*)y)[(int64_t)t * out_f + orow] = (uint16_t)f32_to_bf16_rne(sum);
      }
    }
  };

  // Groups of this workgroup: g0, g0 + stride, ... (n of them).  Group k is
  // decoded into tile k & 1; in the step that multiplies group k the waves
  // also decode group k + 1 into the other tile (the matrix cores and the
  // decode's VALU work overlap) and request the rows of group k + 2; one
  // barrier per group.  Requests past the workgroup's last group re-read
  // that group's rows (from L2): every path through the loop then has the
  // same loads in flight, and the waits for a group's rows count only theirs.
  const int g0 = blockIdx.x, stride = gridDim.x;
  if (g0 >= groups) return;
  const int n = (groups - 1 - g0) / stride + 1;
  const int glast = g0 + (n - 1) * stride;
  auto fetch = [&](int gg, Atom (&t)[NA], Ent& en) {
    const int gc = min(gg, glast);
    load_row(gc, t);
    if constexpr (EXACT) load_ent(gc, en);
  };
  Atom A0[NA], A1[NA];
  Ent E0{}, E1{};
  uint8_t* const tile0 = tile;
  uint8_t* const tile1 = tile + kTileBytes;
  float* const red0 = red;
  float* const red1 = red + kRedBytes / 4;
  // x is requested after the first rows: the rows' latency and x's (every
  // workgroup reads all of x from L2) overlap.  The scheduling barriers keep
  // the prologue's requests in the loop's order.
  int g = g0, k = 0;
  __builtin_amdgcn_sched_barrier(0);
  fetch(g, A0, E0);
  __builtin_amdgcn_sched_barrier(0);
  stage_x();
  __builtin_amdgcn_sched_barrier(0);
  fetch(g + stride, A1, E1);
  __builtin_amdgcn_sched_barrier(0);
  decode_into(tile0, A0, E0);
  __syncthreads();
  // one exit (whole pairs of groups, the last one after): with an exit after
  // every group the compiler's wait counting also follows paths that never
  // run and waits for the group still ahead
  for (; k + 2 <= n; k += 2) {
    fetch(g + 2 * stride, A0, E0);
    __builtin_amdgcn_sched_barrier(0);
    mma(tile0, red0);
    decode_into(tile1, A1, E1);
    __syncthreads();
    reduce(g, red0);
    g += stride;
    fetch(g + 2 * stride, A1, E1);
    __builtin_amdgcn_sched_barrier(0);
    mma(tile1, red1);
    decode_into(tile0, A0, E0);
    __syncthreads();
    reduce(g, red1);
    g += stride;
  }
  if (k < n) {
    mma(tile0, red0);
    __syncthreads();
    reduce(g, red0);
  }
}

// Workgroups: one per CU (the LDS tile takes ~66 KB; two workgroups of 8
// waves would halve each wave's registers), at most one per row group.
int64_t rows_grid(int64_t groups) {
  const int cus = device_cus();
  return std::min<int64_t>(groups, cus > 0 ? cus : 256);
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
  const int64_t groups = (out_f + kWaves - 1) / kWaves;
  const int64_t grid = rows_grid(groups);
  const uint32_t *to = ex ? tile_off : nullptr, *te = ex ? tile_ent : nullptr;
  hipStream_t st = (hipStream_t)stream;
#define BF16X_ROWS(NA_, EX_, YF_)                                                                           \
  hipLaunchKernelGGL((gemm_rows_kernel<NA_, EX_, YF_>), dim3((unsigned)grid), dim3(512), 0, st,             \
                     (const uint16_t*)x, (int)M, (const uint32_t*)sign, (const uint32_t*)mant,                 \
                     (const uint32_t*)delta, (const uint16_t*)emax, to, te, (int)out_f, (int)in_f, y)
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
