// Packed-dict kernels for gfx950: one-pass decode and the device conversion of the reference's per-row CSR into a plan.
//
//   decode  <- _bf16x_decode_kernel + _bf16x_fix_ovf_kernel
//              (bf16x_triton_test.py:11-77), fix folded into the same launch
//   csr     <- consumer of the CSR built at bf16x_fused.py:165-179
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/bf16x_hip.h"
#include "bf16x_device.h"
#include "launch_common.h"

namespace bf16x {

constexpr int kTileCols = 65536;

// Last tile t in [lo, hi) with off[t] <= e (the tile holding entry e).
__device__ __forceinline__ int64_t tile_of_entry(const uint32_t* __restrict__ off, int64_t lo, int64_t hi,
                                                 uint32_t e) {
  while (hi - lo > 1) {
    const int64_t mid = (lo + hi) >> 1;
    if (off[mid] <= e) lo = mid; else hi = mid;
  }
  return lo;
}

// Write the exact bits of every plan entry of rows [r0, r1) into out.
__device__ __forceinline__ void apply_plan_rows(const uint32_t* __restrict__ tile_off,
                                                const uint32_t* __restrict__ tile_ent, int64_t r0, int64_t r1,
                                                int64_t in_f, int tpr, uint16_t* __restrict__ out) {
  const uint32_t e0 = tile_off[r0 * tpr], e1 = tile_off[r1 * tpr];
  for (uint32_t e = e0 + threadIdx.x; e < e1; e += blockDim.x) {
    const int64_t t = tile_of_entry(tile_off, r0 * tpr, r1 * tpr, e);
    const uint32_t ent = tile_ent[e];
    const int64_t row = t / tpr, seg = t - row * tpr;
    const int64_t col = seg * kTileCols + (ent >> 16);
    if (col < in_f) out[row * in_f + col] = (uint16_t)(ent & 0xFFFFu);  // a bad plan never writes out of range
  }
}

// --------------------------------------------------------------------------
// decode, in_f % 32 == 0: one lane per 32-element atom
// --------------------------------------------------------------------------
__global__ __launch_bounds__(256) void decode_atoms_kernel(
    const uint32_t* __restrict__ sign, const uint32_t* __restrict__ mant, const uint32_t* __restrict__ delta,
    const uint16_t* __restrict__ emax2, const uint32_t* __restrict__ tile_off,
    const uint32_t* __restrict__ tile_ent, int64_t out_f, int64_t in_f, int tpr, int rows_per_block,
    uint16_t* __restrict__ out) {
  const int64_t P = in_f >> 5;
  const int64_t r0 = (int64_t)blockIdx.x * rows_per_block;
  const int64_t r1 = min(out_f, r0 + rows_per_block);
  for (int64_t ga = r0 * P + threadIdx.x; ga < r1 * P; ga += blockDim.x) {
    const Atom t = load_atom(sign, mant, delta, emax2, ga);
    uint32_t p[16];
    decode_pairs(t, p);
    uint32_t lo[8], hi[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      lo[i] = perm(p[2 * i + 1], p[2 * i], 0x05040100u);  // elements 2i, 2i+1
      hi[i] = perm(p[2 * i + 1], p[2 * i], 0x07060302u);  // elements 16+2i, 17+2i
    }
    u32x4a* o = (u32x4a*)(out + 32 * ga);
    o[0] = u32x4a{lo[0], lo[1], lo[2], lo[3]};
    o[1] = u32x4a{lo[4], lo[5], lo[6], lo[7]};
    o[2] = u32x4a{hi[0], hi[1], hi[2], hi[3]};
    o[3] = u32x4a{hi[4], hi[5], hi[6], hi[7]};
  }
  if (tile_off != nullptr) {
    // every saturated store of the block completes before any exact store
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    apply_plan_rows(tile_off, tile_ent, r0, r1, in_f, tpr, out);
  }
}

// --------------------------------------------------------------------------
// decode, any shape: one thread per element (shapes with in_f % 32 != 0)
// --------------------------------------------------------------------------
__device__ __forceinline__ uint32_t field_at(const uint32_t* __restrict__ w, int64_t bit, int nb) {
  const int64_t wi = bit >> 5;
  const uint32_t sh = (uint32_t)(bit & 31);
  const uint32_t lo = w[wi];
  const uint32_t hi = (sh + nb > 32) ? w[wi + 1] : 0u;  // only read when the field crosses
  return alignbit(hi, lo, sh) & ((1u << nb) - 1u);
}

__global__ __launch_bounds__(256) void decode_elems_kernel(
    const uint32_t* __restrict__ sign, const uint32_t* __restrict__ mant, const uint32_t* __restrict__ delta,
    const uint8_t* __restrict__ emax, const uint32_t* __restrict__ tile_off, const uint32_t* __restrict__ tile_ent,
    int64_t out_f, int64_t in_f, int tpr, int rows_per_block, uint16_t* __restrict__ out) {
  const int64_t r0 = (int64_t)blockIdx.x * rows_per_block;
  const int64_t r1 = min(out_f, r0 + rows_per_block);
  for (int64_t i = r0 * in_f + threadIdx.x; i < r1 * in_f; i += blockDim.x) {
    const uint32_t s = field_at(sign, i, 1);
    const uint32_t m = field_at(mant, i * 7, 7);
    const uint32_t d = field_at(delta, i * 3, 3);
    const int e = (int)emax[i >> 4] - (int)d;
    out[i] = (uint16_t)((s << 15) | ((uint32_t)max(e, 0) << 7) | m);
  }
  if (tile_off != nullptr) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    apply_plan_rows(tile_off, tile_ent, r0, r1, in_f, tpr, out);
  }
}

// --------------------------------------------------------------------------
// reference CSR (col, true delta, row offsets) -> plan entries
// --------------------------------------------------------------------------
__global__ __launch_bounds__(256) void plan_from_csr_kernel(
    const int32_t* __restrict__ olk, const int32_t* __restrict__ old, const int32_t* __restrict__ oloff,
    const uint32_t* __restrict__ sign, const uint32_t* __restrict__ mant, const uint8_t* __restrict__ emax,
    int64_t out_f, int64_t in_f, int64_t n_entries, uint32_t* __restrict__ ent, uint8_t* __restrict__ sat) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= out_f) return;
  const int lane = threadIdx.x & 63;
  const int64_t e0 = max(oloff[row], 0), e1 = min((int64_t)oloff[row + 1], n_entries);
  for (int64_t j = e0 + lane; j < e1; j += 64) {
    const int64_t k = min(max((int64_t)olk[j], (int64_t)0), in_f - 1);  // clamp a bad column
    const int td = old[j];
    const int64_t p = row * in_f + k;
    const uint32_t s = field_at(sign, p, 1);
    const uint32_t m = field_at(mant, p * 7, 7);
    const int em = (int)emax[p >> 4];
    const int e = min(max(em - td, 0), 255);  // bf16x_fused.py:103
    ent[j] = ((uint32_t)k << 16) | (s << 15) | ((uint32_t)e << 7) | m;
    sat[j] = (uint8_t)max(em - 7, 0);
  }
}

}  // namespace bf16x

using namespace bf16x;


extern "C" int bf16x_decode(const int32_t* sign, int64_t n_sign, const int32_t* mant, int64_t n_mant,
                            const int32_t* delta, int64_t n_delta, const uint8_t* emax, int64_t n_emax,
                            const uint32_t* tile_off, const uint32_t* tile_ent, int64_t out_f, int64_t in_f,
                            int32_t sub, int32_t mode, uint16_t* out, bf16x_stream_t stream) {
  if (!sign || !mant || !delta || !emax || !out) return BF16X_EARG;
  if (mode != BF16X_EXACT && mode != BF16X_SATURATED) return BF16X_EARG;
  if (mode == BF16X_EXACT && (!tile_off || !tile_ent)) return BF16X_EARG;
  int rc = check_dict(out_f, in_f, sub, n_sign, n_mant, n_delta, n_emax);
  if (rc) return rc;
  const uint32_t* to = (mode == BF16X_EXACT) ? tile_off : nullptr;
  const int tpr = tiles_per_row(in_f);
  hipStream_t st = (hipStream_t)stream;
  if ((in_f & 31) == 0 && aligned4(sign) && aligned4(mant) && aligned4(delta) && aligned2(emax) &&
      aligned4(out)) {
    const int64_t P = in_f >> 5;
    int64_t rpb = std::max<int64_t>(1, 1024 / P);
    while (rpb > 1 && (out_f + rpb - 1) / rpb < 1024) rpb >>= 1;
    const int64_t grid = (out_f + rpb - 1) / rpb;
    if (grid > INT32_MAX) return BF16X_ESHAPE;
    hipLaunchKernelGGL(decode_atoms_kernel, dim3((unsigned)grid), dim3(256), 0, st, (const uint32_t*)sign,
                       (const uint32_t*)mant, (const uint32_t*)delta, (const uint16_t*)emax, to, tile_ent,
                       out_f, in_f, tpr, (int)rpb, out);
  } else {
    int64_t rpb = std::max<int64_t>(1, 8192 / in_f);
    while (rpb > 1 && (out_f + rpb - 1) / rpb < 1024) rpb >>= 1;
    const int64_t grid = (out_f + rpb - 1) / rpb;
    if (grid > INT32_MAX) return BF16X_ESHAPE;
    hipLaunchKernelGGL(decode_elems_kernel, dim3((unsigned)grid), dim3(256), 0, st, (const uint32_t*)sign,
                       (const uint32_t*)mant, (const uint32_t*)delta, emax, to, tile_ent, out_f, in_f, tpr,
                       (int)rpb, out);
  }
  return launch_status();
}

extern "C" int bf16x_plan_from_csr(const int32_t* olk, const int32_t* old, const int32_t* oloff,
                                   const int32_t* sign, const int32_t* mant, const uint8_t* emax, int64_t out_f,
                                   int64_t in_f, int64_t n_entries, uint32_t* tile_ent, uint8_t* tile_sat,
                                   bf16x_stream_t stream) {
  if (!oloff || !sign || !mant || !emax) return BF16X_EARG;
  if (n_entries < 0 || (n_entries > 0 && (!olk || !old || !tile_ent || !tile_sat))) return BF16X_EARG;
  if (out_f <= 0 || in_f <= 0 || in_f > kTileCols) return BF16X_ESHAPE;
  if (n_entries == 0) return BF16X_OK;
  const int64_t grid = (out_f + 3) / 4;
  hipLaunchKernelGGL(plan_from_csr_kernel, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, olk, old,
                     oloff, (const uint32_t*)sign, (const uint32_t*)mant, emax, out_f, in_f, n_entries, tile_ent, tile_sat);
  return launch_status();
}
