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
// decode, in_f % 32 == 0: one wave per row, 64 atoms (2048 elements) per pass
// --------------------------------------------------------------------------
// Lane l decodes atom l of the pass (coalesced stream loads) into a
// wave-private LDS buffer in natural element order (16-byte chunk q of atom a
// at slot (q + a/4) & 3, conflict free for both the per-atom writes and the
// contiguous reads); EXACT then writes the pass's plan entries over it; the
// buffer is read back so that each store instruction writes 1 KB contiguous.
// The plan entries of a row segment are sorted by column: the pass's entries
// are a prefix of the rest of the list, found with a wave ballot.  LDS
// operations of one wave complete in order, so no barrier is needed.
__device__ __forceinline__ int chunk_slot(int a, int q) { return a * 64 + (((q + (a >> 2)) & 3) << 4); }

__device__ __forceinline__ __amdgpu_buffer_rsrc_t dec_rsrc(const void* p, uint64_t bytes) {
  const uint32_t n = bytes > 0xFFFFFFFFull ? 0xFFFFFFFFu : (uint32_t)bytes;
  return __builtin_amdgcn_make_buffer_rsrc((void*)p, (short)0, (int)n, 0x00020000);
}

template <bool EXACT>
__global__ __launch_bounds__(256) void decode_rows_kernel(
    const uint32_t* __restrict__ sign, const uint32_t* __restrict__ mant, const uint32_t* __restrict__ delta,
    const uint16_t* __restrict__ emax2, const uint32_t* __restrict__ tile_off,
    const uint32_t* __restrict__ tile_ent, int64_t out_f, int64_t in_f, int tpr, uint16_t* __restrict__ out) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[4 * 4096];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t row = (int64_t)blockIdx.x * 4 + wave;
  if (row >= out_f) return;
  uint8_t* buf = lds + wave * 4096;
  const int64_t P = in_f >> 5;
  const int passes = (int)((P + 63) >> 6);
  // the streams stay below 4 GiB per buffer descriptor: offsets are taken
  // from the row's first atom
  const uint64_t a_row = (uint64_t)row * P;
  const __amdgpu_buffer_rsrc_t rs_ = dec_rsrc(sign + a_row, (uint64_t)P * 4);
  const __amdgpu_buffer_rsrc_t rm_ = dec_rsrc(mant + a_row * 7, (uint64_t)P * 28);
  const __amdgpu_buffer_rsrc_t rd_ = dec_rsrc(delta + a_row * 3, (uint64_t)P * 12);
  const __amdgpu_buffer_rsrc_t re_ = dec_rsrc(emax2 + a_row, (uint64_t)P * 2);
  auto load = [&](int c, Atom& t) {
    const uint32_t a = (uint32_t)min((int64_t)c * 64 + lane, P - 1);
    const u32x4 m03 = __builtin_amdgcn_raw_buffer_load_b128(rm_, (int)(a * 28), 0, 0);
    const u32x3 m46 = __builtin_amdgcn_raw_buffer_load_b96(rm_, (int)(a * 28 + 16), 0, 0);
    const u32x3 d02 = __builtin_amdgcn_raw_buffer_load_b96(rd_, (int)(a * 12), 0, 0);
    t.s = __builtin_amdgcn_raw_buffer_load_b32(rs_, (int)(a * 4), 0, 0);
    t.e = __builtin_amdgcn_raw_buffer_load_b16(re_, (int)(a * 2), 0, 0);
    const uint32_t c0 = m03.x, c1 = m03.y, c2 = m03.z, c3 = m03.w, c4 = m46.x, c5 = m46.y, c6 = m46.z;
    t.m[0] = c0; t.m[1] = c1; t.m[2] = c2; t.m[3] = c3; t.m[4] = c4; t.m[5] = c5; t.m[6] = c6;
    const uint32_t e0 = d02.x, e1 = d02.y, e2 = d02.z;
    t.d[0] = e0; t.d[1] = e1; t.d[2] = e2;
  };
  uint16_t* orow = out + row * in_f;
  uint32_t ptr = 0, pend = 0;                   // plan entries of the current segment
  Atom cur, nxt;
  load(0, cur);
  for (int c = 0; c < passes; ++c) {
    if (c + 1 < passes) load(c + 1, nxt);
    uint32_t p[16];
    decode_pairs(cur, p);
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
    if constexpr (EXACT) {
      const int64_t seg = col0 / kTileCols;
      const uint32_t cs = (uint32_t)(col0 - seg * kTileCols);   // pass start within the segment
      if (cs == 0) {
        ptr = tile_off[row * tpr + seg];
        pend = tile_off[row * tpr + seg + 1];
      }
      while (true) {
        const uint32_t idx = ptr + lane;
        const uint32_t ent = idx < pend ? tile_ent[idx] : 0xFFFFFFFFu;
        const uint32_t col = ent >> 16;
        const bool in = idx < pend && col < cs + 2048;
        if (in) {
          const int e = (int)(col - cs);
          *(uint16_t*)(buf + chunk_slot(e >> 5, (e & 31) >> 3) + (e & 7) * 2) = (uint16_t)(ent & 0xFFFFu);
        }
        const uint32_t cnt = (uint32_t)__builtin_popcountll(__ballot(in));
        ptr += cnt;
        if (cnt < 64) break;
      }
    }
    const int64_t nvalid = min((int64_t)2048, in_f - col0);        // elements of this pass
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = 8 * lane + 512 * i;
      const u32x4 v = *(const u32x4*)(buf + chunk_slot(e >> 5, (e & 31) >> 3));
      if (e < nvalid) *(u32x4a*)(orow + col0 + e) = v;
    }
    cur = nxt;
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
      aligned16(out) && (in_f >> 5) * 28 < (int64_t)0xFFFFFFFF) {
    const int64_t grid = (out_f + 3) / 4;      // one wave per row
    if (grid > INT32_MAX) return BF16X_ESHAPE;
    if (to)
      hipLaunchKernelGGL(decode_rows_kernel<true>, dim3((unsigned)grid), dim3(256), 0, st, (const uint32_t*)sign,
                         (const uint32_t*)mant, (const uint32_t*)delta, (const uint16_t*)emax, to, tile_ent,
                         out_f, in_f, tpr, out);
    else
      hipLaunchKernelGGL(decode_rows_kernel<false>, dim3((unsigned)grid), dim3(256), 0, st, (const uint32_t*)sign,
                         (const uint32_t*)mant, (const uint32_t*)delta, (const uint16_t*)emax, to, tile_ent,
                         out_f, in_f, tpr, out);
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
