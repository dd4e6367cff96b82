// Device encoder: bf16 weight -> packed dict, byte-identical to
// bf16x_quantize (opqk_linear.py:291-324) and to bf16x_encode_host.
//
// A thread owns an atom (the 32 elements 32a .. 32a+31): it loads their
// 64 bytes, takes the emax of each 16-element half (sub = 16, opqk_linear.py
// :305-308; elements past N count as exponent 0), and writes sign word a, mant
// words 7a .. 7a+6, delta words 3a .. 3a+2 (3-bit codes min(delta, 7), :314)
// and emax bytes 2a, 2a+1, each clipped to the reference packer's stream
// length; the words the element padding of pack_bits_stream (:53-64) adds
// past the last atom (a few, for small N) are written as zero.  The overflow
// table (delta >= 7, positions ascending, :311-313) is built in three
// launches: atom masks and per-workgroup counts, one-workgroup scan of the
// counts, then each workgroup ranks its atoms' entries and writes them.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/bf16x_hip.h"
#include "bf16x_device.h"
#include "launch_common.h"

namespace {
using namespace bf16x;

constexpr int kAtomsPerBlock = 256;

struct AtomBits {
  uint32_t w[32];        // bf16 bits of the atom's elements (0 past N)
};

__device__ __forceinline__ void load_atom_bits(const uint16_t* __restrict__ wb, int64_t N, int64_t a, AtomBits& t) {
  const int64_t e0 = a * 32;
  if (e0 + 32 <= N) {
    const u32x4* p = (const u32x4*)(wb + e0);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const u32x4 v = p[c];
      const uint32_t x[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        t.w[8 * c + 2 * k] = x[k] & 0xFFFFu;
        t.w[8 * c + 2 * k + 1] = x[k] >> 16;
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < 32; ++j) t.w[j] = e0 + j < N ? (uint32_t)wb[e0 + j] : 0u;
  }
}

__device__ __forceinline__ void atom_emax(const AtomBits& t, uint32_t& em0, uint32_t& em1) {
  em0 = em1 = 0;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    em0 = max(em0, (t.w[j] >> 7) & 0xFFu);
    em1 = max(em1, (t.w[16 + j] >> 7) & 0xFFu);
  }
}

// streams, emax, overflow mask per atom, overflow count per workgroup
__global__ __launch_bounds__(256) void encode_atoms_kernel(const uint16_t* __restrict__ wb, int64_t N,
                                                           int64_t n_atoms, uint32_t* __restrict__ sign, int64_t ws,
                                                           uint32_t* __restrict__ mant, int64_t wm,
                                                           uint32_t* __restrict__ delta, int64_t wd,
                                                           uint8_t* __restrict__ emax, int64_t n_emax,
                                                           uint32_t* __restrict__ masks,
                                                           uint32_t* __restrict__ blk_cnt) {
  __shared__ uint32_t red[4];
  const int64_t a = (int64_t)blockIdx.x * kAtomsPerBlock + threadIdx.x;
  uint32_t cnt = 0;
  if (a < n_atoms) {
    AtomBits t;
    load_atom_bits(wb, N, a, t);
    uint32_t em0, em1;
    atom_emax(t, em0, em1);
    uint32_t sw = 0, mask = 0;
    uint32_t mw[7] = {0, 0, 0, 0, 0, 0, 0}, dw[3] = {0, 0, 0};
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      const uint32_t b = t.w[j];
      const bool valid = a * 32 + j < N;
      const uint32_t em = j < 16 ? em0 : em1;
      const uint32_t d = em - ((b >> 7) & 0xFFu);
      sw |= (b >> 15) << j;
      if (valid && d >= 7) mask |= 1u << j;
      const int mb = 7 * j, db = 3 * j;                          // compile-time after unrolling
      const uint32_t mv = b & 0x7Fu, dv = valid ? min(d, 7u) : 0u;
      mw[mb >> 5] |= mv << (mb & 31);
      if ((mb & 31) + 7 > 32) mw[(mb >> 5) + 1] |= mv >> (32 - (mb & 31));
      dw[db >> 5] |= dv << (db & 31);
      if ((db & 31) + 3 > 32) dw[(db >> 5) + 1] |= dv >> (32 - (db & 31));
    }
    if (a < ws) sign[a] = sw;
#pragma unroll
    for (int k = 0; k < 7; ++k)
      if (7 * a + k < wm) mant[7 * a + k] = mw[k];
#pragma unroll
    for (int k = 0; k < 3; ++k)
      if (3 * a + k < wd) delta[3 * a + k] = dw[k];
    if (2 * a < n_emax) emax[2 * a] = (uint8_t)em0;
    if (2 * a + 1 < n_emax) emax[2 * a + 1] = (uint8_t)em1;
    if (a == n_atoms - 1) {
      // the packer's element padding can reach past the last atom (N = 5:
      // 34 padded elements, 8 mant words): those words are zero
      for (int64_t k = 7 * n_atoms; k < wm; ++k) mant[k] = 0u;
      for (int64_t k = 3 * n_atoms; k < wd; ++k) delta[k] = 0u;
      for (int64_t k = n_atoms; k < ws; ++k) sign[k] = 0u;
    }
    masks[a] = mask;
    cnt = __builtin_popcount(mask);
  }
  // workgroup total
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) cnt += __shfl_xor(cnt, o, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = cnt;
  __syncthreads();
  if (threadIdx.x == 0) blk_cnt[blockIdx.x] = red[0] + red[1] + red[2] + red[3];
}

// exclusive scan of the workgroup counts (one workgroup; chunks of 1024)
__global__ __launch_bounds__(1024) void encode_scan_kernel(const uint32_t* __restrict__ blk_cnt, int64_t n_blk,
                                                           int64_t* __restrict__ blk_off,
                                                           int64_t* __restrict__ n_ovf) {
  __shared__ int64_t part[16];
  __shared__ int64_t carry_s;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  if (tid == 0) carry_s = 0;
  __syncthreads();
  for (int64_t base = 0; base < n_blk; base += 1024) {
    const int64_t i = base + tid;
    const int64_t v = i < n_blk ? (int64_t)blk_cnt[i] : 0;
    // inclusive wave scan
    int64_t s = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int64_t u = __shfl_up(s, o, 64);
      if (lane >= o) s += u;
    }
    if (lane == 63) part[wv] = s;
    __syncthreads();
    int64_t before = carry_s;
    for (int k = 0; k < wv; ++k) before += part[k];
    if (i < n_blk) blk_off[i] = before + s - v;
    __syncthreads();
    if (tid == 1023) {
      int64_t tot = 0;
      for (int k = 0; k < 16; ++k) tot += part[k];
      carry_s += tot;
    }
    __syncthreads();
  }
  if (tid == 0) n_ovf[0] = carry_s;
}

// table entries: rank within the workgroup, then positions and true deltas
__global__ __launch_bounds__(256) void encode_table_kernel(const uint16_t* __restrict__ wb, int64_t N,
                                                           int64_t n_atoms, const uint32_t* __restrict__ masks,
                                                           const int64_t* __restrict__ blk_off,
                                                           int32_t* __restrict__ ovf_idx,
                                                           uint8_t* __restrict__ ovf_val, int64_t cap) {
  __shared__ uint32_t wsum[4];
  const int64_t a = (int64_t)blockIdx.x * kAtomsPerBlock + threadIdx.x;
  const uint32_t mask = a < n_atoms ? masks[a] : 0u;
  const uint32_t c = __builtin_popcount(mask);
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  uint32_t s = c;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t u = __shfl_up(s, o, 64);
    if (lane >= o) s += u;
  }
  if (lane == 63) wsum[wv] = s;
  __syncthreads();
  uint32_t before = 0;
  for (int k = 0; k < wv; ++k) before += wsum[k];
  if (mask == 0) return;
  int64_t pos = blk_off[blockIdx.x] + before + s - c;
  AtomBits t;
  load_atom_bits(wb, N, a, t);
  uint32_t em0, em1;
  atom_emax(t, em0, em1);
  uint32_t m = mask;
  while (m) {
    const int j = __builtin_ctz(m);
    m &= m - 1;
    uint32_t bj = 0;
#pragma unroll
    for (int k = 0; k < 32; ++k)
      if (k == j) bj = t.w[k];
    const uint32_t d = (j < 16 ? em0 : em1) - ((bj >> 7) & 0xFFu);
    if (pos < cap) {
      ovf_idx[pos] = (int32_t)(a * 32 + j);
      ovf_val[pos] = (uint8_t)d;
    }
    ++pos;
  }
}

int64_t n_atoms_of(int64_t N) { return (N + 31) / 32; }
int64_t n_blocks_of(int64_t N) { return (n_atoms_of(N) + kAtomsPerBlock - 1) / kAtomsPerBlock; }

}  // namespace

extern "C" int64_t bf16x_encode_workspace(int64_t out_f, int64_t in_f) {
  if (out_f <= 0 || in_f <= 0) return -1;
  const int64_t N = out_f * in_f;
  const int64_t nb = n_blocks_of(N);
  // masks [atoms] u32, counts [blocks] u32 (padded to 8 bytes), offsets [blocks] i64, 256-byte aligned
  const int64_t b1 = ((n_atoms_of(N) * 4 + 255) / 256) * 256;
  const int64_t b2 = ((nb * 4 + 255) / 256) * 256;
  return b1 + b2 + nb * 8;
}

extern "C" int bf16x_encode(const uint16_t* w_bits, int64_t out_f, int64_t in_f, int32_t sub, int32_t* sign,
                            int64_t n_sign, int32_t* mant, int64_t n_mant, int32_t* delta, int64_t n_delta,
                            uint8_t* emax, int64_t n_emax, int32_t* ovf_idx, uint8_t* ovf_val, int64_t ovf_cap,
                            int64_t* n_ovf, void* workspace, int64_t workspace_bytes, bf16x_stream_t stream) {
  if (!w_bits || !sign || !mant || !delta || !emax || !n_ovf || !workspace) return BF16X_EARG;
  if (ovf_cap < 0 || (ovf_cap > 0 && (!ovf_idx || !ovf_val))) return BF16X_EARG;
  if (out_f <= 0 || in_f <= 0) return BF16X_ESHAPE;
  if (sub != 16) return BF16X_ESUB;
  const int64_t N = out_f * in_f;
  if (N > (int64_t)INT32_MAX) return BF16X_ESHAPE;           // the table stores int32 positions
  const int64_t ws = bf16x_stream_words(N, 1), wm = bf16x_stream_words(N, 7), wd = bf16x_stream_words(N, 3);
  const int64_t ne = (N + 15) / 16;
  if (n_sign < ws || n_mant < wm || n_delta < wd || n_emax < ne) return BF16X_ESTREAM_LEN;
  if (workspace_bytes < bf16x_encode_workspace(out_f, in_f)) return BF16X_ECAPACITY;
  if (!aligned16(w_bits) || !aligned16(workspace) || !aligned4(sign) || !aligned4(mant) || !aligned4(delta) ||
      ((uintptr_t)n_ovf & 7u) || !aligned4(ovf_idx))
    return BF16X_EARG;
  const int64_t na = n_atoms_of(N), nb = n_blocks_of(N);
  if (nb > INT32_MAX) return BF16X_ESHAPE;
  uint32_t* masks = (uint32_t*)workspace;
  uint32_t* cnt = (uint32_t*)((char*)workspace + ((na * 4 + 255) / 256) * 256);
  int64_t* off = (int64_t*)((char*)cnt + ((nb * 4 + 255) / 256) * 256);
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(encode_atoms_kernel, dim3((unsigned)nb), dim3(256), 0, st, w_bits, N, na, (uint32_t*)sign, ws,
                     (uint32_t*)mant, wm, (uint32_t*)delta, wd, emax, ne, masks, cnt);
  int rc = launch_status();
  if (rc) return rc;
  hipLaunchKernelGGL(encode_scan_kernel, dim3(1), dim3(1024), 0, st, cnt, nb, off, n_ovf);
  rc = launch_status();
  if (rc) return rc;
  hipLaunchKernelGGL(encode_table_kernel, dim3((unsigned)nb), dim3(256), 0, st, w_bits, N, na, masks, off, ovf_idx,
                     ovf_val, ovf_cap);
  return launch_status();
}
