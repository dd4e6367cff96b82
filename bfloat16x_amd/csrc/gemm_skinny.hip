// Fused decode + GEMM for few activation rows (M <= 128): the decoded weight
// is the MFMA A operand straight from registers.
//
// Same contract as the tiled kernel in gemm.hip (bf16x_gemm_fused.py:31-114):
// y[M, N] = x[M, K] . W[N, K]^T, fp32 accumulation.
//
// With few rows of x the product is bound by reading and decoding W, like the
// GEMV.  Each wave owns 32 consecutive W rows and a contiguous range of K
// steps of 64 columns.  Per step, lane l decodes atom (2*step + l/32) of row
// l%32 (one atom = 32 elements, loaded as 1 + 7 + 3 dwords + the emax dword),
// so the wave holds a 32 x 64 W tile in registers with no LDS round trip and
// no barrier.  v_mfma_f32_32x32x16_bf16 consumes it as the A operand in four
// k-groups of 8 consecutive elements per lane (A[i][8h + v] = W[row i][k]
// with h = l/32), the B operand is x: lane l loads 16 bytes of x row
// (32c + l%32) at the same k, for each 32-row block c of x.  D register v of
// lane l is y[32c + l%32][row 8(v/4) + 4(l/32) + v%4].
//
// EXACT: the wave's overflow entries for one step are exactly one run of the
// step-major plan (64-column step, 32-row group); lane t holds entries t and
// t + 64 (loaded one step ahead).  The decoded tile goes through a
// wave-private LDS scratch (natural order, 16-byte chunks rotated per lane
// for conflict-free access), the entries are written over it, and the
// operands are read back; LDS operations of one wave complete in order, so no
// barrier is needed.
//
// The waves of a block split K; their accumulators are summed through LDS in
// wave order and the block writes y (coalesced along N).
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>

#include "../../include/bf16x_hip.h"
#include "bf16x_device.h"
#include "launch_common.h"

namespace bf16x {
namespace skinny {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kGroupRows = 32;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, uint64_t bytes) {
  const uint32_t n = bytes > 0xFFFFFFFFull ? 0xFFFFFFFFu : (uint32_t)bytes;
  return __builtin_amdgcn_make_buffer_rsrc((void*)p, (short)0, (int)n, 0x00020000);
}

struct WAtom {
  uint32_t s, m[7], d[3], ew;
};

struct XOps {
  u32x4 g[4];
};

// scratch chunk c of lane l: 16-byte slot ((c + l/4) & 3) of the lane's 64 bytes
__device__ __forceinline__ int scratch_off(int l, int c) { return l * 64 + (((c + (l >> 2)) & 3) << 4); }

template <int NC, int WAVES, bool EXACT, bool YF32>
__global__ __launch_bounds__(64 * WAVES) void gemm_skinny_kernel(
    const uint16_t* __restrict__ x, int64_t M, const uint32_t* __restrict__ sign,
    const uint32_t* __restrict__ mant, const uint32_t* __restrict__ delta, const uint16_t* __restrict__ emax2,
    const uint32_t* __restrict__ kp_off, const uint32_t* __restrict__ kp_ent, int64_t out_f, int64_t in_f,
    void* __restrict__ y) {
  constexpr int SCR = 4096 + 128;                 // patch scratch per wave + one trash slot per lane
  constexpr int RED = NC * 32 * 33 * 4;           // reduction slab per wave (padded rows)
  constexpr int PER_WAVE = SCR > RED ? SCR : RED;
  __shared__ __attribute__((aligned(16))) uint8_t lds[WAVES * PER_WAVE];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t P = in_f >> 5;
  const int S = (int)(in_f >> 6);
  const int G = (int)((out_f + kGroupRows - 1) / kGroupRows);

  // XCD-aware order of the row groups: consecutive groups on one XCD
  const int nb = (int)gridDim.x, b = (int)blockIdx.x;
  const int per = nb / 8, extra = nb - per * 8;
  const int g = nb >= 8 ? ((b & 7) * per + min(b & 7, extra) + (b >> 3)) : b;
  const int64_t n0 = (int64_t)g * kGroupRows;

  // this wave's K steps
  const int sps = (S + WAVES - 1) / WAVES;
  const int s0 = wave * sps;
  const int n = max(0, min(sps, S - s0));

  // ---- W atoms: lane -> (row l%32, atom parity l/32); vector offsets are loop
  // invariant, the step is a uniform scalar offset
  const int hrow = lane & 31, half = lane >> 5;
  const int64_t wrow = min(n0 + hrow, out_f - 1);
  const __amdgpu_buffer_rsrc_t rs_ = rsrc(sign, (uint64_t)out_f * P * 4);
  const __amdgpu_buffer_rsrc_t rm_ = rsrc(mant, (uint64_t)out_f * P * 28);
  const __amdgpu_buffer_rsrc_t rd_ = rsrc(delta, (uint64_t)out_f * P * 12);
  const __amdgpu_buffer_rsrc_t re_ = rsrc(emax2, (uint64_t)out_f * P * 2);
  const uint32_t av = (uint32_t)(wrow * P) + (uint32_t)half;
  const uint32_t vo_m = av * 28, vo_d = av * 12, vo_s = av * 4, vo_e = (av - (uint32_t)half) * 2;
  auto load_w = [&](int j, WAtom& t) {
    const uint32_t sa = 2u * (uint32_t)(s0 + min(j, n - 1));
    const u32x4 m03 = __builtin_amdgcn_raw_buffer_load_b128(rm_, (int)vo_m, (int)(sa * 28), 0);
    const u32x3 m46 = __builtin_amdgcn_raw_buffer_load_b96(rm_, (int)(vo_m + 16), (int)(sa * 28), 0);
    const u32x3 d02 = __builtin_amdgcn_raw_buffer_load_b96(rd_, (int)vo_d, (int)(sa * 12), 0);
    t.s = __builtin_amdgcn_raw_buffer_load_b32(rs_, (int)vo_s, (int)(sa * 4), 0);
    t.ew = __builtin_amdgcn_raw_buffer_load_b32(re_, (int)vo_e, (int)(sa * 2), 0);
    const uint32_t c0 = m03.x, c1 = m03.y, c2 = m03.z, c3 = m03.w, c4 = m46.x, c5 = m46.y, c6 = m46.z;
    t.m[0] = c0; t.m[1] = c1; t.m[2] = c2; t.m[3] = c3; t.m[4] = c4; t.m[5] = c5; t.m[6] = c6;
    const uint32_t e0 = d02.x, e1 = d02.y, e2 = d02.z;
    t.d[0] = e0; t.d[1] = e1; t.d[2] = e2;
  };

  // ---- x operands: lane l reads 64 bytes of x row (32c + l%32) at k = 64 step + 32 half
  const uint64_t x_bytes = (uint64_t)M * in_f * 2;
  const __amdgpu_buffer_rsrc_t rx_ = rsrc(x, x_bytes);
  uint32_t vx[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int64_t xr = min((int64_t)(32 * c + hrow), M - 1);
    vx[c] = (uint32_t)((xr * in_f + 32 * half) * 2);
  }
  auto load_x = [&](int j, XOps (&xo)[NC]) {
    const uint32_t ks = (uint32_t)(s0 + min(j, n - 1)) * 128u;
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        xo[c].g[q] = __builtin_amdgcn_raw_buffer_load_b128(rx_, (int)(vx[c] + 16 * q), (int)ks, 0);
  };

  // ---- step-major plan run of (step, this group): entries lane, lane + 64
  const __amdgpu_buffer_rsrc_t roff = rsrc(kp_off, ((uint64_t)S * 2 * G + 1) * 4);
  uint32_t kp_total = 0;
  if constexpr (EXACT) kp_total = kp_off[(int64_t)S * 2 * G];
  const __amdgpu_buffer_rsrc_t rent = rsrc(kp_ent, (uint64_t)kp_total * 4);
  // run bounds are read two steps before the entries, the entries two steps
  // before their use, all with vector loads issued in consumption order
  struct Bounds { uint32_t bb, be; };
  struct Run { uint32_t beg, end, e0, e1; };
  auto load_bounds = [&](int j, Bounds& bd) {
    const int s = s0 + min(j, n - 1);
    bd.bb = __builtin_amdgcn_raw_buffer_load_b32(roff, (s * 2 * G + 2 * g) * 4, 0, 0);       // 16-row groups
    bd.be = __builtin_amdgcn_raw_buffer_load_b32(roff, (s * 2 * G + 2 * g + 2) * 4, 0, 0);   // 2g and 2g + 1
  };
  auto load_run = [&](const Bounds& bd, Run& r) {
    r.beg = __builtin_amdgcn_readfirstlane(bd.bb);
    r.end = __builtin_amdgcn_readfirstlane(bd.be);
    r.e0 = __builtin_amdgcn_raw_buffer_load_b32(rent, (int)((r.beg + lane) * 4), 0, 0);
    r.e1 = __builtin_amdgcn_raw_buffer_load_b32(rent, (int)((r.beg + lane + 64) * 4), 0, 0);
  };
  uint8_t* scr = lds + wave * PER_WAVE;
  // Entries past the run's end go to this lane's trash slot: the store is
  // unconditional, so the entry is not first used under a divergent branch
  // (which would make the compiler wait for every outstanding load).
  auto patch_one = [&](uint32_t e, bool live) {
    const int r = (int)(e >> 22) & 31, c = (int)(e >> 16) & 63;
    const int owner = r + 32 * (c >> 5), el = c & 31;
    const int off = live ? scratch_off(owner, el >> 3) + (el & 7) * 2 : 4096 + 2 * lane;
    *(uint16_t*)(scr + off) = (uint16_t)(e & 0xFFFFu);
  };

  f32x16 acc[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[c][v] = 0.f;

  // one step: decode, (patch), 4 k-groups x NC column blocks of MFMA
  auto compute = [&](const WAtom& w, const XOps (&xo)[NC], const Run& R) {
    Atom t;
    t.s = w.s;
#pragma unroll
    for (int i = 0; i < 7; ++i) t.m[i] = w.m[i];
#pragma unroll
    for (int i = 0; i < 3; ++i) t.d[i] = w.d[i];
    t.e = (uint16_t)(w.ew >> (16 * half));
    uint32_t p[16];
    decode_pairs(t, p);
    u32x4 a[4];                                   // natural order: a[q] = elements 8q .. 8q+7
#pragma unroll
    for (int q = 0; q < 2; ++q) {            // pairs 8q .. 8q+7 hold elements 8q.. (low) and 16+8q.. (high)
      a[q] = u32x4{perm(p[8 * q + 1], p[8 * q], 0x05040100u), perm(p[8 * q + 3], p[8 * q + 2], 0x05040100u),
                   perm(p[8 * q + 5], p[8 * q + 4], 0x05040100u), perm(p[8 * q + 7], p[8 * q + 6], 0x05040100u)};
      a[q + 2] = u32x4{perm(p[8 * q + 1], p[8 * q], 0x07060302u), perm(p[8 * q + 3], p[8 * q + 2], 0x07060302u),
                       perm(p[8 * q + 5], p[8 * q + 4], 0x07060302u), perm(p[8 * q + 7], p[8 * q + 6], 0x07060302u)};
    }
    if constexpr (EXACT) {
#pragma unroll
      for (int q = 0; q < 4; ++q) *(u32x4*)(scr + scratch_off(lane, q)) = a[q];
      patch_one(R.e0, R.beg + lane < R.end);
      patch_one(R.e1, R.beg + lane + 64 < R.end);
      for (uint32_t e = R.beg + 128 + lane; e < R.end; e += 64) patch_one(kp_ent[e], true);   // dense runs (rare)
#pragma unroll
      for (int q = 0; q < 4; ++q) a[q] = *(const u32x4*)(scr + scratch_off(lane, q));
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      bf16x8_t av8;
      __builtin_memcpy(&av8, &a[q], 16);
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        bf16x8_t bv8;
        __builtin_memcpy(&bv8, &xo[c].g[q], 16);
        acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av8, bv8, acc[c], 0, 0, 0);
      }
    }
  };

  if (n > 0) {
    // two steps in flight (ping-pong registers), issued in consumption order
    WAtom A, B;
    XOps xa[NC], xb[NC];
    Run ra{}, rb{};
    Bounds ba{}, bb{};
    if constexpr (EXACT) {
      load_bounds(0, ba);
      load_bounds(1, bb);
      load_run(ba, ra);
      load_run(bb, rb);
      load_bounds(2, ba);
      load_bounds(3, bb);
    }
    __builtin_amdgcn_sched_barrier(0);
    load_x(0, xa);
    load_w(0, A);
    __builtin_amdgcn_sched_barrier(0);
    load_x(1, xb);
    load_w(1, B);
    __builtin_amdgcn_sched_barrier(0);
    int j = 0;
    for (; j + 1 < n; j += 2) {
      compute(A, xa, ra);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (EXACT) {
        load_run(ba, ra);              // step j + 2
        load_bounds(j + 4, ba);
      }
      load_x(j + 2, xa);
      load_w(j + 2, A);
      __builtin_amdgcn_sched_barrier(0);
      compute(B, xb, rb);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (EXACT) {
        load_run(bb, rb);              // step j + 3
        load_bounds(j + 5, bb);
      }
      load_x(j + 3, xb);
      load_w(j + 3, B);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (j < n) compute(A, xa, ra);
  }

  // ---- reduce over the waves: slab [wave][x row j][W row i] (33-float rows)
  __syncthreads();
  float* red = (float*)lds;
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int i = 8 * (v >> 2) + 4 * half + (v & 3);
      const int jx = 32 * c + hrow;
      red[(wave * NC * 32 + jx) * 33 + i] = acc[c][v];
    }
  __syncthreads();
  for (int o = threadIdx.x; o < NC * 32 * 32; o += 64 * WAVES) {
    const int jx = o >> 5, i = o & 31;
    const int64_t row = n0 + i;
    if (jx >= M || row >= out_f) continue;
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) s += red[(w * NC * 32 + jx) * 33 + i];
    if constexpr (YF32) ((float*)y)[jx * out_f + row] = s;
    else ((uint16_t*)y)[jx * out_f + row] = (uint16_t)f32_to_bf16_rne(s);
  }
}

}  // namespace skinny
}  // namespace bf16x

// Launcher used by bf16x_gemm for M <= 128 (declared in gemm.hip).
int bf16x_gemm_skinny_launch(const uint16_t* x, int64_t M, const uint32_t* s, const uint32_t* m, const uint32_t* d,
                             const uint16_t* e, const uint32_t* kp_off, const uint32_t* kp_ent, int64_t out_f,
                             int64_t in_f, bool exact, bool yf32, void* y, hipStream_t st) {
  using namespace bf16x::skinny;
  const int64_t G = (out_f + kGroupRows - 1) / kGroupRows;
  if (G > INT32_MAX) return BF16X_ESHAPE;
  // waves per block (K split): enough resident waves to stream W
  int waves = G >= 512 ? 4 : (G >= 256 ? 8 : 16);
  if (const int64_t t = tuning(BF16X_TUNE_SKINNY_WAVES); t > 0) waves = (int)t;
  const int nc = M <= 32 ? 1 : (M <= 64 ? 2 : 4);
  // register budget: 16 waves per block leave 128 VGPRs per lane (one column
  // block), 8 waves 256 (two); four column blocks run 4 waves per block
  if (nc == 2 && waves > 8) waves = 8;
  if (nc == 4) waves = 4;
#define BF16X_SK(NC_, W_)                                                                                      \
  do {                                                                                                       \
    if (exact) {                                                                                             \
      if (yf32) hipLaunchKernelGGL((gemm_skinny_kernel<NC_, W_, true, true>), dim3((unsigned)G), dim3(64 * W_), 0, st, \
                                   x, M, s, m, d, e, kp_off, kp_ent, out_f, in_f, y);                         \
      else hipLaunchKernelGGL((gemm_skinny_kernel<NC_, W_, true, false>), dim3((unsigned)G), dim3(64 * W_), 0, st, x, \
                              M, s, m, d, e, kp_off, kp_ent, out_f, in_f, y);                                 \
    } else {                                                                                                 \
      if (yf32) hipLaunchKernelGGL((gemm_skinny_kernel<NC_, W_, false, true>), dim3((unsigned)G), dim3(64 * W_), 0, \
                                   st, x, M, s, m, d, e, kp_off, kp_ent, out_f, in_f, y);                     \
      else hipLaunchKernelGGL((gemm_skinny_kernel<NC_, W_, false, false>), dim3((unsigned)G), dim3(64 * W_), 0, st, \
                              x, M, s, m, d, e, kp_off, kp_ent, out_f, in_f, y);                              \
    }                                                                                                        \
  } while (0)
#define BF16X_SK_W(NC_, W16_)                    \
  do {                                           \
    switch (waves) {                             \
      case 4: BF16X_SK(NC_, 4); break;           \
      case 8: BF16X_SK(NC_, 8); break;           \
      case 16: BF16X_SK(NC_, W16_); break;       \
      default: return BF16X_EARG;                \
    }                                            \
  } while (0)
  switch (nc) {
    case 1: BF16X_SK_W(1, 16); break;
    case 2: BF16X_SK_W(2, 8); break;
    default: BF16X_SK(4, 4); break;
  }
#undef BF16X_SK_W
#undef BF16X_SK
  return BF16X_OK;
}
