// Fused decode + GEMM for few activation rows (M <= 64) with v_mfma_f32_16x16x32_bf16.
//
// y[M, N] = x[M, K] . W[N, K]^T, fp32 accumulation (bf16x_gemm_fused.py:31-114 contract;
// EXACT applies the step-major overflow plan).
//
// Load pattern.  A wave owns 16 W rows; per step of 128 columns lane l loads
// and decodes atom 4s + (l % 4) of row l / 4, so each quad of lanes reads one
// row's 4 consecutive atoms (112 contiguous mantissa bytes): the texture unit
// serves a quad from one or two cache lines, as for a row-contiguous read.
// The MFMA wants lane l to hold row l % 16 (below), so the decoded words are
// exchanged through a wave-private LDS scratch: written in load order, read
// back in MFMA order (LDS operations of one wave complete in issue order).
// In EXACT mode the step's two plan runs (64-column steps of the wave's
// 16-row group) are written over the scratch in between.
//
// k order.  MFMA i (i < 4) takes pair words 4i .. 4i+3 of atom q = l / 16 of
// row r = l % 16 as lane l's A fragment: an MFMA sums over its 32 k values in
// any order, so with A's k index kk = 8q + 2c + h standing for element
// 4i + c + 16h of atom q, B must hold x at the same elements.  x is therefore
// first rewritten in the decoder's pair order (word 16a + j = x[32a + j] |
// x[32a + 16 + j] << 16), and B's fragment for MFMA i is words 16q + 4i .. +3
// of the token's step row: the pairs are never unpermuted.
//
// Tiles.  A workgroup is 4 waves = 64 W rows and one K split of `sps` steps;
// the x tile of a step (MP tokens x 128 columns) is loaded once per
// workgroup into LDS (double buffered, one barrier per step) and read by the
// four waves.  Loads are issued in the order they are consumed: step j
// issues the plan entries of step j+1, the plan bounds of j+2, the atoms of
// j+kDepth (a ring of kDepth atom registers) and x of j+3 (ping-pong).  With K
// split over workgroups the fp32 partials go to the workspace and a second
// launch sums them in split order.
//
// Operand layout of v_mfma_f32_16x16x32_bf16 (lane l): A[l%16][8(l/16)+v'],
// B[8(l/16)+v'][l%16] (v' < 8), D register v = D[4(l/16)+v][l%16]; the GPU
// tests check the product against the plain one.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>

#include <algorithm>

#include "../../include/bf16x_hip.h"
#include "bf16x_device.h"
#include "launch_common.h"

namespace bf16x {
namespace skinny2 {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kStep = 128;                 // columns per step (4 atoms per row)
constexpr int kRowsWave = 16;
constexpr int kWaves = 4;
constexpr int kRowsBlock = kRowsWave * kWaves;
constexpr int kGroupRows = 32;             // G counts groups of 32 rows; the plan has 2 G groups of 16
constexpr int kXStride = 272;              // bytes per token row of the LDS x tile (256 + 16: bank skew)
constexpr int kScratch = 64 * 64 + 64 * 4; // per-wave patch scratch + one trash word per lane
constexpr int kMaxRows = 64;               // activation rows served

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, uint64_t bytes) {
  const uint32_t n = bytes > 0xFFFFFFFFull ? 0xFFFFFFFFu : (uint32_t)bytes;
  return __builtin_amdgcn_make_buffer_rsrc((void*)p, (short)0, (int)n, 0x00020000);
}

struct WAtom {
  uint32_t s, m[7], d[3];
  uint32_t ew;     // dword holding this atom's emax pair (and its neighbour's)
};
struct Bounds { uint32_t b0, e0, b1, e1; };
struct Ents { uint32_t v[2]; };

// KQ waves share each 16-row group and take consecutive 128-column steps of
// it (a workgroup step is KQ steps): the KQ load instructions that read a
// row's adjacent segments are issued together, so the L1 fetches each cache
// line once for all of them (requests to a line already in flight are
// merged) instead of once per step.  The KQ partial sums of a row group are
// added in wave order at the end.
template <int NC, int KQ, bool EXACT, bool PARTIAL, bool YF32>
__global__ __launch_bounds__(256 * KQ) void gemm_skinny2_kernel(
    const uint16_t* __restrict__ x, int64_t M, const uint32_t* __restrict__ sign,
    const uint32_t* __restrict__ mant, const uint32_t* __restrict__ delta, const uint16_t* __restrict__ emax2,
    const uint32_t* __restrict__ kp_off, const uint32_t* __restrict__ kp_ent, int64_t out_f, int64_t in_f,
    int sps, void* __restrict__ out) {
  constexpr int D = KQ == 1 ? 4 : 2;               // workgroup steps of W atoms in flight (even)
  constexpr int NT = 256 * KQ;                     // threads
  constexpr int MP = NC * 16;                      // tokens padded to whole MFMA blocks
  constexpr int XROW = 256 * KQ + 16;              // bytes per token row of the LDS x tile (+16: bank skew)
  constexpr int XBUF = MP * XROW;
  constexpr int XC = 16 * KQ;                      // 16-byte x chunks per token row
  constexpr int XI = (MP * XC + NT - 1) / NT;      // x chunks per thread per workgroup step
  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * XBUF + kWaves * KQ * kScratch];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wg = wave / KQ, kq = wave - (wave / KQ) * KQ;     // row group, step within the workgroup step
  const int64_t P = in_f >> 5;
  const int S = (int)(in_f / kStep);
  const int G = (int)((out_f + kGroupRows - 1) / kGroupRows);
  const int nb_rows = (int)((out_f + kRowsBlock - 1) / kRowsBlock);
  const int tile = (int)blockIdx.x % nb_rows, split = (int)blockIdx.x / nb_rows;
  const int s0 = split * sps;
  const int n = max(0, min(sps, S - s0));                     // steps of this workgroup
  const int nm = (n + KQ - 1) / KQ;                           // workgroup steps
  const int last = max(n - 1, 0);
  const int64_t n0w = (int64_t)tile * kRowsBlock + wg * kRowsWave;      // this wave's first row
  const int r = lane & 15, q = lane >> 4;          // MFMA role: row r, atom q of the step
  const int rl = lane >> 2, ql = lane & 3;         // load role: row rl, atom ql of the step
  // step (within the split) of this wave at workgroup step m, clamped into it
  auto wstep = [&](int m) { return min(m * KQ + kq, last); };

  // ---- W atoms: lane -> (row n0w + rl, atom 4 s + ql); the step enters as a
  // uniform scalar offset
  const int64_t wrow = min(n0w + rl, out_f - 1);
  const __amdgpu_buffer_rsrc_t rs_ = rsrc(sign, (uint64_t)out_f * P * 4);
  const __amdgpu_buffer_rsrc_t rm_ = rsrc(mant, (uint64_t)out_f * P * 28);
  const __amdgpu_buffer_rsrc_t rd_ = rsrc(delta, (uint64_t)out_f * P * 12);
  const __amdgpu_buffer_rsrc_t re_ = rsrc(emax2, (uint64_t)out_f * P * 2);
  const uint32_t av = (uint32_t)(wrow * P) + (uint32_t)ql;
  const uint32_t vo_m = av * 28, vo_d = av * 12, vo_s = av * 4, vo_e = (av & ~1u) * 2;
  const uint32_t esh = 16u * (av & 1u);            // P % 4 == 0: the parity of the atom index is step-invariant
  auto load_w = [&](int m, WAtom& t) {
    const uint32_t sa = 4u * (uint32_t)(s0 + wstep(m));
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

  // ---- x tile of a workgroup step (KQ steps) in pair order: chunk c = i * NT
  // + tid is (token c / XC, pair words 4 (c % 4) .. +3 of atom c % XC / 4),
  // made from the 4 elements at 32a + 4 (c % 4) and the 4 elements 16 further.
  // The tile starts at the workgroup step's first step; its steps past the
  // split are not multiplied (their columns may lie past the row: buffer
  // reads past x return 0, other reads stay inside x).
  const __amdgpu_buffer_rsrc_t rx_ = rsrc(x, (uint64_t)M * in_f * 2);
  uint32_t vx[XI];
  int xs_off[XI];
#pragma unroll
  for (int i = 0; i < XI; ++i) {
    const int c = i * NT + tid;
    const int tok = min(c / XC, MP - 1);
    const int64_t tg = min((int64_t)tok, M - 1);
    const int cr = c % XC;
    vx[i] = (uint32_t)(tg * in_f * 2 + (cr >> 2) * 64 + (cr & 3) * 8);
    xs_off[i] = tok * XROW + cr * 16;
  }
  struct XRaw { u32x2a lo, hi; };
  auto load_x = [&](int m, XRaw (&xr)[XI]) {
    const uint32_t ks = (uint32_t)(s0 + min(m * KQ, last)) * (kStep * 2);
#pragma unroll
    for (int i = 0; i < XI; ++i) {
      const u32x2 a = __builtin_amdgcn_raw_buffer_load_b64(rx_, (int)vx[i], (int)ks, 0);
      const u32x2 b = __builtin_amdgcn_raw_buffer_load_b64(rx_, (int)(vx[i] + 32), (int)ks, 0);
      const uint32_t a0 = a.x, a1 = a.y, b0 = b.x, b1 = b.y;
      xr[i].lo = u32x2a{a0, a1};
      xr[i].hi = u32x2a{b0, b1};
    }
  };
  auto store_x = [&](const XRaw (&xr)[XI], uint8_t* xb) {
#pragma unroll
    for (int i = 0; i < XI; ++i) {
      if (i * NT + tid < MP * XC) {
        const uint32_t l0 = xr[i].lo.x, l1 = xr[i].lo.y, h0 = xr[i].hi.x, h1 = xr[i].hi.y;
        *(u32x4*)(xb + xs_off[i]) = u32x4{perm(h0, l0, 0x05040100u), perm(h0, l0, 0x07060302u),
                                          perm(h1, l1, 0x05040100u), perm(h1, l1, 0x07060302u)};
      }
    }
  };

  // ---- plan: runs (2 s, h) and (2 s + 1, h) of this wave's step s and
  // 16-row group h: exactly this wave's rows
  const int G2 = 2 * G, h16 = (int)(n0w / kRowsWave);
  uint32_t kp_total = 0;
  if constexpr (EXACT) kp_total = kp_off[(int64_t)2 * S * G2];
  const __amdgpu_buffer_rsrc_t roff = rsrc(kp_off, ((uint64_t)2 * S * G2 + 1) * 4);
  const __amdgpu_buffer_rsrc_t rent = rsrc(kp_ent, (uint64_t)kp_total * 4);
  auto load_bounds = [&](int m, Bounds& b) {
    const int s = s0 + wstep(m);
    const int o0 = ((2 * s) * G2 + h16) * 4, o1 = ((2 * s + 1) * G2 + h16) * 4;
    b.b0 = __builtin_amdgcn_raw_buffer_load_b32(roff, o0, 0, 0);
    b.e0 = __builtin_amdgcn_raw_buffer_load_b32(roff, o0 + 4, 0, 0);
    b.b1 = __builtin_amdgcn_raw_buffer_load_b32(roff, o1, 0, 0);
    b.e1 = __builtin_amdgcn_raw_buffer_load_b32(roff, o1 + 4, 0, 0);
  };
  // entry `lane` of each run (reads past the plan return 0)
  auto load_ents = [&](const Bounds& b, Ents& en) {
    const uint32_t b0 = __builtin_amdgcn_readfirstlane(b.b0), b1 = __builtin_amdgcn_readfirstlane(b.b1);
    en.v[0] = __builtin_amdgcn_raw_buffer_load_b32(rent, (int)((b0 + (uint32_t)lane) * 4), 0, 0);
    en.v[1] = __builtin_amdgcn_raw_buffer_load_b32(rent, (int)((b1 + (uint32_t)lane) * 4), 0, 0);
  };
  // ---- scratch: slot t = row + 16 * atom (the MFMA lane of that row and
  // atom) holds the 16 pair words in four 16-byte chunks; chunk k sits at
  // position k ^ (t / 4 % 4) ^ (t / 16), so that the 16 lanes an LDS cycle
  // serves for a 16-byte access hit 16 different 16-byte bank groups both
  // when written in load order (slots r + 16 * {0..3} of four rows) and when
  // read in MFMA order (16 consecutive slots)
  uint8_t* scr = lds + 2 * XBUF + wave * kScratch;
  uint8_t* trash = scr + 64 * 64 + lane * 4;
  auto chunk = [&](int t, int k) { return scr + t * 64 + ((k ^ (t >> 2) ^ (t >> 4)) & 3) * 16; };
  // entry (row & 255) << 22 | (column in its 64-column step) << 16 | bits, of
  // run `which`: element (row % 16, column) of the 128-column step is pair
  // word column % 16, half (column % 32) / 16, of slot row % 16 + 16 *
  // (column / 32).  The store is unconditional (trash when not live) so the
  // entry is not first used under a divergent branch.
  auto patch = [&](uint32_t e, int which, bool live) {
    const int rg = (int)(e >> 22) & 31;
    const int col = (int)((e >> 16) & 63) + 64 * which;
    const int t = (rg & 15) + 16 * (col >> 5);
    const int el = col & 31;
    uint8_t* dst = live ? chunk(t, (el & 15) >> 2) + 4 * (el & 3) + 2 * (el >> 4) : trash;
    *(uint16_t*)dst = (uint16_t)(e & 0xFFFFu);
  };

  f32x4 acc[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Workgroup step m: decode this wave's atoms of m (issued D workgroup steps
  // ago), patch with the entries of m (issued one step ago, bounds bc); issue
  // entries m+1 (bounds bn, read one step ago), bounds m+2 (into bc), atoms
  // m+D (into at); MFMAs from the LDS x tile of m (skipped for a step past the
  // split); x of m+1 (registers xs) to the other LDS buffer, then x of m+3
  // into xs; barrier.
  auto step = [&](int m, WAtom& at, XRaw (&xs)[XI], Ents& ec, Ents& en, Bounds& bc, const Bounds& bn) {
    uint32_t w[16];
    {
      Atom t;
      t.s = at.s;
#pragma unroll
      for (int i = 0; i < 7; ++i) t.m[i] = at.m[i];
#pragma unroll
      for (int i = 0; i < 3; ++i) t.d[i] = at.d[i];
      t.e = (uint16_t)(at.ew >> esh);
      decode_pairs(t, w);
    }
    // load order -> MFMA order through the scratch
    const int tw = rl + 16 * ql;
#pragma unroll
    for (int k = 0; k < 4; ++k) *(u32x4*)chunk(tw, k) = u32x4{w[4 * k], w[4 * k + 1], w[4 * k + 2], w[4 * k + 3]};
    if constexpr (EXACT) {
      const uint32_t b0 = __builtin_amdgcn_readfirstlane(bc.b0), e0 = __builtin_amdgcn_readfirstlane(bc.e0);
      const uint32_t b1 = __builtin_amdgcn_readfirstlane(bc.b1), e1 = __builtin_amdgcn_readfirstlane(bc.e1);
      patch(ec.v[0], 0, b0 + (uint32_t)lane < e0);
      patch(ec.v[1], 1, b1 + (uint32_t)lane < e1);
      for (uint32_t e = b0 + 64u + (uint32_t)lane; e < e0; e += 64) patch(kp_ent[e], 0, true);   // dense runs (rare)
      for (uint32_t e = b1 + 64u + (uint32_t)lane; e < e1; e += 64) patch(kp_ent[e], 1, true);
    }
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const u32x4 v = *(const u32x4*)chunk(lane, k);
      const uint32_t v0 = v.x, v1 = v.y, v2 = v.z, v3 = v.w;
      w[4 * k] = v0; w[4 * k + 1] = v1; w[4 * k + 2] = v2; w[4 * k + 3] = v3;
    }
    // the scheduler must not move loads across these points: the issue order
    // is the consumption order
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (EXACT) {
      load_ents(bn, en);
      load_bounds(m + 2, bc);
    }
    load_w(m + D, at);
    __builtin_amdgcn_sched_barrier(0);
    if (KQ == 1 || m * KQ + kq < n) {
      const uint8_t* xb = lds + (m & 1) * XBUF + 256 * kq;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        bf16x8_t a;
        const uint32_t aw[4] = {w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]};
        __builtin_memcpy(&a, aw, 16);
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const bf16x8_t b = *(const bf16x8_t*)(xb + (16 * c + r) * XROW + (16 * q + 4 * i) * 4);
          acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[c], 0, 0, 0);
        }
      }
    }
    store_x(xs, lds + ((m + 1) & 1) * XBUF);
    __builtin_amdgcn_sched_barrier(0);
    load_x(m + 3, xs);
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
  };

  // ---- prologue: x(0) to LDS; then the loads in flight at the loop entry in
  // the order steps -D .. -1 would have issued them: atoms 0 .. D-2, x 1,
  // entries 0, bounds 1, atoms D-1, x 2
  WAtom A[D];
  Bounds Bd[2] = {};
  Ents E[2] = {};
  XRaw X[2][XI];
  if constexpr (EXACT) load_bounds(0, Bd[0]);
  load_x(0, X[0]);
  store_x(X[0], lds);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int u = 0; u + 1 < D; ++u) load_w(u, A[u]);
  load_x(1, X[1]);
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (EXACT) {
    load_ents(Bd[0], E[0]);
    load_bounds(1, Bd[1]);
  }
  load_w(D - 1, A[D - 1]);
  load_x(2, X[0]);
  __builtin_amdgcn_sched_barrier(0);
  __syncthreads();
  // registers at workgroup step m: atoms in A[m % D], x of m+1 in
  // X[(m+1) % 2], entries of m in E[m % 2], bounds of m in Bd[m % 2] and of
  // m+1 in the other
  int m = 0;
  for (; m + D - 1 < nm; m += D) {
#pragma unroll
    for (int u = 0; u < D; ++u) step(m + u, A[u], X[(u + 1) & 1], E[u & 1], E[(u + 1) & 1], Bd[u & 1], Bd[(u + 1) & 1]);
  }
#pragma unroll
  for (int u = 0; u + 1 < D; ++u)
    if (m + u < nm) step(m + u, A[u], X[(u + 1) & 1], E[u & 1], E[(u + 1) & 1], Bd[u & 1], Bd[(u + 1) & 1]);
  if (n == 0) return;

  // ---- the KQ waves of a row group add their sums in wave order
  if constexpr (KQ > 1) {
    float* red = (float*)lds;                      // [row group][kq - 1][NC * 4][64] (the x buffers are free)
    if (kq > 0) {
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int v = 0; v < 4; ++v) red[((wg * (KQ - 1) + kq - 1) * NC * 4 + c * 4 + v) * 64 + lane] = acc[c][v];
    }
    __syncthreads();
    if (kq > 0) return;
#pragma unroll
    for (int k = 1; k < KQ; ++k)
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[c][v] += red[((wg * (KQ - 1) + k - 1) * NC * 4 + c * 4 + v) * 64 + lane];
  }

  // ---- results: D[4(l/16) + v][l % 16] = W row n0w + 4q + v, token 16c + r
  const int64_t row0 = n0w + 4 * q;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int64_t tok = 16 * c + r;
    if (tok >= M) continue;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int64_t row = row0 + v;
      if (row >= out_f) continue;
      const float val = acc[c][v];
      if constexpr (PARTIAL) ((float*)out)[((int64_t)split * M + tok) * out_f + row] = val;
      else if constexpr (YF32) ((float*)out)[tok * out_f + row] = val;
      else ((uint16_t*)out)[tok * out_f + row] = (uint16_t)f32_to_bf16_rne(val);
    }
  }
}

// y = the sum of the K splits' fp32 partials in split order; four
// consecutive elements per thread (16-byte loads) where count % 4 == 0
template <bool YF32, bool VEC>
__global__ __launch_bounds__(256) void skinny2_reduce_kernel(const float* __restrict__ ws, int64_t count, int nsplit,
                                                             void* __restrict__ y) {
  typedef float f32x4v __attribute__((ext_vector_type(4)));
  if constexpr (VEC) {
    for (int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4; i < count; i += (int64_t)gridDim.x * 256 * 4) {
      f32x4v s = *(const f32x4v*)(ws + i);
      for (int k = 1; k < nsplit; ++k) s += *(const f32x4v*)(ws + (int64_t)k * count + i);
      if constexpr (YF32) {
        *(f32x4v*)((float*)y + i) = s;
      } else {
        const float v0 = s.x, v1 = s.y, v2 = s.z, v3 = s.w;
        *(u32x2a*)((uint16_t*)y + i) = u32x2a{f32_to_bf16_rne(v0) | (f32_to_bf16_rne(v1) << 16),
                                              f32_to_bf16_rne(v2) | (f32_to_bf16_rne(v3) << 16)};
      }
    }
  } else {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < count; i += (int64_t)gridDim.x * 256) {
      float s = ws[i];
      for (int k = 1; k < nsplit; ++k) s += ws[(int64_t)k * count + i];
      if constexpr (YF32) ((float*)y)[i] = s;
      else ((uint16_t*)y)[i] = (uint16_t)f32_to_bf16_rne(s);
    }
  }
}

struct Split {
  int sps, ks;
};

// Token blocks of 16 and waves per row group for M activation rows: KQ = 4
// up to 32 rows (16 waves per workgroup), 2 above (8 waves: the x tile of 4
// steps for 64 tokens would not fit beside the scratch, the tile of 2 steps
// does; 64 rows at 14336 x 4096: 47 us against 55 us with one wave per
// row group).  The override BF16X_TUNE_SKINNY2_KQ = 1 or 2 replaces it.
int nc_for(int64_t M) { return M <= 16 ? 1 : (M <= 32 ? 2 : 4); }
int kq_for(int64_t M) {
  const int64_t k = tuning(BF16X_TUNE_SKINNY2_KQ);
  if (k == 1) return 1;
  if (k == 2) return 2;
  return nc_for(M) <= 2 ? 4 : 2;
}

// Workgroups of the (NC, KQ, EXACT) kernel resident at once on the current
// device, from the runtime's occupancy calculation (registers and LDS of the
// compiled kernel); 3 (KQ = 1) or 1 (KQ = 2, 4) per CU on 256 CUs when there
// is no device to ask.
template <int NC, int KQ, bool EXACT>
int64_t resident_slots() {
  static int64_t cache[64];
  const int64_t dflt = KQ == 1 ? 768 : 256;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return dflt;
  if (cache[dev] > 0) return cache[dev];
  int per_cu = 0, cus = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, gemm_skinny2_kernel<NC, KQ, EXACT, true, false>,
                                                   256 * KQ, 0) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || per_cu <= 0 || cus <= 0)
    return dflt;
  cache[dev] = (int64_t)per_cu * cus;
  return cache[dev];
}

int64_t slots_for(int64_t M, bool exact) {
  const int nc = nc_for(M), kq = kq_for(M);
  if (kq == 4) {
    if (nc == 1) return exact ? resident_slots<1, 4, true>() : resident_slots<1, 4, false>();
    return exact ? resident_slots<2, 4, true>() : resident_slots<2, 4, false>();
  }
  if (kq == 2) {
    if (nc == 4) return exact ? resident_slots<4, 2, true>() : resident_slots<4, 2, false>();
    if (nc == 2) return exact ? resident_slots<2, 2, true>() : resident_slots<2, 2, false>();
    return exact ? resident_slots<1, 2, true>() : resident_slots<1, 2, false>();
  }
  if (nc == 1) return exact ? resident_slots<1, 1, true>() : resident_slots<1, 1, false>();
  if (nc == 2) return exact ? resident_slots<2, 1, true>() : resident_slots<2, 1, false>();
  return exact ? resident_slots<4, 1, true>() : resident_slots<4, 1, false>();
}

// K split: as many splits as keep the grid within one round of resident
// workgroups, at least 2 workgroup steps each, steps per split a multiple of
// KQ.  A second, partial round would cost a whole workgroup lifetime for a
// few workgroups.
Split skinny2_split(int64_t M, int64_t out_f, int64_t in_f, bool exact) {
  const int64_t tiles = (out_f + kRowsBlock - 1) / kRowsBlock;
  const int64_t S = in_f / kStep;
  const int64_t kq = kq_for(M);
  int64_t ks = slots_for(M, exact) / tiles;
  ks = std::max<int64_t>(1, std::min<int64_t>(ks, S / (2 * kq)));
  if (const int64_t t = tuning(BF16X_TUNE_SKINNY2_SPLIT); t > 0) ks = std::min<int64_t>(t, S);
  Split sp;
  int64_t sps = (S + ks - 1) / ks;
  sps = (sps + kq - 1) / kq * kq;
  sp.sps = (int)sps;
  sp.ks = (int)((S + sps - 1) / sps);
  return sp;
}

}  // namespace skinny2
}  // namespace bf16x

// Workspace of the few-row kernel: the fp32 partials of a K split (the larger
// of the exact and the saturated kernel's split).
int64_t bf16x_gemm_skinny2_workspace(int64_t M, int64_t out_f, int64_t in_f) {
  using namespace bf16x::skinny2;
  const Split a = skinny2_split(M, out_f, in_f, true), b = skinny2_split(M, out_f, in_f, false);
  const Split sp = a.ks > b.ks ? a : b;
  return sp.ks > 1 ? (int64_t)sp.ks * M * out_f * 4 : 0;
}

// Shapes are validated by bf16x_gemm (in_f % 128 == 0 here, 32-bit offsets).
int bf16x_gemm_skinny2_launch(const uint16_t* x, int64_t M, const uint32_t* s, const uint32_t* m,
                              const uint32_t* d, const uint16_t* e, const uint32_t* kp_off, const uint32_t* kp_ent,
                              int64_t out_f, int64_t in_f, bool exact, bool yf32, void* y, void* workspace,
                              int64_t workspace_bytes, hipStream_t st) {
  using namespace bf16x::skinny2;
  if (M <= 0 || M > kMaxRows || in_f % kStep != 0) return BF16X_ESHAPE;
  const Split sp = skinny2_split(M, out_f, in_f, exact);
  const bool partial = sp.ks > 1;
  if (partial && (!workspace || workspace_bytes < bf16x_gemm_skinny2_workspace(M, out_f, in_f) ||
                  ((uintptr_t)workspace & 3)))
    return BF16X_ECAPACITY;
  const int64_t tiles = (out_f + kRowsBlock - 1) / kRowsBlock;
  const int64_t grid = tiles * sp.ks;
  if (grid > INT32_MAX) return BF16X_ESHAPE;
  float* part = (float*)workspace;
  void* out = partial ? (void*)part : y;
  const int nc = nc_for(M), kq = kq_for(M);
#define BF16X_S2(NC_, KQ_, EX_, PA_, YF_)                                                                    \
  hipLaunchKernelGGL((gemm_skinny2_kernel<NC_, KQ_, EX_, PA_, YF_>), dim3((unsigned)grid), dim3(256 * KQ_), 0, st, \
                     x, M, s, m, d, e, kp_off, kp_ent, out_f, in_f, sp.sps, out)
#define BF16X_S2_NC(NC_, KQ_)                                                                             \
  do {                                                                                                   \
    if (partial) {                                                                                       \
      if (exact) BF16X_S2(NC_, KQ_, true, true, false);                                                  \
      else BF16X_S2(NC_, KQ_, false, true, false);                                                       \
    } else if (exact) {                                                                                  \
      if (yf32) BF16X_S2(NC_, KQ_, true, false, true);                                                   \
      else BF16X_S2(NC_, KQ_, true, false, false);                                                       \
    } else {                                                                                             \
      if (yf32) BF16X_S2(NC_, KQ_, false, false, true);                                                  \
      else BF16X_S2(NC_, KQ_, false, false, false);                                                      \
    }                                                                                                    \
  } while (0)
  if (kq == 4) {
    if (nc == 1) BF16X_S2_NC(1, 4);
    else BF16X_S2_NC(2, 4);
  } else if (kq == 2) {
    if (nc == 1) BF16X_S2_NC(1, 2);
    else if (nc == 2) BF16X_S2_NC(2, 2);
    else BF16X_S2_NC(4, 2);
  } else {
    switch (nc) {
      case 1: BF16X_S2_NC(1, 1); break;
      case 2: BF16X_S2_NC(2, 1); break;
      default: BF16X_S2_NC(4, 1); break;
    }
  }
#undef BF16X_S2_NC
#undef BF16X_S2
  if (partial) {
    const int64_t count = M * out_f;
    const bool vec = count % 4 == 0 && aligned16(workspace) && aligned16(y);
    const int64_t blocks = std::min<int64_t>(((vec ? count / 4 : count) + 255) / 256, 4096);
#define BF16X_S2R(YF_, VEC_)                                                                                 \
  hipLaunchKernelGGL((skinny2_reduce_kernel<YF_, VEC_>), dim3((unsigned)blocks), dim3(256), 0, st, (const float*)part, \
                     count, sp.ks, y)
    if (yf32) { if (vec) BF16X_S2R(true, true); else BF16X_S2R(true, false); }
    else { if (vec) BF16X_S2R(false, true); else BF16X_S2R(false, false); }
#undef BF16X_S2R
  }
  return BF16X_OK;
}
