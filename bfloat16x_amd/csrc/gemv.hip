// Fused decode + GEMV (batch 1) on gfx950.
//
// Replaces _bf16x_gemv_fused_kernel / bf16x_fused_gemv (bf16x_fused.py:32-127):
// y[n] = sum_k W[n,k] x[k], fp32 accumulation, y stored as bf16 (RNE).  The
// main loop accumulates the saturated weight (code 7 -> exponent emax-7);
// the plan entries of the row then add (w_exact - w_sat) * x[k], the
// correction overlay of bf16x_fused.py:83-109.
//
// Work split.  A row's P = in_f/32 atoms are divided among G waves of a
// 4-wave workgroup (G = 1, 2, 4); lane l of part g owns atoms
// g*ceil(P/G) + 64*s + l, s < NS, of EVERY row the workgroup visits.  The
// x values of those atoms are therefore loaded once per wave, kept in VGPRs
// in the decoder's (j, j+16) pairing, and no LDS is needed for x.  A
// workgroup visits `iters` groups of 4/G rows; each wave software-pipelines
// its rows: while row r is decoded and reduced, the atoms and the plan
// entries of row r+4/G are already in flight, and the (emax, x[k]) gathers
// of row r's entries were issued before that prefetch so that waiting for
// them never waits for the prefetch (vector loads complete in issue order).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "../../include/bf16x_hip.h"
#include "bf16x_device.h"
#include "launch_common.h"
#include "gemv_pipe.h"

namespace bf16x {

template <int NS, int G, int XT, bool EXACT, bool FULL, int EPI = 0, int XM = 0, int RES = 0>
__global__ __launch_bounds__(256) void gemv_pipe_kernel(
    const void* __restrict__ x, const uint32_t* __restrict__ sign, const uint32_t* __restrict__ mant,
    const uint32_t* __restrict__ delta, const uint16_t* __restrict__ emax2,
    const uint32_t* __restrict__ tile_off, const uint32_t* __restrict__ tile_ent,
    const uint8_t* __restrict__ tile_sat, int64_t out_f, int64_t in_f, int iters, uint16_t* __restrict__ y,
    NormArgs na = NormArgs{nullptr, nullptr, nullptr, 0.f, nullptr, 0}, ResArgs ra = ResArgs{nullptr, nullptr, nullptr}) {
  extern __shared__ uint32_t lds[];
  // Row blocks in dispatch order for the plain GEMV (consecutive workgroups,
  // which the dispatcher spreads over the XCDs, take consecutive rows: 0.9 %
  // faster at 14336x4096, 4-5 % at 4096x4096 and 1024x4096 than contiguous
  // per-XCD ranges); the harness variants keep the per-XCD ranges, which
  // the layer launch mirrors slot for slot.
  constexpr bool kPlain = EPI == 0 && XM == 0 && RES == 0;
  const int lb = kPlain ? (int)blockIdx.x : xcd_row_block((int)blockIdx.x, (int)gridDim.x);
  gemv_pipe_body<NS, G, XT, EXACT, FULL, EPI, XM, RES>(x, sign, mant, delta, emax2, tile_off, tile_ent, tile_sat,
                                                        out_f, in_f, iters, y, na, ra, (int)threadIdx.x, 0,
                                                        (int)blockIdx.x, lb, lds);
}

// Long rows (in_f > 4096, bf16 x): one wave per row, the row streamed in NP
// passes of 64 atoms (lane l takes atom 64c + l of pass c) through a
// two-slot register ring that runs on across the wave's rows, so the next
// row's first atoms are in flight while a row's last pass is decoded.  x is
// staged once per workgroup in LDS (the pipelined kernel's lane-major
// layout); the workgroup's 4 waves take rows base + 4i + wave, i < iters.
// No cross-wave reduction and no barrier in the main loop (the split-K
// kernel above exchanges partial sums through LDS once per row).  Plan
// offsets are read two rows ahead and the first 64 NP entries of a row one
// row ahead; a row with more entries (rare) parks its fp32 sum in LDS and
// gets its remaining entries after the last row (a loop inside the row loop
// would make the compiler keep the whole pass schedule's registers live).
constexpr int kLongMaxIters = 16;

// Rows of up to 7 passes are held to 128 VGPRs (4 waves per SIMD, the
// occupancy the launch shapes assume; the prologue's raw x took some
// variants just past it).
template <int NP, int XS, bool EXACT, bool FULL, int RES = 0>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(NP <= 7 ? 4 : 1))) void gemv_long_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ sign, const uint32_t* __restrict__ mant,
    const uint32_t* __restrict__ delta, const uint16_t* __restrict__ emax2,
    const uint32_t* __restrict__ tile_off, const uint32_t* __restrict__ tile_ent,
    const uint8_t* __restrict__ tile_sat, int64_t out_f, int64_t in_f, int iters, uint16_t* __restrict__ y,
    ResArgs ra = ResArgs{nullptr, nullptr, nullptr}) {
  static_assert(NP >= 2, "at least two passes per row");
  constexpr int NB = NP;                        // entry batches of 64 read ahead per row (3.1 % of it)
  extern __shared__ uint32_t lds[];
  __shared__ float dpart[4][kLongMaxIters];     // parked rows: fp32 sum and row index i
  __shared__ int drow[4][kLongMaxIters];
  // uniform: the row enters the loads as a scalar offset
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int64_t P = in_f >> 5;

  const __amdgpu_buffer_rsrc_t rs_ = buf_rsrc(sign, (uint64_t)out_f * P * 4);
  const __amdgpu_buffer_rsrc_t rm_ = buf_rsrc(mant, (uint64_t)out_f * P * 28);
  const __amdgpu_buffer_rsrc_t rd_ = buf_rsrc(delta, (uint64_t)out_f * P * 12);
  const __amdgpu_buffer_rsrc_t re_ = buf_rsrc(emax2, (uint64_t)out_f * P * 2);
  const __amdgpu_buffer_rsrc_t roff = buf_rsrc(tile_off, (uint64_t)(out_f + 1) * 4);
  const __amdgpu_buffer_rsrc_t rent = buf_rsrc(tile_ent, 0xFFFFFFFFull);   // reads clamped into the row
  const __amdgpu_buffer_rsrc_t rsat = buf_rsrc(tile_sat, 0xFFFFFFFFull);

  // XCD-aware order (contiguous row ranges per XCD), as the harness variants of the pipelined kernel
  const int nb = (int)gridDim.x, b = (int)blockIdx.x;
  const int per = nb / 8, extra = nb - per * 8;
  const int lb = nb >= 8 ? ((b & 7) * per + min(b & 7, extra) + (b >> 3)) : b;
  const int64_t base = (int64_t)lb * iters * 4 + wave;
  auto row_of = [&](int i) { return min(base + 4 * (int64_t)min(i, iters - 1), out_f - 1); };
  auto load_pass = [&](int i, int c, Atom& t) {
    const uint32_t sa = (uint32_t)(row_of(i) * P);
    const uint32_t va = (uint32_t)min((int64_t)(64 * c + lane), P - 1);
    t = load_atom_buf(rs_, rm_, rd_, re_, va, sa);
  };
  auto load_off = [&](int i, uint32_t& b0, uint32_t& b1) {
    const int rc = (int)row_of(i);
    b0 = __builtin_amdgcn_raw_buffer_load_b32(roff, rc * 4, 0, 0);
    b1 = __builtin_amdgcn_raw_buffer_load_b32(roff, rc * 4 + 4, 0, 0);
  };
  auto load_ents = [&](uint32_t b0, uint32_t b1, uint32_t* ent, uint8_t* sat) {
    const uint32_t last = b1 > 0 ? b1 - 1 : 0;
#pragma unroll
    for (int k = 0; k < NB; ++k) {
      const uint32_t e = min(b0 + (uint32_t)(lane + 64 * k), last);
      ent[k] = __builtin_amdgcn_raw_buffer_load_b32(rent, (int)(e * 4), 0, 0);
      sat[k] = __builtin_amdgcn_raw_buffer_load_b8(rsat, (int)e, 0, 0);
    }
  };
  auto x_at = [&](uint32_t k) -> float {
    const uint32_t a = k >> 5, j = k & 15, hi = (k >> 4) & 1;
    const uint32_t wd = lds[((((a >> 6) * 4) + (j >> 2)) * 64 + (a & 63)) * 4 + (j & 3)];
    return hi ? bf16hi_to_f32(wd) : bf16lo_to_f32(wd);
  };

  // prologue, in the order the data is needed: offsets of rows 0 and 1, x
  // (raw words, registers), the first two passes; x to LDS in pair order,
  // waiting for x alone; the entries of row 0 (their addresses wait for the
  // offsets, so they go out after the passes)
  uint32_t ob0 = 0, ob1 = 0, on0 = 0, on1 = 0;
  if constexpr (EXACT) {
    load_off(0, ob0, ob1);
    load_off(1, on0, on1);
  }
  // (RES = 1 keeps x in pair order from its loads, which the compiler then
  // issues after the passes: the raw x registers live across the passes
  // took that variant past 128 VGPRs, i.e. from 4 to 3 waves per SIMD)
  constexpr bool kRawX = RES == 0;
  uint32_t xs[XS][16];
#pragma unroll
  for (int i = 0; i < XS; ++i) {
    const int64_t a = min((int64_t)(threadIdx.x + 256 * i), P - 1);
    if constexpr (kRawX) {
      if (threadIdx.x + 256 * i < NP * 64) load_x_raw(x, a, xs[i]);
    } else {
      load_x_atom<BF16X_BF16>(x, a, xs[i]);
    }
  }
  Atom R[2];
  load_pass(0, 0, R[0]);
  load_pass(0, 1, R[1]);
  __builtin_amdgcn_sched_barrier(0);
  uint32_t ent[NB] = {};
  uint8_t sat[NB] = {};
  if constexpr (EXACT && !kRawX) load_ents(ob0, ob1, ent, sat);
#pragma unroll
  for (int i = 0; i < XS; ++i) {
    const int a = threadIdx.x + 256 * i;
    if (a < NP * 64) {
      if constexpr (kRawX) to_pair_order(xs[i]);
      u32x4* dst = (u32x4*)lds + (a >> 6) * 4 * 64 + (a & 63);
#pragma unroll
      for (int c = 0; c < 4; ++c) dst[c * 64] = u32x4{xs[i][4 * c], xs[i][4 * c + 1], xs[i][4 * c + 2], xs[i][4 * c + 3]};
    }
  }
  // raw x: the entries after the x stores, when its registers are free
  if constexpr (EXACT && kRawX) load_ents(ob0, ob1, ent, sat);
  __syncthreads();

  const u32x4* xl = (const u32x4*)lds + lane;
  float acc0 = 0.f, acc1 = 0.f;
  bool more = false;                            // uniform: the row has entries past the batches
  int nparked = 0;                              // uniform
  [[maybe_unused]] float res_ss = 0.f;          // RES = 1: sum of h^2 of this wave's rows (lane 63)
  auto store_row = [&](int64_t r, float tot, uint32_t rin) {  // lane 63; rin: the row's residual
    const uint32_t yb = f32_to_bf16_rne(tot);
    y[r] = (uint16_t)yb;
    if constexpr (RES == 1) {
      const float h = bf16lo_to_f32(f32_to_bf16_rne(bf16lo_to_f32(yb) + bf16lo_to_f32(rin)));
      ra.res_out[r] = (uint16_t)(__float_as_uint(h) >> 16);
      res_ss += h * h;
    }
  };
  // row i; its pass c sits in ring slot (PAR + c) % 2 and is refilled with
  // the pass two ahead (in this row or the next) once decoded
  auto do_row = [&](int i, auto par) {
    constexpr int PAR = decltype(par)::value;
    // RES: the row's residual, requested before this row's refills so that
    // waiting for it at the store does not wait for them
    [[maybe_unused]] uint32_t rin = 0;
    if constexpr (RES == 1) rin = ra.res_in[row_of(i)];
#pragma unroll
    for (int c = 0; c < NP; ++c) {
      Atom& cur = R[(PAR + c) & 1];
      uint32_t xr[16];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const u32x4 v = xl[(c * 4 + q) * 64];
        xr[4 * q] = v.x; xr[4 * q + 1] = v.y; xr[4 * q + 2] = v.z; xr[4 * q + 3] = v.w;
      }
      if (FULL || c < NP - 1) {
        dot_atom<BF16X_BF16>(cur, xr, acc0, acc1);
      } else {
        float t0 = 0.f, t1 = 0.f;
        dot_atom<BF16X_BF16>(cur, xr, t0, t1);
        const bool live = (int64_t)(64 * c + lane) < P;
        acc0 += live ? t0 : 0.f;
        acc1 += live ? t1 : 0.f;
      }
      if (c + 2 < NP) load_pass(i, c + 2, cur);
      else load_pass(i + 1, c + 2 - NP, cur);
      // keep each refill right behind its decode (the issue order is the
      // consumption order)
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (EXACT) {
#pragma unroll
      for (int k = 0; k < NB; ++k) {
        const uint32_t e = ob0 + (uint32_t)(lane + 64 * k);
        const uint32_t kk = min(ent[k] >> 16, (uint32_t)in_f - 1);
        const uint32_t sbits = (ent[k] & 0x807Fu) | ((uint32_t)sat[k] << 7);
        const float cc = (bf16lo_to_f32(ent[k]) - bf16lo_to_f32(sbits)) * x_at(kk);
        acc0 += (e < ob1) ? cc : 0.f;
      }
      more = __builtin_amdgcn_readfirstlane(ob1) > __builtin_amdgcn_readfirstlane(ob0) + 64u * NB;
      uint32_t nn0, nn1;
      load_off(i + 2, nn0, nn1);
      load_ents(on0, on1, ent, sat);
      ob0 = on0; ob1 = on1; on0 = nn0; on1 = nn1;
    }
    const float tot = wave_sum_dpp(acc0 + acc1);
    const int64_t r = base + 4 * (int64_t)i;
    if (EXACT && more) {                        // finished after the last row
      if (lane == 63) {
        dpart[wave][nparked] = tot;
        drow[wave][nparked] = i;
      }
      ++nparked;
    } else if (lane == 63 && r < out_f) {
      store_row(r, tot, rin);
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
  // parked rows: entries past the read-ahead batches (same wave's LDS
  // writes, read back in issue order)
  for (int d = 0; d < nparked; ++d) {
    const int i = __builtin_amdgcn_readfirstlane(drow[wave][d]);
    const int64_t r = base + 4 * (int64_t)i;
    const uint32_t b0 = tile_off[row_of(i)], b1 = tile_off[row_of(i) + 1];
    float a = 0.f;
    for (uint32_t e = b0 + 64u * NB + (uint32_t)lane; e < b1; e += 64) {
      const uint32_t en = tile_ent[e];
      const uint32_t kk = min(en >> 16, (uint32_t)in_f - 1);
      const uint32_t sbits = (en & 0x807Fu) | ((uint32_t)tile_sat[e] << 7);
      a = fmaf(bf16lo_to_f32(en) - bf16lo_to_f32(sbits), x_at(kk), a);
    }
    const float tot = wave_sum_dpp(a) + dpart[wave][d];
    if (lane == 63 && r < out_f) store_row(r, tot, RES == 1 ? (uint32_t)ra.res_in[r] : 0u);
  }
  if constexpr (RES == 1) {
    __shared__ float rpart[4];
    if (lane == 63) rpart[wave] = res_ss;
    __syncthreads();
    if (threadIdx.x == 0) ra.slots[blockIdx.x] = (rpart[0] + rpart[1]) + (rpart[2] + rpart[3]);
  }
}

// Any in_f % 32 == 0 (e.g. beyond the pipelined kernel's 16384 columns):
// one wave per row, x values read from global memory per atom.
template <int XT>
__global__ __launch_bounds__(256) void gemv_generic_kernel(
    const void* __restrict__ x, const uint32_t* __restrict__ sign, const uint32_t* __restrict__ mant,
    const uint32_t* __restrict__ delta, const uint16_t* __restrict__ emax2,
    const uint32_t* __restrict__ tile_off, const uint32_t* __restrict__ tile_ent, int64_t out_f,
    int64_t in_f, int tpr, uint16_t* __restrict__ y) {
  constexpr int XW = (XT == BF16X_BF16) ? 16 : 32;
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= out_f) return;
  const int64_t P = in_f >> 5;
  const uint8_t* emax = (const uint8_t*)emax2;
  float acc0 = 0.f, acc1 = 0.f;
  for (int64_t a = lane; a < P; a += 64) {
    uint32_t xr[XW];
    load_x_atom<XT>(x, a, xr);
    dot_atom<XT>(load_atom(sign, mant, delta, emax2, r * P + a), xr, acc0, acc1);
  }
  if (tile_off != nullptr) {
    for (int seg = 0; seg < tpr; ++seg) {
      const int64_t t = r * tpr + seg;
      for (int64_t e = (int64_t)tile_off[t] + lane; e < (int64_t)tile_off[t + 1]; e += 64) {
        const uint32_t en = tile_ent[e];
        const int64_t k = (int64_t)seg * kPlanTileCols + (en >> 16);
        if (k < in_f) acc0 = fmaf(entry_delta(en, emax[(r * in_f + k) >> 4]), load_x_elem<XT>(x, k), acc0);
      }
    }
  }
  const float tot = wave_sum(acc0 + acc1);
  if (lane == 0) y[r] = (uint16_t)f32_to_bf16_rne(tot);
}

}  // namespace bf16x

using namespace bf16x;

namespace {

// Launch-shape overrides (bf16x_set_tuning), 0 = use the built-in heuristic.
int gemv_iters_override() { return (int)std::max<int64_t>(0, tuning(BF16X_TUNE_GEMV_ITERS)); }
int gemv_g_override() { return (int)std::max<int64_t>(0, tuning(BF16X_TUNE_GEMV_G)); }

// BF16X_TUNE_GEMV_LONG = 0 sends long rows to the split-K kernel instead.
bool gemv_long_enabled() { return tuning(BF16X_TUNE_GEMV_LONG) != 0; }

// Long rows (bf16 x, 4096 < in_f <= 16384): the one-wave-per-row kernel
// (4096 x 14336 exact: 20.5 us against 22.4 us for the split-K kernel;
// 2048 x 14336: 11.5 against 13.3).
// rows per wave of the long-row kernel (measured): 4 from 2048 groups of 4
// rows, 2 from 1024
// Rows per wave of the long-row kernel.  With the residual epilogue (RES)
// one row per wave up to 2047 row groups: measured faster in the Llama decode
// step (down and o GEMVs, 1024 groups: 338 against 335 tok/s).
int long_iters(int64_t groups, bool res = false) {
  int iters = gemv_iters_override();
  if (iters <= 0) iters = groups >= 2048 ? 4 : (groups >= 1024 && !res ? 2 : 1);
  return std::min(iters, kLongMaxIters);
}

template <int RES = 0>
int launch_gemv_long(const void* x, const uint32_t* sign, const uint32_t* mant, const uint32_t* delta,
                     const uint16_t* emax2, const uint32_t* to, const uint32_t* te, const uint8_t* ts,
                     int64_t out_f, int64_t in_f, uint16_t* y, hipStream_t st,
                     ResArgs ra = ResArgs{nullptr, nullptr, nullptr}) {
  const int64_t P = in_f >> 5;
  const int np = (int)((P + 63) / 64);
  const bool full = P % 64 == 0;
  const size_t lds = (size_t)np * 4 * 64 * 16;
  const int64_t groups = (out_f + 3) / 4;
  const int iters = long_iters(groups, RES != 0);
  const int64_t grid = (groups + iters - 1) / iters;
  if (grid > INT32_MAX) return BF16X_ESHAPE;
#define BF16X_LONG1(NP_, EX_, FU_)                                                                              \
  hipLaunchKernelGGL((gemv_long_kernel<NP_, 2, EX_, FU_, RES>), dim3((unsigned)grid), dim3(256), lds, st,        \
                     (const uint16_t*)x, sign, mant, delta, emax2, to, te, ts, out_f, in_f, iters, y, ra)
#define BF16X_LONG(NP_)                                                                                        \
  case NP_:                                                                                                    \
    if (to) { if (full) BF16X_LONG1(NP_, true, true); else BF16X_LONG1(NP_, true, false); }                    \
    else { if (full) BF16X_LONG1(NP_, false, true); else BF16X_LONG1(NP_, false, false); }                     \
    break;
  switch (np) {
    BF16X_LONG(3) BF16X_LONG(4) BF16X_LONG(5) BF16X_LONG(6) BF16X_LONG(7) BF16X_LONG(8)
    default: return BF16X_ESHAPE;
  }
#undef BF16X_LONG
#undef BF16X_LONG1
  return launch_status();
}

template <int XT>
int launch_gemv(const void* x, const uint32_t* sign, const uint32_t* mant, const uint32_t* delta,
                const uint16_t* emax2, const uint32_t* to, const uint32_t* te, const uint8_t* ts, int64_t out_f,
                int64_t in_f, uint16_t* y, hipStream_t st) {
  const int64_t P = in_f >> 5;
  const int tpr = tiles_per_row(in_f);
  // (rows of up to 4096 columns stay on the split-K kernel: measured faster
  // there in exact mode, 20.9 against 21.8 us at 14336 x 4096)
  if (XT == BF16X_BF16 && gemv_long_enabled() && P > 128 && P <= 512 && tpr == 1 &&
      (out_f + 1) * P * 28 < (int64_t)0xFFFFFFFF)
    return launch_gemv_long(x, sign, mant, delta, emax2, to, te, ts, out_f, in_f, y, st);
  // parts of 64*NS atoms per wave; G = ceil(P / (64*NS)) waves per row.
  // NS = 2, and a row that one wave takes whole (in_f <= 4096) stays whole
  // at every row count (launches queued on the GPU, one wave per row against
  // two half rows: 1024x4096 4.15 against 4.50 us, 3072x4096 6.67 against
  // 7.04, 1024x3072 3.94 against 4.30, 512x4096 3.66 against 3.84); wider
  // rows split over more waves when rows are few (NS = 1, more waves in
  // flight).
  int NS = (P > 64) ? 2 : 1;
  int G = (int)((P + 64 * NS - 1) / (64 * NS));
  if (NS == 2 && G > 1 && out_f * G < 4096 && (P + 63) / 64 <= 4) { NS = 1; G = (int)((P + 63) / 64); }
  if (G == 3) G = 4;  // the fourth part of each row is empty
  const int g_req = gemv_g_override();
  if (g_req == 1 || g_req == 2 || g_req == 4) {
    const int ns_req = (P + 64 * g_req - 1) / (64 * g_req);
    if (ns_req >= 1 && ns_req <= 2) { NS = ns_req; G = g_req; }
  }
  const int xw = (XT == BF16X_BF16) ? 16 : 32;
  const size_t lds = (size_t)G * NS * 64 * (xw / 4) * 16;
  if (G <= 4 && tpr == 1 && (out_f + 1) * P * 28 < (int64_t)0xFFFFFFFF && lds + 64 <= 65536) {
    const bool full = (XT == BF16X_BF16) && P == (int64_t)G * 64 * NS;
    const int rpi = 4 / G;
    const int64_t groups = (out_f + rpi - 1) / rpi;
    // Row groups per workgroup (measured at the configuration-2 and -4
    // shapes): 2 from 1024 groups on (6144 x 4096: 10.6 us against 11.7 us
    // with 1; 4096 x 4096: 8.2 against 8.5); 4 for rows split over 4 waves
    // (long rows) from 2048 groups on, where the 4096 x 14336 grid then fits
    // one round of resident workgroups (21.6 us against 23.0 us with 2).
    int iters = gemv_iters_override();
    if (iters <= 0) iters = groups >= 2048 ? (G == 4 ? 4 : 2) : (groups >= 1024 ? 2 : 1);
    const int64_t grid = (groups + iters - 1) / iters;
    if (grid > INT32_MAX) return BF16X_ESHAPE;
#define BF16X_PIPE1(NS_, G_, EX_, FULL_)                                                             \
  hipLaunchKernelGGL((gemv_pipe_kernel<NS_, G_, XT, EX_, FULL_>), dim3((unsigned)grid), dim3(256), lds, st, x, \
                     sign, mant, delta, emax2, to, te, ts, out_f, in_f, iters, y)
#define BF16X_PIPE(NS_, G_)                                                                            \
  do {                                                                                               \
    if (to != nullptr) {                                                                             \
      if (full) BF16X_PIPE1(NS_, G_, true, (XT == BF16X_BF16)); else BF16X_PIPE1(NS_, G_, true, false); \
    } else {                                                                                         \
      if (full) BF16X_PIPE1(NS_, G_, false, (XT == BF16X_BF16)); else BF16X_PIPE1(NS_, G_, false, false); \
    }                                                                                                \
  } while (0)
    if (NS == 1) {
      if (G == 1) BF16X_PIPE(1, 1); else if (G == 2) BF16X_PIPE(1, 2); else BF16X_PIPE(1, 4);
    } else {
      if (G == 1) BF16X_PIPE(2, 1); else if (G == 2) BF16X_PIPE(2, 2); else BF16X_PIPE(2, 4);
    }
#undef BF16X_PIPE
#undef BF16X_PIPE1
  } else {
    const int64_t grid = (out_f + 3) / 4;
    if (grid > INT32_MAX) return BF16X_ESHAPE;
    hipLaunchKernelGGL((gemv_generic_kernel<XT>), dim3((unsigned)grid), dim3(256), 0, st, x, sign, mant, delta,
                       emax2, to, te, out_f, in_f, tpr, y);
  }
  return launch_status();
}

// One-wave-per-row GEMV variants (G = 1, in_f <= 4096): EPI = 1 SwiGLU
// epilogue (iters = 2), XM = 1 RMSNorm staging.
template <int EPI, int XM>
int launch_gemv_g1(const void* x, const uint32_t* sign, const uint32_t* mant, const uint32_t* delta,
                   const uint16_t* emax2, const uint32_t* to, const uint32_t* te, const uint8_t* ts, int64_t out_f,
                   int64_t in_f, uint16_t* y, NormArgs na, hipStream_t st) {
  const int64_t P = in_f >> 5;
  if ((EPI == 1 && out_f % 8 != 0) || P > 128 || tiles_per_row(in_f) != 1 ||
      (out_f + 1) * P * 28 >= (int64_t)0xFFFFFFFF)
    return BF16X_ESHAPE;
  const int NS = P > 64 ? 2 : 1;
  const bool full = P == (int64_t)64 * NS;
  const size_t lds = (size_t)NS * 64 * 4 * 16;
  const int64_t groups = (out_f + 3) / 4;
  int iters = EPI == 1 ? 2 : (groups >= 1024 ? 2 : 1);
  if (XM != 0) {
    // every workgroup normalises x in its prologue (with its own pass over
    // x): at least groups / 2048 row groups per workgroup (the override
    // BF16X_TUNE_GEMV_XM_SLOTS replaces 2048).  Measured in the Llama decode step (gate_up, 7168
    // groups): 2048 -> 1792 workgroups, 7 per CU, 334.8 tok/s; 1024 -> 896,
    // 3.5 per CU, 327.5; 512 -> 512, 333.0; 4096 -> 3584, 309.6
    int64_t slots = 2048;
    if (const int64_t t = tuning(BF16X_TUNE_GEMV_XM_SLOTS); t > 0) slots = t;
    iters = std::max<int64_t>(iters, (groups + slots - 1) / slots);
    if (EPI == 1) iters += iters & 1;
  }
  // EPI = 1: an even iters starts every workgroup on a row group of 8 (out_f % 8 == 0)
  const int64_t grid = (groups + iters - 1) / iters;
  if (grid > INT32_MAX) return BF16X_ESHAPE;
#define BF16X_G1(NS_, EX_, FULL_)                                                                                \
  hipLaunchKernelGGL((gemv_pipe_kernel<NS_, 1, BF16X_BF16, EX_, FULL_, EPI, XM>), dim3((unsigned)grid), dim3(256), \
                     lds, st, x, sign, mant, delta, emax2, to, te, ts, out_f, in_f, iters, y, na)
  if (NS == 2) {
    if (to) { if (full) BF16X_G1(2, true, true); else BF16X_G1(2, true, false); }
    else { if (full) BF16X_G1(2, false, true); else BF16X_G1(2, false, false); }
  } else {
    if (to) { if (full) BF16X_G1(1, true, true); else BF16X_G1(1, true, false); }
    else { if (full) BF16X_G1(1, false, true); else BF16X_G1(1, false, false); }
  }
#undef BF16X_G1
  return launch_status();
}

int check_gemv_args(const void* x, const int32_t* sign, int64_t n_sign, const int32_t* mant, int64_t n_mant,
                    const int32_t* delta, int64_t n_delta, const uint8_t* emax, int64_t n_emax,
                    const uint32_t* tile_off, const uint32_t* tile_ent, const uint8_t* tile_sat, int64_t out_f,
                    int64_t in_f, int32_t mode, const uint16_t* y) {
  if (!x || !sign || !mant || !delta || !emax || !y) return BF16X_EARG;
  if (mode != BF16X_EXACT && mode != BF16X_SATURATED) return BF16X_EARG;
  const int rc = check_dict(out_f, in_f, 16, n_sign, n_mant, n_delta, n_emax);
  if (rc) return rc;
  if (in_f % 32 != 0) return BF16X_ESHAPE;
  if (mode == BF16X_EXACT && (!tile_off || !tile_ent || !tile_sat)) return BF16X_EARG;
  if (!aligned4(x) || !aligned4(sign) || !aligned4(mant) || !aligned4(delta) || !aligned2(emax) || !aligned2(y))
    return BF16X_EARG;
  return BF16X_OK;
}

}  // namespace

extern "C" int bf16x_gemv_swiglu(const void* x, const int32_t* sign, int64_t n_sign, const int32_t* mant,
                                 int64_t n_mant, const int32_t* delta, int64_t n_delta, const uint8_t* emax,
                                 int64_t n_emax, const uint32_t* tile_off, const uint32_t* tile_ent,
                                 const uint8_t* tile_sat, int64_t out_f, int64_t in_f, int32_t mode, uint16_t* y,
                                 bf16x_stream_t stream) {
  const int rc = check_gemv_args(x, sign, n_sign, mant, n_mant, delta, n_delta, emax, n_emax, tile_off, tile_ent,
                                 tile_sat, out_f, in_f, mode, y);
  if (rc) return rc;
  const bool ex = mode == BF16X_EXACT;
  return launch_gemv_g1<1, 0>(x, (const uint32_t*)sign, (const uint32_t*)mant, (const uint32_t*)delta,
                              (const uint16_t*)emax, ex ? tile_off : nullptr, ex ? tile_ent : nullptr,
                              ex ? tile_sat : nullptr, out_f, in_f, y, NormArgs{nullptr, nullptr, nullptr, 0.f},
                              (hipStream_t)stream);
}

namespace {

// Rows per workgroup of the one-wave-per-row pipelined kernel with the
// residual epilogue: 2 from 1024 groups of 4 rows (as the plain GEMV), 1
// below.
int res_pipe_iters(int64_t groups) {
  const int it = gemv_iters_override();
  return it > 0 ? it : (groups >= 1024 ? 2 : 1);
}

}  // namespace

// Workgroups of bf16x_gemv_residual = the slots it writes; -1 for shapes it
// does not take.
extern "C" int64_t bf16x_gemv_residual_slots(int64_t out_f, int64_t in_f) {
  if (out_f <= 0 || in_f <= 0 || in_f % 32 != 0 || in_f > 16384) return -1;
  const int64_t P = in_f >> 5, groups = (out_f + 3) / 4;
  if ((out_f + 1) * P * 28 >= (int64_t)0xFFFFFFFF) return -1;
  const int64_t it = P <= 128 ? res_pipe_iters(groups) : long_iters(groups, true);
  return (groups + it - 1) / it;
}

extern "C" int bf16x_gemv_residual(const void* x, const uint16_t* residual_in, uint16_t* residual_out, float* slots,
                                   int64_t n_slots, const int32_t* sign, int64_t n_sign, const int32_t* mant,
                                   int64_t n_mant, const int32_t* delta, int64_t n_delta, const uint8_t* emax,
                                   int64_t n_emax, const uint32_t* tile_off, const uint32_t* tile_ent,
                                   const uint8_t* tile_sat, int64_t out_f, int64_t in_f, int32_t mode, uint16_t* y,
                                   bf16x_stream_t stream) {
  const int rc = check_gemv_args(x, sign, n_sign, mant, n_mant, delta, n_delta, emax, n_emax, tile_off, tile_ent,
                                 tile_sat, out_f, in_f, mode, y);
  if (rc) return rc;
  if (!residual_in || !residual_out || !slots) return BF16X_EARG;
  if ((const void*)residual_out == x || residual_out == y || (const void*)residual_in == (const void*)y)
    return BF16X_EARG;
  if (!aligned2(residual_in) || !aligned2(residual_out) || !aligned4(slots)) return BF16X_EARG;
  const int64_t need = bf16x_gemv_residual_slots(out_f, in_f);
  if (need < 0) return BF16X_ESHAPE;
  if (n_slots < need) return BF16X_ECAPACITY;
  const bool ex = mode == BF16X_EXACT;
  const uint32_t *to = ex ? tile_off : nullptr, *te = ex ? tile_ent : nullptr;
  const uint8_t* ts = ex ? tile_sat : nullptr;
  const uint32_t* s = (const uint32_t*)sign;
  const uint32_t* m = (const uint32_t*)mant;
  const uint32_t* d = (const uint32_t*)delta;
  const uint16_t* e = (const uint16_t*)emax;
  hipStream_t st = (hipStream_t)stream;
  const ResArgs ra{residual_in, residual_out, slots};
  const int64_t P = in_f >> 5;
  if (P > 128) {
    const int r2 = launch_gemv_long<1>(x, s, m, d, e, to, te, ts, out_f, in_f, y, st, ra);
    return r2;
  }
  const int NS = P > 64 ? 2 : 1;
  const bool full = P == (int64_t)64 * NS;
  const size_t lds = (size_t)NS * 64 * 4 * 16;
  const int64_t groups = (out_f + 3) / 4;
  const int iters = res_pipe_iters(groups);
  const int64_t grid = (groups + iters - 1) / iters;
  const NormArgs na{nullptr, nullptr, nullptr, 0.f, nullptr, 0};
#define BF16X_R1(NS_, EX_, FULL_)                                                                                  \
  hipLaunchKernelGGL((gemv_pipe_kernel<NS_, 1, BF16X_BF16, EX_, FULL_, 0, 0, 1>), dim3((unsigned)grid), dim3(256), lds, \
                     st, x, s, m, d, e, to, te, ts, out_f, in_f, iters, y, na, ra)
  if (NS == 2) {
    if (to) { if (full) BF16X_R1(2, true, true); else BF16X_R1(2, true, false); }
    else { if (full) BF16X_R1(2, false, true); else BF16X_R1(2, false, false); }
  } else {
    if (to) { if (full) BF16X_R1(1, true, true); else BF16X_R1(1, true, false); }
    else { if (full) BF16X_R1(1, false, true); else BF16X_R1(1, false, false); }
  }
#undef BF16X_R1
  return launch_status();
}

extern "C" int bf16x_gemv_prenormed(const void* h, const uint16_t* norm_weight, float eps, const float* slots,
                                    int64_t n_slots, const int32_t* sign, int64_t n_sign, const int32_t* mant,
                                    int64_t n_mant, const int32_t* delta, int64_t n_delta, const uint8_t* emax,
                                    int64_t n_emax, const uint32_t* tile_off, const uint32_t* tile_ent,
                                    const uint8_t* tile_sat, int64_t out_f, int64_t in_f, int32_t mode,
                                    int32_t epilogue, uint16_t* y, bf16x_stream_t stream) {
  const int rc = check_gemv_args(h, sign, n_sign, mant, n_mant, delta, n_delta, emax, n_emax, tile_off, tile_ent,
                                 tile_sat, out_f, in_f, mode, y);
  if (rc) return rc;
  if (!norm_weight || !slots || n_slots <= 0 || (epilogue != 0 && epilogue != 1)) return BF16X_EARG;
  if (n_slots > 64 * kMaxSlotsPerLane) return BF16X_ECAPACITY;
  if (!aligned4(norm_weight) || !aligned4(slots)) return BF16X_EARG;
  const bool ex = mode == BF16X_EXACT;
  const NormArgs na{nullptr, norm_weight, nullptr, eps, slots, (int)n_slots};
  const uint32_t *to = ex ? tile_off : nullptr, *te = ex ? tile_ent : nullptr;
  const uint8_t* ts = ex ? tile_sat : nullptr;
  if (epilogue == 1)
    return launch_gemv_g1<1, 2>(h, (const uint32_t*)sign, (const uint32_t*)mant, (const uint32_t*)delta,
                                (const uint16_t*)emax, to, te, ts, out_f, in_f, y, na, (hipStream_t)stream);
  return launch_gemv_g1<0, 2>(h, (const uint32_t*)sign, (const uint32_t*)mant, (const uint32_t*)delta,
                              (const uint16_t*)emax, to, te, ts, out_f, in_f, y, na, (hipStream_t)stream);
}

extern "C" int bf16x_gemv_norm(const void* x, const uint16_t* residual_in, const uint16_t* norm_weight,
                               uint16_t* residual_out, float eps, const int32_t* sign, int64_t n_sign,
                               const int32_t* mant, int64_t n_mant, const int32_t* delta, int64_t n_delta,
                               const uint8_t* emax, int64_t n_emax, const uint32_t* tile_off,
                               const uint32_t* tile_ent, const uint8_t* tile_sat, int64_t out_f, int64_t in_f,
                               int32_t mode, int32_t epilogue, uint16_t* y, bf16x_stream_t stream) {
  const int rc = check_gemv_args(x, sign, n_sign, mant, n_mant, delta, n_delta, emax, n_emax, tile_off, tile_ent,
                                 tile_sat, out_f, in_f, mode, y);
  if (rc) return rc;
  if (!norm_weight || (epilogue != 0 && epilogue != 1)) return BF16X_EARG;
  if (!aligned4(norm_weight) || (residual_in && !aligned4(residual_in)) || (residual_out && !aligned4(residual_out)))
    return BF16X_EARG;
  if (residual_out && (residual_out == residual_in || (const void*)residual_out == x)) return BF16X_EARG;
  const bool ex = mode == BF16X_EXACT;
  const NormArgs na{residual_in, norm_weight, residual_out, eps};
  const uint32_t *to = ex ? tile_off : nullptr, *te = ex ? tile_ent : nullptr;
  const uint8_t* ts = ex ? tile_sat : nullptr;
  if (epilogue == 1)
    return launch_gemv_g1<1, 1>(x, (const uint32_t*)sign, (const uint32_t*)mant, (const uint32_t*)delta,
                                (const uint16_t*)emax, to, te, ts, out_f, in_f, y, na, (hipStream_t)stream);
  return launch_gemv_g1<0, 1>(x, (const uint32_t*)sign, (const uint32_t*)mant, (const uint32_t*)delta,
                              (const uint16_t*)emax, to, te, ts, out_f, in_f, y, na, (hipStream_t)stream);
}

extern "C" int bf16x_gemv(const void* x, int32_t x_dtype, const int32_t* sign, int64_t n_sign,
                          const int32_t* mant, int64_t n_mant, const int32_t* delta, int64_t n_delta,
                          const uint8_t* emax, int64_t n_emax, const uint32_t* tile_off,
                          const uint32_t* tile_ent, const uint8_t* tile_sat, int64_t out_f, int64_t in_f,
                          int32_t sub, int32_t mode, uint16_t* y, bf16x_stream_t stream) {
  if (!x || !sign || !mant || !delta || !emax || !y) return BF16X_EARG;
  if (mode != BF16X_EXACT && mode != BF16X_SATURATED) return BF16X_EARG;
  if (mode == BF16X_EXACT && (!tile_off || !tile_ent || !tile_sat)) return BF16X_EARG;
  if (x_dtype != BF16X_BF16 && x_dtype != BF16X_F16 && x_dtype != BF16X_F32) return BF16X_EDTYPE;
  int rc = check_dict(out_f, in_f, sub, n_sign, n_mant, n_delta, n_emax);
  if (rc) return rc;
  if ((in_f & 31) != 0) return BF16X_ESHAPE;
  if (!aligned4(sign) || !aligned4(mant) || !aligned4(delta) || !aligned2(emax) || !aligned4(x)) return BF16X_EARG;
  const uint32_t* to = (mode == BF16X_EXACT) ? tile_off : nullptr;
  const uint32_t* te = (mode == BF16X_EXACT) ? tile_ent : nullptr;
  const uint8_t* ts = (mode == BF16X_EXACT) ? tile_sat : nullptr;
  hipStream_t st = (hipStream_t)stream;
  const uint32_t* s = (const uint32_t*)sign;
  const uint32_t* m = (const uint32_t*)mant;
  const uint32_t* d = (const uint32_t*)delta;
  const uint16_t* e = (const uint16_t*)emax;
  switch (x_dtype) {
    case BF16X_BF16: return launch_gemv<BF16X_BF16>(x, s, m, d, e, to, te, ts, out_f, in_f, y, st);
    case BF16X_F16: return launch_gemv<BF16X_F16>(x, s, m, d, e, to, te, ts, out_f, in_f, y, st);
    default: return launch_gemv<BF16X_F32>(x, s, m, d, e, to, te, ts, out_f, in_f, y, st);
  }
}
