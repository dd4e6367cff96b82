// Fused decode + GEMM (prefill / multi-token) on gfx950.
//
// Replaces _bf16x_gemm_fused_kernel / bf16x_fused_gemm (bf16x_gemm_fused.py:31-114):
// y[M, N] = x[M, K] . W[N, K]^T with W decoded on the fly, fp32 accumulation.
// SATURATED reproduces the reference kernel's numerics (code 7 -> exponent
// emax-7, bf16x_gemm_fused.py:84-87); EXACT applies the overflow plan and
// multiplies by the lossless weight.
//
// Work decomposition.  A workgroup (4 waves, WM x WN) owns an output tile of
// BM x BN (BN = 128) and a range of K steps of 64 (all of K, or one split of
// it when the tile count alone cannot fill the 256 CUs; split partials are
// fp32 and summed by a second kernel in a fixed order).  Per step:
//   * x tile  BM x 64 bf16: 16-byte loads into registers two steps ahead,
//     written to LDS (double buffered).  128-byte rows; 16-byte chunk c of
//     row r is stored at c ^ ((r >> 1) & 7), which makes the MFMA operand
//     reads (16 lanes x 16 B per LDS cycle, same chunk, 16 rows) conflict free.
//   * W tile  128 x 64 bf16: thread t decodes atom (2 * step + (t & 1)) of tile
//     row t >> 1 in registers (atoms loaded two steps ahead, ping-pong
//     registers) and writes it to LDS in natural order with the same swizzle.
//     W uses a ring of 3 buffers: in the iteration that multiplies step j, step
//     j + 2 is decoded and step j + 1 (decoded one iteration earlier, so every
//     thread's stores are visible) is patched, with one barrier per step.
//   * EXACT patches come from the step-major plan: entries grouped by (64-column
//     step, 16-row group), so the 128 rows of a tile at one step are one
//     contiguous run; thread t applies entries t and t + 256 of the run (loaded
//     one iteration ahead), a loop handles longer runs.
//   * v_mfma_f32_32x32x16_bf16 with A = x (32 rows x 16 k) and B = W^T (16 k x
//     32 columns), each operand 8 consecutive bf16 per lane from LDS.
// Operand layout (checked on the device): lane l holds A[l%32][8*(l/32)+v],
// B[8*(l/32)+v][l%32]; result register v of lane l is D[8*(v/4)+4*(l/32)+v%4][l%32].
//
// Step-major plan (built on the device from the row plan by bf16x_kplan_build):
//   kp_off uint32 [S*G2 + 1], S = in_f / 64 steps, G2 = 2 ceil(out_f / 32)
//     groups of 16 rows; run (s, h) = [kp_off[s*G2 + h], kp_off[s*G2 + h + 1]),
//     ordered by row, column, so the run of the 32 rows 32g .. 32g+31 is
//     [kp_off[s*G2 + 2g], kp_off[s*G2 + 2g + 2]);
//   kp_ent uint32: (row & 255) << 22 | (column & 63) << 16 | exact bf16 bits.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>

#include "../../include/bf16x_hip.h"
#include "bf16x_device.h"
#include "launch_common.h"

namespace bf16x {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kBK = 64;          // K per pipeline step
constexpr int kRowBytes = 128;   // one LDS tile row (64 bf16)
constexpr int kBN = 128;         // W rows per tile: 2 atoms x 128 rows = 256 decode threads
constexpr int kGroupRows = 32;   // rows per step-major plan group

__device__ __forceinline__ int swz(int row, int chunk) { return chunk ^ ((row >> 1) & 7); }

// the words of one atom as loaded (emax as the dword of the step's two atoms)
struct WAtom {
  uint32_t s, m[7], d[3], ew;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t gemm_rsrc(const void* p, uint64_t bytes) {
  const uint32_t n = bytes > 0xFFFFFFFFull ? 0xFFFFFFFFu : (uint32_t)bytes;
  return __builtin_amdgcn_make_buffer_rsrc((void*)p, (short)0, (int)n, 0x00020000);
}

template <int WM, int WN, int NM, int NN, bool EXACT, bool PARTIAL, bool YF32>
__global__ __launch_bounds__(256) void gemm_kernel(
    const uint16_t* __restrict__ x, int64_t M, const uint32_t* __restrict__ sign,
    const uint32_t* __restrict__ mant, const uint32_t* __restrict__ delta, const uint16_t* __restrict__ emax2,
    const uint32_t* __restrict__ kp_off, const uint32_t* __restrict__ kp_ent, int64_t out_f, int64_t in_f,
    int steps_per_split, void* __restrict__ y) {
  static_assert(WM * WN == 4, "4 waves");
  constexpr int BM = WM * 32 * NM;
  constexpr int BN = WN * 32 * NN;
  static_assert(BN == kBN, "one atom per thread per step");
  constexpr int X_BYTES = BM * kRowBytes;
  constexpr int W_BYTES = BN * kRowBytes;
  // 80 KB at 128 x 128: two blocks per CU
  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * X_BYTES + 3 * W_BYTES];
  uint8_t* const wbase = lds + 2 * X_BYTES;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: no divergent control flow on it
  const int wm = wave / WN, wn = wave % WN;
  const int64_t P = in_f >> 5;                  // atoms per row
  const int S = (int)(in_f >> 6);               // steps of 64 columns
  const int G = (int)((out_f + kGroupRows - 1) / kGroupRows);
  const int G2 = 2 * G;                         // 16-row groups of the plan

  // XCD-aware tile order: blocks are dispatched round-robin over 8 XCDs; give
  // each XCD a contiguous run of tiles, M fastest, so the M tiles that share a
  // W column block run on one XCD and share its L2.
  const int nb = (int)gridDim.x, b = (int)blockIdx.x;
  const int per = nb / 8, extra = nb - per * 8;
  const int lb = nb >= 8 ? ((b & 7) * per + min(b & 7, extra) + (b >> 3)) : b;
  const int mtiles = (int)((M + BM - 1) / BM);
  const int ntiles = (int)((out_f + BN - 1) / BN);
  const int64_t m0 = (int64_t)(lb % mtiles) * BM;
  const int nt = (lb / mtiles) % ntiles;
  const int kb = lb / mtiles / ntiles;
  const int64_t n0 = (int64_t)nt * BN;
  const int s0 = kb * steps_per_split;
  const int n = min(steps_per_split, S - s0);   // steps of this block (>= 1)

  // ---- W decode role: thread -> (tile row, atom parity).  The row differs per
  // thread, so the whole atom index goes in the vector offset.
  const int drow = tid >> 1, dpar = tid & 1;
  const int64_t wrow = min(n0 + drow, out_f - 1);
  const __amdgpu_buffer_rsrc_t rs_ = gemm_rsrc(sign, (uint64_t)out_f * P * 4);
  const __amdgpu_buffer_rsrc_t rm_ = gemm_rsrc(mant, (uint64_t)out_f * P * 28);
  const __amdgpu_buffer_rsrc_t rd_ = gemm_rsrc(delta, (uint64_t)out_f * P * 12);
  const __amdgpu_buffer_rsrc_t re_ = gemm_rsrc(emax2, (uint64_t)out_f * P * 2);
  // per-thread vector offsets are loop invariant; the step enters as a
  // uniform scalar offset (no per-step address arithmetic on the VALU)
  const uint32_t av = (uint32_t)(wrow * P) + (uint32_t)dpar;
  const uint32_t vo_m = av * 28, vo_d = av * 12, vo_s = av * 4;
  const uint32_t vo_e = (av - (uint32_t)dpar) * 2;  // dword with the emax pairs of both atoms of the step
  auto load_w = [&](int j, WAtom& t) {
    const uint32_t sa = 2u * (uint32_t)(s0 + min(j, n - 1));   // first atom of the step in the row
    const u32x4 m03 = __builtin_amdgcn_raw_buffer_load_b128(rm_, (int)vo_m, (int)(sa * 28), 0);
    const u32x3 m46 = __builtin_amdgcn_raw_buffer_load_b96(rm_, (int)(vo_m + 16), (int)(sa * 28), 0);
    const u32x3 d02 = __builtin_amdgcn_raw_buffer_load_b96(rd_, (int)vo_d, (int)(sa * 12), 0);
    t.s = __builtin_amdgcn_raw_buffer_load_b32(rs_, (int)vo_s, (int)(sa * 4), 0);
    // a full dword (both atoms' emax pairs) kept raw until the decode: a
    // 16-bit load, or a value computed from the load here, is carried around
    // the loop in a form that makes the compiler wait for all loads at the
    // loop top
    t.ew = __builtin_amdgcn_raw_buffer_load_b32(re_, (int)vo_e, (int)(sa * 2), 0);
    const uint32_t c0 = m03.x, c1 = m03.y, c2 = m03.z, c3 = m03.w, c4 = m46.x, c5 = m46.y, c6 = m46.z;
    t.m[0] = c0; t.m[1] = c1; t.m[2] = c2; t.m[3] = c3; t.m[4] = c4; t.m[5] = c5; t.m[6] = c6;
    const uint32_t e0 = d02.x, e1 = d02.y, e2 = d02.z;
    t.d[0] = e0; t.d[1] = e1; t.d[2] = e2;
  };

  // ---- decode one atom into W buffer wb (natural order, swizzled chunks)
  auto store_w = [&](const WAtom& w, uint8_t* wb) {
    Atom t;
    t.s = w.s;
#pragma unroll
    for (int i = 0; i < 7; ++i) t.m[i] = w.m[i];
#pragma unroll
    for (int i = 0; i < 3; ++i) t.d[i] = w.d[i];
    t.e = (uint16_t)(w.ew >> (16 * dpar));
    uint32_t p[16];
    decode_pairs(t, p);
    uint32_t q[16];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      q[i] = perm(p[2 * i + 1], p[2 * i], 0x05040100u);      // elements 2i, 2i+1
      q[8 + i] = perm(p[2 * i + 1], p[2 * i], 0x07060302u);  // elements 16+2i, 17+2i
    }
    uint8_t* rowp = wb + drow * kRowBytes;
#pragma unroll
    for (int c = 0; c < 4; ++c)
      *(u32x4*)(rowp + swz(drow, 4 * dpar + c) * 16) = u32x4{q[4 * c], q[4 * c + 1], q[4 * c + 2], q[4 * c + 3]};
  };

  // ---- step-major plan: the run of this tile's rows at a step, its entries
  const int g0 = (int)(n0 / kGroupRows), g1 = min(g0 + BN / kGroupRows, G);
  uint32_t kp_total = 0;
  if constexpr (EXACT) kp_total = kp_off[(int64_t)S * G2];
  const __amdgpu_buffer_rsrc_t rent = gemm_rsrc(kp_ent, (uint64_t)kp_total * 4);
  // Bounds are read with vector loads (scalar loads would share lgkmcnt with
  // the LDS operand reads and force a full wait on each of them).
  const __amdgpu_buffer_rsrc_t roff = gemm_rsrc(kp_off, ((uint64_t)S * G2 + 1) * 4);
  struct Run { uint32_t beg, end, e0, e1; };
  struct Bounds { uint32_t beg, end; };
  auto run_bounds = [&](int j, Bounds& r) {
    const int s = s0 + min(j, n - 1);
    r.beg = __builtin_amdgcn_raw_buffer_load_b32(roff, (s * G2 + 2 * g0) * 4, 0, 0);
    r.end = __builtin_amdgcn_raw_buffer_load_b32(roff, (s * G2 + 2 * g1) * 4, 0, 0);
  };
  auto load_run = [&](const Bounds& bd, Run& r) {   // entries t and t + 256 (reads past the plan return 0)
    r.beg = __builtin_amdgcn_readfirstlane(bd.beg);
    r.end = __builtin_amdgcn_readfirstlane(bd.end);
    r.e0 = __builtin_amdgcn_raw_buffer_load_b32(rent, (int)((r.beg + tid) * 4), 0, 0);
    r.e1 = __builtin_amdgcn_raw_buffer_load_b32(rent, (int)((r.beg + tid + 256) * 4), 0, 0);
  };
  // Entries past the run's end go to a trash slot: the store is
  // unconditional, so the entry is not first used under a divergent branch
  // (which would make the compiler wait for every outstanding load).  The
  // slot is the first bytes of this thread's own chunk of the x buffer that
  // it fills later in the same iteration (free until then, and overwritten
  // by that store in program order).
  auto patch_one = [&](uint32_t e, uint8_t* wb, uint8_t* trash, bool live) {
    const int r = (int)(e >> 22) & (BN - 1), c = (int)(e >> 16) & 63;
    uint8_t* dst = live ? wb + r * kRowBytes + swz(r, c >> 3) * 16 + (c & 7) * 2 : trash;
    *(uint16_t*)dst = (uint16_t)(e & 0xFFFFu);
  };
  auto apply_run = [&](const Run& r, uint8_t* wb, uint8_t* trash) {
    patch_one(r.e0, wb, trash, r.beg + tid < r.end);
    patch_one(r.e1, wb, trash, r.beg + tid + 256 < r.end);
    for (uint32_t e = r.beg + 512 + tid; e < r.end; e += 256)   // dense runs (rare)
      patch_one(kp_ent[e], wb, trash, true);
  };

  // ---- x tile: 16-byte chunk c = i*256 + tid of the step's BM x 64 tile is
  // (row c >> 3, chunk c & 7): each wave reads 8 whole 128-byte row segments.
  // Loaded into registers at the top of an iteration and written to LDS at its
  // end (plain loads only: LDS-DMA loads mixed with register loads make the
  // compiler wait for every load before each use).
  constexpr int XI = BM / 32;                   // chunks per thread per step
  const uint64_t x_bytes = (uint64_t)M * in_f * 2;
  const __amdgpu_buffer_rsrc_t rx_ = gemm_rsrc(x, x_bytes);
  uint32_t vx[XI];                              // byte offset of chunk i at step 0
#pragma unroll
  for (int i = 0; i < XI; ++i) {
    const int64_t gm = min(m0 + i * 32 + (tid >> 3), M - 1);
    vx[i] = (uint32_t)((gm * in_f + (tid & 7) * 8) * 2);
  }
  auto load_x = [&](int j, u32x4 (&xr)[XI]) {
    const uint32_t ks = (uint32_t)(s0 + min(j, n - 1)) * (kBK * 2);
#pragma unroll
    for (int i = 0; i < XI; ++i) xr[i] = __builtin_amdgcn_raw_buffer_load_b128(rx_, (int)vx[i], (int)ks, 0);
  };
  // chunk i of this thread goes to row 32i + tid/8 (so the swizzle term
  // ((row >> 1) & 7) = (tid >> 4) & 7 does not depend on i)
  const int xs_off = (tid >> 3) * kRowBytes + ((tid & 7) ^ ((tid >> 4) & 7)) * 16;
  auto store_x = [&](const u32x4 (&xr)[XI], uint8_t* xb) {
#pragma unroll
    for (int i = 0; i < XI; ++i) *(u32x4*)(xb + xs_off + i * 32 * kRowBytes) = xr[i];
  };

  // ---- accumulators
  f32x16 acc[NM][NN];
#pragma unroll
  for (int i = 0; i < NM; ++i)
#pragma unroll
    for (int j = 0; j < NN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  // MFMAs of one step: four k-quarters of 16; the operands of quarter q + 1 are
  // read from LDS while quarter q multiplies
  auto load_ops = [&](int q, const uint8_t* xb, const uint8_t* wb, bf16x8_t (&ao)[NM], bf16x8_t (&bo)[NN]) {
    const int lc = 2 * q + (lane >> 5);  // logical 16-byte chunk: k = 16q + 8*(lane/32)
#pragma unroll
    for (int jj = 0; jj < NN; ++jj) {
      const int r = (wn * NN + jj) * 32 + (lane & 31);
      bo[jj] = *(const bf16x8_t*)(wb + r * kRowBytes + swz(r, lc) * 16);
    }
#pragma unroll
    for (int i = 0; i < NM; ++i) {
      const int r = (wm * NM + i) * 32 + (lane & 31);
      ao[i] = *(const bf16x8_t*)(xb + r * kRowBytes + swz(r, lc) * 16);
    }
  };
  auto mfma_step = [&](const uint8_t* xb, const uint8_t* wb) {
    bf16x8_t ao[2][NM], bo[2][NN];
    load_ops(0, xb, wb, ao[0], bo[0]);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (q < 3) load_ops(q + 1, xb, wb, ao[(q + 1) & 1], bo[(q + 1) & 1]);
#pragma unroll
      for (int i = 0; i < NM; ++i)
#pragma unroll
        for (int jj = 0; jj < NN; ++jj)
          acc[i][jj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ao[q & 1][i], bo[q & 1][jj], acc[i][jj], 0, 0, 0);
    }
  };

  // ---- prologue: x of step 0, W of steps 0 and 1 decoded, step 0 patched;
  // atoms of steps 2 and 3 in flight, run bounds of step 2 read
  WAtom A, B;
  Run R0{}, R1{};
  Bounds Bn{};
  if constexpr (EXACT) {
    Bounds b0, b1;
    run_bounds(0, b0);
    run_bounds(1, b1);
    load_run(b0, R0);
    load_run(b1, R1);
  }
  u32x4 xA[XI], xB[XI];
  load_x(0, xA);
  load_w(0, A);
  load_w(1, B);
  store_x(xA, lds);
  store_w(A, wbase);
  store_w(B, wbase + W_BYTES);
  if constexpr (EXACT) run_bounds(2, Bn);
  // the loads in flight at the loop entry are issued in the same order as at
  // the end of a loop iteration (x, atoms, x, atoms), so the waits the
  // compiler derives for the loop hold on both paths into it
  __builtin_amdgcn_sched_barrier(0);
  load_x(1, xA);
  __builtin_amdgcn_sched_barrier(0);
  load_w(2, A);
  __builtin_amdgcn_sched_barrier(0);
  load_x(2, xB);
  __builtin_amdgcn_sched_barrier(0);
  load_w(3, B);
  __builtin_amdgcn_sched_barrier(0);
  __syncthreads();
  if constexpr (EXACT) {
    apply_run(R0, wbase, lds + X_BYTES + xs_off);   // x buffer 1 is first filled in iteration 0
    __syncthreads();
  }

  // ---- main loop, unrolled by two for the ping-pong atom registers.
  // Iteration j: load the plan run of j+2; MFMAs of step j, decode j+2, patch
  // j+1, store x(j+1); load x(j+3) and the atoms of j+4; barrier.  Loads are
  // issued in the order they are consumed (vmcnt completes in order), so x and
  // the atoms have two iterations to arrive (ping-pong registers for both).
  // Steps past the block's range re-read its last step (in bounds, results
  // unused).
  int wcur = 0;                        // W buffer of step j: (j % 3) * W_BYTES
  auto iter = [&](int j, WAtom& at, u32x4 (&xr)[XI], Run& Rp, Run& Rl) {
    const int w1 = wcur + W_BYTES == 3 * W_BYTES ? 0 : wcur + W_BYTES;
    const int w2 = w1 + W_BYTES == 3 * W_BYTES ? 0 : w1 + W_BYTES;
    if constexpr (EXACT) {
      load_run(Bn, Rl);                // run of step j + 2 (bounds read one iteration ago)
      run_bounds(j + 3, Bn);
    }
    // the scheduler must not move loads across these two points: the issue
    // order is the consumption order
    __builtin_amdgcn_sched_barrier(0);
    mfma_step(lds + (j & 1) * X_BYTES, wbase + wcur);
    store_w(at, wbase + w2);
    if constexpr (EXACT) apply_run(Rp, wbase + w1, lds + ((j + 1) & 1) * X_BYTES + xs_off);
    store_x(xr, lds + ((j + 1) & 1) * X_BYTES);
    __builtin_amdgcn_sched_barrier(0);
    load_x(j + 3, xr);
    __builtin_amdgcn_sched_barrier(0);
    load_w(j + 4, at);
    __syncthreads();
    wcur = w1;
  };
  int j = 0;
  for (; j + 1 < n; j += 2) {
    iter(j, A, xA, R1, R0);            // patch step j+1 from R1, load run j+2 into R0
    iter(j + 1, B, xB, R0, R1);        // patch step j+2 from R0, load run j+3 into R1
  }
  if (j < n) iter(j, A, xA, R1, R0);

  // ---- store: register v of lane l -> row 8(v/4) + 4(l/32) + v%4, column l%32
  float* yp = (float*)y;
  if constexpr (PARTIAL) yp += (int64_t)kb * M * out_f;
#pragma unroll
  for (int i = 0; i < NM; ++i) {
#pragma unroll
    for (int jj = 0; jj < NN; ++jj) {
      const int64_t col = n0 + (wn * NN + jj) * 32 + (lane & 31);
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t row = m0 + (wm * NM + i) * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        if (row < M && col < out_f) {
          if constexpr (PARTIAL || YF32) yp[row * out_f + col] = acc[i][jj][v];
          else ((uint16_t*)y)[row * out_f + col] = (uint16_t)f32_to_bf16_rne(acc[i][jj][v]);
        }
      }
    }
  }
}

// y = sum over splits of the fp32 partials, in split order
template <bool YF32>
__global__ __launch_bounds__(256) void gemm_reduce_kernel(const float* __restrict__ ws, int64_t count, int nsplit,
                                                          void* __restrict__ y) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < count; i += (int64_t)gridDim.x * 256) {
    float s = ws[i];
    for (int k = 1; k < nsplit; ++k) s += ws[(int64_t)k * count + i];
    if constexpr (YF32) ((float*)y)[i] = s;
    else ((uint16_t*)y)[i] = (uint16_t)f32_to_bf16_rne(s);
  }
}

// ---------------------------------------------------------------------------
// Step-major plan from the row plan (one tile per row, in_f <= 65536).  One
// 64-lane block per 32-row group; lane r < 32 walks the entries of row
// g*32 + r, which are sorted by column; lanes 0-15 and 16-31 make the runs of
// the 16-row groups 2g and 2g + 1.  Pass 1 counts each (step, 16-row group)
// run, a one-block scan turns counts into offsets, pass 2 writes the entries.
// GE: entries of the GGUF side table (column | bits << 16) instead of the row
// plan's (column << 16 | bits).
// ---------------------------------------------------------------------------
template <bool FILL, bool GE>
__global__ __launch_bounds__(64) void kplan_pass_kernel(const uint32_t* __restrict__ tile_off,
                                                        const uint32_t* __restrict__ tile_ent, int64_t out_f,
                                                        int S, int G2, uint32_t* __restrict__ kp_off,
                                                        uint32_t* __restrict__ kp_ent) {
  const int g = blockIdx.x, lane = threadIdx.x;
  const int h = 2 * g + (lane >= 16 ? 1 : 0);    // 16-row group of this lane's row
  const int64_t row = (int64_t)g * kGroupRows + lane;
  const bool live = lane < kGroupRows && row < out_f;
  uint32_t p = live ? tile_off[row] : 0, pe = live ? tile_off[row + 1] : 0;
  for (int s = 0; s < S; ++s) {
    uint32_t c = 0;
    // column >> 6 == s
    while (p + c < pe && ((GE ? tile_ent[p + c] & 0xFFFFu : tile_ent[p + c] >> 16) >> 6) == (uint32_t)s) ++c;
    uint32_t incl = c;                   // inclusive prefix over the lanes
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint32_t v = __shfl_up(incl, o);
      if (lane >= o) incl += v;
    }
    const uint32_t lo = __shfl(incl, 15);  // entries of the first 16-row group
    const uint32_t all = __shfl(incl, 63);
    if constexpr (!FILL) {
      if (lane == 0) {
        kp_off[(int64_t)s * G2 + 2 * g] = lo;
        kp_off[(int64_t)s * G2 + 2 * g + 1] = all - lo;
      }
    } else {
      const uint32_t base = kp_off[(int64_t)s * G2 + h] + (lane >= 16 ? incl - lo : incl) - c;
      for (uint32_t i = 0; i < c; ++i) {
        const uint32_t e = tile_ent[p + i];
        const uint32_t col = GE ? e & 0xFFFFu : e >> 16, bits = GE ? e >> 16 : e & 0xFFFFu;
        kp_ent[base + i] = ((uint32_t)(row & 255) << 22) | ((col & 63u) << 16) | bits;
      }
    }
    p += c;
  }
}

// exclusive scan of a[0..n) in place, a[n] = total (one block)
__global__ __launch_bounds__(1024) void kplan_scan_kernel(uint32_t* __restrict__ a, int64_t n) {
  __shared__ uint32_t part[1024];
  const int t = threadIdx.x;
  const int64_t chunk = (n + 1023) / 1024;
  const int64_t b = min((int64_t)t * chunk, n), e = min(b + chunk, n);
  uint32_t s = 0;
  for (int64_t i = b; i < e; ++i) s += a[i];
  part[t] = s;
  __syncthreads();
  for (int o = 1; o < 1024; o <<= 1) {
    const uint32_t v = t >= o ? part[t - o] : 0u;
    __syncthreads();
    part[t] += v;
    __syncthreads();
  }
  uint32_t run = part[t] - s;
  for (int64_t i = b; i < e; ++i) {
    const uint32_t v = a[i];
    a[i] = run;
    run += v;
  }
  if (t == 1023) a[n] = part[1023];
}

// Exclusive scan of a[0..n) in place on `st`, a[n] = the total (one block).
void scan_offsets(uint32_t* a, int64_t n, hipStream_t st) {
  hipLaunchKernelGGL(kplan_scan_kernel, dim3(1), dim3(1024), 0, st, a, n);
}

}  // namespace bf16x

using namespace bf16x;

extern "C" int64_t bf16x_kplan_size(int64_t out_f, int64_t in_f) {
  if (out_f <= 0 || in_f < kBK) return 0;
  return (in_f / kBK) * 2 * ((out_f + kGroupRows - 1) / kGroupRows) + 1;
}

namespace {
template <bool GE>
int kplan_build(const uint32_t* tile_off, const uint32_t* tile_ent, int64_t out_f, int64_t in_f, uint32_t* kp_off,
                uint32_t* kp_ent, bf16x_stream_t stream) {
  if (!tile_off || !tile_ent || !kp_off || !kp_ent) return BF16X_EARG;
  if (out_f <= 0 || in_f <= 0 || (in_f % kBK) != 0 || tiles_per_row(in_f) != 1) return BF16X_ESHAPE;
  const int64_t S = in_f / kBK, G = (out_f + kGroupRows - 1) / kGroupRows, G2 = 2 * G;
  if (G2 > INT32_MAX || S * G2 + 1 > (int64_t)INT32_MAX) return BF16X_ESHAPE;
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL((kplan_pass_kernel<false, GE>), dim3((unsigned)G), dim3(64), 0, st, tile_off, tile_ent, out_f,
                     (int)S, (int)G2, kp_off, kp_ent);
  scan_offsets(kp_off, S * G2, st);
  hipLaunchKernelGGL((kplan_pass_kernel<true, GE>), dim3((unsigned)G), dim3(64), 0, st, tile_off, tile_ent, out_f,
                     (int)S, (int)G2, kp_off, kp_ent);
  return launch_status();
}
}  // namespace

extern "C" int bf16x_kplan_build(const uint32_t* tile_off, const uint32_t* tile_ent, int64_t out_f, int64_t in_f,
                                 uint32_t* kp_off, uint32_t* kp_ent, bf16x_stream_t stream) {
  return kplan_build<false>(tile_off, tile_ent, out_f, in_f, kp_off, kp_ent, stream);
}

extern "C" int bf16x_gguf_kplan_build(const uint32_t* row_off, const uint32_t* entries, int64_t out_f, int64_t in_f,
                                      uint32_t* kp_off, uint32_t* kp_ent, bf16x_stream_t stream) {
  return kplan_build<true>(row_off, entries, out_f, in_f, kp_off, kp_ent, stream);
}

// wave-specialised kernel (gemm_ws.hip): M >= ws_rows()
int64_t bf16x_gemm_ws_workspace(int64_t M, int64_t out_f, int64_t in_f);
int bf16x_gemm_ws_launch(const uint16_t* x, int64_t M, const uint32_t* s, const uint32_t* m, const uint32_t* d,
                         const uint16_t* e, const uint8_t* blocks, const uint32_t* kp_off, const uint32_t* kp_ent,
                         int64_t out_f, int64_t in_f, bool exact, bool yf32, void* y, void* workspace,
                         int64_t workspace_bytes, hipStream_t st);

// few-row kernel (gemm_skinny.hip): M <= skinny_rows()
int bf16x_gemm_skinny_launch(const uint16_t* x, int64_t M, const uint32_t* s, const uint32_t* m, const uint32_t* d,
                             const uint16_t* e, const uint32_t* kp_off, const uint32_t* kp_ent, int64_t out_f,
                             int64_t in_f, bool exact, bool yf32, void* y, hipStream_t st);

// few-row MFMA kernel (gemm_skinny2.hip): M <= skinny2_rows(), in_f % 128 == 0
int64_t bf16x_gemm_skinny2_workspace(int64_t M, int64_t out_f, int64_t in_f);
int bf16x_gemm_skinny2_launch(const uint16_t* x, int64_t M, const uint32_t* s, const uint32_t* m,
                              const uint32_t* d, const uint16_t* e, const uint32_t* kp_off, const uint32_t* kp_ent,
                              int64_t out_f, int64_t in_f, bool exact, bool yf32, void* y, void* workspace,
                              int64_t workspace_bytes, hipStream_t st);

namespace {

// Largest M served by the 16x16x32-MFMA few-row kernel (at most 64).
int64_t skinny2_rows() {
  int64_t r = 64;
  if (const int64_t t = tuning(BF16X_TUNE_GEMM_SKINNY2_MAX); t >= 0) r = t;
  return r < 0 ? 0 : (r > 64 ? 64 : r);
}

bool use_skinny2(int64_t M, int64_t in_f) { return M <= skinny2_rows() && in_f % 128 == 0; }

// Smallest M served by the wave-specialised kernel (256-row tiles).
int64_t ws_rows() {
  const int64_t t = tuning(BF16X_TUNE_GEMM_WS_MIN_ROWS);
  return t >= 0 ? t : 192;
}


// Largest M served by the few-row kernel (at most 128, its column-block
// limit; measured faster than the tiled kernel up to 32 rows).
int64_t skinny_rows() {
  int64_t r = 32;
  if (const int64_t t = tuning(BF16X_TUNE_GEMM_SKINNY_MAX); t >= 0) r = t;
  return r < 0 ? 0 : (r > 128 ? 128 : r);
}

// M >= ws_rows() and past both few-row kernels
bool use_ws(int64_t M, int64_t in_f) { return M >= ws_rows() && !use_skinny2(M, in_f) && M > skinny_rows(); }

struct GemmShape {
  int bm;        // rows of x per tile
  int nsplit;    // K splits
  int sps;       // steps per split
};

// Tile height and K split.  BM = 256 above 128 rows (W decoded once per 256
// rows of x).  Then K is split while the tile count leaves CUs idle: the split
// minimises (rounds of resident blocks) x (steps per block), with a charge of
// 15% per extra split (fp32 partials written and summed, per-block prologue),
// smallest split on ties.
GemmShape gemm_shape(int64_t M, int64_t out_f, int64_t in_f) {
  GemmShape g;
  g.bm = M <= 32 ? 32 : M <= 64 ? 64 : M <= 128 ? 128 : 256;
  if (const int64_t t = tuning(BF16X_TUNE_GEMM_BM); t >= 0) g.bm = (int)t;
  const int64_t S = in_f / kBK;
  const int64_t tiles = ((M + g.bm - 1) / g.bm) * ((out_f + kBN - 1) / kBN);
  const int64_t slots = 256 * (g.bm <= 128 ? 2 : 1);   // resident blocks (LDS: 66 / 80 / 112 KB)
  int best = 1;
  double best_cost = 1e30;
  for (int k = 1; k <= 32 && k * 4 <= S; ++k) {
    const int64_t sps = (S + k - 1) / k, ks = (S + sps - 1) / sps;
    const double cost = (double)((tiles * ks + slots - 1) / slots) * sps * (1.0 + 0.15 * (ks - 1));
    if (cost < best_cost - 1e-9) { best_cost = cost; best = (int)ks; }
  }
  if (const int64_t t = tuning(BF16X_TUNE_GEMM_SPLIT); t >= 0) best = (int)std::min<int64_t>(t, S);
  if (best < 1) best = 1;
  g.sps = (int)((S + best - 1) / best);
  g.nsplit = (int)((S + g.sps - 1) / g.sps);
  return g;
}

}  // namespace

extern "C" int64_t bf16x_gemm_workspace(int64_t M, int64_t out_f, int64_t in_f) {
  if (M <= 0 || out_f <= 0 || in_f < kBK) return 0;
  if (use_skinny2(M, in_f)) return bf16x_gemm_skinny2_workspace(M, out_f, in_f);
  if (M <= skinny_rows()) return 0;
  if (use_ws(M, in_f)) return bf16x_gemm_ws_workspace(M, out_f, in_f);
  const GemmShape g = gemm_shape(M, out_f, in_f);
  return g.nsplit > 1 ? (int64_t)g.nsplit * M * out_f * 4 : 0;
}

extern "C" int bf16x_gemm(const void* x, int32_t x_dtype, int64_t M, const int32_t* sign, int64_t n_sign,
                          const int32_t* mant, int64_t n_mant, const int32_t* delta, int64_t n_delta,
                          const uint8_t* emax, int64_t n_emax, const uint32_t* kp_off, const uint32_t* kp_ent,
                          int64_t out_f, int64_t in_f, int32_t sub, int32_t mode, void* y, int32_t y_dtype,
                          void* workspace, int64_t workspace_bytes, bf16x_stream_t stream) {
  if (!x || !sign || !mant || !delta || !emax || !y) return BF16X_EARG;
  if (mode != BF16X_EXACT && mode != BF16X_SATURATED) return BF16X_EARG;
  if (mode == BF16X_EXACT && (!kp_off || !kp_ent)) return BF16X_EARG;
  if (x_dtype != BF16X_BF16 || (y_dtype != BF16X_BF16 && y_dtype != BF16X_F32)) return BF16X_EDTYPE;
  if (M <= 0) return BF16X_ESHAPE;
  int rc = check_dict(out_f, in_f, sub, n_sign, n_mant, n_delta, n_emax);
  if (rc) return rc;
  if ((in_f % kBK) != 0 || tiles_per_row(in_f) != 1) return BF16X_ESHAPE;
  // 32-bit buffer offsets: the packed mantissa stream and x must stay below 4 GiB
  if (out_f * (in_f >> 5) * 28 >= (int64_t)0xFFFFFFFF || M * in_f * 2 >= (int64_t)0xFFFFFFFF) return BF16X_ESHAPE;
  if (!aligned4(sign) || !aligned4(mant) || !aligned4(delta) || !aligned2(emax) || !aligned16(x) || !aligned4(y))
    return BF16X_EARG;
  hipStream_t st = (hipStream_t)stream;
  if (use_skinny2(M, in_f)) {
    rc = bf16x_gemm_skinny2_launch((const uint16_t*)x, M, (const uint32_t*)sign, (const uint32_t*)mant,
                                   (const uint32_t*)delta, (const uint16_t*)emax, kp_off, kp_ent, out_f, in_f,
                                   mode == BF16X_EXACT, y_dtype == BF16X_F32, y, workspace, workspace_bytes, st);
    return rc ? rc : launch_status();
  }
  if (M <= skinny_rows()) {
    rc = bf16x_gemm_skinny_launch((const uint16_t*)x, M, (const uint32_t*)sign, (const uint32_t*)mant,
                                  (const uint32_t*)delta, (const uint16_t*)emax, kp_off, kp_ent, out_f, in_f,
                                  mode == BF16X_EXACT, y_dtype == BF16X_F32, y, st);
    return rc ? rc : launch_status();
  }
  if (use_ws(M, in_f)) {
    rc = bf16x_gemm_ws_launch((const uint16_t*)x, M, (const uint32_t*)sign, (const uint32_t*)mant,
                              (const uint32_t*)delta, (const uint16_t*)emax, nullptr, kp_off, kp_ent, out_f, in_f,
                              mode == BF16X_EXACT, y_dtype == BF16X_F32, y, workspace, workspace_bytes, st);
    return rc ? rc : launch_status();
  }
  const GemmShape g = gemm_shape(M, out_f, in_f);
  if (g.bm != 32 && g.bm != 64 && g.bm != 128 && g.bm != 256) return BF16X_EARG;
  const bool split = g.nsplit > 1;
  if (split && (!workspace || workspace_bytes < (int64_t)g.nsplit * M * out_f * 4 || !aligned4(workspace)))
    return BF16X_ECAPACITY;
  const int64_t grid = ((M + g.bm - 1) / g.bm) * ((out_f + kBN - 1) / kBN) * g.nsplit;
  if (grid > INT32_MAX) return BF16X_ESHAPE;
  const bool exact = mode == BF16X_EXACT, yf = y_dtype == BF16X_F32;
  const uint16_t* xb = (const uint16_t*)x;
  const uint32_t* s = (const uint32_t*)sign;
  const uint32_t* m = (const uint32_t*)mant;
  const uint32_t* d = (const uint32_t*)delta;
  const uint16_t* e = (const uint16_t*)emax;
  void* out = split ? workspace : y;
#define BF16X_GEMM1(WM_, WN_, NM_, NN_, EX_, PA_, YF_)                                                       \
  hipLaunchKernelGGL((gemm_kernel<WM_, WN_, NM_, NN_, EX_, PA_, YF_>), dim3((unsigned)grid), dim3(256), 0, st, xb, \
                     M, s, m, d, e, kp_off, kp_ent, out_f, in_f, g.sps, out)
#define BF16X_GEMM(WM_, WN_, NM_, NN_)                                                                         \
  do {                                                                                                       \
    if (split) {                                                                                             \
      if (exact) BF16X_GEMM1(WM_, WN_, NM_, NN_, true, true, false);                                         \
      else BF16X_GEMM1(WM_, WN_, NM_, NN_, false, true, false);                                              \
    } else if (exact) {                                                                                      \
      if (yf) BF16X_GEMM1(WM_, WN_, NM_, NN_, true, false, true);                                            \
      else BF16X_GEMM1(WM_, WN_, NM_, NN_, true, false, false);                                              \
    } else {                                                                                                 \
      if (yf) BF16X_GEMM1(WM_, WN_, NM_, NN_, false, false, true);                                           \
      else BF16X_GEMM1(WM_, WN_, NM_, NN_, false, false, false);                                             \
    }                                                                                                        \
  } while (0)
  switch (g.bm) {
    case 32: BF16X_GEMM(1, 4, 1, 1); break;    //  32 x 128
    case 64: BF16X_GEMM(1, 4, 2, 1); break;    //  64 x 128
    case 128: BF16X_GEMM(2, 2, 2, 2); break;   // 128 x 128
    default: BF16X_GEMM(2, 2, 4, 2); break;    // 256 x 128
  }
#undef BF16X_GEMM
#undef BF16X_GEMM1
  if (split) {
    const int64_t count = M * out_f;
    const int64_t blocks = std::min<int64_t>((count + 255) / 256, 4096);
    if (yf)
      hipLaunchKernelGGL(gemm_reduce_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, st, (const float*)workspace,
                         count, g.nsplit, y);
    else
      hipLaunchKernelGGL(gemm_reduce_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, st, (const float*)workspace,
                         count, g.nsplit, y);
  }
  return launch_status();
}
