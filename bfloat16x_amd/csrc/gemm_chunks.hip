// Fused decode + GEMM for up to 64 activation rows: a workgroup's weight rows
// are streamed in column chunks, each chunk decoded once into LDS and
// multiplied by every token.
//
// y[M, N] = x[M, K] . W[N, K]^T, fp32 accumulation, 1 <= M <= 64
// (bf16x_gemm_fused.py:97-114 at its small blocks; EXACT writes the plan's
// entries over the decoded tile, read from the chunk plan, which groups them
// by (256-column chunk, row)).
//
// Why: at tens of tokens the product is still bound by the weight stream,
// but x no longer fits in registers for a whole row (64 tokens x 4096
// columns is 512 KB), so the row-streaming kernel of gemm_rows.hip cannot
// serve it, and the 16x16x32 kernel of gemm_skinny2.hip reads W as 16 rows
// x 4 atoms per load instruction and restages x through LDS at every step.
// Here a workgroup walks K in chunks, its rows of a chunk are read with CA
// consecutive atoms of a row per CA lanes (CA = 8, 16 or 32), and x goes
// from memory straight into MFMA operand registers, each element loaded
// once per workgroup.
//
// Layout.  One workgroup of 8 waves per CU owns a contiguous run of at most
// ROWS = 16 RT weight rows and walks K in chunks of CA atoms (32 CA columns).
// For chunk c:
//  * decode: lane l of wave w takes atom i % CA of tile row i / CA for
//    i = 64 APL w + 64 s + l, s < APL = RT CA / 32, so a load instruction
//    reads 64 / CA rows x CA consecutive atoms of each stream; the atom is
//    decoded, put in natural column order and written to the chunk's LDS
//    tile; in EXACT mode the same wave then writes the plan entries of its
//    rows (RPW = 64 APL / CA rows per wave) over them: one run of the chunk
//    plan per 256 columns, its bounds read by scalar loads;
//  * barrier;
//  * product: the waves of a token group split the chunk's columns (KS
//    k-steps of 32 each) and multiply them for every row tile and their
//    token tiles: v_mfma_f32_16x16x32_bf16 with A = 16 tile rows (LDS) and
//    B = 16 tokens of x (registers).
// The tile is double-buffered, so one barrier per chunk orders the decode of
// chunk c + 1 after the reads of chunk c - 1.  Atoms are requested two
// chunks ahead (three register sets, the loop unrolled by three), plan
// bounds three and their entries two, x one.  At the end the partial
// products of a token group's waves (each over its own columns) are added in
// wave order through LDS.
//
// Where the time goes (14336x4096, M = 16, 2 waves per SIMD): decode VALU
// about 10 us per SIMD, LDS about 2 conflict cycles per instruction cycle;
// the waves run the chunk phases in step, so decode, LDS traffic and the
// weight stream overlap only in part (saturated 23 us, exact 27 us, against
// 19.5 us for the batch-1 GEMV on the same weight).
//
// LDS tile: row r at r * (64 CA + 16) bytes (a 16-byte skew per row), atom a
// at 64 a within it, natural 16-byte chunk q (columns 8q .. 8q + 7 of the
// atom) at ((q ^ (a >> 2)) & 3) * 16.
//
// Operand layout of v_mfma_f32_16x16x32_bf16 (lane l): A[l%16][8(l/16)+v'],
// B[8(l/16)+v'][l%16] (v' < 8), D register v = D[4(l/16)+v][l%16]: tile row
// 4(l/16) + v, token l%16.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "../../include/bf16x_hip.h"
#include "bf16x_device.h"
#include "gemv_pipe.h"
#include "launch_common.h"

namespace bf16x {
namespace chunks {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kMaxTokens = 64;
constexpr int kPlanCols = 256;                 // columns per chunk of the chunk plan
// Byte offset that lies past the end of every buffer a kernel reads (the
// launcher keeps each stream below 2^31 bytes): a lane with nothing to load
// uses it and the buffer's range check returns zeros.
constexpr uint32_t kDead = 0x7FFFFF00u;

__device__ __forceinline__ int tile_chunk(int a, int q) { return (q ^ (a >> 2)) & 3; }

// The words of one atom as loaded (e kept 16-bit, as Atom::e: a 32-bit e is
// a widened copy of the load, which the compiler places at the loop latch,
// where it waits for every load in flight: the chunks requested ahead).
struct Raw {
  uint32_t s, m[7], d[3];
  uint16_t e;
};

// Per-lane byte offsets of one atom slot in the four streams (the atom's
// position at chunk 0); chunk c adds c * CA atoms through the scalar offset.
struct Slot {
  uint32_t s, m, d, e;
};

__device__ __forceinline__ void load_raw(__amdgpu_buffer_rsrc_t rs, __amdgpu_buffer_rsrc_t rm,
                                         __amdgpu_buffer_rsrc_t rd, __amdgpu_buffer_rsrc_t re, const Slot& v,
                                         uint32_t ca, Raw& t) {
  const u32x4 m03 = __builtin_amdgcn_raw_buffer_load_b128(rm, (int)v.m, (int)(ca * 28), 0);
  const u32x3 m46 = __builtin_amdgcn_raw_buffer_load_b96(rm, (int)(v.m + 16), (int)(ca * 28), 0);
  const u32x3 d02 = __builtin_amdgcn_raw_buffer_load_b96(rd, (int)v.d, (int)(ca * 12), 0);
  t.s = __builtin_amdgcn_raw_buffer_load_b32(rs, (int)v.s, (int)(ca * 4), 0);
  t.e = __builtin_amdgcn_raw_buffer_load_b16(re, (int)v.e, (int)(ca * 2), 0);
  const uint32_t a0 = m03.x, a1 = m03.y, a2 = m03.z, a3 = m03.w, a4 = m46.x, a5 = m46.y, a6 = m46.z;
  t.m[0] = a0; t.m[1] = a1; t.m[2] = a2; t.m[3] = a3; t.m[4] = a4; t.m[5] = a5; t.m[6] = a6;
  const uint32_t b0 = d02.x, b1 = d02.y, b2 = d02.z;
  t.d[0] = b0; t.d[1] = b1; t.d[2] = b2;
}

// Decoded atom in natural order: word k = element 2k | element 2k + 1 << 16.
__device__ __forceinline__ void decode_natural(const Raw& r, uint32_t (&n)[16]) {
  Atom t;
  t.s = r.s;
#pragma unroll
  for (int k = 0; k < 7; ++k) t.m[k] = r.m[k];
#pragma unroll
  for (int k = 0; k < 3; ++k) t.d[k] = r.d[k];
  t.e = (uint16_t)r.e;
  uint32_t p[16];                               // p[j] = element j | element j + 16 << 16
  decode_pairs(t, p);
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    n[k] = perm(p[2 * k + 1], p[2 * k], 0x05040100u);
    n[8 + k] = perm(p[2 * k + 1], p[2 * k], 0x07060302u);
  }
}

// Workgroup b owns weight rows [b R, min((b + 1) R, out_f)), R = rows_per_wg
// <= 16 RT.  (cp_off, cp_ent) is the chunk plan (bf16x_cplan_build): the
// entries of rows [r0, r1) with columns in [256 p, 256 (p + 1)) are
// cp_ent[cp_off[p out_f + r0] .. cp_off[p out_f + r1]).  Tokens: TG groups of
// TTW 16-token tiles; the 8 / TG waves of a group split the chunk's columns.
template <int RT, int CA, int TG, int TTW, bool EXACT, bool YF32>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void gemm_chunks_kernel(
    const uint16_t* __restrict__ x, int M, const uint32_t* __restrict__ sign, const uint32_t* __restrict__ mant,
    const uint32_t* __restrict__ delta, const uint16_t* __restrict__ emax2, const uint32_t* __restrict__ cp_off,
    const uint32_t* __restrict__ cp_ent, int out_f, int in_f, int rows_per_wg, void* __restrict__ y) {
  constexpr int ROWS = 16 * RT;
  constexpr int APL = RT * CA / 32;            // atoms per lane per chunk
  constexpr int WPG = kWaves / TG;             // waves per token group
  constexpr int KS = CA / WPG;                 // k-steps of 32 columns per wave per chunk
  constexpr int RPW = 64 * APL / CA;           // tile rows decoded per wave
  constexpr int RS = CA * 64 + 16;             // tile row stride, bytes
  constexpr int TILE = ROWS * RS;
  constexpr int PPC = CA * 32 / kPlanCols;     // plan chunks per chunk (entry runs per wave)
  // entry loads (of 64) per run; one at CA = 8 measured 1-2 us slower (the
  // loop for longer runs then runs in about 1 % of the chunks)
  constexpr int NBR = PPC == 1 ? 2 : 1;
  constexpr int RED = kWaves * RT * TTW * 64 * 16;
  constexpr int BIG = 2 * TILE > RED ? 2 * TILE : RED;
  static_assert(APL >= 1 && (64 * APL) % CA == 0 && KS >= 1 && CA % WPG == 0, "chunk shape");
  static_assert(PPC >= 1 && RPW <= 256 && (ROWS & (ROWS - 1)) == 0, "plan runs");
  // two tile slots (the partial products at the end), one trash word per lane
  __shared__ __attribute__((aligned(16))) uint8_t lds[BIG + 256];
  uint8_t* const trash = lds + BIG;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tg = wave / WPG, kp = wave % WPG; // token group, column part
  const int rbeg = blockIdx.x * rows_per_wg;
  const int rend = min(rbeg + rows_per_wg, out_f);
  if (rbeg >= rend) return;
  const int P = in_f >> 5;                     // atoms per row
  const int C = P / CA;                        // chunks

  // ---- decode slots: tile row lr[s], atom la[s] of the chunk
  const __amdgpu_buffer_rsrc_t rs_ = buf_rsrc(sign, (uint64_t)out_f * P * 4);
  const __amdgpu_buffer_rsrc_t rm_ = buf_rsrc(mant, (uint64_t)out_f * P * 28);
  const __amdgpu_buffer_rsrc_t rd_ = buf_rsrc(delta, (uint64_t)out_f * P * 12);
  const __amdgpu_buffer_rsrc_t re_ = buf_rsrc(emax2, (uint64_t)out_f * P * 2);
  Slot vs[APL];
#pragma unroll
  for (int s = 0; s < APL; ++s) {
    const int i = 64 * APL * wave + 64 * s + lane;
    const int row = rbeg + i / CA;
    const uint32_t at = (uint32_t)row * (uint32_t)P + (uint32_t)(i % CA);
    const bool live = row < rend;
    vs[s] = Slot{live ? at * 4 : kDead, live ? at * 28 : kDead, live ? at * 12 : kDead, live ? at * 2 : kDead};
  }
  // chunk c's atoms; chunks past the last one load nothing
  auto load_chunk = [&](int c, Raw (&t)[APL]) {
    const bool cl = c < C;
    const uint32_t ca = (uint32_t)(cl ? c : 0) * CA;
#pragma unroll
    for (int s = 0; s < APL; ++s) {
      const Slot v = cl ? vs[s] : Slot{kDead, kDead, kDead, kDead};
      load_raw(rs_, rm_, rd_, re_, v, ca, t[s]);
    }
  };

  // ---- plan: chunk c's entries of this wave's rows are PPC runs of the
  // chunk plan, run j = cp_ent[cp_off[p out_f + rw0] .. cp_off[p out_f +
  // rw1]) for plan chunk p = PPC c + j; the bounds are read with scalar
  // loads one chunk before the entries, the entries two chunks before their
  // chunk (NBR loads of 64 per run; a longer run loops over the rest)
  const int rw0 = min(rbeg + RPW * wave, rend), rw1 = min(rbeg + RPW * (wave + 1), rend);
  const __amdgpu_buffer_rsrc_t rpe = buf_rsrc(cp_ent, 0xFFFFFFFFull);
  struct Bounds {
    uint32_t beg[PPC], end[PPC];
  };
  auto load_bounds = [&](int c, Bounds& o) {
#pragma unroll
    for (int j = 0; j < PPC; ++j) {
      o.beg[j] = o.end[j] = 0u;
      if (EXACT && c < C && rw0 < rw1) {
        const int64_t p = (int64_t)(PPC * c + j) * out_f;
        o.beg[j] = cp_off[p + rw0];
        o.end[j] = cp_off[p + rw1];
      }
    }
  };
  struct Ents {
    uint32_t e[PPC * NBR];
    uint32_t valid;                            // bit j NBR + b: slot b of run j holds an entry
    bool more;                                 // a run is longer than NBR * 64 entries
  };
  // a slot past its run reads a word of the plan that exists (the run's
  // first, or entry 0) and is not written
  auto load_ents = [&](const Bounds& o, Ents& en) {
    en.valid = 0u;
    en.more = false;
    if constexpr (EXACT) {
      bool more = false;
#pragma unroll
      for (int j = 0; j < PPC; ++j) {
        const uint32_t n = o.end[j] - o.beg[j];
        more |= n > (uint32_t)(64 * NBR);
#pragma unroll
        for (int b = 0; b < NBR; ++b) {
          const uint32_t k = (uint32_t)(64 * b + lane);
          en.valid |= k < n ? (1u << (j * NBR + b)) : 0u;
          en.e[j * NBR + b] = __builtin_amdgcn_raw_buffer_load_b32(rpe, (int)((k < n ? k : 0u) * 4), (int)(o.beg[j] * 4), 0);
        }
      }
      en.more = more;
    }
  };

  // ---- x of token tile t of this wave's group, k-step ks of chunk c at
  // voffset vx[t] + ks * 64 and scalar offset c * CA * 64; tokens past M read
  // zeros, and so does every lane past the last chunk
  const __amdgpu_buffer_rsrc_t rx = buf_rsrc(x, (uint64_t)M * in_f * 2);
  uint32_t vx[TTW];
#pragma unroll
  for (int t = 0; t < TTW; ++t)
    vx[t] = (uint32_t)(16 * (TTW * tg + t) + (lane & 15)) * (uint32_t)in_f * 2 + (uint32_t)(lane >> 4) * 16 +
            (uint32_t)(kp * KS) * 64;
  auto load_x = [&](int c, bf16x8_t (&X)[TTW][KS]) {
    const bool cl = c < C;
    const uint32_t so = (uint32_t)(cl ? c : 0) * CA * 64;
#pragma unroll
    for (int t = 0; t < TTW; ++t)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rx, (int)(cl ? vx[t] + ks * 64 : kDead), (int)so, 0);
        X[t][ks] = __builtin_bit_cast(bf16x8_t, v);
      }
  };

  f32x4 acc[RT][TTW];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int t = 0; t < TTW; ++t) acc[rt][t] = f32x4{0.f, 0.f, 0.f, 0.f};

  // decode chunk c (atoms in t) into `tile`, then its plan entries over it
  auto decode = [&](int c, const Raw (&t)[APL], const Ents& en, uint8_t* tile) {
#pragma unroll
    for (int s = 0; s < APL; ++s) {
      const int i = 64 * APL * wave + 64 * s + lane, r = i / CA, a = i % CA;
      uint32_t n[16];
      decode_natural(t[s], n);
      uint8_t* rowp = tile + r * RS + a * 64;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *(u32x4*)(rowp + tile_chunk(a, q) * 16) = u32x4{n[4 * q], n[4 * q + 1], n[4 * q + 2], n[4 * q + 3]};
    }
    if constexpr (EXACT) {
      // entry: (row & 255) << 24 | (column within its 256-column plan chunk)
      // << 16 | exact bits; run j covers columns 256 j .. of this chunk
      auto patch_one = [&](int j, uint32_t e, bool live) {
        const int r = (int)(((e >> 24) - (uint32_t)rbeg) & 255u) & (ROWS - 1);
        const int col = kPlanCols * j + (int)((e >> 16) & 255u);
        const int a = (col >> 5) & (CA - 1), el = col & 31;
        uint8_t* dst = tile + r * RS + a * 64 + tile_chunk(a, el >> 3) * 16 + (el & 7) * 2;
        __asm__ volatile("" : "+v"(e));
        *(uint16_t*)(live ? dst : trash + lane * 4) = (uint16_t)(e & 0xFFFFu);
      };
#pragma unroll
      for (int j = 0; j < PPC; ++j)
#pragma unroll
        for (int b = 0; b < NBR; ++b) patch_one(j, en.e[j * NBR + b], (en.valid >> (j * NBR + b)) & 1u);
      // runs longer than NBR * 64 entries (rare): the rest, bounds read again
      if (en.more) {
        Bounds o;
        load_bounds(c, o);
        for (int j = 0; j < PPC; ++j)
          for (uint32_t e = o.beg[j] + 64 * NBR + (uint32_t)lane; e < o.end[j]; e += 64) patch_one(j, cp_ent[e], true);
      }
    }
  };

  // products of one chunk from `tile` with x in X
  auto multiply = [&](const bf16x8_t (&X)[TTW][KS], const uint8_t* tile) {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int a = KS * kp + ks, q = lane >> 4;
      const uint8_t* ap = tile + (lane & 15) * RS + a * 64 + tile_chunk(a, q) * 16;
      bf16x8_t A[RT];
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) A[rt] = *(const bf16x8_t*)(ap + rt * 16 * RS);
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int t = 0; t < TTW; ++t)
          acc[rt][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[rt], X[t][ks], acc[rt][t], 0, 0, 0);
    }
  };

  // Chunk c.  Requests chunk c + 2's entries (their bounds were read in the
  // previous chunk), chunk c + 1's x, chunk c + 2's atoms, in this order, and
  // the bounds of chunk c + 3.  Vector loads complete in issue order, so the
  // waits below (c's entries and atoms, c's x) never wait for the atoms of
  // c + 1 or c + 2.  Then chunk c is decoded into slot c & 1, the barrier,
  // the products.
  Raw A0[APL], A1[APL], A2[APL];
  Bounds B0{}, B1{}, B2{};
  Ents E0{}, E1{}, E2{};
  bf16x8_t X0[TTW][KS], X1[TTW][KS], X2[TTW][KS];
  auto iter = [&](int c, const Raw (&acur)[APL], Raw (&anx2)[APL], const Bounds& bnx2, Bounds& bnx3,
                  const Ents& ecur, Ents& enx2, const bf16x8_t (&xcur)[TTW][KS], bf16x8_t (&xnx1)[TTW][KS]) {
    load_ents(bnx2, enx2);
    load_x(c + 1, xnx1);
    load_chunk(c + 2, anx2);
    load_bounds(c + 3, bnx3);
    __builtin_amdgcn_sched_barrier(0);
    uint8_t* tile = lds + (c & 1) * TILE;
    decode(c, acur, ecur, tile);
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    multiply(xcur, tile);
  };

  // prologue: the requests of chunks -3 .. -1 that exist; set k of each kind
  // holds chunk c' with c' % 3 == k
  load_bounds(0, B0);
  load_bounds(1, B1);
  load_ents(B0, E0);
  load_chunk(0, A0);
  load_bounds(2, B2);
  load_ents(B1, E1);
  load_x(0, X0);
  load_chunk(1, A1);
  int c = 0;
  for (; c + 3 <= C; c += 3) {
    iter(c, A0, A2, B2, B0, E0, E2, X0, X1);
    iter(c + 1, A1, A0, B0, B1, E1, E0, X1, X2);
    iter(c + 2, A2, A1, B1, B2, E2, E1, X2, X0);
  }
  if (c < C) iter(c, A0, A2, B2, B0, E0, E2, X0, X1);
  if (c + 1 < C) iter(c + 1, A1, A0, B0, B1, E1, E0, X1, X2);

  // ---- partial products of a token group's waves, added in wave order
  __syncthreads();
  f32x4* red = (f32x4*)lds;                    // [wave][rt][t][lane]
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int t = 0; t < TTW; ++t) red[((wave * RT + rt) * TTW + t) * 64 + lane] = acc[rt][t];
  __syncthreads();
  constexpr int PER_WAVE = RT * TTW * 64;      // partial vectors per wave
  for (int u = tid; u < TG * PER_WAVE; u += kThreads) {
    const int g = u / PER_WAVE, v = u % PER_WAVE;
    const int rt = v / (TTW * 64), t = (v / 64) % TTW, l = v & 63;
    f32x4 sum = red[(g * WPG) * PER_WAVE + v];
#pragma unroll
    for (int w = 1; w < WPG; ++w) sum += red[(g * WPG + w) * PER_WAVE + v];
    const int token = 16 * (TTW * g + t) + (l & 15);
    const int row0 = rbeg + 16 * rt + 4 * (l >> 4);
    if (token < M) {
      const float vv[4] = {sum.x, sum.y, sum.z, sum.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        if (row0 + k < rend) {
          if constexpr (YF32) ((float*)y)[(int64_t)token * out_f + row0 + k] = vv[k];
          else ((uint16_t*)y)[(int64_t)token * out_f + row0 + k] = (uint16_t)f32_to_bf16_rne(vv[k]);
        }
      }
    }
  }
}

// ---- chunk plan from the row plan.  Plan chunk p is columns [256 p, 256
// (p + 1)); its entries are grouped by (p, row), rows in order, each row's in
// column order, so the entries of consecutive rows in one plan chunk are one
// run.  One thread per (row r, plan chunk p): its row's entries in p by
// binary search (a row's entries are sorted by column), the count in pass 1,
// the entries re-encoded as (r & 255) << 24 | (column - 256 p) << 16 | bits
// in pass 2, after a scan of the counts has made them offsets.
template <bool FILL>
__global__ __launch_bounds__(256) void cplan_pass_kernel(const uint32_t* __restrict__ tile_off,
                                                         const uint32_t* __restrict__ tile_ent, int64_t out_f, int C5,
                                                         uint32_t* __restrict__ cp_off,
                                                         uint32_t* __restrict__ cp_ent) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= out_f * C5) return;
  const int64_t r = i % out_f, p = i / out_f;   // i = p out_f + r: the output index
  auto lower = [&](uint32_t col) {              // first entry of row r at column >= col
    uint32_t lo = tile_off[r], hi = tile_off[r + 1];
    while (lo < hi) {
      const uint32_t mid = lo + (hi - lo) / 2;
      if ((tile_ent[mid] >> 16) < col) lo = mid + 1;
      else hi = mid;
    }
    return lo;
  };
  const uint32_t b = lower((uint32_t)p * kPlanCols), e = lower((uint32_t)(p + 1) * kPlanCols);
  if constexpr (!FILL) {
    cp_off[i] = e - b;
  } else {
    const uint32_t dst = cp_off[i];
    for (uint32_t k = b; k < e; ++k) {
      const uint32_t v = tile_ent[k];
      cp_ent[dst + (k - b)] = ((uint32_t)(r & 255) << 24) | (((v >> 16) - (uint32_t)p * kPlanCols) << 16) |
                              (v & 0xFFFFu);
    }
  }
}

// Rows per workgroup: the weight's rows spread evenly over one workgroup per
// CU, at most 64.
int rows_per_wg(int64_t out_f) {
  const int cus = device_cus() > 0 ? device_cus() : 256;
  return (int)std::min<int64_t>(64, std::max<int64_t>(1, (out_f + cus - 1) / cus));
}

}  // namespace chunks
}  // namespace bf16x

using namespace bf16x;

extern "C" int64_t bf16x_cplan_size(int64_t out_f, int64_t in_f) {
  if (out_f <= 0 || in_f <= 0 || in_f % chunks::kPlanCols != 0 || in_f > kPlanTileCols) return BF16X_ESHAPE;
  return out_f * (in_f / chunks::kPlanCols) + 1;
}

extern "C" int bf16x_cplan_build(const uint32_t* tile_off, const uint32_t* tile_ent, int64_t out_f, int64_t in_f,
                                 uint32_t* cp_off, uint32_t* cp_ent, bf16x_stream_t stream) {
  if (!tile_off || !tile_ent || !cp_off || !cp_ent) return BF16X_EARG;
  const int64_t n = bf16x_cplan_size(out_f, in_f);
  if (n < 0) return (int)n;
  if (n > (int64_t)INT32_MAX) return BF16X_ESHAPE;
  const int C5 = (int)(in_f / chunks::kPlanCols);
  const unsigned blocks = (unsigned)((n - 1 + 255) / 256);
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL((chunks::cplan_pass_kernel<false>), dim3(blocks), dim3(256), 0, st, tile_off, tile_ent, out_f,
                     C5, cp_off, cp_ent);
  scan_offsets(cp_off, n - 1, st);
  hipLaunchKernelGGL((chunks::cplan_pass_kernel<true>), dim3(blocks), dim3(256), 0, st, tile_off, tile_ent, out_f,
                     C5, cp_off, cp_ent);
  return launch_status();
}

extern "C" int bf16x_gemm_chunks(const void* x, int32_t x_dtype, int64_t M, const int32_t* sign, int64_t n_sign,
                                 const int32_t* mant, int64_t n_mant, const int32_t* delta, int64_t n_delta,
                                 const uint8_t* emax, int64_t n_emax, const uint32_t* cp_off,
                                 const uint32_t* cp_ent, int64_t out_f, int64_t in_f, int32_t sub, int32_t mode,
                                 void* y, int32_t y_dtype, bf16x_stream_t stream) {
  using namespace bf16x::chunks;
  if (!x || !sign || !mant || !delta || !emax || !y) return BF16X_EARG;
  if (mode != BF16X_EXACT && mode != BF16X_SATURATED) return BF16X_EARG;
  const bool ex = mode == BF16X_EXACT;
  if (ex && (!cp_off || !cp_ent)) return BF16X_EARG;
  if (x_dtype != BF16X_BF16 || (y_dtype != BF16X_BF16 && y_dtype != BF16X_F32)) return BF16X_EDTYPE;
  const int rc = check_dict(out_f, in_f, sub, n_sign, n_mant, n_delta, n_emax);
  if (rc) return rc;
  if (M <= 0 || M > kMaxTokens || in_f % kPlanCols != 0 || in_f > kPlanTileCols) return BF16X_ESHAPE;
  // every stream and x below kDead bytes (the offset of lanes that load nothing)
  if (out_f * (in_f >> 5) * 28 >= (int64_t)kDead || M * in_f * 2 >= (int64_t)kDead) return BF16X_ESHAPE;
  if (!aligned4(sign) || !aligned4(mant) || !aligned4(delta) || !aligned2(emax) || !aligned16(x) || !aligned4(y))
    return BF16X_EARG;
  const int rpw = rows_per_wg(out_f);
  const int64_t grid = (out_f + rpw - 1) / rpw;
  // Row tiles for rpw rows, and atoms per row and chunk (CA atoms = 32 CA
  // columns, in_f % (32 CA) == 0).  One 16-row tile takes 1024-column chunks
  // (one atom per lane) up to 32 tokens (more would hold x of 32 k-steps per
  // wave), else two tiles with rows past rpw left empty; two tiles take 512
  // columns; four take 256 (BF16X_TUNE_CHUNK_ATOMS = 16: 512 up to 32
  // tokens; measured 1-2 us slower at 14336x4096 and 14336x2048).
  int rt = rpw <= 16 ? 1 : rpw <= 32 ? 2 : 4;
  if (rt == 1 && (in_f % 1024 != 0 || M > 32)) rt = 2;
  if (rt == 2 && in_f % 512 != 0) rt = 4;
  const int ca4 = (tuning(BF16X_TUNE_CHUNK_ATOMS) == 16 && M <= 32 && in_f % 512 == 0) ? 16 : 8;
  const int tk = M <= 16 ? 0 : M <= 32 ? 1 : 2;  // token layout: (groups, tiles per wave) (1,1), (1,2), (2,2)
  const uint32_t *po = ex ? cp_off : nullptr, *pe = ex ? cp_ent : nullptr;
  hipStream_t st = (hipStream_t)stream;
#define BF16X_CH(RT_, CA_, TG_, TTW_, EX_, YF_)                                                             \
  hipLaunchKernelGGL((gemm_chunks_kernel<RT_, CA_, TG_, TTW_, EX_, YF_>), dim3((unsigned)grid), dim3(kThreads), \
                     0, st, (const uint16_t*)x, (int)M, (const uint32_t*)sign, (const uint32_t*)mant,          \
                     (const uint32_t*)delta, (const uint16_t*)emax, po, pe, (int)out_f, (int)in_f, rpw, y)
#define BF16X_CH_MODE(RT_, CA_, TG_, TTW_)                                                                  \
  do {                                                                                                      \
    if (ex) { if (y_dtype == BF16X_F32) BF16X_CH(RT_, CA_, TG_, TTW_, true, true);                          \
              else BF16X_CH(RT_, CA_, TG_, TTW_, true, false); }                                            \
    else { if (y_dtype == BF16X_F32) BF16X_CH(RT_, CA_, TG_, TTW_, false, true);                            \
           else BF16X_CH(RT_, CA_, TG_, TTW_, false, false); }                                              \
  } while (0)
#define BF16X_CH_TK(RT_, CA_)                                                                               \
  do {                                                                                                      \
    if (tk == 0) BF16X_CH_MODE(RT_, CA_, 1, 1);                                                             \
    else if (tk == 1) BF16X_CH_MODE(RT_, CA_, 1, 2);                                                        \
    else BF16X_CH_MODE(RT_, CA_, 2, 2);                                                                     \
  } while (0)
#define BF16X_CH_TK32(RT_, CA_)                                                                             \
  do {                                                                                                      \
    if (tk == 0) BF16X_CH_MODE(RT_, CA_, 1, 1);                                                             \
    else BF16X_CH_MODE(RT_, CA_, 1, 2);                                                                     \
  } while (0)
  if (rt == 1) BF16X_CH_TK32(1, 32);
  else if (rt == 2) BF16X_CH_TK(2, 16);
  else if (ca4 == 8) BF16X_CH_TK(4, 8);
  else BF16X_CH_TK32(4, 16);
#undef BF16X_CH_TK32
#undef BF16X_CH_TK
#undef BF16X_CH_MODE
#undef BF16X_CH
  return launch_status();
}
