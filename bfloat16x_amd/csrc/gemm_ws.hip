// Fused decode + GEMM for many rows (prefill) on gfx950: wave-specialised
// workgroups.
//
// Replaces _bf16x_gemm_fused_kernel / bf16x_fused_gemm (bf16x_gemm_fused.py:31-114)
// for M of a few hundred rows and more: y[M, N] = x[M, K] . W[N, K]^T with W
// decoded on the fly, fp32 accumulation.  SATURATED reproduces the reference
// kernel's numerics (code 7 -> exponent emax-7, bf16x_gemm_fused.py:84-87);
// EXACT writes the overflow plan's entries over the decoded tile and
// multiplies by the lossless weight.
//
// Measured on MI355X, and the reason for the structure:
//  * VALU instructions in an MFMA wave's own instruction stream do not run
//    under its MFMAs (the step time is close to the sum of both), but an
//    MFMA wave and a VALU wave sharing a SIMD overlap.  Decoding a W element
//    takes ~5 VALU lane-ops, so the decode runs in waves of its own.
//  * LDS sustains ~70 B/clk per CU for writes (ds_write or direct loads) and
//    130-220 B/clk for 16-byte reads.  Register budget (two waves per SIMD,
//    256 registers each) limits an MFMA wave to 128 accumulators.
//
// A workgroup is 8 waves and owns an output tile of 256 x rows (tokens) by 128
// W rows over a range of 64-column K steps (all of K, or one split of it when
// the tile count alone leaves CUs idle; split partials are fp32 and summed in
// split order by a second kernel).
//  * Waves 4-7 decode.  Wave 4+p decodes rows 32p .. 32p+31 of the W tile at
//    each step (lane l: row l%32, atom l/32 of the step), writes them to LDS
//    in natural order and writes the EXACT plan entries of the same rows over
//    them (one wave: its LDS writes land in order).  Atoms and plan entries
//    are requested two steps ahead into registers, the plan offsets one step
//    before their entries.
//  * Waves 0-3 (one per SIMD) issue the MFMAs: wave c owns tokens
//    64c .. 64c+63 and all 128 W rows, 2 x 4 accumulators of
//    v_mfma_f32_32x32x16_bf16.  Each token row belongs to one wave, so x does
//    not pass through LDS: a wave requests its x operands of the next step
//    (8 16-byte loads per lane) straight into registers.  x is first
//    rewritten in MFMA operand order (x_op_kernel, into the workspace), so
//    each of those loads reads 1 KB contiguous: loading the operands from
//    row-major x touches 32 rows per instruction, and the vector memory
//    pipeline's rate in cache lines per clock, not bytes, then set the step
//    time.  W operands come from LDS; each k-quarter first requests the next
//    quarter's 4, then runs its 8 MFMAs.
//  * LDS traffic is the W tile only: 16 KB written and 64 KB read per step.
//    With the x tile staged in LDS as well (144 KB per step), the kernel ran
//    at half this speed: LDS, not the MFMAs, set the step time.
//  * LDS: 2 W slots of 16 KB; one barrier per step.  Tile rows are 128
//    bytes; 16-byte chunk c of row r sits at c ^ ((r >> 1) & 7), so 16 lanes
//    reading one logical chunk of 16 consecutive rows touch 16 different
//    16-byte bank groups (64 banks).
//  * MFMA k-slots: in k-quarter q, lanes 0-31 hold 8 columns of the step's
//    first half and lanes 32-63 the same 8 of its second half, for x (A
//    operand) and W (B operand) alike: columns 4q .. 4q+3 and 16+4q .. 19+4q
//    of the half, interleaved (the order the decode leaves them in, see
//    chunk_of).  Result register v of lane l is D[8(v/4) + 4(l/32) + v%4][l%32]:
//    token row, W row.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "../../include/bf16x_hip.h"
#include "bf16x_device.h"
#include "launch_common.h"

namespace bf16x {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kStep = 64;              // K columns per step
constexpr int kRowB = 128;             // bytes of one LDS tile row (64 bf16)
constexpr int kBM = 256;               // tokens per tile
constexpr int kBN = 128;               // W rows per tile
constexpr int kWSlot = kBN * kRowB;    // 16 KB

__device__ __forceinline__ int swz(int row, int chunk) { return chunk ^ ((row >> 1) & 7); }

// K order inside a 64-column step.  decode_pairs leaves element j of an atom
// in the low half of word j and element 16 + j in the high half; W is stored
// as decoded (no permute), so 16-byte chunk c of atom h (words 4c .. 4c+3)
// holds atom columns 4c, 16+4c, 4c+1, 17+4c, 4c+2, 18+4c, 4c+3, 19+4c.  x_op
// writes x's operand chunks in the same column order, so both MFMA operands
// see one permutation of K.  Column c (0..63) of a step sits in chunk
// chunk_of(c) of the step's 8, at bf16 position pos_of(c).
__device__ __forceinline__ int chunk_of(int c) { return ((c >> 5) << 2) | ((c >> 2) & 3); }
__device__ __forceinline__ int pos_of(int c) { return ((c & 3) << 1) | ((c >> 4) & 1); }

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, uint64_t bytes) {
  const uint32_t n = bytes > 0xFFFFFFFFull ? 0xFFFFFFFFu : (uint32_t)bytes;
  return __builtin_amdgcn_make_buffer_rsrc((void*)p, (short)0, (int)n, 0x00020000);
}

// the words of one atom as loaded (emax as the dword holding both atoms of the step)
struct Raw {
  uint32_t s, m[7], d[3], ew;
};
// a GGUF block as loaded: the 48 bytes from the dword at or below it
struct RawG {
  u32x4 q0, q1, q2;
};

// Block -> work.  Blocks [0, full) each own one output tile over all of K
// (tiles 0 .. full-1); the remaining blocks split K for the last `ltiles`
// tiles in `lunits`-unit ranges (units: steps, or four-step groups) and write
// fp32 partials, summed by ws_tile_reduce_kernel.  full is a multiple of the
// resident block count, so the split blocks fill the last round.  Within
// each range the order is XCD-aware: blocks go round-robin over 8 XCDs, and
// each XCD gets a contiguous run of tiles, M fastest, so the M tiles that
// share a W tile run on one XCD at the same time and share its L2.
struct WsGrid {
  int mtiles, full, ltiles, lunits;
  int bm;         // tokens per tile (kBM)
};
struct WsWork {
  int64_t m0, n0;
  int u0, nu;     // first unit and unit count of this block
  int lt;         // split tile index (0 .. ltiles-1), or -1 for a full tile
  int kb;         // K range of a split tile
};
__device__ __forceinline__ int xcd_order(int b, int nb) {
  const int per = nb / 8, extra = nb - per * 8;
  return nb >= 8 ? ((b & 7) * per + min(b & 7, extra) + (b >> 3)) : b;
}
__device__ __forceinline__ WsWork ws_work(const WsGrid& g, int units) {
  const int nb = (int)gridDim.x, b = (int)blockIdx.x;
  WsWork w;
  int tile;
  if (b < g.full) {
    tile = xcd_order(b, g.full);
    w.lt = -1; w.kb = 0; w.u0 = 0; w.nu = units;
  } else {
    const int lb = xcd_order(b - g.full, nb - g.full);
    w.lt = lb % g.ltiles; w.kb = lb / g.ltiles;
    tile = g.full + w.lt;
    w.u0 = w.kb * g.lunits;
    w.nu = min(g.lunits, units - w.u0);
  }
  w.m0 = (int64_t)(tile % g.mtiles) * g.bm;
  w.n0 = (int64_t)(tile / g.mtiles) * kBN;
  return w;
}

// The output tile from the MFMA waves' accumulators: register v of lane l ->
// token row 8(v/4) + 4(l/32) + v%4, W row l%32.  A split tile's partial goes
// to its own BM x 128 fp32 tile of `part` (all of it: rows past M and
// columns past out_f hold zeros), in K-range order.  NI: 32-token tiles per
// wave (the wave owns tokens NI 32 wave .. + NI 32 - 1 of the tile).
template <bool YF32, int NI = 2>
__device__ __forceinline__ void ws_store(const f32x16 (&acc)[NI][4], const WsWork& w, int wave, int lane, int64_t M,
                                         int64_t out_f, int ltiles, void* __restrict__ y, float* __restrict__ part) {
  constexpr int BM = 4 * 32 * NI;
  const int lr = lane & 31, h = lane >> 5;
  if (w.lt >= 0) {
    float* pt = part + ((int64_t)w.kb * ltiles + w.lt) * (BM * kBN);
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int r = wave * 32 * NI + i * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
          pt[r * kBN + jj * 32 + lr] = acc[i][jj][v];
        }
    return;
  }
#pragma unroll
  for (int i = 0; i < NI; ++i) {
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int64_t col = w.n0 + jj * 32 + lr;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t row = w.m0 + wave * 32 * NI + i * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
        if (row < M && col < out_f) {
          if constexpr (YF32) ((float*)y)[row * out_f + col] = acc[i][jj][v];
          else ((uint16_t*)y)[row * out_f + col] = (uint16_t)f32_to_bf16_rne(acc[i][jj][v]);
        }
      }
    }
  }
}

// GG: W is GGUF half-blocks (`blocks`, 46 bytes per 32 elements, row-major;
// the dict stream pointers are unused), decoded with the zero marker
// (bf16x_gguf_block.py:76-87).  Otherwise W is the packed dict.
template <bool GG, bool EXACT, bool YF32>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void gemm_ws_kernel(
    const uint16_t* __restrict__ x, int64_t M, const uint32_t* __restrict__ sign,
    const uint32_t* __restrict__ mant, const uint32_t* __restrict__ delta, const uint16_t* __restrict__ emax2,
    const uint8_t* __restrict__ blocks, const uint32_t* __restrict__ kp_off, const uint32_t* __restrict__ kp_ent,
    int64_t out_f, int64_t in_f, WsGrid grid, void* __restrict__ y, float* __restrict__ part) {
  __shared__ __attribute__((aligned(16))) uint8_t wlds[2 * kWSlot];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  const int S = (int)(in_f >> 6);
  const WsWork wk = ws_work(grid, S);           // units are steps
  const int64_t m0 = wk.m0, n0 = wk.n0;
  const int s0 = wk.u0;
  const int n = wk.nu;                          // steps of this block (>= 1)

  if (wave >= 4) {
    // ===================== staging waves =====================
    const int pw = wave - 4;                    // 0..3
    const int64_t P = in_f >> 5;                // atoms per row
    const int r = 32 * pw + (lane & 31), a = lane >> 5;
    using RawT = typename std::conditional<GG, RawG, Raw>::type;
    const uint64_t wat = (uint64_t)(out_f - n0) * P;   // atoms from the tile's first row
    __amdgpu_buffer_rsrc_t rs_, rm_, rd_, re_, rb_;
    uint32_t vo_s = 0, vo_m = 0, vo_d = 0, vo_e = 0, vo_b = 0, sh = 0;
    // rows past out_f read zeros (buffer range check on the vector offset);
    // their outputs are not stored
    const uint32_t av = (uint32_t)(r * P) + (uint32_t)a;
    if constexpr (GG) {
      // the tile's first block starts at a multiple of 4 bytes (n0 % 128 == 0);
      // the range is the rest of the blocks rounded up to 4 bytes, which the
      // caller guarantees readable.  Block (r, 2s + a) is at av * 46 + s * 92:
      // its offset modulo 4 (0 or 2) does not depend on s.
      rb_ = rsrc(blocks + (uint64_t)n0 * P * 46, (wat * 46 + 3) & ~3ull);
      vo_b = av * 46;
      sh = (vo_b & 2u) * 8u;
      vo_b &= ~3u;
    } else {
      rs_ = rsrc(sign + n0 * P, wat * 4);
      rm_ = rsrc(mant + n0 * P * 7, wat * 28);
      rd_ = rsrc(delta + n0 * P * 3, wat * 12);
      re_ = rsrc(emax2 + n0 * P, wat * 2);
      vo_s = av * 4; vo_m = av * 28; vo_d = av * 12; vo_e = (uint32_t)(r * P) * 2;
    }
    auto load_atoms = [&](int j, RawT& t) {
      const uint32_t s = (uint32_t)(s0 + min(j, n - 1));
      if constexpr (GG) {
        t.q0 = __builtin_amdgcn_raw_buffer_load_b128(rb_, (int)vo_b, (int)(s * 92), 0);
        t.q1 = __builtin_amdgcn_raw_buffer_load_b128(rb_, (int)(vo_b + 16), (int)(s * 92), 0);
        t.q2 = __builtin_amdgcn_raw_buffer_load_b128(rb_, (int)(vo_b + 32), (int)(s * 92), 0);
      } else {
        const u32x4 m03 = __builtin_amdgcn_raw_buffer_load_b128(rm_, (int)vo_m, (int)(s * 56), 0);
        const u32x3 m46 = __builtin_amdgcn_raw_buffer_load_b96(rm_, (int)(vo_m + 16), (int)(s * 56), 0);
        const u32x3 d02 = __builtin_amdgcn_raw_buffer_load_b96(rd_, (int)vo_d, (int)(s * 24), 0);
        t.s = __builtin_amdgcn_raw_buffer_load_b32(rs_, (int)vo_s, (int)(s * 8), 0);
        // the full dword (both atoms' emax pairs) is kept raw until the decode:
        // a value computed from a load at the load site makes the compiler wait
        // for it there
        t.ew = __builtin_amdgcn_raw_buffer_load_b32(re_, (int)vo_e, (int)(s * 4), 0);
        const uint32_t c0 = m03.x, c1 = m03.y, c2 = m03.z, c3 = m03.w, c4 = m46.x, c5 = m46.y, c6 = m46.z;
        t.m[0] = c0; t.m[1] = c1; t.m[2] = c2; t.m[3] = c3; t.m[4] = c4; t.m[5] = c5; t.m[6] = c6;
        const uint32_t e0 = d02.x, e1 = d02.y, e2 = d02.z;
        t.d[0] = e0; t.d[1] = e1; t.d[2] = e2;
      }
    };
    const int wst = r * kRowB;                  // this lane's W row in slot 0
    auto store_w = [&](const RawT& w, int slot) {
      uint32_t p[16];
      if constexpr (GG) {
        decode_pairs<true>(gguf_atom(GgufRaw{w.q0, w.q1, w.q2, sh}), p);
      } else {
        Atom t;
        t.s = w.s;
#pragma unroll
        for (int i = 0; i < 7; ++i) t.m[i] = w.m[i];
#pragma unroll
        for (int i = 0; i < 3; ++i) t.d[i] = w.d[i];
        t.e = (uint16_t)(w.ew >> (16 * a));
        decode_pairs(t, p);
      }
      // chunk c = pairs 4c .. 4c+3 as decoded: K order kchunk(c), as x_op writes x
#pragma unroll
      for (int c = 0; c < 4; ++c)
        *(u32x4*)(wlds + wst + slot * kWSlot + swz(r, 4 * a + c) * 16) =
            u32x4{p[4 * c], p[4 * c + 1], p[4 * c + 2], p[4 * c + 3]};
    };

    // EXACT plan: run of this wave's 32-row group at step s
    const int64_t G = (out_f + 31) / 32, G2 = 2 * G;
    const int64_t g = min(n0 / 32 + pw, G);
    uint32_t kp_total = 0;
    if constexpr (EXACT) kp_total = kp_off[S * G2];
    const __amdgpu_buffer_rsrc_t rent = rsrc(kp_ent, (uint64_t)kp_total * 4);
    const __amdgpu_buffer_rsrc_t roff = rsrc(kp_off, ((uint64_t)S * G2 + 1) * 4);
    const uint32_t ob = (uint32_t)(2 * g) * 4, oe = (uint32_t)min(2 * g + 2, G2) * 4;
    struct Off { uint32_t beg, end; };
    struct Ent { uint32_t beg, end, e0, e1; };
    auto load_off = [&](int j, Off& o) {
      const uint32_t s = (uint32_t)(s0 + min(j, n - 1));
      o.beg = __builtin_amdgcn_raw_buffer_load_b32(roff, (int)ob, (int)(s * G2 * 4), 0);
      o.end = __builtin_amdgcn_raw_buffer_load_b32(roff, (int)oe, (int)(s * G2 * 4), 0);
    };
    auto load_ent = [&](const Off& o, Ent& e) {
      e.beg = __builtin_amdgcn_readfirstlane(o.beg);
      e.end = __builtin_amdgcn_readfirstlane(o.end);
      e.e0 = __builtin_amdgcn_raw_buffer_load_b32(rent, (int)((e.beg + lane) * 4), 0, 0);
      e.e1 = __builtin_amdgcn_raw_buffer_load_b32(rent, (int)((e.beg + lane + 64) * 4), 0, 0);
    };
    // The entry is used outside the branch first (the empty asm), so the
    // compiler waits for its load there with an exact count: a loaded value
    // first used under a divergent branch makes it wait for every
    // outstanding load.
    auto patch_one = [&](uint32_t e, int slot, bool live) {
      const int rr = (int)(e >> 22) & (kBN - 1), c = (int)(e >> 16) & 63;
      const uint32_t dst = (uint32_t)(slot * kWSlot + rr * kRowB + swz(rr, chunk_of(c)) * 16 + pos_of(c) * 2);
      __asm__ volatile("" : "+v"(e));
      if (live) *(uint16_t*)(wlds + dst) = (uint16_t)(e & 0xFFFFu);
    };
    auto patch = [&](const Ent& e, int slot) {
      patch_one(e.e0, slot, e.beg + lane < e.end);
      patch_one(e.e1, slot, e.beg + lane + 64 < e.end);
      for (uint32_t k = e.beg + 128 + lane; k < e.end; k += 64)   // dense runs (rare)
        patch_one(kp_ent[k], slot, true);
    };

    RawT A0, A1;
    Off O0{}, O1{};
    Ent E0{}, E1{};
    // prologue: the requests of steps 0 and 1 (atoms, plan entries), step 0
    // decoded, the requests of step 2.  The loads in flight at the loop entry
    // are then the requests of 1 and 2, the pattern at the top of every
    // iteration, so the waits the compiler derives hold on both paths into
    // the loop
    if constexpr (EXACT) {
      load_off(0, O0);
      load_off(1, O1);
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (EXACT) { load_ent(O0, E0); load_off(2, O0); }
    load_atoms(0, A0);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (EXACT) { load_ent(O1, E1); load_off(3, O1); }
    load_atoms(1, A1);
    __builtin_amdgcn_sched_barrier(0);
    store_w(A0, 0);
    if constexpr (EXACT) patch(E0, 0);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (EXACT) { load_ent(O0, E0); load_off(4, O0); }
    load_atoms(2, A0);
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();

    // iteration j: step j + 1 decoded (W slot (j + 1) & 1) from its register
    // set, then the atoms of j + 3 requested into that set with the plan
    // entries of j + 3 and the offsets of j + 5
    auto iter = [&](int j, RawT& at, Off& o, Ent& e, int slot) {
      store_w(at, slot);
      if constexpr (EXACT) patch(e, slot);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (EXACT) { load_ent(o, e); load_off(j + 5, o); }
      load_atoms(j + 3, at);
      __builtin_amdgcn_sched_barrier(0);
      __syncthreads();
    };
    int j = 0;
    for (; j + 1 < n; j += 2) {
      iter(j, A1, O1, E1, 1);
      iter(j + 1, A0, O0, E0, 0);
    }
    if (j < n) iter(j, A1, O1, E1, 1);
    return;
  }

  // ===================== MFMA waves =====================
  const int lr = lane & 31, h = lane >> 5;
  // x operand of token tile i, k-quarter q at step s: 1 KB of x in operand
  // order (x_op_kernel), lane l's 16 bytes at l * 16.  The block's tiles
  // start at tile m0 / 32; rows past M hold zeros (outputs not stored).
  const int64_t S64 = S;
  const __amdgpu_buffer_rsrc_t rx_ = rsrc(x + m0 * in_f, (uint64_t)(((M + 31) / 32) * 32 - m0) * (uint64_t)in_f * 2);
  const uint32_t vx0 = (uint32_t)(2 * wave * S64 * 4096 + lane * 16);
  const uint32_t vx1 = vx0 + (uint32_t)(S64 * 4096);
  // the x operands of one step: [token tile][k-quarter]
  auto load_x = [&](int j, bf16x8_t (&X)[2][4]) {
    const uint32_t ks = (uint32_t)(s0 + min(j, n - 1)) * 4096;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rx_, (int)((i ? vx1 : vx0) + q * 1024), (int)ks, 0);
        X[i][q] = __builtin_bit_cast(bf16x8_t, v);
      }
  };
  // W operand of W tile jj, k-quarter q (the swizzle term depends on lr only)
  uint32_t wo[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) wo[q] = (uint32_t)(lr * kRowB + swz(lr, 4 * h + q) * 16);
  auto load_w = [&](int q, int ws, bf16x8_t (&wb)[4]) {
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) wb[jj] = *(const bf16x8_t*)(wlds + wo[q] + ws * kWSlot + jj * 32 * kRowB);
  };
  f32x16 acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int jj = 0; jj < 4; ++jj)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][jj][v] = 0.f;
  auto mfma = [&](int t, const bf16x8_t (&X)[2][4], int q, const bf16x8_t (&wb)[4]) {
    const int i = t >> 2, jj = t & 3;
    acc[i][jj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(X[i][q], wb[jj], acc[i][jj], 0, 0, 0);
  };
#define BF16X_SG(mask, cnt) __builtin_amdgcn_sched_group_barrier(mask, cnt, 0)
  bf16x8_t X0[2][4], X1[2][4], W0[4], W1[4];
  // one step from W slot ws with x in X; x of step j + 1 requested into Xn
  // (the set the previous step used) at the start
  auto step = [&](int j, int ws, const bf16x8_t (&X)[2][4], bf16x8_t (&Xn)[2][4]) {
    load_x(j + 1, Xn);
    // quarter 0: the next quarter's W reads, then 8 MFMAs
    load_w(1, ws, W1);
#pragma unroll
    for (int t = 0; t < 8; ++t) mfma(t, X, 0, W0);
    BF16X_SG(0x020, 8);
    BF16X_SG(0x100, 4);
    BF16X_SG(0x008, 8);
    __builtin_amdgcn_sched_barrier(0);
    load_w(2, ws, W0);
#pragma unroll
    for (int t = 0; t < 8; ++t) mfma(t, X, 1, W1);
    BF16X_SG(0x100, 4);
    BF16X_SG(0x008, 8);
    __builtin_amdgcn_sched_barrier(0);
    load_w(3, ws, W1);
#pragma unroll
    for (int t = 0; t < 8; ++t) mfma(t, X, 2, W0);
    BF16X_SG(0x100, 4);
    BF16X_SG(0x008, 8);
    __builtin_amdgcn_sched_barrier(0);
    // last quarter: 4 MFMAs, the barrier, the next step's quarter-0 W reads
    // under the other 4
#pragma unroll
    for (int t = 0; t < 4; ++t) mfma(t, X, 3, W1);
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    load_w(0, ws ^ 1, W0);
#pragma unroll
    for (int t = 4; t < 8; ++t) mfma(t, X, 3, W1);
    BF16X_SG(0x100, 4);
    BF16X_SG(0x008, 4);
    __builtin_amdgcn_sched_barrier(0);
  };
#undef BF16X_SG
  load_x(0, X0);
  __syncthreads();
  load_w(0, 0, W0);
  int j = 0;
  for (; j + 1 < n; j += 2) {
    step(j, 0, X0, X1);
    step(j + 1, 1, X1, X0);
  }
  if (j < n) step(j, 0, X0, X1);
  ws_store<YF32>(acc, wk, wave, lane, M, out_f, grid.ltiles, y, part);
}

// ---------------------------------------------------------------------------
// Four-step groups (in_f % 256 == 0): the kernel above with the W tile of one
// barrier interval 256 columns wide (64 KB per slot, two slots), so that the
// decode waves read runs of consecutive atoms of a row.  In round i (0..3)
// lane l of decode wave 4 + p takes tile row 32p + 8i + l/8 and atom l%8 of
// the group: a load instruction reads 8 rows x 8 consecutive atoms (368
// contiguous bytes of a GGUF row, 224 of a mantissa stream) instead of 32
// rows x 2 atoms, about 1.7x fewer cache lines per instruction (a timing copy
// of the one-step kernel with this access pattern ran 11-24 % faster).  Each
// round's registers are refilled with the next group's atoms as soon as they
// are decoded, so one set of 4 rounds is in flight while the other is decoded.
// Tile rows are 512 bytes; 16-byte chunk c of row r sits at
// c ^ (((c >> 4) & 1) << 1) ^ (r & 15): the MFMA waves' reads (16 rows, one
// chunk) and the decode waves' writes (2 rows x 8 atoms, one chunk of each)
// each touch 16 different 16-byte bank groups.  The MFMA waves run the
// one-step kernel's step four times per barrier.
// ---------------------------------------------------------------------------
constexpr int kGroup = 4;                    // 64-column steps per group
constexpr int kRowB4 = kGroup * kRowB;       // 512 bytes per tile row
constexpr int kWSlot4 = kBN * kRowB4;        // 64 KB

__device__ __forceinline__ int swz4(int row, int chunk) { return chunk ^ (((chunk >> 4) & 1) << 1) ^ (row & 15); }

template <bool GG, bool EXACT, bool YF32>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void gemm_ws4_kernel(
    const uint16_t* __restrict__ x, int64_t M, const uint32_t* __restrict__ sign,
    const uint32_t* __restrict__ mant, const uint32_t* __restrict__ delta, const uint16_t* __restrict__ emax2,
    const uint8_t* __restrict__ blocks, const uint32_t* __restrict__ kp_off, const uint32_t* __restrict__ kp_ent,
    int64_t out_f, int64_t in_f, WsGrid grid, void* __restrict__ y, float* __restrict__ part) {
  // two W slots, then 256 bytes where the plan patch lanes with no entry write
  __shared__ __attribute__((aligned(16))) uint8_t wlds[2 * kWSlot4 + 256];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  const int S = (int)(in_f >> 6);
  const WsWork wk = ws_work(grid, S / kGroup);  // units are groups
  const int64_t m0 = wk.m0, n0 = wk.n0;
  const int g0 = wk.u0;
  const int ng = wk.nu;                         // groups of this block (>= 1)

  if (wave >= 4) {
    // ===================== decode waves =====================
    const int pw = wave - 4;                    // 0..3
    const int64_t P = in_f >> 5;                // atoms per row (a multiple of 8)
    const int a = lane & 7, rq = lane >> 3;     // atom of the group, row within a round
    using RawT = typename std::conditional<GG, RawG, Raw>::type;
    const uint64_t wat = (uint64_t)(out_f - n0) * P;
    __amdgpu_buffer_rsrc_t rs_, rm_, rd_, re_, rb_;
    uint32_t vo_s = 0, vo_m = 0, vo_d = 0, vo_e = 0, vo_b = 0, sh = 0;
    // round 0's atom from the tile's first atom; rows past out_f read zeros
    // (buffer range check), their outputs are not stored
    const uint32_t av = (uint32_t)((32 * pw + rq) * P) + (uint32_t)a;
    const uint32_t rstep = (uint32_t)(8 * P);   // atoms from one round's row to the next
    if constexpr (GG) {
      // P is even, so block av sits at av * 46, which is 2 (a & 1) modulo 4
      rb_ = rsrc(blocks + (uint64_t)n0 * P * 46, (wat * 46 + 3) & ~3ull);
      vo_b = (av * 46) & ~3u;
      sh = 16u * (uint32_t)(a & 1);
    } else {
      rs_ = rsrc(sign + n0 * P, wat * 4);
      rm_ = rsrc(mant + n0 * P * 7, wat * 28);
      rd_ = rsrc(delta + n0 * P * 3, wat * 12);
      re_ = rsrc(emax2 + n0 * P, wat * 2);
      vo_s = av * 4; vo_m = av * 28; vo_d = av * 12; vo_e = (av & ~1u) * 2;
    }
    // the atoms of round i of group gj (clamped to the block's last group)
    auto load_round = [&](int gj, int i, RawT& t) {
      const uint32_t ra = (uint32_t)(g0 + min(gj, ng - 1)) * 8u + (uint32_t)i * rstep;
      if constexpr (GG) {
        t.q0 = __builtin_amdgcn_raw_buffer_load_b128(rb_, (int)vo_b, (int)(ra * 46), 0);
        t.q1 = __builtin_amdgcn_raw_buffer_load_b128(rb_, (int)(vo_b + 16), (int)(ra * 46), 0);
        t.q2 = __builtin_amdgcn_raw_buffer_load_b128(rb_, (int)(vo_b + 32), (int)(ra * 46), 0);
      } else {
        const u32x4 m03 = __builtin_amdgcn_raw_buffer_load_b128(rm_, (int)vo_m, (int)(ra * 28), 0);
        const u32x3 m46 = __builtin_amdgcn_raw_buffer_load_b96(rm_, (int)(vo_m + 16), (int)(ra * 28), 0);
        const u32x3 d02 = __builtin_amdgcn_raw_buffer_load_b96(rd_, (int)vo_d, (int)(ra * 12), 0);
        t.s = __builtin_amdgcn_raw_buffer_load_b32(rs_, (int)vo_s, (int)(ra * 4), 0);
        t.ew = __builtin_amdgcn_raw_buffer_load_b32(re_, (int)vo_e, (int)(ra * 2), 0);
        const uint32_t c0 = m03.x, c1 = m03.y, c2 = m03.z, c3 = m03.w, c4 = m46.x, c5 = m46.y, c6 = m46.z;
        t.m[0] = c0; t.m[1] = c1; t.m[2] = c2; t.m[3] = c3; t.m[4] = c4; t.m[5] = c5; t.m[6] = c6;
        const uint32_t e0 = d02.x, e1 = d02.y, e2 = d02.z;
        t.d[0] = e0; t.d[1] = e1; t.d[2] = e2;
      }
    };
    auto store_round = [&](const RawT& w, int i, int slot) {
      uint32_t p[16];
      if constexpr (GG) {
        decode_pairs<true>(gguf_atom(GgufRaw{w.q0, w.q1, w.q2, sh}), p);
      } else {
        Atom t;
        t.s = w.s;
#pragma unroll
        for (int k = 0; k < 7; ++k) t.m[k] = w.m[k];
#pragma unroll
        for (int k = 0; k < 3; ++k) t.d[k] = w.d[k];
        t.e = (uint16_t)(w.ew >> (16 * (a & 1)));
        decode_pairs(t, p);
      }
      const int r = 32 * pw + 8 * i + rq;
      uint8_t* row = wlds + slot * kWSlot4 + r * kRowB4;
#pragma unroll
      for (int c = 0; c < 4; ++c)
        *(u32x4*)(row + swz4(r, 4 * a + c) * 16) = u32x4{p[4 * c], p[4 * c + 1], p[4 * c + 2], p[4 * c + 3]};
    };

    // EXACT plan: the runs of this wave's 32-row group at the 4 steps of a group
    const int64_t G = (out_f + 31) / 32, G2 = 2 * G;
    const int64_t gr = min(n0 / 32 + pw, G);
    uint32_t kp_total = 0;
    if constexpr (EXACT) kp_total = kp_off[S * G2];
    const __amdgpu_buffer_rsrc_t rent = rsrc(kp_ent, (uint64_t)kp_total * 4);
    const __amdgpu_buffer_rsrc_t roff = rsrc(kp_off, ((uint64_t)S * G2 + 1) * 4);
    const uint32_t ob = (uint32_t)(2 * gr) * 4, oe = (uint32_t)min(2 * gr + 2, G2) * 4;
    struct Off { uint32_t beg[kGroup], end[kGroup]; };
    struct Ent { uint32_t beg[kGroup], end[kGroup], e0[kGroup], e1[kGroup]; };
    auto load_off = [&](int gj, Off& o) {
      const uint32_t s0 = (uint32_t)(g0 + min(gj, ng - 1)) * kGroup;
#pragma unroll
      for (int u = 0; u < kGroup; ++u) {
        o.beg[u] = __builtin_amdgcn_raw_buffer_load_b32(roff, (int)ob, (int)((s0 + u) * G2 * 4), 0);
        o.end[u] = __builtin_amdgcn_raw_buffer_load_b32(roff, (int)oe, (int)((s0 + u) * G2 * 4), 0);
      }
    };
    auto load_ent = [&](const Off& o, Ent& e) {
#pragma unroll
      for (int u = 0; u < kGroup; ++u) {
        e.beg[u] = __builtin_amdgcn_readfirstlane(o.beg[u]);
        e.end[u] = __builtin_amdgcn_readfirstlane(o.end[u]);
        e.e0[u] = __builtin_amdgcn_raw_buffer_load_b32(rent, (int)((e.beg[u] + lane) * 4), 0, 0);
        e.e1[u] = __builtin_amdgcn_raw_buffer_load_b32(rent, (int)((e.beg[u] + lane + 64) * 4), 0, 0);
      }
    };
    // entry -> its bf16 in the group tile (step u of the group); a lane past
    // the run writes its own word of the spare area instead (no exec-mask
    // branch); the empty asm makes the compiler wait for the entry's load
    // there
    auto patch_one = [&](uint32_t e, int slot, int u, bool live) {
      const int rr = (int)(e >> 22) & (kBN - 1), c = (int)(e >> 16) & 63;
      const uint32_t dst =
          (uint32_t)(slot * kWSlot4 + rr * kRowB4 + swz4(rr, 8 * u + chunk_of(c)) * 16 + pos_of(c) * 2);
      __asm__ volatile("" : "+v"(e));
      *(uint16_t*)(wlds + (live ? dst : (uint32_t)(2 * kWSlot4 + lane * 4))) = (uint16_t)(e & 0xFFFFu);
    };
    // the first 64 entries of each step's run; runs longer than 64 (rare)
    // behind one uniform branch
    auto patch = [&](const Ent& e, int slot) {
      uint32_t longest = 0;
#pragma unroll
      for (int u = 0; u < kGroup; ++u) {
        patch_one(e.e0[u], slot, u, e.beg[u] + lane < e.end[u]);
        longest = max(longest, e.end[u] - e.beg[u]);
      }
      if (longest > 64) {
#pragma unroll
        for (int u = 0; u < kGroup; ++u) {
          if (e.beg[u] + lane + 64 < e.end[u]) patch_one(e.e1[u], slot, u, true);
          for (uint32_t k = e.beg[u] + 128 + lane; k < e.end[u]; k += 64)   // dense runs
            patch_one(kp_ent[k], slot, u, true);
        }
      }
    };

    RawT R[4];
    Off O{};
    Ent E{};
    // prologue: group 0's plan offsets and entries and group 1's offsets,
    // group 0's atoms; group 0 decoded round by round, each round's registers
    // refilled with group 1's atoms; then group 1's entries and group 2's
    // offsets.  The loads in flight at the loop entry are then 4 rounds of
    // atoms, entries, offsets, as at the end of every iteration.
    if constexpr (EXACT) load_off(0, O);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (EXACT) { load_ent(O, E); load_off(1, O); }
#pragma unroll
    for (int i = 0; i < 4; ++i) load_round(0, i, R[i]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      store_round(R[i], i, 0);
      __builtin_amdgcn_sched_barrier(0);
      load_round(1, i, R[i]);
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (EXACT) {
      patch(E, 0);
      __builtin_amdgcn_sched_barrier(0);
      load_ent(O, E);
      load_off(2, O);
    }
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();

    // iteration j: group j + 1 decoded into slot (j + 1) & 1, round by round,
    // each round's registers refilled with group j + 2's atoms; its plan
    // entries patched, then group j + 2's entries and group j + 3's offsets
    auto iter = [&](int j, int slot) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        store_round(R[i], i, slot);
        __builtin_amdgcn_sched_barrier(0);
        load_round(j + 2, i, R[i]);
        __builtin_amdgcn_sched_barrier(0);
      }
      if constexpr (EXACT) {
        patch(E, slot);
        __builtin_amdgcn_sched_barrier(0);
        load_ent(O, E);
        load_off(j + 3, O);
      }
      __builtin_amdgcn_sched_barrier(0);
      __syncthreads();
    };
    int j = 0;
    for (; j + 1 < ng; j += 2) {
      iter(j, 1);
      iter(j + 1, 0);
    }
    if (j < ng) iter(j, 1);
    return;
  }

  // ===================== MFMA waves =====================
  const int lr = lane & 31, h = lane >> 5;
  const int n = ng * kGroup;                  // steps of this block
  const int s0 = g0 * kGroup;
  const int64_t S64 = S;
  const __amdgpu_buffer_rsrc_t rx_ = rsrc(x + m0 * in_f, (uint64_t)(((M + 31) / 32) * 32 - m0) * (uint64_t)in_f * 2);
  const uint32_t vx0 = (uint32_t)(2 * wave * S64 * 4096 + lane * 16);
  const uint32_t vx1 = vx0 + (uint32_t)(S64 * 4096);
  auto load_x = [&](int jx, bf16x8_t (&X)[2][4]) {
    const uint32_t ks = (uint32_t)(s0 + min(jx, n - 1)) * 4096;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rx_, (int)((i ? vx1 : vx0) + q * 1024), (int)ks, 0);
        X[i][q] = __builtin_bit_cast(bf16x8_t, v);
      }
  };
  // W operand of row tile jj, k-quarter q at step u of the group in slot
  // `slot`: chunk 8u + 4h + q of row jj*32 + lr.  The chunk's swizzle splits
  // into a per-lane part (wo[q]) and a constant of u, joined with one XOR;
  // the slot is bit 16 of the address and jj an immediate offset.
  uint32_t wo[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) wo[q] = (uint32_t)(lr * kRowB4 + (((4 * h + q) ^ (lr & 15)) * 16));
  auto load_w = [&](int q, int u, int slot, bf16x8_t (&wb)[4]) {
    const uint32_t ku = (uint32_t)(((8 * u) ^ ((u >> 1) << 1)) * 16) | ((uint32_t)slot << 16);
    const uint32_t o = wo[q] ^ ku;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) wb[jj] = *(const bf16x8_t*)(wlds + o + jj * 32 * kRowB4);
  };
  f32x16 acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int jj = 0; jj < 4; ++jj)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][jj][v] = 0.f;
  auto mfma = [&](int t, const bf16x8_t (&X)[2][4], int q, const bf16x8_t (&wb)[4]) {
    const int i = t >> 2, jj = t & 3;
    acc[i][jj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(X[i][q], wb[jj], acc[i][jj], 0, 0, 0);
  };
#define BF16X_SG(mask, cnt) __builtin_amdgcn_sched_group_barrier(mask, cnt, 0)
  bf16x8_t X0[2][4], X1[2][4], W0[4], W1[4];
  // step u of the group in `slot` (block step jx) with x in X; x of step
  // jx + 1 requested into Xn first.  The last quarter's second half reads
  // the next step's quarter-0 W operands: after the group's barrier from the
  // other slot at u == 3, from the same slot otherwise.
  auto step = [&](int jx, int u, int slot, const bf16x8_t (&X)[2][4], bf16x8_t (&Xn)[2][4]) {
    load_x(jx + 1, Xn);
    load_w(1, u, slot, W1);
#pragma unroll
    for (int t = 0; t < 8; ++t) mfma(t, X, 0, W0);
    BF16X_SG(0x020, 8);
    BF16X_SG(0x100, 4);
    BF16X_SG(0x008, 8);
    __builtin_amdgcn_sched_barrier(0);
    load_w(2, u, slot, W0);
#pragma unroll
    for (int t = 0; t < 8; ++t) mfma(t, X, 1, W1);
    BF16X_SG(0x100, 4);
    BF16X_SG(0x008, 8);
    __builtin_amdgcn_sched_barrier(0);
    load_w(3, u, slot, W1);
#pragma unroll
    for (int t = 0; t < 8; ++t) mfma(t, X, 2, W0);
    BF16X_SG(0x100, 4);
    BF16X_SG(0x008, 8);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < 4; ++t) mfma(t, X, 3, W1);
    __builtin_amdgcn_sched_barrier(0);
    if (u == kGroup - 1) {
      __syncthreads();
      load_w(0, 0, slot ^ 1, W0);
    } else {
      load_w(0, u + 1, slot, W0);
    }
#pragma unroll
    for (int t = 4; t < 8; ++t) mfma(t, X, 3, W1);
    BF16X_SG(0x100, 4);
    BF16X_SG(0x008, 4);
    __builtin_amdgcn_sched_barrier(0);
  };
#undef BF16X_SG
  auto group = [&](int jg, int slot) {
    step(4 * jg + 0, 0, slot, X0, X1);
    step(4 * jg + 1, 1, slot, X1, X0);
    step(4 * jg + 2, 2, slot, X0, X1);
    step(4 * jg + 3, 3, slot, X1, X0);
  };
  load_x(0, X0);
  __syncthreads();
  load_w(0, 0, 0, W0);
  int jg = 0;
  for (; jg + 1 < ng; jg += 2) {
    group(jg, 0);
    group(jg + 1, 1);
  }
  if (jg < ng) group(jg, 0);
  ws_store<YF32>(acc, wk, wave, lane, M, out_f, grid.ltiles, y, part);
}

// x [M, K] -> operand order: 32-row tile T, step s (64 columns), k-quarter q
// is 1 KB at ((T * S + s) * 4 + q) * 1024, lane l = lr + 32 h holding row
// 32 T + lr, columns 64 s + 32 h + {4q, 16+4q, 4q+1, 17+4q, .., 4q+3, 19+4q}
// (the MFMA A operand of the fused kernels, in the K order of the W tile).
// Rows past M (up to the 32-row boundary) are zeros.  One thread per
// (T, s, l): it reads the 64 contiguous bytes of its row's 32 columns (lanes
// l and l + 32 take the two halves of a 128-byte row segment) and writes its
// 16 bytes of each of the 4 k-quarters (each a contiguous 1 KB per wave).
__global__ __launch_bounds__(256) void x_op_kernel(const uint16_t* __restrict__ x, int64_t M, int64_t in_f,
                                                   int64_t units, u32x4* __restrict__ xo) {
  const int64_t S = in_f / 64;
  for (int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x; u < units; u += (int64_t)gridDim.x * 256) {
    const int l = (int)(u & 63);
    const int64_t ts = u >> 6, T = ts / S, s = ts - T * S;
    const int64_t row = T * 32 + (l & 31);
    uint32_t w[16] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
    if (row < M) {
      const u32x4a* src = (const u32x4a*)(x + row * in_f + s * 64 + (l >> 5) * 32);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const u32x4a v = src[c];
        const uint32_t v0 = v.x, v1 = v.y, v2 = v.z, v3 = v.w;
        w[4 * c] = v0; w[4 * c + 1] = v1; w[4 * c + 2] = v2; w[4 * c + 3] = v3;
      }
    }
    // quarter q: columns 4q .. 4q+3 (words 2q, 2q+1) and 16+4q .. 19+4q (words 8+2q, 9+2q)
#pragma unroll
    for (int q = 0; q < 4; ++q)
      xo[(ts * 4 + q) * 64 + l] = u32x4{perm(w[8 + 2 * q], w[2 * q], 0x05040100u),
                                        perm(w[8 + 2 * q], w[2 * q], 0x07060302u),
                                        perm(w[9 + 2 * q], w[2 * q + 1], 0x05040100u),
                                        perm(w[9 + 2 * q], w[2 * q + 1], 0x07060302u)};
  }
}

// y over the split tiles: the sum of each element's fp32 partials in K-range
// order (partial tile layout as ws_store writes it).  One thread per element
// of the split tiles' 256 x 128 partials, in order.
template <bool YF32>
__global__ __launch_bounds__(256) void ws_tile_reduce_kernel(const float* __restrict__ part, WsGrid g, int nsplit,
                                                             int64_t M, int64_t out_f, void* __restrict__ y,
                                                             bool yal) {
  // four consecutive columns of one tile row per thread (kBN % 4 == 0): 16-byte
  // partial loads, an 8-byte (bf16) or 16-byte (fp32) store when the row's
  // four outputs are in range and aligned (yal: y is 16-byte aligned)
  const int64_t tsz = (int64_t)g.bm * kBN;
  const int64_t count = (int64_t)g.ltiles * tsz;
  typedef float f32x4v __attribute__((ext_vector_type(4)));
  for (int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4; i < count; i += (int64_t)gridDim.x * 256 * 4) {
    const int lt = (int)(i / tsz), e = (int)(i % tsz);
    const int tile = g.full + lt;
    const int64_t row = (int64_t)(tile % g.mtiles) * g.bm + e / kBN;
    const int64_t col = (int64_t)(tile / g.mtiles) * kBN + e % kBN;
    if (row >= M || col >= out_f) continue;
    f32x4v s = *(const f32x4v*)(part + i);
    for (int k = 1; k < nsplit; ++k) s += *(const f32x4v*)(part + (int64_t)k * count + i);
    const float v[4] = {s.x, s.y, s.z, s.w};
    const int64_t o = row * out_f + col;
    if (yal && col + 3 < out_f && (o & 3) == 0) {
      if constexpr (YF32) {
        *(f32x4v*)((float*)y + o) = s;
      } else {
        const uint32_t lo = f32_to_bf16_rne(v[0]) | (f32_to_bf16_rne(v[1]) << 16);
        const uint32_t hi = f32_to_bf16_rne(v[2]) | (f32_to_bf16_rne(v[3]) << 16);
        *(u32x2a*)((uint16_t*)y + o) = u32x2a{lo, hi};
      }
    } else {
      for (int c = 0; c < 4 && col + c < out_f; ++c) {
        if constexpr (YF32) ((float*)y)[o + c] = v[c];
        else ((uint16_t*)y)[o + c] = (uint16_t)f32_to_bf16_rne(v[c]);
      }
    }
  }
}

struct WsShape {
  WsGrid g;
  int nsplit;       // K ranges of a split tile (1: no split tiles)
  int64_t grid;     // blocks
  bool grouped;     // four-step-group kernel (units are groups, else steps)
};

// Four-step groups when K allows (the grouped kernel reads W in runs of
// consecutive atoms); BF16X_TUNE_GEMM_WS_GROUPED = 0 keeps the one-step kernel.
bool ws_grouped(int64_t in_f) {
  return (in_f / kStep) % kGroup == 0 && tuning(BF16X_TUNE_GEMM_WS_GROUPED) != 0;
}

// Resident blocks of the wave-specialised kernels: one per CU (128 KB of LDS
// and 8 waves of 256 registers each); 256 CUs when there is no device to ask.
int64_t ws_resident() {
  static int64_t cache[64];
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] > 0) return cache[dev];
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) return 256;
  cache[dev] = cus;
  return cus;
}

// Tiles run whole-K in full rounds of resident blocks; the f tiles of the
// last, partial round (all tiles when there are fewer than one round) are
// split into s = min(resident / f, 16) K ranges of at least one group (four
// steps for the one-step kernel) so that they fill that round:
// T = 896 tiles on 256 CUs run as 3 rounds of whole tiles and one round of
// 128 tiles x 2 half-K blocks (3.5 rounds instead of 4), with fp32 partials
// only for those 128 tiles.  BF16X_TUNE_GEMM_WS_SPLIT > 0 splits every tile
// into that many K ranges instead; BF16X_TUNE_GEMM_WS_RESIDENT > 0 replaces
// the resident block count (tests reach the mixed plan with few tiles).
WsShape ws_shape(int64_t M, int64_t out_f, int64_t in_f) {
  WsShape w;
  w.grouped = ws_grouped(in_f);
  const int64_t bm = kBM;
  const int64_t mt = (M + bm - 1) / bm, nt = (out_f + kBN - 1) / kBN;
  const int64_t S = in_f / kStep, tiles = mt * nt;
  const int64_t units = w.grouped ? S / kGroup : S;
  const int64_t max_split = std::max<int64_t>(1, std::min<int64_t>(16, w.grouped ? units : units / 4));
  const int64_t forced_c = tuning(BF16X_TUNE_GEMM_WS_RESIDENT);
  const int64_t C = forced_c > 0 ? forced_c : ws_resident();
  int64_t f = tiles % C, s = f ? std::min<int64_t>(C / f, max_split) : 1;
  const int64_t forced = tuning(BF16X_TUNE_GEMM_WS_SPLIT);
  if (forced > 0) {
    f = tiles;
    s = std::min<int64_t>(forced, w.grouped ? units : S);
  }
  const int64_t lunits = (units + s - 1) / s, ks = (units + lunits - 1) / lunits;
  w.g.mtiles = (int)mt;
  w.g.bm = (int)bm;
  if (ks <= 1) {
    w.g.full = (int)tiles; w.g.ltiles = 0; w.g.lunits = (int)units; w.nsplit = 1;
    w.grid = tiles;
  } else {
    w.g.full = (int)(tiles - f); w.g.ltiles = (int)f; w.g.lunits = (int)lunits; w.nsplit = (int)ks;
    w.grid = (tiles - f) + f * ks;
  }
  return w;
}

}  // namespace
}  // namespace bf16x

using namespace bf16x;

namespace {
// workspace: x in operand order (rows rounded up to 32), then the split partials
int64_t ws_xop_bytes(int64_t M, int64_t in_f) { return ((M + 31) / 32) * 32 * in_f * 2; }
}  // namespace

int64_t bf16x_gemm_ws_workspace(int64_t M, int64_t out_f, int64_t in_f) {
  const WsShape w = ws_shape(M, out_f, in_f);
  return ws_xop_bytes(M, in_f) + (w.nsplit > 1 ? (int64_t)w.nsplit * w.g.ltiles * ((int64_t)w.g.bm * kBN) * 4 : 0);
}

// Launch of the wave-specialised kernel; arguments checked by the caller
// (bf16x_gemm for the packed dict; bf16x_gguf_gemm for GGUF blocks, given
// as `blocks` with the dict pointers null).
int bf16x_gemm_ws_launch(const uint16_t* x, int64_t M, const uint32_t* s, const uint32_t* m, const uint32_t* d,
                         const uint16_t* e, const uint8_t* blocks, const uint32_t* kp_off, const uint32_t* kp_ent,
                         int64_t out_f, int64_t in_f, bool exact, bool yf32, void* y, void* workspace,
                         int64_t workspace_bytes, hipStream_t st) {
  const WsShape w = ws_shape(M, out_f, in_f);
  const int64_t xop = ws_xop_bytes(M, in_f);
  if (!workspace || !aligned16(workspace) || workspace_bytes < bf16x_gemm_ws_workspace(M, out_f, in_f))
    return BF16X_ECAPACITY;
  if (xop >= (int64_t)0xFFFFFFFF) return BF16X_ESHAPE;
  if (w.grid > INT32_MAX) return BF16X_ESHAPE;
  const int64_t units = xop / 64;   // (32-row tile, step, lane): 4 chunks of 16 bytes each
  hipLaunchKernelGGL(x_op_kernel, dim3((unsigned)std::min<int64_t>((units + 255) / 256, 8192)), dim3(256), 0, st,
                     x, M, in_f, units, (u32x4*)workspace);
  const uint16_t* xo = (const uint16_t*)workspace;
  float* part = (float*)((uint8_t*)workspace + xop);
  const dim3 grid((unsigned)w.grid);
#define BF16X_WS1(GG_, EX_, YF_)                                                                                   \
  do {                                                                                                           \
    if (w.grouped)                                                                                               \
      hipLaunchKernelGGL((gemm_ws4_kernel<GG_, EX_, YF_>), grid, dim3(512), 0, st, xo, M, s, m, d, e, blocks,       \
                         kp_off, kp_ent, out_f, in_f, w.g, y, part);                                              \
    else                                                                                                         \
      hipLaunchKernelGGL((gemm_ws_kernel<GG_, EX_, YF_>), grid, dim3(512), 0, st, xo, M, s, m, d, e, blocks,        \
                         kp_off, kp_ent, out_f, in_f, w.g, y, part);                                              \
  } while (0)
#define BF16X_WS(GG_)                                        \
  do {                                                       \
    if (exact) {                                             \
      if (yf32) BF16X_WS1(GG_, true, true);                  \
      else BF16X_WS1(GG_, true, false);                      \
    } else {                                                 \
      if (yf32) BF16X_WS1(GG_, false, true);                 \
      else BF16X_WS1(GG_, false, false);                     \
    }                                                        \
  } while (0)
  if (blocks) BF16X_WS(true);
  else BF16X_WS(false);
#undef BF16X_WS
#undef BF16X_WS1
  if (w.nsplit > 1) {
    const int64_t count = (int64_t)w.g.ltiles * ((int64_t)w.g.bm * kBN);
    const int64_t blocks_r = std::min<int64_t>((count / 4 + 255) / 256, 4096);
    if (yf32)
      hipLaunchKernelGGL(ws_tile_reduce_kernel<true>, dim3((unsigned)blocks_r), dim3(256), 0, st,
                         (const float*)part, w.g, w.nsplit, M, out_f, y, aligned16(y));
    else
      hipLaunchKernelGGL(ws_tile_reduce_kernel<false>, dim3((unsigned)blocks_r), dim3(256), 0, st,
                         (const float*)part, w.g, w.nsplit, M, out_f, y, aligned16(y));
  }
  return launch_status();
}
