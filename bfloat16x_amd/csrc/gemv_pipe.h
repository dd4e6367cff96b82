// The pipelined decode+GEMV workgroup body and its helpers, shared by the
// GEMV kernels (gemv.hip) and the harness launch that runs a GEMV and the
// decode attention together (llama_kernels.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "../../include/bf16x_hip.h"
#include "bf16x_device.h"

namespace bf16x {

template <int XT>
__device__ __forceinline__ float load_x_elem(const void* __restrict__ x, int64_t k) {
  if constexpr (XT == BF16X_BF16) return __uint_as_float((uint32_t)((const uint16_t*)x)[k] << 16);
  else if constexpr (XT == BF16X_F32) return ((const float*)x)[k];
  else return (float)((const _Float16*)x)[k];
}

// x values of atom a from global memory in pair order: bf16 -> 16 words
// (x[32a+j] | x[32a+16+j] << 16), fp16/fp32 -> 32 fp32 words (pair j at 2j, 2j+1).
template <int XT>
__device__ __forceinline__ void load_x_atom(const void* __restrict__ x, int64_t a, uint32_t* xr) {
  if constexpr (XT == BF16X_BF16) {
    const uint16_t* xb = (const uint16_t*)x + 32 * a;
    const u32x4a v0 = *(const u32x4a*)(xb);
    const u32x4a v1 = *(const u32x4a*)(xb + 8);
    const u32x4a v2 = *(const u32x4a*)(xb + 16);
    const u32x4a v3 = *(const u32x4a*)(xb + 24);
    const uint32_t lo[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    const uint32_t hi[8] = {v2.x, v2.y, v2.z, v2.w, v3.x, v3.y, v3.z, v3.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      xr[2 * i] = perm(hi[i], lo[i], 0x05040100u);
      xr[2 * i + 1] = perm(hi[i], lo[i], 0x07060302u);
    }
  } else {
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      xr[2 * j] = __float_as_uint(load_x_elem<XT>(x, 32 * a + j));
      xr[2 * j + 1] = __float_as_uint(load_x_elem<XT>(x, 32 * a + 16 + j));
    }
  }
}

// bf16 x values of atom a as loaded (natural order: word k = elements 2k,
// 2k + 1), for a caller that puts them in pair order later (to_pair_order):
// the loads can then be issued ahead of others without waiting for them.
__device__ __forceinline__ void load_x_raw(const void* __restrict__ x, int64_t a, uint32_t* xr) {
  const u32x4a* xb = (const u32x4a*)((const uint16_t*)x + 32 * a);
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const u32x4a v = xb[c];
    xr[4 * c] = v.x; xr[4 * c + 1] = v.y; xr[4 * c + 2] = v.z; xr[4 * c + 3] = v.w;
  }
}

// Natural -> pair order in place (word j = element j | element j + 16 << 16).
__device__ __forceinline__ void to_pair_order(uint32_t* xr) {
  uint32_t t[16];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    t[2 * k] = perm(xr[8 + k], xr[k], 0x05040100u);
    t[2 * k + 1] = perm(xr[8 + k], xr[k], 0x07060302u);
  }
#pragma unroll
  for (int k = 0; k < 16; ++k) xr[k] = t[k];
}

// Dot of an atom's 16 decoded pair words with bf16 x in pair order.
__device__ __forceinline__ void dot_pairs_bf16(const uint32_t* w, const uint32_t* xr, float& acc0, float& acc1) {
#pragma unroll
  for (int j = 0; j < 16; j += 2) {
    acc0 = dot2_bf16(w[j], xr[j], acc0);
    acc1 = dot2_bf16(w[j + 1], xr[j + 1], acc1);
  }
}

template <int XT>
__device__ __forceinline__ void dot_atom(const Atom& t, const uint32_t* xr, float& acc0, float& acc1) {
  uint32_t w[16];
  decode_pairs(t, w);
  if constexpr (XT == BF16X_BF16) {
    dot_pairs_bf16(w, xr, acc0, acc1);
  } else {
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      acc0 = fmaf(bf16lo_to_f32(w[j]), __uint_as_float(xr[2 * j]), acc0);
      acc1 = fmaf(bf16hi_to_f32(w[j]), __uint_as_float(xr[2 * j + 1]), acc1);
    }
  }
}

// (w_exact - w_sat) for a plan entry's exact bits and the element's emax
__device__ __forceinline__ float entry_delta(uint32_t ent, uint32_t em) {
  const uint32_t ex = ent & 0xFFFFu;
  const uint32_t sat = (ex & 0x807Fu) | ((uint32_t)max((int)em - 7, 0) << 7);
  return bf16lo_to_f32(ex) - bf16lo_to_f32(sat);
}

// Buffer cache policy SC1: a load is coherent at agent scope (it does not
// return a line another XCD's writes have made stale in this XCD's L2), a
// store is written through to the agent's coherence point, as the agent-
// scope atomic loads and stores are.
constexpr int kCoherentLoad = 16;

// Raw buffer descriptor (gfx9 word 3) over `bytes` bytes at p.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* p, uint64_t bytes) {
  const uint32_t n = bytes > 0xFFFFFFFFull ? 0xFFFFFFFFu : (uint32_t)bytes;
  return __builtin_amdgcn_make_buffer_rsrc((void*)p, (short)0, (int)n, 0x00020000);
}

// Atom at byte offsets (vo: this lane's atom within the row, so: the row base;
// both in atoms) of the four streams, through raw buffer loads.
__device__ __forceinline__ Atom load_atom_buf(__amdgpu_buffer_rsrc_t rs, __amdgpu_buffer_rsrc_t rm,
                                              __amdgpu_buffer_rsrc_t rd, __amdgpu_buffer_rsrc_t re,
                                              uint32_t va, uint32_t sa) {
  Atom t;
  const u32x4 m03 = __builtin_amdgcn_raw_buffer_load_b128(rm, (int)(va * 28), (int)(sa * 28), 0);
  const u32x3 m46 = __builtin_amdgcn_raw_buffer_load_b96(rm, (int)(va * 28 + 16), (int)(sa * 28), 0);
  const u32x3 d02 = __builtin_amdgcn_raw_buffer_load_b96(rd, (int)(va * 12), (int)(sa * 12), 0);
  t.s = __builtin_amdgcn_raw_buffer_load_b32(rs, (int)(va * 4), (int)(sa * 4), 0);
  t.e = __builtin_amdgcn_raw_buffer_load_b16(re, (int)(va * 2), (int)(sa * 2), 0);
  const uint32_t a0 = m03.x, a1 = m03.y, a2 = m03.z, a3 = m03.w;
  const uint32_t a4 = m46.x, a5 = m46.y, a6 = m46.z;
  t.m[0] = a0; t.m[1] = a1; t.m[2] = a2; t.m[3] = a3;
  t.m[4] = a4; t.m[5] = a5; t.m[6] = a6;
  const uint32_t b0 = d02.x, b1 = d02.y, b2 = d02.z;
  t.d[0] = b0; t.d[1] = b1; t.d[2] = b2;
  return t;
}

// XCD-aware order: workgroups are dispatched round-robin over the 8 XCDs
// (block b runs on XCD b % 8); give each XCD a contiguous range of row blocks
// so the small per-row plan chunks of neighbouring rows share its L2.
__device__ __forceinline__ int xcd_row_block(int b, int nb) {
  const int per = nb / 8, extra = nb - per * 8;  // XCD x gets per (+1 if x < extra) blocks
  const int xcd = b & 7, slot_in_xcd = b >> 3;
  return (nb >= 8) ? (xcd * per + min(xcd, extra) + slot_in_xcd) : b;
}

// bf16 x values of atom a in pair order (as load_x_atom) through agent-
// coherent buffer loads: x written by other workgroups of the same launch.
__device__ __forceinline__ void load_x_atom_coherent(__amdgpu_buffer_rsrc_t rx, int64_t a, uint32_t* xr) {
  const u32x4 v0 = __builtin_amdgcn_raw_buffer_load_b128(rx, (int)(a * 64), 0, kCoherentLoad);
  const u32x4 v1 = __builtin_amdgcn_raw_buffer_load_b128(rx, (int)(a * 64 + 16), 0, kCoherentLoad);
  const u32x4 v2 = __builtin_amdgcn_raw_buffer_load_b128(rx, (int)(a * 64 + 32), 0, kCoherentLoad);
  const u32x4 v3 = __builtin_amdgcn_raw_buffer_load_b128(rx, (int)(a * 64 + 48), 0, kCoherentLoad);
  const uint32_t lo[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
  const uint32_t hi[8] = {v2.x, v2.y, v2.z, v2.w, v3.x, v3.y, v3.z, v3.w};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    xr[2 * i] = perm(hi[i], lo[i], 0x05040100u);
    xr[2 * i + 1] = perm(hi[i], lo[i], 0x07060302u);
  }
}

// The wait a GEMV workgroup takes before it stages x (none: every standalone
// launch).  An active PRE (iters <= 2) is called by every thread of the
// hardware workgroup after the atoms and plan entries of all the wave's rows
// are requested; x is then read with agent-coherent loads.
struct NoPreWait {
  static constexpr bool active = false;
  __device__ void operator()() const {}
};

// Pipelined decode+GEMV.
//
// Work split: a row's P atoms are cut into parts of 64*NS atoms (the last
// part may be shorter); wave part g of a row owns atoms g*64*NS + 64*s + l
// for lane l, step s < NS.  G = ceil(P / (64*NS)) waves share a row.
//
// LDS holds x once, lane-major: [part][step][chunk][lane] x 16 bytes, so the
// main loop reads its chunk with one ds_read_b128 at lane*16 + an immediate
// (conflict free), and the correction overlay finds x[k] by shifts and masks.
// Plan entries carry a byte of saturated exponent max(emax-7, 0), so the
// overlay needs no emax gather; row offsets are read with vector loads (a
// scalar load would share its wait counter with the LDS reads and stall
// every row on the offsets' latency).  All loads are unconditional (indices
// clamped): loads under divergent branches make the compiler wait for every
// outstanding load, which would serialise the prefetch.
// EPI = 1 (SwiGLU epilogue, G = 1, iters = 2): the weight's rows come in
// groups of 8, [gate_4b .. gate_4b+3, up_4b .. up_4b+3], so a wave computes
// gate_i in its first iteration and up_i in its second and writes
// y[i] = bf16(bf16(silu(bf16(gate_i))) * bf16(up_i)) (out_f / 2 outputs): the
// rounding sequence of an unfused GEMV followed by silu(gate) * up in bf16.
//
// XM = 1 (RMSNorm staging, bf16 x): the x the rows are multiplied with is
// RMSNorm(h) * w with h = bf16(x + res_in) (or x when res_in is null),
// computed by every workgroup from x, res_in and w while it stages x, with
// the roundings of the standalone RMSNorm kernel (bf16(bf16(h * rsqrt(mean
// (h^2) + eps)) * w)); workgroup 0 also stores h to res_out (a buffer no
// workgroup of this launch reads).
// XM = 2 (pre-summed RMSNorm staging): x is h itself and the sum of h^2 comes
// from the slots a RES = 1 launch left (NormArgs::slots / nslots): the
// staging only scales.
struct NormArgs {
  const uint16_t* res_in;
  const uint16_t* w;
  uint16_t* res_out;
  float eps;
  const float* slots;   // XM = 2: partial sums of squares of x, summed in slot order
  int nslots;
};

// RES = 1 (G = 1): the residual epilogue.  Row r's output y_r (stored as
// bf16) is added to the residual stream, h_r = bf16(y_r + res_in[r]) goes to
// res_out[r], and workgroup b stores the sum of h_r^2 over its rows to
// slots[b] (its waves' sums added in wave order): the next projection's
// RMSNorm (XM = 2) then needs no pass of its own over h.
struct ResArgs {
  const uint16_t* res_in;
  uint16_t* res_out;
  float* slots;
};

// Sum of slots[0 .. n), n <= 64 kMaxSlotsPerLane, in a fixed order: lane l
// adds slots l, l + 64, ... (all loaded first, so their latencies overlap),
// then the DPP wave sum; the same in every wave, returned in all lanes.
constexpr int kMaxSlotsPerLane = 16;
struct SlotLoads { float v[kMaxSlotsPerLane]; };
__device__ __forceinline__ void slot_load(const float* __restrict__ slots, int n, int lane, SlotLoads& sl) {
#pragma unroll
  for (int k = 0; k < kMaxSlotsPerLane; ++k) sl.v[k] = slots[min(lane + 64 * k, n - 1)];
}
__device__ __forceinline__ float slot_sum(const SlotLoads& sl, int n, int lane) {
  float v = 0.f;
#pragma unroll
  for (int k = 0; k < kMaxSlotsPerLane; ++k) v += (lane + 64 * k < n) ? sl.v[k] : 0.f;
  v = wave_sum_dpp(v);
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

//
// The body of one 256-thread workgroup: `tid` is the thread within it, `vb`
// its index among the launch's workgroups (the slot a RES = 1 workgroup
// writes, none when negative; XM = 1 workgroup 0 stores h), `lb` the row block it takes (rows
// lb * iters * 4 / G + ...), `lds` its x staging area.  SUBS > 1: SUBS such
// workgroups share one hardware workgroup of 256 SUBS threads (sub = which;
// every barrier is taken by all of them, the same number of times).
template <int NS, int G, int XT, bool EXACT, bool FULL, int EPI = 0, int XM = 0, int RES = 0, int SUBS = 1,
          class PRE = NoPreWait, bool YC = false>
__device__ __forceinline__ void gemv_pipe_body(
    const void* __restrict__ x, const uint32_t* __restrict__ sign, const uint32_t* __restrict__ mant,
    const uint32_t* __restrict__ delta, const uint16_t* __restrict__ emax2,
    const uint32_t* __restrict__ tile_off, const uint32_t* __restrict__ tile_ent,
    const uint8_t* __restrict__ tile_sat, int64_t out_f, int64_t in_f, int iters, uint16_t* __restrict__ y,
    NormArgs na, ResArgs ra, int tid, int sub, int vb, int lb, uint32_t* __restrict__ lds, PRE pre = PRE{}) {
  static_assert(RES == 0 || (G == 1 && EPI == 0), "the residual epilogue is for one wave per row");
  static_assert(!PRE::active || (XM == 0 && XT == BF16X_BF16), "a waiting workgroup stages plain bf16 x");
  static_assert(!YC || (G == 1 && EPI == 0), "coherent stores of y: one wave per row");
  constexpr int RPI = 4 / G;                              // rows per workgroup iteration
  constexpr int XW = (XT == BF16X_BF16) ? 16 : 32;        // x words per atom
  constexpr int NC = XW / 4;                              // 16-byte chunks per atom
  constexpr int NB = NS;                                  // prefetched entry batches per wave
  constexpr int APW = 64 * NS;                            // atoms per wave part
  __shared__ float part_all[SUBS][2][4];
  float (&part)[2][4] = part_all[sub];
  const int wave = tid >> 6, lane = tid & 63;
  const int rs = wave / G, g = wave - (wave / G) * G;
  const int64_t P = in_f >> 5;

  // x[k] (fp32) from the lane-major layout
  auto x_at = [&](uint32_t k) -> float {
    const uint32_t a = k >> 5, j = k & 15, hi = (k >> 4) & 1;
    const uint32_t chunk_row = (a >> 6) * NC;  // (part*NS + step) * NC
    if constexpr (XT == BF16X_BF16) {
      const uint32_t wd = lds[((chunk_row + (j >> 2)) * 64 + (a & 63)) * 4 + (j & 3)];
      return hi ? bf16hi_to_f32(wd) : bf16lo_to_f32(wd);
    } else {
      return __uint_as_float(lds[((chunk_row + (j >> 1)) * 64 + (a & 63)) * 4 + (j & 1) * 2 + hi]);
    }
  };

  const __amdgpu_buffer_rsrc_t rs_ = buf_rsrc(sign, (uint64_t)out_f * P * 4);
  const __amdgpu_buffer_rsrc_t rm_ = buf_rsrc(mant, (uint64_t)out_f * P * 28);
  const __amdgpu_buffer_rsrc_t rd_ = buf_rsrc(delta, (uint64_t)out_f * P * 12);
  const __amdgpu_buffer_rsrc_t re_ = buf_rsrc(emax2, (uint64_t)out_f * P * 2);
  const __amdgpu_buffer_rsrc_t roff = buf_rsrc(tile_off, (uint64_t)(out_f + 1) * 4);
  // entry reads are clamped into [.., row end - 1] (see load_ents), so these
  // descriptors need no length: the plan holds at least one entry word
  const __amdgpu_buffer_rsrc_t rent = buf_rsrc(tile_ent, 0xFFFFFFFFull);
  const __amdgpu_buffer_rsrc_t rsat = buf_rsrc(tile_sat, 0xFFFFFFFFull);

  // this lane's atoms (fixed for every row), clamped into the row
  uint32_t va[NS];
  bool live[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int64_t a = (int64_t)g * APW + 64 * s + lane;
    live[s] = FULL || a < P;
    va[s] = (uint32_t)min(a, P - 1);  // idle lanes re-read the row's last atom
  }
  const uint32_t ebase = (uint32_t)(g * 64 + lane);  // this lane's entry slot within a row

  auto row_clamp = [&](int64_t rr) { return min(rr, out_f - 1); };
  auto load_row = [&](int64_t rr, Atom* dst) {
    const uint32_t sa = (uint32_t)(row_clamp(rr) * P);
#pragma unroll
    for (int s = 0; s < NS; ++s) dst[s] = load_atom_buf(rs_, rm_, rd_, re_, va[s], sa);
  };
  auto load_off = [&](int64_t rr, uint32_t& b0, uint32_t& b1) {  // vector loads, all lanes alike
    const int rc = (int)row_clamp(rr);
    b0 = __builtin_amdgcn_raw_buffer_load_b32(roff, rc * 4, 0, 0);
    b1 = __builtin_amdgcn_raw_buffer_load_b32(roff, rc * 4 + 4, 0, 0);
  };
  auto load_ents = [&](uint32_t b0, uint32_t b1, uint32_t* ent, uint8_t* sat) {
    const uint32_t last = b1 > 0 ? b1 - 1 : 0;  // slots past the row end re-read a valid entry
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const uint32_t e = min(b0 + ebase + (uint32_t)(b * 64 * G), last);
      ent[b] = __builtin_amdgcn_raw_buffer_load_b32(rent, (int)(e * 4), 0, 0);
      sat[b] = __builtin_amdgcn_raw_buffer_load_b8(rsat, (int)e, 0, 0);
    }
  };

  int64_t r = (int64_t)__builtin_amdgcn_readfirstlane((int)((int64_t)lb * iters * RPI + rs));
  int64_t rn = r + RPI;
  uint32_t eb = 0, ee = 0, ebn = 0, een = 0;
  // two named buffers in ping-pong (a rotation would copy registers whose
  // loads are still in flight, forcing a wait for them)
  Atom bufA[NS], bufB[NS];
  uint32_t entA[NB], entB[NB];
  uint8_t satA[NB], satB[NB];  // kept 8-bit (see Atom::e)
  // prologue, in the order the first row needs its data (vector loads
  // complete in issue order, so a wait for a load also waits for every load
  // issued before it): row offsets, this thread's x values, the row's atoms,
  // then the entries (which need the offsets).  bf16 x that this kernel
  // stages from memory is loaded as raw words by the threads that store it
  // and put in pair order at the LDS store, so the store waits for x alone,
  // not for the row's atoms behind it (the permutation next to the loads
  // made the compiler issue them after the atoms, or wait for them before
  // issuing the atoms)
  if constexpr (EXACT) {
    load_off(r, eb, ee);
    load_off(rn, ebn, een);
  }
  [[maybe_unused]] uint32_t rin_pre[2] = {0u, 0u};
  [[maybe_unused]] uint32_t wdec[PRE::active ? 2 : 1][PRE::active ? NS : 1][16];
  if constexpr (PRE::active) {
    // x comes from other workgroups of this launch: the wave's rows (iters
    // <= 2), their entries and residuals are requested and the rows decoded
    // while the workgroup waits for it
    load_row(r, bufA);
    if (iters == 2) load_row(rn, bufB);
    if constexpr (EXACT) {
      load_ents(eb, ee, entA, satA);
      if (iters == 2) load_ents(ebn, een, entB, satB);
    }
    if constexpr (RES == 1) {
      rin_pre[0] = ra.res_in[min(r, out_f - 1)];
      rin_pre[1] = ra.res_in[min(rn, out_f - 1)];
    }
#pragma unroll
    for (int s = 0; s < NS; ++s) decode_pairs(bufA[s], wdec[0][s]);
    if (iters == 2) {
#pragma unroll
      for (int s = 0; s < NS; ++s) decode_pairs(bufB[s], wdec[1][s]);
    }
    pre();
  }
  [[maybe_unused]] const __amdgpu_buffer_rsrc_t rx = buf_rsrc(x, (uint64_t)in_f * 2);
  constexpr int XSLOTS = (G * APW + 255) / 256;  // x atoms staged per thread (<= 2)
  [[maybe_unused]] SlotLoads slot_v;
  if constexpr (XM == 2) slot_load(na.slots, na.nslots, lane, slot_v);   // first: the norm waits for them
  uint32_t xs_reg[XSLOTS][XW];
  [[maybe_unused]] uint32_t wn_reg[XM != 0 ? XSLOTS : 1][XM != 0 ? XW : 1];
  [[maybe_unused]] float ssq = 0.f;
#pragma unroll
  for (int i = 0; i < XSLOTS; ++i) {
    const int slot = tid + 256 * i;
    if constexpr (XM == 2) {
      static_assert(XT == BF16X_BF16, "the RMSNorm staging takes bf16 x");
      const int64_t a = min((int64_t)slot, P - 1);
      if (slot < G * APW) {                                // h and w raw (natural order)
        load_x_raw(x, a, xs_reg[i]);
        load_x_raw(na.w, a, wn_reg[i]);
      } else {
#pragma unroll
        for (int k = 0; k < 16; ++k) xs_reg[i][k] = wn_reg[i][k] = 0u;
      }
    } else if constexpr (XM == 1) {
      static_assert(XT == BF16X_BF16, "the RMSNorm staging takes bf16 x");
      const int64_t a = min((int64_t)slot, P - 1);
      const uint16_t* xa = (const uint16_t*)x + 32 * a;
      uint32_t hw[16];                                     // h, natural order, bf16 pairs
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const u32x4a xv = *(const u32x4a*)(xa + 8 * c);
        u32x4a rv = u32x4a{0u, 0u, 0u, 0u};
        if (na.res_in) rv = *(const u32x4a*)(na.res_in + 32 * a + 8 * c);
        const uint32_t xw4[4] = {xv.x, xv.y, xv.z, xv.w}, rw4[4] = {rv.x, rv.y, rv.z, rv.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          uint32_t lo = xw4[k] & 0xFFFFu, hi = xw4[k] >> 16;
          if (na.res_in) {
            lo = f32_to_bf16_rne(bf16lo_to_f32(xw4[k]) + bf16lo_to_f32(rw4[k]));
            hi = f32_to_bf16_rne(bf16hi_to_f32(xw4[k]) + bf16hi_to_f32(rw4[k]));
          }
          hw[4 * c + k] = lo | (hi << 16);
        }
      }
      load_x_atom<XT>(na.w, a, wn_reg[i]);
      if (slot < P) {
#pragma unroll
        for (int k = 0; k < 16; ++k) {
          const float lo = bf16lo_to_f32(hw[k]), hi = bf16hi_to_f32(hw[k]);
          ssq += lo * lo + hi * hi;
        }
        if (vb == 0 && na.res_out) {
#pragma unroll
          for (int c = 0; c < 4; ++c)
            *(u32x4a*)(na.res_out + 32 * a + 8 * c) = u32x4a{hw[4 * c], hw[4 * c + 1], hw[4 * c + 2], hw[4 * c + 3]};
        }
      }
      // natural -> pair order (element j, j + 16), as load_x_atom
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        xs_reg[i][2 * k] = perm(hw[8 + k], hw[k], 0x05040100u);
        xs_reg[i][2 * k + 1] = perm(hw[8 + k], hw[k], 0x07060302u);
      }
    } else if constexpr (PRE::active) {
      load_x_atom_coherent(rx, min((int64_t)slot, P - 1), xs_reg[i]);
    } else if constexpr (XT == BF16X_BF16) {
      if (slot < G * APW) load_x_raw(x, min((int64_t)slot, P - 1), xs_reg[i]);  // slot index = atom index
    } else {
      load_x_atom<XT>(x, min((int64_t)slot, P - 1), xs_reg[i]);
    }
  }
  if constexpr (!PRE::active) load_row(r, bufA);
  // the entries' addresses wait for the offsets: not before the atom loads
  __builtin_amdgcn_sched_barrier(0);
  // the first row's entries go out before the staging waits (XM = 1 waits for
  // its loads and a barrier before the x stores)
  if constexpr (EXACT && XM != 0) load_ents(eb, ee, entA, satA);
  if constexpr (XM != 0) {
    // sum of squares over the row, then x = bf16(bf16(h * s) * w) in place
    float tot;
    if constexpr (XM == 2) {
      tot = slot_sum(slot_v, na.nslots, lane);
    } else {
      __shared__ float nred_all[SUBS][4];
      float (&nred)[4] = nred_all[sub];
      float v = wave_sum_dpp(ssq);
      if (lane == 63) nred[wave] = v;
      __syncthreads();
      tot = (nred[0] + nred[1]) + (nred[2] + nred[3]);
    }
    const float sc = 1.0f / sqrtf(tot / (float)in_f + na.eps);
    // bf16(bf16(h * s) * w) per pair, each rounding one v_cvt_pk_bf16_f32
    // (round to nearest even, as f32_to_bf16_rne for finite values)
#pragma unroll
    for (int i = 0; i < XSLOTS; ++i)
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        const uint32_t h = xs_reg[i][k], w = wn_reg[i][k];
        const uint32_t hs = pk_bf16(bf16lo_to_f32(h) * sc, bf16hi_to_f32(h) * sc);
        xs_reg[i][k] = pk_bf16(bf16lo_to_f32(hs) * bf16lo_to_f32(w), bf16hi_to_f32(hs) * bf16hi_to_f32(w));
      }
  }
#pragma unroll
  for (int i = 0; i < XSLOTS; ++i) {
    const int slot = tid + 256 * i;
    if (slot < G * APW) {
      if constexpr (XM == 2 || (XM == 0 && !PRE::active && XT == BF16X_BF16)) to_pair_order(xs_reg[i]);
      u32x4* dst = (u32x4*)lds + (int64_t)((slot >> 6) * NC) * 64 + (slot & 63);
#pragma unroll
      for (int c = 0; c < NC; ++c)
        dst[c * 64] = u32x4{xs_reg[i][4 * c], xs_reg[i][4 * c + 1], xs_reg[i][4 * c + 2], xs_reg[i][4 * c + 3]};
    }
  }
  if constexpr (EXACT && XM == 0 && !PRE::active) load_ents(eb, ee, entA, satA);
  __syncthreads();

  const u32x4* xl = (const u32x4*)lds + (int64_t)(g * NS) * NC * 64 + lane;
  float gate_keep = 0.f;                                  // EPI = 1: this wave's gate output
  [[maybe_unused]] float res_ss = 0.f;                    // RES = 1: sum of h^2 of this wave's rows (lane 63)
  auto body = [&](auto prefetch, int it, Atom* cur, uint32_t* ent, uint8_t* sat, Atom* nxt, uint32_t* entn,
                  uint8_t* satn) {
    constexpr bool PF = decltype(prefetch)::value;
    // RES: this row's residual, requested before the prefetch so that waiting
    // for it at the store does not wait for the next row's loads
    [[maybe_unused]] uint32_t rin = 0;
    if constexpr (RES == 1) rin = PRE::active ? rin_pre[it & 1] : ra.res_in[min(r, out_f - 1)];
    // prefetch: offsets two rows ahead, then the next row's entries and atoms
    const int64_t rnn = rn + RPI;
    uint32_t ebnn = 0, eenn = 0;
    if constexpr (PF) {
      if constexpr (EXACT) {
        load_off(rnn, ebnn, eenn);
        load_ents(ebn, een, entn, satn);
      }
      load_row(rn, nxt);
    }
    // keep the prefetch ahead of the decode: without this the scheduler sinks
    // the loads below the waits for this row's data and the pipeline drains
    __builtin_amdgcn_sched_barrier(0);
    // decode + dot of this row
    float acc0 = 0.f, acc1 = 0.f;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      uint32_t xr[XW];
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const u32x4 v = xl[(s * NC + c) * 64];
        xr[4 * c] = v.x; xr[4 * c + 1] = v.y; xr[4 * c + 2] = v.z; xr[4 * c + 3] = v.w;
      }
      if constexpr (PRE::active) {      // rows decoded before the wait
        if constexpr (FULL) {
          dot_pairs_bf16(wdec[it & 1][s], xr, acc0, acc1);
        } else {
          float t0 = 0.f, t1 = 0.f;
          dot_pairs_bf16(wdec[it & 1][s], xr, t0, t1);
          acc0 += live[s] ? t0 : 0.f;
          acc1 += live[s] ? t1 : 0.f;
        }
      } else if constexpr (FULL) {
        dot_atom<XT>(cur[s], xr, acc0, acc1);
      } else {
        float t0 = 0.f, t1 = 0.f;
        dot_atom<XT>(cur[s], xr, t0, t1);
        acc0 += live[s] ? t0 : 0.f;
        acc1 += live[s] ? t1 : 0.f;
      }
    }
    // correction overlay: (w_exact - w_sat) * x[k]
    if constexpr (EXACT) {
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const uint32_t e = eb + ebase + (uint32_t)(b * 64 * G);
        const uint32_t k = min(ent[b] >> 16, (uint32_t)in_f - 1);
        const uint32_t sbits = (ent[b] & 0x807Fu) | ((uint32_t)sat[b] << 7);
        const float c = (bf16lo_to_f32(ent[b]) - bf16lo_to_f32(sbits)) * x_at(k);
        acc0 += (e < ee) ? c : 0.f;
      }
      // rows with more entries than the prefetched batches (rare)
      for (uint32_t e = eb + ebase + (uint32_t)(NB * 64 * G); e < ee; e += 64 * G) {
        const uint32_t en = tile_ent[e];
        const uint32_t k = min(en >> 16, (uint32_t)in_f - 1);
        const uint32_t sbits = (en & 0x807Fu) | ((uint32_t)tile_sat[e] << 7);
        acc0 = fmaf(bf16lo_to_f32(en) - bf16lo_to_f32(sbits), x_at(k), acc0);
      }
    }
    // reduce and store
    const float tot = wave_sum_dpp(acc0 + acc1);
    if constexpr (G == 1 && EPI == 1) {
      const float yb = bf16lo_to_f32(f32_to_bf16_rne(tot));
      if ((it & 1) == 0) {
        gate_keep = yb;
      } else if (lane == 63 && r < out_f) {
        const float sg = bf16lo_to_f32(f32_to_bf16_rne(gate_keep / (1.0f + __expf(-gate_keep))));
        y[(r >> 3) * 4 + (r & 3)] = (uint16_t)f32_to_bf16_rne(sg * yb);
      }
    } else if constexpr (G == 1) {
      if (lane == 63 && r < out_f) {
        const uint32_t yb = f32_to_bf16_rne(tot);
        if constexpr (YC)   // read by other workgroups of this launch: written through to the coherence point
          __builtin_amdgcn_raw_buffer_store_b16((uint16_t)yb, buf_rsrc(y, (uint64_t)out_f * 2), (int)(r * 2), 0,
                                                kCoherentLoad);
        else
          y[r] = (uint16_t)yb;
        if constexpr (RES == 1) {
          const float h = bf16lo_to_f32(f32_to_bf16_rne(bf16lo_to_f32(yb) + bf16lo_to_f32(rin)));
          ra.res_out[r] = (uint16_t)(__float_as_uint(h) >> 16);
          res_ss += h * h;
        }
      }
    } else {
      if (lane == 63) part[it & 1][wave] = tot;
      __syncthreads();
      if (g == 0 && lane == 0 && r < out_f) {
        float sum = 0.f;
#pragma unroll
        for (int i = 0; i < G; ++i) sum += part[it & 1][rs * G + i];
        y[r] = (uint16_t)f32_to_bf16_rne(sum);
      }
    }
    eb = ebn; ee = een; ebn = ebnn; een = eenn;
    r = rn; rn = rnn;
  };
  int it = 0;
  if constexpr (PRE::active) {
    // iters <= 2: every row of the wave was requested before the wait
    body(std::false_type{}, 0, bufA, entA, satA, bufB, entB, satB);
    if (iters == 2) body(std::false_type{}, 1, bufB, entB, satB, bufA, entA, satA);
  } else {
    for (; it + 2 < iters; it += 2) {
      body(std::true_type{}, it, bufA, entA, satA, bufB, entB, satB);
      body(std::true_type{}, it + 1, bufB, entB, satB, bufA, entA, satA);
    }
    if (iters - it == 2) {
      body(std::true_type{}, it, bufA, entA, satA, bufB, entB, satB);
      body(std::false_type{}, it + 1, bufB, entB, satB, bufA, entA, satA);
    } else {
      body(std::false_type{}, it, bufA, entA, satA, bufB, entB, satB);
    }
  }
  if constexpr (RES == 1) {
    __shared__ float rpart_all[SUBS][4];
    float (&rpart)[4] = rpart_all[sub];
    if (lane == 63) rpart[wave] = res_ss;
    __syncthreads();
    if (tid == 0 && vb >= 0) ra.slots[vb] = (rpart[0] + rpart[1]) + (rpart[2] + rpart[3]);
  }
}

}  // namespace bf16x
