// Host-side C++ of the BF16X engine: the packed-dict encoder and the
// overflow-plan builder.  No GPU work happens here.
//
// bf16x_encode_host   -> bf16x_quantize (opqk_linear.py:291-324), byte-identical
//                        output including the element padding of
//                        pack_bits_stream (opqk_linear.py:53-64).
// bf16x_plan_host     -> the overflow preparation of Bf16xFused.__init__
//                        (bf16x_fused.py:165-182), re-encoded as per-tile
//                        CSR offsets + 4-byte entries (column, exact bits).
#include <stdint.h>
#include <string.h>

#include <sched.h>

#include <algorithm>
#include <cstdlib>
#include <thread>
#include <vector>

#include "../../include/bf16x_hip.h"

namespace {

constexpr int64_t kTileCols = 65536;

int64_t words_of(int64_t n, int32_t b) {
  const int64_t pad = ((-n * b) % 32 + 32) % 32;  // elements appended by the packer
  const int64_t nbits = (n + pad) * b;
  return (nbits + 31) / 32;
}

// Default thread count: the CPUs this process may run on (affinity mask),
// capped by OMP_NUM_THREADS when set (the share a job scheduler grants) and 64.
int host_threads(int32_t req) {
  if (req > 0) return req;
  int n = (int)std::thread::hardware_concurrency();
  cpu_set_t set;
  if (sched_getaffinity(0, sizeof(set), &set) == 0 && CPU_COUNT(&set) > 0) n = CPU_COUNT(&set);
  if (const char* e = std::getenv("OMP_NUM_THREADS")) {
    const int v = std::atoi(e);
    if (v > 0) n = std::min(n, v);
  }
  return n > 0 ? std::min(n, 64) : 4;
}

template <class F>
void parallel_for(int64_t n_items, int nthreads, F&& f) {
  if (n_items <= 0) return;
  nthreads = (int)std::min<int64_t>(nthreads, n_items);
  if (nthreads <= 1) {
    f(0, n_items);
    return;
  }
  std::vector<std::thread> th;
  th.reserve(nthreads);
  const int64_t per = (n_items + nthreads - 1) / nthreads;
  for (int t = 0; t < nthreads; ++t) {
    const int64_t b = t * per, e = std::min(n_items, b + per);
    if (b >= e) break;
    th.emplace_back([&f, b, e] { f(b, e); });
  }
  for (auto& x : th) x.join();
}

// Bit writer into a word array that stops at `limit` words.
struct BitSink {
  uint32_t* w;
  int64_t limit;
  void put(int64_t bitpos, uint32_t v, int nbits) {
    const int64_t wi = bitpos >> 5;
    const int sh = (int)(bitpos & 31);
    const uint64_t x = (uint64_t)v << sh;
    if (wi < limit) w[wi] |= (uint32_t)x;
    if (sh + nbits > 32 && wi + 1 < limit) w[wi + 1] |= (uint32_t)(x >> 32);
  }
};

}  // namespace

extern "C" int64_t bf16x_stream_words(int64_t n, int32_t bits) {
  if (n < 0 || bits <= 0 || bits > 32) return -1;
  return words_of(n, bits);
}

extern "C" int64_t bf16x_plan_tiles(int64_t out_f, int64_t in_f) {
  if (out_f <= 0 || in_f <= 0) return -1;
  return out_f * ((in_f + kTileCols - 1) / kTileCols);
}

extern "C" int bf16x_encode_host(const uint16_t* w_bits, int64_t out_f, int64_t in_f, int32_t sub,
                                 int32_t* sign, int32_t* mant, int32_t* delta, uint8_t* emax,
                                 int32_t* ovf_idx, uint8_t* ovf_val, int64_t ovf_cap, int64_t* n_ovf,
                                 int32_t n_threads) {
  if (!w_bits || !sign || !mant || !delta || !emax || !n_ovf) return BF16X_EARG;
  if (out_f <= 0 || in_f <= 0 || sub <= 0 || sub > 4096) return BF16X_ESHAPE;
  if (ovf_cap < 0 || (ovf_cap > 0 && (!ovf_idx || !ovf_val))) return BF16X_EARG;
  const int64_t N = out_f * in_f;
  if (N > (int64_t)INT32_MAX) return BF16X_ESHAPE;  // the table stores int32 positions
  const int64_t ws = words_of(N, 1), wm = words_of(N, 7), wd = words_of(N, 3);
  memset(sign, 0, ws * 4);
  memset(mant, 0, wm * 4);
  memset(delta, 0, wd * 4);
  const int64_t nsub = (N + sub - 1) / sub;

  // work unit: a run of elements that starts on a 32-element and a sub-run
  // boundary, so streams, emax and table counts split cleanly between threads
  const int64_t unit = 32 * (int64_t)sub;
  const int64_t n_units = (N + unit - 1) / unit;
  const int nth = host_threads(n_threads);
  std::vector<int64_t> cnt(n_units + 1, 0);

  auto expo_at = [&](int64_t i) -> int32_t { return (w_bits[i] >> 7) & 0xFF; };

  parallel_for(n_units, nth, [&](int64_t ub, int64_t ue) {
    BitSink ss{(uint32_t*)sign, ws}, sm{(uint32_t*)mant, wm}, sd{(uint32_t*)delta, wd};
    for (int64_t u = ub; u < ue; ++u) {
      const int64_t e0 = u * unit, e1 = std::min(N, e0 + unit);
      int64_t c = 0;
      for (int64_t s0 = e0; s0 < e1; s0 += sub) {
        const int64_t s1 = std::min(N, s0 + sub);
        int32_t em = 0;  // tail of the last run is padded with e = 0
        for (int64_t i = s0; i < s1; ++i) em = std::max(em, expo_at(i));
        emax[s0 / sub] = (uint8_t)em;
        for (int64_t i = s0; i < s1; ++i) {
          const uint32_t b = w_bits[i];
          const int32_t d = em - (int32_t)((b >> 7) & 0xFF);
          if (d >= 7) ++c;
          ss.put(i, (b >> 15) & 1u, 1);
          sm.put(i * 7, b & 0x7Fu, 7);
          sd.put(i * 3, (uint32_t)std::min(d, 7), 3);
        }
      }
      cnt[u + 1] = c;
    }
  });
  (void)nsub;
  for (int64_t u = 0; u < n_units; ++u) cnt[u + 1] += cnt[u];
  const int64_t total = cnt[n_units];
  *n_ovf = total;
  if (total > ovf_cap) return BF16X_ECAPACITY;
  parallel_for(n_units, nth, [&](int64_t ub, int64_t ue) {
    for (int64_t u = ub; u < ue; ++u) {
      int64_t o = cnt[u];
      const int64_t e0 = u * unit, e1 = std::min(N, e0 + unit);
      for (int64_t i = e0; i < e1; ++i) {
        const int32_t d = (int32_t)emax[i / sub] - expo_at(i);
        if (d >= 7) {
          ovf_idx[o] = (int32_t)i;
          ovf_val[o] = (uint8_t)d;
          ++o;
        }
      }
    }
  });
  return BF16X_OK;
}

namespace {
inline uint32_t get_bits(const int32_t* words, int64_t nwords, int64_t bit, int nb) {
  const int64_t wi = bit >> 5;
  const int sh = (int)(bit & 31);
  uint64_t v = (uint32_t)words[wi];
  if (sh + nb > 32 && wi + 1 < nwords) v |= (uint64_t)(uint32_t)words[wi + 1] << 32;
  return (uint32_t)(v >> sh) & ((1u << nb) - 1u);
}
}  // namespace

extern "C" int bf16x_plan_host(const int32_t* ovf_idx, const uint8_t* ovf_val, int64_t n_ovf,
                               const int32_t* sign, int64_t n_sign, const int32_t* mant, int64_t n_mant,
                               const int32_t* delta, int64_t n_delta, const uint8_t* emax, int64_t n_emax,
                               int64_t out_f, int64_t in_f, int32_t check,
                               uint32_t* tile_off, uint32_t* tile_ent, uint8_t* tile_sat, int64_t ent_cap,
                               int64_t* n_fix) {
  if (!sign || !mant || !emax || !tile_off || !n_fix) return BF16X_EARG;
  if (n_ovf < 0 || (n_ovf > 0 && (!ovf_idx || !ovf_val))) return BF16X_EARG;
  if (check && !delta) return BF16X_EARG;
  if (out_f <= 0 || in_f <= 0) return BF16X_ESHAPE;
  const int64_t N = out_f * in_f;
  if (n_sign < words_of(N, 1) || n_mant < words_of(N, 7) || n_emax < (N + 15) / 16 ||
      (check && n_delta < words_of(N, 3)))
    return BF16X_ESTREAM_LEN;
  const int64_t tpr = (in_f + kTileCols - 1) / kTileCols;
  const int64_t n_tiles = out_f * tpr;
  memset(tile_off, 0, (n_tiles + 1) * sizeof(uint32_t));
  // pass 1: validate and count entries per tile (kept entries: true delta > 7)
  int64_t kept = 0, prev = -1;
  for (int64_t j = 0; j < n_ovf; ++j) {
    const int64_t p = ovf_idx[j];
    const int v = ovf_val[j];
    if (check) {
      if (p <= prev || p < 0 || p >= N || v < 7) return BF16X_ETABLE;
      if (get_bits(delta, n_delta, p * 3, 3) != 7u) return BF16X_ETABLE;
      if (v > emax[p / 16]) return BF16X_ETABLE;
      prev = p;
    } else if (p < 0 || p >= N) {
      return BF16X_ETABLE;  // never index out of range, even unchecked
    }
    if (v > 7) {
      const int64_t row = p / in_f, col = p % in_f;
      tile_off[row * tpr + col / kTileCols + 1] += 1;
      ++kept;
    }
  }
  if (check >= 2) {
    // every code-7 element must be listed (full scan)
    int64_t j = 0;
    for (int64_t i = 0; i < N; ++i) {
      if (get_bits(delta, n_delta, i * 3, 3) == 7u) {
        while (j < n_ovf && ovf_idx[j] < i) ++j;
        if (j >= n_ovf || ovf_idx[j] != i) return BF16X_ETABLE;
      }
    }
  }
  *n_fix = kept;
  if (kept > (int64_t)UINT32_MAX) return BF16X_ESHAPE;
  for (int64_t t = 0; t < n_tiles; ++t) tile_off[t + 1] += tile_off[t];
  if (kept > ent_cap) return BF16X_ECAPACITY;
  if (kept > 0 && (!tile_ent || !tile_sat)) return BF16X_EARG;
  // pass 2: entries in table order (ascending position = tile order, then column)
  int64_t o = 0;
  for (int64_t j = 0; j < n_ovf; ++j) {
    const int v = ovf_val[j];
    if (v <= 7) continue;
    const int64_t p = ovf_idx[j];
    const int64_t col = (p % in_f) % kTileCols;
    const uint32_t s = get_bits(sign, n_sign, p, 1);
    const uint32_t m = get_bits(mant, n_mant, p * 7, 7);
    const int em = emax[p / 16];
    const uint32_t e = (uint32_t)(em - v) & 0xFFu;  // opqk_linear.py:375
    tile_sat[o] = (uint8_t)std::max(em - 7, 0);
    tile_ent[o++] = ((uint32_t)col << 16) | (s << 15) | (e << 7) | m;
  }
  return BF16X_OK;
}

// ---------------------------------------------------------------------------
// GGUF half-block codec (bf16x_gguf_block.py:29-73)
// ---------------------------------------------------------------------------

// fp32 -> bf16 bits as fp32_to_bf16_bits (bf16x_gguf_block.py:44-49): NaNs
// get the quiet bit (bit 22) before the round-to-nearest-even add, whose
// carry may run into the sign for the largest NaN patterns, as there.
extern "C" int bf16x_fp32_to_bf16_host(const float* x, int64_t n, uint16_t* out, int32_t n_threads) {
  if (n < 0 || (n > 0 && (!x || !out))) return BF16X_EARG;
  parallel_for(n, host_threads(n_threads), [&](int64_t b, int64_t e) {
    for (int64_t i = b; i < e; ++i) {
      uint32_t u;
      memcpy(&u, x + i, 4);
      if ((u & 0x7FFFFFFFu) > 0x7F800000u) u = (u & 0xFFFF0000u) | 0x00400000u;
      out[i] = (uint16_t)(((uint64_t)u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
    }
  });
  return BF16X_OK;
}

// bf16 bits (n_blocks * 32, row-major) -> n_blocks 46-byte blocks
// (bf16x_gguf_block.py:57-73): emax per 16-element half floored at 7,
// code = min(emax - e, 7), fields LSB-first.
extern "C" int bf16x_gguf_quantize_host(const uint16_t* bits, int64_t n_blocks, uint8_t* out, int32_t n_threads) {
  if (n_blocks < 0 || (n_blocks > 0 && (!bits || !out))) return BF16X_EARG;
  parallel_for(n_blocks, host_threads(n_threads), [&](int64_t b, int64_t e) {
    for (int64_t k = b; k < e; ++k) {
      const uint16_t* w = bits + 32 * k;
      uint8_t* o = out + 46 * k;
      uint32_t emax[2] = {7u, 7u};
      for (int j = 0; j < 32; ++j) emax[j >> 4] = std::max(emax[j >> 4], (uint32_t)((w[j] >> 7) & 0xFF));
      uint32_t sign = 0, mw[7] = {0, 0, 0, 0, 0, 0, 0}, dw[3] = {0, 0, 0};
      for (int j = 0; j < 32; ++j) {
        const uint32_t ex = (w[j] >> 7) & 0xFF;
        sign |= (uint32_t)(w[j] >> 15) << j;
        const uint64_t mb = 7 * j, db = 3 * j;
        const uint64_t m = (uint64_t)(w[j] & 0x7F) << (mb & 31);
        mw[mb >> 5] |= (uint32_t)m;
        if ((mb & 31) + 7 > 32) mw[(mb >> 5) + 1] |= (uint32_t)(m >> 32);
        const uint64_t d = (uint64_t)std::min<uint32_t>(emax[j >> 4] - ex, 7u) << (db & 31);
        dw[db >> 5] |= (uint32_t)d;
        if ((db & 31) + 3 > 32) dw[(db >> 5) + 1] |= (uint32_t)(d >> 32);
      }
      o[0] = (uint8_t)emax[0];
      o[1] = (uint8_t)emax[1];
      memcpy(o + 2, &sign, 4);
      memcpy(o + 6, mw, 28);
      memcpy(o + 34, dw, 12);
    }
  });
  return BF16X_OK;
}

// ---------------------------------------------------------------------------
// GGUF lossless side table (bf16x_gguf_block.py:96-185): the elements the
// half-block quantizer turns into the zero marker although they are not
// +-0: exponent delta >= 7 below the half-block max floored at 7 (:121-128).
// Entries are (column | bf16 bits << 16), the little-endian reading of the
// reference's {u16 col, u16 bf16_bits} pairs, sorted by row then column.
namespace {
inline bool gguf_ovf_elem(const uint16_t* blk, int j, const uint32_t emax[2]) {
  const uint32_t ex = (blk[j] >> 7) & 0xFF;
  return emax[j >> 4] - ex >= 7 && (blk[j] & 0x7FFF) != 0;
}
inline void gguf_block_emax(const uint16_t* blk, uint32_t emax[2]) {
  emax[0] = emax[1] = 7u;
  for (int j = 0; j < 32; ++j) emax[j >> 4] = std::max(emax[j >> 4], (uint32_t)((blk[j] >> 7) & 0xFF));
}
}  // namespace

extern "C" int bf16x_gguf_ovf_pack_host(const uint16_t* bits, int64_t rows, int64_t cols, uint32_t* row_off,
                                        uint32_t* entries, int64_t cap, int64_t* n_entries, int32_t n_threads) {
  if (rows < 0 || cols <= 0 || cols % 32 != 0 || cols > 65536 || !n_entries) return BF16X_EARG;
  if (rows > 0 && (!bits || !row_off)) return BF16X_EARG;
  if (rows * cols > ((int64_t)1 << 40)) return BF16X_ESHAPE;
  const int nth = host_threads(n_threads);
  std::vector<int64_t> cnt(rows + 1, 0);
  parallel_for(rows, nth, [&](int64_t b, int64_t e) {
    for (int64_t r = b; r < e; ++r) {
      int64_t c = 0;
      for (int64_t k = 0; k < cols; k += 32) {
        const uint16_t* blk = bits + r * cols + k;
        uint32_t emax[2];
        gguf_block_emax(blk, emax);
        for (int j = 0; j < 32; ++j) c += gguf_ovf_elem(blk, j, emax);
      }
      cnt[r + 1] = c;
    }
  });
  for (int64_t r = 0; r < rows; ++r) cnt[r + 1] += cnt[r];
  *n_entries = cnt[rows];
  if (cnt[rows] > 0xFFFFFFFFll) return BF16X_ESHAPE;
  for (int64_t r = 0; r <= rows; ++r) row_off[r] = (uint32_t)cnt[r];
  if (cnt[rows] > cap) return BF16X_ECAPACITY;
  if (cnt[rows] > 0 && !entries) return BF16X_EARG;
  parallel_for(rows, nth, [&](int64_t b, int64_t e) {
    for (int64_t r = b; r < e; ++r) {
      int64_t o = cnt[r];
      for (int64_t k = 0; k < cols; k += 32) {
        const uint16_t* blk = bits + r * cols + k;
        uint32_t emax[2];
        gguf_block_emax(blk, emax);
        for (int j = 0; j < 32; ++j)
          if (gguf_ovf_elem(blk, j, emax)) entries[o++] = (uint32_t)(k + j) | ((uint32_t)blk[j] << 16);
      }
    }
  });
  return BF16X_OK;
}

extern "C" int bf16x_gguf_ovf_check_host(const uint8_t* blocks, int64_t n_bytes, int64_t rows, int64_t cols,
                                         const uint32_t* row_off, const uint32_t* entries, int64_t n_entries) {
  if (rows <= 0 || cols <= 0 || cols % 32 != 0 || cols > 65536 || n_entries < 0) return BF16X_EARG;
  if (!blocks || !row_off || (n_entries > 0 && !entries)) return BF16X_EARG;
  const int64_t per_row = cols / 32 * 46;
  if (n_bytes < rows * per_row) return BF16X_ESTREAM_LEN;
  if (row_off[0] != 0 || (int64_t)row_off[rows] != n_entries) return BF16X_ETABLE;
  for (int64_t r = 0; r < rows; ++r) {
    if (row_off[r + 1] < row_off[r]) return BF16X_ETABLE;
    int64_t prev = -1;
    for (uint32_t e = row_off[r]; e < row_off[r + 1]; ++e) {
      const int64_t col = entries[e] & 0xFFFF;
      const uint32_t b16 = entries[e] >> 16;
      if (col <= prev || col >= cols) return BF16X_ETABLE;   // sorted, unique, in range
      prev = col;
      // the element must decode as the zero marker (code 7) with the entry's
      // sign and mantissa: the consumers correct by (exact - marker value)
      const uint8_t* blk = blocks + r * per_row + (col / 32) * 46;
      const int j = (int)(col % 32);
      uint32_t sign, mw[7], dw[3];
      memcpy(&sign, blk + 2, 4);
      memcpy(mw, blk + 6, 28);
      memcpy(dw, blk + 34, 12);
      const uint64_t db = 3 * (uint64_t)j, mb = 7 * (uint64_t)j;
      const uint64_t dpair = ((uint64_t)dw[std::min<uint64_t>((db >> 5) + 1, 2)] << 32) | dw[db >> 5];
      const uint32_t code = (uint32_t)(dpair >> (db & 31)) & 7u;
      const uint64_t mpair = ((uint64_t)mw[std::min<uint64_t>((mb >> 5) + 1, 6)] << 32) | mw[mb >> 5];
      const uint32_t mant = (uint32_t)(mpair >> (mb & 31)) & 0x7Fu;
      const uint32_t sgn = (sign >> j) & 1u;
      if (code != 7u || mant != (b16 & 0x7Fu) || sgn != (b16 >> 15)) return BF16X_ETABLE;
    }
  }
  return BF16X_OK;
}
