// Decoder-stack kernels of the Llama-style harness (include/bf16x_llama.h):
// everything of one decoder layer except the BF16X linears, as few launches
// as the data dependences allow, so that a decode step is a fixed launch
// sequence a HIP graph captures.  The token position is read from device
// memory (`pos`, `state`), never passed by value, so one captured graph
// serves every step.
//
// All of these are small next to the linears at batch 1 (a few MB per layer
// against ~340 MB of packed weights): they are written for few launches and
// plain coalesced access, not for peak bandwidth.
#include "bf16x_device.h"
#include "gemv_pipe.h"
#include "launch_common.h"
#include "../../include/bf16x_llama.h"

namespace {
using namespace bf16x;

__device__ __forceinline__ float bfv(uint32_t b16) { return __uint_as_float(b16 << 16); }
__device__ __forceinline__ uint16_t to_bf(float f) { return (uint16_t)f32_to_bf16_rne(f); }
__device__ __forceinline__ float round_bf(float f) { return bfv(f32_to_bf16_rne(f)); }

// Sum over a 256-thread block; every thread gets the total.  `red` holds 4
// floats; the trailing barrier lets the caller reuse it.
__device__ __forceinline__ float block_sum256(float v, float* red) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  const float t = (red[0] + red[1]) + (red[2] + red[3]);
  __syncthreads();
  return t;
}

__device__ __forceinline__ float block_max256(float v, float* red) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  const float t = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  return t;
}

// ---------------------------------------------------------------------------
// RMSNorm with the residual stream: one block of 256 threads per row, a
// thread holds up to 4 chunks of 8 elements (n <= 8192) in registers between
// the sum of squares and the scaling.
constexpr int kNormChunks = 4;

__global__ __launch_bounds__(256) void rmsnorm_kernel(const uint16_t* __restrict__ x,
                                                      const int64_t* __restrict__ row_idx, int64_t x_rows,
                                                      uint16_t* __restrict__ res, const uint16_t* __restrict__ w,
                                                      uint16_t* __restrict__ out, int n, float eps, int flags) {
  __shared__ float red[4];
  const int64_t r = blockIdx.x;
  int64_t xr = r;
  if (row_idx) {
    const int64_t t = row_idx[r];
    xr = t < 0 ? 0 : (t >= x_rows ? x_rows - 1 : t);
  }
  const uint16_t* xp = x + xr * n;
  uint16_t* rp = res ? res + r * n : nullptr;
  float h[kNormChunks][8];
  u32x4 wreg[kNormChunks];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < kNormChunks; ++c) {
    const int i = (c * 256 + (int)threadIdx.x) * 8;
    if (i < n) {
      wreg[c] = *(const u32x4*)(w + i);       // issued with x / residual: one memory round trip fewer
      const u32x4 xv = *(const u32x4*)(xp + i);
      u32x4 rv = {0u, 0u, 0u, 0u};
      if (flags & BF16X_NORM_ADD) rv = *(const u32x4*)(rp + i);
      const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
      const uint32_t rw[4] = {rv.x, rv.y, rv.z, rv.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        float a = bf16lo_to_f32(xw[k]), b = bf16hi_to_f32(xw[k]);
        if (flags & BF16X_NORM_ADD) {
          a = round_bf(a + bf16lo_to_f32(rw[k]));
          b = round_bf(b + bf16hi_to_f32(rw[k]));
        }
        h[c][2 * k] = a;
        h[c][2 * k + 1] = b;
        ss += a * a + b * b;
      }
      if (flags & BF16X_NORM_STORE) {
        u32x4 hv;
        hv.x = f32_to_bf16_rne(h[c][0]) | (f32_to_bf16_rne(h[c][1]) << 16);
        hv.y = f32_to_bf16_rne(h[c][2]) | (f32_to_bf16_rne(h[c][3]) << 16);
        hv.z = f32_to_bf16_rne(h[c][4]) | (f32_to_bf16_rne(h[c][5]) << 16);
        hv.w = f32_to_bf16_rne(h[c][6]) | (f32_to_bf16_rne(h[c][7]) << 16);
        *(u32x4*)(rp + i) = hv;
      }
    }
  }
  const float tot = block_sum256(ss, red);
  const float s = 1.0f / sqrtf(tot / (float)n + eps);
  uint16_t* op = out + r * n;
#pragma unroll
  for (int c = 0; c < kNormChunks; ++c) {
    const int i = (c * 256 + (int)threadIdx.x) * 8;
    if (i < n) {
      const u32x4 wv = wreg[c];
      const uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
      uint32_t o[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float a = round_bf(h[c][2 * k] * s) * bf16lo_to_f32(ww[k]);
        const float b = round_bf(h[c][2 * k + 1] * s) * bf16hi_to_f32(ww[k]);
        o[k] = f32_to_bf16_rne(a) | (f32_to_bf16_rne(b) << 16);
      }
      *(u32x4*)(op + i) = u32x4{o[0], o[1], o[2], o[3]};
    }
  }
}

// ---------------------------------------------------------------------------
// Rotary embedding + KV append.  One wave per (token, head) of the fused qkv
// row; lane i owns dims i and i + 64 (the rotate-half pair).  head_dim 128.
__global__ __launch_bounds__(256) void rope_kv_kernel(const uint16_t* __restrict__ qkv, const int32_t* __restrict__ pos,
                                                      const float* __restrict__ cs, int H, int KV, int max_len,
                                                      uint16_t* __restrict__ q_out, uint16_t* __restrict__ kc,
                                                      uint16_t* __restrict__ vc) {
  const int t = blockIdx.x;
  const int hw = blockIdx.y * 4 + (int)(threadIdx.x >> 6);
  const int i = threadIdx.x & 63;
  if (hw >= H + 2 * KV) return;
  const int p = pos[0] + t;
  const uint16_t* src = qkv + ((int64_t)t * (H + 2 * KV) + hw) * 128;
  const uint16_t a16 = src[i], b16 = src[i + 64];
  if (hw >= H + KV) {                       // v head: plain copy into the cache
    if (p >= 0 && p < max_len) {
      uint16_t* dst = vc + ((int64_t)(hw - H - KV) * max_len + p) * 128;
      dst[i] = a16;
      dst[i + 64] = b16;
    }
    return;
  }
  const int pc = p < 0 ? 0 : (p >= max_len ? max_len - 1 : p);
  const float c = cs[((int64_t)pc * 64 + i) * 2], s = cs[((int64_t)pc * 64 + i) * 2 + 1];
  const float a = bfv(a16), b = bfv(b16);
  const uint16_t ra = to_bf(a * c - b * s), rb = to_bf(b * c + a * s);
  if (hw < H) {
    uint16_t* dst = q_out + ((int64_t)t * H + hw) * 128;
    dst[i] = ra;
    dst[i + 64] = rb;
  } else if (p >= 0 && p < max_len) {
    uint16_t* dst = kc + ((int64_t)(hw - H) * max_len + p) * 128;
    dst[i] = ra;
    dst[i + 64] = rb;
  }
}

// ---------------------------------------------------------------------------
// Causal GQA attention, one block per (head, query).  Scores: a thread per
// key (the 256-byte key row read as 16 dwordx4, q broadcast from LDS);
// softmax over the scores kept in LDS; P.V: wave w takes keys j = w mod 4,
// lane l dims 2l, 2l+1 (one coalesced 256-byte row per key), the four
// partial sums reduced through LDS.  head_dim 128.
__global__ __launch_bounds__(256) void attention_kernel(const uint16_t* __restrict__ q,
                                                        const uint16_t* __restrict__ kc,
                                                        const uint16_t* __restrict__ vc,
                                                        const int32_t* __restrict__ pos, int H, int KV, int max_len,
                                                        float scale, uint16_t* __restrict__ out) {
  extern __shared__ float sc[];           // [max_len] scores, then probabilities
  __shared__ float qs[128];
  __shared__ float red[4];
  __shared__ float part[4][128];
  const int h = blockIdx.x, t = blockIdx.y;
  const int kvh = h / (H / KV);
  const int p = pos[0] + t;
  const int n = p + 1 < 0 ? 0 : (p + 1 > max_len ? max_len : p + 1);
  const int tid = threadIdx.x, wv = tid >> 6, lane = tid & 63;
  uint16_t* op = out + ((int64_t)t * H + h) * 128;
  if (tid < 128) qs[tid] = bfv(q[((int64_t)t * H + h) * 128 + tid]) * scale;
  __syncthreads();
  const uint16_t* K = kc + (int64_t)kvh * max_len * 128;
  float mx = -INFINITY;
  for (int j = tid; j < n; j += 256) {
    const u32x4* kr = (const u32x4*)(K + (int64_t)j * 128);
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int c = 0; c < 16; ++c) {
      const u32x4 kv = kr[c];
      const uint32_t kw[4] = {kv.x, kv.y, kv.z, kv.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        s0 = fmaf(qs[8 * c + 2 * e], bf16lo_to_f32(kw[e]), s0);
        s1 = fmaf(qs[8 * c + 2 * e + 1], bf16hi_to_f32(kw[e]), s1);
      }
    }
    const float s = s0 + s1;
    sc[j] = s;
    mx = fmaxf(mx, s);
  }
  const float M = block_max256(mx, red);
  float sum = 0.f;
  for (int j = tid; j < n; j += 256) {
    const float e = __expf(sc[j] - M);
    sc[j] = e;
    sum += e;
  }
  const float L = block_sum256(sum, red);   // its barriers also publish sc[]
  const uint32_t* V = (const uint32_t*)(vc + (int64_t)kvh * max_len * 128);
  float a0 = 0.f, a1 = 0.f, b0 = 0.f, b1 = 0.f;
  int j = wv;
  for (; j + 4 < n; j += 8) {
    const uint32_t v0 = V[(int64_t)j * 64 + lane], v1 = V[(int64_t)(j + 4) * 64 + lane];
    const float p0 = sc[j], p1 = sc[j + 4];
    a0 = fmaf(p0, bf16lo_to_f32(v0), a0);
    a1 = fmaf(p0, bf16hi_to_f32(v0), a1);
    b0 = fmaf(p1, bf16lo_to_f32(v1), b0);
    b1 = fmaf(p1, bf16hi_to_f32(v1), b1);
  }
  if (j < n) {
    const uint32_t v0 = V[(int64_t)j * 64 + lane];
    a0 = fmaf(sc[j], bf16lo_to_f32(v0), a0);
    a1 = fmaf(sc[j], bf16hi_to_f32(v0), a1);
  }
  part[wv][2 * lane] = a0 + b0;
  part[wv][2 * lane + 1] = a1 + b1;
  __syncthreads();
  if (tid < 128) {
    const float o = (part[0][tid] + part[1][tid]) + (part[2][tid] + part[3][tid]);
    op[tid] = n > 0 ? to_bf(o / L) : (uint16_t)0;
  }
}

// ---------------------------------------------------------------------------
// Decode attention (one token) with the rotary embedding and the KV append
// folded in, split over the keys: workgroup (g, s) serves the G query heads
// of KV head g over key range s of S (the n = pos + 1 keys cut into S equal
// ranges), so that the K and V rows of the whole context are read by S x KV
// workgroups at once instead of KV.
//   0. every workgroup rotates the group's q heads (kept in LDS as fp32 of the
//      bf16-rounded value x scale) and the new k, takes the new v; workgroup
//      s = 0 appends the new k / v row to the caches.  The new key (position
//      p, the last of the range) is always used from LDS: a cache row written
//      in this launch is never read back;
//   1. four lanes per key, 32 dims each (4 dwordx4 of the 256-byte row), G
//      partial dot products reduced over the four lanes (the rows of the
//      first 64 keys, K and V, are loaded at entry, before step 0);
//   2. max and exponentials per head over the range;
//   3. P.V: wave w takes keys w, w + 4, ... of the range, lane l dims 2l, 2l+1,
//      16 row loads issued before their FMAs; the 4 wave sums reduced in LDS;
//   4. the range's (max, sum, unnormalised output) go to the workspace; the
//      last workgroup of KV head g to finish (a device-scope counter per KV
//      head, which that workgroup resets to zero) rescales and combines the
//      S ranges and writes the output.
// Same arithmetic as rope_kv_kernel followed by attention_kernel.
constexpr int kDecMaxSplits = 32;

template <int G>
__global__ __launch_bounds__(256) void attn_decode_kernel(const uint16_t* __restrict__ qkv,
                                                          const int32_t* __restrict__ pos,
                                                          const float* __restrict__ cs, int H, int KV, int max_len,
                                                          float scale, uint16_t* __restrict__ kc,
                                                          uint16_t* __restrict__ vc, float* __restrict__ ws,
                                                          uint32_t* __restrict__ cnt, uint16_t* __restrict__ out) {
  extern __shared__ float lds[];          // scores [G][range]; later wave sums [4][G][128]
  __shared__ float qs[G][128];
  __shared__ float kp[128], vp[128];
  __shared__ float red[G][4];
  __shared__ float ml[kDecMaxSplits][G][2];
  __shared__ int last;
  const int g = blockIdx.x, sp = blockIdx.y, S = gridDim.y;
  const int tid = threadIdx.x, wv = tid >> 6, lane = tid & 63;
  // Key ranges are fixed by the cache length, not by the position: range sp
  // is [sp * chunk, (sp + 1) * chunk) cut to the n keys in use, so the K and V
  // rows of its first 64 keys are requested at entry, together with the
  // position, and their latency overlaps the position's and the rotary step.
  const int chunk = (max_len + S - 1) / S;
  const int jf = sp * chunk;
  const int q4 = tid & 3;
  const uint16_t* K = kc + (int64_t)g * max_len * 128;
  const uint32_t* V = (const uint32_t*)(vc + (int64_t)g * max_len * 128);
  u32x4 kraw[4];
  uint32_t vraw[16];
  {
    // rows past the keys in use are read (clamped into the cache) and never used
    const int jk = min(jf + (tid >> 2), max_len - 1);
    const u32x4* kr = (const u32x4*)(K + (int64_t)jk * 128 + 32 * q4);
#pragma unroll
    for (int c = 0; c < 4; ++c) kraw[c] = kr[c];
#pragma unroll
    for (int u = 0; u < 16; ++u) vraw[u] = V[(int64_t)min(jf + wv + 4 * u, max_len - 1) * 64 + lane];
  }
  const int p = pos[0];
  const bool cur = p >= 0 && p < max_len;                        // the new row fits in the cache
  const int n_old = p < 0 ? 0 : (p > max_len ? max_len : p);     // cached keys 0 .. n_old - 1
  const int n = n_old + (cur ? 1 : 0);
  const int j0 = jf < n ? jf : n;
  const int j1 = j0 + chunk < n ? j0 + chunk : n;
  const int jc = j1 < n_old ? j1 : n_old;                        // end of the cached keys of the range
  auto load_k = [&](int base) {
    const int j = base + (tid >> 2);
    const u32x4* kr = (const u32x4*)(K + (int64_t)(j < jc ? j : 0) * 128 + 32 * q4);
#pragma unroll
    for (int c = 0; c < 4; ++c) kraw[c] = j < jc ? kr[c] : u32x4{0u, 0u, 0u, 0u};
  };
  auto load_v = [&](int base) {
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int j = base + 4 * u;
      vraw[u] = j < jc ? V[(int64_t)j * 64 + lane] : 0u;
    }
  };
  // 0. rotary embedding, KV append
  {
    const int pc = p < 0 ? 0 : (p >= max_len ? max_len - 1 : p);
    const float c = cs[((int64_t)pc * 64 + lane) * 2], sn = cs[((int64_t)pc * 64 + lane) * 2 + 1];
    for (int hh = wv; hh < G + 2; hh += 4) {
      const int head = hh < G ? g * G + hh : (hh == G ? H + g : H + KV + g);
      const uint16_t* src = qkv + (int64_t)head * 128;
      const uint16_t a16 = src[lane], b16 = src[lane + 64];
      if (hh <= G) {
        const float a = bfv(a16), b = bfv(b16);
        const uint32_t ra = f32_to_bf16_rne(a * c - b * sn), rb = f32_to_bf16_rne(b * c + a * sn);
        if (hh < G) {
          qs[hh][lane] = bfv(ra) * scale;
          qs[hh][lane + 64] = bfv(rb) * scale;
        } else {
          kp[lane] = bfv(ra);
          kp[lane + 64] = bfv(rb);
          if (cur && sp == 0) {
            uint16_t* dst = kc + ((int64_t)g * max_len + p) * 128;
            dst[lane] = (uint16_t)ra;
            dst[lane + 64] = (uint16_t)rb;
          }
        }
      } else {
        vp[lane] = bfv(a16);
        vp[lane + 64] = bfv(b16);
        if (cur && sp == 0) {
          uint16_t* dst = vc + ((int64_t)g * max_len + p) * 128;
          dst[lane] = a16;
          dst[lane + 64] = b16;
        }
      }
    }
  }
  __syncthreads();
  // 1. scores, four lanes per key
  float mx[G];
#pragma unroll
  for (int h = 0; h < G; ++h) mx[h] = -INFINITY;
  for (int base = j0; base < j1; base += 64) {
    if (base != j0) load_k(base);                                // ranges longer than 64 keys
    const int j = base + (tid >> 2);
    float s[G];
#pragma unroll
    for (int h = 0; h < G; ++h) s[h] = 0.f;
    if (j < j1) {
      float kf[32];
      if (j < n_old) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const u32x4 kv = kraw[c];
          const uint32_t kw[4] = {kv.x, kv.y, kv.z, kv.w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            kf[8 * c + 2 * e] = bf16lo_to_f32(kw[e]);
            kf[8 * c + 2 * e + 1] = bf16hi_to_f32(kw[e]);
          }
        }
      } else {                                                   // the new key (j == p)
#pragma unroll
        for (int e = 0; e < 32; ++e) kf[e] = kp[32 * q4 + e];
      }
#pragma unroll
      for (int e = 0; e < 32; ++e)
#pragma unroll
        for (int h = 0; h < G; ++h) s[h] = fmaf(qs[h][32 * q4 + e], kf[e], s[h]);
    }
#pragma unroll
    for (int h = 0; h < G; ++h) {
      s[h] += __shfl_xor(s[h], 1, 64);
      s[h] += __shfl_xor(s[h], 2, 64);
    }
    if (j < j1 && q4 == 0) {
#pragma unroll
      for (int h = 0; h < G; ++h) {
        lds[h * chunk + (j - j0)] = s[h];
        mx[h] = fmaxf(mx[h], s[h]);
      }
    }
  }
  float M[G], L[G];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    float v = mx[h];
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    if (lane == 0) red[h][wv] = v;
  }
  __syncthreads();
#pragma unroll
  for (int h = 0; h < G; ++h) M[h] = fmaxf(fmaxf(red[h][0], red[h][1]), fmaxf(red[h][2], red[h][3]));
  __syncthreads();
  // 2. exponentials and sums
  float sum[G];
#pragma unroll
  for (int h = 0; h < G; ++h) sum[h] = 0.f;
  for (int j = j0 + tid; j < j1; j += 256) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float e = __expf(lds[h * chunk + (j - j0)] - M[h]);
      lds[h * chunk + (j - j0)] = e;
      sum[h] += e;
    }
  }
#pragma unroll
  for (int h = 0; h < G; ++h) {
    const float v = wave_sum(sum[h]);
    if (lane == 0) red[h][wv] = v;
  }
  __syncthreads();                         // also publishes the exponentials
#pragma unroll
  for (int h = 0; h < G; ++h) L[h] = (red[h][0] + red[h][1]) + (red[h][2] + red[h][3]);
  // 3. P.V
  float acc[G][2];
#pragma unroll
  for (int h = 0; h < G; ++h) acc[h][0] = acc[h][1] = 0.f;
  for (int base = j0 + wv; base < j1; base += 64) {
    if (base != j0 + wv) load_v(base);                           // ranges longer than 64 keys
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int j = base + 4 * u;
      if (j < j1) {
        float v0 = bf16lo_to_f32(vraw[u]), v1 = bf16hi_to_f32(vraw[u]);
        if (j >= n_old) {                                        // the new value row (j == p)
          v0 = vp[2 * lane];
          v1 = vp[2 * lane + 1];
        }
#pragma unroll
        for (int h = 0; h < G; ++h) {
          const float pr = lds[h * chunk + (j - j0)];
          acc[h][0] = fmaf(pr, v0, acc[h][0]);
          acc[h][1] = fmaf(pr, v1, acc[h][1]);
        }
      }
    }
  }
  __syncthreads();                         // every wave is done with the exponentials
#pragma unroll
  for (int h = 0; h < G; ++h) {
    lds[(wv * G + h) * 128 + 2 * lane] = acc[h][0];
    lds[(wv * G + h) * 128 + 2 * lane + 1] = acc[h][1];
  }
  __syncthreads();
  // 4. this range's partial result, then the combine by the last workgroup
  float* wo = ws + ((int64_t)g * S + sp) * G * 130;              // [G][128] outputs, [G][2] (max, sum)
  for (int e = tid; e < G * 128; e += 256) {
    const int h = e >> 7, d = e & 127;
    wo[e] = (lds[(0 * G + h) * 128 + d] + lds[(1 * G + h) * 128 + d]) +
            (lds[(2 * G + h) * 128 + d] + lds[(3 * G + h) * 128 + d]);
  }
  if (tid < G) {
    float Mh = M[0], Lh = L[0];
#pragma unroll
    for (int k = 1; k < G; ++k)
      if (tid == k) {
        Mh = M[k];
        Lh = L[k];
      }
    wo[G * 128 + 2 * tid] = Mh;
    wo[G * 128 + 2 * tid + 1] = Lh;
  }
  // The barrier orders every thread's partial stores before thread 0's
  // device-scope release fence and count; the last workgroup's thread 0
  // fences (acquire) before the barrier that releases its readers.
  __syncthreads();
  if (tid == 0) {
    __threadfence();
    last = atomicAdd(&cnt[g], 1u) == (uint32_t)(S - 1);
    if (last) __threadfence();
  }
  __syncthreads();
  if (!last) return;
  const float* wg = ws + (int64_t)g * S * G * 130;
  for (int e = tid; e < S * G; e += 256) {
    const int k = e / G, h = e - k * G;
    ml[k][h][0] = wg[(int64_t)k * G * 130 + G * 128 + 2 * h];
    ml[k][h][1] = wg[(int64_t)k * G * 130 + G * 128 + 2 * h + 1];
  }
  __syncthreads();
  for (int e = tid; e < G * 128; e += 256) {
    const int h = e >> 7;
    float Mall = -INFINITY;
    for (int k = 0; k < S; ++k) Mall = fmaxf(Mall, ml[k][h][0]);
    float o = 0.f, l = 0.f;
    for (int k = 0; k < S; ++k) {
      const float f = ml[k][h][1] > 0.f ? __expf(ml[k][h][0] - Mall) : 0.f;
      o = fmaf(wg[(int64_t)k * G * 130 + e], f, o);
      l = fmaf(ml[k][h][1], f, l);
    }
    out[(int64_t)g * G * 128 + e] = l > 0.f ? to_bf(o / l) : (uint16_t)0;
  }
  if (tid == 0) atomicExch(&cnt[g], 0u);
}


// ---------------------------------------------------------------------------
// SwiGLU over 8 columns per thread.
// PAIRS8: a 16-byte chunk of 8 gate_up columns holds gate 4b .. 4b+3 and
// up 4b .. 4b+3; two chunks give 8 outputs.
template <bool PAIRS8>
__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* __restrict__ gu, int64_t T, int F,
                                                       uint16_t* __restrict__ out) {
  const int64_t chunks = T * (F / 8);
  for (int64_t id = (int64_t)blockIdx.x * 256 + threadIdx.x; id < chunks; id += (int64_t)gridDim.x * 256) {
    const int64_t t = id / (F / 8);
    const int c = (int)(id - t * (F / 8)) * 8;
    u32x4 gv, uv;
    if constexpr (PAIRS8) {
      const u32x4 a = *(const u32x4*)(gu + t * 2 * F + 2 * c);       // gate c..c+3, up c..c+3
      const u32x4 b = *(const u32x4*)(gu + t * 2 * F + 2 * c + 8);   // gate c+4..c+7, up c+4..c+7
      gv = u32x4{a.x, a.y, b.x, b.y};
      uv = u32x4{a.z, a.w, b.z, b.w};
    } else {
      gv = *(const u32x4*)(gu + t * 2 * F + c);
      uv = *(const u32x4*)(gu + t * 2 * F + F + c);
    }
    const uint32_t g[4] = {gv.x, gv.y, gv.z, gv.w}, u[4] = {uv.x, uv.y, uv.z, uv.w};
    uint32_t o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float g0 = bf16lo_to_f32(g[k]), g1 = bf16hi_to_f32(g[k]);
      const float s0 = round_bf(g0 / (1.0f + __expf(-g0))), s1 = round_bf(g1 / (1.0f + __expf(-g1)));
      o[k] = f32_to_bf16_rne(s0 * bf16lo_to_f32(u[k])) | (f32_to_bf16_rne(s1 * bf16hi_to_f32(u[k])) << 16);
    }
    *(u32x4*)(out + t * F + c) = u32x4{o[0], o[1], o[2], o[3]};
  }
}

// ---------------------------------------------------------------------------
// Greedy step: one block of 1024 threads, (value, index) reduced with the
// first index winning ties, then the token, history and counters written by
// thread 0.
__device__ __forceinline__ void better(float& v, int& i, float v2, int i2) {
  if (v2 > v || (v2 == v && i2 < i)) {
    v = v2;
    i = i2;
  }
}

// Greedy argmax over kGreedyBlocks workgroups: workgroup b scans logits
// [b span, (b + 1) span) (span a multiple of 8), its thread 0 publishes the
// workgroup's best (value, index) and counts itself; the last one to count
// (a device-scope counter it puts back to zero) reduces the partial results
// across its first wave and writes the token, the history entry and the state.
// The (value, then lower index) order makes the result the first maximum
// whatever the order.  The counter and the partial results live in the
// caller's workspace (GreedyWs): launches with different workspaces are
// independent; launches that share one must not overlap.
constexpr int kGreedyBlocks = 32;
struct GreedyWs {
  uint32_t count;                 // zero between launches (the last workgroup puts it back)
  uint32_t pad[63];
  float val[kGreedyBlocks];
  int idx[kGreedyBlocks];
};

__global__ __launch_bounds__(1024) void greedy_kernel(const uint16_t* __restrict__ logits, int V,
                                                      int64_t* __restrict__ token, int32_t* __restrict__ state,
                                                      int32_t* __restrict__ hist, int hist_len,
                                                      GreedyWs* __restrict__ ws) {
  __shared__ float rv[16];
  __shared__ int ri[16];
  __shared__ bool last;
  float bv = -INFINITY;
  int bi = 0x7FFFFFFF;
  const int tid = threadIdx.x, b = (int)blockIdx.x;
  const int span = ((V + 8 * kGreedyBlocks - 1) / (8 * kGreedyBlocks)) * 8;
  const int lo = min(b * span, V), hi = min(lo + span, V);
  const int full = lo + ((hi - lo) & ~7);
  // kBatch 8-logit groups per thread requested before any is compared (a
  // range of up to 16384 logits is one memory round trip), then compared in
  // index order
  constexpr int kBatch = 2;
  for (int base = lo + tid * 8; base < full; base += 1024 * 8 * kBatch) {
    u32x4 v[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int i = base + u * 1024 * 8;
      v[u] = i < full ? *(const u32x4*)(logits + i) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int i = base + u * 1024 * 8;
      if (i < full) {
        const u32x4 vu = v[u];
        const uint32_t w[4] = {vu.x, vu.y, vu.z, vu.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          better(bv, bi, bf16lo_to_f32(w[k]), i + 2 * k);
          better(bv, bi, bf16hi_to_f32(w[k]), i + 2 * k + 1);
        }
      }
    }
  }
  if (tid < hi - full) better(bv, bi, bfv(logits[full + tid]), full + tid);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) better(bv, bi, __shfl_xor(bv, o, 64), __shfl_xor(bi, o, 64));
  if ((tid & 63) == 0) {
    rv[tid >> 6] = bv;
    ri[tid >> 6] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    for (int k = 1; k < 16; ++k) better(bv, bi, rv[k], ri[k]);
    __hip_atomic_store(&ws->val[b], bv, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&ws->idx[b], bi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = __hip_atomic_fetch_add(&ws->count, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) ==
           (uint32_t)(kGreedyBlocks - 1);
  }
  __syncthreads();
  if (!last || tid >= 64) return;
  // the last workgroup's first wave: lane k reads workgroup k's result
  static_assert(kGreedyBlocks <= 64, "one partial result per lane");
  bv = -INFINITY;
  bi = 0x7FFFFFFF;
  if (tid < kGreedyBlocks) {
    bv = __hip_atomic_load(&ws->val[tid], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    bi = __hip_atomic_load(&ws->idx[tid], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) better(bv, bi, __shfl_xor(bv, o, 64), __shfl_xor(bi, o, 64));
  if (tid != 0) return;
  __hip_atomic_store(&ws->count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (bi == 0x7FFFFFFF) bi = 0;          // every logit NaN: token 0
  token[0] = bi;
  const int c = state[1];
  if (c >= 0 && c < hist_len) hist[c] = bi;
  state[1] = c + 1;
  state[0] = state[0] + 1;
}

}  // namespace

extern "C" int bf16x_rmsnorm(const uint16_t* x, const int64_t* row_idx, int64_t x_rows, uint16_t* residual,
                             const uint16_t* weight, uint16_t* out, int64_t rows, int64_t n, float eps, int32_t flags,
                             bf16x_stream_t stream) {
  if (!x || !weight || !out || rows < 0 || (flags & ~(BF16X_NORM_ADD | BF16X_NORM_STORE))) return BF16X_EARG;
  if (n <= 0 || n % 8 != 0 || n > kNormChunks * 256 * 8 || rows > INT32_MAX) return BF16X_ESHAPE;
  if (row_idx && x_rows <= 0) return BF16X_EARG;
  if (flags && !residual) return BF16X_EARG;
  if (!aligned16(x) || !aligned16(weight) || !aligned16(out) || (residual && !aligned16(residual)))
    return BF16X_EARG;
  if (rows == 0) return BF16X_OK;
  hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)rows), dim3(256), 0, (hipStream_t)stream, x, row_idx, x_rows,
                     residual, weight, out, (int)n, eps, (int)flags);
  return launch_status();
}

extern "C" int bf16x_rope_kv(const uint16_t* qkv, int64_t tokens, const int32_t* pos, const float* cos_sin,
                             int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, int64_t max_len, uint16_t* q_out,
                             uint16_t* k_cache, uint16_t* v_cache, bf16x_stream_t stream) {
  if (!qkv || !pos || !cos_sin || !q_out || !k_cache || !v_cache || tokens < 0) return BF16X_EARG;
  if (head_dim != 128 || n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads != 0 || n_heads > 4096 ||
      max_len <= 0 || max_len > INT32_MAX / 2 || tokens > 65535)
    return BF16X_ESHAPE;
  if (!aligned4(cos_sin) || !aligned2(qkv) || !aligned2(q_out) || !aligned2(k_cache) || !aligned2(v_cache))
    return BF16X_EARG;
  if (tokens == 0) return BF16X_OK;
  const int heads = (int)(n_heads + 2 * n_kv_heads);
  hipLaunchKernelGGL(rope_kv_kernel, dim3((unsigned)tokens, (unsigned)((heads + 3) / 4)), dim3(256), 0,
                     (hipStream_t)stream, qkv, pos, cos_sin, (int)n_heads, (int)n_kv_heads, (int)max_len, q_out,
                     k_cache, v_cache);
  return launch_status();
}

// ---------------------------------------------------------------------------
// Causal GQA attention for many query rows (prefill) on bf16 MFMA
// (v_mfma_f32_16x16x32_bf16), flash-attention style: workgroup (query tile
// of 64 rows, head h), 4 waves, wave w owns queries t0 + 16 w .. + 15; K and
// V of the KV head stream through LDS in blocks of 32 keys (double
// buffered, one barrier per block) and every query keeps a running softmax.
// Same results as attention_kernel up to fp32 summation order: scores are
// exact bf16 products summed in fp32 and scaled after the sum, the
// probabilities enter P.V as two bf16 terms (hi + lo, 16 significant bits)
// and the output is divided by the fp32 sum once, at the end.
// Operand layout of the 16x16x32 MFMA (lane l, g = l / 16): A[l % 16][8 g +
// v'], B[8 g + v'][l % 16], D register v = D[4 g + v][l % 16].  Both
// products are computed transposed so that lane l always serves query
// l % 16:
//  * S^T = K Q^T: A = K rows (16 keys x 32 dims) from LDS, B = Q^T from
//    registers (the query row's 8 dims of the chunk); lane l then holds the
//    scores of keys 4 g + v (and 16 + 4 g + v) for its query;
//  * O^T = V^T P^T: B = P^T straight from those registers (k slot 8 g + v'
//    = key 4 g + v' for v' < 4, key 16 + 4 g + v' - 4 otherwise), A = V^T
//    read from a transposed copy of the V block in LDS whose columns are in
//    that slot order; lane l accumulates dims 16 dt + 4 g + v of its query.
// LDS rows are padded (K: 272 bytes, V^T: 80 bytes) so that the 16 lanes of
// an operand read touch 16 different 16-byte bank groups.
namespace {
constexpr int kFaQ = 64;                  // query rows per workgroup
constexpr int kFaMinTokens = 16;          // bf16x_attention takes this kernel from this many rows on
constexpr int kFaK = 32;                  // keys per block
constexpr int kFaKRow = 272;              // bytes per K row in LDS (256 + 16)
constexpr int kFaVRow = 80;               // bytes per V^T row in LDS (64 + 16)
constexpr int kFaD = 4;                   // key blocks in flight in registers

typedef __bf16 fa_bf16x8 __attribute__((ext_vector_type(8)));
typedef float fa_f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int fa_slot(int key) {   // V^T column of key 0..31
  return key < 16 ? 8 * (key >> 2) + (key & 3) : 8 * ((key - 16) >> 2) + 4 + (key & 3);
}

__global__ __launch_bounds__(256) void attention_mfma_kernel(const uint16_t* __restrict__ q,
                                                             const uint16_t* __restrict__ kc,
                                                             const uint16_t* __restrict__ vc,
                                                             const int32_t* __restrict__ pos, int T, int H, int KV,
                                                             int max_len, float scale, uint16_t* __restrict__ out) {
  __shared__ __attribute__((aligned(16))) uint8_t ks[2][kFaK * kFaKRow];
  __shared__ __attribute__((aligned(16))) uint8_t vts[2][128 * kFaVRow];
  const int t0 = (int)blockIdx.x * kFaQ, h = (int)blockIdx.y;
  const int kvh = h / (H / KV);
  const int tid = threadIdx.x, lane = tid & 63, gl = lane >> 4, ql = lane & 15;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int p0 = pos[0];
  const int t = t0 + 16 * w + ql;                              // this lane's query row
  const int pq = p0 + t;                                       // its position: keys 0 .. pq
  const int nq = t < T ? max(0, min(pq + 1, max_len)) : 0;     // keys this query sees
  const int tlast = min(t0 + kFaQ - 1, T - 1);
  const int nmax = max(0, min(p0 + tlast + 1, max_len));       // keys any query of the tile sees
  const int nblk = (nmax + kFaK - 1) / kFaK;

  // Q^T operands: chunk c = dims 32 c + 8 gl .. + 7 of the lane's query
  fa_bf16x8 qb[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    u32x4 v = u32x4{0u, 0u, 0u, 0u};
    if (t < T) v = *(const u32x4*)(q + ((int64_t)t * H + h) * 128 + 32 * c + 8 * gl);
    qb[c] = __builtin_bit_cast(fa_bf16x8, v);
  }

  // staging: thread (key tid / 8, 32-byte part tid % 8) of K, (dims 8 (tid % 16) .. +7, keys 2 (tid / 16), +1) of V
  const uint16_t* K = kc + (int64_t)kvh * max_len * 128;
  const uint16_t* V = vc + (int64_t)kvh * max_len * 128;
  const int kk = tid >> 3, kp = tid & 7, vd = tid & 15, vk = 2 * (tid >> 4);
  // key blocks in flight in registers: block k is loaded into set k % kFaD
  // kFaD iterations before it is staged in LDS (one iteration before its use)
  u32x4 kr[kFaD][2], vr[kFaD][2];
  auto load_block = [&](int b, u32x4 (&k2)[2], u32x4 (&v2)[2]) {
    const int last = nmax - 1;                                 // rows past the context: a valid row (masked)
    const uint16_t* kp_ = K + (int64_t)min(kFaK * b + kk, last) * 128 + 16 * kp;
    k2[0] = *(const u32x4*)kp_;
    k2[1] = *(const u32x4*)(kp_ + 8);
    v2[0] = *(const u32x4*)(V + (int64_t)min(kFaK * b + vk, last) * 128 + 8 * vd);
    v2[1] = *(const u32x4*)(V + (int64_t)min(kFaK * b + vk + 1, last) * 128 + 8 * vd);
  };
  auto store_block = [&](int slot, const u32x4 (&k2)[2], const u32x4 (&v2)[2]) {
    uint8_t* kd = ks[slot] + kk * kFaKRow + 32 * kp;
    *(u32x4*)kd = k2[0];
    *(u32x4*)(kd + 16) = k2[1];
    const uint32_t a[4] = {v2[0].x, v2[0].y, v2[0].z, v2[0].w}, b[4] = {v2[1].x, v2[1].y, v2[1].z, v2[1].w};
    uint8_t* vd_ = vts[slot] + (8 * vd) * kFaVRow + 2 * fa_slot(vk);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      *(uint32_t*)(vd_ + (2 * e) * kFaVRow) = (a[e] & 0xFFFFu) | (b[e] << 16);
      *(uint32_t*)(vd_ + (2 * e + 1) * kFaVRow) = (a[e] >> 16) | (b[e] & 0xFFFF0000u);
    }
  };

  float m = -INFINITY, l = 0.f;
  fa_f32x4 o[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) o[dt] = fa_f32x4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int b, int slot) {
    // S^T = K Q^T for keys 32 b + 16 kt + (0 .. 15)
    fa_f32x4 sacc[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      sacc[kt] = fa_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const fa_bf16x8 a =
            *(const fa_bf16x8*)(ks[slot] + (16 * kt + ql) * kFaKRow + 64 * c + 16 * gl);
        sacc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qb[c], sacc[kt], 0, 0, 0);
      }
    }
    // running softmax of the lane's query over the block (its 8 keys here,
    // the other 24 in lanes ql + 16, + 32, + 48)
    float sv[8];
    float mb = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int j = kFaK * b + 16 * kt + 4 * gl + v;
        const float sc = j < nq ? sacc[kt][v] * scale : -INFINITY;
        sv[4 * kt + v] = sc;
        mb = fmaxf(mb, sc);
      }
    mb = fmaxf(mb, __shfl_xor(mb, 16, 64));
    mb = fmaxf(mb, __shfl_xor(mb, 32, 64));
    const float mn = fmaxf(m, mb);
    const float alpha = mn == -INFINITY ? 1.f : __expf(m - mn);
    float ps = 0.f;
    uint32_t phi[4], plo[4];
#pragma unroll
    for (int k = 0; k < 8; k += 2) {
      const float e0 = sv[k] == -INFINITY ? 0.f : __expf(sv[k] - mn);
      const float e1 = sv[k + 1] == -INFINITY ? 0.f : __expf(sv[k + 1] - mn);
      ps += e0 + e1;
      phi[k >> 1] = pk_bf16(e0, e1);
      plo[k >> 1] = pk_bf16(e0 - bf16lo_to_f32(phi[k >> 1]), e1 - bf16hi_to_f32(phi[k >> 1]));
    }
    ps += __shfl_xor(ps, 16, 64);
    ps += __shfl_xor(ps, 32, 64);
    l = l * alpha + ps;
    m = mn;
    const fa_bf16x8 bhi = __builtin_bit_cast(fa_bf16x8, u32x4{phi[0], phi[1], phi[2], phi[3]});
    const fa_bf16x8 blo = __builtin_bit_cast(fa_bf16x8, u32x4{plo[0], plo[1], plo[2], plo[3]});
    // O^T = alpha O^T + V^T P^T
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      o[dt] *= alpha;
      const fa_bf16x8 a = *(const fa_bf16x8*)(vts[slot] + (16 * dt + ql) * kFaVRow + 16 * gl);
      o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bhi, o[dt], 0, 0, 0);
      o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, blo, o[dt], 0, 0, 0);
    }
  };

  if (nblk > 0) {
#pragma unroll
    for (int d = 0; d < kFaD; ++d)
      if (d < nblk) load_block(d, kr[d], vr[d]);
    store_block(0, kr[0], vr[0]);
    if (kFaD < nblk) load_block(kFaD, kr[0], vr[0]);
  }
  __syncthreads();
  for (int b0 = 0; b0 < nblk; b0 += kFaD) {
#pragma unroll
    for (int u = 0; u < kFaD; ++u) {
      const int b = b0 + u;
      if (b < nblk) {
        if (b + 1 < nblk) {
          // block b + 1 (register set (u + 1) % kFaD) into the other slot: its
          // last readers passed the previous barrier; then block b + 1 + kFaD
          // into the freed registers
          store_block((b + 1) & 1, kr[(u + 1) % kFaD], vr[(u + 1) % kFaD]);
          if (b + 1 + kFaD < nblk) load_block(b + 1 + kFaD, kr[(u + 1) % kFaD], vr[(u + 1) % kFaD]);
        }
        compute(b, b & 1);
        __syncthreads();
      }
    }
  }
  if (t < T) {
    const float inv = l > 0.f ? 1.f / l : 0.f;
    uint16_t* op = out + ((int64_t)t * H + h) * 128 + 4 * gl;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const uint32_t lo = f32_to_bf16_rne(o[dt][0] * inv) | (f32_to_bf16_rne(o[dt][1] * inv) << 16);
      const uint32_t hi = f32_to_bf16_rne(o[dt][2] * inv) | (f32_to_bf16_rne(o[dt][3] * inv) << 16);
      *(uint2*)(op + 16 * dt) = make_uint2(lo, hi);
    }
  }
}
}  // namespace

extern "C" int bf16x_attention(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                               const int32_t* pos, int64_t tokens, int64_t n_heads, int64_t n_kv_heads,
                               int64_t head_dim, int64_t max_len, float scale, uint16_t* out,
                               bf16x_stream_t stream) {
  if (!q || !k_cache || !v_cache || !pos || !out || tokens < 0) return BF16X_EARG;
  if (head_dim != 128 || n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads != 0 || n_heads > 65535 ||
      max_len <= 0 || max_len > 16384 || tokens > 65535)
    return BF16X_ESHAPE;
  if (!aligned16(k_cache) || !aligned4(v_cache) || !aligned2(q) || !aligned2(out)) return BF16X_EARG;
  if (tokens == 0) return BF16X_OK;
  // many query rows: the MFMA kernel (from kFaMinTokens rows, or as the
  // override BF16X_TUNE_ATTN_MFMA says: 0 never, 1 always)
  // (it loads q and V rows 16 bytes at a time and stores 8-byte runs of out)
  const int64_t mf = tuning(BF16X_TUNE_ATTN_MFMA);
  const bool mf_aligned = aligned16(q) && aligned16(v_cache) && aligned8(out);
  if (mf == 1 && !mf_aligned) return BF16X_EARG;
  if (mf == 1 || (mf != 0 && tokens >= kFaMinTokens && mf_aligned)) {
    hipLaunchKernelGGL(attention_mfma_kernel, dim3((unsigned)((tokens + kFaQ - 1) / kFaQ), (unsigned)n_heads),
                       dim3(256), 0, (hipStream_t)stream, q, k_cache, v_cache, pos, (int)tokens, (int)n_heads,
                       (int)n_kv_heads, (int)max_len, scale, out);
    return launch_status();
  }
  hipLaunchKernelGGL(attention_kernel, dim3((unsigned)n_heads, (unsigned)tokens), dim3(256),
                     (size_t)max_len * sizeof(float), (hipStream_t)stream, q, k_cache, v_cache, pos, (int)n_heads,
                     (int)n_kv_heads, (int)max_len, scale, out);
  return launch_status();
}

// Decode attention for short contexts (max_len <= kDec1MaxLen): one
// workgroup of 8 waves per KV head, no second pass and no cross-workgroup
// combine.  The split kernel above spends ~10 us on its fixed chain (ranges
// from the position, partials, device-scope counter, combine); this one
// starts at ~6 us but streams a KV head's keys through one CU at ~2 us per
// block of 128 keys, so it wins up to ~256 keys (measured: 1 key 5.8 vs
// 9.9 us, 300 keys 10.8 vs 12.7, 600 keys 16.6 vs 13.7).
// Keys are taken in blocks of 128, wave w keys 16w .. 16w+15 of a block, four
// lanes per key for the scores (lane q of a key holds 16-byte chunk q of
// each 64-byte quarter of the row, dims 32c + 8q .. 32c + 8q + 7: each K
// load instruction then reads 64 contiguous bytes of each of its 16 keys,
// half the cache-line accesses of a lane-per-quarter layout; measured
// 13.3 -> 11.6 us per launch at 600 keys) and lane l dims 2l, 2l+1 for
// P.V.  Each wave keeps a running softmax (max, sum, unnormalised output per
// head) over its keys; K and V of the next block are in flight while a block
// is processed.  At the end the 8 waves' states are combined in LDS in wave
// order.  The new row (position p) is rotated and appended as in
// rope_kv_kernel and read from LDS.
// Per-head variant (PH, W = 16 waves, NB blocks of 256 keys): one workgroup
// per QUERY head (the group's K and V rows are read by its G workgroups, from
// L2), and the rows of all NB blocks are requested at entry, before the
// position is known (clamped into the cache; a row at or past the position
// is replaced by the new row from LDS, as above), so a context of up to
// 16 W NB keys costs one memory round trip instead of a chain of blocks or
// the split kernel's partials and counter.  The first workgroup of a group
// appends the new row.
constexpr int kDec1MaxLen = 256;
constexpr int kDec1Waves = 8;
constexpr int kDecHWaves = 16;
constexpr int kDecHBlocks = 3;
constexpr int kDecHMaxLen = 16 * kDecHWaves * kDecHBlocks;   // 768

// The layer launch (layer_front_kernel: the qkv GEMV, the decode attention and
// optionally the o projection as one launch) orders its stages with
// counters in device memory instead of launch boundaries.  A stage stores
// what the next one reads with agent-coherent (write-through) stores; its
// workgroups count themselves on counter (s, XCD of the workgroup) once
// every wave's stores are complete (s_waitcnt vmcnt(0), then a barrier and
// thread 0's device-scope atomic).  No release fence: its L2 write-back took
// ~0.3 us per workgroup and they queue per XCD (7 us in the decode step).
// Per-XCD counters because ~200 device-scope atomics on one address
// serialise, ~5 us.  A waiting workgroup's thread 0 polls until the eight
// counters of the stage before add up to its workgroup count; the data is
// then read with agent-coherent loads (an acquire fence would invalidate the
// XCD's L2, ~3 us).  The counters are never reset by
// the launch that uses them: each launch zeroes those of the launch before
// it (`clear`), which stream order has finished.  The waits are bounded:
// past kSyncSpinLimit polls the workgroup sets `err` and goes on.
constexpr int kSyncXcds = 8;
constexpr int kSyncStride = 64;                 // words: one 256-byte line per counter
constexpr int kSyncStages = 2;                  // counted stages: the qkv GEMV, the attention
constexpr int kSyncErrWord = kSyncStages * kSyncXcds * kSyncStride;
constexpr uint32_t kSyncSpinLimit = 1u << 19;   // a few tenths of a second of polls
constexpr int kWaitVmcnt0 = 0x0F70;             // s_waitcnt vmcnt(0) expcnt(7) lgkmcnt(15) (gfx9 encoding)

__device__ __forceinline__ uint32_t* sync_counter(uint32_t* sync, int stage, int xcd) {
  return sync + (stage * kSyncXcds + xcd) * kSyncStride;
}

// Thread 0 waits until the counters of `stage` reach `target`; then the
// barrier releases the workgroup.  Called by every thread.
__device__ __forceinline__ void sync_wait(uint32_t* sync, int stage, uint32_t target) {
  if (threadIdx.x == 0) {
    auto counted = [&]() {
      uint32_t t = 0;
#pragma unroll
      for (int x = 0; x < kSyncXcds; ++x)
        t += __hip_atomic_load(sync_counter(sync, stage, x), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return t;
    };
    uint32_t spins = 0;
    while (counted() < target) {
      __builtin_amdgcn_s_sleep(2);
      if (++spins == kSyncSpinLimit) {
        __hip_atomic_store(sync + kSyncErrWord, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
    }
  }
  __syncthreads();
}

// Every wave's stores are complete, then thread 0 counts the workgroup on
// (stage, xcd).  Called by every thread.
__device__ __forceinline__ void sync_count(uint32_t* sync, int stage, int xcd) {
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  __syncthreads();
  if (threadIdx.x == 0)
    __hip_atomic_fetch_add(sync_counter(sync, stage, xcd), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// WAIT: the attention workgroups of the layer launch wait for the qkv GEMV
// (stage 0, `target` workgroups) before reading qkv, and count themselves on
// stage 1 when their output is stored.
struct AttnSync {
  uint32_t* sync;
  uint32_t target;
};

template <int G, int W, bool PH, int NB, bool WAIT = false>
__device__ __forceinline__ void attn_decode1_body(const uint16_t* __restrict__ qkv, const int32_t* __restrict__ pos,
                                                  const float* __restrict__ cs, int H, int KV, int max_len,
                                                  float scale, uint16_t* __restrict__ kc, uint16_t* __restrict__ vc,
                                                  uint16_t* __restrict__ out, int blk, int tid, AttnSync sync) {
  __shared__ uint32_t qs2[G][64];          // rotated q as bf16 pairs (dims 2i, 2i+1)
  __shared__ uint32_t kp2[64];             // the new key, likewise
  __shared__ float vp[128];
  constexpr int kBlock = 16 * W;           // keys per block
  __shared__ float ps[W][G][16];           // per wave: the scores of its 16 keys of a block
  __shared__ float pw[W][G][16];           // per wave: their probabilities
  __shared__ float wm[W][G], wl[W][G];     // per wave: running max and sum
  __shared__ float wacc[W][G][128];        // per wave: unnormalised output
  // PH: workgroup = query head hq of KV head g (G == 1); else workgroup = KV head g, query heads g G + h
  // PH: block b serves query head (b % KV) gq + b / KV, so the gq workgroups
  // of a KV head are KV blocks apart: with KV = 8 they run on one XCD
  // (blocks go round-robin over the 8 XCDs) and share its L2 for the K / V rows
  const int gq = H / KV;
  const int g = PH ? blk % KV : blk;
  const int hq0 = PH ? g * gq + blk / KV : g * G;
  const bool writer = !PH || blk < KV;                     // appends the new K / V row
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kg = lane >> 2, q4 = lane & 3;
  // NB > 0: the entry loads are issued before the position is read,
  // clamped into the cache instead of to the cached rows
  const int p = NB > 0 ? 0 : pos[0];
  const int jmax_entry = max_len - 1;
  // this KV head's cache rows through buffer descriptors: 32-bit offsets, the
  // key index of a V load uniform (a scalar offset)
  const uint64_t head_bytes = (uint64_t)max_len * 256;
  const __amdgpu_buffer_rsrc_t rk =
      __builtin_amdgcn_make_buffer_rsrc((void*)(kc + (int64_t)g * max_len * 128), (short)0, (int)head_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rv =
      __builtin_amdgcn_make_buffer_rsrc((void*)(vc + (int64_t)g * max_len * 128), (short)0, (int)head_bytes, 0x00020000);
  int jmax = jmax_entry;
  auto load_k = [&](int b, u32x4 (&kr)[4]) {
    const int j = min(kBlock * b + 16 * w + kg, jmax);
    const int off = j * 256 + 16 * q4;
#pragma unroll
    for (int c = 0; c < 4; ++c) kr[c] = __builtin_amdgcn_raw_buffer_load_b128(rk, off + 64 * c, 0, 0);
  };
  auto load_v = [&](int b, uint32_t (&vr)[16]) {
#pragma unroll
    for (int u = 0; u < 16; ++u)
      vr[u] = __builtin_amdgcn_raw_buffer_load_b32(rv, 4 * lane, min(kBlock * b + 16 * w + u, jmax) * 256, 0);
  };
  constexpr int NR = NB > 0 ? NB : 2;      // blocks of K / V rows in registers
  u32x4 kR[NR][4];
  uint32_t vR[NR][16];
  if constexpr (NB > 0) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      load_k(b, kR[b]);
      load_v(b, vR[b]);
    }
  }
  const int pp = NB > 0 ? pos[0] : p;
  const bool cur = pp >= 0 && pp < max_len;                      // the new row fits in the cache
  const int n_old = pp < 0 ? 0 : (pp > max_len ? max_len : pp);  // cached keys 0 .. n_old - 1
  const int n = n_old + (cur ? 1 : 0);
  const int nb = (n + kBlock - 1) / kBlock;
  jmax = n_old > 0 ? n_old - 1 : 0;                              // later loads: clamped to a cached row
  if constexpr (NB == 0) {
    load_k(0, kR[0]);
    load_v(0, vR[0]);
    load_k(1, kR[1]);
    load_v(1, vR[1]);
  }
  if constexpr (WAIT) sync_wait(sync.sync, 0, sync.target);
  // rotary embedding of the q heads and the new key, KV append
  {
    const int pc = pp < 0 ? 0 : (pp >= max_len ? max_len - 1 : pp);
    for (int hh = w; hh < G + 2; hh += W) {
      const float c = cs[((int64_t)pc * 64 + lane) * 2], sn = cs[((int64_t)pc * 64 + lane) * 2 + 1];
      const int head = hh < G ? hq0 + hh : (hh == G ? H + g : H + KV + g);
      const uint16_t* src = qkv + (int64_t)head * 128;
      uint16_t a16, b16;
      if constexpr (WAIT) {
        // written by other workgroups of this launch (other XCDs): loads
        // that are coherent at agent scope, issued after the count was seen
        const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc((void*)src, (short)0, 256, 0x00020000);
        a16 = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(rq, 2 * lane, 0, kCoherentLoad);
        b16 = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(rq, 2 * lane + 128, 0, kCoherentLoad);
      } else {
        a16 = src[lane];
        b16 = src[lane + 64];
      }
      if (hh <= G) {
        const float a = bfv(a16), b = bfv(b16);
        const uint32_t ra = f32_to_bf16_rne(a * c - b * sn), rb = f32_to_bf16_rne(b * c + a * sn);
        uint16_t* d16 = (uint16_t*)(hh < G ? qs2[hh] : kp2);
        d16[lane] = (uint16_t)ra;
        d16[lane + 64] = (uint16_t)rb;
        if (hh == G) {
          if (cur && writer) {
            uint16_t* dst = kc + ((int64_t)g * max_len + pp) * 128;
            dst[lane] = (uint16_t)ra;
            dst[lane + 64] = (uint16_t)rb;
          }
        }
      } else {
        vp[lane] = bfv(a16);
        vp[lane + 64] = bfv(b16);
        if (cur && writer) {
          uint16_t* dst = vc + ((int64_t)g * max_len + pp) * 128;
          dst[lane] = a16;
          dst[lane + 64] = b16;
        }
      }
    }
  }
  __syncthreads();

  float m[G], l[G], acc[G][2];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.f;
    acc[h][0] = acc[h][1] = 0.f;
  }
  auto block = [&](int b, u32x4 (&kr)[4], uint32_t (&vr)[16]) {
    // scores of key j: four lanes, 32 dims (16 bf16 pairs) each, exact
    // products in fp32 (v_dot2), scaled after the sum
    const int j = kBlock * b + 16 * w + kg;
    uint32_t kw[16];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const u32x4 kv = kr[c];
      const uint32_t k0 = kv.x, k1 = kv.y, k2 = kv.z, k3 = kv.w;
      kw[4 * c] = k0; kw[4 * c + 1] = k1; kw[4 * c + 2] = k2; kw[4 * c + 3] = k3;
    }
    if (j >= n_old) {                                            // the new key (j == p), or past the end
#pragma unroll
      for (int e = 0; e < 16; ++e) kw[e] = kp2[16 * (e >> 2) + 4 * q4 + (e & 3)];
    }
    float sc[G];
#pragma unroll
    for (int h = 0; h < G; ++h) sc[h] = 0.f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const u32x4 qv = *(const u32x4*)&qs2[h][16 * c + 4 * q4];
        const uint32_t q0 = qv.x, q1 = qv.y, q2 = qv.z, q3 = qv.w;
        sc[h] = dot2_bf16(kw[4 * c], q0, sc[h]);
        sc[h] = dot2_bf16(kw[4 * c + 1], q1, sc[h]);
        sc[h] = dot2_bf16(kw[4 * c + 2], q2, sc[h]);
        sc[h] = dot2_bf16(kw[4 * c + 3], q3, sc[h]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int h = 0; h < G; ++h) {
      // sum over the key's four lanes (DPP quad permutations)
      float t = sc[h];
      t += __builtin_amdgcn_update_dpp(0.f, t, 0xB1, 0xF, 0xF, false);   // quad_perm [1, 0, 3, 2]
      t += __builtin_amdgcn_update_dpp(0.f, t, 0x4E, 0xF, 0xF, false);   // quad_perm [2, 3, 0, 1]
      sc[h] = j < n ? t * scale : -INFINITY;
      if (q4 == 0) ps[w][h][kg] = sc[h];
    }
    __builtin_amdgcn_wave_barrier();                             // LDS operations of a wave complete in order
    // running softmax over this wave's keys: every lane reads the block's 16
    // scores (broadcast reads) instead of reducing across lanes
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float mb = -INFINITY;
#pragma unroll
      for (int u4 = 0; u4 < 16; u4 += 4) {
        const float4 s4 = *(const float4*)&ps[w][h][u4];
        mb = fmaxf(fmaxf(mb, fmaxf(s4.x, s4.y)), fmaxf(s4.z, s4.w));
      }
      const float mn = fmaxf(m[h], mb);
      const float f = mn == -INFINITY ? 1.f : __expf(m[h] - mn);        // m = -inf: nothing to rescale
      const float pe = sc[h] == -INFINITY ? 0.f : __expf(sc[h] - mn);
      if (q4 == 0) pw[w][h][kg] = pe;
      // each key's first lane sums its own probability; the wave's lanes are
      // added once, at the end
      l[h] = fmaf(l[h], f, q4 == 0 ? pe : 0.f);
      acc[h][0] *= f;
      acc[h][1] *= f;
      m[h] = mn;
    }
    __builtin_amdgcn_wave_barrier();
    // P.V over the wave's 16 keys, lane l dims 2l, 2l + 1 (a key at or past
    // n_old is the new value row: held in LDS; past the end its p is 0)
    const float vn0 = vp[2 * lane], vn1 = vp[2 * lane + 1];
    float v0[16], v1[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const bool nw = kBlock * b + 16 * w + u >= n_old;         // uniform
      v0[u] = nw ? vn0 : bf16lo_to_f32(vr[u]);
      v1[u] = nw ? vn1 : bf16hi_to_f32(vr[u]);
    }
#pragma unroll
    for (int h = 0; h < G; ++h) {
#pragma unroll
      for (int u4 = 0; u4 < 16; u4 += 4) {
        const float4 pr4 = *(const float4*)&pw[w][h][u4];
        const float pr[4] = {pr4.x, pr4.y, pr4.z, pr4.w};
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          acc[h][0] = fmaf(pr[u], v0[u4 + u], acc[h][0]);
          acc[h][1] = fmaf(pr[u], v1[u4 + u], acc[h][1]);
        }
      }
    }
    __builtin_amdgcn_wave_barrier();
    if constexpr (NB == 0) {
      // the next block but one into these registers
      load_k(b + 2, kr);
      load_v(b + 2, vr);
    }
  };
  if constexpr (NB > 0) {
#pragma unroll
    for (int b = 0; b < NB; ++b)
      if (b < nb) block(b, kR[b], vR[b]);
  } else {
    int b = 0;
    for (; b + 1 < nb; b += 2) {
      block(b, kR[0], vR[0]);
      block(b + 1, kR[1], vR[1]);
    }
    if (b < nb) block(b, kR[0], vR[0]);
  }

  // combine the waves in wave order
#pragma unroll
  for (int h = 0; h < G; ++h) {
    const float lw = wave_sum_dpp(l[h]);                         // lane 63: the wave's sum
    if (lane == 63) {
      wm[w][h] = m[h];
      wl[w][h] = lw;
    }
  }
#pragma unroll
  for (int h = 0; h < G; ++h) {
    wacc[w][h][2 * lane] = acc[h][0];
    wacc[w][h][2 * lane + 1] = acc[h][1];
  }
  __syncthreads();
  for (int e = tid; e < G * 128; e += 64 * W) {
    const int h = e >> 7, d = e & 127;
    float M = -INFINITY;
#pragma unroll
    for (int k = 0; k < W; ++k) M = fmaxf(M, wm[k][h]);
    float L = 0.f, o = 0.f;
#pragma unroll
    for (int k = 0; k < W; ++k) {
      const float f = wm[k][h] == -INFINITY ? 0.f : __expf(wm[k][h] - M);
      L = fmaf(wl[k][h], f, L);
      o = fmaf(wacc[k][h][d], f, o);
    }
    const uint16_t ob = (uint16_t)f32_to_bf16_rne(L > 0.f ? o / L : 0.f);
    if constexpr (WAIT)   // read by the o projection's workgroups of this launch
      __builtin_amdgcn_raw_buffer_store_b16(ob, __builtin_amdgcn_make_buffer_rsrc(out, (short)0, H * 256, 0x00020000),
                                            (hq0 + h) * 256 + 2 * d, 0, kCoherentLoad);
    else
      out[(int64_t)(hq0 + h) * 128 + d] = ob;
  }
  if constexpr (WAIT) sync_count(sync.sync, 1, blk & (kSyncXcds - 1));
}

template <int G, int W = kDec1Waves, bool PH = false, int NB = 0>
__global__ __launch_bounds__(64 * W) void attn_decode1_kernel(const uint16_t* __restrict__ qkv,
                                                            const int32_t* __restrict__ pos,
                                                            const float* __restrict__ cs, int H, int KV,
                                                            int max_len, float scale, uint16_t* __restrict__ kc,
                                                            uint16_t* __restrict__ vc, uint16_t* __restrict__ out) {
  attn_decode1_body<G, W, PH, NB>(qkv, pos, cs, H, KV, max_len, scale, kc, vc, out, (int)blockIdx.x,
                                  (int)threadIdx.x, AttnSync{nullptr, 0u});
}


static int host_dec_splits(int64_t max_len) {
  const int64_t s = (max_len + 63) / 64;
  return (int)(s < 1 ? 1 : (s > kDecMaxSplits ? kDecMaxSplits : s));
}

extern "C" int64_t bf16x_attention_decode_lds(int64_t n_heads, int64_t n_kv_heads, int64_t max_len) {
  if (n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads != 0 || max_len <= 0 || max_len > INT32_MAX / 8)
    return -1;
  const int64_t G = n_heads / n_kv_heads;
  if (G != 1 && G != 2 && G != 4 && G != 8) return -1;
  const int64_t S = host_dec_splits(max_len);
  const int64_t range = (max_len + S - 1) / S;
  const int64_t bytes = 4 * std::max<int64_t>(G * range, 4 * G * 128);
  return bytes <= 48 * 1024 ? bytes : -1;
}

extern "C" int64_t bf16x_attention_decode_workspace(int64_t n_heads, int64_t n_kv_heads, int64_t max_len) {
  if (bf16x_attention_decode_lds(n_heads, n_kv_heads, max_len) < 0) return -1;
  const int64_t G = n_heads / n_kv_heads;
  // counters first (one per KV head, 256-byte aligned block), then the partial results
  return 256 * ((4 * n_kv_heads + 255) / 256) + 4 * n_kv_heads * host_dec_splits(max_len) * G * 130;
}

extern "C" int bf16x_attention_decode(const uint16_t* qkv, const int32_t* pos, const float* cos_sin, int64_t n_heads,
                                      int64_t n_kv_heads, int64_t head_dim, int64_t max_len, float scale,
                                      uint16_t* k_cache, uint16_t* v_cache, void* workspace, int64_t workspace_bytes,
                                      uint16_t* out, bf16x_stream_t stream) {
  if (!qkv || !pos || !cos_sin || !k_cache || !v_cache || !out || !workspace) return BF16X_EARG;
  if (head_dim != 128 || n_kv_heads > 65535) return BF16X_ESHAPE;
  const int64_t lds = bf16x_attention_decode_lds(n_heads, n_kv_heads, max_len);
  if (lds < 0) return BF16X_ESHAPE;
  if (workspace_bytes < bf16x_attention_decode_workspace(n_heads, n_kv_heads, max_len)) return BF16X_ECAPACITY;
  if (!aligned16(k_cache) || !aligned16(workspace) || !aligned4(v_cache) || !aligned4(cos_sin) || !aligned2(qkv) ||
      !aligned2(out))
    return BF16X_EARG;
  const int G = (int)(n_heads / n_kv_heads);
  hipStream_t st = (hipStream_t)stream;
  if (max_len <= kDec1MaxLen && tuning(BF16X_TUNE_ATTN_SPLIT) != 1) {
#define BF16X_DEC1(GG)                                                                                          \
  hipLaunchKernelGGL(attn_decode1_kernel<GG>, dim3((unsigned)n_kv_heads), dim3(64 * kDec1Waves), 0, st, qkv, pos, \
                     cos_sin,                                                                                   \
                     (int)n_heads, (int)n_kv_heads, (int)max_len, scale, k_cache, v_cache, out)
    switch (G) {
      case 1: BF16X_DEC1(1); break;
      case 2: BF16X_DEC1(2); break;
      case 4: BF16X_DEC1(4); break;
      default: BF16X_DEC1(8); break;
    }
#undef BF16X_DEC1
    return launch_status();
  }
  if (max_len <= kDecHMaxLen && tuning(BF16X_TUNE_ATTN_SPLIT) != 1) {
    hipLaunchKernelGGL((attn_decode1_kernel<1, kDecHWaves, true, kDecHBlocks>), dim3((unsigned)n_heads),
                       dim3(64 * kDecHWaves), 0, st, qkv, pos, cos_sin, (int)n_heads, (int)n_kv_heads, (int)max_len,
                       scale, k_cache, v_cache, out);
    return launch_status();
  }
  const int S = host_dec_splits(max_len);
  uint32_t* cnt = (uint32_t*)workspace;
  float* part = (float*)((char*)workspace + 256 * ((4 * n_kv_heads + 255) / 256));
#define BF16X_DEC(GG)                                                                                            \
  hipLaunchKernelGGL(attn_decode_kernel<GG>, dim3((unsigned)n_kv_heads, (unsigned)S), dim3(256), (size_t)lds, st, \
                     qkv, pos, cos_sin, (int)n_heads, (int)n_kv_heads, (int)max_len, scale, k_cache, v_cache, part, \
                     cnt, out)
  switch (G) {
    case 1: BF16X_DEC(1); break;
    case 2: BF16X_DEC(2); break;
    case 4: BF16X_DEC(4); break;
    default: BF16X_DEC(8); break;
  }
#undef BF16X_DEC
  return launch_status();
}

// ---------------------------------------------------------------------------
// The front of a decoder layer for one decode token in one launch: the qkv
// projection (with its RMSNorm from the residual GEMV's slots), the decode
// attention and, optionally, the o projection with the residual add.
// Hardware workgroups of 1024 threads, in dispatch order:
//  - 0 .. H-1: the per-query-head attention workgroups of attn_decode1_kernel
//    (16 waves, the 768-row variant); they request their K / V rows and the
//    position at entry, i.e. while the GEMV streams its weights;
//  - nq qkv GEMV workgroups, each four 4-wave workgroups of gemv_pipe_body
//    (XM = 2, the rows of bf16x_gemv_prenormed); they wait for nothing;
//  - no o GEMV workgroups (four of gemv_pipe_body with the residual epilogue
//    each, the rows and slots of bf16x_gemv_residual); they request their
//    first rows, then wait for the attention.
// Stages are ordered by the counters of `sync` (see sync_wait).  The
// attention workgroups wait for the qkv workgroups, which are dispatched
// after them: those waits end because the attention workgroups (one per CU
// at most) hold no more than half of the device's CUs, which the launcher
// checks against the device's CU count, so the qkv workgroups always find
// CUs to run on.  The o workgroups, which wait for the attention, are
// dispatched after every qkv workgroup, so they cannot keep one from
// starting.  Outputs are bit-identical to bf16x_gemv_prenormed,
// bf16x_attention_decode and bf16x_gemv_residual in sequence.
constexpr int kQaSubs = 4;                      // GEMV workgroups per hardware workgroup
constexpr int kQaThreads = 64 * kDecHWaves;     // 1024
static_assert(kQaThreads == 256 * kQaSubs, "four 256-thread GEMV workgroups per attention-sized workgroup");
// x staging of one GEMV workgroup (NS = 2): 8 KB.  The four GEMV workgroups
// of a hardware workgroup stage the same x (it depends only on the thread's
// slot), so they share one copy: each thread's store is made by the
// matching thread of every workgroup with the same value, before the barrier
// that every reader waits at.
constexpr int kQaSubLdsWords = 2 * 64 * 4 * 4;

// The o projection's wait: the attention workgroups (stage 1) are done.
struct OWait {
  static constexpr bool active = true;
  uint32_t* sync;
  uint32_t target;
  __device__ void operator()() const { sync_wait(sync, 1, target); }
};

// Inverse of xcd_row_block(., nb): the block index of a standalone launch of
// nb workgroups whose row block is q (its slot of bf16x_gemv_residual).
__device__ __forceinline__ int xcd_block_of_row_block(int q, int nb) {
  if (nb < 8) return q;
  const int per = nb / 8, extra = nb - per * 8;
  int x = 0;
#pragma unroll
  for (int t = 1; t < 8; ++t) x += q >= t * per + min(t, extra) ? 1 : 0;
  return (q - (x * per + min(x, extra))) * 8 + x;
}

struct OStage {
  const uint16_t* res_in;
  uint16_t* res_out;
  float* slots;
  const uint32_t* sign;
  const uint32_t* mant;
  const uint32_t* delta;
  const uint16_t* emax2;
  const uint32_t* tile_off;
  const uint32_t* tile_ent;
  const uint8_t* tile_sat;
  int64_t out_f;
  uint16_t* y;
  int nblocks;         // workgroups of the standalone residual launch (its slots)
  int iters;           // row groups of 4 per workgroup there
};

template <bool EXACT, bool FULL>
__global__ __launch_bounds__(kQaThreads) void layer_front_kernel(
    const uint16_t* h, const uint32_t* __restrict__ sign, const uint32_t* __restrict__ mant,
    const uint32_t* __restrict__ delta, const uint16_t* __restrict__ emax2, const uint32_t* __restrict__ tile_off,
    const uint32_t* __restrict__ tile_ent, const uint8_t* __restrict__ tile_sat, int64_t out_f, int64_t in_f,
    int iters, NormArgs na, uint16_t* qkv, const int32_t* __restrict__ pos, const float* __restrict__ cs, int H,
    int KV, int max_len, float scale, uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, uint16_t* attn_out,
    int nq, OStage os, uint32_t* sync, uint32_t* clear) {
  extern __shared__ uint32_t qa_lds[];
  const int b = (int)blockIdx.x;
  if (b == 0 && threadIdx.x == 0 && clear != nullptr) {
    // the launch before this one (finished: stream order) used `clear`
#pragma unroll
    for (int c = 0; c < kSyncStages * kSyncXcds; ++c) clear[c * kSyncStride] = 0u;
  }
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);   // kept in a scalar register
  const int sub = wave >> 2;
  if (b < H) {
    attn_decode1_body<1, kDecHWaves, true, kDecHBlocks, true>(qkv, pos, cs, H, KV, max_len, scale, kc, vc,
                                                              attn_out, b, (int)threadIdx.x,
                                                              AttnSync{sync, (uint32_t)nq});
    return;
  }
  // H % 8 == 0 and nq % 8 == 0 (checked by the launcher): GEMV workgroup gb
  // of either stage runs on XCD gb % 8
  if (b < H + nq) {
    const int gb = b - H;
    const int lb = kQaSubs * xcd_row_block(gb, nq) + sub;
    gemv_pipe_body<2, 1, BF16X_BF16, EXACT, FULL, 0, 2, 0, kQaSubs, NoPreWait, true>(
        h, sign, mant, delta, emax2, tile_off, tile_ent, tile_sat, out_f, in_f, iters, qkv, na,
        ResArgs{nullptr, nullptr, nullptr}, (int)threadIdx.x & 255, sub, kQaSubs * gb + sub, lb, qa_lds);
    sync_count(sync, 0, gb & (kSyncXcds - 1));
    return;
  }
  const int ob = b - H - nq, nob = (int)gridDim.x - H - nq;
  const int lb = kQaSubs * xcd_row_block(ob, nob) + sub;       // row groups lb iters ..
  gemv_pipe_body<2, 1, BF16X_BF16, EXACT, FULL, 0, 0, 1, kQaSubs, OWait>(
      attn_out, os.sign, os.mant, os.delta, os.emax2, os.tile_off, os.tile_ent, os.tile_sat, os.out_f,
      (int64_t)H * 128, os.iters, os.y, NormArgs{nullptr, nullptr, nullptr, 0.f, nullptr, 0},
      ResArgs{os.res_in, os.res_out, os.slots}, (int)threadIdx.x & 255, sub,
      lb < os.nblocks ? xcd_block_of_row_block(lb, os.nblocks) : -1, lb, qa_lds, OWait{sync, (uint32_t)H});
}

extern "C" int64_t bf16x_layer_front_sync_bytes(void) { return 4 * (kSyncErrWord + 4); }

extern "C" int bf16x_layer_front_decode(
    const void* h, const uint16_t* norm_weight, float eps, const float* slots, int64_t n_slots, const int32_t* sign,
    int64_t n_sign, const int32_t* mant, int64_t n_mant, const int32_t* delta, int64_t n_delta, const uint8_t* emax,
    int64_t n_emax, const uint32_t* tile_off, const uint32_t* tile_ent, const uint8_t* tile_sat, int64_t out_f,
    int64_t in_f, int32_t mode, uint16_t* qkv, const int32_t* pos, const float* cos_sin, int64_t n_heads,
    int64_t n_kv_heads, int64_t head_dim, int64_t max_len, float scale, uint16_t* k_cache, uint16_t* v_cache,
    uint16_t* attn_out, const uint16_t* o_residual_in, uint16_t* o_residual_out, float* o_slots, int64_t o_n_slots,
    const int32_t* o_sign, int64_t o_n_sign, const int32_t* o_mant, int64_t o_n_mant, const int32_t* o_delta,
    int64_t o_n_delta, const uint8_t* o_emax, int64_t o_n_emax, const uint32_t* o_tile_off,
    const uint32_t* o_tile_ent, const uint8_t* o_tile_sat, int64_t o_out_f, uint16_t* o_y, void* sync,
    void* sync_clear, int64_t sync_bytes, bf16x_stream_t stream) {
  if (!h || !norm_weight || !slots || !sign || !mant || !delta || !emax || !qkv || !pos || !cos_sin || !k_cache ||
      !v_cache || !sync || !attn_out)
    return BF16X_EARG;
  if (mode != BF16X_EXACT && mode != BF16X_SATURATED) return BF16X_EARG;
  const bool ex = mode == BF16X_EXACT;
  if (ex && (!tile_off || !tile_ent || !tile_sat)) return BF16X_EARG;
  int rc = check_dict(out_f, in_f, 16, n_sign, n_mant, n_delta, n_emax);
  if (rc) return rc;
  if (sync_bytes < bf16x_layer_front_sync_bytes()) return BF16X_ECAPACITY;
  if (sync_clear == sync) return BF16X_EARG;
  if (n_slots <= 0) return BF16X_EARG;
  if (n_slots > 64 * kMaxSlotsPerLane) return BF16X_ECAPACITY;
  // the attention side: the per-query-head kernel's shapes; the waiting
  // attention workgroups must hold at most half of this device's CUs
  if (head_dim != 128 || n_kv_heads <= 0 || n_heads <= 0 || n_heads % n_kv_heads != 0 || n_heads % 8 != 0 ||
      n_heads > 128 || max_len <= kDec1MaxLen || max_len > kDecHMaxLen)
    return BF16X_ESHAPE;
  if (2 * n_heads > device_cus()) return BF16X_ESHAPE;
  // the GEMV side: 64 < in_f / 32 <= 128 (two 64-atom steps per wave, one
  // wave per row), out_f = the qkv rows of the attention
  if (out_f != (n_heads + 2 * n_kv_heads) * 128) return BF16X_ESHAPE;
  const int64_t P = in_f >> 5;
  if (in_f % 32 != 0 || P <= 64 || P > 128 || (out_f + 1) * P * 28 >= (int64_t)0xFFFFFFFF) return BF16X_ESHAPE;
  if (!aligned4(h) || !aligned4(norm_weight) || !aligned4(slots) || !aligned4(sign) || !aligned4(mant) ||
      !aligned4(delta) || !aligned2(emax) || !aligned16(k_cache) || !aligned4(v_cache) || !aligned4(cos_sin) ||
      !aligned4(qkv) || !aligned4(attn_out) || !aligned16(sync) || !aligned16(sync_clear))
    return BF16X_EARG;
  // the o stage (optional: o_sign NULL): a packed dict [o_out_f, n_heads * 128]
  // in the same mode and with in_f's step count, residual buffers of o_out_f
  const bool has_o = o_sign != nullptr;
  OStage os{};
  int64_t no = 0;
  int o_iters = 1;
  if (has_o) {
    if (!o_residual_in || !o_residual_out || !o_slots || !o_mant || !o_delta || !o_emax || !o_y) return BF16X_EARG;
    if (ex && (!o_tile_off || !o_tile_ent || !o_tile_sat)) return BF16X_EARG;
    if (n_heads * 128 != in_f) return BF16X_ESHAPE;
    rc = check_dict(o_out_f, in_f, 16, o_n_sign, o_n_mant, o_n_delta, o_n_emax);
    if (rc) return rc;
    if ((o_out_f + 1) * P * 28 >= (int64_t)0xFFFFFFFF) return BF16X_ESHAPE;
    // o_slots may be `slots`: the o stage writes them after every qkv
    // workgroup has read its sums (it waits for the attention, which waits
    // for the qkv GEMV)
    if ((const void*)o_residual_out == (const void*)o_residual_in || o_residual_out == o_y ||
        (const void*)o_residual_out == h)
      return BF16X_EARG;
    // the o workgroups take the row groups of the standalone residual
    // launch's workgroups (1 or 2 groups of 4 rows each) and write their
    // slots (through the XCD mapping)
    const int64_t nb_res = bf16x_gemv_residual_slots(o_out_f, in_f);
    const int64_t groups_o = (o_out_f + 3) / 4;
    if (nb_res <= 0) return BF16X_ESHAPE;
    o_iters = (int)((groups_o + nb_res - 1) / nb_res);
    if (o_iters > 2 || (groups_o + o_iters - 1) / o_iters != nb_res) return BF16X_ESHAPE;
    if (o_n_slots < nb_res) return BF16X_ECAPACITY;
    if (!aligned4(o_sign) || !aligned4(o_mant) || !aligned4(o_delta) || !aligned2(o_emax) ||
        !aligned2(o_residual_in) || !aligned2(o_residual_out) || !aligned4(o_slots) || !aligned2(o_y))
      return BF16X_EARG;
    no = (nb_res + kQaSubs - 1) / kQaSubs;
    os = OStage{o_residual_in, o_residual_out, o_slots, (const uint32_t*)o_sign, (const uint32_t*)o_mant,
                (const uint32_t*)o_delta, (const uint16_t*)o_emax, ex ? o_tile_off : nullptr,
                ex ? o_tile_ent : nullptr, ex ? o_tile_sat : nullptr, o_out_f, o_y, (int)nb_res, o_iters};
  }
  const bool full = P == 128;
  // GEMV rows per 4-wave workgroup as the standalone launch (bf16x_gemv_prenormed)
  const int64_t groups = (out_f + 3) / 4;
  const int iters = groups >= 1024 ? 2 : 1;
  const int64_t vblocks = (groups + iters - 1) / iters;
  const int64_t nq = 8 * ((vblocks + 8 * kQaSubs - 1) / (8 * kQaSubs));   // a multiple of 8 (XCD mapping)
  if (nq + n_heads + no > INT32_MAX) return BF16X_ESHAPE;
  const NormArgs na{nullptr, norm_weight, nullptr, eps, slots, (int)n_slots};
  const size_t lds = (size_t)kQaSubLdsWords * 4;
  const uint32_t *to = ex ? tile_off : nullptr, *te = ex ? tile_ent : nullptr;
  const uint8_t* ts = ex ? tile_sat : nullptr;
#define BF16X_LF(EX_, FULL_)                                                                                      \
  hipLaunchKernelGGL((layer_front_kernel<EX_, FULL_>), dim3((unsigned)(n_heads + nq + no)), dim3(kQaThreads), lds, \
                     (hipStream_t)stream, (const uint16_t*)h, (const uint32_t*)sign, (const uint32_t*)mant,         \
                     (const uint32_t*)delta, (const uint16_t*)emax, to, te, ts, out_f, in_f, iters, na, qkv, pos,  \
                     cos_sin, (int)n_heads, (int)n_kv_heads, (int)max_len, scale, k_cache, v_cache, attn_out,     \
                     (int)nq, os, (uint32_t*)sync, (uint32_t*)sync_clear)
  if (ex) { if (full) BF16X_LF(true, true); else BF16X_LF(true, false); }
  else { if (full) BF16X_LF(false, true); else BF16X_LF(false, false); }
#undef BF16X_LF
  return launch_status();
}

extern "C" int bf16x_silu_mul(const uint16_t* gate_up, int64_t tokens, int64_t ffn, int32_t layout, uint16_t* out,
                              bf16x_stream_t stream) {
  if (!gate_up || !out || tokens < 0 || (layout != BF16X_SPLIT && layout != BF16X_PAIRS8)) return BF16X_EARG;
  if (ffn <= 0 || ffn % 8 != 0 || ffn > INT32_MAX / 2) return BF16X_ESHAPE;
  if (!aligned16(gate_up) || !aligned16(out)) return BF16X_EARG;
  if (tokens == 0) return BF16X_OK;
  const int64_t chunks = tokens * (ffn / 8);
  const int64_t grid = std::min<int64_t>((chunks + 255) / 256, 8192);
  if (layout == BF16X_PAIRS8)
    hipLaunchKernelGGL(silu_mul_kernel<true>, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, gate_up,
                       tokens, (int)ffn, out);
  else
    hipLaunchKernelGGL(silu_mul_kernel<false>, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, gate_up,
                       tokens, (int)ffn, out);
  return launch_status();
}

extern "C" int64_t bf16x_greedy_workspace_bytes(void) { return (int64_t)sizeof(GreedyWs); }

extern "C" int bf16x_greedy(const uint16_t* logits, int64_t vocab, int64_t* token, int32_t* state, int32_t* history,
                            int64_t history_len, void* workspace, int64_t workspace_bytes, bf16x_stream_t stream) {
  if (!logits || !token || !state || (!history && history_len > 0) || history_len < 0 || !workspace)
    return BF16X_EARG;
  if (workspace_bytes < (int64_t)sizeof(GreedyWs)) return BF16X_ECAPACITY;
  if (!aligned16(workspace)) return BF16X_EARG;
  // greedy_kernel steps its int indices by 1024 * 8 per batch element and
  // 2 elements per batch, its ranges by a multiple of 8: the last indices
  // must not overflow
  if (vocab <= 0 || vocab > INT32_MAX - 4 * 1024 * 8 * kGreedyBlocks || history_len > INT32_MAX) return BF16X_ESHAPE;
  if (!aligned16(logits) || !aligned4(state) || ((uintptr_t)token & 7u)) return BF16X_EARG;
  hipLaunchKernelGGL(greedy_kernel, dim3(kGreedyBlocks), dim3(1024), 0, (hipStream_t)stream, logits, (int)vocab,
                     token, state, history, (int)history_len, (GreedyWs*)workspace);
  return launch_status();
}
