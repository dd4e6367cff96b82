/*
 * bf16x_llama.h -- decoder-stack kernels of the Llama-style harness that
 * drives the BF16X linears (libbf16x_hip.so, same library as bf16x_hip.h).
 *
 * None of these entry points has a counterpart in the reference's own code:
 * the reference's harness (bench_fused_cpm5.py:27-57) runs the ops between the
 * linears (RMSNorm, rotary embedding, KV cache, attention, SwiGLU, greedy
 * argmax) through Hugging Face transformers modules in PyTorch.  They exist so
 * that one decode step is a short, fixed sequence of launches that a HIP
 * graph can capture, with the token position kept on the device.
 *
 * Conventions (as in bf16x_hip.h): device pointers, an explicit stream, an
 * int status (0 ok, < 0 BF16X_E* invalid argument, > 0 hipError_t).
 * Activations are bf16 (uint16 bits), row-major; arithmetic is fp32.
 *
 * Layouts
 *  - qkv      [tokens][(n_heads + 2 n_kv_heads) * head_dim]: q heads, then k
 *             heads, then v heads (one fused projection)
 *  - q        [tokens][n_heads][head_dim]
 *  - k/v cache [n_kv_heads][max_len][head_dim] per layer
 *  - cos_sin  fp32 [max_len][head_dim / 2][2] (cos, sin) of position x
 *             inverse frequency, rotate-half convention (pairs i, i + d/2)
 *  - gate_up  [tokens][2 ffn]: gate columns, then up columns
 *  - pos      int32 on the device: position of the first token of the call
 *  - state    int32 [2] on the device: {position of the next token, number
 *             of tokens written to history}
 */
#ifndef BF16X_LLAMA_H
#define BF16X_LLAMA_H

#include <stdint.h>

#include "bf16x_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* flags of bf16x_rmsnorm */
enum { BF16X_NORM_ADD = 1, BF16X_NORM_STORE = 2 };

/* RMSNorm of `rows` rows of n elements, with the residual stream folded in.
 * Row r of the input is x[r] (or x[row_idx[r]], an embedding gather, when
 * row_idx is not NULL; indices are clamped to [0, x_rows)).  With
 * BF16X_NORM_ADD, h = bf16(x + residual[r]), else h = x; with
 * BF16X_NORM_STORE, residual[r] = h.  out[r] = bf16(bf16(h * rsqrt(mean(h^2)
 * + eps)) * weight): the two roundings of the Hugging Face LlamaRMSNorm.
 * n % 8 == 0, n <= 8192; x, residual, weight, out 16-byte aligned. */
int bf16x_rmsnorm(const uint16_t* x, const int64_t* row_idx, int64_t x_rows, uint16_t* residual,
                  const uint16_t* weight, uint16_t* out, int64_t rows, int64_t n, float eps, int32_t flags,
                  bf16x_stream_t stream);

/* Rotary embedding of the q and k heads of `tokens` tokens at positions
 * *pos + t, q written to q_out, rotated k and plain v appended to the caches
 * at those positions (positions >= max_len are not written).  head_dim 128. */
int bf16x_rope_kv(const uint16_t* qkv, int64_t tokens, const int32_t* pos, const float* cos_sin,
                  int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, int64_t max_len,
                  uint16_t* q_out, uint16_t* k_cache, uint16_t* v_cache, bf16x_stream_t stream);

/* Causal grouped-query attention: query t (position *pos + t) of head h
 * attends to keys 0 .. *pos + t of kv head h / (n_heads / n_kv_heads);
 * softmax(scale q.k) v in fp32, out [tokens][n_heads * head_dim] bf16.
 * head_dim 128, max_len <= 16384. */
int bf16x_attention(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache, const int32_t* pos,
                    int64_t tokens, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, int64_t max_len,
                    float scale, uint16_t* out, bf16x_stream_t stream);

/* One decode token (at position *pos) through rotary embedding, KV append and
 * attention in one launch: bf16x_rope_kv followed by bf16x_attention with
 * tokens = 1.  Up to max_len = 256 one workgroup per KV head takes all keys,
 * up to max_len = 768 one workgroup per query head (all K / V rows requested
 * at once), in both cases without touching the workspace; above, the keys are split into ranges
 * served by separate workgroups whose partial results meet in `workspace`
 * (bf16x_attention_decode_workspace bytes, 16-byte aligned, required in both
 * cases).  The workspace starts with one counter per KV head
 * that must be zero before the first call; every call leaves it zero, so the
 * caller zeroes the workspace once when allocating it.  Calls sharing a
 * workspace must not overlap.  qkv [(n_heads + 2 n_kv_heads) * 128],
 * out [n_heads * 128].  bf16x_attention_decode_lds(...) gives the bytes of
 * workgroup memory used, -1 when the shape is not supported (head ratio other
 * than 1, 2, 4, 8, or max_len too long); the workspace query returns -1 then. */
int64_t bf16x_attention_decode_lds(int64_t n_heads, int64_t n_kv_heads, int64_t max_len);
int64_t bf16x_attention_decode_workspace(int64_t n_heads, int64_t n_kv_heads, int64_t max_len);
int bf16x_attention_decode(const uint16_t* qkv, const int32_t* pos, const float* cos_sin, int64_t n_heads,
                           int64_t n_kv_heads, int64_t head_dim, int64_t max_len, float scale,
                           uint16_t* k_cache, uint16_t* v_cache, void* workspace, int64_t workspace_bytes,
                           uint16_t* out, bf16x_stream_t stream);

/* SwiGLU: out[t][i] = bf16(bf16(silu(gate_i)) * up_i) of the gate_up row t.
 * layout 0: gate columns 0 .. ffn-1, then up columns (gate_i at i, up_i at
 * ffn + i); layout 1 (BF16X_PAIRS8): groups of 8 columns [gate 4b .. 4b+3,
 * up 4b .. 4b+3] (gate_i at 8(i/4) + i%4, up_i at 8(i/4) + 4 + i%4), the row
 * order bf16x_gemv_swiglu consumes.  ffn % 8 == 0, 16-byte aligned buffers. */
enum { BF16X_SPLIT = 0, BF16X_PAIRS8 = 1 };
int bf16x_silu_mul(const uint16_t* gate_up, int64_t tokens, int64_t ffn, int32_t layout, uint16_t* out,
                   bf16x_stream_t stream);

/* Fused decode+GEMV with the SwiGLU epilogue: a packed dict [2 ffn, in_f]
 * whose rows are in the BF16X_PAIRS8 order gives out[i] = bf16(bf16(silu(
 * bf16(W x)_gate_i)) * bf16(W x)_up_i), i < ffn, with the rounding of
 * bf16x_gemv followed by bf16x_silu_mul.  x bf16 (4-byte aligned), 2 ffn % 8
 * == 0, in_f <= 4096 (one wave per row); arguments otherwise as bf16x_gemv
 * (sub 16).  Replaces the gate/up projections and the activation of the
 * reference harness's MLP (three modules of the Hugging Face model). */
int bf16x_gemv_swiglu(const void* x, const int32_t* sign, int64_t n_sign, const int32_t* mant, int64_t n_mant,
                      const int32_t* delta, int64_t n_delta, const uint8_t* emax, int64_t n_emax,
                      const uint32_t* tile_off, const uint32_t* tile_ent, const uint8_t* tile_sat, int64_t out_f,
                      int64_t in_f, int32_t mode, uint16_t* out, bf16x_stream_t stream);

/* Fused decode+GEMV whose input is normalised inside the kernel: with
 * h = bf16(x + residual_in) (h = x when residual_in is NULL), the rows are
 * multiplied with bf16(bf16(h * rsqrt(mean(h^2) + eps)) * norm_weight), the
 * bf16x_rmsnorm result; h is stored to residual_out (NULL: not stored; it
 * must not alias x or residual_in).  epilogue 0: y = the GEMV (out_f values);
 * 1: the SwiGLU epilogue of bf16x_gemv_swiglu.  One token, in_f <= 4096,
 * x / residuals / norm_weight 4-byte aligned.  Folds the RMSNorm (and the
 * residual add) that precedes a projection into it. */
int bf16x_gemv_norm(const void* x, const uint16_t* residual_in, const uint16_t* norm_weight,
                    uint16_t* residual_out, float eps, const int32_t* sign, int64_t n_sign, const int32_t* mant,
                    int64_t n_mant, const int32_t* delta, int64_t n_delta, const uint8_t* emax, int64_t n_emax,
                    const uint32_t* tile_off, const uint32_t* tile_ent, const uint8_t* tile_sat, int64_t out_f,
                    int64_t in_f, int32_t mode, int32_t epilogue, uint16_t* y, bf16x_stream_t stream);

/* Fused decode+GEMV with the residual add of the layer it closes (the o and
 * down projections): y = W . x as bf16x_gemv (bf16 x, in_f <= 16384), then
 * h = bf16(y + residual_in) is stored to residual_out (residual_out may be
 * residual_in; it must not alias x or y) and each workgroup b stores the sum
 * of h^2 over its rows to slots[b], b < bf16x_gemv_residual_slots(out_f,
 * in_f) (n_slots at least that; fp32, 4-byte aligned).  The next projection's
 * RMSNorm then takes its sum of squares from the slots
 * (bf16x_gemv_prenormed) instead of a launch of its own.  Folds the residual
 * add and the statistics of the reference harness's post-attention /
 * post-MLP RMSNorm into the projection before it. */
int64_t bf16x_gemv_residual_slots(int64_t out_f, int64_t in_f);
int bf16x_gemv_residual(const void* x, const uint16_t* residual_in, uint16_t* residual_out, float* slots,
                        int64_t n_slots, const int32_t* sign, int64_t n_sign, const int32_t* mant, int64_t n_mant,
                        const int32_t* delta, int64_t n_delta, const uint8_t* emax, int64_t n_emax,
                        const uint32_t* tile_off, const uint32_t* tile_ent, const uint8_t* tile_sat, int64_t out_f,
                        int64_t in_f, int32_t mode, uint16_t* y, bf16x_stream_t stream);

/* Fused decode+GEMV of RMSNorm(h) * norm_weight with the sum of h^2 given as
 * n_slots partial sums (the slots of a bf16x_gemv_residual launch, added in
 * slot order): the rows are multiplied with bf16(bf16(h * rsqrt(sum / in_f +
 * eps)) * norm_weight).  epilogue 0 / 1 as bf16x_gemv_norm; h and norm_weight
 * bf16, 4-byte aligned, in_f <= 4096. */
int bf16x_gemv_prenormed(const void* h, const uint16_t* norm_weight, float eps, const float* slots, int64_t n_slots,
                         const int32_t* sign, int64_t n_sign, const int32_t* mant, int64_t n_mant,
                         const int32_t* delta, int64_t n_delta, const uint8_t* emax, int64_t n_emax,
                         const uint32_t* tile_off, const uint32_t* tile_ent, const uint8_t* tile_sat, int64_t out_f,
                         int64_t in_f, int32_t mode, int32_t epilogue, uint16_t* y, bf16x_stream_t stream);

/* The front of a decoder layer for one decode token in one launch: the qkv
 * projection bf16x_gemv_prenormed (epilogue 0) into qkv, the decode attention
 * bf16x_attention_decode (tokens = 1) into attn_out, and, when o_sign is not
 * NULL, the o projection with the residual add bf16x_gemv_residual(attn_out,
 * o_residual_in, o_residual_out, o_slots, o_*) into o_y; results are
 * bit-identical to those launches in sequence.  The stages are ordered by
 * device counters in `sync` instead of launch boundaries: the attention
 * workgroups request their K / V cache rows while the qkv projection streams
 * its weights, and the o projection's workgroups request their first rows
 * while the attention runs.  Shapes: head_dim 128, n_heads % 8 == 0,
 * n_heads <= 128, 256 < max_len <= 768 (the one-workgroup-per-query-head
 * attention), out_f = (n_heads + 2 n_kv_heads) * 128, 2048 < in_f <= 4096,
 * in_f % 32 == 0; the o stage: o dict [o_out_f, in_f] with in_f = n_heads *
 * 128, in the same mode, a shape bf16x_gemv_residual runs with one or two
 * groups of 4 rows per workgroup (it writes the bf16x_gemv_residual_slots(
 * o_out_f, in_f) slots of that launch).  `sync`: bf16x_layer_front_sync_bytes()
 * bytes, 16-byte aligned, all zero when the launch starts; the launch zeroes
 * `sync_clear` (NULL: none; never `sync`), which must be the buffer of a
 * launch that stream order has finished.  Consecutive launches therefore use
 * different buffers, each clearing its predecessor's.  Word 1024 of `sync`
 * becomes 1 if a wait ran out (a few tenths of a second; the outputs are then
 * not valid); the caller clears it. */
int64_t bf16x_layer_front_sync_bytes(void);
int bf16x_layer_front_decode(const void* h, const uint16_t* norm_weight, float eps, const float* slots, int64_t n_slots,
                             const int32_t* sign, int64_t n_sign, const int32_t* mant, int64_t n_mant,
                             const int32_t* delta, int64_t n_delta, const uint8_t* emax, int64_t n_emax,
                             const uint32_t* tile_off, const uint32_t* tile_ent, const uint8_t* tile_sat,
                             int64_t out_f, int64_t in_f, int32_t mode, uint16_t* qkv, const int32_t* pos,
                             const float* cos_sin, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim,
                             int64_t max_len, float scale, uint16_t* k_cache, uint16_t* v_cache, uint16_t* attn_out,
                             const uint16_t* o_residual_in, uint16_t* o_residual_out, float* o_slots,
                             int64_t o_n_slots, const int32_t* o_sign, int64_t o_n_sign, const int32_t* o_mant,
                             int64_t o_n_mant, const int32_t* o_delta, int64_t o_n_delta, const uint8_t* o_emax,
                             int64_t o_n_emax, const uint32_t* o_tile_off, const uint32_t* o_tile_ent,
                             const uint8_t* o_tile_sat, int64_t o_out_f, uint16_t* o_y, void* sync,
                             void* sync_clear, int64_t sync_bytes, bf16x_stream_t stream);

/* Bytes of bf16x_greedy's workspace. */
int64_t bf16x_greedy_workspace_bytes(void);

/* Greedy step: token[0] = argmax(logits[0 .. vocab)) (the first maximum),
 * history[state[1]] = token[0] when state[1] < history_len, then state[1]++
 * and state[0]++.  logits 16-byte aligned.  The launch's workgroups meet in
 * `workspace` (bf16x_greedy_workspace_bytes, 16-byte aligned, zeroed once by
 * the caller before its first use; every call puts its counter, the first
 * word, back to zero): calls
 * with different workspaces are independent, calls sharing one must not
 * overlap (stream order, one graph replay at a time). */
int bf16x_greedy(const uint16_t* logits, int64_t vocab, int64_t* token, int32_t* state, int32_t* history,
                 int64_t history_len, void* workspace, int64_t workspace_bytes, bf16x_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* BF16X_LLAMA_H */
