/*
 * bf16x_hip.h -- C ABI of the MI355X (gfx950) BF16X engine (libbf16x_hip.so).
 *
 * The reference repository (dfytensor/bfloat16x) has no C ABI: its operator
 * API is a set of Python functions that launch Triton kernels on the current
 * torch stream.  Each entry point below replaces one of those functions (or a
 * step inside one); the replaced interface is cited as file:line of the
 * reference.  A Python/ctypes binding that mirrors the reference's call
 * surface lives in bfloat16x_amd/.
 *
 * Conventions
 *  - Plain pointers and sizes.  "dev" pointers are HIP device memory,
 *    "host" pointers are ordinary host memory.  No entry point allocates
 *    device memory; device outputs and workspaces are caller-owned.
 *  - Packed-dict streams (the layout of bf16x_quantize, opqk_linear.py:291-324):
 *      sign  int32 words, bit i = sign of flat element i (LSB-first)
 *      mant  int32 words, 7 bits per element, LSB-first global bit stream
 *      delta int32 words, 3 bits per element (code min(delta, 7))
 *      emax  uint8, one per 16 consecutive flat elements
 *    Stream lengths are given in words/bytes so the library can check them;
 *    streams padded with extra words (the reference's _pad1) are accepted.
 *  - Overflow plan: the sparse table entries whose true delta exceeds 7,
 *    grouped per tile (tile = one row, or one 65536-column segment of a row
 *    when in_f > 65536), for emax runs of 16 elements:
 *      tile_off uint32 [n_tiles + 1]  CSR offsets into tile_ent
 *      tile_ent uint32 [n_fix]        (column within tile << 16) | exact bf16 bits
 *      tile_sat uint8  [n_fix]        saturated exponent max(emax - 7, 0) of the
 *                                     entry's element (used by the GEMV overlay)
 *    Built by bf16x_plan_host() or bf16x_plan_from_csr().
 *  - All device work is enqueued on `stream` (a hipStream_t; NULL = the
 *    default stream) and is asynchronous.
 *  - Return value: 0 = success, < 0 = invalid argument (see BF16X_E*),
 *    > 0 = a hipError_t reported by the runtime.
 *  - Entry points keep no state between calls, and concurrent calls on
 *    different streams are safe when their output and workspace buffers
 *    differ, with one exception: bf16x_gguf_gemv_noalloc stages x in one
 *    fixed array per device, so its calls on one device must not overlap.
 *    Calls that share a workspace or counter buffer (bf16x_greedy's
 *    workspace, bf16x_layer_front_decode's sync buffers) must not overlap
 *    either.  bf16x_set_tuning changes kernel choices for the whole process.
 */
#ifndef BF16X_HIP_H
#define BF16X_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* bf16x_stream_t; /* hipStream_t */

enum {
  BF16X_OK = 0,
  BF16X_EARG = -1,         /* null pointer / bad enum / negative size        */
  BF16X_ESHAPE = -2,       /* unsupported or inconsistent shape              */
  BF16X_ESTREAM_LEN = -3,  /* a stream is shorter than the shape requires    */
  BF16X_ETABLE = -4,       /* malformed overflow table                        */
  BF16X_ECAPACITY = -5,    /* output capacity too small (count reported)      */
  BF16X_ESUB = -6,         /* sub != 16 is not supported by the GPU kernels   */
  BF16X_EDTYPE = -7        /* unsupported dtype code                          */
};

/* dtype codes for activations / outputs */
enum { BF16X_BF16 = 0, BF16X_F16 = 1, BF16X_F32 = 2 };

/* decode / GEMM weight semantics */
enum {
  BF16X_EXACT = 0,     /* lossless: table deltas applied (needs a plan)                   */
  BF16X_SATURATED = 1  /* code 7 -> exponent emax-7, no table (bf16x_gemm_fused.py:84-87) */
};

/* Library version string, e.g. "bf16x-hip 0.1.0 gfx950". */
const char* bf16x_version(void);
/* Human-readable text for a status code. */
const char* bf16x_status_string(int status);

/* Words of pack_bits_stream(n values, bits) -- opqk_linear.py:53-64: the
 * packer pads (-n*bits) % 32 *elements* before packing. */
int64_t bf16x_stream_words(int64_t n, int32_t bits);

/* ------------------------------------------------------------------------
 * Host encoder.  Replaces bf16x_quantize(w, sub) (opqk_linear.py:291-324),
 * byte-identical output.  w_bits: host bf16 bit patterns [out_f * in_f].
 * Outputs (host): sign/mant/delta of bf16x_stream_words(N, 1/7/3) words,
 * emax of ceil(N/sub) bytes, table of up to ovf_cap entries.  *n_ovf always
 * receives the table size; BF16X_ECAPACITY if it exceeds ovf_cap (streams
 * and emax are complete in that case).  n_threads <= 0: all host cores.
 * ------------------------------------------------------------------------ */
int bf16x_encode_host(const uint16_t* w_bits, int64_t out_f, int64_t in_f, int32_t sub,
                      int32_t* sign, int32_t* mant, int32_t* delta, uint8_t* emax,
                      int32_t* ovf_idx, uint8_t* ovf_val, int64_t ovf_cap, int64_t* n_ovf,
                      int32_t n_threads);

/* Device encoder: the same dict as bf16x_encode_host (byte-identical) from a
 * bf16 weight in device memory, sub = 16 (BF16X_ESUB otherwise).  Replaces
 * bf16x_quantize on a CUDA tensor (opqk_linear.py:291-324) and the chunked
 * GPU compressor (compress_bf16x_gpu.py:20-39): no temporaries beyond the
 * outputs and a workspace of bf16x_encode_workspace bytes (16-byte aligned).
 * The table count is written to *n_ovf (device int64); entries past ovf_cap
 * are not written, so a caller whose cap was short re-runs with a larger one.
 * Streams have at least bf16x_stream_words(N, b) words. */
int64_t bf16x_encode_workspace(int64_t out_f, int64_t in_f);
int bf16x_encode(const uint16_t* w_bits, int64_t out_f, int64_t in_f, int32_t sub,
                 int32_t* sign, int64_t n_sign, int32_t* mant, int64_t n_mant, int32_t* delta, int64_t n_delta,
                 uint8_t* emax, int64_t n_emax, int32_t* ovf_idx, uint8_t* ovf_val, int64_t ovf_cap,
                 int64_t* n_ovf, void* workspace, int64_t workspace_bytes, bf16x_stream_t stream);

/* ------------------------------------------------------------------------
 * Host plan builder.  Replaces the overflow preparation of Bf16xFused.__init__
 * (bf16x_fused.py:165-182: keep val > 7, per-row CSR) with tile offsets and
 * 4-byte entries carrying the exact bf16 bits.  Inputs are the host dict.
 * check: 0 = trust the table, 1 = also verify order/range/val >= 7 and that
 * each listed element carries code 7 (BF16X_ETABLE otherwise).
 * tile_off: host [out_f * tiles_per_row + 1]; tile_ent: host, capacity ent_cap.
 * *n_fix receives the entry count (BF16X_ECAPACITY if > ent_cap).
 * ------------------------------------------------------------------------ */
int64_t bf16x_plan_tiles(int64_t out_f, int64_t in_f);
int bf16x_plan_host(const int32_t* ovf_idx, const uint8_t* ovf_val, int64_t n_ovf,
                    const int32_t* sign, int64_t n_sign, const int32_t* mant, int64_t n_mant,
                    const int32_t* delta, int64_t n_delta, const uint8_t* emax, int64_t n_emax,
                    int64_t out_f, int64_t in_f, int32_t check,
                    uint32_t* tile_off, uint32_t* tile_ent, uint8_t* tile_sat, int64_t ent_cap,
                    int64_t* n_fix);

/* ------------------------------------------------------------------------
 * Device plan from the reference's per-row CSR (olk col int32, old true
 * delta int32, oloff int32 [out_f + 1]) -- the arguments of
 * bf16x_fused_gemv (bf16x_fused.py:114) built at bf16x_fused.py:165-179.
 * Writes tile_ent and tile_sat (dev, n_entries = oloff[out_f] each); tile_off
 * is oloff itself (requires in_f <= 65536).  All pointers dev.
 * ------------------------------------------------------------------------ */
int bf16x_plan_from_csr(const int32_t* olk, const int32_t* old, const int32_t* oloff,
                        const int32_t* sign, const int32_t* mant, const uint8_t* emax,
                        int64_t out_f, int64_t in_f, int64_t n_entries,
                        uint32_t* tile_ent, uint8_t* tile_sat, bf16x_stream_t stream);

/* ------------------------------------------------------------------------
 * One-pass decode.  Replaces bf16x_decode_triton (bf16x_triton_test.py:80-108)
 * = _bf16x_decode_kernel (:11-52) + _bf16x_fix_ovf_kernel (:55-77): the
 * table fix is applied in the same launch from the per-tile plan.
 * mode BF16X_EXACT needs tile_off/tile_ent; BF16X_SATURATED ignores them.
 * out: dev bf16 [out_f * in_f].  All pointers dev.
 * ------------------------------------------------------------------------ */
int bf16x_decode(const int32_t* sign, int64_t n_sign, const int32_t* mant, int64_t n_mant,
                 const int32_t* delta, int64_t n_delta, const uint8_t* emax, int64_t n_emax,
                 const uint32_t* tile_off, const uint32_t* tile_ent,
                 int64_t out_f, int64_t in_f, int32_t sub, int32_t mode,
                 uint16_t* out, bf16x_stream_t stream);

/* ------------------------------------------------------------------------
 * Fused decode + GEMV, batch 1.  Replaces bf16x_fused_gemv
 * (bf16x_fused.py:114-127) / _bf16x_gemv_fused_kernel (:32-111):
 * y[n] = sum_k W[n,k] * x[k], fp32 accumulation, y stored as bf16.
 * x: dev [in_f] of x_dtype.  mode EXACT applies the plan (tile_off,
 * tile_ent, tile_sat), SATURATED ignores it.  Requires in_f % 32 == 0.
 * All pointers dev.
 * ------------------------------------------------------------------------ */
int bf16x_gemv(const void* x, int32_t x_dtype,
               const int32_t* sign, int64_t n_sign, const int32_t* mant, int64_t n_mant,
               const int32_t* delta, int64_t n_delta, const uint8_t* emax, int64_t n_emax,
               const uint32_t* tile_off, const uint32_t* tile_ent, const uint8_t* tile_sat,
               int64_t out_f, int64_t in_f, int32_t sub, int32_t mode,
               uint16_t* y, bf16x_stream_t stream);

/* ------------------------------------------------------------------------
 * Step-major overflow plan for the GEMM (no reference counterpart: the
 * reference GEMM has no overflow correction, bf16x_gemm_fused.py:9-12).
 * Built on the device from the row plan (tile_off / tile_ent of
 * bf16x_plan_host or bf16x_plan_from_csr): entries regrouped by (64-column
 * step s, 16-row group h), run (s, h) = [kp_off[s*G2 + h], kp_off[s*G2 + h
 * + 1]).  kp_off: uint32 [bf16x_kplan_size(out_f, in_f)] = [S*G2 + 1] with
 * S = in_f/64, G2 = 2 ceil(out_f/32); kp_ent: uint32 [n_fix],
 * (row & 255) << 22 | (col & 63) << 16 | exact bf16 bits.
 * Requires in_f % 64 == 0 and in_f <= 65536.  All pointers dev.
 * ------------------------------------------------------------------------ */
int64_t bf16x_kplan_size(int64_t out_f, int64_t in_f);
int bf16x_kplan_build(const uint32_t* tile_off, const uint32_t* tile_ent, int64_t out_f, int64_t in_f,
                      uint32_t* kp_off, uint32_t* kp_ent, bf16x_stream_t stream);

/* ------------------------------------------------------------------------
 * Fused decode + GEMM (prefill / multi-token).  Replaces bf16x_fused_gemm
 * (bf16x_gemm_fused.py:97-114) / _bf16x_gemm_fused_kernel (:31-94):
 * y[M, out_f] = x[M, in_f] . W^T, fp32 accumulation (bf16 MFMA).
 * mode SATURATED reproduces the reference kernel (code 7 -> emax-7, no
 * table); EXACT applies the step-major plan (kp_off, kp_ent) for the
 * lossless weight.  x: dev bf16 [M, in_f], 16-byte aligned; y: dev
 * [M, out_f] of y_dtype (BF16X_BF16 or BF16X_F32).  Requires in_f % 64 == 0
 * and in_f <= 65536.  The call needs a workspace of
 * bf16x_gemm_workspace(M, out_f, in_f) bytes (0 = none; 16-byte aligned):
 * the fp32 partial products when K is split over workgroups for
 * parallelism; a smaller one returns BF16X_ECAPACITY.  All pointers dev.
 * ------------------------------------------------------------------------ */
int64_t bf16x_gemm_workspace(int64_t M, int64_t out_f, int64_t in_f);
int bf16x_gemm(const void* x, int32_t x_dtype, int64_t M,
               const int32_t* sign, int64_t n_sign, const int32_t* mant, int64_t n_mant,
               const int32_t* delta, int64_t n_delta, const uint8_t* emax, int64_t n_emax,
               const uint32_t* kp_off, const uint32_t* kp_ent,
               int64_t out_f, int64_t in_f, int32_t sub, int32_t mode,
               void* y, int32_t y_dtype, void* workspace, int64_t workspace_bytes,
               bf16x_stream_t stream);

/* ------------------------------------------------------------------------
 * Fused decode + GEMM for few activation rows, the same product as
 * bf16x_gemm at the reference's smallest block (bf16x_gemm_fused.py:97-114,
 * BM = 16): y[M, out_f] = x[M, in_f] . W^T, fp32 accumulation, for
 * 1 <= M <= 16 and in_f 2048 or 4096.  Each weight row is read once, in the
 * GEMV's pattern, with the ROW plan (tile_off, tile_ent of bf16x_plan_host /
 * bf16x_plan_from_csr) for EXACT; no workspace.  x: dev bf16 [M, in_f],
 * y: dev [M, out_f] of y_dtype (BF16X_BF16 or BF16X_F32), both 4-byte
 * aligned.  Other M or in_f return BF16X_ESHAPE.  All pointers dev.
 * ------------------------------------------------------------------------ */
int bf16x_gemm_rows(const void* x, int32_t x_dtype, int64_t M,
                    const int32_t* sign, int64_t n_sign, const int32_t* mant, int64_t n_mant,
                    const int32_t* delta, int64_t n_delta, const uint8_t* emax, int64_t n_emax,
                    const uint32_t* tile_off, const uint32_t* tile_ent,
                    int64_t out_f, int64_t in_f, int32_t sub, int32_t mode,
                    void* y, int32_t y_dtype, bf16x_stream_t stream);

/* ------------------------------------------------------------------------
 * Chunk plan for bf16x_gemm_chunks (no reference counterpart: the reference
 * GEMM has no overflow correction, bf16x_gemm_fused.py:9-12).  Built on the
 * device from the row plan (tile_off / tile_ent of bf16x_plan_host or
 * bf16x_plan_from_csr; a row's entries sorted by column, as every plan
 * builder here writes them): the entries regrouped by (256-column chunk p,
 * row r), so that those of rows [r0, r1) in chunk p are the one run
 * cp_ent[cp_off[p * out_f + r0] .. cp_off[p * out_f + r1]), each entry
 * (r & 255) << 24 | (column - 256 p) << 16 | exact bf16 bits.
 * cp_off: uint32 [bf16x_cplan_size(out_f, in_f)] = [out_f * in_f / 256 + 1];
 * cp_ent: uint32 [n_fix + 1] (the last word is never an entry).  Requires
 * in_f % 256 == 0 and in_f <= 65536 (bf16x_cplan_size returns BF16X_ESHAPE
 * otherwise).  All pointers dev.
 * ------------------------------------------------------------------------ */
int64_t bf16x_cplan_size(int64_t out_f, int64_t in_f);
int bf16x_cplan_build(const uint32_t* tile_off, const uint32_t* tile_ent, int64_t out_f, int64_t in_f,
                      uint32_t* cp_off, uint32_t* cp_ent, bf16x_stream_t stream);

/* ------------------------------------------------------------------------
 * Fused decode + GEMM for up to 64 activation rows, the product of
 * bf16x_gemm at the reference's small blocks (bf16x_gemm_fused.py:97-114,
 * BM = 16 .. 64): y[M, out_f] = x[M, in_f] . W^T, fp32 accumulation, for
 * 1 <= M <= 64, in_f % 256 == 0 and in_f <= 65536.  A workgroup per CU
 * streams its rows of W in column chunks (each stream read once), decodes a
 * chunk into LDS once and multiplies it by every token; no workspace.  EXACT
 * takes the chunk plan (cp_off, cp_ent of bf16x_cplan_build).  x: dev bf16
 * [M, in_f], 16-byte aligned; y: dev [M, out_f] of y_dtype (BF16X_BF16 or
 * BF16X_F32), 4-byte aligned.  Other shapes return BF16X_ESHAPE.  All
 * pointers dev.
 * ------------------------------------------------------------------------ */
int bf16x_gemm_chunks(const void* x, int32_t x_dtype, int64_t M,
                      const int32_t* sign, int64_t n_sign, const int32_t* mant, int64_t n_mant,
                      const int32_t* delta, int64_t n_delta, const uint8_t* emax, int64_t n_emax,
                      const uint32_t* cp_off, const uint32_t* cp_ent,
                      int64_t out_f, int64_t in_f, int32_t sub, int32_t mode,
                      void* y, int32_t y_dtype, bf16x_stream_t stream);

/* ========================================================================
 * GGUF half-block variant (bf16x_gguf_block.py, GGML_TYPE_BF16X): blocks of
 * 32 row-major weights, 46 bytes = [emax[2] | sign[4] | mant[28] |
 * delta[12]], emax floored at 7, code min(emax - e, 7), code 7 decodes to
 * exponent 0 (zero marker, :84).  A weight [out_f, in_f] (in_f % 32 == 0)
 * is out_f * in_f / 32 consecutive blocks.  Device block buffers must be
 * 4-byte aligned and readable up to the block bytes rounded up to a
 * multiple of 4 (n_bytes counts that length).
 * ======================================================================== */

/* fp32 -> bf16 bits with the reference's rounding (fp32_to_bf16_bits,
 * bf16x_gguf_block.py:44-49: NaN quieted, then round to nearest even).
 * Host pointers; n_threads <= 0 = hardware concurrency. */
int bf16x_fp32_to_bf16_host(const float* x, int64_t n, uint16_t* out, int32_t n_threads);

/* bf16 bits [n_blocks * 32] -> blocks [n_blocks * 46] (quantize_blocks,
 * bf16x_gguf_block.py:57-73, after its fp32 -> bf16 rounding).  Host. */
int bf16x_gguf_quantize_host(const uint16_t* bits, int64_t n_blocks, uint8_t* out, int32_t n_threads);

/* Device decode (dequantize_blocks, bf16x_gguf_block.py:76-87): blocks ->
 * out [out_f, in_f] of out_dtype BF16X_BF16 or BF16X_F32 (16-byte aligned). */
int bf16x_gguf_decode(const uint8_t* blocks, int64_t n_bytes, int64_t out_f, int64_t in_f,
                      void* out, int32_t out_dtype, bf16x_stream_t stream);

/* Device decode + GEMV, y[out_f] = W . x, x bf16 [in_f], y of y_dtype
 * (BF16X_BF16 / BF16X_F32), fp32 accumulation.  The reference keeps this
 * product in llama.cpp's GGML_TYPE_BF16X mat-vec kernels (README.md:121,
 * 138), outside the Python sources.  workspace: dev, 16-byte aligned,
 * bf16x_gguf_gemv_workspace(in_f) bytes (x rearranged in decode order). */
int64_t bf16x_gguf_gemv_workspace(int64_t in_f);
int bf16x_gguf_gemv(const void* x, int32_t x_dtype, const uint8_t* blocks, int64_t n_bytes,
                    int64_t out_f, int64_t in_f, void* y, int32_t y_dtype,
                    void* workspace, int64_t workspace_bytes, bf16x_stream_t stream);

/* bf16x_gguf_gemv without a workspace argument.  No counterpart in the
 * reference: for callers that cannot allocate device memory (code under
 * graph capture, tight serving loops, harnesses that forbid it).  The
 * workspace is a fixed 128 KB device array inside the library, one copy per
 * GPU held for the life of the process, so in_f is limited to 65536
 * (BF16X_ECAPACITY beyond it).  The stream must belong to the current
 * device.  Every call on a GPU uses that GPU's array: calls that overlap on
 * one GPU race.  Allocates nothing. */
int bf16x_gguf_gemv_noalloc(const void* x, int32_t x_dtype, const uint8_t* blocks, int64_t n_bytes,
                            int64_t out_f, int64_t in_f, void* y, int32_t y_dtype, bf16x_stream_t stream);

/* GGUF lossless side table (bf16x_gguf_block.py:96-193).  The table of a
 * weight [rows, cols] is the reference's blob without its 8-byte header:
 *   row_off uint32 [rows + 1]   entry index where each row starts
 *   entries uint32 [n_entries]  column | bf16 bits << 16 (the reference's
 *                               {u16 col, u16 bf16_bits}, little endian),
 *                               sorted by row then column
 * holding every element the half-block quantizer turns into the zero marker
 * although it is not +-0 (exponent delta >= 7, :121-128).
 * bf16x_gguf_ovf_pack_host -> pack_ovf (:131-148), host; row_off is always
 * filled and *n_entries set, BF16X_ECAPACITY if cap is too small.  cols <= 65536.
 * bf16x_gguf_ovf_check_host: validates a table against its blocks (offsets
 * monotone and consistent, columns strictly increasing and in range, and each
 * entry on a zero-marker element with the entry's sign and mantissa), the
 * condition under which the device consumers below are exact.  Host. */
int bf16x_gguf_ovf_pack_host(const uint16_t* bits, int64_t rows, int64_t cols, uint32_t* row_off,
                             uint32_t* entries, int64_t cap, int64_t* n_entries, int32_t n_threads);
int bf16x_gguf_ovf_check_host(const uint8_t* blocks, int64_t n_bytes, int64_t rows, int64_t cols,
                              const uint32_t* row_off, const uint32_t* entries, int64_t n_entries);

/* bf16x_gguf_decode with the table applied (dequantize_lossless,
 * bf16x_gguf_block.py:174-178): the original bf16 bits of every element.
 * Device; row_off / entries device pointers (entries: at least one word). */
int bf16x_gguf_decode_lossless(const uint8_t* blocks, int64_t n_bytes, int64_t out_f, int64_t in_f,
                               const uint32_t* row_off, const uint32_t* entries, int64_t n_entries,
                               void* out, int32_t out_dtype, bf16x_stream_t stream);

/* bf16x_gguf_gemv over the lossless weight: each row adds (exact - marker)
 * x[col] for its table entries (the sparse correction of the reference's
 * llama.cpp path, README.md:303-312).  The table must pass
 * bf16x_gguf_ovf_check_host against the same blocks.  Device. */
int bf16x_gguf_gemv_lossless(const void* x, int32_t x_dtype, const uint8_t* blocks, int64_t n_bytes,
                             int64_t out_f, int64_t in_f, const uint32_t* row_off, const uint32_t* entries,
                             int64_t n_entries, void* y, int32_t y_dtype, void* workspace,
                             int64_t workspace_bytes, bf16x_stream_t stream);

/* Fused decode + GEMM over GGUF blocks: y[M, out_f] = x[M, in_f] . W^T with
 * W decoded on the fly (dequantize_blocks, bf16x_gguf_block.py:76-87),
 * fp32 accumulation (bf16 MFMA).  No counterpart in the reference, which
 * stops at the decode; it replaces dequantize_blocks followed by a matmul.
 * kp_off / kp_ent: NULL for the near-lossless weight, or the step-major plan
 * of the lossless table (bf16x_gguf_kplan_build) for the exact weight.
 * x: dev bf16 [M, in_f], 16-byte aligned; y: dev [M, out_f] of y_dtype
 * (BF16X_BF16 or BF16X_F32).  Requires in_f % 64 == 0 (and in_f <= 65536
 * with a plan).  Workspace: bf16x_gguf_gemm_workspace(M, out_f, in_f) bytes,
 * 16-byte aligned (x in operand order, fp32 partials when K is split);
 * smaller returns BF16X_ECAPACITY.  Device. */
int64_t bf16x_gguf_gemm_workspace(int64_t M, int64_t out_f, int64_t in_f);
int bf16x_gguf_gemm(const void* x, int32_t x_dtype, int64_t M, const uint8_t* blocks, int64_t n_bytes,
                    const uint32_t* kp_off, const uint32_t* kp_ent, int64_t out_f, int64_t in_f, void* y,
                    int32_t y_dtype, void* workspace, int64_t workspace_bytes, bf16x_stream_t stream);

/* Step-major plan of a lossless GGUF table for bf16x_gguf_gemm: the table's
 * (row_off, entries) in place of bf16x_kplan_build's row plan, same output
 * (kp_off [bf16x_kplan_size(out_f, in_f)], kp_ent [n_entries, >= 1 word]).
 * Requires in_f % 64 == 0 and in_f <= 65536.  Device. */
int bf16x_gguf_kplan_build(const uint32_t* row_off, const uint32_t* entries, int64_t out_f, int64_t in_f,
                           uint32_t* kp_off, uint32_t* kp_ent, bf16x_stream_t stream);

/* ------------------------------------------------------------------------
 * Kernel-choice overrides: a test and tuning-sweep hook with no counterpart
 * in the reference.  Every entry point above chooses its kernel and launch
 * shape from its arguments alone; a key set here to a value >= 0 replaces
 * one of those choices for the whole process until it is set back to -1
 * (automatic, the initial state).  Process-wide and unsynchronised: change
 * it only while no other thread launches.  BF16X_EARG for an unknown key.
 * ------------------------------------------------------------------------ */
enum {
  BF16X_TUNE_GEMM_SKINNY2_MAX = 0, /* largest M of the 16x16x32 few-row GEMM (0..64)              */
  BF16X_TUNE_GEMM_SKINNY_MAX = 1,  /* largest M of the older few-row GEMM (0..128)                */
  BF16X_TUNE_GEMM_BM = 2,          /* tile height of the tiled GEMM (32, 64, 128 or 256)          */
  BF16X_TUNE_GEMM_SPLIT = 3,       /* K splits of the tiled GEMM                                  */
  BF16X_TUNE_GEMM_WS_MIN_ROWS = 4, /* smallest M of the wave-specialised GEMM                     */
  BF16X_TUNE_GEMM_WS_SPLIT = 5,    /* K splits of the wave-specialised GEMM                       */
  BF16X_TUNE_SKINNY_WAVES = 6,     /* waves per workgroup of the older few-row GEMM (1..4)        */
  BF16X_TUNE_SKINNY2_KQ = 7,       /* waves per row group of the 16x16x32 few-row GEMM (1, 2, 4)  */
  BF16X_TUNE_SKINNY2_SPLIT = 8,    /* K splits of the 16x16x32 few-row GEMM                       */
  BF16X_TUNE_GEMV_ITERS = 9,       /* row groups per workgroup of the GEMVs                       */
  BF16X_TUNE_GEMV_G = 10,          /* K parts of the split-K GEMV (1, 2 or 4)                     */
  BF16X_TUNE_GEMV_LONG = 11,       /* 0: rows of 4097-16384 columns on the split-K GEMV           */
  BF16X_TUNE_GEMV_XM_SLOTS = 12,   /* workgroup target of the normalising GEMVs                   */
  BF16X_TUNE_GGUF_LONG = 13,       /* 0: GGUF GEMV without the long-row kernel                    */
  BF16X_TUNE_GGUF_ITERS = 14,      /* rows per wave of the GGUF long-row GEMV                     */
  BF16X_TUNE_ATTN_SPLIT = 15,      /* 1: decode attention always on the split-key kernel          */
  BF16X_TUNE_GEMM_WS_GROUPED = 16, /* 0: the wave-specialised GEMM in one-step (64-column) tiles   */
  BF16X_TUNE_GEMM_WS_RESIDENT = 17,/* resident blocks the wave-specialised GEMM plans its rounds for */
  BF16X_TUNE_ATTN_MFMA = 18,       /* prefill attention: 0 the scalar kernel, 1 the MFMA kernel       */
  BF16X_TUNE_CHUNK_ATOMS = 19,     /* atoms per row and chunk of the chunked few-row GEMM (8, 16, 32) */
  BF16X_TUNE_COUNT = 20
};
int bf16x_set_tuning(int32_t key, int64_t value);
/* Current value of a key (-1 = automatic; also returned for an unknown key). */
int64_t bf16x_get_tuning(int32_t key);

#ifdef __cplusplus
}
#endif

#endif /* BF16X_HIP_H */
