/*
 * dk_amd.h — C ABI of the MI355X (gfx950) batch-1 decode kernel library libdk_amd.so.
 *
 * Drop-in boundary for the six ops that the reference's pybind module `decode_kernels` exports
 * (kernels/bindings.cpp:90-99) plus the INT4 format producer of runtime/quant.py. Every entry point:
 *   - takes raw device pointers, integer sizes and a HIP stream handle (hipStream_t passed as void*; NULL = default
 *     stream); no torch or C++ types cross the boundary;
 *   - validates its arguments on the host before any HIP call, mirroring the TORCH_CHECKs of kernels/bindings.cpp,
 *     and returns DK_OK (0) or a DK_ERR_* code; dk_last_error() then gives a thread-local message;
 *   - allocates nothing, keeps no state between calls and launches only on `stream`, so calls are capturable into a
 *     hipGraph (stream capture);
 *   - reads device-resident `pos` (int32[1]) where the reference does, so one captured graph serves every step.
 *
 * Layouts (all row-major, contiguous, fp16 = IEEE binary16):
 *   packed  int32 [N, K/8]     word j holds elements 8j..8j+7; element 8j+2i at bits [4i,4i+4), 8j+2i+1 at
 *                              [16+4i, 20+4i)   (runtime/quant.py:9-12)
 *   sz      fp16  [N, K/G, 2]  (scale, zero) per group, interleaved (runtime/quant.py:122-124)
 *   kc, vc  fp16  [pages, n_kv, P, D]; token t of the sequence lives in page bt[t / P], slot t % P
 *   o_part  fp32  [n_q, max_splits, D]; m_part, l_part fp32 [n_q, max_splits]
 */
#ifndef DK_AMD_H
#define DK_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum dk_status {
  DK_OK = 0,
  DK_ERR_NULL = 1,    /* a required pointer is NULL                                   */
  DK_ERR_ALIGN = 2,   /* a pointer that is read/written 16 bytes at a time is not 16 B aligned */
  DK_ERR_SHAPE = 3,   /* sizes inconsistent or out of the supported range               */
  DK_ERR_DOMAIN = 4,  /* a knob outside its domain (stage, R, version, group, page ...) */
  DK_ERR_LAUNCH = 5   /* the HIP launch itself failed (message carries hipGetErrorString) */
};

/* Message of the last failing call on this thread ("" if none). */
const char* dk_last_error(void);

/* hipRuntimeGetVersion() as seen by this library (lets a host check that it shares one HIP runtime). */
int dk_runtime_version(void);

/*
 * W4A16 GEMV  y[N] = dequant(W)[N,K] . x[K]   (fp16 in/out, fp32 accumulation)
 * Replaces gemv_w4a16 (kernels/bindings.cpp:27-38) -> gemv_w4a16_launch (kernels/gemv_w4a16.cu:248-267).
 * stage 0: one wave per row, per-element dequant fp16((q-z)*s) then fp32 FMA (the reference's exact-dequant ladder
 *          rung, kernels/gemv_w4a16.cu:16-36); `warps` = rows (waves) per workgroup (0 = 4).
 * stage 1, 2: every wave streams R whole rows (R in {1,2,4,8}; stage 1 forces R = 1), `warps` waves per workgroup
 *          (1..16, 0 = 4), pf in 0..3 = 2^pf column steps of 16-byte loads in flight per lane (capped at 16 / R);
 *          x is staged in LDS, so K <= 32768 (as the reference's gemv_rb<R,PF>, kernels/gemv_w4a16.cu:39-100).
 * stage 3: split-K: the workgroup's `warps` waves (1..16, 0 = one per 64 columns of 32 weights) share R rows,
 *          pf in {0,1} = one-step prefetch (for narrow N).
 * stage 4: row tiles: a row group of ceil(K / 2048) waves covers K once, one 32-weight column per lane with its
 *          x slice in registers, and walks 2^pf tiles (pf in 0..3) of R rows (R in {1,2,4,8}), the next tile's loads
 *          in flight while the current one is computed. `warps` = waves per workgroup: 0 (one row group) or a
 *          multiple of ceil(K / 2048) up to 16 (warps / ceil(K / 2048) row groups of consecutive row runs per
 *          workgroup); K <= 32768. The default when no tuning entry exists.
 * Requires K % 32 == 0, group a power of two >= 32 with K % group == 0, packed and x 16-byte aligned.
 */
int dk_gemv_w4a16(int stage, int R, int warps, int pf, const void* packed, const void* sz, const void* x, void* y,
                  int N, int K, int group, void* stream);

/*
 * W4A16 GEMV whose input is the residual + RMSNorm of the reference's add_rmsnorm, computed inside the GEMV
 * (no counterpart in the reference's binding: it fuses add_rmsnorm, kernels/bindings.cpp:64-72, with the gemv_w4a16
 * that runtime/model.py:189-196,219-228 calls right after it):
 *   xn = x + delta (fp16 add; delta may be NULL), or xn = the row *row of x when row != NULL (x is then an embedding
 *        table [*, K] and delta must be NULL: the decode step's embedding gather);
 *   y  = dequant(W) . (norm_w * fp16(float(xn) * rsqrt(mean(float(xn)^2) + eps)))
 *   x_out (if not NULL) receives xn; it must not alias x or delta (the residual stream is double-buffered).
 * Rounding points as dk_add_rmsnorm and dk_gemv_w4a16. stage must be 4; R, warps and pf as for stage 4; K <= 32768.
 */
int dk_gemv_w4a16_rmsnorm(int stage, int R, int warps, int pf, const void* packed, const void* sz, const void* x,
                          const int64_t* row, const void* delta, const void* norm_w, float eps, void* x_out, void* y,
                          int N, int K, int group, void* stream);

/*
 * The gate|up W4A16 GEMV with SwiGLU applied to its output: fuses gemv_w4a16 of the MLP's gate|up projection with
 * swiglu (kernels/bindings.cpp:27-38 then :74-79, as runtime/model.py:226-227 calls them; no single counterpart in
 * the reference's binding). The N = 2I weight rows are stored interleaved, row 2i = gate row i and row 2i + 1 = up
 * row i (a row permutation of the reference's [gate; up] stack, quantized per row exactly as before); writes
 * act[i] = fp16(silu(float(g_i))) * u_i for i < I, where g_i and u_i are the fp16 GEMV outputs of the two rows, so
 * the result equals gemv_w4a16 followed by swiglu bit for bit. Input: x as dk_gemv_w4a16 when norm_w is NULL (row,
 * delta and x_out must then be NULL), else the residual + RMSNorm input of dk_gemv_w4a16_rmsnorm. stage must be 4,
 * N even and R * 2^pf >= 2.
 */
int dk_gemv_w4a16_gate_up(int stage, int R, int warps, int pf, const void* packed, const void* sz, const void* x,
                          const int64_t* row, const void* delta, const void* norm_w, float eps, void* x_out, void* act,
                          int N, int K, int group, void* stream);

/*
 * The qkv W4A16 GEMV with RoPE + KV append applied to its output: fuses gemv_w4a16 of the attention's qkv
 * projection with rope_append (kernels/bindings.cpp:27-38 then the rope_append binding, as runtime/model.py:220-221
 * calls them; no single counterpart in the reference's binding). The N = (n_q + 2 n_kv) * head_dim weight rows are
 * stored per head as rotation pairs, row h*D + 2j = row h*D + j and row h*D + 2j + 1 = row h*D + j + D/2 of the
 * reference's layout (a row permutation, quantized per row exactly as before). Writes qkv in the reference's order
 * and the cache exactly as gemv_w4a16 followed by dk_rope_append would: q rotated in qkv, k and v as projected in
 * qkv, rotated k and v at the cache slot of *pos (none when *pos is outside [0, max_pos) or its page is unmapped).
 * Input: x as dk_gemv_w4a16 when norm_w is NULL (row, delta and x_out must then be NULL), else the residual +
 * RMSNorm input of dk_gemv_w4a16_rmsnorm. stage must be 4 and R * 2^pf >= 2.
 */
int dk_gemv_w4a16_qkv_rope(int stage, int R, int warps, int pf, const void* packed, const void* sz, const void* x,
                           const int64_t* row, const void* delta, const void* norm_w, float eps, void* x_out,
                           void* qkv, const float* cos_t, const float* sin_t, const int32_t* pos, const int32_t* bt,
                           void* kc, void* vc, int n_q, int n_kv, int head_dim, int page, int max_pos, int n_pages,
                           int n_bt, int K, int group, void* stream);

/*
 * y = dequant(W) . x where x is the attention output merged from dk_paged_attention_split's partials inside this
 * launch: the combine of paged_attention (kernels/paged_attention.cu:368-427, the log-sum-exp merge of the live
 * splits of each head, x rounded to fp16 as the combine rounds its output) followed by gemv_w4a16 of the o
 * projection (runtime/model.py:220-222), one launch instead of two. Every workgroup merges all of x (one thread per
 * 8 values) into LDS while its weight loads are in flight. With at most one live split (or none, max_pos > 0 and
 * *pos outside [0, max_pos): the RoPE split kernel's skip) x is read from attn, the output the split kernel wrote.
 * o_part [n_q, max_splits, head_dim], m_part / l_part [n_q, max_splits] fp32; attn [n_q * head_dim] fp16;
 * ctx = min(*pos + 1, n_bt * page), live splits = min(ceil(ctx / part_size), max_splits). K = n_q * head_dim,
 * head_dim 64 or 128, max_splits 1..16; stage 4, R and pf as for stage 4, warps = waves per workgroup with
 * 64 warps >= K / 8 and warps <= 8 (a multiple of ceil(K / 2048)); o_part and attn 16-byte aligned. No single
 * counterpart in the reference.
 */
int dk_gemv_w4a16_attn(int stage, int R, int warps, int pf, const void* packed, const void* sz, const float* o_part,
                       const float* m_part, const float* l_part, const void* attn, const int32_t* pos, int n_bt,
                       int page, int part_size, int max_splits, int max_pos, int n_q, int head_dim, void* y, int N,
                       int K, int group, void* stream);

/*
 * fp16-weight GEMV y[N] = W[N, K] . x[K] (W row-major fp16, fp32 accumulation, fp16 out). Replaces the fp16 LM head's
 * torch.mm(x, W^T) (runtime/model.py:187 of the reference; cuBLAS there, no custom kernel). R rows per tile (1, 2, 4),
 * warps waves per workgroup (0 = 4; 1, 2, 4, 8), 2^pf tiles per wave (pf 0..3). K % 8 == 0, K <= 4096 and
 * R * ceil(K / 512) rounded up to a power of two <= 16. w and x 16-byte aligned.
 */
int dk_gemv_f16(int R, int warps, int pf, const void* w, const void* x, void* y, int N, int K, void* stream);

/*
 * dk_gemv_f16 whose input is the residual + RMSNorm of dk_add_rmsnorm: x_out (optional, must not alias x or delta)
 * receives x + delta (fp16 add; delta may be NULL) and y = W . (norm_w * fp16(float(x + delta) * r)),
 * r = 1 / sqrt(sum / K + eps). Fuses the decode step's final add_rmsnorm with the fp16 LM head
 * (kernels/bindings.cpp:64-72 then runtime/model.py:187; no counterpart in the reference's binding).
 */
int dk_gemv_f16_rmsnorm(int R, int warps, int pf, const void* w, const void* x, const void* delta, const void* norm_w,
                        float eps, void* x_out, void* y, int N, int K, void* stream);

/*
 * rope_append for a batch of M tokens (prefill): row m of qkv [M, (n_q + 2 n_kv) head_dim] is token *pos + m; each
 * row is rotated and appended exactly as dk_rope_append does for one token (kernels/bindings.cpp:81-88 per row).
 * No counterpart in the reference, which appends prompt tokens one decode step at a time.
 */
int dk_rope_append_rows(void* qkv, const float* cos_t, const float* sin_t, const int32_t* pos, const int32_t* bt,
                        void* kc, void* vc, int M, int n_q, int n_kv, int head_dim, int page, int max_pos,
                        int n_pages, int n_bt, void* stream);

/*
 * Residual + RMSNorm of M rows (prefill), each with dk_add_rmsnorm's rounding points: xn = x_in[src] + delta[r]
 * (delta may be NULL; src = rows[r] when rows != NULL, e.g. the embedding rows of the prompt's tokens, else r),
 * x_out[r] = xn, out[r] = w * fp16(float(xn) * rsqrt-term). x_in has n_src rows (M when rows is NULL); a gathered
 * index outside [0, n_src) is not read: that row's x_out and out are NaN. x_out may equal x_in when rows is NULL; out
 * aliases nothing; H as for dk_add_rmsnorm. No counterpart in the reference (its add_rmsnorm is one vector,
 * kernels/bindings.cpp:64-72).
 */
int dk_rmsnorm_rows(const void* x_in, const int64_t* rows, int n_src, const void* delta, const void* w, void* x_out,
                    void* out, int M, int H, float eps, void* stream);

/*
 * dk_rmsnorm_rows without a gather, its delta given as the fp32 split partials dk_gemm_w4a16_ws leaves with epilogue
 * 2: delta[r] = fp16(sum over s < splits of parts[s * part_stride + r * H + n]), summed in split order as the GEMM's
 * own reduce launch sums them, so x_out and out are bit for bit those of dk_gemm_w4a16_ws (epilogue 0) followed by
 * dk_rmsnorm_rows; the reduce launch is folded into this one. part_stride (floats) a multiple of 4, >= H when
 * splits > 1 (the partials of rows [0, M) of one split are contiguous: M * H for a whole output, larger for a slice
 * of its rows); splits 1..64; parts 16-byte aligned and overlapping neither x_out nor out; x_out may be x_in. No
 * counterpart in the reference.
 */
int dk_rmsnorm_rows_parts(const void* x_in, const float* parts, int splits, long long part_stride, const void* w,
                          void* x_out, void* out, int M, int H, float eps, void* stream);

/*
 * Causal paged attention of M prompt rows (prefill): row m (position *pos + m) attends tokens [0, *pos + m] of the
 * cache, which must already hold them (dk_rope_append_rows); q is the first n_q heads of qkv row m, already rotated.
 * out [M, n_q * head_dim] fp16. Tokens at positions >= max_ctx (and past the block table) are neither read nor
 * attended; pass *pos + M to attend the whole prefix. fp32 scores and softmax, as dk_paged_attention. No counterpart
 * in the reference (it teacher-forces prompts through the decode step).
 */
int dk_attention_prefill(const void* qkv, const int32_t* pos, const int32_t* bt, int n_bt, const void* kc,
                         const void* vc, int n_pages, int page, int n_q, int n_kv, int head_dim, int M, int max_ctx,
                         void* out, void* stream);

/*
 * W4A16 GEMM for prefill: Y[M, N] = X[M, K] . dequant(W)[N, K]^T, X and Y fp16 row-major, W in the GEMV's packed
 * format; fp32 accumulation over exact products of X and the reference's dequantized fp16 weight. epilogue 0 writes
 * Y [M, N]; epilogue 1 treats columns (2i, 2i + 1) as an interleaved (gate, up) pair and writes act [M, N/2] =
 * fp16(silu(float(gate))) * up. No counterpart in the reference, which teacher-forces prompts through the decode step
 * (the prefill row of the scope). K % 32 == 0, group a power of two >= 32.
 */
int dk_gemm_w4a16(const void* packed, const void* sz, const void* x, void* y, int M, int N, int K, int group,
                  int epilogue, void* stream);

/*
 * dk_gemm_w4a16 with a caller-provided workspace for split-K: shapes whose weight rows are too few to fill the CUs
 * (e.g. 4096 x 14336 or 4096 x 4096 at M 512) split K over S workgroups per tile, write fp32 partials [S, M, N] to
 * the workspace and sum them in a second launch, in split order (the result does not depend on scheduling; its fp32
 * summation order differs from the unsplit kernel's). dk_gemm_w4a16_workspace_bytes returns the bytes a shape needs
 * (0: it does not split; epilogue 1 never splits). workspace NULL runs dk_gemm_w4a16; otherwise it must hold that
 * many bytes, be 16-byte aligned and overlap neither x nor y. epilogue 2 (shapes that split only; y unused, may be
 * NULL): the partials alone, left in the workspace for a reader that sums them (dk_rmsnorm_rows_parts), which saves
 * the second launch. Like dk_gemm_w4a16, no counterpart in the reference.
 */
size_t dk_gemm_w4a16_workspace_bytes(int M, int N, int K, int group, int epilogue);
int dk_gemm_w4a16_ws(const void* packed, const void* sz, const void* x, void* y, int M, int N, int K, int group,
                     int epilogue, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Read-bandwidth probe: `blocks` workgroups of `threads` threads read the first floor(bytes / 16) 16-byte words of buf
 * once, workgroup b the b-th of `blocks` contiguous slabs of n / blocks or n / blocks + 1 of the n words, in rounds of
 * unroll x threads words (every lane's `unroll` loads of a round in flight together). With
 * sink_words >= blocks * threads / 64 (one slot per wave) wave w of workgroup b stores the sum of the 32-bit words it
 * read (mod 2^32) to sink[b * threads / 64 + w], so the slots add up to the sum of every 32-bit word read (a check that
 * the whole buffer was streamed); with a smaller sink (the reference's callers pass one word) nothing is written.
 * Replaces bw_read (kernels/bindings.cpp:40-43, the reference's read microbenchmark, kernels/gemv_w4a16.cu:133-153):
 * same knobs (grid, workgroup size, loads in flight per lane), own kernel. unroll in {1, 2, 4, 8, 16}; threads a
 * multiple of 64 in [64, 1024]; blocks in [1, 2^22]; bytes >= 16; buf 16-byte and sink 4-byte aligned.
 */
int dk_bw_read(const void* buf, size_t bytes, uint32_t* sink, int sink_words, int blocks, int threads, int unroll,
               void* stream);

/*
 * Paged split-K GQA decode attention for one query token at ctx = *pos + 1 (device int32). The version selects the
 * split kernel: 1-3 (the reference's three kernel versions) the fastest this build has for the arguments, the lean
 * MFMA kernel (see dk_attention_decode's impl 3) whenever it takes the part size and page, else the block kernel;
 * 4 the block kernel; 5 the lean kernel (rejected where it does not fit).
 * Replaces paged_attention (kernels/bindings.cpp:45-62) -> paged_attention_launch (kernels/paged_attention.cu:429-461).
 * Grid = n_kv x max_splits workgroups; split s covers tokens [s*part_size, (s+1)*part_size) of the live context;
 * splits past ceil(ctx/part_size) exit; with one live split the output is written directly, otherwise each split
 * writes unnormalized o and its (m, l) and a combine kernel merges them with the log-sum-exp rule.
 * head_dim in {64, 128}; n_q / n_kv in {1, 2, 4, 8}; page a power of two; version in 1..5. Context is clamped to n_bt * page (tokens without a
 * block-table entry do not exist); a block-table entry outside [0, n_pages) masks its tokens; tokens past
 * max_splits * part_size are not attended (as in the reference). softmax scale 1/sqrt(head_dim). q, kc, vc and
 * o_part 16-byte aligned.
 */
int dk_paged_attention(int version, const void* q, const void* kc, const void* vc, const int32_t* bt,
                       const int32_t* pos, int n_q, int n_kv, int head_dim, int page, int n_pages, int n_bt,
                       int part_size, int max_splits, float* o_part, float* m_part, float* l_part, void* out,
                       void* stream);

/*
 * The first of dk_paged_attention's two kernels alone: the split kernel (same arguments, checks and split rules),
 * without the combine. With one live split it writes out itself; otherwise out is left as it was and the partials
 * are for a consumer that merges them, dk_gemv_w4a16_attn. It has no single counterpart in the reference: it is the
 * paged_attn_partial launch of paged_attention_launch (kernels/paged_attention.cu:429-461), the reference's combine
 * (:368-427) moving into the o projection that follows in the decode step (runtime/model.py:220-222).
 */
int dk_paged_attention_split(int version, const void* q, const void* kc, const void* vc, const int32_t* bt,
                             const int32_t* pos, int n_q, int n_kv, int head_dim, int page, int n_pages, int n_bt,
                             int part_size, int max_splits, float* o_part, float* m_part, float* l_part, void* out,
                             void* stream);

/*
 * dk_paged_attention without caller-provided split buffers, for callers that cannot allocate device memory (code
 * under hipGraph capture that must not call hipMalloc, tight serving loops, harnesses that forbid allocation). It
 * has no counterpart in the reference. The split partials live in a library-owned device array of
 * DK_NOALLOC_SCRATCH_BYTES bytes, one per GPU, held until the process ends; the call allocates nothing. Every call
 * on a GPU shares that GPU's array: calls that overlap on one GPU (two streams, two threads) race, so serialize them.
 * Nothing in the array has to start at zero (every partial the combine reads is written by the same call). Must be
 * called with the stream's device current (its first call on a device resolves the array's address there).
 * Arguments, limits and results as dk_paged_attention; additionally the partials of n_q x max_splits x head_dim must
 * fit: dk_paged_attention_noalloc_bytes(n_q, head_dim, max_splits) <= DK_NOALLOC_SCRATCH_BYTES, else DK_ERR_SHAPE.
 */
#define DK_NOALLOC_SCRATCH_BYTES (4u << 20)
int dk_paged_attention_noalloc(int version, const void* q, const void* kc, const void* vc, const int32_t* bt,
                               const int32_t* pos, int n_q, int n_kv, int head_dim, int page, int n_pages, int n_bt,
                               int part_size, int max_splits, void* out, void* stream);

/* Bytes of scratch dk_paged_attention_noalloc needs for these sizes (0 for non-positive sizes). */
size_t dk_paged_attention_noalloc_bytes(int n_q, int head_dim, int max_splits);

/*
 * Fused decode attention: rope_append followed by paged_attention with one fewer launch, for callers that own the
 * whole decode step (no counterpart in the reference's binding: it fuses rope_append, kernels/bindings.cpp:81-88,
 * and the split kernel of paged_attention, kernels/bindings.cpp:45-62, as runtime/model.py:205-213 calls them back to
 * back). qkv: the fused [q | k | v] vector, fp16 [(n_q + 2 n_kv) * head_dim], read only (q is rotated in registers,
 * not written back). k (rotated) and v of position *pos are written into page bt[pos / page], slot pos % page exactly
 * as dk_rope_append writes them, and the attention over ctx = *pos + 1 tokens uses them. Split partials go to
 * o_part / m_part / l_part and a combine kernel merges them, as for dk_paged_attention. impl selects the split
 * kernel: 0 or 1 = the block kernel (v_dot2 scores, LDS p.V), 3 = the lean MFMA kernel (16 x 16 f16 tiles, scalar
 * page lookups, one memory round trip for K / V; needs page >= 16 and a part_size that is a multiple of 16 up to 512,
 * 256 at head_dim 128).
 * The runtime picks impl and part_size per context from its measured policy table. If *pos is outside [0, max_pos)
 * nothing is touched. Other arguments and limits as dk_rope_append / dk_paged_attention.
 */
int dk_attention_decode(const void* qkv, const float* cos_t, const float* sin_t, int max_pos, const int32_t* pos,
                        const int32_t* bt, int n_bt, void* kc, void* vc, int n_pages, int page, int n_q, int n_kv,
                        int head_dim, int part_size, int max_splits, int impl, float* o_part, float* m_part,
                        float* l_part, void* out, void* stream);

/*
 * Fused residual add + RMSNorm:  x <- x + delta (fp16 add, written back; skipped if delta == NULL);
 * out = w * fp16(float(x) * rsqrt(mean(float(x)^2) + eps)).
 * Replaces add_rmsnorm (kernels/bindings.cpp:64-72) -> add_rmsnorm_launch (kernels/fused_norm.cu:56-58).
 * H % 8 == 0, H >= 8. Up to H = 65536 the row is held in registers (8 chunks of 8 for each of 1024 threads); a longer
 * row is normalised in two passes over memory, and then x, delta and out must not alias. x, delta, w, out 16-byte
 * aligned.
 */
int dk_add_rmsnorm(void* x, const void* delta, const void* w, void* out, int H, float eps, void* stream);

/*
 * Fused SwiGLU: out[i] = fp16(silu(float(gu[i]))) * gu[I + i] (fp16 product).
 * Replaces swiglu (kernels/bindings.cpp:74-79) -> swiglu_launch (kernels/fused_swiglu.cu:23-26).
 * I % 8 == 0; gu, out 16-byte aligned.
 */
int dk_swiglu(const void* gu, void* out, int I, void* stream);

/*
 * RoPE (rotate_half pairs (i, i + D/2), fp32 tables [max_pos, D/2]) on q and k of the fused qkv vector at position
 * *pos (device int32); q rotated in place, k rotated and v copied into page bt[pos / page], slot pos % page.
 * Replaces rope_append (kernels/bindings.cpp:81-88) -> rope_append_launch (kernels/rope_kv.cu:34-38).
 * head_dim in {64, 128}; page a power of two. If *pos >= max_pos nothing is touched; if pos / page >= n_bt or the
 * block-table entry is outside [0, n_pages) q is still rotated but nothing is written to the caches.
 */
int dk_rope_append(void* qkv, const float* cos_t, const float* sin_t, const int32_t* pos, const int32_t* bt,
                   void* kc, void* vc, int n_q, int n_kv, int head_dim, int page, int max_pos, int n_pages,
                   int n_bt, void* stream);

/*
 * Greedy token pick closing a decode step: *tok = argmax(logits[0..V)) (int64; lowest index among equal maxima, NaN
 * ranks highest as in torch.argmax), then *pos += 1 if pos != NULL. Replaces the two torch ops
 * `torch.argmax(self.logits, out=self.tok)` and `self.pos += 1` of runtime/model.py:232-233 with one launch.
 */
int dk_argmax_advance(const void* logits, int V, int64_t* tok, int32_t* pos, void* stream);

/*
 * The same pick and advance spread over ceil(V / 4096) workgroups (one launch), for large vocabularies: the
 * workgroups meet through `work`, two uint64 words of device memory that must be zero before the first call and that
 * every call leaves zero again (calls that overlap on one work buffer race). Same result as dk_argmax_advance,
 * including ties and NaN. No reference counterpart (runtime/model.py:232-233 is torch.argmax + pos += 1).
 */
int dk_argmax_advance_split(const void* logits, int V, int64_t* tok, int32_t* pos, uint64_t* work, void* stream);

/*
 * INT4 format producer on the GPU: round-to-nearest asymmetric group quantization of fp16 W [N, K] and packing,
 * bit-identical to runtime/quant.py quantize (:42-48, RTN branch of group_params :20-28) + pack (:100-109) +
 * pack_scale_zero (:122-124). Writes packed int32 [N, K/8] and sz fp16 [N, K/G, 2].
 * clip = 1: quantize(clip=True), the per-group range clipping of group_params (:17-38): the group's [min, max] is
 * shrunk by the factor of (1.0, 0.95, ..., 0.7) with the smallest squared rounding error (summed in fp64; the
 * reference sums in fp32, so only near-ties of two factors can resolve differently). clip = 0: RTN.
 * group a power of two in [32, 512] with K % group == 0.
 */
int dk_quantize_w4(const void* w, void* packed, void* sz, int N, int K, int group, int clip, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* DK_AMD_H */
