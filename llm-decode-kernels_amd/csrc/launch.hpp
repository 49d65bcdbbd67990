// Internal launchers (host side). Arguments are validated by the C ABI layer (dk_api.hip) before these run.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "dk_amd.h"

namespace dk {

// W4A16 GEMV. stage 0: exact per-element dequant, `waves` rows per workgroup. stage 1/2: each wave streams R whole
// rows, `waves` waves per workgroup, 2^pf column steps in flight, x staged in LDS (K <= kGemvRowsMaxK). stage 3: the
// workgroup's `waves` waves split K for R rows, pf = one-step prefetch. stage 4: row groups of ceil(K / 2048) waves
// walk 2^pf tiles of R rows; `waves` = waves per workgroup (0 = one row group).
constexpr int kGemvRowsMaxK = 32768;  // x in LDS: K * 2 bytes <= 64 KB per workgroup
void launch_gemv_w4a16(int stage, int R, int waves, int pf, const void* packed, const void* sz, const void* x,
                       void* y, int N, int K, int log2G, hipStream_t st);
// x operand of the fused row-tile GEMVs (prologue 0 = plain x, 1 = residual + RMSNorm; see gemv_w4a16.hip).
// The RoPE + KV-append epilogue of the qkv GEMV: the arguments of the reference's rope_append op
// (kernels/bindings.cpp rope_append) with the head count split into q and kv heads.
struct GemvRope {
  const float* cos_t;     // [max_pos, D / 2]
  const float* sin_t;
  const int32_t* pos;     // device position of the token
  const int32_t* bt;      // block table [n_bt]
  void* kc;               // [n_pages, n_kv, 2^log2P, D]
  void* vc;
  int n_q, n_kv, log2D, log2P, max_pos, n_pages, n_bt;
};
// The attention-combine prologue of the o projection: the split kernel's partials, merged into x by every workgroup
// (the arguments of the reference's combine, kernels/paged_attention.cu:368-427, plus the attention output the split
// kernel writes itself when a single split is live).
struct GemvCombine {
  const float* o_part;    // [n_q, max_splits, D] unnormalised split outputs
  const float* m_part;    // [n_q, max_splits] split maxima
  const float* l_part;    // [n_q, max_splits] split sums
  const void* attn;       // [n_q * D] fp16: the output when at most one split is live
  const int32_t* pos;     // device position: ctx = min(pos + 1, cap)
  int cap;                // n_bt << log2(page)
  int part_size, max_splits;
  int max_pos;            // > 0: the RoPE split kernel's range check (pos outside [0, max_pos): nothing was written)
  int log2D;
};
struct GemvInput {
  const void* x;          // plain: the input vector; rmsnorm: the residual stream (or the embedding table)
  const int64_t* row;     // rmsnorm: device row index into x (embedding gather) or null
  const void* delta;      // rmsnorm: residual delta or null
  const void* norm_w;     // rmsnorm: weight
  float eps;
  void* x_out;            // rmsnorm: receives x + delta (written by workgroup 0) or null
  GemvRope rope;          // epilogue 2 only
  GemvCombine comb;       // prologue 2 only
};
// epilogue 0 = one fp16 output per row, 1 = SwiGLU of interleaved gate / up row pairs (N / 2 outputs), 2 = RoPE +
// KV append of rotation-pair rows (qkv rows stored per head as j, j + D/2 for j < D/2; N outputs in head order).
// prologue 2 = the attention combine (GemvCombine; epilogue 0 only): the workgroup needs one thread per 8 values of
// x (64 warps >= K / 8, warps <= kGemvCombineMaxWarps) and max_splits <= kGemvCombineMaxSplits.
constexpr int kGemvCombineMaxSplits = 16;
constexpr int kGemvCombineMaxWarps = 8;
void launch_gemv_w4a16_fused(int prologue, int epilogue, int R, int warps, int pf, const void* packed, const void* sz,
                             const GemvInput& in, void* y, int N, int K, int log2G, hipStream_t st);
// Default configuration for a shape: (stage, R, waves, pf).
void gemv_default_config(int N, int K, int* stage, int* R, int* waves, int* pf);

// fp16-weight GEMV (the fp16 LM head): each wave owns R-row tiles of whole rows, 2^pf tiles per wave, `waves` waves
// per workgroup (0 = 4); prologue 0 = plain x, 1 = residual + RMSNorm (GemvInput without row). K <= kGemvF16MaxK and
// R * ceil(K / 512) <= kGemvF16MaxLoads (16-byte loads per lane per tile).
constexpr int kGemvF16MaxK = 4096;
constexpr int kGemvF16MaxLoads = 16;
void launch_gemv_f16(int prologue, int R, int waves, int pf, const void* w, const GemvInput& in, void* y, int N,
                     int K, hipStream_t st);

// W4A16 GEMM (prefill): Y[M, N] = X[M, K] . dequant(W)^T; epilogue 1 = SwiGLU of interleaved gate/up column pairs
// (Y [M, N/2]). K % 32 == 0, group >= 32.
void launch_gemm_w4a16(const void* packed, const void* sz, const void* x, void* y, int M, int N, int K, int log2G,
                       int epilogue, void* ws, hipStream_t st);
// bytes of fp32 split-K partials launch_gemm_w4a16 uses for this shape when given a workspace (0: it does not split)
size_t gemm_w4a16_workspace_bytes(int M, int N, int K, int log2G, int epilogue);

// Read-ceiling probe (read_probe.hip): `blocks` workgroups of `threads` threads, workgroup b streaming the b-th of
// `blocks` equal contiguous slabs in rounds of depth x threads 16-byte words; with sink_words >= blocks x W (W =
// threads / 64) sink[b W + w] receives the sum of the 32-bit words wave w of workgroup b read, else nothing is written.
// depth in {1,2,4,8,16}.
void launch_read_probe(const void* buf, size_t bytes, uint32_t* sink, uint32_t sink_words, int blocks, int threads,
                       int depth, hipStream_t st);

// Paged attention arguments. q: the query heads [n_q * D] (reference op) or the fused qkv vector (decode op).
struct AttnLaunch {
  const void* q;
  const float* cos_t;  // RoPE tables [max_pos, D/2] (decode op only)
  const float* sin_t;
  int max_pos;
  const int32_t* pos;
  const int32_t* bt;
  int n_bt;
  void* kc;
  void* vc;
  int n_pages;
  int log2P;
  int n_q, n_kv, head_dim, part_size, max_splits;
  float* o_part;
  float* m_part;
  float* l_part;
  void* out;
  int impl;            // 0 or 1 = block kernel; 3 = lean MFMA kernel
  bool split_only;     // the split kernel alone: the consumer merges the partials (gemv prologue 2)
};
// The lean MFMA kernel: pages of at least 16 tokens, splits of whole 16-token tiles, at most 8 waves x 4 tiles (x 2
// tiles at head_dim 128, whose RoPE variant would not fit 4 tiles in registers).
inline int attn_lean_max_part(int head_dim) { return head_dim == 128 ? 256 : 512; }
inline bool attn_lean_fits(int part_size, int log2P, int head_dim) {
  return log2P >= 4 && part_size % 16 == 0 && part_size <= attn_lean_max_part(head_dim);
}
inline bool attn_use_lean(const AttnLaunch& a) {
  return a.impl == 3 && attn_lean_fits(a.part_size, a.log2P, a.head_dim);
}
// Reference-compatible op: split kernel + combine kernel.
void launch_paged_attention(const AttnLaunch& a, hipStream_t st);
// Fused decode op: RoPE + KV append + split-K attention, then the combine kernel.
void launch_attention_decode(const AttnLaunch& a, hipStream_t st);

// Causal attention of M prompt rows (prefill): row m at position *pos + m attends tokens [0, *pos + m] of the cache
// (tokens at max_ctx and beyond are neither read nor attended); q is the first n_q heads of qkv row m, already rotated.
void launch_attention_prefill(const void* qkv, const int32_t* pos, const int32_t* bt, int n_bt, const void* kc,
                              const void* vc, int n_pages, int log2P, int n_q, int n_kv, int head_dim, int M,
                              int max_ctx, void* out, hipStream_t st);

// Residual + RMSNorm with the row in registers: up to 8 16-byte chunks for each of 1024 threads.
constexpr int kRowNormMaxH = 8 * 8 * 1024;
void launch_add_rmsnorm(void* x, const void* delta, const void* w, void* out, int H, float eps, hipStream_t st);
void launch_swiglu(const void* gu, void* out, int I, hipStream_t st);
// rows > 1: a batch of tokens, row y of qkv [rows, (n_q + 2 n_kv) head_dim] at position *pos + y (prefill)
void launch_rope_append(void* qkv, const float* cos_t, const float* sin_t, const int32_t* pos, const int32_t* bt,
                        void* kc, void* vc, int n_q, int n_kv, int head_dim, int log2P, int max_pos, int n_pages,
                        int n_bt, int rows, hipStream_t st);
void launch_rmsnorm_rows(const void* x_in, const int64_t* rows, int n_src, const void* delta, const void* w, void* x_out,
                         void* out, int M, int H, float eps, hipStream_t st);
// the same with the delta given as split-K GEMM partials (fp32, split s of row r at parts + s * pstride + r * H)
void launch_rmsnorm_rows_parts(const void* x_in, const float* parts, int splits, long long pstride, const void* w,
                               void* x_out, void* out, int M, int H, float eps, hipStream_t st);

void launch_argmax_advance(const void* logits, int V, int64_t* tok, int32_t* pos, hipStream_t st);
void launch_argmax_split(const void* logits, int V, int64_t* tok, int32_t* pos, unsigned long long* work,
                         hipStream_t st);

void launch_quantize_w4(const void* w, void* packed, void* sz, int N, int K, int log2G, int clip, hipStream_t st);


}  // namespace dk
