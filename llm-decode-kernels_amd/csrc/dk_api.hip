// C ABI of libdk_amd.so (declared in include/dk_amd.h): host-side validation, then one launch on the caller's stream.
// The checks mirror the TORCH_CHECKs of the reference binding layer (kernels/bindings.cpp:18-88) so a bad argument
// is reported as an error code and a message instead of a fault inside a captured graph.
#include <stdarg.h>
#include <stdio.h>

#include <mutex>

#include "dk_amd.h"
#include "launch.hpp"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool aligned4(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 3u) == 0; }
bool pow2(long long v) { return v > 0 && (v & (v - 1)) == 0; }
bool ranges_overlap(const void* a, size_t na, const void* b, size_t nb) {
  const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
  return x < y + nb && y < x + na;
}
int ilog2(long long v) {
  int r = 0;
  while ((1LL << r) < v) ++r;
  return r;
}

// Clear a stale error before launching so that the check after the launch reports this launch only.
void clear_error() { (void)hipGetLastError(); }

int launched(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(DK_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  g_err[0] = '\0';
  return DK_OK;
}

}  // namespace

extern "C" {

const char* dk_last_error(void) { return g_err; }

int dk_runtime_version(void) {
  int v = 0;
  if (hipRuntimeGetVersion(&v) != hipSuccess) return -1;
  return v;
}

// Waves of one stage-4 row group: one 32-weight column per lane covers K.
static int tile_waves(int K) { return (K / 32 + 63) / 64; }

int dk_gemv_w4a16(int stage, int R, int warps, int pf, const void* packed, const void* sz, const void* x, void* y,
                  int N, int K, int group, void* stream) {
  if (!packed || !sz || !x || !y) return fail(DK_ERR_NULL, "gemv_w4a16: null pointer argument");
  if (stage < 0 || stage > 4) return fail(DK_ERR_DOMAIN, "gemv_w4a16: stage must be 0..4, got %d", stage);
  if (R != 1 && R != 2 && R != 4 && R != 8) return fail(DK_ERR_DOMAIN, "gemv: R must be 1,2,4,8, got %d", R);
  if (warps < 0 || warps > 16) return fail(DK_ERR_DOMAIN, "gemv_w4a16: warps must be 0..16, got %d", warps);
  if (stage == 3 ? (pf != 0 && pf != 1) : (pf < 0 || pf > 3))
    return fail(DK_ERR_DOMAIN, "gemv_w4a16: pf must be %s for stage %d, got %d", stage == 3 ? "0 or 1" : "0..3",
                stage, pf);
  if (stage == 4 && K > 0 && warps != 0 && warps % tile_waves(K) != 0)
    return fail(DK_ERR_SHAPE, "gemv_w4a16: stage 4 needs warps 0 or a multiple of ceil(K / 2048) = %d (whole row "
                "groups), got warps=%d K=%d", tile_waves(K), warps, K);
  if ((stage == 1 || stage == 2 || stage == 4) && K > dk::kGemvRowsMaxK)
    return fail(DK_ERR_SHAPE, "gemv_w4a16: stage %d stages x in LDS and needs K <= %d, got %d", stage,
                dk::kGemvRowsMaxK, K);
  if (N <= 0 || K <= 0) return fail(DK_ERR_SHAPE, "gemv_w4a16: N and K must be positive (N=%d K=%d)", N, K);
  if (K % 32 != 0 || K % group != 0)
    return fail(DK_ERR_SHAPE, "K must be a multiple of 32 and of the group size (K=%d group=%d)", K, group);
  if (group < 32) return fail(DK_ERR_DOMAIN, "group must be >= 32 (one uint4 never straddles a group), got %d", group);
  if (!pow2(group)) return fail(DK_ERR_DOMAIN, "group must be a power of two, got %d", group);
  if (!aligned16(packed)) return fail(DK_ERR_ALIGN, "packed must be 16B aligned");
  if (!aligned16(x)) return fail(DK_ERR_ALIGN, "x must be 16B aligned");
  if (!aligned4(sz)) return fail(DK_ERR_ALIGN, "sz must be 4B aligned");
  if (stage == 1) R = 1;
  clear_error();
  dk::launch_gemv_w4a16(stage, R, warps, pf, packed, sz, x, y, N, K, ilog2(group), (hipStream_t)stream);
  return launched("gemv_w4a16");
}

// Checks shared by the fused row-tile GEMVs (stage 4 only).
static int check_fused_gemv(const char* what, int stage, int R, int warps, int pf, const void* packed, const void* sz,
                            int N, int K, int group) {
  if (!packed || !sz) return fail(DK_ERR_NULL, "%s: null pointer argument", what);
  if (stage != 4) return fail(DK_ERR_DOMAIN, "%s: the fused variants exist for stage 4 only, got %d", what, stage);
  if (R != 1 && R != 2 && R != 4 && R != 8) return fail(DK_ERR_DOMAIN, "gemv: R must be 1,2,4,8, got %d", R);
  if (warps < 0 || warps > 16) return fail(DK_ERR_DOMAIN, "%s: warps must be 0..16, got %d", what, warps);
  if (pf < 0 || pf > 3) return fail(DK_ERR_DOMAIN, "%s: pf must be 0..3 for stage 4, got %d", what, pf);
  if (N <= 0 || K <= 0) return fail(DK_ERR_SHAPE, "%s: N and K must be positive (N=%d K=%d)", what, N, K);
  if (warps != 0 && warps % tile_waves(K) != 0)
    return fail(DK_ERR_SHAPE, "%s: warps must be 0 or a multiple of ceil(K / 2048) = %d (whole row groups), got %d",
                what, tile_waves(K), warps);
  if (K > dk::kGemvRowsMaxK) return fail(DK_ERR_SHAPE, "%s: K <= %d required, got %d", what, dk::kGemvRowsMaxK, K);
  if (K % 32 != 0 || K % group != 0)
    return fail(DK_ERR_SHAPE, "K must be a multiple of 32 and of the group size (K=%d group=%d)", K, group);
  if (group < 32) return fail(DK_ERR_DOMAIN, "group must be >= 32 (one uint4 never straddles a group), got %d", group);
  if (!pow2(group)) return fail(DK_ERR_DOMAIN, "group must be a power of two, got %d", group);
  if (!aligned16(packed)) return fail(DK_ERR_ALIGN, "packed must be 16B aligned");
  if (!aligned4(sz)) return fail(DK_ERR_ALIGN, "sz must be 4B aligned");
  return DK_OK;
}

int dk_gemv_w4a16_rmsnorm(int stage, int R, int warps, int pf, const void* packed, const void* sz, const void* x,
                          const int64_t* row, const void* delta, const void* norm_w, float eps, void* x_out, void* y,
                          int N, int K, int group, void* stream) {
  const int rc = check_fused_gemv("gemv_w4a16_rmsnorm", stage, R, warps, pf, packed, sz, N, K, group);
  if (rc != DK_OK) return rc;
  if (!x || !norm_w || !y) return fail(DK_ERR_NULL, "gemv_w4a16_rmsnorm: null pointer argument");
  if (!aligned16(x) || !aligned16(norm_w) || (delta && !aligned16(delta)) || (x_out && !aligned16(x_out)))
    return fail(DK_ERR_ALIGN, "x, delta, norm_w and x_out must be 16B aligned");
  if (row && (reinterpret_cast<uintptr_t>(row) & 7u)) return fail(DK_ERR_ALIGN, "row must be 8B aligned");
  if (x_out && (x_out == x || (delta && x_out == delta)))
    return fail(DK_ERR_DOMAIN, "gemv_w4a16_rmsnorm: x_out must not alias x or delta (other workgroups still read them)");
  clear_error();
  dk::GemvInput in{x, row, delta, norm_w, eps, x_out};
  dk::launch_gemv_w4a16_fused(1, 0, R, warps, pf, packed, sz, in, y, N, K, ilog2(group), (hipStream_t)stream);
  return launched("gemv_w4a16_rmsnorm");
}


int dk_gemv_w4a16_gate_up(int stage, int R, int warps, int pf, const void* packed, const void* sz, const void* x,
                          const int64_t* row, const void* delta, const void* norm_w, float eps, void* x_out, void* act,
                          int N, int K, int group, void* stream) {
  const int rc = check_fused_gemv("gemv_w4a16_gate_up", stage, R, warps, pf, packed, sz, N, K, group);
  if (rc != DK_OK) return rc;
  if (N % 2 != 0) return fail(DK_ERR_SHAPE, "gemv_w4a16_gate_up: N (interleaved gate/up rows) must be even, got %d", N);
  if ((R << pf) < 2)
    return fail(DK_ERR_DOMAIN, "gemv_w4a16_gate_up: the row tile R * 2^pf must hold a gate/up pair (>= 2), got R=%d "
                "pf=%d", R, pf);
  if (!x || !act) return fail(DK_ERR_NULL, "gemv_w4a16_gate_up: null pointer argument");
  if (!norm_w && (row || delta || x_out))
    return fail(DK_ERR_DOMAIN, "gemv_w4a16_gate_up: row, delta and x_out belong to the RMSNorm input (norm_w)");
  if (!aligned16(x) || (norm_w && !aligned16(norm_w)) || (delta && !aligned16(delta)) || (x_out && !aligned16(x_out)))
    return fail(DK_ERR_ALIGN, "x, delta, norm_w and x_out must be 16B aligned");
  if (row && (reinterpret_cast<uintptr_t>(row) & 7u)) return fail(DK_ERR_ALIGN, "row must be 8B aligned");
  if (x_out && (x_out == x || (delta && x_out == delta)))
    return fail(DK_ERR_DOMAIN, "gemv_w4a16_gate_up: x_out must not alias x or delta (other workgroups still read them)");
  if (act == x || (delta && act == delta))
    return fail(DK_ERR_DOMAIN, "gemv_w4a16_gate_up: act must not alias x or delta");
  clear_error();
  dk::GemvInput in{x, row, delta, norm_w, eps, x_out};
  dk::launch_gemv_w4a16_fused(norm_w ? 1 : 0, 1, R, warps, pf, packed, sz, in, act, N, K, ilog2(group),
                              (hipStream_t)stream);
  return launched("gemv_w4a16_gate_up");
}

int dk_gemv_w4a16_qkv_rope(int stage, int R, int warps, int pf, const void* packed, const void* sz, const void* x,
                           const int64_t* row, const void* delta, const void* norm_w, float eps, void* x_out,
                           void* qkv, const float* cos_t, const float* sin_t, const int32_t* pos, const int32_t* bt,
                           void* kc, void* vc, int n_q, int n_kv, int head_dim, int page, int max_pos, int n_pages,
                           int n_bt, int K, int group, void* stream) {
  if (head_dim != 64 && head_dim != 128)
    return fail(DK_ERR_SHAPE, "gemv_w4a16_qkv_rope: head_dim must be 64 or 128, got %d", head_dim);
  if (n_q <= 0 || n_kv <= 0 || n_q > 65535 || n_kv > 65535)
    return fail(DK_ERR_SHAPE, "gemv_w4a16_qkv_rope: bad head counts (n_q=%d n_kv=%d)", n_q, n_kv);
  const int N = (n_q + 2 * n_kv) * head_dim;
  const int rc = check_fused_gemv("gemv_w4a16_qkv_rope", stage, R, warps, pf, packed, sz, N, K, group);
  if (rc != DK_OK) return rc;
  if ((R << pf) < 2)
    return fail(DK_ERR_DOMAIN, "gemv_w4a16_qkv_rope: the row tile R * 2^pf must hold a rotation pair (>= 2), got R=%d "
                "pf=%d", R, pf);
  if (!x || !qkv || !cos_t || !sin_t || !pos || !bt || !kc || !vc)
    return fail(DK_ERR_NULL, "gemv_w4a16_qkv_rope: null pointer argument");
  if (!pow2(page)) return fail(DK_ERR_DOMAIN, "page size must be a power of two, got %d", page);
  if (max_pos < 1 || n_pages < 1 || n_bt < 1)
    return fail(DK_ERR_SHAPE, "gemv_w4a16_qkv_rope: empty rope table, cache or block table");
  if (!norm_w && (row || delta || x_out))
    return fail(DK_ERR_DOMAIN, "gemv_w4a16_qkv_rope: row, delta and x_out belong to the RMSNorm input (norm_w)");
  if (!aligned16(x) || (norm_w && !aligned16(norm_w)) || (delta && !aligned16(delta)) || (x_out && !aligned16(x_out)))
    return fail(DK_ERR_ALIGN, "x, delta, norm_w and x_out must be 16B aligned");
  if (row && (reinterpret_cast<uintptr_t>(row) & 7u)) return fail(DK_ERR_ALIGN, "row must be 8B aligned");
  if (x_out && (x_out == x || (delta && x_out == delta)))
    return fail(DK_ERR_DOMAIN, "gemv_w4a16_qkv_rope: x_out must not alias x or delta (other workgroups still read them)");
  if (qkv == x || (delta && qkv == delta))
    return fail(DK_ERR_DOMAIN, "gemv_w4a16_qkv_rope: qkv must not alias x or delta");
  clear_error();
  dk::GemvInput in{x, row, delta, norm_w, eps, x_out,
                   {cos_t, sin_t, pos, bt, kc, vc, n_q, n_kv, ilog2(head_dim), ilog2(page), max_pos, n_pages, n_bt}};
  dk::launch_gemv_w4a16_fused(norm_w ? 1 : 0, 2, R, warps, pf, packed, sz, in, qkv, N, K, ilog2(group),
                              (hipStream_t)stream);
  return launched("gemv_w4a16_qkv_rope");
}

// Checks shared by the fp16 GEMVs.
static int check_gemv_f16(const char* what, int R, int warps, int pf, const void* w, const void* x, const void* y,
                          int N, int K) {
  if (!w || !x || !y) return fail(DK_ERR_NULL, "%s: null pointer argument", what);
  if (R != 1 && R != 2 && R != 4) return fail(DK_ERR_DOMAIN, "%s: R must be 1, 2 or 4, got %d", what, R);
  if (warps != 0 && warps != 1 && warps != 2 && warps != 4 && warps != 8)
    return fail(DK_ERR_DOMAIN, "%s: warps must be 0 (default), 1, 2, 4 or 8, got %d", what, warps);
  if (pf < 0 || pf > 3) return fail(DK_ERR_DOMAIN, "%s: pf must be 0..3, got %d", what, pf);
  if (N <= 0 || K <= 0) return fail(DK_ERR_SHAPE, "%s: N and K must be positive (N=%d K=%d)", what, N, K);
  if (K % 8 != 0 || K > dk::kGemvF16MaxK)
    return fail(DK_ERR_SHAPE, "%s: K must be a multiple of 8 and <= %d, got %d", what, dk::kGemvF16MaxK, K);
  const int chunks = ((K >> 3) + 63) / 64;
  const int c_pow2 = chunks <= 1 ? 1 : chunks <= 2 ? 2 : chunks <= 4 ? 4 : 8;
  if (R * c_pow2 > dk::kGemvF16MaxLoads)
    return fail(DK_ERR_DOMAIN, "%s: R * %d chunks per lane exceeds %d loads per tile (K=%d: R <= %d)", what, c_pow2,
                dk::kGemvF16MaxLoads, K, dk::kGemvF16MaxLoads / c_pow2);
  if (!aligned16(w) || !aligned16(x)) return fail(DK_ERR_ALIGN, "%s: w and x must be 16B aligned", what);
  if (reinterpret_cast<uintptr_t>(y) & 1u) return fail(DK_ERR_ALIGN, "%s: y must be 2B aligned", what);
  return DK_OK;
}

int dk_gemv_f16(int R, int warps, int pf, const void* w, const void* x, void* y, int N, int K, void* stream) {
  const int rc = check_gemv_f16("gemv_f16", R, warps, pf, w, x, y, N, K);
  if (rc != DK_OK) return rc;
  clear_error();
  dk::GemvInput in{x, nullptr, nullptr, nullptr, 0.f, nullptr};
  dk::launch_gemv_f16(0, R, warps, pf, w, in, y, N, K, (hipStream_t)stream);
  return launched("gemv_f16");
}

int dk_gemv_f16_rmsnorm(int R, int warps, int pf, const void* w, const void* x, const void* delta, const void* norm_w,
                        float eps, void* x_out, void* y, int N, int K, void* stream) {
  const int rc = check_gemv_f16("gemv_f16_rmsnorm", R, warps, pf, w, x, y, N, K);
  if (rc != DK_OK) return rc;
  if (!norm_w) return fail(DK_ERR_NULL, "gemv_f16_rmsnorm: null pointer argument");
  if (!aligned16(norm_w) || (delta && !aligned16(delta)) || (x_out && !aligned16(x_out)))
    return fail(DK_ERR_ALIGN, "gemv_f16_rmsnorm: delta, norm_w and x_out must be 16B aligned");
  if (x_out && (x_out == x || (delta && x_out == delta)))
    return fail(DK_ERR_DOMAIN, "gemv_f16_rmsnorm: x_out must not alias x or delta (other waves still read them)");
  clear_error();
  dk::GemvInput in{x, nullptr, delta, norm_w, eps, x_out};
  dk::launch_gemv_f16(1, R, warps, pf, w, in, y, N, K, (hipStream_t)stream);
  return launched("gemv_f16_rmsnorm");
}

static int gemm_check(const void* packed, const void* sz, const void* x, void* y, int M, int N, int K, int group,
                      int epilogue) {
  if (!packed || !sz || !x || !y) return fail(DK_ERR_NULL, "gemm_w4a16: null pointer argument");
  if (M <= 0 || N <= 0 || K <= 0) return fail(DK_ERR_SHAPE, "gemm_w4a16: M, N and K must be positive");
  if (M > 65535 * 64) return fail(DK_ERR_SHAPE, "gemm_w4a16: M too large (%d)", M);
  if (K % 32 != 0 || K % group != 0)
    return fail(DK_ERR_SHAPE, "K must be a multiple of 32 and of the group size (K=%d group=%d)", K, group);
  if (group < 32 || !pow2(group))
    return fail(DK_ERR_DOMAIN, "group must be a power of two >= 32, got %d", group);
  if (epilogue != 0 && epilogue != 1)
    return fail(DK_ERR_DOMAIN, "gemm_w4a16: epilogue must be 0 (rows) or 1 (SwiGLU of gate/up pairs), got %d", epilogue);
  if (epilogue == 1 && N % 2 != 0)
    return fail(DK_ERR_SHAPE, "gemm_w4a16: the SwiGLU epilogue needs an even N (interleaved gate/up), got %d", N);
  if (!aligned16(packed) || !aligned16(x)) return fail(DK_ERR_ALIGN, "gemm_w4a16: packed and x must be 16B aligned");
  if (!aligned4(sz)) return fail(DK_ERR_ALIGN, "gemm_w4a16: sz must be 4B aligned");
  if (y == x) return fail(DK_ERR_DOMAIN, "gemm_w4a16: y must not alias x");
  return DK_OK;
}

int dk_gemm_w4a16(const void* packed, const void* sz, const void* x, void* y, int M, int N, int K, int group,
                  int epilogue, void* stream) {
  const int rc = gemm_check(packed, sz, x, y, M, N, K, group, epilogue);
  if (rc != DK_OK) return rc;
  clear_error();
  dk::launch_gemm_w4a16(packed, sz, x, y, M, N, K, ilog2(group), epilogue, nullptr, (hipStream_t)stream);
  return launched("gemm_w4a16");
}

size_t dk_gemm_w4a16_workspace_bytes(int M, int N, int K, int group, int epilogue) {
  if (M <= 0 || N <= 0 || K <= 0 || group < 32 || !pow2(group) || K % group != 0) return 0;
  return dk::gemm_w4a16_workspace_bytes(M, N, K, ilog2(group), epilogue);
}

int dk_gemm_w4a16_ws(const void* packed, const void* sz, const void* x, void* y, int M, int N, int K, int group,
                     int epilogue, void* workspace, size_t workspace_bytes, void* stream) {
  const bool parts = epilogue == 2;  // the fp32 split partials alone, left in the workspace (y unused)
  const int rc = gemm_check(packed, sz, x, parts ? workspace : y, M, N, K, group, parts ? 0 : epilogue);
  if (rc != DK_OK) return rc;
  const size_t need = dk::gemm_w4a16_workspace_bytes(M, N, K, ilog2(group), epilogue);
  if (parts && need == 0)
    return fail(DK_ERR_DOMAIN, "gemm_w4a16_ws: epilogue 2 (split partials only) needs a shape that splits "
                               "(gemm_w4a16_workspace_bytes > 0)");
  if (workspace != nullptr) {
    if (workspace_bytes < need)
      return fail(DK_ERR_SHAPE, "gemm_w4a16_ws: workspace of %zu bytes, this shape needs %zu", workspace_bytes, need);
    if (!aligned16(workspace)) return fail(DK_ERR_ALIGN, "gemm_w4a16_ws: workspace must be 16B aligned");
    if (!parts && need > 0 && ranges_overlap(workspace, need, y, (size_t)M * N * 2))
      return fail(DK_ERR_DOMAIN, "gemm_w4a16_ws: workspace must not overlap y");
    if (need > 0 && ranges_overlap(workspace, need, x, (size_t)M * K * 2))
      return fail(DK_ERR_DOMAIN, "gemm_w4a16_ws: workspace must not overlap x");
  }
  clear_error();
  dk::launch_gemm_w4a16(packed, sz, x, y, M, N, K, ilog2(group), epilogue, need > 0 ? workspace : nullptr,
                        (hipStream_t)stream);
  return launched("gemm_w4a16_ws");
}

int dk_bw_read(const void* buf, size_t bytes, uint32_t* sink, int sink_words, int blocks, int threads, int unroll,
               void* stream) {
  if (!buf || !sink) return fail(DK_ERR_NULL, "bw_read: null pointer argument");
  if (!aligned16(buf)) return fail(DK_ERR_ALIGN, "buf must be 16B aligned");
  if (!aligned4(sink)) return fail(DK_ERR_ALIGN, "bw_read: sink must be 4B aligned");
  if (bytes < 16) return fail(DK_ERR_SHAPE, "bw_read: the buffer must hold at least one 16-byte word, got %zu B", bytes);
  if (sink_words < 1) return fail(DK_ERR_SHAPE, "bw_read: sink_words must be >= 1, got %d", sink_words);
  if (blocks < 1 || blocks > (1 << 22))
    return fail(DK_ERR_SHAPE, "bw_read: blocks must be 1..%d, got %d", 1 << 22, blocks);
  if (threads < 64 || threads > 1024 || threads % 64 != 0)
    return fail(DK_ERR_SHAPE, "bw_read: threads must be a multiple of 64 in [64, 1024], got %d", threads);
  if (unroll != 1 && unroll != 2 && unroll != 4 && unroll != 8 && unroll != 16)
    return fail(DK_ERR_DOMAIN, "bw_read: unroll must be 1, 2, 4, 8 or 16, got %d", unroll);
  clear_error();
  dk::launch_read_probe(buf, bytes, sink, (uint32_t)sink_words, blocks, threads, unroll, (hipStream_t)stream);
  return launched("bw_read");
}

}  // extern "C"

namespace {

// Argument checks shared by dk_paged_attention and dk_paged_attention_noalloc (everything but the split buffers).
int check_paged_attention(int version, const void* q, const void* kc, const void* vc, const int32_t* bt,
                          const int32_t* pos, int n_q, int n_kv, int head_dim, int page, int n_pages, int n_bt,
                          int part_size, int max_splits, const void* out) {
  if (!q || !kc || !vc || !bt || !pos || !out) return fail(DK_ERR_NULL, "paged_attention: null pointer argument");
  if (head_dim != 64 && head_dim != 128)
    return fail(DK_ERR_SHAPE, "paged_attention: head_dim must be 64 or 128, got %d", head_dim);
  if (n_q <= 0 || n_kv <= 0 || n_q % n_kv != 0)
    return fail(DK_ERR_SHAPE, "heads-per-group must be 1/2/4/8 (n_q=%d n_kv=%d)", n_q, n_kv);
  const int hpg = n_q / n_kv;
  if (hpg != 1 && hpg != 2 && hpg != 4 && hpg != 8)
    return fail(DK_ERR_SHAPE, "heads-per-group must be 1/2/4/8, got %d", hpg);
  if (!pow2(page)) return fail(DK_ERR_DOMAIN, "page size must be a power of two, got %d", page);
  if (part_size <= 0) return fail(DK_ERR_DOMAIN, "part_size must be > 0");
  if (version < 1 || version > 5)
    return fail(DK_ERR_DOMAIN, "attention version must be 1..5, got %d", version);
  if (version == 5 && !dk::attn_lean_fits(part_size, ilog2(page), head_dim))
    return fail(DK_ERR_DOMAIN, "paged_attention: version 5 needs pages of >= 16 tokens and a part_size that is a "
                "multiple of 16 up to %d (part_size %d, page %d)", dk::attn_lean_max_part(head_dim), part_size, page);
  if (max_splits < 1 || max_splits > 65535)
    return fail(DK_ERR_SHAPE, "paged_attention: max_splits must be 1..65535, got %d", max_splits);
  if (n_pages < 1 || n_bt < 1) return fail(DK_ERR_SHAPE, "paged_attention: empty cache or block table");
  if (n_kv > 65535 || n_q > 65535) return fail(DK_ERR_SHAPE, "paged_attention: too many heads");
  if (!aligned16(q) || !aligned16(kc) || !aligned16(vc))
    return fail(DK_ERR_ALIGN, "q, kc and vc must be 16B aligned");
  return DK_OK;
}

// Split kernel of a paged_attention version: 1-3 (the reference's versions, kernels/bindings.cpp:56) the lean MFMA
// kernel wherever it takes the part size and page, else the block kernel; 4 the block kernel; 5 the lean kernel.
int attention_impl_of(int version, int part_size, int page, int head_dim) {
  if (version == 4) return 1;
  if (version == 5) return 3;
  return dk::attn_lean_fits(part_size, ilog2(page), head_dim) ? 3 : 1;
}

void launch_reference_attention(int version, const void* q, const void* kc, const void* vc, const int32_t* bt,
                                const int32_t* pos, int n_q, int n_kv, int head_dim, int page, int n_pages, int n_bt,
                                int part_size, int max_splits, float* o_part, float* m_part, float* l_part,
                                void* out, void* stream, bool split_only = false) {
  const dk::AttnLaunch a{q, nullptr, nullptr, 0, pos, bt, n_bt, const_cast<void*>(kc), const_cast<void*>(vc), n_pages,
                         ilog2(page), n_q, n_kv, head_dim, part_size, max_splits, o_part, m_part, l_part, out,
                         attention_impl_of(version, part_size, page, head_dim), split_only};
  dk::launch_paged_attention(a, (hipStream_t)stream);
}

// ---- scratch of dk_paged_attention_noalloc ---------------------------------------------------------------------
// The split partials of the allocation-free attention live in this file-scope device array; every GPU the library
// runs on holds its own copy until the process ends, and every call on a GPU shares it (calls that overlap on one
// GPU race). In host code the name `scratch` is a stand-in, not a device address: the entry point's first call on a
// device resolves the device address with hipGetSymbolAddress, with that device current, keeps it per device, and
// only that address is ever passed to a kernel.
static __device__ __align__(256) unsigned char scratch[DK_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

int scratch_of_current_device(void** ptr) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(DK_ERR_LAUNCH, "paged_attention_noalloc: no current device (or device id >= %d)", kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(DK_ERR_LAUNCH, "paged_attention_noalloc: hipGetSymbolAddress of the scratch array failed: %s",
                  hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return DK_OK;
}

size_t round256(size_t b) { return (b + 255) & ~(size_t)255; }

}  // namespace

extern "C" {

int dk_paged_attention(int version, const void* q, const void* kc, const void* vc, const int32_t* bt,
                       const int32_t* pos, int n_q, int n_kv, int head_dim, int page, int n_pages, int n_bt,
                       int part_size, int max_splits, float* o_part, float* m_part, float* l_part, void* out,
                       void* stream) {
  if (!o_part || !m_part || !l_part) return fail(DK_ERR_NULL, "paged_attention: null pointer argument");
  const int rc = check_paged_attention(version, q, kc, vc, bt, pos, n_q, n_kv, head_dim, page, n_pages, n_bt,
                                       part_size, max_splits, out);
  if (rc != DK_OK) return rc;
  if (!aligned16(o_part)) return fail(DK_ERR_ALIGN, "o_part must be 16B aligned");
  clear_error();
  launch_reference_attention(version, q, kc, vc, bt, pos, n_q, n_kv, head_dim, page, n_pages, n_bt, part_size,
                             max_splits, o_part, m_part, l_part, out, stream);
  return launched("paged_attention");
}

int dk_paged_attention_split(int version, const void* q, const void* kc, const void* vc, const int32_t* bt,
                             const int32_t* pos, int n_q, int n_kv, int head_dim, int page, int n_pages, int n_bt,
                             int part_size, int max_splits, float* o_part, float* m_part, float* l_part, void* out,
                             void* stream) {
  if (!o_part || !m_part || !l_part) return fail(DK_ERR_NULL, "paged_attention_split: null pointer argument");
  const int rc = check_paged_attention(version, q, kc, vc, bt, pos, n_q, n_kv, head_dim, page, n_pages, n_bt,
                                       part_size, max_splits, out);
  if (rc != DK_OK) return rc;
  if (!aligned16(o_part)) return fail(DK_ERR_ALIGN, "o_part must be 16B aligned");
  clear_error();
  launch_reference_attention(version, q, kc, vc, bt, pos, n_q, n_kv, head_dim, page, n_pages, n_bt, part_size,
                             max_splits, o_part, m_part, l_part, out, stream, true);
  return launched("paged_attention_split");
}

int dk_gemv_w4a16_attn(int stage, int R, int warps, int pf, const void* packed, const void* sz, const float* o_part,
                       const float* m_part, const float* l_part, const void* attn, const int32_t* pos, int n_bt,
                       int page, int part_size, int max_splits, int max_pos, int n_q, int head_dim, void* y, int N,
                       int K, int group, void* stream) {
  const int rc = check_fused_gemv("gemv_w4a16_attn", stage, R, warps, pf, packed, sz, N, K, group);
  if (rc != DK_OK) return rc;
  if (!o_part || !m_part || !l_part || !attn || !pos || !y)
    return fail(DK_ERR_NULL, "gemv_w4a16_attn: null pointer argument");
  if (head_dim != 64 && head_dim != 128)
    return fail(DK_ERR_SHAPE, "gemv_w4a16_attn: head_dim must be 64 or 128, got %d", head_dim);
  if (n_q <= 0 || (long long)n_q * head_dim != K)
    return fail(DK_ERR_SHAPE, "gemv_w4a16_attn: K must be n_q * head_dim (K=%d n_q=%d head_dim=%d)", K, n_q,
                head_dim);
  if (max_splits < 1 || max_splits > dk::kGemvCombineMaxSplits)
    return fail(DK_ERR_SHAPE, "gemv_w4a16_attn: max_splits must be 1..%d, got %d", dk::kGemvCombineMaxSplits,
                max_splits);
  if (part_size <= 0) return fail(DK_ERR_DOMAIN, "gemv_w4a16_attn: part_size must be > 0");
  if (!pow2(page)) return fail(DK_ERR_DOMAIN, "gemv_w4a16_attn: page size must be a power of two, got %d", page);
  if (n_bt < 1 || ((long long)n_bt << ilog2(page)) > (1ll << 30))
    return fail(DK_ERR_SHAPE, "gemv_w4a16_attn: n_bt must be >= 1 with n_bt * page <= 2^30, got %d", n_bt);
  if (max_pos < 0) return fail(DK_ERR_DOMAIN, "gemv_w4a16_attn: max_pos must be >= 0 (0 = no range check)");
  if (warps * 64 < K / 8 || warps > dk::kGemvCombineMaxWarps)
    return fail(DK_ERR_SHAPE, "gemv_w4a16_attn: the workgroup needs one thread per 8 values of x and at most %d "
                "waves: warps %d..%d for K=%d, got %d", dk::kGemvCombineMaxWarps, (K / 8 + 63) / 64,
                dk::kGemvCombineMaxWarps, K, warps);
  if (!aligned16(o_part) || !aligned16(attn)) return fail(DK_ERR_ALIGN, "o_part and attn must be 16B aligned");
  if (!aligned4(m_part) || !aligned4(l_part)) return fail(DK_ERR_ALIGN, "m_part and l_part must be 4B aligned");
  if (y == attn || y == o_part || y == m_part || y == l_part)
    return fail(DK_ERR_DOMAIN, "gemv_w4a16_attn: y must not alias attn, o_part, m_part or l_part (every workgroup "
                "reads all of them while others write y)");
  dk::GemvInput in{};
  in.comb = dk::GemvCombine{o_part, m_part, l_part, attn, pos, n_bt << ilog2(page), part_size, max_splits, max_pos,
                            ilog2(head_dim)};
  clear_error();
  dk::launch_gemv_w4a16_fused(2, 0, R, warps, pf, packed, sz, in, y, N, K, ilog2(group), (hipStream_t)stream);
  return launched("gemv_w4a16_attn");
}

size_t dk_paged_attention_noalloc_bytes(int n_q, int head_dim, int max_splits) {
  if (n_q <= 0 || head_dim <= 0 || max_splits <= 0) return 0;
  const size_t cells = (size_t)n_q * (size_t)max_splits;
  return round256(cells * (size_t)head_dim * 4) + 2 * round256(cells * 4);
}

int dk_paged_attention_noalloc(int version, const void* q, const void* kc, const void* vc, const int32_t* bt,
                               const int32_t* pos, int n_q, int n_kv, int head_dim, int page, int n_pages, int n_bt,
                               int part_size, int max_splits, void* out, void* stream) {
  const int rc = check_paged_attention(version, q, kc, vc, bt, pos, n_q, n_kv, head_dim, page, n_pages, n_bt,
                                       part_size, max_splits, out);
  if (rc != DK_OK) return rc;
  const size_t need = dk_paged_attention_noalloc_bytes(n_q, head_dim, max_splits);
  if (need > (size_t)DK_NOALLOC_SCRATCH_BYTES)
    return fail(DK_ERR_SHAPE, "paged_attention_noalloc: the split partials of %d heads x %d splits x head_dim %d "
                "need %zu bytes, more than the %u-byte scratch array; use dk_paged_attention with caller buffers "
                "or a larger part_size", n_q, max_splits, head_dim, need, (unsigned)DK_NOALLOC_SCRATCH_BYTES);
  void* base = nullptr;
  const int rs = scratch_of_current_device(&base);
  if (rs != DK_OK) return rs;
  const size_t cells = (size_t)n_q * (size_t)max_splits;
  unsigned char* b = static_cast<unsigned char*>(base);
  float* o_part = reinterpret_cast<float*>(b);
  float* m_part = reinterpret_cast<float*>(b + round256(cells * (size_t)head_dim * 4));
  float* l_part = reinterpret_cast<float*>(b + round256(cells * (size_t)head_dim * 4) + round256(cells * 4));
  clear_error();
  launch_reference_attention(version, q, kc, vc, bt, pos, n_q, n_kv, head_dim, page, n_pages, n_bt, part_size,
                             max_splits, o_part, m_part, l_part, out, stream);
  return launched("paged_attention_noalloc");
}

int dk_attention_decode(const void* qkv, const float* cos_t, const float* sin_t, int max_pos, const int32_t* pos,
                        const int32_t* bt, int n_bt, void* kc, void* vc, int n_pages, int page, int n_q, int n_kv,
                        int head_dim, int part_size, int max_splits, int impl, float* o_part, float* m_part,
                        float* l_part, void* out, void* stream) {
  if (!qkv || !cos_t || !sin_t || !pos || !bt || !kc || !vc || !o_part || !m_part || !l_part || !out)
    return fail(DK_ERR_NULL, "attention_decode: null pointer argument");
  if (impl < 0 || impl > 3 || impl == 2)
    return fail(DK_ERR_DOMAIN, "attention_decode: impl must be 0, 1 or 3, got %d", impl);
  if (head_dim != 64 && head_dim != 128)
    return fail(DK_ERR_SHAPE, "attention_decode: head_dim must be 64 or 128, got %d", head_dim);
  if (n_q <= 0 || n_kv <= 0 || n_q % n_kv != 0)
    return fail(DK_ERR_SHAPE, "heads-per-group must be 1/2/4/8 (n_q=%d n_kv=%d)", n_q, n_kv);
  const int hpg = n_q / n_kv;
  if (hpg != 1 && hpg != 2 && hpg != 4 && hpg != 8)
    return fail(DK_ERR_SHAPE, "heads-per-group must be 1/2/4/8, got %d", hpg);
  if (!pow2(page)) return fail(DK_ERR_DOMAIN, "page size must be a power of two, got %d", page);
  if (part_size <= 0) return fail(DK_ERR_DOMAIN, "part_size must be > 0");
  if (max_splits < 1 || max_splits > 65535)
    return fail(DK_ERR_SHAPE, "attention_decode: max_splits must be 1..65535, got %d", max_splits);
  if (n_pages < 1 || n_bt < 1 || max_pos < 1)
    return fail(DK_ERR_SHAPE, "attention_decode: empty cache, block table or rope table");
  if (n_kv > 65535 || n_q > 65535) return fail(DK_ERR_SHAPE, "attention_decode: too many heads");
  if (!aligned16(qkv) || !aligned16(kc) || !aligned16(vc))
    return fail(DK_ERR_ALIGN, "qkv, kc and vc must be 16B aligned");
  if (!aligned16(o_part)) return fail(DK_ERR_ALIGN, "o_part must be 16B aligned");
  clear_error();
  if (impl == 3 && !dk::attn_lean_fits(part_size, ilog2(page), head_dim))
    return fail(DK_ERR_DOMAIN, "attention_decode: impl 3 needs pages of >= 16 tokens and a part_size that is a "
                "multiple of 16 up to %d (part_size %d, page %d)", dk::attn_lean_max_part(head_dim), part_size, page);
  const dk::AttnLaunch a{qkv, cos_t, sin_t, max_pos, pos, bt, n_bt, kc, vc, n_pages, ilog2(page), n_q, n_kv,
                         head_dim, part_size, max_splits, o_part, m_part, l_part, out, impl};
  dk::launch_attention_decode(a, (hipStream_t)stream);
  return launched("attention_decode");
}

int dk_add_rmsnorm(void* x, const void* delta, const void* w, void* out, int H, float eps, void* stream) {
  if (!x || !w || !out) return fail(DK_ERR_NULL, "add_rmsnorm: null pointer argument");
  if (H <= 0 || H % 8 != 0)
    return fail(DK_ERR_SHAPE, "add_rmsnorm: H must be a positive multiple of 8, got %d", H);
  if (!aligned16(x)) return fail(DK_ERR_ALIGN, "x must be 16B aligned");
  if (!aligned16(w)) return fail(DK_ERR_ALIGN, "w must be 16B aligned");
  if (!aligned16(out)) return fail(DK_ERR_ALIGN, "out must be 16B aligned");
  if (delta && !aligned16(delta)) return fail(DK_ERR_ALIGN, "delta must be 16B aligned");
  if (H > dk::kRowNormMaxH && (out == x || (delta && (out == delta || x == delta))))
    return fail(DK_ERR_DOMAIN, "add_rmsnorm: for H > %d (two passes over the row in memory) x, delta and out must "
                "not alias", dk::kRowNormMaxH);
  clear_error();
  dk::launch_add_rmsnorm(x, delta, w, out, H, eps, (hipStream_t)stream);
  return launched("add_rmsnorm");
}

int dk_swiglu(const void* gu, void* out, int I, void* stream) {
  if (!gu || !out) return fail(DK_ERR_NULL, "swiglu: null pointer argument");
  if (I <= 0 || I % 8 != 0) return fail(DK_ERR_SHAPE, "swiglu: I must be a positive multiple of 8, got %d", I);
  if (!aligned16(gu)) return fail(DK_ERR_ALIGN, "gu must be 16B aligned");
  if (!aligned16(out)) return fail(DK_ERR_ALIGN, "out must be 16B aligned");
  clear_error();
  dk::launch_swiglu(gu, out, I, (hipStream_t)stream);
  return launched("swiglu");
}

int dk_rope_append(void* qkv, const float* cos_t, const float* sin_t, const int32_t* pos, const int32_t* bt,
                   void* kc, void* vc, int n_q, int n_kv, int head_dim, int page, int max_pos, int n_pages,
                   int n_bt, void* stream) {
  if (!qkv || !cos_t || !sin_t || !pos || !bt || !kc || !vc)
    return fail(DK_ERR_NULL, "rope_append: null pointer argument");
  if (head_dim != 64 && head_dim != 128)
    return fail(DK_ERR_SHAPE, "rope_append: head_dim must be 64 or 128, got %d", head_dim);
  if (n_q <= 0 || n_kv <= 0 || n_q > 65535 || n_kv > 65535)
    return fail(DK_ERR_SHAPE, "rope_append: bad head counts (n_q=%d n_kv=%d)", n_q, n_kv);
  if (!pow2(page)) return fail(DK_ERR_DOMAIN, "page size must be a power of two, got %d", page);
  if (max_pos < 1 || n_pages < 1 || n_bt < 1)
    return fail(DK_ERR_SHAPE, "rope_append: empty rope table, cache or block table");
  clear_error();
  dk::launch_rope_append(qkv, cos_t, sin_t, pos, bt, kc, vc, n_q, n_kv, head_dim, ilog2(page), max_pos, n_pages,
                         n_bt, 1, (hipStream_t)stream);
  return launched("rope_append");
}

int dk_rope_append_rows(void* qkv, const float* cos_t, const float* sin_t, const int32_t* pos, const int32_t* bt,
                        void* kc, void* vc, int M, int n_q, int n_kv, int head_dim, int page, int max_pos,
                        int n_pages, int n_bt, void* stream) {
  if (!qkv || !cos_t || !sin_t || !pos || !bt || !kc || !vc)
    return fail(DK_ERR_NULL, "rope_append_rows: null pointer argument");
  if (head_dim != 64 && head_dim != 128)
    return fail(DK_ERR_SHAPE, "rope_append_rows: head_dim must be 64 or 128, got %d", head_dim);
  if (n_q <= 0 || n_kv <= 0 || n_q > 65535 || n_kv > 65535)
    return fail(DK_ERR_SHAPE, "rope_append_rows: bad head counts (n_q=%d n_kv=%d)", n_q, n_kv);
  if (M < 1 || M > 65535) return fail(DK_ERR_SHAPE, "rope_append_rows: M must be 1..65535, got %d", M);
  if (!pow2(page)) return fail(DK_ERR_DOMAIN, "page size must be a power of two, got %d", page);
  if (max_pos < 1 || n_pages < 1 || n_bt < 1)
    return fail(DK_ERR_SHAPE, "rope_append_rows: empty rope table, cache or block table");
  clear_error();
  dk::launch_rope_append(qkv, cos_t, sin_t, pos, bt, kc, vc, n_q, n_kv, head_dim, ilog2(page), max_pos, n_pages,
                         n_bt, M, (hipStream_t)stream);
  return launched("rope_append_rows");
}

int dk_rmsnorm_rows(const void* x_in, const int64_t* rows, int n_src, const void* delta, const void* w, void* x_out,
                    void* out, int M, int H, float eps, void* stream) {
  if (!x_in || !w || !x_out || !out) return fail(DK_ERR_NULL, "rmsnorm_rows: null pointer argument");
  if (M < 1 || M > (1 << 24)) return fail(DK_ERR_SHAPE, "rmsnorm_rows: M must be 1..2^24, got %d", M);
  if (H <= 0 || H % 8 != 0 || H > dk::kRowNormMaxH)
    return fail(DK_ERR_SHAPE, "rmsnorm_rows: H must be a positive multiple of 8 (<= %d), got %d", dk::kRowNormMaxH, H);
  if (!aligned16(x_in) || !aligned16(w) || !aligned16(x_out) || !aligned16(out) || (delta && !aligned16(delta)))
    return fail(DK_ERR_ALIGN, "rmsnorm_rows: x_in, delta, w, x_out and out must be 16B aligned");
  if (rows && (reinterpret_cast<uintptr_t>(rows) & 7u)) return fail(DK_ERR_ALIGN, "rmsnorm_rows: rows must be 8B aligned");
  if (out == x_in || out == x_out || (delta && out == delta))
    return fail(DK_ERR_DOMAIN, "rmsnorm_rows: out must not alias x_in, x_out or delta");
  if (rows && x_out == x_in) return fail(DK_ERR_DOMAIN, "rmsnorm_rows: a gathered x_in must not be x_out");
  if (rows ? n_src < 1 : n_src != M)
    return fail(DK_ERR_SHAPE, "rmsnorm_rows: n_src (rows of x_in) must be >= 1 with rows, M without, got %d", n_src);
  clear_error();
  dk::launch_rmsnorm_rows(x_in, rows, n_src, delta, w, x_out, out, M, H, eps, (hipStream_t)stream);
  return launched("rmsnorm_rows");
}

int dk_rmsnorm_rows_parts(const void* x_in, const float* parts, int splits, long long part_stride, const void* w,
                          void* x_out, void* out, int M, int H, float eps, void* stream) {
  if (!x_in || !parts || !w || !x_out || !out) return fail(DK_ERR_NULL, "rmsnorm_rows_parts: null pointer argument");
  if (M < 1 || M > (1 << 24)) return fail(DK_ERR_SHAPE, "rmsnorm_rows_parts: M must be 1..2^24, got %d", M);
  if (H <= 0 || H % 8 != 0 || H > dk::kRowNormMaxH)
    return fail(DK_ERR_SHAPE, "rmsnorm_rows_parts: H must be a positive multiple of 8 (<= %d), got %d",
                dk::kRowNormMaxH, H);
  if (splits < 1 || splits > 64) return fail(DK_ERR_SHAPE, "rmsnorm_rows_parts: splits must be 1..64, got %d", splits);
  if (part_stride % 4 != 0 || (splits > 1 && part_stride < (long long)H))
    return fail(DK_ERR_SHAPE, "rmsnorm_rows_parts: part_stride must be a multiple of 4 and >= H, got %lld", part_stride);
  if (!aligned16(x_in) || !aligned16(parts) || !aligned16(w) || !aligned16(x_out) || !aligned16(out))
    return fail(DK_ERR_ALIGN, "rmsnorm_rows_parts: x_in, parts, w, x_out and out must be 16B aligned");
  if (out == x_in || out == x_out) return fail(DK_ERR_DOMAIN, "rmsnorm_rows_parts: out must not alias x_in or x_out");
  const size_t pbytes = ((size_t)(splits - 1) * (size_t)part_stride + (size_t)M * H) * sizeof(float);
  if (ranges_overlap(parts, pbytes, x_out, (size_t)M * H * 2) || ranges_overlap(parts, pbytes, out, (size_t)M * H * 2))
    return fail(DK_ERR_DOMAIN, "rmsnorm_rows_parts: parts must not overlap x_out or out");
  clear_error();
  dk::launch_rmsnorm_rows_parts(x_in, parts, splits, part_stride, w, x_out, out, M, H, eps, (hipStream_t)stream);
  return launched("rmsnorm_rows_parts");
}

int dk_attention_prefill(const void* qkv, const int32_t* pos, const int32_t* bt, int n_bt, const void* kc,
                         const void* vc, int n_pages, int page, int n_q, int n_kv, int head_dim, int M, int max_ctx,
                         void* out, void* stream) {
  if (!qkv || !pos || !bt || !kc || !vc || !out) return fail(DK_ERR_NULL, "attention_prefill: null pointer argument");
  if (head_dim != 64 && head_dim != 128)
    return fail(DK_ERR_SHAPE, "attention_prefill: head_dim must be 64 or 128, got %d", head_dim);
  if (n_q <= 0 || n_kv <= 0 || n_q % n_kv != 0)
    return fail(DK_ERR_SHAPE, "heads-per-group must be 1/2/4/8 (n_q=%d n_kv=%d)", n_q, n_kv);
  const int hpg = n_q / n_kv;
  if (hpg != 1 && hpg != 2 && hpg != 4 && hpg != 8)
    return fail(DK_ERR_SHAPE, "heads-per-group must be 1/2/4/8, got %d", hpg);
  if (n_kv > 65535) return fail(DK_ERR_SHAPE, "attention_prefill: too many kv heads");
  if (M < 1 || M > 65535) return fail(DK_ERR_SHAPE, "attention_prefill: M must be 1..65535, got %d", M);
  if (!pow2(page)) return fail(DK_ERR_DOMAIN, "page size must be a power of two, got %d", page);
  if (n_pages < 1 || n_bt < 1) return fail(DK_ERR_SHAPE, "attention_prefill: empty cache or block table");
  if (max_ctx < 1) return fail(DK_ERR_DOMAIN, "attention_prefill: max_ctx must be >= 1, got %d", max_ctx);
  if (!aligned16(qkv) || !aligned16(kc) || !aligned16(vc))
    return fail(DK_ERR_ALIGN, "qkv, kc and vc must be 16B aligned");
  clear_error();
  dk::launch_attention_prefill(qkv, pos, bt, n_bt, kc, vc, n_pages, ilog2(page), n_q, n_kv, head_dim, M, max_ctx, out,
                               (hipStream_t)stream);
  return launched("attention_prefill");
}

int dk_argmax_advance(const void* logits, int V, int64_t* tok, int32_t* pos, void* stream) {
  if (!logits || !tok) return fail(DK_ERR_NULL, "argmax_advance: null pointer argument");
  if (V <= 0) return fail(DK_ERR_SHAPE, "argmax_advance: V must be positive, got %d", V);
  if (!aligned4(tok) || (pos && !aligned4(pos))) return fail(DK_ERR_ALIGN, "tok and pos must be 4B aligned");
  clear_error();
  dk::launch_argmax_advance(logits, V, tok, pos, (hipStream_t)stream);
  return launched("argmax_advance");
}

int dk_argmax_advance_split(const void* logits, int V, int64_t* tok, int32_t* pos, uint64_t* work, void* stream) {
  if (!logits || !tok || !work) return fail(DK_ERR_NULL, "argmax_advance_split: null pointer argument");
  if (V <= 0) return fail(DK_ERR_SHAPE, "argmax_advance_split: V must be positive, got %d", V);
  if (!aligned4(tok) || (pos && !aligned4(pos))) return fail(DK_ERR_ALIGN, "tok and pos must be 4B aligned");
  if (reinterpret_cast<uintptr_t>(work) & 7u) return fail(DK_ERR_ALIGN, "argmax_advance_split: work must be 8B aligned");
  clear_error();
  dk::launch_argmax_split(logits, V, tok, pos, reinterpret_cast<unsigned long long*>(work), (hipStream_t)stream);
  return launched("argmax_advance_split");
}

int dk_quantize_w4(const void* w, void* packed, void* sz, int N, int K, int group, int clip, void* stream) {
  if (!w || !packed || !sz) return fail(DK_ERR_NULL, "quantize_w4: null pointer argument");
  if (N <= 0 || K <= 0) return fail(DK_ERR_SHAPE, "quantize_w4: N and K must be positive");
  if (!pow2(group) || group < 32 || group > 512)
    return fail(DK_ERR_DOMAIN, "quantize_w4: group must be a power of two in [32, 512], got %d", group);
  if (K % group != 0) return fail(DK_ERR_SHAPE, "quantize_w4: K=%d is not a multiple of group=%d", K, group);
  if ((long long)N * (K / 8) > (1LL << 40)) return fail(DK_ERR_SHAPE, "quantize_w4: matrix too large");
  if (!aligned16(w)) return fail(DK_ERR_ALIGN, "w must be 16B aligned");
  if (!aligned4(packed) || !aligned4(sz)) return fail(DK_ERR_ALIGN, "packed and sz must be 4B aligned");
  clear_error();
  if (clip != 0 && clip != 1) return fail(DK_ERR_DOMAIN, "quantize_w4: clip must be 0 or 1, got %d", clip);
  dk::launch_quantize_w4(w, packed, sz, N, K, ilog2(group), clip, (hipStream_t)stream);
  return launched("quantize_w4");
}


}  // extern "C"
