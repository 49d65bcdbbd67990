// Paged split-K GQA decode attention (one query token) on gfx950, with an optional fused RoPE + KV append.
//
// Cache layout (runtime/model.py:117-120 of the reference): kc / vc fp16 [pages, n_kv, P, D]; token t of the
// sequence lives in physical page bt[t / P], slot t % P, so one (page, kv head) holds P contiguous D-vectors.
// Context = min(*pos + 1, n_bt * P) read from device memory, so one captured graph serves every decode step.
//
// Grid (n_kv, max_splits), 256 threads. Workgroup (kvh, s) owns tokens [s*PS, min(ctx, (s+1)*PS)) for all HPG query
// heads of kv head kvh, so every K/V byte is read from HBM once. Splits past ceil(ctx / PS) exit at once.
// The split is processed in blocks of TB tokens, three phases per block:
//   1. token-major: lane (g, c) of a wave holds the 16-byte slice c (dims 8c..8c+7) of token slot g; CPL = D/8 lanes
//      cover one token, so one wave load reads TPL = 64/CPL consecutive tokens (1 KB contiguous inside a page).
//      Scores q.k per head: v_dot2_f32_f16 on the fp16 pairs (exact products, fp32 sums), summed over the CPL lanes
//      with DPP, times 1/sqrt(D) in fp32. Scores go to LDS s_s[h][t], the V slices to LDS s_v[t][.].
//   2. head-major: the 256/HPG threads of head h each read all TB scores of the block (LDS broadcast), update the
//      running maximum M, compute p = exp(s - M) for their share of tokens into s_p[h][t].
//   3. head-major: thread (h, j) owns dims [j*DPT, (j+1)*DPT) of head h: acc = a*acc + sum_t p[h][t] V[t][dims],
//      l = a*l + sum_t p[h][t] with a = exp(M_old - M_new) (the online-softmax rescale between blocks).
// No cross-lane reduction of the output is ever needed: every output element is accumulated by one thread.
// With one live split the normalised output acc / l is written directly. Otherwise each split writes unnormalized
// o, m = M, l, and the combine
//     M* = max_s m_s;  L = sum_s e^(m_s - M*) l_s;  O = sum_s e^(m_s - M*) o_s / L
// runs in a second kernel, one workgroup per query head (split lanes x 4-dim groups issue all their partial loads at
// once, keep an online maximum, and merge through LDS).
//
// ROPE mode (fused decode step): q and the new k come from the fused qkv vector, rotated with the rotate_half
// convention (pairs (i, i + D/2), fp32 tables), each product rounded separately as the reference's elementwise fp32
// ops do; rotated values are rounded to fp16 (reference/ref_ops.py:36-53). The workgroup that owns token pos
// (split pos / PS, or the last live split if the cap is smaller) writes k and v into page bt[pos / P], slot pos % P,
// and uses the fresh values for token pos itself instead of the cache. If *pos is outside [0, max_pos) nothing is
// touched.
#include "common.hpp"
#include "launch.hpp"
#include "attn_common.hpp"

namespace dk {
namespace {

constexpr int kAttnThreads = 256;
constexpr int kAttnWaves = kAttnThreads / kWave;
constexpr int kNL = 2;  // token loads (of K and of V) per lane per block

template <int D, int HPG>
struct AttnShape {
  static constexpr int CPL = D / 8;                      // lanes per token row
  static constexpr int TPL = kWave / CPL;                // tokens per wave load
  static constexpr int TB = kAttnWaves * kNL * TPL;      // tokens per block (64 at D=64, 32 at D=128)
  static constexpr int NTH = kAttnThreads / HPG;         // threads per head in phases 2-3
  static constexpr int DPT = (HPG * D >= kAttnThreads) ? HPG * D / kAttnThreads : 1;  // dims per thread
};

__device__ __forceinline__ int attn_context(const int32_t* pos_ptr, int n_bt, int log2P) {
  const long long cap = (long long)n_bt << log2P;
  const long long ctx = (long long)(*pos_ptr) + 1;
  return (int)(ctx < cap ? ctx : cap);
}

template <int D, int HPG, bool ROPE>
__global__ void __launch_bounds__(kAttnThreads)
attn_decode_kernel(const f16* __restrict__ qsrc, const float* __restrict__ cos_t, const float* __restrict__ sin_t,
                   int max_pos, const int32_t* __restrict__ pos_ptr, const int32_t* __restrict__ bt, int n_bt,
                   f16* __restrict__ kc, f16* __restrict__ vc, int n_pages, int log2P, int n_q, int n_kv, int PS,
                   int max_splits, float scale, float* __restrict__ o_part, float* __restrict__ m_part,
                   float* __restrict__ l_part, f16* __restrict__ out) {
  using S = AttnShape<D, HPG>;
  constexpr int CPL = S::CPL, TPL = S::TPL, TB = S::TB, NTH = S::NTH, DPT = S::DPT;
  __shared__ float s_s[HPG][TB];
  __shared__ float s_p[HPG][TB];
  __shared__ u32x4 s_v[TB][CPL];

  const int kvh = blockIdx.x, split = blockIdx.y;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int g = lane / CPL, c = lane % CPL;
  const int P = 1 << log2P;
  // A split that starts past the last block-table token can hold no token (and split * PS may not fit an int).
  const long long t0l = (long long)split * PS;
  const bool reachable = t0l < ((long long)n_bt << log2P);
  const int t0 = reachable ? (int)t0l : 0;

  // Independent loads first: block-table entries of this lane's tokens in blocks 0 and 1, the q slices, the new k / v.
  // (Tokens past the split or the table get page -1; the live bound t1 is applied once pos is known.)
  int pg[kNL], pgn[kNL];
#pragma unroll
  for (int jn = 0; jn < kNL; ++jn) {
    const int tl = (wave * kNL + jn) * TPL + g;
    const int lp = (t0 + tl) >> log2P, lpn = (t0 + TB + tl) >> log2P;
    pg[jn] = (reachable && tl < PS && lp < n_bt) ? bt[lp] : -1;
    pgn[jn] = (reachable && TB + tl < PS && lpn < n_bt) ? bt[lpn] : -1;
  }
  // K / V of block 0 go out as soon as their pages are known, before anything that needs *pos (the RoPE tables, the
  // context bound): tokens past the context are masked in phase 1 (score -inf, V slice zero), so speculative loads
  // of the split's first block never reach the result. Only valid cache pages are read.
  u32x4 kr[kNL], vr[kNL], kn[kNL], vn[kNL];
#pragma unroll
  for (int jn = 0; jn < kNL; ++jn) {
    const int t = t0 + (wave * kNL + jn) * TPL + g;
    if (pg[jn] >= 0 && pg[jn] < n_pages) {
      const size_t off = ((((size_t)pg[jn] * n_kv + blockIdx.x) << log2P) + (t & (P - 1))) * D + 8 * c;
      kr[jn] = load_stream(reinterpret_cast<const u32x4*>(kc + off));
      vr[jn] = load_stream(reinterpret_cast<const u32x4*>(vc + off));
    } else {
      kr[jn] = u32x4{0u, 0u, 0u, 0u};
      vr[jn] = kr[jn];
    }
  }
  const int pos = *pos_ptr;
  const int cp = (c + CPL / 2) % CPL;  // partner slice for RoPE
  const bool first_half = c < CPL / 2;
  u32x4 qraw[HPG], qpart[HPG];
#pragma unroll
  for (int h = 0; h < HPG; ++h) {
    const f16* qh = qsrc + (size_t)(kvh * HPG + h) * D;
    qraw[h] = *reinterpret_cast<const u32x4*>(qh + 8 * c);
    if constexpr (ROPE) qpart[h] = *reinterpret_cast<const u32x4*>(qh + 8 * cp);
  }
  u32x4 knew = {0u, 0u, 0u, 0u}, vnew = {0u, 0u, 0u, 0u};
  if constexpr (ROPE) {
    const f16* kh = qsrc + (size_t)(n_q + kvh) * D;
    const f16* vh = qsrc + (size_t)(n_q + n_kv + kvh) * D;
    const u32x4 kown = *reinterpret_cast<const u32x4*>(kh + 8 * c);
    const u32x4 kpar = *reinterpret_cast<const u32x4*>(kh + 8 * cp);
    vnew = *reinterpret_cast<const u32x4*>(vh + 8 * c);
    if (pos < 0 || pos >= max_pos) return;  // uniform: nothing is touched
    const int ti = (8 * c) % (D / 2);
    float cs[8], sn[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      cs[e] = cos_t[(size_t)pos * (D / 2) + ti + e];
      sn[e] = sin_t[(size_t)pos * (D / 2) + ti + e];
    }
#pragma unroll
    for (int h = 0; h < HPG; ++h) qraw[h] = rope_slice<D>(qraw[h], qpart[h], cs, sn, first_half);
    knew = rope_slice<D>(kown, kpar, cs, sn, first_half);
  }
  const int ctx = attn_context(pos_ptr, n_bt, log2P);
  const int nsplit = attn_splits(ctx, PS, max_splits);
  if (ROPE) {
    // the workgroup owning token pos (or the last live split when the cap is below pos) appends k, v
    const int owner = min(pos / PS, nsplit - 1);
    if (split == owner && wave == 0 && lane < CPL) {
      const int lp = pos >> log2P;
      const int page = lp < n_bt ? bt[lp] : -1;
      if (page >= 0 && page < n_pages) {
        const size_t off = ((((size_t)page * n_kv + kvh) << log2P) + (pos & (P - 1))) * D + 8 * c;
        *reinterpret_cast<u32x4*>(kc + off) = knew;
        *reinterpret_cast<u32x4*>(vc + off) = vnew;
      }
    }
  }
  if (split >= nsplit || !reachable) return;
  const int t1 = (int)min((long long)ctx, t0l + PS);
  const int nblk = (t1 - t0 + TB - 1) / TB;

  // K / V of this lane's tokens in block b: pages pgb[], -1 = no token
  auto issue_kv = [&](int tb, const int (&pgb)[kNL], u32x4 (&kk)[kNL], u32x4 (&vv)[kNL]) {
#pragma unroll
    for (int jn = 0; jn < kNL; ++jn) {
      const int t = tb + (wave * kNL + jn) * TPL + g;
      if (t < t1 && pgb[jn] >= 0 && pgb[jn] < n_pages) {
        const size_t off = ((((size_t)pgb[jn] * n_kv + kvh) << log2P) + (t & (P - 1))) * D + 8 * c;
        kk[jn] = load_stream(reinterpret_cast<const u32x4*>(kc + off));
        vv[jn] = load_stream(reinterpret_cast<const u32x4*>(vc + off));
      } else {
        kk[jn] = u32x4{0u, 0u, 0u, 0u};
        vv[jn] = kk[jn];
      }
    }
  };

  const int h3 = tid / NTH, j3 = tid % NTH, d0 = j3 * DPT;
  float M = -INFINITY, l = 0.f, acc[DPT];
#pragma unroll
  for (int e = 0; e < DPT; ++e) acc[e] = 0.f;

  for (int b = 0; b < nblk; ++b) {
    const int tb = t0 + b * TB;
    // ---- pipeline: K / V of block b + 1 (pages loaded one block ahead) and pages of block b + 2 go out now, so
    // their latency overlaps the three phases of block b
    int pg2[kNL];
    if (b + 1 < nblk) issue_kv(tb + TB, pgn, kn, vn);
#pragma unroll
    for (int jn = 0; jn < kNL; ++jn) {
      const int t = tb + 2 * TB + (wave * kNL + jn) * TPL + g;
      const int lp = t >> log2P;
      pg2[jn] = (b + 2 < nblk && t < t1 && lp < n_bt) ? bt[lp] : -1;
    }
    // ---- phase 1: scores and V slices of this block (token-major)
#pragma unroll
    for (int jn = 0; jn < kNL; ++jn) {
      const int tl = (wave * kNL + jn) * TPL + g;
      const int t = tb + tl;
      const bool ok = t < t1 && pg[jn] >= 0 && pg[jn] < n_pages;
      u32x4 kk = kr[jn], vv = vr[jn];
      if (ROPE && t == pos && ok) {  // the cache slot of pos is being written by this launch: use the fresh k, v
        kk = knew;
        vv = vnew;
      }
      float sc[HPG];
#pragma unroll
      for (int h = 0; h < HPG; ++h) {
        float a = 0.f;
        a = dot2(as_f16x2(qraw[h].x), as_f16x2(kk.x), a);
        a = dot2(as_f16x2(qraw[h].y), as_f16x2(kk.y), a);
        a = dot2(as_f16x2(qraw[h].z), as_f16x2(kk.z), a);
        a = dot2(as_f16x2(qraw[h].w), as_f16x2(kk.w), a);
        sc[h] = group_sum_dpp<CPL>(a) * scale;
      }
#pragma unroll
      for (int h = 0; h < HPG; ++h)
        if (c == h) s_s[h][tl] = ok ? sc[h] : -INFINITY;
      s_v[tl][c] = ok ? vv : u32x4{0u, 0u, 0u, 0u};
    }
    __syncthreads();
    // ---- phase 2: block maximum and probabilities (head-major)
    float bm = -INFINITY;
#pragma unroll
    for (int t = 0; t < TB; t += 4) {
      const float4 v4 = *reinterpret_cast<const float4*>(&s_s[h3][t]);
      bm = fmaxf(bm, fmaxf(fmaxf(v4.x, v4.y), fmaxf(v4.z, v4.w)));
    }
    const float Mn = fmaxf(M, bm);
    const float alpha = (M == -INFINITY) ? 0.f : __expf(M - Mn);
    for (int t = j3; t < TB; t += NTH) {
      const float sv = s_s[h3][t];
      s_p[h3][t] = (sv == -INFINITY) ? 0.f : __expf(sv - Mn);
    }
    M = Mn;
    __syncthreads();
    // ---- phase 3: rescale and accumulate p . V (head-major)
    l *= alpha;
#pragma unroll
    for (int e = 0; e < DPT; ++e) acc[e] *= alpha;
    if (d0 < D) {
      const f16* vbase = reinterpret_cast<const f16*>(&s_v[0][0]) + d0;
#pragma unroll 4
      for (int t = 0; t < TB; ++t) {
        const float p = s_p[h3][t];
        l += p;
        const f16* vt = vbase + (size_t)t * D;
#pragma unroll
        for (int e = 0; e < DPT; ++e) acc[e] = fmaf(p, (float)vt[e], acc[e]);
      }
    }
    __syncthreads();
    // ---- rotate the pipeline registers
#pragma unroll
    for (int jn = 0; jn < kNL; ++jn) {
      kr[jn] = kn[jn];
      vr[jn] = vn[jn];
      pg[jn] = pgn[jn];
      pgn[jn] = pg2[jn];
    }
  }

  const int head = kvh * HPG + h3;
  if (nsplit == 1) {
    if (d0 < D) {
      const float inv = l > 0.f ? 1.0f / l : 0.f;
#pragma unroll
      for (int e = 0; e < DPT; ++e) out[(size_t)head * D + d0 + e] = (f16)(acc[e] * inv);
    }
    return;
  }
  if (d0 >= D) return;
#pragma unroll
  for (int e = 0; e < DPT; ++e) o_part[((size_t)head * max_splits + split) * D + d0 + e] = acc[e];
  if (j3 == 0) {
    m_part[(size_t)head * max_splits + split] = M;
    l_part[(size_t)head * max_splits + split] = l;
  }
}

// Combine of the split partials of one query head per workgroup: thread (sl, d4) takes splits sl, sl + SLN, ... and
// dims [4 d4, 4 d4 + 4); every lane keeps an online maximum over its splits (loads of B splits in flight), then the
// SLN split lanes merge through LDS with the same max-rescale rule. The first B SLN splits' loads go out before *pos
// is read (clamped to the buffer's max_splits; splits past the live count are dropped by select once it is known), so
// the position's round trip overlaps theirs. The launcher picks B so that one batch covers max_splits (up to
// 16 SLN splits): every later batch would be one more dependent round trip.
template <int D, int B>
__global__ void __launch_bounds__(kAttnThreads)
attn_combine_kernel(const float* __restrict__ o_part, const float* __restrict__ m_part,
                    const float* __restrict__ l_part, const int32_t* __restrict__ pos_ptr, int max_pos, int n_bt,
                    int log2P, int PS, int max_splits, f16* __restrict__ out) {
  constexpr int NG = D / 4;                 // 4-dim groups per head
  constexpr int SLN = kAttnThreads / NG;    // split lanes
  __shared__ float s_m[SLN], s_l[SLN];
  __shared__ float4 s_a[SLN][NG];
  const int head = blockIdx.x, tid = threadIdx.x, sl = tid / NG, d4 = tid % NG;
  const float* m = m_part + (size_t)head * max_splits;
  const float* l = l_part + (size_t)head * max_splits;
  const float* op = o_part + (size_t)head * max_splits * D + 4 * d4;
  float ms[B], ls[B];
  float4 os[B];
#pragma unroll
  for (int k = 0; k < B; ++k) {  // first batch, speculative (in bounds of the partial buffers)
    const int s = min(sl + k * SLN, max_splits - 1);
    ms[k] = m[s];
    ls[k] = l[s];
    os[k] = *reinterpret_cast<const float4*>(op + (size_t)s * D);
  }
  // No early return before the first batch is consumed: the compiler would sink its loads below the test.
  const int pos = *pos_ptr;
  const bool skip = max_pos > 0 && (pos < 0 || pos >= max_pos);  // decode op: the split kernel did nothing
  const long long cap = (long long)n_bt << log2P;
  const int nsplit = skip ? 0 : attn_splits((int)((long long)pos + 1 < cap ? (long long)pos + 1 : cap), PS, max_splits);
  float M = -INFINITY, L = 0.f;
  float4 a = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = sl; s0 < nsplit; s0 += B * SLN) {
    if (s0 != sl) {
#pragma unroll
      for (int k = 0; k < B; ++k) {
        const int s = min(s0 + k * SLN, max_splits - 1);
        ms[k] = m[s];
        ls[k] = l[s];
        os[k] = *reinterpret_cast<const float4*>(op + (size_t)s * D);
      }
    }
#pragma unroll
    for (int k = 0; k < B; ++k) {  // splits past the live count: dropped (their partials are stale or never written)
      if (s0 + k * SLN >= nsplit) {
        ms[k] = -INFINITY;
        ls[k] = 0.f;
        os[k] = float4{0.f, 0.f, 0.f, 0.f};
      }
    }
    float Mn = M;
#pragma unroll
    for (int k = 0; k < B; ++k) Mn = fmaxf(Mn, ms[k]);
    if (Mn == -INFINITY) continue;
    const float r = (M == -INFINITY) ? 0.f : __expf(M - Mn);
    L *= r;
    a.x *= r;
    a.y *= r;
    a.z *= r;
    a.w *= r;
#pragma unroll
    for (int k = 0; k < B; ++k) {
      const float w = (ms[k] == -INFINITY) ? 0.f : __expf(ms[k] - Mn);
      L = fmaf(w, ls[k], L);
      a.x = fmaf(w, os[k].x, a.x);
      a.y = fmaf(w, os[k].y, a.y);
      a.z = fmaf(w, os[k].z, a.z);
      a.w = fmaf(w, os[k].w, a.w);
    }
    M = Mn;
  }
  if (nsplit <= 1) return;  // uniform: one live split wrote the output itself (or none was live)
  if (d4 == 0) {
    s_m[sl] = M;
    s_l[sl] = L;
  }
  s_a[sl][d4] = a;
  __syncthreads();
  if (tid < NG) {
    float Mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < SLN; ++i) Mx = fmaxf(Mx, s_m[i]);
    float Lt = 0.f;
    float4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < SLN; ++i) {
      const float w = (s_m[i] == -INFINITY) ? 0.f : __expf(s_m[i] - Mx);
      Lt = fmaf(w, s_l[i], Lt);
      o.x = fmaf(w, s_a[i][tid].x, o.x);
      o.y = fmaf(w, s_a[i][tid].y, o.y);
      o.z = fmaf(w, s_a[i][tid].z, o.z);
      o.w = fmaf(w, s_a[i][tid].w, o.w);
    }
    const float inv = Lt > 0.f ? 1.0f / Lt : 0.f;
    f16* dst = out + (size_t)head * D + 4 * tid;
    dst[0] = (f16)(o.x * inv);
    dst[1] = (f16)(o.y * inv);
    dst[2] = (f16)(o.z * inv);
    dst[3] = (f16)(o.w * inv);
  }
}

// ---------------------------------------------------------------------------------------------------------------
// MFMA formulation of the split workgroup (the arithmetic of the lean kernel below): the HPG query heads of a kv head
// are the columns of 16 x 16 matrix tiles, 16 tokens are the rows.
//   QK^T: S[token][head] = K_tile (16 tokens x D) . Q^T (D x 16 heads) with v_mfma_f32_16x16x16_f16 (fp16 products are
//         exact, fp32 sums), D / 16 steps. Lane l = 16 g + c of a wave feeds K row c (its token) and q head c, both
//         over dims [D/4 g, D/4 (g+1)): any bijection of the reduction index is valid as long as both operands use it,
//         and this one makes each lane's operand D/8 contiguous bytes of one row. The accumulator leaves lane l with
//         S[tokens 4g .. 4g+3][head c] -- exactly the A-operand layout of P (head c, tokens 4g + v) for the next MFMA.
//   P.V:  O[head][dim] += P (16 heads x 16 tokens) . V (16 tokens x 16 dims) per 16-dim tile. p is fp32; it is fed
//         as p_hi = fp16(p) plus p_lo = fp16(p - p_hi) in two MFMAs (about 22 significant bits, products with the fp16
//         V exact, fp32 accumulation), so the result keeps the fp32 quality of the reference's softmax. Output column c
//         of dim tile t holds dim (D/16) c + t, so each lane's V operand is D/16 contiguous dims of 4 token rows.
// An earlier kernel of this shape (8 waves, the split's block-table pages staged in LDS) was never chosen by the
// attention tuner over the lean kernel or the block kernel and was removed.
constexpr int kMfmaWaves = 8;

template <int D>
struct MfmaAttnShape {
  static constexpr int KD = D / 4;              // dims of a K row / q head per lane in the QK^T operands
  static constexpr int KW = KD / 8;             // their 16-byte chunks
  static constexpr int QS = D / 16;             // QK^T MFMA steps
  static constexpr int VD = D / 16;             // dims of a V row per lane in the P.V operand (= P.V dim tiles)
  static constexpr int NB = D == 64 ? 4 : 2;    // 16-token tiles per wave per round
  static constexpr int RT = kMfmaWaves * NB;    // tiles per round
};

// ---------------------------------------------------------------------------------------------------------------
// Lean MFMA split kernel (impl 3) for pages of at least 16 tokens: the MFMA arithmetic above (16 x 16 f16 tiles, p as
// fp16 hi + lo parts) with a schedule cut down to two dependent memory round trips:
//   * every kernel argument is read into scalar registers at entry (left to itself the compiler loads some of them
//     only where they are first used, and each such late load is one more round trip on the critical path);
//   * each wave owns NT 16-token tiles of the split (tile j = wave + NW i); a tile lies in one page, so its page is a
//     wave-uniform scalar load, issued at entry together with *pos -- no block-table staging and no barrier;
//   * then the q slices (for RoPE also their partners and the new k / v), then, once the pages are in, K and V of all
//     the wave's tiles at once, then the RoPE tables of *pos;
//   * one online-softmax round per wave, one LDS merge of the NW waves (the per-head weights computed once).
// The reduction index of QK^T is split so that the 16-byte K load w of lane (g, c) reads dims 8 (4 w + g) .. + 8 of
// its token row: the four lanes g of a token read 64 contiguous bytes per load (the q operand uses the same
// bijection), which halves the cache lines one K load touches at head_dim 128. Splits, partials, output and the
// RoPE / append behaviour are those of the block kernel.
constexpr int kLeanMaxWaves = 8;

// Arguments in the order the kernel needs them (position, block table and split geometry for the page lookups, then
// the q and K / V pointers), so that the first ones are preloaded into scalar registers at launch.
template <int D, int HPG, bool ROPE, int NW, int NT>
__global__ void __launch_bounds__(NW * kWave)
attn_lean_kernel(const int32_t* __restrict__ pos_ptr, const int32_t* __restrict__ bt, int n_bt, int log2P, int PS,
                 int n_pages, const f16* __restrict__ qsrc, f16* __restrict__ kc, f16* __restrict__ vc, int n_kv,
                 int n_q, int max_splits, float scale, const float* __restrict__ cos_t,
                 const float* __restrict__ sin_t, int max_pos, float* __restrict__ o_part, float* __restrict__ m_part,
                 float* __restrict__ l_part, f16* __restrict__ out) {
  using S = MfmaAttnShape<D>;
  constexpr int KW = S::KW, QS = S::QS, VD = S::VD, CPL = D / 8;
  __shared__ float s_m[NW][HPG], s_l[NW][HPG], s_w[NW][HPG];
  __shared__ float s_o[NW][HPG][D];

  const int kvh = blockIdx.x, split = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, g = lane >> 4;
  const int P = 1 << log2P;
  const long long t0l = (long long)split * PS;
  const bool reachable = t0l < ((long long)n_bt << log2P);
  const int t0 = reachable ? (int)t0l : 0;

  // ---- scalar loads: the position and the page of each of this wave's tiles (independent of the position)
  const int pos = *pos_ptr;
  int pg[NT];
#pragma unroll
  for (int i = 0; i < NT; ++i) {
    const int tl = (wave + NW * i) << 4;  // tile start within the split
    const int lp = (t0 + tl) >> log2P;
    const bool in = reachable && tl < PS && lp < n_bt;
    const int e = bt[in ? lp : 0];
    pg[i] = (in && e >= 0 && e < n_pages) ? e : -1;
  }
  // every other argument into scalar registers now (see above). After the two lookups: an asm statement counts as
  // a possible memory write, and loads after it are no longer issued as scalar loads.
  asm volatile("" ::"s"(qsrc), "s"(cos_t), "s"(sin_t), "s"(max_pos), "s"(kc), "s"(vc), "s"(n_q), "s"(n_kv),
               "s"(max_splits), "s"(scale), "s"(o_part), "s"(m_part), "s"(l_part), "s"(out));
  // ---- q operand (head col of the group, zero for col >= HPG): slice 4 w + g of the head for word group w; for RoPE
  // the partner slices and the new k (same slices) and v (dims VD col ..)
  const bool qlive = col < HPG;
  const f16* qh = qsrc + (size_t)(kvh * HPG + (qlive ? col : 0)) * D;
  u32x4 qr[KW], knew[KW];
  VRow<VD> vnew{};
#pragma unroll
  for (int w = 0; w < KW; ++w) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(qh + 8 * (4 * w + g));
    qr[w] = qlive ? v : u32x4{0u, 0u, 0u, 0u};
    knew[w] = u32x4{0u, 0u, 0u, 0u};
  }
  u32x4 qp[KW], ko[KW], kp[KW];
  if constexpr (ROPE) {
    const f16* kh = qsrc + (size_t)(n_q + kvh) * D;
    const f16* vh = qsrc + (size_t)(n_q + n_kv + kvh) * D;
#pragma unroll
    for (int w = 0; w < KW; ++w) {
      const int c = 4 * w + g, pc = (c + CPL / 2) % CPL;
      qp[w] = *reinterpret_cast<const u32x4*>(qh + 8 * pc);
      ko[w] = *reinterpret_cast<const u32x4*>(kh + 8 * c);
      kp[w] = *reinterpret_cast<const u32x4*>(kh + 8 * pc);
    }
#pragma unroll
    for (int i = 0; i < VD / 2; ++i) vnew.w[i] = reinterpret_cast<const uint32_t*>(vh + VD * col)[i];
  }
  // ---- K / V of every tile of the wave: K row col, V rows 4 g + v (speculative past the context: masked below)
  auto row_off = [&](int page, int t) -> size_t {
    return ((((size_t)page * n_kv + kvh) << log2P) + (t & (P - 1))) * D;
  };
  u32x4 kr[NT][KW];
  VRow<VD> vr[NT][4];
#pragma unroll
  for (int i = 0; i < NT; ++i) {
    const int ts = t0 + ((wave + NW * i) << 4);
    if (pg[i] >= 0) {  // uniform per wave
#pragma unroll
      for (int w = 0; w < KW; ++w)
        kr[i][w] = load_stream(reinterpret_cast<const u32x4*>(kc + row_off(pg[i], ts + col) + 8 * (4 * w + g)));
#pragma unroll
      for (int v = 0; v < 4; ++v) vr[i][v] = load_vrow<VD>(vc + row_off(pg[i], ts + 4 * g + v) + VD * col);
    } else {
#pragma unroll
      for (int w = 0; w < KW; ++w) kr[i][w] = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int v = 0; v < 4; ++v) {
#pragma unroll
        for (int k = 0; k < VD / 2; ++k) vr[i][v].w[k] = 0u;
      }
    }
  }
  if constexpr (ROPE) {
    if (pos < 0 || pos >= max_pos) return;  // uniform: nothing is touched
#pragma unroll
    for (int w = 0; w < KW; ++w) {
      const int c = 4 * w + g;
      const int ti = (8 * c) % (D / 2);
      float cs[8], sn[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        cs[e] = cos_t[(size_t)pos * (D / 2) + ti + e];
        sn[e] = sin_t[(size_t)pos * (D / 2) + ti + e];
      }
      qr[w] = qlive ? rope_slice<D>(qr[w], qp[w], cs, sn, c < CPL / 2) : qr[w];
      knew[w] = rope_slice<D>(ko[w], kp[w], cs, sn, c < CPL / 2);
    }
  }
  const long long cap = (long long)n_bt << log2P;
  const int ctx = (int)((long long)pos + 1 < cap ? (long long)pos + 1 : cap);
  const int nsplit = attn_splits(ctx, PS, max_splits);
  if (ROPE) {
    // the workgroup owning token pos (or the last live split when the cap is below pos) appends k, v
    const int owner = min(pos / PS, nsplit - 1);
    if (split == owner && wave == 0) {
      const int lp = pos >> log2P;
      const int page = lp < n_bt ? bt[lp] : -1;
      if (page >= 0 && page < n_pages) {
        const size_t row = row_off(page, pos);
        if (col == 0) {
#pragma unroll
          for (int w = 0; w < KW; ++w) *reinterpret_cast<u32x4*>(kc + row + 8 * (4 * w + g)) = knew[w];
        }
        if (g == 0) {
#pragma unroll
          for (int i = 0; i < VD / 2; ++i) reinterpret_cast<uint32_t*>(vc + row + VD * col)[i] = vnew.w[i];
        }
      }
    }
  }
  if (split >= nsplit || !reachable) return;  // uniform per workgroup
  const int t1 = (int)min((long long)ctx, t0l + PS);
  const bool pos_here = ROPE && pos >= t0 && pos < t1;  // this split attends token pos (its slot has a page)

  // ---- scores of all the wave's tiles: sc[i][v] = score of token ts_i + 4 g + v for head col
  f4 sc[NT];
  float rmax = -INFINITY;
#pragma unroll
  for (int i = 0; i < NT; ++i) {
    const int ts = t0 + ((wave + NW * i) << 4);
    const bool tile = pg[i] >= 0;
    if constexpr (ROPE) {  // the slot of pos is being written by this launch: use the fresh k, v
      if (pos_here && tile && ts + col == pos) {
#pragma unroll
        for (int w = 0; w < KW; ++w) kr[i][w] = knew[w];
      }
#pragma unroll
      for (int v = 0; v < 4; ++v)
        if (pos_here && tile && ts + 4 * g + v == pos) vr[i][v] = vnew;
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) {  // rows past the context: zero V (a stale row must not reach p . V as NaN)
      const bool keep = tile && ts + 4 * g + v < t1;
#pragma unroll
      for (int k = 0; k < VD / 2; ++k) vr[i][v].w[k] = keep ? vr[i][v].w[k] : 0u;
    }
    f4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < QS; ++q) {
      const int i0 = 2 * q, i1 = 2 * q + 1;
      c = mfma16(as_h4(kr[i][i0 >> 2][i0 & 3], kr[i][i1 >> 2][i1 & 3]), as_h4(qr[i0 >> 2][i0 & 3], qr[i1 >> 2][i1 & 3]),
                 c);
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const bool live = tile && ts + 4 * g + v < t1;
      sc[i][v] = live ? c[v] * scale : -INFINITY;
      rmax = fmaxf(rmax, sc[i][v]);
    }
  }
  // ---- one online-softmax round per wave (m, l of head col; acc rows = heads 4 g + v)
  const float m = rows_max(rmax);
  float ps = 0.f;
#pragma unroll
  for (int i = 0; i < NT; ++i) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float pv = (sc[i][v] == -INFINITY) ? 0.f : __expf(sc[i][v] - m);
      sc[i][v] = pv;
      ps += pv;
    }
  }
  const float l = rows_sum(ps);
  f4 acc[VD];
#pragma unroll
  for (int t = 0; t < VD; ++t) acc[t] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < NT; ++i) {
    h4 phi, plo;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      phi[v] = (f16)sc[i][v];
      plo[v] = (f16)(sc[i][v] - (float)phi[v]);
    }
#pragma unroll
    for (int t = 0; t < VD; ++t) {
      // B operand of dim tile t: dim VD col + t of tokens 4 g + 0..3
      const int wi = t >> 1;
      const uint32_t sel = (t & 1) ? 0x07060302u : 0x05040100u;
      const uint32_t lo = __builtin_amdgcn_perm(vr[i][1].w[wi], vr[i][0].w[wi], sel);
      const uint32_t hi = __builtin_amdgcn_perm(vr[i][3].w[wi], vr[i][2].w[wi], sel);
      const h4 vb = as_h4(lo, hi);
      acc[t] = mfma16(phi, vb, acc[t]);
      acc[t] = mfma16(plo, vb, acc[t]);
    }
  }
  // ---- merge the waves: (m, l) of head col in lanes col < HPG of row 0, O rows = heads 4 g + v
  if (g == 0 && col < HPG) {
    s_m[wave][col] = m;
    s_l[wave][col] = l;
  }
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int hh = 4 * g + v;
    if (hh < HPG) {
#pragma unroll
      for (int t = 0; t < VD; ++t) s_o[wave][hh][VD * col + t] = acc[t][v];
    }
  }
  __syncthreads();
  // per head: M = max over the waves, wave weights e^(m_w - M) (divided by L for a direct output); head hh's M and L
  // go to the partials (thread hh of the loop below keeps them)
  float Mh = -INFINITY, Lh = 0.f;
  if (tid < HPG) {
#pragma unroll
    for (int w = 0; w < NW; ++w) Mh = fmaxf(Mh, s_m[w][tid]);
    float ww[NW];
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      ww[w] = (s_m[w][tid] == -INFINITY) ? 0.f : __expf(s_m[w][tid] - Mh);
      Lh = fmaf(ww[w], s_l[w][tid], Lh);
    }
    const float inv = nsplit == 1 ? (Lh > 0.f ? 1.0f / Lh : 0.f) : 1.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) s_w[w][tid] = ww[w] * inv;
  }
  __syncthreads();
  for (int o = tid; o < HPG * D; o += NW * kWave) {
    const int hh = o / D, d = o % D;
    float O = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) O = fmaf(s_w[w][hh], s_o[w][hh][d], O);
    const int head = kvh * HPG + hh;
    if (nsplit == 1) {
      out[(size_t)head * D + d] = (f16)O;
    } else {
      store_through(o_part + ((size_t)head * max_splits + split) * D + d, O);
    }
  }
  if (nsplit > 1 && tid < HPG) {
    const int head = kvh * HPG + tid;
    store_through(m_part + (size_t)head * max_splits + split, Mh);
    store_through(l_part + (size_t)head * max_splits + split, Lh);
  }
}

// The combine with the smallest batch B in {4, 8, 16} whose B * SLN splits cover max_splits (16 beyond: the kernel
// then loops over batches).
template <int D>
void launch_combine(const AttnLaunch& a, bool rope, hipStream_t st) {
  constexpr int SLN = kAttnThreads / (D / 4);
  const int mp = rope ? a.max_pos : 0;
  if (a.max_splits <= 4 * SLN)
    hipLaunchKernelGGL((attn_combine_kernel<D, 4>), dim3(a.n_q), dim3(kAttnThreads), 0, st, a.o_part, a.m_part,
                       a.l_part, a.pos, mp, a.n_bt, a.log2P, a.part_size, a.max_splits, (f16*)a.out);
  else if (a.max_splits <= 8 * SLN)
    hipLaunchKernelGGL((attn_combine_kernel<D, 8>), dim3(a.n_q), dim3(kAttnThreads), 0, st, a.o_part, a.m_part,
                       a.l_part, a.pos, mp, a.n_bt, a.log2P, a.part_size, a.max_splits, (f16*)a.out);
  else
    hipLaunchKernelGGL((attn_combine_kernel<D, 16>), dim3(a.n_q), dim3(kAttnThreads), 0, st, a.o_part, a.m_part,
                       a.l_part, a.pos, mp, a.n_bt, a.log2P, a.part_size, a.max_splits, (f16*)a.out);
}

template <int D, int HPG, bool ROPE, int NW, int NT>
void launch_lean(const AttnLaunch& a, hipStream_t st) {
  const float scale = 1.0f / sqrtf((float)D);
  hipLaunchKernelGGL((attn_lean_kernel<D, HPG, ROPE, NW, NT>), dim3(a.n_kv, a.max_splits), dim3(NW * kWave), 0, st,
                     a.pos, a.bt, a.n_bt, a.log2P, a.part_size, a.n_pages, (const f16*)a.q, (f16*)a.kc, (f16*)a.vc,
                     a.n_kv, a.n_q, a.max_splits, scale, a.cos_t, a.sin_t, a.max_pos, a.o_part, a.m_part, a.l_part,
                     (f16*)a.out);
}

// waves: the smallest power of two >= min(tiles, 8); tiles per wave NT = ceil(tiles / waves) in {1, 2, 4} (2 at most
// at head_dim 128)
template <int D, int HPG, bool ROPE, int NW>
void launch_lean_nt(const AttnLaunch& a, int nt, hipStream_t st) {
  if (nt == 1) {
    launch_lean<D, HPG, ROPE, NW, 1>(a, st);
  } else if (nt == 2 || D == 128) {
    launch_lean<D, HPG, ROPE, NW, 2>(a, st);
  } else {
    if constexpr (D == 64) launch_lean<D, HPG, ROPE, NW, 4>(a, st);
  }
}

template <int D, int HPG, bool ROPE>
void launch_lean_any(const AttnLaunch& a, hipStream_t st) {
  const int tiles = a.part_size >> 4;
  int waves = 1;
  while (waves < tiles && waves < kLeanMaxWaves) waves <<= 1;
  const int nt = (tiles + waves - 1) / waves;
  switch (waves) {
    case 1: launch_lean_nt<D, HPG, ROPE, 1>(a, nt, st); break;
    case 2: launch_lean_nt<D, HPG, ROPE, 2>(a, nt, st); break;
    case 4: launch_lean_nt<D, HPG, ROPE, 4>(a, nt, st); break;
    default: launch_lean_nt<D, HPG, ROPE, 8>(a, nt, st); break;
  }
}

template <int D, int HPG, bool ROPE>
void launch_attn(const AttnLaunch& a, hipStream_t st) {
  const float scale = 1.0f / sqrtf((float)D);
  if (attn_use_lean(a)) {
    launch_lean_any<D, HPG, ROPE>(a, st);
    if (a.max_splits > 1 && !a.split_only) launch_combine<D>(a, ROPE, st);
    return;
  }
  hipLaunchKernelGGL((attn_decode_kernel<D, HPG, ROPE>), dim3(a.n_kv, a.max_splits), dim3(kAttnThreads), 0,
                     st, (const f16*)a.q, a.cos_t, a.sin_t, a.max_pos, a.pos, a.bt, a.n_bt, (f16*)a.kc, (f16*)a.vc,
                     a.n_pages, a.log2P, a.n_q, a.n_kv, a.part_size, a.max_splits, scale, a.o_part, a.m_part,
                     a.l_part, (f16*)a.out);
  if (a.max_splits > 1 && !a.split_only) launch_combine<D>(a, ROPE, st);
}

template <int D, bool ROPE>
void launch_attn_hpg(const AttnLaunch& a, hipStream_t st) {
  switch (a.n_q / a.n_kv) {
    case 1: launch_attn<D, 1, ROPE>(a, st); break;
    case 2: launch_attn<D, 2, ROPE>(a, st); break;
    case 4: launch_attn<D, 4, ROPE>(a, st); break;
    default: launch_attn<D, 8, ROPE>(a, st); break;
  }
}

// ---------------------------------------------------------------------------------------------------------------
// Prefill attention: causal attention of M prompt rows (row m at position pos + m) over the paged cache, which already
// holds their K / V. A workgroup owns one kv head and QB = 64 / HPG consecutive rows, and runs KVS groups of four
// waves. Wave w of every group has the same 16 MFMA columns, (row, query head) pairs, PW = 16 / HPG rows x HPG heads,
// so every column does work; group h takes the 64-token blocks b with b % KVS == h. The K / V of the tokens
// [0, last row's position] stream through LDS in rounds of KVS blocks (double-buffered, the next rounds' loads in
// flight in registers during the current round's MFMAs), one block per group, read there by the group's four waves.
// With KVS = 2, two waves share each SIMD and each works through half the blocks: the launcher takes it when the grid
// leaves CUs with one workgroup or none, where a lone wave per SIMD waits on its own per-block chain (about 430 vector
// instructions around 48 MFMAs); with more workgroups than CUs the grid fills the SIMDs by itself (KVS = 1).
// Per 16-token tile the math is the MFMA decode kernel's: S^T = K . Q^T (the accumulator is P's A operand as is), the
// causal bound of each column applied to its own scores, online softmax once per block, P . V with p as fp16 hi + lo
// parts and V operands built by byte permutes from 4 token rows. The groups' states (running max, sum, accumulator per
// column) meet in LDS at the end and group 0 merges them in group order. Every column's tokens go to the same group in
// the same order whatever workgroup or batch its row is in (block b to group b % KVS, from token 0), and a block
// wholly past a column's bound changes nothing for it, so a row's result does not depend on how the prompt is
// batched; for a given KVS. The launch's KVS depends on the grid, so the split of a prompt into launches can change it.
constexpr int kPfGroupWaves = 4, kPfBlock = 64, kPfPages = 2048, kPfRing = 2;
// Running maximum of a column that has seen no token yet: a finite stand-in for -infinity, so that exp(max_old -
// max_new) and exp(score - max) never meet -inf - (-inf); exp(-1e30 - x) is 0 for every score x.
constexpr float kPfNoMax = -1e30f;

// Keeps loads where they are written (no sinking to their first use; see the K / V ring below).
__device__ __forceinline__ void pf_fence() { asm volatile("" ::: "memory"); }

template <int D, int HPG, int KVS>
__global__ void __launch_bounds__(kPfGroupWaves * kWave * KVS)
attn_prefill_kernel(const f16* __restrict__ qkv, const int32_t* __restrict__ pos_ptr, const int32_t* __restrict__ bt,
                    int n_bt, const f16* kc, const f16* vc, int n_pages, int log2P, int n_q, int n_kv, int M,
                    int ctx_cap, float scale, f16* __restrict__ out) {
  // (kc, vc without __restrict__: the fences must order their loads)
  using S = MfmaAttnShape<D>;
  constexpr int KD = S::KD, KW = S::KW, QS = S::QS, VD = S::VD;
  constexpr int NTH = kPfGroupWaves * kWave * KVS;       // threads
  constexpr int PW = 16 / HPG;                           // rows per wave
  constexpr int QB = kPfGroupWaves * PW;                 // rows per workgroup
  constexpr int ROW = D + 8;                             // padded LDS row: 16 rows of one K read in distinct banks
  constexpr int CH = D / 8;                              // 16-byte chunks per K / V row
  constexpr int SB = kPfBlock * KVS;                     // tokens per round (one block per group)
  constexpr int LPT = SB * CH / NTH;                     // 16-byte K (and V) loads per thread per round
  constexpr int RPI = NTH / CH;                          // token rows covered per load index
  __shared__ __align__(16) f16 Ks[2][SB][ROW];
  __shared__ __align__(16) f16 Vs[2][SB][ROW];
  __shared__ int s_pg[kPfPages];

  const int kvh = blockIdx.x, qb = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave / kPfGroupWaves, gw = wave % kPfGroupWaves;  // group, and the wave's columns within it
  const int col = lane & 15, g = lane >> 4;
  const int P = 1 << log2P;
  const int pos0 = *pos_ptr;
  // this lane's query column: prompt row m, head h; tokens t <= lim are attended
  const int mw = qb * QB + gw * PW;                      // the wave's first row
  const int m = mw + col / HPG;
  const int h = kvh * HPG + col % HPG;
  const bool live = m < M;
  const int lim = live ? min(pos0 + m, ctx_cap - 1) : -1;  // the cap bounds the mask as well as the loads
  const int mlast = min(qb * QB + QB, M) - 1;
  const int ctx = (int)max(0LL, min((long long)pos0 + mlast + 1, (long long)ctx_cap));  // tokens [0, ctx) are read
  const int npg = (ctx + P - 1) >> log2P;
  const bool staged = npg <= kPfPages;  // uniform: block-table pages in LDS, else read per token from global
  if (staged)
    for (int i = tid; i < npg; i += NTH) s_pg[i] = bt[i];
  u32x4 qr[KW];
  {
    const f16* qh = qkv + (size_t)(live ? m : 0) * (n_q + 2 * n_kv) * D + (size_t)h * D;
#pragma unroll
    for (int w = 0; w < KW; ++w)
      qr[w] = live ? *reinterpret_cast<const u32x4*>(qh + KD * g + 8 * w) : u32x4{0u, 0u, 0u, 0u};
  }
  __syncthreads();  // s_pg

  // K / V ring: round r's loads go into register slot r % kPfRing kPfRing rounds before the round is computed and are
  // staged into LDS buffer r & 1 one round before. Thread: chunk tid % CH of token rows tid / CH + RPI i of the round;
  // tokens past ctx or without a page read page 0's row (every cache has one) and are zeroed by select.
  const int nrnd = (ctx + SB - 1) / SB;
  u32x4 kk[kPfRing][LPT], vv[kPfRing][LPT];
  bool ok[kPfRing][LPT];
  auto fetch = [&](int rnd, int slot) {
    const int b0 = min(rnd, nrnd - 1) * SB;  // past the end: a re-read of the last round, never staged
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      const int t = b0 + tid / CH + RPI * i;
      const int lp = t >> log2P;
      int pg = t < ctx ? (staged ? s_pg[lp] : bt[lp]) : -1;
      if (pg >= n_pages) pg = -1;
      const size_t off =
          ((((size_t)(pg < 0 ? 0 : pg) * n_kv + kvh) << log2P) + (t & (P - 1))) * D + 8 * (tid % CH);
      kk[slot][i] = load_stream(reinterpret_cast<const u32x4*>(kc + off));
      vv[slot][i] = load_stream(reinterpret_cast<const u32x4*>(vc + off));
      ok[slot][i] = pg >= 0;
    }
  };
  auto stage = [&](int buf, int slot) {
    const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      const int r = tid / CH + RPI * i;
      *reinterpret_cast<u32x4*>(&Ks[buf][r][8 * (tid % CH)]) = ok[slot][i] ? kk[slot][i] : z;
      *reinterpret_cast<u32x4*>(&Vs[buf][r][8 * (tid % CH)]) = ok[slot][i] ? vv[slot][i] : z;
    }
  };

  float mrun = kPfNoMax, l = 0.f;
  f4 acc[VD];
#pragma unroll
  for (int t = 0; t < VD; ++t) acc[t] = f4{0.f, 0.f, 0.f, 0.f};

  // the group's block of round rnd (tokens t0 .. t0 + 63, LDS rows r0 .. r0 + 63 of buffer buf)
  auto compute = [&](int t0, int buf) {
    const int r0 = grp * kPfBlock;
    // ---- scores of the block's four 16-token tiles: sc[tt][v] = score of token 16 tt + 4 g + v for column col
    f4 sc[4];
    float rmax = -INFINITY;
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      u32x4 kr[KW];
#pragma unroll
      for (int w = 0; w < KW; ++w)
        kr[w] = *reinterpret_cast<const u32x4*>(&Ks[buf][r0 + 16 * tt + col][KD * g + 8 * w]);
      f4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q = 0; q < QS; ++q) {
        const int i0 = 2 * q, i1 = 2 * q + 1;
        c = mfma16(as_h4(kr[i0 >> 2][i0 & 3], kr[i1 >> 2][i1 & 3]), as_h4(qr[i0 >> 2][i0 & 3], qr[i1 >> 2][i1 & 3]),
                   c);
      }
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int t = t0 + 16 * tt + 4 * g + v;
        sc[tt][v] = t <= lim ? c[v] * scale : -INFINITY;
        rmax = fmaxf(rmax, sc[tt][v]);
      }
    }
    // ---- online softmax, once per block (mrun is finite, so is mn: a masked score gives exp(-inf) = 0)
    rmax = rows_max(rmax);
    const float mn = fmaxf(mrun, rmax);
    const float alpha = __expf(mrun - mn);
    float ps = 0.f;
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float pv = __expf(sc[tt][v] - mn);
        sc[tt][v] = pv;
        ps += pv;
      }
    }
    l = alpha * l + rows_sum(ps);
    mrun = mn;
    // the accumulator's rows are columns 4 g + v: their rescale factors live in lanes 4 g + v
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float av = __shfl(alpha, 4 * g + v, kWave);
#pragma unroll
      for (int t = 0; t < VD; ++t) acc[t][v] *= av;
    }
    // ---- P . V: p as fp16 hi + lo parts; V rows 16 tt + 4 g + v, dims VD col .. VD col + VD - 1
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      h4 phi, plo;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        phi[v] = (f16)sc[tt][v];
        plo[v] = (f16)(sc[tt][v] - (float)phi[v]);
      }
      VRow<VD> vr[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const f16* src = &Vs[buf][r0 + 16 * tt + 4 * g + v][VD * col];
        if constexpr (VD == 4) {
          const u32x2 x = *reinterpret_cast<const u32x2*>(src);
          vr[v].w[0] = x.x;
          vr[v].w[1] = x.y;
        } else {
          const u32x4 x = *reinterpret_cast<const u32x4*>(src);
#pragma unroll
          for (int i = 0; i < 4; ++i) vr[v].w[i] = x[i];
        }
      }
#pragma unroll
      for (int t = 0; t < VD; ++t) {
        const int wi = t >> 1;
        const uint32_t sel = (t & 1) ? 0x07060302u : 0x05040100u;
        const uint32_t lo = __builtin_amdgcn_perm(vr[1].w[wi], vr[0].w[wi], sel);
        const uint32_t hi = __builtin_amdgcn_perm(vr[3].w[wi], vr[2].w[wi], sel);
        const h4 vb = as_h4(lo, hi);
        acc[t] = mfma16(phi, vb, acc[t]);
        acc[t] = mfma16(plo, vb, acc[t]);
      }
    }
  };
  // round rnd (u = rnd % kPfRing, a constant wherever this is called): the group's block from LDS buffer rnd & 1, stage
  // round rnd + 1 from its slot into the other buffer (every wave finished reading it before the last barrier), refill
  // that slot with round rnd + 1 + kPfRing. (Branching around the compute of blocks past the wave's rows, or around the
  // rescale when no maximum moved, measured slower: up to 1.6x at head dim 128.)
  auto step = [&](int rnd, int u) {
    compute((rnd * KVS + grp) * kPfBlock, rnd & 1);
    const int ns = (u + 1) % kPfRing;
    stage((rnd + 1) & 1, ns);  // past the end: a stale slot into an unread buffer
    pf_fence();
    fetch(rnd + 1 + kPfRing, ns);
    pf_fence();
    __syncthreads();
  };
  if (nrnd > 0) {  // uniform
#pragma unroll
    for (int u = 0; u < kPfRing; ++u) {
      fetch(u, u);
      pf_fence();
    }
    stage(0, 0);
    pf_fence();
    fetch(kPfRing, 0);
    pf_fence();
    __syncthreads();
    // whole groups of kPfRing rounds in the loop, the remainder after it (no exit between a group's rounds, which
    // would leave a path where another slot's loads are the newest and the in-order waits drain everything)
    int r0 = 0;
    for (; r0 + kPfRing <= nrnd; r0 += kPfRing) {
#pragma unroll
      for (int u = 0; u < kPfRing; ++u) step(r0 + u, u);
    }
#pragma unroll
    for (int u = 0; u + 1 < kPfRing; ++u)
      if (r0 + u < nrnd) step(r0 + u, u);
  }
  // ---- merge: groups 1 .. KVS - 1 leave max and sum per column and the accumulator per lane in LDS (over the K / V
  // buffers, which every wave has finished reading at the last barrier); group 0 merges them in group order
  static_assert(KVS == 1 || (2 * KVS * kPfGroupWaves * 16 + (KVS - 1) * kPfGroupWaves * kWave * 4 * VD) * 4 <=
                                (int)sizeof(Ks), "merge scratch fits the K buffers");
  float* s_ml = reinterpret_cast<float*>(&Ks[0][0][0]);          // [2][KVS][waves][16]: max, then sum
  float* s_acc = s_ml + 2 * KVS * kPfGroupWaves * 16;           // [KVS - 1][waves][lanes][VD][4]
  if constexpr (KVS > 1) {
    if (g == 0) {
      s_ml[(grp * kPfGroupWaves + gw) * 16 + col] = mrun;
      s_ml[((KVS + grp) * kPfGroupWaves + gw) * 16 + col] = l;
    }
    if (grp > 0) {
      f4* dst = reinterpret_cast<f4*>(s_acc) + (((grp - 1) * kPfGroupWaves + gw) * kWave + lane) * VD;
#pragma unroll
      for (int t = 0; t < VD; ++t) dst[t] = acc[t];
    }
    __syncthreads();
    if (grp > 0) return;  // uniform per wave; no barrier follows
  }
  // ---- output: acc[t][v] = O[column 4 g + v][dim VD col + t]
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int cc = 4 * g + v;
    float inv;
    if constexpr (KVS == 1) {
      const float lv = __shfl(l, cc, kWave);  // the column's sum lives in lane 4 g + v
      inv = lv > 0.f ? 1.0f / lv : 0.f;
    } else {
      float mx = kPfNoMax;
#pragma unroll
      for (int hh = 0; hh < KVS; ++hh) mx = fmaxf(mx, s_ml[(hh * kPfGroupWaves + gw) * 16 + cc]);
      float wg[KVS], tot = 0.f;  // group hh's weight exp(m_hh - max) (0 for a group that saw no token)
#pragma unroll
      for (int hh = 0; hh < KVS; ++hh) {
        wg[hh] = __expf(s_ml[(hh * kPfGroupWaves + gw) * 16 + cc] - mx);
        tot = fmaf(wg[hh], s_ml[((KVS + hh) * kPfGroupWaves + gw) * 16 + cc], tot);
      }
      inv = tot > 0.f ? 1.0f / tot : 0.f;
#pragma unroll
      for (int t = 0; t < VD; ++t) {
        float o = wg[0] * acc[t][v];
#pragma unroll
        for (int hh = 1; hh < KVS; ++hh)
          o = fmaf(wg[hh], s_acc[((((hh - 1) * kPfGroupWaves + gw) * kWave + lane) * VD + t) * 4 + v], o);
        acc[t][v] = o;
      }
    }
    const int mm = mw + cc / HPG, hh = kvh * HPG + cc % HPG;
    if (mm < M) {
      f16* dst = out + (size_t)mm * n_q * D + (size_t)hh * D + VD * col;
#pragma unroll
      for (int t = 0; t < VD; ++t) dst[t] = (f16)(acc[t][v] * inv);
    }
  }
}

// Grids of at most this many workgroups (one round of the 256 CUs) run two wave groups per workgroup (KVS = 2).
constexpr int kPfSplitGrid = 256;

template <int D>
void launch_prefill_hpg(const void* qkv, const int32_t* pos, const int32_t* bt, int n_bt, const void* kc,
                        const void* vc, int n_pages, int log2P, int n_q, int n_kv, int M, int max_ctx, void* out,
                        hipStream_t st) {
  const float scale = 1.0f / sqrtf((float)D);
  const int cap = (int)min((long long)max_ctx, (long long)n_bt << log2P);
#define DK_PREFILL_KVS(H, KVS)                                                                                      \
  hipLaunchKernelGGL((attn_prefill_kernel<D, H, KVS>), dim3(n_kv, rb), dim3(kPfGroupWaves * kWave * KVS), 0, st,  \
                     (const f16*)qkv, pos, bt, n_bt, (const f16*)kc, (const f16*)vc, n_pages, log2P, n_q, n_kv, M, cap, \
                     scale, (f16*)out)
#define DK_PREFILL(H)                                                                                               \
  {                                                                                                                 \
    const int rb = (M + kPfGroupWaves * (16 / H) - 1) / (kPfGroupWaves * (16 / H));                                 \
    if ((long long)n_kv * rb <= kPfSplitGrid)                                                                       \
      DK_PREFILL_KVS(H, 2);                                                                                         \
    else                                                                                                            \
      DK_PREFILL_KVS(H, 1);                                                                                         \
  }
  switch (n_q / n_kv) {
    case 1: DK_PREFILL(1); break;
    case 2: DK_PREFILL(2); break;
    case 4: DK_PREFILL(4); break;
    default: DK_PREFILL(8); break;
  }
#undef DK_PREFILL
#undef DK_PREFILL_KVS
}

}  // namespace

void launch_attention_prefill(const void* qkv, const int32_t* pos, const int32_t* bt, int n_bt, const void* kc,
                              const void* vc, int n_pages, int log2P, int n_q, int n_kv, int head_dim, int M,
                              int max_ctx, void* out, hipStream_t st) {
  if (head_dim == 64)
    launch_prefill_hpg<64>(qkv, pos, bt, n_bt, kc, vc, n_pages, log2P, n_q, n_kv, M, max_ctx, out, st);
  else
    launch_prefill_hpg<128>(qkv, pos, bt, n_bt, kc, vc, n_pages, log2P, n_q, n_kv, M, max_ctx, out, st);
}

void launch_paged_attention(const AttnLaunch& a, hipStream_t st) {
  if (a.head_dim == 64)
    launch_attn_hpg<64, false>(a, st);
  else
    launch_attn_hpg<128, false>(a, st);
}

void launch_attention_decode(const AttnLaunch& a, hipStream_t st) {
  if (a.head_dim == 64)
    launch_attn_hpg<64, true>(a, st);
  else
    launch_attn_hpg<128, true>(a, st);
}

}  // namespace dk
