// Paged split-K GQA decode attention (one query token) on gfx950.
//
// Cache layout (runtime/model.py:117-120 of the reference): kc / vc fp16 [pages, n_kv, P, D]; token t of the
// sequence lives in physical page bt[t / P], slot t % P, so one (page, kv head) holds P contiguous D-vectors.
// Context = *pos + 1 read from device memory, so one captured graph serves every decode step.
//
// Grid (n_kv, max_splits); workgroup (kvh, s) = 4 waves owns tokens [s*PS, min(ctx, (s+1)*PS)) for all HPG query
// heads of kv head kvh, so every K/V byte is read from HBM once. Splits past the live count exit.
//
// Lane map (wave64): CPL = D/8 lanes hold one token row (16 B each), so a wave load covers TPL = 64/CPL consecutive
// tokens (8 at D = 64, 4 at D = 128) = 1 KB contiguous inside a page. Each wave walks its own chunks of
// CH = 2*TPL tokens (chunks interleaved across the 4 waves) and keeps its own online-softmax state:
//     m' = max(m, chunk max);  a = e^(m - m');  l' = a l + sum e^(s - m');  o' = a o + sum e^(s - m') v
// Scores reduce over the CPL lanes of a row; the chunk max reduces over the token lanes. l and o stay per-lane
// partials over the lane's tokens (all CPL lanes of a token see the same p) until one cross-lane reduction at the
// end; the 4 waves then merge through LDS with the same max-rescale rule. With one live split the normalised output
// is written directly; otherwise each split writes unnormalized o and its (m, l), and the combine kernel computes
//     M = max_s m_s;  L = sum_s e^(m_s - M) l_s;  O = sum_s e^(m_s - M) o_s / L.
// Scores are fp32 with q pre-scaled by 1/sqrt(D) in fp32.
#include "common.hpp"
#include "launch.hpp"

namespace dk {
namespace {

constexpr int kAttnWaves = 4;

__device__ __forceinline__ int live_context(const int32_t* pos_ptr, int n_bt, int log2P) {
  const long long cap = (long long)n_bt << log2P;
  const long long ctx = (long long)(*pos_ptr) + 1;
  return (int)(ctx < cap ? ctx : cap);
}

__device__ __forceinline__ int live_splits(int ctx, int PS, int max_splits) {
  if (ctx <= 0) return 0;
  const int n = (ctx + PS - 1) / PS;
  return n < max_splits ? n : max_splits;
}

template <int D, int HPG>
__global__ void __launch_bounds__(256)
attn_split_kernel(const f16* __restrict__ q, const f16* __restrict__ kc, const f16* __restrict__ vc,
                  const int32_t* __restrict__ bt, const int32_t* __restrict__ pos_ptr, int n_kv, int log2P,
                  int n_pages, int n_bt, int PS, int max_splits, float scale, float* __restrict__ o_part,
                  float* __restrict__ m_part, float* __restrict__ l_part, f16* __restrict__ out) {
  constexpr int NW = kAttnWaves;
  constexpr int CPL = D / 8;
  constexpr int TPL = kWave / CPL;
  constexpr int SL = 2;
  constexpr int CH = TPL * SL;
  __shared__ float red[NW][HPG][D];
  __shared__ float wm[NW][HPG], wl[NW][HPG];

  const int kvh = blockIdx.x, split = blockIdx.y;
  const int ctx = live_context(pos_ptr, n_bt, log2P);
  const int nsplit = live_splits(ctx, PS, max_splits);
  if (split >= nsplit) return;
  const int t0 = split * PS;
  const int t1 = min(ctx, t0 + PS);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int g = lane / CPL, c = lane % CPL;
  const int P = 1 << log2P;

  float qv[HPG][8];
#pragma unroll
  for (int h = 0; h < HPG; ++h) {
    const u32x4 raw = *reinterpret_cast<const u32x4*>(q + (size_t)(kvh * HPG + h) * D + c * 8);
    unpack8(raw, qv[h]);
#pragma unroll
    for (int e = 0; e < 8; ++e) qv[h][e] *= scale;
  }

  float m[HPG], l[HPG], acc[HPG][8];
#pragma unroll
  for (int h = 0; h < HPG; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[h][e] = 0.f;
  }

  for (int cs = t0 + wave * CH; cs < t1; cs += NW * CH) {
    u32x4 kr[SL], vr[SL];
    bool ok[SL];
#pragma unroll
    for (int j = 0; j < SL; ++j) {
      const int t = cs + j * TPL + g;
      bool live = t < t1;
      int page = 0;
      if (live) {
        page = bt[t >> log2P];
        live = page >= 0 && page < n_pages;
      }
      ok[j] = live;
      if (live) {
        const size_t base = ((((size_t)page * n_kv + kvh) << log2P) + (t & (P - 1))) * D + c * 8;
        kr[j] = load_stream(reinterpret_cast<const u32x4*>(kc + base));
        vr[j] = load_stream(reinterpret_cast<const u32x4*>(vc + base));
      } else {
        kr[j] = u32x4{0u, 0u, 0u, 0u};
        vr[j] = kr[j];
      }
    }
    float s[SL][HPG];
#pragma unroll
    for (int j = 0; j < SL; ++j) {
      float kf[8];
      unpack8(kr[j], kf);
#pragma unroll
      for (int h = 0; h < HPG; ++h) {
        float a = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) a = fmaf(kf[e], qv[h][e], a);
        a = group_sum<CPL>(a);
        s[j][h] = ok[j] ? a : -INFINITY;
      }
    }
#pragma unroll
    for (int h = 0; h < HPG; ++h) {
      float cm = s[0][h];
#pragma unroll
      for (int j = 1; j < SL; ++j) cm = fmaxf(cm, s[j][h]);
      cm = strided_max<CPL>(cm);
      const float mn = fmaxf(m[h], cm);
      const float al = (mn == -INFINITY) ? 1.f : __expf(m[h] - mn);
      m[h] = mn;
      l[h] *= al;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[h][e] *= al;
    }
#pragma unroll
    for (int j = 0; j < SL; ++j) {
      float vf[8];
      unpack8(vr[j], vf);
#pragma unroll
      for (int h = 0; h < HPG; ++h) {
        const float p = ok[j] ? __expf(s[j][h] - m[h]) : 0.f;
        l[h] += p;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[h][e] = fmaf(p, vf[e], acc[h][e]);
      }
    }
  }

  // per-lane partials -> per-wave totals (reduce over the TPL token lanes that share c)
#pragma unroll
  for (int h = 0; h < HPG; ++h) {
    l[h] = strided_sum<CPL>(l[h]);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[h][e] = strided_sum<CPL>(acc[h][e]);
  }
  if (g == 0) {
#pragma unroll
    for (int h = 0; h < HPG; ++h)
#pragma unroll
      for (int e = 0; e < 8; ++e) red[wave][h][c * 8 + e] = acc[h][e];
  }
  if (lane == 0) {
#pragma unroll
    for (int h = 0; h < HPG; ++h) {
      wm[wave][h] = m[h];
      wl[wave][h] = l[h];
    }
  }
  __syncthreads();
  for (int i = tid; i < HPG * D; i += NW * kWave) {
    const int h = i / D, d = i % D, head = kvh * HPG + h;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, wm[w][h]);
    float o = 0.f, L = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float a = (wm[w][h] == -INFINITY) ? 0.f : __expf(wm[w][h] - M);
      o = fmaf(a, red[w][h][d], o);
      L = fmaf(a, wl[w][h], L);
    }
    if (nsplit == 1) {
      out[(size_t)head * D + d] = (f16)(L > 0.f ? o / L : 0.f);
    } else {
      o_part[((size_t)head * max_splits + split) * D + d] = o;
      if (d == 0) {
        m_part[(size_t)head * max_splits + split] = M;
        l_part[(size_t)head * max_splits + split] = L;
      }
    }
  }
}

// One workgroup per query head; 256 threads = 256/D split lanes x D dims.
template <int D>
__global__ void __launch_bounds__(256)
attn_combine_kernel(const float* __restrict__ o_part, const float* __restrict__ m_part,
                    const float* __restrict__ l_part, const int32_t* __restrict__ pos_ptr, int n_bt, int log2P,
                    int PS, int max_splits, f16* __restrict__ out) {
  constexpr int NT = 256, NWV = NT / kWave, SLN = NT / D;
  __shared__ float sred[NWV];
  __shared__ float osum[SLN][D];
  const int head = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nsplit = live_splits(live_context(pos_ptr, n_bt, log2P), PS, max_splits);
  if (nsplit <= 1) return;
  const float* m = m_part + (size_t)head * max_splits;
  const float* l = l_part + (size_t)head * max_splits;

  float mx = -INFINITY;
  for (int s = tid; s < nsplit; s += NT) mx = fmaxf(mx, m[s]);
  mx = group_max<kWave>(mx);
  if (lane == 0) sred[wave] = mx;
  __syncthreads();
  float M = sred[0];
#pragma unroll
  for (int w = 1; w < NWV; ++w) M = fmaxf(M, sred[w]);
  __syncthreads();

  float L = 0.f;
  for (int s = tid; s < nsplit; s += NT)
    if (m[s] != -INFINITY) L = fmaf(__expf(m[s] - M), l[s], L);
  L = group_sum<kWave>(L);
  if (lane == 0) sred[wave] = L;
  __syncthreads();
  L = 0.f;
#pragma unroll
  for (int w = 0; w < NWV; ++w) L += sred[w];

  const int d = tid % D, sl = tid / D;
  const float* op = o_part + (size_t)head * max_splits * D + d;
  float o = 0.f;
  for (int s = sl; s < nsplit; s += SLN)
    if (m[s] != -INFINITY) o = fmaf(__expf(m[s] - M), op[(size_t)s * D], o);
  osum[sl][d] = o;
  __syncthreads();
  if (tid < D) {
    float v = 0.f;
#pragma unroll
    for (int i = 0; i < SLN; ++i) v += osum[i][tid];
    out[(size_t)head * D + tid] = (f16)(L > 0.f ? v / L : 0.f);
  }
}

template <int D, int HPG>
void launch_split(const void* q, const void* kc, const void* vc, const int32_t* bt, const int32_t* pos, int n_kv,
                  int log2P, int n_pages, int n_bt, int PS, int max_splits, float* o_part, float* m_part,
                  float* l_part, void* out, hipStream_t st) {
  const float scale = 1.0f / sqrtf((float)D);
  hipLaunchKernelGGL((attn_split_kernel<D, HPG>), dim3(n_kv, max_splits), dim3(kAttnWaves * kWave), 0, st,
                     (const f16*)q, (const f16*)kc, (const f16*)vc, bt, pos, n_kv, log2P, n_pages, n_bt, PS,
                     max_splits, scale, o_part, m_part, l_part, (f16*)out);
}

template <int D>
void launch_d(int hpg, const void* q, const void* kc, const void* vc, const int32_t* bt, const int32_t* pos, int n_q,
              int n_kv, int log2P, int n_pages, int n_bt, int PS, int max_splits, float* o_part, float* m_part,
              float* l_part, void* out, hipStream_t st) {
  switch (hpg) {
    case 1: launch_split<D, 1>(q, kc, vc, bt, pos, n_kv, log2P, n_pages, n_bt, PS, max_splits, o_part, m_part, l_part, out, st); break;
    case 2: launch_split<D, 2>(q, kc, vc, bt, pos, n_kv, log2P, n_pages, n_bt, PS, max_splits, o_part, m_part, l_part, out, st); break;
    case 4: launch_split<D, 4>(q, kc, vc, bt, pos, n_kv, log2P, n_pages, n_bt, PS, max_splits, o_part, m_part, l_part, out, st); break;
    default: launch_split<D, 8>(q, kc, vc, bt, pos, n_kv, log2P, n_pages, n_bt, PS, max_splits, o_part, m_part, l_part, out, st); break;
  }
  if (max_splits > 1)
    hipLaunchKernelGGL((attn_combine_kernel<D>), dim3(n_q), dim3(256), 0, st, o_part, m_part, l_part, pos, n_bt,
                       log2P, PS, max_splits, (f16*)out);
}

}  // namespace

void launch_paged_attention(const void* q, const void* kc, const void* vc, const int32_t* bt, const int32_t* pos,
                            int n_q, int n_kv, int head_dim, int log2P, int n_pages, int n_bt, int part_size,
                            int max_splits, float* o_part, float* m_part, float* l_part, void* out, hipStream_t st) {
  const int hpg = n_q / n_kv;
  if (head_dim == 64)
    launch_d<64>(hpg, q, kc, vc, bt, pos, n_q, n_kv, log2P, n_pages, n_bt, part_size, max_splits, o_part, m_part,
                 l_part, out, st);
  else
    launch_d<128>(hpg, q, kc, vc, bt, pos, n_q, n_kv, log2P, n_pages, n_bt, part_size, max_splits, o_part, m_part,
                  l_part, out, st);
}

}  // namespace dk
