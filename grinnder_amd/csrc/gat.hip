// GAT attention for gfx950: SDDMM logits, edge softmax and attention-weighted
// aggregation (forward), and the fused softmax/SDDMM gradient (backward).
//
// Semantics follow PyG GATConv as the reference uses it (grinnder/nn/gat.py:
// 54-61,69-78: bipartite input (x, x[:B]), add_self_loops=False, attention
// dropout 0, LeakyReLU slope 0.2, softmax denominator + 1e-16).  Heads H,
// channels C per head, features laid out [row, H*C].
//
//   s[j,h] = <Hs[j,h,:], att_src[h,:]>       j < E (source rows)
//   d[i,h] = <Hs[i,h,:], att_dst[h,:]>       i < B (destination rows)
//   t = s[j] + d[i];  v = LeakyReLU(t);  m[i] = max_j v;
//   den[i] = sum_j exp(v - m[i]) + 1e-16;  alpha = exp(v - m[i]) / den[i]
//   O[i] = sum_j alpha_ij Hs[j]
//
// Work decomposition mirrors the GCN aggregation: one wavefront per plan
// unit (row, edge range, slot); rows longer than the plan's segment length
// are reduced by an ordered fixup pass, so results are deterministic.
#include <cfloat>

#include "gr_internal.h"

namespace gr_gat {

constexpr int kMaxHeads = 16;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

__device__ __forceinline__ float leaky(float t) { return t > 0.f ? t : 0.2f * t; }

__device__ __forceinline__ int64_t wave_id() {
  return (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
}

template <int VEC>
__device__ __forceinline__ void ld(const float* __restrict__ p, float (&r)[VEC]) {
  if constexpr (VEC == 4) {
    const float4 t = *reinterpret_cast<const float4*>(p);
    r[0] = t.x; r[1] = t.y; r[2] = t.z; r[3] = t.w;
  } else {
    r[0] = *p;
  }
}

template <int VEC>
__device__ __forceinline__ void st(float* __restrict__ p, const float (&r)[VEC]) {
  if constexpr (VEC == 4) {
    *reinterpret_cast<float4*>(p) = make_float4(r[0], r[1], r[2], r[3]);
  } else {
    *p = r[0];
  }
}

// ------------------------------------------------------------- scores --

// One wavefront per source row j: s[j,:] and, for j < B, d[j,:].
__global__ __launch_bounds__(256) void gat_scores_kernel(const float* __restrict__ hs, int64_t ldh,
                                                         int64_t n_src, int64_t n_dst, int H,
                                                         int C, const float* __restrict__ att_src,
                                                         const float* __restrict__ att_dst,
                                                         float* __restrict__ s,
                                                         float* __restrict__ d) {
  const int lane = threadIdx.x & 63;
  const int64_t j = wave_id();
  if (j >= n_src) return;
  const float* row = hs + j * ldh;
  const bool is_dst = j < n_dst;
  for (int h = 0; h < H; ++h) {
    float ps = 0.f, pd = 0.f;
    for (int c = lane; c < C; c += 64) {
      const float x = row[h * C + c];
      ps = fmaf(x, att_src[h * C + c], ps);
      if (is_dst) pd = fmaf(x, att_dst[h * C + c], pd);
    }
    ps = wave_sum(ps);
    pd = wave_sum(pd);
    if (lane == 0) {
      s[j * H + h] = ps;
      if (is_dst) d[j * H + h] = pd;
    }
  }
}

// ------------------------------------------------------ softmax stats --

// Per unit: m = max_e v_e and sum_e exp(v_e - m) for each head (two passes
// over the unit's edges, lanes parallel over edges).  Unsplit rows write
// m[i,h] and den[i,h] = sum + 1e-16; split rows write (m_k, sum_k) partials.
__global__ __launch_bounds__(256) void gat_stats_kernel(const int4* __restrict__ units,
                                                        int64_t n_units,
                                                        const int32_t* __restrict__ idx,
                                                        const float* __restrict__ s,
                                                        const float* __restrict__ d, int H,
                                                        float* __restrict__ m,
                                                        float* __restrict__ den,
                                                        float* __restrict__ ws) {
  const int lane = threadIdx.x & 63;
  const int64_t wid = wave_id();
  if (wid >= n_units) return;
  const int4 w = units[wid];
  const int i = w.x;
  for (int h = 0; h < H; ++h) {
    const float di = d[(int64_t)i * H + h];
    float mx = -FLT_MAX;
    for (int e = w.y + lane; e < w.z; e += 64) {
      const float v = leaky(s[(int64_t)idx[e] * H + h] + di);
      mx = fmaxf(mx, v);
    }
    mx = wave_max(mx);
    float sum = 0.f;
    for (int e = w.y + lane; e < w.z; e += 64) {
      const float v = leaky(s[(int64_t)idx[e] * H + h] + di);
      sum += expf(v - mx);
    }
    sum = wave_sum(sum);
    if (lane == 0) {
      if (w.w < 0) {
        const bool empty = w.z <= w.y;
        m[(int64_t)i * H + h] = empty ? 0.f : mx;
        den[(int64_t)i * H + h] = empty ? 1.f : sum + 1e-16f;
      } else {
        ws[(int64_t)w.w * 2 * H + h] = mx;
        ws[(int64_t)w.w * 2 * H + H + h] = sum;
      }
    }
  }
}

// Split rows: m = max_k m_k, den = sum_k sum_k * exp(m_k - m) + 1e-16, in
// slot order.
__global__ __launch_bounds__(256) void gat_stats_fixup(const int32_t* __restrict__ fix,
                                                       int64_t n_fix, const float* __restrict__ ws,
                                                       int H, float* __restrict__ m,
                                                       float* __restrict__ den) {
  const int lane = threadIdx.x & 63;
  const int64_t wid = wave_id();
  if (wid >= n_fix) return;
  const int row = fix[3 * wid + 0], first = fix[3 * wid + 1], n = fix[3 * wid + 2];
  for (int h = lane; h < H; h += 64) {
    float mx = -FLT_MAX;
    for (int k = 0; k < n; ++k) mx = fmaxf(mx, ws[(int64_t)(first + k) * 2 * H + h]);
    float sum = 0.f;
    for (int k = 0; k < n; ++k) {
      const float* p = ws + (int64_t)(first + k) * 2 * H;
      sum += p[H + h] * expf(p[h] - mx);
    }
    m[(int64_t)row * H + h] = mx;
    den[(int64_t)row * H + h] = sum + 1e-16f;
  }
}

// ---------------------------------------------------------- aggregate --

// O[i,:] = sum_e alpha_e Hs[col_e,:]; alpha recomputed from (s, d, m, den).
// Writes O (no bias) and, if y != NULL, Y = O + bias.
template <int VEC, int NCH, int U>
__global__ __launch_bounds__(256) void gat_aggregate_kernel(
    const int4* __restrict__ units, int64_t n_units, const int32_t* __restrict__ idx,
    const float* __restrict__ hs, int64_t ldh, const float* __restrict__ s,
    const float* __restrict__ d, const float* __restrict__ m, const float* __restrict__ den,
    int H, int C, const float* __restrict__ bias, float* __restrict__ o,
    float* __restrict__ y, int64_t ldy, float* __restrict__ ws) {
  const int lane = threadIdx.x & 63;
  const int64_t wid = wave_id();
  if (wid >= n_units) return;
  const int4 w = units[wid];
  const int HC = H * C;
  const int64_t i = w.x;

  int foff[NCH], fld[NCH], hd[NCH];
  bool fvalid[NCH];
  float dh[NCH], mh[NCH], rden[NCH];
#pragma unroll
  for (int ch = 0; ch < NCH; ++ch) {
    foff[ch] = (ch * 64 + lane) * VEC;
    fvalid[ch] = foff[ch] < HC;
    fld[ch] = fvalid[ch] ? foff[ch] : HC - VEC;
    hd[ch] = fld[ch] / C;
    dh[ch] = d[i * H + hd[ch]];
    mh[ch] = m[i * H + hd[ch]];
    rden[ch] = den[i * H + hd[ch]];
  }
  float acc[NCH][VEC];
#pragma unroll
  for (int ch = 0; ch < NCH; ++ch)
#pragma unroll
    for (int j = 0; j < VEC; ++j) acc[ch][j] = 0.f;

  int e = w.y;
  const int end = w.z;
  for (; e < end; e += U) {
    int c[U];
    bool ok[U];
#pragma unroll
    for (int k = 0; k < U; ++k) {
      ok[k] = e + k < end;
      c[k] = ok[k] ? idx[e + k] : idx[e];
    }
    float r[U][NCH][VEC];
    float sv[U][NCH];
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const float* row = hs + (int64_t)c[k] * ldh;
#pragma unroll
      for (int ch = 0; ch < NCH; ++ch) {
        ld<VEC>(row + fld[ch], r[k][ch]);
        sv[k][ch] = s[(int64_t)c[k] * H + hd[ch]];
      }
    }
#pragma unroll
    for (int k = 0; k < U; ++k) {
#pragma unroll
      for (int ch = 0; ch < NCH; ++ch) {
        const float a = ok[k] ? expf(leaky(sv[k][ch] + dh[ch]) - mh[ch]) / rden[ch] : 0.f;
#pragma unroll
        for (int j = 0; j < VEC; ++j) acc[ch][j] = fmaf(a, r[k][ch][j], acc[ch][j]);
      }
    }
  }

  if (w.w < 0) {
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) {
      if (!fvalid[ch]) continue;
      st<VEC>(o + i * HC + foff[ch], acc[ch]);
      if (y != nullptr) {
        float b[VEC];
        if (bias != nullptr) {
          ld<VEC>(bias + foff[ch], b);
        } else {
#pragma unroll
          for (int j = 0; j < VEC; ++j) b[j] = 0.f;
        }
#pragma unroll
        for (int j = 0; j < VEC; ++j) b[j] += acc[ch][j];
        st<VEC>(y + i * ldy + foff[ch], b);
      }
    }
  } else {
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch)
      if (fvalid[ch]) st<VEC>(ws + (int64_t)w.w * HC + foff[ch], acc[ch]);
  }
}

__global__ __launch_bounds__(256) void gat_aggregate_fixup(const int32_t* __restrict__ fix,
                                                           int64_t n_fix,
                                                           const float* __restrict__ ws, int HC,
                                                           const float* __restrict__ bias,
                                                           float* __restrict__ o,
                                                           float* __restrict__ y, int64_t ldy) {
  const int lane = threadIdx.x & 63;
  const int64_t wid = wave_id();
  if (wid >= n_fix) return;
  const int row = fix[3 * wid + 0], first = fix[3 * wid + 1], n = fix[3 * wid + 2];
  for (int f = lane; f < HC; f += 64) {
    float acc = 0.f;
    for (int k = 0; k < n; ++k) acc += ws[(int64_t)(first + k) * HC + f];
    o[(int64_t)row * HC + f] = acc;
    if (y != nullptr) y[(int64_t)row * ldy + f] = acc + (bias != nullptr ? bias[f] : 0.f);
  }
}

// ----------------------------------------------------------- backward --

// Column-parallel (CSC) pass over source rows j.  For each edge (i, j):
//   alpha = exp(LeakyReLU(s_j + d_i) - m_i) / den_i
//   g_alpha = <GO_i, Hs_j>  (per head);  g_e = alpha (g_alpha - c_i)
//   g_t = g_e * (t > 0 ? 1 : 0.2)
//   dHs_j += alpha GO_i;  ds_j += g_t;  gdd[csr position of e] = g_e * (t > 0 ? 0 : -0.8)
// and finally dHs_j += ds_j * att_src.  c_i = <GO_i, O_i> per head equals
// sum_k alpha_ik g_alpha_ik.
//
// gdd feeds dd_i = sum_j g_t,ij.  Softmax is invariant to a shift of row i's
// logits, so sum_j g_e,ij = c_i (1 - sum_j alpha_ij) = c_i * 1e-16 / den_i
// exactly; summing g_t directly would cancel to fp32 noise.  The destination
// pass therefore forms dd_i = sum_j g_e,ij (slope_ij - 1) + c_i * 1e-16 / den_i,
// the same value without the cancellation.
template <int VEC, int NCH, int U>
__global__ __launch_bounds__(256) void gat_bwd_src_kernel(
    const int4* __restrict__ units, int64_t n_units, const int32_t* __restrict__ row_idx,
    const int32_t* __restrict__ perm, const float* __restrict__ hs, int64_t ldh,
    const float* __restrict__ go, const float* __restrict__ s, const float* __restrict__ d,
    const float* __restrict__ m, const float* __restrict__ den, const float* __restrict__ cdot,
    const float* __restrict__ att_src, int H, int C, float* __restrict__ dhs,
    float* __restrict__ ds, float* __restrict__ gt, float* __restrict__ ws) {
  const int lane = threadIdx.x & 63;
  const int64_t wid = wave_id();
  if (wid >= n_units) return;
  const int4 w = units[wid];
  const int HC = H * C;
  const int64_t j = w.x;

  int foff[NCH], fld[NCH], hd[NCH];
  bool fvalid[NCH], head_lead[NCH];
  float hsj[NCH][VEC], sj[NCH];
#pragma unroll
  for (int ch = 0; ch < NCH; ++ch) {
    foff[ch] = (ch * 64 + lane) * VEC;
    fvalid[ch] = foff[ch] < HC;
    fld[ch] = fvalid[ch] ? foff[ch] : HC - VEC;
    hd[ch] = fld[ch] / C;
    head_lead[ch] = fvalid[ch] && (foff[ch] == hd[ch] * C);
    ld<VEC>(hs + j * ldh + fld[ch], hsj[ch]);
    if (!fvalid[ch]) {
#pragma unroll
      for (int q = 0; q < VEC; ++q) hsj[ch][q] = 0.f;
    }
    sj[ch] = s[j * H + hd[ch]];
  }
  float acc[NCH][VEC];
  float dsl[NCH];
#pragma unroll
  for (int ch = 0; ch < NCH; ++ch) {
    dsl[ch] = 0.f;
#pragma unroll
    for (int q = 0; q < VEC; ++q) acc[ch][q] = 0.f;
  }

  for (int e = w.y; e < w.z; e += U) {
    int ii[U];
    bool ok[U];
#pragma unroll
    for (int k = 0; k < U; ++k) {
      ok[k] = e + k < w.z;
      ii[k] = ok[k] ? row_idx[e + k] : row_idx[e];
    }
    float g[U][NCH][VEC];
#pragma unroll
    for (int k = 0; k < U; ++k)
#pragma unroll
      for (int ch = 0; ch < NCH; ++ch) ld<VEC>(go + (int64_t)ii[k] * HC + fld[ch], g[k][ch]);
#pragma unroll
    for (int k = 0; k < U; ++k) {
      // Per-lane partial dot products, then one wave reduction per head.
      float pd[NCH];
#pragma unroll
      for (int ch = 0; ch < NCH; ++ch) {
        float t = 0.f;
#pragma unroll
        for (int q = 0; q < VEC; ++q) t = fmaf(g[k][ch][q], hsj[ch][q], t);
        pd[ch] = t;
      }
      float ga[NCH];
      if (H == 1) {
        float t = 0.f;
#pragma unroll
        for (int ch = 0; ch < NCH; ++ch) t += pd[ch];
        t = wave_sum(t);
#pragma unroll
        for (int ch = 0; ch < NCH; ++ch) ga[ch] = t;
      } else {
#pragma unroll
        for (int ch = 0; ch < NCH; ++ch) ga[ch] = 0.f;
        for (int h = 0; h < H; ++h) {
          float t = 0.f;
#pragma unroll
          for (int ch = 0; ch < NCH; ++ch) t += (hd[ch] == h && fvalid[ch]) ? pd[ch] : 0.f;
          t = wave_sum(t);
#pragma unroll
          for (int ch = 0; ch < NCH; ++ch)
            if (hd[ch] == h) ga[ch] = t;
        }
      }
      const int64_t i = ii[k];
#pragma unroll
      for (int ch = 0; ch < NCH; ++ch) {
        const int64_t ih = i * H + hd[ch];
        const float tt = sj[ch] + d[ih];
        const float a = expf(leaky(tt) - m[ih]) / den[ih];
        const float ge = a * (ga[ch] - cdot[ih]);
        const bool pos = tt > 0.f;
        if (ok[k]) {
          dsl[ch] += pos ? ge : 0.2f * ge;
#pragma unroll
          for (int q = 0; q < VEC; ++q) acc[ch][q] = fmaf(a, g[k][ch][q], acc[ch][q]);
          if (head_lead[ch]) gt[(int64_t)perm[e + k] * H + hd[ch]] = pos ? 0.f : -0.8f * ge;
        }
      }
    }
  }

  if (w.w < 0) {
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) {
      if (!fvalid[ch]) continue;
      float a[VEC];
      ld<VEC>(att_src + foff[ch], a);
#pragma unroll
      for (int q = 0; q < VEC; ++q) a[q] = fmaf(dsl[ch], a[q], acc[ch][q]);
      st<VEC>(dhs + j * HC + foff[ch], a);
      if (head_lead[ch]) ds[j * H + hd[ch]] = dsl[ch];
    }
  } else {
    // Slot layout [acc (H*C) | ds (H)], each part padded to 4 floats.
    const int hc4 = ((HC + 3) / 4) * 4;
    float* p = ws + (int64_t)w.w * (hc4 + ((H + 3) / 4) * 4);
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) {
      if (!fvalid[ch]) continue;
      st<VEC>(p + foff[ch], acc[ch]);
      if (head_lead[ch]) p[hc4 + hd[ch]] = dsl[ch];
    }
  }
}

__global__ __launch_bounds__(256) void gat_bwd_src_fixup(const int32_t* __restrict__ fix,
                                                         int64_t n_fix,
                                                         const float* __restrict__ ws, int H,
                                                         int C, const float* __restrict__ att_src,
                                                         float* __restrict__ dhs,
                                                         float* __restrict__ ds) {
  const int lane = threadIdx.x & 63;
  const int64_t wid = wave_id();
  if (wid >= n_fix) return;
  const int row = fix[3 * wid + 0], first = fix[3 * wid + 1], n = fix[3 * wid + 2];
  const int HC = H * C;
  const int hc4 = ((HC + 3) / 4) * 4;
  const int stride = hc4 + ((H + 3) / 4) * 4;
  for (int f = lane; f < HC; f += 64) {
    const int h = f / C;
    float acc = 0.f, dsum = 0.f;
    for (int k = 0; k < n; ++k) {
      const float* p = ws + (int64_t)(first + k) * stride;
      acc += p[f];
      dsum += p[hc4 + h];
    }
    dhs[(int64_t)row * HC + f] = fmaf(dsum, att_src[f], acc);
    if (f == h * C) ds[(int64_t)row * H + h] = dsum;
  }
}

// Row-parallel (CSR) pass over destination rows i:
// dd[i,h] = sum_e gdd[e,h] + c[i,h] * 1e-16 / den[i,h] and
// dHs[i,:] += dd[i,h(f)] * att_dst[f].
__global__ __launch_bounds__(256) void gat_bwd_dst_kernel(const int4* __restrict__ units,
                                                          int64_t n_units,
                                                          const float* __restrict__ gt, int H,
                                                          int C,
                                                          const float* __restrict__ att_dst,
                                                          const float* __restrict__ cdot,
                                                          const float* __restrict__ den,
                                                          float* __restrict__ dd,
                                                          float* __restrict__ dhs,
                                                          float* __restrict__ ws) {
  const int lane = threadIdx.x & 63;
  const int64_t wid = wave_id();
  if (wid >= n_units) return;
  const int4 w = units[wid];
  const int HC = H * C;
  float part[kMaxHeads];
  for (int h = 0; h < H; ++h) {
    float p = 0.f;
    for (int e = w.y + lane; e < w.z; e += 64) p += gt[(int64_t)e * H + h];
    part[h] = wave_sum(p);
    if (w.w < 0) {
      const int64_t ih = (int64_t)w.x * H + h;
      part[h] += cdot[ih] * (1e-16f / den[ih]);
    }
  }
  if (w.w < 0) {
    if (lane < H) {
      float v = 0.f;
      for (int h = 0; h < H; ++h)
        if (h == lane) v = part[h];
      dd[(int64_t)w.x * H + lane] = v;
    }
    for (int f = lane; f < HC; f += 64) {
      const int h = f / C;
      float v = 0.f;
      for (int q = 0; q < H; ++q)
        if (q == h) v = part[q];
      float* p = dhs + (int64_t)w.x * HC + f;
      *p = fmaf(v, att_dst[f], *p);
    }
  } else if (lane < H) {
    float v = 0.f;
    for (int h = 0; h < H; ++h)
      if (h == lane) v = part[h];
    ws[(int64_t)w.w * H + lane] = v;
  }
}

__global__ __launch_bounds__(256) void gat_bwd_dst_fixup(const int32_t* __restrict__ fix,
                                                         int64_t n_fix,
                                                         const float* __restrict__ ws, int H,
                                                         int C,
                                                         const float* __restrict__ att_dst,
                                                         const float* __restrict__ cdot,
                                                         const float* __restrict__ den,
                                                         float* __restrict__ dd,
                                                         float* __restrict__ dhs) {
  const int lane = threadIdx.x & 63;
  const int64_t wid = wave_id();
  if (wid >= n_fix) return;
  const int row = fix[3 * wid + 0], first = fix[3 * wid + 1], n = fix[3 * wid + 2];
  const int HC = H * C;
  for (int f = lane; f < HC; f += 64) {
    const int h = f / C;
    float v = 0.f;
    for (int k = 0; k < n; ++k) v += ws[(int64_t)(first + k) * H + h];
    const int64_t ih = (int64_t)row * H + h;
    v += cdot[ih] * (1e-16f / den[ih]);
    float* p = dhs + (int64_t)row * HC + f;
    *p = fmaf(v, att_dst[f], *p);
    if (f == h * C) dd[(int64_t)row * H + h] = v;
  }
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

inline unsigned blocks_for(int64_t waves) { return (unsigned)((waves + 3) / 4); }

}  // namespace gr_gat

using namespace gr_gat;

namespace {

int check_heads(int64_t H, int64_t C) {
  GR_REQUIRE(H >= 1 && H <= kMaxHeads, "gat: heads %lld outside [1, %d]", (long long)H,
             kMaxHeads);
  GR_REQUIRE(C >= 1 && H * C <= 1024, "gat: H*C = %lld outside [1, 1024]", (long long)(H * C));
  return GR_OK;
}

// Vector width and chunk count for a row of HC <= 1024 features: float4 when
// every float4 lies inside one head and rows are 16-byte aligned; nch is the
// number of 64-lane chunks rounded up to a power of two (1..16).
void pick_shape(int64_t HC, int64_t C, bool aligned, int* vec, int* nch) {
  *vec = (C % 4 == 0 && HC % 4 == 0 && aligned) ? 4 : 1;
  const int64_t chunks = (HC + *vec - 1) / *vec;
  int n = 1;
  while (n * 64 < chunks) n <<= 1;
  *nch = n;
}

}  // namespace

extern "C" int gr_gat_scores(const float* hs, int64_t ldh, int64_t n_src, int64_t n_dst,
                             int64_t heads, int64_t channels, const float* att_src,
                             const float* att_dst, float* s, float* d, void* stream) {
  gr::clear_error();
  int rc = check_heads(heads, channels);
  if (rc) return rc;
  GR_REQUIRE(n_src >= 0 && n_dst >= 0 && n_dst <= n_src, "gat_scores: bad row counts");
  GR_REQUIRE(ldh >= heads * channels, "gat_scores: ldh < H*C");
  if (n_src == 0) return GR_OK;
  GR_REQUIRE(hs && att_src && att_dst && s && (d || n_dst == 0), "gat_scores: NULL pointer");
  hipLaunchKernelGGL(gat_scores_kernel, dim3(blocks_for(n_src)), dim3(256), 0,
                     gr::as_stream(stream), hs, ldh, n_src, n_dst, (int)heads, (int)channels,
                     att_src, att_dst, s, d);
  GR_HIP_CHECK(hipGetLastError());
  return GR_OK;
}

extern "C" int gr_gat_softmax_stats(const int32_t* units, int64_t n_units, const int32_t* fixups,
                                    int64_t n_fix, const int32_t* idx, const float* s,
                                    const float* d, int64_t heads, float* m, float* den,
                                    float* workspace, int64_t n_slots, void* stream) {
  gr::clear_error();
  GR_REQUIRE(heads >= 1 && heads <= kMaxHeads, "gat_softmax_stats: bad heads");
  GR_REQUIRE(n_units >= 0 && n_fix >= 0 && n_slots >= 0, "gat_softmax_stats: negative extent");
  GR_REQUIRE(n_fix == 0 || (fixups && workspace), "gat_softmax_stats: NULL fixups/workspace");
  if (n_units == 0) return GR_OK;
  GR_REQUIRE(units && aligned16(units) && s && d && m && den,
             "gat_softmax_stats: NULL or misaligned pointer");
  hipStream_t st = gr::as_stream(stream);
  hipLaunchKernelGGL(gat_stats_kernel, dim3(blocks_for(n_units)), dim3(256), 0, st,
                     reinterpret_cast<const int4*>(units), n_units, idx, s, d, (int)heads, m, den,
                     workspace);
  GR_HIP_CHECK(hipGetLastError());
  if (n_fix > 0) {
    hipLaunchKernelGGL(gat_stats_fixup, dim3(blocks_for(n_fix)), dim3(256), 0, st, fixups, n_fix,
                       workspace, (int)heads, m, den);
    GR_HIP_CHECK(hipGetLastError());
  }
  return GR_OK;
}

template <int VEC, int NCH>
static hipError_t launch_gat_agg(hipStream_t st, const int4* units, int64_t n_units,
                                 const int32_t* idx, const float* hs, int64_t ldh, const float* s,
                                 const float* d, const float* m, const float* den, int H, int C,
                                 const float* bias, float* o, float* y, int64_t ldy, float* ws) {
  constexpr int U = NCH == 1 ? 8 : (NCH == 2 ? 4 : (NCH == 4 ? 2 : 1));
  hipLaunchKernelGGL((gat_aggregate_kernel<VEC, NCH, U>), dim3(blocks_for(n_units)), dim3(256), 0,
                     st, units, n_units, idx, hs, ldh, s, d, m, den, H, C, bias, o, y, ldy, ws);
  return hipGetLastError();
}

extern "C" int gr_gat_aggregate(const int32_t* units, int64_t n_units, const int32_t* fixups,
                                int64_t n_fix, const int32_t* idx, const float* hs, int64_t ldh,
                                const float* s, const float* d, const float* m, const float* den,
                                int64_t heads, int64_t channels, const float* bias, float* o,
                                float* y, int64_t ldy, float* workspace, int64_t n_slots,
                                void* stream) {
  gr::clear_error();
  int rc = check_heads(heads, channels);
  if (rc) return rc;
  const int64_t HC = heads * channels;
  GR_REQUIRE(ldh >= HC && (y == nullptr || ldy >= HC), "gat_aggregate: bad leading dims");
  GR_REQUIRE(n_fix == 0 || (fixups && workspace), "gat_aggregate: NULL fixups/workspace");
  if (n_units == 0) return GR_OK;
  GR_REQUIRE(units && aligned16(units) && idx && hs && s && d && m && den && o,
             "gat_aggregate: NULL or misaligned pointer");
  const bool al = aligned16(hs) && aligned16(o) && ldh % 4 == 0 &&
                  (y == nullptr || (aligned16(y) && ldy % 4 == 0)) &&
                  (bias == nullptr || aligned16(bias)) &&
                  (workspace == nullptr || aligned16(workspace));
  int vec, nch;
  pick_shape(HC, channels, al, &vec, &nch);
  hipStream_t st = gr::as_stream(stream);
  const int4* u4 = reinterpret_cast<const int4*>(units);
  const int H = (int)heads, C = (int)channels;
  hipError_t err;
  if (vec == 4) {
    if (nch == 1) err = launch_gat_agg<4, 1>(st, u4, n_units, idx, hs, ldh, s, d, m, den, H, C, bias, o, y, ldy, workspace);
    else if (nch == 2) err = launch_gat_agg<4, 2>(st, u4, n_units, idx, hs, ldh, s, d, m, den, H, C, bias, o, y, ldy, workspace);
    else err = launch_gat_agg<4, 4>(st, u4, n_units, idx, hs, ldh, s, d, m, den, H, C, bias, o, y, ldy, workspace);
  } else {
    if (nch == 1) err = launch_gat_agg<1, 1>(st, u4, n_units, idx, hs, ldh, s, d, m, den, H, C, bias, o, y, ldy, workspace);
    else if (nch == 2) err = launch_gat_agg<1, 2>(st, u4, n_units, idx, hs, ldh, s, d, m, den, H, C, bias, o, y, ldy, workspace);
    else if (nch == 4) err = launch_gat_agg<1, 4>(st, u4, n_units, idx, hs, ldh, s, d, m, den, H, C, bias, o, y, ldy, workspace);
    else if (nch == 8) err = launch_gat_agg<1, 8>(st, u4, n_units, idx, hs, ldh, s, d, m, den, H, C, bias, o, y, ldy, workspace);
    else err = launch_gat_agg<1, 16>(st, u4, n_units, idx, hs, ldh, s, d, m, den, H, C, bias, o, y, ldy, workspace);
  }
  GR_HIP_CHECK(err);
  if (n_fix > 0) {
    hipLaunchKernelGGL(gat_aggregate_fixup, dim3(blocks_for(n_fix)), dim3(256), 0, st, fixups,
                       n_fix, workspace, (int)HC, bias, o, y, ldy);
    GR_HIP_CHECK(hipGetLastError());
  }
  return GR_OK;
}

template <int VEC, int NCH>
static hipError_t launch_gat_bwd(hipStream_t st, const int4* units, int64_t n_units,
                                 const int32_t* row_idx, const int32_t* perm, const float* hs,
                                 int64_t ldh, const float* go, const float* s, const float* d,
                                 const float* m, const float* den, const float* cdot,
                                 const float* att_src, int H, int C, float* dhs, float* ds,
                                 float* gt, float* ws) {
  constexpr int U = NCH == 1 ? 4 : (NCH <= 4 ? 2 : 1);
  hipLaunchKernelGGL((gat_bwd_src_kernel<VEC, NCH, U>), dim3(blocks_for(n_units)), dim3(256), 0,
                     st, units, n_units, row_idx, perm, hs, ldh, go, s, d, m, den, cdot, att_src,
                     H, C, dhs, ds, gt, ws);
  return hipGetLastError();
}

extern "C" int gr_gat_backward_src(const int32_t* units, int64_t n_units, const int32_t* fixups,
                                   int64_t n_fix, const int32_t* row_idx, const int32_t* perm,
                                   const float* hs, int64_t ldh, const float* go, const float* s,
                                   const float* d, const float* m, const float* den,
                                   const float* cdot, const float* att_src, int64_t heads,
                                   int64_t channels, float* dhs, float* ds, float* gt,
                                   float* workspace, int64_t n_slots, void* stream) {
  gr::clear_error();
  int rc = check_heads(heads, channels);
  if (rc) return rc;
  const int64_t HC = heads * channels;
  GR_REQUIRE(ldh >= HC, "gat_backward_src: ldh < H*C");
  GR_REQUIRE(n_fix == 0 || (fixups && workspace), "gat_backward_src: NULL fixups/workspace");
  if (n_units == 0) return GR_OK;
  GR_REQUIRE(units && aligned16(units) && row_idx && perm && hs && go && s && d && m && den &&
                 cdot && att_src && dhs && ds && gt,
             "gat_backward_src: NULL or misaligned pointer");
  const bool al = aligned16(hs) && aligned16(go) && aligned16(dhs) && aligned16(att_src) &&
                  ldh % 4 == 0 && (workspace == nullptr || aligned16(workspace));
  int vec, nch;
  pick_shape(HC, channels, al, &vec, &nch);
  hipStream_t st = gr::as_stream(stream);
  const int4* u4 = reinterpret_cast<const int4*>(units);
  const int H = (int)heads, C = (int)channels;
  hipError_t err;
  if (vec == 4) {
    if (nch == 1) err = launch_gat_bwd<4, 1>(st, u4, n_units, row_idx, perm, hs, ldh, go, s, d, m, den, cdot, att_src, H, C, dhs, ds, gt, workspace);
    else if (nch == 2) err = launch_gat_bwd<4, 2>(st, u4, n_units, row_idx, perm, hs, ldh, go, s, d, m, den, cdot, att_src, H, C, dhs, ds, gt, workspace);
    else err = launch_gat_bwd<4, 4>(st, u4, n_units, row_idx, perm, hs, ldh, go, s, d, m, den, cdot, att_src, H, C, dhs, ds, gt, workspace);
  } else {
    if (nch == 1) err = launch_gat_bwd<1, 1>(st, u4, n_units, row_idx, perm, hs, ldh, go, s, d, m, den, cdot, att_src, H, C, dhs, ds, gt, workspace);
    else if (nch == 2) err = launch_gat_bwd<1, 2>(st, u4, n_units, row_idx, perm, hs, ldh, go, s, d, m, den, cdot, att_src, H, C, dhs, ds, gt, workspace);
    else if (nch == 4) err = launch_gat_bwd<1, 4>(st, u4, n_units, row_idx, perm, hs, ldh, go, s, d, m, den, cdot, att_src, H, C, dhs, ds, gt, workspace);
    else if (nch == 8) err = launch_gat_bwd<1, 8>(st, u4, n_units, row_idx, perm, hs, ldh, go, s, d, m, den, cdot, att_src, H, C, dhs, ds, gt, workspace);
    else err = launch_gat_bwd<1, 16>(st, u4, n_units, row_idx, perm, hs, ldh, go, s, d, m, den, cdot, att_src, H, C, dhs, ds, gt, workspace);
  }
  GR_HIP_CHECK(err);
  if (n_fix > 0) {
    hipLaunchKernelGGL(gat_bwd_src_fixup, dim3(blocks_for(n_fix)), dim3(256), 0, st, fixups,
                       n_fix, workspace, H, C, att_src, dhs, ds);
    GR_HIP_CHECK(hipGetLastError());
  }
  return GR_OK;
}

extern "C" int gr_gat_backward_dst(const int32_t* units, int64_t n_units, const int32_t* fixups,
                                   int64_t n_fix, const float* gt, const float* att_dst,
                                   const float* cdot, const float* den, int64_t heads,
                                   int64_t channels, float* dd, float* dhs, float* workspace,
                                   int64_t n_slots, void* stream) {
  gr::clear_error();
  int rc = check_heads(heads, channels);
  if (rc) return rc;
  GR_REQUIRE(n_fix == 0 || (fixups && workspace), "gat_backward_dst: NULL fixups/workspace");
  if (n_units == 0) return GR_OK;
  GR_REQUIRE(units && aligned16(units) && gt && att_dst && cdot && den && dd && dhs,
             "gat_backward_dst: NULL or misaligned pointer");
  hipStream_t st = gr::as_stream(stream);
  hipLaunchKernelGGL(gat_bwd_dst_kernel, dim3(blocks_for(n_units)), dim3(256), 0, st,
                     reinterpret_cast<const int4*>(units), n_units, gt, (int)heads, (int)channels,
                     att_dst, cdot, den, dd, dhs, workspace);
  GR_HIP_CHECK(hipGetLastError());
  if (n_fix > 0) {
    hipLaunchKernelGGL(gat_bwd_dst_fixup, dim3(blocks_for(n_fix)), dim3(256), 0, st, fixups,
                       n_fix, workspace, (int)heads, (int)channels, att_dst, cdot, den, dd, dhs);
    GR_HIP_CHECK(hipGetLastError());
  }
  return GR_OK;
}
