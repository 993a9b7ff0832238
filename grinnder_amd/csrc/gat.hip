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
//
// alpha is formed once per edge: the statistics pass stores
// exp(v - m_k) with the unit's own max m_k, and after the split rows are
// combined each unit rescales its edges in place,
//   alpha = exp(v - m_k) * exp(m_k - m) / den     (exp(0) = 1 for whole rows),
// so the aggregation (for one head: the GCN SpMM kernel with alpha as the
// edge values) and the backward read alpha instead of re-deriving it.
#include <algorithm>
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

// s[j,:] and, for j < B, d[j,:]: a wavefront covers a row's H*C features
// in NCH chunks of VEC per lane and keeps U rows in flight; grid-stride.
template <int VEC, int NCH, int U>
__global__ __launch_bounds__(256) void gat_scores_kernel(const float* __restrict__ hs, int64_t ldh,
                                                         int64_t n_src, int64_t n_dst, int H,
                                                         int C, const float* __restrict__ att_src,
                                                         const float* __restrict__ att_dst,
                                                         float* __restrict__ s,
                                                         float* __restrict__ d) {
  const int lane = threadIdx.x & 63;
  const int64_t wid = wave_id();
  const int64_t nwaves = (int64_t)gridDim.x * 4;
  const int HC = H * C;
  int fld[NCH], hd[NCH];
  float as[NCH][VEC], ad[NCH][VEC];
#pragma unroll
  for (int ch = 0; ch < NCH; ++ch) {
    const int foff = (ch * 64 + lane) * VEC;
    const bool valid = foff < HC;
    fld[ch] = valid ? foff : HC - VEC;
    hd[ch] = fld[ch] / C;
    ld<VEC>(att_src + fld[ch], as[ch]);
    ld<VEC>(att_dst + fld[ch], ad[ch]);
    if (!valid) {
#pragma unroll
      for (int q = 0; q < VEC; ++q) as[ch][q] = ad[ch][q] = 0.f;
    }
  }
  for (int64_t r0 = wid * U; r0 < n_src; r0 += nwaves * U) {
    float x[U][NCH][VEC];
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int64_t r = r0 + k < n_src ? r0 + k : n_src - 1;
#pragma unroll
      for (int ch = 0; ch < NCH; ++ch) ld<VEC>(hs + r * ldh + fld[ch], x[k][ch]);
    }
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int64_t r = r0 + k;
      if (r >= n_src) break;
      for (int h = 0; h < H; ++h) {
        float ps = 0.f, pd = 0.f;
#pragma unroll
        for (int ch = 0; ch < NCH; ++ch) {
          if (hd[ch] != h) continue;
#pragma unroll
          for (int q = 0; q < VEC; ++q) {
            ps = fmaf(x[k][ch][q], as[ch][q], ps);
            pd = fmaf(x[k][ch][q], ad[ch][q], pd);
          }
        }
        ps = wave_sum(ps);
        if (lane == 0) s[r * H + h] = ps;
        if (r < n_dst) {
          pd = wave_sum(pd);
          if (lane == 0) d[r * H + h] = pd;
        }
      }
    }
  }
}

// ------------------------------------------------------ softmax stats --

// Per unit: m = max_e v_e and sum_e exp(v_e - m) for each head (two passes
// over the unit's edges, lanes parallel over edges); ex[e,h] = exp(v_e - m)
// with this unit's max.  Unsplit rows write m[i,h] and den[i,h] = sum +
// 1e-16; split rows write (m_k, sum_k) partials.
__global__ __launch_bounds__(256) void gat_stats_kernel(const int4* __restrict__ units,
                                                        int64_t n_units,
                                                        const int32_t* __restrict__ idx,
                                                        const float* __restrict__ s,
                                                        const float* __restrict__ d, int H,
                                                        float* __restrict__ m,
                                                        float* __restrict__ den,
                                                        float* __restrict__ ex,
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
      const float x = expf(v - mx);
      ex[(int64_t)e * H + h] = x;
      sum += x;
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

// In place over ex: alpha[e,h] = ex[e,h] * exp(m_k - m[i,h]) / den[i,h], with
// m_k the unit's own max (the row max for whole rows, where the factor is 1).
__global__ __launch_bounds__(256) void gat_alpha_kernel(const int4* __restrict__ units,
                                                        int64_t n_units, int H,
                                                        const float* __restrict__ m,
                                                        const float* __restrict__ den,
                                                        const float* __restrict__ ws,
                                                        float* __restrict__ ex) {
  const int lane = threadIdx.x & 63;
  const int64_t wid = wave_id();
  if (wid >= n_units) return;
  const int4 w = units[wid];
  for (int h = 0; h < H; ++h) {
    const int64_t ih = (int64_t)w.x * H + h;
    const float mi = m[ih];
    const float mk = w.w < 0 ? mi : ws[(int64_t)w.w * 2 * H + h];
    const float corr = expf(mk - mi);
    const float dn = den[ih];
    for (int e = w.y + lane; e < w.z; e += 64) {
      float* p = ex + (int64_t)e * H + h;
      *p = (*p * corr) / dn;
    }
  }
}

// y[r, f] = o[r, f] + bias[f] (bias may be NULL) for r < rows, f < HC.
__global__ __launch_bounds__(256) void gat_add_bias(const float* __restrict__ o, int64_t rows,
                                                    int HC, const float* __restrict__ bias,
                                                    float* __restrict__ y, int64_t ldy) {
  const int64_t n = rows * HC;
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t k = (int64_t)blockIdx.x * 256 + threadIdx.x; k < n; k += stride) {
    const int64_t r = k / HC;
    const int f = (int)(k - r * HC);
    y[r * ldy + f] = o[k] + (bias != nullptr ? bias[f] : 0.f);
  }
}

// ---------------------------------------------------------- aggregate --

// O[i,:] = sum_e alpha[e, h(f)] Hs[col_e,:] for several heads (one head goes
// through the GCN SpMM kernel).  Writes O (no bias) and, if y != NULL,
// Y = O + bias.
template <int VEC, int NCH, int U>
__global__ __launch_bounds__(256) void gat_aggregate_kernel(
    const int4* __restrict__ units, int64_t n_units, const int32_t* __restrict__ idx,
    const float* __restrict__ hs, int64_t ldh, const float* __restrict__ alpha, int H, int C,
    const float* __restrict__ bias, float* __restrict__ o, float* __restrict__ y, int64_t ldy,
    float* __restrict__ ws) {
  const int lane = threadIdx.x & 63;
  const int64_t wid = wave_id();
  if (wid >= n_units) return;
  const int4 w = units[wid];
  const int HC = H * C;
  const int64_t i = w.x;

  int foff[NCH], fld[NCH], hd[NCH];
  bool fvalid[NCH];
#pragma unroll
  for (int ch = 0; ch < NCH; ++ch) {
    foff[ch] = (ch * 64 + lane) * VEC;
    fvalid[ch] = foff[ch] < HC;
    fld[ch] = fvalid[ch] ? foff[ch] : HC - VEC;
    hd[ch] = fld[ch] / C;
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
    float av[U][NCH];
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const float* row = hs + (int64_t)c[k] * ldh;
#pragma unroll
      for (int ch = 0; ch < NCH; ++ch) {
        ld<VEC>(row + fld[ch], r[k][ch]);
        av[k][ch] = alpha[(int64_t)(ok[k] ? e + k : e) * H + hd[ch]];
      }
    }
#pragma unroll
    for (int k = 0; k < U; ++k) {
#pragma unroll
      for (int ch = 0; ch < NCH; ++ch) {
        const float a = ok[k] ? av[k][ch] : 0.f;
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

// Column-parallel (CSC) pass over source rows j.  For each edge (i, j), with
// alpha read through the CSC -> CSR permutation:
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
//
// G lanes per edge: with one head and rows of at most G vectors, a wavefront
// takes 64 / G edges of the unit at once (slot `sub` takes edges sub,
// sub + 64/G, ...); the slots' partial dHs_j and ds_j are combined in a fixed
// butterfly order at the end.
template <int G>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int off = G / 2; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

template <int VEC, int NCH, int U, int G>
__global__ __launch_bounds__(256) void gat_bwd_src_kernel(
    const int4* __restrict__ units, int64_t n_units, const int32_t* __restrict__ row_idx,
    const int32_t* __restrict__ perm, const float* __restrict__ hs, int64_t ldh,
    const float* __restrict__ go, const float* __restrict__ s, const float* __restrict__ d,
    const float* __restrict__ alpha, const float* __restrict__ cdot,
    const float* __restrict__ att_src, int H, int C, float* __restrict__ dhs,
    float* __restrict__ ds, float* __restrict__ gt, float* __restrict__ ws) {
  constexpr int EPI = 64 / G;
  const int lane = threadIdx.x & 63;
  const int sub = lane / G;
  const int li = lane % G;
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
    foff[ch] = (ch * G + li) * VEC;
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

  for (int e = w.y; e < w.z; e += U * EPI) {
    int ii[U], pe[U];
    bool ok[U];
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int ek = e + k * EPI + sub;
      ok[k] = ek < w.z;
      const int el = ok[k] ? ek : w.y;
      ii[k] = row_idx[el];
      pe[k] = perm[el];
    }
    float g[U][NCH][VEC];
#pragma unroll
    for (int k = 0; k < U; ++k)
#pragma unroll
      for (int ch = 0; ch < NCH; ++ch) ld<VEC>(go + (int64_t)ii[k] * HC + fld[ch], g[k][ch]);
#pragma unroll
    for (int k = 0; k < U; ++k) {
      // Per-lane partial dot products, then one reduction per head.
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
        t = group_sum<G>(t);
#pragma unroll
        for (int ch = 0; ch < NCH; ++ch) ga[ch] = t;
      } else {
        // Several heads: G == 64 (one edge per wavefront).
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
        const float a = alpha[(int64_t)pe[k] * H + hd[ch]];
        const float ge = a * (ga[ch] - cdot[ih]);
        const bool pos = tt > 0.f;
        if (ok[k]) {
          dsl[ch] += pos ? ge : 0.2f * ge;
#pragma unroll
          for (int q = 0; q < VEC; ++q) acc[ch][q] = fmaf(a, g[k][ch][q], acc[ch][q]);
          if (head_lead[ch]) gt[(int64_t)pe[k] * H + hd[ch]] = pos ? 0.f : -0.8f * ge;
        }
      }
    }
  }
  // Combine the edge slots (no-op for G == 64).
#pragma unroll
  for (int off = G; off < 64; off <<= 1) {
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) {
      dsl[ch] += __shfl_xor(dsl[ch], off, 64);
#pragma unroll
      for (int q = 0; q < VEC; ++q) acc[ch][q] += __shfl_xor(acc[ch][q], off, 64);
    }
  }
  if (sub != 0) return;

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
  const int64_t HC = heads * channels;
  const bool al = aligned16(hs) && ldh % 4 == 0 && aligned16(att_src) && aligned16(att_dst);
  int vec, nch;
  pick_shape(HC, channels, al, &vec, &nch);
  hipStream_t st = gr::as_stream(stream);
  const int H = (int)heads, C = (int)channels;
  // U rows in flight per wavefront; enough wavefronts to fill the chip.
  auto grid = [&](int u) {
    const int64_t waves = (n_src + u - 1) / u;
    return dim3((unsigned)std::min<int64_t>(4096, (waves + 3) / 4));
  };
#define GR_SC(V, N, U)                                                                   \
  hipLaunchKernelGGL((gat_scores_kernel<V, N, U>), grid(U), dim3(256), 0, st, hs, ldh, n_src, \
                     n_dst, H, C, att_src, att_dst, s, d)
  if (vec == 4) {
    if (nch == 1) GR_SC(4, 1, 4); else if (nch == 2) GR_SC(4, 2, 2); else GR_SC(4, 4, 1);
  } else {
    if (nch == 1) GR_SC(1, 1, 4); else if (nch == 2) GR_SC(1, 2, 2); else if (nch == 4) GR_SC(1, 4, 1);
    else if (nch == 8) GR_SC(1, 8, 1); else GR_SC(1, 16, 1);
  }
#undef GR_SC
  GR_HIP_CHECK(hipGetLastError());
  return GR_OK;
}

extern "C" int gr_gat_softmax_stats(const int32_t* units, int64_t n_units, const int32_t* fixups,
                                    int64_t n_fix, const int32_t* idx, const float* s,
                                    const float* d, int64_t heads, float* m, float* den,
                                    float* alpha, float* workspace, int64_t n_slots,
                                    void* stream) {
  gr::clear_error();
  GR_REQUIRE(heads >= 1 && heads <= kMaxHeads, "gat_softmax_stats: bad heads");
  GR_REQUIRE(n_units >= 0 && n_fix >= 0 && n_slots >= 0, "gat_softmax_stats: negative extent");
  GR_REQUIRE(n_fix == 0 || (fixups && workspace), "gat_softmax_stats: NULL fixups/workspace");
  if (n_units == 0) return GR_OK;
  GR_REQUIRE(units && aligned16(units) && s && d && m && den && alpha,
             "gat_softmax_stats: NULL or misaligned pointer");
  hipStream_t st = gr::as_stream(stream);
  const int4* u4 = reinterpret_cast<const int4*>(units);
  hipLaunchKernelGGL(gat_stats_kernel, dim3(blocks_for(n_units)), dim3(256), 0, st, u4, n_units,
                     idx, s, d, (int)heads, m, den, alpha, workspace);
  GR_HIP_CHECK(hipGetLastError());
  if (n_fix > 0) {
    hipLaunchKernelGGL(gat_stats_fixup, dim3(blocks_for(n_fix)), dim3(256), 0, st, fixups, n_fix,
                       workspace, (int)heads, m, den);
    GR_HIP_CHECK(hipGetLastError());
  }
  hipLaunchKernelGGL(gat_alpha_kernel, dim3(blocks_for(n_units)), dim3(256), 0, st, u4, n_units,
                     (int)heads, m, den, workspace, alpha);
  GR_HIP_CHECK(hipGetLastError());
  return GR_OK;
}

template <int VEC, int NCH>
static hipError_t launch_gat_agg(hipStream_t st, const int4* units, int64_t n_units,
                                 const int32_t* idx, const float* hs, int64_t ldh,
                                 const float* alpha, int H, int C, const float* bias, float* o,
                                 float* y, int64_t ldy, float* ws) {
  constexpr int U = NCH == 1 ? 8 : (NCH == 2 ? 4 : (NCH == 4 ? 2 : 1));
  hipLaunchKernelGGL((gat_aggregate_kernel<VEC, NCH, U>), dim3(blocks_for(n_units)), dim3(256), 0,
                     st, units, n_units, idx, hs, ldh, alpha, H, C, bias, o, y, ldy, ws);
  return hipGetLastError();
}

extern "C" int gr_gat_aggregate(const int32_t* units, int64_t n_units, const int32_t* fixups,
                                int64_t n_fix, const int32_t* idx, const float* hs, int64_t ldh,
                                const float* alpha, int64_t n_dst, int64_t heads,
                                int64_t channels, const float* bias, float* o, float* y,
                                int64_t ldy, float* workspace, int64_t n_slots, void* stream) {
  gr::clear_error();
  int rc = check_heads(heads, channels);
  if (rc) return rc;
  const int64_t HC = heads * channels;
  GR_REQUIRE(n_dst >= 0, "gat_aggregate: negative row count");
  GR_REQUIRE(ldh >= HC && (y == nullptr || ldy >= HC), "gat_aggregate: bad leading dims");
  GR_REQUIRE(n_fix == 0 || (fixups && workspace), "gat_aggregate: NULL fixups/workspace");
  if (n_units == 0) return GR_OK;
  GR_REQUIRE(units && aligned16(units) && idx && hs && alpha && o,
             "gat_aggregate: NULL or misaligned pointer");
  hipStream_t st = gr::as_stream(stream);
  const int H = (int)heads, C = (int)channels;
  if (H == 1) {
    // One head: O = A_alpha Hs is the GCN SpMM with alpha as edge values.
    rc = gr_gcn_aggregate(units, n_units, fixups, n_fix, idx, alpha, hs, ldh, o, HC, nullptr,
                          n_dst, HC, workspace, n_slots, stream);
    if (rc) return rc;
    if (y != nullptr && n_dst > 0) {
      const int64_t n = n_dst * HC;
      hipLaunchKernelGGL(gat_add_bias, dim3((unsigned)std::min<int64_t>(8192, (n + 255) / 256)),
                         dim3(256), 0, st, o, n_dst, (int)HC, bias, y, ldy);
      GR_HIP_CHECK(hipGetLastError());
    }
    return GR_OK;
  }
  const bool al = aligned16(hs) && aligned16(o) && ldh % 4 == 0 &&
                  (y == nullptr || (aligned16(y) && ldy % 4 == 0)) &&
                  (bias == nullptr || aligned16(bias)) &&
                  (workspace == nullptr || aligned16(workspace));
  int vec, nch;
  pick_shape(HC, channels, al, &vec, &nch);
  const int4* u4 = reinterpret_cast<const int4*>(units);
  hipError_t err;
  if (vec == 4) {
    if (nch == 1) err = launch_gat_agg<4, 1>(st, u4, n_units, idx, hs, ldh, alpha, H, C, bias, o, y, ldy, workspace);
    else if (nch == 2) err = launch_gat_agg<4, 2>(st, u4, n_units, idx, hs, ldh, alpha, H, C, bias, o, y, ldy, workspace);
    else err = launch_gat_agg<4, 4>(st, u4, n_units, idx, hs, ldh, alpha, H, C, bias, o, y, ldy, workspace);
  } else {
    if (nch == 1) err = launch_gat_agg<1, 1>(st, u4, n_units, idx, hs, ldh, alpha, H, C, bias, o, y, ldy, workspace);
    else if (nch == 2) err = launch_gat_agg<1, 2>(st, u4, n_units, idx, hs, ldh, alpha, H, C, bias, o, y, ldy, workspace);
    else if (nch == 4) err = launch_gat_agg<1, 4>(st, u4, n_units, idx, hs, ldh, alpha, H, C, bias, o, y, ldy, workspace);
    else if (nch == 8) err = launch_gat_agg<1, 8>(st, u4, n_units, idx, hs, ldh, alpha, H, C, bias, o, y, ldy, workspace);
    else err = launch_gat_agg<1, 16>(st, u4, n_units, idx, hs, ldh, alpha, H, C, bias, o, y, ldy, workspace);
  }
  GR_HIP_CHECK(err);
  if (n_fix > 0) {
    hipLaunchKernelGGL(gat_aggregate_fixup, dim3(blocks_for(n_fix)), dim3(256), 0, st, fixups,
                       n_fix, workspace, (int)HC, bias, o, y, ldy);
    GR_HIP_CHECK(hipGetLastError());
  }
  return GR_OK;
}

template <int VEC, int NCH, int G = 64>
static hipError_t launch_gat_bwd(hipStream_t st, const int4* units, int64_t n_units,
                                 const int32_t* row_idx, const int32_t* perm, const float* hs,
                                 int64_t ldh, const float* go, const float* s, const float* d,
                                 const float* alpha, const float* cdot, const float* att_src,
                                 int H, int C, float* dhs, float* ds, float* gt, float* ws) {
  constexpr int U = G < 64 ? 2 : (NCH == 1 ? 4 : (NCH <= 4 ? 2 : 1));
  hipLaunchKernelGGL((gat_bwd_src_kernel<VEC, NCH, U, G>), dim3(blocks_for(n_units)), dim3(256), 0,
                     st, units, n_units, row_idx, perm, hs, ldh, go, s, d, alpha, cdot, att_src,
                     H, C, dhs, ds, gt, ws);
  return hipGetLastError();
}

extern "C" int gr_gat_backward_src(const int32_t* units, int64_t n_units, const int32_t* fixups,
                                   int64_t n_fix, const int32_t* row_idx, const int32_t* perm,
                                   const float* hs, int64_t ldh, const float* go, const float* s,
                                   const float* d, const float* alpha,
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
  GR_REQUIRE(units && aligned16(units) && row_idx && perm && hs && go && s && d && alpha &&
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
  const int64_t chunks = (HC + vec - 1) / vec;
  if (H == 1 && chunks <= 32) {
    // Narrow single-head rows: several edges per wavefront.
    if (vec == 4) {
      if (chunks <= 8) err = launch_gat_bwd<4, 1, 8>(st, u4, n_units, row_idx, perm, hs, ldh, go, s, d, alpha, cdot, att_src, H, C, dhs, ds, gt, workspace);
      else if (chunks <= 16) err = launch_gat_bwd<4, 1, 16>(st, u4, n_units, row_idx, perm, hs, ldh, go, s, d, alpha, cdot, att_src, H, C, dhs, ds, gt, workspace);
      else err = launch_gat_bwd<4, 1, 32>(st, u4, n_units, row_idx, perm, hs, ldh, go, s, d, alpha, cdot, att_src, H, C, dhs, ds, gt, workspace);
    } else {
      if (chunks <= 8) err = launch_gat_bwd<1, 1, 8>(st, u4, n_units, row_idx, perm, hs, ldh, go, s, d, alpha, cdot, att_src, H, C, dhs, ds, gt, workspace);
      else if (chunks <= 16) err = launch_gat_bwd<1, 1, 16>(st, u4, n_units, row_idx, perm, hs, ldh, go, s, d, alpha, cdot, att_src, H, C, dhs, ds, gt, workspace);
      else err = launch_gat_bwd<1, 1, 32>(st, u4, n_units, row_idx, perm, hs, ldh, go, s, d, alpha, cdot, att_src, H, C, dhs, ds, gt, workspace);
    }
  } else if (vec == 4) {
    if (nch == 1) err = launch_gat_bwd<4, 1>(st, u4, n_units, row_idx, perm, hs, ldh, go, s, d, alpha, cdot, att_src, H, C, dhs, ds, gt, workspace);
    else if (nch == 2) err = launch_gat_bwd<4, 2>(st, u4, n_units, row_idx, perm, hs, ldh, go, s, d, alpha, cdot, att_src, H, C, dhs, ds, gt, workspace);
    else err = launch_gat_bwd<4, 4>(st, u4, n_units, row_idx, perm, hs, ldh, go, s, d, alpha, cdot, att_src, H, C, dhs, ds, gt, workspace);
  } else {
    if (nch == 1) err = launch_gat_bwd<1, 1>(st, u4, n_units, row_idx, perm, hs, ldh, go, s, d, alpha, cdot, att_src, H, C, dhs, ds, gt, workspace);
    else if (nch == 2) err = launch_gat_bwd<1, 2>(st, u4, n_units, row_idx, perm, hs, ldh, go, s, d, alpha, cdot, att_src, H, C, dhs, ds, gt, workspace);
    else if (nch == 4) err = launch_gat_bwd<1, 4>(st, u4, n_units, row_idx, perm, hs, ldh, go, s, d, alpha, cdot, att_src, H, C, dhs, ds, gt, workspace);
    else if (nch == 8) err = launch_gat_bwd<1, 8>(st, u4, n_units, row_idx, perm, hs, ldh, go, s, d, alpha, cdot, att_src, H, C, dhs, ds, gt, workspace);
    else err = launch_gat_bwd<1, 16>(st, u4, n_units, row_idx, perm, hs, ldh, go, s, d, alpha, cdot, att_src, H, C, dhs, ds, gt, workspace);
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
