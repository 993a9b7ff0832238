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
// so the aggregation and the backward read alpha instead of re-deriving it.
// With one head the statistics, alpha and the aggregation run as one fused
// pass per unit (gat_fwd_fused); several heads use the statistics kernel and
// then gat_aggregate_kernel.
#include <algorithm>
#include <atomic>
#include <cfloat>

#include "gr_internal.h"
#include "ln_row.h"
#include "wave.h"

namespace gr_gat {

constexpr int kMaxHeads = 16;

using gr_wave::wave_max;
using gr_wave::wave_sum;

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

// cdot[i,h] = <a[i,h,:], b[i,h,:]> (the backward's c_i = <GO_i, O_i>): the
// same row walk as the scores kernel with a second row in place of the
// attention vectors.
template <int VEC, int NCH, int U>
__global__ __launch_bounds__(256) void gat_row_dot_kernel(const float* __restrict__ a,
                                                          int64_t lda,
                                                          const float* __restrict__ b,
                                                          int64_t ldb, int64_t rows, int H,
                                                          int C, float* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t wid = wave_id();
  const int64_t nwaves = (int64_t)gridDim.x * 4;
  const int HC = H * C;
  int fld[NCH], hd[NCH];
  bool valid[NCH];
#pragma unroll
  for (int ch = 0; ch < NCH; ++ch) {
    const int foff = (ch * 64 + lane) * VEC;
    valid[ch] = foff < HC;
    fld[ch] = valid[ch] ? foff : HC - VEC;
    hd[ch] = fld[ch] / C;
  }
  for (int64_t r0 = wid * U; r0 < rows; r0 += nwaves * U) {
    float x[U][NCH][VEC], z[U][NCH][VEC];
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int64_t r = r0 + k < rows ? r0 + k : rows - 1;
#pragma unroll
      for (int ch = 0; ch < NCH; ++ch) {
        ld<VEC>(a + r * lda + fld[ch], x[k][ch]);
        ld<VEC>(b + r * ldb + fld[ch], z[k][ch]);
      }
    }
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int64_t r = r0 + k;
      if (r >= rows) break;
      for (int h = 0; h < H; ++h) {
        float p = 0.f;
#pragma unroll
        for (int ch = 0; ch < NCH; ++ch) {
          if (hd[ch] != h || !valid[ch]) continue;
#pragma unroll
          for (int q = 0; q < VEC; ++q) p = fmaf(x[k][ch][q], z[k][ch][q], p);
        }
        p = wave_sum(p);
        if (lane == 0) out[r * H + h] = p;
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

// ------------------------------------------------ fused forward, H = 1 --

// One head: the edge softmax and the weighted aggregation in one pass per
// plan unit (row i, edges [y, z), slot).
//   Pass 1, lanes parallel over the unit's edges: m = max_e v_e and
//   sum = sum_e exp(v_e - m); a unit of up to kFwdChunks * 64 edges keeps
//   every edge's (col, exp(v - m)) in registers, a longer one the first 64
//   edges' (col, v).
//   Pass 2, in 64-edge chunks: lane l forms the weight of edge l of the chunk,
//   exp(v - m) / den for a whole row (den = sum + 1e-16) or the unscaled
//   exp(v - m_k) of a split row's unit, stores it as alpha, and the wavefront
//   aggregates the chunk's rows with column ids and weights taken from the
//   owning lanes (readlane when the whole wavefront takes one edge, a
//   cross-lane permute for G-lane edge slots).
// Edges are assigned to slots and summed in the same order as in the GCN
// SpMM kernel, so whole rows give the same bits as gr_gat_softmax_stats
// followed by gr_gat_aggregate.  Split rows leave (acc_k, m_k, sum_k) in
// their workspace slot for gat_fused_fixup.
// 64-edge chunks of a unit whose column ids and logits gat_fwd_fused keeps in
// registers (gr_spmm_plan's units hold at most 512 edges).
constexpr int kFwdChunks = 8;

// The conv bias + LayerNorm + activation after the attention (the GAT
// model's epilogue, grinnder/nn/gat.py:74-78), fused into the whole-row
// store of one-head rows held by a full wavefront (G = 64): with gamma set,
// a row writes h = O + bias, out = act(LN(h)) (into y, row stride ldy) and
// the row's mean and rstd, and neither O nor Y + bias; ln_relu_store_row
// forms them exactly as the dense epilogue does from the same h.
struct GatLn {
  const float* gamma = nullptr;
  const float* beta = nullptr;
  float eps = 0.f;
  int act = GR_ACT_ELU;
  float* h = nullptr;
  float* mean = nullptr;
  float* rstd = nullptr;
};

template <int VEC, int NCH>
__device__ __forceinline__ void ln_epilogue(float (&acc)[NCH][VEC], const bool (&fvalid)[NCH],
                                            const int (&foff)[NCH], const int (&fld)[NCH],
                                            int C, const float* __restrict__ bias,
                                            const GatLn& ln, int64_t i, float* __restrict__ y,
                                            int64_t ldy, int lane) {
  if (bias != nullptr) {
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) {
      float b[VEC];
      ld<VEC>(bias + fld[ch], b);
#pragma unroll
      for (int q = 0; q < VEC; ++q) acc[ch][q] += b[q];
    }
  }
  if (ln.act == GR_ACT_ELU)
    gr_ln::ln_relu_store_row<VEC, NCH, GR_ACT_ELU>(acc, fvalid, foff, C, ln.gamma, ln.beta,
                                                   ln.eps, ln.h + i * C, y + i * ldy,
                                                   ln.mean + i, ln.rstd + i, lane);
  else
    gr_ln::ln_relu_store_row<VEC, NCH, GR_ACT_RELU>(acc, fvalid, foff, C, ln.gamma, ln.beta,
                                                    ln.eps, ln.h + i * C, y + i * ldy,
                                                    ln.mean + i, ln.rstd + i, lane);
}

template <int VEC, int G, int NCH, int U>
__global__ __launch_bounds__(256) void gat_fwd_fused(
    const int4* __restrict__ units, int64_t n_units, const int32_t* __restrict__ idx,
    const float* __restrict__ hs, int64_t ldh, const float* __restrict__ s,
    const float* __restrict__ d, int C, const float* __restrict__ bias, float* __restrict__ m,
    float* __restrict__ den, float* __restrict__ alpha, float* __restrict__ o,
    float* __restrict__ y, int64_t ldy, float* __restrict__ ws, int64_t ws_stride,
    int min_len, GatLn ln) {
  constexpr int EPI = 64 / G;
  const int lane = threadIdx.x & 63;
  const int64_t wid = wave_id();
  if (wid >= n_units) return;
  const int4 w = units[wid];
  const int slot = (EPI == 1) ? 0 : lane / G;
  const int sub = (EPI == 1) ? lane : lane % G;
  const int64_t i = w.x;
  const int len = w.z - w.y;
  // Whole rows shorter than min_len are gat_fwd_rows' work.
  if (w.w < 0 && len < min_len) return;

  int foff[NCH], fld[NCH];
  bool fvalid[NCH];
#pragma unroll
  for (int ch = 0; ch < NCH; ++ch) {
    foff[ch] = (ch * G + sub) * VEC;
    fvalid[ch] = foff[ch] < C;
    fld[ch] = fvalid[ch] ? foff[ch] : C - VEC;
  }

  if (len <= 0) {
    // A row without edges (never a split unit): m = 0, den = 1, O = 0.
    if (lane == 0) {
      m[i] = 0.f;
      den[i] = 1.f;
    }
    if constexpr (G == 64) {
      if (ln.gamma != nullptr) {
        float z[NCH][VEC];
#pragma unroll
        for (int ch = 0; ch < NCH; ++ch)
#pragma unroll
          for (int q = 0; q < VEC; ++q) z[ch][q] = 0.f;
        ln_epilogue<VEC, NCH>(z, fvalid, foff, fld, C, bias, ln, i, y, ldy, lane);
        return;
      }
    }
    if (slot != 0) return;
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) {
      if (!fvalid[ch]) continue;
      float z[VEC];
#pragma unroll
      for (int q = 0; q < VEC; ++q) z[q] = 0.f;
      st<VEC>(o + i * C + foff[ch], z);
      if (y != nullptr) {
        if (bias != nullptr) ld<VEC>(bias + foff[ch], z);
        st<VEC>(y + i * ldy + foff[ch], z);
      }
    }
    return;
  }

  // Every load below is unconditional (indices clamped into the unit), so
  // the compiler can wait for each one alone: lanes past the unit's end read
  // its last edge and get weight 0.  Vector loads return in issue order: the
  // column ids and logits go out first, then the first U row gathers, which
  // are independent of the statistics and stay in flight while they run.
  const float di = d[i];
  float r[U][NCH][VEC];
  float acc[NCH][VEC];
#pragma unroll
  for (int ch = 0; ch < NCH; ++ch)
#pragma unroll
    for (int q = 0; q < VEC; ++q) acc[ch][q] = 0.f;
  // First U row gathers of the 64-edge chunk whose column ids are c0.
  auto gather_first = [&](int c0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      int c;
      if constexpr (EPI == 1) {
        c = __builtin_amdgcn_readlane(c0, u);
      } else {
        c = __shfl(c0, u * EPI + slot, 64);
      }
      const float* row = hs + (int64_t)c * ldh;
#pragma unroll
      for (int ch = 0; ch < NCH; ++ch) ld<VEC>(row + fld[ch], r[u][ch]);
    }
  };
  // Aggregation of one 64-edge chunk: n edges from b, lane l holding column
  // id cl and weight al of edge b + l; the first U gathers of the unit's
  // first chunk are already in r.
  auto aggregate_chunk = [&](int n, bool first, int cl, float al) {
    for (int k = 0; k < n; k += EPI * U) {
      int c[U];
      float a[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if constexpr (EPI == 1) {
          c[u] = __builtin_amdgcn_readlane(cl, k + u);
          a[u] = __builtin_bit_cast(float,
                                    __builtin_amdgcn_readlane(__builtin_bit_cast(int, al), k + u));
        } else {
          const int t = k + u * EPI + slot;
          c[u] = __shfl(cl, t, 64);
          a[u] = __shfl(al, t, 64);
        }
      }
      if (!(first && k == 0)) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const float* row = hs + (int64_t)c[u] * ldh;
#pragma unroll
          for (int ch = 0; ch < NCH; ++ch) ld<VEC>(row + fld[ch], r[u][ch]);
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int ch = 0; ch < NCH; ++ch)
#pragma unroll
          for (int q = 0; q < VEC; ++q) acc[ch][q] = fmaf(a[u], r[u][ch][q], acc[ch][q]);
    }
  };
  const bool whole = w.w < 0;
  float mx, sum, dn;
  const int nchunks = (len + 63) >> 6;
  if (nchunks <= kFwdChunks) {
    // Units of up to kFwdChunks * 64 edges (every unit of gr_spmm_plan's
    // 512-edge segments): all column ids and logits are loaded at once and
    // kept in registers, so the unit costs one index load, one logit load
    // and its row gathers in sequence, not three passes over the logits.
    // Chunk k's values sit in cb[k] / eb[k]; the aggregation shifts them
    // down one chunk at a time so that every register index is static.
    int cb[kFwdChunks];
    float eb[kFwdChunks];
#pragma unroll
    for (int k = 0; k < kFwdChunks; ++k) {
      cb[k] = 0;
      eb[k] = 0.f;
      if (k < nchunks) cb[k] = idx[w.y + min(k * 64 + lane, len - 1)];
    }
#pragma unroll
    for (int k = 0; k < kFwdChunks; ++k)
      if (k < nchunks) eb[k] = s[cb[k]];
    gather_first(cb[0]);
    mx = -FLT_MAX;
#pragma unroll
    for (int k = 0; k < kFwdChunks; ++k)
      if (k < nchunks) {
        eb[k] = leaky(eb[k] + di);
        if (k * 64 + lane < len) mx = fmaxf(mx, eb[k]);
      }
    mx = wave_max(mx);
    sum = 0.f;
#pragma unroll
    for (int k = 0; k < kFwdChunks; ++k)
      if (k < nchunks) {
        eb[k] = k * 64 + lane < len ? expf(eb[k] - mx) : 0.f;
        sum += eb[k];
      }
    sum = wave_sum(sum);
    dn = whole ? sum + 1e-16f : 1.f;
    for (int k = 0; k < nchunks; ++k) {
      const int b = w.y + k * 64;
      const int n = min(64, w.z - b);
      const bool ok = lane < n;
      const int cl = cb[0];
      const float al = ok ? eb[0] / dn : 0.f;
#pragma unroll
      for (int q = 0; q + 1 < kFwdChunks; ++q) {
        cb[q] = cb[q + 1];
        eb[q] = eb[q + 1];
      }
      aggregate_chunk(n, k == 0, cl, al);
      if (ok && alpha != nullptr) alpha[b + lane] = al;
    }
  } else {
    // Longer units: statistics in two passes over the logits, the first 64
    // edges' (col, v) kept in registers.
    const int c0 = idx[w.y + min(lane, len - 1)];
    const float s0 = s[c0];
    gather_first(c0);
    const float v0 = lane < len ? leaky(s0 + di) : -FLT_MAX;
    mx = v0;
    for (int b = w.y + 64; b < w.z; b += 64) {
      const float v = leaky(s[idx[min(b + lane, w.z - 1)]] + di);
      if (b + lane < w.z) mx = fmaxf(mx, v);
    }
    mx = wave_max(mx);
    sum = lane < len ? expf(v0 - mx) : 0.f;
    for (int b = w.y + 64; b < w.z; b += 64) {
      const float v = leaky(s[idx[min(b + lane, w.z - 1)]] + di);
      if (b + lane < w.z) sum += expf(v - mx);
    }
    sum = wave_sum(sum);
    dn = whole ? sum + 1e-16f : 1.f;
    // Stores wait until a chunk's row loads are consumed: on gfx9 a wait for
    // a load also waits for every store issued before it.
    for (int b = w.y; b < w.z; b += 64) {
      const int n = min(64, w.z - b);
      const bool ok = lane < n;
      const bool first = b == w.y;
      int cl;
      float al;
      if (first) {
        cl = c0;
        al = ok ? expf(v0 - mx) / dn : 0.f;
      } else {
        cl = idx[b + min(lane, n - 1)];
        const float v = leaky(s[cl] + di);
        al = ok ? expf(v - mx) / dn : 0.f;
      }
      aggregate_chunk(n, first, cl, al);
      if (ok && alpha != nullptr) alpha[b + lane] = al;
    }
  }

  if (lane == 0) {
    if (whole) {
      m[i] = mx;
      den[i] = dn;
    } else {
      float* stt = ws + (int64_t)w.w * ws_stride + ws_stride - 4;
      stt[0] = mx;
      stt[1] = sum;
    }
  }
  if constexpr (EPI > 1) {
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch)
#pragma unroll
      for (int q = 0; q < VEC; ++q) acc[ch][q] = gr_wave::slot_sum<G>(acc[ch][q]);
  }
  if constexpr (G == 64) {
    if (whole && ln.gamma != nullptr) {
      ln_epilogue<VEC, NCH>(acc, fvalid, foff, fld, C, bias, ln, i, y, ldy, lane);
      return;
    }
  }
  if (slot != 0) return;
  if (whole) {
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) {
      if (!fvalid[ch]) continue;
      st<VEC>(o + i * C + foff[ch], acc[ch]);
      if (y != nullptr) {
        float b[VEC];
        if (bias != nullptr) {
          ld<VEC>(bias + foff[ch], b);
        } else {
#pragma unroll
          for (int q = 0; q < VEC; ++q) b[q] = 0.f;
        }
#pragma unroll
        for (int q = 0; q < VEC; ++q) b[q] += acc[ch][q];
        st<VEC>(y + i * ldy + foff[ch], b);
      }
    }
  } else {
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch)
      if (fvalid[ch]) st<VEC>(ws + (int64_t)w.w * ws_stride + foff[ch], acc[ch]);
  }
}

// Split rows of the fused forward: one workgroup per (split row, 256
// features).  m = max_k m_k, den = sum_k sum_k exp(m_k - m) + 1e-16 and
// O = sum_k acc_k exp(m_k - m) / den, in slot order.
__global__ __launch_bounds__(256) void gat_fused_fixup(const int32_t* __restrict__ fix,
                                                       const float* __restrict__ ws,
                                                       int64_t ws_stride, int C,
                                                       const float* __restrict__ bias,
                                                       float* __restrict__ m,
                                                       float* __restrict__ den,
                                                       float* __restrict__ o,
                                                       float* __restrict__ y, int64_t ldy) {
  const int64_t r = blockIdx.x;
  const int row = fix[3 * r + 0], first = fix[3 * r + 1], n = fix[3 * r + 2];
  const float* stats = ws + ws_stride - 4;  // (m_k, sum_k) of slot k at stats[k * ws_stride]
  float mx = -FLT_MAX;
  for (int k = 0; k < n; ++k) mx = fmaxf(mx, stats[(int64_t)(first + k) * ws_stride]);
  float sum = 0.f;
  for (int k = 0; k < n; ++k) {
    const float* st = stats + (int64_t)(first + k) * ws_stride;
    sum += st[1] * expf(st[0] - mx);
  }
  const float dn = sum + 1e-16f;
  const int f = blockIdx.y * 256 + threadIdx.x;
  if (f < C) {
    float acc = 0.f;
    int k = 0;
    for (; k + 4 <= n; k += 4) {
      const float* p = ws + (int64_t)(first + k) * ws_stride;
      const float a0 = p[f], a1 = p[ws_stride + f], a2 = p[2 * ws_stride + f],
                  a3 = p[3 * ws_stride + f];
      acc = fmaf(a0, expf(p[ws_stride - 4] - mx), acc);
      acc = fmaf(a1, expf(p[2 * ws_stride - 4] - mx), acc);
      acc = fmaf(a2, expf(p[3 * ws_stride - 4] - mx), acc);
      acc = fmaf(a3, expf(p[4 * ws_stride - 4] - mx), acc);
    }
    for (; k < n; ++k) {
      const float* p = ws + (int64_t)(first + k) * ws_stride;
      acc = fmaf(p[f], expf(p[ws_stride - 4] - mx), acc);
    }
    acc /= dn;
    o[(int64_t)row * C + f] = acc;
    if (y != nullptr) y[(int64_t)row * ldy + f] = acc + (bias != nullptr ? bias[f] : 0.f);
  }
  if (blockIdx.y == 0 && threadIdx.x == 0) {
    m[row] = mx;
    den[row] = dn;
  }
}

// Split rows of the forward with the LayerNorm epilogue (GatLn): one
// workgroup per split row, thread t owning features t, t + 256, ... (C <=
// 1024).  O as gat_fused_fixup forms it, h = O + bias, the row's statistics
// by the fixed-order workgroup reduction of the GCN epilogue's fixup, then
// out = act(LN(h)).
__global__ __launch_bounds__(256) void gat_fused_fixup_ln(const int32_t* __restrict__ fix,
                                                          const float* __restrict__ ws,
                                                          int64_t ws_stride, int C,
                                                          const float* __restrict__ bias,
                                                          float* __restrict__ m,
                                                          float* __restrict__ den, GatLn ln,
                                                          float* __restrict__ y, int64_t ldy) {
  __shared__ float red[4];
  const int64_t r = blockIdx.x;
  const int row = fix[3 * r + 0], first = fix[3 * r + 1], n = fix[3 * r + 2];
  const float* stats = ws + ws_stride - 4;
  float mx = -FLT_MAX;
  for (int k = 0; k < n; ++k) mx = fmaxf(mx, stats[(int64_t)(first + k) * ws_stride]);
  float sum = 0.f;
  for (int k = 0; k < n; ++k) {
    const float* st = stats + (int64_t)(first + k) * ws_stride;
    sum += st[1] * expf(st[0] - mx);
  }
  const float dn = sum + 1e-16f;
  float hv[4];
  float sacc = 0.f;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int f = threadIdx.x + q * 256;
    float a = 0.f;
    if (f < C) {
      float acc = 0.f;
      for (int k = 0; k < n; ++k) {
        const float* p = ws + (int64_t)(first + k) * ws_stride;
        acc = fmaf(p[f], expf(p[ws_stride - 4] - mx), acc);
      }
      a = acc / dn + (bias != nullptr ? bias[f] : 0.f);
    }
    hv[q] = a;
    sacc += a;
  }
  const float mu = gr_ln::block_sum256(sacc, red) / (float)C;
  float qv = 0.f;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float dlt = hv[q] - mu;
    qv += threadIdx.x + q * 256 < C ? dlt * dlt : 0.f;
  }
  const float rs = 1.0f / sqrtf(gr_ln::block_sum256(qv, red) / (float)C + ln.eps);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int f = threadIdx.x + q * 256;
    if (f >= C) continue;
    const float yv = gr_ln::ln_affine(hv[q], mu, rs, ln.gamma[f], ln.beta[f]);
    ln.h[(int64_t)row * C + f] = hv[q];
    y[(int64_t)row * ldy + f] = ln.act == GR_ACT_ELU ? gr_ln::act_fwd<GR_ACT_ELU>(yv)
                                                     : gr_ln::act_fwd<GR_ACT_RELU>(yv);
  }
  if (threadIdx.x == 0) {
    m[row] = mx;
    den[row] = dn;
    ln.mean[row] = mu;
    ln.rstd[row] = rs;
  }
}

// Split units of the fused forward, one wavefront per unit, after the fixup:
// alpha = exp(v - m_k) * exp(m_k - m) / den.  Launched over the first n_slots
// units, which gr_spmm_plan fills with the split rows' units (unit k holds
// slot k).
__global__ __launch_bounds__(256) void gat_fused_alpha_split(const int4* __restrict__ units,
                                                             int64_t n_split,
                                                             const float* __restrict__ m,
                                                             const float* __restrict__ den,
                                                             const float* __restrict__ ws,
                                                             int64_t ws_stride,
                                                             float* __restrict__ alpha) {
  const int lane = threadIdx.x & 63;
  const int64_t wid = wave_id();
  if (wid >= n_split) return;
  const int4 w = units[wid];
  if (w.w < 0) return;
  const float corr = expf(ws[(int64_t)w.w * ws_stride + ws_stride - 4] - m[w.x]);
  const float dn = den[w.x];
  for (int e = w.y + lane; e < w.z; e += 64) alpha[e] = (alpha[e] * corr) / dn;
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
using gr_wave::group_sum;

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
  for (int ch = 0; ch < NCH; ++ch) {
    dsl[ch] = gr_wave::slot_sum<G>(dsl[ch]);
#pragma unroll
    for (int q = 0; q < VEC; ++q) acc[ch][q] = gr_wave::slot_sum<G>(acc[ch][q]);
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

// With src_rows the row goes to dhs row src_rows[row] and is added to what
// that row holds (accumulate into a gradient matrix of all partitions' rows).
__global__ __launch_bounds__(256) void gat_bwd_src_fixup(const int32_t* __restrict__ fix,
                                                         int64_t n_fix,
                                                         const float* __restrict__ ws, int H,
                                                         int C, const float* __restrict__ att_src,
                                                         float* __restrict__ dhs,
                                                         float* __restrict__ ds,
                                                         const int32_t* __restrict__ src_rows) {
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
    const float v = fmaf(dsum, att_src[f], acc);
    if (src_rows != nullptr) {
      dhs[(int64_t)src_rows[row] * HC + f] += v;
    } else {
      dhs[(int64_t)row * HC + f] = v;
    }
    if (f == h * C) ds[(int64_t)row * H + h] = dsum;
  }
}

// One head: the same pass as gat_bwd_src_kernel with the per-edge scalars
// batched.  For each 64-edge chunk of the unit, lane l loads edge l's
// destination row, CSR position, alpha, d and cdot (two coalesced loads and
// three gathers, all issued before the chunk's go-row loads), and the
// wavefront takes them from the owning lane (readlane when the whole
// wavefront works on one edge, a cross-lane permute for G-lane edge slots).
// The chunk's gdd values are collected in lane l and stored once, after the
// chunk's row loads have been consumed: on gfx9 a wait for a load also waits
// for every store issued before it.  Edges are assigned to slots and summed
// in the same order as in gat_bwd_src_kernel.
//
// ATT: the wavefront also forms its share of the attention-vector gradient
// datt_src = sum_j ds_j Hs_j while Hs_j is in its registers.  The grid is
// then `waves` wavefronts (at most what the GPU holds at once); wavefront w
// takes units w, w + waves, w + 2 waves, ..., adds each unit's (partial) ds
// times Hs_j to its own sum, and writes that sum to att_part[w]; the caller
// reduces the rows of att_part in order.  The result does not depend on
// scheduling.  A split column's share is formed per unit from its partial ds
// (the sum over its units is the same quantity, re-associated).
//
// With rec (not NULL): instead of alpha (through the CSC -> CSR permutation),
// d and cdot, each edge reads its destination's record rec[i] = (d_i, m_i,
// den_i, c_i) (one 16-byte load, where the three gathers cost a 128-byte line
// each) and forms alpha_ij = exp(LeakyReLU(s_j + d_i) - m_i) / den_i, the
// forward's own expression: for a whole row it gives the forward's bits.
template <int VEC, int G, int NCH, int U, bool ATT>
__global__ __launch_bounds__(256) void gat_bwd_src_h1(
    const int4* __restrict__ units, int64_t n_units, const int32_t* __restrict__ row_idx,
    const int32_t* __restrict__ perm, const float* __restrict__ hs, int64_t ldh,
    const float* __restrict__ go, const float* __restrict__ s, const float* __restrict__ d,
    const float* __restrict__ alpha, const float* __restrict__ cdot,
    const float4* __restrict__ rec,
    const float* __restrict__ att_src, int C, float* __restrict__ dhs, float* __restrict__ ds,
    float* __restrict__ gt, float* __restrict__ ws, int min_len,
    const int32_t* __restrict__ src_rows, float* __restrict__ att_part, int64_t waves) {
  constexpr int EPI = 64 / G;
  const int lane = threadIdx.x & 63;
  const int slot = (EPI == 1) ? 0 : lane / G;
  const int sub = (EPI == 1) ? lane : lane % G;
  const int64_t first = wave_id();
  if (first >= n_units || (ATT && first >= waves)) return;
  int foff[NCH];
  bool fvalid[NCH];
  float att[NCH][VEC];
#pragma unroll
  for (int ch = 0; ch < NCH; ++ch) {
    foff[ch] = (ch * G + sub) * VEC;
    fvalid[ch] = foff[ch] < C;
#pragma unroll
    for (int q = 0; q < VEC; ++q) att[ch][q] = 0.f;
  }
  const int64_t stride = ATT ? waves : n_units;
  for (int64_t wid = first; wid < n_units; wid += stride) {
    const int4 w = units[wid];
    // Whole columns shorter than min_len are gat_bwd_src_rows' work.
    if (w.w < 0 && w.z - w.y < min_len) continue;
    const int64_t j = w.x;
    // With src_rows, column j's rows of Hs, s and dHs are row src_rows[j] of
    // matrices of all partitions' rows, and dHs is added to, not written.
    const int64_t jr = src_rows != nullptr ? (int64_t)src_rows[j] : j;

    int fld[NCH];
    float hsj[NCH][VEC];
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) {
      fld[ch] = fvalid[ch] ? foff[ch] : C - VEC;
      ld<VEC>(hs + jr * ldh + fld[ch], hsj[ch]);
      if (!fvalid[ch]) {
#pragma unroll
        for (int q = 0; q < VEC; ++q) hsj[ch][q] = 0.f;
      }
    }
    const float sj = s[jr];
    float acc[NCH][VEC];
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch)
#pragma unroll
      for (int q = 0; q < VEC; ++q) acc[ch][q] = 0.f;
    float dsl = 0.f;

    for (int b = w.y; b < w.z; b += 64) {
      const int n = min(64, w.z - b);
      const int el = b + min(lane, n - 1);
      const int il = row_idx[el];
      const int pl = perm[el];
      float al, dl, cl;
      if (rec != nullptr) {
        const float4 r = rec[il];
        dl = r.x;
        cl = r.w;
        al = expf(leaky(sj + dl) - r.y) / r.z;
      } else {
        al = alpha[pl];
        dl = d[il];
        cl = cdot[il];
      }
      float gtv = 0.f;
      for (int k = 0; k < n; k += EPI * U) {
        int ii[U];
        float a[U], dv[U], cv[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          if constexpr (EPI == 1) {
            ii[u] = __builtin_amdgcn_readlane(il, k + u);
            a[u] = __builtin_bit_cast(float,
                                      __builtin_amdgcn_readlane(__builtin_bit_cast(int, al), k + u));
            dv[u] = __builtin_bit_cast(float,
                                       __builtin_amdgcn_readlane(__builtin_bit_cast(int, dl), k + u));
            cv[u] = __builtin_bit_cast(float,
                                       __builtin_amdgcn_readlane(__builtin_bit_cast(int, cl), k + u));
          } else {
            const int t = k + u * EPI + slot;
            ii[u] = __shfl(il, t, 64);
            a[u] = __shfl(al, t, 64);
            dv[u] = __shfl(dl, t, 64);
            cv[u] = __shfl(cl, t, 64);
          }
        }
        float g[U][NCH][VEC];
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
          for (int ch = 0; ch < NCH; ++ch) ld<VEC>(go + (int64_t)ii[u] * C + fld[ch], g[u][ch]);
#pragma unroll
        for (int u = 0; u < U; ++u) {
          float t = 0.f;
#pragma unroll
          for (int ch = 0; ch < NCH; ++ch)
#pragma unroll
            for (int q = 0; q < VEC; ++q) t = fmaf(g[u][ch][q], hsj[ch][q], t);
          const float ga = gr_wave::group_sum<G>(t);
          const float ge = a[u] * (ga - cv[u]);
          const bool pos = sj + dv[u] > 0.f;
          const int te = k + u * EPI + slot;  // this slot's edge in the chunk
          if (te < n) {
            dsl += pos ? ge : 0.2f * ge;
#pragma unroll
            for (int ch = 0; ch < NCH; ++ch)
#pragma unroll
              for (int q = 0; q < VEC; ++q) acc[ch][q] = fmaf(a[u], g[u][ch][q], acc[ch][q]);
          }
          const float gv = pos ? 0.f : -0.8f * ge;
          // Lane k + u * EPI + s collects the value of slot s.
          const int src = lane - k - u * EPI;
          if constexpr (EPI == 1) {
            if (src == 0) gtv = gv;
          } else {
            const float v = __shfl(gv, (src & (EPI - 1)) * G, 64);
            if (src >= 0 && src < EPI) gtv = v;
          }
        }
      }
      if (lane < n) gt[pl] = gtv;
    }

    dsl = gr_wave::slot_sum<G>(dsl);
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch)
#pragma unroll
      for (int q = 0; q < VEC; ++q) acc[ch][q] = gr_wave::slot_sum<G>(acc[ch][q]);
    if constexpr (ATT) {
#pragma unroll
      for (int ch = 0; ch < NCH; ++ch)
#pragma unroll
        for (int q = 0; q < VEC; ++q) att[ch][q] = fmaf(dsl, hsj[ch][q], att[ch][q]);
    }
    if (slot == 0) {
      if (w.w < 0) {
#pragma unroll
        for (int ch = 0; ch < NCH; ++ch) {
          if (!fvalid[ch]) continue;
          float av[VEC];
          ld<VEC>(att_src + foff[ch], av);
#pragma unroll
          for (int q = 0; q < VEC; ++q) av[q] = fmaf(dsl, av[q], acc[ch][q]);
          if (src_rows != nullptr) {
            float old[VEC];
            ld<VEC>(dhs + jr * C + foff[ch], old);
#pragma unroll
            for (int q = 0; q < VEC; ++q) av[q] += old[q];
            st<VEC>(dhs + jr * C + foff[ch], av);
          } else {
            st<VEC>(dhs + j * C + foff[ch], av);
          }
        }
        if (lane == 0) ds[j] = dsl;
      } else {
        // Slot layout [acc (C) | ds], each part padded to 4 floats.
        const int c4 = ((C + 3) / 4) * 4;
        float* p = ws + (int64_t)w.w * (c4 + 4);
#pragma unroll
        for (int ch = 0; ch < NCH; ++ch)
          if (fvalid[ch]) st<VEC>(p + foff[ch], acc[ch]);
        if (lane == 0) p[c4] = dsl;
      }
    }
  }  // units of this wavefront
  if constexpr (ATT) {
    if (slot == 0) {
      float* p = att_part + first * C;
#pragma unroll
      for (int ch = 0; ch < NCH; ++ch)
        if (fvalid[ch]) st<VEC>(p + foff[ch], att[ch]);
    }
  }
}

// ------------------------------------------------- narrow single-head rows --
//
// One head of at most G * VEC channels (G <= 16): 64 / G whole plan units
// per wavefront, one per group of G lanes, each lane owning VEC channels.  A
// wavefront per unit would spend most of its time in the dependent loads
// that start a unit, for a handful of short gathers (C5's 20-wide layer has
// 13 edges per destination row and 4.4 per source column); here 64 / G
// units share that latency.  The members of a wavefront are stepped to the
// longest member's length, so the group reductions (DPP within 16-lane rows)
// and the shuffles always run with every lane active; loads and stores of
// edges past a member's end are masked.  The plan lists whole units by
// length class, so the members have similar lengths.

// Longest unit of the wavefront (every lane gets it).
__device__ __forceinline__ int wave_longest(int len) {
  return (int)gr_wave::wave_max((float)len);
}

// Forward: softmax statistics over the row, then the aggregation
// O_i = sum_e alpha_e Hs[col_e]; alpha, m, den and O as gat_fwd_fused writes
// them for a whole row.  Lane sub of a group holds edges sub, G + sub, ...
// of at most R * G: their column ids and logits are loaded once and kept in
// registers, so a row costs one dependent index load, one logit load and one
// round of U-wide row gathers per G edges.  Longer rows are left to
// gat_fwd_fused.
template <int VEC, int G, int R, int U>
__global__ __launch_bounds__(256) void gat_fwd_rows(
    const int4* __restrict__ units, int64_t n_units, const int32_t* __restrict__ idx,
    const float* __restrict__ hs, int64_t ldh, const float* __restrict__ s,
    const float* __restrict__ d, int C, const float* __restrict__ bias, float* __restrict__ m,
    float* __restrict__ den, float* __restrict__ alpha, float* __restrict__ o,
    float* __restrict__ y, int64_t ldy) {
  constexpr int RPW = 64 / G;
  const int lane = threadIdx.x & 63;
  const int grp = lane / G, sub = lane % G, base = grp * G;
  const int64_t wid = wave_id();
  if (wid * RPW >= n_units) return;
  const int64_t u = wid * RPW + grp;
  const int4 wu = u < n_units ? units[u] : make_int4(0, 0, 0, -1);
  const bool active = u < n_units && wu.z - wu.y <= R * G;
  const int4 w = active ? wu : make_int4(0, 0, 0, -1);
  const int64_t i = w.x;
  const int len = w.z - w.y;
  const int steps = wave_longest(len);
  const int foff = sub * VEC;
  const bool fvalid = foff < C;
  const int fld = fvalid ? foff : C - VEC;
  const float di = len > 0 ? d[i] : 0.f;

  int cr[R];
  float vr[R];
#pragma unroll
  for (int r = 0; r < R; ++r) cr[r] = r * G + sub < len ? idx[w.y + r * G + sub] : 0;
  // The first U row gathers need only column ids: they go out before the
  // logits, so the two loads' latencies overlap.
  float rp[U][VEC];
#pragma unroll
  for (int q = 0; q < U; ++q) {
    const int c = __shfl(cr[0], base + q, 64);
    if (q < len) {
      ld<VEC>(hs + (int64_t)c * ldh + fld, rp[q]);
    } else {
#pragma unroll
      for (int v = 0; v < VEC; ++v) rp[q][v] = 0.f;
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r)
    vr[r] = r * G + sub < len ? leaky(s[cr[r]] + di) : -FLT_MAX;

  // Pass 1: max, then the sum of exp(v - max).
  float mx = vr[0];
#pragma unroll
  for (int r = 1; r < R; ++r) mx = fmaxf(mx, vr[r]);
  mx = gr_wave::group_max<G>(mx);
  float sum = 0.f;
#pragma unroll
  for (int r = 0; r < R; ++r)
    if (r * G + sub < len) sum += expf(vr[r] - mx);
  sum = gr_wave::group_sum<G>(sum);
  const float dn = sum + 1e-16f;

  // Pass 2: the group takes edge k + q's column and weight from lane q.
  float acc[VEC];
#pragma unroll
  for (int q = 0; q < VEC; ++q) acc[q] = 0.f;
  auto gather = [&](int k, int cl, float al) {
    const int n = min(G, steps - k);
    for (int q0 = 0; q0 < n; q0 += U) {
      int c[U];
      float a[U];
#pragma unroll
      for (int q = 0; q < U; ++q) {
        const int src = base + min(q0 + q, G - 1);
        c[q] = __shfl(cl, src, 64);
        const float aq = __shfl(al, src, 64);
        a[q] = k + q0 + q < len ? aq : 0.f;
      }
      float rr[U][VEC];
#pragma unroll
      for (int q = 0; q < U; ++q) {
        if (k + q0 == 0) {
#pragma unroll
          for (int v = 0; v < VEC; ++v) rr[q][v] = rp[q][v];
        } else if (k + q0 + q < len) {
          ld<VEC>(hs + (int64_t)c[q] * ldh + fld, rr[q]);
        } else {
#pragma unroll
          for (int v = 0; v < VEC; ++v) rr[q][v] = 0.f;
        }
      }
#pragma unroll
      for (int q = 0; q < U; ++q)
#pragma unroll
        for (int v = 0; v < VEC; ++v) acc[v] = fmaf(a[q], rr[q][v], acc[v]);
    }
  };
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int k = r * G;
    if (k >= steps) break;
    const bool ok = k + sub < len;
    const float al = ok ? expf(vr[r] - mx) / dn : 0.f;
    gather(k, cr[r], al);
    if (ok && alpha != nullptr) alpha[w.y + k + sub] = al;
  }

  if (!active) return;
  if (sub == 0) {
    m[i] = len > 0 ? mx : 0.f;
    den[i] = len > 0 ? dn : 1.f;
  }
  if (!fvalid) return;
  st<VEC>(o + i * C + foff, acc);
  if (y != nullptr) {
    float b[VEC];
    if (bias != nullptr) {
      ld<VEC>(bias + foff, b);
    } else {
#pragma unroll
      for (int q = 0; q < VEC; ++q) b[q] = 0.f;
    }
#pragma unroll
    for (int q = 0; q < VEC; ++q) b[q] += acc[q];
    st<VEC>(y + i * ldy + foff, b);
  }
}

// Backward, column-parallel (CSC) over source rows j: for each edge (i, j),
// g_alpha = <GO_i, Hs_j> (a group sum), g_e = alpha (g_alpha - c_i),
// ds_j += slope * g_e, dHs_j += alpha GO_i; the destination part of g_t is
// collected in the lane that owns the edge and stored at its CSR position.
// Writes dHs_j = acc + ds_j att_src and ds_j, as gat_bwd_src_h1 does for a
// whole column.  Columns of more than max_len edges are left to
// gat_bwd_src_h1.
// With rec (not NULL): the destination records instead of alpha, d and
// cdot, as in gat_bwd_src_h1.
template <int VEC, int G, int U>
__global__ __launch_bounds__(256) void gat_bwd_src_rows(
    const int4* __restrict__ units, int64_t n_units, const int32_t* __restrict__ row_idx,
    const int32_t* __restrict__ perm, const float* __restrict__ hs, int64_t ldh,
    const float* __restrict__ go, const float* __restrict__ s, const float* __restrict__ d,
    const float* __restrict__ alpha, const float* __restrict__ cdot,
    const float4* __restrict__ rec,
    const float* __restrict__ att_src, int C, float* __restrict__ dhs, float* __restrict__ ds,
    float* __restrict__ gt, int max_len) {
  constexpr int RPW = 64 / G;
  const int lane = threadIdx.x & 63;
  const int grp = lane / G, sub = lane % G, base = grp * G;
  const int64_t wid = wave_id();
  if (wid * RPW >= n_units) return;
  const int64_t u = wid * RPW + grp;
  const int4 wu = u < n_units ? units[u] : make_int4(0, 0, 0, -1);
  const bool active = u < n_units && wu.z - wu.y <= max_len;
  const int4 w = active ? wu : make_int4(0, 0, 0, -1);
  const int64_t j = w.x;
  const int len = w.z - w.y;
  const int steps = wave_longest(len);
  const int foff = sub * VEC;
  const bool fvalid = foff < C;
  const int fld = fvalid ? foff : C - VEC;

  float hsj[VEC];
  if (active && fvalid) {
    ld<VEC>(hs + j * ldh + fld, hsj);
  } else {
#pragma unroll
    for (int q = 0; q < VEC; ++q) hsj[q] = 0.f;
  }
  const float sj = active ? s[j] : 0.f;
  float acc[VEC];
#pragma unroll
  for (int q = 0; q < VEC; ++q) acc[q] = 0.f;
  float dsl = 0.f;

  for (int k = 0; k < steps; k += G) {
    const int t = k + sub;
    const bool ok = t < len;
    int il = 0, pl = 0;
    float al = 0.f, dl = 0.f, cl = 0.f;
    if (ok) {
      il = row_idx[w.y + t];
      pl = perm[w.y + t];
      if (rec != nullptr) {
        const float4 r = rec[il];
        dl = r.x;
        cl = r.w;
        al = expf(leaky(sj + dl) - r.y) / r.z;
      } else {
        al = alpha[pl];
        dl = d[il];
        cl = cdot[il];
      }
    }
    float gtv = 0.f;
    const int n = min(G, steps - k);
    for (int q0 = 0; q0 < n; q0 += U) {
      // The row gathers need only the destination ids: they go out before
      // the per-edge scalars are shuffled (which waits for their loads).
      float g[U][VEC];
#pragma unroll
      for (int q = 0; q < U; ++q) {
        const int iq = __shfl(il, base + min(q0 + q, G - 1), 64);
        if (k + q0 + q < len) {
          ld<VEC>(go + (int64_t)iq * C + fld, g[q]);
        } else {
#pragma unroll
          for (int v = 0; v < VEC; ++v) g[q][v] = 0.f;
        }
      }
      float a[U], dv[U], cv[U];
#pragma unroll
      for (int q = 0; q < U; ++q) {
        const int src = base + min(q0 + q, G - 1);
        a[q] = __shfl(al, src, 64);
        dv[q] = __shfl(dl, src, 64);
        cv[q] = __shfl(cl, src, 64);
      }
#pragma unroll
      for (int q = 0; q < U; ++q) {
        float tdot = 0.f;
#pragma unroll
        for (int v = 0; v < VEC; ++v) tdot = fmaf(g[q][v], hsj[v], tdot);
        const float ga = gr_wave::group_sum<G>(tdot);
        const bool valid = q0 + q < n && k + q0 + q < len;
        const float ge = valid ? a[q] * (ga - cv[q]) : 0.f;
        const bool pos = sj + dv[q] > 0.f;
        dsl += pos ? ge : 0.2f * ge;
#pragma unroll
        for (int v = 0; v < VEC; ++v) acc[v] = fmaf(valid ? a[q] : 0.f, g[q][v], acc[v]);
        if (sub == q0 + q) gtv = pos ? 0.f : -0.8f * ge;
      }
    }
    if (ok) gt[pl] = gtv;
  }

  if (!active) return;
  if (fvalid) {
    float av[VEC];
    ld<VEC>(att_src + foff, av);
#pragma unroll
    for (int q = 0; q < VEC; ++q) av[q] = fmaf(dsl, av[q], acc[q]);
    st<VEC>(dhs + j * C + foff, av);
  }
  if (sub == 0) ds[j] = dsl;
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

// One head: the same sums, 64 / G units per wavefront (G lanes each, VEC
// floats a lane, NCH chunks of G * VEC floats).  The row's dHs, att_dst, c_i
// and den_i do not depend on the edge sum, so they are loaded first and their
// latency overlaps the g_t loads; the edge loop keeps four loads in flight.
template <int VEC, int G, int NCH>
__global__ __launch_bounds__(256) void gat_bwd_dst_h1(
    const int4* __restrict__ units, int64_t n_units, const float* __restrict__ gt, int C,
    const float* __restrict__ att_dst, const float* __restrict__ cdot,
    const float* __restrict__ den, float* __restrict__ dd, float* __restrict__ dhs,
    float* __restrict__ ws) {
  constexpr int RPW = 64 / G;
  const int lane = threadIdx.x & 63;
  const int grp = lane / G, sub = lane % G;
  const int64_t wid = wave_id();
  if (wid * RPW >= n_units) return;
  const int64_t u = wid * RPW + grp;
  const bool active = u < n_units;
  const int4 w = active ? units[u] : make_int4(0, 0, 0, -1);
  const bool whole = active && w.w < 0;
  const int64_t i = w.x;

  int foff[NCH];
  bool fvalid[NCH];
  float hv[NCH][VEC], av[NCH][VEC];
#pragma unroll
  for (int ch = 0; ch < NCH; ++ch) {
    foff[ch] = (ch * G + sub) * VEC;
    fvalid[ch] = foff[ch] < C;
    const int fld = fvalid[ch] ? foff[ch] : C - VEC;
    if (whole) {
      ld<VEC>(dhs + i * C + fld, hv[ch]);
      ld<VEC>(att_dst + fld, av[ch]);
    } else {
#pragma unroll
      for (int q = 0; q < VEC; ++q) hv[ch][q] = av[ch][q] = 0.f;
    }
  }
  const float ci = whole ? cdot[i] : 0.f;
  const float dn = whole ? den[i] : 1.f;

  float p = 0.f;
#pragma unroll 4
  for (int e = w.y + sub; e < w.z; e += G) p += gt[e];
  p = gr_wave::group_sum<G>(p);
  if (!active) return;
  if (whole) {
    const float v = p + ci * (1e-16f / dn);
    if (sub == 0) dd[i] = v;
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) {
      if (!fvalid[ch]) continue;
      float o[VEC];
#pragma unroll
      for (int q = 0; q < VEC; ++q) o[q] = fmaf(v, av[ch][q], hv[ch][q]);
      st<VEC>(dhs + i * C + foff[ch], o);
    }
  } else if (sub == 0) {
    ws[w.w] = p;
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

extern "C" int gr_gat_row_dot(const float* a, int64_t lda, const float* b, int64_t ldb,
                              int64_t rows, int64_t heads, int64_t channels, float* out,
                              void* stream) {
  gr::clear_error();
  int rc = check_heads(heads, channels);
  if (rc) return rc;
  GR_REQUIRE(rows >= 0, "gat_row_dot: negative row count");
  GR_REQUIRE(lda >= heads * channels && ldb >= heads * channels, "gat_row_dot: bad leading dims");
  if (rows == 0) return GR_OK;
  GR_REQUIRE(a && b && out, "gat_row_dot: NULL pointer");
  const int64_t HC = heads * channels;
  const bool al = aligned16(a) && aligned16(b) && lda % 4 == 0 && ldb % 4 == 0;
  int vec, nch;
  pick_shape(HC, channels, al, &vec, &nch);
  hipStream_t st = gr::as_stream(stream);
  const int H = (int)heads, C = (int)channels;
  auto grid = [&](int u) {
    const int64_t waves = (rows + u - 1) / u;
    return dim3((unsigned)std::min<int64_t>(4096, (waves + 3) / 4));
  };
#define GR_RD(V, N, U)                                                                 \
  hipLaunchKernelGGL((gat_row_dot_kernel<V, N, U>), grid(U), dim3(256), 0, st, a, lda, b, ldb, \
                     rows, H, C, out)
  if (vec == 4) {
    if (nch == 1) GR_RD(4, 1, 4); else if (nch == 2) GR_RD(4, 2, 2); else GR_RD(4, 4, 1);
  } else {
    if (nch == 1) GR_RD(1, 1, 4); else if (nch == 2) GR_RD(1, 2, 2); else if (nch == 4) GR_RD(1, 4, 1);
    else if (nch == 8) GR_RD(1, 8, 1); else GR_RD(1, 16, 1);
  }
#undef GR_RD
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
  // The GCN kernel takes rows of up to 256 vectors: any C <= 256, wider rows
  // only as float4 vectors.
  const bool gcn_ok = C <= 256 || (C % 4 == 0 && aligned16(hs) && ldh % 4 == 0 && aligned16(o) &&
                                   (workspace == nullptr || aligned16(workspace)));
  if (H == 1 && gcn_ok) {
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

template <int VEC, int G, int NCH>
static hipError_t launch_fused(hipStream_t st, const int4* units, int64_t n_units,
                               const int32_t* idx, const float* hs, int64_t ldh, const float* s,
                               const float* d, int C, const float* bias, float* m, float* den,
                               float* alpha, float* o, float* y, int64_t ldy, float* ws,
                               int64_t ws_stride, int min_len, const GatLn& ln) {
  constexpr int EPI = 64 / G;
  // Narrow rows (4 or more edge slots of at most 16 lanes) keep 4 edges a
  // slot in flight: with the unit's logits in registers this measured faster
  // than 8 (5.58 against 5.75 ms for the 20-wide forward of C5's 64
  // partitions) and than 2 (5.98 ms).
  constexpr int U = (EPI == 1) ? ((NCH == 1) ? 8 : (NCH == 2 ? 4 : 2)) : 4;
  hipLaunchKernelGGL((gat_fwd_fused<VEC, G, NCH, U>), dim3(blocks_for(n_units)), dim3(256), 0,
                     st, units, n_units, idx, hs, ldh, s, d, C, bias, m, den, alpha, o, y, ldy,
                     ws, ws_stride, min_len, ln);
  return hipGetLastError();
}

template <int VEC>
static hipError_t dispatch_fused(int chunks, hipStream_t st, const int4* units, int64_t n_units,
                                 const int32_t* idx, const float* hs, int64_t ldh,
                                 const float* s, const float* d, int C, const float* bias,
                                 float* m, float* den, float* alpha, float* o, float* y,
                                 int64_t ldy, float* ws, int64_t ws_stride, int min_len = 0,
                                 const GatLn& ln = GatLn{}) {
#define GR_FU(G, N)                                                                       \
  return launch_fused<VEC, G, N>(st, units, n_units, idx, hs, ldh, s, d, C, bias, m, den, \
                                 alpha, o, y, ldy, ws, ws_stride, min_len, ln)
  if (chunks <= 8) GR_FU(8, 1);
  if (chunks <= 16) GR_FU(16, 1);
  if (chunks <= 32) GR_FU(32, 1);
  if (chunks <= 64) GR_FU(64, 1);
  if (chunks <= 128) GR_FU(64, 2);
  GR_FU(64, 4);
#undef GR_FU
}

template <int VEC>
static hipError_t launch_fwd_rows(int chunks, hipStream_t st, const int4* units, int64_t n,
                                  const int32_t* idx, const float* hs, int64_t ldh,
                                  const float* s, const float* d, int C, const float* bias,
                                  float* m, float* den, float* alpha, float* o, float* y,
                                  int64_t ldy);

// Longest whole row gat_fwd_rows takes (R * G of the instance launch_fwd_rows
// picks for `chunks`).
constexpr int fwd_rows_max_len(int chunks) { return chunks <= 4 ? 16 : 32; }

// Longest whole column gat_bwd_src_rows takes.
constexpr int kBwdRowsMaxLen = 32;

extern "C" int gr_gat_forward(const int32_t* units, int64_t n_units, const int32_t* fixups,
                              int64_t n_fix, const int32_t* idx, const float* hs, int64_t ldh,
                              const float* s, const float* d, int64_t n_dst, int64_t heads,
                              int64_t channels, const float* bias, float* m, float* den,
                              float* alpha, float* o, float* y, int64_t ldy, float* workspace,
                              int64_t ws_floats, int64_t n_slots, void* stream) {
  gr::clear_error();
  int rc = check_heads(heads, channels);
  if (rc) return rc;
  const int64_t HC = heads * channels;
  GR_REQUIRE(n_units >= 0 && n_fix >= 0 && n_slots >= 0 && n_dst >= 0,
             "gat_forward: negative extent");
  GR_REQUIRE(ldh >= HC && (y == nullptr || ldy >= HC), "gat_forward: bad leading dims");
  const int64_t hc4 = (HC + 3) / 4 * 4;
  const int64_t need = n_slots * (hc4 + (2 * heads + 3) / 4 * 4);
  GR_REQUIRE(n_fix == 0 || (fixups && workspace && ws_floats >= need),
             "gat_forward: workspace of %lld floats, %lld needed",
             (long long)ws_floats, (long long)need);
  if (n_units == 0) return GR_OK;
  GR_REQUIRE(units && aligned16(units) && idx && hs && s && d && m && den && o &&
                 (alpha != nullptr || heads == 1),
             "gat_forward: NULL or misaligned pointer (alpha may be NULL for one head)");
  hipStream_t st = gr::as_stream(stream);
  if (heads > 1) {
    // Several heads: statistics, then the aggregation.
    rc = gr_gat_softmax_stats(units, n_units, fixups, n_fix, idx, s, d, heads, m, den, alpha,
                              workspace, n_slots, stream);
    if (rc) return rc;
    return gr_gat_aggregate(units, n_units, fixups, n_fix, idx, hs, ldh, alpha, n_dst, heads,
                            channels, bias, o, y, ldy, workspace, n_slots, stream);
  }
  const int C = (int)channels;
  const bool al = aligned16(hs) && ldh % 4 == 0 && aligned16(o) &&
                  (y == nullptr || (aligned16(y) && ldy % 4 == 0)) &&
                  (bias == nullptr || aligned16(bias)) &&
                  (workspace == nullptr || aligned16(workspace));
  const int vec = (C % 4 == 0 && al) ? 4 : 1;
  const int chunks = (C + vec - 1) / vec;
  const int64_t ws_stride = hc4 + 4;
  const int4* u4 = reinterpret_cast<const int4*>(units);
  hipError_t err;
  if (chunks <= 16) {
    // Narrow: split rows and long whole rows one per wavefront
    // (gat_fwd_fused), the other whole rows several per wavefront
    // (gat_fwd_rows, after the plan's first n_slots units, the split ones).
    const int64_t n_split = std::min(n_slots, n_units);
    const int min_len = fwd_rows_max_len(chunks) + 1;
    if (vec == 4)
      err = dispatch_fused<4>(chunks, st, u4, n_units, idx, hs, ldh, s, d, C, bias, m, den,
                              alpha, o, y, ldy, workspace, ws_stride, min_len);
    else
      err = dispatch_fused<1>(chunks, st, u4, n_units, idx, hs, ldh, s, d, C, bias, m, den,
                              alpha, o, y, ldy, workspace, ws_stride, min_len);
    GR_HIP_CHECK(err);
    if (n_units > n_split) {
      if (vec == 4)
        err = launch_fwd_rows<4>(chunks, st, u4 + n_split, n_units - n_split, idx, hs, ldh, s, d,
                                 C, bias, m, den, alpha, o, y, ldy);
      else
        err = launch_fwd_rows<1>(chunks, st, u4 + n_split, n_units - n_split, idx, hs, ldh, s, d,
                                 C, bias, m, den, alpha, o, y, ldy);
    }
  } else if (vec == 4) {
    err = dispatch_fused<4>(chunks, st, u4, n_units, idx, hs, ldh, s, d, C, bias, m, den, alpha,
                            o, y, ldy, workspace, ws_stride);
  } else if (chunks <= 256) {
    err = dispatch_fused<1>(chunks, st, u4, n_units, idx, hs, ldh, s, d, C, bias, m, den, alpha,
                            o, y, ldy, workspace, ws_stride);
  } else {
    // Unaligned rows wider than 256 floats: statistics, then the aggregation.
    GR_REQUIRE(alpha != nullptr, "gat_forward: unaligned rows wider than 256 floats need alpha");
    rc = gr_gat_softmax_stats(units, n_units, fixups, n_fix, idx, s, d, 1, m, den, alpha,
                              workspace, n_slots, stream);
    if (rc) return rc;
    return gr_gat_aggregate(units, n_units, fixups, n_fix, idx, hs, ldh, alpha, n_dst, 1,
                            channels, bias, o, y, ldy, workspace, n_slots, stream);
  }
  GR_HIP_CHECK(err);
  if (n_fix > 0) {
    GR_REQUIRE(n_fix <= INT32_MAX && n_slots <= n_units, "gat_forward: inconsistent plan");
    hipLaunchKernelGGL(gat_fused_fixup, dim3((unsigned)n_fix, (unsigned)((C + 255) / 256)),
                       dim3(256), 0, st, fixups, workspace, ws_stride, C, bias, m, den, o, y,
                       ldy);
    GR_HIP_CHECK(hipGetLastError());
    if (alpha != nullptr) {
      hipLaunchKernelGGL(gat_fused_alpha_split, dim3(blocks_for(n_slots)), dim3(256), 0, st, u4,
                         n_slots, m, den, workspace, ws_stride, alpha);
      GR_HIP_CHECK(hipGetLastError());
    }
  }
  return GR_OK;
}

extern "C" int gr_gat_forward_ln(const int32_t* units, int64_t n_units, const int32_t* fixups,
                                 int64_t n_fix, const int32_t* idx, const float* hs,
                                 int64_t ldh, const float* s, const float* d, int64_t n_dst,
                                 int64_t channels, const float* bias, const float* gamma,
                                 const float* beta, float eps, int32_t act, float* m, float* den,
                                 float* h, float* out, int64_t ldo, float* mean, float* rstd,
                                 float* workspace, int64_t ws_floats, int64_t n_slots,
                                 void* stream) {
  gr::clear_error();
  const int64_t C = channels;
  GR_REQUIRE(C % 4 == 0 && C > 128 && C <= 1024,
             "gat_forward_ln: one head of 132..1024 channels, a multiple of 4");
  GR_REQUIRE(act == GR_ACT_RELU || act == GR_ACT_ELU, "gat_forward_ln: unknown activation %d",
             (int)act);
  GR_REQUIRE(n_units >= 0 && n_fix >= 0 && n_slots >= 0 && n_dst >= 0,
             "gat_forward_ln: negative extent");
  GR_REQUIRE(ldh >= C && ldh % 4 == 0 && ldo >= C && ldo % 4 == 0,
             "gat_forward_ln: bad leading dims");
  const int64_t ws_stride = C + 4;
  GR_REQUIRE(n_fix == 0 || (fixups && workspace && ws_floats >= n_slots * ws_stride &&
                            n_slots <= n_units),
             "gat_forward_ln: workspace of %lld floats, %lld needed", (long long)ws_floats,
             (long long)(n_slots * ws_stride));
  if (n_units == 0) return GR_OK;
  GR_REQUIRE(units && aligned16(units) && idx && hs && aligned16(hs) && s && d && m && den &&
                 gamma && aligned16(gamma) && beta && aligned16(beta) && h && aligned16(h) &&
                 out && aligned16(out) && mean && rstd && (bias == nullptr || aligned16(bias)) &&
                 (workspace == nullptr || aligned16(workspace)),
             "gat_forward_ln: NULL or misaligned pointer");
  hipStream_t st = gr::as_stream(stream);
  GatLn ln;
  ln.gamma = gamma;
  ln.beta = beta;
  ln.eps = eps;
  ln.act = act;
  ln.h = h;
  ln.mean = mean;
  ln.rstd = rstd;
  const int4* u4 = reinterpret_cast<const int4*>(units);
  GR_HIP_CHECK(dispatch_fused<4>((int)(C / 4), st, u4, n_units, idx, hs, ldh, s, d, (int)C, bias,
                                 m, den, nullptr, nullptr, out, ldo, workspace, ws_stride, 0,
                                 ln));
  if (n_fix > 0) {
    GR_REQUIRE(n_fix <= INT32_MAX, "gat_forward_ln: too many split rows");
    hipLaunchKernelGGL(gat_fused_fixup_ln, dim3((unsigned)n_fix), dim3(256), 0, st, fixups,
                       workspace, ws_stride, (int)C, bias, m, den, ln, out, ldo);
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

// Wavefronts of gat_bwd_src_h1<VEC, G, NCH, U, true> the current device holds
// at once (the kernel's occupancy times the CUs), counted once per device;
// 0 when the query fails.
template <int VEC, int G, int NCH, int U>
static int64_t resident_waves_h1() {
  constexpr int kDevices = 64;
  static std::atomic<int64_t> cached[kDevices];
  int dev = 0, cus = 0, blocks = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
  if (dev < kDevices) {
    const int64_t c = cached[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(
          &blocks, gat_bwd_src_h1<VEC, G, NCH, U, true>, 256, 0) != hipSuccess ||
      cus <= 0 || blocks <= 0)
    return 0;
  const int64_t waves = (int64_t)cus * blocks * 4;
  if (dev < kDevices) cached[dev].store(waves, std::memory_order_relaxed);
  return waves;
}

// att_part == nullptr: one wavefront per unit.  Otherwise the grid is
// min(n_units, att_rows, resident waves) wavefronts that also form the
// attention-vector gradient's partial sums (gat_bwd_src_h1's ATT); *att_waves
// gets that count (0 when the occupancy query fails: an error).
template <int VEC, int G, int NCH>
static hipError_t launch_bwd_h1(hipStream_t st, const int4* units, int64_t n_units,
                                const int32_t* row_idx, const int32_t* perm, const float* hs,
                                int64_t ldh, const float* go, const float* s, const float* d,
                                const float* alpha, const float* cdot, const float4* rec,
                                const float* att_src, int C, float* dhs, float* ds, float* gt,
                                float* ws, int min_len, const int32_t* src_rows,
                                float* att_part = nullptr, int64_t att_rows = 0,
                                int64_t* att_waves = nullptr) {
  constexpr int EPI = 64 / G;
  // Eight edges a slot in flight measured slower here (0.194 against 0.185 ms
  // for a C5 partition's 20-wide backward): each edge also does a group sum.
  constexpr int U = (EPI == 1) ? ((NCH == 1) ? 8 : (NCH == 2 ? 4 : 2)) : (EPI == 2 ? 4 : 2);
  if (att_part == nullptr) {
    hipLaunchKernelGGL((gat_bwd_src_h1<VEC, G, NCH, U, false>), dim3(blocks_for(n_units)),
                       dim3(256), 0, st, units, n_units, row_idx, perm, hs, ldh, go, s, d, alpha,
                       cdot, rec, att_src, C, dhs, ds, gt, ws, min_len, src_rows, nullptr,
                       (int64_t)0);
    return hipGetLastError();
  }
  const int64_t waves = std::min(std::min(n_units, att_rows), resident_waves_h1<VEC, G, NCH, U>());
  *att_waves = waves;
  if (waves <= 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL((gat_bwd_src_h1<VEC, G, NCH, U, true>), dim3(blocks_for(waves)), dim3(256),
                     0, st, units, n_units, row_idx, perm, hs, ldh, go, s, d, alpha, cdot, rec,
                     att_src, C, dhs, ds, gt, ws, min_len, src_rows, att_part, waves);
  return hipGetLastError();
}

template <int VEC>
static hipError_t dispatch_bwd_h1(int chunks, hipStream_t st, const int4* units,
                                  int64_t n_units, const int32_t* row_idx, const int32_t* perm,
                                  const float* hs, int64_t ldh, const float* go, const float* s,
                                  const float* d, const float* alpha, const float* cdot,
                                  const float4* rec, const float* att_src, int C, float* dhs,
                                  float* ds, float* gt, float* ws, int min_len = 0,
                                  const int32_t* src_rows = nullptr, float* att_part = nullptr,
                                  int64_t att_rows = 0, int64_t* att_waves = nullptr) {
#define GR_BH(G, N)                                                                       \
  return launch_bwd_h1<VEC, G, N>(st, units, n_units, row_idx, perm, hs, ldh, go, s, d,   \
                                  alpha, cdot, rec, att_src, C, dhs, ds, gt, ws, min_len,  \
                                  src_rows, att_part, att_rows, att_waves)
  if (chunks <= 8) GR_BH(8, 1);
  if (chunks <= 16) GR_BH(16, 1);
  if (chunks <= 32) GR_BH(32, 1);
  if (chunks <= 64) GR_BH(64, 1);
  if (chunks <= 128) GR_BH(64, 2);
  GR_BH(64, 4);
#undef GR_BH
}

// Narrow single-head units (chunks <= 16 vectors): groups of 4, 8 or 16 lanes.
template <int VEC>
static hipError_t launch_fwd_rows(int chunks, hipStream_t st, const int4* units, int64_t n,
                                  const int32_t* idx, const float* hs, int64_t ldh,
                                  const float* s, const float* d, int C, const float* bias,
                                  float* m, float* den, float* alpha, float* o, float* y,
                                  int64_t ldy) {
#define GR_FR(G, R, U)                                                                    \
  static_assert(R * G == fwd_rows_max_len(G), "gat_fwd_rows takes R * G edges");           \
  hipLaunchKernelGGL((gat_fwd_rows<VEC, G, R, U>),                                          \
                     dim3(blocks_for((n + 64 / G - 1) / (64 / G))), dim3(256), 0, st, units, n, \
                     idx, hs, ldh, s, d, C, bias, m, den, alpha, o, y, ldy)
  if (chunks <= 4) {
    GR_FR(4, 4, 4);
  } else if (chunks <= 8) {
    GR_FR(8, 4, 8);
  } else {
    GR_FR(16, 2, 8);
  }
#undef GR_FR
  return hipGetLastError();
}

template <int VEC>
static hipError_t launch_bwd_rows(int chunks, hipStream_t st, const int4* units, int64_t n,
                                  const int32_t* row_idx, const int32_t* perm, const float* hs,
                                  int64_t ldh, const float* go, const float* s, const float* d,
                                  const float* alpha, const float* cdot, const float4* rec,
                                  const float* att_src, int C, float* dhs, float* ds, float* gt) {
#define GR_BR(G)                                                                             \
  hipLaunchKernelGGL((gat_bwd_src_rows<VEC, G, (G < 8 ? G : 8)>),                            \
                     dim3(blocks_for((n + 64 / G - 1) / (64 / G))), dim3(256), 0, st, units, n, \
                     row_idx, perm, hs, ldh, go, s, d, alpha, cdot, rec, att_src, C, dhs, ds, \
                     gt, kBwdRowsMaxLen)
  if (chunks <= 4) GR_BR(4);
  else if (chunks <= 8) GR_BR(8);
  else GR_BR(16);
#undef GR_BR
  return hipGetLastError();
}

// gr_gat_backward_src, with rec (one head) in place of alpha, d and cdot.
static int backward_src(const int32_t* units, int64_t n_units, const int32_t* fixups,
                        int64_t n_fix, const int32_t* row_idx, const int32_t* perm,
                        const float* hs, int64_t ldh, const float* go, const float* s,
                        const float* d, const float* alpha, const float* cdot, const float4* rec,
                        const float* att_src, int64_t heads, int64_t channels, float* dhs,
                        float* ds, float* gt, float* workspace, int64_t n_slots, void* stream) {
  int rc = check_heads(heads, channels);
  if (rc) return rc;
  const int64_t HC = heads * channels;
  GR_REQUIRE(ldh >= HC, "gat_backward_src: ldh < H*C");
  GR_REQUIRE(n_fix == 0 || (fixups && workspace), "gat_backward_src: NULL fixups/workspace");
  GR_REQUIRE(rec == nullptr || heads == 1, "gat_backward_src: records take one head");
  if (n_units == 0) return GR_OK;
  GR_REQUIRE(units && aligned16(units) && row_idx && perm && hs && go && s &&
                 (rec != nullptr ? aligned16(rec) : (d && alpha && cdot)) && att_src && dhs &&
                 ds && gt,
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
  GR_REQUIRE(rec == nullptr || chunks <= 256,
             "gat_backward_src: records take rows of at most 256 vectors (1024 aligned floats)");
  if (H == 1 && chunks <= 16) {
    // Narrow: split columns and long whole columns one per wavefront
    // (gat_bwd_src_h1), the other whole columns several per wavefront
    // (gat_bwd_src_rows, after the plan's first n_slots units).
    const int64_t n_split = std::min(n_slots, n_units);
    if (vec == 4)
      err = dispatch_bwd_h1<4>((int)chunks, st, u4, n_units, row_idx, perm, hs, ldh, go, s, d,
                               alpha, cdot, rec, att_src, C, dhs, ds, gt, workspace,
                               kBwdRowsMaxLen + 1);
    else
      err = dispatch_bwd_h1<1>((int)chunks, st, u4, n_units, row_idx, perm, hs, ldh, go, s, d,
                               alpha, cdot, rec, att_src, C, dhs, ds, gt, workspace,
                               kBwdRowsMaxLen + 1);
    GR_HIP_CHECK(err);
    if (n_units > n_split) {
      if (vec == 4)
        err = launch_bwd_rows<4>((int)chunks, st, u4 + n_split, n_units - n_split, row_idx, perm,
                                 hs, ldh, go, s, d, alpha, cdot, rec, att_src, C, dhs, ds, gt);
      else
        err = launch_bwd_rows<1>((int)chunks, st, u4 + n_split, n_units - n_split, row_idx, perm,
                                 hs, ldh, go, s, d, alpha, cdot, rec, att_src, C, dhs, ds, gt);
    }
  } else if (H == 1 && chunks <= 256) {
    if (vec == 4)
      err = dispatch_bwd_h1<4>((int)chunks, st, u4, n_units, row_idx, perm, hs, ldh, go, s, d,
                               alpha, cdot, rec, att_src, C, dhs, ds, gt, workspace);
    else
      err = dispatch_bwd_h1<1>((int)chunks, st, u4, n_units, row_idx, perm, hs, ldh, go, s, d,
                               alpha, cdot, rec, att_src, C, dhs, ds, gt, workspace);
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
                       n_fix, workspace, H, C, att_src, dhs, ds, nullptr);
    GR_HIP_CHECK(hipGetLastError());
  }
  return GR_OK;
}

extern "C" int gr_gat_backward_src(const int32_t* units, int64_t n_units, const int32_t* fixups,
                                   int64_t n_fix, const int32_t* row_idx, const int32_t* perm,
                                   const float* hs, int64_t ldh, const float* go, const float* s,
                                   const float* d, const float* alpha,
                                   const float* cdot, const float* att_src, int64_t heads,
                                   int64_t channels, float* dhs, float* ds, float* gt,
                                   float* workspace, int64_t n_slots, void* stream) {
  gr::clear_error();
  return backward_src(units, n_units, fixups, n_fix, row_idx, perm, hs, ldh, go, s, d, alpha,
                      cdot, nullptr, att_src, heads, channels, dhs, ds, gt, workspace, n_slots,
                      stream);
}

// gr_gat_backward_src_into, with rec in place of alpha, d and cdot.
static int backward_src_into(const int32_t* units, int64_t n_units, const int32_t* fixups,
                             int64_t n_fix, const int32_t* row_idx, const int32_t* perm,
                             const float* hs, int64_t ldh, const int32_t* src_rows,
                             const float* go, const float* s, const float* d,
                             const float* alpha, const float* cdot, const float4* rec,
                             const float* att_src, int64_t heads, int64_t channels, float* dz,
                             float* ds, float* gt, float* workspace, int64_t n_slots,
                             float* att_part, int64_t att_rows, int64_t* att_waves,
                             void* stream) {
  int rc = check_heads(heads, channels);
  if (rc) return rc;
  const int64_t C = channels;
  GR_REQUIRE(heads == 1 && C % 4 == 0 && C > 64 && C <= 1024,
             "gat_backward_src_into: one head of 68..1024 channels, a multiple of 4");
  GR_REQUIRE(ldh >= C && ldh % 4 == 0, "gat_backward_src_into: bad ldh");
  GR_REQUIRE(n_fix == 0 || (fixups && workspace), "gat_backward_src_into: NULL fixups/workspace");
  GR_REQUIRE(att_part == nullptr || (att_rows >= 1 && att_waves != nullptr &&
                                     aligned16(att_part)),
             "gat_backward_src_into: att_part needs att_rows >= 1, att_waves and 16-byte "
             "alignment");
  if (att_waves != nullptr) *att_waves = 0;
  if (n_units == 0) return GR_OK;
  GR_REQUIRE(units && aligned16(units) && row_idx && perm && hs && aligned16(hs) && src_rows &&
                 go && aligned16(go) && s &&
                 (rec != nullptr ? aligned16(rec) : (d && alpha && cdot)) && att_src &&
                 aligned16(att_src) && dz && aligned16(dz) && ds && gt &&
                 (workspace == nullptr || aligned16(workspace)),
             "gat_backward_src_into: NULL or misaligned pointer");
  hipStream_t st = gr::as_stream(stream);
  const int4* u4 = reinterpret_cast<const int4*>(units);
  const hipError_t err = dispatch_bwd_h1<4>((int)(C / 4), st, u4, n_units, row_idx, perm, hs,
                                            ldh, go, s, d, alpha, cdot, rec, att_src, (int)C, dz,
                                            ds, gt, workspace, 0, src_rows, att_part, att_rows,
                                            att_waves);
  GR_REQUIRE(att_part == nullptr || *att_waves > 0,
             "gat_backward_src_into: occupancy query for the attention partials failed");
  GR_HIP_CHECK(err);
  if (n_fix > 0) {
    hipLaunchKernelGGL(gat_bwd_src_fixup, dim3(blocks_for(n_fix)), dim3(256), 0, st, fixups,
                       n_fix, workspace, 1, (int)C, att_src, dz, ds, src_rows);
    GR_HIP_CHECK(hipGetLastError());
  }
  return GR_OK;
}

extern "C" int gr_gat_backward_src_into(const int32_t* units, int64_t n_units,
                                        const int32_t* fixups, int64_t n_fix,
                                        const int32_t* row_idx, const int32_t* perm,
                                        const float* hs, int64_t ldh, const int32_t* src_rows,
                                        const float* go, const float* s, const float* d,
                                        const float* alpha, const float* cdot,
                                        const float* att_src, int64_t heads, int64_t channels,
                                        float* dz, float* ds, float* gt, float* workspace,
                                        int64_t n_slots, float* att_part, int64_t att_rows,
                                        int64_t* att_waves, void* stream) {
  gr::clear_error();
  return backward_src_into(units, n_units, fixups, n_fix, row_idx, perm, hs, ldh, src_rows, go,
                           s, d, alpha, cdot, nullptr, att_src, heads, channels, dz, ds, gt,
                           workspace, n_slots, att_part, att_rows, att_waves, stream);
}

extern "C" int gr_gat_backward_src_h1(const int32_t* units, int64_t n_units,
                                      const int32_t* fixups, int64_t n_fix,
                                      const int32_t* row_idx, const int32_t* perm,
                                      const float* hs, int64_t ldh, const int32_t* src_rows,
                                      const float* go, const float* s, const float* rec,
                                      const float* att_src, int64_t channels, float* dhs,
                                      float* ds, float* gt, float* workspace, int64_t n_slots,
                                      float* att_part, int64_t att_rows, int64_t* att_waves,
                                      void* stream) {
  gr::clear_error();
  const float4* r = reinterpret_cast<const float4*>(rec);
  GR_REQUIRE(n_units == 0 || rec != nullptr, "gat_backward_src_h1: NULL rec");
  if (src_rows == nullptr) {
    GR_REQUIRE(att_part == nullptr, "gat_backward_src_h1: att_part needs src_rows");
    return backward_src(units, n_units, fixups, n_fix, row_idx, perm, hs, ldh, go, s, nullptr,
                        nullptr, nullptr, r, att_src, 1, channels, dhs, ds, gt, workspace,
                        n_slots, stream);
  }
  return backward_src_into(units, n_units, fixups, n_fix, row_idx, perm, hs, ldh, src_rows, go,
                           s, nullptr, nullptr, nullptr, r, att_src, 1, channels, dhs, ds, gt,
                           workspace, n_slots, att_part, att_rows, att_waves, stream);
}

namespace gr_gat {

__global__ __launch_bounds__(256) void gat_record_kernel(const float* __restrict__ d,
                                                         const float* __restrict__ m,
                                                         const float* __restrict__ den,
                                                         const float* __restrict__ cdot,
                                                         int64_t n, float4* __restrict__ rec) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) rec[i] = make_float4(d[i], m[i], den[i], cdot[i]);
}

}  // namespace gr_gat

extern "C" int gr_gat_dst_record(const float* d, const float* m, const float* den,
                                 const float* cdot, int64_t n_dst, float* rec, void* stream) {
  gr::clear_error();
  GR_REQUIRE(n_dst >= 0, "gat_dst_record: negative extent");
  if (n_dst == 0) return GR_OK;
  GR_REQUIRE(d && m && den && cdot && rec && aligned16(rec),
             "gat_dst_record: NULL or misaligned pointer");
  hipLaunchKernelGGL(gat_record_kernel, dim3((unsigned)((n_dst + 255) / 256)), dim3(256), 0,
                     gr::as_stream(stream), d, m, den, cdot, n_dst,
                     reinterpret_cast<float4*>(rec));
  GR_HIP_CHECK(hipGetLastError());
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
  const int4* u4 = reinterpret_cast<const int4*>(units);
  const int C = (int)channels;
  const int vec = (C % 4 == 0 && aligned16(dhs) && aligned16(att_dst)) ? 4 : 1;
  const int chunks = (C + vec - 1) / vec;
  if (heads == 1 && chunks <= 256) {
    // G lanes a row: at least 16 (a long row's edge sum), else the smallest
    // power of two that covers the row's vectors.
#define GR_DH(V, G, N)                                                                        \
  hipLaunchKernelGGL((gat_bwd_dst_h1<V, G, N>), dim3(blocks_for((n_units + 64 / G - 1) / (64 / G))), \
                     dim3(256), 0, st, u4, n_units, gt, C, att_dst, cdot, den, dd, dhs, workspace)
    if (vec == 4) {
      if (chunks <= 16) GR_DH(4, 16, 1);
      else if (chunks <= 32) GR_DH(4, 32, 1);
      else if (chunks <= 64) GR_DH(4, 64, 1);
      else if (chunks <= 128) GR_DH(4, 64, 2);
      else GR_DH(4, 64, 4);
    } else {
      if (chunks <= 16) GR_DH(1, 16, 1);
      else if (chunks <= 32) GR_DH(1, 32, 1);
      else if (chunks <= 64) GR_DH(1, 64, 1);
      else if (chunks <= 128) GR_DH(1, 64, 2);
      else GR_DH(1, 64, 4);
    }
#undef GR_DH
  } else {
    hipLaunchKernelGGL(gat_bwd_dst_kernel, dim3(blocks_for(n_units)), dim3(256), 0, st, u4,
                       n_units, gt, (int)heads, C, att_dst, cdot, den, dd, dhs, workspace);
  }
  GR_HIP_CHECK(hipGetLastError());
  if (n_fix > 0) {
    hipLaunchKernelGGL(gat_bwd_dst_fixup, dim3(blocks_for(n_fix)), dim3(256), 0, st, fixups,
                       n_fix, workspace, (int)heads, (int)channels, att_dst, cdot, den, dd, dhs);
    GR_HIP_CHECK(hipGetLastError());
  }
  return GR_OK;
}
