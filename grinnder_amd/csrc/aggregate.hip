// GCN neighbour aggregation for gfx950 (CDNA4): Y = A * X (+ bias), fp32.
//
// Work decomposition (see gr_spmm_plan in graph_prep.cpp): one 64-lane
// wavefront per plan unit = (row, edge range, slot).  Lanes are split into
// EPI = 64 / G edge slots of G lanes; each lane owns VEC consecutive floats of
// NCH chunks of the gathered row, so one wavefront-wide load fetches EPI
// neighbour rows at once with 4*VEC-byte accesses.  Each loop iteration
// keeps U loads per slot in flight to cover HBM latency.  Partial sums of
// the EPI slots are combined with cross-lane shuffles; rows longer than the
// plan's segment length are summed by a second, ordered pass, so results do
// not depend on scheduling (no atomics).
#include <atomic>
#include <mutex>
#include <type_traits>

#include "gr_internal.h"
#include "ln_row.h"
#include "wave.h"

namespace gr_agg {

template <int VEC>
__device__ __forceinline__ void load_vec(const float* __restrict__ p, float (&r)[VEC]) {
  if constexpr (VEC == 4) {
    const float4 t = *reinterpret_cast<const float4*>(p);
    r[0] = t.x; r[1] = t.y; r[2] = t.z; r[3] = t.w;
  } else if constexpr (VEC == 2) {
    const float2 t = *reinterpret_cast<const float2*>(p);
    r[0] = t.x; r[1] = t.y;
  } else {
    r[0] = *p;
  }
}

template <int VEC>
__device__ __forceinline__ void store_vec(float* __restrict__ p, const float (&r)[VEC]) {
  if constexpr (VEC == 4) {
    *reinterpret_cast<float4*>(p) = make_float4(r[0], r[1], r[2], r[3]);
  } else if constexpr (VEC == 2) {
    *reinterpret_cast<float2*>(p) = make_float2(r[0], r[1]);
  } else {
    *p = r[0];
  }
}

// One wavefront per plan unit; 4 wavefronts per 256-thread workgroup.
// With orow, output row r goes to y row orow[r] and is added to what that row
// holds (the rows of one launch are distinct, so each element has one writer).
template <int VEC, int G, int NCH, int U>
__global__ __launch_bounds__(256) void aggregate_units(
    const int4* __restrict__ units, int64_t n_units, const int32_t* __restrict__ idx,
    const float* __restrict__ val, const float* __restrict__ x, int64_t ldx,
    float* __restrict__ y, int64_t ldy, const float* __restrict__ bias, int dim,
    float* __restrict__ ws, int64_t n_slots, const int32_t* __restrict__ orow) {
  constexpr int EPI = 64 / G;
  const int lane = threadIdx.x & 63;
  const int64_t wid =
      (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  if (wid >= n_units) return;
  const int4 w = units[wid];
  const int slot = (EPI == 1) ? 0 : lane / G;
  const int sub = (EPI == 1) ? lane : lane % G;

  float acc[NCH][VEC];
#pragma unroll
  for (int ch = 0; ch < NCH; ++ch)
#pragma unroll
    for (int j = 0; j < VEC; ++j) acc[ch][j] = 0.f;

  // Lanes past the row end load the row's last vector instead (same cache
  // line, no branch around the loads) and never store.
  bool fvalid[NCH];
  int foff[NCH];
  int fld[NCH];
#pragma unroll
  for (int ch = 0; ch < NCH; ++ch) {
    foff[ch] = (ch * G + sub) * VEC;
    fvalid[ch] = foff[ch] < dim;
    fld[ch] = fvalid[ch] ? foff[ch] : dim - VEC;
  }

  int e = w.y;
  const int end = w.z;
  // Full iterations: EPI * U edges, all in range.
  for (; e + EPI * U <= end; e += EPI * U) {
    int c[U];
    float v[U];
#pragma unroll
    for (int k = 0; k < U; ++k) {
      c[k] = idx[e + k * EPI + slot];
      v[k] = val[e + k * EPI + slot];
    }
    float r[U][NCH][VEC];
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const float* row = x + (int64_t)c[k] * ldx;
#pragma unroll
      for (int ch = 0; ch < NCH; ++ch) load_vec<VEC>(row + fld[ch], r[k][ch]);
    }
#pragma unroll
    for (int k = 0; k < U; ++k)
#pragma unroll
      for (int ch = 0; ch < NCH; ++ch)
#pragma unroll
        for (int j = 0; j < VEC; ++j) acc[ch][j] = fmaf(v[k], r[k][ch][j], acc[ch][j]);
  }
  // Tail: masked iterations of EPI * TU edges.  Out-of-range slots re-read
  // the first tail edge's row (in bounds, cached) with weight 0.
  constexpr int TU = (U < 4) ? U : 4;
  if (e < end) {
    const int safe_c = idx[e];
    for (; e < end; e += EPI * TU) {
      int c[TU];
      float v[TU];
#pragma unroll
      for (int k = 0; k < TU; ++k) {
        const int ee = e + k * EPI + slot;
        const bool ok = ee < end;
        c[k] = ok ? idx[ee] : safe_c;
        v[k] = ok ? val[ee] : 0.f;
      }
      float r[TU][NCH][VEC];
#pragma unroll
      for (int k = 0; k < TU; ++k) {
        const float* row = x + (int64_t)c[k] * ldx;
#pragma unroll
        for (int ch = 0; ch < NCH; ++ch) load_vec<VEC>(row + fld[ch], r[k][ch]);
      }
#pragma unroll
      for (int k = 0; k < TU; ++k)
#pragma unroll
        for (int ch = 0; ch < NCH; ++ch)
#pragma unroll
          for (int j = 0; j < VEC; ++j) acc[ch][j] = fmaf(v[k], r[k][ch][j], acc[ch][j]);
    }
  }

  // Combine the EPI edge slots (lanes sub, sub+G, sub+2G, ...).
  if constexpr (EPI > 1) {
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch)
#pragma unroll
      for (int j = 0; j < VEC; ++j) acc[ch][j] = gr_wave::slot_sum<G>(acc[ch][j]);
  }
  if (slot != 0) return;

  if (w.w < 0) {
    float* out = y + (int64_t)(orow != nullptr ? orow[w.x] : w.x) * ldy;
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) {
      if (!fvalid[ch]) continue;
      if (bias != nullptr) {
        float b[VEC];
        load_vec<VEC>(bias + foff[ch], b);
#pragma unroll
        for (int j = 0; j < VEC; ++j) acc[ch][j] += b[j];
      }
      if (orow != nullptr) {
        float o[VEC];
        load_vec<VEC>(out + foff[ch], o);
#pragma unroll
        for (int j = 0; j < VEC; ++j) acc[ch][j] = o[j] + acc[ch][j];
      }
      store_vec<VEC>(out + foff[ch], acc[ch]);
    }
  } else if (w.w < n_slots) {
    // A slot outside the caller's n_slots * dim workspace is never written.
    float* out = ws + (int64_t)w.w * dim;
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) {
      if (fvalid[ch]) store_vec<VEC>(out + foff[ch], acc[ch]);
    }
  }
}

// Ordered reduction of the partial sums of split rows: one workgroup per
// (split row, 256-feature chunk), one thread per feature; the slot loop is
// unrolled so its loads are independent.  Slots at or past n_slots (outside
// the workspace) are never read.
__global__ __launch_bounds__(256) void aggregate_fixup(const int32_t* __restrict__ fix,
                                                       const float* __restrict__ ws, int dim,
                                                       int64_t n_slots, float* __restrict__ y,
                                                       int64_t ldy,
                                                       const float* __restrict__ bias,
                                                       const int32_t* __restrict__ orow) {
  const int64_t r = blockIdx.x;
  const int f = blockIdx.y * 256 + threadIdx.x;
  if (f >= dim) return;
  const int row = fix[3 * r + 0];
  const int first = fix[3 * r + 1];
  const int n = (int)max((int64_t)0, min((int64_t)fix[3 * r + 2], n_slots - first));
  const float* p = ws + (int64_t)first * dim + f;
  float s = 0.f;
  int k = 0;
  for (; k + 4 <= n; k += 4) {
    const float a = p[(int64_t)(k + 0) * dim];
    const float b = p[(int64_t)(k + 1) * dim];
    const float c = p[(int64_t)(k + 2) * dim];
    const float d = p[(int64_t)(k + 3) * dim];
    s += a;
    s += b;
    s += c;
    s += d;
  }
  for (; k < n; ++k) s += p[(int64_t)k * dim];
  if (bias != nullptr) s += bias[f];
  if (orow != nullptr) {
    float* o = y + (int64_t)orow[row] * ldy + f;
    *o = *o + s;
  } else {
    y[(int64_t)row * ldy + f] = s;
  }
}

// ---------------------------------------------------------------------------
// Fused epilogue: h = A*X + bias, then LayerNorm(h; gamma, beta, eps) and
// ReLU, for rows held by one wavefront (G = 64 lanes, NCH chunks of VEC).
// Writes h (kept for the backward), out = ReLU(LN(h)) and the row statistics
// mean / rstd.  LayerNorm uses the biased variance of the row, as torch does.

// The row LayerNorm helpers (ln_row.h).
using gr_ln::act_fwd;
using gr_ln::act_grad;
using gr_ln::block_sum256;
using gr_ln::ln_affine;
using gr_ln::ln_relu_store_row;
using gr_ln::wave_sum64;

template <int VEC, int NCH, int U>
__global__ __launch_bounds__(256) void aggregate_ln_relu_units(
    const int4* __restrict__ units, int64_t n_units, const int32_t* __restrict__ idx,
    const float* __restrict__ val, const float* __restrict__ x, int64_t ldx,
    const float* __restrict__ bias, const float* __restrict__ gamma,
    const float* __restrict__ beta, float eps, int dim, float* __restrict__ h,
    float* __restrict__ out, float* __restrict__ mean, float* __restrict__ rstd,
    float* __restrict__ ws) {
  const int lane = threadIdx.x & 63;
  const int64_t wid =
      (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  if (wid >= n_units) return;
  const int4 w = units[wid];
  float acc[NCH][VEC];
  bool fvalid[NCH];
  int foff[NCH], fld[NCH];
#pragma unroll
  for (int ch = 0; ch < NCH; ++ch) {
    foff[ch] = (ch * 64 + lane) * VEC;
    fvalid[ch] = foff[ch] < dim;
    fld[ch] = fvalid[ch] ? foff[ch] : dim - VEC;
#pragma unroll
    for (int j = 0; j < VEC; ++j) acc[ch][j] = 0.f;
  }
  int e = w.y;
  const int end = w.z;
  for (; e + U <= end; e += U) {
    int c[U];
    float v[U];
#pragma unroll
    for (int k = 0; k < U; ++k) {
      c[k] = idx[e + k];
      v[k] = val[e + k];
    }
    float r[U][NCH][VEC];
#pragma unroll
    for (int k = 0; k < U; ++k)
#pragma unroll
      for (int ch = 0; ch < NCH; ++ch) load_vec<VEC>(x + (int64_t)c[k] * ldx + fld[ch], r[k][ch]);
#pragma unroll
    for (int k = 0; k < U; ++k)
#pragma unroll
      for (int ch = 0; ch < NCH; ++ch)
#pragma unroll
        for (int j = 0; j < VEC; ++j) acc[ch][j] = fmaf(v[k], r[k][ch][j], acc[ch][j]);
  }
  // Tail: masked iterations of TU edges; out-of-range slots re-read the
  // first tail edge's row with weight 0.
  constexpr int TU = (U < 4) ? U : 4;
  if (e < end) {
    const int safe_c = idx[e];
    for (; e < end; e += TU) {
      int c[TU];
      float v[TU];
#pragma unroll
      for (int k = 0; k < TU; ++k) {
        const bool ok = e + k < end;
        c[k] = ok ? idx[e + k] : safe_c;
        v[k] = ok ? val[e + k] : 0.f;
      }
      float r[TU][NCH][VEC];
#pragma unroll
      for (int k = 0; k < TU; ++k)
#pragma unroll
        for (int ch = 0; ch < NCH; ++ch)
          load_vec<VEC>(x + (int64_t)c[k] * ldx + fld[ch], r[k][ch]);
#pragma unroll
      for (int k = 0; k < TU; ++k)
#pragma unroll
        for (int ch = 0; ch < NCH; ++ch)
#pragma unroll
          for (int j = 0; j < VEC; ++j) acc[ch][j] = fmaf(v[k], r[k][ch][j], acc[ch][j]);
    }
  }
  if (w.w >= 0) {
    float* p = ws + (int64_t)w.w * dim;
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch)
      if (fvalid[ch]) store_vec<VEC>(p + foff[ch], acc[ch]);
    return;
  }
  if (bias != nullptr) {
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) {
      float b[VEC];
      load_vec<VEC>(bias + fld[ch], b);
#pragma unroll
      for (int j = 0; j < VEC; ++j) acc[ch][j] += b[j];
    }
  }
  const int64_t row = w.x;
  ln_relu_store_row<VEC, NCH>(acc, fvalid, foff, dim, gamma, beta, eps, h + row * dim,
                              out + row * dim, mean + row, rstd + row, lane);
}

// Split rows of the fused epilogue: one workgroup per split row.  Each thread
// owns features f = tid, tid + 256, ... (dim <= 1024): ordered sum of the
// partials + bias into h, then the row's LayerNorm statistics by a fixed-order
// workgroup reduction, then out = ReLU(LN(h)).

__global__ __launch_bounds__(256) void aggregate_ln_relu_fixup(
    const int32_t* __restrict__ fix, const float* __restrict__ ws, int dim,
    const float* __restrict__ bias, const float* __restrict__ gamma,
    const float* __restrict__ beta, float eps, float* __restrict__ h, float* __restrict__ out,
    float* __restrict__ mean, float* __restrict__ rstd) {
  __shared__ float red[4];
  const int64_t r = blockIdx.x;
  const int row = fix[3 * r + 0], first = fix[3 * r + 1], n = fix[3 * r + 2];
  float hv[4];
  float s = 0.f;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int f = threadIdx.x + q * 256;
    float a = 0.f;
    if (f < dim) {
      const float* p = ws + (int64_t)first * dim + f;
      for (int k = 0; k < n; ++k) a += p[(int64_t)k * dim];
      if (bias != nullptr) a += bias[f];
      h[(int64_t)row * dim + f] = a;
    }
    hv[q] = a;
    s += a;
  }
  const float mu = block_sum256(s, red) / (float)dim;
  float qv = 0.f;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int f = threadIdx.x + q * 256;
    const float dlt = hv[q] - mu;
    qv += f < dim ? dlt * dlt : 0.f;
  }
  const float rs = 1.0f / sqrtf(block_sum256(qv, red) / (float)dim + eps);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int f = threadIdx.x + q * 256;
    if (f < dim) out[(int64_t)row * dim + f] = fmaxf(ln_affine(hv[q], mu, rs, gamma[f], beta[f]), 0.f);
  }
  if (threadIdx.x == 0) {
    mean[row] = mu;
    rstd[row] = rs;
  }
}

// Backward of act(LayerNorm(h)): for each row, with xh = (h - mean) * rstd,
// y = xh * gamma + beta and gy = g * act'(y):
//   gh = rstd * (gy*gamma - mean(gy*gamma) - xh * mean(gy*gamma*xh)),
// and per-wavefront partial sums of dgamma = sum gy*xh, dbeta = sum gy
// (reduced afterwards in wavefront order).  With part_bias != NULL the
// per-wavefront column sums of gh itself are kept too: the gradient of the
// bias added before the LayerNorm, without a second read of gh.
// Grid-stride over rows.
template <int VEC, int NCH, int ACT, int P>
__global__ __launch_bounds__(256) void ln_relu_backward(
    const float* __restrict__ g, const float* __restrict__ h, const float* __restrict__ mean,
    const float* __restrict__ rstd, const float* __restrict__ gamma,
    const float* __restrict__ beta, int dim, int64_t rows, float* __restrict__ gh,
    float* __restrict__ part_gamma, float* __restrict__ part_beta,
    float* __restrict__ part_bias, const float* __restrict__ shift,
    float* __restrict__ rowdot) {
  const int lane = threadIdx.x & 63;
  const int64_t wid =
      (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int64_t nwaves = (int64_t)gridDim.x * 4;
  bool fvalid[NCH];
  int foff[NCH], fld[NCH];
  float gam[NCH][VEC], bet[NCH][VEC], dg[NCH][VEC], db[NCH][VEC], dh[NCH][VEC];
  float shf[NCH][VEC];
#pragma unroll
  for (int ch = 0; ch < NCH; ++ch) {
    foff[ch] = (ch * 64 + lane) * VEC;
    fvalid[ch] = foff[ch] < dim;
    fld[ch] = fvalid[ch] ? foff[ch] : dim - VEC;
    load_vec<VEC>(gamma + fld[ch], gam[ch]);
    load_vec<VEC>(beta + fld[ch], bet[ch]);
    if (shift != nullptr) {
      load_vec<VEC>(shift + fld[ch], shf[ch]);
    } else {
#pragma unroll
      for (int j = 0; j < VEC; ++j) shf[ch][j] = 0.f;
    }
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      dg[ch][j] = 0.f;
      db[ch][j] = 0.f;
      dh[ch][j] = 0.f;
    }
  }
  const float inv_d = 1.0f / (float)dim;
  // A ring of P rows in flight: the wavefront's rows are r = wid + k nwaves;
  // slot k % P holds row k's loads, issued P rows before its use (a loaded
  // row's latency is several microseconds, one row's work a few hundred
  // cycles).  Rows are consumed in the same order as with one row in flight.
  float gn[P][NCH][VEC], hn[P][NCH][VEC], mu_n[P], rs_n[P];
  auto issue = [&](int slot, int64_t r) {
    if (r < rows) {
      mu_n[slot] = mean[r];
      rs_n[slot] = rstd[r];
#pragma unroll
      for (int ch = 0; ch < NCH; ++ch) {
        load_vec<VEC>(g + r * dim + fld[ch], gn[slot][ch]);
        load_vec<VEC>(h + r * dim + fld[ch], hn[slot][ch]);
      }
    }
  };
#pragma unroll
  for (int k = 0; k < P; ++k) issue(k, wid + k * nwaves);
  for (int64_t r0 = wid; r0 < rows; r0 += P * nwaves) {
#pragma unroll
    for (int k = 0; k < P; ++k) {
      const int64_t r = r0 + k * nwaves;
      if (r >= rows) break;
      const float mu = mu_n[k], rs = rs_n[k];
      float gv[NCH][VEC], hc[NCH][VEC], xh[NCH][VEC], gx[NCH][VEC];
#pragma unroll
      for (int ch = 0; ch < NCH; ++ch)
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
          gv[ch][j] = gn[k][ch][j];
          hc[ch][j] = hn[k][ch][j];
        }
      issue(k, r + P * nwaves);
      float s1 = 0.f, s2 = 0.f;
#pragma unroll
      for (int ch = 0; ch < NCH; ++ch) {
        const float* hv = hc[ch];
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
          const float y = ln_affine(hv[j], mu, rs, gam[ch][j], bet[ch][j]);
          const float gy = fvalid[ch] ? gv[ch][j] * act_grad<ACT>(y) : 0.f;
          xh[ch][j] = (hv[j] - mu) * rs;
          gx[ch][j] = gy * gam[ch][j];
          dg[ch][j] = fmaf(gy, xh[ch][j], dg[ch][j]);
          db[ch][j] += gy;
          s1 += gx[ch][j];
          s2 = fmaf(gx[ch][j], xh[ch][j], s2);
        }
      }
      s1 = wave_sum64(s1) * inv_d;
      s2 = wave_sum64(s2) * inv_d;
      float dot = 0.f;
#pragma unroll
      for (int ch = 0; ch < NCH; ++ch) {
        if (!fvalid[ch]) continue;
        float o[VEC];
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
          o[j] = rs * (gx[ch][j] - s1 - xh[ch][j] * s2);
          dh[ch][j] += o[j];
          dot = fmaf(o[j], hc[ch][j] - shf[ch][j], dot);
        }
        store_vec<VEC>(gh + r * dim + foff[ch], o);
      }
      if (rowdot != nullptr) {
        dot = wave_sum64(dot);
        if (lane == 0) rowdot[r] = dot;
      }
    }
  }
#pragma unroll
  for (int ch = 0; ch < NCH; ++ch) {
    if (!fvalid[ch]) continue;
    store_vec<VEC>(part_gamma + wid * dim + foff[ch], dg[ch]);
    store_vec<VEC>(part_beta + wid * dim + foff[ch], db[ch]);
    if (part_bias != nullptr) store_vec<VEC>(part_bias + wid * dim + foff[ch], dh[ch]);
  }
}

// The LayerNorm/activation backward of ln_relu_backward with its incoming
// gradient formed in place: g = dz B (dz [rows, K] the next layer's gradient
// of its projection, K <= 64; B [K, D] row-major, the next layer's W), on the
// matrix cores, so g never goes to memory.  D = 16 NB.
//
// A pair of wavefronts takes 16 rows at a time, each wavefront half of the
// columns (grid-stride over 32-row steps per workgroup): it holds g for its
// rows and columns as NB / 2 blocks of v_mfma_f32_16x16x4_f32 (lane (lr, lk)
// holds columns c0 + b * 16 + lr of rows 4 lk + q), reads h in the same
// layout (64 contiguous bytes per row per instruction), and the two halves'
// row sums meet in LDS, added in half order by both, before the outputs are
// formed.  Half the columns per wavefront leaves room for two wavefronts per
// SIMD, so one's loads overlap the other's work; each also loads the next
// step's dz, h, mean and rstd while computing this one.  B, gamma and beta
// are staged in LDS once per workgroup (B's row stride D + 16: the four rows
// one instruction reads start 16 banks apart).  Partials of dgamma, dbeta
// and dbias per pair, reduced in order afterwards (colsum_final3).  k runs in
// KS slices of 16 (K <= 16 KS) with the k order of gemm_nt_kernel (MFMA s of a
// slice sums k = 4 q + s over the lane quads q), zeros past K.  With DOT it
// also forms rowdot[r] = <gh_r, h_r - shift>, the two halves added in half
// order.  KS and DOT are template arguments so the common case (K <= 32, no
// dot) keeps its registers within two wavefronts per SIMD; two per SIMD are
// asked of the compiler (it then holds the accumulators in the VGPR half
// of the register file, without spills, at every instance).
constexpr int kLnpMaxK = 64;

template <int NB>
constexpr size_t lnp_lds_bytes(int kpad) {
  return ((size_t)kpad * (16 * NB + 16) + 3 * 16 * NB + 4 * 2 * 2 * 4 * 3) * sizeof(float);
}

template <int NB, int ACT, int KS, bool DOT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void
ln_act_backward_product(
    const float* __restrict__ dz, int64_t ldz, int K, const float* __restrict__ bmat,
    const float* __restrict__ h, const float* __restrict__ mean,
    const float* __restrict__ rstd, const float* __restrict__ gamma,
    const float* __restrict__ beta, int64_t rows, float* __restrict__ gh,
    float* __restrict__ part_gamma, float* __restrict__ part_beta,
    float* __restrict__ part_bias, const float* __restrict__ shift,
    float* __restrict__ rowdot) {
  typedef float floatx4 __attribute__((ext_vector_type(4)));
  constexpr int D = 16 * NB;
  constexpr int NH = NB / 2;  // blocks per wavefront
  constexpr int LDB = D + 16;
  static_assert(NB % 2 == 0, "two halves of whole 16-column blocks");
  extern __shared__ float lnp_smem[];
  const int kpad = (K + 15) / 16 * 16;
  float* Bs = lnp_smem;
  float* GB = Bs + kpad * LDB;  // gamma [D], beta [D], shift [D]
  float* red = GB + 3 * D;      // [q][pair][half][lk][s1, s2], then [q][pair][half][lk] dots
  for (int i = threadIdx.x; i < kpad * D; i += 256) {
    const int k = i / D, c = i % D;
    Bs[k * LDB + c] = k < K ? bmat[(int64_t)k * D + c] : 0.f;
  }
  for (int i = threadIdx.x; i < D; i += 256) {
    GB[i] = gamma[i];
    GB[D + i] = beta[i];
    if (DOT) GB[2 * D + i] = shift != nullptr ? shift[i] : 0.f;
  }
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int lr = lane & 15;
  const int lk = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int pair = wave >> 1;
  const int hf = wave & 1;
  const int c0 = hf * (D / 2);
  float pg[NH], pb[NH], ph[NH];
#pragma unroll
  for (int b = 0; b < NH; ++b) {
    pg[b] = 0.f;
    pb[b] = 0.f;
    ph[b] = 0.f;
  }
  const float inv_d = 1.0f / (float)D;
  const int nslices = kpad / 16;
  constexpr int kMaxSlices = KS;
  float4 dzn[kMaxSlices];
  float hn[4][NH], mun[4], rsn[4];
  // Without the row dot every load is issued (rows past the end read the
  // last row, k past K the row's first k) and the values that are not the
  // step's are zeroed after, and gh leaves through a buffer resource (below):
  // with no branch around them the compiler counts the loads and stores, and
  // its wait for a step's values does not also wait for the stores after
  // them.  The row-dot forms keep guarded loads and stores, which fit their
  // registers.
  constexpr bool kCounted = !DOT;
  auto prefetch = [&](int64_t r0) {
    const int64_t ra = r0 + lr;
    const int64_t rac = ra < rows ? ra : rows - 1;
#pragma unroll
    for (int sl = 0; sl < kMaxSlices; ++sl) {
      const int k0 = sl * 16 + lk * 4;
      const bool ok = sl < nslices && ra < rows && k0 < K;
      if constexpr (kCounted) {
        const float4 v = *reinterpret_cast<const float4*>(dz + rac * ldz + (ok ? k0 : 0));
        dzn[sl] = ok ? v : make_float4(0.f, 0.f, 0.f, 0.f);
      } else {
        dzn[sl] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (ok) dzn[sl] = *reinterpret_cast<const float4*>(dz + ra * ldz + k0);
      }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int64_t row = r0 + lk * 4 + q;
      const bool valid = row < rows;
      if constexpr (kCounted) {
        const int64_t rowc = valid ? row : rows - 1;
        const float m = mean[rowc], rsd = rstd[rowc];
        mun[q] = valid ? m : 0.f;
        rsn[q] = valid ? rsd : 0.f;
#pragma unroll
        for (int b = 0; b < NH; ++b) {
          const float hv = h[rowc * D + c0 + b * 16 + lr];
          hn[q][b] = valid ? hv : 0.f;
        }
      } else {
        mun[q] = valid ? mean[row] : 0.f;
        rsn[q] = valid ? rstd[row] : 0.f;
#pragma unroll
        for (int b = 0; b < NH; ++b) hn[q][b] = valid ? h[row * D + c0 + b * 16 + lr] : 0.f;
      }
    }
  };
  const int64_t step = (int64_t)gridDim.x * 32;
  if ((int64_t)blockIdx.x * 32 < rows) prefetch((int64_t)blockIdx.x * 32 + 16 * pair);
  // The loop bound is the workgroup's (not the pair's): every wavefront
  // reaches every barrier; a pair past the last row computes zeros.
  for (int64_t rb = (int64_t)blockIdx.x * 32; rb < rows; rb += step) {
    const int64_t r0 = rb + 16 * pair;
    float4 dzc[kMaxSlices];
    float hv[4][NH], muv[4], rsv[4];
#pragma unroll
    for (int sl = 0; sl < kMaxSlices; ++sl) dzc[sl] = dzn[sl];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      muv[q] = mun[q];
      rsv[q] = rsn[q];
#pragma unroll
      for (int b = 0; b < NH; ++b) hv[q][b] = hn[q][b];
    }
    if (kCounted)
      prefetch(rb + step < rows ? r0 + step : r0);  // issued either way
    else if (rb + step < rows)
      prefetch(r0 + step);
    // The step's rows of gh through a buffer resource that ends at the last
    // row: rows past it are sent past the end and dropped.
    const int nrow = (int)(rows - r0 < 16 ? (rows - r0 > 0 ? rows - r0 : 0) : 16);  // uniform
    const auto ghb = gr_wave::buffer(gh + r0 * D, (uint32_t)nrow * D * 4);
    floatx4 acc[NH];
#pragma unroll
    for (int b = 0; b < NH; ++b) acc[b] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int sl = 0; sl < kMaxSlices; ++sl) {
      if (sl >= nslices) break;
      const int k0 = sl * 16 + lk * 4;
      const float a[4] = {dzc[sl].x, dzc[sl].y, dzc[sl].z, dzc[sl].w};
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const float* brow = Bs + (k0 + st) * LDB + c0 + lr;
#pragma unroll
        for (int b = 0; b < NH; ++b)
          acc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[st], brow[b * 16], acc[b], 0, 0, 0);
      }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int64_t row = r0 + lk * 4 + q;
      const bool valid = row < rows;
      const float mu = muv[q], rs = rsv[q];
      // Two passes over the half row: the sums, then the outputs, with x-hat
      // and the masked gradient formed again in the second (fewer values
      // live across the row reductions).
      float s1 = 0.f, s2 = 0.f;
#pragma unroll
      for (int b = 0; b < NH; ++b) {
        const int c = c0 + b * 16 + lr;
        const float gm = GB[c];
        const float y = ln_affine(hv[q][b], mu, rs, gm, GB[D + c]);
        const float gy = acc[b][q] * act_grad<ACT>(y);
        const float xh = (hv[q][b] - mu) * rs;
        const float gx = gy * gm;
        pg[b] = fmaf(gy, xh, pg[b]);
        pb[b] += gy;
        s1 += gx;
        s2 = fmaf(gx, xh, s2);
      }
      s1 = gr_wave::group_sum<16>(s1);
      s2 = gr_wave::group_sum<16>(s2);
      float* rq = red + q * 32 + pair * 16;
      if (lr == 0) {
        rq[hf * 8 + lk * 2 + 0] = s1;
        rq[hf * 8 + lk * 2 + 1] = s2;
      }
      __syncthreads();
      s1 = (rq[lk * 2 + 0] + rq[8 + lk * 2 + 0]) * inv_d;
      s2 = (rq[lk * 2 + 1] + rq[8 + lk * 2 + 1]) * inv_d;
      float dot = 0.f;
#pragma unroll
      for (int b = 0; b < NH; ++b) {
        const int c = c0 + b * 16 + lr;
        const float gm = GB[c];
        const float y = ln_affine(hv[q][b], mu, rs, gm, GB[D + c]);
        const float gx = acc[b][q] * act_grad<ACT>(y) * gm;
        const float xh = (hv[q][b] - mu) * rs;
        const float o = rs * (gx - s1 - xh * s2);
        ph[b] += o;
        if (DOT) dot = fmaf(o, hv[q][b] - GB[2 * D + c], dot);
        if constexpr (kCounted)
          gr_wave::buffer_store(ghb, valid ? (uint32_t)((lk * 4 + q) * D + c) * 4
                                           : gr_wave::kBufferDrop, o);
        else if (valid)
          gh[row * D + c] = o;
      }
      if constexpr (DOT) {
        dot = gr_wave::group_sum<16>(dot);
        if (lr == 0) red[128 + q * 16 + pair * 8 + hf * 4 + lk] = dot;
      }
    }
    if constexpr (DOT) {
      // The halves' dots meet after the last row's outputs (the next write
      // of this region follows the next step's first barrier).
      __syncthreads();
      if (hf == 0 && lr == 0) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int64_t row = r0 + lk * 4 + q;
          const float* rd = red + 128 + q * 16 + pair * 8;
          if (row < rows) rowdot[row] = rd[lk] + rd[4 + lk];
        }
      }
    }
  }
  // The four lane quads hold the same columns for different rows.
#pragma unroll
  for (int b = 0; b < NH; ++b) {
    pg[b] = gr_wave::slot_sum<16>(pg[b]);
    pb[b] = gr_wave::slot_sum<16>(pb[b]);
    ph[b] = gr_wave::slot_sum<16>(ph[b]);
  }
  if (lk == 0) {
    const int64_t prow = (int64_t)blockIdx.x * 2 + pair;
#pragma unroll
    for (int b = 0; b < NH; ++b) {
      const int c = c0 + b * 16 + lr;
      part_gamma[prow * D + c] = pg[b];
      part_beta[prow * D + c] = pb[b];
      if (part_bias != nullptr) part_bias[prow * D + c] = ph[b];
    }
  }
}

// Dense epilogue of a layer whose product was formed outside the aggregation
// (or by the GAT aggregation): h = z + bias, out = act(LayerNorm(h)), with the
// same row statistics and affine expression as the fused aggregation epilogue.  One wavefront per row,
// grid-stride.  h may be z itself (ldz == dim): each lane reads its elements
// of the row before the row statistics are reduced, and writes them after.
template <int VEC, int NCH, int ACT>
__global__ __launch_bounds__(256) void bias_ln_relu_rows(
    const float* z, int64_t ldz, const float* __restrict__ bias,
    const float* __restrict__ gamma, const float* __restrict__ beta, float eps, int dim,
    int64_t rows, float* h, float* __restrict__ out, float* __restrict__ mean,
    float* __restrict__ rstd) {
  const int lane = threadIdx.x & 63;
  const int64_t wid =
      (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int64_t nwaves = (int64_t)gridDim.x * 4;
  bool fvalid[NCH];
  int foff[NCH], fld[NCH];
  float bv[NCH][VEC];
#pragma unroll
  for (int ch = 0; ch < NCH; ++ch) {
    foff[ch] = (ch * 64 + lane) * VEC;
    fvalid[ch] = foff[ch] < dim;
    fld[ch] = fvalid[ch] ? foff[ch] : dim - VEC;
    if (bias != nullptr) {
      load_vec<VEC>(bias + fld[ch], bv[ch]);
    } else {
#pragma unroll
      for (int j = 0; j < VEC; ++j) bv[ch][j] = 0.f;
    }
  }
  // The next row's load is issued before the current row is reduced.
  float zn[NCH][VEC];
  if (wid < rows) {
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) load_vec<VEC>(z + wid * ldz + fld[ch], zn[ch]);
  }
  for (int64_t r = wid; r < rows; r += nwaves) {
    float acc[NCH][VEC];
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch)
#pragma unroll
      for (int j = 0; j < VEC; ++j) acc[ch][j] = zn[ch][j] + bv[ch][j];
    const int64_t rn = r + nwaves;
    if (rn < rows) {
#pragma unroll
      for (int ch = 0; ch < NCH; ++ch) load_vec<VEC>(z + rn * ldz + fld[ch], zn[ch]);
    }
    ln_relu_store_row<VEC, NCH, ACT>(acc, fvalid, foff, dim, gamma, beta, eps, h + r * dim,
                                     out + r * dim, mean + r, rstd + r, lane);
  }
}

// Column sums of a [rows, dim] matrix, two passes, fixed order: workgroup b
// sums rows [b*chunk, (b+1)*chunk) into part[b, :]; then part is reduced over
// b in ascending order.  Each thread owns columns f = tid, tid + 256, ...
// Weighted form: x[r, f] is scaled by w[r * ldw + f / group] (per-row weights
// shared by groups of `group` columns, e.g. one weight per attention head).
template <bool WEIGHTED>
__global__ __launch_bounds__(256) void colsum_partial(const float* __restrict__ x, int64_t rows,
                                                      int dim, int64_t ldx,
                                                      const float* __restrict__ w, int64_t ldw,
                                                      int group, int64_t chunk,
                                                      float* __restrict__ part,
                                                      const int32_t* __restrict__ xrows) {
  const int64_t r0 = (int64_t)blockIdx.x * chunk;
  const int64_t r1 = r0 + chunk < rows ? r0 + chunk : rows;
  for (int f = threadIdx.x; f < dim; f += 256) {
    const int wf = WEIGHTED ? f / group : 0;
    auto val = [&](int64_t r) {
      const int64_t xr = xrows != nullptr ? (int64_t)xrows[r] : r;
      const float v = x[xr * ldx + f];
      if constexpr (WEIGHTED) return v * w[r * ldw + wf];
      else return v;
    };
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
    int64_t r = r0;
    for (; r + 4 <= r1; r += 4) {
      a0 += val(r + 0);
      a1 += val(r + 1);
      a2 += val(r + 2);
      a3 += val(r + 3);
    }
    for (; r < r1; ++r) a0 += val(r);
    part[(int64_t)blockIdx.x * dim + f] = (a0 + a1) + (a2 + a3);
  }
}

// The same sums with 16-byte loads, for dim % 4 == 0 (dim <= 1024), ldx % 4
// == 0, a 16-byte aligned x and, weighted, group % 4 == 0 (the 4 columns of
// a vector share one weight).  A workgroup takes RL = 256 / (dim / 4) rows at
// a time: thread t owns the 4 columns of slot t % (dim / 4) in rows r0 + t /
// (dim / 4) + k RL, with four accumulators (four rows in flight); the row
// lanes' sums are then added in lane order through LDS.  Every step is in a
// fixed order.
template <bool WEIGHTED>
__global__ __launch_bounds__(256) void colsum_partial4(const float* __restrict__ x, int64_t rows,
                                                       int dim, int64_t ldx,
                                                       const float* __restrict__ w,
                                                       int64_t ldw, int group, int64_t chunk,
                                                       float* __restrict__ part,
                                                       const int32_t* __restrict__ xrows) {
  __shared__ float4 red[256];
  const int q = dim / 4;
  const int rl_n = 256 / q;
  const int slot = threadIdx.x % q;
  const int rl = threadIdx.x / q;
  const bool active = rl < rl_n;
  const int64_t r0 = (int64_t)blockIdx.x * chunk;
  const int64_t r1 = r0 + chunk < rows ? r0 + chunk : rows;
  float4 a0 = make_float4(0.f, 0.f, 0.f, 0.f), a1 = a0;
  if (active) {
    const int f = slot * 4;
    auto val = [&](int64_t r) {
      const int64_t xr = xrows != nullptr ? (int64_t)xrows[r] : r;
      float4 v = *reinterpret_cast<const float4*>(x + xr * ldx + f);
      if constexpr (WEIGHTED) {
        const float wt = w[r * ldw + f / group];
        v.x *= wt;
        v.y *= wt;
        v.z *= wt;
        v.w *= wt;
      }
      return v;
    };
    float4 a2 = a0, a3 = a0;
    int64_t r = r0 + rl;
    for (; r + 3 * rl_n < r1; r += 4 * rl_n) {
      const float4 v0 = val(r), v1 = val(r + rl_n), v2 = val(r + 2 * rl_n),
                   v3 = val(r + 3 * rl_n);
      a0.x += v0.x; a0.y += v0.y; a0.z += v0.z; a0.w += v0.w;
      a1.x += v1.x; a1.y += v1.y; a1.z += v1.z; a1.w += v1.w;
      a2.x += v2.x; a2.y += v2.y; a2.z += v2.z; a2.w += v2.w;
      a3.x += v3.x; a3.y += v3.y; a3.z += v3.z; a3.w += v3.w;
    }
    for (; r < r1; r += rl_n) {
      const float4 v0 = val(r);
      a0.x += v0.x; a0.y += v0.y; a0.z += v0.z; a0.w += v0.w;
    }
    a0.x += a1.x; a0.y += a1.y; a0.z += a1.z; a0.w += a1.w;
    a2.x += a3.x; a2.y += a3.y; a2.z += a3.z; a2.w += a3.w;
    a0.x += a2.x; a0.y += a2.y; a0.z += a2.z; a0.w += a2.w;
  }
  red[threadIdx.x] = a0;
  __syncthreads();
  if (rl == 0) {
    float4 t = red[slot];
    for (int k = 1; k < rl_n; ++k) {
      const float4 v = red[k * q + slot];
      t.x += v.x; t.y += v.y; t.z += v.z; t.w += v.w;
    }
    *reinterpret_cast<float4*>(part + (int64_t)blockIdx.x * dim + slot * 4) = t;
  }
}

// Column sums of part[nblk, dim] over nblk, deterministic: a workgroup owns
// 4 columns; its 64 row groups each sum rows g, g+64, ... of their column in
// order, then the 64 group sums are added in group order.
constexpr int kFinalCols = 4;
constexpr int kFinalGroups = 64;

__global__ __launch_bounds__(256) void colsum_final(const float* __restrict__ part, int nblk,
                                                    int dim, float* __restrict__ out) {
  __shared__ float red[kFinalGroups][kFinalCols + 1];
  const int cl = threadIdx.x % kFinalCols;
  const int grp = threadIdx.x / kFinalCols;
  const int f = blockIdx.x * kFinalCols + cl;
  float s = 0.f;
  if (f < dim) {
    int b = grp;
    for (; b + 3 * kFinalGroups < nblk; b += 4 * kFinalGroups) {
      const float a0 = part[(int64_t)b * dim + f];
      const float a1 = part[(int64_t)(b + kFinalGroups) * dim + f];
      const float a2 = part[(int64_t)(b + 2 * kFinalGroups) * dim + f];
      const float a3 = part[(int64_t)(b + 3 * kFinalGroups) * dim + f];
      s += a0;
      s += a1;
      s += a2;
      s += a3;
    }
    for (; b < nblk; b += kFinalGroups) s += part[(int64_t)b * dim + f];
  }
  red[grp][cl] = s;
  __syncthreads();
  if (grp == 0 && f < dim) {
    float t = 0.f;
    for (int g = 0; g < kFinalGroups; ++g) t += red[g][cl];
    out[f] = t;
  }
}

// colsum_final over up to three partial matrices of the same shape, laid out
// one after the other (part + y * nblk * dim for y = blockIdx.y), into out0,
// out1, out2: one launch for the LayerNorm backward's dgamma, dbeta and dbias,
// with the same sums in the same order as three colsum_final launches.
__global__ __launch_bounds__(256) void colsum_final3(const float* __restrict__ part, int nblk,
                                                     int dim, float* __restrict__ out0,
                                                     float* __restrict__ out1,
                                                     float* __restrict__ out2) {
  __shared__ float red[kFinalGroups][kFinalCols + 1];
  const int y = blockIdx.y;
  const float* __restrict__ p = part + (int64_t)y * nblk * dim;
  float* __restrict__ out = y == 0 ? out0 : (y == 1 ? out1 : out2);
  const int cl = threadIdx.x % kFinalCols;
  const int grp = threadIdx.x / kFinalCols;
  const int f = blockIdx.x * kFinalCols + cl;
  float s = 0.f;
  if (f < dim) {
    int b = grp;
    for (; b + 3 * kFinalGroups < nblk; b += 4 * kFinalGroups) {
      const float a0 = p[(int64_t)b * dim + f];
      const float a1 = p[(int64_t)(b + kFinalGroups) * dim + f];
      const float a2 = p[(int64_t)(b + 2 * kFinalGroups) * dim + f];
      const float a3 = p[(int64_t)(b + 3 * kFinalGroups) * dim + f];
      s += a0;
      s += a1;
      s += a2;
      s += a3;
    }
    for (; b < nblk; b += kFinalGroups) s += p[(int64_t)b * dim + f];
  }
  red[grp][cl] = s;
  __syncthreads();
  if (grp == 0 && f < dim) {
    float t = 0.f;
    for (int g = 0; g < kFinalGroups; ++g) t += red[g][cl];
    out[f] = t;
  }
}

inline unsigned final_blocks(int64_t dim) {
  return (unsigned)((dim + kFinalCols - 1) / kFinalCols);
}

// Narrow rows (at most G * VEC floats, G <= 16): 64 / G whole rows per
// wavefront step (a batch), one per group of G lanes, each lane owning VEC
// consecutive floats of its row.  Most short rows hold a handful of edges
// (an R-MAT graph's rows are mostly the self loop alone), so a batch is bound
// by its chain of dependent loads (unit, column ids, gathered rows), not by
// bytes.  The wavefronts therefore stride over the batches and load the next
// batch's unit's first U column ids and weights, and the unit after it,
// before the current batch's gathers.  Each group keeps U of its row's edges
// in flight; the plan lists whole rows by length class, so the groups of a
// wavefront run similar trip counts.  All lanes of a group read the same
// column id and weight (one broadcast load).  A row's edges are summed in
// edge order; the result is deterministic.
template <int VEC, int G, int U>
__global__ __launch_bounds__(256) void aggregate_rows(
    const int4* __restrict__ units, int64_t n_units, const int32_t* __restrict__ idx,
    const float* __restrict__ val, const float* __restrict__ x, int64_t ldx,
    float* __restrict__ y, int64_t ldy, const float* __restrict__ bias, int dim,
    const int32_t* __restrict__ orow) {
  constexpr int RPW = 64 / G;
  const int lane = threadIdx.x & 63;
  const int grp = lane / G;
  const int sub = lane % G;
  const int64_t nb = (n_units + RPW - 1) / RPW;
  const int64_t stride = (int64_t)gridDim.x * 4;
  int64_t b =
      (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  if (b >= nb) return;
  // When G does not divide 64 the last 64 % G lanes form no group; they and
  // the groups past the last unit hold no row (x = -1, no edges).
  auto unit_of = [&](int64_t bb) {
    const int64_t u = bb * RPW + grp;
    return grp < RPW && u < n_units ? units[u] : make_int4(-1, 0, 0, -1);
  };
  // The first U edges of a unit; past its end the last edge's id again, with
  // weight 0 (an empty unit reads nothing).
  auto first_edges = [&](int4 w, int (&c)[U], float (&v)[U]) {
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int ee = min(w.y + k, w.z - 1);
      c[k] = w.z > w.y ? idx[ee] : 0;
      v[k] = w.y + k < w.z ? val[ee] : 0.f;
    }
  };
  const int foff = sub * VEC;
  const bool fvalid = foff < dim;
  const int fld = fvalid ? foff : dim - VEC;

  int4 w = unit_of(b);
  int4 wn = unit_of(b + stride);
  int c0[U];
  float v0[U];
  first_edges(w, c0, v0);
  while (true) {
    int c1[U];
    float v1[U];
    first_edges(wn, c1, v1);
    const int4 wnn = unit_of(b + 2 * stride);

    float acc[VEC];
#pragma unroll
    for (int j = 0; j < VEC; ++j) acc[j] = 0.f;
    const int end = w.z;
    if (end > w.y) {
      // Edges w.y .. w.y + U - 1: with fewer, the missing ones re-read the
      // last edge's row (in bounds, cached) with weight 0.
      float r[U][VEC];
#pragma unroll
      for (int k = 0; k < U; ++k) load_vec<VEC>(x + (int64_t)c0[k] * ldx + fld, r[k]);
#pragma unroll
      for (int k = 0; k < U; ++k)
#pragma unroll
        for (int j = 0; j < VEC; ++j) acc[j] = fmaf(v0[k], r[k][j], acc[j]);
    }
    int e = w.y + U;
    for (; e + U <= end; e += U) {
      int c[U];
      float v[U];
#pragma unroll
      for (int k = 0; k < U; ++k) {
        c[k] = idx[e + k];
        v[k] = val[e + k];
      }
      float r[U][VEC];
#pragma unroll
      for (int k = 0; k < U; ++k) load_vec<VEC>(x + (int64_t)c[k] * ldx + fld, r[k]);
#pragma unroll
      for (int k = 0; k < U; ++k)
#pragma unroll
        for (int j = 0; j < VEC; ++j) acc[j] = fmaf(v[k], r[k][j], acc[j]);
    }
    if (e < end) {
      int c[U];
      float v[U];
#pragma unroll
      for (int k = 0; k < U; ++k) {
        const int ee = min(e + k, end - 1);
        c[k] = idx[ee];
        v[k] = e + k < end ? val[ee] : 0.f;
      }
      float r[U][VEC];
#pragma unroll
      for (int k = 0; k < U; ++k) load_vec<VEC>(x + (int64_t)c[k] * ldx + fld, r[k]);
#pragma unroll
      for (int k = 0; k < U; ++k)
#pragma unroll
        for (int j = 0; j < VEC; ++j) acc[j] = fmaf(v[k], r[k][j], acc[j]);
    }
    if (w.x >= 0 && fvalid) {
      float* out = y + (int64_t)(orow != nullptr ? orow[w.x] : w.x) * ldy + foff;
      if (orow != nullptr) {
        float o[VEC];
        load_vec<VEC>(out, o);
#pragma unroll
        for (int j = 0; j < VEC; ++j) acc[j] = o[j] + acc[j];
      } else if (bias != nullptr) {
        float bb[VEC];
        load_vec<VEC>(bias + foff, bb);
#pragma unroll
        for (int j = 0; j < VEC; ++j) acc[j] += bb[j];
      }
      store_vec<VEC>(out, acc);
    }

    b += stride;
    if (b >= nb) break;
    w = wn;
    wn = wnn;
#pragma unroll
    for (int k = 0; k < U; ++k) {
      c0[k] = c1[k];
      v0[k] = v1[k];
    }
  }
}

template <int VEC, int G>
hipError_t launch_rows(const int4* units, int64_t n_units, const int32_t* idx, const float* val,
                       const float* x, int64_t ldx, float* y, int64_t ldy, const float* bias,
                       int dim, const int32_t* orow, hipStream_t s) {
  constexpr int RPW = 64 / G;
  const int64_t waves = (n_units + RPW - 1) / RPW;
  // Enough wavefronts to fill the device; each strides over the batches.
  const int64_t blocks = std::max<int64_t>(1, std::min<int64_t>((waves + 3) / 4, 8192));
  hipLaunchKernelGGL((aggregate_rows<VEC, G, 8>), dim3((unsigned)blocks), dim3(256), 0, s, units,
                     n_units, idx, val, x, ldx, y, ldy, bias, dim, orow);
  return hipGetLastError();
}

// Whole rows of a narrow pass: groups of exactly `chunks` lanes (any count
// up to 16; the kernel needs no cross-lane reduction), so 64 / chunks rows
// share a wavefront (12 for 20-float rows).
template <int VEC, int G = 1>
hipError_t dispatch_rows(int chunks, const int4* units, int64_t n_units, const int32_t* idx,
                         const float* val, const float* x, int64_t ldx, float* y, int64_t ldy,
                         const float* bias, int dim, const int32_t* orow, hipStream_t s) {
  if constexpr (G < 16) {
    if (chunks > G)
      return dispatch_rows<VEC, G + 1>(chunks, units, n_units, idx, val, x, ldx, y, ldy, bias,
                                       dim, orow, s);
  }
  return launch_rows<VEC, G>(units, n_units, idx, val, x, ldx, y, ldy, bias, dim, orow, s);
}

template <int VEC, int G, int NCH>
hipError_t launch_units(const int4* units, int64_t n_units, const int32_t* idx,
                        const float* val, const float* x, int64_t ldx, float* y, int64_t ldy,
                        const float* bias, int dim, float* ws, int64_t n_slots,
                        const int32_t* orow, hipStream_t s) {
  constexpr int EPI = 64 / G;
  // Narrow rows (4 or more edge slots of at most 16 lanes) keep 8 edges a
  // slot in flight: a 512-edge split unit then takes 8 rounds of loads, not 32.
  constexpr int U = (EPI == 1) ? ((NCH == 1) ? 8 : (NCH == 2 ? 4 : 2)) : (EPI == 2 ? 4 : 8);
  const int64_t blocks = (n_units + 3) / 4;
  hipLaunchKernelGGL((aggregate_units<VEC, G, NCH, U>), dim3((unsigned)blocks), dim3(256), 0, s,
                     units, n_units, idx, val, x, ldx, y, ldy, bias, dim, ws, n_slots, orow);
  return hipGetLastError();
}

template <int VEC>
hipError_t dispatch_g(int chunks, const int4* units, int64_t n_units, const int32_t* idx,
                      const float* val, const float* x, int64_t ldx, float* y, int64_t ldy,
                      const float* bias, int dim, float* ws, int64_t n_slots,
                      const int32_t* orow, hipStream_t s) {
  if (chunks <= 8)
    return launch_units<VEC, 8, 1>(units, n_units, idx, val, x, ldx, y, ldy, bias, dim, ws, n_slots,
                                       orow, s);
  if (chunks <= 16)
    return launch_units<VEC, 16, 1>(units, n_units, idx, val, x, ldx, y, ldy, bias, dim, ws, n_slots,
                                       orow, s);
  if (chunks <= 32)
    return launch_units<VEC, 32, 1>(units, n_units, idx, val, x, ldx, y, ldy, bias, dim, ws, n_slots,
                                       orow, s);
  if (chunks <= 64)
    return launch_units<VEC, 64, 1>(units, n_units, idx, val, x, ldx, y, ldy, bias, dim, ws, n_slots,
                                       orow, s);
  if (chunks <= 128)
    return launch_units<VEC, 64, 2>(units, n_units, idx, val, x, ldx, y, ldy, bias, dim, ws, n_slots,
                                       orow, s);
  return launch_units<VEC, 64, 4>(units, n_units, idx, val, x, ldx, y, ldy, bias, dim, ws, n_slots,
                                       orow, s);
}

inline bool aligned(const void* p, int bytes) {
  return (reinterpret_cast<uintptr_t>(p) % bytes) == 0;
}

// y[rows[r]][j] += x[r][j] over n rows of dv V-wide elements.  The rows are
// distinct (the caller's contract), so every element of y has one writer: no
// atomics, and the result is the same as adding the rows one at a time.  A
// row id outside [0, y_rows) is skipped rather than written.  Flat over
// elements (I: the index type), four independent read-add-writes in flight
// per lane.
template <typename V, typename I>
__global__ __launch_bounds__(256) void scatter_add_rows(const V* __restrict__ x, I n, I dv,
                                                       I ldx, const int64_t* __restrict__ rows,
                                                       V* __restrict__ y, I ldy, int64_t y_rows) {
  const I total = n * dv;
  const I stride = (I)gridDim.x * 256;
  for (I base = (I)blockIdx.x * 256 + (I)threadIdx.x; base < total; base += 4 * stride) {
    V xv[4], yv[4];
    V* dst[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const I i = base + u * stride;
      dst[u] = nullptr;
      if (i < total) {
        const I r = i / dv;
        const I j = i - r * dv;
        const int64_t t = rows[r];
        if (t >= 0 && t < y_rows) {
          dst[u] = y + (I)t * ldy + j;
          xv[u] = x[r * ldx + j];
          yv[u] = *dst[u];
        }
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (dst[u] != nullptr) *dst[u] = yv[u] + xv[u];
  }
}

// y[r][j] = x[rows[r]][j] over n rows of dv V-wide elements; a row id
// outside [0, x_rows) yields a zero row.  Flat over elements, as
// scatter_add_rows, so narrow rows still keep every lane busy.
template <typename V, typename I>
__global__ __launch_bounds__(256) void gather_rows(const V* __restrict__ x, I ldx,
                                                  const int64_t* __restrict__ rows,
                                                  int64_t x_rows, I n, I dv,
                                                  V* __restrict__ y, I ldy) {
  const I total = n * dv;
  const I stride = (I)gridDim.x * 256;
  for (I base = (I)blockIdx.x * 256 + (I)threadIdx.x; base < total; base += 4 * stride) {
    V v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const I i = base + u * stride;
      if (i < total) {
        const I r = i / dv;
        const I j = i - r * dv;
        const int64_t t = rows[r];
        if (t >= 0 && t < x_rows)
          v[u] = x[(I)t * ldx + j];
        else
          v[u] = V{};
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const I i = base + u * stride;
      if (i < total) {
        const I r = i / dv;
        y[r * ldy + (i - r * dv)] = v[u];
      }
    }
  }
}

template <typename V, typename I>
void launch_gather_rows(const float* x, int64_t ldx, const int64_t* rows, int64_t x_rows,
                        int64_t n, int64_t dim, float* y, int64_t ldy, hipStream_t s) {
  constexpr int W = sizeof(V) / sizeof(float);
  const int64_t total = n * (dim / W);
  const int64_t want = (total + 1023) / 1024;
  const unsigned grid = (unsigned)std::max<int64_t>(1, std::min<int64_t>(want, 1 << 20));
  hipLaunchKernelGGL((gather_rows<V, I>), dim3(grid), dim3(256), 0, s,
                     reinterpret_cast<const V*>(x), (I)(ldx / W), rows, x_rows, (I)n,
                     (I)(dim / W), reinterpret_cast<V*>(y), (I)(ldy / W));
}

template <typename V, typename I>
void launch_scatter_add_rows(const float* x, int64_t n, int64_t dim, int64_t ldx,
                             const int64_t* rows, float* y, int64_t ldy, int64_t y_rows,
                             hipStream_t s) {
  constexpr int W = sizeof(V) / sizeof(float);
  const int64_t total = n * (dim / W);
  const int64_t want = (total + 1023) / 1024;
  const unsigned grid = (unsigned)std::max<int64_t>(1, std::min<int64_t>(want, 1 << 20));
  hipLaunchKernelGGL((scatter_add_rows<V, I>), dim3(grid), dim3(256), 0, s,
                     reinterpret_cast<const V*>(x), (I)n, (I)(dim / W), (I)(ldx / W), rows,
                     reinterpret_cast<V*>(y), (I)(ldy / W), y_rows);
}

}  // namespace gr_agg

namespace gr_agg {

int aggregate_entry(const int32_t* units, int64_t n_units, const int32_t* fixups, int64_t n_fix,
                    const int32_t* idx, const float* val, const float* x, int64_t ldx,
                    float* y, int64_t ldy, const float* bias, int64_t rows, int64_t dim,
                    float* workspace, int64_t n_slots, const int32_t* orow, void* stream);

}  // namespace gr_agg

extern "C" int gr_gcn_aggregate(const int32_t* units, int64_t n_units, const int32_t* fixups,
                                int64_t n_fix, const int32_t* idx, const float* val,
                                const float* x, int64_t ldx, float* y, int64_t ldy,
                                const float* bias, int64_t rows, int64_t dim, float* workspace,
                                int64_t n_slots, void* stream) {
  gr::clear_error();
  return gr_agg::aggregate_entry(units, n_units, fixups, n_fix, idx, val, x, ldx, y, ldy, bias,
                                 rows, dim, workspace, n_slots, nullptr, stream);
}

// Scratch of gr_gcn_aggregate_noalloc: the split-row partial sums live in
// this file-scope device array instead of a caller workspace.  Each GPU the
// library runs on holds its own copy until the process ends.  Host code
// never uses the array's name as a device address: its address on each
// device comes from hipGetSymbolAddress, taken once per device with that
// device current, and only that address reaches kernels.
__device__ __align__(256) float scratch[GR_NOALLOC_SCRATCH_FLOATS];

namespace gr_agg {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device (looked up once).
int scratch_address(float** out) {
  int dev = -1;
  GR_HIP_CHECK(hipGetDevice(&dev));
  GR_REQUIRE(dev >= 0 && dev < kMaxDevices, "gcn_aggregate_noalloc: device %d unsupported",
             dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    GR_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    GR_REQUIRE(p != nullptr, "gcn_aggregate_noalloc: no device address for the scratch");
    g_scratch_ptr[dev] = static_cast<float*>(p);
  }
  *out = g_scratch_ptr[dev];
  return GR_OK;
}

}  // namespace gr_agg

extern "C" int gr_gcn_aggregate_noalloc(const int32_t* units, int64_t n_units,
                                        const int32_t* fixups, int64_t n_fix,
                                        const int32_t* idx, const float* val, const float* x,
                                        int64_t ldx, float* y, int64_t ldy, const float* bias,
                                        int64_t rows, int64_t dim, int64_t n_slots,
                                        void* stream) {
  gr::clear_error();
  GR_REQUIRE(dim >= 1 && n_slots >= 0, "gcn_aggregate_noalloc: bad dim or n_slots");
  GR_REQUIRE(n_slots <= GR_NOALLOC_SCRATCH_FLOATS / dim,
             "gcn_aggregate_noalloc: %lld split slots of %lld floats exceed the scratch of "
             "%lld floats; use gr_gcn_aggregate with a workspace",
             (long long)n_slots, (long long)dim, (long long)GR_NOALLOC_SCRATCH_FLOATS);
  GR_REQUIRE(n_fix >= 0 && n_slots >= 2 * n_fix,
             "gcn_aggregate_noalloc: n_slots %lld is below the 2 * n_fix = %lld slots of the "
             "plan's split rows; pass the n_slots gr_spmm_plan returned",
             (long long)n_slots, (long long)(2 * n_fix));
  float* ws = nullptr;
  if (n_fix > 0 && n_units > 0) {
    const int rc = gr_agg::scratch_address(&ws);
    if (rc != GR_OK) return rc;
  }
  // Split units store every element of their slot before the fixup reads
  // it, so nothing in the scratch needs clearing between calls.
  return gr_agg::aggregate_entry(units, n_units, fixups, n_fix, idx, val, x, ldx, y, ldy, bias,
                                 rows, dim, ws, n_slots, nullptr, stream);
}

extern "C" int gr_gcn_aggregate_into(const int32_t* units, int64_t n_units,
                                     const int32_t* fixups, int64_t n_fix, const int32_t* idx,
                                     const float* val, const float* x, int64_t ldx,
                                     const int32_t* out_rows, float* y, int64_t ldy,
                                     int64_t rows, int64_t dim, float* workspace,
                                     int64_t n_slots, void* stream) {
  gr::clear_error();
  GR_REQUIRE(out_rows != nullptr || n_units == 0, "gcn_aggregate_into: NULL out_rows");
  return gr_agg::aggregate_entry(units, n_units, fixups, n_fix, idx, val, x, ldx, y, ldy,
                                 nullptr, rows, dim, workspace, n_slots, out_rows, stream);
}

int gr_agg::aggregate_entry(const int32_t* units, int64_t n_units, const int32_t* fixups,
                            int64_t n_fix, const int32_t* idx, const float* val,
                            const float* x, int64_t ldx, float* y, int64_t ldy,
                            const float* bias, int64_t rows, int64_t dim, float* workspace,
                            int64_t n_slots, const int32_t* orow, void* stream) {
  using namespace gr_agg;
  GR_REQUIRE(n_units >= 0 && n_fix >= 0 && n_slots >= 0 && rows >= 0,
             "gcn_aggregate: negative extent");
  GR_REQUIRE(dim >= 1 && dim <= 1024, "gcn_aggregate: dim %lld outside [1, 1024]",
             (long long)dim);
  GR_REQUIRE(ldx >= dim && ldy >= dim, "gcn_aggregate: ldx/ldy smaller than dim");
  GR_REQUIRE(n_units == 0 || (units != nullptr && y != nullptr && x != nullptr),
             "gcn_aggregate: NULL units/x/y");
  GR_REQUIRE(n_fix == 0 || (fixups != nullptr && workspace != nullptr),
             "gcn_aggregate: NULL fixups/workspace with n_fix > 0");
  // Every split row of a plan has at least two units, each with a slot of its
  // own, so a plan with n_fix split rows needs n_slots >= 2 * n_fix.  (The
  // kernels also never touch a slot at or past n_slots.)
  GR_REQUIRE(n_slots >= 2 * n_fix,
             "gcn_aggregate: n_slots %lld is below the 2 * n_fix = %lld slots of the plan's "
             "split rows; pass the n_slots gr_spmm_plan returned",
             (long long)n_slots, (long long)(2 * n_fix));
  GR_REQUIRE(aligned(units, 16), "gcn_aggregate: units must be 16-byte aligned");
  if (n_units == 0) return GR_OK;
  hipStream_t s = gr::as_stream(stream);

  int vec = 1;
  if (dim % 4 == 0 && ldx % 4 == 0 && ldy % 4 == 0 && aligned(x, 16) && aligned(y, 16) &&
      (bias == nullptr || aligned(bias, 16)) && (workspace == nullptr || aligned(workspace, 16))) {
    vec = 4;
  } else if (dim % 2 == 0 && ldx % 2 == 0 && ldy % 2 == 0 && aligned(x, 8) && aligned(y, 8) &&
             (bias == nullptr || aligned(bias, 8)) &&
             (workspace == nullptr || aligned(workspace, 8))) {
    vec = 2;
  }
  const int d = static_cast<int>(dim);
  const int chunks = (d + vec - 1) / vec;
  GR_REQUIRE(chunks <= 256, "gcn_aggregate: dim %d too wide for vector width %d", d, vec);
  const int4* u4 = reinterpret_cast<const int4*>(units);
  // Narrow widths: the plan's n_slots split units come first (gr_spmm_plan)
  // and run one per wavefront; the whole rows after them run several per
  // wavefront (aggregate_rows).  Unlike the attention kernels, a group here
  // takes a long row in one pass with U edges in flight, which measured
  // faster than handing long rows back to aggregate_units.
  const bool narrow = chunks <= 16;
  const int64_t n_wide = narrow ? std::min(n_slots, n_units) : n_units;
  hipError_t err = hipSuccess;
  if (n_wide > 0) {
    if (vec == 4)
      err = dispatch_g<4>(chunks, u4, n_wide, idx, val, x, ldx, y, ldy, bias, d, workspace,
                          n_slots, orow, s);
    else if (vec == 2)
      err = dispatch_g<2>(chunks, u4, n_wide, idx, val, x, ldx, y, ldy, bias, d, workspace,
                          n_slots, orow, s);
    else
      err = dispatch_g<1>(chunks, u4, n_wide, idx, val, x, ldx, y, ldy, bias, d, workspace,
                          n_slots, orow, s);
    GR_HIP_CHECK(err);
  }
  if (narrow && n_units > n_wide) {
    const int4* rows = u4 + n_wide;
    const int64_t n_rows = n_units - n_wide;
    if (vec == 4)
      err = dispatch_rows<4>(chunks, rows, n_rows, idx, val, x, ldx, y, ldy, bias, d, orow, s);
    else if (vec == 2)
      err = dispatch_rows<2>(chunks, rows, n_rows, idx, val, x, ldx, y, ldy, bias, d, orow, s);
    else
      err = dispatch_rows<1>(chunks, rows, n_rows, idx, val, x, ldx, y, ldy, bias, d, orow, s);
    GR_HIP_CHECK(err);
  }
  if (n_fix > 0) {
    GR_REQUIRE(n_fix <= INT32_MAX, "gcn_aggregate: too many split rows");
    const int threads = d >= 256 ? 256 : ((d + 63) / 64) * 64;
    hipLaunchKernelGGL(aggregate_fixup, dim3((unsigned)n_fix, (unsigned)((d + 255) / 256)),
                       dim3(threads), 0, s, fixups, workspace, d, n_slots, y, ldy, bias, orow);
    GR_HIP_CHECK(hipGetLastError());
  }
  return GR_OK;
}

extern "C" int gr_gather_rows(const float* x, int64_t x_rows, int64_t ldx,
                              const int64_t* rows, int64_t n, int64_t dim, float* y,
                              int64_t ldy, void* stream) {
  gr::clear_error();
  GR_REQUIRE(n >= 0 && dim >= 1 && ldx >= dim && ldy >= dim && x_rows >= 0,
             "gather_rows: bad shape");
  if (n == 0) return GR_OK;
  GR_REQUIRE(rows != nullptr && y != nullptr && (x != nullptr || x_rows == 0),
             "gather_rows: NULL pointer");
  hipStream_t s = gr::as_stream(stream);
  const bool vec = dim % 4 == 0 && ldx % 4 == 0 && ldy % 4 == 0 && gr_agg::aligned(x, 16) &&
                   gr_agg::aligned(y, 16);
  // 32-bit element indices when every offset fits (see gr_scatter_add_rows).
  const bool narrow = n * ldy < (int64_t(1) << 30) && x_rows * ldx < (int64_t(1) << 31);
  if (vec && narrow)
    gr_agg::launch_gather_rows<float4, int32_t>(x, ldx, rows, x_rows, n, dim, y, ldy, s);
  else if (vec)
    gr_agg::launch_gather_rows<float4, int64_t>(x, ldx, rows, x_rows, n, dim, y, ldy, s);
  else if (narrow)
    gr_agg::launch_gather_rows<float, int32_t>(x, ldx, rows, x_rows, n, dim, y, ldy, s);
  else
    gr_agg::launch_gather_rows<float, int64_t>(x, ldx, rows, x_rows, n, dim, y, ldy, s);
  GR_HIP_CHECK(hipGetLastError());
  return GR_OK;
}

extern "C" int gr_scatter_add_rows(const float* x, int64_t n, int64_t dim, int64_t ldx,
                                   const int64_t* rows, float* y, int64_t y_rows, int64_t ldy,
                                   void* stream) {
  gr::clear_error();
  GR_REQUIRE(n >= 0 && dim >= 1 && ldx >= dim && ldy >= dim && y_rows >= 0,
             "scatter_add_rows: bad shape");
  if (n == 0) return GR_OK;
  GR_REQUIRE(x != nullptr && rows != nullptr && y != nullptr, "scatter_add_rows: NULL pointer");
  hipStream_t s = gr::as_stream(stream);
  const bool vec = dim % 4 == 0 && ldx % 4 == 0 && ldy % 4 == 0 && gr_agg::aligned(x, 16) &&
                   gr_agg::aligned(y, 16);
  // 32-bit element indices when every offset fits: below 2^30 elements of x
  // the loop's index (at most total + 4 grid strides, a stride at most 2^28)
  // stays below 2^31 too.
  const bool narrow = n * ldx < (int64_t(1) << 30) && y_rows * ldy < (int64_t(1) << 31);
  if (vec && narrow)
    gr_agg::launch_scatter_add_rows<float4, int32_t>(x, n, dim, ldx, rows, y, ldy, y_rows, s);
  else if (vec)
    gr_agg::launch_scatter_add_rows<float4, int64_t>(x, n, dim, ldx, rows, y, ldy, y_rows, s);
  else if (narrow)
    gr_agg::launch_scatter_add_rows<float, int32_t>(x, n, dim, ldx, rows, y, ldy, y_rows, s);
  else
    gr_agg::launch_scatter_add_rows<float, int64_t>(x, n, dim, ldx, rows, y, ldy, y_rows, s);
  GR_HIP_CHECK(hipGetLastError());
  return GR_OK;
}

extern "C" int gr_column_sum(const float* x, int64_t rows, int64_t dim, int64_t ldx,
                             const int32_t* xrows, const float* w, int64_t ldw, int64_t group,
                             float* out, float* workspace, int64_t workspace_floats,
                             void* stream) {
  gr::clear_error();
  GR_REQUIRE(rows >= 0 && dim >= 1 && ldx >= dim, "column_sum: bad shape");
  GR_REQUIRE(out != nullptr && (rows == 0 || x != nullptr), "column_sum: NULL pointer");
  GR_REQUIRE(w == nullptr || (group >= 1 && ldw >= (dim + group - 1) / group),
             "column_sum: weights need group >= 1 and ldw >= ceil(dim / group)");
  hipStream_t s = gr::as_stream(stream);
  const int64_t nblk_max = workspace_floats / dim;
  GR_REQUIRE(workspace != nullptr && nblk_max >= 1,
             "column_sum: workspace must hold at least dim floats");
  // ~256 rows per workgroup (enough loads in flight for small row counts),
  // at most 4096 partial rows.
  int64_t nblk = rows == 0 ? 1 : (rows + 255) / 256;
  if (nblk > 4096) nblk = 4096;
  if (nblk > nblk_max) nblk = nblk_max;
  const int64_t chunk = rows == 0 ? 0 : (rows + nblk - 1) / nblk;
  const bool vec4 = dim % 4 == 0 && dim <= 1024 && ldx % 4 == 0 &&
                    (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
                    (reinterpret_cast<uintptr_t>(workspace) & 15) == 0 &&
                    (w == nullptr || group % 4 == 0);
  if (vec4 && w != nullptr)
    hipLaunchKernelGGL(gr_agg::colsum_partial4<true>, dim3((unsigned)nblk), dim3(256), 0, s, x,
                       rows, (int)dim, ldx, w, ldw, (int)group, chunk, workspace, xrows);
  else if (vec4)
    hipLaunchKernelGGL(gr_agg::colsum_partial4<false>, dim3((unsigned)nblk), dim3(256), 0, s,
                       x, rows, (int)dim, ldx, nullptr, 0, 4, chunk, workspace, xrows);
  else if (w != nullptr)
    hipLaunchKernelGGL(gr_agg::colsum_partial<true>, dim3((unsigned)nblk), dim3(256), 0, s, x,
                       rows, (int)dim, ldx, w, ldw, (int)group, chunk, workspace, xrows);
  else
    hipLaunchKernelGGL(gr_agg::colsum_partial<false>, dim3((unsigned)nblk), dim3(256), 0, s, x,
                       rows, (int)dim, ldx, nullptr, 0, 1, chunk, workspace, xrows);
  GR_HIP_CHECK(hipGetLastError());
  hipLaunchKernelGGL(gr_agg::colsum_final, dim3(gr_agg::final_blocks(dim)), dim3(256), 0, s,
                     workspace, (int)nblk, (int)dim, out);
  GR_HIP_CHECK(hipGetLastError());
  return GR_OK;
}

namespace {

template <int VEC, int NCH>
hipError_t launch_ln_relu(const int4* units, int64_t n_units, const int32_t* idx,
                          const float* val, const float* x, int64_t ldx, const float* bias,
                          const float* gamma, const float* beta, float eps, int dim, float* h,
                          float* out, float* mean, float* rstd, float* ws, hipStream_t s) {
  constexpr int U = NCH == 1 ? 8 : (NCH == 2 ? 4 : 2);
  hipLaunchKernelGGL((gr_agg::aggregate_ln_relu_units<VEC, NCH, U>),
                     dim3((unsigned)((n_units + 3) / 4)), dim3(256), 0, s, units, n_units, idx,
                     val, x, ldx, bias, gamma, beta, eps, dim, h, out, mean, rstd, ws);
  return hipGetLastError();
}

bool fused_shape(int64_t dim, int* vec, int* nch) {
  *vec = dim % 4 == 0 ? 4 : 1;
  const int64_t chunks = dim / *vec + (dim % *vec ? 1 : 0);
  if (chunks <= 64) *nch = 1;
  else if (chunks <= 128) *nch = 2;
  else if (chunks <= 256) *nch = 4;
  else return false;
  return true;
}

}  // namespace

extern "C" int gr_gcn_aggregate_ln_relu(const int32_t* units, int64_t n_units,
                                        const int32_t* fixups, int64_t n_fix, const int32_t* idx,
                                        const float* val, const float* x, int64_t ldx,
                                        const float* bias, const float* gamma, const float* beta,
                                        float eps, int64_t rows, int64_t dim, float* h,
                                        float* out, float* mean, float* rstd, float* workspace,
                                        int64_t n_slots, void* stream) {
  gr::clear_error();
  GR_REQUIRE(n_units >= 0 && n_fix >= 0 && rows >= 0, "gcn_aggregate_ln_relu: negative extent");
  int vec, nch;
  GR_REQUIRE(dim >= 1 && fused_shape(dim, &vec, &nch),
             "gcn_aggregate_ln_relu: dim %lld unsupported (max 1024)", (long long)dim);
  GR_REQUIRE(ldx >= dim, "gcn_aggregate_ln_relu: ldx < dim");
  GR_REQUIRE(gamma && beta && h && out && mean && rstd, "gcn_aggregate_ln_relu: NULL output");
  GR_REQUIRE(n_fix == 0 || (fixups && workspace), "gcn_aggregate_ln_relu: NULL fixups/workspace");
  if (n_units == 0) return GR_OK;
  GR_REQUIRE(units && gr_agg::aligned(units, 16) && idx && val && x,
             "gcn_aggregate_ln_relu: NULL or misaligned input");
  if (vec == 4) {
    const bool al = gr_agg::aligned(x, 16) && ldx % 4 == 0 && gr_agg::aligned(h, 16) &&
                    gr_agg::aligned(out, 16) && gr_agg::aligned(gamma, 16) &&
                    gr_agg::aligned(beta, 16) && (bias == nullptr || gr_agg::aligned(bias, 16)) &&
                    (workspace == nullptr || gr_agg::aligned(workspace, 16));
    if (!al) {
      GR_REQUIRE(dim <= 256, "gcn_aggregate_ln_relu: misaligned rows wider than 256");
      vec = 1;
      nch = dim <= 64 ? 1 : (dim <= 128 ? 2 : 4);
    }
  }
  hipStream_t s = gr::as_stream(stream);
  const int4* u4 = reinterpret_cast<const int4*>(units);
  const int d = (int)dim;
  hipError_t err;
  if (vec == 4) {
    if (nch == 1) err = launch_ln_relu<4, 1>(u4, n_units, idx, val, x, ldx, bias, gamma, beta, eps, d, h, out, mean, rstd, workspace, s);
    else if (nch == 2) err = launch_ln_relu<4, 2>(u4, n_units, idx, val, x, ldx, bias, gamma, beta, eps, d, h, out, mean, rstd, workspace, s);
    else err = launch_ln_relu<4, 4>(u4, n_units, idx, val, x, ldx, bias, gamma, beta, eps, d, h, out, mean, rstd, workspace, s);
  } else {
    if (nch == 1) err = launch_ln_relu<1, 1>(u4, n_units, idx, val, x, ldx, bias, gamma, beta, eps, d, h, out, mean, rstd, workspace, s);
    else if (nch == 2) err = launch_ln_relu<1, 2>(u4, n_units, idx, val, x, ldx, bias, gamma, beta, eps, d, h, out, mean, rstd, workspace, s);
    else err = launch_ln_relu<1, 4>(u4, n_units, idx, val, x, ldx, bias, gamma, beta, eps, d, h, out, mean, rstd, workspace, s);
  }
  GR_HIP_CHECK(err);
  if (n_fix > 0) {
    GR_REQUIRE(n_fix <= INT32_MAX, "gcn_aggregate_ln_relu: too many split rows");
    hipLaunchKernelGGL(gr_agg::aggregate_ln_relu_fixup, dim3((unsigned)n_fix), dim3(256), 0, s,
                       fixups, workspace, d, bias, gamma, beta, eps, h, out, mean, rstd);
    GR_HIP_CHECK(hipGetLastError());
  }
  return GR_OK;
}

namespace gr_agg {

// Waves of `kernel` (256-thread workgroups) that the device holds at once.
inline int64_t resident_waves(const void* kernel) {
  int dev = 0, cus = 0, nb = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, kernel, 256, 0) != hipSuccess)
    return 8192;
  return (int64_t)std::max(nb, 1) * std::max(cus, 1) * 4;
}

// The LayerNorm/activation backward with the grid one resident wave per
// slot (each wave keeps P rows in flight), then the ordered column sums of
// the per-wave partials.
template <int V, int N, int P>
int run_ln_backward_p(int32_t act, const float* g, const float* h, const float* mean,
                      const float* rstd, const float* gamma, const float* beta, int64_t rows,
                      int64_t dim, float* gh, float* dgamma, float* dbeta, float* dbias,
                      const float* shift, float* rowdot, float* workspace,
                      int64_t workspace_floats, hipStream_t s);

template <int V, int N>
int run_ln_backward(int32_t act, const float* g, const float* h, const float* mean,
                    const float* rstd, const float* gamma, const float* beta, int64_t rows,
                    int64_t dim, float* gh, float* dgamma, float* dbeta, float* dbias,
                    const float* shift, float* rowdot, float* workspace,
                    int64_t workspace_floats, hipStream_t s) {
  // Eight rows in flight at 256 floats a row (measured on one box, ReLU, 256
  // wide: 2.45M rows 1.42 ms against 1.53 with six, 1.76 with four; 10M rows
  // 5.87 against 6.43 and 6.75 ms; ten gain nothing more).
  return run_ln_backward_p<V, N, N == 1 ? 8 : 1>(act, g, h, mean, rstd, gamma, beta, rows, dim,
                                                 gh, dgamma, dbeta, dbias, shift, rowdot,
                                                 workspace, workspace_floats, s);
}

template <int V, int N, int P>
int run_ln_backward_p(int32_t act, const float* g, const float* h, const float* mean,
                      const float* rstd, const float* gamma, const float* beta, int64_t rows,
                      int64_t dim, float* gh, float* dgamma, float* dbeta, float* dbias,
                      const float* shift, float* rowdot, float* workspace,
                      int64_t workspace_floats, hipStream_t s) {
  const void* kern = act == GR_ACT_RELU
                         ? reinterpret_cast<const void*>(&ln_relu_backward<V, N, GR_ACT_RELU, P>)
                         : reinterpret_cast<const void*>(&ln_relu_backward<V, N, GR_ACT_ELU, P>);
  static int64_t resident[2] = {0, 0};
  int64_t& res = resident[act == GR_ACT_RELU ? 0 : 1];
  if (res == 0) res = resident_waves(kern);
  // Wavefront count: the resident waves, fewer for few rows, bounded by the
  // workspace (nparts * nwaves * dim floats of partials).
  int64_t nwaves = std::min<int64_t>(res, std::max<int64_t>(4, (rows + 15) / 16));
  nwaves = (nwaves + 3) / 4 * 4;
  const int nparts = dbias != nullptr ? 3 : 2;
  const int64_t cap = (workspace_floats / dim - 1) / nparts / 4 * 4;
  GR_REQUIRE(cap >= 4, "ln_relu_backward: workspace too small");
  if (nwaves > cap) nwaves = cap;
  float* pg = workspace;
  float* pb = workspace + nwaves * dim;
  float* ph = dbias != nullptr ? workspace + 2 * nwaves * dim : nullptr;
  const int d = (int)dim;
  const unsigned blocks = (unsigned)(nwaves / 4);
  if (act == GR_ACT_RELU)
    hipLaunchKernelGGL((ln_relu_backward<V, N, GR_ACT_RELU, P>), dim3(blocks), dim3(256), 0, s,
                       g, h, mean, rstd, gamma, beta, d, rows, gh, pg, pb, ph, shift, rowdot);
  else
    hipLaunchKernelGGL((ln_relu_backward<V, N, GR_ACT_ELU, P>), dim3(blocks), dim3(256), 0, s, g,
                       h, mean, rstd, gamma, beta, d, rows, gh, pg, pb, ph, shift, rowdot);
  GR_HIP_CHECK(hipGetLastError());
  // dgamma / dbeta (/ dbias) = column sums of the partials, in wavefront
  // order: the partial matrices follow one another in the workspace, and
  // one launch reduces all of them.
  hipLaunchKernelGGL(colsum_final3, dim3(final_blocks(d), (unsigned)nparts), dim3(256), 0, s, pg,
                     (int)nwaves, d, dgamma, dbeta, dbias);
  GR_HIP_CHECK(hipGetLastError());
  return GR_OK;
}

}  // namespace gr_agg

extern "C" int gr_ln_act_backward(const float* g, const float* h, const float* mean,
                                  const float* rstd, const float* gamma, const float* beta,
                                  int32_t act, int64_t rows, int64_t dim, float* gh, float* dgamma,
                                  float* dbeta, float* dbias, const float* shift, float* rowdot,
                                  float* workspace, int64_t workspace_floats, void* stream) {
  gr::clear_error();
  int vec, nch;
  GR_REQUIRE(rows >= 0 && dim >= 1 && fused_shape(dim, &vec, &nch),
             "ln_relu_backward: dim %lld unsupported", (long long)dim);
  GR_REQUIRE(act == GR_ACT_RELU || act == GR_ACT_ELU, "ln_act_backward: unknown activation %d",
             act);
  GR_REQUIRE(gamma && beta && dgamma && dbeta && workspace &&
                 (rows == 0 || (g && h && mean && rstd && gh)),
             "ln_relu_backward: NULL pointer");
  const bool al = gr_agg::aligned(g, 16) && gr_agg::aligned(h, 16) && gr_agg::aligned(gh, 16) &&
                  gr_agg::aligned(gamma, 16) && gr_agg::aligned(beta, 16) &&
                  gr_agg::aligned(workspace, 16) && (shift == nullptr || gr_agg::aligned(shift, 16));
  if (vec == 4 && !al) {
    GR_REQUIRE(dim <= 256, "ln_relu_backward: misaligned rows wider than 256");
    vec = 1;
    nch = dim <= 64 ? 1 : (dim <= 128 ? 2 : 4);
  }
  hipStream_t s = gr::as_stream(stream);
  if (vec == 4) {
    if (nch == 1)
      return gr_agg::run_ln_backward<4, 1>(act, g, h, mean, rstd, gamma, beta, rows, dim, gh,
                                           dgamma, dbeta, dbias, shift, rowdot, workspace, workspace_floats, s);
    if (nch == 2)
      return gr_agg::run_ln_backward<4, 2>(act, g, h, mean, rstd, gamma, beta, rows, dim, gh,
                                           dgamma, dbeta, dbias, shift, rowdot, workspace, workspace_floats, s);
    return gr_agg::run_ln_backward<4, 4>(act, g, h, mean, rstd, gamma, beta, rows, dim, gh,
                                         dgamma, dbeta, dbias, shift, rowdot, workspace, workspace_floats, s);
  }
  if (nch == 1)
    return gr_agg::run_ln_backward<1, 1>(act, g, h, mean, rstd, gamma, beta, rows, dim, gh,
                                         dgamma, dbeta, dbias, shift, rowdot, workspace, workspace_floats, s);
  if (nch == 2)
    return gr_agg::run_ln_backward<1, 2>(act, g, h, mean, rstd, gamma, beta, rows, dim, gh,
                                         dgamma, dbeta, dbias, shift, rowdot, workspace, workspace_floats, s);
  return gr_agg::run_ln_backward<1, 4>(act, g, h, mean, rstd, gamma, beta, rows, dim, gh,
                                       dgamma, dbeta, dbias, shift, rowdot, workspace, workspace_floats, s);
}

namespace gr_agg {

template <int NB>
int run_ln_backward_product(int32_t act, const float* dz, int64_t ldz, int K, const float* bmat,
                            const float* h, const float* mean, const float* rstd,
                            const float* gamma, const float* beta, int64_t rows, float* gh,
                            float* dgamma, float* dbeta, float* dbias, const float* shift,
                            float* rowdot, float* workspace, int64_t workspace_floats,
                            hipStream_t s) {
  constexpr int D = 16 * NB;
  const int kpad = (K + 15) / 16 * 16;
  const size_t lds = lnp_lds_bytes<NB>(kpad);
  // The instance: activation, k slices (K <= 32 or <= 64), with or without
  // the row dot.
  const void* kern = nullptr;
  auto pick = [&](auto actc, auto ksc, auto dotc) {
    kern = reinterpret_cast<const void*>(
        &ln_act_backward_product<NB, decltype(actc)::value, decltype(ksc)::value,
                                 decltype(dotc)::value>);
  };
  auto pick_ks = [&](auto actc, auto dotc) {
    if (kpad <= 32) pick(actc, std::integral_constant<int, 2>{}, dotc);
    else pick(actc, std::integral_constant<int, 4>{}, dotc);
  };
  auto pick_dot = [&](auto actc) {
    if (rowdot != nullptr) pick_ks(actc, std::true_type{});
    else pick_ks(actc, std::false_type{});
  };
  if (act == GR_ACT_RELU) pick_dot(std::integral_constant<int, GR_ACT_RELU>{});
  else pick_dot(std::integral_constant<int, GR_ACT_ELU>{});
  // Workgroups the device holds at once with this LDS size (recomputed per
  // call: the size depends on K).
  int dev = 0, cus = 0, per_cu = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, 256, lds) != hipSuccess)
    per_cu = 1, cus = 256;
  int64_t wgs = std::min<int64_t>((int64_t)std::max(per_cu, 1) * std::max(cus, 1),
                                  std::max<int64_t>(1, (rows + 31) / 32));
  // Partial rows: two per workgroup (one per wavefront pair).
  const int nparts = dbias != nullptr ? 3 : 2;
  const int64_t cap = (workspace_floats / D - 1) / nparts / 2;
  GR_REQUIRE(cap >= 1, "ln_act_backward_product: workspace too small");
  if (wgs > cap) wgs = cap;
  const int64_t prows = 2 * wgs;
  float* pg = workspace;
  float* pb = workspace + prows * D;
  float* ph = dbias != nullptr ? workspace + 2 * prows * D : nullptr;
  void* args[] = {&dz,   &ldz, &K,  &bmat, &h,  &mean, &rstd,  &gamma, &beta,
                  &rows, &gh,  &pg, &pb,   &ph, &shift, &rowdot};
  GR_HIP_CHECK(hipLaunchKernel(kern, dim3((unsigned)wgs), dim3(256), args, lds, s));
  GR_HIP_CHECK(hipGetLastError());
  hipLaunchKernelGGL(colsum_final3, dim3(final_blocks(D), (unsigned)nparts), dim3(256), 0, s, pg,
                     (int)prows, D, dgamma, dbeta, dbias);
  GR_HIP_CHECK(hipGetLastError());
  return GR_OK;
}

}  // namespace gr_agg

extern "C" int gr_ln_act_backward_product(const float* dz, int64_t ldz, int64_t k,
                                          const float* bmat, const float* h, const float* mean,
                                          const float* rstd, const float* gamma,
                                          const float* beta, int32_t act, int64_t rows,
                                          int64_t dim, float* gh, float* dgamma, float* dbeta,
                                          float* dbias, const float* shift, float* rowdot,
                                          float* workspace, int64_t workspace_floats,
                                          void* stream) {
  gr::clear_error();
  GR_REQUIRE(rows >= 0 && (dim == 64 || dim == 128 || dim == 192 || dim == 256),
             "ln_act_backward_product: dim %lld must be 64, 128, 192 or 256", (long long)dim);
  GR_REQUIRE(k >= 1 && k <= gr_agg::kLnpMaxK && k % 4 == 0 && ldz >= k && ldz % 4 == 0,
             "ln_act_backward_product: k %lld must be a multiple of 4 in [4, %d], ldz a "
             "multiple of 4 >= k", (long long)k, gr_agg::kLnpMaxK);
  GR_REQUIRE(act == GR_ACT_RELU || act == GR_ACT_ELU,
             "ln_act_backward_product: unknown activation %d", act);
  GR_REQUIRE(bmat && gamma && beta && dgamma && dbeta && workspace &&
                 (rows == 0 || (dz && h && mean && rstd && gh)),
             "ln_act_backward_product: NULL pointer");
  GR_REQUIRE(rows == 0 || gr_agg::aligned(dz, 16),
             "ln_act_backward_product: dz not 16-byte aligned");
  hipStream_t s = gr::as_stream(stream);
  auto run = [&](auto nb) {
    return gr_agg::run_ln_backward_product<decltype(nb)::value>(
        act, dz, ldz, (int)k, bmat, h, mean, rstd, gamma, beta, rows, gh, dgamma, dbeta, dbias,
        shift, rowdot, workspace, workspace_floats, s);
  };
  switch (dim) {
    case 64: return run(std::integral_constant<int, 4>{});
    case 128: return run(std::integral_constant<int, 8>{});
    case 192: return run(std::integral_constant<int, 12>{});
    default: return run(std::integral_constant<int, 16>{});
  }
}

extern "C" int gr_bias_ln_act(const float* z, int64_t ldz, const float* bias,
                              const float* gamma, const float* beta, float eps, int32_t act,
                              int64_t rows, int64_t dim, float* h, float* out, float* mean,
                              float* rstd, void* stream) {
  gr::clear_error();
  int vec, nch;
  GR_REQUIRE(rows >= 0 && dim >= 1 && fused_shape(dim, &vec, &nch),
             "bias_ln_relu: dim %lld unsupported (max 1024)", (long long)dim);
  GR_REQUIRE(ldz >= dim, "bias_ln_relu: ldz < dim");
  GR_REQUIRE(act == GR_ACT_RELU || act == GR_ACT_ELU, "bias_ln_act: unknown activation %d", act);
  GR_REQUIRE(h != z || ldz == dim, "bias_ln_relu: in-place h needs ldz == dim");
  if (rows == 0) return GR_OK;
  GR_REQUIRE(z && gamma && beta && h && out && mean && rstd, "bias_ln_relu: NULL pointer");
  if (vec == 4) {
    const bool al = gr_agg::aligned(z, 16) && ldz % 4 == 0 && gr_agg::aligned(h, 16) &&
                    gr_agg::aligned(out, 16) && gr_agg::aligned(gamma, 16) &&
                    gr_agg::aligned(beta, 16) && (bias == nullptr || gr_agg::aligned(bias, 16));
    if (!al) {
      GR_REQUIRE(dim <= 256, "bias_ln_relu: misaligned rows wider than 256");
      vec = 1;
      nch = dim <= 64 ? 1 : (dim <= 128 ? 2 : 4);
    }
  }
  hipStream_t s = gr::as_stream(stream);
  const int d = (int)dim;
  const unsigned blocks = (unsigned)std::min<int64_t>(8192, (rows + 3) / 4);
#define GR_BLR(V, N)                                                                        \
  do {                                                                                      \
    if (act == GR_ACT_RELU)                                                                 \
      hipLaunchKernelGGL((gr_agg::bias_ln_relu_rows<V, N, GR_ACT_RELU>), dim3(blocks),      \
                         dim3(256), 0, s, z, ldz, bias, gamma, beta, eps, d, rows, h, out,  \
                         mean, rstd);                                                       \
    else                                                                                    \
      hipLaunchKernelGGL((gr_agg::bias_ln_relu_rows<V, N, GR_ACT_ELU>), dim3(blocks),       \
                         dim3(256), 0, s, z, ldz, bias, gamma, beta, eps, d, rows, h, out,  \
                         mean, rstd);                                                       \
  } while (0)
  if (vec == 4) {
    if (nch == 1) GR_BLR(4, 1); else if (nch == 2) GR_BLR(4, 2); else GR_BLR(4, 4);
  } else {
    if (nch == 1) GR_BLR(1, 1); else if (nch == 2) GR_BLR(1, 2); else GR_BLR(1, 4);
  }
#undef GR_BLR
  GR_HIP_CHECK(hipGetLastError());
  return GR_OK;
}
