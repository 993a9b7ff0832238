// LayerNorm + activation of one row held by a wavefront, shared by the
// aggregation kernels' fused epilogues (GCN: aggregate.hip, GAT: gat.hip)
// and the dense epilogue, so every path forms a row's statistics and output
// with the same arithmetic (bit for bit on the same h).
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/grinnder_amd.h"
#include "wave.h"

namespace gr_ln {

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

__device__ __forceinline__ float wave_sum64(float v) { return gr_wave::wave_sum(v); }

// y = (h - mean) * rstd * gamma + beta; the backward recomputes it with the
// same expression so the activation's branch is bit-identical.
__device__ __forceinline__ float ln_affine(float h, float mean, float rstd, float g, float b) {
  return fmaf((h - mean) * rstd, g, b);
}

// Activations after the LayerNorm: ReLU (GCN) and ELU with alpha = 1 (GAT),
// and their derivatives as functions of the pre-activation y.
template <int ACT>
__device__ __forceinline__ float act_fwd(float y) {
  if constexpr (ACT == GR_ACT_RELU) return fmaxf(y, 0.f);
  else return y > 0.f ? y : expm1f(y);
}

// ELU's derivative exp(y) for y <= 0 on the hardware base-2 exponential:
// relative error about |y| 2^-24 from rounding y log2(e), plus the
// instruction's own (1 ulp); below y = -87 it flushes to zero.
template <int ACT>
__device__ __forceinline__ float act_grad(float y) {
  if constexpr (ACT == GR_ACT_RELU) return y > 0.f ? 1.f : 0.f;
  else return y > 0.f ? 1.f : __builtin_amdgcn_exp2f(y * 1.44269504f);
}

template <int VEC, int NCH, int ACT = GR_ACT_RELU>
__device__ __forceinline__ void ln_relu_store_row(float (&acc)[NCH][VEC], const bool (&fvalid)[NCH],
                                                  const int (&foff)[NCH], int dim,
                                                  const float* __restrict__ gamma,
                                                  const float* __restrict__ beta, float eps,
                                                  float* __restrict__ hrow, float* __restrict__ orow,
                                                  float* __restrict__ mean_out,
                                                  float* __restrict__ rstd_out, int lane) {
  float s = 0.f;
#pragma unroll
  for (int ch = 0; ch < NCH; ++ch)
#pragma unroll
    for (int j = 0; j < VEC; ++j) s += fvalid[ch] ? acc[ch][j] : 0.f;
  const float mean = wave_sum64(s) / (float)dim;
  float q = 0.f;
#pragma unroll
  for (int ch = 0; ch < NCH; ++ch)
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      const float dlt = acc[ch][j] - mean;
      q += fvalid[ch] ? dlt * dlt : 0.f;
    }
  const float var = wave_sum64(q) / (float)dim;
  const float rstd = 1.0f / sqrtf(var + eps);
#pragma unroll
  for (int ch = 0; ch < NCH; ++ch) {
    if (!fvalid[ch]) continue;
    float g[VEC], b[VEC], o[VEC];
    load_vec<VEC>(gamma + foff[ch], g);
    load_vec<VEC>(beta + foff[ch], b);
#pragma unroll
    for (int j = 0; j < VEC; ++j) o[j] = act_fwd<ACT>(ln_affine(acc[ch][j], mean, rstd, g[j], b[j]));
    store_vec<VEC>(hrow + foff[ch], acc[ch]);
    store_vec<VEC>(orow + foff[ch], o);
  }
  if (lane == 0) {
    *mean_out = mean;
    *rstd_out = rstd;
  }
}

// Sum over a 256-thread workgroup in a fixed order (every thread gets it).
__device__ __forceinline__ float block_sum256(float v, float* red) {
  v = wave_sum64(v);
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wv] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

}  // namespace gr_ln
