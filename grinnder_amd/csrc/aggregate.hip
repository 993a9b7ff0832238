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
#include "gr_internal.h"

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
template <int VEC, int G, int NCH, int U>
__global__ __launch_bounds__(256) void aggregate_units(
    const int4* __restrict__ units, int64_t n_units, const int32_t* __restrict__ idx,
    const float* __restrict__ val, const float* __restrict__ x, int64_t ldx,
    float* __restrict__ y, int64_t ldy, const float* __restrict__ bias, int dim,
    float* __restrict__ ws) {
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
    for (int off = G; off < 64; off <<= 1)
#pragma unroll
      for (int ch = 0; ch < NCH; ++ch)
#pragma unroll
        for (int j = 0; j < VEC; ++j) acc[ch][j] += __shfl_xor(acc[ch][j], off, 64);
  }
  if (slot != 0) return;

  if (w.w < 0) {
    float* out = y + (int64_t)w.x * ldy;
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) {
      if (!fvalid[ch]) continue;
      if (bias != nullptr) {
        float b[VEC];
        load_vec<VEC>(bias + foff[ch], b);
#pragma unroll
        for (int j = 0; j < VEC; ++j) acc[ch][j] += b[j];
      }
      store_vec<VEC>(out + foff[ch], acc[ch]);
    }
  } else {
    float* out = ws + (int64_t)w.w * dim;
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) {
      if (fvalid[ch]) store_vec<VEC>(out + foff[ch], acc[ch]);
    }
  }
}

// Ordered reduction of the partial sums of split rows: one workgroup per
// (split row, 256-feature chunk), one thread per feature; the slot loop is
// unrolled so its loads are independent.
__global__ __launch_bounds__(256) void aggregate_fixup(const int32_t* __restrict__ fix,
                                                       const float* __restrict__ ws, int dim,
                                                       float* __restrict__ y, int64_t ldy,
                                                       const float* __restrict__ bias) {
  const int64_t r = blockIdx.x;
  const int f = blockIdx.y * 256 + threadIdx.x;
  if (f >= dim) return;
  const int row = fix[3 * r + 0];
  const int first = fix[3 * r + 1];
  const int n = fix[3 * r + 2];
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
  y[(int64_t)row * ldy + f] = s;
}

// Column sums of a [rows, dim] matrix, two passes, fixed order: workgroup b
// sums rows [b*chunk, (b+1)*chunk) into part[b, :]; then part is reduced over
// b in ascending order.  Each thread owns columns f = tid, tid + 256, ...
__global__ __launch_bounds__(256) void colsum_partial(const float* __restrict__ x, int64_t rows,
                                                      int dim, int64_t ldx, int64_t chunk,
                                                      float* __restrict__ part) {
  const int64_t r0 = (int64_t)blockIdx.x * chunk;
  const int64_t r1 = r0 + chunk < rows ? r0 + chunk : rows;
  for (int f = threadIdx.x; f < dim; f += 256) {
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
    int64_t r = r0;
    for (; r + 4 <= r1; r += 4) {
      a0 += x[(r + 0) * ldx + f];
      a1 += x[(r + 1) * ldx + f];
      a2 += x[(r + 2) * ldx + f];
      a3 += x[(r + 3) * ldx + f];
    }
    for (; r < r1; ++r) a0 += x[r * ldx + f];
    part[(int64_t)blockIdx.x * dim + f] = (a0 + a1) + (a2 + a3);
  }
}

__global__ __launch_bounds__(256) void colsum_final(const float* __restrict__ part, int nblk,
                                                    int dim, float* __restrict__ out) {
  const int f = blockIdx.x * 256 + threadIdx.x;
  if (f >= dim) return;
  float s = 0.f;
  for (int b = 0; b < nblk; ++b) s += part[(int64_t)b * dim + f];
  out[f] = s;
}

template <int VEC, int G, int NCH>
hipError_t launch_units(const int4* units, int64_t n_units, const int32_t* idx,
                        const float* val, const float* x, int64_t ldx, float* y, int64_t ldy,
                        const float* bias, int dim, float* ws, hipStream_t s) {
  constexpr int EPI = 64 / G;
  constexpr int U = (EPI == 1) ? ((NCH == 1) ? 8 : (NCH == 2 ? 4 : 2)) : (EPI == 2 ? 4 : 2);
  const int64_t blocks = (n_units + 3) / 4;
  hipLaunchKernelGGL((aggregate_units<VEC, G, NCH, U>), dim3((unsigned)blocks), dim3(256), 0, s,
                     units, n_units, idx, val, x, ldx, y, ldy, bias, dim, ws);
  return hipGetLastError();
}

template <int VEC>
hipError_t dispatch_g(int chunks, const int4* units, int64_t n_units, const int32_t* idx,
                      const float* val, const float* x, int64_t ldx, float* y, int64_t ldy,
                      const float* bias, int dim, float* ws, hipStream_t s) {
  if (chunks <= 8)
    return launch_units<VEC, 8, 1>(units, n_units, idx, val, x, ldx, y, ldy, bias, dim, ws, s);
  if (chunks <= 16)
    return launch_units<VEC, 16, 1>(units, n_units, idx, val, x, ldx, y, ldy, bias, dim, ws, s);
  if (chunks <= 32)
    return launch_units<VEC, 32, 1>(units, n_units, idx, val, x, ldx, y, ldy, bias, dim, ws, s);
  if (chunks <= 64)
    return launch_units<VEC, 64, 1>(units, n_units, idx, val, x, ldx, y, ldy, bias, dim, ws, s);
  if (chunks <= 128)
    return launch_units<VEC, 64, 2>(units, n_units, idx, val, x, ldx, y, ldy, bias, dim, ws, s);
  return launch_units<VEC, 64, 4>(units, n_units, idx, val, x, ldx, y, ldy, bias, dim, ws, s);
}

inline bool aligned(const void* p, int bytes) {
  return (reinterpret_cast<uintptr_t>(p) % bytes) == 0;
}

}  // namespace gr_agg

extern "C" int gr_gcn_aggregate(const int32_t* units, int64_t n_units, const int32_t* fixups,
                                int64_t n_fix, const int32_t* idx, const float* val,
                                const float* x, int64_t ldx, float* y, int64_t ldy,
                                const float* bias, int64_t rows, int64_t dim, float* workspace,
                                int64_t n_slots, void* stream) {
  using namespace gr_agg;
  gr::clear_error();
  GR_REQUIRE(n_units >= 0 && n_fix >= 0 && n_slots >= 0 && rows >= 0,
             "gcn_aggregate: negative extent");
  GR_REQUIRE(dim >= 1 && dim <= 1024, "gcn_aggregate: dim %lld outside [1, 1024]",
             (long long)dim);
  GR_REQUIRE(ldx >= dim && ldy >= dim, "gcn_aggregate: ldx/ldy smaller than dim");
  GR_REQUIRE(n_units == 0 || (units != nullptr && y != nullptr && x != nullptr),
             "gcn_aggregate: NULL units/x/y");
  GR_REQUIRE(n_fix == 0 || (fixups != nullptr && workspace != nullptr),
             "gcn_aggregate: NULL fixups/workspace with n_fix > 0");
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
  hipError_t err;
  if (vec == 4)
    err = dispatch_g<4>(chunks, u4, n_units, idx, val, x, ldx, y, ldy, bias, d, workspace, s);
  else if (vec == 2)
    err = dispatch_g<2>(chunks, u4, n_units, idx, val, x, ldx, y, ldy, bias, d, workspace, s);
  else
    err = dispatch_g<1>(chunks, u4, n_units, idx, val, x, ldx, y, ldy, bias, d, workspace, s);
  GR_HIP_CHECK(err);
  if (n_fix > 0) {
    GR_REQUIRE(n_fix <= INT32_MAX, "gcn_aggregate: too many split rows");
    const int threads = d >= 256 ? 256 : ((d + 63) / 64) * 64;
    hipLaunchKernelGGL(aggregate_fixup, dim3((unsigned)n_fix, (unsigned)((d + 255) / 256)),
                       dim3(threads), 0, s, fixups, workspace, d, y, ldy, bias);
    GR_HIP_CHECK(hipGetLastError());
  }
  return GR_OK;
}

extern "C" int gr_column_sum(const float* x, int64_t rows, int64_t dim, int64_t ldx, float* out,
                             float* workspace, int64_t workspace_floats, void* stream) {
  gr::clear_error();
  GR_REQUIRE(rows >= 0 && dim >= 1 && ldx >= dim, "column_sum: bad shape");
  GR_REQUIRE(out != nullptr && (rows == 0 || x != nullptr), "column_sum: NULL pointer");
  hipStream_t s = gr::as_stream(stream);
  const int64_t nblk_max = workspace_floats / dim;
  GR_REQUIRE(workspace != nullptr && nblk_max >= 1,
             "column_sum: workspace must hold at least dim floats");
  int64_t nblk = rows == 0 ? 1 : (rows + 2047) / 2048;  // ~2048 rows per workgroup
  if (nblk > 1024) nblk = 1024;
  if (nblk > nblk_max) nblk = nblk_max;
  const int64_t chunk = rows == 0 ? 0 : (rows + nblk - 1) / nblk;
  hipLaunchKernelGGL(gr_agg::colsum_partial, dim3((unsigned)nblk), dim3(256), 0, s, x, rows, (int)dim,
                     ldx, chunk, workspace);
  GR_HIP_CHECK(hipGetLastError());
  hipLaunchKernelGGL(gr_agg::colsum_final, dim3((unsigned)((dim + 255) / 256)), dim3(256), 0, s,
                     workspace, (int)nblk, (int)dim, out);
  GR_HIP_CHECK(hipGetLastError());
  return GR_OK;
}
