// Masked softmax cross-entropy and argmax accuracy over the logit rows of a
// partition, fp32, in one pass over the logits, which also writes the
// loss gradient before its scalar scale (the caller's backward multiplies).
//
// Row r carries a mask byte: bit 0 = train (contributes to the loss),
// bit 1 = val, bit 2 = test (contribute to the accuracy counts).  For a row,
//   m = max_c x_c,  lse = m + log(sum_c exp(x_c - m)),  nll = lse - x_y,
//   pred = the first c with x_c == m,
// the arithmetic of torch's log_softmax + NLL and argmax.  Sums and counts
// are reduced in a fixed order (per-workgroup partials in double, then one
// ordered pass), so results do not depend on scheduling.  Labels of train /
// val / test rows outside [0, C) are counted and reported, not read.
// Gradient rows: g[r, c] = exp(x_c - lse) - [c == y] on train rows, 0 on the
// others, i.e. d(sum of train nll)/dx, the backward of log_softmax + NLL.
#include <algorithm>

#include "gr_internal.h"

namespace gr_loss {

constexpr int kStats = 7;  // nll_sum, train_n, val_ok, val_n, test_ok, test_n, bad_labels
constexpr int kMaxBlocks = 1024;

template <int G>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
  for (int off = G / 2; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, G));
  return v;
}

template <int G>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int off = G / 2; off >= 1; off >>= 1) v += __shfl_xor(v, off, G);
  return v;
}

template <int G>
__device__ __forceinline__ int group_min_int(int v) {
#pragma unroll
  for (int off = G / 2; off >= 1; off >>= 1) v = min(v, __shfl_xor(v, off, G));
  return v;
}

// G lanes per row (64 / G rows per wavefront); each lane owns columns
// lane_in_row + k * G.  Grid-stride over row groups; per-thread partial
// statistics, then an ordered reduction inside the workgroup.
template <int G>
__global__ __launch_bounds__(256) void xent_forward(const float* __restrict__ x, int64_t ld,
                                                   int64_t rows, int C,
                                                   const int64_t* __restrict__ labels,
                                                   const uint8_t* __restrict__ mask,
                                                   float* __restrict__ lse_out,
                                                   float* __restrict__ grad, int64_t ldg,
                                                   double* __restrict__ part) {
  constexpr int RPW = 64 / G;  // rows per wavefront
  const int lane = threadIdx.x & 63;
  const int sub = lane / G;
  const int li = lane % G;
  const int64_t wave = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t nwaves = (int64_t)gridDim.x * 4;
  double acc[kStats];
#pragma unroll
  for (int k = 0; k < kStats; ++k) acc[k] = 0.0;
  for (int64_t r0 = wave * RPW; r0 < rows; r0 += nwaves * RPW) {
    const int64_t r = r0 + sub;
    const bool live = r < rows;
    const float* row = x + (live ? r : 0) * ld;
    float m = -INFINITY;
    for (int c = li; c < C; c += G) m = fmaxf(m, live ? row[c] : -INFINITY);
    m = group_max<G>(m);
    float s = 0.f;
    int first = C;
    for (int c = li; c < C; c += G) {
      const float v = live ? row[c] : 0.f;
      s += expf(v - m);
      if (v == m && c < first) first = c;
    }
    s = group_sum<G>(s);
    first = group_min_int<G>(first);
    const float lse = m + logf(s);
    const uint8_t mk = live ? mask[r] : 0;
    const int64_t y = live ? labels[r] : 0;
    const bool ok_label = y >= 0 && y < C;
    // x_y: the one lane owning column y contributes it.
    float xy = 0.f;
    if (ok_label && (int)(y % G) == li) xy = row[y];
    xy = group_sum<G>(xy);
    if (grad != nullptr && live) {
      const bool train = (mk & 1) && ok_label;
      float* g = grad + r * ldg;
      for (int c = li; c < C; c += G)
        g[c] = train ? expf(row[c] - lse) - (c == (int)y ? 1.f : 0.f) : 0.f;
    }
    if (li == 0 && live) {
      if (lse_out != nullptr) lse_out[r] = lse;
      if (mk != 0 && !ok_label) {
        acc[6] += 1.0;
      } else {
        if (mk & 1) {
          acc[0] += (double)(lse - xy);
          acc[1] += 1.0;
        }
        const double hit = (first == (int)y) ? 1.0 : 0.0;
        if (mk & 2) {
          acc[2] += hit;
          acc[3] += 1.0;
        }
        if (mk & 4) {
          acc[4] += hit;
          acc[5] += 1.0;
        }
      }
    }
  }
  // Ordered reduction of the 256 threads' partials (only li == 0 lanes hold
  // non-zero values; the tree order is fixed).
  __shared__ double red[kStats][256];
#pragma unroll
  for (int k = 0; k < kStats; ++k) red[k][threadIdx.x] = acc[k];
  __syncthreads();
  for (int w = 128; w >= 1; w >>= 1) {
    if ((int)threadIdx.x < w) {
#pragma unroll
      for (int k = 0; k < kStats; ++k) red[k][threadIdx.x] += red[k][threadIdx.x + w];
    }
    __syncthreads();
  }
  if (threadIdx.x < kStats) part[(int64_t)blockIdx.x * kStats + threadIdx.x] = red[threadIdx.x][0];
}

// Sums the per-workgroup partials in workgroup order; writes the loss (sum,
// or mean over train rows when `mean`) and the integer statistics.
__global__ __launch_bounds__(64) void xent_finish(const double* __restrict__ part, int nblk,
                                                  int mean, float* __restrict__ loss,
                                                  int64_t* __restrict__ stats) {
  double t = 0.0;
  if (threadIdx.x < kStats)
    for (int b = 0; b < nblk; ++b) t += part[(int64_t)b * kStats + threadIdx.x];
  // Lane k holds statistic k; the mean needs the train count (lane 1).
  const double n_train = __shfl(t, 1, 64);
  if (threadIdx.x == 0) {
    *loss = (float)((mean && n_train > 0.0) ? t / n_train : t);
  } else if (threadIdx.x < kStats) {
    stats[threadIdx.x - 1] = (int64_t)t;
  }
}

inline int lanes_for(int64_t C) {
  if (C <= 8) return 8;
  if (C <= 16) return 16;
  if (C <= 32) return 32;
  return 64;
}

inline int64_t blocks_for(int64_t rows, int G) {
  const int64_t rows_per_block = 4 * (64 / G);
  return std::max<int64_t>(1, std::min<int64_t>(kMaxBlocks, (rows + rows_per_block - 1) /
                                                                 rows_per_block));
}

}  // namespace gr_loss

extern "C" int gr_xent_forward(const float* logits, int64_t ld, int64_t rows, int64_t classes,
                               const int64_t* labels, const uint8_t* mask, int32_t mean,
                               float* lse, float* grad, int64_t ldg, float* loss,
                               int64_t* stats, double* workspace, int64_t workspace_doubles,
                               void* stream) {
  using namespace gr_loss;
  gr::clear_error();
  GR_REQUIRE(rows >= 0 && classes >= 1 && classes <= (1 << 24) && ld >= classes,
             "xent_forward: bad shape (%lld rows, %lld classes, ld %lld)", (long long)rows,
             (long long)classes, (long long)ld);
  GR_REQUIRE(loss && stats && workspace, "xent_forward: NULL output");
  GR_REQUIRE(rows == 0 || (logits && labels && mask), "xent_forward: NULL input");
  GR_REQUIRE(grad == nullptr || ldg >= classes, "xent_forward: ldg < classes");
  const int G = lanes_for(classes);
  const int64_t nblk = blocks_for(rows, G);
  GR_REQUIRE(workspace_doubles >= nblk * kStats, "xent_forward: workspace of %lld doubles, "
             "%lld needed", (long long)workspace_doubles, (long long)(nblk * kStats));
  hipStream_t s = gr::as_stream(stream);
  const int c = (int)classes;
#define GR_XF(GG)                                                                            \
  hipLaunchKernelGGL((xent_forward<GG>), dim3((unsigned)nblk), dim3(256), 0, s, logits, ld, \
                     rows, c, labels, mask, lse, grad, ldg, workspace)
  if (G == 8) GR_XF(8); else if (G == 16) GR_XF(16); else if (G == 32) GR_XF(32); else GR_XF(64);
#undef GR_XF
  GR_HIP_CHECK(hipGetLastError());
  hipLaunchKernelGGL(xent_finish, dim3(1), dim3(64), 0, s, workspace, (int)nblk, (int)mean, loss,
                     stats);
  GR_HIP_CHECK(hipGetLastError());
  return GR_OK;
}
