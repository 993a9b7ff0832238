// Masked softmax cross-entropy and argmax accuracy over the logit rows of a
// partition, fp32, in one pass over the logits, which also writes the
// loss gradient before its scalar scale (the caller's backward multiplies).
//
// Row r carries a mask byte: bit 0 = train (contributes to the loss),
// bit 1 = val, bit 2 = test (contribute to the accuracy counts).  For a row,
//   m = max_c x_c,  lse = m + log(sum_c exp(x_c - m)),  nll = lse - x_y,
//   pred = the first c with x_c == m,
// the arithmetic of torch's log_softmax + NLL and argmax.  Sums and counts
// are reduced in a fixed order (per-workgroup partials in double, then a
// fixed tree), so results do not depend on scheduling.  Labels of train /
// val / test rows outside [0, C) are counted and reported, not read.
// Gradient rows: g[r, c] = exp(x_c - lse) - [c == y] on train rows, 0 on the
// others, i.e. d(sum of train nll)/dx, the backward of log_softmax + NLL.
#include <algorithm>

#include "gr_internal.h"
#include "wave.h"

namespace gr_loss {

constexpr int kStats = 7;  // nll_sum, train_n, val_ok, val_n, test_ok, test_n, bad_labels

using gr_wave::group_max;
using gr_wave::group_min_int;
using gr_wave::group_sum;

// Accumulates one row's contribution to the seven statistics.
__device__ __forceinline__ void add_row_stats(double (&acc)[kStats], uint8_t mk, bool ok_label,
                                              float lse, float xy, bool hit) {
  if (mk != 0 && !ok_label) {
    acc[6] += 1.0;
    return;
  }
  if (mk & 1) {
    acc[0] += (double)(lse - xy);
    acc[1] += 1.0;
  }
  if (mk & 2) {
    acc[2] += hit ? 1.0 : 0.0;
    acc[3] += 1.0;
  }
  if (mk & 4) {
    acc[4] += hit ? 1.0 : 0.0;
    acc[5] += 1.0;
  }
}

// Ordered sum of the workgroup's 256 per-thread statistics into part[blockIdx]:
// a butterfly inside each wavefront, then the 4 wavefront sums in order.
__device__ __forceinline__ void block_stats(double (&acc)[kStats], double* __restrict__ part) {
  __shared__ double red[4][kStats];
#pragma unroll
  for (int k = 0; k < kStats; ++k) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) acc[k] += __shfl_xor(acc[k], off, 64);
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
#pragma unroll
    for (int k = 0; k < kStats; ++k) red[wave][k] = acc[k];
  }
  __syncthreads();
  if (threadIdx.x < kStats) {
    const int k = threadIdx.x;
    part[(int64_t)blockIdx.x * kStats + k] = ((red[0][k] + red[1][k]) + red[2][k]) + red[3][k];
  }
}

// C <= 63: one thread per row.  The workgroup's 256 rows are loaded with
// coalesced accesses into LDS (row stride CP = C rounded up to odd, so the
// per-thread row walks hit distinct banks), each thread reduces its row from
// LDS, writes its gradient row back into LDS, and the workgroup stores the
// gradient rows with coalesced accesses.
constexpr int kRowsPerBlock = 256;
constexpr int kSmallC = 63;  // 256 rows x 63 floats = 63 KiB of LDS, within 64 KiB

__global__ __launch_bounds__(256) void xent_rows_small(const float* __restrict__ x, int64_t ld,
                                                       int64_t rows, int C,
                                                       const int64_t* __restrict__ labels,
                                                       const uint8_t* __restrict__ mask,
                                                       float* __restrict__ lse_out,
                                                       float* __restrict__ grad, int64_t ldg,
                                                       double* __restrict__ part) {
  extern __shared__ float tile[];  // kRowsPerBlock * (C | 1) floats
  const int CP = C | 1;
  const int64_t row0 = (int64_t)blockIdx.x * kRowsPerBlock;
  const int nr = (int)min<int64_t>(kRowsPerBlock, rows - row0);
  const int n = nr * C;
  // Dense rows of odd width: the tile is a straight copy (16-byte accesses
  // when aligned); otherwise element by element into the padded layout.
  const bool linear = CP == C && ld == C;
  if (linear) {
    const float* src = x + row0 * C;
    if ((reinterpret_cast<uintptr_t>(src) & 15) == 0) {
      const int n4 = n / 4;
      for (int i = threadIdx.x; i < n4; i += 256)
        reinterpret_cast<float4*>(tile)[i] = reinterpret_cast<const float4*>(src)[i];
      for (int i = n4 * 4 + threadIdx.x; i < n; i += 256) tile[i] = src[i];
    } else {
      for (int i = threadIdx.x; i < n; i += 256) tile[i] = src[i];
    }
  } else if ((ld & 3) == 0 && ld - C < 4 && (reinterpret_cast<uintptr_t>(x) & 15) == 0) {
    // Rows padded to a multiple of 4 columns in a 16-byte aligned buffer (the
    // trainer's logit blocks): each row's first C columns, as independent
    // 16-byte pieces, several in flight per thread.  A piece that reaches
    // past column C - 1 is read element by element up to it, so no read
    // leaves the C columns of a row.
    const float* src = x + row0 * ld;
    const int q = (int)(ld >> 2);  // pieces per row
    const int n4 = nr * q;
#pragma unroll 4
    for (int i = threadIdx.x; i < n4; i += 256) {
      const int r = i / q, c = (i - r * q) * 4;
      if (c >= C) continue;
      const float* p = src + (int64_t)r * ld + c;
      float* trow = tile + r * CP + c;
      if (c + 4 <= C) {
        const float4 v = *reinterpret_cast<const float4*>(p);
        trow[0] = v.x;
        trow[1] = v.y;
        trow[2] = v.z;
        trow[3] = v.w;
      } else {
        for (int j = 0; c + j < C; ++j) trow[j] = p[j];
      }
    }
  } else {
    // (r, c) of element i advance by (256 / C, 256 % C) per step.
    const int dq = 256 / C, dr = 256 - dq * C;
    int r = threadIdx.x / C, c = threadIdx.x - r * C;
    for (int i = threadIdx.x; i < n; i += 256) {
      tile[r * CP + c] = x[(row0 + r) * ld + c];
      r += dq;
      c += dr;
      if (c >= C) {
        c -= C;
        ++r;
      }
    }
  }
  __syncthreads();
  double acc[kStats];
#pragma unroll
  for (int k = 0; k < kStats; ++k) acc[k] = 0.0;
  const int t = threadIdx.x;
  if (t < nr) {
    float* row = tile + t * CP;
    float m = row[0];
    int first = 0;
    for (int c = 1; c < C; ++c) {
      const float v = row[c];
      if (v > m) {
        m = v;
        first = c;
      }
    }
    float s = 0.f;
    for (int c = 0; c < C; ++c) s += expf(row[c] - m);
    const float lse = m + logf(s);
    const int64_t r = row0 + t;
    const uint8_t mk = mask[r];
    const int64_t y = labels[r];
    const bool ok_label = y >= 0 && y < C;
    const float xy = ok_label ? row[y] : 0.f;
    if (lse_out != nullptr) lse_out[r] = lse;
    add_row_stats(acc, mk, ok_label, lse, xy, first == (int)y);
    if (grad != nullptr) {
      const bool train = (mk & 1) && ok_label;
      for (int c = 0; c < C; ++c)
        row[c] = train ? expf(row[c] - lse) - (c == (int)y ? 1.f : 0.f) : 0.f;
    }
  }
  if (grad != nullptr) {
    __syncthreads();
    float* dst = grad + row0 * ldg;
    if (CP == C && ldg == C) {
      if ((reinterpret_cast<uintptr_t>(dst) & 15) == 0) {
        const int n4 = n / 4;
        for (int i = threadIdx.x; i < n4; i += 256)
          reinterpret_cast<float4*>(dst)[i] = reinterpret_cast<const float4*>(tile)[i];
        for (int i = n4 * 4 + threadIdx.x; i < n; i += 256) dst[i] = tile[i];
      } else {
        for (int i = threadIdx.x; i < n; i += 256) dst[i] = tile[i];
      }
    } else {
      const int dq = 256 / C, dr = 256 - dq * C;
      int r = threadIdx.x / C, c = threadIdx.x - r * C;
      for (int i = threadIdx.x; i < n; i += 256) {
        dst[(int64_t)r * ldg + c] = tile[r * CP + c];
        r += dq;
        c += dr;
        if (c >= C) {
          c -= C;
          ++r;
        }
      }
    }
  }
  block_stats(acc, part);
}

// C > 63: one wavefront per row (lanes over columns), 64 rows per wavefront
// of a 256-row workgroup.
__global__ __launch_bounds__(256) void xent_rows_wide(const float* __restrict__ x, int64_t ld,
                                                      int64_t rows, int C,
                                                      const int64_t* __restrict__ labels,
                                                      const uint8_t* __restrict__ mask,
                                                      float* __restrict__ lse_out,
                                                      float* __restrict__ grad, int64_t ldg,
                                                      double* __restrict__ part) {
  const int lane = threadIdx.x & 63;
  const int64_t row0 = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6) * 64;
  double acc[kStats];
#pragma unroll
  for (int k = 0; k < kStats; ++k) acc[k] = 0.0;
  for (int64_t r = row0; r < row0 + 64 && r < rows; ++r) {
    const float* row = x + r * ld;
    float m = -INFINITY;
    for (int c = lane; c < C; c += 64) m = fmaxf(m, row[c]);
    m = group_max<64>(m);
    float s = 0.f;
    int first = C;
    for (int c = lane; c < C; c += 64) {
      const float v = row[c];
      s += expf(v - m);
      if (v == m && c < first) first = c;
    }
    s = group_sum<64>(s);
    first = group_min_int<64>(first);
    const float lse = m + logf(s);
    const uint8_t mk = mask[r];
    const int64_t y = labels[r];
    const bool ok_label = y >= 0 && y < C;
    if (grad != nullptr) {
      const bool train = (mk & 1) && ok_label;
      float* g = grad + r * ldg;
      for (int c = lane; c < C; c += 64)
        g[c] = train ? expf(row[c] - lse) - (c == (int)y ? 1.f : 0.f) : 0.f;
    }
    if (lane == 0) {
      if (lse_out != nullptr) lse_out[r] = lse;
      add_row_stats(acc, mk, ok_label, lse, ok_label ? row[y] : 0.f, first == (int)y);
    }
  }
  block_stats(acc, part);
}

// Sums the per-workgroup partials: thread t adds workgroups t, t+256, ... in
// order, then a fixed tree over the 256 threads; writes the loss (sum, or
// mean over train rows when `mean`) and the integer statistics.
__global__ __launch_bounds__(256) void xent_finish(const double* __restrict__ part, int64_t nblk,
                                                   int mean, float* __restrict__ loss,
                                                   int64_t* __restrict__ stats) {
  double acc[kStats];
#pragma unroll
  for (int k = 0; k < kStats; ++k) acc[k] = 0.0;
  for (int64_t b = threadIdx.x; b < nblk; b += 256) {
#pragma unroll
    for (int k = 0; k < kStats; ++k) acc[k] += part[b * kStats + k];
  }
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
  if (threadIdx.x == 0) {
    const double n_train = red[1][0];
    *loss = (float)((mean && n_train > 0.0) ? red[0][0] / n_train : red[0][0]);
  } else if (threadIdx.x < kStats) {
    stats[threadIdx.x - 1] = (int64_t)red[threadIdx.x][0];
  }
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
  const int64_t nblk = std::max<int64_t>(1, (rows + kRowsPerBlock - 1) / kRowsPerBlock);
  GR_REQUIRE(nblk <= INT32_MAX, "xent_forward: too many rows");
  GR_REQUIRE(workspace_doubles >= nblk * kStats, "xent_forward: workspace of %lld doubles, "
             "%lld needed", (long long)workspace_doubles, (long long)(nblk * kStats));
  hipStream_t s = gr::as_stream(stream);
  const int c = (int)classes;
  // With rows == 0 the single workgroup writes zero partials.
  if (classes <= kSmallC)
    hipLaunchKernelGGL(xent_rows_small, dim3((unsigned)nblk), dim3(256),
                       (size_t)kRowsPerBlock * (c | 1) * sizeof(float), s, logits, ld, rows, c,
                       labels, mask, lse, grad, ldg, workspace);
  else
    hipLaunchKernelGGL(xent_rows_wide, dim3((unsigned)nblk), dim3(256), 0, s, logits, ld, rows, c,
                       labels, mask, lse, grad, ldg, workspace);
  GR_HIP_CHECK(hipGetLastError());
  hipLaunchKernelGGL(xent_finish, dim3(1), dim3(256), 0, s, workspace, nblk, (int)mean, loss,
                     stats);
  GR_HIP_CHECK(hipGetLastError());
  return GR_OK;
}
