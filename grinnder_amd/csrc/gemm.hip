// Weight-gradient GEMM for the dense per-layer transform: C[M,N] = A^T B with
// A [K, M] and B [K, N] row-major and K (the node count) in the millions,
// M, N <= a few hundred.  fp32 on the gfx950 matrix cores
// (v_mfma_f32_16x16x4_f32), deterministic split-K.
//
// Workgroup tile 128 x 128 (4 wavefronts as 2 x 2 tiles of 64 x 64, each
// 4 x 4 MFMA blocks of 16 x 16); K is walked in steps of 16 rows staged in LDS,
// with the next step's global loads issued before the current step's MFMAs.
// Workgroup (tile t, chunk z) owns the K rows [z*kchunk, (z+1)*kchunk) and
// writes its partial tile to part[z]; the partials are then summed over z in
// order, so the result does not depend on scheduling.
//
// Workgroups are dispatched round-robin over the 8 XCDs (linear id mod 8), and
// each XCD has its own L2.  The linear id is decoded so that the T output tiles
// of one K chunk are consecutive workgroups of the same XCD: the A and B rows
// of that chunk are fetched from HBM once and re-read from that XCD's L2.
#include <algorithm>

#include "gr_internal.h"

namespace gr_gemm {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int TM = 128;
constexpr int TN = 128;
constexpr int TK = 16;
constexpr int PAD = 16;  // LDS row padding: rows k and k+1 land 16 banks apart

// Loads rows [k, k + TK) x columns [c0, c0 + 128) of a row-major [K, ld]
// matrix into registers: 2048 floats per workgroup, 8 per thread.  Out-of-range
// elements read as 0.
template <int VEC>
__device__ __forceinline__ void load_tile(const float* __restrict__ src, int64_t ld, int64_t k,
                                          int64_t k_end, int c0, int cols, float (&r)[8]) {
  const int tid = threadIdx.x;
  if constexpr (VEC == 4) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int idx = tid + i * 256;  // 512 float4 slots: 16 rows x 32
      const int row = idx >> 5;
      const int c = c0 + (idx & 31) * 4;
      const int64_t kr = k + row;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (kr < k_end && c < cols) v = *reinterpret_cast<const float4*>(src + kr * ld + c);
      r[i * 4 + 0] = v.x;
      r[i * 4 + 1] = v.y;
      r[i * 4 + 2] = v.z;
      r[i * 4 + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int idx = tid + i * 256;  // 2048 slots: 16 rows x 128
      const int row = idx >> 7;
      const int c = c0 + (idx & 127);
      const int64_t kr = k + row;
      r[i] = (kr < k_end && c < cols) ? src[kr * ld + c] : 0.f;
    }
  }
}

template <int VEC>
__device__ __forceinline__ void store_tile(float (*lds)[TM + PAD], const float (&r)[8]) {
  const int tid = threadIdx.x;
  if constexpr (VEC == 4) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int idx = tid + i * 256;
      const int row = idx >> 5;
      const int c = (idx & 31) * 4;
      *reinterpret_cast<float4*>(&lds[row][c]) =
          make_float4(r[i * 4 + 0], r[i * 4 + 1], r[i * 4 + 2], r[i * 4 + 3]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int idx = tid + i * 256;
      lds[idx >> 7][idx & 127] = r[i];
    }
  }
}

constexpr int kXcds = 8;

template <int VA, int VB>
__global__ __launch_bounds__(256) void gemm_tn_splitk(const float* __restrict__ A, int64_t lda,
                                                      const float* __restrict__ B, int64_t ldb,
                                                      int M, int N, int64_t K, int64_t kchunk,
                                                      int nchunks, int tiles_m, int tiles,
                                                      float* __restrict__ part) {
  __shared__ float As[TK][TM + PAD];
  __shared__ float Bs[TK][TN + PAD];
  const int w = blockIdx.x;
  const int q = w / kXcds;
  const int t = q % tiles;
  const int z = (q / tiles) * kXcds + w % kXcds;
  if (z >= nchunks) return;  // whole workgroup: no barrier is pending
  const int m0 = (t % tiles_m) * TM;
  const int n0 = (t / tiles_m) * TN;
  const int64_t k_begin = (int64_t)z * kchunk;
  const int64_t k_end = k_begin + kchunk < K ? k_begin + kchunk : K;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = (wave & 1) * 64;
  const int wn = (wave >> 1) * 64;
  const int lr = lane & 15;  // row (A) / column (B) inside a 16-block
  const int lk = lane >> 4;  // k inside a 4-step

  floatx4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  float ra[8], rb[8];
  load_tile<VA>(A, lda, k_begin, k_end, m0, M, ra);
  load_tile<VB>(B, ldb, k_begin, k_end, n0, N, rb);
  for (int64_t k = k_begin; k < k_end; k += TK) {
    __syncthreads();  // previous step's MFMA reads of the LDS tiles are done
    store_tile<VA>(As, ra);
    store_tile<VB>(Bs, rb);
    __syncthreads();
    if (k + TK < k_end) {
      load_tile<VA>(A, lda, k + TK, k_end, m0, M, ra);
      load_tile<VB>(B, ldb, k + TK, k_end, n0, N, rb);
    }
#pragma unroll
    for (int kk = 0; kk < TK; kk += 4) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = As[kk + lk][wm + i * 16 + lr];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = Bs[kk + lk][wn + j * 16 + lr];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[j], acc[i][j], 0, 0, 0);
    }
  }

  // 16x16 result block: lane holds column lr, rows 4*lk + r (r = 0..3).
  float* out = part + (int64_t)z * M * N;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + wn + j * 16 + lr;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + wm + i * 16 + lk * 4 + r;
        if (m < M && n < N) out[(int64_t)m * N + n] = acc[i][j][r];
      }
    }
}

// C[e] = sum_z part[z][e] in z order (e over M*N elements, grid-stride).
__global__ __launch_bounds__(256) void sum_partials(const float* __restrict__ part, int splits,
                                                    int64_t elems, float beta,
                                                    float* __restrict__ c) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < elems; e += stride) {
    float s = 0.f;
    int z = 0;
    for (; z + 4 <= splits; z += 4) {
      const float a0 = part[(int64_t)(z + 0) * elems + e];
      const float a1 = part[(int64_t)(z + 1) * elems + e];
      const float a2 = part[(int64_t)(z + 2) * elems + e];
      const float a3 = part[(int64_t)(z + 3) * elems + e];
      s += a0;
      s += a1;
      s += a2;
      s += a3;
    }
    for (; z < splits; ++z) s += part[(int64_t)z * elems + e];
    c[e] = beta != 0.f ? fmaf(beta, c[e], s) : s;
  }
}

}  // namespace gr_gemm

extern "C" int gr_gemm_tn_workspace(int64_t m, int64_t n, int64_t k, int64_t* splits,
                                    int64_t* workspace_floats) {
  gr::clear_error();
  GR_REQUIRE(m >= 1 && n >= 1 && k >= 0 && splits && workspace_floats,
             "gemm_tn_workspace: bad arguments");
  const int64_t tiles = ((m + 127) / 128) * ((n + 127) / 128);
  // About 1024 workgroups (4 per CU, one per SIMD each) in multiples of the
  // XCD count, with at least 8 K-steps per workgroup.
  int64_t s = (1024 + tiles - 1) / tiles;
  s = (s + 7) / 8 * 8;
  const int64_t max_s = std::max<int64_t>(1, k / (8 * 16));
  if (s > max_s) s = max_s;
  if (s > 4096) s = 4096;
  if (s < 1) s = 1;
  *splits = s;
  *workspace_floats = s * m * n;
  return GR_OK;
}

extern "C" int gr_gemm_tn(const float* a, int64_t lda, const float* b, int64_t ldb, int64_t m,
                          int64_t n, int64_t k, float beta, float* c, float* workspace,
                          int64_t workspace_floats, int64_t splits, void* stream) {
  using namespace gr_gemm;
  gr::clear_error();
  GR_REQUIRE(m >= 1 && n >= 1 && k >= 0 && m <= 65535 * 128 && n <= 65535 * 128,
             "gemm_tn: bad shape %lld x %lld x %lld", (long long)m, (long long)n, (long long)k);
  GR_REQUIRE(lda >= m && ldb >= n, "gemm_tn: leading dimension too small");
  GR_REQUIRE(splits >= 1 && splits <= 65535, "gemm_tn: splits %lld out of range",
             (long long)splits);
  GR_REQUIRE(c != nullptr && workspace != nullptr && (k == 0 || (a && b)),
             "gemm_tn: NULL pointer");
  hipStream_t s = gr::as_stream(stream);
  int64_t kchunk = (k + splits - 1) / splits;
  kchunk = (kchunk + TK - 1) / TK * TK;
  if (kchunk == 0) kchunk = TK;
  const int64_t used = k == 0 ? 1 : (k + kchunk - 1) / kchunk;
  GR_REQUIRE(used <= splits, "gemm_tn: internal chunking error");
  GR_REQUIRE(workspace_floats >= used * m * n,
             "gemm_tn: workspace of %lld floats, %lld needed", (long long)workspace_floats,
             (long long)(used * m * n));
  const bool va = (lda % 4 == 0) && (m % 4 == 0) && (reinterpret_cast<uintptr_t>(a) % 16 == 0);
  const bool vb = (ldb % 4 == 0) && (n % 4 == 0) && (reinterpret_cast<uintptr_t>(b) % 16 == 0);
  const int tiles_m = (int)((m + TM - 1) / TM);
  const int tiles = tiles_m * (int)((n + TN - 1) / TN);
  const int64_t nwg = (used + kXcds - 1) / kXcds * kXcds * tiles;
  GR_REQUIRE(nwg <= INT32_MAX, "gemm_tn: too many workgroups");
  const dim3 grid((unsigned)nwg);
  if (va && vb)
    hipLaunchKernelGGL((gemm_tn_splitk<4, 4>), grid, dim3(256), 0, s, a, lda, b, ldb, (int)m,
                       (int)n, k, kchunk, (int)used, tiles_m, tiles, workspace);
  else if (va)
    hipLaunchKernelGGL((gemm_tn_splitk<4, 1>), grid, dim3(256), 0, s, a, lda, b, ldb, (int)m,
                       (int)n, k, kchunk, (int)used, tiles_m, tiles, workspace);
  else if (vb)
    hipLaunchKernelGGL((gemm_tn_splitk<1, 4>), grid, dim3(256), 0, s, a, lda, b, ldb, (int)m,
                       (int)n, k, kchunk, (int)used, tiles_m, tiles, workspace);
  else
    hipLaunchKernelGGL((gemm_tn_splitk<1, 1>), grid, dim3(256), 0, s, a, lda, b, ldb, (int)m,
                       (int)n, k, kchunk, (int)used, tiles_m, tiles, workspace);
  GR_HIP_CHECK(hipGetLastError());
  const int64_t elems = m * n;
  const unsigned blocks = (unsigned)std::min<int64_t>(4096, (elems + 255) / 256);
  hipLaunchKernelGGL(sum_partials, dim3(blocks), dim3(256), 0, s, workspace, (int)used, elems,
                     beta, c);
  GR_HIP_CHECK(hipGetLastError());
  return GR_OK;
}
