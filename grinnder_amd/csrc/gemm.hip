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
#include "wave.h"

namespace gr_gemm {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int TM = 128;
constexpr int TN = 128;
constexpr int TK = 16;
constexpr int PAD = 16;  // LDS row padding: rows k and k+1 land 16 banks apart

// Loads rows [k, k + TK) x columns [c0, c0 + W) of a row-major [K, ld] matrix
// into registers: 16 * W floats per workgroup, W / 16 per thread (W = 128 or
// 64).  Out-of-range elements read as 0.
template <int VEC, int W>
__device__ __forceinline__ void load_tile(const float* __restrict__ src, int64_t ld, int64_t k,
                                          int64_t k_end, int c0, int cols,
                                          float (&r)[W / 16]) {
  const int tid = threadIdx.x;
  if constexpr (VEC == 4) {
    constexpr int Q = W / 4;  // float4 slots per row
#pragma unroll
    for (int i = 0; i < W / 64; ++i) {
      const int idx = tid + i * 256;
      const int row = idx / Q;
      const int c = c0 + (idx % Q) * 4;
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
    for (int i = 0; i < W / 16; ++i) {
      const int idx = tid + i * 256;
      const int row = idx / W;
      const int c = c0 + (idx % W);
      const int64_t kr = k + row;
      r[i] = (kr < k_end && c < cols) ? src[kr * ld + c] : 0.f;
    }
  }
}

template <int VEC, int W>
__device__ __forceinline__ void store_tile(float (*lds)[W + PAD], const float (&r)[W / 16]) {
  const int tid = threadIdx.x;
  if constexpr (VEC == 4) {
    constexpr int Q = W / 4;
#pragma unroll
    for (int i = 0; i < W / 64; ++i) {
      const int idx = tid + i * 256;
      const int row = idx / Q;
      const int c = (idx % Q) * 4;
      *reinterpret_cast<float4*>(&lds[row][c]) =
          make_float4(r[i * 4 + 0], r[i * 4 + 1], r[i * 4 + 2], r[i * 4 + 3]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < W / 16; ++i) {
      const int idx = tid + i * 256;
      lds[idx / W][idx % W] = r[i];
    }
  }
}

constexpr int kXcds = 8;

// BN = 128 or 64 output columns per workgroup (64 for narrow N).
template <int VA, int VB, int BN>
__global__ __launch_bounds__(256) void gemm_tn_splitk(const float* __restrict__ A, int64_t lda,
                                                      const float* __restrict__ B, int64_t ldb,
                                                      int M, int N, int64_t K, int64_t kchunk,
                                                      int nchunks, int tiles_m, int tiles,
                                                      float* __restrict__ part) {
  constexpr int NJ = BN / 32;  // 16-column blocks per wavefront
  __shared__ float As[TK][TM + PAD];
  __shared__ float Bs[TK][BN + PAD];
  const int w = blockIdx.x;
  const int q = w / kXcds;
  const int t = q % tiles;
  const int z = (q / tiles) * kXcds + w % kXcds;
  if (z >= nchunks) return;  // whole workgroup: no barrier is pending
  const int m0 = (t % tiles_m) * TM;
  const int n0 = (t / tiles_m) * BN;
  const int64_t k_begin = (int64_t)z * kchunk;
  const int64_t k_end = k_begin + kchunk < K ? k_begin + kchunk : K;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = (wave & 1) * 64;
  const int wn = (wave >> 1) * (BN / 2);
  const int lr = lane & 15;  // row (A) / column (B) inside a 16-block
  const int lk = lane >> 4;  // k inside a 4-step

  floatx4 acc[4][NJ];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  float ra[TM / 16], rb[BN / 16];
  load_tile<VA, TM>(A, lda, k_begin, k_end, m0, M, ra);
  load_tile<VB, BN>(B, ldb, k_begin, k_end, n0, N, rb);
  for (int64_t k = k_begin; k < k_end; k += TK) {
    __syncthreads();  // previous step's MFMA reads of the LDS tiles are done
    store_tile<VA, TM>(As, ra);
    store_tile<VB, BN>(Bs, rb);
    __syncthreads();
    if (k + TK < k_end) {
      load_tile<VA, TM>(A, lda, k + TK, k_end, m0, M, ra);
      load_tile<VB, BN>(B, ldb, k + TK, k_end, n0, N, rb);
    }
#pragma unroll
    for (int kk = 0; kk < TK; kk += 4) {
      float a[4], b[NJ];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = As[kk + lk][wm + i * 16 + lr];
#pragma unroll
      for (int j = 0; j < NJ; ++j) b[j] = Bs[kk + lk][wn + j * 16 + lr];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[j], acc[i][j], 0, 0, 0);
    }
  }

  // 16x16 result block: lane holds column lr, rows 4*lk + r (r = 0..3).
  float* out = part + (int64_t)z * M * N;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int n = n0 + wn + j * 16 + lr;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + wm + i * 16 + lk * 4 + r;
        if (m < M && n < N) out[(int64_t)m * N + n] = acc[i][j][r];
      }
    }
}

// C = sum_z part[z] in z order over the rows x cols partial tiles
// (grid-stride).  With `trans` the partial holds C^T: element (r, q) goes to
// c[q * rows + r].
__global__ __launch_bounds__(256) void sum_partials(const float* __restrict__ part, int splits,
                                                    int64_t rows, int64_t cols, float beta,
                                                    int trans, float* __restrict__ c) {
  const int64_t elems = rows * cols;
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
    const int64_t d = trans ? (e % cols) * rows + e / cols : e;
    c[d] = beta != 0.f ? fmaf(beta, c[d], s) : s;
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
  // A narrow product (m <= 64 < n) runs as C^T = B^T A, so the narrow side
  // falls on 64-column tiles instead of wasting rows of 128-row tiles; the
  // partials are summed into C with a transposed store.
  const bool swap = m <= 64 && n > 64;
  const float* pa = swap ? b : a;
  const float* pb = swap ? a : b;
  const int64_t pm = swap ? n : m, pn = swap ? m : n;
  const int64_t plda = swap ? ldb : lda, pldb = swap ? lda : ldb;
  const bool va = (plda % 4 == 0) && (pm % 4 == 0) && (reinterpret_cast<uintptr_t>(pa) % 16 == 0);
  const bool vb = (pldb % 4 == 0) && (pn % 4 == 0) && (reinterpret_cast<uintptr_t>(pb) % 16 == 0);
  const bool narrow = pn <= 64;
  const int bn = narrow ? 64 : TN;
  const int tiles_m = (int)((pm + TM - 1) / TM);
  const int tiles = tiles_m * (int)((pn + bn - 1) / bn);
  const int64_t nwg = (used + kXcds - 1) / kXcds * kXcds * tiles;
  GR_REQUIRE(nwg <= INT32_MAX, "gemm_tn: too many workgroups");
  const dim3 grid((unsigned)nwg);
#define GR_GT(VA_, VB_, BN_)                                                                   \
  hipLaunchKernelGGL((gemm_tn_splitk<VA_, VB_, BN_>), grid, dim3(256), 0, s, pa, plda, pb, pldb, \
                     (int)pm, (int)pn, k, kchunk, (int)used, tiles_m, tiles, workspace)
  if (narrow) {
    if (va && vb) GR_GT(4, 4, 64); else if (va) GR_GT(4, 1, 64);
    else if (vb) GR_GT(1, 4, 64); else GR_GT(1, 1, 64);
  } else {
    if (va && vb) GR_GT(4, 4, 128); else if (va) GR_GT(4, 1, 128);
    else if (vb) GR_GT(1, 4, 128); else GR_GT(1, 1, 128);
  }
#undef GR_GT
  GR_HIP_CHECK(hipGetLastError());
  const int64_t elems = m * n;
  const unsigned blocks = (unsigned)std::min<int64_t>(4096, (elems + 255) / 256);
  hipLaunchKernelGGL(sum_partials, dim3(blocks), dim3(256), 0, s, workspace, (int)used, pm, pn,
                     beta, (int)swap, c);
  GR_HIP_CHECK(hipGetLastError());
  return GR_OK;
}

// ---------------------------------------------------------------------------
// Dense layer transform with the LayerNorm epilogue in the accumulators:
//   z = x W^T, h = z + bias, out = act(LayerNorm(h)), mean, rstd
// for x [rows, din] (ldx-strided) and W^T [din, dout] (row-major, the
// transposed weight) with dout = 16 * NB <= 256.
// A workgroup takes 64 rows; each wavefront owns 16 complete output rows
// (NB blocks of v_mfma_f32_16x16x4_f32 across the row), so the row statistics
// are reduced inside the wavefront.  K is walked in chunks of 16 columns of x
// and W staged through LDS.  The epilogue uses the same expressions as the
// other LayerNorm epilogues (biased variance, y = (h - mean) * rstd * gamma +
// beta), so the LayerNorm backward applies unchanged.
namespace gr_gemm {

constexpr int LT_ROWS = 64;
constexpr int LT_K = 16;

template <int ACT>
__device__ __forceinline__ float lt_act(float y) {
  if constexpr (ACT == GR_ACT_RELU) return fmaxf(y, 0.f);
  else return y > 0.f ? y : expm1f(y);
}

template <int NB, int ACT>
__global__ __launch_bounds__(256) void linear_ln_act_kernel(
    const float* __restrict__ x, int64_t ldx, int64_t rows, int din,
    const float* __restrict__ wt, const float* __restrict__ bias,
    const float* __restrict__ gamma, const float* __restrict__ beta, float eps,
    float* __restrict__ h, float* __restrict__ out, float* __restrict__ mean,
    float* __restrict__ rstd) {
  constexpr int DOUT = 16 * NB;
  constexpr int WPT = DOUT * LT_K / 256;  // W^T chunk floats per thread (NB)
  __shared__ __align__(16) float Ws[LT_K][DOUT + 16];  // Ws[k][c] = W^T[k0 + k][c]
  static_assert(16 * (DOUT + 4) <= LT_K * (DOUT + 16), "epilogue stage must fit the W tile");
  __shared__ float Xs[LT_ROWS][LT_K + 1];  // Xs[r][k] = x[row0 + r][k0 + k]
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int lr = lane & 15;
  const int lk = lane >> 4;
  const int64_t row0 = (int64_t)blockIdx.x * LT_ROWS;

  floatx4 acc[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) acc[b] = floatx4{0.f, 0.f, 0.f, 0.f};

  // Chunk loads: W^T rows k0..k0+15 (contiguous DOUT floats each) and the
  // 64 x 16 block of x; element e of this thread is e * 256 + tid.
  float wr[WPT], xr[4];
  auto load_chunk = [&](int k0) {
#pragma unroll
    for (int e = 0; e < WPT; ++e) {
      const int i = e * 256 + tid;
      const int k = i / DOUT, c = i % DOUT;
      wr[e] = (k0 + k < din) ? wt[(int64_t)(k0 + k) * DOUT + c] : 0.f;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = e * 256 + tid;
      const int r = i / LT_K, k = i % LT_K;
      xr[e] = (row0 + r < rows && k0 + k < din) ? x[(row0 + r) * ldx + k0 + k] : 0.f;
    }
  };
  load_chunk(0);
  for (int k0 = 0; k0 < din; k0 += LT_K) {
    __syncthreads();  // the previous chunk's reads of Ws / Xs are done
#pragma unroll
    for (int e = 0; e < WPT; ++e) {
      const int i = e * 256 + tid;
      Ws[i / DOUT][i % DOUT] = wr[e];
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = e * 256 + tid;
      Xs[i / LT_K][i % LT_K] = xr[e];
    }
    __syncthreads();
    if (k0 + LT_K < din) load_chunk(k0 + LT_K);
    const int kmax = din - k0 < LT_K ? din - k0 : LT_K;
    for (int kk = 0; kk < kmax; kk += 4) {
      const float a = Xs[wave * 16 + lr][kk + lk];
#pragma unroll
      for (int b = 0; b < NB; ++b)
        acc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, Ws[kk + lk][b * 16 + lr], acc[b], 0, 0,
                                                       0);
    }
  }

  // Lane holds rows 4 * lk + q (q = 0..3) of the wavefront's 16, columns
  // b * 16 + lr.  Row reductions: the 16 lanes sharing lk.
  if (bias != nullptr) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const float bb = bias[b * 16 + lr];
#pragma unroll
      for (int q = 0; q < 4; ++q) acc[b][q] += bb;
    }
  }
  const float inv_d = 1.0f / (float)DOUT;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int64_t row = row0 + wave * 16 + lk * 4 + q;
    float s = 0.f;
#pragma unroll
    for (int b = 0; b < NB; ++b) s += acc[b][q];
    s = gr_wave::group_sum<16>(s);  // the 16 lanes of this row block
    const float mu = s * inv_d;
    float v = 0.f;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const float dlt = acc[b][q] - mu;
      v += dlt * dlt;
    }
    v = gr_wave::group_sum<16>(v);
    const float rs = 1.0f / sqrtf(v * inv_d + eps);
    // Stage the 4 rows {4 * lk + q} of this wavefront in LDS (reusing the W
    // tile), then store them with 16-byte accesses along each row.
    __syncthreads();
    float* stage = &Ws[0][0] + wave * 4 * (DOUT + 4);
#pragma unroll
    for (int b = 0; b < NB; ++b) stage[lk * (DOUT + 4) + b * 16 + lr] = acc[b][q];
    __syncthreads();
    if (row < rows) {
      const float* srow = stage + lk * (DOUT + 4);
      for (int c = lr * 4; c < DOUT; c += 64) {
        const float4 hv = *reinterpret_cast<const float4*>(srow + c);
        const float4 gg = *reinterpret_cast<const float4*>(gamma + c);
        const float4 bt = *reinterpret_cast<const float4*>(beta + c);
        float4 o;
        o.x = lt_act<ACT>(fmaf((hv.x - mu) * rs, gg.x, bt.x));
        o.y = lt_act<ACT>(fmaf((hv.y - mu) * rs, gg.y, bt.y));
        o.z = lt_act<ACT>(fmaf((hv.z - mu) * rs, gg.z, bt.z));
        o.w = lt_act<ACT>(fmaf((hv.w - mu) * rs, gg.w, bt.w));
        *reinterpret_cast<float4*>(h + row * DOUT + c) = hv;
        *reinterpret_cast<float4*>(out + row * DOUT + c) = o;
      }
      if (lr == 0) {
        mean[row] = mu;
        rstd[row] = rs;
      }
    }
  }
}

}  // namespace gr_gemm

extern "C" int gr_linear_ln_act(const float* x, int64_t ldx, int64_t rows, int64_t din,
                                const float* wt, int64_t dout, const float* bias,
                                const float* gamma, const float* beta, float eps, int32_t act,
                                float* h, float* out, float* mean, float* rstd, void* stream) {
  using namespace gr_gemm;
  gr::clear_error();
  GR_REQUIRE(rows >= 0 && din >= 1 && ldx >= din, "linear_ln_act: bad shape");
  GR_REQUIRE(dout >= 16 && dout <= 256 && dout % 16 == 0,
             "linear_ln_act: dout %lld must be a multiple of 16 in [16, 256]", (long long)dout);
  GR_REQUIRE(act == GR_ACT_RELU || act == GR_ACT_ELU, "linear_ln_act: unknown activation %d",
             act);
  if (rows == 0) return GR_OK;
  GR_REQUIRE(x && wt && gamma && beta && h && out && mean && rstd,
             "linear_ln_act: NULL pointer");
  auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  GR_REQUIRE(al16(gamma) && al16(beta) && al16(h) && al16(out),
             "linear_ln_act: gamma, beta, h and out must be 16-byte aligned");
  const int64_t blocks = (rows + LT_ROWS - 1) / LT_ROWS;
  GR_REQUIRE(blocks <= INT32_MAX, "linear_ln_act: too many rows");
  hipStream_t s = gr::as_stream(stream);
  const int nb = (int)(dout / 16);
#define GR_LT(NB)                                                                              \
  do {                                                                                         \
    if (act == GR_ACT_RELU)                                                                    \
      hipLaunchKernelGGL((linear_ln_act_kernel<NB, GR_ACT_RELU>), dim3((unsigned)blocks),      \
                         dim3(256), 0, s, x, ldx, rows, (int)din, wt, bias, gamma, beta, eps, h, \
                         out, mean, rstd);                                                     \
    else                                                                                       \
      hipLaunchKernelGGL((linear_ln_act_kernel<NB, GR_ACT_ELU>), dim3((unsigned)blocks),       \
                         dim3(256), 0, s, x, ldx, rows, (int)din, wt, bias, gamma, beta, eps, h, \
                         out, mean, rstd);                                                     \
  } while (0)
  switch (nb) {
    case 1: GR_LT(1); break;
    case 2: GR_LT(2); break;
    case 3: GR_LT(3); break;
    case 4: GR_LT(4); break;
    case 5: GR_LT(5); break;
    case 6: GR_LT(6); break;
    case 7: GR_LT(7); break;
    case 8: GR_LT(8); break;
    case 9: GR_LT(9); break;
    case 10: GR_LT(10); break;
    case 11: GR_LT(11); break;
    case 12: GR_LT(12); break;
    case 13: GR_LT(13); break;
    case 14: GR_LT(14); break;
    case 15: GR_LT(15); break;
    default: GR_LT(16); break;
  }
#undef GR_LT
  GR_HIP_CHECK(hipGetLastError());
  return GR_OK;
}
