// Weight-gradient GEMM for the dense per-layer transform: C[M,N] = A^T B with
// A [K, M] and B [K, N] row-major and K (the node count) in the millions,
// M, N <= a few hundred.  fp32 on the gfx950 matrix cores
// (v_mfma_f32_16x16x4_f32 or v_mfma_f32_32x32x2_f32), deterministic split-K.
//
// Workgroup tile 128 x 128 (4 wavefronts as 2 x 2 tiles of 64 x 64, each
// 4 x 4 MFMA blocks of 16 x 16 or 2 x 2 of 32 x 32); K is walked in steps of
// 16 rows staged in LDS,
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
#include <type_traits>

#include "gr_internal.h"
#include "wave.h"

namespace gr_gemm {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

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

template <int VEC, int W, int P = PAD>
__device__ __forceinline__ void store_tile(float (*lds)[W + P], const float (&r)[W / 16]) {
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
// Largest K the split-K weight-gradient product runs on 32 x 32 blocks with
// 128-column tiles (64-column tiles always take them).  Measured on one box:
// at K = 2.45M the 32 x 32 form is level at 256 x 256 and 10% faster at
// 256 x 100 (11% for 64-column tiles, 48 x 256); at K = 10M it is 2-3%
// slower (256 x 256 and 256 x 1024).
constexpr int64_t kTn32MaxK = int64_t(1) << 22;

// BN = 128, 64 or 32 output columns per workgroup (64 and 32 for narrow N;
// 32 takes B with 4-byte loads).  BLK = 16: each wavefront's 64 x BN/2 tile
// as 16 x 16 blocks of v_mfma_f32_16x16x4_f32; BLK = 32: as 32 x 32 blocks of
// v_mfma_f32_32x32x2_f32 (BN 64 or 128), with rows of the LDS tiles 32 floats
// apart mod 64 banks so the two k rows a 32x32x2 step reads fall on
// distinct banks.
template <int VA, int VB, int BN, int BLK = 16>
__global__ __launch_bounds__(256) void gemm_tn_splitk(const float* __restrict__ A, int64_t lda,
                                                      const float* __restrict__ B, int64_t ldb,
                                                      int M, int N, int64_t K, int64_t kchunk,
                                                      int nchunks, int tiles_m, int tiles,
                                                      float* __restrict__ part) {
  static_assert(BLK == 16 || (BLK == 32 && BN >= 64), "32 x 32 blocks need 64+ columns");
  constexpr int P = BLK == 16 ? PAD : 32;
  constexpr int MI = 64 / BLK;          // row blocks per wavefront
  constexpr int NJ = BN / 2 / BLK;      // column blocks per wavefront
  constexpr int KSTEP = 64 / BLK;       // k per MFMA: 4 or 2
  typedef typename std::conditional<BLK == 16, floatx4, floatx16>::type accx;
  __shared__ float As[TK][TM + P];
  __shared__ float Bs[TK][BN + P];
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
  const int lr = lane % BLK;  // row (A) / column (B) inside a block
  const int lk = lane / BLK;  // k inside an MFMA step

  accx acc[MI][NJ];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[i][j] = accx{};

  float ra[TM / 16], rb[BN / 16];
  load_tile<VA, TM>(A, lda, k_begin, k_end, m0, M, ra);
  load_tile<VB, BN>(B, ldb, k_begin, k_end, n0, N, rb);
  for (int64_t k = k_begin; k < k_end; k += TK) {
    __syncthreads();  // previous step's MFMA reads of the LDS tiles are done
    store_tile<VA, TM, P>(As, ra);
    store_tile<VB, BN, P>(Bs, rb);
    __syncthreads();
    if (k + TK < k_end) {
      load_tile<VA, TM>(A, lda, k + TK, k_end, m0, M, ra);
      load_tile<VB, BN>(B, ldb, k + TK, k_end, n0, N, rb);
    }
#pragma unroll
    for (int kk = 0; kk < TK; kk += KSTEP) {
      float a[MI], b[NJ];
#pragma unroll
      for (int i = 0; i < MI; ++i) a[i] = As[kk + lk][wm + i * BLK + lr];
#pragma unroll
      for (int j = 0; j < NJ; ++j) b[j] = Bs[kk + lk][wn + j * BLK + lr];
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          if constexpr (BLK == 16)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[j], acc[i][j], 0, 0, 0);
          else
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[j], acc[i][j], 0, 0, 0);
        }
    }
  }

  // BLK = 16: lane holds column lr, rows 4 lk + r (r < 4).  BLK = 32: lane
  // holds column lr, rows 8 (r / 4) + 4 lk + r % 4 (r < 16).
  constexpr int RPL = BLK == 16 ? 4 : 16;
  float* out = part + (int64_t)z * M * N;
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int n = n0 + wn + j * BLK + lr;
#pragma unroll
      for (int r = 0; r < RPL; ++r) {
        const int row = BLK == 16 ? lk * 4 + r : (r / 4) * 8 + lk * 4 + r % 4;
        const int m = m0 + wm + i * BLK + row;
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
  // At most 32 columns (a 19- or 20-wide layer's dW): 32-column tiles, so the
  // matrix cores do not work on 44 padded columns of 64; the product is then
  // bound by streaming the wide operand.
  const bool narrow32 = pn <= 32;
  const int bn = narrow32 ? 32 : narrow ? 64 : TN;
  const int tiles_m = (int)((pm + TM - 1) / TM);
  const int tiles = tiles_m * (int)((pn + bn - 1) / bn);
  const int64_t nwg = (used + kXcds - 1) / kXcds * kXcds * tiles;
  GR_REQUIRE(nwg <= INT32_MAX, "gemm_tn: too many workgroups");
  const dim3 grid((unsigned)nwg);
#define GR_GT(VA_, VB_, BN_, BLK_)                                                             \
  hipLaunchKernelGGL((gemm_tn_splitk<VA_, VB_, BN_, BLK_>), grid, dim3(256), 0, s, pa, plda, pb, \
                     pldb, (int)pm, (int)pn, k, kchunk, (int)used, tiles_m, tiles, workspace)
  // 32 x 32 blocks for 64-column tiles, and for 128-column tiles up to
  // kTn32MaxK rows of K; 16 x 16 for 32-column tiles.
  const bool b32 = k <= kTn32MaxK;
  if (narrow32) {
    if (va) GR_GT(4, 1, 32, 16); else GR_GT(1, 1, 32, 16);
  } else if (narrow) {
    if (va && vb) GR_GT(4, 4, 64, 32); else if (va) GR_GT(4, 1, 64, 32);
    else if (vb) GR_GT(1, 4, 64, 32); else GR_GT(1, 1, 64, 32);
  } else {
    if (b32) {
      if (va && vb) GR_GT(4, 4, 128, 32); else if (va) GR_GT(4, 1, 128, 32);
      else if (vb) GR_GT(1, 4, 128, 32); else GR_GT(1, 1, 128, 32);
    } else {
      if (va && vb) GR_GT(4, 4, 128, 16); else if (va) GR_GT(4, 1, 128, 16);
      else if (vb) GR_GT(1, 4, 128, 16); else GR_GT(1, 1, 128, 16);
    }
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
// Row-block product C[M, N] = A[M, K] B[N, K]^T (+ bias[N]), all row-major:
// the dense transform's forward y = x W^T + b (B = W) and its input gradient
// dx = dy W (B = W^T).  M is the node count (millions), N and K at most a few
// thousand.
//
// Both operands are K-contiguous, so a thread's 16-byte load takes 4
// consecutive k of one row, and the tiles are staged in LDS as [row][k] with
// a 4-float pad (row stride 20 or 36 floats: the 16 rows a quarter-wavefront
// reads with ds_read_b128 fall on distinct banks).  For v_mfma_f32_16x16x4_f32 lane
// (r, q) supplies row r of the 16-block at k = 4 step + q; here the lane
// reads k = 4q .. 4q + 3 of a 16-k slice in one ds_read_b128 and feeds them
// to four consecutive MFMAs, so MFMA s of the slice sums k = 4q + s over q.
// A and B use the same order, so every k is paired correctly; only the
// order of the fp32 sums differs from a k-ascending loop.
//
// Workgroup: 4 wavefronts as WMW x (4 / WMW), each owning MI x NJ blocks of
// BLK x BLK; K in steps of KS with the next step's loads in registers while
// the current step's MFMAs run.  The column tiles of one row tile are
// consecutive workgroups of one XCD, so A is read from HBM once and from that
// XCD's L2 after.  Each output element is one workgroup's sum over K in a
// fixed order: the result is deterministic.
namespace gr_gemm {

// A [ROWS, KS] slice of a row-major matrix (rows r0.., columns k0..) into
// registers; elements outside [rows) x [K) read as 0.  V = 4 needs K % 4 == 0,
// ld % 4 == 0 and a 16-byte aligned base.
template <int V, int ROWS, int KS>
struct NtTile {
  static constexpr int LDK = KS + 4;
  static constexpr int SPR = KS / V;  // slots per row
  static constexpr int SLOTS = ROWS * SPR;
  static constexpr int PER = (SLOTS + 255) / 256;  // a 16 x 32 tile has 128 float4 slots
  float r[PER][V];

  __device__ __forceinline__ void load(const float* __restrict__ src, int64_t ld, int64_t r0,
                                       int64_t rows, int k0, int K) {
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int slot = threadIdx.x + p * 256;
      const int64_t row = r0 + slot / SPR;
      const int k = k0 + (slot % SPR) * V;
      const bool in = (SLOTS % 256 == 0 || slot < SLOTS) && row < rows && k < K;
      if constexpr (V == 4) {
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (in) v = *reinterpret_cast<const float4*>(src + row * ld + k);
        r[p][0] = v.x;
        r[p][1] = v.y;
        r[p][2] = v.z;
        r[p][3] = v.w;
      } else {
        r[p][0] = in ? src[row * ld + k] : 0.f;
      }
    }
  }

  __device__ __forceinline__ void store(float (*lds)[LDK]) const {
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int slot = threadIdx.x + p * 256;
      if (SLOTS % 256 != 0 && slot >= SLOTS) continue;
      float* d = &lds[slot / SPR][(slot % SPR) * V];
      if constexpr (V == 4) {
        *reinterpret_cast<float4*>(d) = make_float4(r[p][0], r[p][1], r[p][2], r[p][3]);
      } else {
        *d = r[p][0];
      }
    }
  }
};

// BLK = 16: v_mfma_f32_16x16x4_f32 blocks; lane (r, q) = (lane % 16, lane / 16)
// reads k = 4q .. 4q + 3 of a 16-k slice.  BLK = 32: v_mfma_f32_32x32x2_f32
// blocks; lane (r, q) = (lane % 32, lane / 32) reads k = 4q .. 4q + 3 of an
// 8-k slice, and MFMA s of the slice takes the k pair (s, 4 + s).
// DB: two LDS buffers, one barrier per K step (step s computes from buffer
// s % 2 while step s + 1's tile, already in registers, goes to the other).
// OCC: the waves per SIMD the register allocation must allow.
template <int VA, int VB, int MI, int NJ, int WMW, int KS, int BLK, int OCC, bool DB>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(OCC, 8))) void gemm_nt_kernel(
    const float* __restrict__ A, int64_t lda, const float* __restrict__ B, int64_t ldb,
    const float* __restrict__ bias, float* __restrict__ C, int64_t ldc, int64_t M, int N, int K,
    int64_t tiles_m, int tiles_n) {
  constexpr int WNW = 4 / WMW;
  constexpr int TM = BLK * MI * WMW;
  constexpr int TN = BLK * NJ * WNW;
  constexpr int LDK = KS + 4;
  constexpr int SLICE = BLK == 16 ? 16 : 8;  // k per fragment read
  constexpr int NBUF = DB ? 2 : 1;
  typedef typename std::conditional<BLK == 16, floatx4, floatx16>::type accx;
  __shared__ __align__(16) float As[NBUF][TM][LDK];
  __shared__ __align__(16) float Bs[NBUF][TN][LDK];

  const int64_t w = blockIdx.x;
  const int64_t q = w / kXcds;
  const int64_t tm = (q / tiles_n) * kXcds + w % kXcds;
  if (tm >= tiles_m) return;  // whole workgroup: no barrier is pending
  const int tn = (int)(q % tiles_n);
  const int64_t m0 = tm * TM;
  const int n0 = tn * TN;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = (wave % WMW) * (BLK * MI);
  const int wn = (wave / WMW) * (BLK * NJ);
  const int lr = lane % BLK;
  const int lq = lane / BLK;

  accx acc[MI][NJ];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[i][j] = accx{};

  auto compute = [&](int buf) {
#pragma unroll
    for (int h = 0; h < KS / SLICE; ++h) {
      floatx4 a[MI], b[NJ];
#pragma unroll
      for (int i = 0; i < MI; ++i)
        a[i] = *reinterpret_cast<const floatx4*>(&As[buf][wm + i * BLK + lr][h * SLICE + lq * 4]);
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        b[j] = *reinterpret_cast<const floatx4*>(&Bs[buf][wn + j * BLK + lr][h * SLICE + lq * 4]);
#pragma unroll
      for (int st = 0; st < 4; ++st)
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
          for (int j = 0; j < NJ; ++j) {
            if constexpr (BLK == 16)
              acc[i][j] =
                  __builtin_amdgcn_mfma_f32_16x16x4f32(a[i][st], b[j][st], acc[i][j], 0, 0, 0);
            else
              acc[i][j] =
                  __builtin_amdgcn_mfma_f32_32x32x2f32(a[i][st], b[j][st], acc[i][j], 0, 0, 0);
          }
    }
  };

  float bcol[NJ];  // this lane's bias column of each block
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int n = n0 + wn + j * BLK + lr;
    bcol[j] = bias != nullptr && n < N ? bias[n] : 0.f;
  }

  NtTile<VA, TM, KS> ta;
  NtTile<VB, TN, KS> tb;
  ta.load(A, lda, m0, M, 0, K);
  tb.load(B, ldb, n0, N, 0, K);
  if constexpr (DB) {
    // Buffer (s + 1) % 2 was last read in step s - 1, before the barrier
    // that ended it.
    ta.store(As[0]);
    tb.store(Bs[0]);
    if (KS < K) {
      ta.load(A, lda, m0, M, KS, K);
      tb.load(B, ldb, n0, N, KS, K);
    }
    __syncthreads();
    int buf = 0;
    for (int k0 = 0; k0 < K; k0 += KS) {
      compute(buf);
      if (k0 + KS < K) {
        ta.store(As[buf ^ 1]);
        tb.store(Bs[buf ^ 1]);
        if (k0 + 2 * KS < K) {
          ta.load(A, lda, m0, M, k0 + 2 * KS, K);
          tb.load(B, ldb, n0, N, k0 + 2 * KS, K);
        }
      }
      __syncthreads();
      buf ^= 1;
    }
  } else {
    for (int k0 = 0; k0 < K; k0 += KS) {
      __syncthreads();  // the previous step's reads of the LDS tiles are done
      ta.store(As[0]);
      tb.store(Bs[0]);
      __syncthreads();
      if (k0 + KS < K) {
        ta.load(A, lda, m0, M, k0 + KS, K);
        tb.load(B, ldb, n0, N, k0 + KS, K);
      }
      compute(0);
    }
  }

  // BLK = 16: lane holds column lr, rows 4 lq + r (r < 4).  BLK = 32: lane
  // holds column lr, rows 8 (r / 4) + 4 lq + r % 4 (r < 16).
  // The bias was loaded before the K loop and is added to every accumulator
  // ahead of the stores: a load consumed between guarded stores would make
  // each store wait for all earlier ones (the vector-memory counter retires
  // in issue order).
  constexpr int RPL = BLK == 16 ? 4 : 16;
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int r = 0; r < RPL; ++r) acc[i][j][r] += bcol[j];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int n = n0 + wn + j * BLK + lr;
    if (n >= N) continue;
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int r = 0; r < RPL; ++r) {
        const int row = BLK == 16 ? lq * 4 + r : (r / 4) * 8 + lq * 4 + r % 4;
        const int64_t m = m0 + wm + i * BLK + row;
        if (m < M) C[m * ldc + n] = acc[i][j][r];
      }
  }
}

template <int VA, int VB, int MI, int NJ, int WMW, int KS, int BLK, int OCC = 1, bool DB = false>
static hipError_t launch_nt(const float* a, int64_t lda, const float* b, int64_t ldb,
                            const float* bias, float* c, int64_t ldc, int64_t m, int n, int k,
                            hipStream_t s) {
  constexpr int TM = BLK * MI * WMW;
  constexpr int TN = BLK * NJ * (4 / WMW);
  const int64_t tiles_m = (m + TM - 1) / TM;
  const int tiles_n = (n + TN - 1) / TN;
  const int64_t nwg = (tiles_m + kXcds - 1) / kXcds * kXcds * tiles_n;
  if (nwg > INT32_MAX) return hipErrorInvalidValue;
  hipLaunchKernelGGL((gemm_nt_kernel<VA, VB, MI, NJ, WMW, KS, BLK, OCC, DB>), dim3((unsigned)nwg),
                     dim3(256), 0, s, a, lda, b, ldb, bias, c, ldc, m, n, k, tiles_m, tiles_n);
  return hipGetLastError();
}

// Tile shape by the product's shape, as measured on the dense transform's
// products (MI355X, fp32):
//   n > 64, k > 256: 128 x 128 tiles of 32 x 32 blocks, 32-k steps (126-128
//     TFLOP/s for 625k and 1M x 256 x 1024, against 124 with 16 x 16 blocks);
//   n > 64, k <= 256: 128 x 128 tiles of 32 x 32 blocks, 16-k double-buffered
//     steps at 4 waves per SIMD (114-117 TFLOP/s for 2.45M x 256 x 256, and
//     30% faster than the first form for k = 48 or 20);
//   33..48 columns: 256 x 48 tiles (no padded columns); 49..64: 256 x 64;
//   17..32 and <= 16 columns: 256 x 32 / 256 x 16.
// hipBLASLt's own kernels run these products at 116-128 TFLOP/s with 82%
// MFMA-busy cycles against 70-79% here.  A persistent grid, fragment reads
// one slice ahead, explicit instruction interleaving and 64 x 128 wavefront
// tiles were each measured and gained nothing; double-buffered LDS pays only
// in the 16-k, 4-waves-per-SIMD form above.
template <int VA, int VB>
static hipError_t dispatch_nt(const float* a, int64_t lda, const float* b, int64_t ldb,
                              const float* bias, float* c, int64_t ldc, int64_t m, int n, int k,
                              hipStream_t s) {
#define GR_NT(MI, NJ, WMW, KS, BLK, ...) \
  return launch_nt<VA, VB, MI, NJ, WMW, KS, BLK, ##__VA_ARGS__>(a, lda, b, ldb, bias, c, ldc, m, n, k, s)
  if (n > 64) {
    if (k <= 256) GR_NT(2, 2, 2, 16, 32, 4, true);
    GR_NT(2, 2, 2, 32, 32);
  }
  if (n > 48) GR_NT(4, 4, 4, 16, 16, 1, true);
  if (n > 32) GR_NT(4, 3, 4, 32, 16);
  if (n > 16) GR_NT(4, 2, 4, 32, 16);
  GR_NT(4, 1, 4, 32, 16);
#undef GR_NT
}

// Products with a short reduction (k <= 64: a layer's input gradient
// dZ W through a narrow layer) whose operands are not 16-byte aligned.  A
// wavefront owns 128 columns (2 adjacent ones per lane, their rows of B held
// in registers) and a run of SK_ROWS rows of C; lane kk holds A[r][kk],
// loaded SK_PD rows ahead, and row r's k values reach every lane by
// v_readlane, so no LDS is used.  Each row is one 8-byte store per lane: 512 contiguous
// bytes per wavefront.  The k FMAs per element run on the vector units
// (non-packed fp32, 4 cycles per wavefront instruction), which bound the
// kernel: 59 us for 156k x 256 x 19 (2.7 TB/s of C), 1.6 ms for
// 2.45M x 256 x 47, against 90 us and 2.1 ms for the matrix-core kernel with
// 4-byte loads.  Sums run in k order from 0, then the bias is added.
constexpr int SK_ROWS = 64;  // rows of C per wavefront
constexpr int SK_PD = 4;     // rows of A loaded ahead

template <int KMAX, bool V2>
__global__ __launch_bounds__(256) void gemm_nt_short_k(
    const float* __restrict__ A, int64_t lda, const float* __restrict__ B, int64_t ldb,
    const float* __restrict__ bias, float* __restrict__ C, int64_t ldc, int64_t M, int N,
    int K) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int j = blockIdx.y * 128 + 2 * lane;
  const int64_t r_begin = ((int64_t)blockIdx.x * 4 + wave) * SK_ROWS;
  if (r_begin >= M) return;
  const int64_t r_end = min(M, r_begin + SK_ROWS);
  // Columns past N read column N - 1 and are never stored.
  const int64_t j0 = min(j, N - 1), j1 = min(j + 1, N - 1);
  float b0[KMAX], b1[KMAX];
#pragma unroll
  for (int kk = 0; kk < KMAX; ++kk) {
    b0[kk] = kk < K ? B[j0 * ldb + kk] : 0.f;
    b1[kk] = kk < K ? B[j1 * ldb + kk] : 0.f;
  }
  const float bias0 = bias != nullptr ? bias[j0] : 0.f;
  const float bias1 = bias != nullptr ? bias[j1] : 0.f;
  // Lanes k >= K hold 0 (and b is 0 there): their terms add +0.
  const bool kin = lane < K;
  const int kl = min(lane, K - 1);
  // Rows r .. r + SK_PD - 1 of A in flight (rows past the run re-read its
  // last row).
  float an[SK_PD];
#pragma unroll
  for (int q = 0; q < SK_PD; ++q) an[q] = A[min(r_begin + q, r_end - 1) * lda + kl];
  for (int64_t r = r_begin; r < r_end; ++r) {
    const float ac = kin ? an[0] : 0.f;
#pragma unroll
    for (int q = 0; q + 1 < SK_PD; ++q) an[q] = an[q + 1];
    an[SK_PD - 1] = A[min(r + SK_PD, r_end - 1) * lda + kl];
    float c0 = 0.f, c1 = 0.f;
#pragma unroll
    for (int kk = 0; kk < KMAX; ++kk) {
      const float a = __builtin_bit_cast(
          float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ac), kk));
      c0 = fmaf(a, b0[kk], c0);
      c1 = fmaf(a, b1[kk], c1);
    }
    float* cr = C + r * ldc + j;
    if constexpr (V2) {
      if (j < N) *reinterpret_cast<float2*>(cr) = make_float2(c0 + bias0, c1 + bias1);
    } else {
      if (j < N) cr[0] = c0 + bias0;
      if (j + 1 < N) cr[1] = c1 + bias1;
    }
  }
}

template <int KMAX>
static hipError_t launch_short_k(const float* a, int64_t lda, const float* b, int64_t ldb,
                                 const float* bias, float* c, int64_t ldc, int64_t m, int n,
                                 int k, bool v2, hipStream_t s) {
  const int64_t gx = (m + 4 * SK_ROWS - 1) / (4 * SK_ROWS);
  const int gy = (n + 127) / 128;
  if (gx > INT32_MAX) return hipErrorInvalidValue;
  if (v2)
    hipLaunchKernelGGL((gemm_nt_short_k<KMAX, true>), dim3((unsigned)gx, (unsigned)gy), dim3(256),
                       0, s, a, lda, b, ldb, bias, c, ldc, m, n, k);
  else
    hipLaunchKernelGGL((gemm_nt_short_k<KMAX, false>), dim3((unsigned)gx, (unsigned)gy),
                       dim3(256), 0, s, a, lda, b, ldb, bias, c, ldc, m, n, k);
  return hipGetLastError();
}

// Short-K form (K a multiple of 32 up to 256, 16-byte rows of A and B, N a
// multiple of 4, millions of rows): each workgroup keeps a block of NT = 16 NJ
// columns of B in LDS as [column][k] for the whole launch (133 KB at
// NT = 128) and its 16 wavefronts walk blocks of 16 MI rows of A, with no
// barrier after the fill.  A lane's two 16-byte loads of A take k = 8 lk ..
// 8 lk + 7 of a 32-k chunk (one 128-byte line of each row a chunk), straight
// from HBM one chunk ahead; its two ds_read_b128 of B the same eight k, and
// MFMA s of the chunk sums k = 8 lk + s over lk.  The workgroups of the column
// blocks of one row stream are on one XCD, so A is read from HBM once.  Each
// lane quad transposes its 4 x 4 blocks, so C leaves the accumulators as
// 16-byte row stores.  Measured against gemm_nt_kernel on one box: 2.45M x 48
// x 256 0.69 against 0.80 ms; at 20 columns the two are equal, so narrower
// products keep the tiled kernel, and wider ones take the 32 x 32 form below.
constexpr int RS_KST = 256 + 4;  // LDS row stride: 16 lanes' reads fall on distinct banks
constexpr int RS_WAVES = 16;
constexpr int64_t kResidentMinRows = 1 << 16;

struct A8 {
  float4 lo, hi;
};

// NCH = K / 32 when known at compile time (even), else 0: as in
// gemm_nt_resident32 below, the chunks of a block are then unrolled with the
// block's stores after its last chunk, one chunk of A ahead.
template <int MI, int NJ, int NCH>
__global__ __launch_bounds__(1024) void gemm_nt_resident(
    const float* __restrict__ A, int64_t lda, const float* __restrict__ B, int64_t ldb,
    const float* __restrict__ bias, float* __restrict__ C, int64_t ldc, int64_t M, int N, int K,
    int tiles_n) {
  static_assert(NCH % 2 == 0 && NCH <= 8, "NCH: an even chunk count up to 8, or 0");
  constexpr int NT = 16 * NJ, RB = 16 * MI;
  __shared__ __align__(16) float Bs[NT * RS_KST];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 15, lk = lane >> 4;
  const int g = blockIdx.x, slot = g / kXcds, tile = slot % tiles_n;
  const int64_t stream = (int64_t)(slot / tiles_n) * kXcds + g % kXcds;
  const int64_t nstreams = (int64_t)gridDim.x / tiles_n;
  const int n0 = tile * NT;
  // The bias of this lane's column of each block, loaded once: it is added to
  // the accumulators before the stores, so no store waits on a load.  Loaded
  // before B's fill, whose loads complete after it, so that no load is in
  // flight when the chunk loop starts.
  float bcol[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int n = n0 + j * 16 + lr;
    bcol[j] = bias != nullptr && n < N ? bias[n] : 0.f;
  }
  const int kq = K / 4;
  for (int i = tid; i < NT * kq; i += 1024) {
    const int c = i / kq, k = (i % kq) * 4;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (n0 + c < N) v = *reinterpret_cast<const float4*>(B + (int64_t)(n0 + c) * ldb + k);
    *reinterpret_cast<float4*>(&Bs[c * RS_KST + k]) = v;
  }
  __syncthreads();
  const int64_t nblk = (M + RB - 1) / RB;
  const int64_t step = nstreams * RS_WAVES;
  const int64_t blk0 = stream * RS_WAVES + wave;
  if (blk0 >= nblk) return;
  const int nch = NCH > 0 ? NCH : K / 32;
  const int qc = lane & 3, qa = (lane >> 2) & 3;
  const float* bl = Bs + lr * RS_KST + 8 * lk;

  // Chunk c of block b into dst.  Loads are unconditional: past the
  // wavefront's last block a load re-reads block blk0 (and is never used).
  // The block's base is uniform; lanes add 32-bit offsets (lda < 2^20,
  // checked by the dispatch).
  auto load_at = [&](A8 (&dst)[MI], int64_t b, int c) {
    const int64_t bb = b < nblk ? b : blk0;
    const float* ab = A + bb * RB * lda;
    const int rows = (int)(M - bb * RB < RB ? M - bb * RB : RB);  // uniform
#pragma unroll
    for (int i = 0; i < MI; ++i) {
      const int r = i * 16 + lr;  // rows past M read the block's first
      const int off = (r < rows ? r : 0) * (int)lda + c * 32 + 8 * lk;
      dst[i].lo = *reinterpret_cast<const float4*>(ab + off);
      dst[i].hi = *reinterpret_cast<const float4*>(ab + off + 4);
    }
  };
  floatx4 acc[MI][NJ];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  auto mma = [&](const A8 (&cur)[MI], int c) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const float4 b0 = *reinterpret_cast<const float4*>(bl + j * 16 * RS_KST + c * 32);
      const float4 b1 = *reinterpret_cast<const float4*>(bl + j * 16 * RS_KST + c * 32 + 4);
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(cur[i].lo.x, b0.x, acc[i][j], 0, 0, 0);
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(cur[i].lo.y, b0.y, acc[i][j], 0, 0, 0);
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(cur[i].lo.z, b0.z, acc[i][j], 0, 0, 0);
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(cur[i].lo.w, b0.w, acc[i][j], 0, 0, 0);
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(cur[i].hi.x, b1.x, acc[i][j], 0, 0, 0);
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(cur[i].hi.y, b1.y, acc[i][j], 0, 0, 0);
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(cur[i].hi.z, b1.z, acc[i][j], 0, 0, 0);
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(cur[i].hi.w, b1.w, acc[i][j], 0, 0, 0);
      }
    }
  };
  // Block b is complete: rows 16 i + 4 lk + q, columns 16 j + lr; after the
  // quad transpose row 16 i + 4 lk + qc, columns 16 j + 4 qa .. + 3.
  auto store_block = [&](int64_t b) {
    float* cb = C + b * RB * ldc;  // uniform; lanes add 32-bit offsets (ldc < 2^20)
    const int rows = (int)(M - b * RB < RB ? M - b * RB : RB);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int col = n0 + j * 16 + 4 * qa;
      const bool cin = col < N;  // N % 4 == 0: the four columns are in or out together
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        float v0 = acc[i][j][0] + bcol[j], v1 = acc[i][j][1] + bcol[j],
              v2 = acc[i][j][2] + bcol[j], v3 = acc[i][j][3] + bcol[j];
        gr_wave::quad_transpose(v0, v1, v2, v3, qc);
        const int r = i * 16 + 4 * lk + qc;
        if (cin && r < rows)
          *reinterpret_cast<float4*>(cb + r * (int)ldc + col) = make_float4(v0, v1, v2, v3);
        acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
      }
    }
  };

  A8 x0[MI], x1[MI];
  load_at(x0, blk0, 0);
  if constexpr (NCH > 0) {
    for (int64_t b = blk0; b < nblk; b += step) {
#pragma unroll
      for (int c = 0; c < NCH; c += 2) {
        load_at(x1, b, c + 1);
        __builtin_amdgcn_sched_barrier(0);
        mma(x0, c);
        load_at(x0, c + 2 < NCH ? b : b + step, c + 2 < NCH ? c + 2 : 0);
        __builtin_amdgcn_sched_barrier(0);
        mma(x1, c + 1);
      }
      store_block(b);
    }
  } else {
    // Runtime chunk count: cursors (block, chunk) of the next chunk to load
    // and to compute, advanced by counting.
    const int64_t T = (nblk - blk0 + step - 1) / step * nch;
    int64_t lb = blk0, cb = blk0;
    int lc = 1, cc = 0;
    if (lc == nch) {
      lc = 0;
      lb += step;
    }
    auto step_chunk = [&](A8 (&nxt)[MI], const A8 (&cur)[MI]) {
      load_at(nxt, lb, lc);
      if (++lc == nch) {
        lc = 0;
        lb += step;
      }
      __builtin_amdgcn_sched_barrier(0);
      mma(cur, cc);
      if (++cc == nch) {
        store_block(cb);
        cc = 0;
        cb += step;
      }
    };
    for (int64_t t = 0; t < T; t += 2) {
      step_chunk(x1, x0);
      if (t + 1 >= T) break;
      step_chunk(x0, x1);
    }
  }
}

// The same resident-B product on v_mfma_f32_32x32x2_f32 blocks, for more than
// 64 columns: a wavefront owns 32 rows and NJ 32-column blocks (lane (r, q) =
// (lane % 32, lane / 32) loads k = 16 q .. 16 q + 15 of row r's 32-k chunk as
// four 16-byte pieces and reads the same k of its B column, MFMA s of the
// chunk summing k = 16 q + s over q), so a lane's operand reads per flop are
// half the 16 x 16 form's.  One chunk of A ahead.
//
// NCH = K / 32 when it is known at compile time (even), else 0.  With NCH the
// chunks of a block are unrolled and the block's stores follow its last chunk,
// so the only wait on memory inside a block is for the chunk about to be
// used; with a runtime chunk count the stores sit inside the chunk loop, and
// the compiler's waits there also cover loads issued for later chunks.
// Measured at 2.45M x 256 x 256 (K = 256; SQ_VALU_MFMA_BUSY_CYCLES over
// GRBM_GUI_ACTIVE cycles): the matrix pipe busy 81.5% of the kernel's cycles
// with the runtime loop, 87.7% with the unrolled one, on every operand tried
// (zeros, ReLU-sparse, randn); 2.57-2.75 -> 2.42-2.56 ms, same bits.  The
// clock under this load varies from box to box and with the data (1.8-2.3
// GHz against 2.4 for a copy), which sets the rest of the rate.
template <int NJ, int NCH>
__global__ __launch_bounds__(1024) void gemm_nt_resident32(
    const float* __restrict__ A, int64_t lda, const float* __restrict__ B, int64_t ldb,
    const float* __restrict__ bias, float* __restrict__ C, int64_t ldc, int64_t M, int N, int K,
    int tiles_n) {
  static_assert(NCH % 2 == 0 && NCH <= 8, "NCH: an even chunk count up to 8, or 0");
  constexpr int NT = 32 * NJ, RB = 32;
  __shared__ __align__(16) float Bs[NT * RS_KST];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, q = lane >> 5;
  const int g = blockIdx.x, slot = g / kXcds, tile = slot % tiles_n;
  const int64_t stream = (int64_t)(slot / tiles_n) * kXcds + g % kXcds;
  const int64_t nstreams = (int64_t)gridDim.x / tiles_n;
  const int n0 = tile * NT;
  // The bias of this lane's column of each block, loaded once before B's fill
  // (as in gemm_nt_resident).
  float bcol[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int n = n0 + j * 32 + l32;
    bcol[j] = bias != nullptr && n < N ? bias[n] : 0.f;
  }
  const int kq = K / 4;
  for (int i = tid; i < NT * kq; i += 1024) {
    const int c = i / kq, k = (i % kq) * 4;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (n0 + c < N) v = *reinterpret_cast<const float4*>(B + (int64_t)(n0 + c) * ldb + k);
    *reinterpret_cast<float4*>(&Bs[c * RS_KST + k]) = v;
  }
  __syncthreads();
  const int64_t nblk = (M + RB - 1) / RB;
  const int64_t step = nstreams * RS_WAVES;
  const int64_t blk0 = stream * RS_WAVES + wave;
  if (blk0 >= nblk) return;
  const int nch = NCH > 0 ? NCH : K / 32;
  const float* bl = Bs + l32 * RS_KST + 16 * q;
  const int qc = lane & 3, qa = (lane >> 2) & 7;

  struct A16 {
    float4 v[4];
  };
  // Chunk c of block b into dst.  Loads are unconditional: past the
  // wavefront's last block a load re-reads block blk0 (and is never used).
  // The block's base is uniform (scalar registers) and a lane adds a 32-bit
  // offset (lda < 2^20, checked by the dispatch).
  auto load_at = [&](A16& dst, int64_t b, int c) {
    const int64_t bb = b < nblk ? b : blk0;
    const float* ab = A + bb * RB * lda;
    const int rows = (int)(M - bb * RB < RB ? M - bb * RB : RB);  // uniform
    const int off = (l32 < rows ? l32 : 0) * (int)lda + 16 * q + c * 32;
#pragma unroll
    for (int u = 0; u < 4; ++u) dst.v[u] = *reinterpret_cast<const float4*>(ab + off + 4 * u);
  };
  floatx16 acc[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) acc[j] = floatx16{};
  auto mma = [&](const A16& cur, int c) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      float4 bv[4];
#pragma unroll
      for (int u = 0; u < 4; ++u)
        bv[u] = *reinterpret_cast<const float4*>(bl + j * 32 * RS_KST + c * 32 + 4 * u);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(cur.v[u].x, bv[u].x, acc[j], 0, 0, 0);
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(cur.v[u].y, bv[u].y, acc[j], 0, 0, 0);
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(cur.v[u].z, bv[u].z, acc[j], 0, 0, 0);
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(cur.v[u].w, bv[u].w, acc[j], 0, 0, 0);
      }
    }
  };
  // Block b is complete.  Lane holds column 32 j + l32, rows 8 (e / 4) + 4 q
  // + e % 4 (e < 16); after each quad transpose, row 8 gq + 4 q + qc, columns
  // 32 j + 4 qa .. + 3.
  auto store_block = [&](int64_t b) {
    float* cb = C + b * RB * ldc;  // uniform; lanes add 32-bit offsets (ldc < 2^20)
    const int rows = (int)(M - b * RB < RB ? M - b * RB : RB);
    const int rl = 4 * q + qc;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int col = n0 + j * 32 + 4 * qa;
      const bool cin = col < N;  // N % 4 == 0
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        float v0 = acc[j][4 * gq + 0] + bcol[j], v1 = acc[j][4 * gq + 1] + bcol[j],
              v2 = acc[j][4 * gq + 2] + bcol[j], v3 = acc[j][4 * gq + 3] + bcol[j];
        gr_wave::quad_transpose(v0, v1, v2, v3, qc);
        if (cin && 8 * gq + rl < rows)
          *reinterpret_cast<float4*>(cb + (8 * gq + rl) * (int)ldc + col) =
              make_float4(v0, v1, v2, v3);
      }
      acc[j] = floatx16{};
    }
  };

  A16 x0, x1;
  load_at(x0, blk0, 0);
  if constexpr (NCH > 0) {
    // Two chunk buffers in turn; the scheduling barriers keep each load ahead
    // of the products before it (the compiler otherwise sinks the loads to
    // the end of the chunk).
    for (int64_t b = blk0; b < nblk; b += step) {
#pragma unroll
      for (int c = 0; c < NCH; c += 2) {
        load_at(x1, b, c + 1);
        __builtin_amdgcn_sched_barrier(0);
        mma(x0, c);
        load_at(x0, c + 2 < NCH ? b : b + step, c + 2 < NCH ? c + 2 : 0);
        __builtin_amdgcn_sched_barrier(0);
        mma(x1, c + 1);
      }
      store_block(b);
    }
  } else {
    // Runtime chunk count: cursors (block, chunk) of the next chunk to load
    // and to compute, advanced by counting.
    const int64_t T = (nblk - blk0 + step - 1) / step * nch;
    int64_t lb = blk0, cb = blk0;
    int lc = 1, cc = 0;
    if (lc == nch) {
      lc = 0;
      lb += step;
    }
    auto step_chunk = [&](A16& nxt, const A16& cur) {
      load_at(nxt, lb, lc);
      if (++lc == nch) {
        lc = 0;
        lb += step;
      }
      __builtin_amdgcn_sched_barrier(0);
      mma(cur, cc);
      if (++cc == nch) {
        store_block(cb);
        cc = 0;
        cb += step;
      }
    };
    for (int64_t t = 0; t < T; t += 2) {
      step_chunk(x1, x0);
      if (t + 1 >= T) break;
      step_chunk(x0, x1);
    }
  }
}

template <int MI, int NJ>
static hipError_t launch_resident(const float* a, int64_t lda, const float* b, int64_t ldb,
                                  const float* bias, float* c, int64_t ldc, int64_t m, int n,
                                  int k, int tiles_n, int grid, hipStream_t s) {
  if (k == 256)
    hipLaunchKernelGGL((gemm_nt_resident<MI, NJ, 8>), dim3((unsigned)grid), dim3(1024), 0, s, a,
                       lda, b, ldb, bias, c, ldc, m, n, k, tiles_n);
  else
    hipLaunchKernelGGL((gemm_nt_resident<MI, NJ, 0>), dim3((unsigned)grid), dim3(1024), 0, s, a,
                       lda, b, ldb, bias, c, ldc, m, n, k, tiles_n);
  return hipGetLastError();
}

// The resident forms for 32 < n <= 256: the 32 x 32 form past 64 columns
// (two column blocks past 128), the 16 x 16 form below, where MI * NJ <= 8
// keeps its accumulators and two chunks of A within 128 registers (16
// wavefronts a CU).  Workgroups: a whole number of XCD rounds per column
// block, four per CU for the 32 x 32 form and two for the 16 x 16 one (the
// counts measured best; the LDS holds one at a time, the rest queue).
static hipError_t dispatch_resident(const float* a, int64_t lda, const float* b, int64_t ldb,
                                    const float* bias, float* c, int64_t ldc, int64_t m, int n,
                                    int k, hipStream_t s) {
  int dev = 0, cus = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return e;
  const int tiles_n = (n + 127) / 128;
  if (n > 64) {
    // 32 x 32 blocks, 128-column blocks of B, four workgroups per CU.
    const int per = kXcds * tiles_n;
    const int grid = std::max(per, 4 * cus / per * per);
    if (k == 256)
      hipLaunchKernelGGL((gemm_nt_resident32<4, 8>), dim3((unsigned)grid), dim3(1024), 0, s, a,
                         lda, b, ldb, bias, c, ldc, m, n, k, tiles_n);
    else
      hipLaunchKernelGGL((gemm_nt_resident32<4, 0>), dim3((unsigned)grid), dim3(1024), 0, s, a,
                         lda, b, ldb, bias, c, ldc, m, n, k, tiles_n);
    return hipGetLastError();
  }
  // 33..64 columns: 16 x 16 blocks, one column block, two workgroups per CU.
  const int grid = std::max(kXcds, 2 * cus / kXcds * kXcds);
  if (n <= 48) return launch_resident<2, 3>(a, lda, b, ldb, bias, c, ldc, m, n, k, 1, grid, s);
  return launch_resident<1, 4>(a, lda, b, ldb, bias, c, ldc, m, n, k, 1, grid, s);
}

}  // namespace gr_gemm

extern "C" int gr_gemm_nt(const float* a, int64_t lda, const float* b, int64_t ldb, int64_t m,
                          int64_t n, int64_t k, const float* bias, float* c, int64_t ldc,
                          void* stream) {
  using namespace gr_gemm;
  gr::clear_error();
  GR_REQUIRE(m >= 0 && n >= 1 && k >= 1 && n <= (1 << 20) && k <= (1 << 24),
             "gemm_nt: bad shape %lld x %lld x %lld", (long long)m, (long long)n, (long long)k);
  GR_REQUIRE(lda >= k && ldb >= k && ldc >= n, "gemm_nt: leading dimension too small");
  if (m == 0) return GR_OK;
  GR_REQUIRE(a != nullptr && b != nullptr && c != nullptr, "gemm_nt: NULL pointer");
  const bool va = k % 4 == 0 && lda % 4 == 0 && reinterpret_cast<uintptr_t>(a) % 16 == 0;
  const bool vb = k % 4 == 0 && ldb % 4 == 0 && reinterpret_cast<uintptr_t>(b) % 16 == 0;
  hipStream_t s = gr::as_stream(stream);
  hipError_t err;
  if (va && vb && k % 32 == 0 && k <= 256 && n > 32 && n <= 256 && n % 4 == 0 && ldc % 4 == 0 &&
      reinterpret_cast<uintptr_t>(c) % 16 == 0 &&
      (bias == nullptr || reinterpret_cast<uintptr_t>(bias) % 16 == 0) &&
      m >= kResidentMinRows && lda < (1 << 20) && ldc < (1 << 20)) {
    err = dispatch_resident(a, lda, b, ldb, bias, c, ldc, m, (int)n, (int)k, s);
  } else if (k <= 64 && n >= 64 && !(va && vb)) {
    // Short reduction with rows of A or B that 16-byte loads cannot take
    // (k or ld not a multiple of 4, as for a 19- or 47-wide gradient): on the
    // vector units as a stream of C's rows (gemm_nt_short_k), 1.3-1.6x faster
    // than the matrix-core kernel with 4-byte loads.  With aligned rows the
    // matrix cores stay faster (1.0 against 1.9 ms for 2.45M x 256 x 48).
    const bool v2 = n % 2 == 0 && ldc % 2 == 0 && reinterpret_cast<uintptr_t>(c) % 8 == 0;
#define GR_SK(KM) launch_short_k<KM>(a, lda, b, ldb, bias, c, ldc, m, (int)n, (int)k, v2, s)
    // The k loop runs to KMAX: the instance just above k.
    if (k <= 8) err = GR_SK(8);
    else if (k <= 16) err = GR_SK(16);
    else if (k <= 20) err = GR_SK(20);
    else if (k <= 24) err = GR_SK(24);
    else if (k <= 32) err = GR_SK(32);
    else if (k <= 40) err = GR_SK(40);
    else if (k <= 48) err = GR_SK(48);
    else if (k <= 56) err = GR_SK(56);
    else err = GR_SK(64);
#undef GR_SK
  } else if (va && vb)
    err = dispatch_nt<4, 4>(a, lda, b, ldb, bias, c, ldc, m, (int)n, (int)k, s);
  else if (va)
    err = dispatch_nt<4, 1>(a, lda, b, ldb, bias, c, ldc, m, (int)n, (int)k, s);
  else if (vb)
    err = dispatch_nt<1, 4>(a, lda, b, ldb, bias, c, ldc, m, (int)n, (int)k, s);
  else
    err = dispatch_nt<1, 1>(a, lda, b, ldb, bias, c, ldc, m, (int)n, (int)k, s);
  GR_REQUIRE(err != hipErrorInvalidValue, "gemm_nt: too many workgroups for %lld rows",
             (long long)m);
  GR_HIP_CHECK(err);
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

// Resident form of the same transform for dout = 256 and 16-byte rows of x
// with din <= 100 (the aggregate-first layer 0 of a 100-feature graph).  One
// workgroup of 12 (ELU: 8) wavefronts per CU keeps W (as [column][k], row stride ks
// with ks / 4 odd, so the 16 columns a quarter-wavefront reads with
// ds_read_b128 fall on distinct banks), bias, gamma and beta in LDS for the
// launch; each wavefront then walks 16-row blocks on its own, with no
// workgroup barrier:
//   - the next block's rows of x are loaded into registers before this
//     block's MFMAs, as 16-byte pieces (lane quarter lk takes k = 16 g +
//     4 lk .. + 3 of 16-k group g), turned by a 4 x 4 transpose across the
//     lane quarters into the order linear_ln_act_kernel sums in (step j of
//     group g: k = 16 g + 4 j + lk), with W's groups stored transposed to
//     match, so the two kernels give the same bits; the din % 16 tail takes
//     k = 16 G + 4 j + lk directly, one 4-byte load a step;
//   - the epilogue reads its parameters from LDS, not from global memory:
//     the vector-memory counter retires in issue order, so a global load
//     issued after the block's stores would hold the wavefront until those
//     stores had completed.  Only the next block's loads precede them, so
//     the stores drain while the next block's MFMAs run.
// Rows are staged four at a time in the wavefront's own LDS rows and stored
// as 16-byte pieces of whole rows, as in linear_ln_act_kernel.
constexpr int LR_DOUT = 256;
constexpr int LR_STAGE = LR_DOUT + 16;  // staged row stride (floats)
constexpr int LR_GMAX = 6;              // 16-k groups held in registers: din <= 100
constexpr int LR_KS_MAX = 100;
// Wavefronts per workgroup: 12 (three per SIMD) fit ReLU's registers; ELU's
// expm1f needs more, so it runs eight.
template <int ACT>
constexpr int lr_waves() {
  return ACT == GR_ACT_RELU ? 12 : 8;
}

// LDS row stride for din (a multiple of 4): din itself when din / 4 is odd,
// else din + 4.
inline int lr_row_stride(int din) { return (din / 4) % 2 ? din : din + 4; }

template <int ACT, int LR_WAVES = lr_waves<ACT>()>
__global__ __launch_bounds__(LR_WAVES * 64) void linear_ln_act_resident(
    const float* __restrict__ x, int64_t ldx, int64_t rows, int din, int ks,
    const float* __restrict__ wt, const float* __restrict__ bias,
    const float* __restrict__ gamma, const float* __restrict__ beta, float eps,
    float* __restrict__ h, float* __restrict__ out, float* __restrict__ mean,
    float* __restrict__ rstd) {
  constexpr int NB = LR_DOUT / 16;
  constexpr int LR_LDS = LR_DOUT * LR_KS_MAX + 3 * LR_DOUT + LR_WAVES * 4 * LR_STAGE;
  __shared__ __align__(16) float lds[LR_LDS];
  float* Ws = lds;                          // Ws[c * ks + k] = W^T[k][c]
  float* par = lds + LR_DOUT * LR_KS_MAX;   // bias | gamma | beta
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lr = lane & 15, lk = lane >> 4;
  const int G = din >> 4, tail = (din & 15) >> 2;
  for (int i = tid; i < din * LR_DOUT; i += LR_WAVES * 64) {
    const int k = i / LR_DOUT, c = i % LR_DOUT;
    // Inside each full 16-k group, k = 16 g + 4 b + a sits at 16 g + 4 a + b:
    // a lane's ds_read_b128 at 16 g + 4 lk gives k = 16 g + 4 j + lk in
    // component j.
    const int p = k < 16 * G ? (k & ~15) | ((k & 3) << 2) | ((k >> 2) & 3) : k;
    Ws[c * ks + p] = wt[i];
  }
  for (int i = tid; i < LR_DOUT; i += LR_WAVES * 64) {
    par[i] = bias != nullptr ? bias[i] : 0.f;
    par[LR_DOUT + i] = gamma[i];
    par[2 * LR_DOUT + i] = beta[i];
  }
  __syncthreads();

  float* stage = lds + LR_DOUT * LR_KS_MAX + 3 * LR_DOUT + wave * 4 * LR_STAGE;
  const int64_t nblk = (rows + 15) / 16;
  const int64_t step = (int64_t)gridDim.x * LR_WAVES;
  const float* wl = Ws + lr * ks;

  struct XR {
    float4 v[LR_GMAX];
    float t[3];
  };
  auto load = [&](XR& d, int64_t blk) {
    if (blk >= nblk) return;
    int64_t r = blk * 16 + lr;
    if (r >= rows) r = rows - 1;  // read a valid row; its results are not stored
    const float* p = x + r * ldx;
#pragma unroll
    for (int g = 0; g < LR_GMAX; ++g)
      if (g < G) d.v[g] = *reinterpret_cast<const float4*>(p + 16 * g + 4 * lk);
#pragma unroll
    for (int j = 0; j < 3; ++j)
      if (j < tail) d.t[j] = p[16 * G + lk + 4 * j];
  };

  XR cur, nxt;
  int64_t blk = (int64_t)blockIdx.x * LR_WAVES + wave;
  load(cur, blk);
  const float inv_d = 1.0f / (float)LR_DOUT;
  for (; blk < nblk; blk += step) {
    load(nxt, blk + step);
    floatx4 acc[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[b] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int g = 0; g < LR_GMAX; ++g) {
      if (g < G) {
        // Lane (lr, lk) loaded k = 16 g + 4 lk .. + 3 of its row; after the
        // transpose its component j is k = 16 g + 4 j + lk, the k that lane
        // quarter lk takes in step j of linear_ln_act_kernel's 16-k chunk,
        // so both kernels sum the same products in the same order.
        gr_wave::row_transpose4(cur.v[g]);
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          const float4 bw = *reinterpret_cast<const float4*>(wl + b * 16 * ks + 16 * g + 4 * lk);
          acc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(cur.v[g].x, bw.x, acc[b], 0, 0, 0);
          acc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(cur.v[g].y, bw.y, acc[b], 0, 0, 0);
          acc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(cur.v[g].z, bw.z, acc[b], 0, 0, 0);
          acc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(cur.v[g].w, bw.w, acc[b], 0, 0, 0);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      if (j < tail) {
#pragma unroll
        for (int b = 0; b < NB; ++b)
          acc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(
              cur.t[j], wl[b * 16 * ks + 16 * G + lk + 4 * j], acc[b], 0, 0, 0);
      }
    }

    // Lane holds rows 4 lk + q of the block, columns 16 b + lr.
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const float bb = par[b * 16 + lr];
#pragma unroll
      for (int q = 0; q < 4; ++q) acc[b][q] += bb;
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int64_t row = blk * 16 + lk * 4 + q;
      float s = 0.f;
#pragma unroll
      for (int b = 0; b < NB; ++b) s += acc[b][q];
      s = gr_wave::group_sum<16>(s);
      const float mu = s * inv_d;
      float v = 0.f;
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const float dlt = acc[b][q] - mu;
        v += dlt * dlt;
      }
      v = gr_wave::group_sum<16>(v);
      const float rs = 1.0f / sqrtf(v * inv_d + eps);
      // The wavefront's LDS operations complete in issue order, so this
      // stage's writes follow the previous q's reads without a barrier.
#pragma unroll
      for (int b = 0; b < NB; ++b) stage[lk * LR_STAGE + b * 16 + lr] = acc[b][q];
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      if (row < rows) {
        const float* srow = stage + lk * LR_STAGE;
#pragma unroll
        for (int i = 0; i < LR_DOUT / 64; ++i) {
          const int c = lr * 4 + 64 * i;
          const float4 hv = *reinterpret_cast<const float4*>(srow + c);
          const float4 gg = *reinterpret_cast<const float4*>(par + LR_DOUT + c);
          const float4 bt = *reinterpret_cast<const float4*>(par + 2 * LR_DOUT + c);
          float4 o;
          o.x = lt_act<ACT>(fmaf((hv.x - mu) * rs, gg.x, bt.x));
          o.y = lt_act<ACT>(fmaf((hv.y - mu) * rs, gg.y, bt.y));
          o.z = lt_act<ACT>(fmaf((hv.z - mu) * rs, gg.z, bt.z));
          o.w = lt_act<ACT>(fmaf((hv.w - mu) * rs, gg.w, bt.w));
          *reinterpret_cast<float4*>(h + row * LR_DOUT + c) = hv;
          *reinterpret_cast<float4*>(out + row * LR_DOUT + c) = o;
        }
        if (lr == 0) {
          mean[row] = mu;
          rstd[row] = rs;
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    cur = nxt;
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
  if (dout == LR_DOUT && din % 4 == 0 && din <= LR_KS_MAX &&
      lr_row_stride((int)din) <= LR_KS_MAX && ldx % 4 == 0 && al16(x) &&
      rows >= kResidentMinRows) {
    int dev = 0, cus = 0;
    GR_HIP_CHECK(hipGetDevice(&dev));
    GR_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    // One workgroup per CU (the LDS holds one).
    if (act == GR_ACT_RELU)
      hipLaunchKernelGGL((linear_ln_act_resident<GR_ACT_RELU>), dim3((unsigned)cus),
                         dim3(lr_waves<GR_ACT_RELU>() * 64), 0, s, x, ldx, rows, (int)din,
                         lr_row_stride((int)din), wt, bias, gamma, beta, eps, h, out, mean, rstd);
    else
      hipLaunchKernelGGL((linear_ln_act_resident<GR_ACT_ELU>), dim3((unsigned)cus),
                         dim3(lr_waves<GR_ACT_ELU>() * 64), 0, s, x, ldx, rows, (int)din,
                         lr_row_stride((int)din), wt, bias, gamma, beta, eps, h, out, mean, rstd);
    GR_HIP_CHECK(hipGetLastError());
    return GR_OK;
  }
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
