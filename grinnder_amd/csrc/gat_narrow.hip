// Narrow one-head GAT attention for gfx950: C <= 24 channels (a multiple of
// 4), the shape of C5's 19-class layer (held 20 wide).  Same semantics as
// gat.hip (PyG GATConv as grinnder/nn/gat.py:54-61,69-78 uses it: LeakyReLU
// slope 0.2, softmax denominator + 1e-16, bipartite input (x, x[:B])).
//
// Why a separate path.  At this width a neighbour row is 80 bytes and its
// logit s_j another 4: on MI355X every L2 miss fetches a whole 128-byte line
// (rocprofv3's request-size counters: a random 80-byte row costs 1.625 lines,
// a random 4-byte value a whole line).  The general kernels pay per edge a
// row plus the logit in the forward, and in the backward a gradient row plus
// alpha (through the CSC -> CSR permutation), d_i and c_i, and write the
// destination part of each edge through the permutation.  Here every edge
// costs one line in each direction:
//
// - Packed source rows of 32 floats (128 bytes, line-aligned):
//     Zx[j] = [Hs_j (C) | 0 .. | 24: s_j | 0 ..]
//   A group of 8 lanes holds one row, lane k floats 4k..4k+3; lanes 0-5 the
//   channels, lane 6 the logit s_j (and the scalars of the GX lines below).
//   The destination halves d_i stay a dense vector: a row reads its own d_i
//   next to its neighbours' rows, and d_i alone in a packed line would cost
//   a whole line in the backward.
// - Forward: online softmax, one pass over the row's edges: each group keeps
//   a running max m, sum and weighted sums, rescaled by exp(m_old - m_new)
//   once per block of U edges.  It also forms, for the backward,
//     N_i = sum_{j: t_ij <= 0} alpha_ij Hs_j   and   S_i = sum_{t <= 0} alpha_ij,
//   kept with m_i, den_i in F[i] = [N_i (C) | C: m_i, den_i, S_i, 0], rows
//   of C + 4 floats.  No alpha is stored, and O_i is stored only when the
//   layer has no bias (else the backward takes O_i = Y_i - bias).
// - Backward, destination rows (one pass over rows, no edges):
//     c_i = <G_i, O_i>,  dd_i = sum_j g_t,ij
//         = -0.8 (<G_i, N_i> - c_i S_i) + c_i 1e-16 / den_i,
//   because sum_j g_e,ij = c_i 1e-16 / den_i exactly (softmax is invariant to
//   a shift of row i's logits) and g_t = g_e on t > 0, 0.2 g_e on t <= 0.
//   No per-edge value is written or gathered for it.  Each row leaves a
//   packed line for the source pass:
//     GX[i] = [dL/dO_i (C) | 0 .. | 24: d_i, 25: m_i, 26: 1/den_i, 27: c_i,
//              28: dd_i | 0 ..]
// - Backward, source columns (CSC): per edge one GX line gives G_i and the
//   record; alpha_ij = exp(LeakyReLU(s_j + d_i) - m_i) / den_i is recomputed;
//   dHs_j = sum_i alpha_ij G_i + ds_j att_src + (j < B) dd_j att_dst.
//
// Work decomposition as the other aggregation kernels: whole rows (columns)
// of at most kRowsMax edges run eight to a wavefront, one per 8-lane group;
// longer rows and the units of split rows one to a wavefront, as eight
// 8-lane edge slots, combined in a fixed order; split rows finish in an
// ordered fixup.  Deterministic: no atomics.
//
// Most rows are short (C5's R-MAT graph: 59% of its rows hold only the self
// loop), so the grouped kernels are bound by the chain unit -> column ids ->
// gathered lines of each batch of eight rows, not by bytes.  Their
// wavefronts stride over the batches and issue the next batch's column ids
// and the unit after it before the current batch's gathers.
#include <algorithm>
#include <cfloat>

#include "gr_internal.h"
#include "wave.h"

namespace gr_gatn {

constexpr int kW = 32;        // floats per packed row (one 128-byte line)
constexpr int kMaxC = 24;     // channels a packed row holds
constexpr int kRowsMax = 32;  // longest whole row the grouped kernels take
constexpr int kFwdWs = 52;    // forward split slot: acc (24) | N (24) | m, sum, S, 0
constexpr int kBwdWs = 28;    // backward split slot: acc (24) | ds, 0, 0, 0

__device__ __forceinline__ float leaky(float t) { return t > 0.f ? t : 0.2f * t; }

__device__ __forceinline__ int64_t wave_id() {
  return (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
}

__device__ __forceinline__ float4 ld4(const float* __restrict__ p) {
  return *reinterpret_cast<const float4*>(p);
}

__device__ __forceinline__ void st4(float* __restrict__ p, float4 v) {
  *reinterpret_cast<float4*>(p) = v;
}

__device__ __forceinline__ float dot4(float4 a, float4 b) {
  return fmaf(a.w, b.w, fmaf(a.z, b.z, fmaf(a.y, b.y, a.x * b.x)));
}

__device__ __forceinline__ float4 fma4(float s, float4 a, float4 c) {
  return make_float4(fmaf(s, a.x, c.x), fmaf(s, a.y, c.y), fmaf(s, a.z, c.z), fmaf(s, a.w, c.w));
}

__device__ __forceinline__ float4 scale4(float s, float4 a) {
  return make_float4(s * a.x, s * a.y, s * a.z, s * a.w);
}

__device__ __forceinline__ float4 zero4() { return make_float4(0.f, 0.f, 0.f, 0.f); }

// Lane K of this lane's 8-lane group, for every lane: DPP row_newbcast
// (lane K and lane 8 + K of each 16-lane row) and a select by group.
template <int K>
__device__ __forceinline__ float bcast8(float v) {
  static_assert(K >= 0 && K < 8, "lane of an 8-lane group");
  const float lo = gr_wave::dpp<0x150 + K>(v);
  const float hi = gr_wave::dpp<0x158 + K>(v);
  return (threadIdx.x & 8) ? hi : lo;
}

// Maximum over the 8 lanes that share lane % 8 (the wavefront's edge slots).
__device__ __forceinline__ float slot_max8(float v) {
  v = fmaxf(v, gr_wave::dpp<0x128>(v));  // row_ror:8 = lane ^ 8 within a row
  v = fmaxf(v, gr_wave::xor16(v));
  return fmaxf(v, gr_wave::xor32(v));
}

__device__ __forceinline__ float4 slot_sum4(float4 v) {
  return make_float4(gr_wave::slot_sum<8>(v.x), gr_wave::slot_sum<8>(v.y),
                     gr_wave::slot_sum<8>(v.z), gr_wave::slot_sum<8>(v.w));
}

// Longest unit of the wavefront (every lane gets it).
__device__ __forceinline__ int wave_longest(int len) {
  return (int)gr_wave::wave_max((float)len);
}

// ----------------------------------------------------------------- pack --

// Zx rows of the n_src source rows: Hs and the logit s_j, taken from s_pre or
// formed here as gat_scores_kernel forms it (for C <= 24 its wavefront sum
// reduces to this group sum, bit for bit), which then also writes the
// destination halves d_out [n_dst] and, when s_out is given, s_out [n_src].
__global__ __launch_bounds__(256) void gatn_pack(const float* __restrict__ hs, int64_t ldh,
                                                 int64_t n_src, int64_t n_dst, int C,
                                                 const float* __restrict__ s_pre,
                                                 const float* __restrict__ att_src,
                                                 const float* __restrict__ att_dst,
                                                 float* __restrict__ zx,
                                                 float* __restrict__ s_out,
                                                 float* __restrict__ d_out) {
  const int lane = threadIdx.x & 63, grp = lane >> 3, sub = lane & 7;
  const bool data = sub * 4 < C;
  float4 as = zero4(), ad = zero4();
  if (s_pre == nullptr && data) {
    as = ld4(att_src + sub * 4);
    ad = ld4(att_dst + sub * 4);
  }
  const int64_t nwaves = (int64_t)gridDim.x * 4;
  for (int64_t r0 = wave_id() * 8; r0 < n_src; r0 += nwaves * 8) {
    const int64_t r = r0 + grp;
    const bool act = r < n_src;
    const int64_t rr = act ? r : n_src - 1;
    const float4 h = data ? ld4(hs + rr * ldh + sub * 4) : zero4();
    float sv;
    if (s_pre != nullptr) {
      sv = s_pre[rr];
    } else {
      float ps = 0.f, pd = 0.f;
      ps = fmaf(h.x, as.x, ps);
      pd = fmaf(h.x, ad.x, pd);
      ps = fmaf(h.y, as.y, ps);
      pd = fmaf(h.y, ad.y, pd);
      ps = fmaf(h.z, as.z, ps);
      pd = fmaf(h.z, ad.z, pd);
      ps = fmaf(h.w, as.w, ps);
      pd = fmaf(h.w, ad.w, pd);
      sv = gr_wave::group_sum<8>(ps);
      const float dsum = gr_wave::group_sum<8>(pd);
      if (act && sub == 0 && r < n_dst) d_out[r] = dsum;
      if (act && sub == 0 && s_out != nullptr) s_out[r] = sv;
    }
    float4 out = h;
    if (sub == 6) out = make_float4(sv, 0.f, 0.f, 0.f);
    if (sub == 7) out = zero4();
    if (act) st4(zx + r * kW + sub * 4, out);
  }
}

// -------------------------------------------------------------- forward --

// Running softmax state of one row (or edge slot): max m, sum of
// exp(v - m), the same restricted to t <= 0, and the two weighted row sums.
struct Online {
  float m = -FLT_MAX, sum = 0.f, sneg = 0.f;
  float4 acc = zero4(), nacc = zero4();

  // Takes U edges: logits v[q] (valid[q]) and rows z[q] (this lane's part).
  template <int U>
  __device__ __forceinline__ void take(const float (&v)[U], const bool (&valid)[U],
                                       const float4 (&z)[U]) {
    float mb = m;
#pragma unroll
    for (int q = 0; q < U; ++q)
      if (valid[q]) mb = fmaxf(mb, v[q]);
    const float sc = expf(m - mb);  // 1 when the max stays (or nothing came yet)
    sum *= sc;
    sneg *= sc;
    acc = scale4(sc, acc);
    nacc = scale4(sc, nacc);
#pragma unroll
    for (int q = 0; q < U; ++q) {
      const float p = valid[q] ? expf(v[q] - mb) : 0.f;
      const float pn = v[q] <= 0.f ? p : 0.f;
      sum += p;
      sneg += pn;
      acc = fma4(p, z[q], acc);
      nacc = fma4(pn, z[q], nacc);
    }
    m = mb;
  }
};

// Where a finished row goes: O (optional when Y is given), Y = O + bias
// (optional, row stride ldy) and the state rows F (row stride fs = C + 4).
struct RowOut {
  const float* bias;
  float* o;
  float* y;
  int64_t ldy;
  float* F;
  int fs;
};

// Finishes a whole row from its state: O, N / den, S / den, m, den.
__device__ __forceinline__ void finish_row(const Online& st, bool nonempty, int64_t i, int sub,
                                           int C, const RowOut& out) {
  const float dn = nonempty ? st.sum + 1e-16f : 1.f;
  float* Fi = out.F + i * out.fs;
  if (sub * 4 < C) {
    const float4 ov = make_float4(st.acc.x / dn, st.acc.y / dn, st.acc.z / dn, st.acc.w / dn);
    if (out.o != nullptr) st4(out.o + i * C + sub * 4, ov);
    if (out.y != nullptr) {
      const float4 b = out.bias != nullptr ? ld4(out.bias + sub * 4) : zero4();
      st4(out.y + i * out.ldy + sub * 4,
          make_float4(ov.x + b.x, ov.y + b.y, ov.z + b.z, ov.w + b.w));
    }
    st4(Fi + sub * 4,
        make_float4(st.nacc.x / dn, st.nacc.y / dn, st.nacc.z / dn, st.nacc.w / dn));
  }
  if (sub * 4 == C) st4(Fi + C, make_float4(nonempty ? st.m : 0.f, dn, st.sneg / dn, 0.f));
}

// A group with no row: unit (-1, 0, 0, -1), no edges.
__device__ __forceinline__ int4 no_unit() { return make_int4(-1, 0, 0, -1); }

// Group grp's unit of batch b (batches of 8 consecutive units): a whole row
// of at most maxlen edges, else no_unit().
__device__ __forceinline__ int4 batch_unit(const int4* __restrict__ units, int64_t n_units,
                                           int64_t b, int grp, int maxlen) {
  const int64_t u = b * 8 + grp;
  if (u >= n_units) return no_unit();
  const int4 w = units[u];
  return w.w < 0 && w.z - w.y <= maxlen ? w : no_unit();
}

// Lane sub's id of edge sub of a unit (0 past the end): the first block of
// eight edges, which holds the whole of most rows.
__device__ __forceinline__ int first_id(int4 w, int sub, const int32_t* __restrict__ ids) {
  return sub < w.z - w.y ? ids[w.y + sub] : 0;
}

// The remaining ids of a unit: lane sub holds edges 8 + sub, 16 + sub, ...
// (0 past the end); c[0] is first_id's.
template <int R>
__device__ __forceinline__ void rest_ids(int4 w, int sub, const int32_t* __restrict__ ids,
                                         int (&c)[R]) {
  const int len = w.z - w.y;
#pragma unroll
  for (int r = 1; r < R; ++r) c[r] = r * 8 + sub < len ? ids[w.y + r * 8 + sub] : 0;
}

// Whole rows of at most R * 8 edges, one per 8-lane group, eight rows (a
// batch) per wavefront step; the wavefronts stride over the batches.  Lane
// sub holds the column ids of edges sub, 8 + sub, ...; blocks of U edges are
// gathered (one packed line each) and folded into the running state.
template <int R, int U>
__global__ __launch_bounds__(256) void gatn_fwd_rows(const int4* __restrict__ units,
                                                     int64_t n_units,
                                                     const int32_t* __restrict__ idx,
                                                     const float* __restrict__ zx,
                                                     const float* __restrict__ dv, int C,
                                                     RowOut out) {
  const int lane = threadIdx.x & 63, grp = lane >> 3, sub = lane & 7, base = grp * 8;
  const int64_t nb = (n_units + 7) / 8;
  const int64_t stride = (int64_t)gridDim.x * 4;
  int64_t b = wave_id();
  if (b >= nb) return;
  int4 w = batch_unit(units, n_units, b, grp, R * 8);
  int4 wn = batch_unit(units, n_units, b + stride, grp, R * 8);
  int c0 = first_id(w, sub, idx);
  float di = w.z > w.y ? dv[w.x] : 0.f;
  while (true) {
    // The next batch's first ids and d (its unit came one step ago) and the
    // unit after it, then this batch's remaining ids, before its gathers.
    const int c0n = first_id(wn, sub, idx);
    const float dn = wn.z > wn.y ? dv[wn.x] : 0.f;
    const int4 wnn = batch_unit(units, n_units, b + 2 * stride, grp, R * 8);
    int cr[R];
    cr[0] = c0;
    rest_ids<R>(w, sub, idx, cr);

    const int len = w.z - w.y;
    const int steps = wave_longest(len);
    Online st;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (r * 8 < steps) {
#pragma unroll
        for (int q0 = 0; q0 < 8; q0 += U) {
          float4 z[U];
          bool valid[U];
#pragma unroll
          for (int q = 0; q < U; ++q) {
            const int c = __shfl(cr[r], base + q0 + q, 64);
            valid[q] = r * 8 + q0 + q < len;
            z[q] = valid[q] ? ld4(zx + (int64_t)c * kW + sub * 4) : zero4();
          }
          float v[U];
#pragma unroll
          for (int q = 0; q < U; ++q) v[q] = leaky(bcast8<6>(z[q].x) + di);
          st.take<U>(v, valid, z);
        }
      }
    }
    if (w.x >= 0) finish_row(st, len > 0, w.x, sub, C, out);

    b += stride;
    if (b >= nb) break;
    w = wn;
    wn = wnn;
    c0 = c0n;
    di = dn;
  }
}

// Split rows and whole rows longer than the grouped kernel takes: one unit
// per wavefront, its edges in eight 8-lane slots (slot k takes edges k,
// 8 + k, ... of each 64-edge chunk), the slots' states merged at the end in
// a fixed order.  A split row's unit leaves (acc, N, m, sum, S) in its slot
// of the workspace.
template <int U>
__global__ __launch_bounds__(256) void gatn_fwd_units(const int4* __restrict__ units,
                                                      const int32_t* __restrict__ which,
                                                      int64_t n_units,
                                                      const int32_t* __restrict__ idx,
                                                      const float* __restrict__ zx,
                                                      const float* __restrict__ dv, int C,
                                                      RowOut out, float* __restrict__ ws) {
  const int lane = threadIdx.x & 63, slot = lane >> 3, sub = lane & 7;
  const int64_t wid = wave_id();
  if (wid >= n_units) return;
  const int4 w = units[which != nullptr ? (int64_t)which[wid] : wid];
  const int len = w.z - w.y;
  if (w.w < 0 && len <= kRowsMax) return;  // the grouped kernel's row
  const int64_t i = w.x;
  const float di = dv[i];
  Online st;
  for (int b = w.y; b < w.z; b += 64) {
    const int n = min(64, w.z - b);
    const int cl = idx[b + min(lane, n - 1)];
#pragma unroll
    for (int t0 = 0; t0 < 8; t0 += U) {
      if (t0 * 8 >= n) break;
      float4 z[U];
      bool valid[U];
#pragma unroll
      for (int q = 0; q < U; ++q) {
        const int e = (t0 + q) * 8 + slot;
        const int c = __shfl(cl, e, 64);
        valid[q] = e < n;
        z[q] = valid[q] ? ld4(zx + (int64_t)c * kW + sub * 4) : zero4();
      }
      float v[U];
#pragma unroll
      for (int q = 0; q < U; ++q) v[q] = leaky(bcast8<6>(z[q].x) + di);
      st.take<U>(v, valid, z);
    }
  }
  // Merge the slots: rescale each to the unit's max, then sum in slot order.
  const float mx = slot_max8(st.m);
  const float sc = expf(st.m - mx);
  Online all;
  all.m = mx;
  all.sum = gr_wave::slot_sum<8>(st.sum * sc);
  all.sneg = gr_wave::slot_sum<8>(st.sneg * sc);
  all.acc = slot_sum4(scale4(sc, st.acc));
  all.nacc = slot_sum4(scale4(sc, st.nacc));
  if (slot != 0) return;
  if (w.w < 0) {
    finish_row(all, true, i, sub, C, out);
    return;
  }
  float* p = ws + (int64_t)w.w * kFwdWs;
  if (sub * 4 < C) {
    st4(p + sub * 4, all.acc);
    st4(p + kMaxC + sub * 4, all.nacc);
  }
  if (sub == 0) st4(p + 2 * kMaxC, make_float4(all.m, all.sum, all.sneg, 0.f));
}

// Split rows: one wavefront per row, lane f < C a channel, the units' states
// merged in slot order.
__global__ __launch_bounds__(256) void gatn_fwd_fixup(const int32_t* __restrict__ fix,
                                                      int64_t n_fix,
                                                      const float* __restrict__ ws, int C,
                                                      RowOut out) {
  const int lane = threadIdx.x & 63;
  const int64_t wid = wave_id();
  if (wid >= n_fix) return;
  const int row = fix[3 * wid + 0], first = fix[3 * wid + 1], n = fix[3 * wid + 2];
  float mx = -FLT_MAX;
  for (int k = 0; k < n; ++k) mx = fmaxf(mx, ws[(int64_t)(first + k) * kFwdWs + 2 * kMaxC]);
  float sum = 0.f, sneg = 0.f, acc = 0.f, nacc = 0.f;
  for (int k = 0; k < n; ++k) {
    const float* p = ws + (int64_t)(first + k) * kFwdWs;
    const float sc = expf(p[2 * kMaxC] - mx);
    sum = fmaf(p[2 * kMaxC + 1], sc, sum);
    sneg = fmaf(p[2 * kMaxC + 2], sc, sneg);
    if (lane < C) {
      acc = fmaf(p[lane], sc, acc);
      nacc = fmaf(p[kMaxC + lane], sc, nacc);
    }
  }
  const float dn = sum + 1e-16f;
  const int64_t i = row;
  float* Fi = out.F + i * out.fs;
  if (lane < C) {
    const float ov = acc / dn;
    if (out.o != nullptr) out.o[i * C + lane] = ov;
    if (out.y != nullptr)
      out.y[i * out.ldy + lane] = ov + (out.bias != nullptr ? out.bias[lane] : 0.f);
    Fi[lane] = nacc / dn;
  }
  if (lane == 0) st4(Fi + C, make_float4(mx, dn, sneg / dn, 0.f));
}

// ------------------------------------------------------------- backward --

// Destination rows: c_i, dd_i and the GX line of each row.  Eight rows a
// wavefront, grid-stride over wavefronts.  O_i is read from `out` (row
// stride ldo), less the bias when one is given (out then holds Y).
__global__ __launch_bounds__(256) void gatn_bwd_dst(int64_t n_dst, const float* __restrict__ go,
                                                    int64_t ldg, const float* __restrict__ out,
                                                    int64_t ldo, const float* __restrict__ bias,
                                                    const float* __restrict__ F, int fs,
                                                    const float* __restrict__ dv, int C,
                                                    float* __restrict__ gx,
                                                    float* __restrict__ dd) {
  const int lane = threadIdx.x & 63, grp = lane >> 3, sub = lane & 7;
  const bool data = sub * 4 < C;
  const float4 b = data && bias != nullptr ? ld4(bias + sub * 4) : zero4();
  const int64_t nwaves = (int64_t)gridDim.x * 4;
  for (int64_t r0 = wave_id() * 8; r0 < n_dst; r0 += nwaves * 8) {
    const int64_t r = r0 + grp;
    const bool act = r < n_dst;
    const int64_t rr = act ? r : n_dst - 1;
    const float4 g = data ? ld4(go + rr * ldg + sub * 4) : zero4();
    float4 ov = data ? ld4(out + rr * ldo + sub * 4) : zero4();
    ov = make_float4(ov.x - b.x, ov.y - b.y, ov.z - b.z, ov.w - b.w);
    const float4 nv = data ? ld4(F + rr * fs + sub * 4) : zero4();
    const float4 st = ld4(F + rr * fs + C);  // m, den, S
    const float di = dv[rr];
    const float c = gr_wave::group_sum<8>(dot4(g, ov));
    const float u = gr_wave::group_sum<8>(dot4(g, nv));
    const float ddv = fmaf(-0.8f, fmaf(-c, st.z, u), c * (1e-16f / st.y));
    float4 line = g;
    if (sub == 6) line = make_float4(di, st.x, 1.f / st.y, c);
    if (sub == 7) line = make_float4(ddv, 0.f, 0.f, 0.f);
    if (act) {
      st4(gx + r * kW + sub * 4, line);
      if (sub == 0) dd[r] = ddv;
    }
  }
}

// One edge of the source pass: the GX line g of destination i (this lane's
// part), the column's s_j and Hs_j part; accumulates alpha G_i and ds_j.
__device__ __forceinline__ void bwd_edge(float4 g, bool valid, float sj, float4 hsj,
                                         float4& acc, float& dsl) {
  const float ga = gr_wave::group_sum<8>(dot4(g, hsj));
  const float di = bcast8<6>(g.x), mi = bcast8<6>(g.y), inv = bcast8<6>(g.z),
              ci = bcast8<6>(g.w);
  const float t = sj + di;
  const float al = valid ? expf(leaky(t) - mi) * inv : 0.f;
  const float ge = al * (ga - ci);
  dsl += t > 0.f ? ge : 0.2f * ge;
  acc = fma4(al, g, acc);
}

// Writes dHs_j = acc + ds_j att_src (+ dd_j att_dst for j < n_dst).
__device__ __forceinline__ void finish_col(float4 acc, float dsl, int64_t j, int64_t n_dst,
                                           int sub, int C, const float* __restrict__ gx,
                                           const float* __restrict__ att_src,
                                           const float* __restrict__ att_dst,
                                           float* __restrict__ dhs, float* __restrict__ ds) {
  if (sub * 4 < C) {
    float4 v = fma4(dsl, ld4(att_src + sub * 4), acc);
    if (j < n_dst) v = fma4(gx[j * kW + 28], ld4(att_dst + sub * 4), v);
    st4(dhs + j * C + sub * 4, v);
  }
  if (sub == 0) ds[j] = dsl;
}

// Whole columns of at most R * 8 edges, one per 8-lane group, eight columns
// (a batch) per wavefront step, the wavefronts striding over the batches as
// in gatn_fwd_rows.
template <int R, int U>
__global__ __launch_bounds__(256) void gatn_bwd_rows(const int4* __restrict__ units,
                                                     int64_t n_units,
                                                     const int32_t* __restrict__ row_idx,
                                                     const float* __restrict__ zx,
                                                     const float* __restrict__ gx, int C,
                                                     int64_t n_dst,
                                                     const float* __restrict__ att_src,
                                                     const float* __restrict__ att_dst,
                                                     float* __restrict__ dhs,
                                                     float* __restrict__ ds) {
  const int lane = threadIdx.x & 63, grp = lane >> 3, sub = lane & 7, base = grp * 8;
  const int64_t nb = (n_units + 7) / 8;
  const int64_t stride = (int64_t)gridDim.x * 4;
  int64_t b = wave_id();
  if (b >= nb) return;
  int4 w = batch_unit(units, n_units, b, grp, R * 8);
  int4 wn = batch_unit(units, n_units, b + stride, grp, R * 8);
  int i0 = first_id(w, sub, row_idx);
  float4 hz = ld4(zx + (int64_t)max(w.x, 0) * kW + sub * 4);
  while (true) {
    // The next batch's first row ids and own lines, the unit after it, then
    // this batch's remaining row ids, before its gathers.
    const int i0n = first_id(wn, sub, row_idx);
    const float4 hzn = ld4(zx + (int64_t)max(wn.x, 0) * kW + sub * 4);
    const int4 wnn = batch_unit(units, n_units, b + 2 * stride, grp, R * 8);
    int ir[R];
    ir[0] = i0;
    rest_ids<R>(w, sub, row_idx, ir);

    const int len = w.z - w.y;
    const int steps = wave_longest(len);
    const float sj = bcast8<6>(hz.x);
    const float4 hsj = sub * 4 < C ? hz : zero4();
    float4 acc = zero4();
    float dsl = 0.f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (r * 8 < steps) {
#pragma unroll
        for (int q0 = 0; q0 < 8; q0 += U) {
          float4 g[U];
          bool valid[U];
#pragma unroll
          for (int q = 0; q < U; ++q) {
            const int ii = __shfl(ir[r], base + q0 + q, 64);
            valid[q] = r * 8 + q0 + q < len;
            g[q] = valid[q] ? ld4(gx + (int64_t)ii * kW + sub * 4) : zero4();
          }
#pragma unroll
          for (int q = 0; q < U; ++q) bwd_edge(g[q], valid[q], sj, hsj, acc, dsl);
        }
      }
    }
    if (w.x >= 0) finish_col(acc, dsl, w.x, n_dst, sub, C, gx, att_src, att_dst, dhs, ds);

    b += stride;
    if (b >= nb) break;
    w = wn;
    wn = wnn;
    i0 = i0n;
    hz = hzn;
  }
}

// Split columns and long whole columns: one unit per wavefront, eight 8-lane
// edge slots, summed in slot order.  A split column's unit leaves (acc, ds)
// in its workspace slot.
template <int U>
__global__ __launch_bounds__(256) void gatn_bwd_units(const int4* __restrict__ units,
                                                      const int32_t* __restrict__ which,
                                                      int64_t n_units,
                                                      const int32_t* __restrict__ row_idx,
                                                      const float* __restrict__ zx,
                                                      const float* __restrict__ gx, int C,
                                                      int64_t n_dst,
                                                      const float* __restrict__ att_src,
                                                      const float* __restrict__ att_dst,
                                                      float* __restrict__ dhs,
                                                      float* __restrict__ ds,
                                                      float* __restrict__ ws) {
  const int lane = threadIdx.x & 63, slot = lane >> 3, sub = lane & 7;
  const int64_t wid = wave_id();
  if (wid >= n_units) return;
  const int4 w = units[which != nullptr ? (int64_t)which[wid] : wid];
  if (w.w < 0 && w.z - w.y <= kRowsMax) return;  // the grouped kernel's column
  const int64_t j = w.x;
  const float4 hz = ld4(zx + j * kW + sub * 4);
  const float sj = bcast8<6>(hz.x);
  const float4 hsj = sub * 4 < C ? hz : zero4();
  float4 acc = zero4();
  float dsl = 0.f;
  for (int b = w.y; b < w.z; b += 64) {
    const int n = min(64, w.z - b);
    const int il = row_idx[b + min(lane, n - 1)];
#pragma unroll
    for (int t0 = 0; t0 < 8; t0 += U) {
      if (t0 * 8 >= n) break;
      float4 g[U];
      bool valid[U];
#pragma unroll
      for (int q = 0; q < U; ++q) {
        const int e = (t0 + q) * 8 + slot;
        const int ii = __shfl(il, e, 64);
        valid[q] = e < n;
        g[q] = valid[q] ? ld4(gx + (int64_t)ii * kW + sub * 4) : zero4();
      }
#pragma unroll
      for (int q = 0; q < U; ++q) bwd_edge(g[q], valid[q], sj, hsj, acc, dsl);
    }
  }
  acc = slot_sum4(acc);
  dsl = gr_wave::slot_sum<8>(dsl);
  if (slot != 0) return;
  if (w.w < 0) {
    finish_col(acc, dsl, j, n_dst, sub, C, gx, att_src, att_dst, dhs, ds);
    return;
  }
  float* p = ws + (int64_t)w.w * kBwdWs;
  if (sub * 4 < C) st4(p + sub * 4, acc);
  if (sub == 0) st4(p + kMaxC, make_float4(dsl, 0.f, 0.f, 0.f));
}

// Split columns: the units' (acc, ds) summed in slot order, then finished as
// a whole column.
__global__ __launch_bounds__(256) void gatn_bwd_fixup(const int32_t* __restrict__ fix,
                                                      int64_t n_fix,
                                                      const float* __restrict__ ws, int C,
                                                      int64_t n_dst,
                                                      const float* __restrict__ gx,
                                                      const float* __restrict__ att_src,
                                                      const float* __restrict__ att_dst,
                                                      float* __restrict__ dhs,
                                                      float* __restrict__ ds) {
  const int lane = threadIdx.x & 63;
  const int64_t wid = wave_id();
  if (wid >= n_fix) return;
  const int col = fix[3 * wid + 0], first = fix[3 * wid + 1], n = fix[3 * wid + 2];
  float acc = 0.f, dsl = 0.f;
  for (int k = 0; k < n; ++k) {
    const float* p = ws + (int64_t)(first + k) * kBwdWs;
    dsl += p[kMaxC];
    if (lane < C) acc += p[lane];
  }
  const int64_t j = col;
  if (lane < C) {
    float v = fmaf(dsl, att_src[lane], acc);
    if (j < n_dst) v = fmaf(gx[j * kW + 28], att_dst[lane], v);
    dhs[j * C + lane] = v;
  }
  if (lane == 0) ds[j] = dsl;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

inline unsigned blocks_for(int64_t waves) { return (unsigned)((waves + 3) / 4); }

// Wavefronts for the grid-stride row passes: enough to fill the device.
inline unsigned stride_blocks(int64_t rows) {
  const int64_t waves = (rows + 7) / 8;
  return (unsigned)std::max<int64_t>(1, std::min<int64_t>(blocks_for(waves), 8192));
}

}  // namespace gr_gatn

using namespace gr_gatn;

extern "C" int gr_gat_narrow_pack(const float* hs, int64_t ldh, int64_t n_src, int64_t n_dst,
                                  int64_t channels, const float* att_src, const float* att_dst,
                                  float* zx, float* s, float* d, void* stream) {
  gr::clear_error();
  const int64_t C = channels;
  GR_REQUIRE(C >= 4 && C <= kMaxC && C % 4 == 0,
             "gat_narrow_pack: channels %lld not a multiple of 4 in [4, %d]", (long long)C,
             kMaxC);
  GR_REQUIRE(n_src >= 0 && n_dst >= 0 && n_dst <= n_src && ldh >= C && ldh % 4 == 0,
             "gat_narrow_pack: bad extents");
  if (n_src == 0) return GR_OK;
  GR_REQUIRE(hs && aligned16(hs) && zx && aligned16(zx) && att_src && aligned16(att_src) &&
                 att_dst && aligned16(att_dst) && s && (n_dst == 0 || d),
             "gat_narrow_pack: NULL or misaligned pointer");
  hipLaunchKernelGGL(gatn_pack, dim3(stride_blocks(n_src)), dim3(256), 0, gr::as_stream(stream),
                     hs, ldh, n_src, n_dst, (int)C, (const float*)nullptr, att_src, att_dst, zx,
                     s, d);
  GR_HIP_CHECK(hipGetLastError());
  return GR_OK;
}

extern "C" int gr_gat_narrow_forward(const int32_t* units, int64_t n_units,
                                     const int32_t* fixups, int64_t n_fix,
                                     const int32_t* long_units, int64_t n_long,
                                     const int32_t* idx,
                                     const float* hs, int64_t ldh, int64_t n_src, int64_t n_dst,
                                     int64_t channels, const float* s_pre, const float* d_pre,
                                     const float* att_src, const float* att_dst,
                                     const float* bias, float* zx, float* o, float* y,
                                     int64_t ldy, float* d_state, float* f_state,
                                     float* workspace, int64_t ws_floats, int64_t n_slots,
                                     void* stream) {
  gr::clear_error();
  const int64_t C = channels;
  GR_REQUIRE(C >= 4 && C <= kMaxC && C % 4 == 0,
             "gat_narrow_forward: channels %lld not a multiple of 4 in [4, %d]", (long long)C,
             kMaxC);
  GR_REQUIRE(n_units >= 0 && n_fix >= 0 && n_slots >= 0 && n_src >= 0 && n_dst >= 0 &&
                 n_dst <= n_src,
             "gat_narrow_forward: bad extents");
  GR_REQUIRE(n_slots >= 2 * n_fix && n_slots <= n_units,
             "gat_narrow_forward: n_slots %lld inconsistent with the plan (n_fix %lld)",
             (long long)n_slots, (long long)n_fix);
  GR_REQUIRE(n_fix == 0 || (fixups != nullptr && workspace != nullptr &&
                            ws_floats >= n_slots * kFwdWs && aligned16(workspace)),
             "gat_narrow_forward: workspace of %lld floats, %lld needed",
             (long long)ws_floats, (long long)(n_slots * kFwdWs));
  GR_REQUIRE(ldh >= C && ldh % 4 == 0 && (y == nullptr || (ldy >= C && ldy % 4 == 0)),
             "gat_narrow_forward: bad leading dims");
  GR_REQUIRE(long_units == nullptr || (n_long >= n_slots && n_long <= n_units),
             "gat_narrow_forward: n_long %lld outside [n_slots, n_units]", (long long)n_long);
  GR_REQUIRE((s_pre == nullptr) == (d_pre == nullptr),
             "gat_narrow_forward: give both logit halves or neither");
  GR_REQUIRE(o != nullptr || y != nullptr, "gat_narrow_forward: neither o nor y given");
  GR_REQUIRE(hs != nullptr || d_pre != nullptr,
             "gat_narrow_forward: packed rows (hs NULL) need d_pre");
  if (n_src == 0) return GR_OK;
  GR_REQUIRE(zx && aligned16(zx) &&
                 (hs == nullptr || (aligned16(hs) &&
                                    (s_pre != nullptr ||
                                     (att_src && aligned16(att_src) && att_dst &&
                                      aligned16(att_dst) && (n_dst == 0 || d_state))))),
             "gat_narrow_forward: NULL or misaligned pointer");
  hipStream_t st = gr::as_stream(stream);
  if (hs != nullptr) {
    hipLaunchKernelGGL(gatn_pack, dim3(stride_blocks(n_src)), dim3(256), 0, st, hs, ldh, n_src,
                       n_dst, (int)C, s_pre, att_src, att_dst, zx, (float*)nullptr, d_state);
    GR_HIP_CHECK(hipGetLastError());
  }
  if (n_units == 0) return GR_OK;
  GR_REQUIRE(units && aligned16(units) && idx && (o == nullptr || aligned16(o)) && f_state &&
                 aligned16(f_state) && (y == nullptr || aligned16(y)) &&
                 (bias == nullptr || aligned16(bias)),
             "gat_narrow_forward: NULL or misaligned pointer");
  const float* dv = d_pre != nullptr ? d_pre : d_state;
  const RowOut out{bias, o, y, ldy, f_state, (int)C + 4};
  const int4* u4 = reinterpret_cast<const int4*>(units);
  const int64_t n_first = long_units != nullptr ? n_long : n_units;
  if (n_first > 0) {
    hipLaunchKernelGGL((gatn_fwd_units<4>), dim3(blocks_for(n_first)), dim3(256), 0, st, u4,
                       long_units, n_first, idx, zx, dv, (int)C, out, workspace);
    GR_HIP_CHECK(hipGetLastError());
  }
  const int64_t n_whole = n_units - n_slots;
  if (n_whole > 0) {
    hipLaunchKernelGGL((gatn_fwd_rows<kRowsMax / 8, 4>), dim3(stride_blocks(n_whole)),
                       dim3(256), 0, st, u4 + n_slots, n_whole, idx, zx, dv, (int)C, out);
    GR_HIP_CHECK(hipGetLastError());
  }
  if (n_fix > 0) {
    hipLaunchKernelGGL(gatn_fwd_fixup, dim3(blocks_for(n_fix)), dim3(256), 0, st, fixups,
                       n_fix, workspace, (int)C, out);
    GR_HIP_CHECK(hipGetLastError());
  }
  return GR_OK;
}

extern "C" int gr_gat_narrow_backward(const int32_t* units, int64_t n_units,
                                      const int32_t* fixups, int64_t n_fix,
                                      const int32_t* long_units, int64_t n_long,
                                      const int32_t* row_idx, const float* zx, const float* d,
                                      int64_t n_src, int64_t n_dst, int64_t channels,
                                      const float* go, int64_t ldg, const float* out,
                                      int64_t ldo, const float* bias, const float* f_state,
                                      const float* att_src, const float* att_dst, float* gx,
                                      float* dhs, float* ds, float* dd, float* workspace,
                                      int64_t ws_floats, int64_t n_slots, void* stream) {
  gr::clear_error();
  const int64_t C = channels;
  GR_REQUIRE(C >= 4 && C <= kMaxC && C % 4 == 0,
             "gat_narrow_backward: channels %lld not a multiple of 4 in [4, %d]", (long long)C,
             kMaxC);
  GR_REQUIRE(n_units >= 0 && n_fix >= 0 && n_slots >= 0 && n_src >= 0 && n_dst >= 0 &&
                 n_dst <= n_src,
             "gat_narrow_backward: bad extents");
  GR_REQUIRE(n_slots >= 2 * n_fix && n_slots <= n_units,
             "gat_narrow_backward: n_slots %lld inconsistent with the plan (n_fix %lld)",
             (long long)n_slots, (long long)n_fix);
  GR_REQUIRE(n_fix == 0 || (fixups != nullptr && workspace != nullptr &&
                            ws_floats >= n_slots * kBwdWs && aligned16(workspace)),
             "gat_narrow_backward: workspace of %lld floats, %lld needed",
             (long long)ws_floats, (long long)(n_slots * kBwdWs));
  GR_REQUIRE(ldg >= C && ldg % 4 == 0 && ldo >= C && ldo % 4 == 0,
             "gat_narrow_backward: bad leading dims");
  GR_REQUIRE(long_units == nullptr || (n_long >= n_slots && n_long <= n_units),
             "gat_narrow_backward: n_long %lld outside [n_slots, n_units]", (long long)n_long);
  GR_REQUIRE(zx && aligned16(zx) && gx && aligned16(gx) && att_src && aligned16(att_src) &&
                 att_dst && aligned16(att_dst) && dhs && aligned16(dhs) && ds && dd,
             "gat_narrow_backward: NULL or misaligned pointer");
  hipStream_t st = gr::as_stream(stream);
  if (n_dst > 0) {
    GR_REQUIRE(go && aligned16(go) && out && aligned16(out) && f_state && aligned16(f_state) &&
                   d && (bias == nullptr || aligned16(bias)),
               "gat_narrow_backward: NULL or misaligned pointer");
    hipLaunchKernelGGL(gatn_bwd_dst, dim3(stride_blocks(n_dst)), dim3(256), 0, st, n_dst, go,
                       ldg, out, ldo, bias, f_state, (int)C + 4, d, (int)C, gx, dd);
    GR_HIP_CHECK(hipGetLastError());
  }
  if (n_units == 0) return GR_OK;
  GR_REQUIRE(units && aligned16(units) && row_idx, "gat_narrow_backward: NULL plan");
  const int4* u4 = reinterpret_cast<const int4*>(units);
  const int64_t n_first = long_units != nullptr ? n_long : n_units;
  if (n_first > 0) {
    hipLaunchKernelGGL((gatn_bwd_units<4>), dim3(blocks_for(n_first)), dim3(256), 0, st, u4,
                       long_units, n_first, row_idx, zx, gx, (int)C, n_dst, att_src, att_dst,
                       dhs, ds, workspace);
    GR_HIP_CHECK(hipGetLastError());
  }
  const int64_t n_whole = n_units - n_slots;
  if (n_whole > 0) {
    hipLaunchKernelGGL((gatn_bwd_rows<kRowsMax / 8, 4>), dim3(stride_blocks(n_whole)),
                       dim3(256), 0, st, u4 + n_slots, n_whole, row_idx, zx, gx, (int)C, n_dst,
                       att_src, att_dst, dhs, ds);
    GR_HIP_CHECK(hipGetLastError());
  }
  if (n_fix > 0) {
    hipLaunchKernelGGL(gatn_bwd_fixup, dim3(blocks_for(n_fix)), dim3(256), 0, st, fixups, n_fix,
                       workspace, (int)C, n_dst, gx, att_src, att_dst, dhs, ds);
    GR_HIP_CHECK(hipGetLastError());
  }
  return GR_OK;
}
