/*
 * CPU oracle for the partitioned GNN layer hot path — TEST INFRASTRUCTURE.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as a checker or as the timed CPU baseline; the
 * product (grinnder_amd) never calls it.
 *
 * Plain, sequential C restatements of the arithmetic the reference performs
 * through third-party libraries (PyG GCNConv/GATConv, torch_sparse spmm_sum),
 * accumulated in double precision.  Each function cites the reference call
 * site whose semantics it restates.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* GCN aggregation Y = A Z + b over a CSR [rows x cols] (rows = destination
 * nodes), as PyG GCNConv(normalize=False) computes it with a SparseTensor
 * adjacency: message_and_aggregate = spmm(adj_t, x, reduce="sum") then
 * "+ bias" (grinnder/nn/gcn.py:53-56,65; grinnder/engine/trainer.py:
 * 288-302).  Also the backward dZ = A^T G when called with the transpose. */
void orc_spmm_csr(int64_t rows, const int64_t* rowptr, const int64_t* col,
                  const float* val, const float* x, int64_t ldx, int64_t dim,
                  const float* bias, double* out) {
  for (int64_t i = 0; i < rows; ++i) {
    double* o = out + i * dim;
    for (int64_t f = 0; f < dim; ++f) o[f] = bias ? (double)bias[f] : 0.0;
    for (int64_t e = rowptr[i]; e < rowptr[i + 1]; ++e) {
      const double w = val ? (double)val[e] : 1.0;
      const float* xr = x + col[e] * ldx;
      for (int64_t f = 0; f < dim; ++f) o[f] += w * (double)xr[f];
    }
  }
}

/* orc_spmm_csr restricted to the n_sel rows listed in `sel`: out row k is
 * row sel[k] of A Z (+ b).  Lets a caller check sampled rows of a pass at
 * full size without running every row. */
void orc_spmm_rows(int64_t n_sel, const int64_t* sel, const int64_t* rowptr,
                   const int64_t* col, const float* val, const float* x,
                   int64_t ldx, int64_t dim, const float* bias, double* out) {
  for (int64_t k = 0; k < n_sel; ++k) {
    const int64_t i = sel[k];
    double* o = out + k * dim;
    for (int64_t f = 0; f < dim; ++f) o[f] = bias ? (double)bias[f] : 0.0;
    for (int64_t e = rowptr[i]; e < rowptr[i + 1]; ++e) {
      const double w = val ? (double)val[e] : 1.0;
      const float* xr = x + col[e] * ldx;
      for (int64_t f = 0; f < dim; ++f) o[f] += w * (double)xr[f];
    }
  }
}

/* Transposed aggregation dZ[c] = sum_{(r,c)} val * G[r] computed directly
 * from the CSR (scatter form), independent of any CSC construction. */
void orc_spmm_csr_t(int64_t rows, int64_t cols, const int64_t* rowptr,
                    const int64_t* col, const float* val, const float* g,
                    int64_t dim, double* out) {
  memset(out, 0, sizeof(double) * (size_t)(cols * dim));
  for (int64_t i = 0; i < rows; ++i) {
    for (int64_t e = rowptr[i]; e < rowptr[i + 1]; ++e) {
      const double w = val ? (double)val[e] : 1.0;
      double* o = out + col[e] * dim;
      const float* gr = g + i * dim;
      for (int64_t f = 0; f < dim; ++f) o[f] += w * (double)gr[f];
    }
  }
}

static double leaky(double t) { return t > 0.0 ? t : 0.2 * t; }

/* PyG GATConv forward over a bipartite CSR [B x E] with x_src = Hs (all E
 * rows) and x_dst = Hs[:B] (grinnder/nn/gat.py:54-61,72-73):
 *   alpha_src = <Hs_j, att_src>, alpha_dst = <Hs_i, att_dst>,
 *   e = LeakyReLU_{0.2}(alpha_src_j + alpha_dst_i),
 *   alpha = exp(e - max_row e) / (sum_row exp(e - max) + 1e-16)  (PyG softmax),
 *   O_i = sum_j alpha_ij Hs_j,  out = concat ? O : mean_h O,  + bias.
 * Outputs: out [B, concat ? H*C : C], alpha [nnz*H] (edge-major), also the
 * pre-activation t [nnz*H] for the backward. */
void orc_gat_forward(int64_t B, int64_t E, const int64_t* rowptr,
                     const int64_t* col, const float* hs, int64_t H, int64_t C,
                     const float* att_src, const float* att_dst,
                     const float* bias, int32_t concat, double* out,
                     double* alpha, double* tpre) {
  const int64_t HC = H * C;
  double* s = (double*)calloc((size_t)(E * H), sizeof(double));
  double* d = (double*)calloc((size_t)((B > 0 ? B : 1) * H), sizeof(double));
  for (int64_t j = 0; j < E; ++j)
    for (int64_t h = 0; h < H; ++h) {
      double a = 0.0;
      for (int64_t c = 0; c < C; ++c) a += (double)hs[j * HC + h * C + c] * att_src[h * C + c];
      s[j * H + h] = a;
    }
  for (int64_t i = 0; i < B; ++i)
    for (int64_t h = 0; h < H; ++h) {
      double a = 0.0;
      for (int64_t c = 0; c < C; ++c) a += (double)hs[i * HC + h * C + c] * att_dst[h * C + c];
      d[i * H + h] = a;
    }
  const int64_t out_w = concat ? HC : C;
  double* o = (double*)calloc((size_t)HC, sizeof(double));
  for (int64_t i = 0; i < B; ++i) {
    memset(o, 0, sizeof(double) * (size_t)HC);
    for (int64_t h = 0; h < H; ++h) {
      double mx = -INFINITY;
      for (int64_t e = rowptr[i]; e < rowptr[i + 1]; ++e) {
        const double t = s[col[e] * H + h] + d[i * H + h];
        tpre[e * H + h] = t;
        const double v = leaky(t);
        if (v > mx) mx = v;
      }
      double sum = 0.0;
      for (int64_t e = rowptr[i]; e < rowptr[i + 1]; ++e)
        sum += exp(leaky(tpre[e * H + h]) - mx);
      sum += 1e-16;
      for (int64_t e = rowptr[i]; e < rowptr[i + 1]; ++e) {
        const double a = exp(leaky(tpre[e * H + h]) - mx) / sum;
        alpha[e * H + h] = a;
        for (int64_t c = 0; c < C; ++c) o[h * C + c] += a * (double)hs[col[e] * HC + h * C + c];
      }
    }
    for (int64_t f = 0; f < out_w; ++f) {
      double v;
      if (concat) {
        v = o[f];
      } else {
        v = 0.0;
        for (int64_t h = 0; h < H; ++h) v += o[h * C + f];
        v /= (double)H;
      }
      out[i * out_w + f] = v + (bias ? (double)bias[f] : 0.0);
    }
  }
  free(o);
  free(s);
  free(d);
}

/* Gradient of orc_gat_forward (the chain rule through PyG's softmax, message
 * and attention dot products; grinnder/nn/gat.py:73).  gy = dL/dout.
 * Outputs (double): dhs [E*H*C] (through both x_src and x_dst = Hs[:B]),
 * datt_src [H*C], datt_dst [H*C], dbias [out_w]. */
void orc_gat_backward(int64_t B, int64_t E, const int64_t* rowptr,
                      const int64_t* col, const float* hs, int64_t H, int64_t C,
                      const float* att_src, const float* att_dst,
                      int32_t concat, const double* alpha, const double* tpre,
                      const float* gy, double* dhs, double* datt_src,
                      double* datt_dst, double* dbias) {
  const int64_t HC = H * C;
  const int64_t out_w = concat ? HC : C;
  memset(dhs, 0, sizeof(double) * (size_t)(E * HC));
  memset(datt_src, 0, sizeof(double) * (size_t)HC);
  memset(datt_dst, 0, sizeof(double) * (size_t)HC);
  memset(dbias, 0, sizeof(double) * (size_t)out_w);
  double* ds = (double*)calloc((size_t)(E * H), sizeof(double));
  double* dd = (double*)calloc((size_t)((B > 0 ? B : 1) * H), sizeof(double));
  double* go = (double*)calloc((size_t)HC, sizeof(double));
  for (int64_t i = 0; i < B; ++i) {
    for (int64_t f = 0; f < out_w; ++f) dbias[f] += gy[i * out_w + f];
    for (int64_t h = 0; h < H; ++h)
      for (int64_t c = 0; c < C; ++c)
        go[h * C + c] = concat ? (double)gy[i * out_w + h * C + c]
                               : (double)gy[i * out_w + c] / (double)H;
    for (int64_t h = 0; h < H; ++h) {
      /* d alpha, then the softmax Jacobian-vector product. */
      double csum = 0.0;
      for (int64_t e = rowptr[i]; e < rowptr[i + 1]; ++e) {
        double ga = 0.0;
        for (int64_t c = 0; c < C; ++c) ga += go[h * C + c] * (double)hs[col[e] * HC + h * C + c];
        csum += alpha[e * H + h] * ga;
      }
      for (int64_t e = rowptr[i]; e < rowptr[i + 1]; ++e) {
        const int64_t j = col[e];
        const double a = alpha[e * H + h];
        double ga = 0.0;
        for (int64_t c = 0; c < C; ++c) ga += go[h * C + c] * (double)hs[j * HC + h * C + c];
        const double ge = a * (ga - csum);
        const double gt = ge * (tpre[e * H + h] > 0.0 ? 1.0 : 0.2);
        ds[j * H + h] += gt;
        dd[i * H + h] += gt;
        for (int64_t c = 0; c < C; ++c) dhs[j * HC + h * C + c] += a * go[h * C + c];
      }
    }
  }
  for (int64_t j = 0; j < E; ++j)
    for (int64_t h = 0; h < H; ++h)
      for (int64_t c = 0; c < C; ++c) {
        dhs[j * HC + h * C + c] += ds[j * H + h] * att_src[h * C + c];
        datt_src[h * C + c] += ds[j * H + h] * (double)hs[j * HC + h * C + c];
      }
  for (int64_t i = 0; i < B; ++i)
    for (int64_t h = 0; h < H; ++h)
      for (int64_t c = 0; c < C; ++c) {
        dhs[i * HC + h * C + c] += dd[i * H + h] * att_dst[h * C + c];
        datt_dst[h * C + c] += dd[i * H + h] * (double)hs[i * HC + h * C + c];
      }
  free(go);
  free(ds);
  free(dd);
}

/* Halo gather of csrc/cuda/async_transfer.cu:60-120 (and the Python fallback
 * grinnder/buffer/host.py:314-324): dst = [srcs[pid] | srcs[p][b_p] for p
 * ascending, p != pid].  Returns the number of rows written. */
int64_t orc_gather_partitions(int32_t pid, int32_t num_parts,
                              const float* const* srcs, const int64_t* src_rows,
                              int64_t dim, const int64_t* const* boundaries,
                              const int64_t* boundary_lens, float* dst) {
  int64_t off = 0;
  memcpy(dst, srcs[pid], sizeof(float) * (size_t)(src_rows[pid] * dim));
  off = src_rows[pid];
  for (int32_t p = 0; p < num_parts; ++p) {
    if (p == pid || boundary_lens[p] == 0) continue;
    for (int64_t k = 0; k < boundary_lens[p]; ++k) {
      memcpy(dst + (off + k) * dim, srcs[p] + boundaries[p][k] * dim, sizeof(float) * (size_t)dim);
    }
    off += boundary_lens[p];
  }
  return off;
}

/* Halo-gradient scatter-add of csrc/cuda/async_transfer.cu:122-186: the
 * self block is D2H'd and added to the previous values, then each other
 * partition receives index_put_(accumulate=True) in ascending order,
 * indices in order, in fp32 (the reference's arithmetic type). */
int64_t orc_scatter_partitions(int32_t pid, int32_t num_parts, const float* src,
                               int64_t dim, float* const* dsts,
                               const int64_t* dst_rows,
                               const int64_t* const* boundaries,
                               const int64_t* boundary_lens) {
  for (int64_t i = 0; i < dst_rows[pid] * dim; ++i) {
    const float prev = dsts[pid][i];
    dsts[pid][i] = src[i] + prev;
  }
  int64_t off = dst_rows[pid];
  for (int32_t p = 0; p < num_parts; ++p) {
    if (p == pid || boundary_lens[p] == 0) continue;
    for (int64_t k = 0; k < boundary_lens[p]; ++k) {
      float* row = dsts[p] + boundaries[p][k] * dim;
      const float* g = src + (off + k) * dim;
      for (int64_t f = 0; f < dim; ++f) row[f] = row[f] + g[f];
    }
    off += boundary_lens[p];
  }
  return off;
}
