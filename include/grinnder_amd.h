/*
 * grinnder_amd.h — C ABI of the MI355X (gfx950) partitioned-GNN-layer library
 * (libgrinnder_amd.so).
 *
 * Conventions shared by every entry point:
 *   - Returns int status: 0 on success, a negative GR_E* code on failure.
 *     The message of the most recent failure on the calling thread is
 *     available from gr_last_error().  Nothing is launched or copied when a
 *     precondition check fails (checks run before the first enqueue).
 *   - Plain pointers and int64 extents only.  "stream" is a hipStream_t
 *     passed as void* (NULL means the legacy default stream).
 *   - The library never frees caller memory.  Device work is enqueued on the
 *     given stream and is asynchronous unless stated otherwise.
 *   - Index arrays crossing the boundary in the reference's layout are int64
 *     (rowptr, col, boundaries); device-resident index arrays produced by the
 *     preparation calls below are int32.
 *
 * Reference interfaces replaced (paths relative to the GriNNder repository):
 *   csrc/grinnder_ops.cpp:7-34          pybind op table of grinnder._C
 *   csrc/cuda/async_transfer.cu:17-186  h2d/d2h copies, gather/scatter
 *   csrc/cpu/subgraph.cpp:8-114         build_subgraph
 *   grinnder/data/partition.py:178-228  _build_partition_subgraph (boundaries)
 *   torch_sparse spmm_sum / csr2csc, called through PyG GCNConv
 *       (grinnder/nn/gcn.py:53-56,65; grinnder/engine/trainer.py:288-302)
 *   PyG GATConv attention + softmax + aggregation
 *       (grinnder/nn/gat.py:54-61,69-78)
 */
#ifndef GRINNDER_AMD_H
#define GRINNDER_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------------ */
/* Status                                                                    */
/* ------------------------------------------------------------------------ */

#define GR_OK 0
#define GR_EINVAL (-1)   /* bad argument / size mismatch / index out of range */
#define GR_EHIP (-2)     /* HIP runtime call failed */
#define GR_ENOMEM (-3)   /* host allocation failed */
#define GR_EUNSUP (-4)   /* shape or dtype not supported */

/* Activations of the LayerNorm epilogues. */
#define GR_ACT_RELU 0    /* max(y, 0): GCN.forward_layer, grinnder/nn/gcn.py:64-72 */
#define GR_ACT_ELU 1     /* y > 0 ? y : exp(y) - 1: GAT.forward_layer, gat.py:74-78 */

/* Message of the last failure on this thread ("" if none). */
const char* gr_last_error(void);

/* ABI version of this library (major * 100 + minor). */
int gr_abi_version(void);

/* Hex SHA-256 of the sources and device flags this library was built from
 * (build identity, no reference counterpart): a loader compares it with the
 * sources beside it and refuses a stale binary. */
const char* gr_source_hash(void);

/* ------------------------------------------------------------------------ */
/* Host <-> device transfers (grinnder._C transfer ops)                      */
/* ------------------------------------------------------------------------ */

/* Replaces h2d_copy_async, csrc/cuda/async_transfer.cu:40-58.
 * Copies nbytes from host memory to device memory on `stream`.  Pinned host
 * memory gives a truly asynchronous DMA; pageable memory is accepted and is
 * staged by the runtime.  The copy is recorded in the H2D completion queue
 * consumed by gr_h2d_synchronize(). */
int gr_h2d_copy_async(const void* src_host, void* dst_dev, int64_t nbytes,
                      void* stream);

/* Replaces d2h_copy_async, csrc/cuda/async_transfer.cu:20-38. */
int gr_d2h_copy_async(const void* src_dev, void* dst_host, int64_t nbytes,
                      void* stream);

/* Replaces h2d_synchronize / d2h_synchronize,
 * csrc/cuda/async_transfer.cu:17-18 and csrc/thread_pool.h:65-70: waits
 * for the OLDEST queued operation of that direction (FIFO, one entry per
 * call) and returns its error, if any.  Returns 0 when the queue is empty. */
int gr_h2d_synchronize(void);
int gr_d2h_synchronize(void);

/* Replaces gather_partitions, csrc/cuda/async_transfer.cu:60-120.
 * dst (device, dst_rows x row_bytes) receives
 *   [ srcs[pid] (all src_rows[pid] rows)
 *   | srcs[p][boundaries[p][k]] for p = 0..num_parts-1, p != pid,
 *     boundary_lens[p] > 0, k in order ].
 * srcs are host partition buffers (pinned: rows are read by a device kernel
 * over PCIe; pageable: rows are gathered by host threads into a pinned
 * staging slot and copied by DMA).  boundaries are host int64 arrays
 * (entries for p == pid, NULL pointers and zero lengths are skipped).
 * Errors (GR_EINVAL) if the rows do not add up to dst_rows or if a boundary
 * index is out of range — checked before anything is enqueued. */
int gr_gather_partitions(int32_t pid, int32_t num_parts,
                         const void* const* srcs, const int64_t* src_rows,
                         void* dst, int64_t dst_rows, int64_t row_bytes,
                         const int64_t* const* boundaries,
                         const int64_t* boundary_lens, void* stream);

/* Replaces scatter_partitions, csrc/cuda/async_transfer.cu:122-186.
 * fp32 accumulate of src (device, src_rows x dim) into host partitions:
 *   dsts[pid][r]           += src[r]            r < dst_rows[pid]
 *   dsts[p][boundaries[p][k]] += src[off + k]   p ascending, p != pid
 * Pinned destinations are updated by one device kernel (read-add-write over
 * PCIe, asynchronous on `stream`); pageable destinations are updated on the
 * host after a D2H copy (synchronous).  Repeated indices inside one boundary
 * are accumulated sequentially in index order, like index_put_(accumulate).
 * Errors (GR_EINVAL) on row-count mismatch or out-of-range index. */
int gr_scatter_partitions(int32_t pid, int32_t num_parts, const float* src,
                          int64_t src_rows, int64_t dim, float* const* dsts,
                          const int64_t* dst_rows,
                          const int64_t* const* boundaries,
                          const int64_t* boundary_lens, void* stream);

/* Exact-size pinned (page-locked, device-mapped) host allocation for the
 * host partition buffers (the reference allocates them with torch, optionally
 * pinned, grinnder/buffer/host.py:27-45).  GR_ENOMEM if the driver refuses;
 * callers then fall back to pageable memory as the reference does.
 * gr_host_free releases a pointer returned by gr_host_alloc (NULL is a no-op). */
int gr_host_alloc(int64_t nbytes, void** out);
int gr_host_free(void* p);

/* ------------------------------------------------------------------------ */
/* Partition bookkeeping (host, bit-exact)                                   */
/* ------------------------------------------------------------------------ */

/* Replaces build_subgraph, csrc/cpu/subgraph.cpp:8-114 (int64 only, as the
 * reference reads data_ptr<int64_t>).  Two calls:
 *   1) out_col == NULL: writes *out_nnz and *out_num_nodes (seeds + newly
 *      discovered neighbours) and returns.
 *   2) with out_rowptr [n_idx+1 or out_num_nodes+1 if !bipartite],
 *      out_col [nnz], out_value [nnz] (NULL if value == NULL) and
 *      out_n_id [num_nodes]: fills them.
 * Seeds get ids [0, n_idx); unseen neighbours get n_idx, n_idx+1, ... in
 * first-seen order of a row-major scan.  value is copied as raw
 * value_elem_size-byte elements. */
int gr_build_subgraph(const int64_t* rowptr, const int64_t* col,
                      const void* value, int64_t value_elem_size,
                      int64_t num_rows, const int64_t* idx, int64_t n_idx,
                      int32_t bipartite, int64_t* out_rowptr, int64_t* out_col,
                      void* out_value, int64_t* out_n_id, int64_t* out_nnz,
                      int64_t* out_num_nodes);

/* Replaces the boundary split and column remap of _build_partition_subgraph,
 * grinnder/data/partition.py:195-225.  Given n_id[batch_size:] (global ids of
 * the halo in discovery order) and the partition pointer ptr[num_parts+1]:
 *   boundary_lens[p] = number of halo nodes owned by p (0 for p == pid),
 *   boundary_flat = concatenation over p ascending of (n_id - ptr[p]) in
 *                   discovery order (length n_halo),
 *   col (in place, length nnz): halo columns c >= batch_size are remapped to
 *       batch_size + (position of c's node in boundary_flat).
 * Errors if a halo node lies in partition pid or outside [0, ptr[P]). */
int gr_partition_boundaries(int32_t pid, int32_t num_parts, const int64_t* ptr,
                            int64_t batch_size, const int64_t* halo_ids,
                            int64_t n_halo, int64_t* col, int64_t nnz,
                            int64_t* boundary_flat, int64_t* boundary_lens);

/* Graph partitioner (replaces the grdpart GrinnderPartitioner / Spinner call
 * of build_partitioned_graph, grinnder/data/partition.py:285-300; grdpart is
 * not available, so this is the library's own algorithm): breadth-first
 * visit order (bfs_order != 0; else id order) of the undirected graph, then
 * linear deterministic greedy assignment with partition capacity
 * ceil(capacity * n / num_parts).  Outputs perm [n] (new position -> node
 * id; nodes grouped by partition, visit order inside a partition) and
 * ptr [num_parts + 1] (partition p = perm[ptr[p]:ptr[p+1]]). */
int gr_partition_graph(const int64_t* src, const int64_t* dst, int64_t m,
                       int64_t n, int32_t num_parts, double capacity,
                       int32_t bfs_order, int64_t* perm, int64_t* ptr);

/* ------------------------------------------------------------------------ */
/* Aggregation-side preparation (host, done once per partition adjacency)    */
/* ------------------------------------------------------------------------ */

/* Deterministic CSR -> CSC transpose of a rows x cols matrix (no reference
 * counterpart in the repository: replaces torch_sparse csr2csc, which the
 * reference's SparseTensor recomputes on every backward,
 * grinnder/engine/trainer.py:288-302).  Within each column the entries are
 * ordered by (row, CSR position) — a stable transpose.
 *   colptr [cols+1] int64, row_idx [nnz] int32, val_t [nnz] f32 (skipped if
 *   val or val_t is NULL), perm [nnz] int32 = CSR position of each CSC entry
 *   (skipped if NULL). */
int gr_csr_transpose(const int64_t* rowptr, const int64_t* col,
                     const float* val, int64_t rows, int64_t cols,
                     int64_t* colptr, int32_t* row_idx, float* val_t,
                     int32_t* perm);

/* Work plan for the row-parallel aggregation kernels.  A row whose length
 * exceeds seg_len is split into ceil(len / seg_len) units whose partial sums
 * go to a workspace and are reduced in unit order by a second kernel, so the
 * result is deterministic.  Units of split rows come first (they start
 * early), then single-unit rows in row order.
 *   units [n_units*4] int32 = (row, edge_begin, edge_end, slot or -1)
 *   fixups [n_fix*3] int32   = (row, first_slot, n_slots)
 * Two calls: with units == NULL only the counts are written. */
int gr_spmm_plan(const int64_t* rowptr, int64_t rows, int32_t seg_len,
                 int32_t* units, int64_t* n_units, int32_t* fixups,
                 int64_t* n_fix, int64_t* n_slots);

/* gr_spmm_plan with the whole rows ordered block by block: block k is rows
 * [block_ptr[k], block_ptr[k+1]) (block_ptr[0] = 0, block_ptr[n_blocks] =
 * rows), and within a block by length class as gr_spmm_plan orders them; the
 * split rows' units still come first.  No counterpart in the reference: the
 * plan of an adjacency that stacks several partitions' rows (one pass for all
 * of them), so that each partition's rows still run together and its gathered
 * source rows stay in cache as in a pass of its own. */
int gr_spmm_plan_blocked(const int64_t* rowptr, int64_t rows, int32_t seg_len,
                         const int64_t* block_ptr, int64_t n_blocks, int32_t* units,
                         int64_t* n_units, int32_t* fixups, int64_t* n_fix,
                         int64_t* n_slots);

/* ------------------------------------------------------------------------ */
/* GCN aggregation (device)                                                  */
/* ------------------------------------------------------------------------ */

/* Y[r, :D] = sum_e val[e] * X[idx[e], :D] (+ bias[:D] if bias != NULL) for
 * every row r of the plan, fp32, deterministic (no atomics).  Replaces the
 * torch_sparse spmm_sum forward of PyG GCNConv (grinnder/nn/gcn.py:53-56,65;
 * adjacency from grinnder/engine/trainer.py:288-302) when called with the
 * CSR plan, and its backward dZ = A^T G when called with the CSC plan of
 * gr_csr_transpose.  Rows with no edges get bias (or 0).
 *   X: ldx-strided device rows (ldx >= D), Y: ldy-strided (ldy >= D).
 *   workspace: n_slots * D floats (may be NULL when n_slots == 0). */
int gr_gcn_aggregate(const int32_t* units, int64_t n_units,
                     const int32_t* fixups, int64_t n_fix,
                     const int32_t* idx, const float* val, const float* x,
                     int64_t ldx, float* y, int64_t ldy, const float* bias,
                     int64_t rows, int64_t dim, float* workspace,
                     int64_t n_slots, void* stream);

/* Floats of the per-GPU scratch behind gr_gcn_aggregate_noalloc (32 MiB). */
#define GR_NOALLOC_SCRATCH_FLOATS (8LL << 20)

/* No counterpart in the reference.  gr_gcn_aggregate for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc): the same kernels and results, with the
 * split-row partial sums in a static per-GPU scratch of
 * GR_NOALLOC_SCRATCH_FLOATS floats instead of a caller workspace.  Rejects
 * n_slots * dim above that maximum (use gr_gcn_aggregate then).  Allocates
 * nothing; the scratch address is looked up once per GPU on the first call
 * there.  Every call on one GPU shares that GPU's scratch: calls that
 * overlap on one GPU (two streams, two threads) race.  No clearing is
 * needed between calls: each call writes every slot element it reads. */
int gr_gcn_aggregate_noalloc(const int32_t* units, int64_t n_units,
                             const int32_t* fixups, int64_t n_fix,
                             const int32_t* idx, const float* val, const float* x,
                             int64_t ldx, float* y, int64_t ldy, const float* bias,
                             int64_t rows, int64_t dim, int64_t n_slots, void* stream);

/* No counterpart in the reference: gr_gcn_aggregate with an output row map,
 * for the backward of projected layers (grinnder_amd/engine/trainer.py),
 * which add the gradient of a partition's gathered rows straight into the
 * layer's dZ instead of materialising it and scattering it afterwards:
 *   y[out_rows[r]] += sum_e val[e] * X[idx[e]]   for each plan row r.
 * out_rows must be distinct within one call (each y row has one writer, so
 * the result is deterministic); the sum is formed exactly as by
 * gr_gcn_aggregate and then added once.  No bias. */
int gr_gcn_aggregate_into(const int32_t* units, int64_t n_units,
                          const int32_t* fixups, int64_t n_fix,
                          const int32_t* idx, const float* val, const float* x,
                          int64_t ldx, const int32_t* out_rows, float* y,
                          int64_t ldy, int64_t rows, int64_t dim,
                          float* workspace, int64_t n_slots, void* stream);

/* No counterpart in the reference: the row gather from an HBM-resident
 * matrix that the trainer's projected and gathered layers do on the device
 * where the reference gathers halo rows from host buffers
 * (gather_partitions, csrc/cuda/async_transfer.cu:60-120):
 *   y[r][j] = x[rows[r]][j]   for r < n, j < dim,
 * x [x_rows, dim] with row stride ldx, y [n, dim] with row stride ldy, rows
 * device int64; a row id outside [0, x_rows) gives a zero row. */
int gr_gather_rows(const float* x, int64_t x_rows, int64_t ldx, const int64_t* rows,
                   int64_t n, int64_t dim, float* y, int64_t ldy, void* stream);

/* No counterpart in the reference: the backward of a row gather from an
 * HBM-resident matrix (the trainer's projected and gathered layers, which
 * take a partition's rows on the device where the reference gathers them
 * from host buffers and scatters their gradient back with
 * scatter_partitions, csrc/cuda/async_transfer.cu:122-186):
 *   y[rows[r]][j] += x[r][j]   for r < n, j < dim,
 * x [n, dim] with row stride ldx, y [y_rows, dim] with row stride ldy, rows
 * device int64.  rows must be distinct within one call (each y row has one
 * writer: no atomics, deterministic, the same as adding the rows one at a
 * time); a row id outside [0, y_rows) is skipped. */
int gr_scatter_add_rows(const float* x, int64_t n, int64_t dim, int64_t ldx,
                        const int64_t* rows, float* y, int64_t y_rows, int64_t ldy,
                        void* stream);

/* Fused GCN layer epilogue (bias + LayerNorm + ReLU of grinnder/nn/gcn.py:
 * 64-72, LayerNorm of torch with biased variance and eps):
 *   h[r]   = sum_e val[e] * X[idx[e]] + bias       (written, kept for backward)
 *   out[r] = max((h[r] - mean_r) * rstd_r * gamma + beta, 0)
 *   mean[r], rstd[r] = 1 / sqrt(var_r + eps)
 * Same plan / workspace conventions as gr_gcn_aggregate; h and out are
 * dense [rows, dim] (dim <= 1024).  No reference counterpart as one call: it
 * fuses PyG GCNConv's aggregation with the LayerNorm and ReLU that follow it. */
int gr_gcn_aggregate_ln_relu(const int32_t* units, int64_t n_units,
                             const int32_t* fixups, int64_t n_fix,
                             const int32_t* idx, const float* val,
                             const float* x, int64_t ldx, const float* bias,
                             const float* gamma, const float* beta, float eps,
                             int64_t rows, int64_t dim, float* h, float* out,
                             float* mean, float* rstd, float* workspace,
                             int64_t n_slots, void* stream);

/* Backward of out = act(LayerNorm(h)) (act = GR_ACT_RELU or GR_ACT_ELU) given
 * g = dL/dout: writes
 * gh = dL/dh [rows, dim], dgamma [dim], dbeta [dim] and, when dbias != NULL,
 * dbias = sum_rows gh (the gradient of a bias added before the LayerNorm)
 * (deterministic: per-wavefront partials reduced in order).  When rowdot !=
 * NULL it also writes rowdot[r] = sum_f gh[r, f] * (h[r, f] - shift[f])
 * (shift NULL: 0): with h = o + b and shift = b this is <dL/do_r, o_r>, the
 * c_i of the attention backward of a GATConv whose output feeds the
 * LayerNorm (grinnder/nn/gat.py:74-78), formed while gh is in registers.
 * workspace: at least (k * 4 + 1) * dim floats with k = 3 when dbias != NULL,
 * else 2; up to (k * 8192 + 1) * dim are used. */
int gr_ln_act_backward(const float* g, const float* h, const float* mean,
                       const float* rstd, const float* gamma, const float* beta,
                       int32_t act, int64_t rows, int64_t dim, float* gh,
                       float* dgamma, float* dbeta, float* dbias, const float* shift,
                       float* rowdot, float* workspace, int64_t workspace_floats,
                       void* stream);

/* gr_ln_act_backward with g = dL/dout formed inside the pass as g = dz B:
 * dz [rows, k] (row stride ldz, 16-byte aligned; k <= 64 and ldz multiples
 * of 4), B [k, dim] row-major, dim in {64, 128, 192, 256}.  In the reference
 * model this g is the input gradient dZ W of the next layer's Linear
 * (grinnder/nn/gcn.py:53-56, torch's Linear backward), which the reference
 * writes out and the LayerNorm/ReLU backward (grinnder/nn/gcn.py:64-73,
 * torch's LayerNorm and ReLU backward) reads back; here the product stays
 * in the matrix cores' accumulators.  Outputs, shift/rowdot and workspace
 * as gr_ln_act_backward; act = GR_ACT_RELU or GR_ACT_ELU. */
int gr_ln_act_backward_product(const float* dz, int64_t ldz, int64_t k, const float* b,
                               const float* h, const float* mean, const float* rstd,
                               const float* gamma, const float* beta, int32_t act,
                               int64_t rows, int64_t dim, float* gh, float* dgamma,
                               float* dbeta, float* dbias, const float* shift,
                               float* rowdot, float* workspace, int64_t workspace_floats,
                               void* stream);

/* Column sums out[f] = sum_i X[i, f] (w == NULL), or weighted sums
 * out[f] = sum_i w[i * ldw + f / group] * X[i, f] (fp32, deterministic: fixed
 * row chunks, partials reduced in chunk order); with xrows != NULL, row i of
 * X is row xrows[i] of x.  Replaces the bias gradient of PyG GCNConv's /
 * GATConv's "+ bias" (grinnder/nn/gcn.py:53-56, grinnder/nn/gat.py:54-61)
 * and, weighted by ds / dd with group = C, GATConv's attention-vector
 * gradients d att_src[h] = sum_j ds[j,h] Hs[j,h,:].
 * workspace: at least D floats (up to 4096 * D are used for parallelism). */
int gr_column_sum(const float* x, int64_t rows, int64_t dim, int64_t ldx,
                  const int32_t* xrows, const float* w, int64_t ldw, int64_t group,
                  float* out, float* workspace, int64_t workspace_floats, void* stream);

/* Dense form of the fused epilogue, for a layer whose product Z was formed
 * outside the aggregation (aggregate-first GCN: Z = (A X) W^T; GAT output):
 *   h = Z + bias, out = act(LayerNorm(h)), mean, rstd
 * with the same expressions as gr_gcn_aggregate_ln_relu, so gr_ln_act_backward
 * is its backward.  Z is ldz-strided; h, out dense [rows, dim]; h may be Z
 * itself when ldz == dim.  Replaces the LayerNorm + ReLU that follow the conv
 * in grinnder/nn/gcn.py:64-72 (act = GR_ACT_RELU) and the LayerNorm + ELU of
 * grinnder/nn/gat.py:74-78 (act = GR_ACT_ELU). */
int gr_bias_ln_act(const float* z, int64_t ldz, const float* bias,
                   const float* gamma, const float* beta, float eps, int32_t act,
                   int64_t rows, int64_t dim, float* h, float* out, float* mean,
                   float* rstd, void* stream);

/* ------------------------------------------------------------------------ */
/* Loss and accuracy                                                         */
/* ------------------------------------------------------------------------ */

/* Masked softmax cross-entropy and argmax accuracy of a partition's logits
 * [rows, classes] (ld-strided), one pass.  mask[r]: bit 0 train, bit 1 val,
 * bit 2 test; labels int64.  Replaces the per-partition
 * F.cross_entropy(out[train], y[train], reduction="sum") of
 * grinnder/engine/trainer.py:709-721 (mean = 0) and the fast path's
 * reduction="mean" (trainer.py:430-453, mean = 1), and the argmax accuracy of
 * compute_micro_f1 (grinnder/utils.py:24-44) for val and test rows.
 * Outputs (device): *loss (fp32; 0 when there are no train rows), stats[6] =
 * {train rows, val correct, val rows, test correct, test rows, rows with a
 * label outside [0, classes)} (the caller raises on the last), lse[r] =
 * log-sum-exp of row r (may be NULL), and, when grad != NULL, the gradient of
 * the train-row nll sum, grad[r, c] = softmax(x_r)_c - [c == y_r] on train
 * rows and 0 elsewhere (ldg-strided); the caller scales it by dL/dloss (and
 * 1 / train rows for the mean).  Sums are reduced in a fixed order in double.
 * workspace: 7 * max(1, ceil(rows / 256)) doubles. */
int gr_xent_forward(const float* logits, int64_t ld, int64_t rows,
                    int64_t classes, const int64_t* labels, const uint8_t* mask,
                    int32_t mean, float* lse, float* grad, int64_t ldg,
                    float* loss, int64_t* stats, double* workspace,
                    int64_t workspace_doubles, void* stream);

/* ------------------------------------------------------------------------ */
/* Dense transform                                                           */
/* ------------------------------------------------------------------------ */

/* C[M, N] = A^T B (+ beta * C) with A [K, M] (lda-strided rows) and B [K, N]
 * (ldb-strided rows), fp32 on the matrix cores, split over K into `splits`
 * chunks whose partial tiles are summed in chunk order (deterministic).  This
 * is the weight gradient dW = dZ^T X of the conv's dense transform (the
 * Linear inside PyG GCNConv / GATConv of grinnder/nn/gcn.py:53-56 and
 * grinnder/nn/gat.py:54-61), whose K is the partition's row count.
 * gr_gemm_tn_workspace returns the default split count and the workspace size
 * in floats (splits * M * N) for a shape. */
int gr_gemm_tn_workspace(int64_t m, int64_t n, int64_t k, int64_t* splits,
                         int64_t* workspace_floats);
int gr_gemm_tn(const float* a, int64_t lda, const float* b, int64_t ldb,
               int64_t m, int64_t n, int64_t k, float beta, float* c,
               float* workspace, int64_t workspace_floats, int64_t splits,
               void* stream);

/* C[M, N] = A B^T (+ bias[N]) with A [M, K], B [N, K] and C [M, N] row-major
 * (lda-, ldb-, ldc-strided rows), fp32 on the matrix cores; each element is
 * one workgroup's sum over K (no split, deterministic).  With B = W [out, in]
 * this is the forward x W^T + b of the conv's dense transform (the Linear of
 * PyG GCNConv / GATConv, grinnder/nn/gcn.py:53-56, grinnder/nn/gat.py:54-61);
 * with B = W^T it is the input gradient dx = dy W.  bias may be NULL; m may be
 * 0 (nothing to do). */
int gr_gemm_nt(const float* a, int64_t lda, const float* b, int64_t ldb,
               int64_t m, int64_t n, int64_t k, const float* bias, float* c,
               int64_t ldc, void* stream);

/* Dense layer transform with the LayerNorm epilogue in the GEMM accumulators:
 *   h = x W^T + bias, out = act(LayerNorm(h; gamma, beta, eps)), mean, rstd
 * for x [rows, din] (ldx-strided), wt = W^T [din, dout] row-major (the
 * transposed [dout, din] weight), dout a multiple of 16 in [16, 256]; h, out
 * dense [rows, dout]; gamma, beta, h and out 16-byte aligned.  fp32 on the matrix cores.  The
 * epilogue's expressions are those of gr_bias_ln_act, so gr_ln_act_backward is
 * its backward.  A row's result does not depend on the row count (the
 * large-row form keeps W in LDS and sums in the same order, same bits).
 * Replaces the Linear of an aggregate-first GCNConv (PyG GCNConv's lin,
 * grinnder/nn/gcn.py:53-56) followed by the LayerNorm and ReLU of
 * grinnder/nn/gcn.py:64-72. */
int gr_linear_ln_act(const float* x, int64_t ldx, int64_t rows, int64_t din,
                     const float* wt, int64_t dout, const float* bias,
                     const float* gamma, const float* beta, float eps, int32_t act,
                     float* h, float* out, float* mean, float* rstd, void* stream);

/* ------------------------------------------------------------------------ */
/* GAT attention (device)                                                    */
/*                                                                           */
/* Replace PyG GATConv's attention path as the reference calls it            */
/* (grinnder/nn/gat.py:54-61 heads/concat/add_self_loops=False; :69-78       */
/* bipartite input (x, x[:B])): logits s_j + d_i, LeakyReLU(0.2), edge       */
/* softmax with max subtraction and +1e-16 in the denominator, and the       */
/* alpha-weighted sum of source rows.  Because the reference applies one     */
/* shared lin to x and to x[:B], destination features are the first B rows  */
/* of Hs.  Layout: Hs [E, H*C] (row stride ldh), s [E,H], d/m/den [B,H].     */
/* ------------------------------------------------------------------------ */

/* s[j,h] = <Hs[j,h,:], att_src[h,:]> for j < n_src and
 * d[i,h] = <Hs[i,h,:], att_dst[h,:]> for i < n_dst. */
int gr_gat_scores(const float* hs, int64_t ldh, int64_t n_src, int64_t n_dst,
                  int64_t heads, int64_t channels, const float* att_src,
                  const float* att_dst, float* s, float* d, void* stream);

/* out[r,h] = <a[r, h*C:(h+1)*C], b[r, h*C:(h+1)*C]> for r < rows: the
 * backward's cdot_i = <go_i, O_i> per head (PyG GATConv backward through
 * softmax, grinnder/nn/gat.py:54-61). */
int gr_gat_row_dot(const float* a, int64_t lda, const float* b, int64_t ldb,
                   int64_t rows, int64_t heads, int64_t channels, float* out,
                   void* stream);

/* Edge softmax over each CSR row: m[i,h] = max_j LeakyReLU(s_j + d_i),
 * den[i,h] = sum exp(v - m) + 1e-16 (rows without edges: m = 0, den = 1) and
 * the attention weights alpha[e,h] = exp(v_e - m) / den [nnz, H] (CSR order).
 * Uses the CSR plan of gr_spmm_plan; workspace: n_slots * 2H floats. */
int gr_gat_softmax_stats(const int32_t* units, int64_t n_units,
                         const int32_t* fixups, int64_t n_fix,
                         const int32_t* idx, const float* s, const float* d,
                         int64_t heads, float* m, float* den, float* alpha,
                         float* workspace, int64_t n_slots, void* stream);

/* O[i,:] = sum_e alpha[e, h] Hs[idx[e],:] (alpha from gr_gat_softmax_stats),
 * written to o [n_dst, H*C]; when y is not NULL also Y = O + bias (bias may be
 * NULL) with row stride ldy.  workspace: n_slots * H*C floats. */
int gr_gat_aggregate(const int32_t* units, int64_t n_units,
                     const int32_t* fixups, int64_t n_fix, const int32_t* idx,
                     const float* hs, int64_t ldh, const float* alpha,
                     int64_t n_dst, int64_t heads, int64_t channels,
                     const float* bias, float* o, float* y, int64_t ldy,
                     float* workspace, int64_t n_slots, void* stream);

/* The whole attention forward after the scores: edge softmax (m, den, alpha
 * as gr_gat_softmax_stats) and O = sum_e alpha Hs[idx[e]] into o [n_dst, H*C],
 * plus Y = O + bias into y when y is not NULL (bias may be NULL).  One head
 * runs as one fused pass per plan unit (the softmax statistics, the weights
 * and the weighted row sums together); whole rows give the same bits as
 * gr_gat_softmax_stats followed by gr_gat_aggregate.  Several heads run those
 * two.  units / fixups as gr_spmm_plan lays them out (split rows' units first,
 * unit k holding slot k).
 * workspace: ws_floats >= n_slots * (round_up(H*C, 4) + round_up(2H, 4)).
 * alpha may be NULL with one head (rows of at most 256 vectors): it is then
 * not stored (gr_gat_backward_src_h1 recomputes it).
 * Replaces the attention / softmax / propagate sequence of PyG GATConv as
 * grinnder/nn/gat.py:54-61,73 calls it. */
int gr_gat_forward(const int32_t* units, int64_t n_units, const int32_t* fixups,
                   int64_t n_fix, const int32_t* idx, const float* hs, int64_t ldh,
                   const float* s, const float* d, int64_t n_dst, int64_t heads,
                   int64_t channels, const float* bias, float* m, float* den,
                   float* alpha, float* o, float* y, int64_t ldy, float* workspace,
                   int64_t ws_floats, int64_t n_slots, void* stream);

/* One head of C channels (a multiple of 4 in 132..1024): gr_gat_forward with
 * the GAT model's epilogue after the conv (bias, LayerNorm(gamma, beta,
 * eps) and act = GR_ACT_ELU or GR_ACT_RELU; grinnder/nn/gat.py:74-78) in the
 * same pass: each row writes h = O + bias [n_dst, C], out = act(LN(h)) (row
 * stride ldo), mean and rstd [n_dst], and m, den as gr_gat_forward; neither
 * O nor alpha.  The row statistics and output are formed as gr_bias_ln_act
 * forms them from the same h (bit for bit for whole rows).
 * workspace: n_slots * (C + 4) floats.  No counterpart in the reference: it
 * fuses the conv and the LayerNorm that follows it. */
int gr_gat_forward_ln(const int32_t* units, int64_t n_units, const int32_t* fixups,
                      int64_t n_fix, const int32_t* idx, const float* hs, int64_t ldh,
                      const float* s, const float* d, int64_t n_dst, int64_t channels,
                      const float* bias, const float* gamma, const float* beta, float eps,
                      int32_t act, float* m, float* den, float* h, float* out, int64_t ldo,
                      float* mean, float* rstd, float* workspace, int64_t ws_floats,
                      int64_t n_slots, void* stream);

/* Backward over source rows j (CSC plan, row_idx/perm from
 * gr_csr_transpose; alpha [nnz, H] in CSR order from gr_gat_softmax_stats).
 * go = dL/dO [B, H*C]; cdot[i,h] = <go_i,h, O_i,h>.
 * With g_e = alpha (<go_i, Hs_j> - cdot_i) and g_t = g_e * (t > 0 ? 1 : 0.2),
 * writes dhs [E, H*C] = sum_i alpha_ij go_i + ds_j * att_src,
 * ds [E,H] = sum_i g_t,ij and gt [nnz,H] (CSR order) = g_e * (t > 0 ? 0 : -0.8),
 * the per-edge part of dd_i = sum_j g_t,ij left after the exact softmax
 * shift-invariance identity sum_j g_e,ij = cdot_i * 1e-16 / den_i.
 * workspace: n_slots * (round_up(H*C, 4) + round_up(H, 4)) floats. */
int gr_gat_backward_src(const int32_t* units, int64_t n_units,
                        const int32_t* fixups, int64_t n_fix,
                        const int32_t* row_idx, const int32_t* perm,
                        const float* hs, int64_t ldh, const float* go,
                        const float* s, const float* d, const float* alpha,
                        const float* cdot,
                        const float* att_src, int64_t heads, int64_t channels,
                        float* dhs, float* ds, float* gt, float* workspace,
                        int64_t n_slots, void* stream);

/* gr_gat_backward_src for one head of C channels (a multiple of 4 in
 * 68..1024) read in place: source column j's rows of Hs and s are row
 * src_rows[j] of hs ([N, ldh]) and s ([N]), matrices of all partitions' rows,
 * and dHs_j is added into row src_rows[j] of dz ([N, C], dense) instead of
 * being written (the src_rows of one partition are distinct).  Replaces the
 * gather of the partition's rows of lin(x) before PyG GATConv's attention
 * (grinnder/nn/gat.py:72-73) and the scatter of their gradient after it; ds
 * and gt stay per partition.  workspace as gr_gat_backward_src.
 * att_part (optional, 16-byte aligned, att_rows x C floats): the pass also
 * forms the attention-vector gradient sum_j ds_j Hs_j (PyG GATConv's
 * att_src gradient) while Hs_j is in registers: *att_waves (> 0) rows of
 * att_part get per-wavefront partial sums, whose column sums taken in row
 * order (gr_column_sum) are that gradient.  att_part NULL: att_rows and
 * att_waves are ignored. */
int gr_gat_backward_src_into(const int32_t* units, int64_t n_units,
                             const int32_t* fixups, int64_t n_fix,
                             const int32_t* row_idx, const int32_t* perm,
                             const float* hs, int64_t ldh, const int32_t* src_rows,
                             const float* go, const float* s, const float* d,
                             const float* alpha, const float* cdot,
                             const float* att_src, int64_t heads, int64_t channels,
                             float* dz, float* ds, float* gt, float* workspace,
                             int64_t n_slots, float* att_part, int64_t att_rows,
                             int64_t* att_waves, void* stream);

/* One head: the destination records rec[i] = (d_i, m_i, den_i, cdot_i),
 * [n_dst, 4] floats (16-byte aligned), from the forward's logit half d, row
 * max m and denominator den and the backward's cdot, for
 * gr_gat_backward_src_h1.  No counterpart in the reference: it packs what
 * PyG GATConv's autograd keeps per destination row into one 16-byte load. */
int gr_gat_dst_record(const float* d, const float* m, const float* den,
                      const float* cdot, int64_t n_dst, float* rec, void* stream);

/* gr_gat_backward_src (src_rows NULL: dhs [E, C] written) or
 * gr_gat_backward_src_into (src_rows given: dHs added into dhs = dz, with
 * the optional att_part partial sums) for one head, with the destination
 * records of gr_gat_dst_record in place of alpha, d and cdot: each edge
 * recomputes alpha_ij = exp(LeakyReLU(s_j + d_i) - m_i) / den_i (for a whole
 * row the forward's own value), so gr_gat_forward may run with alpha NULL.
 * The same outputs (ds, gt, workspace) as those entries; C at most 1024
 * (at most 256 when the rows are not 16-byte aligned).  Replaces the same
 * PyG GATConv backward (grinnder/nn/gat.py:54-61,73). */
int gr_gat_backward_src_h1(const int32_t* units, int64_t n_units,
                           const int32_t* fixups, int64_t n_fix,
                           const int32_t* row_idx, const int32_t* perm,
                           const float* hs, int64_t ldh, const int32_t* src_rows,
                           const float* go, const float* s, const float* rec,
                           const float* att_src, int64_t channels, float* dhs,
                           float* ds, float* gt, float* workspace, int64_t n_slots,
                           float* att_part, int64_t att_rows, int64_t* att_waves,
                           void* stream);

/* The packed source lines of gr_gat_narrow_forward, with the logit halves,
 * formed once for rows that several passes read (the projected matrix of a
 * layer): zx [n_src, 32] = [Hs_j (C) | 0 .. | 24: s_j | 0 ..], s [n_src] and
 * d [n_dst], s and d as gr_gat_scores forms them (bit for bit at these
 * widths).  The logits of PyG's GATConv (grinnder/nn/gat.py:69-72). */
int gr_gat_narrow_pack(const float* hs, int64_t ldh, int64_t n_src, int64_t n_dst,
                       int64_t channels, const float* att_src, const float* att_dst,
                       float* zx, float* s, float* d, void* stream);

/* Narrow one-head attention (C channels, a multiple of 4 up to 24): the
 * forward of gr_gat_forward (PyG GATConv as grinnder/nn/gat.py:54-61,69-78
 * calls it) with every edge reading one 128-byte packed line.
 *   zx [n_src, 32]: source row j packed as [Hs_j (C) | 0 .. | 24: s_j |
 *     0 ..].  With hs NULL, zx is an input (from gr_gat_narrow_pack over the
 *     same rows) and d_pre must be given.  Else zx is written from hs: the
 *     logit halves are taken from s_pre / d_pre when given (both or
 *     neither); else they are formed from att_src / att_dst as
 *     gr_gat_scores forms them, and the destination halves are written to
 *     d_state [n_dst].  The kernels read d_i from d_pre or d_state.
 *   o [n_dst, C] = O (optional when y is given); y (optional, row stride
 *     ldy) = O + bias (bias optional).
 *   f_state [n_dst, C + 4]: written; [N_i (C) | m_i, den_i, S_i, 0] with
 *     N_i = sum_{t_ij <= 0} alpha_ij Hs_j and S_i = sum_{t_ij <= 0} alpha_ij,
 *     what gr_gat_narrow_backward needs instead of alpha (which is not
 *     formed).
 *   long_units (optional, device int32 [n_long]): indices of the plan units
 *     that are split or longer than 32 edges (run one per wavefront); NULL:
 *     every unit is examined.  workspace: n_slots * 52 floats.
 * The softmax runs online (one pass; the running max rescales the sums), so
 * results equal gr_gat_forward's to rounding, not bit for bit.  No
 * counterpart in the reference beyond the GATConv it replaces. */
int gr_gat_narrow_forward(const int32_t* units, int64_t n_units,
                          const int32_t* fixups, int64_t n_fix,
                          const int32_t* long_units, int64_t n_long,
                          const int32_t* idx, const float* hs, int64_t ldh,
                          int64_t n_src, int64_t n_dst, int64_t channels,
                          const float* s_pre, const float* d_pre,
                          const float* att_src, const float* att_dst,
                          const float* bias, float* zx, float* o, float* y,
                          int64_t ldy, float* d_state, float* f_state,
                          float* workspace, int64_t ws_floats, int64_t n_slots,
                          void* stream);

/* Backward of gr_gat_narrow_forward over the CSC plan (units / fixups /
 * long_units of the transposed adjacency, row_idx from gr_csr_transpose).
 * zx, f_state: the forward's; d: the destination halves it read (d_pre or
 * d_state); out (row stride ldo): its o, or its y with `bias` (O = y - bias).
 *   First, per destination row, c_i = <go_i, O_i> and
 *     dd_i = -0.8 (<go_i, N_i> - c_i S_i) + c_i 1e-16 / den_i (= sum_j g_t,ij:
 *     sum_j g_e,ij is exactly c_i 1e-16 / den_i), written to dd [n_dst], and
 *     gx [n_dst, 32] = [go_i (C) | 0 .. | 24: d_i, 25: m_i, 26: 1 / den_i,
 *     27: c_i, 28: dd_i | 0 ..];
 *   then, per source column j, with alpha_ij recomputed from s_j and gx_i,
 *     dhs [n_src, C] = sum_i alpha_ij go_i + ds_j att_src
 *                      + (j < n_dst) dd_j att_dst,
 *     ds [n_src] = sum_i g_t,ij.
 * go: row stride ldg (a multiple of 4).  workspace: n_slots * 28 floats.
 * Replaces the backward of the same PyG GATConv. */
int gr_gat_narrow_backward(const int32_t* units, int64_t n_units,
                           const int32_t* fixups, int64_t n_fix,
                           const int32_t* long_units, int64_t n_long,
                           const int32_t* row_idx, const float* zx, const float* d,
                           int64_t n_src, int64_t n_dst, int64_t channels,
                           const float* go, int64_t ldg, const float* out,
                           int64_t ldo, const float* bias, const float* f_state,
                           const float* att_src, const float* att_dst, float* gx,
                           float* dhs, float* ds, float* dd, float* workspace,
                           int64_t ws_floats, int64_t n_slots, void* stream);

/* Backward over destination rows i (CSR plan):
 * dd[i,h] = sum_e gt[e,h] + cdot[i,h] * 1e-16 / den[i,h] (= sum_j g_t,ij) and
 * dhs[i,:] += dd[i,h(f)] * att_dst[f].  Must run after
 * gr_gat_backward_src on the same stream.  workspace: n_slots * H floats. */
int gr_gat_backward_dst(const int32_t* units, int64_t n_units,
                        const int32_t* fixups, int64_t n_fix, const float* gt,
                        const float* att_dst, const float* cdot,
                        const float* den, int64_t heads, int64_t channels,
                        float* dd, float* dhs, float* workspace,
                        int64_t n_slots, void* stream);

/* ------------------------------------------------------------------------ */
/* Host <-> storage I/O (grinnder._C.IoUringEngine)                          */
/* ------------------------------------------------------------------------ */

/* Asynchronous file engine replacing IoUringEngine (csrc/cpu/
 * io_uring_engine.cpp:15-245; constructor :227-230).  liburing is absent, so
 * requests run on `threads` worker threads with pread/pwrite, each request
 * cut into 8 MiB chunks processed in parallel.  Host only. */
int gr_io_create(int32_t threads, void** engine);

/* Waits for every request, then frees the engine (~IoUringEngineImpl,
 * io_uring_engine.cpp:25-28).  Reports the first failed request. */
int gr_io_destroy(void* engine);

/* submit_read / submit_write (io_uring_engine.cpp:32-108): nbytes at
 * file `offset` into / from `buf`, which must stay valid until the request
 * is waited for.  A write creates or truncates the file to offset + nbytes
 * (the reference opens with O_TRUNC).  Returns the request's handle.  Open
 * failures are reported here; I/O failures by gr_io_wait. */
int gr_io_submit(void* engine, int32_t write, const char* path, void* buf,
                 int64_t offset, int64_t nbytes, int64_t* handle);

/* wait (io_uring_engine.cpp:110-136): blocks until the request is done and
 * forgets the handle; a failed or short transfer is returned as an error
 * (the reference throws). */
int gr_io_wait(void* engine, int64_t handle);

/* wait_all (io_uring_engine.cpp:138-160). */
int gr_io_wait_all(void* engine);

/* poll (io_uring_engine.cpp:162-178): *done = 1 once the request finished
 * (it still has to be waited for). */
int gr_io_poll(void* engine, int64_t handle, int32_t* done);

/* pending (io_uring_engine.cpp:180-187): requests submitted and not done. */
int gr_io_pending(void* engine, int64_t* count);

/* ------------------------------------------------------------------------ */
/* Synthetic inputs (no reference counterpart)                               */
/* ------------------------------------------------------------------------ */

/* Seeded R-MAT edge sampler: sample i (i in [first, first+n)) picks, for each
 * of `scale` levels, a quadrant with probabilities (a, b, c, 1-a-b-c) using a
 * counter-based 64-bit hash of (seed, i, level), so the sample stream is
 * independent of thread count.  Writes src[n], dst[n] (int64).  Host,
 * multi-threaded (nthreads <= 0: hardware concurrency). */
int gr_rmat_sample(uint64_t seed, int32_t scale, double a, double b, double c,
                   int64_t first, int64_t n, int64_t* src, int64_t* dst,
                   int32_t nthreads);

/* Counter-based N(0,1) feature rows: out[i, :dim] depends only on
 * (seed, ids[i]), so any subset of a large feature matrix is produced on
 * demand (Box-Muller on SplitMix64 uniforms).  Host, multi-threaded. */
int gr_gaussian_rows(uint64_t seed, const int64_t* ids, int64_t n, int64_t dim,
                     float* out, int32_t nthreads);

#ifdef __cplusplus
}
#endif

#endif /* GRINNDER_AMD_H */
