// Host-side partition bookkeeping and aggregation-plan preparation.
//
// Everything here is integer work that must be bit-exact with the reference
// (build_subgraph, boundary ordering) or deterministic by construction
// (CSR->CSC transpose, work plans).  It runs once per partition adjacency,
// never inside the training loop.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

#include "gr_internal.h"

namespace {

// Dense old-id -> new-id map used by the subgraph extraction.  The reference
// uses std::unordered_map (csrc/cpu/subgraph.cpp:27); a dense array gives the
// same mapping (same insertion order, last assignment wins for repeated
// seeds) with O(1) loads and no hashing.
struct DenseMap {
  std::vector<int64_t> slot;
  explicit DenseMap(int64_t n) : slot(static_cast<size_t>(n), -1) {}
};

}  // namespace

extern "C" int gr_build_subgraph(const int64_t* rowptr, const int64_t* col,
                                 const void* value, int64_t value_elem_size,
                                 int64_t num_rows, const int64_t* idx,
                                 int64_t n_idx, int32_t bipartite,
                                 int64_t* out_rowptr, int64_t* out_col,
                                 void* out_value, int64_t* out_n_id,
                                 int64_t* out_nnz, int64_t* out_num_nodes) {
  gr::clear_error();
  GR_REQUIRE(rowptr != nullptr && num_rows >= 0 && n_idx >= 0,
             "build_subgraph: invalid rowptr/num_rows/n_idx");
  GR_REQUIRE(n_idx == 0 || idx != nullptr, "build_subgraph: idx is NULL");
  GR_REQUIRE(out_nnz != nullptr && out_num_nodes != nullptr,
             "build_subgraph: out_nnz/out_num_nodes are NULL");
  if (value != nullptr) {
    GR_REQUIRE(value_elem_size == 1 || value_elem_size == 2 ||
                   value_elem_size == 4 || value_elem_size == 8,
               "build_subgraph: value element size %lld unsupported",
               (long long)value_elem_size);
  }

  // Pass 0: validate seeds, count edges, find the id range to map.
  int64_t nnz = 0;
  int64_t max_id = num_rows - 1;
  for (int64_t i = 0; i < n_idx; ++i) {
    const int64_t v = idx[i];
    GR_REQUIRE(v >= 0 && v < num_rows, "build_subgraph: seed %lld out of range [0, %lld)",
               (long long)v, (long long)num_rows);
    const int64_t b = rowptr[v], e = rowptr[v + 1];
    GR_REQUIRE(b >= 0 && e >= b, "build_subgraph: rowptr not monotone at row %lld",
               (long long)v);
    nnz += e - b;
    if (col != nullptr) {
      for (int64_t j = b; j < e; ++j) {
        GR_REQUIRE(col[j] >= 0, "build_subgraph: negative column %lld", (long long)col[j]);
        max_id = std::max(max_id, col[j]);
      }
    }
  }
  GR_REQUIRE(nnz == 0 || col != nullptr, "build_subgraph: col is NULL");

  DenseMap map(max_id + 1);
  for (int64_t i = 0; i < n_idx; ++i) map.slot[idx[i]] = i;

  const bool fill = out_col != nullptr;
  if (fill) {
    GR_REQUIRE(out_rowptr != nullptr && out_n_id != nullptr,
               "build_subgraph: output arrays are NULL");
    GR_REQUIRE(value == nullptr || out_value != nullptr,
               "build_subgraph: out_value is NULL while value is given");
  }

  // Pass 1: row-major scan; unseen neighbours get the next id in first-seen
  // order (csrc/cpu/subgraph.cpp:56-75 and :79-98).
  int64_t n_new = 0;
  int64_t offset = 0;
  if (fill) out_rowptr[0] = 0;
  const size_t esz = static_cast<size_t>(value_elem_size);
  for (int64_t i = 0; i < n_idx; ++i) {
    const int64_t v = idx[i];
    for (int64_t j = rowptr[v]; j < rowptr[v + 1]; ++j) {
      const int64_t w = col[j];
      int64_t id = map.slot[w];
      if (id < 0) {
        id = n_idx + n_new;
        map.slot[w] = id;
        if (fill) out_n_id[id] = w;
        ++n_new;
      }
      if (fill) {
        out_col[offset] = id;
        if (value != nullptr) {
          std::memcpy(static_cast<char*>(out_value) + offset * esz,
                      static_cast<const char*>(value) + j * esz, esz);
        }
      }
      ++offset;
    }
    if (fill) out_rowptr[i + 1] = offset;
  }

  *out_nnz = nnz;
  *out_num_nodes = n_idx + n_new;
  if (!fill) return GR_OK;

  for (int64_t i = 0; i < n_idx; ++i) out_n_id[i] = idx[i];
  // Non-bipartite: boundary nodes get empty rows (subgraph.cpp:102-107).
  if (!bipartite) {
    for (int64_t k = 0; k < n_new; ++k) out_rowptr[n_idx + 1 + k] = nnz;
  }
  return GR_OK;
}

extern "C" int gr_partition_boundaries(int32_t pid, int32_t num_parts,
                                       const int64_t* ptr, int64_t batch_size,
                                       const int64_t* halo_ids, int64_t n_halo,
                                       int64_t* col, int64_t nnz,
                                       int64_t* boundary_flat,
                                       int64_t* boundary_lens) {
  gr::clear_error();
  GR_REQUIRE(num_parts >= 1 && pid >= 0 && pid < num_parts && ptr != nullptr,
             "partition_boundaries: bad pid %d / num_parts %d", pid, num_parts);
  GR_REQUIRE(boundary_lens != nullptr, "partition_boundaries: boundary_lens is NULL");
  GR_REQUIRE(n_halo == 0 || (halo_ids != nullptr && boundary_flat != nullptr),
             "partition_boundaries: halo arrays are NULL");
  for (int32_t p = 0; p < num_parts; ++p) {
    GR_REQUIRE(ptr[p + 1] >= ptr[p], "partition_boundaries: ptr not monotone");
  }

  // Owner of each halo node (partitions are contiguous id ranges).
  std::vector<int32_t> owner(static_cast<size_t>(n_halo));
  std::vector<int64_t> count(static_cast<size_t>(num_parts), 0);
  for (int64_t k = 0; k < n_halo; ++k) {
    const int64_t g = halo_ids[k];
    GR_REQUIRE(g >= ptr[0] && g < ptr[num_parts],
               "partition_boundaries: halo node %lld outside all partitions", (long long)g);
    const int64_t* it = std::upper_bound(ptr, ptr + num_parts + 1, g);
    const int32_t p = static_cast<int32_t>((it - ptr) - 1);
    GR_REQUIRE(p != pid, "partition_boundaries: halo node %lld lies in partition %d itself",
               (long long)g, pid);
    owner[k] = p;
    ++count[p];
  }

  // Stable grouping by owner ascending (partition.py:201-212): discovery
  // order is kept inside each group.
  std::vector<int64_t> start(static_cast<size_t>(num_parts), 0);
  int64_t run = 0;
  for (int32_t p = 0; p < num_parts; ++p) {
    start[p] = run;
    run += count[p];
    boundary_lens[p] = count[p];
  }
  std::vector<int64_t> new_pos(static_cast<size_t>(n_halo));
  for (int64_t k = 0; k < n_halo; ++k) {
    const int32_t p = owner[k];
    const int64_t pos = start[p]++;
    new_pos[k] = pos;
    boundary_flat[pos] = halo_ids[k] - ptr[p];
  }

  // Column remap: discovery order -> partition order (partition.py:213-225).
  if (n_halo > 0 && col != nullptr) {
    for (int64_t e = 0; e < nnz; ++e) {
      const int64_t c = col[e];
      if (c >= batch_size) {
        GR_REQUIRE(c - batch_size < n_halo, "partition_boundaries: column %lld out of range",
                   (long long)c);
        col[e] = batch_size + new_pos[c - batch_size];
      }
    }
  }
  return GR_OK;
}

extern "C" int gr_csr_transpose(const int64_t* rowptr, const int64_t* col,
                                const float* val, int64_t rows, int64_t cols,
                                int64_t* colptr, int32_t* row_idx, float* val_t,
                                int32_t* perm) {
  gr::clear_error();
  GR_REQUIRE(rowptr != nullptr && colptr != nullptr && rows >= 0 && cols >= 0,
             "csr_transpose: invalid arguments");
  const int64_t nnz = rowptr[rows];
  GR_REQUIRE(nnz == 0 || (col != nullptr && row_idx != nullptr),
             "csr_transpose: col/row_idx are NULL");
  GR_REQUIRE(rows <= INT32_MAX && nnz <= INT32_MAX,
             "csr_transpose: rows/nnz exceed int32 (%lld/%lld)", (long long)rows,
             (long long)nnz);

  std::vector<int64_t> next(static_cast<size_t>(cols) + 1, 0);
  for (int64_t e = 0; e < nnz; ++e) {
    const int64_t c = col[e];
    GR_REQUIRE(c >= 0 && c < cols, "csr_transpose: column %lld out of range [0, %lld)",
               (long long)c, (long long)cols);
    ++next[c + 1];
  }
  for (int64_t c = 0; c < cols; ++c) next[c + 1] += next[c];
  std::memcpy(colptr, next.data(), sizeof(int64_t) * (static_cast<size_t>(cols) + 1));

  // Stable placement: CSR order is row-major, so each column receives its
  // entries in (row, position) order.
  const bool with_val = val != nullptr && val_t != nullptr;
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t e = rowptr[r]; e < rowptr[r + 1]; ++e) {
      const int64_t dst = next[col[e]]++;
      row_idx[dst] = static_cast<int32_t>(r);
      if (with_val) val_t[dst] = val[e];
      if (perm != nullptr) perm[dst] = static_cast<int32_t>(e);
    }
  }
  return GR_OK;
}

namespace {

// The plan of gr_spmm_plan / gr_spmm_plan_blocked: whole rows ordered block
// by block (one block [0, rows) when block_ptr is NULL).
int spmm_plan_impl(const int64_t* rowptr, int64_t rows, int32_t seg_len,
                   const int64_t* block_ptr, int64_t n_blocks, int32_t* units,
                   int64_t* n_units, int32_t* fixups, int64_t* n_fix, int64_t* n_slots) {
  GR_REQUIRE(rowptr != nullptr && rows >= 0 && seg_len > 0,
             "spmm_plan: invalid arguments");
  GR_REQUIRE(n_units != nullptr && n_fix != nullptr && n_slots != nullptr,
             "spmm_plan: count outputs are NULL");
  GR_REQUIRE(rows <= INT32_MAX && rowptr[rows] <= INT32_MAX,
             "spmm_plan: rows/nnz exceed int32");
  if (block_ptr != nullptr) {
    GR_REQUIRE(n_blocks >= 1 && block_ptr[0] == 0 && block_ptr[n_blocks] == rows,
               "spmm_plan: blocks must cover [0, %lld)", (long long)rows);
    for (int64_t k = 0; k < n_blocks; ++k)
      GR_REQUIRE(block_ptr[k] <= block_ptr[k + 1], "spmm_plan: block %lld not monotone",
                 (long long)k);
  }

  int64_t nu = 0, nf = 0, ns = 0;
  for (int64_t r = 0; r < rows; ++r) {
    const int64_t len = rowptr[r + 1] - rowptr[r];
    GR_REQUIRE(len >= 0, "spmm_plan: rowptr not monotone at row %lld", (long long)r);
    if (len > seg_len) {
      const int64_t k = (len + seg_len - 1) / seg_len;
      nu += k;
      ns += k;
      ++nf;
    } else {
      ++nu;
    }
  }
  *n_units = nu;
  *n_fix = nf;
  *n_slots = ns;
  if (units == nullptr) return GR_OK;
  GR_REQUIRE(nf == 0 || fixups != nullptr, "spmm_plan: fixups is NULL");

  int64_t u = 0, f = 0, slot = 0;
  // Split rows first.
  for (int64_t r = 0; r < rows; ++r) {
    const int64_t b = rowptr[r], e = rowptr[r + 1];
    if (e - b <= seg_len) continue;
    fixups[3 * f + 0] = static_cast<int32_t>(r);
    fixups[3 * f + 1] = static_cast<int32_t>(slot);
    int32_t k = 0;
    for (int64_t s = b; s < e; s += seg_len, ++k) {
      units[4 * u + 0] = static_cast<int32_t>(r);
      units[4 * u + 1] = static_cast<int32_t>(s);
      units[4 * u + 2] = static_cast<int32_t>(std::min<int64_t>(s + seg_len, e));
      units[4 * u + 3] = static_cast<int32_t>(slot++);
      ++u;
    }
    fixups[3 * f + 2] = k;
    ++f;
  }
  // Whole rows next, block by block, by length class within a block
  // (longest class first, row order within a class): kernels that give one
  // wavefront several rows then get rows of similar length together, the
  // longest rows start first, and a block's rows run together.
  auto length_class = [](int64_t len) {
    int c = 0;
    while (len > 0) {
      ++c;
      len >>= 1;
    }
    return c;  // 0 for empty rows, floor(log2(len)) + 1 otherwise
  };
  const int top = length_class(seg_len);
  const int64_t nb = block_ptr != nullptr ? n_blocks : 1;
  for (int64_t blk = 0; blk < nb; ++blk) {
    const int64_t r0 = block_ptr != nullptr ? block_ptr[blk] : 0;
    const int64_t r1 = block_ptr != nullptr ? block_ptr[blk + 1] : rows;
    for (int cls = top; cls >= 0; --cls) {
      for (int64_t r = r0; r < r1; ++r) {
        const int64_t b = rowptr[r], e = rowptr[r + 1];
        if (e - b > seg_len || length_class(e - b) != cls) continue;
        units[4 * u + 0] = static_cast<int32_t>(r);
        units[4 * u + 1] = static_cast<int32_t>(b);
        units[4 * u + 2] = static_cast<int32_t>(e);
        units[4 * u + 3] = -1;
        ++u;
      }
    }
  }
  return GR_OK;
}

}  // namespace

extern "C" int gr_spmm_plan(const int64_t* rowptr, int64_t rows, int32_t seg_len,
                            int32_t* units, int64_t* n_units, int32_t* fixups,
                            int64_t* n_fix, int64_t* n_slots) {
  gr::clear_error();
  return spmm_plan_impl(rowptr, rows, seg_len, nullptr, 0, units, n_units, fixups, n_fix,
                        n_slots);
}

extern "C" int gr_spmm_plan_blocked(const int64_t* rowptr, int64_t rows, int32_t seg_len,
                                    const int64_t* block_ptr, int64_t n_blocks,
                                    int32_t* units, int64_t* n_units, int32_t* fixups,
                                    int64_t* n_fix, int64_t* n_slots) {
  gr::clear_error();
  GR_REQUIRE(block_ptr != nullptr, "spmm_plan: block_ptr is NULL");
  return spmm_plan_impl(rowptr, rows, seg_len, block_ptr, n_blocks, units, n_units, fixups,
                        n_fix, n_slots);
}

namespace {

// SplitMix64 finaliser (Steele, Lea, Flood 2014): a bijective 64-bit mixer.
inline uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

}  // namespace

extern "C" int gr_rmat_sample(uint64_t seed, int32_t scale, double a, double b,
                              double c, int64_t first, int64_t n, int64_t* src,
                              int64_t* dst, int32_t nthreads) {
  gr::clear_error();
  GR_REQUIRE(scale >= 1 && scale <= 40, "rmat_sample: scale %d out of range", scale);
  GR_REQUIRE(a >= 0 && b >= 0 && c >= 0 && a + b + c <= 1.0,
             "rmat_sample: invalid probabilities");
  GR_REQUIRE(n >= 0 && first >= 0, "rmat_sample: invalid range");
  GR_REQUIRE(n == 0 || (src != nullptr && dst != nullptr), "rmat_sample: NULL outputs");
  // Quadrant thresholds on a 32-bit uniform integer.
  const double two32 = 4294967296.0;
  const uint64_t ta = static_cast<uint64_t>(a * two32);
  const uint64_t tab = static_cast<uint64_t>((a + b) * two32);
  const uint64_t tabc = static_cast<uint64_t>((a + b + c) * two32);
  const uint64_t key = mix64(seed ^ 0x5851F42D4C957F2Dull);

  auto work = [&](int64_t lo, int64_t hi) {
    for (int64_t i = lo; i < hi; ++i) {
      const uint64_t ctr = static_cast<uint64_t>(first + i);
      uint64_t s = 0, d = 0;
      uint64_t bits = 0;
      for (int32_t lvl = 0; lvl < scale; ++lvl) {
        uint32_t u;
        if ((lvl & 1) == 0) {
          bits = mix64(key + 0x9E3779B97F4A7C15ull * (ctr * 32u + static_cast<uint64_t>(lvl >> 1) + 1u));
          u = static_cast<uint32_t>(bits);
        } else {
          u = static_cast<uint32_t>(bits >> 32);
        }
        uint64_t sb, db;
        if (u < ta) {
          sb = 0; db = 0;
        } else if (u < tab) {
          sb = 0; db = 1;
        } else if (u < tabc) {
          sb = 1; db = 0;
        } else {
          sb = 1; db = 1;
        }
        s = (s << 1) | sb;
        d = (d << 1) | db;
      }
      src[i] = static_cast<int64_t>(s);
      dst[i] = static_cast<int64_t>(d);
    }
  };

  int32_t nt = nthreads > 0 ? nthreads : static_cast<int32_t>(std::thread::hardware_concurrency());
  if (nt < 1) nt = 1;
  if (n < (int64_t)1 << 16) nt = 1;
  if (nt == 1) {
    work(0, n);
    return GR_OK;
  }
  std::vector<std::thread> pool;
  const int64_t chunk = (n + nt - 1) / nt;
  for (int32_t t = 0; t < nt; ++t) {
    const int64_t lo = t * chunk, hi = std::min<int64_t>(n, lo + chunk);
    if (lo >= hi) break;
    pool.emplace_back(work, lo, hi);
  }
  for (auto& th : pool) th.join();
  return GR_OK;
}

// ------------------------------------------------------------ partitioner --
//
// The reference delegates partitioning to grdpart (not available).  This is
// the library's own deterministic partitioner:
//   1. undirected adjacency of the COO graph (both directions, counting sort),
//   2. breadth-first order (components visited in id order, neighbours in
//      adjacency order) — or the natural id order,
//   3. linear deterministic greedy streaming assignment in that order:
//      p* = argmax_p |N(v) ∩ P_p| * (1 - |P_p| / cap), cap = ceil(capacity*n/P),
//      ties -> lighter partition, then lower id; full partitions are skipped,
//   4. perm = nodes grouped by partition, each group in visit order (so a
//      partition's rows are also BFS-local), ptr = group offsets.
extern "C" int gr_partition_graph(const int64_t* src, const int64_t* dst, int64_t m, int64_t n,
                                  int32_t num_parts, double capacity, int32_t bfs_order,
                                  int64_t* perm, int64_t* ptr) {
  gr::clear_error();
  GR_REQUIRE(n >= 1 && n <= INT32_MAX && m >= 0, "partition_graph: bad sizes");
  GR_REQUIRE(num_parts >= 1 && num_parts <= 4096 && num_parts <= n,
             "partition_graph: num_parts %d invalid for %lld nodes", num_parts, (long long)n);
  GR_REQUIRE(capacity >= 1.0, "partition_graph: capacity must be >= 1");
  GR_REQUIRE(m == 0 || (src != nullptr && dst != nullptr), "partition_graph: NULL edges");
  GR_REQUIRE(perm != nullptr && ptr != nullptr, "partition_graph: NULL outputs");

  // 1. symmetric adjacency (self-loops dropped), int32 ids.
  std::vector<int64_t> off(static_cast<size_t>(n) + 1, 0);
  for (int64_t e = 0; e < m; ++e) {
    const int64_t a = src[e], b = dst[e];
    GR_REQUIRE(a >= 0 && a < n && b >= 0 && b < n, "partition_graph: edge (%lld, %lld) out of range",
               (long long)a, (long long)b);
    if (a == b) continue;
    ++off[a + 1];
    ++off[b + 1];
  }
  for (int64_t v = 0; v < n; ++v) off[v + 1] += off[v];
  std::vector<int32_t> adj(static_cast<size_t>(off[n]));
  {
    std::vector<int64_t> fill(off.begin(), off.end() - 1);
    for (int64_t e = 0; e < m; ++e) {
      const int64_t a = src[e], b = dst[e];
      if (a == b) continue;
      adj[fill[a]++] = static_cast<int32_t>(b);
      adj[fill[b]++] = static_cast<int32_t>(a);
    }
  }

  // 2. visit order.
  std::vector<int32_t> order(static_cast<size_t>(n));
  if (bfs_order) {
    std::vector<uint8_t> seen(static_cast<size_t>(n), 0);
    int64_t head = 0, tail = 0;
    for (int64_t s = 0; s < n; ++s) {
      if (seen[s]) continue;
      seen[s] = 1;
      order[tail++] = static_cast<int32_t>(s);
      while (head < tail) {
        const int32_t v = order[head++];
        for (int64_t k = off[v]; k < off[v + 1]; ++k) {
          const int32_t u = adj[k];
          if (!seen[u]) {
            seen[u] = 1;
            order[tail++] = u;
          }
        }
      }
    }
  } else {
    for (int64_t v = 0; v < n; ++v) order[v] = static_cast<int32_t>(v);
  }

  // 3. greedy assignment.
  const int32_t P = num_parts;
  std::vector<int32_t> part(static_cast<size_t>(n), -1);
  std::vector<int64_t> load(P, 0);
  const int64_t cap = static_cast<int64_t>(std::ceil(capacity * static_cast<double>(n) / P));
  std::vector<int64_t> cnt(P, 0);
  std::vector<int32_t> touched;
  touched.reserve(P);
  for (int64_t i = 0; i < n; ++i) {
    const int32_t v = order[i];
    touched.clear();
    for (int64_t k = off[v]; k < off[v + 1]; ++k) {
      const int32_t q = part[adj[k]];
      if (q < 0) continue;
      if (cnt[q]++ == 0) touched.push_back(q);
    }
    int32_t best = -1;
    double best_score = -1.0;
    for (int32_t q : touched) {
      if (load[q] >= cap) continue;
      const double score = static_cast<double>(cnt[q]) *
                           (1.0 - static_cast<double>(load[q]) / static_cast<double>(cap));
      if (score > best_score || (score == best_score &&
                                 (load[q] < load[best] || (load[q] == load[best] && q < best)))) {
        best = q;
        best_score = score;
      }
    }
    for (int32_t q : touched) cnt[q] = 0;
    if (best < 0 || best_score <= 0.0) {
      best = 0;
      for (int32_t q = 1; q < P; ++q)
        if (load[q] < load[best]) best = q;
    }
    part[v] = best;
    ++load[best];
  }

  // 4. group by partition, keeping visit order inside each group.
  ptr[0] = 0;
  for (int32_t q = 0; q < P; ++q) ptr[q + 1] = ptr[q] + load[q];
  std::vector<int64_t> pos(ptr, ptr + P);
  for (int64_t i = 0; i < n; ++i) {
    const int32_t v = order[i];
    perm[pos[part[v]]++] = v;
  }
  return GR_OK;
}

// Counter-based N(0,1) rows: out[i, j] depends only on (seed, ids[i], j), so a
// partition's feature rows can be produced on demand, in any order, by any
// number of threads.  Uniforms from the SplitMix64 mixer, normals by the
// Box-Muller transform on (j & ~1, j | 1) pairs.
extern "C" int gr_gaussian_rows(uint64_t seed, const int64_t* ids, int64_t n, int64_t dim,
                                float* out, int32_t nthreads) {
  gr::clear_error();
  GR_REQUIRE(n >= 0 && dim >= 1, "gaussian_rows: bad shape");
  GR_REQUIRE(n == 0 || (ids != nullptr && out != nullptr), "gaussian_rows: NULL pointer");
  const uint64_t key = mix64(seed ^ 0xD1B54A32D192ED03ull);
  auto work = [&](int64_t lo, int64_t hi) {
    for (int64_t i = lo; i < hi; ++i) {
      const uint64_t row = static_cast<uint64_t>(ids[i]);
      float* o = out + i * dim;
      for (int64_t j = 0; j < dim; j += 2) {
        const uint64_t h = mix64(key + 0x9E3779B97F4A7C15ull * (row * 0x100000001B3ull + static_cast<uint64_t>(j >> 1) + 1));
        // 24-bit uniforms in (0, 1] and [0, 1).
        const double u1 = (static_cast<double>(h >> 40) + 1.0) / 16777216.0;
        const double u2 = static_cast<double>((h >> 16) & 0xFFFFFF) / 16777216.0;
        const double r = std::sqrt(-2.0 * std::log(u1));
        const double t = 6.283185307179586 * u2;
        o[j] = static_cast<float>(r * std::cos(t));
        if (j + 1 < dim) o[j + 1] = static_cast<float>(r * std::sin(t));
      }
    }
  };
  int32_t nt = nthreads > 0 ? nthreads : static_cast<int32_t>(std::thread::hardware_concurrency());
  if (nt < 1) nt = 1;
  if (n * dim < (int64_t)1 << 18) nt = 1;
  if (nt == 1) {
    work(0, n);
    return GR_OK;
  }
  std::vector<std::thread> pool;
  const int64_t chunk = (n + nt - 1) / nt;
  for (int32_t t = 0; t < nt; ++t) {
    const int64_t lo = t * chunk, hi = std::min<int64_t>(n, lo + chunk);
    if (lo >= hi) break;
    pool.emplace_back(work, lo, hi);
  }
  for (auto& th : pool) th.join();
  return GR_OK;
}
