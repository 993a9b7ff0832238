// Host <-> device transfers and the halo gather / gradient scatter-add.
//
// MI355X design: host partition buffers that are pinned (hipHostMalloc, as
// torch's pin_memory allocates them) are mapped into the GPU's address space,
// so halo rows are moved by a device kernel that reads (gather) or
// read-add-writes (scatter) them over PCIe in place — no host thread touches
// the rows and everything stays ordered on the caller's stream.  Pageable
// buffers, which a device cannot address, take a host-thread path through a
// pinned staging slot.  Completion of every enqueued transfer is recorded in
// a per-direction FIFO of events, drained one entry per *_synchronize call.
#include <algorithm>
#include <cstring>
#include <deque>
#include <mutex>
#include <thread>
#include <vector>

#include "gr_internal.h"

namespace {

// ---------------------------------------------------------------- events --

struct EventFifo {
  std::mutex m;
  std::deque<hipEvent_t> q;
};

EventFifo& h2d_fifo() {
  static EventFifo f;
  return f;
}
EventFifo& d2h_fifo() {
  static EventFifo f;
  return f;
}

constexpr size_t kMaxQueued = 4096;

// Pinned staging slots hold at most this many bytes (pageable paths chunk).
constexpr int64_t kChunkBytes = int64_t(64) << 20;

int fifo_push(EventFifo& f, hipStream_t s) {
  hipEvent_t ev = nullptr;
  GR_HIP_CHECK(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
  hipError_t e = hipEventRecord(ev, s);
  if (e != hipSuccess) {
    (void)hipEventDestroy(ev);
    return gr::fail(GR_EHIP, "hipEventRecord failed: %s", hipGetErrorString(e));
  }
  hipEvent_t drop = nullptr;
  {
    std::lock_guard<std::mutex> lk(f.m);
    f.q.push_back(ev);
    if (f.q.size() > kMaxQueued) {
      drop = f.q.front();
      f.q.pop_front();
    }
  }
  if (drop != nullptr) {
    // Bound the queue: the oldest entry is waited for and retired.
    hipError_t se = hipEventSynchronize(drop);
    (void)hipEventDestroy(drop);
    if (se != hipSuccess)
      return gr::fail(GR_EHIP, "hipEventSynchronize failed: %s", hipGetErrorString(se));
  }
  return GR_OK;
}

int fifo_pop_wait(EventFifo& f) {
  hipEvent_t ev = nullptr;
  {
    std::lock_guard<std::mutex> lk(f.m);
    if (f.q.empty()) return GR_OK;
    ev = f.q.front();
    f.q.pop_front();
  }
  hipError_t se = hipEventSynchronize(ev);
  (void)hipEventDestroy(ev);
  if (se != hipSuccess)
    return gr::fail(GR_EHIP, "transfer failed: %s", hipGetErrorString(se));
  return GR_OK;
}

// ------------------------------------------------------- pinned staging --

// A small ring of pinned host slots.  A slot is reused only after the event
// recorded behind its last consumer has completed.  Slots are only ever
// filled or drained by the host and copied by hipMemcpyAsync (never read by
// a kernel through a mapped pointer), so when the driver refuses pinned
// memory (a cap that the host partitions may have used up) a slot falls
// back to pageable memory: the copies then run at pageable speed, but run.
struct Staging {
  std::mutex m;
  struct Slot {
    void* ptr = nullptr;
    size_t bytes = 0;
    bool pageable = false;  // ptr from std::malloc, not hipHostMalloc
    hipEvent_t done = nullptr;
    bool busy = false;
    void* dev = nullptr;  // device twin (address tables), on device `dev_id`
    size_t dev_bytes = 0;
    int dev_id = -1;
  };
  Slot slots[4];
  int next = 0;
};

Staging& staging() {
  static Staging s;
  return s;
}

// Returns a pinned slot of at least `bytes`; *slot_id identifies it for
// staging_release.  The slot stays private to the caller until released.
int staging_acquire(size_t bytes, void** out, int* slot_id) {
  Staging& st = staging();
  std::lock_guard<std::mutex> lk(st.m);
  int i = -1;
  for (int t = 0; t < 4; ++t) {
    const int c = (st.next + t) % 4;
    if (!st.slots[c].busy) {
      i = c;
      break;
    }
  }
  if (i < 0) return gr::fail(GR_EINVAL, "staging: all pinned slots are in use");
  st.next = (i + 1) % 4;
  Staging::Slot& sl = st.slots[i];
  if (sl.done != nullptr) {
    GR_HIP_CHECK(hipEventSynchronize(sl.done));
  }
  if (sl.bytes < bytes) {
    if (sl.ptr != nullptr) {
      if (sl.pageable)
        std::free(sl.ptr);
      else
        GR_HIP_CHECK(hipHostFree(sl.ptr));
    }
    sl.ptr = nullptr;
    sl.bytes = 0;
    size_t want = std::max<size_t>(bytes, size_t(1) << 20);
    sl.pageable = hipHostMalloc(&sl.ptr, want, hipHostMallocDefault) != hipSuccess;
    if (sl.pageable) {
      (void)hipGetLastError();  // the refusal is handled here, not reported later
      sl.ptr = std::malloc(want);
      GR_REQUIRE(sl.ptr != nullptr, "staging: cannot allocate %zu host bytes", want);
    }
    sl.bytes = want;
  }
  if (sl.done == nullptr) GR_HIP_CHECK(hipEventCreateWithFlags(&sl.done, hipEventDisableTiming));
  sl.busy = true;
  *out = sl.ptr;
  *slot_id = i;
  return GR_OK;
}

// Copies the first `bytes` of an acquired slot to its device twin on stream
// s and returns the twin's address: kernels then read the table from HBM
// instead of issuing a dependent PCIe read per access.  The twin grows with
// the largest table seen and is reused under the slot's ownership rules.
int staging_to_device(int slot_id, size_t bytes, hipStream_t s, void** out) {
  Staging& st = staging();
  int dev = 0;
  GR_HIP_CHECK(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lk(st.m);
  Staging::Slot& sl = st.slots[slot_id];
  if (sl.dev_bytes < bytes || sl.dev_id != dev) {
    if (sl.dev != nullptr) GR_HIP_CHECK(hipFree(sl.dev));
    sl.dev = nullptr;
    sl.dev_bytes = 0;
    const size_t want = std::max<size_t>(bytes, size_t(1) << 20);
    GR_HIP_CHECK(hipMalloc(&sl.dev, want));
    sl.dev_bytes = want;
    sl.dev_id = dev;
  }
  GR_HIP_CHECK(hipMemcpyAsync(sl.dev, sl.ptr, bytes, hipMemcpyHostToDevice, s));
  *out = sl.dev;
  return GR_OK;
}

int staging_release(int slot_id, hipStream_t s) {
  Staging& st = staging();
  std::lock_guard<std::mutex> lk(st.m);
  st.slots[slot_id].busy = false;
  GR_HIP_CHECK(hipEventRecord(st.slots[slot_id].done, s));
  return GR_OK;
}

// ------------------------------------------------------- pointer kinds --

enum class MemKind { kPageable, kPinned, kDevice };

MemKind classify(const void* p, void** dev_alias) {
  hipPointerAttribute_t attr;
  std::memset(&attr, 0, sizeof(attr));
  hipError_t e = hipPointerGetAttributes(&attr, p);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    *dev_alias = nullptr;
    return MemKind::kPageable;
  }
  if (attr.type == hipMemoryTypeDevice) {
    *dev_alias = const_cast<void*>(p);
    return MemKind::kDevice;
  }
  if (attr.type == hipMemoryTypeHost) {
    *dev_alias = attr.devicePointer != nullptr ? attr.devicePointer : const_cast<void*>(p);
    return MemKind::kPinned;
  }
  *dev_alias = nullptr;
  return MemKind::kPageable;
}

// ------------------------------------------------------------- kernels --

// The zero-copy kernels below read or write host memory over PCIe.  32
// workgroups (128 wavefronts) with 4 accesses in flight per lane saturate the
// link (56.7 GB/s measured on MI355X for 4 KiB rows), while larger grids hold
// wave slots for the whole transfer: an HBM-streaming kernel on another stream
// ran 10-12x slower beside a gather of 256 or more workgroups, and 1.03x
// slower beside one of 32.  A transfer overlapped with compute must not take
// the compute units away from it.
constexpr unsigned kZeroCopyWorkgroups = 32;
constexpr int kZeroCopyUnroll = 4;

// dst[i] for i over n_rows * row_elems elements: element j of row r comes from
// the device-visible address src_rows[r].  Flat over elements, so rows narrower
// than a wavefront still keep the link busy.
template <typename T>
__global__ __launch_bounds__(256) void gather_rows_kernel(const uint64_t* __restrict__ src_rows,
                                                          int64_t n_rows, T* __restrict__ dst,
                                                          int64_t row_elems) {
  const int64_t total = n_rows * row_elems;
  const int64_t nthreads = (int64_t)gridDim.x * 256;
  for (int64_t base = (int64_t)blockIdx.x * 256 + threadIdx.x; base < total;
       base += kZeroCopyUnroll * nthreads) {
    T v[kZeroCopyUnroll];
#pragma unroll
    for (int u = 0; u < kZeroCopyUnroll; ++u) {
      const int64_t i = base + u * nthreads;
      if (i < total) {
        const int64_t r = i / row_elems;
        v[u] = reinterpret_cast<const T*>(src_rows[r])[i - r * row_elems];
      }
    }
#pragma unroll
    for (int u = 0; u < kZeroCopyUnroll; ++u) {
      const int64_t i = base + u * nthreads;
      if (i < total) dst[i] = v[u];
    }
  }
}

// target[r][j] += src[r][j] over n_rows rows of `dim` (in V units): rows
// r < n_intra go to intra + r * dim, the rest to the addresses in halo_rows.
// Every target row is distinct within one launch (checked on the host), so
// each element has one writer: no atomics, deterministic.
template <typename V>
__global__ __launch_bounds__(256) void scatter_add_rows_kernel(
    const V* __restrict__ src, int64_t dim, V* __restrict__ intra, int64_t n_intra,
    const uint64_t* __restrict__ halo_rows, int64_t n_rows) {
  const int64_t total = n_rows * dim;
  const int64_t nthreads = (int64_t)gridDim.x * 256;
  for (int64_t base = (int64_t)blockIdx.x * 256 + threadIdx.x; base < total;
       base += kZeroCopyUnroll * nthreads) {
    V* dp[kZeroCopyUnroll];
    V dv[kZeroCopyUnroll], sv[kZeroCopyUnroll];
#pragma unroll
    for (int u = 0; u < kZeroCopyUnroll; ++u) {
      const int64_t i = base + u * nthreads;
      if (i < total) {
        const int64_t r = i / dim;
        const int64_t j = i - r * dim;
        V* row = (r < n_intra) ? intra + r * dim
                               : reinterpret_cast<V*>(halo_rows[r - n_intra]);
        dp[u] = row + j;
        dv[u] = *dp[u];
        sv[u] = src[i];
      }
    }
#pragma unroll
    for (int u = 0; u < kZeroCopyUnroll; ++u) {
      const int64_t i = base + u * nthreads;
      if (i < total) *dp[u] = dv[u] + sv[u];
    }
  }
}

unsigned grid_for_elems(int64_t elems) {
  const int64_t want = (elems + 256 * kZeroCopyUnroll - 1) / (256 * kZeroCopyUnroll);
  return (unsigned)std::max<int64_t>(1, std::min<int64_t>(want, kZeroCopyWorkgroups));
}

void parallel_for(int64_t n, int64_t grain, const std::function<void(int64_t, int64_t)>& fn) {
  int nt = (int)std::min<int64_t>(8, std::max<int64_t>(1, n / std::max<int64_t>(1, grain)));
  if (nt <= 1) {
    fn(0, n);
    return;
  }
  std::vector<std::thread> th;
  const int64_t chunk = (n + nt - 1) / nt;
  for (int t = 0; t < nt; ++t) {
    const int64_t lo = t * chunk, hi = std::min(n, lo + chunk);
    if (lo < hi) th.emplace_back(fn, lo, hi);
  }
  for (auto& x : th) x.join();
}

}  // namespace

// ------------------------------------------------------------------ API --

extern "C" int gr_h2d_copy_async(const void* src_host, void* dst_dev, int64_t nbytes,
                                 void* stream) {
  gr::clear_error();
  GR_REQUIRE(nbytes >= 0, "h2d_copy_async: negative size");
  GR_REQUIRE(nbytes == 0 || (src_host != nullptr && dst_dev != nullptr),
             "h2d_copy_async: NULL pointer");
  hipStream_t s = gr::as_stream(stream);
  if (nbytes > 0)
    GR_HIP_CHECK(hipMemcpyAsync(dst_dev, src_host, (size_t)nbytes, hipMemcpyHostToDevice, s));
  return fifo_push(h2d_fifo(), s);
}

extern "C" int gr_d2h_copy_async(const void* src_dev, void* dst_host, int64_t nbytes,
                                 void* stream) {
  gr::clear_error();
  GR_REQUIRE(nbytes >= 0, "d2h_copy_async: negative size");
  GR_REQUIRE(nbytes == 0 || (src_dev != nullptr && dst_host != nullptr),
             "d2h_copy_async: NULL pointer");
  hipStream_t s = gr::as_stream(stream);
  if (nbytes > 0)
    GR_HIP_CHECK(hipMemcpyAsync(dst_host, src_dev, (size_t)nbytes, hipMemcpyDeviceToHost, s));
  return fifo_push(d2h_fifo(), s);
}

extern "C" int gr_h2d_synchronize(void) {
  gr::clear_error();
  return fifo_pop_wait(h2d_fifo());
}

extern "C" int gr_d2h_synchronize(void) {
  gr::clear_error();
  return fifo_pop_wait(d2h_fifo());
}

extern "C" int gr_gather_partitions(int32_t pid, int32_t num_parts, const void* const* srcs,
                                    const int64_t* src_rows, void* dst, int64_t dst_rows,
                                    int64_t row_bytes, const int64_t* const* boundaries,
                                    const int64_t* boundary_lens, void* stream) {
  gr::clear_error();
  GR_REQUIRE(num_parts >= 1 && pid >= 0 && pid < num_parts,
             "gather_partitions: pid %d outside [0, %d)", pid, num_parts);
  GR_REQUIRE(srcs != nullptr && src_rows != nullptr && boundary_lens != nullptr,
             "gather_partitions: NULL argument arrays");
  GR_REQUIRE(row_bytes > 0 && dst_rows >= 0, "gather_partitions: bad row size");
  GR_REQUIRE(dst != nullptr || dst_rows == 0, "gather_partitions: NULL dst");

  // Validate the whole layout before enqueuing anything
  // (async_transfer.cu:110-113 asserts offset == dst.size(0)).
  int64_t total = src_rows[pid];
  int64_t halo = 0;
  for (int32_t p = 0; p < num_parts; ++p) {
    if (p == pid || boundary_lens[p] <= 0) continue;
    GR_REQUIRE(boundaries != nullptr && boundaries[p] != nullptr,
               "gather_partitions: boundary %d is NULL", p);
    GR_REQUIRE(srcs[p] != nullptr, "gather_partitions: source %d is NULL", p);
    const int64_t* b = boundaries[p];
    for (int64_t k = 0; k < boundary_lens[p]; ++k) {
      GR_REQUIRE(b[k] >= 0 && b[k] < src_rows[p],
                 "gather_partitions: boundary[%d][%lld] = %lld out of range [0, %lld)", p,
                 (long long)k, (long long)b[k], (long long)src_rows[p]);
    }
    halo += boundary_lens[p];
  }
  total += halo;
  GR_REQUIRE(total == dst_rows,
             "Gather: copied size mismatch with destination (%lld rows vs %lld)",
             (long long)total, (long long)dst_rows);
  void* alias = nullptr;
  GR_REQUIRE(classify(dst, &alias) != MemKind::kPageable || dst_rows == 0,
             "gather_partitions: destination must be device memory");

  hipStream_t s = gr::as_stream(stream);
  char* d = static_cast<char*>(dst);
  const int64_t intra = src_rows[pid];
  if (intra > 0) {
    GR_REQUIRE(srcs[pid] != nullptr, "gather_partitions: source %d is NULL", pid);
    GR_HIP_CHECK(hipMemcpyAsync(d, srcs[pid], (size_t)(intra * row_bytes),
                                hipMemcpyHostToDevice, s));
  }

  if (halo > 0) {
    // Device-visible sources?
    std::vector<char*> dev_src(num_parts, nullptr);
    bool all_pinned = true;
    for (int32_t p = 0; p < num_parts; ++p) {
      if (p == pid || boundary_lens[p] <= 0) continue;
      void* a = nullptr;
      MemKind k = classify(srcs[p], &a);
      GR_REQUIRE(k != MemKind::kDevice, "gather_partitions: source %d is device memory", p);
      if (k != MemKind::kPinned) all_pinned = false;
      dev_src[p] = static_cast<char*>(a);
    }
    void* stage = nullptr;
    int slot = -1;
    if (all_pinned) {
      int rc = staging_acquire((size_t)halo * sizeof(uint64_t), &stage, &slot);
      if (rc != GR_OK) return rc;
      uint64_t* table = static_cast<uint64_t*>(stage);
      int64_t o = 0;
      for (int32_t p = 0; p < num_parts; ++p) {
        if (p == pid || boundary_lens[p] <= 0) continue;
        const int64_t* b = boundaries[p];
        for (int64_t k = 0; k < boundary_lens[p]; ++k)
          table[o++] = reinterpret_cast<uint64_t>(dev_src[p] + b[k] * row_bytes);
      }
      void* table_dev = nullptr;
      rc = staging_to_device(slot, (size_t)halo * sizeof(uint64_t), s, &table_dev);
      if (rc != GR_OK) {
        staging_release(slot, s);
        return rc;
      }
      char* out = d + intra * row_bytes;
      // 16-byte accesses when every row start is 16-byte aligned.
      bool al16 = row_bytes % 16 == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0;
      for (int32_t p = 0; p < num_parts && al16; ++p)
        if (dev_src[p] != nullptr && reinterpret_cast<uintptr_t>(dev_src[p]) % 16 != 0)
          al16 = false;
      const uint64_t* tab = static_cast<const uint64_t*>(table_dev);
      if (al16) {
        hipLaunchKernelGGL(gather_rows_kernel<uint4>, dim3(grid_for_elems(halo * row_bytes / 16)),
                           dim3(256), 0, s, tab, halo, reinterpret_cast<uint4*>(out),
                           row_bytes / 16);
      } else if (row_bytes % 4 == 0) {
        hipLaunchKernelGGL(gather_rows_kernel<uint32_t>,
                           dim3(grid_for_elems(halo * row_bytes / 4)), dim3(256), 0, s, tab,
                           halo, reinterpret_cast<uint32_t*>(out), row_bytes / 4);
      } else {
        hipLaunchKernelGGL(gather_rows_kernel<unsigned char>, dim3(grid_for_elems(halo * row_bytes)),
                           dim3(256), 0, s, tab, halo, reinterpret_cast<unsigned char*>(out),
                           row_bytes);
      }
      GR_HIP_CHECK(hipGetLastError());
    } else {
      // Pageable sources: host threads gather rows into pinned staging chunks
      // of at most kChunkBytes, each copied by DMA as soon as it is full.
      const int64_t rows_per_chunk = std::max<int64_t>(1, kChunkBytes / row_bytes);
      std::vector<const char*> row_src((size_t)halo);
      int64_t o = 0;
      for (int32_t p = 0; p < num_parts; ++p) {
        if (p == pid || boundary_lens[p] <= 0) continue;
        const int64_t* b = boundaries[p];
        const char* base = static_cast<const char*>(srcs[p]);
        for (int64_t k = 0; k < boundary_lens[p]; ++k) row_src[o++] = base + b[k] * row_bytes;
      }
      for (int64_t r0 = 0; r0 < halo; r0 += rows_per_chunk) {
        const int64_t n = std::min(rows_per_chunk, halo - r0);
        int rc = staging_acquire((size_t)(n * row_bytes), &stage, &slot);
        if (rc != GR_OK) return rc;
        char* st = static_cast<char*>(stage);
        parallel_for(n, 4096, [&](int64_t lo, int64_t hi) {
          for (int64_t k = lo; k < hi; ++k)
            std::memcpy(st + k * row_bytes, row_src[r0 + k], (size_t)row_bytes);
        });
        hipError_t e = hipMemcpyAsync(d + (intra + r0) * row_bytes, stage, (size_t)(n * row_bytes),
                                      hipMemcpyHostToDevice, s);
        rc = staging_release(slot, s);
        GR_HIP_CHECK(e);
        if (rc != GR_OK) return rc;
      }
      return fifo_push(h2d_fifo(), s);
    }
    int rc = staging_release(slot, s);
    if (rc != GR_OK) return rc;
  }
  return fifo_push(h2d_fifo(), s);
}

extern "C" int gr_scatter_partitions(int32_t pid, int32_t num_parts, const float* src,
                                     int64_t src_rows, int64_t dim, float* const* dsts,
                                     const int64_t* dst_rows, const int64_t* const* boundaries,
                                     const int64_t* boundary_lens, void* stream) {
  gr::clear_error();
  GR_REQUIRE(num_parts >= 1 && pid >= 0 && pid < num_parts,
             "scatter_partitions: pid %d outside [0, %d)", pid, num_parts);
  GR_REQUIRE(dsts != nullptr && dst_rows != nullptr && boundary_lens != nullptr,
             "scatter_partitions: NULL argument arrays");
  GR_REQUIRE(dim > 0 && src_rows >= 0, "scatter_partitions: bad shape");
  GR_REQUIRE(src != nullptr || src_rows == 0, "scatter_partitions: NULL src");

  // Validate layout and detect repeated indices inside a boundary.
  int64_t total = dst_rows[pid];
  int64_t halo = 0;
  bool repeated = false;
  for (int32_t p = 0; p < num_parts; ++p) {
    if (p == pid || boundary_lens[p] <= 0) continue;
    GR_REQUIRE(boundaries != nullptr && boundaries[p] != nullptr,
               "scatter_partitions: boundary %d is NULL", p);
    GR_REQUIRE(dsts[p] != nullptr, "scatter_partitions: destination %d is NULL", p);
    const int64_t* b = boundaries[p];
    std::vector<uint8_t> seen((size_t)std::max<int64_t>(dst_rows[p], 0), 0);
    for (int64_t k = 0; k < boundary_lens[p]; ++k) {
      GR_REQUIRE(b[k] >= 0 && b[k] < dst_rows[p],
                 "scatter_partitions: boundary[%d][%lld] = %lld out of range [0, %lld)", p,
                 (long long)k, (long long)b[k], (long long)dst_rows[p]);
      if (seen[b[k]]) repeated = true;
      seen[b[k]] = 1;
    }
    halo += boundary_lens[p];
  }
  total += halo;
  GR_REQUIRE(total == src_rows,
             "Scatter: copied size mismatch with source (%lld rows vs %lld)", (long long)total,
             (long long)src_rows);
  if (src_rows == 0) return fifo_push(d2h_fifo(), gr::as_stream(stream));
  void* alias = nullptr;
  GR_REQUIRE(classify(src, &alias) == MemKind::kDevice,
             "scatter_partitions: source must be device memory");

  hipStream_t s = gr::as_stream(stream);
  std::vector<float*> dev_dst(num_parts, nullptr);
  bool all_pinned = !repeated;
  for (int32_t p = 0; p < num_parts && all_pinned; ++p) {
    if (p != pid && boundary_lens[p] <= 0) continue;
    if (dst_rows[p] == 0) continue;
    void* a = nullptr;
    MemKind k = classify(dsts[p], &a);
    GR_REQUIRE(k != MemKind::kDevice, "scatter_partitions: destination %d is device memory", p);
    if (k != MemKind::kPinned) all_pinned = false;
    dev_dst[p] = static_cast<float*>(a);
  }

  if (all_pinned) {
    void* stage = nullptr;
    int slot = -1;
    const uint64_t* table_dev = nullptr;
    if (halo > 0) {
      int rc = staging_acquire((size_t)halo * sizeof(uint64_t), &stage, &slot);
      if (rc != GR_OK) return rc;
      uint64_t* table = static_cast<uint64_t*>(stage);
      int64_t o = 0;
      for (int32_t p = 0; p < num_parts; ++p) {
        if (p == pid || boundary_lens[p] <= 0) continue;
        const int64_t* b = boundaries[p];
        for (int64_t k = 0; k < boundary_lens[p]; ++k)
          table[o++] = reinterpret_cast<uint64_t>(dev_dst[p] + b[k] * dim);
      }
      void* tdev = nullptr;
      rc = staging_to_device(slot, (size_t)halo * sizeof(uint64_t), s, &tdev);
      if (rc != GR_OK) {
        staging_release(slot, s);
        return rc;
      }
      table_dev = static_cast<const uint64_t*>(tdev);
    }
    bool al16 = dim % 4 == 0 && reinterpret_cast<uintptr_t>(src) % 16 == 0;
    for (int32_t p = 0; p < num_parts && al16; ++p)
      if (dev_dst[p] != nullptr && reinterpret_cast<uintptr_t>(dev_dst[p]) % 16 != 0)
        al16 = false;
    if (al16) {
      hipLaunchKernelGGL(scatter_add_rows_kernel<float4>, dim3(grid_for_elems(src_rows * dim / 4)),
                         dim3(256), 0, s, reinterpret_cast<const float4*>(src), dim / 4,
                         reinterpret_cast<float4*>(dev_dst[pid]), dst_rows[pid], table_dev,
                         src_rows);
    } else {
      hipLaunchKernelGGL(scatter_add_rows_kernel<float>, dim3(grid_for_elems(src_rows * dim)),
                         dim3(256), 0, s, src, dim, dev_dst[pid], dst_rows[pid], table_dev,
                         src_rows);
    }
    GR_HIP_CHECK(hipGetLastError());
    if (slot >= 0) {
      int rc = staging_release(slot, s);
      if (rc != GR_OK) return rc;
    }
    return fifo_push(d2h_fifo(), s);
  }

  // Host path: D2H in pinned staging chunks of at most kChunkBytes, each
  // accumulated on the host in row order (self block first, then partitions
  // ascending, indices in order) before the next chunk is fetched.
  std::vector<float*> row_dst((size_t)src_rows);
  for (int64_t r = 0; r < dst_rows[pid]; ++r) row_dst[r] = dsts[pid] + r * dim;
  {
    int64_t o = dst_rows[pid];
    for (int32_t p = 0; p < num_parts; ++p) {
      if (p == pid || boundary_lens[p] <= 0) continue;
      const int64_t* b = boundaries[p];
      for (int64_t k = 0; k < boundary_lens[p]; ++k) row_dst[o++] = dsts[p] + b[k] * dim;
    }
  }
  const int64_t row_bytes = dim * (int64_t)sizeof(float);
  const int64_t rows_per_chunk = std::max<int64_t>(1, kChunkBytes / row_bytes);
  for (int64_t r0 = 0; r0 < src_rows; r0 += rows_per_chunk) {
    const int64_t n = std::min(rows_per_chunk, src_rows - r0);
    void* stage = nullptr;
    int slot = -1;
    int rc = staging_acquire((size_t)(n * row_bytes), &stage, &slot);
    if (rc != GR_OK) return rc;
    hipError_t e = hipMemcpyAsync(stage, src + r0 * dim, (size_t)(n * row_bytes),
                                  hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) {
      staging_release(slot, s);
      return gr::fail(GR_EHIP, "scatter_partitions D2H failed: %s", hipGetErrorString(e));
    }
    const float* g = static_cast<const float*>(stage);
    if (repeated) {
      for (int64_t k = 0; k < n; ++k) {
        float* row = row_dst[r0 + k];
        const float* in = g + k * dim;
        for (int64_t j = 0; j < dim; ++j) row[j] = row[j] + in[j];
      }
    } else {
      parallel_for(n, 1024, [&](int64_t lo, int64_t hi) {
        for (int64_t k = lo; k < hi; ++k) {
          float* row = row_dst[r0 + k];
          const float* in = g + k * dim;
          for (int64_t j = 0; j < dim; ++j) row[j] = row[j] + in[j];
        }
      });
    }
    rc = staging_release(slot, s);
    if (rc != GR_OK) return rc;
  }
  return fifo_push(d2h_fifo(), s);
}

namespace {

// Gives every staging slot a pinned chunk of kChunkBytes, once, before the
// first host partition is pinned: partitions may use up the driver's pinned
// cap, and the slots would then run from pageable memory.  Best effort.
void reserve_staging() {
  static std::once_flag once;
  std::call_once(once, [] {
    void* p[4] = {};
    int ids[4] = {-1, -1, -1, -1};
    for (int k = 0; k < 4; ++k)
      if (staging_acquire((size_t)kChunkBytes, &p[k], &ids[k]) != GR_OK) ids[k] = -1;
    for (int k = 0; k < 4; ++k)
      if (ids[k] >= 0) (void)staging_release(ids[k], nullptr);
    gr::clear_error();
  });
}

}  // namespace

extern "C" int gr_host_alloc(int64_t nbytes, void** out) {
  gr::clear_error();
  GR_REQUIRE(out != nullptr && nbytes >= 0, "host_alloc: bad arguments");
  *out = nullptr;
  if (nbytes == 0) return GR_OK;
  reserve_staging();
  hipError_t e = hipHostMalloc(out, (size_t)nbytes, hipHostMallocDefault);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    *out = nullptr;
    return gr::fail(GR_ENOMEM, "hipHostMalloc(%lld) failed: %s", (long long)nbytes,
                    hipGetErrorString(e));
  }
  return GR_OK;
}

extern "C" int gr_host_free(void* p) {
  gr::clear_error();
  if (p != nullptr) GR_HIP_CHECK(hipHostFree(p));
  return GR_OK;
}
