// Host <-> storage I/O engine (the role of the reference's IoUringEngine,
// csrc/cpu/io_uring_engine.cpp:15-245): asynchronous whole-buffer reads and
// writes of files, identified by integer handles, with wait / poll /
// wait_all / pending.
//
// liburing is not available here, so requests run on a pool of worker
// threads with pread/pwrite.  A request is cut into chunks of kChunkBytes
// that the workers process in parallel (NVMe drives want many requests in
// flight); the request completes when its last chunk does.  A failing chunk
// (open, short read, I/O error) records its message, and wait() returns it
// as an error instead of throwing or swallowing it.
//
// Writes create or truncate the file to the request's end, as the
// reference's O_TRUNC open does, so a file holds exactly the bytes written:
// raw row-major data, no header.
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <condition_variable>
#include <cstring>
#include <deque>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "gr_internal.h"

namespace gr_io {

constexpr int64_t kChunkBytes = 8 << 20;

struct Request {
  int fd = -1;
  bool write = false;
  char* buf = nullptr;
  int64_t offset = 0;
  int64_t nbytes = 0;
  std::string path;
  int64_t chunks_left = 0;  // guarded by Engine::mu
  bool done = false;        // guarded by Engine::mu
  std::string error;        // guarded by Engine::mu (first failure)
};

struct Chunk {
  std::shared_ptr<Request> req;
  int64_t begin, end;       // byte range within the request
};

class Engine {
 public:
  explicit Engine(int threads) {
    for (int i = 0; i < threads; ++i) workers_.emplace_back([this] { run(); });
  }

  ~Engine() {
    {
      std::lock_guard<std::mutex> lock(mu);
      stop_ = true;
    }
    work_cv_.notify_all();
    for (auto& t : workers_) t.join();
    for (auto& kv : requests_) close_fd(*kv.second);
  }

  int submit(bool write, const char* path, void* buf, int64_t offset, int64_t nbytes,
             int64_t* handle) {
    auto req = std::make_shared<Request>();
    req->write = write;
    req->buf = static_cast<char*>(buf);
    req->offset = offset;
    req->nbytes = nbytes;
    req->path = path;
    req->fd = write ? ::open(path, O_WRONLY | O_CREAT | O_TRUNC | O_CLOEXEC, 0644)
                    : ::open(path, O_RDONLY | O_CLOEXEC);
    if (req->fd < 0)
      return gr::fail(GR_EINVAL, "io engine: cannot open %s for %s: %s", path,
                      write ? "writing" : "reading", std::strerror(errno));
    if (write && ::ftruncate(req->fd, offset + nbytes) != 0) {
      const int e = errno;
      ::close(req->fd);
      return gr::fail(GR_EINVAL, "io engine: cannot size %s: %s", path, std::strerror(e));
    }
    const int64_t n_chunks = nbytes == 0 ? 0 : (nbytes + kChunkBytes - 1) / kChunkBytes;
    std::lock_guard<std::mutex> lock(mu);
    req->chunks_left = n_chunks;
    const int64_t h = next_handle_++;
    requests_[h] = req;
    if (n_chunks == 0) {
      req->done = true;
      close_fd(*req);
    }
    for (int64_t c = 0; c < n_chunks; ++c)
      queue_.push_back(Chunk{req, c * kChunkBytes, std::min(nbytes, (c + 1) * kChunkBytes)});
    *handle = h;
    work_cv_.notify_all();
    return GR_OK;
  }

  // Blocks until the request is done; forgets it; reports its error.
  int wait(int64_t h) {
    std::unique_lock<std::mutex> lock(mu);
    auto it = requests_.find(h);
    if (it == requests_.end())
      return gr::fail(GR_EINVAL, "io engine: unknown or already waited handle %lld",
                      (long long)h);
    std::shared_ptr<Request> req = it->second;
    done_cv_.wait(lock, [&] { return req->done; });
    requests_.erase(h);
    if (!req->error.empty()) return gr::fail(GR_EINVAL, "%s", req->error.c_str());
    return GR_OK;
  }

  int wait_all() {
    std::vector<int64_t> handles;
    {
      std::lock_guard<std::mutex> lock(mu);
      for (auto& kv : requests_) handles.push_back(kv.first);
    }
    int rc = GR_OK;
    std::string first_error;
    for (int64_t h : handles) {
      const int r = wait(h);
      if (r != GR_OK && rc == GR_OK) {
        rc = r;
        first_error = gr::last_error_cstr();
      }
    }
    if (rc != GR_OK) return gr::fail(rc, "%s", first_error.c_str());
    return GR_OK;
  }

  int poll(int64_t h, int32_t* done) {
    std::lock_guard<std::mutex> lock(mu);
    auto it = requests_.find(h);
    if (it == requests_.end())
      return gr::fail(GR_EINVAL, "io engine: unknown or already waited handle %lld",
                      (long long)h);
    *done = it->second->done ? 1 : 0;
    return GR_OK;
  }

  int64_t pending() {
    std::lock_guard<std::mutex> lock(mu);
    int64_t n = 0;
    for (auto& kv : requests_)
      if (!kv.second->done) ++n;
    return n;
  }


 private:
  static void close_fd(Request& r) {
    if (r.fd >= 0) {
      ::close(r.fd);
      r.fd = -1;
    }
  }

  void run() {
    for (;;) {
      Chunk c;
      {
        std::unique_lock<std::mutex> lock(mu);
        work_cv_.wait(lock, [&] { return stop_ || !queue_.empty(); });
        if (queue_.empty()) return;  // stopping and drained
        c = std::move(queue_.front());
        queue_.pop_front();
      }
      std::string err = transfer(c);
      // A chunk publishes its result and its completion under one lock, so
      // the request is marked done only after every chunk's error (if any)
      // is recorded, and wait() sees the first failure.
      std::lock_guard<std::mutex> lock(mu);
      if (!err.empty() && c.req->error.empty()) c.req->error = std::move(err);
      if (--c.req->chunks_left == 0) {
        c.req->done = true;
        close_fd(*c.req);
        done_cv_.notify_all();
      }
    }
  }

  static std::string transfer(const Chunk& c) {
    Request& r = *c.req;
    int64_t pos = c.begin;
    while (pos < c.end) {
      const size_t want = (size_t)std::min<int64_t>(c.end - pos, 1 << 30);
      const ssize_t got = r.write ? ::pwrite(r.fd, r.buf + pos, want, r.offset + pos)
                                  : ::pread(r.fd, r.buf + pos, want, r.offset + pos);
      if (got < 0) {
        if (errno == EINTR) continue;
        return "io engine: " + std::string(r.write ? "write to " : "read from ") + r.path +
               " failed: " + std::strerror(errno);
      }
      if (got == 0)
        return "io engine: " + r.path + " is shorter than the " + std::to_string(r.nbytes) +
               " bytes requested at offset " + std::to_string(r.offset);
      pos += got;
    }
    return std::string();
  }

  std::mutex mu;
  std::vector<std::thread> workers_;
  std::deque<Chunk> queue_;
  std::condition_variable work_cv_, done_cv_;
  std::unordered_map<int64_t, std::shared_ptr<Request>> requests_;
  int64_t next_handle_ = 0;
  bool stop_ = false;
};

Engine* as_engine(void* e) { return static_cast<Engine*>(e); }

}  // namespace gr_io

extern "C" int gr_io_create(int32_t threads, void** engine) {
  gr::clear_error();
  GR_REQUIRE(engine != nullptr, "io_create: NULL output");
  GR_REQUIRE(threads >= 1 && threads <= 256, "io_create: threads %d outside [1, 256]",
             threads);
  try {
    *engine = new gr_io::Engine(threads);
  } catch (const std::exception& e) {
    return gr::fail(GR_ENOMEM, "io_create: %s", e.what());
  }
  return GR_OK;
}

extern "C" int gr_io_destroy(void* engine) {
  gr::clear_error();
  if (engine == nullptr) return GR_OK;
  gr_io::Engine* e = gr_io::as_engine(engine);
  const int rc = e->wait_all();
  delete e;
  return rc;
}

extern "C" int gr_io_submit(void* engine, int32_t write, const char* path, void* buf,
                            int64_t offset, int64_t nbytes, int64_t* handle) {
  gr::clear_error();
  GR_REQUIRE(engine != nullptr && path != nullptr && handle != nullptr,
             "io_submit: NULL engine, path or handle");
  GR_REQUIRE(offset >= 0 && nbytes >= 0, "io_submit: negative offset or size");
  GR_REQUIRE(nbytes == 0 || buf != nullptr, "io_submit: NULL buffer");
  return gr_io::as_engine(engine)->submit(write != 0, path, buf, offset, nbytes, handle);
}

extern "C" int gr_io_wait(void* engine, int64_t handle) {
  gr::clear_error();
  GR_REQUIRE(engine != nullptr, "io_wait: NULL engine");
  return gr_io::as_engine(engine)->wait(handle);
}

extern "C" int gr_io_wait_all(void* engine) {
  gr::clear_error();
  GR_REQUIRE(engine != nullptr, "io_wait_all: NULL engine");
  return gr_io::as_engine(engine)->wait_all();
}

extern "C" int gr_io_poll(void* engine, int64_t handle, int32_t* done) {
  gr::clear_error();
  GR_REQUIRE(engine != nullptr && done != nullptr, "io_poll: NULL engine or output");
  return gr_io::as_engine(engine)->poll(handle, done);
}

extern "C" int gr_io_pending(void* engine, int64_t* count) {
  gr::clear_error();
  GR_REQUIRE(engine != nullptr && count != nullptr, "io_pending: NULL engine or output");
  *count = gr_io::as_engine(engine)->pending();
  return GR_OK;
}
