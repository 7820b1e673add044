// Cold-record reads straight from the split file (cold_weights.bin), the
// native counterpart of ColdWeightStore's mmap and per-record slicing
// (splitter.py:317-403): the requested records of one section are copied,
// in request order, into a caller buffer (normally pinned host memory, from
// which one contiguous hipMemcpyAsync moves them to the device).
//
// Two ways to read:
//   mmap   the file is mapped read-only, as the reference maps it
//          (splitter.py:322-323); each record is one memcpy out of the
//          mapping (the page cache serves warm pages, faults bring in the rest).
//   direct the file is opened with O_DIRECT: records are read by pread of
//          whole 4 KB pages into per-thread aligned bounce buffers, bypassing
//          the page cache, and copied out from there.  Sections start on 4096
//          (splitter.py:250-254) but records are 6400 bytes at 16 + 6400 k, so
//          a record covers two or three pages; records whose page ranges meet
//          or lie within the read gap (16 KB unless set) of each other are read
//          with one pread: on a device bound by its operation rate, reading a
//          gap costs less than another operation.
// A read is split over a fixed pool of threads by contiguous runs of the
// records sorted by file position; each thread plans and issues its own
// reads.  The call returns when every record is in place.  A staged read
// (read, then copy to the device) overlaps the two: the threads take chunks
// of the request in order and the caller enqueues the copy of each finished
// run from the front while the rest are still being read.
#include <errno.h>
#include <fcntl.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>
#include <emmintrin.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <condition_variable>
#include <functional>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include <hip/hip_runtime.h>

#include "oi2.h"

namespace oi2 {
void set_error(const char* fmt, ...);
void clear_error();
}  // namespace oi2

namespace {

constexpr size_t kRec = 6400;          // NEURON_RECORD_BYTES (splitter.py:75-76)
constexpr size_t kHeader = 16;         // <HHIq section header (splitter.py:230)
constexpr size_t kPage = 4096;
constexpr size_t kBounce = 1 << 20;    // per-thread O_DIRECT bounce buffer
constexpr size_t kGapBytes = 16384;    // default gap one O_DIRECT read may span

// A fixed pool: run(n, fn) calls fn(0..n-1) spread over the threads and
// returns when all calls are done.
class Pool {
 public:
  explicit Pool(int n) {
    for (int i = 0; i < n; ++i) workers_.emplace_back([this] { loop(); });
  }
  ~Pool() {
    {
      std::lock_guard<std::mutex> l(mu_);
      stop_ = true;
    }
    cv_.notify_all();
    for (auto& t : workers_) t.join();
  }
  int size() const { return (int)workers_.size(); }
  void run(int n, const std::function<void(int)>& fn) {
    start(n, fn);
    wait();
  }
  // start(n, fn) hands out fn(0..n-1) and returns at once; wait() returns
  // when every call is done.  fn must stay alive until wait() returns.
  void start(int n, const std::function<void(int)>& fn) {
    std::lock_guard<std::mutex> l(mu_);
    fn_ = &fn;
    next_ = 0;
    total_ = n;
    done_ = 0;
    ++gen_;
    cv_.notify_all();
  }
  void wait() {
    std::unique_lock<std::mutex> l(mu_);
    done_cv_.wait(l, [&] { return done_ == total_; });
    fn_ = nullptr;
  }

 private:
  void loop() {
    uint64_t seen = 0;
    std::unique_lock<std::mutex> l(mu_);
    for (;;) {
      cv_.wait(l, [&] { return stop_ || (gen_ != seen && next_ < total_); });
      if (stop_) return;
      while (next_ < total_) {
        const int i = next_++;
        const std::function<void(int)>* fn = fn_;
        l.unlock();
        (*fn)(i);
        l.lock();
        if (++done_ == total_) done_cv_.notify_all();
      }
      seen = gen_;
    }
  }
  std::vector<std::thread> workers_;
  std::mutex mu_;
  std::condition_variable cv_, done_cv_;
  const std::function<void(int)>* fn_ = nullptr;
  int next_ = 0, total_ = 0, done_ = 0;
  uint64_t gen_ = 0;
  bool stop_ = false;
};

}  // namespace

struct oi2_file_store {
  int fd = -1;                        // buffered descriptor (mmap source)
  int dfd = -1;                       // O_DIRECT descriptor (direct mode)
  const uint8_t* map = nullptr;
  size_t size = 0;
  bool direct = false;
  std::vector<uint64_t> sec_off, sec_n;
  std::vector<void*> bounce;          // per part: kBounce bytes, 4096-aligned
  size_t gap = kGapBytes;             // O_DIRECT: largest gap between records one read spans
  Pool* pool = nullptr;
  std::mutex call_mu;                 // one read at a time per handle
};

namespace {

// One record into a 16-byte aligned destination with non-temporal stores:
// a cached store first reads the destination line (for ownership), so a plain
// copy moves each byte over the memory bus three times; streaming stores
// write it once.  On a host where the read and the device copy share the
// memory bandwidth that is a quarter less traffic per staged record.
inline void copy_record_nt(uint8_t* dst, const uint8_t* src) {
  static_assert(kRec % 64 == 0, "whole 64-byte lines");
  __m128i* d = reinterpret_cast<__m128i*>(dst);
  const __m128i* s = reinterpret_cast<const __m128i*>(src);
  for (size_t k = 0; k < kRec / 16; k += 4) {
    const __m128i a = _mm_loadu_si128(s + k), b = _mm_loadu_si128(s + k + 1);
    const __m128i c = _mm_loadu_si128(s + k + 2), e = _mm_loadu_si128(s + k + 3);
    _mm_stream_si128(d + k, a);
    _mm_stream_si128(d + k + 1, b);
    _mm_stream_si128(d + k + 2, c);
    _mm_stream_si128(d + k + 3, e);
  }
}

// Copy out records [b, e) of `order` (indices into slots, sorted by file
// position) from the mapping: streaming stores into a 16-byte aligned
// destination (the whole run fenced at its end), else memcpy.
void read_mapped(oi2_file_store* fs, uint64_t base, const int32_t* slots, const int32_t* order, int b,
                 int e, uint8_t* dst) {
  const bool nt = (reinterpret_cast<uintptr_t>(dst) & 15) == 0;
  for (int k = b; k < e; ++k) {
    const int i = order[k];
    const uint8_t* src = fs->map + base + kHeader + (uint64_t)slots[i] * kRec;
    if (nt)
      copy_record_nt(dst + (size_t)i * kRec, src);
    else
      memcpy(dst + (size_t)i * kRec, src, kRec);
  }
  if (nt) _mm_sfence();
}

// The same with O_DIRECT page reads through this part's bounce buffer.
int read_direct(oi2_file_store* fs, int part, uint64_t base, const int32_t* slots, const int32_t* order,
                int b, int e, uint8_t* dst) {
  uint8_t* buf = static_cast<uint8_t*>(fs->bounce[part]);
  int k = b;
  while (k < e) {
    // one pread: records k .. k2-1 whose page ranges are contiguous (or
    // within fs->gap bytes of each other) and fit the bounce buffer
    const uint64_t first = base + kHeader + (uint64_t)slots[order[k]] * kRec;
    const uint64_t p0 = first / kPage * kPage;
    uint64_t p1 = (first + kRec + kPage - 1) / kPage * kPage;
    int k2 = k + 1;
    while (k2 < e) {
      const uint64_t s = base + kHeader + (uint64_t)slots[order[k2]] * kRec;
      const uint64_t q0 = s / kPage * kPage, q1 = (s + kRec + kPage - 1) / kPage * kPage;
      if (q0 > p1 + fs->gap || q1 - p0 > kBounce) break;
      p1 = std::max(p1, q1);
      ++k2;
    }
    const size_t want = (size_t)(p1 - p0);
    size_t got = 0;
    while (got < want) {
      const ssize_t r = pread(fs->dfd, buf + got, want - got, (off_t)(p0 + got));
      if (r < 0) {
        if (errno == EINTR) continue;
        return errno;
      }
      if (r == 0) break;   // the file ends inside the last page: its tail reads short
      got += (size_t)r;
    }
    for (int j = k; j < k2; ++j) {
      const int i = order[j];
      const uint64_t s = base + kHeader + (uint64_t)slots[i] * kRec;
      if (s + kRec > p0 + got) return EIO;
      memcpy(dst + (size_t)i * kRec, buf + (s - p0), kRec);
    }
    k = k2;
  }
  return 0;
}

void close_store(oi2_file_store* fs) {
  delete fs->pool;
  for (void* b : fs->bounce) free(b);
  if (fs->map) munmap(const_cast<uint8_t*>(fs->map), fs->size);
  if (fs->fd >= 0) close(fs->fd);
  if (fs->dfd >= 0) close(fs->dfd);
  delete fs;
}

}  // namespace

extern "C" {

int oi2_file_store_open(const char* path, const uint64_t* index, int32_t n_sections, int32_t direct_io,
                        int32_t threads, oi2_file_store** out) {
  oi2::clear_error();
  if (!path || !out || (n_sections > 0 && !index) || n_sections < 0) {
    oi2::set_error("file store: null path, index or output, or negative section count");
    return OI2_EINVAL;
  }
  if (threads < 1 || threads > 64) {
    oi2::set_error("file store: threads %d out of range 1 .. 64", threads);
    return OI2_EINVAL;
  }
  auto* fs = new oi2_file_store();
  fs->fd = open(path, O_RDONLY | O_CLOEXEC);
  if (fs->fd < 0) {
    oi2::set_error("file store: cannot open %s: %s", path, strerror(errno));
    close_store(fs);
    return OI2_EINVAL;
  }
  struct stat st;
  if (fstat(fs->fd, &st) != 0) {
    oi2::set_error("file store: cannot stat %s: %s", path, strerror(errno));
    close_store(fs);
    return OI2_EINVAL;
  }
  fs->size = (size_t)st.st_size;
  fs->sec_off.resize(n_sections);
  fs->sec_n.resize(n_sections);
  for (int s = 0; s < n_sections; ++s) {
    fs->sec_off[s] = index[2 * s];
    fs->sec_n[s] = index[2 * s + 1];
    if (fs->sec_n[s] && fs->sec_off[s] + kHeader + fs->sec_n[s] * kRec > fs->size) {
      oi2::set_error("file store: section %d (offset %llu, %llu records) runs past the file's %zu bytes",
                     s, (unsigned long long)fs->sec_off[s], (unsigned long long)fs->sec_n[s], fs->size);
      close_store(fs);
      return OI2_EINVAL;
    }
  }
  fs->direct = direct_io != 0;
  if (fs->direct) {
    fs->dfd = open(path, O_RDONLY | O_DIRECT | O_CLOEXEC);
    if (fs->dfd < 0) {
      oi2::set_error("file store: O_DIRECT open of %s failed: %s", path, strerror(errno));
      close_store(fs);
      return OI2_EUNSUPPORTED;
    }
    for (int t = 0; t < threads; ++t) {
      void* b = nullptr;
      if (posix_memalign(&b, kPage, kBounce) != 0) {
        oi2::set_error("file store: bounce buffer allocation failed");
        close_store(fs);
        return OI2_ENOMEM;
      }
      fs->bounce.push_back(b);
    }
  } else if (fs->size > 0) {
    void* m = mmap(nullptr, fs->size, PROT_READ, MAP_SHARED, fs->fd, 0);
    if (m == MAP_FAILED) {
      oi2::set_error("file store: mmap of %s failed: %s", path, strerror(errno));
      close_store(fs);
      return OI2_EINVAL;
    }
    fs->map = static_cast<const uint8_t*>(m);
  }
  fs->pool = new Pool(threads);
  *out = fs;
  return OI2_OK;
}

}  // extern "C"

namespace {

// Checks a request; OI2_OK, or an error code with the message set.
int check_request(oi2_file_store* fs, int32_t section, const int32_t* slots, int32_t n, const void* dst) {
  if (!fs) {
    oi2::set_error("file store: null handle");
    return OI2_EINVAL;
  }
  if (section < 0 || section >= (int32_t)fs->sec_off.size()) {
    oi2::set_error("file store: section %d out of range (%zu sections)", section, fs->sec_off.size());
    return OI2_EINVAL;
  }
  if (n < 0 || (n > 0 && (!slots || !dst))) {
    oi2::set_error("file store: null slots or destination, or negative count");
    return OI2_EINVAL;
  }
  const uint64_t n_rec = fs->sec_n[section];
  for (int i = 0; i < n; ++i)
    if (slots[i] < 0 || (uint64_t)slots[i] >= n_rec) {
      oi2::set_error("file store: slot %d of item %d outside section %d's %llu records", slots[i], i,
                     section, (unsigned long long)n_rec);
      return OI2_EINVAL;
    }
  return OI2_OK;
}

// Records per chunk of a staged request, and the least a copy moves unless
// it is the request's last.
constexpr int kStageChunkMapped = 32;
constexpr int kStageChunkDirect = 128;   // O_DIRECT: fewer, longer page runs
constexpr size_t kCopyMin = 1 << 20;

}  // namespace

extern "C" {

int oi2_file_store_read(oi2_file_store* fs, int32_t section, const int32_t* slots, int32_t n, uint8_t* dst) {
  oi2::clear_error();
  int rc = check_request(fs, section, slots, n, dst);
  if (rc != OI2_OK || n == 0) return rc;
  std::lock_guard<std::mutex> lock(fs->call_mu);
  // plan: items in file order, split into one contiguous run per thread
  std::vector<int32_t> order(n);
  for (int i = 0; i < n; ++i) order[i] = i;
  std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return slots[a] < slots[b]; });
  const int parts = std::min(fs->pool->size(), n);
  const uint64_t base = fs->sec_off[section];
  std::vector<int> err(parts, 0);
  fs->pool->run(parts, [&](int p) {
    const int b = (int)((int64_t)n * p / parts), e = (int)((int64_t)n * (p + 1) / parts);
    if (fs->direct)
      err[p] = read_direct(fs, p, base, slots, order.data(), b, e, dst);
    else
      read_mapped(fs, base, slots, order.data(), b, e, dst);
  });
  for (int p = 0; p < parts; ++p)
    if (err[p]) {
      oi2::set_error("file store: read of section %d failed: %s", section, strerror(err[p]));
      return OI2_EIO;
    }
  return OI2_OK;
}

// Read and copy overlap: the request is cut into chunks of consecutive items
// (request order), which the pool's threads take in order and read (each
// chunk in file order); this thread enqueues one hipMemcpyAsync for every
// run of finished chunks from the front of the request once the run holds at
// least kCopyMin bytes (or ends the request), so the link carries the first
// records while the later ones are still being read.
int oi2_file_store_stage(oi2_file_store* fs, int32_t section, const int32_t* slots, int32_t n,
                         uint8_t* host_buf, uint8_t* dst, void* stream) {
  oi2::clear_error();
  int rc = check_request(fs, section, slots, n, host_buf);
  if (rc != OI2_OK || n == 0) return rc;
  if (!dst) {
    oi2::set_error("file store: null device destination");
    return OI2_EINVAL;
  }
  std::lock_guard<std::mutex> lock(fs->call_mu);
  const int K = fs->direct ? kStageChunkDirect : kStageChunkMapped;
  const int n_chunks = (n + K - 1) / K;
  std::vector<int32_t> order(n);
  for (int i = 0; i < n; ++i) order[i] = i;
  for (int c = 0; c < n_chunks; ++c)
    std::stable_sort(order.begin() + (size_t)c * K, order.begin() + std::min(n, (c + 1) * K),
                     [&](int a, int b) { return slots[a] < slots[b]; });
  const uint64_t base = fs->sec_off[section];
  const int parts = std::min(fs->pool->size(), n_chunks);
  std::vector<int> err(parts, 0);
  std::vector<uint8_t> done(n_chunks, 0);   // guarded by mu
  std::atomic<int> next{0};
  std::mutex mu;
  std::condition_variable cv;
  const std::function<void(int)> fn = [&](int p) {
    for (int c; (c = next.fetch_add(1)) < n_chunks;) {
      const int b = c * K, e = std::min(n, b + K);
      int r = 0;
      if (fs->direct)
        r = read_direct(fs, p, base, slots, order.data(), b, e, host_buf);
      else
        read_mapped(fs, base, slots, order.data(), b, e, host_buf);
      if (r && !err[p]) err[p] = r;
      {
        std::lock_guard<std::mutex> l(mu);
        done[c] = 1;
      }
      cv.notify_one();
    }
  };
  fs->pool->start(parts, fn);
  hipError_t he = hipSuccess;
  for (int copied = 0; copied < n_chunks;) {
    int e = copied;
    {
      std::unique_lock<std::mutex> l(mu);
      cv.wait(l, [&] {
        while (e < n_chunks && done[e]) ++e;
        return e == n_chunks || (size_t)(e - copied) * K * kRec >= kCopyMin;
      });
    }
    const size_t b0 = (size_t)copied * K * kRec, b1 = (size_t)std::min(n, e * K) * kRec;
    if (he == hipSuccess)
      he = hipMemcpyAsync(dst + b0, host_buf + b0, b1 - b0, hipMemcpyHostToDevice, (hipStream_t)stream);
    copied = e;
  }
  fs->pool->wait();
  for (int p = 0; p < parts; ++p)
    if (err[p]) {
      oi2::set_error("file store: read of section %d failed: %s", section, strerror(err[p]));
      return OI2_EIO;
    }
  if (he != hipSuccess) {
    oi2::set_error("file store: hipMemcpyAsync of %d records failed: %s", n, hipGetErrorString(he));
    return OI2_EHIP;
  }
  return OI2_OK;
}

int oi2_file_store_set_read_gap(oi2_file_store* fs, int64_t bytes) {
  oi2::clear_error();
  if (!fs || bytes < 0 || bytes > (int64_t)(kBounce / 2)) {
    oi2::set_error("file store: null handle or read gap %lld outside 0 .. %zu", (long long)bytes,
                   kBounce / 2);
    return OI2_EINVAL;
  }
  fs->gap = (size_t)bytes;
  return OI2_OK;
}

int oi2_file_store_close(oi2_file_store* fs) {
  oi2::clear_error();
  if (fs) close_store(fs);
  return OI2_OK;
}

}  // extern "C"
