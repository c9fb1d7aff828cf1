// Asynchronous file I/O of the HKV NVMe tier (host code). A spill or reload moves a list of host
// buffers to or from one file, each buffer at a 4 KiB-aligned offset, on a worker thread, with
// O_DIRECT when the file system takes it: page-aligned buffers go straight to the device, other
// buffers, 4 KiB tails and buffers the kernel cannot pin (EFAULT: GPU-registered host memory)
// through an aligned bounce buffer. The file is opened (created) by the
// caller's thread, so it exists when the call returns; errors of the transfer are reported by
// wa_io_wait.
//
// Reference semantics: pipeline/hkv/tiering.py:89-105 (torch.save / torch.load of a chunk blob).
#include <errno.h>
#include <fcntl.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "common.h"

namespace {

constexpr int64_t kAlign = 4096;
constexpr int64_t kBounce = 8 << 20;

int64_t round_up(int64_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

struct IoJob {
  std::thread worker;
  std::atomic<int> finished{0};
  int rc = WA_OK;
  std::string err;
  int direct = 0;
  ~IoJob() {
    if (worker.joinable()) worker.join();  // a transfer nobody waited for still completes
  }
};

std::mutex g_mu;
std::map<int64_t, std::shared_ptr<IoJob>> g_jobs;
int64_t g_next = 1;

// Move exactly `n` bytes at `off` (retrying short transfers and interrupts). With `efault`, an
// EFAULT (a buffer the kernel cannot pin for direct I/O, e.g. GPU-registered host memory) is
// reported there instead of as an error.
bool xfer(int fd, bool write, char* p, int64_t n, int64_t off, std::string& err, bool* efault = nullptr) {
  while (n > 0) {
    const ssize_t r = write ? pwrite(fd, p, (size_t)n, (off_t)off) : pread(fd, p, (size_t)n, (off_t)off);
    if (r < 0 && errno == EINTR) continue;
    if (r < 0 && errno == EFAULT && efault) {
      *efault = true;
      return false;
    }
    if (r <= 0) {
      err = std::string(write ? "write" : "read") + " failed at offset " + std::to_string(off) + ": " +
            (r < 0 ? strerror(errno) : "unexpected end of file");
      return false;
    }
    p += r;
    n -= r;
    off += r;
  }
  return true;
}

void run_job(IoJob* job, int fd, bool write, std::vector<char*> bufs, std::vector<int64_t> sizes) {
  char* bounce = nullptr;
  std::string err;
  bool ok = true;
  if (job->direct && posix_memalign((void**)&bounce, (size_t)kAlign, (size_t)kBounce) != 0) {
    ok = false;
    err = "no memory for the bounce buffer";
  }
  int64_t off = 0;
  bool bounce_all = false;  // set once a buffer refused direct transfers
  for (size_t i = 0; ok && i < bufs.size(); ++i) {
    char* b = bufs[i];
    const int64_t size = sizes[i];
    int64_t done = 0;
    if (!job->direct) {
      ok = xfer(fd, write, b, size, off, err);
    } else {
      if (!bounce_all && ((uintptr_t)b % kAlign) == 0) {
        const int64_t body = size / kAlign * kAlign;
        bool efault = false;
        ok = xfer(fd, write, b, body, off, err, &efault);
        done = body;
        if (efault) {  // redo the whole buffer through the bounce buffer
          ok = true;
          done = 0;
          bounce_all = true;
        }
      }
      while (ok && done < size) {
        const int64_t piece = std::min(size - done, kBounce), padded = round_up(piece);
        if (write) {
          memcpy(bounce, b + done, (size_t)piece);
          memset(bounce + piece, 0, (size_t)(padded - piece));
          ok = xfer(fd, true, bounce, padded, off + done, err);
        } else {
          ok = xfer(fd, false, bounce, padded, off + done, err);
          if (ok) memcpy(b + done, bounce, (size_t)piece);
        }
        done += piece;
      }
    }
    off += round_up(size);
  }
  if (ok && write && !job->direct) {
    // keep the buffered file the same length as a direct one (whole 4 KiB pieces)
    if (ftruncate(fd, (off_t)off) != 0) {
      ok = false;
      err = std::string("ftruncate failed: ") + strerror(errno);
    }
  }
  free(bounce);
  close(fd);
  if (!ok) {
    job->rc = WA_ERR_IO;
    job->err = err;
  }
  job->finished.store(1);
}

int64_t start_job(const char* path, bool write, const void* const* bufs, const int64_t* sizes, int64_t n,
                  int32_t direct) {
  WA_CHECK_ARG(path && (n == 0 || (bufs && sizes)) && n >= 0, "wa_io: null argument");
  for (int64_t i = 0; i < n; ++i)
    WA_CHECK_ARG(sizes[i] >= 0 && (sizes[i] == 0 || bufs[i]), "wa_io: buffer %lld is null", (long long)i);
  const int base = write ? (O_WRONLY | O_CREAT | O_TRUNC) : O_RDONLY;
  int fd = -1, used_direct = 0;
  if (direct) {
    fd = open(path, base | O_DIRECT, 0644);
    if (fd >= 0) used_direct = 1;
  }
  if (fd < 0) fd = open(path, base, 0644);  // the file system refuses O_DIRECT: buffered I/O
  if (fd < 0) return wa_fail(WA_ERR_IO, "wa_io: cannot open %s: %s", path, strerror(errno));
  auto job = std::make_shared<IoJob>();
  job->direct = used_direct;
  std::vector<char*> b((size_t)n);
  std::vector<int64_t> s((size_t)n);
  for (int64_t i = 0; i < n; ++i) {
    b[(size_t)i] = (char*)bufs[i];
    s[(size_t)i] = sizes[i];
  }
  int64_t handle;
  {
    std::lock_guard<std::mutex> lock(g_mu);
    handle = g_next++;
    g_jobs[handle] = job;
  }
  job->worker = std::thread(run_job, job.get(), fd, write, std::move(b), std::move(s));
  return handle;
}

std::shared_ptr<IoJob> find_job(int64_t handle) {
  std::lock_guard<std::mutex> lock(g_mu);
  auto it = g_jobs.find(handle);
  return it == g_jobs.end() ? nullptr : it->second;
}

}  // namespace

extern "C" int64_t wa_io_write_async(const char* path, const void* const* bufs, const int64_t* sizes, int64_t n,
                                     int32_t direct) {
  return start_job(path, true, bufs, sizes, n, direct);
}

extern "C" int64_t wa_io_read_async(const char* path, void* const* bufs, const int64_t* sizes, int64_t n,
                                    int32_t direct) {
  return start_job(path, false, (const void* const*)bufs, sizes, n, direct);
}

extern "C" int wa_io_done(int64_t handle) {
  auto job = find_job(handle);
  WA_CHECK_ARG(job != nullptr, "wa_io_done: unknown handle %lld", (long long)handle);
  return job->finished.load();
}

extern "C" int wa_io_direct(int64_t handle) {
  auto job = find_job(handle);
  WA_CHECK_ARG(job != nullptr, "wa_io_direct: unknown handle %lld", (long long)handle);
  return job->direct;
}

extern "C" int wa_io_wait(int64_t handle) {
  std::shared_ptr<IoJob> job;
  {
    std::lock_guard<std::mutex> lock(g_mu);
    auto it = g_jobs.find(handle);
    WA_CHECK_ARG(it != g_jobs.end(), "wa_io_wait: unknown handle %lld", (long long)handle);
    job = it->second;
    g_jobs.erase(it);
  }
  if (job->worker.joinable()) job->worker.join();
  if (job->rc != WA_OK) return wa_fail(job->rc, "wa_io: %s", job->err.c_str());
  return WA_OK;
}
