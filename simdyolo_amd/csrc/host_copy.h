// Host-side copies between pageable caller buffers and pinned staging
// memory, shared by the context's staged copies and the model's host-buffer
// pipeline.
#pragma once

#include <algorithm>
#include <atomic>
#include <condition_variable>
#include <cstdint>
#include <cstring>
#include <mutex>
#include <thread>
#include <vector>

namespace sy {

// Host threads that split large memcpys between pageable caller buffers and
// pinned staging (one thread reaches about a quarter of the host's copy
// bandwidth).  copy() hands each worker a contiguous part, copies the first
// part itself and returns when every part is done.
class CopyPool {
 public:
  explicit CopyPool(int workers) {
    for (int i = 0; i < workers; ++i) threads_.emplace_back([this, i] { loop(i); });
  }
  ~CopyPool() {
    {
      std::lock_guard<std::mutex> lock(mu_);
      stop_ = true;
      ++gen_;
    }
    cv_.notify_all();
    for (auto& t : threads_) t.join();
  }
  void copy(void* dst, const void* src, size_t bytes) { run((char*)dst, (const char*)src, bytes); }
  // Writes one byte of every page of [dst, dst + bytes): a freshly allocated
  // caller buffer takes its page faults here, in parallel and while the GPU
  // works, instead of inside the copy that fills it later.
  void touch(void* dst, size_t bytes) { run((char*)dst, nullptr, bytes); }

 private:
  static void part_job(char* d, const char* s, size_t n) {
    if (s) {
      memcpy(d, s, n);
    } else {
      for (size_t off = 0; off < n; off += 4096) ((volatile char*)d)[off] = 0;
      if (n) ((volatile char*)d)[n - 1] = 0;
    }
  }
  void run(char* dst, const char* src, size_t bytes) {
    const size_t parts = threads_.size() + 1;
    if (bytes < (size_t(1) << 20) || parts == 1) {
      part_job(dst, src, bytes);
      return;
    }
    // Page-multiple parts that together cover every byte (a part of the
    // floor quotient rounded up could end parts * part short of bytes).
    const size_t part = ((bytes + parts - 1) / parts + 4095) & ~size_t(4095);
    {
      std::lock_guard<std::mutex> lock(mu_);
      dst_ = dst;
      src_ = src;
      bytes_ = bytes;
      part_ = part;
      pending_.store((int)threads_.size(), std::memory_order_relaxed);
      ++gen_;
    }
    cv_.notify_all();
    part_job(dst, src, std::min(part, bytes));
    while (pending_.load(std::memory_order_acquire) > 0) std::this_thread::yield();
  }
  void loop(int i) {
    uint64_t seen = 0;
    for (;;) {
      char* d;
      const char* s;
      size_t n, part;
      {
        std::unique_lock<std::mutex> lock(mu_);
        cv_.wait(lock, [&] { return gen_ != seen; });
        seen = gen_;
        if (stop_) return;
        d = dst_;
        s = src_;
        n = bytes_;
        part = part_;
      }
      const size_t lo = std::min(n, (size_t)(i + 1) * part), hi = std::min(n, (size_t)(i + 2) * part);
      if (hi > lo) part_job(d + lo, s ? s + lo : nullptr, hi - lo);
      pending_.fetch_sub(1, std::memory_order_release);
    }
  }
  std::vector<std::thread> threads_;
  std::mutex mu_;
  std::condition_variable cv_;
  uint64_t gen_ = 0;
  bool stop_ = false;
  char* dst_ = nullptr;
  const char* src_ = nullptr;
  size_t bytes_ = 0, part_ = 0;
  std::atomic<int> pending_{0};
};

}  // namespace sy
