// Fixed set of worker threads over an atomic task counter (rust/moe-rt/src/pool.rs:96-199), shared by the oracle
// (oracle.cpp) and the CPU port (cpu_port.cpp). Test infrastructure only.
#pragma once
#include <atomic>
#include <condition_variable>
#include <cstdint>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

namespace orc {

// The caller works too; run() returns once every task has ended.
class Pool {
 public:
  explicit Pool(int threads) {
    for (int i = 1; i < threads; i++) ws_.emplace_back([this] { worker(); });
  }
  ~Pool() {
    {
      std::lock_guard<std::mutex> l(mu_);
      stop_ = true;
    }
    cv_.notify_all();
    for (auto& t : ws_) t.join();
  }
  int threads() const { return (int)ws_.size() + 1; }
  void run(size_t n, const std::function<void(size_t)>& f) {
    if (ws_.empty() || n <= 1) {
      for (size_t i = 0; i < n; i++) f(i);
      return;
    }
    {
      std::lock_guard<std::mutex> l(mu_);
      f_ = &f;
      n_ = n;
      next_.store(0);
      busy_ = (int)ws_.size();
      gen_++;
    }
    cv_.notify_all();
    for (size_t i; (i = next_.fetch_add(1)) < n;) f(i);
    std::unique_lock<std::mutex> l(mu_);
    done_.wait(l, [&] { return busy_ == 0; });
    f_ = nullptr;
  }

 private:
  void worker() {
    uint64_t seen = 0;
    for (;;) {
      const std::function<void(size_t)>* f;
      size_t n;
      {
        std::unique_lock<std::mutex> l(mu_);
        cv_.wait(l, [&] { return stop_ || gen_ != seen; });
        if (stop_) return;
        seen = gen_;
        f = f_;
        n = n_;
      }
      for (size_t i; (i = next_.fetch_add(1)) < n;) (*f)(i);
      std::lock_guard<std::mutex> l(mu_);
      if (--busy_ == 0) done_.notify_one();
    }
  }
  std::vector<std::thread> ws_;
  std::mutex mu_;
  std::condition_variable cv_, done_;
  const std::function<void(size_t)>* f_ = nullptr;
  size_t n_ = 0;
  std::atomic<size_t> next_{0};
  int busy_ = 0;
  uint64_t gen_ = 0;
  bool stop_ = false;
};

}  // namespace orc
