// Host utilities of libmoert: GGML Q8_0/Q4_0 quantisers, fp16 rounding, and the seeded synthetic-data
// generator used to build random-init models (no device code).
#include <algorithm>
#include <cmath>
#include <condition_variable>
#include <cstring>
#include <memory>
#include <mutex>
#include <thread>
#include <vector>

#include "host_utils.h"

namespace moert {

uint16_t host_f2h(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  uint16_t sign = (uint16_t)((x >> 16) & 0x8000);
  uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) return sign | 0x7c00 | (ax > 0x7f800000u ? 0x200 : 0);
  if (ax >= 0x477ff000u) return sign | 0x7c00;
  if (ax < 0x38800000u) {
    float a;
    std::memcpy(&a, &ax, 4);
    return sign | (uint16_t)std::nearbyint(a * 16777216.0f);
  }
  uint32_t h = (((ax >> 23) - 112) << 10) | ((ax & 0x7fffffu) >> 13);
  uint32_t rem = ax & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
  return sign | (uint16_t)h;
}

float host_h2f(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000) << 16, e = (h >> 10) & 31, m = h & 1023, u;
  if (e == 0) {
    float v = (float)m * 5.9604644775390625e-8f;
    return sign ? -v : v;
  }
  if (e == 31)
    u = sign | 0x7f800000u | (m << 13);
  else
    u = sign | ((e + 112) << 23) | (m << 13);
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

size_t dtype_bytes(int dtype, size_t n) {
  if (dtype == 1) return n / 32 * 34;
  if (dtype == 2) return n / 32 * 18;
  return n * 4;
}

// GGML Q8_0: d = amax / 127, q = round(x / d) (x * (1/d), rounded half away from zero), d stored as fp16.
void quantize_q8_0_block(const float* x, uint8_t* out) {
  float amax = 0.0f;
  for (int i = 0; i < 32; i++) amax = std::max(amax, std::fabs(x[i]));
  float d = amax / 127.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
  uint16_t dh = host_f2h(d);
  out[0] = (uint8_t)(dh & 0xff);
  out[1] = (uint8_t)(dh >> 8);
  for (int i = 0; i < 32; i++) {
    float v = std::round(x[i] * id);
    v = std::min(127.0f, std::max(-127.0f, v));
    out[2 + i] = (uint8_t)(int8_t)v;
  }
}

// GGML Q4_0: m = the element of largest magnitude (with its sign), d = m / -8, q = clamp(round(x / d) + 8, 0, 15);
// byte i holds element i (low nibble) and element i + 16 (high nibble).
void quantize_q4_0_block(const float* x, uint8_t* out) {
  float amax = 0.0f, mx = 0.0f;
  for (int i = 0; i < 32; i++)
    if (std::fabs(x[i]) > amax) {
      amax = std::fabs(x[i]);
      mx = x[i];
    }
  float d = mx / -8.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
  uint16_t dh = host_f2h(d);
  out[0] = (uint8_t)(dh & 0xff);
  out[1] = (uint8_t)(dh >> 8);
  for (int i = 0; i < 16; i++) {
    int a = (int)std::round(x[i] * id) + 8, b = (int)std::round(x[16 + i] * id) + 8;
    a = std::min(15, std::max(0, a));
    b = std::min(15, std::max(0, b));
    out[2 + i] = (uint8_t)(a | (b << 4));
  }
}

int quantize(const float* x, size_t n, int dtype, void* out) {
  if (n % 32) return -2;
  uint8_t* o = (uint8_t*)out;
  if (dtype == 1)
    for (size_t b = 0; b < n / 32; b++) quantize_q8_0_block(x + b * 32, o + b * 34);
  else if (dtype == 2)
    for (size_t b = 0; b < n / 32; b++) quantize_q4_0_block(x + b * 32, o + b * 18);
  else if (dtype == 0)
    std::memcpy(out, x, n * 4);
  else
    return -2;
  return 0;
}

static inline uint64_t splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

// Element i of stream `stream`: Box-Muller on the pair (i/2) of two counter-based uniforms; even i takes the
// cosine branch, odd i the sine branch. Any sub-range is reproducible on its own.
static void normal_range(uint64_t seed, uint64_t stream, size_t i0, size_t i1, float scale, float offset, float* out) {
  uint64_t key = splitmix64(seed ^ splitmix64(stream + 0x5851F42D4C957F2Dull));
  for (size_t i = i0; i < i1;) {
    size_t k = i / 2;
    uint64_t a = splitmix64(key + 2 * k), b = splitmix64(key + 2 * k + 1);
    double u1 = ((double)(a >> 11) + 0.5) * (1.0 / 9007199254740992.0);
    double u2 = (double)(b >> 11) * (1.0 / 9007199254740992.0);
    double r = std::sqrt(-2.0 * std::log(u1)), t = 6.283185307179586 * u2;
    if ((i & 1) == 0) {
      out[i - i0] = (float)(r * std::cos(t)) * scale + offset;
      i++;
      if (i < i1) {
        out[i - i0] = (float)(r * std::sin(t)) * scale + offset;
        i++;
      }
    } else {
      out[i - i0] = (float)(r * std::sin(t)) * scale + offset;
      i++;
    }
  }
}

void parallel_for(size_t n, size_t grain, const std::function<void(size_t, size_t)>& f) {
  unsigned hw = std::thread::hardware_concurrency();
  parallel_for_n(n, grain, (int)std::min<unsigned>(hw ? hw : 1, 16), f);
}

namespace {

// Worker threads that live for the process, so that a parallel loop costs a wake-up, not thread creation. One loop
// runs at a time; the caller works on it too. Each loop has its own chunk counters, so a worker that wakes late for
// an earlier loop finds its chunks taken and never calls that loop's function.
struct Job {
  const std::function<void(size_t, size_t)>* f;
  size_t n, grain, chunks;
  int limit;  // workers with id + 1 < limit take part (the caller is the last participant)
  std::atomic<size_t> next{0}, done{0};
};

class Workers {
 public:
  static Workers& get() {
    static Workers* w = new Workers();  // never destroyed: the threads sleep until the process ends
    return *w;
  }
  int size() const { return (int)threads_.size(); }

  void run(size_t n, size_t grain, int threads, const std::function<void(size_t, size_t)>& f) {
    std::lock_guard<std::mutex> one(run_mu_);
    auto job = std::make_shared<Job>();
    job->f = &f;
    job->n = n;
    job->grain = grain;
    job->chunks = (n + grain - 1) / grain;
    job->limit = threads;
    {
      std::lock_guard<std::mutex> l(mu_);
      cur_ = job;
      gen_++;
    }
    cv_.notify_all();
    work(*job);
    std::unique_lock<std::mutex> l(mu_);
    done_cv_.wait(l, [&] { return job->done.load() == job->chunks; });
  }

 private:
  Workers() {
    const unsigned hw = std::thread::hardware_concurrency();
    const int n = (int)std::min<unsigned>(hw ? hw : 1, 64) - 1;
    for (int i = 0; i < n; i++) threads_.emplace_back([this, i] { loop(i); });
    for (auto& t : threads_) t.detach();
  }

  void work(Job& j) {
    for (size_t c; (c = j.next.fetch_add(1)) < j.chunks;) {
      (*j.f)(c * j.grain, std::min(j.n, (c + 1) * j.grain));
      if (j.done.fetch_add(1) + 1 == j.chunks) {
        std::lock_guard<std::mutex> l(mu_);
        done_cv_.notify_all();
      }
    }
  }

  void loop(int id) {
    uint64_t seen = 0;
    for (;;) {
      std::shared_ptr<Job> job;
      {
        std::unique_lock<std::mutex> l(mu_);
        cv_.wait(l, [&] { return gen_ != seen; });
        seen = gen_;
        job = cur_;
      }
      if (id + 1 < job->limit) work(*job);
    }
  }

  std::mutex run_mu_, mu_;
  std::condition_variable cv_, done_cv_;
  std::shared_ptr<Job> cur_;
  uint64_t gen_ = 0;
  std::vector<std::thread> threads_;
};

}  // namespace

void parallel_for_n(size_t n, size_t grain, int threads, const std::function<void(size_t, size_t)>& f) {
  const size_t chunks = (n + grain - 1) / grain;
  if (threads <= 1 || chunks <= 1) {
    f(0, n);
    return;
  }
  Workers& w = Workers::get();
  w.run(n, grain, std::min(threads, w.size() + 1), f);
}

int synth_normal(uint64_t seed, uint64_t stream, size_t n, float scale, float offset, float* out) {
  parallel_for(n, 1 << 16, [&](size_t a, size_t b) { normal_range(seed, stream, a, b, scale, offset, out + a); });
  return 0;
}

int synth_quantized(uint64_t seed, uint64_t stream, size_t n, float scale, int dtype, void* out) {
  if (n % 32) return -2;
  if (dtype == 0) return synth_normal(seed, stream, n, scale, 0.0f, (float*)out);
  size_t bb = dtype == 1 ? 34 : 18;
  parallel_for(n, 1 << 16, [&](size_t a, size_t b) {
    std::vector<float> tmp(b - a);
    normal_range(seed, stream, a, b, scale, 0.0f, tmp.data());
    uint8_t* o = (uint8_t*)out + a / 32 * bb;
    for (size_t k = 0; k < (b - a) / 32; k++) {
      if (dtype == 1)
        quantize_q8_0_block(tmp.data() + k * 32, o + k * bb);
      else
        quantize_q4_0_block(tmp.data() + k * 32, o + k * bb);
    }
  });
  return 0;
}

int synth_fp16(uint64_t seed, uint64_t stream, size_t n, float scale, uint16_t* out) {
  parallel_for(n, 1 << 16, [&](size_t a, size_t b) {
    std::vector<float> tmp(b - a);
    normal_range(seed, stream, a, b, scale, 0.0f, tmp.data());
    for (size_t k = 0; k < b - a; k++) out[a + k] = host_f2h(tmp[k]);
  });
  return 0;
}

}  // namespace moert
