// Host utilities of libmoert (no device code).
#pragma once
#include <stddef.h>
#include <stdint.h>

#include <atomic>
#include <functional>

namespace moert {

uint16_t host_f2h(float f);
float host_h2f(uint16_t h);
size_t dtype_bytes(int dtype, size_t n);
int quantize(const float* x, size_t n, int dtype, void* out);
int synth_normal(uint64_t seed, uint64_t stream, size_t n, float scale, float offset, float* out);
int synth_quantized(uint64_t seed, uint64_t stream, size_t n, float scale, int dtype, void* out);
int synth_fp16(uint64_t seed, uint64_t stream, size_t n, float scale, uint16_t* out);
// f(begin, end) over [0, n) in chunks of `grain`, on up to 16 threads.
void parallel_for(size_t n, size_t grain, const std::function<void(size_t, size_t)>& f);
// The same on at most `threads` threads (1: the calling thread only).
void parallel_for_n(size_t n, size_t grain, int threads, const std::function<void(size_t, size_t)>& f);

}  // namespace moert
