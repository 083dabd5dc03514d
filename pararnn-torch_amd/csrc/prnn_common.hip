// Library-wide pieces of the C ABI: error buffer, ABI version, word clear,
// deterministic mode.
#include <atomic>
#include <mutex>

#include "prnn_host.h"

namespace prnn {

char* last_error_buffer() {
  static thread_local char buf[512] = {0};
  return buf;
}

__global__ void clear_words_kernel(int* __restrict__ p, size_t n) {
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
    p[i] = 0;
}

namespace {
std::atomic<int> g_deterministic{0};
}

int deterministic() { return g_deterministic.load(std::memory_order_relaxed); }

namespace {
std::atomic<int> g_spin_limit{kSpinLimitDefault};
}

int spin_limit() { return g_spin_limit.load(std::memory_order_relaxed); }

namespace {
std::atomic<int> g_timing{0};
std::mutex g_timing_mu;
hipEvent_t g_ev[2] = {nullptr, nullptr};
bool g_timed = false;  // a begin/end pair has been recorded
}  // namespace

void timing_begin(hipStream_t stream) {
  if (!g_timing.load(std::memory_order_relaxed)) return;
  std::lock_guard<std::mutex> lk(g_timing_mu);
  for (hipEvent_t& e : g_ev)
    if (e == nullptr && hipEventCreate(&e) != hipSuccess) e = nullptr;
  if (g_ev[0] && g_ev[1]) {
    g_timed = false;
    (void)hipEventRecord(g_ev[0], stream);
  }
}

void timing_end(hipStream_t stream) {
  if (!g_timing.load(std::memory_order_relaxed)) return;
  std::lock_guard<std::mutex> lk(g_timing_mu);
  if (g_ev[0] && g_ev[1] && hipEventRecord(g_ev[1], stream) == hipSuccess) g_timed = true;
}

int clear_words(int* p, size_t n, hipStream_t stream) {
  if (n == 0) return PRNN_OK;
  size_t blocks = (n + 255) / 256;
  if (blocks > 1024) blocks = 1024;
  clear_words_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream>>>(p, n);
  PRNN_HIP(hipGetLastError());
  return PRNN_OK;
}

}  // namespace prnn

extern "C" PRNN_API int prnn_abi_version(void) { return 10; }

extern "C" PRNN_API const char* prnn_last_error(void) { return prnn::last_error_buffer(); }

extern "C" PRNN_API void prnn_set_deterministic(int on) {
  prnn::g_deterministic.store(on ? 1 : 0, std::memory_order_relaxed);
}

extern "C" PRNN_API int prnn_deterministic(void) { return prnn::deterministic(); }

extern "C" PRNN_API void prnn_set_spin_limit(int rounds) {
  prnn::g_spin_limit.store(rounds > 0 ? rounds : prnn::kSpinLimitDefault,
                           std::memory_order_relaxed);
}

extern "C" PRNN_API void prnn_set_kernel_timing(int on) {
  prnn::g_timing.store(on ? 1 : 0, std::memory_order_relaxed);
}

extern "C" PRNN_API float prnn_last_kernel_ms(void) {
  std::lock_guard<std::mutex> lk(prnn::g_timing_mu);
  if (!prnn::g_timed) return -1.f;
  float ms = -1.f;
  if (hipEventSynchronize(prnn::g_ev[1]) != hipSuccess ||
      hipEventElapsedTime(&ms, prnn::g_ev[0], prnn::g_ev[1]) != hipSuccess)
    return -1.f;
  return ms;
}
