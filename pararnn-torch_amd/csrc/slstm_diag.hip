// ParaSLSTM mix='diag' C entry points (rectangular batches and packed
// streams) and the allocation-free Newton entry point.
#include "slstm_diag_impl.h"

#include <mutex>

using namespace prnn;

extern "C" PRNN_API size_t prnn_slstm_init_workspace_size(int B, int T, int d, int picard_iters,
                                                          int dtype) {
  if (slstm::check_dims(B, T, d, dtype) != PRNN_OK || picard_iters < 0) return 0;
  size_t total = 0;
  slstm::carve_init(nullptr, B, T, d, picard_iters, dtype, &total);
  return total;
}

namespace {

int init_call(const void* wx, const void* r, const void* h0, void* states, int B, int T, int d,
              int picard_iters, float eps, int dtype, void* workspace, size_t workspace_bytes,
              int tag_base, void* stream, const slstm::Packed& pk) {
  int rc = slstm::check_dims(B, T, d, dtype);
  if (rc != PRNN_OK) return rc;
  rc = slstm::check_tag_base(tag_base);
  if (rc != PRNN_OK) return rc;
  rc = slstm::check_packed(pk, B, T);
  if (rc != PRNN_OK) return rc;
  if (picard_iters < 0 || picard_iters > slstm::kMaxStages - 2)
    return fail(PRNN_ERR_VALUE, "picard_iters must be in [0, %d], got %d",
                slstm::kMaxStages - 2, picard_iters);
  if (!wx || !r || !states || !workspace)
    return fail(PRNN_ERR_VALUE, "wx, r, states and workspace must be non-null");
  size_t need = 0;
  slstm::InitWs w = slstm::carve_init(workspace, B, T, d, picard_iters, dtype, &need,
                                      pk.cu != nullptr);
  if (workspace_bytes < need)
    return fail(PRNN_ERR_VALUE, "workspace too small: %zu < %zu bytes", workspace_bytes, need);
  w.lb.tag_base = tag_base;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return with_storage(dtype, [&](auto tag) {
    using TX = decltype(tag);
    const TX* wx_ = static_cast<const TX*>(wx);
    const TX* r_ = static_cast<const TX*>(r);
    const TX* h0_ = static_cast<const TX*>(h0);
    TX* st_ = static_cast<TX*>(states);
    if constexpr (std::is_same<TX, f16>::value)
      return slstm::run_init_f16(wx_, r_, h0_, st_, B, T, d, picard_iters, eps, w, s, pk);
    else
      return slstm::run_init(wx_, r_, h0_, st_, B, T, d, picard_iters, eps, w, s, pk);
  });
}

int newton_call(const void* wx, const void* r, const void* h0, const void* states, void* out,
                int B, int T, int d, int max_iters, float omega, float eps, int dtype,
                void* workspace, size_t workspace_bytes, int tag_base, void* stream,
                const slstm::Packed& pk) {
  int rc = slstm::check_dims(B, T, d, dtype);
  if (rc != PRNN_OK) return rc;
  rc = slstm::check_tag_base(tag_base);
  if (rc != PRNN_OK) return rc;
  rc = slstm::check_packed(pk, B, T);
  if (rc != PRNN_OK) return rc;
  if (max_iters < 0 || max_iters > slstm::kMaxStages - 1)
    return fail(PRNN_ERR_VALUE, "max_iters must be in [0, %d], got %d", slstm::kMaxStages - 1,
                max_iters);
  if (!wx || !r || !states || !out || !workspace)
    return fail(PRNN_ERR_VALUE, "wx, r, states, out and workspace must be non-null");
  if (out == states) return fail(PRNN_ERR_VALUE, "out must not alias states");
  size_t need = 0;
  slstm::NewtonWs w = slstm::carve_newton(workspace, B, T, d, max_iters, dtype, &need,
                                          pk.cu != nullptr);
  if (workspace_bytes < need)
    return fail(PRNN_ERR_VALUE, "workspace too small: %zu < %zu bytes", workspace_bytes, need);
  w.lb.tag_base = tag_base;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return with_storage(dtype, [&](auto tag) {
    using TX = decltype(tag);
    const TX* wx_ = static_cast<const TX*>(wx);
    const TX* r_ = static_cast<const TX*>(r);
    const TX* h0_ = static_cast<const TX*>(h0);
    const TX* g_ = static_cast<const TX*>(states);
    TX* o_ = static_cast<TX*>(out);
    if constexpr (std::is_same<TX, f16>::value)
      return slstm::run_newton_f16(wx_, r_, h0_, g_, o_, B, T, d, max_iters, omega, eps, w, s,
                                   pk);
    else
      return slstm::run_newton(wx_, r_, h0_, g_, o_, B, T, d, max_iters, omega, eps, w, s, pk);
  });
}

const slstm::Packed kRect{nullptr, nullptr, 0};

}  // namespace

extern "C" PRNN_API int prnn_slstm_init_ex(const void* wx, const void* r, const void* h0,
                                           void* states, int B, int T, int d, int picard_iters,
                                           float eps, int dtype, void* workspace,
                                           size_t workspace_bytes, int tag_base, void* stream) {
  return init_call(wx, r, h0, states, B, T, d, picard_iters, eps, dtype, workspace,
                   workspace_bytes, tag_base, stream, kRect);
}

extern "C" PRNN_API int prnn_slstm_init(const void* wx, const void* r, const void* h0,
                                        void* states, int B, int T, int d, int picard_iters,
                                        float eps, int dtype, void* workspace,
                                        size_t workspace_bytes, void* stream) {
  return prnn_slstm_init_ex(wx, r, h0, states, B, T, d, picard_iters, eps, dtype, workspace,
                            workspace_bytes, 0, stream);
}

extern "C" PRNN_API size_t prnn_slstm_newton_workspace_size(int B, int T, int d, int max_iters,
                                                            int dtype) {
  if (slstm::check_dims(B, T, d, dtype) != PRNN_OK || max_iters < 0) return 0;
  size_t total = 0;
  slstm::carve_newton(nullptr, B, T, d, max_iters, dtype, &total);
  return total;
}

extern "C" PRNN_API int prnn_slstm_newton_ex(const void* wx, const void* r, const void* h0,
                                             const void* states, void* out, int B, int T, int d,
                                             int max_iters, float omega, float eps, int dtype,
                                             void* workspace, size_t workspace_bytes,
                                             int tag_base, void* stream) {
  return newton_call(wx, r, h0, states, out, B, T, d, max_iters, omega, eps, dtype, workspace,
                     workspace_bytes, tag_base, stream, kRect);
}

extern "C" PRNN_API size_t prnn_slstm_init_packed_workspace_size(int T, int d, int picard_iters,
                                                                 int dtype) {
  if (slstm::check_dims(1, T, d, dtype) != PRNN_OK || picard_iters < 0) return 0;
  size_t total = 0;
  slstm::carve_init(nullptr, 1, T, d, picard_iters, dtype, &total, true);
  return total;
}

extern "C" PRNN_API int prnn_slstm_init_packed(const void* wx, const void* r, const void* h0,
                                               void* states, int T, int d, int picard_iters,
                                               float eps, int dtype, const int* cu_seqlens,
                                               int n_seq, const int* block_table,
                                               void* workspace, size_t workspace_bytes,
                                               int tag_base, void* stream) {
  if (!cu_seqlens) return fail(PRNN_ERR_VALUE, "cu_seqlens must be non-null");
  return init_call(wx, r, h0, states, 1, T, d, picard_iters, eps, dtype, workspace,
                   workspace_bytes, tag_base, stream,
                   slstm::Packed{cu_seqlens, block_table, n_seq});
}

extern "C" PRNN_API size_t prnn_slstm_newton_packed_workspace_size(int T, int d, int max_iters,
                                                                   int dtype) {
  if (slstm::check_dims(1, T, d, dtype) != PRNN_OK || max_iters < 0) return 0;
  size_t total = 0;
  slstm::carve_newton(nullptr, 1, T, d, max_iters, dtype, &total, true);
  return total;
}

extern "C" PRNN_API int prnn_slstm_newton_packed(const void* wx, const void* r, const void* h0,
                                                 const void* states, void* out, int T, int d,
                                                 int max_iters, float omega, float eps,
                                                 int dtype, const int* cu_seqlens, int n_seq,
                                                 const int* block_table, void* workspace,
                                                 size_t workspace_bytes, int tag_base,
                                                 void* stream) {
  if (!cu_seqlens) return fail(PRNN_ERR_VALUE, "cu_seqlens must be non-null");
  return newton_call(wx, r, h0, states, out, 1, T, d, max_iters, omega, eps, dtype, workspace,
                     workspace_bytes, tag_base, stream,
                     slstm::Packed{cu_seqlens, block_table, n_seq});
}

extern "C" PRNN_API int prnn_slstm_newton(const void* wx, const void* r, const void* h0,
                                          const void* states, void* out, int B, int T, int d,
                                          int max_iters, float omega, float eps, int dtype,
                                          void* workspace, size_t workspace_bytes, void* stream) {
  return prnn_slstm_newton_ex(wx, r, h0, states, out, B, T, d, max_iters, omega, eps, dtype,
                              workspace, workspace_bytes, 0, stream);
}

namespace {

int step_call(const void* wx, const void* r, const void* h0, const void* in, int in_f32,
              float* out, int B, int T, int d, float omega, float eps, int dtype,
              void* workspace, size_t workspace_bytes, int tag_base, void* stream,
              const slstm::Packed& pk) {
  int rc = slstm::check_dims(B, T, d, dtype);
  if (rc != PRNN_OK) return rc;
  rc = slstm::check_tag_base(tag_base);
  if (rc != PRNN_OK) return rc;
  rc = slstm::check_packed(pk, B, T);
  if (rc != PRNN_OK) return rc;
  if (!wx || !r || !in || !out || !workspace)
    return fail(PRNN_ERR_VALUE, "wx, r, in, out and workspace must be non-null");
  if (static_cast<const void*>(out) == in) return fail(PRNN_ERR_VALUE, "out must not alias in");
  size_t need = 0;
  slstm::NewtonWs w = slstm::carve_newton(workspace, B, T, d, 1, dtype, &need, pk.cu != nullptr);
  if (workspace_bytes < need)
    return fail(PRNN_ERR_VALUE, "workspace too small: %zu < %zu bytes", workspace_bytes, need);
  w.lb.tag_base = tag_base;
  hipStream_t s = static_cast<hipStream_t>(stream);
  rc = slstm::clear_status(w.lb, s);
  if (rc != PRNN_OK) return rc;
  const bool packed = pk.cu != nullptr;
  timing_begin(s);
#define PRNN_STEP(TX, TIN)                                                                   \
  do {                                                                                       \
    const TX* wx_ = static_cast<const TX*>(wx);                                              \
    const TX* r_ = static_cast<const TX*>(r);                                                \
    const TX* h0_ = static_cast<const TX*>(h0);                                              \
    const TIN* in_ = static_cast<const TIN*>(in);                                            \
    if (packed)                                                                              \
      slstm::launch_newton_packed<TX, TIN, float>(wx_, r_, h0_, in_, out, T, d, omega, eps, \
                                                  w.lb, 1, s, pk);                           \
    else                                                                                     \
      slstm::launch_newton<TX, TIN, float>(wx_, r_, h0_, in_, out, B, T, d, omega, eps,     \
                                           w.lb, 1, s);                                      \
  } while (0)
  if (dtype == PRNN_F32) {
    PRNN_STEP(float, float);
  } else if (dtype == PRNN_F16) {
    const f16* wx_ = static_cast<const f16*>(wx);
    const f16* r_ = static_cast<const f16*>(r);
    const f16* h0_ = static_cast<const f16*>(h0);
    if (packed && in_f32)
      slstm::launch_newton_packed<f16, float, float>(wx_, r_, h0_, static_cast<const float*>(in),
                                                     out, T, d, omega, eps, w.lb, 1, s, pk);
    else if (packed)
      slstm::launch_newton_packed<f16, f16, float>(wx_, r_, h0_, static_cast<const f16*>(in),
                                                   out, T, d, omega, eps, w.lb, 1, s, pk);
    else
      slstm::launch_newton_step_f16(in_f32, wx_, r_, h0_, in, out, B, T, d, omega, eps, w.lb, s);
  } else if (in_f32)
    PRNN_STEP(bf16, float);
  else
    PRNN_STEP(bf16, bf16);
#undef PRNN_STEP
  timing_end(s);
  PRNN_HIP(hipGetLastError());
  return PRNN_OK;
}

}  // namespace

extern "C" PRNN_API int prnn_slstm_newton_step(const void* wx, const void* r, const void* h0,
                                               const void* in, int in_f32, float* out, int B,
                                               int T, int d, float omega, float eps, int dtype,
                                               void* workspace, size_t workspace_bytes,
                                               int tag_base, void* stream) {
  return step_call(wx, r, h0, in, in_f32, out, B, T, d, omega, eps, dtype, workspace,
                   workspace_bytes, tag_base, stream, kRect);
}

extern "C" PRNN_API int prnn_slstm_newton_step_packed(const void* wx, const void* r,
                                                      const void* h0, const void* in, int in_f32,
                                                      float* out, int T, int d, float omega,
                                                      float eps, int dtype,
                                                      const int* cu_seqlens, int n_seq,
                                                      const int* block_table, void* workspace,
                                                      size_t workspace_bytes, int tag_base,
                                                      void* stream) {
  if (!cu_seqlens) return fail(PRNN_ERR_VALUE, "cu_seqlens must be non-null");
  return step_call(wx, r, h0, in, in_f32, out, 1, T, d, omega, eps, dtype, workspace,
                   workspace_bytes, tag_base, stream,
                   slstm::Packed{cu_seqlens, block_table, n_seq});
}

extern "C" PRNN_API int prnn_slstm_lookback_status(const void* workspace, int* status,
                                                   void* stream) {
  if (!workspace || !status) return fail(PRNN_ERR_VALUE, "workspace and status must be non-null");
  // The ticket counters lead every sLSTM workspace; the status word follows them.
  const int* word = static_cast<const int*>(workspace) + slstm::kMaxStages;
  hipStream_t s = static_cast<hipStream_t>(stream);
  PRNN_HIP(hipMemcpyAsync(status, word, sizeof(int), hipMemcpyDeviceToHost, s));
  PRNN_HIP(hipStreamSynchronize(s));
  return PRNN_OK;
}

// ---- allocation-free Newton entry point ------------------------------------
// For callers that cannot allocate device memory (code under HIP graph
// capture, serving loops, harnesses that forbid hipMalloc): the workspace is a
// file-scope device array instead of a caller buffer.  Each GPU holds its own
// copy for the life of the process.  Host code never passes the array's name
// to a kernel (on the host that name is only a stand-in): the device address
// of each GPU's copy is looked up once per device with hipGetSymbolAddress
// and used from then on.
namespace {

constexpr size_t kScratchBytes = size_t(64) << 20;  // 64 MiB per GPU
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

int scratch_for_current_device(void** out) {
  int dev = 0;
  PRNN_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(PRNN_ERR_RUNTIME, "device %d is beyond the %d devices supported", dev,
                kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(PRNN_ERR_RUNTIME, "hipGetSymbolAddress(scratch) on device %d: %s", dev,
                  hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return PRNN_OK;
}

}  // namespace

extern "C" PRNN_API size_t prnn_slstm_newton_noalloc_max_bytes(void) { return kScratchBytes; }

extern "C" PRNN_API int prnn_slstm_newton_noalloc(const void* wx, const void* r, const void* h0,
                                                  const void* states, void* out, int B, int T,
                                                  int d, int max_iters, float omega, float eps,
                                                  int dtype, void* stream) {
  int rc = slstm::check_dims(B, T, d, dtype);
  if (rc != PRNN_OK) return rc;
  if (max_iters < 0 || max_iters > slstm::kMaxStages - 1)
    return fail(PRNN_ERR_VALUE, "max_iters must be in [0, %d], got %d", slstm::kMaxStages - 1,
                max_iters);
  const size_t need = prnn_slstm_newton_workspace_size(B, T, d, max_iters, dtype);
  if (need > kScratchBytes)
    return fail(PRNN_ERR_VALUE,
                "prnn_slstm_newton_noalloc: B=%d T=%d d=%d K=%d needs %zu bytes of scratch, "
                "above the %zu-byte maximum (use prnn_slstm_newton with a workspace)",
                B, T, d, max_iters, need, kScratchBytes);
  void* ws = nullptr;
  rc = scratch_for_current_device(&ws);
  if (rc != PRNN_OK) return rc;
  // tag_base 0: every look-back word the call reads is cleared first by a
  // fill kernel on `stream`, so whatever an earlier call left in the array
  // does not matter.
  return prnn_slstm_newton_ex(wx, r, h0, states, out, B, T, d, max_iters, omega, eps, dtype, ws,
                              kScratchBytes, 0, stream);
}
