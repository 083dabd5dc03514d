// ParaSLSTM mix='diag' Newton iteration with the reference's eager rounding
// (scan_backend='eager'): one launch per iteration, states in the storage
// dtype in and out.  The kernel is slstm_newton_kernel with EAGER = true (see
// cell_jac_eager); fp32, bf16 and fp16 storage, rectangular batches and
// packed streams, in a translation unit of its own so that it compiles in
// parallel with the others.
#include "slstm_diag_impl.h"

using namespace prnn;

namespace prnn {
namespace slstm {

template <typename TX, bool PK>
constexpr Shape eager_shape() {
  if constexpr (PK) return sizeof(TX) == 4 ? kNewtonEagerPackedF32 : kNewtonEagerPacked;
  return sizeof(TX) == 4 ? kNewtonEagerF32 : kNewtonEager;
}

template <typename TX, bool PK>
static void launch_newton_eager(const TX* wx, const TX* r, const TX* h0, const TX* hin, TX* hout,
                                int B, int T, int d, float omega, float eps, const Lookback& lb,
                                hipStream_t stream, const Packed& pk) {
  constexpr Shape sh = eager_shape<TX, PK>();
  const Geo g = geometry(B, T, d, sh);
#define PRNN_LAUNCH(DD)                                                                     \
  slstm_newton_kernel<TX, TX, TX, sh.L, sh.W, DD, PK, true>                                 \
      <<<dim3(g.n_tiles), dim3(64 * sh.W), 0, stream>>>(                                    \
          wx, r, h0, hin, hout, B, T, d, g.n_cb, omega, eps, lb.counters + 1, lb.agg,       \
          lb.incl, lb.tag_base + 1, lb.spin(), pk)
  if (deterministic())
    PRNN_LAUNCH(true);
  else
    PRNN_LAUNCH(false);
#undef PRNN_LAUNCH
}

}  // namespace slstm
}  // namespace prnn

namespace {

int eager_call(const void* wx, const void* r, const void* h0, const void* in, void* out, int B,
               int T, int d, float omega, float eps, int dtype, void* workspace,
               size_t workspace_bytes, int tag_base, void* stream, const slstm::Packed& pk) {
  int rc = slstm::check_dims(B, T, d, dtype);
  if (rc != PRNN_OK) return rc;
  rc = slstm::check_tag_base(tag_base);
  if (rc != PRNN_OK) return rc;
  rc = slstm::check_packed(pk, B, T);
  if (rc != PRNN_OK) return rc;
  if (!wx || !r || !in || !out || !workspace)
    return fail(PRNN_ERR_VALUE, "wx, r, in, out and workspace must be non-null");
  if (out == in) return fail(PRNN_ERR_VALUE, "out must not alias in");
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
  with_storage(dtype, [&](auto tag) {
    using TX = decltype(tag);
    const TX* wx_ = static_cast<const TX*>(wx);
    const TX* r_ = static_cast<const TX*>(r);
    const TX* h0_ = static_cast<const TX*>(h0);
    const TX* in_ = static_cast<const TX*>(in);
    TX* out_ = static_cast<TX*>(out);
    if (packed)
      slstm::launch_newton_eager<TX, true>(wx_, r_, h0_, in_, out_, 1, T, d, omega, eps, w.lb, s,
                                           pk);
    else
      slstm::launch_newton_eager<TX, false>(wx_, r_, h0_, in_, out_, B, T, d, omega, eps, w.lb,
                                            s, pk);
    return PRNN_OK;
  });
  timing_end(s);
  PRNN_HIP(hipGetLastError());
  return PRNN_OK;
}

}  // namespace

extern "C" PRNN_API int prnn_slstm_newton_eager(const void* wx, const void* r, const void* h0,
                                                const void* in, void* out, int B, int T, int d,
                                                float omega, float eps, int dtype,
                                                void* workspace, size_t workspace_bytes,
                                                int tag_base, void* stream) {
  return eager_call(wx, r, h0, in, out, B, T, d, omega, eps, dtype, workspace, workspace_bytes,
                    tag_base, stream, slstm::Packed{nullptr, nullptr, 0});
}

extern "C" PRNN_API int prnn_slstm_newton_eager_packed(const void* wx, const void* r,
                                                       const void* h0, const void* in, void* out,
                                                       int T, int d, float omega, float eps,
                                                       int dtype, const int* cu_seqlens,
                                                       int n_seq, const int* block_table,
                                                       void* workspace, size_t workspace_bytes,
                                                       int tag_base, void* stream) {
  if (!cu_seqlens) return fail(PRNN_ERR_VALUE, "cu_seqlens must be non-null");
  return eager_call(wx, r, h0, in, out, 1, T, d, omega, eps, dtype, workspace, workspace_bytes,
                    tag_base, stream, slstm::Packed{cu_seqlens, block_table, n_seq});
}
