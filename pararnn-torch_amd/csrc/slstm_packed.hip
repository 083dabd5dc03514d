// ParaSLSTM mix='diag' launches for packed streams (cu_seqlens): one stream
// of B = 1 whose sequences restart at their heads inside the kernels (see
// Packed in slstm_scan.h).  Default tile shapes only; deterministic mode
// selects the DET instantiation.  Kept apart from slstm_diag.hip so the two
// sets of kernel instantiations compile in parallel.
#include "slstm_kernels.h"

namespace prnn {
namespace slstm {

void launch_picard_packed(const bf16* wx, const bf16* r, const bf16* h0, bf16* out, int T, int d,
                          int P, float eps, const Lookback& lb, unsigned long long* hlast,
                          hipStream_t stream, const Packed& pk) {
  constexpr Shape sh = kPicardPacked;
  const Geo g = geometry(1, T, d, sh);
#define PRNN_LAUNCH(DD)                                                                         \
  slstm_picard_fused_kernel<sh.L, sh.W, 3, DD, true>                                            \
      <<<dim3(g.n_tiles), dim3(64 * sh.W), 0, stream>>>(                                        \
      wx, r, h0, out, 1, T, d, g.n_cb, g.n_tiles, P, eps, lb.counters + 1, lb.agg, lb.incl,   \
      hlast, lb.tag_base, lb.spin(), pk)
  if (deterministic())
    PRNN_LAUNCH(true);
  else
    PRNN_LAUNCH(false);
#undef PRNN_LAUNCH
}

void launch_frozen_packed(bool has_h, bool full_out, const float* wx, const float* r,
                          const float* h0, const float* src, float* out_full, float* out_h, int T,
                          int d, float eps, const Lookback& lb, int epoch, hipStream_t stream,
                          const Packed& pk) {
  constexpr Shape sh = kFrozenPackedF32;
  const Geo g = geometry(1, T, d, sh);
  const dim3 grid(g.n_tiles), block(64 * sh.W);
  int* ctr = lb.counters + epoch;
#define PRNN_FROZEN(HH, FO, DD)                                                               \
  slstm_frozen_kernel<float, sh.L, sh.W, HH, FO, DD, true><<<grid, block, 0, stream>>>(      \
      wx, r, h0, src, out_full, out_h, 1, T, d, g.n_cb, eps, ctr, lb.agg, lb.incl,            \
      lb.tag_base + epoch, lb.spin(), pk)
#define PRNN_FROZEN_DET(HH, FO) \
  if (deterministic()) PRNN_FROZEN(HH, FO, true); else PRNN_FROZEN(HH, FO, false)
  if (has_h) {
    if (full_out) PRNN_FROZEN_DET(true, true); else PRNN_FROZEN_DET(true, false);
  } else {
    if (full_out) PRNN_FROZEN_DET(false, true); else PRNN_FROZEN_DET(false, false);
  }
#undef PRNN_FROZEN_DET
#undef PRNN_FROZEN
}

template <typename TX>
void launch_newton_fused_packed(const TX* wx, const TX* r, const TX* h0, const TX* guess, TX* out,
                                int T, int d, int K, float omega, float eps, const Lookback& lb,
                                unsigned long long* hlast, hipStream_t stream, const Packed& pk) {
  constexpr Shape sh = sizeof(TX) == 4 ? kNewtonFusedPackedF32 : kNewtonFusedPacked;
  const Geo g = geometry(1, T, d, sh);
#define PRNN_LAUNCH(DD)                                                                        \
  slstm_newton_fused_kernel<TX, sh.L, sh.W, 2, DD, true>                                       \
      <<<dim3(g.n_tiles), dim3(64 * sh.W), 0, stream>>>(                                       \
          wx, r, h0, guess, out, 1, T, d, g.n_cb, g.n_tiles, K, omega, eps, lb.counters + 1,   \
          lb.agg, lb.incl, hlast, lb.tag_base, lb.spin(), pk)
  if (deterministic())
    PRNN_LAUNCH(true);
  else
    PRNN_LAUNCH(false);
#undef PRNN_LAUNCH
}

template <typename TX, typename TIN, typename TOUT>
void launch_newton_packed(const TX* wx, const TX* r, const TX* h0, const TIN* hin, TOUT* hout,
                          int T, int d, float omega, float eps, const Lookback& lb, int epoch,
                          hipStream_t stream, const Packed& pk) {
  constexpr Shape sh = sizeof(TX) == 4 ? kNewtonPackedF32
                       : sizeof(TIN) == 4 ? kNewtonPackedWork : kNewtonPackedGuess;
  const Geo g = geometry(1, T, d, sh);
#define PRNN_LAUNCH(DD)                                                                     \
  slstm_newton_kernel<TX, TIN, TOUT, sh.L, sh.W, DD, true>                                  \
      <<<dim3(g.n_tiles), dim3(64 * sh.W), 0, stream>>>(                                    \
          wx, r, h0, hin, hout, 1, T, d, g.n_cb, omega, eps, lb.counters + epoch, lb.agg, \
          lb.incl, lb.tag_base + epoch, lb.spin(), pk)
  if (deterministic())
    PRNN_LAUNCH(true);
  else
    PRNN_LAUNCH(false);
#undef PRNN_LAUNCH
}

template void launch_newton_fused_packed<float>(const float*, const float*, const float*,
                                                const float*, float*, int, int, int, float,
                                                float, const Lookback&, unsigned long long*,
                                                hipStream_t, const Packed&);
template void launch_newton_fused_packed<bf16>(const bf16*, const bf16*, const bf16*,
                                               const bf16*, bf16*, int, int, int, float, float,
                                               const Lookback&, unsigned long long*, hipStream_t,
                                               const Packed&);
// K = 1 (result in the storage dtype) and the early-exit step (fp32 result)
template void launch_newton_packed<float, float, float>(const float*, const float*, const float*,
                                                        const float*, float*, int, int, float,
                                                        float, const Lookback&, int, hipStream_t,
                                                        const Packed&);
template void launch_newton_packed<bf16, bf16, bf16>(const bf16*, const bf16*, const bf16*,
                                                     const bf16*, bf16*, int, int, float, float,
                                                     const Lookback&, int, hipStream_t,
                                                     const Packed&);
template void launch_newton_packed<bf16, bf16, float>(const bf16*, const bf16*, const bf16*,
                                                      const bf16*, float*, int, int, float, float,
                                                      const Lookback&, int, hipStream_t,
                                                      const Packed&);
template void launch_newton_packed<bf16, float, float>(const bf16*, const bf16*, const bf16*,
                                                       const float*, float*, int, int, float,
                                                       float, const Lookback&, int, hipStream_t,
                                                       const Packed&);

}  // namespace slstm
}  // namespace prnn
