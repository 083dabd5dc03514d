// Launchers of the packed-stream kernels (cu_seqlens): one stream of B = 1
// whose sequences restart at their heads inside the kernels (see Packed in
// slstm_scan.h).  Default tile shapes only; deterministic mode selects the
// DET instantiation.  Included by the translation units that instantiate
// them per storage type (slstm_packed.hip: fp32 and bf16; slstm_packed_f16.hip:
// fp16), so the instantiations compile in parallel.
#pragma once

#include "slstm_kernels.h"

namespace prnn {
namespace slstm {

template <typename TN>
void launch_picard_packed(const TN* wx, const TN* r, const TN* h0, TN* out, int T, int d,
                          int P, float eps, const Lookback& lb, unsigned long long* hlast,
                          hipStream_t stream, const Packed& pk) {
  constexpr Shape sh = kPicardPacked;
  const Geo g = geometry(1, T, d, sh);
#define PRNN_LAUNCH(DD)                                                                         \
  slstm_picard_fused_kernel<TN, sh.L, sh.W, 3, DD, true>                                   \
      <<<dim3(g.n_tiles), dim3(64 * sh.W), 0, stream>>>(                                        \
      wx, r, h0, out, 1, T, d, g.n_cb, g.n_tiles, P, eps, lb.counters + 1, lb.agg, lb.incl,   \
      hlast, lb.tag_base, lb.spin(), pk)
  if (deterministic())
    PRNN_LAUNCH(true);
  else
    PRNN_LAUNCH(false);
#undef PRNN_LAUNCH
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

}  // namespace slstm
}  // namespace prnn
