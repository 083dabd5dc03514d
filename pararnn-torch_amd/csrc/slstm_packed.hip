// ParaSLSTM mix='diag' launches for packed streams (cu_seqlens), fp32 and
// bf16 storage (launchers in slstm_packed_impl.h).  Kept apart from
// slstm_diag.hip so the two sets of kernel instantiations compile in parallel.
#include "slstm_packed_impl.h"

namespace prnn {
namespace slstm {

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

template void launch_picard_packed<bf16>(const bf16*, const bf16*, const bf16*, bf16*, int, int,
                                         int, float, const Lookback&, unsigned long long*,
                                         hipStream_t, const Packed&);
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
