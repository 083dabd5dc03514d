// ParaSLSTM mix='diag' launches for packed streams (cu_seqlens), fp16
// storage (launchers in slstm_packed_impl.h), in a translation unit of their
// own so they compile in parallel with the others.
#include "slstm_packed_impl.h"

namespace prnn {
namespace slstm {

template void launch_picard_packed<f16>(const f16*, const f16*, const f16*, f16*, int, int, int,
                                        float, const Lookback&, unsigned long long*, hipStream_t,
                                        const Packed&);
template void launch_newton_fused_packed<f16>(const f16*, const f16*, const f16*, const f16*,
                                              f16*, int, int, int, float, float, const Lookback&,
                                              unsigned long long*, hipStream_t, const Packed&);
// K = 1 (result in the storage dtype) and the early-exit step (fp32 result)
template void launch_newton_packed<f16, f16, f16>(const f16*, const f16*, const f16*, const f16*,
                                                  f16*, int, int, float, float, const Lookback&,
                                                  int, hipStream_t, const Packed&);
template void launch_newton_packed<f16, f16, float>(const f16*, const f16*, const f16*,
                                                    const f16*, float*, int, int, float, float,
                                                    const Lookback&, int, hipStream_t,
                                                    const Packed&);
template void launch_newton_packed<f16, float, float>(const f16*, const f16*, const f16*,
                                                      const float*, float*, int, int, float, float,
                                                      const Lookback&, int, hipStream_t,
                                                      const Packed&);

}  // namespace slstm
}  // namespace prnn
