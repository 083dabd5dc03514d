// ParaSLSTM mix='diag' rectangular launches in fp16 storage (default tile
// shapes), in a translation unit of their own so they compile in parallel
// with the fp32 / bf16 ones in slstm_diag.hip.
#include "slstm_diag_impl.h"

namespace prnn {
namespace slstm {

int run_init_f16(const f16* wx, const f16* r, const f16* h0, f16* states, int B, int T, int d,
                 int P, float eps, const InitWs& w, hipStream_t stream, const Packed& pk) {
  return run_init(wx, r, h0, states, B, T, d, P, eps, w, stream, pk);
}

int run_newton_f16(const f16* wx, const f16* r, const f16* h0, const f16* guess, f16* out, int B,
                   int T, int d, int K, float omega, float eps, const NewtonWs& w,
                   hipStream_t stream, const Packed& pk) {
  return run_newton(wx, r, h0, guess, out, B, T, d, K, omega, eps, w, stream, pk);
}

void launch_newton_step_f16(bool in_f32, const f16* wx, const f16* r, const f16* h0,
                            const void* in, float* out, int B, int T, int d, float omega,
                            float eps, const Lookback& lb, hipStream_t stream) {
  if (in_f32)
    launch_newton<f16, float, float>(wx, r, h0, static_cast<const float*>(in), out, B, T, d,
                                     omega, eps, lb, 1, stream);
  else
    launch_newton<f16, f16, float>(wx, r, h0, static_cast<const f16*>(in), out, B, T, d, omega,
                                   eps, lb, 1, stream);
}

}  // namespace slstm
}  // namespace prnn
