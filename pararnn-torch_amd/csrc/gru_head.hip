// ParaGRU mix='head' Newton + scan kernels for gfx950 (CDNA4).
#include "prnn_host.h"

extern "C" PRNN_API size_t prnn_gru_head_newton_workspace_size(int, int, int, int, int, int) {
  return 256;
}

extern "C" PRNN_API int prnn_gru_head_newton(const void*, const void*, const void*, const void*,
                                             const void*, void*, int, int, int, int, int, float,
                                             int, void*, size_t, void*) {
  return prnn::fail(PRNN_ERR_RUNTIME, "prnn_gru_head_newton: not built yet");
}
