// ParaSLSTM mix='diag' host side: tile shapes, workspaces and the launches of
// the kernels in slstm_kernels.h for rectangular batches (packed streams
// launch through slstm_packed_impl.h).  Included by slstm_diag.hip (the C
// entry points; fp32 and bf16 instantiations) and slstm_diag_f16.hip (the
// fp16 instantiations, behind the non-template wrappers declared at the end).
#pragma once

#include "slstm_kernels.h"

#include <stdio.h>
#include <stdlib.h>

#include <mutex>
#include <type_traits>

// ===========================================================================
// Host entry points
// ===========================================================================
namespace prnn {
namespace slstm {

// Tile shapes (L steps per lane x W waves).  Selected once per process;
// PRNN_SLSTM_TILES="<frozen L>x<W>,<newton L>x<W>" overrides the default for
// tuning runs (only the instantiated shapes are accepted).  Deterministic mode
// always runs the default shapes (the only ones instantiated for it).
// bf16 frozen tiles stash 2 registers per step, fp32 ones 4 (one fp32 shape).
static const Shape kFrozenShapes[] = {{64, 4}, {32, 8}, {32, 4}, {64, 2}};
// Newton tiles stash wx and the guess: 4 to 6 registers per step in bf16, 8 in fp32.
static const Shape kNewtonShapes[] = {{32, 8}, {32, 4}, {24, 4}, {16, 8}, {64, 4}};

struct Tiles {
  Shape frozen;
  Shape newton_guess;  // Newton launches that read the bf16 guess
  Shape newton_work;   // Newton launches that read the fp32 work trajectory
};

static Tiles tiles() {
  static Tiles t = [] {
    Tiles r{kFrozenDefault, kNewtonGuessDefault, kNewtonWorkDefault};
    if (const char* e = getenv("PRNN_SLSTM_TILES")) {
      int fl, fw, gl, gw, wl, ww;
      if (sscanf(e, "%dx%d,%dx%d,%dx%d", &fl, &fw, &gl, &gw, &wl, &ww) == 6) {
        for (const Shape& s : kFrozenShapes)
          if (s.L == fl && s.W == fw) r.frozen = s;
        for (const Shape& s : kNewtonShapes) {
          if (s.L == gl && s.W == gw) r.newton_guess = s;
          if (s.L == wl && s.W == ww) r.newton_work = s;
        }
      }
    }
    return r;
  }();
  return t;
}

// fp16 storage is compiled in the default shapes only (the tuning shapes are
// bf16's): every shape query below answers the default for it.
static Shape frozen_shape(int dtype) {
  if (!narrow(dtype)) return kFrozenF32;
  return deterministic() || dtype == PRNN_F16 ? kFrozenDefault : tiles().frozen;
}
// Shape of a Newton launch; `work_in` when it reads the fp32 work trajectory.
static Shape newton_shape(int dtype, bool work_in) {
  if (!narrow(dtype)) return kNewtonF32;
  if (deterministic() || dtype == PRNN_F16)
    return work_in ? kNewtonWorkDefault : kNewtonGuessDefault;
  return work_in ? tiles().newton_work : tiles().newton_guess;
}

// All Picard passes in one launch (bf16 storage); PRNN_SLSTM_PICARD_FUSED=0
// selects one launch per pass instead (the fp32 path always does).
static bool picard_fused(int dtype) {
  static const bool on = [] {
    const char* e = getenv("PRNN_SLSTM_PICARD_FUSED");
    return !(e && atoi(e) == 0);
  }();
  return narrow(dtype) && on;
}

// Shapes of the fused launch: wx, the stage's pre-activations and h stay in
// registers (4.5 per step).  PRNN_SLSTM_PICARD_TILES="<L>x<W>" for tuning.
static const Shape kPicardShapes[] = {{24, 4}, {16, 4}, {20, 4}, {32, 4}};

static Shape picard_shape(int dtype) {
  static const Shape s = [] {
    Shape r = kPicardDefault;
    if (const char* e = getenv("PRNN_SLSTM_PICARD_TILES")) {
      int l, w;
      if (sscanf(e, "%dx%d", &l, &w) == 2)
        for (const Shape& c : kPicardShapes)
          if (c.L == l && c.W == w) r = c;
    }
    return r;
  }();
  return deterministic() || dtype == PRNN_F16 ? kPicardDefault : s;
}

struct InitWs {
  Lookback lb;
  void* hbuf[2];
  unsigned long long* hlast;  // fused launch: [P][tile][64] tagged last-step h
  bool fused;
};

static InitWs carve_init(void* base, int B, int T, int d, int P, int dtype, size_t* total,
                         bool packed = false) {
  Carver cv(base);
  InitWs w;
  // packed bf16 streams always take the single-launch warm start
  w.fused = packed ? narrow(dtype) : picard_fused(dtype);
  w.hbuf[0] = w.hbuf[1] = nullptr;
  w.hlast = nullptr;
  if (w.fused) {
    // Stage-indexed look-back words (a tile may run stages ahead of the
    // tiles that still read its earlier stages), cleared with the counters.
    const Geo g = geometry(B, T, d, packed ? kPicardPacked : picard_shape(dtype));
    w.lb = carve_lookback(cv, g, 3 * (P + 1), 4 * (P + 1));
    w.hlast = static_cast<unsigned long long*>(
        cv.take(sizeof(unsigned long long) * static_cast<size_t>(P) * kCB * g.n_tiles));
    w.lb.clear_words = (cv.used - (reinterpret_cast<char*>(w.lb.counters) - cv.base)) / sizeof(int);
  } else {
    const Geo g = geometry(B, T, d, packed ? kFrozenPackedF32 : frozen_shape(dtype));
    w.lb = carve_lookback(cv, g, 3, 4);
    const size_t hb = static_cast<size_t>(B) * T * d * elem_size(dtype);
    w.hbuf[0] = P >= 1 ? cv.take(hb) : nullptr;
    w.hbuf[1] = P >= 2 ? cv.take(hb) : nullptr;
  }
  *total = cv.used;
  return w;
}

// All K Newton iterations in one launch (the fp32 iterate stays in
// registers), K = 1 included: the per-iteration kernel, which holds the guess
// packed, measured no faster for a single iteration (and 1.8x slower on packed
// streams, where its head handling leaves one wave per SIMD).
// PRNN_SLSTM_NEWTON_FUSED=0 selects one launch per iteration throughout; the
// residual-gated early-exit path always runs one launch per iteration.
static bool newton_fused(int K) {
  static const bool on = [] {
    const char* e = getenv("PRNN_SLSTM_NEWTON_FUSED");
    return !(e && atoi(e) == 0);
  }();
  return on && K >= 1;
}

// Shapes of the fused launch: wx (2 registers per step in bf16, 4 in fp32)
// and the fp32 iterate (4) stay in registers.
// PRNN_SLSTM_NEWTON_FUSED_TILES="<L>x<W>" for tuning (bf16).
static const Shape kNewtonFusedShapes[] = {{20, 4}, {16, 4}, {24, 4}, {16, 8}};

static Shape newton_fused_shape(int dtype) {
  static const Shape s = [] {
    Shape r = kNewtonFusedDefault;
    if (const char* e = getenv("PRNN_SLSTM_NEWTON_FUSED_TILES")) {
      int l, w;
      if (sscanf(e, "%dx%d", &l, &w) == 2)
        for (const Shape& c : kNewtonFusedShapes)
          if (c.L == l && c.W == w) r = c;
    }
    return r;
  }();
  if (!narrow(dtype)) return kNewtonFusedF32;
  return deterministic() || dtype == PRNN_F16 ? kNewtonFusedDefault : s;
}

struct NewtonWs {
  Lookback lb;
  float* work[2];
  unsigned long long* hlast;  // fused launch: [K-1][tile][4][64] tagged last-step state
  bool fused;
};

static NewtonWs carve_newton(void* base, int B, int T, int d, int K, int dtype, size_t* total,
                             bool packed = false) {
  Carver cv(base);
  NewtonWs w;
  // packed streams always take the single-launch path
  w.fused = packed ? K >= 1 : newton_fused(K);
  w.work[0] = w.work[1] = nullptr;
  w.hlast = nullptr;
  if (w.fused) {
    // Iteration-indexed look-back words (a tile may run iterations ahead of
    // the tiles that still read its earlier ones), cleared with the counters.
    Geo g = geometry(B, T, d,
                     !packed ? newton_fused_shape(dtype)
                     : narrow(dtype) ? kNewtonFusedPacked : kNewtonFusedPackedF32);
    if (K == 1) {
      // A one-iteration workspace also serves the single-iteration launches
      // (the residual-gated step and the eager iteration), whose tiles may be
      // shorter: size the words for the largest tile count.
      const Shape one[3] = {
          !packed ? newton_shape(dtype, false) : narrow(dtype) ? kNewtonPackedGuess : kNewtonPackedF32,
          !packed ? newton_shape(dtype, true) : narrow(dtype) ? kNewtonPackedWork : kNewtonPackedF32,
          !packed ? (narrow(dtype) ? kNewtonEager : kNewtonEagerF32)
          : narrow(dtype) ? kNewtonEagerPacked : kNewtonEagerPackedF32};
      for (const Shape& sh : one) {
        const Geo gs = geometry(B, T, d, sh);
        if (gs.n_tiles > g.n_tiles) g = gs;
      }
    }
    w.lb = carve_lookback(cv, g, 4 * K, 20 * K);
    w.hlast = static_cast<unsigned long long*>(
        cv.take(sizeof(unsigned long long) * static_cast<size_t>(K - 1) * 4 * kCB * g.n_tiles));
    w.lb.clear_words = (cv.used - (reinterpret_cast<char*>(w.lb.counters) - cv.base)) / sizeof(int);
    *total = cv.used;
    return w;
  }
  // Launches of one call share the look-back arrays: size them for the
  // largest tile count of the shapes a launch may take.
  const Geo g1 = geometry(B, T, d, newton_shape(dtype, false));
  const Geo g2 = geometry(B, T, d, newton_shape(dtype, true));
  const Geo g3 = geometry(B, T, d, narrow(dtype) ? kNewtonPackedGuess : kNewtonPackedF32);
  const Geo g4 = geometry(B, T, d, narrow(dtype) ? kNewtonPackedWork : kNewtonPackedF32);
  Geo g = g1.n_tiles >= g2.n_tiles ? g1 : g2;
  if (g3.n_tiles > g.n_tiles) g = g3;
  if (g4.n_tiles > g.n_tiles) g = g4;
  if (K == 1) {
    const Geo ge = geometry(B, T, d, narrow(dtype) ? kNewtonEager : kNewtonEagerF32);
    if (ge.n_tiles > g.n_tiles) g = ge;
  }
  w.lb = carve_lookback(cv, g, 4, 20);
  const size_t wb = static_cast<size_t>(B) * T * 4 * d * sizeof(float);
  w.work[0] = K >= 2 ? static_cast<float*>(cv.take(wb)) : nullptr;
  w.work[1] = K >= 3 ? static_cast<float*>(cv.take(wb)) : nullptr;
  *total = cv.used;
  return w;
}

template <typename TX, int L, int W, bool DET>
static void launch_frozen(bool has_h, bool full_out, const TX* wx, const TX* r, const TX* h0,
                          const TX* src, TX* out_full, TX* out_h, int B, int T, int d, float eps,
                          const Lookback& lb, int epoch, hipStream_t stream) {
  constexpr bool PK = false;
  const Packed pk{nullptr, nullptr, 0};
  const Geo g = geometry(B, T, d, Shape{L, W});
  const dim3 grid(g.n_tiles), block(64 * W);
  int* ctr = lb.counters + epoch;
#define PRNN_FROZEN(HH, FO)                                                                    \
  slstm_frozen_kernel<TX, L, W, HH, FO, DET, PK><<<grid, block, 0, stream>>>(                  \
      wx, r, h0, src, out_full, out_h, B, T, d, g.n_cb, eps, ctr, lb.agg, lb.incl,             \
      lb.tag_base + epoch, lb.spin(), pk)
  if (has_h) {
    if (full_out) PRNN_FROZEN(true, true); else PRNN_FROZEN(true, false);
  } else {
    if (full_out) PRNN_FROZEN(false, true); else PRNN_FROZEN(false, false);
  }
#undef PRNN_FROZEN
}

template <typename TX>
static void frozen_pass(bool has_h, bool full_out, const TX* wx, const TX* r, const TX* h0,
                        const TX* src, TX* out_full, TX* out_h, int B, int T, int d, float eps,
                        const Lookback& lb, int epoch, hipStream_t stream, const Packed& pk) {
#define PRNN_LAUNCH(LL, WW, DD)                                                              \
  return launch_frozen<TX, LL, WW, DD>(has_h, full_out, wx, r, h0, src, out_full, out_h, B, T, \
                                       d, eps, lb, epoch, stream)
  if constexpr (sizeof(TX) == 4) {
    // packed streams: fp32 only (bf16 takes the single-launch warm start)
    if (pk.cu != nullptr)
      return launch_frozen_packed(has_h, full_out, wx, r, h0, src, out_full, out_h, T, d, eps,
                                  lb, epoch, stream, pk);
    if (deterministic()) PRNN_LAUNCH(kFrozenF32.L, kFrozenF32.W, true);
    PRNN_LAUNCH(kFrozenF32.L, kFrozenF32.W, false);
  } else {
  if (deterministic()) PRNN_LAUNCH(kFrozenDefault.L, kFrozenDefault.W, true);
  if constexpr (std::is_same<TX, f16>::value) {
    PRNN_LAUNCH(kFrozenDefault.L, kFrozenDefault.W, false);
  } else {
  const Shape sh = frozen_shape(dtype_code<TX>());
#define PRNN_SHAPE(LL, WW) \
  if (sh.L == LL && sh.W == WW) PRNN_LAUNCH(LL, WW, false);
  PRNN_SHAPE(64, 4)
  PRNN_SHAPE(32, 8)
  PRNN_SHAPE(32, 4)
  PRNN_SHAPE(64, 2)
#undef PRNN_SHAPE
  }
  }
#undef PRNN_LAUNCH
}

template <typename TX>
static int run_init(const TX* wx, const TX* r, const TX* h0, TX* states, int B, int T, int d,
                    int P, float eps, const InitWs& w, hipStream_t stream, const Packed& pk) {
  int rc = clear_status(w.lb, stream);
  if (rc != PRNN_OK) return rc;
  if constexpr (sizeof(TX) == 2) {
    if (w.fused) {
      const Shape sh = pk.cu != nullptr ? kPicardDefault : picard_shape(dtype_code<TX>());
      const Geo g = geometry(B, T, d, sh);
#define PRNN_LAUNCH(LL, WW, WPE, DD)                                                             \
  slstm_picard_fused_kernel<TX, LL, WW, WPE, DD, false>                                          \
      <<<dim3(g.n_tiles), dim3(64 * WW), 0, stream>>>(                                           \
          wx, r, h0, states, B, T, d, g.n_cb, g.n_tiles, P, eps, w.lb.counters + 1, w.lb.agg,   \
          w.lb.incl, w.hlast, w.lb.tag_base, w.lb.spin(), Packed{nullptr, nullptr, 0})
#define PRNN_SHAPE(LL, WW, WPE) \
  else if (sh.L == LL && sh.W == WW) PRNN_LAUNCH(LL, WW, WPE, false);
      static_assert(kPicardDefault.L == 24 && kPicardDefault.W == 4, "default Picard shape");
      timing_begin(stream);
      if (pk.cu != nullptr)
        launch_picard_packed(wx, r, h0, states, T, d, P, eps, w.lb, w.hlast, stream, pk);
      else if (deterministic()) PRNN_LAUNCH(24, 4, 3, true);
      else if constexpr (std::is_same<TX, f16>::value) PRNN_LAUNCH(24, 4, 3, false);
      PRNN_SHAPE(24, 4, 3)
      PRNN_SHAPE(16, 4, 4)
      PRNN_SHAPE(20, 4, 3)
      PRNN_SHAPE(32, 4, 2)
#undef PRNN_SHAPE
#undef PRNN_LAUNCH
      timing_end(stream);
      PRNN_HIP(hipGetLastError());
      return PRNN_OK;
    }
  }
  // Pass 0: zero-hidden scan (pre = wx); passes 1..P freeze wx + R h_prev.
  timing_begin(stream);
  for (int p = 0; p <= P; ++p) {
    const TX* src = p == 0 ? nullptr : static_cast<const TX*>(w.hbuf[(p - 1) & 1]);
    const bool last = p == P;
    TX* out_h = last ? nullptr : static_cast<TX*>(w.hbuf[p & 1]);
    frozen_pass<TX>(p > 0, last, wx, r, h0, src, last ? states : nullptr, out_h, B, T, d, eps,
                    w.lb, p + 1, stream, pk);
    PRNN_HIP(hipGetLastError());
  }
  timing_end(stream);
  return PRNN_OK;
}

template <typename TX, typename TIN, typename TOUT, int L, int W, bool DET>
static void launch_newton_shape(const TX* wx, const TX* r, const TX* h0, const TIN* hin,
                                TOUT* hout, int B, int T, int d, float omega, float eps,
                                const Lookback& lb, int epoch, hipStream_t stream) {
  const Geo g = geometry(B, T, d, Shape{L, W});
  slstm_newton_kernel<TX, TIN, TOUT, L, W, DET, false>
      <<<dim3(g.n_tiles), dim3(64 * W), 0, stream>>>(
          wx, r, h0, hin, hout, B, T, d, g.n_cb, omega, eps, lb.counters + epoch, lb.agg,
          lb.incl, lb.tag_base + epoch, lb.spin(), Packed{nullptr, nullptr, 0});
}

template <typename TX, typename TIN, typename TOUT>
static void launch_newton(const TX* wx, const TX* r, const TX* h0, const TIN* hin, TOUT* hout,
                          int B, int T, int d, float omega, float eps, const Lookback& lb,
                          int epoch, hipStream_t stream) {
#define PRNN_LAUNCH(LL, WW, DD)                                                          \
  return launch_newton_shape<TX, TIN, TOUT, LL, WW, DD>(wx, r, h0, hin, hout, B, T, d, omega, \
                                                        eps, lb, epoch, stream)
  if constexpr (sizeof(TX) == 4) {
    if (deterministic()) PRNN_LAUNCH(kNewtonF32.L, kNewtonF32.W, true);
    PRNN_LAUNCH(kNewtonF32.L, kNewtonF32.W, false);
  } else {
  if (deterministic()) {
    constexpr Shape dd = sizeof(TIN) == 4 ? kNewtonWorkDefault : kNewtonGuessDefault;
    PRNN_LAUNCH(dd.L, dd.W, true);
  }
  if constexpr (std::is_same<TX, f16>::value) {
    constexpr Shape dd = sizeof(TIN) == 4 ? kNewtonWorkDefault : kNewtonGuessDefault;
    PRNN_LAUNCH(dd.L, dd.W, false);
  } else {
  const Shape sh = newton_shape(dtype_code<TX>(), sizeof(TIN) == 4);
#define PRNN_SHAPE(LL, WW) \
  if (sh.L == LL && sh.W == WW) PRNN_LAUNCH(LL, WW, false);
  PRNN_SHAPE(32, 8)
  PRNN_SHAPE(32, 4)
  PRNN_SHAPE(24, 4)
  PRNN_SHAPE(16, 8)
  PRNN_SHAPE(64, 4)
#undef PRNN_SHAPE
  }
  }
#undef PRNN_LAUNCH
}


template <typename TX>
static int run_newton(const TX* wx, const TX* r, const TX* h0, const TX* guess, TX* out, int B,
                      int T, int d, int K, float omega, float eps, const NewtonWs& w,
                      hipStream_t stream, const Packed& pk) {
  int rc = clear_status(w.lb, stream);
  if (rc != PRNN_OK) return rc;
  if (K == 0) {
    PRNN_HIP(hipMemcpyAsync(out, guess, static_cast<size_t>(B) * T * 4 * d * sizeof(TX),
                            hipMemcpyDeviceToDevice, stream));
    return PRNN_OK;
  }
  if (w.fused) {
    const Shape sh = newton_fused_shape(dtype_code<TX>());
    const Geo g = geometry(B, T, d, sh);
#define PRNN_LAUNCH(LL, WW, WPE, DD)                                                             \
  slstm_newton_fused_kernel<TX, LL, WW, WPE, DD, false>                                          \
      <<<dim3(g.n_tiles), dim3(64 * WW), 0, stream>>>(                                           \
          wx, r, h0, guess, out, B, T, d, g.n_cb, g.n_tiles, K, omega, eps, w.lb.counters + 1,   \
          w.lb.agg, w.lb.incl, w.hlast, w.lb.tag_base, w.lb.spin(), Packed{nullptr, nullptr, 0})
#define PRNN_SHAPE(LL, WW, WPE) \
  else if (sh.L == LL && sh.W == WW) PRNN_LAUNCH(LL, WW, WPE, false);
    static_assert(kNewtonFusedF32.L == 16 && kNewtonFusedF32.W == 4, "fp32 fused shape");
    static_assert(kNewtonFusedDefault.L == 20 && kNewtonFusedDefault.W == 4, "default shape");
    timing_begin(stream);
    if (pk.cu != nullptr) {
      launch_newton_fused_packed<TX>(wx, r, h0, guess, out, T, d, K, omega, eps, w.lb, w.hlast,
                                     stream, pk);
    } else if constexpr (sizeof(TX) == 4) {
      if (deterministic()) PRNN_LAUNCH(16, 4, 2, true);
      PRNN_SHAPE(16, 4, 2)
    } else {
      if (deterministic()) PRNN_LAUNCH(20, 4, 2, true);
      else if constexpr (std::is_same<TX, f16>::value) PRNN_LAUNCH(20, 4, 2, false);
      PRNN_SHAPE(20, 4, 2)
      PRNN_SHAPE(16, 4, 2)
      PRNN_SHAPE(24, 4, 2)
      PRNN_SHAPE(16, 8, 2)
    }
#undef PRNN_SHAPE
#undef PRNN_LAUNCH
    timing_end(stream);
    PRNN_HIP(hipGetLastError());
    return PRNN_OK;
  }
  timing_begin(stream);
  if (pk.cu != nullptr) {
    // K = 1 on a packed stream
    launch_newton_packed<TX, TX, TX>(wx, r, h0, guess, out, T, d, omega, eps, w.lb, 1, stream,
                                     pk);
    timing_end(stream);
    PRNN_HIP(hipGetLastError());
    return PRNN_OK;
  }
  for (int k = 1; k <= K; ++k) {
    const bool first = k == 1, last = k == K;
    const float* win = first ? nullptr : w.work[(k - 2) & 1];
    float* wout = last ? nullptr : w.work[(k - 1) & 1];
    if (first && last)
      launch_newton<TX, TX, TX>(wx, r, h0, guess, out, B, T, d, omega, eps, w.lb, k, stream);
    else if (first)
      launch_newton<TX, TX, float>(wx, r, h0, guess, wout, B, T, d, omega, eps, w.lb, k, stream);
    else if (last)
      launch_newton<TX, float, TX>(wx, r, h0, win, out, B, T, d, omega, eps, w.lb, k, stream);
    else
      launch_newton<TX, float, float>(wx, r, h0, win, wout, B, T, d, omega, eps, w.lb, k, stream);
    PRNN_HIP(hipGetLastError());
  }
  timing_end(stream);
  return PRNN_OK;
}

// fp16 storage, instantiated in slstm_diag_f16.hip.
int run_init_f16(const f16* wx, const f16* r, const f16* h0, f16* states, int B, int T, int d,
                 int P, float eps, const InitWs& w, hipStream_t stream, const Packed& pk);
int run_newton_f16(const f16* wx, const f16* r, const f16* h0, const f16* guess, f16* out, int B,
                   int T, int d, int K, float omega, float eps, const NewtonWs& w,
                   hipStream_t stream, const Packed& pk);
// One rectangular Newton iteration with an fp32 result; `in` is fp32 when in_f32, else fp16.
void launch_newton_step_f16(bool in_f32, const f16* wx, const f16* r, const f16* h0,
                            const void* in, float* out, int B, int T, int d, float omega,
                            float eps, const Lookback& lb, hipStream_t stream);

// A packed stream is one batch row of T steps holding n_seq non-empty
// sequences: cu_seqlens must rise strictly from 0 to T (the kernels locate
// heads by a binary search and a per-wave bit mask, which an empty sequence
// would make ambiguous).  The device cannot check the offsets without a host
// copy, so only what the sizes imply is rejected here.
static int check_packed(const slstm::Packed& pk, int B, int T) {
  if (pk.cu == nullptr) return PRNN_OK;
  if (B != 1) return fail(PRNN_ERR_VALUE, "a packed stream has B = 1, got B = %d", B);
  if (pk.n_seq < 1 || pk.n_seq > T)
    return fail(PRNN_ERR_VALUE, "n_seq must be in [1, T], got %d (T = %d)", pk.n_seq, T);
  return PRNN_OK;
}

}  // namespace slstm
}  // namespace prnn
