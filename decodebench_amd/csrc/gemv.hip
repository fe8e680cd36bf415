// gemv.hip -- launcher of the decode GEMV family and its fp16-weight kernels.
//
// F1 (RMSNorm -> GEMV), F2 (gate/up GEMV + SwiGLU), the RMSNorm -> gate/up
// + SwiGLU pair of the decode-layer chain and the plain projection share one
// kernel template (gemv_valu.h).  This file instantiates its fp16-weight half
// and chooses the launch shape; gemv_fp8.hip instantiates the e4m3 half, and
// batches from 3 rows (2 for the e4m3 norm and gate/up modes and for plain
// rows longer than 4096) go to the MFMA kernels (gemv_mfma.hip): the
// crossovers measured on MI355X.
#include <mutex>
#include <unordered_map>

#include "gemv_valu.h"

namespace dbk {

GemvFn gemv_pick_f16(GemvMode mode, int nb, int u) { return gemv_pick<false>(mode, nb, u); }

namespace {

// Chunks per lane per k-step: the largest U in {8,7,4,2,1} whose step
// (64*U chunks) divides the row exactly; otherwise 8 with a masked tail.
int pick_chunks_per_lane(int chunks) {
  static const int cand[] = {8, 7, 4, 2, 1};
  for (int u : cand)
    if (chunks % (kWave * u) == 0) return u;
  if (chunks <= kWave) return 1;
  if (chunks <= 2 * kWave) return 2;
  if (chunks <= 4 * kWave) return 4;
  return 8;
}

// Number of waves: as many as 32 per CU, every wave owning the same number
// of row groups (ceil(groups / waves)).  Waves beyond what fits on a CU at
// once start as earlier ones finish; a launch of many short waves keeps the
// most weight bytes in flight (measured on MI355X: never slower than fewer,
// longer waves, and 10% faster for the fp8 gate/up pair).
int waves_for(int groups, int slots) {
  const int per = (groups + slots - 1) / slots;
  return (groups + per - 1) / per;
}

int pick_waves(int groups, int cu_count) {
  const int forced = tuning().gemv_waves_per_cu;
  return waves_for(groups, cu_count * (forced > 0 ? forced : 32));
}

// fp16 F1 at one batch row with 2 rows per wave instead of 1 (see
// launch_gemv).
GemvFn gemv_pick_f1_two_rows(int u) {
  constexpr int WV = gemv_wg_waves(kGemvRmsNorm, false, 1);
  switch (u) {
    case 1: return gemv_kernel<kGemvRmsNorm, 1, 2, 1, false, WV>;
    case 2: return gemv_kernel<kGemvRmsNorm, 1, 2, 2, false, WV>;
    case 4: return gemv_kernel<kGemvRmsNorm, 1, 2, 4, false, WV>;
    case 7: return gemv_kernel<kGemvRmsNorm, 1, 2, 7, false, WV>;
    default: return gemv_kernel<kGemvRmsNorm, 1, 2, 8, false, WV>;
  }
}

}  // namespace

hipError_t allow_large_lds(const void* fn, size_t dynamic_bytes) {
  static std::mutex mu;
  static std::unordered_map<const void*, size_t> limit;
  std::lock_guard<std::mutex> lock(mu);
  auto it = limit.find(fn);
  if (it == limit.end()) {
    // Whatever the 160 KB of LDS leave beside the kernel's static LDS, at
    // most 152 KB.
    hipFuncAttributes attr;
    hipError_t e = hipFuncGetAttributes(&attr, fn);
    if (e != hipSuccess) return e;
    size_t cap = (size_t)160 * 1024 - attr.sharedSizeBytes;
    if (cap > (size_t)152 * 1024) cap = (size_t)152 * 1024;
    e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)cap);
    if (e != hipSuccess) return e;
    it = limit.emplace(fn, cap).first;
  }
  return dynamic_bytes <= it->second ? hipSuccess : hipErrorInvalidValue;
}

hipError_t launch_gemv(GemvMode mode, const void* x, const void* gamma,
                       const GemvWeights& w, void* y, int B, int K, int N, float eps,
                       int cu_count, hipStream_t stream) {
  const int forced_min = tuning().gemv_mfma_min_batch;
  // At 3 rows the VALU kernel would run two 2-row passes, 1.5-1.8x the MFMA
  // time.  At 2 rows (graph back-to-back, us, VALU / MFMA) MFMA takes the
  // e4m3 modes with a norm or two matrices (F1 [4096, 4096] 5.87 / 5.46,
  // F1-QKV 7.17 / 6.81, gate/up pair 22.4 / 19.2, RMSNorm -> gate/up 23.2 /
  // 19.8) and rows longer than 4096 (down projection [4096, 14336] fp16
  // 20.9 / 20.1, e4m3 14.0 / 11.7); the VALU kernel keeps fp16 F1 (7.72 /
  // 7.88; F1-QKV 10.36 / 10.16-10.46), the fp16 pair (35.4 / 36.9,
  // RMSNorm -> gate/up 36.5 / 36.8) and the plain projection at K = 4096
  // (fp16 6.95 / 7.24, e4m3 4.54 / 5.11).
  const bool mfma_at_two = (w.fp8 && mode != kGemvPlain) || (mode == kGemvPlain && K > 4096);
  const int auto_min = mfma_at_two ? 2 : 3;
  const int mfma_min = forced_min > 0 ? forced_min : auto_min;
  if (B >= mfma_min && gemv_mfma_supported(mode, B, K, N))
    return launch_gemv_mfma(mode, x, gamma, w, y, B, K, N, eps, cu_count, stream);
  GemvArgs a;
  a.x = static_cast<const _Float16*>(x);
  a.gamma = static_cast<const _Float16*>(gamma);
  a.w0 = w.w0;
  a.w1 = w.w1;
  a.s0 = w.s0;
  a.s1 = w.s1;
  a.y = static_cast<_Float16*>(y);
  a.B = B;
  a.K = K;
  a.N = N;
  a.eps = eps;
  a.kchunks = K / 8;
  a.wchunks = w.fp8 ? K / 16 : K / 8;
  // Activation chunks one k-step spans (two per weight chunk for fp8); the
  // row is padded to whole k-steps.  Near the LDS budget a masked 8-chunk
  // step can pad an e4m3 row past it (K = 77808: 4863 weight chunks pad to
  // 5120, 160 KB of activations); fewer chunks per lane pad less.
  int U = pick_chunks_per_lane(a.wchunks);
  auto padded_chunks = [&](int u) {
    return (a.wchunks + kWave * u - 1) / (kWave * u) * kWave * u * (w.fp8 ? 2 : 1);
  };
  while (U > 1 && (size_t)padded_chunks(U) * 16 > 152 * 1024) U = U >= 7 ? 4 : U / 2;
  a.steps = (a.wchunks + kWave * U - 1) / (kWave * U);
  a.kp8 = padded_chunks(U);
  // Batch rows per workgroup pass: as many as the batch and the LDS budget
  // (152 KB of the 160 KB per CU) allow.
  int nb = B >= 8 ? 8 : (B >= 4 ? 4 : (B >= 2 ? 2 : 1));
  while (nb > 1 && (size_t)nb * a.kp8 * 16 > 152 * 1024) nb /= 2;
  int R = gemv_rows_per_group(mode, w.fp8, U, nb);
  // fp16 F1 at one batch row (8-wave workgroups): 2 rows per wave when that
  // gives every CU the same number of whole workgroups (N / 16 a multiple of
  // the CU count), else 1.  Measured at K = 4096: N = 4096 with 2 rows
  // 6.90 -> 6.64 us (one workgroup per CU); N = 6144 with 2 rows 9.21 ->
  // 10.18 us (1.5 workgroups per CU).
  const bool f1_two_rows = !w.fp8 && mode == kGemvRmsNorm && nb == 1 && R == 1 &&
                           ((N + 15) / 16) % cu_count == 0;
  if (f1_two_rows) {
    R = 2;
    // Two rows of 4 chunks per lane keep the 8 KB tile of the one-row shape
    // (F1 at N = 4096: 6.77 -> 6.64 us against 8 chunks).  Fewer chunks per
    // lane pad the activation row no more, so the LDS size only shrinks.
    if (U == 8) {
      U = 4;
      a.steps = (a.wchunks + kWave * U - 1) / (kWave * U);
      a.kp8 = padded_chunks(U);
    }
  }
  // e4m3 plain projection at one batch row with rows longer than 4096: 8-wave
  // workgroups of one row per wave (see kWavesFp8PlainLong).
  const bool fp8_long_rows = w.fp8 && mode == kGemvPlain && nb == 1 && K > 4096;
  if (fp8_long_rows) R = 1;
  a.groups = (N + R - 1) / R;
  const GemvFn fn = f1_two_rows     ? gemv_pick_f1_two_rows(U)
                    : fp8_long_rows ? gemv_pick_fp8_plain_long(U)
                    : w.fp8         ? gemv_pick_fp8(mode, nb, U)
                                    : gemv_pick_f16(mode, nb, U);
  const size_t lds = (size_t)nb * a.kp8 * 16;
  if (lds > 48 * 1024) {
    hipError_t e = allow_large_lds(reinterpret_cast<const void*>(fn), lds);
    if (e != hipSuccess) return e;
  }
  const int wv = fp8_long_rows ? kWavesFp8PlainLong : gemv_wg_waves(mode, w.fp8, nb);
  // fp16 F1 with one row per wave: one 8-wave workgroup per CU, each wave
  // walking its rows in turn, so every CU streams the same rows and runs the
  // activation prologue once.  Measured on MI355X (graph back-to-back):
  // F1-QKV 9.2 -> 9.05 us; with up to 32 waves per CU the 768 workgroups of
  // 8 rows run in two rounds (two resident per CU at 91 VGPRs) and some CUs
  // take a fourth.  e4m3 F1 (4-wave workgroups of 2 rows) takes one
  // workgroup per CU the same way: F1-QKV 6.07-6.11 -> 5.75-5.79 us, F1
  // 4.67 -> 4.58-4.61 us.  The plain projection keeps the default (the fp16
  // decode layer measured 0.1-0.5 us slower with it), except the e4m3 rows
  // longer than 4096, whose 8-wave workgroups of one row per wave gain from
  // it (down projection [4096, 14336] 11.08-11.12 -> 10.73-10.79 us; a sweep
  // of 1-16 workgroups' worth of waves per CU found nothing better for the
  // fp16 projections or RMSNorm -> gate/up).
  const bool persistent = ((mode == kGemvRmsNorm && nb == 1 &&
                            (w.fp8 || (R == 1 && wv == 8))) ||
                           fp8_long_rows) &&
                          tuning().gemv_waves_per_cu <= 0;
  const int waves = persistent ? waves_for(a.groups, cu_count * wv)
                               : pick_waves(a.groups, cu_count);
  dim3 grid((waves + wv - 1) / wv, (B + nb - 1) / nb);
  // F2's single-wave workgroups of one row number their row groups by XCD in
  // 32-row slices, so each XCD writes whole output sectors: WRITE_SIZE drops
  // from 8x its 28 KB output to about 1x.  RMSNorm -> gate/up keeps launch
  // order (the fp16 decode layer measured 0.4 us slower with the slices).
  a.xcd_rows = (mode == kGemvSwiGLU && wv == 1 && R == 1 && grid.x % 8 == 0) ? 1 : 0;
  hipLaunchKernelGGL(fn, grid, dim3(wv * kWave), lds, stream, a);
  return hipGetLastError();
}

}  // namespace dbk
