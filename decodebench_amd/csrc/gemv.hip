// gemv.hip -- batch-1 (to batch-8 per pass) fused GEMV kernels for gfx950.
//
// F1 (RMSNorm -> GEMV) and F2 (gate/up GEMV + SwiGLU) share one kernel body:
//
//  * A workgroup is 4 waves.  The activation rows it needs (x, or the
//    RMS-normalised x for F1) are built ONCE per workgroup in LDS; the
//    normalised vector never goes to HBM.
//  * Each wave owns groups of R consecutive weight rows and streams them with
//    128-bit non-temporal loads: lane l reads the 16-byte chunks l, l+64, ...
//    of a row, so one load instruction covers 1 KB of contiguous weights.
//  * Loads for the next (group, k-step) tile are issued before the current
//    tile is consumed (two register buffers), and the first tile is issued
//    before the F1 norm prologue so the prologue hides under HBM latency.
//  * Dot products are v_dot2_f32_f16 with fp32 accumulators; a group ends with
//    a DPP row reduction plus four v_readlane and a single fp16 store per
//    output.
//  * F2 keeps gate and up accumulators side by side and applies SiLU(g)*u in
//    registers, so neither projection is ever written.
//
// Rounding follows the reference stages (src/decodebench/demos/
// llama_decode.py:36-43 and 77-87): F1 rounds x*inv_rms to fp16 and then the
// product with gamma to fp16 before the GEMV; F2 rounds both projections to
// fp16, SiLU to fp16 and the final product to fp16.
#include <mutex>
#include <unordered_set>

#include "db_device.h"
#include "db_kernels.h"

namespace dbk {

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;

struct GemvArgs {
  const _Float16* x;      // [B, K]
  const _Float16* gamma;  // [K]         (RMSNorm mode)
  const _Float16* w0;     // [N, K]      (gate in SwiGLU mode)
  const _Float16* w1;     // [N, K]      (up, SwiGLU mode only)
  _Float16* y;            // [B, N]
  int B, K, N;
  int kchunks;            // 16-byte chunks per row = K / 8
  int steps;              // k-steps per row group
  int kp8;                // padded chunks per LDS activation row
  int groups;             // row groups = ceil(N / R)
  float eps;
};

__device__ __forceinline__ float silu(float g) {
  return g / (1.0f + __expf(-g));
}

template <int MODE, int NB, int R, int U>
__global__ __launch_bounds__(kThreads) void gemv_kernel(GemvArgs a) {
  constexpr int NW = (MODE == kGemvSwiGLU) ? 2 : 1;  // weight matrices
  extern __shared__ __align__(16) unsigned char lds_raw[];
  u4* xs = reinterpret_cast<u4*>(lds_raw);           // [NB][kp8]
  __shared__ float red[kWaves][NB];

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // wave-uniform
  const int b0 = blockIdx.y * NB;
  const int nb = min(NB, a.B - b0);
  const int stride_waves = gridDim.x * kWaves;
  const int last_chunk = a.kchunks - 1;

  const _Float16* wmat[2] = {a.w0, a.w1};

  // ---- tile loader: R rows x U chunks per lane (x2 for SwiGLU) ----------
  auto load_tile = [&](u4 (&dst)[NW][R][U], int grp, int st) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = min(grp * R + r, a.N - 1);
#pragma unroll
      for (int m = 0; m < NW; ++m) {
        const _Float16* wr = wmat[m] + (size_t)row * a.K;
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int c = min(st * (kWave * U) + u * kWave + lane, last_chunk);
          dst[m][r][u] = ld_stream(wr + (size_t)c * 8);
        }
      }
    }
  };

  // ---- activation chunks (and gamma) of the first kPre passes -> registers.
  // They are loaded before the first weight tile, so they arrive first and
  // the activation prologue overlaps the weight stream instead of waiting
  // behind it (loads complete in issue order).  The loads are unconditional
  // (clamped addresses, masked afterwards) and their uses straight-line, so
  // the compiler waits for them alone and not for the weights.
  constexpr int kPre = 2;  // covers K <= 2 * 256 * 8 = 4096 with no reload
  u4 xr[kPre][NB];
  u4 gr[kPre];
#pragma unroll
  for (int i = 0; i < kPre; ++i) {
    const int c = min((int)threadIdx.x + i * kThreads, a.kchunks - 1);
    gr[i] = u4{0, 0, 0, 0};
    if constexpr (MODE == kGemvRmsNorm) gr[i] = ld16(a.gamma + (size_t)c * 8);
#pragma unroll
    for (int b = 0; b < NB; ++b)
      xr[i][b] = ld16(a.x + (size_t)(b0 + min(b, nb - 1)) * a.K + (size_t)c * 8);
  }
  __builtin_amdgcn_sched_barrier(0);

  // The first tile load is unconditional (a wave past the last group loads
  // the last group's tile and never uses it), so no branch merges a state
  // with and without the weight loads in flight.
  u4 wbuf[2][NW][R][U];
  int grp = blockIdx.x * kWaves + wave;
  int st = 0;
  load_tile(wbuf[0], min(grp, a.groups - 1), 0);
  __builtin_amdgcn_sched_barrier(0);

  const u4 zero4 = {0, 0, 0, 0};
#pragma unroll
  for (int i = 0; i < kPre; ++i) {
    const bool valid_c = (int)threadIdx.x + i * kThreads < a.kchunks;
    gr[i] = valid_c ? gr[i] : zero4;
#pragma unroll
    for (int b = 0; b < NB; ++b) xr[i][b] = (valid_c && b < nb) ? xr[i][b] : zero4;
  }
  // Passes beyond kPre (K > 4096) read x and gamma again.
  const int c_rest = threadIdx.x + kPre * kThreads;
  auto x_rest = [&](int c, int b) -> u4 {
    return (c < a.kchunks && b < nb) ? ld16(a.x + (size_t)(b0 + b) * a.K + (size_t)c * 8)
                                     : zero4;
  };

  // ---- activation rows -> LDS (once per workgroup) ----------------------
  if constexpr (MODE == kGemvRmsNorm) {
    float ss[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) ss[b] = 0.0f;
    auto add_sq = [&](const u4& v, float& acc) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const h2 p = as_h2(v[j]);
        const float lo = (float)p[0], hi = (float)p[1];
        acc += lo * lo + hi * hi;
      }
    };
#pragma unroll
    for (int i = 0; i < kPre; ++i)
#pragma unroll
      for (int b = 0; b < NB; ++b) add_sq(xr[i][b], ss[b]);
    for (int c = c_rest; c < a.kchunks; c += kThreads)
#pragma unroll
      for (int b = 0; b < NB; ++b) add_sq(x_rest(c, b), ss[b]);
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const float sum = wave_sum(ss[b]);
      if (lane == 0) red[wave][b] = sum;
    }
    __syncthreads();
    float inv[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const float tot = (red[0][b] + red[1][b]) + (red[2][b] + red[3][b]);
      inv[b] = 1.0f / sqrtf(tot / (float)a.K + a.eps);
    }
    // fp16(x * inv_rms), then fp16(that * gamma): the fp16 x fp16 product is
    // exact in fp32, so one rounding matches torch.  Zero chunks stay zero.
    auto norm = [&](const u4& xv, const u4& gv, float iv) -> u4 {
      u4 out;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const h2 xp = as_h2(xv[j]);
        const h2 gp = as_h2(gv[j]);
        const float n0 = (float)to_h((float)xp[0] * iv);
        const float n1 = (float)to_h((float)xp[1] * iv);
        out[j] = pack_h2(n0 * (float)gp[0], n1 * (float)gp[1]);
      }
      return out;
    };
#pragma unroll
    for (int i = 0; i < kPre; ++i) {
      const int c = threadIdx.x + i * kThreads;
      if (c < a.kp8)
#pragma unroll
        for (int b = 0; b < NB; ++b) xs[b * a.kp8 + c] = norm(xr[i][b], gr[i], inv[b]);
    }
    for (int c = c_rest; c < a.kp8; c += kThreads) {
      const u4 gv = c < a.kchunks ? ld16(a.gamma + (size_t)c * 8) : zero4;
#pragma unroll
      for (int b = 0; b < NB; ++b) xs[b * a.kp8 + c] = norm(x_rest(c, b), gv, inv[b]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < kPre; ++i) {
      const int c = threadIdx.x + i * kThreads;
      if (c < a.kp8)
#pragma unroll
        for (int b = 0; b < NB; ++b) xs[b * a.kp8 + c] = xr[i][b];
    }
    for (int c = c_rest; c < a.kp8; c += kThreads)
#pragma unroll
      for (int b = 0; b < NB; ++b) xs[b * a.kp8 + c] = x_rest(c, b);
  }
  __syncthreads();

  // ---- main loop: consume tile (grp, st), prefetch the next -------------
  float acc[NW][R][NB];
#pragma unroll
  for (int m = 0; m < NW; ++m)
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int b = 0; b < NB; ++b) acc[m][r][b] = 0.0f;

  auto consume = [&](u4 (&cur)[NW][R][U], u4 (&nxt)[NW][R][U]) -> bool {
    int ngrp = grp, nst = st + 1;
    if (nst == a.steps) {
      nst = 0;
      ngrp = grp + stride_waves;
    }
    if (ngrp < a.groups) load_tile(nxt, ngrp, nst);

#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = st * (kWave * U) + u * kWave + lane;
      u4 xv[NB];
#pragma unroll
      for (int b = 0; b < NB; ++b) xv[b] = xs[b * a.kp8 + c];
#pragma unroll
      for (int m = 0; m < NW; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int b = 0; b < NB; ++b)
            acc[m][r][b] = dot8(cur[m][r][u], xv[b], acc[m][r][b]);
    }

    if (st == a.steps - 1) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int row = grp * R + r;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          float out;
          if constexpr (MODE == kGemvSwiGLU) {
            const float g = (float)to_h(wave_sum(acc[0][r][b]));
            const float u = (float)to_h(wave_sum(acc[1][r][b]));
            out = (float)to_h(silu(g)) * u;
          } else {
            out = wave_sum(acc[0][r][b]);
          }
          if (lane == 0 && row < a.N && b < nb)
            a.y[(size_t)(b0 + b) * a.N + row] = to_h(out);
#pragma unroll
          for (int m = 0; m < NW; ++m) acc[m][r][b] = 0.0f;
        }
      }
    }
    grp = ngrp;
    st = nst;
    return grp < a.groups;
  };

  if (grp < a.groups) {
    for (;;) {
      if (!consume(wbuf[0], wbuf[1])) break;
      if (!consume(wbuf[1], wbuf[0])) break;
    }
  }
}

using KernelFn = void (*)(GemvArgs);

template <int MODE, int NB, int R>
KernelFn pick_u(int u) {
  switch (u) {
    case 1: return gemv_kernel<MODE, NB, R, 1>;
    case 2: return gemv_kernel<MODE, NB, R, 2>;
    case 4: return gemv_kernel<MODE, NB, R, 4>;
    case 7: return gemv_kernel<MODE, NB, R, 7>;
    default: return gemv_kernel<MODE, NB, R, 8>;
  }
}

template <int MODE, int R>
KernelFn pick_nb(int nb, int u) {
  switch (nb) {
    case 1: return pick_u<MODE, 1, R>(u);
    case 2: return pick_u<MODE, 2, R>(u);
    case 4: return pick_u<MODE, 4, R>(u);
    default: return pick_u<MODE, 8, R>(u);
  }
}

// Rows per wave group: two rows for single-matrix modes, one gate/up row
// pair for SwiGLU -- both keep 16 x 16 B loads in flight per lane per tile.
constexpr int rows_per_group(GemvMode mode) { return mode == kGemvSwiGLU ? 1 : 2; }

// Chunks per lane per k-step: the largest U in {8,7,4,2,1} whose step
// (64*U chunks) divides the row exactly; otherwise 8 with a masked tail.
int pick_chunks_per_lane(int kchunks) {
  static const int cand[] = {8, 7, 4, 2, 1};
  for (int u : cand)
    if (kchunks % (kWave * u) == 0) return u;
  if (kchunks <= kWave) return 1;
  if (kchunks <= 2 * kWave) return 2;
  if (kchunks <= 4 * kWave) return 4;
  return 8;
}

// Number of waves.  Every wave gets ceil(groups / waves) row groups; a
// wave-per-CU budget is good when the chip's wave slots are >= 95% busy for
// the whole kernel.  Prefer the largest such budget (more loads in flight),
// else the best-balanced one.
int waves_for(int groups, int slots) {
  const int per = (groups + slots - 1) / slots;
  return (groups + per - 1) / per;
}

int pick_waves(int groups, int cu_count) {
  const int forced = tuning().gemv_waves_per_cu;
  if (forced > 0) return waves_for(groups, cu_count * forced);
  int best = 1;
  double best_eff = -1.0;
  for (int wpc : {16, 12, 8, 4}) {
    const int slots = cu_count * wpc;
    const int per = (groups + slots - 1) / slots;
    const double eff = (double)groups / ((double)per * slots);
    if (eff >= 0.95) return waves_for(groups, slots);
    if (eff > best_eff) {
      best_eff = eff;
      best = waves_for(groups, slots);
    }
  }
  return best;
}

// Raise a kernel's dynamic-LDS limit to the 152 KB activation budget, once
// per kernel function (the attribute is per function, not per launch).
hipError_t allow_large_lds(const void* fn) {
  static std::mutex mu;
  static std::unordered_set<const void*> done;
  std::lock_guard<std::mutex> lock(mu);
  if (done.count(fn)) return hipSuccess;
  hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                     152 * 1024);
  if (e == hipSuccess) done.insert(fn);
  return e;
}

}  // namespace

hipError_t launch_gemv(GemvMode mode, const void* x, const void* gamma,
                       const void* w0, const void* w1, void* y, int B, int K,
                       int N, float eps, int cu_count, hipStream_t stream) {
  if (B >= tuning().gemv_mfma_min_batch && gemv_mfma_supported(B, K, N))
    return launch_gemv_mfma(mode, x, gamma, w0, w1, y, B, K, N, eps, cu_count, stream);
  const int R = rows_per_group(mode);
  GemvArgs a;
  a.x = static_cast<const _Float16*>(x);
  a.gamma = static_cast<const _Float16*>(gamma);
  a.w0 = static_cast<const _Float16*>(w0);
  a.w1 = static_cast<const _Float16*>(w1);
  a.y = static_cast<_Float16*>(y);
  a.B = B;
  a.K = K;
  a.N = N;
  a.eps = eps;
  a.kchunks = K / 8;
  const int U = pick_chunks_per_lane(a.kchunks);
  a.steps = (a.kchunks + kWave * U - 1) / (kWave * U);
  a.kp8 = a.steps * kWave * U;
  a.groups = (N + R - 1) / R;

  // Batch rows per workgroup pass: as many as the batch and the LDS budget
  // (152 KB of the 160 KB per CU) allow.
  int nb = B >= 8 ? 8 : (B >= 4 ? 4 : (B >= 2 ? 2 : 1));
  while (nb > 1 && (size_t)nb * a.kp8 * 16 > 152 * 1024) nb /= 2;
  KernelFn fn;
  switch (mode) {
    case kGemvRmsNorm: fn = pick_nb<kGemvRmsNorm, 2>(nb, U); break;
    case kGemvSwiGLU: fn = pick_nb<kGemvSwiGLU, 1>(nb, U); break;
    default: fn = pick_nb<kGemvPlain, 2>(nb, U); break;
  }
  const size_t lds = (size_t)nb * a.kp8 * 16;
  if (lds > 48 * 1024) {
    hipError_t e = allow_large_lds(reinterpret_cast<const void*>(fn));
    if (e != hipSuccess) return e;
  }
  const int waves = pick_waves(a.groups, cu_count);
  dim3 grid((waves + kWaves - 1) / kWaves, (B + nb - 1) / nb);
  hipLaunchKernelGGL(fn, grid, dim3(kThreads), lds, stream, a);
  return hipGetLastError();
}

}  // namespace dbk
