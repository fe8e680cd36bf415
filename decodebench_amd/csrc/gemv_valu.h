// gemv_valu.h -- the batch-1 (to batch-8 per pass) GEMV kernel template for
// gfx950, shared by the fp16-weight (gemv.hip) and fp8-weight (gemv_fp8.hip)
// translation units, which instantiate disjoint halves of it.
//
//  * A workgroup is 4 waves (1 for the fp16 gate/up pair and 8 for the
//    other fp16 modes at one batch row, see gemv_wg_waves).  The
//    activation rows it needs (x, or the RMS-normalised x) are built ONCE
//    per workgroup in LDS; the normalised vector never goes to HBM.
//  * Each wave owns groups of R consecutive weight rows and streams them with
//    128-bit non-temporal loads: lane l reads the 16-byte chunks l, l+64, ...
//    of a row, so one load instruction covers 1 KB of contiguous weights.
//  * Loads for the next (group, k-step) tile are issued before the current
//    tile is consumed (two register buffers).  They are buffer loads whose
//    resource covers only valid rows, so the prefetch past a wave's last
//    tile reads nothing and every load is unconditional; and the first tile
//    is issued before the norm prologue so the prologue hides under HBM
//    latency.
//  * Dot products are v_dot2_f32_f16 with fp32 accumulators; a group ends with
//    a DPP row reduction plus four v_readlane and a single fp16 store per
//    output.
//  * The SwiGLU modes keep gate and up accumulators side by side and apply
//    SiLU(g)*u in registers, so neither projection is ever written.
//  * fp8 weights (OCP e4m3): a 16-byte chunk is 16 weights.  Each 32-bit word
//    is widened to two fp16 pairs by v_cvt_scalef32_pk_f16_fp8 (exact: every
//    e4m3 value is an fp16 value) and dotted against two fp16 activation
//    chunks; the row's fp32 scale multiplies the reduced sum, loaded with the
//    tile so it arrives with the weights.
//
// Rounding follows the reference stages (src/decodebench/demos/
// llama_decode.py:36-43 and 77-87): the norm rounds x*inv_rms to fp16 and
// then the product with gamma to fp16 before the GEMV; SwiGLU rounds both
// projections to fp16, SiLU to fp16 and the final product to fp16.
#pragma once

#include "db_device.h"
#include "db_kernels.h"

namespace dbk {

// Waves per workgroup.  Measured on MI355X at K = 4096, one batch row
// (graph back-to-back, interleaved runs): the fp16 gate/up pair streams
// fastest with single-wave workgroups, which start and retire independently
// (F2 35.2 -> 33.9 us, RMSNorm->F2 36.3 -> 35.7 us); fp16 F1 and the plain
// projection with 8 waves sharing one activation prologue (F1-QKV 9.51 ->
// 9.21 us, F1 6.90 -> 6.75 us, plain [4096, 14336] 19.17 -> 18.45 us,
// [14336, 4096] 19.18 -> 18.85 us); every other batch and weight type is
// fastest with 4 waves (single waves cost up to 1.5x on the e4m3
// projections and F1, 8 waves lose on e4m3 F1).
constexpr int gemv_wg_waves(int mode, bool fp8, int nb) {
  if (fp8 || nb != 1) return 4;
  return gemv_is_swiglu(mode) ? 1 : 8;
}

struct GemvArgs {
  const _Float16* x;      // [B, K]
  const _Float16* gamma;  // [K]         (norm modes)
  const void* w0;         // [N, K]      (gate in the SwiGLU modes)
  const void* w1;         // [N, K]      (up, SwiGLU modes only)
  const float* s0;        // [N]         fp8 row scales of w0
  const float* s1;        // [N]         fp8 row scales of w1
  _Float16* y;            // [B, N]
  int B, K, N;
  int kchunks;            // 16-byte activation chunks per row = K / 8
  int wchunks;            // 16-byte weight chunks per row (K / 8 fp16, K / 16 fp8)
  int steps;              // k-steps per row group
  int kp8;                // padded activation chunks per LDS row
  int groups;             // row groups = ceil(N / R)
  int xcd_rows;           // 1: row groups numbered so that every 32 groups of
                          // output rows belong to one XCD (see phys below)
  float eps;
};

using GemvFn = void (*)(GemvArgs);

// Kernel choice per weight type (each defined in its own translation unit).
GemvFn gemv_pick_f16(GemvMode mode, int nb, int u);
GemvFn gemv_pick_fp8(GemvMode mode, int nb, int u);
// The e4m3 plain projection at one batch row with rows longer than 4096:
// 8-wave workgroups of one row per wave, which share each workgroup's
// activation fill (K x 2 bytes) among twice the weight bytes (measured:
// [4096, 14336] 11.80 -> 11.02 us, e4m3 decode layer 53.4 -> 52.6 us; at
// K = 4096 they cost 0.24 us, so shorter rows keep the default).
constexpr int kWavesFp8PlainLong = 8;
GemvFn gemv_pick_fp8_plain_long(int u);

// Raise a kernel's dynamic-LDS limit to what the 160 KB of LDS leave beside
// its static LDS (at most 152 KB), once per kernel function (the attribute
// is per function, not per launch), and check that `dynamic_bytes` fits.
// Defined in gemv.hip.
hipError_t allow_large_lds(const void* fn, size_t dynamic_bytes);

// Rows per wave group, measured on MI355X at the decode shapes: fp16 keeps
// 16 loads of 16 bytes per lane per tile (2 rows x 8 chunks, or the gate/up
// pair x 1 row), except F1 and the plain projection at one batch row,
// whose 8-wave workgroups take 1 row per wave (8 KB tiles; 1 row at two
// batch rows measured slower; the launcher gives F1 2 rows where that
// fills every CU with whole workgroups); e4m3 rows are half as long, and 2
// rows per group (8 loads for one matrix, 16 for the pair) beat both 1 and
// 4 rows at K = 4096.
constexpr int gemv_rows_per_group(int mode, bool fp8, int u, int nb) {
  const int nw = gemv_is_swiglu(mode) ? 2 : 1;
  if (!fp8 && nw == 1 && nb == 1) return 1;
  if (!fp8) return nw == 2 ? 1 : 2;
  return u <= 4 ? 2 : (nw == 1 ? 2 : 1);
}

namespace {

__device__ __forceinline__ float gemv_silu(float g) {
  return g / (1.0f + __expf(-g));
}

// 16 e4m3 weights -> two chunks of 8 fp16 (lo: weights 0..7, hi: 8..15).
__device__ __forceinline__ void e4m3x16_to_h(const u4& w, u4& lo, u4& hi) {
  lo[0] = __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w[0], 1.0f, false));
  lo[1] = __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w[0], 1.0f, true));
  lo[2] = __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w[1], 1.0f, false));
  lo[3] = __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w[1], 1.0f, true));
  hi[0] = __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w[2], 1.0f, false));
  hi[1] = __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w[2], 1.0f, true));
  hi[2] = __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w[3], 1.0f, false));
  hi[3] = __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w[3], 1.0f, true));
}

template <int MODE, int NB, int R, int U, bool FP8, int WV>
__global__ __launch_bounds__(WV * kWave) void gemv_kernel(GemvArgs a) {
  constexpr bool kNorm = gemv_has_norm(MODE);
  constexpr int NW = gemv_is_swiglu(MODE) ? 2 : 1;  // weight matrices
  constexpr int kThreads = WV * kWave;
  constexpr int kWaves = WV;
  extern __shared__ __align__(16) unsigned char lds_raw[];
  u4* xs = reinterpret_cast<u4*>(lds_raw);           // [NB][kp8]
  __shared__ float red[kWaves][NB];

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // wave-uniform
  const int b0 = blockIdx.y * NB;
  const int nb = min(NB, a.B - b0);
  const int stride_waves = gridDim.x * kWaves;
  const size_t row_bytes = FP8 ? (size_t)a.K : (size_t)a.K * 2;

  const unsigned char* wmat[2] = {static_cast<const unsigned char*>(a.w0),
                                  static_cast<const unsigned char*>(a.w1)};
  // A wave walks logical groups q = grp0, grp0 + stride_waves, ...  With
  // xcd_rows set (single-wave workgroups of one row, a grid of a multiple of
  // 8) every q of a workgroup has q % 8 == blockIdx.x % 8, the class of
  // workgroups that share an XCD, and q maps to the physical group
  //   256 (j / 32) + 32 (q % 8) + j % 32,   j = q / 8:
  // each block of 256 rows still goes to the 256 workgroups that come up
  // together, but its 32-row slices (64 bytes of fp16 outputs, two whole
  // 32-byte sectors) go to one XCD each, so every output sector is written
  // back once instead of once per XCD.  Measured on MI355X (F2, batch 1,
  // interleaved): 33.78-33.82 us against 33.82-33.89 us for launch order;
  // 16- and 8-row slices streamed 0.2-0.3 us slower, whole contiguous
  // eighths of the matrix per XCD 1.5x slower (34.2 -> 51.6 us).
  const int gspan = a.xcd_rows ? (a.groups + 255) / 256 * 256 : a.groups;
  auto phys = [&](int q) {
    return a.xcd_rows ? ((q >> 8) << 8) + ((q & 7) << 5) + ((q >> 3) & 31) : q;
  };

  // ---- tile loader: R rows x U chunks per lane (x2 for SwiGLU), issued in
  // the order consume() uses them (chunk-major), so each wait is for the
  // oldest loads only.  The loads go through buffer resources that cover the
  // group's valid rows: a tile past the wave's last group (or rows past N)
  // reads zeros without touching memory, so every tile load is issued
  // unconditionally.  fp8 tiles add one vector load that brings the NW x R
  // row scales (lane m*R + r holds the scale of matrix m, row r); a vector
  // load keeps the scalar-memory counter, which LDS reads share, clear.
  auto load_tile = [&](u4 (&dst)[NW][R][U], float& sc, int grp, int st) {
    const int pg = phys(grp);
    const bool live = pg < a.groups;
    const int g = live ? pg : a.groups - 1;  // base stays inside the matrix
    const int rows = live ? min(R, a.N - g * R) : 0;
    __amdgpu_buffer_rsrc_t rs[NW];
#pragma unroll
    for (int m = 0; m < NW; ++m)
      rs[m] = make_rsrc(wmat[m] + (size_t)g * R * row_bytes, rows * (int)row_bytes);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int off = (st * (kWave * U) + u * kWave + lane) * 16;
#pragma unroll
      for (int m = 0; m < NW; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r) dst[m][r][u] = ld_buf_stream(rs[m], r * (int)row_bytes + off);
    }
    if constexpr (FP8) {
      const int sl = lane % (NW * R);
      // A select of the two kernel-argument pointers, not an index into a
      // local pointer array: the compiler then knows the scales are global
      // memory.  Through the array it issued a flat load, after which every
      // wait became vmcnt(0), and the activation staging waited for the
      // whole first weight tile (read in the ISA).
      const float* sp = sl < R ? a.s0 : a.s1;
      sc = sp[min(g * R + sl % R, a.N - 1)];
    }
  };

  // ---- activation chunks (and gamma) of the first kPre passes -> registers.
  // They are loaded before the first weight tile, so they arrive first and
  // the activation prologue overlaps the weight stream instead of waiting
  // behind it (loads complete in issue order).  The loads are unconditional
  // (clamped addresses, masked afterwards) and their uses straight-line, so
  // the compiler waits for them alone and not for the weights.
  // Passes of 16-byte chunks per thread covering K <= 4096 with no reload.
  constexpr int kPre = 512 / kThreads >= 1 ? 512 / kThreads : 1;
  static_assert((kPre * kThreads & (kPre * kThreads - 1)) == 0, "slot count: power of 2");
  // Pass i of thread t fills chunk pre_chunk(i), a permutation of the
  // kPre * kThreads slots rotated by 1 KB per workgroup: workgroups on one
  // XCD (w, w + 8, ...) and on neighbouring XCDs start on different parts
  // of x, which every workgroup reads.
  const int rot = 64 * (((int)blockIdx.x + ((int)blockIdx.x >> 3)) & 7);
  auto pre_chunk = [&](int i) {
    return ((int)threadIdx.x + i * kThreads + rot) & (kPre * kThreads - 1);
  };
  u4 xr[kPre][NB];
  u4 gr[kPre];
#pragma unroll
  for (int i = 0; i < kPre; ++i) {
    const int c = min(pre_chunk(i), a.kchunks - 1);
    gr[i] = u4{0, 0, 0, 0};
    if constexpr (kNorm) gr[i] = ld16(a.gamma + (size_t)c * 8);
#pragma unroll
    for (int b = 0; b < NB; ++b)
      xr[i][b] = ld16(a.x + (size_t)(b0 + min(b, nb - 1)) * a.K + (size_t)c * 8);
  }
  __builtin_amdgcn_sched_barrier(0);

  // The wave's tiles are (group, k-step) pairs: groups grp0, grp0 + stride,
  // ... below a.groups, each in a.steps k-steps.  The first tile is requested
  // before the activation prologue (a wave with no group requests an empty
  // tile, which reads nothing).
  u4 wbuf[2][NW][R][U];
  float wsc[2] = {0.0f, 0.0f};
  const int grp0 = blockIdx.x * kWaves + wave;
  const int ntiles =
      grp0 < gspan ? (gspan - grp0 + stride_waves - 1) / stride_waves * a.steps : 0;
  load_tile(wbuf[0], wsc[0], grp0, 0);
  __builtin_amdgcn_sched_barrier(0);

  const u4 zero4 = {0, 0, 0, 0};
#pragma unroll
  for (int i = 0; i < kPre; ++i) {
    const bool valid_c = pre_chunk(i) < a.kchunks;
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
  if constexpr (kNorm) {
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
      float tot = 0.0f;
#pragma unroll
      for (int v = 0; v < kWaves; ++v) tot += red[v][b];
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
      const int c = pre_chunk(i);
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
      const int c = pre_chunk(i);
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

  // Dot products of tile (grp, st); after the row group's last k-step, the
  // reduction, epilogue and fp16 store (rows past N store nothing).
  auto consume = [&](const u4 (&cur)[NW][R][U], float csc, int grp, int st) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = st * (kWave * U) + u * kWave + lane;  // weight chunk
      if constexpr (FP8) {
        u4 xlo[NB], xhi[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          xlo[b] = xs[b * a.kp8 + 2 * c];
          xhi[b] = xs[b * a.kp8 + 2 * c + 1];
        }
#pragma unroll
        for (int m = 0; m < NW; ++m)
#pragma unroll
          for (int r = 0; r < R; ++r) {
            u4 wl, wh;
            e4m3x16_to_h(cur[m][r][u], wl, wh);
#pragma unroll
            for (int b = 0; b < NB; ++b)
              acc[m][r][b] = dot8(wh, xhi[b], dot8(wl, xlo[b], acc[m][r][b]));
          }
      } else {
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
    }

    if (st == a.steps - 1) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int row = phys(grp) * R + r;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          float out;
          if constexpr (NW == 2) {
            float g = wave_sum(acc[0][r][b]);
            float u = wave_sum(acc[1][r][b]);
            if constexpr (FP8) {
              g *= lane_value(csc, r);
              u *= lane_value(csc, R + r);
            }
            g = (float)to_h(g);
            u = (float)to_h(u);
            out = (float)to_h(gemv_silu(g)) * u;
          } else {
            out = wave_sum(acc[0][r][b]);
            if constexpr (FP8) out *= lane_value(csc, r);
          }
          if (lane == 0 && row < a.N && b < nb)
            a.y[(size_t)(b0 + b) * a.N + row] = to_h(out);
#pragma unroll
          for (int m = 0; m < NW; ++m) acc[m][r][b] = 0.0f;
        }
      }
    }
  };

  auto advance = [&](int& grp, int& st) {
    if (++st == a.steps) {
      st = 0;
      grp += stride_waves;
    }
  };

  // Two register buffers, one straight-line path: the next tile's load is
  // always issued before the current tile is consumed, so the compiler's
  // wait before each use is for the current tile alone and the next one
  // stays in flight.  With an even tile count the last load of the loop is
  // an empty tile (it reads nothing); an odd count ends with the tile the
  // loop (or the prologue) already requested.
  int ga = grp0, sa = 0;
  int t = 0;
  for (; t + 2 <= ntiles; t += 2) {
    int gb = ga, sb = sa;
    advance(gb, sb);
    load_tile(wbuf[1], wsc[1], gb, sb);
    __builtin_amdgcn_sched_barrier(0);  // all of the next tile goes out first
    consume(wbuf[0], wsc[0], ga, sa);
    ga = gb;
    sa = sb;
    advance(ga, sa);
    load_tile(wbuf[0], wsc[0], ga, sa);
    __builtin_amdgcn_sched_barrier(0);
    consume(wbuf[1], wsc[1], gb, sb);
  }
  if (t < ntiles) consume(wbuf[0], wsc[0], ga, sa);
}

// Kernel table of one weight type: mode x batch rows per pass x chunks per
// lane, with R fixed by gemv_rows_per_group.
template <int MODE, int NB, bool FP8>
GemvFn gemv_pick_u(int u) {
  constexpr int WV = gemv_wg_waves(MODE, FP8, NB);
  switch (u) {
    case 1: return gemv_kernel<MODE, NB, gemv_rows_per_group(MODE, FP8, 1, NB), 1, FP8, WV>;
    case 2: return gemv_kernel<MODE, NB, gemv_rows_per_group(MODE, FP8, 2, NB), 2, FP8, WV>;
    case 4: return gemv_kernel<MODE, NB, gemv_rows_per_group(MODE, FP8, 4, NB), 4, FP8, WV>;
    case 7: return gemv_kernel<MODE, NB, gemv_rows_per_group(MODE, FP8, 7, NB), 7, FP8, WV>;
    default: return gemv_kernel<MODE, NB, gemv_rows_per_group(MODE, FP8, 8, NB), 8, FP8, WV>;
  }
}

template <int MODE, bool FP8>
GemvFn gemv_pick_nb(int nb, int u) {
  switch (nb) {
    case 1: return gemv_pick_u<MODE, 1, FP8>(u);
    case 2: return gemv_pick_u<MODE, 2, FP8>(u);
    case 4: return gemv_pick_u<MODE, 4, FP8>(u);
    default: return gemv_pick_u<MODE, 8, FP8>(u);
  }
}

template <bool FP8>
GemvFn gemv_pick(GemvMode mode, int nb, int u) {
  switch (mode) {
    case kGemvRmsNorm: return gemv_pick_nb<kGemvRmsNorm, FP8>(nb, u);
    case kGemvSwiGLU: return gemv_pick_nb<kGemvSwiGLU, FP8>(nb, u);
    case kGemvRmsNormSwiGLU: return gemv_pick_nb<kGemvRmsNormSwiGLU, FP8>(nb, u);
    default: return gemv_pick_nb<kGemvPlain, FP8>(nb, u);
  }
}

}  // namespace

}  // namespace dbk
