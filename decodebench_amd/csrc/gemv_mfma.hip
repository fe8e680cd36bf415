// gemv_mfma.hip -- batched decode GEMV on MFMA for gfx950: gemv_mfma_kernel
// (passes of 16 or 32 batch rows), and the kernels that also stream the
// activations, gemv_mfma_long_kernel (rows longer than 4096) and
// gemv_mfma_tile16_kernel (the gate/up pair above 16 rows).
//
// y[B,N] = op(x[B,K]) . W^T for the four GEMV modes of gemv.hip (plain,
// RMSNorm-fused F1, gate/up + SwiGLU F2, RMSNorm -> gate/up + SwiGLU) with
// fp16 or e4m3 weights when the batch is large enough that the VALU
// dot-product path becomes instruction-bound (at batch 8 it runs at a third
// of HBM speed).  The weights are still read exactly once; MFMA does the
// multiply-adds.
//
// Decomposition
//  * One persistent workgroup per CU and pass, 8 waves (above 16 rows the
//    passes split the CUs, see launch_gemv_mfma).  Each wave owns one K-slice
//    (K / 8 columns) of every weight row, split into halves h = 0, 1.
//  * Weight rows are taken in groups of 8, which spreads N / 8 groups evenly
//    over the CUs at N = 4096, 6144 and 14336.  One v_mfma_f32_16x16x32_f16
//    covers 8 rows x both halves: A-operand rows 0..7 are the group's rows
//    over half 0 and rows 8..15 the same rows over half 1; B-operand columns
//    0..7 are 8 batch rows over half 0 and columns 8..15 the same batch rows
//    over half 1.  D[m][n] + D[m+8][n+8] is then the slice's dot product of
//    weight row m and batch row n (the off-diagonal quarters are dropped),
//    and every loaded weight byte is used.
//  * The activation slice of up to 16 batch rows (two column tiles of 8)
//    stays in registers for the whole kernel in that B-operand layout;
//    lane (g, n) holds x[b][k0 + 32 t + 8 g .. + 7] of its half.
//  * Workgroup w owns groups w, w + grid, ...; each wave streams its slice of
//    them with 16-byte loads through two register sets of one group each
//    (load set B, consume A, reload A, consume B).
//  * Each wave's partial sums (8 rows x 16 batch per group) go to LDS; after
//    the last group the workgroup reduces the 8 K-slices and applies the
//    epilogue (fp16 rounding, or SiLU(g) * u with the reference's rounding
//    points), storing only the final fp16 outputs.
//  * Norm modes: each wave sums x^2 over its slice and the 8 partial sums
//    meet in LDS; every wave multiplies its own x registers by gamma (read
//    from an LDS copy), fp16(x * gamma), and the epilogue scales each batch
//    row's sums by its inv_rms: y = fp16(inv_rms * sum_k W fp16(x gamma)),
//    so the statistic is off the path to the first product.  (32-row XB
//    passes normalise as the torch stage rounds, see norm_mul.)
// Batches above 16 run as passes of 16 rows (grid.y).  For one weight
// matrix the passes of a row group run on one XCD at the same time, so the
// later passes read its weights from L2 (see launch_gemv_mfma); 32-row
// passes with rows 16..31 of x in LDS (XB) remain as a tuning option.
// Plain GEMV with longer rows (K a multiple of 2048 above 4096, the down
// projection) and the gate/up pair above 16 rows, with or without the
// RMSNorm, take kernels that stream x as well: gemv_mfma_long_kernel and
// gemv_mfma_tile16_kernel (below).
#include "gemv_valu.h"

namespace dbk {

namespace {

constexpr int kWavesM = 8;

// fp16(fp16(x * inv) * gamma) on 8 packed halves.  x * inv is one
// v_fma_mix per half (f16 x f32 + 0, written to the low or high half of the
// result), which rounds the exact product to fp16 once; the torch stage
// rounds it to fp32 and then to fp16, and the two differ by one fp16 ulp in
// 360 of 4,063,232 (x, inv) pairs (every finite fp16 x against 64 values of
// inv, checked on MI355X).  The product with gamma is one v_pk_mul_f16 per
// pair: the exact fp16 x fp16 product rounded once, as the fp32 product the
// stage rounds.  Three VALU operations per pair against seven through fp32
// conversions.
__device__ __forceinline__ u4 norm_mul(const u4& x, const u4& g, float inv) {
  u4 out;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    unsigned r;
    asm("v_fma_mixlo_f16 %0, %1, %2, 0 op_sel_hi:[1,0,0]\n\t"
        "v_fma_mixhi_f16 %0, %1, %2, 0 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
        : "=&v"(r)
        : "v"(x[j]), "v"(inv));
    out[j] = __builtin_bit_cast(unsigned, as_h2(r) * as_h2(g[j]));
  }
  return out;
}
// LDS slot of lane (g4, h, r8) at k-step t within a (batch tile, k-step)
// block of 64 activation chunks, where staged and XB activations live: the
// low four bits are XOR-swizzled by g4 and t so that both the staging
// writes (one row's chunks: fixed r8, every t, h, g4) and the operand reads
// (64 consecutive lanes) spread over all LDS banks; unswizzled, the writes
// of one instruction met in 2 bank groups (a 32-way conflict).
__device__ __forceinline__ int xslot(int g, int h, int r, int t) {
  return 16 * g + ((8 * h + r) ^ (g | ((t & 1) << 2)));
}
constexpr int kThreadsM = kWavesM * kWave;
constexpr int kRowsPerGroup = 8;
constexpr int kBatchTile = 16;
// Groups per workgroup: 16 keeps the gate/up pair of N = 14336 (3584
// groups) on one workgroup per CU, 14 groups each.
constexpr int kMaxGroupsPerWg = 16;

struct MfmaArgs {
  const _Float16* x;      // [B, K]
  const _Float16* gamma;  // [K]     (norm modes)
  const void* w0;         // [N, K]  fp16 or e4m3 (gate in the SwiGLU modes)
  const void* w1;         // [N, K]  (up, SwiGLU modes only)
  const float* s0;        // [N]     e4m3 row scales of w0
  const float* s1;        // [N]     e4m3 row scales of w1
  _Float16* y;            // [B, N]
  int B, K, N;
  int groups;             // ceil(N / 8)
  int gpw;                // groups per workgroup (<= kMaxGroupsPerWg)
  int part_off;           // 16-byte units from the activation staging area to the
                          // partial sums: 0 when they share it, else past it
  float eps;
};

// KH: k-steps (32 columns each) per half slice, K / 512.
// BT: batch column tiles of 8 (1 for batch <= 8, 2 for <= 16).
// FP8: e4m3 weights.  A 16-byte load then holds 16 weights, the A operands
// of two k-steps after v_cvt_scalef32_pk_f16_fp8 widening.  The activations
// are loaded in the same column order, so the dot products are unchanged;
// the row scales multiply the reduced sums in the epilogue.
// XB (one weight matrix, BT = 2; a tuning option, db_tune("gemv_xb", 1)): a
// pass is 32 batch rows.  Rows 16..31 get two more column tiles whose
// activation slices are written once to LDS (each wave its own, 16 KB x KH /
// 8 per wave) and read back per group, so every weight tile feeds 32 rows in
// one workgroup; the default instead runs two 16-row passes that share the
// weights through an XCD's L2.
template <int MODE, int KH, int BT, bool FP8, bool XB>
__global__ __launch_bounds__(kThreadsM) void gemv_mfma_kernel(MfmaArgs a) {
  constexpr int NWM = gemv_is_swiglu(MODE) ? 2 : 1;
  constexpr int KW = FP8 ? KH / 2 : KH;  // 16-byte weight loads per row and slice
  static_assert(!XB || (BT == 2 && NWM == 1), "LDS batch tiles: one matrix, two register tiles");
  constexpr int NBT = XB ? BT + 2 : BT;   // batch column tiles of 8 in a pass
  constexpr int kPass = 8 * NBT;          // batch rows per pass
  constexpr int kXbU4 = XB ? kWavesM * 2 * KH * kWave : 0;
  // Dynamic LDS: [XB activation tiles: wave][tile][k-step][lane] u4, then
  // the partial sums [group < gpw][matrix][wave][batch < kPass][row], the
  // 8 K-slice partial sums of every output of the workgroup.
  extern __shared__ __align__(16) unsigned char dyn_lds[];
  u4* xbuf = reinterpret_cast<u4*>(dyn_lds);
  u4* const stage_area = reinterpret_cast<u4*>(dyn_lds + (size_t)kXbU4 * 16);
  float* part = reinterpret_cast<float*>(stage_area + a.part_off);
  auto slot = [&](int j, int m, int v, int n) -> float* {
    return part + ((((j * NWM + m) * kWavesM + v) * kPass + n) * kRowsPerGroup);
  };
  __shared__ float red[kWavesM][kPass];
  // gamma's LDS copy: static (a K / 8-chunk slice per wave), or with XB all
  // of gamma at the start of the partial-sum region, which nothing writes
  // before the XB prologue's barriers.
  __shared__ u4 s_gamma_own[gemv_has_norm(MODE) && !XB ? kThreadsM : 1];
  u4* const s_gamma = XB ? reinterpret_cast<u4*>(part) : s_gamma_own;

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int c16 = lane & 15;  // A row m / B column n
  const int g4 = lane >> 4;   // k-group
  const int r8 = c16 & 7;     // weight row in the group / batch row in the tile
  const int half = c16 >> 3;  // which half of the slice this lane covers
  const int b0 = blockIdx.y * kPass;
  const int nb = min(kPass, a.B - b0);
  // Wave v of workgroup w owns slice s = (v + w + w / 8) mod 8, columns
  // [s, s+1) * K / 8: workgroups on one XCD (w, w + 8, ...) and on
  // neighbouring XCDs start on different slices, so the 256 reads of x are
  // spread over its whole extent (x arrives 1.5x sooner at batch 16 than
  // with one order everywhere; e4m3 batches 4-8% faster).
  // The slice's columns are dealt out so that the two halves of a row are
  // adjacent in every load instruction:
  // fp16 k-step t covers 64 t + 32 h + 8 g4 (half h, lane group g4), e4m3
  // load p covers 128 p + 64 h + 16 g4 (k-steps 2p and 2p + 1).  One load
  // instruction then reads 8 full 128-byte lines, one per weight row.  The
  // activations follow the same order; the dot products do not depend on it.
  const int sbase =
      ((wave + (int)blockIdx.x + ((int)blockIdx.x >> 3)) & (kWavesM - 1)) * KH * 64;
  const int kcol = sbase + 32 * half + 8 * g4;  // fp16: this lane's column for k-step 0
  // Column of this lane's activation chunk for k-step t.
  auto xcol = [&](int t) {
    if constexpr (FP8) return sbase + 128 * (t >> 1) + 64 * half + 16 * g4 + 8 * (t & 1);
    return kcol + 64 * t;
  };

  // ---- the workgroup's groups: rows of group j are 8 (w + grid j) .. +7 --
  const int my_groups = min(a.gpw, (a.groups - (int)blockIdx.x + (int)gridDim.x - 1) /
                                       (int)gridDim.x);
  const unsigned char* wmat[2] = {static_cast<const unsigned char*>(a.w0),
                                  static_cast<const unsigned char*>(a.w1)};
  // A register set holds one group; j past the workgroup's last group
  // re-reads that one.  Every load_set is unconditional: after a load under
  // a branch the compiler merges the two paths' outstanding loads and waits
  // for all of them (vmcnt(0)) where one set would do.  With the first
  // group's load conditional, the normalisation's gamma store and barrier
  // waited for that group's weights (seen in the ISA); unconditional, they
  // stay in flight, which made F1 at 16 rows 11.05 -> 9.72 us, F1-QKV at 16
  // and 32 rows 13.13 -> 11.97 and 16.93 -> 15.92 us, e4m3 F1-QKV at 4-32
  // rows 4-6% faster (graph back-to-back, interleaved runs).
  auto load_set = [&](u4 (&dst)[NWM][KW], int j) {
    const int grp = blockIdx.x + gridDim.x * max(min(j, my_groups - 1), 0);
    const int row = min(grp * kRowsPerGroup + r8, a.N - 1);
#pragma unroll
    for (int m = 0; m < NWM; ++m)
#pragma unroll
      for (int t = 0; t < KW; ++t)
        dst[m][t] = FP8 ? ld_stream(wmat[m] + (size_t)row * a.K + xcol(2 * t))
                        : ld_stream(reinterpret_cast<const _Float16*>(wmat[m]) +
                                    (size_t)row * a.K + kcol + 64 * t);
  };

  // ---- activation slice -> registers (B operand) ------------------------
  // Two ways in.  Direct: each lane loads its own B operands; a load
  // instruction then covers 8 batch rows x 128 bytes, 8 KB apart.  Staged:
  // each wave loads its slice of every batch row contiguously -- lane l
  // takes the slice's 16-byte chunk l, two rows per instruction when the
  // slice is 32 chunks -- writes each chunk to the LDS slot of the lane and
  // k-step that use it and reads its operands back.  Measured on MI355X:
  // the direct pattern reads x (which all 256 workgroups read) 2.1x slower
  // than contiguous rows for the same 16 KB per wave (4.6 vs 2.2 us per
  // launch); staging makes one weight matrix at 9-32 rows 1.2-2.5 us
  // faster (F1-QKV B = 16 14.5 -> 13.0 us, B = 32 21.7 -> 19.0 us, F1
  // B = 16 12.6 -> 10.9 us, e4m3 F1-QKV B = 16 10.8 -> 9.7 us), while the
  // gate/up pair at B = 16 (1.1 us) loses: there the weights, not x, set the
  // pace, and the staging delays their first requests.  The norm modes
  // stage at every batch, since their weights stay in flight through the
  // normalisation: F1 at 3-8 rows (F1-QKV B = 3 10.70 -> 10.28 us, B = 8
  // 10.86 -> 10.32 us, F1 B = 8 8.55 -> 7.96 us, e4m3 F1-QKV B = 8 7.79 ->
  // 6.97 us, e4m3 F1 B = 8 6.40 -> 5.54 us) and RMSNorm -> gate/up at 3-16
  // rows (fp16 B = 8 37.7 -> 36.8 us, B = 16 39.8 -> 38.5 us, e4m3 B = 16
  // 23.2 -> 21.8 us).  The plain projection at one batch tile would wait for
  // a staging barrier and does not (+0.4-0.6 us at 3-4 rows, even at 8).
  // The staging area is the wave's XB tiles, or a per-wave part of the
  // dynamic LDS that the partial sums follow (part_off) or share; when they
  // share it, a barrier before the first partial-sum store (in consume)
  // keeps every wave's read-back ahead of them.
  constexpr bool kStage = gemv_has_norm(MODE) || (NWM == 1 && BT == 2);
  const u4 zero4 = {0, 0, 0, 0};
  u4 xr[BT][KH];
  u4 xb[XB ? 2 : 1][KH];  // XB: rows 16..31 (norm modes: for their x^2 sums)
  u4 gchunk = {0, 0, 0, 0};
  // gamma for the LDS copy the normalisation reads.  XB: thread t fetches
  // 16-byte chunk t of all of gamma (K / 8 <= 512 chunks), shared by the
  // waves; otherwise lane l of each wave fetches chunk l of the wave's own
  // K-slice (8 KH chunks) for a wave-private copy, so no wave waits for
  // another's before its first product.
  auto load_gamma = [&]() {
    if constexpr (gemv_has_norm(MODE)) {
      if constexpr (XB)
        gchunk = ld16(a.gamma + 8 * min((int)threadIdx.x, a.K / 8 - 1));
      else
        gchunk = ld16(a.gamma + sbase + 8 * min(lane, 8 * KH - 1));
    }
  };
  u4 wa[NWM][KW];
  if constexpr (kStage) {
    constexpr int kSliceChunks = 8 * KH;                // 16-byte chunks of a row's slice
    constexpr int kRowsPerLoad = kWave / kSliceChunks;  // 1 (K = 4096) or 2 (K = 2048)
    constexpr int kLoads = 8 * BT / kRowsPerLoad;       // per 8 BT rows
    const int lchunk = lane % kSliceChunks;
    const int lrow = lane / kSliceChunks;
    // Consumer of chunk c: fp16 c = 8 t + 4 h + g4, e4m3 column order
    // c = 16 (t >> 1) + 8 h + 2 g4 + (t & 1); lane 16 g4 + 8 h + r8.
    const int ct = FP8 ? 2 * (lchunk >> 4) + (lchunk & 1) : lchunk >> 3;
    const int ch = FP8 ? (lchunk >> 3) & 1 : (lchunk >> 2) & 1;
    const int cg = FP8 ? (lchunk >> 1) & 3 : lchunk & 3;
    u4* const stage =
        (XB ? xbuf : stage_area) + (size_t)wave * BT * KH * kWave;
    auto load_rows = [&](u4 (&dst)[kLoads], int r0) {
#pragma unroll
      for (int i = 0; i < kLoads; ++i) {
        const int rho = r0 + i * kRowsPerLoad + lrow;
        dst[i] = ld16(a.x + (size_t)(b0 + min(rho, nb - 1)) * a.K + sbase + 8 * lchunk);
      }
    };
    auto put_rows = [&](const u4 (&v)[kLoads], int r0) {
#pragma unroll
      for (int i = 0; i < kLoads; ++i) {
        const int rho = i * kRowsPerLoad + lrow;  // row within the 8 BT block
        stage[((rho >> 3) * KH + ct) * kWave + xslot(cg, ch, rho & 7, ct)] =
            r0 + rho < nb ? v[i] : zero4;
      }
    };
    auto get_rows = [&](u4 (&dst)[BT][KH]) {
#pragma unroll
      for (int bt = 0; bt < BT; ++bt)
#pragma unroll
        for (int t = 0; t < KH; ++t)
          dst[bt][t] = stage[(bt * KH + t) * kWave + xslot(g4, half, r8, t)];
    };
    u4 xl[kLoads];
    load_rows(xl, 0);
    u4 xlb[XB ? kLoads : 1];
    if constexpr (XB) load_rows(xlb, 16);
    load_gamma();
    __builtin_amdgcn_sched_barrier(0);
    put_rows(xl, 0);
    wave_lds_order();
    get_rows(xr);
    if constexpr (XB) {
      // Rows 16..31 go to their LDS tiles, the same per-wave area, after
      // rows 0..15 have been read back (a wave's LDS accesses complete in
      // order).
      wave_lds_order();
      put_rows(xlb, 16);
      wave_lds_order();
      if constexpr (gemv_has_norm(MODE)) get_rows(xb);
    }
    // The partial sums later share the staging area: a barrier before the
    // first partial-sum store (in consume) keeps every wave's read-back ahead
    // of them.
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (XB && gemv_has_norm(MODE)) {
      // Rows 16..31: their x^2 sums, from the copy read back from their LDS
      // tiles (where they are normalised in place after the cross-wave sum).
#pragma unroll
      for (int bt = 0; bt < 2; ++bt) {
        float sb = 0.0f;
#pragma unroll
        for (int t = 0; t < KH; ++t) sb = dot8(xb[bt][t], xb[bt][t], sb);
        sb += __shfl_xor(sb, 8);
        sb += __shfl_xor(sb, 16);
        sb += __shfl_xor(sb, 32);
        if (lane < 8) red[wave][8 * (BT + bt) + lane] = sb;
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    load_set(wa, 0);
  } else {
#pragma unroll
    for (int bt = 0; bt < BT; ++bt) {
      const int xrow = b0 + min(8 * bt + r8, nb - 1);
#pragma unroll
      for (int t = 0; t < KH; ++t)
        xr[bt][t] = ld16(a.x + (size_t)xrow * a.K + (FP8 ? xcol(t) : kcol + 64 * t));
    }
    load_gamma();
    __builtin_amdgcn_sched_barrier(0);
    auto mask_rows = [&]() {  // batch rows past the batch read as zeros
#pragma unroll
      for (int bt = 0; bt < BT; ++bt) {
        const bool valid = 8 * bt + r8 < nb;
#pragma unroll
        for (int t = 0; t < KH; ++t) xr[bt][t] = valid ? xr[bt][t] : zero4;
      }
    };
    if constexpr (BT == 1) {
      // With one batch tile the wave waits for its x slice before requesting
      // weights (batch 3-8 ran 0.4-1.3 us faster).
      mask_rows();
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): x and gamma are here
      __builtin_amdgcn_sched_barrier(0);
      load_set(wa, 0);
    } else {
      // With two, set A goes out with x: the masking, which needs x, comes
      // after the request (before it, the compiler waited for all of x
      // first; gate/up pair at 16 rows 38.2 -> 37.5 us, e4m3 22.1 -> 21.7).
      load_set(wa, 0);
      __builtin_amdgcn_sched_barrier(0);
      mask_rows();
    }
  }
  __builtin_amdgcn_sched_barrier(0);


  if constexpr (gemv_has_norm(MODE)) {
    // x^2 over this slice per batch row: in-lane, then over the two halves
    // (lanes 8 apart) and the 4 k-groups (lanes 16 apart).
    float ss[BT];
#pragma unroll
    for (int bt = 0; bt < BT; ++bt) {
      ss[bt] = 0.0f;
#pragma unroll
      for (int t = 0; t < KH; ++t) ss[bt] = dot8(xr[bt][t], xr[bt][t], ss[bt]);
      ss[bt] += __shfl_xor(ss[bt], 8);
      ss[bt] += __shfl_xor(ss[bt], 16);
      ss[bt] += __shfl_xor(ss[bt], 32);
      if (lane < 8) red[wave][8 * bt + lane] = ss[bt];
    }
    if constexpr (XB) {
      if ((int)threadIdx.x < a.K / 8) s_gamma[threadIdx.x] = gchunk;
      __syncthreads();
    } else {
      // The wave's slice of gamma (chunks sbase / 8 ..), read back by the
      // wave's own lanes.
      if (lane < 8 * KH) s_gamma[wave * kWave + lane] = gchunk;
      wave_lds_order();
    }
    if constexpr (XB) {
      // rows 16..31: normalised in place in their LDS tiles
#pragma unroll
      for (int bt = 0; bt < 2; ++bt) {
        float tot = 0.0f;
#pragma unroll
        for (int v = 0; v < kWavesM; ++v) tot += red[v][8 * (BT + bt) + r8];
        const float inv = 1.0f / sqrtf(tot / (float)a.K + a.eps);
#pragma unroll
        for (int t = 0; t < KH; ++t) {
          const u4 gv = s_gamma[(FP8 ? xcol(t) : kcol + 64 * t) / 8];
          u4& xv = xbuf[((wave * 2 + bt) * KH + t) * kWave + xslot(g4, half, r8, t)];
          xv = norm_mul(xv, gv, inv);
        }
      }
    }
#pragma unroll
    for (int bt = 0; bt < BT; ++bt) {
      if constexpr (XB) {
        float tot = 0.0f;
#pragma unroll
        for (int v = 0; v < kWavesM; ++v) tot += red[v][8 * bt + r8];
        const float inv = 1.0f / sqrtf(tot / (float)a.K + a.eps);
#pragma unroll
        for (int t = 0; t < KH; ++t)
          xr[bt][t] = norm_mul(xr[bt][t], s_gamma[(FP8 ? xcol(t) : kcol + 64 * t) / 8], inv);
      } else {
        // fp16(x * gamma), one v_pk_mul_f16 per pair; inv_rms is applied to
        // the reduced sums in the epilogue.  Against normalising here as the
        // stage rounds (fp16(fp16(x * inv_rms) * gamma), norm_mul) this is
        // 0.3-0.6 us faster at 4-32 rows (F1-QKV B = 16 11.67 -> 11.26 us,
        // B = 32 15.85 -> 15.25 us, F1 B = 32 12.1 -> 11.5 us, e4m3 F1-QKV
        // B = 32 11.14 -> 10.6 us); the outputs move 4.4e-4 (rel-L2) from
        // the stage and stay 4.5e-4 from the fp64 oracle.
#pragma unroll
        for (int t = 0; t < KH; ++t) {
          const u4 gv = s_gamma[wave * kWave + ((FP8 ? xcol(t) : kcol + 64 * t) - sbase) / 8];
          u4 o;
#pragma unroll
          for (int q = 0; q < 4; ++q)
            o[q] = __builtin_bit_cast(unsigned, as_h2(xr[bt][t][q]) * as_h2(gv[q]));
          xr[bt][t] = o;
        }
      }
    }
    // gamma shares the partial-sum region under XB: every wave must be done
    // with it before the first partial sum is stored.
    if constexpr (XB) __syncthreads();
  }

  // ---- stream the groups ------------------------------------------------
  auto consume = [&](const u4 (&src)[NWM][KW], int j) {
    if (j >= my_groups) return;
    {
#pragma unroll
      for (int m = 0; m < NWM; ++m) {
        // e4m3: the A operands of the KH k-steps, widened to fp16 once per
        // group; fp16: the loaded registers themselves.
        u4 av[FP8 ? KH : 1];
        if constexpr (FP8) {
#pragma unroll
          for (int t = 0; t < KW; ++t) e4m3x16_to_h(src[m][t], av[2 * t], av[2 * t + 1]);
        }
#pragma unroll
        for (int bt = 0; bt < BT; ++bt) {
          f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int t = 0; t < KH; ++t) {
            const u4 at = FP8 ? av[FP8 ? t : 0] : src[m][FP8 ? 0 : t];
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, at),
                                                         __builtin_bit_cast(h8, xr[bt][t]), acc,
                                                         0, 0, 0);
          }
          // D[4 g4 + i][c16]: rows 0..7 x columns 0..7 (half 0) live in lanes
          // (g4 < 2, c16 < 8); their half-1 partners sit 40 lanes higher.
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[i] += __shfl(acc[i], lane + 40);
          // The first partial-sum store of the workgroup: a staging area it
          // shares must have been read back by every wave (j is uniform, and
          // every workgroup consumes group 0 first, exactly once).
          if constexpr (kStage && !XB)
            if (a.part_off == 0 && m == 0 && bt == 0 && j == 0) __syncthreads();
          if (g4 < 2 && c16 < 8)
            *reinterpret_cast<f4*>(slot(j, m, wave, 8 * bt + c16) + 4 * g4) = acc;
        }
        if constexpr (XB) {
          // rows 16..31: the same A operands against the LDS tiles
#pragma unroll
          for (int bt = 0; bt < 2; ++bt) {
            f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int t = 0; t < KH; ++t) {
              const u4 at = FP8 ? av[FP8 ? t : 0] : src[m][FP8 ? 0 : t];
              const u4 bx = xbuf[((wave * 2 + bt) * KH + t) * kWave + xslot(g4, half, r8, t)];
              acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, at),
                                                           __builtin_bit_cast(h8, bx), acc, 0, 0,
                                                           0);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] += __shfl(acc[i], lane + 40);
            if (g4 < 2 && c16 < 8)
              *reinterpret_cast<f4*>(slot(j, m, wave, 8 * (BT + bt) + c16) + 4 * g4) = acc;
          }
        }
      }
    }
  };

  {
    // Two register sets; the steady loop loads and consumes set B inside
    // one iteration, which keeps the compiler from draining all loads at
    // the loop header.
    u4 wb[NWM][KW];
    int j = 0;
    for (; j + 3 <= my_groups; j += 2) {
      load_set(wb, j + 1);
      consume(wa, j);
      load_set(wa, j + 2);
      consume(wb, j + 1);
    }
    // One or two groups remain; set A holds the first.  Each case is
    // straight-line code (see load_set).
    if (j + 1 < my_groups) {
      load_set(wb, j + 1);
      consume(wa, j);
      consume(wb, j + 1);
    } else {
      consume(wa, j);
    }
  }

  __syncthreads();

  // ---- reduce the 8 K-slices, epilogue, fp16 store ----------------------
  const int nout = my_groups * kPass * kRowsPerGroup;
  for (int idx = threadIdx.x; idx < nout; idx += kThreadsM) {
    const int jj = idx / (kPass * kRowsPerGroup);
    const int n = (idx / kRowsPerGroup) % kPass;
    const int r = idx % kRowsPerGroup;
    const int row = (blockIdx.x + gridDim.x * jj) * kRowsPerGroup + r;
    if (n >= nb || row >= a.N) continue;
    float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
    for (int v = 0; v < kWavesM; ++v) {
      s0 += slot(jj, 0, v, n)[r];
      if constexpr (NWM == 2) s1 += slot(jj, NWM - 1, v, n)[r];
    }
    if constexpr (gemv_has_norm(MODE) && !XB) {
      float tot = 0.0f;
#pragma unroll
      for (int v = 0; v < kWavesM; ++v) tot += red[v][n];
      const float inv = 1.0f / sqrtf(tot / (float)a.K + a.eps);
      s0 *= inv;
      if constexpr (NWM == 2) s1 *= inv;
    }
    if constexpr (FP8) {
      s0 *= a.s0[row];
      if constexpr (NWM == 2) s1 *= a.s1[row];
    }
    float out;
    if constexpr (NWM == 2) {
      const float gq = (float)to_h(s0);
      const float uq = (float)to_h(s1);
      out = (float)to_h(gemv_silu(gq)) * uq;
    } else {
      out = s0;
    }
    a.y[(size_t)(b0 + n) * a.N + row] = to_h(out);
  }
}

// ---- long rows: K a multiple of 2048 above 4096 ---------------------------
// At K = 14336 (the down projection) a 16-row activation slice would take
// 224 VGPRs, so here both operands stream.  Wave v of workgroup w owns the
// same XCD-staggered K / 8 slice as above and walks it in chunks of KC
// k-steps (64 KC columns, dealt out over the halves and lane groups as
// above).  Per chunk it loads the pass's BT batch tiles of x and the chunk
// of each of the workgroup's GPW groups, and the MFMA sums accumulate in
// registers across chunks; two register sets alternate (load chunk c + 1,
// consume chunk c).  Batch rows past the batch read x's last row and rows
// past N read W's last row: batch column n of an MFMA sees only x row n and
// output row m only weight row m, and those columns and rows are never
// stored.  Plain GEMV only: a norm would need all of x before the first
// product.
// XS: x is loaded contiguously -- lane l takes 16-byte piece l % 8 KC of
// the chunk of batch row l / 8 KC, 64 / (8 KC) rows per instruction -- and
// staged through the wave's LDS tile (the xslot layout) into B operands;
// otherwise each lane loads its own B operands (8 batch rows x 128 bytes
// per instruction).
template <int KC, int BT, int GPW, bool FP8, bool XS>
__global__ __launch_bounds__(kThreadsM) void gemv_mfma_long_kernel(MfmaArgs a) {
  constexpr int KWC = FP8 ? KC / 2 : KC;  // 16-byte weight loads per row and chunk
  constexpr int kPass = 8 * BT;
  constexpr int kXL = BT * KC;            // x loads per chunk, either way
  static_assert(!FP8 || KC % 2 == 0, "an e4m3 load spans two k-steps");
  // [group][wave][batch][row quad]: rows 4 i .. 4 i + 3 of a group
  __shared__ f4 part[GPW][kWavesM][kPass][2];
  // XS: each wave's x tile, [batch tile][k-step][slot] (BT KC KB per wave)
  extern __shared__ __align__(16) unsigned char dyn_lds[];

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int c16 = lane & 15;
  const int g4 = lane >> 4;
  const int r8 = c16 & 7;
  const int half = c16 >> 3;
  const int bx = blockIdx.x;
  const int b0 = blockIdx.y * kPass;
  const int nb = min(kPass, a.B - b0);
  const int slice = a.K / kWavesM;
  const int nch = slice / (64 * KC);
  const int sbase = ((wave + bx + (bx >> 3)) & (kWavesM - 1)) * slice;
  // This lane's first column: fp16 k-step t of chunk c covers
  // 64 (KC c + t) + 32 h + 8 g4; e4m3 load p covers 64 KC c + 128 p + 64 h
  // + 16 g4 (k-steps 2p and 2p + 1, x 8 columns apart).
  const int lcol = sbase + (FP8 ? 64 * half + 16 * g4 : 32 * half + 8 * g4);
  const int my_groups = min(GPW, (a.groups - bx + (int)gridDim.x - 1) / (int)gridDim.x);

  // x.  Direct: a pointer per batch tile.  Staged: load i covers rows
  // rho = i R + l / (8 KC) (R = 64 / (8 KC) rows per instruction), at a
  // 32-bit byte offset from the pass's first row (so the loads take the
  // scalar-base form); rows past the batch read its last row.  Its piece goes
  // to LDS slot ((rho >> 3) KC + ct) 64 + xslot(cg, ch, rho & 7, ct), where
  // rho & 7 = (i R & 7) | l / (8 KC) carries nothing into the bits xslot's
  // swizzle touches: the slot is put_base[(i R & 7) / R] plus a constant.
  constexpr int kPieces = 8 * KC;
  constexpr int kRowsPerLd = kWave / kPieces;
  constexpr int kPutVariants = 8 / kRowsPerLd;
  const _Float16* xp[XS ? 1 : BT];
  unsigned xoff_b[XS ? kXL : 1];
  int put_base[XS ? kPutVariants : 1];
  int get_base[2];
  if constexpr (XS) {
    const int piece = lane % kPieces;
    const int lrow = lane / kPieces;
    // consumer of piece cc: fp16 cc = 8 t + 4 h + g4, e4m3 cc = 16 (t >> 1)
    // + 8 h + 2 g4 + (t & 1)
    const int ct = FP8 ? 2 * (piece >> 4) + (piece & 1) : piece >> 3;
    const int ch = FP8 ? (piece >> 3) & 1 : (piece >> 2) & 1;
    const int cg = FP8 ? (piece >> 1) & 3 : piece & 3;
    xp[0] = a.x + (size_t)b0 * a.K + sbase;
#pragma unroll
    for (int i = 0; i < kXL; ++i)
      xoff_b[i] = 2u * ((unsigned)min(i * kRowsPerLd + lrow, nb - 1) * (unsigned)a.K +
                        8u * (unsigned)piece);
    const int sw = cg | ((ct & 1) << 2);
#pragma unroll
    for (int v = 0; v < kPutVariants; ++v)
      put_base[v] = ct * kWave + 16 * cg + (((8 * ch) | lrow) ^ sw ^ (v * kRowsPerLd));
#pragma unroll
    for (int p = 0; p < 2; ++p) get_base[p] = xslot(g4, half, r8, p);
  } else {
#pragma unroll
    for (int bt = 0; bt < BT; ++bt)
      xp[bt] = a.x + (size_t)(b0 + min(8 * bt + r8, nb - 1)) * a.K + lcol;
  }
  u4* const tile = reinterpret_cast<u4*>(dyn_lds) + (size_t)wave * kXL * kWave;
  const unsigned char* wp[GPW];
  const int esz = FP8 ? 1 : 2;
#pragma unroll
  for (int q = 0; q < GPW; ++q) {
    const int grp = bx + (int)gridDim.x * min(q, my_groups - 1);
    const int row = min(grp * kRowsPerGroup + r8, a.N - 1);
    wp[q] = static_cast<const unsigned char*>(a.w0) + ((size_t)row * a.K + lcol) * esz;
  }
  auto xoff = [](int t) { return FP8 ? 128 * (t >> 1) + 8 * (t & 1) : 64 * t; };

  auto load = [&](u4 (&xs)[kXL], u4 (&ws)[GPW][KWC], int c) {
    const int c0 = 64 * KC * c;
#pragma unroll
    for (int q = 0; q < GPW; ++q)
#pragma unroll
      for (int p = 0; p < KWC; ++p)
        ws[q][p] = ld_stream(wp[q] + (size_t)(c0 + 64 * p * (FP8 ? 2 : 1)) * esz);
    if constexpr (XS) {
      const unsigned char* xc = reinterpret_cast<const unsigned char*>(xp[0] + c0);
#pragma unroll
      for (int i = 0; i < kXL; ++i) xs[i] = ld16(xc + xoff_b[i]);
    } else {
#pragma unroll
      for (int i = 0; i < kXL; ++i) xs[i] = ld16(xp[i / KC] + c0 + xoff(i % KC));
    }
  };
  f4 acc[GPW][BT];
#pragma unroll
  for (int q = 0; q < GPW; ++q)
#pragma unroll
    for (int bt = 0; bt < BT; ++bt) acc[q][bt] = f4{0.0f, 0.0f, 0.0f, 0.0f};
  auto consume = [&](const u4 (&xl)[kXL], const u4 (&ws)[GPW][KWC]) {
    u4 xs[kXL];
    if constexpr (XS) {
      // A wave's LDS accesses complete in order: the previous chunk's reads
      // are done before these writes land.
      wave_lds_order();
#pragma unroll
      for (int i = 0; i < kXL; ++i)
        tile[((i * kRowsPerLd) >> 3) * KC * kWave + put_base[((i * kRowsPerLd) & 7) / kRowsPerLd]] =
            xl[i];
      wave_lds_order();
#pragma unroll
      for (int bt = 0; bt < BT; ++bt)
#pragma unroll
        for (int t = 0; t < KC; ++t)
          xs[bt * KC + t] = tile[(bt * KC + t) * kWave + get_base[t & 1]];
    } else {
#pragma unroll
      for (int i = 0; i < kXL; ++i) xs[i] = xl[i];
    }
    u4 av[GPW][KC];
#pragma unroll
    for (int q = 0; q < GPW; ++q) {
      if constexpr (FP8) {
#pragma unroll
        for (int p = 0; p < KWC; ++p) e4m3x16_to_h(ws[q][p], av[q][2 * p], av[q][2 * p + 1]);
      } else {
#pragma unroll
        for (int t = 0; t < KC; ++t) av[q][t] = ws[q][t];
      }
    }
#pragma unroll
    for (int t = 0; t < KC; ++t)
#pragma unroll
      for (int q = 0; q < GPW; ++q)
#pragma unroll
        for (int bt = 0; bt < BT; ++bt)
          acc[q][bt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
              __builtin_bit_cast(h8, av[q][t]), __builtin_bit_cast(h8, xs[bt * KC + t]),
              acc[q][bt], 0, 0, 0);
  };

  u4 xa[kXL], wa[GPW][KWC], xb[kXL], wb[GPW][KWC];
  // Left to itself the compiler issued set B's loads only after consume(A)
  // had waited for all of set A (vmcnt(0) at the loop header, read in the
  // ISA), so one chunk was in flight at a time.  A scheduling barrier after
  // each load keeps the next chunk in flight, and the tail is straight-line
  // code per case (a load under a branch merges two paths into a vmcnt(0)).
  // Measured with fp16 weights ([4096, 14336], µs): B = 3 19.6 -> 19.2,
  // B = 32 32.0 -> 30.9, B = 48 53.5 -> 46.8 (its register spill shrank
  // from 44 to 12 bytes), B = 64 48.3 -> 45.6.  The e4m3 kernels keep the
  // compiler's order: the barrier cost 0.4 us at B = 16, and the split tail
  // added a spill to 32 rows x 4 groups (B = 48-64 +2 us).  32 rows x 4
  // groups take no barrier (it raised the spill).
  constexpr bool kPrefetchFirst = !FP8 && BT * GPW < 16;
  load(xa, wa, 0);
  int c = 0;
  for (; c + 3 <= nch; c += 2) {
    load(xb, wb, c + 1);
    if constexpr (kPrefetchFirst) __builtin_amdgcn_sched_barrier(0);
    consume(xa, wa);
    load(xa, wa, c + 2);
    if constexpr (kPrefetchFirst) __builtin_amdgcn_sched_barrier(0);
    consume(xb, wb);
  }
  // One or two chunks remain; set A holds the first.
  if constexpr (FP8) {
    if (c + 1 < nch) load(xb, wb, c + 1);
    consume(xa, wa);
    if (c + 1 < nch) consume(xb, wb);
  } else if (c + 1 < nch) {
    load(xb, wb, c + 1);
    if constexpr (kPrefetchFirst) __builtin_amdgcn_sched_barrier(0);
    consume(xa, wa);
    consume(xb, wb);
  } else {
    consume(xa, wa);
  }

  // D[4 g4 + i][c16]: rows 0..7 x batch 0..7 (half 0) in lanes (g4 < 2,
  // c16 < 8), their half-1 partners 40 lanes higher.
#pragma unroll
  for (int q = 0; q < GPW; ++q)
#pragma unroll
    for (int bt = 0; bt < BT; ++bt) {
      f4 v = acc[q][bt];
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] += __shfl(v[i], lane + 40);
      if (g4 < 2 && c16 < 8) part[q][wave][8 * bt + c16][g4] = v;
    }
  __syncthreads();

  // ---- reduce the 8 K-slices, row scales, fp16 store ---------------------
  const float* pf = reinterpret_cast<const float*>(&part[0][0][0][0]);
  for (int idx = threadIdx.x; idx < my_groups * kPass * kRowsPerGroup; idx += kThreadsM) {
    const int q = idx / (kPass * kRowsPerGroup);
    const int n = (idx / kRowsPerGroup) % kPass;
    const int r = idx % kRowsPerGroup;
    const int row = (bx + (int)gridDim.x * q) * kRowsPerGroup + r;
    if (n >= nb || row >= a.N) continue;
    float s = 0.0f;
#pragma unroll
    for (int v = 0; v < kWavesM; ++v) s += pf[((q * kWavesM + v) * kPass + n) * kRowsPerGroup + r];
    if constexpr (FP8) s *= a.s0[row];
    a.y[(size_t)(b0 + n) * a.N + row] = to_h(s);
  }
}

// ---- streamed activations on full 16-row tiles ----------------------------
// The kernel above spends three quarters of every accumulator: an 8-row
// group over two half slices fills one v_mfma_f32_16x16x32_f16, but only
// its two diagonal 8 x 8 blocks are dot products.  For the gate/up pair at
// 32 rows that would be 7 groups x 2 matrices x 4 tiles of accumulators
// (224 registers) on a CU's 56 rows; a version built that way had the
// register allocator move accumulators through a shared temporary between
// MFMAs and ran 1.6x slower (e4m3).  Here an MFMA
// takes 16 weight rows (two of the workgroup's 8-row groups) against 16
// batch rows over the same 32 columns, and every element of D is an output:
// A row m = row m & 7 of group 2j + (m >> 3), k-group g4 = columns
// 32 s + 8 g4 of k-step s (fp16) or, for e4m3, columns 64 (s >> 1) +
// 16 g4 + 8 (s & 1); B column n = batch row 16 bt + n over the same columns.
// Loading those A operands directly would read 16 rows x 64 bytes (half
// lines) per instruction.  Instead each 8-row group is loaded as above --
// lane (g4, h, r8) takes row r8, half h of a 128-byte line, 8 whole lines
// per instruction -- and the two groups of a tile are merged into its A
// operands with one DPP row_ror:8 move per register: lanes 8..15 of each
// 16-lane row of the first group's register take lanes 0..7 of the
// second's (the tile's half-0 operand), and lanes 0..7 of the second's take
// lanes 8..15 of the first's (its half-1 operand).
// Waves own K / WV slices as above and walk them in chunks of KC k-steps;
// accumulators stay in registers; the K-slice partial sums meet in LDS with
// the same layout and epilogue as above.  A workgroup owns up to 2 T
// groups; a last tile with one group duplicates it in rows 8..15, which are
// not stored.  Launched with N a multiple of 8 and 2 N K bytes below 4 GiB
// (32-bit lane offsets; every row of a live group below N).
// NORM (RMSNorm -> gate/up, K <= 4096): before the stream each wave sums x^2
// over its slice for every batch row of the pass; each streamed x chunk is
// then normalised as fp16(fp16(x * inv_rms) * gamma).
__device__ __forceinline__ u4 tile_half0(const u4& g0, const u4& g1) {
  u4 t;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    t[i] = (unsigned)__builtin_amdgcn_update_dpp((int)g0[i], (int)g1[i], kRowRor8, 0xf, 0xc,
                                                 false);
  return t;
}
__device__ __forceinline__ u4 tile_half1(const u4& g0, const u4& g1) {
  u4 t;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    t[i] = (unsigned)__builtin_amdgcn_update_dpp((int)g1[i], (int)g0[i], kRowRor8, 0xf, 0x3,
                                                 false);
  return t;
}

template <int NWM, int WV, int KC, int BT16, int T, bool FP8, bool NORM>
__global__ __launch_bounds__(WV * kWave) void gemv_mfma_tile16_kernel(MfmaArgs a) {
  constexpr int kThreads = WV * kWave;
  constexpr int kStepsPerLoad = FP8 ? 2 : 1;  // k-steps in a 16-byte A operand
  constexpr int LS = 2 * kStepsPerLoad;       // k-steps per line load (both halves)
  static_assert(KC % LS == 0, "a chunk holds whole lines");
  constexpr int KWC = KC / LS;                // line loads per group and chunk
  constexpr int NG = 2 * T;                   // 8-row groups
  constexpr int kPass = 16 * BT16;
  constexpr int kXL = BT16 * KC;
  static_assert((WV & (WV - 1)) == 0, "waves per workgroup: a power of 2");
  extern __shared__ __align__(16) unsigned char dyn_lds[];
  float* const part = reinterpret_cast<float*>(dyn_lds);  // [2T][NWM][WV][kPass][8]

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int c16 = lane & 15;
  const int g4 = lane >> 4;
  const int bx = blockIdx.x;
  const int grid = gridDim.x;
  const int b0 = blockIdx.y * kPass;
  const int nb = min(kPass, a.B - b0);
  const int slice = a.K / WV;
  const int nch = slice / (32 * KC);  // chunks of KC k-steps of 32 columns
  const int sbase = ((wave + bx + (bx >> 3)) & (WV - 1)) * slice;
  const int xcol0 = sbase + (FP8 ? 16 * g4 : 8 * g4);
  const int my_groups = min(a.gpw, (a.groups - bx + grid - 1) / grid);
  const int esz = FP8 ? 1 : 2;
  const unsigned char* wmat[2] = {static_cast<const unsigned char*>(a.w0),
                                  static_cast<const unsigned char*>(a.w1)};

  // Weight lane offset: row r8 of the group, half h of the line; groups are
  // gstride apart (group q of the workgroup is bx + grid q).
  const int r8 = c16 & 7;
  const int half = c16 >> 3;
  const int wcol0 = sbase + (FP8 ? 64 * half + 16 * g4 : 32 * half + 8 * g4);
  const unsigned woff = ((unsigned)(bx * kRowsPerGroup + r8) * (unsigned)a.K +
                         (unsigned)wcol0) * esz;
  const size_t gstride = (size_t)grid * kRowsPerGroup * a.K * esz;
  const _Float16* xp[BT16];
#pragma unroll
  for (int bt = 0; bt < BT16; ++bt)
    xp[bt] = a.x + (size_t)(b0 + min(16 * bt + c16, nb - 1)) * a.K + xcol0;
  // Column offset of line load p within a chunk, and of k-step t's
  // activations.
  auto wcol = [](int p) { return (FP8 ? 128 : 64) * p; };
  auto xcol = [](int t) { return FP8 ? 64 * (t >> 1) + 8 * (t & 1) : 32 * t; };

  // NORM: gamma at the activations' columns, loaded with each chunk.
  constexpr int kGL = NORM ? KC : 1;
  auto load = [&](u4 (&xs)[kXL], u4 (&gs)[kGL], u4 (&ws)[NG][NWM][KWC], int c) {
    const int c0 = 32 * KC * c;
#pragma unroll
    for (int j = 0; j < NG; ++j) {
      // Groups past the workgroup's last re-read that one (rows not stored).
      const size_t goff = gstride * min(j, my_groups - 1);
#pragma unroll
      for (int m = 0; m < NWM; ++m)
#pragma unroll
        for (int p = 0; p < KWC; ++p)
          ws[j][m][p] = ld_stream(wmat[m] + goff + (size_t)(c0 + wcol(p)) * esz + woff);
    }
#pragma unroll
    for (int i = 0; i < kXL; ++i) xs[i] = ld16(xp[i / KC] + c0 + xcol(i % KC));
    if constexpr (NORM) {
#pragma unroll
      for (int t = 0; t < KC; ++t) gs[t] = ld16(a.gamma + xcol0 + c0 + xcol(t));
    }
  };
  f4 acc[T][NWM][BT16];
#pragma unroll
  for (int j = 0; j < T; ++j)
#pragma unroll
    for (int m = 0; m < NWM; ++m)
#pragma unroll
      for (int bt = 0; bt < BT16; ++bt) acc[j][m][bt] = f4{0.0f, 0.0f, 0.0f, 0.0f};
  // A operand u (16 bytes, kStepsPerLoad k-steps from k-step t0) of tile j.
  auto mma = [&](const u4& u, int j, int m, int t0, const u4 (&xs)[kXL]) {
    u4 av[kStepsPerLoad];
    if constexpr (FP8) e4m3x16_to_h(u, av[0], av[1]);
    else av[0] = u;
#pragma unroll
    for (int s = 0; s < kStepsPerLoad; ++s)
#pragma unroll
      for (int bt = 0; bt < BT16; ++bt)
        acc[j][m][bt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
            __builtin_bit_cast(h8, av[s]), __builtin_bit_cast(h8, xs[bt * KC + t0 + s]),
            acc[j][m][bt], 0, 0, 0);
  };
  float inv[BT16];  // NORM: 1 / rms of this lane's batch rows
  auto consume = [&](const u4 (&xl)[kXL], const u4 (&gs)[kGL], const u4 (&ws)[NG][NWM][KWC]) {
    // NORM: fp16(fp16(x * inv_rms) * gamma), the torch stage's rounding
    // points (see norm_mul).
    u4 xs[kXL];
#pragma unroll
    for (int i = 0; i < kXL; ++i) xs[i] = NORM ? norm_mul(xl[i], gs[i % KC], inv[i / KC]) : xl[i];
#pragma unroll
    for (int p = 0; p < KWC; ++p)
#pragma unroll
      for (int j = 0; j < T; ++j)
#pragma unroll
        for (int m = 0; m < NWM; ++m) {
          const u4& g0 = ws[2 * j][m][p];
          const u4& g1 = ws[2 * j + 1][m][p];
          mma(tile_half0(g0, g1), j, m, LS * p, xs);
          mma(tile_half1(g0, g1), j, m, LS * p + kStepsPerLoad, xs);
        }
  };

  u4 xa[kXL], ga[kGL], wa[NG][NWM][KWC], xb[kXL], gb[kGL], wb[NG][NWM][KWC];
  load(xa, ga, wa, 0);  // in flight during the statistic below
  if constexpr (NORM) {
    // x^2 over this wave's K slice for every batch row of the pass, 8 rows
    // at a time (lane l takes 16-byte pieces l and l + 64 of a row's slice,
    // which covers K <= 4096), then over the waves in LDS.
    __shared__ float red[WV][kPass];
    const int pieces = slice / 8;
    const u4 zero4 = {0, 0, 0, 0};
    for (int r0 = 0; r0 < nb; r0 += 8) {
      u4 v[8][2];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const _Float16* xr = a.x + (size_t)(b0 + min(r0 + i, nb - 1)) * a.K + sbase;
#pragma unroll
        for (int h = 0; h < 2; ++h)
          v[i][h] = lane + 64 * h < pieces ? ld16(xr + 8 * (lane + 64 * h)) : zero4;
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float ss = wave_sum(dot8(v[i][1], v[i][1], dot8(v[i][0], v[i][0], 0.0f)));
        if (lane == 0 && r0 + i < nb) red[wave][r0 + i] = ss;
      }
    }
    __syncthreads();
#pragma unroll
    for (int bt = 0; bt < BT16; ++bt) {
      const int r = min(16 * bt + c16, nb - 1);
      float tot = 0.0f;
#pragma unroll
      for (int w = 0; w < WV; ++w) tot += red[w][r];
      inv[bt] = 1.0f / sqrtf(tot / (float)a.K + a.eps);
    }
  }
  int c = 0;
  // A scheduling barrier after each load keeps the next chunk in flight
  // while the current one is consumed (otherwise the compiler sinks the
  // loads below the current chunk's waits), and the tail is straight-line
  // code per case.  Measured at [14336, 4096], 17-32 rows (µs): fp16 pair
  // 39.7 -> 39.2 (B = 17), 42.1 -> 41.8 (B = 32); RMSNorm -> gate/up 46.4
  // -> 44.8, 50.3 -> 48.9; e4m3 pair 27.9 -> 27.4 (B = 32), RMSNorm ->
  // gate/up 32.6 -> 31.3, 36.3 -> 34.8.
  for (; c + 3 <= nch; c += 2) {
    load(xb, gb, wb, c + 1);
    __builtin_amdgcn_sched_barrier(0);
    consume(xa, ga, wa);
    load(xa, ga, wa, c + 2);
    __builtin_amdgcn_sched_barrier(0);
    consume(xb, gb, wb);
  }
  if (c + 1 < nch) {
    load(xb, gb, wb, c + 1);
    __builtin_amdgcn_sched_barrier(0);
    consume(xa, ga, wa);
    consume(xb, gb, wb);
  } else {
    consume(xa, ga, wa);
  }

  // D[4 g4 + i][c16] = tile row 4 g4 + i (group 2j + (g4 >> 1), row
  // 4 (g4 & 1) + i) against batch row 16 bt + c16.
  auto slot = [&](int q, int m, int v, int n) {
    return part + ((((q * NWM + m) * WV + v) * kPass + n) * kRowsPerGroup);
  };
#pragma unroll
  for (int j = 0; j < T; ++j) {
    const int q = 2 * j + (g4 >> 1);
    if (q < my_groups) {
#pragma unroll
      for (int m = 0; m < NWM; ++m)
#pragma unroll
        for (int bt = 0; bt < BT16; ++bt)
          *reinterpret_cast<f4*>(slot(q, m, wave, 16 * bt + c16) + 4 * (g4 & 1)) =
              acc[j][m][bt];
    }
  }
  __syncthreads();

  for (int idx = threadIdx.x; idx < my_groups * kPass * kRowsPerGroup; idx += kThreads) {
    const int q = idx / (kPass * kRowsPerGroup);
    const int n = (idx / kRowsPerGroup) % kPass;
    const int r = idx % kRowsPerGroup;
    const int row = (bx + grid * q) * kRowsPerGroup + r;
    if (n >= nb) continue;
    float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
    for (int v = 0; v < WV; ++v) {
      s0 += slot(q, 0, v, n)[r];
      if constexpr (NWM == 2) s1 += slot(q, NWM - 1, v, n)[r];
    }
    if constexpr (FP8) {
      s0 *= a.s0[row];
      if constexpr (NWM == 2) s1 *= a.s1[row];
    }
    float out = s0;
    if constexpr (NWM == 2) {
      const float gq = (float)to_h(s0);
      const float uq = (float)to_h(s1);
      out = (float)to_h(gemv_silu(gq)) * uq;
    }
    a.y[(size_t)(b0 + n) * a.N + row] = to_h(out);
  }
}

using MfmaFn = void (*)(MfmaArgs);

// One group per register set, two sets alternating (load set B, consume A,
// reload A, consume B), so each wave has one or two groups of weights in
// flight.  Measured on MI355X (graph back-to-back) against requesting all
// of a workgroup's groups (up to 4) before the prologue, or sets of 2: F1-QKV
// B = 4 10.95 -> 10.4 us, B = 8 11.45 -> 10.8-11.1 us, e4m3 B = 16 11.4 ->
// 10.9 us, fp16 B = 16 14.7-14.8 -> 14.3-14.6 us.  The more weight requests
// all CUs have outstanding while x (which every workgroup reads) is still
// on its way, the later x arrives.
template <int MODE, int KH, bool FP8>
MfmaFn pick_bt(int bt) {
  return bt == 1 ? gemv_mfma_kernel<MODE, KH, 1, FP8, false>
                 : gemv_mfma_kernel<MODE, KH, 2, FP8, false>;
}

template <int MODE, bool FP8>
MfmaFn pick_kh(int kh, int bt) {
  return kh == 4 ? pick_bt<MODE, 4, FP8>(bt) : pick_bt<MODE, 8, FP8>(bt);
}

// 32-row passes of one weight matrix (XB).
template <int MODE, bool FP8>
MfmaFn pick_xb(int kh) {
  return kh == 4 ? gemv_mfma_kernel<MODE, 4, 2, FP8, true>
                 : gemv_mfma_kernel<MODE, 8, 2, FP8, true>;
}

template <bool FP8>
MfmaFn pick_mode(GemvMode mode, int kh, int bt, bool xb) {
  if (xb) return mode == kGemvRmsNorm ? pick_xb<kGemvRmsNorm, FP8>(kh)
                                      : pick_xb<kGemvPlain, FP8>(kh);
  switch (mode) {
    case kGemvRmsNorm: return pick_kh<kGemvRmsNorm, FP8>(kh, bt);
    case kGemvSwiGLU: return pick_kh<kGemvSwiGLU, FP8>(kh, bt);
    case kGemvRmsNormSwiGLU: return pick_kh<kGemvRmsNormSwiGLU, FP8>(kh, bt);
    default: return pick_kh<kGemvPlain, FP8>(kh, bt);
  }
}

// Four groups of 32 batch rows in 4-k-step chunks would spill (256 VGPRs
// and scratch); that combination takes 2-k-step chunks.
template <int KC, int BT, bool FP8, bool XS>
MfmaFn pick_long_gpw(int gpw) {
  constexpr int KC4 = KC == 4 && BT == 4 ? 2 : KC;
  return gpw == 1 ? gemv_mfma_long_kernel<KC, BT, 1, FP8, XS>
                  : gpw == 2 ? gemv_mfma_long_kernel<KC, BT, 2, FP8, XS>
                             : gemv_mfma_long_kernel<KC4, BT, 4, FP8, XS>;
}

template <int KC, bool FP8, bool XS>
MfmaFn pick_long_bt(int bt, int gpw) {
  return bt == 1 ? pick_long_gpw<KC, 1, FP8, XS>(gpw)
                 : bt == 2 ? pick_long_gpw<KC, 2, FP8, XS>(gpw)
                           : pick_long_gpw<KC, 4, FP8, XS>(gpw);
}

template <bool FP8, bool XS>
MfmaFn pick_long_kc(int kc, int bt, int gpw) {
  return kc == 2 ? pick_long_bt<2, FP8, XS>(bt, gpw) : pick_long_bt<4, FP8, XS>(bt, gpw);
}

template <bool FP8>
MfmaFn pick_long(int kc, int bt, int gpw, bool xs) {
  return xs ? pick_long_kc<FP8, true>(kc, bt, gpw) : pick_long_kc<FP8, false>(kc, bt, gpw);
}

// The gate/up pair on 16-row tiles: 4 waves, 2 (fp16) or 4 (e4m3, whose
// whole lines span 4 k-steps) k-steps per chunk, 16 or 32 batch rows, 1, 2
// or 4 tiles (2, 4 or 8 groups).
constexpr int kPairWaves = 4;

template <int KC, int BT16, bool FP8, bool NORM>
MfmaFn pick_pair_t(int t) {
  return t == 1 ? gemv_mfma_tile16_kernel<2, kPairWaves, KC, BT16, 1, FP8, NORM>
         : t == 2 ? gemv_mfma_tile16_kernel<2, kPairWaves, KC, BT16, 2, FP8, NORM>
                  : gemv_mfma_tile16_kernel<2, kPairWaves, KC, BT16, 4, FP8, NORM>;
}

// fp16 with the norm takes 2-k-step chunks only (4 would spill at 32 rows).
template <bool FP8, bool NORM>
MfmaFn pick_pair_n(int kc, int bt16, int t) {
  if constexpr (!FP8 && NORM) {
    (void)kc;
    return bt16 == 1 ? pick_pair_t<2, 1, FP8, NORM>(t) : pick_pair_t<2, 2, FP8, NORM>(t);
  } else {
    if constexpr (!FP8) {
      if (kc == 2)
        return bt16 == 1 ? pick_pair_t<2, 1, FP8, NORM>(t) : pick_pair_t<2, 2, FP8, NORM>(t);
    }
    return bt16 == 1 ? pick_pair_t<4, 1, FP8, NORM>(t) : pick_pair_t<4, 2, FP8, NORM>(t);
  }
}

template <bool FP8>
MfmaFn pick_pair(int kc, int bt16, int t, bool norm) {
  return norm ? pick_pair_n<FP8, true>(kc, bt16, t) : pick_pair_n<FP8, false>(kc, bt16, t);
}

}  // namespace

// Long rows (plain GEMV, K a multiple of 2048 above 4096): both operands
// stream in K chunks.
static bool long_rows(GemvMode mode, int K) {
  return mode == kGemvPlain && K > 4096 && K % 2048 == 0;
}

// The gate/up pair from pair_min rows (K a multiple of 2048, N of 8): x
// streams, one pass up to 32 rows.
static bool pair_rows(GemvMode mode, int B, int K, int N) {
  const int pair_min = tuning().gemv_pair_min_batch > 0 ? tuning().gemv_pair_min_batch : 17;
  // The RMSNorm mode's statistic pass covers K <= 4096 (2 pieces per lane).
  const bool mode_ok = mode == kGemvSwiGLU || (mode == kGemvRmsNormSwiGLU && K <= 4096);
  return mode_ok && K % 2048 == 0 && N % kRowsPerGroup == 0 &&
         (size_t)2 * N * K * 2 < ((size_t)1 << 32) && B >= pair_min;
}

bool gemv_mfma_supported(GemvMode mode, int B, int K, int N) {
  if (B < 2 || N < 1) return false;
  if (long_rows(mode, K) || pair_rows(mode, B, K, N)) return true;
  if (K != 2048 && K != 4096) return false;  // K / 512 = 4 or 8 k-steps per half
  const int groups = (N + kRowsPerGroup - 1) / kRowsPerGroup;
  return groups <= 256 * kMaxGroupsPerWg;
}

static hipError_t launch_gemv_mfma_long(const MfmaArgs& a0, bool fp8, int cu_count,
                                        hipStream_t stream) {
  MfmaArgs a = a0;
  // Batch tiles of 8 per pass: up to 32 rows in one pass, so the weights
  // are read once up to batch 32.
  const int bt = a.B <= 8 ? 1 : a.B <= 16 ? 2 : 4;
  // Chunk size, measured at [4096, 14336] (µs, staged x, 2 groups per
  // workgroup, 4- against 2-k-step chunks): e4m3 at 3-8 rows 11.9 / 13.4
  // against 13.3 / 14.2 (its 2-k-step sets hold only 2 KB of weights per
  // wave); fp16 at 8 rows 21.5 against 21.1, at 16 rows 25.3 against 24.8;
  // at 32 rows the 4-k-step sets spill.
  int kc = tuning().gemv_long_kc;
  if (kc == 0) kc = fp8 && bt == 1 ? 4 : 2;
  // Row groups per workgroup: the fewest (1, 2 or 4) that put every pass's
  // workgroups on the CUs at once.  Above 32 rows the passes of a row group
  // then run side by side on one XCD (grid.x a multiple of 8, as in
  // launch_gemv_mfma) and share its L2 copy of the weights: [4096, 14336]
  // on 128 workgroups of 4 groups per pass against 256 of 2: fp16 B = 64
  // 64.1 -> 48.6 us, B = 96 97.5 -> 91.9 us, e4m3 B = 33-64 42-47 -> 33 us.
  // At one pass, 4 groups per workgroup on half the CUs measured slower
  // (fp16 B = 32 32.3 -> 45.7 us).
  const int passes = (a.B + 8 * bt - 1) / (8 * bt);
  int gpw = tuning().gemv_long_gpw;
  if (gpw == 0) {
    gpw = 4;
    for (int g = 1; g < 4; g *= 2)
      if ((a.groups + g - 1) / g * passes <= cu_count) {
        gpw = g;
        break;
      }
  }
  a.gpw = gpw;
  int grid = (a.groups + gpw - 1) / gpw;
  if (passes > 1) grid = min(a.groups, (grid + 7) / 8 * 8);
  if (bt == 4 && gpw == 4) kc = 2;
  const bool xs = tuning().gemv_long_stage != 1;
  const MfmaFn fn = fp8 ? pick_long<true>(kc, bt, gpw, xs) : pick_long<false>(kc, bt, gpw, xs);
  const size_t lds = xs ? (size_t)kWavesM * bt * kc * kWave * 16 : 0;
  if (lds > 48 * 1024) {
    hipError_t e = allow_large_lds(reinterpret_cast<const void*>(fn), lds);
    if (e != hipSuccess) return e;
  }
  dim3 g(grid, (a.B + 8 * bt - 1) / (8 * bt));
  hipLaunchKernelGGL(fn, g, dim3(kThreadsM), lds, stream, a);
  return hipGetLastError();
}

// The gate/up pair from 17 rows, measured at [14336, 4096] (µs, graph back to
// back; 16-row passes / streamed on 8-row halves / on 16-row tiles loaded
// directly / on 16-row tiles merged from whole lines): fp16 B = 17 74.1 /
// 43.5 / 53.0 / 39.7, B = 32 76.2 / 44.4 / 55.1 / 42.0; e4m3 B = 17 40.5 /
// 43.7 / 29.3 / 25.5, B = 32 42.4 / 45.3 / 32.0 / 28.1.  The halves hold
// four times the accumulators (the register allocator then moved them
// through a shared temporary between MFMAs); the direct tiles read half
// lines.  4-k-step fp16 chunks measured 1.5-2.3 us slower, 8-wave
// workgroups 5-6 us slower.
static hipError_t launch_gemv_mfma_pair(const MfmaArgs& a0, bool norm, bool fp8, int cu_count,
                                        hipStream_t stream) {
  MfmaArgs a = a0;
  // The kernel's 32-bit lane offsets (see gemv_mfma_tile16_kernel).
  if (a.N % kRowsPerGroup != 0 ||
      (size_t)2 * a.N * a.K * (fp8 ? 1 : 2) >= ((size_t)1 << 32))
    return hipErrorInvalidValue;
  const int bt16 = a.B <= 16 ? 1 : 2;  // passes of 16 or 32 rows
  const int kc = fp8 ? 4 : !norm && tuning().gemv_long_kc == 4 ? 4 : 2;
  int gpw = (a.groups + cu_count - 1) / cu_count;
  if (gpw > 8) gpw = 8;
  const int t = gpw <= 2 ? 1 : gpw <= 4 ? 2 : 4;
  a.gpw = gpw;
  const int grid = (a.groups + gpw - 1) / gpw;
  const MfmaFn fn =
      fp8 ? pick_pair<true>(kc, bt16, t, norm) : pick_pair<false>(kc, bt16, t, norm);
  const size_t lds = sizeof(float) * 2 * t * 2 * kPairWaves * 16 * bt16 * kRowsPerGroup;
  if (lds > 48 * 1024) {
    hipError_t e = allow_large_lds(reinterpret_cast<const void*>(fn), lds);
    if (e != hipSuccess) return e;
  }
  dim3 g(grid, (a.B + 16 * bt16 - 1) / (16 * bt16));
  hipLaunchKernelGGL(fn, g, dim3(kPairWaves * kWave), lds, stream, a);
  return hipGetLastError();
}

hipError_t launch_gemv_mfma(GemvMode mode, const void* x, const void* gamma,
                            const GemvWeights& w, void* y, int B, int K, int N, float eps,
                            int cu_count, hipStream_t stream) {
  MfmaArgs a;
  a.part_off = 0;
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
  a.groups = (N + kRowsPerGroup - 1) / kRowsPerGroup;
  if (long_rows(mode, K)) return launch_gemv_mfma_long(a, w.fp8, cu_count, stream);
  if (pair_rows(mode, B, K, N))
    return launch_gemv_mfma_pair(a, mode == kGemvRmsNormSwiGLU, w.fp8, cu_count, stream);
  const int kh = K / 512;
  const int nwm = gemv_is_swiglu(mode) ? 2 : 1;
  // One weight matrix above 16 rows: P = ceil(B / 16) passes of 16 rows
  // (grid.y), each on CUs / P workgroups, a multiple of 8.  Workgroup
  // (x, y) is then linear id x + grid.x * y, so with workgroups dealt to
  // the 8 XCDs in turn every pass of a row group runs on the same XCD at
  // the same time, and its weight lines come from HBM once and from that
  // XCD's L2 for the other passes, while each CU reads 16 rows of x rather
  // than 32.  Measured on MI355X (graph back-to-back) against 32-row passes
  // on the full grid (XB below): F1 [4096, 4096] B = 32 16.2 -> 13.2 us,
  // B = 64 29.8 -> 20.1 us; F1-QKV [6144, 4096] B = 17 17.4 -> 16.7 us,
  // B = 32 18.0 -> 16.9 us, B = 64 33.5 -> 27.4 us; e4m3 F1-QKV B = 32
  // 15.5 -> 11.8 us.  A grid that is not a multiple of 8 loses the shared
  // L2 (F1-QKV B = 48 on 77 workgroups per pass: 28.3 against 23.8 us on
  // 80), and 8-row passes on twice the workgroups were slower at 16 and 32
  // rows.
  const int passes = (B + kBatchTile - 1) / kBatchTile;
  const bool split_passes = nwm == 1 && passes > 1 && tuning().gemv_xb == 0;
  int grid = min(a.groups, cu_count);
  if (split_passes) {
    const int forced = tuning().gemv_pass_grid;
    grid = min(a.groups, max(8, (forced > 0 ? forced : cu_count / passes) / 8 * 8));
  }
  a.gpw = (a.groups + grid - 1) / grid;
  if (a.gpw > kMaxGroupsPerWg) a.gpw = kMaxGroupsPerWg;
  // Spread the groups evenly: every workgroup owns gpw or gpw - 1 groups
  // (or, on a split-pass grid rounded up to a multiple of 8, at least one).
  grid = (a.groups + a.gpw - 1) / a.gpw;
  if (split_passes) grid = min(a.groups, (grid + 7) / 8 * 8);
  // gemv_xb: 32-row passes when the LDS holds rows 16..31 of x (16 KB x KH)
  // next to the 32-column partial sums.
  const size_t xb_bytes = (size_t)kWavesM * 2 * kh * kWave * 16;
  const size_t part32 = sizeof(float) * a.gpw * nwm * kWavesM * 32 * kRowsPerGroup;
  const bool xb = !split_passes && nwm == 1 && B > kBatchTile && xb_bytes + part32 <= 152 * 1024;
  const int bt = xb || B >= 9 ? 2 : 1;  // batch column tiles held in registers
  const int pass = xb ? 32 : kBatchTile;
  const MfmaFn fn = w.fp8 ? pick_mode<true>(mode, kh, bt, xb) : pick_mode<false>(mode, kh, bt, xb);
  // The activation staging (the norm modes, and one matrix at two batch
  // tiles) without XB -- each wave's slice of the pass's rows, 16 bytes per
  // lane per row tile and k-step -- shares the partial-sum region.
  const bool staged = gemv_has_norm(mode) || (nwm == 1 && bt == 2);
  const size_t stage_bytes = staged ? (size_t)kWavesM * bt * kh * kWave * 16 : 0;
  const size_t part16 = sizeof(float) * a.gpw * nwm * kWavesM * 8 * bt * kRowsPerGroup;
  size_t lds = xb ? xb_bytes + part32 : (part16 > stage_bytes ? part16 : stage_bytes);
  a.part_off = 0;
  if (staged && !xb) {
    // Partial sums past the staging area where both fit: then no wave waits
    // for the others' read-back before its first partial-sum store.
    const size_t both = stage_bytes + part16;
    if (both <= 48 * 1024 || allow_large_lds(reinterpret_cast<const void*>(fn), both) == hipSuccess) {
      lds = both;
      a.part_off = (int)(stage_bytes / 16);
    }
  }
  if (lds > 48 * 1024) {
    hipError_t e = allow_large_lds(reinterpret_cast<const void*>(fn), lds);
    if (e != hipSuccess) return e;
  }
  dim3 g(grid, (B + pass - 1) / pass);
  hipLaunchKernelGGL(fn, g, dim3(kThreadsM), lds, stream, a);
  return hipGetLastError();
}

}  // namespace dbk
