// db_kernels.h -- host-side launchers shared by the kernel files and the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>

#include "decodebench_hip.h"

namespace dbk {

// Launch geometry knobs; defaults are the tuned MI355X values.  They can be
// changed at run time through db_tune() for launch-shape sweeps; each host
// thread has its own set.
struct Tuning {
  int gemv_waves_per_cu = 0;   // 0: the default, 32 waves per CU
  int gemv_mfma_min_batch = 0; // smallest batch that takes the MFMA GEMV
                               // (0: the measured crossovers, 2 or 3 rows
                               // by mode and weight type, see launch_gemv)
  int f4_blocks_per_cu = 1;    // target F4 workgroups per CU
  int f4_min_tiles = 8;        // minimum 16-row tiles per F4 split
  int f4_waves = 0;            // waves per F4 workgroup (4 or 8; 0: auto)
  int f4_merge = 0;            // split merge: 0 automatic (in the same launch where
                               // the grid numbering allows), 1 the same, 2 second launch
  int f4_misplace = 0;         // test hook: F4 split s acts as if off its XCD when
                               // s % k == k - 1 (0: off)
  int f4_line = 0;             // F4 score layout: 0 auto, 1 whole-line K loads, 2 plain
  int f4_combine_groups = 0;   // split groups per F4 merge workgroup (0: auto)
  int f4_depth = 0;            // F4 tiles in flight per wave: 0 auto, 1 or 2
  int gemv_long_kc = 0;        // streamed-x MFMA GEMV k-steps per chunk: 0 auto, 2 or 4
  int gemv_long_gpw = 0;       // long-row MFMA GEMV row groups per workgroup: 0 auto, 1, 2, 4
  int gemv_long_stage = 0;     // long-row MFMA GEMV x: 0 auto, 1 direct, 2 LDS-staged
  int gemv_pair_min_batch = 0; // gate/up pair rows from which x streams (0: 17)
  int stream_waves = 0;        // db_stream_read waves per workgroup: 0 (4), 1, 2 or 4
  int gemv_pass_grid = 0;      // one-matrix MFMA GEMV above 16 rows: workgroups per
                               // 16-row pass (0: CUs / passes; else a multiple of 8)
  int gemv_xb = 0;             // 1: 32-row passes (rows 16..31 of x in LDS) on the
                               // full grid instead
  int f4_launch = 0;           // measurement hook for the two-launch F4: 0 both
                               // launches, 1 the split kernel only, 2 the merge only
};
Tuning& tuning();

// Compute units of the current device (cached per device ordinal).
int device_cu_count(int* err);
// XCDs (accelerator complex dies) of the current device, cached likewise.
int device_xcc_count(int* err);

enum GemvMode : int {
  kGemvPlain = 0,
  kGemvRmsNorm = 1,
  kGemvSwiGLU = 2,
  kGemvRmsNormSwiGLU = 3,
};

constexpr bool gemv_has_norm(int mode) {
  return mode == kGemvRmsNorm || mode == kGemvRmsNormSwiGLU;
}
constexpr bool gemv_is_swiglu(int mode) {
  return mode == kGemvSwiGLU || mode == kGemvRmsNormSwiGLU;
}

// Weights of one GEMV call: one matrix (two for the SwiGLU modes), fp16 or
// OCP e4m3 with one fp32 scale per output row.
struct GemvWeights {
  const void* w0;     // [N, K]  (gate in the SwiGLU modes)
  const void* w1;     // [N, K]  (up, SwiGLU modes only)
  const float* s0;    // [N]     row scales of w0 (fp8 only)
  const float* s1;    // [N]     row scales of w1 (fp8 SwiGLU only)
  bool fp8;
};

// y[B,N] = op(x[B,K]) . W^T  (fp16 activations in/out, fp32 accumulation).
//   kGemvPlain          : y = x W^T
//   kGemvRmsNorm        : y = fp16(fp16(x * rsqrt(mean(x^2) + eps)) * gamma) W^T
//   kGemvSwiGLU         : y = fp16(silu(fp16(x Wg^T)) * fp16(x Wu^T))
//   kGemvRmsNormSwiGLU  : the SwiGLU mode on the RMS-normalised x
// With fp8 weights every projection is fp32(sum) * row scale before its
// fp16 rounding.
hipError_t launch_gemv(GemvMode mode, const void* x, const void* gamma,
                       const GemvWeights& w, void* y, int B, int K, int N, float eps,
                       int cu_count, hipStream_t stream);

// MFMA variant for batches of up to 16 rows per pass (gemv_mfma.hip), fp16
// or e4m3 weights, K in {2048, 4096}.
bool gemv_mfma_supported(GemvMode mode, int B, int K, int N);
hipError_t launch_gemv_mfma(GemvMode mode, const void* x, const void* gamma,
                            const GemvWeights& w, void* y, int B, int K, int N, float eps,
                            int cu_count, hipStream_t stream);

// Split-KV GQA decode attention with the log-sum-exp combine in-kernel.
size_t f4_workspace_bytes(int B, int Hq, int Hkv, int S, int D);
int f4_choose_splits(int B, int Hkv, int L, int cu_count);
// How a call of S splits runs: the splits actually used (never more than
// the 16-row tiles of L), tiles per split, whether the workgroups of a
// (batch, kv-head) pair are numbered onto one XCD, and whether the splits
// are merged in the same launch (else in a second one).
struct F4Plan {
  int splits;
  int tiles_per_split;
  bool xcd_map;
  bool fused_merge;
};
F4Plan f4_plan(int B, int Hkv, int L, int S, int nxcc, bool allow_fused_merge);
// nxcc: the device's XCD count (the in-launch merge runs only with 8).
// allow_fused_merge = false keeps the merge in the second launch whatever
// db_tune("f4_merge") says, so the workspace tickets are never read.
hipError_t launch_f4(const void* q, const void* k, const void* v, void* o,
                     void* ws, int B, int Hq, int Hkv, int L, int D, int S,
                     float scale, int nxcc, hipStream_t stream,
                     bool allow_fused_merge = true);

// Bytes of the per-device scratch array behind db_f4_splitkv_noalloc.
constexpr size_t kF4ScratchBytes = DB_F4_SCRATCH_BYTES;
// Device address of that array on the current device (looked up once per
// device with hipGetSymbolAddress).
hipError_t f4_scratch_address(void** out);

// Read-only streaming probe (stream_probe.hip): `bytes` (a multiple of
// kb_per_wave KB, kb_per_wave in {4, 8, 16}) read once, kb_per_wave KB per
// wave; sink needs bytes / 16 words and is written only when the folded
// data equals `magic`.
hipError_t launch_stream_read(const void* src, size_t bytes, int kb_per_wave, unsigned magic,
                              unsigned* sink, hipStream_t stream);

}  // namespace dbk
