// abi.hip -- the extern "C" surface of libdecodebench_hip.so.
//
// Each entry point checks its whole argument contract first and returns
// DB_ERR_INVALID without touching the HIP runtime when it is broken, so the
// checks can be exercised on a host without a GPU.  Only then is the device
// queried (CU count, cached per device) and the kernel launched on the
// caller's stream.
#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <atomic>

#include "../../include/decodebench_hip.h"
#include "../../include/decodebench_hip_tuning.h"
#include "db_kernels.h"

namespace dbk {

// The knobs are per host thread: a value one thread sets through db_tune
// changes only the launches that thread makes.
Tuning& tuning() {
  static thread_local Tuning t;
  return t;
}

namespace {
// A positive device attribute of the current device, cached per device.
int device_attribute(hipDeviceAttribute_t attr, std::atomic<int> (&cache)[64], int* err) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    *err = (int)e;
    return 0;
  }
  if (dev >= 0 && dev < 64) {
    const int c = cache[dev].load(std::memory_order_relaxed);
    if (c > 0) {
      *err = 0;
      return c;
    }
  }
  int value = 0;
  e = hipDeviceGetAttribute(&value, attr, dev);
  if (e != hipSuccess || value <= 0) {
    *err = e != hipSuccess ? (int)e : (int)hipErrorInvalidValue;
    return 0;
  }
  if (dev >= 0 && dev < 64) cache[dev].store(value, std::memory_order_relaxed);
  *err = 0;
  return value;
}
}  // namespace

int device_cu_count(int* err) {
  static std::atomic<int> cache[64];
  return device_attribute(hipDeviceAttributeMultiprocessorCount, cache, err);
}

int device_xcc_count(int* err) {
  static std::atomic<int> cache[64];
  return device_attribute(hipDeviceAttributeNumberOfXccs, cache, err);
}

int f4_max_splits(int G);

}  // namespace dbk

namespace {

thread_local char g_err[512];

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_err[0] = '\0';
  return DB_OK;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return ok();
  return fail((int)e, "%s: HIP error %d (%s)", what, (int)e, hipGetErrorString(e));
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// LDS budget of one GEMV workgroup for its activation rows (gfx950: 160 KB
// per CU; keep 8 KB for static arrays).
constexpr size_t kGemvLdsBudget = 152 * 1024;

bool aligned4(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 3u) == 0; }

// Common GEMV contract.  W2/scale2 belong to the second matrix of the SwiGLU
// entry points (NULL otherwise; `pair` says whether one is expected).
int check_gemv(const char* fn, const void* x, const void* W, const void* y,
               int B, int K, int N, int w_dtype, const void* scale,
               const void* W2, const void* scale2, bool pair) {
  if (!x || !W || !y || (pair && !W2))
    return fail(DB_ERR_INVALID, "%s: null tensor pointer", fn);
  if (B < 1 || N < 1 || K < 8)
    return fail(DB_ERR_INVALID, "%s: need B >= 1, N >= 1, K >= 8 (got B=%d K=%d N=%d)",
                fn, B, K, N);
  if (K % 8 != 0) return fail(DB_ERR_INVALID, "%s: K=%d must be a multiple of 8", fn, K);
  if ((size_t)K * 16 > kGemvLdsBudget * 8)
    return fail(DB_ERR_INVALID, "%s: K=%d exceeds the LDS activation budget", fn, K);
  if (!aligned16(x) || !aligned16(W) || !aligned16(y) || (W2 && !aligned16(W2)))
    return fail(DB_ERR_INVALID, "%s: tensors must be 16-byte aligned", fn);
  if (w_dtype == DB_DTYPE_F16) {
    if (scale || scale2)
      return fail(DB_ERR_INVALID, "%s: fp16 weights take no scale vector", fn);
  } else if (w_dtype == DB_DTYPE_FP8_E4M3) {
    if (K % 16 != 0)
      return fail(DB_ERR_INVALID, "%s: K=%d must be a multiple of 16 for fp8 weights", fn, K);
    if (!scale || (pair && !scale2))
      return fail(DB_ERR_INVALID, "%s: fp8 weights need a per-row fp32 scale vector", fn);
    if (!aligned4(scale) || (scale2 && !aligned4(scale2)))
      return fail(DB_ERR_INVALID, "%s: scale vectors must be 4-byte aligned", fn);
  } else {
    return fail(DB_ERR_INVALID, "%s: unknown weight dtype %d", fn, w_dtype);
  }
  return DB_OK;
}

int check_norm(const char* fn, const void* g, float eps) {
  if (!g) return fail(DB_ERR_INVALID, "%s: null gain pointer", fn);
  if (!aligned16(g)) return fail(DB_ERR_INVALID, "%s: tensors must be 16-byte aligned", fn);
  if (!(eps >= 0.0f) || !isfinite(eps))
    return fail(DB_ERR_INVALID, "%s: eps must be finite and >= 0", fn);
  return DB_OK;
}

dbk::GemvWeights weights(int w_dtype, const void* w0, const void* w1, const float* s0,
                         const float* s1) {
  return dbk::GemvWeights{w0, w1, s0, s1, w_dtype == DB_DTYPE_FP8_E4M3};
}

int run_gemv(const char* fn, dbk::GemvMode mode, const void* x, const void* g,
             const dbk::GemvWeights& w, void* y, int B, int K, int N, float eps,
             void* stream) {
  int err = 0;
  const int cus = dbk::device_cu_count(&err);
  if (err) return hip_status((hipError_t)err, fn);
  return hip_status(dbk::launch_gemv(mode, x, g, w, y, B, K, N, eps, cus, (hipStream_t)stream),
                    fn);
}

__global__ void null_kernel() {}

}  // namespace

extern "C" {

int db_abi_version(void) { return DB_ABI_VERSION; }

const char* db_last_error(void) { return g_err; }

int db_device_cu_count(int* cu_count) {
  if (!cu_count) return fail(DB_ERR_INVALID, "db_device_cu_count: null output");
  int err = 0;
  const int c = dbk::device_cu_count(&err);
  if (err) return hip_status((hipError_t)err, "db_device_cu_count");
  *cu_count = c;
  return ok();
}

int db_f1_rmsnorm_gemv(const void* x, const void* g, const void* W,
                       const float* w_scale, void* y, int B, int K, int N,
                       float eps, int w_dtype, void* stream) {
  const char* fn = "db_f1_rmsnorm_gemv";
  int rc = check_norm(fn, g, eps);
  if (!rc) rc = check_gemv(fn, x, W, y, B, K, N, w_dtype, w_scale, nullptr, nullptr, false);
  if (rc) return rc;
  return run_gemv(fn, dbk::kGemvRmsNorm, x, g, weights(w_dtype, W, nullptr, w_scale, nullptr),
                  y, B, K, N, eps, stream);
}

int db_f2_gateup_swiglu(const void* x, const void* Wg, const void* Wu,
                        const float* sg, const float* su, void* y, int B,
                        int K, int N, int w_dtype, void* stream) {
  const char* fn = "db_f2_gateup_swiglu";
  int rc = check_gemv(fn, x, Wg, y, B, K, N, w_dtype, sg, Wu, su, true);
  if (rc) return rc;
  return run_gemv(fn, dbk::kGemvSwiGLU, x, nullptr, weights(w_dtype, Wg, Wu, sg, su), y, B,
                  K, N, 0.0f, stream);
}

int db_f2_rmsnorm_gateup_swiglu(const void* x, const void* g, const void* Wg,
                                const void* Wu, const float* sg, const float* su,
                                void* y, int B, int K, int N, float eps,
                                int w_dtype, void* stream) {
  const char* fn = "db_f2_rmsnorm_gateup_swiglu";
  int rc = check_norm(fn, g, eps);
  if (!rc) rc = check_gemv(fn, x, Wg, y, B, K, N, w_dtype, sg, Wu, su, true);
  if (rc) return rc;
  return run_gemv(fn, dbk::kGemvRmsNormSwiGLU, x, g, weights(w_dtype, Wg, Wu, sg, su), y, B,
                  K, N, eps, stream);
}

int db_gemv(const void* x, const void* W, const float* w_scale, void* y, int B,
            int K, int N, int w_dtype, void* stream) {
  const char* fn = "db_gemv";
  int rc = check_gemv(fn, x, W, y, B, K, N, w_dtype, w_scale, nullptr, nullptr, false);
  if (rc) return rc;
  return run_gemv(fn, dbk::kGemvPlain, x, nullptr, weights(w_dtype, W, nullptr, w_scale, nullptr),
                  y, B, K, N, 0.0f, stream);
}

int db_f4_default_splits(int B, int Hkv, int L, int cu_count) {
  if (B < 1 || Hkv < 1 || L < 1 || cu_count < 1) return 1;
  return dbk::f4_choose_splits(B, Hkv, L, cu_count);
}

size_t db_f4_workspace_bytes(int B, int Hq, int Hkv, int L, int D, int S) {
  if (B < 1 || Hq < 1 || Hkv < 1 || Hq % Hkv || L < 1 || D < 1 || S <= 1) return 0;
  return dbk::f4_workspace_bytes(B, Hq, Hkv, S, D);
}

}  // extern "C"

namespace {

// Argument contract shared by the F4 entry points (workspace aside).
int check_f4(const char* fn, const void* q, const void* k, const void* v, const void* o,
             int B, int Hq, int Hkv, int L, int D, int S, float scale) {
  if (!q || !k || !v || !o) return fail(DB_ERR_INVALID, "%s: null tensor pointer", fn);
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o))
    return fail(DB_ERR_INVALID, "%s: tensors must be 16-byte aligned", fn);
  if (B < 1 || Hq < 1 || Hkv < 1 || L < 1)
    return fail(DB_ERR_INVALID, "%s: need B, Hq, Hkv, L >= 1 (got %d %d %d %d)", fn, B,
                Hq, Hkv, L);
  if (D != 128) return fail(DB_ERR_INVALID, "%s: head_dim D=%d, only 128 is supported", fn, D);
  if (Hq % Hkv != 0)
    return fail(DB_ERR_INVALID, "%s: Hq=%d is not a multiple of Hkv=%d", fn, Hq, Hkv);
  const int G = Hq / Hkv;
  if (G != 1 && G != 2 && G != 4 && G != 8)
    return fail(DB_ERR_INVALID, "%s: query heads per KV head G=%d not in {1,2,4,8}", fn, G);
  if (S < 1 || S > 256 || S > dbk::f4_max_splits(G))
    return fail(DB_ERR_INVALID, "%s: split count S=%d outside [1, 256]", fn, S);
  if (!isfinite(scale)) return fail(DB_ERR_INVALID, "%s: scale must be finite", fn);
  if ((size_t)B * Hkv * L * D >= ((size_t)1 << 40))
    return fail(DB_ERR_INVALID, "%s: KV cache too large", fn);
  return DB_OK;
}

// Splits a call actually runs: never more than the 16-row tiles of L.
int f4_effective_splits(int L, int S) {
  const int ntiles = (L + 15) / 16;
  return S < ntiles ? S : ntiles;
}

// The launch-geometry knobs of db_tune / db_tune_get: name, field, the
// values accepted (checked before anything changes) and, for one knob, how
// a value is stored.
struct Knob {
  const char* name;
  int dbk::Tuning::*field;
  bool (*valid)(int);
  const char* rule;
  int (*normalise)(int);
};

const Knob kKnobs[] = {
    {"gemv_waves_per_cu", &dbk::Tuning::gemv_waves_per_cu, [](int) { return true; },
     "any value (<= 0: the default)", [](int v) { return v > 0 ? v : 0; }},
    {"gemv_mfma_min_batch", &dbk::Tuning::gemv_mfma_min_batch,
     [](int v) { return v == 0 || v >= 2; }, "0 (automatic) or >= 2", nullptr},
    {"f4_blocks_per_cu", &dbk::Tuning::f4_blocks_per_cu, [](int v) { return v >= 1; }, ">= 1",
     nullptr},
    {"f4_min_tiles", &dbk::Tuning::f4_min_tiles, [](int v) { return v >= 1; }, ">= 1", nullptr},
    {"f4_waves", &dbk::Tuning::f4_waves, [](int v) { return v == 0 || v == 4 || v == 8; },
     "0, 4 or 8", nullptr},
    {"f4_merge", &dbk::Tuning::f4_merge, [](int v) { return v >= 0 && v <= 2; },
     "0 (automatic), 1 (in the same launch where possible) or 2 (second launch)", nullptr},
    {"f4_misplace", &dbk::Tuning::f4_misplace, [](int v) { return v >= 0; },
     ">= 0 (0: off)", nullptr},
    {"f4_line", &dbk::Tuning::f4_line, [](int v) { return v >= 0 && v <= 2; },
     "0 (auto), 1 (whole lines) or 2", nullptr},
    {"f4_combine_groups", &dbk::Tuning::f4_combine_groups,
     [](int v) { return v == 0 || v == 1 || v == 2 || v == 4 || v == 8; }, "0, 1, 2, 4 or 8",
     nullptr},
    {"f4_depth", &dbk::Tuning::f4_depth, [](int v) { return v >= 0 && v <= 2; }, "0, 1 or 2",
     nullptr},
    {"gemv_long_kc", &dbk::Tuning::gemv_long_kc, [](int v) { return v == 0 || v == 2 || v == 4; },
     "0, 2 or 4", nullptr},
    {"gemv_long_gpw", &dbk::Tuning::gemv_long_gpw,
     [](int v) { return v == 0 || v == 1 || v == 2 || v == 4; }, "0, 1, 2 or 4", nullptr},
    {"gemv_long_stage", &dbk::Tuning::gemv_long_stage, [](int v) { return v >= 0 && v <= 2; },
     "0, 1 or 2", nullptr},
    {"gemv_pair_min_batch", &dbk::Tuning::gemv_pair_min_batch,
     [](int v) { return v == 0 || v >= 2; }, "0 (automatic) or >= 2", nullptr},
    {"stream_waves", &dbk::Tuning::stream_waves,
     [](int v) { return v == 0 || v == 1 || v == 2 || v == 4; }, "0, 1, 2 or 4", nullptr},
    {"gemv_pass_grid", &dbk::Tuning::gemv_pass_grid, [](int v) { return v >= 0 && v % 8 == 0; },
     "0 (automatic) or a multiple of 8", nullptr},
    {"gemv_xb", &dbk::Tuning::gemv_xb, [](int v) { return v == 0 || v == 1; }, "0 or 1",
     nullptr},
    {"f4_launch", &dbk::Tuning::f4_launch, [](int v) { return v >= 0 && v <= 2; },
     "0 (both launches), 1 (split kernel only) or 2 (merge only)", nullptr},
};

const Knob* find_knob(const char* key) {
  for (const Knob& k : kKnobs)
    if (!strcmp(k.name, key)) return &k;
  return nullptr;
}

}  // namespace

extern "C" {

int db_f4_splitkv(const void* q, const void* k, const void* v, void* o,
                  void* ws, size_t ws_bytes, int B, int Hq, int Hkv, int L,
                  int D, int S, float scale, void* stream) {
  const char* fn = "db_f4_splitkv";
  const int rc = check_f4(fn, q, k, v, o, B, Hq, Hkv, L, D, S, scale);
  if (rc) return rc;
  const int s_eff = f4_effective_splits(L, S);
  if (s_eff > 1) {
    const size_t need = dbk::f4_workspace_bytes(B, Hq, Hkv, S, D);
    if (!ws) return fail(DB_ERR_INVALID, "%s: S=%d needs a workspace", fn, S);
    if (!aligned16(ws)) return fail(DB_ERR_INVALID, "%s: workspace must be 16-byte aligned", fn);
    if (ws_bytes < need)
      return fail(DB_ERR_INVALID, "%s: workspace %zu bytes < %zu required", fn, ws_bytes,
                  need);
  }
  int err = 0;
  const int nxcc = dbk::device_xcc_count(&err);
  if (err) return hip_status((hipError_t)err, fn);
  return hip_status(dbk::launch_f4(q, k, v, o, ws, B, Hq, Hkv, L, D, S, scale, nxcc,
                                   (hipStream_t)stream),
                    fn);
}

int db_f4_splitkv_noalloc(const void* q, const void* k, const void* v, void* o,
                          int B, int Hq, int Hkv, int L, int D, int S,
                          float scale, void* stream) {
  const char* fn = "db_f4_splitkv_noalloc";
  const int rc = check_f4(fn, q, k, v, o, B, Hq, Hkv, L, D, S, scale);
  if (rc) return rc;
  const int s_eff = f4_effective_splits(L, S);
  void* ws = nullptr;
  if (s_eff > 1) {
    const size_t need = dbk::f4_workspace_bytes(B, Hq, Hkv, s_eff, D);
    if (need > DB_F4_SCRATCH_BYTES)
      return fail(DB_ERR_INVALID,
                  "%s: %d splits of B=%d x Hq=%d need %zu bytes of partial records, more "
                  "than the %zu-byte scratch array; use fewer splits or db_f4_splitkv",
                  fn, s_eff, B, Hq, need, (size_t)DB_F4_SCRATCH_BYTES);
    const hipError_t e = dbk::f4_scratch_address(&ws);
    if (e != hipSuccess) return hip_status(e, fn);
  }
  return hip_status(dbk::launch_f4(q, k, v, o, ws, B, Hq, Hkv, L, D, s_eff, scale, /*nxcc=*/1,
                                   (hipStream_t)stream, /*allow_fused_merge=*/false),
                    fn);
}

int db_stream_read(const void* src, size_t bytes, int kb_per_wave, unsigned magic,
                   unsigned* sink, void* stream) {
  const char* fn = "db_stream_read";
  if (!src || !sink) return fail(DB_ERR_INVALID, "%s: null pointer", fn);
  if (!aligned16(src) || !aligned16(sink))
    return fail(DB_ERR_INVALID, "%s: src and sink must be 16-byte aligned", fn);
  if (kb_per_wave != 4 && kb_per_wave != 8 && kb_per_wave != 16)
    return fail(DB_ERR_INVALID, "%s: kb_per_wave=%d not in {4, 8, 16}", fn, kb_per_wave);
  const size_t chunk = (size_t)kb_per_wave * 1024;
  if (bytes == 0 || bytes % chunk)
    return fail(DB_ERR_INVALID, "%s: bytes=%zu is not a positive multiple of %zu", fn, bytes,
                chunk);
  if (bytes / chunk > ((size_t)1 << 31))
    return fail(DB_ERR_INVALID, "%s: bytes=%zu is too large", fn, bytes);
  return hip_status(dbk::launch_stream_read(src, bytes, kb_per_wave, magic, sink,
                                            (hipStream_t)stream),
                    fn);
}

int db_stream_capture_id(void* stream, unsigned long long* capture_id) {
  if (!capture_id) return fail(DB_ERR_INVALID, "db_stream_capture_id: null output");
  hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
  unsigned long long id = 0;
  const hipError_t e = hipStreamGetCaptureInfo((hipStream_t)stream, &status, &id);
  if (e != hipSuccess) return hip_status(e, "db_stream_capture_id");
  *capture_id = status == hipStreamCaptureStatusActive ? id : 0;
  return ok();
}

int db_null_kernel(void* stream) {
  hipLaunchKernelGGL(null_kernel, dim3(1), dim3(256), 0, (hipStream_t)stream);
  return hip_status(hipGetLastError(), "db_null_kernel");
}

int db_tune(const char* key, int value) {
  if (!key) return fail(DB_ERR_INVALID, "db_tune: null key");
  const Knob* k = find_knob(key);
  if (!k) return fail(DB_ERR_INVALID, "db_tune: unknown key '%s'", key);
  if (!k->valid(value)) return fail(DB_ERR_INVALID, "db_tune: %s must be %s", key, k->rule);
  dbk::tuning().*(k->field) = k->normalise ? k->normalise(value) : value;
  return ok();
}

int db_f4_launch_info(int B, int Hq, int Hkv, int L, int S, int* splits, int* launches) {
  const char* fn = "db_f4_launch_info";
  if (!splits || !launches) return fail(DB_ERR_INVALID, "%s: null output", fn);
  if (B < 1 || Hq < 1 || Hkv < 1 || L < 1 || Hq % Hkv != 0 || S < 1 || S > 256)
    return fail(DB_ERR_INVALID, "%s: invalid shape", fn);
  int err = 0;
  const int nxcc = dbk::device_xcc_count(&err);
  if (err) return hip_status((hipError_t)err, fn);
  const dbk::F4Plan p = dbk::f4_plan(B, Hkv, L, S, nxcc, true);
  *splits = p.splits;
  *launches = p.splits > 1 && !p.fused_merge && dbk::tuning().f4_launch == 0 ? 2 : 1;
  return ok();
}

int db_tune_get(const char* key, int* value) {
  if (!key || !value) return fail(DB_ERR_INVALID, "db_tune_get: null argument");
  const Knob* k = find_knob(key);
  if (!k) return fail(DB_ERR_INVALID, "db_tune_get: unknown key '%s'", key);
  *value = dbk::tuning().*(k->field);
  return ok();
}

}  // extern "C"
