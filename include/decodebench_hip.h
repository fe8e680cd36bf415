/* decodebench_hip.h -- C ABI of libdecodebench_hip.so (MI355X / gfx950).
 *
 * The fused decode hot path of DecodeBench behind plain C entry points:
 * pointers, sizes and a HIP stream handle, no C++ or torch types.  Every
 * tensor is dense, row-major and 16-byte aligned; fp16 data is IEEE binary16.
 *
 * Conventions shared by every entry point
 *  - Return value: DB_OK (0) on success; DB_ERR_INVALID (-1) when an argument
 *    breaks the contract (checked before any HIP call, so it also works on a
 *    machine without a GPU); DB_ERR_UNSUPPORTED (-2) for a valid but not yet
 *    implemented combination; a positive value is the hipError_t the HIP
 *    runtime reported for the launch.  db_last_error() describes the last
 *    non-zero return on the calling thread.
 *  - The library never allocates, frees or synchronises and never reads
 *    device memory on the host; the caller owns every buffer, including the
 *    F4 workspace.  Kernels are launched only on `stream` (NULL = the legacy
 *    default stream), so a call can be captured into a hipGraph.
 *  - Calls are reentrant; two calls that share an F4 workspace must not
 *    overlap in time.
 *
 * Reference interfaces replaced (paths relative to the reference repository
 * animeshsri14/Decodebench):
 *  - the fused CUDA kernels f1_kernel / f2_kernel / f4_partial_kernel +
 *    f4_reduce_kernel, each taking the by-value parameter block KernelArgs
 *    (validation/include/decodebench_val/kernel_args.h:24-103), with launch
 *    geometry chosen by the native harness
 *    (validation/src/bench/bench_variant.cu:376-387, 558-565, 714-719, 753-763);
 *  - the torch-extension FFI pattern the reference documents for plugging a
 *    kernel into Sequence stages and Sequence.profile(fused=...)
 *    (examples/custom_kernel/bindings.cpp:13-30, kernel.cu:60-73).
 */
#ifndef DECODEBENCH_HIP_H
#define DECODEBENCH_HIP_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DB_ABI_VERSION 1

#define DB_OK 0
#define DB_ERR_INVALID (-1)
#define DB_ERR_UNSUPPORTED (-2)

/* Weight element types accepted by the GEMV entry points. */
#define DB_DTYPE_F16 0
#define DB_DTYPE_FP8_E4M3 1 /* OCP e4m3fn + per-output-row fp32 scale */

/* ABI revision of this header (DB_ABI_VERSION). */
int db_abi_version(void);

/* Message for the last non-zero return on this thread ("" if none). */
const char* db_last_error(void);

/* Compute units of the current HIP device (the F4 split policy uses it). */
int db_device_cu_count(int* cu_count);

/* F1: y[B,N] = fp16( xh[B,K] . W[N,K]^T ), where
 *       xh = fp16( fp16( x * rsqrt(mean(x^2, -1) + eps) ) * g )
 *     with the statistic in fp32 and the GEMV accumulated in fp32.
 * Replaces f1_kernel(KernelArgs) (validation/src/kernels/fused/f1.cu:18-84)
 * and the reference stages rmsnorm + gemv
 * (src/decodebench/demos/llama_decode.py:36-43).
 * Contract: B >= 1, N >= 1, K >= 8 and K % 8 == 0; x [B,K], g [K], W [N,K],
 * y [B,N] fp16.  w_dtype must be DB_DTYPE_F16 (w_scale NULL) or
 * DB_DTYPE_FP8_E4M3: W then holds N*K OCP e4m3fn bytes, K % 16 == 0, and
 * w_scale [N] fp32 (4-byte aligned) multiplies each row's fp32 dot product
 * before its fp16 rounding: y = fp16(w_scale[n] * sum_k e4m3(W[n,k]) xh[k]). */
int db_f1_rmsnorm_gemv(const void* x, const void* g, const void* W,
                       const float* w_scale, void* y, int B, int K, int N,
                       float eps, int w_dtype, void* stream);

/* F2: y[B,N] = fp16( fp16(silu(fp16(x Wg^T))) * fp16(x Wu^T) ), fp32
 * accumulation; the gate and up projections never leave registers.
 * Replaces f2_kernel(KernelArgs) (validation/src/kernels/fused/f2.cu:17-76)
 * and the reference stages gate, up, swiglu
 * (src/decodebench/demos/llama_decode.py:77-87).
 * Contract as db_f1_rmsnorm_gemv; sg/su are the per-row scales of Wg/Wu
 * when w_dtype is DB_DTYPE_FP8_E4M3, else NULL. */
int db_f2_gateup_swiglu(const void* x, const void* Wg, const void* Wu,
                        const float* sg, const float* su, void* y, int B,
                        int K, int N, int w_dtype, void* stream);

/* RMSNorm -> F2 in one kernel: y = F2(xh) with xh the F1 normalisation of x
 * (fp32 statistic, fp16(fp16(x * inv_rms) * g)), built once per workgroup in
 * LDS, so neither the normalised vector nor the gate/up projections reach
 * HBM.  It is the post-attention half of the decode-layer chain (rmsnorm
 * followed by gate, up, swiglu, src/decodebench/demos/llama_decode.py:36-39,
 * 77-87); the reference has no single fused kernel for the pair, so this
 * replaces the f1 prologue of f1_kernel (validation/src/kernels/fused/
 * f1.cu:18-50) feeding f2_kernel (f2.cu:17-76).
 * Contract as db_f2_gateup_swiglu, plus g [K] fp16 and eps as in
 * db_f1_rmsnorm_gemv. */
int db_f2_rmsnorm_gateup_swiglu(const void* x, const void* g, const void* Wg,
                                const void* Wu, const float* sg, const float* su,
                                void* y, int B, int K, int N, float eps,
                                int w_dtype, void* stream);

/* Plain GEMV y[B,N] = fp16( x[B,K] . W[N,K]^T ) with fp32 accumulation: the
 * unfused projection of the decode-layer chain (O and down projections).
 * Replaces gemv_kernel(KernelArgs) (validation/src/kernels/unfused/gemv.cu:15-48)
 * and the reference stage gemv (src/decodebench/demos/llama_decode.py:41-43).
 * Contract as db_f1_rmsnorm_gemv. */
int db_gemv(const void* x, const void* W, const float* w_scale, void* y,
            int B, int K, int N, int w_dtype, void* stream);

/* Split count the library picks for F4 when the caller has no preference:
 * about one (batch, kv-head, split) workgroup per CU of `cu_count` while
 * every split keeps at least eight 16-row tiles.  Replaces the fixed L/128 default and
 * DECODEBENCH_F4_SPLITS override of the reference harness
 * (validation/src/bench/bench_variant.cu:714-719). */
int db_f4_default_splits(int B, int Hkv, int L, int cu_count);

/* Bytes of caller-owned workspace db_f4_splitkv needs for S splits (0 when
 * S == 1): one 256-byte split-ticket line per (batch, kv-head) pair, then the
 * per-split partial records.  The workspace must be zero-filled before its
 * first use; every call leaves the tickets (the first 8 bytes of each line)
 * at zero again, so a workspace is zeroed once and then reused by any number
 * of calls (including graph replays).  Bytes 8-11 of a pair's line count the
 * in-launch merges that found the pair's splits on different XCDs and
 * recomputed them (a diagnostic; the library never resets it).  Calls that
 * overlap in time (concurrent streams, concurrently replayed graphs) need
 * workspaces of their own. */
size_t db_f4_workspace_bytes(int B, int Hq, int Hkv, int L, int D, int S);

/* F4: o[b,h,:] = softmax(scale * q[b,h,:] . K[b,h/G,:,:]^T) . V[b,h/G,:,:]
 * for G = Hq / Hkv query heads per KV head (grouped-query attention), fp32
 * softmax and accumulation, fp16 output.  The KV length is cut into S splits
 * whose partial (max, exp-sum, unnormalised output) records go to the
 * workspace and are merged by log-sum-exp: by the last split of each
 * (batch, kv-head) pair to finish, in the same launch, when B * Hkv is a
 * multiple of 8 on a device of 8 XCDs (the launch then aims every split of a
 * pair at one XCD and the merge reads the records from that XCD's L2; if
 * the workgroups of a pair report different XCDs, the merger recomputes
 * every split of the pair, so the result never depends on placement);
 * otherwise in a second launch on the same stream.  One launch when S == 1.
 * Replaces f4_partial_kernel + f4_reduce_kernel
 * (validation/src/kernels/fused/f4.cu:173-319) and the reference stages
 * scores, softmax, weighted_v (src/decodebench/demos/llama_decode.py:120-134).
 * Contract: q [B,Hq,D], K and V [B,Hkv,L,D], o [B,Hq,D] fp16; D == 128;
 * Hq % Hkv == 0 with G in {1,2,4,8}; L >= 1; 1 <= S <= 256; ws holds at least
 * db_f4_workspace_bytes(B,Hq,Hkv,L,D,S) bytes (ignored when S == 1). */
int db_f4_splitkv(const void* q, const void* k, const void* v, void* o,
                  void* ws, size_t ws_bytes, int B, int Hq, int Hkv, int L,
                  int D, int S, float scale, void* stream);

/* Size of the per-device scratch array behind db_f4_splitkv_noalloc. */
#define DB_F4_SCRATCH_BYTES ((size_t)4 << 20)

/* F4 without a workspace argument and without any allocation: the same
 * computation and kernels as db_f4_splitkv, with the split partial records
 * kept in a library-owned device array of DB_F4_SCRATCH_BYTES (4 MiB) per
 * GPU, held from the first call on that GPU until the process ends.  The
 * split merge always runs in the second launch, so nothing in the array has
 * to start at zero (its ticket lines are never read).
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under hipGraph capture that must not call hipMalloc,
 * tight serving loops, harnesses that forbid allocation).  It calls no
 * hipMalloc/hipFree; its first call on a device looks up the array's device
 * address (hipGetSymbolAddress), so make that first call outside stream
 * capture.
 * Every call on one GPU shares that GPU's array: calls that overlap in time
 * on one GPU (concurrent streams, concurrently replayed graphs) race and
 * give wrong results; serialise them or use db_f4_splitkv with one workspace
 * per stream.
 * Contract as db_f4_splitkv, plus: the S' = min(S, ceil(L / 16)) splits must
 * fit, db_f4_workspace_bytes(B,Hq,Hkv,L,D,S') <= DB_F4_SCRATCH_BYTES, else
 * DB_ERR_INVALID (checked before any HIP call).  At the library's default
 * split count (about one workgroup per CU) that holds up to G = 8. */
int db_f4_splitkv_noalloc(const void* q, const void* k, const void* v, void* o,
                          int B, int Hq, int Hkv, int L, int D, int S,
                          float scale, void* stream);

/* Capture state of `stream`: *capture_id is the id of the hipGraph capture
 * the stream is recording into (unique per capture), or 0 when it is not
 * capturing.  Host plumbing with no counterpart in the reference: the
 * Python ops use it to give every capture its own F4 workspace. */
int db_stream_capture_id(void* stream, unsigned long long* capture_id);

/* Launch an empty kernel (one workgroup of 256 threads) on `stream`: the
 * launch-overhead probe of the calibration.  Replaces null_kernel and its
 * 500-launch stream / graph timing loop (validation/src/bench/
 * calibrate.cu:42-104), whose timing the Python calibration does with HIP
 * events. */
int db_null_kernel(void* stream);

/* Read `bytes` bytes at `src` once and discard them: the single-launch
 * streaming floor of this GPU, used by the calibration (bytes one launch
 * moves vs its time) and as a read-only, known-size reference for the HBM
 * traffic counters.  Every wave reads one contiguous chunk of kb_per_wave KB
 * (4, 8 or 16) with 16-byte non-temporal loads, 1 KB per wave-wide load
 * instruction, all issued before any is used; workgroups of 4 waves, or 1
 * or 2 with db_tune("stream_waves", n).  The loaded words are folded
 * into one value per lane, stored to sink[] only if it equals `magic`
 * (choose a value that cannot occur, e.g. with src zero-filled and magic
 * non-zero), so the kernel reads `bytes` and writes nothing.
 * Contract: src and sink 16-byte aligned and non-null, bytes a positive
 * multiple of kb_per_wave * 1024, sink holding bytes / 16 unsigned words.
 * Replaces the read side of the cuBLAS bandwidth reference of the G2 gate
 * (validation/src/bench/calibrate.cu:113-230) as the measure of what one
 * launch can stream; no kernel of the reference is its counterpart. */
int db_stream_read(const void* src, size_t bytes, int kb_per_wave, unsigned magic,
                   unsigned* sink, void* stream);


#ifdef __cplusplus
}
#endif

#endif /* DECODEBENCH_HIP_H */
