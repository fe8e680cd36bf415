// ref_shim.cpp -- C-linkage entry points onto the reference's own CPU
// reference (TEST INFRASTRUCTURE, built only into oracle/_ref/).
//
// Compiled together with the reference source file
// validation/src/reference/cpu_reference.cpp, read in place from the
// reference checkout; nothing of the reference is copied.  The wrappers only
// forward arguments so ctypes can call the reference functions declared in
// validation/src/reference/cpu_reference.h:8-30.
#include "cpu_reference.h"

extern "C" {

void ref_rmsnorm(const float* x, const float* gamma, float* out, int d, float eps) {
  rmsnorm_ref(x, gamma, out, d, eps);
}

void ref_gemv(const float* W, const float* x, float* out, int d_out, int d_in) {
  gemv_ref(W, x, out, d_out, d_in);
}

float ref_silu(float x) { return silu_ref(x); }

void ref_swiglu(const float* g, const float* u, float* out, int n) {
  swiglu_ref(g, u, out, n);
}

void ref_softmax(const float* scores, float* probs, int n_heads, int seq_len) {
  softmax_ref(scores, probs, n_heads, seq_len);
}

void ref_attention(const float* q, const float* K, const float* V, float* out,
                   int n_heads, int seq_len, int head_dim) {
  attention_ref(q, K, V, out, n_heads, seq_len, head_dim);
}

}  // extern "C"
