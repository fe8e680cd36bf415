// flashdecode.hip -- split-KV GQA decode attention (F4) for gfx950.
//
// One launch computes o[b, h, :] = softmax(scale * q[b,h] . K[b,h/G]^T) V[b,h/G]
// for every query head h of a batch of single-token queries, G = Hq / Hkv
// query heads sharing each KV head.
//
// Decomposition
//  * A workgroup (4 waves) owns one (batch, kv-head) pair and one split of the
//    KV length; all G query heads of the pair are handled together, so every
//    K/V byte is read from HBM exactly once.
//  * Workgroups of one pair are numbered so that they all land on the same
//    XCD (workgroup i runs on XCD i % 8); their partial results then stay in
//    that XCD's L2 for the combine.
//  * A wave walks 16-row tiles.  Scores for the tile come from four
//    v_mfma_f32_16x16x32_f16: A = the 16 x 128 K tile straight from HBM
//    (16 B per lane per k-step), B = Q^T with the G query heads as columns
//    (zero-padded to 16).  The accumulator lands as S[key 4g+i][head n] in
//    lane 16g+n, register i.
//  * Online softmax runs in base 2 (scale * log2 e folded into the scores) on
//    the 4 keys each lane holds; the tile max crosses rows with two lane
//    swaps.  Probabilities reach the P.V lanes through DPP row_newbcast, since
//    lane (r, c) of the P.V layout needs keys 4r..4r+3, which live in row r.
//  * P.V is fp32 FMA on the VALU: lane (r, c) owns d = 8c..8c+7 of every head
//    for the V rows 4r..4r+3 of each tile.
//  * The 4 waves merge through LDS; with S > 1 splits each workgroup writes
//    an unnormalised partial (o, m, l) and the last workgroup of the pair to
//    finish (a device-scope counter) merges the S partials by log-sum-exp and
//    writes the fp16 output, then re-arms the counter for the next call.
//
// The merge follows the reference's two-phase split-KV form
// (validation/src/kernels/fused/f4.cu:160-319): per-split max m, exp-sum l
// and unnormalised o, merged as o = sum_s e^{m_s-M} o_s / sum_s e^{m_s-M} l_s.
#include "db_device.h"
#include "db_kernels.h"

namespace dbk {

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kD = 128;
constexpr int kTile = 16;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_huge_valf();

struct F4Args {
  const _Float16* q;   // [B, Hq, D]
  const _Float16* k;   // [B, Hkv, L, D]
  const _Float16* v;   // [B, Hkv, L, D]
  _Float16* o;         // [B, Hq, D]
  unsigned* counters;  // [B * Hkv]   zero between calls
  float* part;         // [B * Hkv, S, G * (D + 2)]
  int B, Hq, Hkv, L, S;
  int ntiles;          // ceil(L / 16)
  int tps;             // tiles per split
  int xcd_map;         // 1: all splits of a pair on one XCD
  float scale_log2;    // scale * log2(e)
};

template <int G>
__device__ __forceinline__ float bcast_head(float v, int h) {
  // h is a compile-time constant at every call site after unrolling.
  switch (h) {
    case 0: return row_bcast<0>(v);
    case 1: return row_bcast<1>(v);
    case 2: return row_bcast<2>(v);
    case 3: return row_bcast<3>(v);
    case 4: return row_bcast<4>(v);
    case 5: return row_bcast<5>(v);
    case 6: return row_bcast<6>(v);
    default: return row_bcast<7>(v);
  }
}

__device__ __forceinline__ float xor_lanes(float v, int m) {
  return __shfl_xor(v, m);
}

template <int G>
__global__ __launch_bounds__(kThreads) void f4_kernel(F4Args a) {
  static_assert(G >= 1 && G <= 8, "query heads per KV head");
  constexpr int kPart = G * (kD + 2);  // floats per partial record

  __shared__ __align__(16) float s_o[kWaves][G][kD];  // per-wave outputs
  __shared__ float s_m[kWaves][G];
  __shared__ float s_l[kWaves][G];
  __shared__ int s_last;

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int n16 = lane & 15;  // MFMA column / P.V d-chunk
  const int g4 = lane >> 4;   // MFMA k-group / P.V row group

  int pair, split;
  if (a.xcd_map) {
    const int xcd = blockIdx.x & 7, local = blockIdx.x >> 3;
    pair = xcd + 8 * (local / a.S);
    split = local % a.S;
  } else {
    pair = blockIdx.x / a.S;
    split = blockIdx.x % a.S;
  }
  const int b = pair / a.Hkv;
  const int kvh = pair % a.Hkv;
  const size_t kv_base = (size_t)pair * a.L * kD;
  const _Float16* Kp = a.k + kv_base;
  const _Float16* Vp = a.v + kv_base;
  const size_t q_base = ((size_t)b * a.Hq + (size_t)kvh * G) * kD;

  // B operand (Q^T): lane (g4, n16) holds q[head n16][d chunk g4 + 4t].
  h8 qop[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    u4 raw = {0, 0, 0, 0};
    if (n16 < G) raw = ld16(a.q + q_base + (size_t)n16 * kD + (g4 + 4 * t) * 8);
    qop[t] = __builtin_bit_cast(h8, raw);
  }

  const int t_begin = split * a.tps;
  const int t_end = min(a.ntiles, t_begin + a.tps);
  const int last_row = a.L - 1;

  float o[G][8];
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int i = 0; i < 8; ++i) o[h][i] = 0.0f;
  float m_run = kNegInf;  // per head n16 (uniform over g4)
  float l_run = 0.0f;     // partial over this lane's keys

  auto load_tile = [&](u4 (&kt)[4], u4 (&vt)[4], int tile) {
    const int row0 = tile * kTile;
    const int kr = min(row0 + n16, last_row);
#pragma unroll
    for (int t = 0; t < 4; ++t)
      kt[t] = ld_stream(Kp + (size_t)kr * kD + (g4 + 4 * t) * 8);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int vr = min(row0 + 4 * g4 + j, last_row);
      vt[j] = ld_stream(Vp + (size_t)vr * kD + n16 * 8);
    }
  };

  auto compute_tile = [&](const u4 (&kt)[4], const u4 (&vt)[4], int tile) {
    f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int t = 0; t < 4; ++t)
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(
          __builtin_bit_cast(h8, kt[t]), qop[t], acc, 0, 0, 0);

    const int key0 = tile * kTile + 4 * g4;
    float s[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      s[i] = (key0 + i < a.L) ? acc[i] * a.scale_log2 : kNegInf;
    float tmax = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
    tmax = fmaxf(tmax, xor_lanes(tmax, 16));
    tmax = fmaxf(tmax, xor_lanes(tmax, 32));
    const float m_new = fmaxf(m_run, tmax);
    const float alpha = fast_exp2(m_run - m_new);
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] = fast_exp2(s[i] - m_new);
    l_run = l_run * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
    m_run = m_new;

    // Rescale the running output only when some head's max moved.
    if (__any(alpha != 1.0f)) {
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float ah = bcast_head<G>(alpha, h);
#pragma unroll
        for (int i = 0; i < 8; ++i) o[h][i] *= ah;
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float vf[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const h2 pr = as_h2(vt[j][i]);
        vf[2 * i] = (float)pr[0];
        vf[2 * i + 1] = (float)pr[1];
      }
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float ph = bcast_head<G>(p[j], h);
#pragma unroll
        for (int i = 0; i < 8; ++i) o[h][i] = fmaf(ph, vf[i], o[h][i]);
      }
    }
  };

  // ---- stream this wave's tiles: wave w takes t_begin + w, + 4, ... -----
  {
    u4 kb[2][4], vb[2][4];
    int tile = t_begin + wave;
    if (tile < t_end) load_tile(kb[0], vb[0], tile);
    for (;;) {
      if (tile >= t_end) break;
      int nxt = tile + kWaves;
      if (nxt < t_end) load_tile(kb[1], vb[1], nxt);
      compute_tile(kb[0], vb[0], tile);
      tile = nxt;
      if (tile >= t_end) break;
      nxt = tile + kWaves;
      if (nxt < t_end) load_tile(kb[0], vb[0], nxt);
      compute_tile(kb[1], vb[1], tile);
      tile = nxt;
    }
  }

  // ---- merge the 4 waves of the workgroup through LDS -------------------
  float l_tot = l_run + xor_lanes(l_run, 16);
  l_tot += xor_lanes(l_tot, 32);
  if (lane < G) {
    s_m[wave][lane] = m_run;
    s_l[wave][lane] = l_tot;
  }
  // Sum the four row groups (g4) of the P.V layout: same d, disjoint keys.
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      o[h][i] += xor_lanes(o[h][i], 16);
      o[h][i] += xor_lanes(o[h][i], 32);
    }
  if (g4 == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float* dst = &s_o[wave][h][n16 * 8];
      *reinterpret_cast<f4*>(dst) = f4{o[h][0], o[h][1], o[h][2], o[h][3]};
      *reinterpret_cast<f4*>(dst + 4) = f4{o[h][4], o[h][5], o[h][6], o[h][7]};
    }
  }
  __syncthreads();

  const size_t rec = ((size_t)pair * a.S + split) * kPart;
  for (int idx = threadIdx.x; idx < G * kD; idx += kThreads) {
    const int h = idx / kD, d = idx % kD;
    float M = kNegInf;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, s_m[w][h]);
    float ow = 0.0f, lw = 0.0f;
    if (M != kNegInf) {
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const float e = fast_exp2(s_m[w][h] - M);
        ow += e * s_o[w][h][d];
        lw += e * s_l[w][h];
      }
    }
    if (a.S == 1) {
      a.o[q_base + (size_t)h * kD + d] = to_h(ow / lw);
    } else {
      a.part[rec + idx] = ow;
      if (d == 0) {
        a.part[rec + G * kD + h] = M;
        a.part[rec + G * kD + G + h] = lw;
      }
    }
  }
  if (a.S == 1) return;

  // ---- split combine: the last workgroup of the pair merges S partials ---
  __threadfence();  // publish this thread's partial stores device-wide
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned prev = __hip_atomic_fetch_add(
        &a.counters[pair], 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    s_last = (prev == (unsigned)(a.S - 1));
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();  // acquire side: see every other workgroup's partials

  // Reuse s_o as scratch: weights w[s][h] = e^{m_s - M_h} / L_h.
  float* s_w = &s_o[0][0][0];
  constexpr int kScratch = kWaves * G * kD;
  const float* base = a.part + (size_t)pair * a.S * kPart;
  const int sg = a.S * G;  // <= kScratch / 2 (checked on the host)
  for (int i = threadIdx.x; i < sg; i += kThreads) {
    const int s = i / G, h = i % G;
    s_w[i] = base[(size_t)s * kPart + G * kD + h];              // m
    s_w[sg + i] = base[(size_t)s * kPart + G * kD + G + h];     // l
  }
  __syncthreads();
  if (threadIdx.x < G) {
    const int h = threadIdx.x;
    float M = kNegInf;
    for (int s = 0; s < a.S; ++s) M = fmaxf(M, s_w[s * G + h]);
    float Lsum = 0.0f;
    for (int s = 0; s < a.S; ++s) {
      const float ms = s_w[s * G + h];
      if (ms != kNegInf) Lsum += fast_exp2(ms - M) * s_w[sg + s * G + h];
    }
    s_m[0][h] = M;
    s_l[0][h] = 1.0f / Lsum;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < sg; i += kThreads) {
    const int h = i % G;
    const float ms = s_w[i];
    s_w[i] = (ms == kNegInf) ? 0.0f : fast_exp2(ms - s_m[0][h]) * s_l[0][h];
  }
  __syncthreads();
  static_assert(kScratch >= 2, "scratch");
  for (int idx = threadIdx.x; idx < G * kD; idx += kThreads) {
    const int h = idx / kD;
    float acc = 0.0f;
    int s = 0;
    for (; s + 8 <= a.S; s += 8) {
      float vals[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) vals[u] = base[(size_t)(s + u) * kPart + idx];
#pragma unroll
      for (int u = 0; u < 8; ++u) acc = fmaf(s_w[(s + u) * G + h], vals[u], acc);
    }
    for (; s < a.S; ++s) acc = fmaf(s_w[s * G + h], base[(size_t)s * kPart + idx], acc);
    a.o[q_base + idx] = to_h(acc);
  }
  if (threadIdx.x == 0)
    __hip_atomic_store(&a.counters[pair], 0u, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

using F4Fn = void (*)(F4Args);

F4Fn pick_f4(int G) {
  switch (G) {
    case 1: return f4_kernel<1>;
    case 2: return f4_kernel<2>;
    case 4: return f4_kernel<4>;
    default: return f4_kernel<8>;
  }
}

constexpr size_t kCounterBytes(int pairs) {
  return (((size_t)pairs * sizeof(unsigned)) + 255) / 256 * 256;
}

}  // namespace

// Largest split count the in-kernel combine supports for group size G: the
// S x G (m, l) pairs must fit in the workgroup's LDS scratch.
int f4_max_splits(int G) { return (kWaves * G * kD) / (2 * G); }

size_t f4_workspace_bytes(int B, int Hq, int Hkv, int S, int D) {
  const int G = Hq / Hkv;
  const int pairs = B * Hkv;
  return kCounterBytes(pairs) +
         (size_t)pairs * S * G * (D + 2) * sizeof(float);
}

int f4_choose_splits(int B, int Hkv, int L, int cu_count) {
  const Tuning& t = tuning();
  const int ntiles = (L + kTile - 1) / kTile;
  const int pairs = B * Hkv;
  const int target = cu_count * t.f4_blocks_per_cu;
  int S = (target + pairs - 1) / pairs;
  const int max_by_tiles = ntiles / (t.f4_min_tiles > 0 ? t.f4_min_tiles : 1);
  S = min(S, max(1, max_by_tiles));
  S = min(S, 256);
  return max(S, 1);
}

hipError_t launch_f4(const void* q, const void* k, const void* v, void* o,
                     void* ws, int B, int Hq, int Hkv, int L, int D, int S,
                     float scale, hipStream_t stream) {
  (void)D;
  const int G = Hq / Hkv;
  const int pairs = B * Hkv;
  F4Args a;
  a.q = static_cast<const _Float16*>(q);
  a.k = static_cast<const _Float16*>(k);
  a.v = static_cast<const _Float16*>(v);
  a.o = static_cast<_Float16*>(o);
  a.counters = static_cast<unsigned*>(ws);
  a.part = ws ? reinterpret_cast<float*>(static_cast<char*>(ws) +
                                         kCounterBytes(pairs))
              : nullptr;
  a.B = B;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.L = L;
  a.ntiles = (L + kTile - 1) / kTile;
  // Never more splits than tiles: every split then owns at least one tile.
  a.S = min(S, a.ntiles);
  a.tps = (a.ntiles + a.S - 1) / a.S;
  a.S = (a.ntiles + a.tps - 1) / a.tps;
  a.xcd_map = (pairs % 8 == 0) ? 1 : 0;
  a.scale_log2 = scale * kLog2e;
  hipLaunchKernelGGL(pick_f4(G), dim3(pairs * a.S), dim3(kThreads), 0, stream, a);
  return hipGetLastError();
}

}  // namespace dbk
