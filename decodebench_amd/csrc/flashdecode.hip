// flashdecode.hip -- split-KV GQA decode attention (F4) for gfx950.
//
// One launch computes o[b, h, :] = softmax(scale * q[b,h] . K[b,h/G]^T) V[b,h/G]
// for every query head h of a batch of single-token queries, G = Hq / Hkv
// query heads sharing each KV head.
//
// Decomposition
//  * A workgroup (NW waves) owns one (batch, kv-head) pair and one split of
//    the KV length; all G query heads of the pair are handled together, so
//    every K/V byte is read from HBM exactly once.  The host sizes the split
//    count so the grid is about one workgroup per CU.
//  * Workgroups of one pair are numbered so that they all land on the same
//    XCD (workgroups i and i + 8 run on one XCD: the dispatcher deals them
//    out round-robin over the 8 XCDs).
//  * A wave walks 16-row tiles of its split (tile w, w + NW, ...) with two
//    register sets of one tile each.  With DEPTH 2 one or two tiles (8-16
//    KB) of K and V are in flight per wave; with DEPTH 1 a wave requests its
//    next tile as soon as the oldest one has arrived and consumes the oldest
//    while the next is in flight.
//  * Scores for a tile come from four v_mfma_f32_16x16x32_f16: A = the
//    K tile straight from HBM, B = Q^T with the G query heads as columns.
//    The operands split each 128-byte line into its even and odd 16-byte
//    chunks (even A rows / B columns 0-7 take the even ones), so every K
//    load instruction reads 8 keys x one whole line; one DPP row rotation
//    folds the two halves of each score, which land in the same 16-lane
//    row of the accumulator.
//  * Online softmax runs in base 2 (scale * log2 e folded into the scores) on
//    the 4 keys each lane holds; the tile max crosses rows with two lane
//    swaps.  The fp16 probabilities are already the B operand (P^T) of the
//    P.V product in the score accumulator's layout.
//  * P.V is eight v_mfma_f32_16x16x16_f16 per tile (O^T = V^T P^T, one per 16
//    dims of D).  Their A operand (V^T) comes from the wave's copy of the V
//    tile in LDS through the gfx950 transposing read ds_read_b64_tr_b16, so
//    the VALU does no per-key multiply-adds and the outputs need no
//    cross-lane reduction at the end.
//  * The waves merge through LDS.  With S = 1 the workgroup writes the fp16
//    output.  With S > 1 splits each workgroup writes an unnormalised partial
//    record (o, and the pair (m, l) per head), and the S records of every
//    (pair, head) are merged by log-sum-exp in one of two ways:
//      - in the same launch (the default where every split of a pair is
//        aimed at one XCD): each workgroup waits for its record stores to
//        land in its XCD's L2, takes a ticket from its pair's line in the
//        workspace with one atomic add that also reports its XCD, and the
//        workgroup that draws the last ticket reads every record from that
//        L2 (device-scope loads, which skip the CU's L1), merges, writes the
//        output and resets the ticket.  If the tickets show a split that ran
//        on another XCD, whose record its L2 cannot see, the merger
//        recomputes every split of the pair first, so placement changes
//        only the speed.  Measured on MI355X at batch 1: 9.75 against
//        10.05 us for the second launch at L = 8192, 23.6 against 23.9 us at
//        L = 32768.  The first version took its tickets from one shared
//        line (1.7 us lost to contention) with write-through stores and
//        coherent loads, and measured 2 us slower than the second launch;
//      - in a second, small launch (f4_combine), ordered by the kernel
//        boundary (when a pair's splits are not aimed at one XCD, and for
//        db_f4_splitkv_noalloc, whose scratch tickets are never read).
//
// The merge follows the reference's two-phase split-KV form
// (validation/src/kernels/fused/f4.cu:160-319): per-split max m, exp-sum l
// and unnormalised o, merged as o = sum_s e^{m_s-M} o_s / sum_s e^{m_s-M} l_s.
#include <atomic>
#include <mutex>

#include "db_device.h"
#include "db_kernels.h"

namespace dbk {

namespace {

constexpr int kD = 128;
constexpr int kTile = 16;
constexpr int kMergeChunk = 8;
// Row stride (halves) of a V tile in LDS: 128 + 16 padding keeps the four
// rows one transposed read touches in different banks.
constexpr int kVStride = 144;

typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef short s4 __attribute__((ext_vector_type(4)));
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_huge_valf();

struct F4Args {
  const _Float16* q;   // [B, Hq, D]
  const _Float16* k;   // [B, Hkv, L, D]
  const _Float16* v;   // [B, Hkv, L, D]
  _Float16* o;         // [B, Hq, D]
  unsigned* ticket;    // [B * Hkv][kTicketWords] split ticket line per pair
                       // (zero between calls)
  float2* ml;          // [B * Hkv, G, S]    (max, exp-sum) per split, base 2
  float* opart;        // [B * Hkv, S, G, D] unnormalised split outputs
  int fused_merge;     // 1: the last split of a pair merges in this launch
  int B, Hq, Hkv, L, S;
  int ntiles;          // ceil(L / 16)
  int tps;             // tiles per split
  int xcd_map;         // 1: all splits of a pair on one XCD
  int misplace_every;  // test hook: split s reports a foreign XCD if s % k == k - 1 (0: off)
  float scale_log2;    // scale * log2(e)
};

__device__ __forceinline__ float xor_lanes(float v, int m) {
  return __shfl_xor(v, m);
}

// exp2(m - M) with exp2(-inf - x) = 0 also when M is -inf.
__device__ __forceinline__ float weight2(float m, float M) {
  return m == kNegInf ? 0.0f : fast_exp2(m - M);
}

// s_waitcnt vmcnt(0) with the other counters left alone (gfx9 encoding).
constexpr int kVmcnt0 = 0x0F70;
// Cache-policy bit sc1 (device scope) of a buffer load: the load always
// misses the CU's vector L1 and reads the XCD's L2, where the other CUs'
// record stores have landed (a workgroup-scope load may hit a stale L1
// line).  On MI355X it costs what a plain L2 hit does (165 vs 165 ns).
constexpr int kSc1 = 16;
// s_getreg_b32 operand of HW_REG_XCC_ID bits [3:0]: the XCD a wave runs on.
constexpr int kXccIdReg = (3 << 11) | 20;
// One 256-byte line per (batch, kv-head) pair, its first 8 bytes the split
// ticket: arrivals in bits 0-15, the sum of the arrivals' XCC ids in bits
// 16-31 and the sum of their squares in bits 32-47; word kRecomputeWord
// counts the merges that had to recompute the pair.  A line of its own per
// pair: with the 8 tickets of a batch-1 call in one line, the 256 atomics of
// a call contended for it and the in-launch merge measured 1.7 us slower
// (12.16 vs 10.42 us at L = 8192).
constexpr int kTicketWords = 64;
constexpr int kRecomputeWord = 2;

template <int G, int NW, bool LINE, int DEPTH>
__global__ __launch_bounds__(NW * kWave) void f4_kernel(F4Args a) {
  static_assert(G >= 1 && G <= 8, "query heads per KV head");
  constexpr int kThreads = NW * kWave;

  // Per-wave V tile; after its last tile a wave leaves its G x D outputs in
  // the same bytes for the workgroup merge.
  __shared__ __align__(16) _Float16 s_v[NW][kTile][kVStride];
  static_assert(sizeof(float) * G * kD <= sizeof(s_v[0]), "wave outputs fit a V tile");
  auto s_o = [&](int w, int h) { return reinterpret_cast<float*>(&s_v[w][0][0]) + h * kD; };
  // Per head, the running max and exp-sum of every wave: a head's NW values
  // are contiguous, so the workgroup merge reads them in 16-byte loads.
  __shared__ __align__(16) float s_m[G][NW];
  __shared__ __align__(16) float s_l[G][NW];

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // wave-uniform
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

  // Score operands: A = K (keys as rows), B = Q^T (heads as columns); a
  // 16-byte "chunk" c of a K or q row is its halves 8c..8c+7.  Two layouts:
  //
  //  LINE (whole-line K loads): one K load instruction reads 8 keys x one
  //   128-byte line (line t = chunks 8t..8t+7).  A (key group kg = keys
  //   8kg..8kg+7): lane (g4, n16), the A row m = n16, holds K[key 8kg +
  //   (n16 >> 1)][chunk 8t + 2 g4 + (n16 & 1)]: row 2j carries the even
  //   chunks of key j, row 2j + 1 the odd ones.  B: lane (g4, n16), column
  //   n16, holds q[head n16 & 7][chunk 8t + 2 g4 + (n16 >> 3)] (zero for
  //   heads >= G): columns 0-7 pair with the even chunks, 8-15 with the odd
  //   ones.  Over the two lines the score of key j and head h < 8 is
  //   D[2j][h] + D[2j + 1][h + 8]; both terms sit in the same 16-lane row of
  //   the accumulator (registers 2r and 2r + 1, lanes h and h + 8), so one
  //   DPP row rotation folds them; the other accumulator entries are
  //   discarded.
  //  Plain: one K load instruction reads 16 keys x 64 bytes.  A: lane
  //   (g4, n16) holds K[key n16][chunk g4 + 4t]; B: q[head n16][chunk
  //   g4 + 4t] (zero for heads >= G); the accumulator is the score matrix.
  //
  // Measured on MI355X (32 q / 8 kv heads, graph back-to-back): whole lines
  // are faster at batch 1 (L = 8192 10.75 -> 10.53 us, L = 32768 24.43 ->
  // 24.21 us) and wherever a wave walks 1-2 tiles (batch 4 and 8 at
  // L = 1024: 0.2-0.4 us), and slower once larger batches stream long
  // splits (batch 4 / 8 at L = 8192: +0.2 / +1.0 us, at L = 32768: +3 us),
  // so the launcher picks by tiles per wave and pair count.
  // q is read through a buffer resource that covers the pair's G heads
  // only: lanes of heads >= G get zeros without a branch (with the load
  // under a branch the compiler copied its result inside the branch and
  // waited for it there, before the first K/V tile was requested).
  h8 qop[LINE ? 2 : 4];
  const __amdgpu_buffer_rsrc_t r_q = make_rsrc(a.q + q_base, G * kD * (int)sizeof(_Float16));
#pragma unroll
  for (int t = 0; t < (LINE ? 2 : 4); ++t) {
    const int head = LINE ? (n16 & 7) : n16;
    const int chunk = LINE ? 8 * t + 2 * g4 + (n16 >> 3) : g4 + 4 * t;
    qop[t] = __builtin_bit_cast(
        h8, __builtin_amdgcn_raw_buffer_load_b128(r_q, (head * kD + chunk * 8) * 2, 0, 0));
  }
  // Tile key held in slot j (j = 0..3) of lane group g4 after the scores:
  // 4 g4 + j for the plain layout; key_of(j) = 2 g4 + (j & 1) + 8 (j >> 1)
  // after the LINE fold.  That is also the key order of the P^T operand
  // below, so LDS row 4 g4 + j of the V tile must hold that key.  V is
  // always loaded four whole consecutive rows (1 KB) per instruction --
  // vt[j] of lane group g4 is key 4 g4 + j -- and for LINE the permutation
  // is applied to the LDS row it is written to: key k goes to row
  // v_row(k) = 4 ((k & 7) >> 1) + (k & 1) + 2 (k >> 3).
  auto key_of = [&](int j) { return LINE ? 2 * g4 + (j & 1) + 8 * (j >> 1) : 4 * g4 + j; };
  auto v_row = [](int k) { return LINE ? 4 * ((k & 7) >> 1) + (k & 1) + 2 * (k >> 3) : k; };
  // LINE: lanes n16 >= 8 fold entries that are not scores; their scale is
  // zero, which keeps them finite and equal to zero (a multiply, not a
  // select, so the DPP before it always runs with every lane enabled).
  const float lane_scale = (!LINE || n16 < 8) ? a.scale_log2 : 0.0f;

  // ---- one split: stream its tiles, merge the waves, write its record ----
  // Called for the workgroup's own split, and by a merging workgroup that
  // recomputes every split of its pair.
  auto run_split = [&](int split) {
    const int t_begin = split * a.tps;
    const int t_end = min(a.ntiles, t_begin + a.tps);
    const int first = t_begin + wave;
    const int nt = first < t_end ? (t_end - first + NW - 1) / NW : 0;
    // Global index of this wave's k-th tile.
    auto tile_of = [&](int k) { return first + NW * k; };
    const int last_row = a.L - 1;

    // O^T accumulators: lane (g4, n16) holds O[head n16][16 b + 4 g4 + i].
    f4 o[kD / 16];
#pragma unroll
    for (int b = 0; b < kD / 16; ++b) o[b] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    float m_run = kNegInf;  // per head n16 (uniform over g4)
    float l_run = 0.0f;     // partial over this lane's keys

    // LINE: kt[2 kg + t] = key group kg, line t; plain: kt[t] = chunks
    // g4 + 4t of key n16.  vt[j]: V row 4 g4 + j of the tile.
    auto load_tile = [&](u4 (&kt)[4], u4 (&vt)[4], int tile) {
      const int row0 = tile * kTile;
      if constexpr (LINE) {
#pragma unroll
        for (int kg = 0; kg < 2; ++kg) {
          const int kr = min(row0 + 8 * kg + (n16 >> 1), last_row);
#pragma unroll
          for (int t = 0; t < 2; ++t)
            kt[2 * kg + t] =
                ld_stream(Kp + (size_t)kr * kD + (8 * t + 2 * g4 + (n16 & 1)) * 8);
        }
      } else {
        const int kr = min(row0 + n16, last_row);
#pragma unroll
        for (int t = 0; t < 4; ++t) kt[t] = ld_stream(Kp + (size_t)kr * kD + (g4 + 4 * t) * 8);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int vr = min(row0 + 4 * g4 + j, last_row);
        vt[j] = ld_stream(Vp + (size_t)vr * kD + n16 * 8);
      }
    };

    // V^T operands come from a per-wave row-major copy of the V tile in LDS
    // (rows in the key order above), read back with ds_read_b64_tr_b16: lane
    // 16g + 4r + q supplies the address of LDS row 4g + r, column d0 + 4q, and
    // receives rows 4g .. 4g+3 of column d0 + (lane & 15) -- tile keys
    // key_of(0..3) of lane group g -- the A-operand layout of
    // v_mfma_f32_16x16x16_f16 for O^T = V^T P^T.
    _Float16* vbuf = &s_v[wave][0][0];
    auto compute_tile = [&](const u4 (&kt)[4], const u4 (&vt)[4], int tile) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        *reinterpret_cast<u4*>(vbuf + v_row(4 * g4 + j) * kVStride + 8 * n16) = vt[j];
      // The transposed reads below take rows other lanes wrote here; they stay
      // after these writes because the compiler cannot prove the lane-derived
      // addresses disjoint (so keeps program order) and a wave's LDS accesses
      // execute in order.  (wave_lds_order() here measured 0.13 us slower at
      // batch 1, L = 8192: its fences also pin the global loads.)

      // s[j]: scaled score of tile key key_of(j) (-inf past L).
      float s[4];
      if constexpr (LINE) {
        f4 d[2];
#pragma unroll
        for (int kg = 0; kg < 2; ++kg) {
          d[kg] = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int t = 0; t < 2; ++t)
            d[kg] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                __builtin_bit_cast(h8, kt[2 * kg + t]), qop[t], d[kg], 0, 0, 0);
        }
        // key_of(j) = 8 kg + 2 g4 + r with kg = j >> 1, r = j & 1
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const f4& dk = d[j >> 1];
          const int r = j & 1;
          s[j] = (dk[2 * r] + dpp<kRowRor8>(dk[2 * r + 1])) * lane_scale;
        }
      } else {
        f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int t = 0; t < 4; ++t)
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, kt[t]), qop[t],
                                                       acc, 0, 0, 0);
#pragma unroll
        for (int j = 0; j < 4; ++j) s[j] = acc[j] * lane_scale;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (tile * kTile + key_of(j) >= a.L) s[j] = kNegInf;
      float tmax = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
      tmax = fmaxf(tmax, xor_lanes(tmax, 16));
      tmax = fmaxf(tmax, xor_lanes(tmax, 32));
      const float m_new = fmaxf(m_run, tmax);
      const float alpha = fast_exp2(m_run - m_new);
      // P^T operand: lane (g4, n16) holds P[key key_of(j)][head n16] in slot
      // j, the order the V tile was written in.  p is rounded to fp16 for the
      // product (as the reference stage rounds p before P.V) and the exp-sum
      // adds the rounded values, so numerator and denominator agree.
      h4 pb;
#pragma unroll
      for (int i = 0; i < 4; ++i) pb[i] = (_Float16)fast_exp2(s[i] - m_new);
      l_run = l_run * alpha + (((float)pb[0] + (float)pb[1]) + ((float)pb[2] + (float)pb[3]));
      m_run = m_new;

      // Rescale the running output only when some head's max moved; alpha of
      // head n16 lives in the lanes that hold that head's outputs.
      if (__any(alpha != 1.0f)) {
#pragma unroll
        for (int b = 0; b < kD / 16; ++b) o[b] *= alpha;
      }
#pragma unroll
      for (int b = 0; b < kD / 16; ++b) {
        const h4 va = __builtin_bit_cast(
            h4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (__attribute__((address_space(3))) s4*)(
                        vbuf + (4 * g4 + (n16 >> 2)) * kVStride + 16 * b + 4 * (n16 & 3))));
        o[b] = __builtin_amdgcn_mfma_f32_16x16x16f16(va, pb, o[b], 0, 0, 0);
      }
    };

    // ---- stream this wave's tiles ------------------------------------------
    // Two register sets of one tile each: an iteration loads set B, consumes
    // set A, reloads A and consumes B, so one or two tiles are in flight and
    // every wait is for one tile.  (Set B is loaded and consumed in the same
    // iteration, which keeps the compiler from draining all loads at the loop
    // header.)  Measured on MI355X against sets of two tiles (two to four in
    // flight): 24.5 vs 25.0 us at batch 1, L = 32768, and 1-1.5% faster at
    // batch 4 and 8; deeper queues per wave only spread the tiles' arrival
    // times and lengthen the tail of the slowest wave.  DEPTH 1 (a tuning
    // option for the 8-wave whole-line kernel) waits for the oldest tile
    // before requesting the next, so each wave keeps one tile in flight while
    // it computes.
    // Timestamps of an instrumented copy there show the waves of one
    // workgroup finishing up to 4-6 us apart; handing tiles out from an LDS
    // counter instead of the fixed w, w + NW, ... walk (so that faster waves
    // take more) measured slower at every shape (0.2-0.9 us), as did
    // interleaving the splits' tiles (split s taking tiles s, s + S, ...).
    if (nt > 0) {
      u4 ka[4], va[4], kb[4], vb[4];
      load_tile(ka, va, tile_of(0));
      if constexpr (DEPTH == 1) {
        // One tile in flight: wait for the oldest tile, request the next one,
        // then consume the oldest.
        for (int k = 0; k < nt; k += 2) {
          __builtin_amdgcn_s_waitcnt(kVmcnt0);
          if (k + 1 < nt) load_tile(kb, vb, tile_of(k + 1));
          __builtin_amdgcn_sched_barrier(0);
          compute_tile(ka, va, tile_of(k));
          if (k + 1 >= nt) break;
          __builtin_amdgcn_s_waitcnt(kVmcnt0);
          if (k + 2 < nt) load_tile(ka, va, tile_of(k + 2));
          __builtin_amdgcn_sched_barrier(0);
          compute_tile(kb, vb, tile_of(k + 1));
        }
      } else {
        int k = 0;
        for (; k + 3 <= nt; k += 2) {
          load_tile(kb, vb, tile_of(k + 1));
          compute_tile(ka, va, tile_of(k));
          load_tile(ka, va, tile_of(k + 2));
          compute_tile(kb, vb, tile_of(k + 1));
        }
        // One or two tiles remain; set A holds tile k.  Each case is
        // straight-line code: after a load under a branch the compiler merged
        // the two paths and had tile k wait for tile k + 1's loads as well
        // (vmcnt(7..0) where vmcnt(15..8) would do, read in the ISA), so at
        // two tiles per wave nothing overlapped the second tile's arrival
        // (batch 1, L = 8192: 10.40 -> 9.98 us; batch 8, L = 1024 10.38 ->
        // 10.06 us).
        if (k + 1 < nt) {
          load_tile(kb, vb, tile_of(k + 1));
          // Request all of tile k + 1 before waiting for tile k: left to
          // itself the compiler issued two of its eight loads, then waited
          // for tile k's first load (about 2 us under a full-chip stream)
          // before requesting the other six.
          __builtin_amdgcn_sched_barrier(0);
          compute_tile(ka, va, tile_of(k));
          compute_tile(kb, vb, tile_of(k + 1));
        } else {
          compute_tile(ka, va, tile_of(k));
        }
      }
    }

    // ---- merge the waves of the workgroup through LDS ---------------------
    float l_tot = l_run + xor_lanes(l_run, 16);
    l_tot += xor_lanes(l_tot, 32);
    if (lane < G) {
      s_m[lane][wave] = m_run;
      s_l[lane][wave] = l_tot;
    }
    if (n16 < G) {
#pragma unroll
      for (int b = 0; b < kD / 16; ++b)
        *reinterpret_cast<f4*>(s_o(wave, n16) + 16 * b + 4 * g4) = o[b];
    }
    __syncthreads();

    // With S > 1 a split's partial record is its running max m_s and exp-sum
    // l_s (base 2) and its unnormalised output o_s, all fp32, written with
    // plain stores: they land in this XCD's L2, where the in-launch merge
    // reads them, and the kernel boundary makes them visible to the second
    // launch otherwise.  (fp16 records of o_s / l_s, half the bytes, measured
    // 0.45 us slower per call at batch 1, L = 8192 and 32768, with the merge
    // in a second launch.)
    // One thread per float4 slot of the G x D outputs: 16-byte LDS reads and
    // one 16-byte store per thread, a quarter of the instructions of one
    // thread per output (bitwise the same results; measured on MI355X,
    // interleaved, us: batch 1 L = 1024 5.55 -> 5.47, L = 8192 9.58 -> 9.45,
    // L = 32768 23.30 -> 23.22, batch 4 L = 8192 22.87 -> 22.80, batch 8
    // L = 1024 8.91 -> 8.82).
    for (int idx = threadIdx.x; idx < G * kD / 4; idx += kThreads) {
      const int h = idx / (kD / 4), d4 = idx % (kD / 4);
      float M = kNegInf;
#pragma unroll
      for (int w = 0; w < NW; ++w) M = fmaxf(M, s_m[h][w]);
      f4 ow = {0.0f, 0.0f, 0.0f, 0.0f};
      float lw = 0.0f;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const float e = weight2(s_m[h][w], M);
        ow += e * *reinterpret_cast<const f4*>(s_o(w, h) + 4 * d4);
        lw += e * s_l[h][w];
      }
      if (a.S == 1) {
        uint2 packed;
        packed.x = pack_h2(ow[0] / lw, ow[1] / lw);
        packed.y = pack_h2(ow[2] / lw, ow[3] / lw);
        *reinterpret_cast<uint2*>(a.o + q_base + (size_t)h * kD + (size_t)d4 * 4) = packed;
      } else {
        *reinterpret_cast<f4*>(a.opart + (((size_t)pair * a.S + split) * G + h) * kD +
                               (size_t)d4 * 4) = ow;
        if (d4 == 0) a.ml[((size_t)pair * G + h) * a.S + split] = make_float2(M, lw);
      }
    }
  };  // run_split

  // ---- in-launch merge: the last split of the pair to arrive merges ------
  // The merger reads the split records from its own XCD's L2, so every
  // split must have been computed on that XCD.  The numbering aims all
  // splits of a pair at one XCD (workgroup i and i + 8 share one: the
  // dispatcher deals workgroups out round-robin over the 8 XCDs, starting
  // where the previous launch stopped), and each workgroup reports where it
  // really ran: its arrival adds (1, x, x^2) for its hardware XCC id x to
  // the pair's 64-bit ticket.  The last of S arrivals, on XCD m, finds
  // sum x = S m and sum x^2 = S m^2 exactly when every x equals m
  // (Cauchy-Schwarz holds with equality only for equal terms).  Otherwise
  // it recomputes every split of the pair itself before merging, so results
  // never depend on where a workgroup runs; only speed does.
  // (Read after the split's stream: any scalar work placed before it delays
  // the first tile loads.)
  run_split(split);
  if (a.S == 1 || !a.fused_merge) return;
  unsigned xid = __builtin_amdgcn_s_getreg(kXccIdReg);
  if (a.misplace_every > 0 && split % a.misplace_every == a.misplace_every - 1)
    xid ^= 8u | (unsigned)(split & 7);  // test hook: report a foreign XCD
  __shared__ unsigned long long s_tk;
  unsigned long long* const tk =
      reinterpret_cast<unsigned long long*>(a.ticket + (size_t)pair * kTicketWords);

  // Release: every thread's record stores have completed (reached this XCD's
  // L2) before the ticket is taken.
  __builtin_amdgcn_s_waitcnt(kVmcnt0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned long long inc =
        1ull | ((unsigned long long)xid << 16) | ((unsigned long long)(xid * xid) << 32);
    s_tk = __hip_atomic_fetch_add(tk, inc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + inc;
  }
  __syncthreads();
  {
    const unsigned long long t = s_tk;
    const unsigned S = (unsigned)a.S;
    if ((unsigned)(t & 0xFFFFu) != S) return;
    if ((unsigned)((t >> 16) & 0xFFFFu) != S * xid ||
        (unsigned)((t >> 32) & 0xFFFFu) != S * xid * xid) {
      // Some split ran on another XCD: recompute every split of the pair
      // here (a cold path; the fast path above stays straight-line code).
      // Count the pair's recomputes (never reset here): a diagnostic that
      // shows whether calls stay on the fast path.
      if (threadIdx.x == 0)
        __hip_atomic_fetch_add(a.ticket + (size_t)pair * kTicketWords + kRecomputeWord, 1u,
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      for (int s = 0; s < a.S; ++s) {
        __syncthreads();  // the previous record loop's LDS reads are done
        run_split(s);
      }
      __builtin_amdgcn_s_waitcnt(kVmcnt0);  // the recomputed records are in L2
      __syncthreads();
    }
  }

  // ---- merge the S records of the pair -----------------------------------
  // At most 8 splits: thread `slot` merges every split of float4 slot `slot`
  // of the G x D outputs itself (all loads in flight at once) and writes
  // it, with no LDS and no barrier.  Measured on MI355X against the grouped
  // merge below (interleaved runs, us): batch 1 L = 1024 (8 splits) 6.60 ->
  // 5.88, batch 4 L = 8192 23.9 -> 23.1, batch 8 L = 1024 9.9 -> 9.2, batch 4
  // L = 32768 78.2 -> 77.5.  (Two waves merge here, and the shuffled (m, l)
  // loads of the grouped merge below only add latency: +0.05-0.07 us at
  // batch 1 L = 1024, batch 4 L = 8192 and batch 8 L = 1024.)
  if (a.S <= kMergeChunk) {
    constexpr int kSlots = G * kD / 4;
    static_assert(kSlots <= kThreads, "one thread per slot");
    const __amdgpu_buffer_rsrc_t r_ml =
        make_rsrc(a.ml + (size_t)pair * G * a.S, G * a.S * (int)sizeof(float2));
    const __amdgpu_buffer_rsrc_t r_op =
        make_rsrc(a.opart + (size_t)pair * a.S * G * kD, a.S * G * kD * (int)sizeof(float));
    const int slot = threadIdx.x;
    if (slot < kSlots) {
      const int h = slot / (kD / 4), d4 = slot % (kD / 4);
      f4 ov[kMergeChunk];
      float2 mv[kMergeChunk];
#pragma unroll
      for (int j = 0; j < kMergeChunk; ++j) {
        // splits past S read zero bytes (out of the buffers' range)
        ov[j] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(
                                           r_op, ((j * G + h) * kD + 4 * d4) * 4, 0, kSc1));
        mv[j] = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(
                                               r_ml, (h * a.S + j) * 8, 0, kSc1));
        if (j >= a.S) mv[j].x = kNegInf;
      }
      float M = kNegInf;
#pragma unroll
      for (int j = 0; j < kMergeChunk; ++j) M = fmaxf(M, mv[j].x);
      float Ls = 0.0f;
      f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int j = 0; j < kMergeChunk; ++j) {
        const float w = weight2(mv[j].x, M);
        Ls = fmaf(w, mv[j].y, Ls);
        acc += w * ov[j];
      }
      const float inv = 1.0f / Ls;
      uint2 packed;
      packed.x = pack_h2(acc[0] * inv, acc[1] * inv);
      packed.y = pack_h2(acc[2] * inv, acc[3] * inv);
      *reinterpret_cast<uint2*>(a.o + q_base + (size_t)h * kD + (size_t)d4 * 4) = packed;
    }
  } else
  // More splits: thread (grp, slot) owns float4 slot `slot` of the G x D outputs and the
  // splits grp, grp + kGrp, ...; the loads of a chunk of 8 splits are issued
  // at once (16-byte buffer loads that miss the vector L1 and hit the XCD's
  // L2), so S <= 8 kGrp costs one round trip; the split groups then meet in
  // LDS.  The chunk's (m, l) pairs come in one 8-byte load per lane (lane j
  // of a half-wave, whose lanes share one head and group, loads split j) and
  // reach the other lanes by shuffles.  Here the merging CU's load
  // instructions, not its bytes, set the pace: eight (m, l) loads per thread
  // beside the eight record loads measured 0.2 us slower (batch 1, L = 8192
  // 9.67 against 9.48 us, L = 32768 23.4 against 23.2), while records of
  // half the bytes in as many instructions had gained nothing.  (Split
  // groups as adjacent lanes merged by lane exchanges instead, with four
  // splits per load instruction, measured 1 us slower at batch 1, L = 8192
  // and 32768.)
  {
    constexpr int kSlots = G * kD / 4;
    constexpr int kGrp = kThreads / kSlots;  // >= 1: kThreads >= 256 >= kSlots
    // (M, L, o[4]) per split group and float4 slot, in the V-tile LDS, which
    // no wave reads any more.
    static_assert(sizeof(float) * kGrp * kSlots * 6 <= sizeof(s_v), "merge scratch");
    auto s_merge = reinterpret_cast<float (*)[kSlots][6]>(&s_v[0][0][0]);
    const int slot = threadIdx.x % kSlots, grp = threadIdx.x / kSlots;
    const int h = slot / (kD / 4), d4 = slot % (kD / 4);
    const __amdgpu_buffer_rsrc_t r_ml =
        make_rsrc(a.ml + (size_t)pair * G * a.S, G * a.S * (int)sizeof(float2));
    const __amdgpu_buffer_rsrc_t r_op =
        make_rsrc(a.opart + (size_t)pair * a.S * G * kD, a.S * G * kD * (int)sizeof(float));
    float M = kNegInf, Ls = 0.0f;
    f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int s0 = grp; s0 < a.S; s0 += 8 * kGrp) {
      f4 ov[8];
      float2 mv[8];
      // (m, l) of split s0 + (lane & 7) kGrp of this lane's head; a split past
      // S reads the next head's entry or zero bytes, and its m is set to -inf
      // below.
      const float2 mls = __builtin_bit_cast(
          float2, __builtin_amdgcn_raw_buffer_load_b64(
                      r_ml, (h * a.S + s0 + (lane & 7) * kGrp) * 8, 0, kSc1));
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        // splits past S read zero bytes (out of the buffer's range)
        const int sj = s0 + j * kGrp;
        ov[j] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(
                                           r_op, ((sj * G + h) * kD + 4 * d4) * 4, 0, kSc1));
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        mv[j].x = __shfl(mls.x, (lane & 32) + j);
        mv[j].y = __shfl(mls.y, (lane & 32) + j);
        if (s0 + j * kGrp >= a.S) mv[j].x = kNegInf;
      }
      float Mn = M;
#pragma unroll
      for (int j = 0; j < 8; ++j) Mn = fmaxf(Mn, mv[j].x);
      const float r = weight2(M, Mn);
      Ls *= r;
      acc *= r;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float w = weight2(mv[j].x, Mn);
        Ls = fmaf(w, mv[j].y, Ls);
        acc += w * ov[j];
      }
      M = Mn;
    }
    float* c = &s_merge[grp][slot][0];
    c[0] = M;
    c[1] = Ls;
    c[2] = acc[0];
    c[3] = acc[1];
    c[4] = acc[2];
    c[5] = acc[3];
    __syncthreads();
    if (grp == 0) {
      float Mt = kNegInf;
#pragma unroll
      for (int gi = 0; gi < kGrp; ++gi) Mt = fmaxf(Mt, s_merge[gi][slot][0]);
      float Lt = 0.0f;
      f4 at = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int gi = 0; gi < kGrp; ++gi) {
        const float* cc = s_merge[gi][slot];
        const float w = weight2(cc[0], Mt);
        Lt = fmaf(w, cc[1], Lt);
        at += w * f4{cc[2], cc[3], cc[4], cc[5]};
      }
      const float inv = 1.0f / Lt;
      uint2 packed;
      packed.x = pack_h2(at[0] * inv, at[1] * inv);
      packed.y = pack_h2(at[2] * inv, at[3] * inv);
      *reinterpret_cast<uint2*>(a.o + q_base + (size_t)h * kD + (size_t)d4 * 4) = packed;
    }
  }
  if (threadIdx.x == 0) __hip_atomic_store(tk, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Second launch of a split call: one workgroup of kGroups x 32 threads per
// (pair, query head).  Thread (grp, d4) merges the splits grp, grp +
// kGroups, ... of float4 slot d4 by online log-sum-exp in base 2 (all loads
// of a chunk of 8 splits are issued together), then the groups merge
// through LDS and write the fp16 output.  The launcher picks kGroups so that
// a thread's splits make one chunk, with at least one whole wave (measured on
// MI355X, 32 q / 8 kv heads: 32 splits with 4 groups beat 8 by 0.15 us at
// batch 1, L = 8192 and 32768; 16 or 32 groups cost 0.4-2 us; 4-8 splits run
// best with 2 groups, 0.2-0.4 us ahead of 8; one group of 32 threads, or one
// wave holding 16 splits per lane, lost 0.1-2 us).  The kernel boundary orders the partial stores of the first
// launch before these loads.
template <int kGroups>
__global__ __launch_bounds__(kGroups * 32) void f4_combine(F4Args a, int G) {
  __shared__ float s_c[kGroups][kD / 4][6];
  // blockIdx = h * pairs + pair: with the XCD-aware numbering of the first
  // launch, the merge of a pair runs on the XCD whose L2 holds its partials.
  const int pairs = a.B * a.Hkv;
  const int pair = blockIdx.x % pairs, h = blockIdx.x / pairs;
  const int d4 = threadIdx.x & (kD / 4 - 1), grp = threadIdx.x / (kD / 4);
  const f4* opart4 = reinterpret_cast<const f4*>(a.opart);
  const float2* mlp = a.ml + ((size_t)pair * G + h) * a.S;
  float M = kNegInf, Ls = 0.0f;
  f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int s0 = grp; s0 < a.S; s0 += kGroups * kMergeChunk) {
    f4 ov[kMergeChunk];
    float2 mv[kMergeChunk];
#pragma unroll
    for (int j = 0; j < kMergeChunk; ++j) {
      const int s = s0 + kGroups * j;
      if (s < a.S) {
        ov[j] = opart4[(((size_t)pair * a.S + s) * G + h) * (kD / 4) + d4];
        mv[j] = mlp[s];
      } else {
        ov[j] = f4{0.0f, 0.0f, 0.0f, 0.0f};
        mv[j] = make_float2(kNegInf, 0.0f);
      }
    }
    float Mn = M;
#pragma unroll
    for (int j = 0; j < kMergeChunk; ++j) Mn = fmaxf(Mn, mv[j].x);
    const float r = weight2(M, Mn);
    Ls *= r;
    acc *= r;
#pragma unroll
    for (int j = 0; j < kMergeChunk; ++j) {
      const float w = weight2(mv[j].x, Mn);
      Ls = fmaf(w, mv[j].y, Ls);
      acc += w * ov[j];
    }
    M = Mn;
  }
  float* c = s_c[grp][d4];
  c[0] = M;
  c[1] = Ls;
  c[2] = acc[0];
  c[3] = acc[1];
  c[4] = acc[2];
  c[5] = acc[3];
  __syncthreads();
  if (grp != 0) return;
  float Mt = kNegInf;
#pragma unroll
  for (int gi = 0; gi < kGroups; ++gi) Mt = fmaxf(Mt, s_c[gi][d4][0]);
  float Lt = 0.0f;
  f4 at = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int gi = 0; gi < kGroups; ++gi) {
    const float* cc = s_c[gi][d4];
    const float w = weight2(cc[0], Mt);
    Lt = fmaf(w, cc[1], Lt);
    at += w * f4{cc[2], cc[3], cc[4], cc[5]};
  }
  const float inv = 1.0f / Lt;
  const int b = pair / a.Hkv, kvh = pair % a.Hkv;
  const size_t o_base = ((size_t)b * a.Hq + (size_t)kvh * G + h) * kD;
  uint2 packed;
  packed.x = pack_h2(at[0] * inv, at[1] * inv);
  packed.y = pack_h2(at[2] * inv, at[3] * inv);
  *reinterpret_cast<uint2*>(a.o + o_base + (size_t)d4 * 4) = packed;
}

using F4Fn = void (*)(F4Args);

template <int NW, bool LINE, int DEPTH>
F4Fn pick_heads(int G) {
  switch (G) {
    case 1: return f4_kernel<1, NW, LINE, DEPTH>;
    case 2: return f4_kernel<2, NW, LINE, DEPTH>;
    case 4: return f4_kernel<4, NW, LINE, DEPTH>;
    default: return f4_kernel<8, NW, LINE, DEPTH>;
  }
}

// One tile in flight (DEPTH 1) is built for the 8-wave whole-line kernel only.
F4Fn pick_kernel(int G, int waves, bool line, int depth) {
  if (waves == 8) {
    if (line) return depth == 1 ? pick_heads<8, true, 1>(G) : pick_heads<8, true, 2>(G);
    return pick_heads<8, false, 2>(G);
  }
  return line ? pick_heads<4, true, 2>(G) : pick_heads<4, false, 2>(G);
}

size_t round256(size_t n) { return (n + 255) / 256 * 256; }

}  // namespace

// Largest split count of one launch.
int f4_max_splits(int G) {
  (void)G;
  return 256;
}

// Workspace: [tickets: pairs x 256 B][ml: pairs x G x S float2][opart:
// pairs x S x G x D fp32], the regions 256-byte aligned.
size_t f4_workspace_bytes(int B, int Hq, int Hkv, int S, int D) {
  const int G = Hq / Hkv;
  const size_t pairs = (size_t)B * Hkv;
  return pairs * kTicketWords * sizeof(unsigned) + round256(pairs * G * S * sizeof(float2)) +
         pairs * S * G * D * sizeof(float);
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

F4Plan f4_plan(int B, int Hkv, int L, int S, int nxcc, bool allow_fused_merge) {
  F4Plan p;
  const int ntiles = (L + kTile - 1) / kTile;
  // Never more splits than tiles: every split then owns at least one tile.
  p.splits = min(S, ntiles);
  p.tiles_per_split = (ntiles + p.splits - 1) / p.splits;
  p.splits = (ntiles + p.tiles_per_split - 1) / p.tiles_per_split;
  p.xcd_map = (B * Hkv) % 8 == 0;
  // The in-launch merge needs the XCD-aware numbering (every split of a pair
  // aimed at one XCD) on a device of 8 XCDs, where that numbering follows
  // the dispatch order.  It replaces the second launch's boundary with one
  // ticket and one L2 round trip (see f4_kernel); db_tune("f4_merge", 2)
  // keeps the second launch.
  p.fused_merge = allow_fused_merge && p.splits > 1 && p.xcd_map && nxcc == 8 &&
                  tuning().f4_merge != 2;
  return p;
}

hipError_t launch_f4(const void* q, const void* k, const void* v, void* o,
                     void* ws, int B, int Hq, int Hkv, int L, int D, int S,
                     float scale, int nxcc, hipStream_t stream, bool allow_fused_merge) {
  const int G = Hq / Hkv;
  const int pairs = B * Hkv;
  const F4Plan plan = f4_plan(B, Hkv, L, S, nxcc, allow_fused_merge);
  F4Args a;
  a.q = static_cast<const _Float16*>(q);
  a.k = static_cast<const _Float16*>(k);
  a.v = static_cast<const _Float16*>(v);
  a.o = static_cast<_Float16*>(o);
  a.B = B;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.L = L;
  a.ntiles = (L + kTile - 1) / kTile;
  a.S = plan.splits;
  a.tps = plan.tiles_per_split;
  // The partial areas are laid out for the caller's S (the size it
  // allocated); the kernels use the first a.S <= S records of each pair.
  char* base = static_cast<char*>(ws);
  const size_t ticket_bytes = (size_t)pairs * kTicketWords * sizeof(unsigned);
  const size_t ml_bytes = round256((size_t)pairs * G * S * sizeof(float2));
  a.ticket = reinterpret_cast<unsigned*>(base);
  a.ml = base ? reinterpret_cast<float2*>(base + ticket_bytes) : nullptr;
  a.opart = base ? reinterpret_cast<float*>(base + ticket_bytes + ml_bytes) : nullptr;
  a.xcd_map = plan.xcd_map ? 1 : 0;
  a.fused_merge = plan.fused_merge ? 1 : 0;
  a.misplace_every = tuning().f4_misplace;
  a.scale_log2 = scale * kLog2e;
  (void)D;
  // With at most 8 (batch, kv-head) pairs (batch 1): 8 waves where a split
  // holds at least 16 tiles or there are at least 32 splits (whose merge
  // takes 8 waves to split its loads); with more pairs, 8 waves only where
  // they walk 2 tiles each (16 tiles per split, whole-line loads).  4 waves
  // otherwise, which at larger batches stream long splits in the plain
  // layout.  Measured on MI355X (32 q / 8 kv heads, interleaved, us, 4 / 8
  // waves):
  //   batch 1: L = 1024 5.32 / 5.48, 2048 6.09 / 6.54, 4096 7.59 / 7.50,
  //            8192 9.67 / 9.47, 16384 14.42 / 14.07, 32768 23.47 / 23.22
  //   batch 2: L = 8192 14.06 / 14.50, 32768 41.33 / 42.10
  //   batch 4: L = 1024 6.60 / 6.68, 2048 9.00 / 8.88, 4096 13.56 / 13.66,
  //            8192 22.60 / 22.80, 32768 77.09 / 77.69
  //   batch 8: L = 1024 9.03 / 8.88, 2048 13.68 / 13.71, 4096 22.60 / 22.74,
  //            8192 40.83 / 40.98, 32768 150.5 / 152.1
  const int auto_waves =
      pairs <= 8 ? (a.tps >= 16 || a.S >= 32 ? 8 : 4) : (a.tps == 16 ? 8 : 4);
  int waves = tuning().f4_waves > 0 ? tuning().f4_waves : auto_waves;
  // Whole-line K loads when a wave walks at most 2 tiles or there are at
  // most 8 (batch, kv-head) pairs; the plain layout streams long splits of
  // larger batches faster (see f4_kernel).
  const int tiles_per_wave = (a.tps + waves - 1) / waves;
  const bool line = tuning().f4_line == 1 ||
                    (tuning().f4_line == 0 && (tiles_per_wave <= 2 || pairs <= 8));
  // Two tiles in flight per wave.  One (DEPTH 1, db_tune("f4_depth", 1))
  // was 0.2 us faster at batch 1, L = 32768 until the two-tile tail became
  // straight-line code; since then it is slower there (24.00 against 23.76
  // us) and at L = 16384 (14.85 against 14.48 us), and 0.3 us slower at
  // L = 1024.
  const int depth = tuning().f4_depth > 0 ? tuning().f4_depth : 2;
  // db_tune("f4_launch", 1 or 2) launches one of the two kernels of the
  // two-launch form alone: a measurement hook that times each half back to
  // back (the merge alone reads whatever records the workspace holds).
  const int only = a.S > 1 && !a.fused_merge ? tuning().f4_launch : 0;
  if (only != 2)
    hipLaunchKernelGGL(pick_kernel(G, waves, line, depth), dim3(pairs * a.S),
                       dim3(waves * kWave), 0, stream, a);
  if (a.S > 1 && !a.fused_merge && only != 1) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int forced = tuning().f4_combine_groups;
    const int want = forced > 0 ? forced : (a.S + kMergeChunk - 1) / kMergeChunk;
    // at least one whole wave: 32-thread workgroups measured slower
    const int groups = want <= 1 ? (forced == 1 ? 1 : 2) : want <= 2 ? 2 : want <= 4 ? 4 : 8;
    const auto fn = groups == 1   ? f4_combine<1>
                    : groups == 2 ? f4_combine<2>
                    : groups == 4 ? f4_combine<4>
                                  : f4_combine<8>;
    hipLaunchKernelGGL(fn, dim3(pairs * G), dim3(groups * 32), 0, stream, a, G);
  }
  return hipGetLastError();
}

// ---- scratch of the allocation-free entry point ---------------------------
// db_f4_splitkv_noalloc keeps its split partial records (the workspace
// layout above, tickets unused because it always merges in the second
// launch) in this file-scope device array.  Every GPU the library runs on
// holds its own copy until the process ends, and every call on that GPU
// reuses it.  In host code `scratch` names a host-side shadow, not device
// memory: the device address comes from hipGetSymbolAddress, looked up once
// per device with that device current, and only that address is passed to
// the kernels.
static __device__ __align__(256) unsigned char scratch[kF4ScratchBytes];

hipError_t f4_scratch_address(void** out) {
  constexpr int kMaxDevices = 64;
  static std::atomic<void*> addr[kMaxDevices];
  static std::mutex mu;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  void* p = addr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(mu);
    p = addr[dev].load(std::memory_order_relaxed);
    if (!p) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess) return e;
      if (!p) return hipErrorInvalidSymbol;
      addr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return hipSuccess;
}

}  // namespace dbk
