// stream_probe.hip -- the single-launch streaming floor of this GPU.
//
// A read-only kernel that does nothing but pull bytes from HBM the way the
// decode kernels do (16-byte non-temporal loads, 1 KB per wave-wide load
// instruction), so that its time for a given byte count is the best any
// single launch of that size can do here: launch and ramp cost plus the
// transfer.  Calibration times it against the fused kernels' byte counts
// (decodebench_amd.calibrate.stream_floor), and the counter pipeline uses it
// as a read-only calibration of known size for FETCH_SIZE.
//
// Shape: every wave reads one contiguous chunk of KB kilobytes, issuing all
// of its KB loads before using any, then exits; workgroups of WV = 1, 2 or 4
// waves (tuning key "stream_waves", default 4).  Measured on MI355X, graph
// back to back: 1-wave workgroups of 4 KB are the fastest form at 33.6 MB
// (5.98-6.01 against 6.05-6.09 us with 4 waves); cached loads (6.5 us),
// buffer loads (6.1 us) and direct-to-LDS loads (6.5 us) are slower.  The
// loaded words are folded into one value that is stored only when it equals
// `magic`, which the caller picks so that it never does: the loads cannot be
// optimised away and the kernel writes nothing.
#include "db_device.h"
#include "db_kernels.h"

namespace dbk {

namespace {

template <int KB, int WV>
__global__ __launch_bounds__(WV * kWave) void stream_read_kernel(
    const unsigned char* src, long long nwaves, unsigned magic, unsigned* sink) {
  const long long wave = (long long)blockIdx.x * WV + threadIdx.x / kWave;
  if (wave >= nwaves) return;
  const int lane = threadIdx.x & (kWave - 1);
  const u4* p = reinterpret_cast<const u4*>(src + wave * (KB * 1024LL)) + lane;
  u4 v[KB];
#pragma unroll
  for (int i = 0; i < KB; ++i) v[i] = ld_stream(p + kWave * i);
  unsigned acc = 0;
#pragma unroll
  for (int i = 0; i < KB; ++i) acc ^= (v[i][0] ^ v[i][1]) ^ (v[i][2] ^ v[i][3]);
  if (acc == magic) sink[wave * kWave + lane] = acc;
}

}  // namespace

template <int KB, int WV>
static void launch_kb_wv(const unsigned char* s, long long nwaves, unsigned magic,
                         unsigned* sink, hipStream_t stream) {
  const unsigned grid = (unsigned)((nwaves + WV - 1) / WV);
  hipLaunchKernelGGL((stream_read_kernel<KB, WV>), dim3(grid), dim3(WV * kWave), 0, stream, s,
                     nwaves, magic, sink);
}

template <int KB>
static void launch_kb(int waves, const unsigned char* s, long long nwaves, unsigned magic,
                      unsigned* sink, hipStream_t stream) {
  if (waves == 1) launch_kb_wv<KB, 1>(s, nwaves, magic, sink, stream);
  else if (waves == 2) launch_kb_wv<KB, 2>(s, nwaves, magic, sink, stream);
  else launch_kb_wv<KB, 4>(s, nwaves, magic, sink, stream);
}

hipError_t launch_stream_read(const void* src, size_t bytes, int kb_per_wave, unsigned magic,
                              unsigned* sink, hipStream_t stream) {
  const long long nwaves = (long long)(bytes / ((size_t)kb_per_wave * 1024));
  const int waves = tuning().stream_waves > 0 ? tuning().stream_waves : 4;
  const auto* s = static_cast<const unsigned char*>(src);
  switch (kb_per_wave) {
    case 4: launch_kb<4>(waves, s, nwaves, magic, sink, stream); break;
    case 8: launch_kb<8>(waves, s, nwaves, magic, sink, stream); break;
    default: launch_kb<16>(waves, s, nwaves, magic, sink, stream); break;
  }
  return hipGetLastError();
}

}  // namespace dbk
