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
// of its KB loads before using any, then exits; workgroups of 4 waves.  The
// loaded words are folded into one value that is stored only when it equals
// `magic`, which the caller picks so that it never does: the loads cannot be
// optimised away and the kernel writes nothing.
#include "db_device.h"
#include "db_kernels.h"

namespace dbk {

namespace {

constexpr int kProbeWaves = 4;

template <int KB>
__global__ __launch_bounds__(kProbeWaves * kWave) void stream_read_kernel(
    const unsigned char* src, long long nwaves, unsigned magic, unsigned* sink) {
  const long long wave = (long long)blockIdx.x * kProbeWaves + threadIdx.x / kWave;
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

hipError_t launch_stream_read(const void* src, size_t bytes, int kb_per_wave, unsigned magic,
                              unsigned* sink, hipStream_t stream) {
  const long long nwaves = (long long)(bytes / ((size_t)kb_per_wave * 1024));
  const unsigned grid = (unsigned)((nwaves + kProbeWaves - 1) / kProbeWaves);
  const auto* s = static_cast<const unsigned char*>(src);
  switch (kb_per_wave) {
    case 4:
      hipLaunchKernelGGL(stream_read_kernel<4>, dim3(grid), dim3(kProbeWaves * kWave), 0, stream,
                         s, nwaves, magic, sink);
      break;
    case 8:
      hipLaunchKernelGGL(stream_read_kernel<8>, dim3(grid), dim3(kProbeWaves * kWave), 0, stream,
                         s, nwaves, magic, sink);
      break;
    default:
      hipLaunchKernelGGL(stream_read_kernel<16>, dim3(grid), dim3(kProbeWaves * kWave), 0,
                         stream, s, nwaves, magic, sink);
      break;
  }
  return hipGetLastError();
}

}  // namespace dbk
