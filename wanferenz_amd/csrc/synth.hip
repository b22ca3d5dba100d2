// Counter-based synthetic fill (the portable generator of wanferenz_amd/synth.py).
//
// draw(key, i) = mix64(key + (i + 1) * phi), mix64 = the splitmix64 finaliser.
// Integer-only, so the bytes are identical to the numpy generator and any
// slice of a multi-GB expert bank can be regenerated on the host for checking.
#include "common.h"

namespace wz {

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__global__ __launch_bounds__(256) void synth_fill_kernel(uint8_t* __restrict__ dst, int64_t n,
                                                         uint64_t key, int64_t start, int mode,
                                                         int lo_i, int span, float lo_f,
                                                         float scale_f) {
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
    const uint64_t z = mix64(key + uint64_t(start + i + 1) * 0x9E3779B97F4A7C15ull);
    if (mode == 3) {
      const float k = float(z >> 41) * (1.0f / 8388608.0f);
      reinterpret_cast<float*>(dst)[i] = __fadd_rn(lo_f, __fmul_rn(k, scale_f));  // no FMA contraction
    } else if (mode == 1) {
      dst[i] = uint8_t(lo_i + int(z % uint64_t(span)));
    } else {
      uint8_t b = uint8_t(z & 0xFFu);
      if (mode == 2 && (b & 0x7Fu) == 0x7Fu) b = 0;
      dst[i] = b;
    }
  }
}

}  // namespace wz

extern "C" int wz_synth_fill(void* dst, int64_t n, uint64_t key, int64_t start, int mode, double lo,
                             double hi, hipStream_t stream) {
  using namespace wz;
  if (n < 0 || mode < 0 || mode > 3) return set_error(WZ_EINVAL, "synth_fill: bad n/mode");
  if (n == 0) return WZ_OK;
  if (!dst) return set_error(WZ_EINVAL, "synth_fill: null dst");
  const int span = int(hi) - int(lo) + 1;
  if (mode == 1 && (span <= 0 || lo < 0 || hi > 255)) return set_error(WZ_EINVAL, "synth_fill: bad e8m0 window");
  int64_t blocks = (n + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(synth_fill_kernel, dim3(unsigned(blocks)), dim3(256), 0, stream,
                     static_cast<uint8_t*>(dst), n, key, start, mode, int(lo), span, float(lo),
                     float(hi - lo));
  return check_launch("synth_fill");
}
