// Measurement probe for bench.py: the cost of summing every workgroup's
// partial vector of `outputs` values into one vector with device-scope
// atomics, as a split-K product whose partial sums cross workgroups would.
// Every workgroup adds one value per output, into copy (group % copies) of
// the vector; threads take outputs tid, tid + 256, ... so each wave's atomic
// covers 64 consecutive elements.
// Modes:
//   0  int64 atomic add of round(v * 2^32) (exact fixed-point sums, the same
//      result in any order);
//   1  int32 atomic add of round(v * 2^16);
//   2  float32 atomic add (hardware float atomics; order-dependent rounding);
//   3  plain int64 stores of each workgroup's partials to its own row (no
//      atomics: the traffic baseline).
// The values are small exact multiples of 2^-8, so every mode's sum is exact
// and the host can check it.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

__device__ __forceinline__ float partial(int group, int i) {
  return static_cast<float>(((group * 131 + i * 7) & 255) - 128) * (1.f / 256.f);
}

template <int MODE>
__global__ __launch_bounds__(256) void atomic_sum_kernel(void* acc, int outputs, int copies) {
  const int64_t base = static_cast<int64_t>(blockIdx.x % copies) * outputs;
  for (int i = threadIdx.x; i < outputs; i += blockDim.x) {
    const float v = partial(blockIdx.x, i);
    if constexpr (MODE == 0) {
      __hip_atomic_fetch_add(static_cast<long long*>(acc) + base + i, static_cast<long long>(v * 4294967296.0f),
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else if constexpr (MODE == 1) {
      __hip_atomic_fetch_add(static_cast<int*>(acc) + base + i, static_cast<int>(v * 65536.0f), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
    } else if constexpr (MODE == 2) {
      unsafeAtomicAdd(static_cast<float*>(acc) + base + i, v);
    } else {
      static_cast<long long*>(acc)[static_cast<int64_t>(blockIdx.x) * outputs + i] =
          static_cast<long long>(v * 4294967296.0f);
    }
  }
}

}  // namespace

// acc: int64 [copies * outputs] (mode 0; mode 3: int64 [groups * outputs]),
// int32 (mode 1) or float32 (mode 2) [copies * outputs], zeroed by the caller.
extern "C" int32_t mie_probe_atomic_sum(int32_t mode, int32_t groups, int32_t outputs, int32_t copies, void* acc,
                                        void* stream) {
  if (mode < 0 || mode > 3 || groups <= 0 || groups > 65535 || outputs <= 0 || outputs > (1 << 20) || !acc ||
      copies <= 0 || copies > groups)
    return 1;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(groups), block(256);
  switch (mode) {
    case 0: atomic_sum_kernel<0><<<grid, block, 0, st>>>(acc, outputs, copies); break;
    case 1: atomic_sum_kernel<1><<<grid, block, 0, st>>>(acc, outputs, copies); break;
    case 2: atomic_sum_kernel<2><<<grid, block, 0, st>>>(acc, outputs, copies); break;
    default: atomic_sum_kernel<3><<<grid, block, 0, st>>>(acc, outputs, copies); break;
  }
  return hipGetLastError() == hipSuccess ? 0 : 2;
}
