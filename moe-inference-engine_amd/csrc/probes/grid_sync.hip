// Measurement probe for bench.py: the cost of a grid-wide barrier inside one
// cooperative launch, to set against a kernel boundary in a graph
// (mie_probe_noop).  Each iteration every workgroup writes a slice of a
// vector, all workgroups meet at a counter, and each then reads and checks
// values from eight other workgroups' slices (double-buffered by iteration
// parity).  Modes:
//   0  plain stores; every thread fences at agent scope before and after
//      the barrier (__threadfence);
//   1  device-scope relaxed atomic stores and loads for the data (they bypass
//      the non-coherent per-XCD L2), workgroup-scope fences around the
//      barrier: no L2 writeback;
//   2  plain stores; one agent-scope release fence per workgroup before its
//      arrival and one acquire fence after the wait (one L2 writeback per
//      workgroup);
//   3  the data as in mode 1 (device-scope atomic stores and loads) and the
//      fences as in mode 2: formally ordered, with nothing dirty in the L2
//      for the release to write back.
// Every wait is bounded: a wave that spins past the limit raises a global
// flag, every waiter leaves once the flag is up, and the launch reports it,
// so the grid always drains.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

__device__ inline unsigned load_agent(unsigned* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int MODE>
__global__ __launch_bounds__(256) void barrier_kernel(unsigned* counter, float* vec, int* err, int* bad, int iters,
                                                      int per_group, long spin_limit) {
  const int G = gridDim.x;
  __shared__ int stop;
  if (threadIdx.x == 0) stop = 0;
  __syncthreads();
  int wrong = 0;
  for (int it = 0; it < iters; ++it) {
    float* buf = vec + static_cast<size_t>(it & 1) * G * per_group;
    for (int i = threadIdx.x; i < per_group; i += blockDim.x) {
      const float v = static_cast<float>((it * 7 + blockIdx.x * 3 + i) & 0xffff);
      if (MODE == 1 || MODE == 3) {
        __hip_atomic_store(&buf[blockIdx.x * per_group + i], v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      } else {
        buf[blockIdx.x * per_group + i] = v;
      }
    }
    if (MODE == 0) __threadfence();
    if (MODE == 1 || MODE == 3) __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __syncthreads();
    if (threadIdx.x == 0) {
      if (MODE == 2 || MODE == 3) __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
      __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const unsigned target = static_cast<unsigned>(it + 1) * G;
      long spins = 0;
      while (load_agent(counter) < target) {
        if (++spins > spin_limit) {
          __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          break;
        }
        if (__hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) break;
        __builtin_amdgcn_s_sleep(1);
      }
      if (MODE == 2 || MODE == 3) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
      if (__hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) stop = 1;
    }
    __syncthreads();
    if (MODE == 0) __threadfence();
    if (MODE == 1 || MODE == 3) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    if (stop) break;
    for (int j = threadIdx.x; j < 32; j += blockDim.x) {
      const int src = (blockIdx.x + 1 + (j >> 2) * 37) % G;
      const int i = (j & 3) * (per_group / 4);
      const float want = static_cast<float>((it * 7 + src * 3 + i) & 0xffff);
      float* p = &buf[src * per_group + i];
      const float got = MODE == 1 || MODE == 3 ? __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                               : *p;
      wrong += got != want;
    }
  }
  if (wrong) atomicAdd(bad, wrong);
}

}  // namespace

// One cooperative launch of `groups` workgroups running `iters` barriers in
// `mode`; scratch: counter (4 B), vec (2 * groups * per_group floats), err and
// bad (4 B each), all cleared by the caller.  Returns 0, 1 for bad arguments,
// 2 when the runtime refused the cooperative launch.
extern "C" int32_t mie_probe_grid_barrier(int32_t mode, int32_t groups, int32_t iters, int32_t per_group,
                                          void* counter, void* vec, void* err, void* bad, int64_t spin_limit,
                                          void* stream) {
  if (groups <= 0 || iters <= 0 || per_group < 4 || !counter || !vec || !err || !bad || spin_limit <= 0) return 1;
  long limit = static_cast<long>(spin_limit);
  void* args[] = {&counter, &vec, &err, &bad, &iters, &per_group, &limit};
  const void* fn = nullptr;
  switch (mode) {
    case 0: fn = reinterpret_cast<const void*>(&barrier_kernel<0>); break;
    case 1: fn = reinterpret_cast<const void*>(&barrier_kernel<1>); break;
    case 2: fn = reinterpret_cast<const void*>(&barrier_kernel<2>); break;
    case 3: fn = reinterpret_cast<const void*>(&barrier_kernel<3>); break;
    default: return 1;
  }
  const hipError_t e = hipLaunchCooperativeKernel(fn, dim3(groups), dim3(256), args, 0,
                                                  static_cast<hipStream_t>(stream));
  return e == hipSuccess ? 0 : 2;
}
