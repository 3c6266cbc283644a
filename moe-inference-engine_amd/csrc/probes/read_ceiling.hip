// Measurement probes for bench.py (not part of the C ABI of libmie_paged.so):
//
//   mie_probe_read_chunks  reads 2 KiB chunks - the size of one bf16 (block,
//                          head) tile of the paged pools at block 16 x
//                          head_dim 64 - at the chunk ids it is given, either
//                          into registers with non-temporal 16-byte loads (the
//                          decode kernels' way) or into an LDS ring with
//                          global_load_lds (the "LDS-staged tile" way), with
//                          `depth` chunks in flight per wave.  Random ids give
//                          the ceiling of the decode's access pattern.
//   mie_probe_noop         an empty kernel, for the launch floor of a graph.
//
// Every wave reads whole chunks inside the buffer (ids are checked on the
// host), folds them into one word per lane and writes it, so no load is dead.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
constexpr int kChunk = 2048;

template <int D>
__global__ __launch_bounds__(256) void read_registers(const char* __restrict__ buf, const int32_t* __restrict__ ids,
                                                      int32_t n_ids, uint32_t* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int nwaves = (gridDim.x * blockDim.x) >> 6;
  uint32_t acc = 0;
  for (int c = wave * D; c < n_ids; c += nwaves * D) {
    u32x4 v[D][2];
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int id = ids[c + d < n_ids ? c + d : c];
      const char* p = buf + static_cast<int64_t>(id) * kChunk + lane * 16;
      v[d][0] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
      v[d][1] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p + 1024));
    }
#pragma unroll
    for (int d = 0; d < D; ++d)
      acc ^= v[d][0].x ^ v[d][0].y ^ v[d][0].z ^ v[d][0].w ^ v[d][1].x ^ v[d][1].y ^ v[d][1].z ^ v[d][1].w;
  }
  out[wave * 64 + lane] = acc;
}

template <int S>
__global__ __launch_bounds__(256) void read_lds(const char* __restrict__ buf, const int32_t* __restrict__ ids,
                                                int32_t n_ids, uint32_t* __restrict__ out) {
  __shared__ __align__(16) char ring[4][S][kChunk];
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int nwaves = (gridDim.x * blockDim.x) >> 6;
  uint32_t acc = 0;
  for (int c = wave * S; c < n_ids; c += nwaves * S) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int id = ids[c + s < n_ids ? c + s : c];
      const char* p = buf + static_cast<int64_t>(id) * kChunk + lane * 16;
      // C-style casts: the builtin takes global and LDS address-space pointers.
      __builtin_amdgcn_global_load_lds((const void __attribute__((address_space(1)))*)p,
                                       (void __attribute__((address_space(3)))*)&ring[w][s][0], 16, 0, 0);
      __builtin_amdgcn_global_load_lds((const void __attribute__((address_space(1)))*)(p + 1024),
                                       (void __attribute__((address_space(3)))*)&ring[w][s][1024], 16, 0, 0);
    }
    __builtin_amdgcn_s_waitcnt(0);  // this wave's LDS loads have landed (each wave owns its ring slice)
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const u32x4 a = *reinterpret_cast<const u32x4*>(&ring[w][s][lane * 16]);
      const u32x4 b = *reinterpret_cast<const u32x4*>(&ring[w][s][1024 + lane * 16]);
      acc ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w;
    }
    __builtin_amdgcn_s_waitcnt(0);  // reads of the ring are done before the next loads overwrite it
  }
  out[wave * 64 + lane] = acc;
}

__global__ void noop_kernel() {}

}  // namespace

// kind 0: registers (depth 1, 2, 4 or 8 chunks in flight per wave); kind 1:
// global_load_lds into an LDS ring (depth 1, 2 or 4).  `groups` workgroups of
// 4 waves; `out` holds groups * 256 words.  ids index 2 KiB chunks of `buf`,
// which holds buf_chunks of them.  Returns 0, or 1 for bad arguments, 2 for a
// failed launch.
extern "C" int32_t mie_probe_read_chunks(int32_t kind, int32_t depth, const void* buf, int64_t buf_chunks,
                                         const int32_t* ids, int32_t n_ids, int32_t groups, uint32_t* out,
                                         void* stream) {
  if (!buf || !ids || !out || n_ids <= 0 || groups <= 0 || buf_chunks <= 0) return 1;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const char* b = static_cast<const char*>(buf);
  if (kind == 0) {
    switch (depth) {
      case 1: read_registers<1><<<groups, 256, 0, st>>>(b, ids, n_ids, out); break;
      case 2: read_registers<2><<<groups, 256, 0, st>>>(b, ids, n_ids, out); break;
      case 4: read_registers<4><<<groups, 256, 0, st>>>(b, ids, n_ids, out); break;
      case 8: read_registers<8><<<groups, 256, 0, st>>>(b, ids, n_ids, out); break;
      default: return 1;
    }
  } else if (kind == 1) {
    switch (depth) {
      case 1: read_lds<1><<<groups, 256, 0, st>>>(b, ids, n_ids, out); break;
      case 2: read_lds<2><<<groups, 256, 0, st>>>(b, ids, n_ids, out); break;
      case 4: read_lds<4><<<groups, 256, 0, st>>>(b, ids, n_ids, out); break;
      default: return 1;
    }
  } else {
    return 1;
  }
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

extern "C" int32_t mie_probe_noop(int32_t groups, void* stream) {
  if (groups <= 0) return 1;
  noop_kernel<<<groups, 256, 0, static_cast<hipStream_t>(stream)>>>();
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

// L2 reuse across kernel boundaries: workgroup w reads region (w + shift) mod
// gridDim.x of `buf` (per_group_bytes each, 16-byte loads, folded into `out`).
// Read once with shift s and again with shift 0: the second launch hits the
// L2 of its own XCD when s is a multiple of 8 (the dispatcher places
// workgroup i on XCD i mod 8), only the last-level cache otherwise.
namespace {
__global__ __launch_bounds__(256) void read_region_kernel(const u32x4* __restrict__ buf, int32_t per_group_vec,
                                                          int32_t shift, uint32_t* __restrict__ out) {
  const int region = (static_cast<int>(blockIdx.x) + shift) % static_cast<int>(gridDim.x);
  const u32x4* p = buf + static_cast<int64_t>(region) * per_group_vec;
  uint32_t acc = 0;
  for (int i = threadIdx.x; i < per_group_vec; i += 256) {
    const u32x4 v = p[i];
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  out[blockIdx.x * 256 + threadIdx.x] = acc;
}
}  // namespace

extern "C" int32_t mie_probe_read_regions(const void* buf, int64_t buf_bytes, int32_t groups, int32_t per_group_bytes,
                                          int32_t shift, uint32_t* out, void* stream) {
  if (!buf || !out || groups <= 0 || per_group_bytes <= 0 || per_group_bytes % 16 || shift < 0 ||
      static_cast<int64_t>(groups) * per_group_bytes > buf_bytes)
    return 1;
  read_region_kernel<<<groups, 256, 0, static_cast<hipStream_t>(stream)>>>(static_cast<const u32x4*>(buf),
                                                                         per_group_bytes / 16, shift, out);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}
