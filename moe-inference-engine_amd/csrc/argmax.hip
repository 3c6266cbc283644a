// Greedy pick of a decode step: the index of the largest of n float32 logits,
// written as an int64 token id - Model.generate's torch.argmax(logits, -1) at
// temperature 0 (src/moe_engine/model.py:603).
//
// torch.argmax returns the first index of the maximum and treats NaN as larger
// than any number; both rules are kept (mie::argmax_take).  One workgroup of
// 1024 threads reads the row with 16-byte loads, up to 16 per thread in
// flight (65536 logits per round; the miniMoE vocabulary is 50257), keeps a
// (value, index) pair per thread and merges the pairs with wave butterflies
// and LDS.  With no second workgroup there are no semaphores to clear, so the
// launch can sit inside a captured graph.
//
// The same merge finishes the LM head's fused pick (launch_argmax_pairs): the
// projection kernel leaves one (value, index) pair per workgroup and one
// workgroup here reduces them.
#include <limits.h>

#include "mie_common.h"

namespace {

constexpr int kThreads = 1024;
constexpr int kVecPerThread = 16;  // float4 loads per thread per round
constexpr int kPairsPerThread = 8;

// The workgroup's pick from every thread's (v, i); thread 0 returns it.
__device__ __forceinline__ void block_argmax(float& v, int& i) {
  __shared__ float s_v[kThreads / 64];
  __shared__ int s_i[kThreads / 64];
  mie::wave_argmax(v, i);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    s_v[wave] = v;
    s_i[wave] = i;
  }
  __syncthreads();
  if (threadIdx.x == 0)
    for (int w = 1; w < kThreads / 64; ++w) mie::argmax_take(v, i, s_v[w], s_i[w]);
}

__global__ __launch_bounds__(kThreads) void argmax_kernel(const float* __restrict__ x, int n, int64_t* out) {
  float v = -INFINITY;
  int idx = INT_MAX;  // past every real index: loses every tie
  int done = 0;
  if ((reinterpret_cast<uintptr_t>(x) & 15) == 0) {
    const float4* xv = reinterpret_cast<const float4*>(x);
    const int nv = n >> 2;
    for (int j0 = 0; j0 < nv; j0 += kVecPerThread * kThreads) {
      float4 t[kVecPerThread];
#pragma unroll
      for (int u = 0; u < kVecPerThread; ++u) {
        const int j = j0 + u * kThreads + threadIdx.x;
        t[u] = j < nv ? xv[j] : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
      }
#pragma unroll
      for (int u = 0; u < kVecPerThread; ++u) {
        const int e = 4 * (j0 + u * kThreads + threadIdx.x);  // past n for padding: never wins
        mie::argmax_take(v, idx, t[u].x, e);
        mie::argmax_take(v, idx, t[u].y, e + 1);
        mie::argmax_take(v, idx, t[u].z, e + 2);
        mie::argmax_take(v, idx, t[u].w, e + 3);
      }
    }
    done = nv << 2;
  }
  for (int i = done + threadIdx.x; i < n; i += kThreads) mie::argmax_take(v, idx, x[i], i);
  block_argmax(v, idx);
  if (threadIdx.x == 0) *out = idx < n ? idx : 0;
}

__global__ __launch_bounds__(kThreads) void argmax_pairs_kernel(const mie::ArgmaxPair* __restrict__ p, int n,
                                                                int limit, int64_t* out, int32_t* advance,
                                                                int n_advance) {
  float v = -INFINITY;
  int idx = INT_MAX;
  for (int j0 = 0; j0 < n; j0 += kPairsPerThread * kThreads) {
    mie::ArgmaxPair t[kPairsPerThread];
#pragma unroll
    for (int u = 0; u < kPairsPerThread; ++u) {
      const int j = j0 + u * kThreads + threadIdx.x;
      t[u] = j < n ? p[j] : mie::ArgmaxPair{-INFINITY, INT_MAX};
    }
#pragma unroll
    for (int u = 0; u < kPairsPerThread; ++u) mie::argmax_take(v, idx, t[u].v, t[u].i);
  }
  block_argmax(v, idx);
  if (threadIdx.x == 0) *out = idx < limit ? idx : 0;
  if (threadIdx.x < n_advance) advance[threadIdx.x] += 1;
}

}  // namespace

namespace mie {
int32_t launch_argmax_pairs(const ArgmaxPair* pairs, int32_t n, int32_t limit, int64_t* out, int32_t* advance,
                            int32_t n_advance, hipStream_t stream) {
  argmax_pairs_kernel<<<1, kThreads, 0, stream>>>(pairs, n, limit, out, advance, n_advance);
  return check_launch("argmax_pairs_kernel");
}
}  // namespace mie

extern "C" int32_t mie_argmax(const void* x, int64_t n, void* out, int32_t dtype, void* stream) {
  if (dtype != MIE_DTYPE_F32) return mie::fail(MIE_ERR_UNSUPPORTED, "mie_argmax: float32 only");
  if (n <= 0 || n > INT32_MAX - kVecPerThread * 4 * kThreads)
    return mie::fail(MIE_ERR_INVALID, "mie_argmax: n=%lld", static_cast<long long>(n));
  if (!x || !out) return mie::fail(MIE_ERR_INVALID, "mie_argmax: null pointer");
  argmax_kernel<<<1, kThreads, 0, static_cast<hipStream_t>(stream)>>>(static_cast<const float*>(x),
                                                                       static_cast<int>(n),
                                                                       static_cast<int64_t*>(out));
  return mie::check_launch("argmax_kernel");
}

extern "C" int32_t mie_argmax_pairs(const void* workspace, int64_t workspace_bytes, int32_t vocab, void* out,
                                    void* stream) {
  const int64_t need = mie_lm_head_workspace(vocab);
  if (need <= 0) return mie::fail(MIE_ERR_INVALID, "mie_argmax_pairs: vocab %d", vocab);
  if (!workspace || !out) return mie::fail(MIE_ERR_INVALID, "mie_argmax_pairs: null pointer");
  if (workspace_bytes < need)
    return mie::fail(MIE_ERR_INVALID, "mie_argmax_pairs: the picks of %d logits take %lld bytes (got %lld)", vocab,
                     static_cast<long long>(need), static_cast<long long>(workspace_bytes));
  if (reinterpret_cast<uintptr_t>(workspace) % alignof(mie::ArgmaxPair) ||
      reinterpret_cast<uintptr_t>(out) % alignof(int64_t))
    return mie::fail(MIE_ERR_INVALID, "mie_argmax_pairs: misaligned workspace or token");
  return mie::launch_argmax_pairs(static_cast<const mie::ArgmaxPair*>(workspace),
                                  static_cast<int32_t>(need / static_cast<int64_t>(sizeof(mie::ArgmaxPair))), vocab,
                                  static_cast<int64_t*>(out), nullptr, 0, static_cast<hipStream_t>(stream));
}
