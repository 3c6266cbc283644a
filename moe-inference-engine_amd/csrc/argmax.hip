// Greedy pick of a decode step: the index of the largest of n float32 logits,
// written as an int64 token id - Model.generate's torch.argmax(logits, -1) at
// temperature 0 (src/moe_engine/model.py:603).
//
// torch.argmax returns the first index of the maximum and treats NaN as larger
// than any number; both rules are kept.  One workgroup of 1024 threads reads
// the row with coalesced strided loads (50257 logits = 200 KB at the miniMoE
// vocabulary), keeps a (value, index) pair per thread and merges the pairs
// with wave butterflies and LDS.  With no second workgroup there are no
// semaphores to clear, so the launch can sit inside a captured graph.
#include "mie_common.h"

namespace {

constexpr int kThreads = 1024;

constexpr int kUnroll = 8;  // loads in flight per thread before the compares

// (va, ia) replaced by (vb, ib) when b comes first in torch.argmax's order.
// The order is total over (value, index), so the pairs may be merged in any
// order.
__device__ __forceinline__ void take_better(float& va, int& ia, float vb, int ib) {
  const bool a_nan = va != va, b_nan = vb != vb;
  bool b_wins;
  if (a_nan || b_nan) {
    b_wins = b_nan && (!a_nan || ib < ia);
  } else {
    b_wins = vb > va || (vb == va && ib < ia);
  }
  if (b_wins) {
    va = vb;
    ia = ib;
  }
}

__global__ __launch_bounds__(kThreads) void argmax_kernel(const float* __restrict__ x, int n, int64_t* out) {
  __shared__ float s_v[kThreads / 64];
  __shared__ int s_i[kThreads / 64];
  float v = -INFINITY;
  int idx = n;  // past every real index: loses every tie
  int i = threadIdx.x;
  for (; i + (kUnroll - 1) * kThreads < n; i += kUnroll * kThreads) {
    float t[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) t[u] = x[i + u * kThreads];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) take_better(v, idx, t[u], i + u * kThreads);
  }
  for (; i < n; i += kThreads) take_better(v, idx, x[i], i);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(v, off);
    const int oi = __shfl_xor(idx, off);
    take_better(v, idx, ov, oi);
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    s_v[wave] = v;
    s_i[wave] = idx;
  }
  __syncthreads();
  if (threadIdx.x != 0) return;
  for (int w = 1; w < kThreads / 64; ++w) take_better(v, idx, s_v[w], s_i[w]);
  *out = idx < n ? idx : 0;
}

}  // namespace

extern "C" int32_t mie_argmax(const void* x, int64_t n, void* out, int32_t dtype, void* stream) {
  if (dtype != MIE_DTYPE_F32) return mie::fail(MIE_ERR_UNSUPPORTED, "mie_argmax: float32 only");
  if (n <= 0 || n > INT32_MAX - kUnroll * kThreads)
    return mie::fail(MIE_ERR_INVALID, "mie_argmax: n=%lld", static_cast<long long>(n));
  if (!x || !out) return mie::fail(MIE_ERR_INVALID, "mie_argmax: null pointer");
  argmax_kernel<<<1, kThreads, 0, static_cast<hipStream_t>(stream)>>>(static_cast<const float*>(x), static_cast<int>(n),
                                                                       static_cast<int64_t*>(out));
  return mie::check_launch("argmax_kernel");
}
