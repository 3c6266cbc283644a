// Fused top-k mixture-of-experts for one decode token (float32), no host sync.
//
// Replaces, for a single token, the reference's PyTorch MoE path
// (src/moe_engine/model.py:443-461), whose per-expert torch.where forces a
// device-to-host sync for every expert of every layer, and plays the role of
// its Triton fused MoE (src/moe_engine/fused_moe.py:119-380):
//
//   logits = W_r x                       (E logits, float32)
//   ids    = the top_k logits' experts   (largest first, lower id on ties)
//   w      = softmax(logits[ids])
//   out    = sum over ids in increasing id of  w_e * (W2_e GELU(W1_e x + b1_e) + b2_e)
//
// The sum runs in increasing expert id from zero, the order in which the
// reference's index_add_ loop accumulates (model.py:455-460).  GELU is the
// exact erf form of torch.nn.GELU().
//
// Three launches: route (one workgroup), W1 + GELU (one wavefront per 4 rows
// of each selected expert), W2 + weighted sum (one wavefront per output).  The
// expert weights stay where the model keeps them: the kernels get per-expert
// pointer arrays and read only the selected experts' rows, each wave load a
// coalesced 1 KiB run of a row.  The GEMVs are HBM-bound (2 * top_k * dim *
// hidden * 4 bytes per token), so there is no MFMA work here.
#include <math.h>

#include "mie_common.h"

namespace {

constexpr int kMaxExperts = 64;
constexpr int kMaxTopK = 8;

struct MoeArgs {
  const float* x;
  const float* router;  // [E, dim]
  const float* w1[kMaxExperts];  // [hidden, dim] each
  const float* b1[kMaxExperts];  // [hidden]
  const float* w2[kMaxExperts];  // [dim, hidden]
  const float* b2[kMaxExperts];  // [dim]
  int32_t E, top_k, dim, hidden;
  float* out;      // [dim]
  int32_t* ids;    // workspace: [top_k] selected experts, increasing id
  float* weights;  // workspace: [top_k] their softmax weights
  float* h;        // workspace: [top_k, hidden]
};

// Dot product of a float32 row with a float32 vector, one wavefront, both
// 16-byte aligned with n a multiple of 4: lanes take 16-byte slices.
__device__ __forceinline__ float wave_dot(const float* __restrict__ row, const float* __restrict__ v, int n, int lane) {
  float s = 0.f;
  for (int i = lane * 4; i < n; i += 256) {
    const float4 a = *reinterpret_cast<const float4*>(row + i);
    const float4 b = *reinterpret_cast<const float4*>(v + i);
    s = fmaf(a.x, b.x, s);
    s = fmaf(a.y, b.y, s);
    s = fmaf(a.z, b.z, s);
    s = fmaf(a.w, b.w, s);
  }
  return mie::wave_sum(s);
}

__global__ __launch_bounds__(256) void moe_route_kernel(MoeArgs a) {
  __shared__ float logits[kMaxExperts];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  for (int e = wave; e < a.E; e += 4) {
    const float s = wave_dot(a.router + static_cast<int64_t>(e) * a.dim, a.x, a.dim, lane);
    if (lane == 0) logits[e] = s;
  }
  __syncthreads();
  if (threadIdx.x != 0) return;
  int ids[kMaxTopK];
  float vals[kMaxTopK];
  uint64_t taken = 0;
  for (int k = 0; k < a.top_k; ++k) {
    int best = -1;
    for (int e = 0; e < a.E; ++e) {
      if ((taken >> e) & 1) continue;
      if (best < 0 || logits[e] > logits[best]) best = e;
    }
    taken |= uint64_t{1} << best;
    ids[k] = best;
    vals[k] = logits[best];
  }
  // softmax over the selected logits (vals[0] is their maximum)
  float p[kMaxTopK];
  float sum = 0.f;
  for (int k = 0; k < a.top_k; ++k) {
    p[k] = expf(vals[k] - vals[0]);
    sum += p[k];
  }
  for (int k = 0; k < a.top_k; ++k) p[k] /= sum;
  // increasing expert id, carrying the weights
  for (int i = 1; i < a.top_k; ++i) {
    for (int j = i; j > 0 && ids[j - 1] > ids[j]; --j) {
      const int ti = ids[j];
      ids[j] = ids[j - 1];
      ids[j - 1] = ti;
      const float tp = p[j];
      p[j] = p[j - 1];
      p[j - 1] = tp;
    }
  }
  for (int k = 0; k < a.top_k; ++k) {
    a.ids[k] = ids[k];
    a.weights[k] = p[k];
  }
}

// grid = (ceil(hidden / 16), top_k); each wave computes 4 rows of one expert.
__global__ __launch_bounds__(256) void moe_w1_gelu_kernel(MoeArgs a) {
  const int k = blockIdx.y;
  const int e = a.ids[k];
  const float* __restrict__ w = a.w1[e];
  const float* __restrict__ b = a.b1[e];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int r0 = (blockIdx.x * 4 + wave) * 4;
#pragma unroll
  for (int rr = 0; rr < 4; ++rr) {
    const int r = r0 + rr;
    if (r >= a.hidden) break;
    const float s = wave_dot(w + static_cast<int64_t>(r) * a.dim, a.x, a.dim, lane) + b[r];
    if (lane == 0) a.h[static_cast<int64_t>(k) * a.hidden + r] = 0.5f * s * (1.f + erff(s * 0.70710678118654752440f));
  }
}

// grid = ceil(dim / 4); each wave owns one output element across the experts.
__global__ __launch_bounds__(256) void moe_w2_reduce_kernel(MoeArgs a) {
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int j = blockIdx.x * 4 + wave;
  if (j >= a.dim) return;
  float acc = 0.f;
  for (int k = 0; k < a.top_k; ++k) {
    const int e = a.ids[k];
    const float y = wave_dot(a.w2[e] + static_cast<int64_t>(j) * a.hidden, a.h + static_cast<int64_t>(k) * a.hidden,
                             a.hidden, lane) +
                    a.b2[e][j];
    acc = acc + a.weights[k] * y;
  }
  if (lane == 0) a.out[j] = acc;
}

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

}  // namespace

extern "C" int64_t mie_moe_decode_workspace_bytes(int32_t top_k, int32_t hidden) {
  if (top_k <= 0 || hidden <= 0) return 0;
  return 256 + static_cast<int64_t>(top_k) * hidden * 4;  // ids and weights, then h (16-byte aligned)
}

extern "C" int32_t mie_moe_decode(const void* x, const void* router_weight, const void* const* w1,
                                  const void* const* b1, const void* const* w2, const void* const* b2,
                                  int32_t num_experts, int32_t top_k, int32_t dim, int32_t hidden, void* out,
                                  void* workspace, int64_t workspace_bytes, int32_t dtype, void* stream) {
  if (dtype != MIE_DTYPE_F32) return mie::fail(MIE_ERR_UNSUPPORTED, "mie_moe_decode: float32 only");
  if (num_experts <= 0 || num_experts > kMaxExperts || top_k <= 0 || top_k > kMaxTopK || top_k > num_experts)
    return mie::fail(MIE_ERR_INVALID, "mie_moe_decode: experts=%d top_k=%d (at most %d and %d)", num_experts, top_k,
                     kMaxExperts, kMaxTopK);
  if (dim <= 0 || hidden <= 0 || dim % 4 != 0 || hidden % 4 != 0)
    return mie::fail(MIE_ERR_INVALID, "mie_moe_decode: dim=%d hidden=%d must be positive multiples of 4", dim, hidden);
  if (!x || !router_weight || !w1 || !b1 || !w2 || !b2 || !out || !workspace)
    return mie::fail(MIE_ERR_INVALID, "mie_moe_decode: null pointer");
  if (workspace_bytes < mie_moe_decode_workspace_bytes(top_k, hidden) || !aligned16(workspace))
    return mie::fail(MIE_ERR_WORKSPACE, "mie_moe_decode: needs a 16-byte aligned workspace of %lld bytes",
                     static_cast<long long>(mie_moe_decode_workspace_bytes(top_k, hidden)));
  MoeArgs a;
  a.x = static_cast<const float*>(x);
  a.router = static_cast<const float*>(router_weight);
  bool ok = aligned16(x) && aligned16(router_weight);
  for (int e = 0; e < num_experts; ++e) {
    a.w1[e] = static_cast<const float*>(w1[e]);
    a.b1[e] = static_cast<const float*>(b1[e]);
    a.w2[e] = static_cast<const float*>(w2[e]);
    a.b2[e] = static_cast<const float*>(b2[e]);
    ok = ok && a.w1[e] && a.b1[e] && a.w2[e] && a.b2[e] && aligned16(a.w1[e]) && aligned16(a.w2[e]);
  }
  if (!ok) return mie::fail(MIE_ERR_INVALID, "mie_moe_decode: null or misaligned weight pointer");
  for (int e = num_experts; e < kMaxExperts; ++e) a.w1[e] = a.b1[e] = a.w2[e] = a.b2[e] = nullptr;
  a.E = num_experts;
  a.top_k = top_k;
  a.dim = dim;
  a.hidden = hidden;
  a.out = static_cast<float*>(out);
  a.ids = static_cast<int32_t*>(workspace);
  a.weights = reinterpret_cast<float*>(static_cast<char*>(workspace) + 128);
  a.h = reinterpret_cast<float*>(static_cast<char*>(workspace) + 256);
  hipStream_t st = static_cast<hipStream_t>(stream);
  moe_route_kernel<<<1, 256, 0, st>>>(a);
  int32_t rc = mie::check_launch("moe_route_kernel");
  if (rc != MIE_OK) return rc;
  moe_w1_gelu_kernel<<<dim3((hidden + 15) / 16, top_k), 256, 0, st>>>(a);
  rc = mie::check_launch("moe_w1_gelu_kernel");
  if (rc != MIE_OK) return rc;
  moe_w2_reduce_kernel<<<(dim + 3) / 4, 256, 0, st>>>(a);
  return mie::check_launch("moe_w2_reduce_kernel");
}
