// Fused top-k mixture-of-experts for one decode token (float32), no host sync.
//
// Replaces, for a single token, the reference's PyTorch MoE path
// (src/moe_engine/model.py:443-461), whose per-expert torch.where forces a
// device-to-host sync for every expert of every layer, and serves the
// interface of its Triton fused MoE (src/moe_engine/fused_moe.py:274-380):
//
//   logits = W_r x                       (E router logits, float32)
//   ids    = the top_k experts by logit  (largest first, lower id on ties)
//   w      = softmax(logits[ids])        (in the same order)
//   h[s]   = GELU(W1[ids[s]] x + b1[ids[s]])           for each slot s
//   out    = sum over the slots in increasing expert id, starting from 0, of
//            round(w[s] * (W2[ids[s]] h[s] + b2[ids[s]]))
//
// The sum runs in increasing expert id with a separate rounding of each
// product, the order and rounding in which the reference's index_add_ loop
// accumulates (model.py:455-460).  GELU is the exact erf form of nn.GELU().
//
// Expert weights live in four canonical contiguous storages - W1 [E, hidden,
// dim], b1 [E, hidden], W2 [E, dim, hidden], b2 [E, dim] - so a selected
// expert is a device-side offset; the route never leaves the GPU.
//
// Three launches.  The GEMVs are HBM-bound (2 * top_k * dim * hidden * 4
// bytes per token, ~12.6 MB at d 768 / FFN 2048 / top-2): each wave issues all
// of its weight loads (non-temporal: a token's experts are streamed once)
// before it reduces, so a launch keeps the whole working set in flight.
#include <math.h>

#include "mie_common.h"

namespace {

constexpr int kMaxExperts = 64;
constexpr int kMaxTopK = 8;

typedef float f32x4_t __attribute__((ext_vector_type(4)));

struct MoeArgs {
  const float* x;       // [dim]
  const float* router;  // [E, dim]
  const float* w1;      // [E, hidden, dim]
  const float* b1;      // [E, hidden]
  const float* w2;      // [E, dim, hidden]
  const float* b2;      // [E, dim]
  int32_t E, top_k, dim, hidden;
  float* logits;   // [E]
  int32_t* ids;    // [top_k], largest logit first
  float* weights;  // [top_k], same order
  float* h;        // [top_k, hidden], same order
  float* out;      // [dim]
};

__device__ __forceinline__ f32x4_t load4(const float* p) { return *reinterpret_cast<const f32x4_t*>(p); }
__device__ __forceinline__ f32x4_t stream4(const float* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(p));
}
__device__ __forceinline__ float dot4(f32x4_t a, f32x4_t b, float s) {
  s = fmaf(a.x, b.x, s);
  s = fmaf(a.y, b.y, s);
  s = fmaf(a.z, b.z, s);
  return fmaf(a.w, b.w, s);
}

// Dot product of a row with a vector over one wavefront (16-byte slices per lane).
__device__ __forceinline__ float wave_dot(const float* __restrict__ row, const float* __restrict__ v, int n, int lane) {
  float s = 0.f;
  for (int i = lane * 4; i < n; i += 256) s = dot4(load4(row + i), load4(v + i), s);
  return mie::wave_sum(s);
}

// One workgroup: E router dot products, then top-k and softmax on one lane.
__global__ __launch_bounds__(256) void moe_route_kernel(MoeArgs a) {
  __shared__ float logits[kMaxExperts];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  for (int e = wave; e < a.E; e += 4) {
    const float s = wave_dot(a.router + static_cast<int64_t>(e) * a.dim, a.x, a.dim, lane);
    if (lane == 0) {
      logits[e] = s;
      a.logits[e] = s;
    }
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
  // softmax over the selected logits; vals[0] is their maximum
  float p[kMaxTopK];
  float sum = 0.f;
  for (int k = 0; k < a.top_k; ++k) {
    p[k] = expf(vals[k] - vals[0]);
    sum += p[k];
  }
  for (int k = 0; k < a.top_k; ++k) {
    a.ids[k] = ids[k];
    a.weights[k] = p[k] / sum;
  }
}

// Sums four per-lane partials r0..r3 over the wave with 3 cross-lane moves and
// a 16-lane reduction instead of four full reductions: after the xor-32 and
// xor-16 exchanges, lanes 16q..16q+15 hold partials of row q only.  Returns
// row (lane >> 4)'s total in every lane.
__device__ __forceinline__ float wave_sum4(float r0, float r1, float r2, float r3, int lane) {
  const bool hi = lane & 32;
  const float a0 = (hi ? r2 : r0) + __shfl_xor(hi ? r0 : r2, 32);
  const float a1 = (hi ? r3 : r1) + __shfl_xor(hi ? r1 : r3, 32);
  const bool mid = lane & 16;
  const float b = (mid ? a1 : a0) + __shfl_xor(mid ? a0 : a1, 16);
  return mie::group_sum<16>(b);
}

// grid = (ceil(hidden / 16), top_k); each wave computes 4 rows of slot
// blockIdx.y's expert.  hidden % 4 == 0, so a wave's rows are all valid or
// all past the end.
__global__ __launch_bounds__(256) void moe_w1_gelu_kernel(MoeArgs a) {
  const int k = blockIdx.y;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int r0 = (blockIdx.x * 4 + wave) * 4;
  if (r0 >= a.hidden) return;
  const int e = a.ids[k];
  const int64_t dim = a.dim;
  const float* __restrict__ w = a.w1 + (static_cast<int64_t>(e) * a.hidden + r0) * dim;
  float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll 4
  for (int i = lane * 4; i < a.dim; i += 256) {
    const f32x4_t q0 = stream4(w + i);
    const f32x4_t q1 = stream4(w + dim + i);
    const f32x4_t q2 = stream4(w + 2 * dim + i);
    const f32x4_t q3 = stream4(w + 3 * dim + i);
    const f32x4_t xv = load4(a.x + i);
    s0 = dot4(q0, xv, s0);
    s1 = dot4(q1, xv, s1);
    s2 = dot4(q2, xv, s2);
    s3 = dot4(q3, xv, s3);
  }
  const float s = wave_sum4(s0, s1, s2, s3, lane);
  if ((lane & 15) == 0) {
    const int r = r0 + (lane >> 4);
    const float pre = s + a.b1[static_cast<int64_t>(e) * a.hidden + r];
    a.h[static_cast<int64_t>(k) * a.hidden + r] = 0.5f * pre * (1.f + erff(pre * 0.70710678118654752440f));
  }
}

// grid = ceil(dim / 4); each wave owns one output element and reads that row
// of every selected expert's W2 at once.
template <int K>
__global__ __launch_bounds__(256) void moe_w2_reduce_kernel(MoeArgs a) {
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int j = blockIdx.x * 4 + wave;
  if (j >= a.dim) return;
  int e[K];
  const float* __restrict__ row[K];
#pragma unroll
  for (int s = 0; s < K; ++s) {
    e[s] = a.ids[s];
    row[s] = a.w2 + (static_cast<int64_t>(e[s]) * a.dim + j) * a.hidden;
  }
  float acc[K];
#pragma unroll
  for (int s = 0; s < K; ++s) acc[s] = 0.f;
#pragma unroll 2
  for (int i = lane * 4; i < a.hidden; i += 256) {
    f32x4_t q[K];
#pragma unroll
    for (int s = 0; s < K; ++s) q[s] = stream4(row[s] + i);
#pragma unroll
    for (int s = 0; s < K; ++s) acc[s] = dot4(q[s], load4(a.h + static_cast<int64_t>(s) * a.hidden + i), acc[s]);
  }
#pragma unroll
  for (int s = 0; s < K; ++s) acc[s] = mie::wave_sum(acc[s]);
  if (lane != 0) return;
  // Slots in increasing expert id (ids are distinct): slot s goes rank[s]-th.
  int rank[K];
#pragma unroll
  for (int s = 0; s < K; ++s) {
    rank[s] = 0;
#pragma unroll
    for (int t = 0; t < K; ++t) rank[s] += e[t] < e[s];
  }
  float out = 0.f;
#pragma unroll
  for (int r = 0; r < K; ++r) {
#pragma unroll
    for (int s = 0; s < K; ++s) {
      if (rank[s] == r) {
        const float y = acc[s] + a.b2[static_cast<int64_t>(e[s]) * a.dim + j];
        out = __fadd_rn(out, __fmul_rn(a.weights[s], y));
      }
    }
  }
  a.out[j] = out;
}

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

int32_t check_route_args(const char* who, const void* x, const void* router_weight, int32_t num_experts,
                         int32_t top_k, int32_t dim, const void* logits, const void* ids, const void* weights,
                         int32_t dtype) {
  if (dtype != MIE_DTYPE_F32) return mie::fail(MIE_ERR_UNSUPPORTED, "%s: float32 only", who);
  if (num_experts <= 0 || num_experts > kMaxExperts || top_k <= 0 || top_k > kMaxTopK || top_k > num_experts)
    return mie::fail(MIE_ERR_INVALID, "%s: experts=%d top_k=%d (at most %d and %d)", who, num_experts, top_k,
                     kMaxExperts, kMaxTopK);
  if (dim <= 0 || dim % 4 != 0) return mie::fail(MIE_ERR_INVALID, "%s: dim=%d must be a positive multiple of 4", who, dim);
  if (!x || !router_weight || !logits || !ids || !weights) return mie::fail(MIE_ERR_INVALID, "%s: null pointer", who);
  if (!aligned16(x) || !aligned16(router_weight))
    return mie::fail(MIE_ERR_INVALID, "%s: x and the router weight must be 16-byte aligned", who);
  return MIE_OK;
}

MoeArgs make_args(const void* x, const void* router_weight, int32_t num_experts, int32_t top_k, int32_t dim,
                  int32_t hidden, void* logits, void* ids, void* weights) {
  MoeArgs a{};
  a.x = static_cast<const float*>(x);
  a.router = static_cast<const float*>(router_weight);
  a.E = num_experts;
  a.top_k = top_k;
  a.dim = dim;
  a.hidden = hidden;
  a.logits = static_cast<float*>(logits);
  a.ids = static_cast<int32_t*>(ids);
  a.weights = static_cast<float*>(weights);
  return a;
}

template <int K>
void launch_w2(const MoeArgs& a, hipStream_t st) {
  moe_w2_reduce_kernel<K><<<(a.dim + 3) / 4, 256, 0, st>>>(a);
}

}  // namespace

extern "C" int32_t mie_moe_route(const void* x, const void* router_weight, int32_t num_experts, int32_t top_k,
                                 int32_t dim, void* router_logits, void* expert_ids, void* route_weights,
                                 int32_t dtype, void* stream) {
  int32_t rc = check_route_args("mie_moe_route", x, router_weight, num_experts, top_k, dim, router_logits,
                                expert_ids, route_weights, dtype);
  if (rc != MIE_OK) return rc;
  const MoeArgs a = make_args(x, router_weight, num_experts, top_k, dim, 0, router_logits, expert_ids, route_weights);
  moe_route_kernel<<<1, 256, 0, static_cast<hipStream_t>(stream)>>>(a);
  return mie::check_launch("moe_route_kernel");
}

extern "C" int32_t mie_moe_decode(const void* x, const void* router_weight, const void* w1, const void* b1,
                                  const void* w2, const void* b2, int32_t num_experts, int32_t top_k, int32_t dim,
                                  int32_t hidden, void* router_logits, void* expert_ids, void* route_weights,
                                  void* hidden_act, void* out, int32_t dtype, void* stream) {
  int32_t rc = check_route_args("mie_moe_decode", x, router_weight, num_experts, top_k, dim, router_logits,
                                expert_ids, route_weights, dtype);
  if (rc != MIE_OK) return rc;
  if (hidden <= 0 || hidden % 4 != 0)
    return mie::fail(MIE_ERR_INVALID, "mie_moe_decode: hidden=%d must be a positive multiple of 4", hidden);
  if (!w1 || !b1 || !w2 || !b2 || !hidden_act || !out) return mie::fail(MIE_ERR_INVALID, "mie_moe_decode: null pointer");
  if (!aligned16(w1) || !aligned16(w2) || !aligned16(hidden_act))
    return mie::fail(MIE_ERR_INVALID, "mie_moe_decode: W1, W2 and the hidden buffer must be 16-byte aligned");
  MoeArgs a = make_args(x, router_weight, num_experts, top_k, dim, hidden, router_logits, expert_ids, route_weights);
  a.w1 = static_cast<const float*>(w1);
  a.b1 = static_cast<const float*>(b1);
  a.w2 = static_cast<const float*>(w2);
  a.b2 = static_cast<const float*>(b2);
  a.h = static_cast<float*>(hidden_act);
  a.out = static_cast<float*>(out);
  hipStream_t st = static_cast<hipStream_t>(stream);
  moe_route_kernel<<<1, 256, 0, st>>>(a);
  rc = mie::check_launch("moe_route_kernel");
  if (rc != MIE_OK) return rc;
  moe_w1_gelu_kernel<<<dim3((hidden + 15) / 16, top_k), 256, 0, st>>>(a);
  rc = mie::check_launch("moe_w1_gelu_kernel");
  if (rc != MIE_OK) return rc;
  switch (top_k) {
    case 1: launch_w2<1>(a, st); break;
    case 2: launch_w2<2>(a, st); break;
    case 3: launch_w2<3>(a, st); break;
    case 4: launch_w2<4>(a, st); break;
    case 5: launch_w2<5>(a, st); break;
    case 6: launch_w2<6>(a, st); break;
    case 7: launch_w2<7>(a, st); break;
    default: launch_w2<8>(a, st); break;
  }
  return mie::check_launch("moe_w2_reduce_kernel");
}
