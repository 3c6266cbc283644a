// Fused top-k mixture-of-experts for one decode token (float32 or bfloat16),
// no host sync.
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
// Storage is float32 or bfloat16 (weights, x, the GELU activations and the
// output; the routing logits and weights are float32 in both, as the
// reference keeps routing in float32, model.py:448-452).  Every product and
// sum runs in float32.  For bfloat16 each result is rounded where the
// reference's PyTorch path stores a bfloat16 tensor: the norm's output, each
// Linear's output (its float32 sum plus bias, rounded once), GELU's, the
// route weight, the weighted product and each partial sum of index_add_, and
// the residual add.  For float32 none of these roundings changes a value.
//
// Expert weights live in four canonical contiguous storages - W1 [E, hidden,
// dim], b1 [E, hidden], W2 [E, dim, hidden], b2 [E, dim] - so a selected
// expert is a device-side offset; the route never leaves the GPU.
//
// Two launches.  Every W1 workgroup computes the routing itself (x into LDS,
// the E router dot products, top-k) - the router is 24 KiB at E = 8, d = 768
// and stays in L2 - so no launch waits on a separate route kernel; workgroup
// (0, 0) writes the routing outputs, which the W2 launch reads.  The block
// form also folds in the block's norm (out = x + MoE(LayerNorm(x)),
// model.py:494-498): the norm goes into W1's LDS staging and the residual add
// into W2's store.
//
// The GEMVs are HBM-bound (2 * top_k * dim * hidden * 4 bytes per token,
// ~12.6 MB at d 768 / FFN 2048 / top-2): each wave issues all of its weight
// loads (non-temporal: a token's experts are streamed once) before it
// reduces, so a launch keeps the whole working set in flight.
#include <math.h>

#include "mie_common.h"

namespace {

constexpr int kMaxExperts = 64;
constexpr int kMaxTopK = 8;
constexpr int kMaxDim = 2048;  // the W1 kernel holds x in 8 four-element loads per lane
// W2 kernel: four-element loads per lane per slot per round, 8 for top-1 and
// top-2 and 16 / K beyond, so a round holds 16 weight and 16 hidden loads.
template <int K>
constexpr int kW2Chunks = K <= 2 ? 8 : (16 / K > 0 ? 16 / K : 1);

typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef long long i64x2_t __attribute__((ext_vector_type(2)));

using mie::Mem;

// Pointers marked T hold the storage type (float32 or bfloat16).
struct MoeArgs {
  const void* x;       // T [dim]
  const void* router;  // T [E, dim]
  const void* w1;      // T [E, hidden, dim]
  const void* b1;      // T [E, hidden]
  const void* w2;      // T [E, dim, hidden]
  const void* b2;      // T [E, dim]
  int32_t E, top_k, dim, hidden;
  const void* ln_w;      // T; block form: norm weight [dim] (NULL: no norm)
  const void* ln_b;      // T; block form: norm bias [dim] or NULL
  float ln_eps;
  const void* residual;  // T; block form: x, added to the output
  // Accumulator form (after mie_attn_out_acc): the block's input to the MoE
  // half is h = x + (acc * 2^-32 + b_out), formed in the W1 launch (h_out
  // written by workgroup (0, 0)); the W2 launch adds h_out as the residual
  // and clears acc for the next token.
  const unsigned long long* acc;  // [dim + 1]; acc[dim] != 0: a partial was not representable
  const void* b_out;              // T [dim] or NULL
  void* h_out;                    // T [dim]
  unsigned long long* acc_clear;  // W2: acc to clear, or NULL
  float* logits;   // float32 [E]
  int32_t* ids;    // [top_k], largest logit first
  float* weights;  // float32 [top_k], same order
  void* h;         // T [top_k, hidden], same order
  void* out;       // T [dim]
};

__device__ __forceinline__ float dot4(f32x4_t a, f32x4_t b, float s) {
  s = fmaf(a.x, b.x, s);
  s = fmaf(a.y, b.y, s);
  s = fmaf(a.z, b.z, s);
  return fmaf(a.w, b.w, s);
}

// Dot product of a row with a vector over one wavefront (four elements per
// lane per step), in float32.
template <typename T>
__device__ __forceinline__ float wave_dot(const T* __restrict__ row, const T* __restrict__ v, int n, int lane) {
  float s = 0.f;
  for (int i = lane * 4; i < n; i += 256) s = dot4(Mem<T>::load4(row + i), Mem<T>::load4(v + i), s);
  return mie::wave_sum(s);
}

// (v, i) against (ov, oi): the larger logit wins, the lower expert id on
// ties, and NaN counts as larger than every number (torch.topk's order) - a
// total order, so any reduction tree gives the same pick, and a NaN logit is
// picked like any other, so the pick is always an expert that is not yet
// taken (a taken expert holds -inf and an id past 63).  Compares and selects,
// no branches.
__device__ __forceinline__ void topk_take(float& v, int& i, float ov, int oi) {
  const bool v_nan = v != v, o_nan = ov != ov;
  const bool lower = oi < i;
  // ov > v and ov == v are false when either is NaN.
  const bool b = (o_nan & (!v_nan | lower)) | (ov > v) | ((ov == v) & lower);
  v = b ? ov : v;
  i = b ? oi : i;
}

template <int CTRL>
__device__ __forceinline__ void topk_dpp(float& v, int& i) {
  topk_take(v, i, mie::dpp<CTRL>(v), __builtin_amdgcn_update_dpp(0, i, CTRL, 0xF, 0xF, false));
}

// Top-k over a wave: lane e holds expert e's logit (-inf for lanes >= E).
// Round kk takes the largest logit not yet taken, the lower expert id on ties;
// ids and weights (the softmax of the selected logits) come out uniform across
// the wave.  Fixed-size loops keep both arrays in registers.
__device__ __forceinline__ void wave_topk(float logit, int top_k, int num_experts, int lane, int* ids,
                                          float* weights) {
  bool taken = false;
  float vals[kMaxTopK];
#pragma unroll
  for (int kk = 0; kk < kMaxTopK; ++kk) {
    ids[kk] = 0;
    vals[kk] = 0.f;
    if (kk < top_k) {
      // A taken expert also loses every tie, so a repeated -inf cannot pick it twice.
      float v = taken ? -INFINITY : logit;
      int idx = taken ? lane + 64 : lane;
      // Only the lanes holding experts take part: DPP stages over 2, 4, 8 and
      // 16 lanes (quad xor-1 and xor-2, then half-row and row mirrors), then
      // cross-row exchanges for more than 16 experts.
      topk_dpp<0xB1>(v, idx);
      topk_dpp<0x4E>(v, idx);
      if (num_experts > 4) topk_dpp<0x141>(v, idx);
      if (num_experts > 8) topk_dpp<0x140>(v, idx);
      if (num_experts > 16) topk_take(v, idx, __shfl_xor(v, 16), __shfl_xor(idx, 16));
      if (num_experts > 32) topk_take(v, idx, __shfl_xor(v, 32), __shfl_xor(idx, 32));
      // Lane 0 holds the pick; every lane takes it from a scalar register.
      idx = __builtin_amdgcn_readfirstlane(idx);
      v = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v)));
      ids[kk] = idx;
      vals[kk] = v;
      taken = taken || lane == idx;
    }
  }
  // softmax over the selected logits; vals[0] is their maximum
  float sum = 0.f;
#pragma unroll
  for (int kk = 0; kk < kMaxTopK; ++kk) {
    weights[kk] = kk < top_k ? expf(vals[kk] - vals[0]) : 0.f;
    sum += weights[kk];
  }
#pragma unroll
  for (int kk = 0; kk < kMaxTopK; ++kk) weights[kk] /= sum;
}

// One workgroup: E router dot products, then top-k and softmax on wave 0.
template <typename T>
__global__ __launch_bounds__(256) void moe_route_kernel(MoeArgs a) {
  __shared__ float logits[kMaxExperts];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const T* router = static_cast<const T*>(a.router);
  for (int e = wave; e < a.E; e += 4) {
    const float s = wave_dot(router + static_cast<int64_t>(e) * a.dim, static_cast<const T*>(a.x), a.dim, lane);
    if (lane == 0) {
      logits[e] = s;
      a.logits[e] = s;
    }
  }
  __syncthreads();
  if (wave != 0) return;
  int ids[kMaxTopK];
  float p[kMaxTopK];
  wave_topk(lane < a.E ? logits[lane] : -INFINITY, a.top_k, a.E, lane, ids, p);
#pragma unroll
  for (int kk = 0; kk < kMaxTopK; ++kk) {
    if (kk < a.top_k && lane == kk) {
      a.ids[kk] = ids[kk];
      a.weights[kk] = p[kk];
    }
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

// grid = (ceil(hidden / 16), top_k), 256 threads; NCH = ceil(dim / 256)
// 16-byte loads per lane.  Each wave loads x (and the norm parameters) in the
// lane layout of its dot products and normalises with wave reductions, and
// loads the router rows of experts wave and wave + 4; the logits meet in LDS
// behind the kernel's one barrier, every wave takes the top-k itself, then
// computes 4 rows of slot blockIdx.y's expert.  hidden % 4 == 0, so a wave's
// rows are all valid or all past the end.
template <typename T, int NCH, bool NORM, bool ACC = false>
__global__ __launch_bounds__(256) void moe_w1_gelu_kernel(MoeArgs a) {
  using M = Mem<T>;
  __shared__ float s_logits[kMaxExperts];
  const T* __restrict__ xs = static_cast<const T*>(a.x);
  const T* __restrict__ router = static_cast<const T*>(a.router);
  const T* __restrict__ ln_w = static_cast<const T*>(a.ln_w);
  const T* __restrict__ ln_b = static_cast<const T*>(a.ln_b);
  const int k = blockIdx.y;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int dim = a.dim;
  const int e0 = wave, e1 = wave + 4;

  // 1. All global reads that do not depend on the routing, in one memory
  //    round.  The vectors every wave needs - x (with the attention's sums
  //    and out_proj's bias, h) and the norm's weight and bias - are read
  //    once per workgroup: wave w reads chunks w, w + 4, ... of them, forms h
  //    there and leaves the three chunks in LDS, where every wave picks up the
  //    whole vectors in its own lane layout after the barrier.  Each wave's
  //    two router rows go out after its share, so waiting for the share does
  //    not wait for them.
  __shared__ __align__(16) float s_vec[3][kMaxDim];  // h, norm weight, norm bias
  f32x4_t y[NCH], gw[NCH], gb[NCH], q0[NCH], q1[NCH];
  const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};
  constexpr int NS = (NCH + 3) / 4;  // chunks of the shared vectors per wave
  constexpr int NA = ACC ? NS : 1;
  typename M::raw4 ry[NS], rgw[NS], rgb[NS], bo[NA];
  i64x2_t acc_lo[NA], acc_hi[NA];
  long long acc_flag = 0;
  const typename M::raw4 zr = M::zero_raw();
#pragma unroll
  for (int u = 0; u < NS; ++u) {
    const int c = wave + 4 * u;
    const int i = c * 256 + lane * 4;
    const int ic = c < NCH && i < dim ? i : 0;  // in bounds; dropped below
    ry[u] = M::load_raw(xs + ic);
    rgw[u] = NORM ? M::load_raw(ln_w + ic) : zr;
    // Without a norm bias the weight is read in its place (a valid address,
    // so no branch splits the round) and the value is dropped below.
    rgb[u] = NORM ? M::load_raw((ln_b ? ln_b : ln_w) + ic) : zr;
    if constexpr (ACC) {
      bo[u] = M::load_raw((a.b_out ? static_cast<const T*>(a.b_out) : xs) + ic);
      acc_lo[u] = *reinterpret_cast<const i64x2_t*>(a.acc + ic);
      acc_hi[u] = *reinterpret_cast<const i64x2_t*>(a.acc + ic + 2);
    }
  }
  if constexpr (ACC) acc_flag = *reinterpret_cast<const long long*>(a.acc + dim);
  {
    typename M::raw4 rq0[NCH], rq1[NCH];
    // Rows past E and columns past dim read row 0, column 0 (in bounds) and
    // are zeroed once loaded: a load under a branch would make the wave wait
    // for every load issued before it at the join.
    const int r0 = e0 < a.E ? e0 : 0, r1 = e1 < a.E ? e1 : 0;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int i = c * 256 + lane * 4;
      const int ic = i < dim ? i : 0;
      rq0[c] = M::load_raw(router + static_cast<int64_t>(r0) * dim + ic);
      rq1[c] = M::load_raw(router + static_cast<int64_t>(r1) * dim + ic);
    }
    // Keep the scheduler from sinking any of these loads below the first use
    // of the ones before them (which would cost a memory round).
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const bool valid = c * 256 + lane * 4 < dim;
      q0[c] = valid && e0 < a.E ? M::widen(rq0[c]) : zero;
      q1[c] = valid && e1 < a.E ? M::widen(rq1[c]) : zero;
    }
  }
  // h = x + (acc * 2^-32 + b_out) in the accumulator form: the attention
  // output projection summed over heads in fixed point (int64 -> float is one
  // rounding, the power of two scale is exact), its bias, then the residual -
  // the rounding points of x + out_proj(a): the projection's output, then the
  // sum, each rounded to the storage type.  Otherwise h = x.
#pragma unroll
  for (int u = 0; u < NS; ++u) {
    const int c = wave + 4 * u;
    if (c >= NCH) continue;
    const int i = c * 256 + lane * 4;
    f32x4_t hv = M::widen(ry[u]);
    if constexpr (ACC) {
      f32x4_t o = {static_cast<float>(acc_lo[u].x), static_cast<float>(acc_lo[u].y),
                   static_cast<float>(acc_hi[u].x), static_cast<float>(acc_hi[u].y)};
      o *= 2.3283064365386963e-10f;  // 2^-32
      if (a.b_out) o += M::widen(bo[u]);
      hv = M::R4(hv + M::R4(o));
      if (acc_flag != 0) hv = f32x4_t{NAN, NAN, NAN, NAN};
      if (blockIdx.x == 0 && blockIdx.y == 0 && i < dim) M::put4(static_cast<T*>(a.h_out) + i, hv);
    }
    const bool valid = i < dim;
    *reinterpret_cast<f32x4_t*>(&s_vec[0][i]) = valid ? hv : zero;
    *reinterpret_cast<f32x4_t*>(&s_vec[1][i]) = valid ? M::widen(rgw[u]) : zero;
    *reinterpret_cast<f32x4_t*>(&s_vec[2][i]) = valid && ln_b ? M::widen(rgb[u]) : zero;
  }
  __syncthreads();
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int i = c * 256 + lane * 4;
    y[c] = *reinterpret_cast<const f32x4_t*>(&s_vec[0][i]);
    gw[c] = *reinterpret_cast<const f32x4_t*>(&s_vec[1][i]);
    gb[c] = *reinterpret_cast<const f32x4_t*>(&s_vec[2][i]);
  }

  // 2. The block's LayerNorm (float32, biased variance), per wave.
  if constexpr (NORM) {
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) s += y[c].x + y[c].y + y[c].z + y[c].w;
    const float mean = mie::wave_sum(s) / dim;
    float q = 0.f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      if (c * 256 + lane * 4 < dim) {
        const f32x4_t d = y[c] - mean;
        q = dot4(d, d, q);
      }
    }
    const float rstd = rsqrtf(mie::wave_sum(q) / dim + a.ln_eps);
#pragma unroll
    // The norm's output is what the reference feeds the router and the
    // experts: rounded to the storage type.
    for (int c = 0; c < NCH; ++c) y[c] = M::R4((y[c] - mean) * rstd * gw[c] + gb[c]);
  }

  // 3. Router logits: experts wave and wave + 4 from registers, any others
  //    (E > 8) loaded now.
  {
    float l0 = 0.f, l1 = 0.f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      l0 = dot4(q0[c], y[c], l0);
      l1 = dot4(q1[c], y[c], l1);
    }
    l0 = mie::wave_sum(l0);
    l1 = mie::wave_sum(l1);
    if (lane == 0) {
      if (e0 < a.E) s_logits[e0] = l0;
      if (e1 < a.E) s_logits[e1] = l1;
    }
    for (int e = wave + 8; e < a.E; e += 4) {
      float l = 0.f;
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        const int i = c * 256 + lane * 4;
        if (i < dim) l = dot4(M::load4(router + static_cast<int64_t>(e) * dim + i), y[c], l);
      }
      l = mie::wave_sum(l);
      if (lane == 0) s_logits[e] = l;
    }
  }
  __syncthreads();

  // 4. Top-k in every wave; workgroup (0, 0) publishes the routing.
  int ids[kMaxTopK];
  float p[kMaxTopK];
  const float logit = lane < a.E ? s_logits[lane] : -INFINITY;
  wave_topk(logit, a.top_k, a.E, lane, ids, p);
  if (blockIdx.x == 0 && blockIdx.y == 0 && wave == 0) {
    if (lane < a.E) a.logits[lane] = logit;
#pragma unroll
    for (int kk = 0; kk < kMaxTopK; ++kk) {
      if (kk < a.top_k && lane == kk) {
        a.ids[kk] = ids[kk];
        a.weights[kk] = p[kk];
      }
    }
  }
  int e = ids[0];
#pragma unroll
  for (int kk = 1; kk < kMaxTopK; ++kk) e = kk == k ? ids[kk] : e;

  // 5. Four rows of the selected expert's W1, GELU, into h[k].
  const int r0 = (blockIdx.x * 4 + wave) * 4;
  if (r0 >= a.hidden) return;
  const T* __restrict__ w = static_cast<const T*>(a.w1) + (static_cast<int64_t>(e) * a.hidden + r0) * dim;
  // The bias of the row this lane stores, read with the weights rather than
  // after the reduction.
  const int r_out = r0 + (lane >> 4);
  const float bias = (lane & 15) == 0 && r_out < a.hidden
                         ? M::get(static_cast<const T*>(a.b1) + static_cast<int64_t>(e) * a.hidden + r_out)
                         : 0.f;
  // All 4 x NCH row loads go out before the first multiply: unconditional,
  // with lanes past dim reading element 0 (y is zero there, and the product
  // is dropped below), since a load under a branch makes the compiler wait
  // for it before the next one.
  typename M::raw4 wv[4][NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int i = c * 256 + lane * 4;
    const int ic = i < dim ? i : 0;
#pragma unroll
    for (int r = 0; r < 4; ++r) wv[r][c] = M::stream_raw(w + r * dim + ic);
  }
  float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    if (c * 256 + lane * 4 < dim) {
      s0 = dot4(M::widen(wv[0][c]), y[c], s0);
      s1 = dot4(M::widen(wv[1][c]), y[c], s1);
      s2 = dot4(M::widen(wv[2][c]), y[c], s2);
      s3 = dot4(M::widen(wv[3][c]), y[c], s3);
    }
  }
  const float t = wave_sum4(s0, s1, s2, s3, lane);
  if ((lane & 15) == 0) {
    const float pre = M::R(t + bias);  // the Linear's output
    M::put(static_cast<T*>(a.h) + static_cast<int64_t>(k) * a.hidden + r_out,
           0.5f * pre * (1.f + erff(pre * 0.70710678118654752440f)));
  }
}

// grid = ceil(dim / 4); each wave owns one output element and reads that row
// of every selected expert's W2 at once.
template <typename T, int K, bool RESID>
__global__ __launch_bounds__(256) void moe_w2_reduce_kernel(MoeArgs a) {
  using M = Mem<T>;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int j = blockIdx.x * 4 + wave;
  if (j >= a.dim) return;
  int e[K];
  float wt[K], bias[K];
  const T* __restrict__ row[K];
  const T* __restrict__ hs = static_cast<const T*>(a.h);
#pragma unroll
  for (int s = 0; s < K; ++s) {
    e[s] = a.ids[s];
    row[s] = static_cast<const T*>(a.w2) + (static_cast<int64_t>(e[s]) * a.dim + j) * a.hidden;
  }
  // The epilogue's reads go out with the row loads, not after the reduction.
#pragma unroll
  for (int s = 0; s < K; ++s) {
    wt[s] = a.weights[s];
    bias[s] = M::get(static_cast<const T*>(a.b2) + static_cast<int64_t>(e[s]) * a.dim + j);
  }
  const float res = RESID ? M::get(static_cast<const T*>(a.residual) + j) : 0.f;
  if (a.acc_clear && lane == 0) {
    // The attention's fixed-point sums were consumed by the W1 launch: ready
    // for the next token.
    a.acc_clear[j] = 0ull;
    if (j == 0) a.acc_clear[a.dim] = 0ull;
  }
  float acc[K];
#pragma unroll
  for (int s = 0; s < K; ++s) acc[s] = 0.f;
  // Rounds of kW2Chunks<K> 16-byte chunks per lane, every load of a round issued
  // before its first multiply: one memory latency per 256 * kW2Chunks<K> hidden
  // values (one round at FFN width 2048).  Each lane still accumulates its
  // chunks in increasing order.
  for (int i0 = lane * 4; i0 < a.hidden; i0 += 256 * kW2Chunks<K>) {
    typename M::raw4 q[K][kW2Chunks<K>], hv[K][kW2Chunks<K>];
#pragma unroll
    for (int u = 0; u < kW2Chunks<K>; ++u) {
      const int i = i0 + u * 256;
      const bool valid = i < a.hidden;
#pragma unroll
      for (int s = 0; s < K; ++s) {
        q[s][u] = valid ? M::stream_raw(row[s] + i) : M::zero_raw();
        hv[s][u] = valid ? M::load_raw(hs + static_cast<int64_t>(s) * a.hidden + i) : M::zero_raw();
      }
    }
#pragma unroll
    for (int u = 0; u < kW2Chunks<K>; ++u) {
      if (i0 + u * 256 >= a.hidden) break;
#pragma unroll
      for (int s = 0; s < K; ++s) acc[s] = dot4(M::widen(q[s][u]), M::widen(hv[s][u]), acc[s]);
    }
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
        // The expert's output (its Linear's, rounded), the route weight in
        // the storage type, their product, and the running sum, each rounded
        // as index_add_ stores it.
        const float y = M::R(acc[s] + bias[s]);
        out = M::R(__fadd_rn(out, M::R(__fmul_rn(M::R(wt[s]), y))));
      }
    }
  }
  M::put(static_cast<T*>(a.out) + j, RESID ? __fadd_rn(res, out) : out);
}

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

int32_t check_route_args(const char* who, const void* x, const void* router_weight, int32_t num_experts,
                         int32_t top_k, int32_t dim, const void* logits, const void* ids, const void* weights,
                         int32_t dtype) {
  if (dtype != MIE_DTYPE_F32 && dtype != MIE_DTYPE_BF16)
    return mie::fail(MIE_ERR_UNSUPPORTED, "%s: float32 or bfloat16 only (dtype %d)", who, dtype);
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
  a.x = x;
  a.router = router_weight;
  a.E = num_experts;
  a.top_k = top_k;
  a.dim = dim;
  a.hidden = hidden;
  a.logits = static_cast<float*>(logits);
  a.ids = static_cast<int32_t*>(ids);
  a.weights = static_cast<float*>(weights);
  return a;
}

template <typename T, int K>
void launch_w2(const MoeArgs& a, hipStream_t st) {
  if (a.residual) {
    moe_w2_reduce_kernel<T, K, true><<<(a.dim + 3) / 4, 256, 0, st>>>(a);
  } else {
    moe_w2_reduce_kernel<T, K, false><<<(a.dim + 3) / 4, 256, 0, st>>>(a);
  }
}

}  // namespace

extern "C" int32_t mie_moe_route(const void* x, const void* router_weight, int32_t num_experts, int32_t top_k,
                                 int32_t dim, void* router_logits, void* expert_ids, void* route_weights,
                                 int32_t dtype, void* stream) {
  int32_t rc = check_route_args("mie_moe_route", x, router_weight, num_experts, top_k, dim, router_logits,
                                expert_ids, route_weights, dtype);
  if (rc != MIE_OK) return rc;
  const MoeArgs a = make_args(x, router_weight, num_experts, top_k, dim, 0, router_logits, expert_ids, route_weights);
  if (dtype == MIE_DTYPE_F32) {
    moe_route_kernel<float><<<1, 256, 0, static_cast<hipStream_t>(stream)>>>(a);
  } else {
    moe_route_kernel<uint16_t><<<1, 256, 0, static_cast<hipStream_t>(stream)>>>(a);
  }
  return mie::check_launch("moe_route_kernel");
}

namespace {

int32_t check_expert_args(const char* who, int32_t hidden, int32_t dim, const void* w1, const void* b1,
                          const void* w2, const void* b2, const void* hidden_act, const void* out) {
  if (hidden <= 0 || hidden % 4 != 0)
    return mie::fail(MIE_ERR_INVALID, "%s: hidden=%d must be a positive multiple of 4", who, hidden);
  if (dim > kMaxDim) return mie::fail(MIE_ERR_UNSUPPORTED, "%s: dim %d above %d", who, dim, kMaxDim);
  if (!w1 || !b1 || !w2 || !b2 || !hidden_act || !out) return mie::fail(MIE_ERR_INVALID, "%s: null pointer", who);
  if (!aligned16(w1) || !aligned16(w2) || !aligned16(hidden_act))
    return mie::fail(MIE_ERR_INVALID, "%s: W1, W2 and the hidden buffer must be 16-byte aligned", who);
  return MIE_OK;
}

template <typename T, int NCH>
void launch_w1(const MoeArgs& a, hipStream_t st) {
  const dim3 grid((a.hidden + 15) / 16, a.top_k);
  if (a.acc) {
    if (a.ln_w) {
      moe_w1_gelu_kernel<T, NCH, true, true><<<grid, 256, 0, st>>>(a);
    } else {
      moe_w1_gelu_kernel<T, NCH, false, true><<<grid, 256, 0, st>>>(a);
    }
    return;
  }
  if (a.ln_w) {
    moe_w1_gelu_kernel<T, NCH, true><<<grid, 256, 0, st>>>(a);
  } else {
    moe_w1_gelu_kernel<T, NCH, false><<<grid, 256, 0, st>>>(a);
  }
}

template <typename T>
int32_t launch_experts_as(const MoeArgs& a, hipStream_t st) {
  switch ((a.dim + 255) / 256) {
    case 1: launch_w1<T, 1>(a, st); break;
    case 2: launch_w1<T, 2>(a, st); break;
    case 3: launch_w1<T, 3>(a, st); break;
    case 4: launch_w1<T, 4>(a, st); break;
    case 5: launch_w1<T, 5>(a, st); break;
    case 6: launch_w1<T, 6>(a, st); break;
    case 7: launch_w1<T, 7>(a, st); break;
    default: launch_w1<T, 8>(a, st); break;
  }
  int32_t rc = mie::check_launch("moe_w1_gelu_kernel");
  if (rc != MIE_OK) return rc;
  switch (a.top_k) {
    case 1: launch_w2<T, 1>(a, st); break;
    case 2: launch_w2<T, 2>(a, st); break;
    case 3: launch_w2<T, 3>(a, st); break;
    case 4: launch_w2<T, 4>(a, st); break;
    case 5: launch_w2<T, 5>(a, st); break;
    case 6: launch_w2<T, 6>(a, st); break;
    case 7: launch_w2<T, 7>(a, st); break;
    default: launch_w2<T, 8>(a, st); break;
  }
  return mie::check_launch("moe_w2_reduce_kernel");
}

// dtype was checked: float32 or bfloat16.
int32_t launch_experts(const MoeArgs& a, int32_t dtype, hipStream_t st) {
  return dtype == MIE_DTYPE_F32 ? launch_experts_as<float>(a, st) : launch_experts_as<uint16_t>(a, st);
}

}  // namespace

extern "C" int32_t mie_moe_decode(const void* x, const void* router_weight, const void* w1, const void* b1,
                                  const void* w2, const void* b2, int32_t num_experts, int32_t top_k, int32_t dim,
                                  int32_t hidden, void* router_logits, void* expert_ids, void* route_weights,
                                  void* hidden_act, void* out, int32_t dtype, void* stream) {
  int32_t rc = check_route_args("mie_moe_decode", x, router_weight, num_experts, top_k, dim, router_logits,
                                expert_ids, route_weights, dtype);
  if (rc != MIE_OK) return rc;
  rc = check_expert_args("mie_moe_decode", hidden, dim, w1, b1, w2, b2, hidden_act, out);
  if (rc != MIE_OK) return rc;
  MoeArgs a = make_args(x, router_weight, num_experts, top_k, dim, hidden, router_logits, expert_ids, route_weights);
  a.w1 = w1;
  a.b1 = b1;
  a.w2 = w2;
  a.b2 = b2;
  a.h = hidden_act;
  a.out = out;
  return launch_experts(a, dtype, static_cast<hipStream_t>(stream));
}

namespace mie {

int32_t moe_decode_block_check(const void* x, const void* ln_weight, const void* ln_bias, const void* router_weight,
                               const void* w1, const void* b1, const void* w2, const void* b2, int32_t num_experts,
                               int32_t top_k, int32_t dim, int32_t hidden, const void* router_logits,
                               const void* expert_ids, const void* route_weights, const void* hidden_act,
                               const void* out, int32_t dtype) {
  int32_t rc = check_route_args("mie_moe_decode_block", x, router_weight, num_experts, top_k, dim, router_logits,
                                expert_ids, route_weights, dtype);
  if (rc != MIE_OK) return rc;
  rc = check_expert_args("mie_moe_decode_block", hidden, dim, w1, b1, w2, b2, hidden_act, out);
  if (rc != MIE_OK) return rc;
  if (!ln_weight && ln_bias) return mie::fail(MIE_ERR_INVALID, "mie_moe_decode_block: a norm bias needs a weight");
  return MIE_OK;
}

int32_t moe_decode_block_acc_check(const void* x, const void* acc, const void* b_out, const void* h_out,
                                   const void* ln_weight, const void* ln_bias, const void* router_weight,
                                   const void* w1, const void* b1, const void* w2, const void* b2,
                                   int32_t num_experts, int32_t top_k, int32_t dim, int32_t hidden,
                                   const void* router_logits, const void* expert_ids, const void* route_weights,
                                   const void* hidden_act, const void* out, int32_t dtype) {
  const int32_t rc = moe_decode_block_check(x, ln_weight, ln_bias, router_weight, w1, b1, w2, b2, num_experts,
                                            top_k, dim, hidden, router_logits, expert_ids, route_weights,
                                            hidden_act, out, dtype);
  if (rc != MIE_OK) return rc;
  if (!acc || !h_out || reinterpret_cast<uintptr_t>(acc) % 16 || !aligned16(h_out) || !aligned16(b_out))
    return mie::fail(MIE_ERR_INVALID, "mie_moe_decode_block_acc: acc and h_out (and b_out) must be non-NULL and "
                                      "16-byte aligned");
  if (h_out == x)
    return mie::fail(MIE_ERR_INVALID, "mie_moe_decode_block_acc: h_out must not alias x (the W1 launch reads x "
                                      "while it writes h_out)");
  return MIE_OK;
}

}  // namespace mie

extern "C" int32_t mie_moe_decode_block(const void* x, const void* ln_weight, const void* ln_bias, float ln_eps,
                                        const void* router_weight, const void* w1, const void* b1, const void* w2,
                                        const void* b2, int32_t num_experts, int32_t top_k, int32_t dim,
                                        int32_t hidden, void* router_logits, void* expert_ids, void* route_weights,
                                        void* hidden_act, void* out, int32_t dtype, void* stream) {
  const int32_t rc = mie::moe_decode_block_check(x, ln_weight, ln_bias, router_weight, w1, b1, w2, b2, num_experts,
                                                 top_k, dim, hidden, router_logits, expert_ids, route_weights,
                                                 hidden_act, out, dtype);
  if (rc != MIE_OK) return rc;
  MoeArgs a = make_args(x, router_weight, num_experts, top_k, dim, hidden, router_logits, expert_ids, route_weights);
  a.ln_w = ln_weight;
  a.ln_b = ln_bias;
  a.ln_eps = ln_eps;
  a.residual = x;
  a.w1 = w1;
  a.b1 = b1;
  a.w2 = w2;
  a.b2 = b2;
  a.h = hidden_act;
  a.out = out;
  return launch_experts(a, dtype, static_cast<hipStream_t>(stream));
}

extern "C" int32_t mie_moe_decode_block_acc(const void* x, const void* acc, const void* b_out, void* h_out,
                                            const void* ln_weight, const void* ln_bias, float ln_eps,
                                            const void* router_weight, const void* w1, const void* b1,
                                            const void* w2, const void* b2, int32_t num_experts, int32_t top_k,
                                            int32_t dim, int32_t hidden, void* router_logits, void* expert_ids,
                                            void* route_weights, void* hidden_act, void* out, int32_t dtype,
                                            void* stream) {
  int32_t rc = mie::moe_decode_block_acc_check(x, acc, b_out, h_out, ln_weight, ln_bias, router_weight, w1, b1, w2,
                                               b2, num_experts, top_k, dim, hidden, router_logits, expert_ids,
                                               route_weights, hidden_act, out, dtype);
  if (rc != MIE_OK) return rc;
  MoeArgs a = make_args(h_out, router_weight, num_experts, top_k, dim, hidden, router_logits, expert_ids,
                        route_weights);
  a.x = x;  // the W1 launch reads x and forms h_out
  a.acc = static_cast<const unsigned long long*>(acc);
  a.b_out = b_out;
  a.h_out = h_out;
  a.acc_clear = static_cast<unsigned long long*>(const_cast<void*>(acc));
  a.ln_w = ln_weight;
  a.ln_b = ln_bias;
  a.ln_eps = ln_eps;
  a.residual = h_out;
  a.w1 = w1;
  a.b1 = b1;
  a.w2 = w2;
  a.b2 = b2;
  a.h = hidden_act;
  a.out = out;
  return launch_experts(a, dtype, static_cast<hipStream_t>(stream));
}
