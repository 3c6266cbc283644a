// QKV projection of one decode token written straight into the paged pools.
//
// The reference computes, per layer and token (src/moe_engine/model.py:228-247):
//
//   y        = LayerNorm(x)                      (the block's attn_norm)
//   qkv      = in_proj_weight @ y + in_proj_bias [3*dim]
//   q, k, v  = qkv[0:dim], qkv[dim:2dim], qkv[2dim:3dim], each [H, D]
//   cache.write: pool[bt[p // BS], h, p % BS, :] = k[h, :]  (and v)
//
// as three launches (norm, GEMM, append) plus the GEMM's argument upload.  Here
// one launch does all of it: every workgroup normalises x into LDS (x is 3 KiB
// at dim 768, so recomputing it per workgroup is cheaper than another launch),
// then each wave computes two rows of the projection and stores them where they
// belong - q into q_out, K and V into their pool slots.
//
// Rounding points follow the reference for each dtype: the norm is computed in
// float32 and rounded to the model dtype before the projection (bf16 models
// feed bf16 activations to the GEMM); the projection accumulates in float32,
// adds the bias, and rounds once to the model dtype.
//
// The projection reads 3*dim*dim*elt bytes of weights once: HBM-bound
// (0.5 flop/B in float32).  Weight loads are issued before the norm so their
// latency overlaps it; they carry the non-temporal hint (each layer's weights
// are streamed once per token).
#include "mie_common.h"

namespace {

constexpr int kRowsPerWave = 2;
constexpr int kRowsPerGroup = 4 * kRowsPerWave;
constexpr int kMaxDim = 4096;  // the largest dim built: 8 loads x 64 lanes x 8 bf16

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

struct QkvArgs {
  const void* x;
  const void* ln_w;  // NULL: no norm
  const void* ln_b;
  float ln_eps;
  const void* w_in;  // [3*dim, dim]
  const void* b_in;  // [3*dim] or NULL
  int32_t dim;
  char* k_pool;  // one layer, element strides below
  char* v_pool;
  int64_t sblk, shead;
  int32_t num_blocks;
  const int32_t* block_table;
  int32_t bt_len;
  const int32_t* position_dev;  // NULL: use position
  int32_t position;
  void* q_out;  // [dim]
  int32_t head_dim;
  mie::FastDiv bs;
};

template <typename DT> struct Elt;
template <> struct Elt<float> {
  static constexpr int kPerVec = 4;  // elements per 16-byte load
  static __device__ __forceinline__ float load(const void* p, int i) { return static_cast<const float*>(p)[i]; }
  static __device__ __forceinline__ float round(float v) { return v; }
  static __device__ __forceinline__ void store(void* p, int64_t i, float v) { static_cast<float*>(p)[i] = v; }
  static __device__ __forceinline__ void widen(u32x4_t w, float* out) {
    out[0] = __uint_as_float(w.x);
    out[1] = __uint_as_float(w.y);
    out[2] = __uint_as_float(w.z);
    out[3] = __uint_as_float(w.w);
  }
};
template <> struct Elt<uint16_t> {  // bfloat16
  static constexpr int kPerVec = 8;
  static __device__ __forceinline__ float load(const void* p, int i) {
    return __uint_as_float(static_cast<uint32_t>(static_cast<const uint16_t*>(p)[i]) << 16);
  }
  static __device__ __forceinline__ float round(float v) { return __uint_as_float(mie::f32_to_bf16_bits(v) << 16); }
  static __device__ __forceinline__ void store(void* p, int64_t i, float v) {
    static_cast<uint16_t*>(p)[i] = static_cast<uint16_t>(mie::f32_to_bf16_bits(v));
  }
  static __device__ __forceinline__ void widen(u32x4_t w, float* out) {
    out[0] = mie::bf16_lo(w.x);
    out[1] = mie::bf16_hi(w.x);
    out[2] = mie::bf16_lo(w.y);
    out[3] = mie::bf16_hi(w.y);
    out[4] = mie::bf16_lo(w.z);
    out[5] = mie::bf16_hi(w.z);
    out[6] = mie::bf16_lo(w.w);
    out[7] = mie::bf16_hi(w.w);
  }
};

// Sum of one float over the 256-thread workgroup; every thread gets the total.
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = mie::wave_sum(v);
  const int wave = threadIdx.x >> 6;
  __syncthreads();  // `red` may still be read from a previous call
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];
}

// grid = ceil(3*dim / 8), 256 threads.  NCH = 16-byte loads per lane per row
// (ceil(dim / (64 * elements per load))).
template <typename DT, int NCH>
__global__ __launch_bounds__(256) void qkv_append_kernel(QkvArgs a) {
  using E = Elt<DT>;
  constexpr int EPV = E::kPerVec;
  __shared__ float y[kMaxDim];
  __shared__ float red[4];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int dim = a.dim;
  const int rows = 3 * dim;
  const int r0 = blockIdx.x * kRowsPerGroup + wave * kRowsPerWave;
  // Rows past the end repeat row r0 (or the last row) and are not stored.
  const int ra = min(r0, rows - 1);
  const int rb = min(r0 + 1, rows - 1);

  // 1. Weight loads first: they do not depend on the norm.
  u32x4_t wa[NCH], wb[NCH];
  const DT* w = static_cast<const DT*>(a.w_in);
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int i = (c * 64 + lane) * EPV;
    if (i < dim) {
      wa[c] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(w + static_cast<int64_t>(ra) * dim + i));
      wb[c] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(w + static_cast<int64_t>(rb) * dim + i));
    }
  }

  // 2. Every other global read is issued now too, so the launch waits on one
  //    round trip: x and the norm parameters (thread t holds elements t,
  //    t + 256, ...; XPT of them cover dim) and the bias of the row this lane
  //    will store.
  constexpr int XPT = NCH * EPV / 4;
  float xv[XPT], gw[XPT], gb[XPT];
#pragma unroll
  for (int k = 0; k < XPT; ++k) {
    const int i = threadIdx.x + k * 256;
    xv[k] = i < dim ? E::load(a.x, i) : 0.f;
    gw[k] = a.ln_w && i < dim ? E::load(a.ln_w, i) : 0.f;
    gb[k] = a.ln_b && i < dim ? E::load(a.ln_b, i) : 0.f;
  }
  const int r_store = r0 + ((lane >> 5) & 1);
  const float bias = a.b_in && (lane & 31) == 0 && r_store < rows ? E::load(a.b_in, r_store) : 0.f;

  // 3. x, normalised when ln_w is given and rounded as the reference's norm
  //    output is, into LDS as float.
  if (a.ln_w) {
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < XPT; ++k) s += xv[k];  // zero past dim
    const float mean = block_sum(s, red) / dim;
    float q = 0.f;
#pragma unroll
    for (int k = 0; k < XPT; ++k) {
      const float d = threadIdx.x + k * 256 < dim ? xv[k] - mean : 0.f;
      q = fmaf(d, d, q);
    }
    const float rstd = rsqrtf(block_sum(q, red) / dim + a.ln_eps);
#pragma unroll
    for (int k = 0; k < XPT; ++k) {
      const int i = threadIdx.x + k * 256;
      if (i < dim) y[i] = E::round((xv[k] - mean) * rstd * gw[k] + gb[k]);
    }
  } else {
#pragma unroll
    for (int k = 0; k < XPT; ++k) {
      const int i = threadIdx.x + k * 256;
      if (i < dim) y[i] = xv[k];
    }
  }
  __syncthreads();

  // 4. Two dot products per wave.
  float sa = 0.f, sb = 0.f;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int i = (c * 64 + lane) * EPV;
    if (i < dim) {
      float fa[EPV], fb[EPV];
      E::widen(wa[c], fa);
      E::widen(wb[c], fb);
#pragma unroll
      for (int e = 0; e < EPV; ++e) {
        const float yv = y[i + e];
        sa = fmaf(fa[e], yv, sa);
        sb = fmaf(fb[e], yv, sb);
      }
    }
  }
  // Lanes 0-31 finish row a, lanes 32-63 row b.
  const bool hi = lane & 32;
  float t = (hi ? sb : sa) + __shfl_xor(hi ? sa : sb, 32);
  t = mie::group_sum<32>(t);
  if ((lane & 31) != 0) return;
  const int r = r_store;
  if (r >= rows) return;

  // 5. Store: q, or the K / V row of the token's pool slot.
  const float out = t + bias;
  if (r < dim) {
    E::store(a.q_out, r, out);
    return;
  }
  const bool is_v = r >= 2 * dim;
  const int j = r - (is_v ? 2 * dim : dim);
  const int h = j / a.head_dim;
  const int d = j - h * a.head_dim;
  const int pos = a.position_dev ? *a.position_dev : a.position;
  if (pos < 0) return;
  const uint32_t lb = a.bs.div(static_cast<uint32_t>(pos));
  const uint32_t slot = static_cast<uint32_t>(pos) - lb * a.bs.d;
  if (lb >= static_cast<uint32_t>(a.bt_len)) return;
  const int32_t phys = a.block_table[lb];
  if (phys < 0 || phys >= a.num_blocks) return;
  E::store(is_v ? a.v_pool : a.k_pool, phys * a.sblk + h * a.shead + static_cast<int64_t>(slot) * a.head_dim + d, out);
}

template <typename DT>
int32_t launch(const QkvArgs& a, hipStream_t st) {
  const int nch = (a.dim + 64 * Elt<DT>::kPerVec - 1) / (64 * Elt<DT>::kPerVec);
  const int groups = (3 * a.dim + kRowsPerGroup - 1) / kRowsPerGroup;
  switch (nch) {
    case 1: qkv_append_kernel<DT, 1><<<groups, 256, 0, st>>>(a); break;
    case 2: qkv_append_kernel<DT, 2><<<groups, 256, 0, st>>>(a); break;
    case 3: qkv_append_kernel<DT, 3><<<groups, 256, 0, st>>>(a); break;
    case 4: qkv_append_kernel<DT, 4><<<groups, 256, 0, st>>>(a); break;
    case 5: qkv_append_kernel<DT, 5><<<groups, 256, 0, st>>>(a); break;
    case 6: qkv_append_kernel<DT, 6><<<groups, 256, 0, st>>>(a); break;
    case 7: qkv_append_kernel<DT, 7><<<groups, 256, 0, st>>>(a); break;
    case 8: qkv_append_kernel<DT, 8><<<groups, 256, 0, st>>>(a); break;
    default: return mie::fail(MIE_ERR_UNSUPPORTED, "mie_qkv_append: dim %d is too large", a.dim);
  }
  return mie::check_launch("qkv_append_kernel");
}

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

}  // namespace

extern "C" int32_t mie_qkv_append_supported(int32_t dim, int32_t dtype) {
  if (dim <= 0) return 0;
  if (dtype == MIE_DTYPE_F32) return dim % 4 == 0 && dim <= 8 * 64 * 4;
  if (dtype == MIE_DTYPE_BF16) return dim % 8 == 0 && dim <= 8 * 64 * 8;
  return 0;
}

extern "C" int32_t mie_qkv_append(const void* x, const void* ln_weight, const void* ln_bias, float ln_eps,
                                  const void* w_in, const void* b_in, int32_t dim, void* k_pool, void* v_pool,
                                  int64_t pool_stride_block, int64_t pool_stride_head, int32_t num_blocks,
                                  const int32_t* block_table, int32_t block_table_len, const int32_t* position_dev,
                                  int32_t position, void* q_out, int32_t num_heads, int32_t head_dim,
                                  int32_t block_size, int32_t dtype, void* stream) {
  if (!mie_qkv_append_supported(dim, dtype))
    return mie::fail(MIE_ERR_UNSUPPORTED, "mie_qkv_append: dim %d with dtype %d is not built", dim, dtype);
  if (num_heads <= 0 || head_dim <= 0 || num_heads * head_dim != dim)
    return mie::fail(MIE_ERR_INVALID, "mie_qkv_append: heads %d x head_dim %d != dim %d", num_heads, head_dim, dim);
  if (block_size <= 0 || num_blocks <= 0 || block_table_len < 0)
    return mie::fail(MIE_ERR_INVALID, "mie_qkv_append: block_size %d, num_blocks %d, table length %d", block_size,
                     num_blocks, block_table_len);
  if (!x || !w_in || !k_pool || !v_pool || !block_table || !q_out)
    return mie::fail(MIE_ERR_INVALID, "mie_qkv_append: null pointer");
  if ((ln_weight == nullptr) != (ln_bias == nullptr) && ln_bias != nullptr)
    return mie::fail(MIE_ERR_INVALID, "mie_qkv_append: a norm bias needs a norm weight");
  if (!aligned16(w_in))
    return mie::fail(MIE_ERR_INVALID, "mie_qkv_append: the projection weight must be 16-byte aligned");
  if (pool_stride_head < static_cast<int64_t>(block_size) * head_dim ||
      pool_stride_block < static_cast<int64_t>(num_heads) * pool_stride_head)
    return mie::fail(MIE_ERR_INVALID, "mie_qkv_append: pool strides (%lld, %lld) overlap",
                     static_cast<long long>(pool_stride_block), static_cast<long long>(pool_stride_head));
  if (!position_dev && position < 0) return mie::fail(MIE_ERR_INVALID, "mie_qkv_append: position %d", position);
  QkvArgs a;
  a.x = x;
  a.ln_w = ln_weight;
  a.ln_b = ln_bias;
  a.ln_eps = ln_eps;
  a.w_in = w_in;
  a.b_in = b_in;
  a.dim = dim;
  a.k_pool = static_cast<char*>(k_pool);
  a.v_pool = static_cast<char*>(v_pool);
  a.sblk = pool_stride_block;
  a.shead = pool_stride_head;
  a.num_blocks = num_blocks;
  a.block_table = block_table;
  a.bt_len = block_table_len;
  a.position_dev = position_dev;
  a.position = position;
  a.q_out = q_out;
  a.head_dim = head_dim;
  a.bs = mie::FastDiv::make(static_cast<uint32_t>(block_size));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == MIE_DTYPE_F32) return launch<float>(a, st);
  return launch<uint16_t>(a, st);
}
