// Token plus positional embedding of decode tokens (src/moe_engine/model.py:558):
//
//   out[i, :] = round(token_table[token_ids[i], :] + pos_table[positions[i], :])
//
// summed in float32 and rounded once to the model dtype, as torch adds two
// float32 or bfloat16 tensors.  One workgroup per token: the id and the
// position are read first, then the two rows.  In a captured decode step the
// position comes from device memory, so one launch replaces two row
// selections, an add and the position's conversion to int64.
//
// An id or position outside its table writes a NaN row (torch raises a device
// assertion there; a NaN row makes every later logit NaN instead of reading
// out of bounds).
#include "mie_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kPerThread = 4;

template <typename DT> struct Row;
template <> struct Row<float> {
  static __device__ __forceinline__ float load(const void* p, int64_t i) { return static_cast<const float*>(p)[i]; }
  static __device__ __forceinline__ void store(void* p, int64_t i, float v) { static_cast<float*>(p)[i] = v; }
};
template <> struct Row<uint16_t> {  // bfloat16
  static __device__ __forceinline__ float load(const void* p, int64_t i) {
    return __uint_as_float(static_cast<uint32_t>(static_cast<const uint16_t*>(p)[i]) << 16);
  }
  static __device__ __forceinline__ void store(void* p, int64_t i, float v) {
    static_cast<uint16_t*>(p)[i] = static_cast<uint16_t>(mie::f32_to_bf16_bits(v));
  }
};

template <typename DT>
__global__ __launch_bounds__(kThreads) void embed_kernel(const int64_t* __restrict__ ids,
                                                         const int32_t* __restrict__ positions, int32_t position0,
                                                         const void* tok, int32_t vocab, const void* pos_table,
                                                         int32_t max_positions, int32_t dim, void* out) {
  using E = Row<DT>;
  const int i = blockIdx.x;
  const int64_t id = ids[i];
  const int64_t p = positions ? positions[i] : static_cast<int64_t>(position0) + i;
  const bool ok = id >= 0 && id < vocab && p >= 0 && p < max_positions;
  const int64_t o = static_cast<int64_t>(i) * dim;
  // kPerThread elements per thread per round, all loads before the stores
  // (one round up to dim 1024).
  for (int d0 = threadIdx.x; d0 < dim; d0 += kThreads * kPerThread) {
    float t[kPerThread], q[kPerThread];
#pragma unroll
    for (int u = 0; u < kPerThread; ++u) {
      const int d = d0 + u * kThreads;
      t[u] = ok && d < dim ? E::load(tok, id * dim + d) : 0.f;
      q[u] = ok && d < dim ? E::load(pos_table, p * dim + d) : 0.f;
    }
#pragma unroll
    for (int u = 0; u < kPerThread; ++u) {
      const int d = d0 + u * kThreads;
      if (d < dim) E::store(out, o + d, ok ? t[u] + q[u] : NAN);
    }
  }
}

}  // namespace

extern "C" int32_t mie_embed(const void* token_ids, const int32_t* positions, int32_t position, int32_t n,
                             const void* token_table, int32_t vocab, const void* pos_table, int32_t max_positions,
                             int32_t dim, void* out, int32_t dtype, void* stream) {
  if (dtype != MIE_DTYPE_F32 && dtype != MIE_DTYPE_BF16)
    return mie::fail(MIE_ERR_UNSUPPORTED, "mie_embed: dtype %d (float32 and bfloat16 are built)", dtype);
  if (n < 0 || n > 65535 || dim <= 0 || vocab <= 0 || max_positions <= 0)
    return mie::fail(MIE_ERR_INVALID, "mie_embed: n %d, dim %d, vocab %d, max_positions %d", n, dim, vocab,
                     max_positions);
  if (!positions && position < 0) return mie::fail(MIE_ERR_INVALID, "mie_embed: position %d", position);
  if (n == 0) return MIE_OK;
  if (!token_ids || !token_table || !pos_table || !out) return mie::fail(MIE_ERR_INVALID, "mie_embed: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t* ids = static_cast<const int64_t*>(token_ids);
  if (dtype == MIE_DTYPE_F32) {
    embed_kernel<float><<<n, kThreads, 0, st>>>(ids, positions, position, token_table, vocab, pos_table,
                                                max_positions, dim, out);
  } else {
    embed_kernel<uint16_t><<<n, kThreads, 0, st>>>(ids, positions, position, token_table, vocab, pos_table,
                                                   max_positions, dim, out);
  }
  return mie::check_launch("embed_kernel");
}
