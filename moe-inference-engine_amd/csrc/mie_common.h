// Shared helpers for the gfx950 paged-KV kernels: error state, element sizes,
// fast division by a runtime block size, bf16 <-> f32 conversion and the
// 64-lane wavefront reductions the decode kernels use.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mie_paged_kv.h"

namespace mie {

// Records `msg` as this thread's last error and returns `code`.
int32_t fail(int32_t code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

inline int elt_size(int32_t dtype) {
  switch (dtype) {
    case MIE_DTYPE_F32: return 4;
    case MIE_DTYPE_BF16: return 2;
    case MIE_DTYPE_F16: return 2;
    case MIE_DTYPE_F64: return 8;
    default: return 0;
  }
}

// Maps a launch failure to MIE_ERR_LAUNCH with the runtime's message.
int32_t check_launch(const char* what);

// mie_kv_append with `pos_bias` added to every position: pos_bias = -1 with
// positions = the sequences' lengths appends each sequence's last token.
int32_t kv_append_impl(void* k_pool, void* v_pool, int64_t pool_stride_block, int64_t pool_stride_head,
                       int32_t num_blocks, const void* k_new, const void* v_new, int64_t new_stride_b,
                       int64_t new_stride_h, int64_t new_stride_s, const int32_t* block_tables,
                       int64_t block_table_stride, const int32_t* positions, int32_t position, int32_t pos_bias,
                       int32_t batch, int32_t seq_len, int32_t num_heads, int32_t head_dim, int32_t block_size,
                       int32_t dtype, void* stream);

// Unsigned division by a runtime divisor d >= 1 for numerators n < 2^31:
//   q = (umulhi(n, magic) + n) >> shift,  shift = ceil(log2 d),
//   magic = floor(2^32 * (2^shift - d) / d) + 1
// (Granlund & Montgomery, "Division by invariant integers using
// multiplication", PLDI 1994, round-up variant).  n + umulhi(n, magic) < 2^32
// holds because n < 2^31 and umulhi(n, magic) <= n.
struct FastDiv {
  uint32_t d;
  uint32_t magic;
  uint32_t shift;

  static FastDiv make(uint32_t divisor) {
    FastDiv f;
    f.d = divisor;
    uint32_t s = 0;
    while ((1ull << s) < divisor) ++s;
    f.shift = s;
    f.magic = static_cast<uint32_t>(((1ull << 32) * ((1ull << s) - divisor)) / divisor + 1);
    return f;
  }
  __device__ __forceinline__ uint32_t div(uint32_t n) const {
    return (__umulhi(n, magic) + n) >> shift;
  }
};

// ---- bf16 <-> f32 ---------------------------------------------------------
// A bf16 value is the high half of the f32 with the same sign/exponent, so the
// widening is a shift; narrowing rounds to nearest even (NaN kept quiet).
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Written as a select, not an early return: as a branch the NaN test made
// the compiler wrap every element's rounding in its own exec-mask branch.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t rounded = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  const uint32_t quiet_nan = (u >> 16) | 0x40u;
  return (u & 0x7fffffffu) > 0x7f800000u ? quiet_nan : rounded;
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
}

// ---- element storage: float32 or bfloat16 ----------------------------------
// Kernels that take either dtype hold four consecutive elements per lane (16
// bytes of float32, 8 of bfloat16, held as uint16_t) and work on them in
// float32; R() rounds a float32 result to the storage type (the identity for
// float32).  raw4 is the loaded form: a kernel that wants many loads in
// flight keeps raw words and widens them where it uses them, since a widen
// right after each load makes the compiler wait for that load first.
typedef float mem_f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int mem_u32x2 __attribute__((ext_vector_type(2)));
template <typename T> struct Mem;
template <> struct Mem<float> {
  typedef mem_f32x4 raw4;
  static __device__ __forceinline__ raw4 load_raw(const float* p) { return *reinterpret_cast<const raw4*>(p); }
  static __device__ __forceinline__ raw4 stream_raw(const float* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const raw4*>(p));
  }
  static __device__ __forceinline__ raw4 zero_raw() { return raw4{0.f, 0.f, 0.f, 0.f}; }
  static __device__ __forceinline__ mem_f32x4 widen(raw4 r) { return r; }
  static __device__ __forceinline__ mem_f32x4 load4(const float* p) { return *reinterpret_cast<const mem_f32x4*>(p); }
  static __device__ __forceinline__ mem_f32x4 stream4(const float* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const mem_f32x4*>(p));
  }
  static __device__ __forceinline__ float get(const float* p) { return *p; }
  static __device__ __forceinline__ void put(float* p, float v) { *p = v; }
  static __device__ __forceinline__ void put4(float* p, mem_f32x4 v) { *reinterpret_cast<mem_f32x4*>(p) = v; }
  static __device__ __forceinline__ float R(float v) { return v; }
  static __device__ __forceinline__ mem_f32x4 R4(mem_f32x4 v) { return v; }
};
template <> struct Mem<uint16_t> {
  typedef mem_u32x2 raw4;
  static __device__ __forceinline__ raw4 load_raw(const uint16_t* p) { return *reinterpret_cast<const raw4*>(p); }
  static __device__ __forceinline__ raw4 stream_raw(const uint16_t* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const raw4*>(p));
  }
  static __device__ __forceinline__ raw4 zero_raw() { return raw4{0u, 0u}; }
  static __device__ __forceinline__ mem_f32x4 widen(mem_u32x2 w) {
    return mem_f32x4{bf16_lo(w.x), bf16_hi(w.x), bf16_lo(w.y), bf16_hi(w.y)};
  }
  static __device__ __forceinline__ mem_f32x4 load4(const uint16_t* p) {
    return widen(*reinterpret_cast<const mem_u32x2*>(p));
  }
  static __device__ __forceinline__ mem_f32x4 stream4(const uint16_t* p) {
    return widen(__builtin_nontemporal_load(reinterpret_cast<const mem_u32x2*>(p)));
  }
  static __device__ __forceinline__ float get(const uint16_t* p) {
    return __uint_as_float(static_cast<uint32_t>(*p) << 16);
  }
  static __device__ __forceinline__ void put(uint16_t* p, float v) { *p = static_cast<uint16_t>(f32_to_bf16_bits(v)); }
  static __device__ __forceinline__ void put4(uint16_t* p, mem_f32x4 v) {
    *reinterpret_cast<mem_u32x2*>(p) = mem_u32x2{pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w)};
  }
  static __device__ __forceinline__ float R(float v) { return __uint_as_float(f32_to_bf16_bits(v) << 16); }
  static __device__ __forceinline__ mem_f32x4 R4(mem_f32x4 v) { return mem_f32x4{R(v.x), R(v.y), R(v.z), R(v.w)}; }
};

// ---- wavefront reductions -------------------------------------------------
// DPP controls (CDNA3/4 ISA): quad_perm [1,0,3,2] = 0xB1, [2,3,0,1] = 0x4E,
// row_half_mirror = 0x141 (lane i <-> 7-i within 8), row_mirror = 0x140
// (i <-> 15-i within 16).  Applied in this order each stage pairs lanes whose
// partial sums cover disjoint halves, so after log2(N) stages every lane of an
// aligned N-lane group holds the group total.
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

// Sum over aligned groups of N lanes (N a power of two <= 64); all 64 lanes of
// the wave must be active.
template <int N>
__device__ __forceinline__ float group_sum(float x) {
  if constexpr (N >= 2) x += dpp<0xB1>(x);
  if constexpr (N >= 4) x += dpp<0x4E>(x);
  if constexpr (N >= 8) x += dpp<0x141>(x);
  if constexpr (N >= 16) x += dpp<0x140>(x);
  if constexpr (N >= 32) x += __shfl_xor(x, 16);
  if constexpr (N >= 64) x += __shfl_xor(x, 32);
  return x;
}

__device__ __forceinline__ float wave_max(float x) {
  for (int off = 32; off >= 1; off >>= 1) x = fmaxf(x, __shfl_xor(x, off));
  return x;
}
// Sum over the wave, in every lane: four DPP stages inside each 16-lane row,
// then two cross-row exchanges (group_sum<64>).
__device__ __forceinline__ float wave_sum(float x) { return group_sum<64>(x); }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ---- greedy pick -------------------------------------------------------------
// torch.argmax's order: the larger value wins, NaN counts as larger than every
// number, and between equal values (or two NaNs) the lower index wins.  The
// order is total over (value, index), so pairs may be merged in any order.
// Written with bitwise operators on the comparisons so it compiles to
// compares and selects, not branches.
__device__ __forceinline__ void argmax_take(float& va, int& ia, float vb, int ib) {
  const bool a_nan = va != va, b_nan = vb != vb;
  const bool lower = ib < ia;
  // vb > va and vb == va are false when either is NaN.
  const bool b_wins = (b_nan & (!a_nan | lower)) | (vb > va) | ((vb == va) & lower);
  va = b_wins ? vb : va;
  ia = b_wins ? ib : ia;
}

// Merges (v, i) over the 64 lanes; every lane ends with the wave's pick.
__device__ __forceinline__ void wave_argmax(float& v, int& i) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(v, off);
    const int oi = __shfl_xor(i, off);
    argmax_take(v, i, ov, oi);
  }
}

// One workgroup's pick: (-inf, INT32_MAX) when it had no rows.
struct ArgmaxPair {
  float v;
  int32_t i;
};

}  // namespace mie

namespace mie {
// Reduces n per-workgroup picks to the final index, written as int64 to *out
// (0 if no pair holds an index below `limit`), then adds one to each of the
// n_advance int32 counters at `advance`.  One workgroup; nothing to clear
// beforehand.
int32_t launch_argmax_pairs(const ArgmaxPair* pairs, int32_t n, int32_t limit, int64_t* out, int32_t* advance,
                            int32_t n_advance, hipStream_t stream);
}  // namespace mie

namespace mie {
// Host-only argument checks of the entry points mie_block_plan_init stores a
// plan for: each returns what its entry point would return for these
// arguments before launching anything (MIE_OK when it would launch).
// paged_decode_check checks one sequence of one token (batch 1, ctx 1); the
// split workspace is checked per call.
int32_t qkv_append_check(const void* x, const void* ln_weight, const void* ln_bias, const void* w_in, int32_t dim,
                         const void* k_pool, const void* v_pool, int64_t pool_stride_block, int64_t pool_stride_head,
                         int32_t num_blocks, const int32_t* block_table, int32_t block_table_len,
                         const int32_t* position_dev, int32_t position, const void* q_out, int32_t num_heads,
                         int32_t head_dim, int32_t block_size, int32_t dtype);
int32_t linear_residual_check(const void* x, const void* weight, const void* out, int32_t rows, int32_t cols,
                              int32_t dtype);
int32_t paged_decode_check(const void* q, const void* k_pool, const void* v_pool, int64_t pool_stride_block,
                           int64_t pool_stride_head, int32_t num_blocks, const int32_t* block_table,
                           int32_t num_heads, int32_t head_dim, int32_t block_size, void* out, int32_t dtype);
int32_t moe_decode_block_check(const void* x, const void* ln_weight, const void* ln_bias, const void* router_weight,
                               const void* w1, const void* b1, const void* w2, const void* b2, int32_t num_experts,
                               int32_t top_k, int32_t dim, int32_t hidden, const void* router_logits,
                               const void* expert_ids, const void* route_weights, const void* hidden_act,
                               const void* out, int32_t dtype);
}  // namespace mie

namespace mie {
// Block-table entries the fused attention + output projection holds in LDS:
// it serves contexts of at most this many blocks.
constexpr int32_t kAttnOutMaxBlocks = 1024;
// Host checks and launch of the fused attention + output projection
// (attn_out.hip, mie_attn_out_acc) and the MoE half that consumes its
// fixed-point sums (mie_moe_decode_block_acc).
int32_t attn_out_check(const void* q, const void* k_pool, const void* v_pool, int64_t pool_stride_block,
                       int64_t pool_stride_head, int32_t num_blocks, const int32_t* block_table,
                       int32_t block_table_len, int32_t max_ctx, int32_t num_heads, int32_t head_dim,
                       int32_t block_size, const void* w_out, const void* acc, int32_t dtype);
int32_t attn_out_launch(const void* q, const void* k_pool, const void* v_pool, int64_t pool_stride_block,
                        int64_t pool_stride_head, int32_t num_blocks, const int32_t* block_table,
                        int32_t block_table_len, const int32_t* ctx_dev, int32_t ctx, int32_t max_ctx,
                        int32_t num_heads, int32_t head_dim, int32_t block_size, float scale, const void* w_out,
                        void* acc, int32_t dtype, hipStream_t stream);
int32_t moe_decode_block_acc_check(const void* x, const void* acc, const void* b_out, const void* h_out,
                                   const void* ln_weight, const void* ln_bias, const void* router_weight,
                                   const void* w1, const void* b1, const void* w2, const void* b2,
                                   int32_t num_experts, int32_t top_k, int32_t dim, int32_t hidden,
                                   const void* router_logits, const void* expert_ids, const void* route_weights,
                                   const void* hidden_act, const void* out, int32_t dtype);
}  // namespace mie

namespace mie {
// The embedding folded into layer 0's QKV launch: x = round(token_table[
// *token_id] + pos_table[position]) (float32 sum, one rounding; NaN for an id
// or position outside its table), stored to x_out by the launch for the
// block's residual.
struct QkvEmbedding {
  const int64_t* token_id;  // device
  const void* token_table;  // [vocab, dim]
  int32_t vocab;
  const void* pos_table;    // [max_positions, dim]
  int32_t max_positions;
  void* x_out;              // [dim]
};
int32_t qkv_embedding_check(const QkvEmbedding& e, int32_t dim);
// mie_qkv_append with x formed from the embedding tables.
int32_t qkv_append_embedded(const QkvEmbedding& e, const void* ln_weight, const void* ln_bias, float ln_eps,
                            const void* w_in, const void* b_in, int32_t dim, void* k_pool, void* v_pool,
                            int64_t pool_stride_block, int64_t pool_stride_head, int32_t num_blocks,
                            const int32_t* block_table, int32_t block_table_len, const int32_t* position_dev,
                            int32_t position, void* q_out, int32_t num_heads, int32_t head_dim, int32_t block_size,
                            int32_t dtype, void* stream);
}  // namespace mie
