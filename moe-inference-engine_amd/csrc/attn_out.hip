// Decode attention of one token fused with the attention's output projection.
//
// The reference's attention half of a decoder block for one decode token
// (src/moe_engine/model.py:226-269 and :495) is, after the QKV projection and
// the cache write:
//
//   a_h  = softmax(scale * q_h . K_h^T) . V_h          for each head h
//   o    = out_proj(a) = W_out a + b_out               (W_out [dim, dim], a = [a_0 .. a_{H-1}])
//   h    = x + o
//
// Done as two launches (a decode kernel writing a, then a GEMV over all of a)
// the projection waits for every head.  Here one launch computes, for each
// head h and each block of output rows r, the head's attention and that head's
// share of the rows:
//
//   y_hr[i] = sum_{d < D} W_out[i, h*D + d] * a_h[d]     i in rows block r
//
// and adds y_hr[i] into acc[i] with a 64-bit integer atomic on a fixed-point
// value round(y_hr[i] * 2^32).  Integer addition is exact and associative, so
// acc[i] = sum_h round(y_hr[i] * 2^32) comes out bit-identical whatever order
// the workgroups finish in - deterministic, with no cross-workgroup handoff
// (which on MI355X needs an L2 writeback per publishing workgroup) and no
// second launch.  The consumer (the MoE W1 launch of the same block,
// mie_moe_decode_block_acc) forms h = x + (float(acc) * 2^-32 + b_out), and
// its W2 launch clears acc for the next token.  A partial of 2^31 / H or
// more in magnitude (or not a number) is not added - the sum of the H heads'
// partials could leave int64 - but sets acc[dim] instead, and the consumer
// then writes NaN.
//
// Work decomposition: grid (8 * R * ceil(H / 8)) workgroups of W waves (4, or
// 8 when the launch's context bound exceeds one round of 4: kShortMaxCtx).  The
// hardware dispatches workgroup i to XCD i mod 8, so workgroup (8 j + x) is
// head x + 8 (j / R), rows block j % R: the R workgroups of a head share one
// XCD's L2, and the head's K/V, which each of them reads, comes from HBM once.
// Inside a workgroup the W waves split the context (token t goes to wave
// (t / TPL) mod W) and merge their softmax states in LDS; then each wave
// computes TPL rows per wave load of its share of the row block.  Everything
// that does not depend on the attention - q, the block table, this
// workgroup's W_out slice - is read in the first memory round; the K/V tiles
// in the second (one round per kBatch * TPL tokens per wave, 32 at head_dim 64).
//
// float32 or bfloat16 (q, the pools and W_out in one dtype; every product and
// sum in float32, the head's attention output rounded to the dtype before the
// projection, as the decode kernels store it), head_dim 32, 64 or 128,
// contexts up to kMaxTable blocks.  A context block whose id lies outside the
// pool is never read; the head's attention is then NaN (as the decode kernels
// write), which sets acc[dim].
#include <math.h>

#include "mie_common.h"

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kMaxTable = mie::kAttnOutMaxBlocks;  // block-table entries held in LDS
constexpr int kBatch = 8;         // wave loads of K (and of V) per memory round
// Rows of W_out per workgroup, in wave loads of TPL rows: 12 of them, 48 rows
// at head_dim 64 (R = 16 workgroups per head at dim 768, 192 in all).
// Measured on MI355X (config 1, kernel trace, 4 waves): 24 wave loads (R = 8)
// 7.0 us per launch, 12 with plain K/V loads 5.6 us, 8 with plain loads 5.7 us.
constexpr int kRowLoads = 12;
// Waves per workgroup.  A wave's share of the context is one memory round per
// kBatch * TPL of its tokens, so a workgroup covers W * kBatch * TPL tokens a
// round (128 for 4 waves at head_dim 64).  Four waves are fastest for short
// contexts, eight past one round of four.  Config 1's graphed step on MI355X
// (ms per token, 4 / 8 / 16 waves): 64 tokens 0.292 / 0.299 / 0.320, 128
// 0.299 / 0.302 / 0.322, 192 0.316 / 0.307 / 0.325, 256 0.323 / 0.315 / 0.332,
// 512 0.352 / 0.332 / 0.335, 1024 0.409 / 0.375 / 0.372.
constexpr int kShortWaves = 4, kLongWaves = 8;
constexpr int kShortMaxCtx = 128;  // contexts (the launch's bound) the short form takes
constexpr float kFix = 4294967296.0f;  // 2^32

typedef float f32x4_t __attribute__((ext_vector_type(4)));

struct AttnOutArgs {
  const void* q;  // T [H * D]
  const void* k;  // T: one layer's pools
  const void* v;
  int64_t sblk, shead;  // element strides
  int32_t num_blocks;
  const int32_t* bt;
  int32_t bt_len;
  const int32_t* ctx_dev;  // device context length (or NULL: ctx)
  int32_t ctx;
  int32_t max_ctx;  // contexts are clamped to this (host bound for ctx_dev)
  int32_t nblk_max;  // ceil(max_ctx / block_size) <= kMaxTable
  int32_t H;
  mie::FastDiv bs;
  float qk_scale;  // scale * log2(e)
  const void* w;  // T: W_out [dim, dim] row-major
  int32_t dim;
  int32_t R;  // row blocks per head
  int32_t rows_per_block;
  unsigned long long* acc;  // [dim + 1]
  float fix_limit;  // |y| below this: the sum over the H heads stays inside int64
};

template <int D>
struct Shape {
  static constexpr int LPT = D / 4;   // lanes per row, 16 bytes each
  static constexpr int TPL = 64 / LPT;  // rows per wave load
};

__device__ __forceinline__ float dot4(f32x4_t a, f32x4_t b, float s) {
  s = fmaf(a.x, b.x, s);
  s = fmaf(a.y, b.y, s);
  s = fmaf(a.z, b.z, s);
  return fmaf(a.w, b.w, s);
}

// Log-sum-exp merge of (m, l, o) with (m2, l2, o2) in the log2 domain; a state
// with m = -inf holds no token.
__device__ __forceinline__ void merge_state(float& m, float& l, f32x4_t& o, float m2, float l2, f32x4_t o2) {
  const float mm = fmaxf(m, m2);
  const float c1 = m == -INFINITY ? 0.f : mie::fast_exp2(m - mm);
  const float c2 = m2 == -INFINITY ? 0.f : mie::fast_exp2(m2 - mm);
  l = l * c1 + l2 * c2;
  o = o * c1 + o2 * c2;
  m = mm;
}

template <typename T, int D, int kWaves>
__global__ __launch_bounds__(64 * kWaves) void attn_out_kernel(AttnOutArgs a) {
  using M = mie::Mem<T>;
  constexpr int LPT = Shape<D>::LPT;
  constexpr int TPL = Shape<D>::TPL;
  constexpr int kThreads = 64 * kWaves;
  constexpr int kRowSteps = (kRowLoads + kWaves - 1) / kWaves;  // wave loads of W_out rows per wave
  __shared__ int32_t s_bt[kMaxTable];
  __shared__ float s_ml[kWaves][2];
  __shared__ __align__(16) float s_o[kWaves][D];
  __shared__ __align__(16) float s_attn[D];

  const int xcd = blockIdx.x & 7;
  const int j = blockIdx.x >> 3;
  const int h = xcd + 8 * (j / a.R);
  const int rblk = j % a.R;
  if (h >= a.H) return;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int g = lane / LPT;          // row within a wave load
  const int c4 = (lane % LPT) * 4;   // this lane's 4 columns of a row

  // First memory round, all loads independent: the block table up to the
  // host's bound (nblk_max entries, at most 1024 = 4 per thread) and the live
  // length, then q and this workgroup's W_out rows.  Vector loads complete in
  // issue order, so the table goes first: the K/V round waits only for it (an
  // L2 hit), while the W_out rows (from HBM) stay in flight until the
  // projection.
  constexpr int kTablePerThread = kMaxTable / kThreads;
  int tb[kTablePerThread];
#pragma unroll
  for (int u = 0; u < kTablePerThread; ++u) {
    const int i = u * kThreads + static_cast<int>(threadIdx.x);
    const int ic = i < a.bt_len ? i : 0;  // bt_len >= 1
    tb[u] = u * kThreads < a.nblk_max ? a.bt[ic] : 0;
  }
  int ctx = a.ctx_dev ? *a.ctx_dev : a.ctx;
  const typename M::raw4 qraw = M::load_raw(static_cast<const T*>(a.q) + h * D + c4);
  typename M::raw4 wv[kRowSteps];
  const int row0 = rblk * a.rows_per_block;
  const int row_end = min(a.dim, row0 + a.rows_per_block);
#pragma unroll
  for (int s = 0; s < kRowSteps; ++s) {
    int row = row0 + (s * kWaves + wave) * TPL + g;
    row = row < row_end ? row : row0;  // in bounds; the product is dropped below
    wv[s] = M::stream_raw(static_cast<const T*>(a.w) + static_cast<int64_t>(row) * a.dim + h * D + c4);
  }
  ctx = ctx < 0 ? 0 : (ctx > a.max_ctx ? a.max_ctx : ctx);
  const int nblk = static_cast<int>(a.bs.div(static_cast<uint32_t>(ctx + a.bs.d - 1)));  // <= nblk_max
  int bad = 0;
#pragma unroll
  for (int u = 0; u < kTablePerThread; ++u) {
    const int i = u * kThreads + static_cast<int>(threadIdx.x);
    if (i < nblk) {
      const int blk = i < a.bt_len ? tb[u] : -1;
      s_bt[i] = blk;
      bad |= blk < 0 || blk >= a.num_blocks;
    }
  }
  // A context block outside the pool (never read) makes the head's attention
  // NaN.  Each wave posts its own flag (a ballot, no initialisation needed)
  // and the barrier publishes them with the table: __syncthreads_or would read
  // the workgroup size from the launch's hidden arguments, 256 more bytes of
  // kernel arguments per launch.
  __shared__ int s_badw[kWaves];
  const unsigned long long wave_bad = __ballot(bad);
  if (lane == 0) s_badw[wave] = wave_bad != 0;
  __syncthreads();
  bool any_bad = false;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) any_bad |= s_badw[w] != 0;

  // Later memory rounds: this wave's tokens t = (step * 4 + wave) * TPL + g, kBatch wave
  // loads of K and V per round; online softmax per TPL-row group.
  const T* kh = static_cast<const T*>(a.k) + static_cast<int64_t>(h) * a.shead + c4;
  const T* vh = static_cast<const T*>(a.v) + static_cast<int64_t>(h) * a.shead + c4;
  float m = -INFINITY, l = 0.f;
  f32x4_t o = {0.f, 0.f, 0.f, 0.f};
  const int steps = (ctx + kWaves * TPL - 1) / (kWaves * TPL);
  for (int s0 = 0; s0 < steps; s0 += kBatch) {
    typename M::raw4 kv[kBatch], vv[kBatch];
    bool valid[kBatch];
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      const int t = ((s0 + b) * kWaves + wave) * TPL + g;
      valid[b] = t < ctx;
      const int tc = valid[b] ? t : 0;  // rows past the context re-read token 0, masked below
      const uint32_t lb = a.bs.div(static_cast<uint32_t>(tc));
      int blk = s_bt[lb];
      blk = blk >= 0 && blk < a.num_blocks ? blk : 0;  // never dereferenced outside the pool (any_bad is set)
      const int64_t off = static_cast<int64_t>(blk) * a.sblk + static_cast<int64_t>(tc - lb * a.bs.d) * D;
      // Plain (temporal) loads: the R workgroups of this head run on one XCD
      // and read the same K/V, so all but the first hit its L2.
      kv[b] = M::load_raw(kh + off);
      vv[b] = M::load_raw(vh + off);
    }
    // Every K and V load of the round is issued before the first score: the
    // scheduler would otherwise reuse load registers and start later loads
    // only after earlier ones returned.  At most one or two workgroups per
    // CU, so the registers this holds cost no occupancy that is used.
    __builtin_amdgcn_sched_barrier(0);
    float sc[kBatch];
    float mb = m;
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      sc[b] = mie::group_sum<LPT>(dot4(M::widen(qraw), M::widen(kv[b]), 0.f)) * a.qk_scale;
      sc[b] = valid[b] ? sc[b] : -INFINITY;
      mb = fmaxf(mb, sc[b]);
    }
    // Branch-free, so that the V loads issue beside the K loads instead of
    // after the scores: a batch with no valid row leaves mb = m = -inf, every
    // p = 0 and alpha = 0 on a state that is still empty.
    const float alpha = m == -INFINITY ? 0.f : mie::fast_exp2(m - mb);
    l *= alpha;
    o *= alpha;
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      const float p = valid[b] ? mie::fast_exp2(sc[b] - mb) : 0.f;
      l += p;
      o += p * M::widen(vv[b]);
    }
    m = mb;
  }
  // Merge the TPL row groups of the wave (lanes g * LPT + c hold the same
  // columns for every g), then the W waves through LDS.
#pragma unroll
  for (int off = LPT; off < 64; off <<= 1) {
    const float m2 = __shfl_xor(m, off), l2 = __shfl_xor(l, off);
    f32x4_t o2;
    o2.x = __shfl_xor(o.x, off);
    o2.y = __shfl_xor(o.y, off);
    o2.z = __shfl_xor(o.z, off);
    o2.w = __shfl_xor(o.w, off);
    merge_state(m, l, o, m2, l2, o2);
  }
  if (lane < LPT) {
    *reinterpret_cast<f32x4_t*>(&s_o[wave][c4]) = o;
    if (lane == 0) {
      s_ml[wave][0] = m;
      s_ml[wave][1] = l;
    }
  }
  __syncthreads();
  if (threadIdx.x < LPT) {
    float mm = s_ml[0][0], ll = s_ml[0][1];
    f32x4_t oo = *reinterpret_cast<const f32x4_t*>(&s_o[0][c4]);
#pragma unroll
    for (int w = 1; w < kWaves; ++w)
      merge_state(mm, ll, oo, s_ml[w][0], s_ml[w][1], *reinterpret_cast<const f32x4_t*>(&s_o[w][c4]));
    // No key at all: scaled_dot_product_attention's zeros.  A context block
    // outside the pool gives NaN, as the decode kernels write.
    f32x4_t r = M::R4(ll > 0.f ? oo / ll : f32x4_t{0.f, 0.f, 0.f, 0.f});
    if (any_bad) r = f32x4_t{NAN, NAN, NAN, NAN};
    *reinterpret_cast<f32x4_t*>(&s_attn[c4]) = r;
  }
  __syncthreads();

  // This head's share of the rows: y = W_out[row, h*D : (h+1)*D] . a_h.
  const f32x4_t av = *reinterpret_cast<const f32x4_t*>(&s_attn[c4]);
#pragma unroll
  for (int s = 0; s < kRowSteps; ++s) {
    const int row = row0 + (s * kWaves + wave) * TPL + g;
    const float y = mie::group_sum<LPT>(dot4(M::widen(wv[s]), av, 0.f));
    if (lane % LPT == 0 && row < row_end) {
      if (fabsf(y) < a.fix_limit) {
        const long long fx = llrintf(y * kFix);
        atomicAdd(a.acc + row, static_cast<unsigned long long>(fx));
      } else {
        atomicOr(a.acc + a.dim, 1ull);  // not representable (or NaN): the consumer writes NaN
      }
    }
  }
}

}  // namespace

namespace mie {

int32_t attn_out_check(const void* q, const void* k_pool, const void* v_pool, int64_t pool_stride_block,
                       int64_t pool_stride_head, int32_t num_blocks, const int32_t* block_table,
                       int32_t block_table_len, int32_t max_ctx, int32_t num_heads, int32_t head_dim,
                       int32_t block_size, const void* w_out, const void* acc, int32_t dtype) {
  if (dtype != MIE_DTYPE_F32 && dtype != MIE_DTYPE_BF16)
    return mie::fail(MIE_ERR_UNSUPPORTED, "mie_attn_out_acc: float32 or bfloat16 only (dtype %d)", dtype);
  if (head_dim != 32 && head_dim != 64 && head_dim != 128)
    return mie::fail(MIE_ERR_UNSUPPORTED, "mie_attn_out_acc: head_dim %d (32, 64 or 128)", head_dim);
  if (num_heads <= 0 || num_heads > 4096 || block_size <= 0 || num_blocks <= 0 || block_table_len <= 0)
    return mie::fail(MIE_ERR_INVALID, "mie_attn_out_acc: heads %d, block_size %d, blocks %d, table %d", num_heads,
                     block_size, num_blocks, block_table_len);
  if (max_ctx < 0 || (static_cast<int64_t>(max_ctx) + block_size - 1) / block_size > kMaxTable)
    return mie::fail(MIE_ERR_UNSUPPORTED, "mie_attn_out_acc: contexts up to %d blocks (max_ctx %d, block %d)",
                     kMaxTable, max_ctx, block_size);
  if (!q || !k_pool || !v_pool || !block_table || !w_out || !acc)
    return mie::fail(MIE_ERR_INVALID, "mie_attn_out_acc: null pointer");
  if (pool_stride_head < static_cast<int64_t>(block_size) * head_dim ||
      pool_stride_block < static_cast<int64_t>(num_heads) * pool_stride_head || pool_stride_head % 4 ||
      pool_stride_block % 4)
    return mie::fail(MIE_ERR_INVALID, "mie_attn_out_acc: pool strides overlap or are not multiples of 4");
  auto a16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  if (!a16(q) || !a16(k_pool) || !a16(v_pool) || !a16(w_out) || reinterpret_cast<uintptr_t>(acc) % 8)
    return mie::fail(MIE_ERR_INVALID, "mie_attn_out_acc: q, the pools and W_out must be 16-byte aligned, acc 8");
  return MIE_OK;
}

int32_t attn_out_launch(const void* q, const void* k_pool, const void* v_pool, int64_t pool_stride_block,
                        int64_t pool_stride_head, int32_t num_blocks, const int32_t* block_table,
                        int32_t block_table_len, const int32_t* ctx_dev, int32_t ctx, int32_t max_ctx,
                        int32_t num_heads, int32_t head_dim, int32_t block_size, float scale, const void* w_out,
                        void* acc, int32_t dtype, hipStream_t stream) {
  AttnOutArgs a{};
  a.q = q;
  a.k = k_pool;
  a.v = v_pool;
  a.sblk = pool_stride_block;
  a.shead = pool_stride_head;
  a.num_blocks = num_blocks;
  a.bt = block_table;
  a.bt_len = block_table_len;
  a.ctx_dev = ctx_dev;
  a.ctx = ctx;
  a.max_ctx = max_ctx;
  a.nblk_max = static_cast<int32_t>((static_cast<int64_t>(max_ctx) + block_size - 1) / block_size);
  a.H = num_heads;
  a.bs = mie::FastDiv::make(static_cast<uint32_t>(block_size));
  a.qk_scale = scale * kLog2e;
  a.w = w_out;
  a.dim = num_heads * head_dim;
  a.acc = static_cast<unsigned long long*>(acc);
  a.fix_limit = 2147483648.0f / static_cast<float>(num_heads);  // H partials of |y| * 2^32 < 2^63 / H
  const int tpl = 64 / (head_dim / 4);
  a.rows_per_block = kRowLoads * tpl;
  a.R = (a.dim + a.rows_per_block - 1) / a.rows_per_block;
  const dim3 grid(8 * a.R * ((num_heads + 7) / 8));
  const bool f32 = dtype == MIE_DTYPE_F32;
  const bool short_ctx = max_ctx <= kShortMaxCtx;
#define MIE_ATTN_OUT_CASE(DD)                                                             \
  case DD:                                                                                \
    if (short_ctx) {                                                                      \
      if (f32) attn_out_kernel<float, DD, kShortWaves><<<grid, 64 * kShortWaves, 0, stream>>>(a);       \
      else attn_out_kernel<uint16_t, DD, kShortWaves><<<grid, 64 * kShortWaves, 0, stream>>>(a);        \
    } else {                                                                              \
      if (f32) attn_out_kernel<float, DD, kLongWaves><<<grid, 64 * kLongWaves, 0, stream>>>(a);         \
      else attn_out_kernel<uint16_t, DD, kLongWaves><<<grid, 64 * kLongWaves, 0, stream>>>(a);          \
    }                                                                                     \
    break;
  switch (head_dim) {
    MIE_ATTN_OUT_CASE(32)
    MIE_ATTN_OUT_CASE(64)
    default:
    MIE_ATTN_OUT_CASE(128)
  }
#undef MIE_ATTN_OUT_CASE
  return mie::check_launch("attn_out_kernel");
}

}  // namespace mie

extern "C" int32_t mie_attn_out_acc(const void* q, const void* k_pool, const void* v_pool,
                                    int64_t pool_stride_block, int64_t pool_stride_head, int32_t num_blocks,
                                    const int32_t* block_table, int32_t block_table_len, const int32_t* ctx_dev,
                                    int32_t ctx, int32_t max_ctx, int32_t num_heads, int32_t head_dim,
                                    int32_t block_size, float scale, const void* w_out, void* acc, int32_t dtype,
                                    void* stream) {
  int32_t rc = mie::attn_out_check(q, k_pool, v_pool, pool_stride_block, pool_stride_head, num_blocks, block_table,
                                   block_table_len, max_ctx, num_heads, head_dim, block_size, w_out, acc, dtype);
  if (rc != MIE_OK) return rc;
  if (!ctx_dev && (ctx < 0 || ctx > max_ctx))
    return mie::fail(MIE_ERR_INVALID, "mie_attn_out_acc: ctx %d outside [0, max_ctx=%d]", ctx, max_ctx);
  return mie::attn_out_launch(q, k_pool, v_pool, pool_stride_block, pool_stride_head, num_blocks, block_table,
                              block_table_len, ctx_dev, ctx, max_ctx, num_heads, head_dim, block_size, scale, w_out,
                              acc, dtype, static_cast<hipStream_t>(stream));
}
