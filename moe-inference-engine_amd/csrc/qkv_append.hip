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
// one launch does all of it: every wave normalises x itself (x is 3 KiB at dim
// 768, so recomputing it per wave is cheaper than another launch or a
// barrier), then computes two rows of the projection and stores them where
// they belong - q into q_out, K and V into their pool slots.
//
// Rounding points follow the reference for each dtype: the norm is computed in
// float32 and rounded to the model dtype before the projection (bf16 models
// feed bf16 activations to the GEMM); the projection accumulates in float32,
// adds the bias, and rounds once to the model dtype.
//
// The same body, with a residual epilogue instead of the pool stores, is the
// attention's output projection plus the block's residual add
// (model.py:269 and the block's `x + attention(...)`): out = residual +
// round(W @ x + b) - one launch in place of a GEMM and an add.
//
// With the norm and a pick epilogue it is the decode step's head
// (model.py:564-565 final_norm + output_projection, then generate's greedy
// torch.argmax, model.py:603): logits = round(W @ LayerNorm(x) + b), and each
// workgroup leaves the (value, index) of its largest logit, in torch.argmax's
// order, for a one-workgroup merge - two launches in place of the norm, the
// GEMM and a multi-workgroup argmax.
//
// A projection reads rows*cols*elt bytes of weights once: HBM-bound
// (0.5 flop/B in float32).  Weight loads are issued before the norm so their
// latency overlaps it; they carry the non-temporal hint (each layer's weights
// are streamed once per token).
#include <limits.h>

#include "mie_common.h"

namespace {

constexpr int kRowsPerWave = 2;   // QKV and output projections
constexpr int kHeadRowsPerWave = 4;  // the LM head: fewer waves re-normalising x
constexpr int kWavesPerGroup = 4;

enum Mode { kQkv, kLinear, kHead };

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

struct QkvArgs {
  int32_t rows;  // 3*dim for the QKV projection
  const void* residual;  // linear form: NULL or [rows]
  void* out;             // linear form: [rows]
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
  mie::ArgmaxPair* picks;  // head form: one per workgroup, or NULL for logits only
  // QKV form with the embedding folded in (layer 0 of a decode step): x is
  // round(token_table[*token_id] + pos_table[position]) rather than read, and
  // workgroup 0 stores it to x_out (the block's residual).  NULL: x is read.
  const int64_t* token_id;
  const void* tok_table;
  int32_t vocab;
  const void* pos_table;
  int32_t max_pos;
  void* x_out;
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

// Sums R per-lane partials (one per row) over the wave with a transposed
// butterfly: exchange k (lane bit 5 - k) keeps the upper or lower half of the
// rows, so after log2(R) exchanges lanes [q * 64 / R, (q + 1) * 64 / R) hold
// partials of row q only, which one group sum finishes.  Returns row
// lane / (64 / R)'s total in every lane.
template <int R>
__device__ __forceinline__ float reduce_rows(const float (&v)[R], int lane) {
  float cur[R];
#pragma unroll
  for (int i = 0; i < R; ++i) cur[i] = v[i];
#pragma unroll
  for (int step = 0; (1 << step) < R; ++step) {
    const int off = 32 >> step;
    const int half = R >> (step + 1);
    const bool up = lane & off;
#pragma unroll
    for (int i = 0; i < half; ++i) cur[i] = (up ? cur[i + half] : cur[i]) + __shfl_xor(up ? cur[i] : cur[i + half], off);
  }
  return mie::group_sum<64 / R>(cur[0]);
}

// grid = ceil(rows / (4 * R)), 256 threads.  NCH = 16-byte loads
// per lane per row (ceil(dim / (64 * elements per load))).  QKV: rows = 3*dim
// stored as q and the K/V pool rows; else rows outputs stored to out
// (+ residual).
//
// Every wave loads x and the norm parameters itself, in the lane layout of its
// weight loads (lane l holds elements (c * 64 + l) * EPV ... + EPV - 1 of chunk
// c), and normalises with wave reductions: no LDS and no barrier, so all of a
// wave's global reads - weights, x, norm, bias, residual - are issued together
// and the launch waits on one memory round trip.
template <typename DT, int NCH, int MODE, int R>
__device__ __forceinline__ void projection_body(const QkvArgs& a) {
  constexpr bool QKV = MODE == kQkv;
  using E = Elt<DT>;
  constexpr int EPV = E::kPerVec;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int dim = a.dim;
  const int rows = a.rows;
  const int r0 = (blockIdx.x * kWavesPerGroup + wave) * R;

  // 0. QKV: the token's position, read first; the block-table read that
  //    depends on it is issued after the weight loads, so both overlap them.
  int pos = -1;
  if constexpr (QKV) pos = a.position_dev ? *a.position_dev : a.position;

  // 1. All global reads, unconditional so that they go out together: a load
  //    under a branch whose result merges with a default at the join makes
  //    the compiler wait for it there, before the loads after the branch.
  //    Lanes past dim read element 0 and are zeroed afterwards; an absent norm
  //    parameter, bias or residual reads a stand-in that is then ignored.
  //    Rows past the end repeat the last row and are not stored.
  u32x4_t wr[R][NCH], xw[NCH], gw[NCH], gb[NCH];
  const DT* w = static_cast<const DT*>(a.w_in);
  // Embedding folded in: x's two rows, at addresses that depend on the token
  // id and the position (read above with the position); an id or position
  // outside its table reads row 0 and the row becomes NaN, as mie_embed
  // writes it.
  const bool embed = QKV && a.tok_table != nullptr;
  int64_t tok_id = 0;
  bool emb_ok = true;
  if (QKV && embed) {
    tok_id = *a.token_id;
    emb_ok = tok_id >= 0 && tok_id < a.vocab && pos >= 0 && pos < a.max_pos;
  }
  const DT* x = embed ? static_cast<const DT*>(a.tok_table) + (emb_ok ? tok_id : 0) * dim
                      : static_cast<const DT*>(a.x);
  const DT* xp = static_cast<const DT*>(embed ? a.pos_table : a.x) + (embed && emb_ok ? static_cast<int64_t>(pos) * dim : 0);
  u32x4_t pw[NCH];
  const bool norm = a.ln_w != nullptr;
  const DT* ln_w = norm ? static_cast<const DT*>(a.ln_w) : x;
  const DT* ln_b = a.ln_b ? static_cast<const DT*>(a.ln_b) : x;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int i = (c * 64 + lane) * EPV;
    const int ic = i < dim ? i : 0;
#pragma unroll
    for (int r = 0; r < R; ++r)
      wr[r][c] = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4_t*>(w + static_cast<int64_t>(min(r0 + r, rows - 1)) * dim + ic));
    xw[c] = *reinterpret_cast<const u32x4_t*>(x + ic);
    if (embed) pw[c] = *reinterpret_cast<const u32x4_t*>(xp + ic);
    gw[c] = *reinterpret_cast<const u32x4_t*>(ln_w + ic);
    gb[c] = *reinterpret_cast<const u32x4_t*>(ln_b + ic);
  }
  constexpr int kGroup = 64 / R;  // lanes that finish one row
  const int r_store = r0 + lane / kGroup;
  const bool storing = lane % kGroup == 0 && r_store < rows;
  const int r_read = storing ? r_store : 0;  // w_in holds at least rows elements
  const float bias_raw = E::load(a.b_in ? a.b_in : a.w_in, r_read);
  const float res_raw = E::load(!QKV && a.residual ? a.residual : a.w_in, r_read);
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const u32x4_t zero = {0u, 0u, 0u, 0u};
    const bool in = (c * 64 + lane) * EPV < dim;
#pragma unroll
    for (int r = 0; r < R; ++r) wr[r][c] = in ? wr[r][c] : zero;
    xw[c] = in ? xw[c] : zero;
    gb[c] = a.ln_b ? gb[c] : zero;
  }
  const float bias = a.b_in && storing ? bias_raw : 0.f;
  const float res = !QKV && a.residual && storing ? res_raw : 0.f;
  // The pool slot for the wave's K / V rows (wave-uniform); phys < 0 skips
  // the store, as the append kernel skips an unmapped block.
  int32_t phys = -1;
  uint32_t slot = 0;
  if constexpr (QKV) {
    if (r0 + R > a.dim && pos >= 0) {
      const uint32_t lb = a.bs.div(static_cast<uint32_t>(pos));
      slot = static_cast<uint32_t>(pos) - lb * a.bs.d;
      phys = lb < static_cast<uint32_t>(a.bt_len) ? a.block_table[lb] : -1;
    }
  }

  // 2. x, normalised when ln_w is given (float32 mean and biased variance, then
  //    rounded to the model dtype as the reference's norm output is), in
  //    registers; elements past dim are zero.
  float y[NCH][EPV];
#pragma unroll
  for (int c = 0; c < NCH; ++c) E::widen(xw[c], y[c]);
  if (embed) {
    // x = token row + positional row, summed in float32 and rounded once
    // (mie_embed's arithmetic); workgroup 0 keeps it as the block's residual.
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      float q[EPV];
      E::widen(pw[c], q);
      const bool in = (c * 64 + lane) * EPV < dim;
#pragma unroll
      for (int e = 0; e < EPV; ++e) y[c][e] = in ? (emb_ok ? E::round(y[c][e] + q[e]) : NAN) : 0.f;
    }
    if (blockIdx.x == 0 && wave == 0) {
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        const int i = (c * 64 + lane) * EPV;
        if (i < dim) {
#pragma unroll
          for (int e = 0; e < EPV; ++e) E::store(a.x_out, i + e, y[c][e]);
        }
      }
    }
  }
  if (norm) {
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
      for (int e = 0; e < EPV; ++e) s += y[c][e];
    const float mean = mie::wave_sum(s) / dim;
    float q = 0.f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const bool valid = (c * 64 + lane) * EPV < dim;
#pragma unroll
      for (int e = 0; e < EPV; ++e) {
        const float d = valid ? y[c][e] - mean : 0.f;
        q = fmaf(d, d, q);
      }
    }
    const float rstd = rsqrtf(mie::wave_sum(q) / dim + a.ln_eps);
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      float fw[EPV], fb[EPV];
      E::widen(gw[c], fw);
      E::widen(gb[c], fb);
#pragma unroll
      for (int e = 0; e < EPV; ++e) y[c][e] = E::round((y[c][e] - mean) * rstd * fw[e] + fb[e]);
    }
  }

  // 3. R dot products per wave (zero weights past dim).
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    acc[r] = 0.f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      float f[EPV];
      E::widen(wr[r][c], f);
#pragma unroll
      for (int e = 0; e < EPV; ++e) acc[r] = fmaf(f[e], y[c][e], acc[r]);
    }
  }
  const float t = reduce_rows<R>(acc, lane);
  if constexpr (MODE == kHead) {
    const float logit = E::round(t + bias);
    if (storing) E::store(a.out, r_store, logit);
    if (a.picks) {  // kernel argument: every wave takes the same branch
      __shared__ float s_v[kWavesPerGroup];
      __shared__ int s_i[kWavesPerGroup];
      float v = storing ? logit : -INFINITY;
      int i = storing ? r_store : INT_MAX;
      mie::wave_argmax(v, i);
      if (lane == 0) {
        s_v[wave] = v;
        s_i[wave] = i;
      }
      __syncthreads();
      if (threadIdx.x == 0) {
        for (int w = 1; w < kWavesPerGroup; ++w) mie::argmax_take(v, i, s_v[w], s_i[w]);
        a.picks[blockIdx.x] = mie::ArgmaxPair{v, i};
      }
    }
    return;
  }
  if (!storing) return;
  const int r = r_store;

  // 5. Store: the linear form's output, q, or the K / V row of the token's
  //    pool slot.
  if constexpr (!QKV) {
    E::store(a.out, r, a.residual ? res + E::round(t + bias) : t + bias);
    return;
  }
  const float out = t + bias;
  if (r < dim) {
    E::store(a.q_out, r, out);
    return;
  }
  const bool is_v = r >= 2 * dim;
  const int j = r - (is_v ? 2 * dim : dim);
  const int h = j / a.head_dim;
  const int d = j - h * a.head_dim;
  if (phys < 0 || phys >= a.num_blocks) return;
  E::store(is_v ? a.v_pool : a.k_pool, phys * a.sblk + h * a.shead + static_cast<int64_t>(slot) * a.head_dim + d, out);
}

template <typename DT, int NCH>
__global__ __launch_bounds__(256) void qkv_append_kernel(QkvArgs a) {
  projection_body<DT, NCH, kQkv, kRowsPerWave>(a);
}

template <typename DT, int NCH>
__global__ __launch_bounds__(256) void linear_residual_kernel(QkvArgs a) {
  projection_body<DT, NCH, kLinear, kRowsPerWave>(a);
}

template <typename DT, int NCH>
__global__ __launch_bounds__(256) void lm_head_kernel(QkvArgs a) {
  projection_body<DT, NCH, kHead, kHeadRowsPerWave>(a);
}

constexpr int rows_per_wave(int mode) { return mode == kHead ? kHeadRowsPerWave : kRowsPerWave; }

int32_t groups_for(int mode, int rows) {
  const int per_group = kWavesPerGroup * rows_per_wave(mode);
  return (rows + per_group - 1) / per_group;
}

template <typename DT, int MODE>
int32_t launch(const QkvArgs& a, hipStream_t st) {
  const int nch = (a.dim + 64 * Elt<DT>::kPerVec - 1) / (64 * Elt<DT>::kPerVec);
  const int groups = groups_for(MODE, a.rows);
#define MIE_PROJ_CASE(N)                                             \
  case N:                                                            \
    if (MODE == kQkv) {                                              \
      qkv_append_kernel<DT, N><<<groups, 256, 0, st>>>(a);           \
    } else if (MODE == kLinear) {                                    \
      linear_residual_kernel<DT, N><<<groups, 256, 0, st>>>(a);      \
    } else {                                                         \
      lm_head_kernel<DT, N><<<groups, 256, 0, st>>>(a);              \
    }                                                                \
    break;
  switch (nch) {
    MIE_PROJ_CASE(1) MIE_PROJ_CASE(2) MIE_PROJ_CASE(3) MIE_PROJ_CASE(4)
    MIE_PROJ_CASE(5) MIE_PROJ_CASE(6) MIE_PROJ_CASE(7) MIE_PROJ_CASE(8)
    default: return mie::fail(MIE_ERR_UNSUPPORTED, "projection: width %d is too large", a.dim);
  }
#undef MIE_PROJ_CASE
  return mie::check_launch(MODE == kQkv ? "qkv_append_kernel"
                                        : (MODE == kLinear ? "linear_residual_kernel" : "lm_head_kernel"));
}

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

}  // namespace

extern "C" int32_t mie_qkv_append_supported(int32_t dim, int32_t dtype) {
  if (dim <= 0) return 0;
  if (dtype == MIE_DTYPE_F32) return dim % 4 == 0 && dim <= 8 * 64 * 4;
  if (dtype == MIE_DTYPE_BF16) return dim % 8 == 0 && dim <= 8 * 64 * 8;
  return 0;
}

namespace mie {

int32_t qkv_append_check(const void* x, const void* ln_weight, const void* ln_bias, const void* w_in, int32_t dim,
                         const void* k_pool, const void* v_pool, int64_t pool_stride_block, int64_t pool_stride_head,
                         int32_t num_blocks, const int32_t* block_table, int32_t block_table_len,
                         const int32_t* position_dev, int32_t position, const void* q_out, int32_t num_heads,
                         int32_t head_dim, int32_t block_size, int32_t dtype) {
  if (!mie_qkv_append_supported(dim, dtype))
    return mie::fail(MIE_ERR_UNSUPPORTED, "mie_qkv_append: dim %d with dtype %d is not built", dim, dtype);
  if (num_heads <= 0 || head_dim <= 0 || num_heads * head_dim != dim)
    return mie::fail(MIE_ERR_INVALID, "mie_qkv_append: heads %d x head_dim %d != dim %d", num_heads, head_dim, dim);
  if (block_size <= 0 || num_blocks <= 0 || block_table_len < 0)
    return mie::fail(MIE_ERR_INVALID, "mie_qkv_append: block_size %d, num_blocks %d, table length %d", block_size,
                     num_blocks, block_table_len);
  if (!x || !w_in || !k_pool || !v_pool || !block_table || !q_out)
    return mie::fail(MIE_ERR_INVALID, "mie_qkv_append: null pointer");
  if (ln_bias && !ln_weight) return mie::fail(MIE_ERR_INVALID, "mie_qkv_append: a norm bias needs a norm weight");
  if (!aligned16(w_in) || !aligned16(x) || !aligned16(ln_weight) || !aligned16(ln_bias))
    return mie::fail(MIE_ERR_INVALID, "mie_qkv_append: x, the norm parameters and the projection weight must be "
                                      "16-byte aligned");
  if (pool_stride_head < static_cast<int64_t>(block_size) * head_dim ||
      pool_stride_block < static_cast<int64_t>(num_heads) * pool_stride_head)
    return mie::fail(MIE_ERR_INVALID, "mie_qkv_append: pool strides (%lld, %lld) overlap",
                     static_cast<long long>(pool_stride_block), static_cast<long long>(pool_stride_head));
  if (!position_dev && position < 0) return mie::fail(MIE_ERR_INVALID, "mie_qkv_append: position %d", position);
  return MIE_OK;
}

int32_t linear_residual_check(const void* x, const void* weight, const void* out, int32_t rows, int32_t cols,
                              int32_t dtype) {
  if (!mie_qkv_append_supported(cols, dtype))
    return mie::fail(MIE_ERR_UNSUPPORTED, "mie_linear_residual: width %d with dtype %d is not built", cols, dtype);
  if (rows <= 0) return mie::fail(MIE_ERR_INVALID, "mie_linear_residual: rows %d", rows);
  if (!x || !weight || !out) return mie::fail(MIE_ERR_INVALID, "mie_linear_residual: null pointer");
  if (!aligned16(weight) || !aligned16(x))
    return mie::fail(MIE_ERR_INVALID, "mie_linear_residual: x and the weight must be 16-byte aligned");
  return MIE_OK;
}

}  // namespace mie

namespace {

int32_t qkv_launch(const void* x, const void* ln_weight, const void* ln_bias, float ln_eps, const void* w_in,
                   const void* b_in, int32_t dim, void* k_pool, void* v_pool, int64_t pool_stride_block,
                   int64_t pool_stride_head, int32_t num_blocks, const int32_t* block_table, int32_t block_table_len,
                   const int32_t* position_dev, int32_t position, void* q_out, int32_t num_heads, int32_t head_dim,
                   int32_t block_size, int32_t dtype, void* stream, const mie::QkvEmbedding* embed) {
  QkvArgs a{};
  a.rows = 3 * dim;
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
  if (embed) {
    a.token_id = embed->token_id;
    a.tok_table = embed->token_table;
    a.vocab = embed->vocab;
    a.pos_table = embed->pos_table;
    a.max_pos = embed->max_positions;
    a.x_out = embed->x_out;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == MIE_DTYPE_F32) return launch<float, kQkv>(a, st);
  return launch<uint16_t, kQkv>(a, st);
}

}  // namespace

namespace mie {

int32_t qkv_embedding_check(const QkvEmbedding& e, int32_t dim) {
  if (!e.token_id || !e.token_table || !e.pos_table || !e.x_out || e.vocab <= 0 || e.max_positions <= 0)
    return mie::fail(MIE_ERR_INVALID, "embedding: null pointer, vocab %d or positions %d", e.vocab, e.max_positions);
  if (!aligned16(e.token_table) || !aligned16(e.pos_table) || !aligned16(e.x_out))
    return mie::fail(MIE_ERR_INVALID, "embedding: the tables and the output row must be 16-byte aligned");
  if (reinterpret_cast<uintptr_t>(e.token_id) % 8) return mie::fail(MIE_ERR_INVALID, "embedding: misaligned token id");
  (void)dim;
  return MIE_OK;
}

int32_t qkv_append_embedded(const QkvEmbedding& e, const void* ln_weight, const void* ln_bias, float ln_eps,
                            const void* w_in, const void* b_in, int32_t dim, void* k_pool, void* v_pool,
                            int64_t pool_stride_block, int64_t pool_stride_head, int32_t num_blocks,
                            const int32_t* block_table, int32_t block_table_len, const int32_t* position_dev,
                            int32_t position, void* q_out, int32_t num_heads, int32_t head_dim, int32_t block_size,
                            int32_t dtype, void* stream) {
  // The stand-in x only passes the shared checks; the kernel reads the tables.
  int32_t rc = qkv_append_check(e.x_out, ln_weight, ln_bias, w_in, dim, k_pool, v_pool, pool_stride_block,
                                pool_stride_head, num_blocks, block_table, block_table_len, position_dev, position,
                                q_out, num_heads, head_dim, block_size, dtype);
  if (rc != MIE_OK) return rc;
  rc = qkv_embedding_check(e, dim);
  if (rc != MIE_OK) return rc;
  return qkv_launch(nullptr, ln_weight, ln_bias, ln_eps, w_in, b_in, dim, k_pool, v_pool, pool_stride_block,
                    pool_stride_head, num_blocks, block_table, block_table_len, position_dev, position, q_out,
                    num_heads, head_dim, block_size, dtype, stream, &e);
}

}  // namespace mie

extern "C" int32_t mie_qkv_append(const void* x, const void* ln_weight, const void* ln_bias, float ln_eps,
                                  const void* w_in, const void* b_in, int32_t dim, void* k_pool, void* v_pool,
                                  int64_t pool_stride_block, int64_t pool_stride_head, int32_t num_blocks,
                                  const int32_t* block_table, int32_t block_table_len, const int32_t* position_dev,
                                  int32_t position, void* q_out, int32_t num_heads, int32_t head_dim,
                                  int32_t block_size, int32_t dtype, void* stream) {
  const int32_t rc = mie::qkv_append_check(x, ln_weight, ln_bias, w_in, dim, k_pool, v_pool, pool_stride_block,
                                           pool_stride_head, num_blocks, block_table, block_table_len, position_dev,
                                           position, q_out, num_heads, head_dim, block_size, dtype);
  if (rc != MIE_OK) return rc;
  return qkv_launch(x, ln_weight, ln_bias, ln_eps, w_in, b_in, dim, k_pool, v_pool, pool_stride_block,
                    pool_stride_head, num_blocks, block_table, block_table_len, position_dev, position, q_out,
                    num_heads, head_dim, block_size, dtype, stream, nullptr);
}

extern "C" int32_t mie_linear_residual(const void* x, const void* weight, const void* bias, const void* residual,
                                       void* out, int32_t rows, int32_t cols, int32_t dtype, void* stream) {
  const int32_t rc = mie::linear_residual_check(x, weight, out, rows, cols, dtype);
  if (rc != MIE_OK) return rc;
  QkvArgs a{};
  a.rows = rows;
  a.residual = residual;
  a.out = out;
  a.x = x;
  a.w_in = weight;
  a.b_in = bias;
  a.dim = cols;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == MIE_DTYPE_F32) return launch<float, kLinear>(a, st);
  return launch<uint16_t, kLinear>(a, st);
}

extern "C" int64_t mie_lm_head_workspace(int32_t vocab) {
  return vocab > 0 ? static_cast<int64_t>(groups_for(kHead, vocab)) * sizeof(mie::ArgmaxPair) : 0;
}

extern "C" int32_t mie_lm_head(const void* x, const void* ln_weight, const void* ln_bias, float ln_eps,
                               const void* weight, const void* bias, int32_t vocab, int32_t dim, void* logits,
                               void* token_out, void* workspace, int64_t workspace_bytes, int32_t* advance,
                               int32_t n_advance, int32_t dtype, void* stream) {
  if (!mie_qkv_append_supported(dim, dtype))
    return mie::fail(MIE_ERR_UNSUPPORTED, "mie_lm_head: width %d with dtype %d is not built", dim, dtype);
  if (vocab <= 0 || vocab > INT32_MAX - 64) return mie::fail(MIE_ERR_INVALID, "mie_lm_head: vocab %d", vocab);
  if (!x || !weight || !logits) return mie::fail(MIE_ERR_INVALID, "mie_lm_head: null pointer");
  if (ln_bias && !ln_weight) return mie::fail(MIE_ERR_INVALID, "mie_lm_head: a norm bias needs a norm weight");
  if (!aligned16(weight) || !aligned16(x) || !aligned16(ln_weight) || !aligned16(ln_bias))
    return mie::fail(MIE_ERR_INVALID, "mie_lm_head: x, the norm parameters and the weight must be 16-byte aligned");
  const int64_t need = mie_lm_head_workspace(vocab);
  if ((token_out || workspace) && (!workspace || workspace_bytes < need))
    return mie::fail(MIE_ERR_INVALID, "mie_lm_head: the pick needs a %lld-byte workspace (got %lld)",
                     static_cast<long long>(need), static_cast<long long>(workspace ? workspace_bytes : 0));
  if (n_advance < 0 || n_advance > 64 || (n_advance > 0 && (!advance || !token_out)))
    return mie::fail(MIE_ERR_INVALID, "mie_lm_head: %d counters to advance (at most 64, with a token)", n_advance);
  if (workspace && (reinterpret_cast<uintptr_t>(workspace) % alignof(mie::ArgmaxPair) ||
                    reinterpret_cast<uintptr_t>(token_out) % alignof(int64_t)))
    return mie::fail(MIE_ERR_INVALID, "mie_lm_head: misaligned workspace or token");
  QkvArgs a{};
  a.rows = vocab;
  a.out = logits;
  a.x = x;
  a.ln_w = ln_weight;
  a.ln_b = ln_bias;
  a.ln_eps = ln_eps;
  a.w_in = weight;
  a.b_in = bias;
  a.dim = dim;
  a.picks = static_cast<mie::ArgmaxPair*>(workspace);  // NULL: no picks
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int32_t rc = dtype == MIE_DTYPE_F32 ? launch<float, kHead>(a, st) : launch<uint16_t, kHead>(a, st);
  if (rc != MIE_OK || !token_out) return rc;
  return mie::launch_argmax_pairs(a.picks, groups_for(kHead, vocab), vocab, static_cast<int64_t*>(token_out), advance,
                                  n_advance, st);
}
