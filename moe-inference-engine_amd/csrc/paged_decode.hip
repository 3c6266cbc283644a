// Direct paged decode attention for gfx950 (MI355X).
//
// Replaces the reference's Triton _paged_decode_kernel
// (src/moe_engine/paged_attention.py:46-110): per (sequence, head)
//   out = softmax(scale * q . K^T) . V   over tokens [0, ctx) of a paged pool.
//
// Work decomposition.  One 64-lane wavefront owns one (sequence, head,
// partition) work item; a workgroup holds WAVES heads of the same sequence and
// partition, so its waves walk the same block-table entries and neighbouring
// (block, head) tiles.  grid = (partitions, ceil(H / WAVES), batch); work items
// past a sequence's last partition exit at once, so ragged batches need no
// host-side work list and no device-to-host read of the lengths.
//
// Lane layout.  A token's head_dim row is split into NV slices of VEC elements
// (VB = 16 bytes for f32 and bf16), held by LPT = next_pow2(NV) consecutive
// lanes; one wave load therefore reads TPL = 64 / LPT whole token rows, and for
// block_size >= TPL those rows are one contiguous run of the (block, head)
// tile: a fully coalesced 1 KiB access.  A tile is ROWS such loads of K and of
// V, all issued before any arithmetic.
//
// Online softmax.  Each TPL-lane group keeps its own running (max, sum, acc)
// over the tokens it reads, so the per-tile work needs no cross-group
// communication: scores are reduced only across the LPT lanes of a token with
// DPP (quad_perm / row_half_mirror / row_mirror), and the groups are merged
// once per work item with log-sum-exp shuffles.  Scores are kept in the log2
// domain (q.k * scale * log2 e) so every exponential is one v_exp_f32.
//
// Split context.  With more than one partition per sequence the work item
// writes its (max, sum, acc[D]) partial to the workspace and a second kernel
// merges the partials of each (sequence, head); a sequence that fits one
// partition is normalised and written by the first kernel.
#include <math.h>

#include "mie_common.h"

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kWaves = 4;            // heads (wavefronts) per workgroup
constexpr int kSinglePassCtx = 256;  // auto plan: one partition up to this context
constexpr int kTargetItems = 16384;  // auto plan: grid work items to aim below

constexpr int next_pow2(int x) {
  int p = 1;
  while (p < x) p <<= 1;
  return p;
}

template <int DT> struct Elt;
template <> struct Elt<MIE_DTYPE_F32> { static constexpr int size = 4; };
template <> struct Elt<MIE_DTYPE_BF16> { static constexpr int size = 2; };

template <int DT, int D>
struct Geometry {
  static constexpr int ELT = Elt<DT>::size;
  static constexpr int VEC = (16 / ELT) < D ? (16 / ELT) : D;  // elements per lane load
  static constexpr int VB = VEC * ELT;                          // bytes per lane load
  static constexpr int NW = VB / 4;                             // 32-bit words per lane load
  static constexpr int NV = D / VEC;                            // lanes with data per token
  static constexpr int LPT = next_pow2(NV);                     // lanes per token
  static constexpr int TPL = 64 / LPT;                          // tokens per wave load
  static constexpr int ROWS_BY_REGS = 16 / NW;                  // <= 64 B of K per lane per tile
  static constexpr int ROWS_BY_TILE = (64 / TPL) > 0 ? 64 / TPL : 1;
  static constexpr int ROWS = ROWS_BY_REGS < ROWS_BY_TILE ? ROWS_BY_REGS : ROWS_BY_TILE;
  static constexpr int TILE = ROWS * TPL;  // tokens per tile (a power of two)
  static_assert(D % VEC == 0, "head_dim must be a multiple of the lane vector");
  static_assert(VB == 8 || VB == 16, "lane loads are 8 or 16 bytes");
  static_assert(LPT <= 64, "head_dim too large for one wavefront");
};

template <int NW> struct Words { uint32_t w[NW]; };

template <int NW>
__device__ __forceinline__ Words<NW> load_words(const char* p) {
  Words<NW> r;
  if constexpr (NW == 4) {
    const uint4 x = *reinterpret_cast<const uint4*>(p);
    r.w[0] = x.x; r.w[1] = x.y; r.w[2] = x.z; r.w[3] = x.w;
  } else {
    const uint2 x = *reinterpret_cast<const uint2*>(p);
    r.w[0] = x.x; r.w[1] = x.y;
  }
  return r;
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

struct DecodeArgs {
  const char* q;
  int64_t q_sb, q_sh;  // elements
  const char* k;
  const char* v;
  int64_t kv_sblk, kv_sh;  // elements
  int32_t num_blocks;
  const int32_t* bt;
  int64_t bt_stride;
  uint32_t bt_cap;  // entries readable per table row
  const int32_t* ctx_lens;
  int32_t ctx_len;
  int32_t max_ctx;
  int32_t H;
  mie::FastDiv bs;
  float qk_scale;  // scale * log2(e)
  char* out;
  int64_t o_sb, o_sh;  // elements
  int32_t out_f32;
  float* ws_ml;   // [B, H, max_parts, 2]  (running max in log2 units, sum)
  float* ws_acc;  // [B, H, max_parts, D]
  int32_t max_parts;
  int32_t part_shift;  // partition = 1 << part_shift tokens
};

__device__ __forceinline__ int seq_ctx(const DecodeArgs& a, int b) {
  int c = a.ctx_lens ? a.ctx_lens[b] : a.ctx_len;
  c = c < 0 ? 0 : c;
  return c < a.max_ctx ? c : a.max_ctx;
}

// Writes VEC consecutive outputs starting at `dst` (element pointer math done
// by the caller) in f32 or the kernel's dtype.
template <int DT, int VEC>
__device__ __forceinline__ void store_out(char* base, int64_t elem_off, const float* val, bool f32) {
  if (f32 || DT == MIE_DTYPE_F32) {
    float* p = reinterpret_cast<float*>(base) + elem_off;
#pragma unroll
    for (int i = 0; i < VEC; i += 4) {
      if constexpr (VEC >= 4) {
        *reinterpret_cast<float4*>(p + i) = make_float4(val[i], val[i + 1], val[i + 2], val[i + 3]);
      }
    }
  } else {
    uint32_t* p = reinterpret_cast<uint32_t*>(reinterpret_cast<uint16_t*>(base) + elem_off);
    if constexpr (VEC == 8) {
      *reinterpret_cast<uint4*>(p) =
          make_uint4(mie::pack_bf16x2(val[0], val[1]), mie::pack_bf16x2(val[2], val[3]),
                     mie::pack_bf16x2(val[4], val[5]), mie::pack_bf16x2(val[6], val[7]));
    } else {
      *reinterpret_cast<uint2*>(p) =
          make_uint2(mie::pack_bf16x2(val[0], val[1]), mie::pack_bf16x2(val[2], val[3]));
    }
  }
}

template <int DT, int D>
__global__ __launch_bounds__(64 * kWaves) void paged_decode_kernel(DecodeArgs a) {
  using G = Geometry<DT, D>;
  constexpr int ELT = G::ELT, VEC = G::VEC, NW = G::NW, LPT = G::LPT, TPL = G::TPL;
  constexpr int ROWS = G::ROWS, TILE = G::TILE;

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int h = blockIdx.y * kWaves + wave;
  if (h >= a.H) return;
  const int b = blockIdx.z;
  const int part = blockIdx.x;
  const int ctx = seq_ctx(a, b);
  const int nparts = (ctx + (1 << a.part_shift) - 1) >> a.part_shift;

  const int g = lane / LPT;   // token group within a wave load
  const int jl = lane % LPT;  // slice of the head_dim row
  const bool jv = jl < G::NV;

  if (ctx == 0) {  // no keys: scaled_dot_product_attention returns zeros
    if (part == 0 && g == 0 && jv) {
      float zero[VEC];
#pragma unroll
      for (int i = 0; i < VEC; ++i) zero[i] = 0.f;
      store_out<DT, VEC>(a.out, b * a.o_sb + h * a.o_sh + jl * VEC, zero, a.out_f32);
    }
    return;
  }
  if (part >= nparts) return;
  const int t_begin = part << a.part_shift;
  const int t_end = min(ctx, t_begin + (1 << a.part_shift));

  // Query slice for this lane: bf16 stays packed for v_dot2; f32 is pre-scaled.
  Words<NW> qw;
#pragma unroll
  for (int w = 0; w < NW; ++w) qw.w[w] = 0u;
  if (jv) qw = load_words<NW>(a.q + (b * a.q_sb + h * a.q_sh + jl * VEC) * ELT);
  float qf[VEC];
  if constexpr (DT == MIE_DTYPE_F32) {
#pragma unroll
    for (int i = 0; i < VEC; ++i) qf[i] = __uint_as_float(qw.w[i]) * a.qk_scale;
  }

  const int32_t* bt = a.bt + b * a.bt_stride;
  const int64_t lane_off = (h * a.kv_sh + jl * VEC) * ELT;
  const char* kbase = a.k + lane_off;
  const char* vbase = a.v + lane_off;
  const int64_t blk_bytes = a.kv_sblk * ELT;

  float m = -INFINITY, l = 0.f;
  float acc[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) acc[i] = 0.f;
  bool bad = false;

  for (int t0 = t_begin; t0 < t_end; t0 += TILE) {
    Words<NW> kr[ROWS], vr[ROWS];
    bool valid[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
      const int t = t0 + r * TPL + g;
      bool ok = t < t_end;
      int64_t off = 0;
      if (ok) {
        const uint32_t blk = a.bs.div(static_cast<uint32_t>(t));
        const uint32_t slot = static_cast<uint32_t>(t) - blk * a.bs.d;
        const int32_t phys = blk < a.bt_cap ? bt[blk] : -1;
        if (phys < 0 || phys >= a.num_blocks) {
          bad = true;
          ok = false;
        }
        off = phys * blk_bytes + static_cast<int64_t>(slot) * (D * ELT);
      }
      valid[r] = ok;
#pragma unroll
      for (int w = 0; w < NW; ++w) { kr[r].w[w] = 0u; vr[r].w[w] = 0u; }
      if (ok && jv) {
        kr[r] = load_words<NW>(kbase + off);
        vr[r] = load_words<NW>(vbase + off);
      }
    }

    float s[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
      float part_dot = 0.f;
      if constexpr (DT == MIE_DTYPE_BF16) {
#pragma unroll
        for (int w = 0; w < NW; ++w)
          part_dot = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, kr[r].w[w]),
                                                     __builtin_bit_cast(bf16x2_t, qw.w[w]),
                                                     part_dot, false);
        s[r] = mie::group_sum<LPT>(part_dot) * a.qk_scale;
      } else {
#pragma unroll
        for (int i = 0; i < VEC; ++i) part_dot = fmaf(__uint_as_float(kr[r].w[i]), qf[i], part_dot);
        s[r] = mie::group_sum<LPT>(part_dot);
      }
      s[r] = valid[r] ? s[r] : -INFINITY;
    }

    float tmax = s[0];
#pragma unroll
    for (int r = 1; r < ROWS; ++r) tmax = fmaxf(tmax, s[r]);
    const float m_new = fmaxf(m, tmax);
    const float mref = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = mie::fast_exp2(m - mref);
    float p[ROWS];
    float psum = 0.f;
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
      p[r] = mie::fast_exp2(s[r] - mref);
      psum += p[r];
    }
    l = l * alpha + psum;
#pragma unroll
    for (int i = 0; i < VEC; ++i) acc[i] *= alpha;
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
      if constexpr (DT == MIE_DTYPE_BF16) {
#pragma unroll
        for (int w = 0; w < NW; ++w) {
          acc[2 * w] = fmaf(p[r], mie::bf16_lo(vr[r].w[w]), acc[2 * w]);
          acc[2 * w + 1] = fmaf(p[r], mie::bf16_hi(vr[r].w[w]), acc[2 * w + 1]);
        }
      } else {
#pragma unroll
        for (int i = 0; i < VEC; ++i) acc[i] = fmaf(p[r], __uint_as_float(vr[r].w[i]), acc[i]);
      }
    }
    m = m_new;
  }

  // Merge the TPL token groups (lanes jl, jl + LPT, ...) with log-sum-exp.
#pragma unroll
  for (int off = LPT; off < 64; off <<= 1) {
    const float mo = __shfl_xor(m, off);
    const float lo = __shfl_xor(l, off);
    const float mn = fmaxf(m, mo);
    const float mr = mn == -INFINITY ? 0.f : mn;
    const float ca = mie::fast_exp2(m - mr);
    const float cb = mie::fast_exp2(mo - mr);
    l = l * ca + lo * cb;
#pragma unroll
    for (int i = 0; i < VEC; ++i) acc[i] = acc[i] * ca + __shfl_xor(acc[i], off) * cb;
    m = mn;
  }
  bad = __any(bad);

  if (g != 0 || !jv) return;
  if (nparts == 1) {
    const float inv = bad ? NAN : 1.f / l;
    float val[VEC];
#pragma unroll
    for (int i = 0; i < VEC; ++i) val[i] = acc[i] * inv;
    store_out<DT, VEC>(a.out, b * a.o_sb + h * a.o_sh + jl * VEC, val, a.out_f32);
  } else {
    const int64_t item = (static_cast<int64_t>(b) * a.H + h) * a.max_parts + part;
    float* dst = a.ws_acc + item * D + jl * VEC;
#pragma unroll
    for (int i = 0; i < VEC; i += 4) *reinterpret_cast<float4*>(dst + i) = make_float4(acc[i], acc[i + 1], acc[i + 2], acc[i + 3]);
    if (jl == 0) {
      a.ws_ml[2 * item] = bad ? NAN : m;
      a.ws_ml[2 * item + 1] = l;
    }
  }
}

// Merge the partition partials of one (sequence, head):
//   M = max_i m_i,  w_i = 2^(m_i - M),  out = sum_i w_i acc_i / sum_i w_i l_i.
// 256 threads: COLS = D columns x RROWS partition lanes, combined through LDS.
template <int DT, int D>
__global__ __launch_bounds__(256) void paged_decode_reduce_kernel(DecodeArgs a) {
  constexpr int RROWS = 256 / D > 0 ? 256 / D : 1;
  __shared__ float red[256];
  __shared__ float stat[2];
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  const int ctx = seq_ctx(a, b);
  const int nparts = (ctx + (1 << a.part_shift) - 1) >> a.part_shift;
  if (nparts <= 1) return;
  const int tid = threadIdx.x;
  const int64_t base = (static_cast<int64_t>(b) * a.H + h) * a.max_parts;
  const float* ml = a.ws_ml + 2 * base;

  // Global max, then the weighted sum of the partition sums (wave 0 only).
  if (tid < 64) {
    float mx = -INFINITY;
    for (int i = tid; i < nparts; i += 64) mx = fmaxf(mx, ml[2 * i]);
    mx = mie::wave_max(mx);
    const float mr = mx == -INFINITY ? 0.f : mx;
    float ls = 0.f;
    for (int i = tid; i < nparts; i += 64) ls += ml[2 * i + 1] * mie::fast_exp2(ml[2 * i] - mr);
    ls = mie::wave_sum(ls);
    if (tid == 0) {
      stat[0] = mr;
      stat[1] = ls;
    }
  }
  __syncthreads();
  const float mr = stat[0];
  const float inv = 1.f / stat[1];

  const int col = tid % D;
  const int row = tid / D;
  float accv = 0.f;
  if (row < RROWS) {
    const float* acc = a.ws_acc + base * D + col;
    for (int i = row; i < nparts; i += RROWS) accv += acc[static_cast<int64_t>(i) * D] * mie::fast_exp2(ml[2 * i] - mr);
  }
  red[tid] = accv;
  __syncthreads();
  if (tid < D) {
    float sum = 0.f;
    for (int r = 0; r < RROWS; ++r) sum += red[r * D + tid];
    sum *= inv;
    const int64_t o = b * a.o_sb + h * a.o_sh + tid;
    if (a.out_f32 || DT == MIE_DTYPE_F32) {
      reinterpret_cast<float*>(a.out)[o] = sum;
    } else {
      reinterpret_cast<uint16_t*>(a.out)[o] = static_cast<uint16_t>(mie::f32_to_bf16_bits(sum));
    }
  }
}

// ---- host side --------------------------------------------------------------

template <int DT, int D>
constexpr int tile_of() { return Geometry<DT, D>::TILE; }

// Head dims built for each dtype.  Each needs D % VEC == 0 (VEC = 4 for f32,
// min(8, D) for bf16) and D <= 256.
#define MIE_FOR_EACH_HEAD_DIM(X) X(4) X(8) X(16) X(32) X(64) X(96) X(128) X(256)

int tile_for(int dtype, int head_dim) {
#define MIE_TILE_CASE(DD)                                            \
  case DD:                                                           \
    return dtype == MIE_DTYPE_F32 ? tile_of<MIE_DTYPE_F32, DD>()     \
                                  : tile_of<MIE_DTYPE_BF16, DD>();
  if (dtype != MIE_DTYPE_F32 && dtype != MIE_DTYPE_BF16) return 0;
  switch (head_dim) {
    MIE_FOR_EACH_HEAD_DIM(MIE_TILE_CASE)
    default: return 0;
  }
#undef MIE_TILE_CASE
}

int ilog2(uint32_t x) {
  int s = 0;
  while ((1u << s) < x) ++s;
  return s;
}

int32_t plan(int32_t batch, int32_t num_heads, int32_t head_dim, int32_t max_ctx, int32_t dtype,
             int32_t requested, int32_t* part_out, int64_t* ws_out, int32_t* max_parts_out) {
  const int tile = tile_for(dtype, head_dim);
  if (tile == 0)
    return mie::fail(MIE_ERR_UNSUPPORTED, "mie_paged_decode: head_dim %d dtype %d not built", head_dim,
                     dtype);
  if (batch < 0 || num_heads <= 0 || max_ctx < 0)
    return mie::fail(MIE_ERR_INVALID, "mie_paged_decode: bad shape batch=%d heads=%d max_ctx=%d", batch,
                     num_heads, max_ctx);
  int64_t part;
  if (requested > 0) {
    if ((requested & (requested - 1)) != 0 || requested % tile != 0)
      return mie::fail(MIE_ERR_INVALID,
                       "mie_paged_decode: partition_tokens %d must be a power of two and a multiple "
                       "of the %d-token tile",
                       requested, tile);
    part = requested;
  } else if (max_ctx <= kSinglePassCtx) {
    part = tile;
    while (part < max_ctx) part <<= 1;
  } else {
    part = tile;
    const int64_t rows = static_cast<int64_t>(batch) * num_heads;
    while (part < max_ctx && rows * ((max_ctx + part - 1) / part) > kTargetItems) part <<= 1;
  }
  if (part > (int64_t{1} << 30)) part = int64_t{1} << 30;
  const int64_t max_parts = max_ctx > 0 ? (max_ctx + part - 1) / part : 1;
  if (max_parts > 0x7fffffff) return mie::fail(MIE_ERR_INVALID, "mie_paged_decode: too many partitions");
  *part_out = static_cast<int32_t>(part);
  *max_parts_out = static_cast<int32_t>(max_parts);
  *ws_out = max_parts > 1 ? static_cast<int64_t>(batch) * num_heads * max_parts * (head_dim + 2) * 4 : 0;
  return MIE_OK;
}

template <int DT, int D>
int32_t launch(DecodeArgs& a, int batch, hipStream_t st) {
  const dim3 grid(a.max_parts, (a.H + kWaves - 1) / kWaves, batch);
  paged_decode_kernel<DT, D><<<grid, 64 * kWaves, 0, st>>>(a);
  int32_t rc = mie::check_launch("paged_decode_kernel");
  if (rc != MIE_OK || a.max_parts <= 1) return rc;
  paged_decode_reduce_kernel<DT, D><<<dim3(a.H, batch), 256, 0, st>>>(a);
  return mie::check_launch("paged_decode_reduce_kernel");
}

int32_t dispatch(int dtype, int head_dim, DecodeArgs& a, int batch, hipStream_t st) {
#define MIE_LAUNCH_CASE(DD)                                                          \
  case DD:                                                                           \
    return dtype == MIE_DTYPE_F32 ? launch<MIE_DTYPE_F32, DD>(a, batch, st)          \
                                  : launch<MIE_DTYPE_BF16, DD>(a, batch, st);
  switch (head_dim) {
    MIE_FOR_EACH_HEAD_DIM(MIE_LAUNCH_CASE)
    default: return mie::fail(MIE_ERR_UNSUPPORTED, "mie_paged_decode: head_dim %d not built", head_dim);
  }
#undef MIE_LAUNCH_CASE
}

bool aligned(const void* p, int n) { return reinterpret_cast<uintptr_t>(p) % n == 0; }

}  // namespace

extern "C" int32_t mie_paged_decode_supported(int32_t head_dim, int32_t dtype) {
  return tile_for(dtype, head_dim) != 0 ? 1 : 0;
}

extern "C" int32_t mie_paged_decode_plan(int32_t batch, int32_t num_heads, int32_t head_dim,
                                         int32_t max_ctx_len, int32_t dtype, int32_t partition_tokens,
                                         int32_t* partition_tokens_out, int64_t* workspace_bytes_out) {
  int32_t part = 0, max_parts = 0;
  int64_t ws = 0;
  const int32_t rc = plan(batch, num_heads, head_dim, max_ctx_len, dtype, partition_tokens, &part, &ws,
                          &max_parts);
  if (rc != MIE_OK) return rc;
  if (partition_tokens_out) *partition_tokens_out = part;
  if (workspace_bytes_out) *workspace_bytes_out = ws;
  return MIE_OK;
}

extern "C" int32_t mie_paged_decode(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                    const void* k_pool, const void* v_pool, int64_t pool_stride_block,
                                    int64_t pool_stride_head, int32_t num_blocks,
                                    const int32_t* block_tables, int64_t block_table_stride,
                                    const int32_t* ctx_lens, int32_t ctx_len, int32_t max_ctx_len,
                                    int32_t batch, int32_t num_heads, int32_t head_dim,
                                    int32_t block_size, float scale, void* out, int64_t out_stride_b,
                                    int64_t out_stride_h, int32_t out_dtype, void* workspace,
                                    int64_t workspace_bytes, int32_t partition_tokens, int32_t dtype,
                                    void* stream) {
  int32_t part = 0, max_parts = 0;
  int64_t ws = 0;
  int32_t rc = plan(batch, num_heads, head_dim, max_ctx_len, dtype, partition_tokens, &part, &ws,
                    &max_parts);
  if (rc != MIE_OK) return rc;
  if (batch == 0) return MIE_OK;
  if (block_size <= 0 || num_blocks <= 0)
    return mie::fail(MIE_ERR_INVALID, "mie_paged_decode: block_size=%d num_blocks=%d", block_size,
                     num_blocks);
  if (!ctx_lens && (ctx_len < 0 || ctx_len > max_ctx_len))
    return mie::fail(MIE_ERR_INVALID, "mie_paged_decode: ctx_len %d outside [0, max_ctx_len=%d]", ctx_len,
                     max_ctx_len);
  if (batch > 65535 || num_heads > 65535 * kWaves)
    return mie::fail(MIE_ERR_INVALID, "mie_paged_decode: batch or heads too large");
  if (out_dtype != MIE_DTYPE_F32 && out_dtype != dtype)
    return mie::fail(MIE_ERR_UNSUPPORTED, "mie_paged_decode: out_dtype %d must be f32 or the input dtype",
                     out_dtype);
  if (!q || !k_pool || !v_pool || !block_tables || !out)
    return mie::fail(MIE_ERR_INVALID, "mie_paged_decode: null pointer");
  if (pool_stride_head < static_cast<int64_t>(block_size) * head_dim ||
      pool_stride_block < static_cast<int64_t>(num_heads) * pool_stride_head)
    return mie::fail(MIE_ERR_INVALID, "mie_paged_decode: pool strides overlap");
  if (ws > 0 && (!workspace || workspace_bytes < ws || !aligned(workspace, 16)))
    return mie::fail(MIE_ERR_WORKSPACE, "mie_paged_decode: needs a 16-byte aligned workspace of %lld bytes",
                     static_cast<long long>(ws));

  // Every vector access must be naturally aligned: lane loads are 8 or 16
  // bytes, outputs are written VEC elements at a time.
  const int elt = mie::elt_size(dtype);
  const int vec = dtype == MIE_DTYPE_F32 ? 4 : (head_dim < 8 ? head_dim : 8);
  const int vb = vec * elt;
  const int ob = vec * mie::elt_size(out_dtype);
  const bool ok_align = aligned(q, vb) && aligned(k_pool, vb) && aligned(v_pool, vb) &&
                        (q_stride_b * elt) % vb == 0 && (q_stride_h * elt) % vb == 0 &&
                        (pool_stride_block * elt) % vb == 0 && (pool_stride_head * elt) % vb == 0 &&
                        aligned(out, ob) && (out_stride_b * mie::elt_size(out_dtype)) % ob == 0 &&
                        (out_stride_h * mie::elt_size(out_dtype)) % ob == 0;
  if (!ok_align) return mie::fail(MIE_ERR_INVALID, "mie_paged_decode: misaligned q / pool / out");

  DecodeArgs a;
  a.q = static_cast<const char*>(q);
  a.q_sb = q_stride_b;
  a.q_sh = q_stride_h;
  a.k = static_cast<const char*>(k_pool);
  a.v = static_cast<const char*>(v_pool);
  a.kv_sblk = pool_stride_block;
  a.kv_sh = pool_stride_head;
  a.num_blocks = num_blocks;
  a.bt = block_tables;
  a.bt_stride = block_table_stride;
  a.bt_cap = static_cast<uint32_t>(block_table_stride > 0 ? block_table_stride : num_blocks);
  a.ctx_lens = ctx_lens;
  a.ctx_len = ctx_len;
  a.max_ctx = max_ctx_len;
  a.H = num_heads;
  a.bs = mie::FastDiv::make(static_cast<uint32_t>(block_size));
  a.qk_scale = scale * kLog2e;
  a.out = static_cast<char*>(out);
  a.o_sb = out_stride_b;
  a.o_sh = out_stride_h;
  a.out_f32 = out_dtype == MIE_DTYPE_F32 && dtype != MIE_DTYPE_F32 ? 1 : 0;
  a.max_parts = max_parts;
  a.part_shift = ilog2(static_cast<uint32_t>(part));
  if (max_parts > 1) {
    a.ws_acc = static_cast<float*>(workspace);
    a.ws_ml = a.ws_acc + static_cast<int64_t>(batch) * num_heads * max_parts * head_dim;
  } else {
    a.ws_acc = nullptr;
    a.ws_ml = nullptr;
  }
  return dispatch(dtype, head_dim, a, batch, static_cast<hipStream_t>(stream));
}
