// Direct paged decode attention for gfx950 (MI355X).
//
// Replaces the reference's Triton _paged_decode_kernel
// (src/moe_engine/paged_attention.py:46-110): per (sequence, head)
//   out = softmax(scale * q . K^T) . V   over tokens [0, ctx) of a paged pool.
//
// Work decomposition.  One 64-lane wavefront owns one (sequence, head,
// partition) work item; a workgroup holds WAVES heads of the same sequence and
// partition, so its waves walk the same block-table entries and neighbouring
// (block, head) tiles.  For batches up to kFlatMaxBatch the workgroups form a
// flat list of exactly the batch's work items (each maps its index with a
// prefix scan over the sequence lengths on the device), sized exactly when the
// caller passes a host copy of the lengths - a grid padded to the longest
// sequence spends ~18 % of a ragged batch's time on workgroups that only exit.
// Larger batches use grid = (partitions, ceil(H / WAVES), batch).  Partitions
// are short (a few hundred tokens) so the hardware dispatcher keeps refilling
// CUs with fresh work items and the kernel ends without a long tail.
//
// Lane layout.  A token's head_dim row is split into NV slices of VEC elements
// (VB = 16 bytes for f32 and bf16), held by LPT = next_pow2(NV) consecutive
// lanes; one wave load reads TPL = 64 / LPT whole token rows, and for
// block_size a multiple of TPL those rows are one contiguous run of the
// (block, head) tile: a fully coalesced 1 KiB access.  A tile is ROWS such
// loads of K and of V.  Tiles are software pipelined: the loads of tile i+1 are
// issued before tile i is consumed.  K/V loads carry the non-temporal hint
// (each byte is read once; measured ~15 % faster on config 4 than plain loads).
//
// Block ids.  When the block size is a power of two that is a multiple of TPL
// and a partition spans at most 64 blocks (the FAST path, the common case), the
// partition's block ids are read once, one per lane, and each row's id is a
// readlane (a scalar) - no table load on the per-tile critical path.  Other
// shapes read the table per row with a fast division by the block size.
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
// merges the partials of each (sequence, head) in one pass; a sequence that
// fits one partition is normalised and written by the first kernel.
#include <math.h>

#include <algorithm>
#include <mutex>

#include "mie_common.h"

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kWaves = 4;            // heads (wavefronts) per workgroup
constexpr int kWindow = 64;          // FAST path: block ids held one per lane
// Automatic partition size: the smallest power of two (>= the tile) that keeps
// B * H * ceil(max_ctx / P) at or below kTargetItems wavefronts AND every
// sequence at or below kMaxParts partitions, capped at the FAST window.  The
// first bound is where a partition sweep on MI355X (P = 64 .. 2048 tokens,
// 12 heads x 64, bf16 and fp32) was fastest in every long-context shape:
// about 3072 wavefronts, 12 per CU - 1 x 32768 at P = 128, 1 x 131072 at
// 512, 8 x 32768 at 1024 (123 us against 133 us at 12288 wavefronts).  The
// second bounds the merge work per (sequence, head).
constexpr int kTargetItems = 3072;  // auto plan: wavefronts to stay below
constexpr int kMaxParts = 256;       // auto plan: partitions per sequence to stay below
// Merge of split contexts: float4 columns of a head per reduce workgroup (8:
// two workgroups per head at head_dim 64), so each thread holds the partials
// of at most 8 partitions in registers per 256 partitions.
constexpr int RW_COLS = 8;
// Occupancy floor for the main kernels: every built shape fits 4 waves/SIMD
// (<= 128 VGPRs) without spills; at 3 waves/SIMD config 4 runs ~8 % slower.
constexpr int kMinWaves = 4;
// Batches up to this size use the flat work list (its per-workgroup scan reads
// ceil(B / 64) chunks of lengths); larger batches use the grid form.
constexpr int kFlatMaxBatch = 512;
// Workgroup form: one workgroup of kSplitWaves waves per (sequence, head).
// Each wave reads its slice as a serial chain of tiles (~2 us per tile when
// latency-bound), so the automatic plan takes this form for at most
// kWgMaxRows (sequence, head) rows when every slice is short (max_ctx <=
// kWgShortCtx: at most 64 tokens per wave) or when there are enough rows to
// fill the GPU with workgroups (rows >= kWgMinRows, max_ctx <= kWgMaxCtx).
// Measured on MI355X (per call, graph replays), workgroup form vs the
// partition plan: 1 x 96 tokens 3.9 vs 6.8 us, 1 x 512 5.4 vs 7.0, 21 x 1000
// 13.6 vs 16.3, 16 x 4096 33.5 vs 35.3, 64 x 2048 68.7 vs 73.3, 64 x 4096
// 124.5 vs 130.7, 16 x 8192 62.3 vs 72.3, config 4 (64 x U[512, 8192])
// 127.4 vs 130.9; but 1 x 2048 10.6 vs 7.3, 4 x 4096 25 vs 14 and 128 x 512
// (1536 rows, one workgroup per CU at a time) 45.7 vs 42.3.  Below kWgMinRows
// rows a long context would leave CUs idle.
constexpr int kSplitWaves = 16;
// Workgroup form: half the partition kernels' tile (16 tokens for bf16 and
// f32 at head_dim 64): 69 instead of 103 VGPRs (7 instead of 4 waves per
// SIMD) for the same bytes in flight per CU.  Config 4 on MI355X: 119.8 us
// against 121.7-124.7 us with the partition tile, 121.8 us at a quarter of it
// (graph-replayed decode launches).
constexpr int kWgTileWords = 8;
constexpr int kWgOrderMax = 1024;  // batches the workgroup form can dispatch longest first
constexpr int kWgShortCtx = 1024;
constexpr int kWgMinRows = 128;
constexpr int kWgMaxRows = 1024;
constexpr int kWgMaxCtx = 8192;

constexpr int next_pow2(int x) {
  int p = 1;
  while (p < x) p <<= 1;
  return p;
}

template <int DT> struct Elt;
template <> struct Elt<MIE_DTYPE_F32> { static constexpr int size = 4; };
template <> struct Elt<MIE_DTYPE_BF16> { static constexpr int size = 2; };

// KW: 32-bit words of K each lane holds per tile (the tile's rows are
// KW / NW wave loads).  The partition kernels use 16 (64 B of K, 64 B of V per
// lane per tile, two tiles in flight); the workgroup form uses kWgTileWords.
template <int DT, int D, int KW = 16>
struct Geometry {
  static constexpr int ELT = Elt<DT>::size;
  static constexpr int VEC = (16 / ELT) < D ? (16 / ELT) : D;  // elements per lane load
  static constexpr int VB = VEC * ELT;                          // bytes per lane load
  static constexpr int NW = VB / 4;                             // 32-bit words per lane load
  static constexpr int NV = D / VEC;                            // lanes with data per token
  static constexpr int LPT = next_pow2(NV);                     // lanes per token
  static constexpr int TPL = 64 / LPT;                          // tokens per wave load
  static constexpr int ROWS_BY_REGS = KW / NW > 0 ? KW / NW : 1;  // <= 4 * KW bytes of K per lane per tile
  static constexpr int ROWS_BY_TILE = (64 / TPL) > 0 ? 64 / TPL : 1;
  static constexpr int ROWS = ROWS_BY_REGS < ROWS_BY_TILE ? ROWS_BY_REGS : ROWS_BY_TILE;
  static constexpr int TILE = ROWS * TPL;  // tokens per tile (a power of two)
  static_assert(D % VEC == 0, "head_dim must be a multiple of the lane vector");
  static_assert(VB == 8 || VB == 16, "lane loads are 8 or 16 bytes");
  static_assert(LPT <= 64, "head_dim too large for one wavefront");
};

template <int NW> struct Words { uint32_t w[NW]; };

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

template <int NW>
__device__ __forceinline__ Words<NW> load_words(const char* p) {
  Words<NW> r;
  if constexpr (NW == 4) {
    const u32x4_t x = *reinterpret_cast<const u32x4_t*>(p);
    r.w[0] = x.x; r.w[1] = x.y; r.w[2] = x.z; r.w[3] = x.w;
  } else {
    const u32x2_t x = *reinterpret_cast<const u32x2_t*>(p);
    r.w[0] = x.x; r.w[1] = x.y;
  }
  return r;
}

// Streaming load of data read exactly once (global_load ... nt).
template <int NW>
__device__ __forceinline__ Words<NW> load_words_nt(const char* p) {
  Words<NW> r;
  if constexpr (NW == 4) {
    const u32x4_t x = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
    r.w[0] = x.x; r.w[1] = x.y; r.w[2] = x.z; r.w[3] = x.w;
  } else {
    const u32x2_t x = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(p));
    r.w[0] = x.x; r.w[1] = x.y;
  }
  return r;
}

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
  // Fused append (workgroup form): the new token's K/V rows [B, H, D]; NULL
  // for a plain decode.  The token is the sequence's last (position ctx - 1).
  const char* k_new;
  const char* v_new;
  int64_t new_sb, new_sh;  // elements
  // Workgroup form with FAST block ids: > 0 when every block a sequence can
  // use (ceil(max_ctx / block_size) <= kWindow) fits one window.  Each wave
  // then reads table entries [0, win_blocks) at its start, alongside the
  // context length, instead of after it.
  int32_t win_blocks;
};

__device__ __forceinline__ int seq_ctx(const DecodeArgs& a, int b) {
  int c = a.ctx_lens ? a.ctx_lens[b] : a.ctx_len;
  c = c < 0 ? 0 : c;
  return c < a.max_ctx ? c : a.max_ctx;
}

// Writes N consecutive outputs at element offset `elem_off` of `base`, in f32
// or in the kernel's dtype (N a multiple of 4).
template <int DT, int N>
__device__ __forceinline__ void store_out(char* base, int64_t elem_off, const float* val, bool f32) {
  if (f32 || DT == MIE_DTYPE_F32) {
    float* p = reinterpret_cast<float*>(base) + elem_off;
#pragma unroll
    for (int i = 0; i < N; i += 4)
      *reinterpret_cast<float4*>(p + i) = make_float4(val[i], val[i + 1], val[i + 2], val[i + 3]);
  } else {
    uint32_t* p = reinterpret_cast<uint32_t*>(reinterpret_cast<uint16_t*>(base) + elem_off);
#pragma unroll
    for (int i = 0; i < N; i += 4)
      *reinterpret_cast<uint2*>(p + i / 2) =
          make_uint2(mie::pack_bf16x2(val[i], val[i + 1]), mie::pack_bf16x2(val[i + 2], val[i + 3]));
  }
}

// Online softmax of sequence b, head h over tokens [t_begin, t_end) (t_begin
// a multiple of the tile; for FAST the range spans at most kWindow blocks),
// computed by one full wavefront.  Returns the range's state merged over the
// wave: m (running max, log2 units) and l are uniform across lanes; acc holds
// the head_dim slice jl = lane % LPT; bad is wave-uniform and set when a block
// id outside the pool was met.
//
// YIELD: the wave lowers its issue priority (s_setprio 3, 2, 1, 0) as it
// passes each quarter of its tiles, and ends at 0.  The workgroup form splits
// one sequence among 16 waves with equal slices, and the SIMD's arbiter
// favours the oldest ready wave: on MI355X (config 4) waves 0-3 finished at
// 0.68 of the workgroup's time, waves 12-14 at 0.97.  A wave that gets ahead
// now yields to the waves behind it (spread 0.31 -> 0.12).  Only the timing
// changes: every wave reads the same tokens and the result is bit-identical.
template <int DT, int D, bool FAST, int KW = 16, bool YIELD = false>
__device__ __forceinline__ void attend_range(const DecodeArgs& a, int b, int h, int t_begin, int t_end, int lane,
                                             float& m, float& l, float* acc, bool& bad, int32_t win_ids = -1) {
  using G = Geometry<DT, D, KW>;
  constexpr int ELT = G::ELT, VEC = G::VEC, NW = G::NW, LPT = G::LPT, TPL = G::TPL;
  constexpr int ROWS = G::ROWS, TILE = G::TILE;
  constexpr int64_t ROW_BYTES = static_cast<int64_t>(D) * ELT;

  const int g = lane / LPT;   // token group within a wave load
  const int jl = lane % LPT;  // slice of the head_dim row
  const bool jv = jl < G::NV;

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
  // A lane without head_dim data (jl >= NV) reads its row's first vector.
  const int64_t lane_off = (h * a.kv_sh + (jv ? jl : 0) * VEC) * ELT;
  const char* kbase = a.k + lane_off;
  const char* vbase = a.v + lane_off;
  const int64_t blk_bytes = a.kv_sblk * ELT;

  bad = false;
  int fb = 0;
  int32_t ids = 0;
  if constexpr (FAST) {  // the partition's block ids, one per lane
    const int first = t_begin >> a.bs.shift;
    const int last = (t_end - 1) >> a.bs.shift;
    if (a.win_blocks > 0) {  // entries [0, win_blocks), read by the caller
      ids = win_ids;
      bad = __any(lane >= first && lane <= last && (ids < 0 || ids >= a.num_blocks));
    } else {
      fb = first;
      const uint32_t idx = static_cast<uint32_t>(fb + lane);
      const bool mine = lane <= last - fb;  // <= kWindow blocks by the plan
      ids = (mine && idx < a.bt_cap) ? bt[idx] : -1;
      bad = __any(mine && (ids < 0 || ids >= a.num_blocks));
    }
  }

  // Every load is unconditional, so that a tile's loads go out together and
  // the wait before consuming the previous tile counts exactly the loads in
  // flight: a load under a branch makes the compiler assume the other path and
  // wait for everything.  Rows past the range re-read the range's last row,
  // and a table entry outside the pool reads block 0 (its sequence is already
  // marked bad); consume() masks both.
  const int last_row = (t_end - 1) & ~(TPL - 1);
  auto issue = [&](int t0, Words<NW>* kr, Words<NW>* vr) {
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
      int64_t off;
      if constexpr (FAST) {
        const int tr = min(t0 + r * TPL, last_row);  // first token of the row (wave-uniform)
        int phys = __builtin_amdgcn_readlane(ids, (tr >> a.bs.shift) - fb);
        phys = static_cast<uint32_t>(phys) < static_cast<uint32_t>(a.num_blocks) ? phys : 0;
        off = phys * blk_bytes + static_cast<int64_t>((tr & (a.bs.d - 1)) + g) * ROW_BYTES;
      } else {
        const int t_raw = t0 + r * TPL + g;
        const int t = min(t_raw, t_end - 1);
        const uint32_t blk = a.bs.div(static_cast<uint32_t>(t));
        const uint32_t slot = static_cast<uint32_t>(t) - blk * a.bs.d;
        const int32_t entry = bt[min(blk, a.bt_cap - 1)];
        const bool ok = blk < a.bt_cap && entry >= 0 && entry < a.num_blocks;
        bad = bad || (!ok && t_raw < t_end);
        off = (ok ? entry : 0) * blk_bytes + static_cast<int64_t>(slot) * ROW_BYTES;
      }
      kr[r] = load_words_nt<NW>(kbase + off);
      vr[r] = load_words_nt<NW>(vbase + off);
    }
  };

  m = -INFINITY;
  l = 0.f;
#pragma unroll
  for (int i = 0; i < VEC; ++i) acc[i] = 0.f;

  auto consume = [&](int t0, const Words<NW>* kr_in, const Words<NW>* vr_in) {
    // Rows past the range and lanes without head_dim data hold stand-in
    // values: zero them so that no Inf or NaN stored there reaches the sums.
    Words<NW> kr[ROWS], vr[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
      const bool live = t0 + r * TPL + g < t_end;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        kr[r].w[w] = (G::NV < LPT && !jv) ? 0u : kr_in[r].w[w];
        vr[r].w[w] = live ? vr_in[r].w[w] : 0u;
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
                                                     __builtin_bit_cast(bf16x2_t, qw.w[w]), part_dot, false);
        s[r] = mie::group_sum<LPT>(part_dot) * a.qk_scale;
      } else {
#pragma unroll
        for (int i = 0; i < VEC; ++i) part_dot = fmaf(__uint_as_float(kr[r].w[i]), qf[i], part_dot);
        s[r] = mie::group_sum<LPT>(part_dot);
      }
      s[r] = t0 + r * TPL + g < t_end ? s[r] : -INFINITY;
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
  };

  // Two register sets: tile i+1 is in flight while tile i is consumed.  The
  // steady state issues unconditionally; the last one or two tiles are peeled,
  // so no tile past the range is read.
  Words<NW> kA[ROWS], vA[ROWS], kB[ROWS], vB[ROWS];
  const int ntiles = (t_end - t_begin + TILE - 1) / TILE;  // >= 1
  [[maybe_unused]] const int q1 = ntiles / 4, q2 = ntiles / 2, q3 = (3 * ntiles) / 4;
  if constexpr (YIELD) __builtin_amdgcn_s_setprio(3);
  issue(t_begin, kA, vA);
  int t0 = t_begin;
  for (int i = 0; i + 2 < ntiles; i += 2, t0 += 2 * TILE) {
    if constexpr (YIELD) {
      if (i >= q3) __builtin_amdgcn_s_setprio(0);
      else if (i >= q2) __builtin_amdgcn_s_setprio(1);
      else if (i >= q1) __builtin_amdgcn_s_setprio(2);
    }
    issue(t0 + TILE, kB, vB);
    consume(t0, kA, vA);
    issue(t0 + 2 * TILE, kA, vA);
    consume(t0 + TILE, kB, vB);
  }
  if (t0 + TILE < t_end) {
    issue(t0 + TILE, kB, vB);
    consume(t0, kA, vA);
    consume(t0 + TILE, kB, vB);
  } else {
    consume(t0, kA, vA);
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
  if constexpr (!FAST) bad = __any(bad);
  if constexpr (YIELD) __builtin_amdgcn_s_setprio(0);
}

// One work item: sequence b (ctx tokens, ctx > 0), head h, partition `part`,
// computed by one full wavefront.
template <int DT, int D, bool FAST>
__device__ __forceinline__ void decode_item(const DecodeArgs& a, int b, int h, int part, int ctx, int lane) {
  using G = Geometry<DT, D>;
  constexpr int VEC = G::VEC;
  const int nparts = (ctx + (1 << a.part_shift) - 1) >> a.part_shift;
  const int t_begin = part << a.part_shift;
  const int t_end = min(ctx, t_begin + (1 << a.part_shift));
  float m, l, acc[VEC];
  bool bad;
  attend_range<DT, D, FAST>(a, b, h, t_begin, t_end, lane, m, l, acc, bad);

  const int g = lane / G::LPT;
  const int jl = lane % G::LPT;
  if (g != 0 || jl >= G::NV) return;
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
    for (int i = 0; i < VEC; i += 4)
      *reinterpret_cast<float4*>(dst + i) = make_float4(acc[i], acc[i + 1], acc[i + 2], acc[i + 3]);
    if (jl == 0) {
      a.ws_ml[2 * item] = bad ? NAN : m;
      a.ws_ml[2 * item + 1] = l;
    }
  }
}

// Writes zeros for a sequence with no keys (what scaled_dot_product_attention
// returns for an empty key set).
template <int DT, int D>
__device__ __forceinline__ void zero_item(const DecodeArgs& a, int b, int h, int lane) {
  using G = Geometry<DT, D>;
  const int jl = lane % G::LPT;
  if (lane / G::LPT != 0 || jl >= G::NV) return;
  float zero[G::VEC];
#pragma unroll
  for (int i = 0; i < G::VEC; ++i) zero[i] = 0.f;
  store_out<DT, G::VEC>(a.out, b * a.o_sb + h * a.o_sh + jl * G::VEC, zero, a.out_f32);
}

// Grid form: grid = (max partitions, ceil(H / WAVES), batch); workgroups past
// a sequence's last partition exit.  Used for batches above kFlatMaxBatch.
template <int DT, int D, bool FAST>
__global__ __launch_bounds__(64 * kWaves) __attribute__((amdgpu_waves_per_eu(kMinWaves, 8)))
void paged_decode_grid_kernel(DecodeArgs a) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int h = blockIdx.y * kWaves + wave;
  if (h >= a.H) return;
  const int b = blockIdx.z;
  const int part = blockIdx.x;
  const int ctx = seq_ctx(a, b);
  if (ctx == 0) {
    if (part == 0) zero_item<DT, D>(a, b, h, lane);
    return;
  }
  if (part >= (ctx + (1 << a.part_shift) - 1) >> a.part_shift) return;
  decode_item<DT, D, FAST>(a, b, h, part, ctx, lane);
}

// Flat form: blockIdx.x enumerates the batch's real work items, sequence by
// sequence, head group by head group, partition fastest; a sequence with
// ctx == 0 has one item per head group (it writes zeros).  Each wave maps its
// item with a 64-lane inclusive prefix scan of the per-sequence item counts,
// 64 sequences per step, so no workgroup exists for a partition past a
// sequence's end.  When the launch is an upper bound rather than the exact
// count, the surplus workgroups find no item and exit.
template <int DT, int D, bool FAST>
__global__ __launch_bounds__(64 * kWaves) __attribute__((amdgpu_waves_per_eu(kMinWaves, 8)))
void paged_decode_flat_kernel(DecodeArgs a, int batch, int head_groups) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int item = blockIdx.x;
  const int shift = a.part_shift;
  int base = 0;  // items of the sequences before this chunk
  int b = -1, part = 0, hg = 0, seq_ctx_len = 0;
  for (int c0 = 0; c0 < batch; c0 += 64) {
    const int bb = c0 + lane;
    const int ctx = bb < batch ? seq_ctx(a, bb) : 0;
    const int parts = max(1, (ctx + (1 << shift) - 1) >> shift);
    const int n = bb < batch ? parts * head_groups : 0;
    int incl = n;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int y = __shfl_up(incl, off);
      if (lane >= off) incl += y;
    }
    const int chunk_items = __shfl(incl, 63);
    if (item < base + chunk_items) {
      // The item's coordinates are wave-uniform; readfirstlane tells the
      // compiler so, keeping them (and every token index and block address
      // derived from them) in scalar registers.
      const int owner = __ffsll(static_cast<unsigned long long>(__ballot(incl > item - base))) - 1;
      const int local =
          __builtin_amdgcn_readfirstlane(item - base - (__shfl(incl, owner) - __shfl(n, owner)));
      const int seq_parts = __builtin_amdgcn_readfirstlane(__shfl(parts, owner));
      hg = local / seq_parts;
      part = local - hg * seq_parts;
      b = c0 + owner;
      seq_ctx_len = __builtin_amdgcn_readfirstlane(__shfl(ctx, owner));
      break;
    }
    base += chunk_items;
  }
  // The scan's registers are dead from here on.
  const int h = hg * kWaves + wave;
  if (b < 0 || h >= a.H) return;
  if (seq_ctx_len == 0) {
    zero_item<DT, D>(a, b, h, lane);
    return;
  }
  decode_item<DT, D, FAST>(a, b, h, part, seq_ctx_len, lane);
}

// Workgroup form: grid = (H, batch), one workgroup of kSplitWaves waves per
// (sequence, head).  Wave w takes the w-th tile-aligned slice of the context,
// so a short context is read by 16 waves at once instead of one; the waves'
// (max, sum, acc) states are merged through LDS and the workgroup writes the
// output: one launch, no workspace.
//
// A workgroup's time grows with its sequence's length and a CU holds one such
// workgroup at a time, so the order of dispatch sets the tail of a ragged
// batch.  When the caller gives host lengths, row y of the grid takes
// order.seq[y]: the sequences longest first (ties by index), which the
// hardware dispatches first - config 4 runs ~2 % faster, a ragged 48 x
// U[64, 8192] ~15 %.  Ranking on the device instead delays every workgroup's
// start by a global load and two barriers, ~5 % on uniform batches.
struct WgOrder {
  int32_t n;  // 0: grid order
  uint16_t seq[kWgOrderMax];
};

template <int DT, int D, bool FAST>
__global__ __launch_bounds__(64 * kSplitWaves) __attribute__((amdgpu_waves_per_eu(kMinWaves, 8)))
void paged_decode_wg_kernel(DecodeArgs a, WgOrder order) {
  using G = Geometry<DT, D, kWgTileWords>;
  constexpr int VEC = G::VEC, NW = G::NW, LPT = G::LPT, ELT = G::ELT;
  constexpr int kStates = kSplitWaves + 1;  // the waves' slices, then a fused append's new token
  __shared__ float s_m[kStates], s_l[kStates];
  __shared__ float s_acc[kStates][D];
  __shared__ int s_bad;
  // At least 72 VGPRs, so at most 7 waves per SIMD (28 per CU): one 16-wave
  // workgroup runs per CU at a time.  At 8 waves per SIMD (the f32 shapes
  // compile to <= 64 VGPRs) two whole workgroups share a CU, twice the random
  // read streams per CU; on MI355X that measured 2.5 % slower at config 4's
  // shape in f32, and 30 % slower for a 64-VGPR bf16 build.  Emits no code.
  asm volatile("" ::: "v71");
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int h = blockIdx.x;
  const int b = order.n > 0 ? order.seq[blockIdx.y] : blockIdx.y;
  int32_t win_ids = -1;
  if constexpr (FAST) {
    if (lane < a.win_blocks && static_cast<uint32_t>(lane) < a.bt_cap) win_ids = a.bt[b * a.bt_stride + lane];
  }
  const int ctx = seq_ctx(a, b);
  // With a fused append the new token (the last, ctx - 1) comes from the
  // caller's rows, not the pool: the waves read tokens [0, ctx - 1), the last
  // wave - whose slice is the shortest - stores the rows into the pool and
  // supplies the token's (max, sum, acc) state from registers.
  const bool append = a.k_new != nullptr && ctx > 0;
  const int pool_ctx = append ? ctx - 1 : ctx;
  const int per_wave = (pool_ctx + kSplitWaves - 1) / kSplitWaves;
  const int chunk = (per_wave + G::TILE - 1) / G::TILE * G::TILE;
  const int t_begin = min(pool_ctx, wave * chunk);
  const int t_end = min(pool_ctx, t_begin + chunk);
  if (threadIdx.x == 0) s_bad = 0;
  float m = -INFINITY, l = 0.f, acc[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) acc[i] = 0.f;
  bool bad = false;
  if (t_begin < t_end)
    attend_range<DT, D, FAST, kWgTileWords, true>(a, b, h, t_begin, t_end, lane, m, l, acc, bad, win_ids);
  __syncthreads();  // s_bad is cleared
  const int g = lane / LPT;
  const int jl = lane % LPT;
  const bool jv = jl < G::NV;
  if (lane == 0) {
    s_m[wave] = m;
    s_l[wave] = l;
    if (bad) s_bad = 1;
  }
  if (g == 0 && jv) {
#pragma unroll
    for (int i = 0; i < VEC; ++i) s_acc[wave][jl * VEC + i] = acc[i];
  }
  if (append && wave == kSplitWaves - 1) {
    const int64_t row = (b * a.new_sb + h * a.new_sh + jl * VEC) * ELT;
    Words<NW> kw, vw, qw;
#pragma unroll
    for (int w = 0; w < NW; ++w) kw.w[w] = vw.w[w] = qw.w[w] = 0u;
    if (jv) {
      kw = load_words<NW>(a.k_new + row);
      vw = load_words<NW>(a.v_new + row);
      qw = load_words<NW>(a.q + (b * a.q_sb + h * a.q_sh + jl * VEC) * ELT);
    }
    // Store the rows at position ctx - 1 (bounds-checked like the append kernel).
    const uint32_t p = static_cast<uint32_t>(ctx - 1);
    const uint32_t lb = a.bs.div(p);
    const int32_t phys = lb < a.bt_cap ? a.bt[b * a.bt_stride + lb] : -1;
    const bool ok = phys >= 0 && phys < a.num_blocks;
    if (ok && g == 0 && jv) {
      const int64_t off = (phys * a.kv_sblk + h * a.kv_sh + static_cast<int64_t>(p - lb * a.bs.d) * D + jl * VEC) * ELT;
      if constexpr (NW == 4) {
        *reinterpret_cast<u32x4_t*>(const_cast<char*>(a.k) + off) = u32x4_t{kw.w[0], kw.w[1], kw.w[2], kw.w[3]};
        *reinterpret_cast<u32x4_t*>(const_cast<char*>(a.v) + off) = u32x4_t{vw.w[0], vw.w[1], vw.w[2], vw.w[3]};
      } else {
        *reinterpret_cast<u32x2_t*>(const_cast<char*>(a.k) + off) = u32x2_t{kw.w[0], kw.w[1]};
        *reinterpret_cast<u32x2_t*>(const_cast<char*>(a.v) + off) = u32x2_t{vw.w[0], vw.w[1]};
      }
    }
    // The token's score, computed as the pool path computes one (consume()).
    float dot = 0.f;
    if constexpr (DT == MIE_DTYPE_BF16) {
#pragma unroll
      for (int w = 0; w < NW; ++w)
        dot = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, kw.w[w]), __builtin_bit_cast(bf16x2_t, qw.w[w]),
                                              dot, false);
      dot = mie::group_sum<LPT>(dot) * a.qk_scale;
    } else {
#pragma unroll
      for (int i = 0; i < VEC; ++i) dot = fmaf(__uint_as_float(kw.w[i]), __uint_as_float(qw.w[i]) * a.qk_scale, dot);
      dot = mie::group_sum<LPT>(dot);
    }
    if (lane == 0) {
      s_m[kSplitWaves] = dot;
      s_l[kSplitWaves] = 1.f;
      if (!ok) s_bad = 1;
    }
    if (g == 0 && jv) {
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        if constexpr (DT == MIE_DTYPE_BF16) {
          s_acc[kSplitWaves][jl * VEC + 2 * w] = mie::bf16_lo(vw.w[w]);
          s_acc[kSplitWaves][jl * VEC + 2 * w + 1] = mie::bf16_hi(vw.w[w]);
        } else {
          s_acc[kSplitWaves][jl * VEC + w] = __uint_as_float(vw.w[w]);
        }
      }
    }
  }
  __syncthreads();
  // Threads 0 .. D/4-1 merge four output elements each.
  const int col = threadIdx.x * 4;
  if (col >= D) return;
  const int states = append ? kStates : kSplitWaves;
  float mx = -INFINITY;
  for (int w = 0; w < states; ++w) mx = fmaxf(mx, s_m[w]);
  const float mr = mx == -INFINITY ? 0.f : mx;
  float lt = 0.f;
  float o[4] = {0.f, 0.f, 0.f, 0.f};
  for (int w = 0; w < states; ++w) {
    const float wt = mie::fast_exp2(s_m[w] - mr);
    lt += s_l[w] * wt;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] += s_acc[w][col + i] * wt;
  }
  // No keys: zeros, as scaled_dot_product_attention returns for an empty set.
  const float inv = ctx == 0 ? 0.f : (s_bad ? NAN : 1.f / lt);
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] *= inv;
  store_out<DT, 4>(a.out, b * a.o_sb + h * a.o_sh + col, o, a.out_f32);
}

// Merge the partition partials of one (sequence, head) in one pass:
//   M = max_i m_i,  w_i = 2^(m_i - M),  out = sum_i w_i acc_i / sum_i w_i l_i.
// 256 threads = COLS column threads (4 elements each) x PL partition lanes.
// Each thread folds its partitions (i = pl, pl + PL, ...) into a running
// (m, l, acc) with the same rescaling as the main kernel, so all partial loads
// are independent; the PL states of a column are then merged through LDS.
template <int DT, int D>
__global__ __launch_bounds__(256) void paged_decode_reduce_kernel(DecodeArgs a) {
  // One workgroup per (sequence, head, chunk of RW_COLS float4 columns).
  // Every thread first issues all of its loads - its partition's (m, l) and
  // the acc columns of RW_NPT partitions - in one memory round, before the
  // sequence's length is known (a device length is one more load, issued
  // beside them), and only then joins the workgroup-wide max: the merge
  // waits on one round trip, not on a chain of them.  Partitions past the
  // sequence's last (up to the launch's bound, max_parts) are read and
  // dropped with selects, so neither stale workspace nor a NaN partial (a
  // bad block id) reaches the output except through its own weight.  More
  // than 256 partitions (a caller-chosen partition size) are taken 256 at a
  // time with the running sums rescaled.
  constexpr int COLS = D / 4;
  constexpr int CW = RW_COLS < COLS ? RW_COLS : COLS;  // float4 columns per workgroup
  constexpr int PL = 256 / CW;                         // partition lanes
  constexpr int NPT = 256 / PL;                        // partitions per thread per 256
  __shared__ float s_max[4], s_sum[4];
  __shared__ float s_w[256];
  __shared__ float4 s_o[4][CW];
  const int h = blockIdx.x / (COLS / CW);
  const int chunk = blockIdx.x % (COLS / CW);
  const int b = blockIdx.y;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int c = tid % CW, g = tid / CW;
  const int64_t base = (static_cast<int64_t>(b) * a.H + h) * a.max_parts;
  const float2* ml = reinterpret_cast<const float2*>(a.ws_ml) + base;
  const float* accs = a.ws_acc + base * D + (chunk * CW + c) * 4;
  const int last = a.max_parts - 1;

  float2 mlv = ml[min(tid, last)];
  float4 av[NPT];
#pragma unroll
  for (int i = 0; i < NPT; ++i) av[i] = *reinterpret_cast<const float4*>(accs + static_cast<int64_t>(min(g + i * PL, last)) * D);
  const int ctx = seq_ctx(a, b);
  const int nparts = (ctx + (1 << a.part_shift) - 1) >> a.part_shift;
  // A sequence of one partition (its output is already written) takes the
  // same path with every partition masked and stores nothing: no branch on
  // the length stands between the loads above and their issue.
  const bool merge = nparts > 1;

  float M = -INFINITY, L = 0.f;
  float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int p0 = 0;;) {
    const bool mine = p0 + tid < nparts;
    const float mt = mine ? mlv.x : -INFINITY;
    const float wmax = mie::wave_max(mt);
    if (lane == 0) s_max[wave] = wmax;
    __syncthreads();
    const float mn = fmaxf(M, fmaxf(fmaxf(s_max[0], s_max[1]), fmaxf(s_max[2], s_max[3])));
    const float mr = mn == -INFINITY ? 0.f : mn;
    const float keep = mie::fast_exp2(M - mr);  // 0 for the first 256
    const float w = mine ? mie::fast_exp2(mt - mr) : 0.f;
    s_w[tid] = w;
    const float lsum = mie::wave_sum(mine ? mlv.y * w : 0.f);
    if (lane == 0) s_sum[wave] = lsum;
    __syncthreads();
    L = L * keep + ((s_sum[0] + s_sum[1]) + (s_sum[2] + s_sum[3]));
    o.x *= keep;
    o.y *= keep;
    o.z *= keep;
    o.w *= keep;
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
      const int q = g + i * PL;
      const bool in = p0 + q < nparts;
      const float wi = s_w[q];
      o.x = in ? fmaf(wi, av[i].x, o.x) : o.x;
      o.y = in ? fmaf(wi, av[i].y, o.y) : o.y;
      o.z = in ? fmaf(wi, av[i].z, o.z) : o.z;
      o.w = in ? fmaf(wi, av[i].w, o.w) : o.w;
    }
    M = mn;
    p0 += 256;
    if (p0 >= nparts) break;
    __syncthreads();  // s_max, s_sum and s_w are rewritten by the next 256
    mlv = ml[min(p0 + tid, last)];
#pragma unroll
    for (int i = 0; i < NPT; ++i)
      av[i] = *reinterpret_cast<const float4*>(accs + static_cast<int64_t>(min(p0 + g + i * PL, last)) * D);
  }
  // Sum over the partition lanes: lanes c, c + CW, ... of a wave hold the
  // same columns, then the four waves through LDS.
#pragma unroll
  for (int off = CW; off < 64; off <<= 1) {
    o.x += __shfl_xor(o.x, off);
    o.y += __shfl_xor(o.y, off);
    o.z += __shfl_xor(o.z, off);
    o.w += __shfl_xor(o.w, off);
  }
  if (lane < CW) s_o[wave][lane] = o;
  __syncthreads();
  if (tid >= CW || !merge) return;
  const float4 v0 = s_o[0][tid], v1 = s_o[1][tid], v2 = s_o[2][tid], v3 = s_o[3][tid];
  const float inv = 1.f / L;
  float r[4] = {((v0.x + v1.x) + (v2.x + v3.x)) * inv, ((v0.y + v1.y) + (v2.y + v3.y)) * inv,
                ((v0.z + v1.z) + (v2.z + v3.z)) * inv, ((v0.w + v1.w) + (v2.w + v3.w)) * inv};
  store_out<DT, 4>(a.out, b * a.o_sb + h * a.o_sh + (chunk * CW + c) * 4, r, a.out_f32);
}

// ---- host side --------------------------------------------------------------

// Head dims built for each dtype.  Each needs D % VEC == 0 (VEC = 4 for f32,
// min(8, D) for bf16), D % 4 == 0 and D <= 256.
#define MIE_FOR_EACH_HEAD_DIM(X) X(4) X(8) X(16) X(32) X(64) X(96) X(128) X(256)

struct KernelShape {
  int tile;  // tokens per tile; 0 = (dtype, head_dim) not built
  int tpl;   // tokens per wave load
};

template <int DT, int D>
constexpr KernelShape shape_of() {
  return KernelShape{Geometry<DT, D>::TILE, Geometry<DT, D>::TPL};
}

KernelShape shape_for(int dtype, int head_dim) {
#define MIE_SHAPE_CASE(DD)                                         \
  case DD:                                                         \
    return dtype == MIE_DTYPE_F32 ? shape_of<MIE_DTYPE_F32, DD>()  \
                                  : shape_of<MIE_DTYPE_BF16, DD>();
  if (dtype != MIE_DTYPE_F32 && dtype != MIE_DTYPE_BF16) return KernelShape{0, 0};
  switch (head_dim) {
    MIE_FOR_EACH_HEAD_DIM(MIE_SHAPE_CASE)
    default: return KernelShape{0, 0};
  }
#undef MIE_SHAPE_CASE
}

int ilog2(uint32_t x) {
  int s = 0;
  while ((1u << s) < x) ++s;
  return s;
}

bool is_pow2(int64_t x) { return x > 0 && (x & (x - 1)) == 0; }

struct Plan {
  int32_t part;
  int32_t max_parts;
  int64_t ws_bytes;
  bool fast;
  bool wg;  // workgroup form (one workgroup per (sequence, head), no merge launch)
};

int32_t plan(int32_t batch, int32_t num_heads, int32_t head_dim, int32_t block_size, int32_t max_ctx,
             int32_t dtype, int32_t requested, Plan* out) {
  const KernelShape ks = shape_for(dtype, head_dim);
  if (ks.tile == 0)
    return mie::fail(MIE_ERR_UNSUPPORTED, "mie_paged_decode: head_dim %d dtype %d not built", head_dim,
                     dtype);
  if (batch < 0 || num_heads <= 0 || max_ctx < 0 || block_size <= 0)
    return mie::fail(MIE_ERR_INVALID,
                     "mie_paged_decode: bad shape batch=%d heads=%d block_size=%d max_ctx=%d", batch,
                     num_heads, block_size, max_ctx);
  const bool fast_blocks = is_pow2(block_size) && block_size % ks.tpl == 0;
  const int64_t fast_cap = static_cast<int64_t>(kWindow) * block_size;  // FAST: <= kWindow blocks
  const int64_t rows = static_cast<int64_t>(batch) * num_heads;
  const bool wg = requested == -1 ||
                  (requested == 0 && rows <= kWgMaxRows &&
                   (max_ctx <= kWgShortCtx || (rows >= kWgMinRows && max_ctx <= kWgMaxCtx)));
  if (requested < -1)
    return mie::fail(MIE_ERR_INVALID, "mie_paged_decode: partition_tokens %d (0 = automatic, -1 = workgroup form)",
                     requested);
  if (wg) {
    // One partition per sequence, split among the workgroup's waves in
    // tile-aligned slices.
    int64_t part = ks.tile;
    while (part < max_ctx && part < (int64_t{1} << 30)) part <<= 1;
    const int64_t per_wave = (static_cast<int64_t>(max_ctx) + kSplitWaves - 1) / kSplitWaves;
    const int64_t slice = (per_wave + ks.tile - 1) / ks.tile * ks.tile;
    out->part = static_cast<int32_t>(part);
    out->max_parts = 1;
    out->ws_bytes = 0;
    // A slice starts on a tile boundary, not necessarily a block boundary, so it
    // touches at most (slice + block_size - 2) / block_size + 1 blocks.
    out->fast = fast_blocks && slice + block_size <= fast_cap;
    out->wg = true;
    return MIE_OK;
  }
  int64_t part;
  if (requested > 0) {
    if (!is_pow2(requested) || requested % ks.tile != 0)
      return mie::fail(MIE_ERR_INVALID,
                       "mie_paged_decode: partition_tokens %d must be a power of two and a multiple "
                       "of the %d-token tile",
                       requested, ks.tile);
    part = requested;
  } else {
    part = ks.tile;
    while (part < max_ctx && (rows * ((max_ctx + part - 1) / part) > kTargetItems ||
                              (max_ctx + part - 1) / part > kMaxParts))
      part <<= 1;
    if (fast_blocks && part > fast_cap && ks.tile <= fast_cap) part = fast_cap;
  }
  if (part > (int64_t{1} << 30)) part = int64_t{1} << 30;
  const int64_t max_parts = max_ctx > 0 ? (max_ctx + part - 1) / part : 1;
  if (max_parts > 0x7fffffff) return mie::fail(MIE_ERR_INVALID, "mie_paged_decode: too many partitions");
  out->part = static_cast<int32_t>(part);
  out->max_parts = static_cast<int32_t>(max_parts);
  out->ws_bytes = max_parts > 1 ? static_cast<int64_t>(batch) * num_heads * max_parts * (head_dim + 2) * 4 : 0;
  out->fast = fast_blocks && part <= fast_cap;
  out->wg = false;
  return MIE_OK;
}

// wg: the workgroup form; else flat_items > 0: the flat work list with that
// many workgroups; 0: the grid form.
template <int DT, int D>
int32_t launch(DecodeArgs& a, int batch, bool fast, bool wg, const WgOrder& order, int64_t flat_items,
               hipStream_t st) {
  const int head_groups = (a.H + kWaves - 1) / kWaves;
  if (wg) {
    const dim3 grid(a.H, batch);
    if (fast) {
      paged_decode_wg_kernel<DT, D, true><<<grid, 64 * kSplitWaves, 0, st>>>(a, order);
    } else {
      paged_decode_wg_kernel<DT, D, false><<<grid, 64 * kSplitWaves, 0, st>>>(a, order);
    }
    return mie::check_launch("paged_decode_wg_kernel");
  }
  if (flat_items > 0) {
    const dim3 grid(static_cast<uint32_t>(flat_items));
    if (fast) {
      paged_decode_flat_kernel<DT, D, true><<<grid, 64 * kWaves, 0, st>>>(a, batch, head_groups);
    } else {
      paged_decode_flat_kernel<DT, D, false><<<grid, 64 * kWaves, 0, st>>>(a, batch, head_groups);
    }
  } else {
    const dim3 grid(a.max_parts, head_groups, batch);
    if (fast) {
      paged_decode_grid_kernel<DT, D, true><<<grid, 64 * kWaves, 0, st>>>(a);
    } else {
      paged_decode_grid_kernel<DT, D, false><<<grid, 64 * kWaves, 0, st>>>(a);
    }
  }
  int32_t rc = mie::check_launch("paged_decode_kernel");
  if (rc != MIE_OK || a.max_parts <= 1) return rc;
  constexpr int kCols = D / 4;
  constexpr int kChunks = kCols / (RW_COLS < kCols ? RW_COLS : kCols);
  paged_decode_reduce_kernel<DT, D><<<dim3(a.H * kChunks, batch), 256, 0, st>>>(a);
  return mie::check_launch("paged_decode_reduce_kernel");
}

int32_t dispatch(int dtype, int head_dim, DecodeArgs& a, int batch, bool fast, bool wg, const WgOrder& order,
                 int64_t flat_items, hipStream_t st) {
#define MIE_LAUNCH_CASE(DD)                                                                                \
  case DD:                                                                                                 \
    return dtype == MIE_DTYPE_F32 ? launch<MIE_DTYPE_F32, DD>(a, batch, fast, wg, order, flat_items, st)   \
                                  : launch<MIE_DTYPE_BF16, DD>(a, batch, fast, wg, order, flat_items, st);
  switch (head_dim) {
    MIE_FOR_EACH_HEAD_DIM(MIE_LAUNCH_CASE)
    default: return mie::fail(MIE_ERR_UNSUPPORTED, "mie_paged_decode: head_dim %d not built", head_dim);
  }
#undef MIE_LAUNCH_CASE
}

bool aligned(const void* p, int n) { return reinterpret_cast<uintptr_t>(p) % n == 0; }

}  // namespace

extern "C" int32_t mie_paged_decode_supported(int32_t head_dim, int32_t dtype) {
  return shape_for(dtype, head_dim).tile != 0 ? 1 : 0;
}

extern "C" int32_t mie_paged_decode_plan(int32_t batch, int32_t num_heads, int32_t head_dim,
                                         int32_t block_size, int32_t max_ctx_len, int32_t dtype,
                                         int32_t partition_tokens, int32_t* partition_tokens_out,
                                         int64_t* workspace_bytes_out) {
  Plan p;
  const int32_t rc = plan(batch, num_heads, head_dim, block_size, max_ctx_len, dtype, partition_tokens, &p);
  if (rc != MIE_OK) return rc;
  if (partition_tokens_out) *partition_tokens_out = p.part;
  if (workspace_bytes_out) *workspace_bytes_out = p.ws_bytes;
  return MIE_OK;
}

namespace {

// mie_paged_decode, and with k_new / v_new (rows [B, H, D]) mie_paged_decode_append.
int32_t decode_impl(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k_pool, const void* v_pool,
                    int64_t pool_stride_block, int64_t pool_stride_head, int32_t num_blocks,
                    const int32_t* block_tables, int64_t block_table_stride, const int32_t* ctx_lens,
                    const int32_t* ctx_lens_host, int32_t ctx_len, int32_t max_ctx_len, int32_t batch,
                    int32_t num_heads, int32_t head_dim, int32_t block_size, float scale, void* out,
                    int64_t out_stride_b, int64_t out_stride_h, int32_t out_dtype, void* workspace,
                    int64_t workspace_bytes, int32_t partition_tokens, const void* k_new, const void* v_new,
                    int64_t new_stride_b, int64_t new_stride_h, int32_t dtype, void* stream,
                    bool check_only = false) {
  Plan p;
  int32_t rc = plan(batch, num_heads, head_dim, block_size, max_ctx_len, dtype, partition_tokens, &p);
  if (rc != MIE_OK) return rc;
  if (batch == 0) return MIE_OK;
  if (num_blocks <= 0)
    return mie::fail(MIE_ERR_INVALID, "mie_paged_decode: num_blocks=%d", num_blocks);
  if (!ctx_lens && (ctx_len < 0 || ctx_len > max_ctx_len))
    return mie::fail(MIE_ERR_INVALID, "mie_paged_decode: ctx_len %d outside [0, max_ctx_len=%d]", ctx_len,
                     max_ctx_len);
  if (batch > 65535 || num_heads > 65535 * kWaves || (p.wg && num_heads > 65535))
    return mie::fail(MIE_ERR_INVALID, "mie_paged_decode: batch or heads too large");
  if (out_dtype != MIE_DTYPE_F32 && out_dtype != dtype)
    return mie::fail(MIE_ERR_UNSUPPORTED, "mie_paged_decode: out_dtype %d must be f32 or the input dtype",
                     out_dtype);
  if (!q || !k_pool || !v_pool || !block_tables || !out)
    return mie::fail(MIE_ERR_INVALID, "mie_paged_decode: null pointer");
  if (pool_stride_head < static_cast<int64_t>(block_size) * head_dim ||
      pool_stride_block < static_cast<int64_t>(num_heads) * pool_stride_head)
    return mie::fail(MIE_ERR_INVALID, "mie_paged_decode: pool strides overlap");
  if (p.ws_bytes > 0 && (!workspace || workspace_bytes < p.ws_bytes || !aligned(workspace, 16)))
    return mie::fail(MIE_ERR_WORKSPACE, "mie_paged_decode: needs a 16-byte aligned workspace of %lld bytes",
                     static_cast<long long>(p.ws_bytes));

  // Every vector access must be naturally aligned: lane loads are 8 or 16
  // bytes, outputs are written 4 or VEC elements at a time.
  const int elt = mie::elt_size(dtype);
  const int oelt = mie::elt_size(out_dtype);
  const int vec = dtype == MIE_DTYPE_F32 ? 4 : (head_dim < 8 ? head_dim : 8);
  const int vb = vec * elt;
  const int ob = 4 * oelt;
  const bool ok_align = aligned(q, vb) && aligned(k_pool, vb) && aligned(v_pool, vb) &&
                        (q_stride_b * elt) % vb == 0 && (q_stride_h * elt) % vb == 0 &&
                        (pool_stride_block * elt) % vb == 0 && (pool_stride_head * elt) % vb == 0 &&
                        aligned(out, vec * oelt) && (out_stride_b * oelt) % (vec * oelt) == 0 &&
                        (out_stride_h * oelt) % (vec * oelt) == 0 && (vec * oelt) % ob == 0;
  if (!ok_align) return mie::fail(MIE_ERR_INVALID, "mie_paged_decode: misaligned q / pool / out");
  if ((k_new == nullptr) != (v_new == nullptr))
    return mie::fail(MIE_ERR_INVALID, "mie_paged_decode_append: pass both k_new and v_new");
  if (k_new && !(aligned(k_new, vb) && aligned(v_new, vb) && (new_stride_b * elt) % vb == 0 &&
                 (new_stride_h * elt) % vb == 0))
    return mie::fail(MIE_ERR_INVALID, "mie_paged_decode_append: misaligned new rows");
  if (k_new && !ctx_lens && ctx_len < 1)
    return mie::fail(MIE_ERR_INVALID, "mie_paged_decode_append: ctx_len %d leaves no slot for the new token", ctx_len);
  if (check_only) return MIE_OK;

  DecodeArgs a{};
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
  a.max_parts = p.max_parts;
  a.part_shift = ilog2(static_cast<uint32_t>(p.part));
  if (p.max_parts > 1) {
    a.ws_acc = static_cast<float*>(workspace);
    a.ws_ml = a.ws_acc + static_cast<int64_t>(batch) * num_heads * p.max_parts * head_dim;
  } else {
    a.ws_acc = nullptr;
    a.ws_ml = nullptr;
  }
  // Work items for the flat form: exact when the lengths are known on the host
  // (a host copy, or one scalar length), otherwise the grid's upper bound.
  int64_t flat_items = 0;
  if (batch <= kFlatMaxBatch) {
    const int64_t head_groups = (num_heads + kWaves - 1) / kWaves;
    auto items_of = [&](int64_t c) {
      c = c < 0 ? 0 : (c > max_ctx_len ? max_ctx_len : c);
      const int64_t parts = (c + p.part - 1) / p.part;
      return (parts > 0 ? parts : 1) * head_groups;
    };
    if (!ctx_lens) {
      flat_items = batch * items_of(ctx_len);
    } else if (ctx_lens_host) {
      for (int b = 0; b < batch; ++b) flat_items += items_of(ctx_lens_host[b]);
    } else {
      flat_items = static_cast<int64_t>(batch) * p.max_parts * head_groups;
    }
    if (flat_items > 0x7fffffff) flat_items = 0;  // beyond a 1-D grid: use the grid form
  }
  // Longest first for the workgroup form when host lengths are given.
  WgOrder order{};
  if (p.wg && ctx_lens && ctx_lens_host && batch > 1 && batch <= kWgOrderMax) {
    for (int b = 0; b < batch; ++b) order.seq[b] = static_cast<uint16_t>(b);
    auto len = [&](int b) {
      const int c = ctx_lens_host[b];
      return c < 0 ? 0 : (c > max_ctx_len ? max_ctx_len : c);
    };
    // A total order (length descending, then index), so the in-place sort gives
    // the stable order without a temporary buffer.
    std::sort(order.seq, order.seq + batch,
              [&](uint16_t x, uint16_t y) { return len(x) > len(y) || (len(x) == len(y) && x < y); });
    order.n = batch;
  }
  if (p.wg && p.fast) {
    const int64_t blocks = (static_cast<int64_t>(max_ctx_len) + block_size - 1) / block_size;
    if (blocks <= kWindow) a.win_blocks = static_cast<int32_t>(blocks);
  }
  if (k_new) {
    if (p.wg) {
      // The decode kernel stores the rows and attends to the new token itself.
      a.k_new = static_cast<const char*>(k_new);
      a.v_new = static_cast<const char*>(v_new);
      a.new_sb = new_stride_b;
      a.new_sh = new_stride_h;
    } else {
      // Partition form: append each sequence's last token first (same stream).
      const int32_t rc = mie::kv_append_impl(const_cast<void*>(k_pool), const_cast<void*>(v_pool), pool_stride_block,
                                             pool_stride_head, num_blocks, k_new, v_new, new_stride_b, new_stride_h, 0,
                                             block_tables, block_table_stride, ctx_lens, ctx_len, -1, batch, 1,
                                             num_heads, head_dim, block_size, dtype, stream);
      if (rc != MIE_OK) return rc;
    }
  }
  return dispatch(dtype, head_dim, a, batch, p.fast, p.wg, order, flat_items, static_cast<hipStream_t>(stream));
}

}  // namespace

extern "C" int32_t mie_paged_decode(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                    const void* k_pool, const void* v_pool, int64_t pool_stride_block,
                                    int64_t pool_stride_head, int32_t num_blocks,
                                    const int32_t* block_tables, int64_t block_table_stride,
                                    const int32_t* ctx_lens, const int32_t* ctx_lens_host,
                                    int32_t ctx_len, int32_t max_ctx_len,
                                    int32_t batch, int32_t num_heads, int32_t head_dim,
                                    int32_t block_size, float scale, void* out, int64_t out_stride_b,
                                    int64_t out_stride_h, int32_t out_dtype, void* workspace,
                                    int64_t workspace_bytes, int32_t partition_tokens, int32_t dtype,
                                    void* stream) {
  return decode_impl(q, q_stride_b, q_stride_h, k_pool, v_pool, pool_stride_block, pool_stride_head, num_blocks,
                     block_tables, block_table_stride, ctx_lens, ctx_lens_host, ctx_len, max_ctx_len, batch,
                     num_heads, head_dim, block_size, scale, out, out_stride_b, out_stride_h, out_dtype, workspace,
                     workspace_bytes, partition_tokens, nullptr, nullptr, 0, 0, dtype, stream);
}

extern "C" int32_t mie_paged_decode_append(const void* q, int64_t q_stride_b, int64_t q_stride_h, void* k_pool,
                                           void* v_pool, int64_t pool_stride_block, int64_t pool_stride_head,
                                           int32_t num_blocks, const int32_t* block_tables,
                                           int64_t block_table_stride, const int32_t* ctx_lens,
                                           const int32_t* ctx_lens_host, int32_t ctx_len, int32_t max_ctx_len,
                                           int32_t batch, int32_t num_heads, int32_t head_dim, int32_t block_size,
                                           float scale, void* out, int64_t out_stride_b, int64_t out_stride_h,
                                           int32_t out_dtype, void* workspace, int64_t workspace_bytes,
                                           int32_t partition_tokens, const void* k_new, const void* v_new,
                                           int64_t new_stride_b, int64_t new_stride_h, int32_t dtype, void* stream) {
  if (!k_new || !v_new) return mie::fail(MIE_ERR_INVALID, "mie_paged_decode_append: null new rows");
  return decode_impl(q, q_stride_b, q_stride_h, k_pool, v_pool, pool_stride_block, pool_stride_head, num_blocks,
                     block_tables, block_table_stride, ctx_lens, ctx_lens_host, ctx_len, max_ctx_len, batch,
                     num_heads, head_dim, block_size, scale, out, out_stride_b, out_stride_h, out_dtype, workspace,
                     workspace_bytes, partition_tokens, k_new, v_new, new_stride_b, new_stride_h, dtype, stream);
}

namespace mie {

int32_t paged_decode_check(const void* q, const void* k_pool, const void* v_pool, int64_t pool_stride_block,
                           int64_t pool_stride_head, int32_t num_blocks, const int32_t* block_table,
                           int32_t num_heads, int32_t head_dim, int32_t block_size, void* out, int32_t dtype) {
  const int64_t row = static_cast<int64_t>(num_heads) * head_dim;
  return decode_impl(q, row, head_dim, k_pool, v_pool, pool_stride_block, pool_stride_head, num_blocks, block_table,
                     0, nullptr, nullptr, 1, 1, 1, num_heads, head_dim, block_size, 1.0f, out, row, head_dim, dtype,
                     nullptr, 0, 0, nullptr, nullptr, 0, 0, dtype, nullptr, /*check_only=*/true);
}

}  // namespace mie

// ---- the allocation-free variant ---------------------------------------------

// Split-context workspace of mie_paged_decode_noalloc: one copy per GPU the
// library runs on, held until the process ends.  In host code `scratch` is a
// stand-in for the symbol, not a device address; kernels get the address that
// hipGetSymbolAddress returns for the current device.
static __device__ __align__(256) unsigned char scratch[MIE_PAGED_DECODE_NOALLOC_MAX_WORKSPACE];

namespace {

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxScratchDevices];  // per device, resolved on its first call

// The scratch array's device address on the device `stream` belongs to (the
// current device for the null stream), resolved once per device with that
// device current.
int32_t scratch_address(hipStream_t stream, void** out) {
  int current = -1;
  hipError_t e = hipGetDevice(&current);
  if (e != hipSuccess) return mie::fail(MIE_ERR_LAUNCH, "mie_paged_decode_noalloc: hipGetDevice: %s",
                                        hipGetErrorString(e));
  int dev = current;
  if (stream) {
    hipDevice_t sd = 0;
    e = hipStreamGetDevice(stream, &sd);
    if (e != hipSuccess)
      return mie::fail(MIE_ERR_INVALID, "mie_paged_decode_noalloc: hipStreamGetDevice: %s", hipGetErrorString(e));
    dev = static_cast<int>(sd);
  }
  if (dev < 0 || dev >= kMaxScratchDevices)
    return mie::fail(MIE_ERR_INVALID, "mie_paged_decode_noalloc: device %d beyond the %d supported", dev,
                     kMaxScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    if (dev != current && (e = hipSetDevice(dev)) != hipSuccess)
      return mie::fail(MIE_ERR_LAUNCH, "mie_paged_decode_noalloc: hipSetDevice(%d): %s", dev, hipGetErrorString(e));
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (dev != current) (void)hipSetDevice(current);
    if (e != hipSuccess || !ptr)
      return mie::fail(MIE_ERR_LAUNCH, "mie_paged_decode_noalloc: hipGetSymbolAddress(scratch) on device %d: %s",
                       dev, hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return MIE_OK;
}

}  // namespace

extern "C" int32_t mie_paged_decode_noalloc(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                            const void* k_pool, const void* v_pool, int64_t pool_stride_block,
                                            int64_t pool_stride_head, int32_t num_blocks,
                                            const int32_t* block_tables, int64_t block_table_stride,
                                            const int32_t* ctx_lens, const int32_t* ctx_lens_host, int32_t ctx_len,
                                            int32_t max_ctx_len, int32_t batch, int32_t num_heads,
                                            int32_t head_dim, int32_t block_size, float scale, void* out,
                                            int64_t out_stride_b, int64_t out_stride_h, int32_t out_dtype,
                                            int32_t partition_tokens, int32_t dtype, void* stream) {
  Plan p;
  int32_t rc = plan(batch, num_heads, head_dim, block_size, max_ctx_len, dtype, partition_tokens, &p);
  if (rc != MIE_OK) return rc;
  if (p.ws_bytes > MIE_PAGED_DECODE_NOALLOC_MAX_WORKSPACE)
    return mie::fail(MIE_ERR_WORKSPACE,
                     "mie_paged_decode_noalloc: this decode needs a %lld-byte split workspace, above the "
                     "%lld bytes of the library's scratch; call mie_paged_decode with a workspace",
                     static_cast<long long>(p.ws_bytes),
                     static_cast<long long>(MIE_PAGED_DECODE_NOALLOC_MAX_WORKSPACE));
  void* ws = nullptr;
  rc = scratch_address(static_cast<hipStream_t>(stream), &ws);
  if (rc != MIE_OK) return rc;
  return decode_impl(q, q_stride_b, q_stride_h, k_pool, v_pool, pool_stride_block, pool_stride_head, num_blocks,
                     block_tables, block_table_stride, ctx_lens, ctx_lens_host, ctx_len, max_ctx_len, batch,
                     num_heads, head_dim, block_size, scale, out, out_stride_b, out_stride_h, out_dtype, ws,
                     MIE_PAGED_DECODE_NOALLOC_MAX_WORKSPACE, partition_tokens, nullptr, nullptr, 0, 0, dtype, stream);
}

