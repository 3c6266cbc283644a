// KV append (scatter through block tables) and KV gather (blocks -> contiguous).
//
// Both are pure copies, so they are bit-exact for any element type: a thread
// moves one VB-byte vector of one (token, head) row, where VB is the widest of
// 16/8/4/2 bytes that divides the row (head_dim * element size).  Consecutive
// threads take consecutive vectors of a row and then consecutive rows, so every
// wavefront reads and writes contiguous runs of the (block, head) tile.
#include "mie_common.h"

namespace {

// Threads per workgroup of both kernels, a constant rather than blockDim: reading
// blockDim makes the kernel take the launch's hidden arguments, 256 more bytes of
// kernel arguments per launch.
constexpr int kCopyThreads = 256;

template <int VB> struct Raw;
template <> struct Raw<16> { using T = uint4; };
template <> struct Raw<8> { using T = uint2; };
template <> struct Raw<4> { using T = uint32_t; };
template <> struct Raw<2> { using T = uint16_t; };

struct AppendArgs {
  char* k_pool;
  char* v_pool;
  int64_t pool_sblk;   // bytes
  int64_t pool_shead;  // bytes
  int32_t num_blocks;
  const char* k_new;
  const char* v_new;
  int64_t new_sb, new_sh, new_ss;  // bytes
  const int32_t* block_tables;
  int64_t bt_stride;  // elements
  uint32_t bt_cap;    // entries readable per table row
  const int32_t* positions;
  int32_t position;
  int32_t pos_bias;  // added to the position: -1 appends at a length's last slot
  int32_t seq_len;
  int32_t num_heads;
  int32_t row_bytes;
  int32_t vecs_per_row;
  int32_t vecs_per_kv;  // num_heads * vecs_per_row
  mie::FastDiv bs;      // block_size
};

// grid = (ceil(2 * vecs_per_kv / kCopyThreads), seq_len, batch): one token row set
// (all heads of K and V) per (y, z).
template <int VB>
__global__ __launch_bounds__(kCopyThreads) void kv_append_kernel(AppendArgs a) {
  using T = typename Raw<VB>::T;
  const int i = blockIdx.x * kCopyThreads + threadIdx.x;
  if (i >= 2 * a.vecs_per_kv) return;
  const int s = blockIdx.y;
  const int b = blockIdx.z;
  const bool is_v = i >= a.vecs_per_kv;
  const int r = is_v ? i - a.vecs_per_kv : i;
  const int h = r / a.vecs_per_row;
  const int vec = r - h * a.vecs_per_row;

  // The new row's vector does not depend on the position or the table, so it
  // is read first and travels with those reads.
  const char* src = (is_v ? a.v_new : a.k_new) + b * a.new_sb + h * a.new_sh + s * a.new_ss +
                    static_cast<int64_t>(vec) * VB;
  const T v = *reinterpret_cast<const T*>(src);
  const int pos = (a.positions ? a.positions[b] : a.position) + a.pos_bias + s;
  if (pos < 0) return;
  const uint32_t blk = a.bs.div(static_cast<uint32_t>(pos));
  const uint32_t slot = static_cast<uint32_t>(pos) - blk * a.bs.d;
  if (blk >= a.bt_cap) return;
  const int32_t phys = a.block_tables[b * a.bt_stride + blk];
  if (phys < 0 || phys >= a.num_blocks) return;
  char* dst = (is_v ? a.v_pool : a.k_pool) + phys * a.pool_sblk + h * a.pool_shead +
              static_cast<int64_t>(slot) * a.row_bytes + static_cast<int64_t>(vec) * VB;
  *reinterpret_cast<T*>(dst) = v;
}

struct GatherArgs {
  const char* k_pool;
  const char* v_pool;
  int64_t pool_sblk, pool_shead;  // bytes
  int32_t num_blocks;
  const int32_t* block_table;
  int32_t length;
  char* k_out;
  char* v_out;
  int64_t out_sh, out_st;  // bytes
  int32_t row_bytes;
  mie::FastDiv vecs_per_row;
  mie::FastDiv bs;
};

// grid = (ceil(length * vecs_per_row / kCopyThreads), num_heads, 2 [K, V]).
template <int VB>
__global__ __launch_bounds__(kCopyThreads) void kv_gather_kernel(GatherArgs a) {
  using T = typename Raw<VB>::T;
  const uint32_t i = blockIdx.x * kCopyThreads + threadIdx.x;
  const uint32_t t = a.vecs_per_row.div(i);
  if (t >= static_cast<uint32_t>(a.length)) return;
  const uint32_t vec = i - t * a.vecs_per_row.d;
  const int h = blockIdx.y;
  const bool is_v = blockIdx.z != 0;

  const uint32_t blk = a.bs.div(t);
  const uint32_t slot = t - blk * a.bs.d;
  const int32_t phys = a.block_table[blk];
  if (phys < 0 || phys >= a.num_blocks) return;

  const char* src = (is_v ? a.v_pool : a.k_pool) + phys * a.pool_sblk + h * a.pool_shead +
                    static_cast<int64_t>(slot) * a.row_bytes + static_cast<int64_t>(vec) * VB;
  char* dst = (is_v ? a.v_out : a.k_out) + h * a.out_sh + static_cast<int64_t>(t) * a.out_st +
              static_cast<int64_t>(vec) * VB;
  *reinterpret_cast<T*>(dst) = *reinterpret_cast<const T*>(src);
}

// Widest vector that divides the row and every byte stride the kernel adds to
// it, so each vector access is naturally aligned.
int pick_vec_bytes(int row_bytes, std::initializer_list<int64_t> byte_strides,
                   std::initializer_list<const void*> ptrs) {
  for (int vb : {16, 8, 4, 2}) {
    bool ok = row_bytes % vb == 0;
    for (int64_t s : byte_strides) ok = ok && (s % vb == 0);
    for (const void* p : ptrs) ok = ok && (reinterpret_cast<uintptr_t>(p) % vb == 0);
    if (ok) return vb;
  }
  return 0;
}

}  // namespace

int32_t mie::kv_append_impl(void* k_pool, void* v_pool, int64_t pool_stride_block, int64_t pool_stride_head,
                            int32_t num_blocks, const void* k_new, const void* v_new, int64_t new_stride_b,
                            int64_t new_stride_h, int64_t new_stride_s, const int32_t* block_tables,
                            int64_t block_table_stride, const int32_t* positions, int32_t position,
                            int32_t pos_bias, int32_t batch, int32_t seq_len, int32_t num_heads,
                            int32_t head_dim, int32_t block_size, int32_t dtype, void* stream) {
  const int elt = mie::elt_size(dtype);
  if (elt == 0) return mie::fail(MIE_ERR_UNSUPPORTED, "mie_kv_append: unknown dtype %d", dtype);
  if (batch < 0 || seq_len < 0 || num_heads <= 0 || head_dim <= 0 || block_size <= 0 ||
      num_blocks <= 0)
    return mie::fail(MIE_ERR_INVALID,
                     "mie_kv_append: bad shape batch=%d seq_len=%d heads=%d head_dim=%d "
                     "block_size=%d num_blocks=%d",
                     batch, seq_len, num_heads, head_dim, block_size, num_blocks);
  if (batch == 0 || seq_len == 0) return MIE_OK;
  if (!k_pool || !v_pool || !k_new || !v_new || !block_tables)
    return mie::fail(MIE_ERR_INVALID, "mie_kv_append: null pointer");
  if (!positions && position + pos_bias < 0)
    return mie::fail(MIE_ERR_INVALID, "mie_kv_append: negative position %d", position + pos_bias);
  if (seq_len > 65535 || batch > 65535)
    return mie::fail(MIE_ERR_INVALID, "mie_kv_append: batch/seq_len above 65535");
  if (pool_stride_head < static_cast<int64_t>(block_size) * head_dim ||
      pool_stride_block < static_cast<int64_t>(num_heads) * pool_stride_head)
    return mie::fail(MIE_ERR_INVALID, "mie_kv_append: pool strides overlap");

  AppendArgs a{};
  a.k_pool = static_cast<char*>(k_pool);
  a.v_pool = static_cast<char*>(v_pool);
  a.pool_sblk = pool_stride_block * elt;
  a.pool_shead = pool_stride_head * elt;
  a.num_blocks = num_blocks;
  a.k_new = static_cast<const char*>(k_new);
  a.v_new = static_cast<const char*>(v_new);
  a.new_sb = new_stride_b * elt;
  a.new_sh = new_stride_h * elt;
  a.new_ss = new_stride_s * elt;
  a.block_tables = block_tables;
  a.bt_stride = block_table_stride;
  a.bt_cap = static_cast<uint32_t>(block_table_stride > 0 ? block_table_stride : num_blocks);
  a.positions = positions;
  a.position = position;
  a.pos_bias = pos_bias;
  a.seq_len = seq_len;
  a.num_heads = num_heads;
  a.row_bytes = head_dim * elt;
  a.bs = mie::FastDiv::make(static_cast<uint32_t>(block_size));

  const int vb = pick_vec_bytes(a.row_bytes, {a.pool_sblk, a.pool_shead, a.new_sb, a.new_sh, a.new_ss},
                                {k_pool, v_pool, k_new, v_new});
  if (vb == 0) return mie::fail(MIE_ERR_INVALID, "mie_kv_append: misaligned rows");
  a.vecs_per_row = a.row_bytes / vb;
  a.vecs_per_kv = num_heads * a.vecs_per_row;

  const int threads = kCopyThreads;
  dim3 grid((2 * a.vecs_per_kv + threads - 1) / threads, seq_len, batch);
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (vb) {
    case 16: kv_append_kernel<16><<<grid, threads, 0, st>>>(a); break;
    case 8: kv_append_kernel<8><<<grid, threads, 0, st>>>(a); break;
    case 4: kv_append_kernel<4><<<grid, threads, 0, st>>>(a); break;
    default: kv_append_kernel<2><<<grid, threads, 0, st>>>(a); break;
  }
  return mie::check_launch("mie_kv_append");
}

extern "C" int32_t mie_kv_append(void* k_pool, void* v_pool, int64_t pool_stride_block,
                                 int64_t pool_stride_head, int32_t num_blocks, const void* k_new,
                                 const void* v_new, int64_t new_stride_b, int64_t new_stride_h,
                                 int64_t new_stride_s, const int32_t* block_tables,
                                 int64_t block_table_stride, const int32_t* positions,
                                 int32_t position, int32_t batch, int32_t seq_len,
                                 int32_t num_heads, int32_t head_dim, int32_t block_size,
                                 int32_t dtype, void* stream) {
  return mie::kv_append_impl(k_pool, v_pool, pool_stride_block, pool_stride_head, num_blocks, k_new, v_new,
                             new_stride_b, new_stride_h, new_stride_s, block_tables, block_table_stride, positions,
                             position, 0, batch, seq_len, num_heads, head_dim, block_size, dtype, stream);
}

extern "C" int32_t mie_kv_gather(const void* k_pool, const void* v_pool, int64_t pool_stride_block,
                                 int64_t pool_stride_head, int32_t num_blocks,
                                 const int32_t* block_table, int32_t length, void* k_out,
                                 void* v_out, int64_t out_stride_h, int64_t out_stride_t,
                                 int32_t num_heads, int32_t head_dim, int32_t block_size,
                                 int32_t dtype, void* stream) {
  const int elt = mie::elt_size(dtype);
  if (elt == 0) return mie::fail(MIE_ERR_UNSUPPORTED, "mie_kv_gather: unknown dtype %d", dtype);
  if (length < 0 || num_heads <= 0 || head_dim <= 0 || block_size <= 0 || num_blocks <= 0)
    return mie::fail(MIE_ERR_INVALID,
                     "mie_kv_gather: bad shape length=%d heads=%d head_dim=%d block_size=%d "
                     "num_blocks=%d",
                     length, num_heads, head_dim, block_size, num_blocks);
  if (length == 0) return MIE_OK;
  if (!k_pool || !v_pool || !k_out || !v_out || !block_table)
    return mie::fail(MIE_ERR_INVALID, "mie_kv_gather: null pointer");
  if (num_heads > 65535) return mie::fail(MIE_ERR_INVALID, "mie_kv_gather: too many heads");
  // The table holds at most num_blocks entries, so no sequence is longer.
  if (static_cast<int64_t>(length) > static_cast<int64_t>(num_blocks) * block_size)
    return mie::fail(MIE_ERR_INVALID, "mie_kv_gather: length %d exceeds num_blocks * block_size", length);
  if (pool_stride_head < static_cast<int64_t>(block_size) * head_dim ||
      pool_stride_block < static_cast<int64_t>(num_heads) * pool_stride_head)
    return mie::fail(MIE_ERR_INVALID, "mie_kv_gather: pool strides overlap");

  GatherArgs a;
  a.k_pool = static_cast<const char*>(k_pool);
  a.v_pool = static_cast<const char*>(v_pool);
  a.pool_sblk = pool_stride_block * elt;
  a.pool_shead = pool_stride_head * elt;
  a.num_blocks = num_blocks;
  a.block_table = block_table;
  a.length = length;
  a.k_out = static_cast<char*>(k_out);
  a.v_out = static_cast<char*>(v_out);
  a.out_sh = out_stride_h * elt;
  a.out_st = out_stride_t * elt;
  a.row_bytes = head_dim * elt;
  a.bs = mie::FastDiv::make(static_cast<uint32_t>(block_size));

  const int vb = pick_vec_bytes(a.row_bytes, {a.pool_sblk, a.pool_shead, a.out_sh, a.out_st},
                                {k_pool, v_pool, k_out, v_out});
  if (vb == 0) return mie::fail(MIE_ERR_INVALID, "mie_kv_gather: misaligned rows");
  const int vpr = a.row_bytes / vb;
  a.vecs_per_row = mie::FastDiv::make(static_cast<uint32_t>(vpr));
  const int64_t total = static_cast<int64_t>(length) * vpr;
  if (total >= (int64_t{1} << 31))
    return mie::fail(MIE_ERR_INVALID, "mie_kv_gather: length * row vectors exceeds 2^31");

  const int threads = kCopyThreads;
  dim3 grid(static_cast<uint32_t>((total + threads - 1) / threads), num_heads, 2);
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (vb) {
    case 16: kv_gather_kernel<16><<<grid, threads, 0, st>>>(a); break;
    case 8: kv_gather_kernel<8><<<grid, threads, 0, st>>>(a); break;
    case 4: kv_gather_kernel<4><<<grid, threads, 0, st>>>(a); break;
    default: kv_gather_kernel<2><<<grid, threads, 0, st>>>(a); break;
  }
  return mie::check_launch("mie_kv_gather");
}

// ---- block-table mirror append ------------------------------------------------
//
// The host allocator takes a new block once every block_size tokens and
// appends its id to the sequence's device table.  A torch copy of a host list
// is a pageable host-to-device transfer (a staging copy the host waits for)
// plus an indexing launch; here the ids travel in the kernel arguments, so the
// host only queues one small launch and never waits.

namespace {

constexpr int kTableAppendMax = 16;

struct TableAppend {
  int32_t* table;
  int32_t start;
  int32_t count;
  int32_t ids[kTableAppendMax];
};

__global__ __launch_bounds__(64) void block_table_append_kernel(TableAppend a) {
  const int i = threadIdx.x;
  if (i < a.count) a.table[a.start + i] = a.ids[i];
}

}  // namespace

extern "C" int32_t mie_block_table_append(int32_t* table, int32_t table_len, int32_t start, const int32_t* ids,
                                          int32_t count, void* stream) {
  if (count < 0 || count > kTableAppendMax)
    return mie::fail(MIE_ERR_INVALID, "mie_block_table_append: count %d outside [0, %d]", count, kTableAppendMax);
  if (count == 0) return MIE_OK;
  if (!table || !ids) return mie::fail(MIE_ERR_INVALID, "mie_block_table_append: null pointer");
  if (start < 0 || table_len < 0 || static_cast<int64_t>(start) + count > table_len)
    return mie::fail(MIE_ERR_INVALID, "mie_block_table_append: entries [%d, %d) outside a table of %d", start,
                     start + count, table_len);
  TableAppend a;
  a.table = table;
  a.start = start;
  a.count = count;
  for (int i = 0; i < kTableAppendMax; ++i) a.ids[i] = i < count ? ids[i] : 0;
  mie::clear_error();
  block_table_append_kernel<<<1, 64, 0, static_cast<hipStream_t>(stream)>>>(a);
  return mie::check_launch("mie_block_table_append");
}
