/*
 * mie_paged_kv.h - C ABI of the MI355X (gfx950) paged-KV decode path.
 *
 * One shared library, libmie_paged.so, exports these entry points.  They
 * replace the tensor work under the reference engine's paged KV cache
 * (maokner/moe-inference-engine):
 *
 *   mie_kv_append     <- PagedKVCache.write     src/moe_engine/model.py:167-184
 *   mie_kv_gather     <- PagedKVCache.read      src/moe_engine/model.py:186-201
 *   mie_paged_decode  <- paged_attention.decode src/moe_engine/paged_attention.py:113-154
 *                        and _paged_decode_kernel src/moe_engine/paged_attention.py:46-110
 *   mie_paged_decode_append <- cache.write then paged_attention.decode for a
 *                        decode token (model.py:247 then :260), in one launch
 *   mie_qkv_append    <- CachedAttention.forward's QKV projection and
 *                        cache.write for one decode token  src/moe_engine/model.py:228-247
 *   mie_linear_residual <- out_proj + the block's residual add  src/moe_engine/model.py:269, :495
 *   mie_moe_route     <- fused_moe.route         src/moe_engine/fused_moe.py:274-309
 *   mie_moe_decode    <- fused_moe.decode        src/moe_engine/fused_moe.py:312-380
 *   mie_moe_decode_block <- the block's x + moe(moe_norm(x)) for one token  src/moe_engine/model.py:496-497
 *   mie_argmax        <- Model.generate's greedy torch.argmax   src/moe_engine/model.py:603
 *   mie_lm_head       <- final_norm + output_projection (model.py:564-565) and,
 *                        optionally, the greedy argmax (:603) for one token
 *   mie_argmax_pairs  <- Model.generate's greedy torch.argmax (model.py:603) of
 *                        logits mie_lm_head just wrote, from its per-workgroup picks
 *   mie_embed         <- token_embedding(ids) + positional_embedding(pos)  src/moe_engine/model.py:558
 *   mie_attn_out_acc  <- paged_attention.decode then out_proj for one decode
 *                        token (model.py:260 then :269), per head, summed into
 *                        a fixed-point accumulator row: one launch
 *   mie_moe_decode_block_acc <- the block's x + out_proj(a) (model.py:495) and
 *                        x + moe(moe_norm(x)) (:496-497) after mie_attn_out_acc
 *   mie_block_plan_init, mie_block_decode <- one TransformerMoEBlock.forward for one
 *                        decode token (model.py:494-498 with :226-269): four or
 *                        five launches above from a stored plan, one call per token
 *   mie_block_plan_set_embedding, mie_block_decode_embed <- the embedding (model.py:558)
 *                        and the first block, the embedding inside the QKV launch
 *   mie_blocks_decode <- Model.forward's embedding and blocks for one decode token
 *                        (model.py:558-562): every block plan in one call
 *
 * Conventions shared by every entry point
 *   - Pointers are device pointers unless stated otherwise.  The library
 *     allocates nothing and never synchronises the device: every launch is
 *     queued on `stream` (a hipStream_t; NULL is the legacy default stream).
 *   - Strides are in ELEMENTS, 64-bit.  The innermost (head_dim) axis of every
 *     tensor must be contiguous.
 *   - A KV pool for ONE layer is [num_blocks, num_heads, block_size, head_dim]
 *     with the (block_size, head_dim) tile of each (block, head) contiguous:
 *     the element (blk, h, slot, d) lives at
 *         blk * pool_stride_block + h * pool_stride_head + slot * head_dim + d.
 *     Callers pass the base pointer of the layer they address
 *     (k_pool + layer * layer_stride), as the reference does with k_pool[layer]
 *     (paged_attention.py:121-122).
 *   - Logical token t of a sequence lives in physical block
 *     block_table[t / block_size] at slot t % block_size
 *     (paged_attention.py:86-88, model.py:145-147).
 *   - A block-table row holds block_table_stride entries (num_blocks entries
 *     when the stride is 0, as for the per-sequence mirror); logical blocks
 *     past the row are never read.
 *   - Block ids outside [0, num_blocks) are never dereferenced: append skips
 *     the row, gather leaves the output row unwritten, decode writes NaN for
 *     the affected (sequence, head).
 *   - Every function returns MIE_OK (0) or a non-zero MIE_ERR_* code, with a
 *     message available from mie_last_error() on the calling thread.
 */
#ifndef MIE_PAGED_KV_H
#define MIE_PAGED_KV_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types of pools, new K/V rows, queries and outputs. */
enum mie_dtype {
  MIE_DTYPE_F32 = 0,
  MIE_DTYPE_BF16 = 1,
  MIE_DTYPE_F16 = 2, /* append / gather only */
  MIE_DTYPE_F64 = 3  /* append / gather only */
};

enum mie_status {
  MIE_OK = 0,
  MIE_ERR_INVALID = 1,     /* bad argument: shape, stride, pointer, size */
  MIE_ERR_UNSUPPORTED = 2, /* valid but not built: dtype / head_dim combination */
  MIE_ERR_WORKSPACE = 3,   /* split-context workspace missing or too small */
  MIE_ERR_LAUNCH = 4       /* the HIP runtime rejected a launch */
};

/* Library ABI version (MIE_ABI_VERSION below). */
int32_t mie_abi_version(void);
#define MIE_ABI_VERSION 16

/* Message for the last non-zero status returned on this thread ("" if none). */
const char* mie_last_error(void);

/*
 * Measurement only, no counterpart in the reference: launches `workgroups`
 * (1 .. 2^20) workgroups of 256 threads of an empty kernel on `stream`, so a
 * caller can time the launch floor that a latency-bound call cannot go under.
 */
int32_t mie_empty_launch(int32_t workgroups, void* stream);

/*
 * KV append: scatter new K/V rows into the pool through block tables.
 * Replaces PagedKVCache.write (model.py:167-184): the decode store
 * pool[l, bt[p // BS], :, p % BS] = k[0, :, 0] (model.py:173-178) for seq_len
 * 1 and the prefill scatter pool[l, blocks, :, slots] = k[0].transpose(0, 1)
 * (model.py:179-184) for seq_len > 1, for `batch` sequences in one launch:
 *
 *   for b < batch, s < seq_len, h < num_heads, d < head_dim, p = pos(b) + s:
 *     pool[bt_b[p / block_size], h, p % block_size, d] = new[b, h, s, d]
 *
 * where pos(b) = positions[b] if `positions` is non-NULL (device int32[batch])
 * else `position`, and bt_b = block_tables + b * block_table_stride.  The K and
 * V sources share strides new_stride_{b,h,s}.  K and V are written by the same
 * launch; the copy is bit-exact for every dtype.  Blocks must already be
 * reserved in the tables (the host allocator does that, model.py:125-143).
 */
int32_t mie_kv_append(void* k_pool, void* v_pool, int64_t pool_stride_block,
                      int64_t pool_stride_head, int32_t num_blocks,
                      const void* k_new, const void* v_new, int64_t new_stride_b,
                      int64_t new_stride_h, int64_t new_stride_s,
                      const int32_t* block_tables, int64_t block_table_stride,
                      const int32_t* positions, int32_t position, int32_t batch,
                      int32_t seq_len, int32_t num_heads, int32_t head_dim,
                      int32_t block_size, int32_t dtype, void* stream);

/*
 * KV gather: copy one sequence's first `length` tokens of K and V out of the
 * pool into contiguous-by-token outputs.  Replaces PagedKVCache.read
 * (model.py:186-201), which returns pool[l, bt[:nb]].transpose(0, 1)
 * .reshape(H, -1, D)[:, :length]:
 *
 *   out[h * out_stride_h + t * out_stride_t + d] =
 *       pool[bt[t / block_size], h, t % block_size, d]   for t < length
 *
 * Bit-exact for every dtype.  K and V outputs share strides.
 */
int32_t mie_kv_gather(const void* k_pool, const void* v_pool, int64_t pool_stride_block,
                      int64_t pool_stride_head, int32_t num_blocks,
                      const int32_t* block_table, int32_t length, void* k_out,
                      void* v_out, int64_t out_stride_h, int64_t out_stride_t,
                      int32_t num_heads, int32_t head_dim, int32_t block_size,
                      int32_t dtype, void* stream);

/*
 * Block-table mirror append: table[start + i] = ids[i] for i < count, where
 * `table` is a device int32 table of `table_len` entries and `ids` is HOST
 * memory, read before the call returns (the ids travel in the launch's
 * arguments).  Replaces the device-mirror update of PagedKVCache._reserve
 * (model.py:135-143), block_table_device[start:start + n] =
 * torch.tensor(taken), which is a pageable host-to-device copy the host waits
 * for plus an indexing launch.  0 <= count <= 16; the entries must lie inside
 * the table.  One launch, queued on `stream`; the host does not wait.
 */
int32_t mie_block_table_append(int32_t* table, int32_t table_len, int32_t start, const int32_t* ids,
                               int32_t count, void* stream);

/*
 * Direct paged decode attention for `batch` sequences with one query token
 * each.  Replaces paged_attention.decode (paged_attention.py:113-154) and
 * _paged_decode_kernel (paged_attention.py:46-110), which computes for one
 * sequence, per head,  out = softmax(q . K^T * scale) . V  over logical tokens
 * [0, ctx_len) read in place through the block table:
 *
 *   out[b, h, :] = sum_t softmax_t(scale * <q[b, h, :], K_b[t, h, :]>) V_b[t, h, :]
 *
 * with ctx_len(b) = min(ctx_lens[b], max_ctx_len) if `ctx_lens` is non-NULL
 * (device int32[batch]) else `ctx_len` for every sequence; ctx_len(b) == 0
 * writes zeros (what scaled_dot_product_attention returns for no keys).
 * `ctx_lens_host` (optional, host int32[batch]) is a host copy of the same
 * lengths: with it the launch holds exactly the batch's work items, without it
 * the launch is sized for max_ctx_len and the surplus workgroups exit.  When
 * given, its work-item count must not be below that of ctx_lens.
 * q, K and V share `dtype` (F32 or BF16); `out_dtype` is F32 or `dtype`.
 * Accumulation is fp32 throughout.
 *
 * Split context: the tokens of each sequence are cut into partitions of
 * `partition_tokens` tokens (0 = choose automatically; otherwise a power of two
 * that is a multiple of the kernel tile, see mie_paged_decode_plan).  When a
 * sequence needs more than one partition, per-partition (max, sum, acc[D])
 * partials go to `workspace` and a second launch merges them (log-sum-exp);
 * a sequence with one partition is written by the first launch directly.
 * `workspace` must hold mie_paged_decode_plan()'s workspace_bytes; it may be
 * NULL when that is 0.  Nothing in the workspace needs clearing.
 */
int32_t mie_paged_decode(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                         const void* k_pool, const void* v_pool,
                         int64_t pool_stride_block, int64_t pool_stride_head,
                         int32_t num_blocks, const int32_t* block_tables,
                         int64_t block_table_stride, const int32_t* ctx_lens,
                         const int32_t* ctx_lens_host,
                         int32_t ctx_len, int32_t max_ctx_len, int32_t batch,
                         int32_t num_heads, int32_t head_dim, int32_t block_size,
                         float scale, void* out, int64_t out_stride_b,
                         int64_t out_stride_h, int32_t out_dtype, void* workspace,
                         int64_t workspace_bytes, int32_t partition_tokens,
                         int32_t dtype, void* stream);

/*
 * A decode step's append and attention together (model.py:247 then :260 for
 * B sequences): each sequence's new token is its LAST context token, so
 * k_new[b] / v_new[b] ([B, H, D] rows, element strides new_stride_b /
 * new_stride_h, inner axis contiguous, `dtype`) are stored at position
 * ctx_b - 1 through the block table, exactly as mie_kv_append stores them,
 * and the output is mie_paged_decode's over tokens [0, ctx_b) with that token
 * included.  The pools are written.  When the plan takes the workgroup form
 * this is ONE launch: the decode kernel stores the rows and takes the new
 * token's score and value from the rows it loaded, without reading them back;
 * otherwise the append runs as its own launch before the decode, on the same
 * stream.  A sequence with ctx_b = 0 gets no append and a zero output; a new
 * token whose block id is outside the pool is not stored and its output is
 * NaN.  Other arguments and limits as mie_paged_decode.
 */
int32_t mie_paged_decode_append(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                void* k_pool, void* v_pool, int64_t pool_stride_block,
                                int64_t pool_stride_head, int32_t num_blocks,
                                const int32_t* block_tables, int64_t block_table_stride,
                                const int32_t* ctx_lens, const int32_t* ctx_lens_host,
                                int32_t ctx_len, int32_t max_ctx_len, int32_t batch,
                                int32_t num_heads, int32_t head_dim, int32_t block_size,
                                float scale, void* out, int64_t out_stride_b,
                                int64_t out_stride_h, int32_t out_dtype, void* workspace,
                                int64_t workspace_bytes, int32_t partition_tokens,
                                const void* k_new, const void* v_new, int64_t new_stride_b,
                                int64_t new_stride_h, int32_t dtype, void* stream);

/*
 * Host-only planning query for mie_paged_decode (no device work).  Given the
 * launch shape it returns the partition size the decode will use
 * (`partition_tokens` = 0 asks for the automatic choice) and the workspace
 * bytes it needs (0 when every sequence fits one partition).
 */
int32_t mie_paged_decode_plan(int32_t batch, int32_t num_heads, int32_t head_dim,
                              int32_t block_size, int32_t max_ctx_len, int32_t dtype,
                              int32_t partition_tokens,
                              int32_t* partition_tokens_out,
                              int64_t* workspace_bytes_out);

/* 1 if mie_paged_decode is built for (head_dim, dtype), else 0. */
int32_t mie_paged_decode_supported(int32_t head_dim, int32_t dtype);

/*
 * QKV projection of ONE decode token written straight into the pools
 * (CachedAttention.forward, model.py:228-234, and PagedKVCache.write,
 * model.py:167-178, in one launch):
 *
 *   y   = LayerNorm(x; ln_weight, ln_bias, ln_eps)   (y = x when ln_weight is NULL)
 *   qkv = w_in[3*dim, dim] . y + b_in                (b_in may be NULL)
 *   q_out[0:dim]                               = qkv[0:dim]
 *   k_pool[bt[p/BS], h, p%BS, :] (and v_pool)  = qkv[dim + h*D : dim + (h+1)*D]
 *                                                (and qkv[2*dim + ...])
 *
 * p is *position_dev when that is non-NULL (a device int32, so a captured graph
 * can advance it), else `position`.  block_table holds block_table_len entries;
 * a logical block past it or a block id outside [0, num_blocks) skips the K/V
 * stores, as mie_kv_append does.  The norm is computed in float32 and rounded to
 * the model dtype, the projection accumulates in float32 and rounds once: the
 * reference's rounding points.  dim = num_heads * head_dim; x, the norm
 * parameters, w_in, b_in, q_out and the pools share `dtype` (f32 or bf16);
 * x, the norm parameters and w_in are 16-byte aligned.  mie_qkv_append_supported(dim, dtype) says whether
 * the shape is built (dim <= 2048 f32 / 4096 bf16, a multiple of 4 / 8).
 */
int32_t mie_qkv_append(const void* x, const void* ln_weight, const void* ln_bias,
                       float ln_eps, const void* w_in, const void* b_in, int32_t dim,
                       void* k_pool, void* v_pool, int64_t pool_stride_block,
                       int64_t pool_stride_head, int32_t num_blocks,
                       const int32_t* block_table, int32_t block_table_len,
                       const int32_t* position_dev, int32_t position, void* q_out,
                       int32_t num_heads, int32_t head_dim, int32_t block_size,
                       int32_t dtype, void* stream);

/* 1 if mie_qkv_append is built for (dim, dtype), else 0. */
int32_t mie_qkv_append_supported(int32_t dim, int32_t dtype);

/*
 * One-token linear layer with a residual add (the attention's out_proj and the
 * block's `x + attention(...)`, model.py:269 and :495, in one launch):
 *
 *   out[r] = residual[r] + round(weight[r, :] . x + bias[r])     r < rows
 *
 * (out = weight . x + bias when residual is NULL; bias may be NULL).  weight is
 * [rows, cols] row-major; x [cols] and weight 16-byte aligned; bias, residual and out
 * [rows] share `dtype` (f32 or bf16); out may alias residual, not x.  The
 * rounding points are the reference's: the projection is rounded to the model
 * dtype, then the sum.  Built for the widths mie_qkv_append_supported(cols,
 * dtype) accepts.
 */
int32_t mie_linear_residual(const void* x, const void* weight, const void* bias,
                            const void* residual, void* out, int32_t rows, int32_t cols,
                            int32_t dtype, void* stream);

/*
 * Router and top-k of the fused MoE decode for ONE token (fused_moe.route,
 * fused_moe.py:274-309), x and router_weight in `dtype` (float32 or
 * bfloat16), the logits and route weights float32 in both:
 *
 *   router_logits[e] = router_weight[e, :] . x            e < num_experts
 *   expert_ids[s]    = the top_k experts, largest logit first, lower id on ties
 *   route_weights[s] = softmax over the selected logits, in the same order
 *
 * x [dim] and router_weight [num_experts, dim] contiguous and 16-byte aligned,
 * dim a multiple of 4, num_experts <= 64, top_k <= 8.  One launch.
 */
int32_t mie_moe_route(const void* x, const void* router_weight, int32_t num_experts,
                      int32_t top_k, int32_t dim, void* router_logits, void* expert_ids,
                      void* route_weights, int32_t dtype, void* stream);

/*
 * Fused top-k mixture of experts for ONE decode token, with no
 * device-to-host synchronisation.  Replaces MoEFeedForward's PyTorch path for
 * a single token (model.py:443-461; its torch.where syncs once per expert) and
 * serves the reference's Triton fused MoE decode (fused_moe.py:312-380):
 * mie_moe_route, then
 *
 *   hidden_act[s] = GELU(w1[e_s] . x + b1[e_s])          e_s = expert_ids[s]
 *   out = sum over the slots in increasing e_s, from 0, of
 *         round(route_weights[s] * (w2[e_s] . hidden_act[s] + b2[e_s]))
 *
 * with GELU the exact erf form and the sum in the order and rounding of the
 * reference's index_add_ loop (model.py:455-460).  Expert weights are the
 * canonical contiguous storages w1 [E, hidden, dim], b1 [E, hidden], w2 [E,
 * dim, hidden], b2 [E, dim]; hidden_act is [top_k, hidden], out [dim].  x, the
 * router weight, w1, w2 and hidden_act are 16-byte aligned; dim and hidden are
 * multiples of 4.  The routing outputs are those of mie_moe_route.  Two
 * launches on `stream` (the W1 launch routes in every workgroup); nothing
 * needs clearing beforehand.  dim <= 2048.
 *
 * dtype (float32 or bfloat16) is that of x, the weights, hidden_act and out;
 * router_logits and route_weights are float32 either way, the routing the
 * reference keeps in float32 (model.py:448-452).  Sums run in float32.  In
 * bfloat16 each value is rounded where the reference's PyTorch path stores
 * one: each Linear's output (sum plus bias, rounded once), GELU's, the route
 * weight, the weighted product and each partial sum of the expert-id-ordered
 * sum.
 */
int32_t mie_moe_decode(const void* x, const void* router_weight, const void* w1,
                       const void* b1, const void* w2, const void* b2, int32_t num_experts,
                       int32_t top_k, int32_t dim, int32_t hidden, void* router_logits,
                       void* expert_ids, void* route_weights, void* hidden_act, void* out,
                       int32_t dtype, void* stream);

/*
 * The MoE half of a decoder block for ONE token (model.py:496-497):
 *
 *   out = x + MoE(LayerNorm(x; ln_weight, ln_bias, ln_eps))
 *
 * with MoE as in mie_moe_decode (routing outputs and hidden_act filled the
 * same way) and the norm skipped when ln_weight is NULL.  The norm uses the
 * biased variance in float32 (nn.LayerNorm), its output rounded to `dtype`;
 * the residual add rounds once.  Same arguments, dtypes and limits as
 * mie_moe_decode; out may alias x.  Two launches.
 */
int32_t mie_moe_decode_block(const void* x, const void* ln_weight, const void* ln_bias,
                             float ln_eps, const void* router_weight, const void* w1,
                             const void* b1, const void* w2, const void* b2,
                             int32_t num_experts, int32_t top_k, int32_t dim, int32_t hidden,
                             void* router_logits, void* expert_ids, void* route_weights,
                             void* hidden_act, void* out, int32_t dtype, void* stream);

/*
 * Greedy pick (Model.generate at temperature 0, model.py:603): the index
 * of the largest of x[0..n) (float32), as torch.argmax returns it - the first
 * index of the maximum, NaN counting as larger than every number - written to
 * *out as int64.  One launch of one workgroup; nothing to clear beforehand.
 * 0 < n < 2^31 - 65536.
 */
int32_t mie_argmax(const void* x, int64_t n, void* out, int32_t dtype, void* stream);

/*
 * Token plus positional embedding (model.py:558) of n tokens:
 *     out[i, :] = round(token_table[token_ids[i], :] + pos_table[pos_i, :])
 * with pos_i = positions[i] (device int32) or, when positions is NULL,
 * position + i.  token_ids are int64; tables [vocab, dim] and
 * [max_positions, dim] and out [n, dim] in `dtype` (float32 or bfloat16),
 * summed in float32 and rounded once.  An id or position outside its table
 * writes a row of NaN.  n <= 65535.
 */
int32_t mie_embed(const void* token_ids, const int32_t* positions, int32_t position, int32_t n,
                  const void* token_table, int32_t vocab, const void* pos_table, int32_t max_positions, int32_t dim,
                  void* out, int32_t dtype, void* stream);

/*
 * The decode step's head for one token (model.py:564-565, then :603):
 *     logits[v] = round(W[v, :] . round(LayerNorm(x)) + bias[v])   v < vocab
 * with the norm skipped when ln_weight is NULL and the bias when bias is NULL
 * (rounding as mie_qkv_append).  x [dim], W [vocab, dim] row-major (the tied
 * token embedding), logits [vocab], all in `dtype` (float32 or bfloat16);
 * dim as for mie_qkv_append_supported.  x, W and the norm parameters 16-byte
 * aligned.
 *
 * workspace (mie_lm_head_workspace(vocab) bytes, 4-byte aligned, or NULL):
 * the launch also leaves there each workgroup's pick of its rows - the
 * largest stored logit in torch.argmax's order (first index of the maximum,
 * NaN largest) - at no extra launch.  token_out (int64, or NULL; needs the
 * workspace): the index of the largest logit, merged from those picks by a
 * second one-workgroup launch.  Without token_out, mie_argmax_pairs makes the
 * same merge later.  Nothing needs clearing beforehand, so both launches can
 * be captured in a graph.
 *
 * advance (device int32[n_advance], n_advance <= 64; needs token_out): each
 * counter is incremented by one after the pick, in the same launch - a
 * captured decode step advances its device position and context length there.
 * NULL / 0 for none.
 */
int64_t mie_lm_head_workspace(int32_t vocab);
int32_t mie_lm_head(const void* x, const void* ln_weight, const void* ln_bias, float ln_eps, const void* weight,
                    const void* bias, int32_t vocab, int32_t dim, void* logits, void* token_out, void* workspace,
                    int64_t workspace_bytes, int32_t* advance, int32_t n_advance, int32_t dtype, void* stream);

/*
 * Greedy pick (model.py:603) of the logits a mie_lm_head call of the same
 * `vocab` wrote together with `workspace`: the per-workgroup picks there are
 * merged into *out (int64) in one launch of one workgroup - the index
 * torch.argmax returns for those logits, as long as neither they nor the
 * workspace were written since.  Queue it on the head's stream, or after it.
 */
int32_t mie_argmax_pairs(const void* workspace, int64_t workspace_bytes, int32_t vocab, void* out, void* stream);

/*
 * mie_paged_decode without the workspace arguments: an entry point that
 * allocates nothing, neither inside the library nor through the caller.  It
 * has no counterpart in the reference.  It is for callers that cannot call
 * hipMalloc or take memory from an allocator: code under HIP graph capture,
 * tight serving loops, harnesses that forbid allocation.
 *
 * The split-context workspace is a device array inside the library of
 * MIE_PAGED_DECODE_NOALLOC_MAX_WORKSPACE bytes, one per GPU, held until the
 * process ends.  A decode whose plan needs more (mie_paged_decode_plan's
 * workspace_bytes) fails with MIE_ERR_WORKSPACE before anything is launched.
 * The first call on a device looks the array's address up
 * (hipGetSymbolAddress) with that device current, so make it outside graph
 * capture.  Every call on one GPU shares that GPU's array: calls that can
 * overlap on one GPU (different streams, no ordering between them) race and
 * must be serialised by the caller.  Nothing in the array needs clearing; each
 * call writes every partial it reads.  Arguments, results and kernels are
 * those of mie_paged_decode.
 */
#define MIE_PAGED_DECODE_NOALLOC_MAX_WORKSPACE ((int64_t)16 << 20)
int32_t mie_paged_decode_noalloc(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                 const void* k_pool, const void* v_pool, int64_t pool_stride_block,
                                 int64_t pool_stride_head, int32_t num_blocks,
                                 const int32_t* block_tables, int64_t block_table_stride,
                                 const int32_t* ctx_lens, const int32_t* ctx_lens_host,
                                 int32_t ctx_len, int32_t max_ctx_len, int32_t batch,
                                 int32_t num_heads, int32_t head_dim, int32_t block_size,
                                 float scale, void* out, int64_t out_stride_b, int64_t out_stride_h,
                                 int32_t out_dtype, int32_t partition_tokens, int32_t dtype,
                                 void* stream);

/*
 * Decode attention of ONE token fused with the attention's output projection
 * (paged_attention.decode, paged_attention.py:113-154, then out_proj,
 * model.py:269), one launch.  For each head h the launch computes
 *
 *   a_h = softmax(scale * q_h . K_h^T) . V_h   over tokens [0, ctx)   (as mie_paged_decode)
 *   y_h = W_out[:, h*D : (h+1)*D] . a_h        (W_out [dim, dim] row-major, dim = H * D)
 *
 * and adds round(y_h[i] * 2^32) into acc[i] (int64, dim + 1 entries) with
 * integer atomics, so acc[i] = sum_h round(y_h[i] * 2^32) is exact and the
 * same whatever order the workgroups run in.  A y_h[i] of magnitude 2^31 / H
 * or more (or NaN) is not added - the sum of H such partials could leave
 * int64 - and acc[dim] is set instead.  acc must hold zeros
 * beforehand (mie_moe_decode_block_acc clears it after use).  ctx is *ctx_dev
 * when ctx_dev is non-NULL (device int32), else `ctx`; either is clamped to
 * max_ctx, and max_ctx spans at most 1024 blocks.  q [H * D], the pools (one
 * layer, element strides, as mie_paged_decode) and W_out are in `dtype`
 * (float32 or bfloat16) and 16-byte aligned; every product and sum is float32,
 * and in bfloat16 a_h is rounded to bfloat16 before the projection, as the
 * decode stores it.  head_dim 32, 64 or 128; block_table holds block_table_len
 * entries (ids outside the pool are skipped, as in the decode).
 */
int32_t mie_attn_out_acc(const void* q, const void* k_pool, const void* v_pool, int64_t pool_stride_block,
                         int64_t pool_stride_head, int32_t num_blocks, const int32_t* block_table,
                         int32_t block_table_len, const int32_t* ctx_dev, int32_t ctx, int32_t max_ctx,
                         int32_t num_heads, int32_t head_dim, int32_t block_size, float scale, const void* w_out,
                         void* acc, int32_t dtype, void* stream);

/*
 * The rest of a decoder block after mie_attn_out_acc (model.py:495-497):
 *
 *   h_out = x + round(acc * 2^-32 + b_out)          (NaN everywhere when acc[dim] != 0)
 *   out   = h_out + MoE(LayerNorm(h_out))           (as mie_moe_decode_block)
 *
 * and acc cleared to zeros for the next token.  Two launches: h_out is formed
 * in the W1 launch (every workgroup forms it in registers, one stores it), the
 * W2 launch adds it and clears acc.  Arguments and limits as
 * mie_moe_decode_block; in bfloat16 the projection's output and the
 * residual are each rounded to bfloat16 (as mie_linear_residual stores them).
 * acc (int64 [dim + 1]), h_out and b_out (may be NULL) 16-byte aligned; h_out
 * must not alias x.
 */
int32_t mie_moe_decode_block_acc(const void* x, const void* acc, const void* b_out, void* h_out,
                                 const void* ln_weight, const void* ln_bias, float ln_eps, const void* router_weight,
                                 const void* w1, const void* b1, const void* w2, const void* b2, int32_t num_experts,
                                 int32_t top_k, int32_t dim, int32_t hidden, void* router_logits, void* expert_ids,
                                 void* route_weights, void* hidden_act, void* out, int32_t dtype, void* stream);

/*
 * One decoder block for ONE decode token (TransformerMoEBlock.forward,
 * model.py:494-498, with the attention half model.py:226-269) from a launch
 * plan stored in caller-owned host memory of mie_block_plan_bytes() bytes.
 * mie_block_decode(plan, x, counters, position, stream) issues, on `stream`:
 *
 * with an accumulator (`acc` non-NULL, used when mie_attn_out_acc is built for
 * the shape - float32 or bfloat16, head_dim 32, 64 or 128 - and ignored otherwise) and
 * position + 1 <= 1024, four launches:
 *   mie_qkv_append(x, attn norm, in_proj, pools, block_table, position) -> q
 *   mie_attn_out_acc(q, pools, block_table, ctx = position + 1, out_proj) -> acc
 *   mie_moe_decode_block_acc(x, acc, out_proj bias, moe norm, router, experts) -> h, out
 * otherwise five (six when the decode splits the context into partitions
 * and merges them):
 *   mie_qkv_append(...)                                                   -> q
 *   mie_paged_decode(q, pools, block_table, ctx = position + 1)           -> attn
 *   mie_linear_residual(attn, out_proj, residual x)                        -> h
 *   mie_moe_decode_block(h, moe norm, router, experts)                     -> out
 *
 * with the other arguments those entry points take stored by
 * mie_block_plan_init: the block's weights and norms, the layer's pools
 * (element strides) and block table, the rows q, attn and h ([num_heads *
 * head_dim], [num_heads * head_dim], [dim], written by the call), the MoE
 * scratch, the output row and the accumulator (int64 [dim + 1], zeros when
 * the plan is made; each four-launch call leaves it zeroed again).  The
 * results are those of calling the entry points in turn.
 *
 * `counters` (device int32[2], or NULL): the position and the context length
 * are then read on the device (counters[0], counters[1]), so a captured graph
 * can advance them, and `position` is the largest position a call may see: it
 * sizes the launches and picks the form.  `workspace` (may be NULL) serves
 * the five-launch form's split context; a call whose decode needs more than
 * workspace_bytes (see mie_paged_decode_plan at batch 1 and max_ctx_len =
 * position + 1) fails with MIE_ERR_WORKSPACE before anything is launched, and
 * the caller initialises the plan again with a larger workspace.  The plan
 * holds pointers only: the caller keeps every buffer alive while the plan is
 * used, and one plan serves calls in stream order.
 *
 * mie_block_plan_init makes every host check of the launches (built width,
 * head_dim and dtype, shapes, strides,
 * alignment, null pointers) and fails with their status, so an initialised
 * plan never stops between launches.  The decode reads at most
 * block_table_len table entries (block_table_len >= 1).  mie_block_decode
 * checks x (non-NULL, 16-byte aligned, not one of the plan's rows) and
 * rejects a position at or past block_table_len * block_size, both before
 * launching.
 */
int64_t mie_block_plan_bytes(void);
int32_t mie_block_plan_init(void* plan, int64_t plan_bytes, int32_t dim, int32_t num_heads, int32_t head_dim,
                            int32_t block_size, int32_t dtype, const void* attn_ln_weight,
                            const void* attn_ln_bias, float attn_ln_eps, const void* w_in, const void* b_in,
                            const void* w_out, const void* b_out, void* k_pool, void* v_pool,
                            int64_t pool_stride_block, int64_t pool_stride_head, int32_t num_blocks,
                            const int32_t* block_table, int32_t block_table_len, float scale, void* q,
                            void* attn, void* h, void* workspace, int64_t workspace_bytes,
                            const void* moe_ln_weight, const void* moe_ln_bias, float moe_ln_eps,
                            const void* router_weight, const void* w1, const void* b1, const void* w2,
                            const void* b2, int32_t num_experts, int32_t top_k, int32_t hidden,
                            void* router_logits, void* expert_ids, void* route_weights, void* hidden_act,
                            void* out, void* acc);
int32_t mie_block_decode(const void* plan, const void* x, const int32_t* counters, int32_t position, void* stream);
/*
 * The number of launches mie_block_decode issues for `position` (the largest
 * position, with counters): 4 (attention fused with out_proj), 5, or 6 when
 * the decode splits the context and merges its partials.  Negative
 * (-MIE_ERR_*) for a bad plan or position.  Issues nothing.
 */
int32_t mie_block_plan_launches(const void* plan, int32_t position);

/*
 * Layer 0 of a decode step with the embedding folded into its QKV launch
 * (token_embedding(ids) + positional_embedding(pos), model.py:558, then the
 * first block): mie_block_plan_set_embedding stores the token table [vocab,
 * dim], the positional table [max_positions, dim] (both the model dtype,
 * 16-byte aligned) and a row x_out [dim] in a plan; mie_block_decode_embed
 * (plan, token_id, counters, position, stream) is then mie_block_decode with
 * x = round(token_table[*token_id] + pos_table[position]) (a float32 sum
 * rounded once, as mie_embed; NaN for an id or position outside its table),
 * formed inside the QKV launch from the device int64 token id and stored to
 * x_out, the block's residual.  One launch fewer than mie_embed followed by
 * mie_block_decode, with the same results.
 */
int32_t mie_block_plan_set_embedding(void* plan, const void* token_table, int32_t vocab, const void* pos_table,
                                     int32_t max_positions, void* x_out);
int32_t mie_block_decode_embed(const void* plan, const int64_t* token_id, const int32_t* counters,
                               int32_t position, void* stream);

/*
 * The embedding and every block of the decoder for one decode token in one
 * call (Model.forward's blocks, model.py:558-562): plans[0] is a plan with
 * the embedding set (as for mie_block_decode_embed), and plans[i] for i > 0
 * takes plans[i - 1]'s output row `out` as its input x.  The launches are
 * those of mie_block_decode_embed(plans[0], ...) followed by
 * mie_block_decode(plans[i], out of plans[i - 1], ...), in order, bit for
 * bit.  Every plan is checked before the first launch, so an error -
 * MIE_ERR_WORKSPACE when a split context outgrew a plan's workspace
 * included - launches nothing; the caller can then run the blocks one by one.
 * 1 <= num_plans <= 256.
 */
int32_t mie_blocks_decode(const void* const* plans, int32_t num_plans, const int64_t* token_id,
                          const int32_t* counters, int32_t position, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MIE_PAGED_KV_H */
