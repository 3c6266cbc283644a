// One decoder block for one decode token from a stored launch plan.
//
// The block of the reference (src/moe_engine/model.py:494-498, attention half
// :226-269) for a single new token is, with a plan that holds an accumulator
// row and a context of at most kFusedMaxCtx tokens, four launches of this
// library: the QKV projection into the pool (mie_qkv_append), the attention
// fused with the output projection (mie_attn_out_acc: per-head shares summed
// in fixed point into the accumulator), and the MoE half forming the residual
// sum itself (mie_moe_decode_block_acc, two launches).  Otherwise it is five:
// mie_qkv_append, the paged decode attention (mie_paged_decode), out_proj
// with the residual add (mie_linear_residual) and the MoE half
// (mie_moe_decode_block).  Issued one by one from Python, each costs a
// foreign call of two dozen arguments; the eager decode step is then bound by
// the host.  Here the arguments that do not change from token to token
// (weights, pools, table, scratch rows, shapes) are stored once in
// caller-owned host memory, and each token is one call with the input row,
// the position (or a device counter pair, for a captured graph) and the
// stream.  The launches and their arguments are exactly those of the entry
// points named, so the results are bit-identical to calling them in turn.
// mie_block_plan_init makes every host check those entry points make, so a
// call that passes its own checks launches the whole block.
#include <string.h>

#include "mie_common.h"

namespace {

constexpr uint32_t kPlanMagic = 0x6d696562;  // "mieb"

struct BlockPlan {
  uint32_t magic;
  int32_t dtype;
  int32_t dim, num_heads, head_dim, block_size;
  // attention half
  const void *attn_ln_w, *attn_ln_b;
  float attn_ln_eps;
  const void *w_in, *b_in, *w_out, *b_out;
  void *k_pool, *v_pool;
  int64_t pool_stride_block, pool_stride_head;
  int32_t num_blocks;
  const int32_t* block_table;
  int32_t block_table_len;
  float scale;
  void *q, *attn, *h;
  void* workspace;
  int64_t workspace_bytes;
  // MoE half
  const void *moe_ln_w, *moe_ln_b;
  float moe_ln_eps;
  const void *router, *w1, *b1, *w2, *b2;
  int32_t num_experts, top_k, hidden;
  void *router_logits, *expert_ids, *route_weights, *hidden_act, *out;
  // fused attention + output projection (mie_attn_out_acc): fixed-point sums
  // [dim + 1], or NULL for the five-launch form only
  void* acc;
  // Layer 0 with the embedding folded into its QKV launch
  // (mie_block_plan_set_embedding): the tables and the row x is formed in.
  const void* tok_table;
  int32_t vocab;
  const void* pos_table;
  int32_t max_positions;
  void* x_emb;
};

// Contexts the four-launch form serves: each of a head's workgroups reads the
// head's whole context, so past this length the partitioned decode (every CU
// on one head's context) plus the separate projection launch is faster.
// Measured at config 1's shape (eager decode step, ms, four / five launches):
// 64 tokens 0.338 / 0.361, 256 0.351 / 0.384, 512 0.371 / 0.407, 1024
// 0.425 / 0.473, 1536 0.475 / 0.419, 2040 0.526 / 0.419 - past 1024 the
// five-launch decode takes its partition form.
constexpr int32_t kFusedMaxCtx = 1024;

// Blocks one mie_blocks_decode call runs.
constexpr int32_t kMaxStepBlocks = 256;

}  // namespace

extern "C" int64_t mie_block_plan_bytes(void) { return static_cast<int64_t>(sizeof(BlockPlan)); }

extern "C" int32_t mie_block_plan_init(
    void* plan, int64_t plan_bytes, int32_t dim, int32_t num_heads, int32_t head_dim, int32_t block_size,
    int32_t dtype, const void* attn_ln_weight, const void* attn_ln_bias, float attn_ln_eps, const void* w_in,
    const void* b_in, const void* w_out, const void* b_out, void* k_pool, void* v_pool, int64_t pool_stride_block,
    int64_t pool_stride_head, int32_t num_blocks, const int32_t* block_table, int32_t block_table_len, float scale,
    void* q, void* attn, void* h, void* workspace, int64_t workspace_bytes, const void* moe_ln_weight,
    const void* moe_ln_bias, float moe_ln_eps, const void* router_weight, const void* w1, const void* b1,
    const void* w2, const void* b2, int32_t num_experts, int32_t top_k, int32_t hidden, void* router_logits,
    void* expert_ids, void* route_weights, void* hidden_act, void* out, void* acc) {
  if (!plan || plan_bytes < static_cast<int64_t>(sizeof(BlockPlan)))
    return mie::fail(MIE_ERR_INVALID, "mie_block_plan_init: plan needs %lld bytes",
                     static_cast<long long>(sizeof(BlockPlan)));
  if (dim <= 0 || num_heads <= 0 || head_dim <= 0 || block_size <= 0 || workspace_bytes < 0)
    return mie::fail(MIE_ERR_INVALID, "mie_block_plan_init: dim %d heads %d head_dim %d block_size %d", dim,
                     num_heads, head_dim, block_size);
  if (!q || !attn || !h || !out)
    return mie::fail(MIE_ERR_INVALID, "mie_block_plan_init: null scratch or output row");
  if (block_table_len <= 0)
    return mie::fail(MIE_ERR_INVALID, "mie_block_plan_init: block table of %d entries", block_table_len);
  // Every check the five launches would make, made now, so that a plan that
  // initialises never fails half-way through a block.  x is the per-call
  // input: a stand-in that passes the checks here, checked in mie_block_decode.
  const void* x_stand_in = reinterpret_cast<const void*>(static_cast<uintptr_t>(256));
  int32_t rc = mie::qkv_append_check(x_stand_in, attn_ln_weight, attn_ln_bias, w_in, dim, k_pool, v_pool,
                                     pool_stride_block, pool_stride_head, num_blocks, block_table, block_table_len,
                                     nullptr, 0, q, num_heads, head_dim, block_size, dtype);
  if (rc != MIE_OK) return rc;
  rc = mie::paged_decode_check(q, k_pool, v_pool, pool_stride_block, pool_stride_head, num_blocks, block_table,
                               num_heads, head_dim, block_size, attn, dtype);
  if (rc != MIE_OK) return rc;
  rc = mie::linear_residual_check(attn, w_out, h, dim, dim, dtype);
  if (rc != MIE_OK) return rc;
  rc = mie::moe_decode_block_check(h, moe_ln_weight, moe_ln_bias, router_weight, w1, b1, w2, b2, num_experts, top_k,
                                   dim, hidden, router_logits, expert_ids, route_weights, hidden_act, out, dtype);
  if (rc != MIE_OK) return rc;
  if (acc) {
    rc = mie::attn_out_check(q, k_pool, v_pool, pool_stride_block, pool_stride_head, num_blocks, block_table,
                             block_table_len, 1, num_heads, head_dim, block_size, w_out, acc, dtype);
    if (rc == MIE_ERR_UNSUPPORTED) {
      acc = nullptr;  // a shape the fused attention is not built for: the five-launch form serves every call
      mie::clear_error();
    } else if (rc != MIE_OK) {
      return rc;
    }
  }
  if (acc) {
    rc = mie::moe_decode_block_acc_check(x_stand_in, acc, b_out, h, moe_ln_weight, moe_ln_bias, router_weight, w1,
                                         b1, w2, b2, num_experts, top_k, dim, hidden, router_logits, expert_ids,
                                         route_weights, hidden_act, out, dtype);
    if (rc != MIE_OK) return rc;
  }
  BlockPlan p{};
  p.magic = kPlanMagic;
  p.dtype = dtype;
  p.dim = dim;
  p.num_heads = num_heads;
  p.head_dim = head_dim;
  p.block_size = block_size;
  p.attn_ln_w = attn_ln_weight;
  p.attn_ln_b = attn_ln_bias;
  p.attn_ln_eps = attn_ln_eps;
  p.w_in = w_in;
  p.b_in = b_in;
  p.w_out = w_out;
  p.b_out = b_out;
  p.k_pool = k_pool;
  p.v_pool = v_pool;
  p.pool_stride_block = pool_stride_block;
  p.pool_stride_head = pool_stride_head;
  p.num_blocks = num_blocks;
  p.block_table = block_table;
  p.block_table_len = block_table_len;
  p.scale = scale;
  p.q = q;
  p.attn = attn;
  p.h = h;
  p.workspace = workspace;
  p.workspace_bytes = workspace ? workspace_bytes : 0;
  p.moe_ln_w = moe_ln_weight;
  p.moe_ln_b = moe_ln_bias;
  p.moe_ln_eps = moe_ln_eps;
  p.router = router_weight;
  p.w1 = w1;
  p.b1 = b1;
  p.w2 = w2;
  p.b2 = b2;
  p.num_experts = num_experts;
  p.top_k = top_k;
  p.hidden = hidden;
  p.router_logits = router_logits;
  p.expert_ids = expert_ids;
  p.route_weights = route_weights;
  p.hidden_act = hidden_act;
  p.out = out;
  p.acc = acc;
  memcpy(plan, &p, sizeof(p));
  return MIE_OK;
}

namespace {

// The block's QKV launch: x read, or formed from the embedding tables.
int32_t qkv(const BlockPlan& p, const mie::QkvEmbedding& emb, bool embed, const void* x, const int32_t* pos_dev,
            int32_t position, void* stream) {
  if (embed)
    return mie::qkv_append_embedded(emb, p.attn_ln_w, p.attn_ln_b, p.attn_ln_eps, p.w_in, p.b_in, p.dim, p.k_pool,
                                    p.v_pool, p.pool_stride_block, p.pool_stride_head, p.num_blocks, p.block_table,
                                    p.block_table_len, pos_dev, position, p.q, p.num_heads, p.head_dim,
                                    p.block_size, p.dtype, stream);
  return mie_qkv_append(x, p.attn_ln_w, p.attn_ln_b, p.attn_ln_eps, p.w_in, p.b_in, p.dim, p.k_pool, p.v_pool,
                        p.pool_stride_block, p.pool_stride_head, p.num_blocks, p.block_table, p.block_table_len,
                        pos_dev, position, p.q, p.num_heads, p.head_dim, p.block_size, p.dtype, stream);
}

}  // namespace

namespace {

// One block call, checked: the plan, its input row and the position, and
// whether the launches it would make fit the plan (the fused form, or the
// decode's split-context workspace).  Nothing is launched here.
struct BlockCall {
  BlockPlan p;
  mie::QkvEmbedding emb;
  bool embed;
  const void* x;
  const int32_t* pos_dev;
  const int32_t* ctx_dev;
  int32_t position, max_ctx;
  bool fused;
  int64_t ws_need;
};

// x: the block's input row, or (with token_id) NULL and the row formed from
// the plan's embedding tables by the QKV launch.
int32_t check_call(const void* plan, const void* x, const int64_t* token_id, const int32_t* counters,
                   int32_t position, BlockCall* c) {
  if (!plan) return mie::fail(MIE_ERR_INVALID, "mie_block_decode: null plan");
  BlockPlan& p = c->p;
  memcpy(&p, plan, sizeof(p));
  if (p.magic != kPlanMagic) return mie::fail(MIE_ERR_INVALID, "mie_block_decode: plan not initialised");
  c->emb = mie::QkvEmbedding{};
  c->embed = token_id != nullptr;
  if (token_id) {
    if (!p.tok_table)
      return mie::fail(MIE_ERR_INVALID, "mie_block_decode_embed: the plan has no embedding (mie_block_plan_set_embedding)");
    if (reinterpret_cast<uintptr_t>(token_id) % 8)
      return mie::fail(MIE_ERR_INVALID, "mie_block_decode_embed: misaligned token id");
    c->emb = mie::QkvEmbedding{token_id, p.tok_table, p.vocab, p.pos_table, p.max_positions, p.x_emb};
    x = p.x_emb;
  }
  if (!x || reinterpret_cast<uintptr_t>(x) % 16 != 0 || position < 0)
    return mie::fail(MIE_ERR_INVALID, "mie_block_decode: x %p (16-byte aligned) position %d", x, position);
  if (static_cast<int64_t>(position) >= static_cast<int64_t>(p.block_table_len) * p.block_size)
    return mie::fail(MIE_ERR_INVALID, "mie_block_decode: position %d lies past the %d-entry block table", position,
                     p.block_table_len);
  if (x == p.h || x == p.q || x == p.attn)
    return mie::fail(MIE_ERR_INVALID, "mie_block_decode: x aliases one of the plan's intermediate rows");
  c->x = x;
  // With counters the position and context length are read on the device
  // (counters[0], counters[1]) and `position` bounds them: it sizes the
  // launch and chooses the form.
  c->pos_dev = counters;
  c->ctx_dev = counters ? counters + 1 : nullptr;
  c->position = position;
  c->max_ctx = position + 1;
  c->fused = p.acc && c->max_ctx <= kFusedMaxCtx &&
             (static_cast<int64_t>(c->max_ctx) + p.block_size - 1) / p.block_size <= mie::kAttnOutMaxBlocks;
  c->ws_need = 0;
  if (c->fused) return MIE_OK;
  // The decode's split-context workspace is checked before anything is
  // launched, so a call that cannot finish changes nothing.
  const int32_t rc = mie_paged_decode_plan(1, p.num_heads, p.head_dim, p.block_size, c->max_ctx, p.dtype, 0, nullptr,
                                           &c->ws_need);
  if (rc != MIE_OK) return rc;
  if (c->ws_need > p.workspace_bytes)
    return mie::fail(MIE_ERR_WORKSPACE, "mie_block_decode: position %d needs a %lld-byte workspace, plan has %lld",
                     position, static_cast<long long>(c->ws_need), static_cast<long long>(p.workspace_bytes));
  return MIE_OK;
}

// The launches of a checked call.
int32_t launch_call(const BlockCall& c, void* stream) {
  const BlockPlan& p = c.p;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  int32_t rc = qkv(p, c.emb, c.embed, c.x, c.pos_dev, c.position, stream);
  if (rc != MIE_OK) return rc;
  if (c.fused) {
    // Four launches: QKV into the pool, attention with the output projection
    // summed into acc, then the MoE half forming x + out_proj(a) itself.
    rc = mie::attn_out_launch(p.q, p.k_pool, p.v_pool, p.pool_stride_block, p.pool_stride_head, p.num_blocks,
                              p.block_table, p.block_table_len, c.ctx_dev, c.max_ctx, c.max_ctx, p.num_heads,
                              p.head_dim, p.block_size, p.scale, p.w_out, p.acc, p.dtype, st);
    if (rc != MIE_OK) return rc;
    return mie_moe_decode_block_acc(c.x, p.acc, p.b_out, p.h, p.moe_ln_w, p.moe_ln_b, p.moe_ln_eps, p.router, p.w1,
                                    p.b1, p.w2, p.b2, p.num_experts, p.top_k, p.dim, p.hidden, p.router_logits,
                                    p.expert_ids, p.route_weights, p.hidden_act, p.out, p.dtype, stream);
  }
  const int64_t row = static_cast<int64_t>(p.num_heads) * p.head_dim;
  rc = mie_paged_decode(p.q, row, p.head_dim, p.k_pool, p.v_pool, p.pool_stride_block, p.pool_stride_head,
                        p.num_blocks, p.block_table, p.block_table_len, c.ctx_dev, nullptr, c.max_ctx, c.max_ctx, 1,
                        p.num_heads, p.head_dim, p.block_size, p.scale, p.attn, row, p.head_dim, p.dtype,
                        c.ws_need ? p.workspace : nullptr, c.ws_need, 0, p.dtype, stream);
  if (rc != MIE_OK) return rc;
  rc = mie_linear_residual(p.attn, p.w_out, p.b_out, c.x, p.h, p.dim, p.dim, p.dtype, stream);
  if (rc != MIE_OK) return rc;
  return mie_moe_decode_block(p.h, p.moe_ln_w, p.moe_ln_b, p.moe_ln_eps, p.router, p.w1, p.b1, p.w2, p.b2,
                              p.num_experts, p.top_k, p.dim, p.hidden, p.router_logits, p.expert_ids,
                              p.route_weights, p.hidden_act, p.out, p.dtype, stream);
}

int32_t block_decode(const void* plan, const void* x, const int64_t* token_id, const int32_t* counters,
                     int32_t position, void* stream) {
  BlockCall c;
  const int32_t rc = check_call(plan, x, token_id, counters, position, &c);
  return rc != MIE_OK ? rc : launch_call(c, stream);
}

}  // namespace

extern "C" int32_t mie_block_plan_launches(const void* plan, int32_t position) {
  if (!plan) return -mie::fail(MIE_ERR_INVALID, "mie_block_plan_launches: null plan");
  BlockPlan p;
  memcpy(&p, plan, sizeof(p));
  if (p.magic != kPlanMagic) return -mie::fail(MIE_ERR_INVALID, "mie_block_plan_launches: plan not initialised");
  if (position < 0) return -mie::fail(MIE_ERR_INVALID, "mie_block_plan_launches: position %d", position);
  const int32_t max_ctx = position + 1;
  if (p.acc && max_ctx <= kFusedMaxCtx &&
      (static_cast<int64_t>(max_ctx) + p.block_size - 1) / p.block_size <= mie::kAttnOutMaxBlocks)
    return 4;
  int64_t ws_need = 0;
  const int32_t rc = mie_paged_decode_plan(1, p.num_heads, p.head_dim, p.block_size, max_ctx, p.dtype, 0, nullptr,
                                           &ws_need);
  if (rc != MIE_OK) return -rc;
  return ws_need > 0 ? 6 : 5;  // a split context adds the partials' merge launch
}

extern "C" int32_t mie_block_decode(const void* plan, const void* x, const int32_t* counters, int32_t position,
                                    void* stream) {
  return block_decode(plan, x, nullptr, counters, position, stream);
}

extern "C" int32_t mie_block_decode_embed(const void* plan, const int64_t* token_id, const int32_t* counters,
                                          int32_t position, void* stream) {
  if (!token_id) return mie::fail(MIE_ERR_INVALID, "mie_block_decode_embed: null token id");
  return block_decode(plan, nullptr, token_id, counters, position, stream);
}

extern "C" int32_t mie_block_plan_set_embedding(void* plan, const void* token_table, int32_t vocab,
                                                const void* pos_table, int32_t max_positions, void* x_out) {
  if (!plan) return mie::fail(MIE_ERR_INVALID, "mie_block_plan_set_embedding: null plan");
  BlockPlan p;
  memcpy(&p, plan, sizeof(p));
  if (p.magic != kPlanMagic) return mie::fail(MIE_ERR_INVALID, "mie_block_plan_set_embedding: plan not initialised");
  const int64_t one = 0;
  const mie::QkvEmbedding e{&one, token_table, vocab, pos_table, max_positions, x_out};
  const int32_t rc = mie::qkv_embedding_check(e, p.dim);
  if (rc != MIE_OK) return rc;
  if (x_out == p.q || x_out == p.attn || x_out == p.h || x_out == p.out)
    return mie::fail(MIE_ERR_INVALID, "mie_block_plan_set_embedding: x_out aliases one of the plan's rows");
  p.tok_table = token_table;
  p.vocab = vocab;
  p.pos_table = pos_table;
  p.max_positions = max_positions;
  p.x_emb = x_out;
  memcpy(plan, &p, sizeof(p));
  return MIE_OK;
}

extern "C" int32_t mie_blocks_decode(const void* const* plans, int32_t num_plans, const int64_t* token_id,
                                     const int32_t* counters, int32_t position, void* stream) {
  if (!plans || num_plans <= 0 || num_plans > kMaxStepBlocks)
    return mie::fail(MIE_ERR_INVALID, "mie_blocks_decode: %d plans (1 to %d)", num_plans, kMaxStepBlocks);
  if (!token_id) return mie::fail(MIE_ERR_INVALID, "mie_blocks_decode: null token id");
  // Every block is checked before the first launch, so a call that cannot
  // finish (a split context that outgrew a plan's workspace included)
  // launches nothing; the second pass checks each block again (a few hundred
  // nanoseconds) and launches it.  Block i > 0 reads block i - 1's output row.
  for (int pass = 0; pass < 2; ++pass) {
    const void* prev_out = nullptr;
    for (int32_t i = 0; i < num_plans; ++i) {
      BlockCall c;
      int32_t rc = check_call(plans[i], prev_out, i == 0 ? token_id : nullptr, counters, position, &c);
      if (rc != MIE_OK) return rc;
      if (c.p.out == prev_out)
        return mie::fail(MIE_ERR_INVALID, "mie_blocks_decode: blocks %d and %d share an output row", i - 1, i);
      prev_out = c.p.out;
      if (pass == 1 && (rc = launch_call(c, stream)) != MIE_OK) return rc;
    }
  }
  return MIE_OK;
}
