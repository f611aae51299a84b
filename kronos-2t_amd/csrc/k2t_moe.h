// Sparse-MoE expert banks (.k2tm shards in HBM) and the one-token MoE feed-forward.
#pragma once
#include "../../include/k2t_hip.h"
#include "k2t_internal.h"

// nf_expert_byte_layout (moe_800b.rs:1332-1375) of one expert record.
struct ExpertLayout {
    size_t gu_rows, dn_rows;
    size_t gu_cb_off, dn_cb_off;
    size_t gu_pair_off, gu_pair_bytes;
    size_t dn_pair_off, dn_pair_bytes;
    size_t aligned_bytes;
};

struct k2t_experts {
    k2t_ctx *ctx = nullptr;
    k2t_k2tm_header hdr{};
    ExpertLayout lay{};
    uint8_t *d_bytes = nullptr;  // the whole shard (header page + records) in HBM
    size_t len = 0;
    bool owns = false;
    k2t_mat gu{}, dn{};  // shapes of one expert's gate_up / down (pair pointers unused)
};

namespace k2t {

ExpertLayout expert_layout(size_t d_model, size_t d_ff, int bits, size_t sgc);

// One MoE layer: a layer of a bank plus its fp32 router (device arrays).
struct MoeLayer {
    const k2t_experts *bank;
    int shard_layer;
    const float *router_w;  // [E][d_model]
    const float *router_b;  // [E] or NULL
    int top_k, norm_topk, scoring;
    // Shared expert (SharedMoeExpert, sparse_moe.rs:209-312), applied to every token: an NF
    // gate_up in [gate; up] row order and its down, an optional sigmoid gate row, and its
    // device buffer [2 * inter gate_up | d output | 64 (gate scale)].
    const k2t_mat *sh_gu = nullptr, *sh_dn = nullptr;
    const float *sh_gate = nullptr;  // [d_model] or NULL (scale 1)
    float *sh_buf = nullptr;
};

// Device workspace of one MoE forward.
struct MoeWork {
    float *gu;      // [top_k][2*d_ff] gate_up outputs, [gate64, up64] blocks
    float *eo;      // [top_k][d_model] expert outputs
    unsigned long long *words;  // [2E + 2] router logits (or partial dots and sums) as {epoch, value} words
    unsigned long long *pub;    // [K2T_MOE_MAX_TOPK] sorted route ids as {epoch, id} words
    float *wts;                 // [top_k]
    int *ids;                   // [top_k]
    uint32_t *ctr;              // route-call counter (epoch source)
    int *err;                   // raised when the route wait times out
    // exact-order mode (the context's exact flag): inv_rms, the int8 activation of x_norm
    // and the slots' down activations
    float *rms;
    int8_t *aq, *mq;            // [d], [top_k][d_ff]
    float *as, *ms;             // [d / 64], [top_k][d_ff / 64]
    int32_t *asum, *msum;
};

// Workspace size; the words and the counter must start zeroed (model: at allocation;
// the standalone entry point: launch_moe_clear before each call).
size_t moe_work_floats(const k2t_experts *b, int top_k);
void launch_moe_clear(hipStream_t st, const MoeWork &ws, int E);
MoeWork moe_work_carve(float *base, const k2t_experts *b, int top_k);
void check_moe_args(const k2t_experts *bank, int shard_layer, int top_k, int scoring);

// hidden += MoE(RMSNorm(hidden) * post_norm) for one token, on ctx->stream.
void launch_moe_ffn(k2t_ctx *ctx, const MoeLayer &L, float *hidden, const float *post_norm, float eps,
                    const MoeWork &ws);

}  // namespace k2t
