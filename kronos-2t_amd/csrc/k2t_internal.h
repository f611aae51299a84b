// Host-side objects behind the C ABI (include/k2t_hip.h) and the kernel launchers.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/k2t_hip.h"

#include <stdexcept>
#include <string>

struct k2t_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    int max_segments = 0;  // cap on waves (K segments) per GEMV workgroup; 0 = automatic
    int exact = 0;         // 1: bit-exact fmaf-chain epilogue
    int stage_x = 1;       // 1: single-token GEMVs stage the int8 activation through LDS
    int mfma = 1;          // 1: batched NF4 GEMVs on the matrix cores (k2t_ctx_set_mfma)
    int num_cus = 256;
    // small device scratch (debug entry points): grown on demand
    float *scratch = nullptr;
    size_t scratch_cap = 0;  // floats
    float *rms_scratch = nullptr;
    size_t rms_cap = 0;
    // grouped-query attention span words of k2t_attn_decode ({payload, epoch}, zeroed when
    // allocated), then its counters {epoch, merges done} and timeout word
    unsigned long long *gqa_words = nullptr;
    size_t gqa_cap = 0;  // words
    // Hadamard sign masks of 64-blocks 0..kSignBlocks-1 (bit i = sign of element i),
    // uploaded at creation for the GEMV's fused activation builder.
    uint64_t *signs = nullptr;
};
constexpr int kSignBlocks = 512;  // K <= 32768

enum k2t_fmt : int32_t { K2T_FMT_NIBBLE4 = 1, K2T_FMT_NF = 2 };

struct k2t_mat {
    k2t_ctx *ctx = nullptr;
    int device = 0;
    int32_t fmt = 0;
    int32_t rows = 0, cols = 0;
    int32_t nc = 0, stripes = 0, pairs = 0, has_tail = 0;
    int32_t hp = 0;           // bit-plane: hi planes (0..2)
    int32_t bits = 0, sgc = 1;  // NF
    uint32_t cb[4] = {0, 0, 0, 0};  // NF codebook bytes 0-15
    const uint8_t *pair = nullptr, *tail = nullptr;
    size_t pair_len = 0, tail_len = 0;
    bool owns = false;
    int32_t nf3_lane = 0;  // NF3 stripe-chunks in lane order (launch_nf3_lane_order)
};

namespace k2t {

struct Error : std::runtime_error {
    int code;
    Error(int c, const std::string &m) : std::runtime_error(m), code(c) {}
};

void hip_check(hipError_t e, const char *what);
void set_last_error(const std::string &msg);

// Grows the context's scratch buffer (synchronous allocation).
void ensure_scratch(k2t_ctx *ctx, size_t floats);

// Rearranges NF3 stripe-chunks in place into the lane order the GEMV streams fastest:
// nrec matrices rec_stride bytes apart, each `pairs` pair records of ptot bytes (or, with
// tail set, one tail stripe), nc chunks, scale groups of sgc chunks.
void launch_nf3_lane_order(hipStream_t st, uint8_t *base, size_t rec_stride, int nrec, size_t ptot, int pairs,
                           int nc, int sgc, bool tail);

struct GemvPlan {
    int stripe_mode;   // 1: one workgroup per stripe, 0: per stripe pair
    int rb_lo, rb_hi;  // row blocks: pairs (then the odd tail stripe), or stripes
    int nseg, cps;     // waves per workgroup (K segments) and chunks per wave
};
void launch_stream_read(hipStream_t st, const void *src, size_t bytes, uint32_t *sink);
GemvPlan plan_gemv(const k2t_ctx *ctx, const k2t_mat *m, int s0, int s1);

void launch_gemv(k2t_ctx *ctx, const k2t_mat *m, const int8_t *xq, const float *xs,
                 const int32_t *xsum, int ntok, int s0, int s1, float *out, size_t out_stride,
                 int32_t *dots);

// GEMV whose int8 activation is built by each wave from an fp32 source (one token):
//   K2T_XS_RMSNORM: src = hidden[K], w = norm weights -> RMSNorm + FWHT + int8
//   K2T_XS_SWIGLU : src = interleaved gate_up[2K]      -> SwiGLU + FWHT + int8
// Codes equal those of rmsnorm_act / swiglu_act followed by launch_gemv.
//   K2T_XS_STAGED : a ready int8 activation (xq, xs, xsum) staged through LDS per wave
//   K2T_XS_STAGED_DMA: as K2T_XS_STAGED, staged by direct-to-LDS loads (see gemv_kernel)
enum { K2T_XS_GLOBAL = 0, K2T_XS_RMSNORM = 1, K2T_XS_SWIGLU = 2, K2T_XS_STAGED = 3, K2T_XS_STAGED_DMA = 5 };
// gu_split = 1: a split [gate; up] matrix whose rows are written in [gate64, up64] blocks.
void launch_gemv_fused(k2t_ctx *ctx, const k2t_mat *m, int xs_mode, const float *src, const float *w, float eps,
                       float *out, bool accumulate, int gu_split = 0);
uint64_t hadamard_sign_mask_host(uint64_t block);

// Grouped GEMV over sparse-MoE experts of one .k2tm bank (see GemvParams::route): slot z
// streams the matrix of expert route[z]; `geom` gives the matrix shape and format (its
// pair pointer is unused).  One token; the activation is built by the fused builder from
// src + z * slot_src.
struct GemvGroup {
    const int *route;
    int nslots;
    const uint8_t *bank;
    size_t stride;
    uint32_t mat_off, cb_off;
    size_t slot_out, slot_src;
    int gu_split;
    // Routing inside the launch (gate_up only; rt_w = NULL: route[] is ready on entry):
    // the router rows rt_w [rt_E][d] (+ rt_b), logit words rt_words [rt_E], the published
    // sorted ids rt_pub [nslots], the call counter rt_ctr (advanced by a later launch) and
    // the timeout flag rt_err; ids / weights also land in route / rt_wts.
    const float *rt_w = nullptr, *rt_b = nullptr;
    unsigned long long *rt_words = nullptr, *rt_pub = nullptr;
    const uint32_t *rt_ctr = nullptr;
    int *rt_err = nullptr;
    float *rt_wts = nullptr;
    int rt_E = 0, rt_norm = 0, rt_scoring = 0;
    uint32_t rt_spin = 0;
    // A ready int8 activation (xs_mode 0): per slot (slot_act 1: row z of xq / xs / xsum)
    // or shared by every slot (slot_act 0).
    const int8_t *xq = nullptr;
    const float *xs = nullptr;
    const int32_t *xsum = nullptr;
    int slot_act = 0;
};
// GEMV of a ready int8 activation (ntok tokens); gu_split 1 writes a [gate; up] matrix's
// rows in [gate64, up64] blocks.
// Tile-major copy of an activation for the matrix-core GEMV (act_tile_store), written by
// the kernel that quantizes the activation; null: the GEMV makes its own copy.
struct ActTiles {
    int8_t *xt = nullptr;
    float *st = nullptr;
    int32_t *ut = nullptr;  // the chunks' code sums (read by bit-plane matrices)
};
void launch_gemv_ex(k2t_ctx *ctx, const k2t_mat *m, const int8_t *xq, const float *xs, const int32_t *xsum, int ntok,
                    float *out, size_t out_stride, bool accumulate, int gu_split = 0, ActTiles tiles = ActTiles{});
void launch_swiglu_act(hipStream_t st, const uint64_t *signs, const float *gu, int inter, int ntok, int8_t *q,
                       float *s, int32_t *sums, bool exact, ActTiles tiles = ActTiles{});
// Batched NF4 / bit-plane GEMV on the matrix cores (k2t_gemm_mfma.hip): kMfmaMinTokens or
// more tokens of a ready int8 activation, outputs equal to the exact-order GEMV's.
constexpr int kMfmaMinTokens = 16;
bool gemm_mfma_supported(const k2t_mat *m, int ntok);
void launch_gemm_mfma(k2t_ctx *ctx, const k2t_mat *m, const int8_t *xq, const float *xs, const int32_t *xsum,
                      int ntok, float *out, size_t out_stride, bool accum, ActTiles tiles = ActTiles{});
// gate_up (interleaved [gate64, up64] blocks) from producer tiles with the SwiGLU + FWHT +
// int8 of the down input (q / s / sums [token][rows / 128], its tiles into out_tiles,
// which must not be `tiles`) as the epilogue; false (nothing launched) when the plain
// launch would not take 64-token workgroups, or for other shapes.
bool launch_gemm_mfma_swiglu(k2t_ctx *ctx, const k2t_mat *gu, ActTiles tiles, int ntok, int8_t *q, float *s,
                             int32_t *sums, ActTiles out_tiles);
void launch_gemv_grouped(k2t_ctx *ctx, const k2t_mat *geom, const GemvGroup &g, int xs_mode, const float *src,
                         const float *w, float eps, float *out);

// KV cache geometry (QuantKvRawPtrs, real_llm.rs:1096-1122): `cap` slots per (layer, KV
// head); with a sliding window (window > 0), positions below `sinks` keep their own slot
// and later ones wrap in a ring of `ring` slots.  bits 8: int8 codes [slot][hd] and one
// f32 scale per slot; bits 4: NF4 nibbles [slot][hd/2] and one BF16 scale per 64-block
// [slot][hd/64] (stored in the same buffers).
struct KvRing {
    int cap, window, sinks, ring, bits;
};

// The post-processing of a qkv row's heads (qkv_post_kernel's arguments): bias, q / k
// RMSNorm weights, the RoPE table, the positions, and the K / V cache it stores into.
struct QkvPostDev {
    const float *bias, *qn, *kn, *rope;
    float eps;
    const int *pos_dev;
    int nq, nkv, layer;
    KvRing kr;
    int8_t *kq, *vq;
    float *ks, *vs;
};
// The qkv projection (head size 64) on the matrix cores from producer tiles, with
// qkv_post_kernel's work as the epilogue: q heads into out, K / V into the cache; false
// (nothing launched) where it does not apply.
bool launch_gemm_mfma_qkv(k2t_ctx *ctx, const k2t_mat *qkv, ActTiles tiles, int ntok, float *out, size_t out_stride,
                          const QkvPostDev &qp);

// Workspace of the grouped-query decode attention kernel: the span words
// ([q head][span][2 + hd] {payload, epoch}, zeroed once) and two counters {epoch of the
// last launch, merge workgroups done} (zeroed once); err receives 3 on a wait timeout.
struct GqaWork {
    unsigned long long *words;
    unsigned int *cnt;
    int *err;
};

// One-token decode attention that also does qkv_post's work (bias, QK-norm, RoPE, K/V
// store): q is then the raw qkv row.
struct AttnPost {
    int on;
    const float *bias, *qn, *kn, *rope;
    float eps;
};

bool gqa_eligible(int nsplit, int ntok, int nq, int nkv, int hd, const KvRing &kr);
size_t gqa_words(int cap, int nq, int hd, int ntok);
// Raises (and clears) a grouped-query attention wait timeout that a k2t_attn_decode call
// on this context left in its span-word workspace; called after a stream sync.
void check_gqa_timeout(k2t_ctx *ctx);

// The model takes ownership of `mat` (destroyed with the model).
void model_adopt(k2t_model *m, k2t_mat *mat);

void launch_act_quant(k2t_ctx *ctx, const float *x, const float *w, const float *inv_rms, int K,
                      int ntok, int8_t *q, float *scales, int32_t *sums);
void launch_inv_rms(k2t_ctx *ctx, const float *x, float eps, int K, int ntok, float *inv_rms);
void launch_expf_map(hipStream_t st, const float *x, float *y, size_t n);
// inv_rms per token with the x86 reference's sum-of-squares order (exact-order mode).
void launch_inv_rms_x86(hipStream_t st, const float *x, float eps, int K, int ntok, float *inv_rms);

}  // namespace k2t
