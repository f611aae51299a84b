// Decode engine: the GPU counterpart of RealLlamaEngine's SDOT paths
// (forward_token_sdot_megakernel real_llm.rs:6794-7403, forward_prompt 7407-7446,
// generate_greedy 7880-7915).  The host only enqueues kernels; the token position
// and the greedy token live in device memory, so a decode step is captured once into
// a HIP graph and replayed.
#include <float.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <vector>

#include "../../include/k2t_hip.h"
#include "k2t_decode_mk.h"
#include "k2t_internal.h"
#include "k2t_moe.h"

namespace k2t {
void launch_rmsnorm_act(hipStream_t st, const uint64_t *signs, const float *x, const float *w, float eps, int K,
                        int ntok, int8_t *q, float *s, int32_t *sums, ActTiles tiles = ActTiles{});
void launch_qkv_post(hipStream_t st, float *qkv, const float *bias, const float *qn, const float *kn, float eps,
                     const float *rope, const int *pos_dev, int nq,
                     int nkv, int hd, int ntok, int layer, KvRing kr, int8_t *kq, int8_t *vq, float *ks, float *vs,
                     bool exact);
void launch_attention_exact(hipStream_t st, const float *q, int q_stride, const int8_t *kq, const int8_t *vq,
                            const float *ks, const float *vs, const int *pos_dev, int layer, int nq, int nkv, int hd,
                            KvRing kr, float attn_scale, int ntok, int max_positions, float *out_f);
void launch_attention(hipStream_t st, const float *q, int q_stride, int8_t *kq, int8_t *vq, float *ks, float *vs,
                      const AttnPost &post, const int *pos_dev, int layer, int nq, int nkv, int hd, KvRing kr,
                      float attn_scale, int nsplit, int ntok, float *part, float *out_f, int8_t *aq, float *as,
                      int32_t *asum, const GqaWork &gqa, int ctx_bound = 0, ActTiles tiles = ActTiles{},
                      bool mfma = false);
int attn_max_splits(int max_seq);
int gqa_spans(int cap);
void launch_embed(hipStream_t st, const k2t_mat *m, const int *tokens, int ntok, float *out);
void launch_kv_synthetic(hipStream_t st, int8_t *kq, int8_t *vq, float *ks, float *vs, int layers_kv, int cap,
                         int n_pos, int hd, int bits, uint64_t seed);
void launch_kv_store(hipStream_t st, const float *heads, int n, int hd, int bits, int8_t *qbuf, float *sbuf);
void launch_embed_rows(hipStream_t st, const void *rows, bool bf16, const int *tokens, int ntok, int d, float *out);
void launch_advance_pos(hipStream_t st, int *pos, int n);
void launch_argmax(hipStream_t st, const float *x, int n, int *out_idx);

// Greedy pick (argmax_scalar, real_llm.rs:9914-9924): largest value, lowest index on ties,
// NaN never wins.  One workgroup.
__global__ __launch_bounds__(1024) void argmax_kernel(const float *__restrict__ x, int n, int *__restrict__ out) {
    __shared__ float bv[16];
    __shared__ int bi[16];
    float best = -INFINITY;
    int idx = 0x7fffffff;
    // Each thread scans its indices in increasing order (keeps the lowest index among
    // equals), eight loads in flight.
    int i = threadIdx.x;
    for (; i + 7 * (int)blockDim.x < n; i += 8 * blockDim.x) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) v[u] = x[i + u * blockDim.x];
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (v[u] > best) {
                best = v[u];
                idx = i + u * blockDim.x;
            }
    }
    for (; i < n; i += blockDim.x) {
        const float v = x[i];
        if (v > best) {
            best = v;
            idx = i;
        }
    }
    for (int m = 32; m >= 1; m >>= 1) {
        const float ov = xor_lane(best, m);
        const int oi = xor_lane(idx, m);
        if (ov > best || (ov == best && oi < idx)) {
            best = ov;
            idx = oi;
        }
    }
    if ((threadIdx.x & 63) == 0) {
        bv[threadIdx.x >> 6] = best;
        bi[threadIdx.x >> 6] = idx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float b = bv[0];
        int bix = bi[0];
        for (int w = 1; w < (int)(blockDim.x >> 6); w++)
            if (bv[w] > b || (bv[w] == b && bi[w] < bix)) {
                b = bv[w];
                bix = bi[w];
            }
        out[0] = bix == 0x7fffffff ? 0 : bix;
    }
}

void launch_argmax(hipStream_t st, const float *x, int n, int *out_idx) {
    hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(1024), 0, st, x, n, out_idx);
    hip_check(hipGetLastError(), "argmax launch");
}

}  // namespace k2t

// Device scratch of k2t_attn_decode_noalloc: the span partials (n_heads * splits *
// (head_dim + 2) floats) and the position word in the first kNoAllocScratchFloats floats;
// then the grouped-query kernel's span words (kNoAllocGqaWords 64-bit {payload, epoch}
// words), its counters {epoch, merges done} and its timeout word.  Device memory starts
// zeroed, and the words' epochs only grow, so nothing here is ever cleared (but after a
// timeout).  One copy per GPU, held until the process ends.  Host code never passes this
// name to a kernel or a copy: it is a host-side stand-in there; noalloc_scratch() looks up
// each device's own address.
constexpr size_t kNoAllocScratchFloats = (size_t)1 << 20;  // 4 MiB
constexpr size_t kNoAllocGqaWords = (size_t)1 << 19;       // 4 MiB
constexpr size_t kNoAllocTotalFloats = kNoAllocScratchFloats + 2 * (kNoAllocGqaWords + 2);
static __device__ __align__(256) float scratch[kNoAllocTotalFloats];

namespace k2t {
__global__ void store_int_kernel(int *dst, int v) {
    if (threadIdx.x == 0) dst[0] = v;
}
}  // namespace k2t

using namespace k2t;

namespace {
constexpr int kMaxNoAllocDevices = 64;
std::mutex g_noalloc_mu;
float *g_noalloc_ptr[kMaxNoAllocDevices] = {};

// The address of `scratch` on `device` (which must be current), looked up once per
// device with hipGetSymbolAddress.
float *noalloc_scratch(int device) {
    if (device < 0 || device >= kMaxNoAllocDevices) throw Error(K2T_E_ARG, "device index out of range");
    std::lock_guard<std::mutex> lock(g_noalloc_mu);
    if (!g_noalloc_ptr[device]) {
        void *p = nullptr;
        hip_check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
        g_noalloc_ptr[device] = static_cast<float *>(p);
    }
    return g_noalloc_ptr[device];
}
// The grouped-query words, counters and timeout word of one scratch region.
GqaWork gqa_work_at(unsigned long long *words, size_t cap) {
    return GqaWork{words, reinterpret_cast<unsigned int *>(words + cap), reinterpret_cast<int *>(words + cap + 1)};
}

GqaWork noalloc_gqa(int device) {
    float *base = noalloc_scratch(device);
    return gqa_work_at(reinterpret_cast<unsigned long long *>(base + kNoAllocScratchFloats), kNoAllocGqaWords);
}

// k2t_attn_decode's grouped-query workspace on the context (zeroed whenever it grows).
GqaWork ctx_gqa(k2t_ctx *ctx, size_t words) {
    if (words > ctx->gqa_cap) {
        hip_check(hipStreamSynchronize(ctx->stream), "gqa workspace sync");
        if (ctx->gqa_words) hip_check(hipFree(ctx->gqa_words), "hipFree");
        ctx->gqa_words = nullptr;
        ctx->gqa_cap = 0;
        const size_t bytes = (words + 2) * sizeof(unsigned long long);
        hipError_t e = hipMalloc((void **)&ctx->gqa_words, bytes);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            throw Error(K2T_E_NOMEM, std::string("hipMalloc failed: ") + hipGetErrorString(e));
        }
        hip_check(hipMemset(ctx->gqa_words, 0, bytes), "gqa workspace clear");
        ctx->gqa_cap = words;
    }
    return gqa_work_at(ctx->gqa_words, ctx->gqa_cap);
}

// Reads a region's timeout word after a sync; on a timeout clears the region (its epochs
// start over) and raises.
void raise_gqa_timeout(const GqaWork &g, size_t cap) {
    int e = 0;
    hip_check(hipMemcpy(&e, g.err, sizeof(int), hipMemcpyDeviceToHost), "gqa timeout word");
    if (!e) return;
    hip_check(hipMemset(g.words, 0, (cap + 2) * sizeof(unsigned long long)), "gqa workspace clear");
    throw Error(K2T_E_HIP, "grouped-query attention: span wait timed out");
}

}  // namespace

namespace k2t {
void check_gqa_timeout(k2t_ctx *ctx) {
    if (ctx->gqa_words) raise_gqa_timeout(gqa_work_at(ctx->gqa_words, ctx->gqa_cap), ctx->gqa_cap);
    bool seen = false;
    {
        std::lock_guard<std::mutex> lock(g_noalloc_mu);
        seen = ctx->device >= 0 && ctx->device < kMaxNoAllocDevices && g_noalloc_ptr[ctx->device] != nullptr;
    }
    if (seen) raise_gqa_timeout(noalloc_gqa(ctx->device), kNoAllocGqaWords);
}
}  // namespace k2t

struct k2t_model {
    k2t_ctx *ctx = nullptr;
    k2t_model_config cfg{};
    hipStream_t stream = nullptr;
    struct Layer {
        const k2t_mat *qkv = nullptr, *o = nullptr, *gu = nullptr, *down = nullptr;
        float *in_norm = nullptr, *post_norm = nullptr, *bias = nullptr;
        float *q_norm = nullptr, *k_norm = nullptr;  // per-head RMSNorm weights [hd] (Qwen3)
        bool has_moe = false;
        MoeLayer moe{};  // sparse-MoE feed-forward in place of gate_up / down
    };
    std::vector<Layer> layers;
    const k2t_mat *head = nullptr;
    float *final_norm = nullptr;
    // embedding source (embed_token_into's precedence, real_llm.rs:8063-8097)
    int embed_kind = K2T_EMBED_TIED;
    void *embed_rows = nullptr;          // f32 / bf16 rows [vocab][hidden] (device)
    const k2t_mat *embed_mat = nullptr;  // NF4 embedding matrix
    std::vector<k2t_mat *> owned;        // matrices the model destroys (k2tb loader)
    KvRing ring{};                       // KV slots: cap = max_seq, or a sliding-window ring
    float *moe_ws = nullptr;             // MoE workspace (largest layer's need)
    size_t moe_ws_floats = 0;
    float *rope = nullptr;  // [max_seq][hd] = cos | sin halves
    int8_t *kq = nullptr, *vq = nullptr;
    float *ks = nullptr, *vs = nullptr;
    int *pos_dev = nullptr;  // [0] position, [1..] tokens
    int *tokens = nullptr;
    int max_batch = 0;
    float *hidden = nullptr, *qkv = nullptr, *gu = nullptr, *logits = nullptr, *attn_part = nullptr;
    unsigned long long *attn_words = nullptr;  // grouped-query attention span words
    unsigned int *attn_cnt = nullptr;          // {its epoch, merge workgroups done}
    int8_t *xq = nullptr;
    float *xs = nullptr;
    int32_t *xsum = nullptr;
    // the activation's tile-major copy for matrix-core GEMVs (written by its producer)
    int8_t *xt = nullptr;
    float *st = nullptr;
    int32_t *ut = nullptr;
    ActTiles dtiles;  // the down input's tiles when gate_up's epilogue writes them (apart from xt)
    int pos = 0;
    bool use_graph = true;
    // 1: exact-order steps (the x86 reference's operation order throughout: in-order GEMV
    // epilogue, sequential sums of squares, its exp, sequential softmax and V sums)
    int exact = 0;
    float *rms_x86 = nullptr;  // [max_batch] inv_rms of the exact-order steps
    float *attn_f = nullptr;   // [max_batch][n_heads * head_dim] exact-order attention output
    hipGraphExec_t graph = nullptr;
    bool graph_pk = false;  // the captured step is the persistent kernel
    std::vector<void *> allocs;
    // persistent single-launch decode step (fast epilogue, NF4 or 4-plane weights)
    int persistent = 1;  // 0 off, 1 single-format models, 2 also mixed 4/5-plane models
    bool mk_ok = false;
    size_t mk_lds = 0;
    uint32_t *step_dev = nullptr;
    int *err_dev = nullptr;
    unsigned long long *ll_ha = nullptr, *ll_hb = nullptr, *ll_qkv = nullptr, *ll_apart = nullptr, *ll_oact = nullptr, *ll_gact = nullptr,
                       *ll_best = nullptr;
    MkLayer *mk_layers = nullptr;
    int mk_head_off = 0;  // first workgroup of the persistent kernel's lm_head phase
    int mk_nsp = 1;       // attention spans per q head in the persistent kernel
    unsigned long long *mk_terms = nullptr;  // exact-order variant: epilogue operands per workgroup
};

namespace {

void *dalloc(k2t_model *m, size_t bytes) {
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, bytes ? bytes : 16);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        throw Error(K2T_E_NOMEM, std::string("hipMalloc failed: ") + hipGetErrorString(e));
    }
    m->allocs.push_back(p);
    return p;
}

void arg(bool ok, const char *msg) {
    if (!ok) throw Error(K2T_E_ARG, msg);
}

template <typename F>
int32_t mguard(F &&fn) {
    try {
        fn();
        return K2T_OK;
    } catch (const Error &e) {
        set_last_error(e.what());
        return e.code;
    } catch (const std::exception &e) {
        set_last_error(e.what());
        return K2T_E_INTERNAL;
    } catch (...) {
        set_last_error("unknown error");
        return K2T_E_INTERNAL;
    }
}

// real_llm.rs:9212-9232 build_rope_table: inv_freq in f64 -> f32, angle pos*freq in f32.
std::vector<float> rope_table(int hd, float theta, int max_seq) {
    const int half = hd / 2;
    std::vector<float> inv(half), t((size_t)max_seq * hd);
    for (int i = 0; i < half; i++) inv[i] = (float)(1.0 / pow((double)theta, (double)(2 * i) / (double)hd));
    for (int p = 0; p < max_seq; p++)
        for (int i = 0; i < half; i++) {
            const float a = (float)p * inv[i];
            t[(size_t)p * hd + i] = cosf(a);
            t[(size_t)p * hd + half + i] = sinf(a);
        }
    return t;
}

void ensure_batch(k2t_model *m, int n) {
    if (n <= m->max_batch) return;
    throw Error(K2T_E_ARG, "token batch larger than the model's max batch");
}

// The exact-order forward pass (k2t_model_set_exact): every operation in the x86
// reference's order (forward_token_sdot_megakernel's portable paths, real_llm.rs:6794-7403):
// RMSNorm with the sequential four-accumulator sum of squares, GEMVs with the in-order
// fmaf epilogue (the context's exact mode, set by the caller), q / k norm, RoPE from the
// host table and the K / V store per head, attention with sequential softmax and V sums,
// SwiGLU and softmax with the x86 build's exp.  Same device buffers as forward().
void forward_exact(k2t_model *m, int ntok, bool with_logits) {
    const k2t_model_config &c = m->cfg;
    hipStream_t st = m->stream;
    k2t_ctx *ctx = m->ctx;
    const int hd = c.head_dim, nq = c.n_heads, nkv = c.n_kv_heads, d = c.hidden, inter = c.intermediate;
    const float attn_scale = 1.0f / sqrtf((float)hd);
    if (m->embed_kind == K2T_EMBED_F32 || m->embed_kind == K2T_EMBED_BF16)
        launch_embed_rows(st, m->embed_rows, m->embed_kind == K2T_EMBED_BF16, m->tokens, ntok, c.hidden, m->hidden);
    else
        launch_embed(st, m->embed_kind == K2T_EMBED_NF4 ? m->embed_mat : m->head, m->tokens, ntok, m->hidden);
    auto norm_act = [&](const float *x, const float *w) {
        launch_inv_rms_x86(st, x, c.rms_eps, d, ntok, m->rms_x86);
        launch_act_quant(ctx, x, w, m->rms_x86, d, ntok, m->xq, m->xs, m->xsum);
    };
    for (int l = 0; l < c.n_layers; l++) {
        const auto &L = m->layers[l];
        norm_act(m->hidden, L.in_norm);
        launch_gemv_ex(ctx, L.qkv, m->xq, m->xs, m->xsum, ntok, m->qkv, (size_t)(nq + 2 * nkv) * hd, false);
        launch_qkv_post(st, m->qkv, L.bias, L.q_norm, L.k_norm, c.rms_eps, m->rope, m->pos_dev, nq, nkv, hd, ntok, l,
                        m->ring, m->kq, m->vq, m->ks, m->vs, true);
        launch_attention_exact(st, m->qkv, (nq + 2 * nkv) * hd, m->kq, m->vq, m->ks, m->vs, m->pos_dev, l, nq, nkv, hd,
                               m->ring, attn_scale, ntok, c.max_seq, m->attn_f);
        launch_act_quant(ctx, m->attn_f, nullptr, nullptr, nq * hd, ntok, m->xq, m->xs, m->xsum);
        launch_gemv_ex(ctx, L.o, m->xq, m->xs, m->xsum, ntok, m->hidden, d, true);
        if (L.has_moe) {
            // (the MoE feed-forward keeps its own order: router dot and combine as in
            // launch_moe_ffn)
            MoeWork ws = moe_work_carve(m->moe_ws, L.moe.bank, L.moe.top_k);
            ws.err = m->err_dev;
            for (int t = 0; t < ntok; t++) launch_moe_ffn(ctx, L.moe, m->hidden + (size_t)t * d, L.post_norm, c.rms_eps, ws);
            continue;
        }
        norm_act(m->hidden, L.post_norm);
        launch_gemv_ex(ctx, L.gu, m->xq, m->xs, m->xsum, ntok, m->gu, (size_t)2 * inter, false);
        launch_swiglu_act(st, ctx->signs, m->gu, inter, ntok, m->xq, m->xs, m->xsum, true);
        launch_gemv_ex(ctx, L.down, m->xq, m->xs, m->xsum, ntok, m->hidden, d, true);
    }
    if (with_logits) {
        const float *last = m->hidden + (size_t)(ntok - 1) * d;
        launch_inv_rms_x86(st, last, c.rms_eps, d, 1, m->rms_x86);
        launch_act_quant(ctx, last, m->final_norm, m->rms_x86, d, 1, m->xq, m->xs, m->xsum);
        launch_gemv_ex(ctx, m->head, m->xq, m->xs, m->xsum, 1, m->logits, c.vocab, false);
    }
    launch_advance_pos(st, m->pos_dev, ntok);
}

// Where the producer of the activation of `w` writes the tile-major copy: the model's
// tile buffers when that GEMV runs on the matrix cores, else nowhere.
ActTiles act_tiles_for(const k2t_model *m, const k2t_mat *w, int ntok) {
    return m->ctx->mfma == 1 && gemm_mfma_supported(w, ntok) ? ActTiles{m->xt, m->st, m->ut} : ActTiles{};
}

// One forward pass over `ntok` tokens already in m->tokens, positions pos..pos+ntok-1.
// Logits (of the last token) go to m->logits; the device position advances by ntok.
// ctx_bound: the position after the batch's last token when the host knows it (prefill;
// never a captured step, whose position moves between replays), else 0.
void forward(k2t_model *m, int ntok, bool with_logits, int ctx_bound = 0) {
    if (m->exact) {
        forward_exact(m, ntok, with_logits);
        return;
    }
    const k2t_model_config &c = m->cfg;
    hipStream_t st = m->stream;
    k2t_ctx *ctx = m->ctx;
    const int hd = c.head_dim, nq = c.n_heads, nkv = c.n_kv_heads, d = c.hidden, inter = c.intermediate;
    const float attn_scale = 1.0f / sqrtf((float)hd);
    const int nsplit = attn_max_splits(m->ring.window > 0 ? std::min(c.max_seq, m->ring.window) : c.max_seq);
    if (m->embed_kind == K2T_EMBED_F32 || m->embed_kind == K2T_EMBED_BF16)
        launch_embed_rows(st, m->embed_rows, m->embed_kind == K2T_EMBED_BF16, m->tokens, ntok, c.hidden, m->hidden);
    else
        launch_embed(st, m->embed_kind == K2T_EMBED_NF4 ? m->embed_mat : m->head, m->tokens, ntok, m->hidden);
    // One token: the RMSNorm / SwiGLU + FWHT + int8 activations are built inside the GEMVs
    // (each wave for its own chunks); batches use the standalone kernels.  Same codes.
    const bool fused = ntok == 1;
    for (int l = 0; l < c.n_layers; l++) {
        const auto &L = m->layers[l];
        bool qkv_posted = false;
        if (fused) {
            launch_gemv_fused(ctx, L.qkv, K2T_XS_RMSNORM, m->hidden, L.in_norm, c.rms_eps, m->qkv, false);
        } else {
            const ActTiles tq = act_tiles_for(m, L.qkv, ntok);
            launch_rmsnorm_act(st, ctx->signs, m->hidden, L.in_norm, c.rms_eps, d, ntok, m->xq, m->xs, m->xsum, tq);
            // head size 64 with producer tiles: qkv_post's work as the GEMV's epilogue
            qkv_posted = hd == 64 && tq.xt &&
                         launch_gemm_mfma_qkv(ctx, L.qkv, tq, ntok, m->qkv, (size_t)(nq + 2 * nkv) * hd,
                                              QkvPostDev{L.bias, L.q_norm, L.k_norm, m->rope, c.rms_eps, m->pos_dev,
                                                         nq, nkv, l, m->ring, m->kq, m->vq, m->ks, m->vs});
            if (!qkv_posted)
                launch_gemv_ex(ctx, L.qkv, m->xq, m->xs, m->xsum, ntok, m->qkv, (size_t)(nq + 2 * nkv) * hd, false,
                               0, tq);
        }
        // One token: qkv_post's work runs inside the attention kernel.  A batch stores every
        // token's K / V first (a later token of the batch attends to them).
        AttnPost post{};
        if (ntok == 1) {
            post = AttnPost{1, L.bias, L.q_norm, L.k_norm, m->rope, c.rms_eps};
        } else if (!qkv_posted) {
            launch_qkv_post(st, m->qkv, L.bias, L.q_norm, L.k_norm, c.rms_eps, m->rope, m->pos_dev, nq, nkv, hd, ntok,
                            l, m->ring, m->kq, m->vq, m->ks, m->vs, false);
        }
        const ActTiles to = act_tiles_for(m, L.o, ntok);  // (none for one token: the grouped kernel writes none)
        launch_attention(st, m->qkv, (nq + 2 * nkv) * hd, m->kq, m->vq, m->ks, m->vs, post, m->pos_dev, l, nq, nkv,
                         hd, m->ring, attn_scale, nsplit, ntok, m->attn_part, nullptr, m->xq, m->xs, m->xsum,
                         GqaWork{m->attn_words, m->attn_cnt, m->err_dev}, ctx_bound, to, ctx->mfma != 0);
        launch_gemv_ex(ctx, L.o, m->xq, m->xs, m->xsum, ntok, m->hidden, d, true, 0, to);
        if (L.has_moe) {
            // one token at a time: each token has its own routes (forward_layer_single)
            MoeWork ws = moe_work_carve(m->moe_ws, L.moe.bank, L.moe.top_k);
            ws.err = m->err_dev;  // timeouts surface through the model's error word
            for (int t = 0; t < ntok; t++) launch_moe_ffn(ctx, L.moe, m->hidden + (size_t)t * d, L.post_norm, c.rms_eps, ws);
        } else if (fused) {
            launch_gemv_fused(ctx, L.gu, K2T_XS_RMSNORM, m->hidden, L.post_norm, c.rms_eps, m->gu, false);
            launch_gemv_fused(ctx, L.down, K2T_XS_SWIGLU, m->gu, nullptr, 0.0f, m->hidden, true);
        } else {
            const ActTiles tg = act_tiles_for(m, L.gu, ntok), td = act_tiles_for(m, L.down, ntok);
            launch_rmsnorm_act(st, ctx->signs, m->hidden, L.post_norm, c.rms_eps, d, ntok, m->xq, m->xs, m->xsum, tg);
            // gate_up with the SwiGLU epilogue when both GEMVs take producer tiles (the
            // gate_up kernel reads only tg, so it may overwrite xq; its tiles go apart)
            if (tg.xt && td.xt &&
                launch_gemm_mfma_swiglu(ctx, L.gu, tg, ntok, m->xq, m->xs, m->xsum, m->dtiles)) {
                launch_gemv_ex(ctx, L.down, m->xq, m->xs, m->xsum, ntok, m->hidden, d, true, 0, m->dtiles);
            } else {
                launch_gemv_ex(ctx, L.gu, m->xq, m->xs, m->xsum, ntok, m->gu, (size_t)2 * inter, false, 0, tg);
                launch_swiglu_act(st, ctx->signs, m->gu, inter, ntok, m->xq, m->xs, m->xsum, false, td);
                launch_gemv_ex(ctx, L.down, m->xq, m->xs, m->xsum, ntok, m->hidden, d, true, 0, td);
            }
        }
    }
    if (with_logits) {
        const float *last = m->hidden + (size_t)(ntok - 1) * d;
        launch_gemv_fused(ctx, m->head, K2T_XS_RMSNORM, last, m->final_norm, c.rms_eps, m->logits, false);
    }
    launch_advance_pos(st, m->pos_dev, ntok);
}

void check_ready(k2t_model *m) {
    for (size_t l = 0; l < m->layers.size(); l++)
        arg(m->layers[l].qkv && m->layers[l].o && ((m->layers[l].gu && m->layers[l].down) || m->layers[l].has_moe),
            "a layer is not set");
    arg(m->head != nullptr, "lm_head is not set");
}

// The model's GEMVs run on its own stream with its epilogue mode; the context's settings
// are restored afterwards.
struct StreamSwap {
    k2t_ctx *ctx;
    hipStream_t saved;
    int saved_exact;
    StreamSwap(k2t_model *m) : ctx(m->ctx), saved(m->ctx->stream), saved_exact(m->ctx->exact) {
        ctx->stream = m->stream;
        ctx->exact = m->exact;
    }
    ~StreamSwap() {
        ctx->stream = saved;
        ctx->exact = saved_exact;
    }
};

// The persistent kernel needs the fast epilogue and one weight format for every matrix.
bool mk_format(const k2t_model *m, int &fmt, int &hp) {
    fmt = -1;
    hp = 0;
    if (!m->head) return false;
    for (const auto &L : m->layers) {
        if (!L.qkv || !L.o || !L.gu || !L.down) return false;
        for (const k2t_mat *x : {L.qkv, L.o, L.gu, L.down})
            if (!decode_mk_format(mat_dev(x, false), fmt, hp)) return false;
    }
    return decode_mk_format(mat_dev(m->head, false), fmt, hp);
}

bool use_persistent(const k2t_model *m) {
    int fmt, hp;
    // the sliding-window ring and the NF4 KV cache run on the per-operation path
    if (m->ring.window > 0 || m->ring.bits != 8) return false;
    for (const auto &L : m->layers)
        if (L.has_moe || L.q_norm || L.k_norm) return false;  // these run on the per-operation path
    return m->persistent && m->mk_ok && mk_format(m, fmt, hp);
}

// Destroys the captured decode graph after the stream has drained: a replay enqueued
// earlier may still be reading the executable graph's kernel arguments.
void drop_graph(k2t_model *m) {
    if (!m->graph) return;
    hip_check(hipSetDevice(m->ctx->device), "hipSetDevice");
    hip_check(hipStreamSynchronize(m->stream), "sync before graph destroy");
    (void)hipGraphExecDestroy(m->graph);
    m->graph = nullptr;
}

// Whether the decode step at position `pos` (attending pos + 1 positions) runs the
// persistent kernel.
bool persistent_at(const k2t_model *m, int pos) { return use_persistent(m) && pos + 1 <= kMkMaxContext; }

// Uploads the layer table of the persistent kernel (matrix views and launch shapes).
void upload_mk_layers(k2t_model *m) {
    int fmt, hp;
    mk_format(m, fmt, hp);
    const int nw = decode_mk_threads(hp) / 64;
    std::vector<MkLayer> h(m->layers.size());
    for (size_t l = 0; l < m->layers.size(); l++) {
        const auto &L = m->layers[l];
#ifdef K2T_MK_O_NSEG
        h[l].o = mat_dev(L.o, false, 0, nw, K2T_MK_O_NSEG);
#else
        h[l].o = mat_dev(L.o, false, 0, nw);
#endif
        h[l].gu = mat_dev(L.gu, true, 0, nw);
        h[l].down = mat_dev(L.down, false, 0, nw);
        // qkv follows down: fewer, longer qkv tasks where that lets the two phases use
        // disjoint workgroups (the phases' task lists are laid end to end).
        h[l].qkv = mat_dev(L.qkv, false, 0, nw);
        for (int cap = h[l].qkv.nseg / 2;
             cap >= 1 && mk_phase_tasks(h[l].qkv, nw) + mk_phase_tasks(h[l].down, nw) > m->ctx->num_cus; cap /= 2)
            h[l].qkv = mat_dev(L.qkv, false, cap, nw);
        h[l].in_norm = L.in_norm;
        h[l].post_norm = L.post_norm;
        h[l].bias = L.bias;
    }
    // phase task lists laid end to end over the grid (one workgroup per CU)
    const int nwg = m->ctx->num_cus;
    // attention spans per q head (the kernel uses fewer while the context is short): 2 in
    // the 512-thread kernel (1.7B nf4g128 decode at context 261-389: 1186 -> 1203 tok/s;
    // 3 spans 1144-1159), 4 in the 256-thread one (135M p55454 at 512-640: 1038 -> 1259
    // tok/s)
    const int max_spans = mk_max_spans(nw * 64);
    m->mk_nsp = std::max(1, std::min(max_spans, nwg / m->cfg.n_heads));
#ifdef K2T_MK_SPANS
    m->mk_nsp = std::max(1, std::min({K2T_MK_SPANS, max_spans, nwg / m->cfg.n_heads}));
#endif
    if (m->exact) m->mk_nsp = 1;  // one task per head: sequential softmax and V sums
    int cursor = 0;
    for (auto &x : h) {
        const int tasks[5] = {mk_phase_tasks(x.qkv, nw), m->cfg.n_heads * m->mk_nsp, mk_phase_tasks(x.o, nw),
                              mk_phase_tasks(x.gu, nw), mk_phase_tasks(x.down, nw)};
        for (int k = 0; k < 5; k++) {
            x.off[k] = cursor;
            cursor = (cursor + tasks[k]) % nwg;
        }
    }
    m->mk_head_off = cursor;
    hip_check(hipMemcpy(m->mk_layers, h.data(), h.size() * sizeof(MkLayer), hipMemcpyHostToDevice), "layer table");
}

// One decode step as a single persistent kernel, then the position / step advance.
void forward_mk(k2t_model *m) {
    const k2t_model_config &c = m->cfg;
    MkParams P{};
    P.layers = m->mk_layers;
    P.L = c.n_layers;
    int fmt, hp;
    mk_format(m, fmt, hp);
    const int nw = decode_mk_threads(hp) / 64;
    // lm_head: one wave per stripe (its whole K range, up to 4 fragments in flight), so a
    // workgroup takes 8 stripes per round and the phase runs in fewer rounds (1.7B: 2
    // instead of 6, 1427 -> 1438 tok/s; 135M 1504 -> 1516)
    P.head = mat_dev(m->head, false, 1, nw);
    P.head_off = m->mk_head_off;
    P.embed = mat_dev(m->embed_kind == K2T_EMBED_NF4 ? m->embed_mat : m->head, false, 0, nw);
    P.erows = m->embed_rows;
    P.ekind = m->embed_kind;
    P.final_norm = m->final_norm;
    P.d = c.hidden;
    P.nq = c.n_heads;
    P.nkv = c.n_kv_heads;
    P.hd = c.head_dim;
    P.inter = c.intermediate;
    P.vocab = c.vocab;
    P.max_seq = c.max_seq;
    P.kmax = std::max(c.hidden, c.intermediate);
    P.eps = c.rms_eps;
    P.attn_scale = 1.0f / sqrtf((float)c.head_dim);
    P.rope = m->rope;
    P.pos_dev = m->pos_dev;
    P.tokens = m->tokens;
    P.step_dev = m->step_dev;
    P.kq = m->kq;
    P.vq = m->vq;
    P.ks = m->ks;
    P.vs = m->vs;
    P.HA = m->ll_ha;
    P.HB = m->ll_hb;
    P.QKV = m->ll_qkv;
    P.OACT = m->ll_oact;
    P.APART = m->ll_apart;
    P.nsp = m->mk_nsp;
    P.GACT = m->ll_gact;
    P.rep = kMkRep;
    P.BEST = m->ll_best;
    P.logits = m->logits;
    P.signs = m->ctx->signs;
    P.err = m->err_dev;
    P.spin_limit = 1u << 22;
#ifdef K2T_MK_TRACE
    // measurement build: eager steps dump the phase trace to $K2T_MK_TRACE
    // (one buffer for the process, regrown when a model with more layers is traced)
    static unsigned long long *trace = nullptr;
    static size_t trace_cap = 0;
    const size_t ntr = (size_t)m->ctx->num_cus * (c.n_layers + 1) * 6 * 6;
    if (getenv("K2T_MK_TRACE") && !m->use_graph) {
        if (ntr > trace_cap) {
            hip_check(hipStreamSynchronize(m->stream), "sync");
            if (trace) hip_check(hipFree(trace), "trace free");
            trace = nullptr;
            trace_cap = 0;
            hip_check(hipMalloc(&trace, ntr * 8), "trace");
            trace_cap = ntr;
        }
        hip_check(hipMemset(trace, 0, ntr * 8), "trace clear");
        P.trace = trace;
    }
#endif
    // the kernel also writes the greedy next token and advances the position and step
    P.exterm = m->exact ? m->mk_terms : nullptr;
    launch_decode_mk(m->stream, P, fmt, hp, m->ctx->num_cus, m->mk_lds, m->exact != 0);
#ifdef K2T_MK_TRACE
    if (P.trace) {
        std::vector<unsigned long long> h(ntr);
        hip_check(hipStreamSynchronize(m->stream), "sync");
        hip_check(hipMemcpy(h.data(), trace, ntr * 8, hipMemcpyDeviceToHost), "trace copy");
        if (FILE *f = fopen(getenv("K2T_MK_TRACE"), "wb")) {
            fwrite(h.data(), 8, ntr, f);
            fclose(f);
        }
    }
#endif
}

// Raises the persistent kernel's dependency-timeout flag as an error (after a sync).
void check_mk_error(k2t_model *m) {
    if (!m->err_dev) return;
    int e = 0;
    hip_check(hipMemcpy(&e, m->err_dev, sizeof(int), hipMemcpyDeviceToHost), "error flag");
    if (e) {
        (void)hipMemset(m->err_dev, 0, sizeof(int));
        // a timed-out wait leaves the grouped-query attention's counters and words
        // inconsistent: start its epochs over
        (void)hipMemset(m->attn_cnt, 0, 2 * sizeof(unsigned int));
        (void)hipMemset(m->attn_words, 0,
                        (size_t)gqa_spans(m->cfg.max_seq) * m->cfg.n_heads * (2 + m->cfg.head_dim) *
                            sizeof(unsigned long long));
        throw Error(K2T_E_INTERNAL, e == 2   ? "MoE route selection: router wait timed out"
                                    : e == 3 ? "grouped-query attention: span wait timed out"
                                             : "persistent decode kernel: dependency wait timed out");
    }
}

// One decode step at host position m->pos (pk = persistent_at(m, m->pos)).
void decode_step(k2t_model *m, bool pk) {
    StreamSwap sw(m);
    // the context crossed kMkMaxContext: capture the other path (an earlier step of a
    // generate() loop may still be replaying the old graph; drop_graph waits for it)
    if (m->graph && m->graph_pk != pk) drop_graph(m);
    if (!m->use_graph) {
        if (pk) {
            upload_mk_layers(m);
            forward_mk(m);
        } else {
            forward(m, 1, true);
        }
        return;
    }
    if (!m->graph) {
        if (pk) upload_mk_layers(m);
        hipGraph_t g = nullptr;
        hip_check(hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal), "begin capture");
        try {
            if (pk) forward_mk(m);
            else forward(m, 1, true);
        } catch (...) {
            (void)hipStreamEndCapture(m->stream, &g);
            if (g) (void)hipGraphDestroy(g);
            throw;
        }
        hip_check(hipStreamEndCapture(m->stream, &g), "end capture");
        hipError_t e = hipGraphInstantiate(&m->graph, g, nullptr, nullptr, 0);
        (void)hipGraphDestroy(g);
        hip_check(e, "graph instantiate");
        m->graph_pk = pk;
    }
    hip_check(hipGraphLaunch(m->graph, m->stream), "graph launch");
}

}  // namespace

namespace k2t {
void model_adopt(k2t_model *m, k2t_mat *mat) { m->owned.push_back(mat); }
}  // namespace k2t

extern "C" {

int32_t k2t_model_create(k2t_ctx *ctx, const k2t_model_config *cfg, int32_t max_batch, k2t_model **out) {
    return mguard([&] {
        arg(ctx && cfg && out, "NULL argument");
        *out = nullptr;
        const k2t_model_config &c = *cfg;
        arg(c.n_layers > 0 && c.hidden > 0 && c.n_heads > 0 && c.n_kv_heads > 0 && c.intermediate > 0 && c.vocab > 0,
            "non-positive model dimension");
        arg(c.head_dim == 64 || c.head_dim == 128, "head_dim must be 64 or 128 (Hadamard KV cache)");
        arg(c.n_heads % c.n_kv_heads == 0, "n_heads must be a multiple of n_kv_heads");
        arg(c.n_heads * c.head_dim <= 32768, "q_dim too large");
        arg(c.hidden % 64 == 0 && c.intermediate % 64 == 0, "hidden and intermediate must be multiples of 64");
        arg(c.max_seq > 0 && c.max_seq <= 1 << 20, "max_seq out of range");
        arg(max_batch >= 1 && max_batch <= 4096, "max_batch out of range");
        hip_check(hipSetDevice(ctx->device), "hipSetDevice");
        k2t_model *m = new k2t_model();
        try {
            m->ctx = ctx;
            m->cfg = c;
            m->ring = KvRing{c.max_seq, 0, 0, 0, 8};
            m->max_batch = max_batch;
            m->layers.resize(c.n_layers);
            hip_check(hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking), "stream create");
            const size_t slots = (size_t)c.n_layers * c.n_kv_heads * c.max_seq;
            m->kq = (int8_t *)dalloc(m, slots * c.head_dim);
            m->vq = (int8_t *)dalloc(m, slots * c.head_dim);
            m->ks = (float *)dalloc(m, slots * sizeof(float));
            m->vs = (float *)dalloc(m, slots * sizeof(float));
            auto rt = rope_table(c.head_dim, c.rope_theta, c.max_seq);
            m->rope = (float *)dalloc(m, rt.size() * sizeof(float));
            hip_check(hipMemcpy(m->rope, rt.data(), rt.size() * sizeof(float), hipMemcpyHostToDevice), "rope upload");
            m->pos_dev = (int *)dalloc(m, (size_t)(max_batch + 1) * sizeof(int));
            m->tokens = m->pos_dev + 1;
            hip_check(hipMemset(m->pos_dev, 0, (size_t)(max_batch + 1) * sizeof(int)), "pos clear");
            const size_t qkv_w = (size_t)(c.n_heads + 2 * c.n_kv_heads) * c.head_dim;
            const size_t kmax = std::max({c.hidden, c.intermediate, c.n_heads * c.head_dim});
            m->hidden = (float *)dalloc(m, (size_t)max_batch * c.hidden * sizeof(float));
            m->qkv = (float *)dalloc(m, (size_t)max_batch * qkv_w * sizeof(float));
            m->gu = (float *)dalloc(m, (size_t)max_batch * 2 * c.intermediate * sizeof(float));
            m->logits = (float *)dalloc(m, (size_t)c.vocab * sizeof(float));
            m->attn_part = (float *)dalloc(
                m, (size_t)max_batch * c.n_heads * attn_max_splits(c.max_seq) * (2 + c.head_dim) * sizeof(float));
            // grouped-query attention: span words (one token) and the epoch / done counters,
            // zeroed once (epochs only grow, so no launch clears them)
            const size_t gw = (size_t)gqa_spans(c.max_seq) * c.n_heads * (2 + c.head_dim);
            m->attn_words = (unsigned long long *)dalloc(m, gw * sizeof(unsigned long long));
            hip_check(hipMemset(m->attn_words, 0, gw * sizeof(unsigned long long)), "span words clear");
            m->attn_cnt = (unsigned int *)dalloc(m, 2 * sizeof(unsigned int));
            hip_check(hipMemset(m->attn_cnt, 0, 2 * sizeof(unsigned int)), "counter clear");
            m->rms_x86 = (float *)dalloc(m, (size_t)max_batch * sizeof(float));
            m->attn_f = (float *)dalloc(m, (size_t)max_batch * c.n_heads * c.head_dim * sizeof(float));
            m->xq = (int8_t *)dalloc(m, (size_t)max_batch * kmax);
            m->xs = (float *)dalloc(m, (size_t)max_batch * (kmax / 64) * sizeof(float));
            m->xsum = (int32_t *)dalloc(m, (size_t)max_batch * (kmax / 64) * sizeof(int32_t));
            const size_t ntile = (size_t)((max_batch + 15) / 16) * (kmax / 64);
            m->xt = (int8_t *)dalloc(m, ntile * 1024);
            m->st = (float *)dalloc(m, ntile * 16 * sizeof(float));
            m->ut = (int32_t *)dalloc(m, ntile * 16 * sizeof(int32_t));
            m->dtiles.xt = (int8_t *)dalloc(m, ntile * 1024);
            m->dtiles.st = (float *)dalloc(m, ntile * 16 * sizeof(float));
            m->dtiles.ut = (int32_t *)dalloc(m, ntile * 16 * sizeof(int32_t));
            // persistent decode kernel state
            // the persistent kernel's phases assume the megakernel shape q_dim == hidden
            m->mk_ok = decode_mk_supported(c, ctx->num_cus) && c.n_heads * c.head_dim == c.hidden;
            m->mk_lds = decode_mk_lds_bytes(c);
            m->step_dev = (uint32_t *)dalloc(m, 16);
            m->err_dev = (int *)m->step_dev + 1;
            const uint32_t one[4] = {1u, 0u, 0u, 0u};
            hip_check(hipMemcpy(m->step_dev, one, sizeof(one), hipMemcpyHostToDevice), "step init");
            // HA, HB, OACT and GACT in kMkRep copies, QKV and BEST once
            const size_t oact = (size_t)(c.n_heads * c.head_dim / 64) * 18, gact = (size_t)(c.intermediate / 64) * 18;
            const size_t apart = (size_t)c.n_heads * kMkSpans * (2 + c.head_dim);
            const size_t words =
                kMkRep * (2 * (size_t)c.hidden + oact + gact) + qkv_w + 2 * (size_t)ctx->num_cus + apart;
            m->ll_ha = (unsigned long long *)dalloc(m, words * 8);
            hip_check(hipMemset(m->ll_ha, 0, words * 8), "hand-off clear");
            m->ll_hb = m->ll_ha + kMkRep * (size_t)c.hidden;
            m->ll_oact = m->ll_hb + kMkRep * (size_t)c.hidden;
            m->ll_gact = m->ll_oact + kMkRep * oact;
            m->ll_qkv = m->ll_gact + kMkRep * gact;
            m->ll_best = m->ll_qkv + qkv_w;
            m->ll_apart = m->ll_best + 2 * (size_t)ctx->num_cus;
            m->mk_layers = (MkLayer *)dalloc(m, (size_t)c.n_layers * sizeof(MkLayer));
        } catch (...) {
            k2t_model_destroy(m);
            throw;
        }
        *out = m;
    });
}

void k2t_model_destroy(k2t_model *m) {
    if (!m) return;
    (void)hipSetDevice(m->ctx ? m->ctx->device : 0);
    if (m->stream) (void)hipStreamSynchronize(m->stream);
    if (m->graph) (void)hipGraphExecDestroy(m->graph);
    for (void *p : m->allocs) (void)hipFree(p);
    for (k2t_mat *x : m->owned) k2t_mat_destroy(x);
    if (m->stream) (void)hipStreamDestroy(m->stream);
    delete m;
}

int32_t k2t_model_set_layer(k2t_model *m, int32_t layer, const k2t_mat *qkv, const k2t_mat *o,
                            const k2t_mat *gate_up, const k2t_mat *down, const float *in_norm,
                            const float *post_norm, const float *qkv_bias) {
    return mguard([&] {
        arg(m != nullptr, "model is NULL");
        arg(layer >= 0 && layer < m->cfg.n_layers, "layer out of range");
        arg(qkv && o && in_norm && post_norm, "NULL argument");
        arg((gate_up == nullptr) == (down == nullptr), "gate_up and down must both be set, or both NULL (MoE layer)");
        const k2t_model_config &c = m->cfg;
        const int qkv_rows = (c.n_heads + 2 * c.n_kv_heads) * c.head_dim;
        arg(qkv->rows == qkv_rows && qkv->cols == c.hidden, "qkv shape mismatch");
        arg(o->rows == c.hidden && o->cols == c.n_heads * c.head_dim, "o_proj shape mismatch");
        if (gate_up) {
            arg(gate_up->rows == 2 * c.intermediate && gate_up->cols == c.hidden, "gate_up shape mismatch");
            arg(down->rows == c.hidden && down->cols == c.intermediate, "down_proj shape mismatch");
            arg(gate_up->ctx == m->ctx && down->ctx == m->ctx, "matrix of another context");
        }
        for (const k2t_mat *x : {qkv, o}) arg(x->ctx == m->ctx, "matrix of another context");
        auto &L = m->layers[layer];
        hip_check(hipSetDevice(m->ctx->device), "hipSetDevice");
        if (!L.in_norm) L.in_norm = (float *)dalloc(m, c.hidden * sizeof(float));
        if (!L.post_norm) L.post_norm = (float *)dalloc(m, c.hidden * sizeof(float));
        hip_check(hipMemcpy(L.in_norm, in_norm, c.hidden * sizeof(float), hipMemcpyHostToDevice), "norm upload");
        hip_check(hipMemcpy(L.post_norm, post_norm, c.hidden * sizeof(float), hipMemcpyHostToDevice), "norm upload");
        if (qkv_bias) {
            if (!L.bias) L.bias = (float *)dalloc(m, (size_t)qkv_rows * sizeof(float));
            hip_check(hipMemcpy(L.bias, qkv_bias, (size_t)qkv_rows * sizeof(float), hipMemcpyHostToDevice),
                      "bias upload");
        } else {
            L.bias = nullptr;
        }
        L.qkv = qkv;
        L.o = o;
        L.gu = gate_up;
        L.down = down;
        if (gate_up) L.has_moe = false;
        drop_graph(m);
    });
}

int32_t k2t_model_set_head(k2t_model *m, const k2t_mat *lm_head, const float *final_norm) {
    return mguard([&] {
        arg(m && lm_head && final_norm, "NULL argument");
        arg(lm_head->rows == m->cfg.vocab && lm_head->cols == m->cfg.hidden, "lm_head shape mismatch");
        arg(m->embed_kind != K2T_EMBED_TIED || lm_head->fmt != K2T_FMT_NF || lm_head->bits == 4,
            "a tied lm_head (the embedding table) must be NF4 or bit planes");
        arg(lm_head->ctx == m->ctx, "matrix of another context");
        hip_check(hipSetDevice(m->ctx->device), "hipSetDevice");
        if (!m->final_norm) m->final_norm = (float *)dalloc(m, m->cfg.hidden * sizeof(float));
        hip_check(hipMemcpy(m->final_norm, final_norm, m->cfg.hidden * sizeof(float), hipMemcpyHostToDevice),
                  "norm upload");
        m->head = lm_head;
        drop_graph(m);
    });
}

int32_t k2t_model_set_qk_norm(k2t_model *m, int32_t layer, const float *q_norm, const float *k_norm) {
    return mguard([&] {
        arg(m != nullptr, "model is NULL");
        arg(layer >= 0 && layer < m->cfg.n_layers, "layer out of range");
        auto &L = m->layers[layer];
        const size_t hd = (size_t)m->cfg.head_dim;
        hip_check(hipSetDevice(m->ctx->device), "hipSetDevice");
        auto put = [&](float *&dst, const float *src) {
            if (!src) {
                dst = nullptr;
                return;
            }
            if (!dst) dst = (float *)dalloc(m, hd * sizeof(float));
            hip_check(hipMemcpy(dst, src, hd * sizeof(float), hipMemcpyHostToDevice), "qk norm upload");
        };
        put(L.q_norm, q_norm);
        put(L.k_norm, k_norm);
        drop_graph(m);
    });
}

int32_t k2t_model_set_moe(k2t_model *m, int32_t layer, const k2t_experts *bank, int32_t shard_layer,
                          const float *router_w, const float *router_bias, int32_t top_k, int32_t norm_topk_prob,
                          int32_t scoring) {
    return mguard([&] {
        arg(m && router_w, "NULL argument");
        arg(layer >= 0 && layer < m->cfg.n_layers, "layer out of range");
        check_moe_args(bank, shard_layer, top_k, scoring);
        arg(bank->ctx == m->ctx, "expert bank of another context");
        arg(bank->hdr.d_model == m->cfg.hidden, "expert d_model does not match the model's hidden size");
        auto &L = m->layers[layer];
        arg(L.qkv != nullptr, "set the layer's attention first (k2t_model_set_layer with NULL gate_up / down)");
        arg(L.gu == nullptr, "the layer has a dense feed-forward");
        hip_check(hipSetDevice(m->ctx->device), "hipSetDevice");
        const size_t E = (size_t)bank->hdr.experts_per_layer, d = (size_t)m->cfg.hidden;
        float *rw = (float *)dalloc(m, E * d * sizeof(float));
        hip_check(hipMemcpy(rw, router_w, E * d * sizeof(float), hipMemcpyHostToDevice), "router upload");
        float *rb = nullptr;
        if (router_bias) {
            rb = (float *)dalloc(m, E * sizeof(float));
            hip_check(hipMemcpy(rb, router_bias, E * sizeof(float), hipMemcpyHostToDevice), "router upload");
        }
        const size_t need = moe_work_floats(bank, top_k);
        if (need > m->moe_ws_floats) {
            m->moe_ws = (float *)dalloc(m, need * sizeof(float));
            m->moe_ws_floats = need;
            // the route hand-off words and the call counter start at epoch 0
            hip_check(hipMemset(m->moe_ws, 0, need * sizeof(float)), "moe workspace clear");
        }
        L.moe = MoeLayer{bank, shard_layer, rw, rb, top_k, norm_topk_prob ? 1 : 0, scoring};
        L.has_moe = true;
        drop_graph(m);
    });
}

int32_t k2t_model_set_moe_shared(k2t_model *m, int32_t layer, const k2t_mat *gate_up, const k2t_mat *down,
                                 const float *gate_weight) {
    return mguard([&] {
        arg(m != nullptr, "model is NULL");
        arg(layer >= 0 && layer < m->cfg.n_layers, "layer out of range");
        auto &L = m->layers[layer];
        arg(L.has_moe, "set the layer's MoE first (k2t_model_set_moe)");
        drop_graph(m);
        if (!gate_up) {
            L.moe.sh_gu = L.moe.sh_dn = nullptr;
            L.moe.sh_gate = nullptr;
            return;
        }
        const int d = m->cfg.hidden;
        arg(down != nullptr, "down is NULL");
        arg(gate_up->ctx == m->ctx && down->ctx == m->ctx, "matrix of another context");
        arg(gate_up->fmt == K2T_FMT_NF && down->fmt == K2T_FMT_NF, "the shared expert's matrices must be NF");
        arg(gate_up->cols == d && gate_up->rows % 128 == 0, "shared gate_up must be [2*inter][hidden], inter % 64 == 0");
        const int inter = gate_up->rows / 2;
        arg(down->rows == d && down->cols == inter, "shared down must be [hidden][inter]");
        hip_check(hipSetDevice(m->ctx->device), "hipSetDevice");
        // [2 * inter gate_up | d output | 64 (gate scale) | exact mode: inter int8 codes,
        //  inter / 64 scales and sums of the down activation]
        L.moe.sh_buf = (float *)dalloc(m, ((size_t)2 * inter + d + 64 + inter / 4 + 2 * (inter / 64) + 64) * sizeof(float));
        float *g = nullptr;
        if (gate_weight) {
            g = (float *)dalloc(m, (size_t)d * sizeof(float));
            hip_check(hipMemcpy(g, gate_weight, (size_t)d * sizeof(float), hipMemcpyHostToDevice), "gate upload");
        }
        L.moe.sh_gu = gate_up;
        L.moe.sh_dn = down;
        L.moe.sh_gate = g;
    });
}

int32_t k2t_model_set_embedding(k2t_model *m, int32_t kind, const void *rows, const k2t_mat *nf4) {
    return mguard([&] {
        arg(m != nullptr, "model is NULL");
        const k2t_model_config &c = m->cfg;
        hip_check(hipSetDevice(m->ctx->device), "hipSetDevice");
        if (kind == K2T_EMBED_TIED) {
            arg(!m->head || m->head->fmt != K2T_FMT_NF || m->head->bits == 4,
                "a tied lm_head (the embedding table) must be NF4 or bit planes");
        } else if (kind == K2T_EMBED_F32 || kind == K2T_EMBED_BF16) {
            arg(rows != nullptr, "embedding rows are NULL");
            const size_t bytes = (size_t)c.vocab * c.hidden * (kind == K2T_EMBED_F32 ? 4 : 2);
            void *d = dalloc(m, bytes);
            hip_check(hipMemcpy(d, rows, bytes, hipMemcpyHostToDevice), "embedding upload");
            m->embed_rows = d;
        } else if (kind == K2T_EMBED_NF4) {
            arg(nf4 != nullptr, "embedding matrix is NULL");
            arg(nf4->ctx == m->ctx, "matrix of another context");
            arg(nf4->fmt == K2T_FMT_NF && nf4->bits == 4, "the embedding matrix must be NF4");
            arg(nf4->rows == c.vocab && nf4->cols == c.hidden, "embedding matrix shape mismatch");
            m->embed_mat = nf4;
        } else {
            arg(false, "unknown embedding kind");
        }
        m->embed_kind = kind;
        drop_graph(m);
    });
}

int32_t k2t_model_set_graph(k2t_model *m, int32_t enable) {
    return mguard([&] {
        arg(m != nullptr, "model is NULL");
        m->use_graph = enable != 0;
    });
}

int32_t k2t_model_stream(const k2t_model *m, void **hip_stream) {
    return mguard([&] {
        arg(m && hip_stream, "NULL argument");
        *hip_stream = (void *)m->stream;
    });
}

int32_t k2t_model_set_exact(k2t_model *m, int32_t exact) {
    return mguard([&] {
        arg(m != nullptr, "model is NULL");
        drop_graph(m);
        if (exact && m->mk_ok && !m->mk_terms) {
            // the exact-order persistent kernel's per-workgroup epilogue operands: one GEMV
            // round (kMkTermRows rows) of the widest input
            const k2t_model_config &c = m->cfg;
            const size_t nc = (size_t)std::max(c.hidden, c.intermediate) / 64;
            hip_check(hipSetDevice(m->ctx->device), "hipSetDevice");
            m->mk_terms = (unsigned long long *)dalloc(
                m, (size_t)m->ctx->num_cus * kMkTermRows * nc * sizeof(unsigned long long));
        }
        m->exact = exact ? 1 : 0;
    });
}

int32_t k2t_model_set_kv_window(k2t_model *m, int32_t window, int32_t sink_tokens) {
    return mguard([&] {
        arg(m != nullptr, "model is NULL");
        arg(window >= 0 && sink_tokens >= 0, "window and sink_tokens must be >= 0");
        const k2t_model_config &c = m->cfg;
        hip_check(hipSetDevice(m->ctx->device), "hipSetDevice");
        hip_check(hipStreamSynchronize(m->stream), "sync");
        // QuantizedKvCache::new_with_opts (real_llm.rs:1235-1257): a window of at least 8
        // that leaves room for the ring's 512-slot batch slack; otherwise the full cache.
        constexpr int kRingSlack = 512;
        if (window >= 8 && window + kRingSlack < c.max_seq) {
            const int s = std::min(sink_tokens, window / 2);
            const int rl = (window - s) + kRingSlack;
            m->ring = KvRing{s + rl, window, s, rl, m->ring.bits};
        } else {
            m->ring = KvRing{c.max_seq, 0, 0, 0, m->ring.bits};
        }
        // set_kv_sliding_window starts a new context (real_llm.rs:1764-1790)
        hip_check(hipMemset(m->pos_dev, 0, sizeof(int)), "pos reset");
        m->pos = 0;
        drop_graph(m);
    });
}

int32_t k2t_model_set_kv_bits(k2t_model *m, int32_t bits) {
    return mguard([&] {
        arg(m != nullptr, "model is NULL");
        arg(bits == 4 || bits == 8, "KV bits must be 4 or 8");
        hip_check(hipSetDevice(m->ctx->device), "hipSetDevice");
        hip_check(hipStreamSynchronize(m->stream), "sync");
        // set_kv_bits (real_llm.rs:1732-1752): a new cache, position 0.  The NF4 nibbles
        // and BF16 block scales fit in the int8 buffers (hd/2 <= hd bytes, hd/64 BF16 <= one f32).
        m->ring.bits = bits;
        hip_check(hipMemset(m->pos_dev, 0, sizeof(int)), "pos reset");
        m->pos = 0;
        drop_graph(m);
    });
}

int32_t k2t_model_kv_bits(const k2t_model *m, int32_t *bits) {
    return mguard([&] {
        arg(m && bits, "NULL argument");
        *bits = m->ring.bits;
    });
}

int32_t k2t_model_kv_window(const k2t_model *m, int32_t *window, int32_t *sink_tokens) {
    return mguard([&] {
        arg(m && window && sink_tokens, "NULL argument");
        *window = m->ring.window;
        *sink_tokens = m->ring.sinks;
    });
}

int32_t k2t_model_kv_synthetic(k2t_model *m, int32_t n_pos, uint64_t seed) {
    return mguard([&] {
        arg(m != nullptr, "model is NULL");
        arg(n_pos >= 0 && n_pos < m->cfg.max_seq, "n_pos must be in [0, max_seq)");
        const k2t_model_config &c = m->cfg;
        hip_check(hipSetDevice(m->ctx->device), "hipSetDevice");
        hip_check(hipStreamSynchronize(m->stream), "sync");
        launch_kv_synthetic(m->stream, m->kq, m->vq, m->ks, m->vs, c.n_layers * c.n_kv_heads, m->ring.cap,
                            std::min(n_pos, m->ring.cap), c.head_dim, m->ring.bits, seed);
        hip_check(hipMemcpyAsync(m->pos_dev, &n_pos, sizeof(int), hipMemcpyHostToDevice, m->stream), "pos set");
        hip_check(hipStreamSynchronize(m->stream), "sync");
        m->pos = n_pos;
    });
}

int32_t k2t_model_reset(k2t_model *m) {
    return mguard([&] {
        arg(m != nullptr, "model is NULL");
        hip_check(hipSetDevice(m->ctx->device), "hipSetDevice");
        hip_check(hipStreamSynchronize(m->stream), "sync");
        hip_check(hipMemset(m->pos_dev, 0, sizeof(int)), "pos reset");
        m->pos = 0;
    });
}

int32_t k2t_model_position(const k2t_model *m, int32_t *pos) {
    return mguard([&] {
        arg(m && pos, "NULL argument");
        *pos = m->pos;
    });
}

int32_t k2t_model_decode(k2t_model *m, int32_t token, float *logits_host) {
    return mguard([&] {
        arg(m != nullptr, "model is NULL");
        check_ready(m);
        arg(token >= 0 && token < m->cfg.vocab, "token out of range");
        arg(m->pos < m->cfg.max_seq, "context full (max_seq reached)");
        hip_check(hipSetDevice(m->ctx->device), "hipSetDevice");
        hip_check(hipMemcpyAsync(m->tokens, &token, sizeof(int), hipMemcpyHostToDevice, m->stream), "token upload");
        decode_step(m, persistent_at(m, m->pos));
        m->pos += 1;
        if (logits_host) {
            hip_check(hipMemcpyAsync(logits_host, m->logits, (size_t)m->cfg.vocab * sizeof(float),
                                     hipMemcpyDeviceToHost, m->stream),
                      "logits download");
            hip_check(hipStreamSynchronize(m->stream), "sync");
            check_mk_error(m);
        }
    });
}

int32_t k2t_model_prefill(k2t_model *m, const int32_t *tokens, int32_t n, float *logits_host) {
    return mguard([&] {
        arg(m && tokens, "NULL argument");
        check_ready(m);
        arg(n >= 1, "empty prompt");
        arg(m->pos + n <= m->cfg.max_seq, "prompt exceeds max_seq");
        for (int i = 0; i < n; i++) arg(tokens[i] >= 0 && tokens[i] < m->cfg.vocab, "token out of range");
        hip_check(hipSetDevice(m->ctx->device), "hipSetDevice");
        StreamSwap sw(m);
        // A batch stores all its K/V before any of its tokens attends.  With the window ring
        // that is safe for up to the ring's batch slack (512 slots) of tokens: beyond it a
        // later token would overwrite a slot an earlier one still reads.
        const int chunk = m->ring.window > 0 ? std::min(m->max_batch, 512) : m->max_batch;
        for (int i0 = 0; i0 < n; i0 += chunk) {
            const int nb = std::min(chunk, n - i0);
            hip_check(hipMemcpyAsync(m->tokens, tokens + i0, nb * sizeof(int), hipMemcpyHostToDevice, m->stream),
                      "token upload");
            forward(m, nb, i0 + nb == n, m->pos + i0 + nb);
            // the token buffer is reused by the next chunk: wait for this one
            hip_check(hipStreamSynchronize(m->stream), "sync");
        }
        m->pos += n;
        if (logits_host) {
            hip_check(hipMemcpyAsync(logits_host, m->logits, (size_t)m->cfg.vocab * sizeof(float),
                                     hipMemcpyDeviceToHost, m->stream),
                      "logits download");
            hip_check(hipStreamSynchronize(m->stream), "sync");
        }
    });
}

int32_t k2t_model_generate(k2t_model *m, int32_t first_token, int32_t n_steps, int32_t *tokens_out) {
    return mguard([&] {
        arg(m != nullptr, "model is NULL");
        check_ready(m);
        arg(n_steps >= 0, "n_steps < 0");
        arg(first_token >= 0 && first_token < m->cfg.vocab, "token out of range");
        arg(m->pos + n_steps <= m->cfg.max_seq, "generation exceeds max_seq");
        hip_check(hipSetDevice(m->ctx->device), "hipSetDevice");
        hip_check(hipMemcpyAsync(m->tokens, &first_token, sizeof(int), hipMemcpyHostToDevice, m->stream),
                  "token upload");
        std::vector<int> host;
        int *dev_out = nullptr;
        if (tokens_out && n_steps > 0) dev_out = (int *)dalloc(m, (size_t)n_steps * sizeof(int));
        for (int i = 0; i < n_steps; i++) {
            const bool pk = persistent_at(m, m->pos + i);
            decode_step(m, pk);
            // greedy: the next input token is argmax of these logits, written on the device
            // (by the persistent kernel itself, or by argmax_kernel after the per-op step)
            if (!pk) launch_argmax(m->stream, m->logits, m->cfg.vocab, m->tokens);
            if (dev_out)
                hip_check(hipMemcpyAsync(dev_out + i, m->tokens, sizeof(int), hipMemcpyDeviceToDevice, m->stream),
                          "token copy");
        }
        m->pos += n_steps;
        if (dev_out) {
            hip_check(hipMemcpyAsync(tokens_out, dev_out, (size_t)n_steps * sizeof(int), hipMemcpyDeviceToHost,
                                     m->stream),
                      "tokens download");
        }
        hip_check(hipStreamSynchronize(m->stream), "sync");
        if (dev_out) {
            (void)hipFree(dev_out);
            m->allocs.pop_back();
        }
        check_mk_error(m);
    });
}

int32_t k2t_model_logits(k2t_model *m, const float **d_logits) {
    return mguard([&] {
        arg(m && d_logits, "NULL argument");
        *d_logits = m->logits;
    });
}

int32_t k2t_model_sync(k2t_model *m) {
    return mguard([&] {
        arg(m != nullptr, "model is NULL");
        hip_check(hipSetDevice(m->ctx->device), "hipSetDevice");
        hip_check(hipStreamSynchronize(m->stream), "sync");
        check_mk_error(m);
    });
}

int32_t k2t_model_set_persistent(k2t_model *m, int32_t enable) {
    return mguard([&] {
        arg(m != nullptr, "model is NULL");
        arg(enable >= 0 && enable <= 2, "persistent mode must be 0, 1 or 2");
        m->persistent = enable;
        drop_graph(m);
    });
}

int32_t k2t_model_persistent_active(const k2t_model *m, int32_t *active) {
    return mguard([&] {
        arg(m && active, "NULL argument");
        *active = persistent_at(m, m->pos) ? 1 : 0;
    });
}

int32_t k2t_kv_store(k2t_ctx *ctx, int32_t bits, const float *d_heads, int32_t n, int32_t head_dim, void *d_q,
                     void *d_scales) {
    return mguard([&] {
        arg(ctx && d_heads && d_q && d_scales, "NULL argument");
        arg(bits == 4 || bits == 8, "KV bits must be 4 or 8");
        arg(head_dim == 64 || head_dim == 128, "head_dim must be 64 or 128");
        arg(n >= 0 && n <= (1 << 24), "n out of range");
        if (n == 0) return;
        hip_check(hipSetDevice(ctx->device), "hipSetDevice");
        launch_kv_store(ctx->stream, d_heads, n, head_dim, bits, (int8_t *)d_q, (float *)d_scales);
    });
}

namespace {
// k2t_attn_decode's body.  noalloc: the partials and the position live in the static
// `scratch` array (no allocation, no host-to-device copy); otherwise in the context's
// scratch, grown on demand.
void attn_decode_impl(k2t_ctx *ctx, int32_t bits, const float *d_q, int32_t n_heads, int32_t n_kv_heads,
                      int32_t head_dim, const void *d_kq, const void *d_ks, const void *d_vq, const void *d_vs,
                      int32_t cap, int32_t seq, int32_t window, int32_t sink_tokens, float attn_scale, float *d_out,
                      bool noalloc) {
    arg(ctx && d_q && d_kq && d_ks && d_vq && d_vs && d_out, "NULL argument");
    arg(bits == 4 || bits == 8, "KV bits must be 4 or 8");
    arg(head_dim == 64 || head_dim == 128, "head_dim must be 64 or 128");
    arg(n_heads > 0 && n_kv_heads > 0 && n_heads % n_kv_heads == 0, "n_heads must be a multiple of n_kv_heads");
    arg(seq >= 1 && cap >= 1 && seq <= (1 << 24), "seq / cap out of range");
    KvRing kr{cap, 0, 0, 0, bits};
    if (window > 0) {
        arg(window >= 8 && sink_tokens >= 0 && sink_tokens <= window / 2, "window >= 8 and sinks <= window / 2");
        arg(cap > window, "a windowed cache needs cap > window");
        kr = KvRing{cap, window, sink_tokens, cap - sink_tokens, bits};
    } else {
        arg(seq <= cap, "seq exceeds the cache");
    }
    const int act = window > 0 ? std::min(seq, window) : seq;
    const int nsplit = attn_max_splits(act);
    hip_check(hipSetDevice(ctx->device), "hipSetDevice");
    // grouped queries at long context: the model's grouped-query kernel (each K / V tile
    // read once for the G q heads of its KV head), with span words that persist across
    // calls (context workspace, or the fixed no-alloc region)
    GqaWork gq{};
    if (gqa_eligible(nsplit, 1, n_heads, n_kv_heads, head_dim, kr)) {
        const size_t words = gqa_words(cap, n_heads, head_dim, 1);
        if (noalloc) {
            if (words > kNoAllocGqaWords)
                throw Error(K2T_E_ARG, "k2t_attn_decode_noalloc: ceil(cap / 128) * n_heads * (head_dim + 2) = " +
                                           std::to_string(words) + " span words exceeds its fixed scratch region of " +
                                           std::to_string(kNoAllocGqaWords));
            gq = noalloc_gqa(ctx->device);
        } else {
            gq = ctx_gqa(ctx, words);
        }
    }
    const size_t part = (size_t)n_heads * nsplit * (2 + head_dim);
    float *pp;
    if (noalloc) {
        if (part + 64 > kNoAllocScratchFloats)
            throw Error(K2T_E_ARG, "k2t_attn_decode_noalloc: n_heads * ceil(positions / 256) * (head_dim + 2) = " +
                                       std::to_string(part) + " floats exceeds its fixed scratch of " +
                                       std::to_string(kNoAllocScratchFloats - 64) + " floats");
        pp = noalloc_scratch(ctx->device);
    } else {
        ensure_scratch(ctx, part + 64);
        pp = ctx->scratch;
    }
    int *pos = reinterpret_cast<int *>(pp + part);
    const int p0 = seq - 1;
    if (noalloc) {
        hipLaunchKernelGGL(store_int_kernel, dim3(1), dim3(64), 0, ctx->stream, pos, p0);
        hip_check(hipGetLastError(), "position store launch");
    } else {
        hip_check(hipMemcpyAsync(pos, &p0, sizeof(int), hipMemcpyHostToDevice, ctx->stream), "pos upload");
    }
    // read-only on the cache (no post stage: the caller's queries are final)
    launch_attention(ctx->stream, d_q, n_heads * head_dim, (int8_t *)d_kq, (int8_t *)d_vq, (float *)d_ks,
                     (float *)d_vs, AttnPost{}, pos, 0, n_heads, n_kv_heads, head_dim, kr, attn_scale, nsplit, 1, pp,
                     d_out, nullptr, nullptr, nullptr, gq);
    // the copied position lives on this function's stack; the no-alloc variant stores it
    // with a kernel and stays asynchronous
    if (!noalloc) hip_check(hipStreamSynchronize(ctx->stream), "sync");
}
}  // namespace

int32_t k2t_attn_decode(k2t_ctx *ctx, int32_t bits, const float *d_q, int32_t n_heads, int32_t n_kv_heads,
                        int32_t head_dim, const void *d_kq, const void *d_ks, const void *d_vq, const void *d_vs,
                        int32_t cap, int32_t seq, int32_t window, int32_t sink_tokens, float attn_scale,
                        float *d_out) {
    return mguard([&] {
        attn_decode_impl(ctx, bits, d_q, n_heads, n_kv_heads, head_dim, d_kq, d_ks, d_vq, d_vs, cap, seq, window,
                         sink_tokens, attn_scale, d_out, false);
    });
}

int32_t k2t_attn_decode_noalloc(k2t_ctx *ctx, int32_t bits, const float *d_q, int32_t n_heads, int32_t n_kv_heads,
                                int32_t head_dim, const void *d_kq, const void *d_ks, const void *d_vq,
                                const void *d_vs, int32_t cap, int32_t seq, int32_t window, int32_t sink_tokens,
                                float attn_scale, float *d_out) {
    return mguard([&] {
        attn_decode_impl(ctx, bits, d_q, n_heads, n_kv_heads, head_dim, d_kq, d_ks, d_vq, d_vs, cap, seq, window,
                         sink_tokens, attn_scale, d_out, true);
    });
}

}  // extern "C"
