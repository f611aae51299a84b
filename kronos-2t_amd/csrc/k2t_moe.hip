// Sparse-MoE feed-forward for one token (SparseMoeRuntime::forward_layer_single,
// sparse_moe.rs:961-1084) over NF3 / NF4 expert records of a .k2tm shard held in HBM.
//
// Every expert of every layer stays resident (a 30B-A3B shard is ~11 GB of the 288 GB),
// so there is no paging.  Per token and MoE layer:
//   1. moe_route_kernel    x_norm = RMSNorm(hidden) * post_norm, logits = W_router x_norm
//                          (+ bias), one wave per expert; then, in the same launch,
//                          softmax / topk-softmax / sigmoid, top-k, renormalize, sort by
//                          expert id (route_sorted, sparse_moe.rs:86-182) on one wave;
//   3. grouped gate_up GEMV: slot z streams expert route[z]'s gate_up pairs with the int8
//      activation of x_norm built in LDS (populate_fwht of x_norm); rows are written in
//      [gate64, up64] blocks;
//   4. grouped down GEMV: SwiGLU + FWHT (chunk c) + int8 of slot z's gate_up, built in
//      LDS, times expert route[z]'s down pairs;
//   5. moe_combine_kernel  proj = sum_z w_z * out_z in route order, hidden += proj.
#include <float.h>
#include <math.h>
#include <string.h>

#include <string>

#include "../../include/k2t_hip.h"
#include "k2t_device.h"
#include "k2t_expf.h"
#include "k2t_internal.h"
#include "k2t_moe.h"
#include "k2t_route.h"

namespace k2t {

// ---------------------------------------------------------------- .k2tm layout
// K2tmShardHeader (moe_800b.rs:792-854) and nf_expert_byte_layout (moe_800b.rs:1311-1375).
constexpr size_t kK2tmPage = 16384;
static const char kK2tmMagic[12] = {'K', '2', 'T', 'M', '8', '0', '0', 'B', '_', 'V', '1', '\0'};

static size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

ExpertLayout expert_layout(size_t d_model, size_t d_ff, int bits, size_t sgc) {
    ExpertLayout L{};
    const size_t chunk_b = bits == 3 ? 384 : 512;
    sgc = sgc < 1 ? 1 : sgc;
    L.gu_rows = 2 * d_ff;
    L.dn_rows = d_model;
    const size_t gu_chunks = d_model / 64, gu_sg = (gu_chunks + sgc - 1) / sgc;
    const size_t dn_chunks = d_ff / 64, dn_sg = (dn_chunks + sgc - 1) / sgc;
    L.gu_pair_bytes = (L.gu_rows / 32) * (gu_sg * 64 + gu_chunks * 2 * chunk_b);
    L.dn_pair_bytes = (L.dn_rows / 32) * (dn_sg * 64 + dn_chunks * 2 * chunk_b);
    L.gu_cb_off = 0;
    L.dn_cb_off = 16;
    L.gu_pair_off = 64;
    L.dn_pair_off = align_up(L.gu_pair_off + L.gu_pair_bytes, 64);
    L.aligned_bytes = align_up(L.dn_pair_off + L.dn_pair_bytes, kK2tmPage);
    return L;
}

static void decode_header(const uint8_t *page, size_t len, k2t_k2tm_header *h) {
    if (!page || len < kK2tmPage) throw Error(K2T_E_ARG, "k2tm header shorter than 16384 bytes");
    if (memcmp(page, kK2tmMagic, 12) != 0) throw Error(K2T_E_ARG, "bad k2tm header magic");
    uint64_t w[7];
    memcpy(w, page + 16, sizeof(w));
    h->num_layers = (int64_t)w[0];
    h->experts_per_layer = (int64_t)w[1];
    h->d_model = (int64_t)w[2];
    h->d_ff_expert = (int64_t)w[3];
    h->scale_group_chunks = (int64_t)w[4];
    h->aligned_expert_bytes = (int64_t)w[5];
    h->bits = (int64_t)w[6];
    const auto bad = [](const char *m) { throw Error(K2T_E_ARG, std::string("k2tm header: ") + m); };
    if (h->num_layers <= 0 || h->num_layers > 4096) bad("layer count out of range");
    if (h->experts_per_layer < 2 || h->experts_per_layer > 1024) bad("experts per layer out of range");
    if (h->d_model <= 0 || h->d_model % 64 || h->d_model > 32768) bad("d_model must be a positive multiple of 64");
    if (h->d_ff_expert <= 0 || h->d_ff_expert % 64 || h->d_ff_expert > 32768)
        bad("d_ff_expert must be a positive multiple of 64");
    if (h->scale_group_chunks < 0 || h->scale_group_chunks > 8) bad("scale_group_chunks out of range");
    if (h->bits != 3 && h->bits != 4)
        throw Error(K2T_E_STATE, "k2tm experts with " + std::to_string(h->bits) + " bits: the HIP GEMV takes NF3 and NF4");
    const ExpertLayout L = expert_layout((size_t)h->d_model, (size_t)h->d_ff_expert, (int)h->bits,
                                         (size_t)h->scale_group_chunks);
    if ((size_t)h->aligned_expert_bytes != L.aligned_bytes) bad("aligned_expert_bytes does not match the NF layout");
}

static size_t total_bytes(const k2t_k2tm_header &h) {
    return kK2tmPage + (size_t)h.num_layers * (size_t)h.experts_per_layer * (size_t)h.aligned_expert_bytes;
}

static void fill_geom(k2t_mat &m, int rows, int cols, int bits, int sgc, size_t pair_bytes) {
    m = k2t_mat{};
    m.fmt = K2T_FMT_NF;
    m.rows = rows;
    m.cols = cols;
    m.nc = cols / 64;
    m.stripes = rows / 16;
    m.pairs = rows / 32;
    m.has_tail = 0;
    m.bits = bits;
    m.sgc = sgc < 1 ? 1 : sgc;
    m.pair_len = pair_bytes;
}

static k2t_experts *make_bank(k2t_ctx *ctx, const k2t_k2tm_header &h) {
    k2t_experts *b = new k2t_experts();
    b->ctx = ctx;
    b->hdr = h;
    b->lay = expert_layout((size_t)h.d_model, (size_t)h.d_ff_expert, (int)h.bits, (size_t)h.scale_group_chunks);
    b->len = total_bytes(h);
    fill_geom(b->gu, (int)b->lay.gu_rows, (int)h.d_model, (int)h.bits, (int)h.scale_group_chunks, b->lay.gu_pair_bytes);
    fill_geom(b->dn, (int)b->lay.dn_rows, (int)h.d_ff_expert, (int)h.bits, (int)h.scale_group_chunks,
              b->lay.dn_pair_bytes);
    b->gu.ctx = b->dn.ctx = ctx;
    return b;
}

// ---------------------------------------------------------------- kernels
// Router logits (route_logit, one wave per expert row) and, in the same launch, the
// selection: wave 0 of workgroup 0 waits for all E words of this call's epoch, then runs
// select_routes.  The epoch is the call counter *ctr + 1; workgroup 0 advances the counter
// after its wait, when every workgroup has read it.
template <int NJ>  // float4 per lane of each vector: d <= 256 * NJ
__global__ __launch_bounds__(256) void moe_route_kernel(const float *__restrict__ x, const float *__restrict__ nw,
                                                        float eps, int d, const float *__restrict__ W,
                                                        const float *__restrict__ bias, int E, int k, int norm_topk,
                                                        int scoring, unsigned long long *__restrict__ words,
                                                        uint32_t *__restrict__ ctr, int *__restrict__ err,
                                                        uint32_t spin_limit, int *__restrict__ ids,
                                                        float *__restrict__ wts) {
    const uint32_t lane = threadIdx.x & 63u;
    const int wave = (int)(threadIdx.x >> 6);
    const int e = (int)blockIdx.x * 4 + wave;
    // The counter as a vector load through a lane offset the compiler cannot see is zero:
    // as a scalar load its wait came first, one round trip before the vector loads.
    int zoff;
    asm volatile("v_mov_b32 %0, 0" : "=v"(zoff));
    const uint32_t epoch = ld_global(ctr + zoff) + 1u;
    if (e < E) route_logit<NJ>(x, nw, eps, d, W, bias, e, lane, epoch, words);
    if (blockIdx.x != 0 || wave != 0) return;
    route_collect(words, E, epoch, spin_limit, err, lane, k, norm_topk, scoring, ids, wts, nullptr);
    if (lane == 0) *ctr = epoch;
}

// Clears the hand-off words and the call counter of a fresh workspace (a kernel, so that a
// captured graph holds no memset node).
__global__ void moe_clear_kernel(unsigned long long *words, int E, unsigned long long *pub, uint32_t *ctr, int *err) {
    for (int i = (int)threadIdx.x; i < 2 * E + 2; i += (int)blockDim.x) words[i] = 0ull;
    if (threadIdx.x < K2T_MOE_MAX_TOPK) pub[threadIdx.x] = 0ull;
    if (threadIdx.x == 0) {
        *ctr = 0u;
        *err = 0;
    }
}

void launch_moe_clear(hipStream_t st, const MoeWork &ws, int E) {
    hipLaunchKernelGGL(moe_clear_kernel, dim3(1), dim3(256), 0, st, ws.words, E, ws.pub, ws.ctr, ws.err);
    hip_check(hipGetLastError(), "moe clear launch");
}

// out.fill(0); out += w_z * expert_z in route order; hidden += out
// (sparse_moe.rs:1001-1003, 1041-1043; real_llm.rs:6714).
// Up to kCombineMax slots have all their loads in flight together (slot min(z, k - 1) is
// read for z >= k and not added); a loop over a run-time k issued one load per round
// trip.  More slots take the loop.
constexpr int kCombineMax = 8;
// With ctr set, thread 0 advances the route-call counter (routing ran inside the gate_up
// launch, whose workgroups have all read it by now).
// With a shared expert (sh != NULL) the sum starts from its output, times the gate scale
// when a gate is present and the scale differs from 1 by more than FLT_EPSILON
// (forward_single then forward_layer_single, sparse_moe.rs:252-312, 989-1000).
__global__ __launch_bounds__(256) void moe_combine_kernel(float *__restrict__ hidden, const float *__restrict__ eo,
                                                          const float *__restrict__ wts, int k, int d,
                                                          uint32_t *__restrict__ ctr, const float *__restrict__ sh,
                                                          const float *__restrict__ sh_scale) {
    const int r = (int)blockIdx.x * 256 + (int)threadIdx.x;
    if (ctr && r == 0) *ctr = *ctr + 1u;
    if (r >= d) return;
    float p = 0.0f;
    if (sh) {
        p = sh[r];
        if (sh_scale) {
            const float g = sh_scale[0];
            if (fabsf(g - 1.0f) > FLT_EPSILON) p = p * g;
        }
    }
    if (k <= kCombineMax) {
        float e[kCombineMax];
#pragma unroll
        for (int z = 0; z < kCombineMax; z++) e[z] = eo[(size_t)min(z, k - 1) * d + r];
        const float h = hidden[r];
#pragma unroll
        for (int z = 0; z < kCombineMax; z++)
            if (z < k) p = p + wts[z] * e[z];
        hidden[r] = h + p;
        return;
    }
    for (int z = 0; z < k; z++) p = p + wts[z] * eo[(size_t)z * d + r];
    hidden[r] = hidden[r] + p;
}

// Exact-order routing (the x86 reference's order; one workgroup): x_norm[i] = (h[i] *
// inv_rms) * w[i] (rms_norm, real_llm.rs:9858-9898, inv_rms in the x86 order), logit e =
// sum_i W[e][i] * x_norm[i] added in i order (dot_f32_moe's portable sum,
// sparse_moe.rs:1644-1656) + bias, one thread per expert; then thread 0 runs route_sorted
// (sparse_moe.rs:86-182): softmax / sigmoid with the x86 build's exp (expf_rn) and
// sequential sums, select_topk_by_score (strict '>' insertion, 185-206), the top-k
// renormalization, and the insertion sort by expert id.
__global__ __launch_bounds__(256) void moe_route_exact_kernel(const float *__restrict__ hidden,
                                                              const float *__restrict__ post_norm,
                                                              const float *__restrict__ inv_rms, int d,
                                                              const float *__restrict__ W, const float *__restrict__ bias,
                                                              int E, int k, int norm_topk, int scoring,
                                                              int *__restrict__ ids, float *__restrict__ wts) {
    __shared__ float xn[4096];
    __shared__ float z[256];
    const int tid = (int)threadIdx.x;
    const float inv = inv_rms[0];
    for (int i = tid; i < d; i += 256) xn[i] = (hidden[i] * inv) * post_norm[i];
    __syncthreads();
    for (int e = tid; e < E; e += 256) {
        const float *row = W + (size_t)e * d;
        float a = 0.0f;
        for (int i = 0; i < d; i++) a = a + row[i] * xn[i];
        if (bias) a = a + bias[e];
        z[e] = a;
    }
    __syncthreads();
    if (tid != 0) return;
    if (scoring == K2T_MOE_SOFTMAX) {
        float mz = -INFINITY;
        for (int e = 0; e < E; e++) mz = fmaxf(mz, z[e]);
        float sum = 0.0f;
        for (int e = 0; e < E; e++) {
            z[e] = expf_rn(z[e] - mz);
            sum = sum + z[e];
        }
        const float inv_all = sum > 0.0f ? 1.0f / sum : 1.0f / (float)E;
        for (int e = 0; e < E; e++) z[e] = z[e] * inv_all;
    } else if (scoring == K2T_MOE_SIGMOID) {
        for (int e = 0; e < E; e++) z[e] = 1.0f / (1.0f + expf_rn(-z[e]));
    }
    int oe[K2T_MOE_MAX_TOPK];
    float ow[K2T_MOE_MAX_TOPK];
    int len = 0;
    for (int e = 0; e < E; e++) {
        const float sv = z[e];
        if (len < k) {
            int pos = len;
            while (pos > 0 && sv > ow[pos - 1]) {
                oe[pos] = oe[pos - 1];
                ow[pos] = ow[pos - 1];
                pos--;
            }
            oe[pos] = e;
            ow[pos] = sv;
            len++;
        } else if (sv > ow[k - 1]) {
            int pos = k - 1;
            while (pos > 0 && sv > ow[pos - 1]) {
                oe[pos] = oe[pos - 1];
                ow[pos] = ow[pos - 1];
                pos--;
            }
            oe[pos] = e;
            ow[pos] = sv;
        }
    }
    if (scoring == K2T_MOE_TOPK_SOFTMAX) {
        float mz = -INFINITY;
        for (int i = 0; i < k; i++) mz = fmaxf(mz, ow[i]);
        float sum = 0.0f;
        for (int i = 0; i < k; i++) {
            ow[i] = expf_rn(ow[i] - mz);
            sum = sum + ow[i];
        }
        const float inv_k = sum > 0.0f ? 1.0f / sum : 1.0f / (float)k;
        for (int i = 0; i < k; i++) ow[i] = ow[i] * inv_k;
    } else if (norm_topk) {
        float sum = 0.0f;
        for (int i = 0; i < k; i++) sum = sum + ow[i];
        if (sum > 0.0f) {
            const float inv_top = 1.0f / sum;
            for (int i = 0; i < k; i++) ow[i] = ow[i] * inv_top;
        }
    }
    for (int i = 1; i < k; i++) {
        const int ce = oe[i];
        const float cw = ow[i];
        int j = i;
        while (j > 0 && oe[j - 1] > ce) {
            oe[j] = oe[j - 1];
            ow[j] = ow[j - 1];
            j--;
        }
        oe[j] = ce;
        ow[j] = cw;
    }
    for (int i = 0; i < k; i++) {
        ids[i] = oe[i];
        wts[i] = ow[i];
    }
}

// Exact-order gate scale of the shared expert: 1 / (1 + exp(-z)), z = sum_i gate[i] *
// x_norm[i] added in i order (dot_f32_moe, sparse_moe.rs:241-250), exp = expf_rn.  One
// thread.
__global__ void moe_shared_gate_exact_kernel(const float *__restrict__ hidden, const float *__restrict__ post_norm,
                                             const float *__restrict__ inv_rms, int d,
                                             const float *__restrict__ gate, float *__restrict__ out) {
    if (threadIdx.x != 0) return;
    const float inv = inv_rms[0];
    float zz = 0.0f;
    for (int i = 0; i < d; i++) zz = zz + gate[i] * ((hidden[i] * inv) * post_norm[i]);
    out[0] = 1.0f / (1.0f + expf_rn(-zz));
}

// Gate scale of the shared expert: 1 / (1 + exp(-dot(gate, x_norm))) with x_norm =
// (hidden * inv_rms) * post_norm (gate_scale, sparse_moe.rs:241-250); inv_rms in the
// fused activation builders' order (row_sumsq_wave), the dot as a fixed tree.  One
// workgroup; the scale goes to out[0].
__global__ __launch_bounds__(256) void moe_shared_gate_kernel(const float *__restrict__ hidden,
                                                              const float *__restrict__ post_norm, float eps, int d,
                                                              const float *__restrict__ gate, float *__restrict__ out) {
    __shared__ float part[5];
    const uint32_t lane = threadIdx.x & 63u;
    const int wave = (int)(threadIdx.x >> 6);
    if (wave == 0) {
        const float ss = row_sumsq_wave(hidden, d, lane);
        if (lane == 0) part[4] = 1.0f / sqrtf(ss / (float)d + eps);
    }
    __syncthreads();
    const float inv = part[4];
    float z = 0.0f;
    for (int i = (int)threadIdx.x; i < d; i += 256) z = fmaf(gate[i], (hidden[i] * inv) * post_norm[i], z);
    z = wave_sum_f(z);
    if (lane == 0) part[wave] = z;
    __syncthreads();
    if (threadIdx.x == 0) {
        const float t = (part[0] + part[1]) + (part[2] + part[3]);
        out[0] = 1.0f / (1.0f + expf(-t));
    }
}

// Exact-order MoE feed-forward (the context's exact mode): every step in the x86
// reference's order.  inv_rms with the four-accumulator sum of squares, the int8
// activation of x_norm once (populate_fwht), routing in moe_route_exact_kernel, the
// expert GEMVs with the in-order epilogue on that activation, SwiGLU with expf_rn, and the
// combine in route order (moe_combine_kernel's arithmetic is already the reference's).
static void launch_moe_ffn_exact(k2t_ctx *ctx, const MoeLayer &L, float *hidden, const float *post_norm, float eps,
                                 const MoeWork &ws) {
    const k2t_experts *b = L.bank;
    const int d = (int)b->hdr.d_model, dff = (int)b->hdr.d_ff_expert, E = (int)b->hdr.experts_per_layer;
    hipStream_t st = ctx->stream;
    launch_inv_rms_x86(st, hidden, eps, d, 1, ws.rms);
    launch_act_quant(ctx, hidden, post_norm, ws.rms, d, 1, ws.aq, ws.as, ws.asum);
    float *sh_out = nullptr, *sh_scale = nullptr;
    if (L.sh_gu) {
        const int inter = L.sh_gu->rows / 2;
        float *sh_gu = L.sh_buf;
        sh_out = L.sh_buf + 2 * (size_t)inter;
        float *tail = sh_out + d + 64;  // the shared expert's down activation
        float *s_s = tail;
        int32_t *s_sum = reinterpret_cast<int32_t *>(tail + inter / 64);
        int8_t *s_q = reinterpret_cast<int8_t *>(tail + 2 * (inter / 64));
        if (L.sh_gate) {
            sh_scale = sh_out + d;
            hipLaunchKernelGGL(moe_shared_gate_exact_kernel, dim3(1), dim3(64), 0, st, hidden, post_norm, ws.rms, d,
                               L.sh_gate, sh_scale);
            hip_check(hipGetLastError(), "moe shared gate launch");
        }
        launch_gemv_ex(ctx, L.sh_gu, ws.aq, ws.as, ws.asum, 1, sh_gu, (size_t)L.sh_gu->rows, false, 1);
        launch_swiglu_act(st, ctx->signs, sh_gu, inter, 1, s_q, s_s, s_sum, true);
        launch_gemv_ex(ctx, L.sh_dn, s_q, s_s, s_sum, 1, sh_out, (size_t)d, false);
    }
    hipLaunchKernelGGL(moe_route_exact_kernel, dim3(1), dim3(256), 0, st, hidden, post_norm, ws.rms, d, L.router_w,
                       L.router_b, E, L.top_k, L.norm_topk, L.scoring, ws.ids, ws.wts);
    hip_check(hipGetLastError(), "moe exact route launch");
    const uint8_t *layer_base = b->d_bytes + kK2tmPage + (size_t)L.shard_layer * E * b->lay.aligned_bytes;
    GemvGroup g{};
    g.route = ws.ids;
    g.nslots = L.top_k;
    g.bank = layer_base;
    g.stride = b->lay.aligned_bytes;
    g.mat_off = (uint32_t)b->lay.gu_pair_off;
    g.cb_off = (uint32_t)b->lay.gu_cb_off;
    g.slot_out = (size_t)2 * dff;
    g.slot_src = 0;
    g.gu_split = 1;
    g.xq = ws.aq;
    g.xs = ws.as;
    g.xsum = ws.asum;
    g.slot_act = 0;
    launch_gemv_grouped(ctx, &b->gu, g, 0, nullptr, nullptr, 0.0f, ws.gu);
    launch_swiglu_act(st, ctx->signs, ws.gu, dff, L.top_k, ws.mq, ws.ms, ws.msum, true);
    g.mat_off = (uint32_t)b->lay.dn_pair_off;
    g.cb_off = (uint32_t)b->lay.dn_cb_off;
    g.slot_out = (size_t)d;
    g.gu_split = 0;
    g.xq = ws.mq;
    g.xs = ws.ms;
    g.xsum = ws.msum;
    g.slot_act = 1;
    launch_gemv_grouped(ctx, &b->dn, g, 0, nullptr, nullptr, 0.0f, ws.eo);
    hipLaunchKernelGGL(moe_combine_kernel, dim3((d + 255) / 256), dim3(256), 0, st, hidden, ws.eo, ws.wts, L.top_k,
                       d, nullptr, sh_out, sh_scale);
    hip_check(hipGetLastError(), "moe combine launch");
}

void launch_moe_ffn(k2t_ctx *ctx, const MoeLayer &L, float *hidden, const float *post_norm, float eps,
                    const MoeWork &ws) {
    if (ctx->exact) {
        launch_moe_ffn_exact(ctx, L, hidden, post_norm, eps, ws);
        return;
    }
    const k2t_experts *b = L.bank;
    const int d = (int)b->hdr.d_model, dff = (int)b->hdr.d_ff_expert, E = (int)b->hdr.experts_per_layer;
    hipStream_t st = ctx->stream;
    // shared expert first (it reads the same x_norm; its output seeds the combine's sum)
    float *sh_out = nullptr, *sh_scale = nullptr;
    if (L.sh_gu) {
        const int inter = L.sh_gu->rows / 2;
        float *sh_gu = L.sh_buf;
        sh_out = L.sh_buf + 2 * (size_t)inter;
        if (L.sh_gate) {
            sh_scale = sh_out + d;
            hipLaunchKernelGGL(moe_shared_gate_kernel, dim3(1), dim3(256), 0, st, hidden, post_norm, eps, d, L.sh_gate,
                               sh_scale);
            hip_check(hipGetLastError(), "moe shared gate launch");
        }
        launch_gemv_fused(ctx, L.sh_gu, K2T_XS_RMSNORM, hidden, post_norm, eps, sh_gu, false, 1);
        launch_gemv_fused(ctx, L.sh_dn, K2T_XS_SWIGLU, sh_gu, nullptr, 0.0f, sh_out, false);
    }
    // d <= 2048: the routing runs in the gate_up launch (one launch fewer per layer);
    // larger rows keep the route kernel.
    const bool fused = d <= 2048;
    if (!fused) {
        if (d <= 4096)
            hipLaunchKernelGGL(moe_route_kernel<16>, dim3((E + 3) / 4), dim3(256), 0, st, hidden, post_norm, eps, d,
                               L.router_w, L.router_b, E, L.top_k, L.norm_topk, L.scoring, ws.words, ws.ctr, ws.err,
                               1u << 22, ws.ids, ws.wts);
        else
            throw Error(K2T_E_ARG, "MoE router: d_model above 4096");
        hip_check(hipGetLastError(), "moe route launch");
    }
    const uint8_t *layer_base = b->d_bytes + kK2tmPage + (size_t)L.shard_layer * E * b->lay.aligned_bytes;
    GemvGroup g{};
    g.route = ws.ids;
    g.nslots = L.top_k;
    g.bank = layer_base;
    g.stride = b->lay.aligned_bytes;
    g.mat_off = (uint32_t)b->lay.gu_pair_off;
    g.cb_off = (uint32_t)b->lay.gu_cb_off;
    g.slot_out = (size_t)2 * dff;
    g.slot_src = 0;
    g.gu_split = 1;
    if (fused) {
        g.rt_w = L.router_w;
        g.rt_b = L.router_b;
        g.rt_words = ws.words;
        g.rt_pub = ws.pub;
        g.rt_ctr = ws.ctr;
        g.rt_err = ws.err;
        g.rt_wts = ws.wts;
        g.rt_E = E;
        g.rt_norm = L.norm_topk;
        g.rt_scoring = L.scoring;
        g.rt_spin = 1u << 22;
    }
    launch_gemv_grouped(ctx, &b->gu, g, K2T_XS_RMSNORM, hidden, post_norm, eps, ws.gu);
    g.rt_w = nullptr;
    g.mat_off = (uint32_t)b->lay.dn_pair_off;
    g.cb_off = (uint32_t)b->lay.dn_cb_off;
    g.slot_out = (size_t)d;
    g.slot_src = (size_t)2 * dff;
    g.gu_split = 0;
    launch_gemv_grouped(ctx, &b->dn, g, K2T_XS_SWIGLU, ws.gu, nullptr, 0.0f, ws.eo);
    hipLaunchKernelGGL(moe_combine_kernel, dim3((d + 255) / 256), dim3(256), 0, st, hidden, ws.eo, ws.wts, L.top_k,
                       d, fused ? ws.ctr : nullptr, sh_out, sh_scale);
    hip_check(hipGetLastError(), "moe combine launch");
}

size_t moe_work_floats(const k2t_experts *b, int top_k) {
    const size_t d = (size_t)b->hdr.d_model, dff = (size_t)b->hdr.d_ff_expert, E = (size_t)b->hdr.experts_per_layer;
    return (size_t)top_k * 2 * dff + (size_t)top_k * d + 4 * E + 4 + 2 * K2T_MOE_MAX_TOPK + 2 * (size_t)top_k + 64 +
           64 + d / 4 + 2 * (d / 64) + (size_t)top_k * dff / 4 + 2 * ((size_t)top_k * dff / 64) + 64;
}

MoeWork moe_work_carve(float *base, const k2t_experts *b, int top_k) {
    const size_t d = (size_t)b->hdr.d_model, dff = (size_t)b->hdr.d_ff_expert, E = (size_t)b->hdr.experts_per_layer;
    MoeWork w;
    float *p = base;  // 256-byte aligned; every region below is a multiple of 64 floats
    w.gu = p;
    p += (size_t)top_k * 2 * dff;
    w.eo = p;
    p += (size_t)top_k * d;
    w.words = reinterpret_cast<unsigned long long *>(p);
    p += 4 * E + 4;
    w.pub = reinterpret_cast<unsigned long long *>(p);
    p += 2 * K2T_MOE_MAX_TOPK;
    w.wts = p;
    p += top_k;
    w.ids = reinterpret_cast<int *>(p);
    p += top_k;
    w.ctr = reinterpret_cast<uint32_t *>(p);
    w.err = reinterpret_cast<int *>(p + 1);
    p += 64;
    w.rms = p;
    p += 64;
    w.as = p;
    p += d / 64;
    w.asum = reinterpret_cast<int32_t *>(p);
    p += d / 64;
    w.ms = p;
    p += (size_t)top_k * dff / 64;
    w.msum = reinterpret_cast<int32_t *>(p);
    p += (size_t)top_k * dff / 64;
    w.aq = reinterpret_cast<int8_t *>(p);
    p += d / 4;
    w.mq = reinterpret_cast<int8_t *>(p);
    return w;
}

void check_moe_args(const k2t_experts *bank, int shard_layer, int top_k, int scoring) {
    if (!bank) throw Error(K2T_E_ARG, "expert bank is NULL");
    if (shard_layer < 0 || shard_layer >= bank->hdr.num_layers) throw Error(K2T_E_ARG, "shard layer out of range");
    if (top_k < 1 || top_k > K2T_MOE_MAX_TOPK || top_k > bank->hdr.experts_per_layer)
        throw Error(K2T_E_ARG, "top_k out of range");
    if (bank->hdr.experts_per_layer > 256) throw Error(K2T_E_ARG, "at most 256 experts per layer");
    if (scoring != K2T_MOE_SOFTMAX && scoring != K2T_MOE_TOPK_SOFTMAX && scoring != K2T_MOE_SIGMOID)
        throw Error(K2T_E_ARG, "unknown router scoring");
    if (bank->hdr.d_model > 4096) throw Error(K2T_E_ARG, "MoE router: d_model above 4096");
    if ((size_t)bank->hdr.d_model > (size_t)kSignBlocks * 64 || (size_t)bank->hdr.d_ff_expert > (size_t)kSignBlocks * 64)
        throw Error(K2T_E_ARG, "expert dimensions exceed the Hadamard sign table");
}

// A converted shard says so in the last 16 bytes of its device header page (zero padding
// in the .k2tm header, past every field), so a later wrap of the same bytes knows their
// order and a second conversion is a no-op.
static const char kLaneMark[16] = {'K', '2', 'T', '-', 'N', 'F', '3', '-', 'L', 'A', 'N', 'E', '-', 'V', '1', '\0'};
static bool bank_marked_lane(const k2t_experts *b) {
    char got[16];
    hip_check(hipSetDevice(b->ctx->device), "hipSetDevice");
    hip_check(hipMemcpy(got, b->d_bytes + kK2tmPage - 16, 16, hipMemcpyDeviceToHost), "k2tm lane mark read");
    return memcmp(got, kLaneMark, 16) == 0;
}

// NF3 expert matrices of every record, in place, into lane order (launch_nf3_lane_order);
// a no-op for NF4 banks and for banks already converted; synchronous.
static void bank_to_lane_order(k2t_experts *b) {
    if (b->hdr.bits != 3 || b->gu.nf3_lane) return;
    if (bank_marked_lane(b)) {
        b->gu.nf3_lane = b->dn.nf3_lane = 1;
        return;
    }
    const int nrec = (int)(b->hdr.num_layers * b->hdr.experts_per_layer);
    uint8_t *rec0 = b->d_bytes + kK2tmPage;
    hipStream_t st = b->ctx->stream;
    hip_check(hipSetDevice(b->ctx->device), "hipSetDevice");
    launch_nf3_lane_order(st, rec0 + b->lay.gu_pair_off, b->lay.aligned_bytes, nrec, b->lay.gu_pair_bytes / b->gu.pairs,
                          b->gu.pairs, b->gu.nc, b->gu.sgc, false);
    launch_nf3_lane_order(st, rec0 + b->lay.dn_pair_off, b->lay.aligned_bytes, nrec, b->lay.dn_pair_bytes / b->dn.pairs,
                          b->dn.pairs, b->dn.nc, b->dn.sgc, false);
    hip_check(hipStreamSynchronize(st), "k2tm nf3 lane order");
    hip_check(hipMemcpy(b->d_bytes + kK2tmPage - 16, kLaneMark, 16, hipMemcpyHostToDevice), "k2tm lane mark");
    b->gu.nf3_lane = b->dn.nf3_lane = 1;
}

}  // namespace k2t

using namespace k2t;

namespace {
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
}  // namespace

extern "C" {

int32_t k2t_k2tm_read_header(const uint8_t *page, size_t len, k2t_k2tm_header *out) {
    return mguard([&] {
        if (!out) throw Error(K2T_E_ARG, "NULL argument");
        decode_header(page, len, out);
    });
}

int32_t k2t_k2tm_expert_layout(int64_t d_model, int64_t d_ff, int32_t bits, int32_t sgc, k2t_k2tm_layout *out) {
    return mguard([&] {
        if (!out) throw Error(K2T_E_ARG, "NULL argument");
        if (d_model <= 0 || d_model % 64 || d_ff <= 0 || d_ff % 64 || (bits != 3 && bits != 4) || sgc < 0 || sgc > 8)
            throw Error(K2T_E_ARG, "bad expert layout parameters");
        const ExpertLayout L = expert_layout((size_t)d_model, (size_t)d_ff, bits, (size_t)sgc);
        out->gu_codebook_off = L.gu_cb_off;
        out->dn_codebook_off = L.dn_cb_off;
        out->gu_pair_off = L.gu_pair_off;
        out->gu_pair_bytes = L.gu_pair_bytes;
        out->dn_pair_off = L.dn_pair_off;
        out->dn_pair_bytes = L.dn_pair_bytes;
        out->aligned_expert_bytes = L.aligned_bytes;
    });
}

int32_t k2t_experts_upload(k2t_ctx *ctx, const uint8_t *k2tm, size_t len, k2t_experts **out) {
    return mguard([&] {
        if (!ctx || !k2tm || !out) throw Error(K2T_E_ARG, "NULL argument");
        *out = nullptr;
        k2t_k2tm_header h;
        decode_header(k2tm, len, &h);
        if (len < total_bytes(h)) throw Error(K2T_E_ARG, "k2tm shard shorter than its header declares");
        k2t_experts *b = make_bank(ctx, h);
        hip_check(hipSetDevice(ctx->device), "hipSetDevice");
        void *d = nullptr;
        const hipError_t e = hipMalloc(&d, b->len);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            delete b;
            throw Error(K2T_E_NOMEM, std::string("hipMalloc failed: ") + hipGetErrorString(e));
        }
        b->d_bytes = (uint8_t *)d;
        b->owns = true;
        const hipError_t c = hipMemcpy(d, k2tm, b->len, hipMemcpyHostToDevice);
        if (c != hipSuccess) {
            k2t_experts_destroy(b);
            hip_check(c, "k2tm upload");
        }
        try {
            bank_to_lane_order(b);  // our own copy: the fast NF3 layout
        } catch (...) {
            k2t_experts_destroy(b);
            throw;
        }
        *out = b;
    });
}

int32_t k2t_experts_nf3_lane_order(k2t_experts *bank) {
    return mguard([&] {
        if (!bank) throw Error(K2T_E_ARG, "NULL argument");
        bank_to_lane_order(bank);
    });
}

int32_t k2t_experts_wrap(k2t_ctx *ctx, const uint8_t *d_k2tm, size_t len, const uint8_t *header_page,
                         k2t_experts **out) {
    return mguard([&] {
        if (!ctx || !d_k2tm || !out) throw Error(K2T_E_ARG, "NULL argument");
        *out = nullptr;
        k2t_k2tm_header h;
        decode_header(header_page, kK2tmPage, &h);
        if (len < total_bytes(h)) throw Error(K2T_E_ARG, "device shard shorter than its header declares");
        if ((uintptr_t)d_k2tm % 256) throw Error(K2T_E_ARG, "device shard must be 256-byte aligned");
        k2t_experts *b = make_bank(ctx, h);
        b->d_bytes = const_cast<uint8_t *>(d_k2tm);
        b->owns = false;
        try {
            if (h.bits == 3 && bank_marked_lane(b)) b->gu.nf3_lane = b->dn.nf3_lane = 1;  // converted before
        } catch (...) {
            delete b;
            throw;
        }
        *out = b;
    });
}

void k2t_experts_destroy(k2t_experts *b) {
    if (!b) return;
    if (b->owns && b->d_bytes) {
        (void)hipSetDevice(b->ctx->device);
        (void)hipFree(b->d_bytes);
    }
    delete b;
}

int32_t k2t_experts_info(const k2t_experts *b, k2t_k2tm_header *out) {
    return mguard([&] {
        if (!b || !out) throw Error(K2T_E_ARG, "NULL argument");
        *out = b->hdr;
    });
}

int32_t k2t_moe_ffn(k2t_ctx *ctx, const k2t_experts *bank, int32_t shard_layer, const float *d_router_w,
                    const float *d_router_bias, int32_t top_k, int32_t norm_topk_prob, int32_t scoring,
                    float *d_hidden, const float *d_post_norm, float eps, int32_t *d_route_ids,
                    float *d_route_weights) {
    return mguard([&] {
        if (!ctx || !d_router_w || !d_hidden || !d_post_norm) throw Error(K2T_E_ARG, "NULL argument");
        check_moe_args(bank, shard_layer, top_k, scoring);
        if (bank->ctx != ctx) throw Error(K2T_E_ARG, "expert bank of another context");
        MoeLayer L{bank, shard_layer, d_router_w, d_router_bias, top_k, norm_topk_prob ? 1 : 0, scoring};
        ensure_scratch(ctx, moe_work_floats(bank, top_k));
        const MoeWork ws = moe_work_carve(ctx->scratch, bank, top_k);
        launch_moe_clear(ctx->stream, ws, (int)bank->hdr.experts_per_layer);  // the scratch is shared
        launch_moe_ffn(ctx, L, d_hidden, d_post_norm, eps, ws);
        if (d_route_ids)
            hip_check(hipMemcpyAsync(d_route_ids, ws.ids, (size_t)top_k * sizeof(int), hipMemcpyDeviceToDevice,
                                     ctx->stream),
                      "route copy");
        if (d_route_weights)
            hip_check(hipMemcpyAsync(d_route_weights, ws.wts, (size_t)top_k * sizeof(float), hipMemcpyDeviceToDevice,
                                     ctx->stream),
                      "route copy");
    });
}

}  // extern "C"
