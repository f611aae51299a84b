// Decode-step device glue around the GEMVs (gfx950): fused RMSNorm + FWHT + int8,
// RoPE + Hadamard int8 KV store, flash-decoding q8 attention with a fused
// IFWHT -> FWHT -> int8 epilogue for o_proj, SwiGLU + FWHT + int8, tied-embedding row
// decode.  Reference: the decode megakernel real_llm.rs:6794-7403 and its helpers.
//
// Every wave-level FWHT uses the butterfly order of hadamard.rs:83-97, so where the
// reference's inputs are reproduced exactly, rotations and int8 codes are bit-exact.
// Sums (inv_rms, softmax denominators, attention accumulations) are tree/parallel
// reductions: those match the reference to fp32 rounding.
#include <float.h>
#include <math.h>

#include <algorithm>

#include "k2t_device.h"
#include "k2t_expf.h"
#include "k2t_internal.h"
#include "k2t_kv_dev.h"

namespace k2t {

// ---------------------------------------------------------------- RMSNorm + FWHT + int8
// One wave per (token, four chunks): the wave computes inv_rms = 1/sqrt(mean(x^2) + eps)
// (real_llm.rs:6929) from the whole row (L2-resident, a few KB) in a fixed order, then
// runs populate_rmsnorm_fwht (simd_lut.rs:2970-2997) on its four chunks at once: lanes
// 16k .. 16k + 15 hold chunk 4 blockIdx.x + k, four consecutive elements each
// (rotate_quant4, the arithmetic of fwht_lane + quant_chunk_store in that layout).  A
// group past the last chunk repeats it and stores nothing.
__global__ __launch_bounds__(64) void rmsnorm_act_kernel(const float *__restrict__ x, const float *__restrict__ w,
                                                         float eps, int K, int8_t *__restrict__ q,
                                                         float *__restrict__ scales, int32_t *__restrict__ sums,
                                                         ActTiles tiles, const uint64_t *__restrict__ signs) {
    const uint32_t lane = threadIdx.x, sl = lane & 15u;
    const int nc = K / 64, tok = blockIdx.y;
    const int cg = 4 * (int)blockIdx.x + (int)(lane >> 4), c = min(cg, nc - 1);
    const float *xt = x + (size_t)tok * K;
    const float4 xv = *reinterpret_cast<const float4 *>(xt + c * 64 + 4 * sl);
    const float4 wv = *reinterpret_cast<const float4 *>(w + c * 64 + 4 * sl);
    const uint64_t mask = signs[c];
    const float ss = row_sumsq_wave(xt, K, lane);
    const float inv_rms = 1.0f / sqrtf(ss / (float)K + eps);
    float v[4] = {(xv.x * inv_rms) * wv.x, (xv.y * inv_rms) * wv.y, (xv.z * inv_rms) * wv.z, (xv.w * inv_rms) * wv.w};
    const Chunk4 r = rotate_quant4(v, mask, sl);
    if (cg < nc) chunk4_store(r, sl, tok, c, nc, q, scales, sums, tiles.xt, tiles.st, tiles.ut);
}

void launch_rmsnorm_act(hipStream_t st, const uint64_t *signs, const float *x, const float *w, float eps, int K,
                        int ntok, int8_t *q, float *s, int32_t *sums, ActTiles tiles) {
    if (K % 64 != 0 || K / 64 > kSignBlocks || !signs) throw Error(K2T_E_INTERNAL, "rmsnorm_act shape");
    hipLaunchKernelGGL(rmsnorm_act_kernel, dim3((K / 64 + 3) / 4, ntok), dim3(64), 0, st, x, w, eps, K, q, s, sums,
                       tiles, signs);
    hip_check(hipGetLastError(), "rmsnorm_act launch");
}

// ---------------------------------------------------------------- qkv post-processing
// One wave per (token, head) of the fused qkv output [q heads | k heads | v heads]:
// optional bias, RoPE on q and k (real_llm.rs:9328-9361, half-split), then k and v go
// through store_hadamard_q8_head (real_llm.rs:8282-8365) into the cache slot of `pos`.
// Positions are read from `pos_dev` (+ token index) so a captured graph can replay.
__global__ __launch_bounds__(64) void qkv_post_kernel(float *__restrict__ qkv, const float *__restrict__ bias,
                                                      const float *__restrict__ qn, const float *__restrict__ kn,
                                                      float eps, const float *__restrict__ rope,
                                                      const int *__restrict__ pos_dev, int nq, int nkv, int hd,
                                                      int row_stride, int layer, KvRing kr, int8_t *__restrict__ kq,
                                                      int8_t *__restrict__ vq, float *__restrict__ ks,
                                                      float *__restrict__ vs, int exact) {
    const uint32_t lane = threadIdx.x;
    const int head = blockIdx.x, tok = blockIdx.y;
    const int pos = pos_dev[0] + tok;
    float *h = qkv + (size_t)tok * row_stride + (size_t)head * hd;
    const int nb = hd / 64;  // 1 or 2 blocks; lane holds element lane (+64)
    float v0, v1;
    head_post(h, head, nq, nkv, hd, bias, qn, kn, eps, rope, pos, lane, v0, v1, exact != 0);
    if (head < nq) {
        h[lane] = v0;
        if (nb > 1) h[64 + lane] = v1;
        return;
    }
    const bool is_k = head < nq + nkv;
    const int kvh = is_k ? head - nq : head - nq - nkv;
    const size_t slot = ((size_t)layer * nkv + kvh) * kr.cap + ring_slot(kr, pos);
    const float r0 = fwht_lane(v0, 0, lane);
    const float r1 = nb > 1 ? fwht_lane(v1, 1, lane) : 0.0f;
    kv_store_head(r0, r1, nb, lane, kr.bits, hd, slot, is_k ? kq : vq, is_k ? ks : vs);
}

// Standalone KV store of n rotated-domain inputs (post-RoPE heads) into slots 0..n-1.
__global__ __launch_bounds__(64) void kv_store_kernel(const float *__restrict__ heads, int hd, int bits,
                                                      int8_t *__restrict__ qbuf, float *__restrict__ sbuf) {
    const uint32_t lane = threadIdx.x;
    const int nb = hd / 64;
    const float *h = heads + (size_t)blockIdx.x * hd;
    const float r0 = fwht_lane(h[lane], 0, lane);
    const float r1 = nb > 1 ? fwht_lane(h[64 + lane], 1, lane) : 0.0f;
    kv_store_head(r0, r1, nb, lane, bits, hd, blockIdx.x, qbuf, sbuf);
}

void launch_kv_store(hipStream_t st, const float *heads, int n, int hd, int bits, int8_t *qbuf, float *sbuf) {
    hipLaunchKernelGGL(kv_store_kernel, dim3(n), dim3(64), 0, st, heads, hd, bits, qbuf, sbuf);
    hip_check(hipGetLastError(), "kv_store launch");
}

void launch_qkv_post(hipStream_t st, float *qkv, const float *bias, const float *qn, const float *kn, float eps,
                     const float *rope, const int *pos_dev, int nq, int nkv, int hd, int ntok, int layer, KvRing kr,
                     int8_t *kq, int8_t *vq, float *ks, float *vs, bool exact) {
    hipLaunchKernelGGL(qkv_post_kernel, dim3(nq + 2 * nkv, ntok), dim3(64), 0, st, qkv, bias, qn, kn, eps, rope,
                       pos_dev, nq, nkv, hd, (nq + 2 * nkv) * hd, layer, kr, kq, vq, ks, vs, exact ? 1 : 0);
    hip_check(hipGetLastError(), "qkv_post launch");
}

// ---------------------------------------------------------------- attention
// Flash-decoding over the int8 Hadamard KV cache (causal_gqa_group_q8, real_llm.rs:8471-8594):
// the query head is rotated and quantized like a KV head, s_t = float(q.k_t)*ks_t*(qs*scale),
// softmax, o = sum_t p_t*vs_t*v_t in the rotated domain.  Grid (q head, split, token); each
// workgroup writes (max, sum, o[hd]) for its KV range; attn_merge_kernel combines them.
constexpr int kAttnSplitLen = 256;
// Contexts up to kAttnWhole positions run one 1024-thread workgroup per (q head, token)
// over every position, and that workgroup also writes the o_proj activation (FINAL): no
// merge kernel.
constexpr int kAttnWhole = 1024;
// Batches whose every token attends to at most this many positions (prefill of a short
// prompt) run a kAttnSmall-thread version of the whole-context kernel.
constexpr int kAttnSmall = 256;
// Span merges over at most this many spans issue all their loads at once.
constexpr int kMergeOneShot = 32;

// Sum of n (a power of two) values in a fixed pairwise tree.
__device__ __forceinline__ float tree_sum(const float *v, int n) {
    float t[16];
    for (int i = 0; i < n; i++) t[i] = v[i];
    for (int w = n; w > 1; w >>= 1)
        for (int i = 0; i < w / 2; i++) t[i] = t[2 * i] + t[2 * i + 1];
    return t[0];
}

// VORD >= NTH: the o partial sums use the position subsets of a VORD-thread workgroup
// (each thread then owns VORD / NTH of them), so a 256-thread launch over at most 256
// positions gives the 1024-thread kernel's results bit for bit.  RING: the cache is a
// sliding-window ring (positions map to slots through the window and ring arithmetic);
// without it index = position = slot, and the kernel carries none of that arithmetic
// (its modulo costs tens of instructions per position).
template <int NTH, bool FINAL, int VORD = NTH, bool RING = true>
__global__ __launch_bounds__(NTH) void attn_partial_kernel(const float *__restrict__ q, int q_stride,
                                                           int8_t *__restrict__ kq, int8_t *__restrict__ vq,
                                                           float *__restrict__ ks, float *__restrict__ vs,
                                                           const int *__restrict__ pos_dev, int layer, int nq, int nkv,
                                                           int hd, KvRing kr, float attn_scale, int nsplit,
                                                           AttnPost post, float *__restrict__ part,
                                                           float *__restrict__ out_f, int8_t *__restrict__ aq,
                                                           float *__restrict__ as, int32_t *__restrict__ asum,
                                                           ActTiles tiles) {
    constexpr int NW = NTH / 64;  // waves
    __shared__ __align__(16) int8_t qi[128];
    __shared__ __align__(16) int8_t kcur[128], vcur[128];  // current position's K / V (post.on)
    __shared__ float cur_s[4];                              // their scales (f32, or BF16 pairs)
    __shared__ float qas_s;
    __shared__ float sc[NTH];
    __shared__ float red[2 * NW];
    __shared__ float opart[VORD * 4];  // [position subset][column]: (VORD / (hd / 4)) * hd
    constexpr int SUBS = VORD / NTH;   // position subsets per thread
    static_assert(VORD % NTH == 0, "VORD must be a multiple of NTH");
    // XCD-aware order: workgroups are dispatched round-robin over the 8 XCDs by linear id,
    // so the q heads that share a KV head and a split get ids congruent mod 8 and run on
    // one XCD, where the K/V tile is fetched from HBM once and then hit in that XCD's L2.
    const int tok = blockIdx.z;
    int head, split;
    {
        const int lin = (int)blockIdx.x + (int)blockIdx.y * (int)gridDim.x;  // < nq * nsplit
        const int grp = nq / nkv, units = nkv * nsplit;                    // (kv head, split) tiles
        const int xcd = lin & 7, r = lin >> 3;
        const int nx = (units + 7) >> 3;  // tiles per XCD lane (the last XCDs may hold fewer)
        const int member = r / nx, ti = xcd + 8 * (r % nx);
        if ((nq * nsplit) % 8 == 0 && units % 8 == 0 && ti < units && member < grp) {
            head = (ti / nsplit) * grp + member;
            split = ti % nsplit;
        } else {
            head = (int)blockIdx.x;
            split = (int)blockIdx.y;
        }
    }
    const int seq = pos_dev[0] + tok + 1;
    const int act = RING ? active_len(kr, seq) : seq;  // attended positions: index idx -> slot of active_pos
    const int t0 = split * NTH, t1 = min(act, t0 + NTH);
    float *pp = part + ((size_t)(tok * nq + head) * nsplit + split) * (2 + hd);
    const uint32_t tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    if (t0 >= t1) {
        if (tid == 0) {
            pp[0] = -INFINITY;
            pp[1] = 0.0f;
        }
        if (tid < (uint32_t)hd) pp[2 + tid] = 0.0f;
        return;
    }
    const int kvh = head / (nq / nkv);
    const float *qh = q + (size_t)tok * q_stride + (size_t)head * hd;
    const int nb = hd / 64;
    // post.on (one token): q is the raw qkv row; this workgroup applies bias, QK-norm and
    // RoPE to its q head, and the workgroups whose split holds the current position build
    // its K / V (qkv_post's arithmetic) in LDS; the first q head of each KV group writes
    // them to the cache.  No workgroup reads the current position's slot from memory.
    const int cur = act - 1;
    const bool covers = post.on && t0 <= cur && cur < t1;
    if (covers && (wv == 1 || wv == 2)) {
        const int hh = wv == 1 ? nq + kvh : nq + nkv + kvh;
        float a0, a1;
        head_post(q + (size_t)tok * q_stride + (size_t)hh * hd, hh, nq, nkv, hd, post.bias, post.qn, post.kn,
                  post.eps, post.rope, seq - 1, lane, a0, a1);
        const float r0 = fwht_lane(a0, 0, lane);
        const float r1 = nb > 1 ? fwht_lane(a1, 1, lane) : 0.0f;
        kv_store_head(r0, r1, nb, lane, kr.bits, hd, 0, wv == 1 ? kcur : vcur, wv == 1 ? cur_s : cur_s + 2);
        if (head % (nq / nkv) == 0) {
            const size_t slot = ((size_t)layer * nkv + kvh) * kr.cap + (RING ? ring_slot(kr, seq - 1) : seq - 1);
            kv_store_head(r0, r1, nb, lane, kr.bits, hd, slot, wv == 1 ? kq : vq, wv == 1 ? ks : vs);
        }
    }
    if (wv == 0) {
        float qv0, qv1;
        if (post.on) {
            head_post(qh, head, nq, nkv, hd, post.bias, post.qn, post.kn, post.eps, post.rope, seq - 1, lane, qv0,
                      qv1);
        } else {
            qv0 = qh[lane];
            qv1 = nb > 1 ? qh[64 + lane] : 0.0f;
        }
        const float r0 = fwht_lane(qv0, 0, lane);
        const float r1 = nb > 1 ? fwht_lane(qv1, 1, lane) : 0.0f;
        const float mx = wave_max_f(fmaxf(fabsf(r0), fabsf(r1)));
        float qs = 0.0f;
        if (mx <= FLT_EPSILON) {
            qi[lane] = 0;
            if (nb > 1) qi[64 + lane] = 0;
        } else {
            const float inv = 127.0f / mx;
            qi[lane] = (int8_t)(int)rintf(r0 * inv);
            if (nb > 1) qi[64 + lane] = (int8_t)(int)rintf(r1 * inv);
            qs = mx / 127.0f;
        }
        if (lane == 0) qas_s = qs * attn_scale;
    }
    __syncthreads();
    const size_t base = ((size_t)layer * nkv + kvh) * kr.cap;
    const float qas = qas_s;
    // slot of the idx-th attended position (identity without a sliding window)
    auto slot_of = [&](int idx) -> size_t {
        return RING ? (size_t)ring_slot(kr, active_pos(kr, idx, seq)) : (size_t)idx;
    };
    // scores: one thread per position
    float smax = -INFINITY;
    float vscale = 0.0f;
    {
        const int t = t0 + (int)tid;
        if (t < t1 && kr.bits == 4) {
            // NF4 KV (causal_gqa_group_q4_or_window, real_llm.rs:8827-8849): per 64-block
            // dot of the codebook values with q, total += float(dot) * ks_g * qs
            const bool here = covers && t == cur;
            const size_t sl = base + slot_of(t);
            // (the current position from LDS, the others from the cache: each read states
            // its memory, so no select of the two pointers becomes a flat access)
            const uint8_t *k4 = reinterpret_cast<const uint8_t *>(kq) + sl * (size_t)(hd / 2);
            const uint16_t *k16 = reinterpret_cast<const uint16_t *>(ks) + sl * (size_t)nb;
            float s = 0.0f;
            for (int g = 0; g < nb; g++) {
                const uint4 *kp = reinterpret_cast<const uint4 *>(k4 + g * 32);
                const uint32_t *qw = reinterpret_cast<const uint32_t *>(qi + g * 64);
                int dot = 0;
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const uint4 a = here ? lds_read16_now(kcur + g * 32 + h * 16) : ld_global(kp + h);
                    const uint32_t w4[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const uint32_t d = w4[j];
                        const uint32_t lo = lut16(d & 0x07070707u, bit3_mask(d), kNf4Cb0, kNf4Cb1, kNf4Cb2, kNf4Cb3);
                        const uint32_t hi =
                            lut16((d >> 4) & 0x07070707u, bit7_mask(d), kNf4Cb0, kNf4Cb1, kNf4Cb2, kNf4Cb3);
                        dot = __builtin_amdgcn_sdot4((int)lo, (int)qw[h * 8 + j], dot, false);
                        dot = __builtin_amdgcn_sdot4((int)hi, (int)qw[h * 8 + 4 + j], dot, false);
                    }
                }
                const uint16_t kb = here ? ld_lds(reinterpret_cast<const uint16_t *>(cur_s) + g) : ld_global(k16 + g);
                s += ((float)dot * __uint_as_float((uint32_t)kb << 16)) * qas;
            }
            vscale = 1.0f;  // the V scales are per 64-block: applied in the V sum
            sc[tid] = s;
            smax = s;
        } else if (t < t1) {
            const bool here = covers && t == cur;
            const size_t sl = base + slot_of(t);
            const uint4 *krow = reinterpret_cast<const uint4 *>(kq + sl * hd);
            const uint4 *qr = reinterpret_cast<const uint4 *>(qi);
            int dot[2] = {0, 0};
            for (int i = 0; i < hd / 16; i++) {
                const uint4 a = here ? lds_read16_now(kcur + 16 * i) : ld_global(krow + i), b = qr[i];
                int d = dot[i >> 2];
                d = __builtin_amdgcn_sdot4((int)a.x, (int)b.x, d, false);
                d = __builtin_amdgcn_sdot4((int)a.y, (int)b.y, d, false);
                d = __builtin_amdgcn_sdot4((int)a.z, (int)b.z, d, false);
                d = __builtin_amdgcn_sdot4((int)a.w, (int)b.w, d, false);
                dot[i >> 2] = d;
            }
            const float kscale = here ? ld_lds(cur_s) : ld_global(ks + sl);
            vscale = here ? ld_lds(cur_s + 2) : ld_global(vs + sl);
            float s;
            if (kr.window > 0 && hd == 128)  // per-64-block terms (causal_gqa_group_q4_or_window, 8823-8868)
                s = ((float)dot[0] * kscale) * qas + ((float)dot[1] * kscale) * qas;
            else  // causal_gqa_group_q8 (8471-8594): one dot per head
                s = ((float)(dot[0] + dot[1]) * kscale) * qas;
            sc[tid] = s;
            smax = s;
        }
    }
    smax = wave_max_f(smax);
    if (lane == 0) red[wv] = smax;
    __syncthreads();
    float m = red[0];
    for (int w = 1; w < NW; w++) m = fmaxf(m, red[w]);
    float psum = 0.0f;
    if (t0 + (int)tid < t1) {
        const float p = expf(sc[tid] - m);
        sc[tid] = p * vscale;  // p_t * vs_t
        psum = p;
    }
    psum = wave_sum_f(psum);
    __syncthreads();
    if (lane == 0) red[NW + wv] = psum;
    // o partial: thread = (position subset ps, 4-column group cg); a dword of V per
    // position, loads batched 4 deep; the position subsets are added in a fixed order.
    const int n = t1 - t0;
    const int ncg = hd / 4;            // 16 or 32 column groups
    const int nps = VORD / ncg;        // position subsets
    const int cg = (int)tid % ncg, ps0 = (int)tid / ncg;
    const int8_t *vcol = vq + base * hd + cg * 4;
#pragma unroll
    for (int sub = 0; sub < SUBS; sub++) {
    const int ps = ps0 + sub * (NTH / ncg);
    float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
    int i = ps;
    if (kr.bits == 4) {
        // NF4 V: this thread's 4 columns are one nibble half of 4 bytes of block g
        const int c0 = cg * 4, g = c0 >> 6, e0 = c0 & 63, hhalf = (e0 >> 5), i0 = e0 & 31;
        const uint32_t off = (uint32_t)(g * 32 + hhalf * 16 + (i0 & 15));
        const bool upper = i0 >= 16;
        const uint8_t *v4 = reinterpret_cast<const uint8_t *>(vq) + base * (size_t)(hd / 2) + off;
        const uint16_t *v16 = reinterpret_cast<const uint16_t *>(vs) + base * (size_t)nb + g;
        for (; i < n; i += nps) {
            const bool here = covers && t0 + i == cur;
            const size_t sl = slot_of(t0 + i);
            const uint32_t d = here ? ld_lds(reinterpret_cast<const uint32_t *>(reinterpret_cast<const uint8_t *>(vcur) + off))
                                    : ld_global(reinterpret_cast<const uint32_t *>(v4 + sl * (size_t)(hd / 2)));
            const uint32_t c = upper ? lut16((d >> 4) & 0x07070707u, bit7_mask(d), kNf4Cb0, kNf4Cb1, kNf4Cb2, kNf4Cb3)
                                     : lut16(d & 0x07070707u, bit3_mask(d), kNf4Cb0, kNf4Cb1, kNf4Cb2, kNf4Cb3);
            const uint16_t vsb = here ? ld_lds(reinterpret_cast<const uint16_t *>(cur_s + 2) + g) : ld_global(v16 + sl * (size_t)nb);
            const float wt = sc[i] * __uint_as_float((uint32_t)vsb << 16);
            a0 = fmaf(wt, (float)(int8_t)(c & 0xFF), a0);
            a1 = fmaf(wt, (float)(int8_t)((c >> 8) & 0xFF), a1);
            a2 = fmaf(wt, (float)(int8_t)((c >> 16) & 0xFF), a2);
            a3 = fmaf(wt, (float)(int8_t)((c >> 24) & 0xFF), a3);
        }
    }
    // the span kernel (32 positions per thread at hd 128) batches 8 deep (30B-A3B decode
    // +1.7% over 4; 16 was slower), the whole-context kernel 4 deep (8: decode unchanged,
    // prefill -12%; 16 slower)
    constexpr int kVB = FINAL ? 4 : 8;
    for (; kr.bits != 4 && i + (kVB - 1) * nps < n; i += kVB * nps) {
        int vv[kVB];
        float ww[kVB];
#pragma unroll
        for (int u = 0; u < kVB; u++) {
            const int idx = t0 + i + u * nps;
            vv[u] = covers && idx == cur ? ld_lds(reinterpret_cast<const int *>(vcur + cg * 4))
                                         : ld_global(reinterpret_cast<const int *>(vcol + slot_of(idx) * hd));
            ww[u] = sc[i + u * nps];
        }
#pragma unroll
        for (int u = 0; u < kVB; u++) {
            a0 = fmaf(ww[u], (float)(int8_t)(vv[u] & 0xFF), a0);
            a1 = fmaf(ww[u], (float)(int8_t)((vv[u] >> 8) & 0xFF), a1);
            a2 = fmaf(ww[u], (float)(int8_t)((vv[u] >> 16) & 0xFF), a2);
            a3 = fmaf(ww[u], (float)(int8_t)((vv[u] >> 24) & 0xFF), a3);
        }
    }
    for (; kr.bits != 4 && i < n; i += nps) {
        const int v = covers && t0 + i == cur ? ld_lds(reinterpret_cast<const int *>(vcur + cg * 4))
                                              : ld_global(reinterpret_cast<const int *>(vcol + slot_of(t0 + i) * hd));
        const float wt = sc[i];
        a0 = fmaf(wt, (float)(int8_t)(v & 0xFF), a0);
        a1 = fmaf(wt, (float)(int8_t)((v >> 8) & 0xFF), a1);
        a2 = fmaf(wt, (float)(int8_t)((v >> 16) & 0xFF), a2);
        a3 = fmaf(wt, (float)(int8_t)((v >> 24) & 0xFF), a3);
    }
    float *op = opart;  // [nps][hd]
    op[ps * hd + cg * 4 + 0] = a0;
    op[ps * hd + cg * 4 + 1] = a1;
    op[ps * hd + cg * 4 + 2] = a2;
    op[ps * hd + cg * 4 + 3] = a3;
    }
    __syncthreads();
    if constexpr (FINAL) {
        // One span covers every position: attn_merge_kernel's arithmetic for one split
        // (its weight exp(m - m) is exactly 1), then ifwht64 per block and the FWHT +
        // int8 of the o_proj chunk (populate_chunk_fwht_raw(None), real_llm.rs:7060-7084).
        const float inv = 1.0f / tree_sum(red + NW, NW);
        if (tid < (uint32_t)hd) {
            float acc = opart[tid];
            for (int k = 1; k < nps; k++) acc += opart[k * hd + tid];
            sc[tid] = acc;  // the scores are no longer needed
        }
        __syncthreads();
        if ((int)wv < nb) {
            const float o = ifwht_lane(sc[wv * 64 + lane] * inv, (uint64_t)wv, lane);
            const size_t hbase = (size_t)tok * nq * hd + (size_t)head * hd;
            if (out_f) out_f[hbase + wv * 64 + lane] = o;
            if (aq) {
                const size_t c = (size_t)head * nb + wv, g = (size_t)tok * nq * nb + c;
                quant_chunk_store(fwht_lane(o, c, lane), lane, aq + g * 64, as + g, asum + g, tiles.xt, tiles.st,
                                  tiles.ut, tok, (int)c, nq * nb);
            }
        }
        return;
    }
    if (tid == 0) {
        pp[0] = m;
        pp[1] = tree_sum(red + NW, NW);
    }
    if (tid < (uint32_t)hd) {
        float acc = opart[tid];
        for (int k = 1; k < nps; k++) acc += opart[k * hd + tid];
        pp[2 + tid] = acc;
    }
}

// ---------------------------------------------------------------- prefill attention on the matrix cores
// A batch of 16 or more tokens over the int8 cache without a window (fast mode).  One
// workgroup per (q head, 16-token query block), 4 waves; wave w takes the 16-position
// tiles w, w + 4, ... of the positions the block attends to, with an online softmax,
// and the workgroup merges its waves' (max, sum, o) in wave order at the end.  Per tile:
//  - scores: v_mfma_i32_16x16x64_i8 with A = K (16 positions x 64 dims, lane l row l%16)
//    and B = the block's int8 q heads (64 dims x 16 tokens): exact integer dots, lane l
//    holding positions 4(l/16) + r of token l%16; s = (float(dot) * ks) * (qs * scale) as
//    causal_gqa_group_q8 (real_llm.rs:8471-8594);
//  - o: four v_mfma_f32_16x16x4f32 per 16 dims, the r-th over positions r, 4 + r, 8 + r,
//    12 + r, with A = V^T (lane l: dim l%16, position 4(l/16) + r) and B = (p * vs)^T
//    (lane l: position 4(l/16) + r, token l%16), which is the score tile's own layout,
//    so no lane exchange is needed; o^T accumulates in fp32 (lane l: dims 4(l/16) + r
//    of token l%16).  (fp16 weights in a 16x16x16 MFMA cost a quarter of the MFMAs but
//    left 2-layer logits at cosine 0.99989 against the oracle, under the fast path's
//    0.9999.)
// The sums run in tile order: the outputs are close to, not bit-equal with, the one-token
// kernel's, which a batch of fewer than 16 tokens still uses.  q quantization and the
// closing ifwht64 / FWHT + int8 of the o_proj chunk are the whole-context kernel's.
typedef float v4f __attribute__((ext_vector_type(4)));
typedef int v4i_t __attribute__((ext_vector_type(4)));

#ifndef K2T_PATT_WAVES
#define K2T_PATT_WAVES 4
#endif
constexpr int kPattWaves = K2T_PATT_WAVES;  // waves per (q head, 16-token block) workgroup

template <int HD>
__global__ __launch_bounds__(64 * kPattWaves) void attn_prefill_mfma_kernel(const float *__restrict__ q, int q_stride,
                                                                const int8_t *__restrict__ kq,
                                                                const int8_t *__restrict__ vq,
                                                                const float *__restrict__ ks,
                                                                const float *__restrict__ vs,
                                                                const int *__restrict__ pos_dev, int layer, int nq,
                                                                int nkv, int cap, float attn_scale, int ntok,
                                                                float *__restrict__ out_f, int8_t *__restrict__ aq,
                                                                float *__restrict__ as, int32_t *__restrict__ asum,
                                                                ActTiles tiles) {
    constexpr int NB = HD / 64;  // 64-dim blocks
    constexpr int DB = HD / 16;  // 16-dim output blocks
    __shared__ __align__(16) int8_t qi[16][HD];
    __shared__ float qas_s[16];
    constexpr int AW = kPattWaves;
    __shared__ float wm[AW][16], wl[AW][16];  // per wave and token: running max and sum
    __shared__ __align__(16) float wo[AW][16][HD + 4];  // per wave: o[token][dim] (padded rows)
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int head = blockIdx.x, tb = blockIdx.y, t0 = tb * 16;
    const int kvh = head / (nq / nkv);
    const int pos0 = pos_dev[0];
    // 1. the block's q heads rotated and quantized (as the whole-context kernel): wave w
    //    takes tokens w, w + 4, w + 8, w + 12 (tokens past the batch repeat the last one)
    for (int j = (int)wave; j < 16; j += AW) {
        const int tok = min(t0 + j, ntok - 1);
        const float *qh = q + (size_t)tok * q_stride + (size_t)head * HD;
        const float r0 = fwht_lane(qh[lane], 0, lane);
        const float r1 = NB > 1 ? fwht_lane(qh[64 + lane], 1, lane) : 0.0f;
        const float mx = wave_max_f(fmaxf(fabsf(r0), fabsf(r1)));
        float qs = 0.0f;
        if (mx <= FLT_EPSILON) {
            qi[j][lane] = 0;
            if (NB > 1) qi[j][64 + lane] = 0;
        } else {
            const float inv = 127.0f / mx;
            qi[j][lane] = (int8_t)(int)rintf(r0 * inv);
            if (NB > 1) qi[j][64 + lane] = (int8_t)(int)rintf(r1 * inv);
            qs = mx / 127.0f;
        }
        if (lane == 0) qas_s[j] = qs * attn_scale;
    }
    __syncthreads();
    const uint32_t li = lane & 15u, lg = lane >> 4;
    // B operand of the score MFMA: token li's dims 64k + 16 lg .. + 15
    v4i_t qb[NB];
#pragma unroll
    for (int k = 0; k < NB; k++) {
        const int4 v = *reinterpret_cast<const int4 *>(&qi[li][64 * k + 16 * lg]);
        qb[k] = v4i_t{v.x, v.y, v.z, v.w};
    }
    const float qas = qas_s[li];
    const int my_tok = t0 + (int)li;          // this lane's token (column of every tile)
    const int my_last = pos0 + my_tok;        // the last position it attends to
    const int n_att = pos0 + min(t0 + 16, ntok);  // positions any token of the block attends to
    const size_t base = ((size_t)layer * nkv + kvh) * cap;
    float m = -INFINITY, l = 0.0f;
    v4f o[DB];
#pragma unroll
    for (int b = 0; b < DB; b++) o[b] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    // A tile's loads (K rows, scales, V words; rows past n_att re-read the last one) are
    // issued a tile ahead: two register sets alternate, so the next tile's loads are in
    // flight while this one computes.
    struct Tile {
        int4 kv[NB];
        float ksc[4], vsc[4];
        uint32_t vw[4][DB / 4];
    };
    auto load_tile = [&](int p0, Tile &T) {
        const int prow = min(p0 + (int)li, n_att - 1);  // K row of this lane (A operand)
#pragma unroll
        for (int k = 0; k < NB; k++)
            T.kv[k] = *reinterpret_cast<const int4 *>(kq + (base + prow) * HD + 64 * k + 16 * lg);
        const int pr = p0 + 4 * (int)lg;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int pc = min(pr + r, n_att - 1);
            T.ksc[r] = ks[base + pc];
            T.vsc[r] = vs[base + pc];
            const int8_t *vrow = vq + (base + pc) * HD + DB * li;
            if constexpr (DB == 8) {
                const uint2 d2 = *reinterpret_cast<const uint2 *>(vrow);
                T.vw[r][0] = d2.x;
                T.vw[r][DB / 4 - 1] = d2.y;
            } else {
                T.vw[r][0] = *reinterpret_cast<const uint32_t *>(vrow);
            }
        }
    };
    auto tile_step = [&](int p0, const Tile &T) {
        // scores of positions p0 + 4 lg + r for token li
        v4i_t acc = {0, 0, 0, 0};
#pragma unroll
        for (int k = 0; k < NB; k++)
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(v4i_t{T.kv[k].x, T.kv[k].y, T.kv[k].z, T.kv[k].w}, qb[k], acc,
                                                         0, 0, 0);
        const int pr = p0 + 4 * (int)lg;  // this lane's first position
        float sc[4];
        float tmax = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int p = pr + r;
            const bool live = p <= my_last && p < n_att;
            sc[r] = live ? ((float)acc[r] * T.ksc[r]) * qas : -INFINITY;
            tmax = fmaxf(tmax, sc[r]);
        }
        tmax = fmaxf(tmax, xor_lane(tmax, 16));
        tmax = fmaxf(tmax, xor_lane(tmax, 32));
        const float mn = fmaxf(m, tmax);
        // (mn = -inf: every position so far masked; nothing accumulated yet)
        const float corr = mn == -INFINITY ? 1.0f : expf(m - mn);
        float psum = 0.0f, w[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float pw = sc[r] == -INFINITY ? 0.0f : expf(sc[r] - mn);
            psum += pw;
            w[r] = pw * T.vsc[r];
        }
        psum += xor_lane(psum, 16);
        psum += xor_lane(psum, 32);
        l = l * corr + psum;
        m = mn;
        // o^T += V^T * (p vs)^T: dim block b holds dims DB m + b (m = 0..15), so A lane l =
        // dim DB li + b, position pr + r, and the lane's DB dims of a position are one load
#pragma unroll
        for (int b = 0; b < DB; b++) {
            o[b] = o[b] * corr;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float va = (float)(int8_t)((T.vw[r][b >> 2] >> (8 * (b & 3))) & 0xFFu);
                o[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(va, w[r], o[b], 0, 0, 0);
            }
        }
    };
    Tile tile_a, tile_b;
    constexpr int TS = 16 * AW;  // a wave's tile stride
    int p0 = 16 * (int)wave;
    load_tile(p0, tile_a);
    for (; p0 < n_att; p0 += 2 * TS) {
        load_tile(p0 + TS, tile_b);
        tile_step(p0, tile_a);
        if (p0 + TS >= n_att) break;
        load_tile(p0 + 2 * TS, tile_a);
        tile_step(p0 + TS, tile_b);
    }
    // 2. merge the waves in order: per token the largest max, then the rescaled sums
    if (lg == 0) {
        wm[wave][li] = m;
        wl[wave][li] = l;
    }
#pragma unroll
    for (int b = 0; b < DB; b++)
#pragma unroll
        for (int r = 0; r < 4; r++) wo[wave][li][DB * (4 * lg + r) + b] = o[b][r];
    // Hadamard sign masks: ifwht64 of blocks 0 .. NB-1, and the o_proj chunks' rotations
    uint64_t mi[NB], mc[NB];
#pragma unroll
    for (int blk = 0; blk < NB; blk++) {
        mi[blk] = __ballot(hadamard_sign_bit((uint64_t)blk, lane) != 0u);
        mc[blk] = __ballot(hadamard_sign_bit((uint64_t)(head * NB + blk), lane) != 0u);
    }
    __syncthreads();
    // Four tokens per wave (the first four waves): lanes 16k .. 16k + 15 hold token 4w + k,
    // four consecutive elements each (butterflies_slice4 / rotate_quant4: the
    // one-element-per-lane ifwht_lane, fwht_lane and quant_chunk_store arithmetic in that
    // layout).
    if (wave < 4) {
        const uint32_t sl = lane & 15u;
        const int j = 4 * (int)wave + (int)lg, tok = t0 + j;
        float M = -INFINITY;
#pragma unroll
        for (int w2 = 0; w2 < AW; w2++) M = fmaxf(M, wm[w2][j]);
        float L = 0.0f, e[AW];
#pragma unroll
        for (int w2 = 0; w2 < AW; w2++) {
            e[w2] = wm[w2][j] == -INFINITY ? 0.0f : expf(wm[w2][j] - M);
            L = fmaf(wl[w2][j], e[w2], L);
        }
        const float inv = 1.0f / L;
        const bool live = tok < ntok;
        const size_t hbase = (size_t)tok * nq * HD + (size_t)head * HD;
#pragma unroll
        for (int blk = 0; blk < NB; blk++) {
            float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int w2 = 0; w2 < AW; w2++) {
                const float4 wq = *reinterpret_cast<const float4 *>(&wo[w2][j][64 * blk + 4 * sl]);
                v[0] = fmaf(wq.x, e[w2], v[0]);
                v[1] = fmaf(wq.y, e[w2], v[1]);
                v[2] = fmaf(wq.z, e[w2], v[2]);
                v[3] = fmaf(wq.w, e[w2], v[3]);
            }
#pragma unroll
            for (int jj = 0; jj < 4; jj++) v[jj] = v[jj] * inv;
            butterflies_slice4(v, sl);
            const uint32_t sb = (uint32_t)(mi[blk] >> (4u * sl)) & 0xFu;
#pragma unroll
            for (int jj = 0; jj < 4; jj++) v[jj] = flip_sign(v[jj] * 0.125f, (sb >> jj) & 1u);
            if (out_f && live)
                *reinterpret_cast<float4 *>(out_f + hbase + 64 * blk + 4 * sl) = make_float4(v[0], v[1], v[2], v[3]);
            if (aq) {
                const int c = head * NB + blk;
                const Chunk4 r = rotate_quant4(v, mc[blk], sl);
                if (live) chunk4_store(r, sl, tok, c, nq * NB, aq, as, asum, tiles.xt, tiles.st, tiles.ut);
            }
        }
    }
}

// Combines the splits of one (token, q head), applies ifwht64 (real_llm.rs:8588-8592), and
// optionally re-rotates each 64-block with its o_proj chunk index and quantizes it
// (populate_chunk_fwht_raw(None), real_llm.rs:7060-7084) -> the o_proj activation.
// One wave; pp holds the `ns` splits of this (token, head), each {max, sum, o[hd]}.
template <int ONESHOT>
__device__ __forceinline__ void merge_head(const float *pp, int ns, int nq, int hd, int head, int tok, uint32_t lane,
                                           float *__restrict__ out_f, int8_t *__restrict__ aq, float *__restrict__ as,
                                           int32_t *__restrict__ asum, ActTiles tiles = ActTiles{}) {
    static_assert(ONESHOT <= 64, "one split per lane");
    const int nb = hd / 64;
    float L = 0.0f, o0 = 0.0f, o1 = 0.0f;
    if (ns <= ONESHOT) {
        // Every load in one round trip: split s's maximum and sum in lane s, and this
        // lane's columns of every split; then the same arithmetic, in split order, as the
        // general path below.
        const bool mine = (int)lane < ns;
        const float mv = mine ? pp[(size_t)lane * (2 + hd)] : -INFINITY;
        const float lm = mine ? pp[(size_t)lane * (2 + hd) + 1] : 0.0f;
        // (every load unconditional, from split min(u, ns - 1), and o1 only used when
        // nb > 1: a load under a branch whose other path writes its register made the
        // compiler wait for each load before the next)
        const int off1 = nb > 1 ? 2 + 64 + (int)lane : 2 + (int)lane;
        float v0[ONESHOT], v1[ONESHOT];
#pragma unroll
        for (int u = 0; u < ONESHOT; u++) {
            const float *ps = pp + (size_t)min(u, ns - 1) * (2 + hd);
            v0[u] = ps[2 + lane];
            v1[u] = ps[off1];
        }
        const float M = wave_max_f(mv);
        const float em = mine ? expf(mv - M) : 0.0f;
#pragma unroll
        for (int u = 0; u < ONESHOT; u++) {
            if (u < ns) {
                const float e = lane_val(em, u);
                L = fmaf(lane_val(lm, u), e, L);
                o0 = fmaf(v0[u], e, o0);
                o1 = fmaf(v1[u], e, o1);
            }
        }
    } else {
        // Split maxima and sums one split per lane (loads in flight together), then the
        // rescaled sums in split order.
        const int off1 = nb > 1 ? 2 + 64 + (int)lane : 2 + (int)lane;
        float M = -INFINITY;
        for (int s = (int)lane; s < ns; s += 64) M = fmaxf(M, pp[(size_t)s * (2 + hd)]);
        M = wave_max_f(M);
        for (int s0 = 0; s0 < ns; s0 += 64) {
            const int s = s0 + (int)lane;
            const float em = s < ns ? expf(pp[(size_t)s * (2 + hd)] - M) : 0.0f;
            const float lm = s < ns ? pp[(size_t)s * (2 + hd) + 1] : 0.0f;
            const int cnt = min(64, ns - s0);
            for (int j0 = 0; j0 < cnt; j0 += 8) {
                float v0[8], v1[8];
    #pragma unroll
                for (int u = 0; u < 8; u++) {  // (unconditional, as above)
                    const float *ps = pp + (size_t)(s0 + min(j0 + u, cnt - 1)) * (2 + hd);
                    v0[u] = ps[2 + lane];
                    v1[u] = ps[off1];
                }
    #pragma unroll
                for (int u = 0; u < 8; u++) {
                    if (j0 + u >= cnt) break;
                    const float e = lane_val(em, j0 + u);
                    L = fmaf(lane_val(lm, j0 + u), e, L);
                    o0 = fmaf(v0[u], e, o0);
                    o1 = fmaf(v1[u], e, o1);
                }
            }
        }
    }
    const float inv = 1.0f / L;
    o0 = ifwht_lane(o0 * inv, 0, lane);
    if (nb > 1) o1 = ifwht_lane(o1 * inv, 1, lane);
    const size_t hbase = (size_t)tok * nq * hd + (size_t)head * hd;
    if (out_f) {
        out_f[hbase + lane] = o0;
        if (nb > 1) out_f[hbase + 64 + lane] = o1;
    }
    if (aq) {
        const int nc_tok = nq * nb;  // o_proj input chunks per token
        const size_t c0 = (size_t)head * nb;
        const size_t g0 = (size_t)tok * nc_tok + c0;
        quant_chunk_store(fwht_lane(o0, c0, lane), lane, aq + g0 * 64, as + g0, asum + g0, tiles.xt, tiles.st,
                          tiles.ut, tok, (int)c0, nc_tok);
        if (nb > 1)
            quant_chunk_store(fwht_lane(o1, c0 + 1, lane), lane, aq + (g0 + 1) * 64, as + g0 + 1, asum + g0 + 1, tiles.xt,
                              tiles.st, tiles.ut, tok, (int)c0 + 1, nc_tok);
    }
}

__global__ __launch_bounds__(64) void attn_merge_kernel(const float *__restrict__ part, int nq, int hd, int nsplit,
                                                        int span_len, KvRing kr, const int *__restrict__ pos_dev,
                                                        float *__restrict__ out_f,
                                                        int8_t *__restrict__ aq, float *__restrict__ as,
                                                        int32_t *__restrict__ asum, ActTiles tiles) {
    const int head = blockIdx.x, tok = blockIdx.y;
    const int act = active_len(kr, pos_dev[0] + tok + 1);
    const int ns = min(nsplit, (act + span_len - 1) / span_len);
    merge_head<kMergeOneShot>(part + (size_t)(tok * nq + head) * nsplit * (2 + hd), ns, nq, hd, head, tok, threadIdx.x,
                              out_f, aq, as, asum, tiles);
}

// Long-context decode attention for grouped queries (int8 KV, no window), one launch.
// Span workgroups, one per (KV head, span of kGqaSpan positions, token), score all
// G = nq / nkv q heads of the group, so each K / V tile is read from memory once instead
// of once per q head.  The tile is copied into LDS by direct-to-LDS loads issued first;
// meanwhile each wave applies bias / QK-norm / RoPE and the Hadamard int8 quantization to
// one q head (and, in the span holding the current position, waves 0 and 1 build that
// position's K / V and store them in the cache).  Per head: s_t = float(q8 . k8_t) * ks_t *
// (qs * scale) as causal_gqa_group_q8 (real_llm.rs:8471-8594), the span's maximum m and
// sum of exp(s_t - m), and o = sum_t (exp(s_t - m) * vs_t) * v8_t, each V element
// converted once for all G heads.  A span workgroup publishes its partials as
// {payload, epoch} words (one agent-scope atomic store each).  Merge workgroups, one per
// (KV head, q head, token), come first in dispatch order and poll (bounded) the words of
// their head's spans until every one carries this launch's epoch, then combine the spans
// (global maximum, exp-weighted sums in span order), apply ifwht64 (real_llm.rs:8588-8592),
// and write the o_proj activation (populate_chunk_fwht_raw(None), real_llm.rs:7060-7084).
// The epoch is one more than the last launch's; the last merge workgroup to finish
// advances it, so the words never need clearing.
#ifndef K2T_GQA_SPAN
#define K2T_GQA_SPAN 128
#endif
constexpr int kGqaSpan = K2T_GQA_SPAN;  // 64 or 128
constexpr int kGqaThreads = 512;
constexpr int kGqaMaxGroup = 8;
// q heads per span workgroup (8, or 4 in a measurement build): a group of more q heads
// than this is split over ceil(G / heads) span workgroups of each span, which read the
// same K / V tile.  Splitting config 5's 8 heads over two workgroups of 4 measured slower
// (417.5 -> 391.7 tok/s: twice the span workgroups and tile reads for half the work each).
#ifndef K2T_GQA_HEADS
#define K2T_GQA_HEADS 8
#endif
constexpr int kGqaHeads = K2T_GQA_HEADS;
// Scores and o sums on the matrix cores (needs one 16-position tile per wave: 128-position
// spans, 8 waves); 0 in a measurement build keeps the dot-product form.
#ifndef K2T_GQA_MFMA
#define K2T_GQA_MFMA 1
#endif
constexpr bool kGqaMfma = K2T_GQA_MFMA != 0 && kGqaSpan == 16 * (kGqaThreads / 64);

#ifdef K2T_GQA_TRACE
// Measurement builds only: wall-clock stamps of layer 0's workgroups, 8 per (KV head, row).
__device__ unsigned long long g_gqa_trace[8 * 128 * 8];
#define GQA_TR(k)                                                                                  \
    do {                                                                                           \
        if (layer == 0 && threadIdx.x == 0 && blockIdx.y < 128 && blockIdx.x < 8)                 \
            g_gqa_trace[((size_t)blockIdx.x * 128 + blockIdx.y) * 8 + (k)] = wall_clock64();       \
    } while (0)
#else
#define GQA_TR(k) \
    do {          \
    } while (0)
#endif

struct GqaArgs {
    const float *q;
    int q_stride;
    int8_t *kq, *vq;
    float *ks, *vs;
    const int *pos_dev;
    int layer, nq, nkv;
    KvRing kr;
    float attn_scale;
    int nspan;
    int hsplit;  // span workgroups per span (each scores SH of the group's q heads)
    AttnPost post;
    unsigned long long *words;  // [token][q head][nspan][2 + hd] {payload, epoch} span words
    unsigned int *cnt;          // {epoch of the last launch, merge workgroups done}
    int *err;
    unsigned int spin_limit;
    float *out_f;
    int8_t *aq;
    float *as;
    int32_t *asum;
};

// SH: q heads per span workgroup (the group's G heads are split over ceil(G / SH) span
// workgroups of each span, which read the same K / V tile).
// MF: steps 3-5 on the matrix cores (see below).
template <int HD, int SH, bool MF>
__global__ __launch_bounds__(kGqaThreads) void attn_gqa_kernel(GqaArgs A) {
    constexpr int P = kGqaSpan, NTH = kGqaThreads, GM = SH;
    constexpr int PW = P / 64, HW = NTH / 64 / PW;  // waves per 64 positions, heads per pass
    static_assert(P % 64 == 0 && GM % HW == 0 && GM <= kGqaMaxGroup, "span shape");
    // K and V tiles [position][hd] (the first half); after the o sums the whole array holds
    // the position subsets' partial sums
    constexpr int kTiles = 2 * P * 128 > NTH * 4 * GM * 4 ? 2 * P * 128 : NTH * 4 * GM * 4;
    __shared__ __align__(16) int8_t tiles[kTiles];
    __shared__ float kst[P], vst[P];
    __shared__ __align__(16) int8_t qi[GM * 128];
    __shared__ float qas[GM];
    __shared__ __align__(16) float sc[P * GM];  // exp(s_t - m) * vs_t per (position, head)
    __shared__ float red_m[GM][MF ? NTH / 64 : PW], red_l[GM][MF ? NTH / 64 : PW];
    __shared__ __align__(16) int8_t kcur[128], vcur[128];
    __shared__ float cur_s[2];
    const int layer = A.layer, nq = A.nq, nkv = A.nkv;
    constexpr int hd = HD;
    const int G = nq / nkv;
    constexpr int nb = HD / 64;
    const int kvh = blockIdx.x, tok = blockIdx.z;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wv = tid >> 6;
    GQA_TR(0);
    const int seq = A.pos_dev[0] + tok + 1;
    const int nact = (seq + P - 1) / P;
    // this launch's epoch: one more than the last launch's (advanced by its last merge
    // workgroup, after every span workgroup of that launch had read it)
    const uint32_t ep = __hip_atomic_load(A.cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
    const size_t pstride = (size_t)A.nspan * (2 + hd);
    if ((int)blockIdx.y < G) {
        // ------------------------------------------------------------ merge workgroup
        // thread (span subset sub, 4-column group cg): spans sub, sub + nsub, ... ascending;
        // per span it polls the words {m, L, o[4 columns]} until they carry this epoch
        const int head = kvh * G + (int)blockIdx.y;
        const unsigned long long *pp = A.words + (size_t)(tok * nq + head) * pstride;
        constexpr int ncg = HD / 4, nsub = NTH / ncg;
        const int cg = (int)tid % ncg, sub = (int)tid / ncg;
        constexpr int kPre = 4;  // spans per thread polled together
        bool ok = true;
        auto poll = [&](int s, unsigned long long (&w)[6]) {
            // (the caller keeps s < nact)
            const unsigned long long *ps = pp + (size_t)s * (2 + hd);
            w[0] = ll_word_load(ps);
            w[1] = ll_word_load(ps + 1);
#pragma unroll
            for (int k = 0; k < 4; k++) w[2 + k] = ll_word_load(ps + 2 + cg * 4 + k);
        };
        // Every slot's words are requested before any is examined (a slot past nact reads
        // span nact - 1's and is then replaced by the empty span {-inf, 0, 0}): under a
        // per-slot branch the compiler waited for each slot's loads before issuing the
        // next slot's.
        unsigned long long wv6[kPre][6];
#pragma unroll
        for (int j = 0; j < kPre; j++) poll(min(sub + j * nsub, nact - 1), wv6[j]);
        uint32_t pending = 0;
#pragma unroll
        for (int j = 0; j < kPre; j++) {
            const bool live = sub + j * nsub < nact;
#pragma unroll
            for (int k = 0; k < 6; k++) {
                if (live && (uint32_t)(wv6[j][k] >> 32) != ep) pending |= 1u << (6 * j + k);
                if (!live) wv6[j][k] = k == 0 ? (unsigned long long)__float_as_uint(-INFINITY) : 0ull;
            }
        }
        for (uint32_t spins = 0; pending != 0 && ok; spins++) {
            if ((spins & 31u) == 31u) {
                if (spins > A.spin_limit) {
                    __hip_atomic_store(A.err, 3, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    ok = false;
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
#pragma unroll
            for (int j = 0; j < kPre; j++) {
                const unsigned long long *ps = pp + (size_t)(sub + j * nsub) * (2 + hd);
#pragma unroll
                for (int k = 0; k < 6; k++)
                    if (pending & (1u << (6 * j + k)))
                        wv6[j][k] = ll_word_load(ps + (k < 2 ? k : 2 + cg * 4 + (k - 2)));
            }
#pragma unroll
            for (int j = 0; j < kPre; j++)
#pragma unroll
                for (int k = 0; k < 6; k++)
                    if ((pending & (1u << (6 * j + k))) && (uint32_t)(wv6[j][k] >> 32) == ep)
                        pending &= ~(1u << (6 * j + k));
        }
        GQA_TR(1);
        // spans past kPre per thread (contexts above nsub * kPre * P positions): one by one
        auto wait6 = [&](int s, unsigned long long (&w)[6]) {
            poll(s, w);
            for (uint32_t spins = 0; ok; spins++) {
                bool cur = true;
#pragma unroll
                for (int k = 0; k < 6; k++) cur = cur && (uint32_t)(w[k] >> 32) == ep;
                if (cur) break;
                if (spins > A.spin_limit) {
                    __hip_atomic_store(A.err, 3, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    ok = false;
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
                poll(s, w);
            }
        };
        auto wf = [](unsigned long long w) { return __uint_as_float((uint32_t)w); };
        float *mred = reinterpret_cast<float *>(tiles);  // [NTH / 64] wave maxima
        // global maximum of the span maxima
        float M = -INFINITY;
#pragma unroll
        for (int j = 0; j < kPre; j++) M = fmaxf(M, wf(wv6[j][0]));
        for (int s = sub + kPre * nsub; s < nact; s += nsub) {
            unsigned long long w[6];
            wait6(s, w);
            M = fmaxf(M, wf(w[0]));
        }
        M = wave_max_f(M);
        if (lane == 0) mred[wv] = M;
        __syncthreads();
        M = mred[0];
        for (int w = 1; w < NTH / 64; w++) M = fmaxf(M, mred[w]);
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
        float L = 0.0f;
        auto add_span = [&](const unsigned long long (&w)[6]) {
            const float e = expf(wf(w[0]) - M);
            L = fmaf(wf(w[1]), e, L);
            acc.x = fmaf(wf(w[2]), e, acc.x);
            acc.y = fmaf(wf(w[3]), e, acc.y);
            acc.z = fmaf(wf(w[4]), e, acc.z);
            acc.w = fmaf(wf(w[5]), e, acc.w);
        };
#pragma unroll
        for (int j = 0; j < kPre; j++)
            if (sub + j * nsub < nact) add_span(wv6[j]);
        for (int s = sub + kPre * nsub; s < nact; s += nsub) {
            unsigned long long w[6];
            wait6(s, w);
            add_span(w);
        }
        // subsets added in order
        float *osub = reinterpret_cast<float *>(tiles) + 64;  // [nsub][hd]
        float *lsub = osub + nsub * hd;                      // [nsub]
        *reinterpret_cast<float4 *>(osub + sub * hd + cg * 4) = acc;
        if (cg == 0) lsub[sub] = L;
        __syncthreads();
        float *ofin = lsub + nsub;  // [hd]
        if ((int)tid < hd) {
            float Lt = lsub[0], o = osub[tid];
            for (int u = 1; u < nsub; u++) {
                Lt += lsub[u];
                o += osub[u * hd + tid];
            }
            ofin[tid] = o * (1.0f / Lt);
        }
        __syncthreads();
        if ((int)wv < nb) {
            const int b = (int)wv;
            const float o = ifwht_lane(ofin[b * 64 + lane], (uint64_t)b, lane);
            const size_t hbase = (size_t)tok * nq * hd + (size_t)head * hd;
            if (A.out_f) A.out_f[hbase + b * 64 + lane] = o;
            if (A.aq) {
                const size_t c = (size_t)head * nb + b, g = (size_t)tok * nq * nb + c;
                quant_chunk_store(fwht_lane(o, c, lane), lane, A.aq + g * 64, A.as + g, A.asum + g);
            }
        }
        // the last merge workgroup of the launch advances the epoch (every span workgroup
        // of this launch has published, so all have read the epoch already)
        if (tid == 0) {
            const unsigned int total = gridDim.x * (unsigned int)G * gridDim.z;
            if (__hip_atomic_fetch_add(A.cnt + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == total - 1u) {
                __hip_atomic_store(A.cnt + 1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(A.cnt, ep, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        GQA_TR(7);
        return;
    }
    // ---------------------------------------------------------------- span workgroup
    // (span, head part hs): q heads h0 .. h0 + GL - 1 of the group
    const int span = ((int)blockIdx.y - G) / A.hsplit, hs = ((int)blockIdx.y - G) % A.hsplit;
    const int h0 = hs * GM, GL = min(GM, G - h0);
    const int t0 = span * P, t1 = min(seq, t0 + P), n = t1 - t0;
    if (n <= 0 || GL <= 0) return;  // spans past the context take no part
    const KvRing kr = A.kr;
    const size_t base = ((size_t)layer * nkv + kvh) * kr.cap;
    int8_t *kt = tiles, *vt = tiles + P * 128;
    // 1. K / V rows t0 .. t0+P-1 (rows past t1 re-read row t1-1), 16 bytes per lane; the
    //    scales by waves 0-3 (K rows 0-63, 64-127, then V)
    {
        constexpr int pieces = P * HD / 16, per_row = HD / 16;
        const uint32_t mk = lds_offset(kt), mvv = lds_offset(vt);
        for (int j = 0; j * NTH < pieces; j++) {
            const int i = j * NTH + (int)tid;
            const int r = min(i / per_row, n - 1), c = i % per_row;
            const size_t off = (base + (size_t)(t0 + r)) * hd + (size_t)c * 16;
            const uint32_t m0 = (uint32_t)__builtin_amdgcn_readfirstlane((int)(j * NTH + wv * 64) * 16);
            lds_dma16(A.kq + off, mk + m0);
            lds_dma16(A.vq + off, mvv + m0);
        }
        if ((int)wv < 2 * PW) {
            const int row = (int)(wv % PW) * 64 + (int)lane;
            const size_t sl = base + (size_t)(t0 + min(row, n - 1));
            const uint32_t m0 = (uint32_t)__builtin_amdgcn_readfirstlane(
                (int)(lds_offset((int)wv < PW ? kst : vst) + (wv % PW) * 256));
            lds_dma4(((int)wv < PW ? A.ks : A.vs) + sl, m0);
        }
    }
    // 2. q head wv (and the current position's K / V where this span holds it)
    const AttnPost &post = A.post;
    const int cur = seq - 1;
    const bool covers = post.on && t0 <= cur && cur < t1;
    if ((int)wv < GL) {
        const int h = (int)wv, head = kvh * G + h0 + h;
        const float *qh = A.q + (size_t)tok * A.q_stride + (size_t)head * hd;
        float qv0, qv1;
        if (post.on) {
            head_post(qh, head, nq, nkv, hd, post.bias, post.qn, post.kn, post.eps, post.rope, cur, lane, qv0, qv1);
        } else {
            qv0 = qh[lane];
            qv1 = nb > 1 ? qh[64 + lane] : 0.0f;
        }
        const float r0 = fwht_lane(qv0, 0, lane);
        const float r1 = nb > 1 ? fwht_lane(qv1, 1, lane) : 0.0f;
        const float mx = wave_max_f(fmaxf(fabsf(r0), fabsf(r1)));
        int8_t *qd = qi + h * 128;
        if (mx <= FLT_EPSILON) {
            qd[lane] = 0;
            if (nb > 1) qd[64 + lane] = 0;
            if (lane == 0) qas[h] = 0.0f;
        } else {
            const float inv = 127.0f / mx;
            qd[lane] = (int8_t)(int)rintf(r0 * inv);
            if (nb > 1) qd[64 + lane] = (int8_t)(int)rintf(r1 * inv);
            if (lane == 0) qas[h] = (mx / 127.0f) * A.attn_scale;
        }
    }
    if (covers && wv < 2) {
        const int hh = wv == 0 ? nq + kvh : nq + nkv + kvh;
        float a0, a1;
        head_post(A.q + (size_t)tok * A.q_stride + (size_t)hh * hd, hh, nq, nkv, hd, post.bias, post.qn, post.kn,
                  post.eps, post.rope, cur, lane, a0, a1);
        const float r0 = fwht_lane(a0, 0, lane);
        const float r1 = nb > 1 ? fwht_lane(a1, 1, lane) : 0.0f;
        kv_store_head(r0, r1, nb, lane, 8, hd, 0, wv == 0 ? kcur : vcur, cur_s + wv);
        // (every head part builds the row for its own tile; the first stores it in the cache)
        if (hs == 0)
            kv_store_head(r0, r1, nb, lane, 8, hd, base + (size_t)cur, wv == 0 ? A.kq : A.vq,
                          wv == 0 ? A.ks : A.vs);
    }
    GQA_TR(2);
    wait_vmcnt<0>();  // this wave's tile copies have landed
    __syncthreads();
    if (covers) {  // the current position's row (its tile copy read the slot before it was written)
        const int r = cur - t0;
        if ((int)tid < hd) {
            kt[r * hd + tid] = kcur[tid];
            vt[r * hd + tid] = vcur[tid];
        }
        if (tid == 0) {
            kst[r] = cur_s[0];
            vst[r] = cur_s[1];
        }
        __syncthreads();
    }
    GQA_TR(3);
    if constexpr (MF) {
        // 3-5 on the matrix cores (the layout of attn_prefill_mfma_kernel with the group's q
        // heads in place of its tokens).  Wave w takes positions 16w .. 16w + 15 of the span:
        //  - scores: v_mfma_i32_16x16x64_i8 with A = K (lane l: position 16w + l%16) and
        //    B = the int8 q heads (lane l: head l%16; heads past the part are zero): exact
        //    integer dots, lane l holding positions 16w + 4(l/16) + r of head l%16;
        //    s = (float(dot) * ks) * qas as before;
        //  - the span's maximum and sum per head: each wave's over its positions, then the
        //    waves' in wave order;
        //  - o^T += V^T (p vs)^T: four v_mfma_f32_16x16x4f32 per 16 dims, the r-th over the
        //    wave's positions 4g + r (g = 0..3), whose weights are the score tile's own
        //    registers; the waves' partial o are added in wave order.
        static_assert(P == 16 * (NTH / 64), "one 16-position tile per wave");
        constexpr int NW = NTH / 64, DB = HD / 16;
        const uint32_t li = lane & 15u, lg = lane >> 4;
        const int pw0 = 16 * (int)wv;
        const bool hl = (int)li < GL;
        v4i_t acc = {0, 0, 0, 0};
#pragma unroll
        for (int k = 0; k < nb; k++) {
            const int4 kv = *reinterpret_cast<const int4 *>(kt + (pw0 + (int)li) * HD + 64 * k + 16 * (int)lg);
            const int4 qv = hl ? *reinterpret_cast<const int4 *>(qi + li * 128 + 64 * k + 16 * lg) : make_int4(0, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(v4i_t{kv.x, kv.y, kv.z, kv.w}, v4i_t{qv.x, qv.y, qv.z, qv.w}, acc,
                                                         0, 0, 0);
        }
        const float qs = hl ? qas[li] : 0.0f;
        const int pr = pw0 + 4 * (int)lg;  // this lane's first position
        float sc4[4];
        float tmax = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            sc4[r] = hl && pr + r < n ? ((float)acc[r] * kst[pr + r]) * qs : -INFINITY;
            tmax = fmaxf(tmax, sc4[r]);
        }
        tmax = fmaxf(tmax, xor_lane(tmax, 16));
        tmax = fmaxf(tmax, xor_lane(tmax, 32));
        if (lg == 0 && hl) red_m[li][wv] = tmax;
        __syncthreads();
        float m = -INFINITY;
        if (hl) {
            m = red_m[li][0];
#pragma unroll
            for (int u = 1; u < NW; u++) m = fmaxf(m, red_m[li][u]);
        }
        float psum = 0.0f, w[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float pe = sc4[r] == -INFINITY ? 0.0f : expf(sc4[r] - m);
            psum += pe;
            w[r] = pe * vst[pr + r];
        }
        psum += xor_lane(psum, 16);
        psum += xor_lane(psum, 32);
        if (lg == 0 && hl) red_l[li][wv] = psum;
        v4f o[DB];
#pragma unroll
        for (int b = 0; b < DB; b++) {
            o[b] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float a = (float)vt[(pr + r) * HD + 16 * b + (int)li];
                o[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, w[r], o[b], 0, 0, 0);
            }
        }
        // the waves' partial o [wave][head][dim] after the K / V tiles (still being read)
        float *opw = reinterpret_cast<float *>(tiles + 2 * P * 128);
        if (hl) {
#pragma unroll
            for (int b = 0; b < DB; b++)
#pragma unroll
                for (int r = 0; r < 4; r++) opw[((int)wv * GM + (int)li) * HD + 16 * b + 4 * (int)lg + r] = o[b][r];
        }
        __syncthreads();
        unsigned long long *pbase =
            A.words + (size_t)(tok * nq + kvh * G + h0) * pstride + (size_t)span * (2 + hd);
        for (int i = (int)tid; i < GL * hd; i += NTH) {
            const int h = i / hd, c = i % hd;
            float ov = opw[h * HD + c];
            for (int u = 1; u < NW; u++) ov += opw[(u * GM + h) * HD + c];
            unsigned long long *pp = pbase + (size_t)h * pstride;
            ll_word_store(pp + 2 + c, __float_as_uint(ov), ep);
            if (c == 0) {
                float mm = red_m[h][0], l = red_l[h][0];
                for (int u = 1; u < NW; u++) {
                    mm = fmaxf(mm, red_m[h][u]);
                    l += red_l[h][u];
                }
                ll_word_store(pp, __float_as_uint(mm), ep);
                ll_word_store(pp + 1, __float_as_uint(l), ep);
            }
        }
    } else {
    // 3. scores: wave w takes position (w & 1) * 64 + lane for heads w / 2 and w / 2 + 4;
    //    lane p reads its K row's 16-byte pieces starting at piece p (no bank conflicts)
    const int p = (int)(wv % PW) * 64 + (int)lane;
    const bool valid = p < n;
    constexpr int KH = GM / HW;  // heads per wave
    float s2[KH];
    {
        constexpr int npc = HD / 16;
        uint4 kr4[8];
#pragma unroll
        for (int i = 0; i < 8; i++)
            if (i < npc) kr4[i] = reinterpret_cast<const uint4 *>(kt + p * hd)[(i + p) & (npc - 1)];
#pragma unroll
        for (int k = 0; k < KH; k++) {
            const int h = (int)(wv / PW) + HW * k;
            s2[k] = -INFINITY;
            if (h < GL) {
                const uint4 *qr = reinterpret_cast<const uint4 *>(qi + h * 128);
                int dot = 0;
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    if (i < npc) {
                        const uint4 a = kr4[i], b = qr[(i + p) & (npc - 1)];
                        dot = __builtin_amdgcn_sdot4((int)a.x, (int)b.x, dot, false);
                        dot = __builtin_amdgcn_sdot4((int)a.y, (int)b.y, dot, false);
                        dot = __builtin_amdgcn_sdot4((int)a.z, (int)b.z, dot, false);
                        dot = __builtin_amdgcn_sdot4((int)a.w, (int)b.w, dot, false);
                    }
                }
                s2[k] = valid ? ((float)dot * kst[p]) * qas[h] : -INFINITY;
                const float m = wave_max_f(s2[k]);
                if (lane == 0) red_m[h][wv % PW] = m;
            }
        }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < KH; k++) {
        const int h = (int)(wv / PW) + HW * k;
        if (h < GL) {
            float m = red_m[h][0];
            for (int u = 1; u < PW; u++) m = fmaxf(m, red_m[h][u]);
            const float e = valid ? expf(s2[k] - m) : 0.0f;
            const float l = wave_sum_f(e);
            sc[p * GM + h] = e * vst[p];
            if (lane == 0) red_l[h][wv % PW] = l;
        }
    }
    for (int i = (int)tid; i < P * GM; i += NTH)
        if ((i & (GM - 1)) >= GL) sc[i] = 0.0f;  // heads past this part
    __syncthreads();
    GQA_TR(4);
    // 4. o partials: thread (position subset sub, 4-column group cg) converts each V
    //    element once and adds it into all heads; the subsets are added in order
    constexpr int ncg = HD / 4, nsub = NTH / ncg, plen = P / nsub;
    const int cg = (int)tid % ncg, sub = (int)tid / ncg;
    float acc[GM][4];
#pragma unroll
    for (int h = 0; h < GM; h++) acc[h][0] = acc[h][1] = acc[h][2] = acc[h][3] = 0.0f;
    {
        const int ta = sub * plen, tb = min(n, ta + plen);
        for (int t = ta; t < tb; t++) {
            const int v = *reinterpret_cast<const int *>(vt + t * hd + cg * 4);
            float w[GM];
            const float4 w0 = *reinterpret_cast<const float4 *>(sc + t * GM);
            w[0] = w0.x;
            w[1] = w0.y;
            w[2] = w0.z;
            w[3] = w0.w;
            if constexpr (GM > 4) {
                const float4 w1 = *reinterpret_cast<const float4 *>(sc + t * GM + 4);
                w[4] = w1.x;
                w[5] = w1.y;
                w[6] = w1.z;
                w[7] = w1.w;
            }
            const float x0 = (float)(int8_t)(v & 0xFF), x1 = (float)(int8_t)((v >> 8) & 0xFF);
            const float x2 = (float)(int8_t)((v >> 16) & 0xFF), x3 = (float)(int8_t)((v >> 24) & 0xFF);
#pragma unroll
            for (int h = 0; h < GM; h++) {
                acc[h][0] = fmaf(w[h], x0, acc[h][0]);
                acc[h][1] = fmaf(w[h], x1, acc[h][1]);
                acc[h][2] = fmaf(w[h], x2, acc[h][2]);
                acc[h][3] = fmaf(w[h], x3, acc[h][3]);
            }
        }
    }
    __syncthreads();  // the tiles are free: they take the subsets' sums [sub][head][hd]
    float *opart = reinterpret_cast<float *>(tiles);
#pragma unroll
    for (int h = 0; h < GM; h++)
        if (h < GL)
            *reinterpret_cast<float4 *>(opart + ((size_t)sub * GL + h) * hd + cg * 4) =
                make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
    __syncthreads();
    // 5. publish {m, L, o[hd]} per head as {payload, epoch} words (one agent-scope store
    //    each: the value and its ready mark arrive together, no fence or counter)
    unsigned long long *pbase =
        A.words + (size_t)(tok * nq + kvh * G + h0) * pstride + (size_t)span * (2 + hd);
    for (int i = (int)tid; i < GL * hd; i += NTH) {
        const int h = i / hd, c = i % hd;
        float o = opart[h * hd + c];
        for (int u = 1; u < nsub; u++) o += opart[((size_t)u * GL + h) * hd + c];
        unsigned long long *pp = pbase + (size_t)h * pstride;
        ll_word_store(pp + 2 + c, __float_as_uint(o), ep);
        if (c == 0) {
            float m = red_m[h][0], l = red_l[h][0];
            for (int u = 1; u < PW; u++) {
                m = fmaxf(m, red_m[h][u]);
                l += red_l[h][u];
            }
            ll_word_store(pp, __float_as_uint(m), ep);
            ll_word_store(pp + 1, __float_as_uint(l), ep);
        }
    }
    }
    GQA_TR(5);
}

#ifdef K2T_GQA_TRACE
extern "C" int k2t_gqa_trace_read(unsigned long long *dst) {
    return hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_gqa_trace), sizeof(g_gqa_trace)) == hipSuccess ? 0 : -1;
}
#endif

// One split (the whole-context kernel) up to kAttnWhole positions, else 256-position spans.
int attn_max_splits(int max_seq) {
    return max_seq <= kAttnWhole ? 1 : (max_seq + kAttnSplitLen - 1) / kAttnSplitLen;
}

// Spans of the grouped-query kernel over a cache of `cap` slots.
int gqa_spans(int cap) { return (cap + kGqaSpan - 1) / kGqaSpan; }

// Whether launch_attention runs the grouped-query kernel (given span words), and the
// words it then needs: [token][q head][span][2 + hd].
bool gqa_eligible(int nsplit, int ntok, int nq, int nkv, int hd, const KvRing &kr) {
    const int group = nq / nkv;
    return nsplit > 1 && ntok == 1 && group >= 2 && group <= kGqaMaxGroup && kr.bits == 8 && kr.window == 0 &&
           (hd == 64 || hd == 128);
}
size_t gqa_words(int cap, int nq, int hd, int ntok) { return (size_t)gqa_spans(cap) * nq * (2 + hd) * ntok; }

// attn_partial_kernel with or without the sliding-window ring arithmetic.
template <int NTH, bool FINAL, int VORD, typename... Args>
void launch_attn_partial(const KvRing &kr, dim3 grid, hipStream_t st, Args... args) {
    if (kr.window > 0 || kr.ring > 0)
        hipLaunchKernelGGL((attn_partial_kernel<NTH, FINAL, VORD, true>), grid, dim3(NTH), 0, st, args...);
    else
        hipLaunchKernelGGL((attn_partial_kernel<NTH, FINAL, VORD, false>), grid, dim3(NTH), 0, st, args...);
}

void launch_attention(hipStream_t st, const float *q, int q_stride, int8_t *kq, int8_t *vq, float *ks, float *vs,
                      const AttnPost &post, const int *pos_dev, int layer, int nq, int nkv, int hd, KvRing kr,
                      float attn_scale,
                      int nsplit, int ntok, float *part, float *out_f, int8_t *aq, float *as, int32_t *asum,
                      const GqaWork &gqa, int ctx_bound, ActTiles tiles, bool mfma) {
    if (mfma && ntok >= 16 && !post.on && kr.bits == 8 && kr.window == 0 && kr.ring == 0 && (hd == 64 || hd == 128)) {
        const dim3 grid(nq, (ntok + 15) / 16);
        if (hd == 128)
            hipLaunchKernelGGL(attn_prefill_mfma_kernel<128>, grid, dim3(64 * kPattWaves), 0, st, q, q_stride, kq, vq, ks, vs,
                               pos_dev, layer, nq, nkv, kr.cap, attn_scale, ntok, out_f, aq, as, asum, tiles);
        else
            hipLaunchKernelGGL(attn_prefill_mfma_kernel<64>, grid, dim3(64 * kPattWaves), 0, st, q, q_stride, kq, vq, ks, vs,
                               pos_dev, layer, nq, nkv, kr.cap, attn_scale, ntok, out_f, aq, as, asum, tiles);
        hip_check(hipGetLastError(), "prefill attention launch");
        return;
    }
    if (nsplit == 1 && ctx_bound > 0 && ctx_bound <= kAttnSmall) {
        // every token of the batch attends to at most kAttnSmall positions: a quarter of the
        // threads, the whole-context kernel's sums (its V position subsets) bit for bit
        launch_attn_partial<kAttnSmall, true, kAttnWhole>(kr, dim3(nq, 1, ntok), st, q, q_stride, kq, vq, ks, vs,
                                                          pos_dev, layer, nq, nkv, hd, kr, attn_scale, 1, post, part,
                                                          out_f, aq, as, asum, tiles);
        hip_check(hipGetLastError(), "attention launch");
        return;
    }
    if (nsplit == 1) {  // the caller sized the context within kAttnWhole (attn_max_splits)
        launch_attn_partial<kAttnWhole, true, kAttnWhole>(kr, dim3(nq, 1, ntok), st, q, q_stride, kq, vq, ks, vs,
                                                          pos_dev, layer, nq, nkv, hd, kr, attn_scale, 1, post, part,
                                                          out_f, aq, as, asum, tiles);
        hip_check(hipGetLastError(), "attention launch");
        return;
    }
    const int group = nq / nkv;
    if (gqa.words && ntok == 1 && group >= 2 && group <= kGqaMaxGroup && kr.bits == 8 && kr.window == 0 &&
        (hd == 64 || hd == 128)) {
        if (tiles.xt) throw Error(K2T_E_INTERNAL, "grouped-query attention writes no activation tiles");
        const int hsplit = (group + kGqaHeads - 1) / kGqaHeads;
        GqaArgs A{q,          q_stride,          kq,   vq,         ks,       vs,       pos_dev, layer,
                  nq,         nkv,               kr,   attn_scale, gqa_spans(kr.cap), hsplit, post, gqa.words,
                  gqa.cnt,    gqa.err,           1u << 20, out_f, aq, as, asum};
        const dim3 grid(nkv, group + A.nspan * hsplit, ntok);
        if (hd == 128)
            hipLaunchKernelGGL((attn_gqa_kernel<128, kGqaHeads, kGqaMfma>), grid, dim3(kGqaThreads), 0, st, A);
        else
            hipLaunchKernelGGL((attn_gqa_kernel<64, kGqaHeads, kGqaMfma>), grid, dim3(kGqaThreads), 0, st, A);
        hip_check(hipGetLastError(), "attn_gqa launch");
        return;
    }
    launch_attn_partial<kAttnSplitLen, false, kAttnSplitLen>(
        kr, dim3(nq, nsplit, ntok), st, q, q_stride, kq, vq, ks, vs, pos_dev, layer, nq, nkv, hd, kr, attn_scale, nsplit,
        post, part, (float *)nullptr, (int8_t *)nullptr, (float *)nullptr, (int32_t *)nullptr, ActTiles{});
    hip_check(hipGetLastError(), "attn_partial launch");
    hipLaunchKernelGGL(attn_merge_kernel, dim3(nq, ntok), dim3(64), 0, st, part, nq, hd, nsplit, kAttnSplitLen, kr,
                       pos_dev, out_f, aq, as, asum, tiles);
    hip_check(hipGetLastError(), "attn_merge launch");
}

// ---------------------------------------------------------------- exact-order attention
// Decode attention in the x86 reference's operation order (causal_gqa_group_q8, portable
// branches real_llm.rs:8533-8545 and 8575-8585; softmax_unnorm_inplace 9590-9600), for the
// exact-order mode.  One wave per (q head, token):
//   q rotated and quantized like a KV head (store_hadamard_q8_head order), qas = qs*scale;
//   s_t = (float(q8 . k8_t) * ks_t) * qas (with a sliding window: the sum over 64-blocks of
//   float(dot_g) * ks_t * qas, causal_gqa_group_q4_or_window's int8 branch), one position
//   per lane;
//   p_t = exp(s_t - max) with the x86 build's exp (expf_rn), in parallel;
//   sum = p_0 + p_1 + ... in position order (lane 0), inv = 1/sum;
//   o[d] += ((p_t * inv) * vs_t) * float(v8_t[d]) for t ascending (a window skips weights of
//   zero), lane d holding columns d and 64 + d;
//   ifwht64 per block, written as fp32 to out_f [token][nq * hd].
// Scores live in dynamic LDS (one float per attended position).
__global__ __launch_bounds__(64) void attn_exact_kernel(const float *__restrict__ q, int q_stride,
                                                        const int8_t *__restrict__ kq, const int8_t *__restrict__ vq,
                                                        const float *__restrict__ ks, const float *__restrict__ vs,
                                                        const int *__restrict__ pos_dev, int layer, int nq, int nkv,
                                                        int hd, KvRing kr, float attn_scale, float *__restrict__ out_f) {
    extern __shared__ float sc[];
    __shared__ int8_t qi[128];
    __shared__ float red[2];
    const uint32_t lane = threadIdx.x;
    const int h = blockIdx.x, tok = blockIdx.y, nb = hd / 64;
    const int pos = pos_dev[0] + tok, seq = pos + 1;
    const int n = active_len(kr, seq);
    const int kvh = h / (nq / nkv);
    const size_t base = ((size_t)layer * nkv + kvh) * kr.cap;
    const float *qr = q + (size_t)tok * q_stride + (size_t)h * hd;
    const float r0 = fwht_lane(qr[lane], 0, lane);
    const float r1 = nb > 1 ? fwht_lane(qr[64 + lane], 1, lane) : 0.0f;
    const float mx = wave_max_f(fmaxf(fabsf(r0), fabsf(r1)));
    float qscale = 0.0f;
    if (mx <= FLT_EPSILON) {
        qi[lane] = 0;
        if (nb > 1) qi[64 + lane] = 0;
    } else {
        const float inv = 127.0f / mx;
        qi[lane] = (int8_t)(int)rintf(r0 * inv);
        if (nb > 1) qi[64 + lane] = (int8_t)(int)rintf(r1 * inv);
        qscale = mx / 127.0f;
    }
    const float qas = qscale * attn_scale;
    __syncthreads();
    float smax = -INFINITY;
    for (int idx = (int)lane; idx < n; idx += 64) {
        const size_t slot = base + ring_slot(kr, active_pos(kr, idx, seq));
        const int8_t *kr8 = kq + slot * hd;
        const float kscale = ks[slot];
        float s;
        if (kr.window > 0) {
            float total = 0.0f;
            for (int g = 0; g < nb; g++) {
                int dot = 0;
                for (int i = 0; i < 64; i++) dot += (int)qi[g * 64 + i] * (int)kr8[g * 64 + i];
                total = total + ((float)dot * kscale) * qas;
            }
            s = total;
        } else {
            int dot = 0;
            for (int i = 0; i < hd; i++) dot += (int)qi[i] * (int)kr8[i];
            s = ((float)dot * kscale) * qas;
        }
        sc[idx] = s;
        smax = fmaxf(smax, s);
    }
    const float m = wave_max_f(smax);
    for (int idx = (int)lane; idx < n; idx += 64) sc[idx] = expf_rn(sc[idx] - m);
    __syncthreads();
    if (lane == 0) {
        float sum = 0.0f;
        for (int idx = 0; idx < n; idx++) sum = sum + sc[idx];
        red[0] = 1.0f / sum;
    }
    __syncthreads();
    const float inv = red[0];
    float o0 = 0.0f, o1 = 0.0f;
    for (int idx = 0; idx < n; idx++) {
        const size_t slot = base + ring_slot(kr, active_pos(kr, idx, seq));
        const float w = (sc[idx] * inv) * vs[slot];
        if (kr.window > 0 && w == 0.0f) continue;
        const int8_t *vr = vq + slot * hd;
        o0 = o0 + w * (float)vr[lane];
        if (nb > 1) o1 = o1 + w * (float)vr[64 + lane];
    }
    float *dst = out_f + (size_t)tok * nq * hd + (size_t)h * hd;
    dst[lane] = ifwht_lane(o0, 0, lane);
    if (nb > 1) dst[64 + lane] = ifwht_lane(o1, 1, lane);
}

// Positions one exact-order attention launch can hold in LDS (one float each).
constexpr int kAttnExactMaxPositions = 32768;

void launch_attention_exact(hipStream_t st, const float *q, int q_stride, const int8_t *kq, const int8_t *vq,
                            const float *ks, const float *vs, const int *pos_dev, int layer, int nq, int nkv, int hd,
                            KvRing kr, float attn_scale, int ntok, int max_positions, float *out_f) {
    if (kr.bits != 8) throw Error(K2T_E_ARG, "exact-order attention needs the int8 KV cache");
    const int npos = kr.window > 0 ? std::min(max_positions, kr.window) : max_positions;
    if (npos > kAttnExactMaxPositions) throw Error(K2T_E_ARG, "exact-order attention: context too long");
    hipLaunchKernelGGL(attn_exact_kernel, dim3(nq, ntok), dim3(64), (size_t)npos * sizeof(float), st, q, q_stride,
                       kq, vq, ks, vs, pos_dev, layer, nq, nkv, hd, kr, attn_scale, out_f);
    hip_check(hipGetLastError(), "attn_exact launch");
}

// ---------------------------------------------------------------- SwiGLU + FWHT + int8
// Interleaved gate_up output: block ic = [gate64(ic), up64(ic)] (simd_lut.rs:3310-3325).
// swiglu_activate_scalar (real_llm.rs:9801-9805), then populate_chunk_fwht_raw with chunk ic.
// EXACT: the exponential of the x86 reference build (expf_rn) instead of the device expf.
// One wave per (token, four chunks), in rmsnorm_act_kernel's four-element layout.
template <bool EXACT>
__global__ __launch_bounds__(64) void swiglu_act_kernel(const float *__restrict__ gu, int inter, int8_t *__restrict__ q,
                                                        float *__restrict__ s, int32_t *__restrict__ sums,
                                                        ActTiles tiles, const uint64_t *__restrict__ signs) {
    const uint32_t lane = threadIdx.x, sl = lane & 15u;
    const int nci = inter / 64, tok = blockIdx.y;
    const int cg = 4 * (int)blockIdx.x + (int)(lane >> 4), ic = min(cg, nci - 1);
    const float *b = gu + (size_t)tok * 2 * inter + (size_t)ic * 128;
    const float4 g4 = *reinterpret_cast<const float4 *>(b + 4 * sl);
    const float4 u4 = *reinterpret_cast<const float4 *>(b + 64 + 4 * sl);
    const float gs[4] = {g4.x, g4.y, g4.z, g4.w}, us[4] = {u4.x, u4.y, u4.z, u4.w};
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; j++) v[j] = (gs[j] / (1.0f + (EXACT ? expf_rn(-gs[j]) : expf(-gs[j])))) * us[j];
    const Chunk4 r = rotate_quant4(v, signs[ic], sl);
    if (cg < nci) chunk4_store(r, sl, tok, ic, nci, q, s, sums, tiles.xt, tiles.st, tiles.ut);
}

void launch_swiglu_act(hipStream_t st, const uint64_t *signs, const float *gu, int inter, int ntok, int8_t *q,
                       float *s, int32_t *sums, bool exact, ActTiles tiles) {
    if (inter % 64 != 0 || inter / 64 > kSignBlocks || !signs) throw Error(K2T_E_INTERNAL, "swiglu_act shape");
    const dim3 grid((inter / 64 + 3) / 4, ntok);
    if (exact)
        hipLaunchKernelGGL(swiglu_act_kernel<true>, grid, dim3(64), 0, st, gu, inter, q, s, sums, tiles, signs);
    else
        hipLaunchKernelGGL(swiglu_act_kernel<false>, grid, dim3(64), 0, st, gu, inter, q, s, sums, tiles, signs);
    hip_check(hipGetLastError(), "swiglu_act launch");
}

// ---------------------------------------------------------------- tied embedding
// embed_token_into (real_llm.rs:8063-8097): row `token` of the quantized lm_head,
// dequantized in the rotated domain (simd_lut.rs:3439-3480 / 5558-5634), then ifwht64.
// One wave per 64-column chunk; tokens come from a device array.
__global__ __launch_bounds__(64) void embed_kernel(const uint8_t *__restrict__ pair, const uint8_t *__restrict__ tail,
                                                   int fmt, int hp, int sgc, size_t ptot, int nc, int np,
                                                   uint32_t cb0, uint32_t cb1, uint32_t cb2, uint32_t cb3,
                                                   const int *__restrict__ tokens, float *__restrict__ out) {
    const uint32_t lane = threadIdx.x;
    const int c = blockIdx.x, tok_i = blockIdx.y;
    const int r = tokens[tok_i];
    const int stripe = r / 16, rl = r % 16, g = rl / 4, j = rl % 4;
    const int k = lane / 16, w = lane % 16, half = w / 8, sub = w / 4, t = w % 4;
    const bool in_pair = stripe < 2 * np;
    const int side = stripe & 1;
    float val;
    if (fmt == K2T_FMT_NIBBLE4) {
        const size_t prec = 1024 + 256 * (size_t)hp + 64, trec = 512 + 128 * (size_t)hp + 32;
        const uint8_t *base = in_pair ? pair + ((size_t)(stripe / 2) * nc + c) * prec : tail + (size_t)c * trec;
        const uint8_t *d = base + (in_pair ? side * 512 : 0);
        const uint8_t *h = base + (in_pair ? 1024 + side * 128 * hp : 512);
        const uint8_t *sp = base + (in_pair ? 1024 + 256 * hp + side * 32 : 512 + 128 * hp);
        const uint8_t byte = d[k * 128 + g * 32 + half * 16 + j * 4 + t];
        int u = (w % 8) < 4 ? (byte & 0x0F) : (byte >> 4);
        if (hp == 1) {
            const uint8_t hb = h[(k / 2) * 64 + g * 16 + j * 4 + t];
            const int bit = (k & 1) == 0 ? 4 + sub : sub;
            u |= ((hb >> bit) & 1) << 4;
        } else if (hp == 2) {
            const int shifts[4] = {4, 6, 2, 0};
            const uint8_t hb = h[k * 64 + g * 16 + j * 4 + t];
            u |= ((hb >> shifts[sub]) & 3) << 4;
        }
        const float delta = __uint_as_float((uint32_t)(sp[rl * 2] | (sp[rl * 2 + 1] << 8)) << 16);
        val = (float)(2 * u - ((1 << (4 + hp)) - 1)) * delta;
    } else {
        const int sg = c / sgc, cst = sg * sgc, sb = c - cst;
        const uint8_t *gb = in_pair ? pair + (size_t)(stripe / 2) * ptot + (size_t)sg * 64 + (size_t)cst * 1024
                                    : tail + (size_t)sg * 32 + (size_t)cst * 512;
        const uint8_t *sp = gb + (in_pair ? side * 32 : 0);
        const uint8_t *d = gb + (in_pair ? 64 + (size_t)sb * 1024 + side * 512 : 32 + (size_t)sb * 512);
        const int sub4 = w / 4;
        const uint8_t byte = d[k * 128 + g * 32 + (sub4 / 2) * 16 + j * 4 + t];
        const int idx = (sub4 & 1) == 0 ? (byte & 0x0F) : (byte >> 4);
        const uint32_t cbw = idx < 4 ? cb0 : idx < 8 ? cb1 : idx < 12 ? cb2 : cb3;
        const int cv = (int)(int8_t)((cbw >> (8 * (idx & 3))) & 0xFF);
        const float delta = __uint_as_float((uint32_t)(sp[rl * 2] | (sp[rl * 2 + 1] << 8)) << 16);
        val = (float)cv * delta;
    }
    out[(size_t)tok_i * nc * 64 + (size_t)c * 64 + lane] = ifwht_lane(val, (uint64_t)c, lane);
}

void launch_embed(hipStream_t st, const k2t_mat *m, const int *tokens, int ntok, float *out) {
    const size_t ptot = m->fmt == K2T_FMT_NF ? (m->pairs ? m->pair_len / m->pairs : 0) : 0;
    hipLaunchKernelGGL(embed_kernel, dim3(m->nc, ntok), dim3(64), 0, st, m->pair, m->tail, m->fmt, m->hp, m->sgc, ptot,
                       m->nc, m->pairs, m->cb[0], m->cb[1], m->cb[2], m->cb[3], tokens, out);
    hip_check(hipGetLastError(), "embed launch");
}

// Untied embedding rows (embed_token_into, real_llm.rs:8073-8085): f32 rows are copied,
// bf16 rows widened; one thread per element.
__global__ __launch_bounds__(256) void embed_rows_kernel(const void *__restrict__ rows, int bf16,
                                                         const int *__restrict__ tokens, int d,
                                                         float *__restrict__ out) {
    const int i = blockIdx.x * 256 + threadIdx.x, t = blockIdx.y;
    if (i >= d) return;
    const size_t src = (size_t)tokens[t] * d + i;
    out[(size_t)t * d + i] = bf16 ? __uint_as_float((uint32_t)((const uint16_t *)rows)[src] << 16)
                                  : ((const float *)rows)[src];
}

void launch_embed_rows(hipStream_t st, const void *rows, bool bf16, const int *tokens, int ntok, int d, float *out) {
    hipLaunchKernelGGL(embed_rows_kernel, dim3((d + 255) / 256, ntok), dim3(256), 0, st, rows, bf16 ? 1 : 0, tokens,
                       d, out);
    hip_check(hipGetLastError(), "embed_rows launch");
}

// Benchmark support: seeded pseudo-random int8 K/V codes and positive scales for cache
// positions [0, n_pos) of every layer and KV head (a counter-based SplitMix64 hash per
// element, so the fill is reproducible and needs no state).
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__global__ __launch_bounds__(256) void kv_synthetic_kernel(int8_t *__restrict__ kq, int8_t *__restrict__ vq,
                                                           float *__restrict__ ks, float *__restrict__ vs,
                                                           int layers_kv, int cap, int n_pos, int hd, int bits,
                                                           uint64_t seed) {
    const size_t slot_lin = blockIdx.x;  // (layer*nkv + kvh) * n_pos + pos
    const int lk = (int)(slot_lin / (size_t)n_pos), pos = (int)(slot_lin % (size_t)n_pos);
    if (lk >= layers_kv) return;
    const size_t slot = (size_t)lk * cap + pos;
    const uint64_t base = seed * 0x9E3779B97F4A7C15ull + slot_lin * 0x100000001B3ull;
    for (int i = (int)threadIdx.x; i < hd; i += (int)blockDim.x) {
        const uint64_t h = mix64(base + (uint64_t)i);
        kq[slot * hd + i] = (int8_t)((int)(h & 0xFF) - 128 == -128 ? -127 : (int)(h & 0xFF) - 128);
        vq[slot * hd + i] = (int8_t)((int)((h >> 8) & 0xFF) - 128 == -128 ? -127 : (int)((h >> 8) & 0xFF) - 128);
    }
    if (threadIdx.x == 0) {
        const uint64_t h = mix64(base ^ 0xD1B54A32D192ED03ull);
        const float a = 0.005f + 0.045f * (float)(h & 0xFFFF) / 65535.0f;
        const float b = 0.005f + 0.045f * (float)((h >> 16) & 0xFFFF) / 65535.0f;
        if (bits == 4) {  // BF16 block scales (the codes above are read as nibbles)
            for (int g = 0; g < hd / 64; g++) {
                reinterpret_cast<uint16_t *>(ks)[slot * (hd / 64) + g] = (uint16_t)(__float_as_uint(a) >> 16);
                reinterpret_cast<uint16_t *>(vs)[slot * (hd / 64) + g] = (uint16_t)(__float_as_uint(b) >> 16);
            }
        } else {
            ks[slot] = a;
            vs[slot] = b;
        }
    }
}

void launch_kv_synthetic(hipStream_t st, int8_t *kq, int8_t *vq, float *ks, float *vs, int layers_kv, int cap,
                         int n_pos, int hd, int bits, uint64_t seed) {
    if (n_pos <= 0) return;
    hipLaunchKernelGGL(kv_synthetic_kernel, dim3((unsigned)((size_t)layers_kv * n_pos)), dim3(128), 0, st, kq, vq, ks,
                       vs, layers_kv, cap, n_pos, hd, bits, seed);
    hip_check(hipGetLastError(), "kv_synthetic launch");
}

// Advances the device position counter after a step (keeps graph replays argument-free).
__global__ void advance_pos_kernel(int *pos, int n) {
    if (threadIdx.x == 0) pos[0] += n;
}

void launch_advance_pos(hipStream_t st, int *pos, int n) {
    hipLaunchKernelGGL(advance_pos_kernel, dim3(1), dim3(64), 0, st, pos, n);
    hip_check(hipGetLastError(), "advance_pos launch");
}

}  // namespace k2t
