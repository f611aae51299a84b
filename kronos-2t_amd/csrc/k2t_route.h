// Sparse-MoE routing on one wave per expert row (device code shared by the standalone
// route kernel and the grouped gate_up GEMV that runs the routing in its own launch).
#pragma once
#include <math.h>

#include "../../include/k2t_hip.h"
#include "k2t_device.h"

namespace k2t {

// 64-bit hand-off words {epoch, value}: one agent-scope atomic store, so the value and its
// ready mark arrive together, with no fence.
__device__ __forceinline__ void word_store(unsigned long long *p, uint32_t v, uint32_t epoch) {
    __hip_atomic_store(p, ((unsigned long long)epoch << 32) | v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long word_load(const unsigned long long *p) {
    return __hip_atomic_load(const_cast<unsigned long long *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Candidate keys: the score's bits made order-preserving as an unsigned number (negative
// values inverted, positive ones with the top bit set; -0 is added to +0 first so the two
// zeros tie as floats do) in the high word, ~index in the low word.  The largest key is
// the largest score with the lowest index among equals, the order of the reference's
// strict comparisons, and it is one unsigned 64-bit comparison: no branch per step.
__device__ __forceinline__ unsigned long long score_key(float v, int idx) {
    uint32_t u = __float_as_uint(v + 0.0f);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)u << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)idx);
}
__device__ __forceinline__ float key_score(unsigned long long k) {
    const uint32_t u = (uint32_t)(k >> 32);
    return __uint_as_float((u & 0x80000000u) ? (u & 0x7FFFFFFFu) : ~u);
}
__device__ __forceinline__ int key_index(unsigned long long k) { return (int)(0xFFFFFFFFu - (uint32_t)k); }

template <int CTRL>
__device__ __forceinline__ void row_rotate_max(unsigned long long &k) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)k, CTRL, 0xF, 0xF, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)(k >> 32), CTRL, 0xF, 0xF, false);
    const unsigned long long o = ((unsigned long long)hi << 32) | lo;
    k = o > k ? o : k;
}
// The largest key of the wave (uniform): rotations by 1, 2, 4 and 8 inside each 16-lane
// row (DPP), then the four rows' results read with v_readlane.
__device__ __forceinline__ unsigned long long wave_max_key(unsigned long long k) {
    row_rotate_max<0x121>(k);  // row_ror:1
    row_rotate_max<0x122>(k);  // row_ror:2
    row_rotate_max<0x124>(k);  // row_ror:4
    row_rotate_max<0x128>(k);  // row_ror:8
    unsigned long long b = 0;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const unsigned long long o = ((unsigned long long)(uint32_t)lane_val((int)(k >> 32), 16 * r) << 32) |
                                     (uint32_t)lane_val((int)(uint32_t)k, 16 * r);
        b = o > b ? o : b;
    }
    return b;
}

// route_sorted (sparse_moe.rs:86-182) for E <= 256 experts on one wave.  With `pub` set,
// id r of the sorted route is also published as the {epoch, id} word pub[r], for
// consumers inside the same launch.  Top-k picks the
// largest score with the lowest id among equals, the order select_topk_by_score's strict
// comparisons give; the top-k sums run in selection order like the reference's loops.
// sc[j] holds the logit of expert lane + 64 j (-inf past E) on entry.
__device__ inline void select_routes(float sc[4], int lane, int E, int k, int norm_topk, int scoring,
                                     int *__restrict__ ids, float *__restrict__ wts,
                                     unsigned long long *__restrict__ pub, uint32_t epoch) {
#pragma unroll
    for (int j = 0; j < 4; j++)
        if (sc[j] != sc[j]) sc[j] = -INFINITY;  // NaN never wins a comparison: rank it last
    if (scoring == K2T_MOE_SOFTMAX) {
        float m = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
        m = wave_max_f(m);
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            sc[j] = lane + 64 * j < E ? expf(sc[j] - m) : 0.0f;
            s += sc[j];
        }
        s = wave_sum_f(s);
        const float inv_all = s > 0.0f ? 1.0f / s : 1.0f / (float)E;
#pragma unroll
        for (int j = 0; j < 4; j++) sc[j] = lane + 64 * j < E ? sc[j] * inv_all : -INFINITY;
    } else if (scoring == K2T_MOE_SIGMOID) {
#pragma unroll
        for (int j = 0; j < 4; j++)
            sc[j] = lane + 64 * j < E && sc[j] == sc[j] ? 1.0f / (1.0f + expf(-sc[j])) : -INFINITY;
    }
    // Selection round r leaves its (id, score) in lane r's registers; a picked key is
    // replaced by 0, below every real key (-inf's included), for the later rounds.
    unsigned long long key[4];
#pragma unroll
    for (int j = 0; j < 4; j++) key[j] = score_key(sc[j], lane + 64 * j);
    int my_id = 0;
    float my_w = 0.0f;
    for (int r = 0; r < k; r++) {
        unsigned long long b = key[0];
#pragma unroll
        for (int j = 1; j < 4; j++) b = key[j] > b ? key[j] : b;
        b = wave_max_key(b);
        const int bi = key_index(b);
        if (lane == r) {
            my_id = min(bi, E - 1);  // every id indexes a record of the bank, whatever the scores
            my_w = key_score(b);
        }
#pragma unroll
        for (int j = 0; j < 4; j++) key[j] = lane + 64 * j == bi ? 0ull : key[j];
    }
    // Weight normalization; the sums run over the selections in selection order.
    if (scoring == K2T_MOE_TOPK_SOFTMAX) {
        const float mz = lane_val(my_w, 0);
        const float ex = lane < k ? expf(my_w - mz) : 0.0f;
        float s = 0.0f;
        for (int r = 0; r < k; r++) s += lane_val(ex, r);
        const float inv = s > 0.0f ? 1.0f / s : 1.0f / (float)k;
        my_w = ex * inv;
    } else if (norm_topk) {
        float s = 0.0f;
        for (int r = 0; r < k; r++) s += lane_val(my_w, r);
        if (s > 0.0f) my_w *= 1.0f / s;
    }
    // Ascending expert id (sparse_moe.rs:170-179): lane r's rank among the k selections
    // (ids are distinct, ties in id order are impossible).
    int rank = 0;
    for (int r = 0; r < k; r++) {
        const int other = lane_val(my_id, r);
        rank += (r != lane && other < my_id) ? 1 : 0;
    }
    if (lane < k) {
        ids[rank] = my_id;
        wts[rank] = my_w;
        if (pub) word_store(pub + rank, (uint32_t)my_id, epoch);
    }
}


// Router logit of expert e on one wave: x_norm = (x * inv_rms) * w formed on the fly
// (rms_norm, real_llm.rs:9858-9898; the sum of squares in the order of the GEMV's fused
// builder, so x_norm matches the expert activations' source), dot as in dot_f32_moe
// (sparse_moe.rs:1644-1655) with a tree reduction, published as words[e] = {epoch, logit}.
// Every load is issued before the first wait: the vectors from clamped indices (masked
// afterwards; a load under a lane condition became a branch per load) and the bias.
// The caller passes a wave-uniform e < E.
template <int NJ>  // float4 per lane of each vector: d <= 256 * NJ
__device__ __forceinline__ void route_logit(const float *__restrict__ x, const float *__restrict__ nw, float eps,
                                            int d, const float *__restrict__ W, const float *__restrict__ bias,
                                            int e, uint32_t lane, uint32_t epoch,
                                            unsigned long long *__restrict__ words) {
    const float4 *x4 = reinterpret_cast<const float4 *>(x);
    const float4 *w4 = reinterpret_cast<const float4 *>(nw);
    const float4 *r4 = reinterpret_cast<const float4 *>(W + (size_t)e * d);
    const int n4 = d / 4;
    float4 xv[NJ], wv[NJ], rv[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int i = min((int)lane + 64 * j, n4 - 1);
        xv[j] = x4[i];
        wv[j] = w4[i];
        rv[j] = r4[i];
    }
    const float bv = bias ? bias[e] : 0.0f;
    const float4 zero4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int j = 0; j < NJ; j++)
        if ((int)lane + 64 * j >= n4) xv[j] = wv[j] = rv[j] = zero4;
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        ss = fmaf(xv[j].x, xv[j].x, ss);
        ss = fmaf(xv[j].y, xv[j].y, ss);
        ss = fmaf(xv[j].z, xv[j].z, ss);
        ss = fmaf(xv[j].w, xv[j].w, ss);
    }
    ss = wave_sum_f(ss);
    const float inv_rms = 1.0f / sqrtf(ss / (float)d + eps);
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        acc = fmaf((xv[j].x * inv_rms) * wv[j].x, rv[j].x, acc);
        acc = fmaf((xv[j].y * inv_rms) * wv[j].y, rv[j].y, acc);
        acc = fmaf((xv[j].z * inv_rms) * wv[j].z, rv[j].z, acc);
        acc = fmaf((xv[j].w * inv_rms) * wv[j].w, rv[j].w, acc);
    }
    acc = wave_sum_f(acc);
    if (lane == 0) word_store(words + e, __float_as_uint(bias ? acc + bv : acc), epoch);
}

// The selection wave: waits (bounded by spin_limit; on timeout raises *err and still
// writes in-range ids) for the E logit words of this epoch, one load each in flight
// together, then runs select_routes.
__device__ inline void route_collect(const unsigned long long *__restrict__ words, int E, uint32_t epoch,
                                     uint32_t spin_limit, int *__restrict__ err, uint32_t lane, int k,
                                     int norm_topk, int scoring, int *__restrict__ ids, float *__restrict__ wts,
                                     unsigned long long *__restrict__ pub) {
    unsigned long long w[4];
#pragma unroll
    for (int j = 0; j < 4; j++) w[j] = word_load(words + min((int)lane + 64 * j, E - 1));
    float sc[4];
    bool ok = true;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int ee = (int)lane + 64 * j;
        sc[j] = -INFINITY;
        if (ee >= E) continue;
        for (uint32_t spins = 0; ok && (uint32_t)(w[j] >> 32) != epoch; spins++) {
            if (spins > spin_limit) {
                ok = false;
                __hip_atomic_store(err, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
            w[j] = word_load(words + ee);
        }
        if (ok) sc[j] = __uint_as_float((uint32_t)w[j]);
    }
    select_routes(sc, (int)lane, E, k, norm_topk, scoring, ids, wts, pub, epoch);
}

// Routing inside a larger launch (d <= 2048): each router row is split over two waves so a
// wave has 48 registers of loads in flight (x, w, r of its half).  Unit u = 2 e + h reads
// half h of row e: parts[u] = {epoch, sum over the half of (x * w) * r} and, for e = 0,
// parts[2 E + h] = {epoch, sum over the half of x * x}.  route_collect_parts forms
// logit_e = (parts[2e] + parts[2e+1]) * inv_rms (+ bias), inv_rms from the two sums of
// squares -- the same RMSNorm-then-dot, with inv_rms applied once to the dot (the fp32
// dot order is not bit-exact against the reference in any case).
__device__ __forceinline__ void route_logit_half(const float *__restrict__ x, const float *__restrict__ nw, int d,
                                                 const float *__restrict__ W, int u, uint32_t lane,
                                                 uint32_t epoch, int E, unsigned long long *__restrict__ parts) {
    constexpr int NJ = 4;
    const int e = u >> 1, h = u & 1;
    const int nh = d / 8;  // float4 per half
    const float4 *x4 = reinterpret_cast<const float4 *>(x) + h * nh;
    const float4 *w4 = reinterpret_cast<const float4 *>(nw) + h * nh;
    const float4 *r4 = reinterpret_cast<const float4 *>(W + (size_t)e * d) + h * nh;
    float4 xv[NJ], wv[NJ], rv[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int i = min((int)lane + 64 * j, nh - 1);
        xv[j] = x4[i];
        wv[j] = w4[i];
        rv[j] = r4[i];
    }
    const float4 zero4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int j = 0; j < NJ; j++)
        if ((int)lane + 64 * j >= nh) xv[j] = wv[j] = rv[j] = zero4;
    float ss = 0.0f, acc = 0.0f;
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        ss = fmaf(xv[j].x, xv[j].x, ss);
        ss = fmaf(xv[j].y, xv[j].y, ss);
        ss = fmaf(xv[j].z, xv[j].z, ss);
        ss = fmaf(xv[j].w, xv[j].w, ss);
        acc = fmaf(xv[j].x * wv[j].x, rv[j].x, acc);
        acc = fmaf(xv[j].y * wv[j].y, rv[j].y, acc);
        acc = fmaf(xv[j].z * wv[j].z, rv[j].z, acc);
        acc = fmaf(xv[j].w * wv[j].w, rv[j].w, acc);
    }
    acc = wave_sum_f(acc);
    if (e == 0) ss = wave_sum_f(ss);
    if (lane == 0) {
        word_store(parts + u, __float_as_uint(acc), epoch);
        if (e == 0) word_store(parts + 2 * E + h, __float_as_uint(ss), epoch);
    }
}

// Bounded wait for a word of this epoch (on timeout raises *err and returns 0).
__device__ __forceinline__ float await_word(const unsigned long long *__restrict__ p, unsigned long long w,
                                            uint32_t epoch, uint32_t spin_limit, int *__restrict__ err, bool &ok) {
    for (uint32_t spins = 0; ok && (uint32_t)(w >> 32) != epoch; spins++) {
        if (spins > spin_limit) {
            ok = false;
            __hip_atomic_store(err, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            break;
        }
        __builtin_amdgcn_s_sleep(1);
        w = word_load(p);
    }
    return ok ? __uint_as_float((uint32_t)w) : 0.0f;
}

__device__ inline void route_collect_parts(const unsigned long long *__restrict__ parts, int E, int d, float eps,
                                           const float *__restrict__ bias, uint32_t epoch, uint32_t spin_limit,
                                           int *__restrict__ err, uint32_t lane, int k, int norm_topk, int scoring,
                                           int *__restrict__ ids, float *__restrict__ wts,
                                           unsigned long long *__restrict__ pub) {
    unsigned long long w[4][2], ws[2];
    float bv[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int e = min((int)lane + 64 * j, E - 1);
        w[j][0] = word_load(parts + 2 * e);
        w[j][1] = word_load(parts + 2 * e + 1);
        bv[j] = bias ? bias[e] : 0.0f;
    }
    ws[0] = word_load(parts + 2 * E);
    ws[1] = word_load(parts + 2 * E + 1);
    bool ok = true;
    const float s0 = await_word(parts + 2 * E, ws[0], epoch, spin_limit, err, ok);
    const float s1 = await_word(parts + 2 * E + 1, ws[1], epoch, spin_limit, err, ok);
    const float inv_rms = 1.0f / sqrtf((s0 + s1) / (float)d + eps);
    float sc[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int e = (int)lane + 64 * j;
        sc[j] = -INFINITY;
        if (e >= E) continue;
        const float p0 = await_word(parts + 2 * e, w[j][0], epoch, spin_limit, err, ok);
        const float p1 = await_word(parts + 2 * e + 1, w[j][1], epoch, spin_limit, err, ok);
        if (ok) sc[j] = bias ? (p0 + p1) * inv_rms + bv[j] : (p0 + p1) * inv_rms;
    }
    select_routes(sc, (int)lane, E, k, norm_topk, scoring, ids, wts, pub, epoch);
}

}  // namespace k2t
