// Device helpers of the KV cache and of a qkv row's head post-processing, shared by the
// model kernels (k2t_model.hip) and the matrix-core GEMV's q / k / v epilogue
// (k2t_gemm_mfma.hip): sliding-window slots, the NF4 KV codebook, the int8 / NF4 K / V
// store of one rotated head, and bias + q / k RMSNorm + RoPE of one head.
#pragma once

#include <float.h>
#include <math.h>

#include "k2t_device.h"
#include "k2t_internal.h"

namespace k2t {

// slot_of_pos (real_llm.rs:1116-1122)
__device__ __forceinline__ int ring_slot(const KvRing &r, int pos) {
    return (r.ring == 0 || pos < r.sinks) ? pos : r.sinks + (pos - r.sinks) % r.ring;
}
// active_kv_len / active_kv_pos (real_llm.rs:8596-8612): the sinks, then the last
// window - sinks positions, once the sequence is longer than the window.
__device__ __forceinline__ int active_len(const KvRing &r, int seq) {
    return (r.window > 0 && seq > r.window) ? r.window : seq;
}
__device__ __forceinline__ int active_pos(const KvRing &r, int idx, int seq) {
    return (r.window > 0 && seq > r.window && idx >= r.sinks) ? (seq - (r.window - r.sinks)) + (idx - r.sinks) : idx;
}

// NF4_DEFAULT_CODEBOOK_I8 (simd_lut.rs:4338-4350) as v_perm table words, bytes 0-15.
constexpr uint32_t kNf4Cb0 = 0xC6B5A081u;  // -127 -96 -75 -58
constexpr uint32_t kNf4Cb1 = 0xFAEEE1D4u;  // -44 -31 -18 -6
constexpr uint32_t kNf4Cb2 = 0x2C1F1206u;  // 6 18 31 44
constexpr uint32_t kNf4Cb3 = 0x7F604B3Au;  // 58 75 96 127

__device__ __forceinline__ int nf4_cb_value(int i) {
    const uint32_t w = i < 4 ? kNf4Cb0 : i < 8 ? kNf4Cb1 : i < 12 ? kNf4Cb2 : kNf4Cb3;
    return (int)(int8_t)((w >> (8 * (i & 3))) & 0xFFu);
}

// nf4_nearest_idx (real_llm.rs:8614-8644): midpoint thresholds of the default codebook.
__device__ __forceinline__ int nf4_nearest_idx(float y) {
    const float a = fabsf(y);
    int p;
    if (a < 37.5f) p = a < 12.0f ? 0 : (a < 24.5f ? 1 : 2);
    else if (a < 85.5f) p = a < 51.0f ? 3 : (a < 66.5f ? 4 : 5);
    else p = a < 111.5f ? 6 : 7;
    return y >= 0.0f ? 8 + p : 7 - p;
}

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float v) {
    const uint32_t b = __float_as_uint(v);
    if ((b & 0x7F800000u) == 0x7F800000u && (b & 0x007FFFFFu)) return (uint16_t)((b >> 16) | 0x40u);
    return (uint16_t)((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16);
}

// store_hadamard_q4_head_raw (real_llm.rs:8646-8700) for one rotated 64-block held one
// element per lane: NF4 codes against 127/max, the least-squares scale num/den summed
// in element order (as the reference's loop), rounded to BF16, then the final codes.
// Byte h*16 + i holds element h*32 + i (low nibble) and h*32 + 16 + i (high nibble).
__device__ __forceinline__ void store_q4_block(float v, uint32_t lane, uint8_t *__restrict__ dst32,
                                               uint16_t *__restrict__ dst_s) {
    const float mx = wave_max_f(fabsf(v));
    if (mx < 1e-30f) {
        if (lane < 32) dst32[lane] = 0x88;
        if (lane == 0) *dst_s = 0;
        return;
    }
    const float inv0 = 127.0f / mx;
    const float c = (float)nf4_cb_value(nf4_nearest_idx(v * inv0));
    const float vc = v * c, cc = c * c;
    float num = 0.0f, den = 0.0f;
#pragma unroll
    for (int j = 0; j < 64; j++) {
        num += lane_val(vc, j);
        den += lane_val(cc, j);
    }
    const float s_ref = (den > 1e-12f && num > 0.0f) ? num / den : mx / 127.0f;
    const uint16_t sb = f32_to_bf16_rne(s_ref);
    const float s_fin = __uint_as_float((uint32_t)sb << 16);
    const float inv_fin = s_fin > 1e-30f ? 1.0f / s_fin : 0.0f;
    const int idx = nf4_nearest_idx(v * inv_fin);
    const int hi = __shfl(idx, (int)lane + 16, kWave);
    if ((lane & 31u) < 16u) dst32[(lane >> 5) * 16 + (lane & 15u)] = (uint8_t)(idx | (hi << 4));
    if (lane == 0) *dst_s = sb;
}

// One rotated head (lane holds elements lane and 64 + lane) into KV slot `slot`: int8 with
// one scale (store_hadamard_q8_head*, real_llm.rs:8282-8365) or NF4 per 64-block.
__device__ __forceinline__ void kv_store_head(float r0, float r1, int nb, uint32_t lane, int bits, int hd, size_t slot,
                                              int8_t *__restrict__ qbuf, float *__restrict__ sbuf) {
    if (bits == 4) {
        uint8_t *q4 = reinterpret_cast<uint8_t *>(qbuf) + slot * (size_t)(hd / 2);
        uint16_t *s16 = reinterpret_cast<uint16_t *>(sbuf) + slot * (size_t)nb;
        store_q4_block(r0, lane, q4, s16);
        if (nb > 1) store_q4_block(r1, lane, q4 + 32, s16 + 1);
        return;
    }
    const float mx = wave_max_f(fmaxf(fabsf(r0), fabsf(r1)));
    int8_t *dst = qbuf + slot * hd;
    float *sdst = sbuf + slot;
    if (mx <= FLT_EPSILON) {
        dst[lane] = 0;
        if (nb > 1) dst[64 + lane] = 0;
        if (lane == 0) *sdst = 0.0f;
        return;
    }
    const float inv = 127.0f / mx;
    dst[lane] = (int8_t)(int)rintf(r0 * inv);
    if (nb > 1) dst[64 + lane] = (int8_t)(int)rintf(r1 * inv);
    if (lane == 0) *sdst = mx / 127.0f;
}

// Bias, per-head q / k RMSNorm (apply_qk_norm_rope / apply_per_head_rms_norm,
// real_llm.rs:8139-8178: inv_rms = 1/sqrt(sum(v^2) * (1/hd) + eps), v = (v*inv_rms)*w,
// before RoPE) and RoPE (q and k heads) of one head of a qkv row; lane holds elements
// lane and 64 + lane.
// head_post_vals works on the head's values already in v0 / v1; head_post loads them.
__device__ __forceinline__ void head_post_vals(int head, int nq, int nkv, int hd, const float *__restrict__ bias,
                                               const float *__restrict__ qn, const float *__restrict__ kn, float eps,
                                               const float *__restrict__ rope, int pos, uint32_t lane, float &v0,
                                               float &v1, bool exact = false) {
    const int nb = hd / 64;
    if (bias) {
        v0 = v0 + bias[head * hd + lane];
        if (nb > 1) v1 = v1 + bias[head * hd + 64 + lane];
    }
    const float *hn = head < nq ? qn : (head < nq + nkv ? kn : nullptr);
    if (hn) {
        float inv_rms;
        if (exact) {
            // the x86 reference's order (dot_f32_fast, real_llm.rs:911-926): four sequential
            // accumulators over elements k, k + 4, ...; every lane runs the same chain
            float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            for (int e = 0; e < hd; e += 4)
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const float x = e + k < 64 ? lane_val(v0, e + k) : lane_val(v1, e + k - 64);
                    acc[k] = acc[k] + x * x;
                }
            const float sum = (acc[0] + acc[1]) + (acc[2] + acc[3]);
            inv_rms = 1.0f / sqrtf(sum / (float)hd + eps);
        } else {
            float ss = v0 * v0;
            if (nb > 1) ss = fmaf(v1, v1, ss);
            ss = wave_sum_f(ss);
            inv_rms = 1.0f / sqrtf(ss * (1.0f / (float)hd) + eps);
        }
        v0 = (v0 * inv_rms) * hn[lane];
        if (nb > 1) v1 = (v1 * inv_rms) * hn[64 + lane];
    }
    if (head < nq + nkv) {
        const float *row = rope + (size_t)pos * hd;
        if (nb == 1) {  // pairs (i, i+32) live in lanes lane and lane^32
            const float other = xor_lane(v0, 32);
            const uint32_t i = lane & 31u;
            const float c = row[i], s = row[32 + i];
            v0 = lane < 32 ? v0 * c - other * s : v0 * c + other * s;
        } else {  // pairs (i, i+64): element lane and 64+lane of this lane
            const float c = row[lane], s = row[64 + lane];
            const float x0 = v0, x1 = v1;
            v0 = x0 * c - x1 * s;
            v1 = x1 * c + x0 * s;
        }
    }
}

// head_post_vals at head size 64 (fast path) with sixteen lanes per head, lane slice sl
// holding elements 4 sl .. 4 sl + 3: the same operations on the same operands.  The
// q / k RMSNorm's sum of squares follows wave_sum_f's pairs (elements i, i ^ 1 and i ^ 2 in
// registers, i ^ 4 .. i ^ 16 by slice exchanges ^1 .. ^4, the halves by ^8; IEEE addition
// commutes, so the bits are the same), RoPE's partner i ^ 32 is slice sl ^ 8.
__device__ __forceinline__ void head_post4(int head, int nq, int nkv, const float *__restrict__ bias,
                                           const float *__restrict__ qn, const float *__restrict__ kn, float eps,
                                           const float *__restrict__ rope, int pos, uint32_t sl, float (&v)[4]) {
    if (bias) {
        const float4 b4 = *reinterpret_cast<const float4 *>(bias + head * 64 + 4 * sl);
        v[0] = v[0] + b4.x;
        v[1] = v[1] + b4.y;
        v[2] = v[2] + b4.z;
        v[3] = v[3] + b4.w;
    }
    const float *hn = head < nq ? qn : (head < nq + nkv ? kn : nullptr);
    if (hn) {
        float ss = (v[0] * v[0] + v[1] * v[1]) + (v[2] * v[2] + v[3] * v[3]);
        ss += xchg1(ss);
        ss += xchg2(ss);
        ss += xchg4(ss);
        ss += xchg8(ss);
        const float inv_rms = 1.0f / sqrtf(ss * (1.0f / 64.0f) + eps);
        const float4 w4 = *reinterpret_cast<const float4 *>(hn + 4 * sl);
        v[0] = (v[0] * inv_rms) * w4.x;
        v[1] = (v[1] * inv_rms) * w4.y;
        v[2] = (v[2] * inv_rms) * w4.z;
        v[3] = (v[3] * inv_rms) * w4.w;
    }
    if (head < nq + nkv) {
        const float *row = rope + (size_t)pos * 64;
        const uint32_t i0 = (4u * sl) & 31u;  // element index mod 32 of v[0]
        const float4 c4 = *reinterpret_cast<const float4 *>(row + i0);
        const float4 s4 = *reinterpret_cast<const float4 *>(row + 32 + i0);
        const float cs[4] = {c4.x, c4.y, c4.z, c4.w}, sn[4] = {s4.x, s4.y, s4.z, s4.w};
        float other[4];
#pragma unroll
        for (int j = 0; j < 4; j++) other[j] = xchg8(v[j]);
        const bool lower = sl < 8u;
#pragma unroll
        for (int j = 0; j < 4; j++) v[j] = lower ? v[j] * cs[j] - other[j] * sn[j] : v[j] * cs[j] + other[j] * sn[j];
    }
}

__device__ __forceinline__ void head_post(const float *__restrict__ h, int head, int nq, int nkv, int hd,
                                          const float *__restrict__ bias, const float *__restrict__ qn,
                                          const float *__restrict__ kn, float eps, const float *__restrict__ rope,
                                          int pos, uint32_t lane, float &v0, float &v1, bool exact = false) {
    v0 = h[lane];
    v1 = hd > 64 ? h[64 + lane] : 0.0f;
    head_post_vals(head, nq, nkv, hd, bias, qn, kn, eps, rope, pos, lane, v0, v1, exact);
}

}  // namespace k2t
