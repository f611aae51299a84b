// Activation rotation + int8 chunk quantization for gfx950.
//
// Replaces Int8ChunkActivation::populate_fwht / populate_rmsnorm_fwht /
// populate_chunk_fwht_raw (simd_lut.rs:2954-3196).  One wavefront per 64-column chunk,
// lane i holds element i: optional (x*inv_rms)*w, sign flip with the chunk's SplitMix64
// mask, x0.125, six butterfly stages through lane exchanges in the reference's order,
// wave max, 127/max, round-half-even, wave sum.  Every float operation is the
// reference's, so q / scales / sums are bit-identical given the same inputs.
#include <float.h>

#include <algorithm>

#include "k2t_device.h"
#include "k2t_expf.h"
#include "k2t_internal.h"

namespace k2t {

__global__ __launch_bounds__(256) void act_quant_kernel(const float *__restrict__ x,
                                                        const float *__restrict__ w,
                                                        const float *__restrict__ inv_rms, int K,
                                                        int total_chunks, int8_t *__restrict__ q,
                                                        float *__restrict__ scales,
                                                        int32_t *__restrict__ sums) {
    const uint32_t lane = threadIdx.x & 63;
    const int gc = blockIdx.x * 4 + (int)(threadIdx.x >> 6);
    if (gc >= total_chunks) return;
    const int nc = K / 64;
    const int tok = gc / nc, c = gc - tok * nc;
    float v = x[(size_t)gc * 64 + lane];
    if (w) v = (v * inv_rms[tok]) * w[(size_t)c * 64 + lane];
    v = flip_sign(v, hadamard_sign_bit((uint64_t)c, lane)) * 0.125f;
    v = wave_butterflies64(v, lane);
    const float mx = wave_max_f(fabsf(v));
    if (mx <= FLT_EPSILON) {
        q[(size_t)gc * 64 + lane] = 0;
        if (lane == 0) {
            scales[gc] = 0.0f;
            sums[gc] = 0;
        }
        return;
    }
    const float inv = 127.0f / mx;
    const int qi = (int)rintf(v * inv);
    const int s = wave_sum_i(qi);
    q[(size_t)gc * 64 + lane] = (int8_t)qi;
    if (lane == 0) {
        scales[gc] = mx / 127.0f;
        sums[gc] = s;
    }
}

// inv_rms[t] = 1 / sqrt(sum(x^2)/K + eps) per token (real_llm.rs:6929), one block per token.
__global__ __launch_bounds__(256) void inv_rms_kernel(const float *__restrict__ x, float eps, int K,
                                                      float *__restrict__ out) {
    __shared__ float part[4];
    const float *xt = x + (size_t)blockIdx.x * K;
    float s = 0.0f;
    for (int i = threadIdx.x; i < K; i += 256) {
        const float v = xt[i];
        s = fmaf(v, v, s);
    }
    s = wave_sum_f(s);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        const float tot = (part[0] + part[1]) + (part[2] + part[3]);
        out[blockIdx.x] = 1.0f / sqrtf(tot / (float)K + eps);
    }
}

// inv_rms[t] = 1 / sqrt(sum(x^2)/K + eps) with the sum of squares in the reference's x86
// order (dot_f32_fast, portable branch, real_llm.rs:911-926; rms_norm 9858-9861): four
// accumulators, acc[k] += x[i+k]*x[i+k] over i = 0, 4, 8, ... (each product rounded, then
// added), (acc0 + acc1) + (acc2 + acc3), then the K % 4 remainder in order.  One wave per
// token; lanes 0-3 hold the accumulators and run their chains sequentially, eight loads
// ahead.  Used by the exact-order decode mode.
__global__ __launch_bounds__(64) void inv_rms_x86_kernel(const float *__restrict__ x, float eps, int K,
                                                         float *__restrict__ out) {
    const uint32_t lane = threadIdx.x;
    const float *xt = x + (size_t)blockIdx.x * K;
    const int n4 = K / 4;
    float acc = 0.0f;
    if (lane < 4) {
        int j = 0;
        for (; j + 8 <= n4; j += 8) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) v[u] = xt[4 * (j + u) + lane];
#pragma unroll
            for (int u = 0; u < 8; u++) acc = acc + v[u] * v[u];
        }
        for (; j < n4; j++) {
            const float v = xt[4 * j + lane];
            acc = acc + v * v;
        }
    }
    const float a0 = lane_val(acc, 0), a1 = lane_val(acc, 1), a2 = lane_val(acc, 2), a3 = lane_val(acc, 3);
    if (lane == 0) {
        float sum = (a0 + a1) + (a2 + a3);
        for (int i = 4 * n4; i < K; i++) sum = sum + xt[i] * xt[i];
        const float mean_sq = sum / (float)K;
        out[blockIdx.x] = 1.0f / sqrtf(mean_sq + eps);
    }
}

void launch_inv_rms_x86(hipStream_t st, const float *x, float eps, int K, int ntok, float *inv_rms) {
    if (ntok <= 0) return;
    hipLaunchKernelGGL(inv_rms_x86_kernel, dim3(ntok), dim3(64), 0, st, x, eps, K, inv_rms);
    hip_check(hipGetLastError(), "inv_rms_x86 launch");
}

// y[i] = expf_rn(x[i]) (k2t_expf_device: the exact-order mode's exponential on the GPU).
__global__ __launch_bounds__(256) void expf_map_kernel(const float *__restrict__ x, float *__restrict__ y, size_t n) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) y[i] = expf_rn(x[i]);
}

void launch_expf_map(hipStream_t st, const float *x, float *y, size_t n) {
    const size_t blocks = std::min<size_t>((n + 255) / 256, 4096);
    hipLaunchKernelGGL(expf_map_kernel, dim3((unsigned)blocks), dim3(256), 0, st, x, y, n);
    hip_check(hipGetLastError(), "expf_map launch");
}

void launch_act_quant(k2t_ctx *ctx, const float *x, const float *w, const float *inv_rms, int K,
                      int ntok, int8_t *q, float *scales, int32_t *sums) {
    const int total = (K / 64) * ntok;
    if (total <= 0) return;
    hipLaunchKernelGGL(act_quant_kernel, dim3((total + 3) / 4), dim3(256), 0, ctx->stream, x, w,
                       inv_rms, K, total, q, scales, sums);
    hip_check(hipGetLastError(), "act_quant launch");
}

void launch_inv_rms(k2t_ctx *ctx, const float *x, float eps, int K, int ntok, float *inv_rms) {
    if (ntok <= 0) return;
    hipLaunchKernelGGL(inv_rms_kernel, dim3(ntok), dim3(256), 0, ctx->stream, x, eps, K, inv_rms);
    hip_check(hipGetLastError(), "inv_rms launch");
}

// Streaming read of `bytes` (measurement of the single-launch HBM read ceiling that the
// GEMVs are compared with): 512 workgroups of 512 threads, each reading one contiguous
// 1/512 of the buffer with four 16-byte nontemporal loads in flight per thread.  The
// XOR of the data is written only if it equals a marker, so the loads are not removed.
__global__ __launch_bounds__(512) void stream_read_kernel(const uint4 *__restrict__ p, size_t n16,
                                                          uint32_t *__restrict__ sink) {
    const size_t per = (n16 + gridDim.x - 1) / gridDim.x;
    const size_t b0 = (size_t)blockIdx.x * per, b1 = min(n16, b0 + per);
    uint32_t acc = 0;
    for (size_t i = b0 + threadIdx.x; i < b1; i += 4 * (size_t)blockDim.x) {
        uint4 v[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const size_t j = i + (size_t)u * blockDim.x;
            v[u] = j < b1 ? load_stream16(p + j) : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < 4; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    if (acc == 0x6B327452u) sink[0] = acc;
}

void launch_stream_read(hipStream_t st, const void *src, size_t bytes, uint32_t *sink) {
    if (bytes == 0) return;
    hipLaunchKernelGGL(stream_read_kernel, dim3(512), dim3(512), 0, st, reinterpret_cast<const uint4 *>(src),
                       bytes / 16, sink);
    hip_check(hipGetLastError(), "stream_read launch");
}

}  // namespace k2t
