// Bandwidth-bound quantized GEMV / 4-token tile for gfx950.
//
// Replaces the stripe-range leaves of the reference's LinearBackend:
//   bit-plane  nibble4_sdot_stripe_range_raw / sdot_decode_neon   (simd_lut.rs:3536-4091)
//              nibble4_sdot_batch_stripe_range / sdot_batch_tile  (simd_lut.rs:4101-4331)
//   NF4        nf_sdot_stripe_range_raw / nf_sdot_decode_neon     (simd_lut.rs:5687-6364)
//              nf_sdot_batch_stripe_range                         (simd_lut.rs:6689-7034)
//
// Work unit = one workgroup per 16-row stripe; its waves split K into segments (as many
// as needed to put ~8 streaming waves on every CU).  Per step a wave reads the stripe's
// 512 nibble bytes of two chunks with one 128-bit load per lane (plus hi-plane bytes /
// BF16 scales), decodes codes (u, or codebook values through a v_perm byte table) and
// accumulates them against int8 activations with v_dot4_i32_i8.  Two DPP steps leave
// every lane with the exact i32 dot of 2 rows for its chunk.
//
// fp32 epilogue: the reference computes f = fma(float(dot)*sx, ws, f) per row in chunk
// order (simd_lut.rs:4030-4059 / 6334-6335).  With one segment the chain runs in
// registers; with several, every (row, chunk) term is staged in LDS and one lane per
// row replays the chain after a barrier.  Either way the result is bit-identical to
// the reference.  No global scratch, atomics or device-scope fences are used.
#include <float.h>

#include <algorithm>

#include "k2t_device.h"
#include "k2t_internal.h"

namespace k2t {

struct GemvParams {
    const uint8_t *pair;
    const uint8_t *tail;
    const int8_t *xq;
    const float *xs;
    const int32_t *xsum;
    float *out;
    int32_t *dots;
    size_t out_stride;
    size_t ptot;  // NF: bytes per pair stream
    int rows, K, nc, np;
    int s_lo, nstripes;  // stripes [s_lo, s_lo + nstripes)
    int nseg, cps;       // K segments per stripe (= waves per workgroup), chunks per segment
    int sgc;
    int tok_base;
    int lds_terms;  // 1: per-chunk terms in LDS (exact chain), 0: ordered partial sums
    uint32_t cb0, cb1, cb2, cb3;
};

// Sum over the 8 lanes of a 16-lane row that share a 4-row group (lane bits 0, 2, 3),
// transposing so that a lane with half=h keeps rows 2h and 2h+1 of its group.
__device__ __forceinline__ void reduce_rows(int a0, int a1, int a2, int a3, uint32_t half,
                                            int &r0, int &r1) {
    int s0 = half ? a0 : a2, s1 = half ? a1 : a3;
    int k0 = half ? a2 : a0, k1 = half ? a3 : a1;
    k0 += dpp_xor1(s0);
    k1 += dpp_xor1(s1);
    k0 += dpp_ror8(k0);
    k1 += dpp_ror8(k1);
    k0 += dpp_ror4(k0);
    k1 += dpp_ror4(k1);
    r0 = k0;
    r1 = k1;
}

// Registers of one fetched stripe-chunk record for one lane.
template <int NT>
struct Frag {
    uint4 w;
    uint4 h;
    uint32_t ws;
    uint2 x[NT];
};

// One workgroup = one 16-row stripe; its nseg waves take consecutive K segments.
// A wave steps over chunk pairs: lanes 0-31 decode chunk c, lanes 32-63 chunk c+1.
// Lane bits: 0 = half (8-column half of a 16-column block), 1 = g bit 0, 2-3 = k
// (16-column block), 4 = g bit 1, 5 = chunk parity.  A lane's 16 bytes are rows
// 4g..4g+3 x 8 columns; each quad of lanes reads 64 contiguous bytes and the row
// reduction stays inside a 16-lane DPP row.
// FMT 0: bit-plane Nibble4 with HP hi planes; FMT 1: NF4 codebook stripes.
template <int FMT, int HP, int NT, bool DOTS>
__global__ __launch_bounds__(1024) void gemv_kernel(GemvParams P) {
    constexpr int U = NT == 1 ? 4 : 2;  // chunk pairs fetched before use
    extern __shared__ float lds[];
    const uint32_t lane = threadIdx.x & 63;
    const int seg = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int s = P.s_lo + (int)blockIdx.x;
    const int tok0 = P.tok_base + (int)blockIdx.y * NT;
    const bool is_tail = s >= 2 * P.np;
    const uint32_t half = lane & 1u;
    const uint32_t g = ((lane >> 1) & 1u) | (((lane >> 4) & 1u) << 1);
    const uint32_t k = (lane >> 2) & 3u;
    const uint32_t par = lane >> 5;
    const uint32_t piece = k * 8u + g * 2u + half;
    const uint32_t sc_lane = (4u * g + 2u * half) * 2u;
    const uint32_t side = (uint32_t)(s & 1);
    const int c0 = seg * P.cps;
    const int c1 = min(P.nc, c0 + P.cps);
    constexpr int MAX_ODD = (1 << (4 + HP)) - 1;
    constexpr size_t PREC = 1024 + 256 * HP + 64;
    constexpr size_t TREC = 512 + 128 * HP + 32;
    const int row0 = s * 16 + (int)(4u * g + 2u * half);

    float f[NT][2];
#pragma unroll
    for (int t = 0; t < NT; t++) f[t][0] = f[t][1] = 0.0f;

    const int8_t *xbase = P.xq + (size_t)tok0 * P.K + k * 16 + half * 8;

    auto fetch = [&](Frag<NT> &fr, int c) {
        const uint8_t *nib, *scp, *hib = nullptr;
        if constexpr (FMT == 0) {
            if (is_tail) {
                const uint8_t *base = P.tail + (size_t)c * TREC;
                nib = base;
                hib = base + 512;
                scp = base + 512 + 128 * HP;
            } else {
                const uint8_t *base = P.pair + ((size_t)(s >> 1) * P.nc + c) * PREC;
                nib = base + side * 512u;
                hib = base + 1024u + side * 128u * HP;
                scp = base + 1024u + 256u * HP + side * 32u;
            }
            nib += piece * 16u;
            hib += (HP == 2 ? k * 64u : (k >> 1) * 64u) + g * 16u;
        } else {
            const int sg = c / P.sgc, cst = sg * P.sgc, sub = c - cst;
            if (is_tail) {
                const uint8_t *gb = P.tail + (size_t)sg * 32 + (size_t)cst * 512;
                nib = gb + 32 + (size_t)sub * 512;
                scp = gb;
            } else {
                const uint8_t *gb = P.pair + (size_t)(s >> 1) * P.ptot + (size_t)sg * 64 + (size_t)cst * 1024;
                nib = gb + 64 + (size_t)sub * 1024 + side * 512u;
                scp = gb + side * 32u;
            }
            nib += piece * 16u;
        }
        fr.w = load_stream16(nib);
        if constexpr (FMT == 0 && HP > 0) fr.h = load_stream16(hib);
        fr.ws = *reinterpret_cast<const uint32_t *>(scp + sc_lane);
#pragma unroll
        for (int t = 0; t < NT; t++) fr.x[t] = *reinterpret_cast<const uint2 *>(xbase + (size_t)t * P.K + c * 64);
    };

    // Decodes one record and returns the exact integer dots of rows row0, row0+1.
    auto dots_of = [&](const Frag<NT> &fr, int c, int (&r)[NT][2]) {
        uint32_t lo[4], hi[4];
        const uint32_t wd[4] = {fr.w.x, fr.w.y, fr.w.z, fr.w.w};
        const uint32_t hd[4] = {fr.h.x, fr.h.y, fr.h.z, fr.h.w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t d = wd[j];
            if constexpr (FMT == 0) {
                uint32_t l = d & 0x0F0F0F0Fu;
                uint32_t h = (d >> 4) & 0x0F0F0F0Fu;
                if constexpr (HP == 2) {
                    // 2-bit hi codes at shifts {4,6} (half 0) / {2,0} (half 1), simd_lut.rs:3376-3384;
                    // the rotations keep bits inside each byte once masked with 0x30.
                    const uint32_t hb = hd[j];
                    l |= __builtin_rotateright32(hb, half ? 30u : 0u) & 0x30303030u;
                    h |= __builtin_rotateright32(hb, half ? 28u : 2u) & 0x30303030u;
                } else if constexpr (HP == 1) {
                    // 1-bit hi code at bit (k even ? 4+sub : sub), sub = 2*half + nibble (3366-3375).
                    const uint32_t hb = hd[j];
                    const uint32_t e = ((k & 1u) ? 28u : 0u) + 2u * half;
                    l |= __builtin_rotateright32(hb, e) & 0x10101010u;
                    h |= __builtin_rotateright32(hb, (e + 1u) & 31u) & 0x10101010u;
                }
                lo[j] = l;
                hi[j] = h;
            } else {
                lo[j] = lut16(d & 0x07070707u, bit7_mask(d << 4), P.cb0, P.cb1, P.cb2, P.cb3);
                hi[j] = lut16((d >> 4) & 0x07070707u, bit7_mask(d), P.cb0, P.cb1, P.cb2, P.cb3);
            }
        }
#pragma unroll
        for (int t = 0; t < NT; t++) {
            int a[4];
#pragma unroll
            for (int j = 0; j < 4; j++)
                a[j] = __builtin_amdgcn_sdot4((int)lo[j], (int)fr.x[t].x,
                                              __builtin_amdgcn_sdot4((int)hi[j], (int)fr.x[t].y, 0, false), false);
            reduce_rows(a[0], a[1], a[2], a[3], half, r[t][0], r[t][1]);
            if constexpr (FMT == 0) {
                const int off = MAX_ODD * P.xsum[(size_t)(tok0 + t) * P.nc + c];
                r[t][0] = 2 * r[t][0] - off;
                r[t][1] = 2 * r[t][1] - off;
            }
        }
    };

    float2 *terms = reinterpret_cast<float2 *>(lds);  // [NT][nc][16] (a = float(dot)*sx, ws)

    for (int cb = c0; cb < c1; cb += 2 * U) {
        Frag<NT> fr[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int c = cb + 2 * u + (int)par;
            if (c < c1) fetch(fr[u], c);
            else fr[u] = Frag<NT>{};
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int ce = cb + 2 * u;  // even chunk of this pair (wave-uniform)
            if (ce >= c1) break;
            const int c = ce + (int)par;
            const bool has_odd = ce + 1 < c1;
            int r[NT][2];
            dots_of(fr[u], c < c1 ? c : ce, r);
            const float ws0 = bf16_lo(fr[u].ws), ws1 = bf16_hi(fr[u].ws);
            if constexpr (DOTS) {
                if (k == 0 && (par == 0 || has_odd)) {
                    if (row0 < P.rows) P.dots[(size_t)row0 * P.nc + c] = r[0][0];
                    if (row0 + 1 < P.rows) P.dots[(size_t)(row0 + 1) * P.nc + c] = r[0][1];
                }
            }
            if (P.nseg > 1 && P.lds_terms) {
                // Exact path for split K: every (row, chunk) term goes to LDS, one lane per
                // row replays the reference's fmaf chain afterwards.
                if (k == 0 && (par == 0 || has_odd)) {
#pragma unroll
                    for (int t = 0; t < NT; t++) {
                        const float sx = P.xs[(size_t)(tok0 + t) * P.nc + c];
                        float2 *tp = terms + ((size_t)t * P.nc + c) * 16 + (4u * g + 2u * half);
                        tp[0] = make_float2((float)r[t][0] * sx, ws0);
                        tp[1] = make_float2((float)r[t][1] * sx, ws1);
                    }
                }
                continue;
            }
            // In-register chain: the odd chunk's dots move to the even lanes.
#pragma unroll
            for (int t = 0; t < NT; t++) {
                const int o0 = __shfl_xor(r[t][0], 32, kWave);
                const int o1 = __shfl_xor(r[t][1], 32, kWave);
                const float ow0 = __shfl_xor(ws0, 32, kWave), ow1 = __shfl_xor(ws1, 32, kWave);
                const float sxe = P.xs[(size_t)(tok0 + t) * P.nc + ce];
                if (sxe != 0.0f) {
                    f[t][0] = fmaf((float)r[t][0] * sxe, ws0, f[t][0]);
                    f[t][1] = fmaf((float)r[t][1] * sxe, ws1, f[t][1]);
                }
                if (has_odd) {
                    const float sxo = P.xs[(size_t)(tok0 + t) * P.nc + ce + 1];
                    if (sxo != 0.0f) {
                        f[t][0] = fmaf((float)o0 * sxo, ow0, f[t][0]);
                        f[t][1] = fmaf((float)o1 * sxo, ow1, f[t][1]);
                    }
                }
            }
        }
    }

    if (P.nseg == 1) {
        if (k == 0 && par == 0) {
#pragma unroll
            for (int t = 0; t < NT; t++) {
                float *o = P.out + (size_t)(tok0 + t) * P.out_stride;
                if (row0 < P.rows) o[row0] = f[t][0];
                if (row0 + 1 < P.rows) o[row0 + 1] = f[t][1];
            }
        }
        return;
    }
    if (!P.lds_terms) {
        // Ordered partial sums (used when the per-chunk terms do not fit in LDS).
        if (k == 0 && par == 0) {
#pragma unroll
            for (int t = 0; t < NT; t++) {
                lds[((size_t)seg * NT + t) * 16 + 4u * g + 2u * half] = f[t][0];
                lds[((size_t)seg * NT + t) * 16 + 4u * g + 2u * half + 1] = f[t][1];
            }
        }
    }
    __syncthreads();
    if (seg != 0 || (int)lane >= 16 * NT) return;
    const int t = (int)lane / 16, rl = (int)lane % 16;
    const int row = s * 16 + rl;
    float acc = 0.0f;
    if (P.lds_terms) {
        const float *xs = P.xs + (size_t)(tok0 + t) * P.nc;
        const float2 *tp = terms + (size_t)t * P.nc * 16 + rl;
        for (int c = 0; c < P.nc; c++) {
            const float2 v = tp[(size_t)c * 16];
            if (xs[c] != 0.0f) acc = fmaf(v.x, v.y, acc);
        }
    } else {
        acc = lds[(size_t)t * 16 + rl];
        for (int sg = 1; sg < P.nseg; sg++) acc += lds[((size_t)sg * NT + t) * 16 + rl];
    }
    if (row < P.rows) P.out[(size_t)(tok0 + t) * P.out_stride + row] = acc;
}

GemvPlan plan_gemv(const k2t_ctx *ctx, const k2t_mat *m, int s0, int s1) {
    GemvPlan p;
    p.s_lo = s0;
    p.nstripes = s1 - s0;
    const int step = m->fmt == K2T_FMT_NF ? std::max(m->sgc, 2) : 2;  // even, scale-group aligned
    const int nunits = (m->nc + step - 1) / step;
    int nseg = 1;
    if (ctx->max_segments != 1 && p.nstripes > 0) {
        const int target = ctx->num_cus * 8;  // waves that keep every CU streaming
        nseg = (target + p.nstripes - 1) / p.nstripes;
        const int cap = ctx->max_segments > 1 ? std::min(ctx->max_segments, 16) : 16;
        nseg = std::max(1, std::min({nseg, cap, nunits}));
    }
    const int ups = (nunits + nseg - 1) / nseg;
    p.cps = ups * step;
    p.nseg = (m->nc + p.cps - 1) / p.cps;
    return p;
}

template <int FMT, int HP, bool DOTS>
static void launch_nt(int nt, dim3 grid, dim3 block, size_t lds, hipStream_t st, const GemvParams &P) {
    switch (nt) {
        case 1: hipLaunchKernelGGL((gemv_kernel<FMT, HP, 1, DOTS>), grid, block, lds, st, P); break;
        case 2: hipLaunchKernelGGL((gemv_kernel<FMT, HP, 2, false>), grid, block, lds, st, P); break;
        case 3: hipLaunchKernelGGL((gemv_kernel<FMT, HP, 3, false>), grid, block, lds, st, P); break;
        default: hipLaunchKernelGGL((gemv_kernel<FMT, HP, 4, false>), grid, block, lds, st, P); break;
    }
}

template <bool DOTS>
static void launch_fmt(const k2t_mat *m, int nt, dim3 grid, dim3 block, size_t lds, hipStream_t st,
                       const GemvParams &P) {
    if (m->fmt == K2T_FMT_NF) launch_nt<1, 0, DOTS>(nt, grid, block, lds, st, P);
    else if (m->hp == 0) launch_nt<0, 0, DOTS>(nt, grid, block, lds, st, P);
    else if (m->hp == 1) launch_nt<0, 1, DOTS>(nt, grid, block, lds, st, P);
    else launch_nt<0, 2, DOTS>(nt, grid, block, lds, st, P);
}

void launch_gemv(k2t_ctx *ctx, const k2t_mat *m, const int8_t *xq, const float *xs,
                 const int32_t *xsum, int ntok, int s0, int s1, float *out, size_t out_stride,
                 int32_t *dots) {
    const int saved = ctx->max_segments;
    if (dots) ctx->max_segments = 1;
    GemvPlan plan = plan_gemv(ctx, m, s0, s1);
    ctx->max_segments = saved;
    if (plan.nstripes <= 0 || ntok <= 0) return;
    GemvParams P{};
    P.pair = m->pair;
    P.tail = m->tail;
    P.xq = xq;
    P.xs = xs;
    P.xsum = xsum;
    P.out = out;
    P.dots = dots;
    P.out_stride = out_stride;
    P.ptot = m->fmt == K2T_FMT_NF ? (m->pairs ? m->pair_len / m->pairs : 0) : 0;
    P.rows = m->rows;
    P.K = m->cols;
    P.nc = m->nc;
    P.np = m->pairs;
    P.s_lo = plan.s_lo;
    P.nstripes = plan.nstripes;
    P.nseg = plan.nseg;
    P.cps = plan.cps;
    P.sgc = m->sgc;
    P.cb0 = m->cb[0];
    P.cb1 = m->cb[1];
    P.cb2 = m->cb[2];
    P.cb3 = m->cb[3];
    const int groups4 = ntok / 4, rem = ntok % 4;
    const dim3 block(64 * plan.nseg);
    auto lds_for = [&](int nt, GemvParams &Q) -> size_t {
        if (plan.nseg == 1) return 0;
        const size_t exact = (size_t)nt * m->nc * 16 * sizeof(float2);
        Q.lds_terms = exact <= 64 * 1024 ? 1 : 0;
        return Q.lds_terms ? exact : (size_t)plan.nseg * nt * 16 * sizeof(float);
    };
    if (groups4 > 0) {
        GemvParams Q = P;
        Q.tok_base = 0;
        const size_t lds = lds_for(4, Q);
        launch_fmt<false>(m, 4, dim3(plan.nstripes, groups4), block, lds, ctx->stream, Q);
        hip_check(hipGetLastError(), "gemv launch");
    }
    if (rem > 0) {
        GemvParams Q = P;
        Q.tok_base = groups4 * 4;
        const size_t lds = lds_for(rem, Q);
        if (dots) launch_fmt<true>(m, rem, dim3(plan.nstripes, 1), block, lds, ctx->stream, Q);
        else launch_fmt<false>(m, rem, dim3(plan.nstripes, 1), block, lds, ctx->stream, Q);
        hip_check(hipGetLastError(), "gemv launch");
    }
}

}  // namespace k2t
