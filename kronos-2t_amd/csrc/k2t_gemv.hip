// Bandwidth-bound quantized GEMV / 4-token tile for gfx950.
//
// Replaces the stripe-range leaves of the reference's LinearBackend:
//   bit-plane  nibble4_sdot_stripe_range_raw / sdot_decode_neon   (simd_lut.rs:3536-4091)
//              nibble4_sdot_batch_stripe_range / sdot_batch_tile  (simd_lut.rs:4101-4331)
//   NF4        nf_sdot_stripe_range_raw / nf_sdot_decode_neon     (simd_lut.rs:5687-6364)
//              nf_sdot_batch_stripe_range                         (simd_lut.rs:6689-7034)
//
// Work unit = one wavefront on (row block, K segment).  A row block is a stripe pair
// (32 rows, one contiguous record per 64-column chunk) or the odd tail stripe.  Per
// chunk the 64 lanes each fetch 16 contiguous bytes of nibbles with one 128-bit load
// (the 1024 nibble bytes of a pair record are read by the wave in one instruction),
// plus their hi-plane bytes / BF16 scales.  Lane bits map to the record as
//   bit0 = half (8-column half of a 16-column block), bit1 = g bit0, bit2-3 = k
//   (16-column block), bit4 = g bit1, bit5 = stripe side,
// so each quad of lanes reads 64 contiguous bytes and the per-row reduction over
// (half, k) stays inside one 16-lane DPP row.  A lane's 16 bytes are 4 rows x 8 columns;
// v_dot4_i32_i8 accumulates codes (u, or codebook values) against int8 activations.
// After two DPP steps every lane holds the exact i32 dot of 2 rows for this chunk and
// runs the fp32 epilogue f = fma(float(dot)*sx, ws, f) in chunk order, i.e. the NEON
// epilogue of simd_lut.rs:4030-4059 / 6334-6335 bit for bit.
//
// When there are too few row blocks to fill 256 CUs, K is split into segments; each
// wave writes its partial chain to scratch and the last wave of a row block (arrival
// counter) adds the partials in segment order.  That path matches the reference to
// fp32 rounding (not bit for bit); integer dots are exact in every mode.
#include <float.h>

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
    float *partial;
    uint32_t *counters;
    int32_t *dots;
    size_t out_stride;
    size_t ptot;  // NF: bytes per pair stream
    int rows, K, nc, np, total_rb;
    int s0, s1;
    int rb_lo, nrb;
    int nseg, cps;
    int rows_pad;
    int sgc;
    int ntok, tok_base;
    uint32_t cb0, cb1, cb2, cb3;
};

// Sum over the 8 lanes of a row-block line (lane bits 0, 2, 3), transposing so that a
// lane with half=h keeps rows 2h and 2h+1 of its 4-row group.
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

// FMT 0: bit-plane Nibble4 (HP hi planes); FMT 1: NF4 codebook stripes.
template <int FMT, int HP, int NT, bool DOTS>
__global__ __launch_bounds__(256) void gemv_kernel(GemvParams P) {
    const uint32_t lane = threadIdx.x & 63;
    const int unit = blockIdx.x * 4 + (int)(threadIdx.x >> 6);
    if (unit >= P.nrb * P.nseg) return;
    const int rb = P.rb_lo + unit / P.nseg;
    const int seg = unit % P.nseg;
    const int tok0 = P.tok_base + (int)blockIdx.y * NT;
    const bool is_tail = rb >= P.np;
    const uint32_t half = lane & 1u;
    const uint32_t g = ((lane >> 1) & 1u) | (((lane >> 4) & 1u) << 1);
    const uint32_t k = (lane >> 2) & 3u;
    const uint32_t lane_side = lane >> 5;
    const uint32_t side = is_tail ? 0u : lane_side;
    const uint32_t piece = k * 8u + g * 2u + half;
    const uint32_t sc_lane = (4u * g + 2u * half) * 2u;
    const int c0 = seg * P.cps;
    const int c1 = min(P.nc, c0 + P.cps);
    constexpr int MAX_ODD = (1 << (4 + HP)) - 1;
    constexpr size_t PREC = 1024 + 256 * HP + 64;
    constexpr size_t TREC = 512 + 128 * HP + 32;

    float f[NT][2];
#pragma unroll
    for (int t = 0; t < NT; t++) f[t][0] = f[t][1] = 0.0f;

    const int8_t *xbase = P.xq + (size_t)tok0 * P.K + k * 16 + half * 8;

#pragma unroll 2
    for (int c = c0; c < c1; c++) {
        const uint8_t *nib, *scp, *hib = nullptr;
        if constexpr (FMT == 0) {
            const uint8_t *base = is_tail ? P.tail + (size_t)c * TREC
                                          : P.pair + ((size_t)rb * P.nc + c) * PREC;
            nib = base + side * 512u + piece * 16u;
            if constexpr (HP > 0) {
                const uint32_t hoff = (HP == 2 ? k * 64u : (k >> 1) * 64u) + g * 16u;
                hib = base + (is_tail ? 512u : 1024u + side * 128u * HP) + hoff;
            }
            scp = base + (is_tail ? 512u + 128u * HP : 1024u + 256u * HP + side * 32u) + sc_lane;
        } else {
            const int sg = c / P.sgc, cst = sg * P.sgc, sub = c - cst;
            if (is_tail) {
                const uint8_t *gb = P.tail + (size_t)sg * 32 + (size_t)cst * 512;
                nib = gb + 32 + (size_t)sub * 512 + piece * 16u;
                scp = gb + sc_lane;
            } else {
                const uint8_t *gb = P.pair + (size_t)rb * P.ptot + (size_t)sg * 64 + (size_t)cst * 1024;
                nib = gb + 64 + (size_t)sub * 1024 + side * 512u + piece * 16u;
                scp = gb + side * 32u + sc_lane;
            }
        }
        const uint4 w4 = *reinterpret_cast<const uint4 *>(nib);
        uint4 h4 = make_uint4(0, 0, 0, 0);
        if constexpr (FMT == 0 && HP > 0) h4 = *reinterpret_cast<const uint4 *>(hib);
        const uint32_t wsw = *reinterpret_cast<const uint32_t *>(scp);

        uint32_t lo[4], hi[4];
        const uint32_t wd[4] = {w4.x, w4.y, w4.z, w4.w};
        const uint32_t hd[4] = {h4.x, h4.y, h4.z, h4.w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t d = wd[j];
            if constexpr (FMT == 0) {
                uint32_t l = d & 0x0F0F0F0Fu;
                uint32_t h = (d >> 4) & 0x0F0F0F0Fu;
                if constexpr (HP == 2) {
                    // 2-bit hi codes at shifts {4,6} (half 0) / {2,0} (half 1), simd_lut.rs:3376-3384.
                    // Rotations keep bits inside each byte once masked with 0x30.
                    const uint32_t hb = hd[j];
                    l |= __builtin_rotateright32(hb, half ? 30u : 0u) & 0x30303030u;
                    h |= __builtin_rotateright32(hb, half ? 28u : 2u) & 0x30303030u;
                } else if constexpr (HP == 1) {
                    // 1-bit hi code at bit (k even ? 4+sub : sub), sub = 2*half + nibble.
                    const uint32_t hb = hd[j];
                    const uint32_t e = ((k & 1u) ? 28u : 0u) + 2u * half;  // rotate amount for lo
                    l |= __builtin_rotateright32(hb, e) & 0x10101010u;
                    h |= __builtin_rotateright32(hb, (e + 1u) & 31u) & 0x10101010u;
                }
                lo[j] = l;
                hi[j] = h;
            } else {
                const uint32_t dh = d >> 4;
                lo[j] = lut16(d & 0x07070707u, bit7_mask(d << 4), P.cb0, P.cb1, P.cb2, P.cb3);
                hi[j] = lut16(dh & 0x07070707u, bit7_mask(d), P.cb0, P.cb1, P.cb2, P.cb3);
            }
        }
        const float ws0 = bf16_lo(wsw), ws1 = bf16_hi(wsw);

#pragma unroll
        for (int t = 0; t < NT; t++) {
            const uint2 xv = *reinterpret_cast<const uint2 *>(xbase + (size_t)t * P.K + c * 64);
            int a[4];
#pragma unroll
            for (int j = 0; j < 4; j++)
                a[j] = __builtin_amdgcn_sdot4((int)lo[j], (int)xv.x,
                                              __builtin_amdgcn_sdot4((int)hi[j], (int)xv.y, 0, false),
                                              false);
            int r0, r1;
            reduce_rows(a[0], a[1], a[2], a[3], half, r0, r1);
            const int tk = tok0 + t;
            if constexpr (FMT == 0) {
                const int off = MAX_ODD * P.xsum[(size_t)tk * P.nc + c];
                r0 = 2 * r0 - off;
                r1 = 2 * r1 - off;
            }
            if constexpr (DOTS) {
                if (k == 0 && !(is_tail && lane_side)) {
                    const int stripe = is_tail ? 2 * P.np : 2 * rb + (int)side;
                    const int row = stripe * 16 + (int)(4u * g + 2u * half);
                    if (row < P.rows) P.dots[(size_t)row * P.nc + c] = r0;
                    if (row + 1 < P.rows) P.dots[(size_t)(row + 1) * P.nc + c] = r1;
                }
            }
            const float sx = P.xs[(size_t)tk * P.nc + c];
            if (sx != 0.0f) {
                f[t][0] = fmaf((float)r0 * sx, ws0, f[t][0]);
                f[t][1] = fmaf((float)r1 * sx, ws1, f[t][1]);
            }
        }
    }

    const int stripe = is_tail ? 2 * P.np : 2 * rb + (int)side;
    const int row = stripe * 16 + (int)(4u * g + 2u * half);
    const bool writer = (k == 0) && !(is_tail && lane_side) && stripe >= P.s0 && stripe < P.s1;
    if (P.nseg == 1) {
        if (writer) {
#pragma unroll
            for (int t = 0; t < NT; t++) {
                float *o = P.out + (size_t)(tok0 + t) * P.out_stride;
                if (row < P.rows) o[row] = f[t][0];
                if (row + 1 < P.rows) o[row + 1] = f[t][1];
            }
        }
        return;
    }
    // Split-K: publish this segment's partial rows, the last arriving wave combines.
    if (writer) {
#pragma unroll
        for (int t = 0; t < NT; t++) {
            float *pp = P.partial + ((size_t)seg * P.ntok + tok0 + t) * P.rows_pad;
            pp[row] = f[t][0];
            pp[row + 1] = f[t][1];
        }
    }
    __threadfence();
    uint32_t old = 0;
    uint32_t *ctr = P.counters + (size_t)blockIdx.y * P.total_rb + rb;
    if (lane == 0) old = atomicAdd(ctr, 1u);
    old = __shfl(old, 0, kWave);
    if (old != (uint32_t)(P.nseg - 1)) return;
    __threadfence();
    const int nrows_blk = is_tail ? 16 : 32;
    const int first_stripe = is_tail ? 2 * P.np : 2 * rb;
    if ((int)lane < nrows_blk) {
        const int r = first_stripe * 16 + (int)lane;
        const int st = first_stripe + (int)lane / 16;
        if (r < P.rows && st >= P.s0 && st < P.s1) {
#pragma unroll
            for (int t = 0; t < NT; t++) {
                float acc = P.partial[((size_t)0 * P.ntok + tok0 + t) * P.rows_pad + r];
                for (int s = 1; s < P.nseg; s++)
                    acc += P.partial[((size_t)s * P.ntok + tok0 + t) * P.rows_pad + r];
                P.out[(size_t)(tok0 + t) * P.out_stride + r] = acc;
            }
        }
    }
    if (lane == 0) *ctr = 0u;
}

GemvPlan plan_gemv(const k2t_ctx *ctx, const k2t_mat *m, int s0, int s1) {
    GemvPlan p;
    p.rb_lo = s0 / 2;
    p.rb_hi = std::min(m->pairs + m->has_tail, (s1 + 1) / 2);
    const int nrb = std::max(p.rb_hi - p.rb_lo, 1);
    const int step = m->fmt == K2T_FMT_NF ? m->sgc : 1;
    const int ngroups = (m->nc + step - 1) / step;
    int nseg = 1;
    if (ctx->max_segments != 1) {
        const int target = ctx->num_cus * 8;  // waves to keep every CU streaming
        nseg = (target + nrb - 1) / nrb;
        if (ctx->max_segments > 1) nseg = std::min(nseg, ctx->max_segments);
        nseg = std::max(1, std::min(nseg, ngroups));
    }
    const int gps = (ngroups + nseg - 1) / nseg;  // scale groups per segment
    p.cps = gps * step;
    p.nseg = (m->nc + p.cps - 1) / p.cps;
    return p;
}

template <int FMT, int HP, bool DOTS>
static void launch_nt(int nt, dim3 grid, hipStream_t s, const GemvParams &P) {
    switch (nt) {
        case 1: hipLaunchKernelGGL((gemv_kernel<FMT, HP, 1, DOTS>), grid, dim3(256), 0, s, P); break;
        case 2: hipLaunchKernelGGL((gemv_kernel<FMT, HP, 2, false>), grid, dim3(256), 0, s, P); break;
        case 3: hipLaunchKernelGGL((gemv_kernel<FMT, HP, 3, false>), grid, dim3(256), 0, s, P); break;
        default: hipLaunchKernelGGL((gemv_kernel<FMT, HP, 4, false>), grid, dim3(256), 0, s, P); break;
    }
}

template <bool DOTS>
static void launch_fmt(const k2t_mat *m, int nt, dim3 grid, hipStream_t s, const GemvParams &P) {
    if (m->fmt == K2T_FMT_NF) {
        launch_nt<1, 0, DOTS>(nt, grid, s, P);
    } else if (m->hp == 0) {
        launch_nt<0, 0, DOTS>(nt, grid, s, P);
    } else if (m->hp == 1) {
        launch_nt<0, 1, DOTS>(nt, grid, s, P);
    } else {
        launch_nt<0, 2, DOTS>(nt, grid, s, P);
    }
}

void launch_gemv(k2t_ctx *ctx, const k2t_mat *m, const int8_t *xq, const float *xs,
                 const int32_t *xsum, int ntok, int s0, int s1, float *out, size_t out_stride,
                 int32_t *dots) {
    int saved = ctx->max_segments;
    if (dots) ctx->max_segments = 1;
    GemvPlan plan = plan_gemv(ctx, m, s0, s1);
    ctx->max_segments = saved;
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
    P.total_rb = m->pairs + m->has_tail;
    P.s0 = s0;
    P.s1 = s1;
    P.rb_lo = plan.rb_lo;
    P.nrb = plan.rb_hi - plan.rb_lo;
    P.nseg = plan.nseg;
    P.cps = plan.cps;
    P.rows_pad = m->stripes * 16;
    P.sgc = m->sgc;
    P.ntok = ntok;
    P.cb0 = m->cb[0];
    P.cb1 = m->cb[1];
    P.cb2 = m->cb[2];
    P.cb3 = m->cb[3];
    if (P.nrb <= 0 || ntok <= 0) return;
    const int groups4 = ntok / 4, rem = ntok % 4;
    if (plan.nseg > 1) {
        ensure_scratch(ctx, (size_t)plan.nseg * ntok * P.rows_pad,
                       (size_t)std::max(groups4, 1) * P.total_rb);
        P.partial = ctx->partial;
        P.counters = ctx->counters;
    }
    const int blocks = (P.nrb * P.nseg + 3) / 4;
    if (groups4 > 0) {
        P.tok_base = 0;
        launch_fmt<false>(m, 4, dim3(blocks, groups4), ctx->stream, P);
        hip_check(hipGetLastError(), "gemv launch");
    }
    if (rem > 0) {
        P.tok_base = groups4 * 4;
        if (dots) launch_fmt<true>(m, rem, dim3(blocks, 1), ctx->stream, P);
        else launch_fmt<false>(m, rem, dim3(blocks, 1), ctx->stream, P);
        hip_check(hipGetLastError(), "gemv launch");
    }
}

}  // namespace k2t
