// Bandwidth-bound quantized GEMV / 4-token tile for gfx950.
//
// Replaces the stripe-range leaves of the reference's LinearBackend:
//   bit-plane  nibble4_sdot_stripe_range_raw / sdot_decode_neon   (simd_lut.rs:3536-4091)
//              nibble4_sdot_batch_stripe_range / sdot_batch_tile  (simd_lut.rs:4101-4331)
//   NF4        nf_sdot_stripe_range_raw / nf_sdot_decode_neon     (simd_lut.rs:5687-6364)
//              nf_sdot_batch_stripe_range                         (simd_lut.rs:6689-7034)
//
// Work unit = one workgroup per stripe pair (32 rows; the odd last stripe alone); its
// waves split K into segments (as many as needed to put ~8 streaming waves on every CU).
// Per chunk a wave reads the pair's contiguous record -- 1024 nibble bytes with one
// 128-bit load per lane, plus hi-plane bytes / BF16 scales -- decodes codes (u, or codebook values through a v_perm byte table) and
// accumulates them against int8 activations with v_dot4_i32_i8.  Two DPP steps leave
// every lane with the exact i32 dot of 2 rows for its chunk.
//
// fp32 epilogue: the reference computes f = fma(float(dot)*sx, ws, f) per row in chunk
// order (simd_lut.rs:4030-4059 / 6334-6335).  With one segment the chain runs in
// registers; with several, every (row, chunk) term is staged in LDS and one lane per
// row replays the chain after a barrier.  Either way the result is bit-identical to
// the reference.  No global scratch, atomics or device-scope fences are used.
#include <float.h>

#include <stdlib.h>

#include <algorithm>

#include "k2t_device.h"
#include "../../include/k2t_hip.h"
#include "k2t_internal.h"
#include "k2t_route.h"

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
    int s0, s1;      // stripes written: [s0, s1)
    int rb_lo;       // first row block (pair index; np = the tail stripe)
    int nseg, cps;   // K segments per row block (= waves per workgroup), chunks per segment
    int sgc;
    int tok_base;
    int lds_terms;  // per-chunk terms staged in LDS (always 1 in this build)
    int stripe_mode;  // 1: a workgroup owns one stripe (16 rows), 0: a stripe pair (32 rows)
    int exact;        // 1: replay the reference's fmaf chain from LDS-staged terms
    int accum;        // 1: out = out + result (residual add, real_llm.rs:7185-7188)
    uint32_t cb0, cb1, cb2, cb3;
    // Fused activation builder (XS != 0): fp32 source row, RMSNorm weights, eps, the
    // Hadamard sign masks and the byte offset of the activation region in LDS.
    const float *xsrc;
    const float *xnorm;
    const uint64_t *signs;
    float eps;
    int xoff;
    // Grouped mode (sparse-MoE experts): workgroup slot z = blockIdx.z streams the matrix of
    // expert route[z] inside the .k2tm bank: record = bank + route[z] * bank_stride, matrix
    // pairs at record + mat_off, 16-byte codebook at record + cb_off.  Output and fp32
    // activation source advance by slot_out / slot_src floats per slot.  gu_split = 1
    // writes rows [0, rows/2) (gate) and [rows/2, rows) (up) in [gate64, up64] blocks.
    const int *route;
    const uint8_t *bank;
    size_t bank_stride;
    uint32_t mat_off, cb_off;
    size_t slot_out, slot_src;
    int gu_split;
    // Grouped mode with a ready int8 activation (XS 0): slot_act = 1 reads activation row z
    // (xq + z * K, xs / xsum + z * nc) for slot z, 0 the same row for every slot.
    int slot_act;
    // Routing in the same launch (XS 1 only, rt_w != NULL): workgroups of plane z = 0 run
    // the router (route_logit_half on every wave, units x * waves + wave stepping by
    // gridDim.x * waves, into rt_words [2 rt_E + 2]; then route_collect_parts on wave 0 of
    // workgroup 0, which writes route[] / rt_wts[]
    // and publishes sorted id r as the word rt_pub[r] = {epoch, id}); plane z >= 1 is slot
    // z - 1, which builds its activation, then waits for its word.  epoch = *rt_ctr + 1;
    // the counter is advanced by a later launch, when every workgroup of this one has read
    // it.
    const float *rt_w, *rt_b;
    unsigned long long *rt_words, *rt_pub;
    const uint32_t *rt_ctr;
    int *rt_err;
    float *rt_wts;
    int rt_E, rt_k, rt_norm, rt_scoring;
    uint32_t rt_spin;
};

// Output index of row r: the [gate64(ic), up64(ic)] interleave of a split gate/up matrix.
__device__ __forceinline__ int gu_out_row(int r, int rows, int split) {
    if (!split) return r;
    const int inter = rows >> 1;
    const int u = r >= inter ? 1 : 0, rr = r - u * inter;
    return (rr >> 6) * 128 + u * 64 + (rr & 63);
}

// Builds the int8 activation chunks [c0, c1) of one token in LDS (xl[c*64 + e],
// xsl[c], xsuml[c]) from an fp32 source:
//   XS 1: v = (x*inv_rms)*w, inv_rms = 1/sqrt(mean(x^2)+eps) computed once per workgroup
//         (populate_rmsnorm_fwht, simd_lut.rs:2970-2997; inv_rms as real_llm.rs:6929)
//   XS 2: v = silu(gate)*up of the interleaved gate_up block c  (real_llm.rs:9801-9805,
//         populate_chunk_fwht_raw with chunk index c, 7207-7296)
// then the signed FWHT-64 of chunk c and int8 quantization (simd_lut.rs:3097-3128).
// Eight lanes per chunk, eight consecutive elements per lane: butterflies h = 1, 2, 4
// run in registers and h = 8, 16, 32 across lanes (^1, ^2, ^4).  Each butterfly adds or
// subtracts the same operands as hadamard.rs:83-97, so the codes, scales and sums equal
// those of the one-element-per-lane kernels (rmsnorm_act / swiglu_act).
// Source registers of one 8-element slice: XS 1 = x (a) and w (b); XS 2 = gate (a), up (b).
struct XSlice {
    float4 a0, a1, b0, b1;
};

template <int XS>
__device__ __forceinline__ void load_slice(const GemvParams &P, const float *src, int c, uint32_t s, XSlice &r) {
    if constexpr (XS == 1) {
        const float4 *x4 = reinterpret_cast<const float4 *>(src + c * 64 + s * 8);
        const float4 *w4 = reinterpret_cast<const float4 *>(P.xnorm + c * 64 + s * 8);
        r.a0 = x4[0];
        r.a1 = x4[1];
        r.b0 = w4[0];
        r.b1 = w4[1];
    } else {
        const float4 *g4 = reinterpret_cast<const float4 *>(src + (size_t)c * 128 + s * 8);
        r.a0 = g4[0];
        r.a1 = g4[1];
        r.b0 = g4[16];
        r.b1 = g4[17];
    }
}

// Turns one loaded slice into its int8 codes (as described above) and stores them in LDS.
template <int XS>
__device__ __forceinline__ void finish_slice(const GemvParams &P, const XSlice &r, int c, bool act, uint32_t s,
                                             float inv_rms, int8_t *xl, float *xsl, int32_t *xsuml) {
    float v[8];
    const float a[8] = {r.a0.x, r.a0.y, r.a0.z, r.a0.w, r.a1.x, r.a1.y, r.a1.z, r.a1.w};
    const float b[8] = {r.b0.x, r.b0.y, r.b0.z, r.b0.w, r.b1.x, r.b1.y, r.b1.z, r.b1.w};
#pragma unroll
    for (int j = 0; j < 8; j++) {
        if constexpr (XS == 1) v[j] = (a[j] * inv_rms) * b[j];
        else v[j] = (a[j] / (1.0f + expf(-a[j]))) * b[j];
    }
    rotate_quant_slice8(v, P.signs[c], s, c, act, xl, xsl, xsuml);
}

// Builds the int8 activation chunks [c0, c1) of one token in LDS in two steps, so that
// the source loads are issued before the first weight loads (loads complete in order):
//   begin(): loads the first 8 chunk slices and, for XS 1, the first kSqPre float4 of
//            every lane's share of the row for sum(x^2);
//   finish(): inv_rms, then codes of every chunk (later slices load after the weights).
constexpr int kSqPre = 8;
template <int XS>
struct XBuilder {
    const GemvParams &P;
    const float *src;
    int c0, c1;
    uint32_t lane, slot, s;
    XSlice first;
    float4 sq[XS == 1 ? kSqPre : 1];

    __device__ XBuilder(const GemvParams &P_, const float *xsrc, int tok, int c0_, int c1_, uint32_t lane_)
        : P(P_), src(xsrc + (size_t)tok * (XS == 2 ? 2 * P_.K : P_.K)), c0(c0_), c1(c1_), lane(lane_),
          slot(lane_ >> 3), s(lane_ & 7u) {}

    __device__ void begin() {
        const int u = (int)slot;
        load_slice<XS>(P, src, c0 + (u < c1 - c0 ? u : 0), s, first);
        if constexpr (XS == 1) {
            const float4 *x4 = reinterpret_cast<const float4 *>(src);
            const int n4 = P.K / 4;
            // (unconditional loads from a clamped index, masked in finish(): under a branch
            // whose other side zeroed the registers the compiler waited for the first load
            // before issuing the rest)
#pragma unroll
            for (int j = 0; j < kSqPre; j++) sq[j] = x4[min((int)lane + 64 * j, n4 - 1)];
        }
    }

    __device__ void finish(int8_t *xl, float *xsl, int32_t *xsuml) {
        float inv_rms = 1.0f;
        if constexpr (XS == 1) {
            // Same fmaf order as row_sumsq_wave: lane l adds float4 l, l+64, ... ascending.
            const float4 *x4 = reinterpret_cast<const float4 *>(src);
            const int n4 = P.K / 4;
            float ss = 0.0f;
#pragma unroll
            for (int j = 0; j < kSqPre; j++) {
                if ((int)lane + 64 * j < n4) {
                    ss = fmaf(sq[j].x, sq[j].x, ss);
                    ss = fmaf(sq[j].y, sq[j].y, ss);
                    ss = fmaf(sq[j].z, sq[j].z, ss);
                    ss = fmaf(sq[j].w, sq[j].w, ss);
                }
            }
            for (int i = (int)lane + 64 * kSqPre; i < n4; i += 64) {
                const float4 v = x4[i];
                ss = fmaf(v.x, v.x, ss);
                ss = fmaf(v.y, v.y, ss);
                ss = fmaf(v.z, v.z, ss);
                ss = fmaf(v.w, v.w, ss);
            }
            ss = wave_sum_f(ss);
            inv_rms = 1.0f / sqrtf(ss / (float)P.K + P.eps);
        }
        const int n = c1 - c0;
        finish_slice<XS>(P, first, c0 + ((int)slot < n ? (int)slot : 0), (int)slot < n, s, inv_rms, xl, xsl, xsuml);
        for (int base = 8; base < n; base += 8) {
            const int u = base + (int)slot;
            const bool act = u < n;
            const int c = c0 + (act ? u : 0);
            XSlice r;
            load_slice<XS>(P, src, c, s, r);
            finish_slice<XS>(P, r, c, act, s, inv_rms, xl, xsl, xsuml);
        }
    }
};

// XS 3: a ready int8 activation in global memory (one token), staged through LDS.  Each
// wave copies the codes, scales and sums of its own chunks [c0, c1) once (c1 - c0 <= 32),
// so the chunk loop issues only weight loads.
template <int FMT>
struct XStage {
    const GemvParams &P;
    int tok, c0, c1;
    uint32_t lane;
    uint4 q[2];
    float sx;
    int32_t sm;

    __device__ XStage(const GemvParams &P_, int tok_, int c0_, int c1_, uint32_t lane_)
        : P(P_), tok(tok_), c0(c0_), c1(c1_), lane(lane_) {}

    __device__ void begin() {
        const int n = c1 - c0, n_u4 = n * 4;
        const uint4 *src = reinterpret_cast<const uint4 *>(P.xq + (size_t)tok * P.K + (size_t)c0 * 64);
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int i = (int)lane + 64 * j;
            q[j] = i < n_u4 ? src[i] : make_uint4(0, 0, 0, 0);
        }
        sx = (int)lane < n ? P.xs[(size_t)tok * P.nc + c0 + lane] : 0.0f;
        sm = 0;
        if constexpr (FMT == 0) sm = (int)lane < n ? P.xsum[(size_t)tok * P.nc + c0 + lane] : 0;
    }

    __device__ void finish(int8_t *xl, float *xsl, int32_t *xsuml) {
        const int n = c1 - c0, n_u4 = n * 4;
        uint4 *dst = reinterpret_cast<uint4 *>(xl + (size_t)c0 * 64);
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int i = (int)lane + 64 * j;
            if (i < n_u4) dst[i] = q[j];
        }
        if ((int)lane < n) {
            xsl[c0 + lane] = sx;
            xsuml[c0 + lane] = sm;
        }
    }
};

// Registers of one fetched chunk for one lane: its 64 nibble bytes (rows 4g..4g+3,
// the lane's 8-column half of each of the four 16-column blocks), hi-plane bytes, the
// BF16 scales of its two output rows and the matching activation bytes.
template <int HP, int NT>
struct Frag {
    uint4 w[4];
    uint4 h[HP == 0 ? 1 : (HP == 1 ? 2 : 4)];
    uint32_t ws;
    uint2 x[NT][4];
    float sx[NT];
    int sum[NT];
};

// One workgroup = one row block (a stripe pair, or the odd tail stripe).  Lane bits:
// 0 = half (8-column half of a 16-column block), 1-2 = g (4-row group), 3 = stripe of the
// pair, 4-5 = q.  Each 16-lane group q of each wave owns one K sub-segment, so a row
// block's K range is split into 4 * nseg sub-segments.  Per chunk a lane loads the four
// 16-byte pieces of its (side, g, half) -- one per 16-column block k -- so a load
// instruction reads two 128-byte runs per group, and the lane accumulates all 32 of its
// columns for 4 rows with v_dot4_i32_i8.  One DPP step over `half` completes the exact
// i32 dot of each (row, chunk).  The fp32 terms float(dot)*sx and ws are staged in LDS
// and one thread per row replays the reference's fmaf chain in chunk order.
// FMT 0: bit-plane Nibble4 with HP hi planes; FMT 1: NF4 codebook stripes; FMT 2: NF3
// codebook stripes (384-byte stripe-chunks of 48-byte triplet blocks; lane bit 0 then
// picks the 32-column half of the chunk instead of an 8-column half of each block).

#ifdef K2T_GEMV_TRACE
// Measurement builds only: wall-clock stamps of the staged batch-1 GEMV (XS 5), 8 per
// (workgroup < 512, wave < 16).
__device__ unsigned long long g_gemv_trace[512 * 16 * 8];
#define GV_TR(k)                                                                                              \
    do {                                                                                                      \
        if (XS == 5 && lane == 0 && blockIdx.x < 512 && wave < 16)                                            \
            g_gemv_trace[((size_t)blockIdx.x * 16 + wave) * 8 + (k)] = wall_clock64();                        \
    } while (0)
extern "C" int k2t_gemv_trace_read(unsigned long long *dst) {
    return hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_gemv_trace), sizeof(g_gemv_trace)) == hipSuccess ? 0 : -1;
}
#else
#define GV_TR(k) \
    do {         \
    } while (0)
#endif

// The two-hi-plane kernel with the fused RMSNorm builder needs more registers than a
// 1024-thread workgroup leaves a lane; its launches are held to kB6NormThreads threads.
constexpr int kB6NormThreads = 512;

template <int FMT, int HP, int NT, bool DOTS, int XS>
__global__ __launch_bounds__(FMT == 0 && HP == 2 && XS == K2T_XS_RMSNORM ? kB6NormThreads : 1024) void gemv_kernel(
    GemvParams P) {
    constexpr int NH = HP == 0 ? 1 : (HP == 1 ? 2 : 4);
    constexpr bool kNF3 = FMT >= 2, kLane = FMT == 3;  // NF3; FMT 3: stripe-chunks in lane order
    extern __shared__ float lds[];
    const uint32_t lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    // Routing in this launch: the epoch of this call (a vector load through a lane offset
    // the compiler cannot see is zero, so no scalar wait comes before the first loads).
    constexpr bool kCanRoute = XS == 1 && NT == 1 && !DOTS;
    const bool fused_route = kCanRoute && P.rt_w != nullptr;
    int slot = (int)blockIdx.z;
    GV_TR(0);
    uint32_t rt_epoch = 0;
    if constexpr (kCanRoute) {
        if (fused_route) {
            int zoff;
            asm volatile("v_mov_b32 %0, 0" : "=v"(zoff));
            rt_epoch = ld_global(P.rt_ctr + zoff) + 1u;
            if (blockIdx.z == 0) {
                const int nw = (int)(blockDim.x >> 6);
                for (int u = (int)blockIdx.x * nw + wave; u < 2 * P.rt_E; u += (int)gridDim.x * nw)
                    route_logit_half(P.xsrc, P.xnorm, P.K, P.rt_w, u, lane, rt_epoch, P.rt_E, P.rt_words);
                if (blockIdx.x == 0 && wave == 0)
                    route_collect_parts(P.rt_words, P.rt_E, P.K, P.eps, P.rt_b, rt_epoch, P.rt_spin, P.rt_err,
                                        lane, P.rt_k, P.rt_norm, P.rt_scoring, const_cast<int *>(P.route),
                                        P.rt_wts, P.rt_pub);
                return;
            }
            slot -= 1;
        }
    }
    const int tok0 = P.tok_base + (int)blockIdx.y * NT;
    const int xtok0 = tok0 + (P.route && P.slot_act ? slot : 0);  // activation row of a ready activation
    const uint32_t half = lane & 1u;
    const uint32_t g = (lane >> 1) & 3u;
    // Pair mode: lane bit 3 = stripe of the pair, bits 4-5 = sub-segment (4 per wave).
    // Stripe mode: bits 3-5 = sub-segment (8 per wave); the workgroup owns one stripe.
    const bool smode = P.stripe_mode != 0;
    // Stripe mode: both stripes of a pair run on one XCD (workgroups are dispatched
    // round-robin over the 8 XCDs by id), so the L2 lines shared by the two halves of a
    // record are fetched from HBM once.  Ids 16a + 8s + j (j < 8) take stripe 2(8a + j) + s.
    int rbi = (int)blockIdx.x;
    if (P.stripe_mode && (gridDim.x & 15u) == 0) {
        const int a = rbi >> 4, s8 = (rbi >> 3) & 1, j = rbi & 7;
        rbi = 2 * (8 * a + j) + s8;
    }
    const int rb = P.rb_lo + rbi;  // pair index, or stripe index in stripe mode
    const bool is_tail = smode ? rb >= 2 * P.np : rb >= P.np;
    const uint32_t lane_side = smode ? 0u : (lane >> 3) & 1u;
    const uint32_t side = smode ? (uint32_t)(rb & 1) : (is_tail ? 0u : lane_side);
    const int pidx = smode ? (rb >> 1) : rb;  // pair whose records hold these rows
    // The wave owns chunks [wave*cps, (wave+1)*cps); its lane groups take them round-robin
    // (chunk granules of sgc for NF), so one load instruction covers consecutive records.
    const int G = smode ? 8 : 4;
    const int q = smode ? (int)(lane >> 3) : (int)(lane >> 4);
    const int cw0 = wave * P.cps;
    const int cw1 = min(P.nc, cw0 + P.cps);
    constexpr int MAX_ODD = (1 << (4 + HP)) - 1;
    constexpr uint32_t PREC = 1024 + 256 * HP + 64;
    constexpr uint32_t TREC = 512 + 128 * HP + 32;
    const int RB = smode ? 16 : 32;  // rows per workgroup
    const uint32_t rloc = (smode ? 0u : side * 16u) + 4u * g + 2u * half;  // first of this lane's 2 rows
    const int stripe = smode ? rb : (is_tail ? 2 * P.np : 2 * rb + (int)side);
    const int row0 = stripe * 16 + (int)(4u * g + 2u * half);
    const bool live = !(is_tail && lane_side);

    // Byte offsets inside one record (per lane), and the record stride / base.
    uint32_t nib_off, hi_off = 0, sc_off;
    if constexpr (FMT == 0) {
        nib_off = (is_tail ? 0u : side * 512u) + g * 32u + half * 16u;
        hi_off = (is_tail ? 512u : 1024u + side * 128u * HP) + g * 16u;
        sc_off = (is_tail ? 512u + 128u * HP : 1024u + 256u * HP + side * 32u);
    } else if constexpr (FMT == 1) {
        nib_off = (is_tail ? 32u : 64u + side * 512u) + g * 32u + half * 16u;
        sc_off = is_tail ? 0u : side * 32u;
    } else {
        // FMT 2: the lane's 48-byte triplet block, read as three consecutive 16-byte
        // pieces (eight lanes of a group touch three 128-byte lines per load); FMT 3: the
        // same pieces stored in lane order (piece k of lane 2g + half at k*128 + 16*(2g +
        // half), nf3_lane_order_kernel), so each load reads one 128-byte run per group.
        nib_off = (is_tail ? 32u : 64u + side * 384u) + (kLane ? (2u * g + half) * 16u : half * 192u + g * 48u);
        sc_off = is_tail ? 0u : side * 32u;
    }
    sc_off += (4u * g + 2u * half) * 2u;
    // Matrix, codebook, output and activation source of this workgroup (grouped mode: of
    // the expert routed to slot blockIdx.z; expert matrices have no tail stripe).
    const uint8_t *pair_p = P.pair;
    uint32_t cb0 = P.cb0, cb1 = P.cb1, cb2 = P.cb2, cb3 = P.cb3;
    float *out_p = P.out;
    const float *xsrc_p = P.xsrc;
    auto bind_expert = [&](int id) {
        const uint8_t *rec = P.bank + (size_t)id * P.bank_stride;
        pair_p = rec + P.mat_off;
        // The codebook as a vector load through a lane offset the compiler cannot see is
        // zero: a uniform address made it a scalar load whose wait (scalar loads are not
        // tracked in issue order) came before the first weight fetch, a second round trip
        // after the route's.  The vector load completes in issue order ahead of the
        // fragments, so its use waits for nothing they need.
        int zoff;
        asm volatile("v_mov_b32 %0, 0" : "=v"(zoff));
        const uint4 cbw = ld_global(reinterpret_cast<const uint4 *>(rec + P.cb_off + zoff));
        cb0 = cbw.x;
        cb1 = cbw.y;
        cb2 = cbw.z;
        cb3 = cbw.w;
    };
    if (P.route) {
        out_p += (size_t)slot * P.slot_out;
        xsrc_p += (size_t)slot * P.slot_src;
        if (!fused_route) bind_expert(P.route[slot]);
    }
    // NF4: the codebook as the two XOR tables of nf4_xlut (two v_perm and one XOR per
    // four codes instead of two v_perm, a select and a bit-3 mask)
    uint32_t xt0 = 0, xt1 = 0, xu0 = 0, xu1 = 0;
    if constexpr (FMT == 1) nf4_xor_tables(cb0, cb1, cb2, cb3, xt0, xt1, xu0, xu1);
    const uint8_t *mbase = is_tail ? P.tail : pair_p + (size_t)pidx * (FMT == 0 ? (size_t)P.nc * PREC : P.ptot);
    // Routing in this launch: the slot's expert id, once wave-uniform word rt_pub[slot]
    // carries this epoch (bounded wait; on timeout *rt_err is raised and expert 0 is read).
    auto await_expert = [&]() {
        unsigned long long w = word_load(P.rt_pub + slot);
        for (uint32_t spins = 0; (uint32_t)(w >> 32) != rt_epoch; spins++) {
            if (spins > P.rt_spin) {
                __hip_atomic_store(P.rt_err, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                w = (unsigned long long)rt_epoch << 32;
                break;
            }
            __builtin_amdgcn_s_sleep(2);
            w = word_load(P.rt_pub + slot);
        }
        bind_expert(min((int)(uint32_t)w, P.rt_E - 1));
        if constexpr (FMT == 1) nf4_xor_tables(cb0, cb1, cb2, cb3, xt0, xt1, xu0, xu1);
        mbase = pair_p + (size_t)pidx * (FMT == 0 ? (size_t)P.nc * PREC : P.ptot);
    };

    auto fetch = [&](Frag<HP, NT> &fr, int c) {
        const uint8_t *rec, *scp;
        if constexpr (FMT == 0) {
            rec = mbase + (size_t)c * (is_tail ? TREC : PREC);
            scp = rec;
        } else {
            constexpr size_t CB = FMT == 1 ? 512 : 384;  // bytes per stripe-chunk
            const int sg = c / P.sgc, cst = sg * P.sgc, sb = c - cst;
            const uint8_t *gb = mbase + (is_tail ? (size_t)sg * 32 + (size_t)cst * CB
                                                 : (size_t)sg * 64 + (size_t)cst * 2 * CB);
            rec = gb + (size_t)sb * (is_tail ? CB : 2 * CB);
            scp = gb;
        }
        if constexpr (kNF3) {
#pragma unroll
            for (int kk = 0; kk < 3; kk++) fr.w[kk] = load_stream16(rec + nib_off + kk * (kLane ? 128 : 16));
        } else {
#pragma unroll
            for (int kk = 0; kk < 4; kk++) fr.w[kk] = load_stream16(rec + nib_off + kk * 128);
        }

        if constexpr (FMT == 0 && HP == 2) {
#pragma unroll
            for (int kk = 0; kk < 4; kk++) fr.h[kk] = load_stream16(rec + hi_off + kk * 64);
        } else if constexpr (FMT == 0 && HP == 1) {
            fr.h[0] = load_stream16(rec + hi_off);
            fr.h[1] = load_stream16(rec + hi_off + 64);
        }
        fr.ws = *reinterpret_cast<const uint32_t *>(scp + sc_off);
        if constexpr (XS != 0) return;
#pragma unroll
        for (int t = 0; t < NT; t++) {
#pragma unroll
            for (int kk = 0; kk < 4; kk++)
                fr.x[t][kk] = *reinterpret_cast<const uint2 *>(P.xq + (size_t)(xtok0 + t) * P.K + c * 64 +
                                                               (kNF3 ? half * 32 + kk * 8 : kk * 16 + half * 8));
            fr.sx[t] = P.xs[(size_t)(xtok0 + t) * P.nc + c];
            if constexpr (FMT == 0) fr.sum[t] = P.xsum[(size_t)(xtok0 + t) * P.nc + c];
        }
    };

    float2 *terms = reinterpret_cast<float2 *>(lds);  // [NT][nc][RB] (a = float(dot)*sx, ws)
    // Fused activation (XS != 0, one token): int8 codes, scales and sums per chunk.
    int8_t *xl = reinterpret_cast<int8_t *>(lds) + P.xoff;
    float *xsl = reinterpret_cast<float *>(xl + P.K);
    int32_t *xsuml = reinterpret_cast<int32_t *>(xsl + P.nc);

    float f[NT][2];  // fast epilogue: this lane group's partial chains
#pragma unroll
    for (int t = 0; t < NT; t++) f[t][0] = f[t][1] = 0.0f;

    auto process = [&](Frag<HP, NT> &fr, int c) {
        if constexpr (XS != 0) {  // activation built in LDS by this wave
#pragma unroll
            for (int kk = 0; kk < 4; kk++)
                fr.x[0][kk] = *reinterpret_cast<const uint2 *>(xl + c * 64 +
                                                              (kNF3 ? half * 32 + kk * 8 : kk * 16 + half * 8));
            fr.sx[0] = xsl[c];
            if constexpr (FMT == 0) fr.sum[0] = xsuml[c];
        }
        int acc[NT][4];
#pragma unroll
        for (int t = 0; t < NT; t++)
#pragma unroll
            for (int j = 0; j < 4; j++) acc[t][j] = 0;
        if constexpr (kNF3) {
            // NF3 triplets (simd_lut.rs:4932-4960): bytes (v0, v1, v2) of row j, column
            // group t hold the 3-bit codes of columns k0*16 + 4q + t (q = 0..3, codes 0-3)
            // and k1*16 + 4q + t (codes 4-7), k0 = 2*half, k1 = k0 + 1.  Four columns per
            // dword; one v_perm reads the 8-entry codebook.
            const uint32_t p0[4] = {fr.w[0].x, fr.w[0].y, fr.w[0].z, fr.w[0].w};
            const uint32_t p1[4] = {fr.w[1].x, fr.w[1].y, fr.w[1].z, fr.w[1].w};
            const uint32_t p2[4] = {fr.w[2].x, fr.w[2].y, fr.w[2].z, fr.w[2].w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t v0 = p0[j], v1 = p1[j], v2 = p2[j];
                const uint32_t id[8] = {v0 & 0x07070707u,
                                        (v0 >> 3) & 0x07070707u,
                                        ((v0 >> 6) & 0x03030303u) | ((v2 >> 4) & 0x04040404u),
                                        v1 & 0x07070707u,
                                        (v1 >> 3) & 0x07070707u,
                                        ((v1 >> 6) & 0x03030303u) | ((v2 >> 5) & 0x04040404u),
                                        v2 & 0x07070707u,
                                        (v2 >> 3) & 0x07070707u};
#pragma unroll
                for (int t = 0; t < NT; t++) {
                    const uint32_t xw[8] = {fr.x[t][0].x, fr.x[t][0].y, fr.x[t][1].x, fr.x[t][1].y,
                                            fr.x[t][2].x, fr.x[t][2].y, fr.x[t][3].x, fr.x[t][3].y};
                    int a = acc[t][j];
#pragma unroll
                    for (int u = 0; u < 8; u++)
                        a = __builtin_amdgcn_sdot4((int)__builtin_amdgcn_perm(cb1, cb0, id[u]), (int)xw[u], a,
                                                   false);
                    acc[t][j] = a;
                }
            }
        }
#pragma unroll
        for (int kk = 0; kk < (kNF3 ? 0 : 4); kk++) {
            const uint32_t wd[4] = {fr.w[kk].x, fr.w[kk].y, fr.w[kk].z, fr.w[kk].w};
            uint4 hv = make_uint4(0, 0, 0, 0);
            if constexpr (HP == 2) hv = fr.h[kk];
            if constexpr (HP == 1) hv = fr.h[kk >> 1];
            const uint32_t hd[4] = {hv.x, hv.y, hv.z, hv.w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t d = wd[j];
                uint32_t lo, hi;
                if constexpr (FMT == 0) {
                    lo = d & 0x0F0F0F0Fu;
                    hi = (d >> 4) & 0x0F0F0F0Fu;
                    if constexpr (HP == 2) {
                        // 2-bit hi codes at shifts {4,6} (half 0) / {2,0} (half 1), simd_lut.rs:3376-3384;
                        // the rotations keep bits inside each byte once masked with 0x30.
                        lo |= __builtin_rotateright32(hd[j], half ? 30u : 0u) & 0x30303030u;
                        hi |= __builtin_rotateright32(hd[j], half ? 28u : 2u) & 0x30303030u;
                    } else if constexpr (HP == 1) {
                        // 1-bit hi code at bit (k even ? 4+sub : sub), sub = 2*half + nibble (3366-3375).
                        const uint32_t e = ((kk & 1) ? 28u : 0u) + 2u * half;
                        lo |= __builtin_rotateright32(hd[j], e) & 0x10101010u;
                        hi |= __builtin_rotateright32(hd[j], (e + 1u) & 31u) & 0x10101010u;
                    }
                } else {
                    lo = nf4_xlut(d & 0x0F0F0F0Fu, xt0, xt1, xu0, xu1);
                    hi = nf4_xlut((d >> 4) & 0x0F0F0F0Fu, xt0, xt1, xu0, xu1);
                }
#pragma unroll
                for (int t = 0; t < NT; t++)
                    acc[t][j] = __builtin_amdgcn_sdot4((int)lo, (int)fr.x[t][kk].x,
                                                       __builtin_amdgcn_sdot4((int)hi, (int)fr.x[t][kk].y, acc[t][j],
                                                                              false),
                                                       false);
            }
        }
        const float ws0 = bf16_lo(fr.ws), ws1 = bf16_hi(fr.ws);
#pragma unroll
        for (int t = 0; t < NT; t++) {
            // Complete the 64-column dots: add the other half's columns (lane ^ 1).
            int a0 = acc[t][0] + dpp_xor1(acc[t][0]);
            int a1 = acc[t][1] + dpp_xor1(acc[t][1]);
            int a2 = acc[t][2] + dpp_xor1(acc[t][2]);
            int a3 = acc[t][3] + dpp_xor1(acc[t][3]);
            int r0 = half ? a2 : a0, r1 = half ? a3 : a1;  // this lane's rows 2*half, 2*half+1
            if constexpr (FMT == 0) {
                const int off = MAX_ODD * fr.sum[t];
                r0 = 2 * r0 - off;
                r1 = 2 * r1 - off;
            }
            if constexpr (DOTS) {
                if (live && t == 0) {
                    if (row0 < P.rows) P.dots[(size_t)row0 * P.nc + c] = r0;
                    if (row0 + 1 < P.rows) P.dots[(size_t)(row0 + 1) * P.nc + c] = r1;
                }
            }
            const float sx = fr.sx[t];
            // The reference skips chunks whose activation scale is 0; fma(-0, +0, f) == f for
            // every f (signed zeros included), so such chunks stage an exactly neutral term.
            if (P.exact) {
                float4 *tp = reinterpret_cast<float4 *>(terms + ((size_t)t * P.nc + c) * RB + rloc);
                *tp = sx != 0.0f ? make_float4((float)r0 * sx, ws0, (float)r1 * sx, ws1)
                                 : make_float4(-0.0f, 0.0f, -0.0f, 0.0f);
            } else {
                const float n0 = fmaf((float)r0 * sx, ws0, f[t][0]);
                const float n1 = fmaf((float)r1 * sx, ws1, f[t][1]);
                f[t][0] = sx != 0.0f ? n0 : f[t][0];
                f[t][1] = sx != 0.0f ? n1 : f[t][1];
            }
        }
    };

    // Chunk of iteration i for this lane group: chunks dealt round-robin over the groups.
    auto chunk_of = [&](int i) { return cw0 + i * G + q; };
    const int iters = (cw1 - cw0 + G - 1) / G;  // wave-uniform
    auto valid = [&](int i) { return i < iters && chunk_of(i) < cw1; };
    if constexpr (NT == 1) {
        // Two fragments in flight: chunk i+1 is fetched before chunk i is processed.
        Frag<HP, NT> fa, fb;
        if constexpr (XS == 3) {
            XStage<FMT> xb(P, tok0, cw0, cw1, lane);
            xb.begin();
            if (valid(0)) fetch(fa, chunk_of(0));
            if (valid(1)) fetch(fb, chunk_of(1));
            xb.finish(xl, xsl, xsuml);
            __builtin_amdgcn_wave_barrier();
        } else if constexpr (XS == 5) {
            // As XS 3, but the wave's activation codes, scales and sums are copied into LDS
            // by direct-to-LDS loads issued before the weight loads, and every weight fetch
            // is issued for all lanes (lane groups past the range re-read an in-range
            // chunk), so the compiler can count them: chunk i is computed as soon as its
            // own loads (and everything issued before them, the activation included) have
            // landed, while chunk i + 1 is still in flight.
            const int n = cw1 - cw0;
            if (n > 0) {
                const int n_u4 = n * 4;
                const uint4 *src = reinterpret_cast<const uint4 *>(P.xq + (size_t)tok0 * P.K + (size_t)cw0 * 64);
                const uint32_t m0 = (uint32_t)__builtin_amdgcn_readfirstlane((int)lds_offset(xl + (size_t)cw0 * 64));
                if ((int)lane < n_u4) lds_dma16(src + lane, m0);
                if ((int)lane + 64 < n_u4) lds_dma16(src + lane + 64, m0 + 1024);
                if ((int)lane < n) {
                    lds_dma4(P.xs + (size_t)tok0 * P.nc + cw0 + lane,
                             (uint32_t)__builtin_amdgcn_readfirstlane((int)lds_offset(xsl + cw0)));
                    if constexpr (FMT == 0)
                        lds_dma4(P.xsum + (size_t)tok0 * P.nc + cw0 + lane,
                                 (uint32_t)__builtin_amdgcn_readfirstlane((int)lds_offset(xsuml + cw0)));
                }
            }
            // The same count of loads is outstanding at every loop entry (fa, fb), so the
            // compiler's waits are exact; at most one fetch of a wave is wasted (iters odd).
            auto fetchc = [&](Frag<HP, NT> &fr, int i) { fetch(fr, max(cw0, min(chunk_of(i), cw1 - 1))); };
            if (iters > 0) {
                fetchc(fa, 0);
                fetchc(fb, 1);
                GV_TR(1);
                // The activation copies were issued before these two fetches: once at most
                // their loads are outstanding, the activation is in LDS.  (The compiler does
                // not know the copies write LDS and could move the activation reads up to
                // its own, later, wait for fa.)
                constexpr int kFetchLoads = (kNF3 ? 3 : 4) + (FMT == 0 ? (HP == 0 ? 0 : HP == 1 ? 2 : 4) : 0) + 1;
                wait_vmcnt<2 * kFetchLoads>();
                GV_TR(2);
                int i = 0;
                for (; i + 2 < iters; i += 2) {
                    if (valid(i)) process(fa, chunk_of(i));
                    fetchc(fa, i + 2);
                    if (valid(i + 1)) process(fb, chunk_of(i + 1));
                    fetchc(fb, i + 3);
                }
#ifdef K2T_GEMV_TRACE
                wait_vmcnt<kFetchLoads>();
                GV_TR(3);
#endif
                if (valid(i)) process(fa, chunk_of(i));
                GV_TR(4);
                if (valid(i + 1)) process(fb, chunk_of(i + 1));
                GV_TR(5);
            }
        } else if constexpr (XS != 0) {
            // Source loads first, then the first weight loads; the wave builds its
            // activation while the weights are in flight.
            XBuilder<XS> xb(P, xsrc_p, tok0, cw0, cw1, lane);
            xb.begin();
            if (fused_route) {
                // The expert is not known yet: the activation is built while the routing runs.
                xb.finish(xl, xsl, xsuml);
                __builtin_amdgcn_wave_barrier();
                await_expert();
                if (valid(0)) fetch(fa, chunk_of(0));
                if (valid(1)) fetch(fb, chunk_of(1));
            } else {
                if (valid(0)) fetch(fa, chunk_of(0));
                if (valid(1)) fetch(fb, chunk_of(1));
                xb.finish(xl, xsl, xsuml);
                __builtin_amdgcn_wave_barrier();
            }
        } else {
            if (valid(0)) fetch(fa, chunk_of(0));
        }
        for (int i = 0; XS != 5 && i < iters; i += 2) {
            if (XS == 0 && valid(i + 1)) fetch(fb, chunk_of(i + 1));
            if (valid(i)) process(fa, chunk_of(i));
            if (valid(i + 2)) fetch(fa, chunk_of(i + 2));
            if (valid(i + 1)) process(fb, chunk_of(i + 1));
            if (XS != 0 && valid(i + 3)) fetch(fb, chunk_of(i + 3));
        }
    } else {
        // Multi-token tiles hold NT activation slices per fragment: one in flight.
        for (int i = 0; i < iters; i++) {
            if (!valid(i)) continue;
            Frag<HP, NT> fa;
            fetch(fa, chunk_of(i));
            process(fa, chunk_of(i));
        }
    }

    if (!P.exact) {
        // Fast epilogue: add the lane groups' partial chains (fixed butterfly order, so the
        // result is deterministic), then the waves' partials in wave order.
#pragma unroll
        for (int t = 0; t < NT; t++)
#pragma unroll
            for (int i = 0; i < 2; i++) {
                float v = f[t][i];
                if (smode) v += __int_as_float(dpp_ror8(__float_as_int(v)));  // lane ^ 8
                v += xor_lane(v, 16);
                v += xor_lane(v, 32);
                f[t][i] = v;
            }
        float *part = lds;  // [nseg][NT][RB]
        if (smode ? lane < 8 : lane < 16) {
#pragma unroll
            for (int t = 0; t < NT; t++) {
                part[((size_t)wave * NT + t) * RB + rloc] = f[t][0];
                part[((size_t)wave * NT + t) * RB + rloc + 1] = f[t][1];
            }
        }
        __syncthreads();
        GV_TR(6);
        const int nrows_blk = (is_tail && !smode) ? 16 : RB;
        const int first_stripe = smode ? rb : (is_tail ? 2 * P.np : 2 * rb);
        for (int idx = (int)threadIdx.x; idx < NT * RB; idx += (int)blockDim.x) {
            const int t = idx / RB, rl = idx % RB;
            if (rl >= nrows_blk) continue;
            const int st = first_stripe + rl / 16;
            const int row = st * 16 + rl % 16;
            if (row >= P.rows || st < P.s0 || st >= P.s1) continue;
            float acc = part[(size_t)t * RB + rl];
            for (int w = 1; w < P.nseg; w++) acc += part[((size_t)w * NT + t) * RB + rl];
            float *o = out_p + (size_t)(tok0 + t) * P.out_stride + gu_out_row(row, P.rows, P.gu_split);
            *o = P.accum ? *o + acc : acc;
        }
        return;
    }
    __syncthreads();
    const int nrows_blk = (is_tail && !smode) ? 16 : RB;
    const int first_stripe = smode ? rb : (is_tail ? 2 * P.np : 2 * rb);
    // One thread per (token, row of the block) replays the chain; LDS reads are batched
    // 16 chunks at a time so their latency overlaps.
    for (int idx = (int)threadIdx.x; idx < NT * RB; idx += (int)blockDim.x) {
        const int t = idx / RB, rl = idx % RB;
        if (rl >= nrows_blk) continue;
        const int st = first_stripe + rl / 16;
        const int row = st * 16 + rl % 16;
        if (row >= P.rows || st < P.s0 || st >= P.s1) continue;
        const float2 *tp = terms + (size_t)t * P.nc * RB + rl;
        float acc = 0.0f;
        int c = 0;
        for (; c + 16 <= P.nc; c += 16) {
            float2 v[16];
#pragma unroll
            for (int u = 0; u < 16; u++) v[u] = tp[(size_t)(c + u) * RB];
#pragma unroll
            for (int u = 0; u < 16; u++) acc = fmaf(v[u].x, v[u].y, acc);
        }
        for (; c < P.nc; c++) {
            const float2 v = tp[(size_t)c * RB];
            acc = fmaf(v.x, v.y, acc);
        }
        float *o = out_p + (size_t)(tok0 + t) * P.out_stride + gu_out_row(row, P.rows, P.gu_split);
        *o = P.accum ? *o + acc : acc;
    }
}

uint64_t hadamard_sign_mask_host(uint64_t block) {
    uint64_t mask = 0;
    for (uint64_t i = 0; i < 64; i++) {
        uint64_t z = 0x9E3779B97F4A7C15ull + block * 0xBF58476D1CE4E5B9ull + (i + 1) * 0x9E3779B97F4A7C15ull;
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        z ^= z >> 31;
        mask |= (z & 1) << i;
    }
    return mask;
}

// NF3 stripe-chunks (384 bytes: 8 triplet blocks of 48 bytes, block 4*half + g holding
// rows 4g..4g+3 of the 32-column half `half`, simd_lut.rs:4932-4960) rearranged in place
// into lane order: 16-byte piece k (k = 0..2) of block (g, half) moves from
// 192*half + 48*g + 16*k to 128*k + 16*(2g + half).  Chunk c of a pair record sits at
// (c / sgc) * 64 + c * 768 + 64 + side * 384 (a 64-byte scale header per scale group,
// then the groups' [side 0, side 1] chunks); of the tail stripe at (c / sgc) * 32 + c * 384
// + 32.  Records: nrec matrices rec_stride bytes apart.  A workgroup of 192 threads takes
// 8 chunks, one thread per 16-byte piece: every piece is read (consecutive threads,
// consecutive pieces) before the barrier and written to its new place after it.
constexpr int kLaneChunksPerBlock = 8;
__global__ __launch_bounds__(192) void nf3_lane_order_kernel(uint8_t *base, size_t rec_stride, int nrec, size_t ptot,
                                                             int pairs, int nc, int sgc, int tail) {
    const size_t per_rec = (size_t)pairs * nc * (tail ? 1 : 2);
    const size_t t = (size_t)blockIdx.x * kLaneChunksPerBlock + threadIdx.x / 24;
    const int op = (int)(threadIdx.x % 24);  // piece index in the reference order
    const bool live = t < per_rec * (size_t)nrec;
    uint4 *q = nullptr;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (live) {
        const size_t r = t / per_rec, u = t % per_rec;
        uint8_t *chunk;
        if (tail) {
            const int c = (int)u;
            chunk = base + r * rec_stride + (size_t)(c / sgc) * 32 + (size_t)c * 384 + 32;
        } else {
            const int side = (int)(u & 1), c = (int)((u >> 1) % (size_t)nc);
            const size_t p = (u >> 1) / (size_t)nc;
            chunk = base + r * rec_stride + p * ptot + (size_t)(c / sgc) * 64 + (size_t)c * 768 + 64 +
                    (size_t)side * 384;
        }
        q = reinterpret_cast<uint4 *>(chunk);
        v = q[op];
    }
    __syncthreads();
    if (live) {
        const int h = op / 12, g = (op % 12) / 3, k = op % 3;
        q[k * 8 + 2 * g + h] = v;
    }
}

void launch_nf3_lane_order(hipStream_t st, uint8_t *base, size_t rec_stride, int nrec, size_t ptot, int pairs,
                           int nc, int sgc, bool tail) {
    if ((((uintptr_t)base) | rec_stride | ptot) % 16)
        throw Error(K2T_E_ARG, "NF3 streams must be 16-byte aligned");
    const size_t n = (size_t)pairs * nc * (tail ? 1 : 2) * (size_t)nrec;
    if (n == 0) return;
    const size_t blocks = (n + kLaneChunksPerBlock - 1) / kLaneChunksPerBlock;
    hipLaunchKernelGGL(nf3_lane_order_kernel, dim3((unsigned)blocks), dim3(24 * kLaneChunksPerBlock), 0, st, base,
                       rec_stride, nrec, ptot, pairs, nc, sgc, tail ? 1 : 0);
    hip_check(hipGetLastError(), "nf3 lane order launch");
}

GemvPlan plan_gemv(const k2t_ctx *ctx, const k2t_mat *m, int s0, int s1) {
    GemvPlan p;
    const int npairs = std::min(m->pairs + m->has_tail, (s1 + 1) / 2) - s0 / 2;
    // Fewer pair blocks than CUs: give each stripe its own workgroup so every CU streams.
    p.stripe_mode = npairs < ctx->num_cus ? 1 : 0;
    if (p.stripe_mode) {
        p.rb_lo = s0;
        p.rb_hi = s1;
    } else {
        p.rb_lo = s0 / 2;
        p.rb_hi = s0 / 2 + npairs;
    }
    const int nrb = std::max(p.rb_hi - p.rb_lo, 1);
    const int G = p.stripe_mode ? 8 : 4;  // lane groups per wave
    // A wave's lane groups take chunks round-robin; one full round keeps every lane busy.
    // Short-lived waves of at most two rounds stream best (~14 waves per CU).  Small
    // matrices keep one full round per wave rather than many mostly idle waves.
    const int target = ctx->num_cus * 14;
    const int round = G;
    int cps = (long)nrb * ((m->nc + 2 * round - 1) / (2 * round)) >= target ? 2 * round : round;
    cps = std::max(cps, (m->nc + 15) / 16);  // at most 16 waves per workgroup
    if (ctx->max_segments > 0) cps = std::max(cps, (m->nc + ctx->max_segments - 1) / ctx->max_segments);
    p.cps = cps;
    p.nseg = (m->nc + cps - 1) / cps;
    return p;
}

template <int FMT, int HP, bool DOTS>
static void launch_nt(int nt, int xs, dim3 grid, dim3 block, size_t lds, hipStream_t st, const GemvParams &P) {
    if (xs == K2T_XS_RMSNORM) {
        hipLaunchKernelGGL((gemv_kernel<FMT, HP, 1, false, K2T_XS_RMSNORM>), grid, block, lds, st, P);
        return;
    }
    if (xs == K2T_XS_SWIGLU) {
        hipLaunchKernelGGL((gemv_kernel<FMT, HP, 1, false, K2T_XS_SWIGLU>), grid, block, lds, st, P);
        return;
    }
    if (xs == K2T_XS_STAGED) {
        hipLaunchKernelGGL((gemv_kernel<FMT, HP, 1, false, K2T_XS_STAGED>), grid, block, lds, st, P);
        return;
    }
    if (xs == K2T_XS_STAGED_DMA) {
        hipLaunchKernelGGL((gemv_kernel<FMT, HP, 1, false, K2T_XS_STAGED_DMA>), grid, block, lds, st, P);
        return;
    }
    switch (nt) {
        case 1: hipLaunchKernelGGL((gemv_kernel<FMT, HP, 1, DOTS, 0>), grid, block, lds, st, P); break;
        case 2: hipLaunchKernelGGL((gemv_kernel<FMT, HP, 2, false, 0>), grid, block, lds, st, P); break;
        case 3: hipLaunchKernelGGL((gemv_kernel<FMT, HP, 3, false, 0>), grid, block, lds, st, P); break;
        default: hipLaunchKernelGGL((gemv_kernel<FMT, HP, 4, false, 0>), grid, block, lds, st, P); break;
    }
}

template <bool DOTS>
static void launch_fmt(const k2t_mat *m, int nt, int xs, dim3 grid, dim3 block, size_t lds, hipStream_t st,
                       const GemvParams &P) {
    if (m->fmt == K2T_FMT_NF && m->bits == 3 && m->nf3_lane) launch_nt<3, 0, DOTS>(nt, xs, grid, block, lds, st, P);
    else if (m->fmt == K2T_FMT_NF && m->bits == 3) launch_nt<2, 0, DOTS>(nt, xs, grid, block, lds, st, P);
    else if (m->fmt == K2T_FMT_NF) launch_nt<1, 0, DOTS>(nt, xs, grid, block, lds, st, P);
    else if (m->hp == 0) launch_nt<0, 0, DOTS>(nt, xs, grid, block, lds, st, P);
    else if (m->hp == 1) launch_nt<0, 1, DOTS>(nt, xs, grid, block, lds, st, P);
    else launch_nt<0, 2, DOTS>(nt, xs, grid, block, lds, st, P);
}

static void launch_gemv_impl(k2t_ctx *ctx, const k2t_mat *m, const int8_t *xq, const float *xs,
                             const int32_t *xsum, int ntok, int s0, int s1, float *out, size_t out_stride,
                             int32_t *dots, bool accum, int xsm = 0, const float *src = nullptr,
                             const float *w = nullptr, float eps = 0.0f, const GemvGroup *grp = nullptr,
                             int gu_split = 0, ActTiles tiles = ActTiles{});

void launch_gemv(k2t_ctx *ctx, const k2t_mat *m, const int8_t *xq, const float *xs,
                 const int32_t *xsum, int ntok, int s0, int s1, float *out, size_t out_stride,
                 int32_t *dots) {
    launch_gemv_impl(ctx, m, xq, xs, xsum, ntok, s0, s1, out, out_stride, dots, false);
}

void launch_gemv_ex(k2t_ctx *ctx, const k2t_mat *m, const int8_t *xq, const float *xs, const int32_t *xsum, int ntok,
                    float *out, size_t out_stride, bool accumulate, int gu_split, ActTiles tiles) {
    launch_gemv_impl(ctx, m, xq, xs, xsum, ntok, 0, m->stripes, out, out_stride, nullptr, accumulate, 0, nullptr,
                     nullptr, 0.0f, nullptr, gu_split, tiles);
}

void launch_gemv_fused(k2t_ctx *ctx, const k2t_mat *m, int xs_mode, const float *src, const float *w, float eps,
                       float *out, bool accumulate, int gu_split) {
    launch_gemv_impl(ctx, m, nullptr, nullptr, nullptr, 1, 0, m->stripes, out, (size_t)m->rows, nullptr, accumulate,
                     xs_mode, src, w, eps, nullptr, gu_split);
}

void launch_gemv_grouped(k2t_ctx *ctx, const k2t_mat *geom, const GemvGroup &g, int xs_mode, const float *src,
                         const float *w, float eps, float *out) {
    if (g.nslots <= 0) return;
    if (geom->has_tail) throw Error(K2T_E_INTERNAL, "grouped gemv: expert matrices have no tail stripe");
    if (xs_mode == 0 && (!g.xq || !g.xs || (!g.xsum && geom->fmt != K2T_FMT_NF)))
        throw Error(K2T_E_INTERNAL, "grouped gemv: no activation");
    launch_gemv_impl(ctx, geom, g.xq, g.xs, g.xsum, 1, 0, geom->stripes, out, (size_t)geom->rows, nullptr, false,
                     xs_mode, src, w, eps, &g);
}

static void launch_gemv_impl(k2t_ctx *ctx, const k2t_mat *m, const int8_t *xq, const float *xs,
                             const int32_t *xsum, int ntok, int s0, int s1, float *out, size_t out_stride,
                             int32_t *dots, bool accum, int xsm, const float *src, const float *w, float eps,
                             const GemvGroup *grp, int gu_split, ActTiles tiles) {
    // 16 or more tokens of a ready activation through an NF4 matrix: the matrix-core
    // kernel (one weight pass per 64 tokens; its outputs equal the exact-order GEMV's)
    if (!dots && !grp && xsm == 0 && gu_split == 0 && s0 == 0 && s1 == m->stripes && ctx->mfma &&
        gemm_mfma_supported(m, ntok)) {
        launch_gemm_mfma(ctx, m, xq, xs, xsum, ntok, out, out_stride, accum, tiles);
        return;
    }
    const int saved = ctx->max_segments;
    if (dots) ctx->max_segments = 1;
    GemvPlan plan = plan_gemv(ctx, m, s0, s1);
    if (xsm == K2T_XS_RMSNORM && m->fmt == K2T_FMT_NIBBLE4 && m->hp == 2 && 64 * plan.nseg > kB6NormThreads) {
        constexpr int kSeg = kB6NormThreads / 64;
        plan.cps = (m->nc + kSeg - 1) / kSeg;
        plan.nseg = (m->nc + plan.cps - 1) / plan.cps;
    }
    ctx->max_segments = saved;
    if (plan.rb_hi <= plan.rb_lo || ntok <= 0) return;
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
    P.s0 = s0;
    P.s1 = s1;
    P.rb_lo = plan.rb_lo;
    P.stripe_mode = plan.stripe_mode;
    P.nseg = plan.nseg;
    P.cps = plan.cps;
    P.sgc = m->sgc;
    P.cb0 = m->cb[0];
    P.cb1 = m->cb[1];
    P.cb2 = m->cb[2];
    P.cb3 = m->cb[3];
    P.gu_split = gu_split;  // (grouped launches set their own below)
    // Tokens per weight pass: 4, fewer when the staged terms would not fit in 64 KB of LDS.
    size_t per_tok = ctx->exact ? (size_t)m->nc * (plan.stripe_mode ? 16 : 32) * sizeof(float2)
                                : (size_t)plan.nseg * 32 * sizeof(float);
    int G = (int)std::max<size_t>(1, std::min<size_t>(4, (64 * 1024) / per_tok));
    // One token from a ready int8 activation: stage it through LDS (XS 3) when each wave's
    // chunk range fits the staging registers.
    if (xsm == 0 && ntok == 1 && !dots && !grp && plan.cps <= 32 && ctx->stage_x)
        // NF4: the activation copied by LDS DMA and exact load waits (measured faster on
        // the 4096x14336 / 14336x4096 GEMVs; bit planes and NF3 measured no faster)
        xsm = m->fmt == K2T_FMT_NF && m->bits == 4 ? K2T_XS_STAGED_DMA : K2T_XS_STAGED;
    if (xsm != 0) {  // one token; its int8 activation is built in LDS after the terms
        if (ntok != 1 || m->cols > kSignBlocks * 64 || !ctx->signs) throw Error(K2T_E_INTERNAL, "fused gemv shape");
        P.xsrc = src;
        P.xnorm = w;
        P.eps = eps;
        P.signs = ctx->signs;  // (XS 3 reads P.xq / P.xs / P.xsum set above)
        P.xoff = (int)((per_tok + 15) / 16 * 16);
        per_tok = (size_t)P.xoff + (size_t)m->cols + 8 * (size_t)m->nc;
        G = 1;
    }
    if (grp) {
        P.route = grp->route;
        P.bank = grp->bank;
        P.bank_stride = grp->stride;
        P.mat_off = grp->mat_off;
        P.cb_off = grp->cb_off;
        P.slot_out = grp->slot_out;
        P.slot_src = grp->slot_src;
        P.gu_split = grp->gu_split;
        P.slot_act = grp->slot_act;
        int planes = grp->nslots;
        if (grp->rt_w) {  // routing in this launch: plane 0 routes, slot z is plane z + 1
            if (xsm != K2T_XS_RMSNORM || m->cols > 2048 || grp->rt_E < 1 || grp->rt_E > 256 || !grp->rt_words ||
                !grp->rt_pub || !grp->rt_ctr || !grp->rt_err || !grp->rt_wts || !grp->route)
                throw Error(K2T_E_INTERNAL, "grouped gemv: routing in the launch needs the RMSNorm source, d <= 2048");
            P.rt_w = grp->rt_w;
            P.rt_b = grp->rt_b;
            P.rt_words = grp->rt_words;
            P.rt_pub = grp->rt_pub;
            P.rt_ctr = grp->rt_ctr;
            P.rt_err = grp->rt_err;
            P.rt_wts = grp->rt_wts;
            P.rt_E = grp->rt_E;
            P.rt_k = grp->nslots;
            P.rt_norm = grp->rt_norm;
            P.rt_scoring = grp->rt_scoring;
            P.rt_spin = grp->rt_spin;
            planes += 1;
        }
        const dim3 block(64 * plan.nseg);
        P.lds_terms = 1;
        P.exact = ctx->exact;
        launch_fmt<false>(m, 1, xsm, dim3(plan.rb_hi - plan.rb_lo, 1, planes), block, per_tok, ctx->stream, P);
        hip_check(hipGetLastError(), "grouped gemv launch");
        return;
    }
    const int groups = ntok / G, rem = ntok % G;
    const dim3 block(64 * plan.nseg);
    P.lds_terms = 1;
    P.exact = ctx->exact;
    P.accum = accum ? 1 : 0;
    if (groups > 0) {
        GemvParams Q = P;
        Q.tok_base = 0;
        if (dots && G == 1)
            launch_fmt<true>(m, 1, 0, dim3(plan.rb_hi - plan.rb_lo, groups), block, per_tok, ctx->stream, Q);
        else
            launch_fmt<false>(m, G, xsm, dim3(plan.rb_hi - plan.rb_lo, groups), block, (size_t)G * per_tok,
                              ctx->stream, Q);
        hip_check(hipGetLastError(), "gemv launch");
    }
    if (rem > 0) {
        GemvParams Q = P;
        Q.tok_base = groups * G;
        if (dots) launch_fmt<true>(m, rem, 0, dim3(plan.rb_hi - plan.rb_lo, 1), block, rem * per_tok, ctx->stream, Q);
        else launch_fmt<false>(m, rem, 0, dim3(plan.rb_hi - plan.rb_lo, 1), block, rem * per_tok, ctx->stream, Q);
        hip_check(hipGetLastError(), "gemv launch");
    }
}

}  // namespace k2t
