// Per-wave building blocks of the quantized GEMV for kernels that own their workgroup
// layout (the persistent decode kernel): lane geometry inside a row block, the fetch of
// one chunk record, and the exact integer dots of a lane's two rows.  Layouts are the
// reference's Nibble4SdotMatrix (simd_lut.rs:3264-3400) and NfSdotMatrix
// (simd_lut.rs:4796-5023); the arithmetic is that of sdot_decode_neon /
// nf_sdot_decode_neon (simd_lut.rs:3766-4091, 6074-6364).
#pragma once
#include "k2t_device.h"

namespace k2t {

// Device view of one quantized matrix plus its launch shape inside the persistent kernel.
struct MatDev {
    const uint8_t *pair, *tail;
    size_t ptot;  // NF: bytes per pair stream
    int rows, nc, np, stripes;
    int fmt, hp, sgc;  // fmt: 0 = bit planes (hp hi planes), 1 = NF4
    uint32_t cb0, cb1, cb2, cb3;  // NF4: the codebook's XOR tables T0 T1 U0 U1 (nf4_xor_tables)
    int smode;  // 1: a wave group owns one stripe (16 rows), 0: a stripe pair (32 rows)
    int nseg;   // waves per row block (K segments), a power of two <= 16
    int cps;    // chunks per wave
};

// HP: hi planes of the bit-plane format (0, 1, 2), or kHpMixed: 0 or 1 per matrix,
// read from MatDev::hp at run time (one kernel for models that mix 4- and 5-plane
// matrices, such as p55454).
constexpr int kHpMixed = 3;

template <int HP>
struct WFrag {
    uint4 w[4];
    uint4 h[HP == 0 ? 1 : (HP == 1 || HP == kHpMixed ? 2 : 4)];
    uint32_t ws;
};

// Hi planes of matrix M under template HP.
template <int HP>
__device__ __forceinline__ int hp_of(const MatDev &M) {
    if constexpr (HP == kHpMixed) return M.hp;
    else return HP;
}

// Lane geometry for row block `rb` (a pair, the odd tail stripe, or a stripe in stripe
// mode).  Lane bits: 0 = 8-column half, 1-2 = 4-row group g, 3 = stripe of the pair (pair
// mode) or a lane-group bit (stripe mode), the rest = lane group (chunks round-robin).
struct Geo {
    uint32_t half, g, side, nib_off, hi_off, sc_off, rloc;
    int q, G, RB, first_stripe, nrows;
    bool is_tail, live;
    const uint8_t *mbase;
};

template <int FMT, int HP>
__device__ __forceinline__ Geo make_geo(const MatDev &M, int rb, uint32_t lane) {
    Geo o;
    const bool smode = M.smode != 0;
    o.half = lane & 1u;
    o.g = (lane >> 1) & 3u;
    o.is_tail = smode ? rb >= 2 * M.np : rb >= M.np;
    const uint32_t lane_side = smode ? 0u : (lane >> 3) & 1u;
    o.side = smode ? (uint32_t)(rb & 1) : (o.is_tail ? 0u : lane_side);
    const int pidx = smode ? (rb >> 1) : rb;
    o.G = smode ? 8 : 4;
    o.q = smode ? (int)(lane >> 3) : (int)(lane >> 4);
    o.RB = smode ? 16 : 32;
    o.rloc = (smode ? 0u : o.side * 16u) + 4u * o.g + 2u * o.half;
    o.first_stripe = smode ? rb : (o.is_tail ? 2 * M.np : 2 * rb);
    o.nrows = (o.is_tail && !smode) ? 16 : o.RB;
    o.live = !(o.is_tail && lane_side);
    const uint32_t hp = (uint32_t)hp_of<HP>(M);
    const uint32_t PREC = 1024 + 256 * hp + 64;
    if constexpr (FMT == 0) {
        o.nib_off = (o.is_tail ? 0u : o.side * 512u) + o.g * 32u + o.half * 16u;
        o.hi_off = (o.is_tail ? 512u : 1024u + o.side * 128u * hp) + o.g * 16u;
        o.sc_off = (o.is_tail ? 512u + 128u * hp : 1024u + 256u * hp + o.side * 32u);
    } else {
        o.nib_off = (o.is_tail ? 32u : 64u + o.side * 512u) + o.g * 32u + o.half * 16u;
        o.hi_off = 0;
        o.sc_off = o.is_tail ? 0u : o.side * 32u;
    }
    o.sc_off += (4u * o.g + 2u * o.half) * 2u;
    o.mbase = o.is_tail ? M.tail : M.pair + (size_t)pidx * (FMT == 0 ? (size_t)M.nc * PREC : M.ptot);
    return o;
}

template <int FMT, int HP>
__device__ __forceinline__ void fetch_w(const MatDev &M, const Geo &o, int c, WFrag<HP> &fr) {
    const uint32_t hp = (uint32_t)hp_of<HP>(M);
    const uint32_t PREC = 1024 + 256 * hp + 64;
    const uint32_t TREC = 512 + 128 * hp + 32;
    const uint8_t *rec, *scp;
    if constexpr (FMT == 0) {
        rec = o.mbase + (size_t)c * (o.is_tail ? TREC : PREC);
        scp = rec;
    } else {
        const int sg = c / M.sgc, cst = sg * M.sgc, sb = c - cst;
        const uint8_t *gb =
            o.mbase + (o.is_tail ? (size_t)sg * 32 + (size_t)cst * 512 : (size_t)sg * 64 + (size_t)cst * 1024);
        rec = gb + (size_t)sb * (o.is_tail ? 512 : 1024);
        scp = gb;
    }
#pragma unroll
    for (int kk = 0; kk < 4; kk++) fr.w[kk] = load_stream16(rec + o.nib_off + kk * 128);
    if constexpr (FMT == 0 && HP == 2) {
#pragma unroll
        for (int kk = 0; kk < 4; kk++) fr.h[kk] = load_stream16(rec + o.hi_off + kk * 64);
    } else if constexpr (FMT == 0 && HP == 1) {
        fr.h[0] = load_stream16(rec + o.hi_off);
        fr.h[1] = load_stream16(rec + o.hi_off + 64);
    } else if constexpr (FMT == 0 && HP == kHpMixed) {
        if (hp == 1) {
            fr.h[0] = load_stream16(rec + o.hi_off);
            fr.h[1] = load_stream16(rec + o.hi_off + 64);
        } else {
            fr.h[0] = fr.h[1] = make_uint4(0, 0, 0, 0);
        }
    }
    fr.ws = *reinterpret_cast<const uint32_t *>(scp + o.sc_off);
}

// Exact i32 dots of this lane's two rows (4g + 2*half, +1) with activation chunk x (the
// lane's 8-byte slices of the four 16-column blocks) and its code sum (bit planes).
template <int FMT, int HP>
__device__ __forceinline__ void chunk_dots(const MatDev &M, const WFrag<HP> &fr, uint32_t half, const uint2 *x,
                                           int xsum, int &r0, int &r1) {
    const int MAX_ODD = (1 << (4 + hp_of<HP>(M))) - 1;
    int acc[4] = {0, 0, 0, 0};
#pragma unroll
    for (int kk = 0; kk < 4; kk++) {
        const uint32_t wd[4] = {fr.w[kk].x, fr.w[kk].y, fr.w[kk].z, fr.w[kk].w};
        uint4 hv = make_uint4(0, 0, 0, 0);
        if constexpr (HP == 2) hv = fr.h[kk];
        if constexpr (HP == 1 || HP == kHpMixed) hv = fr.h[kk >> 1];  // zero for a 4-plane matrix
        const uint32_t hd[4] = {hv.x, hv.y, hv.z, hv.w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t d = wd[j];
            uint32_t lo, hi;
            if constexpr (FMT == 0) {
                lo = d & 0x0F0F0F0Fu;
                hi = (d >> 4) & 0x0F0F0F0Fu;
                if constexpr (HP == 2) {
                    lo |= __builtin_rotateright32(hd[j], half ? 30u : 0u) & 0x30303030u;
                    hi |= __builtin_rotateright32(hd[j], half ? 28u : 2u) & 0x30303030u;
                } else if constexpr (HP == 1 || HP == kHpMixed) {
                    const uint32_t e = ((kk & 1) ? 28u : 0u) + 2u * half;
                    lo |= __builtin_rotateright32(hd[j], e) & 0x10101010u;
                    hi |= __builtin_rotateright32(hd[j], (e + 1u) & 31u) & 0x10101010u;
                }
            } else {
                // NF4: M.cb0..cb3 hold the XOR tables of the codebook (nf4_xor_tables)
                lo = nf4_xlut(d & 0x0F0F0F0Fu, M.cb0, M.cb1, M.cb2, M.cb3);
                hi = nf4_xlut((d >> 4) & 0x0F0F0F0Fu, M.cb0, M.cb1, M.cb2, M.cb3);
            }
            acc[j] = __builtin_amdgcn_sdot4((int)lo, (int)x[kk].x,
                                            __builtin_amdgcn_sdot4((int)hi, (int)x[kk].y, acc[j], false), false);
        }
    }
    const int a0 = acc[0] + dpp_xor1(acc[0]);
    const int a1 = acc[1] + dpp_xor1(acc[1]);
    const int a2 = acc[2] + dpp_xor1(acc[2]);
    const int a3 = acc[3] + dpp_xor1(acc[3]);
    r0 = half ? a2 : a0;
    r1 = half ? a3 : a1;
    if constexpr (FMT == 0) {
        r0 = 2 * r0 - MAX_ODD * xsum;
        r1 = 2 * r1 - MAX_ODD * xsum;
    }
}

// One wave's share (K segment `wseg`) of row block `rb` against the activation held in
// LDS (xl codes, xsl scales, xsuml code sums), in two steps so that a caller can wait for
// its activation while the first weights are in flight: start() requests the first two
// chunk fragments; finish() runs the loop.  The fast epilogue: per-lane-group partial
// fmaf chains, summed across lane groups in a fixed butterfly order; lanes holding a
// row's partial write it to part[rloc], part[rloc + 1] (part = this wave's 32-float
// slot).  Every lane of the wave must take part (cross-lane steps).
template <int FMT, int HP>
struct GemvWave {
    const MatDev &M;
    Geo o;
    int cw0, cw1, iters, G, q;
    uint32_t lane, half;
    WFrag<HP> fa, fb;

    __device__ __forceinline__ GemvWave(const MatDev &M_, int rb, bool active, int wseg, uint32_t lane_)
        : M(M_), o{}, lane(lane_), half(lane_ & 1u) {
        if (active) o = make_geo<FMT, HP>(M, rb, lane);
        G = M.smode ? 8 : 4;
        q = M.smode ? (int)(lane >> 3) : (int)(lane >> 4);
        cw0 = wseg * M.cps;
        cw1 = active ? min(M.nc, cw0 + M.cps) : cw0;
        iters = cw1 > cw0 ? (cw1 - cw0 + G - 1) / G : 0;
    }
    __device__ __forceinline__ int chunk_of(int i) const { return cw0 + i * G + q; }
    __device__ __forceinline__ bool valid(int i) const { return i < iters && chunk_of(i) < cw1; }

    __device__ __forceinline__ void start() {
        if (valid(0)) fetch_w<FMT, HP>(M, o, chunk_of(0), fa);
        if (valid(1)) fetch_w<FMT, HP>(M, o, chunk_of(1), fb);
    }

    __device__ __forceinline__ void finish(const int8_t *xl, const float *xsl, const int32_t *xsuml, float *part) {
        float f0 = 0.0f, f1 = 0.0f;
        for (int i = 0; i < iters; i += 2) {
            if (valid(i)) process(fa, chunk_of(i), xl, xsl, xsuml, f0, f1);
            if (valid(i + 2)) fetch_w<FMT, HP>(M, o, chunk_of(i + 2), fa);
            if (valid(i + 1)) process(fb, chunk_of(i + 1), xl, xsl, xsuml, f0, f1);
            if (valid(i + 3)) fetch_w<FMT, HP>(M, o, chunk_of(i + 3), fb);
        }
        if (M.smode) {
            f0 += __int_as_float(dpp_ror8(__float_as_int(f0)));
            f1 += __int_as_float(dpp_ror8(__float_as_int(f1)));
        }
        f0 += __shfl_xor(f0, 16, kWave);
        f0 += __shfl_xor(f0, 32, kWave);
        f1 += __shfl_xor(f1, 16, kWave);
        f1 += __shfl_xor(f1, 32, kWave);
        const uint32_t rloc = (M.smode ? 0u : ((lane >> 3) & 1u) * 16u) + 4u * ((lane >> 1) & 3u) + 2u * half;
        if (M.smode ? lane < 8 : lane < 16) {
            part[rloc] = f0;
            part[rloc + 1] = f1;
        }
    }

    __device__ __forceinline__ void process(const WFrag<HP> &fr, int c, const int8_t *xl, const float *xsl,
                                            const int32_t *xsuml, float &f0, float &f1) const {
        uint2 x[4];
#pragma unroll
        for (int kk = 0; kk < 4; kk++) x[kk] = *reinterpret_cast<const uint2 *>(xl + c * 64 + kk * 16 + half * 8);
        const float sx = xsl[c];
        const int xsum = FMT == 0 ? xsuml[c] : 0;
        int r0, r1;
        chunk_dots<FMT, HP>(M, fr, half, x, xsum, r0, r1);
        // (a chunk with sx == 0 has all-zero codes: its term is +0, so the reference's skip
        // of such chunks needs no test on this path)
        f0 = fmaf((float)r0 * sx, bf16_lo(fr.ws), f0);
        f1 = fmaf((float)r1 * sx, bf16_hi(fr.ws), f1);
    }
};


// ---------------------------------------------------------------------------------------
// LDS-staged weight stream.  The weight fragments of a wave's share of a row block are
// copied straight into LDS by the memory pipeline (global_load_lds_dwordx4: lane L's 16
// bytes land at M0 + 16 L) instead of into registers, so a wave can have its whole share
// of a GEMV task in flight before its input exists, without holding registers for it.
//
// These loads are issued from inline assembly: the compiler does not track them, and so
// never adds the conservative "all vector memory done" wait it inserts before every LDS
// read that follows an LDS-DMA load it knows of.  Their completion is awaited here with
// explicit vmcnt waits.  Vector memory operations of one wave complete in issue order,
// so a compiler-inserted wait for a later load only waits longer, never too little.
// M0 is set inside each statement; no compiler-generated code of these kernels uses M0
// (the build checks the generated assembly for it).

// Number of 1 KB hi-plane pieces a fragment holds (bit planes with hi planes only).
template <int FMT, int HP>
__host__ __device__ constexpr int frag_hi_pieces() {
    return FMT != 0 ? 0 : (HP == 0 ? 0 : (HP == 2 ? 4 : 2));
}
// LDS bytes of one staged fragment: 4 nibble pieces and the hi pieces (1 KB each: 16
// bytes per lane), then the 4-byte BF16 scale pair of every lane.
template <int FMT, int HP>
__host__ __device__ constexpr int frag_lds_bytes() {
    return (4 + frag_hi_pieces<FMT, HP>()) * 1024 + 256;
}
// Load instructions per staged fragment.
template <int FMT, int HP>
__host__ __device__ constexpr int frag_loads() {
    return 4 + frag_hi_pieces<FMT, HP>() + 1;
}


// GemvWave with its fragments staged in LDS: `slots` points at this wave's F fragment
// slots.  start() requests fragments 0 .. F-1 (the whole share when it has at most F);
// finish() computes fragment i from slot i % F and then requests fragment i + F into it,
// so up to F fragments are in flight.  Lane groups past the wave's chunk range load a
// valid in-range chunk whose bytes are never used: every fragment is exactly frag_loads()
// instructions under wave-uniform control flow, which keeps the vmcnt arithmetic exact.
template <int FMT, int HP, int F>
struct GemvWaveLds {
    static constexpr int NH = frag_hi_pieces<FMT, HP>();
    static constexpr int FB = frag_lds_bytes<FMT, HP>();
    static constexpr int L = frag_loads<FMT, HP>();
    static_assert(F >= 1 && F <= 4 && (F - 1) * L < 64, "fragments in flight: 1 to 4 within vmcnt's range");
    const MatDev &M;
    Geo o;
    int cw0, cw1, iters, G, q;
    uint32_t lane, half, slot0;
    bool active;
    // Strided issue: fragment i's loads read ubase + i * dstep + (this lane's fixed offset
    // v_nib / v_hi / v_h2 / v_sc), when the chunks of one fragment advance every lane's
    // records by the same stride (always for bit planes; NF when sgc divides G).
    bool strided;
    const uint8_t *ubase;
    uint32_t dstep, v_nib, v_hi, v_h2, v_sc;

    __device__ __forceinline__ GemvWaveLds(const MatDev &M_, int rb, bool active_, int wseg, uint32_t lane_,
                                           uint8_t *slots)
        : M(M_), lane(lane_), half(lane_ & 1u), active(active_) {
        o = make_geo<FMT, HP>(M, active ? rb : 0, lane);
        G = M.smode ? 8 : 4;
        q = M.smode ? (int)(lane >> 3) : (int)(lane >> 4);
        cw0 = wseg * M.cps;
        cw1 = active ? min(M.nc, cw0 + M.cps) : cw0;
        iters = cw1 > cw0 ? (cw1 - cw0 + G - 1) / G : 0;
        slot0 = (uint32_t)__builtin_amdgcn_readfirstlane((int)lds_offset(slots));
        const uintptr_t mb = (uintptr_t)o.mbase;
        ubase = (const uint8_t *)(((uintptr_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)mb)) |
                                  ((uintptr_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(mb >> 32)) << 32));
        const uint32_t c0 = (uint32_t)(cw0 + q);  // this lane's chunk of fragment 0
        const uint32_t hp = (uint32_t)hp_of<HP>(M);
        uint32_t rec0, sc0;
        if constexpr (FMT == 0) {
            const uint32_t REC = o.is_tail ? 512u + 128u * hp + 32u : 1024u + 256u * hp + 64u;
            rec0 = c0 * REC;
            sc0 = rec0;
            dstep = (uint32_t)G * REC;
            strided = true;
        } else {
            const uint32_t sgc = (uint32_t)M.sgc, cs = o.is_tail ? 512u : 1024u, gsz = o.is_tail ? 32u : 64u;
            const uint32_t sg0 = c0 / sgc;
            rec0 = sg0 * gsz + c0 * cs;       // group base sg*gsz + (sg*sgc)*cs, plus (c - sg*sgc)*cs
            sc0 = sg0 * (gsz + sgc * cs);     // the group base
            dstep = ((uint32_t)G / sgc) * gsz + (uint32_t)G * cs;
            strided = (uint32_t)G % sgc == 0;
        }
        v_nib = rec0 + o.nib_off;
        v_hi = rec0 + o.hi_off;
        v_h2 = hp != 0 ? v_hi + 64u : v_nib;  // the mixed variant's second hi piece (nibbles again for hp 0)
        if (frag_hi_pieces<FMT, HP>() == 2 && hp == 0) v_hi = v_nib;
        v_sc = sc0 + o.sc_off;
        dstep = (uint32_t)__builtin_amdgcn_readfirstlane((int)dstep);  // uniform (is_tail, G, sgc)
    }
    __device__ __forceinline__ int chunk_of(int i) const { return cw0 + i * G + q; }
    __device__ __forceinline__ bool valid(int i) const { return i < iters && chunk_of(i) < cw1; }

    // Issues fragment i (a clamped in-range chunk when i is past the share).
    __device__ __forceinline__ void issue(int i) {
        const uint32_t base = slot0 + (uint32_t)(i % F) * (uint32_t)FB;
        if (strided && cw0 + (i + 1) * G <= cw1) {  // wave-uniform: every lane's chunk is in the share
            const uintptr_t a = (uintptr_t)(ubase + (size_t)i * dstep);  // wave-uniform: keep it in SGPRs
            const uint8_t *sb = (const uint8_t *)(((uintptr_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)a)) |
                                                  ((uintptr_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32))
                                                   << 32));
            lds_dma16_sa<0>(v_nib, sb, base);
            lds_dma16_sa<128>(v_nib, sb, base + 1024);
            lds_dma16_sa<256>(v_nib, sb, base + 2048);
            lds_dma16_sa<384>(v_nib, sb, base + 3072);
            if constexpr (NH == 4) {
                lds_dma16_sa<0>(v_hi, sb, base + 4096);
                lds_dma16_sa<64>(v_hi, sb, base + 5120);
                lds_dma16_sa<128>(v_hi, sb, base + 6144);
                lds_dma16_sa<192>(v_hi, sb, base + 7168);
            } else if constexpr (NH == 2) {
                lds_dma16_sa<0>(v_hi, sb, base + 4096);
                lds_dma16_sa<0>(v_h2, sb, base + 5120);
            }
            lds_dma4_sa<0>(v_sc, sb, base + (4 + NH) * 1024);
            return;
        }
        const int c = cw1 > cw0 ? min(chunk_of(i), cw1 - 1) : 0;
        const uint32_t hp = (uint32_t)hp_of<HP>(M);
        const uint8_t *rec, *scp;
        if constexpr (FMT == 0) {
            const uint32_t PREC = 1024 + 256 * hp + 64, TREC = 512 + 128 * hp + 32;
            rec = o.mbase + (size_t)c * (o.is_tail ? TREC : PREC);
            scp = rec;
        } else {
            const int sg = c / M.sgc, cst = sg * M.sgc, sb = c - cst;
            const uint8_t *gb =
                o.mbase + (o.is_tail ? (size_t)sg * 32 + (size_t)cst * 512 : (size_t)sg * 64 + (size_t)cst * 1024);
            rec = gb + (size_t)sb * (o.is_tail ? 512 : 1024);
            scp = gb;
        }
#pragma unroll
        for (int kk = 0; kk < 4; kk++) lds_dma16(rec + o.nib_off + kk * 128, base + kk * 1024);
        if constexpr (NH == 4) {
#pragma unroll
            for (int kk = 0; kk < 4; kk++) lds_dma16(rec + o.hi_off + kk * 64, base + (4 + kk) * 1024);
        } else if constexpr (NH == 2) {
            // a 4-plane matrix under the mixed variant has no hi bytes: load the nibble
            // bytes again (in range; chunk_dots ignores them for hp 0)
            const uint8_t *h = hp != 0 ? rec + o.hi_off : rec + o.nib_off;
            lds_dma16(h, base + 4 * 1024);
            lds_dma16(hp != 0 ? h + 64 : h, base + 5 * 1024);
        }
        lds_dma4(scp + o.sc_off, base + (4 + NH) * 1024);
    }

    __device__ __forceinline__ void start() {
#pragma unroll
        for (int i = 0; i < F; i++)
            if (i < iters) issue(i);  // wave-uniform
    }

    // Waits until fragment i has landed while `after` later fragments may stay in flight.
    __device__ __forceinline__ static void wait_frag(int after) {
        if constexpr (F >= 4) {
            if (after >= 3) {
                wait_vmcnt<3 * L>();
                return;
            }
        }
        if constexpr (F >= 3) {
            if (after == 2) {
                wait_vmcnt<2 * L>();
                return;
            }
        }
        if constexpr (F >= 2) {
            if (after == 1) {
                wait_vmcnt<L>();
                return;
            }
        }
        wait_vmcnt<0>();
    }

    __device__ __forceinline__ WFrag<HP> read(int i, const uint8_t *slots) const {
        const uint8_t *b = slots + (size_t)(i % F) * FB;
        WFrag<HP> fr;
#pragma unroll
        for (int kk = 0; kk < 4; kk++) fr.w[kk] = *reinterpret_cast<const uint4 *>(b + kk * 1024 + lane * 16);
        if constexpr (NH > 0) {
#pragma unroll
            for (int j = 0; j < NH; j++) fr.h[j] = *reinterpret_cast<const uint4 *>(b + (4 + j) * 1024 + lane * 16);
            if constexpr (HP == kHpMixed) {
                if (M.hp == 0) fr.h[0] = fr.h[1] = make_uint4(0, 0, 0, 0);
            }
        } else {
            fr.h[0] = make_uint4(0, 0, 0, 0);
        }
        fr.ws = *reinterpret_cast<const uint32_t *>(b + (4 + NH) * 1024 + lane * 4);
        return fr;
    }

    // terms != nullptr (exact-order mode): instead of accumulating, each lane stores the
    // reference's per-chunk epilogue operands of its two rows, {float(dot) * sx, bf16 scale}
    // as one 64-bit word (low half the term), at terms[row_local * nc + c]; a neutral
    // {-0, +0} where sx == 0 (the reference skips such chunks, and fmaf(-0, +0, f) == f).
    // The caller replays each row's fmaf chain in chunk order from those words.
    __device__ __forceinline__ void finish(const uint8_t *slots, const int8_t *xl, const float *xsl,
                                           const int32_t *xsuml, float *part, unsigned long long *trace = nullptr,
                                           unsigned long long *terms = nullptr) {
        float f0 = 0.0f, f1 = 0.0f;
        for (int i = 0; i < iters; i++) {
            // fragments i .. min(i + F, iters) - 1 were requested; wait for i
            wait_frag(min(F, iters - i) - 1);
            if (trace && i == 0 && threadIdx.x == 0) trace[2] = wall_clock64();
            const WFrag<HP> fr = read(i, slots);
            if (terms) {
                if (valid(i)) store_terms(fr, chunk_of(i), xl, xsl, xsuml, terms);
            } else if (valid(i)) {
                process(fr, chunk_of(i), xl, xsl, xsuml, f0, f1);
            }
            if (i + F < iters) {  // wave-uniform
                // the slot's LDS reads must complete before the next fragment overwrites it
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                issue(i + F);
            }
        }
        if (terms) return;
        if (M.smode) {
            f0 += __int_as_float(dpp_ror8(__float_as_int(f0)));
            f1 += __int_as_float(dpp_ror8(__float_as_int(f1)));
        }
        f0 += __shfl_xor(f0, 16, kWave);
        f0 += __shfl_xor(f0, 32, kWave);
        f1 += __shfl_xor(f1, 16, kWave);
        f1 += __shfl_xor(f1, 32, kWave);
        const uint32_t rloc = (M.smode ? 0u : ((lane >> 3) & 1u) * 16u) + 4u * ((lane >> 1) & 3u) + 2u * half;
        if (M.smode ? lane < 8 : lane < 16) {
            part[rloc] = f0;
            part[rloc + 1] = f1;
        }
        if (trace && threadIdx.x == 0) trace[3] = wall_clock64();
    }

    __device__ __forceinline__ void store_terms(const WFrag<HP> &fr, int c, const int8_t *xl, const float *xsl,
                                                const int32_t *xsuml, unsigned long long *terms) const {
        uint2 x[4];
#pragma unroll
        for (int kk = 0; kk < 4; kk++) x[kk] = *reinterpret_cast<const uint2 *>(xl + c * 64 + kk * 16 + half * 8);
        const float sx = xsl[c];
        const int xsum = FMT == 0 ? xsuml[c] : 0;
        int r0, r1;
        chunk_dots<FMT, HP>(M, fr, half, x, xsum, r0, r1);
        const bool on = sx != 0.0f;
        const float t0 = on ? (float)r0 * sx : -0.0f, w0 = on ? bf16_lo(fr.ws) : 0.0f;
        const float t1 = on ? (float)r1 * sx : -0.0f, w1 = on ? bf16_hi(fr.ws) : 0.0f;
        const uint32_t rloc = (M.smode ? 0u : ((lane >> 3) & 1u) * 16u) + 4u * ((lane >> 1) & 3u) + 2u * half;
        unsigned long long *d = terms + (size_t)rloc * M.nc + c;
        __hip_atomic_store(d, ((unsigned long long)__float_as_uint(w0) << 32) | __float_as_uint(t0), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(d + M.nc, ((unsigned long long)__float_as_uint(w1) << 32) | __float_as_uint(t1),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    __device__ __forceinline__ void process(const WFrag<HP> &fr, int c, const int8_t *xl, const float *xsl,
                                            const int32_t *xsuml, float &f0, float &f1) const {
        uint2 x[4];
#pragma unroll
        for (int kk = 0; kk < 4; kk++) x[kk] = *reinterpret_cast<const uint2 *>(xl + c * 64 + kk * 16 + half * 8);
        const float sx = xsl[c];
        const int xsum = FMT == 0 ? xsuml[c] : 0;
        int r0, r1;
        chunk_dots<FMT, HP>(M, fr, half, x, xsum, r0, r1);
        const float n0 = fmaf((float)r0 * sx, bf16_lo(fr.ws), f0);
        const float n1 = fmaf((float)r1 * sx, bf16_hi(fr.ws), f1);
        f0 = sx != 0.0f ? n0 : f0;
        f1 = sx != 0.0f ? n1 : f1;
    }
};

}  // namespace k2t
