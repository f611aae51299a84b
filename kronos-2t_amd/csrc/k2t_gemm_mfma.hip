// Batched quantized GEMV (prefill) on the int8 matrix cores of gfx950: out[t][r] =
// sum_c fmaf(float(dot_{r,c,t}) * sx[t][c], ws[r][c], ...) for up to 64 tokens per weight
// pass, the chunk dots from v_mfma_i32_16x16x64_i8.  NF4 (NfSdotMatrix) and the bit-plane
// formats b4 / b5 / b6 (Nibble4SdotMatrix) share the kernel.
//
// The reference runs prefill through the same kernels as decode, four tokens per weight
// pass (nf_sdot_decode_neon's 4-token tile, simd_lut.rs:6074-6364, and the Nibble4 tile
// nibble4_sdot_batch_stripe_range, 4101-4320).  Here one wave owns one 16-row stripe and 16 to 64 tokens: per 64-column
// chunk it decodes the stripe-chunk's codes to int8 once, then runs one MFMA per 16-token
// block (A: 16 rows x 64 codes, B: 64 activation bytes x 16 tokens), so each weight byte
// is read once per 64 tokens instead of once per 4.
//  - NF4: the codebook value of each code (the codebook as two v_perm XOR tables,
//    nf4_xlut); the MFMA gives the chunk dot.
//  - bit planes: the unsigned code u (4 + hp bits: the nibble and the hi-plane bits); the
//    MFMA gives sum(u * x), and the chunk dot of the odd weights 2u - (2^(4+hp) - 1) is
//    2 * sum(u * x) - (2^(4+hp) - 1) * sum(x), as the reference computes it (simd_lut.rs:
//    4030-4045 and 4304-4309: the sdot of the codes acc, then 2 * acc - max_odd * xsum).
// The epilogue is the reference's per-row chain in chunk order (simd_lut.rs:4030-4059,
// 6334-6335: f = fmaf(float(dot) * sx, scale, f), chunks with sx == 0 skipped), so every
// output equals the exact-order GEMV's (k2t_ctx_set_exact) bit for bit.
//
// Operand layouts of v_mfma_i32_16x16x64_i8 (checked on the GPU): lane l holds 16 bytes of
// A row l % 16 and of B column l % 16; the products pair lane l's byte b of A with lane
// l's byte b of B over the four lane groups l / 16, so any one assignment of the 64
// columns to (l / 16, b) used for both operands gives the dot.  Here byte b of group g is
// column 16g + b.  The 16 x 16 int32 result: lane l holds rows 4 (l / 16) + r, r = 0..3,
// of column l % 16.
//
// Nibble bytes of a stripe-chunk (512 per stripe, the same order in both formats:
// NfSdotMatrix, simd_lut.rs:4796-5023; Nibble4SdotMatrix, 3331-3385): byte e of dword j at
// kk*128 + g*32 + half*16 + 4j holds the codes of row 4g + j, columns kk*16 + half*8 + e
// (low nibble) and kk*16 + half*8 + 4 + e (high nibble).  Row i's columns 16kk .. 16kk+15
// are therefore the dwords at kk*128 + (i/4)*32 + 4(i%4) and 16 bytes further: low / high
// nibbles of the first give columns 0-3 / 4-7, of the second 8-11 / 12-15.  Bit-plane hi
// planes: for 16-byte piece p of a stripe's hi bytes (64 bytes apart), dword j of row
// group g (g*16 + 4j) holds the bits of row 4g + j for columns kk*16 .. kk*16+15, kk = 2p
// and 2p + 1 (one hi plane) or kk = p (two), in the bit positions the decode kernels'
// rotations select (chunk_dots in k2t_gemv_core.h).
#include "../../include/k2t_hip.h"
#include "k2t_device.h"
#include "k2t_internal.h"
#include "k2t_kv_dev.h"

namespace k2t {

namespace {

#ifndef K2T_MFMA_DEPTH
#define K2T_MFMA_DEPTH 4
#endif
#ifndef K2T_MFMA_MIN_WAVES
#define K2T_MFMA_MIN_WAVES 2048
#endif
constexpr int kMfmaDepth = K2T_MFMA_DEPTH;         // chunks in flight per wave (unshared kernels)
#ifndef K2T_MFMA_SH_DEPTH
#define K2T_MFMA_SH_DEPTH 2
#endif
constexpr int kMfmaShDepth = K2T_MFMA_SH_DEPTH;    // the same, kernels sharing activation blocks
constexpr long kMfmaMinWaves = K2T_MFMA_MIN_WAVES;  // 8 waves per CU
#ifndef K2T_MFMA_MAX_BLOCKS
#define K2T_MFMA_MAX_BLOCKS 4
#endif
// 16-token blocks per wave: 4, or 8 in a measurement build (16384 x 2048 at 256 tokens:
// 40.0 -> 41.0 us at 188 VGPRs; 1.7B prefill unchanged)
constexpr int kMfmaMaxBlocks = K2T_MFMA_MAX_BLOCKS;

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));
typedef unsigned v2u __attribute__((ext_vector_type(2)));

struct MfArgs {
    const uint8_t *pair, *tail;
    size_t ptot;  // bytes per pair stream
    int rows, nc, np, stripes, sgc_log2;  // NF scale group = 1 << sgc_log2 chunks
    uint32_t t0, t1, u0, u1;  // NF4 codebook XOR tables (nf4_xor_tables)
    const int8_t *xt;  // activations tile-major: [16-token block][chunk][64 lanes][16 bytes]
    const float *st;   // their scales: [16-token block][chunk][16 tokens]
    const int32_t *ut;  // their code sums (bit planes): [16-token block][chunk][16 tokens]
    int K, ntok, nblk;  // nblk: 16-token blocks in the tiles
    float *out;
    size_t out_stride;
    int accum;
    // SwiGLU epilogue (gate_up with interleaved [gate64, up64] blocks): the down input as
    // int8 chunks, scales and sums ([token][nci]) and its tile-major copy
    int8_t *sq;
    float *ss;
    int32_t *ssum;
    ActTiles stiles;
    int nci;
    QkvPostDev qp;  // q / k / v epilogue (the qkv projection at head size 64)
};

// Everything one chunk needs (one ring stage): the stripe-chunk's codes and scales, the
// activation blocks this wave loads (all NB, or with sharing its own one), their scales.
template <int FMT, int NB, bool SH>
struct MfChunk {
    uint32_t d0, d1;
    uint32_t hv;  // bit planes with hi planes: this lane's hi-plane dword
    uint2 sw;
    int4 x[SH ? (NB + 3) / 4 : NB];  // with sharing: blocks wave, wave + 4
    float sx[NB];
    int32_t su[FMT == 0 ? NB : 1];  // bit planes: the tokens' code sums
};

// Buffer resource of a wave-uniform base (raw, no stride; dword 3 as gfx950 wants it).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t mf_rsrc(const void *base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, 0x7FFFFFFF, 0x00020000);
}

struct MfSrc {
    __amdgpu_buffer_rsrc_t w, x, s, u;  // the stripe's stream (pair or tail), the tiles, scales, sums
};

// Per-lane offsets of a stripe-chunk record, fixed for the wave's life.
struct MfLane {
    uint32_t a_off;  // the lane's first nibble dword (the second is 16 bytes further)
    uint32_t h_off;  // its hi-plane dword (bit planes)
    uint32_t s_off;  // its rows' BF16 scale pair
    uint32_t x_off, sx_off;
};

// Every load is a buffer load: the wave-uniform part of its offset in an SGPR, the
// per-lane part (fixed for the wave's life) in one VGPR, so no 64-bit address adds.
//  - NF: group sg = c / sgc starts at sg * gsz + sg * sgc * cs (gsz = 64 bytes of scales,
//    32 in the tail; cs = 1024 bytes of codes per chunk, 512 in the tail), the chunk's
//    codes at that + gsz + (c - sg * sgc) * cs.
//  - bit planes: chunk c's record at c * REC (REC = 1024 + 256 hp + 64, the tail's
//    512 + 128 hp + 32): codes, hi bytes, scales; the lane offsets point inside it.
template <int FMT, int HP, int NB, bool SH>
__device__ __forceinline__ void mf_fetch(const MfArgs &A, const MfSrc &R, const MfLane &L, bool is_tail, int tb0,
                                         uint32_t wave, int c, MfChunk<FMT, NB, SH> &f) {
    uint32_t rec, sgb;
    if constexpr (FMT == 0) {
        rec = (uint32_t)c * (is_tail ? 512u + 128u * HP + 32u : 1024u + 256u * HP + 64u);
        sgb = rec;
    } else {
        const uint32_t sg = (uint32_t)c >> A.sgc_log2, sb = (uint32_t)c - (sg << A.sgc_log2);
        const uint32_t cs = is_tail ? 512u : 1024u, gsz = is_tail ? 32u : 64u;
        sgb = sg * gsz + (sg << A.sgc_log2) * cs;  // scale-group base
        rec = sgb + gsz + sb * cs;
    }
    f.d0 = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(R.w, L.a_off, rec, 0);
    f.d1 = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(R.w, L.a_off + 16u, rec, 0);
    if constexpr (FMT == 0 && HP > 0) f.hv = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(R.w, L.h_off, rec, 0);
    const v2u sw = __builtin_amdgcn_raw_buffer_load_b64(R.w, L.s_off, sgb, 0);
    f.sw = make_uint2(sw[0], sw[1]);
    if constexpr (SH) {
        // With sharing, wave w loads blocks w, w + 4, ...  The load is unconditional (a
        // wave past the blocks re-reads the last one and stores nothing), so the ring
        // stage's registers hold only the new value: a conditional load kept the old one
        // alive, which cost copies, and a wait for nearly every load, at the loop's back
        // edge.
#pragma unroll
        for (int k = 0; k < (NB + 3) / 4; k++) {
            const int b = min((int)wave + 4 * k, NB - 1);
            const uint32_t tile = (uint32_t)min(tb0 + b, A.nblk - 1) * (uint32_t)A.nc + (uint32_t)c;
            const v4u x = __builtin_amdgcn_raw_buffer_load_b128(R.x, L.x_off, tile * 1024u, 0);
            f.x[k] = make_int4((int)x[0], (int)x[1], (int)x[2], (int)x[3]);
        }
    }
#pragma unroll
    for (int b = 0; b < NB; b++) {
        // blocks past the last repeat it; their outputs are never stored
        const uint32_t tile = (uint32_t)min(tb0 + b, A.nblk - 1) * (uint32_t)A.nc + (uint32_t)c;
        if constexpr (!SH) {
            const v4u x = __builtin_amdgcn_raw_buffer_load_b128(R.x, L.x_off, tile * 1024u, 0);
            f.x[b] = make_int4((int)x[0], (int)x[1], (int)x[2], (int)x[3]);
        }
        f.sx[b] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(R.s, L.sx_off, tile * 64u, 0));
        if constexpr (FMT == 0) f.su[b] = (int32_t)__builtin_amdgcn_raw_buffer_load_b32(R.u, L.sx_off, tile * 64u, 0);
    }
}

// One chunk's decode, MFMAs and epilogue steps.  A chunk whose activation scale is 0
// needs no select: its term float(d) * 0 * ws is +-0, and adding +-0 leaves every
// accumulator unchanged (each starts at +0 and a round-to-nearest sum is -0 only when
// both addends are -0, so no accumulator is ever -0).
// With sharing, `bsh` is this chunk's LDS slot ([NB][64 lanes] of 16 bytes): the waves
// that loaded a block store it, one barrier, then every wave reads every block.  Two
// slots alternate: a wave stores into a slot only after the barrier that all waves
// passed once done reading it.
template <int FMT, int HP, int NB, bool SH>
__device__ __forceinline__ void mf_step(const MfArgs &A, const MfChunk<FMT, NB, SH> &f, float (&acc)[NB][4],
                                        int4 *bsh, uint32_t wave, uint32_t lane) {
    if (SH) {
#pragma unroll
        for (int k = 0; k < (NB + 3) / 4; k++)
            if ((int)wave + 4 * k < NB) bsh[(wave + 4 * k) * 64 + lane] = f.x[k];
        __syncthreads();
    }
    v4i a;
    if constexpr (FMT == 0) {
        // the unsigned codes: nibble, then the hi-plane bits (as chunk_dots places them for
        // kk = lane group, half 0 for the first dword and half 1 for the second)
        uint32_t lo0 = f.d0 & 0x0F0F0F0Fu, hi0 = (f.d0 >> 4) & 0x0F0F0F0Fu;
        uint32_t lo1 = f.d1 & 0x0F0F0F0Fu, hi1 = (f.d1 >> 4) & 0x0F0F0F0Fu;
        if constexpr (HP == 2) {
            lo0 |= f.hv & 0x30303030u;
            hi0 |= __builtin_rotateright32(f.hv, 2u) & 0x30303030u;
            lo1 |= __builtin_rotateright32(f.hv, 30u) & 0x30303030u;
            hi1 |= __builtin_rotateright32(f.hv, 28u) & 0x30303030u;
        } else if constexpr (HP == 1) {
            const uint32_t e = (lane & 16u) ? 28u : 0u;  // odd lane group: the piece's upper bits
            lo0 |= __builtin_rotateright32(f.hv, e) & 0x10101010u;
            hi0 |= __builtin_rotateright32(f.hv, e + 1u) & 0x10101010u;
            lo1 |= __builtin_rotateright32(f.hv, e + 2u) & 0x10101010u;
            hi1 |= __builtin_rotateright32(f.hv, e + 3u) & 0x10101010u;
        }
        a[0] = (int)lo0;
        a[1] = (int)hi0;
        a[2] = (int)lo1;
        a[3] = (int)hi1;
    } else {
        a[0] = (int)nf4_xlut(f.d0 & 0x0F0F0F0Fu, A.t0, A.t1, A.u0, A.u1);
        a[1] = (int)nf4_xlut((f.d0 >> 4) & 0x0F0F0F0Fu, A.t0, A.t1, A.u0, A.u1);
        a[2] = (int)nf4_xlut(f.d1 & 0x0F0F0F0Fu, A.t0, A.t1, A.u0, A.u1);
        a[3] = (int)nf4_xlut((f.d1 >> 4) & 0x0F0F0F0Fu, A.t0, A.t1, A.u0, A.u1);
    }
    const float ws[4] = {bf16_lo(f.sw.x), bf16_hi(f.sw.x), bf16_lo(f.sw.y), bf16_hi(f.sw.y)};
#pragma unroll
    for (int b = 0; b < NB; b++) {
        const int4 xb = SH ? bsh[b * 64 + lane] : f.x[b];
        const v4i bv = {xb.x, xb.y, xb.z, xb.w};
        const v4i zero = {0, 0, 0, 0};
        const v4i d = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, bv, zero, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; r++) {
            int dot = d[r];
            if constexpr (FMT == 0) dot = 2 * dot - ((1 << (4 + HP)) - 1) * f.su[b];
            acc[b][r] = fmaf((float)dot * f.sx[b], ws[r], acc[b][r]);
        }
    }
}

// P chunks in flight per wave: a register ring of P stages, unrolled so that each stage
// is a fixed set of registers (no copies, so the compiler's load waits count only the
// stages issued after the one consumed).  Stage i holds chunks i, i + P, i + 2P, ...;
// fetches past the last chunk re-read the last chunk and are never consumed.  Scheduling
// barriers keep each refill right after the step that frees its stage: left to itself,
// the compiler sank every load of a round below the round's last MFMA and a wait for all
// loads, so no load was in flight during compute (256-token 1.7B prefill: o / down 24.8
// -> 22.9 us, gate_up 40.7 -> 39.6 us).  A software-pipelined form (chunk c's MFMAs
// issued before chunk c - 1's epilogue) measured slower (25.3 / 41.5 us): the register
// allocator then copied ring registers at the loop head, which drained the ring.
//
// SH: the waves of a workgroup share their tokens' activation blocks through LDS (wave
// w < NB loads block w; one barrier per chunk) instead of each loading all NB.  Measured
// (256 tokens): 16384 x 2048 at NB 4, 45.7 -> 40.4 us with P 2; 2048 x 8192 at NB 1,
// 36.9 -> 44-49 us (one loader and a barrier per chunk for 128 chunks): on for NB 4 only.
//
// SW (gate_up only): 8 waves per workgroup, so a workgroup holds one interleaved block ic
// of 128 rows ([gate64(ic), up64(ic)], simd_lut.rs:3310-3325) for its 64 tokens, and its
// epilogue is swiglu_act_kernel's instead of a store: per token, v = (g / (1 + exp(-g)))
// * u (swiglu_activate_scalar, real_llm.rs:9801-9805), the FWHT of chunk ic and the int8
// quantization (populate_chunk_fwht_raw) of the down input, with its tile-major copy.
// The same arithmetic in the same order as that kernel, so the outputs are the same.
//
// QP (qkv, head size 64): a workgroup's 4 stripes are one head's 64 rows, and its epilogue
// is qkv_post_kernel's for each of its tokens: bias, q / k RMSNorm and RoPE
// (head_post_vals), then q back into the qkv rows, k and v rotated and stored in the
// cache slot of their position.  The same arithmetic on the same values, so the cache
// and q equal the separate kernel's.
template <int FMT, int HP, int NB, int P, bool SH, bool SW = false, bool QP = false>
__global__ __launch_bounds__(SW ? 512 : 256) void gemm_mfma_kernel(MfArgs A) {
    constexpr int W = SW ? 8 : 4;  // waves (stripes) per workgroup
    static_assert(!SW || (SH && NB == 4), "the SwiGLU epilogue runs on 64-token workgroups");
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: stripe math on SGPRs
    const int stripe_id = (int)blockIdx.x * W + (int)wave;
    // With sharing every wave takes part in every barrier: a wave past the last stripe
    // runs the last stripe's chunks and stores nothing.
    if (!SH && stripe_id >= A.stripes) return;
    const int stripe = min(stripe_id, A.stripes - 1);
    __shared__ int4 bsh[2][SH ? NB * 64 : 1];
    const int tokb = (int)blockIdx.y * 16 * NB;
    const bool is_tail = stripe >= 2 * A.np;
    const uint32_t side = is_tail ? 0u : (uint32_t)(stripe & 1);
    const uint8_t *mbase = is_tail ? A.tail : A.pair + (size_t)(stripe >> 1) * A.ptot;
    const uint32_t li = lane & 15u, lg = lane >> 4;
    MfLane L;
    L.a_off = (is_tail ? 0u : side * 512u) + lg * 128u + (li >> 2) * 32u + 4u * (li & 3u);
    if constexpr (FMT == 0) {
        const uint32_t hib = is_tail ? 512u : 1024u + side * 128u * HP;  // the stripe's hi bytes
        L.h_off = hib + (HP == 2 ? lg : lg >> 1) * 64u + (li >> 2) * 16u + 4u * (li & 3u);
        L.s_off = (is_tail ? 512u + 128u * HP : 1024u + 256u * HP + side * 32u) + 8u * lg;  // rows 4lg .. 4lg+3
    } else {
        L.h_off = 0;
        L.s_off = (is_tail ? 0u : side * 32u) + 8u * lg;
    }
    L.x_off = lane * 16u;
    L.sx_off = li * 4u;
    const MfSrc R{mf_rsrc(mbase), mf_rsrc(A.xt), mf_rsrc(A.st), mf_rsrc(FMT == 0 ? (const void *)A.ut : A.st)};
    const int tb0 = (int)blockIdx.y * NB;
    float acc[NB][4];
#pragma unroll
    for (int b = 0; b < NB; b++)
#pragma unroll
        for (int r = 0; r < 4; r++) acc[b][r] = 0.0f;
    const int nc = A.nc, last = nc - 1;
    MfChunk<FMT, NB, SH> ring[P];
#pragma unroll
    for (int i = 0; i < P; i++) mf_fetch<FMT, HP, NB, SH>(A, R, L, is_tail, tb0, wave, min(i, last), ring[i]);
    int c0 = 0;
    for (; c0 + P <= nc; c0 += P) {
#pragma unroll
        for (int i = 0; i < P; i++) {
            mf_step<FMT, HP, NB, SH>(A, ring[i], acc, bsh[(c0 + i) & 1], wave, lane);
            __builtin_amdgcn_sched_barrier(0);
            mf_fetch<FMT, HP, NB, SH>(A, R, L, is_tail, tb0, wave, min(c0 + P + i, last), ring[i]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int i = 0; i < P - 1; i++)
        if (c0 + i < nc) mf_step<FMT, HP, NB, SH>(A, ring[i], acc, bsh[(c0 + i) & 1], wave, lane);
    if constexpr (QP) {
        __shared__ __align__(16) float eq[16 * NB][68];  // [token][row of the head] (padded rows)
#pragma unroll
        for (int b = 0; b < NB; b++)
#pragma unroll
            for (int r = 0; r < 4; r++) eq[16 * b + li][wave * 16 + 4 * lg + r] = acc[b][r];
        __syncthreads();
        const QkvPostDev &Q = A.qp;
        const int head = (int)blockIdx.x, pos0 = Q.pos_dev[0];
        if (Q.kr.bits == 8) {
            // Four tokens per wave pass: lanes 16k .. 16k + 15 hold token 4 (pass * W + w) + k,
            // four consecutive elements each (head_post4; the K / V rotation and int8 by
            // rotate_quant4 with block 0's signs: fwht_lane + kv_store_head's int8 branch).
            const uint32_t sl = lane & 15u;
            const uint64_t m0 = __ballot(hadamard_sign_bit(0, lane) != 0u);
            for (int tl0 = 4 * (int)wave; tl0 < 16 * NB; tl0 += 4 * W) {
                if (tokb + tl0 >= A.ntok) break;  // wave-uniform
                const int t = tokb + tl0 + (int)lg;
                const bool live = t < A.ntok;
                const float4 e4 = *reinterpret_cast<const float4 *>(&eq[tl0 + (int)lg][4 * sl]);
                float v[4] = {e4.x, e4.y, e4.z, e4.w};
                head_post4(head, Q.nq, Q.nkv, Q.bias, Q.qn, Q.kn, Q.eps, Q.rope, pos0 + min(t, A.ntok - 1), sl, v);
                if (head < Q.nq) {
                    if (live)
                        *reinterpret_cast<float4 *>(A.out + (size_t)t * A.out_stride + (size_t)head * 64 + 4 * sl) =
                            make_float4(v[0], v[1], v[2], v[3]);
                    continue;
                }
                const Chunk4 r = rotate_quant4(v, m0, sl);
                if (live) {
                    const bool is_k = head < Q.nq + Q.nkv;
                    const int kvh = is_k ? head - Q.nq : head - Q.nq - Q.nkv;
                    const size_t slot = ((size_t)Q.layer * Q.nkv + kvh) * Q.kr.cap + ring_slot(Q.kr, pos0 + t);
                    *reinterpret_cast<uint32_t *>((is_k ? Q.kq : Q.vq) + slot * 64 + 4 * sl) = r.w;
                    if (sl == 0) (is_k ? Q.ks : Q.vs)[slot] = r.scale;
                }
            }
            return;
        }
        for (int tl = (int)wave; tl < 16 * NB; tl += W) {
            const int t = tokb + tl;
            if (t >= A.ntok) break;  // wave-uniform
            float v0 = eq[tl][lane], v1 = 0.0f;
            head_post_vals(head, Q.nq, Q.nkv, 64, Q.bias, Q.qn, Q.kn, Q.eps, Q.rope, pos0 + t, lane, v0, v1);
            if (head < Q.nq) {
                A.out[(size_t)t * A.out_stride + (size_t)head * 64 + lane] = v0;
                continue;
            }
            const bool is_k = head < Q.nq + Q.nkv;
            const int kvh = is_k ? head - Q.nq : head - Q.nq - Q.nkv;
            const size_t slot = ((size_t)Q.layer * Q.nkv + kvh) * Q.kr.cap + ring_slot(Q.kr, pos0 + t);
            kv_store_head(fwht_lane(v0, 0, lane), 0.0f, 1, lane, Q.kr.bits, 64, slot, is_k ? Q.kq : Q.vq,
                          is_k ? Q.ks : Q.vs);
        }
        return;
    }
    if constexpr (SW) {
        __shared__ float4 ep4[64][33];  // [token][row of the block / 4] (+1 float4 of padding)
        float *ep = reinterpret_cast<float *>(ep4);
#pragma unroll
        for (int b = 0; b < NB; b++)
#pragma unroll
            for (int r = 0; r < 4; r++) ep[(16 * b + li) * 132 + wave * 16 + 4 * lg + r] = acc[b][r];
        __syncthreads();
        const int ic = (int)blockIdx.x;
        // Four tokens per wave at a time: lanes 16k .. 16k + 15 hold token tl0 + k, four
        // consecutive elements each (rotate_quant4: the arithmetic of fwht_lane +
        // quant_chunk_store in that layout, so the codes, scales and sums are the same).
        const uint64_t smask = __ballot(hadamard_sign_bit((uint64_t)ic, lane) != 0u);
        const uint32_t sl = lane & 15u;
        for (int tl0 = 4 * (int)wave; tl0 < 16 * NB; tl0 += 4 * W) {
            if (tokb + tl0 >= A.ntok) break;  // wave-uniform
            const int tl = tl0 + (int)(lane >> 4), t = tokb + tl;
            const float4 g4 = ep4[tl][sl], u4 = ep4[tl][16 + sl];
            const float gs[4] = {g4.x, g4.y, g4.z, g4.w}, us[4] = {u4.x, u4.y, u4.z, u4.w};
            float v[4];
#pragma unroll
            for (int j = 0; j < 4; j++) v[j] = (gs[j] / (1.0f + expf(-gs[j]))) * us[j];
            const Chunk4 r = rotate_quant4(v, smask, sl);
            if (t < A.ntok)
                chunk4_store(r, sl, t, ic, A.nci, A.sq, A.ss, A.ssum, A.stiles.xt, A.stiles.st, A.stiles.ut);
        }
        return;
    }
    if (stripe_id >= A.stripes) return;
#pragma unroll
    for (int b = 0; b < NB; b++) {
        const int t = tokb + 16 * b + (int)li;
        if (t >= A.ntok) continue;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int row = stripe * 16 + 4 * (int)lg + r;
            if (row >= A.rows) continue;
            float *o = A.out + (size_t)t * A.out_stride + row;
            *o = A.accum ? *o + acc[b][r] : acc[b][r];
        }
    }
}

// Tile-major copy of the activations: one 16-token x 64-column tile per 1 KB, in the
// order the MFMA's B operand is read (lane l = 16g + t holds token t's columns 16g ..
// 16g + 15), so each B load of a wave is 1 KB contiguous, with the chunk scales (and
// code sums, for bit planes) in 16-token groups.  Tokens past ntok repeat the last token.
// One thread per 16 bytes; blockIdx.y is the 16-token block.
__global__ __launch_bounds__(256) void mf_tile_kernel(const int8_t *xq, const float *xs, const int32_t *xsum, int K,
                                                      int nc, int ntok, int8_t *xt, float *st, int32_t *ut) {
    const int c = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6), tb = (int)blockIdx.y;
    if (c >= nc) return;
    const uint32_t lane = threadIdx.x & 63u, li = lane & 15u, lg = lane >> 4;
    const int tok = min(tb * 16 + (int)li, ntok - 1);
    const size_t tile = (size_t)tb * nc + c;
    *reinterpret_cast<int4 *>(xt + tile * 1024 + lane * 16) =
        *reinterpret_cast<const int4 *>(xq + (size_t)tok * K + (size_t)c * 64 + 16 * lg);
    if (lg == 0) st[tile * 16 + li] = xs[(size_t)tok * nc + c];
    if (lg == 1 && ut) ut[tile * 16 + li] = xsum[(size_t)tok * nc + c];
}

}  // namespace

bool gemm_mfma_supported(const k2t_mat *m, int ntok) {
    if (ntok < kMfmaMinTokens || m->cols % 64 != 0) return false;
    if (m->fmt == K2T_FMT_NF) return m->bits == 4 && (m->sgc & (m->sgc - 1)) == 0;
    return m->fmt == K2T_FMT_NIBBLE4 && m->hp >= 0 && m->hp <= 2;
}

template <int FMT, int HP>
static void launch_gemm_mfma_fmt(hipStream_t st, int nb, dim3 grid, const MfArgs &A) {
    switch (nb) {
        case 1: hipLaunchKernelGGL((gemm_mfma_kernel<FMT, HP, 1, kMfmaDepth, false>), grid, dim3(256), 0, st, A); break;
        case 2: hipLaunchKernelGGL((gemm_mfma_kernel<FMT, HP, 2, kMfmaDepth, false>), grid, dim3(256), 0, st, A); break;
        case 3: hipLaunchKernelGGL((gemm_mfma_kernel<FMT, HP, 3, kMfmaDepth, false>), grid, dim3(256), 0, st, A); break;
        case 4: hipLaunchKernelGGL((gemm_mfma_kernel<FMT, HP, 4, kMfmaShDepth, true>), grid, dim3(256), 0, st, A); break;
        default:
            if constexpr (kMfmaMaxBlocks >= 8)
                hipLaunchKernelGGL((gemm_mfma_kernel<FMT, HP, 8, kMfmaShDepth, true>), grid, dim3(256), 0, st, A);
            break;
    }
}

// Arguments of one launch over all of m's stripes, and the tile-major activation (the
// producer's, else copied here into the context's scratch: 1 KB + 64 B of scales + 64 B
// of code sums per tile).  Returns the 16-token blocks per wave the launch will use.
static int mfma_args(k2t_ctx *ctx, const k2t_mat *m, const int8_t *xq, const float *xs, const int32_t *xsum,
                     int ntok, ActTiles tiles, MfArgs &A) {
    const bool planes = m->fmt == K2T_FMT_NIBBLE4;
    A = MfArgs{};
    A.pair = m->pair;
    A.tail = m->tail;
    A.ptot = m->pairs ? m->pair_len / m->pairs : 0;
    A.rows = m->rows;
    A.nc = m->nc;
    A.np = m->pairs;
    A.stripes = m->stripes;
    A.sgc_log2 = planes ? 0 : __builtin_ctz((unsigned)m->sgc);
    if (!planes) nf4_xor_tables(m->cb[0], m->cb[1], m->cb[2], m->cb[3], A.t0, A.t1, A.u0, A.u1);
    const int blocks = (ntok + 15) / 16;
    int8_t *xt = tiles.xt;
    float *stile = tiles.st;
    int32_t *utile = tiles.ut;
    if (!xt || (planes && !utile)) {
        const size_t ntile = (size_t)blocks * m->nc;
        ensure_scratch(ctx, ntile * (1024 + 64 + 64) / sizeof(float));
        xt = reinterpret_cast<int8_t *>(ctx->scratch);
        stile = ctx->scratch + ntile * 256;
        utile = reinterpret_cast<int32_t *>(ctx->scratch + ntile * 272);
        hipLaunchKernelGGL(mf_tile_kernel, dim3((m->nc + 3) / 4, blocks), dim3(256), 0, ctx->stream, xq, xs, xsum,
                           m->cols, m->nc, ntok, xt, stile, planes ? utile : nullptr);
    }
    A.xt = xt;
    A.nblk = blocks;
    A.st = stile;
    A.ut = utile;
    A.K = m->cols;
    A.ntok = ntok;
    // Tokens per wave: the most 16-token blocks (fewest weight passes) that still give
    // the launch kMfmaMinWaves waves.
    int nb = std::min(kMfmaMaxBlocks, blocks);
    if (nb > 4 && nb < 8) nb = 4;
    while (nb > 1 && (long)m->stripes * ((blocks + nb - 1) / nb) < kMfmaMinWaves) nb = nb > 4 ? 4 : nb > 2 ? 2 : 1;
    return nb;
}

void launch_gemm_mfma(k2t_ctx *ctx, const k2t_mat *m, const int8_t *xq, const float *xs, const int32_t *xsum,
                      int ntok, float *out, size_t out_stride, bool accum, ActTiles tiles) {
    if (!gemm_mfma_supported(m, ntok)) throw Error(K2T_E_INTERNAL, "mfma gemm: unsupported matrix");
    MfArgs A;
    const int nb = mfma_args(ctx, m, xq, xs, xsum, ntok, tiles, A);
    A.out = out;
    A.out_stride = out_stride;
    A.accum = accum ? 1 : 0;
    const dim3 grid((m->stripes + 3) / 4, (ntok + 16 * nb - 1) / (16 * nb));
    hipStream_t st = ctx->stream;
    if (m->fmt == K2T_FMT_NF) launch_gemm_mfma_fmt<1, 0>(st, nb, grid, A);
    else if (m->hp == 0) launch_gemm_mfma_fmt<0, 0>(st, nb, grid, A);
    else if (m->hp == 1) launch_gemm_mfma_fmt<0, 1>(st, nb, grid, A);
    else launch_gemm_mfma_fmt<0, 2>(st, nb, grid, A);
    hip_check(hipGetLastError(), "mfma gemm launch");
}

template <int FMT, int HP>
static void launch_qkv_fmt(hipStream_t st, int nb, dim3 grid, const MfArgs &A) {
    const dim3 blk(256);
    switch (nb) {
        case 1: hipLaunchKernelGGL((gemm_mfma_kernel<FMT, HP, 1, kMfmaDepth, false, false, true>), grid, blk, 0, st, A); break;
        case 2: hipLaunchKernelGGL((gemm_mfma_kernel<FMT, HP, 2, kMfmaDepth, false, false, true>), grid, blk, 0, st, A); break;
        case 3: hipLaunchKernelGGL((gemm_mfma_kernel<FMT, HP, 3, kMfmaDepth, false, false, true>), grid, blk, 0, st, A); break;
        default: hipLaunchKernelGGL((gemm_mfma_kernel<FMT, HP, 4, kMfmaShDepth, true, false, true>), grid, blk, 0, st, A);
    }
}

bool launch_gemm_mfma_qkv(k2t_ctx *ctx, const k2t_mat *qkv, ActTiles tiles, int ntok, float *out, size_t out_stride,
                          const QkvPostDev &qp) {
    if (!gemm_mfma_supported(qkv, ntok) || !tiles.xt || qkv->rows % 64 != 0) return false;
    if (qkv->fmt == K2T_FMT_NIBBLE4 && !tiles.ut) return false;
    MfArgs A;
    const int nb = std::min(4, mfma_args(ctx, qkv, nullptr, nullptr, nullptr, ntok, tiles, A));
    A.out = out;
    A.out_stride = out_stride;
    A.qp = qp;
    const dim3 grid(qkv->rows / 64, (ntok + 16 * nb - 1) / (16 * nb));
    hipStream_t st = ctx->stream;
    if (qkv->fmt == K2T_FMT_NF) launch_qkv_fmt<1, 0>(st, nb, grid, A);
    else if (qkv->hp == 0) launch_qkv_fmt<0, 0>(st, nb, grid, A);
    else if (qkv->hp == 1) launch_qkv_fmt<0, 1>(st, nb, grid, A);
    else launch_qkv_fmt<0, 2>(st, nb, grid, A);
    hip_check(hipGetLastError(), "mfma qkv launch");
    return true;
}

template <int FMT, int HP>
static void launch_swiglu_fmt(hipStream_t st, dim3 grid, const MfArgs &A) {
    hipLaunchKernelGGL((gemm_mfma_kernel<FMT, HP, 4, kMfmaShDepth, true, true>), grid, dim3(512), 0, st, A);
}

bool launch_gemm_mfma_swiglu(k2t_ctx *ctx, const k2t_mat *gu, ActTiles tiles, int ntok, int8_t *q, float *s,
                             int32_t *sums, ActTiles out_tiles) {
    if (!gemm_mfma_supported(gu, ntok) || !tiles.xt || !out_tiles.xt || gu->rows % 128 != 0) return false;
    if (gu->fmt == K2T_FMT_NIBBLE4 && !tiles.ut) return false;
    // Only where the plain GEMV would take 64-token workgroups anyway: forcing them on a
    // small gate_up (135M: 3072 rows, 768 waves at 256 tokens) cost more than the launch
    // the fusion saves (135M prefill 130k -> 123k tok/s).
    MfArgs A;
    if (mfma_args(ctx, gu, nullptr, nullptr, nullptr, ntok, tiles, A) != 4) return false;
    A.sq = q;
    A.ss = s;
    A.ssum = sums;
    A.stiles = out_tiles;
    A.nci = gu->rows / 128;
    const dim3 grid(gu->rows / 128, (ntok + 63) / 64);
    hipStream_t st = ctx->stream;
    if (gu->fmt == K2T_FMT_NF) launch_swiglu_fmt<1, 0>(st, grid, A);
    else if (gu->hp == 0) launch_swiglu_fmt<0, 0>(st, grid, A);
    else if (gu->hp == 1) launch_swiglu_fmt<0, 1>(st, grid, A);
    else launch_swiglu_fmt<0, 2>(st, grid, A);
    hip_check(hipGetLastError(), "mfma gate_up + swiglu launch");
    return true;
}

}  // namespace k2t
