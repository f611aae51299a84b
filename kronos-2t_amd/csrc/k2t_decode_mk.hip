// Persistent single-launch decode step for gfx950: the reference's decode megakernel
// (forward_token_sdot_megakernel, real_llm.rs:6794-7403) as one HIP kernel of one
// workgroup per CU.
//
// The reference runs its phases on a thread pool with a barrier between them.  On
// MI355X a grid barrier is the expensive part (device-scope fences write back the L2 of
// every XCD), so the phases here are linked by data instead: every vector handed from one
// phase to the next is stored as 64-bit words {32-bit payload, 32-bit epoch}, written and
// read with agent-scope atomics (coherent across XCDs, no fence needed because payload
// and flag travel in one word).  A consumer polls exactly the words it needs until their
// epoch matches the current (step, layer, phase); a workgroup with no task in a phase
// goes on to the next one and starts streaming its weights early.  Every poll is bounded:
// on timeout the kernel raises an error flag and all workgroups exit.
//
// Phases per layer (real_llm.rs:6929-7333):
//   1 qkv   : RMSNorm + FWHT + int8 of hidden (built per workgroup in LDS), qkv GEMV
//   2 attn  : per q head: bias, RoPE, int8 Hadamard K/V of this position (stored by the
//             first q head of each KV group), q8 attention over the cache, IFWHT, FWHT
//             with the o_proj chunk index, int8 -> o activation chunks
//   3 o     : o_proj GEMV, hidden_mid = hidden + o
//   4 gu    : RMSNorm + FWHT + int8 of hidden_mid, gate_up GEMV of one [gate64, up64]
//             block per task, SwiGLU + FWHT (chunk ic) + int8 -> down activation chunks
//   5 down  : down GEMV, hidden = hidden_mid + down
// then the final norm and lm_head GEMV (logits).  For greedy generation the same launch
// also picks the next token (argmax_kernel's tie rule: largest value, lowest row) and
// advances the position and the step counter (workgroup 0, after every workgroup's
// per-row maximum has arrived).
#include <float.h>
#include <math.h>

#include <algorithm>
#include <vector>

#include "../../include/k2t_hip.h"
#include "k2t_decode_mk.h"
#include "k2t_expf.h"
#include "k2t_gemv_core.h"
#include "k2t_internal.h"

namespace k2t {

namespace {

// Threads per workgroup: 512 (8 waves, two per SIMD, 256 VGPRs each) for single-format
// models; 256 (one wave per SIMD, 512 VGPRs) for the mixed 4/5-plane variant, whose
// fragments do not fit in 256.  Device helpers take the count as a template parameter.
constexpr int kMaxThreads = 512;
constexpr int kMaxWaves = kMaxThreads / 64;
constexpr int kActWords = 18;  // per 64-element activation chunk: 16 code words, scale, sum
constexpr int kMkFrags = 4;    // weight fragments in flight per wave (LDS slots)
constexpr size_t kMkMaxLds = 160 * 1024;  // LDS of one gfx950 CU (one workgroup per CU)

__device__ __forceinline__ void ll_store(unsigned long long *p, uint32_t v, uint32_t epoch) {
    __hip_atomic_store(p, ((unsigned long long)epoch << 32) | v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ unsigned long long ll_load(const unsigned long long *p) {
    return __hip_atomic_load(const_cast<unsigned long long *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Workgroup barrier for LDS data only.  __syncthreads() also waits for every global
// store and load of the wave to complete (its release fence); hand-off words need no
// ordering (payload and epoch travel in one word) and weight fragments are awaited
// explicitly, so the phases use this barrier and never stall on store acknowledgements.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Polls one word until its epoch matches; false on timeout or when another workgroup
// has raised the error flag.
__device__ bool ll_wait(const MkParams &P, const unsigned long long *p, uint32_t epoch, uint32_t &v) {
    for (uint32_t spins = 0;; spins++) {
        const unsigned long long w = ll_load(p);
        if ((uint32_t)(w >> 32) == epoch) {
            v = (uint32_t)w;
            return true;
        }
        if ((spins & 31u) == 31u) {
            if (__hip_atomic_load(P.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) return false;
            if (spins > P.spin_limit) {
                __hip_atomic_store(P.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                return false;
            }
            __builtin_amdgcn_s_sleep(1);
        }
    }
}

struct Lds {
    float *hbuf;     // [d] fp32 vector being normalised
    int8_t *xl;      // [kmax] int8 activation of the current GEMV
    float *xsl;      // [kmax/64]
    int32_t *xsuml;  // [kmax/64]
    float *part;     // [16][32] wave partials
    float *vec;      // [128] gate_up block / attention vectors
    float *att;      // attention scratch: q, k, v f32 [3*hd], int8 q/k/v [3*hd], opart, scores
    uint8_t *ring;   // GEMV weight fragments staged in LDS (kMkFrags slots per wave); shares
                     // its bytes with `att` (a workgroup runs one task at a time)
    int *flag;       // [4] workgroup flags
};

__host__ __device__ constexpr size_t pad16(size_t b) { return (b + 15) / 16 * 16; }

__device__ Lds carve(const MkParams &P, float *base) {
    Lds L;
    char *p = reinterpret_cast<char *>(base);
    L.hbuf = reinterpret_cast<float *>(p);
    p += pad16((size_t)P.d * 4);
    L.xl = reinterpret_cast<int8_t *>(p);
    p += pad16((size_t)P.kmax);
    L.xsl = reinterpret_cast<float *>(p);
    p += pad16((size_t)(P.kmax / 64) * 4);
    L.xsuml = reinterpret_cast<int32_t *>(p);
    p += pad16((size_t)(P.kmax / 64) * 4);
    L.part = reinterpret_cast<float *>(p);
    p += kMaxWaves * 32 * 4;
    L.vec = reinterpret_cast<float *>(p);
    p += 128 * 4;
    L.flag = reinterpret_cast<int *>(p);
    p += 16;
    // 256-byte alignment by an offset from the base (the dynamic LDS starts at address 0):
    // an integer round trip of the pointer would hide from the compiler that it points to
    // LDS, and every access through it would become a flat access, which waits for the
    // wave's outstanding global loads as well.
    const size_t used = (size_t)(p - reinterpret_cast<char *>(base));
    p = reinterpret_cast<char *>(base) + ((used + 255) & ~(size_t)255);
    L.att = reinterpret_cast<float *>(p);
    L.ring = reinterpret_cast<uint8_t *>(p);
    return L;
}

// Waits for n LL words: each thread issues the loads of its (up to kPoll) words, then
// re-requests all of its words that are not yet current together, one round trip per
// poll, until every one holds `epoch` (bounded like ll_wait).  Payloads go to dst (fp32
// vector, act == false) or are unpacked into the LDS activation (codes, scales, sums;
// act == true).  Returns false (for the whole workgroup) on error.
constexpr int kPoll = 8;
// Only threads t0 .. NTH-1 poll (the others are streaming weights, and a poll of theirs
// would return only after those loads: vector memory completes in issue order).
template <int NTH>
__device__ __forceinline__ bool load_words(const MkParams &P, const Lds &S, const unsigned long long *src, int n,
                                           uint32_t epoch, bool act, float *dst, int t0 = 0) {
    bool ok = true;
    const int np = NTH - t0;
    for (int i0 = (int)threadIdx.x - t0; i0 >= 0 && i0 < n; i0 += np * kPoll) {
        unsigned long long w[kPoll];
#pragma unroll
        for (int k = 0; k < kPoll; k++) {
            const int i = i0 + k * np;
            w[k] = i < n ? ll_load(src + i) : 0ull;
        }
        uint32_t pending = 0;
#pragma unroll
        for (int k = 0; k < kPoll; k++)
            if (i0 + k * np < n && (uint32_t)(w[k] >> 32) != epoch) pending |= 1u << k;
        for (uint32_t spins = 0; pending != 0 && ok; spins++) {
            if ((spins & 31u) == 31u) {
                if (__hip_atomic_load(P.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) {
                    ok = false;
                    break;
                }
                if (spins > P.spin_limit) {
                    __hip_atomic_store(P.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    ok = false;
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
#pragma unroll
            for (int k = 0; k < kPoll; k++)
                if (pending & (1u << k)) w[k] = ll_load(src + i0 + k * np);
#pragma unroll
            for (int k = 0; k < kPoll; k++)
                if ((pending & (1u << k)) && (uint32_t)(w[k] >> 32) == epoch) pending &= ~(1u << k);
        }
#pragma unroll
        for (int k = 0; k < kPoll; k++) {
            const int i = i0 + k * np;
            if (i < n && ok) {
                const uint32_t v = (uint32_t)w[k];
                if (!act) {
                    dst[i] = __uint_as_float(v);
                } else {
                    const int c = i / kActWords, wd = i % kActWords;
                    if (wd < 16) reinterpret_cast<uint32_t *>(S.xl + c * 64)[wd] = v;
                    else if (wd == 16) S.xsl[c] = __uint_as_float(v);
                    else S.xsuml[c] = (int32_t)v;
                }
            }
        }
    }
    // one barrier: S.flag[1] is set to this phase's epoch on failure (no earlier phase had it)
    if (!ok) S.flag[1] = (int)epoch;
    lds_barrier();
    return S.flag[1] != (int)epoch;
}

// Hadamard sign mask of 64-block `block` (wave-uniform) by a scalar load: the table is
// read-only, and a vector load here would also wait for the wave's earlier stores.
__device__ __forceinline__ uint64_t sign_mask_s(const MkParams &P, int block) {
    using CU64 = const __attribute__((address_space(4))) uint64_t;
    return ((CU64 *)P.signs)[__builtin_amdgcn_readfirstlane(block)];
}

// Stores a quantized chunk (simd_lut.rs:3097-3128 arithmetic) held in the four-element
// layout (every 16-lane group holds the whole chunk) as kActWords LL words: word w holds
// the codes of elements 4w .. 4w+3 (byte b = element 4w+b), word 16 the scale, word 17
// the code sum.  Lane group g (lane / 16) writes copies g, g + 4, ...; lane s of a group
// writes word s, and its lane 0 words 16 and 17.
__device__ __forceinline__ void store_act_chunk4(const Chunk4 &r, uint32_t lane, unsigned long long *dst,
                                                 uint32_t epoch, int rep, size_t copy_stride) {
    const uint32_t s = lane & 15u;
    for (int c = (int)(lane >> 4); c < rep; c += 4) {
        unsigned long long *d = dst + (size_t)c * copy_stride;
        ll_store(d + s, r.w, epoch);
        if (s == 0) {
            ll_store(d + 16, __float_as_uint(r.scale), epoch);
            ll_store(d + 17, (uint32_t)r.sum, epoch);
        }
    }
}

// Words per copy of the replicated hand-off vectors.
__device__ __forceinline__ size_t oact_words(const MkParams &P) { return (size_t)(P.nq * P.hd / 64) * kActWords; }
__device__ __forceinline__ size_t gact_words(const MkParams &P) { return (size_t)(P.inter / 64) * kActWords; }
// The copy this workgroup reads (workgroups are dispatched round-robin over the 8 XCDs,
// so copy blockIdx.x mod 4 is shared by the workgroups of two XCDs).
__device__ __forceinline__ size_t my_copy(const MkParams &P) { return (size_t)(blockIdx.x % (unsigned)P.rep); }

// Norm weights and Hadamard sign mask of this lane's first slice (chunk wave*4 + lane/16,
// elements (lane%16)*4 .. +4), requested at the start of a phase, before its weight
// stream and its input wait, so the build after the wait does not wait for them.
struct NormPre {
    float4 a;
    uint64_t sign;
};
template <int NTH>
__device__ __forceinline__ NormPre norm_prefetch(const MkParams &P, const float *w, uint32_t lane, int wave) {
    NormPre r{};
    const int c = wave * 4 + (int)(lane >> 4), cc = c < P.d / 64 ? c : 0;
    if (w && wave * 4 < P.d / 64) {
        r.a = *reinterpret_cast<const float4 *>(w + cc * 64 + (lane & 15u) * 4);
        r.sign = P.signs[cc];
    }
    return r;
}

// RMSNorm + FWHT + int8 of S.hbuf[0..d) into the LDS activation: inv_rms in row_sumsq_wave
// order (bit-identical to rmsnorm_act_kernel); then sixteen lanes per
// chunk, four chunks per wave at once (rotate_quant4).  The first slice of each lane uses
// the prefetched weights and sign mask.
// EX (exact-order variant): inv_rms from the x86 reference's sum of squares instead
// (dot_f32_fast, real_llm.rs:911-926: four sequential accumulators over elements k, k + 4,
// ..., then (acc0 + acc1) + (acc2 + acc3)), lanes 0-3 of wave 0 running the chains.
template <int NTH, bool EX>
__device__ void build_norm_act(const MkParams &P, const Lds &S, const float *w, const NormPre &wp, uint32_t lane,
                               int wave) {
    // 256 threads: every wave computes inv_rms itself (the same order in each), with no
    // barrier between the sum and the slices (135M +0.8%); 512 threads: wave 0 for the
    // workgroup (eight waves reading the row measured 1.1% slower on the 1.7B model)
    float inv_rms;
    if constexpr (EX) {
        if (wave == 0) {
            float acc = 0.0f;
            if (lane < 4)
                for (int j = 0; j < P.d / 4; j++) {
                    const float v = S.hbuf[4 * j + lane];
                    acc = acc + v * v;
                }
            const float sum = (lane_val(acc, 0) + lane_val(acc, 1)) + (lane_val(acc, 2) + lane_val(acc, 3));
            if (lane == 0) S.vec[0] = 1.0f / sqrtf(sum / (float)P.d + P.eps);
        }
        lds_barrier();
        inv_rms = S.vec[0];
    } else if constexpr (NTH == 256) {
        inv_rms = 1.0f / sqrtf(row_sumsq_wave(S.hbuf, P.d, lane) / (float)P.d + P.eps);
    } else {
        if (wave == 0) {
            const float ss = row_sumsq_wave(S.hbuf, P.d, lane);
            if (lane == 0) S.vec[0] = 1.0f / sqrtf(ss / (float)P.d + P.eps);
        }
        lds_barrier();
        inv_rms = S.vec[0];
    }
    const uint32_t s4 = lane & 15u;
    const int nc = P.d / 64;
    auto slice = [&](int c0, const float4 &wa, uint64_t sign) {
        const int c = c0 + (int)(lane >> 4);
        const bool act = c < nc;
        const int cc = act ? c : 0;
        const float4 x = *reinterpret_cast<const float4 *>(S.hbuf + cc * 64 + s4 * 4);
        float v[4] = {(x.x * inv_rms) * wa.x, (x.y * inv_rms) * wa.y, (x.z * inv_rms) * wa.z, (x.w * inv_rms) * wa.w};
        const Chunk4 r = rotate_quant4(v, sign, s4);
        if (act) {
            *reinterpret_cast<uint32_t *>(S.xl + cc * 64 + s4 * 4) = r.w;
            if (s4 == 0) {
                S.xsl[cc] = r.scale;
                S.xsuml[cc] = r.sum;
            }
        }
    };
    if (wave * 4 < nc) slice(wave * 4, wp.a, wp.sign);
    for (int c0 = wave * 4 + NTH / 64 * 4; c0 < nc; c0 += NTH / 64 * 4) {
        const int c = c0 + (int)(lane >> 4), cc = c < nc ? c : 0;
        slice(c0, *reinterpret_cast<const float4 *>(w + cc * 64 + s4 * 4), P.signs[cc]);
    }
    lds_barrier();
}

// The hidden-vector hand-off and the RMSNorm + FWHT + int8 build of the fast variant, with
// two workgroup barriers instead of four: thread t polls words t, t + NTH, ... (each
// load instruction of a wave reads 512 consecutive bytes), stores them to S.hbuf and adds
// their squares in that order; a butterfly per wave; the waves' sums in wave order after
// one barrier, which also carries the timeout flag (S.flag[1] set to the phase's epoch,
// which no earlier phase had).  The slices (rotate_quant4, four elements per lane) then
// read S.hbuf, and a second barrier ends the build.
template <int NTH>
__device__ __forceinline__ bool load_norm_act(const MkParams &P, const Lds &S, const unsigned long long *src,
                                              uint32_t epoch, const float *w, const NormPre &wp, uint32_t lane,
                                              int wave) {
    constexpr int NW = NTH / 64;
    const int d = P.d, nc = d / 64, t = (int)threadIdx.x;
    bool ok = true;
    float ss = 0.0f;
    for (int i0 = t; i0 < d; i0 += NTH * kPoll) {
        unsigned long long wd[kPoll];
#pragma unroll
        for (int k = 0; k < kPoll; k++) {
            const int i = i0 + k * NTH;
            wd[k] = i < d ? ll_load(src + i) : 0ull;
        }
        uint32_t pending = 0;
#pragma unroll
        for (int k = 0; k < kPoll; k++)
            if (i0 + k * NTH < d && (uint32_t)(wd[k] >> 32) != epoch) pending |= 1u << k;
        for (uint32_t spins = 0; pending != 0 && ok; spins++) {
            if ((spins & 31u) == 31u) {
                if (__hip_atomic_load(P.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) {
                    ok = false;
                    break;
                }
                if (spins > P.spin_limit) {
                    __hip_atomic_store(P.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    ok = false;
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
#pragma unroll
            for (int k = 0; k < kPoll; k++)
                if (pending & (1u << k)) wd[k] = ll_load(src + i0 + k * NTH);
#pragma unroll
            for (int k = 0; k < kPoll; k++)
                if ((pending & (1u << k)) && (uint32_t)(wd[k] >> 32) == epoch) pending &= ~(1u << k);
        }
#pragma unroll
        for (int k = 0; k < kPoll; k++) {
            const int i = i0 + k * NTH;
            if (i < d) {
                const float v = __uint_as_float((uint32_t)wd[k]);
                S.hbuf[i] = v;
                ss = fmaf(v, v, ss);
            }
        }
    }
    ss = wave_sum_f(ss);
    if (lane == 0) S.vec[wave] = ss;
    if (!ok) S.flag[1] = (int)epoch;
    lds_barrier();
    if (S.flag[1] == (int)epoch) return false;
    float tot = S.vec[0];
#pragma unroll
    for (int w2 = 1; w2 < NW; w2++) tot += S.vec[w2];
    const float inv_rms = 1.0f / sqrtf(tot / (float)d + P.eps);
    const uint32_t s4 = lane & 15u;
    auto slice = [&](int c0, const float4 &wa, uint64_t sign) {
        const int c = c0 + (int)(lane >> 4);
        const bool act = c < nc;
        const int cc = act ? c : 0;
        const float4 x = *reinterpret_cast<const float4 *>(S.hbuf + cc * 64 + s4 * 4);
        float v[4] = {(x.x * inv_rms) * wa.x, (x.y * inv_rms) * wa.y, (x.z * inv_rms) * wa.z, (x.w * inv_rms) * wa.w};
        const Chunk4 r = rotate_quant4(v, sign, s4);
        if (act) {
            *reinterpret_cast<uint32_t *>(S.xl + cc * 64 + s4 * 4) = r.w;
            if (s4 == 0) {
                S.xsl[cc] = r.scale;
                S.xsuml[cc] = r.sum;
            }
        }
    };
    if (wave * 4 < nc) slice(wave * 4, wp.a, wp.sign);
    for (int c0 = wave * 4 + NW * 4; c0 < nc; c0 += NW * 4) {
        const int c = c0 + (int)(lane >> 4), cc = c < nc ? c : 0;
        slice(c0, *reinterpret_cast<const float4 *>(w + cc * 64 + s4 * 4), P.signs[cc]);
    }
    lds_barrier();
    return true;
}

// Phase kinds of the step's schedule: per layer kQkv, kAttn, kO, kGu, kDown; then kHead.
enum PhaseKind { kQkv = 0, kAttn = 1, kO = 2, kGu = 3, kDown = 4, kHead = 5 };

// Waits for a GEMV phase's input and builds its int8 activation in LDS: the o_proj /
// down_proj activation chunks as produced, or RMSNorm + FWHT + int8 of the hidden vector
// (HA after the embedding or a down phase, HB after an o phase).
template <int NTH, bool EX>
__device__ __forceinline__ bool mk_load_input(const MkParams &P, const Lds &S, const float *norm_w,
                                              const NormPre &wp, int kind, uint32_t epoch, uint32_t lane, int wave,
                                              int t0, int trace_l = -1) {
    if (kind == kO || kind == kDown) {
        const int nch = kind == kO ? P.nq * P.hd / 64 : P.inter / 64;
        const unsigned long long *src = kind == kO ? P.OACT + my_copy(P) * oact_words(P)
                                                   : P.GACT + my_copy(P) * gact_words(P);
        return load_words<NTH>(P, S, src, nch * kActWords, epoch, true, nullptr, t0);
    }
    const unsigned long long *hsrc = (kind == kGu ? P.HB : P.HA) + my_copy(P) * (size_t)P.d;
    if (!EX) return load_norm_act<NTH>(P, S, hsrc, epoch, norm_w, wp, lane, wave);
    if (!load_words<NTH>(P, S, hsrc, P.d, epoch, false, S.hbuf, t0)) return false;
#ifdef K2T_MK_TRACE_IN
    if (P.trace && threadIdx.x == 0 && trace_l >= 0)
        P.trace[(((size_t)blockIdx.x * (P.L + 1) + trace_l) * 6 + kind) * 6 + 2] = wall_clock64();
#endif
    build_norm_act<NTH, EX>(P, S, norm_w, wp, lane, wave);
    return true;
}

// Row r of the tied lm_head, dequantized in the rotated domain and inverse-rotated
// (embed_token_into, real_llm.rs:8063-8097), chunk c, element `lane`.
__device__ float embed_value(const MatDev &M, int r, int c, uint32_t lane) {
    const int stripe = r / 16, rl = r % 16, g = rl / 4, j = rl % 4;
    const int k = lane / 16, w = lane % 16, half = w / 8, sub = w / 4, t = w % 4;
    const bool in_pair = stripe < 2 * M.np;
    const int side = stripe & 1;
    float val;
    if (M.fmt == 0) {
        const int hp = M.hp;
        const size_t prec = 1024 + 256 * (size_t)hp + 64, trec = 512 + 128 * (size_t)hp + 32;
        const uint8_t *base = in_pair ? M.pair + ((size_t)(stripe / 2) * M.nc + c) * prec : M.tail + (size_t)c * trec;
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
            const int sh = sub == 0 ? 4 : sub == 1 ? 6 : sub == 2 ? 2 : 0;
            const uint8_t hb = h[k * 64 + g * 16 + j * 4 + t];
            u |= ((hb >> sh) & 3) << 4;
        }
        const float delta = __uint_as_float((uint32_t)(sp[rl * 2] | (sp[rl * 2 + 1] << 8)) << 16);
        val = (float)(2 * u - ((1 << (4 + hp)) - 1)) * delta;
    } else {
        const int sg = c / M.sgc, cst = sg * M.sgc, sb = c - cst;
        const uint8_t *gb = in_pair ? M.pair + (size_t)(stripe / 2) * M.ptot + (size_t)sg * 64 + (size_t)cst * 1024
                                    : M.tail + (size_t)sg * 32 + (size_t)cst * 512;
        const uint8_t *sp = gb + (in_pair ? side * 32 : 0);
        const uint8_t *d = gb + (in_pair ? 64 + (size_t)sb * 1024 + side * 512 : 32 + (size_t)sb * 512);
        const int sub4 = w / 4;
        const uint8_t byte = d[k * 128 + g * 32 + (sub4 / 2) * 16 + j * 4 + t];
        const int idx = (sub4 & 1) == 0 ? (byte & 0x0F) : (byte >> 4);
        const int cv = (int)(int8_t)(nf4_xlut((uint32_t)idx, M.cb0, M.cb1, M.cb2, M.cb3) & 0xFFu);
        const float delta = __uint_as_float((uint32_t)(sp[rl * 2] | (sp[rl * 2 + 1] << 8)) << 16);
        val = (float)cv * delta;
    }
    return ifwht_lane(val, (uint64_t)c, lane);
}

// Rotates one head (hd = 64 or 128, one or two blocks held as v0/v1 per lane) and
// quantizes it with one scale (store_hadamard_q8_head, real_llm.rs:8282-8365).
__device__ __forceinline__ float quant_head(float v0, float v1, int nb, uint32_t lane, int8_t *dst,
                                            uint64_t sm0, uint64_t sm1) {
    // fwht_lane with the blocks' sign bits from the sign-mask table
    const float r0 = wave_butterflies64(flip_sign(v0, (uint32_t)(sm0 >> lane) & 1u) * 0.125f, lane);
    const float r1 = nb > 1 ? wave_butterflies64(flip_sign(v1, (uint32_t)(sm1 >> lane) & 1u) * 0.125f, lane) : 0.0f;
    const float mx = wave_max_f(fmaxf(fabsf(r0), fabsf(r1)));
    if (mx <= FLT_EPSILON) {
        dst[lane] = 0;
        if (nb > 1) dst[64 + lane] = 0;
        return 0.0f;
    }
    const float inv = 127.0f / mx;
    dst[lane] = (int8_t)(int)rintf(r0 * inv);
    if (nb > 1) dst[64 + lane] = (int8_t)(int)rintf(r1 * inv);
    return mx / 127.0f;
}

// Attention of q head h for the current position (causal_gqa_group_q8,
// real_llm.rs:8471-8594) over span sp of the context: its seq = pos + 1 positions are cut
// into P.nsp spans (span 0: 60% of two, 34% of four; the others equal).  A task of span
// sp > 0 hands its span's
// maximum score m, sum of exp(s_t - m) and o = sum_t exp(s_t - m) vs_t v8_t over as
// 2 + hd words of APART; the span-0 task merges them with its own (global maximum,
// exp-weighted sums in span order) and ends with the o_proj activation chunks of the
// head.  The task whose span holds the current position builds that position's K / V
// (and, for the first q head of its KV group, stores them in the cache).
#ifdef K2T_MK_TRACE
#define ATR(k)                                                                                      \
    do {                                                                                            \
        if (P.trace && threadIdx.x == 0)                                                           \
            P.trace[(((size_t)blockIdx.x * (P.L + 1) + layer) * 6 + 1) * 6 + (k)] = wall_clock64(); \
    } while (0)
// second row of attention stamps (the phase-5 slot, unused below the head layer)
#define ATR2(k)                                                                                     \
    do {                                                                                            \
        if (P.trace && threadIdx.x == 0)                                                           \
            P.trace[(((size_t)blockIdx.x * (P.L + 1) + layer) * 6 + 5) * 6 + (k)] = wall_clock64(); \
    } while (0)
#else
#define ATR(k) \
    do {       \
    } while (0)
#define ATR2(k) \
    do {        \
    } while (0)
#endif

template <int NTH>
__device__ bool attention_head(const MkParams &P, const float *bias, const Lds &S, int layer, int h, int sp, int pos,
                               uint32_t ep_in, uint32_t ep_out, uint32_t lane, int wave) {
    const int hd = P.hd, nb = hd / 64, nq = P.nq, nkv = P.nkv;
    const int group = nq / nkv, kvh = h / group;
    float *qf = S.att, *kf = qf + hd, *vf = kf + hd;
    int8_t *qi = reinterpret_cast<int8_t *>(vf + hd);
    int8_t *kn = qi + 128, *vn = kn + 128;
    float *scal = reinterpret_cast<float *>(vn + 128);  // qas, ks_new, vs_new, m, 1/L
    float *red = scal + 8;                              // [32]
    float *opart = red + 32;                            // [16 waves][hd]
    float *sc = opart + kMaxThreads * 4;                // [min(max_seq, kMkMaxContext)]
    const int t = (int)threadIdx.x;
    const int seq = pos + 1;
    // spans of this step: at least kMkSpanMin positions each, at most the P.nsp allotted
    const int nsp = min(P.nsp, max(1, (seq + kMkSpanMin - 1) / kMkSpanMin));
    if (sp >= nsp) return true;
    // Span 0, which also merges, takes a larger share: 60% of two spans, 34% of four (its
    // merge then starts about when the other spans' words arrive; the rest is split
    // evenly).  1.7B nf4g128 (two spans) 1447 -> 1452 tok/s against halves; 135M p55454
    // (four spans) 1567 -> 1574 against quarters (40%: 1564, 46%: 1534).
#ifndef K2T_MK_SPAN0_4
#define K2T_MK_SPAN0_4 34
#endif
    const int pct0 = nsp == 2 ? 60 : nsp == 4 ? K2T_MK_SPAN0_4 : 100 / nsp;
    const int len0 = nsp == 1 ? seq : (seq * pct0 + 99) / 100;
    const int lenr = nsp == 1 ? 0 : (seq - len0 + nsp - 2) / (nsp - 1);
    const int t0 = min(seq, sp == 0 ? 0 : len0 + (sp - 1) * lenr);
    const int t1 = min(seq, sp == 0 ? len0 : t0 + lenr), n = t1 - t0;
    const bool cover = t0 <= pos && pos < t1;
    const size_t base = ((size_t)layer * nkv + kvh) * P.max_seq;
    const int ncg = hd / 4, nps = NTH / ncg;
    const int cg = t % ncg, ps = t / ncg;
    // 0. past positions' K rows, scales and V slices do not depend on this step: request
    //    this thread's first ones before waiting for q / k / v.
    // (256 threads: 12 covers the 135M model's spans at the bench contexts, 512 positions
    // and more over 4 spans, and measured 1.7% faster than 8 there; 16 was slower than 12.
    // 512 threads: 8; 12 or 16 measured no faster on the 1.7B model)
    constexpr int kVPre = NTH == 256 ? 12 : 8;
    uint4 kpre[8];
    float kspre = 0.0f, vspre = 0.0f;
    if (t0 + t < t1 && t0 + t < pos) {
        const uint4 *kr = reinterpret_cast<const uint4 *>(P.kq + (base + t0 + t) * hd);
#pragma unroll
        for (int i = 0; i < 8; i++)
            if (i < hd / 16) kpre[i] = kr[i];
        kspre = P.ks[base + t0 + t];
        vspre = P.vs[base + t0 + t];
    }
    int vpre[kVPre];
#pragma unroll
    for (int i = 0; i < kVPre; i++) {
        const int tt = t0 + ps + i * nps;
        vpre[i] = tt < t1 && tt < pos ? *reinterpret_cast<const int *>(P.vq + (base + tt) * hd + cg * 4) : 0;
    }
    // RoPE row of this position (waves 0 and 1 rotate q and k): requested before the wait
    float rc = 0.0f, rsn = 0.0f;
    if (wave < 2) {
        const float *rrow = P.rope + (size_t)pos * hd;
        const uint32_t ri = nb == 1 ? (lane & 31u) : lane;
        rc = rrow[ri];
        rsn = rrow[(nb == 1 ? 32u : 64u) + ri];
    }
    // 1. this position's q (and k, v where the span holds it) (+ bias)
    bool ok = true;
    // (up to 3 * 128 words: more than the 256-thread kernel's threads at hd 128)
    for (int e = t; e < (cover ? 3 : 1) * hd && ok; e += NTH) {
        const int part = e / hd, i = e % hd;
        const int row = part == 0 ? h * hd + i : part == 1 ? (nq + kvh) * hd + i : (nq + nkv + kvh) * hd + i;
        uint32_t v = 0;
        ok = ll_wait(P, P.QKV + row, ep_in, v);
        float f = __uint_as_float(v);
        if (bias) f = f + bias[row];
        qf[e] = f;  // qf, kf, vf are contiguous
    }
    if (!ok) S.flag[1] = (int)ep_in;
    lds_barrier();
    ATR(1);
    if (S.flag[1] == (int)ep_in) return false;
    // 2. RoPE (real_llm.rs:9328-9361) on q and k, int8 Hadamard q / k / v
    const size_t slot = base + pos;
    // waves 0, 1, 2 handle q, k, v concurrently
    if (wave == 0 || (cover && wave == 1)) {
        const float *src = wave == 0 ? qf : kf;
        float x0 = src[lane], x1 = nb > 1 ? src[64 + lane] : 0.0f;
        if (nb == 1) {
            const float c = rc, sn = rsn;
            const float xo = __shfl_xor(x0, 32, kWave);
            x0 = lane < 32 ? x0 * c - xo * sn : x0 * c + xo * sn;
        } else {
            const float c = rc, sn = rsn;
            const float a0 = x0, a1 = x1;
            x0 = a0 * c - a1 * sn;
            x1 = a1 * c + a0 * sn;
        }
        int8_t *dst = wave == 0 ? qi : kn;
        const float sc8 = quant_head(x0, x1, nb, lane, dst, sign_mask_s(P, 0), sign_mask_s(P, 1));
        if (lane == 0) scal[wave] = wave == 0 ? sc8 * P.attn_scale : sc8;
        if (wave == 1 && h % group == 0) {  // the first q head of the group stores this position's K
            P.kq[slot * hd + lane] = kn[lane];
            if (nb > 1) P.kq[slot * hd + 64 + lane] = kn[64 + lane];
            if (lane == 0) P.ks[slot] = sc8;
        }
    } else if (cover && wave == 2) {
        const float vsn = quant_head(vf[lane], nb > 1 ? vf[64 + lane] : 0.0f, nb, lane, vn, sign_mask_s(P, 0),
                                     sign_mask_s(P, 1));
        if (lane == 0) scal[2] = vsn;
        if (h % group == 0) {
            P.vq[slot * hd + lane] = vn[lane];
            if (nb > 1) P.vq[slot * hd + 64 + lane] = vn[64 + lane];
            if (lane == 0) P.vs[slot] = vsn;
        }
    }
    lds_barrier();
    ATR(2);
    // The thread whose first position is the current one takes its K row from LDS into the
    // prefetch registers (one wait for the row, not one per piece as below).
    if (t0 + t == pos) {
#pragma unroll
        for (int i = 0; i < 8; i++)
            if (i < hd / 16) kpre[i] = ld_lds(reinterpret_cast<const uint4 *>(kn) + i);
        kspre = ld_lds(scal + 1);
    }
    // 3. scores s_t = float(q8 . k8_t) * ks_t * (qs * scale), t0 <= t < t1
    const float qas = scal[0];
    float smax = -INFINITY;
    for (int tt = t0 + t; tt < t1; tt += NTH) {
        const uint4 *qr = reinterpret_cast<const uint4 *>(qi);
        int dot = 0;
        float kscale;
        if (tt == t0 + t && tt <= pos) {  // prefetched (or, for the current position, copied)
#pragma unroll
            for (int i = 0; i < 8; i++) {
                if (i >= hd / 16) break;
                const uint4 a = kpre[i], b = qr[i];
                dot = __builtin_amdgcn_sdot4((int)a.x, (int)b.x, dot, false);
                dot = __builtin_amdgcn_sdot4((int)a.y, (int)b.y, dot, false);
                dot = __builtin_amdgcn_sdot4((int)a.z, (int)b.z, dot, false);
                dot = __builtin_amdgcn_sdot4((int)a.w, (int)b.w, dot, false);
            }
            kscale = kspre;
        } else {
            // (the current position here only past a thread's first position: spans longer
            // than NTH positions)
            const uint4 *kr = reinterpret_cast<const uint4 *>(P.kq + (base + tt) * hd);
            for (int i = 0; i < hd / 16; i++) {
                const uint4 a = tt == pos ? lds_read16_now(kn + 16 * i) : ld_global(kr + i);
                const uint4 b = qr[i];
                dot = __builtin_amdgcn_sdot4((int)a.x, (int)b.x, dot, false);
                dot = __builtin_amdgcn_sdot4((int)a.y, (int)b.y, dot, false);
                dot = __builtin_amdgcn_sdot4((int)a.z, (int)b.z, dot, false);
                dot = __builtin_amdgcn_sdot4((int)a.w, (int)b.w, dot, false);
            }
            kscale = tt == pos ? ld_lds(scal + 1) : ld_global(P.ks + base + tt);
        }
        const float s = ((float)dot * kscale) * qas;
        sc[tt - t0] = s;
        smax = fmaxf(smax, s);
    }
    smax = wave_max_f(smax);
    if (lane == 0) red[wave] = smax;
    lds_barrier();
    float m = red[0];
    for (int w2 = 1; w2 < (NTH / 64); w2++) m = fmaxf(m, red[w2]);
    lds_barrier();
    ATR(3);
    float psum = 0.0f;
    for (int tt = t0 + t; tt < t1; tt += NTH) {
        const float p = expf(sc[tt - t0] - m);
        const float vsc = tt == pos ? scal[2] : (tt == t0 + t ? vspre : P.vs[base + tt]);
        sc[tt - t0] = p * vsc;  // p_t * vs_t
        psum += p;
    }
    psum = wave_sum_f(psum);
    if (lane == 0) red[16 + wave] = psum;
    lds_barrier();
    // 4. o = sum_t p_t vs_t v_t: thread = (position subset, 4-column group); the subsets
    //    of one wave are added with lane shuffles, then the waves' sums in wave order.
    float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
    auto vacc = [&](int v, float wt) {
        a0 = fmaf(wt, (float)(int8_t)(v & 0xFF), a0);
        a1 = fmaf(wt, (float)(int8_t)((v >> 8) & 0xFF), a1);
        a2 = fmaf(wt, (float)(int8_t)((v >> 16) & 0xFF), a2);
        a3 = fmaf(wt, (float)(int8_t)((v >> 24) & 0xFF), a3);
    };
#pragma unroll
    for (int i = 0; i < kVPre; i++) {  // prefetched slices, positions in ascending order
        const int tt = t0 + ps + i * nps;
        if (tt < t1) vacc(tt == pos ? *reinterpret_cast<const int *>(vn + cg * 4) : vpre[i], sc[tt - t0]);
    }
    // the rest in batches of kVB positions: all of a batch's loads are in flight before
    // its first use (same positions, same order of accumulation)
    constexpr int kVB = NTH == 256 ? 8 : 1;  // 512 threads: 2 measured no faster on the 1.7B model
    for (int tb = t0 + ps + kVPre * nps; tb < t1; tb += kVB * nps) {
        int vb[kVB];
#pragma unroll
        for (int u = 0; u < kVB; u++) {
            const int tt = tb + u * nps;
            vb[u] = tt < pos ? ld_global(reinterpret_cast<const int *>(P.vq + (base + tt) * hd + cg * 4))
                             : ld_lds(reinterpret_cast<const int *>(vn + cg * 4));
        }
#pragma unroll
        for (int u = 0; u < kVB; u++) {
            const int tt = tb + u * nps;
            if (tt < t1) vacc(vb[u], sc[tt - t0]);
        }
    }
    for (int m2 = ncg; m2 < 64; m2 <<= 1) {  // lanes l and l ^ m2 hold the same columns
        a0 += __shfl_xor(a0, m2, kWave);
        a1 += __shfl_xor(a1, m2, kWave);
        a2 += __shfl_xor(a2, m2, kWave);
        a3 += __shfl_xor(a3, m2, kWave);
    }
    if ((int)lane < ncg) {
        opart[wave * hd + cg * 4 + 0] = a0;
        opart[wave * hd + cg * 4 + 1] = a1;
        opart[wave * hd + cg * 4 + 2] = a2;
        opart[wave * hd + cg * 4 + 3] = a3;
    }
    lds_barrier();
    ATR(4);
    bool merged = true;
    if (t < hd) {
        float acc = opart[t];
        for (int w2 = 1; w2 < (NTH / 64); w2++) acc += opart[w2 * hd + t];
        float L = red[16];
        for (int w2 = 1; w2 < (NTH / 64); w2++) L += red[16 + w2];
        const float mm = n > 0 ? m : -INFINITY;
        if (n == 0) L = 0.0f;
        if (sp > 0) {  // hand the span over (an empty span: m = -inf, L = 0, o = 0)
            unsigned long long *dst = P.APART + ((size_t)h * P.nsp + sp) * (2 + hd);
            ll_store(dst + 2 + t, __float_as_uint(acc), ep_out);
            if (t == 0) {
                ll_store(dst, __float_as_uint(mm), ep_out);
                ll_store(dst + 1, __float_as_uint(L), ep_out);
            }
#ifdef K2T_MK_SWAIT
            wait_vmcnt<0>();
            ATR2(0);
#endif
        } else {
            // merge the other spans' {m, L, o[t]}: all loads in flight, then re-polled
            // together until current (attn_merge_kernel's arithmetic, span order)
            constexpr int kSp = mk_max_spans(NTH);
            unsigned long long w[3 * (kSp - 1)];
            const unsigned long long *src = P.APART + (size_t)h * P.nsp * (2 + hd);
            auto addr = [&](int k) { return src + (size_t)(k / 3 + 1) * (2 + hd) + (k % 3 == 2 ? 2 + t : k % 3); };
            // Every word is requested, the unused spans' too (in bounds: APART holds
            // kMkSpans slots per head): with the load under a branch the compiler waited
            // for each load before issuing the next (the other path's zero reuses its
            // register).
            uint32_t pending = 0;
#pragma unroll
            for (int k = 0; k < 3 * (kSp - 1); k++) w[k] = ll_load(addr(k));
#pragma unroll
            for (int k = 0; k < 3 * (kSp - 1); k++)
                if (k / 3 + 1 < nsp && (uint32_t)(w[k] >> 32) != ep_out) pending |= 1u << k;
            for (uint32_t spins = 0; pending != 0 && merged; spins++) {
                if ((spins & 31u) == 31u) {
                    if (__hip_atomic_load(P.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) {
                        merged = false;
                        break;
                    }
                    if (spins > P.spin_limit) {
                        __hip_atomic_store(P.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        merged = false;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                }
#pragma unroll
                for (int k = 0; k < 3 * (kSp - 1); k++)
                    if (pending & (1u << k)) w[k] = ll_load(addr(k));
#pragma unroll
                for (int k = 0; k < 3 * (kSp - 1); k++)
                    if ((pending & (1u << k)) && (uint32_t)(w[k] >> 32) == ep_out) pending &= ~(1u << k);
            }
            ATR2(1);
            float M = mm;
#pragma unroll
            for (int s2 = 1; s2 < kSp; s2++)
                if (s2 < nsp) M = fmaxf(M, __uint_as_float((uint32_t)w[3 * (s2 - 1)]));
            const float e0 = expf(mm - M);
            float Lt = fmaf(L, e0, 0.0f), o = fmaf(acc, e0, 0.0f);
#pragma unroll
            for (int s2 = 1; s2 < kSp; s2++) {
                if (s2 < nsp) {
                    const float e = expf(__uint_as_float((uint32_t)w[3 * (s2 - 1)]) - M);
                    Lt = fmaf(__uint_as_float((uint32_t)w[3 * (s2 - 1) + 1]), e, Lt);
                    o = fmaf(__uint_as_float((uint32_t)w[3 * (s2 - 1) + 2]), e, o);
                }
            }
            qf[t] = o * (1.0f / Lt);  // reuse qf for o
        }
    }
    if (!merged) S.flag[1] = (int)ep_out;
    lds_barrier();
    if (S.flag[1] == (int)ep_out) return false;
    if (sp > 0) return true;  // (the scratch reads are done: the barriers above)
    ATR2(2);
    // 5. ifwht64 per block, then FWHT with the o_proj chunk index + int8 (real_llm.rs:7060-7084)
    //    Four elements per lane (slice s = lane % 16; every 16-lane group holds the block):
    //    two in-register butterfly stages and four lane exchanges per transform.
    if (wave < nb) {
        const uint32_t s4 = lane & 15u;
        const float4 o4 = *reinterpret_cast<const float4 *>(qf + wave * 64 + s4 * 4);
        float v[4] = {o4.x, o4.y, o4.z, o4.w};
        butterflies_slice4(v, s4);  // inverse: butterflies, then x0.125 and the block's signs
        const uint32_t ib = (uint32_t)(sign_mask_s(P, wave) >> (4u * s4)) & 0xFu;
#pragma unroll
        for (int j = 0; j < 4; j++) v[j] = flip_sign(v[j] * 0.125f, (ib >> j) & 1u);
        const int c = h * nb + wave;
        const Chunk4 r = rotate_quant4(v, sign_mask_s(P, c), s4);
        store_act_chunk4(r, lane, P.OACT + (size_t)c * kActWords, ep_out, P.rep, oact_words(P));
    }
    ATR2(3);
    // the next GEMV task stages weights into the LDS bytes that hold qf: every wave must
    // be past its last read of the attention scratch first
    lds_barrier();
    return true;
}

// Attention of q head h in the x86 reference's operation order (exact-order variant; one
// task per head): causal_gqa_group_q8's portable branches (real_llm.rs:8533-8545,
// 8575-8585) and softmax_unnorm_inplace (9590-9600).  Scores one position per thread,
// s_t = (float(q8 . k8_t) * ks_t) * qas; p_t = exp(s_t - max) with the x86 build's exp
// (expf_rn); sum = p_0 + p_1 + ... in position order (thread 0), inv = 1/sum; then thread
// d accumulates o[d] += ((p_t * inv) * vs_t) * float(v8_t[d]) for t ascending (eight
// positions' loads in flight); IFWHT, FWHT with the o_proj chunk index, int8.  The
// position's own K / V come from LDS, as in attention_head, and are stored by the first q
// head of each KV group.
template <int NTH>
__device__ bool attention_head_ex(const MkParams &P, const float *bias, const Lds &S, int layer, int h, int pos,
                                  uint32_t ep_in, uint32_t ep_out, uint32_t lane, int wave) {
    const int hd = P.hd, nb = hd / 64, nq = P.nq, nkv = P.nkv;
    const int group = nq / nkv, kvh = h / group;
    float *qf = S.att, *kf = qf + hd, *vf = kf + hd;
    int8_t *qi = reinterpret_cast<int8_t *>(vf + hd);
    int8_t *kn = qi + 128, *vn = kn + 128;
    float *scal = reinterpret_cast<float *>(vn + 128);  // qas, ks_new, vs_new, inv
    float *red = scal + 8;                              // [32]
    float *sc = red + 32 + kMaxThreads * 4;             // [min(max_seq, kMkMaxContext)]
    const int t = (int)threadIdx.x;
    const int seq = pos + 1;
    const size_t base = ((size_t)layer * nkv + kvh) * P.max_seq;
    float rc = 0.0f, rsn = 0.0f;
    if (wave < 2) {
        const float *rrow = P.rope + (size_t)pos * hd;
        const uint32_t ri = nb == 1 ? (lane & 31u) : lane;
        rc = rrow[ri];
        rsn = rrow[(nb == 1 ? 32u : 64u) + ri];
    }
    bool ok = true;
    for (int e = t; e < 3 * hd && ok; e += NTH) {
        const int part = e / hd, i = e % hd;
        const int row = part == 0 ? h * hd + i : part == 1 ? (nq + kvh) * hd + i : (nq + nkv + kvh) * hd + i;
        uint32_t v = 0;
        ok = ll_wait(P, P.QKV + row, ep_in, v);
        float f = __uint_as_float(v);
        if (bias) f = f + bias[row];
        qf[e] = f;
    }
    if (t == 0) S.flag[0] = 0;
    lds_barrier();
    if (!ok) S.flag[0] = 1;
    lds_barrier();
    if (S.flag[0]) return false;
    const size_t slot = base + pos;
    if (wave == 0 || wave == 1) {
        const float *src = wave == 0 ? qf : kf;
        float x0 = src[lane], x1 = nb > 1 ? src[64 + lane] : 0.0f;
        if (nb == 1) {
            const float xo = __shfl_xor(x0, 32, kWave);
            x0 = lane < 32 ? x0 * rc - xo * rsn : x0 * rc + xo * rsn;
        } else {
            const float a0 = x0, a1 = x1;
            x0 = a0 * rc - a1 * rsn;
            x1 = a1 * rc + a0 * rsn;
        }
        int8_t *dst = wave == 0 ? qi : kn;
        const float sc8 = quant_head(x0, x1, nb, lane, dst, sign_mask_s(P, 0), sign_mask_s(P, 1));
        if (lane == 0) scal[wave] = wave == 0 ? sc8 * P.attn_scale : sc8;
        if (wave == 1 && h % group == 0) {
            P.kq[slot * hd + lane] = kn[lane];
            if (nb > 1) P.kq[slot * hd + 64 + lane] = kn[64 + lane];
            if (lane == 0) P.ks[slot] = sc8;
        }
    } else if (wave == 2) {
        const float vsn = quant_head(vf[lane], nb > 1 ? vf[64 + lane] : 0.0f, nb, lane, vn, sign_mask_s(P, 0),
                                     sign_mask_s(P, 1));
        if (lane == 0) scal[2] = vsn;
        if (h % group == 0) {
            P.vq[slot * hd + lane] = vn[lane];
            if (nb > 1) P.vq[slot * hd + 64 + lane] = vn[64 + lane];
            if (lane == 0) P.vs[slot] = vsn;
        }
    }
    lds_barrier();
    const float qas = scal[0];
    float smax = -INFINITY;
    for (int tt = t; tt < seq; tt += NTH) {
        int dot = 0;
        float kscale;
        const uint4 *qr = reinterpret_cast<const uint4 *>(qi);
        if (tt == pos) {
            for (int i = 0; i < hd / 16; i++) {
                const uint4 a = lds_read16_now(kn + 16 * i), b = qr[i];
                dot = __builtin_amdgcn_sdot4((int)a.x, (int)b.x, dot, false);
                dot = __builtin_amdgcn_sdot4((int)a.y, (int)b.y, dot, false);
                dot = __builtin_amdgcn_sdot4((int)a.z, (int)b.z, dot, false);
                dot = __builtin_amdgcn_sdot4((int)a.w, (int)b.w, dot, false);
            }
            kscale = ld_lds(scal + 1);
        } else {
            const uint4 *kr = reinterpret_cast<const uint4 *>(P.kq + (base + tt) * hd);
            for (int i = 0; i < hd / 16; i++) {
                const uint4 a = ld_global(kr + i), b = qr[i];
                dot = __builtin_amdgcn_sdot4((int)a.x, (int)b.x, dot, false);
                dot = __builtin_amdgcn_sdot4((int)a.y, (int)b.y, dot, false);
                dot = __builtin_amdgcn_sdot4((int)a.z, (int)b.z, dot, false);
                dot = __builtin_amdgcn_sdot4((int)a.w, (int)b.w, dot, false);
            }
            kscale = ld_global(P.ks + base + tt);
        }
        const float sv = ((float)dot * kscale) * qas;
        sc[tt] = sv;
        smax = fmaxf(smax, sv);
    }
    smax = wave_max_f(smax);
    if (lane == 0) red[wave] = smax;
    lds_barrier();
    float m = red[0];
    for (int w2 = 1; w2 < (NTH / 64); w2++) m = fmaxf(m, red[w2]);
    for (int tt = t; tt < seq; tt += NTH) sc[tt] = expf_rn(sc[tt] - m);
    lds_barrier();
    if (t == 0) {
        float sum = 0.0f;
        for (int tt = 0; tt < seq; tt++) sum = sum + sc[tt];
        scal[3] = 1.0f / sum;
    }
    lds_barrier();
    if (t < hd) {
        const float inv = scal[3];
        float o = 0.0f;
        for (int tb = 0; tb < seq; tb += 8) {
            float vsb[8];
            int vb[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int tt = min(tb + u, seq - 1);
                if (tt == pos) {
                    vsb[u] = ld_lds(scal + 2);
                    vb[u] = (int)ld_lds(vn + t);
                } else {
                    vsb[u] = ld_global(P.vs + base + tt);
                    vb[u] = (int)ld_global(P.vq + (base + tt) * hd + t);
                }
            }
#pragma unroll
            for (int u = 0; u < 8; u++)
                if (tb + u < seq) o = o + ((sc[tb + u] * inv) * vsb[u]) * (float)vb[u];
        }
        qf[t] = o;
    }
    lds_barrier();
    if (wave < nb) {
        const uint32_t s4 = lane & 15u;
        const float4 o4 = *reinterpret_cast<const float4 *>(qf + wave * 64 + s4 * 4);
        float v[4] = {o4.x, o4.y, o4.z, o4.w};
        butterflies_slice4(v, s4);
        const uint32_t ib = (uint32_t)(sign_mask_s(P, wave) >> (4u * s4)) & 0xFu;
#pragma unroll
        for (int j = 0; j < 4; j++) v[j] = flip_sign(v[j] * 0.125f, (ib >> j) & 1u);
        const int c = h * nb + wave;
        const Chunk4 r = rotate_quant4(v, sign_mask_s(P, c), s4);
        store_act_chunk4(r, lane, P.OACT + (size_t)c * kActWords, ep_out, P.rep, oact_words(P));
    }
    lds_barrier();
    return true;
}

// Stripe-mode task order with both stripes of a pair on one XCD: with one stripe per
// workgroup, tasks t and t + 8 run on workgroups 8 apart (the same XCD), so the L2 lines
// shared by the two halves of a record are fetched from HBM once.
template <int NW>
__device__ __forceinline__ int xcd_stripe(const MatDev &M, int t, int nblocks) {
    // (with two or more stripes per workgroup, consecutive tasks already pair up)
    if (!M.smode || M.nseg != NW || (nblocks & 15) != 0 || t >= nblocks) return t;
    const int a = t >> 4, s8 = (t >> 3) & 1, j = t & 7;
    return 2 * (8 * a + j) + s8;
}

#ifdef K2T_MK_TRACE
// [workgroup][layer (L = head)][phase][start, input, first fragment, wave 0 done, computed, end]:
// 100 MHz wall clock
#define MK_TR(l, ph, k)                                                                              \
    do {                                                                                             \
        if (P.trace && threadIdx.x == 0)                                                             \
            P.trace[(((size_t)blockIdx.x * (P.L + 1) + (l)) * 6 + (ph)) * 6 + (k)] = wall_clock64(); \
    } while (0)
#else
#define MK_TR(l, ph, k) \
    do {                \
    } while (0)
#endif

// FMT/HP: the one weight format every projection and the head use (mixed-format models
// run the one-kernel-per-operation path).
// EX: the exact-order variant (x86 reference operation order: in-order GEMV epilogue
// chains, sequential sums of squares, expf_rn, one attention task per head with sequential
// softmax and V sums).
template <int FMT, int HP, int NTH, bool EX>
__global__ __launch_bounds__(NTH) void decode_mk_kernel(MkParams P) {
    constexpr int kThreads = NTH;
    constexpr int kWaves = NTH / 64;
    extern __shared__ float lds_raw[];
    const Lds S = carve(P, lds_raw);
    const uint32_t lane = threadIdx.x & 63u;
    const int wave = (int)(threadIdx.x >> 6);
    const int t = (int)threadIdx.x;
    const uint32_t step = *P.step_dev;
    const int pos = *P.pos_dev;
    const uint32_t nph = 2u + 5u * (uint32_t)P.L;
    auto E = [&](int ph) { return step * nph + (uint32_t)ph + 1u; };
    const int d = P.d;
    if (t == 0) S.flag[1] = 0;  // (the waits' timeout flag holds a phase epoch; none is 0)
    // The layer table is read-only for the launch: scalar loads through the constant
    // address space (the four matrix views of a layer are consecutive).
    using CMkLayer = const __attribute__((address_space(4))) MkLayer;
    CMkLayer *LT = (CMkLayer *)P.layers;
    static_assert(offsetof(MkLayer, o) == offsetof(MkLayer, qkv) + sizeof(MatDev) &&
                      offsetof(MkLayer, gu) == offsetof(MkLayer, o) + sizeof(MatDev) &&
                      offsetof(MkLayer, down) == offsetof(MkLayer, gu) + sizeof(MatDev),
                  "MkLayer matrix views must be consecutive");

    // phase 0: embedding -> HA (one wave per 64-element chunk)
    {
        const int token = P.tokens[0];
        for (int c = (int)blockIdx.x * kWaves + wave; c < d / 64; c += (int)gridDim.x * kWaves)
        {
            float v;
            if (P.ekind == K2T_EMBED_F32) {
                v = ((const float *)P.erows)[(size_t)token * d + c * 64 + lane];
            } else if (P.ekind == K2T_EMBED_BF16) {
                v = __uint_as_float((uint32_t)((const uint16_t *)P.erows)[(size_t)token * d + c * 64 + lane] << 16);
            } else {
                v = embed_value(P.embed, token, c, lane);
            }
            for (int r = 0; r < P.rep; r++) ll_store(P.HA + (size_t)r * d + c * 64 + lane, __float_as_uint(v), E(0));
        }
    }
    // phases 1 .. 5L+1: a single GEMV body serves every matrix
    for (int ph = 1; ph < (int)nph; ph++) {
        const int l = (ph - 1) / 5;
        const int kind = ph == (int)nph - 1 ? kHead : (ph - 1) % 5;
        // Each phase's task list starts where the previous phase's ended (MkLayer::off): a
        // workgroup idle in one phase is already streaming its next phase's weights, and
        // no phase's input polls queue behind weight loads that a workgroup issued on
        // finishing the previous phase.
        const int nwg = (int)gridDim.x;
        const int off = kind == kHead ? P.head_off : LT[l].off[kind];
        const int vb = ((int)blockIdx.x + nwg - off) % nwg;  // this workgroup's rank in the phase
        if (kind == kAttn) {
            // task j = (span j / nq, head j % nq): the span-0 tasks (which merge) come first
            const int ntask = P.nq * P.nsp;
            if (vb < ntask) MK_TR(l, 1, 0);
            for (int j = vb; j < ntask; j += nwg) {
                if constexpr (EX) {
                    if (!attention_head_ex<NTH>(P, LT[l].bias, S, l, j, pos, E(ph - 1), E(ph), lane, wave)) return;
                } else {
                    if (!attention_head<NTH>(P, LT[l].bias, S, l, j % P.nq, j / P.nq, pos, E(ph - 1), E(ph), lane,
                                             wave))
                        return;
                }
            }
            if (vb < ntask) MK_TR(l, 1, 5);
            continue;
        }
        // the matrix view in registers, read by scalar loads (a vector load here would wait
        // for the previous phase's hand-off stores to complete: loads return in order)
        const int li = kind == kHead ? 0 : l;
        MatDev Mv = P.head;
        if (kind != kHead) Mv = *(const MatDev *)(&LT[li].qkv + (kind == kQkv ? 0 : kind - 1));
        const MatDev &M = Mv;
        const float *norm_w = kind == kQkv ? LT[li].in_norm : kind == kGu ? LT[li].post_norm : P.final_norm;
        const int nblocks = M.smode ? M.stripes : M.np + (M.stripes & 1);
        const int groups = kWaves / M.nseg;
        if (vb * groups >= nblocks) continue;  // no task here: go on to the next phase
        const NormPre wpre = norm_prefetch<NTH>(P, kind == kO || kind == kDown ? nullptr : norm_w, lane, wave);
        MK_TR(kind == kHead ? P.L : l, kind == kHead ? 0 : kind, 0);
        // ---- GEMV rounds
        const int grp = wave / M.nseg, wseg = wave % M.nseg;
        const int RB = M.smode ? 16 : 32;
        bool ok = true;
        // the output row of thread t in the epilogue of the round at `base` (-1: none)
        auto out_row = [&](int base) {
            if (t >= groups * RB) return -1;
            const int g2 = t / RB, rl = t % RB, rb2 = xcd_stripe<kWaves>(M, base + g2, nblocks);
            if (rb2 >= nblocks) return -1;
            const bool tail = !M.smode && rb2 >= M.np;
            const int first_stripe = M.smode ? rb2 : (tail ? 2 * M.np : 2 * rb2);
            const int row = first_stripe * 16 + rl;
            return rl < (tail ? 16 : RB) && row < M.rows ? row : -1;
        };
        // residual of the o / down epilogue: HB = HA + o (HA from phase ph-3), HA = HB + down
        // (HB from ph-2)
        const unsigned long long *res = (kind == kO ? P.HA : P.HB) + my_copy(P) * (size_t)d;
        const uint32_t er = kind == kO ? E(ph - 3) : E(ph - 2);
        for (int base = vb * groups; base < nblocks; base += nwg * groups) {
            const int rb = xcd_stripe<kWaves>(M, base + grp, nblocks);
            const bool first = base == vb * groups;
            const int orow = out_row(base);
            unsigned long long rpre = 0;
            // The whole of this wave's share (up to kMkFrags fragments) streams into its
            // LDS slots before the input wait; the compute then reads LDS only.
            {
                uint8_t *slots = S.ring + (size_t)wave * kMkFrags * frag_lds_bytes<FMT, HP>();
                GemvWaveLds<FMT, HP, kMkFrags> gw(M, rb, rb < nblocks, wseg, lane, slots);
                gw.start();
                if (first) {
                    if (!mk_load_input<NTH, EX>(P, S, norm_w, wpre, kind, E(ph - 1), lane, wave, 0,
                                            kind == kHead ? -1 : l))
                        return;
                    MK_TR(kind == kHead ? P.L : l, kind == kHead ? 0 : kind, 1);
                }
                // The residual word was written phases ago (the input's producers waited
                // for it): request it now, so it lands during the compute.  The compute
                // reads only LDS (no flat accesses), so nothing waits for this load early.
                if ((kind == kO || kind == kDown) && orow >= 0) rpre = ll_load(res + orow);
                // exact-order variant: this wave's group stages its rows' epilogue operands
                unsigned long long *terms =
                    EX ? P.exterm + (size_t)blockIdx.x * kMkTermRows * M.nc + (size_t)grp * RB * M.nc : nullptr;
#ifdef K2T_MK_TRACE
                unsigned long long *tr = first && P.trace
                    ? P.trace + (((size_t)blockIdx.x * (P.L + 1) + (kind == kHead ? P.L : l)) * 6 + (kind == kHead ? 0 : kind)) * 6
                    : nullptr;
#ifdef K2T_MK_TRACE_IN
                tr = nullptr;
#endif
                gw.finish(slots, S.xl, S.xsl, S.xsuml, S.part + wave * 32, tr, terms);
#else
                gw.finish(slots, S.xl, S.xsl, S.xsuml, S.part + wave * 32, nullptr, terms);
#endif
            }
            if constexpr (EX) {
                // the staged operands must be at the coherence point before other waves read them
                __threadfence();
                __syncthreads();
            }
            lds_barrier();
            if (first) MK_TR(kind == kHead ? P.L : l, kind == kHead ? 0 : kind, 4);
            if (orow >= 0) {
                const int g2 = t / RB, rl = t % RB, row = orow;
                float acc = 0.0f;
                if constexpr (EX) {
                    // the reference's per-row chain f = fmaf(term_c, scale_c, f), c ascending
                    // (simd_lut.rs:4030-4059, 6334-6335), sixteen operand words in flight
                    const unsigned long long *tw =
                        P.exterm + (size_t)blockIdx.x * kMkTermRows * M.nc + ((size_t)g2 * RB + rl) * M.nc;
                    for (int c0 = 0; c0 < M.nc; c0 += 16) {
                        unsigned long long wv[16];
#pragma unroll
                        for (int u = 0; u < 16; u++) wv[u] = ll_load(tw + min(c0 + u, M.nc - 1));
#pragma unroll
                        for (int u = 0; u < 16; u++)
                            if (c0 + u < M.nc)
                                acc = fmaf(__uint_as_float((uint32_t)wv[u]), __uint_as_float((uint32_t)(wv[u] >> 32)),
                                           acc);
                    }
                } else {
                    const float *gp = S.part + (g2 * M.nseg) * 32;
                    acc = gp[rl];
                    for (int w2 = 1; w2 < M.nseg; w2++) acc += gp[w2 * 32 + rl];
                }
                if (kind == kHead) {
                    P.logits[row] = acc;
                } else if (kind == kQkv) {
                    ll_store(P.QKV + row, __float_as_uint(acc), E(ph));
                } else if (kind == kGu) {
                    S.vec[t] = acc;  // the 4 groups = the 4 pairs of block ic
                } else {
#ifdef K2T_MK_TRACE_O
                    if (t == 0 && first) MK_TR(l, 5, kind == kO ? 2 : 4);
#endif
                    uint32_t hv = (uint32_t)rpre;
                    if ((uint32_t)(rpre >> 32) != er && ok && !ll_wait(P, res + row, er, hv)) ok = false;
                    const uint32_t nv = __float_as_uint(__uint_as_float(hv) + acc);
                    for (int r = 0; r < P.rep; r++)
                        ll_store((kind == kO ? P.HB : P.HA) + (size_t)r * d + row, nv, E(ph));
#ifdef K2T_MK_TRACE_O
                    if (t == 0 && first) MK_TR(l, 5, kind == kO ? 3 : 5);
#endif
                }
            }
            lds_barrier();
#ifdef K2T_MK_TRACE_GU
            if (kind == kGu && first) MK_TR(l, 5, 4);
#endif
            if (kind == kGu) {
                if (wave == 0) {
                    const int ic = base / 4;
                    // SwiGLU one element per lane (real_llm.rs:9801-9805), then four
                    // elements per lane for the rotation (one wave: its LDS accesses are
                    // performed in program order)
                    const float g = S.vec[lane], u = S.vec[64 + lane];
                    S.vec[lane] = (g / (1.0f + (EX ? expf_rn(-g) : expf(-g)))) * u;
                    const uint32_t s4 = lane & 15u;
                    const float4 va = *reinterpret_cast<const float4 *>(S.vec + s4 * 4);
                    float v[4] = {va.x, va.y, va.z, va.w};
                    const Chunk4 r = rotate_quant4(v, sign_mask_s(P, ic), s4);
                    store_act_chunk4(r, lane, P.GACT + (size_t)ic * kActWords, E(ph), P.rep, gact_words(P));
#ifdef K2T_MK_TRACE_GU
                    if (first) MK_TR(l, 5, 5);
#endif
                }
                lds_barrier();
            }
        }
        if (!ok) return;
        MK_TR(kind == kHead ? P.L : l, kind == kHead ? 0 : kind, 5);
    }
    // Greedy choice (argmax_scalar, real_llm.rs:9914-9924: largest logit, lowest row on
    // ties) and the position / step advance, inside the launch.  Each workgroup reduces
    // the logits rows it wrote in the lm_head phase (its own stores, visible after the
    // barrier) and hands {value, row} over as two words; workgroup 0 combines them, writes
    // the next input token and advances the position and the step counter.  Every
    // workgroup read the position and step at its start, before its words existed.
    {
        const MatDev &M = P.head;
        const int nwg = (int)gridDim.x;
        const int vb = ((int)blockIdx.x + nwg - P.head_off) % nwg;
        const int nblocks = M.smode ? M.stripes : M.np + (M.stripes & 1);
        const int groups = kWaves / M.nseg;
        const int ntk = (nblocks + groups - 1) / groups;
        const int RB = M.smode ? 16 : 32;
        __syncthreads();
        float bv = -INFINITY;
        int bi = 0x7fffffff;
        for (int tk = vb; tk < ntk; tk += nwg) {
            const int base = tk * groups;
            for (int i = t; i < groups * RB; i += kThreads) {
                const int g2 = i / RB, rl = i % RB, rb2 = xcd_stripe<kWaves>(M, base + g2, nblocks);
                if (rb2 >= nblocks) continue;
                const bool tail = !M.smode && rb2 >= M.np;
                const int first_stripe = M.smode ? rb2 : (tail ? 2 * M.np : 2 * rb2);
                const int row = first_stripe * 16 + rl;
                if (rl >= (tail ? 16 : RB) || row >= M.rows) continue;
                const float v = P.logits[row];
                if (v > bv || (v == bv && row < bi)) {
                    bv = v;
                    bi = row;
                }
            }
        }
        // workgroup reduction: waves, then wave 0 over the wave results
        for (int m2 = 1; m2 < 64; m2 <<= 1) {
            const float ov = __shfl_xor(bv, m2, kWave);
            const int oi = __shfl_xor(bi, m2, kWave);
            if (ov > bv || (ov == bv && oi < bi)) {
                bv = ov;
                bi = oi;
            }
        }
        if (lane == 0) {
            S.vec[wave] = bv;
            S.vec[kWaves + wave] = __int_as_float(bi);
        }
        __syncthreads();
        if (t == 0) {
            for (int w = 1; w < kWaves; w++) {
                const float ov = S.vec[w];
                const int oi = __float_as_int(S.vec[kWaves + w]);
                if (ov > bv || (ov == bv && oi < bi)) {
                    bv = ov;
                    bi = oi;
                }
            }
            ll_store(P.BEST + 2 * blockIdx.x, __float_as_uint(bv), E(nph));
            ll_store(P.BEST + 2 * blockIdx.x + 1, (uint32_t)bi, E(nph));
        }
        if (blockIdx.x != 0) return;
        bv = -INFINITY;
        bi = 0x7fffffff;
        bool ok = true;
        for (int w = t; w < nwg; w += kThreads) {
            uint32_t v = 0, r = 0;
            if (ok && !ll_wait(P, P.BEST + 2 * w, E(nph), v)) ok = false;
            if (ok && !ll_wait(P, P.BEST + 2 * w + 1, E(nph), r)) ok = false;
            const float ov = __uint_as_float(v);
            const int oi = (int)r;
            if (ok && (ov > bv || (ov == bv && oi < bi))) {
                bv = ov;
                bi = oi;
            }
        }
        for (int m2 = 1; m2 < 64; m2 <<= 1) {
            const float ov = __shfl_xor(bv, m2, kWave);
            const int oi = __shfl_xor(bi, m2, kWave);
            if (ov > bv || (ov == bv && oi < bi)) {
                bv = ov;
                bi = oi;
            }
        }
        __syncthreads();
        if (lane == 0) {
            S.vec[wave] = bv;
            S.vec[kWaves + wave] = __int_as_float(bi);
        }
        if (t == 0) S.flag[0] = 0;
        __syncthreads();
        if (!ok) S.flag[0] = 1;
        __syncthreads();
        if (t == 0 && S.flag[0] == 0) {
            for (int w = 1; w < kWaves; w++) {
                const float ov = S.vec[w];
                const int oi = __float_as_int(S.vec[kWaves + w]);
                if (ov > bv || (ov == bv && oi < bi)) {
                    bv = ov;
                    bi = oi;
                }
            }
            P.tokens[0] = bi == 0x7fffffff ? 0 : bi;
            P.pos_dev[0] = pos + 1;
            P.step_dev[0] = step + 1u;
        }
    }
}


}  // namespace

MatDev mat_dev(const k2t_mat *m, bool pair_mode_nseg4, int max_nseg, int nwaves, int min_nseg) {
    const int kWaves = nwaves;
    MatDev d{};
    d.pair = m->pair;
    d.tail = m->tail;
    d.ptot = m->fmt == K2T_FMT_NF ? (m->pairs ? m->pair_len / m->pairs : 0) : 0;
    d.rows = m->rows;
    d.nc = m->nc;
    d.np = m->pairs;
    d.stripes = m->stripes;
    d.fmt = m->fmt == K2T_FMT_NF ? (m->bits == 3 ? 2 : 1) : 0;  // 2: NF3 (per-operation path only)
    d.hp = m->hp;
    d.sgc = m->sgc;
    d.cb0 = m->cb[0];
    d.cb1 = m->cb[1];
    d.cb2 = m->cb[2];
    d.cb3 = m->cb[3];
    if (d.fmt == 1) nf4_xor_tables(m->cb[0], m->cb[1], m->cb[2], m->cb[3], d.cb0, d.cb1, d.cb2, d.cb3);
    if (pair_mode_nseg4) {  // 4 wave groups: the 4 pairs of one [gate64, up64] block
        d.smode = 0;
        d.nseg = kWaves / 4;
    } else {
        // Stripe mode with one round of the 8 lane groups per wave where K allows.
        d.smode = 1;
        const int want = std::max((m->nc + 7) / 8, min_nseg);
        const int cap = max_nseg > 0 ? std::min(max_nseg, kWaves) : kWaves;
        int nseg = 1;
        while (nseg < want && nseg < cap) nseg *= 2;
        d.nseg = nseg;
    }
    d.cps = (m->nc + d.nseg - 1) / d.nseg;
    return d;
}

int mk_phase_tasks(const MatDev &M, int nwaves) {
    const int nblocks = M.smode ? M.stripes : M.np + (M.stripes & 1);
    const int groups = nwaves / M.nseg;
    return (nblocks + groups - 1) / groups;
}

size_t decode_mk_lds_bytes(const k2t_model_config &c) {
    const size_t kmax = std::max(c.hidden, c.intermediate);
    const size_t hd = c.head_dim;
    size_t b = pad16((size_t)c.hidden * 4) + pad16(kmax) + 2 * pad16((kmax / 64) * 4) + kMaxWaves * 32 * 4 + 128 * 4 + 16;
    b = (b + 255) / 256 * 256;
    const size_t att = (3 * hd) * 4 + 3 * 128 + 8 * 4 + 32 * 4 + (size_t)kMaxThreads * 4 * 4 +
                       (size_t)std::min(c.max_seq, kMkMaxContext) * 4;
    // the largest weight ring of the three kernel variants (8 waves x NF4 / 4-plane
    // fragments, 4 waves x mixed-plane fragments)
    const size_t ring = std::max({(size_t)8 * kMkFrags * frag_lds_bytes<1, 0>(),
                                  (size_t)8 * kMkFrags * frag_lds_bytes<0, 0>(),
                                  (size_t)4 * kMkFrags * frag_lds_bytes<0, kHpMixed>(),
                                  (size_t)4 * kMkFrags * frag_lds_bytes<0, 2>()});
    b += std::max(att, ring);
    return (b + 255) / 256 * 256;
}

template <int FMT, int HP, int NTH>
static bool occupancy_ok(size_t lds) {
    int nb = 0, ne = 0;
    return hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, decode_mk_kernel<FMT, HP, NTH, false>, NTH, lds) ==
               hipSuccess &&
           nb >= 1 &&
           hipOccupancyMaxActiveBlocksPerMultiprocessor(&ne, decode_mk_kernel<FMT, HP, NTH, true>, NTH, lds) ==
               hipSuccess &&
           ne >= 1;
}

bool decode_mk_supported(const k2t_model_config &c, int num_cus) {
    if (decode_mk_lds_bytes(c) > kMkMaxLds) return false;
    if (c.hidden > 8192 || c.intermediate > 32768) return false;
    const size_t lds = decode_mk_lds_bytes(c);
    return num_cus > 0 && occupancy_ok<1, 0, 512>(lds) && occupancy_ok<0, 0, 512>(lds) &&
           occupancy_ok<0, kHpMixed, 256>(lds) && occupancy_ok<0, 2, 256>(lds);
}

int decode_mk_threads(int hp) { return hp == kHpMixed || hp == 2 ? 256 : 512; }

bool decode_mk_format(const MatDev &m, int &fmt, int &hp) {
    if (m.fmt == 2) return false;  // NF3 runs on the per-operation path
    // bit planes: any 5-plane matrix selects the 256-thread kernel that reads each matrix's
    // plane count (4 or 5); 6-plane (b6) models run the 256-thread two-hi-plane kernel,
    // which needs every matrix at 6 planes
    const int mhp = m.fmt != 0 ? 0 : m.hp == 2 ? 2 : m.hp == 1 ? kHpMixed : 0;
    if (fmt < 0) {
        fmt = m.fmt;
        hp = mhp;
        return true;
    }
    if (m.fmt != fmt) return false;
    if ((mhp == 2) != (hp == 2)) return false;
    if (mhp == kHpMixed) hp = kHpMixed;
    return true;
}

template <bool EX>
static void launch_mk(hipStream_t st, const MkParams &P, int fmt, int hp, int num_cus, size_t lds) {
    if (fmt == 1) hipLaunchKernelGGL((decode_mk_kernel<1, 0, 512, EX>), dim3(num_cus), dim3(512), lds, st, P);
    else if (hp == 0) hipLaunchKernelGGL((decode_mk_kernel<0, 0, 512, EX>), dim3(num_cus), dim3(512), lds, st, P);
    else if (hp == kHpMixed)
        hipLaunchKernelGGL((decode_mk_kernel<0, kHpMixed, 256, EX>), dim3(num_cus), dim3(256), lds, st, P);
    else if (hp == 2)
        hipLaunchKernelGGL((decode_mk_kernel<0, 2, 256, EX>), dim3(num_cus), dim3(256), lds, st, P);
    else throw Error(K2T_E_INTERNAL, "persistent decode kernel: unsupported weight format");
}

void launch_decode_mk(hipStream_t st, const MkParams &P, int fmt, int hp, int num_cus, size_t lds, bool exact) {
    if (exact) {
        if (!P.exterm || P.nsp != 1) throw Error(K2T_E_INTERNAL, "exact-order persistent kernel: bad parameters");
        launch_mk<true>(st, P, fmt, hp, num_cus, lds);
    } else {
        launch_mk<false>(st, P, fmt, hp, num_cus, lds);
    }
    hip_check(hipGetLastError(), "decode megakernel launch");
}


}  // namespace k2t
