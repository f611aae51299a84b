// Device helpers shared by the gfx950 kernels: Hadamard sign masks, wave-level
// butterflies and reductions (DPP), BF16 decode and byte-table lookups.
#pragma once
#include <float.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace k2t {

constexpr int kWave = 64;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// 128-bit streaming load (nontemporal: weight bytes are read once per pass).
__device__ __forceinline__ uint4 load_stream16(const void *p) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// Loads with the address space stated: where one expression reads either global memory
// or LDS (a select of the two pointers), the compiler emits a flat access, which waits
// for the wave's outstanding global operations as well; a load from each side keeps
// the global load a global load and the LDS read an LDS read.
// (The host pass of a HIP source also parses these bodies; it has no such address spaces.)
template <class T>
__device__ __forceinline__ T ld_global(const T *p) {
#if defined(__HIP_DEVICE_COMPILE__)
    return *(const __attribute__((address_space(1))) T *)p;
#else
    return *p;
#endif
}
template <class T>
__device__ __forceinline__ T ld_lds(const T *p) {
#if defined(__HIP_DEVICE_COMPILE__)
    return *(const __attribute__((address_space(3))) T *)p;
#else
    return *p;
#endif
}

// 16 bytes from LDS, waited for, by inline assembly: for a read that sits on one side
// of a branch whose other side loads the same shape from global memory (the compiler
// would otherwise merge the two into one flat load through a select of the pointers).
__device__ __forceinline__ uint4 lds_read16_now(const void *p) {
    uint4 r;
    const uint32_t a = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
    asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(r) : "v"(a) : "memory");
    return r;
}

// Direct-to-LDS loads (global_load_lds): lane L's bytes land at M0 + size * L.  Issued
// from inline assembly, so the compiler neither tracks them nor inserts its conservative
// "all vector memory done" wait before later LDS reads; callers order them through the
// in-issue-order completion of a wave's vector memory operations.  M0 is set inside each
// statement: no compiler-generated code of these kernels uses M0 (the build checks).
__device__ __forceinline__ uint32_t lds_offset(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

// 16 bytes per lane from p (per-lane address) to LDS [m0 + 16 * lane].
__device__ __forceinline__ void lds_dma16(const void *p, uint32_t m0) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(p), "s"(m0) : "memory");
}
// 4 bytes per lane from p to LDS [m0 + 4 * lane].
__device__ __forceinline__ void lds_dma4(const void *p, uint32_t m0) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" ::"v"(p), "s"(m0) : "memory");
}
// The same from base + voff + OFF: a wave-uniform 64-bit base (SGPRs), a per-lane 32-bit
// offset and an immediate, so a stream that advances by a uniform stride costs its
// waves scalar adds only.  The instruction's immediate offset moves the LDS address as
// well (LDS [M0 + OFF + size * lane]), so M0 is set OFF lower: the bytes still land at
// m0 + size * lane.
template <int OFF>
__device__ __forceinline__ void lds_dma16_sa(uint32_t voff, const void *sbase, uint32_t m0) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1 offset:%3 nt" ::"v"(voff), "s"(sbase),
                 "s"(m0 - (uint32_t)OFF), "i"(OFF)
                 : "memory");
}
template <int OFF>
__device__ __forceinline__ void lds_dma4_sa(uint32_t voff, const void *sbase, uint32_t m0) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dword %0, %1 offset:%3" ::"v"(voff), "s"(sbase),
                 "s"(m0 - (uint32_t)OFF), "i"(OFF)
                 : "memory");
}

// A 64-bit hand-off word {epoch (high half), payload (low half)}, written and read with
// one agent-scope atomic each: coherent across XCDs, and the payload and its ready mark
// arrive together, so neither side needs a fence.
__device__ __forceinline__ void ll_word_store(unsigned long long *p, uint32_t v, uint32_t epoch) {
    __hip_atomic_store(p, ((unsigned long long)epoch << 32) | v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long ll_word_load(const unsigned long long *p) {
    return __hip_atomic_load(const_cast<unsigned long long *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Waits until at most N vector memory operations of this wave are outstanding.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Sign of element `i` of Hadamard block `block` (hadamard.rs:29-44): SplitMix64 state
// seed + block*0xBF58.. advanced i+1 times, finalized, low bit.  Each lane computes its
// own element, so no table is needed.
__device__ __forceinline__ uint32_t hadamard_sign_bit(uint64_t block, uint32_t i) {
    uint64_t z = 0x9E3779B97F4A7C15ull + block * 0xBF58476D1CE4E5B9ull +
                 (uint64_t)(i + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    return (uint32_t)(z & 1);
}

// DPP lane moves inside one 16-lane row.
// (bound_ctrl set: every source lane of these patterns exists, and the compiler can then
// fold the move into the instruction that uses it)
__device__ __forceinline__ int dpp_xor1(int v) { return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, true); }
__device__ __forceinline__ int dpp_ror8(int v) { return __builtin_amdgcn_mov_dpp(v, 0x128, 0xF, 0xF, true); }
__device__ __forceinline__ int dpp_ror4(int v) { return __builtin_amdgcn_mov_dpp(v, 0x124, 0xF, 0xF, true); }

__device__ __forceinline__ float shfl_xor_f(float v, int m) { return __shfl_xor(v, m, kWave); }

// Exchange with lane ^ 1, ^ 2 (DPP quad permutes) and ^ 4 (ds_swizzle bit mode).
__device__ __forceinline__ float xchg1(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true));
}
__device__ __forceinline__ float xchg2(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, true));
}
__device__ __forceinline__ float xchg4(float v) {
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x101F));
}
__device__ __forceinline__ int xchg1(int v) { return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false); }
__device__ __forceinline__ int xchg2(int v) { return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false); }
__device__ __forceinline__ int xchg4(int v) { return __builtin_amdgcn_ds_swizzle(v, 0x101F); }

// Value of lane ^ m (m a power of two below 64) through the cheapest exchange that has
// exactly that partner: DPP quad permutes for 1 and 2, the DPP row rotate by 8 (which is
// lane ^ 8 inside a 16-lane row), ds_swizzle's bit mode for 4 and 16, ds_bpermute across
// the two 32-lane halves.  Every wave reduction and butterfly below pairs the same lanes
// in the same order as a __shfl_xor loop, so their results are unchanged.
__device__ __forceinline__ int xor_lane(int v, int m) {
    switch (m) {
        case 1: return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);
        case 2: return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false);
        case 4: return __builtin_amdgcn_ds_swizzle(v, 0x101F);
        case 8: return __builtin_amdgcn_mov_dpp(v, 0x128, 0xF, 0xF, false);
        case 16: return __builtin_amdgcn_ds_swizzle(v, 0x401F);
        default: return __shfl_xor(v, m, kWave);
    }
}
__device__ __forceinline__ float xor_lane(float v, int m) { return __int_as_float(xor_lane(__float_as_int(v), m)); }

// Lane l's value in every lane, for a wave-uniform l (v_readlane, no LDS round trip): the
// same value as __shfl(v, l).
__device__ __forceinline__ int lane_val(int v, int l) { return __builtin_amdgcn_readlane(v, l); }
__device__ __forceinline__ float lane_val(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// Wave reductions: butterflies inside each 32-lane half, after which every lane of a half
// holds the same bits; the last step combines the two halves' values read from lanes 0
// and 32, which is the butterfly's own last step (max and + are commutative).
__device__ __forceinline__ float wave_max_f(float v) {
#pragma unroll
    for (int m = 1; m < 32; m <<= 1) v = fmaxf(v, xor_lane(v, m));
    return fmaxf(lane_val(v, 0), lane_val(v, 32));
}
__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
    for (int m = 1; m < 32; m <<= 1) v += xor_lane(v, m);
    return lane_val(v, 0) + lane_val(v, 32);
}
__device__ __forceinline__ float wave_sum_f(float v) {
#pragma unroll
    for (int m = 1; m < 32; m <<= 1) v += xor_lane(v, m);
    return lane_val(v, 0) + lane_val(v, 32);
}

// Sum of squares of a K-float row (K a multiple of 64) by one wave, in a fixed order:
// lane l takes float4 l, l+64, ... four loads in flight, fmaf per component, then a
// butterfly sum.  Every kernel that needs inv_rms uses this, so all agree bit for bit.
__device__ __forceinline__ float row_sumsq_wave(const float *xt, int K, uint32_t lane) {
    const float4 *x4 = reinterpret_cast<const float4 *>(xt);
    const int n4 = K / 4;
    float ss = 0.0f;
    int i = (int)lane;
    for (; i + 192 < n4; i += 256) {
        float4 v[4];
#pragma unroll
        for (int u = 0; u < 4; u++) v[u] = x4[i + 64 * u];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            ss = fmaf(v[u].x, v[u].x, ss);
            ss = fmaf(v[u].y, v[u].y, ss);
            ss = fmaf(v[u].z, v[u].z, ss);
            ss = fmaf(v[u].w, v[u].w, ss);
        }
    }
    for (; i < n4; i += 64) {
        const float4 v = x4[i];
        ss = fmaf(v.x, v.x, ss);
        ss = fmaf(v.y, v.y, ss);
        ss = fmaf(v.z, v.z, ss);
        ss = fmaf(v.w, v.w, ss);
    }
    return wave_sum_f(ss);
}

// In-register signed FWHT-64 over one wave (lane i holds element i): butterflies with
// stride h = 1..32 exactly as hadamard.rs:83-97 (lower lane a+b, upper lane a-b).
__device__ __forceinline__ float wave_butterflies64(float v, uint32_t lane) {
#pragma unroll
    for (int h = 1; h < 64; h <<= 1) {
        float p = xor_lane(v, h);
        v = (lane & h) ? (p - v) : (v + p);
    }
    return v;
}

__device__ __forceinline__ float flip_sign(float v, uint32_t neg) {
    return __uint_as_float(__float_as_uint(v) ^ (neg << 31));
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// 16-entry signed-byte table lookup of four 4-bit indices, one per byte.
// `s` holds the low 3 bits of each index, `m` is 0xFF in bytes whose index has bit 3.
// cb0..cb3 = table bytes 0-3, 4-7, 8-11, 12-15.
__device__ __forceinline__ uint32_t lut16(uint32_t s, uint32_t m, uint32_t cb0, uint32_t cb1,
                                          uint32_t cb2, uint32_t cb3) {
    uint32_t lo = __builtin_amdgcn_perm(cb1, cb0, s);
    uint32_t hi = __builtin_amdgcn_perm(cb3, cb2, s);
    return (hi & m) | (lo & ~m);
}

// A 16-entry signed-byte codebook (cb0..cb3, byte i = entry i) as two 8-byte tables T
// (from entries 0-7) and U (entries 8-15) such that, per byte, entry n equals
//   perm(T, n) ^ perm(U, n ^ 8)
// for the 4-bit index n: perm with a selector 0-7 returns that table byte, with 8-11 the
// sign of table byte 1, 3, 5, 7 spread over the byte, with 12 zero, with 13-15 0xFF.  So
// for n < 8 the U lookup returns a fill byte fixed by U's signs, and for n >= 8 the T
// lookup one fixed by T's signs; T and U hold the entries XOR those fills.  The fills
// depend on T's and U's own sign bits, an acyclic chain that every codebook satisfies.
__host__ __device__ __forceinline__ void nf4_xor_tables(uint32_t cb0, uint32_t cb1, uint32_t cb2, uint32_t cb3, uint32_t &t0,
                                               uint32_t &t1, uint32_t &u0, uint32_t &u1) {
    const uint32_t w[4] = {cb0, cb1, cb2, cb3};
    auto sgn = [&](int i) { return (w[i >> 2] >> (8 * (i & 3) + 7)) & 1u; };
    uint32_t eT[8], eU[8];  // fill of the T lookup for entry 8 + j, of the U lookup for entry j
    eT[4] = eU[4] = 0u;
    eT[5] = eT[6] = eT[7] = eU[5] = eU[6] = eU[7] = 1u;
    eT[2] = sgn(5) ^ 1u;  // sign of T[5] = entry 5 ^ fill 1
    eT[3] = sgn(7) ^ 1u;
    eU[2] = sgn(13) ^ 1u;
    eU[3] = sgn(15) ^ 1u;
    eU[1] = sgn(11) ^ eT[3];
    eT[1] = sgn(3) ^ eU[3];
    eU[0] = sgn(9) ^ eT[1];
    eT[0] = sgn(1) ^ eU[1];
    uint32_t t[2] = {0u, 0u}, u[2] = {0u, 0u};
    for (int j = 0; j < 8; j++) {
        const uint32_t lo = (w[j >> 2] >> (8 * (j & 3))) & 0xFFu, hi = (w[2 + (j >> 2)] >> (8 * (j & 3))) & 0xFFu;
        t[j >> 2] |= (lo ^ (eU[j] ? 0xFFu : 0u)) << (8 * (j & 3));
        u[j >> 2] |= (hi ^ (eT[j] ? 0xFFu : 0u)) << (8 * (j & 3));
    }
    t0 = t[0];
    t1 = t[1];
    u0 = u[0];
    u1 = u[1];
}

// Codebook values of four 4-bit indices (one per byte) through the tables above.
__device__ __forceinline__ uint32_t nf4_xlut(uint32_t s, uint32_t t0, uint32_t t1, uint32_t u0, uint32_t u1) {
    return __builtin_amdgcn_perm(t1, t0, s) ^ __builtin_amdgcn_perm(u1, u0, s ^ 0x08080808u);
}

// Byte mask 0xFF where bit 7 of the byte is set (v_perm selectors >= 13 give 0xFF,
// selector 0 picks byte 0 of the zero pool).
__device__ __forceinline__ uint32_t bit7_mask(uint32_t v) {
    return __builtin_amdgcn_perm(0u, 0u, v & 0x80808080u);
}

// Byte mask 0xFF where bit 3 of the byte is set: selector 8 returns the sign of byte 1
// of the second operand (0x80 -> 0xFF), selector 0 its byte 0 (0x00).
__device__ __forceinline__ uint32_t bit3_mask(uint32_t v) {
    return __builtin_amdgcn_perm(0u, 0x8000u, v & 0x08080808u);
}

// Lane `lane`'s byte (column lane of chunk c, token tok), the chunk's scale and its code
// sum in the tile-major copy the matrix-core GEMV reads: per (16-token block, chunk) 1 KB
// in its B operand's lane order (16 bytes per MFMA lane 16 * (col / 16) + tok % 16), 16
// scales and 16 sums.
__device__ __forceinline__ void act_tile_store(int8_t *xt, float *st, int32_t *ut, int tok, int c, int nc,
                                               uint32_t lane, int8_t qv, float scale, int32_t sum) {
    const size_t tile = (size_t)(tok >> 4) * nc + c;
    xt[tile * 1024 + (((lane >> 4) * 16u + (uint32_t)(tok & 15)) * 16u) + (lane & 15u)] = qv;
    if (lane == 0) {
        st[tile * 16 + (tok & 15)] = scale;
        ut[tile * 16 + (tok & 15)] = sum;
    }
}

// Quantizes the 64 values held one per lane (already rotated) to int8 with one scale
// (simd_lut.rs:3097-3128 / 3172-3195).  With xt, also into the tile-major copy (chunk c
// of nc, token tok; st and ut receive the scale and the code sum).
__device__ __forceinline__ void quant_chunk_store(float v, uint32_t lane, int8_t *q, float *scale,
                                                  int32_t *sum, int8_t *xt = nullptr, float *st = nullptr,
                                                  int32_t *ut = nullptr, int tok = 0, int c = 0, int nc = 0) {
    const float mx = wave_max_f(fabsf(v));
    if (mx <= FLT_EPSILON) {
        q[lane] = 0;
        if (lane == 0) {
            *scale = 0.0f;
            *sum = 0;
        }
        if (xt) act_tile_store(xt, st, ut, tok, c, nc, lane, 0, 0.0f, 0);
        return;
    }
    const float inv = 127.0f / mx;
    const int qi = (int)rintf(v * inv);
    const int s = wave_sum_i(qi);
    q[lane] = (int8_t)qi;
    if (lane == 0) {
        *scale = mx / 127.0f;
        *sum = s;
    }
    if (xt) act_tile_store(xt, st, ut, tok, c, nc, lane, (int8_t)qi, mx / 127.0f, s);
}

__device__ __forceinline__ float fwht_lane(float v, uint64_t block, uint32_t lane) {
    v = flip_sign(v, hadamard_sign_bit(block, lane)) * 0.125f;
    return wave_butterflies64(v, lane);
}

// hadamard.rs:193-228 on one block held one element per lane.
__device__ __forceinline__ float ifwht_lane(float v, uint64_t block, uint32_t lane) {
    v = wave_butterflies64(v, lane);
    return flip_sign(v * 0.125f, hadamard_sign_bit(block, lane));
}

// Butterflies h = 1..32 of one 64-element block held as eight consecutive elements per
// lane by eight lanes (lane bits 0-2 = s, element s*8 + j): h = 1, 2, 4 in registers and
// h = 8, 16, 32 across lanes (^1, ^2, ^4).  Each stage adds or subtracts the same operands
// as hadamard.rs:83-97 (lower a+b, upper a-b), in the same stage order as
// wave_butterflies64, so the results are bit-identical to it.
__device__ __forceinline__ void butterflies_slice8(float *v, uint32_t s) {
#pragma unroll
    for (int h = 1; h < 8; h <<= 1)
#pragma unroll
        for (int j = 0; j < 8; j++)
            if (!(j & h)) {
                const float x0 = v[j], x1 = v[j | h];
                v[j] = x0 + x1;
                v[j | h] = x0 - x1;
            }
    // across lanes: lower lane v + p, upper lane p - v, both as p + (+-v) (IEEE addition
    // commutes and a - b is a + (-b), so the bits are those of the two-sided form)
    // (all eight exchanges of a stage are issued before the first add: the ^4 exchange
    // is an LDS round trip, and eight of them back to back share one wait)
#pragma unroll
    for (int m = 1; m < 8; m <<= 1) {
        const uint32_t neg = (s & (uint32_t)m) != 0 ? 0x80000000u : 0u;
        float p[8];
#pragma unroll
        for (int j = 0; j < 8; j++) p[j] = m == 1 ? xchg1(v[j]) : m == 2 ? xchg2(v[j]) : xchg4(v[j]);
#pragma unroll
        for (int j = 0; j < 8; j++) v[j] = p[j] + __uint_as_float(__float_as_uint(v[j]) ^ neg);
    }
}

// One quantized 64-element chunk as eight lanes hold it: codes of elements s*8 .. s*8+3
// (lo) and s*8+4 .. s*8+7 (hi), one byte each; scale and code sum (same in every lane).
struct Chunk8 {
    uint32_t lo, hi;
    float scale;
    int sum;
};

// Signed FWHT-64 + int8 quantization of one chunk in the slice-of-8 layout: sign flip
// with the chunk's mask bits, x0.125, butterflies_slice8, then max, int8 round-half-even,
// scale = max/127 and the code sum (simd_lut.rs:3097-3128 / 3172-3195).  The result
// equals fwht_lane + quant_chunk_store.  All 64 lanes must call it.
__device__ __forceinline__ Chunk8 rotate_quant8(float *v, uint64_t sign_mask, uint32_t s) {
    const uint32_t sb = (uint32_t)(sign_mask >> (8u * s)) & 0xFFu;
#pragma unroll
    for (int j = 0; j < 8; j++) v[j] = flip_sign(v[j], (sb >> j) & 1u) * 0.125f;
    butterflies_slice8(v, s);
    float mx = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j++) mx = fmaxf(mx, fabsf(v[j]));
    mx = fmaxf(mx, xchg1(mx));
    mx = fmaxf(mx, xchg2(mx));
    mx = fmaxf(mx, xchg4(mx));
    Chunk8 r{0u, 0u, 0.0f, 0};
    if (mx > FLT_EPSILON) {
        const float inv = 127.0f / mx;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int qi = (int)rintf(v[j] * inv);
            r.sum += qi;
            if (j < 4) r.lo |= ((uint32_t)qi & 0xFFu) << (8 * j);
            else r.hi |= ((uint32_t)qi & 0xFFu) << (8 * (j - 4));
        }
        r.scale = mx / 127.0f;
    }
    r.sum += xchg1(r.sum);
    r.sum += xchg2(r.sum);
    r.sum += xchg4(r.sum);
    return r;
}

// The same butterflies with four consecutive elements per lane by sixteen lanes (lane
// bits 0-3 = s, element s*4 + j): h = 1, 2 in registers, h = 4 .. 32 across lanes (^1, ^2,
// ^4 by ds_swizzle, ^8 by the DPP row rotate).  For a single chunk per wave this layout
// needs about half the instructions of the eight-element one and still one LDS round
// trip per transform.
__device__ __forceinline__ float xchg8(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xF, 0xF, true));
}
__device__ __forceinline__ int xchg8(int v) { return __builtin_amdgcn_mov_dpp(v, 0x128, 0xF, 0xF, false); }
__device__ __forceinline__ void butterflies_slice4(float *v, uint32_t s) {
#pragma unroll
    for (int h = 1; h < 4; h <<= 1)
#pragma unroll
        for (int j = 0; j < 4; j++)
            if (!(j & h)) {
                const float x0 = v[j], x1 = v[j | h];
                v[j] = x0 + x1;
                v[j | h] = x0 - x1;
            }
#pragma unroll
    for (int m = 1; m < 16; m <<= 1) {
        const uint32_t neg = (s & (uint32_t)m) != 0 ? 0x80000000u : 0u;
        float p[4];
#pragma unroll
        for (int j = 0; j < 4; j++)
            p[j] = m == 1 ? xchg1(v[j]) : m == 2 ? xchg2(v[j]) : m == 4 ? xchg4(v[j]) : xchg8(v[j]);
#pragma unroll
        for (int j = 0; j < 4; j++) v[j] = p[j] + __uint_as_float(__float_as_uint(v[j]) ^ neg);
    }
}

// One quantized chunk as sixteen lanes hold it: the codes of elements s*4 .. s*4+3 (one
// byte each, element s*4 + b in byte b), the scale and the code sum.
struct Chunk4 {
    uint32_t w;
    float scale;
    int sum;
};

// rotate_quant8's arithmetic in the four-element layout.
__device__ __forceinline__ Chunk4 rotate_quant4(float *v, uint64_t sign_mask, uint32_t s) {
    const uint32_t sb = (uint32_t)(sign_mask >> (4u * s)) & 0xFu;
#pragma unroll
    for (int j = 0; j < 4; j++) v[j] = flip_sign(v[j], (sb >> j) & 1u) * 0.125f;
    butterflies_slice4(v, s);
    float mx = fmaxf(fmaxf(0.0f, fabsf(v[0])), fabsf(v[1]));
    mx = fmaxf(fmaxf(mx, fabsf(v[2])), fabsf(v[3]));
    mx = fmaxf(mx, xchg1(mx));
    mx = fmaxf(mx, xchg2(mx));
    mx = fmaxf(mx, xchg4(mx));
    mx = fmaxf(mx, xchg8(mx));
    Chunk4 r{0u, 0.0f, 0};
    if (mx > FLT_EPSILON) {
        const float inv = 127.0f / mx;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int qi = (int)rintf(v[j] * inv);
            r.sum += qi;
            r.w |= ((uint32_t)qi & 0xFFu) << (8 * j);
        }
        r.scale = mx / 127.0f;
    }
    r.sum += xchg1(r.sum);
    r.sum += xchg2(r.sum);
    r.sum += xchg4(r.sum);
    r.sum += xchg8(r.sum);
    return r;
}

// A Chunk4 (sixteen lanes, slice sl) of chunk c, token tok, stored as quant_chunk_store
// stores the one-element-per-lane form: codes q[tok * nc + c][4 sl .. 4 sl + 3] as one
// word, the scale and the code sum; with xt, also into the tile-major copy (the four
// codes are consecutive bytes there too).
__device__ __forceinline__ void chunk4_store(const Chunk4 &r, uint32_t sl, int tok, int c, int nc, int8_t *q,
                                             float *scale, int32_t *sum, int8_t *xt, float *st, int32_t *ut) {
    const size_t gc = (size_t)tok * nc + c;
    *reinterpret_cast<uint32_t *>(q + gc * 64 + 4 * sl) = r.w;
    if (sl == 0) {
        scale[gc] = r.scale;
        sum[gc] = r.sum;
    }
    if (xt) {
        const size_t tile = (size_t)(tok >> 4) * nc + c;
        *reinterpret_cast<uint32_t *>(xt + tile * 1024 + ((sl >> 2) * 16u + (uint32_t)(tok & 15)) * 16u + (sl & 3u) * 4u) =
            r.w;
        if (sl == 0) {
            st[tile * 16 + (tok & 15)] = r.scale;
            ut[tile * 16 + (tok & 15)] = r.sum;
        }
    }
}

// rotate_quant8 into the LDS activation: `act` gates the stores (codes at
// xl[c*64 + s*8], scale xsl[c], sum xsuml[c]).
__device__ __forceinline__ void rotate_quant_slice8(float *v, uint64_t sign_mask, uint32_t s, int c, bool act,
                                                    int8_t *xl, float *xsl, int32_t *xsuml) {
    const Chunk8 r = rotate_quant8(v, sign_mask, s);
    if (act) {
        *reinterpret_cast<uint2 *>(xl + c * 64 + s * 8) = make_uint2(r.lo, r.hi);
        if (s == 0) {
            xsl[c] = r.scale;
            xsuml[c] = r.sum;
        }
    }
}

}  // namespace k2t
