/*
 * k2t_oracle.c -- CPU restatement of kronos-2t's quantized decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (the HIP library under
 * kronos-2t_amd/) links, loads or calls this file.  Only tests/, the smoke()
 * check in __graft_entry__.py and the cpu_baseline leg of bench.py use it,
 * and only as the checker / the timed portable CPU baseline.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the kronos-2t source root).  Floating-point statements follow the Rust code
 * operation by operation: the file is compiled with -ffp-contract=off so that
 * a*b+c stays two roundings unless the reference itself fuses (vfmaq), where
 * fmaf() is written explicitly.
 *
 * Pinning (how each part is checked beyond re-reading it):
 *   FWHT            : brute-force H64*D/8 matrix product in f64, self-inverse,
 *                     inner-product invariance, reference test vectors
 *                     (hadamard.rs:300-330).
 *   populate        : closed-form invariants (|q|<=127, sum==sum(q),
 *                     max|q|==127, zero chunk), reference tests 8843-8905.
 *   bipolar RTN     : brute-force best ratio on tiny inputs, dequant error
 *                     bound, repack invariance (reference test 8745-8766).
 *   NF fit/RTN      : default-codebook fallback, symmetry, monotonicity,
 *                     nearest-centroid property.
 *   GEMV            : per-(row,chunk) integer dots vs a brute-force int64
 *                     product of the dequantized integer grid; the fp32
 *                     epilogue vs the portable dequantize+dot path.
 *   attention       : fp64 naive attention on the dequantized int8 K/V.
 */
#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define STRIPE 16

/* ------------------------------------------------------------------ */
/* FWHT-64 (hadamard.rs)                                               */
/* ------------------------------------------------------------------ */

/* hadamard.rs:29-44 rademacher_sign_masks_64: bit i set <=> element i is negated. */
uint64_t or_sign_bits(uint64_t block_idx) {
    uint64_t state = 0x9E3779B97F4A7C15ULL + block_idx * 0xBF58476D1CE4E5B9ULL;
    uint64_t bits = 0;
    for (int i = 0; i < 64; i++) {
        state += 0x9E3779B97F4A7C15ULL;
        uint64_t z = state;
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
        z ^= z >> 31;
        if (z & 1) bits |= 1ULL << i;
    }
    return bits;
}

static inline float flip_sign(float v, int neg) {
    uint32_t u;
    memcpy(&u, &v, 4);
    if (neg) u ^= 0x80000000u;
    memcpy(&v, &u, 4);
    return v;
}

/* hadamard.rs:83-97: radix-2 butterflies, stride h = 1,2,4,...,32. */
static void butterflies64(float *b) {
    for (int h = 1; h < 64; h *= 2) {
        for (int i = 0; i < 64; i += 2 * h) {
            for (int j = i; j < i + h; j++) {
                float a = b[j], c = b[j + h];
                b[j] = a + c;
                b[j + h] = a - c;
            }
        }
    }
}

/* hadamard.rs:70-99 fwht64_signed_inplace_scalar, one block with an explicit block index. */
void or_fwht64_block(float *b, uint64_t block_idx) {
    uint64_t m = or_sign_bits(block_idx);
    for (int i = 0; i < 64; i++) b[i] = flip_sign(b[i], (int)((m >> i) & 1)) * 0.125f;
    butterflies64(b);
}

/* hadamard.rs:193-228 ifwht64_signed_inplace_scalar, one block. */
void or_ifwht64_block(float *b, uint64_t block_idx) {
    uint64_t m = or_sign_bits(block_idx);
    butterflies64(b);
    for (int i = 0; i < 64; i++) b[i] = flip_sign(b[i] * 0.125f, (int)((m >> i) & 1));
}

void or_fwht64(float *x, size_t n) {
    for (size_t b = 0; b < n / 64; b++) or_fwht64_block(x + 64 * b, b);
}

void or_ifwht64(float *x, size_t n) {
    for (size_t b = 0; b < n / 64; b++) or_ifwht64_block(x + 64 * b, b);
}

/* ------------------------------------------------------------------ */
/* bf16 (simd_lut.rs:1373-1389)                                        */
/* ------------------------------------------------------------------ */

uint16_t or_f32_to_bf16(float v) {
    uint32_t bits;
    memcpy(&bits, &v, 4);
    if ((bits & 0x7F800000u) == 0x7F800000u && (bits & 0x007FFFFFu) != 0)
        return (uint16_t)((bits >> 16) | 0x0040u);
    uint32_t bias = 0x7FFFu + ((bits >> 16) & 1u);
    return (uint16_t)((bits + bias) >> 16);
}

float or_bf16_to_f32(uint16_t b) {
    uint32_t u = ((uint32_t)b) << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* ------------------------------------------------------------------ */
/* Int8ChunkActivation (simd_lut.rs:2921-3256)                         */
/* ------------------------------------------------------------------ */

static void quantize_block64(const float *blk, int8_t *q, float *scale, int32_t *sum) {
    float max_abs = 0.0f;
    for (int i = 0; i < 64; i++) max_abs = fmaxf(max_abs, fabsf(blk[i]));
    if (max_abs <= FLT_EPSILON) {
        memset(q, 0, 64);
        *scale = 0.0f;
        *sum = 0;
        return;
    }
    float inv = 127.0f / max_abs;
    int32_t s = 0;
    for (int i = 0; i < 64; i++) {
        int32_t qv = (int32_t)rintf(blk[i] * inv); /* round_ties_even */
        s += qv;
        q[i] = (int8_t)qv;
    }
    *scale = max_abs / 127.0f;
    *sum = s;
}

/* simd_lut.rs:3134-3196 populate_chunk_fwht_scalar (optional (x*inv_rms)*w, sign flip, x0.125,
 * butterflies, per-chunk int8).  `c_idx` selects the sign masks. */
void or_populate_chunk_fwht(const float *x64, const float *w64, float inv_rms, uint64_t c_idx,
                            int8_t *q64, float *scale, int32_t *sum) {
    float blk[64];
    uint64_t m = or_sign_bits(c_idx);
    for (int i = 0; i < 64; i++) {
        float xn = w64 ? (x64[i] * inv_rms) * w64[i] : x64[i];
        blk[i] = flip_sign(xn, (int)((m >> i) & 1)) * 0.125f;
    }
    butterflies64(blk);
    quantize_block64(blk, q64, scale, sum);
}

/* simd_lut.rs:2954-2997 populate_fwht / populate_rmsnorm_fwht over all chunks of one vector. */
void or_populate_fwht(const float *x, const float *w, float inv_rms, size_t K, int8_t *q,
                      float *scales, int32_t *sums) {
    for (size_t c = 0; c < K / 64; c++)
        or_populate_chunk_fwht(x + 64 * c, w ? w + 64 * c : NULL, inv_rms, c, q + 64 * c,
                               scales + c, sums + c);
}

/* simd_lut.rs:3235-3255 populate_scalar (no rotation). */
void or_populate_plain(const float *x, size_t K, int8_t *q, float *scales, int32_t *sums) {
    for (size_t c = 0; c < K / 64; c++) quantize_block64(x + 64 * c, q + 64 * c, scales + c, sums + c);
}

/* real_llm.rs:9858-9861 with the portable dot order of real_llm.rs:911-926. */
float or_inv_rms(const float *x, size_t n, float eps) {
    float acc[4] = {0, 0, 0, 0};
    size_t i = 0;
    for (; i + 4 <= n; i += 4)
        for (int k = 0; k < 4; k++) acc[k] += x[i + k] * x[i + k];
    float sum = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    for (; i < n; i++) sum += x[i] * x[i];
    float mean_sq = sum / (float)n;
    return 1.0f / sqrtf(mean_sq + eps);
}

/* The same with the aarch64 sum of squares, dot_f32_neon_16 (real_llm.rs:929-962): four
 * 4-lane accumulators fed by fused multiply-adds over 16-element steps, the accumulators
 * added lane-wise as (acc0 + acc1) + (acc2 + acc3), the lanes reduced pairwise
 * (l0 + l1) + (l2 + l3), then the remainder added sequentially (x*y rounded, then +).
 * The reference's NEON and x86 builds differ only by this summation order. */
float or_inv_rms_neon(const float *x, size_t n, float eps) {
    float acc[4][4] = {{0}};
    size_t i = 0;
    for (; i + 16 <= n; i += 16)
        for (int v = 0; v < 4; v++)
            for (int l = 0; l < 4; l++) acc[v][l] = fmaf(x[i + 4 * v + l], x[i + 4 * v + l], acc[v][l]);
    float lane[4];
    for (int l = 0; l < 4; l++) lane[l] = (acc[0][l] + acc[1][l]) + (acc[2][l] + acc[3][l]);
    float sum = (lane[0] + lane[1]) + (lane[2] + lane[3]);
    for (; i < n; i++) sum += x[i] * x[i];
    float mean_sq = sum / (float)n;
    return 1.0f / sqrtf(mean_sq + eps);
}

/* ------------------------------------------------------------------ */
/* Bipolar RTN quantizer (compiler.rs:912-1107, hessian = None)        */
/* ------------------------------------------------------------------ */

/* Returns u codes [rows*cols] and BF16 scales [num_stripes][num_chunks][16]. */
void or_bipolar_rtn(const float *W, size_t rows, size_t cols, int planes, uint8_t *u,
                    uint16_t *scales) {
    static const float ratios[12] = {0.62f, 0.67f, 0.72f, 0.77f, 0.82f, 0.87f,
                                     0.92f, 0.97f, 1.02f, 1.07f, 1.12f, 1.18f};
    const int max_odd = (1 << planes) - 1;
    const float max_u_f = (float)max_odd;
    const float half_off = 0.5f * max_u_f;
    const size_t nc = cols / 64;
    const size_t stripes = (rows + STRIPE - 1) / STRIPE;
    memset(u, 0, rows * cols);
    memset(scales, 0, stripes * nc * STRIPE * sizeof(uint16_t));
    float *work = (float *)malloc(cols * sizeof(float));
    for (size_t r = 0; r < rows; r++) {
        memcpy(work, W + r * cols, cols * sizeof(float));
        or_fwht64(work, cols);
        size_t stripe = r / STRIPE, lane = r % STRIPE;
        for (size_t c = 0; c < nc; c++) {
            const float *sub = work + c * 64;
            float max_abs = 0.0f;
            for (int i = 0; i < 64; i++) max_abs = fmaxf(max_abs, fabsf(sub[i]));
            if (max_abs <= 1e-12f) continue;
            float best_loss = INFINITY;
            uint16_t best_bf16 = 0;
            uint8_t best_u[64], cand[64];
            memset(best_u, 0, 64);
            for (int k = 0; k < 12; k++) {
                uint16_t d = or_f32_to_bf16((max_abs * ratios[k]) / max_u_f);
                float delta = or_bf16_to_f32(d);
                if (delta <= 0.0f) continue;
                float inv2 = 0.5f / delta;
                float loss = 0.0f;
                for (int j = 0; j < 64; j++) {
                    float wj = sub[j];
                    float t = roundf(wj * inv2 + half_off); /* f32::round: half away from zero */
                    if (t < 0.0f) t = 0.0f;
                    if (t > max_u_f) t = max_u_f;
                    int ui = (int)t;
                    cand[j] = (uint8_t)ui;
                    float diff = wj - ((float)(2 * ui - max_odd)) * delta;
                    loss += diff * diff;
                }
                if (loss < best_loss) {
                    best_loss = loss;
                    best_bf16 = d;
                    memcpy(best_u, cand, 64);
                }
            }
            scales[(stripe * nc + c) * STRIPE + lane] = best_bf16;
            memcpy(u + r * cols + c * 64, best_u, 64);
        }
    }
    free(work);
}

/* simd_lut.rs:1771-1795 FusedBipolarLutMatrix::pack_interleaved
 * -> [num_stripes][cols/8][planes][16]. */
void or_pack_interleaved(const uint8_t *u, size_t rows, size_t cols, int planes, uint8_t *out) {
    size_t opr = cols / 8, stripes = (rows + STRIPE - 1) / STRIPE;
    memset(out, 0, stripes * opr * planes * STRIPE);
    for (size_t r = 0; r < rows; r++) {
        size_t stripe = r / STRIPE, lane = r % STRIPE;
        for (size_t o = 0; o < opr; o++) {
            size_t base = (stripe * opr + o) * planes * STRIPE + lane;
            for (int p = 0; p < planes; p++) {
                uint8_t byte = 0;
                for (int k = 0; k < 8; k++) byte |= (uint8_t)(((u[r * cols + o * 8 + k] >> p) & 1) << k);
                out[base + p * STRIPE] = byte;
            }
        }
    }
}

/* simd_lut.rs:1806-1821 unpack_row_codes. */
void or_unpack_row_codes(const uint8_t *inter, size_t rows, size_t cols, int planes, size_t r,
                         uint8_t *out) {
    (void)rows;
    size_t opr = cols / 8, stripe = r / STRIPE, lane = r % STRIPE;
    for (size_t o = 0; o < opr; o++) {
        size_t base = (stripe * opr + o) * planes * STRIPE + lane;
        for (int k = 0; k < 8; k++) out[o * 8 + k] = 0;
        for (int p = 0; p < planes; p++) {
            uint8_t byte = inter[base + p * STRIPE];
            for (int k = 0; k < 8; k++) out[o * 8 + k] |= (uint8_t)(((byte >> k) & 1) << p);
        }
    }
}

/* ------------------------------------------------------------------ */
/* Nibble4SdotMatrix (simd_lut.rs:3264-3480)                           */
/* ------------------------------------------------------------------ */

size_t or_nibble4_pair_rec(int hp) { return 1024 + 256 * (size_t)hp + 64; }
size_t or_nibble4_tail_rec(int hp) { return 512 + 128 * (size_t)hp + 32; }

/* simd_lut.rs:3297-3400 from_bipolar_with_perm.  Input is the on-disk FusedBipolar body
 * (interleaved planes + BF16 chunk scales). pair_out / tail_out must be sized by the caller. */
void or_nibble4_repack(const uint8_t *inter, const uint16_t *bscales, size_t rows, size_t cols,
                       int planes, int interleave_gate_up, uint8_t *pair_out, uint8_t *tail_out) {
    const int hp = planes - 4;
    const size_t nc = cols / 64, stripes = (rows + STRIPE - 1) / STRIPE;
    const size_t num_pairs = stripes / 2;
    const int has_tail = (int)(stripes & 1);
    const size_t p_rec = or_nibble4_pair_rec(hp), t_rec = or_nibble4_tail_rec(hp);
    memset(pair_out, 0, num_pairs * nc * p_rec);
    if (has_tail) memset(tail_out, 0, nc * t_rec);
    const size_t inter_dim = rows / 2;
    uint8_t *codes = (uint8_t *)malloc(cols);
    for (size_t orig_r = 0; orig_r < rows; orig_r++) {
        or_unpack_row_codes(inter, rows, cols, planes, orig_r, codes);
        size_t r = orig_r;
        if (interleave_gate_up) {
            if (orig_r < inter_dim) r = (orig_r / 64) * 2 * 64 + orig_r % 64;
            else {
                size_t up = orig_r - inter_dim;
                r = ((up / 64) * 2 + 1) * 64 + up % 64;
            }
        }
        size_t orig_stripe = orig_r / STRIPE, orig_lane = orig_r % STRIPE;
        size_t stripe = r / STRIPE, lane = r % STRIPE;
        size_t g = lane / 4, j = lane % 4;
        int in_pair = stripe < num_pairs * 2;
        size_t p = stripe / 2, side = stripe & 1;
        for (size_t c = 0; c < nc; c++) {
            uint16_t sc = bscales[(orig_stripe * nc + c) * STRIPE + orig_lane];
            uint8_t *rec;
            size_t data_off, hi_off, sc_off;
            if (in_pair) {
                rec = pair_out + (p * nc + c) * p_rec;
                data_off = side * 512;
                hi_off = 1024 + side * 128 * hp;
                sc_off = 1024 + 256 * hp + side * 32;
            } else {
                rec = tail_out + c * t_rec;
                data_off = 0;
                hi_off = 512;
                sc_off = 512 + 128 * hp;
            }
            rec[sc_off + lane * 2] = (uint8_t)(sc & 0xFF);
            rec[sc_off + lane * 2 + 1] = (uint8_t)(sc >> 8);
            for (size_t sub_col = 0; sub_col < 64; sub_col++) {
                uint8_t uv = codes[c * 64 + sub_col];
                size_t k = sub_col / 16, w = sub_col % 16;
                size_t half = w / 8, sub = w / 4, t = w % 4;
                size_t byte = data_off + k * 128 + g * 32 + half * 16 + j * 4 + t;
                uint8_t lo = uv & 0x0F;
                rec[byte] |= (w % 8) < 4 ? lo : (uint8_t)(lo << 4);
                if (hp == 1) {
                    size_t hb = hi_off + (k / 2) * 64 + g * 16 + j * 4 + t;
                    int bit = (k & 1) == 0 ? 4 + (int)sub : (int)sub;
                    rec[hb] |= (uint8_t)(((uv >> 4) & 1) << bit);
                } else if (hp == 2) {
                    size_t hb = hi_off + k * 64 + g * 16 + j * 4 + t;
                    static const int shifts[4] = {4, 6, 2, 0};
                    rec[hb] |= (uint8_t)(((uv >> 4) & 3) << shifts[sub]);
                }
            }
        }
    }
    free(codes);
}

/* simd_lut.rs:3411-3436 stripe_chunk_ptrs. */
static void n4_ptrs(const uint8_t *pair, const uint8_t *tail, size_t rows, size_t cols, int hp,
                    size_t stripe, size_t c, const uint8_t **d, const uint8_t **h, const uint8_t **s) {
    size_t nc = cols / 64, stripes = (rows + STRIPE - 1) / STRIPE, np = stripes / 2;
    if (stripe < np * 2) {
        const uint8_t *base = pair + ((stripe / 2) * nc + c) * or_nibble4_pair_rec(hp);
        size_t side = stripe & 1;
        *d = base + side * 512;
        *h = base + 1024 + side * 128 * hp;
        *s = base + 1024 + 256 * hp + side * 32;
    } else {
        const uint8_t *base = tail + c * or_nibble4_tail_rec(hp);
        *d = base;
        *h = base + 512;
        *s = base + 512 + 128 * hp;
    }
}

/* Unsigned code u (0..2^(4+hp)-1) of (row r, column col), simd_lut.rs:3439-3480. */
static int n4_code(const uint8_t *d, const uint8_t *h, int hp, size_t lane, size_t sub_col) {
    size_t g = lane / 4, j = lane % 4, k = sub_col / 16, w = sub_col % 16, sub = w / 4, t = w % 4;
    uint8_t byte = d[k * 128 + g * 32 + (w / 8) * 16 + j * 4 + t];
    int uv = (w % 8) < 4 ? (byte & 0x0F) : (byte >> 4);
    if (hp == 1) {
        uint8_t hb = h[(k / 2) * 64 + g * 16 + j * 4 + t];
        int bit = (k & 1) == 0 ? 4 + (int)sub : (int)sub;
        uv |= ((hb >> bit) & 1) << 4;
    } else if (hp == 2) {
        static const int shifts[4] = {4, 6, 2, 0};
        uint8_t hb = h[k * 64 + g * 16 + j * 4 + t];
        uv |= ((hb >> shifts[sub]) & 3) << 4;
    }
    return uv;
}

static float rd_bf16(const uint8_t *p) { return or_bf16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

/* simd_lut.rs:3439-3480 dequantize_row_rotated. */
void or_nibble4_dequant_row(const uint8_t *pair, const uint8_t *tail, size_t rows, size_t cols,
                            int hp, size_t r, float *out) {
    size_t stripe = r / STRIPE, lane = r % STRIPE, nc = cols / 64;
    int max_odd = (1 << (4 + hp)) - 1;
    for (size_t c = 0; c < nc; c++) {
        const uint8_t *d, *h, *s;
        n4_ptrs(pair, tail, rows, cols, hp, stripe, c, &d, &h, &s);
        float delta = rd_bf16(s + lane * 2);
        for (size_t sc = 0; sc < 64; sc++)
            out[c * 64 + sc] = ((float)(2 * n4_code(d, h, hp, lane, sc) - max_odd)) * delta;
    }
}

/* Raw codes of row r (for tests of the layout). */
void or_nibble4_row_codes(const uint8_t *pair, const uint8_t *tail, size_t rows, size_t cols,
                          int hp, size_t r, uint8_t *out) {
    size_t stripe = r / STRIPE, lane = r % STRIPE, nc = cols / 64;
    for (size_t c = 0; c < nc; c++) {
        const uint8_t *d, *h, *s;
        n4_ptrs(pair, tail, rows, cols, hp, stripe, c, &d, &h, &s);
        for (size_t sc = 0; sc < 64; sc++) out[c * 64 + sc] = (uint8_t)n4_code(d, h, hp, lane, sc);
    }
}

/* simd_lut.rs:3766-4091 sdot_decode_neon semantics: per (row, chunk) acc = sum u*xq (i32),
 * dot = 2*acc - M*sums[c]; per row f = fma(float(dot)*sx[c], ws[r,c], f), c ascending, chunks
 * with sx == 0 skipped.  `dots` (optional) receives [rows][nc] integer dots. */
void or_nibble4_gemv(const uint8_t *pair, const uint8_t *tail, size_t rows, size_t cols, int hp,
                     const int8_t *xq, const float *xs, const int32_t *xsum, size_t s0, size_t s1,
                     float *out, int32_t *dots) {
    size_t nc = cols / 64;
    int max_odd = (1 << (4 + hp)) - 1;
    for (size_t s = s0; s < s1; s++) {
        for (size_t lane = 0; lane < STRIPE; lane++) {
            size_t r = s * STRIPE + lane;
            if (r >= rows) break;
            float f = 0.0f;
            for (size_t c = 0; c < nc; c++) {
                const uint8_t *d, *h, *sp;
                n4_ptrs(pair, tail, rows, cols, hp, s, c, &d, &h, &sp);
                int32_t acc = 0;
                for (size_t sc = 0; sc < 64; sc++) acc += n4_code(d, h, hp, lane, sc) * (int32_t)xq[c * 64 + sc];
                int32_t dot = 2 * acc - max_odd * xsum[c];
                if (dots) dots[r * nc + c] = dot;
                if (xs[c] == 0.0f) continue;
                float ws = rd_bf16(sp + lane * 2);
                f = fmaf((float)dot * xs[c], ws, f);
            }
            out[r] = f;
        }
    }
}

/* simd_lut.rs:3558-3581 (non-aarch64 branch of nibble4_sdot_stripe_range_raw): dequantize the
 * row to f32, f32 dot per chunk (sequential), acc += dot * sx. The portable CPU baseline. */
void or_nibble4_gemv_portable(const uint8_t *pair, const uint8_t *tail, size_t rows, size_t cols,
                              int hp, const int8_t *xq, const float *xs, size_t s0, size_t s1,
                              float *out) {
    size_t nc = cols / 64;
    float *row = (float *)malloc(cols * sizeof(float));
    for (size_t s = s0; s < s1; s++) {
        for (size_t lane = 0; lane < STRIPE; lane++) {
            size_t r = s * STRIPE + lane;
            if (r >= rows) break;
            or_nibble4_dequant_row(pair, tail, rows, cols, hp, r, row);
            float acc = 0.0f;
            for (size_t c = 0; c < nc; c++) {
                float dot = 0.0f;
                for (int i = 0; i < 64; i++) dot += row[c * 64 + i] * (float)xq[c * 64 + i];
                acc += dot * xs[c];
            }
            out[r] = acc;
        }
    }
    free(row);
}

/* ------------------------------------------------------------------ */
/* NF codebook stripes (simd_lut.rs:4338-5748, compiler.rs:1404-1866)  */
/* ------------------------------------------------------------------ */

static const int8_t NF5_POS[16] = {3, 8, 13, 19, 24, 30, 36, 42, 49, 56, 64, 72, 82, 93, 107, 127};
static const int8_t NF4_DEF[16] = {-127, -96, -75, -58, -44, -31, -18, -6, 6, 18, 31, 44, 58, 75, 96, 127};
static const int8_t NF3_DEF[16] = {-127, -79, -45, -14, 14, 45, 79, 127, 0, 0, 0, 0, 0, 0, 0, 0};

/* simd_lut.rs:4636-4647 nf_expand_codebook32. */
void or_nf_expand_codebook32(int bits, const int8_t *cb16, int8_t *out32) {
    memset(out32, 0, 32);
    if (bits == 5) {
        for (int m = 0; m < 16; m++) {
            out32[15 - m] = (int8_t)(-cb16[m]);
            out32[16 + m] = cb16[m];
        }
    } else {
        memcpy(out32, cb16, 16);
    }
}

size_t or_nf_chunk_bytes(int bits) { return bits == 5 ? 640 : bits == 4 ? 512 : bits == 3 ? 384 : 256; }

size_t or_nf_pair_total(size_t cols, int bits, size_t sgc) {
    size_t nc = cols / 64, nsg = (nc + sgc - 1) / sgc;
    return nsg * 64 + nc * 2 * or_nf_chunk_bytes(bits);
}

size_t or_nf_tail_total(size_t cols, int bits, size_t sgc) {
    size_t nc = cols / 64, nsg = (nc + sgc - 1) / sgc;
    return nsg * 32 + nc * or_nf_chunk_bytes(bits);
}

/* compiler.rs:1404-1526 fit_empirical_nf_codebook.  Returns mu_top; writes the i8[16] codebook. */
float or_nf_fit_codebook(const float *W, size_t rows, size_t cols, int bits, size_t sgc, int8_t *cb) {
    enum { HIST_BINS = 2000 };
    const float Z_MAX = 5.0f;
    const float BIN_W = Z_MAX / (float)HIST_BINS;
    size_t nc = cols / 64;
    if (sgc < 1) sgc = 1;
    size_t nsg = (nc + sgc - 1) / sgc;
    size_t step = rows / 512;
    if (step < 1) step = 1;
    uint64_t *hist = (uint64_t *)calloc(HIST_BINS, sizeof(uint64_t));
    uint64_t total = 0;
    float *row = (float *)malloc(cols * sizeof(float));
    for (size_t r = 0; r < rows; r += step) {
        memcpy(row, W + r * cols, cols * sizeof(float));
        or_fwht64(row, cols);
        for (size_t sg = 0; sg < nsg; sg++) {
            size_t cs = sg * sgc * 64, ce = (sg + 1) * sgc * 64;
            if (ce > cols) ce = cols;
            float sum_sq = 0.0f;
            for (size_t i = cs; i < ce; i++) sum_sq += row[i] * row[i];
            float rms = sqrtf(sum_sq / (float)(ce - cs));
            if (rms <= 1e-12f) continue;
            float inv_rms = 1.0f / rms;
            for (size_t i = cs; i < ce; i++) {
                float z = fabsf(row[i]) * inv_rms;
                float q = z / BIN_W;
                size_t bin = q >= (float)HIST_BINS ? HIST_BINS - 1 : (size_t)q; /* `as usize` then min */
                if (bin > HIST_BINS - 1) bin = HIST_BINS - 1;
                hist[bin]++;
                total++;
            }
        }
    }
    free(row);
    if (total < 256) {
        free(hist);
        memcpy(cb, bits == 5 ? NF5_POS : bits == 4 ? NF4_DEF : NF3_DEF, 16);
        return bits == 5 ? 3.25f : bits == 4 ? 2.7326f : 2.1520f;
    }
    int half = 1 << (bits - 1);
    double mu[16];
    static const double mu5[16] = {0.068, 0.205, 0.343, 0.483, 0.626, 0.773, 0.925, 1.084,
                                   1.252, 1.432, 1.628, 1.845, 2.092, 2.382, 2.743, 3.250};
    static const double mu4[8] = {0.1284, 0.3881, 0.6568, 0.9424, 1.2562, 1.6180, 2.0690, 2.7326};
    static const double mu3[4] = {0.2451, 0.7560, 1.3439, 2.1520};
    memcpy(mu, bits == 5 ? mu5 : bits == 4 ? mu4 : mu3, (size_t)half * sizeof(double));
    for (int it = 0; it < 24; it++) {
        size_t bounds[17];
        bounds[0] = 0;
        bounds[half] = HIST_BINS;
        for (int m = 0; m < half - 1; m++) {
            double mid = 0.5 * (mu[m] + mu[m + 1]);
            double rb = round(mid / (double)BIN_W);
            size_t b = rb <= 0.0 ? 0 : (size_t)rb;
            if (b < bounds[m]) b = bounds[m];
            if (b > HIST_BINS) b = HIST_BINS;
            bounds[m + 1] = b;
        }
        for (int m = 0; m < half; m++) {
            double w_sum = 0.0;
            uint64_t c_sum = 0;
            for (size_t b = bounds[m]; b < bounds[m + 1]; b++) {
                uint64_t cnt = hist[b];
                if (cnt > 0) {
                    double x = ((double)b + 0.5) * (double)BIN_W;
                    w_sum += (double)cnt * x;
                    c_sum += cnt;
                }
            }
            if (c_sum > 0) mu[m] = w_sum / (double)c_sum;
        }
        for (int m = 1; m < half; m++)
            if (mu[m] <= mu[m - 1] + 1e-4) mu[m] = mu[m - 1] + 0.05;
    }
    free(hist);
    double mu_top = mu[half - 1] > 0.5 ? mu[half - 1] : 0.5;
    int q_pos[16];
    for (int m = 0; m < half; m++) {
        int v = (int)round(127.0 * mu[m] / mu_top);
        q_pos[m] = v < 1 ? 1 : v > 127 ? 127 : v;
    }
    q_pos[half - 1] = 127;
    for (int m = half - 2; m >= 0; m--)
        if (q_pos[m] >= q_pos[m + 1]) q_pos[m] = (q_pos[m + 1] - 1) > 1 ? q_pos[m + 1] - 1 : 1;
    for (int m = 1; m < half; m++)
        if (q_pos[m] <= q_pos[m - 1]) q_pos[m] = (q_pos[m - 1] + 1) < 127 ? q_pos[m - 1] + 1 : 127;
    memset(cb, 0, 16);
    if (bits == 5) {
        for (int m = 0; m < 16; m++) cb[m] = (int8_t)q_pos[m];
    } else {
        for (int m = 0; m < half; m++) {
            cb[half - 1 - m] = (int8_t)(-q_pos[m]);
            cb[half + m] = (int8_t)q_pos[m];
        }
    }
    return (float)mu_top;
}

/* compiler.rs:1660-1699 quant_nearest (decision tree over midpoint thresholds). */
static size_t nf_quant_nearest(float w, float inv_delta, int bits, const float *th) {
    float aw = fabsf(w) * inv_delta;
    size_t half = (size_t)1 << (bits - 1), mag;
    if (bits == 5) {
        if (aw < th[7]) {
            if (aw < th[3]) mag = aw < th[1] ? (size_t)(aw >= th[0]) : 2 + (size_t)(aw >= th[2]);
            else mag = aw < th[5] ? 4 + (size_t)(aw >= th[4]) : 6 + (size_t)(aw >= th[6]);
        } else if (aw < th[11]) {
            mag = aw < th[9] ? 8 + (size_t)(aw >= th[8]) : 10 + (size_t)(aw >= th[10]);
        } else {
            mag = aw < th[13] ? 12 + (size_t)(aw >= th[12]) : 14 + (size_t)(aw >= th[14]);
        }
    } else if (bits == 4) {
        if (aw < th[3]) mag = aw < th[1] ? (size_t)(aw >= th[0]) : 2 + (size_t)(aw >= th[2]);
        else mag = aw < th[5] ? 4 + (size_t)(aw >= th[4]) : 6 + (size_t)(aw >= th[6]);
    } else {
        mag = aw < th[1] ? (size_t)(aw >= th[0]) : 2 + (size_t)(aw >= th[2]);
    }
    return w >= 0.0f ? half + mag : half - 1 - mag;
}

/* compiler.rs:1628-1866 quantize_stripe_batch_nf, hessian = None.
 * idx [rows*cols]; scales [num_stripes][num_scale_groups][16] BF16. */
void or_nf_rtn(const float *W, size_t rows, size_t cols, int bits, size_t sgc, const int8_t *cb16,
               float mu_top, uint8_t *idx, uint16_t *scales) {
    static const float ratios[11] = {0.74f, 0.80f, 0.86f, 0.91f, 0.96f, 1.00f,
                                     1.04f, 1.09f, 1.15f, 1.22f, 1.30f};
    const size_t half = (size_t)1 << (bits - 1), levels = (size_t)1 << bits;
    int8_t cb32[32];
    or_nf_expand_codebook32(bits, cb16, cb32);
    float cb_f[32] = {0};
    for (size_t k = 0; k < levels; k++) cb_f[k] = (float)cb32[k];
    float th[15] = {0};
    for (size_t m = 0; m + 1 < half; m++) th[m] = 0.5f * (cb_f[half + m] + cb_f[half + m + 1]);
    const size_t nc = cols / 64, nsg = (nc + sgc - 1) / sgc, stripes = (rows + STRIPE - 1) / STRIPE;
    memset(scales, 0, stripes * nsg * STRIPE * sizeof(uint16_t));
    float *work = (float *)malloc(cols * sizeof(float));
    uint8_t *best = (uint8_t *)malloc(sgc * 64), *cand = (uint8_t *)malloc(sgc * 64);
    for (size_t r = 0; r < rows; r++) {
        memcpy(work, W + r * cols, cols * sizeof(float));
        or_fwht64(work, cols);
        size_t stripe = r / STRIPE, lane = r % STRIPE;
        for (size_t sg = 0; sg < nsg; sg++) {
            size_t c_start = sg * sgc, c_end = c_start + sgc < nc ? c_start + sgc : nc;
            size_t cs = c_start * 64, glen = (c_end - c_start) * 64;
            const float *sub = work + cs;
            float sum_sq = 0.0f;
            for (size_t j = 0; j < glen; j++) sum_sq += sub[j] * sub[j];
            float rms = sqrtf(sum_sq / (float)glen);
            if (rms <= 1e-12f) {
                memset(idx + r * cols + cs, (int)(half - 1), glen);
                scales[(stripe * nsg + sg) * STRIPE + lane] = 0;
                continue;
            }
            float base_delta = rms * (mu_top / 127.0f);
            float best_loss = INFINITY;
            uint16_t best_bf16 = 0;
            memset(best, 0, glen);
            for (int e = 0; e < 12; e++) {
                uint16_t d;
                if (e < 11) {
                    d = or_f32_to_bf16(base_delta * ratios[e]);
                } else {
                    /* least-squares BF16 refit on the chosen centroids (compiler.rs:1826-1844) */
                    float dot_wc = 0.0f, dot_cc = 0.0f;
                    for (size_t j = 0; j < glen; j++) {
                        float cv = cb_f[best[j]];
                        dot_wc += sub[j] * cv;
                        dot_cc += cv * cv;
                    }
                    if (!(dot_cc > 1e-12f && dot_wc > 0.0f)) break;
                    d = or_f32_to_bf16(dot_wc / dot_cc);
                    if (d == best_bf16) break;
                }
                float delta = or_bf16_to_f32(d);
                if (delta <= 0.0f) continue;
                float inv_delta = 1.0f / delta;
                float loss = 0.0f;
                for (size_t j = 0; j < glen; j++) {
                    size_t k = nf_quant_nearest(sub[j], inv_delta, bits, th);
                    cand[j] = (uint8_t)k;
                    float diff = sub[j] - cb_f[k] * delta;
                    loss += diff * diff;
                }
                if (loss < best_loss) {
                    best_loss = loss;
                    best_bf16 = d;
                    memcpy(best, cand, glen);
                }
            }
            scales[(stripe * nsg + sg) * STRIPE + lane] = best_bf16;
            memcpy(idx + r * cols + cs, best, glen);
        }
    }
    free(work);
    free(best);
    free(cand);
}

/* simd_lut.rs:4874-4960 pack_one_stripe_chunk. */
static void nf_pack_stripe_chunk(const uint8_t *idx, size_t rows, size_t cols, int bits,
                                 size_t stripe, size_t c, uint8_t *dst) {
#define IDX(lane, sc) (((stripe) * STRIPE + (lane)) < rows ? idx[((stripe) * STRIPE + (lane)) * cols + (c) * 64 + (sc)] : 0)
    if (bits == 4 || bits == 5) {
        for (size_t k = 0; k < 4; k++)
            for (size_t g = 0; g < 4; g++)
                for (size_t j = 0; j < 4; j++) {
                    size_t lane = g * 4 + j;
                    for (size_t t = 0; t < 4; t++) {
                        uint8_t lo0 = IDX(lane, k * 16 + t) & 0x0F, hi0 = IDX(lane, k * 16 + 4 + t) & 0x0F;
                        dst[k * 128 + g * 32 + j * 4 + t] = (uint8_t)(lo0 | (hi0 << 4));
                        uint8_t lo1 = IDX(lane, k * 16 + 8 + t) & 0x0F, hi1 = IDX(lane, k * 16 + 12 + t) & 0x0F;
                        dst[k * 128 + g * 32 + 16 + j * 4 + t] = (uint8_t)(lo1 | (hi1 << 4));
                    }
                }
        if (bits == 5) {
            for (size_t g = 0; g < 4; g++)
                for (size_t kp = 0; kp < 2; kp++) {
                    size_t k0 = kp * 2, k1 = k0 + 1;
                    uint8_t *blk = dst + 512 + g * 32 + kp * 16;
                    for (size_t j = 0; j < 4; j++) {
                        size_t lane = g * 4 + j;
                        for (size_t t = 0; t < 4; t++) {
                            uint8_t v = 0;
                            v |= (uint8_t)(((IDX(lane, k0 * 16 + t) >> 4) & 1) << 4);
                            v |= (uint8_t)(((IDX(lane, k0 * 16 + 4 + t) >> 4) & 1) << 5);
                            v |= (uint8_t)(((IDX(lane, k0 * 16 + 8 + t) >> 4) & 1) << 6);
                            v |= (uint8_t)(((IDX(lane, k0 * 16 + 12 + t) >> 4) & 1) << 7);
                            v |= (uint8_t)((IDX(lane, k1 * 16 + t) >> 4) & 1);
                            v |= (uint8_t)(((IDX(lane, k1 * 16 + 4 + t) >> 4) & 1) << 1);
                            v |= (uint8_t)(((IDX(lane, k1 * 16 + 8 + t) >> 4) & 1) << 2);
                            v |= (uint8_t)(((IDX(lane, k1 * 16 + 12 + t) >> 4) & 1) << 3);
                            blk[j * 4 + t] = v;
                        }
                    }
                }
        }
    } else {
        for (size_t kp = 0; kp < 2; kp++) {
            size_t k0 = kp * 2, k1 = k0 + 1;
            for (size_t g = 0; g < 4; g++) {
                uint8_t *blk = dst + kp * 192 + g * 48;
                for (size_t j = 0; j < 4; j++) {
                    size_t lane = g * 4 + j;
                    for (size_t t = 0; t < 4; t++) {
                        size_t b = j * 4 + t;
                        uint8_t i0 = IDX(lane, k0 * 16 + t) & 7, i1 = IDX(lane, k0 * 16 + 4 + t) & 7;
                        uint8_t i2 = IDX(lane, k0 * 16 + 8 + t) & 7, i3 = IDX(lane, k0 * 16 + 12 + t) & 7;
                        uint8_t i4 = IDX(lane, k1 * 16 + t) & 7, i5 = IDX(lane, k1 * 16 + 4 + t) & 7;
                        uint8_t i6 = IDX(lane, k1 * 16 + 8 + t) & 7, i7 = IDX(lane, k1 * 16 + 12 + t) & 7;
                        blk[b] = (uint8_t)(i0 | (i1 << 3) | ((i2 & 3) << 6));
                        blk[16 + b] = (uint8_t)(i3 | (i4 << 3) | ((i5 & 3) << 6));
                        blk[32 + b] = (uint8_t)(i6 | (i7 << 3) | (((i2 >> 2) & 1) << 6) | (((i5 >> 2) & 1) << 7));
                    }
                }
            }
        }
    }
#undef IDX
}

/* simd_lut.rs:4850-5023 NfSdotMatrix::from_indices. */
void or_nf_from_indices(const uint8_t *idx, const uint16_t *scales, size_t rows, size_t cols,
                        int bits, size_t sgc, uint8_t *pair_out, uint8_t *tail_out) {
    size_t stripes = (rows + STRIPE - 1) / STRIPE, np = stripes / 2, nc = cols / 64;
    size_t nsg = (nc + sgc - 1) / sgc, cb = or_nf_chunk_bytes(bits);
    size_t ptot = or_nf_pair_total(cols, bits, sgc), ttot = or_nf_tail_total(cols, bits, sgc);
    memset(pair_out, 0, np * ptot);
    for (size_t p = 0; p < np; p++) {
        size_t sa = 2 * p, sb = sa + 1, cur = p * ptot;
        for (size_t sg = 0; sg < nsg; sg++) {
            for (size_t lane = 0; lane < STRIPE; lane++) {
                uint16_t ua = scales[(sa * nsg + sg) * STRIPE + lane], ub = scales[(sb * nsg + sg) * STRIPE + lane];
                pair_out[cur + lane * 2] = (uint8_t)ua;
                pair_out[cur + lane * 2 + 1] = (uint8_t)(ua >> 8);
                pair_out[cur + 32 + lane * 2] = (uint8_t)ub;
                pair_out[cur + 32 + lane * 2 + 1] = (uint8_t)(ub >> 8);
            }
            cur += 64;
            size_t c0 = sg * sgc, c1 = c0 + sgc < nc ? c0 + sgc : nc;
            for (size_t c = c0; c < c1; c++) {
                nf_pack_stripe_chunk(idx, rows, cols, bits, sa, c, pair_out + cur);
                nf_pack_stripe_chunk(idx, rows, cols, bits, sb, c, pair_out + cur + cb);
                cur += 2 * cb;
            }
        }
    }
    if (stripes & 1) {
        memset(tail_out, 0, ttot);
        size_t st = np * 2, cur = 0;
        for (size_t sg = 0; sg < nsg; sg++) {
            for (size_t lane = 0; lane < STRIPE; lane++) {
                uint16_t ut = scales[(st * nsg + sg) * STRIPE + lane];
                tail_out[cur + lane * 2] = (uint8_t)ut;
                tail_out[cur + lane * 2 + 1] = (uint8_t)(ut >> 8);
            }
            cur += 32;
            size_t c0 = sg * sgc, c1 = c0 + sgc < nc ? c0 + sgc : nc;
            for (size_t c = c0; c < c1; c++) {
                nf_pack_stripe_chunk(idx, rows, cols, bits, st, c, tail_out + cur);
                cur += cb;
            }
        }
    }
}

/* simd_lut.rs:5527-5555 stripe_chunk_ptrs. */
static void nf_ptrs(const uint8_t *pair, const uint8_t *tail, size_t rows, size_t cols, int bits,
                    size_t sgc, size_t stripe, size_t c, const uint8_t **d, const uint8_t **s) {
    size_t stripes = (rows + STRIPE - 1) / STRIPE, np = stripes / 2;
    size_t sg = c / sgc, sub_c = c % sgc, c_start = sg * sgc, cb = or_nf_chunk_bytes(bits);
    if (stripe < np * 2) {
        size_t side = stripe & 1;
        const uint8_t *sgp = pair + (stripe / 2) * or_nf_pair_total(cols, bits, sgc) + sg * 64 + c_start * 2 * cb;
        *s = sgp + side * 32;
        *d = sgp + 64 + sub_c * 2 * cb + side * cb;
    } else {
        const uint8_t *sgp = tail + sg * 32 + c_start * cb;
        *s = sgp;
        *d = sgp + 32 + sub_c * cb;
    }
}

/* Index of (lane, sub_col) inside one stripe-chunk record, simd_lut.rs:5558-5634. */
static int nf_index(const uint8_t *d, int bits, size_t lane, size_t sc) {
    size_t g = lane / 4, j = lane % 4;
    if (bits == 4 || bits == 5) {
        size_t k = sc / 16, w = sc % 16, sub4 = w / 4, t = w % 4, b = j * 4 + t;
        uint8_t byte = d[k * 128 + g * 32 + (sub4 / 2) * 16 + b];
        int lo4 = (sub4 & 1) == 0 ? (byte & 0x0F) : (byte >> 4);
        if (bits == 5) {
            uint8_t hb = d[512 + g * 32 + (k / 2) * 16 + b];
            int shift = (k & 1) == 0 ? 4 + (int)sub4 : (int)sub4;
            return lo4 | (((hb >> shift) & 1) << 4);
        }
        return lo4;
    }
    /* NF3 */
    size_t kk = sc / 16, w = sc % 16, quad = w / 4, t = w % 4, kp = kk / 2, b = j * 4 + t;
    const uint8_t *blk = d + kp * 192 + g * 48;
    uint8_t v0 = blk[b], v1 = blk[16 + b], v2 = blk[32 + b];
    int ids[8] = {v0 & 7, (v0 >> 3) & 7, ((v0 >> 6) & 3) | (((v2 >> 6) & 1) << 2), v1 & 7,
                  (v1 >> 3) & 7, ((v1 >> 6) & 3) | (((v2 >> 7) & 1) << 2), v2 & 7, (v2 >> 3) & 7};
    return ids[(kk & 1) * 4 + quad];
}

void or_nf_row_indices(const uint8_t *pair, const uint8_t *tail, size_t rows, size_t cols, int bits,
                       size_t sgc, size_t r, uint8_t *out) {
    size_t stripe = r / STRIPE, lane = r % STRIPE;
    for (size_t c = 0; c < cols / 64; c++) {
        const uint8_t *d, *s;
        nf_ptrs(pair, tail, rows, cols, bits, sgc, stripe, c, &d, &s);
        for (size_t sc = 0; sc < 64; sc++) out[c * 64 + sc] = (uint8_t)nf_index(d, bits, lane, sc);
    }
}

/* simd_lut.rs:5558-5634 dequantize_row_rotated. */
void or_nf_dequant_row(const uint8_t *pair, const uint8_t *tail, size_t rows, size_t cols, int bits,
                       size_t sgc, const int8_t *cb16, size_t r, float *out) {
    int8_t cb32[32];
    or_nf_expand_codebook32(bits, cb16, cb32);
    size_t stripe = r / STRIPE, lane = r % STRIPE;
    for (size_t c = 0; c < cols / 64; c++) {
        const uint8_t *d, *s;
        nf_ptrs(pair, tail, rows, cols, bits, sgc, stripe, c, &d, &s);
        float delta = rd_bf16(s + lane * 2);
        for (size_t sc = 0; sc < 64; sc++) out[c * 64 + sc] = (float)cb32[nf_index(d, bits, lane, sc)] * delta;
    }
}

/* simd_lut.rs:6074-6364 nf_sdot_decode_neon semantics: a = sum cb[idx]*xq (i32) per (row, chunk);
 * f = fma(float(a)*sx[c], ws[r, c/sgc], f), c ascending, sx == 0 skipped. */
void or_nf_gemv(const uint8_t *pair, const uint8_t *tail, size_t rows, size_t cols, int bits,
                size_t sgc, const int8_t *cb16, const int8_t *xq, const float *xs, size_t s0,
                size_t s1, float *out, int32_t *dots) {
    int8_t cb32[32];
    or_nf_expand_codebook32(bits, cb16, cb32);
    size_t nc = cols / 64;
    for (size_t s = s0; s < s1; s++) {
        for (size_t lane = 0; lane < STRIPE; lane++) {
            size_t r = s * STRIPE + lane;
            if (r >= rows) break;
            float f = 0.0f;
            for (size_t c = 0; c < nc; c++) {
                const uint8_t *d, *sp;
                nf_ptrs(pair, tail, rows, cols, bits, sgc, s, c, &d, &sp);
                int32_t a = 0;
                for (size_t sc = 0; sc < 64; sc++) a += (int32_t)cb32[nf_index(d, bits, lane, sc)] * (int32_t)xq[c * 64 + sc];
                if (dots) dots[r * nc + c] = a;
                if (xs[c] == 0.0f) continue;
                f = fmaf((float)a * xs[c], rd_bf16(sp + lane * 2), f);
            }
            out[r] = f;
        }
    }
}

/* simd_lut.rs:5719-5748 nf_sdot_stripe_range_scalar_raw (portable CPU baseline). */
void or_nf_gemv_portable(const uint8_t *pair, const uint8_t *tail, size_t rows, size_t cols, int bits,
                         size_t sgc, const int8_t *cb16, const int8_t *xq, const float *xs, size_t s0,
                         size_t s1, float *out) {
    size_t nc = cols / 64;
    float *row = (float *)malloc(cols * sizeof(float));
    for (size_t s = s0; s < s1; s++)
        for (size_t lane = 0; lane < STRIPE; lane++) {
            size_t r = s * STRIPE + lane;
            if (r >= rows) break;
            or_nf_dequant_row(pair, tail, rows, cols, bits, sgc, cb16, r, row);
            float acc = 0.0f;
            for (size_t c = 0; c < nc; c++) {
                float dot = 0.0f;
                for (int i = 0; i < 64; i++) dot += row[c * 64 + i] * (float)xq[c * 64 + i];
                acc += dot * xs[c];
            }
            out[r] = acc;
        }
    free(row);
}

/* ------------------------------------------------------------------ */
/* Hadamard int8 KV cache + q8 attention (real_llm.rs)                  */
/* ------------------------------------------------------------------ */

/* real_llm.rs:8282-8365 store_hadamard_q8_head{64,128}_raw (portable branch): FWHT-64 per block
 * (block index 0, 1 within the head), one max over the whole head, int8 + one f32 scale. */
void or_kv_quant_head(const float *src, size_t hd, int8_t *q, float *scale) {
    float rot[128];
    memcpy(rot, src, hd * sizeof(float));
    or_fwht64(rot, hd);
    float max_abs = 0.0f;
    for (size_t i = 0; i < hd; i++) max_abs = fmaxf(max_abs, fabsf(rot[i]));
    if (max_abs <= FLT_EPSILON) {
        memset(q, 0, hd);
        *scale = 0.0f;
        return;
    }
    float inv = 127.0f / max_abs;
    for (size_t i = 0; i < hd; i++) q[i] = (int8_t)(int32_t)rintf(rot[i] * inv);
    *scale = max_abs / 127.0f;
}

/* real_llm.rs:8471-8594 causal_gqa_group_q8, portable branches (8533-8545, 8575-8585) and
 * softmax_unnorm_inplace (9585-9600).  One query head over `seq` positions of one KV head.
 * `scores` is scratch of `seq` floats.  Output is back in the unrotated domain (IFWHT). */
void or_attn_q8_head(const float *q_head, const int8_t *k_q8, const float *ks, const int8_t *v_q8,
                     const float *vs, size_t seq, size_t hd, float attn_scale, float *out,
                     float *scores) {
    int8_t qi[128];
    float q_scale;
    or_kv_quant_head(q_head, hd, qi, &q_scale);
    float qas = q_scale * attn_scale;
    for (size_t t = 0; t < seq; t++) {
        int32_t dot = 0;
        for (size_t i = 0; i < hd; i++) dot += (int32_t)qi[i] * (int32_t)k_q8[t * hd + i];
        scores[t] = (float)dot * ks[t] * qas;
    }
    float mx = -INFINITY;
    for (size_t t = 0; t < seq; t++) mx = fmaxf(mx, scores[t]);
    float sum = 0.0f;
    for (size_t t = 0; t < seq; t++) {
        scores[t] = expf(scores[t] - mx);
        sum += scores[t];
    }
    float inv = 1.0f / sum;
    for (size_t i = 0; i < hd; i++) out[i] = 0.0f;
    for (size_t t = 0; t < seq; t++) {
        float w = (scores[t] * inv) * vs[t];
        for (size_t i = 0; i < hd; i++) out[i] += w * (float)v_q8[t * hd + i];
    }
    or_ifwht64(out, hd);
}

/* causal_gqa_group_q4_or_window, int8 branch (real_llm.rs:8794-8937): the sliding-window
 * path forms each score from per-64-block dots, total += float(dot_g) * ks * qs, and
 * skips positions whose weight p_norm * vs is zero.  k/v rows are the attended
 * positions, already gathered in active_kv_pos order. */
void or_attn_q8_head_window(const float *q_head, const int8_t *k_q8, const float *ks, const int8_t *v_q8,
                            const float *vs, size_t seq, size_t hd, float attn_scale, float *out,
                            float *scores) {
    int8_t qi[128];
    float q_scale;
    or_kv_quant_head(q_head, hd, qi, &q_scale);
    float qas = q_scale * attn_scale;
    for (size_t t = 0; t < seq; t++) {
        float total = 0.0f;
        for (size_t g = 0; g < hd / 64; g++) {
            int32_t dot = 0;
            for (size_t i = 0; i < 64; i++) dot += (int32_t)qi[g * 64 + i] * (int32_t)k_q8[t * hd + g * 64 + i];
            total += (float)dot * ks[t] * qas;
        }
        scores[t] = total;
    }
    float mx = -INFINITY;
    for (size_t t = 0; t < seq; t++) mx = fmaxf(mx, scores[t]);
    float sum = 0.0f;
    for (size_t t = 0; t < seq; t++) {
        scores[t] = expf(scores[t] - mx);
        sum += scores[t];
    }
    float inv = 1.0f / sum;
    for (size_t i = 0; i < hd; i++) out[i] = 0.0f;
    for (size_t t = 0; t < seq; t++) {
        float w = (scores[t] * inv) * vs[t];
        if (w == 0.0f) continue;
        for (size_t i = 0; i < hd; i++) out[i] += w * (float)v_q8[t * hd + i];
    }
    or_ifwht64(out, hd);
}

/* ------------------------------------------------------------------ */
/* Small fp32 glue (real_llm.rs)                                         */
/* ------------------------------------------------------------------ */

/* real_llm.rs:9212-9232 build_rope_table row for `pos`: [cos(half) | sin(half)]. */
void or_rope_row(size_t hd, double theta, size_t pos, float *row) {
    size_t half = hd / 2;
    for (size_t i = 0; i < half; i++) {
        double e = (double)(2 * i) / (double)hd;
        float freq = (float)(1.0 / pow(theta, e));
        float ang = (float)pos * freq;
        row[i] = cosf(ang);
        row[half + i] = sinf(ang);
    }
}

/* real_llm.rs:9328-9361 apply_llama_rope_precomp (half-split rotation). */
void or_rope_apply(float *head, size_t hd, const float *row) {
    size_t half = hd / 2;
    for (size_t i = 0; i < half; i++) {
        float x0 = head[i], x1 = head[half + i], c = row[i], s = row[half + i];
        head[i] = x0 * c - x1 * s;
        head[half + i] = x1 * c + x0 * s;
    }
}

/* real_llm.rs:9801-9805 swiglu_activate_scalar. */
void or_swiglu(const float *g, const float *u, float *out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = (g[i] / (1.0f + expf(-g[i]))) * u[i];
}

/* ------------------------------------------------------------------ */
/* NF4 Hadamard KV cache (real_llm.rs:8614-8700, 8794-8937)             */
/* ------------------------------------------------------------------ */

static const int8_t OR_NF4_CB[16] = {-127, -96, -75, -58, -44, -31, -18, -6, 6, 18, 31, 44, 58, 75, 96, 127};

/* nf4_nearest_idx (real_llm.rs:8614-8644) */
int or_nf4_nearest_idx(float y) {
    float a = fabsf(y);
    int p;
    if (a < 37.5f) p = a < 12.0f ? 0 : (a < 24.5f ? 1 : 2);
    else if (a < 85.5f) p = a < 51.0f ? 3 : (a < 66.5f ? 4 : 5);
    else p = a < 111.5f ? 6 : 7;
    return y >= 0.0f ? 8 + p : 7 - p;
}

/* store_hadamard_q4_head_raw (real_llm.rs:8646-8700): q4 [hd/2] bytes, s16 [hd/64]. */
void or_kv_quant_head_q4(const float *head, size_t hd, uint8_t *q4, uint16_t *s16) {
    float rot[128];
    memcpy(rot, head, hd * sizeof(float));
    or_fwht64(rot, hd);
    for (size_t g = 0; g < hd / 64; g++) {
        const float *blk = rot + g * 64;
        float max_abs = 0.0f;
        for (int i = 0; i < 64; i++) {
            float a = fabsf(blk[i]);
            if (a > max_abs) max_abs = a;
        }
        if (max_abs < 1e-30f) {
            s16[g] = 0;
            memset(q4 + g * 32, 0x88, 32);
            continue;
        }
        float inv0 = 127.0f / max_abs;
        float num = 0.0f, den = 0.0f;
        for (int i = 0; i < 64; i++) {
            float c = (float)OR_NF4_CB[or_nf4_nearest_idx(blk[i] * inv0)];
            num += blk[i] * c;
            den += c * c;
        }
        float s_ref = (den > 1e-12f && num > 0.0f) ? num / den : max_abs / 127.0f;
        uint16_t sb = or_f32_to_bf16(s_ref);
        float sf = or_bf16_to_f32(sb);
        float invf = sf > 1e-30f ? 1.0f / sf : 0.0f;
        s16[g] = sb;
        for (int h = 0; h < 2; h++)
            for (int i = 0; i < 16; i++) {
                int lo = or_nf4_nearest_idx(blk[h * 32 + i] * invf);
                int hi = or_nf4_nearest_idx(blk[h * 32 + 16 + i] * invf);
                q4[g * 32 + h * 16 + i] = (uint8_t)(lo | (hi << 4));
            }
    }
}

/* causal_gqa_group_q4_or_window, NF4 branch (real_llm.rs:8827-8849, 8881-8906), over rows
 * already gathered in attended order: k4/v4 [seq][hd/2], ks16/vs16 [seq][hd/64]. */
void or_attn_q4_head(const float *q_head, const uint8_t *k4, const uint16_t *ks16, const uint8_t *v4,
                     const uint16_t *vs16, size_t seq, size_t hd, float attn_scale, float *out, float *scores) {
    int8_t qi[128];
    float q_scale;
    or_kv_quant_head(q_head, hd, qi, &q_scale);
    const float qs = q_scale * attn_scale;
    const size_t gph = hd / 64, half = hd / 2;
    for (size_t t = 0; t < seq; t++) {
        float total = 0.0f;
        for (size_t g = 0; g < gph; g++) {
            int32_t acc = 0;
            const uint8_t *kp = k4 + t * half + g * 32;
            for (int h = 0; h < 2; h++)
                for (int i = 0; i < 16; i++) {
                    uint8_t b = kp[h * 16 + i];
                    acc += OR_NF4_CB[b & 0x0F] * qi[g * 64 + h * 32 + i] + OR_NF4_CB[b >> 4] * qi[g * 64 + h * 32 + 16 + i];
                }
            total += (float)acc * or_bf16_to_f32(ks16[t * gph + g]) * qs;
        }
        scores[t] = total;
    }
    float mx = -INFINITY;
    for (size_t t = 0; t < seq; t++) mx = fmaxf(mx, scores[t]);
    float sum = 0.0f;
    for (size_t t = 0; t < seq; t++) {
        scores[t] = expf(scores[t] - mx);
        sum += scores[t];
    }
    float inv = 1.0f / sum;
    for (size_t i = 0; i < hd; i++) out[i] = 0.0f;
    for (size_t t = 0; t < seq; t++) {
        float p_norm = scores[t] * inv;
        if (p_norm == 0.0f) continue;
        for (size_t g = 0; g < gph; g++) {
            float w = p_norm * or_bf16_to_f32(vs16[t * gph + g]);
            if (w == 0.0f) continue;
            const uint8_t *vp = v4 + t * half + g * 32;
            for (int h = 0; h < 2; h++)
                for (int i = 0; i < 16; i++) {
                    uint8_t b = vp[h * 16 + i];
                    out[g * 64 + h * 32 + i] += w * (float)OR_NF4_CB[b & 0x0F];
                    out[g * 64 + h * 32 + 16 + i] += w * (float)OR_NF4_CB[b >> 4];
                }
        }
    }
    or_ifwht64(out, hd);
}

/* ------------------------------------------------------------------ */
/* exp of the x86 reference build                                      */
/* ------------------------------------------------------------------ */

/* The x86 reference takes f32::exp from the platform libm (softmax_unnorm_inplace,
 * real_llm.rs:9590-9600; swiglu_activate_scalar, 9801-9805): glibc's expf, which this
 * oracle calls directly.  Test support: counts the inputs x, over the fp32 bit patterns
 * [lo, hi), where fn(x) and expf(x) differ in any bit, on `threads` threads; *first gets
 * the lowest such bit pattern (0xFFFFFFFF when none). */
typedef float (*or_f2f)(float);
typedef struct {
    or_f2f fn;
    uint64_t lo, hi, bad;
    uint32_t first;
} or_exp_job;

static void *or_exp_worker(void *p) {
    or_exp_job *j = (or_exp_job *)p;
    j->bad = 0;
    j->first = 0xFFFFFFFFu;
    for (uint64_t b = j->lo; b < j->hi; b++) {
        const uint32_t u = (uint32_t)b;
        float x, a, r;
        memcpy(&x, &u, 4);
        a = j->fn(x);
        r = expf(x);
        if (memcmp(&a, &r, 4) != 0) {
            if (j->bad == 0) j->first = u;
            j->bad++;
        }
    }
    return NULL;
}

uint64_t or_expf_mismatches(or_f2f fn, uint64_t lo, uint64_t hi, int threads, uint32_t *first) {
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    or_exp_job jobs[64];
    pthread_t th[64];
    const uint64_t span = hi > lo ? hi - lo : 0;
    for (int t = 0; t < threads; t++) {
        jobs[t].fn = fn;
        jobs[t].lo = lo + span * (uint64_t)t / (uint64_t)threads;
        jobs[t].hi = lo + span * (uint64_t)(t + 1) / (uint64_t)threads;
        pthread_create(&th[t], NULL, or_exp_worker, &jobs[t]);
    }
    uint64_t bad = 0;
    uint32_t f = 0xFFFFFFFFu;
    for (int t = 0; t < threads; t++) {
        pthread_join(th[t], NULL);
        bad += jobs[t].bad;
        if (jobs[t].bad && jobs[t].first < f) f = jobs[t].first;
    }
    if (first) *first = f;
    return bad;
}

/* expf over an array (test support: the libm results a device routine is compared with). */
void or_expf_array(const float *x, float *y, size_t n) {
    for (size_t i = 0; i < n; i++) y[i] = expf(x[i]);
}
