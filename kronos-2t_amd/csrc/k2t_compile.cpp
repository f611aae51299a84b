// Offline weight compiler (host, multi-threaded): Hadamard RTN quantization straight
// into the device layouts.
//
//   bit planes : compile_hadamard_gptq_bipolar with no Hessian (compiler.rs:912-1107),
//                then the Nibble4SdotMatrix layout of from_bipolar_with_perm
//                (simd_lut.rs:3297-3400), optionally gate_up-interleaved;
//   NF4        : fit_empirical_nf_codebook (compiler.rs:1404-1526), RTN + least-squares
//                BF16 refit (compiler.rs:1628-1866), NfSdotMatrix::from_indices
//                (simd_lut.rs:4850-5023) and to_gate_up_interleaved (5500-5523).
//
// Work is split over destination stripes; each worker quantizes the 16 source rows of
// its stripe and writes its disjoint records, so the bytes equal the reference's
// two-step (quantize, then pack/repack) output.  Every float expression keeps the
// reference's operation order (the file is built with fp contraction off).
#include <math.h>
#include <string.h>

#include <algorithm>
#include <cfloat>
#include <cstdint>
#include <thread>
#include <vector>

#include "../../include/k2t_hip.h"
#include "k2t_internal.h"
#include "k2t_pack.h"

namespace k2t {
namespace host {

static uint64_t sign_bits(uint64_t block) {
    uint64_t st = 0x9E3779B97F4A7C15ULL + block * 0xBF58476D1CE4E5B9ULL, bits = 0;
    for (int i = 0; i < 64; i++) {
        st += 0x9E3779B97F4A7C15ULL;
        uint64_t z = st;
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
        z ^= z >> 31;
        bits |= (z & 1ULL) << i;
    }
    return bits;
}

struct SignTable {
    std::vector<uint64_t> m;
    explicit SignTable(size_t blocks) : m(blocks) {
        for (size_t b = 0; b < blocks; b++) m[b] = sign_bits(b);
    }
};

// hadamard.rs:70-99 on a full row (block index = chunk index).
static void fwht_row(float *x, size_t n, const SignTable &st) {
    for (size_t b = 0; b < n / 64; b++) {
        float *v = x + 64 * b;
        const uint64_t m = st.m[b];
        for (int i = 0; i < 64; i++) {
            uint32_t u;
            memcpy(&u, &v[i], 4);
            u ^= (uint32_t)((m >> i) & 1ULL) << 31;
            float f;
            memcpy(&f, &u, 4);
            v[i] = f * 0.125f;
        }
        for (int h = 1; h < 64; h <<= 1)
            for (int i = 0; i < 64; i += 2 * h)
                for (int j = i; j < i + h; j++) {
                    const float a = v[j], c = v[j + h];
                    v[j] = a + c;
                    v[j + h] = a - c;
                }
    }
}

static uint16_t to_bf16(float v) {
    uint32_t bits;
    memcpy(&bits, &v, 4);
    if ((bits & 0x7F800000u) == 0x7F800000u && (bits & 0x007FFFFFu)) return (uint16_t)((bits >> 16) | 0x40u);
    return (uint16_t)((bits + 0x7FFFu + ((bits >> 16) & 1u)) >> 16);
}
static float from_bf16(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static size_t source_row(size_t r, size_t rows, bool interleave) { return gate_up_source_row(r, rows, interleave); }

// ---------------------------------------------------------------- bit planes

// compiler.rs:1038-1084 for one 64-column chunk: returns the BF16 scale, writes u codes.
static uint16_t bipolar_chunk(const float *sub, int planes, uint8_t *u) {
    static const float ratios[12] = {0.62f, 0.67f, 0.72f, 0.77f, 0.82f, 0.87f,
                                     0.92f, 0.97f, 1.02f, 1.07f, 1.12f, 1.18f};
    const int max_odd = (1 << planes) - 1;
    const float max_u_f = (float)max_odd, half_off = 0.5f * max_u_f;
    float max_abs = 0.0f;
    for (int i = 0; i < 64; i++) max_abs = fmaxf(max_abs, fabsf(sub[i]));
    memset(u, 0, 64);
    if (max_abs <= 1e-12f) return 0;
    float best_loss = INFINITY;
    uint16_t best = 0;
    uint8_t cand[64];
    for (int k = 0; k < 12; k++) {
        const uint16_t d = to_bf16((max_abs * ratios[k]) / max_u_f);
        const float delta = from_bf16(d);
        if (delta <= 0.0f) continue;
        const float inv2 = 0.5f / delta;
        float loss = 0.0f;
        for (int j = 0; j < 64; j++) {
            const float wj = sub[j];
            float t = roundf(wj * inv2 + half_off);
            t = t < 0.0f ? 0.0f : (t > max_u_f ? max_u_f : t);
            const int ui = (int)t;
            cand[j] = (uint8_t)ui;
            const float diff = wj - (float)(2 * ui - max_odd) * delta;
            loss += diff * diff;
        }
        if (loss < best_loss) {
            best_loss = loss;
            best = d;
            memcpy(u, cand, 64);
        }
    }
    return best;
}

static void compile_bipolar(const float *W, size_t rows, size_t cols, int planes, bool interleave,
                            int threads, uint8_t *pair, uint8_t *tail) {
    const int hp = planes - 4;
    const size_t nc = cols / 64, stripes = (rows + 15) / 16, np = stripes / 2;
    const size_t prec = 1024 + 256 * (size_t)hp + 64, trec = 512 + 128 * (size_t)hp + 32;
    SignTable st(nc);
    memset(pair, 0, np * nc * prec);
    if (stripes & 1) memset(tail, 0, nc * trec);
    parallel_for(stripes, threads, [&](size_t s) {
        std::vector<float> row(cols);
        std::vector<uint8_t> codes(cols);
        const bool in_pair = s < np * 2;
        const size_t p = s / 2, side = s & 1;
        for (size_t lane = 0; lane < 16; lane++) {
            const size_t r = s * 16 + lane;
            if (r >= rows) break;
            memcpy(row.data(), W + source_row(r, rows, interleave) * cols, cols * sizeof(float));
            fwht_row(row.data(), cols, st);
            const N4RecOffsets off = n4_offsets(in_pair, side, hp);
            for (size_t c = 0; c < nc; c++) {
                const uint16_t sc = bipolar_chunk(row.data() + c * 64, planes, codes.data() + c * 64);
                uint8_t *rec = in_pair ? pair + (p * nc + c) * prec : tail + c * trec;
                n4_place_chunk(rec, off, hp, lane, codes.data() + c * 64, sc);
            }
        }
    });
}

// ---------------------------------------------------------------- NF4

static float fit_nf_codebook(const float *W, size_t rows, size_t cols, int bits, size_t sgc, int8_t *cb,
                             const SignTable &st) {
    const int HIST = 2000;
    const float BIN_W = 5.0f / 2000.0f;
    const size_t nc = cols / 64, nsg = (nc + sgc - 1) / sgc;
    const size_t step = std::max<size_t>(rows / 512, 1);
    std::vector<uint64_t> hist(HIST, 0);
    uint64_t total = 0;
    std::vector<float> row(cols);
    for (size_t r = 0; r < rows; r += step) {
        memcpy(row.data(), W + r * cols, cols * sizeof(float));
        fwht_row(row.data(), cols, st);
        for (size_t sg = 0; sg < nsg; sg++) {
            const size_t cs = sg * sgc * 64, ce = std::min(cols, (sg + 1) * sgc * 64);
            float ss = 0.0f;
            for (size_t i = cs; i < ce; i++) ss += row[i] * row[i];
            const float rms = sqrtf(ss / (float)(ce - cs));
            if (rms <= 1e-12f) continue;
            const float inv = 1.0f / rms;
            for (size_t i = cs; i < ce; i++) {
                const float q = (fabsf(row[i]) * inv) / BIN_W;
                const size_t bin = q >= (float)HIST ? (size_t)HIST - 1 : (size_t)q;
                hist[std::min(bin, (size_t)HIST - 1)]++;
                total++;
            }
        }
    }
    static const int8_t NF4_DEFAULT[16] = {-127, -96, -75, -58, -44, -31, -18, -6,
                                           6,    18,  31,  44,  58,  75,  96,  127};
    static const int8_t NF3_DEFAULT[16] = {-127, -79, -45, -14, 14, 45, 79, 127, 0, 0, 0, 0, 0, 0, 0, 0};
    if (total < 256) {
        memcpy(cb, bits == 3 ? NF3_DEFAULT : NF4_DEFAULT, 16);
        return bits == 3 ? 2.1520f : 2.7326f;
    }
    // Lloyd-Max start points of the positive half (compiler.rs:1404-1526)
    const int half = 1 << (bits - 1);
    double mu[8] = {0.1284, 0.3881, 0.6568, 0.9424, 1.2562, 1.6180, 2.0690, 2.7326};
    if (bits == 3) {
        const double mu3[4] = {0.2451, 0.7560, 1.3439, 2.1520};
        for (int m = 0; m < 4; m++) mu[m] = mu3[m];
    }
    for (int it = 0; it < 24; it++) {
        size_t bounds[9];
        bounds[0] = 0;
        bounds[half] = HIST;
        for (int m = 0; m < half - 1; m++) {
            const double rb = round(0.5 * (mu[m] + mu[m + 1]) / (double)BIN_W);
            size_t b = rb <= 0.0 ? 0 : (size_t)rb;
            bounds[m + 1] = std::min<size_t>(std::max(b, bounds[m]), HIST);
        }
        for (int m = 0; m < half; m++) {
            double ws = 0.0;
            uint64_t cs = 0;
            for (size_t b = bounds[m]; b < bounds[m + 1]; b++)
                if (hist[b]) {
                    ws += (double)hist[b] * (((double)b + 0.5) * (double)BIN_W);
                    cs += hist[b];
                }
            if (cs) mu[m] = ws / (double)cs;
        }
        for (int m = 1; m < half; m++)
            if (mu[m] <= mu[m - 1] + 1e-4) mu[m] = mu[m - 1] + 0.05;
    }
    const double top = std::max(mu[half - 1], 0.5);
    int q[8];
    for (int m = 0; m < half; m++) q[m] = std::min(127, std::max(1, (int)round(127.0 * mu[m] / top)));
    q[half - 1] = 127;
    for (int m = half - 2; m >= 0; m--)
        if (q[m] >= q[m + 1]) q[m] = std::max(q[m + 1] - 1, 1);
    for (int m = 1; m < half; m++)
        if (q[m] <= q[m - 1]) q[m] = std::min(q[m - 1] + 1, 127);
    memset(cb, 0, 16);
    for (int m = 0; m < half; m++) {
        cb[half - 1 - m] = (int8_t)(-q[m]);
        cb[half + m] = (int8_t)q[m];
    }
    return (float)top;
}

// compiler.rs:1660-1699 quant_nearest: decision tree over the midpoints of the positive half.
template <int BITS>
static inline size_t nf_nearest(float w, float inv_delta, const float *th) {
    constexpr size_t half = (size_t)1 << (BITS - 1);
    const float aw = fabsf(w) * inv_delta;
    size_t mag;
    if constexpr (BITS == 4) {
        if (aw < th[3]) mag = aw < th[1] ? (size_t)(aw >= th[0]) : 2 + (size_t)(aw >= th[2]);
        else mag = aw < th[5] ? 4 + (size_t)(aw >= th[4]) : 6 + (size_t)(aw >= th[6]);
    } else {
        mag = aw < th[1] ? (size_t)(aw >= th[0]) : 2 + (size_t)(aw >= th[2]);
    }
    return w >= 0.0f ? half + mag : half - 1 - mag;
}

// One scale group of one row: returns the BF16 scale and writes indices.
template <int BITS>
static uint16_t nf_group(const float *sub, size_t glen, const float *cbf, const float *th, float mu_top,
                         uint8_t *best, uint8_t *cand) {
    static const float ratios[11] = {0.74f, 0.80f, 0.86f, 0.91f, 0.96f, 1.00f,
                                     1.04f, 1.09f, 1.15f, 1.22f, 1.30f};
    float ss = 0.0f;
    for (size_t j = 0; j < glen; j++) ss += sub[j] * sub[j];
    const float rms = sqrtf(ss / (float)glen);
    if (rms <= 1e-12f) {
        memset(best, (1 << (BITS - 1)) - 1, glen);
        return 0;
    }
    const float base = rms * (mu_top / 127.0f);
    float best_loss = INFINITY;
    uint16_t bestd = 0;
    memset(best, 0, glen);
    auto eval = [&](uint16_t d) {
        const float delta = from_bf16(d);
        if (delta <= 0.0f) return;
        const float inv = 1.0f / delta;
        float loss = 0.0f;
        for (size_t j = 0; j < glen; j++) {
            const size_t k = nf_nearest<BITS>(sub[j], inv, th);
            cand[j] = (uint8_t)k;
            const float diff = sub[j] - cbf[k] * delta;
            loss += diff * diff;
        }
        if (loss < best_loss) {
            best_loss = loss;
            bestd = d;
            memcpy(best, cand, glen);
        }
    };
    for (int e = 0; e < 11; e++) eval(to_bf16(base * ratios[e]));
    float wc = 0.0f, cc = 0.0f;
    for (size_t j = 0; j < glen; j++) {
        const float cv = cbf[best[j]];
        wc += sub[j] * cv;
        cc += cv * cv;
    }
    if (cc > 1e-12f && wc > 0.0f) {
        const uint16_t ls = to_bf16(wc / cc);
        if (ls != bestd) eval(ls);
    }
    return bestd;
}

// NF3 stripe-chunk (simd_lut.rs:4932-4960): for each column pair-block kp (16-column
// blocks 2kp, 2kp+1), row group g and (row j, column t) three bytes at
// kp*192 + g*48 + {0, 16, 32} + j*4 + t pack the eight 3-bit codes of columns
// 16*k + 4*quad + t (k in {2kp, 2kp+1}, quad 0..3): v0 = i0 | i1<<3 | (i2&3)<<6,
// v1 = i3 | i4<<3 | (i5&3)<<6, v2 = i6 | i7<<3 | (i2>>2)<<6 | (i5>>2)<<7.
static void pack_nf3_chunk(const uint8_t *idx, size_t cols, size_t c, size_t s, size_t rows, uint8_t *dst) {
    for (size_t kp = 0; kp < 2; kp++)
        for (size_t g = 0; g < 4; g++)
            for (size_t j = 0; j < 4; j++) {
                const size_t lane = g * 4 + j;
                const bool live = s * 16 + lane < rows;
                const uint8_t *ir = idx + lane * cols + c * 64;
                for (size_t t = 0; t < 4; t++) {
                    uint8_t i[8];
                    for (size_t u = 0; u < 8; u++) {
                        const size_t k = 2 * kp + u / 4, quad = u % 4;
                        i[u] = live ? ir[k * 16 + quad * 4 + t] & 7 : 0;
                    }
                    uint8_t *blk = dst + kp * 192 + g * 48 + j * 4 + t;
                    blk[0] = (uint8_t)(i[0] | (i[1] << 3) | ((i[2] & 3) << 6));
                    blk[16] = (uint8_t)(i[3] | (i[4] << 3) | ((i[5] & 3) << 6));
                    blk[32] = (uint8_t)(i[6] | (i[7] << 3) | (((i[2] >> 2) & 1) << 6) | (((i[5] >> 2) & 1) << 7));
                }
            }
}

template <int BITS>
static void compile_nf(const float *W, size_t rows, size_t cols, size_t sgc, bool interleave, int threads,
                       int8_t *cb, float *mu_out, uint8_t *pair, uint8_t *tail) {
    constexpr size_t CB = BITS == 3 ? 384 : 512;  // bytes per stripe-chunk
    constexpr int half = 1 << (BITS - 1);
    const size_t nc = cols / 64, nsg = (nc + sgc - 1) / sgc, stripes = (rows + 15) / 16, np = stripes / 2;
    const size_t ptot = nsg * 64 + nc * 2 * CB, ttot = nsg * 32 + nc * CB;
    SignTable st(nc);
    const float mu_top = fit_nf_codebook(W, rows, cols, BITS, sgc, cb, st);
    if (mu_out) *mu_out = mu_top;
    float cbf[16], th[7];
    for (int k = 0; k < 16; k++) cbf[k] = (float)cb[k];
    for (int m = 0; m + 1 < half; m++) th[m] = 0.5f * (cbf[half + m] + cbf[half + m + 1]);
    memset(pair, 0, np * ptot);
    if (stripes & 1) memset(tail, 0, ttot);
    parallel_for(stripes, threads, [&](size_t s) {
        std::vector<float> row(cols);
        std::vector<uint8_t> idx(16 * cols, 0), best(sgc * 64), cand(sgc * 64);
        std::vector<uint16_t> scales(16 * nsg, 0);
        for (size_t lane = 0; lane < 16; lane++) {
            const size_t r = s * 16 + lane;
            if (r >= rows) break;
            memcpy(row.data(), W + source_row(r, rows, interleave) * cols, cols * sizeof(float));
            fwht_row(row.data(), cols, st);
            for (size_t sg = 0; sg < nsg; sg++) {
                const size_t c0 = sg * sgc, c1 = std::min(nc, c0 + sgc), glen = (c1 - c0) * 64;
                scales[lane * nsg + sg] =
                    nf_group<BITS>(row.data() + c0 * 64, glen, cbf, th, mu_top, best.data(), cand.data());
                memcpy(idx.data() + lane * cols + c0 * 64, best.data(), glen);
            }
        }
        // Pack (simd_lut.rs:4874-4923): rows past `rows` keep index 0.
        const bool in_pair = s < np * 2;
        const size_t side = s & 1;
        for (size_t sg = 0; sg < nsg; sg++) {
            const size_t c0 = sg * sgc, c1 = std::min(nc, c0 + sgc);
            uint8_t *gb = in_pair ? pair + (s / 2) * ptot + sg * 64 + c0 * 2 * CB : tail + sg * 32 + c0 * CB;
            uint8_t *sp = gb + (in_pair ? side * 32 : 0);
            for (size_t lane = 0; lane < 16; lane++) {
                sp[lane * 2] = (uint8_t)scales[lane * nsg + sg];
                sp[lane * 2 + 1] = (uint8_t)(scales[lane * nsg + sg] >> 8);
            }
            for (size_t c = c0; c < c1; c++) {
                uint8_t *dst = in_pair ? gb + 64 + (c - c0) * 2 * CB + side * CB : gb + 32 + (c - c0) * CB;
                if constexpr (BITS == 3) {
                    pack_nf3_chunk(idx.data(), cols, c, s, rows, dst);
                    continue;
                }
                for (size_t k = 0; k < 4; k++)
                    for (size_t g = 0; g < 4; g++)
                        for (size_t j = 0; j < 4; j++) {
                            const size_t lane = g * 4 + j;
                            const uint8_t *ir = idx.data() + lane * cols + c * 64 + k * 16;
                            const bool live = s * 16 + lane < rows;
                            for (size_t t = 0; t < 4; t++) {
                                const uint8_t lo0 = live ? ir[t] & 15 : 0, hi0 = live ? ir[4 + t] & 15 : 0;
                                const uint8_t lo1 = live ? ir[8 + t] & 15 : 0, hi1 = live ? ir[12 + t] & 15 : 0;
                                dst[k * 128 + g * 32 + j * 4 + t] = (uint8_t)(lo0 | (hi0 << 4));
                                dst[k * 128 + g * 32 + 16 + j * 4 + t] = (uint8_t)(lo1 | (hi1 << 4));
                            }
                        }
            }
        }
    });
}

// Counter-based N(0, std): SplitMix64 of (seed, pair index) -> two uniforms -> Box-Muller.
static void synth_normal(uint64_t seed, float stdv, float *out, size_t n, int threads) {
    const size_t pairs = (n + 1) / 2, blk = 1 << 16;
    parallel_for((pairs + blk - 1) / blk, threads, [&](size_t b) {
        const size_t p0 = b * blk, p1 = std::min(pairs, p0 + blk);
        for (size_t p = p0; p < p1; p++) {
            uint64_t z = seed * 0xD1B54A32D192ED03ULL + p * 0x9E3779B97F4A7C15ULL;
            uint64_t h[2];
            for (int k = 0; k < 2; k++) {
                z += 0x9E3779B97F4A7C15ULL;
                uint64_t x = z;
                x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ULL;
                x = (x ^ (x >> 27)) * 0x94D049BB133111EBULL;
                h[k] = x ^ (x >> 31);
            }
            const double u1 = ((double)(h[0] >> 11) + 0.5) * (1.0 / 9007199254740992.0);
            const double u2 = (double)(h[1] >> 11) * (1.0 / 9007199254740992.0);
            const double rad = sqrt(-2.0 * log(u1)) * (double)stdv;
            out[2 * p] = (float)(rad * cos(6.283185307179586 * u2));
            if (2 * p + 1 < n) out[2 * p + 1] = (float)(rad * sin(6.283185307179586 * u2));
        }
    });
}

}  // namespace host
}  // namespace k2t

using namespace k2t;

extern "C" {

int32_t k2t_stream_sizes(int32_t fmt, int32_t rows, int32_t cols, int32_t planes_or_bits, int32_t sgc,
                         size_t *pair_len, size_t *tail_len) {
    if (!pair_len || !tail_len || rows <= 0 || cols <= 0 || cols % 64) return K2T_E_ARG;
    const size_t stripes = (size_t)(rows + 15) / 16, nc = (size_t)cols / 64;
    if (fmt == 1) {
        if (planes_or_bits < 4 || planes_or_bits > 6) return K2T_E_ARG;
        const size_t hp = (size_t)planes_or_bits - 4;
        *pair_len = (stripes / 2) * nc * (1024 + 256 * hp + 64);
        *tail_len = (stripes & 1) * nc * (512 + 128 * hp + 32);
        return K2T_OK;
    }
    if (fmt == 2) {
        if ((planes_or_bits != 3 && planes_or_bits != 4) || sgc < 1 || sgc > 8) return K2T_E_ARG;
        const size_t nsg = (nc + sgc - 1) / sgc, cb = planes_or_bits == 3 ? 384 : 512;
        *pair_len = (stripes / 2) * (nsg * 64 + nc * 2 * cb);
        *tail_len = (stripes & 1) * (nsg * 32 + nc * cb);
        return K2T_OK;
    }
    return K2T_E_ARG;
}

int32_t k2t_compile_bipolar(const float *W, int32_t rows, int32_t cols, int32_t planes,
                            int32_t interleave_gate_up, int32_t threads, uint8_t *pair, size_t pair_len,
                            uint8_t *tail, size_t tail_len) {
    size_t pl = 0, tl = 0;
    if (!W || k2t_stream_sizes(1, rows, cols, planes, 1, &pl, &tl) != K2T_OK) return K2T_E_ARG;
    if (pl != pair_len || tl != tail_len || (pl && !pair) || (tl && !tail)) return K2T_E_ARG;
    if (interleave_gate_up && rows % 128) return K2T_E_ARG;
    try {
        host::compile_bipolar(W, (size_t)rows, (size_t)cols, planes, interleave_gate_up != 0, threads, pair, tail);
    } catch (...) {
        return K2T_E_INTERNAL;
    }
    return K2T_OK;
}

int32_t k2t_compile_nf(const float *W, int32_t rows, int32_t cols, int32_t bits, int32_t sgc,
                       int32_t interleave_gate_up, int32_t threads, int8_t *codebook16, float *mu_top,
                       uint8_t *pair, size_t pair_len, uint8_t *tail, size_t tail_len) {
    size_t pl = 0, tl = 0;
    if (!W || !codebook16 || k2t_stream_sizes(2, rows, cols, bits, sgc, &pl, &tl) != K2T_OK) return K2T_E_ARG;
    if (pl != pair_len || tl != tail_len || (pl && !pair) || (tl && !tail)) return K2T_E_ARG;
    if (interleave_gate_up && rows % 128) return K2T_E_ARG;
    try {
        if (bits == 3)
            host::compile_nf<3>(W, (size_t)rows, (size_t)cols, (size_t)sgc, interleave_gate_up != 0, threads,
                                codebook16, mu_top, pair, tail);
        else
            host::compile_nf<4>(W, (size_t)rows, (size_t)cols, (size_t)sgc, interleave_gate_up != 0, threads,
                                codebook16, mu_top, pair, tail);
    } catch (...) {
        return K2T_E_INTERNAL;
    }
    return K2T_OK;
}

int32_t k2t_synth_normal(uint64_t seed, float stdv, float *out, size_t n, int32_t threads) {
    if (!out && n) return K2T_E_ARG;
    try {
        host::synth_normal(seed, stdv, out, n, threads);
    } catch (...) {
        return K2T_E_INTERNAL;
    }
    return K2T_OK;
}

}  // extern "C"
