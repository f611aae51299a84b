// Host-side placement of one row's 64 bipolar codes into a Nibble4SdotMatrix record
// (from_bipolar_with_perm, simd_lut.rs:3297-3400), shared by the weight compiler and
// the .k2tb loader.
#pragma once
#include <stddef.h>
#include <stdint.h>

#include <algorithm>
#include <thread>
#include <vector>

namespace k2t {
namespace host {

// Byte offsets inside the record of (stripe side): nibble data, hi planes, BF16 scales.
struct N4RecOffsets {
    size_t data, hi, scales;
};

// Runs fn(i) for i in [0, n) on up to `threads` host threads (0 = all cores), in
// contiguous index blocks.
template <typename F>
inline void parallel_for(size_t n, int threads, F &&fn) {
    if (threads <= 0) threads = (int)std::max(1u, std::thread::hardware_concurrency());
    threads = (int)std::min<size_t>((size_t)threads, std::max<size_t>(n, 1));
    if (threads <= 1) {
        for (size_t i = 0; i < n; i++) fn(i);
        return;
    }
    std::vector<std::thread> pool;
    const size_t per = (n + threads - 1) / threads;
    for (int t = 0; t < threads; t++) {
        const size_t b = t * per, e = std::min(n, b + per);
        if (b >= e) break;
        pool.emplace_back([&, b, e] {
            for (size_t i = b; i < e; i++) fn(i);
        });
    }
    for (auto &th : pool) th.join();
}

// Source row of destination row `r` under the [gate64(ic), up64(ic)] interleave of a
// gate_up matrix with `rows` = 2 * intermediate rows (repack_sdot, real_llm.rs:3657-3702).
inline size_t gate_up_source_row(size_t r, size_t rows, bool interleave) {
    if (!interleave) return r;
    const size_t blk = r / 64, off = r % 64, inter_dim = rows / 2;
    return (blk / 2) * 64 + off + ((blk & 1) ? inter_dim : 0);
}

inline size_t n4_pair_rec(int hp) { return 1024 + 256 * (size_t)hp + 64; }
inline size_t n4_tail_rec(int hp) { return 512 + 128 * (size_t)hp + 32; }

inline N4RecOffsets n4_offsets(bool in_pair, size_t side, int hp) {
    if (in_pair) return {side * 512, 1024 + side * 128 * (size_t)hp, 1024 + 256 * (size_t)hp + side * 32};
    return {0, 512, 512 + 128 * (size_t)hp};
}

// ORs codes u[0..63] of row `lane` (0..15 within its stripe) of one chunk into `rec`,
// and stores its BF16 scale.  `rec` must start zeroed.
inline void n4_place_chunk(uint8_t *rec, const N4RecOffsets &o, int hp, size_t lane, const uint8_t *u,
                           uint16_t scale) {
    rec[o.scales + lane * 2] = (uint8_t)scale;
    rec[o.scales + lane * 2 + 1] = (uint8_t)(scale >> 8);
    const size_t g = lane / 4, j = lane % 4;
    for (size_t k = 0; k < 4; k++)
        for (size_t w = 0; w < 16; w++) {
            const uint8_t uv = u[k * 16 + w];
            const size_t half = w / 8, sub = w / 4, t = w % 4;
            const uint8_t lo = uv & 0x0F;
            rec[o.data + k * 128 + g * 32 + half * 16 + j * 4 + t] |= (w % 8) < 4 ? lo : (uint8_t)(lo << 4);
            if (hp == 1) {
                const int bit = (k & 1) == 0 ? 4 + (int)sub : (int)sub;
                rec[o.hi + (k / 2) * 64 + g * 16 + j * 4 + t] |= (uint8_t)(((uv >> 4) & 1) << bit);
            } else if (hp == 2) {
                static const int sh[4] = {4, 6, 2, 0};
                rec[o.hi + k * 64 + g * 16 + j * 4 + t] |= (uint8_t)(((uv >> 4) & 3) << sh[sub]);
            }
        }
}

}  // namespace host
}  // namespace k2t
