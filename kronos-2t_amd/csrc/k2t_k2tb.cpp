// .k2tb compiled-model reader (host): the cache written by RealLlamaEngine::save_bipolar
// (real_llm.rs:3705-3895) and read by load_bipolar (real_llm.rs:3902-4190), followed by
// the repack_sdot step (real_llm.rs:3657-3702) that turns it into the layouts the GEMV
// streams, and an upload of the whole model to one device.
//
// File format (all integers u64 little endian, `f32s` = u64 count + count f32 LE):
//   magic  "K2TBIPOLAR1\n" (v1) | "K2TKRONOS2\n" (v2) | "K2TKRONOS3\n" (v3)
//          | "K2TKRONOS4\n" (v4) | "K2TKRONOS6\n" (v6)
//   mode words [6]; n_layers
//   per layer: f32s in_norm, f32s post_norm, [v3+] f32s qkv_bias, [v6] f32s q_norm,
//              f32s k_norm, then 4 matrices qkv, o, gate_up, down
//   f32s final_norm, matrix lm_head, f32s embed_f32_rows,
//   [v3+] u64 n + n bf16 embed rows, [v4+] u64 has_nf4_embed (+ matrix)
// Matrix (v1: body of tag 0 without the tag):
//   tag 0 FusedBipolar: rows, cols, planes, n + n bytes interleaved planes
//                       [stripes][cols/8][planes][16], n + n u16 scales [stripes][nc][16]
//   tag 1 Vq2, tag 3 Q2c: not on this path (rejected with a message)
//   tag 2 NfSdot:  rows, cols, bits, sgc, 16 codebook bytes, n + pair stream, n + tail
//
// The file is memory-mapped; every read is bounds-checked, so a truncated or corrupt
// file returns K2T_E_ARG with a message instead of reading past the mapping.
#include <fcntl.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <string>
#include <vector>

#include "../../include/k2t_hip.h"
#include "k2t_internal.h"
#include "k2t_pack.h"

using namespace k2t;
using namespace k2t::host;

namespace {

struct Span {
    size_t off = 0, len = 0;  // bytes
};

struct MatRec {
    int tag = -1;
    size_t rows = 0, cols = 0, planes_or_bits = 0, sgc = 1;
    int8_t cb[16] = {0};
    Span a, b;  // bipolar: planes, scales (u16); NF: pair, tail
};

struct LayerRec {
    Span in_norm, post_norm, bias, q_norm, k_norm;  // f32 payloads
    MatRec m[4];
};

struct Cursor {
    const uint8_t *base;
    size_t len, pos;
    const uint8_t *take(size_t n) {
        if (n > len - pos) throw Error(K2T_E_ARG, "truncated .k2tb file at byte " + std::to_string(pos));
        const uint8_t *p = base + pos;
        pos += n;
        return p;
    }
    uint64_t u64() {
        uint64_t v;
        memcpy(&v, take(8), 8);
        return v;
    }
    size_t count(size_t elem) {
        const uint64_t n = u64();
        if (n > (len - pos) / elem) throw Error(K2T_E_ARG, "truncated .k2tb file at byte " + std::to_string(pos));
        return (size_t)n;
    }
    Span f32s() {
        const size_t n = count(4);
        Span s{pos, n};
        take(n * 4);
        return s;
    }
};

}  // namespace

struct k2t_k2tb {
    void *map = nullptr;
    size_t len = 0;
    int version = 0;
    uint64_t mode[6] = {0};
    std::vector<LayerRec> layers;
    Span final_norm, embed_f32, embed_bf16;
    MatRec head, embed_nf4;
    bool has_embed_nf4 = false;
    const uint8_t *bytes() const { return (const uint8_t *)map; }
};

namespace {

MatRec read_bipolar_body(Cursor &c) {
    MatRec m;
    m.tag = 0;
    m.rows = c.u64();
    m.cols = c.u64();
    m.planes_or_bits = c.u64();
    const size_t n = c.count(1);
    m.a = {c.pos, n};
    c.take(n);
    const size_t ns = c.count(2);
    m.b = {c.pos, ns};
    c.take(ns * 2);
    return m;
}

MatRec read_matrix(Cursor &c, int version) {
    if (version == 1) return read_bipolar_body(c);
    const uint64_t tag = c.u64();
    if (tag == 0) return read_bipolar_body(c);
    if (tag == 2) {
        MatRec m;
        m.tag = 2;
        m.rows = c.u64();
        m.cols = c.u64();
        m.planes_or_bits = c.u64();
        m.sgc = std::max<uint64_t>(c.u64(), 1);
        memcpy(m.cb, c.take(16), 16);
        const size_t pl = c.count(1);
        m.a = {c.pos, pl};
        c.take(pl);
        const size_t tl = c.count(1);
        m.b = {c.pos, tl};
        c.take(tl);
        return m;
    }
    if (tag == 1) throw Error(K2T_E_STATE, ".k2tb holds a VQ2 matrix: not supported by the HIP path");
    if (tag == 3) throw Error(K2T_E_STATE, ".k2tb holds a Q2C matrix: not supported by the HIP path");
    throw Error(K2T_E_ARG, "unknown matrix tag in .k2tb file");
}

void parse(k2t_k2tb *f) {
    static const struct {
        const char *magic;
        int version;
    } magics[] = {{"K2TKRONOS6\n", 6}, {"K2TKRONOS5\n", 5}, {"K2TKRONOS4\n", 4},
                  {"K2TKRONOS3\n", 3}, {"K2TKRONOS2\n", 2}, {"K2TBIPOLAR1\n", 1}};
    Cursor c{f->bytes(), f->len, 0};
    for (const auto &mg : magics) {
        const size_t n = strlen(mg.magic);
        if (f->len >= n && memcmp(f->bytes(), mg.magic, n) == 0) {
            f->version = mg.version;
            c.pos = n;
            break;
        }
    }
    if (!f->version) throw Error(K2T_E_ARG, "bad .k2tb magic");
    if (f->version == 5)
        throw Error(K2T_E_STATE, "K2TKRONOS5 (sparse-MoE core with .k2tm experts) is not supported by this loader");
    for (auto &w : f->mode) w = c.u64();
    const size_t nl = c.u64();
    if (nl == 0 || nl > 4096) throw Error(K2T_E_ARG, "implausible layer count in .k2tb file");
    f->layers.resize(nl);
    for (auto &L : f->layers) {
        L.in_norm = c.f32s();
        L.post_norm = c.f32s();
        if (f->version >= 3) L.bias = c.f32s();
        if (f->version >= 6) {
            L.q_norm = c.f32s();
            L.k_norm = c.f32s();
        }
        for (auto &m : L.m) m = read_matrix(c, f->version);
    }
    f->final_norm = c.f32s();
    f->head = read_matrix(c, f->version);
    f->embed_f32 = c.f32s();
    if (f->version >= 3) {
        const size_t n = c.count(2);
        f->embed_bf16 = {c.pos, n};
        c.take(n * 2);
    }
    if (f->version >= 4 && c.u64() != 0) {
        f->embed_nf4 = read_matrix(c, f->version);
        if (f->embed_nf4.tag != 2) throw Error(K2T_E_ARG, "expected an NfSdot untied embedding matrix");
        f->has_embed_nf4 = true;
    }
}

template <typename F>
int32_t guard(F &&fn) {
    try {
        fn();
        return K2T_OK;
    } catch (const Error &e) {
        set_last_error(e.what());
        return e.code;
    } catch (const std::exception &e) {
        set_last_error(e.what());
        return K2T_E_INTERNAL;
    } catch (...) {
        set_last_error("unknown error");
        return K2T_E_INTERNAL;
    }
}

const MatRec &pick(const k2t_k2tb *f, int layer, int which) {
    if (layer >= 0) {
        if (layer >= (int)f->layers.size() || which < 0 || which > 3) throw Error(K2T_E_ARG, "matrix index out of range");
        return f->layers[layer].m[which];
    }
    if (which == 4) return f->head;
    if (which == 5 && f->has_embed_nf4) return f->embed_nf4;
    throw Error(K2T_E_ARG, "matrix index out of range");
}

// Describes the repacked form of m (format, stream sizes) and validates its sizes.
void describe(const MatRec &m, int interleave, k2t_k2tb_matrix_info *info) {
    memset(info, 0, sizeof(*info));
    info->tag = m.tag;
    info->rows = (int32_t)m.rows;
    info->cols = (int32_t)m.cols;
    info->planes_or_bits = (int32_t)m.planes_or_bits;
    info->sgc = (int32_t)m.sgc;
    memcpy(info->codebook, m.cb, 16);
    if (m.rows == 0 || m.cols == 0 || m.cols % 64 || m.rows > (1u << 24) || m.cols > (1u << 20))
        throw Error(K2T_E_ARG, "bad matrix shape in .k2tb file");
    if (interleave && m.rows % 128) throw Error(K2T_E_ARG, "gate_up interleaving needs rows divisible by 128");
    const size_t stripes = (m.rows + 15) / 16, nc = m.cols / 64;
    size_t pl = 0, tl = 0;
    if (m.tag == 0) {
        if (m.planes_or_bits < 4 || m.planes_or_bits > 6)
            throw Error(K2T_E_STATE, "bit-plane matrix with " + std::to_string(m.planes_or_bits) +
                                         " planes: the SDOT layout needs 4..6 planes");
        if (m.a.len != stripes * (m.cols / 8) * m.planes_or_bits * 16 || m.b.len != stripes * nc * 16)
            throw Error(K2T_E_ARG, "bit-plane matrix payload sizes do not match its shape");
        info->fmt = 1;
    } else {
        if (m.planes_or_bits != 3 && m.planes_or_bits != 4)
            throw Error(K2T_E_STATE, "NF matrix with " + std::to_string(m.planes_or_bits) +
                                         " bits: the HIP GEMV takes NF3 and NF4");
        info->fmt = 2;
    }
    if (k2t_stream_sizes(info->fmt, info->rows, info->cols, info->planes_or_bits, info->sgc, &pl, &tl) != K2T_OK)
        throw Error(K2T_E_ARG, "bad matrix parameters in .k2tb file");
    if (m.tag == 2 && (m.a.len != pl || m.b.len != tl))
        throw Error(K2T_E_ARG, "NF matrix stream sizes do not match its shape");
    info->pair_len = pl;
    info->tail_len = tl;
}

// Nibble4SdotMatrix::from_bipolar_with_perm (simd_lut.rs:3297-3400): per destination
// stripe, unpack each source row's plane codes and place them into the records.
void repack_bipolar(const uint8_t *file, const MatRec &m, bool interleave, uint8_t *pair, uint8_t *tail) {
    const size_t rows = m.rows, cols = m.cols, planes = m.planes_or_bits, nc = cols / 64, opr = cols / 8;
    const int hp = (int)planes - 4;
    const size_t stripes = (rows + 15) / 16, np = stripes / 2;
    const size_t prec = n4_pair_rec(hp), trec = n4_tail_rec(hp);
    const uint8_t *planes_b = file + m.a.off;
    const uint8_t *scales_b = file + m.b.off;
    memset(pair, 0, np * nc * prec);
    if (stripes & 1) memset(tail, 0, nc * trec);
    parallel_for(stripes, 0, [&](size_t s) {
        uint8_t codes[64];
        const bool in_pair = s < np * 2;
        const size_t p = s / 2, side = s & 1;
        const N4RecOffsets off = n4_offsets(in_pair, side, hp);
        for (size_t lane = 0; lane < 16; lane++) {
            const size_t r = s * 16 + lane;
            if (r >= rows) break;
            const size_t sr = gate_up_source_row(r, rows, interleave);
            const size_t ss = sr / 16, sl = sr % 16;
            for (size_t c = 0; c < nc; c++) {
                // unpack_row_codes (simd_lut.rs:1805-1822) for the chunk's 8 octets
                for (size_t o = 0; o < 8; o++) {
                    const uint8_t *ob = planes_b + ((ss * opr + c * 8 + o) * planes) * 16 + sl;
                    for (size_t k = 0; k < 8; k++) {
                        uint8_t u = 0;
                        for (size_t pl = 0; pl < planes; pl++) u |= (uint8_t)(((ob[pl * 16] >> k) & 1) << pl);
                        codes[o * 8 + k] = u;
                    }
                }
                const uint8_t *sp = scales_b + ((ss * nc + c) * 16 + sl) * 2;
                const uint16_t sc = (uint16_t)(sp[0] | (sp[1] << 8));
                uint8_t *rec = in_pair ? pair + (p * nc + c) * prec : tail + c * trec;
                n4_place_chunk(rec, off, hp, lane, codes, sc);
            }
        }
    });
}

// NfSdotMatrix streams as stored; gate_up swaps 64-row blocks (two pairs) into the
// [gate64(ic), up64(ic)] order (to_gate_up_interleaved, simd_lut.rs:5500-5523).
void copy_nf(const uint8_t *file, const MatRec &m, bool interleave, uint8_t *pair, uint8_t *tail) {
    if (!interleave) {
        memcpy(pair, file + m.a.off, m.a.len);
    } else {
        const size_t pairs = (m.rows + 31) / 32, ptot = pairs ? m.a.len / pairs : 0;
        const size_t nci = m.rows / 128, blk = 2 * ptot;
        for (size_t ic = 0; ic < nci; ic++) {
            memcpy(pair + (2 * ic) * blk, file + m.a.off + ic * blk, blk);
            memcpy(pair + (2 * ic + 1) * blk, file + m.a.off + (nci + ic) * blk, blk);
        }
    }
    if (m.b.len) memcpy(tail, file + m.b.off, m.b.len);
}

void extract(const k2t_k2tb *f, const MatRec &m, bool interleave, uint8_t *pair, uint8_t *tail) {
    if (m.tag == 0)
        repack_bipolar(f->bytes(), m, interleave, pair, tail);
    else
        copy_nf(f->bytes(), m, interleave, pair, tail);
}

}  // namespace

extern "C" {

int32_t k2t_k2tb_open(const char *path, k2t_k2tb **out) {
    return guard([&] {
        if (!path || !out) throw Error(K2T_E_ARG, "NULL argument");
        *out = nullptr;
        const int fd = open(path, O_RDONLY);
        if (fd < 0) throw Error(K2T_E_ARG, std::string("cannot open ") + path + ": " + strerror(errno));
        struct stat st;
        if (fstat(fd, &st) != 0 || st.st_size < 16) {
            close(fd);
            throw Error(K2T_E_ARG, std::string("empty or unreadable .k2tb file: ") + path);
        }
        void *map = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
        close(fd);
        if (map == MAP_FAILED) throw Error(K2T_E_ARG, std::string("mmap failed: ") + strerror(errno));
        k2t_k2tb *f = new k2t_k2tb();
        f->map = map;
        f->len = (size_t)st.st_size;
        try {
            parse(f);
        } catch (...) {
            k2t_k2tb_close(f);
            throw;
        }
        *out = f;
    });
}

void k2t_k2tb_close(k2t_k2tb *f) {
    if (!f) return;
    if (f->map) munmap(f->map, f->len);
    delete f;
}

int32_t k2t_k2tb_header(const k2t_k2tb *f, int32_t *version, int32_t *n_layers, uint64_t *mode_words6) {
    return guard([&] {
        if (!f) throw Error(K2T_E_ARG, "NULL argument");
        if (version) *version = f->version;
        if (n_layers) *n_layers = (int32_t)f->layers.size();
        if (mode_words6) memcpy(mode_words6, f->mode, sizeof(f->mode));
    });
}

int32_t k2t_k2tb_matrix(const k2t_k2tb *f, int32_t layer, int32_t which, int32_t interleave_gate_up,
                        k2t_k2tb_matrix_info *info, uint8_t *pair, size_t pair_cap, uint8_t *tail, size_t tail_cap) {
    return guard([&] {
        if (!f || !info) throw Error(K2T_E_ARG, "NULL argument");
        const MatRec &m = pick(f, layer, which);
        describe(m, interleave_gate_up, info);
        if (!pair && !tail) return;  // size query
        if (!pair || pair_cap < info->pair_len || (info->tail_len && (!tail || tail_cap < info->tail_len)))
            throw Error(K2T_E_ARG, "output buffers smaller than the repacked streams");
        extract(f, m, interleave_gate_up != 0, pair, tail);
    });
}

int32_t k2t_k2tb_vector(const k2t_k2tb *f, int32_t layer, int32_t which, size_t *count, void *out, size_t cap) {
    return guard([&] {
        if (!f || !count) throw Error(K2T_E_ARG, "NULL argument");
        Span s;
        size_t elem = 4;
        if (layer >= 0) {
            if (layer >= (int)f->layers.size()) throw Error(K2T_E_ARG, "layer out of range");
            const LayerRec &L = f->layers[layer];
            const Span *v[5] = {&L.in_norm, &L.post_norm, &L.bias, &L.q_norm, &L.k_norm};
            if (which < 0 || which > 4) throw Error(K2T_E_ARG, "vector index out of range");
            s = *v[which];
        } else if (which == 0) {
            s = f->final_norm;
        } else if (which == 1) {
            s = f->embed_f32;
        } else if (which == 2) {
            s = f->embed_bf16;
            elem = 2;
        } else {
            throw Error(K2T_E_ARG, "vector index out of range");
        }
        *count = s.len;
        if (!out) return;
        if (cap < s.len) throw Error(K2T_E_ARG, "output buffer too small");
        memcpy(out, f->bytes() + s.off, s.len * elem);
    });
}

int32_t k2t_model_load_k2tb(k2t_ctx *ctx, const k2t_model_config *cfg, const char *path, int32_t max_batch,
                            k2t_model **out) {
    k2t_k2tb *f = nullptr;
    k2t_model *model = nullptr;
    const int32_t rc = guard([&] {
        if (!ctx || !cfg || !path || !out) throw Error(K2T_E_ARG, "NULL argument");
        *out = nullptr;
        int32_t e = k2t_k2tb_open(path, &f);
        if (e) throw Error(e, k2t_last_error());
        const k2t_model_config &c = *cfg;
        if ((int)f->layers.size() != c.n_layers) throw Error(K2T_E_ARG, "layer count does not match the config");
        e = k2t_model_create(ctx, cfg, max_batch, &model);
        if (e) throw Error(e, k2t_last_error());
        auto vec = [&](const Span &s, size_t want, const char *what) -> const float * {
            if (s.len == 0) return nullptr;
            if (s.len != want) throw Error(K2T_E_ARG, std::string(what) + " length does not match the config");
            return (const float *)(f->bytes() + s.off);  // f32 LE payload; read through memcpy below
        };
        auto upload = [&](const MatRec &m, bool gu) -> k2t_mat * {
            k2t_k2tb_matrix_info info;
            describe(m, gu, &info);
            std::vector<uint8_t> pair(info.pair_len), tail(info.tail_len);
            extract(f, m, gu, pair.data(), tail.data());
            k2t_mat *h = nullptr;
            int32_t r;
            if (info.fmt == 1)
                r = k2t_mat_upload_nibble4(ctx, info.rows, info.cols, info.planes_or_bits - 4, pair.data(),
                                           pair.size(), tail.empty() ? nullptr : tail.data(), tail.size(), &h);
            else
                r = k2t_mat_upload_nf(ctx, info.rows, info.cols, info.planes_or_bits, info.sgc, info.codebook,
                                      pair.data(), pair.size(), tail.empty() ? nullptr : tail.data(), tail.size(), &h);
            if (r) throw Error(r, k2t_last_error());
            model_adopt(model, h);
            return h;
        };
        auto copy_f32 = [&](const float *p, size_t n) {
            std::vector<float> v(n);
            if (p) memcpy(v.data(), p, n * 4);
            return v;
        };
        const size_t qkv_rows = (size_t)(c.n_heads + 2 * c.n_kv_heads) * c.head_dim;
        for (int l = 0; l < c.n_layers; l++) {
            const LayerRec &L = f->layers[l];
            if (L.q_norm.len || L.k_norm.len)
                throw Error(K2T_E_STATE, "per-head q_norm / k_norm (K2TKRONOS6) is not supported by the HIP path");
            const float *in = vec(L.in_norm, c.hidden, "input_norm");
            const float *post = vec(L.post_norm, c.hidden, "post_attn_norm");
            if (!in || !post) throw Error(K2T_E_ARG, "missing RMSNorm weights");
            const float *bias = vec(L.bias, qkv_rows, "qkv_bias");
            k2t_mat *qkv = upload(L.m[0], false), *o = upload(L.m[1], false);
            k2t_mat *gu = upload(L.m[2], true), *dn = upload(L.m[3], false);
            const auto vin = copy_f32(in, c.hidden), vpost = copy_f32(post, c.hidden);
            const auto vbias = copy_f32(bias, bias ? qkv_rows : 0);
            e = k2t_model_set_layer(model, l, qkv, o, gu, dn, vin.data(), vpost.data(), bias ? vbias.data() : nullptr);
            if (e) throw Error(e, k2t_last_error());
        }
        const float *fn = vec(f->final_norm, c.hidden, "final_norm");
        if (!fn) throw Error(K2T_E_ARG, "missing final norm");
        const size_t vh = (size_t)c.vocab * c.hidden;
        // embed_token_into's precedence (real_llm.rs:8063-8097): f32 rows, bf16 rows,
        // NF4 matrix, else the tied lm_head.
        int32_t ekind = K2T_EMBED_TIED;
        if (f->embed_f32.len) {
            if (f->embed_f32.len != vh) throw Error(K2T_E_ARG, "f32 embedding size does not match the config");
            ekind = K2T_EMBED_F32;
        } else if (f->embed_bf16.len) {
            if (f->embed_bf16.len != vh) throw Error(K2T_E_ARG, "bf16 embedding size does not match the config");
            ekind = K2T_EMBED_BF16;
        } else if (f->has_embed_nf4) {
            ekind = K2T_EMBED_NF4;
        }
        if (ekind != K2T_EMBED_TIED) {
            const void *rows = nullptr;
            const k2t_mat *em = nullptr;
            if (ekind == K2T_EMBED_F32) rows = f->bytes() + f->embed_f32.off;
            if (ekind == K2T_EMBED_BF16) rows = f->bytes() + f->embed_bf16.off;
            if (ekind == K2T_EMBED_NF4) em = upload(f->embed_nf4, false);
            e = k2t_model_set_embedding(model, ekind, rows, em);
            if (e) throw Error(e, k2t_last_error());
        }
        const k2t_mat *head = upload(f->head, false);
        const auto vfn = copy_f32(fn, c.hidden);
        e = k2t_model_set_head(model, head, vfn.data());
        if (e) throw Error(e, k2t_last_error());
        *out = model;
        model = nullptr;
    });
    k2t_model_destroy(model);
    k2t_k2tb_close(f);
    return rc;
}

}  // extern "C"
