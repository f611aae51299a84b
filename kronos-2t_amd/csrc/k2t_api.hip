// C ABI of include/k2t_hip.h: argument validation, object lifetime, error mapping.
// Mirrors the FFI conventions of src/ffi/mobile_ffi.rs:76-168 (i32 status codes, a
// thread-local last error, catch-all at every entry, destroy(NULL) is a no-op).
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <string>
#include <vector>

#include "../../include/k2t_hip.h"
#include "k2t_expf.h"
#include "k2t_internal.h"

namespace k2t {

static thread_local std::string g_last_error;

void set_last_error(const std::string &msg) { g_last_error = msg; }

void hip_check(hipError_t e, const char *what) {
    if (e != hipSuccess) throw Error(K2T_E_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

static void arg_check(bool ok, const char *msg) {
    if (!ok) throw Error(K2T_E_ARG, msg);
}

template <typename F>
static int32_t guarded(F &&fn) {
    try {
        fn();
        return K2T_OK;
    } catch (const Error &e) {
        g_last_error = e.what();
        return e.code;
    } catch (const std::bad_alloc &) {
        g_last_error = "host allocation failed";
        return K2T_E_NOMEM;
    } catch (const std::exception &e) {
        g_last_error = e.what();
        return K2T_E_INTERNAL;
    } catch (...) {
        g_last_error = "unknown error";
        return K2T_E_INTERNAL;
    }
}

static void device_alloc(void **p, size_t bytes) {
    hipError_t e = hipMalloc(p, bytes ? bytes : 16);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        throw Error(K2T_E_NOMEM, std::string("hipMalloc failed: ") + hipGetErrorString(e));
    }
}

void ensure_scratch(k2t_ctx *ctx, size_t floats) {
    hip_check(hipSetDevice(ctx->device), "hipSetDevice");
    if (floats <= ctx->scratch_cap) return;
    // Queued kernels may still use the old buffer.
    hip_check(hipStreamSynchronize(ctx->stream), "scratch sync");
    if (ctx->scratch) hip_check(hipFree(ctx->scratch), "hipFree");
    ctx->scratch = nullptr;
    ctx->scratch_cap = 0;
    const size_t cap = std::max(floats, (size_t)1 << 16);
    device_alloc((void **)&ctx->scratch, cap * sizeof(float));
    ctx->scratch_cap = cap;
}

static size_t nibble4_pair_len(int rows, int cols, int hp) {
    size_t stripes = (size_t)(rows + 15) / 16;
    return (stripes / 2) * (size_t)(cols / 64) * (1024 + 256 * (size_t)hp + 64);
}
static size_t nibble4_tail_len(int rows, int cols, int hp) {
    size_t stripes = (size_t)(rows + 15) / 16;
    return (stripes & 1) * (size_t)(cols / 64) * (512 + 128 * (size_t)hp + 32);
}
// Bytes per stripe-chunk: NF4 512 (nibbles), NF3 384 (48-byte triplet blocks),
// NfSdotMatrix::chunk_bytes (simd_lut.rs:4826-4833).
static size_t nf_chunk_bytes(int bits) { return bits == 3 ? 384 : 512; }
static size_t nf_pair_len(int rows, int cols, int bits, int sgc) {
    size_t stripes = (size_t)(rows + 15) / 16, nc = (size_t)cols / 64, nsg = (nc + sgc - 1) / sgc;
    return (stripes / 2) * (nsg * 64 + nc * 2 * nf_chunk_bytes(bits));
}
static size_t nf_tail_len(int rows, int cols, int bits, int sgc) {
    size_t stripes = (size_t)(rows + 15) / 16, nc = (size_t)cols / 64, nsg = (nc + sgc - 1) / sgc;
    return (stripes & 1) * (nsg * 32 + nc * nf_chunk_bytes(bits));
}

static void fill_common(k2t_mat *m, int rows, int cols) {
    m->rows = rows;
    m->cols = cols;
    m->nc = cols / 64;
    m->stripes = (rows + 15) / 16;
    m->pairs = m->stripes / 2;
    m->has_tail = m->stripes & 1;
}

static void check_shape(int rows, int cols) {
    arg_check(rows > 0 && cols > 0, "rows and cols must be positive");
    arg_check(cols % 64 == 0, "cols must be a multiple of 64");
    arg_check(cols <= 32768 && rows <= (1 << 26), "matrix too large (cols <= 32768, rows <= 2^26)");
}

static void upload_streams(k2t_mat *m, const uint8_t *pair, size_t pl, const uint8_t *tail,
                           size_t tl, bool device_src) {
    if (device_src) {
        arg_check(pl == 0 || pair, "pair stream is NULL");
        arg_check(tl == 0 || tail, "tail stream is NULL");
        arg_check(((uintptr_t)pair % 16) == 0 && ((uintptr_t)tail % 16) == 0,
                  "device streams must be 16-byte aligned");
        m->pair = pair;
        m->tail = tail;
        m->owns = false;
        return;
    }
    arg_check(pl == 0 || pair, "pair stream is NULL");
    arg_check(tl == 0 || tail, "tail stream is NULL");
    void *dp = nullptr, *dt = nullptr;
    hip_check(hipSetDevice(m->ctx->device), "hipSetDevice");
    device_alloc(&dp, pl);
    if (tl) {
        try {
            device_alloc(&dt, tl);
        } catch (...) {
            (void)hipFree(dp);
            throw;
        }
    }
    if (pl) hip_check(hipMemcpy(dp, pair, pl, hipMemcpyHostToDevice), "upload pair stream");
    if (tl) hip_check(hipMemcpy(dt, tail, tl, hipMemcpyHostToDevice), "upload tail stream");
    m->pair = (const uint8_t *)dp;
    m->tail = (const uint8_t *)dt;
    m->owns = true;
}

static k2t_mat *make_nibble4(k2t_ctx *ctx, int rows, int cols, int hp, const void *pair, size_t pl,
                             const void *tail, size_t tl, bool device_src) {
    arg_check(ctx != nullptr, "ctx is NULL");
    check_shape(rows, cols);
    arg_check(hp >= 0 && hp <= 2, "hi_planes must be 0, 1 or 2");
    arg_check(pl == nibble4_pair_len(rows, cols, hp), "pair stream length does not match the Nibble4 layout");
    arg_check(tl == nibble4_tail_len(rows, cols, hp), "tail stream length does not match the Nibble4 layout");
    k2t_mat *m = new k2t_mat();
    m->ctx = ctx;
    m->device = ctx->device;
    m->fmt = K2T_FMT_NIBBLE4;
    m->hp = hp;
    fill_common(m, rows, cols);
    m->pair_len = pl;
    m->tail_len = tl;
    try {
        upload_streams(m, (const uint8_t *)pair, pl, (const uint8_t *)tail, tl, device_src);
    } catch (...) {
        delete m;
        throw;
    }
    return m;
}

// NF3 streams in place into lane order (a no-op for other formats and for matrices
// already converted); synchronous.
static void nf3_to_lane_order(k2t_mat *m) {
    if (m->fmt != K2T_FMT_NF || m->bits != 3 || m->nf3_lane) return;
    hip_check(hipSetDevice(m->device), "hipSetDevice");
    if (m->pairs)
        launch_nf3_lane_order(m->ctx->stream, const_cast<uint8_t *>(m->pair), 0, 1, m->pair_len / m->pairs, m->pairs,
                              m->nc, m->sgc, false);
    if (m->has_tail)
        launch_nf3_lane_order(m->ctx->stream, const_cast<uint8_t *>(m->tail), 0, 1, 0, 1, m->nc, m->sgc, true);
    hip_check(hipStreamSynchronize(m->ctx->stream), "nf3 lane order");
    m->nf3_lane = 1;
}

static k2t_mat *make_nf(k2t_ctx *ctx, int rows, int cols, int bits, int sgc, const int8_t *cb,
                        const void *pair, size_t pl, const void *tail, size_t tl, bool device_src) {
    arg_check(ctx != nullptr, "ctx is NULL");
    check_shape(rows, cols);
    arg_check(bits == 3 || bits == 4, "NF codebook stripes must have 3 or 4 bits");
    arg_check(sgc >= 1 && sgc <= 8, "scale_group_chunks must be in 1..8");
    arg_check(cb != nullptr, "codebook is NULL");
    arg_check(pl == nf_pair_len(rows, cols, bits, sgc), "pair stream length does not match the NF layout");
    arg_check(tl == nf_tail_len(rows, cols, bits, sgc), "tail stream length does not match the NF layout");
    k2t_mat *m = new k2t_mat();
    m->ctx = ctx;
    m->device = ctx->device;
    m->fmt = K2T_FMT_NF;
    m->bits = bits;
    m->sgc = sgc;
    for (int i = 0; i < 4; i++)
        m->cb[i] = (uint32_t)(uint8_t)cb[4 * i] | ((uint32_t)(uint8_t)cb[4 * i + 1] << 8) |
                   ((uint32_t)(uint8_t)cb[4 * i + 2] << 16) | ((uint32_t)(uint8_t)cb[4 * i + 3] << 24);
    fill_common(m, rows, cols);
    m->pair_len = pl;
    m->tail_len = tl;
    try {
        upload_streams(m, (const uint8_t *)pair, pl, (const uint8_t *)tail, tl, device_src);
        if (!device_src && bits == 3) nf3_to_lane_order(m);  // our own copy: the fast layout
    } catch (...) {
        k2t_mat_destroy(m);
        throw;
    }
    return m;
}

}  // namespace k2t

using namespace k2t;

extern "C" {

const char *k2t_version(void) { return "k2t-hip 0.1.0 gfx950"; }

const char *k2t_last_error(void) { return g_last_error.c_str(); }

int32_t k2t_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return n;
}

int32_t k2t_ctx_create(int32_t device, k2t_ctx **out) {
    return guarded([&] {
        arg_check(out != nullptr, "out is NULL");
        *out = nullptr;
        int n = 0;
        hip_check(hipGetDeviceCount(&n), "hipGetDeviceCount");
        arg_check(device >= 0 && device < n, "device index out of range");
        hip_check(hipSetDevice(device), "hipSetDevice");
        k2t_ctx *c = new k2t_ctx();
        c->device = device;
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) == hipSuccess && cus > 0)
            c->num_cus = cus;
        uint64_t masks[kSignBlocks];
        for (int b = 0; b < kSignBlocks; b++) masks[b] = hadamard_sign_mask_host((uint64_t)b);
        hipError_t e = hipMalloc(&c->signs, sizeof(masks));
        if (e == hipSuccess) e = hipMemcpy(c->signs, masks, sizeof(masks), hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            if (c->signs) (void)hipFree(c->signs);
            delete c;
            hip_check(e, "sign table");
        }
        *out = c;
    });
}

void k2t_ctx_destroy(k2t_ctx *ctx) {
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    if (ctx->scratch) (void)hipFree(ctx->scratch);
    if (ctx->rms_scratch) (void)hipFree(ctx->rms_scratch);
    if (ctx->gqa_words) (void)hipFree(ctx->gqa_words);
    if (ctx->signs) (void)hipFree(ctx->signs);
    delete ctx;
}

int32_t k2t_ctx_set_stream(k2t_ctx *ctx, void *hip_stream) {
    return guarded([&] {
        arg_check(ctx != nullptr, "ctx is NULL");
        ctx->stream = (hipStream_t)hip_stream;
    });
}

int32_t k2t_ctx_sync(k2t_ctx *ctx) {
    return guarded([&] {
        arg_check(ctx != nullptr, "ctx is NULL");
        hip_check(hipSetDevice(ctx->device), "hipSetDevice");
        hip_check(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
        check_gqa_timeout(ctx);
    });
}

int32_t k2t_ctx_set_splitk(k2t_ctx *ctx, int32_t max_segments) {
    return guarded([&] {
        arg_check(ctx != nullptr, "ctx is NULL");
        arg_check(max_segments >= 0 && max_segments <= 4096, "max_segments out of range");
        ctx->max_segments = max_segments;
    });
}

int32_t k2t_ctx_set_exact(k2t_ctx *ctx, int32_t exact) {
    return guarded([&] {
        arg_check(ctx != nullptr, "ctx is NULL");
        ctx->exact = exact ? 1 : 0;
    });
}

int32_t k2t_ctx_set_mfma(k2t_ctx *ctx, int32_t enable) {
    return guarded([&] {
        arg_check(ctx != nullptr, "ctx is NULL");
        arg_check(enable >= 0 && enable <= 2, "mfma mode must be 0, 1 or 2");
        ctx->mfma = enable;
    });
}

int32_t k2t_malloc(k2t_ctx *ctx, size_t bytes, void **d_out) {
    return guarded([&] {
        arg_check(ctx && d_out, "NULL argument");
        hip_check(hipSetDevice(ctx->device), "hipSetDevice");
        device_alloc(d_out, bytes);
    });
}

int32_t k2t_free(k2t_ctx *ctx, void *d_ptr) {
    return guarded([&] {
        arg_check(ctx != nullptr, "ctx is NULL");
        if (!d_ptr) return;
        hip_check(hipSetDevice(ctx->device), "hipSetDevice");
        hip_check(hipFree(d_ptr), "hipFree");
    });
}

int32_t k2t_memcpy_h2d(k2t_ctx *ctx, void *d_dst, const void *src, size_t bytes) {
    return guarded([&] {
        arg_check(ctx && (bytes == 0 || (d_dst && src)), "NULL argument");
        hip_check(hipSetDevice(ctx->device), "hipSetDevice");
        hip_check(hipMemcpyAsync(d_dst, src, bytes, hipMemcpyHostToDevice, ctx->stream), "h2d copy");
        hip_check(hipStreamSynchronize(ctx->stream), "h2d sync");
    });
}

int32_t k2t_memcpy_d2h(k2t_ctx *ctx, void *dst, const void *d_src, size_t bytes) {
    return guarded([&] {
        arg_check(ctx && (bytes == 0 || (dst && d_src)), "NULL argument");
        hip_check(hipSetDevice(ctx->device), "hipSetDevice");
        hip_check(hipMemcpyAsync(dst, d_src, bytes, hipMemcpyDeviceToHost, ctx->stream), "d2h copy");
        hip_check(hipStreamSynchronize(ctx->stream), "d2h sync");
    });
}

int32_t k2t_mat_upload_nibble4(k2t_ctx *ctx, int32_t rows, int32_t cols, int32_t hi_planes,
                               const uint8_t *pair, size_t pair_len, const uint8_t *tail,
                               size_t tail_len, k2t_mat **out) {
    return guarded([&] {
        arg_check(out != nullptr, "out is NULL");
        *out = make_nibble4(ctx, rows, cols, hi_planes, pair, pair_len, tail, tail_len, false);
    });
}

int32_t k2t_mat_upload_nf(k2t_ctx *ctx, int32_t rows, int32_t cols, int32_t bits, int32_t sgc,
                          const int8_t *codebook16, const uint8_t *pair, size_t pair_len,
                          const uint8_t *tail, size_t tail_len, k2t_mat **out) {
    return guarded([&] {
        arg_check(out != nullptr, "out is NULL");
        *out = make_nf(ctx, rows, cols, bits, sgc, codebook16, pair, pair_len, tail, tail_len, false);
    });
}

int32_t k2t_mat_wrap_nibble4(k2t_ctx *ctx, int32_t rows, int32_t cols, int32_t hi_planes,
                             const void *d_pair, size_t pair_len, const void *d_tail,
                             size_t tail_len, k2t_mat **out) {
    return guarded([&] {
        arg_check(out != nullptr, "out is NULL");
        *out = make_nibble4(ctx, rows, cols, hi_planes, d_pair, pair_len, d_tail, tail_len, true);
    });
}

int32_t k2t_mat_wrap_nf(k2t_ctx *ctx, int32_t rows, int32_t cols, int32_t bits, int32_t sgc,
                        const int8_t *codebook16, const void *d_pair, size_t pair_len,
                        const void *d_tail, size_t tail_len, k2t_mat **out) {
    return guarded([&] {
        arg_check(out != nullptr, "out is NULL");
        *out = make_nf(ctx, rows, cols, bits, sgc, codebook16, d_pair, pair_len, d_tail, tail_len, true);
    });
}

int32_t k2t_mat_nf3_lane_order(k2t_mat *m) {
    return guarded([&] {
        arg_check(m != nullptr, "mat is NULL");
        nf3_to_lane_order(m);
    });
}

void k2t_mat_destroy(k2t_mat *m) {
    if (!m) return;
    if (m->owns) {
        // hipFree waits for work queued on the device; the context may already be gone.
        (void)hipSetDevice(m->device);
        if (m->pair) (void)hipFree((void *)m->pair);
        if (m->tail) (void)hipFree((void *)m->tail);
    }
    delete m;
}

int32_t k2t_mat_info(const k2t_mat *m, int32_t *rows, int32_t *cols, int32_t *stripes, uint64_t *bytes) {
    return guarded([&] {
        arg_check(m != nullptr, "mat is NULL");
        if (rows) *rows = m->rows;
        if (cols) *cols = m->cols;
        if (stripes) *stripes = m->stripes;
        if (bytes) *bytes = m->pair_len + m->tail_len + (m->fmt == K2T_FMT_NF ? 16 : 0);
    });
}

int32_t k2t_act_quant(k2t_ctx *ctx, const float *d_x, const float *d_norm_w, const float *d_inv_rms,
                      int32_t K, int32_t ntok, int8_t *d_q, float *d_scales, int32_t *d_sums) {
    return guarded([&] {
        arg_check(ctx != nullptr, "ctx is NULL");
        arg_check(K > 0 && K % 64 == 0, "K must be a positive multiple of 64");
        arg_check(ntok >= 0, "ntok must be >= 0");
        arg_check(!d_norm_w || d_inv_rms, "norm weights need inv_rms");
        arg_check(ntok == 0 || (d_x && d_q && d_scales && d_sums), "NULL buffer");
        hip_check(hipSetDevice(ctx->device), "hipSetDevice");
        launch_act_quant(ctx, d_x, d_norm_w, d_inv_rms, K, ntok, d_q, d_scales, d_sums);
    });
}

int32_t k2t_act_quant_rmsnorm(k2t_ctx *ctx, const float *d_x, const float *d_norm_w, float eps,
                              int32_t K, int32_t ntok, int8_t *d_q, float *d_scales, int32_t *d_sums) {
    return guarded([&] {
        arg_check(ctx != nullptr, "ctx is NULL");
        arg_check(K > 0 && K % 64 == 0, "K must be a positive multiple of 64");
        arg_check(ntok >= 0, "ntok must be >= 0");
        arg_check(ntok == 0 || (d_x && d_norm_w && d_q && d_scales && d_sums), "NULL buffer");
        if (ntok == 0) return;
        hip_check(hipSetDevice(ctx->device), "hipSetDevice");
        if ((size_t)ntok > ctx->rms_cap) {
            hip_check(hipStreamSynchronize(ctx->stream), "scratch sync");
            if (ctx->rms_scratch) hip_check(hipFree(ctx->rms_scratch), "hipFree");
            ctx->rms_scratch = nullptr;
            size_t cap = std::max((size_t)ntok, (size_t)1024);
            device_alloc((void **)&ctx->rms_scratch, cap * sizeof(float));
            ctx->rms_cap = cap;
        }
        launch_inv_rms(ctx, d_x, eps, K, ntok, ctx->rms_scratch);
        launch_act_quant(ctx, d_x, d_norm_w, ctx->rms_scratch, K, ntok, d_q, d_scales, d_sums);
    });
}

int32_t k2t_gemv(k2t_ctx *ctx, const k2t_mat *m, const int8_t *d_xq, const float *d_xs,
                 const int32_t *d_xsum, int32_t ntok, int32_t s0, int32_t s1, float *d_out,
                 size_t out_stride) {
    return guarded([&] {
        arg_check(ctx && m, "NULL ctx or matrix");
        arg_check(m->ctx == ctx, "matrix belongs to another context");
        arg_check(ntok >= 0, "ntok must be >= 0");
        if (s1 < 0) s1 = m->stripes;
        arg_check(s0 >= 0 && s0 <= s1 && s1 <= m->stripes, "stripe range out of bounds");
        if (ntok == 0 || s0 == s1) return;
        arg_check(d_xq && d_xs && d_out, "NULL buffer");
        arg_check(m->fmt != K2T_FMT_NIBBLE4 || d_xsum, "bit-plane GEMV needs activation sums");
        arg_check(ntok == 1 || out_stride >= (size_t)m->rows, "out_stride smaller than rows");
        arg_check(((uintptr_t)d_xq % 8) == 0, "activations must be 8-byte aligned");
        hip_check(hipSetDevice(ctx->device), "hipSetDevice");
        launch_gemv(ctx, m, d_xq, d_xs, d_xsum, ntok, s0, s1, d_out, ntok == 1 ? (size_t)m->rows : out_stride,
                    nullptr);
    });
}

float k2t_expf_host(float x) { return expf_rn(x); }

int32_t k2t_expf_device(k2t_ctx *ctx, const float *d_x, float *d_y, size_t n) {
    return guarded([&] {
        arg_check(ctx && d_x && d_y, "NULL argument");
        if (n == 0) return;
        hip_check(hipSetDevice(ctx->device), "hipSetDevice");
        launch_expf_map(ctx->stream, d_x, d_y, n);
    });
}

int32_t k2t_stream_read_probe(k2t_ctx *ctx, const void *d_src, size_t bytes, uint32_t *d_sink) {
    return guarded([&] {
        arg_check(ctx && d_src && d_sink, "NULL argument");
        arg_check(bytes % 16 == 0 && ((uintptr_t)d_src & 15) == 0, "bytes and d_src must be 16-byte aligned");
        hip_check(hipSetDevice(ctx->device), "hipSetDevice");
        launch_stream_read(ctx->stream, d_src, bytes, d_sink);
    });
}

int32_t k2t_gemv_chunk_dots(k2t_ctx *ctx, const k2t_mat *m, const int8_t *d_xq, const int32_t *d_xsum,
                            int32_t *d_dots) {
    return guarded([&] {
        arg_check(ctx && m, "NULL ctx or matrix");
        arg_check(m->ctx == ctx, "matrix belongs to another context");
        arg_check(d_xq && d_dots, "NULL buffer");
        arg_check(m->fmt != K2T_FMT_NIBBLE4 || d_xsum, "bit-plane GEMV needs activation sums");
        hip_check(hipSetDevice(ctx->device), "hipSetDevice");
        // The scales are irrelevant to the integer dots; a scratch row of ones keeps the
        // fp32 epilogue well defined.  The float output goes to the split-K scratch.
        const size_t nc = (size_t)m->nc;
        ensure_scratch(ctx, nc + (size_t)m->stripes * 16);
        float *ones = ctx->scratch;
        std::vector<float> h(nc, 1.0f);
        hip_check(hipMemcpyAsync(ones, h.data(), nc * sizeof(float), hipMemcpyHostToDevice, ctx->stream),
                  "h2d");
        launch_gemv(ctx, m, d_xq, ones, d_xsum, 1, 0, m->stripes, ctx->scratch + nc, (size_t)m->rows, d_dots);
        hip_check(hipStreamSynchronize(ctx->stream), "sync");
    });
}

}  // extern "C"
