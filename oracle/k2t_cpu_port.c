/*
 * TEST INFRASTRUCTURE ONLY: the timed CPU baseline of bench.py (its cpu_baseline leg),
 * never part of the product library.
 *
 * The reference's portable x86 decode step (forward_token_sdot_megakernel's order,
 * real_llm.rs:6794-7403, with the non-aarch64 leaves) driven from C: per layer RMSNorm +
 * FWHT + int8 (simd_lut.rs:2954-2997), the qkv GEMV, RoPE (real_llm.rs:9328-9361) and the
 * Hadamard int8 K/V store (8282-8365), q8 attention per q head (8533-8545, 8575-8585),
 * FWHT + int8 of the heads, the o GEMV and residual, RMSNorm + gate_up GEMV, SwiGLU
 * (9801-9805) + FWHT + int8, the down GEMV and residual; then the final norm and the
 * lm_head GEMV.  Every GEMV is the portable dequantize + fp32 dot path
 * (nf_sdot_stripe_range_scalar_raw, simd_lut.rs:5719-5748, and its bit-plane twin
 * 3558-3581), split over a pool of host threads by stripe ranges the way the reference's
 * pool deals them out (real_llm.rs:829-836: grain ((S / (2T)) & !1) clamped to 2..128,
 * chunks taken in order by whichever thread is free).  The arithmetic is the oracle's
 * (k2t_oracle.c); this file adds only the C decode loop and the thread pool, and the
 * Makefile builds the pair at -O3 -march=native into libk2t_cpu_port.so, separately from
 * the parity oracle.  The embedding is the tied quantized head's row (embed_token_into,
 * real_llm.rs:8063-8097).
 */
#define _POSIX_C_SOURCE 200809L
#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* the oracle functions this loop calls (k2t_oracle.c) */
void or_populate_fwht(const float *x, const float *w, float inv_rms, size_t K, int8_t *q, float *scales,
                      int32_t *sums);
float or_inv_rms(const float *x, size_t n, float eps);
void or_nibble4_gemv_portable(const uint8_t *pair, const uint8_t *tail, size_t rows, size_t cols, int hp,
                              const int8_t *xq, const float *xs, size_t s0, size_t s1, float *out);
void or_nf_gemv_portable(const uint8_t *pair, const uint8_t *tail, size_t rows, size_t cols, int bits,
                         size_t sgc, const int8_t *cb16, const int8_t *xq, const float *xs, size_t s0, size_t s1,
                         float *out);
void or_nibble4_dequant_row(const uint8_t *pair, const uint8_t *tail, size_t rows, size_t cols, int hp, size_t r,
                            float *out);
void or_nf_dequant_row(const uint8_t *pair, const uint8_t *tail, size_t rows, size_t cols, int bits, size_t sgc,
                       const int8_t *cb16, size_t r, float *out);
void or_ifwht64(float *x, size_t n);
void or_kv_quant_head(const float *src, size_t hd, int8_t *q, float *scale);
void or_attn_q8_head(const float *q_head, const int8_t *k_q8, const float *ks, const int8_t *v_q8,
                     const float *vs, size_t seq, size_t hd, float attn_scale, float *out, float *scores);
void or_rope_row(size_t hd, double theta, size_t pos, float *row);
void or_rope_apply(float *head, size_t hd, const float *row);
void or_swiglu(const float *g, const float *u, float *out, size_t n);

typedef struct {
    int fmt; /* 0 bit planes, 1 NF */
    int hp, bits, sgc;
    size_t rows, cols;
    const uint8_t *pair, *tail;
    int8_t cb[16];
} cp_mat;

typedef struct cp_model cp_model;

/* one GEMV job of the pool */
typedef struct {
    const cp_mat *m;
    const int8_t *xq;
    const float *xs;
    float *out;
    size_t stripes, grain;
    atomic_size_t next;
} cp_job;

struct cp_model {
    int L, d, nq, nkv, hd, inter, vocab, max_seq, threads;
    float eps;
    double theta;
    cp_mat *mats; /* 4 per layer (qkv, o, gate_up interleaved, down), then the head */
    const float **in_norm, **post_norm, *final_norm;
    int8_t *kq, *vq;
    float *ks, *vs;
    int pos;
    /* scratch */
    float *hidden, *qkv, *gu, *att, *tmp, *scores, *rope;
    int8_t *xq;
    float *xs;
    int32_t *xsum;
    /* pool */
    pthread_t *th;
    pthread_barrier_t start, done;
    cp_job job;
    int quit;
};

static void run_job(cp_job *j) {
    for (;;) {
        size_t s0 = atomic_fetch_add(&j->next, j->grain);
        if (s0 >= j->stripes) break;
        size_t s1 = s0 + j->grain < j->stripes ? s0 + j->grain : j->stripes;
        const cp_mat *m = j->m;
        if (m->fmt == 0)
            or_nibble4_gemv_portable(m->pair, m->tail, m->rows, m->cols, m->hp, j->xq, j->xs, s0, s1, j->out);
        else
            or_nf_gemv_portable(m->pair, m->tail, m->rows, m->cols, m->bits, (size_t)m->sgc, m->cb, j->xq, j->xs, s0,
                                s1, j->out);
    }
}

static void *worker(void *p) {
    cp_model *m = (cp_model *)p;
    for (;;) {
        pthread_barrier_wait(&m->start);
        if (m->quit) break;
        run_job(&m->job);
        pthread_barrier_wait(&m->done);
    }
    return NULL;
}

/* out[0..rows) = m . x over the pool (the calling thread takes part) */
static void gemv(cp_model *md, const cp_mat *m, float *out) {
    cp_job *j = &md->job;
    j->m = m;
    j->xq = md->xq;
    j->xs = md->xs;
    j->out = out;
    j->stripes = (m->rows + 15) / 16;
    size_t g = (j->stripes / (2 * (size_t)md->threads)) & ~(size_t)1;
    j->grain = g < 2 ? 2 : g > 128 ? 128 : g;
    atomic_store(&j->next, 0);
    if (md->threads > 1) pthread_barrier_wait(&md->start);
    run_job(j);
    if (md->threads > 1) pthread_barrier_wait(&md->done);
}

cp_model *cp_model_create(int n_layers, int hidden, int n_heads, int n_kv_heads, int head_dim, int inter,
                          int vocab, int max_seq, float eps, double rope_theta, int threads) {
    cp_model *m = (cp_model *)calloc(1, sizeof(cp_model));
    m->L = n_layers;
    m->d = hidden;
    m->nq = n_heads;
    m->nkv = n_kv_heads;
    m->hd = head_dim;
    m->inter = inter;
    m->vocab = vocab;
    m->max_seq = max_seq;
    m->eps = eps;
    m->theta = rope_theta;
    m->threads = threads < 1 ? 1 : threads;
    m->mats = (cp_mat *)calloc((size_t)4 * n_layers + 1, sizeof(cp_mat));
    m->in_norm = (const float **)calloc((size_t)n_layers, sizeof(float *));
    m->post_norm = (const float **)calloc((size_t)n_layers, sizeof(float *));
    const size_t slots = (size_t)n_layers * n_kv_heads * max_seq;
    m->kq = (int8_t *)calloc(slots * head_dim, 1);
    m->vq = (int8_t *)calloc(slots * head_dim, 1);
    m->ks = (float *)calloc(slots, sizeof(float));
    m->vs = (float *)calloc(slots, sizeof(float));
    const size_t qkv_w = (size_t)(n_heads + 2 * n_kv_heads) * head_dim;
    size_t kmax = (size_t)hidden > (size_t)inter ? (size_t)hidden : (size_t)inter;
    if ((size_t)n_heads * head_dim > kmax) kmax = (size_t)n_heads * head_dim;
    m->hidden = (float *)calloc(hidden, sizeof(float));
    m->qkv = (float *)calloc(qkv_w, sizeof(float));
    m->gu = (float *)calloc((size_t)2 * inter, sizeof(float));
    m->att = (float *)calloc((size_t)n_heads * head_dim, sizeof(float));
    m->tmp = (float *)calloc(kmax > (size_t)hidden ? kmax : (size_t)hidden, sizeof(float));
    m->scores = (float *)calloc((size_t)max_seq, sizeof(float));
    m->rope = (float *)calloc((size_t)head_dim, sizeof(float));
    m->xq = (int8_t *)calloc(kmax, 1);
    m->xs = (float *)calloc(kmax / 64, sizeof(float));
    m->xsum = (int32_t *)calloc(kmax / 64, sizeof(int32_t));
    if (m->threads > 1) {
        pthread_barrier_init(&m->start, NULL, (unsigned)m->threads);
        pthread_barrier_init(&m->done, NULL, (unsigned)m->threads);
        m->th = (pthread_t *)calloc((size_t)m->threads - 1, sizeof(pthread_t));
        for (int t = 0; t < m->threads - 1; t++) pthread_create(&m->th[t], NULL, worker, m);
    }
    return m;
}

/* Matrix idx = 4*layer + {0 qkv, 1 o, 2 gate_up (interleaved), 3 down}; 4*L = head.  fmt 0:
 * bit planes with hp hi planes; fmt 1: NF with `bits`, sgc and codebook cb.  The byte
 * streams are borrowed (the caller keeps them alive). */
void cp_model_set_matrix(cp_model *m, int idx, int fmt, int hp, int bits, int sgc, size_t rows, size_t cols,
                         const uint8_t *pair, const uint8_t *tail, const int8_t *cb) {
    cp_mat *x = &m->mats[idx];
    x->fmt = fmt;
    x->hp = hp;
    x->bits = bits;
    x->sgc = sgc;
    x->rows = rows;
    x->cols = cols;
    x->pair = pair;
    x->tail = tail;
    if (cb) memcpy(x->cb, cb, 16);
}

/* Norm weights (borrowed); layer = -1 sets the final norm. */
void cp_model_set_norms(cp_model *m, int layer, const float *in_norm, const float *post_norm) {
    if (layer < 0) {
        m->final_norm = in_norm;
        return;
    }
    m->in_norm[layer] = in_norm;
    m->post_norm[layer] = post_norm;
}

/* Positions 0 .. n_pos-1 of every layer's cache filled with seeded int8 K/V and scales in
 * [0.005, 0.05) (a prefilled context for timing); the position becomes n_pos. */
void cp_model_seed_kv(cp_model *m, int n_pos, uint64_t seed) {
    uint64_t s = seed * 0x9E3779B97F4A7C15ull + 1;
    for (int l = 0; l < m->L; l++)
        for (int h = 0; h < m->nkv; h++)
            for (int p = 0; p < n_pos; p++) {
                const size_t slot = ((size_t)l * m->nkv + h) * m->max_seq + p;
                for (int i = 0; i < m->hd; i++) {
                    s ^= s << 13;
                    s ^= s >> 7;
                    s ^= s << 17;
                    m->kq[slot * m->hd + i] = (int8_t)((int)(s % 255) - 127);
                    m->vq[slot * m->hd + i] = (int8_t)((int)((s >> 20) % 255) - 127);
                }
                m->ks[slot] = 0.005f + 0.045f * (float)((s >> 33) % 1000) / 1000.0f;
                m->vs[slot] = 0.005f + 0.045f * (float)((s >> 43) % 1000) / 1000.0f;
            }
    m->pos = n_pos;
}

static void embed(cp_model *m, int token) {
    const cp_mat *h = &m->mats[4 * m->L];
    if (h->fmt == 0)
        or_nibble4_dequant_row(h->pair, h->tail, h->rows, h->cols, h->hp, (size_t)token, m->hidden);
    else
        or_nf_dequant_row(h->pair, h->tail, h->rows, h->cols, h->bits, (size_t)h->sgc, h->cb, (size_t)token,
                          m->hidden);
    or_ifwht64(m->hidden, (size_t)m->d);
}

/* One decode step of `token` at the current position; logits (vocab floats) if not NULL. */
void cp_model_decode(cp_model *m, int token, float *logits) {
    const int d = m->d, nq = m->nq, nkv = m->nkv, hd = m->hd, inter = m->inter, pos = m->pos;
    const float scale = 1.0f / sqrtf((float)hd);
    embed(m, token);
    or_rope_row((size_t)hd, (double)(float)m->theta, (size_t)pos, m->rope);
    for (int l = 0; l < m->L; l++) {
        const cp_mat *W = &m->mats[4 * l];
        or_populate_fwht(m->hidden, m->in_norm[l], or_inv_rms(m->hidden, (size_t)d, m->eps), (size_t)d, m->xq, m->xs,
                         m->xsum);
        gemv(m, &W[0], m->qkv);
        for (int h = 0; h < nq + nkv; h++) or_rope_apply(m->qkv + (size_t)h * hd, (size_t)hd, m->rope);
        for (int h = 0; h < nkv; h++) {
            const size_t slot = ((size_t)l * nkv + h) * m->max_seq + pos;
            or_kv_quant_head(m->qkv + (size_t)(nq + h) * hd, (size_t)hd, m->kq + slot * hd, m->ks + slot);
            or_kv_quant_head(m->qkv + (size_t)(nq + nkv + h) * hd, (size_t)hd, m->vq + slot * hd, m->vs + slot);
        }
        const int group = nq / nkv;
        for (int h = 0; h < nq; h++) {
            const size_t base = ((size_t)l * nkv + h / group) * m->max_seq;
            or_attn_q8_head(m->qkv + (size_t)h * hd, m->kq + base * hd, m->ks + base, m->vq + base * hd, m->vs + base,
                            (size_t)pos + 1, (size_t)hd, scale, m->att + (size_t)h * hd, m->scores);
        }
        or_populate_fwht(m->att, NULL, 0.0f, (size_t)nq * hd, m->xq, m->xs, m->xsum);
        gemv(m, &W[1], m->tmp);
        for (int i = 0; i < d; i++) m->hidden[i] = m->hidden[i] + m->tmp[i];
        or_populate_fwht(m->hidden, m->post_norm[l], or_inv_rms(m->hidden, (size_t)d, m->eps), (size_t)d, m->xq,
                         m->xs, m->xsum);
        gemv(m, &W[2], m->gu);
        for (int ic = 0; ic < inter / 64; ic++)
            or_swiglu(m->gu + (size_t)ic * 128, m->gu + (size_t)ic * 128 + 64, m->tmp + (size_t)ic * 64, 64);
        or_populate_fwht(m->tmp, NULL, 0.0f, (size_t)inter, m->xq, m->xs, m->xsum);
        gemv(m, &W[3], m->tmp);
        for (int i = 0; i < d; i++) m->hidden[i] = m->hidden[i] + m->tmp[i];
    }
    m->pos++;
    if (!logits) return;
    or_populate_fwht(m->hidden, m->final_norm, or_inv_rms(m->hidden, (size_t)d, m->eps), (size_t)d, m->xq, m->xs,
                     m->xsum);
    gemv(m, &m->mats[4 * m->L], logits);
}

void cp_model_destroy(cp_model *m) {
    if (!m) return;
    if (m->threads > 1) {
        m->quit = 1;
        pthread_barrier_wait(&m->start);
        for (int t = 0; t < m->threads - 1; t++) pthread_join(m->th[t], NULL);
        pthread_barrier_destroy(&m->start);
        pthread_barrier_destroy(&m->done);
        free(m->th);
    }
    free(m->mats);
    free(m->in_norm);
    free(m->post_norm);
    free(m->kq);
    free(m->vq);
    free(m->ks);
    free(m->vs);
    free(m->hidden);
    free(m->qkv);
    free(m->gu);
    free(m->att);
    free(m->tmp);
    free(m->scores);
    free(m->rope);
    free(m->xq);
    free(m->xs);
    free(m->xsum);
    free(m);
}
