/*
 * k2t_hip.h -- C ABI of the MI355X (gfx950) kernels for kronos-2t's quantized
 * decode hot path.
 *
 * The reference's per-projection "backend trait" is the LinearBackend enum and
 * its stripe-range leaf kernels (src/model/real_llm.rs:525-544, 711-892;
 * src/kernels/simd_lut.rs).  Each entry point below names the reference item
 * it replaces.  A Rust host binds this header with a plain `extern "C"` block
 * declaring the same signatures; nothing here uses C++ or torch types.
 *
 * Conventions (mirroring include/kronos_ffi.h and src/ffi/mobile_ffi.rs:101-168):
 *   - every function returns int32_t: 0 = ok, < 0 = error code (K2T_E_*);
 *     k2t_last_error() returns a thread-local message for the last failure;
 *   - no C++ exception crosses the ABI; HIP errors map to K2T_E_HIP;
 *   - *_destroy(NULL) is a no-op;
 *   - pointers named d_* are device pointers; everything else is host memory;
 *   - calls are asynchronous on the context's stream (k2t_ctx_set_stream);
 *     the caller synchronizes (k2t_ctx_sync) before reading results;
 *   - a context owns scratch used by split-K GEMVs: use one context per
 *     stream; two calls that overlap on one context race.
 *
 * Data layouts are the reference's, unchanged:
 *   - bit-plane matrices: Nibble4SdotMatrix pair/tail streams
 *     (simd_lut.rs:3264-3400): per stripe pair and 64-column chunk a record of
 *     1024 + 256*hp + 64 bytes; odd last stripe in 512 + 128*hp + 32-byte records;
 *   - NF matrices: NfSdotMatrix pair/tail streams (simd_lut.rs:4796-5023):
 *     per pair and scale group 64 B of BF16 scales then sgc * 2 * 512 B (NF4);
 *   - activations: Int8ChunkActivation (simd_lut.rs:2921-2937): int8 q[K],
 *     f32 scales[K/64], i32 sums[K/64] per token, tokens back to back;
 *   - int8 Hadamard KV cache: QuantizedKvCache (real_llm.rs:1209-1412):
 *     slot = (layer*n_kv + kvh)*cap + pos, q8 at slot*hd, one f32 scale per slot.
 */
#ifndef K2T_HIP_H
#define K2T_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define K2T_OK 0
#define K2T_E_ARG (-1)     /* bad argument: NULL, shape, alignment, range */
#define K2T_E_HIP (-2)     /* HIP runtime error */
#define K2T_E_NOMEM (-3)   /* device allocation failed */
#define K2T_E_STATE (-4)   /* wrong object state / unsupported format */
#define K2T_E_INTERNAL (-5)

typedef struct k2t_ctx k2t_ctx;
typedef struct k2t_mat k2t_mat;
typedef struct k2t_experts k2t_experts; /* sparse-MoE expert bank (.k2tm shard in HBM) */

/* Library version string ("k2t-hip <semver> gfx950"). */
const char *k2t_version(void);

/* Thread-local message of the last failing call on this thread
 * (replaces kronos_last_error, mobile_ffi.rs:159-168). Never NULL. */
const char *k2t_last_error(void);

/* Number of visible HIP devices (0 when no GPU / no driver). Never fails. */
int32_t k2t_device_count(void);

/* ---- context ---------------------------------------------------------- */

/* Creates a context on `device` (its own scratch, default stream 0).
 * Replaces the per-engine SpinThreadPool + activation scratch
 * (thread_pool.rs:96-175, real_llm.rs:3610-3653). */
int32_t k2t_ctx_create(int32_t device, k2t_ctx **out);
void k2t_ctx_destroy(k2t_ctx *ctx);
/* Sets the hipStream_t (passed as void*) used by later calls; NULL = default stream. */
int32_t k2t_ctx_set_stream(k2t_ctx *ctx, void *hip_stream);
/* Blocks until all work queued on the context's stream is done. */
int32_t k2t_ctx_sync(k2t_ctx *ctx);
/* Cap on the K segments (waves per workgroup) k2t_gemv may use: 0 = automatic. */
int32_t k2t_ctx_set_splitk(k2t_ctx *ctx, int32_t max_segments);
/* fp32 epilogue of k2t_gemv.  exact = 1 replays the reference's per-row fmaf chain
 * in chunk order (simd_lut.rs:4030-4059, 6334-6335) and is bit-identical to it;
 * exact = 0 (default) sums per-segment chains in a fixed order: deterministic and
 * within a few ulp of the reference, and faster for long K.  Integer per-(row, chunk)
 * dots are exact in both modes. */
int32_t k2t_ctx_set_exact(k2t_ctx *ctx, int32_t exact);
/* Batched NF4 and bit-plane (b4 / b5 / b6) GEMVs (16 or more tokens of a ready activation
 * over the whole matrix, k2t_gemv and the model's prefill): enable = 1 (default) runs
 * them on the int8 matrix cores, one weight pass per 64 tokens, with outputs equal to the
 * exact-order epilogue's in either mode; 0 runs the 4-token weight passes of the
 * reference's tiles (nf_sdot_decode_neon, simd_lut.rs:6074-6364;
 * nibble4_sdot_batch_stripe_range, 4101-4320).  2: matrix cores, but a model's prefill does not have the
 * activation's producer write the tile-major copy the GEMV reads (the GEMV copies it
 * itself); same outputs as 1, for checking.  A backend choice of this build; the
 * reference has no counterpart.  K2T_E_ARG for other values. */
int32_t k2t_ctx_set_mfma(k2t_ctx *ctx, int32_t enable);

/* ---- device memory helpers (tests, benches, non-torch callers) ---------- */
int32_t k2t_malloc(k2t_ctx *ctx, size_t bytes, void **d_out);
int32_t k2t_free(k2t_ctx *ctx, void *d_ptr);
int32_t k2t_memcpy_h2d(k2t_ctx *ctx, void *d_dst, const void *src, size_t bytes);
int32_t k2t_memcpy_d2h(k2t_ctx *ctx, void *dst, const void *d_src, size_t bytes);

/* ---- matrices ----------------------------------------------------------- */

/* Uploads a Nibble4SdotMatrix (simd_lut.rs:3264-3277) as produced by
 * from_bipolar_with_perm (3297-3400): hi_planes = planes - 4 (0, 1 or 2).
 * pair_len must equal (stripes/2)*(cols/64)*(1024+256*hi_planes+64) and
 * tail_len (stripes&1)*(cols/64)*(512+128*hi_planes+32).  Bytes are copied. */
int32_t k2t_mat_upload_nibble4(k2t_ctx *ctx, int32_t rows, int32_t cols, int32_t hi_planes,
                               const uint8_t *pair, size_t pair_len, const uint8_t *tail,
                               size_t tail_len, k2t_mat **out);

/* Uploads an NfSdotMatrix (simd_lut.rs:4796-4842) with `bits` = 4 (NF4, 512-byte
 * stripe-chunks) or 3 (NF3, 384-byte stripe-chunks of 48-byte triplet blocks,
 * simd_lut.rs:4932-4960) and scale_group_chunks = sgc (1..8).  Lengths follow pair_total_bytes /
 * tail_total_bytes (simd_lut.rs:4834-4842).  codebook = the matrix's i8[16]. */
int32_t k2t_mat_upload_nf(k2t_ctx *ctx, int32_t rows, int32_t cols, int32_t bits, int32_t sgc,
                          const int8_t *codebook16, const uint8_t *pair, size_t pair_len,
                          const uint8_t *tail, size_t tail_len, k2t_mat **out);

/* Same as the uploads, but the streams already live in device memory; the
 * matrix borrows them (caller keeps them alive; destroy does not free them). */
int32_t k2t_mat_wrap_nibble4(k2t_ctx *ctx, int32_t rows, int32_t cols, int32_t hi_planes,
                             const void *d_pair, size_t pair_len, const void *d_tail,
                             size_t tail_len, k2t_mat **out);
int32_t k2t_mat_wrap_nf(k2t_ctx *ctx, int32_t rows, int32_t cols, int32_t bits, int32_t sgc,
                        const int8_t *codebook16, const void *d_pair, size_t pair_len,
                        const void *d_tail, size_t tail_len, k2t_mat **out);
/* No counterpart in the reference: a device-layout step.  An NF3 matrix's streams
 * rearranged IN PLACE into lane order (see k2t_experts_nf3_lane_order); k2t_mat_upload_nf
 * stores NF3 in this order, k2t_mat_wrap_nf leaves the borrowed bytes in the reference
 * layout until this call.  Results are unchanged; no-op for other formats and matrices
 * already converted; synchronous.  A dense stream carries no mark: wrap converted bytes
 * again only with a matrix that is then converted by no one (or re-upload them).  Every
 * other handle that already wraps the same bytes keeps reading them in the reference
 * order and gives wrong results afterwards: destroy such handles before converting. */
int32_t k2t_mat_nf3_lane_order(k2t_mat *m);
void k2t_mat_destroy(k2t_mat *m);
/* rows, cols, stripes and streamed bytes (pair + tail + codebook). */
int32_t k2t_mat_info(const k2t_mat *m, int32_t *rows, int32_t *cols, int32_t *stripes,
                     uint64_t *bytes);

/* ---- activations --------------------------------------------------------- */

/* Int8ChunkActivation::populate_fwht / populate_rmsnorm_fwht
 * (simd_lut.rs:2954-3196): per token t and chunk c of d_x[t*K ..],
 * optional (x*inv_rms[t])*w, signed FWHT-64 with the chunk's sign masks,
 * int8 round-half-even, scale = max/127, i32 sum.  d_norm_w and d_inv_rms may
 * both be NULL (plain FWHT); if d_norm_w is set, d_inv_rms must be too. */
int32_t k2t_act_quant(k2t_ctx *ctx, const float *d_x, const float *d_norm_w,
                      const float *d_inv_rms, int32_t K, int32_t ntok, int8_t *d_q,
                      float *d_scales, int32_t *d_sums);

/* RMSNorm + FWHT + int8 with inv_rms = 1/sqrt(mean(x^2) + eps) computed on the
 * device (real_llm.rs:6929 + simd_lut.rs:2970).  The sum of squares is a tree
 * reduction, so inv_rms may differ from the CPU's in the last ulp. */
int32_t k2t_act_quant_rmsnorm(k2t_ctx *ctx, const float *d_x, const float *d_norm_w, float eps,
                              int32_t K, int32_t ntok, int8_t *d_q, float *d_scales,
                              int32_t *d_sums);

/* ---- GEMV / multi-token tile -------------------------------------------- */

/* nibble4_sdot_stripe_range_raw (simd_lut.rs:3536-3582) and
 * nf_sdot_stripe_range_raw (5687-5713) for stripes [s0, s1) (s1 = -1: all),
 * and for ntok > 1 their batch variants nibble4_sdot_batch_stripe_range /
 * nf_sdot_batch_stripe_range (4101, 6689): token t reads d_xq + t*K,
 * d_xs + t*K/64, d_xsum + t*K/64 and writes d_out[t*out_stride + row].
 * Weights are read once per 4 tokens.  d_xsum is required for bit-plane
 * matrices and ignored for NF ones.  Per-(row, chunk) integer dots are exact;
 * with split-K disabled the fp32 result is bit-identical to the reference's
 * in-order fmaf epilogue.  16 or more tokens over the whole matrix (NF4 or bit
 * planes, k2t_ctx_set_mfma): one weight pass per 64 tokens on the matrix
 * cores, outputs bit-identical to that epilogue in either mode; such a call
 * copies the activation into the context's scratch, which it grows first if it
 * is too small (a synchronous allocation, so the first such call of a size
 * must not be inside a stream capture). */
int32_t k2t_gemv(k2t_ctx *ctx, const k2t_mat *m, const int8_t *d_xq, const float *d_xs,
                 const int32_t *d_xsum, int32_t ntok, int32_t s0, int32_t s1, float *d_out,
                 size_t out_stride);

/* Debug/parity: writes the exact integer dot of every (row, chunk) for one
 * token into d_dots[row * (K/64) + chunk] (Σ q·xq for bit-plane, Σ cb[idx]·xq
 * for NF).  No reference counterpart (the NEON kernel keeps them in registers,
 * simd_lut.rs:4030-4059); used to prove bit-exact integer accumulation. */
int32_t k2t_gemv_chunk_dots(k2t_ctx *ctx, const k2t_mat *m, const int8_t *d_xq,
                            const int32_t *d_xsum, int32_t *d_dots);

/* Measurement: one streaming read of `bytes` (16-byte aligned) from d_src, asynchronous on
 * the context's stream; d_sink receives a word only if the data's XOR equals a marker.
 * No reference counterpart: it gives the single-launch HBM read ceiling that the GEMV's
 * bandwidth is read against. */
/* Parity support (no reference counterpart): the exponential the exact-order mode uses,
 * which returns glibc's expf result for every fp32 input (f32::exp of the x86 reference
 * build, real_llm.rs:9595 and 9803).  k2t_expf_host runs the routine on the host;
 * k2t_expf_device applies it on the GPU to n floats (d_x to d_y, on the context's stream). */
float k2t_expf_host(float x);
int32_t k2t_expf_device(k2t_ctx *ctx, const float *d_x, float *d_y, size_t n);
int32_t k2t_stream_read_probe(k2t_ctx *ctx, const void *d_src, size_t bytes, uint32_t *d_sink);

/* ---- offline weight compiler (host memory, multi-threaded) ------------- */

/* Byte lengths of the pair / tail streams: fmt 1 = bit planes (planes 4..6),
 * fmt 2 = NF (bits 3 or 4, sgc 1..8).  Nibble4SdotMatrix::pair_rec_bytes /
 * NfSdotMatrix::pair_total_bytes (simd_lut.rs:3281-3288, 4834-4842). */
int32_t k2t_stream_sizes(int32_t fmt, int32_t rows, int32_t cols, int32_t planes_or_bits, int32_t sgc,
                         size_t *pair_len, size_t *tail_len);

/* compile_hadamard_gptq_bipolar without a Hessian (compiler.rs:912-1107: per-row
 * FWHT-64, 12-ratio RTN search, BF16 scale per row and chunk) followed by
 * Nibble4SdotMatrix::from_bipolar_with_perm (simd_lut.rs:3297-3400), written
 * directly into the caller's pair/tail buffers.  W is row-major [rows][cols] f32.
 * threads <= 0 uses every hardware thread. */
int32_t k2t_compile_bipolar(const float *W, int32_t rows, int32_t cols, int32_t planes,
                            int32_t interleave_gate_up, int32_t threads, uint8_t *pair, size_t pair_len,
                            uint8_t *tail, size_t tail_len);

/* compile_hadamard_gptq_nf without a Hessian for NF4 / NF3 (compiler.rs:1404-1866:
 * fitted Lloyd-Max codebook, 11-ratio RTN + least-squares BF16 refit) followed by
 * NfSdotMatrix::from_indices (simd_lut.rs:4850-5023) and, if requested,
 * to_gate_up_interleaved (5500-5523).  Writes the codebook and mu_top (nullable).
 * bits = 3 or 4. */
int32_t k2t_compile_nf(const float *W, int32_t rows, int32_t cols, int32_t bits, int32_t sgc,
                       int32_t interleave_gate_up, int32_t threads, int8_t *codebook16, float *mu_top,
                       uint8_t *pair, size_t pair_len, uint8_t *tail, size_t tail_len);

/* Seeded N(0, std) samples (SplitMix64 counter + Box-Muller) for synthetic
 * random-init weights; deterministic for a given (seed, n) at any thread count.
 * No reference counterpart (the reference loads checkpoints). */
int32_t k2t_synth_normal(uint64_t seed, float stddev, float *out, size_t n, int32_t threads);

/* ---- decode engine ------------------------------------------------------ */

/* Llama-family decoder shape (LlamaConfig, real_llm.rs:100-403); head_dim 64 or 128.
 * q_dim = n_heads * head_dim may differ from hidden (the generic decode path,
 * real_llm.rs:6485-6792); the persistent decode kernel needs q_dim == hidden (the
 * megakernel shape, real_llm.rs:6412-6452).  For MoE models `intermediate` is the dense
 * size (any positive multiple of 64 when every layer is MoE). */
typedef struct k2t_model_config {
    int32_t n_layers, hidden, n_heads, n_kv_heads, head_dim, intermediate, vocab, max_seq;
    float rms_eps;
    float rope_theta; /* effective theta (real_llm.rs:415-422) */
} k2t_model_config;

typedef struct k2t_model k2t_model;

/* Allocates the int8 Hadamard KV cache (QuantizedKvCache, real_llm.rs:1209-1412, full
 * max_seq capacity), the RoPE table (real_llm.rs:9212-9232) and workspaces for up to
 * max_batch tokens per forward pass. */
int32_t k2t_model_create(k2t_ctx *ctx, const k2t_model_config *cfg, int32_t max_batch, k2t_model **out);
void k2t_model_destroy(k2t_model *m);
/* Layer weights (borrowed matrices of the same context; gate_up must be row-interleaved
 * into [gate64(ic), up64(ic)] blocks as after repack_sdot, real_llm.rs:3657-3702) and
 * RMSNorm weights / optional qkv bias (host arrays, copied). */
int32_t k2t_model_set_layer(k2t_model *m, int32_t layer, const k2t_mat *qkv, const k2t_mat *o,
                            const k2t_mat *gate_up, const k2t_mat *down, const float *in_norm,
                            const float *post_norm, const float *qkv_bias);
/* Tied quantized lm_head (also the embedding table, embed_token_into real_llm.rs:8063-8097)
 * and the final norm. */
int32_t k2t_model_set_head(k2t_model *m, const k2t_mat *lm_head, const float *final_norm);
/* Embedding source, in embed_token_into's precedence (real_llm.rs:8063-8097):
 *   K2T_EMBED_TIED (default): row `token` of the quantized lm_head, dequantized in the
 *                   rotated domain and inverse-rotated (the lm_head must be NF4 or bit planes);
 *   K2T_EMBED_F32 / K2T_EMBED_BF16: untied rows [vocab][hidden] (host array, copied);
 *   K2T_EMBED_NF4:  an NF4 matrix [vocab][hidden] of the same context (borrowed),
 *                   read like the tied head (embed_nf4, real_llm.rs:8086-8090). */
#define K2T_EMBED_TIED 0
#define K2T_EMBED_F32 1
#define K2T_EMBED_BF16 2
#define K2T_EMBED_NF4 3
int32_t k2t_model_set_embedding(k2t_model *m, int32_t kind, const void *rows, const k2t_mat *nf4);
/* Per-head q / k RMSNorm weights [head_dim] (Qwen3 q_norm / k_norm; apply_qk_norm_rope,
 * real_llm.rs:8139-8178, applied before RoPE); NULL clears. */
int32_t k2t_model_set_qk_norm(k2t_model *m, int32_t layer, const float *q_norm, const float *k_norm);
/* Makes `layer` a sparse-MoE layer (set its attention first with k2t_model_set_layer and
 * gate_up = down = NULL): layer `shard_layer` of the expert bank (borrowed), an fp32
 * router [E][hidden] (+ bias [E] or NULL; host arrays, copied), top_k experts per
 * token, norm_topk_prob and scoring as in route_sorted (sparse_moe.rs:86-182).  The
 * feed-forward is forward_layer_single (sparse_moe.rs:961-1084) per token. */
int32_t k2t_model_set_moe(k2t_model *m, int32_t layer, const k2t_experts *bank, int32_t shard_layer,
                          const float *router_w, const float *router_bias, int32_t top_k, int32_t norm_topk_prob,
                          int32_t scoring);
/* The shared expert of a sparse-MoE layer (SharedMoeExpert with the NF backend,
 * sparse_moe.rs:209-312, applied in forward_layer_single 989-1000): gate_up, an NF matrix
 * [2 * inter][hidden] in [gate; up] row order (inter a multiple of 64), and down
 * [hidden][inter], both borrowed; gate_weight (host [hidden], copied) or NULL.  Each
 * token's MoE output becomes shared(x_norm) * scale + sum_k w_k expert_k(x_norm), with
 * scale = sigmoid(gate_weight . x_norm) (1 without a gate), before the residual add.
 * Call after k2t_model_set_moe; gate_up = NULL removes the shared expert. */
int32_t k2t_model_set_moe_shared(k2t_model *m, int32_t layer, const k2t_mat *gate_up, const k2t_mat *down,
                                 const float *gate_weight);
/* set_kv_sliding_window (real_llm.rs:1764-1790): an O(1) sliding-window + attention-sink
 * ring for the int8 KV cache (QuantizedKvCache::new_with_opts, real_llm.rs:1235-1257).
 * window >= 8 with window + 512 < max_seq enables it: sinks = min(sink_tokens, window/2),
 * ring = window - sinks + 512 slots; attention then covers the sinks and the last
 * window - sinks positions (active_kv_pos, real_llm.rs:8596-8612).  Any other window
 * (0 included) restores the full causal cache.  Resets the position to 0. */
int32_t k2t_model_set_kv_window(k2t_model *m, int32_t window, int32_t sink_tokens);
/* set_kv_bits (real_llm.rs:1732-1752): 8 (default) = int8 Hadamard KV with one f32 scale
 * per head; 4 = NF4-codebook Hadamard KV with a refined BF16 scale per 64-block
 * (store_hadamard_q4_head_raw, real_llm.rs:8646-8700).  Resets the position to 0. */
int32_t k2t_model_set_kv_bits(k2t_model *m, int32_t bits);
int32_t k2t_model_kv_bits(const k2t_model *m, int32_t *bits);
/* Active (window, sinks); (0, 0) for the full cache. */
int32_t k2t_model_kv_window(const k2t_model *m, int32_t *window, int32_t *sink_tokens);
/* Benchmark support (no reference counterpart): fills cache positions [0, n_pos) of every
 * layer with seeded pseudo-random int8 K/V and positive scales and sets the position to
 * n_pos, so a decode step runs at that context without a prefill. */
int32_t k2t_model_kv_synthetic(k2t_model *m, int32_t n_pos, uint64_t seed);
/* 1 (default): capture the decode step once and replay it as a HIP graph. */
int32_t k2t_model_set_graph(k2t_model *m, int32_t enable);
/* Operation order of this model's steps; default 0 = fast.
 * exact = 1 runs every step in the x86 reference build's operation order
 * (forward_token_sdot_megakernel's portable paths, real_llm.rs:6794-7403): GEMVs with the
 * in-order fmaf epilogue (k2t_ctx_set_exact), RMSNorm and q / k norm with the sequential
 * four-accumulator sum of squares (dot_f32_fast, real_llm.rs:911-926), softmax and SwiGLU
 * with glibc's expf results (k2t_expf_host), attention with sequential softmax and V sums
 * (real_llm.rs:8533-8545, 8575-8585, 9590-9600), and sparse-MoE layers with the sequential
 * router dot, route_sorted with glibc's expf and in-order sums (sparse_moe.rs:86-206,
 * 1644-1656).  Logits then equal the x86 reference's bit for bit with the int8 KV cache
 * (the NF4 KV cache is refused with K2T_E_ARG at the step).  Exact steps run the
 * persistent kernel's exact-order variant where the persistent kernel applies, else the
 * per-operation path; they are slower and meant for parity checks. */
int32_t k2t_model_set_exact(k2t_model *m, int32_t exact);
/* 1 (default): a decode step runs as one persistent kernel (one workgroup per CU) whose
 * phases hand vectors over through {payload, epoch} words instead of kernel boundaries:
 * the shape of forward_token_sdot_megakernel (real_llm.rs:6794-7403).  0: one kernel per
 * operation.  Used only with the fast epilogue, when every matrix is NF4 or every matrix
 * has 4 bit planes, and the device and model shape allow it (see
 * k2t_model_persistent_active); otherwise the per-operation path runs.  Bit-plane models
 * that mix 4- and 5-plane matrices (p55454) run a 256-thread variant.  2: the same as 1
 * (kept for callers of the earlier interface, where 1 left mixed-plane models on the
 * per-operation path).  A step that attends more than 1024 positions runs the
 * per-operation path (a few workgroups per head scanning the context are slower there). */
int32_t k2t_model_set_persistent(k2t_model *m, int32_t enable);
/* The hipStream_t (as void*) this model's steps are enqueued on: for the caller's own
 * events around a step (bench timing) or waits.  Measurement support, no reference
 * counterpart. */
int32_t k2t_model_stream(const k2t_model *m, void **hip_stream);
/* Whether the next decode step (at the current position) runs the persistent kernel. */
int32_t k2t_model_persistent_active(const k2t_model *m, int32_t *active);
/* reset_context: position back to 0. */
int32_t k2t_model_reset(k2t_model *m);
int32_t k2t_model_position(const k2t_model *m, int32_t *pos);
/* forward_token (real_llm.rs:6455, megakernel 6794-7403): one decode step; logits of
 * `token` are copied to logits_host (vocab floats) when it is not NULL. */
int32_t k2t_model_decode(k2t_model *m, int32_t token, float *logits_host);
/* forward_prompt (real_llm.rs:7407-7446): the prompt in batches of max_batch tokens,
 * GEMVs reading each weight record once per 4 tokens; logits of the last token. */
int32_t k2t_model_prefill(k2t_model *m, const int32_t *tokens, int32_t n, float *logits_host);
/* generate_greedy's decode loop (real_llm.rs:7895-7907): feeds first_token, then
 * n_steps decode steps whose next token is the argmax of the logits, chosen on the
 * device.  tokens_out (nullable) receives the n_steps argmax tokens. */
int32_t k2t_model_generate(k2t_model *m, int32_t first_token, int32_t n_steps, int32_t *tokens_out);
/* Device pointer of the last logits (valid after a step; read after k2t_model_sync). */
int32_t k2t_model_logits(k2t_model *m, const float **d_logits);
int32_t k2t_model_sync(k2t_model *m);

/* ---- KV cache and attention ops ------------------------------------------- */

/* Hadamard KV store of n post-RoPE heads [n][head_dim] into slots 0..n-1:
 * bits 8: int8 d_q [n][hd] and f32 d_scales [n] (store_hadamard_q8_head*,
 * real_llm.rs:8282-8365); bits 4: NF4 nibbles d_q [n][hd/2] and BF16 d_scales [n][hd/64]
 * (store_hadamard_q4_head_raw, real_llm.rs:8646-8700).  The engine's own store is the same code. */
int32_t k2t_kv_store(k2t_ctx *ctx, int32_t bits, const float *d_heads, int32_t n, int32_t head_dim, void *d_q,
                     void *d_scales);
/* Decode attention of one token (causal_gqa_attention_q8, real_llm.rs:8938-8988, and the
 * window / NF4 path causal_gqa_group_q4_or_window, 8794-8937): queries d_q [n_heads][hd]
 * (post-RoPE), a KV cache of n_kv_heads x cap slots in k2t_kv_store's layout, `seq`
 * positions (window > 0: a sink + ring cache of cap slots, ring = cap - sinks, as
 * k2t_model_set_kv_window lays it out); d_out [n_heads][hd] receives the attention output
 * after ifwht64.  Synchronizes the context's stream. */
int32_t k2t_attn_decode(k2t_ctx *ctx, int32_t bits, const float *d_q, int32_t n_heads, int32_t n_kv_heads,
                        int32_t head_dim, const void *d_kq, const void *d_ks, const void *d_vq, const void *d_vs,
                        int32_t cap, int32_t seq, int32_t window, int32_t sink_tokens, float attn_scale,
                        float *d_out);
/* k2t_attn_decode without any allocation.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  Same arguments and results as k2t_attn_decode
 * (the same kernels), but the span partials and the position word live in a fixed 4 MiB
 * device array inside the library (one per GPU, kept until the process ends): calls with
 * n_heads * ceil(min(seq, window or seq) / 256) * (head_dim + 2) > 1048512 floats (for
 * contexts above 1024 positions; at most 1024 positions use a single span) return
 * K2T_E_ARG.  Asynchronous on the context's stream (the caller synchronizes).  Every call
 * on one GPU shares that array: calls that overlap on one GPU (other streams, other
 * contexts, other host threads) race. */
int32_t k2t_attn_decode_noalloc(k2t_ctx *ctx, int32_t bits, const float *d_q, int32_t n_heads, int32_t n_kv_heads,
                                int32_t head_dim, const void *d_kq, const void *d_ks, const void *d_vq,
                                const void *d_vs, int32_t cap, int32_t seq, int32_t window, int32_t sink_tokens,
                                float attn_scale, float *d_out);

/* ---- sparse-MoE experts (.k2tm shards) ------------------------------------- */

/* K2tmShardHeader (moe_800b.rs:792-854): page 0 of a .k2tm shard ("K2TM800B_V1\0", then
 * seven u64 words at byte 16).  Records follow at 16384 + (layer*E + e)*aligned bytes. */
typedef struct k2t_k2tm_header {
    int64_t num_layers, experts_per_layer, d_model, d_ff_expert, scale_group_chunks, aligned_expert_bytes, bits;
} k2t_k2tm_header;
/* nf_expert_byte_layout (moe_800b.rs:1332-1375): offsets inside one expert record. */
typedef struct k2t_k2tm_layout {
    int64_t gu_codebook_off, dn_codebook_off, gu_pair_off, gu_pair_bytes, dn_pair_off, dn_pair_bytes,
        aligned_expert_bytes;
} k2t_k2tm_layout;

/* Router scoring (MoeRouterScoring, sparse_moe.rs:86-182). */
#define K2T_MOE_SOFTMAX 0      /* softmax over all experts, top-k, optional renormalization */
#define K2T_MOE_TOPK_SOFTMAX 1 /* top-k logits, softmax over them (gpt-oss) */
#define K2T_MOE_SIGMOID 2      /* sigmoid scores, top-k, optional renormalization */
#define K2T_MOE_MAX_TOPK 16

/* Decodes and validates a header page (len >= 16384); experts must be NF3 or NF4 and
 * aligned_expert_bytes must equal the layout of the declared shape. */
int32_t k2t_k2tm_read_header(const uint8_t *page, size_t len, k2t_k2tm_header *out);
int32_t k2t_k2tm_expert_layout(int64_t d_model, int64_t d_ff, int32_t bits, int32_t sgc, k2t_k2tm_layout *out);
/* A whole shard (header page + every record) copied into HBM (MoeExpertBackend::ZeroCopyMmap,
 * sparse_moe.rs:1025-1045, with HBM in place of the mapping: no paging).  NF3 experts are
 * stored in lane order (k2t_experts_nf3_lane_order). */
int32_t k2t_experts_upload(k2t_ctx *ctx, const uint8_t *k2tm, size_t len, k2t_experts **out);
/* A shard already in device memory (borrowed; 256-byte aligned), described by its host
 * header page.  The bytes stay in the .k2tm layout until k2t_experts_nf3_lane_order (a
 * shard it converted earlier is recognised by its mark and read in lane order). */
int32_t k2t_experts_wrap(k2t_ctx *ctx, const uint8_t *d_k2tm, size_t len, const uint8_t *header_page,
                         k2t_experts **out);
/* No counterpart in the reference: a device-layout step.  Rearranges every NF3 expert
 * matrix of the bank IN PLACE (the borrowed bytes of a wrapped bank included) so that each
 * 384-byte stripe-chunk (8 triplet blocks of 48 bytes, simd_lut.rs:4932-4960) holds 16-byte
 * piece k of block (g, half) at 128*k + 16*(2g + half) instead of 192*half + 48*g + 16*k:
 * the grouped GEMV then reads one 128-byte run per lane group and load.  Results are
 * unchanged.  No-op for NF4 banks and for banks already converted; synchronous.  The bytes
 * are no longer in the .k2tm layout afterwards; the conversion writes a 16-byte mark into
 * the last 16 bytes of the device header page (zero padding in the format), so a later
 * k2t_experts_wrap of the same bytes reads them in lane order and converting again is a
 * no-op.  A handle reads the mark when it wraps the bytes: every other handle that already
 * wraps the same bytes keeps the reference order and gives wrong MoE outputs afterwards,
 * so destroy such handles before converting (and wrap again). */
int32_t k2t_experts_nf3_lane_order(k2t_experts *bank);
void k2t_experts_destroy(k2t_experts *b);
int32_t k2t_experts_info(const k2t_experts *b, k2t_k2tm_header *out);
/* One token through one MoE layer (forward_layer_single, sparse_moe.rs:961-1084, plus the
 * residual add of real_llm.rs:6711-6714):
 *   x_norm = RMSNorm(hidden) * post_norm; routes = route_sorted(router, x_norm);
 *   hidden += sum over routes of w * down(SwiGLU(gate_up(x_norm)))
 * router_w: device f32 [E][d_model] (bias [E] or NULL).  route ids / weights (device,
 * top_k each, nullable) receive the routing.  Uses the context's scratch.  With the
 * context in exact mode (k2t_ctx_set_exact) every step follows the x86 reference's order
 * (sequential router dot, glibc-identical expf, in-order GEMV epilogues). */
int32_t k2t_moe_ffn(k2t_ctx *ctx, const k2t_experts *bank, int32_t shard_layer, const float *d_router_w,
                    const float *d_router_bias, int32_t top_k, int32_t norm_topk_prob, int32_t scoring,
                    float *d_hidden, const float *d_post_norm, float eps, int32_t *d_route_ids,
                    float *d_route_weights);

/* ---- .k2tb compiled models ------------------------------------------------ */

/* A memory-mapped .k2tb file: the cache of RealLlamaEngine::save_bipolar
 * (real_llm.rs:3705-3895), versions 1-4 and 6, as read by load_bipolar
 * (real_llm.rs:3902-4190).  Every read is bounds-checked: a truncated or corrupt file
 * returns K2T_E_ARG; matrices this path cannot run (VQ2, Q2C, NF2/NF5, 2-3 bit planes)
 * and K2TKRONOS5 MoE cores return K2T_E_STATE. */
typedef struct k2t_k2tb k2t_k2tb;
typedef struct k2t_k2tb_matrix_info {
    int32_t tag;            /* cache tag: 0 FusedBipolar, 2 NfSdot */
    int32_t fmt;            /* stream format after repack: 1 Nibble4 (bit planes), 2 NF */
    int32_t rows, cols;
    int32_t planes_or_bits; /* bit planes (4..6) or NF bits (3, 4) */
    int32_t sgc;            /* NF scale-group chunks */
    int8_t codebook[16];    /* NF codebook */
    size_t pair_len, tail_len; /* repacked stream sizes */
} k2t_k2tb_matrix_info;

int32_t k2t_k2tb_open(const char *path, k2t_k2tb **out);
void k2t_k2tb_close(k2t_k2tb *f);
/* Version (1..6), layer count, the six mode words (RealWeightMode, real_llm.rs:3790-3848). */
int32_t k2t_k2tb_header(const k2t_k2tb *f, int32_t *version, int32_t *n_layers, uint64_t *mode_words6);
/* One matrix in the layout the GEMV streams (repack_sdot, real_llm.rs:3657-3702):
 * bit-plane bodies become Nibble4SdotMatrix records (from_bipolar_with_perm,
 * simd_lut.rs:3297-3400), NF streams are copied; interleave_gate_up = 1 reorders rows
 * into [gate64(ic), up64(ic)] blocks (simd_lut.rs:5500-5523 for NF).
 * layer >= 0: which 0 qkv, 1 o, 2 gate_up, 3 down; layer = -1: which 4 lm_head,
 * 5 NF4 embedding.  pair = tail = NULL fills `info` only (size query). */
int32_t k2t_k2tb_matrix(const k2t_k2tb *f, int32_t layer, int32_t which, int32_t interleave_gate_up,
                        k2t_k2tb_matrix_info *info, uint8_t *pair, size_t pair_cap, uint8_t *tail,
                        size_t tail_cap);
/* Vectors: layer >= 0: which 0 input_norm, 1 post_attn_norm, 2 qkv_bias, 3 q_norm,
 * 4 k_norm (f32); layer = -1: 0 final_norm, 1 f32 embedding rows (f32), 2 bf16
 * embedding rows (uint16).  *count = elements (0 when absent); out = NULL queries. */
int32_t k2t_k2tb_vector(const k2t_k2tb *f, int32_t layer, int32_t which, size_t *count, void *out, size_t cap);
/* load_bipolar + repack_sdot (real_llm.rs:3902-4190, 3657-3702) onto the context's
 * device: creates the model for `cfg` (LlamaConfig from config.json, whose layer count
 * must match the file), uploads every matrix (owned by the model) and sets the layers,
 * head and embedding. */
int32_t k2t_model_load_k2tb(k2t_ctx *ctx, const k2t_model_config *cfg, const char *path, int32_t max_batch,
                            k2t_model **out);

#ifdef __cplusplus
}
#endif

#endif /* K2T_HIP_H */
