// Host/device interface of the persistent single-launch decode kernel (k2t_decode_mk.hip).
#pragma once
#include "../../include/k2t_hip.h"
#include "k2t_gemv_core.h"
#include "k2t_internal.h"

namespace k2t {

// Most positions one decode step of the persistent kernel attends.  Its attention phase
// gives each q head one workgroup that scans the whole context, so past this many
// positions the per-operation path (256-position spans over many workgroups) runs
// instead; the kernel's LDS score buffer is sized for this bound, not for max_seq.
// 1024 is a rounded crossover: a 1.7B nf4g128 context sweep measured the two paths
// level at 1029-1093 positions (972 against 964 tok/s) and the persistent kernel
// behind beyond (724 against 944 tok/s at 2053-2117, 391 against 880 at 4101-4165).
constexpr int kMkMaxContext = 1024;
// Copies of the broadcast hand-off vectors: one per pair of MI355X's 8 XCDs (a workgroup
// reads copy blockIdx.x mod 4).  8 copies (one per XCD) measured 1440 against 1447 tok/s
// on the 1.7B nf4g128 decode, 1545 against 1555 on the 135M p55454 one (the writers'
// epilogues store half as many words); 2 copies 1432 / 1547.
constexpr int kMkRep = 4;
// Most spans the attention phase cuts one q head's context into, and the fewest
// positions per span.
constexpr int kMkSpans = 4;
// ... and in the 512-thread kernels (the 1.7B nf4g128 decode at context 261-389: 2 spans
// 1203 tok/s, 3 spans 1144-1159).
constexpr int kMkSpans512 = 2;
// Most spans per q head of the kernel with NTH threads per workgroup.
__host__ __device__ constexpr int mk_max_spans(int nth) { return nth == 512 ? kMkSpans512 : kMkSpans; }
constexpr int kMkSpanMin = 128;
// Rows of one GEMV round of a workgroup (wave groups x rows per group), the most the
// exact-order variant stages epilogue operands for.
constexpr int kMkTermRows = 128;

struct MkLayer {
    MatDev qkv, o, gu, down;
    const float *in_norm, *post_norm, *bias;
    // First workgroup of each phase's task list (qkv, attention, o, gate_up, down): the
    // lists are laid end to end over the grid, so consecutive phases use disjoint
    // workgroups wherever their task counts allow.
    int off[5];
};

struct MkParams {
    const MkLayer *layers;
    int L;
    MatDev head;
    int head_off;        // first workgroup of the lm_head phase
    MatDev embed;        // NF4 / bit-plane embedding table (ekind 0 tied, 3 NF4)
    const void *erows;   // f32 (ekind 1) or bf16 (ekind 2) embedding rows
    int ekind;
    const float *final_norm;
    int d, nq, nkv, hd, inter, vocab, max_seq, kmax;
    float eps, attn_scale;
    const float *rope;
    int *pos_dev;      // advanced by the kernel's last step (with step_dev)
    int *tokens;       // input token; the kernel's last step writes the greedy next token
    uint32_t *step_dev;
    int8_t *kq, *vq;
    float *ks, *vs;
    // hand-off vectors as {payload, epoch} words.  HA, HB, OACT and GACT, which every
    // workgroup of the next phase reads, exist in `rep` copies ([rep][n] words); writers
    // store every copy and a reader polls the copy of its XCD, so each line is polled by
    // one XCD's workgroups instead of the whole grid.
    unsigned long long *HA, *HB, *QKV, *OACT, *GACT;
    int rep;
    // attention spans per q head (1 .. kMkSpans); APART holds the spans 1 .. nsp-1 of each
    // head as {max, sum, o[hd]} words, [nq][nsp][2 + hd]
    int nsp;
    unsigned long long *APART;
    unsigned long long *BEST;  // [2 * grid] per-workgroup lm_head maximum {value, row} words
    float *logits;
    const uint64_t *signs;  // Hadamard sign masks of 64-blocks (bit i = element i)
    int *err;
    uint32_t spin_limit;
    // Exact-order variant only: per workgroup, the GEMV epilogue operands of one round
    // ({term, scale} words, [row of the round][chunk]; kMkTermRows * kmax/64 words each).
    unsigned long long *exterm;
    // Measurement builds only (compiled with -DK2T_MK_TRACE): per workgroup, layer and
    // phase the wall clock at the task's start, input arrival and end.
    unsigned long long *trace;
};

// pair_mode_nseg4: gate_up layout (4 wave groups = one [gate64, up64] block of 4 pairs).
// max_nseg (> 0) caps the K segments per row block in stripe mode (more rows per
// workgroup, fewer workgroups for the phase).
// nwaves: waves per workgroup of the kernel that will run (decode_mk_threads / 64).
// min_nseg (> 0) asks for at least that many K segments (fewer rows per workgroup, more
// workgroups for the phase).
MatDev mat_dev(const k2t_mat *m, bool pair_mode_nseg4, int max_nseg = 0, int nwaves = 8, int min_nseg = 0);
// Workgroup tasks of a GEMV phase of the persistent kernel.
int mk_phase_tasks(const MatDev &M, int nwaves = 8);
// Threads per workgroup of the persistent kernel for the format decode_mk_format chose.
int decode_mk_threads(int hp);
size_t decode_mk_lds_bytes(const k2t_model_config &c);
bool decode_mk_supported(const k2t_model_config &c, int num_cus);
// Accumulates the common weight format of the model's matrices (fmt < 0: first call);
// false when a matrix differs (the persistent kernel needs one format family).  Bit-plane
// models with any 5-plane matrix get hp = kHpMixed: the 256-thread kernel that reads
// each matrix's plane count (4 or 5).
bool decode_mk_format(const MatDev &m, int &fmt, int &hp);
// exact: the exact-order variant (x86 reference operation order; P.exterm set, P.nsp 1).
void launch_decode_mk(hipStream_t st, const MkParams &P, int fmt, int hp, int num_cus, size_t lds, bool exact);

}  // namespace k2t
