// Internal launch helpers shared by the kernel-level C ABI (ops.c) and the
// decode engine (engine.c). These do not arm an entry point: failures
// longjmp to whichever exported call is running.
#pragma once
#include "hipx.h"
#include "ssf.h"
#include "sml-hip.h"

struct sml_hip_mat {
    sml_kmat k;          // device pointers; k.rows is the row count
    sml_kmat * kdev;     // the same descriptor in device memory, then room for a (gate, up) pair (small-M GEMM tables)
    sml_kmat up_k;       // the up descriptor kdev[1..2] was last written for
    int pair_set;
    int nbits, cols;
    void * mem;          // the single allocation holding planes and fields
    void * tiled_mem;    // Q4: the MFMA GEMM's tiled copy (k.tiled), or NULL
    size_t bytes;        // planes + fields bytes (what one GEMV streams)
    int placed;          // mem lies in a region the caller owns (mat_place): not freed here
};


sml_hip_mat * mat_upload(const uint8_t * const planes[4], const uint16_t * sd, const uint8_t * sq,
                         const uint16_t * md, const uint8_t * mq, int rows, int cols, int nbits,
                         int scale6, int minneg);
sml_hip_mat * mat_from_record(const ssf_file * f, const ssf_record * r);
void mat_free(sml_hip_mat * m);
// The bytes of one matrix's allocation (planes, fields, descriptors).
size_t mat_block_bytes(int rows, int cols, int nbits);
// Uploads after mat_place(base, cap) take consecutive bytes of that device
// region instead of allocations of their own (base NULL: allocate again);
// mat_place_used() is how far they reached.
void mat_place(void * base, size_t cap);
size_t mat_place_used(void);

// Exact mode (the reference's float order in GEMVs, norms, attention, router)
void ops_set_exact(int on);
int ops_exact(void);

void op_normq(hipStream_t st, float * x, const float * resid, const float * w, float eps, int n,
              int nout, const int32_t * const * perm, int8_t * const * q, float * const * scale,
              int32_t * const * sums, float * normed, int per256);
// Optional fusions of a GEMV launch: x != NULL computes the activation in the
// kernel's prologue (RMSNorm with norm_w if not NULL, gather through perm if
// not NULL, per-32 quantization) instead of reading q/scale/sums; hq != NULL
// (SwiGLU only, rows a multiple of 32) also quantizes h per 32 into
// hq/hscale/hsums.
typedef struct {
    const float * x;
    const float * norm_w;
    const int32_t * perm;
    float eps;
    int8_t * hq;
    float * hscale;
    int32_t * hsums;
    int2 * amax;                  // one-matrix GEMVs: each row block's (max, lowest index) pair
} gemv_fuse;
// Widest input the fused prologue takes (hq: the 1024-thread SwiGLU kernels).
int gemv_fuse_max_cols(int hq);
// y = W.x (+ bias, + resid for SML_EPI_RESIDUAL) for one matrix m; SwiGLU
// (up != NULL): y = silu(gate.x + bias) * (up.x + up_bias). Returns the
// number of row blocks of the plain GEMV forms (fu->amax's pair count), 0
// for the others.
int op_gemv(hipStream_t st, const sml_hip_mat * m, const sml_hip_mat * up, int epi, const int8_t * q,
            const float * scale, const int32_t * sums, float * y, const float * bias, const float * up_bias,
            const float * resid, const gemv_fuse * fu);
// Small-M GEMM over ngroups matrix groups (device table tab: one matrix per
// group, or gate/up pairs for SwiGLU; hk: the host copies of a single group's
// descriptors, or NULL); m_all rows (count == NULL) or count[e]
// rows per group, at most mt (1, 4, 8 or 16). The activation regime:
enum {
    GEMM_PER32 = 0,     // per-32 activations; Q4 above 8 rows on MFMA (fp32 order differs from the GEMV's)
    GEMM_PER256 = 1,    // per-256 activations; Q4 on MFMA with the integer superblock epilogue
    GEMM_EXACT = 2,     // per-32 activations, every row the GEMV's arithmetic bit for bit
    GEMM_REF = 3,       // exact mode: per-32 activations, every row the exact (reference-order) GEMV's bit for bit
};
void op_gemm(hipStream_t st, const sml_kmat * tab, const sml_kmat * hk, int ngroups, int swiglu, int nbits, int rows, int cols,
             const int32_t * count, int m_all, int mt, int mmax, const int8_t * q, const float * scale,
             const int32_t * sums, float * y, const float * bias, const float * resid, int regime);
int gemm_mt(int m);
// One matrix holding the rows of several FLAT records of one width and input
// width, stacked in order (the q, k and v projections as one GEMV).
sml_hip_mat * mat_stack(const ssf_file * f, const ssf_record * const * recs, int n);
void op_embed(hipStream_t st, const sml_hip_mat * m, const int32_t * tok, const int32_t * pos,
              const int32_t * perm, float * x);
// rows embeddings: row b of x [rows][cols] from token tok[b] (pos NULL)
void op_embed_rows(hipStream_t st, const sml_hip_mat * m, const int32_t * tok, const int32_t * pos, int rows,
                   const int32_t * perm, float * x);
// op_normq over rows vectors: every pointer advances by n (scale, sums by n/32) per row
// While deferral is on, a split-K product leaves its slice sums pending;
// op_ksum_normq_rows adds them (into x, which must be the product's output)
// while it normalizes and quantizes the rows, op_ksum_flush adds them alone.
void ops_defer_ksum(int on);
void ops_ksum_reset(void);      // off, and anything pending dropped (a failed call's leftovers)
int ops_ksum_pending(void);
void op_ksum_flush(hipStream_t st);
void op_ksum_normq_rows(hipStream_t st, float * x, const float * w, float eps, int n, int rows, int nout,
                        const int32_t * const * perm, int8_t * const * q, float * const * scale,
                        int32_t * const * sums, int per256);
void op_normq_rows(hipStream_t st, float * x, const float * resid, const float * w, float eps, int n, int rows,
                   int nout, const int32_t * const * perm, int8_t * const * q, float * const * scale,
                   int32_t * const * sums, float * normed, int per256);
// Decode attention for one sequence. cnt: n_kv zeroed counters (the merge then
// runs in the attention launch itself, see sml_kattn.cnt), or NULL for a
// separate merge launch. n_pos (<= n_ctx) bounds the positions the launch
// may attend: the split size follows n_ctx, and only the splits below n_pos
// are launched (the results equal launching all of them).
void op_attention(hipStream_t st, const float * q, const float * k, const float * v, uint16_t * kc, uint16_t * vc,
                  const float * cos_t, const float * sin_t, const int32_t * pos, int n_head, int n_kv,
                  int hd, int n_ctx, int n_pos, float * part, float * out, int8_t * q_out, float * s_out,
                  int32_t * u_out, int * cnt);
// Attention for nseq sequences in one launch: sequence b's q, k, v at
// qkv + b * qkv_stride (q, then k, then v), its cache kc_slots[slot[b]] +
// layer_off, its position pos[b]; part, out and the quantized out hold one
// sequence's worth per b. causal: entries may be positions of one sequence
// (prompt reading), so every k and v is rotated and written by one launch
// before any entry attends; 1 keeps the decode kernel's arithmetic per entry
// (bit-exact with stepping), 2 runs the wave-per-position kernel (faster,
// its own fp32 order). The quantized out is per 32 values, or per 256 when
// q256 (decode steps, causal 0, of an even head count only). n_pos bounds
// every entry's position as in op_attention (the flash prompt form splits
// the whole n_ctx range).
// Exact mode's batched prompt rows (head_dim 128): every row's K/V written,
// then each row's reference-order attention over positions 0..pos[b];
// sc holds nrows * n_head * n_ctx floats of scores.
void op_attention_rows_exact(hipStream_t st, const float * qkv, int qkv_stride, uint16_t * kc, uint16_t * vc,
                             const float * cos_t, const float * sin_t, const int32_t * pos, int nrows, int n_head,
                             int n_kv, int n_ctx, int n_pos, float * sc, float * out, int8_t * q_out, float * s_out,
                             int32_t * u_out);
void op_attention_batch(hipStream_t st, const float * qkv, int qkv_stride, uint16_t * const * kc_slots,
                        uint16_t * const * vc_slots, const int32_t * slot, size_t layer_off, const float * cos_t,
                        const float * sin_t, const int32_t * pos, int nseq, int n_head, int n_kv, int hd, int n_ctx,
                        int n_pos, float * part, float * out, int8_t * q_out, float * s_out, int32_t * u_out,
                        int causal, int exact, int q256);
// Whether op_gemm computes every row with the GEMV's arithmetic in this regime
// for m_all rows (the exact regime, or per-32 rows the VALU kernel takes).
int gemm_exact(int regime, int m_all);
// Greedy pick over n logits (the first maximum; NaN never wins). part:
// scratch of ARGMAX_MAX_PARTS pairs for the two-stage pick of n >=
// ARGMAX_TWO_STAGE_MIN, or NULL for one workgroup.
#define ARGMAX_TWO_STAGE_MIN 8192
#define ARGMAX_MAX_PARTS 1024
void op_argmax(hipStream_t st, const float * logits, int n, int32_t * tok, int32_t * pos, int32_t * hist,
               int hist_n, int2 * part);
// The greedy pick's second stage over nparts (max, lowest index) pairs (a
// GEMV's amax row blocks); logits[0] keeps the reference's NaN rule.
void op_argmax_pairs(hipStream_t st, const int2 * pairs, int nparts, const float * logits, int32_t * tok,
                     int32_t * pos, int32_t * hist, int hist_n);
void op_advance(hipStream_t st, int32_t * pos);
void op_silu_mul(hipStream_t st, float * g, const float * u, int n);

// One MoE FFN layer: router, experts and (shared between layers) scratch.
struct sml_hip_moe {
    int nexp, k, n_embd, n_ff, tmax, nbits;
    unsigned flags;
    float * router, * router_b;
    sml_hip_mat ** mats;          // [nexp][3]: gate, up, down
    sml_kmat * tab_gu, * tab_d;   // device tables
    const int32_t ** ptab_gu, ** ptab_d;   // device tables of device permutations, or NULL (identity)
    void * work;                  // scratch: logits, route, lists, activations, h, expert outputs
    float * logits, * w, * h, * yd;
    int32_t * sel, * slot, * count, * list;
    int8_t * qx, * qh;
    float * sx, * sh;
    int32_t * ux, * uh;
    void * owned[192];            // every device allocation: up to 2 permutations per expert + buffers
    int nowned;
    size_t expert_bytes;
    int per256;                   // activations quantized per 256 values (the batched regime)
    // routing modes (sml_kmoe_route): correction bias, weight scale, groups
    float * exp_bias;
    float scale;
    int groups, topk_group;
    // the shared expert (shx[0] NULL: none): gate, up, down; its gate vector
    // (NULL: weight 1), permutations and scratch
    sml_hip_mat * shx[3];
    sml_kmat * sh_gu;             // device table: gate, up
    const int32_t * sh_perm_gu, * sh_perm_d;
    float * shgate;
    int sh_ff;
    float * sg, * sh_h, * sh_y;   // [tmax], [tmax][sh_ff], [tmax][n_embd]
    int8_t * sh_q;                // [tmax][max(n_embd, sh_ff)]
    float * sh_s;
    int32_t * sh_u;
};
// Experts of layer `layer` for up to tmax tokens per call; scratch shared with
// `share` (a loaded layer of the same shape) when not NULL.
sml_hip_moe * moe_load(const ssf_file * f, int layer, int tmax, const sml_hip_moe * share);
void moe_free(sml_hip_moe * m);
// out[t] = (resid[t] +) sum over the chosen experts of w * FFN_e(x[t]).
void op_moe(hipStream_t st, sml_hip_moe * m, const float * x, int T, float * out, const float * resid);
