// Kernel-level C ABI of the MI355X (gfx950) decode path.
//
// Plain pointers and sizes only. Device pointers come from sml_hip_malloc (or
// any HIP allocation in the same process). Every call returns 0 on success and
// -1 on failure (sml_hip_last_error() says why), or NULL for constructors;
// nothing ends the process. Each entry point names the reference CPU/GPU
// interface it replaces; the GPU forward pass itself is in sml-gpu.h.
#pragma once
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

// ------------------------------------------------------------ device plumbing
// replaces the driver binding of sml/sml-gpu-drv.h:13-216 (cu_open, MemAlloc,
// MemcpyHtoD/DtoH, cu_check)
int          sml_hip_init(int device, char * why, int nwhy);
const char * sml_hip_last_error(void);
void *       sml_hip_malloc(size_t n);
int          sml_hip_free(void * p);
int          sml_hip_h2d(void * dst, const void * src, size_t n);
int          sml_hip_d2h(void * dst, const void * src, size_t n);
int          sml_hip_memset(void * p, int value, size_t n);
int          sml_hip_sync(void);
// Test hook: make the n-th HIP call from now fail (n < 0 disables). Every
// call the library makes counts, in sml_gpu_* entry points too; the entry
// point that meets the failure returns its failure value.
void         sml_hip_fail_after(long n);
// HIP calls the library has made so far (to place sml_hip_fail_after).
long         sml_hip_call_count(void);
// Exact mode on (1) or off (0) for the launches below: Q4/Q8 GEMVs, norms,
// attention and the MoE router then follow the float order of the reference's
// x86 build (sml/sml-kernel.c:572-727,836-866; sml/sml-run.c:147-152,180-287,
// 339-372,393-426,3075-3080), so their outputs equal its CPU path bit for bit.
// No counterpart in the reference's GPU ABI, whose kernels it grades against
// the CPU with a tolerance (sml/sml-gpu-fwd.c:2565-2601).
void         sml_hip_set_exact(int on);

// ------------------------------------------------------------ matrices
// A quantized FLAT matrix resident in HBM (the file's planes and fields;
// 6-bit group fields are widened to bytes with the min bias moved to 127).
// replaces the reference's per-tensor upload up_tensor (sml/sml-gpu-fwd.c:99-160)
typedef struct sml_hip_mat sml_hip_mat;
sml_hip_mat * sml_hip_mat_upload(const uint8_t * const planes[4], const uint16_t * sd, const uint8_t * sq,
                                 const uint16_t * md, const uint8_t * mq,
                                 int rows, int cols, int nbits, int scale6, int minneg);
// The same, for record `name` of an SSF file.
sml_hip_mat * sml_hip_mat_from_file(const char * path, const char * name);
// A matrix given as GGUF Q4_K blocks (ggml's block_q4_K: per 256 weights of a
// row fp16 d, fp16 dmin, 12 bytes of 6-bit sub-block scales and mins, 128
// bytes of 4-bit codes; rows x cols/256 blocks of 144 bytes, row-major),
// repacked on the host into the FLAT Q4 layout: sd = d, md = dmin, sq = the
// sub-block scale, mq = 127 - the sub-block min, code bytes as they are. The
// arithmetic is ggml's weight d*sc*q - dmin*m exactly, so every GEMV and GEMM
// above runs it. No counterpart in the reference, which reads GGUF only
// through transformers into fp16 and re-quantizes (tooling/sml_gguf.py:1-35).
sml_hip_mat * sml_hip_mat_from_q4k(const void * blocks, int rows, int cols);
// The host repack alone (no GPU): FLAT Q4 plane [rows][cols/2], sd and md
// [rows][cols/256], sq and mq [rows][cols/32]. Returns 0, or -1 on a shape
// that is not whole blocks.
int           sml_hip_q4k_repack(const void * blocks, int rows, int cols, uint8_t * plane, uint16_t * sd,
                                 uint8_t * sq, uint16_t * md, uint8_t * mq);
// A matrix given as GGUF Q5_K blocks (ggml's block_q5_K: 176 bytes per 256
// weights, rows of cols/256 blocks), repacked on the host into a FLAT Q5
// record: Q4_K's fields, the low nibbles as the 4-bit plane and the fifth
// bits as the 1-bit plane. The arithmetic is ggml's weight
// d*sc*(q + 16*h) - dmin*m exactly. No counterpart in the reference (GGUF
// goes through transformers there, tooling/sml_gguf.py:1-35).
sml_hip_mat * sml_hip_mat_from_q5k(const void * blocks, int rows, int cols);
// The host repack alone (no GPU): 4-bit plane [rows][cols/2], 1-bit plane
// [rows][cols/8], sd and md [rows][cols/256], sq and mq [rows][cols/32].
// Returns 0, or -1 on a shape that is not whole blocks.
int           sml_hip_q5k_repack(const void * blocks, int rows, int cols, uint8_t * plane4, uint8_t * plane1,
                                 uint16_t * sd, uint8_t * sq, uint16_t * md, uint8_t * mq);
void          sml_hip_mat_free(sml_hip_mat * m);
int           sml_hip_mat_info(const sml_hip_mat * m, int * rows, int * cols, int * nbits);
// Bytes the matrix occupies in HBM (codes + fields): what one GEMV streams.
size_t        sml_hip_mat_bytes(const sml_hip_mat * m);

// ------------------------------------------------------------ activations
// RMSNorm (w != NULL) of x after x += resid (resid != NULL), gathered through
// perm (NULL = identity), quantized per 32 (per256 = 0) or per 256 values.
// replaces sml_quantize_act / sml_quantize_act_sb (sml/sml-kernel.h:136,318),
// sml_gather (:151) and rms_norm (sml/sml-run.c:147-152), as one kernel like
// the reference GPU's sml_g_normq2 (sml/sml-gpu-fast.cu:64-111)
int sml_hip_normq(float * x, const float * resid, const float * w, float eps, int n,
                  const int32_t * perm, int8_t * q, float * scale, int32_t * sums, int per256);

// ------------------------------------------------------------ GEMV
// y = W.x for the quantized activation (q, scale, sums) of x, any FLAT width.
// replaces sml_matvec_rows_flat4 / _flat6 / _flat8 / sml_matvec_rows +
// sml_matvec_bits1 (sml/sml-kernel.h:239,246,212,190,206) as dispatched by
// issue_rows_act (sml/sml-run.c:612-680); y is written, not accumulated.
int sml_hip_matvec(const sml_hip_mat * m, const int8_t * q, const float * scale, const int32_t * sums,
                   float * y);
// h = silu(gate.x) * (up.x), the fused gate/up of sml_g_ffns (sml/sml-gpu-fast.cu:319-354)
int sml_hip_matvec_swiglu(const sml_hip_mat * gate, const sml_hip_mat * up, const int8_t * q,
                          const float * scale, const int32_t * sums, float * h);
// y = W.a where a is the per-32 quantization of RMSNorm(x) (w != NULL; w NULL:
// x itself) gathered through perm (NULL = identity), computed inside the GEMV's
// prologue by every workgroup instead of by a separate launch; cols <= 4096.
// The activation equals sml_hip_normq's bit for bit, so y equals
// sml_hip_normq + sml_hip_matvec. replaces sml_g_normq2 + sml_g_qdmv2
// (sml/sml-gpu-fast.cu:64-111,267-288), on the CPU rms_norm + sml_gather +
// sml_quantize_act + the matvec (sml/sml-run.c:147-152,612-680)
int sml_hip_matvec_normq(const sml_hip_mat * m, const float * x, const float * w, float eps, const int32_t * perm,
                         float * y);
// sml_hip_matvec_swiglu with its two fusions: x != NULL computes the activation
// in the prologue as sml_hip_matvec_normq does (cols <= 4096; q/scale/sums
// unused), otherwise q/scale/sums are read; hq != NULL
// also writes the per-32 quantization of h in order (rows a multiple of 32)
// into hq/hscale/hsums, equal to sml_hip_normq of h without norm.
// replaces sml_g_ffns + sml_g_quantw2 (sml/sml-gpu-fast.cu:319-354,522-543)
int sml_hip_matvec_swiglu_fused(const sml_hip_mat * gate, const sml_hip_mat * up, const float * x, const float * w,
                                float eps, const int32_t * perm, const int8_t * q, const float * scale,
                                const int32_t * sums, float * h, int8_t * hq, float * hscale, int32_t * hsums);
// Time `iters` back-to-back launches of sml_hip_matvec, rotating over `ncopy`
// matrices of one shape (so repeats are not served from cache), with HIP
// events on the launch stream. ms_total receives the elapsed milliseconds.
int sml_hip_time_matvec(const sml_hip_mat * const * mats, int ncopy, const int8_t * q, const float * scale,
                        const int32_t * sums, float * y, int iters, float * ms_total);
// The same launches of a Q4 GEMV in its 2-rows-by-4-chunks shape (the roofline
// workload's), instrumented: for the last launch, per row block, the GPU's
// 100 MHz real-time clock at entry, at the first weight word's arrival, when
// the first pass's and the last pass's weights have all arrived, and at exit
// (5 values a block into ts, host memory, at most max_blocks blocks). Returns
// the block count, or -1. A measurement tool (no counterpart in the
// reference); its waits for the timestamps serialize the loads slightly.
int sml_hip_gemv_timeline(const sml_hip_mat * const * mats, int ncopy, const int8_t * q, const float * scale,
                          const int32_t * sums, float * y, int iters, unsigned long long * ts, int max_blocks);

// Calibration: time `iters` launches of a plain streaming read of `bytes`
// from each buffer in turn (grid workgroups of 256 threads, 128-bit loads).
// No counterpart in the reference: it measures what one kernel can read from
// HBM on this machine, the denominator next to the GEMV's achieved bandwidth.
int sml_hip_time_read(const void * const * bufs, int nbuf, size_t bytes, int grid, int iters, float * ms_total);
// Calibration: copy `bytes` (a multiple of 16) with one plain 128-bit
// streaming kernel and wait for it. No counterpart in the reference: its HBM
// read and write counters give the scale for the GEMV's counter readings.
int sml_hip_copy(void * dst, const void * src, size_t bytes);

// ------------------------------------------------------------ small-M GEMM
// y[r] = W.a[r] for nrow (1..65536) activation rows a[r] (q [nrow][cols],
// scale and sums [nrow][cols/32]) into y [nrow][rows]: each weight streams
// once for up to 16 rows (more rows run in slices of 16). replaces
// sml_matvec_batch_flat4 / batch_group for the exact per-32 regime
// (sml/sml-kernel.c:1008-1021, sml/sml-run.c:2058-2183)
int sml_hip_gemm(const sml_hip_mat * m, const int8_t * q, const float * scale, const int32_t * sums, int nrow,
                 float * y);
// h[r] = silu(gate.a[r]) * (up.a[r]) for nrow rows, h [nrow][gate rows]
// (the batched gate/up of moe_expert_batch, sml/sml-run.c:3166-3185)
int sml_hip_gemm_swiglu(const sml_hip_mat * gate, const sml_hip_mat * up, const int8_t * q, const float * scale,
                        const int32_t * sums, int nrow, float * h);
// The same two products for activations quantized per 256 values
// (sml_hip_normq with per256 = 1, the batched regime's sml_quantize_act_sb).
// Q4 with more than 8 rows and input widths a multiple of 256 runs on MFMA,
// summing each superblock's sq_g*dot_g and (mq_g-127)*sum_g in integers and
// applying the fp32 scales once per 256 columns; the rest runs the per-group
// kernels, which are exact on such activations (the scale repeats in every
// group). Above 16 rows (prompt reading) Q4 runs on the prompt GEMM: tiles of
// 128 weight rows (SwiGLU: 64) x 64 positions, the weight and activation
// tiles staged in LDS, the same integer superblock sums; other widths run in
// slices of 16 rows.
// replaces sml_matvec_batch_flat4_sb and sml_rlp_matvec
// (sml/sml-kernel.c:1414-1435,1820-1840) as batch_group dispatches them in
// the prompt and default multi-sequence regimes (sml/sml-run.c:2090-2150)
int sml_hip_gemm_sb(const sml_hip_mat * m, const int8_t * q, const float * scale, const int32_t * sums, int nrow,
                    float * y);
int sml_hip_gemm_swiglu_sb(const sml_hip_mat * gate, const sml_hip_mat * up, const int8_t * q, const float * scale,
                           const int32_t * sums, int nrow, float * h);

// ------------------------------------------------------------ MoE expert FFN
// One MoE FFN layer resident in HBM: the f32 router (and bias) and every
// expert's gate/up/down of record blk.<layer>.ffn_{gate,up,down}.<e>.weight,
// for up to max_tokens (1..16) tokens per call. Routing modes: top-k with
// softmax over the chosen (moe_flags bit 0, Mixtral/Granite) or over all
// experts; other modes, shared experts and expert biases are refused.
// replaces the expert weights of sml_load_layers (sml/sml-run.c:1676-1745)
typedef struct sml_hip_moe sml_hip_moe;
sml_hip_moe * sml_hip_moe_from_file(const char * path, int layer, int max_tokens);
void          sml_hip_moe_free(sml_hip_moe * m);
int           sml_hip_moe_info(const sml_hip_moe * m, int * nexp, int * k, int * n_ff, size_t * expert_bytes);
// Activation regime of the expert products: per256 = 0 (default) quantizes
// per 32 values, as the stepped moe_ffn does (sml/sml-run.c:3071-3124);
// 1 per 256, as moe_ffn_batch does in the batched regimes
// (sml/sml-run.c:3153-3241 through batch_group, sml/sml-run.c:2103-2127).
int           sml_hip_moe_regime(sml_hip_moe * m, int per256);
// out[t] = sum over the chosen experts j of w[t][j] * FFN_e(x[t]) for T tokens
// of normed input x [T][n_embd]: the router in double (sml/sml-run.c:3075-3080),
// sml_moe_route's choice (sml/sml-run.c:2925-3037), each chosen expert's
// weights read once for all tokens that chose it (moe_ffn_batch,
// sml/sml-run.c:3189-3241), outputs added in choice order. sel/w ([T][k])
// and logits ([T][nexp]) receive the routing when not NULL. Device pointers.
int sml_hip_moe_ffn(sml_hip_moe * m, const float * x, int T, float * out, int32_t * sel, float * w, float * logits);
// Time `iters` calls (HIP events); count_out (host, nexp) gets the tokens per
// expert of the last call when not NULL.
int sml_hip_moe_time(sml_hip_moe * m, const float * x, int T, float * out, int iters, float * ms_total,
                     int32_t * count_out);

// ------------------------------------------------------------ GPTQ-style 4-bit
// A GPTQ (AutoGPTQ / optimum) 4-bit matrix resident in HBM as its own three
// arrays, rows = outputs, cols = inputs: qweight int32 [cols/8][rows] (8 codes
// along the input, lowest nibble first), qzeros int32 [cols/128][rows/8] (8
// zero codes along the output), scales fp16 [cols/128][rows]; group 128,
// identity g_idx (desc_act: sml_hip_gptq_upload_gidx); zero_add 1 for the v1 files (stored zero = zero - 1), 0 for
// v2. Weight = (code - zero) * scale, the layout tooling/sml_unpack.py:66-95
// (dequant_gptq) converts offline; the reference engine has no GPU kernel for
// it. rows % 8 == 0, cols % 128 == 0.
typedef struct sml_hip_gptq sml_hip_gptq;
sml_hip_gptq * sml_hip_gptq_upload(const int32_t * qweight, const int32_t * qzeros, const uint16_t * scales,
                                   int rows, int cols, int group, int zero_add);
// The same with GPTQ's desc_act: g_idx int32 [cols], input k's group, every
// group holding exactly `group` inputs (the activation-order layout GPTQ
// writes); NULL or an identity g_idx is the upload above. The input columns
// are reordered stably by g_idx so each group's codes are contiguous, and the
// GEMV gathers x through that order; sml_hip_gptq_unpack then returns codes
// in it (device column i is input column i of the stable sort by g_idx).
// Follows dequant_gptq's g_idx branch (tooling/sml_unpack.py:90-96).
sml_hip_gptq * sml_hip_gptq_upload_gidx(const int32_t * qweight, const int32_t * qzeros, const uint16_t * scales,
                                        const int32_t * g_idx, int rows, int cols, int group, int zero_add);
void           sml_hip_gptq_free(sml_hip_gptq * m);
// An AWQ 4-bit matrix (AutoAWQ GEMM layout, what tooling/sml_unpack.py:78,
// 100-118 dequant_awq reads): qweight int32 [cols][rows/8] with 8 outputs per
// word, output 8j+k in nibble (0, 4, 1, 5, 2, 6, 3, 7)[k]; qzeros int32
// [cols/128][rows/8] packed the same way, or NULL for the default zero 8;
// scales fp16 [cols/128][rows]; weight = (code - zero) * scale. Repacked on
// the host into the GPTQ device layout, so every sml_hip_gptq_* call takes
// it. The reference converts AWQ copies offline and has no kernel for it.
sml_hip_gptq * sml_hip_awq_upload(const int32_t * qweight, const int32_t * qzeros, const uint16_t * scales,
                                  int rows, int cols, int group);
// Bytes the matrix occupies in HBM (qweight + qzeros + scales).
size_t         sml_hip_gptq_bytes(const sml_hip_gptq * m);
// y = W.x with fp32 x (no activation quantization).
int sml_hip_gptq_matvec(const sml_hip_gptq * m, const float * x, float * y);
// Codes [nrows][cols] and zeros [nrows][cols/128] (stored zero + zero_add) of
// rows [row0, row0+nrows): the integers dequant_gptq works on
// (tooling/sml_unpack.py:66-76,84-89).
int sml_hip_gptq_unpack(const sml_hip_gptq * m, int row0, int nrows, uint8_t * codes, uint8_t * zeros);
// Time `iters` launches of sml_hip_gptq_matvec rotating over `ncopy` matrices.
int sml_hip_gptq_time(const sml_hip_gptq * const * mats, int ncopy, const float * x, float * y, int iters,
                      float * ms_total);

// ------------------------------------------------------------ unpack / embed
// Integer code of every weight of rows [row0, row0+nrows), one byte each,
// permuted column order: the unpack truth of sml_dequant_row_* (sml/sml-kernel.c:2134-2260)
int sml_hip_unpack(const sml_hip_mat * m, int row0, int nrows, uint8_t * out);
// Row *tok dequantized and scattered through perm into x (sml/sml-run.c:3291-3344)
int sml_hip_embed(const sml_hip_mat * m, const int32_t * tok, const int32_t * perm, float * x);

// ------------------------------------------------------------ attention
// RoPE q and k at position *pos (halved pairs, table rows of `half` floats),
// write k and v as fp16 into the layer's cache at *pos, then softmax attention
// of every query head over positions [0, *pos] into out (n_head*hd floats).
// replaces rope_tab + f32_to_f16 + attn_head (sml/sml-run.c:339-372,3414-3434)
// and the reference GPU's sml_g_attn2 (sml/sml-gpu-fast.cu:363-453).
// hd must be 128; n_head/n_kv at most 8; part needs attn_part_floats().
size_t sml_hip_attn_part_floats(int n_head, int hd, int n_ctx);
int sml_hip_attention(float * q, const float * k, const float * v, uint16_t * kcache, uint16_t * vcache,
                      const float * cos_t, const float * sin_t, const int32_t * pos,
                      int n_head, int n_kv, int hd, int n_ctx, float * part, float * out);
// Causal attention of a prompt chunk: rows b = 0..n_rows-1 are positions
// pos0+b of one sequence, each row of qkv its q, k and v ((n_head + 2*n_kv)*hd
// floats); every row's k is rotated and its k and v written to the cache
// before any row attends, then row b's heads attend over [0, pos0+b] into out
// (n_rows x n_head*hd). The level-2 prompt's attention (the MFMA flash kernel,
// its KV range split and merged as the grid needs; SML_ATTN_FLASH=0: a wave
// per position), replacing the rope + f32_to_f16 + ms_attn of the reference's
// batched prompt body (sml/sml-run.c:2192-2210,2368-2378). hd must be 128,
// n_kv at most 8; part holds n_rows*n_head*ceil(n_ctx/128)*(hd+2) floats.
int sml_hip_attention_prompt(const float * qkv, int n_rows, int pos0, uint16_t * kcache, uint16_t * vcache,
                             const float * cos_t, const float * sin_t, int n_head, int n_kv, int hd, int n_ctx,
                             float * part, float * out);
// The sum of n values (0..16384, each >= 0) in the order of a serial float
// loop, sum = sum + x[i] for i = 0, 1, ... (the softmax sum of attn_row,
// sml/sml-run.c:280-287), as exact-mode attention computes it: bit for bit
// that loop's result, mostly in parallel. *out is device memory.
int sml_hip_softmax_sum(const float * x, int n, float * out);
// The same, with out also quantized per 32 values for the o product (the
// codes, scales and sums of sml_quantize_act, sml/sml-kernel.c:86-106), as the
// decode step runs it when the o product reads the heads in order.
int sml_hip_attention_q(float * q, const float * k, const float * v, uint16_t * kcache, uint16_t * vcache,
                        const float * cos_t, const float * sin_t, const int32_t * pos,
                        int n_head, int n_kv, int hd, int n_ctx, float * part, float * out,
                        int8_t * q_out, float * s_out, int32_t * u_out);

// ------------------------------------------------------------ argmax
// First-max greedy pick into *tok (sml_sample_greedy, sml/sml-run.c:3539-3544).
// From 8192 logits it runs in two stages over a scratch buffer of 8 KB that
// this call allocates and frees (the decode step keeps its own); it returns
// once the pick is done.
int sml_hip_argmax(const float * logits, int n, int32_t * tok);
// The same pick, allocating nothing: its two-stage scratch (1024 pairs, 8 KB)
// is a device array the library holds per GPU for the life of the process.
// No counterpart in the reference; it is for callers that cannot allocate
// device memory (code under HIP graph capture, tight serving loops). Takes
// 1..2^30 logits; enqueues on the null stream without waiting. Calls that
// overlap on one GPU (other streams or threads) share the scratch and race.
int sml_hip_argmax_noalloc(const float * logits, int n, int32_t * tok);

#ifdef __cplusplus
}
#endif
