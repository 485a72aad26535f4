// CPU ORACLE — test infrastructure only.
//
// A plain-C restatement of the reference SML engine's CPU path for the
// quantized decode hot path. Only tests/, __graft_entry__.smoke() and
// bench.py's cpu_baseline leg may load it, and only as the checker or the
// reported CPU baseline: the GPU library never links, calls or falls back to
// anything here.
//
// Every function names the reference file:line it follows. How each one is
// pinned (reference build, closed forms, brute force) is listed in the tests
// that exercise it; none is left unpinned.
#pragma once
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

// Activation quantization, one scale per 32 values.
// follows sml/sml-kernel.c:86-106 (scalar arm; the AVX2 arm at :44-85 is the
// same arithmetic bit for bit)
void orc_quantize_act(const float * x, int n, int8_t * q, float * scale, int32_t * sums);
// One scale per 256 values, written into every group of the superblock.
// follows sml/sml-kernel.c:165-184
void orc_quantize_act_sb(const float * x, int n, int8_t * q, float * scale, int32_t * sums);

// A quantized FLAT tensor as stored in the file: planes in storage order and the
// four field arrays. scale6 / minneg are the file flags (sml/sml-kernel.h:64-98).
typedef struct {
    const uint8_t  * plane[4];
    const uint16_t * sd;
    const uint8_t  * sq;
    const uint16_t * md;      // NULL: symmetric file (no min)
    const uint8_t  * mq;
    int rows, cols, nbits;
    int scale6, minneg;
} orc_tensor;

// Integer code of every weight of one row (permuted column order).
// Plane order follows tooling/sml_quantize.py:104-106 (FLAT_PLANES) and the
// reads follow sml/sml-kernel.c:231-263 (2-bit), :2134-2157 (nibbles),
// :2160-2170 (1-bit), :2174-2198 (Q8), :2235-2260 (Q6), dispatched as
// sml/sml-run.c:586-603,3300-3335.
void orc_unpack_row(const orc_tensor * t, int row, uint8_t * codes);

// Group g's step and min of one row: step = f16(sd)*sq, min = f16(md)*(mq - bias),
// bias 127 (8-bit fields), 31 (6-bit), 63 (6-bit negative-only).
// follows sml/sml-kernel.c:206-215,254-258,2146-2149
float orc_step(const orc_tensor * t, int row, int g);
float orc_min(const orc_tensor * t, int row, int g);

// One row dequantized, code*step + min, in permuted order.
// follows sml/sml-kernel.c:2134-2157 (and the per-width forms listed above)
void orc_dequant_row(const orc_tensor * t, int row, float * out);

// y[r] = sum over groups of step*s*dot + min*s*sum  for r in [row0, row1), no
// accumulation into y (callers of the reference zero y first, sml/sml-run.c:757).
// The per-group arithmetic follows the scalar arm sml/sml-kernel.c:2027-2066
// (flat4) and :1934-1971 (2-bit planes), with the plane dispatch of
// sml/sml-run.c:612-680 folded into one integer dot over the unpacked code
// (the code is linear in its planes, so the integer dot is the same number).
void orc_matvec(const orc_tensor * t, const int8_t * q, const float * scale, const int32_t * sums,
                float * y, int row0, int row1);

// RMSNorm with a double sum of squares. follows sml/sml-run.c:147-152
void orc_rms_norm(float * out, const float * x, const float * w, int n, float eps);
// cos/sin table, halved pairs. follows sml/sml-run.c:1383-1393
void orc_rope_table(float theta, int half, int n_ctx, float * cos_t, float * sin_t);
// follows sml/sml-run.c:339-372 (halved pairs branch)
void orc_rope(float * x, int n_head, int head_dim, int half, const float * cos_row, const float * sin_row);
// fp16 round-to-nearest-even encode / decode. follows sml/sml-run.c:68-77,85-109
uint16_t orc_f32_to_f16(float f);
float    orc_f16_to_f32(uint16_t h);
// Decode attention of one head over positions [0, pos], keys/values fp16,
// `stride` halves apart. follows sml/sml-run.c:180-266 (scalar arm) and
// softmax :280-287
void orc_attn_head(const float * qh, const uint16_t * kc, const uint16_t * vc, size_t stride,
                   int pos, int hd, float inv, float * scratch, float * out);
// g = g/(1+exp(-g)) * u. follows sml/sml-run.c:451-454
void orc_silu_mul(float * g, const float * u, int n);
// Top-k routing, ties to the lower index; moe_flags bit 0 renormalises over
// the chosen. follows sml/sml-run.c:3010-3035
int orc_moe_route(const float * lg, int ne, int k, unsigned moe_flags, int * sel, float * w);
// Every routing mode of sml_moe_route (sml/sml-run.c:2925-3037): moe_flags
// bit 0 normalizes the chosen weights (softmax over the chosen in plain
// top-k), bit 1 scores by sigmoid, bit 2 is PhiMoE's sparsemixer (scale:
// its jitter), bit 3 scores a group by its best expert (else its best two);
// exp_bias (NULL: none) shifts the choice, groups/topk_group keep the best
// groups' experts; scale multiplies the weights. expf is the C library's.
int orc_moe_route2(const float * lg, int ne, int k, unsigned moe_flags, float scale, int groups, int topk_group,
                   const float * exp_bias, int * sel, float * w);
// Router logits with a double accumulator. follows sml/sml-run.c:3075-3080
void orc_router(const float * router, const float * x, int ne, int n_embd, float * lg);
// First-max greedy pick. follows sml/sml-run.c:3539-3544
int orc_argmax(const float * logits, int n);

// GPTQ-style 4-bit (tooling/sml_unpack.py:66-95): qweight int32 [cols/8][rows]
// (8 codes along the input, lowest nibble first), qzeros int32
// [cols/group][rows/8] (8 zero codes along the output), scales fp16
// [cols/group][rows]; zero = stored + zero_add (1 for the v1 files);
// g = input // group (identity g_idx).
// Codes (cols) and zeros (cols/group) of one output row.
void orc_gptq_unpack_row(const int32_t * qweight, const int32_t * qzeros, int rows, int cols, int group,
                         int zero_add, int row, uint8_t * codes, uint8_t * zeros);
// Weights of one output row: (float) (code - zero) * (float) scale.
void orc_gptq_dequant_row(const int32_t * qweight, const int32_t * qzeros, const uint16_t * scales, int rows,
                          int cols, int group, int zero_add, int row, float * out);
// y = W.x with the dequantized weights, summed in double.
void orc_gptq_matvec(const int32_t * qweight, const int32_t * qzeros, const uint16_t * scales, int rows, int cols,
                     int group, int zero_add, const float * x, float * y);
// desc_act: input k takes group g_idx[k]'s zero and scale.
void orc_gptq_dequant_row_gidx(const int32_t * qweight, const int32_t * qzeros, const uint16_t * scales,
                               const int32_t * g_idx, int rows, int cols, int group, int zero_add, int row,
                               float * out);
void orc_gptq_matvec_gidx(const int32_t * qweight, const int32_t * qzeros, const uint16_t * scales,
                          const int32_t * g_idx, int rows, int cols, int group, int zero_add, const float * x,
                          float * y);
void orc_awq_unpack_row(const int32_t * qweight, const int32_t * qzeros, int rows, int cols, int group, int row,
                        uint8_t * codes, uint8_t * zeros);
void orc_awq_dequant_row(const int32_t * qweight, const int32_t * qzeros, const uint16_t * scales, int rows,
                         int cols, int group, int row, float * out);

// ---------------------------------------------------------------- GGUF Q4_K
// One row of ggml's block_q4_K blocks (cols/256 blocks of 144 bytes: fp16 d,
// fp16 dmin, 12 bytes of packed 6-bit sub-block scales and mins, 128 bytes of
// codes) dequantized by the published formula (ggml's dequantize_row_q4_K):
// per 64 weights, sub-blocks 2c and 2c+1 take the low and high nibbles of the
// same 32 code bytes, y = (d*sc)*q - dmin*m.
void orc_q4k_dequant_row(const uint8_t * blocks, int cols, float * out);
void orc_q5k_dequant_row(const uint8_t * blocks, int cols, float * out);
// One row of ggml's Q8_0 (type 8: 34-byte blocks of fp16 d and 32 int8
// codes, y = d*q), Q4_0 (type 2: 18-byte blocks of fp16 d and 16 code bytes,
// the low nibbles weights 0..15 and the high ones 16..31, y = d*(q - 8)) or
// Q6_K (type 14: 210-byte blocks of ql[128], qh[64], int8 scales[16] and
// fp16 d; per 128 weights, weight l+32k takes bits 4(k/2) of ql[l + 32(k&1)]
// and bits 2k of qh[l], y = (d*scales[i/16])*(q - 32)) blocks dequantized by
// the published formulas (ggml's dequantize_row_q8_0 / _q4_0 / _q6_K, which
// gguf-py's numpy restatement follows in the same float order), then rounded
// to fp16 as the float16 copy transformers writes. Returns -1 for another
// type or a width that is not whole blocks.
int orc_gguf_dequant_f16_row(int type, const uint8_t * blocks, int cols, float * out);

// ---------------------------------------------------------------- expf restated
// The C library's expf (glibc 2.35, x86-64 with FMA) from its published
// algorithm, as the GPU's exact attention and routing restate it: x*32/ln2 =
// k + r in double (k rounded through the 1.5*2^52 shift, both products
// fused), 2^(k/32) from a 32-entry table of 2^(i/32), 2^(r/32) by a cubic,
// one rounding to float. Used for x <= 0.
float orc_expf_published(float x);
// Count of floats x <= 0 (every stride-th bit pattern from -0.0 down to
// -inf) where orc_expf_published(x) and the library's expf(x) differ in bits.
long orc_expf_mismatches(unsigned stride);

// ---------------------------------------------------------------- decoder
// A whole decode step over an SSF file (Llama / Qwen2 / Mixtral family: RMSNorm,
// halved RoPE, GQA, SwiGLU, optional q/k/v bias, tied or untied head, top-k MoE).
// follows sml/sml-run.c:3243-3523 for those features.
typedef struct orc_model orc_model;
orc_model * orc_model_open(const char * path, int n_ctx);
void        orc_model_close(orc_model * m);
// logits of token at position pos (positions must be fed in order from 0)
const float * orc_forward(orc_model * m, int token, int pos);
int orc_n_vocab(const orc_model * m);
void orc_model_per256(orc_model * m, int on);
// Tensor view by name, for single-matrix checks.
int orc_model_tensor(const orc_model * m, const char * name, orc_tensor * out, const int32_t ** perm);


// ---------------------------------------------------------------- re-quantization (sml_oracle_quant.c)
// The reference quantizer's searches and encoder for a tensor without
// calibration feedback, the step a GPTQ/AWQ copy takes after the unpacker.
// follows sml/sml-quant.c:20-95 (sml_asym_grid), in its build's FMA order
void orc_asym_grid(const float * wp, int rows, int cols, int group, int nbits, int rem, const float * wt,
                   const float * facs, int ncand, int iters, int refit, float * out_l, float * out_s);
// follows sml/sml-quant.c:101-137 (sml_field_search)
void orc_field_search(const float * w, int rows, int cols, int group, const float * dv, const float * dm,
                      int32_t * q8, int32_t * mq8, int nmax, int hi, int moff, int mmax, const float * wt, int radius);
// the range factors of tooling/sml_grid_c.py:41-42; returns their count
int orc_grid_facs(int ncand, float * facs);
// follows tooling/sml_quantize.py:320-363 (two_level, 8-bit fields)
void orc_two_level(const float * v, int rows, int ng, int gps, int is_signed, uint16_t * d16, uint8_t * q8, float * eff);
// follows tooling/sml_quantize.py:565-572 (the codes of encode)
void orc_requant_codes(const float * wp, int rows, int cols, const float * eff_s, const float * eff_m, int nmax,
                       uint8_t * codes);
// follows tooling/sml_quantize.py:479 (ascending max |w|; ties by column index)
void orc_perm_maxabs(const float * w, int rows, int cols, int32_t * perm);
// follows tooling/sml_unpack.py:66-118 (GPTQ 2/4/8-bit, AWQ 4-bit; fp16 result)
void orc_unpack_dequant_f16(const int32_t * qweight, const int32_t * qzeros, const uint16_t * scales,
                            const int32_t * g_idx, int rows, int cols, int bits, int group, int zero_add, int awq,
                            float * out);
// follows tooling/sml_quantize.py:426-581 (run + encode with no activations)
void orc_requant(const float * w, int rows, int cols, int nbits, const int32_t * perm_in, const float * wt, int radius,
                 uint8_t * codes, uint16_t * sd, uint8_t * sq, uint16_t * md, uint8_t * mq, int32_t * perm);

#ifdef __cplusplus
}
#endif
