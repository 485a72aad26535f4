// Ingest on the GPU: a GPTQ or AWQ tensor (or any float tensor) re-quantized
// into SSF FLAT planes and two-level fields at a width of its own -- the
// reference's route for a quantized copy (tooling/sml_unpack.py dequantizes
// it to float16, then tooling/sml_quantize.py encodes it) for a tensor without
// calibration feedback -- with the quantizer's two searches as drop-ins for
// its fused C library.
//
// The two searches take and return HOST arrays with the reference library's
// own prototypes, so the reference's loader (tooling/sml_grid_c.py) binds
// this library in place of sml-quant's. The tensor-level calls take device
// arrays (sml_hip_malloc). Calls return 0, or -1 with sml_hip_last_error().
#pragma once
#include <stddef.h>
#include <stdint.h>

#include "sml-hip.h"

#ifdef __cplusplus
extern "C" {
#endif

// ------------------------------------------------------------ drop-ins for sml/sml-quant.c
// Per-group (min, step) of the asymmetric grid: ncand candidate ranges
// (facs), each refitted by weighted least squares (iters rounds, when refit)
// before the choice. wp: rows x cols, columns already permuted; wt: cols
// normalised weights or NULL for ones; out_l, out_s: rows x cols/group.
// Groups: a multiple of 8 up to 256. Bit for bit the reference library's
// results. No return value, as there: a failure is printed to stderr and the
// outputs are NaN.
// replaces sml/sml-quant.c:38-95 (sml_asym_grid)
void sml_asym_grid(const float * wp, int rows, int cols, int group, int nbits, int rem, const float * wt,
                   const float * facs, int ncand, int iters, int refit, float * out_l, float * out_s);
// Each group's step field q8 and min field mq8 moved to the best neighbour
// within +-radius by weighted error with the codes re-derived; dv, dm: rows x
// cols/group, each group's superblock scale. A failure is printed and the
// fields are left as given.
// replaces sml/sml-quant.c:101-137 (sml_field_search)
void sml_field_search(const float * w, int rows, int cols, int group, const float * dv, const float * dm,
                      int32_t * q8, int32_t * mq8, int nmax, int hi, int moff, int mmax, const float * wt, int radius);
// The same two searches, returning 0 or -1.
int sml_hip_asym_grid(const float * wp, int rows, int cols, int group, int nbits, int rem, const float * wt,
                      const float * facs, int ncand, int iters, int refit, float * out_l, float * out_s);
int sml_hip_field_search(const float * w, int rows, int cols, int group, const float * dv, const float * dm,
                         int32_t * q8, int32_t * mq8, int nmax, int hi, int moff, int mmax, const float * wt,
                         int radius);

// ------------------------------------------------------------ whole tensors (device arrays)
// GPTQ (bits 2, 4, 8: qweight int32 [cols/per][rows] along the input, qzeros
// int32 [groups][rows/per] along the output, stored zero + zero_add, scales
// fp16 [groups][rows], g_idx [cols] or NULL for k / group) or AWQ (awq = 1,
// 4 bits: qweight [cols][rows/8] along the output in nibble order
// 0,4,1,5,2,6,3,7, qzeros likewise or NULL for zero 8) dequantized to out
// [rows][cols] (rows = outputs) as (code - zero) * scale in fp32 rounded to
// fp16, the float16 copy the unpacker writes.
// replaces tooling/sml_unpack.py:66-118 (_unpack_ints, dequant_gptq, dequant_awq)
int sml_hip_unpack_dequant(const int32_t * qweight, const int32_t * qzeros, const uint16_t * scales,
                           const int32_t * g_idx, int rows, int cols, int bits, int group, int zero_add, int awq,
                           float * out);
// GGUF blocks of ggml type Q8_0 (8), Q4_0 (2) or Q6_K (14), row-major with
// each row's blocks in order (cols a multiple of 32, of 256 for Q6_K),
// dequantized to out [rows][cols] by ggml's published formulas and rounded
// to fp16: the float16 copy transformers writes from a GGUF before the
// reference re-quantizes it (sml_hip_requant takes it from there).
// replaces tooling/sml_gguf.py:19-27 (the GGUF read through transformers) for
// one tensor of these types
int sml_hip_gguf_dequant(int type, const uint8_t * blocks, int rows, int cols, float * out);
// Re-quantize w [rows][cols] (cols a multiple of 256) into SSF FLAT width
// nbits (2..8): column order perm_in (NULL: ascending max |w| over the rows,
// ties by column), the asymmetric grid (20 candidates, 3 refits), two-level
// 8-bit steps and mins, the field search of radius `radius` (the quantizer's
// default 2; 0 skips it), then every code. wt: cols normalised weights in the
// permuted order, or NULL. Out: the width's planes (storage order, row-major,
// as sml_hip_mat_upload takes them), sd/md [rows][cols/256] fp16, sq/mq
// [rows][cols/32], perm [cols], and codes [rows][cols] (permuted order) when
// not NULL. Allocates its own scratch (about 4 bytes per weight).
// replaces tooling/sml_quantize.py:426-651 (Quantizer.run, encode and _write
// for a tensor without activations)
int sml_hip_requant(const float * w, int rows, int cols, int nbits, const int32_t * perm_in, const float * wt,
                    int radius, uint8_t * const planes[3], uint16_t * sd, uint8_t * sq, uint16_t * md, uint8_t * mq,
                    int32_t * perm, uint8_t * codes);
// GPU time (ms, HIP events) of the last sml_hip_requant's kernels.
float sml_hip_requant_last_ms(void);
// The re-quantized arrays (device) as a matrix every GEMV/GEMM takes.
sml_hip_mat * sml_hip_mat_from_requant(uint8_t * const planes[3], const uint16_t * sd, const uint8_t * sq,
                                       const uint16_t * md, const uint8_t * mq, int rows, int cols, int nbits);
// Write one quantized matrix (host arrays) as an SSF file holding record
// `name`, in the layout the reference loader reads (sml/sml-model.h:78-160).
// replaces tooling/sml_quantize.py:598-651 (Quantizer._write) for one record
int sml_hip_ssf_write_quant(const char * path, const char * name, int rows, int cols, int nbits,
                            const uint8_t * const planes[3], const uint16_t * sd, const uint8_t * sq,
                            const uint16_t * md, const uint8_t * mq, const int32_t * perm);

#ifdef __cplusplus
}
#endif
