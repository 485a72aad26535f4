// Internal launch helpers shared by the kernel-level C ABI (ops.c) and the
// decode engine (engine.c). These do not arm an entry point: failures
// longjmp to whichever exported call is running.
#pragma once
#include "hipx.h"
#include "ssf.h"
#include "sml-hip.h"

struct sml_hip_mat {
    sml_kmat k;          // device pointers; k.rows is the row count
    int nbits, cols;
    void * mem;          // the single allocation holding planes and fields
    size_t bytes;        // planes + fields bytes (what one GEMV streams)
};


sml_hip_mat * mat_upload(const uint8_t * const planes[4], const uint16_t * sd, const uint8_t * sq,
                         const uint16_t * md, const uint8_t * mq, int rows, int cols, int nbits,
                         int scale6, int minneg);
sml_hip_mat * mat_from_record(const ssf_file * f, const ssf_record * r);
void mat_free(sml_hip_mat * m);

void op_normq(hipStream_t st, float * x, const float * resid, const float * w, float eps, int n,
              int nout, const int32_t * const * perm, int8_t * const * q, float * const * scale,
              int32_t * const * sums, float * normed, int per256);
void op_gemv(hipStream_t st, const sml_hip_mat * const * mats, int nm, int epi, const int8_t * q,
             const float * scale, const int32_t * sums, float * const * y, const float * const * bias,
             const float * resid);
void op_embed(hipStream_t st, const sml_hip_mat * m, const int32_t * tok, const int32_t * pos,
              const int32_t * perm, float * x);
void op_attention(hipStream_t st, const float * q, const float * k, const float * v, uint16_t * kc, uint16_t * vc,
                  const float * cos_t, const float * sin_t, const int32_t * pos, int n_head, int n_kv,
                  int hd, int n_ctx, float * part, float * out, int8_t * q_out, float * s_out,
                  int32_t * u_out);
void op_argmax(hipStream_t st, const float * logits, int n, int32_t * tok, int32_t * pos, int32_t * hist,
               int hist_n);
void op_advance(hipStream_t st, int32_t * pos);
void op_silu_mul(hipStream_t st, float * g, const float * u, int n);
