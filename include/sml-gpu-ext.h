// Extensions of the GPU forward pass that the reference's sml-gpu.h does not
// declare. Each names what in the reference it corresponds to.
#pragma once
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

// Release the model, the KV cache and every device buffer (the reference keeps
// them for the life of the process). Safe to call when nothing is open.
void sml_gpu_close(void);

// Greedy decoding with no host round trip per token: starting from token tok
// at position pos, run n steps, each feeding its argmax to the next, and write
// the n chosen ids to out. The per-token work is one captured HIP graph
// replay, as the reference's grading loop does with its CUDA graph
// (sml/sml-gpu-fwd.c:2626-2661). Returns n, or -1 on failure.
int sml_gpu_generate(int tok, int pos, int n, int * out);

// Elapsed GPU milliseconds of the last sml_gpu_generate call, or of the
// kernels of the last sml_gpu_step_multi call without its logits copy (HIP
// events on the decode stream), or -1.
float sml_gpu_last_ms(void);

// Weight bytes one decode step streams (every quantized matrix the step reads,
// codes and fields), the reference's bytes_moved measure (sml/sml-run.c:821-828).
uint64_t sml_gpu_weight_bytes(void);

// Last failure message.
const char * sml_gpu_last_error(void);

// Exact mode: with SML_EXACT=1 in the environment at sml_gpu_open, every
// kernel of the step follows the float order of the reference's x86 build
// (sml_forward, sml/sml-run.c:3243-3523): Q4/Q8 GEMV lanes and FMAs,
// serial sums of squares, attention scores, softmax sum and P.V as serial
// chains, the C library's expf, the SiLU polynomial. Logits then equal the
// reference's CPU path bit for bit, so greedy ids are identical for any
// number of steps. It is slower (the serial chains are latency-bound) and
// serves one sequence. Prompts of dense Q4/Q8 models are read batched, 64
// positions a chunk, with the same arithmetic per position (logits equal to
// stepping the prompt, bit for bit); others a token at a time. Returns 1 when
// the open model runs exact, else 0.
int sml_gpu_exact(void);

// ---------------------------------------------------------------- several sequences
// The multi-sequence step sml-batched drives on the CPU through
// sml_forward_multi (sml/sml-run.h:290-294, sml/sml-batched.c:82-130), with
// its activation regime (sml/sml-run.c:2579-2596): SML_MULTI=exact, or at
// most SML_MULTI_EXACT_MAX (default 2) sequences, quantizes per 32 values, so
// every sequence's logits equal decoding it alone, bit for bit; otherwise
// every product's input is quantized per 256 values (sml_quantize_act_sb) and
// Q4 products sum each superblock in integers, as sml_rlp_matvec does.
//
// Give the open model ns (1..16) KV cache slots; slot 0 is the cache
// sml_gpu_step / sml_gpu_prefill use. Every layer's q, k and v must share one
// permutation and width (and gate/up likewise). Returns ns, or 0.
int sml_gpu_slots(int ns);
// sml_gpu_prefill into slot `slot`'s cache; logits of the last id (the
// library's host buffer), NULL on failure.
const float * sml_gpu_prefill_slot(int slot, const int * ids, int pos0, int n);
// One token for each of ns sequences: sequence b feeds tok[b] at position
// pos[b] into slot slot[b] (distinct slots). Each weight matrix is read once
// for all of them. Logits land in logits_out[b * n_vocab] (caller's host
// memory). Returns ns, or 0.
int sml_gpu_step_multi(const int * tok, const int * pos, const int * slot, int ns, float * logits_out);

#ifdef __cplusplus
}
#endif
