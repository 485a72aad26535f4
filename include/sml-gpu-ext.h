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

// Elapsed GPU milliseconds of the last sml_gpu_generate call (HIP events on
// the decode stream), or -1.
float sml_gpu_last_ms(void);

// Weight bytes one decode step streams (every quantized matrix the step reads,
// codes and fields), the reference's bytes_moved measure (sml/sml-run.c:821-828).
uint64_t sml_gpu_weight_bytes(void);

// Last failure message.
const char * sml_gpu_last_error(void);

#ifdef __cplusplus
}
#endif
