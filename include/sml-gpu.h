// The GPU forward pass of the SML engine as a C library, for sml-server.
//
// The seven prototypes below are the reference's drop-in boundary
// (sml/sml-gpu.h:11-34), kept identical so the reference's caller
// (sml/sml-server.c:216-265,1554-1685) links against this MI355X library
// unchanged. One model and one KV cache per process; positions are absolute,
// so a prompt may continue a prefix the cache already holds. Every call
// returns NULL (or 0) on failure instead of ending the process, and the
// caller serves on the CPU. Returned logits live in a library-owned host
// buffer of n_vocab floats, valid until the next call. Not re-entrant.
#pragma once

#ifdef __cplusplus
extern "C" {
#endif

// Load the model onto the GPU. gpu_layers <= 0 or >= the layer count puts
// every layer on the card; a smaller count (the reference's GPU/CPU split)
// is refused with a reason. threads is accepted for the CPU side of a split
// and unused. Returns 1, or 0 with the reason in why.
// replaces sml/sml-gpu.h:11 (sml/sml-gpu-fwd.c:2353-2380)
int sml_gpu_open(const char * path, int n_ctx, int threads, int gpu_layers, char * why, int nwhy);

// Read ids[0..n) at positions pos0..pos0+n-1; logits after the last one.
// NULL if pos0 + n > n_ctx. replaces sml/sml-gpu.h:14 (sml/sml-gpu-fwd.c:2388-2402)
const float * sml_gpu_prefill(const int * ids, int pos0, int n);

// One token at position pos; its logits. NULL if pos >= n_ctx.
// replaces sml/sml-gpu.h:17 (sml/sml-gpu-fwd.c:2404-2412)
const float * sml_gpu_step(int tok, int pos);

// Layers on the card, and (in *of) of how many. replaces sml/sml-gpu.h:20
int sml_gpu_layers(int * of);

// How a prompt is read: 0 a token at a time through the decode graph; 1 (the
// default) batched in chunks of 16 positions with every product in the
// GEMV's arithmetic, equal to stepping bit for bit; 2 batched with the Q4
// products on the matrix cores (MFMA), equal to float rounding. Exact mode
// (SML_EXACT=1) reads prompts a token at a time whatever the level.
// replaces sml/sml-gpu.h:26 (sml/sml-gpu-fwd.c:2420-2423)
void sml_gpu_prompt_mode(int level);

// A split model decoding on the CPU: 1 if on. Every layer is on the card
// here, so this is always 0. replaces sml/sml-gpu.h:28
int sml_gpu_decode_cpu(int on);

// A middle stage after the GPU's layers (split models only); recorded and
// unused since every layer runs on the card. replaces sml/sml-gpu.h:34
void sml_gpu_set_middle(int layers, int (*fn)(float * rows, int pos0, int n));

#ifdef __cplusplus
}
#endif
