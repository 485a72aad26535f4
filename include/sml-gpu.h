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

// Load the model onto the GPU. gpu_layers > 0 keeps that many leading
// layers' matrices in HBM and streams the rest (a split): their matrices
// stay in pinned host memory and cross to one staging region in HBM ahead of
// each use, so every layer still computes on the card and the logits equal
// the whole model's bit for bit. gpu_layers <= 0: SML_GPU_LAYERS if set,
// else every layer when the matrices, the K/V cache and a reserve
// (SML_SPLIT_RESERVE_MB, 1024) fit in the free HBM, else the leading layers
// that fit. A split of a mixture-of-experts model is refused. threads is
// accepted for the reference's CPU side of a split and unused. Returns 1, or
// 0 with the reason in why.
// replaces sml/sml-gpu.h:11 (sml/sml-gpu-fwd.c:2353-2380)
int sml_gpu_open(const char * path, int n_ctx, int threads, int gpu_layers, char * why, int nwhy);

// Read ids[0..n) at positions pos0..pos0+n-1; logits after the last one.
// NULL if pos0 + n > n_ctx. replaces sml/sml-gpu.h:14 (sml/sml-gpu-fwd.c:2388-2402)
const float * sml_gpu_prefill(const int * ids, int pos0, int n);

// One token at position pos; its logits. NULL if pos >= n_ctx.
// replaces sml/sml-gpu.h:17 (sml/sml-gpu-fwd.c:2404-2412)
const float * sml_gpu_step(int tok, int pos);

// Layers whose matrices stay in HBM, and (in *of) of how many; fewer means
// a split. replaces sml/sml-gpu.h:20
int sml_gpu_layers(int * of);

// How a prompt is read: 0 a token at a time through the decode graph; 1 (the
// default) batched in chunks of 32 positions (16 with MoE layers) with every
// product in the GEMV's arithmetic, equal to stepping bit for bit; 2 batched
// with the Q4 products on the matrix cores (MFMA), equal to float rounding.
// Exact mode (SML_EXACT=1) takes 2 as 1: chunks of 64 positions in the
// reference CPU path's float order, equal to its stepping bit for bit.
// replaces sml/sml-gpu.h:26 (sml/sml-gpu-fwd.c:2420-2423)
void sml_gpu_prompt_mode(int level);

// A split model decoding on the CPU: 1 if on. A split here decodes on the
// card (its streamed layers included), so this is always 0.
// replaces sml/sml-gpu.h:28
int sml_gpu_decode_cpu(int on);

// A middle stage of a split model: after the layers kept in HBM, fn(rows,
// pos0, n) runs the next `layers` layers on the n hidden rows (n x n_embd
// floats in host memory, positions pos0.., in place) and returns 1, or 0 to
// fail the call; the layers after them continue on the card. Prompts hand
// over one chunk at a time, in order. Slot 0 only: the batched step and
// other slots' prompts fail while a stage is set. layers 0 or fn NULL
// removes it; a model without a split never calls it. replaces
// sml/sml-gpu.h:34
void sml_gpu_set_middle(int layers, int (*fn)(float * rows, int pos0, int n));

#ifdef __cplusplus
}
#endif
