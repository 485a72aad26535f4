// The allocation-free greedy pick: sml_hip_argmax without its per-call
// scratch allocation, for callers that cannot allocate device memory (code
// under HIP graph capture, tight serving loops, harnesses that forbid it).
//
// The two-stage pick (per-workgroup (value, index) pairs, then one
// workgroup over them) needs ARGMAX_MAX_PARTS pairs of scratch. Here they live
// in a file-scope device array, one copy per GPU for the life of the process.
// Its address comes from the runtime once per device, with that device
// current; the host never hands the array's own name to a kernel. Every call
// on a GPU shares that GPU's array: calls that overlap on one GPU (other
// streams, other threads) race. Stage 1 writes every pair stage 2 reads, so
// nothing needs clearing between calls.
#include <hip/hip_runtime.h>

extern "C" {
#include "ops.h"
}

#define NOALLOC_MAX_DEVICES 64

static __device__ __align__(256) int2 scratch[ARGMAX_MAX_PARTS];
static int2 * scratch_dev[NOALLOC_MAX_DEVICES];      // the array's device address, per GPU

// Largest input the entry point takes (the pick indexes logits with int).
#define NOALLOC_ARGMAX_MAX_N (1 << 30)

static int2 * scratch_on(int device) {
    if (device < 0 || device >= NOALLOC_MAX_DEVICES) hx_failf("device %d out of range", device);
    if (!scratch_dev[device]) {
        void * p = NULL;
        HX(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        scratch_dev[device] = (int2 *) p;
    }
    return scratch_dev[device];
}

extern "C" int sml_hip_argmax_noalloc(const float * logits, int n, int32_t * tok) {
    HX_ENTRY(-1);
    if (!hx.inited) hx_init(0);
    if (!logits || !tok || n < 1 || n > NOALLOC_ARGMAX_MAX_N)
        hx_failf("argmax_noalloc takes 1..%d logits (got %d)", NOALLOC_ARGMAX_MAX_N, n);
    int2 * part = n >= ARGMAX_TWO_STAGE_MIN ? scratch_on(hx.device) : NULL;
    op_argmax(0, logits, n, tok, NULL, NULL, 0, part);
    HX_LEAVE();
    return 0;
}
