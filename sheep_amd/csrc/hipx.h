// Thin HIP binding for the C host: the role sml/sml-gpu-drv.h plays over the
// CUDA driver API in the reference (entry points, error reporting), here over
// the HIP runtime. Every HIP call goes through HX(); a failure records a
// message and longjmps to the innermost armed entry point, which returns its
// failure value (NULL / 0 / -1) to the caller instead of ending the process --
// the reference's library-mode contract (sml/sml-gpu-fwd.c:23-27).
#pragma once
#include <setjmp.h>
#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#include "kargs.h"

typedef struct {
    jmp_buf * jb;                 // innermost armed entry point, NULL when none
    char      err[512];
    int       inited;
    int       device;
    hipModule_t mod;
    hipModule_t mod_ingest;       // the ingest kernels (built without contraction)
    int       ncu;                // compute units of the device
    long      fail_after;         // test hook: fail the Nth HIP call from now (< 0: off)
    long      calls;              // HIP calls made through HX() so far
    float   * kpart;              // split-K GEMM partial products (HX_KPART floats on the device),
                                  // shared by every launch: one stream at a time
} hx_state;

#define HX_KPART (1 << 20)
// the split-K partial buffer, allocated at its first use (the engine asks for
// it at load, before any graph capture)
float * hx_kpart(void);

extern hx_state hx;

void hx_fail(const char * what, hipError_t e);
void hx_failf(const char * fmt, ...);

static inline void hx_check(hipError_t e, const char * what) {
    hx.calls++;
    if (hx.fail_after >= 0 && hx.fail_after-- == 0) e = hipErrorUnknown;
    if (e != hipSuccess) hx_fail(what, e);
}
#define HX(call) hx_check((call), #call)

// Arm an entry point: ENTRY_BEGIN(fail_value) ... ENTRY_END
#define HX_ENTRY(failval)                                        \
    jmp_buf hx_jb_;                                              \
    jmp_buf * hx_prev_ = hx.jb;                                  \
    if (setjmp(hx_jb_)) { hx.jb = hx_prev_; return failval; }    \
    hx.jb = &hx_jb_
#define HX_LEAVE() (hx.jb = hx_prev_)

// Load the embedded gfx950 code object and pick the device (idempotent).
void hx_init(int device);
hipFunction_t hx_fn(const char * name);
void hx_launch(const char * name, unsigned gx, unsigned gy, unsigned bx, size_t shmem,
               hipStream_t st, void * args);
// the same with a z dimension to the grid
void hx_launch3(const char * name, unsigned gx, unsigned gy, unsigned gz, unsigned bx, size_t shmem,
                hipStream_t st, void * args);
void * hx_malloc(size_t n);
