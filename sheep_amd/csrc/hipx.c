#include "hipx.h"

#include <stdarg.h>
#include <stdio.h>
#include <string.h>

hx_state hx = { .fail_after = -1, .device = -1 };

#define FN_CACHE 256
static struct { char name[64]; hipFunction_t f; } fn_cache[FN_CACHE];
static int fn_n;

// the gfx950 code objects, linked in from kernels.hsaco and ingest.hsaco
// (code_object.S)
extern const unsigned char sml_code_object[];
extern const unsigned char sml_ingest_object[];

void hx_fail(const char * what, hipError_t e) {
    snprintf(hx.err, sizeof hx.err, "%s: %s", what, hipGetErrorString(e));
    if (hx.jb) longjmp(*hx.jb, 1);
    fprintf(stderr, "sml-hip: unarmed failure: %s\n", hx.err);
}

void hx_failf(const char * fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(hx.err, sizeof hx.err, fmt, ap);
    va_end(ap);
    if (hx.jb) longjmp(*hx.jb, 1);
    fprintf(stderr, "sml-hip: unarmed failure: %s\n", hx.err);
}

void hx_init(int device) {
    if (hx.inited && hx.device == device) return;
    int n = 0;
    HX(hipGetDeviceCount(&n));
    if (device < 0 || device >= n) hx_failf("device %d of %d", device, n);
    HX(hipSetDevice(device));
    hipDeviceProp_t p;
    HX(hipGetDeviceProperties(&p, device));
    if (strncmp(p.gcnArchName, "gfx950", 6) != 0)
        hx_failf("device %d is %s; this library carries gfx950 code only", device, p.gcnArchName);
    if (hx.inited) {
        hx.inited = 0;            // a failure from here on leaves no stale module in use
        fn_n = 0;
        HX(hipModuleUnload(hx.mod));
        HX(hipModuleUnload(hx.mod_ingest));
    }
    HX(hipModuleLoadData(&hx.mod, sml_code_object));
    HX(hipModuleLoadData(&hx.mod_ingest, sml_ingest_object));
    fn_n = 0;
    hx.ncu = p.multiProcessorCount > 0 ? p.multiProcessorCount : 256;
    if (hx.kpart) {
        void * old = hx.kpart;
        hx.kpart = NULL;
        HX(hipFree(old));
    }
    hx.device = device;
    hx.inited = 1;
}


float * hx_kpart(void) {
    if (!hx.kpart) HX(hipMalloc((void **) &hx.kpart, (size_t) HX_KPART * sizeof(float)));
    return hx.kpart;
}

hipFunction_t hx_fn(const char * name) {
    for (int i = 0; i < fn_n; i++)
        if (strcmp(fn_cache[i].name, name) == 0) return fn_cache[i].f;
    hipFunction_t f;
    HX(hipModuleGetFunction(&f, strncmp(name, "sml_ing_", 8) == 0 ? hx.mod_ingest : hx.mod, name));
    if (fn_n < FN_CACHE) {
        snprintf(fn_cache[fn_n].name, sizeof fn_cache[fn_n].name, "%s", name);
        fn_cache[fn_n].f = f;
        fn_n++;
    }
    return f;
}

void hx_launch(const char * name, unsigned gx, unsigned gy, unsigned bx, size_t shmem,
               hipStream_t st, void * args) {
    hx_launch3(name, gx, gy, 1, bx, shmem, st, args);
}

void hx_launch3(const char * name, unsigned gx, unsigned gy, unsigned gz, unsigned bx, size_t shmem,
                hipStream_t st, void * args) {
    void * params[] = { args };
    HX(hipModuleLaunchKernel(hx_fn(name), gx, gy, gz, bx, 1, 1, (unsigned) shmem, st, params, NULL));
}

void * hx_malloc(size_t n) {
    void * p = NULL;
    HX(hipMalloc(&p, n ? n : 1));
    return p;
}
