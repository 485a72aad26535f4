// Ingest on the GPU: a GPTQ/AWQ tensor, or any float tensor, re-quantized
// into SSF FLAT planes and two-level fields at a width of its own, as the
// reference quantizer does for a tensor without calibration feedback
// (tooling/sml_unpack.py:66-118 then tooling/sml_quantize.py:426-651), with
// the quantizer's two searches as drop-ins for its fused C library
// (sml/sml-quant.c: sml_asym_grid, sml_field_search).
#include "ops.h"
#include "sml-quant.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define OP_BEGIN(fail) HX_ENTRY(fail); if (!hx.inited) hx_init(0)
#define ING_GMAX 256

static unsigned blocks(int64_t n) { return (unsigned) ((n + 255) / 256); }
static float g_last_ms;

// ------------------------------------------------------------ launches (device pointers)

static void ing_grid(hipStream_t st, const float * wp, int rows, int cols, int group, int nbits, int rem,
                     const float * wt, const float * facs, int ncand, int iters, int refit, float * out_l, float * out_s) {
    sml_king_grid a;
    memset(&a, 0, sizeof a);
    a.wp = wp; a.wt = wt; a.facs = facs; a.out_l = out_l; a.out_s = out_s;
    a.rows = rows; a.cols = cols; a.group = group; a.nbits = nbits; a.rem = rem;
    a.ncand = ncand; a.iters = iters; a.refit = refit;
    const char * k = group != 32 ? "sml_ing_grid" : wt ? "sml_ing_grid32w" : "sml_ing_grid32";
    hx_launch(k, blocks((int64_t) rows * (cols / group)), 1, 256, 0, st, &a);
}

static void ing_field(hipStream_t st, sml_king_field * a) {
    hx_launch("sml_ing_field", blocks((int64_t) a->rows * (a->cols / a->group)), 1, 256, 0, st, a);
}

static void check_search(int rows, int cols, int group, int nbits) {
    if (rows <= 0 || cols <= 0 || group <= 0 || group % 8 || group > ING_GMAX || cols % group)
        hx_failf("search over %dx%d in groups of %d: groups must be a multiple of 8 up to %d dividing the row",
                 rows, cols, group, ING_GMAX);
    if (nbits < 1 || nbits > 16) hx_failf("code width %d", nbits);
    if ((int64_t) rows * cols > ((int64_t) 1 << 40)) hx_failf("tensor too large");
}

// Every entry of the device index array idx [n] in [0, bound): the kernels
// index with it, so it is checked on the host first.
static void check_index(const int32_t * idx, int n, int bound, const char * what) {
    int32_t * h = malloc((size_t) n * sizeof(int32_t));
    if (!h) hx_failf("out of host memory");
    const hipError_t e = hipMemcpy(h, idx, (size_t) n * sizeof(int32_t), hipMemcpyDeviceToHost);
    int bad = -1;
    if (e == hipSuccess)
        for (int i = 0; i < n && bad < 0; i++) if (h[i] < 0 || h[i] >= bound) bad = i;
    const int32_t v = bad >= 0 ? h[bad] : 0;
    free(h);
    HX(e);
    if (bad >= 0) hx_failf("%s[%d] = %d is outside 0..%d", what, bad, v, bound - 1);
}

// ------------------------------------------------------------ the searches, host arrays (the reference's C ABI)

int sml_hip_asym_grid(const float * wp, int rows, int cols, int group, int nbits, int rem, const float * wt,
                      const float * facs, int ncand, int iters, int refit, float * out_l, float * out_s) {
    OP_BEGIN(-1);
    check_search(rows, cols, group, nbits);
    if (rem < 0 || rem >= nbits || ncand < 1 || ncand > 4096 || iters < 0) hx_failf("grid search arguments");
    const size_t nw = (size_t) rows * cols, ng = nw / (size_t) group;
    float * d = NULL;
    jmp_buf * outer = hx.jb;
    jmp_buf jb;
    if (setjmp(jb)) { hx.jb = outer; if (d) hipFree(d); longjmp(*outer, 1); }
    hx.jb = &jb;
    d = hx_malloc((nw + (wt ? (size_t) cols : 0) + (size_t) ncand + 2 * ng) * sizeof(float));
    float * dwp = d, * dwt = wt ? d + nw : NULL, * dfacs = d + nw + (wt ? (size_t) cols : 0), * dl = dfacs + ncand,
          * ds = dl + ng;
    HX(hipMemcpy(dwp, wp, nw * sizeof(float), hipMemcpyHostToDevice));
    if (wt) HX(hipMemcpy(dwt, wt, (size_t) cols * sizeof(float), hipMemcpyHostToDevice));
    HX(hipMemcpy(dfacs, facs, (size_t) ncand * sizeof(float), hipMemcpyHostToDevice));
    ing_grid(0, dwp, rows, cols, group, nbits, rem, dwt, dfacs, ncand, iters, refit, dl, ds);
    HX(hipMemcpy(out_l, dl, ng * sizeof(float), hipMemcpyDeviceToHost));
    HX(hipMemcpy(out_s, ds, ng * sizeof(float), hipMemcpyDeviceToHost));
    HX(hipFree(d));
    d = NULL;
    hx.jb = outer;
    HX_LEAVE();
    return 0;
}

int sml_hip_field_search(const float * w, int rows, int cols, int group, const float * dv, const float * dm,
                         int32_t * q8, int32_t * mq8, int nmax, int hi, int moff, int mmax, const float * wt,
                         int radius) {
    OP_BEGIN(-1);
    check_search(rows, cols, group, 1);
    if (radius < 0 || radius > 64 || hi < 1 || mmax < 0 || nmax < 0) hx_failf("field search arguments");
    const size_t nw = (size_t) rows * cols, ng = nw / (size_t) group;
    void * d = NULL;
    jmp_buf * outer = hx.jb;
    jmp_buf jb;
    if (setjmp(jb)) { hx.jb = outer; if (d) hipFree(d); longjmp(*outer, 1); }
    hx.jb = &jb;
    d = hx_malloc((nw + (wt ? (size_t) cols : 0) + 4 * ng) * 4);
    float * dw = d, * dwt = wt ? dw + nw : NULL, * ddv = dw + nw + (wt ? (size_t) cols : 0), * ddm = ddv + ng;
    int32_t * dq = (int32_t *) (ddm + ng), * dmq = dq + ng;
    HX(hipMemcpy(dw, w, nw * 4, hipMemcpyHostToDevice));
    if (wt) HX(hipMemcpy(dwt, wt, (size_t) cols * 4, hipMemcpyHostToDevice));
    HX(hipMemcpy(ddv, dv, ng * 4, hipMemcpyHostToDevice));
    HX(hipMemcpy(ddm, dm, ng * 4, hipMemcpyHostToDevice));
    HX(hipMemcpy(dq, q8, ng * 4, hipMemcpyHostToDevice));
    HX(hipMemcpy(dmq, mq8, ng * 4, hipMemcpyHostToDevice));
    sml_king_field a;
    memset(&a, 0, sizeof a);
    a.w = dw; a.dv = ddv; a.dm = ddm; a.q8 = dq; a.mq8 = dmq; a.wt = dwt;
    a.rows = rows; a.cols = cols; a.group = group; a.nmax = nmax; a.hi = hi; a.moff = moff; a.mmax = mmax;
    a.radius = radius;
    ing_field(0, &a);
    HX(hipMemcpy(q8, dq, ng * 4, hipMemcpyDeviceToHost));
    HX(hipMemcpy(mq8, dmq, ng * 4, hipMemcpyDeviceToHost));
    HX(hipFree(d));
    d = NULL;
    hx.jb = outer;
    HX_LEAVE();
    return 0;
}

// The reference library's own prototypes (sml/sml-quant.c:38-40,99-101), so
// its loader (tooling/sml_grid_c.py) can bind this library in its place.
// They return nothing, as there: a failure is printed and the outputs are
// filled with NaN (the grid) or left as they came in (the field search,
// whose inputs are a valid answer), never read as a result.
void sml_asym_grid(const float * wp, int rows, int cols, int group, int nbits, int rem, const float * wt,
                   const float * facs, int ncand, int iters, int refit, float * out_l, float * out_s) {
    if (sml_hip_asym_grid(wp, rows, cols, group, nbits, rem, wt, facs, ncand, iters, refit, out_l, out_s) != 0) {
        fprintf(stderr, "sml_asym_grid: %s\n", hx.err);
        if (rows > 0 && cols > 0 && group > 0)
            for (size_t i = 0; i < (size_t) rows * (size_t) (cols / group); i++) out_l[i] = out_s[i] = NAN;
    }
}

void sml_field_search(const float * w, int rows, int cols, int group, const float * dv, const float * dm,
                      int32_t * q8, int32_t * mq8, int nmax, int hi, int moff, int mmax, const float * wt, int radius) {
    if (sml_hip_field_search(w, rows, cols, group, dv, dm, q8, mq8, nmax, hi, moff, mmax, wt, radius) != 0)
        fprintf(stderr, "sml_field_search: %s (fields left as given)\n", hx.err);
}

// ------------------------------------------------------------ the whole tensor, device arrays

int sml_hip_unpack_dequant(const int32_t * qweight, const int32_t * qzeros, const uint16_t * scales,
                           const int32_t * g_idx, int rows, int cols, int bits, int group, int zero_add, int awq,
                           float * out) {
    OP_BEGIN(-1);
    if (rows <= 0 || cols <= 0 || group <= 0 || cols % group) hx_failf("unpack shape %dx%d, group %d", rows, cols, group);
    if (awq ? bits != 4 || rows % 8 : (bits != 2 && bits != 4 && bits != 8) || cols % (32 / bits) || rows % (32 / bits))
        hx_failf("%s %d-bit %dx%d: not a packing this unpacker reads", awq ? "AWQ" : "GPTQ", bits, rows, cols);
    if (!awq && !qzeros) hx_failf("GPTQ needs its zeros");
    if (awq && g_idx) hx_failf("AWQ has no g_idx");
    if (g_idx) check_index(g_idx, cols, cols / group, "g_idx");
    sml_king_dequant a;
    memset(&a, 0, sizeof a);
    a.qweight = (const uint32_t *) qweight; a.qzeros = (const uint32_t *) qzeros; a.scales = scales; a.g_idx = g_idx;
    a.out = out; a.rows = rows; a.cols = cols; a.bits = bits; a.group = group; a.zero_add = zero_add; a.awq = awq;
    hx_launch("sml_ing_dequant", blocks((int64_t) rows * cols), 1, 256, 0, 0, &a);
    HX_LEAVE();
    return 0;
}

int sml_hip_gguf_dequant(int type, const uint8_t * blocks, int rows, int cols, float * out) {
    OP_BEGIN(-1);
    const int qk = type == 14 ? 256 : 32;
    if (type != 8 && type != 2 && type != 14) hx_failf("ggml type %d: only Q8_0 (8), Q4_0 (2) and Q6_K (14) dequantize here", type);
    if (rows <= 0 || cols <= 0 || cols % qk) hx_failf("ggml type %d: %dx%d is not whole blocks of %d", type, rows, cols, qk);
    sml_king_gguf a;
    memset(&a, 0, sizeof a);
    a.blocks = blocks; a.out = out; a.rows = rows; a.cols = cols; a.type = type;
    hx_launch("sml_ing_gguf", (unsigned) (((int64_t) rows * cols + 255) / 256), 1, 256, 0, 0, &a);
    HX_LEAVE();
    return 0;
}

// The candidate range factors the quantizer tries (20: six over 0.6..0.85,
// fourteen over 0.88..1.04), numpy's linspace in double rounded to float,
// as tooling/sml_grid_c.py:41-42 builds them.
static __attribute__((noinline)) int grid_facs(int ncand, float * facs) {
    const int n1 = ncand / 3 > 2 ? ncand / 3 : 2, n2 = ncand - ncand / 3 > 2 ? ncand - ncand / 3 : 2;
    const double a[2] = { 0.6, 0.88 }, b[2] = { 0.85, 1.04 };
    const int cnt[2] = { n1, n2 };
    int k = 0;
    for (int s = 0; s < 2; s++) {
        const double step = (b[s] - a[s]) / (double) (cnt[s] - 1);
        for (int i = 0; i < cnt[s]; i++) {
            volatile double v = (double) i * step;     // two roundings, as numpy's y*step then += start
            double u = v + a[s];
            if (i == cnt[s] - 1) u = b[s];
            facs[k++] = (float) u;
        }
    }
    return k;
}

int sml_hip_requant(const float * w, int rows, int cols, int nbits, const int32_t * perm_in, const float * wt,
                    int radius, uint8_t * const planes[3], uint16_t * sd, uint8_t * sq, uint16_t * md, uint8_t * mq,
                    int32_t * perm, uint8_t * codes) {
    float facs[64];
    const int nf = grid_facs(20, facs);
    OP_BEGIN(-1);
    if (rows <= 0 || cols <= 0 || cols % 256) hx_failf("re-quantization of %dx%d: the row must be whole superblocks of 256", rows, cols);
    if (nbits < 2 || nbits > 8) hx_failf("SSF width %d (2..8)", nbits);
    if (radius < 0 || radius > 64) hx_failf("field search radius %d", radius);
    int pb[SSF_MAX_PLANES];
    const int np = ssf_flat_planes(nbits, pb);
    for (int i = 0; i < np; i++) if (!planes[i]) hx_failf("plane %d of width %d missing", i, nbits);
    const size_t nw = (size_t) rows * cols, ng = nw / 32;
    const int nsb = cols / 256;
    void * d = NULL;
    hipEvent_t e0 = NULL, e1 = NULL;
    jmp_buf * outer = hx.jb;
    jmp_buf jb;
    if (setjmp(jb)) {
        hx.jb = outer;
        if (d) hipFree(d);
        if (e0) hipEventDestroy(e0);
        if (e1) hipEventDestroy(e1);
        longjmp(*outer, 1);
    }
    hx.jb = &jb;
    // scratch: wp, mins, steps, eff_s, eff_m, keys, factors, column-max partials, rank counts
    const size_t bytes = nw * 4 + 4 * ng * 4 + (size_t) cols * 4 + 64 * 4 + (size_t) cols * 128 * 4 + (size_t) cols * 4;
    d = hx_malloc(bytes);
    float * wp = d, * mins = wp + nw, * steps = mins + ng, * es = steps + ng, * em = es + ng, * key = em + ng,
          * dfacs = key + cols, * part = dfacs + 64;
    int32_t * cnt = (int32_t *) (part + (size_t) cols * 128);
    HX(hipEventCreate(&e0));
    HX(hipEventCreate(&e1));
    HX(hipMemcpy(dfacs, facs, (size_t) nf * 4, hipMemcpyHostToDevice));
    HX(hipEventRecord(e0, 0));
    if (perm_in) {
        check_index(perm_in, cols, cols, "perm");
        HX(hipMemcpyAsync(perm, perm_in, (size_t) cols * 4, hipMemcpyDeviceToDevice, 0));
    }
    else {
        const int chunk = rows > 64 * 128 ? (rows + 127) / 128 : 64, nchunk = (rows + chunk - 1) / chunk;
        sml_king_colmax c = { w, part, rows, cols, chunk };
        hx_launch("sml_ing_colmax", blocks(cols), (unsigned) nchunk, 256, 0, 0, &c);
        sml_king_colfold cf = { part, key, cols, nchunk };
        hx_launch("sml_ing_colfold", blocks(cols), 1, 256, 0, 0, &cf);
        const int slice = 1024, nslice = (cols + slice - 1) / slice;
        HX(hipMemsetAsync(cnt, 0, (size_t) cols * 4, 0));
        sml_king_rank k = { key, cnt, perm, cols, slice };
        hx_launch("sml_ing_rank", blocks(cols), (unsigned) nslice, 256, 0, 0, &k);
        hx_launch("sml_ing_scatter", blocks(cols), 1, 256, 0, 0, &k);
    }
    sml_king_gather gth = { w, perm, wp, rows, cols };
    hx_launch("sml_ing_gather", blocks((int64_t) nw), 1, 256, 0, 0, &gth);
    ing_grid(0, wp, rows, cols, 32, nbits, 0, wt, dfacs, nf, 3, 1, mins, steps);
    sml_king_two t2;
    memset(&t2, 0, sizeof t2);
    t2.v = steps; t2.d16 = sd; t2.q8 = sq; t2.eff = es; t2.rows = rows; t2.ng = cols / 32; t2.gps = 8; t2.is_signed = 0;
    hx_launch("sml_ing_two", blocks((int64_t) rows * nsb), 1, 256, 0, 0, &t2);
    t2.v = mins; t2.d16 = md; t2.q8 = mq; t2.eff = em; t2.is_signed = 1;
    hx_launch("sml_ing_two", blocks((int64_t) rows * nsb), 1, 256, 0, 0, &t2);
    if (radius) {
        sml_king_field f;
        memset(&f, 0, sizeof f);
        f.w = wp; f.d16 = sd; f.md16 = md; f.gps = 8; f.sq = sq; f.mq = mq; f.eff_s = es; f.eff_m = em; f.wt = wt;
        f.rows = rows; f.cols = cols; f.group = 32; f.nmax = (1 << nbits) - 1; f.hi = 255; f.moff = 127; f.mmax = 254;
        f.radius = radius;
        ing_field(0, &f);
    }
    sml_king_pack pk;
    memset(&pk, 0, sizeof pk);
    pk.wp = wp; pk.eff_s = es; pk.eff_m = em; pk.codes = codes; pk.rows = rows; pk.cols = cols; pk.nbits = nbits;
    for (int i = 0; i < np; i++) pk.plane[i] = planes[i];
    hx_launch("sml_ing_pack", blocks((int64_t) rows * (cols / 128)), 1, 256, 0, 0, &pk);
    HX(hipEventRecord(e1, 0));
    HX(hipEventSynchronize(e1));
    HX(hipEventElapsedTime(&g_last_ms, e0, e1));
    HX(hipEventDestroy(e0)); e0 = NULL;
    HX(hipEventDestroy(e1)); e1 = NULL;
    HX(hipFree(d));
    d = NULL;
    (void) nsb;
    hx.jb = outer;
    HX_LEAVE();
    return 0;
}

float sml_hip_requant_last_ms(void) { return g_last_ms; }

// A re-quantized tensor (device arrays, as sml_hip_requant leaves them) as a
// GEMV-ready matrix: fetched to the host and uploaded in the file's layout.
sml_hip_mat * sml_hip_mat_from_requant(uint8_t * const planes[3], const uint16_t * sd, const uint8_t * sq,
                                       const uint16_t * md, const uint8_t * mq, int rows, int cols, int nbits) {
    OP_BEGIN(NULL);
    if (rows <= 0 || cols <= 0 || cols % 256 || nbits < 2 || nbits > 8) hx_failf("re-quantized matrix %dx%d width %d", rows, cols, nbits);
    int pb[SSF_MAX_PLANES];
    const int np = ssf_flat_planes(nbits, pb);
    const size_t R = (size_t) rows, ng = (size_t) cols / 32, ns = (size_t) cols / 256;
    size_t psz[SSF_MAX_PLANES], tot = 0;
    for (int i = 0; i < np; i++) { psz[i] = R * ssf_plane_row_bytes(pb[i], cols); tot += psz[i]; }
    tot += 2 * R * ng + 4 * R * ns;
    uint8_t * h = malloc(tot);
    if (!h) hx_failf("out of host memory");
    sml_hip_mat * m = NULL;
    jmp_buf * outer = hx.jb;
    jmp_buf jb;
    if (setjmp(jb)) { hx.jb = outer; free(h); longjmp(*outer, 1); }
    hx.jb = &jb;
    const uint8_t * hp[4] = { NULL, NULL, NULL, NULL };
    uint8_t * cur = h;
    for (int i = 0; i < np; i++) {
        HX(hipMemcpy(cur, planes[i], psz[i], hipMemcpyDeviceToHost));
        hp[i] = cur;
        cur += psz[i];
    }
    uint8_t * hsq = cur, * hmq = hsq + R * ng;
    uint16_t * hsd = (uint16_t *) (hmq + R * ng), * hmd = hsd + R * ns;
    HX(hipMemcpy(hsq, sq, R * ng, hipMemcpyDeviceToHost));
    HX(hipMemcpy(hmq, mq, R * ng, hipMemcpyDeviceToHost));
    HX(hipMemcpy(hsd, sd, R * ns * 2, hipMemcpyDeviceToHost));
    HX(hipMemcpy(hmd, md, R * ns * 2, hipMemcpyDeviceToHost));
    m = mat_upload(hp, hsd, hsq, hmd, hmq, rows, cols, nbits, 0, 0);
    hx.jb = outer;
    free(h);
    HX_LEAVE();
    return m;
}

int sml_hip_ssf_write_quant(const char * path, const char * name, int rows, int cols, int nbits,
                            const uint8_t * const planes[3], const uint16_t * sd, const uint8_t * sq,
                            const uint16_t * md, const uint8_t * mq, const int32_t * perm) {
    char why[256] = "";
    const uint8_t * pl[SSF_MAX_PLANES] = { planes[0], planes[1], planes[2], NULL };
    if (!ssf_write_quant(path, name, rows, cols, nbits, pl, sd, sq, md, mq, perm, why, sizeof why)) {
        snprintf(hx.err, sizeof hx.err, "%s", why);
        return -1;
    }
    return 0;
}
