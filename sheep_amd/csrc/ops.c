// Kernel-level C ABI (include/sml-hip.h): matrix upload and single launches of
// the gfx950 kernels, used by the decode engine, the tests and the benches.
#include "ops.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "sml-hip.h"
#include "ssf.h"

static size_t al256(size_t x) { return (x + 255u) & ~(size_t) 255u; }

int sml_hip_init(int device, char * why, int nwhy) {
    HX_ENTRY(0);
    hx_init(device);
    HX_LEAVE();
    return 1;
}

// The entry points below report failure through their return value; init is
// implicit (device 0) the first time any of them runs.
#define OP_BEGIN(fail) HX_ENTRY(fail); if (!hx.inited) hx_init(0)

const char * sml_hip_last_error(void) { return hx.err; }
void sml_hip_fail_after(long n) { hx.fail_after = n; }

void * sml_hip_malloc(size_t n) { OP_BEGIN(NULL); void * p = hx_malloc(n); HX_LEAVE(); return p; }
int sml_hip_free(void * p) { OP_BEGIN(-1); if (p) HX(hipFree(p)); HX_LEAVE(); return 0; }
int sml_hip_h2d(void * d, const void * s, size_t n) { OP_BEGIN(-1); HX(hipMemcpy(d, s, n, hipMemcpyHostToDevice)); HX_LEAVE(); return 0; }
int sml_hip_d2h(void * d, const void * s, size_t n) { OP_BEGIN(-1); HX(hipMemcpy(d, s, n, hipMemcpyDeviceToHost)); HX_LEAVE(); return 0; }
int sml_hip_memset(void * p, int v, size_t n) { OP_BEGIN(-1); HX(hipMemset(p, v, n)); HX_LEAVE(); return 0; }
int sml_hip_sync(void) { OP_BEGIN(-1); HX(hipDeviceSynchronize()); HX_LEAVE(); return 0; }

// ------------------------------------------------------------ matrices

// 6-bit group field g of one row (four values in three bytes, sml/sml-kernel.h:79-86)
static uint32_t field6(const uint8_t * row, size_t g) {
    const uint8_t * p = row + (g >> 2) * 3;
    const uint32_t b0 = p[0], b1 = p[1], b2 = p[2];
    switch (g & 3) {
    case 0: return b0 & 63u;
    case 1: return ((b0 >> 6) | (b1 << 2)) & 63u;
    case 2: return ((b1 >> 4) | (b2 << 4)) & 63u;
    default: return (b2 >> 2) & 63u;
    }
}

sml_hip_mat * mat_upload(const uint8_t * const planes[4], const uint16_t * sd, const uint8_t * sq,
                         const uint16_t * md, const uint8_t * mq, int rows, int cols, int nbits,
                         int scale6, int minneg) {
    if (rows <= 0 || cols <= 0 || cols % 128 || nbits < 2 || nbits > 8)
        hx_failf("matrix %dx%d width %d: shape or width not supported", rows, cols, nbits);
    int pb[SSF_MAX_PLANES];
    const int np = ssf_flat_planes(nbits, pb);
    const size_t R = (size_t) rows, ng = (size_t) cols / 32, ns = (size_t) SSF_NSUPER(cols);
    size_t off[5], sz[5], tot = 0;
    for (int i = 0; i < 3; i++) sz[i] = i < np ? R * ssf_plane_row_bytes(pb[i], cols) : 0;
    sz[3] = R * ng * 2;          // (sq, mq) per group
    sz[4] = R * ns * 4;          // (sd, md) per superblock
    for (int i = 0; i < 5; i++) { off[i] = tot; tot += al256(sz[i]); }
    // the fields interleaved on the host: 8-bit (or widened 6-bit) values, min bias 127
    uint8_t * fq = malloc(sz[3]);
    uint16_t * fd = malloc(sz[4]);
    if (!fq || !fd) { free(fq); free(fd); hx_failf("out of host memory"); }
    const size_t grow = scale6 ? (ng / 4) * 3 : ng;
    const uint32_t madd = scale6 ? (minneg ? 64u : 96u) : 0u;   // (v - 31) = (v + 96) - 127; (v - 63) = (v + 64) - 127
    for (size_t r = 0; r < R; r++) {
        for (size_t g = 0; g < ng; g++) {
            const uint32_t q = scale6 ? field6(sq + r * grow, g) : sq[r * grow + g];
            const uint32_t m = mq ? (scale6 ? field6(mq + r * grow, g) + madd : mq[r * grow + g]) : 127u;
            fq[(r * ng + g) * 2] = (uint8_t) q;
            fq[(r * ng + g) * 2 + 1] = (uint8_t) m;
        }
        for (size_t k = 0; k < ns; k++) {
            fd[(r * ns + k) * 2] = sd[r * ns + k];
            fd[(r * ns + k) * 2 + 1] = md ? md[r * ns + k] : 0;
        }
    }
    sml_hip_mat * m = calloc(1, sizeof *m);
    if (!m) { free(fq); free(fd); hx_failf("out of host memory"); }
    jmp_buf * outer = hx.jb;
    jmp_buf jb;
    if (setjmp(jb)) {
        hx.jb = outer;
        free(fq); free(fd);
        if (m->mem) hipFree(m->mem);
        free(m);
        longjmp(*outer, 1);
    }
    hx.jb = &jb;
    m->mem = hx_malloc(tot);
    uint8_t * base = (uint8_t *) m->mem;
    for (int i = 0; i < np; i++) {
        HX(hipMemcpy(base + off[i], planes[i], sz[i], hipMemcpyHostToDevice));
        m->k.plane[i] = base + off[i];
    }
    HX(hipMemcpy(base + off[3], fq, sz[3], hipMemcpyHostToDevice));
    HX(hipMemcpy(base + off[4], fd, sz[4], hipMemcpyHostToDevice));
    hx.jb = outer;
    free(fq);
    free(fd);
    m->k.sqmq = base + off[3];
    m->k.sdmd = (const uint16_t *) (base + off[4]);
    m->k.rows = rows;
    m->nbits = nbits;
    m->cols = cols;
    // the bytes a GEMV streams: the file's planes and fields at 8 bits
    m->bytes = sz[0] + sz[1] + sz[2] + R * ng * (mq ? 2 : 1) + R * ns * (md ? 4 : 2);
    return m;
}

sml_hip_mat * sml_hip_mat_upload(const uint8_t * const planes[4], const uint16_t * sd, const uint8_t * sq,
                                 const uint16_t * md, const uint8_t * mq,
                                 int rows, int cols, int nbits, int scale6, int minneg) {
    OP_BEGIN(NULL);
    sml_hip_mat * m = mat_upload(planes, sd, sq, md, mq, rows, cols, nbits, scale6, minneg);
    HX_LEAVE();
    return m;
}

sml_hip_mat * mat_from_record(const ssf_file * f, const ssf_record * r) {
    if (r->kind != SSF_KIND_QUANT || r->layout != SSF_LAYOUT_FLAT)
        hx_failf("tensor %.64s is not a FLAT quantized record", r->name);
    const uint8_t * planes[4] = { 0 };
    for (int i = 0; i < 4; i++) planes[i] = r->plane_off[i] ? (const uint8_t *) ssf_at(f, r->plane_off[i]) : NULL;
    const int six = (f->hdr->flags & SSF_FLAG_SCALE6) != 0, neg = (f->hdr->flags & SSF_FLAG_MINNEG) != 0;
    return mat_upload(planes, (const uint16_t *) ssf_at(f, r->sd_off), (const uint8_t *) ssf_at(f, r->sq_off),
                      r->mq_bytes ? (const uint16_t *) ssf_at(f, r->md_off) : NULL,
                      r->mq_bytes ? (const uint8_t *) ssf_at(f, r->mq_off) : NULL,
                      (int) r->rows, (int) r->cols, (int) r->nbits, six, neg);
}

sml_hip_mat * sml_hip_mat_from_file(const char * path, const char * name) {
    OP_BEGIN(NULL);
    ssf_file f;
    char why[256];
    if (!ssf_open(&f, path, why, sizeof why)) hx_failf("%s", why);
    const ssf_record * r = ssf_find(&f, name);
    if (!r) { ssf_close(&f); hx_failf("%s has no tensor %s", path, name); }
    jmp_buf * outer = hx.jb;
    jmp_buf jb;
    if (setjmp(jb)) { ssf_close(&f); hx.jb = outer; longjmp(*outer, 1); }
    hx.jb = &jb;
    sml_hip_mat * m = mat_from_record(&f, r);
    hx.jb = outer;
    ssf_close(&f);
    HX_LEAVE();
    return m;
}

void mat_free(sml_hip_mat * m) {
    if (!m) return;
    if (m->mem) HX(hipFree(m->mem));
    free(m);
}

void sml_hip_mat_free(sml_hip_mat * m) {
    HX_ENTRY();
    mat_free(m);
    HX_LEAVE();
}

int sml_hip_mat_info(const sml_hip_mat * m, int * rows, int * cols, int * nbits) {
    if (!m) return -1;
    if (rows) *rows = m->k.rows;
    if (cols) *cols = m->cols;
    if (nbits) *nbits = m->nbits;
    return 0;
}

size_t sml_hip_mat_bytes(const sml_hip_mat * m) { return m ? m->bytes : 0; }

// ------------------------------------------------------------ launches

void op_normq(hipStream_t st, float * x, const float * resid, const float * w, float eps, int n,
              int nout, const int32_t * const * perm, int8_t * const * q, float * const * scale,
              int32_t * const * sums, float * normed, int per256) {
    if (n <= 0 || n % 32 || n > 16384) hx_failf("normq width %d not supported", n);
    sml_knormq a;
    memset(&a, 0, sizeof a);
    a.x = x; a.resid = resid; a.norm_w = w; a.eps = eps; a.n = n; a.nout = nout;
    for (int i = 0; i < nout; i++) { a.perm[i] = perm[i]; a.q[i] = q[i]; a.scale[i] = scale[i]; a.sums[i] = sums[i]; }
    a.normed = normed; a.per256 = per256;
    if (!resid && !normed && !per256) {
        sml_knormq2 b;
        memset(&b, 0, sizeof b);
        b.x = x; b.norm_w = w; b.eps = eps; b.n = n; b.nout = nout;
        for (int i = 0; i < nout; i++) { b.perm[i] = perm[i]; b.q[i] = q[i]; b.scale[i] = scale[i]; b.sums[i] = sums[i]; }
        hx_launch("sml_normq2", (unsigned) ((n + 255) / 256), 1, 256, 0, st, &b);
        return;
    }
    hx_launch("sml_normq", 1, 1, 1024, (size_t) n * 4, st, &a);
}

int sml_hip_normq(float * x, const float * resid, const float * w, float eps, int n,
                  const int32_t * perm, int8_t * q, float * scale, int32_t * sums, int per256) {
    OP_BEGIN(-1);
    op_normq(0, x, resid, w, eps, n, 1, &perm, &q, &scale, &sums, NULL, per256);
    HX_LEAVE();
    return 0;
}

static int env_int(const char * name, int dflt) {
    const char * e = getenv(name);
    return e && *e ? atoi(e) : dflt;
}

// Shape of a GEMV launch: NI chunks per lane (enough that one pass covers a
// row: ng <= 64*NI, at most 8), RB rows per wave (more rows per wave for tall
// matrices, so ~2048+ waves carry the whole matrix at once while the loads a
// lane holds stay within RB*NI <= 16). SML_GEMV_RB / SML_GEMV_NI override.
static void pick_shape(int rows, int cols, int swiglu, int * rb, int * ni) {
    const int ng = cols / 32;
    int i = 1;
    while (i < 8 && 64 * i < ng) i *= 2;
    int r = 1;
    while (r < 4 && rows / (2 * r) >= 2048 && 2 * r * i <= 16) r *= 2;
    if (swiglu) r = r < 2 ? 2 : r;
    if (r == 4 && i == 8) i = 4;
    if (r == 1 && i == 1) i = 2;
    const int fr = env_int("SML_GEMV_RB", 0), fi = env_int("SML_GEMV_NI", 0);
    if (fr == 1 || fr == 2 || fr == 4) r = swiglu && fr == 1 ? 2 : fr;
    if (fi == 1 || fi == 2 || fi == 4 || fi == 8) i = fi;
    if (r == 1 && i == 1) i = 2;
    if (r == 4 && i == 8) i = 4;
    *rb = r;
    *ni = i;
}

void op_gemv(hipStream_t st, const sml_hip_mat * const * mats, int nm, int epi, const int8_t * q,
             const float * scale, const int32_t * sums, float * const * y, const float * const * bias,
             const float * resid) {
    if (nm < 1 || nm > SML_MAX_MATS) hx_failf("gemv of %d matrices", nm);
    sml_kgemv a;
    memset(&a, 0, sizeof a);
    const int nb = mats[0]->nbits, cols = mats[0]->cols;
    int tot = 0;
    for (int i = 0; i < nm; i++) {
        if (mats[i]->nbits != nb || mats[i]->cols != cols) hx_failf("gemv group mixes shapes or widths");
        a.m[i] = mats[i]->k;
        a.m[i].y = y[i];
        a.m[i].bias = bias ? bias[i] : NULL;
        a.m[i].row_begin = tot;
        tot += mats[i]->k.rows;
    }
    if (epi == SML_EPI_SWIGLU && (nm != 2 || mats[0]->k.rows != mats[1]->k.rows))
        hx_failf("swiglu needs gate and up of one shape");
    a.nmat = nm; a.cols = cols; a.epi = epi;
    a.q = q; a.scale = scale; a.sums = sums; a.resid = resid;
    a.total_rows = epi == SML_EPI_SWIGLU ? mats[0]->k.rows : tot;
    int rb, ni;
    pick_shape(a.total_rows, cols, epi == SML_EPI_SWIGLU, &rb, &ni);
    const int rows_per_wave = epi == SML_EPI_SWIGLU ? rb / 2 : rb;
    const int waves = (a.total_rows + rows_per_wave - 1) / rows_per_wave;
    const int wgs = (waves + 3) / 4;
    const int wg = env_int("SML_GEMV_WG", 256), nt = env_int("SML_GEMV_NT", 1);
    char name[48];
    if (nb == 4 && (wg != 256 || !nt) && (wg == 256 || wg == 512 || wg == 1024)) {
        snprintf(name, sizeof name, "sml_gemv_q%d_r%d_i%d_w%d_t%d", nb, rb, ni, wg, nt ? 1 : 0);
        const int wpg = wg / 64;
        hx_launch(name, (unsigned) ((waves + wpg - 1) / wpg), 1, (unsigned) wg,
                  (size_t) cols + 8u * (size_t) (cols / 32), st, &a);
        return;
    }
    snprintf(name, sizeof name, "sml_gemv_q%d_r%d_i%d", nb, rb, ni);
    hx_launch(name, (unsigned) wgs, 1, 256, (size_t) cols + 8u * (size_t) (cols / 32), st, &a);
}

int sml_hip_matvec(const sml_hip_mat * m, const int8_t * q, const float * scale, const int32_t * sums, float * y) {
    OP_BEGIN(-1);
    op_gemv(0, &m, 1, SML_EPI_STORE, q, scale, sums, &y, NULL, NULL);
    HX_LEAVE();
    return 0;
}

int sml_hip_matvec_swiglu(const sml_hip_mat * gate, const sml_hip_mat * up, const int8_t * q,
                          const float * scale, const int32_t * sums, float * h) {
    OP_BEGIN(-1);
    const sml_hip_mat * ms[2] = { gate, up };
    float * ys[2] = { h, h };
    op_gemv(0, ms, 2, SML_EPI_SWIGLU, q, scale, sums, ys, NULL, NULL);
    HX_LEAVE();
    return 0;
}

int sml_hip_time_matvec(const sml_hip_mat * const * mats, int ncopy, const int8_t * q, const float * scale,
                        const int32_t * sums, float * y, int iters, float * ms_total) {
    OP_BEGIN(-1);
    hipEvent_t e0, e1;
    HX(hipEventCreate(&e0));
    HX(hipEventCreate(&e1));
    HX(hipEventRecord(e0, 0));
    for (int i = 0; i < iters; i++) op_gemv(0, &mats[i % ncopy], 1, SML_EPI_STORE, q, scale, sums, &y, NULL, NULL);
    HX(hipEventRecord(e1, 0));
    HX(hipEventSynchronize(e1));
    HX(hipEventElapsedTime(ms_total, e0, e1));
    HX(hipEventDestroy(e0));
    HX(hipEventDestroy(e1));
    HX_LEAVE();
    return 0;
}

int sml_hip_unpack(const sml_hip_mat * m, int row0, int nrows, uint8_t * out) {
    OP_BEGIN(-1);
    if (row0 < 0 || nrows < 0 || row0 + nrows > m->k.rows) hx_failf("unpack rows out of range");
    sml_kunpack a;
    memset(&a, 0, sizeof a);
    a.m = m->k; a.nbits = m->nbits; a.cols = m->cols; a.row0 = row0; a.nrows = nrows; a.out = out;
    const long work = (long) nrows * (m->cols / 32);
    if (work > 0) hx_launch("sml_unpack", (unsigned) ((work + 255) / 256), 1, 256, 0, 0, &a);
    HX_LEAVE();
    return 0;
}

void op_embed(hipStream_t st, const sml_hip_mat * m, const int32_t * tok, const int32_t * pos,
              const int32_t * perm, float * x) {
    sml_kembed a;
    memset(&a, 0, sizeof a);
    a.m = m->k; a.nbits = m->nbits; a.cols = m->cols; a.tok = tok; a.pos = pos; a.perm = perm; a.x = x;
    hx_launch("sml_embed", (unsigned) ((m->cols / 32 + 63) / 64), 1, 64, 0, st, &a);
}

int sml_hip_embed(const sml_hip_mat * m, const int32_t * tok, const int32_t * perm, float * x) {
    OP_BEGIN(-1);
    op_embed(0, m, tok, NULL, perm, x);
    HX_LEAVE();
    return 0;
}

#define ATTN_CHUNK 128

size_t sml_hip_attn_part_floats(int n_head, int hd, int n_ctx) {
    const int ns = (n_ctx + ATTN_CHUNK - 1) / ATTN_CHUNK;
    return (size_t) n_head * ns * (size_t) (hd + 2);
}

void op_attention(hipStream_t st, const float * q, const float * k, const float * v, uint16_t * kc, uint16_t * vc,
                  const float * cos_t, const float * sin_t, const int32_t * pos, int n_head, int n_kv,
                  int hd, int n_ctx, float * part, float * out, int8_t * q_out, float * s_out,
                  int32_t * u_out) {
    if (hd != 128 || n_kv <= 0 || n_head % n_kv || n_head / n_kv > 8)
        hx_failf("attention shape (heads %d/%d, head_dim %d) not supported", n_head, n_kv, hd);
    const int ns = (n_ctx + ATTN_CHUNK - 1) / ATTN_CHUNK;
    sml_kattn a;
    memset(&a, 0, sizeof a);
    a.q = q; a.k = k; a.v = v; a.kcache = kc; a.vcache = vc; a.cos_t = cos_t; a.sin_t = sin_t; a.pos = pos;
    a.part = part; a.out = out; a.q_out = q_out; a.s_out = s_out; a.u_out = u_out;
    a.n_head = n_head; a.n_kv = n_kv; a.nsplit = ns;
    a.inv = 1.0f / __builtin_sqrtf((float) hd);
    hx_launch("sml_attn", (unsigned) ns, (unsigned) n_kv, 256, 0, st, &a);
    hx_launch("sml_attn_merge", (unsigned) n_head, 1, (unsigned) hd, 0, st, &a);
}

int sml_hip_attention(float * q, const float * k, const float * v, uint16_t * kcache, uint16_t * vcache,
                      const float * cos_t, const float * sin_t, const int32_t * pos,
                      int n_head, int n_kv, int hd, int n_ctx, float * part, float * out) {
    OP_BEGIN(-1);
    op_attention(0, q, k, v, kcache, vcache, cos_t, sin_t, pos, n_head, n_kv, hd, n_ctx, part, out,
                 NULL, NULL, NULL);
    HX_LEAVE();
    return 0;
}

void op_argmax(hipStream_t st, const float * logits, int n, int32_t * tok, int32_t * pos, int32_t * hist,
               int hist_n) {
    sml_kargmax a;
    memset(&a, 0, sizeof a);
    a.logits = logits; a.n = n; a.tok = tok; a.pos = pos; a.hist = hist; a.hist_n = hist_n;
    hx_launch("sml_argmax", 1, 1, 1024, 0, st, &a);
}

void op_advance(hipStream_t st, int32_t * pos) {
    sml_kadvance a = { pos };
    hx_launch("sml_advance", 1, 1, 64, 0, st, &a);
}

void op_silu_mul(hipStream_t st, float * g, const float * u, int n) {
    sml_ksilu a = { g, u, n };
    hx_launch("sml_silu_mul", (unsigned) ((n + 255) / 256), 1, 256, 0, st, &a);
}

int sml_hip_argmax(const float * logits, int n, int32_t * tok) {
    OP_BEGIN(-1);
    op_argmax(0, logits, n, tok, NULL, NULL, 0);
    HX_LEAVE();
    return 0;
}

int sml_hip_copy(void * dst, const void * src, size_t bytes) {
    OP_BEGIN(-1);
    if (!dst || !src || bytes % 16) hx_failf("copy arguments");
    sml_kcopy a;
    a.src = src; a.dst = dst; a.bytes = bytes;
    uint64_t words = bytes / 16, grid = (words + 255) / 256;
    if (grid > 8192) grid = 8192;
    if (grid < 1) grid = 1;
    hx_launch("sml_copy_stream", (unsigned) grid, 1, 256, 0, 0, &a);
    HX(hipStreamSynchronize(0));
    HX_LEAVE();
    return 0;
}

int sml_hip_time_read(const void * const * bufs, int nbuf, size_t bytes, int grid, int iters, float * ms_total) {
    OP_BEGIN(-1);
    const int pattern = getenv("SML_READ_PATTERN") ? atoi(getenv("SML_READ_PATTERN")) : 0;
    if (nbuf < 1 || bytes % 16 || grid < 1) hx_failf("read calibration arguments");
    uint32_t * sink = hx_malloc((size_t) grid * 16);
    hipEvent_t e0, e1;
    HX(hipEventCreate(&e0));
    HX(hipEventCreate(&e1));
    sml_kread a;
    a.bytes = bytes; a.sink = sink; a.pattern = pattern;
    a.src = bufs[0];
    hx_launch("sml_read_stream", (unsigned) grid, 1, 256, 0, 0, &a);
    HX(hipEventRecord(e0, 0));
    for (int i = 0; i < iters; i++) {
        a.src = bufs[i % nbuf];
        hx_launch("sml_read_stream", (unsigned) grid, 1, 256, 0, 0, &a);
    }
    HX(hipEventRecord(e1, 0));
    HX(hipEventSynchronize(e1));
    HX(hipEventElapsedTime(ms_total, e0, e1));
    HX(hipEventDestroy(e0));
    HX(hipEventDestroy(e1));
    HX(hipFree(sink));
    HX_LEAVE();
    return 0;
}
