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

sml_hip_mat * mat_upload(const uint8_t * const planes[4], const uint16_t * sd, const uint8_t * sq,
                         const uint16_t * md, const uint8_t * mq, int rows, int cols, int nbits,
                         int scale6, int minneg) {
    if (rows <= 0 || cols <= 0 || cols % 128 || nbits < 2 || nbits > 8)
        hx_failf("matrix %dx%d width %d: shape or width not supported", rows, cols, nbits);
    int pb[SSF_MAX_PLANES];
    const int np = ssf_flat_planes(nbits, pb);
    const size_t R = (size_t) rows, ng = (size_t) cols / 32, ns = (size_t) SSF_NSUPER(cols);
    size_t off[8], sz[8];
    size_t tot = 0;
    for (int i = 0; i < np; i++) { sz[i] = R * ssf_plane_row_bytes(pb[i], cols); }
    sz[3] = R * ns * 2; sz[4] = R * ng; sz[5] = md ? R * ns * 2 : 0; sz[6] = mq ? R * ng : 0;
    for (int i = np; i < 3; i++) sz[i] = 0;
    for (int i = 0; i < 7; i++) { off[i] = tot; tot += al256(sz[i]); }
    sml_hip_mat * m = calloc(1, sizeof *m);
    if (!m) hx_failf("out of host memory");
    m->mem = hx_malloc(tot);
    uint8_t * base = (uint8_t *) m->mem;
    m->nbits = nbits;
    m->cols = cols;
    m->bytes = 0;
    for (int i = 0; i < 7; i++) m->bytes += sz[i];
    for (int i = 0; i < np; i++) {
        HX(hipMemcpy(base + off[i], planes[i], sz[i], hipMemcpyHostToDevice));
        m->k.plane[i] = base + off[i];
    }
    HX(hipMemcpy(base + off[3], sd, sz[3], hipMemcpyHostToDevice));
    if (md) HX(hipMemcpy(base + off[5], md, sz[5], hipMemcpyHostToDevice));
    if (!scale6) {
        HX(hipMemcpy(base + off[4], sq, sz[4], hipMemcpyHostToDevice));
        if (mq) HX(hipMemcpy(base + off[6], mq, sz[6], hipMemcpyHostToDevice));
    } else {
        // widen 6-bit fields (four in three bytes, sml/sml-kernel.h:79-86) to bytes; the
        // min moves to the 8-bit bias: (v - 31) = (v + 96) - 127, negative-only (v - 63) = (v + 64) - 127
        uint8_t * w = malloc(R * ng);
        if (!w) hx_failf("out of host memory");
        for (int pass = 0; pass < (mq ? 2 : 1); pass++) {
            const uint8_t * src = pass ? mq : sq;
            const int add = pass ? (minneg ? 64 : 96) : 0;
            for (size_t r = 0; r < R; r++)
                for (size_t g = 0; g < ng; g++) {
                    const uint8_t * p = src + r * (ng / 4) * 3 + (g >> 2) * 3;
                    const uint32_t b0 = p[0], b1 = p[1], b2 = p[2];
                    uint32_t v;
                    switch (g & 3) {
                    case 0: v = b0 & 63u; break;
                    case 1: v = ((b0 >> 6) | (b1 << 2)) & 63u; break;
                    case 2: v = ((b1 >> 4) | (b2 << 4)) & 63u; break;
                    default: v = (b2 >> 2) & 63u; break;
                    }
                    w[r * ng + g] = (uint8_t) (v + (uint32_t) add);
                }
            HX(hipMemcpy(base + off[pass ? 6 : 4], w, R * ng, hipMemcpyHostToDevice));
        }
        free(w);
    }
    m->k.sd = (const uint16_t *) (base + off[3]);
    m->k.sq = base + off[4];
    m->k.md = md ? (const uint16_t *) (base + off[5]) : NULL;
    m->k.mq = mq ? base + off[6] : NULL;
    m->k.rows = rows;
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

// rows per wave step: 2 where every matrix allows it (SML_GEMV_RB overrides)
static int pick_rb(int nbits, const int * rows, int nm) {
    int rb = env_int("SML_GEMV_RB", 2);
    if (rb != 1 && rb != 2 && rb != 4) rb = 2;
    if (rb == 4 && nbits != 4) rb = 2;
    for (int i = 0; i < nm; i++) while (rb > 1 && rows[i] % rb) rb /= 2;
    return rb;
}

void op_gemv(hipStream_t st, const sml_hip_mat * const * mats, int nm, int epi, const int8_t * q,
             const float * scale, const int32_t * sums, float * const * y, const float * const * bias,
             const float * resid) {
    if (nm < 1 || nm > SML_MAX_MATS) hx_failf("gemv of %d matrices", nm);
    sml_kgemv a;
    memset(&a, 0, sizeof a);
    const int nb = mats[0]->nbits, cols = mats[0]->cols;
    int rows[SML_MAX_MATS], tot = 0;
    for (int i = 0; i < nm; i++) {
        if (mats[i]->nbits != nb || mats[i]->cols != cols) hx_failf("gemv group mixes shapes or widths");
        a.m[i] = mats[i]->k;
        a.m[i].y = y[i];
        a.m[i].bias = bias ? bias[i] : NULL;
        a.m[i].row_begin = tot;
        rows[i] = mats[i]->k.rows;
        tot += rows[i];
    }
    if (epi == SML_EPI_SWIGLU && (nm != 2 || rows[0] != rows[1])) hx_failf("swiglu needs gate and up of one shape");
    a.nmat = nm; a.cols = cols; a.epi = epi;
    a.q = q; a.scale = scale; a.sums = sums; a.resid = resid;
    const int rb = pick_rb(nb, rows, nm);
    a.total_rows = epi == SML_EPI_SWIGLU ? rows[0] : tot;
    const int nrb = a.total_rows / rb;
    int wgs = (nrb + 3) / 4;
    const int cap = env_int("SML_GEMV_WG_CAP", 0);
    if (cap > 0 && wgs > cap) wgs = cap;
    char name[32];
    snprintf(name, sizeof name, "sml_gemv_q%d_r%d", nb, rb);
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

#define ATTN_CHUNK 64

size_t sml_hip_attn_part_floats(int n_head, int hd, int n_ctx) {
    const int ns = (n_ctx + ATTN_CHUNK - 1) / ATTN_CHUNK;
    return (size_t) n_head * ns * (size_t) (hd + 2);
}

void op_attention(hipStream_t st, float * q, const float * k, const float * v, uint16_t * kc, uint16_t * vc,
                  const float * cos_t, const float * sin_t, const int32_t * pos, int n_head, int n_kv,
                  int hd, int n_ctx, float * part, float * out) {
    if (hd != 128 || n_kv <= 0 || n_head % n_kv || n_head / n_kv > 8)
        hx_failf("attention shape (heads %d/%d, head_dim %d) not supported", n_head, n_kv, hd);
    sml_kropekv r;
    memset(&r, 0, sizeof r);
    r.q = q; r.k = k; r.v = v; r.kcache = kc; r.vcache = vc; r.cos_t = cos_t; r.sin_t = sin_t; r.pos = pos;
    r.n_head = n_head; r.n_kv = n_kv; r.hd = hd; r.half = hd / 2;
    hx_launch("sml_rope_kv", 1, 1, 256, 0, st, &r);
    const int ns = (n_ctx + ATTN_CHUNK - 1) / ATTN_CHUNK;
    sml_kattn a;
    memset(&a, 0, sizeof a);
    a.q = q; a.kcache = kc; a.vcache = vc; a.pos = pos; a.part = part;
    a.n_head = n_head; a.n_kv = n_kv; a.hd = hd; a.chunk = ATTN_CHUNK; a.nsplit = ns;
    a.inv = 1.0f / __builtin_sqrtf((float) hd);
    hx_launch("sml_attn_part", (unsigned) ns, (unsigned) n_kv, 256, 0, st, &a);
    sml_kattn_comb c;
    memset(&c, 0, sizeof c);
    c.part = part; c.pos = pos; c.out = out; c.n_head = n_head; c.hd = hd; c.chunk = ATTN_CHUNK; c.nsplit = ns;
    hx_launch("sml_attn_combine", (unsigned) n_head, 1, (unsigned) hd, 0, st, &c);
}

int sml_hip_attention(float * q, const float * k, const float * v, uint16_t * kcache, uint16_t * vcache,
                      const float * cos_t, const float * sin_t, const int32_t * pos,
                      int n_head, int n_kv, int hd, int n_ctx, float * part, float * out) {
    OP_BEGIN(-1);
    op_attention(0, q, k, v, kcache, vcache, cos_t, sin_t, pos, n_head, n_kv, hd, n_ctx, part, out);
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
