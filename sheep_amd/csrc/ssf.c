// SSF reader, validator and seeded synthetic-model writer.
//
// Validation follows the reference loader's acceptance rules
// (sml/sml-model.c:26-72 record ranges, :173-260 header checks); anything this
// GPU path does not execute (LADDER codes, exact-f32 files, Hadamard rotation)
// is accepted here and refused later by the engine with a reason.
#define _GNU_SOURCE
#include "ssf.h"

#include <fcntl.h>
#include <limits.h>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

_Static_assert(sizeof(ssf_header) == 4 + 4 + 7 * 4 + 2 * 4 + 2 * 4 + 4 * 4 + 8 + 6 * 8
                   + 2 * 4 + 2 * 4 + 4 * 4 + 3 * 4 + 2 * 4 + 2 * 4 + 4 + 2 * 4
                   + 3 * 4 + 2 * 4 + 4 + 2 * 4, "ssf_header layout");

static void say(char * why, int nwhy, const char * fmt, ...) {
    if (!why || nwhy <= 0) return;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(why, (size_t) nwhy, fmt, ap);
    va_end(ap);
}

// ------------------------------------------------------------------ fp16

uint16_t ssf_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t e8 = (x >> 23) & 0xffu;
    uint32_t m = x & 0x7fffffu;
    if (e8 == 0xffu) return (uint16_t) (sign | 0x7c00u | (m ? 0x200u : 0u));
    const int e = (int) e8 - 127 + 15;
    if (e >= 31) return (uint16_t) (sign | 0x7c00u);
    if (e <= 0) {                                  // subnormal half or zero
        if (e < -10) return (uint16_t) sign;
        m |= 0x800000u;
        const uint32_t sh = (uint32_t) (14 - e);
        uint32_t v = m >> sh;
        const uint32_t rest = m & ((1u << sh) - 1u), half = 1u << (sh - 1u);
        if (rest > half || (rest == half && (v & 1u))) v++;
        return (uint16_t) (sign | v);
    }
    uint32_t v = ((uint32_t) e << 10) | (m >> 13);
    const uint32_t rest = m & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (v & 1u))) v++;   // carries into the exponent correctly
    return (uint16_t) (sign | v);
}

float ssf_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t) (h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu, bits;
    if (e == 0) {
        if (!m) bits = sign;
        else {                                     // normalise a subnormal
            int sh = 0;
            while (!(m & 0x400u)) { m <<= 1; sh++; }
            m &= 0x3ffu;
            bits = sign | ((uint32_t) (127 - 15 + 1 - sh) << 23) | (m << 13);
        }
    } else if (e == 31) bits = sign | 0x7f800000u | (m << 13);
    else bits = sign | ((e - 15 + 127) << 23) | (m << 13);
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

// ------------------------------------------------------------------ reader

static int inside(size_t size, uint64_t off, uint64_t n) {
    return off <= (uint64_t) size && n <= (uint64_t) size - off;
}
static int payload(size_t size, uint64_t off, uint64_t n) {
    return off >= SSF_HEADER_BYTES && inside(size, off, n);
}

int ssf_flat_planes(int nbits, int bits_out[SSF_MAX_PLANES]) {
    // lowest code bits first, except Q6, whose 2-bit plane (bits 4-5) comes first
    static const int tab[9][4] = {
        {0}, {0}, {2}, {2, 1}, {4}, {4, 1}, {2, 4}, {4, 2, 1}, {4, 4} };
    static const int cnt[9] = { 0, 0, 1, 2, 1, 2, 2, 3, 2 };
    if (nbits < 2 || nbits > 8) return 0;
    for (int i = 0; i < cnt[nbits]; i++) bits_out[i] = tab[nbits][i];
    return cnt[nbits];
}

int ssf_open(ssf_file * f, const char * path, char * why, int nwhy) {
    memset(f, 0, sizeof *f);
    const int fd = open(path, O_RDONLY);
    if (fd < 0) { say(why, nwhy, "cannot open %s", path); return 0; }
    struct stat st;
    if (fstat(fd, &st) != 0) { close(fd); say(why, nwhy, "cannot stat %s", path); return 0; }
    if ((size_t) st.st_size < SSF_HEADER_BYTES) {
        close(fd);
        say(why, nwhy, "%s is smaller than the SSF header", path);
        return 0;
    }
    void * base = mmap(NULL, (size_t) st.st_size, PROT_READ, MAP_SHARED, fd, 0);
    close(fd);
    if (base == MAP_FAILED) { say(why, nwhy, "cannot map %s", path); return 0; }
    f->base = (const uint8_t *) base;
    f->size = (size_t) st.st_size;
    f->hdr = (const ssf_header *) f->base;
    const ssf_header * h = f->hdr;
    const char * bad = NULL;
    if (memcmp(h->magic, SSF_MAGIC, 4) != 0) bad = "not an SSF file";
    else if (h->version > SSF_VERSION_MAX) bad = "format version newer than 9";
    else if (h->version < 8) bad = "format older than v8 (no FLAT layout)";
    else if (!h->n_levels || h->n_levels > SSF_MAX_PLANES || !h->n_tensors) bad = "invalid level or tensor counts";
    else if ((h->flags & ~(SSF_FLAG_HADAMARD | SSF_FLAG_SCALE6 | SSF_FLAG_MINNEG | SSF_FLAG_EXACT)) ||
             ((h->flags & SSF_FLAG_MINNEG) && !(h->flags & SSF_FLAG_SCALE6))) bad = "unsupported model flags";
    else if (h->table_off < SSF_HEADER_BYTES || h->table_off > f->size ||
             h->n_tensors > (f->size - h->table_off) / sizeof(ssf_record)) bad = "tensor table outside the file";
    else if ((h->json_n && (h->json_off < SSF_HEADER_BYTES || !inside(f->size, h->json_off, h->json_n))) ||
             (h->tok_n && (h->tok_off < SSF_HEADER_BYTES || !inside(f->size, h->tok_off, h->tok_n))))
        bad = "metadata ranges outside the file";
    else if (h->group != SSF_GROUP) bad = "group size is not 32";
    if (bad) { say(why, nwhy, "%s: %s", path, bad); ssf_close(f); return 0; }
    f->recs = (const ssf_record *) (f->base + h->table_off);
    for (uint64_t i = 0; i < h->n_tensors; i++) {
        const ssf_record * r = &f->recs[i];
        const char * issue = NULL;
        if (!r->rows || !r->cols || r->rows > INT_MAX || r->cols > INT_MAX) issue = "invalid dimensions";
        else if (r->kind == SSF_KIND_F32) {
            if (r->f32_bytes != (uint64_t) r->rows * r->cols * 4u || !payload(f->size, r->f32_off, r->f32_bytes))
                issue = "invalid f32 payload";
        } else if (r->kind != SSF_KIND_QUANT) issue = "unknown tensor kind";
        else if (r->layout > SSF_LAYOUT_FLAT || (r->layout == SSF_LAYOUT_FLAT && (r->nbits < 2 || r->nbits > 8)))
            issue = "invalid code layout";
        if (!issue && r->kind == SSF_KIND_QUANT) {
            const uint64_t off[5] = { r->sd_off, r->sq_off, r->perm_off, r->md_off, r->mq_off };
            const uint64_t len[5] = { r->sd_bytes, r->sq_bytes, r->perm_bytes, r->md_bytes, r->mq_bytes };
            for (int j = 0; j < 5 && !issue; j++)
                if (len[j] && !payload(f->size, off[j], len[j])) issue = "metadata outside the file";
            for (int j = 0; j < SSF_MAX_PLANES && !issue; j++)
                if (r->plane_bytes[j] && !payload(f->size, r->plane_off[j], r->plane_bytes[j]))
                    issue = "codes outside the file";
        }
        if (issue) {
            say(why, nwhy, "%s: tensor %llu (%.*s): %s", path, (unsigned long long) i,
                SSF_NAME_LEN, r->name, issue);
            ssf_close(f);
            return 0;
        }
    }
    return 1;
}

void ssf_close(ssf_file * f) {
    if (f->base) munmap((void *) f->base, f->size);
    memset(f, 0, sizeof *f);
}

const ssf_record * ssf_find(const ssf_file * f, const char * name) {
    for (uint64_t i = 0; i < f->hdr->n_tensors; i++)
        if (strncmp(f->recs[i].name, name, SSF_NAME_LEN) == 0) return &f->recs[i];
    return NULL;
}

const ssf_record * ssf_findf(const ssf_file * f, const char * fmt, int layer) {
    char nm[SSF_NAME_LEN + 16];
    snprintf(nm, sizeof nm, fmt, layer);
    return ssf_find(f, nm);
}

// ------------------------------------------------------------------ generators

uint64_t ssf_splitmix64(uint64_t * s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

double ssf_normal(uint64_t * s) {
    // Box-Muller, one value per call (the second is discarded to keep the
    // stream position a pure function of the call count)
    double u1 = (double) ((ssf_splitmix64(s) >> 11) + 1) * 0x1.0p-53;
    double u2 = (double) (ssf_splitmix64(s) >> 11) * 0x1.0p-53;
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

static uint64_t key(uint64_t seed, uint64_t a, uint64_t b) {
    uint64_t s = seed ^ (a * 0xD1B54A32D192ED03ull) ^ (b * 0x8CB92BA72F3D8DD7ull);
    return ssf_splitmix64(&s);
}

// ------------------------------------------------------------------ writer

typedef struct {
    const char * name;
    int kind;                 // SSF_KIND_*
    int rows, cols, nbits;
    int perm_key;             // tensors with equal perm_key share one permutation array
    int zero_mean;            // QUANT: mins at -(2^b - 1)/2 steps
    int fill;                 // F32: 0 = 1+N(0,s), 1 = N(0,s)
    float sigma;
    // QUANT given by the caller instead of generated: planes, fields, perm
    const uint8_t * g_planes[SSF_MAX_PLANES];
    const uint16_t * g_sd, * g_md;
    const uint8_t * g_sq, * g_mq;
    const int32_t * g_perm;
    ssf_record rec;
} plan_t;

typedef struct { plan_t * v; int n, cap; } plan_list;

static plan_t * plan_add(plan_list * l) {
    if (l->n == l->cap) {
        l->cap = l->cap ? l->cap * 2 : 64;
        l->v = realloc(l->v, (size_t) l->cap * sizeof(plan_t));
    }
    memset(&l->v[l->n], 0, sizeof(plan_t));
    return &l->v[l->n++];
}

static uint64_t align256(uint64_t x) { return (x + 255u) & ~(uint64_t) 255u; }

static char * sdup(const char * fmt, ...) {
    char buf[SSF_NAME_LEN + 32];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    return strdup(buf);
}

static void add_quant(plan_list * l, const char * name, int rows, int cols, int nbits, int perm_key, int zero_mean) {
    plan_t * p = plan_add(l);
    p->name = name; p->kind = SSF_KIND_QUANT; p->rows = rows; p->cols = cols; p->nbits = nbits;
    p->perm_key = perm_key; p->zero_mean = zero_mean;
}

static void add_f32(plan_list * l, const char * name, int count, int fill, float sigma) {
    plan_t * p = plan_add(l);
    p->name = name; p->kind = SSF_KIND_F32; p->rows = 1; p->cols = count; p->fill = fill; p->sigma = sigma;
}

// pack one row's integer codes (permuted column order) into the planes of width nbits
static void pack_row(const uint8_t * code, int cols, int nbits, uint8_t * const planes[SSF_MAX_PLANES]) {
    int pb[SSF_MAX_PLANES];
    const int np = ssf_flat_planes(nbits, pb);
    // bit offset of each plane within the code
    int shift[SSF_MAX_PLANES], s = 0;
    if (nbits == 6) { shift[0] = 4; shift[1] = 0; }
    else for (int i = 0; i < np; i++) { shift[i] = s; s += pb[i]; }
    const int ng = cols / SSF_GROUP;
    for (int i = 0; i < np; i++) {
        uint8_t * d = planes[i];
        const int sh = shift[i];
        if (pb[i] == 4) {
            // 64-byte quad = groups 4q..4q+3: bytes 0-31 lo/hi = groups 4q/4q+1, 32-63 = 4q+2/4q+3
            for (int q = 0; q < ng / 4; q++)
                for (int half = 0; half < 2; half++)
                    for (int j = 0; j < 32; j++) {
                        const int g0 = 4 * q + 2 * half;
                        const int lo = (code[g0 * 32 + j] >> sh) & 15, hi = (code[(g0 + 1) * 32 + j] >> sh) & 15;
                        d[q * 64 + half * 32 + j] = (uint8_t) (lo | (hi << 4));
                    }
        } else if (pb[i] == 2) {
            // 32-byte pack = 128 weights; bit-plane k of byte j is group 4p+k, column j
            for (int p = 0; p < cols / 128; p++)
                for (int j = 0; j < 32; j++) {
                    uint8_t b = 0;
                    for (int k = 0; k < 4; k++) b |= (uint8_t) (((code[p * 128 + k * 32 + j] >> sh) & 3) << (2 * k));
                    d[p * 32 + j] = b;
                }
        } else {
            // 4 bytes per group, bit j (least significant first) is weight j
            for (int g = 0; g < ng; g++)
                for (int by = 0; by < 4; by++) {
                    uint8_t b = 0;
                    for (int k = 0; k < 8; k++) b |= (uint8_t) (((code[g * 32 + by * 8 + k] >> sh) & 1) << k);
                    d[g * 4 + by] = b;
                }
        }
    }
}

static int write_at(int fd, const void * buf, size_t n, uint64_t off) {
    const uint8_t * p = (const uint8_t *) buf;
    while (n) {
        const ssize_t w = pwrite(fd, p, n, (off_t) off);
        if (w <= 0) return 0;
        p += w; n -= (size_t) w; off += (uint64_t) w;
    }
    return 1;
}

static void make_perm(int32_t * perm, int cols, int random, uint64_t seed, int perm_key) {
    for (int i = 0; i < cols; i++) perm[i] = i;
    if (!random) return;
    uint64_t s = key(seed, 0x5045524dull, (uint64_t) perm_key);
    for (int i = cols - 1; i > 0; i--) {
        const int j = (int) (ssf_splitmix64(&s) % (uint64_t) (i + 1));
        const int32_t t = perm[i]; perm[i] = perm[j]; perm[j] = t;
    }
}

// Fill one quantized matrix: fields by the two-level encoding of random group
// steps (sd = f16(max step / 255), sq = clip(rint(step / sd), 1, 255); mins at
// -zp steps: md = f16(max |min| / 127), mq = clip(rint(min / md) + 127, 0, 254)),
// codes uniform over [0, 2^b - 1]. zp is 2^(b-1), or (2^b - 1)/2 for a
// zero-mean matrix: a uniform code then averages the min back to zero, so no
// common term runs through every row of a decoder. Rows are independent streams, so the fill
// runs in parallel and stays deterministic.
static void fill_quant(const plan_t * p, uint64_t seed, int tidx, uint8_t * const planes[SSF_MAX_PLANES],
                       uint16_t * sd, uint8_t * sq, uint16_t * md, uint8_t * mq, float sigma) {
    const int rows = p->rows, cols = p->cols, nb = p->nbits;
    const int ng = cols / SSF_GROUP, ns = SSF_NSUPER(cols);
    int pb[SSF_MAX_PLANES];
    const int np = ssf_flat_planes(nb, pb);
    const float qmax = (float) ((1 << (nb - 1)) - 1);
    const float zp = p->zero_mean ? 0.5f * (float) ((1 << nb) - 1) : (float) (1 << (nb - 1));
    #pragma omp parallel
    {
        uint8_t * code = malloc((size_t) cols);
        float * step = malloc((size_t) ng * sizeof(float));
        float * mins = malloc((size_t) ng * sizeof(float));
        #pragma omp for schedule(static)
        for (int r = 0; r < rows; r++) {
            uint64_t s = key(seed, (uint64_t) tidx, (uint64_t) r);
            for (int g = 0; g < ng; g++) step[g] = (float) fabs(ssf_normal(&s) * sigma) / qmax;
            for (int k = 0; k < ns; k++) {
                const int g0 = k * 8, g1 = g0 + 8 < ng ? g0 + 8 : ng;
                float mx = 0.0f;
                for (int g = g0; g < g1; g++) if (step[g] > mx) mx = step[g];
                const uint16_t d = ssf_f32_to_f16(mx / 255.0f);
                float dv = ssf_f16_to_f32(d);
                if (dv == 0.0f) dv = 1e-8f;
                sd[(size_t) r * ns + k] = d;
                float mmax = 0.0f;
                for (int g = g0; g < g1; g++) {
                    float q = rintf(step[g] / dv);
                    q = q < 1.0f ? 1.0f : q > 255.0f ? 255.0f : q;
                    sq[(size_t) r * ng + g] = (uint8_t) q;
                    mins[g] = -zp * (ssf_f16_to_f32(d) * q);
                    if (-mins[g] > mmax) mmax = -mins[g];
                }
                const uint16_t m16 = ssf_f32_to_f16(mmax / 127.0f);
                float mv = ssf_f16_to_f32(m16);
                if (mv == 0.0f) mv = 1e-8f;
                md[(size_t) r * ns + k] = m16;
                for (int g = g0; g < g1; g++) {
                    float q = rintf(mins[g] / mv) + 127.0f;
                    q = q < 0.0f ? 0.0f : q > 254.0f ? 254.0f : q;
                    mq[(size_t) r * ng + g] = (uint8_t) q;
                }
            }
            const uint32_t mask = (1u << nb) - 1u;
            for (int c = 0; c < cols; c += 8) {
                const uint64_t z = ssf_splitmix64(&s);
                for (int k = 0; k < 8; k++) code[c + k] = (uint8_t) ((z >> (8 * k)) & mask);
            }
            uint8_t * rp[SSF_MAX_PLANES];
            for (int i = 0; i < np; i++) rp[i] = planes[i] + (size_t) r * ssf_plane_row_bytes(pb[i], cols);
            pack_row(code, cols, nb, rp);
        }
        free(code); free(step); free(mins);
    }
}

static int write_plan(const char * path, ssf_header * h, plan_list * l, uint64_t seed, int random_perm,
                      float step_sigma, char * why, int nwhy) {
    // layout: header, table, then every array 256-byte aligned
    h->n_tensors = (uint64_t) l->n;
    h->table_off = SSF_HEADER_BYTES;
    uint64_t off = align256(h->table_off + (uint64_t) l->n * sizeof(ssf_record));
    // permutation arrays, one per distinct key
    int nkeys = 0;
    const int32_t ** kperm = calloc((size_t) l->n, sizeof(int32_t *));
    int * keys = calloc((size_t) l->n, sizeof(int));
    uint64_t * koff = calloc((size_t) l->n, sizeof(uint64_t));
    int * kcols = calloc((size_t) l->n, sizeof(int));
    for (int i = 0; i < l->n; i++) {
        plan_t * p = &l->v[i];
        ssf_record * r = &p->rec;
        memset(r, 0, sizeof *r);
        strncpy(r->name, p->name, SSF_NAME_LEN);
        r->kind = (uint32_t) p->kind; r->rows = (uint32_t) p->rows; r->cols = (uint32_t) p->cols;
        if (p->kind == SSF_KIND_F32) {
            r->f32_off = off; r->f32_bytes = (uint64_t) p->rows * p->cols * 4u;
            off = align256(off + r->f32_bytes);
            continue;
        }
        r->group = SSF_GROUP;
        r->layout = SSF_LAYOUT_FLAT; r->nbits = (uint32_t) p->nbits;
        int k = -1;
        for (int j = 0; j < nkeys; j++) if (keys[j] == p->perm_key && kcols[j] == p->cols) k = j;
        if (k < 0) {
            k = nkeys++;
            keys[k] = p->perm_key; kcols[k] = p->cols; koff[k] = off; kperm[k] = p->g_perm;
            off = align256(off + (uint64_t) p->cols * 4u);
        }
        r->perm_off = koff[k]; r->perm_bytes = (uint64_t) p->cols * 4u;
        const uint64_t ng = (uint64_t) p->cols / SSF_GROUP, ns = (uint64_t) SSF_NSUPER(p->cols);
        r->sd_off = off; r->sd_bytes = (uint64_t) p->rows * ns * 2u; off = align256(off + r->sd_bytes);
        r->sq_off = off; r->sq_bytes = (uint64_t) p->rows * ng;      off = align256(off + r->sq_bytes);
        r->md_off = off; r->md_bytes = (uint64_t) p->rows * ns * 2u; off = align256(off + r->md_bytes);
        r->mq_off = off; r->mq_bytes = (uint64_t) p->rows * ng;      off = align256(off + r->mq_bytes);
        int pb[SSF_MAX_PLANES];
        const int np = ssf_flat_planes(p->nbits, pb);
        for (int j = 0; j < np; j++) {
            r->plane_off[j] = off;
            r->plane_bytes[j] = (uint64_t) p->rows * ssf_plane_row_bytes(pb[j], p->cols);
            off = align256(off + r->plane_bytes[j]);
        }
    }
    const uint64_t total = off;
    char tmp[4096];
    snprintf(tmp, sizeof tmp, "%s.part", path);
    const int fd = open(tmp, O_RDWR | O_CREAT | O_TRUNC, 0644);
    int ok = fd >= 0 && ftruncate(fd, (off_t) total) == 0;
    if (!ok) say(why, nwhy, "cannot create %s", tmp);
    uint8_t * head = calloc(1, SSF_HEADER_BYTES);
    memcpy(head, h, sizeof *h);
    if (ok) ok = write_at(fd, head, SSF_HEADER_BYTES, 0);
    free(head);
    for (int i = 0; ok && i < l->n; i++)
        ok = write_at(fd, &l->v[i].rec, sizeof(ssf_record), h->table_off + (uint64_t) i * sizeof(ssf_record));
    for (int k = 0; ok && k < nkeys; k++) {
        if (kperm[k]) { ok = write_at(fd, kperm[k], (size_t) kcols[k] * 4u, koff[k]); continue; }
        int32_t * perm = malloc((size_t) kcols[k] * 4u);
        make_perm(perm, kcols[k], random_perm, seed, keys[k]);
        ok = write_at(fd, perm, (size_t) kcols[k] * 4u, koff[k]);
        free(perm);
    }
    for (int i = 0; ok && i < l->n; i++) {
        const plan_t * p = &l->v[i];
        const ssf_record * r = &p->rec;
        if (p->kind == SSF_KIND_F32) {
            const size_t cnt = (size_t) p->rows * p->cols;
            float * v = malloc(cnt * sizeof(float));
            uint64_t s = key(seed, (uint64_t) i, 0xF32ull);
            for (size_t j = 0; j < cnt; j++) {
                const float z = (float) ssf_normal(&s) * p->sigma;
                v[j] = p->fill == 0 ? 1.0f + z : z;
            }
            ok = write_at(fd, v, cnt * sizeof(float), r->f32_off);
            free(v);
            continue;
        }
        int pb[SSF_MAX_PLANES];
        const int np = ssf_flat_planes(p->nbits, pb);
        if (p->g_sd) {
            ok = write_at(fd, p->g_sd, r->sd_bytes, r->sd_off) && write_at(fd, p->g_sq, r->sq_bytes, r->sq_off) &&
                 write_at(fd, p->g_md, r->md_bytes, r->md_off) && write_at(fd, p->g_mq, r->mq_bytes, r->mq_off);
            for (int j = 0; ok && j < np; j++) ok = write_at(fd, p->g_planes[j], r->plane_bytes[j], r->plane_off[j]);
            if (!ok) say(why, nwhy, "write failed on %s", p->name);
            continue;
        }
        uint8_t * planes[SSF_MAX_PLANES] = { 0 };
        for (int j = 0; j < np; j++) planes[j] = malloc(r->plane_bytes[j]);
        uint16_t * sd = malloc(r->sd_bytes), * md = malloc(r->md_bytes);
        uint8_t * sq = malloc(r->sq_bytes), * mq = malloc(r->mq_bytes);
        fill_quant(p, seed, i, planes, sd, sq, md, mq, step_sigma);
        ok = write_at(fd, sd, r->sd_bytes, r->sd_off) && write_at(fd, sq, r->sq_bytes, r->sq_off) &&
             write_at(fd, md, r->md_bytes, r->md_off) && write_at(fd, mq, r->mq_bytes, r->mq_off);
        for (int j = 0; j < np; j++) {
            if (ok) ok = write_at(fd, planes[j], r->plane_bytes[j], r->plane_off[j]);
            free(planes[j]);
        }
        free(sd); free(md); free(sq); free(mq);
        if (!ok) say(why, nwhy, "write failed on %s", p->name);
    }
    if (fd >= 0) close(fd);
    free(keys); free(koff); free(kcols); free(kperm);
    if (ok && rename(tmp, path) != 0) { ok = 0; say(why, nwhy, "cannot rename %s", tmp); }
    if (!ok) unlink(tmp);
    return ok;
}

static void base_header(ssf_header * h) {
    memset(h, 0, sizeof *h);
    memcpy(h->magic, SSF_MAGIC, 4);
    h->version = 9;
    h->group = SSF_GROUP;
    h->n_levels = 1;
    h->level_bits[0] = 4;      // the FLAT file signature the reference loader admits
}

int ssf_synth_model(const char * path, const ssf_synth_spec * sp, char * why, int nwhy) {
    if (sp->nbits < 2 || sp->nbits > 8 || !sp->n_layer || !sp->n_head || !sp->n_head_kv ||
        sp->n_embd % sp->n_head || sp->n_embd % 128 || sp->n_ff % 128 || sp->n_head % sp->n_head_kv) {
        say(why, nwhy, "synthetic spec out of range");
        return 0;
    }
    ssf_header h;
    base_header(&h);
    h.n_layer = sp->n_layer; h.n_embd = sp->n_embd; h.n_head = sp->n_head; h.n_head_kv = sp->n_head_kv;
    h.n_ff = sp->n_ff; h.n_vocab = sp->n_vocab; h.n_ctx_train = sp->n_ctx_train;
    h.rope_theta = sp->rope_theta; h.rms_eps = sp->rms_eps;
    h.n_expert_used = sp->n_expert ? (uint32_t) sp->n_expert_used : 0;
    h.moe_flags = sp->n_expert ? sp->moe_flags : 0;
    if (sp->n_expert) {
        h.moe_scale = sp->moe_scale;
        h.moe_groups = sp->moe_groups;
        h.moe_topk_group = sp->moe_topk_group;
    }
    if (sp->n_ff_shexp < 0 || sp->n_ff_shexp % 128) {
        say(why, nwhy, "shared expert width %d (a multiple of 128)", sp->n_ff_shexp);
        return 0;
    }
    const int hd = (int) (sp->n_embd / sp->n_head);
    const int nq = (int) sp->n_head * hd, nkv = (int) sp->n_head_kv * hd;
    const int E = (int) sp->n_embd, F = (int) sp->n_ff, b = sp->nbits;
    plan_list l = { 0 };
    int pk = 0;   // permutation keys: members of one shared-activation group share one
    add_quant(&l, "token_embd.weight", (int) sp->n_vocab, E, b, pk++, sp->zero_mean);
    if (!sp->tied) add_quant(&l, "output.weight", (int) sp->n_vocab, E, b, pk++, sp->zero_mean);
    add_f32(&l, "output_norm.weight", E, 0, 0.02f);
    for (int L = 0; L < (int) sp->n_layer; L++) {
        add_f32(&l, sdup("blk.%d.attn_norm.weight", L), E, 0, 0.02f);
        const int kqkv = pk++;
        add_quant(&l, sdup("blk.%d.attn_q.weight", L), nq, E, b, kqkv, sp->zero_mean);
        add_quant(&l, sdup("blk.%d.attn_k.weight", L), nkv, E, b, kqkv, sp->zero_mean);
        add_quant(&l, sdup("blk.%d.attn_v.weight", L), nkv, E, b, kqkv, sp->zero_mean);
        if (sp->qkv_bias) {
            add_f32(&l, sdup("blk.%d.attn_q.bias", L), nq, 1, 0.02f);
            add_f32(&l, sdup("blk.%d.attn_k.bias", L), nkv, 1, 0.02f);
            add_f32(&l, sdup("blk.%d.attn_v.bias", L), nkv, 1, 0.02f);
        }
        add_quant(&l, sdup("blk.%d.attn_output.weight", L), E, nq, b, pk++, sp->zero_mean);
        add_f32(&l, sdup("blk.%d.ffn_norm.weight", L), E, 0, 0.02f);
        if (sp->n_expert) {
            add_f32(&l, sdup("blk.%d.ffn_gate_inp.weight", L), sp->n_expert * E, 1, sp->router_sigma);
            for (int e = 0; e < sp->n_expert; e++) {
                const int kgu = pk++;
                add_quant(&l, sdup("blk.%d.ffn_gate.%d.weight", L, e), F, E, b, kgu, sp->zero_mean);
                add_quant(&l, sdup("blk.%d.ffn_up.%d.weight", L, e), F, E, b, kgu, sp->zero_mean);
                add_quant(&l, sdup("blk.%d.ffn_down.%d.weight", L, e), E, F, b, pk++, sp->zero_mean);
            }
            if (sp->exp_bias) add_f32(&l, sdup("blk.%d.exp_probs_b.weight", L), sp->n_expert, 1, 0.05f);
            if (sp->n_ff_shexp) {
                const int FS = sp->n_ff_shexp, kgu = pk++;
                add_quant(&l, sdup("blk.%d.ffn_gate_shexp.weight", L), FS, E, b, kgu, sp->zero_mean);
                add_quant(&l, sdup("blk.%d.ffn_up_shexp.weight", L), FS, E, b, kgu, sp->zero_mean);
                add_quant(&l, sdup("blk.%d.ffn_down_shexp.weight", L), E, FS, b, pk++, sp->zero_mean);
                if (sp->shexp_gate) add_f32(&l, sdup("blk.%d.ffn_gate_inp_shexp.weight", L), E, 1, sp->router_sigma);
            }
        } else {
            const int kgu = pk++;
            add_quant(&l, sdup("blk.%d.ffn_gate.weight", L), F, E, b, kgu, sp->zero_mean);
            add_quant(&l, sdup("blk.%d.ffn_up.weight", L), F, E, b, kgu, sp->zero_mean);
            add_quant(&l, sdup("blk.%d.ffn_down.weight", L), E, F, b, pk++, sp->zero_mean);
        }
    }
    const int ok = write_plan(path, &h, &l, sp->seed, sp->random_perm, sp->step_sigma, why, nwhy);
    for (int i = 0; i < l.n; i++)
        if (strncmp(l.v[i].name, "blk.", 4) == 0) free((void *) l.v[i].name);
    free(l.v);
    return ok;
}

int ssf_synth_matrix(const char * path, int rows, int cols, int nbits, int random_perm,
                     float step_sigma, uint64_t seed, char * why, int nwhy) {
    if (rows <= 0 || cols <= 0 || cols % 128 || nbits < 2 || nbits > 8) {
        say(why, nwhy, "matrix shape or width out of range");
        return 0;
    }
    ssf_header h;
    base_header(&h);
    h.n_layer = 0; h.n_embd = (uint32_t) cols; h.n_head = 1; h.n_head_kv = 1;
    plan_list l = { 0 };
    add_quant(&l, "w", rows, cols, nbits, 0, 0);
    const int ok = write_plan(path, &h, &l, seed, random_perm, step_sigma, why, nwhy);
    free(l.v);
    return ok;
}

int ssf_write_quant(const char * path, const char * name, int rows, int cols, int nbits,
                    const uint8_t * const planes[SSF_MAX_PLANES], const uint16_t * sd, const uint8_t * sq,
                    const uint16_t * md, const uint8_t * mq, const int32_t * perm, char * why, int nwhy) {
    int pb[SSF_MAX_PLANES];
    if (rows <= 0 || cols <= 0 || cols % 128 || nbits < 2 || nbits > 8 || !name || strlen(name) >= SSF_NAME_LEN ||
        !sd || !sq || !md || !mq || !perm) {
        say(why, nwhy, "quantized record arguments out of range");
        return 0;
    }
    const int np = ssf_flat_planes(nbits, pb);
    for (int i = 0; i < np; i++)
        if (!planes[i]) { say(why, nwhy, "plane %d of width %d missing", i, nbits); return 0; }
    ssf_header h;
    base_header(&h);
    h.n_layer = 0; h.n_embd = (uint32_t) cols; h.n_head = 1; h.n_head_kv = 1;
    plan_list l = { 0 };
    add_quant(&l, name, rows, cols, nbits, 0, 0);
    plan_t * p = &l.v[0];
    for (int i = 0; i < np; i++) p->g_planes[i] = planes[i];
    p->g_sd = sd; p->g_sq = sq; p->g_md = md; p->g_mq = mq; p->g_perm = perm;
    const int ok = write_plan(path, &h, &l, 0, 0, 0.0f, why, nwhy);
    free(l.v);
    return ok;
}
