// Kernel-level C ABI (include/sml-hip.h): matrix upload and single launches of
// the gfx950 kernels, used by the decode engine, the tests and the benches.
#include "ops.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "sml-hip.h"
#include "ssf.h"

static size_t al256(size_t x) { return (x + 255u) & ~(size_t) 255u; }

// the split-K sums op_gemm left for the next normq (ops_defer_ksum)
static int g_defer, g_pending;
static sml_kksum g_pend;

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

// Exact mode: launches take the forms that follow the reference's float
// order (Q4/Q8 GEMVs, norms, attention, router), so decoding equals its CPU
// path bit for bit.
static int g_exact;
void ops_set_exact(int on) { g_exact = on != 0; }
int ops_exact(void) { return g_exact; }
void sml_hip_set_exact(int on) { ops_set_exact(on); }
void sml_hip_fail_after(long n) { hx.fail_after = n; }
long sml_hip_call_count(void) { return hx.calls; }

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

// Whether Q4 uploads carry the small-M MFMA GEMM's tiled copy (SML_TILED=1;
// off by default): read once per process, so every matrix of a run agrees.
// It doubles the codes and fields a Q4 matrix holds in HBM for 7-11% on the
// 16-row products at 4096 and 14336 columns (per-256 SwiGLU 26.6 -> 24.8 us,
// 4096 x 14336 19.4 -> 17.3; per-32 SwiGLU 29.1 -> 29.7).
static int tiled_on(void) {
    static int on = -1;
    if (on < 0) { const char * e = getenv("SML_TILED"); on = e ? atoi(e) != 0 : 0; }
    return on;
}

// A matrix's single allocation: its code planes, the (sq, mq) group fields,
// the (sd, md) superblock fields and its descriptors, each 256-byte aligned.
// Returns the total; off/sz receive each part's offset and size.
static size_t mat_layout(int rows, int cols, int nbits, size_t off[6], size_t sz[6]) {
    int pb[SSF_MAX_PLANES];
    const int np = ssf_flat_planes(nbits, pb);
    const size_t R = (size_t) rows, ng = (size_t) cols / 32, ns = (size_t) SSF_NSUPER(cols);
    size_t tot = 0;
    for (int i = 0; i < 3; i++) sz[i] = i < np ? R * ssf_plane_row_bytes(pb[i], cols) : 0;
    sz[3] = R * ng * 2;          // (sq, mq) per group
    sz[4] = R * ns * 4;          // (sd, md) per superblock
    sz[5] = 3 * sizeof(sml_kmat);   // the descriptor, then a (gate, up) pair table (small-M GEMM tables)
    for (int i = 0; i < 6; i++) { off[i] = tot; tot += al256(sz[i]); }
    return tot;
}

size_t mat_block_bytes(int rows, int cols, int nbits) {
    size_t off[6], sz[6];
    return mat_layout(rows, cols, nbits, off, sz);
}

// Placement (a model's streamed layers): while a region is set, each upload
// takes the next bytes of [base, base + cap) instead of an allocation of its
// own, and its matrix is marked so that freeing it leaves that memory alone.
static uint8_t * g_place;
static size_t g_place_off, g_place_cap;

void mat_place(void * base, size_t cap) {
    g_place = (uint8_t *) base;
    g_place_off = 0;
    g_place_cap = base ? cap : 0;
}

size_t mat_place_used(void) { return g_place_off; }

sml_hip_mat * mat_upload(const uint8_t * const planes[4], const uint16_t * sd, const uint8_t * sq,
                         const uint16_t * md, const uint8_t * mq, int rows, int cols, int nbits,
                         int scale6, int minneg) {
    if (rows <= 0 || cols <= 0 || cols % 128 || nbits < 2 || nbits > 8)
        hx_failf("matrix %dx%d width %d: shape or width not supported", rows, cols, nbits);
    int pb[SSF_MAX_PLANES];
    const int np = ssf_flat_planes(nbits, pb);
    const size_t R = (size_t) rows, ng = (size_t) cols / 32, ns = (size_t) SSF_NSUPER(cols);
    size_t off[6], sz[6];
    const size_t tot = mat_layout(rows, cols, nbits, off, sz);
    if (g_place && g_place_off + tot > g_place_cap)
        hx_failf("a streamed layer's matrices exceed their %zu-byte staging region", g_place_cap);
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
        if (m->mem && !m->placed) hipFree(m->mem);
        if (m->tiled_mem) hipFree(m->tiled_mem);
        free(m);
        longjmp(*outer, 1);
    }
    hx.jb = &jb;
    if (g_place) {
        m->mem = g_place + g_place_off;
        m->placed = 1;
        g_place_off += tot;
    } else {
        m->mem = hx_malloc(tot);
    }
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
    m->kdev = (sml_kmat *) (base + off[5]);
    // Q4 with SML_TILED=1: the tiled copy the small-M MFMA GEMM streams (one
    // more copy of the codes and fields; without it the GEMM reads the rows
    // as they are)
    if (nbits == 4 && cols % 256 == 0 && tiled_on() && !m->placed) {
        const size_t nt = (size_t) ((rows + 15) / 16) * (size_t) (cols / 256);
        m->tiled_mem = hx_malloc(nt * SML_TILE_Q4);
        sml_ktile t = { m->k.plane[0], m->k.sqmq, m->k.sdmd, (uint8_t *) m->tiled_mem, rows, cols };
        hx_launch("sml_tile_q4", (unsigned) nt, 1, 256, 0, 0, &t);
        HX(hipDeviceSynchronize());
        m->k.tiled = (const uint8_t *) m->tiled_mem;
    }
    HX(hipMemcpy(m->kdev, &m->k, sizeof m->k, hipMemcpyHostToDevice));
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

// ------------------------------------------------------------ GGUF Q4_K blocks
//
// ggml's block_q4_K (the Q4_K_M files' main type): per 256 weights of a row,
// fp16 d and dmin, 12 bytes packing eight 6-bit scales sc_j and mins m_j (one
// per 32 weights), and 128 bytes of 4-bit codes q; a weight is
// d*sc_j*q - dmin*m_j. That is the two-level FLAT Q4 record exactly: per
// superblock sd = d and md = dmin, per group sq = sc_j and mq = 127 - m_j
// (min = md*(mq-127)), and the 128 code bytes are already the FLAT Q4 quads
// (bytes 32c..32c+31 of a block hold sub-blocks 2c (low nibbles) and 2c+1
// (high), as a quad's halves hold groups 4q+2h and 4q+2h+1). So the repack
// moves bytes and fields; nothing is re-quantized or recomputed.
#define Q4K_BLOCK 144

// scale and min of sub-block j from the 12 packed bytes: j < 4 in the low six
// bits of bytes j and j+4; j >= 4 in the nibbles of byte j+4 with the high
// two bits in the top bits of bytes j-4 and j
static void q4k_scale_min(const uint8_t * s, int j, uint8_t * sc, uint8_t * mn) {
    if (j < 4) {
        *sc = s[j] & 63;
        *mn = s[j + 4] & 63;
    } else {
        *sc = (uint8_t) ((s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4));
        *mn = (uint8_t) ((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

// d, dmin and the eight (scale, min) pairs of one K-quant block (Q4_K and
// Q5_K share them) into superblock idx's FLAT fields
static void kq_fields(const uint8_t * blk, size_t idx, uint16_t * sd, uint8_t * sq, uint16_t * md, uint8_t * mq) {
    memcpy(&sd[idx], blk, 2);
    memcpy(&md[idx], blk + 2, 2);
    for (int j = 0; j < 8; j++) {
        uint8_t sc, mn;
        q4k_scale_min(blk + 4, j, &sc, &mn);
        sq[idx * 8 + j] = sc;
        mq[idx * 8 + j] = (uint8_t) (127 - mn);
    }
}

int sml_hip_q4k_repack(const void * blocks, int rows, int cols, uint8_t * plane, uint16_t * sd, uint8_t * sq,
                       uint16_t * md, uint8_t * mq) {
    if (!blocks || rows <= 0 || cols <= 0 || cols % 256 || !plane || !sd || !sq || !md || !mq) return -1;
    const size_t nb = (size_t) cols / 256;
    for (size_t r = 0; r < (size_t) rows; r++)
        for (size_t b = 0; b < nb; b++) {
            const uint8_t * blk = (const uint8_t *) blocks + (r * nb + b) * Q4K_BLOCK;
            kq_fields(blk, r * nb + b, sd, sq, md, mq);
            memcpy(plane + (r * nb + b) * 128, blk + 16, 128);
        }
    return 0;
}

// GGUF Q5_K (ggml's block_q5_K, 176 bytes per 256 weights): d, dmin and the
// twelve scale bytes as in Q4_K, then qh (32 bytes; bit j of byte l is the
// fifth code bit of weight l of sub-block j) and the 128 bytes of low nibbles
// in Q4_K's order. A weight is d*sc_j*(q + 16*h) - dmin*m_j, the two-level
// FLAT Q5 record with Q4_K's fields: its 4-bit plane is the nibbles (already
// FLAT quads) and its 1-bit plane the fifth bits, four bytes per group with
// weight l of the group in bit l%8 of byte l/8.
#define Q5K_BLOCK 176
int sml_hip_q5k_repack(const void * blocks, int rows, int cols, uint8_t * plane4, uint8_t * plane1, uint16_t * sd,
                       uint8_t * sq, uint16_t * md, uint8_t * mq) {
    if (!blocks || rows <= 0 || cols <= 0 || cols % 256 || !plane4 || !plane1 || !sd || !sq || !md || !mq) return -1;
    const size_t nb = (size_t) cols / 256;
    for (size_t r = 0; r < (size_t) rows; r++)
        for (size_t b = 0; b < nb; b++) {
            const uint8_t * blk = (const uint8_t *) blocks + (r * nb + b) * Q5K_BLOCK;
            const uint8_t * qh = blk + 16;
            kq_fields(blk, r * nb + b, sd, sq, md, mq);
            memcpy(plane4 + (r * nb + b) * 128, blk + 48, 128);
            uint8_t * p1 = plane1 + (r * nb + b) * 32;
            for (int j = 0; j < 8; j++)
                for (int by = 0; by < 4; by++) {
                    uint8_t v = 0;
                    for (int k = 0; k < 8; k++) v |= (uint8_t) (((qh[8 * by + k] >> j) & 1) << k);
                    p1[4 * j + by] = v;
                }
        }
    return 0;
}

sml_hip_mat * sml_hip_mat_from_q4k(const void * blocks, int rows, int cols) {
    OP_BEGIN(NULL);
    if (!blocks || rows <= 0 || cols <= 0 || cols % 256) hx_failf("Q4_K matrix %dx%d: not a whole number of blocks", rows, cols);
    const size_t R = (size_t) rows, nb = (size_t) cols / 256;
    uint8_t * plane = malloc(R * nb * 128), * sq = malloc(R * nb * 8), * mq = malloc(R * nb * 8);
    uint16_t * sd = malloc(R * nb * 2), * md = malloc(R * nb * 2);
    if (!plane || !sq || !mq || !sd || !md) {
        free(plane); free(sq); free(mq); free(sd); free(md);
        hx_failf("out of host memory");
    }
    sml_hip_q4k_repack(blocks, rows, cols, plane, sd, sq, md, mq);
    jmp_buf * outer = hx.jb;
    jmp_buf jb;
    if (setjmp(jb)) {
        hx.jb = outer;
        free(plane); free(sq); free(mq); free(sd); free(md);
        longjmp(*outer, 1);
    }
    hx.jb = &jb;
    const uint8_t * planes[4] = { plane, NULL, NULL, NULL };
    sml_hip_mat * m = mat_upload(planes, sd, sq, md, mq, rows, cols, 4, 0, 0);
    hx.jb = outer;
    free(plane); free(sq); free(mq); free(sd); free(md);
    HX_LEAVE();
    return m;
}

sml_hip_mat * sml_hip_mat_from_q5k(const void * blocks, int rows, int cols) {
    OP_BEGIN(NULL);
    if (!blocks || rows <= 0 || cols <= 0 || cols % 256) hx_failf("Q5_K matrix %dx%d: not a whole number of blocks", rows, cols);
    const size_t R = (size_t) rows, nb = (size_t) cols / 256;
    uint8_t * p4 = malloc(R * nb * 128), * p1 = malloc(R * nb * 32), * sq = malloc(R * nb * 8), * mq = malloc(R * nb * 8);
    uint16_t * sd = malloc(R * nb * 2), * md = malloc(R * nb * 2);
    if (!p4 || !p1 || !sq || !mq || !sd || !md) {
        free(p4); free(p1); free(sq); free(mq); free(sd); free(md);
        hx_failf("out of host memory");
    }
    sml_hip_q5k_repack(blocks, rows, cols, p4, p1, sd, sq, md, mq);
    jmp_buf * outer = hx.jb;
    jmp_buf jb;
    if (setjmp(jb)) {
        hx.jb = outer;
        free(p4); free(p1); free(sq); free(mq); free(sd); free(md);
        longjmp(*outer, 1);
    }
    hx.jb = &jb;
    const uint8_t * planes[4] = { p4, p1, NULL, NULL };
    sml_hip_mat * m = mat_upload(planes, sd, sq, md, mq, rows, cols, 5, 0, 0);
    hx.jb = outer;
    free(p4); free(p1); free(sq); free(mq); free(sd); free(md);
    HX_LEAVE();
    return m;
}

// A FLAT record's declared arrays must hold what its shape reads: every plane
// of its width, the step fields (sd, sq) and, when it has a min, md and mq.
// ssf_open has already checked each (offset, bytes) against the file.
static void check_record(const ssf_file * f, const ssf_record * r) {
    const int six = (f->hdr->flags & SSF_FLAG_SCALE6) != 0;
    const uint64_t rows = r->rows, cols = r->cols, ng = cols / 32, ns = (uint64_t) SSF_NSUPER(cols);
    const uint64_t grow = six ? ng / 4 * 3 : ng;
    if (cols % 128) hx_failf("tensor %.64s: %llu columns is not a multiple of 128", r->name, (unsigned long long) cols);
    int pb[SSF_MAX_PLANES];
    const int np = ssf_flat_planes((int) r->nbits, pb);
    for (int p = 0; p < np; p++)
        if (!r->plane_off[p] || r->plane_bytes[p] < rows * ssf_plane_row_bytes(pb[p], (int) cols))
            hx_failf("tensor %.64s: code plane %d is missing or shorter than its shape", r->name, p);
    if (!r->sd_off || !r->sq_off || r->sd_bytes < rows * ns * 2 || r->sq_bytes < rows * grow)
        hx_failf("tensor %.64s: step fields missing or shorter than its shape", r->name);
    if (r->mq_bytes && (!r->md_off || !r->mq_off || r->md_bytes < rows * ns * 2 || r->mq_bytes < rows * grow))
        hx_failf("tensor %.64s: min fields shorter than its shape", r->name);
}

sml_hip_mat * mat_from_record(const ssf_file * f, const ssf_record * r) {
    if (r->kind != SSF_KIND_QUANT || r->layout != SSF_LAYOUT_FLAT)
        hx_failf("tensor %.64s is not a FLAT quantized record", r->name);
    check_record(f, r);
    const uint8_t * planes[4] = { 0 };
    for (int i = 0; i < 4; i++) planes[i] = r->plane_off[i] ? (const uint8_t *) ssf_at(f, r->plane_off[i]) : NULL;
    const int six = (f->hdr->flags & SSF_FLAG_SCALE6) != 0, neg = (f->hdr->flags & SSF_FLAG_MINNEG) != 0;
    return mat_upload(planes, (const uint16_t *) ssf_at(f, r->sd_off), (const uint8_t *) ssf_at(f, r->sq_off),
                      r->mq_bytes ? (const uint16_t *) ssf_at(f, r->md_off) : NULL,
                      r->mq_bytes ? (const uint8_t *) ssf_at(f, r->mq_off) : NULL,
                      (int) r->rows, (int) r->cols, (int) r->nbits, six, neg);
}

// Total rows of records that can be stacked (same FLAT width, input width
// and min presence), or 0.
static size_t stack_rows(const ssf_record * const * recs, int n) {
    size_t rows = 0;
    for (int i = 0; i < n; i++) {
        const ssf_record * r = recs[i];
        if (r->kind != SSF_KIND_QUANT || r->layout != SSF_LAYOUT_FLAT || r->nbits != recs[0]->nbits ||
            r->cols != recs[0]->cols || (r->mq_bytes != 0) != (recs[0]->mq_bytes != 0))
            return 0;
        rows += r->rows;
    }
    return rows;
}

static void free_stack(uint8_t ** pl, uint8_t * sq, uint8_t * mq, uint16_t * sd, uint16_t * md) {
    for (int p = 0; p < 4; p++) free(pl[p]);
    free(sq); free(mq); free(sd); free(md);
}

// Upload the stacked host copy and free it, also when the upload fails.
static sml_hip_mat * upload_stack(uint8_t ** pl, uint8_t * sq, uint8_t * mq, uint16_t * sd, uint16_t * md,
                                  int rows, int cols, int nb, int six, int neg) {
    jmp_buf * outer = hx.jb;
    jmp_buf jb;
    if (setjmp(jb)) { hx.jb = outer; free_stack(pl, sq, mq, sd, md); longjmp(*outer, 1); }
    hx.jb = &jb;
    sml_hip_mat * m = mat_upload((const uint8_t * const *) pl, sd, sq, md, mq, rows, cols, nb, six, neg);
    hx.jb = outer;
    free_stack(pl, sq, mq, sd, md);
    return m;
}

sml_hip_mat * mat_stack(const ssf_file * f, const ssf_record * const * recs, int n) {
    const ssf_record * r0 = recs[0];
    const int nb = (int) r0->nbits, cols = (int) r0->cols, has_min = r0->mq_bytes != 0;
    const size_t rows = stack_rows(recs, n);
    if (!rows) return NULL;
    for (int i = 0; i < n; i++) check_record(f, recs[i]);
    int pb[SSF_MAX_PLANES];
    const int np = ssf_flat_planes(nb, pb);
    const int six = (f->hdr->flags & SSF_FLAG_SCALE6) != 0, neg = (f->hdr->flags & SSF_FLAG_MINNEG) != 0;
    const size_t ng = (size_t) cols / 32, ns = (size_t) SSF_NSUPER(cols), grow = six ? ng / 4 * 3 : ng;
    size_t prb[SSF_MAX_PLANES];
    uint8_t * pl[4] = { 0 };
    uint8_t * sq = malloc(rows * grow), * mq = has_min ? malloc(rows * grow) : NULL;
    uint16_t * sd = malloc(rows * ns * 2), * md = has_min ? malloc(rows * ns * 2) : NULL;
    int ok = sq && sd && (!has_min || (mq && md));
    for (int p = 0; p < np; p++) {
        prb[p] = ssf_plane_row_bytes(pb[p], cols);
        pl[p] = malloc(rows * prb[p]);
        ok = ok && pl[p];
    }
    if (ok) {
        size_t at = 0;
        for (int i = 0; i < n; i++) {
            const ssf_record * r = recs[i];
            const size_t R = r->rows;
            for (int p = 0; p < np; p++) memcpy(pl[p] + at * prb[p], ssf_at(f, r->plane_off[p]), R * prb[p]);
            memcpy(sq + at * grow, ssf_at(f, r->sq_off), R * grow);
            memcpy(sd + at * ns, ssf_at(f, r->sd_off), R * ns * 2);
            if (has_min) {
                memcpy(mq + at * grow, ssf_at(f, r->mq_off), R * grow);
                memcpy(md + at * ns, ssf_at(f, r->md_off), R * ns * 2);
            }
            at += R;
        }
    }
    if (!ok) { free_stack(pl, sq, mq, sd, md); hx_failf("out of host memory"); }
    return upload_stack(pl, sq, mq, sd, md, (int) rows, cols, nb, six, neg);
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
    if (m->mem && !m->placed) HX(hipFree(m->mem));
    if (m->tiled_mem) HX(hipFree(m->tiled_mem));
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
    op_normq_rows(st, x, resid, w, eps, n, 1, nout, perm, q, scale, sums, normed, per256);
}

// Deferred split-K sums. While deferral is on, a split-K product leaves its
// slices, and the next op_ksum_normq_rows adds them as it normalizes the
// rows (sml_ksum_normq: one launch for sml_gemm_ksum + sml_normq2, the same
// bits); op_ksum_flush adds them alone.
void ops_defer_ksum(int on) { g_defer = on; }
void ops_ksum_reset(void) { g_defer = g_pending = 0; }
int ops_ksum_pending(void) { return g_pending; }

void op_ksum_flush(hipStream_t st) {
    if (!g_pending) return;
    g_pending = 0;
    hx_launch("sml_gemm_ksum", (unsigned) (((size_t) g_pend.m * g_pend.rows + 255) / 256), 1, 256, 0, st, &g_pend);
}

void op_ksum_normq_rows(hipStream_t st, float * x, const float * w, float eps, int n, int rows, int nout,
                        const int32_t * const * perm, int8_t * const * q, float * const * scale,
                        int32_t * const * sums, int per256) {
    if (!g_pending) hx_failf("no split-K sums pending");
    int np = 0;
    for (int i = 0; i < nout && i < 3; i++) np += perm[i] != NULL;
    const size_t lds = (size_t) (2 + (np ? nout : 0)) * n * 4;
    if (!w || g_exact || nout < 1 || nout > 3 || n % 32 || n > 4096 || lds > 65536 || g_pend.ks != 4 || g_pend.bias || !g_pend.resid || g_pend.y != x ||
        g_pend.rows != n ||
        g_pend.m != rows) {
        op_ksum_flush(st);
        op_normq_rows(st, x, NULL, w, eps, n, rows, nout, perm, q, scale, sums, NULL, per256);
        return;
    }
    sml_kksumq a;
    memset(&a, 0, sizeof a);
    a.s = g_pend;
    a.q.norm_w = w; a.q.eps = eps; a.q.n = n; a.q.nout = nout; a.q.per256 = per256;
    for (int i = 0; i < nout; i++) { a.q.perm[i] = perm[i]; a.q.q[i] = q[i]; a.q.scale[i] = scale[i]; a.q.sums[i] = sums[i]; }
    g_pending = 0;
    const int ni = n <= 1024 ? 1 : n <= 2048 ? 2 : 4;   // float4s a thread holds
    char name[32];
    snprintf(name, sizeof name, "sml_ksum_normq_%d%s", ni, perm[0] ? "_p" : "");
    hx_launch(name, (unsigned) rows, 1, 256, lds, st, &a);
}

void op_normq_rows(hipStream_t st, float * x, const float * resid, const float * w, float eps, int n, int rows,
                   int nout, const int32_t * const * perm, int8_t * const * q, float * const * scale,
                   int32_t * const * sums, float * normed, int per256) {
    if (rows < 1 || rows > 65535) hx_failf("normq of %d rows", rows);
    if (n <= 0 || n % 32 || n > 16384) hx_failf("normq width %d not supported", n);
    if (nout < 0 || nout > 3) hx_failf("normq of %d outputs (at most 3)", nout);
    sml_knormq a;
    memset(&a, 0, sizeof a);
    a.x = x; a.resid = resid; a.norm_w = w; a.eps = eps; a.n = n; a.nout = nout;
    for (int i = 0; i < nout; i++) { a.perm[i] = perm[i]; a.q[i] = q[i]; a.scale[i] = scale[i]; a.sums[i] = sums[i]; }
    a.normed = normed; a.per256 = per256; a.exact = g_exact;
    if (!resid && !normed) {
        sml_knormq2 b;
        memset(&b, 0, sizeof b);
        b.x = x; b.norm_w = w; b.eps = eps; b.n = n; b.nout = nout; b.per256 = per256; b.exact = g_exact;
        for (int i = 0; i < nout; i++) { b.perm[i] = perm[i]; b.q[i] = q[i]; b.scale[i] = scale[i]; b.sums[i] = sums[i]; }
        hx_launch("sml_normq2", (unsigned) ((n + 255) / 256), (unsigned) rows, 256, 0, st, &b);
        return;
    }
    hx_launch("sml_normq", 1, (unsigned) rows, 1024, (size_t) n * 4, st, &a);
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
// row: ng <= 64*NI, at most 8; SwiGLU and the fused prologue at most 4 and 2),
// RB rows per wave (more rows per wave for tall matrices, so ~2048+ waves
// carry the whole matrix at once while the loads a lane holds stay within
// RB*NI <= 16; SwiGLU takes 2 or 4: one or two gate/up pairs).
// SML_GEMV_RB / SML_GEMV_NI override for tuning sweeps.
// Launch shape of a GEMV: RB rows per wave, NI chunks per lane per pass.
// Measured on MI355X, occupancy beats bytes in flight per wave: at most 4
// chunks per lane (two passes over a 14336-wide row), and the fused-prologue
// kernels run 512-thread workgroups with 4 rows per wave and one chunk per
// pass, so that the fewest workgroups (each repeating the prologue) still
// cover the chip.
static void pick_shape(int rows, int cols, int nbits, int swiglu, int fused, int * rb, int * ni) {
    const int ng = cols / 32;
    const int imax = fused ? 1 : 4;
    int i = 1;
    while (i < imax && 64 * i < ng) i *= 2;
    int r = 1;
    if (fused) {
        r = 4;
        while (r > 1 && rows / (8 * r) < 192) r /= 2;
    } else {
        while (r < 4 && rows / (2 * r) >= 2048 && 2 * r * i <= 16) r *= 2;
        // the two-plane widths' heavier unpack runs better at one row per
        // wave with 4 chunks per pass (4096 x 14336: Q3 9.2 -> 8.5 us, Q5
        // 10.3 -> 9.8, Q8 13.0 -> 12.7; Q4 and Q6 stay at 2 rows)
        if ((nbits == 3 || nbits == 5 || nbits == 8) && r == 2 && i == 4 && !swiglu) r = 1;
        // and tall matrices at two rows per wave rather than four (14336 x
        // 4096: Q3 8.2 -> 7.6 us, Q5 9.2 -> 8.7)
        if ((nbits == 3 || nbits == 5) && r == 4 && !swiglu) r = 2;
        // Q2's long rows in one pass of 8 chunks at one row per wave (4096 x
        // 14336: 6.45 -> 6.21 us)
        if (nbits == 2 && !swiglu && r <= 2 && i == 4 && ng > 256) { r = 1; i = 8; }
    }
    const int fr = env_int("SML_GEMV_RB", 0), fi = env_int("SML_GEMV_NI", 0);
    if (fr == 1 || fr == 2 || fr == 4) r = fr;
    if ((fi == 1 || fi == 2 || fi == 4) && fi <= imax) i = fi;
    if (fi == 8 && !fused && !swiglu && nbits >= 2 && nbits <= 5 && r <= 2) i = 8;   // Q2-Q5, one or two rows per wave
    if (swiglu && r < 2) r = 2;
    if (!swiglu && !fused && r == 1 && i == 1) i = 2;
    *rb = r;
    *ni = i;
}

int gemv_fuse_max_cols(int hq) { (void) hq; return 4096; }

int op_gemv(hipStream_t st, const sml_hip_mat * m, const sml_hip_mat * up, int epi, const int8_t * q,
            const float * scale, const int32_t * sums, float * y, const float * bias, const float * up_bias,
            const float * resid, const gemv_fuse * fu) {
    const int swiglu = epi == SML_EPI_SWIGLU;
    if (swiglu != (up != NULL)) hx_failf("SwiGLU takes gate and up; other GEMVs one matrix");
    if (up && (up->nbits != m->nbits || up->cols != m->cols || up->k.rows != m->k.rows))
        hx_failf("SwiGLU needs gate and up of one shape and width");
    if (epi == SML_EPI_RESIDUAL && !resid) hx_failf("residual GEMV without a residual");
    sml_kgemv a;
    memset(&a, 0, sizeof a);
    const int nb = m->nbits, cols = m->cols;
    a.m[0] = m->k;
    a.m[0].y = y;
    a.m[0].bias = bias;
    if (up) { a.m[1] = up->k; a.m[1].y = y; a.m[1].bias = up_bias; }
    // the kernels address each plane and field array with 32-bit offsets
    if ((uint64_t) m->k.rows * (uint64_t) cols >= (1ull << 32)) hx_failf("matrix too large for one GEMV launch");
    a.cols = cols; a.epi = epi; a.total_rows = m->k.rows;
    a.q = q; a.scale = scale; a.sums = sums; a.resid = resid;
    const int am = fu && fu->x, hq = fu && fu->hq;
    if (am) {
        if (cols > gemv_fuse_max_cols(hq)) hx_failf("fused activation prologue takes at most %d columns", gemv_fuse_max_cols(hq));
        a.x = fu->x; a.norm_w = fu->norm_w; a.perm = fu->perm; a.eps = fu->eps;
    } else if (!q || !scale || !sums) {
        hx_failf("gemv without an activation");
    }
    // exact mode: the norm prologue and the h quantization have exact forms
    // at Q4/Q8 only, h quantization only behind the norm prologue
    if (g_exact && (((am || hq) && nb != 4 && nb != 8) || (hq && !am)))
        hx_failf("exact mode fuses the norm prologue (and h quantization behind it) into Q4/Q8 GEMVs only");
    if (hq) {
        if (!swiglu || a.total_rows % 32) hx_failf("h quantization needs SwiGLU rows in whole groups");
        a.hq = fu->hq; a.hscale = fu->hscale; a.hsums = fu->hsums;
    }
    if (fu && fu->amax) {
        if (swiglu || g_exact) hx_failf("the pick's first stage runs in one-matrix GEMVs outside exact mode");
        a.amax = fu->amax;
    }
    // LDS: int8 codes, per-group (s, s*sum), and the fused prologue's gather buffer
    const size_t lds = ((size_t) cols + 8u * (size_t) (cols / 32) + 15u) / 16u * 16u + (am && fu->perm ? 4u * (size_t) cols : 0u);
    char name[48];
    if (hq && g_exact) {
        // the exact SwiGLU (the reference's float order per row, 64 lanes a
        // row) with 32 outputs per workgroup: 8 waves of 4 gate/up pairs
        // (SML_GEMV_HXWG=1024: 16 waves of 2); the products' exchange buffer
        // (RB KB per wave) follows the codes and fields
        const int wg = env_int("SML_GEMV_HXWG", 512) == 1024 ? 1024 : 512, rb = wg == 1024 ? 4 : 8;
        const size_t base = ((size_t) cols + 8u * (size_t) (cols / 32) + 15u) / 16u * 16u;
        size_t xl = base + (size_t) (wg / 64) * rb * 64 * 16 + (size_t) (wg / 64) * rb * 4;
        if (xl < lds) xl = lds;
        if (xl > 160 * 1024) hx_failf("exact h-quantizing GEMV of %d columns needs %zu bytes of LDS", cols, xl);
        if (wg == 1024) snprintf(name, sizeof name, "sml_gemv_q%d_hxn1024_r4_i1", nb);
        else snprintf(name, sizeof name, "sml_gemv_q%d_hxn_r8_i1", nb);
        hx_launch(name, (unsigned) (a.total_rows / 32), 1, (unsigned) wg, xl, st, &a);
        return 0;
    }
    if (hq) {
        // 16 lanes per row: NI chunks per lane with 16*NI >= groups (a second
        // pass beyond 8)
        int ni = 2;
        const int fi = env_int("SML_GEMV_HNI", 0);
        if (fi == 2 || fi == 4) ni = fi;
        const int wg = am && env_int("SML_GEMV_HWG", 512) == 1024 && ni <= 4 ? 1024 : 512;
        if (a.total_rows % (wg / 16)) hx_failf("h quantization needs rows in whole workgroups");
        unsigned grid = (unsigned) (a.total_rows / (wg / 16));
        const int pw = env_int("SML_GEMV_PERSIST", 0);
        if (pw > 0 && nb == 4 && ni == 2 && wg == 512 && grid > (unsigned) (pw * hx.ncu)) {
            snprintf(name, sizeof name, "sml_gemv_q4_h%s_i2_p", am ? "n" : "");
            grid = (unsigned) (pw * hx.ncu);
        } else if (wg == 1024) snprintf(name, sizeof name, "sml_gemv_q%d_hn1024_i%d", nb, ni);
        else snprintf(name, sizeof name, "sml_gemv_q%d_h%s_i%d", nb, am ? "n" : "", ni);
        hx_launch(name, grid, 1, (unsigned) wg, lds, st, &a);
        return 0;
    }
    int rb, ni;
    pick_shape(a.total_rows, cols, nb, swiglu, am, &rb, &ni);
    if (g_exact && (nb == 4 || nb == 8)) {
        // the reference's float order: each group's products pass through LDS
        // (RB*NI KB per wave) to the lanes that run its superblock chains; with
        // the fused prologue (_xn) they reuse its gather buffer's LDS
        pick_shape(a.total_rows, cols, nb, swiglu, 0, &rb, &ni);
        // one-matrix forms with the prologue: 512 threads and the fast
        // path's row choice, one chunk per pass (6144 x 4096: 9.3 -> 6.9 us,
        // the prologue's share split over twice the threads)
        int wg = 256;
        if (am && !swiglu) {
            pick_shape(a.total_rows, cols, nb, 0, 1, &rb, &ni);
            wg = 512;
        }
        // (tuning, one-matrix forms: SML_GEMV_XRB 1/2/4/8 rows per wave,
        // SML_GEMV_XNI 1/2/4, SML_GEMV_XWG 256/512 threads; not every
        // combination is built)
        if (!swiglu) {
            const int xr = env_int("SML_GEMV_XRB", 0), xi = env_int("SML_GEMV_XNI", 0);
            if (xr == 1 || xr == 2 || xr == 4 || xr == 8) rb = xr;
            if (xi == 1 || xi == 2 || xi == 4) ni = xi;
            const int xw = env_int("SML_GEMV_XWG", 0);
            if (xw == 256 || xw == 512) wg = xw;
        }
        const size_t base = ((size_t) cols + 8u * (size_t) (cols / 32) + 15u) / 16u * 16u;
        size_t xl = base + (size_t) (wg / 64) * ni * rb * 64 * 16 + (size_t) (wg / 64) * rb * 4;
        while (xl > 160 * 1024 && ni > 1) {
            ni /= 2;
            xl = base + (size_t) (wg / 64) * ni * rb * 64 * 16 + (size_t) (wg / 64) * rb * 4;
        }
        if (xl < lds) xl = lds;
        if (xl > 160 * 1024) hx_failf("exact GEMV of %d columns needs %zu bytes of LDS", cols, xl);
        const int rows_per_wave = swiglu ? rb / 2 : rb;
        const int waves = (a.total_rows + rows_per_wave - 1) / rows_per_wave;
        if (swiglu) snprintf(name, sizeof name, "sml_gemv_q%d_s_r%d_i%d_x%s", nb, rb, ni, am ? "n" : "");
        else snprintf(name, sizeof name, "sml_gemv_q%d_r%d_i%d_x%s%s", nb, rb, ni, am ? "n" : "", wg == 512 ? "_w512" : "");
        hx_launch(name, (unsigned) ((waves + wg / 64 - 1) / (wg / 64)), 1, (unsigned) wg, xl, st, &a);
        return 0;
    }
    int wg = 256;
    if (!swiglu && am && env_int("SML_GEMV_WG", 512) != 256) {
        wg = env_int("SML_GEMV_WG", 512) == 1024 ? 1024 : 512;
        if (wg == 1024 && rb > 2) rb = 2;               // the 1024-thread forms hold 1 or 2 rows per wave
    }
    const int rows_per_wave = swiglu ? rb / 2 : rb;
    const int waves = (a.total_rows + rows_per_wave - 1) / rows_per_wave;
    unsigned grid = (unsigned) ((waves + wg / 64 - 1) / (wg / 64));
    const int blocks = (int) grid;                      // row blocks (amax pairs), persistent or not
    // persistent forms (SML_GEMV_PERSIST = workgroups per CU): Q4, plain or
    // with the 512-thread prologue
    const int pw = env_int("SML_GEMV_PERSIST", 0);
    const int pok = pw > 0 && nb == 4 && !swiglu && ni <= 4 && (wg == 256 ? !am : wg == 512 && ni == 1) &&
                    grid > (unsigned) (pw * hx.ncu);
    if (swiglu) snprintf(name, sizeof name, "sml_gemv_q%d_s%s_r%d_i%d", nb, am ? "n" : "", rb, ni);
    else if (wg != 256) snprintf(name, sizeof name, "sml_gemv_q%d_r%d_i%d_n%d%s", nb, rb, ni, wg, pok ? "_p" : "");
    else snprintf(name, sizeof name, "sml_gemv_q%d_r%d_i%d%s%s", nb, rb, ni, am ? "_n" : "", pok ? "_p" : "");
    if (pok) grid = (unsigned) (pw * hx.ncu);
    hx_launch(name, grid, 1, (unsigned) wg, lds, st, &a);
    return blocks;
}

int sml_hip_matvec(const sml_hip_mat * m, const int8_t * q, const float * scale, const int32_t * sums, float * y) {
    OP_BEGIN(-1);
    op_gemv(0, m, NULL, SML_EPI_STORE, q, scale, sums, y, NULL, NULL, NULL, NULL);
    HX_LEAVE();
    return 0;
}

int sml_hip_matvec_swiglu(const sml_hip_mat * gate, const sml_hip_mat * up, const int8_t * q,
                          const float * scale, const int32_t * sums, float * h) {
    OP_BEGIN(-1);
    op_gemv(0, gate, up, SML_EPI_SWIGLU, q, scale, sums, h, NULL, NULL, NULL, NULL);
    HX_LEAVE();
    return 0;
}

int sml_hip_matvec_normq(const sml_hip_mat * m, const float * x, const float * w, float eps, const int32_t * perm,
                         float * y) {
    OP_BEGIN(-1);
    if (!x) hx_failf("matvec_normq needs x");
    gemv_fuse fu;
    memset(&fu, 0, sizeof fu);
    fu.x = x; fu.norm_w = w; fu.eps = eps; fu.perm = perm;
    op_gemv(0, m, NULL, SML_EPI_STORE, NULL, NULL, NULL, y, NULL, NULL, NULL, &fu);
    HX_LEAVE();
    return 0;
}

int sml_hip_matvec_swiglu_fused(const sml_hip_mat * gate, const sml_hip_mat * up, const float * x, const float * w,
                                float eps, const int32_t * perm, const int8_t * q, const float * scale,
                                const int32_t * sums, float * h, int8_t * hq, float * hscale, int32_t * hsums) {
    OP_BEGIN(-1);
    if (hq && (!hscale || !hsums)) hx_failf("h quantization needs hq, hscale and hsums");
    gemv_fuse fu;
    memset(&fu, 0, sizeof fu);
    fu.x = x; fu.norm_w = w; fu.eps = eps; fu.perm = perm;
    fu.hq = hq; fu.hscale = hscale; fu.hsums = hsums;
    op_gemv(0, gate, up, SML_EPI_SWIGLU, q, scale, sums, h, NULL, NULL, NULL, &fu);
    HX_LEAVE();
    return 0;
}

int sml_hip_gemv_timeline(const sml_hip_mat * const * mats, int ncopy, const int8_t * q, const float * scale,
                          const int32_t * sums, float * y, int iters, unsigned long long * ts, int max_blocks) {
    OP_BEGIN(-1);
    if (!mats || ncopy < 1 || iters < 1 || !ts) hx_failf("gemv_timeline arguments");
    const sml_hip_mat * m0 = mats[0];
    if (m0->nbits != 4 || m0->k.rows % 8 || m0->cols % 256) hx_failf("the timeline GEMV takes Q4, rows in blocks of 8");
    const int blocks = m0->k.rows / 8;                  // 4 waves of 2 rows
    if (blocks > max_blocks) hx_failf("%d row blocks, room for %d", blocks, max_blocks);
    unsigned long long * d = hx_malloc((size_t) blocks * 5 * 8);
    jmp_buf * outer = hx.jb;
    jmp_buf jb;
    if (setjmp(jb)) { hipFree(d); longjmp(*outer, 1); }
    hx.jb = &jb;
    const size_t lds = ((size_t) m0->cols + 8u * (size_t) (m0->cols / 32) + 15u) / 16u * 16u;
    for (int i = 0; i < iters; i++) {
        const sml_hip_mat * m = mats[i % ncopy];
        if (m->nbits != 4 || m->k.rows != m0->k.rows || m->cols != m0->cols) hx_failf("gemv_timeline: matrices differ");
        sml_kgemv a;
        memset(&a, 0, sizeof a);
        a.m[0] = m->k;
        a.m[0].y = y;
        a.cols = m->cols; a.epi = SML_EPI_STORE; a.total_rows = m->k.rows;
        a.q = q; a.scale = scale; a.sums = sums; a.ts = d;
        hx_launch("sml_gemv_q4_r2_i4_ts", (unsigned) blocks, 1, 256, lds, 0, &a);
    }
    HX(hipMemcpy(ts, d, (size_t) blocks * 5 * 8, hipMemcpyDeviceToHost));
    hx.jb = outer;
    HX(hipFree(d));
    HX_LEAVE();
    return blocks;
}

int sml_hip_time_matvec(const sml_hip_mat * const * mats, int ncopy, const int8_t * q, const float * scale,
                        const int32_t * sums, float * y, int iters, float * ms_total) {
    OP_BEGIN(-1);
    hipEvent_t e0, e1;
    HX(hipEventCreate(&e0));
    HX(hipEventCreate(&e1));
    HX(hipEventRecord(e0, 0));
    for (int i = 0; i < iters; i++) op_gemv(0, mats[i % ncopy], NULL, SML_EPI_STORE, q, scale, sums, y, NULL, NULL, NULL, NULL);
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
    op_embed_rows(st, m, tok, pos, 1, perm, x);
}

void op_embed_rows(hipStream_t st, const sml_hip_mat * m, const int32_t * tok, const int32_t * pos, int rows,
                   const int32_t * perm, float * x) {
    if (pos && rows != 1) hx_failf("a batch of embeddings takes its tokens directly");
    sml_kembed a;
    memset(&a, 0, sizeof a);
    a.m = m->k; a.nbits = m->nbits; a.cols = m->cols; a.tok = tok; a.pos = pos; a.perm = perm; a.x = x;
    hx_launch("sml_embed", (unsigned) ((m->cols / 32 + 63) / 64), (unsigned) rows, 64, 0, st, &a);
}

int sml_hip_embed(const sml_hip_mat * m, const int32_t * tok, const int32_t * perm, float * x) {
    OP_BEGIN(-1);
    op_embed(0, m, tok, NULL, perm, x);
    HX_LEAVE();
    return 0;
}

#define ATTN_CHUNK 128

#define ATTN_MIN_CHUNK 32         // the shortest split a decode launch takes
size_t sml_hip_attn_part_floats(int n_head, int hd, int n_ctx) {
    const int ns = (n_ctx + ATTN_MIN_CHUNK - 1) / ATTN_MIN_CHUNK;
    return (size_t) n_head * ns * (size_t) (hd + 2);
}

// Positions per split of the 8-wave decode kernels (and the exact prompt
// kernel, which must split as decoding does): 128, or 64 where KV heads x
// splits of 128 leave most CUs idle. Qwen2.5-1.5B shape (2 KV heads, 4096
// positions), 128 / 64 / 32: decode 1097 / 1112 / 1068 tokens/s, a 2048-id
// prompt at level 1 2405 / 2598 / 2665. SML_ATTN_CHUNK overrides (32, 64 or
// 128).
// a decode/prompt attention kernel's name: base, _s<ch> for splits other
// than 128, _d64 for head_dim 64, _r<query heads per workgroup>
static void attn_name(char * name, size_t n, const char * base, int ch, int hd, int rep) {
    char sp[16] = "";
    if (ch != ATTN_CHUNK) snprintf(sp, sizeof sp, "_s%d", ch);
    snprintf(name, n, "%s%s%s_r%d", base, sp, hd == 64 ? "_d64" : "", rep);
}

static int attn_split(int n_kv, int n_ctx, int hd) {
    int ch = ATTN_CHUNK;
    while (ch > 64 && (long) n_kv * ((n_ctx + ch - 1) / ch) < 256) ch /= 2;
    const int ce = env_int("SML_ATTN_CHUNK", 0);
    if (ce == 32 || ce == 64 || ce == 128) ch = ce;
    if (hd == 64 && ch < 64) ch = 64;               // head_dim 64: 64 positions per round of 8 waves
    return ch;
}

void op_attention(hipStream_t st, const float * q, const float * k, const float * v, uint16_t * kc, uint16_t * vc,
                  const float * cos_t, const float * sin_t, const int32_t * pos, int n_head, int n_kv,
                  int hd, int n_ctx, int n_pos, float * part, float * out, int8_t * q_out, float * s_out,
                  int32_t * u_out, int * cnt) {
    if ((hd != 128 && hd != 64) || n_kv <= 0 || n_head % n_kv || n_head / n_kv > 8)
        hx_failf("attention shape (heads %d/%d, head_dim %d) not supported", n_head, n_kv, hd);
    if (hd != 128 && (g_exact || cnt)) hx_failf("head_dim %d: exact mode and the folded merge take head_dim 128", hd);
    if (n_pos < 1 || n_pos > n_ctx) hx_failf("attention over %d of %d positions", n_pos, n_ctx);
    if (g_exact) {
        // the reference's order: RoPE, the KV write and the scores over
        // splits of 128 positions, then a workgroup per query head for the
        // softmax and P.V chains (quantizing its output when asked); the
        // scores pass through the partials buffer ([n_head][n_ctx] floats)
        if (n_ctx > 16384) hx_failf("exact attention holds at most 16384 positions");
        if (sml_hip_attn_part_floats(n_head, hd, n_ctx) < (size_t) n_head * n_ctx)
            hx_failf("exact attention needs %d x %d floats of scores", n_head, n_ctx);
        sml_kattnx x;
        memset(&x, 0, sizeof x);
        x.q = q; x.k = k; x.v = v; x.kc = kc; x.vc = vc; x.cos_t = cos_t; x.sin_t = sin_t;
        x.pos = pos; x.sc = part; x.out = out; x.q_out = q_out; x.s_out = s_out; x.u_out = u_out;
        x.n_head = n_head; x.n_kv = n_kv; x.n_ctx = n_ctx;
        x.inv = 1.0f / __builtin_sqrtf((float) hd);
        hx_launch("sml_attnx_scores", (unsigned) ((n_pos + 127) / 128), (unsigned) n_kv, 256, 0, st, &x);
        // the weights and three 64-position fp16 V tiles
        const size_t lds = (size_t) ((n_ctx + 3) & ~3) * 4 + (size_t) 3 * 64 * 128 * 2;
        hx_launch("sml_attnx_pv", (unsigned) n_head, 1, 512, lds, st, &x);
        return;
    }
    // one sequence: the 8-wave kernel over attn_split positions, the split the
    // exact prompt kernel (sml_attnc8) takes, so prompts read at level 1 equal
    // stepping bit for bit (SML_ATTN_WAVES applies to the batched step only)
    // splits past n_pos are not launched: the merge of the ones that are
    // equals the merge of all (empty splits add exact zeros)
    const int aw = 8;
    const int ch = attn_split(n_kv, n_ctx, hd);
    const int ns = (n_pos + ch - 1) / ch;
    sml_kattn a;
    memset(&a, 0, sizeof a);
    a.q = q; a.k = k; a.v = v; a.kcache = kc; a.vcache = vc; a.cos_t = cos_t; a.sin_t = sin_t; a.pos = pos;
    a.part = part; a.out = out; a.q_out = q_out; a.s_out = s_out; a.u_out = u_out;
    a.n_head = n_head; a.n_kv = n_kv; a.nsplit = ns;
    a.inv = 1.0f / __builtin_sqrtf((float) hd);
    a.cnt = cnt;                                      // the merge runs in the last split of each kv head
    // query-head subsets per kv head: models with few kv heads launch few,
    // heavy workgroups (Qwen2.5-1.5B shape: 2 kv heads x 64 splits), so the
    // kv head's query heads are shared out over up to 256 workgroups, which
    // read the same K/V tiles (each head's arithmetic is unchanged). That
    // shape at 4096 positions, subsets 1 / 2 / 3 / 6: 1096 / 1160 / 1128 /
    // 1096 tokens/s; Llama-3-8B shape (8 x 32 workgroups already): 1 best.
    // SML_ATTN_SUB overrides; the folded merge counts whole kv heads.
    const int rep = n_head / n_kv;
    int nsub = 1;
    for (int d = 2; d <= rep; d++)
        if (rep % d == 0 && (long) n_kv * ns * d <= 256) nsub = d;
    const int se = env_int("SML_ATTN_SUB", 0);
    if (se >= 1 && rep % se == 0) nsub = se;
    if (cnt) nsub = 1;
    a.nsub = nsub;
    char name[40];
    attn_name(name, sizeof name, "sml_attn8", ch, hd, n_head / n_kv / nsub);
    hx_launch(name, (unsigned) ns, (unsigned) (n_kv * nsub), (unsigned) (64 * aw), 0, st, &a);
    if (!cnt) hx_launch(hd == 64 ? "sml_attn_merge_d64" : "sml_attn_merge", (unsigned) n_head, 1, (unsigned) hd, 0, st, &a);
}

// LDS of the prompt flash attention (sml_attnf): two stages of a 64-position
// K tile (272 bytes a row) and its V transposed (128 dims x 144 bytes)
#define ATTNF_LDS (2 * (64 * 272 + 128 * 144))
void op_attention_batch(hipStream_t st, const float * qkv, int qkv_stride, uint16_t * const * kc_slots,
                        uint16_t * const * vc_slots, const int32_t * slot, size_t layer_off, const float * cos_t,
                        const float * sin_t, const int32_t * pos, int nseq, int n_head, int n_kv, int hd, int n_ctx,
                        int n_pos, float * part, float * out, int8_t * q_out, float * s_out, int32_t * u_out,
                        int causal, int exact, int q256) {
    if ((hd != 128 && hd != 64) || n_kv <= 0 || n_head % n_kv || n_head / n_kv > 8)
        hx_failf("attention shape (heads %d/%d, head_dim %d) not supported", n_head, n_kv, hd);
    if (n_pos < 1 || n_pos > n_ctx) hx_failf("attention over %d of %d positions", n_pos, n_ctx);
    if (q_out && q256 && (causal || n_head % 2 || hd != 128))
        hx_failf("the merge quantizes per 256 only decode steps of an even head count of head_dim 128 (%d heads, %d)",
                 n_head, hd);
    // head_dim 64 reads level-2 prompts with the level-1 kernel (the matrix-core
    // and wave-per-position prompt kernels are head_dim 128), at splits of
    // 128 as the level-2 partials are sized
    const int c2_d64 = causal == 2 && hd == 64;
    if (c2_d64) causal = 1;
    if (nseq < 1 || nseq > 65535) hx_failf("attention batch of %d", nseq);
    const int aw = env_int("SML_ATTN_WAVES", nseq >= 4 && !exact ? 4 : 8) == 4 ? 4 : 8;
    // the 8-wave kernels split as decoding does (attn_split); the 4-wave and
    // wave-per-position kernels run splits of 128
    const int bch = env_int("SML_ATTN_BCH", ATTN_CHUNK) == 64 && hd == 128 ? 64 : ATTN_CHUNK;
    const int ch = causal == 2 || c2_d64 ? ATTN_CHUNK : causal == 0 && aw == 4 ? bch : attn_split(n_kv, n_ctx, hd);
    const int ns = (n_pos + ch - 1) / ch;             // splits past n_pos: not launched
    sml_kattn a;
    memset(&a, 0, sizeof a);
    a.q = qkv; a.k = qkv + (size_t) n_head * hd; a.v = a.k + (size_t) n_kv * hd;
    a.qkv_stride = qkv_stride; a.kc_slots = kc_slots; a.vc_slots = vc_slots; a.slot = slot; a.layer_off = layer_off;
    a.cos_t = cos_t; a.sin_t = sin_t; a.pos = pos;
    a.part = part; a.out = out; a.q_out = q_out; a.s_out = s_out; a.u_out = u_out;
    a.n_head = n_head; a.n_kv = n_kv; a.nsplit = ns;
    a.inv = 1.0f / __builtin_sqrtf((float) hd);
    a.kv_written = causal != 0;
    if (causal) {
        if (n_kv > 8) hx_failf("causal attention takes at most 8 kv heads");
        hx_launch(hd == 64 ? "sml_ropekv_d64" : "sml_ropekv", (unsigned) nseq, 1, (unsigned) (hd / 8 * n_kv), 0, st, &a);
    }
    char name[40];
    // many sequences give many workgroups: 4-wave ones, two per CU, then
    // measured faster (16 sequences at ~1k positions: 5.6 against 6.8 ms per
    // step); one sequence, and any step that must equal decoding alone bit
    // for bit (exact), keeps the decode kernel's 8 waves per split
    // causal entries (positions of one sequence) share each split's K/V tile
    // in groups of tpw per workgroup (sml_attnc8); the arithmetic per entry is
    // the one-entry kernel's
    a.nseq = nseq;
    a.tpw = causal ? env_int("SML_ATTN_TPW", 16) : 1;
    if (a.tpw < 1 || a.tpw > 16) a.tpw = 1;
    if (causal == 2 && env_int("SML_ATTN_FLASH", 1)) {
        // MFMA flash form: 16 entries x one kv head per workgroup (a wave per
        // query head), the KV range cut into splits only as far as the grid
        // needs workgroups (then merged); splits of a multiple of 64
        // positions, at most the partial buffer's ceil(n_ctx / 128)
        if (q_out) hx_failf("flash prompt attention does not quantize its output");
        const int rep = n_head / n_kv, nqb = (nseq + 15) / 16;
        const int maxs = (n_ctx + 127) / 128;
        int ns = 1;
        while (ns * 2 <= maxs && ns < 64 && (long) nqb * n_kv * ns < 2L * hx.ncu) ns *= 2;
        a.nsplit = ns;
        a.fchunk = ((n_ctx + ns - 1) / ns + 63) / 64 * 64;
        snprintf(name, sizeof name, "sml_attnf_r%d", rep);
        hx_launch3(name, (unsigned) nqb, (unsigned) n_kv, (unsigned) ns, (unsigned) (64 * rep), ATTNF_LDS, st, &a);
        if (ns > 1) hx_launch3("sml_attn_merge", (unsigned) n_head, 1, (unsigned) nseq, (unsigned) hd, 0, st, &a);
        return;
    }
    if (causal == 2) {
        // a wave per position over an LDS tile (16 positions per workgroup)
        const int rep = n_head / n_kv;
        const size_t lds = (size_t) ATTN_CHUNK * (128 + 8) * 2 + (size_t) ATTN_CHUNK * 128 * 2 +
                           2 * (size_t) 8 * rep * 128 * 4;
        snprintf(name, sizeof name, "sml_attnw_r%d", rep);
        hx_launch3(name, (unsigned) ns, (unsigned) n_kv, (unsigned) ((nseq + 15) / 16), 512, lds, st, &a);
        hx_launch3("sml_attn_merge", (unsigned) n_head, 1, (unsigned) nseq, (unsigned) hd, 0, st, &a);
        return;
    }
    const int nt = causal ? 512 : 64 * aw;
    attn_name(name, sizeof name, a.tpw > 1 || causal ? "sml_attnc8" : aw == 4 ? "sml_attn" : "sml_attn8",
              ch, hd, n_head / n_kv);
    // the 4-wave decode split with its inputs spread over the workgroup
    // (sml_attnb: the same values, half the registers); SML_ATTNB=0 keeps
    // the one-entry body
    if (!causal && aw == 4 && hd == 128 && ch == ATTN_CHUNK && env_int("SML_ATTNB", 1)) {
        snprintf(name, sizeof name, "sml_attnb_r%d", n_head / n_kv);
        hx_launch3(name, (unsigned) n_kv, (unsigned) ns, (unsigned) nseq, (unsigned) nt, 0, st, &a);
    } else {
        hx_launch3(name, (unsigned) ns, (unsigned) n_kv, (unsigned) ((nseq + a.tpw - 1) / a.tpw), (unsigned) nt, 0,
                   st, &a);
    }
    if (q_out && q256) hx_launch3("sml_attn_merge_sb", (unsigned) n_head / 2, 1, (unsigned) nseq, 256, 0, st, &a);
    else hx_launch3(hd == 64 ? "sml_attn_merge_d64" : "sml_attn_merge", (unsigned) n_head, 1, (unsigned) nseq,
                    (unsigned) hd, 0, st, &a);
}

// Exact mode's batched prompt rows: row b = position pos[b] of one sequence,
// its q/k/v at b * qkv_stride of qkv. RoPE and the fp16 K/V write of every
// row first (sml_ropekv: the decode kernels' rotation and rounding), then
// the reference-order scores and P.V of every row (sml_attnx_scores /
// sml_attnx_pv with a row dimension), as decoding each position computes
// them. sc: nrows * n_head * n_ctx floats of scores.
void op_attention_rows_exact(hipStream_t st, const float * qkv, int qkv_stride, uint16_t * kc, uint16_t * vc,
                             const float * cos_t, const float * sin_t, const int32_t * pos, int nrows, int n_head,
                             int n_kv, int n_ctx, int n_pos, float * sc, float * out, int8_t * q_out, float * s_out,
                             int32_t * u_out) {
    const int hd = 128;                               // exact mode's head size
    if (n_kv <= 0 || n_head % n_kv || n_head / n_kv > 8 || n_kv > 8)
        hx_failf("attention shape (heads %d/%d) not supported", n_head, n_kv);
    if (nrows < 1 || nrows > 65535 || n_pos < 1 || n_pos > n_ctx || n_ctx > 16384)
        hx_failf("exact attention rows: %d rows over %d of %d positions", nrows, n_pos, n_ctx);
    sml_kattn r;
    memset(&r, 0, sizeof r);
    r.q = qkv; r.k = qkv + (size_t) n_head * hd; r.v = r.k + (size_t) n_kv * hd;
    r.qkv_stride = qkv_stride; r.kcache = kc; r.vcache = vc; r.cos_t = cos_t; r.sin_t = sin_t; r.pos = pos;
    r.n_head = n_head; r.n_kv = n_kv;
    hx_launch("sml_ropekv", (unsigned) nrows, 1, (unsigned) (hd / 8 * n_kv), 0, st, &r);
    sml_kattnx x;
    memset(&x, 0, sizeof x);
    x.q = r.q; x.k = r.k; x.v = r.v; x.kc = kc; x.vc = vc; x.cos_t = cos_t; x.sin_t = sin_t;
    x.pos = pos; x.sc = sc; x.out = out; x.q_out = q_out; x.s_out = s_out; x.u_out = u_out;
    x.n_head = n_head; x.n_kv = n_kv; x.n_ctx = n_ctx;
    x.inv = 1.0f / __builtin_sqrtf((float) hd);
    x.qkv_stride = qkv_stride;
    x.kv_written = 1;
    hx_launch3("sml_attnx_scores", (unsigned) ((n_pos + 127) / 128), (unsigned) n_kv, (unsigned) nrows, 256, 0, st, &x);
    const size_t lds = (size_t) ((n_ctx + 3) & ~3) * 4 + (size_t) 3 * 64 * 128 * 2;
    hx_launch3("sml_attnx_pv", (unsigned) n_head, (unsigned) nrows, 1, 512, lds, st, &x);
}

int sml_hip_attention(float * q, const float * k, const float * v, uint16_t * kcache, uint16_t * vcache,
                      const float * cos_t, const float * sin_t, const int32_t * pos,
                      int n_head, int n_kv, int hd, int n_ctx, float * part, float * out) {
    OP_BEGIN(-1);
    op_attention(0, q, k, v, kcache, vcache, cos_t, sin_t, pos, n_head, n_kv, hd, n_ctx, n_ctx, part, out,
                 NULL, NULL, NULL, NULL);
    HX_LEAVE();
    return 0;
}

int sml_hip_attention_prompt(const float * qkv, int n_rows, int pos0, uint16_t * kcache, uint16_t * vcache,
                             const float * cos_t, const float * sin_t, int n_head, int n_kv, int hd, int n_ctx,
                             float * part, float * out) {
    OP_BEGIN(-1);
    if ((hd != 128 && hd != 64) || n_kv <= 0 || n_kv > 8 || n_head % n_kv || n_head / n_kv > 8)
        hx_failf("prompt attention shape (heads %d/%d, head_dim %d) not supported", n_head, n_kv, hd);
    if (n_rows < 1 || n_rows > 65535 || pos0 < 0 || pos0 + n_rows > n_ctx)
        hx_failf("prompt attention over positions %d..%d of %d", pos0, pos0 + n_rows - 1, n_ctx);
    // device tables: the one sequence's cache pointers, every row's slot (0)
    // and position
    const size_t tb = 2 * sizeof(void *) + (size_t) n_rows * 8;
    char * h = (char *) calloc(1, tb);
    if (!h) hx_failf("host allocation");
    ((void **) h)[0] = kcache;
    ((void **) h)[1] = vcache;
    int32_t * hp = (int32_t *) (h + 2 * sizeof(void *) + (size_t) n_rows * 4);
    for (int b = 0; b < n_rows; b++) hp[b] = pos0 + b;
    void * t = NULL;
    if (hipMalloc(&t, tb) != hipSuccess || hipMemcpy(t, h, tb, hipMemcpyHostToDevice) != hipSuccess) {
        free(h);
        if (t) hipFree(t);
        hx_failf("prompt attention tables");
    }
    free(h);
    uint16_t * const * slots = (uint16_t * const *) t;
    const int32_t * slot = (const int32_t *) ((char *) t + 2 * sizeof(void *));
    jmp_buf * outer = hx.jb;
    jmp_buf jb;
    if (setjmp(jb)) {
        hipFree(t);
        longjmp(*outer, 1);
    }
    hx.jb = &jb;
    op_attention_batch(0, qkv, (n_head + 2 * n_kv) * hd, slots, slots + 1, slot, 0, cos_t, sin_t, slot + n_rows,
                       n_rows, n_head, n_kv, hd, n_ctx, pos0 + n_rows, part, out, NULL, NULL, NULL, 2, 0, 0);
    HX(hipDeviceSynchronize());
    hx.jb = outer;
    HX(hipFree(t));
    HX_LEAVE();
    return 0;
}

int sml_hip_softmax_sum(const float * x, int n, float * out) {
    OP_BEGIN(-1);
    if (n < 0 || n > 16384) hx_failf("softmax sum of %d values (0..16384)", n);
    sml_ksum a;
    a.x = x; a.out = out; a.n = n;
    hx_launch("sml_sum_seg", 1, 1, 512, (size_t) (n > 0 ? n : 1) * 4, 0, &a);
    HX_LEAVE();
    return 0;
}

int sml_hip_attention_q(float * q, const float * k, const float * v, uint16_t * kcache, uint16_t * vcache,
                        const float * cos_t, const float * sin_t, const int32_t * pos,
                        int n_head, int n_kv, int hd, int n_ctx, float * part, float * out,
                        int8_t * q_out, float * s_out, int32_t * u_out) {
    OP_BEGIN(-1);
    if (!q_out || !s_out || !u_out) hx_failf("attention_q needs its three outputs");
    op_attention(0, q, k, v, kcache, vcache, cos_t, sin_t, pos, n_head, n_kv, hd, n_ctx, n_ctx, part, out,
                 q_out, s_out, u_out, NULL);
    HX_LEAVE();
    return 0;
}

void op_argmax(hipStream_t st, const float * logits, int n, int32_t * tok, int32_t * pos, int32_t * hist,
               int hist_n, int2 * part) {
    sml_kargmax a;
    memset(&a, 0, sizeof a);
    a.logits = logits; a.n = n; a.tok = tok; a.pos = pos; a.hist = hist; a.hist_n = hist_n;
    if (part && n >= ARGMAX_TWO_STAGE_MIN) {
        // a vocabulary's worth: one float4 per thread over many workgroups,
        // then one workgroup over their pairs (one workgroup alone spends
        // ~15 us on 128k logits)
        const int words = n / 4 + 1;
        int np = (words + 255) / 256;
        if (np > ARGMAX_MAX_PARTS) np = ARGMAX_MAX_PARTS;
        a.part = part; a.nparts = np;
        hx_launch("sml_argmax_part", (unsigned) np, 1, 256, 0, st, &a);
    }
    hx_launch("sml_argmax", 1, 1, 1024, 0, st, &a);
}

void op_argmax_pairs(hipStream_t st, const int2 * pairs, int nparts, const float * logits, int32_t * tok,
                     int32_t * pos, int32_t * hist, int hist_n) {
    if (nparts < 1) hx_failf("greedy pick over %d pairs", nparts);
    sml_kargmax a;
    memset(&a, 0, sizeof a);
    a.logits = logits; a.tok = tok; a.pos = pos; a.hist = hist; a.hist_n = hist_n;
    a.part = (int2 *) pairs; a.nparts = nparts;
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
    int2 * part = n >= ARGMAX_TWO_STAGE_MIN ? hx_malloc((size_t) ARGMAX_MAX_PARTS * sizeof(int2)) : NULL;
    op_argmax(0, logits, n, tok, NULL, NULL, 0, part);
    if (part) {
        HX(hipStreamSynchronize(0));
        HX(hipFree(part));
    }
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

// ------------------------------------------------------------ GPTQ-style 4-bit

#define GPTQ_GROUPS_PER_WG 8     // waves (one group of 128 inputs each) per sml_gptq_gemv workgroup

struct sml_hip_gptq {
    uint32_t * qweight, * qzeros;
    uint16_t * scales;
    float * part;
    int * cnt;                   // output blocks' counters (after the partials), zero between launches
    int32_t * perm;              // desc_act: device input i is input perm[i], or NULL
    int rows, cols, zero_add;
    size_t bytes;
};

sml_hip_gptq * sml_hip_gptq_upload(const int32_t * qweight, const int32_t * qzeros, const uint16_t * scales,
                                   int rows, int cols, int group, int zero_add) {
    OP_BEGIN(NULL);
    if (rows <= 0 || cols <= 0 || rows % 8 || cols % 128 || group != 128 || zero_add < 0 || zero_add > 1)
        hx_failf("GPTQ matrix %dx%d group %d: rows must be a multiple of 8, cols of 128, group 128", rows, cols, group);
    sml_hip_gptq * m = calloc(1, sizeof *m);
    if (!m) hx_failf("out of host memory");
    jmp_buf * outer = hx.jb;
    jmp_buf jb;
    if (setjmp(jb)) {
        hx.jb = outer;
        hipFree(m->qweight); hipFree(m->qzeros); hipFree(m->scales); hipFree(m->part);
        free(m);
        longjmp(*outer, 1);
    }
    hx.jb = &jb;
    const size_t R = (size_t) rows, ng = (size_t) cols / 128, nslice = (ng + GPTQ_GROUPS_PER_WG - 1) / GPTQ_GROUPS_PER_WG;
    const size_t bw = (size_t) cols / 8 * R * 4, bz = ng * (R / 8) * 4, bs = ng * R * 2;
    m->qweight = hx_malloc(bw);
    m->qzeros = hx_malloc(bz);
    m->scales = hx_malloc(bs);
    // the partials, then one counter per output block of 128 (the
    // 2-per-lane launch's; the 4-per-lane one uses the first half)
    const size_t nblk = (R + 127) / 128;
    m->part = hx_malloc(nslice * R * 4 + nblk * 4);
    m->cnt = (int *) (m->part + nslice * R);
    HX(hipMemset(m->cnt, 0, nblk * 4));
    HX(hipMemcpy(m->qweight, qweight, bw, hipMemcpyHostToDevice));
    HX(hipMemcpy(m->qzeros, qzeros, bz, hipMemcpyHostToDevice));
    HX(hipMemcpy(m->scales, scales, bs, hipMemcpyHostToDevice));
    hx.jb = outer;
    m->rows = rows; m->cols = cols; m->zero_add = zero_add;
    m->bytes = bw + bz + bs;
    HX_LEAVE();
    return m;
}

// AWQ (tooling/sml_unpack.py:78,100-118): qweight int32 [cols][rows/8] packs
// 8 outputs per word, output 8j+k in nibble awq_nibble[k]; qzeros the same
// way over [cols/group][rows/8], or absent (zero 8); zeros stored as they
// are. Repacked on the host into the GPTQ device layout (codes along the
// input, zeros in natural nibble order, zero_add 0), whose kernels then run
// it unchanged: codes and zeros are moved, never recomputed.
static const int awq_nibble[8] = { 0, 4, 1, 5, 2, 6, 3, 7 };

sml_hip_gptq * sml_hip_awq_upload(const int32_t * qweight, const int32_t * qzeros, const uint16_t * scales,
                                  int rows, int cols, int group) {
    if (rows <= 0 || cols <= 0 || rows % 8 || cols % 128 || group != 128 || !qweight || !scales) {
        snprintf(hx.err, sizeof hx.err, "AWQ matrix %dx%d group %d: rows must be a multiple of 8, cols of 128, "
                 "group 128", rows, cols, group);
        return NULL;
    }
    const size_t R = (size_t) rows, C = (size_t) cols, ng = C / 128;
    uint32_t * gw = calloc(C / 8 * R, 4);
    uint32_t * gz = calloc(ng * (R / 8), 4);
    if (!gw || !gz) {
        free(gw); free(gz);
        snprintf(hx.err, sizeof hx.err, "out of host memory");
        return NULL;
    }
    for (size_t k = 0; k < C; k++)
        for (size_t j = 0; j < R / 8; j++) {
            const uint32_t w = (uint32_t) qweight[k * (R / 8) + j];
            for (int i = 0; i < 8; i++)
                gw[(k / 8) * R + 8 * j + i] |= ((w >> (4 * awq_nibble[i])) & 15u) << (4 * (k % 8));
        }
    for (size_t g = 0; g < ng; g++)
        for (size_t j = 0; j < R / 8; j++) {
            const uint32_t z = qzeros ? (uint32_t) qzeros[g * (R / 8) + j] : 0x88888888u;
            uint32_t o = 0;
            for (int i = 0; i < 8; i++) o |= ((z >> (4 * awq_nibble[i])) & 15u) << (4 * i);
            gz[g * (R / 8) + j] = o;
        }
    sml_hip_gptq * m = sml_hip_gptq_upload((const int32_t *) gw, (const int32_t *) gz, scales, rows, cols, group, 0);
    free(gw);
    free(gz);
    return m;
}

// The column order of a desc_act matrix into HBM (0, or -1 with a reason).
static int gptq_perm_upload(sml_hip_gptq * m, const int32_t * perm, size_t n) {
    OP_BEGIN(-1);
    m->perm = hx_malloc(n * 4);
    HX(hipMemcpy(m->perm, perm, n * 4, hipMemcpyHostToDevice));
    HX_LEAVE();
    return 0;
}

// desc_act (tooling/sml_unpack.py:90-93): g_idx[k] is input k's group,
// groups of `group` inputs in activation order. The input columns are
// reordered on the host, stably by g_idx, so each group's codes are the
// contiguous 128 the GEMV reads (moved, never recomputed), and the GEMV
// gathers x through the same order; scales and zeros stay per group. Every
// group must hold exactly `group` inputs (as GPTQ's desc_act writes them).
sml_hip_gptq * sml_hip_gptq_upload_gidx(const int32_t * qweight, const int32_t * qzeros, const uint16_t * scales,
                                        const int32_t * g_idx, int rows, int cols, int group, int zero_add) {
    if (!g_idx) return sml_hip_gptq_upload(qweight, qzeros, scales, rows, cols, group, zero_add);
    if (rows <= 0 || cols <= 0 || rows % 8 || cols % 128 || group != 128 || !qweight) {
        snprintf(hx.err, sizeof hx.err, "GPTQ matrix %dx%d group %d: rows must be a multiple of 8, cols of 128, "
                 "group 128", rows, cols, group);
        return NULL;
    }
    const size_t R = (size_t) rows, C = (size_t) cols, ng = C / 128;
    int32_t * perm = malloc(C * 4);
    size_t * fill = calloc(ng, sizeof(size_t));
    uint32_t * qw = calloc(C / 8 * R, 4);
    if (!perm || !fill || !qw) {
        free(perm); free(fill); free(qw);
        snprintf(hx.err, sizeof hx.err, "out of host memory");
        return NULL;
    }
    int ident = 1, bad = 0;
    for (size_t k = 0; k < C && !bad; k++) {
        const int32_t g = g_idx[k];
        if (g < 0 || (size_t) g >= ng || fill[g] >= 128) bad = 1;
        else {
            perm[(size_t) g * 128 + fill[g]++] = (int32_t) k;
            ident &= (size_t) g == k / 128;
        }
    }
    if (bad) {
        free(perm); free(fill); free(qw);
        snprintf(hx.err, sizeof hx.err, "g_idx: every group must hold exactly %d of the %d inputs", group, cols);
        return NULL;
    }
    free(fill);
    for (size_t i = 0; i < C; i++) {
        const size_t k = (size_t) perm[i];
        const uint32_t * src = (const uint32_t *) qweight + (k / 8) * R;
        uint32_t * dst = qw + (i / 8) * R;
        const unsigned ss = 4u * (unsigned) (k % 8), ds = 4u * (unsigned) (i % 8);
        for (size_t n = 0; n < R; n++) dst[n] |= ((src[n] >> ss) & 15u) << ds;
    }
    sml_hip_gptq * m = sml_hip_gptq_upload((const int32_t *) qw, qzeros, scales, rows, cols, group, zero_add);
    free(qw);
    if (m && !ident && gptq_perm_upload(m, perm, C) != 0) {
        sml_hip_gptq_free(m);
        m = NULL;
    }
    free(perm);
    return m;
}

void sml_hip_gptq_free(sml_hip_gptq * m) {
    HX_ENTRY();
    if (m) {
        HX(hipFree(m->qweight)); HX(hipFree(m->qzeros)); HX(hipFree(m->scales)); HX(hipFree(m->part));
        if (m->perm) HX(hipFree(m->perm));
        free(m);
    }
    HX_LEAVE();
}

size_t sml_hip_gptq_bytes(const sml_hip_gptq * m) { return m ? m->bytes : 0; }

static void op_gptq(hipStream_t st, const sml_hip_gptq * m, const float * x, float * y) {
    sml_kgptq a;
    memset(&a, 0, sizeof a);
    a.qweight = m->qweight; a.qzeros = m->qzeros; a.scales = m->scales;
    a.x = x; a.part = m->part; a.y = y; a.perm = m->perm;
    a.rows = m->rows; a.cols = m->cols; a.zero_add = m->zero_add;
    a.nslice = (m->cols / 128 + GPTQ_GROUPS_PER_WG - 1) / GPTQ_GROUPS_PER_WG;
    // 2 outputs per lane (128 per wave): twice the waves of 4 per lane, so
    // more of the weight stream overlaps the float dot products (4096 x 14336:
    // 14.8 -> 11.4 us; 1 per lane measured the same as 2)
    const int opl = env_int("SML_GPTQ_OPL", 2) == 4 ? 4 : 2;
    // the slices' sum runs in each output block's last workgroup
    // (SML_GPTQ_FOLD=0: in a second launch, sml_gptq_reduce; the same bits)
    const int fold = env_int("SML_GPTQ_FOLD", 1) != 0;
    a.cnt = fold ? m->cnt : NULL;
    // the integer form (SML_GPTQ_I8=0: the float dot products; 4096 x 14336
    // 11.1 -> 9.4 us, 14336 x 4096 10.9 -> 8.7)
    if (env_int("SML_GPTQ_I8", 1)) {
        hx_launch("sml_gptq_gemv_i8", (unsigned) ((m->rows + 127) / 128), (unsigned) a.nslice,
                  64 * GPTQ_GROUPS_PER_WG, 0, st, &a);
    } else {
        hx_launch(opl == 4 ? "sml_gptq_gemv" : "sml_gptq_gemv2", (unsigned) ((m->rows + 64 * opl - 1) / (64 * opl)),
                  (unsigned) a.nslice, 64 * GPTQ_GROUPS_PER_WG, 0, st, &a);
    }
    if (!fold) hx_launch("sml_gptq_reduce", (unsigned) ((m->rows + 255) / 256), 1, 256, 0, st, &a);
}

int sml_hip_gptq_matvec(const sml_hip_gptq * m, const float * x, float * y) {
    OP_BEGIN(-1);
    if (!m || !x || !y) hx_failf("gptq_matvec arguments");
    op_gptq(0, m, x, y);
    HX_LEAVE();
    return 0;
}

int sml_hip_gptq_unpack(const sml_hip_gptq * m, int row0, int nrows, uint8_t * codes, uint8_t * zeros) {
    OP_BEGIN(-1);
    if (!m || row0 < 0 || nrows <= 0 || row0 + nrows > m->rows) hx_failf("gptq_unpack rows out of range");
    sml_kgptq_unpack a;
    memset(&a, 0, sizeof a);
    a.qweight = m->qweight; a.qzeros = m->qzeros;
    a.rows = m->rows; a.cols = m->cols; a.zero_add = m->zero_add;
    a.row0 = row0; a.nrows = nrows; a.codes = codes; a.zeros = zeros;
    const long n = (long) nrows * (m->cols / 8);
    hx_launch("sml_gptq_unpack", (unsigned) ((n + 255) / 256), 1, 256, 0, 0, &a);
    HX(hipStreamSynchronize(0));
    HX_LEAVE();
    return 0;
}

int sml_hip_gptq_time(const sml_hip_gptq * const * mats, int ncopy, const float * x, float * y, int iters,
                      float * ms_total) {
    OP_BEGIN(-1);
    hipEvent_t e0, e1;
    HX(hipEventCreate(&e0));
    HX(hipEventCreate(&e1));
    HX(hipEventRecord(e0, 0));
    for (int i = 0; i < iters; i++) op_gptq(0, mats[i % ncopy], x, y);
    HX(hipEventRecord(e1, 0));
    HX(hipEventSynchronize(e1));
    HX(hipEventElapsedTime(ms_total, e0, e1));
    HX(hipEventDestroy(e0));
    HX(hipEventDestroy(e1));
    HX_LEAVE();
    return 0;
}

// ------------------------------------------------------------ small-M GEMM

int gemm_mt(int m) { return m <= 1 ? 1 : m <= 4 ? 4 : m <= 8 ? 8 : m <= 16 ? 16 : 32; }

int gemm_exact(int regime, int m_all) {
    if (regime == GEMM_EXACT) return 1;
    if (regime == GEMM_PER256) return 0;
    const char * mode = getenv("SML_MULTI");
    return m_all <= 8 || (mode && !strcmp(mode, "exact")) || !env_int("SML_MGEMM", 1);
}

#define GEMM_TILE 128            // chunks (groups) per pass: 64 lanes x GEMM_NI
// The prompt GEMM (sml_pgemm_q4 / _q6): positions per tile, and its LDS: two
// stages of a 128-row weight tile (144 bytes a row), a PGEMM_BM-position
// activation tile (272 bytes a row) and the positions' scales and sums; Q6
// adds the 2-bit plane's 128-row tile (72 bytes a row)
#define PGEMM_BM 32
#define PGEMM_LDS (2 * (128 * 144 + PGEMM_BM * 272 + PGEMM_BM * 8))
#define PGEMM_LDS6 (PGEMM_LDS + 2 * 128 * 72)
#define GEMM_MAX_ROWS 65536

void op_gemm(hipStream_t st, const sml_kmat * tab, const sml_kmat * hk, int ngroups, int swiglu, int nbits, int rows, int cols,
             const int32_t * count, int m_all, int mt, int mmax, const int8_t * q, const float * scale,
             const int32_t * sums, float * y, const float * bias, const float * resid, int regime) {
    const int per256 = regime == GEMM_PER256;
    if (swiglu && (bias || resid)) hx_failf("SwiGLU GEMM takes no bias or residual");
    if ((uint64_t) rows * (uint64_t) cols >= (1ull << 32)) hx_failf("matrix too large for one GEMM launch");
    if (regime == GEMM_REF) {
        // exact mode's batched prompt: Q4 or Q8 inputs a multiple of 256
        // wide, 16 weight rows x 64 positions per workgroup
        if ((nbits != 4 && nbits != 8) || cols % 256 || count || ngroups != 1 || m_all < 1 ||
            (uint64_t) m_all * cols >= (1ull << 32))
            hx_failf("the exact batched GEMM takes one Q4 or Q8 matrix 256-aligned (%d bits, %d columns)", nbits, cols);
        sml_kgemm a;
        memset(&a, 0, sizeof a);
        a.mats = tab; a.nmat = swiglu ? 2 : 1; a.cols = cols; a.rows = rows;
        a.m_all = m_all; a.mmax = mmax;
        a.q = q; a.scale = scale; a.sums = sums; a.y = y; a.bias = bias; a.resid = resid;
        if (hk) {
            a.inl = 1;
            a.m0[0] = hk[0];
            if (swiglu) a.m0[1] = hk[1];
        }
        char xname[24];
        snprintf(xname, sizeof xname, "sml_xgemm_q%d%s", nbits, swiglu ? "_s" : "");
        hx_launch3(xname, (unsigned) ((rows + 15) / 16),
                   (unsigned) ((m_all + 63) / 64), 1, 256, 0, st, &a);
        return;
    }
    // the widest small-M launch: 32 rows in the exact regime (VALU), else 16
    const int msmall = regime == GEMM_EXACT ? 32 : 16;
    if (!count && m_all > msmall) {
        // prompt-sized: Q4 and Q6 with per-256 activations on the prompt MFMA
        // GEMM (tiles of 128 rows, SwiGLU 64, x PGEMM_BM positions); anything
        // else in slices of msmall rows through the small-M kernels
        if (per256 && (nbits == 4 || nbits == 6) && cols % 256 == 0 && env_int("SML_PGEMM", 1)) {
            const int rt = swiglu ? 64 : 128;
            const uint64_t tiles = (uint64_t) ((rows + rt - 1) / rt) * (uint64_t) ((m_all + PGEMM_BM - 1) / PGEMM_BM);
            if (tiles > 0x7FFFFFFFull || (uint64_t) m_all * (uint64_t) cols >= (1ull << 32))
                hx_failf("prompt GEMM of %d rows x %d positions", rows, m_all);
            sml_kgemm a;
            memset(&a, 0, sizeof a);
            a.mats = tab; a.nmat = swiglu ? 2 : 1; a.cols = cols; a.rows = rows;
            a.m_all = m_all; a.mmax = mmax;
            a.q = q; a.scale = scale; a.sums = sums; a.y = y; a.bias = bias; a.resid = resid;
            char pname[32];
            snprintf(pname, sizeof pname, "sml_pgemm_q%d%s", nbits, swiglu ? "_s" : "");
            hx_launch(pname, (unsigned) tiles, 1, 256, nbits == 6 ? PGEMM_LDS6 : PGEMM_LDS, st, &a);
            return;
        }
        // (the exact regime's VALU kernel takes 32 rows a weight read)
        const int ng = cols / 32, sl = msmall;
        for (int s = 0; s < m_all; s += sl) {
            const int k = m_all - s < sl ? m_all - s : sl;
            op_gemm(st, tab, hk, 1, swiglu, nbits, rows, cols, NULL, k, gemm_mt(k), k, q + (size_t) s * cols,
                    scale + (size_t) s * ng, sums + (size_t) s * ng, y + (size_t) s * rows, bias,
                    resid ? resid + (size_t) s * rows : NULL, regime);
        }
        return;
    }
    if (mt != 1 && mt != 4 && mt != 8 && mt != 16 && (mt != 32 || count)) hx_failf("small-M GEMM of %d rows", mt);
    if (!count && (m_all < 1 || m_all > mt)) hx_failf("small-M GEMM of %d rows", m_all);
    sml_kgemm a;
    memset(&a, 0, sizeof a);
    a.mats = tab; a.nmat = swiglu ? 2 : 1; a.cols = cols; a.rows = rows;
    a.count = count; a.m_all = m_all; a.mmax = mmax;
    a.q = q; a.scale = scale; a.sums = sums; a.y = y; a.bias = bias; a.resid = resid;
    if (hk && ngroups == 1 && !count) {
        a.inl = 1;
        a.m0[0] = hk[0];
        if (swiglu) a.m0[1] = hk[1];
    }
    char name[48];
    // Q4 with more than 8 activation rows runs on MFMA (measured faster
    // there; below, the VALU dot4 kernel wins), with the integer superblock
    // epilogue on per-256 activations, unless the exact regime is asked for
    // (SML_MULTI=exact or GEMM_EXACT: every row bit for bit the GEMV's).
    // Expert groups (count != NULL) hold few rows each (16 tokens top-2 over
    // 8 experts: 2 to 7) and stay on VALU, whose per-group epilogue is exact
    // on per-256 activations too. SML_MGEMM=0 keeps every product on VALU.
    const char * mode = getenv("SML_MULTI");
    const int exact = regime == GEMM_EXACT || (mode && !strcmp(mode, "exact"));
    if (nbits == 4 && cols % 256 == 0 && !count && m_all > 8 && !exact && env_int("SML_MGEMM", 1)) {
        const int nsb0 = cols / 256;
        // very tall products take 2 blocks of 16 rows per workgroup, unless
        // the persistent form applies (it reads the activation rows once per
        // workgroup whatever the height)
        int rb = !swiglu && rows >= 32768 && !(nsb0 <= 16 && env_int("SML_MGEMM_PS", 1)) ? 2 : 1;
        const int fr = env_int("SML_MGEMM_RB", 0);
        if (fr == 1 || fr == 2) rb = fr;
        const int nw = env_int("SML_MGEMM_NW", 8) == 4 ? 4 : 8;
        // inputs too wide for the persistent form (more than 2 superblocks a
        // wave) split into 4 slices of at most 2 a wave: each workgroup then
        // holds one slice's activation operands for all its row tiles instead
        // of reading the whole rows again per tile, and sml_gemm_ksum adds
        // the slices with the bias and the residual. SML_MGEMM_KS=1 keeps one
        // tile per workgroup over the whole input.
        int kslices = 1;
        if (!swiglu && ngroups == 1 && nw == 8 && rb == 1 && nsb0 > 2 * nw && nsb0 % 4 == 0 && nsb0 / 4 <= 2 * nw &&
            (size_t) 4 * (size_t) m_all * (size_t) rows <= HX_KPART && env_int("SML_MGEMM_KS", 4) == 4 &&
            env_int("SML_MGEMM_PS", 1))
            kslices = 4;
        // LDS: each wave's share of the activation group data, then the
        // waves' partial sums (the same memory, after a barrier)
        const int nsb = cols / 256 / kslices, spw = (nsb + nw - 1) / nw;
        const size_t stage = (size_t) nw * spw * (per256 ? 576 : 1024);
        const size_t red = (size_t) nw * (swiglu ? 2 : 1) * rb * 4 * 64 * 4;
        const int ntile = (rows + 16 * rb - 1) / (16 * rb);
        // persistent form where a wave's activation operands fit in registers
        // (at most 2 superblocks per wave: inputs up to 4096 wide): each
        // workgroup reads the activation rows once for several row tiles
        // instead of once per tile. At most one workgroup per CU, each
        // taking the same number of tiles: 2 x 14336 x 4096 SwiGLU at 16
        // rows, 896 tiles on 224 workgroups, 37.3 -> 28.1 us (per-256:
        // 33.5 -> 25.0); a grid above the CU count runs some CUs twice as
        // long (299 workgroups: 39.9 us). SML_MGEMM_PWG sets the cap.
        const int ps = nw == 8 && rb == 1 && spw <= 2 && env_int("SML_MGEMM_PS", 1);
        const size_t lds = ps ? stage + red : stage > red ? stage : red;
        if (lds <= 65536) {
            unsigned grid = (unsigned) ntile;
            if (ps) {
                // the cap counts workgroups of every slice
                int cap = env_int("SML_MGEMM_PWG", hx.ncu) / kslices;
                if (cap < 1) cap = 1;
                const int per = (ntile + cap - 1) / cap;
                grid = (unsigned) ((ntile + per - 1) / per * kslices);
            }
            if (kslices > 1) a.part = hx_kpart();
            snprintf(name, sizeof name, "sml_mgemm_q4%s%s_r%d_w%d%s%s%s", swiglu ? "_s" : "", per256 ? "_sb" : "", rb, nw,
                     ps ? "_p" : "", kslices > 1 ? "_k4" : "", tiled_on() ? "_t" : "");
            hx_launch(name, grid, (unsigned) ngroups, (unsigned) (64 * nw), lds, st, &a);
            if (kslices > 1) {
                sml_kksum k;
                k.part = a.part; k.bias = bias; k.resid = resid; k.y = y; k.ks = kslices; k.m = m_all; k.rows = rows;
                if (g_defer) { g_pend = k; g_pending = 1; }
                else hx_launch("sml_gemm_ksum", (unsigned) (((size_t) m_all * rows + 255) / 256), 1, 256, 0, st, &k);
            }
            return;
        }
    }
    // 4 waves x 2 rows (SwiGLU: 2 gate/up pairs) per workgroup. The LDS
    // stages mt activation rows per pass, so expert groups (counts known only
    // on the device) go to one launch per size class, each with the LDS of
    // its class; each launch skips the other classes' groups at once. Two
    // classes (up to 8 rows, up to mt) measured best on the 16-token
    // Mixtral-shaped layer: 296 us against 395 for one 16-row launch and 304
    // for three classes (SML_GEMM_SPLIT = 1, 0, 2), the smaller launches
    // running one after another.
    const int split = count && mt > 4 ? env_int("SML_GEMM_SPLIT", 1) : 0;
    // expert groups (a few rows each) on 512-thread workgroups: twice the
    // rows share each staging of the activation rows (16-token Mixtral-shaped
    // layer 275.6 -> 266.0 us per-256, 301.0 -> 290.6 per-32; 1024 threads:
    // 316.5 / 333.3). SML_GEMM_WG = 256, 512 or 1024 overrides (Q4).
    int wg = env_int("SML_GEMM_WG", count ? 512 : 256);
    if ((wg != 512 && wg != 1024) || nbits != 4) wg = 256;
    int lo = 0;
    for (int m_t = split >= 2 ? 4 : split == 1 ? 8 : mt; ; m_t *= 2) {
        if (m_t > mt) m_t = mt;
        a.mlo = lo;
        const int w = m_t == 1 ? 256 : wg;
        if (w == 256) snprintf(name, sizeof name, "sml_gemm_q%d%s_m%d", nbits, swiglu ? "_s" : "", m_t);
        else snprintf(name, sizeof name, "sml_gemm_q%d%s_m%d_w%d", nbits, swiglu ? "_s" : "", m_t, w);
        // 32 rows: passes of half the columns, one gate/up pair a wave
        const size_t lds = (size_t) m_t * (m_t == 32 ? GEMM_TILE / 2 : GEMM_TILE) * (32 + 8);
        const int rpw = (m_t == 32 && swiglu ? 4 : 8) * w / 256;   // rows (SwiGLU: outputs) per workgroup
        hx_launch(name, (unsigned) ((rows + rpw - 1) / rpw), (unsigned) ngroups, (unsigned) w, lds, st, &a);
        if (m_t >= mt) break;
        lo = m_t;
    }
}

static void gemm_one(const sml_hip_mat * m, const int8_t * q, const float * scale, const int32_t * sums, int nrow,
                     float * y, int per256) {
    if (!m || nrow < 1 || nrow > GEMM_MAX_ROWS) hx_failf("gemm of %d rows (1..%d)", nrow, GEMM_MAX_ROWS);
    op_gemm(0, m->kdev, &m->k, 1, 0, m->nbits, m->k.rows, m->cols, NULL, nrow, gemm_mt(nrow), nrow, q, scale, sums, y, NULL, NULL,
            per256);
}

static void gemm_swiglu(const sml_hip_mat * gate, const sml_hip_mat * up, const int8_t * q, const float * scale,
                        const int32_t * sums, int nrow, float * h, int per256) {
    if (!gate || !up || nrow < 1 || nrow > GEMM_MAX_ROWS) hx_failf("gemm of %d rows (1..%d)", nrow, GEMM_MAX_ROWS);
    if (up->nbits != gate->nbits || up->cols != gate->cols || up->k.rows != gate->k.rows)
        hx_failf("SwiGLU needs gate and up of one shape and width");
    // the (gate, up) table lives in the gate matrix's allocation, rewritten
    // only when the gate is paired with another up than last time (compared
    // by descriptor, so a new matrix at a freed one's address is caught)
    sml_kmat * pair = gate->kdev + 1;
    if (!gate->pair_set || memcmp(&gate->up_k, &up->k, sizeof up->k)) {
        sml_kmat tab[2] = { gate->k, up->k };
        HX(hipMemcpy(pair, tab, sizeof tab, hipMemcpyHostToDevice));
        ((sml_hip_mat *) gate)->up_k = up->k;
        ((sml_hip_mat *) gate)->pair_set = 1;
    }
    const sml_kmat hk[2] = { gate->k, up->k };
    op_gemm(0, pair, hk, 1, 1, gate->nbits, gate->k.rows, gate->cols, NULL, nrow, gemm_mt(nrow), nrow, q, scale, sums, h, NULL,
            NULL, per256);
}

int sml_hip_gemm(const sml_hip_mat * m, const int8_t * q, const float * scale, const int32_t * sums, int nrow,
                 float * y) {
    OP_BEGIN(-1);
    gemm_one(m, q, scale, sums, nrow, y, 0);
    HX_LEAVE();
    return 0;
}

int sml_hip_gemm_sb(const sml_hip_mat * m, const int8_t * q, const float * scale, const int32_t * sums, int nrow,
                    float * y) {
    OP_BEGIN(-1);
    gemm_one(m, q, scale, sums, nrow, y, 1);
    HX_LEAVE();
    return 0;
}

int sml_hip_gemm_swiglu(const sml_hip_mat * gate, const sml_hip_mat * up, const int8_t * q, const float * scale,
                        const int32_t * sums, int nrow, float * h) {
    OP_BEGIN(-1);
    gemm_swiglu(gate, up, q, scale, sums, nrow, h, 0);
    HX_LEAVE();
    return 0;
}

int sml_hip_gemm_swiglu_sb(const sml_hip_mat * gate, const sml_hip_mat * up, const int8_t * q, const float * scale,
                           const int32_t * sums, int nrow, float * h) {
    OP_BEGIN(-1);
    gemm_swiglu(gate, up, q, scale, sums, nrow, h, 1);
    HX_LEAVE();
    return 0;
}

// ------------------------------------------------------------ MoE expert FFN



static void * moe_own(sml_hip_moe * m, size_t n) {
    if (m->nowned >= (int) (sizeof m->owned / sizeof m->owned[0])) hx_failf("too many MoE allocations");
    void * p = hx_malloc(n);
    m->owned[m->nowned++] = p;
    return p;
}

static void moe_release(sml_hip_moe * m) {
    if (!m) return;
    if (m->mats) for (int i = 0; i < 3 * m->nexp; i++) if (m->mats[i]) { hipFree(m->mats[i]->mem); free(m->mats[i]); }
    free(m->mats);
    for (int i = 0; i < 3; i++) if (m->shx[i]) { hipFree(m->shx[i]->mem); free(m->shx[i]); }
    for (int i = 0; i < m->nowned; i++) hipFree(m->owned[i]);
    free(m);
}

// Upload one permutation (NULL for none or the identity).
static int32_t * moe_perm(sml_hip_moe * m, const ssf_file * f, const ssf_record * r) {
    if (!r->perm_bytes) return NULL;
    const int32_t * p = (const int32_t *) ssf_at(f, r->perm_off);
    int ident = 1;
    for (int i = 0; i < (int) r->cols && ident; i++) ident = p[i] == i;
    if (ident) return NULL;
    for (int i = 0; i < (int) r->cols; i++) if (p[i] < 0 || p[i] >= (int) r->cols) hx_failf("%.64s: permutation out of range", r->name);
    int32_t * d = moe_own(m, (size_t) r->cols * 4);
    HX(hipMemcpy(d, p, (size_t) r->cols * 4, hipMemcpyHostToDevice));
    return d;
}

// The shared expert (sml/sml-run.c:1736-1745,3104-3122): gate, up and down
// run on every token, their output added after the routed experts' times
// sigmoid(ffn_gate_inp_shexp . x) when that gate exists (else times 1).
static void moe_shared_setup(sml_hip_moe * m, const ssf_file * f, int L, int tmax) {
    const ssf_record * g = ssf_findf(f, "blk.%d.ffn_gate_shexp.weight", L);
    const ssf_record * u = ssf_findf(f, "blk.%d.ffn_up_shexp.weight", L);
    const ssf_record * d = ssf_findf(f, "blk.%d.ffn_down_shexp.weight", L);
    if (!u || !d) return;
    if (!g) hx_failf("layer %d: an ungated shared expert (up, activation, down) is not built", L);
    if ((int) g->cols != m->n_embd || u->cols != g->cols || u->rows != g->rows || (int) d->rows != m->n_embd ||
        d->cols != g->rows || u->nbits != g->nbits)
        hx_failf("layer %d: shared expert of unexpected shapes", L);
    m->sh_ff = (int) g->rows;
    m->shx[0] = mat_from_record(f, g);
    m->shx[1] = mat_from_record(f, u);
    m->shx[2] = mat_from_record(f, d);
    const int32_t * pg = moe_perm(m, f, g), * pu = moe_perm(m, f, u);
    if (!((!pg && !pu) || (pg && pu && g->perm_off == u->perm_off)))
        hx_failf("layer %d: shared gate and up read different permutations", L);
    m->sh_perm_gu = pg;
    m->sh_perm_d = moe_perm(m, f, d);
    const sml_kmat t[2] = { m->shx[0]->k, m->shx[1]->k };
    m->sh_gu = moe_own(m, sizeof t);
    HX(hipMemcpy(m->sh_gu, t, sizeof t, hipMemcpyHostToDevice));
    const ssf_record * sg = ssf_findf(f, "blk.%d.ffn_gate_inp_shexp.weight", L);
    if (sg) {
        if (sg->kind != SSF_KIND_F32 || (uint64_t) sg->rows * sg->cols != (uint64_t) m->n_embd)
            hx_failf("layer %d: shared expert gate is not f32 of %d", L, m->n_embd);
        m->shgate = moe_own(m, (size_t) m->n_embd * 4);
        HX(hipMemcpy(m->shgate, ssf_at(f, sg->f32_off), (size_t) m->n_embd * 4, hipMemcpyHostToDevice));
    }
    const size_t T = (size_t) tmax, ne = (size_t) m->n_embd, nf = (size_t) m->sh_ff, w = ne > nf ? ne : nf;
    m->sg = moe_own(m, T * 4);
    m->sh_h = moe_own(m, T * nf * 4);
    m->sh_y = moe_own(m, T * ne * 4);
    m->sh_q = moe_own(m, T * w + T * (w / 32) * 8);
    m->sh_s = (float *) (m->sh_q + T * w);
    m->sh_u = (int32_t *) (m->sh_s + T * (w / 32));
    m->expert_bytes += m->shx[0]->bytes + m->shx[1]->bytes + m->shx[2]->bytes;
}

static void moe_setup(sml_hip_moe * m, const ssf_file * f, int L, int tmax, const sml_hip_moe * share) {
    const ssf_header * h = f->hdr;
    // routing (sml/sml-run.c:2925-3037): flags bits 0-3, moe_scale, groups
    if (h->moe_flags & ~15u) hx_failf("routing mode 0x%x not built (flags bits 0-3)", h->moe_flags);
    if (h->moe_groups > 64) hx_failf("%u expert groups (at most 64)", h->moe_groups);
    char nm[96];
    m->n_embd = (int) h->n_embd;
    m->scale = h->moe_scale;
    m->groups = (int) h->moe_groups;
    m->topk_group = (int) h->moe_topk_group;
    // the router's rows are the experts (sml/sml-run.c:1676-1680)
    const ssf_record * rt = ssf_findf(f, "blk.%d.ffn_gate_inp.weight", L);
    if (!rt) hx_failf("layer %d has no experts (no router)", L);
    if (rt->kind != SSF_KIND_F32 || ((uint64_t) rt->rows * rt->cols) % (uint64_t) m->n_embd)
        hx_failf("layer %d: the router is not f32 n_expert x %d", L, m->n_embd);
    m->nexp = (int) (((uint64_t) rt->rows * rt->cols) / (uint64_t) m->n_embd);
    m->k = (int) h->n_expert_used;
    if (m->k <= 0 || m->k > m->nexp) m->k = m->nexp;
    if (m->k > 16 || m->nexp > 64 || m->nexp < 1) hx_failf("%d of %d experts: at most 16 of 64", m->k, m->nexp);
    m->flags = h->moe_flags;
    m->tmax = tmax;
    // the choice's correction bias (the reference takes it when it holds at
    // least one value per expert, sml/sml-run.c:1743-1745)
    const ssf_record * eb = ssf_findf(f, "blk.%d.exp_probs_b.weight", L);
    if (eb && eb->kind == SSF_KIND_F32 && (uint64_t) eb->rows * eb->cols >= (uint64_t) m->nexp) {
        m->exp_bias = moe_own(m, (size_t) m->nexp * 4);
        HX(hipMemcpy(m->exp_bias, ssf_at(f, eb->f32_off), (size_t) m->nexp * 4, hipMemcpyHostToDevice));
    }
    m->router = moe_own(m, (size_t) m->nexp * m->n_embd * 4);
    HX(hipMemcpy(m->router, ssf_at(f, rt->f32_off), (size_t) m->nexp * m->n_embd * 4, hipMemcpyHostToDevice));
    const ssf_record * rb = ssf_findf(f, "blk.%d.ffn_gate_inp.bias", L);
    if (rb) {
        if (rb->kind != SSF_KIND_F32 || (uint64_t) rb->rows * rb->cols != (uint64_t) m->nexp) hx_failf("router bias shape");
        m->router_b = moe_own(m, (size_t) m->nexp * 4);
        HX(hipMemcpy(m->router_b, ssf_at(f, rb->f32_off), (size_t) m->nexp * 4, hipMemcpyHostToDevice));
    }
    m->mats = calloc((size_t) m->nexp * 3, sizeof *m->mats);
    if (!m->mats) hx_failf("out of host memory");
    sml_kmat * tgu = calloc((size_t) m->nexp * 3, sizeof *tgu);
    const int32_t ** pgu = calloc((size_t) m->nexp * 2, sizeof *pgu);
    if (!tgu || !pgu) { free(tgu); free(pgu); hx_failf("out of host memory"); }
    jmp_buf * outer = hx.jb;
    jmp_buf jb;
    if (setjmp(jb)) { hx.jb = outer; free(tgu); free(pgu); longjmp(*outer, 1); }
    hx.jb = &jb;
    const char * kind[3] = { "gate", "up", "down" };
    int any_gu = 0, any_d = 0;
    for (int e = 0; e < m->nexp; e++) {
        const ssf_record * r[3];
        for (int i = 0; i < 3; i++) {
            snprintf(nm, sizeof nm, "blk.%d.ffn_%s.%d.weight", L, kind[i], e);
            r[i] = ssf_find(f, nm);
            if (!r[i]) hx_failf("model has no %s", nm);
            snprintf(nm, sizeof nm, "blk.%d.ffn_%s.%d.bias", L, kind[i], e);
            if (ssf_find(f, nm)) hx_failf("expert biases not built");
        }
        if ((int) r[0]->cols != m->n_embd || r[1]->cols != r[0]->cols || r[1]->rows != r[0]->rows ||
            (int) r[2]->rows != m->n_embd || r[2]->cols != r[0]->rows || r[1]->nbits != r[0]->nbits)
            hx_failf("expert %d has unexpected shapes", e);
        if (e == 0) { m->n_ff = (int) r[0]->rows; m->nbits = (int) r[0]->nbits; }
        if ((int) r[0]->rows != m->n_ff || (int) r[0]->nbits != m->nbits || (int) r[2]->nbits != m->nbits)
            hx_failf("experts of different widths or sizes not built");
        for (int i = 0; i < 3; i++) {
            m->mats[e * 3 + i] = mat_from_record(f, r[i]);
            m->expert_bytes += e == 0 ? m->mats[e * 3 + i]->bytes : 0;
        }
        tgu[e * 2] = m->mats[e * 3]->k;
        tgu[e * 2 + 1] = m->mats[e * 3 + 1]->k;
        tgu[2 * m->nexp + e] = m->mats[e * 3 + 2]->k;
        const int32_t * pg = moe_perm(m, f, r[0]), * pu = moe_perm(m, f, r[1]);
        const int same = (!pg && !pu) || (pg && pu && r[0]->perm_off == r[1]->perm_off);
        if (!same) hx_failf("expert %d: gate and up read different permutations", e);
        pgu[e] = pg;
        pgu[m->nexp + e] = moe_perm(m, f, r[2]);
        any_gu |= pg != NULL;
        any_d |= pgu[m->nexp + e] != NULL;
    }
    m->tab_gu = moe_own(m, (size_t) m->nexp * 2 * sizeof(sml_kmat));
    m->tab_d = moe_own(m, (size_t) m->nexp * sizeof(sml_kmat));
    HX(hipMemcpy(m->tab_gu, tgu, (size_t) m->nexp * 2 * sizeof(sml_kmat), hipMemcpyHostToDevice));
    HX(hipMemcpy(m->tab_d, tgu + 2 * m->nexp, (size_t) m->nexp * sizeof(sml_kmat), hipMemcpyHostToDevice));
    if (any_gu) {
        m->ptab_gu = moe_own(m, (size_t) m->nexp * sizeof(void *));
        HX(hipMemcpy(m->ptab_gu, pgu, (size_t) m->nexp * sizeof(void *), hipMemcpyHostToDevice));
    }
    if (any_d) {
        m->ptab_d = moe_own(m, (size_t) m->nexp * sizeof(void *));
        HX(hipMemcpy(m->ptab_d, pgu + m->nexp, (size_t) m->nexp * sizeof(void *), hipMemcpyHostToDevice));
    }
    hx.jb = outer;
    free(tgu);
    free(pgu);
    moe_shared_setup(m, f, L, tmax);
    // scratch: this layer's own, or another layer's of the same shape (layers run one after another)
    if (share) {
        if (share->nexp != m->nexp || share->k != m->k || share->n_ff != m->n_ff || share->n_embd != m->n_embd ||
            share->tmax < tmax)
            hx_failf("layer %d: experts of a different shape than layer 0's", L);
        m->logits = share->logits; m->w = share->w; m->sel = share->sel; m->slot = share->slot;
        m->count = share->count; m->list = share->list; m->qx = share->qx; m->sx = share->sx; m->ux = share->ux;
        m->h = share->h; m->qh = share->qh; m->sh = share->sh; m->uh = share->uh; m->yd = share->yd;
        m->tmax = share->tmax;
        return;
    }
    const size_t E = (size_t) m->nexp, T = (size_t) tmax, K = (size_t) m->k, ne = (size_t) m->n_embd, nf = (size_t) m->n_ff;
    m->logits = moe_own(m, T * E * 4);
    m->w = moe_own(m, T * K * 4);
    m->sel = moe_own(m, T * K * 4);
    m->slot = moe_own(m, T * K * 4);
    m->count = moe_own(m, E * 4);
    m->list = moe_own(m, E * T * 4);
    m->qx = moe_own(m, E * T * ne);
    m->sx = moe_own(m, E * T * (ne / 32) * 8);
    m->ux = (int32_t *) (m->sx + E * T * (ne / 32));
    m->h = moe_own(m, E * T * nf * 4);
    m->qh = moe_own(m, E * T * nf + E * T * (nf / 32) * 8);
    m->sh = (float *) (m->qh + E * T * nf);
    m->uh = (int32_t *) (m->sh + E * T * (nf / 32));
    m->yd = moe_own(m, E * T * ne * 4);
}

sml_hip_moe * sml_hip_moe_from_file(const char * path, int layer, int max_tokens) {
    OP_BEGIN(NULL);
    if (max_tokens < 1 || max_tokens > 16) hx_failf("max_tokens %d (1..16)", max_tokens);
    ssf_file f;
    char why[256];
    if (!ssf_open(&f, path, why, sizeof why)) hx_failf("%s", why);
    sml_hip_moe * m = calloc(1, sizeof *m);
    if (!m) { ssf_close(&f); hx_failf("out of host memory"); }
    jmp_buf * outer = hx.jb;
    jmp_buf jb;
    if (setjmp(jb)) { hx.jb = outer; ssf_close(&f); moe_release(m); longjmp(*outer, 1); }
    hx.jb = &jb;
    if (layer < 0 || layer >= (int) f.hdr->n_layer) hx_failf("layer %d of %u", layer, f.hdr->n_layer);
    moe_setup(m, &f, layer, max_tokens, NULL);
    hx.jb = outer;
    ssf_close(&f);
    HX_LEAVE();
    return m;
}

void sml_hip_moe_free(sml_hip_moe * m) {
    HX_ENTRY();
    if (m) HX(hipDeviceSynchronize());
    moe_release(m);
    HX_LEAVE();
}

int sml_hip_moe_regime(sml_hip_moe * m, int per256) {
    if (!m) return -1;
    m->per256 = per256 ? 1 : 0;
    return 0;
}

int sml_hip_moe_info(const sml_hip_moe * m, int * nexp, int * k, int * n_ff, size_t * expert_bytes) {
    if (!m) return -1;
    if (nexp) *nexp = m->nexp;
    if (k) *k = m->k;
    if (n_ff) *n_ff = m->n_ff;
    if (expert_bytes) *expert_bytes = m->expert_bytes;
    return 0;
}

sml_hip_moe * moe_load(const ssf_file * f, int layer, int tmax, const sml_hip_moe * share) {
    sml_hip_moe * m = calloc(1, sizeof *m);
    if (!m) hx_failf("out of host memory");
    jmp_buf * outer = hx.jb;
    jmp_buf jb;
    if (setjmp(jb)) { hx.jb = outer; moe_release(m); longjmp(*outer, 1); }
    hx.jb = &jb;
    moe_setup(m, f, layer, tmax, share);
    hx.jb = outer;
    return m;
}

void moe_free(sml_hip_moe * m) { moe_release(m); }

void op_moe(hipStream_t st, sml_hip_moe * m, const float * x, int T, float * out, const float * resid) {
    sml_kmoe_route r;
    memset(&r, 0, sizeof r);
    r.x = x; r.router = m->router; r.router_b = m->router_b;
    r.T = T; r.n = m->n_embd; r.nexp = m->nexp; r.k = m->k; r.mmax = m->tmax; r.moe_flags = m->flags;
    r.logits = m->logits; r.sel = m->sel; r.w = m->w; r.slot = m->slot; r.count = m->count; r.list = m->list;
    r.exact = g_exact;
    r.exp_bias = m->exp_bias; r.scale = m->scale; r.groups = m->groups; r.topk_group = m->topk_group;
    r.shgate = m->shx[0] ? m->shgate : NULL; r.sg = m->shx[0] ? m->sg : NULL;
    hx_launch("sml_moe_route", (unsigned) T, 1, 512, 0, st, &r);
    hx_launch("sml_moe_plan", 1, 1, 64, 0, st, &r);
    sml_kmquant qa;
    memset(&qa, 0, sizeof qa);
    qa.src = x; qa.mode = 0; qa.perms = m->ptab_gu; qa.n = m->n_embd; qa.mmax = m->tmax; qa.k = m->k;
    qa.count = m->count; qa.list = m->list; qa.q = m->qx; qa.scale = m->sx; qa.sums = m->ux; qa.per256 = m->per256;
    hx_launch("sml_moe_quant", (unsigned) T, (unsigned) m->nexp, 1024, 0, st, &qa);
    const int mt = gemm_mt(T);
    op_gemm(st, m->tab_gu, NULL, m->nexp, 1, m->nbits, m->n_ff, m->n_embd, m->count, 0, mt, m->tmax,
            m->qx, m->sx, m->ux, m->h, NULL, NULL, m->per256);
    sml_kmquant qb = qa;
    qb.src = m->h; qb.mode = 1; qb.perms = m->ptab_d; qb.n = m->n_ff; qb.q = m->qh; qb.scale = m->sh; qb.sums = m->uh;
    hx_launch("sml_moe_quant", (unsigned) T, (unsigned) m->nexp, 1024, 0, st, &qb);
    op_gemm(st, m->tab_d, NULL, m->nexp, 0, m->nbits, m->n_embd, m->n_ff, m->count, 0, mt, m->tmax,
            m->qh, m->sh, m->uh, m->yd, NULL, NULL, m->per256);
    if (m->shx[0]) {
        // the shared expert on every token: its inputs in its permutation,
        // gate/up with SwiGLU, then down, as one dense FFN over the T rows
        const int32_t * pp[1] = { m->sh_perm_gu };
        int8_t * qq[1] = { m->sh_q };
        float * ss[1] = { m->sh_s };
        int32_t * uu[1] = { m->sh_u };
        op_normq_rows(st, (float *) x, NULL, NULL, 0.0f, m->n_embd, T, 1, pp, qq, ss, uu, NULL, m->per256);
        const sml_kmat shk[2] = { m->shx[0]->k, m->shx[1]->k };
        op_gemm(st, m->sh_gu, shk, 1, 1, m->shx[0]->nbits, m->sh_ff, m->n_embd, NULL, T, mt, T, m->sh_q, m->sh_s, m->sh_u,
                m->sh_h, NULL, NULL, m->per256);
        pp[0] = m->sh_perm_d;
        op_normq_rows(st, m->sh_h, NULL, NULL, 0.0f, m->sh_ff, T, 1, pp, qq, ss, uu, NULL, m->per256);
        op_gemm(st, m->shx[2]->kdev, &m->shx[2]->k, 1, 0, m->shx[2]->nbits, m->n_embd, m->sh_ff, NULL, T, mt, T, m->sh_q, m->sh_s,
                m->sh_u, m->sh_y, NULL, NULL, m->per256);
    }
    sml_kmoe_comb c;
    memset(&c, 0, sizeof c);
    c.y = m->yd; c.sel = m->sel; c.slot = m->slot; c.w = m->w; c.T = T; c.n = m->n_embd; c.k = m->k;
    c.mmax = m->tmax; c.out = out; c.resid = resid;
    c.ysh = m->shx[0] ? m->sh_y : NULL; c.sg = m->sg;
    hx_launch("sml_moe_combine", (unsigned) ((m->n_embd + 255) / 256), (unsigned) T, 256, 0, st, &c);
}

int sml_hip_moe_ffn(sml_hip_moe * m, const float * x, int T, float * out, int32_t * sel, float * w, float * logits) {
    OP_BEGIN(-1);
    if (!m || !x || !out || T < 1 || T > m->tmax) hx_failf("moe_ffn of %d tokens (max %d)", T, m ? m->tmax : 0);
    op_moe(0, m, x, T, out, NULL);
    if (sel) HX(hipMemcpyAsync(sel, m->sel, (size_t) T * m->k * 4, hipMemcpyDeviceToDevice, 0));
    if (w) HX(hipMemcpyAsync(w, m->w, (size_t) T * m->k * 4, hipMemcpyDeviceToDevice, 0));
    if (logits) HX(hipMemcpyAsync(logits, m->logits, (size_t) T * m->nexp * 4, hipMemcpyDeviceToDevice, 0));
    HX(hipStreamSynchronize(0));
    HX_LEAVE();
    return 0;
}

int sml_hip_moe_time(sml_hip_moe * m, const float * x, int T, float * out, int iters, float * ms_total,
                     int32_t * count_out) {
    OP_BEGIN(-1);
    if (!m || T < 1 || T > m->tmax || iters < 1) hx_failf("moe_time arguments");
    hipEvent_t e0, e1;
    HX(hipEventCreate(&e0));
    HX(hipEventCreate(&e1));
    op_moe(0, m, x, T, out, NULL);
    HX(hipEventRecord(e0, 0));
    for (int i = 0; i < iters; i++) op_moe(0, m, x, T, out, NULL);
    HX(hipEventRecord(e1, 0));
    HX(hipEventSynchronize(e1));
    HX(hipEventElapsedTime(ms_total, e0, e1));
    HX(hipEventDestroy(e0));
    HX(hipEventDestroy(e1));
    if (count_out) HX(hipMemcpy(count_out, m->count, (size_t) m->nexp * 4, hipMemcpyDeviceToHost));
    HX_LEAVE();
    return 0;
}
