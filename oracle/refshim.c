// CPU ORACLE — test infrastructure only. A thin C wrapper compiled together
// with the reference engine's own CPU sources (sml-kernel.c, sml-pool.c,
// sml-model.c, sml-run.c, read where they lie) into oracle/_ref/libsmlref.so.
// It gives ctypes flat entry points for the reference's context-based API and
// reports the reference's struct layout so the format can be cross-checked.
#include <stddef.h>
#include <stdlib.h>
#include <string.h>

#include "sml-run.h"

// Layout of the reference's packed structs: sizes then field offsets.
void ref_layout(long * out) {
    out[0] = (long) sizeof(sml_hdr);
    out[1] = (long) sizeof(sml_rec);
    out[2] = (long) offsetof(sml_hdr, table_off);
    out[3] = (long) offsetof(sml_hdr, flags);
    out[4] = (long) offsetof(sml_hdr, n_expert_used);
    out[5] = (long) offsetof(sml_hdr, moe_flags);
    out[6] = (long) offsetof(sml_hdr, gdn_dk);
    out[7] = (long) offsetof(sml_rec, perm_off);
    out[8] = (long) offsetof(sml_rec, mq_n);
    out[9] = (long) offsetof(sml_rec, codes_off);
    out[10] = (long) offsetof(sml_rec, nbits);
    out[11] = (long) offsetof(sml_hdr, rope_theta);
}

typedef struct { sml_model m; sml_ctx c; int have_ctx; } ref_h;

void * ref_open(const char * path, int n_ctx, int threads, int with_ctx) {
    ref_h * h = calloc(1, sizeof *h);
    if (!h) return NULL;
    if (!sml_model_open(&h->m, path)) { free(h); return NULL; }
    if (with_ctx) {
        if (!sml_ctx_init(&h->c, &h->m, n_ctx, threads)) { sml_model_close(&h->m); free(h); return NULL; }
        h->have_ctx = 1;
    }
    return h;
}

void ref_close(void * p) {
    ref_h * h = (ref_h *) p;
    if (!h) return;
    if (h->have_ctx) sml_ctx_free(&h->c);
    sml_model_close(&h->m);
    free(h);
}

const float * ref_forward(void * p, int tok, int pos) {
    ref_h * h = (ref_h *) p;
    return sml_forward(&h->c, tok, pos, 0);
}

const float * ref_prefill(void * p, const int32_t * ids, int pos0, int n) {
    ref_h * h = (ref_h *) p;
    return sml_prefill(&h->c, ids, pos0, n, 0);
}

int ref_n_vocab(void * p) { return (int) ((ref_h *) p)->m.hdr->n_vocab; }

// The model's tensor record by name: returns the record's address inside the
// mapped file (its offsets are absolute file offsets) or NULL.
const void * ref_find(void * p, const char * name) { return sml_find(&((ref_h *) p)->m, name); }
const void * ref_base(void * p) { return ((ref_h *) p)->m.base; }

// sml_moe_route with a header carrying only the routing fields.
int ref_moe_route(const float * lg, int ne, int k, unsigned moe_flags, int * sel, float * w) {
    sml_hdr hd;
    sml_layer ly;
    memset(&hd, 0, sizeof hd);
    memset(&ly, 0, sizeof ly);
    hd.n_expert_used = (uint32_t) k;
    hd.moe_flags = moe_flags;
    ly.n_exp = ne;
    float sc[64], ch[64];
    return sml_moe_route(&hd, &ly, lg, sc, ch, sel, w);
}

// sml_moe_route with every routing field: flags, moe_scale, groups,
// topk_group and the layer's correction bias (exp_bias, NULL for none).
int ref_moe_route2(const float * lg, int ne, int k, unsigned moe_flags, float scale, int groups, int topk_group,
                   const float * exp_bias, int * sel, float * w) {
    sml_hdr hd;
    sml_layer ly;
    memset(&hd, 0, sizeof hd);
    memset(&ly, 0, sizeof ly);
    hd.n_expert_used = (uint32_t) k;
    hd.moe_flags = moe_flags;
    hd.moe_scale = scale;
    hd.moe_groups = (uint32_t) groups;
    hd.moe_topk_group = (uint32_t) topk_group;
    ly.n_exp = ne;
    ly.exp_bias = exp_bias;
    float sc[64], ch[64];
    return sml_moe_route(&hd, &ly, lg, sc, ch, sel, w);
}

// Several contexts of one model, set up as sml-batched does
// (sml/sml-batched.c:70-76), for sml_forward_multi.
typedef struct { sml_model m; int ns; sml_ctx * cs; sml_ctx ** cp; } ref_mh;

void * ref_multi_open(const char * path, int n_ctx, int threads, int ns) {
    ref_mh * h = calloc(1, sizeof *h);
    if (!h) return NULL;
    if (!sml_model_open(&h->m, path)) { free(h); return NULL; }
    h->cs = calloc((size_t) ns, sizeof(sml_ctx));
    h->cp = calloc((size_t) ns, sizeof(sml_ctx *));
    for (int s = 0; s < ns; s++) {
        if (!sml_ctx_init(&h->cs[s], &h->m, n_ctx, threads)) {
            for (int t = 0; t < s; t++) sml_ctx_free(&h->cs[t]);
            free(h->cs); free(h->cp); sml_model_close(&h->m); free(h);
            return NULL;
        }
        h->cp[s] = &h->cs[s];
    }
    h->ns = ns;
    return h;
}

// sml_forward on slot `slot`'s context (the stepped, per-32 path)
const float * ref_multi_forward(void * p, int slot, int tok, int pos) {
    ref_mh * h = (ref_mh *) p;
    return sml_forward(h->cp[slot], tok, pos, 0);
}

// One token for each of the first ns slots: sml_forward_multi, whose regime
// the SML_MULTI / SML_MULTI_EXACT_MAX environment picks (read once).
void ref_multi_step(void * p, const int32_t * tok, const int * pos, int ns, float * logits) {
    ref_mh * h = (ref_mh *) p;
    sml_forward_multi(h->cp, tok, pos, ns, 0, logits);
}

void ref_multi_close(void * p) {
    ref_mh * h = (ref_mh *) p;
    if (!h) return;
    for (int s = h->ns - 1; s >= 0; s--) sml_ctx_free(&h->cs[s]);
    free(h->cs); free(h->cp);
    sml_model_close(&h->m);
    free(h);
}

// ---------------------------------------------------------------- CPU GEMV timing
//
// The CPU baseline of the single-GEMV workloads: sml_quantize_act, then the
// width's kernels as issue_rows_act dispatches them (sml/sml-run.c:612-680),
// over row chunks of 32 handed out dynamically to `threads` OpenMP threads
// (matvec's OpenMP branch, sml/sml-run.c:786-797), rotating over `ncopy`
// copies of the planes and fields (bigger together than the last-level cache,
// as sml/sml-kernel-bench.c:72-90 rotates its working set). Returns seconds per
// call (median of 5 trials of `iters` calls).
#include <omp.h>
#include <time.h>

typedef struct { const uint8_t * pl[3]; const uint16_t * sd; const uint8_t * sq; const uint16_t * md; const uint8_t * mq; } ref_wcopy;

static void rows_width(float * y, const ref_wcopy * w, const sml_act * a, int nb, int lo, int hi, int n) {
    switch (nb) {
    case 4: sml_matvec_rows_flat4(y, w->pl[0], w->sd, w->sq, w->md, w->mq, a, lo, hi, n); break;
    case 2: sml_matvec_rows(y, w->pl[0], w->sd, w->sq, w->md, w->mq, a, lo, hi, n, 0, 0.0f); break;
    case 3: sml_matvec_rows(y, w->pl[0], w->sd, w->sq, w->md, w->mq, a, lo, hi, n, 0, 0.0f);
            sml_matvec_bits1(y, w->pl[1], w->sd, w->sq, a, 1, 0, lo, hi, n, 2); break;
    case 5: sml_matvec_rows_flat4(y, w->pl[0], w->sd, w->sq, w->md, w->mq, a, lo, hi, n);
            sml_matvec_bits1(y, w->pl[1], w->sd, w->sq, a, 1, 0, lo, hi, n, 4); break;
    case 6: sml_matvec_rows_flat6(y, w->pl[1], w->pl[0], w->sd, w->sq, w->md, w->mq, a, lo, hi, n); break;
    case 7: sml_matvec_rows_flat6(y, w->pl[0], w->pl[1], w->sd, w->sq, w->md, w->mq, a, lo, hi, n);
            sml_matvec_bits1(y, w->pl[2], w->sd, w->sq, a, 1, 0, lo, hi, n, 6); break;
    case 8: sml_matvec_rows_flat8(y, w->pl[0], w->pl[1], w->sd, w->sq, w->md, w->mq, a, lo, hi, n); break;
    default: break;
    }
}

double ref_time_matvec(const void * const * planes, const void * const * sd, const void * const * sq,
                       const void * const * md, const void * const * mq, int ncopy, int rows, int cols, int nbits,
                       const float * x, int threads, int iters) {
    ref_wcopy * w = calloc((size_t) ncopy, sizeof *w);
    for (int c = 0; c < ncopy; c++) {
        for (int p = 0; p < 3; p++) w[c].pl[p] = (const uint8_t *) planes[3 * c + p];
        w[c].sd = sd[c]; w[c].sq = sq[c]; w[c].md = md[c]; w[c].mq = mq[c];
    }
    sml_act a;
    memset(&a, 0, sizeof a);
    a.q = malloc((size_t) cols);
    a.scale = malloc((size_t) cols / 32 * 4);
    a.sums = malloc((size_t) cols / 32 * 4);
    a.n = cols;
    float * y = malloc((size_t) rows * 4);
    const int nch = (rows + 31) / 32;
    double trial[5];
    omp_set_num_threads(threads);
    for (int t = 0; t < 5; t++) {
        struct timespec t0, t1;
        clock_gettime(CLOCK_MONOTONIC, &t0);
        for (int it = 0; it < iters; it++) {
            const ref_wcopy * cw = &w[it % ncopy];
            sml_quantize_act(&a, x, cols);
            memset(y, 0, (size_t) rows * 4);
            #pragma omp parallel for schedule(dynamic, 1) num_threads(threads)
            for (int k = 0; k < nch; k++) {
                const int lo = k * 32, hi = lo + 32 < rows ? lo + 32 : rows;
                rows_width(y, cw, &a, nbits, lo, hi, cols);
            }
        }
        clock_gettime(CLOCK_MONOTONIC, &t1);
        trial[t] = ((double) (t1.tv_sec - t0.tv_sec) + 1e-9 * (double) (t1.tv_nsec - t0.tv_nsec)) / iters;
    }
    for (int i = 1; i < 5; i++)
        for (int j = i; j > 0 && trial[j] < trial[j - 1]; j--) { const double s = trial[j]; trial[j] = trial[j - 1]; trial[j - 1] = s; }
    free(a.q); free(a.scale); free(a.sums); free(y); free(w);
    return trial[2];
}
