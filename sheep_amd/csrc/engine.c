// The GPU forward pass behind sml-gpu.h, MI355X-native.
//
// One model and one fp16 KV cache per process. A decode step is a fixed
// sequence of gfx950 kernels on one stream -- embed, then per layer
// normq / q-k-v GEMV / RoPE + KV write + split attention / quantize /
// o GEMV + residual / normq / fused gate-up SwiGLU GEMV / quantize /
// down GEMV + residual, then normq / head GEMV / argmax -- captured once into
// HIP graphs and replayed per token. The token and position the graphs read
// live in device memory (a token history array and a position scalar), so
// greedy decoding needs no host round trip per token. The layer math follows
// the reference's CPU forward pass (sml/sml-run.c:3243-3523) for the
// Llama / Qwen2 family (RMSNorm, halved RoPE, GQA, SwiGLU, optional q/k/v
// bias, tied or untied head); other architectures are refused at open by name.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "ops.h"
#include "sml-gpu-ext.h"
#include "sml-gpu.h"

#define MAXACT 3

typedef struct {
    sml_hip_mat * qkv;         // q, k and v rows stacked (one GEMV), or NULL: w[]
    float * bias_qkv;          // their biases stacked, or NULL
    sml_hip_mat * w[3];        // q, k, v when they cannot be stacked
    sml_hip_mat * o, * gate, * up, * down;
    float * bias[3];           // device q/k/v biases, or NULL
    float * an, * fn;          // device norm weights
    int perm_qkv[3], perm_o, perm_gu[2], perm_down;   // index into perms, -1 = identity
    sml_hip_moe * moe;         // a mixture-of-experts FFN in place of gate/up/down, or NULL
    sml_kmat * gu_tab;         // device (gate, up) pair for the batched SwiGLU GEMM
} eng_layer;

#define MAX_SLOTS 16
#define NBKT 8                 // position buckets of the captured steps

static struct {
    int open;
    int n_layer, E, H, KV, hd, F, V, n_ctx;
    float eps;
    eng_layer * L;
    sml_hip_mat * emb, * head;
    int perm_emb, perm_head;
    float * out_norm;
    int nperm;
    int32_t * perm_dev[512];
    const int32_t * perm_host[512];
    int perm_len[512];
    float * x, * q, * k, * v, * att, * hb, * hb2, * logits, * part, * rc, * rs;
    int8_t * aq[MAXACT];
    float * as[MAXACT];
    int32_t * asum[MAXACT];
    float * xn;                // RMSNorm(x) for a MoE FFN's router and experts
    int8_t * hq;               // the SwiGLU kernel's quantized h, input of down
    float * hs;
    int32_t * hsum;
    int fuse;                  // SML_FUSE bits: 1 activation prologues, 2 h quantization (default 3)
    uint16_t * kc, * vc;
    int32_t * hist, * pos, * tok;
    int2 * amax_part;          // pairs of the two-stage greedy pick
    int2 * head_pairs;         // the head GEMV's row blocks' pairs (at most one per row)
    int * acnt;                // merge counters of the decode attention launch (one per kv head)
    float * lg_host;
    int32_t * pin;             // pinned: [0] tok, [1] pos, [2..] prompt ids
    hipStream_t st;
    // Attention launches cover the positions below pos_cap only. A step's
    // graph is captured per position bucket: bucket k covers positions below
    // min(n_ctx, (k + 1) * bkt_len), so a step at a short position launches
    // no workgroups for the splits of the context it cannot reach yet.
    hipGraphExec_t g_body[NBKT], g_tail, g_adv;
    hipGraphExec_t g_multi[17][2][NBKT];   // the batched step per sequence count, regime (per-256), bucket
    int use_graph;
    int pos_cap, bkt_len, nbkt;
    hipEvent_t e0, e1;
    float last_ms;
    uint64_t weight_bytes;
    int prompt_level;
    int exact;                 // SML_EXACT=1 at open: every kernel in the reference's float order
    void * dev[4096];          // every device allocation, freed at close
    int ndev;
    sml_hip_mat * mats[8192];
    int nmats;
    sml_hip_moe * moe_first;   // the MoE layer whose scratch the others share
    // several sequences: a KV cache per slot (slot 0's is kc/vc) and batch buffers
    int nslot, cur_slot;
    uint16_t * kcs[MAX_SLOTS], * vcs[MAX_SLOTS];
    float * mx, * mqkv, * matt, * mh, * mxn, * mlog;
    int8_t * maq;
    float * mas;
    int32_t * masum, * mtok, * mpos, * mslot;
    int32_t * mpin;            // pinned: tokens, positions, slots of a batched step
    float * mlog_host;         // pinned: a batched step's logits, copied on to the caller's buffer
    uint16_t ** kc_tab, ** vc_tab;   // device tables of every slot's cache base
    float * mpart;             // attention partials of every sequence of a batch
    size_t mpart_floats;
    int xchunk;                // exact mode's prompt chunk: its rows' scores fit in mpart
    int32_t * iota;            // device [n_ctx]: 0, 1, 2, ... (prompt chunk positions)
    int32_t * slotid;          // device [MAX_SLOTS][rrows]: row s filled with s
    int rrows;                 // rows of the batched body's buffers: max(MAX_SLOTS, pb)
    int pb;                    // positions per chunk of a level-2 prompt
    int rows_ok;               // 1: the batched body can run this model (-1: not checked yet)
    int rows_ready;            // the batched body's buffers are allocated
    // A layer split: layers below nres keep their matrices in HBM. The rest
    // are streamed: their matrices were laid out in the staging region and
    // kept as pinned host images, one copied back into the region ahead of
    // each use of its layer. nres == n_layer: no split.
    int nres;
    void * stage;
    size_t stage_cap;
    void ** img;               // [n_layer]: a streamed layer's image, else NULL
    size_t * img_n;
    float * mid_host;          // pinned: the hidden rows handed to a middle stage (n_ctx rows)
    float * px;                // a split model's prompt: the residual rows of every position
    int cur_pos;               // position of the first row of the body being launched
} G;

static int (*g_mid_fn)(float *, int, int);
static int g_mid_layers;

// Test hook for callers that cannot reach sml_hip_fail_after (a server
// process): SML_GPU_FAIL=open:N fails the N-th HIP call of sml_gpu_open;
// prefill:N / step:N make the N-th call of that entry point fail at its
// first HIP call. Each entry point then returns its failure value, as after a
// real device error, and the caller's fallback runs.
static struct { char what[16]; long n, seen_prefill, seen_step; } g_fail;

static void fail_hook_read(void) {
    memset(&g_fail, 0, sizeof g_fail);
    const char * e = getenv("SML_GPU_FAIL");
    const char * c = e ? strchr(e, ':') : NULL;
    if (!c || c - e >= (long) sizeof g_fail.what) return;
    memcpy(g_fail.what, e, (size_t) (c - e));
    g_fail.n = atol(c + 1);
}

static void fail_hook(const char * entry, long * seen) {
    if (g_fail.n > 0 && !strcmp(g_fail.what, entry) && ++*seen == g_fail.n) hx.fail_after = 0;
}

static void * dalloc(size_t n) {
    if (G.ndev >= (int) (sizeof G.dev / sizeof G.dev[0])) hx_failf("too many device buffers");
    void * p = hx_malloc(n);
    G.dev[G.ndev++] = p;
    return p;
}

static void * dupload(const void * src, size_t n) {
    void * p = dalloc(n);
    HX(hipMemcpy(p, src, n, hipMemcpyHostToDevice));
    return p;
}

static sml_hip_mat * upmat(const ssf_file * f, const ssf_record * r) {
    if (G.nmats >= (int) (sizeof G.mats / sizeof G.mats[0])) hx_failf("too many matrices");
    sml_hip_mat * m = mat_from_record(f, r);
    G.mats[G.nmats++] = m;
    return m;
}

// Index of the record's permutation among the distinct ones uploaded; -1 for
// the identity (the gather is skipped).
static int perm_of(const ssf_file * f, const ssf_record * r) {
    const int n = (int) r->cols;
    if (!r->perm_bytes) return -1;
    if (!r->perm_off || r->perm_bytes < (uint64_t) n * 4)
        hx_failf("%.64s: permutation shorter than its %d columns", r->name, n);
    const int32_t * p = (const int32_t *) ssf_at(f, r->perm_off);
    int ident = 1;
    for (int i = 0; i < n && ident; i++) ident = p[i] == i;
    if (ident) return -1;
    for (int i = 0; i < G.nperm; i++)
        if (G.perm_len[i] == n && (G.perm_host[i] == p || memcmp(G.perm_host[i], p, (size_t) n * 4) == 0)) return i;
    if (G.nperm >= 512) hx_failf("too many distinct permutations");
    for (int i = 0; i < n; i++) if (p[i] < 0 || p[i] >= n) hx_failf("%.64s: permutation out of range", r->name);
    G.perm_host[G.nperm] = p;
    G.perm_len[G.nperm] = n;
    G.perm_dev[G.nperm] = dupload(p, (size_t) n * 4);
    return G.nperm++;
}

static const int32_t * pdev(int i) { return i < 0 ? NULL : G.perm_dev[i]; }

static float * f32_tensor(const ssf_file * f, const char * fmt, int L, int want) {
    const ssf_record * r = ssf_findf(f, fmt, L);
    if (!r) return NULL;
    if (r->kind != SSF_KIND_F32 || (uint64_t) r->rows * r->cols != (uint64_t) want)
        hx_failf("%.64s: expected %d f32 values", r->name, want);
    return dupload(ssf_at(f, r->f32_off), (size_t) want * 4);
}

static const ssf_record * need(const ssf_file * f, const char * fmt, int L) {
    const ssf_record * r = ssf_findf(f, fmt, L);
    if (!r) {
        char nm[96];
        snprintf(nm, sizeof nm, fmt, L);
        hx_failf("model has no %s", nm);
    }
    return r;
}

// ------------------------------------------------------------ one token

// normq into activation slots for up to three consumers, deduplicating by
// permutation; slot_of[i] receives consumer i's slot
static void prep(float * x, const float * w, const float * resid, int n, const int * perms, int ncons, int * slot_of) {
    const int32_t * pp[MAXACT];
    int8_t * qq[MAXACT];
    float * ss[MAXACT];
    int32_t * uu[MAXACT];
    int ids[MAXACT], nout = 0;
    for (int i = 0; i < ncons; i++) {
        int s = -1;
        for (int j = 0; j < nout; j++) if (ids[j] == perms[i]) s = j;
        if (s < 0) { s = nout++; ids[s] = perms[i]; }
        slot_of[i] = s;
    }
    for (int j = 0; j < nout; j++) { pp[j] = pdev(ids[j]); qq[j] = G.aq[j]; ss[j] = G.as[j]; uu[j] = G.asum[j]; }
    op_normq(G.st, x, resid, w, G.eps, n, nout, pp, qq, ss, uu, NULL, 0);
}

static void gemv1(sml_hip_mat * m, int slot, int epi, float * y, const float * bias, const float * resid) {
    op_gemv(G.st, m, NULL, epi, G.aq[slot], G.as[slot], G.asum[slot], y, bias, NULL, resid, NULL);
}

// the norm prologue is fused into a GEMV of this matrix (in exact mode only
// the Q4/Q8 GEMVs have exact prologues)
static int fusable(const sml_hip_mat * m) { return !G.exact || m->nbits == 4 || m->nbits == 8; }

static void launch_layer(int L) {
    eng_layer * y = &G.L[L];
    const size_t kvd = (size_t) G.KV * G.hd;
    int slot[3];
    // q/k/v: the stacked GEMV computes RMSNorm + quantize of x in its prologue
    if (y->qkv && (G.fuse & 1) && G.E <= gemv_fuse_max_cols(0) && fusable(y->qkv)) {
        gemv_fuse fu;
        memset(&fu, 0, sizeof fu);
        fu.x = G.x; fu.norm_w = y->an; fu.eps = G.eps; fu.perm = pdev(y->perm_qkv[0]);
        op_gemv(G.st, y->qkv, NULL, SML_EPI_STORE, NULL, NULL, NULL, G.q, y->bias_qkv, NULL, NULL, &fu);
    } else {
        prep(G.x, y->an, NULL, G.E, y->perm_qkv, 3, slot);
        if (y->qkv) gemv1(y->qkv, slot[0], SML_EPI_STORE, G.q, y->bias_qkv, NULL);
        else {
            float * outs[3] = { G.q, G.k, G.v };
            for (int i = 0; i < 3; i++) gemv1(y->w[i], slot[i], SML_EPI_STORE, outs[i], y->bias[i], NULL);
        }
    }
    // with an identity o-proj permutation the attention kernel quantizes its
    // own output for the o GEMV; otherwise a gather + quantize follows it
    const int fuse_q = y->perm_o < 0;
    uint16_t * kc = G.cur_slot ? G.kcs[G.cur_slot] : G.kc, * vc = G.cur_slot ? G.vcs[G.cur_slot] : G.vc;
    op_attention(G.st, G.q, G.k, G.v, kc + (size_t) L * G.n_ctx * kvd, vc + (size_t) L * G.n_ctx * kvd,
                 G.rc, G.rs, G.pos, G.H, G.KV, G.hd, G.n_ctx, G.pos_cap, G.part, G.att,
                 fuse_q ? G.aq[0] : NULL, fuse_q ? G.as[0] : NULL, fuse_q ? G.asum[0] : NULL, G.acnt);
    if (fuse_q) slot[0] = 0;
    else prep(G.att, NULL, NULL, G.H * G.hd, &y->perm_o, 1, slot);
    gemv1(y->o, slot[0], SML_EPI_RESIDUAL, G.x, NULL, G.x);
    if (y->moe) {
        // ffn_norm into fp32 for the router, then the routed experts; the
        // combine adds the residual (sml/sml-run.c:3470-3480)
        op_normq(G.st, G.x, NULL, y->fn, G.eps, G.E, 0, NULL, NULL, NULL, NULL, G.xn, 0);
        y->moe->per256 = 0;
        op_moe(G.st, y->moe, G.xn, 1, G.x, G.x);
        return;
    }
    // gate/up: one SwiGLU launch when they share a permutation and width; it
    // also quantizes h for down when down reads h in order
    // (in exact mode only behind the fused norm prologue)
    const int x_fusable = (G.fuse & 1) && fusable(y->gate);
    const int h_fused = (G.fuse & 2) && y->perm_down < 0 && G.F % 32 == 0 &&
                        (!G.exact || (x_fusable && G.E <= gemv_fuse_max_cols(1)));
    if (y->perm_gu[0] == y->perm_gu[1] && y->gate->nbits == y->up->nbits) {
        gemv_fuse fu;
        memset(&fu, 0, sizeof fu);
        const int x_fused = x_fusable && G.E <= gemv_fuse_max_cols(h_fused);
        if (x_fused) { fu.x = G.x; fu.norm_w = y->fn; fu.eps = G.eps; fu.perm = pdev(y->perm_gu[0]); }
        else prep(G.x, y->fn, NULL, G.E, y->perm_gu, 2, slot);
        if (h_fused) { fu.hq = G.hq; fu.hscale = G.hs; fu.hsums = G.hsum; }
        op_gemv(G.st, y->gate, y->up, SML_EPI_SWIGLU, x_fused ? NULL : G.aq[slot[0]], x_fused ? NULL : G.as[slot[0]],
                x_fused ? NULL : G.asum[slot[0]], G.hb, NULL, NULL, NULL, (x_fused || h_fused) ? &fu : NULL);
        if (h_fused) {
            op_gemv(G.st, y->down, NULL, SML_EPI_RESIDUAL, G.hq, G.hs, G.hsum, G.x, NULL, NULL, G.x, NULL);
            return;
        }
    } else {
        prep(G.x, y->fn, NULL, G.E, y->perm_gu, 2, slot);
        gemv1(y->gate, slot[0], SML_EPI_STORE, G.hb, NULL, NULL);
        gemv1(y->up, slot[1], SML_EPI_STORE, G.hb2, NULL, NULL);
        op_silu_mul(G.st, G.hb, G.hb2, G.F);
    }
    prep(G.hb, NULL, NULL, G.F, &y->perm_down, 1, slot);
    gemv1(y->down, slot[0], SML_EPI_RESIDUAL, G.x, NULL, G.x);
}

// A streamed layer's matrices into the staging region. The copy follows the
// previous layer's kernels on the stream, so it overwrites the region only
// once they are done with it.
static void stage_layer(int L) {
    if (L >= G.nres) HX(hipMemcpyAsync(G.stage, G.img[L], G.img_n[L], hipMemcpyHostToDevice, G.st));
}

// A middle stage of a split model (sml_gpu_set_middle): after the layers on
// the card, the caller's function runs the next g_mid_layers layers on the
// n hidden rows (positions pos0..pos0+n-1) in host memory, in place, and the
// layers after them continue here (sml/sml-gpu-fwd.c:1582-1587,1748-1754).
// It returns 0 on failure, which fails the call.
static int mid_on(void) { return G.nres < G.n_layer && g_mid_fn && g_mid_layers > 0; }

static void middle(float * rows, int n, int pos0) {
    if (G.nres + g_mid_layers > G.n_layer)
        hx_failf("a middle stage of %d layers after %d of %d", g_mid_layers, G.nres, G.n_layer);
    // room for a whole prompt (a split model's prompt hands over every row)
    if (!G.mid_host) HX(hipHostMalloc((void **) &G.mid_host, (size_t) G.n_ctx * G.E * 4, 0));
    if (n > G.n_ctx) hx_failf("a middle stage of %d rows", n);
    const size_t b = (size_t) n * G.E * 4;
    HX(hipMemcpyAsync(G.mid_host, rows, b, hipMemcpyDeviceToHost, G.st));
    HX(hipStreamSynchronize(G.st));
    if (!g_mid_fn(G.mid_host, pos0, n)) hx_failf("the middle stage failed at position %d", pos0);
    HX(hipMemcpyAsync(rows, G.mid_host, b, hipMemcpyHostToDevice, G.st));
}

static void launch_body(void) {
    op_embed(G.st, G.emb, G.hist, G.pos, pdev(G.perm_emb), G.x);
    for (int L = 0; L < G.n_layer; L++) {
        if (L == G.nres && mid_on()) {
            middle(G.x, 1, G.cur_pos);
            L += g_mid_layers - 1;
            continue;
        }
        stage_layer(L);
        launch_layer(L);
    }
}

static void launch_tail(void) {
    int slot[1];
    prep(G.x, G.out_norm, NULL, G.E, &G.perm_head, 1, slot);
    if (!G.exact && G.V >= ARGMAX_TWO_STAGE_MIN) {
        // the head GEMV's row blocks write the greedy pick's first stage
        // (one (max, lowest index) pair each), so one workgroup finishes it
        gemv_fuse fu;
        memset(&fu, 0, sizeof fu);
        fu.amax = G.head_pairs;
        const int np = op_gemv(G.st, G.head, NULL, SML_EPI_STORE, G.aq[slot[0]], G.as[slot[0]], G.asum[slot[0]],
                               G.logits, NULL, NULL, NULL, &fu);
        op_argmax_pairs(G.st, G.head_pairs, np, G.logits, G.tok, G.pos, G.hist, G.n_ctx + 1);
        return;
    }
    gemv1(G.head, slot[0], SML_EPI_STORE, G.logits, NULL, NULL);
    op_argmax(G.st, G.logits, G.V, G.tok, G.pos, G.hist, G.n_ctx + 1, G.amax_part);
}

static void launch_adv(void) { op_advance(G.st, G.pos); }

static hipGraphExec_t capture(void (*fn)(void)) {
    hipGraph_t g;
    hipGraphExec_t e;
    HX(hipStreamBeginCapture(G.st, hipStreamCaptureModeThreadLocal));
    // a failure while capturing ends the capture before it propagates, so the
    // stream is usable (and can be destroyed) afterwards
    jmp_buf * outer = hx.jb;
    jmp_buf jb;
    if (setjmp(jb)) {
        hipGraph_t dead = NULL;
        if (hipStreamEndCapture(G.st, &dead) == hipSuccess && dead) hipGraphDestroy(dead);
        hx.jb = outer;
        longjmp(*outer, 1);
    }
    hx.jb = &jb;
    fn();
    hx.jb = outer;
    HX(hipStreamEndCapture(G.st, &g));
    HX(hipGraphInstantiate(&e, g, NULL, NULL, 0));
    HX(hipGraphDestroy(g));
    return e;
}

static int bucket_of(int pos) { const int k = pos / G.bkt_len; return k < G.nbkt ? k : G.nbkt - 1; }
static int bucket_cap(int k) { const int c = (k + 1) * G.bkt_len; return c < G.n_ctx ? c : G.n_ctx; }

// one decode step's body at position pos (the device copy of pos holds it)
static void run_body(int pos) {
    G.cur_pos = pos;
    const int k = bucket_of(pos);
    G.pos_cap = bucket_cap(k);
    if (G.use_graph) HX(hipGraphLaunch(G.g_body[k], G.st));
    else launch_body();
}
static void run_tail(void) { if (G.use_graph) HX(hipGraphLaunch(G.g_tail, G.st)); else launch_tail(); }
static void run_adv(void) { if (G.use_graph) HX(hipGraphLaunch(G.g_adv, G.st)); else launch_adv(); }

// ------------------------------------------------------------ open / close

static void release(void) {
    // best effort: failures while tearing down are ignored
    jmp_buf * outer = hx.jb;
    jmp_buf jb;
    hx.jb = &jb;
    if (!setjmp(jb)) {
        if (G.st) hipStreamSynchronize(G.st);
        for (int k = 0; k < NBKT; k++) if (G.g_body[k]) hipGraphExecDestroy(G.g_body[k]);
        if (G.g_tail) hipGraphExecDestroy(G.g_tail);
        if (G.g_adv) hipGraphExecDestroy(G.g_adv);
        for (int i = 0; i < 17; i++)
            for (int j = 0; j < 2; j++)
                for (int k = 0; k < NBKT; k++) if (G.g_multi[i][j][k]) hipGraphExecDestroy(G.g_multi[i][j][k]);
        for (int i = 0; i < G.nmats; i++) { if (G.mats[i]->mem && !G.mats[i]->placed) hipFree(G.mats[i]->mem); free(G.mats[i]); }
        if (G.img) for (int L = 0; L < G.n_layer; L++) if (G.img[L]) hipHostFree(G.img[L]);
        if (G.mid_host) hipHostFree(G.mid_host);
        if (G.L) for (int L = 0; L < G.n_layer; L++) if (G.L[L].moe) { moe_free(G.L[L].moe); G.L[L].moe = NULL; }
        for (int i = 0; i < G.ndev; i++) hipFree(G.dev[i]);
        if (G.lg_host) hipHostFree(G.lg_host);
        if (G.pin) hipHostFree(G.pin);
        if (G.mpin) hipHostFree(G.mpin);
        if (G.mlog_host) hipHostFree(G.mlog_host);
        if (G.e0) hipEventDestroy(G.e0);
        if (G.e1) hipEventDestroy(G.e1);
        if (G.st) hipStreamDestroy(G.st);
    }
    hx.jb = outer;
    free(G.L);
    free(G.img);
    free(G.img_n);
    memset(&G, 0, sizeof G);
    ops_set_exact(0);
}

void sml_gpu_close(void) { release(); }

static int env_int(const char * name, int dflt) {
    const char * e = getenv(name);
    return e && *e ? atoi(e) : dflt;
}

// Refuse what this path does not compute rather than run it wrong
// (the reference does the same by name, sml/sml-gpu-fwd.c:1813-1865).
static const char * unsupported(const ssf_file * f) {
    const ssf_header * h = f->hdr;
    if (h->flags & SSF_FLAG_HADAMARD) return "Hadamard-rotated weights";
    if (h->flags & SSF_FLAG_EXACT) return "an exact-f32 file";
    if (h->n_levels != 1) return "LADDER codes";
    if (h->norm_type != 0) return "LayerNorm";
    if (h->rope_type != 0) return "interleaved RoPE";
    if (h->arch_bits) return "a non-Llama architecture flag";
    if (h->n_swa) return "sliding-window attention";
    if (h->attn_scale != 0.0f || h->logit_softcap != 0.0f || h->attn_softcap != 0.0f || h->clip_qkv != 0.0f)
        return "attention scale, soft caps or clamps";
    if (h->emb_scale != 0.0f || h->res_scale != 0.0f || h->logit_scale != 0.0f) return "embedding/residual/logit scales";
    if (h->n_rot) return "partial rotary";
    if (ssf_find(f, "rope_freqs") || ssf_find(f, "position_embd.weight")) return "stored or learned positions";
    const char * extra[] = { "blk.0.attn_q_norm.weight", "blk.0.attn_output.bias", "blk.0.ffn_up.bias",
                             "blk.0.ffn_down.bias", "blk.0.attn_norm.bias", "output.bias", "token_embd_norm.weight",
                             "blk.0.attn_post_norm.weight", "blk.0.ffn_post_norm.weight" };
    for (size_t i = 0; i < sizeof extra / sizeof extra[0]; i++)
        if (ssf_find(f, extra[i])) return "tensors of an architecture this path does not compute";
    return NULL;
}

// Bytes the matrices of layer L take in HBM (at most: q, k and v counted
// apart, as when they are not stacked).
static size_t layer_bytes(const ssf_file * f, int L) {
    static const char * nm[] = { "blk.%d.attn_q.weight", "blk.%d.attn_k.weight", "blk.%d.attn_v.weight",
                                 "blk.%d.attn_output.weight", "blk.%d.ffn_gate.weight", "blk.%d.ffn_up.weight",
                                 "blk.%d.ffn_down.weight" };
    size_t b = 0;
    for (size_t i = 0; i < sizeof nm / sizeof nm[0]; i++) {
        const ssf_record * r = ssf_findf(f, nm[i], L);
        if (r && r->kind == SSF_KIND_QUANT && r->nbits >= 2 && r->nbits <= 8 && r->cols % 128 == 0)
            b += mat_block_bytes((int) r->rows, (int) r->cols, (int) r->nbits);
    }
    return b;
}

// How many leading layers keep their matrices in HBM (the reference's
// gpu_layers, sml/sml-gpu-fwd.c:2028-2097): gpu_layers > 0, else
// SML_GPU_LAYERS, else every layer when the matrices, every layer's K/V
// cache, the embedding and head and SML_SPLIT_RESERVE_MB (1024) of scratch
// fit in the free HBM; otherwise the leading layers that fit beside one
// staging region. Streamed layers still compute here: their matrices cross
// the host link ahead of each use, so a split gives the same bits as the
// whole model on the card.
static void split_plan(const ssf_file * f, int n_ctx, int gpu_layers) {
    const int nl = G.n_layer;
    int k = nl;
    const int forced = gpu_layers > 0 ? gpu_layers : env_int("SML_GPU_LAYERS", 0);
    size_t stage = 0;
    if (forced > 0) {
        k = forced < nl ? forced : nl;
    } else {
        size_t fr = 0, tot = 0;
        if (hipMemGetInfo(&fr, &tot) == hipSuccess && fr) {
            size_t fixed = (size_t) 2 * nl * n_ctx * G.KV * G.hd * 2, all = 0;
            const ssf_record * er = ssf_find(f, "token_embd.weight"), * hr = ssf_find(f, "output.weight");
            if (er && er->kind == SSF_KIND_QUANT) fixed += mat_block_bytes((int) er->rows, (int) er->cols, (int) er->nbits);
            if (hr && hr->kind == SSF_KIND_QUANT) fixed += mat_block_bytes((int) hr->rows, (int) hr->cols, (int) hr->nbits);
            fixed += (size_t) env_int("SML_SPLIT_RESERVE_MB", 1024) << 20;
            for (int L = 0; L < nl; L++) {
                const size_t b = layer_bytes(f, L);
                all += b;
                if (b > stage) stage = b;
            }
            if (fixed + all > fr) {
                size_t used = 0;
                k = 0;
                while (k < nl && fixed + stage + used + layer_bytes(f, k) <= fr) used += layer_bytes(f, k++);
                if (k < 1) k = 1;
            }
        }
    }
    G.nres = k;
    if (k == nl) return;
    for (int L = k; L < nl; L++) {
        if (ssf_findf(f, "blk.%d.ffn_gate_inp.weight", L))
            hx_failf("a layer split of a mixture-of-experts model (%d of %d layers) is not built", k, nl);
        const size_t b = layer_bytes(f, L);
        if (b > stage) stage = b;
    }
    if (env_int("SML_TILED", 0)) hx_failf("a layer split streams the matrices as stored (SML_TILED=1 is not taken)");
    G.img = calloc((size_t) nl, sizeof(void *));
    G.img_n = calloc((size_t) nl, sizeof(size_t));
    if (!G.img || !G.img_n) hx_failf("out of host memory");
    G.stage_cap = stage;
    G.stage = dalloc(stage);
}

static void setup(const char * path, int want_ctx, int gpu_layers) {
    ssf_file f;
    char why[512];
    if (!ssf_open(&f, path, why, sizeof why)) hx_failf("%s", why);
    jmp_buf * outer = hx.jb;
    jmp_buf jb;
    if (setjmp(jb)) { mat_place(NULL, 0); ssf_close(&f); hx.jb = outer; longjmp(*outer, 1); }
    hx.jb = &jb;
    const ssf_header * h = f.hdr;
    const char * no = unsupported(&f);
    if (no) hx_failf("this GPU path does not compute %s", no);
    G.n_layer = (int) h->n_layer; G.E = (int) h->n_embd; G.H = (int) h->n_head; G.KV = (int) h->n_head_kv;
    G.F = (int) h->n_ff; G.V = (int) h->n_vocab; G.eps = h->rms_eps;
    const int n_ctx = want_ctx > 0 ? want_ctx : h->n_ctx_train ? (int) h->n_ctx_train : 4096;
    G.n_ctx = n_ctx;
    const ssf_record * q0 = need(&f, "blk.%d.attn_q.weight", 0);
    G.hd = (int) q0->rows / G.H;
    if ((int) q0->rows % G.H || (G.hd != 128 && G.hd != 64) || G.KV <= 0 || G.H % G.KV || G.H / G.KV > 8)
        hx_failf("attention shape (heads %d/%d, head_dim %d) not supported", G.H, G.KV, G.hd);
    hx_init(env_int("SML_DEVICE", 0));
    split_plan(&f, n_ctx, gpu_layers);
    HX(hipStreamCreateWithFlags(&G.st, hipStreamNonBlocking));
    HX(hipEventCreate(&G.e0));
    HX(hipEventCreate(&G.e1));
    const int half = G.hd / 2;
    // weights
    const ssf_record * er = need(&f, "token_embd.weight", 0);
    G.emb = upmat(&f, er);
    G.perm_emb = perm_of(&f, er);
    const ssf_record * hr = ssf_find(&f, "output.weight");
    if (hr) { G.head = upmat(&f, hr); G.perm_head = perm_of(&f, hr); }
    else { G.head = G.emb; G.perm_head = G.perm_emb; }
    G.weight_bytes = G.head->bytes;
    const ssf_record * on = need(&f, "output_norm.weight", 0);
    G.out_norm = f32_tensor(&f, "output_norm.weight", 0, G.E);
    (void) on;
    G.L = calloc((size_t) G.n_layer, sizeof(eng_layer));
    if (!G.L) hx_failf("out of host memory");
    const char * wn[3] = { "blk.%d.attn_q.weight", "blk.%d.attn_k.weight", "blk.%d.attn_v.weight" };
    const char * bn[3] = { "blk.%d.attn_q.bias", "blk.%d.attn_k.bias", "blk.%d.attn_v.bias" };
    const int wrows[3] = { G.H * G.hd, G.KV * G.hd, G.KV * G.hd };
    const int qkv_rows = wrows[0] + wrows[1] + wrows[2];
    for (int L = 0; L < G.n_layer; L++) {
        eng_layer * y = &G.L[L];
        if (L >= G.nres) mat_place(G.stage, G.stage_cap);
        const ssf_record * rq[3];
        for (int i = 0; i < 3; i++) {
            rq[i] = need(&f, wn[i], L);
            if ((int) rq[i]->rows != wrows[i] || (int) rq[i]->cols != G.E) hx_failf("%.64s has an unexpected shape", rq[i]->name);
            y->perm_qkv[i] = perm_of(&f, rq[i]);
            y->bias[i] = f32_tensor(&f, bn[i], L, wrows[i]);
        }
        // q, k and v read the same input: one stacked matrix and one GEMV
        // when they share a permutation and width
        if (y->perm_qkv[1] == y->perm_qkv[0] && y->perm_qkv[2] == y->perm_qkv[0]) {
            if (G.nmats >= (int) (sizeof G.mats / sizeof G.mats[0])) hx_failf("too many matrices");
            y->qkv = mat_stack(&f, rq, 3);
            if (y->qkv) G.mats[G.nmats++] = y->qkv;
        }
        if (y->qkv) {
            if (y->bias[0] || y->bias[1] || y->bias[2]) {
                y->bias_qkv = dalloc((size_t) qkv_rows * 4);
                float * at = y->bias_qkv;
                for (int i = 0; i < 3; i++) {
                    if (y->bias[i]) HX(hipMemcpy(at, y->bias[i], (size_t) wrows[i] * 4, hipMemcpyDeviceToDevice));
                    else HX(hipMemset(at, 0, (size_t) wrows[i] * 4));
                    at += wrows[i];
                }
            }
            G.weight_bytes += y->qkv->bytes;
        } else {
            for (int i = 0; i < 3; i++) { y->w[i] = upmat(&f, rq[i]); G.weight_bytes += y->w[i]->bytes; }
        }
        const ssf_record * r;
        r = need(&f, "blk.%d.attn_output.weight", L); y->o = upmat(&f, r); y->perm_o = perm_of(&f, r);
        if (ssf_findf(&f, "blk.%d.ffn_gate_inp.weight", L)) {
            y->moe = moe_load(&f, L, MAX_SLOTS, G.moe_first);
            if (!G.moe_first) G.moe_first = y->moe;
            // bytes one step reads: the router and the k chosen experts
            G.weight_bytes += (uint64_t) y->moe->k * y->moe->expert_bytes + (uint64_t) y->moe->nexp * G.E * 4;
            if (y->o->k.rows != G.E || y->o->cols != G.H * G.hd) hx_failf("layer %d has unexpected projection shapes", L);
        } else {
            r = need(&f, "blk.%d.ffn_gate.weight", L); y->gate = upmat(&f, r); y->perm_gu[0] = perm_of(&f, r);
            r = need(&f, "blk.%d.ffn_up.weight", L); y->up = upmat(&f, r); y->perm_gu[1] = perm_of(&f, r);
            r = need(&f, "blk.%d.ffn_down.weight", L); y->down = upmat(&f, r); y->perm_down = perm_of(&f, r);
            if (y->o->k.rows != G.E || y->o->cols != G.H * G.hd || y->gate->k.rows != G.F || y->up->k.rows != G.F ||
                y->down->k.rows != G.E || y->down->cols != G.F)
                hx_failf("layer %d has unexpected projection shapes", L);
            G.weight_bytes += y->gate->bytes + y->up->bytes + y->down->bytes;
        }
        if (L >= G.nres) {
            // the layer's matrices as laid out in the staging region, kept on the host
            const size_t used = mat_place_used();
            mat_place(NULL, 0);
            HX(hipHostMalloc(&G.img[L], used, 0));
            HX(hipMemcpy(G.img[L], G.stage, used, hipMemcpyDeviceToHost));
            G.img_n[L] = used;
        }
        y->an = f32_tensor(&f, "blk.%d.attn_norm.weight", L, G.E);
        y->fn = f32_tensor(&f, "blk.%d.ffn_norm.weight", L, G.E);
        if (!y->an || !y->fn) hx_failf("layer %d lacks a norm", L);
        G.weight_bytes += y->o->bytes;
    }
    // RoPE table on the host, exactly as the reference builds it (sml/sml-run.c:1383-1393)
    {
        const size_t nt = (size_t) n_ctx * half;
        float * c = malloc(nt * 4), * s = malloc(nt * 4);
        if (!c || !s) { free(c); free(s); hx_failf("out of host memory"); }
        for (int p = 0; p < n_ctx; p++)
            for (int i = 0; i < half; i++) {
                const float freq = powf(h->rope_theta, -(float) i / (float) half);
                const float a = (float) p * freq;
                c[(size_t) p * half + i] = cosf(a);
                s[(size_t) p * half + i] = sinf(a);
            }
        G.rc = dupload(c, nt * 4);
        G.rs = dupload(s, nt * 4);
        free(c); free(s);
    }
    // activations and cache
    int wide = G.F > G.E ? G.F : G.E;
    if (G.H * G.hd > wide) wide = G.H * G.hd;
    G.x = dalloc((size_t) G.E * 4);
    // q, k and v contiguous: the stacked GEMV writes all three
    G.q = dalloc((size_t) (G.H + 2 * G.KV) * G.hd * 4);
    G.k = G.q + (size_t) G.H * G.hd;
    G.v = G.k + (size_t) G.KV * G.hd;
    G.att = dalloc((size_t) G.H * G.hd * 4);
    G.hb = dalloc((size_t) G.F * 4);
    G.hb2 = dalloc((size_t) G.F * 4);
    G.logits = dalloc((size_t) G.V * 4);
    G.part = dalloc(sml_hip_attn_part_floats(G.H, G.hd, n_ctx) * 4);
    // SML_ATTN_FOLD=1: the merge runs in the attention launch's last split of
    // each kv head (counters, one per kv head, zero between launches). Off by
    // default: measured slower at 4096 positions (Llama-3-8B shape 12.8 us
    // per layer against 8.1 + 3.2 for the two launches; Qwen2.5-1.5B shape
    // 14.8 against 7.8 + 3.9): the last split's device-scope store, count and
    // re-read of every partial from memory sit on the launch's critical path.
    G.acnt = NULL;
    if (env_int("SML_ATTN_FOLD", 0)) {
        G.acnt = dalloc((size_t) G.KV * 4);
        HX(hipMemset(G.acnt, 0, (size_t) G.KV * 4));
    }
    for (int i = 0; i < MAXACT; i++) {
        G.aq[i] = dalloc((size_t) wide);
        G.as[i] = dalloc((size_t) wide / 32 * 4);
        G.asum[i] = dalloc((size_t) wide / 32 * 4);
    }
    G.xn = dalloc((size_t) G.E * 4);
    G.hq = dalloc((size_t) G.F);
    G.hs = dalloc((size_t) G.F / 32 * 4);
    G.hsum = dalloc((size_t) G.F / 32 * 4);
    G.fuse = env_int("SML_FUSE", 3);
    // exact mode: the reference's float order throughout (sml_forward,
    // sml/sml-run.c:3243-3523), so logits equal its CPU path bit for bit.
    // Prompts read a token at a time.
    G.exact = env_int("SML_EXACT", 0) != 0;
    ops_set_exact(G.exact);
    if (G.exact) {
        // the norm prologues and the h quantization have exact forms (Q4/Q8)
        if (n_ctx > 16384) hx_failf("exact mode holds at most 16384 positions");
        if (G.hd != 128) hx_failf("exact mode takes head_dim 128 (this model: %d)", G.hd);
    }
    const size_t kvn = (size_t) G.n_layer * n_ctx * G.KV * G.hd;
    G.kc = dalloc(kvn * 2);
    G.vc = dalloc(kvn * 2);
    HX(hipMemset(G.kc, 0, kvn * 2));
    HX(hipMemset(G.vc, 0, kvn * 2));
    G.hist = dalloc((size_t) (n_ctx + 1) * 4);
    HX(hipMemset(G.hist, 0, (size_t) (n_ctx + 1) * 4));
    G.pos = dalloc(64);
    G.amax_part = dalloc((size_t) ARGMAX_MAX_PARTS * sizeof(int2));
    G.head_pairs = dalloc((size_t) G.V * sizeof(int2));
    G.tok = dalloc(64);
    HX(hipMemset(G.pos, 0, 64));
    HX(hipHostMalloc((void **) &G.lg_host, (size_t) G.V * 4, 0));
    HX(hipHostMalloc((void **) &G.pin, (size_t) (n_ctx + 8) * 4, 0));
    HX(hipDeviceSynchronize());
    // prompt reading: batched (exact) unless SML_GPU_PP=0, as the reference's
    // open does (sml/sml-gpu-fwd.c:2371-2375); in exact mode level 1 is the
    // reference-order batched prompt where every product takes it (rows_check)
    G.prompt_level = env_int("SML_GPU_PP", 1) == 0 ? 0 : 1;
    // level-2 chunk: SML_PB positions (16..4096, default 512); MoE layers
    // take at most MAX_SLOTS rows per call
    G.pb = env_int("SML_PB", 512);
    if (G.pb < MAX_SLOTS) G.pb = MAX_SLOTS;
    if (G.pb > 4096) G.pb = 4096;
    if (G.pb > n_ctx) G.pb = n_ctx > MAX_SLOTS ? n_ctx : MAX_SLOTS;
    if (G.moe_first) G.pb = MAX_SLOTS;
    G.rrows = G.pb;
    G.rows_ok = -1;
    // a split model launches directly: each streamed layer's copy sits
    // between its neighbours' kernels, and a middle stage runs on the host
    G.use_graph = env_int("SML_GRAPH", 1) != 0 && G.nres == G.n_layer;
    // position buckets: at most NBKT, none shorter than 512 positions
    // (SML_POS_BUCKETS=0: one, every launch covering the whole context)
    G.bkt_len = (G.n_ctx + NBKT - 1) / NBKT;
    G.bkt_len = (G.bkt_len + 127) / 128 * 128;
    if (G.bkt_len < 512) G.bkt_len = 512;
    if (!env_int("SML_POS_BUCKETS", 1)) G.bkt_len = G.n_ctx;
    G.nbkt = (G.n_ctx + G.bkt_len - 1) / G.bkt_len;
    G.pos_cap = G.n_ctx;
    if (G.use_graph) {
        for (int k = 0; k < G.nbkt; k++) {
            G.pos_cap = bucket_cap(k);
            G.g_body[k] = capture(launch_body);
        }
        G.pos_cap = G.n_ctx;
        G.g_tail = capture(launch_tail);
        G.g_adv = capture(launch_adv);
    }
    hx.jb = outer;
    ssf_close(&f);
}

int sml_gpu_open(const char * path, int n_ctx, int threads, int gpu_layers, char * why, int nwhy) {
    (void) threads;
    if (G.open) release();
    fail_hook_read();
    if (g_fail.n > 0 && !strcmp(g_fail.what, "open")) hx.fail_after = g_fail.n - 1;
    HX_ENTRY(0);
    jmp_buf * outer = hx.jb;
    jmp_buf jb;
    if (setjmp(jb)) {
        hx.jb = outer;
        if (why && nwhy > 0) snprintf(why, (size_t) nwhy, "%s", hx.err);
        release();
        HX_LEAVE();
        return 0;
    }
    hx.jb = &jb;
    setup(path, n_ctx, gpu_layers);
    hx.jb = outer;
    if (g_fail.n > 0 && !strcmp(g_fail.what, "open")) hx.fail_after = -1;   // the open made fewer calls
    G.open = 1;
    HX_LEAVE();
    return 1;
}

// ------------------------------------------------------------ decode

static void fetch_logits(void) {
    HX(hipMemcpyAsync(G.lg_host, G.logits, (size_t) G.V * 4, hipMemcpyDeviceToHost, G.st));
    HX(hipStreamSynchronize(G.st));
}

const float * sml_gpu_step(int tok, int pos) {
    if (!G.open || pos < 0 || pos >= G.n_ctx || tok < 0 || tok >= G.V) return NULL;
    fail_hook("step", &g_fail.seen_step);
    HX_ENTRY(NULL);
    G.pin[0] = tok;
    G.pin[1] = pos;
    HX(hipMemcpyAsync(G.hist + pos, &G.pin[0], 4, hipMemcpyHostToDevice, G.st));
    HX(hipMemcpyAsync(G.pos, &G.pin[1], 4, hipMemcpyHostToDevice, G.st));
    run_body(pos);
    run_tail();
    fetch_logits();
    HX_LEAVE();
    return G.lg_host;
}

static void prefill_rows(int slot, int pos0, int n);
static int rows_check(void);

// A prompt, batched (prompt level 1 or 2, the reference's default) or a token
// at a time through the decode graph (level 0, SML_GPU_PP=0).
const float * sml_gpu_prefill(const int * ids, int pos0, int n) {
    if (!G.open || n <= 0 || pos0 < 0 || pos0 + n > G.n_ctx) return NULL;
    for (int i = 0; i < n; i++) if (ids[i] < 0 || ids[i] >= G.V) return NULL;
    fail_hook("prefill", &g_fail.seen_prefill);
    HX_ENTRY(NULL);
    memcpy(G.pin + 2, ids, (size_t) n * 4);
    HX(hipMemcpyAsync(G.hist + pos0, G.pin + 2, (size_t) n * 4, hipMemcpyHostToDevice, G.st));
    if (G.prompt_level >= 1 && n > 1 && rows_check()) {
        prefill_rows(0, pos0, n);
        G.pin[1] = pos0 + n - 1;
        HX(hipMemcpyAsync(G.pos, &G.pin[1], 4, hipMemcpyHostToDevice, G.st));
    } else {
        G.pin[1] = pos0;
        HX(hipMemcpyAsync(G.pos, &G.pin[1], 4, hipMemcpyHostToDevice, G.st));
        for (int i = 0; i < n; i++) {
            run_body(pos0 + i);
            if (i + 1 < n) run_adv();
        }
    }
    run_tail();
    fetch_logits();
    HX_LEAVE();
    return G.lg_host;
}

int sml_gpu_generate(int tok, int pos, int n, int * out) {
    if (!G.open || n <= 0 || pos < 0 || pos + n > G.n_ctx || tok < 0 || tok >= G.V) return -1;
    HX_ENTRY(-1);
    G.pin[0] = tok;
    G.pin[1] = pos;
    HX(hipMemcpyAsync(G.hist + pos, &G.pin[0], 4, hipMemcpyHostToDevice, G.st));
    HX(hipMemcpyAsync(G.pos, &G.pin[1], 4, hipMemcpyHostToDevice, G.st));
    HX(hipEventRecord(G.e0, G.st));
    for (int i = 0; i < n; i++) { run_body(pos + i); run_tail(); }
    HX(hipEventRecord(G.e1, G.st));
    HX(hipMemcpyAsync(G.pin + 2, G.hist + pos + 1, (size_t) n * 4, hipMemcpyDeviceToHost, G.st));
    HX(hipStreamSynchronize(G.st));
    HX(hipEventElapsedTime(&G.last_ms, G.e0, G.e1));
    memcpy(out, G.pin + 2, (size_t) n * 4);
    HX_LEAVE();
    return n;
}

float sml_gpu_last_ms(void) { return G.open ? G.last_ms : -1.0f; }
uint64_t sml_gpu_weight_bytes(void) { return G.open ? G.weight_bytes : 0; }
const char * sml_gpu_last_error(void) { return hx.err; }
int sml_gpu_exact(void) { return G.open && G.exact; }

// Layers whose matrices stay in HBM, of how many (a split streams the rest).
int sml_gpu_layers(int * of) {
    if (of) *of = G.open ? G.n_layer : 0;
    return G.open ? G.nres : 0;
}

// 0: prompts a token at a time through the decode graph; 1: batched, exact
// (the default); 2: batched with the Q4 products on MFMA. As the reference's
// (sml/sml-gpu-fwd.c:2420-2423): 2 = every batched kernel, 1 = without the
// matrix-core one, 0 = token at a time.
void sml_gpu_prompt_mode(int level) { G.prompt_level = level <= 0 ? 0 : level >= 2 && !G.exact ? 2 : 1; }

int sml_gpu_decode_cpu(int on) { (void) on; return 0; }

void sml_gpu_set_middle(int layers, int (*fn)(float * rows, int pos0, int n)) {
    g_mid_layers = layers;
    g_mid_fn = fn;
}

// ---------------------------------------------------------------- several sequences
//
// The GPU twin of sml_forward_multi (sml/sml-run.c:2559-2599): each weight
// matrix streams once per step for all sequences through the small-M GEMM;
// attention runs per sequence over that sequence's KV cache slot. The
// activation regime is the reference's choice (sml/sml-run.c:2579-2596):
// SML_MULTI=exact, or at most SML_MULTI_EXACT_MAX (default 2) sequences,
// quantizes per 32 values and gives each row the GEMV's arithmetic, so every
// sequence is bit for bit as decoded alone; otherwise activations are
// quantized per 256 values (sml_quantize_act_sb) and Q4 products sum each
// superblock in integers, the arithmetic of sml_rlp_matvec.

static int multi_per256(int ns) {
    const char * x = getenv("SML_MULTI");
    if (x && !strcmp(x, "exact")) return 0;
    const char * e = getenv("SML_MULTI_EXACT_MAX");
    return ns > (e ? atoi(e) : 2);
}

// Whether the batched body can run this model: q, k and v stacked as one
// matrix, and gate/up sharing a permutation and width (the MoE layers batch
// by themselves). Builds the (gate, up) tables on first use.
// A Q4 matrix 256-aligned: the exact batched GEMM's input
static int xgemm_ok(const sml_hip_mat * m) { return m && (m->nbits == 4 || m->nbits == 8) && m->cols % 256 == 0; }

static int rows_check(void) {
    if (G.rows_ok >= 0) return G.rows_ok;
    for (int L = 0; L < G.n_layer; L++) {
        eng_layer * y = &G.L[L];
        if (!y->qkv || (!y->moe && (y->perm_gu[0] != y->perm_gu[1] || y->gate->nbits != y->up->nbits))) {
            G.rows_ok = 0;
            return 0;
        }
        // exact mode batches prompts of dense Q4/Q8 layers only (the
        // reference-order GEMM); anything else reads them a token at a time
        if (G.exact && (y->moe || !xgemm_ok(y->qkv) || !xgemm_ok(y->o) || !xgemm_ok(y->gate) || !xgemm_ok(y->up) ||
                        !xgemm_ok(y->down))) {
            G.rows_ok = 0;
            return 0;
        }
    }
    // a failure part way leaves rows_ok unset, so the next call finishes the tables
    for (int L = 0; L < G.n_layer; L++) {
        eng_layer * y = &G.L[L];
        if (!y->moe && !y->gu_tab) {
            const sml_kmat t[2] = { y->gate->k, y->up->k };
            y->gu_tab = dupload(t, sizeof t);
        }
    }
    G.rows_ok = 1;
    return 1;
}

static void rows_tables(void) {
    G.kcs[0] = G.kc;
    G.vcs[0] = G.vc;
    HX(hipMemcpy(G.kc_tab, G.kcs, MAX_SLOTS * sizeof(void *), hipMemcpyHostToDevice));
    HX(hipMemcpy(G.vc_tab, G.vcs, MAX_SLOTS * sizeof(void *), hipMemcpyHostToDevice));
}

// The batched body's buffers, for up to MAX_SLOTS rows (sequences, or
// positions of one prompt chunk).
static void rows_alloc(void) {
    if (G.rows_ready) return;     // set last: a failed attempt allocates afresh next time
    const size_t R = (size_t) G.rrows, S = MAX_SLOTS;
    size_t wide = (size_t) (G.F > G.E ? G.F : G.E);
    if ((size_t) G.H * G.hd > wide) wide = (size_t) G.H * G.hd;
    G.mx = dalloc(R * G.E * 4);
    G.mxn = dalloc(R * G.E * 4);
    G.mqkv = dalloc(R * (size_t) (G.H + 2 * G.KV) * G.hd * 4);
    G.matt = dalloc(R * (size_t) G.H * G.hd * 4);
    G.mh = dalloc(R * (size_t) G.F * 4);
    G.mlog = dalloc(S * (size_t) G.V * 4);          // the multi-sequence step's heads
    G.maq = dalloc(R * wide);
    G.mas = dalloc(R * wide / 32 * 4);
    G.masum = dalloc(R * wide / 32 * 4);
    G.mtok = dalloc(S * 4);
    G.mpos = dalloc(S * 4);
    G.mslot = dalloc(S * 4);
    // partials: MAX_SLOTS entries at the decode kernels' finest split, or
    // (level-2 prompts, the wave-per-position kernel) rrows at splits of 128
    size_t part = S * sml_hip_attn_part_floats(G.H, G.hd, G.n_ctx);
    const size_t part_pb = R * (size_t) G.H * (size_t) ((G.n_ctx + 127) / 128) * (size_t) (G.hd + 2);
    if (part_pb > part) part = part_pb;
    G.mpart = dalloc(part * 4);
    G.mpart_floats = part;
    // exact mode reads a prompt in chunks whose reference-order scores
    // ([rows][H][n_ctx] floats) fit in the partials buffer: at most 64 rows
    G.xchunk = (int) (part / ((size_t) G.H * (size_t) G.n_ctx));
    if (G.xchunk > 64) G.xchunk = 64;
    if (G.xchunk > G.rrows) G.xchunk = G.rrows;
    hx_kpart();                                     // the split-K products' buffer, before any capture
    G.kc_tab = dalloc(S * sizeof(void *));
    G.vc_tab = dalloc(S * sizeof(void *));
    HX(hipHostMalloc((void **) &G.mpin, 3 * S * 4, 0));
    HX(hipHostMalloc((void **) &G.mlog_host, S * (size_t) G.V * 4, 0));
    int32_t * h = malloc((size_t) (G.n_ctx > (int) (S * R) ? G.n_ctx : (int) (S * R)) * 4);
    if (!h) hx_failf("out of host memory");
    for (int i = 0; i < G.n_ctx; i++) h[i] = i;
    G.iota = dalloc((size_t) G.n_ctx * 4);
    HX(hipMemcpy(G.iota, h, (size_t) G.n_ctx * 4, hipMemcpyHostToDevice));
    for (int i = 0; i < (int) (S * R); i++) h[i] = i / (int) R;
    G.slotid = dalloc(S * R * 4);
    HX(hipMemcpy(G.slotid, h, S * R * 4, hipMemcpyHostToDevice));
    free(h);
    rows_tables();
    G.rows_ready = 1;
}

int sml_gpu_slots(int ns) {
    if (!G.open || ns < 1 || ns > MAX_SLOTS) return 0;
    HX_ENTRY(0);
    if (G.exact) hx_failf("exact mode decodes one sequence");
    if (!rows_check()) {
        for (int L = 0; L < G.n_layer; L++) {
            eng_layer * y = &G.L[L];
            if (!y->qkv) hx_failf("layer %d: q, k and v are not one matrix; the batched step needs them stacked", L);
        }
        hx_failf("gate and up differ in permutation or width");
    }
    rows_alloc();
    const size_t kvn = (size_t) G.n_layer * G.n_ctx * G.KV * G.hd;
    for (int s = G.nslot > 1 ? G.nslot : 1; s < ns; s++) {
        G.kcs[s] = dalloc(kvn * 2);
        G.vcs[s] = dalloc(kvn * 2);
        HX(hipMemset(G.kcs[s], 0, kvn * 2));
        HX(hipMemset(G.vcs[s], 0, kvn * 2));
    }
    if (ns > G.nslot) G.nslot = ns;
    rows_tables();
    HX(hipDeviceSynchronize());
    HX_LEAVE();
    return ns;
}

// The batched body for ns rows: row b is token tok[b] at position pos[b] of
// slot slot[b]'s cache (device arrays). Every weight matrix streams once for
// all rows. causal: rows may be positions of one sequence (a prompt chunk),
// so K/V are written for every row before any row attends. head: logits of
// every row into G.mlog; otherwise the residuals stay in G.mx.
// Layer L of the batched body for the ns rows of G.mx (defer: leave the
// down product's split-K sums to the next norm).
static void rows_layer(int L, int ns, const int32_t * pos, const int32_t * slot, int regime, int causal, int defer) {
    const size_t kvd = (size_t) G.KV * G.hd, qkv = (size_t) (G.H + 2 * G.KV) * G.hd, hq = (size_t) G.H * G.hd;
    const int mt = gemm_mt(ns), sb = regime == GEMM_PER256;
    eng_layer * y = &G.L[L];
    const int32_t * pp[1];
    int8_t * qq[1] = { G.maq };
    float * ss[1] = { G.mas };
    int32_t * uu[1] = { G.masum };
    pp[0] = pdev(y->perm_qkv[0]);
    if (ops_ksum_pending()) op_ksum_normq_rows(G.st, G.mx, y->an, G.eps, G.E, ns, 1, pp, qq, ss, uu, sb);
    else op_normq_rows(G.st, G.mx, NULL, y->an, G.eps, G.E, ns, 1, pp, qq, ss, uu, NULL, sb);
    op_gemm(G.st, y->qkv->kdev, &y->qkv->k, 1, 0, y->qkv->nbits, (int) qkv, G.E, NULL, ns, mt, ns, G.maq, G.mas, G.masum,
            G.mqkv, y->bias_qkv, NULL, regime);
    // the merge quantizes its output for the o product: per 32, or per
    // 256 in decode steps of an even head count (SML_MERGE_Q256=0 leaves
    // that to its own launch)
    const int fuse_q = y->perm_o < 0 &&
                       (!sb || (!causal && G.H % 2 == 0 && G.hd == 128 && env_int("SML_MERGE_Q256", 1)));
    if (regime == GEMM_REF) {
        // exact mode: one sequence (slot 0), the reference's order
        if (!causal) hx_failf("exact mode batches prompts only");
        op_attention_rows_exact(G.st, G.mqkv, (int) qkv, G.kc + (size_t) L * G.n_ctx * kvd,
                                G.vc + (size_t) L * G.n_ctx * kvd, G.rc, G.rs, pos, ns, G.H, G.KV, G.n_ctx,
                                G.pos_cap, G.mpart, G.matt, fuse_q ? G.maq : NULL, fuse_q ? G.mas : NULL,
                                fuse_q ? G.masum : NULL);
    } else {
        op_attention_batch(G.st, G.mqkv, (int) qkv, G.kc_tab, G.vc_tab, slot, (size_t) L * G.n_ctx * kvd,
                           G.rc, G.rs, pos, ns, G.H, G.KV, G.hd, G.n_ctx, G.pos_cap, G.mpart, G.matt,
                           fuse_q ? G.maq : NULL, fuse_q ? G.mas : NULL, fuse_q ? G.masum : NULL,
                           causal ? (regime == GEMM_EXACT ? 1 : 2) : 0, gemm_exact(regime, ns), sb);
    }
    if (!fuse_q) {
        pp[0] = pdev(y->perm_o);
        op_normq_rows(G.st, G.matt, NULL, NULL, G.eps, (int) hq, ns, 1, pp, qq, ss, uu, NULL, sb);
    }
    op_gemm(G.st, y->o->kdev, &y->o->k, 1, 0, y->o->nbits, G.E, (int) hq, NULL, ns, mt, ns, G.maq, G.mas, G.masum,
            G.mx, NULL, G.mx, regime);
    if (y->moe) {
        op_normq_rows(G.st, G.mx, NULL, y->fn, G.eps, G.E, ns, 0, NULL, NULL, NULL, NULL, G.mxn, sb);
        y->moe->per256 = sb;
        op_moe(G.st, y->moe, G.mxn, ns, G.mx, G.mx);
        y->moe->per256 = 0;
        return;
    }
    pp[0] = pdev(y->perm_gu[0]);
    op_normq_rows(G.st, G.mx, NULL, y->fn, G.eps, G.E, ns, 1, pp, qq, ss, uu, NULL, sb);
    const sml_kmat guk[2] = { y->gate->k, y->up->k };
    op_gemm(G.st, y->gu_tab, guk, 1, 1, y->gate->nbits, G.F, G.E, NULL, ns, mt, ns, G.maq, G.mas, G.masum, G.mh,
            NULL, NULL, regime);
    pp[0] = pdev(y->perm_down);
    op_normq_rows(G.st, G.mh, NULL, NULL, G.eps, G.F, ns, 1, pp, qq, ss, uu, NULL, sb);
    ops_defer_ksum(defer);
    op_gemm(G.st, y->down->kdev, &y->down->k, 1, 0, y->down->nbits, G.E, G.F, NULL, ns, mt, ns, G.maq, G.mas, G.masum,
            G.mx, NULL, G.mx, regime);
    ops_defer_ksum(0);
}

static void launch_rows(int ns, const int32_t * tok, const int32_t * pos, const int32_t * slot, int regime,
                        int causal, int head) {
    const int mt = gemm_mt(ns), sb = regime == GEMM_PER256;
    // SML_KSUM_NORMQ=1: a batched step leaves the down product's split-K
    // sums to the next norm, which adds them as it normalizes (one launch
    // instead of two, the same bits). Off by default: replayed from a graph,
    // the 16-sequence Llama step measured 3.061 ms against 3.047 for the two
    // launches (directly launched, 3.15 against 3.19: the graph already hides
    // most of a launch boundary, and the one workgroup a row of the fused
    // kernel takes longer than the two wide launches' bodies).
    ops_ksum_reset();
    const int defer = head && !mid_on() && regime != GEMM_REF && env_int("SML_KSUM_NORMQ", 0);
    op_embed_rows(G.st, G.emb, tok, NULL, ns, pdev(G.perm_emb), G.mx);
    for (int L = 0; L < G.n_layer; L++) {
        if (L == G.nres && mid_on()) {
            // the rows of one prompt chunk (slot 0), positions cur_pos..
            if (!causal) hx_failf("a middle stage serves one sequence, not a batched step");
            middle(G.mx, ns, G.cur_pos);
            L += g_mid_layers - 1;
            continue;
        }
        stage_layer(L);
        rows_layer(L, ns, pos, slot, regime, causal, defer);
    }
    if (!head) return;
    const int32_t * pp[1] = { pdev(G.perm_head) };
    int8_t * qq[1] = { G.maq };
    float * ss[1] = { G.mas };
    int32_t * uu[1] = { G.masum };
    if (ops_ksum_pending()) op_ksum_normq_rows(G.st, G.mx, G.out_norm, G.eps, G.E, ns, 1, pp, qq, ss, uu, sb);
    else op_normq_rows(G.st, G.mx, NULL, G.out_norm, G.eps, G.E, ns, 1, pp, qq, ss, uu, NULL, sb);
    op_gemm(G.st, G.head->kdev, &G.head->k, 1, 0, G.head->nbits, G.V, G.E, NULL, ns, mt, ns, G.maq, G.mas, G.masum, G.mlog,
            NULL, NULL, regime);
}

// Batched prompt reading, the reference's gpu_prefill (sml/sml-gpu-fwd.c:
// 1418-1603): chunks of positions through the batched body, each weight
// matrix streamed once per chunk; the last position's residual then goes
// through the decode tail (final norm, head, greedy pick). The ids are
// already in G.hist.
//  - level 1: chunks of 32 positions (16 with MoE layers); every product is
//    the GEMV's arithmetic and the attention the decode kernel's, so the
//    cache, the residuals and the logits equal reading the prompt a token at
//    a time, bit for bit.
//  - exact mode: chunks of 64 through the reference-order GEMM and attention.
//  - level 2: chunks of pb (512) positions in the reference's prompt regime
//    (activations per 256 values, integer superblock sums: the CPU engine's
//    default prompt arithmetic, sml/sml-run.c:1929-1945), Q4 products on the
//    prompt MFMA GEMM, attention a wave per position.
// A split model's prompt, layer by layer: each layer runs over every chunk
// before the next starts, so a streamed layer crosses the host link once per
// prompt instead of once per chunk. The residual rows of all n positions
// wait in G.px; the chunks of one layer run in order, so each chunk's
// attention finds the earlier positions' K/V of that layer written, and
// every chunk computes what the chunk-major order does (the same bits). A
// middle stage receives all n rows at once, as the reference's does
// (sml/sml-gpu-fwd.c:1582-1587).
static void prefill_layers(int slot, int pos0, int n, int chunk, int regime) {
    if (!G.px) G.px = dalloc((size_t) G.n_ctx * G.E * 4);
    float * const mx = G.mx;
    jmp_buf * outer = hx.jb;
    jmp_buf jb;
    if (setjmp(jb)) { G.mx = mx; G.pos_cap = G.n_ctx; hx.jb = outer; longjmp(*outer, 1); }
    hx.jb = &jb;
    ops_ksum_reset();
    for (int p0 = 0; p0 < n; p0 += chunk) {
        const int nb = n - p0 < chunk ? n - p0 : chunk;
        op_embed_rows(G.st, G.emb, G.hist + pos0 + p0, NULL, nb, pdev(G.perm_emb), G.px + (size_t) p0 * G.E);
    }
    for (int L = 0; L < G.n_layer; L++) {
        if (L == G.nres && mid_on()) {
            middle(G.px, n, pos0);
            L += g_mid_layers - 1;
            continue;
        }
        stage_layer(L);
        for (int p0 = 0; p0 < n; p0 += chunk) {
            const int nb = n - p0 < chunk ? n - p0 : chunk;
            G.pos_cap = pos0 + p0 + nb;
            G.mx = G.px + (size_t) p0 * G.E;
            rows_layer(L, nb, G.iota + pos0 + p0, G.slotid + (size_t) slot * G.rrows, regime, 1, 0);
        }
    }
    G.mx = mx;
    G.pos_cap = G.n_ctx;
    hx.jb = outer;
    HX(hipMemcpyAsync(G.x, G.px + (size_t) (n - 1) * G.E, (size_t) G.E * 4, hipMemcpyDeviceToDevice, G.st));
}

static void prefill_rows(int slot, int pos0, int n) {
    if (slot != 0 && mid_on()) hx_failf("a middle stage serves slot 0 only");
    rows_alloc();
    // exact mode: the reference-order products and attention, in chunks of
    // xchunk positions
    const int regime = G.exact ? GEMM_REF : G.prompt_level >= 2 ? GEMM_PER256 : GEMM_EXACT;
    // level 1: 32 positions a chunk (the exact-regime GEMM's widest form),
    // 16 where MoE layers take part (the expert kernels' row limit)
    int moe = 0;
    for (int L = 0; L < G.n_layer; L++) moe |= G.L[L].moe != NULL;
    const int c1 = moe ? MAX_SLOTS : (G.rrows < 32 ? G.rrows : 32);
    const int chunk = G.exact ? G.xchunk : G.prompt_level >= 2 ? G.pb : c1;
    if (chunk < 1) hx_failf("exact prompt chunk of %d rows", chunk);
    if (G.nres < G.n_layer) {
        prefill_layers(slot, pos0, n, chunk, regime);
        return;
    }
    int last = 0;
    for (int p0 = 0; p0 < n; p0 += chunk) {
        const int nb = n - p0 < chunk ? n - p0 : chunk;
        G.pos_cap = pos0 + p0 + nb;
        G.cur_pos = pos0 + p0;
        launch_rows(nb, G.hist + pos0 + p0, G.iota + pos0 + p0, G.slotid + (size_t) slot * G.rrows, regime, 1, 0);
        last = nb - 1;
    }
    G.pos_cap = G.n_ctx;
    HX(hipMemcpyAsync(G.x, G.mx + (size_t) last * G.E, (size_t) G.E * 4, hipMemcpyDeviceToDevice, G.st));
}

const float * sml_gpu_prefill_slot(int slot, const int * ids, int pos0, int n) {
    if (slot == 0) return sml_gpu_prefill(ids, pos0, n);
    if (!G.open || slot < 0 || slot >= G.nslot || n <= 0 || pos0 < 0 || pos0 + n > G.n_ctx) return NULL;
    for (int i = 0; i < n; i++) if (ids[i] < 0 || ids[i] >= G.V) return NULL;
    HX_ENTRY(NULL);
    G.pin[1] = pos0 + n - 1;
    memcpy(G.pin + 2, ids, (size_t) n * 4);
    HX(hipMemcpyAsync(G.hist + pos0, G.pin + 2, (size_t) n * 4, hipMemcpyHostToDevice, G.st));
    if (G.prompt_level >= 1 && rows_check()) {
        prefill_rows(slot, pos0, n);
        HX(hipMemcpyAsync(G.pos, &G.pin[1], 4, hipMemcpyHostToDevice, G.st));
        run_tail();
    } else {
        // the captured graphs hold slot 0's cache: other slots launch directly
        G.pin[0] = pos0;
        HX(hipMemcpyAsync(G.pos, &G.pin[0], 4, hipMemcpyHostToDevice, G.st));
        G.cur_slot = slot;
        jmp_buf * outer = hx.jb;
        jmp_buf jb;
        if (setjmp(jb)) { G.cur_slot = 0; hx.jb = outer; longjmp(*outer, 1); }
        hx.jb = &jb;
        if (mid_on()) hx_failf("a middle stage serves slot 0 only");
        for (int i = 0; i < n; i++) {
            G.pos_cap = pos0 + i + 1;
            G.cur_pos = pos0 + i;
            launch_body();
            if (i + 1 < n) launch_adv();
        }
        G.pos_cap = G.n_ctx;
        launch_tail();
        hx.jb = outer;
        G.cur_slot = 0;
    }
    fetch_logits();
    HX_LEAVE();
    return G.lg_host;
}

static int g_multi_ns, g_multi_sb;

static void launch_multi_cur(void) {
    launch_rows(g_multi_ns, G.mtok, G.mpos, G.mslot, g_multi_sb ? GEMM_PER256 : GEMM_PER32, 0, 1);
}

// The batched step reads its tokens, positions and slots from device arrays,
// so one captured graph per (sequence count, regime, position bucket of the
// furthest sequence) serves every step: the ~300 launches of a step are
// replayed, not issued from the host. The regime and the environment
// switches are read when a graph is captured.
static void launch_multi(int ns, int maxpos) {
    g_multi_ns = ns;
    g_multi_sb = multi_per256(ns);
    const int k = bucket_of(maxpos);
    G.pos_cap = bucket_cap(k);
    if (G.use_graph) {
        hipGraphExec_t * g = &G.g_multi[ns][g_multi_sb][k];
        if (!*g) *g = capture(launch_multi_cur);
        HX(hipGraphLaunch(*g, G.st));
    } else {
        launch_multi_cur();
    }
    G.pos_cap = G.n_ctx;
}

int sml_gpu_step_multi(const int * tok, const int * pos, const int * slot, int ns, float * logits_out) {
    if (!G.open || ns < 1 || ns > G.nslot || !tok || !pos || !slot || !logits_out) return 0;
    for (int b = 0; b < ns; b++) {
        if (tok[b] < 0 || tok[b] >= G.V || pos[b] < 0 || pos[b] >= G.n_ctx || slot[b] < 0 || slot[b] >= G.nslot) return 0;
        for (int c = 0; c < b; c++) if (slot[c] == slot[b]) return 0;
    }
    HX_ENTRY(0);
    memcpy(G.mpin, tok, (size_t) ns * 4);
    memcpy(G.mpin + MAX_SLOTS, pos, (size_t) ns * 4);
    memcpy(G.mpin + 2 * MAX_SLOTS, slot, (size_t) ns * 4);
    HX(hipMemcpyAsync(G.mtok, G.mpin, (size_t) ns * 4, hipMemcpyHostToDevice, G.st));
    HX(hipMemcpyAsync(G.mpos, G.mpin + MAX_SLOTS, (size_t) ns * 4, hipMemcpyHostToDevice, G.st));
    HX(hipMemcpyAsync(G.mslot, G.mpin + 2 * MAX_SLOTS, (size_t) ns * 4, hipMemcpyHostToDevice, G.st));
    int maxpos = 0;
    for (int b = 0; b < ns; b++) if (pos[b] > maxpos) maxpos = pos[b];
    HX(hipEventRecord(G.e0, G.st));
    launch_multi(ns, maxpos);
    HX(hipEventRecord(G.e1, G.st));
    // the logits land in pinned memory at the link's rate, then every core
    // copies a share on to the caller's (pageable) buffer: a direct copy to
    // pageable memory stages it through one thread (16 x 128256 logits:
    // ~0.75 ms)
    const size_t nl = (size_t) ns * G.V;
    HX(hipMemcpyAsync(G.mlog_host, G.mlog, nl * 4, hipMemcpyDeviceToHost, G.st));
    HX(hipStreamSynchronize(G.st));
    HX(hipEventElapsedTime(&G.last_ms, G.e0, G.e1));
    const size_t chunk = 1u << 16;
    #pragma omp parallel for schedule(static)
    for (size_t o = 0; o < nl; o += chunk) memcpy(logits_out + o, G.mlog_host + o, (nl - o < chunk ? nl - o : chunk) * 4);
    HX_LEAVE();
    return ns;
}
