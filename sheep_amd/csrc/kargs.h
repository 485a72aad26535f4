// Kernel argument blocks, shared by the gfx950 kernels (kernels.hip, C++) and
// the C host (engine.c). Every kernel takes exactly one of these by value, so
// the host fills the same struct it hands to hipModuleLaunchKernel.
#pragma once
#include <stdint.h>

// One quantized FLAT matrix resident in HBM: the file's code planes in
// storage order, and its four field arrays interleaved pairwise at upload --
// per group (sq, mq) as two bytes, per superblock (sd, md) as two halves --
// so a lane reads its group's fields with two loads instead of four. 6-bit
// files are widened to bytes with the min bias moved to 127; a tensor with
// no min stores mq = 127, md = 0.
typedef struct {
    const uint8_t  * plane[3];
    const uint8_t  * sqmq;        // [rows][ngroups][2]
    const uint16_t * sdmd;        // [rows][nsuper][2]
    const float    * bias;        // added to the output row, or NULL
    float          * y;
    int rows;
    int pad_;
    // Q4: the small-M MFMA GEMM's copy of the codes and fields, one
    // SML_TILE_Q4-byte tile per (16-row block, superblock) holding what the
    // kernel's 64 lanes load for it in lane order (sml_tile_q4), or NULL
    const uint8_t  * tiled;
} sml_kmat;

#define SML_TILE_Q4 2368          // 2048 code bytes, 16 x 16 (sq, mq) bytes, 16 x 4 (sd, md) bytes

// Build the tiled copy of a Q4 matrix: one workgroup per tile.
typedef struct {
    const uint8_t  * plane;
    const uint8_t  * sqmq;
    const uint16_t * sdmd;
    uint8_t * out;
    int rows, cols;
} sml_ktile;

enum { SML_EPI_STORE = 0, SML_EPI_RESIDUAL = 1, SML_EPI_SWIGLU = 2 };

// One GEMV launch over one matrix m[0] (SwiGLU: gate m[0] and up m[1] of one
// shape, h written to m[0].y).
typedef struct {
    sml_kmat m[2];
    int cols;                     // input width
    int total_rows;               // output rows
    int epi;                      // SML_EPI_*
    const int8_t  * q;            // activation, canonical layout (reference sml_act)
    const float   * scale;
    const int32_t * sums;
    const float   * resid;        // SML_EPI_RESIDUAL: y = resid + W.x (resid may alias y)
    // Fused activation prologue (the _n kernels): every workgroup computes the
    // activation itself from the fp32 vector x -- RMSNorm with norm_w (NULL:
    // none), gather through perm (NULL: identity), per-32 int8 quantization --
    // instead of reading q/scale/sums.
    const float   * x;
    const float   * norm_w;
    const int32_t * perm;
    float           eps;
    // SwiGLU h quantization (the _h kernels): each workgroup owns 32
    // consecutive outputs h and also writes their per-32 quantization
    // (identity order) for the down projection.
    int8_t        * hq;
    float         * hscale;
    int32_t       * hsums;
    // the greedy pick's first stage (one-matrix GEMVs, not the exact
    // form): when not NULL, each row block also writes the (max, lowest
    // index) pair of its rows' outputs to amax[block], as sml_argmax_part
    // would for those rows.
    int2          * amax;
    // the timeline kernel (sml_gemv_q4_r2_i4_ts): per row block, the real-time
    // clock (100 MHz) at entry, at the first weight word's arrival, when the
    // first pass's and the last pass's weights have all arrived, and at exit
    unsigned long long * ts;
} sml_kgemv;

// Multi-workgroup RMSNorm + gather + quantize: every workgroup reduces the
// whole vector's sum of squares itself (in double) and quantizes its own 8
// groups (one superblock) of each output.
typedef struct {
    const float   * x;
    const float   * norm_w;       // NULL: no norm
    float           eps;
    int             n;
    int             nout;
    const int32_t * perm[3];
    int8_t        * q[3];
    float         * scale[3];
    int32_t       * sums[3];
    int             per256;       // 1: one scale per 256 values (sml_quantize_act_sb)
    int             exact;        // 1: the sum of squares as the reference's serial chain of double FMAs
} sml_knormq2;

// Gather + optional residual add + optional RMSNorm + per-group int8 quantize.

typedef struct {
    float         * x;            // n floats; updated in place when resid != NULL
    const float   * resid;        // x += resid first, or NULL
    const float   * norm_w;       // RMSNorm weight, or NULL for none
    float           eps;
    int             n;
    int             nout;         // activations to produce (distinct permutations)
    const int32_t * perm[3];      // column permutation per output, NULL = identity
    int8_t        * q[3];
    float         * scale[3];
    int32_t       * sums[3];
    float         * normed;       // optional copy of the normalised vector (pre-gather), or NULL
    int             per256;       // 1: one scale per 256 values (reference prompt regime)
    int             exact;        // 1: the sum of squares as the reference's serial chain of double FMAs
} sml_knormq;

// Integer codes of rows [row0, row0+nrows) of one matrix, one byte per weight.
typedef struct {
    sml_kmat m;
    int nbits, cols, row0, nrows;
    uint8_t * out;
} sml_kunpack;

// Embedding: dequantized row of the token held in device memory, scattered
// back through the permutation.
typedef struct {
    sml_kmat m;
    int nbits, cols;
    const int32_t * tok;          // token ids; row = tok[*pos] when pos != NULL, else *tok
    const int32_t * pos;
    const int32_t * perm;         // NULL = identity
    float * x;
} sml_kembed;


// Decode attention: RoPE of q and k at *pos, the fp16 KV write and the
// split-context scores / softmax / V sums per (split, kv head) workgroup
// (sml_attn), then the merge of the splits per head (sml_attn_merge), which
// can also quantize the output per 32 (identity permutation) for the next GEMV.
typedef struct {
    const float * q;              // n_head * hd, after bias, not rotated
    const float * k, * v;         // n_kv * hd, after bias
    uint16_t * kcache, * vcache;  // layer base, [pos][n_kv * hd] fp16
    const float * cos_t, * sin_t; // [n_ctx][hd/2]
    const int32_t * pos;
    float * part;                 // [n_head][nsplit][hd + 2]
    float * out;                  // n_head * hd
    int8_t * q_out;               // quantized out (or NULL)
    float * s_out;
    int32_t * u_out;
    int n_head, n_kv, nsplit;
    float inv;
    // A batch of sequences (grid z): sequence b reads q, k, v at + b * qkv_stride
    // and position pos[b], uses the cache of its slot (kc_slots[slot[b]] +
    // layer_off when kc_slots is not NULL, else kcache/vcache), and writes part,
    // out and the quantized out at + b times their per-sequence size.
    int qkv_stride;
    uint16_t * const * kc_slots;
    uint16_t * const * vc_slots;
    const int32_t * slot;
    size_t layer_off;
    // 1: sml_ropekv already rotated and wrote every sequence's k and v (several
    // positions of one sequence in one launch attend to each other), so the
    // attention kernel writes nothing
    int kv_written;
    // entries per workgroup (grid z = nseq / tpw, rounded up): above 1 the
    // entries are consecutive positions of one sequence (one slot, positions
    // increasing) and share each split's K/V tile
    int tpw, nseq;
    // one-entry launches (tpw 1): when not NULL, counters [nseq][n_kv], zero
    // between launches. Each workgroup writes its partials coherently at
    // device scope and counts itself in; the last of a kv head's splits
    // merges that head's query heads as sml_attn_merge does and resets the
    // counter, so no merge launch follows. One launch at a time per array.
    int * cnt;
    // sml_attnf (prompt flash form): KV positions per split (grid z), a
    // multiple of 64
    int fchunk;
    // query-head subsets per kv head (the 8-wave kernels; 0 or 1: none):
    // grid y = n_kv * nsub, workgroup y takes kv head y / nsub and its query
    // heads (y % nsub) * REP .. +REP-1 (REP = n_head / n_kv / nsub)
    int nsub;
} sml_kattn;

// Decode attention in the reference's float order (exact mode), two
// launches: RoPE, the fp16 KV write and every position's score
// (sml_attnx_scores: splits of 128 positions x kv heads), then per query head
// the softmax and P.V chains (sml_attnx_pv).
typedef struct {
    const float * q;              // n_head * hd after bias (rotated in registers)
    const float * k;              // n_kv * hd after bias
    const float * v;              // n_kv * hd after bias
    uint16_t * kc, * vc;          // this layer's cache, [n_ctx][n_kv * hd]
    const float * cos_t, * sin_t; // [n_ctx][hd / 2]
    const int32_t * pos;
    float * sc;                   // scores [n_head][n_ctx] between the launches
    float * out;                  // n_head * hd
    int8_t * q_out;               // when non-NULL: out also quantized per 32
    float * s_out;                //   (sml_quantize_act) for the o product
    int32_t * u_out;
    int n_head, n_kv, n_ctx;
    float inv;                    // 1 / sqrtf(hd)
    // rows (grid z of the scores, grid y of P.V): row b is position pos[b],
    // its q/k/v at b * qkv_stride floats, its scores at b * n_head * n_ctx,
    // its output at b * n_head * hd; kv_written: every row's k and v are
    // in the cache already (exact batched prompts; the kernels write none)
    int qkv_stride;
    int kv_written;
} sml_kattnx;


// The softmax sum of the exact attention on its own: n values, one output.
typedef struct {
    const float * x;
    float * out;
    int n;
} sml_ksum;

typedef struct {
    const float * logits;
    int n;
    int32_t * tok;                // argmax written here
    int32_t * pos;                // when non-NULL: hist[*pos + 1] = argmax (if inside), then *pos += 1
    int32_t * hist;
    int hist_n;
    // two-stage pick: sml_argmax_part writes one (max, index) pair per
    // workgroup into part; sml_argmax then reduces nparts pairs (part NULL:
    // sml_argmax scans the logits itself)
    int2 * part;
    int nparts;
} sml_kargmax;

typedef struct {
    int32_t * pos;                // *pos += 1
} sml_kadvance;

typedef struct {
    float * g;                    // g = silu(g) * u
    const float * u;
    int n;
} sml_ksilu;

// Plain streaming read of `bytes` (multiple of 16) for bandwidth calibration:
// every 16-byte word is read once and folded into one word per wave.
typedef struct {
    const uint8_t * src;
    uint64_t bytes;
    uint32_t * sink;              // one word per wave
    int pattern;                  // 0: coalesced grid-stride; 1: each lane 64 contiguous bytes per step
} sml_kread;

// Plain device copy of `bytes` (multiple of 16): the known-size reference
// against which HBM byte counters are scaled.
typedef struct {
    const uint8_t * src;
    uint8_t * dst;
    uint64_t bytes;
} sml_kcopy;

// GPTQ-style 4-bit matrix (rows = outputs, cols = inputs, groups of 128
// inputs, identity g_idx): qweight [cols/8][rows] int32 with 8 codes along
// the input, lowest nibble first; qzeros [cols/128][rows/8] int32 with 8
// zero codes along the output; scales [cols/128][rows] fp16.
typedef struct {
    const uint32_t * qweight;
    const uint32_t * qzeros;
    const uint16_t * scales;
    const float    * x;           // fp32 input, cols
    float          * part;        // [nslice][rows] partial sums (8 groups each)
    float          * y;           // rows
    int rows, cols;
    int zero_add;                 // added to the stored zero: 1 for the v1 files, 0 for v2
    int nslice;                   // cols / 1024 rounded up
    // desc_act files: the input columns were reordered at upload so each
    // group's are contiguous; device input i is input perm[i] (NULL: identity)
    const int32_t * perm;
    // when not NULL, one counter per output block (grid x), zero between
    // launches: each workgroup stores its partials at device scope and counts
    // itself in, and the block's last one adds the slices into y in slice
    // order, as sml_gptq_reduce does, then clears the counter. One launch at
    // a time per matrix (the partials are the matrix's too).
    int * cnt;
} sml_kgptq;

typedef struct {
    const uint32_t * qweight;
    const uint32_t * qzeros;
    int rows, cols, zero_add;
    int row0, nrows;
    uint8_t * codes;              // [nrows][cols]
    uint8_t * zeros;              // [nrows][cols/128], stored zero + zero_add
} sml_kgptq_unpack;

// ------------------------------------------------------------ MoE and small-M GEMM

// Router, top-k routing and the per-expert token lists for T tokens (one
// workgroup).
typedef struct {
    const float   * x;            // [T][n] normed inputs of the expert FFN
    const float   * router;       // [nexp][n]
    const float   * router_b;     // [nexp] or NULL
    int T, n, nexp, k, mmax;
    unsigned moe_flags;
    float   * logits;             // [T][nexp]
    int32_t * sel;                // [T][k] chosen experts, in choice order
    float   * w;                  // [T][k] their weights
    int32_t * slot;               // [T][k] position of (t, j) in its expert's list
    int32_t * count;              // [nexp] tokens per expert
    int32_t * list;               // [nexp][mmax] entries t*k + j, by token then choice
    int exact;                    // 1: each router dot as the reference's serial chain of double FMAs
    // routing modes of sml_moe_route (sml/sml-run.c:2925-3037): flags bit 1
    // sigmoid scores, bit 2 sparsemixer (scale: its jitter), bit 3 groups
    // scored by their best expert; exp_bias [nexp] (NULL: none) shifts the
    // choice; groups / topk_group keep the best groups' experts; scale (0:
    // none) multiplies the weights
    const float * exp_bias;
    float scale;
    int groups, topk_group;
    // shared expert gate (NULL: none): sg[t] = sigmoid(shgate . x[t]), its
    // dot summed as the router's
    const float * shgate;
    float * sg;                   // [T] (1 when there is a shared expert without a gate)
} sml_kmoe_route;

// Per-32 (or per-256) int8 quantization of activation rows into per-expert slots:
// mode 0 gathers row list[e][r] / k of x [T][n]; mode 1 takes row (e, r) of
// src [nexp][mmax][n]. perms: device table of nexp permutations (NULL entries
// or a NULL table: identity).
typedef struct {
    const float   * src;
    int mode;
    const int32_t * const * perms;
    int n, mmax, k;
    const int32_t * count;
    const int32_t * list;
    int8_t * q;                   // [nexp][mmax][n]
    float * scale;                // [nexp][mmax][n/32]
    int32_t * sums;
    int per256;                   // 1: one scale per 256 values (sml_quantize_act_sb)
} sml_kmquant;

// Small-M GEMM over groups of matrices (one per expert, or a single one):
// for group e and its count[e] (or m_all) activation rows, y[e][r] = W_e.a[e][r]
// (SwiGLU: silu(gate.a) * (up.a)). Each group's weights stream once for all
// its rows.
typedef struct {
    const sml_kmat * mats;        // device table: group e's matrices at [e * nmat + i]
    int nmat;                     // 1, or 2 for SwiGLU (gate, up)
    int cols, rows;               // per matrix
    const int32_t * count;        // [ngroups] or NULL
    int m_all;
    int mmax;                     // activation / output slots per group
    const int8_t  * q;            // [ngroups][mmax][cols]
    const float   * scale;        // [ngroups][mmax][cols/32]
    const int32_t * sums;
    float * y;                    // [ngroups][mmax][rows]
    const float * bias;           // [rows] added to each row (plain GEMM only), or NULL
    const float * resid;          // [ngroups][mmax][rows]: y = resid + (W.a + bias), may alias y; or NULL
    int mlo;                      // VALU kernel: groups of mlo rows or fewer are another launch's
    float * part;                 // split-K MFMA kernels: [ks][m_all][rows] partial products
    // one group (count NULL): its matrices' descriptors by value (inl = 1), so
    // the MFMA kernels address the weights from the kernel arguments instead
    // of first reading mats[] from device memory
    int inl;
    sml_kmat m0[2];
} sml_kgemm;

// Split-K sums: y[r][c] = resid[r][c] + (((part[0][r][c] + part[1][r][c]) + ...) + bias[c])
typedef struct {
    const float * part;           // [ks][m][rows]
    const float * bias;           // [rows] or NULL
    const float * resid;          // [m][rows] or NULL (may alias y)
    float * y;                    // [m][rows]
    int ks, m, rows;
} sml_kksum;

// Split-K sums and the next normq of each row in one launch (s.rows == q.n;
// q.x is unused: the rows come from the sums)
typedef struct {
    sml_kksum s;
    sml_knormq2 q;
} sml_kksumq;

// out[t] = sum over j of w[t][j] * y[sel[t][j]][slot[t][j]], in choice order,
// then + sg[t] * ysh[t] (the shared expert) when ysh is not NULL.
typedef struct {
    const float   * y;            // [nexp][mmax][n]
    const int32_t * sel, * slot;
    const float   * w;
    int T, n, k, mmax;
    const float * resid;          // [T][n] added first (may alias out), or NULL
    float * out;                  // [T][n]
    const float * ysh;            // [T][n] or NULL
    const float * sg;             // [T]
} sml_kmoe_comb;

// ---------------------------------------------------------------- ingest
// Re-quantization of a dequantized GPTQ/AWQ tensor (or any float tensor) into
// SSF FLAT codes and two-level fields, on the GPU (ingest.hip).

// GPTQ (bits 2/4/8) or AWQ (4 bits) integers to fp16-rounded floats
// out [rows][cols], rows = outputs.
typedef struct {
    const uint32_t * qweight;
    const uint32_t * qzeros;      // NULL (AWQ only): zero 2^(bits-1)
    const uint16_t * scales;      // [groups][rows] fp16
    const int32_t  * g_idx;       // [cols] or NULL: input k's group is k / group
    float * out;
    int rows, cols, bits, group, zero_add, awq;
} sml_king_dequant;

// GGUF Q8_0 / Q4_0 / Q6_K blocks (ggml type 8 / 2 / 14; row-major, blocks
// along each row) to the float16 copy in fp32: out [rows][cols]
typedef struct { const uint8_t * blocks; float * out; int rows, cols, type; } sml_king_gguf;

// part[y][c] = max over rows [y*chunk, (y+1)*chunk) of |w[r][c]| (NaN wins);
// then key[c] = the max over y of part[y][c]
typedef struct { const float * w; float * part; int rows, cols, chunk; } sml_king_colmax;
typedef struct { const float * part; float * key; int cols, nchunk; } sml_king_colfold;

// cnt[c] += the keys before key[c] among columns [y*slice, (y+1)*slice)
// (ascending key, NaN last, ties by column); then perm[cnt[c]] = c
typedef struct { const float * key; int32_t * cnt; int32_t * perm; int cols, slice; } sml_king_rank;

// wp[r][i] = w[r][perm[i]]
typedef struct { const float * w; const int32_t * perm; float * wp; int rows, cols; } sml_king_gather;

// Per-group (min, step) of the asymmetric grid (one lane per group).
typedef struct {
    const float * wp;             // [rows][cols], columns already permuted
    const float * wt;             // [cols] normalised weights, or NULL for ones
    const float * facs;           // [ncand] range factors
    float * out_l, * out_s;       // [rows][cols/group]
    int rows, cols, group, nbits, rem, ncand, iters, refit;
} sml_king_grid;

// Two-level fields of a [rows][ng] float array, 8-bit: fp16 per superblock of
// gps groups, uint8 per group; is_signed: biased by 127 (mins).
typedef struct {
    const float * v;
    uint16_t * d16;               // [rows][nsb]
    uint8_t * q8;                 // [rows][ng]
    float * eff;                  // [rows][ng], or NULL
    int rows, ng, gps, is_signed;
} sml_king_two;

// The field search: each group's step field q8 and min field mq8 moved to the
// best neighbour within +-radius. Scales per group (dv/dm [rows][ng]) or per
// superblock (d16/md16 fp16 [rows][nsb] with gps groups each).
typedef struct {
    const float * w;              // [rows][cols] (permuted)
    const float * dv, * dm;       // per group, or NULL
    const uint16_t * d16, * md16; // per superblock (when dv is NULL)
    int gps;
    int32_t * q8, * mq8;          // in/out (int32), or NULL
    uint8_t * sq, * mq;           // in/out (uint8, when q8 is NULL)
    float * eff_s, * eff_m;       // out: q8*dv and (mq8 - moff)*dm, or NULL
    const float * wt;             // [cols] or NULL
    int rows, cols, group, nmax, hi, moff, mmax, radius;
} sml_king_field;

// Codes clip(rint((w - M) / max(S, 1e-12)), 0, nmax) of every weight, packed
// into the FLAT planes of width nbits (one thread per 128 weights of a row).
typedef struct {
    const float * wp;             // [rows][cols] (permuted)
    const float * eff_s, * eff_m; // [rows][cols/32]
    uint8_t * plane[3];           // the width's planes, row-major
    uint8_t * codes;              // [rows][cols] codes too, or NULL
    int rows, cols, nbits;
} sml_king_pack;
