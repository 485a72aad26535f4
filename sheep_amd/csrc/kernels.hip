// gfx950 (MI355X) kernels for the quantized decode path. Compiled to a code
// object (--genco) and loaded by the C host with hipModuleLoadData; every
// kernel is extern "C" and takes one argument block from kargs.h.
//
// Wave64 throughout. The GEMV's unit of work is a 16-byte chunk of a row's
// nibble plane: chunk c holds columns 16*(c&1)..+15 of the group pair
// (c&~1, c|1) (the reference's flat-4 layout, sml/sml-kernel.c:2140-2156), so
// one lane loads one 128-bit word per plane, computes partial int8 dot
// products for both groups with v_dot4, swaps one of them with its pair lane
// through DPP, and ends up owning the full dot of group c. Group c's float
// epilogue follows the reference's per-group arithmetic
// (sml/sml-kernel.c:2054-2063): step*(s*dot) + min*(s*sum).
#include <hip/hip_runtime.h>
#include "kargs.h"

#define WAVE 64

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned int v4u __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float h2f(uint16_t h) { return (float) __builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16) f); }

// lane i <-> lane i^1 (DPP quad_perm [1,0,3,2])
__device__ __forceinline__ int pair_swap(int v) { return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false); }

__device__ __forceinline__ float wave_sum(float v) {
    #pragma unroll
    for (int o = 32; o; o >>= 1) v += __shfl_xor(v, o);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
    #pragma unroll
    for (int o = 32; o; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

__device__ __forceinline__ int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// 4 bits (one per column) -> 4 bytes of 0/1
__device__ __forceinline__ uint32_t bits4_to_bytes(uint32_t nib) { return (nib * 0x00204081u) & 0x01010101u; }

// ---------------------------------------------------------------- code chunks
//
// Codes of chunk c of one row, as int8 lanes: ca[i] holds 4 columns of group
// c&~1, cb[i] the same columns of group c|1 (columns 16*(c&1) + 4i .. +3).
// Every width below 8 yields codes <= 127, so one signed dot4 per word serves.
// Plane orders follow tooling/sml_quantize.py:104-106.
template <int NB>
struct Chunk {
    v4u a, b;          // low part (or the whole code)
    v4u ha, hb;        // Q8 only: high nibbles
};

template <int NB>
__device__ __forceinline__ Chunk<NB> load_chunk(const uint8_t * const * pl, size_t row, int cols, int c) {
    Chunk<NB> k;
    const int h = c & 1, ga = c & ~1;
    const size_t nib_row = (size_t) cols / 2, two_row = (size_t) cols / 4, bit_row = (size_t) cols / 8;
    // plane index of each part for this width
    constexpr int P4 = NB == 6 ? 1 : 0;                     // nibble plane
    constexpr int P2 = NB == 6 ? 0 : NB == 7 ? 1 : 0;       // 2-bit plane
    constexpr int P1 = NB == 7 ? 2 : 1;                     // 1-bit plane
    constexpr bool HAS4 = NB == 4 || NB == 5 || NB == 6 || NB == 7 || NB == 8;
    constexpr bool HAS2 = NB == 2 || NB == 3 || NB == 6 || NB == 7;
    constexpr bool HAS1 = NB == 3 || NB == 5 || NB == 7;
    v4u la = {0u, 0u, 0u, 0u}, lb = {0u, 0u, 0u, 0u};
    int sh = 0;
    if constexpr (HAS4) {
        const v4u w = *(const v4u *) (pl[P4] + row * nib_row + (size_t) c * 16);
        la = w & 0x0F0F0F0Fu;
        lb = (w >> 4u) & 0x0F0F0F0Fu;
        sh = 4;
    }
    if constexpr (HAS2) {
        // pack of 32 bytes per 128 weights; bit-plane k of byte j = group 4P+k, column j
        const v4u e = *(const v4u *) (pl[P2] + row * two_row + (size_t) (c >> 2) * 32 + h * 16);
        const unsigned ka = 2u * (unsigned) (ga & 3);
        const v4u ea = (e >> ka) & 0x03030303u, eb = (e >> (ka + 2u)) & 0x03030303u;
        if constexpr (HAS4) { la |= ea << 4u; lb |= eb << 4u; sh = 6; }
        else { la = ea; lb = eb; sh = 2; }
    }
    if constexpr (HAS1) {
        // 4 bytes per group, bit j = column j
        const uint2 wd = *(const uint2 *) (pl[P1] + row * bit_row + (size_t) ga * 4);
        const uint32_t wa = wd.x >> (16 * h), wb = wd.y >> (16 * h);
        #pragma unroll
        for (int i = 0; i < 4; i++) {
            la[i] |= bits4_to_bytes((wa >> (4 * i)) & 15u) << sh;
            lb[i] |= bits4_to_bytes((wb >> (4 * i)) & 15u) << sh;
        }
    }
    k.a = la; k.b = lb;
    if constexpr (NB == 8) {
        const v4u w = *(const v4u *) (pl[1] + row * nib_row + (size_t) c * 16);
        k.ha = w & 0x0F0F0F0Fu;
        k.hb = (w >> 4u) & 0x0F0F0F0Fu;
    }
    return k;
}

// partial dots of the chunk over its 16 columns against activation words xa, xb
template <int NB>
__device__ __forceinline__ void chunk_dots(const Chunk<NB> & k, const v4i xa, const v4i xb, int & da, int & db) {
    int a = 0, b = 0;
    #pragma unroll
    for (int i = 0; i < 4; i++) { a = dot4((int) k.a[i], xa[i], a); b = dot4((int) k.b[i], xb[i], b); }
    if constexpr (NB == 8) {
        int ha = 0, hb = 0;
        #pragma unroll
        for (int i = 0; i < 4; i++) { ha = dot4((int) k.ha[i], xa[i], ha); hb = dot4((int) k.hb[i], xb[i], hb); }
        a += ha << 4;
        b += hb << 4;
    }
    da = a; db = b;
}

// ---------------------------------------------------------------- GEMV
//
// One launch covers up to three matrices that read the same activation (the
// reference's shared-activation groups, sml/sml-run.c:924-1121). Each wave
// takes RB consecutive rows at a time and streams them with one lane per
// 16-byte chunk; the activation (int8 codes, per-group scale and sum) is
// staged once per workgroup in LDS.
#define GEMV_THREADS 256
#define GEMV_U 4

template <int NB, int NR>
__device__ __forceinline__ void gemv_rows(const sml_kmat * const mats[NR], const int rows_idx[NR], int cols,
                                          const int8_t * lq, const float * ls, const int32_t * lsum, float acc[NR]) {
    const int lane = threadIdx.x & (WAVE - 1);
    const int ng = cols / 32, ns = (ng + 7) / 8;
    #pragma unroll
    for (int r = 0; r < NR; r++) acc[r] = 0.0f;
    for (int c0 = 0; c0 < ng; c0 += WAVE * GEMV_U) {
        Chunk<NB> ch[GEMV_U][NR];
        uint32_t sqv[GEMV_U][NR], mqv[GEMV_U][NR];
        uint16_t sdv[GEMV_U][NR], mdv[GEMV_U][NR];
        #pragma unroll
        for (int u = 0; u < GEMV_U; u++) {
            const int c = c0 + u * WAVE + lane;
            if (c < ng) {
                #pragma unroll
                for (int r = 0; r < NR; r++) {
                    const sml_kmat * m = mats[r];
                    const size_t row = (size_t) rows_idx[r];
                    ch[u][r] = load_chunk<NB>(m->plane, row, cols, c);
                    sqv[u][r] = m->sq[row * ng + c];
                    sdv[u][r] = m->sd[row * ns + (c >> 3)];
                    if (m->mq) { mqv[u][r] = m->mq[row * ng + c]; mdv[u][r] = m->md[row * ns + (c >> 3)]; }
                    else { mqv[u][r] = 127u; mdv[u][r] = 0; }
                }
            }
        }
        #pragma unroll
        for (int u = 0; u < GEMV_U; u++) {
            const int c = c0 + u * WAVE + lane;
            if (c < ng) {
                const int off = 32 * (c & ~1) + 16 * (c & 1);
                const v4i xa = *(const v4i *) (lq + off);
                const v4i xb = *(const v4i *) (lq + off + 32);
                const float s = ls[c];
                const float sm = s * (float) lsum[c];
                #pragma unroll
                for (int r = 0; r < NR; r++) {
                    int da, db;
                    chunk_dots<NB>(ch[u][r], xa, xb, da, db);
                    const int odd = c & 1;
                    const int keep = odd ? db : da, send = odd ? da : db;
                    const int dot = keep + pair_swap(send);
                    const float wsc = h2f(sdv[u][r]) * (float) sqv[u][r];
                    const float wmn = h2f(mdv[u][r]) * ((float) mqv[u][r] - 127.0f);
                    acc[r] += wsc * (s * (float) dot);
                    acc[r] += wmn * sm;
                }
            }
        }
    }
    #pragma unroll
    for (int r = 0; r < NR; r++) acc[r] = wave_sum(acc[r]);
}

__device__ __forceinline__ void stage_act(const sml_kgemv & a, int8_t * lq, float * ls, int32_t * lsum) {
    const int n = a.cols, ng = n / 32;
    for (int i = threadIdx.x; i < n / 16; i += blockDim.x) ((v4i *) lq)[i] = ((const v4i *) a.q)[i];
    for (int i = threadIdx.x; i < ng; i += blockDim.x) { ls[i] = a.scale[i]; lsum[i] = a.sums[i]; }
    __syncthreads();
}

template <int NB, int RB>
__device__ void gemv_body(const sml_kgemv & a) {
    extern __shared__ __align__(16) uint8_t lds[];
    int8_t * lq = (int8_t *) lds;
    float * ls = (float *) (lds + a.cols);
    int32_t * lsum = (int32_t *) (lds + a.cols + 4 * (a.cols / 32));
    stage_act(a, lq, ls, lsum);
    const int lane = threadIdx.x & (WAVE - 1);
    const int gw = blockIdx.x * (GEMV_THREADS / WAVE) + (threadIdx.x >> 6);
    const int nw = gridDim.x * (GEMV_THREADS / WAVE);
    if (a.epi == SML_EPI_SWIGLU) {
        // gate row r and up row r together; h[r] = silu(g) * u (sml/sml-run.c:451-454)
        const int nrb = a.total_rows / RB;
        for (int rb = gw; rb < nrb; rb += nw) {
            const sml_kmat * mats[2 * RB];
            int ri[2 * RB];
            #pragma unroll
            for (int r = 0; r < RB; r++) {
                mats[2 * r] = &a.m[0]; mats[2 * r + 1] = &a.m[1];
                ri[2 * r] = ri[2 * r + 1] = rb * RB + r;
            }
            float acc[2 * RB];
            gemv_rows<NB, 2 * RB>(mats, ri, a.cols, lq, ls, lsum, acc);
            if (lane == 0) {
                #pragma unroll
                for (int r = 0; r < RB; r++) {
                    const int row = rb * RB + r;
                    float g = acc[2 * r], u = acc[2 * r + 1];
                    if (a.m[0].bias) g += a.m[0].bias[row];
                    if (a.m[1].bias) u += a.m[1].bias[row];
                    a.m[0].y[row] = (g / (1.0f + expf(-g))) * u;
                }
            }
        }
        return;
    }
    const int nrb = a.total_rows / RB;
    for (int rb = gw; rb < nrb; rb += nw) {
        const int row0 = rb * RB;
        int mi = 0;
        #pragma unroll
        for (int i = 1; i < SML_MAX_MATS; i++) if (i < a.nmat && row0 >= a.m[i].row_begin) mi = i;
        const sml_kmat * m = &a.m[mi];
        const int lrow = row0 - m->row_begin;
        const sml_kmat * mats[RB];
        int ri[RB];
        #pragma unroll
        for (int r = 0; r < RB; r++) { mats[r] = m; ri[r] = lrow + r; }
        float acc[RB];
        gemv_rows<NB, RB>(mats, ri, a.cols, lq, ls, lsum, acc);
        if (lane == 0) {
            #pragma unroll
            for (int r = 0; r < RB; r++) {
                float v = acc[r];
                if (m->bias) v += m->bias[lrow + r];
                if (a.epi == SML_EPI_RESIDUAL) v = a.resid[lrow + r] + v;
                m->y[lrow + r] = v;
            }
        }
    }
}

#define GEMV_KERNEL(NB, RB)                                                                   \
    extern "C" __global__ __launch_bounds__(GEMV_THREADS) void sml_gemv_q##NB##_r##RB(const sml_kgemv a) { \
        gemv_body<NB, RB>(a);                                                                \
    }
GEMV_KERNEL(2, 1) GEMV_KERNEL(2, 2)
GEMV_KERNEL(3, 1) GEMV_KERNEL(3, 2)
GEMV_KERNEL(4, 1) GEMV_KERNEL(4, 2) GEMV_KERNEL(4, 4)
GEMV_KERNEL(5, 1) GEMV_KERNEL(5, 2)
GEMV_KERNEL(6, 1) GEMV_KERNEL(6, 2)
GEMV_KERNEL(7, 1) GEMV_KERNEL(7, 2)
GEMV_KERNEL(8, 1) GEMV_KERNEL(8, 2)

// ---------------------------------------------------------------- norm + quantize
//
// Residual add, RMSNorm with a double sum of squares (sml/sml-run.c:147-152),
// gather through each consumer's permutation and the per-group int8
// quantization (sml/sml-kernel.c:86-106) -- with correctly rounded division
// and square root and round-half-even conversion, so the int8 codes, scales
// and sums equal the reference's bit for bit on the same input.
#define NORMQ_THREADS 1024

extern "C" __global__ __launch_bounds__(NORMQ_THREADS) void sml_normq(const sml_knormq a) {
    extern __shared__ __align__(16) float sx[];
    __shared__ double red[NORMQ_THREADS / WAVE];
    const int n = a.n, tid = threadIdx.x;
    double ss = 0.0;
    for (int i = tid; i < n; i += NORMQ_THREADS) {
        float v = a.x[i];
        if (a.resid) { v = v + a.resid[i]; a.x[i] = v; }
        sx[i] = v;
        ss += (double) v * (double) v;
    }
    if (a.norm_w) {
        #pragma unroll
        for (int o = 32; o; o >>= 1) ss += __shfl_xor(ss, o);
        if ((tid & 63) == 0) red[tid >> 6] = ss;
        __syncthreads();
        double tot = 0.0;
        for (int w = 0; w < NORMQ_THREADS / WAVE; w++) tot += red[w];
        // IEEE division and square root: hipcc's default for HIP is the correctly
        // rounded fp32 divide/sqrt, which the bit-exact parity tests rely on
        const float sc = 1.0f / sqrtf((float) (tot / (double) n) + a.eps);
        for (int i = tid; i < n; i += NORMQ_THREADS) sx[i] = sx[i] * sc * a.norm_w[i];
    }
    __syncthreads();
    if (a.normed) for (int i = tid; i < n; i += NORMQ_THREADS) a.normed[i] = sx[i];
    const int ng = n / 32;
    for (int o = 0; o < a.nout; o++) {
        const int32_t * perm = a.perm[o];
        for (int g = tid; g < ng; g += NORMQ_THREADS) {
            float v[32];
            #pragma unroll
            for (int j = 0; j < 32; j++) v[j] = sx[perm ? perm[g * 32 + j] : g * 32 + j];
            float amax = 0.0f;
            if (a.per256) {
                // sml/sml-kernel.c:165-172: one amax over the superblock
                const int g0 = g & ~7, g1 = g0 + 8 < ng ? g0 + 8 : ng;
                for (int i = g0 * 32; i < g1 * 32; i++) amax = fmaxf(amax, fabsf(sx[perm ? perm[i] : i]));
            } else {
                #pragma unroll
                for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(v[j]));
            }
            const float s = amax / 127.0f;
            const float is = s > 0.0f ? 1.0f / s : 0.0f;
            int sum = 0;
            int8_t * q = a.q[o] + g * 32;
            #pragma unroll
            for (int j = 0; j < 32; j += 4) {
                int w = 0;
                #pragma unroll
                for (int k = 0; k < 4; k++) {
                    int t = (int) __builtin_rintf(v[j + k] * is);
                    t = t > 127 ? 127 : t < -127 ? -127 : t;
                    sum += t;
                    w |= (t & 0xFF) << (8 * k);
                }
                *(int *) (q + j) = w;
            }
            a.scale[o][g] = s;
            a.sums[o][g] = sum;
        }
    }
}

// ---------------------------------------------------------------- unpack / embed

// The integer codes of group g of one row, from the planes (same reads as
// load_chunk, one group at a time).
__device__ void group_codes(const sml_kmat & m, int nb, int cols, size_t row, int g, uint8_t out[32]) {
    int pb[3], np = 0;
    // plane widths in storage order (tooling/sml_quantize.py:104-106)
    switch (nb) {
    case 2: pb[0] = 2; np = 1; break;
    case 3: pb[0] = 2; pb[1] = 1; np = 2; break;
    case 4: pb[0] = 4; np = 1; break;
    case 5: pb[0] = 4; pb[1] = 1; np = 2; break;
    case 6: pb[0] = 2; pb[1] = 4; np = 2; break;
    case 7: pb[0] = 4; pb[1] = 2; pb[2] = 1; np = 3; break;
    default: pb[0] = 4; pb[1] = 4; np = 2; break;
    }
    int shift[3], s = 0;
    if (nb == 6) { shift[0] = 4; shift[1] = 0; }
    else for (int i = 0; i < np; i++) { shift[i] = s; s += pb[i]; }
    for (int j = 0; j < 32; j++) out[j] = 0;
    for (int i = 0; i < np; i++) {
        const uint8_t * p = m.plane[i];
        if (pb[i] == 4) {
            const uint8_t * blk = p + row * (cols / 2) + (size_t) (g >> 2) * 64 + ((g & 2) ? 32 : 0);
            for (int j = 0; j < 32; j++) out[j] |= (uint8_t) ((((g & 1) ? blk[j] >> 4 : blk[j]) & 15) << shift[i]);
        } else if (pb[i] == 2) {
            const uint8_t * pk = p + row * (cols / 4) + (size_t) (g >> 2) * 32;
            for (int j = 0; j < 32; j++) out[j] |= (uint8_t) (((pk[j] >> (2 * (g & 3))) & 3) << shift[i]);
        } else {
            const uint8_t * wd = p + row * (cols / 8) + (size_t) g * 4;
            for (int j = 0; j < 32; j++) out[j] |= (uint8_t) (((wd[j >> 3] >> (j & 7)) & 1) << shift[i]);
        }
    }
}

extern "C" __global__ void sml_unpack(const sml_kunpack a) {
    const int ng = a.cols / 32;
    const long t = (long) blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (long) a.nrows * ng) return;
    const int r = (int) (t / ng), g = (int) (t % ng);
    uint8_t c[32];
    group_codes(a.m, a.nbits, a.cols, (size_t) (a.row0 + r), g, c);
    uint8_t * o = a.out + (size_t) r * a.cols + (size_t) g * 32;
    for (int j = 0; j < 32; j++) o[j] = c[j];
}

// sml/sml-run.c:3291-3344: one row of token_embd, code*step + min, scattered
// back through the permutation
extern "C" __global__ void sml_embed(const sml_kembed a) {
    const int ng = a.cols / 32, ns = (ng + 7) / 8;
    const int g = blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= ng) return;
    const size_t row = (size_t) (a.pos ? a.tok[*a.pos] : *a.tok);
    uint8_t c[32];
    group_codes(a.m, a.nbits, a.cols, row, g, c);
    const float step = h2f(a.m.sd[row * ns + g / 8]) * (float) a.m.sq[row * ng + g];
    const float mn = a.m.mq ? h2f(a.m.md[row * ns + g / 8]) * ((float) a.m.mq[row * ng + g] - 127.0f) : 0.0f;
    for (int j = 0; j < 32; j++) {
        const int col = g * 32 + j;
        a.x[a.perm ? a.perm[col] : col] = (float) c[j] * step + mn;
    }
}

// ---------------------------------------------------------------- attention
//
// RoPE (halved pairs, sml/sml-run.c:339-372) on q and k at position *pos, and
// the fp16 round-to-nearest-even KV write (sml/sml-run.c:68-77,3414-3415).
extern "C" __global__ void sml_rope_kv(const sml_kropekv a) {
    const int pos = *a.pos, half = a.half, hd = a.hd, kvd = a.n_kv * hd;
    const float * cs = a.cos_t + (size_t) pos * half, * sn = a.sin_t + (size_t) pos * half;
    for (int i = threadIdx.x; i < a.n_head * half; i += blockDim.x) {
        const int h = i / half, j = i % half;
        float * v = a.q + (size_t) h * hd;
        const float x0 = v[j], x1 = v[j + half];
        v[j] = x0 * cs[j] - x1 * sn[j];
        v[j + half] = x0 * sn[j] + x1 * cs[j];
    }
    uint16_t * kc = a.kcache + (size_t) pos * kvd, * vc = a.vcache + (size_t) pos * kvd;
    for (int i = threadIdx.x; i < a.n_kv * half; i += blockDim.x) {
        const int h = i / half, j = i % half;
        const float * v = a.k + (size_t) h * hd;
        const float x0 = v[j], x1 = v[j + half];
        kc[h * hd + j] = f2h(x0 * cs[j] - x1 * sn[j]);
        kc[h * hd + j + half] = f2h(x0 * sn[j] + x1 * cs[j]);
    }
    for (int i = threadIdx.x; i < kvd; i += blockDim.x) vc[i] = f2h(a.v[i]);
}

// Split-context decode attention (sml/sml-run.c:180-287 computes the same
// softmax-weighted sum per head in one pass). Workgroup (split, kv head)
// scores its chunk of positions for every query head sharing that KV head,
// keeps an unnormalised partial (max, sum, weighted V), and sml_attn_combine
// merges the partials. head_dim 128, chunk 64.
#define ATTN_THREADS 256
#define ATTN_CHUNK 64
#define ATTN_MAXREP 8

extern "C" __global__ __launch_bounds__(ATTN_THREADS) void sml_attn_part(const sml_kattn a) {
    __shared__ float qs[ATTN_MAXREP][128];
    __shared__ float sc[ATTN_MAXREP][ATTN_CHUNK];
    __shared__ float ov[ATTN_MAXREP][2][128];
    const int kh = blockIdx.y, split = blockIdx.x;
    const int rep = a.n_head / a.n_kv, hd = 128, kvd = a.n_kv * hd;
    const int T = *a.pos + 1, t0 = split * ATTN_CHUNK;
    const int tid = threadIdx.x;
    float * part0 = a.part + ((size_t) (kh * rep) * a.nsplit + split) * (hd + 2);
    if (t0 >= T) {
        // empty split: marks itself so the combine skips it
        for (int j = 0; j < rep; j++)
            if (tid == 0) part0[(size_t) j * a.nsplit * (hd + 2) + hd] = -INFINITY;
        return;
    }
    const int t1 = min(T, t0 + ATTN_CHUNK);
    for (int i = tid; i < rep * hd; i += ATTN_THREADS) qs[i / hd][i % hd] = a.q[(size_t) (kh * rep) * hd + i];
    __syncthreads();
    // scores: 16 lanes per position, 8 dims (16 bytes of K) per lane
    const int grp = tid >> 4, l16 = tid & 15;
    for (int t = t0 + grp; t < t0 + ATTN_CHUNK; t += ATTN_THREADS / 16) {
        float kf[8];
        const bool live = t < t1;
        if (live) {
            const v4i w = *(const v4i *) (a.kcache + (size_t) t * kvd + (size_t) kh * hd + l16 * 8);
            #pragma unroll
            for (int i = 0; i < 4; i++) {
                kf[2 * i] = h2f((uint16_t) (w[i] & 0xFFFF));
                kf[2 * i + 1] = h2f((uint16_t) ((uint32_t) w[i] >> 16));
            }
        } else {
            #pragma unroll
            for (int i = 0; i < 8; i++) kf[i] = 0.0f;
        }
        for (int j = 0; j < rep; j++) {
            float p = 0.0f;
            #pragma unroll
            for (int i = 0; i < 8; i++) p += qs[j][l16 * 8 + i] * kf[i];
            #pragma unroll
            for (int o = 8; o; o >>= 1) p += __shfl_xor(p, o);
            if (l16 == 0) sc[j][t - t0] = live ? p * a.inv : -INFINITY;
        }
    }
    __syncthreads();
    // per head: max and exp over the chunk (one wave per head, one lane per position)
    const int wave = tid >> 6, lane = tid & 63;
    __shared__ float mx_s[ATTN_MAXREP], l_s[ATTN_MAXREP];
    for (int j = wave; j < rep; j += ATTN_THREADS / WAVE) {
        const float s = sc[j][lane];
        const float m = wave_max(s);
        const float p = s == -INFINITY ? 0.0f : expf(s - m);
        const float l = wave_sum(p);
        sc[j][lane] = p;
        if (lane == 0) { mx_s[j] = m; l_s[j] = l; }
    }
    __syncthreads();
    // weighted V: thread (half, d) over positions of its parity
    const int d = tid & 127, hf = tid >> 7;
    float acc[ATTN_MAXREP];
    #pragma unroll
    for (int j = 0; j < ATTN_MAXREP; j++) acc[j] = 0.0f;
    for (int t = t0 + hf; t < t1; t += 2) {
        const float v = h2f(a.vcache[(size_t) t * kvd + (size_t) kh * hd + d]);
        #pragma unroll
        for (int j = 0; j < ATTN_MAXREP; j++) if (j < rep) acc[j] += sc[j][t - t0] * v;
    }
    #pragma unroll
    for (int j = 0; j < ATTN_MAXREP; j++) if (j < rep) ov[j][hf][d] = acc[j];
    __syncthreads();
    if (hf == 0) {
        for (int j = 0; j < rep; j++) {
            float * part = part0 + (size_t) j * a.nsplit * (hd + 2);
            part[d] = ov[j][0][d] + ov[j][1][d];
            if (d == 0) { part[hd] = mx_s[j]; part[hd + 1] = l_s[j]; }
        }
    }
}

extern "C" __global__ void sml_attn_combine(const sml_kattn_comb a) {
    const int h = blockIdx.x, d = threadIdx.x, hd = a.hd;
    const int T = *a.pos + 1, ns = (T + a.chunk - 1) / a.chunk;
    const float * p = a.part + (size_t) h * a.nsplit * (hd + 2);
    float M = -INFINITY;
    for (int s = 0; s < ns; s++) M = fmaxf(M, p[(size_t) s * (hd + 2) + hd]);
    float l = 0.0f, o = 0.0f;
    for (int s = 0; s < ns; s++) {
        const float * ps = p + (size_t) s * (hd + 2);
        const float e = expf(ps[hd] - M);
        l += e * ps[hd + 1];
        o += e * ps[d];
    }
    a.out[(size_t) h * hd + d] = o / l;
}

// ---------------------------------------------------------------- argmax
// First maximum wins (sml/sml-run.c:3539-3544).
extern "C" __global__ __launch_bounds__(1024) void sml_argmax(const sml_kargmax a) {
    __shared__ float bv_s[16];
    __shared__ int bi_s[16];
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int i = threadIdx.x; i < a.n; i += 1024) {
        const float v = a.logits[i];
        if (v > bv) { bv = v; bi = i; }
    }
    #pragma unroll
    for (int o = 32; o; o >>= 1) {
        const float ov = __shfl_xor(bv, o);
        const int oi = __shfl_xor(bi, o);
        if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
    }
    if ((threadIdx.x & 63) == 0) { bv_s[threadIdx.x >> 6] = bv; bi_s[threadIdx.x >> 6] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 16; w++)
            if (bv_s[w] > bv_s[0] || (bv_s[w] == bv_s[0] && bi_s[w] < bi_s[0])) { bv_s[0] = bv_s[w]; bi_s[0] = bi_s[w]; }
        // a NaN first logit is never beaten in the reference's loop
        const float l0 = a.logits[0];
        const int tok = (bi_s[0] == 0x7fffffff || l0 != l0) ? 0 : bi_s[0];
        *a.tok = tok;
        if (a.pos) {
            const int p = *a.pos;
            if (a.hist && p + 1 < a.hist_n) a.hist[p + 1] = tok;
            *a.pos = p + 1;
        }
    }
}

extern "C" __global__ void sml_advance(const sml_kadvance a) {
    if (threadIdx.x == 0 && blockIdx.x == 0) *a.pos += 1;
}

// g = g/(1+exp(-g)) * u  (sml/sml-run.c:451-454)
extern "C" __global__ void sml_silu_mul(const sml_ksilu a) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < a.n) { const float g = a.g[i]; a.g[i] = (g / (1.0f + expf(-g))) * a.u[i]; }
}
