// Re-quantization of a dequantized GPTQ/AWQ tensor (or any float tensor)
// into SSF FLAT codes and two-level fields, on gfx950: the reference
// quantizer's path for a tensor without calibration feedback
// (tooling/sml_quantize.py:426-581), with its two searches in the arithmetic
// of its fused C library (sml/sml-quant.c).
//
// Built with -ffp-contract=off: every multiply and add rounds on its own
// unless written as __builtin_fmaf, and the fused ones are exactly those the
// reference's gcc -O3 build contracts (for groups of 32: d = fma(qv, step, l)
// - g in the grid, the refit's min, the field search's scalar loop). Division
// is IEEE (correctly rounded), rintf rounds to nearest even; so each lane
// computes its group bit for bit as that library does.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kargs.h"

__device__ __forceinline__ float h2f(uint16_t h) { return (float) __builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16) f); }

// ---------------------------------------------------------------- unpack + dequantize
// out[n][k] = fp16((code - zero) * scale) for output n, input k, as the
// unpacker writes the float16 copy the quantizer then reads
// (tooling/sml_unpack.py:66-118, :35-38). A thread per weight, input fastest.
extern "C" __global__ __launch_bounds__(256) void sml_ing_dequant(const sml_king_dequant a) {
    const int64_t i = (int64_t) blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t) a.rows * a.cols) return;
    const int n = (int) (i / a.cols), k = (int) (i % a.cols);
    uint32_t q, z;
    int g;
    if (a.awq) {
        // 8 outputs per word in nibble order 0, 4, 1, 5, 2, 6, 3, 7
        const int sh = 4 * (((n & 7) >> 1) + 4 * (n & 1));
        g = k / a.group;
        q = (a.qweight[(size_t) k * (a.rows / 8) + n / 8] >> sh) & 15u;
        z = a.qzeros ? (a.qzeros[(size_t) g * (a.rows / 8) + n / 8] >> sh) & 15u : 8u;
    } else {
        const int per = 32 / a.bits;
        const uint32_t mask = (1u << a.bits) - 1u;
        g = a.g_idx ? a.g_idx[k] : k / a.group;
        q = (a.qweight[(size_t) (k / per) * a.rows + n] >> (a.bits * (k % per))) & mask;
        z = ((a.qzeros[(size_t) g * (a.rows / per) + n / per] >> (a.bits * (n % per))) & mask) + (uint32_t) a.zero_add;
    }
    const float v = (float) ((int) q - (int) z) * h2f(a.scales[(size_t) g * a.rows + n]);
    a.out[i] = h2f(f2h(v));
}

// GGUF Q8_0, Q4_0 and Q6_K (ggml's published block layouts and
// dequantize_row_* formulas, in their float order: no contraction in this
// file): one thread per weight; the value rounded to fp16 as the float16
// copy transformers writes.
extern "C" __global__ __launch_bounds__(256) void sml_ing_gguf(const sml_king_gguf a) {
    const int64_t i = (int64_t) blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t) a.rows * a.cols) return;
    const int r = (int) (i / a.cols), k = (int) (i % a.cols);
    float v;
    if (a.type == 8) {
        const uint8_t * blk = a.blocks + ((size_t) r * (a.cols / 32) + k / 32) * 34;
        const float d = h2f((uint16_t) (blk[0] | (blk[1] << 8)));
        v = d * (float) (int8_t) blk[2 + k % 32];
    } else if (a.type == 2) {
        const uint8_t * blk = a.blocks + ((size_t) r * (a.cols / 32) + k / 32) * 18;
        const float d = h2f((uint16_t) (blk[0] | (blk[1] << 8)));
        const int j = k % 32, b = blk[2 + (j & 15)];
        v = d * (float) ((j < 16 ? b & 15 : b >> 4) - 8);
    } else {
        const uint8_t * blk = a.blocks + ((size_t) r * (a.cols / 256) + k / 256) * 210;
        const int w = k % 256, h = w / 128, l = w % 32, kk = (w % 128) / 32;   // weight l + 32 kk of half h
        const uint8_t ql = blk[64 * h + l + 32 * (kk & 1)], qh = blk[128 + 32 * h + l];
        const int q = (((ql >> (4 * (kk >> 1))) & 15) | (((qh >> (2 * kk)) & 3) << 4)) - 32;
        const float d = h2f((uint16_t) (blk[208] | (blk[209] << 8)));
        const float sc = (float) (int8_t) blk[192 + w / 16];
        v = d * sc * (float) q;
    }
    a.out[i] = h2f(f2h(v));
}

// ---------------------------------------------------------------- column order
// numpy's max over a column: NaN wins, otherwise the largest
__device__ __forceinline__ float np_max(float m, float x, bool first) {
    if (first) return x;
    if (isnan(m)) return m;
    if (isnan(x)) return x;
    return x > m ? x : m;
}

// Column maxima in two passes: workgroups over (256 columns, a chunk of rows)
// write partial maxima, then one thread per column folds them (max with NaN
// winning does not depend on the order).
extern "C" __global__ __launch_bounds__(256) void sml_ing_colmax(const sml_king_colmax a) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c >= a.cols) return;
    const int r0 = blockIdx.y * a.chunk, r1 = min(a.rows, r0 + a.chunk);
    float m = 0.0f;
    for (int r = r0; r < r1; r++) m = np_max(m, fabsf(a.w[(size_t) r * a.cols + c]), r == r0);
    a.part[(size_t) blockIdx.y * a.cols + c] = m;
}

extern "C" __global__ __launch_bounds__(256) void sml_ing_colfold(const sml_king_colfold a) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c >= a.cols) return;
    float m = 0.0f;
    for (int y = 0; y < a.nchunk; y++) m = np_max(m, a.part[(size_t) y * a.cols + c], y == 0);
    a.key[c] = m;
}

// A stable argsort by counting: the rank of key[c] is the number of columns
// before it in (NaN, key, column) order, counted over column slices by
// workgroups (blockIdx.y) through LDS and added with integer atomics (the
// total does not depend on their order); then perm[rank] = c.
extern "C" __global__ __launch_bounds__(256) void sml_ing_rank(const sml_king_rank a) {
    __shared__ float tile[1024];
    const int c = blockIdx.x * 256 + threadIdx.x;
    const float kc = c < a.cols ? a.key[c] : 0.0f;
    const bool nc = isnan(kc);
    const int j0 = blockIdx.y * a.slice, j1 = min(a.cols, j0 + a.slice);
    int rank = 0;
    for (int t0 = j0; t0 < j1; t0 += 1024) {
        __syncthreads();
        for (int j = threadIdx.x; j < 1024; j += 256) tile[j] = t0 + j < j1 ? a.key[t0 + j] : 0.0f;
        __syncthreads();
        const int tn = j1 - t0 < 1024 ? j1 - t0 : 1024;
        for (int j = 0; j < tn; j++) {
            const float kj = tile[j];
            const bool nj = isnan(kj);
            // NaN keys after every number
            const bool before = nc ? (!nj || t0 + j < c) : (!nj && (kj < kc || (kj == kc && t0 + j < c)));
            rank += before;
        }
    }
    if (c < a.cols && rank) atomicAdd(a.cnt + c, rank);
}

extern "C" __global__ __launch_bounds__(256) void sml_ing_scatter(const sml_king_rank a) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c < a.cols) a.perm[a.cnt[c]] = c;
}

extern "C" __global__ __launch_bounds__(256) void sml_ing_gather(const sml_king_gather a) {
    const int64_t i = (int64_t) blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t) a.rows * a.cols) return;
    const int64_t r = i / a.cols;
    a.wp[i] = a.w[r * a.cols + a.perm[i % a.cols]];
}

// ---------------------------------------------------------------- the asymmetric grid
// Weighted error of one candidate (l, step) over the group, and (STORE) its
// codes into q. follows sml/sml-quant.c:20-33 as the grid's vectorized loop
// computes it: d = fma(qv, step, l) - g, then e = e + (d*d)*w in order. WT
// false: every weight is 1 (the product by 1 is exact, so it is left out).
template <int G, bool WT, bool STORE>
__device__ __forceinline__ float err32(const float (&g)[G], const float * w, float l, float step, float n, int rem,
                                       float (&q)[G]) {
    float e = 0.0f;
    #pragma unroll
    for (int i = 0; i < G; i++) {
        float c = __builtin_rintf((g[i] - l) / step);
        if (c < 0.0f) c = 0.0f;
        if (c > n) c = n;
        if constexpr (STORE) q[i] = c;
        const float qv = rem ? (float) ((((int) c >> rem) << rem) + (1 << (rem - 1))) : c;
        const float d = __builtin_fmaf(qv, step, l) - g[i];
        e = WT ? e + (d * d) * w[i] : e + d * d;
    }
    return e;
}

// One lane per group of 32, the weights and the current codes in registers.
// A refit's candidate codes are not kept: when it wins they are derived again
// from its (min, step) -- the same function, so the same codes -- which
// keeps the lane under 128 registers.
// follows sml/sml-quant.c:38-95 (sml_asym_grid)
template <bool WT>
__device__ __forceinline__ void grid32_body(const sml_king_grid & a) {
    constexpr int G = 32;
    const int ng = a.cols / G;
    const int64_t t = (int64_t) blockIdx.x * 256 + threadIdx.x;
    if (t >= (int64_t) a.rows * ng) return;
    const int j = (int) (t % ng);
    const float * gp = a.wp + (size_t) t * G;        // row r, group j: (r*ng + j)*32
    float g[G], q[G];
    float w[WT ? G : 1];
    #pragma unroll
    for (int i = 0; i < G; i += 4) {
        const float4 v = *(const float4 *) (gp + i);
        g[i] = v.x; g[i + 1] = v.y; g[i + 2] = v.z; g[i + 3] = v.w;
    }
    if constexpr (WT) {
        #pragma unroll
        for (int i = 0; i < G; i++) w[i] = a.wt[(size_t) j * G + i];
    }
    const float n = (float) ((1 << a.nbits) - 1);
    float lo = g[0], hi = g[0], ws = 0.0f;
    #pragma unroll
    for (int i = 0; i < G; i++) {
        if (g[i] < lo) lo = g[i];
        if (g[i] > hi) hi = g[i];
        ws = ws + (WT ? w[i] : 1.0f);
    }
    const float c = (lo + hi) * 0.5f;
    float bl = 0.0f, bs = 0.0f, be = 0.0f;
    for (int k = 0; k < a.ncand; k++) {
        const float half = (hi - lo) * 0.5f * a.facs[k];
        float l = c - half;
        float step = fmaxf(2.0f * half, 1e-12f) / n;
        float e = err32<G, WT, true>(g, w, l, step, n, a.rem, q);
        if (a.refit) {
            for (int it = 0; it < a.iters; it++) {
                float qm = 0.0f, gm = 0.0f;
                #pragma unroll
                for (int i = 0; i < G; i++) {
                    qm = qm + (WT ? w[i] * q[i] : q[i]);
                    gm = gm + (WT ? w[i] * g[i] : g[i]);
                }
                qm = qm / ws;
                gm = gm / ws;
                float var = 0.0f, cov = 0.0f;
                #pragma unroll
                for (int i = 0; i < G; i++) {
                    const float dq = q[i] - qm;
                    const float wdq = WT ? w[i] * dq : dq;
                    var = var + wdq * dq;
                    cov = cov + wdq * (g[i] - gm);
                }
                float s2 = var > 1e-12f ? cov / fmaxf(var, 1e-12f) : step;
                s2 = fmaxf(s2, 1e-12f);
                const float l2 = __builtin_fmaf(-s2, qm, gm);
                const float e2 = err32<G, WT, false>(g, w, l2, s2, n, a.rem, q);
                if (e2 < e) {
                    l = l2; step = s2; e = e2;
                    err32<G, WT, true>(g, w, l, step, n, a.rem, q);
                }
            }
        }
        if (k == 0 || e < be) { bl = l; bs = step; be = e; }
    }
    a.out_l[t] = bl;
    a.out_s[t] = bs;
}

extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(6))) void sml_ing_grid32(const sml_king_grid a) { grid32_body<false>(a); }
extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void sml_ing_grid32w(const sml_king_grid a) { grid32_body<true>(a); }

// Any group that is a multiple of 8 up to 256 (gcc's 8-wide loop covers the
// whole group, so the order is the one above), read from memory; the codes
// of the current candidate are recomputed where the refit needs them (the
// same function of (l, step), so the same values).
__device__ __forceinline__ float errm(const float * g, const float * w, int G, float l, float step, float n, int rem) {
    float e = 0.0f;
    for (int i = 0; i < G; i++) {
        float c = __builtin_rintf((g[i] - l) / step);
        if (c < 0.0f) c = 0.0f;
        if (c > n) c = n;
        const float qv = rem ? (float) ((((int) c >> rem) << rem) + (1 << (rem - 1))) : c;
        const float d = __builtin_fmaf(qv, step, l) - g[i];
        e = e + (d * d) * (w ? w[i] : 1.0f);
    }
    return e;
}
__device__ __forceinline__ float codem(float g, float l, float step, float n) {
    float c = __builtin_rintf((g - l) / step);
    if (c < 0.0f) c = 0.0f;
    if (c > n) c = n;
    return c;
}

extern "C" __global__ __launch_bounds__(256) void sml_ing_grid(const sml_king_grid a) {
    const int G = a.group, ng = a.cols / G;
    const int64_t t = (int64_t) blockIdx.x * 256 + threadIdx.x;
    if (t >= (int64_t) a.rows * ng) return;
    const int j = (int) (t % ng);
    const float * g = a.wp + (size_t) t * G;
    const float * w = a.wt ? a.wt + (size_t) j * G : nullptr;
    const float n = (float) ((1 << a.nbits) - 1);
    float lo = g[0], hi = g[0], ws = 0.0f;
    for (int i = 0; i < G; i++) {
        if (g[i] < lo) lo = g[i];
        if (g[i] > hi) hi = g[i];
        ws = ws + (w ? w[i] : 1.0f);
    }
    const float c = (lo + hi) * 0.5f;
    float bl = 0.0f, bs = 0.0f, be = 0.0f;
    for (int k = 0; k < a.ncand; k++) {
        const float half = (hi - lo) * 0.5f * a.facs[k];
        float l = c - half;
        float step = fmaxf(2.0f * half, 1e-12f) / n;
        float e = errm(g, w, G, l, step, n, a.rem);
        if (a.refit) {
            for (int it = 0; it < a.iters; it++) {
                float qm = 0.0f, gm = 0.0f;
                for (int i = 0; i < G; i++) {
                    const float wi = w ? w[i] : 1.0f;
                    qm = qm + wi * codem(g[i], l, step, n);
                    gm = gm + wi * g[i];
                }
                qm = qm / ws;
                gm = gm / ws;
                float var = 0.0f, cov = 0.0f;
                for (int i = 0; i < G; i++) {
                    const float wi = w ? w[i] : 1.0f;
                    const float dq = codem(g[i], l, step, n) - qm;
                    var = var + (wi * dq) * dq;
                    cov = cov + (wi * dq) * (g[i] - gm);
                }
                float s2 = var > 1e-12f ? cov / fmaxf(var, 1e-12f) : step;
                s2 = fmaxf(s2, 1e-12f);
                const float l2 = __builtin_fmaf(-s2, qm, gm);
                const float e2 = errm(g, w, G, l2, s2, n, a.rem);
                if (e2 < e) { l = l2; step = s2; e = e2; }
            }
        }
        if (k == 0 || e < be) { bl = l; bs = step; be = e; }
    }
    a.out_l[t] = bl;
    a.out_s[t] = bs;
}

// ---------------------------------------------------------------- two-level fields
// One thread per superblock of a row. follows tooling/sml_quantize.py:320-363
// (two_level with 8-bit fields; a zero scale divides as 1e-8)
extern "C" __global__ __launch_bounds__(256) void sml_ing_two(const sml_king_two a) {
    const int nsb = (a.ng + a.gps - 1) / a.gps;
    const int64_t t = (int64_t) blockIdx.x * 256 + threadIdx.x;
    if (t >= (int64_t) a.rows * nsb) return;
    const int64_t r = t / nsb;
    const int s = (int) (t % nsb);
    const float * v = a.v + r * a.ng;
    float mx = 0.0f;
    for (int k = 0; k < a.gps; k++) {
        const int g = s * a.gps + k < a.ng ? s * a.gps + k : a.ng - 1;
        mx = np_max(mx, a.is_signed ? fabsf(v[g]) : v[g], k == 0);
    }
    const uint16_t h = f2h(mx / (a.is_signed ? 127.0f : 255.0f));
    a.d16[t] = h;
    float dv = h2f(h);
    if (dv == 0.0f) dv = 1e-8f;
    for (int k = 0; k < a.gps && s * a.gps + k < a.ng; k++) {
        const int g = s * a.gps + k;
        float x = __builtin_rintf(v[g] / dv);
        float e;
        uint8_t qv;
        if (a.is_signed) {
            x = x + 127.0f;
            x = x < 0.0f ? 0.0f : x > 254.0f ? 254.0f : x;
            qv = (uint8_t) x;
            e = ((float) qv - 127.0f) * dv;
        } else {
            x = x < 1.0f ? 1.0f : x > 255.0f ? 255.0f : x;
            qv = (uint8_t) x;
            e = (float) qv * dv;
        }
        a.q8[r * a.ng + g] = qv;
        if (a.eff) a.eff[r * a.ng + g] = e;
    }
}

// ---------------------------------------------------------------- the field search
// One lane per group. follows sml/sml-quant.c:101-137 (sml_field_search):
// dd = fma(c, S, M) - g, e = fma(dd*dd, w, e) in order.
template <int G>
__device__ __forceinline__ void field_body(const sml_king_field & a, int64_t t, int j, const float * gp) {
    float g[G > 0 ? G : 1];
    if constexpr (G > 0) {
        #pragma unroll
        for (int i = 0; i < G; i += 4) {
            const float4 v = *(const float4 *) (gp + i);
            g[i] = v.x; g[i + 1] = v.y; g[i + 2] = v.z; g[i + 3] = v.w;
        }
    }
    const int GG = G > 0 ? G : a.group;
    const int64_t r = t / (a.cols / GG);
    float d, m;
    if (a.dv) { d = a.dv[t]; m = a.dm[t]; }
    else {
        const int nsb = (a.cols / GG + a.gps - 1) / a.gps;
        d = h2f(a.d16[r * nsb + j / a.gps]);
        m = h2f(a.md16[r * nsb + j / a.gps]);
    }
    const float * wg = a.wt ? a.wt + (size_t) j * GG : nullptr;
    const int qs0 = a.q8 ? a.q8[t] : a.sq[t], qm0 = a.mq8 ? a.mq8[t] : a.mq[t];
    float be = 0.0f;
    int bs = qs0, bm = qm0;
    bool first = true;
    for (int da = -a.radius; da <= a.radius; da++) {
        int qs = qs0 + da;
        if (qs < 1) qs = 1;
        if (qs > a.hi) qs = a.hi;
        const float S = fmaxf((float) qs * d, 1e-12f);
        for (int db = -a.radius; db <= a.radius; db++) {
            int qm = qm0 + db;
            if (qm < 0) qm = 0;
            if (qm > a.mmax) qm = a.mmax;
            const float M = ((float) qm - (float) a.moff) * m;
            float e = 0.0f;
            if constexpr (G > 0) {
                #pragma unroll
                for (int i = 0; i < G; i++) {
                    float c = __builtin_rintf((g[i] - M) / S);
                    if (c < 0.0f) c = 0.0f;
                    if (c > (float) a.nmax) c = (float) a.nmax;
                    const float dd = __builtin_fmaf(c, S, M) - g[i];
                    e = __builtin_fmaf(dd * dd, wg ? wg[i] : 1.0f, e);
                }
            } else {
                for (int i = 0; i < GG; i++) {
                    float c = __builtin_rintf((gp[i] - M) / S);
                    if (c < 0.0f) c = 0.0f;
                    if (c > (float) a.nmax) c = (float) a.nmax;
                    const float dd = __builtin_fmaf(c, S, M) - gp[i];
                    e = __builtin_fmaf(dd * dd, wg ? wg[i] : 1.0f, e);
                }
            }
            if (first || e < be) { be = e; bs = qs; bm = qm; first = false; }
        }
    }
    if (a.q8) { a.q8[t] = bs; a.mq8[t] = bm; }
    else { a.sq[t] = (uint8_t) bs; a.mq[t] = (uint8_t) bm; }
    if (a.eff_s) {
        a.eff_s[t] = (float) bs * d;
        a.eff_m[t] = ((float) bm - (float) a.moff) * m;
    }
}

extern "C" __global__ __launch_bounds__(256) void sml_ing_field(const sml_king_field a) {
    const int ng = a.cols / a.group;
    const int64_t t = (int64_t) blockIdx.x * 256 + threadIdx.x;
    if (t >= (int64_t) a.rows * ng) return;
    const int j = (int) (t % ng);
    const float * gp = a.w + (size_t) t * a.group;
    if (a.group == 32) field_body<32>(a, t, j, gp);
    else field_body<0>(a, t, j, gp);
}

// ---------------------------------------------------------------- codes into planes
// One thread per 128 weights (4 groups) of a row: the codes against the
// stored step and min (tooling/sml_quantize.py:565-572), then each plane of
// the width in the file's layout (tooling/sml_quantize.py:614-651,
// tooling/sml_format.py:392-448): a nibble plane as 64-byte quads (bytes
// 0-31 lo/hi = groups 0/1, bytes 32-63 = groups 2/3), a 2-bit plane as 32
// bytes (bits 2k of byte j = group k, weight j), a 1-bit plane as 4 bytes per
// group (bit i of byte b = weight 8b+i). Q6 stores bits 4-5 first, then the
// low nibble; the other widths take their planes lowest bits first.
extern "C" __global__ __launch_bounds__(256) void sml_ing_pack(const sml_king_pack a) {
    const int nq = a.cols / 128, ng = a.cols / 32;
    const int64_t t = (int64_t) blockIdx.x * 256 + threadIdx.x;
    if (t >= (int64_t) a.rows * nq) return;
    const int64_t r = t / nq;
    const int qd = (int) (t % nq);
    const float nmax = (float) ((1 << a.nbits) - 1);
    uint32_t cw[32];               // 128 codes, 4 per word, weight i in byte i%4 of word i/4
    #pragma unroll
    for (int gg = 0; gg < 4; gg++) {
        const int64_t o = r * ng + 4 * qd + gg;
        const float S = fmaxf(a.eff_s[o], 1e-12f), M = a.eff_m[o];
        const float * wp = a.wp + r * a.cols + (size_t) (4 * qd + gg) * 32;
        #pragma unroll
        for (int i = 0; i < 32; i += 4) {
            const float4 v = *(const float4 *) (wp + i);
            const float x[4] = { v.x, v.y, v.z, v.w };
            uint32_t word = 0;
            #pragma unroll
            for (int b = 0; b < 4; b++) {
                float c = __builtin_rintf((x[b] - M) / S);
                c = c < 0.0f ? 0.0f : c > nmax ? nmax : c;
                word |= (uint32_t) c << (8 * b);
            }
            cw[gg * 8 + i / 4] = word;
        }
    }
    if (a.codes) {
        uint4 * dst = (uint4 *) (a.codes + r * a.cols + (size_t) qd * 128);
        #pragma unroll
        for (int k = 0; k < 8; k++) dst[k] = make_uint4(cw[4 * k], cw[4 * k + 1], cw[4 * k + 2], cw[4 * k + 3]);
    }
    // planes of the width: (bits, shift) in storage order
    int nb[3], sh[3], np = 0;
    switch (a.nbits) {
        case 2: nb[0] = 2; sh[0] = 0; np = 1; break;
        case 3: nb[0] = 2; sh[0] = 0; nb[1] = 1; sh[1] = 2; np = 2; break;
        case 4: nb[0] = 4; sh[0] = 0; np = 1; break;
        case 5: nb[0] = 4; sh[0] = 0; nb[1] = 1; sh[1] = 4; np = 2; break;
        case 6: nb[0] = 2; sh[0] = 4; nb[1] = 4; sh[1] = 0; np = 2; break;
        case 7: nb[0] = 4; sh[0] = 0; nb[1] = 2; sh[1] = 4; nb[2] = 1; sh[2] = 6; np = 3; break;
        default: nb[0] = 4; sh[0] = 0; nb[1] = 4; sh[1] = 4; np = 2; break;
    }
    for (int p = 0; p < np; p++) {
        const uint32_t s = (uint32_t) sh[p];
        if (nb[p] == 4) {
            // byte j of half h: group 2h weight j (lo) | group 2h+1 weight j (hi)
            uint32_t out[16];
            #pragma unroll
            for (int h = 0; h < 2; h++)
                #pragma unroll
                for (int k = 0; k < 8; k++) {
                    const uint32_t lo = (cw[(2 * h) * 8 + k] >> s) & 0x0F0F0F0Fu;
                    const uint32_t hi = (cw[(2 * h + 1) * 8 + k] >> s) & 0x0F0F0F0Fu;
                    out[h * 8 + k] = lo | (hi << 4);
                }
            uint4 * dst = (uint4 *) (a.plane[p] + r * (a.cols / 2) + (size_t) qd * 64);
            #pragma unroll
            for (int k = 0; k < 4; k++) dst[k] = make_uint4(out[4 * k], out[4 * k + 1], out[4 * k + 2], out[4 * k + 3]);
        } else if (nb[p] == 2) {
            uint32_t out[8];
            #pragma unroll
            for (int k = 0; k < 8; k++) {
                uint32_t b = 0;
                #pragma unroll
                for (int gg = 0; gg < 4; gg++) b |= ((cw[gg * 8 + k] >> s) & 0x03030303u) << (2 * gg);
                out[k] = b;
            }
            uint4 * dst = (uint4 *) (a.plane[p] + r * (a.cols / 4) + (size_t) qd * 32);
            dst[0] = make_uint4(out[0], out[1], out[2], out[3]);
            dst[1] = make_uint4(out[4], out[5], out[6], out[7]);
        } else {
            uint32_t out[4];
            #pragma unroll
            for (int gg = 0; gg < 4; gg++) {
                uint32_t word = 0;
                #pragma unroll
                for (int i = 0; i < 32; i++) word |= ((cw[gg * 8 + i / 4] >> (8 * (i % 4) + s)) & 1u) << i;
                out[gg] = word;
            }
            *(uint4 *) (a.plane[p] + r * (a.cols / 8) + (size_t) qd * 16) = make_uint4(out[0], out[1], out[2], out[3]);
        }
    }
}
