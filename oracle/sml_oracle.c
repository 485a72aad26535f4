// CPU ORACLE — test infrastructure only (see sml_oracle.h). Never linked into
// or called by the GPU library.
#include "sml_oracle.h"

#include <fcntl.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

// ------------------------------------------------------------ activations

// sml/sml-kernel.c:86-106: amax over 32, s = amax/127, is = 1/s (0 when s == 0),
// q = lrintf(x*is) clamped to +-127 (lrintf rounds half to even under the
// default rounding mode), sums = sum of q.
void orc_quantize_act(const float * x, int n, int8_t * q, float * scale, int32_t * sums) {
    for (int g = 0; g < n / 32; g++) {
        const float * xs = x + g * 32;
        float amax = 0.0f;
        for (int i = 0; i < 32; i++) { const float v = fabsf(xs[i]); if (v > amax) amax = v; }
        const float s = amax / 127.0f;
        const float is = s > 0.0f ? 1.0f / s : 0.0f;
        int32_t sum = 0;
        for (int i = 0; i < 32; i++) {
            long v = lrintf(xs[i] * is);
            if (v > 127) v = 127;
            if (v < -127) v = -127;
            q[g * 32 + i] = (int8_t) v;
            sum += (int32_t) v;
        }
        scale[g] = s;
        sums[g] = sum;
    }
}

// sml/sml-kernel.c:165-184: one amax per 256 values (the partial last superblock
// uses what it has), the same s/is/rounding, the scale copied into every group.
void orc_quantize_act_sb(const float * x, int n, int8_t * q, float * scale, int32_t * sums) {
    const int ng = n / 32;
    for (int g0 = 0; g0 < ng; g0 += 8) {
        const int g1 = g0 + 8 < ng ? g0 + 8 : ng;
        float amax = 0.0f;
        for (int i = g0 * 32; i < g1 * 32; i++) { const float v = fabsf(x[i]); if (v > amax) amax = v; }
        const float s = amax / 127.0f;
        const float is = s > 0.0f ? 1.0f / s : 0.0f;
        for (int g = g0; g < g1; g++) {
            int32_t sum = 0;
            for (int i = 0; i < 32; i++) {
                long v = lrintf(x[g * 32 + i] * is);
                if (v > 127) v = 127;
                if (v < -127) v = -127;
                q[g * 32 + i] = (int8_t) v;
                sum += (int32_t) v;
            }
            scale[g] = s;
            sums[g] = sum;
        }
    }
}

// ------------------------------------------------------------ fp16

// sml/sml-run.c:85-109 (scalar encode, round to nearest even)
uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u, rawe = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    if (rawe == 0xffu) return (uint16_t) (sign | 0x7c00u | (man ? 0x200u : 0u));
    const int32_t e = (int32_t) rawe - 127 + 15;
    if (e >= 31) return (uint16_t) (sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t) sign;
        man |= 0x800000u;
        const uint32_t sh = (uint32_t) (14 - e);
        uint32_t sub = man >> sh;
        const uint32_t rem = man & ((1u << sh) - 1u), half = 1u << (sh - 1u);
        if (rem > half || (rem == half && (sub & 1u))) sub++;
        return (uint16_t) (sign | sub);
    }
    uint32_t h = ((uint32_t) e << 10) | (man >> 13);
    const uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t) (sign | h);
}

// sml/sml-kernel.c:14-38 (scalar decode)
float orc_f16_to_f32(uint16_t h) {
    uint32_t s = (uint32_t) (h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu, bits;
    if (e == 0) {
        if (m == 0) bits = s;
        else {
            e = 127 - 15 + 1;
            while (!(m & 0x400u)) { m <<= 1; e--; }
            m &= 0x3ffu;
            bits = s | (e << 23) | (m << 13);
        }
    } else if (e == 31) bits = s | 0x7f800000u | (m << 13);
    else bits = s | ((e - 15 + 127) << 23) | (m << 13);
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

// ------------------------------------------------------------ fields and codes

// sml/sml-kernel.h:79-98: four 6-bit values in three bytes
static int field(const uint8_t * base, int g, int six) {
    if (!six) return base[g];
    const uint8_t * p = base + (size_t) (g >> 2) * 3;
    const uint32_t b0 = p[0], b1 = p[1], b2 = p[2];
    switch (g & 3) {
    case 0: return (int) (b0 & 63u);
    case 1: return (int) (((b0 >> 6) | (b1 << 2)) & 63u);
    case 2: return (int) (((b1 >> 4) | (b2 << 4)) & 63u);
    default: return (int) ((b2 >> 2) & 63u);
    }
}

static size_t field_row(const orc_tensor * t) {
    const int ng = t->cols / 32;
    return t->scale6 ? (size_t) (ng / 4) * 3 : (size_t) ng;
}

float orc_step(const orc_tensor * t, int row, int g) {
    const int ns = (t->cols / 32 + 7) / 8;
    return orc_f16_to_f32(t->sd[(size_t) row * ns + g / 8])
         * (float) field(t->sq + (size_t) row * field_row(t), g, t->scale6);
}

float orc_min(const orc_tensor * t, int row, int g) {
    if (!t->mq) return 0.0f;
    const int ns = (t->cols / 32 + 7) / 8;
    const float bias = t->scale6 ? (t->minneg ? 63.0f : 31.0f) : 127.0f;
    return orc_f16_to_f32(t->md[(size_t) row * ns + g / 8])
         * ((float) field(t->mq + (size_t) row * field_row(t), g, t->scale6) - bias);
}

// one plane's bits of every weight of a row, per plane width
static void plane_bits(const uint8_t * plane, int pbits, int row, int cols, int * out) {
    if (pbits == 4) {
        // sml/sml-kernel.c:2140-2156: quad of 64 bytes = 4 groups; first 32 bytes
        // hold groups 4q (low nibble) and 4q+1 (high), the second 32 the next two
        const uint8_t * cp = plane + (size_t) row * (cols / 2);
        for (int g = 0; g < cols / 32; g++) {
            const uint8_t * blk = cp + (size_t) (g / 4) * 64 + ((g % 4) >= 2 ? 32 : 0);
            const int hi = g & 1;
            for (int j = 0; j < 32; j++) out[g * 32 + j] = hi ? (blk[j] >> 4) & 15 : blk[j] & 15;
        }
    } else if (pbits == 2) {
        // sml/sml-kernel.c:243-250: pack of 32 bytes per 128 weights, bit-plane
        // k of byte j is weight 128p + 32k + j
        const uint8_t * cp = plane + (size_t) row * (cols / 4);
        for (int col = 0; col < cols; col++) {
            const int p = col / 128, k = (col % 128) / 32, j = col % 32;
            out[col] = (cp[(size_t) p * 32 + j] >> (2 * k)) & 3;
        }
    } else {
        // sml/sml-kernel.c:2164-2169: 4 bytes per group, bit j = weight j
        const uint8_t * cp = plane + (size_t) row * (cols / 8);
        for (int col = 0; col < cols; col++) {
            const int g = col / 32, j = col % 32;
            out[col] = (cp[(size_t) g * 4 + (j >> 3)] >> (j & 7)) & 1;
        }
    }
}

void orc_unpack_row(const orc_tensor * t, int row, uint8_t * codes) {
    const int n = t->cols;
    int * a = malloc((size_t) n * sizeof(int)), * b = malloc((size_t) n * sizeof(int));
    for (int i = 0; i < n; i++) codes[i] = 0;
    switch (t->nbits) {
    case 2:
        plane_bits(t->plane[0], 2, row, n, a);
        for (int i = 0; i < n; i++) codes[i] = (uint8_t) a[i];
        break;
    case 3: // 2-bit plane + 4 * 1-bit plane (sml/sml-run.c:589-592)
        plane_bits(t->plane[0], 2, row, n, a);
        plane_bits(t->plane[1], 1, row, n, b);
        for (int i = 0; i < n; i++) codes[i] = (uint8_t) (a[i] | (b[i] << 2));
        break;
    case 4:
        plane_bits(t->plane[0], 4, row, n, a);
        for (int i = 0; i < n; i++) codes[i] = (uint8_t) a[i];
        break;
    case 5: // nibble + 16 * 1-bit (sml/sml-run.c:593-595)
        plane_bits(t->plane[0], 4, row, n, a);
        plane_bits(t->plane[1], 1, row, n, b);
        for (int i = 0; i < n; i++) codes[i] = (uint8_t) (a[i] | (b[i] << 4));
        break;
    case 6: // plane 0 = 2-bit high part, plane 1 = nibble (sml/sml-run.c:3319-3326)
        plane_bits(t->plane[0], 2, row, n, a);
        plane_bits(t->plane[1], 4, row, n, b);
        for (int i = 0; i < n; i++) codes[i] = (uint8_t) (b[i] | (a[i] << 4));
        break;
    case 7: { // nibble + 16 * 2-bit + 64 * 1-bit (sml/sml-run.c:596-602)
        int * c = malloc((size_t) n * sizeof(int));
        plane_bits(t->plane[0], 4, row, n, a);
        plane_bits(t->plane[1], 2, row, n, b);
        plane_bits(t->plane[2], 1, row, n, c);
        for (int i = 0; i < n; i++) codes[i] = (uint8_t) (a[i] | (b[i] << 4) | (c[i] << 6));
        free(c);
        break;
    }
    case 8: // low + 16 * high nibble planes (sml/sml-kernel.c:2185-2197)
        plane_bits(t->plane[0], 4, row, n, a);
        plane_bits(t->plane[1], 4, row, n, b);
        for (int i = 0; i < n; i++) codes[i] = (uint8_t) (a[i] | (b[i] << 4));
        break;
    default:
        break;
    }
    free(a); free(b);
}

// The reference build (-O3 with FMA) contracts code*step + min into one fused
// multiply-add; Q3, Q5 and Q7 then add their 1-bit plane's share,
// step*2^shift, to that sum where the bit is set (sml_dequant_bits1_add).
// follows sml/sml-kernel.c:231-263 (2-bit), :2134-2157 (flat4), :2160-2170
// (the 1-bit add), :2174-2198 (flat8), :2235-2260 (flat6), composed per width
// as sml/sml-run.c:3300-3335 does
void orc_dequant_row(const orc_tensor * t, int row, float * out) {
    uint8_t * c = malloc((size_t) t->cols);
    orc_unpack_row(t, row, c);
    const int nb = t->nbits;
    const int shift = nb == 3 ? 2 : nb == 5 ? 4 : nb == 7 ? 6 : 0;     // the 1-bit plane's place
    const int low = shift ? (1 << shift) - 1 : 255;
    for (int g = 0; g < t->cols / 32; g++) {
        const float st = orc_step(t, row, g), mn = orc_min(t, row, g);
        const float add = st * (float) (1 << shift);
        for (int j = 0; j < 32; j++) {
            const int code = c[g * 32 + j];
            float v = fmaf((float) (code & low), st, mn);
            if (shift && (code >> shift) & 1) v = v + add;
            out[g * 32 + j] = v;
        }
    }
    free(c);
}

// Integer dot of group g of one row against the activation codes.
static int32_t group_dot(const uint8_t * c, const int8_t * q, int g) {
    int32_t d = 0;
    for (int j = 0; j < 32; j++) d += (int32_t) c[g * 32 + j] * (int32_t) q[g * 32 + j];
    return d;
}

// Q4 and Q8 in the float order of the reference's x86 build, which is the
// arm its own -march=native build selects on AVX2 hosts:
// matvec_flat4_l8 / sml_matvec_rows_il4 (sml/sml-kernel.c:572-727,836-866).
// Eight lanes, lane j taking group j of every 256-weight superblock in turn:
//   v_j = fma(wsc_j, s_g*dot_g, v_j); v_j = fma(wmin_j, s_g*sum_g, v_j)
// (the reference's mul+add pairs, which its compiler contracts to FMAs),
// wsc = f16(sd)*sq, wmin = f16(md)*(mq - bias); then the lanes fold as
// ((v0+v4)+(v1+v5)) + ((v2+v6)+(v3+v7)). A trailing half superblock (4
// groups) runs four lanes of its own, folded (t0+t1)+(t2+t3) and added last.
static float row_avx2_order(const orc_tensor * t, int r, const uint8_t * c, const int8_t * q,
                            const float * scale, const int32_t * sums) {
    const int ng = t->cols / 32, nblk = ng / 8, tail = ng - nblk * 8;
    float v[8] = { 0 }, vt[4] = { 0 };
    for (int k = 0; k <= nblk; k++) {
        const int nl = k < nblk ? 8 : tail;
        float * acc = k < nblk ? v : vt;
        for (int j = 0; j < nl; j++) {
            const int g = 8 * k + j;
            const float af = scale[g];
            acc[j] = fmaf(orc_step(t, r, g), af * (float) group_dot(c, q, g), acc[j]);
            if (t->mq) acc[j] = fmaf(orc_min(t, r, g), af * (float) sums[g], acc[j]);
        }
    }
    float tot = ((v[0] + v[4]) + (v[1] + v[5])) + ((v[2] + v[6]) + (v[3] + v[7]));
    if (tail) tot += (vt[0] + vt[1]) + (vt[2] + vt[3]);
    return tot;
}

// Other widths: per group step*s*dot + min*s*sum in group order, the scalar
// arm's arithmetic (sml/sml-kernel.c:2027-2066 flat4, :1934-1971 2-bit planes),
// with the plane dispatch of sml/sml-run.c:612-680 folded into one integer dot
// over the unpacked code (the code is linear in its planes).
static float row_group_order(const orc_tensor * t, int r, const uint8_t * c, const int8_t * q,
                             const float * scale, const int32_t * sums) {
    float sum = 0.0f;
    for (int g = 0; g < t->cols / 32; g++) {
        sum += orc_step(t, r, g) * scale[g] * (float) group_dot(c, q, g);
        if (t->mq) sum += orc_min(t, r, g) * scale[g] * (float) sums[g];
    }
    return sum;
}

void orc_matvec(const orc_tensor * t, const int8_t * q, const float * scale, const int32_t * sums,
                float * y, int row0, int row1) {
    const int n = t->cols;
    const int lanes8 = (t->nbits == 4 || t->nbits == 8) && !t->scale6;
    #pragma omp parallel
    {
        uint8_t * c = malloc((size_t) n);
        #pragma omp for schedule(static)
        for (int r = row0; r < row1; r++) {
            orc_unpack_row(t, r, c);
            y[r] = lanes8 ? row_avx2_order(t, r, c, q, scale, sums) : row_group_order(t, r, c, q, scale, sums);
        }
        free(c);
    }
}

// ------------------------------------------------------------ small ops

// sml/sml-run.c:147-152; the sum of squares is the reference build's chain of
// double FMAs, the scaling two float products
void orc_rms_norm(float * out, const float * x, const float * w, int n, float eps) {
    double ss = 0.0;
    for (int i = 0; i < n; i++) ss = fma((double) x[i], (double) x[i], ss);
    const float s = 1.0f / sqrtf((float) (ss / n) + eps);
    for (int i = 0; i < n; i++) out[i] = (x[i] * s) * w[i];
}

void orc_rope_table(float theta, int half, int n_ctx, float * cos_t, float * sin_t) {
    for (int p = 0; p < n_ctx; p++)
        for (int i = 0; i < half; i++) {
            const float freq = powf(theta, -(float) i / (float) half);
            const float a = (float) p * freq;
            cos_t[(size_t) p * half + i] = cosf(a);
            sin_t[(size_t) p * half + i] = sinf(a);
        }
}

// sml/sml-run.c:363-368 as the reference build contracts it:
// x0*cs - x1*sn = fma(x0, cs, -(x1*sn)), x0*sn + x1*cs = fma(x0, sn, x1*cs)
void orc_rope(float * x, int n_head, int head_dim, int half, const float * cs, const float * sn) {
    for (int h = 0; h < n_head; h++) {
        float * v = x + (size_t) h * head_dim;
        for (int i = 0; i < half; i++) {
            const float x0 = v[i], x1 = v[i + half];
            v[i] = fmaf(x0, cs[i], -(x1 * sn[i]));
            v[i + half] = fmaf(x0, sn[i], x1 * cs[i]);
        }
    }
}

// sml/sml-run.c:126-133 (sml_hsum256): eight lanes folded
// ((l0+l4)+(l1+l5)) + ((l2+l6)+(l3+l7))
static float hsum8(const float * l) {
    return ((l[0] + l[4]) + (l[1] + l[5])) + ((l[2] + l[6]) + (l[3] + l[7]));
}

// sml/sml-run.c:180-240 (AVX2 arm, head_dim a multiple of 64) + softmax :280-287.
// Score of position t: eight FMA lanes over the head's dims (lane l takes dims
// l, l+8, ...), folded by hsum8, times inv. Softmax: serial max, expf, a serial
// float sum, one reciprocal, products. Output dim d: one FMA chain over the
// positions in order, a[u]*v[u][d] + o.
void orc_attn_head(const float * qh, const uint16_t * kc, const uint16_t * vc, size_t stride,
                   int pos, int hd, float inv, float * a, float * out) {
    for (int t = 0; t <= pos; t++) {
        const uint16_t * kh = kc + (size_t) t * stride;
        float l[8] = { 0 };
        for (int i = 0; i < hd; i += 8)
            for (int j = 0; j < 8; j++) l[j] = fmaf(qh[i + j], orc_f16_to_f32(kh[i + j]), l[j]);
        a[t] = hsum8(l) * inv;
    }
    float mx = a[0];
    for (int i = 1; i <= pos; i++) if (a[i] > mx) mx = a[i];
    float sum = 0.0f;
    for (int i = 0; i <= pos; i++) { a[i] = expf(a[i] - mx); sum += a[i]; }
    const float iv = 1.0f / sum;
    for (int i = 0; i <= pos; i++) a[i] *= iv;
    for (int i = 0; i < hd; i++) {
        float o = 0.0f;
        for (int u = 0; u <= pos; u++) o = fmaf(a[u], orc_f16_to_f32(vc[(size_t) u * stride + i]), o);
        out[i] = o;
    }
}

// sml/sml-run.c:393-414 (sml_exp_ps) as the reference build runs it: clamp to
// [-88, 88], f = x*log2(e), r = f rounded half-even, g = f - r, 2^g by a
// degree-5 Horner chain of FMAs; the result is p * 2^r.
static float exp_poly(float x, float * p_out, float * scale_out) {
    x = x < -88.0f ? -88.0f : x > 88.0f ? 88.0f : x;
    const float f = x * 1.44269504088896341f;
    const float r = nearbyintf(f);
    const float g = f - r;
    float p = fmaf(1.3697664e-3f, g, 8.3013611e-3f);
    p = fmaf(p, g, 5.5826318e-2f);
    p = fmaf(p, g, 2.4022652e-1f);
    p = fmaf(p, g, 6.9314718e-1f);
    p = fmaf(p, g, 1.0f);
    uint32_t eb = (uint32_t) ((int32_t) r + 127) << 23;
    float sc;
    memcpy(&sc, &eb, 4);
    *p_out = p;
    *scale_out = sc;
    return p * sc;
}

// sml/sml-run.c:416-426 (silu_mul, AVX2 arm; n_ff is a multiple of 8): the
// reference build folds 1 + p*2^r into one FMA, then (g / d) * u.
void orc_silu_mul(float * g, const float * u, int n) {
    for (int i = 0; i < n; i++) {
        float p, sc;
        exp_poly(0.0f - g[i], &p, &sc);
        const float d = fmaf(p, sc, 1.0f);
        g[i] = (g[i] / d) * u[i];
    }
}

int orc_moe_route(const float * lg, int ne, int k, unsigned moe_flags, int * sel, float * w) {
    if (k <= 0 || k > ne) k = ne;
    for (int j = 0; j < k; j++) {
        int best = -1;
        for (int e = 0; e < ne; e++) {
            int taken = 0;
            for (int q = 0; q < j; q++) if (sel[q] == e) taken = 1;
            if (!taken && (best < 0 || lg[e] > lg[best])) best = e;
        }
        sel[j] = best;
    }
    if (moe_flags & 1u) {
        double sum = 0.0;
        for (int j = 0; j < k; j++) { w[j] = expf(lg[sel[j]] - lg[sel[0]]); sum += w[j]; }
        for (int j = 0; j < k; j++) w[j] = (float) (w[j] / sum);
    } else {
        float mx = lg[0];
        for (int e = 1; e < ne; e++) if (lg[e] > mx) mx = lg[e];
        double sum = 0.0;
        for (int e = 0; e < ne; e++) sum += expf(lg[e] - mx);
        for (int j = 0; j < k; j++) w[j] = (float) (expf(lg[sel[j]] - mx) / sum);
    }
    return k;
}

// the best untaken index by key, ties to the lower index
static int orc_best_untaken(const float * key, int ne, const int * sel, int nsel) {
    int best = -1;
    for (int e = 0; e < ne; e++) {
        int taken = 0;
        for (int q = 0; q < nsel; q++) taken |= sel[q] == e;
        if (!taken && (best < 0 || key[e] > key[best])) best = e;
    }
    return best;
}

int orc_moe_route2(const float * lg, int ne, int k, unsigned moe_flags, float scale, int groups, int topk_group,
                   const float * exp_bias, int * sel, float * w) {
    if (k <= 0 || k > ne) k = ne;
    if (ne > 64) return -1;
    if (moe_flags & 4u) {
        // sparsemixer: per pick, the best untaken logit; its weight is 1 over
        // the double sum of exp(l - best) over untaken experts whose gap to
        // the best, relative to max(|l|, best), is within 2 x jitter
        const float eps2 = 2.0f * scale;
        for (int j = 0; j < k; j++) {
            const int b = orc_best_untaken(lg, ne, sel, j);
            const float mx = lg[b];
            double sum = 0.0;
            for (int e = 0; e < ne; e++) {
                int taken = 0;
                for (int q = 0; q < j; q++) taken |= sel[q] == e;
                const float f = fabsf(lg[e]) > mx ? fabsf(lg[e]) : mx;
                if (!taken && (mx - lg[e]) / f <= eps2) sum += exp((double) lg[e] - mx);
            }
            sel[j] = b;
            w[j] = (float) (1.0 / sum);
        }
        return k;
    }
    if ((moe_flags & 2u) || exp_bias || groups > 1) {
        float sc[64], ch[64];
        if (moe_flags & 2u) {
            for (int e = 0; e < ne; e++) sc[e] = 1.0f / (1.0f + expf(-lg[e]));
        } else {
            float mx = lg[0];
            for (int e = 1; e < ne; e++) if (lg[e] > mx) mx = lg[e];
            double sum = 0.0;
            for (int e = 0; e < ne; e++) sum += expf(lg[e] - mx);
            for (int e = 0; e < ne; e++) sc[e] = (float) (expf(lg[e] - mx) / sum);
        }
        for (int e = 0; e < ne; e++) ch[e] = sc[e] + (exp_bias ? exp_bias[e] : 0.0f);
        if (groups > 1 && topk_group < groups && ne % groups == 0) {
            const int per = ne / groups;
            float gs[64];
            int kept[64];
            for (int g = 0; g < groups; g++) {
                float a1 = -1e30f, a2 = -1e30f;
                for (int i = 0; i < per; i++) {
                    const float v = ch[g * per + i];
                    if (v > a1) { a2 = a1; a1 = v; } else if (v > a2) a2 = v;
                }
                gs[g] = (moe_flags & 8u) ? a1 : a1 + (per > 1 ? a2 : 0.0f);
            }
            for (int t = 0; t < topk_group; t++) kept[t] = orc_best_untaken(gs, groups, kept, t);
            for (int e = 0; e < ne; e++) {
                int keep = 0;
                for (int t = 0; t < topk_group; t++) keep |= kept[t] == e / per;
                if (!keep) ch[e] = 0.0f;
            }
        }
        for (int j = 0; j < k; j++) {
            sel[j] = orc_best_untaken(ch, ne, sel, j);
            w[j] = sc[sel[j]];
        }
        if (moe_flags & 1u) {
            float sum = 0.0f;
            for (int j = 0; j < k; j++) sum += w[j];
            for (int j = 0; j < k; j++) w[j] /= sum + 1e-20f;
        }
    } else {
        orc_moe_route(lg, ne, k, moe_flags & 1u, sel, w);
    }
    if (scale != 0.0f) for (int j = 0; j < k; j++) w[j] *= scale;
    return k;
}

void orc_router(const float * router, const float * x, int ne, int n_embd, float * lg) {
    for (int e = 0; e < ne; e++) {
        double s = 0.0;
        for (int i = 0; i < n_embd; i++) s = fma((double) router[(size_t) e * n_embd + i], (double) x[i], s);
        lg[e] = (float) s;
    }
}

int orc_argmax(const float * logits, int n) {
    int best = 0;
    float bv = logits[0];
    for (int i = 1; i < n; i++) if (logits[i] > bv) { bv = logits[i]; best = i; }
    return best;
}

// ------------------------------------------------------------ GPTQ-style 4-bit

// tooling/sml_unpack.py:66-76 (_unpack_ints): word k of column o holds codes
// of inputs 8k..8k+7, input 8k+i in bits 4i..4i+3 (dim 0 for qweight, dim 1
// for qzeros, where word j of a group row holds outputs 8j..8j+7).
void orc_gptq_unpack_row(const int32_t * qweight, const int32_t * qzeros, int rows, int cols, int group,
                         int zero_add, int row, uint8_t * codes, uint8_t * zeros) {
    for (int k = 0; k < cols; k++) {
        const uint32_t w = (uint32_t) qweight[(size_t) (k / 8) * rows + row];
        codes[k] = (uint8_t) ((w >> (4 * (k % 8))) & 15u);
    }
    for (int g = 0; g < cols / group; g++) {
        const uint32_t z = (uint32_t) qzeros[(size_t) g * (rows / 8) + row / 8];
        zeros[g] = (uint8_t) (((z >> (4 * (row % 8))) & 15u) + (uint32_t) zero_add);
    }
}

// tooling/sml_unpack.py:84-95 (dequant_gptq): (w - z[g]).float() * scales[g]
void orc_gptq_dequant_row(const int32_t * qweight, const int32_t * qzeros, const uint16_t * scales, int rows,
                          int cols, int group, int zero_add, int row, float * out) {
    uint8_t * c = malloc((size_t) cols), * z = malloc((size_t) (cols / group));
    orc_gptq_unpack_row(qweight, qzeros, rows, cols, group, zero_add, row, c, z);
    for (int k = 0; k < cols; k++) {
        const int g = k / group;
        out[k] = (float) ((int) c[k] - (int) z[g]) * orc_f16_to_f32(scales[(size_t) g * rows + row]);
    }
    free(c);
    free(z);
}

// the g_idx branch of dequant_gptq (tooling/sml_unpack.py:90-96): input k
// takes the zero and scale of group g_idx[k] (desc_act files)
void orc_gptq_dequant_row_gidx(const int32_t * qweight, const int32_t * qzeros, const uint16_t * scales,
                               const int32_t * g_idx, int rows, int cols, int group, int zero_add, int row,
                               float * out) {
    uint8_t * c = malloc((size_t) cols), * z = malloc((size_t) (cols / group));
    orc_gptq_unpack_row(qweight, qzeros, rows, cols, group, zero_add, row, c, z);
    for (int k = 0; k < cols; k++) {
        const int g = g_idx[k];
        out[k] = (float) ((int) c[k] - (int) z[g]) * orc_f16_to_f32(scales[(size_t) g * rows + row]);
    }
    free(c);
    free(z);
}

void orc_gptq_matvec_gidx(const int32_t * qweight, const int32_t * qzeros, const uint16_t * scales,
                          const int32_t * g_idx, int rows, int cols, int group, int zero_add, const float * x,
                          float * y) {
    #pragma omp parallel
    {
        float * w = malloc((size_t) cols * 4);
        #pragma omp for schedule(static)
        for (int r = 0; r < rows; r++) {
            orc_gptq_dequant_row_gidx(qweight, qzeros, scales, g_idx, rows, cols, group, zero_add, r, w);
            double acc = 0.0;
            for (int k = 0; k < cols; k++) acc += (double) w[k] * (double) x[k];
            y[r] = (float) acc;
        }
        free(w);
    }
}

void orc_gptq_matvec(const int32_t * qweight, const int32_t * qzeros, const uint16_t * scales, int rows, int cols,
                     int group, int zero_add, const float * x, float * y) {
    #pragma omp parallel
    {
        float * w = malloc((size_t) cols * 4);
        #pragma omp for schedule(static)
        for (int r = 0; r < rows; r++) {
            orc_gptq_dequant_row(qweight, qzeros, scales, rows, cols, group, zero_add, r, w);
            double acc = 0.0;
            for (int k = 0; k < cols; k++) acc += (double) w[k] * (double) x[k];
            y[r] = (float) acc;
        }
        free(w);
    }
}

// ------------------------------------------------------------ AWQ 4-bit

// tooling/sml_unpack.py:78,100-118 (dequant_awq): qweight int32 [cols][rows/8]
// packs 8 OUTPUTS per word, output 8j+k of word j in nibble AWQ_REVERSE[k]
// with AWQ_REVERSE = (0, 4, 1, 5, 2, 6, 3, 7); qzeros [cols/group][rows/8]
// the same way, or, absent, zero 2^(bits-1) = 8; no +1 on the zeros.
static const int awq_nibble[8] = { 0, 4, 1, 5, 2, 6, 3, 7 };

void orc_awq_unpack_row(const int32_t * qweight, const int32_t * qzeros, int rows, int cols, int group, int row,
                        uint8_t * codes, uint8_t * zeros) {
    const int sh = 4 * awq_nibble[row % 8];
    for (int k = 0; k < cols; k++)
        codes[k] = (uint8_t) (((uint32_t) qweight[(size_t) k * (rows / 8) + row / 8] >> sh) & 15u);
    for (int g = 0; g < cols / group; g++)
        zeros[g] = qzeros ? (uint8_t) (((uint32_t) qzeros[(size_t) g * (rows / 8) + row / 8] >> sh) & 15u) : 8;
}

// (w - z[g]).float() * scales[g], scales fp16 [cols/group][rows]
void orc_awq_dequant_row(const int32_t * qweight, const int32_t * qzeros, const uint16_t * scales, int rows,
                         int cols, int group, int row, float * out) {
    uint8_t * c = malloc((size_t) cols), * z = malloc((size_t) (cols / group));
    orc_awq_unpack_row(qweight, qzeros, rows, cols, group, row, c, z);
    for (int k = 0; k < cols; k++) {
        const int g = k / group;
        out[k] = (float) ((int) c[k] - (int) z[g]) * orc_f16_to_f32(scales[(size_t) g * rows + row]);
    }
    free(c);
    free(z);
}

// ------------------------------------------------------------ decoder

// The oracle reads the file with its own parser: offsets of the packed
// header and record structs (sml/sml-model.h:78-160), independent of the GPU
// library's reader.
#define H_N_LAYER 8
#define REC_SIZE 248

typedef struct {
    char name[64];
    uint32_t kind, rows, cols;
    uint64_t f32_off, sd_off, sq_off, perm_off, md_off, mq_off, mq_n;
    uint64_t plane_off[4];
    uint32_t nbits;
} orec;

typedef struct {
    const orec * q, * k, * v, * o, * gate, * up, * down;
    const float * an, * fn, * qb, * kb, * vb;
    const float * router;
    int ne;
    const orec ** eg, ** eu, ** ed;
} olayer;

struct orc_model {
    int per256;
    const uint8_t * base;
    size_t size;
    uint32_t n_layer, n_embd, n_head, n_kv, n_ff, n_vocab;
    float theta, eps;
    uint32_t flags, n_expert_used, moe_flags;
    int n_ctx, hd, half;
    orec * recs;
    int nrec;
    olayer * L;
    const orec * emb, * head;
    const float * out_norm;
    float * rc, * rs;
    uint16_t * kc, * vc;
    float * x, * xb, * xg, * q, * k, * v, * att, * hb, * hb2, * logits, * acc, * tmp;
    int8_t * aq;
    float * as;
    int32_t * asum;
};

static uint32_t rd32(const uint8_t * p) { uint32_t v; memcpy(&v, p, 4); return v; }
static uint64_t rd64(const uint8_t * p) { uint64_t v; memcpy(&v, p, 8); return v; }
static float rdf(const uint8_t * p) { float v; memcpy(&v, p, 4); return v; }

static const orec * findrec(const orc_model * m, const char * fmt, int a, int b) {
    char nm[96];
    snprintf(nm, sizeof nm, fmt, a, b);
    for (int i = 0; i < m->nrec; i++) if (strncmp(m->recs[i].name, nm, 64) == 0) return &m->recs[i];
    return NULL;
}

static orc_tensor view(const orc_model * m, const orec * r) {
    orc_tensor t;
    memset(&t, 0, sizeof t);
    for (int i = 0; i < 4; i++) t.plane[i] = r->plane_off[i] ? m->base + r->plane_off[i] : NULL;
    t.sd = (const uint16_t *) (m->base + r->sd_off);
    t.sq = m->base + r->sq_off;
    t.md = r->mq_n ? (const uint16_t *) (m->base + r->md_off) : NULL;
    t.mq = r->mq_n ? m->base + r->mq_off : NULL;
    t.rows = (int) r->rows; t.cols = (int) r->cols; t.nbits = (int) r->nbits;
    t.scale6 = (m->flags & 2u) != 0;
    t.minneg = (m->flags & 4u) != 0;
    return t;
}

int orc_model_tensor(const orc_model * m, const char * name, orc_tensor * out, const int32_t ** perm) {
    for (int i = 0; i < m->nrec; i++)
        if (strncmp(m->recs[i].name, name, 64) == 0) {
            *out = view(m, &m->recs[i]);
            if (perm) *perm = (const int32_t *) (m->base + m->recs[i].perm_off);
            return 1;
        }
    return 0;
}

orc_model * orc_model_open(const char * path, int n_ctx) {
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return NULL;
    struct stat st;
    if (fstat(fd, &st) != 0) { close(fd); return NULL; }
    void * base = mmap(NULL, (size_t) st.st_size, PROT_READ, MAP_SHARED, fd, 0);
    close(fd);
    if (base == MAP_FAILED) return NULL;
    orc_model * m = calloc(1, sizeof *m);
    const uint8_t * h = (const uint8_t *) base;
    m->base = h; m->size = (size_t) st.st_size;
    // header offsets (packed): magic 0, version 4, n_layer 8 .. n_ctx_train 32,
    // rope_theta 36, rms_eps 40, group 44, n_levels 48, level_bits 52..67,
    // n_tensors 68, table_off 76, ..., flags 152, n_expert_used 168, moe_flags 172
    m->n_layer = rd32(h + 8); m->n_embd = rd32(h + 12); m->n_head = rd32(h + 16);
    m->n_kv = rd32(h + 20); m->n_ff = rd32(h + 24); m->n_vocab = rd32(h + 28);
    m->theta = rdf(h + 36); m->eps = rdf(h + 40);
    const uint64_t nt = rd64(h + 68), toff = rd64(h + 76);
    m->flags = rd32(h + 152);
    m->n_expert_used = rd32(h + 168); m->moe_flags = rd32(h + 172);
    m->nrec = (int) nt;
    m->recs = calloc((size_t) nt, sizeof(orec));
    for (uint64_t i = 0; i < nt; i++) {
        const uint8_t * r = h + toff + i * REC_SIZE;
        orec * o = &m->recs[i];
        memcpy(o->name, r, 64);
        o->kind = rd32(r + 64); o->rows = rd32(r + 68); o->cols = rd32(r + 72);
        o->f32_off = rd64(r + 80);
        o->sd_off = rd64(r + 96); o->sq_off = rd64(r + 112); o->perm_off = rd64(r + 128);
        o->md_off = rd64(r + 144); o->mq_off = rd64(r + 160); o->mq_n = rd64(r + 168);
        for (int j = 0; j < 4; j++) o->plane_off[j] = rd64(r + 176 + 8 * j);
        o->nbits = rd32(r + 244);
    }
    m->n_ctx = n_ctx;
    m->hd = (int) (m->n_embd / m->n_head);
    const orec * q0 = findrec(m, "blk.%d.attn_q.weight", 0, 0);
    if (q0 && q0->rows % m->n_head == 0) m->hd = (int) (q0->rows / m->n_head);
    m->half = m->hd / 2;
    m->emb = findrec(m, "token_embd.weight", 0, 0);
    m->head = findrec(m, "output.weight", 0, 0);
    if (!m->head) m->head = m->emb;
    const orec * on = findrec(m, "output_norm.weight", 0, 0);
    m->out_norm = on ? (const float *) (h + on->f32_off) : NULL;
    m->L = calloc(m->n_layer, sizeof(olayer));
    for (int L = 0; L < (int) m->n_layer; L++) {
        olayer * y = &m->L[L];
        y->q = findrec(m, "blk.%d.attn_q.weight", L, 0);
        y->k = findrec(m, "blk.%d.attn_k.weight", L, 0);
        y->v = findrec(m, "blk.%d.attn_v.weight", L, 0);
        y->o = findrec(m, "blk.%d.attn_output.weight", L, 0);
        const orec * r;
        y->an = (r = findrec(m, "blk.%d.attn_norm.weight", L, 0)) ? (const float *) (h + r->f32_off) : NULL;
        y->fn = (r = findrec(m, "blk.%d.ffn_norm.weight", L, 0)) ? (const float *) (h + r->f32_off) : NULL;
        y->qb = (r = findrec(m, "blk.%d.attn_q.bias", L, 0)) ? (const float *) (h + r->f32_off) : NULL;
        y->kb = (r = findrec(m, "blk.%d.attn_k.bias", L, 0)) ? (const float *) (h + r->f32_off) : NULL;
        y->vb = (r = findrec(m, "blk.%d.attn_v.bias", L, 0)) ? (const float *) (h + r->f32_off) : NULL;
        y->gate = findrec(m, "blk.%d.ffn_gate.weight", L, 0);
        y->up = findrec(m, "blk.%d.ffn_up.weight", L, 0);
        y->down = findrec(m, "blk.%d.ffn_down.weight", L, 0);
        const orec * rt = findrec(m, "blk.%d.ffn_gate_inp.weight", L, 0);
        if (rt) {
            y->router = (const float *) (h + rt->f32_off);
            y->ne = (int) (((uint64_t) rt->rows * rt->cols) / m->n_embd);
            y->eg = calloc((size_t) y->ne, sizeof(orec *));
            y->eu = calloc((size_t) y->ne, sizeof(orec *));
            y->ed = calloc((size_t) y->ne, sizeof(orec *));
            for (int e = 0; e < y->ne; e++) {
                y->eg[e] = findrec(m, "blk.%d.ffn_gate.%d.weight", L, e);
                y->eu[e] = findrec(m, "blk.%d.ffn_up.%d.weight", L, e);
                y->ed[e] = findrec(m, "blk.%d.ffn_down.%d.weight", L, e);
            }
        }
    }
    m->rc = malloc((size_t) n_ctx * m->half * sizeof(float));
    m->rs = malloc((size_t) n_ctx * m->half * sizeof(float));
    orc_rope_table(m->theta, m->half, n_ctx, m->rc, m->rs);
    const size_t kvd = (size_t) m->n_kv * m->hd;
    m->kc = calloc((size_t) m->n_layer * n_ctx * kvd, 2);
    m->vc = calloc((size_t) m->n_layer * n_ctx * kvd, 2);
    size_t wide = m->n_ff > m->n_embd ? m->n_ff : m->n_embd;
    if ((size_t) m->n_head * m->hd > wide) wide = (size_t) m->n_head * m->hd;
    m->x = calloc(wide, 4); m->xb = calloc(wide, 4); m->xg = calloc(wide, 4);
    m->q = calloc((size_t) m->n_head * m->hd, 4); m->k = calloc(kvd, 4); m->v = calloc(kvd, 4);
    m->att = calloc((size_t) n_ctx, 4);
    m->hb = calloc(wide, 4); m->hb2 = calloc(wide, 4);
    m->acc = calloc(wide, 4); m->tmp = calloc(wide, 4);
    m->logits = calloc(m->n_vocab, 4);
    m->aq = calloc(wide, 1); m->as = calloc(wide / 32, 4); m->asum = calloc(wide / 32, 4);
    return m;
}

void orc_model_close(orc_model * m) {
    if (!m) return;
    for (int L = 0; L < (int) m->n_layer; L++) { free(m->L[L].eg); free(m->L[L].eu); free(m->L[L].ed); }
    free(m->L); free(m->recs); free(m->rc); free(m->rs); free(m->kc); free(m->vc);
    free(m->x); free(m->xb); free(m->xg); free(m->q); free(m->k); free(m->v); free(m->att);
    free(m->hb); free(m->hb2); free(m->acc); free(m->tmp); free(m->logits);
    free(m->aq); free(m->as); free(m->asum);
    munmap((void *) m->base, m->size);
    free(m);
}

int orc_n_vocab(const orc_model * m) { return (int) m->n_vocab; }

// Activation regime of every product: per 32 values (0, stepped decode) or per
// 256 (1, the batched regime: sml_quantize_act_sb before each product, whose
// per-group kernels are exact on it, sml/sml-kernel.h:314-318,
// sml/sml-run.c:2103-2127).
void orc_model_per256(orc_model * m, int on) { m->per256 = on; }

// ORC_DUMP=<file> appends the residual after the embedding and after every
// layer, in the reference's SML_DUMP format (sml/sml-run.c:2696-2703)
static void dump_x(const float * x, int n) {
    const char * p = getenv("ORC_DUMP");
    if (!p) return;
    FILE * f = fopen(p, "ab");
    if (!f) return;
    fwrite(x, sizeof(float), (size_t) n, f);
    fclose(f);
}

// gather through the tensor's permutation, quantize, matvec (sml/sml-run.c:711-757)
static void mv(orc_model * m, const orec * r, const float * x, float * y) {
    const int n = (int) r->cols;
    const int32_t * perm = (const int32_t *) (m->base + r->perm_off);
    for (int i = 0; i < n; i++) m->xg[i] = x[perm[i]];
    if (m->per256) orc_quantize_act_sb(m->xg, n, m->aq, m->as, m->asum);
    else           orc_quantize_act(m->xg, n, m->aq, m->as, m->asum);
    orc_tensor t = view(m, r);
    orc_matvec(&t, m->aq, m->as, m->asum, y, 0, (int) r->rows);
}

const float * orc_forward(orc_model * m, int token, int pos) {
    const int E = (int) m->n_embd, H = (int) m->n_head, KV = (int) m->n_kv, hd = m->hd;
    const int kvd = KV * hd, rep = H / KV, F = (int) m->n_ff;
    // embedding: dequantized row, scattered back through the permutation (sml/sml-run.c:3291-3344)
    {
        orc_tensor t = view(m, m->emb);
        orc_dequant_row(&t, token, m->xb);
        const int32_t * perm = (const int32_t *) (m->base + m->emb->perm_off);
        for (int i = 0; i < E; i++) m->x[perm[i]] = m->xb[i];
        dump_x(m->x, E);
    }
    for (int L = 0; L < (int) m->n_layer; L++) {
        const olayer * y = &m->L[L];
        orc_rms_norm(m->xb, m->x, y->an, E, m->eps);
        mv(m, y->q, m->xb, m->q);
        mv(m, y->k, m->xb, m->k);
        mv(m, y->v, m->xb, m->v);
        if (y->qb) for (int i = 0; i < H * hd; i++) m->q[i] += y->qb[i];
        if (y->kb) for (int i = 0; i < kvd; i++) m->k[i] += y->kb[i];
        if (y->vb) for (int i = 0; i < kvd; i++) m->v[i] += y->vb[i];
        orc_rope(m->q, H, hd, m->half, m->rc + (size_t) pos * m->half, m->rs + (size_t) pos * m->half);
        orc_rope(m->k, KV, hd, m->half, m->rc + (size_t) pos * m->half, m->rs + (size_t) pos * m->half);
        uint16_t * kl = m->kc + (size_t) L * m->n_ctx * kvd, * vl = m->vc + (size_t) L * m->n_ctx * kvd;
        for (int i = 0; i < kvd; i++) {
            kl[(size_t) pos * kvd + i] = orc_f32_to_f16(m->k[i]);
            vl[(size_t) pos * kvd + i] = orc_f32_to_f16(m->v[i]);
        }
        const float inv = 1.0f / sqrtf((float) hd);
        for (int h = 0; h < H; h++) {
            const int kh = h / rep;
            orc_attn_head(m->q + (size_t) h * hd, kl + (size_t) kh * hd, vl + (size_t) kh * hd, (size_t) kvd,
                          pos, hd, inv, m->att, m->xb + (size_t) h * hd);
        }
        mv(m, y->o, m->xb, m->hb2);
        for (int i = 0; i < E; i++) m->x[i] += m->hb2[i];
        orc_rms_norm(m->xb, m->x, y->fn, E, m->eps);
        if (y->ne) {
            // sml/sml-run.c:3071-3124: router in double, route, experts summed in choice order
            float lg[64];
            int sel[8];
            float w[8];
            orc_router(y->router, m->xb, y->ne, E, lg);
            const int k = orc_moe_route(lg, y->ne, (int) m->n_expert_used, m->moe_flags, sel, w);
            for (int i = 0; i < E; i++) m->acc[i] = 0.0f;
            for (int j = 0; j < k; j++) {
                const int e = sel[j];
                const int fe = (int) y->eu[e]->rows;
                mv(m, y->eg[e], m->xb, m->hb);
                mv(m, y->eu[e], m->xb, m->hb2);
                orc_silu_mul(m->hb, m->hb2, fe);
                mv(m, y->ed[e], m->hb, m->tmp);
                for (int i = 0; i < E; i++) m->acc[i] = fmaf(w[j], m->tmp[i], m->acc[i]);
            }
            for (int i = 0; i < E; i++) m->x[i] += m->acc[i];
            dump_x(m->x, E);
            continue;
        }
        mv(m, y->gate, m->xb, m->hb);
        mv(m, y->up, m->xb, m->hb2);
        orc_silu_mul(m->hb, m->hb2, F);
        mv(m, y->down, m->hb, m->xb);
        for (int i = 0; i < E; i++) m->x[i] += m->xb[i];
        dump_x(m->x, E);
    }
    orc_rms_norm(m->xb, m->x, m->out_norm, E, m->eps);
    mv(m, m->head, m->xb, m->logits);
    return m->logits;
}

// ---------------------------------------------------------------- expf restated
// follows the published algorithm of glibc's expf (sysdeps/ieee754/flt-32/e_expf.c
// in glibc >= 2.27, from ARM's optimized-routines), which the reference's
// softmax and routing call (sml/sml-run.c:180-287,2925-3037)
static const uint64_t ORC_EXPF_TAB[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull };

float orc_expf_published(float x) {
    if (x < -0x1.9fe368p6f) return 0.0f;
    if (x > 0x1.62e42ep6f) return INFINITY;
    const double C0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32, C1 = 0x1.ebfce50fac4f3p-3 / 32 / 32,
                 C2 = 0x1.62e42ff0c52d6p-1 / 32, InvLn2N = 0x1.71547652b82fep+0 * 32, Shift = 0x1.8p+52;
    const double xd = (double) x;
    double kd = fma(InvLn2N, xd, Shift);
    uint64_t ki;
    memcpy(&ki, &kd, 8);
    kd -= Shift;
    const double r = fma(InvLn2N, xd, -kd);
    const uint64_t sb = ORC_EXPF_TAB[ki % 32] + (ki << 47);
    double s;
    memcpy(&s, &sb, 8);
    const double z = fma(C0, r, C1), r2 = r * r;
    double y = fma(C2, r, 1.0);
    y = fma(z, r2, y);
    return (float) (y * s);
}

// every stride-th float <= 0 (-0 to -inf), then (positive) 0 to +inf
long orc_expf_mismatches(unsigned stride) {
    long bad = 0;
    if (stride == 0) stride = 1;
    #pragma omp parallel for reduction(+ : bad) schedule(static)
    for (long long v = 0; v <= 0xff800000ll - 0x80000000ll + 1 + 0x7f800000ll; v += stride) {
        const long long u = v <= 0xff800000ll - 0x80000000ll ? v + 0x80000000ll : v - (0xff800000ll - 0x80000000ll) - 1;
        const uint32_t b = (uint32_t) u;
        float x;
        memcpy(&x, &b, 4);
        const float g = orc_expf_published(x), w = expf(x);
        uint32_t gb, wb;
        memcpy(&gb, &g, 4);
        memcpy(&wb, &w, 4);
        bad += gb != wb;
    }
    return bad;
}

// ---------------------------------------------------------------- GGUF Q4_K
// follows ggml's published block_q4_K format and dequantize_row_q4_K (the
// K-quant layout of llama.cpp's ggml-quants.c); the reference itself reads GGUF
// only through transformers (tooling/sml_gguf.py:1-35)
static void q4k_unpack_scale(const uint8_t * q, int j, float * sc, float * m) {
    unsigned a, b;
    if (j < 4) {
        a = q[j] & 63u;
        b = q[j + 4] & 63u;
    } else {
        a = (q[j + 4] & 15u) | ((unsigned) (q[j - 4] >> 6) << 4);
        b = (q[j + 4] >> 4) | ((unsigned) (q[j] >> 6) << 4);
    }
    *sc = (float) a;
    *m = (float) b;
}

void orc_q4k_dequant_row(const uint8_t * blocks, int cols, float * out) {
    for (int b = 0; b < cols / 256; b++) {
        const uint8_t * blk = blocks + (size_t) b * 144;
        uint16_t dh, mh;
        memcpy(&dh, blk, 2);
        memcpy(&mh, blk + 2, 2);
        const float d = orc_f16_to_f32(dh), dmin = orc_f16_to_f32(mh);
        const uint8_t * q = blk + 16;
        float * y = out + (size_t) b * 256;
        for (int c = 0; c < 4; c++) {
            float s1, m1, s2, m2;
            q4k_unpack_scale(blk + 4, 2 * c, &s1, &m1);
            q4k_unpack_scale(blk + 4, 2 * c + 1, &s2, &m2);
            const float d1 = d * s1, n1 = dmin * m1, d2 = d * s2, n2 = dmin * m2;
            for (int l = 0; l < 32; l++) y[l] = d1 * (float) (q[l] & 15) - n1;
            for (int l = 0; l < 32; l++) y[32 + l] = d2 * (float) (q[l] >> 4) - n2;
            q += 32;
            y += 64;
        }
    }
}

// ggml's Q8_0, Q4_0 and Q6_K blocks (see the header), each weight's float
// value rounded to fp16
int orc_gguf_dequant_f16_row(int type, const uint8_t * blocks, int cols, float * out) {
    const int qk = type == 14 ? 256 : 32;
    const size_t bs = type == 8 ? 34 : type == 2 ? 18 : type == 14 ? 210 : 0;
    if (!bs || cols % qk) return -1;
    for (int b = 0; b < cols / qk; b++) {
        const uint8_t * blk = blocks + (size_t) b * bs;
        float * y = out + (size_t) b * qk;
        uint16_t dh;
        if (type == 8) {
            memcpy(&dh, blk, 2);
            const float d = orc_f16_to_f32(dh);
            for (int i = 0; i < 32; i++) y[i] = d * (float) (int8_t) blk[2 + i];
        } else if (type == 2) {
            memcpy(&dh, blk, 2);
            const float d = orc_f16_to_f32(dh);
            for (int j = 0; j < 16; j++) {
                y[j] = d * (float) ((blk[2 + j] & 15) - 8);
                y[j + 16] = d * (float) ((blk[2 + j] >> 4) - 8);
            }
        } else {
            const uint8_t * ql = blk, * qh = blk + 128;
            const int8_t * sc = (const int8_t *) (blk + 192);
            memcpy(&dh, blk + 208, 2);
            const float d = orc_f16_to_f32(dh);
            for (int half = 0; half < 2; half++) {
                for (int l = 0; l < 32; l++) {
                    const int is = l / 16;
                    const int q1 = ((ql[l] & 15) | (((qh[l] >> 0) & 3) << 4)) - 32;
                    const int q2 = ((ql[l + 32] & 15) | (((qh[l] >> 2) & 3) << 4)) - 32;
                    const int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                    const int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                    y[l] = d * (float) sc[is] * (float) q1;
                    y[l + 32] = d * (float) sc[is + 2] * (float) q2;
                    y[l + 64] = d * (float) sc[is + 4] * (float) q3;
                    y[l + 96] = d * (float) sc[is + 6] * (float) q4;
                }
                y += 128; ql += 64; qh += 32; sc += 8;
            }
        }
    }
    for (int i = 0; i < cols; i++) out[i] = orc_f16_to_f32(orc_f32_to_f16(out[i]));
    return 0;
}

// ggml's block_q5_K and dequantize_row_q5_K: Q4_K's d, dmin and scale bytes,
// then qh[32] (bit j of byte l: the fifth bit of weight l of sub-block j) and
// the low nibbles qs[128] in Q4_K's order; weight d*sc*(q + 16*h) - dmin*m
void orc_q5k_dequant_row(const uint8_t * blocks, int cols, float * out) {
    for (int b = 0; b < cols / 256; b++) {
        const uint8_t * blk = blocks + (size_t) b * 176;
        uint16_t dh, mh;
        memcpy(&dh, blk, 2);
        memcpy(&mh, blk + 2, 2);
        const float d = orc_f16_to_f32(dh), dmin = orc_f16_to_f32(mh);
        const uint8_t * qh = blk + 16, * q = blk + 48;
        float * y = out + (size_t) b * 256;
        for (int c = 0; c < 4; c++) {
            float s1, m1, s2, m2;
            q4k_unpack_scale(blk + 4, 2 * c, &s1, &m1);
            q4k_unpack_scale(blk + 4, 2 * c + 1, &s2, &m2);
            const float d1 = d * s1, n1 = dmin * m1, d2 = d * s2, n2 = dmin * m2;
            for (int l = 0; l < 32; l++) y[l] = d1 * (float) ((q[l] & 15) + ((qh[l] >> (2 * c)) & 1 ? 16 : 0)) - n1;
            for (int l = 0; l < 32; l++) y[32 + l] = d2 * (float) ((q[l] >> 4) + ((qh[l] >> (2 * c + 1)) & 1 ? 16 : 0)) - n2;
            q += 32;
            y += 64;
        }
    }
}
