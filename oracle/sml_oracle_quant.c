// CPU ORACLE — test infrastructure only.
//
// A plain-C restatement of the reference quantizer's re-quantization of a
// float tensor into SSF FLAT codes and two-level fields -- the step a GPTQ or
// AWQ copy goes through after tooling/sml_unpack.py has dequantized it -- for
// checking the GPU ingest kernels. Only tests/ and bench.py's CPU-baseline leg
// load it; the GPU library never links, calls or falls back to it.
//
// The two searches follow sml/sml-quant.c, the fused C library the reference
// quantizer calls first (tooling/sml_quantize.py:55-84, tooling/sml_grid_c.py),
// in the float order of that file's own build line (gcc -O3 -march=native)
// for groups of 32: gcc vectorizes the grid's per-weight loops 8 wide and
// keeps every sum in order, so the sums there are plain multiplies and adds,
// while d = qv*step + l - g, the min of the refit and the field search's
// scalar loop are contracted to fused multiply-adds. Each contraction is
// written out here with fmaf, and this file is compiled with contraction
// off, so the order does not depend on this compiler's choices.
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "sml_oracle.h"

#define GMAX 256

// One candidate (l, step): codes into q, and the weighted squared error.
// follows sml/sml-quant.c:20-33 (err_of) as inlined into the grid: d =
// fma(qv, step, l) - g, e = e + (d*d)*w
static float err_of(const float * g, const float * w, int group, float l, float step, float n, int rem, float * q) {
    float e = 0.0f;
    for (int i = 0; i < group; i++) {
        float c = rintf((g[i] - l) / step);
        if (c < 0.0f) c = 0.0f;
        if (c > n) c = n;
        q[i] = c;
        const float qv = rem ? (float) ((((int) c >> rem) << rem) + (1 << (rem - 1))) : c;
        const float d = fmaf(qv, step, l) - g[i];
        e = e + (d * d) * w[i];
    }
    return e;
}

// follows sml/sml-quant.c:38-95 (sml_asym_grid)
void orc_asym_grid(const float * wp, int rows, int cols, int group, int nbits, int rem, const float * wt,
                   const float * facs, int ncand, int iters, int refit, float * out_l, float * out_s) {
    const int ng = cols / group;
    const float n = (float) ((1 << nbits) - 1);
    float ones[GMAX];
    for (int i = 0; i < GMAX; i++) ones[i] = 1.0f;
#pragma omp parallel for schedule(dynamic, 4)
    for (int r = 0; r < rows; r++) {
        float q[GMAX], q2[GMAX];
        for (int j = 0; j < ng; j++) {
            const float * g = wp + (size_t) r * cols + (size_t) j * group;
            const float * w = wt ? wt + (size_t) j * group : ones;
            float lo = g[0], hi = g[0], ws = 0.0f;
            for (int i = 0; i < group; i++) {
                if (g[i] < lo) lo = g[i];
                if (g[i] > hi) hi = g[i];
                ws += w[i];
            }
            const float c = (lo + hi) * 0.5f;
            float bl = 0, bs = 0, be = 0;
            for (int k = 0; k < ncand; k++) {
                const float half = (hi - lo) * 0.5f * facs[k];
                float l = c - half;
                float step = fmaxf(2.0f * half, 1e-12f) / n;
                float e = err_of(g, w, group, l, step, n, rem, q);
                if (refit) {
                    for (int it = 0; it < iters; it++) {
                        float qm = 0, gm = 0;
                        for (int i = 0; i < group; i++) { qm = qm + w[i] * q[i]; gm = gm + w[i] * g[i]; }
                        qm /= ws;
                        gm /= ws;
                        float var = 0, cov = 0;
                        for (int i = 0; i < group; i++) {
                            const float dq = q[i] - qm;
                            var = var + (w[i] * dq) * dq;
                            cov = cov + (w[i] * dq) * (g[i] - gm);
                        }
                        float s2 = var > 1e-12f ? cov / fmaxf(var, 1e-12f) : step;
                        s2 = fmaxf(s2, 1e-12f);
                        const float l2 = fmaf(-s2, qm, gm);
                        const float e2 = err_of(g, w, group, l2, s2, n, rem, q2);
                        if (e2 < e) {
                            l = l2; step = s2; e = e2;
                            memcpy(q, q2, sizeof(float) * (size_t) group);
                        }
                    }
                }
                if (k == 0 || e < be) { bl = l; bs = step; be = e; }
            }
            out_l[(size_t) r * ng + j] = bl;
            out_s[(size_t) r * ng + j] = bs;
        }
    }
}

// follows sml/sml-quant.c:101-137 (sml_field_search); dd = c*S + M - g is
// fma(c, S, M) - g, e += dd*dd*w is fma(dd*dd, w, e)
void orc_field_search(const float * w, int rows, int cols, int group, const float * dv, const float * dm,
                      int32_t * q8, int32_t * mq8, int nmax, int hi, int moff, int mmax, const float * wt, int radius) {
    const int ng = cols / group;
    float ones[GMAX];
    for (int i = 0; i < GMAX; i++) ones[i] = 1.0f;
#pragma omp parallel for schedule(dynamic, 4)
    for (int r = 0; r < rows; r++) {
        for (int j = 0; j < ng; j++) {
            const float * g = w + (size_t) r * cols + (size_t) j * group;
            const float * wg = wt ? wt + (size_t) j * group : ones;
            const size_t o = (size_t) r * ng + j;
            const float d = dv[o], m = dm[o];
            const int qs0 = q8[o], qm0 = mq8[o];
            float be = 0;
            int bs = qs0, bm = qm0, first = 1;
            for (int a = -radius; a <= radius; a++) {
                int qs = qs0 + a;
                if (qs < 1) qs = 1;
                if (qs > hi) qs = hi;
                const float S = fmaxf((float) qs * d, 1e-12f);
                for (int b = -radius; b <= radius; b++) {
                    int qm = qm0 + b;
                    if (qm < 0) qm = 0;
                    if (qm > mmax) qm = mmax;
                    const float M = ((float) qm - (float) moff) * m;
                    float e = 0;
                    for (int i = 0; i < group; i++) {
                        float c = rintf((g[i] - M) / S);
                        if (c < 0) c = 0;
                        if (c > (float) nmax) c = (float) nmax;
                        const float dd = fmaf(c, S, M) - g[i];
                        e = fmaf(dd * dd, wg[i], e);
                    }
                    if (first || e < be) { be = e; bs = qs; bm = qm; first = 0; }
                }
            }
            q8[o] = bs;
            mq8[o] = bm;
        }
    }
}

// The candidate range factors: numpy's linspace(0.6, 0.85, max(2, ncand/3))
// then linspace(0.88, 1.04, max(2, ncand - ncand/3)), float64 values
// i*step + start with the end point set exactly, rounded to float32.
// follows tooling/sml_grid_c.py:41-42 (the same list as tooling/sml_quantize.py:180-181)
int orc_grid_facs(int ncand, float * facs) {
    const int n1 = ncand / 3 > 2 ? ncand / 3 : 2, n2 = ncand - ncand / 3 > 2 ? ncand - ncand / 3 : 2;
    const double a[2] = { 0.6, 0.88 }, b[2] = { 0.85, 1.04 };
    const int cnt[2] = { n1, n2 };
    int k = 0;
    for (int s = 0; s < 2; s++) {
        const double step = (b[s] - a[s]) / (double) (cnt[s] - 1);
        for (int i = 0; i < cnt[s]; i++) {
            double v = (double) i * step;
            v = v + a[s];
            if (i == cnt[s] - 1) v = b[s];
            facs[k++] = (float) v;
        }
    }
    return k;
}

// fp16 round trip helpers (RNE), as numpy's astype(np.float16)
static uint16_t h_of(float f) { return orc_f32_to_f16(f); }
static float f_of(uint16_t h) { return orc_f16_to_f32(h); }

// fp16 per superblock of gps groups + a uint8 per group, 8-bit fields.
// Unsigned (steps): d = f16(max/255), q = clip(rint(v/d), 1, 255), eff = q*d;
// signed (mins): d = f16(max|v|/127), q = clip(rint(v/d) + 127, 0, 254),
// eff = (q - 127)*d; a zero d divides as 1e-8. A short last superblock repeats
// its last group (numpy's pad mode "edge").
// follows tooling/sml_quantize.py:320-363 (Quantizer.two_level, bits=8, neg=False)
void orc_two_level(const float * v, int rows, int ng, int gps, int is_signed, uint16_t * d16, uint8_t * q8, float * eff) {
    const int nsb = (ng + gps - 1) / gps;
    for (int r = 0; r < rows; r++) {
        const float * vr = v + (size_t) r * ng;
        for (int s = 0; s < nsb; s++) {
            // numpy's max: NaN wins, otherwise the largest
            float mx = 0.0f;
            for (int k = 0; k < gps; k++) {
                const int g = s * gps + k < ng ? s * gps + k : ng - 1;
                const float x = is_signed ? fabsf(vr[g]) : vr[g];
                if (k == 0 || isnan(x) || (!isnan(mx) && x > mx)) mx = isnan(mx) && k ? mx : x;
            }
            const uint16_t h = h_of(mx / (is_signed ? 127.0f : 255.0f));
            d16[(size_t) r * nsb + s] = h;
            float dv = f_of(h);
            if (dv == 0.0f) dv = 1e-8f;
            for (int k = 0; k < gps && s * gps + k < ng; k++) {
                const int g = s * gps + k;
                float t = rintf(vr[g] / dv);
                uint8_t qv;
                float e;
                if (is_signed) {
                    t = t + 127.0f;
                    t = t < 0.0f ? 0.0f : t > 254.0f ? 254.0f : t;
                    qv = (uint8_t) t;
                    e = ((float) qv - 127.0f) * dv;
                } else {
                    t = t < 1.0f ? 1.0f : t > 255.0f ? 255.0f : t;
                    qv = (uint8_t) t;
                    e = (float) qv * dv;
                }
                q8[(size_t) r * ng + g] = qv;
                eff[(size_t) r * ng + g] = e;
            }
        }
    }
}

// Codes of every weight against the stored (effective) step and min:
// clip(rint((w - M) / max(S, 1e-12)), 0, nmax).
// follows tooling/sml_quantize.py:565-572 (encode)
void orc_requant_codes(const float * wp, int rows, int cols, const float * eff_s, const float * eff_m, int nmax,
                       uint8_t * codes) {
    const int ng = cols / 32;
    for (int r = 0; r < rows; r++)
        for (int i = 0; i < cols; i++) {
            const size_t o = (size_t) r * ng + i / 32;
            const float S = fmaxf(eff_s[o], 1e-12f);
            float c = rintf((wp[(size_t) r * cols + i] - eff_m[o]) / S);
            c = c < 0.0f ? 0.0f : c > (float) nmax ? (float) nmax : c;
            codes[(size_t) r * cols + i] = (uint8_t) c;
        }
}

// The column order of a tensor quantized without calibration activations:
// ascending max |w| over the rows, ties (and NaN keys, which sort last) by
// column index. numpy's argsort (tooling/sml_quantize.py:479) leaves the
// order of equal keys to its sort; this oracle and the GPU fix it as stable.
typedef struct { float k; int i; } colkey;
static int colkey_cmp(const void * a, const void * b) {
    const colkey * x = a, * y = b;
    const int nx = isnan(x->k), ny = isnan(y->k);
    if (nx != ny) return nx - ny;
    if (!nx && x->k != y->k) return x->k < y->k ? -1 : 1;
    return x->i - y->i;
}
void orc_perm_maxabs(const float * w, int rows, int cols, int32_t * perm) {
    colkey * v = malloc((size_t) cols * sizeof *v);
    for (int c = 0; c < cols; c++) { v[c].k = 0.0f; v[c].i = c; }
    for (int c = 0; c < cols; c++) {
        float m = fabsf(w[c]);
        for (int r = 1; r < rows; r++) {
            const float a = fabsf(w[(size_t) r * cols + c]);
            if (a > m || isnan(a)) { if (!isnan(m)) m = a; }
        }
        v[c].k = m;
    }
    qsort(v, (size_t) cols, sizeof *v, colkey_cmp);
    for (int c = 0; c < cols; c++) perm[c] = v[c].i;
    free(v);
}

// A GPTQ (bits 2, 4 or 8) or AWQ (4 bits) tensor dequantized to [rows][cols]
// (rows = outputs) and rounded to fp16, as the unpacker hands it to the
// quantizer: (code - zero) * scale in fp32, then float16 (its safetensors
// writer). GPTQ: qweight [cols/per][rows] along the input, qzeros
// [groups][rows/per] along the output, zero + zero_add (1 for v1 files),
// group of input k = g_idx[k] (NULL: k / group). AWQ (awq = 1): qweight
// [cols][rows/8] along the output in nibble order (0, 4, 1, 5, 2, 6, 3, 7),
// qzeros likewise or NULL for zero 8, group k / group.
// follows tooling/sml_unpack.py:66-76 (_unpack_ints), :84-97 (dequant_gptq),
// :100-118 (dequant_awq), :35-38 (Writer.add: float16)
void orc_unpack_dequant_f16(const int32_t * qweight, const int32_t * qzeros, const uint16_t * scales,
                            const int32_t * g_idx, int rows, int cols, int bits, int group, int zero_add, int awq,
                            float * out) {
    static const int rev[8] = { 0, 4, 1, 5, 2, 6, 3, 7 };
    const int per = 32 / bits;
    const uint32_t mask = (1u << bits) - 1u;
    for (int n = 0; n < rows; n++)
        for (int k = 0; k < cols; k++) {
            const int g = awq || !g_idx ? k / group : g_idx[k];
            uint32_t q, z;
            if (awq) {
                // column n of the unpacked [cols][rows] array is word n/8, nibble rev[n%8]
                q = ((uint32_t) qweight[(size_t) k * (rows / 8) + n / 8] >> (4 * rev[n % 8])) & 15u;
                z = qzeros ? ((uint32_t) qzeros[(size_t) g * (rows / 8) + n / 8] >> (4 * rev[n % 8])) & 15u : 8u;
            } else {
                q = ((uint32_t) qweight[(size_t) (k / per) * rows + n] >> (bits * (k % per))) & mask;
                z = (((uint32_t) qzeros[(size_t) g * (rows / per) + n / per] >> (bits * (n % per))) & mask) + (uint32_t) zero_add;
            }
            const float v = (float) ((int) q - (int) z) * f_of(scales[(size_t) g * rows + n]);
            out[(size_t) n * cols + k] = f_of(h_of(v));
        }
}

// The whole re-quantization of one tensor without calibration feedback: the
// column order (perm_in, or ascending max |w|), the asymmetric grid (20
// candidates, 3 refits), two-level steps and mins, the field search of
// radius `radius` (the quantizer's default 2; 0 skips it) and the codes.
// wt: per-column weights in the permuted order, already normalised, or NULL.
// Out: codes [rows][cols] in permuted order, sd/md [rows][cols/256], sq/mq
// [rows][cols/32], perm [cols]. cols a multiple of 256.
// follows tooling/sml_quantize.py:426-581 (Quantizer.run and encode with no
// activations: asym_grid, two_level twice, field_search, the codes)
void orc_requant(const float * w, int rows, int cols, int nbits, const int32_t * perm_in, const float * wt, int radius,
                 uint8_t * codes, uint16_t * sd, uint8_t * sq, uint16_t * md, uint8_t * mq, int32_t * perm) {
    const int ng = cols / 32, nsb = (ng + 7) / 8, nmax = (1 << nbits) - 1;
    if (perm_in) memcpy(perm, perm_in, (size_t) cols * sizeof(int32_t));
    else orc_perm_maxabs(w, rows, cols, perm);
    float * wp = malloc((size_t) rows * cols * sizeof(float));
    for (int r = 0; r < rows; r++)
        for (int i = 0; i < cols; i++) wp[(size_t) r * cols + i] = w[(size_t) r * cols + perm[i]];
    float facs[64];
    const int nf = orc_grid_facs(20, facs);
    float * mins = malloc((size_t) rows * ng * sizeof(float)), * steps = malloc((size_t) rows * ng * sizeof(float));
    orc_asym_grid(wp, rows, cols, 32, nbits, 0, wt, facs, nf, 3, 1, mins, steps);
    float * es = malloc((size_t) rows * ng * sizeof(float)), * em = malloc((size_t) rows * ng * sizeof(float));
    orc_two_level(steps, rows, ng, 8, 0, sd, sq, es);
    orc_two_level(mins, rows, ng, 8, 1, md, mq, em);
    if (radius) {
        float * dv = malloc((size_t) rows * ng * sizeof(float)), * dm = malloc((size_t) rows * ng * sizeof(float));
        int32_t * q8 = malloc((size_t) rows * ng * sizeof(int32_t)), * m8 = malloc((size_t) rows * ng * sizeof(int32_t));
        for (int r = 0; r < rows; r++)
            for (int g = 0; g < ng; g++) {
                const size_t o = (size_t) r * ng + g;
                dv[o] = f_of(sd[(size_t) r * nsb + g / 8]);
                dm[o] = f_of(md[(size_t) r * nsb + g / 8]);
                q8[o] = sq[o];
                m8[o] = mq[o];
            }
        orc_field_search(wp, rows, cols, 32, dv, dm, q8, m8, nmax, 255, 127, 254, wt, radius);
        for (size_t o = 0; o < (size_t) rows * ng; o++) {
            sq[o] = (uint8_t) q8[o];
            mq[o] = (uint8_t) m8[o];
            es[o] = (float) q8[o] * dv[o];
            em[o] = ((float) m8[o] - 127.0f) * dm[o];
        }
        free(dv); free(dm); free(q8); free(m8);
    }
    orc_requant_codes(wp, rows, cols, es, em, nmax, codes);
    free(wp); free(mins); free(steps); free(es); free(em);
}
