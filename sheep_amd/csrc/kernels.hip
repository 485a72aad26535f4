// gfx950 (MI355X) kernels for the quantized decode path. Compiled to a code
// object (--genco) and loaded by the C host with hipModuleLoadData; every
// kernel is extern "C" and takes one argument block from kargs.h.
//
// Wave64 throughout. The GEMV's unit of work is a quad: 128 consecutive
// weights of one row = 4 whole groups of 32, which in the reference's FLAT
// planes is 64 contiguous bytes of the nibble plane (groups 4q, 4q+1 as the
// low/high nibbles of bytes 0-31, groups 4q+2, 4q+3 of bytes 32-63;
// sml/sml-kernel.c:2140-2156), one 32-byte pack of a 2-bit plane and 16
// bytes of a 1-bit plane. One lane streams a quad with 128-bit loads,
// dots it against the int8 activation held in LDS with v_dot4, and applies
// the reference's per-group float epilogue (sml/sml-kernel.c:2054-2063):
// step*(s*dot) + min*(s*sum).
#include <hip/hip_runtime.h>
#include "kargs.h"

#define WAVE 64

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned int v4u __attribute__((ext_vector_type(4)));
typedef unsigned int v2u __attribute__((ext_vector_type(2)));

// Global-memory views of device pointers. A pointer read from a table in
// device memory (expert matrices, KV slots) or selected at run time is
// generic to the compiler, and loads through it become flat loads. A flat
// load counts against the LDS/scalar wait counter as well as the vector
// one, so every LDS or scalar-load wait after it also waits for it, and the
// vector waits can no longer be partial: a kernel that overlaps its weight
// or KV stream with LDS work then runs serially. Every such pointer here
// points to global memory.
#define GLOBAL __attribute__((address_space(1)))
template <typename T> __device__ __forceinline__ T gld(const void * p) { return *(const GLOBAL T *) p; }

// The greedy pick's order: the larger value, the lower index on a tie; NaN is
// never taken (the reference's loop, sml/sml-run.c:3539-3544).
__device__ __forceinline__ void amax_take(float v, int i, float & bv, int & bi) {
    if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
}

// Marks a loaded value as used here. Arithmetic on a loop-invariant load is
// otherwise free to move ahead of the loop, and its wait for the load then
// comes before loads the source issues earlier (the GEMV's weights).
__device__ __forceinline__ void pin(float & v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void pin(int & v) { asm volatile("" : "+v"(v)); }

__device__ __forceinline__ float h2f(uint16_t h) { return (float) __builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16) f); }

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

// Butterflies inside a 16-lane DPP row (quad_perm xor 1, xor 2, then the
// half-row and row mirrors): every lane of the row ends with the row's result.
// A swizzle (xor 16) extends them to 32 lanes.
template <int CTRL> __device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
template <int CTRL> __device__ __forceinline__ int dpp_i(int v) { return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false); }
// Inclusive prefix sums over the 64 lanes: Hillis-Steele inside each
// 16-lane row (row_shr 1, 2, 4, 8; lanes shifted in from outside the row
// add 0), then each row adds the totals of the rows below it.
__device__ __forceinline__ int wave_scan_i(int v) {
    v += dpp_i<0x111>(v); v += dpp_i<0x112>(v); v += dpp_i<0x114>(v); v += dpp_i<0x118>(v);
    const int r0 = __builtin_amdgcn_readlane(v, 15), r1 = __builtin_amdgcn_readlane(v, 31);
    const int r2 = __builtin_amdgcn_readlane(v, 47), row = (threadIdx.x & 63) >> 4;
    return v + (row == 0 ? 0 : row == 1 ? r0 : row == 2 ? r0 + r1 : r0 + r1 + r2);
}
__device__ __forceinline__ float wave_scan_f(float v) {
    v += dpp_f<0x111>(v); v += dpp_f<0x112>(v); v += dpp_f<0x114>(v); v += dpp_f<0x118>(v);
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 15));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 31));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 47));
    const int row = (threadIdx.x & 63) >> 4;
    return v + (row == 0 ? 0.0f : row == 1 ? r0 : row == 2 ? r0 + r1 : (r0 + r1) + r2);
}
__device__ __forceinline__ float sum16(float v) {
    v += dpp_f<0xB1>(v); v += dpp_f<0x4E>(v); v += dpp_f<0x141>(v); v += dpp_f<0x140>(v);
    return v;
}
__device__ __forceinline__ float max16(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v)); v = fmaxf(v, dpp_f<0x4E>(v)); v = fmaxf(v, dpp_f<0x141>(v)); v = fmaxf(v, dpp_f<0x140>(v));
    return v;
}
__device__ __forceinline__ int isum16(int v) {
    v += dpp_i<0xB1>(v); v += dpp_i<0x4E>(v); v += dpp_i<0x141>(v); v += dpp_i<0x140>(v);
    return v;
}
// xor 16 within 32 lanes (ds_swizzle bit mode: and 0x1F, xor 0x10)
__device__ __forceinline__ float swz16_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
}
__device__ __forceinline__ float sum32(float v) { v = sum16(v); return v + swz16_f(v); }
__device__ __forceinline__ float max32(float v) { v = max16(v); return fmaxf(v, swz16_f(v)); }
__device__ __forceinline__ int isum32(int v) { v = isum16(v); return v + __builtin_amdgcn_ds_swizzle(v, 0x401F); }

__device__ __forceinline__ int dot4(unsigned a, int b, int c) { return __builtin_amdgcn_sdot4((int) a, b, c, false); }

// 4 bits (one per column) -> 4 bytes of 0/1
__device__ __forceinline__ unsigned bits4_to_bytes(unsigned nib) { return (nib * 0x00204081u) & 0x01010101u; }

// ---------------------------------------------------------------- chunks
//
// A chunk is 16 bytes of a row's nibble plane: columns 16*(c&1)..+15 of the
// group pair (c&~1, c|1) -- byte i's low nibble belongs to the first group,
// its high nibble to the second (the FLAT layout, sml/sml-kernel.c:2140-2156).
// Lane c of a row loads chunk c, so 64 lanes read 1 KB of contiguous bytes
// per instruction; the other planes' bytes for the same weights are equally
// contiguous across lanes (a 2-bit pack serves two lanes, a 1-bit word pair
// serves a lane pair). Plane orders per width follow
// tooling/sml_quantize.py:104-106: Q2 [2], Q3 [2,1], Q4 [4], Q5 [4,1],
// Q6 [2,4] (the 2-bit plane holds bits 4-5), Q7 [4,2,1], Q8 [4,4].
template <int NB> struct Planes {
    static constexpr bool N4 = NB == 4 || NB == 5 || NB == 6 || NB == 7 || NB == 8;
    static constexpr bool N2 = NB == 2 || NB == 3 || NB == 6 || NB == 7;
    static constexpr bool N1 = NB == 3 || NB == 5 || NB == 7;
    static constexpr int P4 = NB == 6 ? 1 : 0;
    static constexpr int P2 = NB == 7 ? 1 : 0;
    static constexpr int P1 = NB == 7 ? 2 : 1;
    // bytes of each plane per row for `cols` weights
    static __device__ __forceinline__ size_t b4(int cols) { return (size_t) cols / 2; }
    static __device__ __forceinline__ size_t b2(int cols) { return (size_t) cols / 4; }
    static __device__ __forceinline__ size_t b1(int cols) { return (size_t) cols / 8; }
};

template <bool NT, typename T>
__device__ __forceinline__ T ld(const T * p) {
    const GLOBAL T * g = (const GLOBAL T *) p;
    if constexpr (NT) return __builtin_nontemporal_load(g);
    else return *g;
}

template <int NB> struct ChunkW {
    v4u n4;                       // nibble plane word (or zeros)
    v4u h4;                       // Q8 high nibbles
    v4u t2;                       // 2-bit pack half
    v2u o1;                       // 1-bit words of the group pair
};

// Chunk c of one row: pl[] are the planes' bases (uniform), ro[] the row's
// byte offset in each plane. Offsets are 32-bit so the loads address as
// uniform base + per-lane offset, which keeps one VGPR per address.
template <int NB, bool NT>
__device__ __forceinline__ void load_chunk(ChunkW<NB> & w, const uint8_t * const * pl, const uint32_t * ro, int c) {
    using P = Planes<NB>;
    if constexpr (P::N4) w.n4 = ld<NT>((const v4u *) (pl[P::P4] + (ro[P::P4] + (uint32_t) c * 16u)));
    if constexpr (NB == 8) w.h4 = ld<NT>((const v4u *) (pl[1] + (ro[1] + (uint32_t) c * 16u)));
    if constexpr (P::N2) w.t2 = ld<NT>((const v4u *) (pl[P::P2] + (ro[P::P2] + (uint32_t) (c >> 2) * 32u + (uint32_t) (c & 1) * 16u)));
    if constexpr (P::N1) w.o1 = ld<NT>((const v2u *) (pl[P::P1] + (ro[P::P1] + (uint32_t) (c >> 1) * 8u)));
}

// partial dots of chunk c over its 16 columns: da for group c&~1 against
// xa, db for group c|1 against xb
template <int NB>
__device__ __forceinline__ void chunk_dots(const ChunkW<NB> & w, int c, const v4i xa, const v4i xb, int & da, int & db) {
    using P = Planes<NB>;
    v4u ca = {0u, 0u, 0u, 0u}, cb = {0u, 0u, 0u, 0u};
    int sh = 0;
    if constexpr (P::N4) { ca = w.n4 & 0x0F0F0F0Fu; cb = (w.n4 >> 4u) & 0x0F0F0F0Fu; sh = 4; }
    if constexpr (P::N2) {
        const unsigned k = 2u * (unsigned) (c & 2);          // bit-plane of group c&~1 within its pack
        const v4u ea = (w.t2 >> k) & 0x03030303u, eb = (w.t2 >> (k + 2u)) & 0x03030303u;
        if constexpr (P::N4) { ca |= ea << 4u; cb |= eb << 4u; sh = 6; }
        else { ca = ea; cb = eb; sh = 2; }
    }
    if constexpr (P::N1) {
        const unsigned wa = w.o1.x >> (16 * (c & 1)), wb = w.o1.y >> (16 * (c & 1));
        #pragma unroll
        for (int i = 0; i < 4; i++) {
            ca[i] |= bits4_to_bytes((wa >> (4 * i)) & 15u) << sh;
            cb[i] |= bits4_to_bytes((wb >> (4 * i)) & 15u) << sh;
        }
    }
    int a = 0, b = 0;
    #pragma unroll
    for (int i = 0; i < 4; i++) { a = dot4(ca[i], xa[i], a); b = dot4(cb[i], xb[i], b); }
    if constexpr (NB == 8) {
        int ha = 0, hb = 0;
        #pragma unroll
        for (int i = 0; i < 4; i++) {
            ha = dot4(w.h4[i] & 0x0F0F0F0Fu, xa[i], ha);
            hb = dot4((w.h4[i] >> 4u) & 0x0F0F0F0Fu, xb[i], hb);
        }
        a += ha << 4;
        b += hb << 4;
    }
    da = a; db = b;
}

// lane i <-> lane i^1 (DPP quad_perm [1,0,3,2])
__device__ __forceinline__ int pair_swap(int v) { return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false); }

// ---------------------------------------------------------------- GEMV
//
// One launch covers up to three matrices that read the same activation (the
// reference's shared-activation groups, sml/sml-run.c:924-1121), or gate and
// up paired for the fused SwiGLU. A wave owns RB rows and streams them whole:
// lane c takes chunks c, c+64, ... (NI per lane, all loaded before any is
// used), so every load instruction is 1 KB of contiguous bytes per row and a
// 34 MB matrix is in flight at once. The activation is staged in LDS by the
// workgroup, its global loads issued ahead of the weights' (loads return in
// order), as int8 codes and per-group (scale, scale*sum).
// Sum over the wave with DPP: row shifts within each 16-lane row, then the
// row broadcasts; lane 63 ends up with the total.
__device__ __forceinline__ float wave_sum_dpp(float v) {
    int x = __builtin_bit_cast(int, v);
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, true)); x = __builtin_bit_cast(int, v);
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, true)); x = __builtin_bit_cast(int, v);
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, true)); x = __builtin_bit_cast(int, v);
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, true)); x = __builtin_bit_cast(int, v);
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false)); x = __builtin_bit_cast(int, v);
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false));
    return v;
}

// Max / sum over aligned groups of 8 lanes (quad butterflies, then the half-row mirror)
__device__ __forceinline__ float max8(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v)); v = fmaxf(v, dpp_f<0x4E>(v)); return fmaxf(v, dpp_f<0x141>(v));
}
__device__ __forceinline__ int isum8(int v) { v += dpp_i<0xB1>(v); v += dpp_i<0x4E>(v); return v + dpp_i<0x141>(v); }

// One activation code: lrintf(v * is) clamped to +-127, where an out-of-range
// or NaN product converts to INT_MIN as the reference's x86 build does
// (sml/sml-kernel.c:86-106), so it clamps to -127.
__device__ __forceinline__ int quant1(float v, float is) {
    const float r = __builtin_rintf(v * is);
    int t = (r >= -2147483648.0f && r < 2147483648.0f) ? (int) r : (int) 0x80000000u;
    return t > 127 ? 127 : t < -127 ? -127 : t;
}

// SiLU as the reference's x86 build computes it (sml_exp_ps + silu_mul,
// sml/sml-run.c:393-426): the argument clamped to [-88, 88], f = x*log2(e),
// r = f rounded half-even, 2^(f-r) by a degree-5 Horner chain of FMAs, and
// 1 + p*2^r folded into one FMA (how that build's compiler contracts it);
// then g / d. Contraction is off so f and f - r round as written.
__device__ __forceinline__ float silu_ref(float g) {
    #pragma clang fp contract(off)
    float x = 0.0f - g;
    x = fminf(fmaxf(x, -88.0f), 88.0f);
    const float f = x * 1.44269504088896341f;
    const float r = __builtin_rintf(f);
    const float t = f - r;
    float p = __builtin_fmaf(1.3697664e-3f, t, 8.3013611e-3f);
    p = __builtin_fmaf(p, t, 5.5826318e-2f);
    p = __builtin_fmaf(p, t, 2.4022652e-1f);
    p = __builtin_fmaf(p, t, 6.9314718e-1f);
    p = __builtin_fmaf(p, t, 1.0f);
    const float sc = __builtin_bit_cast(float, ((int) r + 127) << 23);
    return g / __builtin_fmaf(p, sc, 1.0f);
}

// expf of the C library the reference runs on (glibc 2.35 on x86-64 with FMA),
// restated from its published algorithm (ARM optimized-routines expf, in
// glibc since 2.27): x*32/ln2 = k + r in double (k rounded half-even through
// the 1.5*2^52 shift, both products fused), 2^(k/32) from a 32-entry table of
// 2^(i/32) with the exponent folded in, 2^(r/32) by a cubic, then one
// rounding to float. Compared on the CPU over every float <= 0 against the
// library, it gives the same bits on all of them; only x <= 0 is used here
// (softmax and routing weights), where anything below -103.97 is 0.
// 2^(i/32) as double bits, less i << 47 (the exponent step of the index)
__constant__ unsigned long long EXPF_TAB[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull };

// tab: the 32-entry table above, or a copy of it (in LDS: a kernel that
// streams global loads keeps its waits for them apart from the lookups)
__device__ __forceinline__ float expf_tab(float x, const unsigned long long * tab) {
    #pragma clang fp contract(off)
    if (x < -0x1.9fe368p6f) return 0.0f;
    const double C0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32, C1 = 0x1.ebfce50fac4f3p-3 / 32 / 32,
                 C2 = 0x1.62e42ff0c52d6p-1 / 32, InvLn2N = 0x1.71547652b82fep+0 * 32, Shift = 0x1.8p+52;
    const double xd = (double) x;
    double kd = __builtin_fma(InvLn2N, xd, Shift);
    const unsigned long long ki = __builtin_bit_cast(unsigned long long, kd);
    kd -= Shift;
    const double r = __builtin_fma(InvLn2N, xd, -kd);
    const double s = __builtin_bit_cast(double, tab[ki % 32] + (ki << 47));
    const double z = __builtin_fma(C0, r, C1), r2 = r * r;
    double y = __builtin_fma(C2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    return (float) (y * s);
}
__device__ __forceinline__ float expf_ref(float x) { return expf_tab(x, EXPF_TAB); }

// Order LDS traffic among the lanes of one wave (its LDS operations execute
// in order; this keeps the compiler from moving them across the point).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The sum of squares as the reference build computes it (sml/sml-run.c:
// 147-152, a serial loop its compiler turns into double FMAs): one lane, in
// order. Loads run ahead of the dependent chain in blocks of 16. x is in
// global memory or in LDS (generic loads: this is the rare fallback of the
// checked parallel sum below).
__device__ __noinline__ double serial_ss(const float * x, int n) {
    double ss = 0.0;
    int i = 0;
    for (; i + 16 <= n; i += 16) {
        float v[16];
        #pragma unroll
        for (int j = 0; j < 16; j++) v[j] = x[i + j];
        #pragma unroll
        for (int j = 0; j < 16; j++) ss = __builtin_fma((double) v[j], (double) v[j], ss);
    }
    for (; i < n; i++) { const float v = x[i]; ss = __builtin_fma((double) v, (double) v, ss); }
    return ss;
}

// float(ss/n) of the serial chain above, from a sum of the same squares taken
// in any order. Every square is exact in double (24-bit mantissas), all are
// nonnegative, so each order's sum lies within (n-1)*2^-53*(1+2^-30) of the
// exact sum, relatively: the serial and the given sum differ by less than
// d = 4*(n+4)*2^-53*s, with a margin for the rounding of d itself. Division
// by n and the float conversion are monotone, so when s-d and s+d give the
// same float that float is the serial chain's; it fails for about one input
// in 10^4 (a rounding boundary inside the window) and for inf/NaN sums, and
// the caller then runs the chain.
__device__ __forceinline__ bool ss_mean_alike(double s, int n, float & out) {
    const double d = s * ((double) (4 * (n + 4)) * 0x1p-53);
    const float lo = (float) ((s - d) / (double) n), hi = (float) ((s + d) / (double) n);
    out = lo;
    return lo == hi;
}

// Fused activation prologue: RMSNorm (double sum of squares, out = x*sc*w,
// sml/sml-run.c:147-152), gather through perm, and the per-32 quantization
// (sml/sml-kernel.c:86-106) of the whole input vector, into the workgroup's
// LDS copy (lq: int8 codes, lsc: per group (s, s*sum)). Thread t holds the
// float4 words t + k*WG (loaded before the weights); 8 consecutive threads
// hold one group of 32. The arithmetic is the normq kernels', so the codes,
// scales and sums are theirs bit for bit.
// EXN: the norm in exact mode, the serial chain's float(ss/n) (ss_mean_alike,
// with the chain itself over x in global memory as its rare fallback).
template <int WG, int FK, bool EXN = false>
__device__ __forceinline__ void fused_act(const sml_kgemv & a, const float4 (&fx)[FK], const float4 (&fw)[FK],
                                          const int4 (&fp)[FK], int8_t * lq, float2 * lsc, float * nrm, double * red) {
    const int n = a.cols, tid = threadIdx.x, n4 = n / 4;
    float sc = 1.0f;
    if (a.norm_w) {
        double ss = 0.0;
        #pragma unroll
        for (int k = 0; k < FK; k++)
            if (tid + k * WG < n4) {
                const float4 v = fx[k];
                ss += (double) v.x * v.x + (double) v.y * v.y + (double) v.z * v.z + (double) v.w * v.w;
            }
        #pragma unroll
        for (int o = 32; o; o >>= 1) ss += __shfl_xor(ss, o);
        if ((tid & 63) == 0) red[tid >> 6] = ss;
        __syncthreads();
        double tot = 0.0;
        #pragma unroll
        for (int w = 0; w < WG / 64; w++) tot += red[w];
        float msq = (float) (tot / (double) n);
        if (EXN && !ss_mean_alike(tot, n, msq)) {
            __syncthreads();                    // every thread has read red (the same decision in all)
            if (tid == 0) red[0] = serial_ss(a.x, n);
            __syncthreads();
            msq = (float) (red[0] / (double) n);
        }
        sc = 1.0f / sqrtf(msq + a.eps);
    }
    float v[FK][4];
    #pragma unroll
    for (int k = 0; k < FK; k++) {
        v[k][0] = fx[k].x; v[k][1] = fx[k].y; v[k][2] = fx[k].z; v[k][3] = fx[k].w;
        if (a.norm_w) {
            v[k][0] = v[k][0] * sc * fw[k].x; v[k][1] = v[k][1] * sc * fw[k].y;
            v[k][2] = v[k][2] * sc * fw[k].z; v[k][3] = v[k][3] * sc * fw[k].w;
        }
    }
    if (a.perm) {
        #pragma unroll
        for (int k = 0; k < FK; k++) {
            const int f = tid + k * WG;
            if (f < n4) *(float4 *) (nrm + 4 * f) = make_float4(v[k][0], v[k][1], v[k][2], v[k][3]);
        }
        __syncthreads();
        #pragma unroll
        for (int k = 0; k < FK; k++)
            if (tid + k * WG < n4) {
                v[k][0] = nrm[fp[k].x]; v[k][1] = nrm[fp[k].y]; v[k][2] = nrm[fp[k].z]; v[k][3] = nrm[fp[k].w];
            }
    }
    #pragma unroll
    for (int k = 0; k < FK; k++) {
        const int f = tid + k * WG;
        if (f >= n4) continue;                  // whole 8-lane groups drop out together (n % 32 == 0)
        const float am = max8(fmaxf(fmaxf(fabsf(v[k][0]), fabsf(v[k][1])), fmaxf(fabsf(v[k][2]), fabsf(v[k][3]))));
        const float s = am / 127.0f;
        const float is = s > 0.0f ? 1.0f / s : 0.0f;
        const int t0 = quant1(v[k][0], is), t1 = quant1(v[k][1], is), t2 = quant1(v[k][2], is), t3 = quant1(v[k][3], is);
        const int sum = isum8(t0 + t1 + t2 + t3);
        ((int *) lq)[f] = (t0 & 0xFF) | (t1 & 0xFF) << 8 | (t2 & 0xFF) << 16 | (int) ((unsigned) t3 << 24);
        if ((tid & 7) == 0) lsc[f >> 3] = make_float2(s, s * (float) sum);
    }
}

// The GEMV body. One wave owns RB output rows (SW: RB/2 gate/up row pairs);
// lane c of the wave streams chunk c, c+64, ... of each row. The argument
// block is only ever read at fixed offsets: a run-time index into it makes
// the compiler copy it to scratch or read it with vector loads that wait
// for every load already in flight (the activation prefetch included).
//
// Chunks past a row's end read the row's last chunk (a broadcast of bytes
// already fetched) and contribute nothing because their activation scale is
// taken as zero; rows past the end read row 0 and are never stored.
// Sum over aligned segments of LPR lanes (16, 32 or 64): the row shifts give
// an inclusive scan inside each 16-lane DPP row, the row broadcasts carry it
// across rows. The segment's last lane ends up with its total.
template <int LPR>
__device__ __forceinline__ float seg_sum(float v) {
    int x = __builtin_bit_cast(int, v);
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, true)); x = __builtin_bit_cast(int, v);
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, true)); x = __builtin_bit_cast(int, v);
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, true)); x = __builtin_bit_cast(int, v);
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, true)); x = __builtin_bit_cast(int, v);
    if constexpr (LPR >= 32) {
        v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false)); x = __builtin_bit_cast(int, v);
    }
    if constexpr (LPR == 64) v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false));
    return v;
}

// blk: the workgroup's row block (blockIdx.x, or each block a persistent
// workgroup takes in turn); first: the activation is not yet in LDS.
// TS: record the row block's timeline (a.ts) into tsh[0..3] (LDS of the
// caller), thread 0's view: entry, the first weight word of the first pass,
// all of the first pass's weights, all of the last pass's.
template <int NB, int RB, int NI, int WG, bool NT, int AM, bool SW, bool HQ, int LPR = 64, bool EX = false,
          bool TS = false>
__device__ void gemv_body(const sml_kgemv & a, int blk = blockIdx.x, bool first = true,
                          unsigned long long * tsh = nullptr) {
    extern __shared__ __align__(16) uint8_t lds[];
    const int n = a.cols, ng = n / 32, ns = (ng + 7) / 8;
    if constexpr (TS) { if (threadIdx.x == 0) tsh[0] = __builtin_amdgcn_s_memrealtime(); }
    int8_t * lq = (int8_t *) lds;
    float2 * lsc = (float2 *) (lds + n);
    const int tid = threadIdx.x, lane = tid & (WAVE - 1);
    // LPR lanes stream one row; a wave holds SUB = 64/LPR rows per row slot
    constexpr int SUB = WAVE / LPR;
    const int l = lane % LPR, u = lane / LPR;
    constexpr int RPW = (SW ? RB / 2 : RB) * SUB;  // output rows per wave
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int row0 = (blk * (WG / WAVE) + wave) * RPW;

    // 1. activation loads (L2-resident, issued first)
    constexpr int SQ = AM == 0 ? 4 : 1, SG = AM == 0 ? 2 : 1;   // staged words per thread per round
    v4i sq_[SQ];
    int sg_i[SG];
    float sg_s[SG];
    int32_t sg_u[SG];
    const int nq16 = n / 16;
    // fused prologue: float4 words of x, norm_w and perm per thread
    constexpr int FK = AM == 0 ? 1 : (WG >= 1024 ? 1 : WG >= 512 ? 2 : 4);
    float4 fx[FK], fw[FK];
    int4 fp[FK];
    if constexpr (AM == 0) {
        #pragma unroll
        for (int k = 0; k < SQ; k++) { const int i = tid + k * WG; if (first && i < nq16) sq_[k] = ((const v4i *) a.q)[i]; }
        #pragma unroll
        for (int k = 0; k < SG; k++) {
            const int i = tid + k * WG;
            sg_i[k] = i;
            if (first && i < ng) { sg_s[k] = a.scale[i]; sg_u[k] = a.sums[i]; }
        }
    } else {
        #pragma unroll
        for (int k = 0; k < FK; k++) {
            const int f = tid + k * WG;
            fx[k] = make_float4(0.f, 0.f, 0.f, 0.f); fw[k] = fx[k]; fp[k] = make_int4(0, 0, 0, 0);
            if (first && f < n / 4) {
                fx[k] = ((const float4 *) a.x)[f];
                if (a.norm_w) fw[k] = ((const float4 *) a.norm_w)[f];
                if (a.perm) fp[k] = ((const int4 *) a.perm)[f];
            }
        }
    }

    // 2. this wave's rows: uniform plane and field bases per row slot, and
    // each lane's 32-bit row offsets (the host keeps every plane under 4 GB)
    using P = Planes<NB>;
    const uint8_t * pl[RB][3];
    uint32_t ro[RB][3];
    const uint8_t * fqb[RB];          // (sq, mq) pairs as one 16-bit word per group
    const uint8_t * fdb[RB];          // (sd, md) pairs as one 32-bit word per superblock
    uint32_t fqo[RB], fdo[RB];
    int orow[RB];
    bool valid[RB];
    #pragma unroll
    for (int s = 0; s < RB; s++) {
        const int grow = row0 + (SW ? (s >> 1) : s) * SUB + u;
        orow[s] = grow;
        valid[s] = grow < a.total_rows;
        const sml_kmat & m = (SW && (s & 1)) ? a.m[1] : a.m[0];
        const uint32_t r = (uint32_t) (valid[s] ? grow : 0);
        pl[s][0] = m.plane[0]; pl[s][1] = m.plane[1]; pl[s][2] = m.plane[2];
        ro[s][0] = ro[s][1] = ro[s][2] = 0;
        if constexpr (P::N4) ro[s][P::P4] = r * (uint32_t) P::b4(n);
        if constexpr (NB == 8) ro[s][1] = r * (uint32_t) P::b4(n);
        if constexpr (P::N2) ro[s][P::P2] = r * (uint32_t) P::b2(n);
        if constexpr (P::N1) ro[s][P::P1] = r * (uint32_t) P::b1(n);
        fqb[s] = m.sqmq;
        fdb[s] = (const uint8_t *) m.sdmd;
        fqo[s] = r * (uint32_t) ng * 2u;
        fdo[s] = r * (uint32_t) ns * 4u;
    }

    float acc[RB];
    #pragma unroll
    for (int s = 0; s < RB; s++) acc[s] = 0.0f;
    // EX: the reference's float order (sml/sml-kernel.c:572-727,836-866).
    // Every group's two products go through LDS to the lane that owns the
    // group's position in a superblock: lane 8*rw + j of the wave runs row
    // rw's chain j, v_j = fma(wsc, s*dot, v_j); v_j = fma(wmin, s*sum, v_j)
    // over the superblocks in order (cm; ct for a trailing half superblock,
    // whose four lanes the reference keeps apart and adds last).
    // (with the fused prologue the exchange buffer takes the LDS of the
    // prologue's gather buffer, which is dead once the activation is staged)
    const int nblk8 = (ng / 8) * 8;
    float4 * exb = nullptr;
    float * ext = nullptr;
    float cm = 0.0f, ct = 0.0f;
    if constexpr (EX) {
        const size_t base = ((size_t) n + 8u * (size_t) ng + 15u) & ~(size_t) 15u;
        exb = (float4 *) (lds + base) + (size_t) wave * (NI * RB * 64);
        ext = (float *) (lds + base + (size_t) (WG / 64) * NI * RB * 64 * 16) + wave * (RB * SUB);
    }
    bool staged = !first;
    using CW = ChunkW<NB>;
    // 3. every weight load of this lane for NI chunks of RB rows, with no
    // branches; chunks past the row's end read its last chunk again
    auto load_pass = [&](int c0, CW (&w)[NI][RB], uint32_t (&fqv)[NI][RB], uint32_t (&fdv)[NI][RB]) {
        #pragma unroll
        for (int i = 0; i < NI; i++) {
            const int c = c0 + i * LPR + l;
            const int cl = c < ng ? c : ng - 1;
            #pragma unroll
            for (int s = 0; s < RB; s++) {
                load_chunk<NB, NT>(w[i][s], pl[s], ro[s], cl);
                fqv[i][s] = gld<uint16_t>(fqb[s] + (fqo[s] + (uint32_t) cl * 2u));
                fdv[i][s] = gld<uint32_t>(fdb[s] + (fdo[s] + (uint32_t) (cl >> 3) * 4u));
            }
        }
    };
    auto stage = [&]() {
        if (!staged) {
            if constexpr (AM == 1) {
                // 4'. the activation computed from x into LDS (the gather
                // buffer starts 16-byte aligned after the codes and fields)
                __shared__ double red[WG / 64];
                #pragma unroll
                for (int k = 0; k < FK; k++) {
                    pin(fx[k].x); pin(fx[k].y); pin(fx[k].z); pin(fx[k].w);
                    pin(fw[k].x); pin(fw[k].y); pin(fw[k].z); pin(fw[k].w);
                    pin(fp[k].x); pin(fp[k].y); pin(fp[k].z); pin(fp[k].w);
                }
                fused_act<WG, FK, EX>(a, fx, fw, fp, lq, lsc, (float *) (lds + ((n + 8 * ng + 15) & ~15)), red);
            } else {
                // 4. activation into LDS (waits only for the activation loads)
                #pragma unroll
                for (int k = 0; k < SG; k++) { pin(sg_s[k]); pin(sg_u[k]); }
                #pragma unroll
                for (int k = 0; k < SQ; k++) { const int idx = tid + k * WG; if (idx < nq16) ((v4i *) lq)[idx] = sq_[k]; }
                #pragma unroll
                for (int k = 0; k < SG; k++) if (sg_i[k] < ng) lsc[sg_i[k]] = make_float2(sg_s[k], sg_s[k] * (float) sg_u[k]);
                // widths beyond one round of staging
                for (int idx = tid + SQ * WG; idx < nq16; idx += WG) ((v4i *) lq)[idx] = ((const v4i *) a.q)[idx];
                for (int g = tid + SG * WG; g < ng; g += WG) lsc[g] = make_float2(a.scale[g], a.scale[g] * (float) a.sums[g]);
            }
            __syncthreads();
            staged = true;
        }
    };
    auto compute_pass = [&](int c0, const CW (&w)[NI][RB], const uint32_t (&fqv)[NI][RB],
                            const uint32_t (&fdv)[NI][RB]) {
        // 5. dots and the per-group epilogue; lane c ends up owning group c
        #pragma unroll
        for (int i = 0; i < NI; i++) {
            const int c = c0 + i * LPR + l;
            const bool live = c < ng;                     // the pair (c&~1, c|1) is live or dead as a whole
            const int cc = live ? c : ng - 1;             // keep LDS reads in range
            const int off = 32 * (cc & ~1) + 16 * (cc & 1);
            const v4i xa = *(const v4i *) (lq + off);
            const v4i xb = *(const v4i *) (lq + off + 32);
            float2 sc = lsc[cc];
            if (!live) sc = make_float2(0.0f, 0.0f);
            const int odd = c & 1;
            #pragma unroll
            for (int s = 0; s < RB; s++) {
                int da, db;
                chunk_dots<NB>(w[i][s], c, xa, xb, da, db);
                const int keep = odd ? db : da, send = odd ? da : db;
                const int dot = keep + pair_swap(send);
                const uint32_t f = fqv[i][s], d2 = fdv[i][s];
                const float wsc = h2f((uint16_t) (d2 & 0xFFFFu)) * (float) (f & 0xFFu);
                const float wmn = h2f((uint16_t) (d2 >> 16)) * ((float) (f >> 8) - 127.0f);
                if constexpr (EX) {
                    exb[(i * RB + s) * 64 + u * LPR + l] = make_float4(wsc, sc.x * (float) dot, wmn, sc.y);
                } else {
                    acc[s] += wsc * (sc.x * (float) dot);
                    acc[s] += wmn * sc.y;
                }
            }
        }
        if constexpr (EX) {
            wave_lds_sync();
            const int rw = lane >> 3, j = lane & 7;
            if (rw < RB * SUB) {
                const int s = rw / SUB, uu = rw % SUB;
                #pragma unroll
                for (int i = 0; i < NI; i++) {
                    #pragma unroll
                    for (int t = 0; t < LPR / 8; t++) {
                        const int g = c0 + i * LPR + 8 * t + j;
                        if (g < ng) {
                            const float4 w4 = exb[(i * RB + s) * 64 + uu * LPR + 8 * t + j];
                            if (g < nblk8) { cm = __builtin_fmaf(w4.x, w4.y, cm); cm = __builtin_fmaf(w4.z, w4.w, cm); }
                            else { ct = __builtin_fmaf(w4.x, w4.y, ct); ct = __builtin_fmaf(w4.z, w4.w, ct); }
                        }
                    }
                }
            }
            wave_lds_sync();
        }
    };
    // (issuing the next pass's loads before this pass's dots, pinned there
    // with a scheduling barrier, measured slower: 7.5 -> 9.4 us at 4096 x 14336)
    for (int c0 = 0; c0 < ng; c0 += LPR * NI) {
        CW w[NI][RB];
        uint32_t fqv[NI][RB], fdv[NI][RB];
        load_pass(c0, w, fqv, fdv);
        if constexpr (TS) {
            // loads return in order: all but the pass's other 3*NI*RB - 1
            // weight loads (Q4: a code word and two field words per chunk
            // and row) have returned once the first code word has
            static_assert(NB == 4 && 3 * NI * RB - 1 < 64, "the timeline kernel counts Q4 loads");
            constexpr int W1 = 3 * NI * RB - 1;
            __builtin_amdgcn_s_waitcnt((W1 & 15) | ((W1 >> 4) << 14) | (7 << 4) | (15 << 8));
            if (c0 == 0 && threadIdx.x == 0) tsh[1] = __builtin_amdgcn_s_memrealtime();
        }
        stage();
        if constexpr (TS) {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            if (threadIdx.x == 0) tsh[c0 == 0 ? 2 : 3] = __builtin_amdgcn_s_memrealtime();
        }
        compute_pass(c0, w, fqv, fdv);
    }
    if constexpr (EX) {
        // fold each row's 8 lanes as the reference does: ((v0+v4)+(v1+v5)) +
        // ((v2+v6)+(v3+v7)), then the trailing four (t0+t1)+(t2+t3), added last
        float v = cm + dpp_f<0x104>(cm);              // lanes j < 4: v_j + v_(j+4)
        v = v + dpp_f<0xB1>(v);                        // lanes 0, 2: s0+s1, s2+s3
        v = v + dpp_f<0x4E>(v);                        // lane 0: (s0+s1)+(s2+s3)
        if (ng != nblk8) {
            float w = ct + dpp_f<0xB1>(ct);
            w = w + dpp_f<0x4E>(w);
            v = v + w;
        }
        const int rw = lane >> 3;
        if ((lane & 7) == 0 && rw < RB * SUB) ext[rw] = v;
        wave_lds_sync();
        #pragma unroll
        for (int s = 0; s < RB; s++) acc[s] = ext[s * SUB + u];
    }
    if constexpr (!EX) {
        #pragma unroll
        for (int s = 0; s < RB; s++) acc[s] = seg_sum<LPR>(acc[s]);
    }
    if constexpr (HQ) {
        // HO consecutive outputs per workgroup (RB/2 gate/up pairs per row
        // slot, whole groups of 32): h = silu(g)*u, then its per-32
        // quantization for the down projection
        constexpr int HO = (WG / WAVE) * RPW;
        static_assert(HO % 32 == 0, "h quantization takes whole groups of 32 per workgroup");
        __shared__ float hb[HO];
        if (l == LPR - 1) {
            #pragma unroll
            for (int s = 0; s < RB; s += 2) {
                const int row = orow[s];
                float h = 0.0f;
                if (valid[s]) {
                    float g = acc[s], u = acc[s + 1];
                    if (a.m[0].bias) g += a.m[0].bias[row];
                    if (a.m[1].bias) u += a.m[1].bias[row];
                    h = silu_ref(g) * u;                          // sml/sml-run.c:416-426
                    a.m[0].y[row] = h;
                }
                hb[wave * RPW + (s >> 1) * SUB + u] = h;
            }
        }
        __syncthreads();
        if (tid < HO) {
            const float v = hb[tid];
            const float s = max32(fabsf(v)) / 127.0f;
            const float is = s > 0.0f ? 1.0f / s : 0.0f;
            const int t = quant1(v, is);
            const int sum = isum32(t);
            const int row = blk * HO + tid;
            if (row < a.total_rows) {
                a.hq[row] = (int8_t) t;
                if ((tid & 31) == 0) { a.hscale[row >> 5] = s; a.hsums[row >> 5] = sum; }
            }
        }
        return;
    }
    if constexpr (!SW && !EX) {
        if (a.amax) {
            // the block's (max, lowest index) pair over its rows' outputs,
            // the values the store below writes
            constexpr int NS = (WG / WAVE) * SUB;
            __shared__ float am_v[NS];
            __shared__ int am_i[NS];
            if (l == LPR - 1) {
                float bv = -INFINITY;
                int bi = 0x7fffffff;
                #pragma unroll
                for (int s = 0; s < RB; s++) {
                    if (!valid[s]) continue;
                    const int row = orow[s];
                    float v = acc[s];
                    if (a.m[0].bias) v += a.m[0].bias[row];
                    if (a.epi == SML_EPI_RESIDUAL) v = a.resid[row] + v;
                    amax_take(v, row, bv, bi);
                }
                am_v[wave * SUB + u] = bv;
                am_i[wave * SUB + u] = bi;
            }
            __syncthreads();
            if (tid == 0) {
                float bv = am_v[0];
                int bi = am_i[0];
                #pragma unroll
                for (int k = 1; k < NS; k++) amax_take(am_v[k], am_i[k], bv, bi);
                a.amax[blk] = make_int2(__float_as_int(bv), bi);
            }
        }
    }
    if (l != LPR - 1) return;
    if constexpr (SW) {
        #pragma unroll
        for (int s = 0; s < RB; s += 2) {
            if (!valid[s]) continue;
            const int row = orow[s];
            float g = acc[s], u = acc[s + 1];
            if (a.m[0].bias) g += a.m[0].bias[row];
            if (a.m[1].bias) u += a.m[1].bias[row];
            a.m[0].y[row] = silu_ref(g) * u;               // sml/sml-run.c:416-426
        }
    } else {
        #pragma unroll
        for (int s = 0; s < RB; s++) {
            if (!valid[s]) continue;
            const int row = orow[s];
            float v = acc[s];
            if (a.m[0].bias) v += a.m[0].bias[row];
            if (a.epi == SML_EPI_RESIDUAL) v = a.resid[row] + v;
            a.m[0].y[row] = v;
        }
    }
}

// Kernel names: sml_gemv_q<bits>_r<rows per wave>_i<chunks per lane>, with
// suffix _n for the fused activation prologue (input width up to 4096);
// sml_gemv_q<bits>_s_r<RB>_i<NI> for SwiGLU (RB/2 gate/up pairs per wave, _sn
// with the prologue); sml_gemv_q<bits>_h_i<NI> for SwiGLU that also
// quantizes h: 16 lanes per row, so 8 waves x 4 pairs = 32 outputs per
// 512-thread workgroup (_hn with the prologue, input width up to 4096).
#define GEMV_KERNEL(NB, RB, NI)                                                                             \
    extern "C" __global__ __launch_bounds__(256) void sml_gemv_q##NB##_r##RB##_i##NI(const sml_kgemv a) {     \
        gemv_body<NB, RB, NI, 256, true, 0, false, false>(a);                                               \
    }
#define GEMV_KERNEL_N(NB, RB, NI)                                                                           \
    extern "C" __global__ __launch_bounds__(256) void sml_gemv_q##NB##_r##RB##_i##NI##_n(const sml_kgemv a) { \
        gemv_body<NB, RB, NI, 256, true, 1, false, false>(a);                                               \
    }
#define GEMV_KERNEL_S(NB, RB, NI)                                                                           \
    extern "C" __global__ __launch_bounds__(256) void sml_gemv_q##NB##_s_r##RB##_i##NI(const sml_kgemv a) {   \
        gemv_body<NB, RB, NI, 256, true, 0, true, false>(a);                                                \
    }                                                                                                       \
    extern "C" __global__ __launch_bounds__(256) void sml_gemv_q##NB##_sn_r##RB##_i##NI(const sml_kgemv a) {  \
        gemv_body<NB, RB, NI, 256, true, 1, true, false>(a);                                                \
    }
#define GEMV_KERNEL_H(NB, NI)                                                                               \
    extern "C" __global__ __launch_bounds__(512) void sml_gemv_q##NB##_h_i##NI(const sml_kgemv a) {       \
        gemv_body<NB, 2, NI, 512, true, 0, true, true, 16>(a);                                              \
    }                                                                                                       \
    extern "C" __global__ __launch_bounds__(512) void sml_gemv_q##NB##_hn_i##NI(const sml_kgemv a) {      \
        gemv_body<NB, 2, NI, 512, true, 1, true, true, 16>(a);                                              \
    }
// Wider workgroups for the fused prologue, which every workgroup computes
// in full: _n512 / _n1024 (input width up to 4096), and _hn1024_i<NI> with
// 64 outputs of h per workgroup.
#define GEMV_KERNEL_NW(NB, RB, NI, W)                                                                       \
    extern "C" __global__ __launch_bounds__(W) void sml_gemv_q##NB##_r##RB##_i##NI##_n##W(const sml_kgemv a) { \
        gemv_body<NB, RB, NI, W, true, 1, false, false>(a);                                                 \
    }
#define GEMV_KERNEL_HW(NB, NI, W)                                                                           \
    extern "C" __global__ __launch_bounds__(W) void sml_gemv_q##NB##_hn##W##_i##NI(const sml_kgemv a) {     \
        gemv_body<NB, 2, NI, W, true, 1, true, true, 16>(a);                                                \
    }
#define GEMV_WIDE(NB)                                                                                       \
    GEMV_KERNEL_NW(NB, 1, 1, 512) GEMV_KERNEL_NW(NB, 2, 1, 512) GEMV_KERNEL_NW(NB, 4, 1, 512)               \
    GEMV_KERNEL_NW(NB, 1, 1, 1024) GEMV_KERNEL_NW(NB, 2, 1, 1024) GEMV_KERNEL_HW(NB, 2, 1024)
#define GEMV_WIDTH(NB)                                                                     \
    GEMV_KERNEL(NB, 1, 2) GEMV_KERNEL(NB, 1, 4)                                            \
    GEMV_KERNEL(NB, 2, 1) GEMV_KERNEL(NB, 2, 2) GEMV_KERNEL(NB, 2, 4)                     \
    GEMV_KERNEL(NB, 4, 1) GEMV_KERNEL(NB, 4, 2) GEMV_KERNEL(NB, 4, 4)                     \
    GEMV_KERNEL_N(NB, 1, 1) GEMV_KERNEL_N(NB, 2, 1) GEMV_KERNEL_N(NB, 4, 1)               \
    GEMV_KERNEL_S(NB, 2, 1) GEMV_KERNEL_S(NB, 2, 2) GEMV_KERNEL_S(NB, 2, 4)               \
    GEMV_KERNEL_S(NB, 4, 1) GEMV_KERNEL_S(NB, 4, 2) GEMV_KERNEL_S(NB, 4, 4)               \
    GEMV_KERNEL_H(NB, 2) GEMV_KERNEL_H(NB, 4) GEMV_WIDE(NB)
GEMV_WIDTH(2) GEMV_WIDTH(3) GEMV_WIDTH(4) GEMV_WIDTH(5) GEMV_WIDTH(6) GEMV_WIDTH(7) GEMV_WIDTH(8)
// the roofline GEMV's shape with its timeline (sml_kgemv.ts): thread 0's
// clock at entry, first weight word, first pass's and last pass's weights
// all in, and at exit after the workgroup's stores
extern "C" __global__ __launch_bounds__(256) void sml_gemv_q4_r2_i4_ts(const sml_kgemv a) {
    __shared__ unsigned long long tsh[4];
    if (threadIdx.x == 0) tsh[3] = 0;
    gemv_body<4, 2, 4, 256, true, 0, false, false, 64, false, true>(a, blockIdx.x, true, tsh);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long * o = a.ts + (size_t) blockIdx.x * 5;
        o[0] = tsh[0]; o[1] = tsh[1]; o[2] = tsh[2]; o[3] = tsh[3] ? tsh[3] : tsh[2];
        o[4] = __builtin_amdgcn_s_memrealtime();
    }
}
// a whole 14336-wide row in one pass (tuning: SML_GEMV_NI=8)
GEMV_KERNEL(4, 1, 8) GEMV_KERNEL(4, 2, 8)
GEMV_KERNEL(2, 1, 8) GEMV_KERNEL(2, 2, 8) GEMV_KERNEL(3, 1, 8) GEMV_KERNEL(3, 2, 8)
GEMV_KERNEL(5, 1, 8) GEMV_KERNEL(5, 2, 8)

// Persistent forms (suffix _p, Q4): a grid of at most a few workgroups per CU,
// each taking row blocks blockIdx.x, +gridDim.x, ...; the activation (or the
// fused prologue's) is staged in LDS once per workgroup.
template <int NB, int RB, int NI, int WG, int AM, bool SW, bool HQ, int LPR = 64>
__device__ void gemv_persistent(const sml_kgemv & a) {
    constexpr int RPWG = (WG / 64) * (SW ? RB / 2 : RB) * (64 / LPR);     // rows (outputs) per block
    const int nblk = (a.total_rows + RPWG - 1) / RPWG;
    for (int b = blockIdx.x; b < nblk; b += gridDim.x) {
        gemv_body<NB, RB, NI, WG, true, AM, SW, HQ, LPR>(a, b, b == (int) blockIdx.x);
        __syncthreads();
    }
}
#define GEMV_KERNEL_P(RB, NI)                                                                               \
    extern "C" __global__ __launch_bounds__(256) void sml_gemv_q4_r##RB##_i##NI##_p(const sml_kgemv a) {     \
        gemv_persistent<4, RB, NI, 256, 0, false, false>(a);                                                \
    }
#define GEMV_KERNEL_NWP(RB)                                                                                 \
    extern "C" __global__ __launch_bounds__(512) void sml_gemv_q4_r##RB##_i1_n512_p(const sml_kgemv a) {     \
        gemv_persistent<4, RB, 1, 512, 1, false, false>(a);                                                 \
    }
GEMV_KERNEL_P(1, 2) GEMV_KERNEL_P(1, 4) GEMV_KERNEL_P(2, 1) GEMV_KERNEL_P(2, 2) GEMV_KERNEL_P(2, 4)
GEMV_KERNEL_P(4, 1) GEMV_KERNEL_P(4, 2) GEMV_KERNEL_P(4, 4)
GEMV_KERNEL_NWP(1) GEMV_KERNEL_NWP(2) GEMV_KERNEL_NWP(4)
extern "C" __global__ __launch_bounds__(512) void sml_gemv_q4_hn_i2_p(const sml_kgemv a) {
    gemv_persistent<4, 2, 2, 512, 1, true, true, 16>(a);
}
extern "C" __global__ __launch_bounds__(512) void sml_gemv_q4_h_i2_p(const sml_kgemv a) {
    gemv_persistent<4, 2, 2, 512, 0, true, true, 16>(a);
}

// The exact forms (suffix _x, Q4 and Q8): the reference's float order per row
// (gemv_body EX), for every shape pick_shape gives an unfused launch.
#define GEMV_KERNEL_X(NB, RB, NI)                                                                           \
    extern "C" __global__ __launch_bounds__(256) void sml_gemv_q##NB##_r##RB##_i##NI##_x(const sml_kgemv a) { \
        gemv_body<NB, RB, NI, 256, true, 0, false, false, 64, true>(a);                                     \
    }
#define GEMV_KERNEL_SX(NB, RB, NI)                                                                          \
    extern "C" __global__ __launch_bounds__(256) void sml_gemv_q##NB##_s_r##RB##_i##NI##_x(const sml_kgemv a) { \
        gemv_body<NB, RB, NI, 256, true, 0, true, false, 64, true>(a);                                      \
    }
// _xn: the same with the fused RMSNorm/gather/quantize prologue (exact norm)
#define GEMV_KERNEL_XN(NB, RB, NI)                                                                          \
    extern "C" __global__ __launch_bounds__(256) void sml_gemv_q##NB##_r##RB##_i##NI##_xn(const sml_kgemv a) { \
        gemv_body<NB, RB, NI, 256, true, 1, false, false, 64, true>(a);                                     \
    }
#define GEMV_KERNEL_SXN(NB, RB, NI)                                                                         \
    extern "C" __global__ __launch_bounds__(256) void sml_gemv_q##NB##_s_r##RB##_i##NI##_xn(const sml_kgemv a) { \
        gemv_body<NB, RB, NI, 256, true, 1, true, false, 64, true>(a);                                      \
    }
// _hxn: the exact SwiGLU with the norm prologue and h quantized per 32 in
// its epilogue (32 outputs per workgroup: 8 waves of 4 pairs, or 16 of 2)
#define GEMV_KERNEL_HXN(NB)                                                                                 \
    extern "C" __global__ __launch_bounds__(512) void sml_gemv_q##NB##_hxn_r8_i1(const sml_kgemv a) {         \
        gemv_body<NB, 8, 1, 512, true, 1, true, true, 64, true>(a);                                         \
    }                                                                                                       \
    extern "C" __global__ __launch_bounds__(1024) void sml_gemv_q##NB##_hxn1024_r4_i1(const sml_kgemv a) {    \
        gemv_body<NB, 4, 1, 1024, true, 1, true, true, 64, true>(a);                                        \
    }
GEMV_KERNEL_HXN(4) GEMV_KERNEL_HXN(8)
#define GEMV_EXACT(NB, K, KS)                                                                               \
    K(NB, 1, 2) K(NB, 1, 4) K(NB, 2, 1) K(NB, 2, 2) K(NB, 2, 4) K(NB, 4, 1) K(NB, 4, 2) K(NB, 4, 4)         \
    KS(NB, 2, 1) KS(NB, 2, 2) KS(NB, 2, 4) KS(NB, 4, 1) KS(NB, 4, 2) KS(NB, 4, 4)
GEMV_EXACT(4, GEMV_KERNEL_X, GEMV_KERNEL_SX) GEMV_EXACT(8, GEMV_KERNEL_X, GEMV_KERNEL_SX)
GEMV_EXACT(4, GEMV_KERNEL_XN, GEMV_KERNEL_SXN) GEMV_EXACT(8, GEMV_KERNEL_XN, GEMV_KERNEL_SXN)
// wider exact forms: 8 rows per wave, and 512-thread workgroups (suffix _w512)
#define GEMV_KERNEL_XW(NB, RB, NI, W, AM, SFX)                                                              \
    extern "C" __global__ __launch_bounds__(W) void sml_gemv_q##NB##_r##RB##_i##NI##_##SFX(const sml_kgemv a) { \
        gemv_body<NB, RB, NI, W, true, AM, false, false, 64, true>(a);                                      \
    }
#define GEMV_EXACT_WIDE(NB)                                                                                 \
    GEMV_KERNEL_XW(NB, 8, 1, 256, 0, x) GEMV_KERNEL_XW(NB, 8, 2, 256, 0, x)                                 \
    GEMV_KERNEL_XW(NB, 8, 1, 512, 0, x_w512) GEMV_KERNEL_XW(NB, 4, 2, 512, 0, x_w512)                       \
    GEMV_KERNEL_XW(NB, 2, 4, 512, 0, x_w512) GEMV_KERNEL_XW(NB, 8, 1, 256, 1, xn)                           \
    GEMV_KERNEL_XW(NB, 8, 1, 512, 1, xn_w512) GEMV_KERNEL_XW(NB, 4, 1, 512, 1, xn_w512)                     \
    GEMV_KERNEL_XW(NB, 2, 2, 512, 1, xn_w512) GEMV_KERNEL_XW(NB, 2, 1, 512, 1, xn_w512)                     \
    GEMV_KERNEL_XW(NB, 1, 1, 512, 1, xn_w512)
GEMV_EXACT_WIDE(4) GEMV_EXACT_WIDE(8)

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
    // row blockIdx.y of a batch (every pointer strided by its row)
    const size_t bo = (size_t) blockIdx.y * n, bg = (size_t) blockIdx.y * (n / 32);
    float * x = a.x + bo;
    const float * resid = a.resid ? a.resid + bo : nullptr;
    double ss = 0.0;
    for (int i = tid; i < n; i += NORMQ_THREADS) {
        float v = x[i];
        if (resid) { v = v + resid[i]; x[i] = v; }
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
        float msq = (float) (tot / (double) n);
        if (a.exact && !ss_mean_alike(tot, n, msq)) {
            // the reference build's loop: ss = fma(x_i, x_i, ss) in order
            // (tot is the same in every thread, so all take this branch)
            __syncthreads();
            if (tid == 0) red[0] = serial_ss(sx, n);
            __syncthreads();
            msq = (float) (red[0] / (double) n);
        }
        // IEEE division and square root: hipcc's default for HIP is the correctly
        // rounded fp32 divide/sqrt, which the bit-exact parity tests rely on
        const float sc = 1.0f / sqrtf(msq + a.eps);
        for (int i = tid; i < n; i += NORMQ_THREADS) sx[i] = sx[i] * sc * a.norm_w[i];
    }
    __syncthreads();
    if (a.normed) for (int i = tid; i < n; i += NORMQ_THREADS) a.normed[bo + i] = sx[i];
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
            int8_t * q = a.q[o] + bo + g * 32;
            #pragma unroll
            for (int j = 0; j < 32; j += 4) {
                int w = 0;
                #pragma unroll
                for (int k = 0; k < 4; k++) {
                    // x86 cvtps2dq (the reference's AVX2 arm) yields INT_MIN for
                    // NaN and out-of-range values; the clamp then gives -127
                    const float r = __builtin_rintf(v[j + k] * is);
                    int t = (r >= -2147483648.0f && r < 2147483648.0f) ? (int) r : (int) 0x80000000u;
                    t = t > 127 ? 127 : t < -127 ? -127 : t;
                    sum += t;
                    w |= (t & 0xFF) << (8 * k);
                }
                *(int *) (q + j) = w;
            }
            a.scale[o][bg + g] = s;
            a.sums[o][bg + g] = sum;
        }
    }
}

// Four values' squares added to a double sum, in sml_normq2's order (its
// callers share it so that their sums agree bit for bit).
__device__ __forceinline__ double ss_add4(double ss, float4 v) {
    return ss + ((double) v.x * v.x + (double) v.y * v.y + (double) v.z * v.z + (double) v.w * v.w);
}

// Multi-workgroup form (the decode path's): workgroup b quantizes elements
// 256b..256b+255 (one superblock) of each output; each reduces the full sum of
// squares first. per256: the superblock's amax meets across the 4 waves in LDS
// (sml/sml-kernel.c:165-172).
extern "C" __global__ __launch_bounds__(256) void sml_normq2(const sml_knormq2 a) {
    __shared__ double red[4];
    __shared__ float wmax[2][4];
    const int n = a.n, tid = threadIdx.x;
    // row blockIdx.y of a batch (every pointer strided by its row)
    const size_t bo = (size_t) blockIdx.y * n, bg = (size_t) blockIdx.y * (n / 32);
    const float * x = a.x + bo;
    const int j = blockIdx.x * 256 + tid;           // element (group j/32) of every output
    const bool ok = j < n;                          // whole groups of 32 (n % 32 == 0)
    // every output's gathered value and norm weight are asked for first: they
    // need only the permutation, not the sum of squares, so their two
    // dependent loads overlap the row's read and its reduction
    float xv[3], wv[3];
    #pragma unroll
    for (int o = 0; o < 3; o++) {
        xv[o] = 0.0f;
        wv[o] = 1.0f;
        if (o < a.nout && ok) {
            const int src = a.perm[o] ? a.perm[o][j] : j;
            xv[o] = x[src];
            if (a.norm_w) wv[o] = a.norm_w[src];
        }
    }
    float sc = 1.0f;
    if (a.norm_w) {
        double ss = 0.0;
        for (int i = tid * 4; i < n; i += 1024) ss = ss_add4(ss, *(const float4 *) (x + i));
        #pragma unroll
        for (int o = 32; o; o >>= 1) ss += __shfl_xor(ss, o);
        if ((tid & 63) == 0) red[tid >> 6] = ss;
        __syncthreads();
        const double tot = red[0] + red[1] + red[2] + red[3];
        float msq = (float) (tot / (double) n);
        if (a.exact && !ss_mean_alike(tot, n, msq)) {
            // the serial chain (the same decision in every thread)
            __syncthreads();
            if (tid == 0) red[0] = serial_ss(x, n);
            __syncthreads();
            msq = (float) (red[0] / (double) n);
        }
        sc = 1.0f / sqrtf(msq + a.eps);
    }
    const int l32 = tid & 31, g = j >> 5;
    #pragma unroll
    for (int o = 0; o < 3; o++) {
        if (o >= a.nout) break;
        const float v = a.norm_w ? xv[o] * sc * wv[o] : xv[o];
        float amax;
        if (a.per256) {
            // double-buffered by output: the next write to this slot follows
            // the next output's barrier, which every reader of it has passed
            const float wm = wave_max(fabsf(v));
            if ((tid & 63) == 0) wmax[o & 1][tid >> 6] = wm;
            __syncthreads();
            amax = fmaxf(fmaxf(wmax[o & 1][0], wmax[o & 1][1]), fmaxf(wmax[o & 1][2], wmax[o & 1][3]));
        } else {
            amax = max32(fabsf(v));
        }
        const float s = amax / 127.0f;
        const float is = s > 0.0f ? 1.0f / s : 0.0f;
        const int t = quant1(v, is);
        const int sum = isum32(t);
        if (!ok) continue;
        a.q[o][bo + j] = (int8_t) t;
        if (l32 == 0) { a.scale[o][bg + g] = s; a.sums[o][bg + g] = sum; }
    }
}

// ---------------------------------------------------------------- unpack / embed

// The integer codes of group g of one row, from the planes (the reads of
// load_chunk / chunk_dots, one group at a time).
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
    // a batch (pos NULL, grid y = rows): row b takes token tok[b] into x + b*cols
    const int b = a.pos ? 0 : (int) blockIdx.y;
    const size_t row = (size_t) (a.pos ? a.tok[*a.pos] : a.tok[b]);
    float * x = a.x + (size_t) b * a.cols;
    const uint8_t * f = a.m.sqmq + (row * ng + g) * 2;
    const uint16_t * d = a.m.sdmd + (row * ns + g / 8) * 2;
    if (a.nbits == 4 && !a.perm) {
        // Q4 in order: the group's 32 bytes as two 16-byte loads (its
        // nibbles, the low or high half of each byte), 8 float4 stores
        const uint8_t * blk = a.m.plane[0] + row * (size_t) (a.cols / 2) + (size_t) (g >> 2) * 64 + ((g & 2) ? 32 : 0);
        const v4u lo = gld<v4u>(blk), hi = gld<v4u>(blk + 16);
        const float step = h2f(d[0]) * (float) f[0];
        const float mn = h2f(d[1]) * ((float) f[1] - 127.0f);
        const unsigned sh = (g & 1) ? 4u : 0u;
        #pragma unroll
        for (int k = 0; k < 8; k++) {
            const unsigned w = k < 4 ? lo[k] : hi[k - 4];
            float4 o;
            o.x = __builtin_fmaf((float) ((w >> sh) & 15u), step, mn);
            o.y = __builtin_fmaf((float) ((w >> (sh + 8)) & 15u), step, mn);
            o.z = __builtin_fmaf((float) ((w >> (sh + 16)) & 15u), step, mn);
            o.w = __builtin_fmaf((float) ((w >> (sh + 24)) & 15u), step, mn);
            *(float4 *) (x + g * 32 + 4 * k) = o;
        }
        return;
    }
    uint8_t c[32];
    group_codes(a.m, a.nbits, a.cols, row, g, c);
    const float step = h2f(d[0]) * (float) f[0];
    const float mn = h2f(d[1]) * ((float) f[1] - 127.0f);
    // the reference's order: fma(code, step, min), then Q3/Q5/Q7 add their
    // 1-bit plane's step*2^shift where the bit is set (sml/sml-kernel.c:2134-2260)
    const int shift = a.nbits == 3 ? 2 : a.nbits == 5 ? 4 : a.nbits == 7 ? 6 : 0;
    const int low = shift ? (1 << shift) - 1 : 255;
    const float add = step * (float) (1 << shift);
    for (int j = 0; j < 32; j++) {
        const int col = g * 32 + j;
        float v = __builtin_fmaf((float) (c[j] & low), step, mn);
        if (shift && (c[j] >> shift) & 1) v = v + add;
        x[a.perm ? a.perm[col] : col] = v;
    }
}

// ---------------------------------------------------------------- attention
//
// Decode attention in one launch (sml/sml-run.c:180-287 per head: scores
// q.k/sqrt(hd), softmax with the running max subtracted, weighted sum of V).
// Workgroup (split, kv head, sequence) covers ATTN_CHUNK positions for the REP
// query heads sharing that KV head with NW waves (8 by default: two per SIMD
// hide the compute phases' latency better than one). Lane (grp = tid/16,
// l16 = tid%16) owns dims 8*l16..+7 of positions t0 + grp + 4*NW*i: 16 lanes
// read 256 contiguous bytes of a position's K (then V) row, so the cache
// streams coalesced.
//
// Latency, not bandwidth, bounds the kernel below a few thousand positions,
// so every global load is issued before the first wait: q, k and v of the
// lane's dims (independent of the position) with the position itself, then
// the whole K/V chunk and the RoPE table row. RoPE is applied in registers
// (the (d, d+64) partner of lane l16 is lane l16^8 of the same DPP row), the
// scores reduce over 16 lanes with DPP, and each wave keeps its own softmax
// max, so the only LDS round trip is the final combine of the waves. The
// workgroup holding position *pos rounds the rotated k and v to fp16, writes
// them to the cache and uses them in place of the row it loaded. A split past
// the position writes an empty partial (max -inf, sum 0), so sml_attn_merge
// needs no position.
#define ATTN_CHUNK 128
#define ATTN_MAXREP 8
#define HD 128

__device__ __forceinline__ void unpack_h8(const v4u w, float (&f)[8]) {
    #pragma unroll
    for (int e = 0; e < 4; e++) { f[2 * e] = h2f((uint16_t) (w[e] & 0xFFFFu)); f[2 * e + 1] = h2f((uint16_t) (w[e] >> 16)); }
}
__device__ __forceinline__ void load_f8(const float * p, float (&f)[8]) {
    const float4 a = *(const float4 *) p, b = *(const float4 *) (p + 4);
    f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w; f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
}
// Rotate the lane's 8 dims by the (d, d+64) pair rule of sml/sml-run.c:363-368:
// lanes 0-7 of a row hold the first halves, lanes 8-15 the second, and
// row_ror:8 brings each lane its partner. The products fuse as the
// reference's x86 build fuses them: x0*c - x1*s = fma(x0, c, -(x1*s)),
// x0*s + x1*c = fma(x0, s, x1*c).
__device__ __forceinline__ void rope8(float (&x)[8], const float (&c)[8], const float (&s)[8], bool lo) {
    float p[8];
    #pragma unroll
    for (int e = 0; e < 8; e++) p[e] = dpp_f<0x128>(x[e]);
    #pragma unroll
    for (int e = 0; e < 8; e++)
        x[e] = lo ? __builtin_fmaf(x[e], c[e], -(p[e] * s[e])) : __builtin_fmaf(p[e], s[e], x[e] * c[e]);
}
// rope8 for a head of LP*8 dims: the (d, d + D/2) partner of a lane is lane
// ^ LP/2 of its position's lanes (LP 16: row_ror:8; LP 8: the half-row
// mirror, then the quad reversal, which together map lane i to i ^ 4)
template <int LP>
__device__ __forceinline__ void rope8p(float (&x)[8], const float (&c)[8], const float (&s)[8], bool lo) {
    if constexpr (LP == 16) {
        rope8(x, c, s, lo);
    } else {
        float p[8];
        #pragma unroll
        for (int e = 0; e < 8; e++) p[e] = dpp_f<0x1B>(dpp_f<0x141>(x[e]));
        #pragma unroll
        for (int e = 0; e < 8; e++)
            x[e] = lo ? __builtin_fmaf(x[e], c[e], -(p[e] * s[e])) : __builtin_fmaf(p[e], s[e], x[e] * c[e]);
    }
}
// the sum over each group of 8 lanes, in every lane of the group
__device__ __forceinline__ float sum8(float v) {
    v += dpp_f<0xB1>(v); v += dpp_f<0x4E>(v); return v + dpp_f<0x141>(v);
}
// Reduce-scatter of four values over the 4 rows of a wave with the gfx950
// row swaps (v_permlane16_swap: rows 1 and 3 of the first operand trade
// places with rows 0 and 2 of the second; v_permlane32_swap: rows 2-3 of the
// first with rows 0-1 of the second). On return a lane of row r holds the
// sum (max) over the rows of its argument r. The operands of each swap are
// always distinct values: the compiler folds a register swapped with itself
// into the wrong result.
__device__ __forceinline__ int fbits(float v) { return __builtin_bit_cast(int, v); }
__device__ __forceinline__ float ibits(int v) { return __builtin_bit_cast(float, v); }
__device__ __forceinline__ float rows_sum4(float a, float b, float c, float d) {
    const auto p = __builtin_amdgcn_permlane16_swap(fbits(a), fbits(b), false, false);
    const auto q = __builtin_amdgcn_permlane16_swap(fbits(c), fbits(d), false, false);
    const float u = ibits(p[0]) + ibits(p[1]), w = ibits(q[0]) + ibits(q[1]);
    const auto r = __builtin_amdgcn_permlane32_swap(fbits(u), fbits(w), false, false);
    return ibits(r[0]) + ibits(r[1]);
}
__device__ __forceinline__ float rows_max4(float a, float b, float c, float d) {
    const auto p = __builtin_amdgcn_permlane16_swap(fbits(a), fbits(b), false, false);
    const auto q = __builtin_amdgcn_permlane16_swap(fbits(c), fbits(d), false, false);
    const float u = fmaxf(ibits(p[0]), ibits(p[1])), w = fmaxf(ibits(q[0]), ibits(q[1]));
    const auto r = __builtin_amdgcn_permlane32_swap(fbits(u), fbits(w), false, false);
    return fmaxf(ibits(r[0]), ibits(r[1]));
}
__device__ __forceinline__ float rl(float v, int lane) { return ibits(__builtin_amdgcn_readlane(fbits(v), lane)); }

// Wave-uniform max / sum over the wave of per-head values x[j] (each the same
// across a row's 16 lanes), four heads per reduce-scatter.
template <int REP>
__device__ __forceinline__ void wave_heads(const float (&x)[REP], float (&out)[REP], bool is_max) {
    #pragma unroll
    for (int g = 0; g < REP; g += 4) {
        const float pad = is_max ? -INFINITY : 0.0f;
        const float a = x[g], b = g + 1 < REP ? x[g + 1 < REP ? g + 1 : g] : pad,
                    c = g + 2 < REP ? x[g + 2 < REP ? g + 2 : g] : pad, d = g + 3 < REP ? x[g + 3 < REP ? g + 3 : g] : pad;
        const float r = is_max ? rows_max4(a, b, c, d) : rows_sum4(a, b, c, d);
        #pragma unroll
        for (int k = 0; k < 4; k++)
            if (g + k < REP) out[g + k] = rl(r, 16 * k);
    }
}

// Merge of the splits of one query head: out = sum_s e_s o_s / sum_s e_s l_s
// with e_s = 2^(m_s - max m) (the split maxima are in base 2). Every split
// has a partial (max -inf for splits past the position), so a batch of 32
// splits is loaded at once with no position read first: lane s of the wave
// takes split s's (max, sum) and its weight e_s, which the dims then read back
// as a scalar. The calling wave holds 64 consecutive dims d of head h (lane =
// d & 63). With q_out set, the head's 128 outputs (4 groups of 32, identity
// permutation) are also quantized for the next GEMV (sml/sml-kernel.c:86-106).
// DEV: the partials were written by other workgroups of the running launch,
// so they are read at device scope.
#define MERGE_BATCH 32
template <bool DEV> __device__ __forceinline__ float ld_part(const float * p) {
    if constexpr (DEV) return __hip_atomic_load((float *) p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else return *p;
}
template <bool DEV> __device__ __forceinline__ float2 ld_part2(const float2 * p) {
    if constexpr (DEV)
        return __builtin_bit_cast(float2, __hip_atomic_load((unsigned long long *) p, __ATOMIC_RELAXED,
                                                            __HIP_MEMORY_SCOPE_AGENT));
    else return *p;
}
// stores of partials that another workgroup of the same launch reads:
// coherent at device scope once the storing wave's vmcnt reaches zero
__device__ __forceinline__ void st_dev(float * p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev2(float2 * p, float2 v) {
    __hip_atomic_store((unsigned long long *) p, __builtin_bit_cast(unsigned long long, v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
// The merged output of dim d of head h of entry b, also stored to a.out.
template <bool DEV, int D = HD>
__device__ __forceinline__ float merge_value(const sml_kattn & a, int b, int h, int d) {
    const int lane = d & 63;
    const float * blk = a.part + (size_t) b * a.n_head * a.nsplit * (D + 2);
    const float * po = blk + (size_t) h * a.nsplit * D;
    const float2 * pml = (const float2 *) (blk + (size_t) a.n_head * a.nsplit * D) + (size_t) h * a.nsplit;
    const size_t ob = (size_t) b * a.n_head * D;
    float M = -INFINITY, L = 0.0f, o = 0.0f;
    // a batch of MERGE_BATCH splits; indices past the last split read split
    // 0 (their weights are zero below)
    auto fetch = [&](int s0, float (&ov)[MERGE_BATCH], float2 & ml) {
        #pragma unroll
        for (int s = 0; s < MERGE_BATCH; s++) {
            const int i = s0 + s < a.nsplit ? s0 + s : 0;
            ov[s] = ld_part<DEV>(po + (size_t) i * D + d);
        }
        const int j = s0 + lane < a.nsplit ? s0 + lane : 0;
        ml = ld_part2<DEV>(pml + j);
    };
    auto fold = [&](int s0, const float (&ov)[MERGE_BATCH], const float2 ml) {
        const int n = min(MERGE_BATCH, a.nsplit - s0);
        const float mj = lane < n ? ml.x : -INFINITY;
        const float Mb = fmaxf(M, rl(max32(mj), 0));         // finite: split 0 is active
        const float r = __builtin_amdgcn_exp2f(M - Mb);      // M = -inf: 0
        const float e = __builtin_amdgcn_exp2f(mj - Mb);     // 0 for splits past the position
        L = L * r + rl(sum32(lane < n ? e * ml.y : 0.0f), 0);
        float acc[4] = {o * r, 0.0f, 0.0f, 0.0f};
        #pragma unroll
        for (int s = 0; s < MERGE_BATCH; s++) {
            const float es = rl(e, s);
            acc[s & 3] += es != 0.0f ? es * ov[s] : 0.0f;     // an empty split's V sums are not read
        }
        o = (acc[0] + acc[1]) + (acc[2] + acc[3]);
        M = Mb;
    };
    float ov[MERGE_BATCH];
    float2 ml;
    fetch(0, ov, ml);
    int s0 = 0;
    // more than one batch: the next batch's loads go out before this one is
    // folded (issued only where a next batch exists, so a one-batch merge
    // waits for nothing extra)
    for (; s0 + MERGE_BATCH < a.nsplit; s0 += MERGE_BATCH) {
        float ovn[MERGE_BATCH];
        float2 mln;
        fetch(s0 + MERGE_BATCH, ovn, mln);
        fold(s0, ov, ml);
        #pragma unroll
        for (int s = 0; s < MERGE_BATCH; s++) ov[s] = ovn[s];
        ml = mln;
    }
    fold(s0, ov, ml);
    const float r = o / L;
    a.out[ob + (size_t) h * D + d] = r;
    return r;
}
template <bool DEV, int D = HD>
__device__ __forceinline__ void merge_head(const sml_kattn & a, int b, int h, int d) {
    const float r = merge_value<DEV, D>(a, b, h, d);
    if (!a.q_out) return;
    const size_t ob = (size_t) b * a.n_head * D;
    const float amax = max32(fabsf(r));
    const float s = amax / 127.0f;
    const float is = s > 0.0f ? 1.0f / s : 0.0f;
    const int t = quant1(r, is);
    const int sum = isum32(t);
    const int g = h * (D / 32) + (d >> 5);
    a.q_out[ob + (size_t) h * D + d] = (int8_t) t;
    if ((d & 31) == 0) { a.s_out[ob / 32 + g] = s; a.u_out[ob / 32 + g] = sum; }
}

// CH: positions per split (128; the one-sequence decode launch also takes 32
// or 64, so that models with few KV heads still fill the chip). D: head_dim
// (128, or 64: a position's 64 dims on 8 lanes, two positions to a 16-lane
// row, whose halves are combined before the cross-row reductions).
template <int REP, int NW, bool CHUNK, int CH = ATTN_CHUNK, int D = HD>
__device__ __forceinline__ void attn_body(const sml_kattn & a) {
    constexpr int LP = D / 8;                                   // lanes per position
    constexpr int NT = 64 * NW, PS = NT / LP, PPL = CH / PS;   // threads, position stride, positions per lane
    static_assert(PPL >= 1 && PPL * PS == CH, "a split covers whole rounds of positions");
    __shared__ float red[NW][REP][D];
    __shared__ float wm[NW][REP], wl[NW][REP];
    // kv head kh; query heads qh0 .. qh0+REP-1 (a subset of the kv head's
    // when nsub > 1: each head's arithmetic is the same whichever workgroup
    // holds it, so the split into subsets changes no bit)
    const int nsub = CHUNK || a.nsub < 1 ? 1 : a.nsub;
    const int kh = (int) blockIdx.y / nsub, qh0 = kh * REP * nsub + ((int) blockIdx.y % nsub) * REP;
    const int split = blockIdx.x, tid = threadIdx.x;
    const int wave = tid >> 6, grp = tid / LP, l16 = tid % LP, kvd = a.n_kv * D;
    // the workgroup's entries b0..b1-1: one, or (tpw > 1) consecutive
    // positions of one sequence, which share this split's K/V tile
    const int tpw = CHUNK ? a.tpw : 1;
    const int b0 = blockIdx.z * tpw, b1 = CHUNK ? min(b0 + tpw, a.nseq) : b0 + 1;
    const int t0 = split * CH, tlast = a.pos[b1 - 1] + 1;
    GLOBAL uint16_t * kcache = (GLOBAL uint16_t *) (a.kc_slots ? a.kc_slots[a.slot[b0]] + a.layer_off : a.kcache);
    GLOBAL uint16_t * vcache = (GLOBAL uint16_t *) (a.vc_slots ? a.vc_slots[a.slot[b0]] + a.layer_off : a.vcache);
    // the first entry's q, k and v load first: loads return in order
    const int half = D / 2;
    float nq[REP][8], nk[8], nv[8], ncs[8], nsn[8];
    auto fetch_qkv = [&](int b) {
        const float * aq = a.q + (size_t) b * a.qkv_stride + (size_t) qh0 * D + l16 * 8;
        const float * ak = a.k + (size_t) b * a.qkv_stride + (size_t) kh * D + l16 * 8;
        const float * av = a.v + (size_t) b * a.qkv_stride + (size_t) kh * D + l16 * 8;
        #pragma unroll
        for (int j = 0; j < REP; j++) load_f8(aq + j * D, nq[j]);
        load_f8(ak, nk);
        load_f8(av, nv);
    };
    auto fetch_rope = [&](int b) {
        const int p = a.pos[b];
        load_f8(a.cos_t + (size_t) p * half + (l16 & (LP / 2 - 1)) * 8, ncs);
        load_f8(a.sin_t + (size_t) p * half + (l16 & (LP / 2 - 1)) * 8, nsn);
    };
    auto fetch = [&](int b) { fetch_qkv(b); fetch_rope(b); };
    // merge folded in (one-entry launches with counters): once every wave's
    // partial stores have completed at device scope, the workgroup counts
    // itself in; the last of the kv head's splits merges its query heads
    // (two waves' worth of dims each) and clears the counter for the next launch
    const bool fold = !CHUNK && a.cnt != nullptr;
    auto fold_merge = [&](int b) {
        __shared__ int last;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        int * cnt = a.cnt + (size_t) b * a.n_kv + kh;
        if (tid == 0)
            last = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (int) gridDim.x - 1;
        __syncthreads();
        if (!last) return;
        constexpr int WPH = D / 64;                   // waves per head
        for (int t = wave; t < WPH * REP; t += NW)
            merge_head<true, D>(a, b, qh0 + t / WPH, (t % WPH) * 64 + (tid & 63));
        if (tid == 0) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };
    // a split past every entry's position (they increase) writes empty
    // partials only. Leaving here, before any K/V load, keeps those loads
    // unconditional below, so the compiler's waits stay partial.
    auto empty = [&](int b) {
        float2 * pml = (float2 *) (a.part + (size_t) b * a.n_head * a.nsplit * (D + 2) +
                                   (size_t) a.n_head * a.nsplit * D) + (size_t) qh0 * a.nsplit;
        if (tid < REP) {
            if (fold) st_dev2(pml + (size_t) tid * a.nsplit + split, make_float2(-INFINITY, 0.0f));
            else pml[(size_t) tid * a.nsplit + split] = make_float2(-INFINITY, 0.0f);
        }
        if (fold) fold_merge(b);
    };
    if (t0 >= tlast) {
        for (int b = b0; b < b1; b++) empty(b);
        return;
    }
    fetch_qkv(b0);
    // the RoPE rows ahead of the tile: loads return in order, and q's rotation
    // comes before the first score
    fetch_rope(b0);
    // all of K, then all of V: loads return in order, so the scores and the
    // softmax run while V is still arriving
    v4u kw[PPL], vw[PPL];
    const int tl = min(tlast, t0 + CH);
    #pragma unroll
    for (int i = 0; i < PPL; i++) {
        int t = t0 + grp + PS * i;
        t = t < tl ? t : t0;                          // in range; masked below
        kw[i] = __builtin_nontemporal_load((const GLOBAL v4u *) (kcache + (size_t) t * kvd + (size_t) kh * D + l16 * 8));
    }
    #pragma unroll
    for (int i = 0; i < PPL; i++) {
        int t = t0 + grp + PS * i;
        t = t < tl ? t : t0;
        vw[i] = __builtin_nontemporal_load((const GLOBAL v4u *) (vcache + (size_t) t * kvd + (size_t) kh * D + l16 * 8));
    }
    // the tile's loads go out before any work on q, k and v: scheduled
    // after it, they would wait for those inputs' arrival first
    __builtin_amdgcn_sched_barrier(0);
    // each entry's arithmetic is the one-entry kernel's, position for position;
    // with few heads the next entry's inputs load while this one computes
    constexpr bool PF = CHUNK && REP <= 4;
    for (int b = b0; b < b1; b++) {
    if (!PF && b > b0) fetch(b);
    float q[REP][8], kn[8], vn[8], cs[8], sn[8];
    #pragma unroll
    for (int e = 0; e < 8; e++) {
        #pragma unroll
        for (int j = 0; j < REP; j++) q[j][e] = nq[j][e];
        kn[e] = nk[e]; vn[e] = nv[e]; cs[e] = ncs[e]; sn[e] = nsn[e];
    }
    if (PF && b + 1 < b1) fetch(b + 1);
    const int pos = a.pos[b], T = pos + 1;
    // partials of entry b: V sums [head][split][D], then (max, sum) [head][split]
    float * blk = a.part + (size_t) b * a.n_head * a.nsplit * (D + 2);
    float * po = blk + (size_t) qh0 * a.nsplit * D;
    float2 * pml = (float2 *) (blk + (size_t) a.n_head * a.nsplit * D) + (size_t) qh0 * a.nsplit;
    if (t0 >= T) {
        empty(b);
        continue;
    }
    const int t1 = min(T, t0 + CH);
    const bool lo = l16 < LP / 2;
    const float sl = a.inv * 1.44269504088896341f;
    #pragma unroll
    for (int j = 0; j < REP; j++) rope8p<LP>(q[j], cs, sn, lo);
    // k rotated, then k and v rounded to fp16 as the cache stores them (sml/sml-run.c:3414-3415)
    rope8p<LP>(kn, cs, sn, lo);
    v4u knew, vnew;
    #pragma unroll
    for (int e = 0; e < 4; e++) {
        knew[e] = (unsigned) f2h(kn[2 * e]) | ((unsigned) f2h(kn[2 * e + 1]) << 16);
        vnew[e] = (unsigned) f2h(vn[2 * e]) | ((unsigned) f2h(vn[2 * e + 1]) << 16);
    }
    if (!a.kv_written && t0 <= pos && pos < t1 && tid < LP && qh0 == kh * REP * nsub) {
        *(GLOBAL v4u *) (kcache + (size_t) pos * kvd + (size_t) kh * D + l16 * 8) = knew;
        *(GLOBAL v4u *) (vcache + (size_t) pos * kvd + (size_t) kh * D + l16 * 8) = vnew;
    }
    // scores: 8 FMAs per lane, summed over the position's LP lanes
    float sc[PPL][REP];
    #pragma unroll
    for (int i = 0; i < PPL; i++) {
        const int t = t0 + grp + PS * i;
        float kf[8];
        unpack_h8(t == pos ? knew : kw[i], kf);
        #pragma unroll
        for (int j = 0; j < REP; j++) {
            float p = 0.0f;
            #pragma unroll
            for (int e = 0; e < 8; e++) p += q[j][e] * kf[e];
            p = LP == 16 ? sum16(p) : sum8(p);
            sc[i][j] = t < t1 ? p * sl : -INFINITY;
        }
    }
    // the wave's softmax over its positions, in base 2 (scores were scaled
    // by log2 e): every lane of a row holds the row's scores, so the row
    // swaps cover the wave
    float m[REP], l[REP], xs[REP];
    #pragma unroll
    for (int j = 0; j < REP; j++) {
        float x = sc[0][j];
        #pragma unroll
        for (int i = 1; i < PPL; i++) x = fmaxf(x, sc[i][j]);
        xs[j] = LP == 16 ? x : fmaxf(x, dpp_f<0x128>(x));   // both positions of a 16-lane row
    }
    wave_heads<REP>(xs, m, true);
    #pragma unroll
    for (int j = 0; j < REP; j++) {
        const float mj = m[j] == -INFINITY ? 0.0f : m[j];   // a wave with no position left
        float ls = 0.0f;
        #pragma unroll
        for (int i = 0; i < PPL; i++) {
            const float p = __builtin_amdgcn_exp2f(sc[i][j] - mj);
            sc[i][j] = p;
            ls += p;
        }
        xs[j] = LP == 16 ? ls : ls + dpp_f<0x128>(ls);
    }
    wave_heads<REP>(xs, l, false);
    // weighted V over the same positions (masked weights are 0)
    float acc[REP][8];
    #pragma unroll
    for (int j = 0; j < REP; j++)
        #pragma unroll
        for (int e = 0; e < 8; e++) acc[j][e] = 0.0f;
    #pragma unroll
    for (int i = 0; i < PPL; i++) {
        const int t = t0 + grp + PS * i;
        float vf[8];
        unpack_h8(t == pos ? vnew : vw[i], vf);
        #pragma unroll
        for (int j = 0; j < REP; j++)
            #pragma unroll
            for (int e = 0; e < 8; e++) acc[j][e] += sc[i][j] * vf[e];
    }
    // sums over the wave's 4 rows (at D = 64 after the two halves of each
    // row), scattered: row r keeps dims l16*8 + 4h + r
    if constexpr (LP == 8) {
        #pragma unroll
        for (int j = 0; j < REP; j++)
            #pragma unroll
            for (int e = 0; e < 8; e++) acc[j][e] += dpp_f<0x128>(acc[j][e]);
    }
    const int row = (tid >> 4) & 3;
    #pragma unroll
    for (int j = 0; j < REP; j++)
        #pragma unroll
        for (int h = 0; h < 2; h++) {
            const float r4 = rows_sum4(acc[j][4 * h], acc[j][4 * h + 1], acc[j][4 * h + 2], acc[j][4 * h + 3]);
            if (LP == 16 || (tid & 15) < 8) red[wave][j][l16 * 8 + 4 * h + row] = r4;
        }
    if ((tid & 63) == 0) {
        #pragma unroll
        for (int j = 0; j < REP; j++) { wm[wave][j] = m[j]; wl[wave][j] = l[j]; }
    }
    __syncthreads();
    // combine the waves: rescale each by 2^(m_w - M)
    for (int idx = tid; idx < REP * D; idx += NT) {
        const int j = idx / D, d = idx % D;
        float M = wm[0][j];
        #pragma unroll
        for (int w = 1; w < NW; w++) M = fmaxf(M, wm[w][j]);
        float o = 0.0f, L = 0.0f;
        #pragma unroll
        for (int w = 0; w < NW; w++) {
            const float e = __builtin_amdgcn_exp2f(wm[w][j] - M);     // M is finite: wave 0 holds t0
            o += e * red[w][j][d];
            L += e * wl[w][j];
        }
        if (fold) {
            st_dev(po + ((size_t) j * a.nsplit + split) * D + d, o);
            if (d == 0) st_dev2(pml + (size_t) j * a.nsplit + split, make_float2(M, L));
        } else {
            po[((size_t) j * a.nsplit + split) * D + d] = o;
            if (d == 0) pml[(size_t) j * a.nsplit + split] = make_float2(M, L);
        }
    }
    if (fold) fold_merge(b);
    if (b + 1 < b1) __syncthreads();                  // red, wm and wl are the next entry's
    }
}

// RoPE of k at each sequence's position and the fp16 write of k and v into
// its slot's cache: the attention kernel's rotation and rounding, lane for
// lane, so the cache holds what that kernel would have written. Runs ahead of
// an attention launch with kv_written set, in which positions of one sequence
// read each other's k and v (prompt reading). Grid: one workgroup per
// sequence; block: D/8 lanes per kv head.
template <int D>
__device__ __forceinline__ void ropekv_body(const sml_kattn & a) {
    constexpr int LP = D / 8;
    const int b = blockIdx.x, tid = threadIdx.x, kh = tid / LP, l16 = tid % LP, kvd = a.n_kv * D;
    const float * ak = a.k + (size_t) b * a.qkv_stride + (size_t) kh * D + l16 * 8;
    const float * av = a.v + (size_t) b * a.qkv_stride + (size_t) kh * D + l16 * 8;
    float kn[8], vn[8];
    load_f8(ak, kn);
    load_f8(av, vn);
    const int pos = a.pos[b], half = D / 2;
    float cs[8], sn[8];
    load_f8(a.cos_t + (size_t) pos * half + (l16 & (LP / 2 - 1)) * 8, cs);
    load_f8(a.sin_t + (size_t) pos * half + (l16 & (LP / 2 - 1)) * 8, sn);
    rope8p<LP>(kn, cs, sn, l16 < LP / 2);
    v4u knew, vnew;
    #pragma unroll
    for (int e = 0; e < 4; e++) {
        knew[e] = (unsigned) f2h(kn[2 * e]) | ((unsigned) f2h(kn[2 * e + 1]) << 16);
        vnew[e] = (unsigned) f2h(vn[2 * e]) | ((unsigned) f2h(vn[2 * e + 1]) << 16);
    }
    GLOBAL uint16_t * kcache = (GLOBAL uint16_t *) (a.kc_slots ? a.kc_slots[a.slot[b]] + a.layer_off : a.kcache);
    GLOBAL uint16_t * vcache = (GLOBAL uint16_t *) (a.vc_slots ? a.vc_slots[a.slot[b]] + a.layer_off : a.vcache);
    *(GLOBAL v4u *) (kcache + (size_t) pos * kvd + (size_t) kh * D + l16 * 8) = knew;
    *(GLOBAL v4u *) (vcache + (size_t) pos * kvd + (size_t) kh * D + l16 * 8) = vnew;
}
extern "C" __global__ __launch_bounds__(128) void sml_ropekv(const sml_kattn a) { ropekv_body<HD>(a); }
extern "C" __global__ __launch_bounds__(128) void sml_ropekv_d64(const sml_kattn a) { ropekv_body<64>(a); }

#define ATTN_KERNEL(R) \
    extern "C" __global__ __launch_bounds__(256) void sml_attn_r##R(const sml_kattn a) { attn_body<R, 4, false>(a); } \
    extern "C" __global__ __launch_bounds__(256) void sml_attn_s64_r##R(const sml_kattn a) { attn_body<R, 4, false, 64>(a); } \
    extern "C" __global__ __launch_bounds__(512) void sml_attn8_r##R(const sml_kattn a) { attn_body<R, 8, false>(a); } \
    extern "C" __global__ __launch_bounds__(512) void sml_attnc8_r##R(const sml_kattn a) { attn_body<R, 8, true>(a); } \
    extern "C" __global__ __launch_bounds__(512) void sml_attn8_s32_r##R(const sml_kattn a) { attn_body<R, 8, false, 32>(a); } \
    extern "C" __global__ __launch_bounds__(512) void sml_attn8_s64_r##R(const sml_kattn a) { attn_body<R, 8, false, 64>(a); } \
    extern "C" __global__ __launch_bounds__(512) void sml_attnc8_s32_r##R(const sml_kattn a) { attn_body<R, 8, true, 32>(a); } \
    extern "C" __global__ __launch_bounds__(512) void sml_attnc8_s64_r##R(const sml_kattn a) { attn_body<R, 8, true, 64>(a); }
ATTN_KERNEL(1) ATTN_KERNEL(2) ATTN_KERNEL(3) ATTN_KERNEL(4) ATTN_KERNEL(5) ATTN_KERNEL(6) ATTN_KERNEL(7) ATTN_KERNEL(8)
// head_dim 64 (suffix _d64): 64 positions per round of 8 waves, so splits of 64 or 128
#define ATTN_KERNEL_D64(R) \
    extern "C" __global__ __launch_bounds__(256) void sml_attn_d64_r##R(const sml_kattn a) { attn_body<R, 4, false, ATTN_CHUNK, 64>(a); } \
    extern "C" __global__ __launch_bounds__(512) void sml_attn8_d64_r##R(const sml_kattn a) { attn_body<R, 8, false, ATTN_CHUNK, 64>(a); } \
    extern "C" __global__ __launch_bounds__(512) void sml_attnc8_d64_r##R(const sml_kattn a) { attn_body<R, 8, true, ATTN_CHUNK, 64>(a); } \
    extern "C" __global__ __launch_bounds__(512) void sml_attn8_s64_d64_r##R(const sml_kattn a) { attn_body<R, 8, false, 64, 64>(a); } \
    extern "C" __global__ __launch_bounds__(512) void sml_attnc8_s64_d64_r##R(const sml_kattn a) { attn_body<R, 8, true, 64, 64>(a); }
ATTN_KERNEL_D64(1) ATTN_KERNEL_D64(2) ATTN_KERNEL_D64(3) ATTN_KERNEL_D64(4) ATTN_KERNEL_D64(5) ATTN_KERNEL_D64(6)
ATTN_KERNEL_D64(7) ATTN_KERNEL_D64(8)

// Batched decode attention (sequences of one new position each, head_dim
// 128, 4 waves, splits of 128 positions): attn_body<REP, 4>'s arithmetic
// value for value, with its per-workgroup inputs spread over the threads.
// The one-entry body loads the REP query heads, k, v and the RoPE rows whole
// into every position lane (64 + 8 REP registers while the tile's 64
// arrive); here thread t holds dims t%64 and t%64 + 64 of query head t/64
// (and t/64 + 4), the rotation's own pair, wave 0 the pair of k and wave 1
// that of v. The rotated heads and the new position's fp16 k and v meet in
// LDS, then every lane takes its 8 dims of each (118 registers at REP 4
// against 191). (Two to eight consecutive splits a workgroup, the next
// split's K and V asked for as each set of registers frees, measured slower:
// 203 registers, 16 sequences at ~1k positions 3.07 -> 3.28-3.45 ms a step.)
template <int REP>
__device__ __forceinline__ void attnb_body(const sml_kattn & a) {
    constexpr int D = HD, LP = 16, NW = 4, PS = 64 * NW / LP, CH = ATTN_CHUNK, PPL = CH / PS;
    constexpr int QR = (REP + NW - 1) / NW;                     // query heads per thread in the prologue
    __shared__ float red[NW][REP][D];
    __shared__ float wm[NW][REP], wl[NW][REP];
    __shared__ __align__(16) float qs[REP][D];
    __shared__ __align__(16) uint16_t kvn[2][D];
    // grid (kv head, split, sequence): the kv heads of one split run side by
    // side, so together they read whole cache rows (n_kv x 256 bytes a
    // position)
    const int kh = blockIdx.x, qh0 = kh * REP, split = blockIdx.y, b = blockIdx.z, tid = threadIdx.x;
    const int wave = tid >> 6, grp = tid / LP, l16 = tid % LP, kvd = a.n_kv * D;
    const int pos = a.pos[b], T = pos + 1, t0 = split * CH, t1 = min(T, t0 + CH);
    float * blk = a.part + (size_t) b * a.n_head * a.nsplit * (D + 2);
    float * po = blk + (size_t) qh0 * a.nsplit * D;
    float2 * pml = (float2 *) (blk + (size_t) a.n_head * a.nsplit * D) + (size_t) qh0 * a.nsplit;
    // a split past the position writes empty partials only
    if (t0 >= T) {
        if (tid < REP) pml[(size_t) tid * a.nsplit + split] = make_float2(-INFINITY, 0.0f);
        return;
    }
    GLOBAL uint16_t * kcache = (GLOBAL uint16_t *) (a.kc_slots ? a.kc_slots[a.slot[b]] + a.layer_off : a.kcache);
    GLOBAL uint16_t * vcache = (GLOBAL uint16_t *) (a.vc_slots ? a.vc_slots[a.slot[b]] + a.layer_off : a.vcache);
    // the prologue's inputs first (loads return in order: the rotation runs
    // while the tile arrives)
    const int d = tid & 63;
    const float * qkv = a.q + (size_t) b * a.qkv_stride;
    const float c = a.cos_t[(size_t) pos * (D / 2) + d], sn = a.sin_t[(size_t) pos * (D / 2) + d];
    float x0[QR], x1[QR];
    #pragma unroll
    for (int r = 0; r < QR; r++) {
        const int j = wave + NW * r < REP ? wave + NW * r : 0;
        x0[r] = qkv[(size_t) (qh0 + j) * D + d];
        x1[r] = qkv[(size_t) (qh0 + j) * D + d + 64];
    }
    const float * kv = (wave == 0 ? a.k : a.v) + (size_t) b * a.qkv_stride + (size_t) kh * D;
    float y0 = 0.0f, y1 = 0.0f;
    if (wave < 2) { y0 = kv[d]; y1 = kv[d + 64]; }
    // the tile: positions t0 + grp + PS*i, clamped into the split's range
    // (the clamped ones are masked)
    v4u kw[PPL], vw[PPL];
    #pragma unroll
    for (int i = 0; i < PPL; i++) {
        int t = t0 + grp + PS * i;
        t = t < t1 ? t : t0;
        kw[i] = __builtin_nontemporal_load((const GLOBAL v4u *) (kcache + (size_t) t * kvd + (size_t) kh * D + l16 * 8));
    }
    #pragma unroll
    for (int i = 0; i < PPL; i++) {
        int t = t0 + grp + PS * i;
        t = t < t1 ? t : t0;
        vw[i] = __builtin_nontemporal_load((const GLOBAL v4u *) (vcache + (size_t) t * kvd + (size_t) kh * D + l16 * 8));
    }
    __builtin_amdgcn_sched_barrier(0);
    // rope8's pair rule: x0*c - x1*s = fma(x0, c, -(x1*s)), x0*s + x1*c = fma(x0, s, x1*c)
    #pragma unroll
    for (int r = 0; r < QR; r++) {
        const int j = wave + NW * r;
        if (j < REP) {
            qs[j][d] = __builtin_fmaf(x0[r], c, -(x1[r] * sn));
            qs[j][d + 64] = __builtin_fmaf(x0[r], sn, x1[r] * c);
        }
    }
    const bool here = t0 <= pos && pos < t1;
    if (wave == 0) {
        // rounded to fp32, then to fp16, as the one-entry body does: the empty
        // asm keeps the compiler from fusing each fma with its conversion
        // (v_fma_mixlo_f16 rounds once, to fp16, and differs at the ties)
        float r0 = __builtin_fmaf(y0, c, -(y1 * sn)), r1 = __builtin_fmaf(y0, sn, y1 * c);
        asm volatile("" : "+v"(r0), "+v"(r1));
        const uint16_t k0 = f2h(r0), k1 = f2h(r1);
        kvn[0][d] = k0;
        kvn[0][d + 64] = k1;
        if (here) {
            kcache[(size_t) pos * kvd + (size_t) kh * D + d] = k0;
            kcache[(size_t) pos * kvd + (size_t) kh * D + d + 64] = k1;
        }
    } else if (wave == 1) {
        const uint16_t v0 = f2h(y0), v1 = f2h(y1);
        kvn[1][d] = v0;
        kvn[1][d + 64] = v1;
        if (here) {
            vcache[(size_t) pos * kvd + (size_t) kh * D + d] = v0;
            vcache[(size_t) pos * kvd + (size_t) kh * D + d + 64] = v1;
        }
    }
    __syncthreads();
    float q[REP][8];
    #pragma unroll
    for (int j = 0; j < REP; j++) {
        const float4 u = *(const float4 *) &qs[j][l16 * 8], w = *(const float4 *) &qs[j][l16 * 8 + 4];
        q[j][0] = u.x; q[j][1] = u.y; q[j][2] = u.z; q[j][3] = u.w;
        q[j][4] = w.x; q[j][5] = w.y; q[j][6] = w.z; q[j][7] = w.w;
    }
    const float sl = a.inv * 1.44269504088896341f;
    // the new position's k and v in place of the (older) cache bytes the
    // tile read there
    if (here) {
        const v4u knew = *(const v4u *) &kvn[0][l16 * 8], vnew = *(const v4u *) &kvn[1][l16 * 8];
        #pragma unroll
        for (int i = 0; i < PPL; i++)
            if (t0 + grp + PS * i == pos) { kw[i] = knew; vw[i] = vnew; }
    }
    float sc[PPL][REP];
    #pragma unroll
    for (int i = 0; i < PPL; i++) {
        const int t = t0 + grp + PS * i;
        float kf[8];
        unpack_h8(kw[i], kf);
        #pragma unroll
        for (int j = 0; j < REP; j++) {
            float p = 0.0f;
            #pragma unroll
            for (int e = 0; e < 8; e++) p += q[j][e] * kf[e];
            p = sum16(p);
            sc[i][j] = t < t1 ? p * sl : -INFINITY;
        }
    }
    float m[REP], l[REP], xs[REP];
    #pragma unroll
    for (int j = 0; j < REP; j++) {
        float x = sc[0][j];
        #pragma unroll
        for (int i = 1; i < PPL; i++) x = fmaxf(x, sc[i][j]);
        xs[j] = x;
    }
    wave_heads<REP>(xs, m, true);
    #pragma unroll
    for (int j = 0; j < REP; j++) {
        const float mj = m[j] == -INFINITY ? 0.0f : m[j];
        float ls = 0.0f;
        #pragma unroll
        for (int i = 0; i < PPL; i++) {
            const float p = __builtin_amdgcn_exp2f(sc[i][j] - mj);
            sc[i][j] = p;
            ls += p;
        }
        xs[j] = ls;
    }
    wave_heads<REP>(xs, l, false);
    float acc[REP][8];
    #pragma unroll
    for (int j = 0; j < REP; j++)
        #pragma unroll
        for (int e = 0; e < 8; e++) acc[j][e] = 0.0f;
    #pragma unroll
    for (int i = 0; i < PPL; i++) {
        float vf[8];
        unpack_h8(vw[i], vf);
        #pragma unroll
        for (int j = 0; j < REP; j++)
            #pragma unroll
            for (int e = 0; e < 8; e++) acc[j][e] += sc[i][j] * vf[e];
    }
    const int row = (tid >> 4) & 3;
    #pragma unroll
    for (int j = 0; j < REP; j++)
        #pragma unroll
        for (int h = 0; h < 2; h++)
            red[wave][j][l16 * 8 + 4 * h + row] =
                rows_sum4(acc[j][4 * h], acc[j][4 * h + 1], acc[j][4 * h + 2], acc[j][4 * h + 3]);
    if ((tid & 63) == 0) {
        #pragma unroll
        for (int j = 0; j < REP; j++) { wm[wave][j] = m[j]; wl[wave][j] = l[j]; }
    }
    __syncthreads();
    for (int idx = tid; idx < REP * D; idx += 64 * NW) {
        const int j = idx / D, dd = idx % D;
        float M = wm[0][j];
        #pragma unroll
        for (int w = 1; w < NW; w++) M = fmaxf(M, wm[w][j]);
        float o = 0.0f, L = 0.0f;
        #pragma unroll
        for (int w = 0; w < NW; w++) {
            const float e = __builtin_amdgcn_exp2f(wm[w][j] - M);
            o += e * red[w][j][dd];
            L += e * wl[w][j];
        }
        po[((size_t) j * a.nsplit + split) * D + dd] = o;
        if (dd == 0) pml[(size_t) j * a.nsplit + split] = make_float2(M, L);
    }
}
#define ATTNB_KERNEL(R) \
    extern "C" __global__ __launch_bounds__(256) void sml_attnb_r##R(const sml_kattn a) { attnb_body<R>(a); }
ATTNB_KERNEL(1) ATTNB_KERNEL(2) ATTNB_KERNEL(3) ATTNB_KERNEL(4) ATTNB_KERNEL(5) ATTNB_KERNEL(6) ATTNB_KERNEL(7)
ATTNB_KERNEL(8)

// ---------------------------------------------------------------- prompt attention, a wave per position
//
// For prompt reading with the matrix-core products (level 2): a workgroup
// (split, kv head, up to 16 consecutive positions of one sequence) stages the
// split's K and V tile in LDS once; each of its 8 waves then takes whole
// positions (w, w + 8): the position's rotated q heads into LDS (the decode
// kernel's rope8, so the same rotated q), scores with a lane per tile
// position (two per lane), the base-2 softmax over the wave, and P.V with a
// lane per head dimension (two per lane). Past the staging no barrier is
// needed. It writes sml_attn's partials, so sml_attn_merge finishes the
// job; fp32 throughout, in its own summation order.
#define ATTNW_WAVES 8
#define ATTNW_ENTRIES 16
#define KROW (HD + 8)       // halves per K row in LDS: 16 bytes of padding, no bank conflicts

template <int REP>
__device__ __forceinline__ void attnw_body(const sml_kattn & a) {
    extern __shared__ __align__(16) uint8_t lds[];
    uint16_t * lk = (uint16_t *) lds;                                   // [ATTN_CHUNK][KROW]
    uint16_t * lv = lk + ATTN_CHUNK * KROW;                              // [ATTN_CHUNK][HD]
    float * lq = (float *) (lv + ATTN_CHUNK * HD);                       // [waves][REP][HD]
    float * lp = lq + ATTNW_WAVES * REP * HD;                            // [waves][ATTN_CHUNK][REP]
    const int kh = blockIdx.y, split = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kvd = a.n_kv * HD, half = HD / 2;
    const int b0 = blockIdx.z * ATTNW_ENTRIES, b1 = min(b0 + ATTNW_ENTRIES, a.nseq);
    const int t0 = split * ATTN_CHUNK, tlast = a.pos[b1 - 1] + 1;
    auto partials = [&](int b, float * & po, float2 * & pml) {
        float * blk = a.part + (size_t) b * a.n_head * a.nsplit * (HD + 2);
        po = blk + (size_t) kh * REP * a.nsplit * HD;
        pml = (float2 *) (blk + (size_t) a.n_head * a.nsplit * HD) + (size_t) kh * REP * a.nsplit;
    };
    if (t0 >= tlast) {                                // no entry reaches this split
        for (int idx = tid; idx < (b1 - b0) * REP; idx += ATTNW_WAVES * 64) {
            float * po;
            float2 * pml;
            partials(b0 + idx / REP, po, pml);
            pml[(size_t) (idx % REP) * a.nsplit + split] = make_float2(-INFINITY, 0.0f);
        }
        return;
    }
    const int tl = min(tlast, t0 + ATTN_CHUNK);
    const GLOBAL uint16_t * kcache = (const GLOBAL uint16_t *) (a.kc_slots ? a.kc_slots[a.slot[b0]] + a.layer_off : a.kcache);
    const GLOBAL uint16_t * vcache = (const GLOBAL uint16_t *) (a.vc_slots ? a.vc_slots[a.slot[b0]] + a.layer_off : a.vcache);
    // the tile: 16 16-byte words per row; rows past the last entry's position
    // repeat row t0 (finite, never weighted)
    for (int i = tid; i < ATTN_CHUNK * 16; i += ATTNW_WAVES * 64) {
        const int r = i >> 4, c = i & 15;
        const int t = t0 + r < tl ? t0 + r : t0;
        const size_t off = (size_t) t * kvd + (size_t) kh * HD + c * 8;
        *(v4u *) (lk + r * KROW + c * 8) = __builtin_nontemporal_load((const GLOBAL v4u *) (kcache + off));
        *(v4u *) (lv + r * HD + c * 8) = __builtin_nontemporal_load((const GLOBAL v4u *) (vcache + off));
    }
    __syncthreads();
    float * qw = lq + wave * REP * HD;
    float * pw = lp + wave * ATTN_CHUNK * REP;
    const int l16 = lane & 15, row = lane >> 4;
    const float sl = a.inv * 1.44269504088896341f;
    for (int b = b0 + wave; b < b1; b += ATTNW_WAVES) {
        const int pos = a.pos[b], T = pos + 1;
        float * po;
        float2 * pml;
        partials(b, po, pml);
        if (t0 >= T) {
            if (lane < REP) pml[(size_t) lane * a.nsplit + split] = make_float2(-INFINITY, 0.0f);
            continue;
        }
        const int n = min(T, t0 + ATTN_CHUNK) - t0;   // this entry's positions in the tile
        // rotated q: a 16-lane row per head, 8 dims per lane, as sml_attn does
        float cs[8], sn[8];
        load_f8(a.cos_t + (size_t) pos * half + (l16 & 7) * 8, cs);
        load_f8(a.sin_t + (size_t) pos * half + (l16 & 7) * 8, sn);
        #pragma unroll
        for (int j0 = 0; j0 < REP; j0 += 4) {
            const int j = j0 + row;
            float q[8];
            load_f8(a.q + (size_t) b * a.qkv_stride + (size_t) (kh * REP + (j < REP ? j : 0)) * HD + l16 * 8, q);
            rope8(q, cs, sn, l16 < 8);
            if (j < REP) {
                *(float4 *) (qw + j * HD + l16 * 8) = make_float4(q[0], q[1], q[2], q[3]);
                *(float4 *) (qw + j * HD + l16 * 8 + 4) = make_float4(q[4], q[5], q[6], q[7]);
            }
        }
        // scores of tile positions lane and lane + 64
        float s0[REP], s1[REP];
        #pragma unroll
        for (int j = 0; j < REP; j++) { s0[j] = 0.0f; s1[j] = 0.0f; }
        #pragma unroll 4
        for (int c = 0; c < HD / 8; c++) {
            float k0[8], k1[8];
            unpack_h8(*(const v4u *) (lk + lane * KROW + c * 8), k0);
            unpack_h8(*(const v4u *) (lk + (lane + 64) * KROW + c * 8), k1);
            #pragma unroll
            for (int j = 0; j < REP; j++) {
                float qv[8];
                load_f8(qw + j * HD + c * 8, qv);
                #pragma unroll
                for (int e = 0; e < 8; e++) { s0[j] += qv[e] * k0[e]; s1[j] += qv[e] * k1[e]; }
            }
        }
        // base-2 softmax per head over the wave (position t0 is valid: lane 0)
        float mj[REP], lj[REP];
        #pragma unroll
        for (int j = 0; j < REP; j++) {
            const float x0 = lane < n ? s0[j] * sl : -INFINITY;
            const float x1 = lane + 64 < n ? s1[j] * sl : -INFINITY;
            const float m = wave_max(fmaxf(x0, x1));
            const float p0 = __builtin_amdgcn_exp2f(x0 - m), p1 = __builtin_amdgcn_exp2f(x1 - m);
            mj[j] = m;
            lj[j] = wave_sum(p0 + p1);
            pw[lane * REP + j] = p0;
            pw[(lane + 64) * REP + j] = p1;
        }
        // P.V for dims 2 lane, 2 lane + 1
        float o0[REP], o1[REP];
        #pragma unroll
        for (int j = 0; j < REP; j++) { o0[j] = 0.0f; o1[j] = 0.0f; }
        for (int t = 0; t < n; t++) {
            const uint32_t vv = *(const uint32_t *) (lv + t * HD + 2 * lane);
            const float v0 = h2f((uint16_t) (vv & 0xFFFFu)), v1 = h2f((uint16_t) (vv >> 16));
            #pragma unroll
            for (int j = 0; j < REP; j++) {
                const float pj = pw[t * REP + j];
                o0[j] += pj * v0;
                o1[j] += pj * v1;
            }
        }
        #pragma unroll
        for (int j = 0; j < REP; j++) {
            *(float2 *) (po + ((size_t) j * a.nsplit + split) * HD + 2 * lane) = make_float2(o0[j], o1[j]);
            if (lane == 0) pml[(size_t) j * a.nsplit + split] = make_float2(mj[j], lj[j]);
        }
    }
}

#define ATTNW_KERNEL(R) \
    extern "C" __global__ __launch_bounds__(64 * ATTNW_WAVES) void sml_attnw_r##R(const sml_kattn a) { attnw_body<R>(a); }
ATTNW_KERNEL(1) ATTNW_KERNEL(2) ATTNW_KERNEL(3) ATTNW_KERNEL(4) ATTNW_KERNEL(5) ATTNW_KERNEL(6) ATTNW_KERNEL(7) ATTNW_KERNEL(8)

// ---------------------------------------------------------------- prompt attention on MFMA (flash form)
//
// For prompt reading at level 2: the entries of a launch are consecutive
// positions of one sequence whose K and V rows sml_ropekv has already
// rotated and written to the cache (fp16). A workgroup takes 16 entries
// (query rows) and one kv head, one wave per query head of the group, and
// walks the KV positions of its split in blocks of 64 with an online
// softmax, on v_mfma_f32_16x16x32_f16 (lane l: A row / B column l%16, k =
// 8(l/16)..+7; D rows 4(l/16)..+3 of column l%16):
//  - S^T = K Q^T: A = the block's K rows (fp16 from the cache), B = the
//    wave's rotated q (rotated as rope8 does) as two fp16 parts, q_hi =
//    fp16(q) and q_lo = fp16(q - q_hi), so the scores carry q to ~2^-22; a
//    lane then holds query l%16 at KV positions 4(l/16)..+3 of each 16-row
//    tile;
//  - the scores times 1/sqrt(hd) log2(e) in fp32, masked past each entry's
//    position; the running max and sum per query in base 2;
//  - O += P V: A = P straight from the S^T layout (the MFMA's k slots
//    8(l/16)..+7 hold KV rows 4(l/16)..+3 of two 16-row tiles), as fp16
//    high and low parts like q (P rounded once to fp16, against a sum of
//    the unrounded P, moved a MoE prompt enough to flip a routed expert),
//    B = V from an LDS copy transposed to [dim][position] at staging, the
//    same slot order.
// One split: the output is written directly; several (few query blocks or
// kv heads, so the grid still fills the chip): sml_attn's partials, merged
// by sml_attn_merge. fp32 accumulation in its own order: graded as level-2
// prompt reading is.
#define FA_KB 64                      // KV positions per block
#define FA_KROW 272                   // LDS bytes per K row (256 + 16)
#define FA_VROW 144                   // LDS bytes per transposed V row (one dim, 64 positions + 16)
#define FA_STAGE (FA_KB * FA_KROW + HD * FA_VROW)
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

template <int REP>
__device__ void attnf_body(const sml_kattn & a) {
    extern __shared__ __align__(16) uint8_t lds[];
    constexpr int NT = 64 * REP;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 4, i16 = lane & 15;
    const int kh = blockIdx.y, h = kh * REP + wave;
    const int b0 = blockIdx.x * 16, nb = min(16, a.nseq - b0);
    const int kvd = a.n_kv * HD, half = HD / 2;
    const GLOBAL uint16_t * kcache = (const GLOBAL uint16_t *) (a.kc_slots ? a.kc_slots[a.slot[b0]] + a.layer_off : a.kcache);
    const GLOBAL uint16_t * vcache = (const GLOBAL uint16_t *) (a.vc_slots ? a.vc_slots[a.slot[b0]] + a.layer_off : a.vcache);
    // this split's KV range, cut at the block's last position
    const int chk = a.fchunk;
    const int t_lo = blockIdx.z * chk, t_end = min(t_lo + chk, a.pos[b0 + nb - 1] + 1);
    // the lane's query (entry b0 + i16, clamped) and its position
    const int bq = b0 + min(i16, nb - 1), posq = a.pos[bq];
    // rotated q of head h, dims 32c + 8g + e, as fp16 B operands (hi, lo)
    v8h qb[4], ql[4];
    {
        float x[4][8];
        const float * qp = a.q + (size_t) bq * a.qkv_stride + (size_t) h * HD;
        #pragma unroll
        for (int c = 0; c < 4; c++) load_f8(qp + 32 * c + 8 * g, x[c]);
        #pragma unroll
        for (int c = 0; c < 2; c++) {
            float cs[8], sn[8];
            load_f8(a.cos_t + (size_t) posq * half + 32 * c + 8 * g, cs);
            load_f8(a.sin_t + (size_t) posq * half + 32 * c + 8 * g, sn);
            #pragma unroll
            for (int e = 0; e < 8; e++) {
                const float lo = x[c][e], hi = x[c + 2][e];
                x[c][e] = __builtin_fmaf(lo, cs[e], -(hi * sn[e]));        // rope8's fused forms
                x[c + 2][e] = __builtin_fmaf(lo, sn[e], hi * cs[e]);
            }
        }
        #pragma unroll
        for (int c = 0; c < 4; c++)
            #pragma unroll
            for (int e = 0; e < 8; e++) {
                qb[c][e] = (_Float16) x[c][e];
                ql[c][e] = (_Float16) (x[c][e] - (float) qb[c][e]);
            }
    }
    const float sl = a.inv * 1.44269504088896341f;
    float m_run = -INFINITY, l_run = 0.0f;                    // for query i16 (the same in its 4 lanes)
    v4f o[8];
    #pragma unroll
    for (int dt = 0; dt < 8; dt++) o[dt] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

    // staging: K rows as they are ([pos][dim], 16-byte words), V transposed
    // to [dim][pos]; words of positions past the range repeat its first row
    v4u kw[(FA_KB * 16 + NT - 1) / NT], vw[(FA_KB * 16 + NT - 1) / NT];
    constexpr int NW = (FA_KB * 16 + NT - 1) / NT;
    auto fetch = [&](int t0) {
        #pragma unroll
        for (int i = 0; i < NW; i++) {
            const int w = tid + i * NT;
            if (w < FA_KB * 16) {
                const int r = w >> 4, c = w & 15;
                const int t = t0 + r < t_end ? t0 + r : t0;
                const size_t off = (size_t) t * kvd + (size_t) kh * HD + c * 8;
                kw[i] = *(const GLOBAL v4u *) (kcache + off);
                vw[i] = *(const GLOBAL v4u *) (vcache + off);
            }
        }
    };
    auto stage = [&](int buf) {
        uint8_t * kb = lds + (size_t) buf * FA_STAGE;
        uint8_t * vb = kb + FA_KB * FA_KROW;
        #pragma unroll
        for (int i = 0; i < NW; i++) {
            const int w = tid + i * NT;
            if (w < FA_KB * 16) {
                const int r = w >> 4, c = w & 15;
                *(v4u *) (kb + r * FA_KROW + c * 16) = kw[i];
                #pragma unroll
                for (int e = 0; e < 4; e++) {
                    *(uint16_t *) (vb + (c * 8 + 2 * e) * FA_VROW + r * 2) = (uint16_t) (vw[i][e] & 0xFFFFu);
                    *(uint16_t *) (vb + (c * 8 + 2 * e + 1) * FA_VROW + r * 2) = (uint16_t) (vw[i][e] >> 16);
                }
            }
        }
    };
    auto compute = [&](int buf, int t0) {
        const uint8_t * kb = lds + (size_t) buf * FA_STAGE;
        const uint8_t * vb = kb + FA_KB * FA_KROW;
        // S^T: 4 tiles of 16 positions x 16 queries
        v4f s[4];
        #pragma unroll
        for (int j = 0; j < 4; j++) {
            s[j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
            #pragma unroll
            for (int c = 0; c < 4; c++) {
                const v8h ka = *(const v8h *) (kb + (16 * j + i16) * FA_KROW + (32 * c + 8 * g) * 2);
                s[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qb[c], s[j], 0, 0, 0);
                s[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, ql[c], s[j], 0, 0, 0);
            }
        }
        // scale, mask and the block's max for the lane's query
        float mx = -INFINITY;
        #pragma unroll
        for (int j = 0; j < 4; j++)
            #pragma unroll
            for (int r = 0; r < 4; r++) {
                const int t = t0 + 16 * j + 4 * g + r;
                const float v = t < t_end && t <= posq ? s[j][r] * sl : -INFINITY;
                s[j][r] = v;
                mx = fmaxf(mx, v);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float m_new = fmaxf(m_run, mx);
        const float mu = m_new == -INFINITY ? 0.0f : m_new;   // no position yet: keep zeros
        const float alpha = __builtin_amdgcn_exp2f(m_run - mu);
        float ls = 0.0f;
        v8h pa[2], pl[2];
        #pragma unroll
        for (int j = 0; j < 4; j++)
            #pragma unroll
            for (int r = 0; r < 4; r++) {
                const float p = __builtin_amdgcn_exp2f(s[j][r] - mu);
                ls += p;
                const _Float16 ph = (_Float16) p;
                pa[j >> 1][4 * (j & 1) + r] = ph;
                pl[j >> 1][4 * (j & 1) + r] = (_Float16) (p - (float) ph);
            }
        ls += __shfl_xor(ls, 16);
        ls += __shfl_xor(ls, 32);
        l_run = l_run * alpha + ls;
        m_run = m_new;
        // rescale O: the lane's rows are queries 4g..4g+3
        float al[4];
        #pragma unroll
        for (int r = 0; r < 4; r++) al[r] = __shfl(alpha, 4 * g + r);
        #pragma unroll
        for (int dt = 0; dt < 8; dt++)
            #pragma unroll
            for (int r = 0; r < 4; r++) o[dt][r] *= al[r];
        // O += P V: per 32 positions u, k slots 8g..8g+3 are rows 4g..4g+3
        // of tile 2u, 8g+4..8g+7 those of tile 2u+1
        #pragma unroll
        for (int dt = 0; dt < 8; dt++) {
            const uint8_t * vr = vb + (16 * dt + i16) * FA_VROW;
            #pragma unroll
            for (int u = 0; u < 2; u++) {
                const v2u lo = *(const v2u *) (vr + (32 * u + 4 * g) * 2);
                const v2u hi = *(const v2u *) (vr + (32 * u + 16 + 4 * g) * 2);
                const v4u w4 = {lo.x, lo.y, hi.x, hi.y};
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa[u], __builtin_bit_cast(v8h, w4), o[dt], 0, 0, 0);
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pl[u], __builtin_bit_cast(v8h, w4), o[dt], 0, 0, 0);
            }
        }
    };

    int buf = 0;
    if (t_lo < t_end) {
        fetch(t_lo);
        stage(0);
        __syncthreads();
        for (int t0 = t_lo; t0 < t_end; t0 += FA_KB) {
            const bool more = t0 + FA_KB < t_end;
            if (more) fetch(t0 + FA_KB);
            compute(buf, t0);
            if (more) stage(buf ^ 1);
            __syncthreads();
            buf ^= 1;
        }
    }

    // the lane's rows: queries 4g..4g+3, dims 16dt + i16
    const bool one = gridDim.z == 1;
    float lq[4], mq[4];
    #pragma unroll
    for (int r = 0; r < 4; r++) { lq[r] = __shfl(l_run, 4 * g + r); mq[r] = __shfl(m_run, 4 * g + r); }
    #pragma unroll
    for (int r = 0; r < 4; r++) {
        const int q = 4 * g + r;
        if (q >= nb) continue;
        const int b = b0 + q;
        if (one) {
            float * out = a.out + (size_t) b * a.n_head * HD + (size_t) h * HD;
            #pragma unroll
            for (int dt = 0; dt < 8; dt++) out[16 * dt + i16] = o[dt][r] / lq[r];
        } else {
            float * blk = a.part + (size_t) b * a.n_head * a.nsplit * (HD + 2);
            float * po = blk + ((size_t) h * a.nsplit + blockIdx.z) * HD;
            float2 * pml = (float2 *) (blk + (size_t) a.n_head * a.nsplit * HD) + (size_t) h * a.nsplit + blockIdx.z;
            #pragma unroll
            for (int dt = 0; dt < 8; dt++) po[16 * dt + i16] = o[dt][r];
            if (i16 == 0) *pml = make_float2(mq[r], lq[r]);
        }
    }
}

#define ATTNF_KERNEL(R) \
    extern "C" __global__ __launch_bounds__(64 * R) void sml_attnf_r##R(const sml_kattn a) { attnf_body<R>(a); }
ATTNF_KERNEL(1) ATTNF_KERNEL(2) ATTNF_KERNEL(3) ATTNF_KERNEL(4) ATTNF_KERNEL(5) ATTNF_KERNEL(6) ATTNF_KERNEL(7) ATTNF_KERNEL(8)

// The merge as its own launch (grid: n_head workgroups of HD threads, z:
// the sequence).
extern "C" __global__ __launch_bounds__(HD) void sml_attn_merge(const sml_kattn a) {
    merge_head<false>(a, blockIdx.z, blockIdx.x, threadIdx.x);
}
extern "C" __global__ __launch_bounds__(64) void sml_attn_merge_d64(const sml_kattn a) {
    merge_head<false, 64>(a, blockIdx.z, blockIdx.x, threadIdx.x);
}

// The merge with its output quantized per 256 values (the rule of
// sml_normq2's per256 form, sml/sml-kernel.c:165-172): two heads of HD = 128
// make one superblock, a workgroup of 256 threads per head pair (grid:
// n_head / 2, z: the sequence); wave w holds dims (w & 1) * 64.. of head
// 2 * blockIdx.x + (w >> 1), as sml_normq2's wave w holds values 64 w.. of
// its superblock, so the maxima, codes and sums are that kernel's bit for bit.
extern "C" __global__ __launch_bounds__(256) void sml_attn_merge_sb(const sml_kattn a) {
    __shared__ float wm[4];
    const int tid = threadIdx.x, wave = tid >> 6, b = blockIdx.z;
    const int h = blockIdx.x * 2 + (wave >> 1), d = (wave & 1) * 64 + (tid & 63);
    const float r = merge_value<false>(a, b, h, d);
    const float m = wave_max(fabsf(r));
    if ((tid & 63) == 0) wm[wave] = m;
    __syncthreads();
    const float amax = fmaxf(fmaxf(wm[0], wm[1]), fmaxf(wm[2], wm[3]));
    const float s = amax / 127.0f;
    const float is = s > 0.0f ? 1.0f / s : 0.0f;
    const int t = quant1(r, is);
    const int sum = isum32(t);
    const size_t ob = (size_t) b * a.n_head * HD, j = (size_t) blockIdx.x * 256 + tid;
    a.q_out[ob + j] = (int8_t) t;
    if ((tid & 31) == 0) { a.s_out[(ob + j) / 32] = s; a.u_out[(ob + j) / 32] = sum; }
}

// ---------------------------------------------------------------- attention in the reference's order
//
// The exact mode's decode attention: the float operations of the
// reference's x86 build, in its order (sml/sml-run.c:180-287,339-372), so
// the output equals its bit for bit. Two launches.
//
// sml_attnx_scores (splits of 128 positions x kv heads, 256 threads): RoPE
// of the kv head's query heads into LDS and, in the split holding the
// position, of k, whose fp16 row and v's are written to the cache (the
// fused products of that build: x0*c - x1*s = fma(x0, c, -(x1*s)),
// x0*s + x1*c = fma(x0, s, x1*c)); then a thread per position computes its
// score for every other query head: eight FMA lanes over the head's dims
// (lane j takes dims j, j+8, ...), folded ((l0+l4)+(l1+l5)) +
// ((l2+l6)+(l3+l7)), times 1/sqrt(hd) (sml/sml-run.c:186-206).
//
// sml_attnx_pv (a workgroup per query head, 8 waves): the scores into LDS,
// their maximum, expf of each score less it (expf_tab: the C library's
// bits), their sum in the order of a serial float chain, one reciprocal and
// the products (sml/sml-run.c:280-287); then output dim d as one FMA chain
// over the positions in order, p_t*v_t[d] + o (sml/sml-run.c:209-229).
//
// A dependent float operation issues every ~8.4 cycles on gfx950 (v_add_f32,
// v_fmac_f32; ~9.5 for v_fma_mix_f32; 2.4 GHz), so a 4096-step chain costs
// at least ~14.5 us. The P.V chains are run as such (one output dim per
// lane), reading V from a three-tile LDS ring of fp16 position pairs that
// loader waves fill with ATTNX_PF tiles of loads in flight. The softmax sum
// is computed exactly but mostly in parallel (serial_sum_seg below). With
// q_out the workgroup also quantizes its head per 32 for the o product (the
// arithmetic of sml_normq2 without a norm, so its codes are bit for bit).
#define ATTNX_CH 128          // positions per scores workgroup
#define ATTNX_TP 64           // positions per V tile
#define ATTNX_PF 6            // V tiles in flight
#define ATTNX_THREADS 512
#define ATTNX_SEG 64          // positions per segment of the softmax sum
#define ATTNX_MAXSEG 256      // 16384 positions

// The serial float sum s = ((e0 + e1) + e2) + ... of n >= 0 values (all >= 0,
// finite) in LDS, exactly, mostly in parallel; called by every thread of
// the workgroup, the result is returned to all.
//
// While the running sum s stays in one binade [2^E, 2^(E+1)), its floats
// are the multiples m*u of u = 2^(E-23), m in [2^23, 2^24), and one step
// rounds s + e to the nearest multiple: m += round(e/u), unless e/u lies
// exactly halfway (then the even neighbour of m + floor(e/u) wins, which
// depends on m). So for a segment of 64 values that starts in binade E,
// contains no such tie and ends with m + K < 2^24, the chain adds exactly
// K = sum of round(e/u) to m. Each segment's K is computed in parallel for
// the binade of its exact prefix sum and the next one up (the chain's
// sum lies within 2^-12 of it, relatively); one wave then walks the
// segments from s = 0, jumping over each run of segments where those
// conditions hold (one prefix sum of their Ks over the lanes) and running
// the float chain over the values of a segment where they do not (the
// first segments, a binade crossing, a tie). The result is the chain's bit
// for bit; tests/test_gpu_exact.py checks it against the oracle's chain on
// inputs with planted ties and crossings.
__device__ __forceinline__ float serial_sum_seg(const float * e, int n, float * fsum, int * segk, int * sege,
                                                float * out) {
    const int tid = threadIdx.x, nseg = (n + ATTNX_SEG - 1) / ATTNX_SEG;
    constexpr int TPS = 8, EPT = ATTNX_SEG / TPS;            // threads per segment, values per thread
    // each segment's sum (8 threads, 8 values each, DPP within the 8 lanes)
    for (int j0 = 0; j0 < nseg; j0 += ATTNX_THREADS / TPS) {
        const int j = j0 + tid / TPS, i0 = j * ATTNX_SEG + (tid % TPS) * EPT;
        float d = 0.0f;
        #pragma unroll
        for (int i = 0; i < EPT; i++) d += i0 + i < n ? e[i0 + i] : 0.0f;
        d += dpp_f<0xB1>(d);
        d += dpp_f<0x4E>(d);
        d += dpp_f<0x141>(d);
        if (j < nseg && tid % TPS == 0) fsum[j] = d;
    }
    __syncthreads();
    // their exclusive prefix, by wave 0 (4 segments a lane, then a scan over
    // the lanes): a binade guess (a float sum in any order is close enough:
    // the candidates are the guess and the binade above, and every use of a
    // candidate is checked exactly)
    if (tid < WAVE) {
        float d[ATTNX_MAXSEG / WAVE];
        float t = 0.0f;
        #pragma unroll
        for (int i = 0; i < ATTNX_MAXSEG / WAVE; i++) {
            const int j = tid * (ATTNX_MAXSEG / WAVE) + i;
            d[i] = t;
            t += j < nseg ? fsum[j] : 0.0f;
        }
        const float before = wave_scan_f(t) - t;
        #pragma unroll
        for (int i = 0; i < ATTNX_MAXSEG / WAVE; i++) {
            const int j = tid * (ATTNX_MAXSEG / WAVE) + i;
            if (j < nseg) fsum[j] = before + d[i];
        }
    }
    __syncthreads();
    // K of each segment for binades E and E+1 (segk[2j + c]; -1: not usable).
    // e*2^(23-E) is exact in float (a power-of-two scaling; a result past the
    // float range is inf and fails the test, one below the normal range is
    // far under 1/2 and rounds to 0 either way)
    for (int j0 = 0; j0 < nseg; j0 += ATTNX_THREADS / TPS) {
        const int j = j0 + tid / TPS, i0 = j * ATTNX_SEG + (tid % TPS) * EPT;
        const float st = j < nseg ? fsum[j] : 0.0f;
        const int eg = st > 0.0f && st < 1e30f ? ilogbf(st) : -1000;   // not finite: never matched
        float x[EPT];
        #pragma unroll
        for (int i = 0; i < EPT; i++) x[i] = i0 + i < n ? e[i0 + i] : 0.0f;
        #pragma unroll
        for (int c = 0; c < 2; c++) {
            int ks = 0, bad = eg + c <= -126 ? 1 : 0;
            #pragma unroll
            for (int i = 0; i < EPT; i++) {
                const float y = __builtin_amdgcn_ldexpf(x[i], 23 - (eg + c));
                bad |= (y >= 16777216.0f) | (y - floorf(y) == 0.5f) | (y != y);
                ks += y < 16777216.0f ? (int) __builtin_rintf(y) : 0;
            }
            ks += dpp_i<0xB1>(ks); ks += dpp_i<0x4E>(ks); ks += dpp_i<0x141>(ks);
            bad |= dpp_i<0xB1>(bad); bad |= dpp_i<0x4E>(bad); bad |= dpp_i<0x141>(bad);
            if (j < nseg && tid % TPS == 0) segk[2 * j + c] = bad || ks >= (1 << 24) ? -1 : ks;
        }
        if (j < nseg && tid % TPS == 0) sege[j] = eg;
    }
    __syncthreads();
    if (tid < WAVE) {
        // the walk, by wave 0. From segment j with the sum's bits sb (binade
        // E), lane l takes segment j+l's K for E where its table has one;
        // a prefix sum of the Ks over the lanes gives the longest run of
        // segments that the chain crosses inside binade E with no tie, and
        // the walk jumps over it. The segment that ends the run (a tie, a
        // carry into the next binade, a binade the table lacks, a sum of 0)
        // is added as the float chain, its values read 16 at a time, the
        // next 16 in flight while the current 16 are added.
        unsigned sb = 0;                                  // the bits of the sum
        int j = 0;
        while (j < nseg) {
            const int jl = j + tid;
            const int m0 = (int) ((sb & 0x7FFFFFu) | 0x800000u);
            int k = -1;
            if (sb >= 0x00800000u && jl < nseg) {
                const int c = (int) (sb >> 23) - 127 - sege[jl];
                k = c == 0 ? segk[2 * jl] : c == 1 ? segk[2 * jl + 1] : -1;
            }
            const int P = wave_scan_i(max(k, 0));          // m0 + P < 2^31: each K < 2^24, 64 of them
            const unsigned long long ok = __builtin_amdgcn_ballot_w64(k >= 0 && m0 + P < (1 << 24));
            const int f = ~ok == 0ull ? WAVE : (int) __builtin_ctzll(~ok);
            if (f > 0) {
                const int pf = __builtin_amdgcn_readlane(P, f - 1);
                sb = (sb & 0xFF800000u) | ((unsigned) (m0 + pf) & 0x7FFFFFu);
                j += f;
            }
            if (f == WAVE || j >= nseg) continue;
            float s = __builtin_bit_cast(float, sb);
            const int i0 = j * ATTNX_SEG, i1 = min(n, i0 + ATTNX_SEG);
            if (i1 - i0 == ATTNX_SEG) {
                const float4 * q = (const float4 *) (e + i0);
                float4 c4[2][4];
                #pragma unroll
                for (int r = 0; r < 4; r++) c4[0][r] = q[r];
                #pragma unroll
                for (int bl = 0; bl < ATTNX_SEG / 16; bl++) {
                    if (bl + 1 < ATTNX_SEG / 16) {
                        #pragma unroll
                        for (int r = 0; r < 4; r++) c4[(bl + 1) & 1][r] = q[4 * (bl + 1) + r];
                    }
                    #pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const float4 v = c4[bl & 1][r];
                        s = s + v.x; s = s + v.y; s = s + v.z; s = s + v.w;
                    }
                }
            } else {
                for (int i = i0; i < i1; i++) s = s + e[i];
            }
            sb = __builtin_amdgcn_readfirstlane(__builtin_bit_cast(unsigned, s));
            j++;
        }
        if (tid == 0) *out = __builtin_bit_cast(float, sb);
    }
    __syncthreads();
    return *out;
}

// serial_sum_seg over n values in global memory (its test entry point)
extern "C" __global__ __launch_bounds__(ATTNX_THREADS) void sml_sum_seg(const sml_ksum a) {
    extern __shared__ __align__(16) float ev[];
    __shared__ float fsum[ATTNX_MAXSEG];
    __shared__ int segk[2 * ATTNX_MAXSEG], sege[ATTNX_MAXSEG];
    __shared__ float tot;
    for (int i = threadIdx.x; i < a.n; i += ATTNX_THREADS) ev[i] = a.x[i];
    __syncthreads();
    const float s = serial_sum_seg(ev, a.n, fsum, segk, sege, &tot);
    if (threadIdx.x == 0) *a.out = s;
}

// K tile rows in LDS: 256 bytes and 16 of padding, so the 8 lanes a
// 16-byte read serves per cycle start on different banks
#define ATTNX_KROW 136
extern "C" __global__ __launch_bounds__(256) void sml_attnx_scores(const sml_kattnx a) {
    #pragma clang fp contract(off)
    __shared__ float qs[ATTN_MAXREP][HD];
    __shared__ __align__(16) uint16_t kt[ATTNX_CH * ATTNX_KROW];
    const int kh = blockIdx.y, t0 = blockIdx.x * ATTNX_CH, tid = threadIdx.x, b = blockIdx.z;
    const int pos = a.pos[b], n = pos + 1, rep = a.n_head / a.n_kv, kvd = a.n_kv * HD;
    if (t0 >= n) return;
    // own: this split holds the position and rotates and writes its k and v
    const bool own = pos < t0 + ATTNX_CH && !a.kv_written;
    const float * aq = a.q + (size_t) b * a.qkv_stride, * ak = a.k + (size_t) b * a.qkv_stride;
    const float * avv = a.v + (size_t) b * a.qkv_stride;
    float * scb = a.sc + (size_t) b * a.n_head * a.n_ctx;
    GLOBAL uint16_t * kc = (GLOBAL uint16_t *) a.kc, * vc = (GLOBAL uint16_t *) a.vc;
    // RoPE inputs first, then the split's K tile, coalesced (16 lanes a row,
    // rows past the position load row t0 and are never read): loads complete
    // in order. Pair idx = tid + 256r is dim pair i of query head j (j = rep:
    // k, in the owning split only); indices past the end load a pair in range
    // and are dropped.
    constexpr int RR = (ATTN_MAXREP + 1) * (HD / 2) / 256 + 1;
    constexpr int KC = ATTNX_CH * HD / 8 / 256;               // 16-byte K chunks per thread
    const int npair = (rep + (own ? 1 : 0)) * (HD / 2);
    const float * cs = a.cos_t + (size_t) pos * (HD / 2), * sn = a.sin_t + (size_t) pos * (HD / 2);
    float x0[RR], x1[RR], c[RR], sv[RR];
    #pragma unroll
    for (int r = 0; r < RR; r++) {
        const int idx = min(tid + 256 * r, npair - 1), j = idx / (HD / 2), i = idx % (HD / 2);
        const float * src = j < rep ? aq + (size_t) (kh * rep + j) * HD : ak + (size_t) kh * HD;
        x0[r] = src[i];
        x1[r] = src[i + HD / 2];
        c[r] = cs[i];
        sv[r] = sn[i];
    }
    const float vnew = avv[(size_t) kh * HD + (tid & (HD - 1))];     // used by the owning split only
    v4u kw[KC];
    #pragma unroll
    for (int r = 0; r < KC; r++) {
        const int ch = tid + 256 * r, tp = t0 + ch / 16;
        kw[r] = __builtin_nontemporal_load((const GLOBAL v4u *) (kc + (size_t) (tp < n ? tp : t0) * kvd +
                                                                (size_t) kh * HD + (ch % 16) * 8));
    }
    // the K tile first, then the position's own row over its stale copy
    #pragma unroll
    for (int r = 0; r < KC; r++) {
        const int ch = tid + 256 * r;
        if (!own || t0 + ch / 16 != pos) *(v4u *) (kt + (ch / 16) * ATTNX_KROW + (ch % 16) * 8) = kw[r];
    }
    #pragma unroll
    for (int r = 0; r < RR; r++) {
        const int idx = tid + 256 * r;
        if (idx >= npair) break;
        const int j = idx / (HD / 2), i = idx % (HD / 2);
        const float y0 = __builtin_fmaf(x0[r], c[r], -(x1[r] * sv[r]));
        const float y1 = __builtin_fmaf(x0[r], sv[r], x1[r] * c[r]);
        if (j < rep) {
            qs[j][i] = y0;
            qs[j][i + HD / 2] = y1;
        } else {
            // the position's own row: to the cache, and the same bits into the tile
            const uint16_t h0 = f2h(y0), h1 = f2h(y1);
            kc[(size_t) pos * kvd + (size_t) kh * HD + i] = h0;
            kc[(size_t) pos * kvd + (size_t) kh * HD + i + HD / 2] = h1;
            kt[(pos - t0) * ATTNX_KROW + i] = h0;
            kt[(pos - t0) * ATTNX_KROW + i + HD / 2] = h1;
        }
    }
    if (own && tid < HD) vc[(size_t) pos * kvd + (size_t) kh * HD + tid] = f2h(vnew);
    __syncthreads();
    const int t = t0 + (tid & (ATTNX_CH - 1));
    if (t >= n) return;
    v4u kr[HD / 8];
    #pragma unroll
    for (int i = 0; i < HD / 8; i++) kr[i] = *(const v4u *) (kt + (tid & (ATTNX_CH - 1)) * ATTNX_KROW + 8 * i);
    for (int j = tid / ATTNX_CH; j < rep; j += 256 / ATTNX_CH) {
        float l[8] = { 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f };
        #pragma unroll
        for (int i = 0; i < HD / 8; i++) {
            float kf[8];
            unpack_h8(kr[i], kf);
            #pragma unroll
            for (int e = 0; e < 8; e++) l[e] = __builtin_fmaf(qs[j][8 * i + e], kf[e], l[e]);
        }
        scb[(size_t) (kh * rep + j) * a.n_ctx + t] =
            (((l[0] + l[4]) + (l[1] + l[5])) + ((l[2] + l[6]) + (l[3] + l[7]))) * a.inv;
    }
}

// A register value the compiler cannot prove equal to another (the row swaps
// must see two distinct operands: a register swapped with itself is folded)
__device__ __forceinline__ unsigned opaque(unsigned x) { asm volatile("" : "+v"(x)); return x; }

extern "C" __global__ __launch_bounds__(ATTNX_THREADS) void sml_attnx_pv(const sml_kattnx a) {
    #pragma clang fp contract(off)
    extern __shared__ __align__(16) float pr[];       // [ncap] scores, then weights; then the V ring
    __shared__ float red[ATTNX_THREADS / WAVE];
    __shared__ float tot;
    __shared__ unsigned long long etab[32];
    __shared__ float fsum[ATTNX_MAXSEG];
    __shared__ int segk[2 * ATTNX_MAXSEG], sege[ATTNX_MAXSEG];
    constexpr int LT = ATTNX_THREADS / 2;                     // loader threads: waves 4..7
    constexpr int CPT = ATTNX_TP * HD / 8 / LT;               // 16-byte chunks per loader per tile
    static_assert(CPT * LT * 8 == ATTNX_TP * HD, "a tile is whole chunks per loader");
    static_assert(LT / 16 % 2 == 0, "a loader wave's rows hold whole position pairs");
    const int h = blockIdx.x, tid = threadIdx.x, rb = blockIdx.y;
    const int kh = h / (a.n_head / a.n_kv), pos = a.pos[rb], n = pos + 1, kvd = a.n_kv * HD;
    const int ncap = (a.n_ctx + 3) & ~3, nt = (n + ATTNX_TP - 1) / ATTNX_TP;
    // waves 4..7 stream V; waves 0 and 1 run the chains (a wave-uniform test)
    const bool loader = __builtin_amdgcn_readfirstlane(tid) >= LT;
    const int lt = tid - LT;
    // the ring: three slots of [ATTNX_TP/2 position pairs][HD dims] words, a
    // word holding one dim of an even position (low half) and of the next
    unsigned * ring = (unsigned *) (pr + ncap);
    const GLOBAL uint16_t * vb = (const GLOBAL uint16_t *) a.vc + (size_t) kh * HD;
    // chunk c of tile k: position k*TP + c/16 (the last position for tiles
    // past the end: a row in range, never used), dims (c%16)*8 .. +7; a
    // loader wave's 16-lane rows hold consecutive positions
    // (32-bit byte offsets from the head's base: a layer's cache is < 4 GB)
    const GLOBAL char * vbase = (const GLOBAL char *) vb;
    auto issue = [&](int k, v4u (&b)[CPT]) {
        #pragma unroll
        for (int r = 0; r < CPT; r++) {
            const int c = lt + r * LT, p = min(k * ATTNX_TP + c / 16, n - 1);
            const unsigned off = ((unsigned) p * (unsigned) kvd + (unsigned) (c % 16) * 8u) * 2u;
            b[r] = __builtin_nontemporal_load((const GLOBAL v4u *) (vbase + off));
        }
    };
    // rows 2i and 2i+1 of a wave trade their chunks (v_permlane16_swap), so
    // each lane holds its 8 dims at an even position and the next; the even
    // row writes the first 4 dims' pair words, the odd row the last 4
    auto stash = [&](int k, const v4u (&b)[CPT]) {
        const int odd = (lt >> 4) & 1;
        #pragma unroll
        for (int r = 0; r < CPT; r++) {
            const int c = lt + r * LT;
            unsigned e[4], o[4];
            #pragma unroll
            for (int i = 0; i < 4; i++) {
                const auto sw = __builtin_amdgcn_permlane16_swap(b[r][i], opaque(b[r][i]), false, false);
                e[i] = sw[0];
                o[i] = sw[1];
            }
            const unsigned e0 = odd ? e[2] : e[0], e1 = odd ? e[3] : e[1];
            const unsigned o0 = odd ? o[2] : o[0], o1 = odd ? o[3] : o[1];
            v4u w;
            w[0] = (e0 & 0xFFFFu) | (o0 << 16);
            w[1] = (e0 >> 16) | (o0 & 0xFFFF0000u);
            w[2] = (e1 & 0xFFFFu) | (o1 << 16);
            w[3] = (e1 >> 16) | (o1 & 0xFFFF0000u);
            *(v4u *) (ring + ((size_t) (k % 3) * (ATTNX_TP / 2) + c / 32) * HD + (c % 16) * 8 + odd * 4) = w;
        }
    };
    // the scores (8 loads per thread in flight, then into LDS) and expf's table
    if (tid < 32) etab[tid] = EXPF_TAB[tid];
    const GLOBAL float * sc = (const GLOBAL float *) a.sc + ((size_t) rb * a.n_head + h) * a.n_ctx;
    for (int base = 0; base < n; base += 8 * ATTNX_THREADS) {
        float v[8];
        #pragma unroll
        for (int i = 0; i < 8; i++) v[i] = sc[min(base + tid + i * ATTNX_THREADS, n - 1)];
        #pragma unroll
        for (int i = 0; i < 8; i++) {
            const int t = base + tid + i * ATTNX_THREADS;
            if (t < n) pr[t] = v[i];
        }
    }
    __syncthreads();
    float m = -__builtin_inff();
    for (int t = tid; t < n; t += ATTNX_THREADS) m = fmaxf(m, pr[t]);
    m = wave_max(m);
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    #pragma unroll
    for (int w = 0; w < ATTNX_THREADS / WAVE; w++) m = fmaxf(m, red[w]);
    for (int t = tid; t < n; t += ATTNX_THREADS) pr[t] = expf_tab(pr[t] - m, etab);
    __syncthreads();
    // the first V tiles go out now, behind every other global load: loads
    // complete in order, so a wait for an earlier one would wait for them too
    v4u buf[ATTNX_PF][CPT];
    if (loader) {
        #pragma unroll
        for (int u = 0; u < ATTNX_PF; u++) issue(u, buf[u]);
    }
    const float iv = 1.0f / serial_sum_seg(pr, n, fsum, segk, sege, &tot);
    for (int t = tid; t < n; t += ATTNX_THREADS) pr[t] = pr[t] * iv;
    // tiles 0 and 1 into the ring; their registers take tiles PF and PF+1
    if (loader) {
        stash(0, buf[0]);
        issue(ATTNX_PF, buf[0]);
        stash(1, buf[1]);
        issue(ATTNX_PF + 1, buf[1]);
    }
    __syncthreads();
    // P.V: threads 0..127 each run one dim's chain over tile k in ring slot
    // k%3 while the loaders move tile k+2 from registers into slot (k+2)%3
    // and issue tile k+2+PF. The two kinds of waves run loops of their own
    // that meet at the same barriers, one per round of a tile, over whole
    // groups of PF rounds (a barrier counts waves, whichever instruction they
    // reach it at). The loaders move a tile and issue one every round, also
    // past the last tile (rows in range, never read), so the loads in flight
    // are the same count at every wait and the compiler's waits stay partial.
    // A chain reads 4 positions per LDS instruction (two pair words 256 bytes
    // apart) and 4 weights per broadcast read, 24 positions ahead (12 of the
    // 15 reads the LDS counter can wait on partially), also into the next
    // tile, which is in the ring a round before its own.
    float o = 0.0f;
    if (loader) {
        for (int kk = 0; kk < nt; kk += ATTNX_PF) {
            #pragma unroll
            for (int u = 0; u < ATTNX_PF; u++) {
                stash(kk + u + 2, buf[(u + 2) % ATTNX_PF]);
                issue(kk + u + 2 + ATTNX_PF, buf[(u + 2) % ATTNX_PF]);
                __syncthreads();
            }
        }
        return;
    }
    constexpr int NB = ATTNX_TP / 8, AH = 3;                  // blocks of 8 positions per tile, blocks ahead
    static_assert(NB % (AH + 1) == 0, "a tile is whole rounds of the read registers");
    const unsigned * vd = ring + tid;
    unsigned vv[AH + 1][4];
    float4 ww[AH + 1][2];
    // block b of tile k: pair words of pairs 4b..4b+3, weights 8b..8b+7 (past
    // the last tile: LDS in range, never used)
    auto ld = [&](int k, int b, unsigned (&v)[4], float4 (&w)[2]) {
        const unsigned * vs = vd + (size_t) (k % 3) * (ATTNX_TP / 2) * HD;
        const float * ps = pr + k * ATTNX_TP;
        #pragma unroll
        for (int j = 0; j < 4; j++) v[j] = vs[(4 * b + j) * HD];
        w[0] = *(const float4 *) (ps + b * 8);
        w[1] = *(const float4 *) (ps + b * 8 + 4);
    };
    if (tid < HD) {
        #pragma unroll
        for (int b = 0; b < AH; b++) ld(0, b, vv[b], ww[b]);
    }
    for (int kk = 0; kk < nt; kk += ATTNX_PF) {
        #pragma unroll
        for (int u = 0; u < ATTNX_PF; u++) {
            const int k = kk + u;
            if (tid < HD && k < nt) {
                const int cnt = min(ATTNX_TP, n - k * ATTNX_TP);
                if (cnt == ATTNX_TP) {
                    #pragma unroll
                    for (int b = 0; b < NB; b++) {
                        const int nb = b + AH;
                        ld(nb < NB ? k : k + 1, nb % NB, vv[nb % (AH + 1)], ww[nb % (AH + 1)]);
                        __builtin_amdgcn_sched_barrier(0);
                        const unsigned (&v)[4] = vv[b % (AH + 1)];
                        const float4 (&w)[2] = ww[b % (AH + 1)];
                        o = __builtin_fmaf(w[0].x, h2f((uint16_t) v[0]), o);
                        o = __builtin_fmaf(w[0].y, h2f((uint16_t) (v[0] >> 16)), o);
                        o = __builtin_fmaf(w[0].z, h2f((uint16_t) v[1]), o);
                        o = __builtin_fmaf(w[0].w, h2f((uint16_t) (v[1] >> 16)), o);
                        o = __builtin_fmaf(w[1].x, h2f((uint16_t) v[2]), o);
                        o = __builtin_fmaf(w[1].y, h2f((uint16_t) (v[2] >> 16)), o);
                        o = __builtin_fmaf(w[1].z, h2f((uint16_t) v[3]), o);
                        o = __builtin_fmaf(w[1].w, h2f((uint16_t) (v[3] >> 16)), o);
                        __builtin_amdgcn_sched_barrier(0);
                    }
                } else {
                    // the last, partial tile
                    const unsigned * vs = vd + (size_t) (k % 3) * (ATTNX_TP / 2) * HD;
                    const float * ps = pr + k * ATTNX_TP;
                    for (int p = 0; p < cnt; p++)
                        o = __builtin_fmaf(ps[p], h2f((uint16_t) (vs[(p / 2) * HD] >> (16 * (p & 1)))), o);
                }
            }
            __syncthreads();
        }
    }
    if (tid >= HD) return;
    const size_t ob = (size_t) rb * a.n_head * HD;
    a.out[ob + (size_t) h * HD + tid] = o;
    if (a.q_out) {
        const float amax = max32(fabsf(o));
        const float s = amax / 127.0f;
        const float is = s > 0.0f ? 1.0f / s : 0.0f;
        const int q = quant1(o, is);
        const int sum = isum32(q);
        const size_t j = ob + (size_t) h * HD + tid;
        a.q_out[j] = (int8_t) q;
        if ((tid & 31) == 0) { a.s_out[j / 32] = s; a.u_out[j / 32] = sum; }
    }
}

// ---------------------------------------------------------------- argmax
// First maximum wins (sml/sml-run.c:3539-3544). One workgroup: every thread
// issues all of its float4 loads (16 per round) before comparing, so the
// 513 KB of a 128k vocabulary arrive in a few round trips.
#define ARGMAX_THREADS 1024
#define ARGMAX_UNROLL 16
// First stage of the two-stage pick: grid-stride over float4 words, one
// (max, lowest index) pair per workgroup. The first-max rule is kept by
// amax_take when the pairs are combined.
#define ARGMAX_PART_THREADS 256
extern "C" __global__ __launch_bounds__(ARGMAX_PART_THREADS) void sml_argmax_part(const sml_kargmax a) {
    __shared__ float bv_s[ARGMAX_PART_THREADS / 64];
    __shared__ int bi_s[ARGMAX_PART_THREADS / 64];
    const int tid = threadIdx.x;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    const bool al = ((uintptr_t) a.logits & 15) == 0;
    const int n4 = al ? a.n / 4 : 0;
    const int stride = gridDim.x * ARGMAX_PART_THREADS;
    const float4 * l4 = (const float4 *) a.logits;
    for (int f = blockIdx.x * ARGMAX_PART_THREADS + tid; f < n4; f += stride) {
        const float4 v = l4[f];
        amax_take(v.x, 4 * f, bv, bi); amax_take(v.y, 4 * f + 1, bv, bi);
        amax_take(v.z, 4 * f + 2, bv, bi); amax_take(v.w, 4 * f + 3, bv, bi);
    }
    for (int i = 4 * n4 + blockIdx.x * ARGMAX_PART_THREADS + tid; i < a.n; i += stride) amax_take(a.logits[i], i, bv, bi);
    #pragma unroll
    for (int o = 32; o; o >>= 1) {
        const float ov = __shfl_xor(bv, o);
        const int oi = __shfl_xor(bi, o);
        amax_take(ov, oi, bv, bi);
    }
    if ((tid & 63) == 0) { bv_s[tid >> 6] = bv; bi_s[tid >> 6] = bi; }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < ARGMAX_PART_THREADS / 64; w++) amax_take(bv_s[w], bi_s[w], bv_s[0], bi_s[0]);
        a.part[blockIdx.x] = make_int2(__float_as_int(bv_s[0]), bi_s[0]);
    }
}

extern "C" __global__ __launch_bounds__(ARGMAX_THREADS) void sml_argmax(const sml_kargmax a) {
    __shared__ float bv_s[ARGMAX_THREADS / 64];
    __shared__ int bi_s[ARGMAX_THREADS / 64];
    const int tid = threadIdx.x;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    if (a.part)
        for (int i = tid; i < a.nparts; i += ARGMAX_THREADS) {
            const int2 p = a.part[i];
            amax_take(__int_as_float(p.x), p.y, bv, bi);
        }
    const bool al = ((uintptr_t) a.logits & 15) == 0;
    const int n4 = a.part ? 0 : al ? a.n / 4 : 0;
    const float4 * l4 = (const float4 *) a.logits;
    for (int base = 0; base < n4; base += ARGMAX_THREADS * ARGMAX_UNROLL) {
        float4 v[ARGMAX_UNROLL];
        #pragma unroll
        for (int k = 0; k < ARGMAX_UNROLL; k++) {
            const int f = base + k * ARGMAX_THREADS + tid;
            v[k] = l4[f < n4 ? f : 0];
        }
        #pragma unroll
        for (int k = 0; k < ARGMAX_UNROLL; k++) {
            const int f = base + k * ARGMAX_THREADS + tid;
            if (f < n4) {
                // NaN never compares greater, as in the reference's loop
                amax_take(v[k].x, 4 * f, bv, bi); amax_take(v[k].y, 4 * f + 1, bv, bi);
                amax_take(v[k].z, 4 * f + 2, bv, bi); amax_take(v[k].w, 4 * f + 3, bv, bi);
            }
        }
    }
    if (!a.part)
        for (int i = 4 * n4 + tid; i < a.n; i += ARGMAX_THREADS) amax_take(a.logits[i], i, bv, bi);
    #pragma unroll
    for (int o = 32; o; o >>= 1) {
        const float ov = __shfl_xor(bv, o);
        const int oi = __shfl_xor(bi, o);
        amax_take(ov, oi, bv, bi);
    }
    if ((tid & 63) == 0) { bv_s[tid >> 6] = bv; bi_s[tid >> 6] = bi; }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < ARGMAX_THREADS / 64; w++) amax_take(bv_s[w], bi_s[w], bv_s[0], bi_s[0]);
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
    if (i < a.n) a.g[i] = silu_ref(a.g[i]) * a.u[i];
}

// ---------------------------------------------------------------- calibration
// A streaming read with the GEMV's access size (128-bit loads), grid-stride:
// what one kernel can pull from HBM on this machine, for the roofline.
extern "C" __global__ __launch_bounds__(256) void sml_read_stream(const sml_kread a) {
    const v4u * p = (const v4u *) a.src;
    const uint64_t nw = a.bytes / 16;
    v4u acc = {0u, 0u, 0u, 0u};
    if (a.pattern == 0) {
        for (uint64_t i = (uint64_t) blockIdx.x * 256 + threadIdx.x; i < nw; i += (uint64_t) gridDim.x * 256)
            acc ^= __builtin_nontemporal_load(p + i);
    } else if (a.pattern == 3 || a.pattern == 4) {
        // tiles of a row-major matrix with 2048-byte rows, one tile per wave
        // step: 3 = 16 rows x 64 bytes (4 lanes per row, the small-M GEMM's
        // operand loads), 4 = 4 rows x 256 bytes (16 lanes per row)
        const uint64_t nrows = a.bytes / 2048;
        const int l = threadIdx.x & 63;
        const uint64_t ntiles = a.pattern == 3 ? (nrows / 16) * 32 : (nrows / 4) * 8;
        for (uint64_t t = (uint64_t) blockIdx.x * 4 + (threadIdx.x >> 6); t < ntiles; t += (uint64_t) gridDim.x * 4) {
            uint64_t row, byte;
            if (a.pattern == 3) { row = (t / 32) * 16 + (l & 15); byte = (t % 32) * 64 + 16 * (l >> 4); }
            else { row = (t / 8) * 4 + (l >> 4); byte = (t % 8) * 256 + 16 * (l & 15); }
            acc ^= __builtin_nontemporal_load(p + (row * 2048 + byte) / 16);
        }
    } else if (a.pattern == 2) {
        // one shot: each thread issues its 4 coalesced words before using any
        const uint64_t base = (uint64_t) blockIdx.x * 1024 + threadIdx.x;
        v4u t[4];
        #pragma unroll
        for (int k = 0; k < 4; k++) { const uint64_t i = base + (uint64_t) k * 256; t[k] = __builtin_nontemporal_load(p + (i < nw ? i : 0)); }
        #pragma unroll
        for (int k = 0; k < 4; k++) acc ^= t[k];
    } else {
        // the GEMV's quad-per-lane shape: lane reads 4 consecutive 16-byte words
        for (uint64_t i = ((uint64_t) blockIdx.x * 256 + threadIdx.x) * 4; i + 3 < nw; i += (uint64_t) gridDim.x * 1024) {
            acc ^= __builtin_nontemporal_load(p + i);
            acc ^= __builtin_nontemporal_load(p + i + 1);
            acc ^= __builtin_nontemporal_load(p + i + 2);
            acc ^= __builtin_nontemporal_load(p + i + 3);
        }
    }
    unsigned v = acc.x ^ acc.y ^ acc.z ^ acc.w;
    #pragma unroll
    for (int o = 32; o; o >>= 1) v ^= __shfl_xor(v, o);
    if ((threadIdx.x & 63) == 0) a.sink[blockIdx.x * 4 + (threadIdx.x >> 6)] = v;
}

// Grid-stride 128-bit copy: reads and writes `bytes` once each.
extern "C" __global__ __launch_bounds__(256) void sml_copy_stream(const sml_kcopy a) {
    const v4u * s = (const v4u *) a.src;
    v4u * d = (v4u *) a.dst;
    const uint64_t nw = a.bytes / 16;
    for (uint64_t i = (uint64_t) blockIdx.x * 256 + threadIdx.x; i < nw; i += (uint64_t) gridDim.x * 256)
        d[i] = __builtin_nontemporal_load(s + i);
}

// ---------------------------------------------------------------- GPTQ-style 4-bit GEMV
//
// The layout of tooling/sml_unpack.py:66-95 (dequant_gptq): weight
// (q - z) * s with q packed 8 per int32 along the input. Consecutive outputs
// are contiguous there, so a lane loads 16 bytes = 4 outputs x 8 inputs and
// a wave streams 256 outputs of one group of 128 inputs (16 loads per lane,
// all issued before any use). The activation stays fp32, staged per wave
// in LDS and read as broadcasts: per group, s * (sum q*x - z * sum x). The GPTQ_WAVES waves of a workgroup cover
// consecutive groups, summed in LDS into one partial per output; the last
// workgroup of each output block (or, without counters, sml_gptq_reduce)
// adds the partials in slice order.
#define GPTQ_WAVES 8
// OPL outputs per lane (4: 256 outputs per wave, 16-byte weight loads; 2:
// 128 per wave, 8-byte loads and twice the waves for the same matrix)
template <int OPL>
__device__ void gptq_body(const sml_kgptq & a) {
    typedef uint32_t vw __attribute__((ext_vector_type(OPL)));
    __shared__ float xs[GPTQ_WAVES][128];
    __shared__ float red[GPTQ_WAVES][64 * OPL];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ngr = a.cols / 128;
    const int g = blockIdx.y * GPTQ_WAVES + w;
    const bool gv = g < ngr;
    const int o = blockIdx.x * (64 * OPL) + lane * OPL;
    const bool ov = o < a.rows;
    const int gc = gv ? g : 0, oc = ov ? o : 0;
    const float * xg = a.x + (size_t) gc * 128;
    // 1. this group's inputs (two per lane, for their sum; through the
    // column order of a desc_act file), every weight word, then the group
    // fields
    float2 xv;
    if (a.perm) {
        const int2 p = ((const int2 *) (a.perm + (size_t) gc * 128))[lane];
        xv = make_float2(a.x[p.x], a.x[p.y]);
    } else {
        xv = ((const float2 *) xg)[lane];
    }
    vw q[16];
    #pragma unroll
    for (int kk = 0; kk < 16; kk++)
        q[kk] = __builtin_nontemporal_load((const vw *) (a.qweight + ((size_t) gc * 16 + kk) * a.rows + oc));
    uint16_t scv[OPL];
    #pragma unroll
    for (int j = 0; j < OPL; j++) scv[j] = a.scales[(size_t) gc * a.rows + oc + j];
    const uint32_t zw = a.qzeros[(size_t) gc * (a.rows / 8) + oc / 8];
    xs[w][2 * lane] = xv.x;
    xs[w][2 * lane + 1] = xv.y;
    const float sx = wave_sum(xv.x + xv.y);
    __syncthreads();
    // 2. sum q*x per output: the low and high nibbles of each byte are
    // inputs 2i and 2i+1 of the word's 8
    float acc[OPL];
    #pragma unroll
    for (int j = 0; j < OPL; j++) acc[j] = 0.0f;
    #pragma unroll
    for (int kk = 0; kk < 16; kk++) {
        const float4 x0 = *(const float4 *) &xs[w][kk * 8], x1 = *(const float4 *) &xs[w][kk * 8 + 4];
        #pragma unroll
        for (int j = 0; j < OPL; j++) {
            const uint32_t wd = q[kk][j], lo = wd & 0x0F0F0F0Fu, hi = (wd >> 4) & 0x0F0F0F0Fu;
            float t = acc[j];
            t = fmaf((float) (lo & 0xFFu), x0.x, t);
            t = fmaf((float) (hi & 0xFFu), x0.y, t);
            t = fmaf((float) ((lo >> 8) & 0xFFu), x0.z, t);
            t = fmaf((float) ((hi >> 8) & 0xFFu), x0.w, t);
            t = fmaf((float) ((lo >> 16) & 0xFFu), x1.x, t);
            t = fmaf((float) ((hi >> 16) & 0xFFu), x1.y, t);
            t = fmaf((float) (lo >> 24), x1.z, t);
            t = fmaf((float) (hi >> 24), x1.w, t);
            acc[j] = t;
        }
    }
    // 3. the group epilogue and the workgroup's sum over its groups
    #pragma unroll
    for (int j = 0; j < OPL; j++) {
        const float s = h2f(scv[j]);
        const float z = (float) (((zw >> (4 * ((oc & 7) + j))) & 15u) + (uint32_t) a.zero_add);
        red[w][lane * OPL + j] = gv ? s * (acc[j] - z * sx) : 0.0f;
    }
    __syncthreads();
    const bool fold = a.cnt != nullptr;
    if (tid < 64 && ov) {
        #pragma unroll
        for (int j = 0; j < OPL; j++) {
            float v = red[0][lane * OPL + j];
            #pragma unroll
            for (int k = 1; k < GPTQ_WAVES; k++) v += red[k][lane * OPL + j];
            float * pp = a.part + (size_t) blockIdx.y * a.rows + o + j;
            if (fold) st_dev(pp, v);
            else *pp = v;
        }
    }
    if (!fold) return;
    // 4. the output block's last workgroup (every slice's partials stored
    // at device scope before it counts itself in) adds the slices in slice
    // order, the reduce kernel's arithmetic, and clears the counter
    __shared__ int last;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0)
        last = __hip_atomic_fetch_add(a.cnt + blockIdx.x, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (int) gridDim.y - 1;
    __syncthreads();
    if (!last) return;
    for (int i = tid; i < 64 * OPL; i += 64 * GPTQ_WAVES) {
        const int oo = blockIdx.x * (64 * OPL) + i;
        if (oo >= a.rows) continue;
        float v = 0.0f;
        for (int s0 = 0; s0 < a.nslice; s0 += 8) {
            float p[8];
            #pragma unroll
            for (int k = 0; k < 8; k++) p[k] = s0 + k < a.nslice ? ld_part<true>(a.part + (size_t) (s0 + k) * a.rows + oo) : 0.0f;
            #pragma unroll
            for (int k = 0; k < 8; k++) v += p[k];
        }
        a.y[oo] = v;
    }
    if (tid == 0) __hip_atomic_store(a.cnt + blockIdx.x, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// The integer form (the default): each group's 128 inputs as 15-bit fixed
// point, x ~ xs*m with xs = max|x|/16319 and m = 128*hi + lo (hi in
// [-128,127], lo in [-64,63], both int8), so the dot products run on
// v_dot4_i32_i8 in exact integers: per 8 codes of a word, the low nibbles
// (inputs 8k, 8k+2, 8k+4, 8k+6) and the high ones (8k+1, ...) against the
// matching bytes of hi and of lo, 4 dot4 and 3 mask instructions against
// the float form's 19. Per group and output, s*xs*(128*dot_hi + dot_lo -
// z*sum m) in fp32; the slice sum, partials and fold are gptq_body's. The
// inputs' rounding to m (within xs/2 <= max|x|/32638) is the only departure
// from the float form, ~3e-5 of the group's largest input.
// OPL outputs per lane (2: 128 per wave, 8-byte weight loads), NW waves
// (groups) per workgroup, one slice of NW groups per grid row
template <int OPL, int NW>
__device__ void gptq_i8_body(const sml_kgptq & a) {
    typedef uint32_t vw __attribute__((ext_vector_type(OPL)));
    __shared__ int4 xq[NW][16];           // per word: (even hi, odd hi, even lo, odd lo) bytes
    __shared__ int8_t xb[NW][4][64];
    __shared__ float red[NW][64 * OPL];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ngr = a.cols / 128;
    const int g = blockIdx.y * NW + w;
    const bool gv = g < ngr;
    const int o = blockIdx.x * (64 * OPL) + lane * OPL;
    const bool ov = o < a.rows;
    const int gc = gv ? g : 0, oc = ov ? o : 0;
    // 1. this group's inputs (two per lane; through the column order of a
    // desc_act file), every weight word, then the group fields
    float2 xv;
    if (a.perm) {
        const int2 p = ((const int2 *) (a.perm + (size_t) gc * 128))[lane];
        xv = make_float2(a.x[p.x], a.x[p.y]);
    } else {
        xv = ((const float2 *) (a.x + (size_t) gc * 128))[lane];
    }
    vw q[16];
    #pragma unroll
    for (int kk = 0; kk < 16; kk++)
        q[kk] = __builtin_nontemporal_load((const vw *) (a.qweight + ((size_t) gc * 16 + kk) * a.rows + oc));
    uint16_t scv[OPL];
    #pragma unroll
    for (int j = 0; j < OPL; j++) scv[j] = a.scales[(size_t) gc * a.rows + oc + j];
    const uint32_t zw = a.qzeros[(size_t) gc * (a.rows / 8) + oc / 8];
    // 2. the inputs as fixed point: lane l holds inputs 2l and 2l+1
    pin(xv.x); pin(xv.y);
    const float amax = wave_max(fmaxf(fabsf(xv.x), fabsf(xv.y)));
    const float xs = amax / 16319.0f;
    const float ixs = xs > 0.0f ? 1.0f / xs : 0.0f;
    const int m0 = (int) __builtin_rintf(xv.x * ixs), m1 = (int) __builtin_rintf(xv.y * ixs);
    const int h0 = (m0 + 64) >> 7, h1 = (m1 + 64) >> 7;          // m = 128*h + l, l in [-64, 63]
    xb[w][0][lane] = (int8_t) h0;
    xb[w][1][lane] = (int8_t) h1;
    xb[w][2][lane] = (int8_t) (m0 - 128 * h0);
    xb[w][3][lane] = (int8_t) (m1 - 128 * h1);
    const int msum = (int) wave_sum((float) (m0 + m1));             // |sum| < 2^22: exact in fp32
    wave_lds_sync();
    if (lane < 16)
        xq[w][lane] = make_int4(((const int *) xb[w][0])[lane], ((const int *) xb[w][1])[lane],
                                ((const int *) xb[w][2])[lane], ((const int *) xb[w][3])[lane]);
    wave_lds_sync();
    // 3. the integer dots of both outputs
    int dh[OPL], dl[OPL];
    #pragma unroll
    for (int j = 0; j < OPL; j++) { dh[j] = 0; dl[j] = 0; }
    #pragma unroll
    for (int kk = 0; kk < 16; kk++) {
        const int4 xw = xq[w][kk];
        #pragma unroll
        for (int j = 0; j < OPL; j++) {
            const int wd = (int) q[kk][j], lo = wd & 0x0F0F0F0F, hi = (wd >> 4) & 0x0F0F0F0F;
            dh[j] = __builtin_amdgcn_sdot4(lo, xw.x, dh[j], false);
            dh[j] = __builtin_amdgcn_sdot4(hi, xw.y, dh[j], false);
            dl[j] = __builtin_amdgcn_sdot4(lo, xw.z, dl[j], false);
            dl[j] = __builtin_amdgcn_sdot4(hi, xw.w, dl[j], false);
        }
    }
    // 4. the group epilogue and the workgroup's sum over its groups
    #pragma unroll
    for (int j = 0; j < OPL; j++) {
        const float s = h2f(scv[j]);
        const int z = (int) (((zw >> (4 * ((oc & 7) + j))) & 15u) + (uint32_t) a.zero_add);
        const int d = 128 * dh[j] + dl[j] - z * msum;              // |d| < 2^27
        red[w][lane * OPL + j] = gv ? (s * xs) * (float) d : 0.0f;
    }
    __syncthreads();
    const bool fold = a.cnt != nullptr;
    if (tid < 64 && ov) {
        #pragma unroll
        for (int j = 0; j < OPL; j++) {
            float v = red[0][lane * OPL + j];
            #pragma unroll
            for (int k = 1; k < NW; k++) v += red[k][lane * OPL + j];
            float * pp = a.part + (size_t) blockIdx.y * a.rows + o + j;
            if (fold) st_dev(pp, v);
            else *pp = v;
        }
    }
    if (!fold) return;
    __shared__ int last;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0)
        last = __hip_atomic_fetch_add(a.cnt + blockIdx.x, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (int) gridDim.y - 1;
    __syncthreads();
    if (!last) return;
    for (int i = tid; i < 64 * OPL; i += 64 * NW) {
        const int oo = blockIdx.x * (64 * OPL) + i;
        if (oo >= a.rows) continue;
        float v = 0.0f;
        for (int s0 = 0; s0 < a.nslice; s0 += 8) {
            float p[8];
            #pragma unroll
            for (int k = 0; k < 8; k++) p[k] = s0 + k < a.nslice ? ld_part<true>(a.part + (size_t) (s0 + k) * a.rows + oo) : 0.0f;
            #pragma unroll
            for (int k = 0; k < 8; k++) v += p[k];
        }
        a.y[oo] = v;
    }
    if (tid == 0) __hip_atomic_store(a.cnt + blockIdx.x, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// 2 outputs per lane and 8 groups per workgroup: 9.4 us at 4096 x 14336
// against 12.0-12.9 for 4 per lane or 4 groups (14336 x 4096: 8.7 against 9.0-9.2)
extern "C" __global__ __launch_bounds__(64 * GPTQ_WAVES) void sml_gptq_gemv_i8(const sml_kgptq a) { gptq_i8_body<2, GPTQ_WAVES>(a); }
extern "C" __global__ __launch_bounds__(64 * GPTQ_WAVES) void sml_gptq_gemv(const sml_kgptq a) { gptq_body<4>(a); }
extern "C" __global__ __launch_bounds__(64 * GPTQ_WAVES) void sml_gptq_gemv2(const sml_kgptq a) { gptq_body<2>(a); }

extern "C" __global__ __launch_bounds__(256) void sml_gptq_reduce(const sml_kgptq a) {
    const int o = blockIdx.x * 256 + threadIdx.x;
    if (o >= a.rows) return;
    float p[8];
    float v = 0.0f;
    for (int s0 = 0; s0 < a.nslice; s0 += 8) {
        #pragma unroll
        for (int k = 0; k < 8; k++) p[k] = s0 + k < a.nslice ? a.part[(size_t) (s0 + k) * a.rows + o] : 0.0f;
        #pragma unroll
        for (int k = 0; k < 8; k++) v += p[k];
    }
    a.y[o] = v;
}

// Integer codes and zeros of rows [row0, row0+nrows): one thread per (row, 8 inputs).
extern "C" __global__ void sml_gptq_unpack(const sml_kgptq_unpack a) {
    const long t = (long) blockIdx.x * blockDim.x + threadIdx.x;
    const int nk = a.cols / 8;
    if (t >= (long) a.nrows * nk) return;
    const int r = (int) (t / nk), kk = (int) (t % nk), o = a.row0 + r;
    const uint32_t wd = a.qweight[(size_t) kk * a.rows + o];
    uint8_t * c = a.codes + (size_t) r * a.cols + (size_t) kk * 8;
    #pragma unroll
    for (int i = 0; i < 8; i++) c[i] = (uint8_t) ((wd >> (4 * i)) & 15u);
    if ((kk & 15) == 0) {
        const int g = kk / 16;
        const uint32_t zw = a.qzeros[(size_t) g * (a.rows / 8) + o / 8];
        a.zeros[(size_t) r * (a.cols / 128) + g] = (uint8_t) (((zw >> (4 * (o & 7))) & 15u) + (uint32_t) a.zero_add);
    }
}

// ---------------------------------------------------------------- MoE: route and plan
//
// sml_moe_route, one workgroup per token: the router logits
// (sml/sml-run.c:3075-3080: a double sum per expert, then (float) + bias),
// one wave per expert at a time, and the shared expert's gate the same way;
// then one thread routes as sml_moe_route does (sml/sml-run.c:2925-3037):
// plain top-k with ties to the lower index and the Mixtral / Granite
// weights (moe_flags bit 0: softmax over the chosen; else softmax over
// all); sigmoid or softmax scores with the correction bias and the best
// groups shaping the choice only; PhiMoE's sparsemixer; then moe_scale.
// sml_moe_plan then lists each expert's tokens in token-then-choice order,
// the order moe_ffn_batch gathers them in (sml/sml-run.c:3211-3219).
#define MOE_ROUTE_THREADS 512
// expf of the C library for any float (the restated one, with its overflow)
__device__ __forceinline__ float expf_any(float x) { return x > 0x1.62e42ep6f ? __builtin_inff() : expf_ref(x); }
// the best index by key not among sel[0..nsel), ties to the lower index
__device__ __forceinline__ int best_untaken(const float * key, int n, const int * sel, int nsel) {
    int best = -1;
    for (int e = 0; e < n; e++) {
        bool taken = false;
        for (int q = 0; q < nsel; q++) taken = taken || sel[q] == e;
        if (!taken && (best < 0 || key[e] > key[best])) best = e;
    }
    return best;
}
extern "C" __global__ __launch_bounds__(MOE_ROUTE_THREADS) void sml_moe_route(const sml_kmoe_route a) {
    __shared__ float lg[65], sc[64], ch[64], gs[64];
    __shared__ int kept[64];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, t = blockIdx.x;
    const float * x = a.x + (size_t) t * a.n;
    const int nrow = a.nexp + (a.shgate ? 1 : 0);          // row nexp: the shared expert's gate
    for (int e = wv; e < nrow; e += MOE_ROUTE_THREADS / 64) {
        const float * r = e < a.nexp ? a.router + (size_t) e * a.n : a.shgate;
        double s0 = 0.0, s1 = 0.0, s2 = 0.0, s3 = 0.0;
        int i = lane * 4;
        for (; i + 3 < a.n; i += 256) {
            const float4 rv = *(const float4 *) (r + i), xv = *(const float4 *) (x + i);
            s0 += (double) rv.x * (double) xv.x;
            s1 += (double) rv.y * (double) xv.y;
            s2 += (double) rv.z * (double) xv.z;
            s3 += (double) rv.w * (double) xv.w;
        }
        double s = (s0 + s1) + (s2 + s3);
        #pragma unroll
        for (int o = 32; o; o >>= 1) s += __shfl_xor(s, o);
        if (a.exact && lane == 0) {
            // the reference's loop, s = fma(r_i, x_i, s) in order (sml/sml-run.c:3075-3080)
            s = 0.0;
            for (int i2 = 0; i2 < a.n; i2++) s = __builtin_fma((double) r[i2], (double) x[i2], s);
        }
        if (lane == 0) {
            if (e < a.nexp) {
                const float v = (float) s + (a.router_b ? a.router_b[e] : 0.0f);
                lg[e] = v;
                a.logits[(size_t) t * a.nexp + e] = v;
            } else {
                a.sg[t] = 1.0f / (1.0f + expf_any(-(float) s));   // sml/sml-run.c:3116-3120
            }
        }
    }
    if (a.sg && !a.shgate && tid == 0) a.sg[t] = 1.0f;
    __syncthreads();
    if (tid != 0) return;
    const int ne = a.nexp, k = a.k;
    int32_t * sel = a.sel + t * k;
    float * w = a.w + t * k;
    int sl[16];
    float wj[16];
    if (a.moe_flags & 4u) {
        // sparsemixer: each pick the best untaken logit, weighted by its share
        // among the untaken experts within 2 x jitter of it
        const float eps2 = 2.0f * a.scale;
        for (int j = 0; j < k; j++) {
            const int b = best_untaken(lg, ne, sl, j);
            const float mx = lg[b];
            double sum = 0.0;
            for (int e = 0; e < ne; e++) {
                bool taken = false;
                for (int q = 0; q < j; q++) taken = taken || sl[q] == e;
                const float f = fabsf(lg[e]) > mx ? fabsf(lg[e]) : mx;
                if (!taken && (mx - lg[e]) / f <= eps2) sum += exp((double) lg[e] - mx);
            }
            sl[j] = b;
            wj[j] = (float) (1.0 / sum);
        }
        for (int j = 0; j < k; j++) { sel[j] = sl[j]; w[j] = wj[j]; }
        return;
    }
    if ((a.moe_flags & 2u) || a.exp_bias || a.groups > 1) {
        // scores; the choice adds the correction bias and keeps only the best
        // groups' experts (a group scored by its best one or two); the weights
        // are the plain scores
        if (a.moe_flags & 2u) {
            for (int e = 0; e < ne; e++) sc[e] = 1.0f / (1.0f + expf_any(-lg[e]));
        } else {
            float mx = lg[0];
            for (int e = 1; e < ne; e++) mx = lg[e] > mx ? lg[e] : mx;
            double sum = 0.0;
            for (int e = 0; e < ne; e++) sum += expf_ref(lg[e] - mx);
            for (int e = 0; e < ne; e++) sc[e] = (float) (expf_ref(lg[e] - mx) / sum);
        }
        for (int e = 0; e < ne; e++) ch[e] = sc[e] + (a.exp_bias ? a.exp_bias[e] : 0.0f);
        const int ng = a.groups, tg = a.topk_group;
        if (ng > 1 && tg < ng && ne % ng == 0) {
            const int per = ne / ng;
            for (int g = 0; g < ng; g++) {
                float b1 = -1e30f, b2 = -1e30f;
                for (int i = 0; i < per; i++) {
                    const float v = ch[g * per + i];
                    if (v > b1) { b2 = b1; b1 = v; } else if (v > b2) b2 = v;
                }
                gs[g] = (a.moe_flags & 8u) ? b1 : b1 + (per > 1 ? b2 : 0.0f);
            }
            for (int q = 0; q < tg; q++) kept[q] = best_untaken(gs, ng, kept, q);
            for (int e = 0; e < ne; e++) {
                bool keep = false;
                for (int q = 0; q < tg; q++) keep = keep || kept[q] == e / per;
                if (!keep) ch[e] = 0.0f;
            }
        }
        for (int j = 0; j < k; j++) {
            sl[j] = best_untaken(ch, ne, sl, j);
            wj[j] = sc[sl[j]];
        }
        if (a.moe_flags & 1u) {
            float sum = 0.0f;
            for (int j = 0; j < k; j++) sum += wj[j];
            for (int j = 0; j < k; j++) wj[j] /= sum + 1e-20f;
        }
    } else {
        for (int j = 0; j < k; j++) sl[j] = best_untaken(lg, ne, sl, j);
        if (a.moe_flags & 1u) {
            double sum = 0.0;
            for (int j = 0; j < k; j++) { wj[j] = expf_ref(lg[sl[j]] - lg[sl[0]]); sum += wj[j]; }
            for (int j = 0; j < k; j++) wj[j] = (float) (wj[j] / sum);
        } else {
            float mx = lg[0];
            for (int e = 1; e < ne; e++) mx = lg[e] > mx ? lg[e] : mx;
            double sum = 0.0;
            for (int e = 0; e < ne; e++) sum += expf_ref(lg[e] - mx);
            for (int j = 0; j < k; j++) wj[j] = (float) (expf_ref(lg[sl[j]] - mx) / sum);
        }
    }
    if (a.scale != 0.0f) for (int j = 0; j < k; j++) wj[j] *= a.scale;
    for (int j = 0; j < k; j++) { sel[j] = sl[j]; w[j] = wj[j]; }
}

// one thread per expert scans the choices (staged in LDS) in order
extern "C" __global__ __launch_bounds__(64) void sml_moe_plan(const sml_kmoe_route a) {
    __shared__ int32_t sel[16 * 16];                  // T * k <= 256
    const int nk = a.T * a.k;
    for (int i = threadIdx.x; i < nk; i += 64) sel[i] = a.sel[i];
    __syncthreads();
    const int e = threadIdx.x;
    if (e >= a.nexp) return;
    int m = 0;
    for (int i = 0; i < nk; i++)
        if (sel[i] == e) {
            a.list[e * a.mmax + m] = i;
            a.slot[i] = m;
            m++;
        }
    a.count[e] = m;
}

// Per-32 quantization of one activation row per workgroup (grid mmax x nexp),
// the normq arithmetic (bit-exact with sml_quantize_act): a thread takes 4
// consecutive values, 8 threads a group, a wave a superblock of 256 (per256:
// one amax over the wave, bit-exact with sml_quantize_act_sb). Every thread
// of the workgroup runs every pass, so the wave-wide max sees all 64 lanes.
#define MOE_QUANT_THREADS 1024
extern "C" __global__ __launch_bounds__(MOE_QUANT_THREADS) void sml_moe_quant(const sml_kmquant a) {
    const int r = blockIdx.x, e = blockIdx.y;
    if (r >= a.count[e]) return;
    const int n = a.n, ng = n / 32;
    const float * src = a.mode == 0 ? a.src + (size_t) (a.list[e * a.mmax + r] / a.k) * n
                                    : a.src + ((size_t) e * a.mmax + r) * n;
    const int32_t * perm = a.perms ? a.perms[e] : nullptr;
    const size_t slot = (size_t) e * a.mmax + r;
    for (int f0 = 0; f0 < n / 4; f0 += MOE_QUANT_THREADS) {
        const int f = f0 + threadIdx.x;
        const bool ok = f < n / 4;                  // whole 8-thread groups (n % 32 == 0)
        float v[4] = { 0.0f, 0.0f, 0.0f, 0.0f };
        if (ok) {
            if (perm) {
                const int4 p = ((const int4 *) perm)[f];
                v[0] = src[p.x]; v[1] = src[p.y]; v[2] = src[p.z]; v[3] = src[p.w];
            } else {
                const float4 q = ((const float4 *) src)[f];
                v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
            }
        }
        const float m4 = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
        const float am = a.per256 ? wave_max(m4) : max8(m4);
        const float s = am / 127.0f;
        const float is = s > 0.0f ? 1.0f / s : 0.0f;
        const int t0 = quant1(v[0], is), t1 = quant1(v[1], is), t2 = quant1(v[2], is), t3 = quant1(v[3], is);
        const int sum = isum8(t0 + t1 + t2 + t3);
        if (!ok) continue;
        ((int *) (a.q + slot * n))[f] = (t0 & 0xFF) | (t1 & 0xFF) << 8 | (t2 & 0xFF) << 16 | (int) ((unsigned) t3 << 24);
        if ((threadIdx.x & 7) == 0) { a.scale[slot * ng + f / 8] = s; a.sums[slot * ng + f / 8] = sum; }
    }
}

// out[t] = sum_j w[t][j] * y[sel][slot] in choice order (sml/sml-run.c:3227-3234)
extern "C" __global__ __launch_bounds__(256) void sml_moe_combine(const sml_kmoe_comb a) {
    const int t = blockIdx.y, i = blockIdx.x * 256 + threadIdx.x;
    if (i >= a.n) return;
    float acc = 0.0f;
    for (int j = 0; j < a.k; j++) {
        const int e = a.sel[t * a.k + j], r = a.slot[t * a.k + j];
        acc = __builtin_fmaf(a.w[t * a.k + j], a.y[((size_t) e * a.mmax + r) * a.n + i], acc);
    }
    const size_t o = (size_t) t * a.n + i;
    if (a.ysh) acc = __builtin_fmaf(a.sg[t], a.ysh[o], acc);          // sml/sml-run.c:3121
    a.out[o] = a.resid ? a.resid[o] + acc : acc;    // the residual add after moe_ffn, sml/sml-run.c:3475-3480
}

// ---------------------------------------------------------------- small-M GEMM
//
// The GEMV's chunk-per-lane streaming with M activation rows: each weight
// chunk is unpacked once and dotted with every row's int8 codes from LDS.
// The input is taken in passes of 64*NI chunks (4096 columns at NI 2; the
// 32-row form takes passes of 2048, so its staging fits the LDS); each pass
// issues its weight loads, then stages that slice of every row's codes and
// (s, s*sum) pairs in LDS. A lane takes chunks lane, lane+64, ... in order
// whatever NI is, so the rows' arithmetic is the GEMV's at every M. Group e
// of the grid's y dimension uses matrix table entry e (an expert) and its
// own activation slots.
#define GEMM_NI 2
template <int NB, int RB, int MT, bool SW, int WG = 256, int NI = GEMM_NI>
__device__ void gemm_body(const sml_kgemm & a) {
    constexpr int TILE = WAVE * NI;
    extern __shared__ __align__(16) uint8_t lds[];
    int8_t * lq = (int8_t *) lds;                       // [MT][TILE * 32]
    float2 * lsc = (float2 *) (lds + MT * TILE * 32);   // [MT][TILE]
    const int e = blockIdx.y;
    const int m = a.count ? a.count[e] : a.m_all;
    if (m <= a.mlo || m > MT) return;                   // another launch's groups (expert counts by size)
    const int n = a.cols, ng = n / 32, ns = (ng + 7) / 8;
    const int tid = threadIdx.x, lane = tid & (WAVE - 1);
    constexpr int RPW = SW ? RB / 2 : RB;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int row0 = (blockIdx.x * (WG / 64) + wave) * RPW;
    const sml_kmat * mt = a.mats + (size_t) e * (SW ? 2 : 1);
    const size_t abase = (size_t) e * a.mmax;
    using P = Planes<NB>;
    const uint8_t * pl[RB][3];
    uint32_t ro[RB][3];
    const uint8_t * fqb[RB];
    const uint8_t * fdb[RB];
    uint32_t fqo[RB], fdo[RB];
    int orow[RB];
    bool valid[RB];
    #pragma unroll
    for (int s = 0; s < RB; s++) {
        const int grow = row0 + (SW ? (s >> 1) : s);
        orow[s] = grow;
        valid[s] = grow < a.rows;
        const sml_kmat & mm = mt[(SW && (s & 1)) ? 1 : 0];
        const uint32_t r = (uint32_t) (valid[s] ? grow : 0);
        pl[s][0] = mm.plane[0]; pl[s][1] = mm.plane[1]; pl[s][2] = mm.plane[2];
        ro[s][0] = ro[s][1] = ro[s][2] = 0;
        if constexpr (P::N4) ro[s][P::P4] = r * (uint32_t) P::b4(n);
        if constexpr (NB == 8) ro[s][1] = r * (uint32_t) P::b4(n);
        if constexpr (P::N2) ro[s][P::P2] = r * (uint32_t) P::b2(n);
        if constexpr (P::N1) ro[s][P::P1] = r * (uint32_t) P::b1(n);
        fqb[s] = mm.sqmq;
        fdb[s] = (const uint8_t *) mm.sdmd;
        fqo[s] = r * (uint32_t) ng * 2u;
        fdo[s] = r * (uint32_t) ns * 4u;
    }
    float acc[RB][MT];
    #pragma unroll
    for (int s = 0; s < RB; s++)
        #pragma unroll
        for (int t = 0; t < MT; t++) acc[s][t] = 0.0f;
    for (int c0 = 0; c0 < ng; c0 += TILE) {
        ChunkW<NB> w[NI][RB];
        uint32_t fqv[NI][RB], fdv[NI][RB];
        #pragma unroll
        for (int i = 0; i < NI; i++) {
            const int c = c0 + i * WAVE + lane;
            const int cl = c < ng ? c : ng - 1;
            #pragma unroll
            for (int s = 0; s < RB; s++) {
                load_chunk<NB, true>(w[i][s], pl[s], ro[s], cl);
                fqv[i][s] = gld<uint16_t>(fqb[s] + (fqo[s] + (uint32_t) cl * 2u));
                fdv[i][s] = gld<uint32_t>(fdb[s] + (fdo[s] + (uint32_t) (cl >> 3) * 4u));
            }
        }
        // this pass's slice of every activation row into LDS
        const int tg = ng - c0 < TILE ? ng - c0 : TILE;  // groups in the slice
        __syncthreads();                                 // the previous pass's reads are done
        for (int idx = tid; idx < m * tg * 2; idx += WG) {
            const int t = idx / (tg * 2), wd = idx % (tg * 2);
            ((v4i *) (lq + t * TILE * 32))[wd] = ((const v4i *) (a.q + (abase + t) * n + (size_t) c0 * 32))[wd];
        }
        for (int idx = tid; idx < m * tg; idx += WG) {
            const int t = idx / tg, g = idx % tg;
            const size_t fi = (abase + t) * ng + c0 + g;
            const float sv = a.scale[fi];
            lsc[t * TILE + g] = make_float2(sv, sv * (float) a.sums[fi]);
        }
        __syncthreads();
        #pragma unroll
        for (int i = 0; i < NI; i++) {
            const int c = c0 + i * WAVE + lane;
            const bool live = c < ng;
            const int cl = (live ? c : ng - 1) - c0;     // index within the slice
            const int off = 32 * (cl & ~1) + 16 * (cl & 1);
            const int odd = c & 1;
            float wsc[RB], wmn[RB];
            #pragma unroll
            for (int s = 0; s < RB; s++) {
                const uint32_t f = fqv[i][s], d2 = fdv[i][s];
                wsc[s] = h2f((uint16_t) (d2 & 0xFFFFu)) * (float) (f & 0xFFu);
                wmn[s] = h2f((uint16_t) (d2 >> 16)) * ((float) (f >> 8) - 127.0f);
            }
            // Q4: the chunk's codes unpacked once for every row (held in
            // registers: left to itself the compiler redoes the masks per row),
            // in the order this lane keeps and sends them: an odd lane keeps
            // the high nibbles (group c|1, against the second 16 codes of the
            // pair) and sends the low ones, so no per-row select is needed
            v4u ua[RB], ub[RB];
            const unsigned shk = odd ? 4u : 0u, shs = 4u - shk;
            const int offk = off + (odd ? 32 : 0), offs = off + (odd ? 0 : 32);
            if constexpr (NB == 4) {
                #pragma unroll
                for (int s = 0; s < RB; s++) {
                    #pragma unroll
                    for (int e = 0; e < 4; e++) {
                        unsigned kp = (w[i][s].n4[e] >> shk) & 0x0F0F0F0Fu, sd = (w[i][s].n4[e] >> shs) & 0x0F0F0F0Fu;
                        asm volatile("" : "+v"(kp), "+v"(sd));
                        ua[s][e] = kp;
                        ub[s][e] = sd;
                    }
                }
            }
            #pragma unroll
            for (int t = 0; t < MT; t++) {
                if (t < m) {
                float2 sc = lsc[t * TILE + cl];
                if (!live) sc = make_float2(0.0f, 0.0f);
                int keep[RB], send[RB];
                if constexpr (NB == 4) {
                    const v4i xk = *(const v4i *) (lq + t * TILE * 32 + offk);
                    const v4i xs = *(const v4i *) (lq + t * TILE * 32 + offs);
                    #pragma unroll
                    for (int s = 0; s < RB; s++) {
                        int k = 0, d = 0;
                        #pragma unroll
                        for (int e = 0; e < 4; e++) { k = dot4(ua[s][e], xk[e], k); d = dot4(ub[s][e], xs[e], d); }
                        keep[s] = k;
                        send[s] = d;
                    }
                } else {
                    const v4i xa = *(const v4i *) (lq + t * TILE * 32 + off);
                    const v4i xb = *(const v4i *) (lq + t * TILE * 32 + off + 32);
                    #pragma unroll
                    for (int s = 0; s < RB; s++) {
                        int da, db;
                        chunk_dots<NB>(w[i][s], c, xa, xb, da, db);
                        keep[s] = odd ? db : da;
                        send[s] = odd ? da : db;
                    }
                }
                #pragma unroll
                for (int s = 0; s < RB; s++) {
                    const int dot = keep[s] + pair_swap(send[s]);
                    acc[s][t] += wsc[s] * (sc.x * (float) dot);
                    acc[s][t] += wmn[s] * sc.y;
                }
                }
            }
        }
    }
    #pragma unroll
    for (int t = 0; t < MT; t++)
        if (t < m) {
            #pragma unroll
            for (int s = 0; s < RB; s++) acc[s][t] = wave_sum_dpp(acc[s][t]);
        }
    if (lane != WAVE - 1) return;
    #pragma unroll
    for (int t = 0; t < MT; t++) {
        if (t >= m) continue;
        float * y = a.y + (abase + t) * a.rows;
        if constexpr (SW) {
            #pragma unroll
            for (int s = 0; s < RB; s += 2) {
                if (!valid[s]) continue;
                const float g = acc[s][t], u = acc[s + 1][t];
                y[orow[s]] = silu_ref(g) * u;                  // sml/sml-run.c:416-426
            }
        } else {
            const float * res = a.resid ? a.resid + (abase + t) * a.rows : nullptr;
            #pragma unroll
            for (int s = 0; s < RB; s++) {
                if (!valid[s]) continue;
                float v = acc[s][t];
                if (a.bias) v += a.bias[orow[s]];
                if (res) v = res[orow[s]] + v;
                y[orow[s]] = v;
            }
        }
    }
}

#define GEMM_KERNEL(NB, MT)                                                                              \
    extern "C" __global__ __launch_bounds__(256) void sml_gemm_q##NB##_m##MT(const sml_kgemm a) {         \
        gemm_body<NB, 2, MT, false>(a);                                                                  \
    }                                                                                                    \
    extern "C" __global__ __launch_bounds__(256) void sml_gemm_q##NB##_s_m##MT(const sml_kgemm a) {       \
        gemm_body<NB, 4, MT, true>(a);                                                                   \
    }
// 32 rows (prompt chunks read at level 1): passes of 2048 columns
#define GEMM_KERNEL_32(NB)                                                                               \
    extern "C" __global__ __launch_bounds__(256) void sml_gemm_q##NB##_m32(const sml_kgemm a) {           \
        gemm_body<NB, 2, 32, false, 256, 1>(a);                                                          \
    }                                                                                                    \
    extern "C" __global__ __launch_bounds__(256) void sml_gemm_q##NB##_s_m32(const sml_kgemm a) {         \
        gemm_body<NB, 2, 32, true, 256, 1>(a);                                                           \
    }
#define GEMM_WIDTH(NB) GEMM_KERNEL(NB, 1) GEMM_KERNEL(NB, 4) GEMM_KERNEL(NB, 8) GEMM_KERNEL(NB, 16) GEMM_KERNEL_32(NB)
GEMM_WIDTH(2) GEMM_WIDTH(3) GEMM_WIDTH(4) GEMM_WIDTH(5) GEMM_WIDTH(6) GEMM_WIDTH(7) GEMM_WIDTH(8)
// Wider workgroups (suffix _w<threads>): the same rows per wave, more waves
// sharing one staging of the activation rows per pass
#define GEMM_KERNEL_W(NB, MT, W)                                                                         \
    extern "C" __global__ __launch_bounds__(W) void sml_gemm_q##NB##_m##MT##_w##W(const sml_kgemm a) {    \
        gemm_body<NB, 2, MT, false, W>(a);                                                               \
    }                                                                                                    \
    extern "C" __global__ __launch_bounds__(W) void sml_gemm_q##NB##_s_m##MT##_w##W(const sml_kgemm a) {  \
        gemm_body<NB, 4, MT, true, W>(a);                                                                \
    }
GEMM_KERNEL_W(4, 4, 512) GEMM_KERNEL_W(4, 8, 512) GEMM_KERNEL_W(4, 16, 512)
GEMM_KERNEL_W(4, 4, 1024) GEMM_KERNEL_W(4, 8, 1024) GEMM_KERNEL_W(4, 16, 1024)

// ---------------------------------------------------------------- small-M GEMM on MFMA (Q4)
//
// The same product as gemm_body for up to 16 activation rows, with the
// per-group integer dots on v_mfma_i32_16x16x32_i8: A = 32 activation codes
// x 16 activation rows, B = 32 codes x 16 weight rows (lane layout, checked
// on the device: lane l holds A row / B column l%16, codes 8*(l/16)..+7, and
// receives D rows 4*(l/16)..+3 of column l%16). So lane l owns weight row
// l%16 of each of its RB blocks of 16 rows (SwiGLU: the gate and up blocks of
// the same rows) and activation rows 4*(l/16)..+3.
//
// Operand loads are 16 bytes per lane, the four lanes of a row contiguous:
// lane c (= l/16) reads bytes 16c..16c+15 of a 64-byte Q4 quad (columns
// 16(c&1)..+15 of groups 4q, 4q+1 if c < 2, else of 4q+2, 4q+3) and bytes
// 16c..16c+15 of an activation row's 64 bytes of 2 groups. One swap between
// lanes l and l+32 (xslice) leaves each lane an 8-byte slice of every group
// of the quad (pair): lane c holds columns 8*(0, 2, 1, 3)[c]..+7, the same
// permutation of k for A and B, so each MFMA's dot is the group's dot. A quad
// load feeds four MFMAs, an activation load two.
//
// Work goes by superblock (8 groups = 256 columns; input widths are
// multiples of 256): one 16-byte load brings a weight row's 8 (sq, mq) field
// pairs and one 4-byte load its (sd, md). The NW waves of a workgroup split
// the superblocks; each wave stages its share of the activation rows' group
// data in its own LDS region (written and read by that wave only, so no
// barrier) and keeps two superblocks' loads in flight: the first two go out
// before the staging, and each computed superblock's registers are refilled
// with the one two ahead.
//
// Two epilogues:
//  - exact (per-32 activations, sml_matvec_batch_flat4): per group
//    step*s*dot + min*s*sum in fp32, the activation's (s, s*sum) staged as
//    [group][row] float pairs;
//  - SB (per-256 activations, sml_matvec_batch_flat4_sb and sml_rlp_matvec,
//    sml/sml-kernel.c:1142-1200,1746-1840): the superblock's sums
//    sum_g sq_g*dot_g and sum_g (mq_g-127)*sum_g add in integers (24-bit
//    multiplies: |dot| <= 32*15*127 < 2^16, sq < 2^8, |sum| <= 32*127), then
//    one fp32 step per superblock: y += isum*(sd*s) + imin*(md*s), with the
//    activation's group sums staged as [group][row] ints and its superblock
//    scale as [superblock][row].
// The waves' partial sums meet in LDS, added in wave order. The float order
// differs from the GEMV's, so rows agree with it to rounding, not bit for bit.
// Two 16-byte loads' worth of k-slices, exchanged between lanes l and l+32
// (v_permlane32_swap): a lane of the first half keeps its dwords 0-1 and
// takes its partner's 0-1, a lane of the second half takes its partner's
// dwords 2-3 and keeps its own 2-3. x and y are then the lane's 8-byte slice
// of two different groups (see mgemm_q4_body). The two operands of each swap
// are distinct registers.
// The tiled copy of a Q4 matrix (sml_kmat.tiled): per 16-row block R and
// superblock b, SML_TILE_Q4 bytes holding exactly what mgemm_q4_body's 64
// lanes load for that block and superblock, in lane order: the codes of its
// two quads as [half p][lane][16 bytes] (lane l = 16c + i: row 16R + i,
// bytes 16c..16c+15 of quad p of the superblock), then each row's 8 (sq, mq)
// pairs, then each row's (sd, md). A wave's code load is then 1 KB of
// contiguous bytes, as the GEMV's is, instead of 16 rows x 64 bytes. Rows
// past the end are zero (their outputs are never stored).
extern "C" __global__ __launch_bounds__(256) void sml_tile_q4(const sml_ktile a) {
    const int nsb = a.cols / 256, ng = a.cols / 32;
    const int t = blockIdx.x, R = t / nsb, b = t % nsb, u = threadIdx.x;
    uint8_t * dst = a.out + (size_t) t * SML_TILE_Q4;
    if (u < 128) {
        const int p = u >> 6, lane = u & 63, c = lane >> 4, row = R * 16 + (lane & 15);
        v4u v = {0u, 0u, 0u, 0u};
        if (row < a.rows) v = *(const v4u *) (a.plane + (size_t) row * (a.cols / 2) + (size_t) b * 128 + 16 * c + 64 * p);
        *(v4u *) (dst + p * 1024 + lane * 16) = v;
    } else if (u < 144) {
        const int i = u - 128, row = R * 16 + i;
        v4u v = {0u, 0u, 0u, 0u};
        if (row < a.rows) v = *(const v4u *) (a.sqmq + ((size_t) row * ng + (size_t) b * 8) * 2);
        *(v4u *) (dst + 2048 + i * 16) = v;
    } else if (u < 160) {
        const int i = u - 144, row = R * 16 + i;
        uint32_t v = 0u;
        if (row < a.rows) v = *(const uint32_t *) (a.sdmd + ((size_t) row * nsb + b) * 2);
        *(uint32_t *) (dst + 2304 + i * 4) = v;
    }
}

__device__ __forceinline__ void xslice(const v4u v, v2u & x, v2u & y) {
    const auto p = __builtin_amdgcn_permlane32_swap((int) v[0], (int) v[2], false, false);
    const auto q = __builtin_amdgcn_permlane32_swap((int) v[1], (int) v[3], false, false);
    x = v2u{(unsigned) p[0], (unsigned) q[0]};
    y = v2u{(unsigned) p[1], (unsigned) q[1]};
}

template <bool SW, bool SB, int RB, int NW, bool PS = false, bool TL = false, int KS = 1>
__device__ void mgemm_q4_body(const sml_kgemm & a) {
    typedef long v1l;
    constexpr int NM = SW ? 2 : 1, NACC = NM * RB * 4;
    extern __shared__ __align__(16) uint8_t lds[];
    const int e = blockIdx.y;
    const int m = a.count ? a.count[e] : a.m_all;
    if (m <= 0) return;
    const int n = a.cols, ng = n / 32, nsb = ng / 8;
    const int tid = threadIdx.x, lane = tid & 63, c = lane >> 4, i16 = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // PS (persistent): the workgroup walks row tiles blockIdx.x, +gridDim.x,
    // ... and keeps the activation operands of its superblocks in registers
    // across them (at most 2 superblocks per wave); otherwise one tile
    // KS > 1 (split-K, persistent): workgroup g takes the input slice g % KS
    // (nsb / KS superblocks) of row tiles g / KS, + gridDim.x / KS, ... and
    // writes its products to a.part[slice]; sml_gemm_ksum adds the slices
    const int ks = KS > 1 ? (int) blockIdx.x % KS : 0;
    const int ntile = (a.rows + 16 * RB - 1) / (16 * RB);
    int tile = KS > 1 ? (int) blockIdx.x / KS : (int) blockIdx.x;
    int rb0 = tile * (16 * RB);
    const int nsbs = nsb / KS, sb0 = ks * nsbs;
    const int s0 = sb0 + wave * nsbs / NW, s1 = sb0 + (wave + 1) * nsbs / NW;   // this wave's superblocks
    const int spw = (nsbs + NW - 1) / NW;                          // region size, in superblocks
    const int gw = (s1 - s0) * 8, gb = s0 * 8;
    const sml_kmat * mt = a.mats + (size_t) e * NM;
    const size_t abase = (size_t) e * a.mmax;
    // this wave's LDS region: its share of the activation rows' group data
    uint8_t * reg = lds + (size_t) wave * spw * (SB ? 576 : 1024);
    int * lsum = (int *) reg;                                      // SB: [spw*8][16]
    float * lscl = (float *) (reg + (size_t) spw * 512);           // SB: [spw][16]
    float2 * lsc = (float2 *) reg;                                 // exact: [spw*8][16]
    const uint8_t * plane[NM];
    const uint8_t * fqb[NM];
    const uint8_t * fdb[NM];
    #pragma unroll
    for (int k = 0; k < NM; k++) {
        if (a.inl) { plane[k] = a.m0[k].plane[0]; fqb[k] = a.m0[k].sqmq; fdb[k] = (const uint8_t *) a.m0[k].sdmd; }
        else { plane[k] = mt[k].plane[0]; fqb[k] = mt[k].sqmq; fdb[k] = (const uint8_t *) mt[k].sdmd; }
    }
    const uint32_t rowb = (uint32_t) n / 2;
    uint32_t boff0[RB], fqo[RB], fdo[RB];
    // TL: the matrices' tiled copies (sml_tile_q4): the block's tile row; the
    // loads then read each tile's bytes in lane order
    const int nbl = (a.rows + 15) / 16;
    const uint8_t * tb[NM][RB];
    auto set_tile = [&](int r0) {
        #pragma unroll
        for (int bk = 0; bk < RB; bk++) {
            const int ra = r0 + bk * 16 + i16;
            const uint32_t rc = (uint32_t) (ra < a.rows ? ra : a.rows - 1);
            boff0[bk] = rc * rowb + 16u * (uint32_t) c;
            fqo[bk] = rc * (uint32_t) ng * 2u;
            fdo[bk] = rc * (uint32_t) nsb * 4u;
            if constexpr (TL) {
                const int blk = min(r0 / 16 + bk, nbl - 1);
                #pragma unroll
                for (int k = 0; k < NM; k++)
                    tb[k][bk] = (a.inl ? a.m0[k].tiled : mt[k].tiled) + (size_t) blk * nsb * SML_TILE_Q4;
            }
        }
    };
    set_tile(rb0);
    const int8_t * qrow = a.q + (abase + (size_t) (i16 < m ? i16 : 0)) * n + 16 * c;
    struct Batch {
        v4u w[2][NM][RB];         // the superblock's 2 quads, 16 bytes per lane
        v4u fq[NM][RB];           // 8 (sq, mq) pairs
        uint32_t fd[NM][RB];      // (sd, md)
        v4u aq[4];                // activation codes, 16 bytes per lane per 2 groups
    };
    // one base address per stream and superblock, the rest immediate offsets
    auto load = [&](Batch & b, int bt) {
        const int g0 = 8 * bt;
        #pragma unroll
        for (int k = 0; k < NM; k++)
            #pragma unroll
            for (int bk = 0; bk < RB; bk++) {
                if constexpr (TL) {
                    const uint8_t * tp = tb[k][bk] + (size_t) bt * SML_TILE_Q4;
                    #pragma unroll
                    for (int p = 0; p < 2; p++) b.w[p][k][bk] = gld<v4u>(tp + p * 1024 + lane * 16);
                    if (c == 0) {
                        b.fq[k][bk] = gld<v4u>(tp + 2048 + i16 * 16);
                        b.fd[k][bk] = gld<uint32_t>(tp + 2304 + i16 * 4);
                    }
                    continue;
                }
                const uint8_t * wp = plane[k] + (boff0[bk] + (uint32_t) g0 * 16u);
                #pragma unroll
                for (int p = 0; p < 2; p++) b.w[p][k][bk] = gld<v4u>(wp + p * 64);
                // a row's fields are the same for its 4 lanes: the first lane
                // of each row loads them, the others take them by ds_bpermute
                if (c == 0) {
                    b.fq[k][bk] = gld<v4u>(fqb[k] + (fqo[bk] + (uint32_t) g0 * 2u));
                    b.fd[k][bk] = gld<uint32_t>(fdb[k] + (fdo[bk] + (uint32_t) bt * 4u));
                }
            }
        if constexpr (!PS) {
            const int8_t * qp = qrow + (size_t) g0 * 32;
            #pragma unroll
            for (int u = 0; u < 4; u++) b.aq[u] = *(const v4u *) (qp + u * 64);
        }
    };
    // the activation operands of one superblock (A of group j from the
    // activation load j/2: x, y)
    auto act_operands = [&](const v4u (&aq)[4], v1l (&av)[8]) {
        #pragma unroll
        for (int u = 0; u < 4; u++) {
            v2u x, y;
            xslice(aq[u], x, y);
            av[2 * u] = (v1l) (((unsigned long) x.y << 32) | x.x);
            av[2 * u + 1] = (v1l) (((unsigned long) y.y << 32) | y.x);
        }
    };
    // the MFMA operands of one superblock: B of group j from quad j/4 (low
    // nibbles of x, high of x, low of y, high of y), A of group j from the
    // activation load j/2 (x, y)
    auto operands = [&](Batch & b, v2u (&wx)[2][NM][RB], v2u (&wy)[2][NM][RB], v1l (&av)[8]) {
        #pragma unroll
        for (int k = 0; k < NM; k++)
            #pragma unroll
            for (int bk = 0; bk < RB; bk++) {
                #pragma unroll
                for (int e = 0; e < 4; e++)
                    b.fq[k][bk][e] = (unsigned) __builtin_amdgcn_ds_bpermute(i16 << 2, (int) b.fq[k][bk][e]);
                b.fd[k][bk] = (unsigned) __builtin_amdgcn_ds_bpermute(i16 << 2, (int) b.fd[k][bk]);
            }
        #pragma unroll
        for (int p = 0; p < 2; p++)
            #pragma unroll
            for (int k = 0; k < NM; k++)
                #pragma unroll
                for (int bk = 0; bk < RB; bk++) xslice(b.w[p][k][bk], wx[p][k][bk], wy[p][k][bk]);
        if constexpr (!PS) act_operands(b.aq, av);
    };
    v1l pav[PS ? 2 : 1][8];
    auto bcodes = [&](const v2u (&wx)[2][NM][RB], const v2u (&wy)[2][NM][RB], int j, int k, int bk) -> v1l {
        const v2u w = (j & 2) ? wy[j >> 2][k][bk] : wx[j >> 2][k][bk];
        const v2u cd = (j & 1) ? ((w >> 4u) & 0x0F0F0F0Fu) : (w & 0x0F0F0F0Fu);
        return (v1l) (((unsigned long) cd.y << 32) | cd.x);
    };
    float acc[NM][RB][4];
    #pragma unroll
    for (int k = 0; k < NM; k++)
        #pragma unroll
        for (int bk = 0; bk < RB; bk++)
            #pragma unroll
            for (int r = 0; r < 4; r++) acc[k][bk][r] = 0.0f;
    auto compute = [&](Batch & b, int bt) {
        const int gl0 = (bt - s0) * 8;
        if constexpr (SB) {
            int is[NM][RB][4];
            float imf[NM][RB][4];
            #pragma unroll
            for (int k = 0; k < NM; k++)
                #pragma unroll
                for (int bk = 0; bk < RB; bk++)
                    #pragma unroll
                    for (int r = 0; r < 4; r++) is[k][bk][r] = 0;
            v2u wx[2][NM][RB], wy[2][NM][RB];
            v1l av[8];
            operands(b, wx, wy, av);
            if constexpr (PS) {
                #pragma unroll
                for (int j = 0; j < 8; j++) av[j] = bt == s0 ? pav[0][j] : pav[PS ? 1 : 0][j];
            }
            #pragma unroll
            for (int j = 0; j < 8; j++) {
                #pragma unroll
                for (int k = 0; k < NM; k++)
                    #pragma unroll
                    for (int bk = 0; bk < RB; bk++) {
                        const v1l bv = bcodes(wx, wy, j, k, bk);
                        v4i d = { 0, 0, 0, 0 };
                        d = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[j], bv, d, 0, 0, 0);
                        const uint32_t f = b.fq[k][bk][j >> 1] >> (16 * (j & 1));
                        const int sq = (int) (f & 0xFFu);
                        #pragma unroll
                        for (int r = 0; r < 4; r++) is[k][bk][r] = __mul24(sq, d[r]) + is[k][bk][r];
                    }
            }
            // the min term sum_g sums[r][g] * (mq[w][g] - 127) on the fp32
            // matrix cores, two K=4 steps over the superblock's 8 groups:
            // A = the activation rows' group sums (lane: row i16, group
            // 4kk + c), B = the weight rows' mq - 127 (lane: group 4kk + c,
            // row i16), D in the integer product's layout. Every product
            // (|sum| <= 32*127, |mq - 127| <= 128) and partial sum stays below
            // 2^24, so the fp32 sums are the integers, exactly
            float amin[2];
            #pragma unroll
            for (int kk = 0; kk < 2; kk++) amin[kk] = (float) lsum[(gl0 + 4 * kk + c) * 16 + i16];
            const uint32_t msh = 16u * (uint32_t) (c & 1) + 8u;
            #pragma unroll
            for (int k = 0; k < NM; k++)
                #pragma unroll
                for (int bk = 0; bk < RB; bk++) {
                    v4f mf = { 0.0f, 0.0f, 0.0f, 0.0f };
                    #pragma unroll
                    for (int kk = 0; kk < 2; kk++) {
                        const uint32_t wd = (c >> 1) ? b.fq[k][bk][2 * kk + 1] : b.fq[k][bk][2 * kk];
                        const float bm = (float) ((int) ((wd >> msh) & 0xFFu) - 127);
                        mf = __builtin_amdgcn_mfma_f32_16x16x4f32(amin[kk], bm, mf, 0, 0, 0);
                    }
                    #pragma unroll
                    for (int r = 0; r < 4; r++) imf[k][bk][r] = mf[r];
                }
            const float4 as = *(const float4 *) &lscl[(bt - s0) * 16 + 4 * c];
            const float asv[4] = {as.x, as.y, as.z, as.w};
            #pragma unroll
            for (int k = 0; k < NM; k++)
                #pragma unroll
                for (int bk = 0; bk < RB; bk++) {
                    const float dsc = h2f((uint16_t) (b.fd[k][bk] & 0xFFFFu)), mdsc = h2f((uint16_t) (b.fd[k][bk] >> 16));
                    #pragma unroll
                    for (int r = 0; r < 4; r++) {
                        acc[k][bk][r] += (float) is[k][bk][r] * (dsc * asv[r]);
                        acc[k][bk][r] += imf[k][bk][r] * (mdsc * asv[r]);
                    }
                }
        } else {
            v2u wx[2][NM][RB], wy[2][NM][RB];
            v1l av[8];
            operands(b, wx, wy, av);
            if constexpr (PS) {
                #pragma unroll
                for (int j = 0; j < 8; j++) av[j] = bt == s0 ? pav[0][j] : pav[PS ? 1 : 0][j];
            }
            #pragma unroll
            for (int j = 0; j < 8; j++) {
                const float4 s01 = *(const float4 *) &lsc[(gl0 + j) * 16 + 4 * c];
                const float4 s23 = *(const float4 *) &lsc[(gl0 + j) * 16 + 4 * c + 2];
                const float sv[4] = {s01.x, s01.z, s23.x, s23.z}, ssv[4] = {s01.y, s01.w, s23.y, s23.w};
                #pragma unroll
                for (int k = 0; k < NM; k++)
                    #pragma unroll
                    for (int bk = 0; bk < RB; bk++) {
                        const v1l bv = bcodes(wx, wy, j, k, bk);
                        v4i d = { 0, 0, 0, 0 };
                        d = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[j], bv, d, 0, 0, 0);
                        const uint32_t f = b.fq[k][bk][j >> 1] >> (16 * (j & 1)), d2 = b.fd[k][bk];
                        const float wsc = h2f((uint16_t) (d2 & 0xFFFFu)) * (float) (f & 0xFFu);
                        const float wmn = h2f((uint16_t) (d2 >> 16)) * ((float) ((f >> 8) & 0xFFu) - 127.0f);
                        #pragma unroll
                        for (int r = 0; r < 4; r++) {
                            acc[k][bk][r] += (wsc * sv[r]) * (float) d[r];
                            acc[k][bk][r] += wmn * ssv[r];
                        }
                    }
            }
        }
    };
    // stage this wave's share, [group][row]; rows past m read row 0 (their
    // outputs are never stored, and no output row reads another's data)
    // four entries per lane per round
    float sv[4];
    int su[4];
    auto stage_ld = [&](int base) {
        #pragma unroll
        for (int u = 0; u < 4; u++) {
            const int idx = base + 64 * u;
            if (idx < gw * 16) {
                const int r = idx / gw, gl = idx - r * gw;
                const size_t fi = (abase + (size_t) (r < m ? r : 0)) * ng + gb + gl;
                sv[u] = a.scale[fi];
                su[u] = a.sums[fi];
            }
        }
    };
    auto stage_st = [&](int base) {
        #pragma unroll
        for (int u = 0; u < 4; u++) {
            const int idx = base + 64 * u;
            if (idx < gw * 16) {
                const int r = idx / gw, gl = idx - r * gw;
                if constexpr (SB) {
                    lsum[gl * 16 + r] = su[u];
                    if ((gl & 7) == 0) lscl[(gl >> 3) * 16 + r] = sv[u];
                } else {
                    lsc[gl * 16 + r] = make_float2(sv[u], sv[u] * (float) su[u]);
                }
            }
        }
    };
    auto stage = [&]() {
        stage_ld(lane);
        stage_st(lane);
        for (int base = lane + 256; base < gw * 16; base += 256) {
            stage_ld(base);
            stage_st(base);
        }
    };
    // the waves' sums of the tile at rows r0.. meet in LDS, in wave order
    // [NW][NACC][64]: over the staging regions, or (PS) after them
    float * red = (float *) (lds + (PS ? (size_t) NW * spw * (SB ? 576 : 1024) : 0));
    auto epilogue = [&](int r0) {
        __syncthreads();                              // every wave is past its staging region / the last tile's sums
        #pragma unroll
        for (int k = 0; k < NM; k++)
            #pragma unroll
            for (int bk = 0; bk < RB; bk++)
                #pragma unroll
                for (int r = 0; r < 4; r++) {
                    red[(wave * NACC + (k * RB + bk) * 4 + r) * 64 + lane] = acc[k][bk][r];
                    acc[k][bk][r] = 0.0f;
                }
        __syncthreads();
        for (int o = tid; o < RB * 256; o += 64 * NW) {
            const int bk = o >> 8, r = (o >> 6) & 3, l = o & 63;
            const int row = r0 + bk * 16 + (l & 15), mr = 4 * (l >> 4) + r;
            if (row >= a.rows || mr >= m) continue;
            float t[NM];
            #pragma unroll
            for (int k = 0; k < NM; k++) {
                float sum = 0.0f;
                #pragma unroll
                for (int w = 0; w < NW; w++) sum += red[(w * NACC + (k * RB + bk) * 4 + r) * 64 + l];
                t[k] = sum;
            }
            if constexpr (KS > 1) {
                a.part[((size_t) ks * a.m_all + mr) * a.rows + row] = t[0];
                continue;
            }
            float * y = a.y + (abase + mr) * a.rows;
            if constexpr (SW) {
                y[row] = silu_ref(t[0]) * t[1];                          // sml/sml-run.c:416-426
            } else {
                float v = t[0];
                if (a.bias) v += a.bias[row];
                if (a.resid) v = a.resid[(abase + mr) * a.rows + row] + v;
                y[row] = v;
            }
        }
    };
    if constexpr (PS) {
        // persistent: the wave's (at most 2) superblocks of activation
        // operands, loaded once for every tile and put in place before the
        // weights are asked for (measured faster than issuing the weights
        // first: 16-row SwiGLU 2x14336x4096 per-256 24.8 against 25.4 us,
        // 6144x4096 10.0 against 10.7; and than keeping two tiles of weights
        // in flight, the next tile's asked for before this one's compute:
        // SwiGLU 22.5 against 23.7 us, at 234 registers against 203)
        const int stride = (int) gridDim.x / KS;
        #pragma unroll
        for (int k = 0; k < 2; k++) {
            v4u aq[4];
            const int bt = s0 + k < s1 ? s0 + k : s0;
            const int8_t * qp = qrow + (size_t) (8 * bt) * 32;
            #pragma unroll
            for (int u = 0; u < 4; u++) aq[u] = *(const v4u *) (qp + u * 64);
            act_operands(aq, pav[k]);
        }
        Batch A, B;
        if (s0 < s1) load(A, s0);
        if (s0 + 1 < s1) load(B, s0 + 1);
        stage();
        for (;;) {
            if (s0 < s1) compute(A, s0);
            if (s0 + 1 < s1) compute(B, s0 + 1);
            // the next tile's weights load while this one's sums meet
            const int next = tile + stride;
            if (next < ntile) {
                set_tile(next * 16 * RB);
                if (s0 < s1) load(A, s0);
                if (s0 + 1 < s1) load(B, s0 + 1);
            }
            epilogue(rb0);
            if (next >= ntile) break;
            tile = next;
            rb0 = tile * (16 * RB);
        }
    } else {
        // one tile: two superblocks in flight, then the activation rows'
        // group data (their latencies overlap), then the wave's superblocks
        // two at a time
        Batch A, B;
        if (s0 < s1) load(A, s0);
        if (s0 + 1 < s1) load(B, s0 + 1);
        stage();
        for (int bt = s0; bt < s1; bt += 2) {
            compute(A, bt);
            if (bt + 2 < s1) load(A, bt + 2);
            if (bt + 1 >= s1) break;
            compute(B, bt + 1);
            if (bt + 3 < s1) load(B, bt + 3);
        }
        epilogue(rb0);
    }
}

#define MGEMM_KERNEL(RB, NW, TL, SUF)                                                                          \
    extern "C" __global__ __launch_bounds__(64 * NW) void sml_mgemm_q4_r##RB##_w##NW##SUF(const sml_kgemm a) {  \
        mgemm_q4_body<false, false, RB, NW, false, TL>(a); }                                                   \
    extern "C" __global__ __launch_bounds__(64 * NW) void sml_mgemm_q4_s_r##RB##_w##NW##SUF(const sml_kgemm a) { \
        mgemm_q4_body<true, false, RB, NW, false, TL>(a); }                                                    \
    extern "C" __global__ __launch_bounds__(64 * NW) void sml_mgemm_q4_sb_r##RB##_w##NW##SUF(const sml_kgemm a) { \
        mgemm_q4_body<false, true, RB, NW, false, TL>(a); }                                                    \
    extern "C" __global__ __launch_bounds__(64 * NW) void sml_mgemm_q4_s_sb_r##RB##_w##NW##SUF(const sml_kgemm a) { \
        mgemm_q4_body<true, true, RB, NW, false, TL>(a); }
// suffix _t: the matrices' tiled copies (sml_kmat.tiled)
MGEMM_KERNEL(1, 4, false, ) MGEMM_KERNEL(2, 4, false, ) MGEMM_KERNEL(1, 8, false, ) MGEMM_KERNEL(2, 8, false, )
MGEMM_KERNEL(1, 4, true, _t) MGEMM_KERNEL(2, 4, true, _t) MGEMM_KERNEL(1, 8, true, _t) MGEMM_KERNEL(2, 8, true, _t)
// Persistent forms (_p): a grid smaller than the tile count, each workgroup
// keeping its activation operands for every tile it takes (input widths of
// at most 2 superblocks per wave)
#define MGEMM_KERNEL_P(RB, NW, TL, SUF)                                                                        \
    extern "C" __global__ __launch_bounds__(64 * NW) void sml_mgemm_q4_r##RB##_w##NW##_p##SUF(const sml_kgemm a) {  \
        mgemm_q4_body<false, false, RB, NW, true, TL>(a); }                                                    \
    extern "C" __global__ __launch_bounds__(64 * NW) void sml_mgemm_q4_s_r##RB##_w##NW##_p##SUF(const sml_kgemm a) { \
        mgemm_q4_body<true, false, RB, NW, true, TL>(a); }                                                     \
    extern "C" __global__ __launch_bounds__(64 * NW) void sml_mgemm_q4_sb_r##RB##_w##NW##_p##SUF(const sml_kgemm a) { \
        mgemm_q4_body<false, true, RB, NW, true, TL>(a); }                                                     \
    extern "C" __global__ __launch_bounds__(64 * NW) void sml_mgemm_q4_s_sb_r##RB##_w##NW##_p##SUF(const sml_kgemm a) { \
        mgemm_q4_body<true, true, RB, NW, true, TL>(a); }
MGEMM_KERNEL_P(1, 8, false, ) MGEMM_KERNEL_P(1, 8, true, _t)
// Split-K persistent forms (_k4): inputs of 17 to 64 superblocks (4352 to
// 16384 wide) in 4 slices, each wave holding at most 2 superblocks of its
// slice; plain products only (the SwiGLU needs whole sums)
#define MGEMM_KERNEL_K(TL, SUF)                                                                                \
    extern "C" __global__ __launch_bounds__(512) void sml_mgemm_q4_r1_w8_p_k4##SUF(const sml_kgemm a) {       \
        mgemm_q4_body<false, false, 1, 8, true, TL, 4>(a); }                                                   \
    extern "C" __global__ __launch_bounds__(512) void sml_mgemm_q4_sb_r1_w8_p_k4##SUF(const sml_kgemm a) {    \
        mgemm_q4_body<false, true, 1, 8, true, TL, 4>(a); }
MGEMM_KERNEL_K(false, ) MGEMM_KERNEL_K(true, _t)

// sml_gemm_ksum and the sml_normq2 that follows it in one launch, one
// workgroup of 256 threads a row. Each thread adds the slices of the
// elements sml_normq2's thread tid sums (4 tid.., + 1024, ...), writes them
// to y and to LDS, and sums their squares in that kernel's order; the norm
// weights and permutations of the row go to LDS beside it. Then each wave
// quantizes whole superblocks (wave w: w, w + 4, ...), 4 consecutive values
// a lane: a superblock's (or a group's) max is a max over the same values as
// sml_normq2's, and its codes, scales and sums follow the same formulas, so
// every value equals the two launches' bit for bit. Needs 4 slices, a
// residual, no bias, a norm, no exact mode, n % 32 == 0 and n <= 1024 NI;
// dynamic LDS (2 + nout) * n * 4 bytes with permutations, 2 n * 4 without.
template <int NI, bool PERM>
__device__ void ksum_normq_body(const sml_kksumq & a) {
    extern __shared__ float xs[];                  // [n] the row, [n] the norm weights, [nout][n] permutations
    __shared__ double red[4];
    const int n = a.q.n, tid = threadIdx.x;
    float * ws = xs + n;
    int * ps = (int *) (ws + n);
    const size_t ro = (size_t) blockIdx.x * n, nn = (size_t) a.s.m * n;
    const float * part = a.s.part + ro;
    // every load of the thread first, before any store to memory (a store
    // could alias a later load and hold it back), and unconditional (indexes
    // past the row clamped to its last float4), so they all go out
    // together: the 4 slices, the residual, the norm weights and the first
    // output's permutation of each of the thread's NI float4s. (No bias: the
    // products this follows have none.)
    // (the norm weights and the permutation go straight to LDS: stores there
    // cannot alias the loads; a clamped index rewrites the row's last float4
    // with its own value)
    float4 p[4][NI], r[NI];
    #pragma unroll
    for (int t = 0; t < NI; t++) {
        const int i = min(tid * 4 + t * 1024, n - 4);
        #pragma unroll
        for (int k = 0; k < 4; k++) p[k][t] = *(const float4 *) (part + (size_t) k * nn + i);
        r[t] = *(const float4 *) (a.s.resid + ro + i);
    }
    // the scheduler otherwise interleaves these with waits for the first
    // loads before the last ones are issued
    __builtin_amdgcn_sched_barrier(0);
    #pragma unroll
    for (int t = 0; t < NI; t++) {
        const int i = min(tid * 4 + t * 1024, n - 4);
        *(float4 *) (ws + i) = *(const float4 *) (a.q.norm_w + i);
        if (PERM) *(int4 *) (ps + i) = *(const int4 *) (a.q.perm[0] + i);
    }
    // the sums are unconditional too (a float4 past the row adds 0 to the
    // sum of squares), so that no load is sunk into the stores' branch
    double ss = 0.0;
    float4 v[NI];
    #pragma unroll
    for (int t = 0; t < NI; t++) {
        const bool in = tid * 4 + t * 1024 < n;
        v[t] = p[0][t];
        #pragma unroll
        for (int k = 1; k < 4; k++) {
            v[t].x += p[k][t].x; v[t].y += p[k][t].y; v[t].z += p[k][t].z; v[t].w += p[k][t].w;
        }
        v[t].x = r[t].x + v[t].x; v[t].y = r[t].y + v[t].y; v[t].z = r[t].z + v[t].z; v[t].w = r[t].w + v[t].w;
        ss = ss_add4(ss, in ? v[t] : make_float4(0.0f, 0.0f, 0.0f, 0.0f));
    }
    #pragma unroll
    for (int t = 0; t < NI; t++) {
        const int i = tid * 4 + t * 1024;
        if (i < n) {
            *(float4 *) (a.s.y + ro + i) = v[t];
            *(float4 *) (xs + i) = v[t];
        }
    }
    for (int o = 1; o < a.q.nout; o++)
        if (a.q.perm[o])
            for (int i = tid * 4; i < n; i += 1024) *(int4 *) (ps + (size_t) o * n + i) = *(const int4 *) (a.q.perm[o] + i);
    #pragma unroll
    for (int o = 32; o; o >>= 1) ss += __shfl_xor(ss, o);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    const double tot = red[0] + red[1] + red[2] + red[3];
    const float msq = (float) (tot / (double) n);
    const float sc = 1.0f / sqrtf(msq + a.q.eps);
    const size_t bg = (size_t) blockIdx.x * (n / 32);
    const int lane = tid & 63;
    for (int j0 = (tid >> 6) * 256; j0 < n; j0 += 1024) {
        const int e = j0 + 4 * lane;                 // this lane's 4 values
        const bool ok = e < n;                       // a last superblock may be partial (whole groups)
        for (int o = 0; o < a.q.nout; o++) {
            float v[4];
            float m = 0.0f;
            #pragma unroll
            for (int i = 0; i < 4; i++) {
                v[i] = 0.0f;
                if (ok) {
                    const int src = a.q.perm[o] ? ps[(size_t) o * n + e + i] : e + i;
                    v[i] = xs[src] * sc * ws[src];
                }
                m = fmaxf(m, fabsf(v[i]));
            }
            const float amax = a.q.per256 ? wave_max(m) : max8(m);
            const float s = amax / 127.0f;
            const float is = s > 0.0f ? 1.0f / s : 0.0f;
            int w = 0, sum = 0;
            #pragma unroll
            for (int i = 0; i < 4; i++) {
                const int t = quant1(v[i], is);
                sum += t;
                w |= (t & 0xFF) << (8 * i);
            }
            sum = isum8(sum);
            if (!ok) continue;
            *(int *) (a.q.q[o] + ro + e) = w;
            if ((lane & 7) == 0) { a.q.scale[o][bg + (e >> 5)] = s; a.q.sums[o][bg + (e >> 5)] = sum; }
        }
    }
}

// one kernel per NI (n <= 1024 NI) and first output's permutation (_p)
#define KSUMQ_KERNEL(NI) \
    extern "C" __global__ __launch_bounds__(256) void sml_ksum_normq_##NI(const sml_kksumq a) { ksum_normq_body<NI, false>(a); } \
    extern "C" __global__ __launch_bounds__(256) void sml_ksum_normq_##NI##_p(const sml_kksumq a) { ksum_normq_body<NI, true>(a); }
KSUMQ_KERNEL(1)
KSUMQ_KERNEL(2)
KSUMQ_KERNEL(4)

// The split-K slices added in slice order, then the bias and the residual
// (the one-launch epilogue's order: v = sum + bias; y = resid + v)
extern "C" __global__ __launch_bounds__(256) void sml_gemm_ksum(const sml_kksum a) {
    const size_t i = (size_t) blockIdx.x * 256 + threadIdx.x, n = (size_t) a.m * a.rows;
    if (i >= n) return;
    float v = a.part[i];
    for (int k = 1; k < a.ks; k++) v += a.part[(size_t) k * n + i];
    if (a.bias) v += a.bias[i % a.rows];
    if (a.resid) v = a.resid[i] + v;
    a.y[i] = v;
}



// ---------------------------------------------------------------- batched GEMM in the reference's order (exact mode)
//
// Y[p][r] = W.a[p] for the positions p of an exact-mode prompt chunk, each
// output the exact GEMV's (gemv_body EX, the reference's flat4 kernel,
// sml/sml-kernel.c:572-727) bit for bit, the weights read once for 64
// positions. Per-32 activations (s_g, sum_g per group). For each (row,
// position) the reference keeps 8 float chains, chain j taking groups j,
// j+8, ... of the row in order:
//     v_j = fma(sd*sq_g, s_g*dot_g, v_j);  v_j = fma(md*(mq_g-127), s_g*sum_g, v_j)
// then ((v0+v4)+(v1+v5)) + ((v2+v6)+(v3+v7)); y = resid + (v + bias).
// The integer dot_g comes from one v_mfma_i32_16x16x32_i8 per group and
// 16 x 16 tile (the operand layout of mgemm_q4_body: lane l holds weight row
// l%16 and positions 4(l/16)..+3 of the wave's 16). A lane runs the chains
// of its own (row, position) pairs over the groups in order, 8 chains x 4
// positions in registers (x 2 for SwiGLU: gate and up), so no value crosses
// lanes before the fold. Workgroup: 4 waves = 64 positions x 16 weight rows;
// the waves read the same weight bytes (L1). Inputs a multiple of 256 wide
// (no trailing half superblock: the caller checks). Q8 (NB 8: two nibble
// planes, code = lo + 16 hi, the reference's flat8 reads the same planes
// with the 4-bit kernel, sml/sml-kernel.c:1066-1073): dot_g = dot_lo +
// 16 dot_hi from two MFMAs, the same integer.
template <bool SW, int NB = 4>
__device__ void xgemm_q4_body(const sml_kgemm & a) {
    #pragma clang fp contract(off)
    static_assert(NB == 4 || NB == 8, "Q4 or Q8");
    constexpr int NP = NB == 8 ? 2 : 1;                       // nibble planes
    typedef long v1l;
    constexpr int NM = SW ? 2 : 1;
    const int n = a.cols, ng = n / 32, nsb = ng / 8, rows = a.rows, m_all = a.m_all;
    const int tid = threadIdx.x, lane = tid & 63, c = lane >> 4, i16 = lane & 15;
    const int wave = tid >> 6;
    const int r0 = (int) blockIdx.x * 16, p0 = (int) blockIdx.y * 64 + wave * 16;
    const int row = min(r0 + i16, rows - 1);
    const uint8_t * plane[NM][NP];
    const uint8_t * fqb[NM];
    const uint8_t * fdb[NM];
    #pragma unroll
    for (int k = 0; k < NM; k++) {
        const sml_kmat & mk = a.inl ? a.m0[k] : a.mats[k];
        #pragma unroll
        for (int pl = 0; pl < NP; pl++) plane[k][pl] = mk.plane[pl] + (size_t) row * (n / 2) + 16 * c;
        fqb[k] = mk.sqmq + (size_t) row * ng * 2;
        fdb[k] = (const uint8_t *) mk.sdmd + (size_t) row * nsb * 4;
    }
    // the A operand's activation row (position p0 + i16) and the lane's four
    // output positions' fields
    const int8_t * qrow = a.q + (size_t) min(p0 + i16, m_all - 1) * n + 16 * c;
    const float * srow[4];
    const int32_t * urow[4];
    #pragma unroll
    for (int r = 0; r < 4; r++) {
        const size_t pr = (size_t) min(p0 + 4 * c + r, m_all - 1);
        srow[r] = a.scale + pr * ng;
        urow[r] = a.sums + pr * ng;
    }
    float ch[NM][4][8];
    #pragma unroll
    for (int k = 0; k < NM; k++)
        #pragma unroll
        for (int r = 0; r < 4; r++)
            #pragma unroll
            for (int j = 0; j < 8; j++) ch[k][r][j] = 0.0f;
    for (int b = 0; b < nsb; b++) {
        v4u w[NM][NP][2], fq[NM];
        uint32_t fd[NM];
        v4u aq[4];
        #pragma unroll
        for (int k = 0; k < NM; k++) {
            #pragma unroll
            for (int pl = 0; pl < NP; pl++)
                #pragma unroll
                for (int p = 0; p < 2; p++) w[k][pl][p] = gld<v4u>(plane[k][pl] + (size_t) b * 128 + p * 64);
            fq[k] = gld<v4u>(fqb[k] + (size_t) b * 16);
            fd[k] = gld<uint32_t>(fdb[k] + (size_t) b * 4);
        }
        #pragma unroll
        for (int u = 0; u < 4; u++) aq[u] = *(const v4u *) (qrow + (size_t) b * 256 + u * 64);
        float sv[4][8];
        int uv[4][8];
        #pragma unroll
        for (int r = 0; r < 4; r++) {
            const float4 s0 = *(const float4 *) (srow[r] + 8 * b), s1 = *(const float4 *) (srow[r] + 8 * b + 4);
            const int4 u0 = *(const int4 *) (urow[r] + 8 * b), u1 = *(const int4 *) (urow[r] + 8 * b + 4);
            sv[r][0] = s0.x; sv[r][1] = s0.y; sv[r][2] = s0.z; sv[r][3] = s0.w;
            sv[r][4] = s1.x; sv[r][5] = s1.y; sv[r][6] = s1.z; sv[r][7] = s1.w;
            uv[r][0] = u0.x; uv[r][1] = u0.y; uv[r][2] = u0.z; uv[r][3] = u0.w;
            uv[r][4] = u1.x; uv[r][5] = u1.y; uv[r][6] = u1.z; uv[r][7] = u1.w;
        }
        // the operands: an 8-byte k-slice of every group in every lane, the
        // same permutation of k for A and B (see mgemm_q4_body)
        v1l av[8];
        #pragma unroll
        for (int u = 0; u < 4; u++) {
            v2u x, y;
            xslice(aq[u], x, y);
            av[2 * u] = (v1l) (((unsigned long) x.y << 32) | x.x);
            av[2 * u + 1] = (v1l) (((unsigned long) y.y << 32) | y.x);
        }
        v2u wx[NM][NP][2], wy[NM][NP][2];
        #pragma unroll
        for (int k = 0; k < NM; k++)
            #pragma unroll
            for (int pl = 0; pl < NP; pl++)
                #pragma unroll
                for (int p = 0; p < 2; p++) xslice(w[k][pl][p], wx[k][pl][p], wy[k][pl][p]);
        #pragma unroll
        for (int j = 0; j < 8; j++) {
            #pragma unroll
            for (int k = 0; k < NM; k++) {
                v4i d = {0, 0, 0, 0};
                #pragma unroll
                for (int pl = NP - 1; pl >= 0; pl--) {
                    const v2u ww = (j & 2) ? wy[k][pl][j >> 2] : wx[k][pl][j >> 2];
                    const v2u cd = (j & 1) ? ((ww >> 4u) & 0x0F0F0F0Fu) : (ww & 0x0F0F0F0Fu);
                    if (pl == 1) {
                        // the high nibbles' dot, times 16, then the low ones added on
                        d = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[j], (v1l) (((unsigned long) cd.y << 32) | cd.x), d, 0, 0, 0);
                        #pragma unroll
                        for (int r = 0; r < 4; r++) d[r] *= 16;
                    } else {
                        d = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[j], (v1l) (((unsigned long) cd.y << 32) | cd.x), d, 0, 0, 0);
                    }
                }
                const uint32_t f = fq[k][j >> 1] >> (16 * (j & 1));
                const float wsc = h2f((uint16_t) (fd[k] & 0xFFFFu)) * (float) (f & 0xFFu);
                const float wmn = h2f((uint16_t) (fd[k] >> 16)) * ((float) ((f >> 8) & 0xFFu) - 127.0f);
                #pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float s = sv[r][j];
                    ch[k][r][j] = __builtin_fmaf(wsc, s * (float) d[r], ch[k][r][j]);
                    ch[k][r][j] = __builtin_fmaf(wmn, s * (float) uv[r][j], ch[k][r][j]);
                }
            }
        }
    }
    if (r0 + i16 >= rows) return;
    #pragma unroll
    for (int r = 0; r < 4; r++) {
        const int p = p0 + 4 * c + r;
        if (p >= m_all) continue;
        float v[NM];
        #pragma unroll
        for (int k = 0; k < NM; k++) {
            const float (&q)[8] = ch[k][r];
            v[k] = ((q[0] + q[4]) + (q[1] + q[5])) + ((q[2] + q[6]) + (q[3] + q[7]));
        }
        float * y = a.y + (size_t) p * rows;
        const int rr = r0 + i16;
        if constexpr (SW) {
            y[rr] = silu_ref(v[0]) * v[1];                                       // sml/sml-run.c:416-426
        } else {
            float o = v[0];
            if (a.bias) o += a.bias[rr];
            if (a.resid) o = a.resid[(size_t) p * rows + rr] + o;
            y[rr] = o;
        }
    }
}
extern "C" __global__ __launch_bounds__(256) void sml_xgemm_q4(const sml_kgemm a) { xgemm_q4_body<false>(a); }
extern "C" __global__ __launch_bounds__(256) void sml_xgemm_q4_s(const sml_kgemm a) { xgemm_q4_body<true>(a); }
extern "C" __global__ __launch_bounds__(256) void sml_xgemm_q8(const sml_kgemm a) { xgemm_q4_body<false, 8>(a); }
extern "C" __global__ __launch_bounds__(256) void sml_xgemm_q8_s(const sml_kgemm a) { xgemm_q4_body<true, 8>(a); }

// ---------------------------------------------------------------- prompt GEMM on MFMA (Q4, per-256 activations)
//
// Y[p][r] = W.a[p] for a chunk of prompt positions p (hundreds) and every row
// r of a Q4 matrix, in the reference's prompt regime (sml_quantize_act_sb and
// flat4_sb_body, sml/sml-kernel.c:115-185,1142-1190): per superblock b of 256
// columns the integer sums
//     isum = sum_g sq_g * dot_g,    imin = sum_g (mq_g - 127) * sum(q_g),
// then y += isum * (sd_b * s_b) + imin * (md_b * s_b) in fp32 (s_b: the
// position's activation scale of superblock b).
//
// Workgroup tile: 128 weight rows x 32 positions (SwiGLU: 64 rows of gate
// and the same 64 rows of up), 4 waves of 32 rows (SwiGLU: 16 gate + 16 up)
// x 32 positions, i.e. 2 x 2 tiles of v_mfma_i32_16x16x32_i8 per group (lane
// layout as in mgemm_q4_body: lane l holds A row / B column l%16 and k =
// 8(l/16)..+7, and receives D rows 4(l/16)..+3 of column l%16, so it owns one
// weight row of each tile and four positions).
//  - dot_g: one MFMA per (tile, group); A = the positions' int8 codes, B =
//    the group's 4-bit codes as bytes; sq_g * dot_g adds up on the VALU in
//    24-bit multiply-adds (|dot_g| < 2^16, sq_g < 2^8).
//  - imin: one MFMA per (tile, group) with B = (mq_g - 128) in every byte
//    (an int8 for every mq_g), so the product is (mq_g - 128) * sum(q_g),
//    accumulated over the superblock's 8 groups in the MFMA's own
//    accumulator; the superblock's sum of q (from the activation's group
//    sums, staged with its scale) then makes it sum_g (mq_g - 127) * sum(q_g).
// Each superblock's weight tile (128 rows x 128 bytes) and activation tile
// (32 positions x 256 bytes) are staged in LDS, double-buffered: the next
// superblock's global loads are in flight while this one computes. In LDS a
// weight row keeps, per k-slice kq, its four 8-byte chunks (quad, half) side
// by side; an activation row keeps, per kq, its 8 groups' 8-byte slices side
// by side (16 bytes of padding per row: no bank conflicts across the 16 rows
// a wave reads at once). The fields (sq, mq per group; sd, md per superblock)
// go straight to registers, one lane per row.
//
// Tiles are numbered so that consecutive ones share their weight rows and
// sit on one XCD (workgroup i runs on XCD i mod 8): the positions' tiles of a
// weight tile find it in that XCD's L2.
//
// Q6 (NB = 6; the file's 4-bit plane holds code bits 0-3 in the Q4 layout,
// its 2-bit plane bits 4-5): the 2-bit plane's tile (128 rows x 64 bytes a
// superblock; per group quad 32 bytes, byte j holding column j of its four
// groups at bits 2(g%4)) is staged beside the nibbles, and each group's B
// operand is nibble | bits << 4, a code 0..63 (|dot_g| < 2^18, sq_g * dot_g
// < 2^26: the integer sums hold). The fields are Q4's (widened to bytes at
// upload). The reference's per-256 Q6 prompt kernel
// (sml_matvec_batch_flat6_sb, sml/sml-kernel.c:1604-1619) sums the 2-bit
// plane's part and the nibbles' part in two fp32 passes; the integers here
// are its integers, the fp32 order another.
#define PG_BN 128
#define PG_BM 32
#define PG_BROW 144
#define PG_AROW 272
#define PG_HROW 72
#define PG_STAGE (PG_BN * PG_BROW + PG_BM * PG_AROW + PG_BM * 8)
#define PG_STAGE6 (PG_STAGE + PG_BN * PG_HROW)

template <int NB, bool SW>
__device__ void pgemm_q4_body(const sml_kgemm & a) {
    constexpr int STG = NB == 6 ? PG_STAGE6 : PG_STAGE;
    typedef long v1l;
    extern __shared__ __align__(16) uint8_t lds[];
    const int n = a.cols, ng = n / 32, nsb = n / 256, m_all = a.m_all, rows = a.rows;
    const int tid = threadIdx.x, lane = tid & 63, kq = lane >> 4, i16 = lane & 15;
    constexpr int MT = PG_BM / 16, AWN = PG_BM / 16;          // m-tiles per wave, activation words per thread
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    constexpr int RT = SW ? PG_BN / 2 : PG_BN;                 // output rows per tile
    const int nrt = (rows + RT - 1) / RT, npt = (m_all + PG_BM - 1) / PG_BM, total = nrt * npt;
    const int id = blockIdx.x, xcd = id & 7, slot = id >> 3, q8 = total >> 3, rem = total & 7;
    const int lid = (xcd < rem ? xcd * (q8 + 1) : rem * (q8 + 1) + (xcd - rem) * q8) + slot;
    const int rt = lid / npt, pt = lid - rt * npt;
    const int r0 = rt * RT, p0 = pt * PG_BM;
    const uint32_t rowb = (uint32_t) n / 2;

    // staging: thread t copies 16-byte words t + 256i of the weight tile
    // (row w/8 = t/8 + 32i, bytes 16(t%8)..; SwiGLU: i < 2 gate, i >= 2 up)
    // and of the activation tile (position t/16 + 16i, bytes 16(t%16)..);
    // rows and positions past the end read the last one. 32-bit offsets:
    // the host keeps rows x cols / 2 and positions x cols below 2^32.
    constexpr int NIB = NB == 6 ? 1 : 0;                        // the nibble plane's index
    const uint8_t * bplane[2] = {a.mats[0].plane[NIB], a.mats[SW ? 1 : 0].plane[NIB]};
    uint32_t boff[4], aoff[AWN];
    // Q6: the 2-bit plane's words (row w/4 = t/4 + 64i, bytes 16(t%4)..)
    const uint8_t * hplane[2] = {a.mats[0].plane[0], a.mats[SW ? 1 : 0].plane[0]};
    uint32_t hoff[2];
    #pragma unroll
    for (int i = 0; i < 2; i++) {
        const int lr = (tid >> 2) + 64 * i, rr = SW ? (lr & 63) : lr;
        hoff[i] = (uint32_t) min(r0 + rr, rows - 1) * ((uint32_t) n / 4) + 16u * (uint32_t) (tid & 3);
    }
    #pragma unroll
    for (int i = 0; i < 4; i++) {
        const int lr = (tid >> 3) + 32 * i, rr = SW ? (lr & 63) : lr;
        boff[i] = (uint32_t) min(r0 + rr, rows - 1) * rowb + 16u * (uint32_t) (tid & 7);
    }
    #pragma unroll
    for (int i = 0; i < AWN; i++)
        aoff[i] = (uint32_t) min(p0 + (tid >> 4) + 16 * i, m_all - 1) * (uint32_t) n + 16u * (uint32_t) (tid & 15);
    const int jb = tid & 7, ja = tid & 15;
    const uint32_t bdst0 = (uint32_t) ((tid >> 3) * PG_BROW + (2 * (jb & 1)) * 32 + (2 * (jb >> 2) + ((jb >> 1) & 1)) * 8);
    const uint32_t adst0 = (uint32_t) (PG_BN * PG_BROW + (tid >> 4) * PG_AROW + (2 * (ja & 1)) * 64 + (ja >> 1) * 8);
    const float * ssrc = a.scale + (size_t) min(p0 + (tid & (PG_BM - 1)), m_all - 1) * ng;
    const int32_t * usrc = a.sums + (size_t) min(p0 + (tid & (PG_BM - 1)), m_all - 1) * ng;
    // this wave's two 16-row blocks (LDS row of the block's first row, and
    // the lane's global row)
    int lrow[2], grow[2];
    #pragma unroll
    for (int t = 0; t < 2; t++) {
        lrow[t] = SW ? t * 64 + 16 * wave : 32 * wave + 16 * t;
        grow[t] = r0 + (SW ? 16 * wave : 32 * wave + 16 * t) + i16;
    }
    const uint8_t * fqb[2];
    const uint8_t * fdb[2];
    #pragma unroll
    for (int t = 0; t < 2; t++) {
        const sml_kmat & m = a.mats[SW ? t : 0];
        const size_t gr = (size_t) min(grow[t], rows - 1);
        fqb[t] = m.sqmq + gr * (size_t) ng * 2;
        fdb[t] = (const uint8_t *) m.sdmd + gr * (size_t) nsb * 4;
    }

    v4u bw[4], aw[AWN], hw[2];
    float sw_ = 0.0f;
    int4 su0 = make_int4(0, 0, 0, 0), su1 = su0;
    v4u fq[2], fqn[2];
    uint32_t fd[2], fdn[2];
    auto fetch = [&](int b, v4u (&q)[2], uint32_t (&d)[2]) {
        #pragma unroll
        for (int i = 0; i < 4; i++)
            bw[i] = __builtin_nontemporal_load((const GLOBAL v4u *) (bplane[SW && i >= 2] + (boff[i] + 128u * (uint32_t) b)));
        if constexpr (NB == 6) {
            #pragma unroll
            for (int i = 0; i < 2; i++)
                hw[i] = __builtin_nontemporal_load((const GLOBAL v4u *) (hplane[SW && i >= 1] + (hoff[i] + 64u * (uint32_t) b)));
        }
        #pragma unroll
        for (int i = 0; i < AWN; i++) aw[i] = *(const v4u *) (a.q + (aoff[i] + 256u * (uint32_t) b));
        if (tid < PG_BM) {
            sw_ = ssrc[8 * b];
            su0 = *(const int4 *) (usrc + 8 * b);
            su1 = *(const int4 *) (usrc + 8 * b + 4);
        }
        #pragma unroll
        for (int t = 0; t < 2; t++) {
            q[t] = gld<v4u>(fqb[t] + (size_t) b * 16);
            d[t] = gld<uint32_t>(fdb[t] + (size_t) b * 4);
        }
    };
    auto stage = [&](int buf) {
        uint8_t * base = lds + (size_t) buf * STG;
        if constexpr (NB == 6) {
            #pragma unroll
            for (int i = 0; i < 2; i++) {
                uint8_t * hd = base + PG_STAGE + ((tid >> 2) + 64 * i) * PG_HROW + 16 * (tid & 3);
                *(v2u *) hd = v2u{hw[i][0], hw[i][1]};
                *(v2u *) (hd + 8) = v2u{hw[i][2], hw[i][3]};
            }
        }
        #pragma unroll
        for (int i = 0; i < 4; i++) {
            uint8_t * bd = base + bdst0 + i * 32 * PG_BROW;
            *(v2u *) bd = v2u{bw[i][0], bw[i][1]};
            *(v2u *) (bd + 32) = v2u{bw[i][2], bw[i][3]};
        }
        #pragma unroll
        for (int i = 0; i < AWN; i++) {
            uint8_t * ad = base + adst0 + i * 16 * PG_AROW;
            *(v2u *) ad = v2u{aw[i][0], aw[i][1]};
            *(v2u *) (ad + 64) = v2u{aw[i][2], aw[i][3]};
        }
        if (tid < PG_BM) {
            float * sd_ = (float *) (base + PG_BN * PG_BROW + PG_BM * PG_AROW);
            sd_[tid] = sw_;
            ((int *) (sd_ + PG_BM))[tid] = (su0.x + su0.y) + (su0.z + su0.w) + ((su1.x + su1.y) + (su1.z + su1.w));
        }
    };

    float acc[2][MT][4];
    #pragma unroll
    for (int t = 0; t < 2; t++)
        #pragma unroll
        for (int mt = 0; mt < MT; mt++)
            #pragma unroll
            for (int r = 0; r < 4; r++) acc[t][mt][r] = 0.0f;

    auto compute = [&](int buf) {
        const uint8_t * base = lds + (size_t) buf * STG;
        const uint8_t * abase = base + PG_BN * PG_BROW;
        const float * sbase = (const float *) (abase + PG_BM * PG_AROW);
        const int * ubase = (const int *) (sbase + PG_BM);
        // the lane's weight row: its 4 chunks of k-slice kq (quad, half)
        v4u pk[2][2];
        #pragma unroll
        for (int t = 0; t < 2; t++) {
            const uint8_t * p = base + (lrow[t] + i16) * PG_BROW + kq * 32;
            pk[t][0] = *(const v4u *) p;
            pk[t][1] = *(const v4u *) (p + 16);
        }
        // Q6: the lane's 8 bytes of k-slice kq in each group quad of the 2-bit plane
        v2u hk[2][2];
        if constexpr (NB == 6) {
            #pragma unroll
            for (int t = 0; t < 2; t++) {
                const uint8_t * p = base + PG_STAGE + (lrow[t] + i16) * PG_HROW + kq * 8;
                hk[t][0] = *(const v2u *) p;
                hk[t][1] = *(const v2u *) (p + 32);
            }
        }
        int is[2][MT][4];
        v4i im[2][MT];
        #pragma unroll
        for (int t = 0; t < 2; t++)
            #pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                im[t][mt] = v4i{0, 0, 0, 0};
                #pragma unroll
                for (int r = 0; r < 4; r++) is[t][mt][r] = 0;
            }
        #pragma unroll
        for (int g = 0; g < 8; g++) {
            // order the groups: the sums so far pass through an (empty)
            // volatile statement, so this group's MFMAs cannot be issued
            // before the last group's multiply-adds have consumed its results
            // (pure arithmetic is otherwise free to move, and all eight
            // groups' products would be held in registers at once)
            #pragma unroll
            for (int t = 0; t < 2; t++)
                #pragma unroll
                for (int mt = 0; mt < MT; mt++)
                    asm volatile("" : "+v"(is[t][mt][0]), "+v"(is[t][mt][1]), "+v"(is[t][mt][2]), "+v"(is[t][mt][3]));
            const int c = 2 * (g >> 2) + ((g >> 1) & 1), sh = 4 * (g & 1);
            v1l bc[2], bm[2];
            int sq[2];
            #pragma unroll
            for (int t = 0; t < 2; t++) {
                unsigned lo = (pk[t][c >> 1][2 * (c & 1)] >> sh) & 0x0F0F0F0Fu;
                unsigned hi = (pk[t][c >> 1][2 * (c & 1) + 1] >> sh) & 0x0F0F0F0Fu;
                if constexpr (NB == 6) {
                    const v2u h = hk[t][g >> 2];
                    lo |= ((h.x >> (2 * (g & 3))) & 0x03030303u) << 4;
                    hi |= ((h.y >> (2 * (g & 3))) & 0x03030303u) << 4;
                }
                bc[t] = (v1l) (((unsigned long) hi << 32) | lo);
                const uint32_t f = fq[t][g >> 1] >> (16 * (g & 1));
                sq[t] = (int) (f & 0xFFu);
                const unsigned m4 = (((f >> 8) & 0xFFu) ^ 0x80u) * 0x01010101u;     // mq - 128 as int8
                bm[t] = (v1l) (((unsigned long) m4 << 32) | m4);
            }
            #pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                const v1l av = *(const v1l *) (abase + (16 * mt + i16) * PG_AROW + kq * 64 + g * 8);
                #pragma unroll
                for (int t = 0; t < 2; t++) {
                    v4i d = {0, 0, 0, 0};
                    d = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, bc[t], d, 0, 0, 0);
                    im[t][mt] = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, bm[t], im[t][mt], 0, 0, 0);
                    #pragma unroll
                    for (int r = 0; r < 4; r++) is[t][mt][r] = __mul24(sq[t], d[r]) + is[t][mt][r];
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        #pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const float4 s4 = *(const float4 *) (sbase + 16 * mt + 4 * kq);
            const int4 u4 = *(const int4 *) (ubase + 16 * mt + 4 * kq);
            const float sv[4] = {s4.x, s4.y, s4.z, s4.w};
            const int uv[4] = {u4.x, u4.y, u4.z, u4.w};
            #pragma unroll
            for (int t = 0; t < 2; t++) {
                const float dsc = h2f((uint16_t) (fd[t] & 0xFFFFu)), mdsc = h2f((uint16_t) (fd[t] >> 16));
                #pragma unroll
                for (int r = 0; r < 4; r++) {
                    acc[t][mt][r] += (float) is[t][mt][r] * (dsc * sv[r]);
                    acc[t][mt][r] += (float) (im[t][mt][r] + uv[r]) * (mdsc * sv[r]);
                }
            }
        }
    };

    fetch(0, fq, fd);
    stage(0);
    __syncthreads();
    for (int b = 0; b < nsb; b++) {
        const bool more = b + 1 < nsb;
        if (more) fetch(b + 1, fqn, fdn);
        compute(b & 1);
        if (more) {
            stage((b + 1) & 1);
            #pragma unroll
            for (int t = 0; t < 2; t++) { fq[t] = fqn[t]; fd[t] = fdn[t]; }
        }
        __syncthreads();
    }

    #pragma unroll
    for (int mt = 0; mt < MT; mt++)
        #pragma unroll
        for (int r = 0; r < 4; r++) {
            const int pos = p0 + 16 * mt + 4 * kq + r;
            if (pos >= m_all) continue;
            float * y = a.y + (size_t) pos * rows;
            if constexpr (SW) {
                const int row = grow[0];
                if (row < rows) y[row] = silu_ref(acc[0][mt][r]) * acc[1][mt][r];        // sml/sml-run.c:416-426
            } else {
                #pragma unroll
                for (int t = 0; t < 2; t++) {
                    const int row = grow[t];
                    if (row >= rows) continue;
                    float v = acc[t][mt][r];
                    if (a.bias) v += a.bias[row];
                    if (a.resid) v = a.resid[(size_t) pos * rows + row] + v;
                    y[row] = v;
                }
            }
        }
}

extern "C" __global__ __launch_bounds__(256, 2) void sml_pgemm_q4(const sml_kgemm a) { pgemm_q4_body<4, false>(a); }
extern "C" __global__ __launch_bounds__(256, 2) void sml_pgemm_q4_s(const sml_kgemm a) { pgemm_q4_body<4, true>(a); }
extern "C" __global__ __launch_bounds__(256, 2) void sml_pgemm_q6(const sml_kgemm a) { pgemm_q4_body<6, false>(a); }
extern "C" __global__ __launch_bounds__(256, 2) void sml_pgemm_q6_s(const sml_kgemm a) { pgemm_q4_body<6, true>(a); }
