/*
 * gfx950 kernels of the packed-weight matrix-vector path.
 *
 * Mapping: one wavefront owns a 64-row tile (lane l = row l of the tile) and
 * walks a contiguous range of K-units of that tile; a workgroup stacks up to
 * 8 such waves along K and a launch may split K further across workgroups.
 * Because every lane of a wave sits at the same K position, the activation
 * values are wave-uniform: the compiler reads them with scalar loads into
 * SGPRs and every FMA takes x as its SGPR operand, so x costs no VGPRs, no
 * LDS and no per-lane traffic. Each lane accumulates its own row, so no
 * cross-lane reduction is needed per row; waves of a workgroup combine
 * through LDS, split workgroups through a workspace with a last-arriver
 * reduction (both in fixed order, so results are run-to-run identical).
 *
 * Decode happens in registers from 16-byte plane loads (see qmv_layout.h):
 * nibbles/bit-fields are isolated four at a time in the bytes of a dword and
 * converted with byte-select conversions.
 *   M == 1: affine terms are factored per scale group,
 *           sum((a*q - b) x) = a*sum(q x) - b*sum(x),
 *           with the group sums of x computed once per unit by the wave.
 *   M >= 2: each weight is decoded exactly (bit-identical to the reference's
 *           dequantisation) and reused for all M positions.
 */
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qmv_kernels.h"

namespace qmv {

/* ---- small device helpers ----------------------------------------------- */

__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits)
{
    const unsigned short s = (unsigned short)(bits & 0xffffu);
    _Float16 h;
    __builtin_memcpy(&h, &s, sizeof h);
    return (float)h;
}

/* Byte k of v as a float; the backend selects v_cvt_f32_ubyte<k>. */
__device__ __forceinline__ float ubyte(uint32_t v, int k)
{
    return (float)((v >> (8 * k)) & 0xffu);
}

/* v with its bit pattern hidden from the optimiser. Applied to a dword of
 * packed codes after masking, so that each byte converts with a single
 * v_cvt_f32_ubyte<k>: otherwise the mask is folded into every byte as a
 * separate bit-field extract before a byte-0 conversion. */
__device__ __forceinline__ uint32_t codes(uint32_t v)
{
    asm("" : "+v"(v));
    return v;
}

__device__ __forceinline__ float sbyte(uint32_t v, int k)
{
    return (float)(int)(int8_t)((v >> (8 * k)) & 0xffu);
}

/* A 4-bit code q held as an integer in bits 0..7 of a 16-bit half reads as
 * the f16 subnormal q * 2^-24 (16q * 2^-24 for a code in bits 4..7), which
 * v_fma_mix_f32 widens exactly inside the FMA. fmaf(f16lo(v), x, s) thus adds
 * q * x * 2^-24 with one rounding: the rounding of fmaf((float)q, x, s') on a
 * sum scaled by 2^-24, which is exact while sums stay above the fp32
 * subnormal range (2^-102 unscaled). One instruction per weight instead of a
 * byte conversion and an FMA. */
__device__ __forceinline__ float f16lo(uint32_t v)
{
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(v & 0xffffu));
}
__device__ __forceinline__ float f16hi(uint32_t v)
{
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(v >> 16));
}

/* Accumulate the 4 byte codes (each < 1024) of dword q against x[0..3], in
 * byte order, on a sum scaled by 2^-24 (f16lo above). */
__device__ __forceinline__ float byte_codes_mix(uint32_t q, const float *x, float a)
{
    /* bytes 0,2 | bytes 1,3 (v_perm_b32 selector 0x0c = zero byte) */
    const uint32_t ev = q & 0x00ff00ffu, od = __builtin_amdgcn_perm(0u, q, 0x0c030c01u);
    a = fmaf(f16lo(ev), x[0], a);
    a = fmaf(f16lo(od), x[1], a);
    a = fmaf(f16hi(ev), x[2], a);
    a = fmaf(f16hi(od), x[3], a);
    return a;
}

/* Accumulate the 4 low-nibble codes of dword dw (bytes 0..3) against x[0..3]
 * into l and the 4 high-nibble codes (as 16q) against x[16..19] into h, in
 * byte order, on sums scaled by 2^-24 (f16lo above). */
__device__ __forceinline__ void q4_dword_mix(uint32_t dw, const float *x, float &l, float &h)
{
    const uint32_t s = dw >> 8;
    const uint32_t le = dw & 0x000f000fu, lo = s & 0x000f000fu; /* bytes 0,2 | 1,3 */
    const uint32_t he = dw & 0x00f000f0u, ho = s & 0x00f000f0u;
    l = fmaf(f16lo(le), x[0], l);
    l = fmaf(f16lo(lo), x[1], l);
    l = fmaf(f16hi(le), x[2], l);
    l = fmaf(f16hi(lo), x[3], l);
    h = fmaf(f16lo(he), x[16], h);
    h = fmaf(f16lo(ho), x[17], h);
    h = fmaf(f16hi(he), x[18], h);
    h = fmaf(f16hi(ho), x[19], h);
}

__device__ __forceinline__ float lane_value(float v, int lane)
{
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

__device__ __forceinline__ float xor_sum(float v, int mask)
{
    return v + __shfl_xor(v, mask, 64);
}

/* Spread 4 bits b0..b3 to bit 4 of bytes 0..3 (fifth bit of Q5_0 codes). */
__device__ __forceinline__ uint32_t spread_bits4(uint32_t b)
{
    return ((b * 0x00204081u) & 0x01010101u) << 4;
}

/* ---- per-format unit storage and loads ---------------------------------- */

struct Q4KUnit { uint4 p[9]; };
struct Q6KUnit { uint4 p[13]; uint32_t d; };
struct Q80Unit { uint4 qs[8]; uint2 d; };
struct Q50Unit { uint4 qs[4]; uint4 qh; uint2 d; };

template <int FMT> struct UnitOf;
template <> struct UnitOf<QMV_FMT_Q4_K> { using T = Q4KUnit; static constexpr int kBytes = 144, kWeights = 256; };
template <> struct UnitOf<QMV_FMT_Q6_K> { using T = Q6KUnit; static constexpr int kBytes = 210, kWeights = 256; };
template <> struct UnitOf<QMV_FMT_Q8_0> { using T = Q80Unit; static constexpr int kBytes = 136, kWeights = 128; };
template <> struct UnitOf<QMV_FMT_Q5_0> { using T = Q50Unit; static constexpr int kBytes = 88, kWeights = 128; };

__device__ __forceinline__ uint4 ld16(const uint8_t *p) { return *(const uint4 *)p; }

__device__ __forceinline__ void load_unit(Q4KUnit &u, const uint8_t *slab, int lane)
{
#pragma unroll
    for (int p = 0; p < 9; ++p) u.p[p] = ld16(slab + p * 1024 + lane * 16);
}

__device__ __forceinline__ void load_unit(Q6KUnit &u, const uint8_t *slab, int lane)
{
#pragma unroll
    for (int p = 0; p < 13; ++p) u.p[p] = ld16(slab + p * 1024 + lane * 16);
    u.d = *(const unsigned short *)(slab + 13312 + lane * 2);
}

__device__ __forceinline__ void load_unit(Q80Unit &u, const uint8_t *slab, int lane)
{
#pragma unroll
    for (int p = 0; p < 8; ++p) u.qs[p] = ld16(slab + p * 1024 + lane * 16);
    u.d = *(const uint2 *)(slab + 8192 + lane * 8);
}

__device__ __forceinline__ void load_unit(Q50Unit &u, const uint8_t *slab, int lane)
{
#pragma unroll
    for (int p = 0; p < 4; ++p) u.qs[p] = ld16(slab + p * 1024 + lane * 16);
    u.qh = ld16(slab + 4096 + lane * 16);
    u.d = *(const uint2 *)(slab + 5120 + lane * 8);
}

__device__ __forceinline__ uint32_t word(const uint4 &v, int e)
{
    return e == 0 ? v.x : e == 1 ? v.y : e == 2 ? v.z : v.w;
}
__device__ __forceinline__ uint32_t word(const uint2 &v, int e) { return e == 0 ? v.x : v.y; }

/* Activations are read through constant-address-space pointers: the
 * activations are read-only while a kernel runs, and the constant space lets
 * uniform reads be scalar loads even where the kernel also stores to global
 * memory (a global-space read is kept scalar only when no store of the
 * kernel could reach it). kGuard marks the partial last unit of a Q8_0/Q5_0
 * row: K is a multiple of 32, so it only lacks whole blocks, whose regions
 * are skipped. */
typedef const float __attribute__((address_space(4))) gfloat;

/* Activation loads are ordered by data dependencies alone. The pointer of
 * region p+1 is passed through an empty asm that also consumes one
 * activation of region p (an SGPR) and the accumulators left by region p-1
 * (VGPRs). So region p's scalar loads have landed before region p+1's are
 * issued, region p-1's FMAs are done (its activations dead) before that, and
 * no optimiser can merge, hoist or sink work across regions: at most two
 * regions of activations are live in SGPRs. The result is still a uniform
 * constant-space pointer, so the loads stay scalar. */
__device__ __forceinline__ gfloat *region_ptr(const float *p, float dep_s, float dep_v0, float dep_v1)
{
    gfloat *g = (gfloat *)p;
    asm("" : "+s"(g) : "s"(dep_s), "v"(dep_v0), "v"(dep_v1));
    return g;
}

/* A value that exists only once every acc[m] exists (an ordering token). */
template <int M>
__device__ __forceinline__ float all_of(const float (&acc)[M])
{
    float t = acc[0];
#pragma unroll
    for (int m = 1; m < M; ++m) asm("" : "+v"(t) : "v"(acc[m]));
    return t;
}

/* A weight word that cannot be decoded before `dep` exists: ties the decode of
 * region r to the accumulators of region r-1 so decodes are not hoisted. */
__device__ __forceinline__ uint32_t after(uint32_t w, float dep)
{
    asm("" : "+v"(w) : "v"(dep));
    return w;
}

/* Sum of the W/64 consecutive x values owned by this lane (W = unit width);
 * shuffles then combine lanes into per-scale-group sums of x. */
template <int W, bool kGuard>
__device__ __forceinline__ float unit_x_partial(const float *__restrict__ xu, int lane, int kleft)
{
    if constexpr (W == 256) {
        const int k = 4 * lane;
        if (kGuard && k >= kleft) return 0.0f;
        const float4 v = *(const float4 *)(xu + k);
        return (v.x + v.y) + (v.z + v.w);
    } else {
        const int k = 2 * lane;
        if (kGuard && k >= kleft) return 0.0f;
        const float2 v = *(const float2 *)(xu + k);
        return v.x + v.y;
    }
}

/* ---- per-format regions --------------------------------------------------
 * A region is a fixed set of weights of one unit together with the K index
 * of each (all compile-time after unrolling). The M == 1 path uses 32-weight
 * regions and factored scale groups; the M >= 2 path uses 8-weight regions of
 * exactly decoded weights. */

/* Q4_K header dwords: h0 = d | dmin << 16, h1 = scale bytes 0..3, h2 =
 * 4..7, h3 = 8..11. Sub-block s < 4: sc = byte s of h1 & 63, m = byte s of
 * h2 & 63; s >= 4: sc = (byte s-4 of h3 & 15) | (byte s-4 of h1 >> 6) << 4,
 * m = (byte s-4 of h3 >> 4) | (byte s-4 of h2 >> 6) << 4. Plane 1 + 2g + h
 * holds qs bytes 32g + 16h .. +15: low nibbles are weights 64g + 16h + i
 * (sub-block 2g), high nibbles 64g + 32 + 16h + i (sub-block 2g + 1). The
 * high nibble is used in place as 16*q (mask 0xF0) with 1/16 folded into its
 * scale, which is exact. */
struct Q4KScales { float a[8]; float m[8]; };

__device__ __forceinline__ Q4KScales q4k_scales(const uint4 &h)
{
    const float d = f16_bits_to_f32(h.x);
    const float dmin = f16_bits_to_f32(h.x >> 16);
    const uint32_t sc_lo = h.y & 0x3f3f3f3fu;
    const uint32_t m_lo = h.z & 0x3f3f3f3fu;
    const uint32_t sc_hi = (h.w & 0x0f0f0f0fu) | ((h.y >> 2) & 0x30303030u);
    const uint32_t m_hi = ((h.w >> 4) & 0x0f0f0f0fu) | ((h.z >> 2) & 0x30303030u);
    Q4KScales s;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t scw = i < 4 ? sc_lo : sc_hi, mw = i < 4 ? m_lo : m_hi;
        const float a = d * ubyte(scw, i & 3);
        s.a[i] = (i & 1) ? a * 0.0625f : a; /* odd sub-blocks use 16*q codes */
        s.m[i] = dmin * ubyte(mw, i & 3);
    }
    return s;
}

template <bool kGuard>
__device__ __forceinline__ float q4k_m1(const Q4KUnit &u, const float *__restrict__ xu, int lane, int kleft)
{
    float xs = unit_x_partial<256, kGuard>(xu, lane, kleft);
    xs = xor_sum(xs, 1); xs = xor_sum(xs, 2); xs = xor_sum(xs, 4); /* 8 lanes = 32 x */
    /* Region p = plane 1+p: x runs [k0, k0+16) (low) and [k0+32, k0+48) (high). */
    float xr[2][32];
    auto load = [&](float (&dst)[32], int p, float ds, float v0, float v1) {
        const int k0 = 64 * (p >> 1) + 16 * (p & 1);
        gfloat *a = region_ptr(xu + k0, ds, v0, v1);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            dst[i] = a[i];
            dst[16 + i] = a[32 + i];
        }
    };
    float slo[4] = {0.0f, 0.0f, 0.0f, 0.0f}, shi[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    load(xr[0], 0, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int p = 0; p < 8; ++p) {
        const int g = p >> 1;
        if (p < 7) {
            const int gp = p > 0 ? (p - 1) >> 1 : 0;
            load(xr[(p + 1) & 1], p + 1, xr[p & 1][0], slo[gp], shi[gp]);
        }
        const float(&x)[32] = xr[p & 1];
        float l0 = 0.0f, l1 = 0.0f, h0 = 0.0f, h1 = 0.0f;
#pragma unroll
        for (int e = 0; e < 4; ++e)
            q4_dword_mix(word(u.p[1 + p], e), x + 4 * e, (e & 1) ? l1 : l0, (e & 1) ? h1 : h0);
        slo[g] += l0 + l1;
        shi[g] += h0 + h1;
    }
    /* slo / shi hold sums scaled by 2^-24 (q4_dword_mix): the scales carry
     * 2^24 (low codes q) and 2^24 / 16 (high codes 16q), exact powers of 2. */
    const Q4KScales s = q4k_scales(u.p[0]);
    float acc = 0.0f;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        acc = fmaf(s.a[2 * g] * 16777216.0f, slo[g], acc);
        acc = fmaf(s.a[2 * g + 1] * 16777216.0f, shi[g], acc);
        acc = fmaf(-s.m[2 * g], lane_value(xs, 16 * g), acc);
        acc = fmaf(-s.m[2 * g + 1], lane_value(xs, 16 * g + 8), acc);
    }
    return acc;
}

/* Region r of 8 exactly decoded Q4_K weights: (g, h, e) = (r >> 3, r >> 2 & 1,
 * r & 3); i < 4 low nibbles, i >= 4 high nibbles of dword e of plane 1+2g+h. */
__device__ __forceinline__ int q4k_k(int r, int i)
{
    const int g = r >> 3, h = (r >> 2) & 1, e = r & 3;
    return 64 * g + 16 * h + 4 * e + (i & 3) + (i >= 4 ? 32 : 0);
}

__device__ __forceinline__ void q4k_w(const Q4KUnit &u, const Q4KScales &s, int r, float (&w)[8], float dep)
{
    const int g = r >> 3, h = (r >> 2) & 1, e = r & 3;
    const uint32_t dw = after(word(u.p[1 + 2 * g + h], e), dep);
    const uint32_t lo = codes(dw & 0x0f0f0f0fu), hi = codes(dw & 0xf0f0f0f0u);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        /* a*q is exact, so the fused form rounds exactly like a*q - m. */
        w[c] = fmaf(s.a[2 * g], ubyte(lo, c), -s.m[2 * g]);
        w[4 + c] = fmaf(s.a[2 * g + 1], ubyte(hi, c), -s.m[2 * g + 1]);
    }
}

/* Q6_K: weight n = 128g + 32r + o, low nibble from ql[64g + 32(r&1) + o]
 * (>> 4 for r >= 2), two high bits from qh[32g + o] >> 2r, code q = low |
 * high << 4 in 0..63, value (q - 32) * d * scales[n / 16]. For (g, half oh =
 * o / 16) the planes are ql 4g+oh (r = 0, 2), ql 4g+2+oh (r = 1, 3) and qh
 * 8+2g+oh; dword e covers o = 16oh + 4e .. +3. */
__device__ __forceinline__ void q6k_codes(uint32_t qa, uint32_t qb, uint32_t qh, uint32_t (&q)[4])
{
    q[0] = codes((qa & 0x0f0f0f0fu) | ((qh << 4) & 0x30303030u));
    q[1] = codes((qb & 0x0f0f0f0fu) | ((qh << 2) & 0x30303030u));
    q[2] = codes(((qa >> 4) & 0x0f0f0f0fu) | (qh & 0x30303030u));
    q[3] = codes(((qb >> 4) & 0x0f0f0f0fu) | ((qh >> 2) & 0x30303030u));
}

__device__ __forceinline__ void q6k_dscales(const Q6KUnit &u, float (&dsc)[16])
{
    const float d = f16_bits_to_f32(u.d);
#pragma unroll
    for (int j = 0; j < 16; ++j) dsc[j] = d * sbyte(word(u.p[12], j >> 2), j & 3);
}

template <bool kGuard>
__device__ __forceinline__ float q6k_m1(const Q6KUnit &u, const float *__restrict__ xu, int lane, int kleft)
{
    float xs = unit_x_partial<256, kGuard>(xu, lane, kleft);
    xs = xor_sum(xs, 1); xs = xor_sum(xs, 2); /* 4 lanes = 16 x = one scale group */
    /* Region p = (g, oh, rp): codes r = 2rp and 2rp+1 of dwords e = 0..3, i.e.
     * x runs [k0, k0+16) and [k0+32, k0+48) with k0 = 128g + 64rp + 16oh. */
    float xr[2][32];
    auto load = [&](float (&dst)[32], int p, float ds, float v0, float v1) {
        const int g = p >> 2, oh = (p >> 1) & 1, rp = p & 1;
        const int k0 = 128 * g + 64 * rp + 16 * oh;
        gfloat *a = region_ptr(xu + k0, ds, v0, v1);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            dst[i] = a[i];
            dst[16 + i] = a[32 + i];
        }
    };
    float sg[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) sg[j] = 0.0f;
    load(xr[0], 0, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int p = 0; p < 8; ++p) {
        const int g = p >> 2, oh = (p >> 1) & 1, rp = p & 1;
        if (p < 7) {
            const int pp = p > 0 ? p - 1 : 0; /* region p-1's two scale groups */
            const int jp = 8 * (pp >> 2) + 4 * (pp & 1) + ((pp >> 1) & 1);
            load(xr[(p + 1) & 1], p + 1, xr[p & 1][0], sg[jp], sg[jp + 2]);
        }
        const float(&x)[32] = xr[p & 1];
        float c00 = 0.0f, c01 = 0.0f, c10 = 0.0f, c11 = 0.0f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t qh = word(u.p[8 + 2 * g + oh], e);
            uint32_t q0, q1;
            if (rp == 0) {
                q0 = (word(u.p[4 * g + oh], e) & 0x0f0f0f0fu) | ((qh << 4) & 0x30303030u);
                q1 = (word(u.p[4 * g + 2 + oh], e) & 0x0f0f0f0fu) | ((qh << 2) & 0x30303030u);
            } else {
                q0 = ((word(u.p[4 * g + oh], e) >> 4) & 0x0f0f0f0fu) | (qh & 0x30303030u);
                q1 = ((word(u.p[4 * g + 2 + oh], e) >> 4) & 0x0f0f0f0fu) | ((qh >> 2) & 0x30303030u);
            }
            q0 = codes(q0);
            q1 = codes(q1);
            float &a0 = (e & 1) ? c01 : c00;
            float &a1 = (e & 1) ? c11 : c10;
            a0 = byte_codes_mix(q0, x + 4 * e, a0);
            a1 = byte_codes_mix(q1, x + 16 + 4 * e, a1);
        }
        const int j0 = 8 * g + 4 * rp + oh; /* r = 2rp: j = 8g + 2r + oh */
        sg[j0] += c00 + c01;
        sg[j0 + 2] += c10 + c11;
    }
    /* sg holds sums of q * x scaled by 2^-24 (byte_codes_mix); the offset
     * term 32 * sum(x) is scaled to match, exactly. */
    float dsc[16];
    q6k_dscales(u, dsc);
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) /* scale group j covers x[16j .. 16j+15] */
        acc = fmaf(dsc[j] * 16777216.0f, fmaf(-1.9073486328125e-6f, lane_value(xs, 4 * j), sg[j]), acc);
    return acc;
}

/* Region r of 8 Q6_K weights: (g, oh, e, rp) with codes r' = 2rp, 2rp+1. */
__device__ __forceinline__ int q6k_k(int r, int i)
{
    const int rp = r & 1, e = (r >> 1) & 3, oh = (r >> 3) & 1, g = r >> 4;
    const int rr = 2 * rp + (i >> 2);
    return 128 * g + 32 * rr + 16 * oh + 4 * e + (i & 3);
}

/* kSignedZeros: also reproduce the reference's sign of zero weights, (d*sc)*0
 * keeps the sign of d*sc (the dequant kernel); the fused form below returns
 * +0 there, which no sum can tell apart (the matvec paths). */
template <bool kSignedZeros>
__device__ __forceinline__ void q6k_w(const Q6KUnit &u, const float (&dsc)[16], int r, float (&w)[8], float dep)
{
    const int rp = r & 1, e = (r >> 1) & 3, oh = (r >> 3) & 1, g = r >> 4;
    uint32_t q[4];
    q6k_codes(after(word(u.p[4 * g + oh], e), dep), after(word(u.p[4 * g + 2 + oh], e), dep),
              after(word(u.p[8 + 2 * g + oh], e), dep), q);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int rr = 2 * rp + (i >> 2);
        const float ds = dsc[8 * g + 2 * rr + oh];
        /* ds*q and 32*ds are exact, so this is ds*(q-32) exactly. */
        if (kSignedZeros) w[i] = ds * (ubyte(q[rr], i & 3) - 32.0f);
        else w[i] = fmaf(ds, ubyte(q[rr], i & 3), -32.0f * ds);
    }
}

/* Q8_0 unit = 4 blocks; signed codes are read as (q ^ 0x80) = q + 128. */
__device__ __forceinline__ float q80_d(const Q80Unit &u, int j)
{
    return f16_bits_to_f32(word(u.d, j >> 1) >> (16 * (j & 1)));
}

template <bool kGuard>
__device__ __forceinline__ float q80_m1(const Q80Unit &u, const float *__restrict__ xu, int lane, int kleft)
{
    float xs = unit_x_partial<128, kGuard>(xu, lane, kleft);
    xs = xor_sum(xs, 1); xs = xor_sum(xs, 2); xs = xor_sum(xs, 4); xs = xor_sum(xs, 8); /* 16 lanes = 32 x */
    float xr[2][32];
    auto load = [&](float (&dst)[32], int j, float ds, float v0, float v1) {
        gfloat *a = region_ptr(xu + 32 * j, ds, v0, v1);
#pragma unroll
        for (int i = 0; i < 32; ++i) dst[i] = a[i];
    };
    /* K is a multiple of 32, so a partial last unit just lacks whole blocks. */
    const int jvalid = kGuard ? kleft / 32 : 4;
    float sj[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    load(xr[0], 0, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        if (j < jvalid) { /* uniform; false only past K in a partial unit */
            if (j + 1 < jvalid) load(xr[(j + 1) & 1], j + 1, xr[j & 1][0], sj[j > 0 ? j - 1 : 0], 0.0f);
            const float(&x)[32] = xr[j & 1];
            float c[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t dw = codes(word(u.qs[2 * j + h], e) ^ 0x80808080u);
#pragma unroll
                    for (int cc = 0; cc < 4; ++cc)
                        c[2 * h + (e & 1)] = fmaf(ubyte(dw, cc), x[16 * h + 4 * e + cc], c[2 * h + (e & 1)]);
                }
            sj[j] = (c[0] + c[1]) + (c[2] + c[3]);
        }
    }
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) acc = fmaf(q80_d(u, j), fmaf(-128.0f, lane_value(xs, 16 * j), sj[j]), acc);
    return acc;
}

/* Region r of 8 Q8_0 weights: (j, h, ep) = (r >> 2, r >> 1 & 1, r & 1). */
__device__ __forceinline__ int q80_k(int r, int i) { return 8 * r + i; }

template <bool kSignedZeros>
__device__ __forceinline__ void q80_w(const Q80Unit &u, const float (&d)[4], int r, float (&w)[8], float dep)
{
    const int j = r >> 2, h = (r >> 1) & 1, ep = r & 1;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t dw = codes(after(word(u.qs[2 * j + h], 2 * ep + (i >> 2)), dep) ^ 0x80808080u);
        if (kSignedZeros) w[i] = d[j] * (ubyte(dw, i & 3) - 128.0f);
        else w[i] = fmaf(d[j], ubyte(dw, i & 3), -128.0f * d[j]); /* d*(q+128) - 128d == d*q */
    }
}

/* Q5_0 unit = 4 blocks. Block j: qs plane j (byte i: low nibble = weight i,
 * high = weight i + 16), qh word j (bit i = fifth bit of weight i). Code q =
 * nib | bit << 4 in 0..31, value d * (q - 16). */
__device__ __forceinline__ void q50_codes(uint32_t dw, uint32_t qh, int e, uint32_t &lo, uint32_t &hi)
{
    lo = codes((dw & 0x0f0f0f0fu) | spread_bits4((qh >> (4 * e)) & 15u));
    hi = codes(((dw >> 4) & 0x0f0f0f0fu) | spread_bits4((qh >> (16 + 4 * e)) & 15u));
}

__device__ __forceinline__ float q50_d(const Q50Unit &u, int j)
{
    return f16_bits_to_f32(word(u.d, j >> 1) >> (16 * (j & 1)));
}

template <bool kGuard>
__device__ __forceinline__ float q50_m1(const Q50Unit &u, const float *__restrict__ xu, int lane, int kleft)
{
    float xs = unit_x_partial<128, kGuard>(xu, lane, kleft);
    xs = xor_sum(xs, 1); xs = xor_sum(xs, 2); xs = xor_sum(xs, 4); xs = xor_sum(xs, 8);
    float xr[2][32];
    auto load = [&](float (&dst)[32], int j, float ds, float v0, float v1) {
        gfloat *a = region_ptr(xu + 32 * j, ds, v0, v1);
#pragma unroll
        for (int i = 0; i < 32; ++i) dst[i] = a[i];
    };
    /* K is a multiple of 32, so a partial last unit just lacks whole blocks. */
    const int jvalid = kGuard ? kleft / 32 : 4;
    float sj[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    load(xr[0], 0, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        if (j < jvalid) { /* uniform; false only past K in a partial unit */
            if (j + 1 < jvalid) load(xr[(j + 1) & 1], j + 1, xr[j & 1][0], sj[j > 0 ? j - 1 : 0], 0.0f);
            const float(&x)[32] = xr[j & 1];
            const uint32_t qh = word(u.qh, j);
            float c[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                uint32_t lo, hi;
                q50_codes(word(u.qs[j], e), qh, e, lo, hi);
#pragma unroll
                for (int cc = 0; cc < 4; ++cc) {
                    c[e & 1] = fmaf(ubyte(lo, cc), x[4 * e + cc], c[e & 1]);
                    c[2 + (e & 1)] = fmaf(ubyte(hi, cc), x[16 + 4 * e + cc], c[2 + (e & 1)]);
                }
            }
            sj[j] = (c[0] + c[1]) + (c[2] + c[3]);
        }
    }
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) acc = fmaf(q50_d(u, j), fmaf(-16.0f, lane_value(xs, 16 * j), sj[j]), acc);
    return acc;
}

/* Region r of 8 Q5_0 weights: (j, e) = (r >> 2, r & 3); i < 4 low, i >= 4 high. */
__device__ __forceinline__ int q50_k(int r, int i)
{
    const int j = r >> 2, e = r & 3;
    return 32 * j + 4 * e + (i & 3) + (i >= 4 ? 16 : 0);
}

template <bool kSignedZeros>
__device__ __forceinline__ void q50_w(const Q50Unit &u, const float (&d)[4], int r, float (&w)[8], float dep)
{
    const int j = r >> 2, e = r & 3;
    uint32_t lo, hi;
    q50_codes(after(word(u.qs[j], e), dep), word(u.qh, j), e, lo, hi);
#pragma unroll
    for (int c = 0; c < 4; ++c) { /* d*q and 16d are exact: d*(q-16) */
        if (kSignedZeros) {
            w[c] = d[j] * (ubyte(lo, c) - 16.0f);
            w[4 + c] = d[j] * (ubyte(hi, c) - 16.0f);
        } else {
            w[c] = fmaf(d[j], ubyte(lo, c), -16.0f * d[j]);
            w[4 + c] = fmaf(d[j], ubyte(hi, c), -16.0f * d[j]);
        }
    }
}

/* ---- format dispatch ------------------------------------------------------ */

/* Per-unit decoded scales used by the exact (M >= 2 and dequant) paths. */
template <int FMT> struct UnitScales;
template <> struct UnitScales<QMV_FMT_Q4_K> { Q4KScales s; };
template <> struct UnitScales<QMV_FMT_Q6_K> { float dsc[16]; };
template <> struct UnitScales<QMV_FMT_Q8_0> { float d[4]; };
template <> struct UnitScales<QMV_FMT_Q5_0> { float d[4]; };

template <int FMT>
__device__ __forceinline__ UnitScales<FMT> unit_scales(const typename UnitOf<FMT>::T &u)
{
    UnitScales<FMT> r;
    if constexpr (FMT == QMV_FMT_Q4_K) r.s = q4k_scales(u.p[0]);
    else if constexpr (FMT == QMV_FMT_Q6_K) q6k_dscales(u, r.dsc);
    else if constexpr (FMT == QMV_FMT_Q8_0) { for (int j = 0; j < 4; ++j) r.d[j] = q80_d(u, j); }
    else { for (int j = 0; j < 4; ++j) r.d[j] = q50_d(u, j); }
    return r;
}

template <int FMT> struct RegionCount { static constexpr int value = UnitOf<FMT>::kWeights / 8; };

template <int FMT>
__device__ __forceinline__ int region_k(int r, int i)
{
    if constexpr (FMT == QMV_FMT_Q4_K) return q4k_k(r, i);
    else if constexpr (FMT == QMV_FMT_Q6_K) return q6k_k(r, i);
    else if constexpr (FMT == QMV_FMT_Q8_0) return q80_k(r, i);
    else return q50_k(r, i);
}

/* Q4_K's fused decode already rounds (and signs zeros) exactly like the
 * reference, so only the other formats distinguish kSignedZeros. */
template <int FMT, bool kSignedZeros = false>
__device__ __forceinline__ void region_w(const typename UnitOf<FMT>::T &u, const UnitScales<FMT> &s, int r,
                                         float (&w)[8], float dep)
{
    if constexpr (FMT == QMV_FMT_Q4_K) q4k_w(u, s.s, r, w, dep);
    else if constexpr (FMT == QMV_FMT_Q6_K) q6k_w<kSignedZeros>(u, s.dsc, r, w, dep);
    else if constexpr (FMT == QMV_FMT_Q8_0) q80_w<kSignedZeros>(u, s.d, r, w, dep);
    else q50_w<kSignedZeros>(u, s.d, r, w, dep);
}

template <int FMT, bool kGuard>
__device__ __forceinline__ float unit_m1(const typename UnitOf<FMT>::T &u, const float *xu, int lane, int kleft)
{
    if constexpr (FMT == QMV_FMT_Q4_K) return q4k_m1<kGuard>(u, xu, lane, kleft);
    else if constexpr (FMT == QMV_FMT_Q6_K) return q6k_m1<kGuard>(u, xu, lane, kleft);
    else if constexpr (FMT == QMV_FMT_Q8_0) return q80_m1<kGuard>(u, xu, lane, kleft);
    else return q50_m1<kGuard>(u, xu, lane, kleft);
}

/* Exact weights for all M positions, in 8-weight regions whose activations
 * are two runs of 4 consecutive k per position. For small M the next
 * region's activations load while this region computes (2 x 8M SGPRs);
 * beyond that each region loads after the previous one finished. */
template <int FMT, int M, bool kGuard>
__device__ __forceinline__ void unit_mn(const typename UnitOf<FMT>::T &u, const float *__restrict__ xu, int ldx,
                                        int kleft, float (&acc)[M], int rb, int re)
{
    constexpr int R = RegionCount<FMT>::value;
    constexpr bool kAhead = M <= 4;
    const UnitScales<FMT> s = unit_scales<FMT>(u);
    float xr[2][8 * M];
    auto load = [&](float (&dst)[8 * M], int r, float ds, float v0, float v1) {
        const int k0 = region_k<FMT>(r, 0), k1 = region_k<FMT>(r, 4);
#pragma unroll
        for (int m = 0; m < M; ++m) {
            gfloat *a = region_ptr(xu + (size_t)m * ldx + k0, ds, v0, v1);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                dst[8 * m + i] = a[region_k<FMT>(r, i) - k0];
                dst[8 * m + 4 + i] = a[region_k<FMT>(r, 4 + i) - k0];
            }
        }
    };
    /* Regions are ordered by block (4 per 32-weight block for Q8_0/Q5_0); a
     * partial last unit lacks whole blocks, since K is a multiple of 32.
     * Only regions [rb, re) run (half a unit: rb = 0 or R / 2, so rb is even
     * and region rb's activations go to xr[0]). */
    const int rvalid = min(kGuard ? (kleft / 32) * 4 : R, re);
    if (kAhead) load(xr[0], rb, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int r = 0; r < R; ++r) {
        if (r >= rb && r < rvalid) { /* uniform */
            const float prev = all_of(acc); /* every FMA of region r-1 is done */
            if (kAhead) {
                if (r + 1 < rvalid) load(xr[(r + 1) & 1], r + 1, xr[r & 1][0], prev, prev);
            } else {
                load(xr[r & 1], r, 0.0f, prev, prev);
            }
            float w[8];
            region_w<FMT>(u, s, r, w, prev);
            const float(&x)[8 * M] = xr[r & 1];
#pragma unroll
            for (int m = 0; m < M; ++m)
#pragma unroll
                for (int i = 0; i < 8; ++i) acc[m] = fmaf(w[i], x[8 * m + i], acc[m]);
        }
    }
}

template <int FMT, int M>
__device__ __forceinline__ void unit_step(const typename UnitOf<FMT>::T &u, const float *__restrict__ x, int ldx,
                                          int cols, int unit, int lane, float (&acc)[M], int rb = 0,
                                          int re = RegionCount<FMT>::value)
{
    constexpr int UW = UnitOf<FMT>::kWeights;
    const int k0 = unit * UW;
    const int kleft = cols - k0;
    const float *xu = x + k0;
    if (UW == 256 || kleft >= UW) {
        if constexpr (M == 1) acc[0] += unit_m1<FMT, false>(u, xu, lane, kleft);
        else unit_mn<FMT, M, false>(u, xu, ldx, kleft, acc, rb, re);
    } else {
        if constexpr (M == 1) acc[0] += unit_m1<FMT, true>(u, xu, lane, kleft);
        else unit_mn<FMT, M, true>(u, xu, ldx, kleft, acc, rb, re);
    }
}

/* Coherent (agent-scope) loads and stores of published partials. */
__device__ __forceinline__ float load_partial(const float *p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_partial(float *p, float v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* Sums of the n partials of M elements: sum[m] = part[m * 64] + part[stride +
 * m * 64] + ... + part[(n - 1) * stride + m * 64] (this lane's elements),
 * each added in split order. The loads of a batch of splits for all M
 * elements go out before any is waited for (about LOADS in flight: 16 keeps
 * the VALU kernels' registers, 64 fits the matrix-core kernel's), so the sums
 * cost ceil(n / batch) memory round trips rather than M times that. */
template <int M, int LOADS, bool kBatch = (M >= 2)>
__device__ __forceinline__ void sum_partials(const float *part, size_t stride, int n, float (&sum)[M])
{
    constexpr int B = LOADS / M > 1 ? LOADS / M : 1;
    /* For batches the loads carry no branch. With room for a pointer per
     * split (LOADS >= 64), splits past n repeat the last one; otherwise they
     * read on from one base pointer, up to B * stride <= QMV_PARTIAL_PAD
     * floats past the tile's partials, which the workspace provides. Neither
     * is added. At one position (kBatch false: M == 1, and the gate and up
     * sums of the paired SwiGLU finish; splits rarely past 4) a condition
     * per load keeps the memory traffic to the partials that exist. */
    constexpr bool kClamp = LOADS >= 64;
    constexpr bool kOverread = !kClamp && kBatch;
    static_assert(!kOverread || B * M * 64 <= QMV_PARTIAL_PAD, "overread within the workspace padding");
    for (int b = 0; b < n; b += B) {
        float v[B][M];
#pragma unroll
        for (int i = 0; i < B; ++i) {
            if constexpr (kClamp) {
                const float *pi = part + (size_t)min(b + i, n - 1) * stride;
#pragma unroll
                for (int m = 0; m < M; ++m) v[i][m] = load_partial(pi + m * 64);
            } else if constexpr (kOverread) {
#pragma unroll
                for (int m = 0; m < M; ++m) v[i][m] = load_partial(part + (size_t)(b + i) * stride + m * 64);
            } else {
#pragma unroll
                for (int m = 0; m < M; ++m)
                    v[i][m] = b + i < n ? load_partial(part + (size_t)(b + i) * stride + m * 64) : 0.0f;
            }
        }
#pragma unroll
        for (int i = 0; i < B; ++i)
            if (b + i < n)
#pragma unroll
                for (int m = 0; m < M; ++m) sum[m] = b + i == 0 ? v[i][m] : sum[m] + v[i][m];
    }
}

/* ---- matvec kernel ---------------------------------------------------------
 * Workgroup = one 64-row tile x one K-split; its waves take consecutive
 * K-units and combine through LDS in wave order. A tile whose K is split
 * across workgroups is finished by the last split to arrive, which adds the
 * published partials in split order. */

/* Minimum resident waves per SIMD the matvec kernels are compiled for (caps
 * VGPRs at 512 / n; 1 leaves register allocation to the compiler);
 * QMV_WAVES_PER_SIMD_M1 / _MN are build-time knobs. */
#ifndef QMV_WAVES_PER_SIMD_M1
#define QMV_WAVES_PER_SIMD_M1 1
#endif
#ifndef QMV_WAVES_PER_SIMD_MN
#define QMV_WAVES_PER_SIMD_MN 1
#endif
template <int FMT, int M> struct MatvecOccupancy {
    static constexpr int value = M == 1 ? QMV_WAVES_PER_SIMD_M1 : QMV_WAVES_PER_SIMD_MN;
};

/* Greedy-argmax merge (src/sampler.cpp:29-51 semantics): the larger value
 * wins, the lower index on equal values, so any merge order gives the same
 * winner. */
__device__ __forceinline__ void argmax_merge(float &v, int &i, float v2, int i2)
{
    if (v2 > v || (v2 == v && i2 < i)) { v = v2; i = i2; }
}

/* Wave-wide argmax of (v, i, bad): every lane ends with the result. */
__device__ __forceinline__ void wave_argmax(float &v, int &i, int &bad)
{
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const float v2 = __shfl_xor(v, o);
        const int i2 = __shfl_xor(i, o);
        bad |= __shfl_xor(bad, o);
        argmax_merge(v, i, v2, i2);
    }
}

/* A tile's argmax candidate as one 64-bit word: value bits, and below the
 * top bit of the high word the row index, with the top bit set if any row of
 * the tile was not finite. */
__device__ __forceinline__ uint64_t pack_candidate(float v, int i, int bad)
{
    return (uint64_t)__float_as_uint(v) | ((uint64_t)((uint32_t)i & 0x7fffffffu | (bad ? 0x80000000u : 0u)) << 32);
}

/* Fused greedy argmax over a single-tensor M = 1 launch, in two levels so
 * that no counter sees more than QMV_ARGMAX_GROUP arrivals (arrivals at one
 * address serialise in the memory-side atomic unit): the wave that holds a
 * tile's final logits reduces them to a candidate, publishes it and counts
 * it in its group of tiles; the last tile of a group reduces the group's
 * candidates and counts the group; the last group reduces the group
 * candidates and writes result[0] = token (or -1) and result[1] = 1 if every
 * logit was finite. Candidates and counts use agent-scope atomics; each last
 * arriver resets its counter. */
#define QMV_ARGMAX_GROUP 64

/* Reduce candidates cand[first .. first + n) (n <= 64), one per lane. */
__device__ __forceinline__ void reduce_candidates(const uint64_t *cand, int first, int n, int lane, float &v, int &i,
                                                  int &bad)
{
    v = -INFINITY;
    i = 0x7fffffff;
    bad = 0;
    if (lane < n) {
        const uint64_t c = __hip_atomic_load(cand + first + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint32_t hi = (uint32_t)(c >> 32);
        bad = (int)(hi >> 31);
        v = __uint_as_float((uint32_t)c);
        i = (int)(hi & 0x7fffffffu);
    }
    wave_argmax(v, i, bad);
}

/* Publish a candidate and count it; true for the last of `expected`. */
__device__ __forceinline__ bool publish_and_count(uint64_t *slot, uint64_t c, unsigned *count, int expected, int lane)
{
    if (lane == 0) __hip_atomic_store(slot, c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    unsigned prev = 0;
    if (lane == 0) prev = __hip_atomic_fetch_add(count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    prev = __builtin_amdgcn_readfirstlane(__builtin_amdgcn_readlane(prev, 0));
    if (prev != (unsigned)expected - 1u) return false;
    if (lane == 0) __hip_atomic_store(count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    asm volatile("" ::: "memory");
    return true;
}

/* Workspace: argmax_cand[tiles + groups] (tile candidates, then group
 * candidates), argmax_count[groups + 1] (group counts, then the top count). */
template <typename P>
__device__ __forceinline__ void publish_tile_candidate(const P &p, int tile, float v, int i, int bad, int lane);

/* This lane's row as an argmax candidate (value, index, non-finite flag),
 * reduced over the wave: every lane ends with the wave's candidate. */
__device__ __forceinline__ void wave_candidate(bool valid, int row, float y, float &v, int &i, int &bad)
{
    const bool fin = isfinite(y);
    v = valid && fin ? y : -INFINITY;
    i = valid && fin ? row : 0x7fffffff;
    bad = valid && !fin;
    wave_argmax(v, i, bad);
}

template <typename P>
__device__ __forceinline__ void tile_argmax(const P &p, int tile, bool valid, int row, float y, int lane)
{
    float v;
    int i, bad;
    wave_candidate(valid, row, y, v, i, bad);
    publish_tile_candidate(p, tile, v, i, bad, lane);
}

/* Publish a tile's candidate (identical in every lane of the calling wave)
 * and run the group and top levels if this wave arrives last. */
template <typename P>
__device__ __forceinline__ void publish_tile_candidate(const P &p, int tile, float v, int i, int bad, int lane)
{
    const int tiles = p.argmax_tiles;
    const int groups = (tiles + QMV_ARGMAX_GROUP - 1) / QMV_ARGMAX_GROUP;
    const int g = tile / QMV_ARGMAX_GROUP;
    const int first = g * QMV_ARGMAX_GROUP;
    const int in_group = min(QMV_ARGMAX_GROUP, tiles - first);
    if (!publish_and_count(p.argmax_cand + tile, pack_candidate(v, i, bad), p.argmax_count + g, in_group, lane))
        return;
    reduce_candidates(p.argmax_cand, first, in_group, lane, v, i, bad);
    if (!publish_and_count(p.argmax_cand + tiles + g, pack_candidate(v, i, bad), p.argmax_count + groups, groups,
                           lane))
        return;
    float bv = -INFINITY;
    int bi = 0x7fffffff, bb = 0;
    for (int f = 0; f < groups; f += 64) {
        reduce_candidates(p.argmax_cand + tiles, f, min(64, groups - f), lane, v, i, bad);
        bb |= bad;
        argmax_merge(bv, bi, v, i);
    }
    if (lane == 0) {
        p.argmax_result[0] = bb || bi == 0x7fffffff ? -1 : bi;
        p.argmax_result[1] = bb ? 0 : 1;
    }
}

/* Index of the job that owns this workgroup (jobs own consecutive ranges of
 * workgroups from their wg_begin), walking the jobs: the prefill kernel's
 * choice. The single-position and matrix-core kernels read every job's start
 * in one batch of scalar loads instead (launch_args), and so does the
 * row-major kernel: each dependent kernel-argument load before the first
 * weight load is a scalar-cache round trip on every wave's critical path
 * (measured on the Qwen2.5-7B set: q|k|v 4.72 -> 4.60 us, o 3.95 -> 3.83,
 * gate|up 16.1-16.9 -> 15.7, the fused SwiGLU 16.8-16.9 -> 15.8-16.1, the
 * M = 8 set 2.282 -> 2.253 ms; down, a single job, unchanged). */
template <typename P>
__device__ __forceinline__ int job_of_block(const P &p)
{
    int j = 0;
    while (j + 1 < p.njobs && (int)blockIdx.x >= p.job[j + 1].wg_begin) ++j;
    return j;
}

/* The workgroup's place in a launch: job, tile, K-split, and this wave's
 * K-units [u_begin, u_end). */
struct WgWork {
    int job, tile, split, u_begin, u_end;
};

/* Kernel arguments a tiled launch needs before its first weight load, read in
 * one batch of scalar loads: the launch-wide values, job 0's fields, and the
 * other jobs' first workgroups (unused job slots start past every workgroup,
 * set by the launchers). The job is the last one starting at or before this
 * workgroup; a job other than 0 then reads its own fields from lines this
 * batch brought into the scalar cache. */
struct LaunchArgs {
    const float *x;
    const uint8_t *w; /* the job's tiled weights */
    int ldx, cols, units, units_per_wave, parts, pair_waves;
    int job, splits, units_per_split, wg_begin;
};

__device__ __forceinline__ LaunchArgs launch_args(const MatvecParams &p)
{
    LaunchArgs a;
    a.x = p.x;
    a.ldx = p.ldx;
    a.cols = p.cols;
    a.units = p.units;
    a.units_per_wave = p.units_per_wave;
    a.parts = p.parts;
    a.pair_waves = p.pair_waves;
    a.w = p.job[0].w;
    a.splits = p.job[0].splits;
    a.units_per_split = p.job[0].units_per_split;
    int begin[QMV_MAX_JOBS];
#pragma unroll
    for (int i = 1; i < QMV_MAX_JOBS; ++i) begin[i] = p.job[i].wg_begin;
    __builtin_amdgcn_sched_barrier(0); /* the loads above go out together */
    /* Materialise the launch-wide values and job 0's fields here, so the
     * compiler neither sinks their loads to their first use nor merges job
     * 0's with the chosen job's into one load that waits for the choice.
     * The pointers pass as integers and come back as global-memory pointers,
     * so their loads stay global (not flat) loads. */
    uint64_t xi = (uint64_t)a.x, wi = (uint64_t)a.w;
    asm volatile("" : "+s"(xi), "+s"(wi));
    a.x = (const float *)(const __attribute__((address_space(1))) float *)xi;
    a.w = (const uint8_t *)(const __attribute__((address_space(1))) uint8_t *)wi;
    asm volatile("" : "+s"(a.ldx), "+s"(a.cols), "+s"(a.units), "+s"(a.units_per_wave));
    asm volatile("" : "+s"(a.parts), "+s"(a.pair_waves), "+s"(a.splits), "+s"(a.units_per_split));
    const int bid = (int)blockIdx.x;
    int j = 0;
#pragma unroll
    for (int i = 1; i < QMV_MAX_JOBS; ++i) j = bid >= begin[i] ? i : j;
    a.wg_begin = 0;
    if (a.pair_waves > 0) j = 0; /* paired SwiGLU: job 0's plan serves both halves */
    a.job = j;
    if (j != 0) {
        a.w = p.job[j].w;
        a.splits = p.job[j].splits;
        a.units_per_split = p.job[j].units_per_split;
        a.wg_begin = p.job[j].wg_begin;
    }
    return a;
}

__device__ __forceinline__ WgWork locate(const LaunchArgs &a, int wave, int items)
{
    WgWork w;
    if (a.pair_waves > 0) { /* paired SwiGLU (job 0 = gate, 1 = up, same plan): gate waves, then up waves */
        const int half = wave >= a.pair_waves ? 1 : 0;
        w.job = half;
        w.tile = blockIdx.x / a.splits;
        w.split = blockIdx.x - w.tile * a.splits;
        const int split_begin = w.split * a.units_per_split;
        const int split_end = min(split_begin + a.units_per_split, a.units);
        w.u_begin = split_begin + (wave - half * a.pair_waves) * a.units_per_wave;
        w.u_end = min(w.u_begin + a.units_per_wave, split_end);
        return w;
    }
    const int local = (int)blockIdx.x - a.wg_begin;
    w.job = a.job;
    w.tile = local / a.splits;
    w.split = local - w.tile * a.splits;
    const int split_begin = w.split * a.units_per_split;
    const int split_end = min(split_begin + a.units_per_split, items);
    w.u_begin = split_begin + wave * a.units_per_wave;
    w.u_end = min(w.u_begin + a.units_per_wave, split_end);
    return w;
}

/* silu(g) * u, as src/transformer_ops.cpp:163-176 computes each element
 * (x / (1 + exp(-x)), then the product with up). */
__device__ __forceinline__ float swiglu_value(float g, float u)
{
    return u * (g / (1.0f + expf(-g)));
}

/* Fused SwiGLU: publish this tile's final gate or up values and count the
 * tile; the second of the pair to arrive reads the other's values and writes
 * up * silu(gate) to job 0's output, then resets the count. */
template <int M>
__device__ __forceinline__ void swiglu_pair(const MatvecParams &p, const WgWork &w, int lane, int row, bool valid,
                                            int npos, const float (&v)[M])
{
    const MatvecJob &out = p.job[0];
    float *mine = p.pair_vals + ((size_t)w.job * out.tiles + w.tile) * M * 64 + lane;
#pragma unroll
    for (int m = 0; m < M; ++m) store_partial(mine + m * 64, v[m]);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    unsigned prev = 0;
    if (lane == 0) prev = __hip_atomic_fetch_add(p.pair_count + w.tile * QMV_COUNTER_STRIDE, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    prev = __builtin_amdgcn_readfirstlane(__builtin_amdgcn_readlane(prev, 0));
    if (prev == 0u) return;
    asm volatile("" ::: "memory");
    const float *other = p.pair_vals + ((size_t)(1 - w.job) * out.tiles + w.tile) * M * 64 + lane;
#pragma unroll
    for (int m = 0; m < M; ++m) {
        const float o = load_partial(other + m * 64);
        const float g = w.job == 0 ? v[m] : o;
        const float u = w.job == 0 ? o : v[m];
        if (valid && m < npos) out.y[(size_t)m * out.ldy + row] = swiglu_value(g, u);
    }
    if (lane == 0) __hip_atomic_store(p.pair_count + w.tile * QMV_COUNTER_STRIDE, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* A tile's final row values v[m] (lane = row within the tile): add the
 * job's addend, then store them, or hand them to the fused SwiGLU, and feed
 * the fused argmax. The addend is read and the output written by the same
 * lane, so an addend that is the output itself (a residual added in place)
 * is safe. */
template <int M>
__device__ __forceinline__ void emit_tile(const MatvecParams &p, const WgWork &w, int lane, int npos, float (&v)[M])
{
    const MatvecJob &job = p.job[w.job];
    const int row = w.tile * 64 + lane;
    const bool valid = row < job.rows;
    if (job.add != nullptr && valid) {
#pragma unroll
        for (int m = 0; m < M; ++m)
            if (m < npos) v[m] += job.add[(size_t)m * job.ldadd + row];
    }
    if (p.swiglu) {
        swiglu_pair<M>(p, w, lane, row, valid, npos, v);
        return;
    }
    if (valid) {
#pragma unroll
        for (int m = 0; m < M; ++m)
            if (m < npos) job.y[(size_t)m * job.ldy + row] = v[m];
    }
    if constexpr (M == 1)
        if (p.argmax_result) tile_argmax(p, w.tile, valid, row, v[0], lane);
}

/* After every wave has written red[wave][m][row] (row = tile row 0..63) and
 * the workgroup has synchronised, wave 0 adds the waves in wave order and
 * emits the rows, or, for a tile split along K, publishes this split's
 * partial; the last split to arrive adds all partials of the tile in split
 * order (a fixed order, so results do not depend on arrival order).
 * Partials and counters are accessed only with agent-scope atomics, which are
 * coherent across the XCDs' L2s without a cache writeback or invalidate: the
 * wait for the partial stores to complete orders them before the arrival
 * count. The last split resets the counter, so the workspace needs no
 * clearing between launches. */
/* Paired SwiGLU finish (M = 1): gate and up sums of the tile, each over its
 * waves in wave order and its splits in split order (the order of the two
 * separate launches), then up * silu(gate) into job 0's y. */
__device__ __forceinline__ void finish_paired(const MatvecParams &p, const WgWork &w, int lane,
                                              const float (*red)[1][64])
{
    const int W = p.pair_waves;
    float g = red[0][0][lane], u = red[W][0][lane];
    for (int v = 1; v < W; ++v) {
        g += red[v][0][lane];
        u += red[W + v][0][lane];
    }
    const MatvecJob &gj = p.job[0], &uj = p.job[1];
    const int S = gj.splits;
    if (S > 1) {
        float *part = p.partials + gj.partial_offset + (size_t)w.tile * S * 128 + lane;
        unsigned *count = p.counters + gj.counter_offset + w.tile * QMV_COUNTER_STRIDE;
        store_partial(part + (size_t)w.split * 128, g);
        store_partial(part + (size_t)w.split * 128 + 64, u);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        unsigned prev = 0;
        if (lane == 0) prev = __hip_atomic_fetch_add(count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        prev = __builtin_amdgcn_readfirstlane(__builtin_amdgcn_readlane(prev, 0));
        if (prev != (unsigned)S - 1u) return;
        asm volatile("" ::: "memory");
        float gu[2];
        sum_partials<2, 16, false>(part, 128, S, gu);
        g = gu[0];
        u = gu[1];
        if (lane == 0) __hip_atomic_store(count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    const int row = w.tile * 64 + lane;
    if (row < gj.rows) {
        if (gj.add != nullptr) g += gj.add[row];
        if (uj.add != nullptr) u += uj.add[row];
        gj.y[row] = swiglu_value(g, u);
    }
}

template <int M, int LOADS = 16>
__device__ __forceinline__ void finish_tile(const MatvecParams &p, const WgWork &w, int nwaves, int lane,
                                            const float (*red)[M][64], int npos = M)
{
    if constexpr (M == 1) {
        if (p.pair_waves > 0) {
            finish_paired(p, w, lane, red);
            return;
        }
    }
    const MatvecJob &job = p.job[w.job];
    float sum[M];
#pragma unroll
    for (int m = 0; m < M; ++m) {
        float s = red[0][m][lane];
        for (int v = 1; v < nwaves; ++v) s += red[v][m][lane];
        sum[m] = s;
    }

    if (job.splits > 1) {
        float *part = p.partials + job.partial_offset + ((size_t)w.tile * job.splits) * M * 64;
        unsigned *count = p.counters + job.counter_offset + w.tile * QMV_COUNTER_STRIDE;
#pragma unroll
        for (int m = 0; m < M; ++m) store_partial(part + ((size_t)w.split * M + m) * 64 + lane, sum[m]);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        unsigned prev = 0;
        if (lane == 0) prev = __hip_atomic_fetch_add(count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        prev = __builtin_amdgcn_readfirstlane(__builtin_amdgcn_readlane(prev, 0));
        if (prev != (unsigned)job.splits - 1u) return;
        asm volatile("" ::: "memory");
        sum_partials<M, LOADS>(part + lane, (size_t)M * 64, job.splits, sum);
        if (lane == 0) __hip_atomic_store(count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    /* One copy of the row epilogue serves both paths. */
    emit_tile<M>(p, w, lane, npos, sum);
}

/* kOne: every wave takes at most one unit (units_per_wave == 1), so no
 * second unit buffer is live and more waves fit per SIMD. */
template <int FMT, int M, bool kOne>
__global__ void __launch_bounds__(QMV_MAX_WAVES * 64)
__attribute__((amdgpu_waves_per_eu(MatvecOccupancy<FMT, M>::value)))
matvec_kernel(MatvecParams p)
{
    using Unit = typename UnitOf<FMT>::T;
    constexpr int SLAB = UnitOf<FMT>::kBytes * 64;
    __shared__ float red[QMV_MAX_WAVES][M][64];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    /* Batches may run half units (p.parts = 2, one work item per wave): a
     * tile then has 2 x units items, item i being half i & 1 of unit i / 2. */
    const LaunchArgs a = launch_args(p);
    const int shift = M >= 2 && kOne && a.parts == 2 ? 1 : 0;
    const WgWork w = locate(a, wave, a.units << shift);
    const uint8_t *wtile = (w.job == a.job ? a.w : p.job[w.job].w) + (size_t)w.tile * a.units * SLAB;
    float acc[M];
#pragma unroll
    for (int m = 0; m < M; ++m) acc[m] = 0.0f;

    if (kOne) {
        if (w.u_begin < w.u_end) {
            constexpr int R = RegionCount<FMT>::value;
            const int u = w.u_begin >> shift, span = R >> shift;
            const int rb = (w.u_begin - (u << shift)) * span;
            Unit q;
            load_unit(q, wtile + (size_t)u * SLAB, lane);
            unit_step<FMT, M>(q, a.x, a.ldx, a.cols, u, lane, acc, rb, rb + span);
        }
    } else if (w.u_begin < w.u_end) {
        /* Two units in flight per wave: the next unit's planes are loading
         * while the current one is decoded. */
        Unit qa, qb;
        load_unit(qa, wtile + (size_t)w.u_begin * SLAB, lane);
        for (int u = w.u_begin; u < w.u_end; u += 2) {
            const bool has_b = u + 1 < w.u_end;
            if (has_b) load_unit(qb, wtile + (size_t)(u + 1) * SLAB, lane);
            unit_step<FMT, M>(qa, a.x, a.ldx, a.cols, u, lane, acc);
            if (u + 2 < w.u_end) load_unit(qa, wtile + (size_t)(u + 2) * SLAB, lane);
            if (has_b) unit_step<FMT, M>(qb, a.x, a.ldx, a.cols, u + 1, lane, acc);
        }
    }

#pragma unroll
    for (int m = 0; m < M; ++m) red[wave][m][lane] = acc[m];
    __syncthreads();
    if (wave != 0) return;
    finish_tile<M>(p, w, blockDim.x >> 6, lane, red);
}

/* ---- M >= 2 on the matrix cores (Q4_K, Q6_K) ---------------------------------
 * Over one scale sub-block a row contributes a * sum(q * x) (- b * sum(x) for
 * Q4_K's minimum), with q the integer codes, exact in bf16. Each activation
 * is split into three bf16 limbs, x = h + m + l with h = bf16(x),
 * m = bf16(x - h), l = bf16(x - h - m): each difference is exact in fp32 and
 * l takes the remaining bits, so the limbs carry x exactly. bf16 MFMA
 * products are exact and accumulate in fp32, so sum(q * x) is an fp32 sum of
 * exact products, as on the VALU path, with the codes decoded once for up to
 * 8 positions.
 *
 * MFMA operand roles (lane l, kc = l / 16, n = l % 16): A = limbs, row i =
 * position (rows >= M repeat position 0 and are never stored), lane l
 * supplies A[n][kc*KL + j]; B = weight
 * codes, column = weight row 16g + n of row group g, lane l supplies
 * B[kc*KL + j][n]; D[i][n] lands in lane n + 16*(i/4), element i % 4. So a
 * lane's accumulator holds positions 4*kc..4*kc+3 of one weight row, and the
 * per-row scales it applies are that row's own. KL = 8 (16x16x32 MFMA, Q4_K
 * sub-blocks of 32) or 4 (16x16x16, Q6_K sub-blocks of 16). Per sub-block the
 * MFMAs of the four row groups are issued limb by limb, so four (five with
 * Q4_K's sum(x)) independent accumulations keep the matrix pipe busy. The
 * codes reach bf16 through the FP8 converter (q4_codes_bf16, q6_codes_bf16
 * below). */
typedef __bf16 bf16x8_t __attribute__((__vector_size__(8 * sizeof(__bf16))));
typedef __bf16 bf16x4_t __attribute__((__vector_size__(4 * sizeof(__bf16))));
typedef float f32x4_t __attribute__((__vector_size__(4 * sizeof(float))));

/* A per-lane pointer that cannot be used before `dep` exists: ties the
 * activation loads of a sub-block to the accumulators of an earlier one, so
 * the loads are not all hoisted to the top of the unrolled unit. */
/* Global-memory (address space 1) views. The ordering asm below hides a
 * pointer's origin, and a generic pointer would then load with flat
 * instructions, which also count against lgkmcnt (so scalar-load waits would
 * wait for them); through these types the loads stay global_load. */
typedef const float __attribute__((address_space(1))) gf32;
typedef const uint8_t __attribute__((address_space(1))) gu8;
typedef const uint32_t __attribute__((address_space(1))) gu32;
typedef const unsigned short __attribute__((address_space(1))) gu16;
typedef unsigned int u32v4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32v2 __attribute__((ext_vector_type(2)));
typedef const u32v4 __attribute__((address_space(1))) gv4;
typedef const u32v2 __attribute__((address_space(1))) gv2;

__device__ __forceinline__ uint4 gload16(gu8 *p)
{
    const u32v4 v = *(gv4 *)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 gload8(gu8 *p)
{
    const u32v2 v = *(gv2 *)p;
    return make_uint2(v.x, v.y);
}

__device__ __forceinline__ gf32 *ptr_after(const float *p, float dep)
{
    gf32 *g = (gf32 *)p;
    asm("" : "+v"(g) : "v"(dep));
    return g;
}

__device__ __forceinline__ gu8 *bytes_after(const uint8_t *p, float dep)
{
    gu8 *g = (gu8 *)p;
    asm("" : "+v"(g) : "v"(dep));
    return g;
}

template <int KL, typename P>
__device__ __forceinline__ void load_x(float (&v)[KL], P *p)
{
#pragma unroll
    for (int j = 0; j < KL; ++j) v[j] = p[j];
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

/* The three bf16 limbs of KL activations of one position (zero when the lane
 * carries no position), two activations at a time: one round-to-nearest-even
 * conversion per limb pair (v_cvt_pk_bf16_f32), and the pair's bf16 values
 * widened back to fp32 by a shift and a mask of the packed bits. */
template <int KL, typename V>
__device__ __forceinline__ void x_limbs(const float (&xv)[KL], bool valid, V &h, V &m, V &l)
{
    static_assert(KL % 2 == 0, "pairs of activations");
#pragma unroll
    for (int j = 0; j < KL; j += 2) {
        const float v0 = valid ? xv[j] : 0.0f, v1 = valid ? xv[j + 1] : 0.0f;
        const bf16x2_t hp = __builtin_convertvector(f32x2_t{v0, v1}, bf16x2_t);
        const uint32_t hb = __builtin_bit_cast(uint32_t, hp);
        const float r0 = v0 - __uint_as_float(hb << 16), r1 = v1 - __uint_as_float(hb & 0xffff0000u);
        const bf16x2_t mp = __builtin_convertvector(f32x2_t{r0, r1}, bf16x2_t);
        const uint32_t mb = __builtin_bit_cast(uint32_t, mp);
        const float s0 = r0 - __uint_as_float(mb << 16), s1 = r1 - __uint_as_float(mb & 0xffff0000u);
        const bf16x2_t lp = __builtin_convertvector(f32x2_t{s0, s1}, bf16x2_t);
        h[j] = hp[0];
        h[j + 1] = hp[1];
        m[j] = mp[0];
        m[j + 1] = mp[1];
        l[j] = lp[0];
        l[j + 1] = lp[1];
    }
}

/* Eight Q4_K codes, bytes 0..3 of lo then of hi (low nibbles, or the high
 * nibbles shifted down), as an exact bf16 MFMA operand. A code q in the low
 * bits of a byte is the FP8 E4M3 pattern of q * 2^-9 (subnormals for 0..7,
 * the first normal binade for 8..15), which v_cvt_scalef32_pk_bf16_fp8
 * converts with the scale 2^9 to bf16(q) exactly, two codes per
 * instruction. */
__device__ __forceinline__ bf16x8_t q4_codes_bf16(uint32_t lo, uint32_t hi, bool high)
{
    lo = (high ? lo >> 4 : lo) & 0x0f0f0f0fu;
    hi = (high ? hi >> 4 : hi) & 0x0f0f0f0fu;
    const bf16x2_t a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 512.0f, false);
    const bf16x2_t b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 512.0f, true);
    const bf16x2_t c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 512.0f, false);
    const bf16x2_t d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 512.0f, true);
    return bf16x8_t{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

/* Four Q6_K codes of one sub-block (4(r>>1)-shifted nibbles of the ql word
 * lw, 2r-shifted 2-bit fields of the qh word hw) as two exact bf16 operands
 * whose sum is q - 32: lo = the low nibble (FP8 E4M3 pattern of lo * 2^-9,
 * scale 2^9) and hi = 16 * (h - 2), from the sign-magnitude E4M3 patterns of
 * h - 2 = -2..1 picked by v_perm_b32 from the table 0x82, 0x81, 0x00, 0x01
 * (scale 2^13). The matrix core adds both products into one accumulator. */
__device__ __forceinline__ void q6_codes_bf16(uint32_t lw, uint32_t hw, int r, bf16x4_t &lo, bf16x4_t &hi)
{
    const uint32_t l = (lw >> (4 * (r >> 1))) & 0x0f0f0f0fu;
    const uint32_t h = __builtin_amdgcn_perm(0u, 0x01008182u, (hw >> (2 * r)) & 0x03030303u);
    const bf16x2_t l0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(l, 512.0f, false);
    const bf16x2_t l1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(l, 512.0f, true);
    const bf16x2_t h0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(h, 8192.0f, false);
    const bf16x2_t h1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(h, 8192.0f, true);
    lo = bf16x4_t{l0[0], l0[1], l1[0], l1[1]};
    hi = bf16x4_t{h0[0], h0[1], h1[0], h1[1]};
}

/* Sub-blocks [SB0, SB0 + NSB) of a Q4_K unit (SB0 even: whole 64-weight code
 * groups). */
template <int M, int SB0, int NSB>
__device__ __forceinline__ void q4k_unit_mfma(const uint8_t *slab, const float *xu, int ldx, int lane,
                                              f32x4_t (&acc)[4])
{
    static_assert(SB0 % 2 == 0 && NSB % 2 == 0 && SB0 + NSB <= 8, "whole code groups");
    constexpr int SB1 = SB0 + NSB;
    const int kc = lane >> 4, n = lane & 15;
    const bool valid = n < M;
    /* Lanes past the batch read position 0 (in bounds): their products land
     * in accumulator rows >= M, which the kernel never stores, so their
     * limbs need not be zeroed. */
    const float *xp = xu + (size_t)(valid ? n : 0) * ldx + 8 * kc;
    /* This lane's bytes of row 16g + n: header, and the 8 qs bytes of its
     * k-chunk in 64-weight group c (plane 1 + 2c + kc/2). */
    const uint8_t *rowp = slab + n * 16;
    const uint8_t *qsp = slab + (1 + (kc >> 1)) * 1024 + n * 16 + 8 * (kc & 1);
    uint4 h[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) h[g] = ld16(rowp + g * 256);
    uint2 q[2][4]; /* codes of group c and c + 1 */
#pragma unroll
    for (int g = 0; g < 4; ++g) q[(SB0 >> 1) & 1][g] = *(const uint2 *)(qsp + (SB0 >> 1) * 2048 + g * 256);
    const bf16x8_t ones = {(__bf16)1.0f, (__bf16)1.0f, (__bf16)1.0f, (__bf16)1.0f,
                           (__bf16)1.0f, (__bf16)1.0f, (__bf16)1.0f, (__bf16)1.0f};
    /* Activations run two sub-blocks ahead (a ring of three): one sub-block of
     * compute does not cover an L2 round trip. */
    float xv[3][8];
    load_x<8>(xv[SB0 % 3], (gf32 *)(xp + 32 * SB0));
    if (SB0 + 1 < SB1) load_x<8>(xv[(SB0 + 1) % 3], (gf32 *)(xp + 32 * (SB0 + 1)));
#pragma unroll
    for (int sb = SB0; sb < SB1; ++sb) {
        const int c = sb >> 1;
        const bool high = sb & 1;
        /* The activations of sub-block sb + 2, and at a group's start the
         * next group's codes, load while this sub-block runs. */
        if (sb + 2 < SB1) load_x<8>(xv[(sb + 2) % 3], ptr_after(xp + 32 * (sb + 2), acc[0][0]));
        if (!high && c + 1 < SB1 / 2) {
            gu8 *nq = bytes_after(qsp + (c + 1) * 2048, acc[1][0]);
#pragma unroll
            for (int g = 0; g < 4; ++g) q[(c + 1) & 1][g] = gload8(nq + g * 256);
        }
        bf16x8_t a0, a1, a2;
        x_limbs<8>(xv[sb % 3], true, a0, a1, a2);
        bf16x8_t b[4];
#pragma unroll
        for (int g = 0; g < 4; ++g)
            b[g] = q4_codes_bf16(q[c & 1][g].x, q[c & 1][g].y, high);
        f32x4_t xs = {0.0f, 0.0f, 0.0f, 0.0f}, d[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) d[g] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
        xs = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, ones, xs, 0, 0, 0);
#pragma unroll
        for (int g = 0; g < 4; ++g) d[g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, b[g], d[g], 0, 0, 0);
        xs = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, ones, xs, 0, 0, 0);
#pragma unroll
        for (int g = 0; g < 4; ++g) d[g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b[g], d[g], 0, 0, 0);
        xs = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2, ones, xs, 0, 0, 0);
#pragma unroll
        for (int g = 0; g < 4; ++g) d[g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2, b[g], d[g], 0, 0, 0);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const uint4 hg = h[g];
            const float dd = f16_bits_to_f32(hg.x), dmin = f16_bits_to_f32(hg.x >> 16);
            uint32_t scw, mw;
            if (sb < 4) {
                scw = hg.y & 0x3f3f3f3fu;
                mw = hg.z & 0x3f3f3f3fu;
            } else {
                scw = (hg.w & 0x0f0f0f0fu) | ((hg.y >> 2) & 0x30303030u);
                mw = ((hg.w >> 4) & 0x0f0f0f0fu) | ((hg.z >> 2) & 0x30303030u);
            }
            const float sa = dd * ubyte(scw, sb & 3);
            const float sm = dmin * ubyte(mw, sb & 3);
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[g][j] = fmaf(sa, d[g][j], fmaf(-sm, xs[j], acc[g][j]));
        }
        /* Scheduling stops here: the scale decode and code conversion of a
         * sub-block stay in it, so only one sub-block's scales are live
         * (without a copy of each header word per sub-block to order them). */
        __builtin_amdgcn_sched_barrier(0);
    }
}

/* Eight Q8_0 codes (the signed bytes of lo, then of hi) as one exact bf16
 * operand: each byte widens to fp32 with a sign-extending conversion, and
 * pairs round to bf16 exactly (|q| <= 128 needs at most 8 significant
 * bits). */
__device__ __forceinline__ bf16x8_t q8_codes_bf16(uint32_t lo, uint32_t hi)
{
    const bf16x2_t a = __builtin_convertvector(f32x2_t{sbyte(lo, 0), sbyte(lo, 1)}, bf16x2_t);
    const bf16x2_t b = __builtin_convertvector(f32x2_t{sbyte(lo, 2), sbyte(lo, 3)}, bf16x2_t);
    const bf16x2_t c = __builtin_convertvector(f32x2_t{sbyte(hi, 0), sbyte(hi, 1)}, bf16x2_t);
    const bf16x2_t d = __builtin_convertvector(f32x2_t{sbyte(hi, 2), sbyte(hi, 3)}, bf16x2_t);
    return bf16x8_t{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

/* Blocks [B0, B0 + NB) of a Q8_0 unit (four 32-weight blocks; block j's
 * codes 0..15 in plane 2j, 16..31 in plane 2j + 1), of which the first
 * `nvalid` lie within K. Lane (kc, n) supplies codes 8kc..8kc+7 of a block
 * of row 16g + n: plane 2j + kc / 2, bytes 8 (kc & 1)... */
template <int M, int B0, int NB>
__device__ __forceinline__ void q80_unit_mfma(const uint8_t *slab, const float *xu, int ldx, int lane, int nvalid,
                                              f32x4_t (&acc)[4])
{
    static_assert(B0 + NB <= 4 && NB >= 1, "blocks of one unit");
    constexpr int B1 = B0 + NB;
    const int kc = lane >> 4, n = lane & 15;
    const bool valid = n < M;
    /* Lanes past the batch read position 0; their rows are never stored. */
    const float *xp = xu + (size_t)(valid ? n : 0) * ldx + 8 * kc;
    const uint8_t *qsp = slab + (kc >> 1) * 1024 + n * 16 + 8 * (kc & 1); /* + 2048 j + 256 g */
    uint2 dw[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) dw[g] = *(const uint2 *)(slab + 8192 + (16 * g + n) * 8);
    uint2 q[2][4];
#pragma unroll
    for (int g = 0; g < 4; ++g) q[B0 & 1][g] = *(const uint2 *)(qsp + B0 * 2048 + g * 256);
    float xv[2][8];
    if (B0 < nvalid) load_x<8>(xv[B0 & 1], (gf32 *)(xp + 32 * B0));
#pragma unroll
    for (int j = B0; j < B1; ++j) {
        if (j >= nvalid) break; /* uniform */
        if (j + 1 < B1 && j + 1 < nvalid) {
            load_x<8>(xv[(j + 1) & 1], ptr_after(xp + 32 * (j + 1), acc[0][0]));
            gu8 *nq = bytes_after(qsp + (j + 1) * 2048, acc[1][0]);
#pragma unroll
            for (int g = 0; g < 4; ++g) q[(j + 1) & 1][g] = gload8(nq + g * 256);
        }
        bf16x8_t a0, a1, a2;
        x_limbs<8>(xv[j & 1], true, a0, a1, a2);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const bf16x8_t b = q8_codes_bf16(q[j & 1][g].x, q[j & 1][g].y);
            f32x4_t d = {0.0f, 0.0f, 0.0f, 0.0f};
            d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, b, d, 0, 0, 0);
            d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b, d, 0, 0, 0);
            d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2, b, d, 0, 0, 0);
            const float sc = f16_bits_to_f32(word(dw[g], j >> 1) >> (16 * (j & 1)));
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[g][i] = fmaf(sc, d[i], acc[g][i]);
        }
        /* One block's codes live at a time (as for Q4_K). */
        __builtin_amdgcn_sched_barrier(0);
    }
}

/* Eight Q5_0 codes b - 16 of one block (b = low nibble | fifth bit << 4) as
 * two exact bf16 operands whose sum is b - 16: the nibbles, whose bytes are
 * the FP8 E4M3 patterns of nib * 2^-9 (scale 2^9), and 16 * (bit - 1), the
 * E4M3 patterns of -1 and 0 picked by v_perm_b32 from the table 0xb8, 0x00
 * with the bit as selector (scale 16). n0, n1: the nibbles of codes 0..3 and
 * 4..7 in the low bits of each byte; bits: the eight fifth bits. */
__device__ __forceinline__ void q5_codes_bf16(uint32_t n0, uint32_t n1, uint32_t bits, bf16x8_t &lo,
                                              bf16x8_t &hi)
{
    const uint32_t s0 = ((bits & 15u) * 0x00204081u) & 0x01010101u;
    const uint32_t s1 = (((bits >> 4) & 15u) * 0x00204081u) & 0x01010101u;
    const uint32_t h0 = __builtin_amdgcn_perm(0u, 0x000000b8u, s0);
    const uint32_t h1 = __builtin_amdgcn_perm(0u, 0x000000b8u, s1);
    const bf16x2_t a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(n0, 512.0f, false);
    const bf16x2_t b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(n0, 512.0f, true);
    const bf16x2_t c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(n1, 512.0f, false);
    const bf16x2_t d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(n1, 512.0f, true);
    const bf16x2_t e = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(h0, 16.0f, false);
    const bf16x2_t f = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(h0, 16.0f, true);
    const bf16x2_t g = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(h1, 16.0f, false);
    const bf16x2_t h = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(h1, 16.0f, true);
    lo = bf16x8_t{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
    hi = bf16x8_t{e[0], e[1], f[0], f[1], g[0], g[1], h[0], h[1]};
}

/* Blocks [B0, B0 + NB) of a Q5_0 unit (four 32-weight blocks), of which the
 * first `nvalid` lie within K (the rest of a partial last unit are zero bytes
 * and their activations are not read). Lane (kc, n) supplies weights
 * 8kc..8kc+7 of a block of row 16g + n: low nibbles of qs bytes 8kc.. for
 * kc < 2, high nibbles of bytes 8(kc - 2).. for kc >= 2, and qh bits 8kc... */
template <int M, int B0, int NB>
__device__ __forceinline__ void q50_unit_mfma(const uint8_t *slab, const float *xu, int ldx, int lane, int nvalid,
                                              f32x4_t (&acc)[4])
{
    static_assert(B0 + NB <= 4 && NB >= 1, "blocks of one unit");
    constexpr int B1 = B0 + NB;
    const int kc = lane >> 4, n = lane & 15;
    const bool valid = n < M;
    /* Lanes past the batch read position 0; their rows are never stored. */
    const float *xp = xu + (size_t)(valid ? n : 0) * ldx + 8 * kc;
    const uint8_t *qsp = slab + n * 16 + 8 * (kc & 1); /* + 1024 j + 256 g */
    const int nsh = 4 * (kc >> 1), bsh = 8 * kc;
    uint2 dw[4]; /* the four f16 d's of row 16g + n */
    uint32_t qh[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        dw[g] = *(const uint2 *)(slab + 5120 + (16 * g + n) * 8);
        qh[g] = *(const uint32_t *)(slab + 4096 + (16 * g + n) * 16 + 4 * B0);
    }
    uint2 q[2][4];
#pragma unroll
    for (int g = 0; g < 4; ++g) q[B0 & 1][g] = *(const uint2 *)(qsp + B0 * 1024 + g * 256);
    float xv[2][8];
    if (B0 < nvalid) load_x<8>(xv[B0 & 1], (gf32 *)(xp + 32 * B0));
#pragma unroll
    for (int j = B0; j < B1; ++j) {
        if (j >= nvalid) break; /* uniform */
        uint32_t qhn[4];
        if (j + 1 < B1 && j + 1 < nvalid) {
            load_x<8>(xv[(j + 1) & 1], ptr_after(xp + 32 * (j + 1), acc[0][0]));
            gu8 *nq = bytes_after(qsp + (j + 1) * 1024, acc[1][0]);
            gu8 *nh = bytes_after(slab + 4096 + n * 16 + 4 * (j + 1), acc[1][0]);
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                q[(j + 1) & 1][g] = gload8(nq + g * 256);
                qhn[g] = *(gu32 *)(nh + g * 256);
            }
        }
        bf16x8_t a0, a1, a2;
        x_limbs<8>(xv[j & 1], true, a0, a1, a2);
        /* Row group by row group: one group's two code operands are live at
         * a time, and its six MFMAs overlap the next group's conversion. */
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            bf16x8_t bl, bh;
            q5_codes_bf16((q[j & 1][g].x >> nsh) & 0x0f0f0f0fu, (q[j & 1][g].y >> nsh) & 0x0f0f0f0fu,
                          (qh[g] >> bsh) & 0xffu, bl, bh);
            f32x4_t d = {0.0f, 0.0f, 0.0f, 0.0f};
            d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, bl, d, 0, 0, 0);
            d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, bh, d, 0, 0, 0);
            d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, bl, d, 0, 0, 0);
            d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, bh, d, 0, 0, 0);
            d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2, bl, d, 0, 0, 0);
            d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2, bh, d, 0, 0, 0);
            const float s = f16_bits_to_f32(word(dw[g], j >> 1) >> (16 * (j & 1)));
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[g][i] = fmaf(s, d[i], acc[g][i]);
        }
        if (j + 1 < B1 && j + 1 < nvalid) {
#pragma unroll
            for (int g = 0; g < 4; ++g) qh[g] = qhn[g];
        }
        /* One block's codes live at a time (as for Q4_K). */
        __builtin_amdgcn_sched_barrier(0);
    }
}

/* Q6_K sub-block j = 8G + 2r + hf (16 weights) takes its low nibbles from
 * ql plane 4G + 2(r & 1) + hf (>> 4 for r >= 2) and its two high bits from qh
 * plane 8 + 2G + hf (>> 2r); sub-blocks are visited by (G, hf), so one set of
 * ql/qh words serves four of them. */
/* Pairs [PR0, PR0 + NPR) of a Q6_K unit (four sub-blocks each). */
template <int M, int PR0, int NPR>
__device__ __forceinline__ void q6k_unit_mfma(const uint8_t *slab, const float *xu, int ldx, int lane,
                                              f32x4_t (&acc)[4])
{
    static_assert(PR0 + NPR <= 4 && NPR >= 1, "pairs of one unit");
    constexpr int T0 = 4 * PR0, T1 = 4 * (PR0 + NPR);
    const int kc = lane >> 4, n = lane & 15;
    const bool valid = n < M;
    /* Lanes past the batch read position 0; their rows are never stored. */
    const float *xp = xu + (size_t)(valid ? n : 0) * ldx + 4 * kc;
    const uint8_t *wp = slab + n * 16 + 4 * kc; /* this lane's dword of row 16g + n in a plane */
    uint4 sc[4];
    float dg[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        sc[g] = ld16(slab + 12 * 1024 + (16 * g + n) * 16);
        dg[g] = f16_bits_to_f32(*(const unsigned short *)(slab + 13312 + (16 * g + n) * 2));
    }
    /* Words of pair (G, hf) and the next pair: ql for r & 1 = 0, 1 and qh. */
    uint32_t w[2][4][3];
    constexpr int G0 = PR0 >> 1, H0 = PR0 & 1;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        w[PR0 & 1][g][0] = *(const uint32_t *)(wp + (4 * G0 + H0) * 1024 + g * 256);
        w[PR0 & 1][g][1] = *(const uint32_t *)(wp + (4 * G0 + 2 + H0) * 1024 + g * 256);
        w[PR0 & 1][g][2] = *(const uint32_t *)(wp + (8 + 2 * G0 + H0) * 1024 + g * 256);
    }
    /* Activations of step t (sub-block j(t)) run two steps ahead. */
    auto sub_of = [](int t) { return 8 * (t >> 3) + 2 * (t & 3) + ((t >> 2) & 1); };
    float xv[3][4];
    load_x<4>(xv[T0 % 3], (gf32 *)(xp + 16 * sub_of(T0)));
    if (T0 + 1 < T1) load_x<4>(xv[(T0 + 1) % 3], (gf32 *)(xp + 16 * sub_of(T0 + 1)));
#pragma unroll
    for (int t = T0; t < T1; ++t) {
        const int pr = t >> 2, r = t & 3; /* pair (G, hf) = (pr >> 1, pr & 1) */
        const int G = pr >> 1, hf = pr & 1;
        const int j = 8 * G + 2 * r + hf;
        if (t + 2 < T1) load_x<4>(xv[(t + 2) % 3], ptr_after(xp + 16 * sub_of(t + 2), acc[0][0]));
        if (r == 0 && pr + 1 < PR0 + NPR) {
            const int Gn = (pr + 1) >> 1, hn = (pr + 1) & 1;
            gu8 *np = bytes_after(wp, acc[1][0]);
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                w[(pr + 1) & 1][g][0] = *(gu32 *)(np + (4 * Gn + hn) * 1024 + g * 256);
                w[(pr + 1) & 1][g][1] = *(gu32 *)(np + (4 * Gn + 2 + hn) * 1024 + g * 256);
                w[(pr + 1) & 1][g][2] = *(gu32 *)(np + (8 + 2 * Gn + hn) * 1024 + g * 256);
            }
        }
        bf16x4_t a0, a1, a2;
        x_limbs<4>(xv[t % 3], true, a0, a1, a2);
        bf16x4_t bl[4], bh[4];
#pragma unroll
        for (int g = 0; g < 4; ++g)
            q6_codes_bf16(w[pr & 1][g][r & 1], w[pr & 1][g][2], r, bl[g], bh[g]);
        f32x4_t d[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) d[g] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            d[g] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a0, bl[g], d[g], 0, 0, 0);
            d[g] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a0, bh[g], d[g], 0, 0, 0);
        }
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            d[g] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a1, bl[g], d[g], 0, 0, 0);
            d[g] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a1, bh[g], d[g], 0, 0, 0);
        }
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            d[g] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a2, bl[g], d[g], 0, 0, 0);
            d[g] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a2, bh[g], d[g], 0, 0, 0);
        }
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const float s = dg[g] * sbyte(word(sc[g], j >> 2), j & 3);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[g][i] = fmaf(s, d[g][i], acc[g][i]);
        }
        /* One sub-block's codes and scale live at a time (see Q4_K). */
        __builtin_amdgcn_sched_barrier(0);
    }
}

/* Q6_K at M <= 8 with two sub-blocks per 16x16x32 MFMA. A batch of at most 8
 * positions leaves A rows 8..15 free, and a K = 32 MFMA costs the issue time
 * of a K = 16 one on gfx950 (measured), so sub-blocks j = 8G + 2r + hf
 * (r = 0, 1) and j + 4 (r + 2) run together: A rows 0..7 hold sub-block j's
 * activations of positions 0..7 in k 0..15 and zeros in k 16..31, rows 8..15
 * zeros in k 0..15 and sub-block j + 4's in k 16..31; B holds j's codes in k
 * 0..15 and j + 4's in k 16..31. So D rows 0..7 are j's sums and rows 8..15
 * j + 4's, each scaled by its own sub-block scale: half the MFMAs and half the
 * scale FMAs of one K = 16 step per sub-block. Both sub-blocks take their
 * codes from the same bytes: the ql plane's low (j) and high (j + 4) nibbles
 * and the qh plane's bit pairs 2r and 2r + 4. Lane (kc, n): kc < 2 carries
 * sub-block j, kc >= 2 sub-block j + 4, weights 8 (kc & 1) .. + 7 of it; its A
 * values are zero unless n < 8 matches kc < 2. D[i][n] lands in lane
 * n + 16 (i / 4), so lanes 32..63 hold the j + 4 sums of the positions that
 * lanes 0..31 hold for j; the two halves are added once per work item, so acc
 * must be zero on entry (the kernel runs one work item per wave). */
template <int M, int PR0, int NPR>
__device__ __forceinline__ void q6k_unit_mfma_pair(const uint8_t *slab, const float *xu, int ldx, int lane,
                                                   f32x4_t (&acc)[4])
{
    static_assert(PR0 + NPR <= 4 && NPR >= 1 && M <= 8, "pairs of one unit, at most 8 positions");
    constexpr int S0 = 2 * PR0, S1 = 2 * (PR0 + NPR); /* step s: pr = s >> 1, rr = s & 1 */
    const int kc = lane >> 4, n = lane & 15;
    const bool second = kc >= 2;
    const bool carries = (n < 8) == !second;
    const int pos = n < 8 ? n : n - 8;
    /* Lanes of positions past the batch read position 0; those rows are never
     * stored. Lanes that carry zeros read in bounds too. */
    const float *xp = xu + (size_t)(pos < M ? pos : 0) * ldx + 8 * (kc & 1) + (second ? 64 : 0);
    const uint8_t *wp = slab + n * 16 + 8 * (kc & 1); /* + plane * 1024 + g * 256 */
    const int nsh = second ? 4 : 0;
    uint4 sc[4];
    float dg[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        sc[g] = ld16(slab + 12 * 1024 + (16 * g + n) * 16);
        dg[g] = f16_bits_to_f32(*(const unsigned short *)(slab + 13312 + (16 * g + n) * 2));
    }
    auto first_sub = [](int st) { return 8 * (st >> 2) + 2 * (st & 1) + ((st >> 1) & 1); };
    auto ql_plane = [](int st) { return 4 * (st >> 2) + 2 * (st & 1) + ((st >> 1) & 1); };
    auto qh_plane = [](int st) { return 8 + 2 * (st >> 2) + ((st >> 1) & 1); };
    /* Codes of step s and s + 1 (ql and qh bytes, 8 of each per lane). */
    uint2 ql[2][4], qh[2][4];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        ql[S0 & 1][g] = *(const uint2 *)(wp + ql_plane(S0) * 1024 + g * 256);
        qh[S0 & 1][g] = *(const uint2 *)(wp + qh_plane(S0) * 1024 + g * 256);
    }
    float xv[2][8];
    load_x<8>(xv[S0 & 1], (gf32 *)(xp + 16 * first_sub(S0)));
#pragma unroll
    for (int st = S0; st < S1; ++st) {
        const int j = first_sub(st), rr = st & 1;
        if (st + 1 < S1) {
            load_x<8>(xv[(st + 1) & 1], ptr_after(xp + 16 * first_sub(st + 1), acc[0][0]));
            gu8 *np = bytes_after(wp, acc[1][0]);
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                ql[(st + 1) & 1][g] = gload8(np + ql_plane(st + 1) * 1024 + g * 256);
                qh[(st + 1) & 1][g] = gload8(np + qh_plane(st + 1) * 1024 + g * 256);
            }
        }
        bf16x8_t a0, a1, a2;
        x_limbs<8>(xv[st & 1], carries, a0, a1, a2);
        const int hsh = 2 * rr + (second ? 4 : 0);
        f32x4_t d[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const uint32_t l0 = (ql[st & 1][g].x >> nsh) & 0x0f0f0f0fu, l1 = (ql[st & 1][g].y >> nsh) & 0x0f0f0f0fu;
            const uint32_t h0 = __builtin_amdgcn_perm(0u, 0x01008182u, (qh[st & 1][g].x >> hsh) & 0x03030303u);
            const uint32_t h1 = __builtin_amdgcn_perm(0u, 0x01008182u, (qh[st & 1][g].y >> hsh) & 0x03030303u);
            const bf16x2_t c0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(l0, 512.0f, false);
            const bf16x2_t c1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(l0, 512.0f, true);
            const bf16x2_t c2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(l1, 512.0f, false);
            const bf16x2_t c3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(l1, 512.0f, true);
            const bf16x2_t e0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(h0, 8192.0f, false);
            const bf16x2_t e1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(h0, 8192.0f, true);
            const bf16x2_t e2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(h1, 8192.0f, false);
            const bf16x2_t e3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(h1, 8192.0f, true);
            const bf16x8_t bl = {c0[0], c0[1], c1[0], c1[1], c2[0], c2[1], c3[0], c3[1]};
            const bf16x8_t bh = {e0[0], e0[1], e1[0], e1[1], e2[0], e2[1], e3[0], e3[1]};
            d[g] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
            d[g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, bl, d[g], 0, 0, 0);
            d[g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, bh, d[g], 0, 0, 0);
            d[g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, bl, d[g], 0, 0, 0);
            d[g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, bh, d[g], 0, 0, 0);
            d[g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2, bl, d[g], 0, 0, 0);
            d[g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2, bh, d[g], 0, 0, 0);
        }
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            /* sub-block j's scale for lanes 0..31, j + 4's (the next scale
             * word, same byte) for lanes 32..63 */
            const uint32_t sw = second ? word(sc[g], (j >> 2) + 1) : word(sc[g], j >> 2);
            const float sg = dg[g] * sbyte(sw, j & 3);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[g][i] = fmaf(sg, d[g][i], acc[g][i]);
        }
        /* One step's codes and scales live at a time (as for Q4_K). */
        __builtin_amdgcn_sched_barrier(0);
    }
    /* Lanes 0..31 add the sub-block j + 4 sums of their positions. */
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[g][i] += __shfl_xor(acc[g][i], 32, 64);
}

/* Part `part` of `parts` (1 or 2; wave-uniform) of one unit: consecutive
 * sub-blocks (Q4_K: 8 / parts, Q6_K: 16 / parts). */
template <int FMT, int M>
__device__ __forceinline__ void unit_part_mfma(const uint8_t *slab, const float *xu, int ldx, int lane, int part,
                                               int parts, int kleft, f32x4_t (&acc)[4])
{
    if constexpr (FMT == QMV_FMT_Q5_0 || FMT == QMV_FMT_Q8_0) {
        /* Q5_0 / Q8_0 units are four 32-weight blocks; K is a multiple of 32. */
        const int nvalid = kleft >= 128 ? 4 : kleft / 32;
        if constexpr (FMT == QMV_FMT_Q5_0) {
            if (parts == 1) q50_unit_mfma<M, 0, 4>(slab, xu, ldx, lane, nvalid, acc);
            else if (part == 0) q50_unit_mfma<M, 0, 2>(slab, xu, ldx, lane, nvalid, acc);
            else q50_unit_mfma<M, 2, 2>(slab, xu, ldx, lane, nvalid, acc);
        } else {
            if (parts == 1) q80_unit_mfma<M, 0, 4>(slab, xu, ldx, lane, nvalid, acc);
            else if (part == 0) q80_unit_mfma<M, 0, 2>(slab, xu, ldx, lane, nvalid, acc);
            else q80_unit_mfma<M, 2, 2>(slab, xu, ldx, lane, nvalid, acc);
        }
    } else if constexpr (FMT == QMV_FMT_Q4_K) {
        if (parts == 1) q4k_unit_mfma<M, 0, 8>(slab, xu, ldx, lane, acc);
        else if (part == 0) q4k_unit_mfma<M, 0, 4>(slab, xu, ldx, lane, acc);
        else q4k_unit_mfma<M, 4, 4>(slab, xu, ldx, lane, acc);
    } else {
        if (parts == 1) q6k_unit_mfma_pair<M, 0, 4>(slab, xu, ldx, lane, acc);
        else if (part == 0) q6k_unit_mfma_pair<M, 0, 2>(slab, xu, ldx, lane, acc);
        else q6k_unit_mfma_pair<M, 2, 2>(slab, xu, ldx, lane, acc);
    }
}

/* Same combine and split-K protocol as matvec_kernel; each wave runs one work
 * item on the matrix cores and scatters its 64 rows x M positions into the
 * combine buffer. A work item is a unit, or with p.parts = 2 half of one: a
 * tile then has units x parts items, in unit-major order, so a launch over
 * rows of few units has twice the waves. */
/* Four resident waves per SIMD (at most 128 VGPRs): these waves are short
 * and latency-bound, so residency matters more than registers. */
template <int FMT, int M>
__global__ void __launch_bounds__(QMV_MAX_WAVES * 64) __attribute__((amdgpu_waves_per_eu(4)))
matvec_mfma_kernel(MatvecParams p)
{
    constexpr int SLAB = UnitOf<FMT>::kBytes * 64;
    __shared__ float red[QMV_MAX_WAVES][M][64];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const LaunchArgs a = launch_args(p);
    const int shift = a.parts == 2 ? 1 : 0;
    const WgWork w = locate(a, wave, a.units << shift);
    const uint8_t *wtile = (w.job == a.job ? a.w : p.job[w.job].w) + (size_t)w.tile * a.units * SLAB;

    f32x4_t acc[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) acc[g] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    /* One work item per wave: the host plans units_per_wave = 1 here. */
    if (w.u_begin < w.u_end) {
        const int u = w.u_begin >> shift;
        constexpr int UW = UnitOf<FMT>::kWeights;
        unit_part_mfma<FMT, M>(wtile + (size_t)u * SLAB, a.x + (size_t)u * UW, a.ldx, lane,
                               w.u_begin - (u << shift), 1 << shift, a.cols - u * UW, acc);
    }

    const int kc = lane >> 4, n = lane & 15;
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (4 * kc + j < M) red[wave][4 * kc + j][16 * g + n] = acc[g][j];
    __syncthreads();
    if (wave != 0) return;
    finish_tile<M, 64>(p, w, blockDim.x >> 6, lane, red);
}

/* ---- Prefill batches (9..32 positions), all four formats: GEMM-shaped -------
 * A workgroup of four waves owns four consecutive 64-row tiles of one tensor
 * (one per wave) and a range of K-units. For each unit the 256 threads stage
 * the unit's activations of all positions once, as the three bf16 limbs (see
 * the matrix-core section above) laid out in MFMA A-fragment order, and each
 * wave then runs its tile's unit with A read from LDS: an activation is
 * loaded and split once per workgroup instead of once per wave, and the
 * codes a wave decodes serve every position block of 16. The next unit's
 * activations are loaded into registers, and its weight headers and first
 * codes issued, while the current unit computes. Each wave finishes its own
 * tile with the split-K protocol of finish_tile, so a position's arithmetic
 * does not depend on the other positions of the launch. */
#define QMV_PF_WAVES QMV_PF_TILES
/* Sub-block (Q4_K, of 8) and step (Q6_K, of 16) at which a wave issues the
 * next unit's first weight loads. */
#ifndef QMV_PF_NEXT_SB
#define QMV_PF_NEXT_SB 6
#endif
#ifndef QMV_PF_NEXT_T
#define QMV_PF_NEXT_T 13
#endif
/* A prefill launch carries P position blocks of 16 (P = 1 for up to 16
 * positions, 2 for up to 32). */

/* The staging buffer is addressed through an explicit LDS pointer type so
 * that every access compiles to ds_read / ds_write. */
typedef __attribute__((address_space(3))) uint8_t lds_u8;

/* An LDS offset that cannot be used before `dep` exists (see ptr_after):
 * keeps a sub-block's A-fragment reads from being hoisted across the unit. */
__device__ __forceinline__ int lds_off_after(int off, float dep)
{
    asm("" : "+v"(off) : "v"(dep));
    return off;
}

/* LDS image of one unit: fragment (limb L, position block pb, k-block b) is
 * 64 lanes x KL bf16, lane 16 kc + n holding A[n][KL kc .. KL kc + KL - 1] =
 * limb L of x[16 pb + n][4 KL b + KL kc ..]. */
template <int KL, int P, int UW = 256> struct PfLayout {
    static constexpr int kBlocks = UW / (4 * KL);      /* 8 (Q4_K), 16 (Q6_K) or 4 (Q5_0) */
    static constexpr int kFrag = 64 * 2 * KL;          /* bytes per fragment */
    static constexpr int kChunks = P * kBlocks * 64;   /* (pb, b, lane) chunks of KL activations */
    static constexpr int kPerThread = kChunks / (QMV_PF_WAVES * 64);
    static constexpr int kBytes = 3 * P * kBlocks * kFrag; /* 24 KB per position block */
    __device__ static int offset(int limb, int pb, int b) { return ((limb * P + pb) * kBlocks + b) * kFrag; }
    /* Q4_K: the sub-block sums of the activations as an A operand of 8
     * sub-blocks (fragment (limb, pb): lane n < 16 holds limb L of
     * sum(x[16 pb + n][32 s .. 32 s + 31]) for s = 0..7; lanes 16..63 hold
     * zeros), after the limb images. */
    static constexpr int kSxBytes = 3 * P * 64 * 16;
    __device__ static int sx_offset(int limb, int pb) { return kBytes + (limb * P + pb) * 64 * 16; }
};

/* Chunk c of a unit: lane = c % 64, block b, position block pb. Blocks from
 * kleft on (past K in a partial last Q5_0 unit) are not read and stage
 * zeros. */
template <int KL, int P, int UW = 256>
__device__ __forceinline__ void pf_load_x(const float *xu, int ldx, int npos, int tid,
                                          float (&xr)[PfLayout<KL, P, UW>::kPerThread][KL], int kleft = UW)
{
    using L = PfLayout<KL, P, UW>;
#pragma unroll
    for (int i = 0; i < L::kPerThread; ++i) {
        const int c = tid + i * QMV_PF_WAVES * 64;
        const int lane = c & 63, rest = c >> 6, b = rest % L::kBlocks, pb = rest / L::kBlocks;
        const int kc = lane >> 4, n = lane & 15, pos = 16 * pb + n;
        const bool in_k = UW == 256 || 4 * KL * b < kleft; /* K is a multiple of 256 for K-quants */
        /* Rows past the batch read position 0 (in bounds) and stage zeros. */
        const float *src = xu + (size_t)(pos < npos ? pos : 0) * ldx + (in_k ? 4 * KL * b + KL * kc : 0);
        float v[KL];
#pragma unroll
        for (int j = 0; j < KL; ++j) v[j] = src[j];
#pragma unroll
        for (int j = 0; j < KL; ++j) xr[i][j] = pos < npos && in_k ? v[j] : 0.0f;
    }
}

template <int KL, int P, int UW = 256, bool kSubSums = false>
__device__ __forceinline__ void pf_store_limbs(lds_u8 *lds, int tid,
                                               const float (&xr)[PfLayout<KL, P, UW>::kPerThread][KL])
{
    using L = PfLayout<KL, P, UW>;
    typedef __bf16 frag_t __attribute__((__vector_size__(KL * sizeof(__bf16))));
#pragma unroll
    for (int i = 0; i < L::kPerThread; ++i) {
        const int c = tid + i * QMV_PF_WAVES * 64;
        const int lane = c & 63, rest = c >> 6, b = rest % L::kBlocks, pb = rest / L::kBlocks;
        frag_t h, m, l;
        x_limbs<KL>(xr[i], true, h, m, l);
        typedef __attribute__((address_space(3))) frag_t lds_frag;
        *(lds_frag *)(lds + L::offset(0, pb, b) + lane * 2 * KL) = h;
        *(lds_frag *)(lds + L::offset(1, pb, b) + lane * 2 * KL) = m;
        *(lds_frag *)(lds + L::offset(2, pb, b) + lane * 2 * KL) = l;
        if constexpr (kSubSums) {
            /* Sub-block b's sum for position 16 pb + n: this lane's KL
             * activations in order, then the four lanes n + 16 kc (the
             * chunk's k quarters) pairwise, the same bits in all four. */
            static_assert(KL == 8, "Q4_K sub-blocks: four chunks of 8");
            float t = xr[i][0];
#pragma unroll
            for (int j = 1; j < KL; ++j) t += xr[i][j];
            t += __shfl_xor(t, 16);
            t += __shfl_xor(t, 32);
            if (lane < 16) {
                const __bf16 th = (__bf16)t;
                const float r = t - (float)th;
                const __bf16 tm = (__bf16)r;
                const __bf16 tl = (__bf16)(r - (float)tm);
                typedef __attribute__((address_space(3))) __bf16 lds_bf16;
                const int at = lane * 16 + b * 2;
                *(lds_bf16 *)(lds + L::sx_offset(0, pb) + at) = th;
                *(lds_bf16 *)(lds + L::sx_offset(1, pb) + at) = tm;
                *(lds_bf16 *)(lds + L::sx_offset(2, pb) + at) = tl;
            }
        }
    }
}

/* One Q4_K unit of this wave's tile against the staged activations; h and q0
 * hold the unit's headers and group-0 codes on entry and those of `next` on
 * return (the caller passes the unit itself when there is no next one: the
 * loads are then harmless repeats, and no branch splits the unrolled body). */
template <int P>
__device__ __forceinline__ void q4k_unit_pf(const uint8_t *slab, const uint8_t *next, const lds_u8 *lds, int lane,
                                            f32x4_t (&acc)[P][4], uint4 (&h)[4], uint2 (&q0)[4])
{
    using L = PfLayout<8, P>;
    const int kc = lane >> 4, n = lane & 15;
    const int qoff = (1 + (kc >> 1)) * 1024 + n * 16 + 8 * (kc & 1);
    const uint8_t *qsp = slab + qoff;
    uint2 q[2][4];
#pragma unroll
    for (int g = 0; g < 4; ++g) q[0][g] = q0[g];
    uint4 hn[4];
    uint2 qn[4];
    /* The minimum terms of the whole unit on the matrix cores:
     * sum_s m_s * sum(x over sub-block s) per row and position, with the
     * staged sub-block sums (exact limbs) as A, k = s < 8, and each row's 8
     * six-bit minimums (exact in bf16) as B; then acc -= dmin * that once. */
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const uint4 hg = h[g];
        const uint32_t mlo = hg.z & 0x3f3f3f3fu;
        const uint32_t mhi = ((hg.w >> 4) & 0x0f0f0f0fu) | ((hg.z >> 2) & 0x30303030u);
        const bf16x8_t bm = {(__bf16)ubyte(mlo, 0), (__bf16)ubyte(mlo, 1), (__bf16)ubyte(mlo, 2),
                             (__bf16)ubyte(mlo, 3), (__bf16)ubyte(mhi, 0), (__bf16)ubyte(mhi, 1),
                             (__bf16)ubyte(mhi, 2), (__bf16)ubyte(mhi, 3)};
        const float dmin = f16_bits_to_f32(hg.x >> 16);
#pragma unroll
        for (int pb = 0; pb < P; ++pb) {
            typedef __attribute__((address_space(3))) const bf16x8_t lds_a;
            f32x4_t dm = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int limb = 0; limb < 3; ++limb)
                dm = __builtin_amdgcn_mfma_f32_16x16x32_bf16(*(lds_a *)(lds + L::sx_offset(limb, pb) + lane * 16), bm,
                                                             dm, 0, 0, 0);
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[pb][g][j] = fmaf(-dmin, dm[j], acc[pb][g][j]);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    /* Group c's codes load two steps before the step that converts them
     * (step 2c - 1, below): group 1's here, groups 2 and 3 at steps 1 and
     * 3, each into the buffer the group before last used. */
    {
        gu8 *nq = bytes_after(qsp + 2048, acc[0][1][0]);
#pragma unroll
        for (int g = 0; g < 4; ++g) q[1][g] = gload8(nq + g * 256);
    }
    /* A software pipeline over the 8 sub-blocks: step sb issues its MFMAs,
     * the code conversion of sub-block sb + 1 (b -> bn) and the scale FMAs
     * of sub-block sb - 1 (dp, sp), none of which depends on the others, so
     * the VALU work runs under the matrix-core work. acc takes the
     * sub-blocks in order, as without the pipeline. */
    bf16x8_t b[4], bn[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) b[g] = q4_codes_bf16(q[0][g].x, q[0][g].y, false);
    f32x4_t dp[P][4];
    float sp[4];
    /* One position block: the activation fragments of sub-block sb + 1 are
     * read from LDS during step sb, as in q6k_unit_pf (gate|up at 16
     * positions 34.1 -> 32.2 µs in a cold graph of its launches, the
     * 16-position decode set 2.582 -> 2.572 ms). Two blocks keep the reads
     * in the step: the 24 more VGPRs take the kernel from 248 to 267 and to
     * one wave per SIMD (gate|up at 32 positions 47.2 -> 60.0 µs). */
    constexpr bool kAhead = P == 1;
    typedef __attribute__((address_space(3))) const bf16x8_t lds_a;
    bf16x8_t fa[P][3], fn[P][3];
    if constexpr (kAhead) {
#pragma unroll
        for (int pb = 0; pb < P; ++pb) {
            const lds_u8 *la = lds + lds_off_after(lane * 16, acc[pb][3][3]);
#pragma unroll
            for (int l = 0; l < 3; ++l) fa[pb][l] = *(lds_a *)(la + L::offset(l, pb, 0));
        }
    }
#pragma unroll
    for (int sb = 0; sb < 8; ++sb) {
        const bool high = sb & 1;
        if (high && (sb + 3) / 2 < 4) {
            const int cn = (sb + 3) / 2;
            gu8 *nq = bytes_after(qsp + cn * 2048, acc[0][1][0]);
#pragma unroll
            for (int g = 0; g < 4; ++g) q[cn & 1][g] = gload8(nq + g * 256);
        }
        if (sb == QMV_PF_NEXT_SB) {
            gu8 *np = bytes_after(next, acc[0][2][0]);
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                hn[g] = gload16(np + n * 16 + g * 256);
                qn[g] = gload8(np + qoff + g * 256);
            }
        }
        if (sb + 1 < 8)
#pragma unroll
            for (int g = 0; g < 4; ++g)
                bn[g] = q4_codes_bf16(q[((sb + 1) >> 1) & 1][g].x, q[((sb + 1) >> 1) & 1][g].y, !high);
        float sa[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const uint4 hg = h[g];
            const float dd = f16_bits_to_f32(hg.x);
            const uint32_t scw = sb < 4 ? hg.y & 0x3f3f3f3fu : (hg.w & 0x0f0f0f0fu) | ((hg.y >> 2) & 0x30303030u);
            sa[g] = dd * ubyte(scw, sb & 3);
        }
        f32x4_t d[P][4];
#pragma unroll
        for (int pb = 0; pb < P; ++pb) {
            bf16x8_t a0, a1, a2;
            if constexpr (kAhead) {
                a0 = fa[pb][0];
                a1 = fa[pb][1];
                a2 = fa[pb][2];
                if (sb + 1 < 8)
#pragma unroll
                    for (int l = 0; l < 3; ++l) fn[pb][l] = *(lds_a *)(lds + lane * 16 + L::offset(l, pb, sb + 1));
            } else {
                const lds_u8 *la = lds + lds_off_after(lane * 16, acc[pb][3][3]);
                a0 = *(lds_a *)(la + L::offset(0, pb, sb));
                a1 = *(lds_a *)(la + L::offset(1, pb, sb));
                a2 = *(lds_a *)(la + L::offset(2, pb, sb));
            }
#pragma unroll
            for (int g = 0; g < 4; ++g) d[pb][g] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int g = 0; g < 4; ++g) d[pb][g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, b[g], d[pb][g], 0, 0, 0);
#pragma unroll
            for (int g = 0; g < 4; ++g) d[pb][g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b[g], d[pb][g], 0, 0, 0);
#pragma unroll
            for (int g = 0; g < 4; ++g) d[pb][g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2, b[g], d[pb][g], 0, 0, 0);
        }
        if (sb > 0)
#pragma unroll
            for (int pb = 0; pb < P; ++pb)
#pragma unroll
                for (int g = 0; g < 4; ++g)
#pragma unroll
                    for (int j = 0; j < 4; ++j) acc[pb][g][j] = fmaf(sp[g], dp[pb][g][j], acc[pb][g][j]);
        /* One step per scheduling region: only the pipeline's hand-over
         * values live across it. */
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            b[g] = bn[g];
            sp[g] = sa[g];
#pragma unroll
            for (int pb = 0; pb < P; ++pb) dp[pb][g] = d[pb][g];
        }
        if constexpr (kAhead)
#pragma unroll
            for (int pb = 0; pb < P; ++pb)
#pragma unroll
                for (int l = 0; l < 3; ++l) fa[pb][l] = fn[pb][l];
    }
#pragma unroll
    for (int pb = 0; pb < P; ++pb)
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[pb][g][j] = fmaf(sp[g], dp[pb][g][j], acc[pb][g][j]);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        h[g] = hn[g];
        q0[g] = qn[g];
    }
}

/* Q6_K: sc, dg and w0 (the first (G, hf) pair's words) hold this unit's on
 * entry and those of `next` on return (as for Q4_K). */
template <int P>
__device__ __forceinline__ void q6k_unit_pf(const uint8_t *slab, const uint8_t *next, const lds_u8 *lds, int lane,
                                            f32x4_t (&acc)[P][4], uint4 (&sc)[4], uint32_t (&dgw)[4],
                                            uint32_t (&w0)[4][3])
{
    using L = PfLayout<4, P>;
    const int kc = lane >> 4, n = lane & 15;
    const int woff = n * 16 + 4 * kc;
    const uint8_t *wp = slab + woff;
    float dg[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) dg[g] = f16_bits_to_f32(dgw[g] & 0xffffu);
    uint32_t w[3][4][3];
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int e = 0; e < 3; ++e) w[0][g][e] = w0[g][e];
    uint4 scn[4];
    uint32_t dgn[4], wn[4][3];
    /* The code words of pair pn (the ql / qh dwords of four sub-blocks) into
     * buffer pn % 3: pair 1 here, pairs 2 and 3 at steps 2 and 6, so each
     * lands 4-5 steps before the step that converts its first codes (step
     * 4 pn - 1) and overwrites the buffer of a pair converted for the last
     * time at step 4 (pn - 3) + 2. Two buffers (loads 3 steps ahead) ran
     * Q6_K at 32 positions 43.6 against 43.3 µs, at 16 35.7 against 35.3. */
    auto load_pair = [&](int pn, gu8 *base) {
        const int Gn = pn >> 1, hn = pn & 1;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            w[pn % 3][g][0] = *(gu32 *)(base + (4 * Gn + hn) * 1024 + g * 256);
            w[pn % 3][g][1] = *(gu32 *)(base + (4 * Gn + 2 + hn) * 1024 + g * 256);
            w[pn % 3][g][2] = *(gu32 *)(base + (8 + 2 * Gn + hn) * 1024 + g * 256);
        }
    };
    load_pair(1, bytes_after(wp, acc[0][1][0]));
    /* Step t's code operands: one combined operand per code (q - 32, exact
     * in bf16), converted once for every position block. The two-operand
     * form of the M <= 8 kernel (q6_codes_bf16) would double the MFMAs of
     * each block, and using it for one block only would make a position's
     * rounding depend on the number of positions in its launch. */
    auto decode = [&](int t, bf16x4_t (&b)[4]) {
        const int pr = t >> 2, r = t & 3;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const uint32_t lw = w[pr % 3][g][r & 1];
            const uint32_t hw = w[pr % 3][g][2];
            const uint32_t c = codes(((lw >> (4 * (r >> 1))) & 0x0f0f0f0fu) | (((hw >> (2 * r)) & 0x03030303u) << 4));
#pragma unroll
            for (int i = 0; i < 4; ++i) b[g][i] = (__bf16)(ubyte(c, i) - 32.0f); /* exact: -32..31 */
        }
    };
    /* A software pipeline over the 16 steps: step t issues its MFMAs, the
     * code conversion of step t + 1 (b -> bn) and the scale FMAs of step
     * t - 1 (dp, sp), none of which depends on the others, so the VALU work
     * runs under the matrix-core work instead of before and after it. acc
     * takes the steps in order, as without the pipeline. */
    bf16x4_t b[4], bn[4];
    decode(0, b);
    f32x4_t dp[P][4];
    float sp[4];
    /* The staged activation fragments of step t (sub-block sub_of(t)) are
     * read from LDS during step t - 1 (fa: this step's, fn: the next
     * step's), so no step waits for its LDS reads: M = 32 decode set
     * 3.430-3.456 -> 3.382-3.387 ms (Q6_K launches 44.8 -> 43.6 µs). The
     * Q4_K unit keeps its reads in the step: the same change takes it from
     * 248 to 267 VGPRs, one wave per SIMD, and the set to 3.81 against 3.47
     * ms. */
    auto sub_of = [](int t) { return 8 * (t >> 3) + 2 * (t & 3) + ((t >> 2) & 1); };
    typedef __attribute__((address_space(3))) const bf16x4_t lds_a;
    bf16x4_t fa[P][3], fn[P][3];
#pragma unroll
    for (int pb = 0; pb < P; ++pb) {
        const lds_u8 *la = lds + lds_off_after(lane * 8, acc[pb][3][3]);
#pragma unroll
        for (int l = 0; l < 3; ++l) fa[pb][l] = *(lds_a *)(la + L::offset(l, pb, sub_of(0)));
    }
#pragma unroll
    for (int t = 0; t < 16; ++t) {
        const int pr = t >> 2, r = t & 3;
        const int G = pr >> 1;
        const int j = 8 * G + 2 * r + (pr & 1);
        if (t == 2 || t == 6) load_pair((t + 6) / 4, bytes_after(wp, acc[0][1][0]));
        if (t == QMV_PF_NEXT_T) {
            gu8 *np = bytes_after(next, acc[0][2][0]);
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                scn[g] = gload16(np + 12 * 1024 + (16 * g + n) * 16);
                dgn[g] = *(gu16 *)(np + 13312 + (16 * g + n) * 2);
                wn[g][0] = *(gu32 *)(np + woff + 0 * 1024 + g * 256);
                wn[g][1] = *(gu32 *)(np + woff + 2 * 1024 + g * 256);
                wn[g][2] = *(gu32 *)(np + woff + 8 * 1024 + g * 256);
            }
        }
        if (t + 1 < 16) decode(t + 1, bn);
        float s[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) s[g] = dg[g] * sbyte(word(sc[g], j >> 2), j & 3);
        f32x4_t d[P][4];
#pragma unroll
        for (int pb = 0; pb < P; ++pb) {
            const bf16x4_t a0 = fa[pb][0], a1 = fa[pb][1], a2 = fa[pb][2];
            if (t + 1 < 16) {
                const lds_u8 *la = lds + lane * 8;
#pragma unroll
                for (int l = 0; l < 3; ++l) fn[pb][l] = *(lds_a *)(la + L::offset(l, pb, sub_of(t + 1)));
            }
#pragma unroll
            for (int g = 0; g < 4; ++g) d[pb][g] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int g = 0; g < 4; ++g) d[pb][g] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a0, b[g], d[pb][g], 0, 0, 0);
#pragma unroll
            for (int g = 0; g < 4; ++g) d[pb][g] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a1, b[g], d[pb][g], 0, 0, 0);
#pragma unroll
            for (int g = 0; g < 4; ++g) d[pb][g] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a2, b[g], d[pb][g], 0, 0, 0);
        }
        if (t > 0)
#pragma unroll
            for (int pb = 0; pb < P; ++pb)
#pragma unroll
                for (int g = 0; g < 4; ++g)
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[pb][g][i] = fmaf(sp[g], dp[pb][g][i], acc[pb][g][i]);
        /* One step per scheduling region: only the pipeline's hand-over
         * values live across it. */
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            b[g] = bn[g];
            sp[g] = s[g];
#pragma unroll
            for (int pb = 0; pb < P; ++pb) dp[pb][g] = d[pb][g];
        }
#pragma unroll
        for (int pb = 0; pb < P; ++pb)
#pragma unroll
            for (int l = 0; l < 3; ++l) fa[pb][l] = fn[pb][l];
    }
#pragma unroll
    for (int pb = 0; pb < P; ++pb)
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[pb][g][i] = fmaf(sp[g], dp[pb][g][i], acc[pb][g][i]);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        sc[g] = scn[g];
        dgw[g] = dgn[g];
#pragma unroll
        for (int e = 0; e < 3; ++e) w0[g][e] = wn[g][e];
    }
}

/* Q8_0: as q50_unit_pf with one code operand per block (q8_codes_bf16); dw
 * and q0 (block 0's codes) carry over to `next`. */
template <int P>
__device__ __forceinline__ void q80_unit_pf(const uint8_t *slab, const uint8_t *next, const lds_u8 *lds, int lane,
                                            int nvalid, f32x4_t (&acc)[P][4], uint2 (&dw)[4], uint2 (&q0)[4])
{
    using L = PfLayout<8, P, 128>;
    const int kc = lane >> 4, n = lane & 15;
    const int qoff = (kc >> 1) * 1024 + n * 16 + 8 * (kc & 1); /* + 2048 j + 256 g */
    const uint8_t *qsp = slab + qoff;
    uint2 q[2][4];
#pragma unroll
    for (int g = 0; g < 4; ++g) q[0][g] = q0[g];
    uint2 dn[4], qn[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        if (j + 1 < 4) {
            gu8 *nq = bytes_after(qsp + (j + 1) * 2048, acc[0][1][0]);
#pragma unroll
            for (int g = 0; g < 4; ++g) q[(j + 1) & 1][g] = gload8(nq + g * 256);
        }
        if (j == 2) {
            gu8 *np = bytes_after(next, acc[0][2][0]);
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                dn[g] = gload8(np + 8192 + (16 * g + n) * 8);
                qn[g] = gload8(np + qoff + g * 256);
            }
        }
        if (j < nvalid) { /* uniform */
            bf16x8_t b[4];
            float sd[4];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                b[g] = q8_codes_bf16(q[j & 1][g].x, q[j & 1][g].y);
                sd[g] = f16_bits_to_f32(word(dw[g], j >> 1) >> (16 * (j & 1)));
            }
#pragma unroll
            for (int pb = 0; pb < P; ++pb) {
                typedef __attribute__((address_space(3))) const bf16x8_t lds_a;
                const lds_u8 *la = lds + lds_off_after(lane * 16, acc[pb][3][3]);
                const bf16x8_t a0 = *(lds_a *)(la + L::offset(0, pb, j));
                const bf16x8_t a1 = *(lds_a *)(la + L::offset(1, pb, j));
                const bf16x8_t a2 = *(lds_a *)(la + L::offset(2, pb, j));
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    f32x4_t d = {0.0f, 0.0f, 0.0f, 0.0f};
                    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, b[g], d, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b[g], d, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2, b[g], d, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[pb][g][i] = fmaf(sd[g], d[i], acc[pb][g][i]);
                }
            }
        }
        /* One block's codes live at a time. */
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        dw[g] = dn[g];
        q0[g] = qn[g];
    }
}

/* Q5_0: the unit's four blocks against the staged activations, each block's
 * two code operands (q5_codes_bf16) converted once for every position block.
 * dw (the four d's), qh (the four qh words) and q0 (block 0's codes) hold
 * this unit's on entry and those of `next` on return (as for Q4_K). Blocks
 * from nvalid on lie past K (zero bytes, zeros staged) and are skipped. */
template <int P>
__device__ __forceinline__ void q50_unit_pf(const uint8_t *slab, const uint8_t *next, const lds_u8 *lds, int lane,
                                            int nvalid, f32x4_t (&acc)[P][4], uint2 (&dw)[4], uint4 (&qh)[4],
                                            uint2 (&q0)[4])
{
    using L = PfLayout<8, P, 128>;
    const int kc = lane >> 4, n = lane & 15;
    const int qoff = n * 16 + 8 * (kc & 1); /* + 1024 j + 256 g */
    const uint8_t *qsp = slab + qoff;
    const int nsh = 4 * (kc >> 1), bsh = 8 * kc;
    uint2 q[2][4];
#pragma unroll
    for (int g = 0; g < 4; ++g) q[0][g] = q0[g];
    uint2 dn[4], qn[4];
    uint4 hn[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        if (j + 1 < 4) {
            gu8 *nq = bytes_after(qsp + (j + 1) * 1024, acc[0][1][0]);
#pragma unroll
            for (int g = 0; g < 4; ++g) q[(j + 1) & 1][g] = gload8(nq + g * 256);
        }
        if (j == 2) {
            gu8 *np = bytes_after(next, acc[0][2][0]);
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                dn[g] = gload8(np + 5120 + (16 * g + n) * 8);
                hn[g] = gload16(np + 4096 + (16 * g + n) * 16);
                qn[g] = gload8(np + qoff + g * 256);
            }
        }
        if (j < nvalid) { /* uniform */
            bf16x8_t bl[4], bh[4];
            float sd[4];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                q5_codes_bf16((q[j & 1][g].x >> nsh) & 0x0f0f0f0fu, (q[j & 1][g].y >> nsh) & 0x0f0f0f0fu,
                              (word(qh[g], j) >> bsh) & 0xffu, bl[g], bh[g]);
                sd[g] = f16_bits_to_f32(word(dw[g], j >> 1) >> (16 * (j & 1)));
            }
#pragma unroll
            for (int pb = 0; pb < P; ++pb) {
                typedef __attribute__((address_space(3))) const bf16x8_t lds_a;
                const lds_u8 *la = lds + lds_off_after(lane * 16, acc[pb][3][3]);
                const bf16x8_t a0 = *(lds_a *)(la + L::offset(0, pb, j));
                const bf16x8_t a1 = *(lds_a *)(la + L::offset(1, pb, j));
                const bf16x8_t a2 = *(lds_a *)(la + L::offset(2, pb, j));
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    f32x4_t d = {0.0f, 0.0f, 0.0f, 0.0f};
                    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, bl[g], d, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, bh[g], d, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, bl[g], d, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, bh[g], d, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2, bl[g], d, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2, bh[g], d, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[pb][g][i] = fmaf(sd[g], d[i], acc[pb][g][i]);
                }
            }
        }
        /* One block's codes live at a time. */
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        dw[g] = dn[g];
        qh[g] = hn[g];
        q0[g] = qn[g];
    }
}

/* The workgroup's place in a prefill launch: job, tile group, K-split; this
 * wave's tile is 4 * group + wave (it may lie past the job's last tile, and
 * then the wave only helps stage). */
__device__ __forceinline__ WgWork locate_pf(const MatvecParams &p, int wave)
{
    WgWork w;
    const int j = job_of_block(p);
    const MatvecJob &job = p.job[j];
    const int local = blockIdx.x - job.wg_begin;
    const int group = local / job.splits;
    w.job = j;
    w.split = local - group * job.splits;
    w.tile = group * QMV_PF_WAVES + wave;
    w.u_begin = w.split * job.units_per_split;
    w.u_end = min(w.u_begin + job.units_per_split, p.units);
    return w;
}

/* Prefill epilogue. A wave's tile values v(m) = val[m * 64 + lane] (m <
 * npos) live in its LDS slice, and the loops over positions stay rolled:
 * unrolled over 32 positions, the epilogue alone would be several times the
 * instruction cache. Same split-K, addend and SwiGLU protocols (and the same
 * partial order) as finish_tile / emit_tile. */
typedef __attribute__((address_space(3))) float lds_f32;

template <int MP>
__device__ __forceinline__ void pf_emit(const MatvecParams &p, const WgWork &w, int lane, lds_f32 *val, int npos)
{
    const MatvecJob &job = p.job[w.job];
    const int row = w.tile * 64 + lane;
    const bool valid = row < job.rows;
    if (job.add != nullptr && valid)
        for (int m = 0; m < npos; ++m) val[m * 64 + lane] += job.add[(size_t)m * job.ldadd + row];
    if (p.swiglu) {
        const MatvecJob &out = p.job[0];
        float *mine = p.pair_vals + ((size_t)w.job * out.tiles + w.tile) * MP * 64 + lane;
        for (int m = 0; m < npos; ++m) store_partial(mine + m * 64, val[m * 64 + lane]);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        unsigned prev = 0;
        if (lane == 0)
            prev = __hip_atomic_fetch_add(p.pair_count + w.tile * QMV_COUNTER_STRIDE, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        prev = __builtin_amdgcn_readfirstlane(__builtin_amdgcn_readlane(prev, 0));
        if (prev == 0u) return;
        asm volatile("" ::: "memory");
        const float *other = p.pair_vals + ((size_t)(1 - w.job) * out.tiles + w.tile) * MP * 64 + lane;
        for (int m0 = 0; m0 < npos; m0 += 8) {
            float o[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) o[i] = m0 + i < npos ? load_partial(other + (m0 + i) * 64) : 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                if (m0 + i >= npos) break;
                const float v = val[(m0 + i) * 64 + lane];
                const float g = w.job == 0 ? v : o[i];
                const float u = w.job == 0 ? o[i] : v;
                if (valid) out.y[(size_t)(m0 + i) * out.ldy + row] = swiglu_value(g, u);
            }
        }
        if (lane == 0) __hip_atomic_store(p.pair_count + w.tile * QMV_COUNTER_STRIDE, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    if (valid)
        for (int m = 0; m < npos; ++m) job.y[(size_t)m * job.ldy + row] = val[m * 64 + lane];
}

template <int MP>
__device__ __forceinline__ void pf_finish(const MatvecParams &p, const WgWork &w, int lane, lds_f32 *val, int npos)
{
    const MatvecJob &job = p.job[w.job];
    const int S = job.splits;
    if (S > 1) {
        /* The tile's partials, split-major; within a split, quad q of lane l
         * (position rows 4q..4q+3) at [split][q][l], so a lane publishes and
         * reads them with 16-byte accesses (MP / 4 per split instead of MP)
         * and each access of the wave covers 1 KiB of consecutive bytes:
         * M = 32 set 3.82 -> 3.74 ms. The accesses are agent-coherent (sc1),
         * as store_partial's, written as global instructions (the buffer
         * forms of the same accesses ran the set in 4.6 ms). The stores are
         * complete at the explicit wait below; the loads complete inside
         * their own asm statement, so no value is read before it lands. */
        float *part = p.partials + job.partial_offset + ((size_t)w.tile * S) * MP * 64;
        unsigned *count = p.counters + job.counter_offset + w.tile * QMV_COUNTER_STRIDE;
        float *mine = part + ((size_t)w.split * (MP / 4) * 64 + lane) * 4;
#pragma unroll
        for (int q = 0; q < MP / 4; ++q) {
            const f32x4_t v = {val[(4 * q) * 64 + lane], val[(4 * q + 1) * 64 + lane], val[(4 * q + 2) * 64 + lane],
                               val[(4 * q + 3) * 64 + lane]};
            asm volatile("global_store_dwordx4 %0, %1, off sc1" ::"v"(mine + q * 256), "v"(v) : "memory");
        }
        /* Deferred finish: pf_reduce_kernel, launched next, sums the tile. */
        if (p.pf_deferred) return;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        unsigned prev = 0;
        if (lane == 0) prev = __hip_atomic_fetch_add(count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        prev = __builtin_amdgcn_readfirstlane(__builtin_amdgcn_readlane(prev, 0));
        if (prev != (unsigned)S - 1u) return;
        asm volatile("" ::: "memory");
        /* 16 quads per round (two splits of 32 position rows, or four of 16),
         * splits past the last repeating it and not added; each position is
         * summed in split order, as sum_partials does. */
        static_assert(MP == 32 || MP == 16, "position rows of a prefill launch");
        constexpr int SB = 64 / MP;
        float sum[MP];
        for (int s0 = 0; s0 < S; s0 += SB) {
            f32x4_t v[16];
            const float *pk[4];
#pragma unroll
            for (int k = 0; k < 4; ++k)
                pk[k] = part + ((size_t)min(s0 + (MP == 32 ? k / 2 : k), S - 1) * (MP / 4) * 64 + lane) * 4 +
                        (MP == 32 ? (k & 1) * 1024 : 0);
            asm volatile("global_load_dwordx4 %0, %16, off sc1\n global_load_dwordx4 %1, %16, off offset:1024 sc1\n"
                         "global_load_dwordx4 %2, %16, off offset:2048 sc1\n global_load_dwordx4 %3, %16, off offset:3072 sc1\n"
                         "global_load_dwordx4 %4, %17, off sc1\n global_load_dwordx4 %5, %17, off offset:1024 sc1\n"
                         "global_load_dwordx4 %6, %17, off offset:2048 sc1\n global_load_dwordx4 %7, %17, off offset:3072 sc1\n"
                         "global_load_dwordx4 %8, %18, off sc1\n global_load_dwordx4 %9, %18, off offset:1024 sc1\n"
                         "global_load_dwordx4 %10, %18, off offset:2048 sc1\n global_load_dwordx4 %11, %18, off offset:3072 sc1\n"
                         "global_load_dwordx4 %12, %19, off sc1\n global_load_dwordx4 %13, %19, off offset:1024 sc1\n"
                         "global_load_dwordx4 %14, %19, off offset:2048 sc1\n global_load_dwordx4 %15, %19, off offset:3072 sc1\n"
                         "s_waitcnt vmcnt(0)"
                         : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]), "=&v"(v[6]),
                           "=&v"(v[7]), "=&v"(v[8]), "=&v"(v[9]), "=&v"(v[10]), "=&v"(v[11]), "=&v"(v[12]),
                           "=&v"(v[13]), "=&v"(v[14]), "=&v"(v[15])
                         : "v"(pk[0]), "v"(pk[1]), "v"(pk[2]), "v"(pk[3])
                         : "memory");
#pragma unroll
            for (int k = 0; k < SB; ++k)
                if (s0 + k < S)
#pragma unroll
                    for (int q = 0; q < MP / 4; ++q)
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const float x = v[k * (MP / 4) + q][e];
                            sum[4 * q + e] = s0 + k == 0 ? x : sum[4 * q + e] + x;
                        }
        }
#pragma unroll
        for (int i = 0; i < MP; ++i)
            if (i < npos) val[i * 64 + lane] = sum[i];
        if (lane == 0) __hip_atomic_store(count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    pf_emit<MP>(p, w, lane, val, npos);
}

template <int FMT, int P>
__global__ void __launch_bounds__(QMV_PF_WAVES * 64) prefill_kernel(MatvecParams p)
{
    constexpr int KL = FMT == QMV_FMT_Q6_K ? 4 : 8;
    constexpr int SLAB = UnitOf<FMT>::kBytes * 64;
    constexpr int UW = UnitOf<FMT>::kWeights;
    constexpr int MP = 16 * P; /* position rows of the launch */
    using L = PfLayout<KL, P, UW>;
    /* The combine buffer (each wave's tile, MP x 64 floats) reuses the
     * staging buffer. */
    constexpr bool kSubSums = FMT == QMV_FMT_Q4_K; /* the minimum terms on the matrix cores (q4k_unit_pf) */
    constexpr int kStage = L::kBytes + (kSubSums ? L::kSxBytes : 0);
    constexpr int kLds = kStage > QMV_PF_WAVES * MP * 64 * 4 ? kStage : QMV_PF_WAVES * MP * 64 * 4;
    __shared__ __attribute__((aligned(16))) uint8_t lds_buf[kLds];
    lds_u8 *lds = (lds_u8 *)lds_buf;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const WgWork w = locate_pf(p, wave);
    const MatvecJob &job = p.job[w.job];
    const bool active = w.tile < job.tiles;
    const int npos = p.positions;
    const uint8_t *wtile = job.w + (size_t)(active ? w.tile : 0) * p.units * SLAB;
    const int kc = lane >> 4, n = lane & 15;

    f32x4_t acc[P][4];
#pragma unroll
    for (int pb = 0; pb < P; ++pb)
#pragma unroll
        for (int g = 0; g < 4; ++g) acc[pb][g] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

    /* First unit's weights (this wave's tile) and activations. */
    uint4 h[4];
    uint2 q0[4], dw[4];
    uint32_t dgw[4], w0[4][3];
    const uint8_t *first = wtile + (size_t)w.u_begin * SLAB;
    if constexpr (FMT == QMV_FMT_Q8_0) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            dw[g] = *(const uint2 *)(first + 8192 + (16 * g + n) * 8);
            q0[g] = *(const uint2 *)(first + (kc >> 1) * 1024 + n * 16 + 8 * (kc & 1) + g * 256);
        }
    } else if constexpr (FMT == QMV_FMT_Q5_0) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            dw[g] = *(const uint2 *)(first + 5120 + (16 * g + n) * 8);
            h[g] = ld16(first + 4096 + (16 * g + n) * 16);
            q0[g] = *(const uint2 *)(first + n * 16 + 8 * (kc & 1) + g * 256);
        }
    } else if constexpr (FMT == QMV_FMT_Q4_K) {
        const int qoff = (1 + (kc >> 1)) * 1024 + n * 16 + 8 * (kc & 1);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            h[g] = ld16(first + n * 16 + g * 256);
            q0[g] = *(const uint2 *)(first + qoff + g * 256);
        }
    } else {
        const int woff = n * 16 + 4 * kc;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            h[g] = ld16(first + 12 * 1024 + (16 * g + n) * 16);
            dgw[g] = *(const unsigned short *)(first + 13312 + (16 * g + n) * 2);
            w0[g][0] = *(const uint32_t *)(first + woff + 0 * 1024 + g * 256);
            w0[g][1] = *(const uint32_t *)(first + woff + 2 * 1024 + g * 256);
            w0[g][2] = *(const uint32_t *)(first + woff + 8 * 1024 + g * 256);
        }
    }
    float xr[L::kPerThread][KL];
    pf_load_x<KL, P, UW>(p.x + (size_t)w.u_begin * UW, p.ldx, npos, tid, xr, p.cols - w.u_begin * UW);
    if constexpr (kSubSums) {
        /* Lanes 16..63 of the sub-sum fragments stay zero (only lanes 0..15
         * are rewritten per unit); the first barrier below orders this. */
        typedef __attribute__((address_space(3))) u32v4 lds_v4;
        for (int i = tid; i < L::kSxBytes / 16; i += QMV_PF_WAVES * 64)
            *(lds_v4 *)(lds + L::kBytes + 16 * i) = u32v4{0u, 0u, 0u, 0u};
    }

    for (int u = w.u_begin; u < w.u_end; ++u) {
        __syncthreads(); /* every wave is done with the previous unit's image */
        pf_store_limbs<KL, P, UW, kSubSums>(lds, tid, xr);
        __syncthreads();
        if (u + 1 < w.u_end)
            pf_load_x<KL, P, UW>(p.x + (size_t)(u + 1) * UW, p.ldx, npos, tid, xr, p.cols - (u + 1) * UW);
        const uint8_t *slab = wtile + (size_t)u * SLAB;
        const uint8_t *next = u + 1 < w.u_end ? slab + SLAB : slab;
        if (active) {
            if constexpr (FMT == QMV_FMT_Q5_0 || FMT == QMV_FMT_Q8_0) {
                const int kleft = p.cols - u * UW; /* K is a multiple of 32 */
                const int nvalid = kleft >= 128 ? 4 : kleft / 32;
                if constexpr (FMT == QMV_FMT_Q5_0) q50_unit_pf<P>(slab, next, lds, lane, nvalid, acc, dw, h, q0);
                else q80_unit_pf<P>(slab, next, lds, lane, nvalid, acc, dw, q0);
            } else if constexpr (FMT == QMV_FMT_Q4_K) {
                q4k_unit_pf<P>(slab, next, lds, lane, acc, h, q0);
            } else {
                q6k_unit_pf<P>(slab, next, lds, lane, acc, h, dgw, w0);
            }
        }
    }

    /* Each wave transposes its tile through its own slice of the (now free)
     * staging buffer, then finishes the tile on its own. */
    __syncthreads();
    lds_f32 *val = (lds_f32 *)lds + wave * MP * 64;
#pragma unroll
    for (int pb = 0; pb < P; ++pb)
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int j = 0; j < 4; ++j) val[(16 * pb + 4 * kc + j) * 64 + 16 * g + n] = acc[pb][g][j];
    if (!active) return;
    pf_finish<MP>(p, w, lane, val, npos);
}

/* ---- dequantisation kernel --------------------------------------------------
 * One wave per (tile, unit); lane = row. Rows outside [first, first+count)
 * and blocks past K are skipped. */
template <int FMT>
__global__ void __launch_bounds__(64)
dequant_kernel(const uint8_t *__restrict__ w, float *__restrict__ out, int rows, int cols,
               int units, int first_row, int row_count)
{
    using Unit = typename UnitOf<FMT>::T;
    constexpr int SLAB = UnitOf<FMT>::kBytes * 64;
    constexpr int UW = UnitOf<FMT>::kWeights;
    const int lane = threadIdx.x;
    const int tile = blockIdx.y + first_row / 64;
    const int unit = blockIdx.x;
    const int row = tile * 64 + lane;
    Unit u;
    load_unit(u, w + ((size_t)tile * units + unit) * SLAB, lane);
    if (row < first_row || row >= first_row + row_count || row >= rows) return;
    float *dst = out + (size_t)(row - first_row) * cols + (size_t)unit * UW;
    const int kleft = cols - unit * UW;
    const UnitScales<FMT> s = unit_scales<FMT>(u);
#pragma unroll
    for (int r = 0; r < RegionCount<FMT>::value; ++r) {
        float w[8];
        region_w<FMT, true>(u, s, r, w, 0.0f);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int k = region_k<FMT>(r, i);
            if (UW == 256 || k < kleft) dst[k] = w[i];
        }
    }
}

/* ---- embedding-row gather -----------------------------------------------------
 * out[i * cols + k] = row ids[i] of the tensor, decoded exactly like
 * dequant_kernel (bit-identical to the block decoders). One lane per
 * (position i, K-unit); the row's bytes of a unit sit at lane id % 64 of its
 * slab. An id outside [0, rows) fills its output row with NaN (ids live in
 * device memory, so the host cannot check them) and, when status is given
 * (set to 1 beforehand), clears status[0], so the caller can fail as the
 * reference does for such a token. */
template <int FMT>
__global__ void __launch_bounds__(64)
gather_rows_kernel(const uint8_t *__restrict__ w, const int *__restrict__ ids, float *__restrict__ out, int rows,
                   int cols, int units, int *__restrict__ status)
{
    using Unit = typename UnitOf<FMT>::T;
    constexpr int SLAB = UnitOf<FMT>::kBytes * 64;
    constexpr int UW = UnitOf<FMT>::kWeights;
    const int i = blockIdx.y;
    const int unit = blockIdx.x * 64 + threadIdx.x;
    if (unit >= units) return;
    const int id = ids[i];
    float *dst = out + (size_t)i * cols + (size_t)unit * UW;
    const int kleft = cols - unit * UW;
    if (id < 0 || id >= rows) {
        for (int k = 0; k < UW && k < kleft; ++k) dst[k] = __builtin_nanf("");
        if (status != nullptr && unit == 0) status[0] = 0;
        return;
    }
    Unit u;
    load_unit(u, w + ((size_t)(id >> 6) * units + unit) * SLAB, id & 63);
    const UnitScales<FMT> s = unit_scales<FMT>(u);
#pragma unroll
    for (int r = 0; r < RegionCount<FMT>::value; ++r) {
        float v[8];
        region_w<FMT, true>(u, s, r, v, 0.0f);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int k = region_k<FMT>(r, e);
            if (UW == 256 || k < kleft) dst[k] = v[e];
        }
    }
}

/* ---- upload repack ----------------------------------------------------------
 * Thread per (tile, unit, lane, block-in-unit): copies one packed block from
 * the row-major GGUF bytes into its planes. */
__device__ __forceinline__ size_t plane_offset(int fmt, int lane, int j, int i)
{
    switch (fmt) {
    case QMV_FMT_Q4_K:
        return (size_t)(i >> 4) * 1024 + lane * 16 + (i & 15);
    case QMV_FMT_Q6_K:
        return i < 208 ? (size_t)(i >> 4) * 1024 + lane * 16 + (i & 15) : 13312 + lane * 2 + (i - 208);
    case QMV_FMT_Q8_0:
        return i < 2 ? 8192 + lane * 8 + 2 * j + i
                     : (size_t)(2 * j + ((i - 2) >> 4)) * 1024 + lane * 16 + ((i - 2) & 15);
    default: /* Q5_0 */
        return i < 2 ? 5120 + lane * 8 + 2 * j + i
             : i < 6 ? 4096 + lane * 16 + 4 * j + (i - 2)
                     : (size_t)j * 1024 + lane * 16 + (i - 6);
    }
}

__global__ void repack_kernel(const uint8_t *__restrict__ raw, uint8_t *__restrict__ out, int fmt,
                              int rows, int blocks_per_row, int units, int blocks_per_unit,
                              int block_bytes, int unit_bytes, long long total)
{
    const long long id = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= total) return;
    const int j = (int)(id % blocks_per_unit);
    const long long r1 = id / blocks_per_unit;
    const int lane = (int)(r1 & 63);
    const long long r2 = r1 >> 6;
    const int unit = (int)(r2 % units);
    const long long tile = r2 / units;
    const long long row = tile * 64 + lane;
    const long long blk = (long long)unit * blocks_per_unit + j;
    if (row >= rows || blk >= blocks_per_row) return;
    const uint8_t *src = raw + (row * blocks_per_row + blk) * block_bytes;
    uint8_t *slab = out + (tile * units + unit) * (size_t)unit_bytes * 64;
    for (int i = 0; i < block_bytes; ++i) slab[plane_offset(fmt, lane, j, i)] = src[i];
}

/* ---- greedy argmax ----------------------------------------------------------
 * Stage 1: each workgroup reduces a chunk to (max, lowest index) and counts
 * non-finite values; stage 2: one workgroup combines in chunk order. */

__global__ void __launch_bounds__(256)
argmax_stage1(const float *__restrict__ logits, int n, float *__restrict__ bval, int *__restrict__ bidx,
              int *__restrict__ bbad)
{
    __shared__ float sv[256];
    __shared__ int si[256];
    __shared__ int sbad[256];
    const int chunk = (n + gridDim.x - 1) / gridDim.x;
    const int begin = blockIdx.x * chunk;
    const int end = min(begin + chunk, n);
    float best = -INFINITY;
    int besti = 0x7fffffff;
    int bad = 0;
    for (int i = begin + threadIdx.x; i < end; i += blockDim.x) {
        const float v = logits[i];
        if (!isfinite(v)) { bad = 1; continue; }
        argmax_merge(best, besti, v, i);
    }
    sv[threadIdx.x] = best;
    si[threadIdx.x] = besti;
    sbad[threadIdx.x] = bad;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) {
            float v = sv[threadIdx.x];
            int i = si[threadIdx.x];
            argmax_merge(v, i, sv[threadIdx.x + s], si[threadIdx.x + s]);
            sv[threadIdx.x] = v;
            si[threadIdx.x] = i;
            sbad[threadIdx.x] |= sbad[threadIdx.x + s];
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        bval[blockIdx.x] = sv[0];
        bidx[blockIdx.x] = si[0];
        bbad[blockIdx.x] = sbad[0];
    }
}

__global__ void __launch_bounds__(64)
argmax_stage2(const float *__restrict__ bval, const int *__restrict__ bidx, const int *__restrict__ bbad,
              int nblocks, int *__restrict__ result)
{
    if (threadIdx.x != 0) return;
    float best = -INFINITY;
    int besti = 0x7fffffff;
    int bad = 0;
    for (int b = 0; b < nblocks; ++b) {
        bad |= bbad[b];
        argmax_merge(best, besti, bval[b], bidx[b]);
    }
    result[0] = bad || besti == 0x7fffffff ? -1 : besti;
    result[1] = bad ? 0 : 1;
}

/* RMSNorm (tensor_rms_norm_f32, src/tensor.cpp:99-136) of one vector per
 * workgroup: out = (x / sqrt(mean(x^2) + eps)) * w. A decode-step vector
 * (3584 floats) is one 16-byte load per thread, held in registers from the
 * sum of squares to the output, so the kernel costs one load round, one
 * reduction and one store round. The sum of squares runs in a fixed order
 * (each thread's elements in index order, a butterfly within the wave, then
 * the wave sums in wave order), so results are deterministic; the division
 * and square root are IEEE-rounded. Each element is read and written by
 * one thread only (the one whose stride covers it), so out may be x itself. */
#define QMV_NORM_THREADS 1024
#define QMV_NORM_REGS 2 /* 16-byte words per thread kept in registers */
__global__ void __launch_bounds__(QMV_NORM_THREADS)
rms_norm_kernel(const float *x, const float *__restrict__ w, int n, float eps, float *out)
{
    const float *xv = x + (size_t)blockIdx.x * n;
    float *ov = out + (size_t)blockIdx.x * n;
    const int tid = threadIdx.x;
    /* 16-byte path when every row start is 16-byte aligned. */
    const bool vec = (n & 3) == 0 && (((uintptr_t)x | (uintptr_t)w | (uintptr_t)out) & 15) == 0;
    const int n4 = vec ? n >> 2 : 0;
    float4 r[QMV_NORM_REGS];
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < QMV_NORM_REGS; ++j) {
        const int i = tid + j * QMV_NORM_THREADS;
        r[j] = i < n4 ? reinterpret_cast<const float4 *>(xv)[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
#pragma unroll
    for (int j = 0; j < QMV_NORM_REGS; ++j) {
        s += r[j].x * r[j].x;
        s += r[j].y * r[j].y;
        s += r[j].z * r[j].z;
        s += r[j].w * r[j].w;
    }
    for (int i = tid + QMV_NORM_REGS * QMV_NORM_THREADS; i < n4; i += QMV_NORM_THREADS) {
        const float4 v = reinterpret_cast<const float4 *>(xv)[i];
        s += v.x * v.x;
        s += v.y * v.y;
        s += v.z * v.z;
        s += v.w * v.w;
    }
    if (!vec)
        for (int i = tid; i < n; i += QMV_NORM_THREADS) s += xv[i] * xv[i];
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o);
    __shared__ float wave_sum[QMV_NORM_THREADS / 64];
    if ((tid & 63) == 0) wave_sum[tid >> 6] = s;
    __syncthreads();
    float total = wave_sum[0];
#pragma unroll
    for (int v = 1; v < QMV_NORM_THREADS / 64; ++v) total += wave_sum[v];
    const float denom = sqrtf(total / (float)n + eps);
    if (vec) {
#pragma unroll
        for (int j = 0; j < QMV_NORM_REGS; ++j) {
            const int i = tid + j * QMV_NORM_THREADS;
            if (i < n4) {
                const float4 g = reinterpret_cast<const float4 *>(w)[i];
                reinterpret_cast<float4 *>(ov)[i] = make_float4((r[j].x / denom) * g.x, (r[j].y / denom) * g.y,
                                                                (r[j].z / denom) * g.z, (r[j].w / denom) * g.w);
            }
        }
        for (int i = tid + QMV_NORM_REGS * QMV_NORM_THREADS; i < n4; i += QMV_NORM_THREADS) {
            const float4 v = reinterpret_cast<const float4 *>(xv)[i];
            const float4 g = reinterpret_cast<const float4 *>(w)[i];
            reinterpret_cast<float4 *>(ov)[i] =
                make_float4((v.x / denom) * g.x, (v.y / denom) * g.y, (v.z / denom) * g.z, (v.w / denom) * g.w);
        }
    } else {
        for (int i = tid; i < n; i += QMV_NORM_THREADS) ov[i] = (xv[i] / denom) * w[i];
    }
}

/* ---- row-major single-position kernel (Q4_K) ---------------------------------
 * For launches too small to fill the chip with 64-row tiles unless K is split
 * across workgroups (whose publish / count / reload tail then dominates), a
 * workgroup owns R whole rows instead, so no row is split across workgroups.
 * It reads the GGUF row-major bytes directly: a Q4_K row is sb super-blocks of
 * 144 bytes, a 16-byte header (d, dmin, 12 scale bytes) then 8 qs planes of 16
 * bytes, all 16-byte aligned. Lane item i of a row is (super-block i / 8, plane
 * i % 8): one 16-byte qs load plus the super-block's header (the same address
 * for the 8 lanes of a super-block, one cache line). Item (s, p), g = p / 2,
 * h = p % 2, holds weights 256s + 64g + 16h + [0, 16) in its low nibbles
 * (sub-block 2g) and 256s + 64g + 32 + 16h + [0, 16) in its high nibbles
 * (sub-block 2g + 1), so each lane keeps those 32 activations in registers
 * and reuses them for its R rows; J items per lane cover rows of up to
 * 8 * 64 * J / 8 super-blocks. A row's lane sums are added with DPP inside
 * each wave, then across the workgroup's waves in wave order, so results are
 * run-to-run identical. */

/* v plus the value DPP control CTRL brings to each lane (all lanes active). */
template <int CTRL>
__device__ __forceinline__ float dpp_plus(float v)
{
    return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

/* Accumulate the 4 low-nibble codes of dword dw (bytes 0..3) against
 * xlo[0..3] into l and the 4 high-nibble codes (as 16q) against xhi[0..3]
 * into h, in byte order, on sums scaled by 2^-24 (f16lo above). */
__device__ __forceinline__ void q4_dword_mix2(uint32_t dw, const float *xlo, const float *xhi, float &l, float &h)
{
    const uint32_t s = dw >> 8;
    const uint32_t le = dw & 0x000f000fu, lo = s & 0x000f000fu; /* bytes 0,2 | 1,3 */
    const uint32_t he = dw & 0x00f000f0u, ho = s & 0x00f000f0u;
    l = fmaf(f16lo(le), xlo[0], l);
    l = fmaf(f16lo(lo), xlo[1], l);
    l = fmaf(f16hi(le), xlo[2], l);
    l = fmaf(f16hi(lo), xlo[3], l);
    h = fmaf(f16lo(he), xhi[0], h);
    h = fmaf(f16lo(ho), xhi[1], h);
    h = fmaf(f16hi(he), xhi[2], h);
    h = fmaf(f16hi(ho), xhi[3], h);
}

/* xv[0] + xv[1] + ... + xv[15], in that order. */
__device__ __forceinline__ float quarter_sum(const float *xv)
{
    float t = xv[0];
#pragma unroll
    for (int e = 1; e < 16; ++e) t += xv[e];
    return t;
}

/* Workgroup barrier for data exchanged through LDS only: waits for this
 * wave's LDS operations, not for its global loads (a fenced __syncthreads
 * would also wait for the weight loads still in flight). The empty asm keeps
 * the compiler from moving memory accesses across it. */
__device__ __forceinline__ void lds_barrier()
{
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F); /* lgkmcnt(0); vmcnt, expcnt not waited */
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

/* Sum of v over each SEG-lane segment of the wave (SEG = 16, 32 or 64), as a
 * wave-uniform value per segment: DPP inside the 16-lane rows, then the rows
 * of a segment by readlane in a fixed order. Every lane must be active. */
template <int SEG>
__device__ __forceinline__ void segment_totals(float v, float (&out)[64 / SEG])
{
    v = dpp_plus<0xB1>(v);  /* quad_perm [1,0,3,2] */
    v = dpp_plus<0x4E>(v);  /* quad_perm [2,3,0,1] */
    v = dpp_plus<0x141>(v); /* row_half_mirror */
    v = dpp_plus<0x140>(v); /* row_mirror */
    if constexpr (SEG == 64) {
        out[0] = (lane_value(v, 0) + lane_value(v, 16)) + (lane_value(v, 32) + lane_value(v, 48));
    } else if constexpr (SEG == 32) {
        out[0] = lane_value(v, 0) + lane_value(v, 16);
        out[1] = lane_value(v, 32) + lane_value(v, 48);
    } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) out[k] = lane_value(v, 16 * k);
    }
}

/* Row-major Q4_K matvec at one position, one 64-weight group per lane.
 *
 * Lane item i of a row is group g = i & 3 of super-block s = i >> 2: qs
 * bytes 32g..32g+31 (two 16-byte loads), whose low nibbles are weights
 * 64g + j of the super-block (sub-block 2g) and high nibbles 64g + 32 + j
 * (sub-block 2g + 1), plus the super-block's 16-byte header, read by its 4
 * lanes as one line. A row has 4 sb items; a lane keeps the 64 activations of
 * its item in VGPRs, with their two half sums, for every row it takes.
 *
 * Two modes, chosen by the row length:
 *  - Shared (sb <= 16, workgroups of QMV_ROWGROUP_WAVES waves): a row takes
 *    one segment of SEG lanes (the smallest of 16, 32, 64 that holds its
 *    items), so a wave holds P = 64 / SEG segments; each wave takes R rows
 *    per segment (rows row0 + w * R * P + r * P + segment). The activation
 *    vector is staged once per workgroup in LDS, in an XOR-swizzled layout
 *    that keeps the lanes' 128-bit reads free of bank conflicts, and every
 *    wave reads its items from there.
 *  - Split (sb > 16, SEG = 64): a row spans the workgroup's waves, which read
 *    their own activations and add their sums in LDS in wave order.
 * Every weight load is issued before any arithmetic; in shared mode the
 * activation loads go first, so waiting for them leaves the weight loads in
 * flight.
 *
 * EPI: QMV_ROWDOT_STORE (y = sum, plus `add` if set), QMV_ROWDOT_SWIGLU
 * (jobs 0 = gate and 1 = up over the same rows: row slots R..2R-1 are job 1's
 * rows, and job 0's y gets up * silu(gate), so the fused result is that of
 * the plain launches' sums bit for bit), QMV_ROWDOT_ARGMAX (one job; y
 * stored, then the greedy argmax of y with one candidate tile per
 * workgroup). Lane i < R * P of a wave emits the wave's row i. Row sums run
 * in a fixed order (DPP within 16 lanes, the 16-lane rows by readlane, waves
 * through LDS in wave order), so repeated launches are bit-identical.
 *
 * NORM (shared mode): the input is first normalised as tensor_rms_norm_f32
 * (src/tensor.cpp:99-136) does, h = (x / denom) * w with denom =
 * sqrt(sum(x^2) / K + eps). The norm weights are staged beside x; each lane
 * multiplies its item's activations by them and sums their squares, and the
 * segment adds the lanes' sums in a fixed order that every wave of the launch
 * repeats (so all find the same denom); each row's sum is divided by denom
 * before its epilogue:
 * sum(W (x * w)) / denom, which differs from the reference's
 * sum(W ((x / denom) * w)) only in rounding. */
typedef void __attribute__((address_space(3))) lds_void;

template <int R, int SEG, int EPI, bool SPLIT, bool NORM = false>
__global__ void __launch_bounds__(QMV_MAX_WAVES * 64) rowgroup_q4k_kernel(RowdotParams p)
{
    static_assert(!SPLIT || SEG == 64, "rows that span waves take whole waves");
    static_assert(!NORM || (!SPLIT && EPI != QMV_ROWDOT_ARGMAX), "the fused norm runs in shared mode, store or SwiGLU");
    constexpr int P = 64 / SEG;
    constexpr int RS = EPI == QMV_ROWDOT_SWIGLU ? 2 * R : R;
    constexpr int XW = QMV_ROWGROUP_WAVES;
    constexpr bool split = SPLIT;
    __shared__ float red[QMV_MAX_WAVES][RS];
    /* Shared mode: 64 items x 16 float4 of activations, then (NORM) the norm
     * weights in the same layout, 16 KiB further. */
    __shared__ float4 xsh[split ? 1 : (NORM ? 2 : 1) * 64 * 16];
    float4 *const wsh = xsh + 64 * 16;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), nw = blockDim.x >> 6;
    /* The job: the last one whose workgroups start at or before this one
     * (starts ascend; launch_rowgroup sets those of unused job slots past
     * every workgroup). Every start is read in one batch of scalar loads with
     * the other arguments the first loads need; the chosen job's fields then
     * come from lines that batch brought into the scalar cache. */
    const int bid = (int)blockIdx.x;
    const uint8_t *jw = p.job[0].w, *const jw1 = p.job[1].w;
    int jrows = p.job[0].rows, jbegin = 0, j = 0;
    const int jrows1 = p.job[1].rows, sb = p.sb;
    const float *const xp = p.x;
    const float *const normw = p.norm_w;
    if constexpr (EPI == QMV_ROWDOT_STORE) {
        int begin[QMV_MAX_JOBS];
#pragma unroll
        for (int i = 1; i < QMV_MAX_JOBS; ++i) begin[i] = p.job[i].wg_begin;
        __builtin_amdgcn_sched_barrier(0); /* the loads above go out together */
#pragma unroll
        for (int i = 1; i < QMV_MAX_JOBS; ++i) j = bid >= begin[i] ? i : j;
        jw = p.job[j].w;
        jrows = p.job[j].rows;
        jbegin = p.job[j].wg_begin;
    } else {
        __builtin_amdgcn_sched_barrier(0); /* the loads above go out together */
    }
    const int local = bid - jbegin;
    const int row0 = split ? local * R : (local * XW + wave) * (R * P);
    const int seg = P > 1 ? lane / SEG : 0;
    const int items = 4 * sb;
    const int it0 = split ? wave * 64 + lane : (lane & (SEG - 1));
    const bool ok = it0 < items;
    /* Lanes past the row's items repeat its last item (in-bounds loads) and
     * drop their sums before the reduction. */
    const int it = min(it0, items - 1);
    const int s = it >> 2, g = it & 3;
    const size_t row_bytes = (size_t)sb * 144;

    /* Shared mode: the activation vector goes straight from memory into LDS
     * (global_load_lds, no VGPRs). Item i's 16 float4 occupy slots 16i..16i+15
     * with float4 c in slot 16i + (c ^ (i & 15)): load j of the workgroup
     * fills items 4j..4j+3 (wave w issues loads j = XW * k + w), each group
     * of 16 lanes reading one item's 256 contiguous bytes in a permuted order,
     * and each lane's 16 reads below hit 16 different slots of every 16
     * consecutive items, so no two lanes of a 16-lane group share a bank.
     * Lanes past the row's items copy its last item into slots nobody reads. */
    constexpr int XS = 16 / XW;
    if constexpr (!split) {
#pragma unroll
        for (int k = 0; k < XS; ++k) {
            const int jl = XW * k + wave;
            const int item = 4 * jl + (lane >> 4);
            const int c = (lane & 15) ^ (item & 15);
            const float4 *src = (const float4 *)xp + (size_t)min(item, items - 1) * 16 + c;
            __builtin_amdgcn_global_load_lds((const void *)src, (lds_void *)(xsh + 64 * jl), 16, 0, 0);
        }
        if constexpr (NORM) {
#pragma unroll
            for (int k = 0; k < XS; ++k) {
                const int jl = XW * k + wave;
                const int item = 4 * jl + (lane >> 4);
                const int c = (lane & 15) ^ (item & 15);
                const float4 *src = (const float4 *)normw + (size_t)min(item, items - 1) * 16 + c;
                __builtin_amdgcn_global_load_lds((const void *)src, (lds_void *)(wsh + 64 * jl), 16, 0, 0);
            }
        }
    }
    /* Issue order: activations, then weights; the wait for the activations
     * then leaves the weight loads in flight. */
    __builtin_amdgcn_sched_barrier(0);

    const int qoff = 144 * s + 16 + 32 * g, hoff = 144 * s;
    uint4 qa[RS], qb[RS], hd[RS];
#pragma unroll
    for (int r = 0; r < RS; ++r) {
        const uint8_t *base = (r < R ? jw : jw1) + (size_t)min(row0 + (r % R) * P + seg, (r < R ? jrows : jrows1) - 1) * row_bytes;
        qa[r] = ld16(base + qoff);
        qb[r] = ld16(base + qoff + 16);
        hd[r] = ld16(base + hoff);
    }
    __builtin_amdgcn_sched_barrier(0);

    float xv[64];
    float norm_total = 0.0f; /* NORM: the vector's sum of squares */
    if constexpr (split) {
        const float *xs = xp + 256 * s + 64 * g;
#pragma unroll
        for (int c = 0; c < 16; ++c) {
            const float4 v = *(const float4 *)(xs + 4 * c);
            xv[4 * c] = v.x;
            xv[4 * c + 1] = v.y;
            xv[4 * c + 2] = v.z;
            xv[4 * c + 3] = v.w;
        }
    } else {
        /* This wave's activation loads (issued first) have landed once at most
         * the 3 * RS weight loads issued after them are outstanding; then every
         * wave's have, after the barrier. */
        constexpr int VM = 3 * RS;
        static_assert(VM < 64, "vmcnt field");
        __builtin_amdgcn_s_waitcnt((VM & 15) | ((VM >> 4) << 14) | (7 << 4) | (15 << 8));
        /* A plain barrier: LDS is coherent within the workgroup once each
         * wave's loads into it have landed (a fenced __syncthreads would also
         * wait for the weight loads). */
        __builtin_amdgcn_s_barrier();
        /* Slot 16 it + (c ^ (it & 15)) = (16 it + (it & 15)) ^ c, as a byte
         * offset: one XOR per read. */
        const uint32_t off0 = (uint32_t)(16 * it + (it & 15)) * 16u;
        if constexpr (!NORM) {
#pragma unroll
            for (int c = 0; c < 16; ++c) {
                const float4 v = *(const float4 *)((const char *)xsh + (off0 ^ (16u * c)));
                xv[4 * c] = v.x;
                xv[4 * c + 1] = v.y;
                xv[4 * c + 2] = v.z;
                xv[4 * c + 3] = v.w;
            }
        } else {
            /* This item's sum of squares of x, in order, and its activations
             * times the norm weights, four float4 of each at a time (the
             * barriers keep the reads from being hoisted, which would hold
             * 64 more registers). Every segment holds every item of the row,
             * so the segment total below is the whole vector's. */
            float ss = 0.0f;
#pragma unroll
            for (int c4 = 0; c4 < 16; c4 += 4) {
#pragma unroll
                for (int c = c4; c < c4 + 4; ++c) {
                    const char *const slot = (const char *)xsh + (off0 ^ (16u * c));
                    const float4 v = *(const float4 *)slot;
                    const float4 wv = *(const float4 *)(slot + 64 * 16 * 16);
                    ss = fmaf(v.x, v.x, ss);
                    ss = fmaf(v.y, v.y, ss);
                    ss = fmaf(v.z, v.z, ss);
                    ss = fmaf(v.w, v.w, ss);
                    xv[4 * c] = v.x * wv.x;
                    xv[4 * c + 1] = v.y * wv.y;
                    xv[4 * c + 2] = v.z * wv.z;
                    xv[4 * c + 3] = v.w * wv.w;
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            float tot_ss[P];
            segment_totals<SEG>(ok ? ss : 0.0f, tot_ss);
            norm_total = tot_ss[0];
        }
    }
    /* Every load is issued before any arithmetic waits for one. */
    __builtin_amdgcn_sched_barrier(0);

    /* Quarter sums of the item's activations, xq[c] over xv[16c..16c+15] in
     * order. Shared mode: wave c of the workgroup (whose lanes hold the same
     * items) sums quarter c alone and the waves exchange them through LDS. */
    float xq[4];
    if constexpr (split) {
#pragma unroll
        for (int c = 0; c < 4; ++c) xq[c] = quarter_sum(xv + 16 * c);
    } else {
        static_assert(XW % 4 == 0, "whole sets of four quarters");
        __shared__ float xqs[4][64];
        const int qw = wave & 3;
        const float t = qw == 0   ? quarter_sum(xv)
                        : qw == 1 ? quarter_sum(xv + 16)
                        : qw == 2 ? quarter_sum(xv + 32)
                                  : quarter_sum(xv + 48);
        if (wave < 4) xqs[qw][lane] = t;
        lds_barrier();
#pragma unroll
        for (int c = 0; c < 4; ++c) xq[c] = xqs[c][lane];
    }
    const float xl = xq[0] + xq[1], xh = xq[2] + xq[3];
    /* Scale/min bytes of sub-blocks 2g, 2g + 1 (header dwords y = bytes
     * 4..7, z = 8..11, w = 12..15 of the super-block): byte pair 2(g & 1)
     * of the dwords; for g >= 2 the 6-bit values are assembled from w's
     * nibbles and the top 2 bits of y (scales) or z (minimums). */
    const int sh = (g & 1) * 16;
    const int shyz = sh + (g >= 2 ? 2 : 0);
    const uint32_t nib = g >= 2 ? 0x0f0fu : 0u;

    float tot[RS][P];
#pragma unroll
    for (int r = 0; r < RS; ++r) {
        /* low / high code sums scaled by 2^-24 (q4_dword_mix2) */
        float l = 0.0f, hs = 0.0f;
#pragma unroll
        for (int e = 0; e < 4; ++e) q4_dword_mix2(word(qa[r], e), xv + 4 * e, xv + 32 + 4 * e, l, hs);
#pragma unroll
        for (int e = 0; e < 4; ++e) q4_dword_mix2(word(qb[r], e), xv + 16 + 4 * e, xv + 48 + 4 * e, l, hs);
        const uint4 h = hd[r];
        const uint32_t sc = (((h.w >> sh) & nib) | ((h.y >> shyz) & ~nib)) & 0x3f3fu;
        const uint32_t mn = (((h.w >> (sh + 4)) & nib) | ((h.z >> shyz) & ~nib)) & 0x3f3fu;
        const float d24 = f16_bits_to_f32(h.x) * 16777216.0f, dmin = f16_bits_to_f32(h.x >> 16);
        /* d * 2^24 * (sc_a * L + sc_b * H / 16) - dmin * (m_a * xl + m_b * xh) */
        float u = ubyte(sc, 0) * l;
        u = fmaf(ubyte(sc, 1), hs * 0.0625f, u);
        float v = ubyte(mn, 0) * xl;
        v = fmaf(ubyte(mn, 1), xh, v);
        float c = d24 * u;
        c = fmaf(-dmin, v, c);
        segment_totals<SEG>(ok ? c : 0.0f, tot[r]);
    }

    if constexpr (split) {
        if (lane == 0) {
#pragma unroll
            for (int r = 0; r < RS; ++r) red[wave][r] = tot[r][0];
        }
        __syncthreads();
        if (wave != 0) return;
#pragma unroll
        for (int r = 0; r < RS; ++r) {
            float t = red[0][r];
            for (int w = 1; w < nw; ++w) t += red[w][r];
            tot[r][0] = t;
        }
    }
    float denom = 1.0f;
    if constexpr (NORM) denom = sqrtf(norm_total / (float)(256 * sb) + p.norm_eps);
    /* Lane i = r * P + segment emits row row0 + i. */
    float out = tot[0][0], up = tot[RS > R ? R : 0][0];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int q = 0; q < P; ++q)
            if (lane == r * P + q) {
                out = tot[r][q];
                if constexpr (EPI == QMV_ROWDOT_SWIGLU) up = tot[R + r][q];
            }
    const int row = row0 + lane;
    const RowdotJob &job = p.job[j];
    const bool valid = lane < R * P && row < jrows;
    if constexpr (NORM) {
        out /= denom;
        up /= denom;
    }
    if constexpr (EPI == QMV_ROWDOT_SWIGLU) {
        if (valid) {
            if (job.add != nullptr) out += job.add[row];
            if (p.job[1].add != nullptr) up += p.job[1].add[row];
            job.y[row] = swiglu_value(out, up);
        }
    } else {
        if (valid) {
            if (job.add != nullptr) out += job.add[row];
            job.y[row] = out;
        }
        if constexpr (EPI == QMV_ROWDOT_ARGMAX) {
            if constexpr (split) {
                tile_argmax(p, (int)blockIdx.x, valid, row, out, lane);
            } else {
                /* One candidate per workgroup: the waves' candidates meet in
                 * LDS and wave 0 publishes their merge. */
                __shared__ uint64_t wcand[XW];
                float v;
                int i, bad;
                wave_candidate(valid, row, out, v, i, bad);
                if (lane == 0) wcand[wave] = pack_candidate(v, i, bad);
                __syncthreads();
                if (wave != 0) return;
                float bv = -INFINITY;
                int bi = 0x7fffffff, bb = 0;
#pragma unroll
                for (int w = 0; w < XW; ++w) {
                    const uint64_t c = wcand[w];
                    const uint32_t hi = (uint32_t)(c >> 32);
                    bb |= (int)(hi >> 31);
                    argmax_merge(bv, bi, __uint_as_float((uint32_t)c), (int)(hi & 0x7fffffffu));
                }
                publish_tile_candidate(p, (int)blockIdx.x, bv, bi, bb, lane);
            }
        }
    }
}

/* ---- row-major Q6_K at one position ------------------------------------------
 * A Q6_K row of sb super-blocks is kept as chunks of 16 super-blocks (the
 * last one m = sb - 16 (ceil(sb / 16) - 1)), chunk c at 3360 c (16 x 210
 * bytes), each in five planes (rowmajor_q6k_kernel writes them from the GGUF
 * row; q6k_row_stride(sb) bytes per row, 210 sb rounded up to 16):
 *   A at 0        64 bytes per super-block: ql[0..31], ql[64..95]
 *   B at 64 m     ql[32..63], ql[96..127]
 *   H at 128 m    qh[0..63]
 *   S at 192 m    16 scale bytes per super-block, reordered (below)
 *   D at 208 m    the super-block's f16 d
 * Item i = 4s + q of a chunk (local super-block s, q = 0..3, half n = q / 2,
 * l0 = 16 (q % 2)) is the 64 weights 128n + l0 + 32k + [0, 16), k = 0..3,
 * of that super-block: bytes 16i..16i+15 of A (low nibbles k = 0, high
 * nibbles k = 2), of B (k = 1, 3) and of H (bits 2k..2k+1 for run k), and
 * the four scales of its sub-blocks 8n + q % 2 + 2k as the bytes k of dword
 * i of S. A weight's code is low | high << 4, its value (code - 32) * d *
 * scale, as the GGUF block defines it (ql[l] low nibble: weight l of the
 * half, ql[l] high: 64 + l, ql[32 + l]: 32 + l and 96 + l, qh[l] bits 0-1,
 * 2-3, 4-5, 6-7: weights l, 32 + l, 64 + l, 96 + l). A wave reads a chunk's
 * planes with consecutive lanes at consecutive addresses, 3360 contiguous
 * bytes per chunk. */

/* Thread per byte of a GGUF super-block: its place in the planes. */
__global__ void rowmajor_q6k_kernel(const uint8_t *__restrict__ raw, uint8_t *__restrict__ out, int sb,
                                    long long total)
{
    const long long id = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= total) return;
    const int i = (int)(id % 210);
    const long long blk = id / 210; /* row * sb + s */
    const int sg = (int)(blk % sb);
    const long long row = blk / sb;
    /* chunk c = sg / 16 of m super-blocks, local super-block s */
    const int c = sg >> 4, s = sg & 15, m = min(16, sb - 16 * c);
    size_t off = (size_t)3360 * c;
    if (i < 128) { /* ql: plane A (w < 32) or B, item 2n + (w / 16) % 2 */
        const int n = i >> 6, w = i & 63;
        off += (w >> 5) * 64 * m + 64 * s + 16 * (2 * n + ((w >> 4) & 1)) + (w & 15);
    } else if (i < 192) { /* qh in order */
        off += 128 * m + 64 * s + (i - 128);
    } else if (i < 208) { /* scale of sub-block t = 8n + 2k + odd -> item 2n + odd, byte k */
        const int t = i - 192, n = t >> 3, odd = t & 1, k = (t & 7) >> 1;
        off += 192 * m + 16 * s + 4 * (2 * n + odd) + k;
    } else {
        off += 208 * m + 2 * s + (i - 208);
    }
    out[row * q6k_row_stride(sb) + off] = raw[blk * 210 + i];
}

/* Row-major Q6_K matvec at one position (rows of more than 16 super-blocks).
 * Each wave computes whole rows: a row is NSL = ceil(sb / 16) slices of up
 * to 16 super-blocks (the row's contiguous plane chunks), one 64-weight item
 * per lane and slice, and the wave takes the slices in turn, loading the next
 * slice's weights before it computes the current one; the lane's sums over
 * its slices are added by DPP, so a row's result is the same in any launch.
 * Workgroup b takes rows b * W .. b * W + W - 1 of the launch (W waves, one
 * row each; the launch's rows are its jobs' rows in job order). The
 * workgroup first copies the activations, straight from memory, into LDS
 * (global_load_lds, 1 KiB contiguous per instruction, 16 KiB per slice),
 * and the four run sums of every slice item into LDS beside them; a lane
 * then reads its item's 64 activations (16 ds_read_b128) and run sums for
 * each slice. EPI: QMV_ROWDOT_STORE (y = sum, plus `add` if set),
 * QMV_ROWDOT_SWIGLU (a wave takes gate row r of job 0, then up row r of job
 * 1, and job 0's y gets up * silu(gate): the plain launch's sums bit for
 * bit), QMV_ROWDOT_ARGMAX (one job; y stored, then the greedy argmax of y
 * with one candidate per workgroup).
 *
 * LDS layout of a slice: 16-byte chunk g of its activations (g = 64 s' +
 * 32 n + 8 k + 4 h + c for local super-block s', half n, run k, item half
 * h = q % 2 and float4 c of the run) sits in slot g ^ m(g), m(g) = bit 5 of
 * g to bit 0, bit 6 to bit 1, bit 7 to bit 3. A read (k, c) of the 16 lanes
 * of a 16-lane group (4 super-blocks x 4 items) then lands on 16 different
 * slots mod 16 (bits 0..3 = c0 ^ n, c1 ^ s'0, h, k0 ^ s'1), so no two of
 * them share a bank. The copy writes slot 64 j + lane of instruction j,
 * reading chunk slot ^ m(slot) (m only reads bits the XOR leaves alone). */
__device__ __forceinline__ int q6k_slot_mix(int g)
{
    return ((g >> 5) & 1) | (((g >> 6) & 1) << 1) | (((g >> 7) & 1) << 3);
}

/* One lane's item of one slice of a row: A, B and H plane pieces, scale
 * dword, d. */
struct Q6Item {
    uint4 a, b, h;
    uint32_t sc, dd;
};

/* Slice j's item of lane it (< 4 m) in the row at `row`: the chunk holds m
 * super-blocks. */
__device__ __forceinline__ Q6Item q6k_load_item(gu8 *row, int j, int m, int it)
{
    gu8 *base = row + 3360 * j;
    Q6Item w;
    w.a = gload16(base + 16 * it);
    w.b = gload16(base + 64 * m + 16 * it);
    w.h = gload16(base + 128 * m + 16 * it);
    w.sc = *(gu32 *)(base + 192 * m + 4 * it);
    w.dd = *(gu16 *)(base + 208 * m + 2 * (it >> 2));
    return w;
}

/* The item's lane sum: d * sum_k scale_k * (sum(code x) - 32 sum(x)) over
 * its four runs (xq: their sums). */
__device__ __forceinline__ float q6k_item_sum(const Q6Item &w, const float *xv, float4 xq)
{
    /* run sums of code * x, scaled by 2^-24 (byte_codes_mix) */
    float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const uint32_t aw = word(w.a, e), bw = word(w.b, e), hw = word(w.h, e);
        const uint32_t q0 = codes((aw & 0x0f0f0f0fu) | ((hw << 4) & 0x30303030u));
        const uint32_t q1 = codes((bw & 0x0f0f0f0fu) | ((hw << 2) & 0x30303030u));
        const uint32_t q2 = codes(((aw >> 4) & 0x0f0f0f0fu) | (hw & 0x30303030u));
        const uint32_t q3 = codes(((bw >> 4) & 0x0f0f0f0fu) | ((hw >> 2) & 0x30303030u));
        s0 = byte_codes_mix(q0, xv + 4 * e, s0);
        s1 = byte_codes_mix(q1, xv + 16 + 4 * e, s1);
        s2 = byte_codes_mix(q2, xv + 32 + 4 * e, s2);
        s3 = byte_codes_mix(q3, xv + 48 + 4 * e, s3);
    }
    /* the offset term scaled by 2^-24 like the sums (32 * 2^-24 = 2^-19,
     * exact) */
    const float k32 = -1.9073486328125e-6f;
    float u = sbyte(w.sc, 0) * fmaf(k32, xq.x, s0);
    u = fmaf(sbyte(w.sc, 1), fmaf(k32, xq.y, s1), u);
    u = fmaf(sbyte(w.sc, 2), fmaf(k32, xq.z, s2), u);
    u = fmaf(sbyte(w.sc, 3), fmaf(k32, xq.w, s3), u);
    return f16_bits_to_f32(w.dd) * 16777216.0f * u;
}

/* Lane item `it`'s 64 activations of a slice region (the layout above). */
__device__ __forceinline__ void q6k_slice_x(const float4 *region, int it, float (&xv)[64])
{
    const int s = it >> 2, q = it & 3;
    const int gbase = 64 * s + 32 * (q >> 1) + 4 * (q & 1);
    /* slot (base | mix) ^ (8k + c): base and 8k + c share no bits */
    const uint32_t off1 = (uint32_t)(gbase | q6k_slot_mix(gbase)) * 16u;
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const float4 v = *(const float4 *)((const char *)region + (off1 ^ (16u * (8 * k + c))));
            xv[16 * k + 4 * c] = v.x;
            xv[16 * k + 4 * c + 1] = v.y;
            xv[16 * k + 4 * c + 2] = v.z;
            xv[16 * k + 4 * c + 3] = v.w;
        }
}

/* SwiGLU workgroups hold at most 8 waves: the gate and up rows' sums then
 * fit their registers (16-wave workgroups leave 128 per lane and spilled). */
#define QMV_ROWLOOP_MAX_WAVES(EPI) ((EPI) == QMV_ROWDOT_SWIGLU ? 8 : 16)

template <int NSL, int PD, int EPI>
__global__ void __launch_bounds__(QMV_ROWLOOP_MAX_WAVES(EPI) * 64) rowloop_q6k_kernel(RowdotParams p)
{
    /* NSL slices of 1024 float4 (activations), then NSL x 64 float4 (run
     * sums of each slice's items) */
    extern __shared__ float4 q6k_xsh[];
    float4 *const xqs = q6k_xsh + 1024 * NSL;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), nw = blockDim.x >> 6;
    const int sb = p.sb;
    const float *const xp = p.x;
    /* Job starts (first rows; unused slots start past every row), in one
     * batch of scalar loads. */
    int begin[QMV_MAX_JOBS];
#pragma unroll
    for (int i = 1; i < QMV_MAX_JOBS; ++i) begin[i] = p.job[i].wg_begin;
    __builtin_amdgcn_sched_barrier(0);

    /* The activations into LDS: every wave copies its share of every slice
     * (1 KiB pieces k = v, v + nw, ... of slice 0, then of slice 1, ...);
     * chunks past the vector repeat its last chunk. */
    const int last = 64 * sb - 1;
#pragma unroll
    for (int sl = 0; sl < NSL; ++sl) {
        for (int k = wave; k < 16; k += nw) {
            const int slot = 64 * k + lane;
            const int g = min(1024 * sl + (slot ^ q6k_slot_mix(slot)), last);
            __builtin_amdgcn_global_load_lds((const void *)((const float4 *)xp + g),
                                             (lds_void *)(q6k_xsh + 1024 * sl + 64 * k), 16, 0, 0);
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    /* This wave's row (global row index; past the launch's rows the wave
     * only helps with the copies and, for the argmax, the candidates), its
     * job and its first slice's weights. SwiGLU: the row of job 0 (gate),
     * then the same row of job 1 (up). */
    const int grow = (int)blockIdx.x * nw + wave;
    const bool has_row = grow < p.groups;
    int jj = 0;
    if constexpr (EPI == QMV_ROWDOT_STORE) {
#pragma unroll
        for (int i = 1; i < QMV_MAX_JOBS; ++i) jj = grow >= begin[i] ? i : jj;
    }
    const RowdotJob &job = p.job[jj];
    const int row = min(grow - job.wg_begin, job.rows - 1);
    const size_t roff = (size_t)row * q6k_row_stride(sb);
    gu8 *const rowp = (gu8 *)(uint64_t)job.w + roff;
    gu8 *const rowp1 = EPI == QMV_ROWDOT_SWIGLU ? (gu8 *)(uint64_t)p.job[1].w + roff : rowp;
    /* Slice j of a row has m super-blocks; lanes past 4 m repeat its last
     * item. */
    auto slice_m = [&](int j) { return min(16, sb - 16 * j); };
    auto load_slice = [&](gu8 *rp, int j) {
        const int m = slice_m(j);
        return q6k_load_item(rp, j, m, min(lane, 4 * m - 1));
    };
    /* Slices j + 1 .. j + PD - 1 are in flight while slice j is computed
     * (PD = 2: one slice ahead). */
    constexpr int AHEAD = PD - 1 < NSL ? PD - 1 : NSL;
    Q6Item wb[PD];
#pragma unroll
    for (int j = 0; j < AHEAD; ++j) wb[j] = load_slice(rowp, j);
    __builtin_amdgcn_sched_barrier(0);

    /* This wave's copies (issued first) have landed once at most the
     * weight loads issued after them are outstanding; then every wave's
     * have, after the barrier. */
    constexpr int VM = 5 * AHEAD;
    __builtin_amdgcn_s_waitcnt((VM & 15) | ((VM >> 4) << 14) | (7 << 4) | (15 << 8));
    __builtin_amdgcn_s_barrier();
    /* Run sums of every slice item: wave v for slices v, v + nw, ... */
    for (int sl = wave; sl < NSL; sl += nw) {
        float xv[64];
        q6k_slice_x(q6k_xsh + 1024 * sl, min(lane, 4 * slice_m(sl) - 1), xv);
        xqs[64 * sl + lane] = make_float4(quarter_sum(xv), quarter_sum(xv + 16), quarter_sum(xv + 32),
                                          quarter_sum(xv + 48));
    }
    lds_barrier();
    if (EPI != QMV_ROWDOT_ARGMAX && !has_row) return;

    /* The row at rp: its slices in turn (slice 0's loads already issued),
     * then the lane sums by DPP. */
    auto row_total = [&](gu8 *rp) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < NSL; ++j) {
            const int m = slice_m(j), it = min(lane, 4 * m - 1);
            if (j + AHEAD < NSL) wb[(j + AHEAD) % PD] = load_slice(rp, j + AHEAD);
            float xv[64];
            q6k_slice_x(q6k_xsh + 1024 * j, it, xv);
            const float c = q6k_item_sum(wb[j % PD], xv, xqs[64 * j + lane]);
            acc += lane < 4 * m ? c : 0.0f;
        }
        float tot[1];
        segment_totals<64>(acc, tot);
        return tot[0];
    };
    float out = 0.0f;
    if (has_row) {
        out = row_total(rowp);
        if (job.add != nullptr) out += job.add[row];
        if constexpr (EPI == QMV_ROWDOT_SWIGLU) {
            /* the up row after the gate row (its first loads go out now) */
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < AHEAD; ++j) wb[j] = load_slice(rowp1, j);
            float up = row_total(rowp1);
            if (p.job[1].add != nullptr) up += p.job[1].add[row];
            if (lane == 0) job.y[row] = swiglu_value(out, up);
        } else {
            if (lane == 0) job.y[row] = out;
        }
    }
    if constexpr (EPI == QMV_ROWDOT_ARGMAX) {
        /* One candidate per workgroup: the waves' rows meet in LDS and wave
         * 0 publishes their merge. */
        __shared__ uint64_t wcand[16];
        float v;
        int i, bad;
        wave_candidate(has_row && lane == 0, row, out, v, i, bad);
        if (lane == 0) wcand[wave] = pack_candidate(v, i, bad);
        __syncthreads();
        if (wave != 0) return;
        float bv = -INFINITY;
        int bi = 0x7fffffff, bb = 0;
        for (int w = 0; w < nw; ++w) {
            const uint64_t c = wcand[w];
            const uint32_t hi = (uint32_t)(c >> 32);
            bb |= (int)(hi >> 31);
            argmax_merge(bv, bi, __uint_as_float((uint32_t)c), (int)(hi & 0x7fffffffu));
        }
        publish_tile_candidate(p, (int)blockIdx.x, bv, bi, bb, lane);
    }
}

/* ---- host-side launchers -------------------------------------------------- */

/* The tiled kernels pick a workgroup's job among all QMV_MAX_JOBS slots
 * (launch_args): unused slots start past every workgroup. */
static MatvecParams with_unused_jobs_last(const MatvecParams &p)
{
    MatvecParams q = p;
    for (int i = q.njobs < 1 ? 1 : q.njobs; i < QMV_MAX_JOBS; ++i) q.job[i].wg_begin = INT_MAX;
    return q;
}

template <int FMT, int M>
static hipError_t launch_matvec_fm(const MatvecParams &p, int grid, int waves, hipStream_t s)
{
    if constexpr (M >= 2) {
        if (p.matrix_cores) {
            hipLaunchKernelGGL((matvec_mfma_kernel<FMT, M>), dim3(grid), dim3(waves * 64), 0, s, p);
            return hipGetLastError();
        }
    }
    if (p.units_per_wave == 1)
        hipLaunchKernelGGL((matvec_kernel<FMT, M, true>), dim3(grid), dim3(waves * 64), 0, s, p);
    else
        hipLaunchKernelGGL((matvec_kernel<FMT, M, false>), dim3(grid), dim3(waves * 64), 0, s, p);
    return hipGetLastError();
}

#define QMV_FOR_M(MACRO, FMT)                                                                          \
    switch (m) {                                                                                       \
    case 1: return MACRO(FMT, 1);                                                                      \
    case 2: return MACRO(FMT, 2);                                                                      \
    case 3: return MACRO(FMT, 3);                                                                      \
    case 4: return MACRO(FMT, 4);                                                                      \
    case 5: return MACRO(FMT, 5);                                                                      \
    case 6: return MACRO(FMT, 6);                                                                      \
    case 7: return MACRO(FMT, 7);                                                                      \
    case 8: return MACRO(FMT, 8);                                                                      \
    default: break;                                                                                    \
    }

#define QMV_LAUNCH(FMT, M) launch_matvec_fm<FMT, M>(p, grid, waves, s)

hipError_t launch_matvec(int fmt, const MatvecParams &params, int m, int grid, int waves, hipStream_t s)
{
    if (params.njobs < 1 || params.njobs > QMV_MAX_JOBS) return hipErrorInvalidValue;
    const MatvecParams p = with_unused_jobs_last(params);
    switch (fmt) {
    case QMV_FMT_Q4_K: QMV_FOR_M(QMV_LAUNCH, QMV_FMT_Q4_K) break;
    case QMV_FMT_Q6_K: QMV_FOR_M(QMV_LAUNCH, QMV_FMT_Q6_K) break;
    case QMV_FMT_Q8_0: QMV_FOR_M(QMV_LAUNCH, QMV_FMT_Q8_0) break;
    case QMV_FMT_Q5_0: QMV_FOR_M(QMV_LAUNCH, QMV_FMT_Q5_0) break;
    default: break;
    }
    return hipErrorInvalidValue;
}

hipError_t launch_rowgroup(const RowdotParams &p, int rows, int seg, int epi, int grid, int waves, hipStream_t s,
                           bool norm)
{
    if (waves < 1 || waves > QMV_MAX_WAVES || grid < 1 || (p.sb <= 16 && waves != QMV_ROWGROUP_WAVES) ||
        (p.sb > 16 && seg != 64))
        return hipErrorInvalidValue;
    if (p.njobs < 1 || p.njobs > QMV_MAX_JOBS) return hipErrorInvalidValue;
    const bool split = p.sb > 16;
    /* The kernel picks a workgroup's job among all QMV_MAX_JOBS slots: unused
     * slots start past every workgroup. */
    RowdotParams q = p;
    for (int i = q.njobs; i < QMV_MAX_JOBS; ++i) q.job[i].wg_begin = INT_MAX;
    if (norm && (split || epi == QMV_ROWDOT_ARGMAX || p.norm_w == nullptr)) return hipErrorInvalidValue;
#define QMV_ROWGROUP(R, SEG, E, SP)                                                                    \
    if (rows == R && seg == SEG && epi == E && split == SP && !norm) {                                 \
        hipLaunchKernelGGL((rowgroup_q4k_kernel<R, SEG, E, SP>), dim3(grid), dim3(waves * 64), 0, s, q); \
        return hipGetLastError();                                                                      \
    }
#define QMV_ROWGROUP_N(R, SEG, E)                                                                      \
    if (rows == R && seg == SEG && epi == E && !split && norm) {                                       \
        hipLaunchKernelGGL((rowgroup_q4k_kernel<R, SEG, E, false, true>), dim3(grid), dim3(waves * 64), 0, s, q); \
        return hipGetLastError();                                                                      \
    }
#define QMV_ROWGROUP_E(R, SEG, SP) QMV_ROWGROUP(R, SEG, QMV_ROWDOT_STORE, SP)                         \
    QMV_ROWGROUP(R, SEG, QMV_ROWDOT_SWIGLU, SP) QMV_ROWGROUP(R, SEG, QMV_ROWDOT_ARGMAX, SP)
    QMV_ROWGROUP_E(1, 64, false) QMV_ROWGROUP_E(2, 64, false) QMV_ROWGROUP_E(4, 64, false)
    QMV_ROWGROUP_E(2, 32, false) QMV_ROWGROUP_E(2, 16, false)
    QMV_ROWGROUP_E(1, 64, true) QMV_ROWGROUP_E(2, 64, true) QMV_ROWGROUP_E(4, 64, true)
#define QMV_ROWGROUP_NE(R, SEG) QMV_ROWGROUP_N(R, SEG, QMV_ROWDOT_STORE) QMV_ROWGROUP_N(R, SEG, QMV_ROWDOT_SWIGLU)
    QMV_ROWGROUP_NE(1, 64) QMV_ROWGROUP_NE(2, 64) QMV_ROWGROUP_NE(4, 64) QMV_ROWGROUP_NE(2, 32)
    QMV_ROWGROUP_NE(2, 16)
#undef QMV_ROWGROUP_NE
#undef QMV_ROWGROUP_E
#undef QMV_ROWGROUP_N
#undef QMV_ROWGROUP
    return hipErrorInvalidValue;
}

hipError_t launch_rowloop_q6k(const RowdotParams &p, int epi, int grid, int waves, hipStream_t s)
{
    const int nsl = (p.sb + 15) / 16;
    if (p.sb <= 16 || nsl > 8 || waves < 1 || waves > QMV_ROWLOOP_MAX_WAVES(epi) || grid < 1 ||
        (long long)grid * waves < p.groups || (long long)(grid - 1) * waves >= p.groups)
        return hipErrorInvalidValue;
    if (p.njobs < 1 || p.njobs > QMV_MAX_JOBS) return hipErrorInvalidValue;
    RowdotParams q = p;
    for (int i = q.njobs; i < QMV_MAX_JOBS; ++i) q.job[i].wg_begin = INT_MAX;
    const size_t lds = (size_t)nsl * (1024 + 64) * 16;
    if ((epi == QMV_ROWDOT_SWIGLU && (p.njobs != 2 || p.job[1].rows != p.job[0].rows)) ||
        (epi == QMV_ROWDOT_ARGMAX && (p.njobs != 1 || p.argmax_tiles != grid)))
        return hipErrorInvalidValue;
    switch (nsl * 4 + epi) {
#define QMV_ROWLOOP_Q6(N, E)                                                                       \
    case N * 4 + E: hipLaunchKernelGGL((rowloop_q6k_kernel<N, 2, E>), dim3(grid), dim3(waves * 64), lds, s, q); break;
#define QMV_ROWLOOP_Q6E(N) QMV_ROWLOOP_Q6(N, QMV_ROWDOT_STORE) QMV_ROWLOOP_Q6(N, QMV_ROWDOT_SWIGLU) \
    QMV_ROWLOOP_Q6(N, QMV_ROWDOT_ARGMAX)
        QMV_ROWLOOP_Q6E(2) QMV_ROWLOOP_Q6E(3) QMV_ROWLOOP_Q6E(4) QMV_ROWLOOP_Q6E(5) QMV_ROWLOOP_Q6E(6)
        QMV_ROWLOOP_Q6E(7) QMV_ROWLOOP_Q6E(8)
#undef QMV_ROWLOOP_Q6E
#undef QMV_ROWLOOP_Q6
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_rowmajor_q6k(const uint8_t *raw, uint8_t *out, int rows, int sb, hipStream_t s)
{
    const long long total = (long long)rows * sb * 210;
    const int threads = 256;
    const long long grid = (total + threads - 1) / threads;
    if (rows < 1 || sb < 1 || grid > 0x7fffffffLL) return hipErrorInvalidValue;
    hipLaunchKernelGGL(rowmajor_q6k_kernel, dim3((unsigned)grid), dim3(threads), 0, s, raw, out, sb, total);
    return hipGetLastError();
}

hipError_t launch_dequant(int fmt, const uint8_t *w, float *out, int rows, int cols, int units,
                          int first_row, int row_count, hipStream_t s)
{
    if (row_count <= 0) return hipSuccess;
    const int t0 = first_row / 64, t1 = (first_row + row_count - 1) / 64;
    const dim3 grid(units, t1 - t0 + 1);
    switch (fmt) {
    case QMV_FMT_Q4_K: hipLaunchKernelGGL(dequant_kernel<QMV_FMT_Q4_K>, grid, dim3(64), 0, s, w, out, rows, cols, units, first_row, row_count); break;
    case QMV_FMT_Q6_K: hipLaunchKernelGGL(dequant_kernel<QMV_FMT_Q6_K>, grid, dim3(64), 0, s, w, out, rows, cols, units, first_row, row_count); break;
    case QMV_FMT_Q8_0: hipLaunchKernelGGL(dequant_kernel<QMV_FMT_Q8_0>, grid, dim3(64), 0, s, w, out, rows, cols, units, first_row, row_count); break;
    case QMV_FMT_Q5_0: hipLaunchKernelGGL(dequant_kernel<QMV_FMT_Q5_0>, grid, dim3(64), 0, s, w, out, rows, cols, units, first_row, row_count); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_gather(int fmt, const uint8_t *w, const int *ids, int count, float *out, int rows, int cols,
                         int units, int *status, hipStream_t s)
{
    const dim3 grid((units + 63) / 64, count);
    switch (fmt) {
    case QMV_FMT_Q4_K: hipLaunchKernelGGL(gather_rows_kernel<QMV_FMT_Q4_K>, grid, dim3(64), 0, s, w, ids, out, rows, cols, units, status); break;
    case QMV_FMT_Q6_K: hipLaunchKernelGGL(gather_rows_kernel<QMV_FMT_Q6_K>, grid, dim3(64), 0, s, w, ids, out, rows, cols, units, status); break;
    case QMV_FMT_Q8_0: hipLaunchKernelGGL(gather_rows_kernel<QMV_FMT_Q8_0>, grid, dim3(64), 0, s, w, ids, out, rows, cols, units, status); break;
    case QMV_FMT_Q5_0: hipLaunchKernelGGL(gather_rows_kernel<QMV_FMT_Q5_0>, grid, dim3(64), 0, s, w, ids, out, rows, cols, units, status); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_repack(int fmt, const uint8_t *raw, uint8_t *out, int rows, int blocks_per_row,
                         int units, int blocks_per_unit, int block_bytes, int unit_bytes, int tiles,
                         hipStream_t s)
{
    const long long total = (long long)tiles * units * 64 * blocks_per_unit;
    const int threads = 256;
    const long long grid = (total + threads - 1) / threads;
    if (grid > 0x7fffffffLL) return hipErrorInvalidValue;
    hipLaunchKernelGGL(repack_kernel, dim3((unsigned)grid), dim3(threads), 0, s, raw, out, fmt, rows,
                       blocks_per_row, units, blocks_per_unit, block_bytes, unit_bytes, total);
    return hipGetLastError();
}

hipError_t launch_argmax(const float *logits, int n, float *bval, int *bidx, int *bbad, int nblocks,
                         int *result, hipStream_t s)
{
    hipLaunchKernelGGL(argmax_stage1, dim3(nblocks), dim3(256), 0, s, logits, n, bval, bidx, bbad);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(argmax_stage2, dim3(1), dim3(64), 0, s, bval, bidx, bbad, nblocks, result);
    return hipGetLastError();
}

/* The deferred split-K finish of a prefill launch: thread (tile, quad q,
 * lane) sums the quad of position rows 4q..4q+3 of row 64 tile + lane over
 * the tile's splits, in split order as pf_finish does (so the values are
 * those of the in-kernel finish bit for bit), with up to 16 splits' loads in
 * flight at once (one round for the usual 14-15 splits; batches of 8 and
 * workgroups of 256 threads measured 0.2-0.5% slower on the M = 32 decode
 * set), then applies pf_emit's addend and SwiGLU epilogues (the up
 * sums of job 1 are read alongside, so no pairing protocol is needed). The
 * partials were written by the previous kernel on this stream, whose end
 * makes them visible: plain loads. */
template <int MP>
__global__ void __launch_bounds__(64) pf_reduce_kernel(MatvecParams p)
{
    const int gid = blockIdx.x * blockDim.x + threadIdx.x;
    const int lane = gid & 63;
    const int q = (gid >> 6) % (MP / 4);
    int t = (gid >> 6) / (MP / 4);
    const int nj = p.swiglu ? 1 : p.njobs;
    int j = 0;
    while (j < nj && t >= p.job[j].tiles) {
        t -= p.job[j].tiles;
        ++j;
    }
    if (j >= nj) return;
    const MatvecJob &job = p.job[j];
    const int row = t * 64 + lane;
    if (row >= job.rows) return;
    const int S = job.splits;
    auto total = [&](const MatvecJob &jb) {
        const float *part = p.partials + jb.partial_offset + ((size_t)t * S) * MP * 64 + ((size_t)q * 64 + lane) * 4;
        f32x4_t sum = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int s0 = 0; s0 < S; s0 += 16) {
            /* splits past the last repeat it and are not added */
            f32x4_t v[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) v[i] = *(const f32x4_t *)(part + (size_t)min(s0 + i, S - 1) * (MP / 4) * 256);
#pragma unroll
            for (int i = 0; i < 16; ++i)
                if (s0 + i < S) sum = s0 + i == 0 ? v[i] : sum + v[i];
        }
        return sum;
    };
    const f32x4_t a = total(job);
    const f32x4_t u = p.swiglu ? total(p.job[1]) : f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int m = 4 * q + e;
        if (m >= p.positions) break;
        float v = a[e];
        if (job.add != nullptr) v += job.add[(size_t)m * job.ldadd + row];
        if (p.swiglu) {
            float w = u[e];
            if (p.job[1].add != nullptr) w += p.job[1].add[(size_t)m * p.job[1].ldadd + row];
            v = swiglu_value(v, w);
        }
        job.y[(size_t)m * job.ldy + row] = v;
    }
}

/* Prefill launches whose in-kernel finish would take this many rounds of
 * partial loads or more (ceil(splits / (64 / rows)); 16 quads per round)
 * finish in pf_reduce_kernel instead. Measured on MI355X (µs per launch,
 * Qwen2.5-7B layer shapes, cold graphs of 28, in-kernel / deferred): at 32
 * positions q|k|v (14 splits, 7 rounds) 18.5 / 16.3, o (7 rounds) 17.5 /
 * 14.4, down (15 splits, 8 rounds) 46.3 / 44.5, gate|up (3 splits, 2 rounds)
 * 47.8 / 49.6; at 16 positions q|k|v (4 rounds) 13.3 / 12.3, o 12.4 / 11.1,
 * down (4 rounds) 35.0 / 35.4, gate|up (1 round) 33.1 / 35.8. In the
 * decode-step set (same box) deferring the launches of 4 rounds or more gave
 * 3.513 against 3.655 ms at 32 positions but 2.612 against 2.600 at 16, so
 * the 4-round launches keep the in-kernel finish. */
#ifndef QMV_PF_DEFER_ROUNDS
#define QMV_PF_DEFER_ROUNDS 5
#endif

static hipError_t launch_prefill_kernel(int fmt, const MatvecParams &p, int rows, int grid, hipStream_t s)
{
    const dim3 g(grid), b(QMV_PF_WAVES * 64);
    if (fmt == QMV_FMT_Q4_K && rows == 16) hipLaunchKernelGGL((prefill_kernel<QMV_FMT_Q4_K, 1>), g, b, 0, s, p);
    else if (fmt == QMV_FMT_Q4_K && rows == 32) hipLaunchKernelGGL((prefill_kernel<QMV_FMT_Q4_K, 2>), g, b, 0, s, p);
    else if (fmt == QMV_FMT_Q6_K && rows == 16) hipLaunchKernelGGL((prefill_kernel<QMV_FMT_Q6_K, 1>), g, b, 0, s, p);
    else if (fmt == QMV_FMT_Q6_K && rows == 32) hipLaunchKernelGGL((prefill_kernel<QMV_FMT_Q6_K, 2>), g, b, 0, s, p);
    else if (fmt == QMV_FMT_Q5_0 && rows == 16) hipLaunchKernelGGL((prefill_kernel<QMV_FMT_Q5_0, 1>), g, b, 0, s, p);
    else if (fmt == QMV_FMT_Q5_0 && rows == 32) hipLaunchKernelGGL((prefill_kernel<QMV_FMT_Q5_0, 2>), g, b, 0, s, p);
    else if (fmt == QMV_FMT_Q8_0 && rows == 16) hipLaunchKernelGGL((prefill_kernel<QMV_FMT_Q8_0, 1>), g, b, 0, s, p);
    else if (fmt == QMV_FMT_Q8_0 && rows == 32) hipLaunchKernelGGL((prefill_kernel<QMV_FMT_Q8_0, 2>), g, b, 0, s, p);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_prefill(int fmt, const MatvecParams &params, int rows, int grid, hipStream_t s)
{
    if (rows != 16 && rows != 32) return hipErrorInvalidValue;
    MatvecParams p = params;
    const int S = p.job[0].splits, per_round = 64 / rows;
    p.pf_deferred = S > 1 && (S + per_round - 1) / per_round >= QMV_PF_DEFER_ROUNDS ? 1 : 0;
    const hipError_t e = launch_prefill_kernel(fmt, p, rows, grid, s);
    if (e != hipSuccess || !p.pf_deferred) return e;
    long long tiles = 0;
    for (int j = 0; j < (p.swiglu ? 1 : p.njobs); ++j) tiles += p.job[j].tiles;
    const long long threads = tiles * (rows / 4) * 64;
    const dim3 rg((unsigned)(threads / 64)), rb(64); /* one wave per workgroup */
    if (rows == 16) hipLaunchKernelGGL((pf_reduce_kernel<16>), rg, rb, 0, s, p);
    else hipLaunchKernelGGL((pf_reduce_kernel<32>), rg, rb, 0, s, p);
    return hipGetLastError();
}

__global__ void __launch_bounds__(256) copy_f32_kernel(const float *__restrict__ src, float *__restrict__ dst, size_t n)
{
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) dst[i] = src[i];
}

hipError_t launch_copy(const float *src, float *dst, size_t n, hipStream_t s)
{
    size_t blocks = (n + 255) / 256;
    if (blocks > 1024) blocks = 1024;
    hipLaunchKernelGGL(copy_f32_kernel, dim3((unsigned)blocks), dim3(256), 0, s, src, dst, n);
    return hipGetLastError();
}

/* dst[0..n) = v with vector stores: clears counters where a memset node
 * must not be used (code a caller may capture into a graph). */
__global__ void __launch_bounds__(256) fill_u32_kernel(unsigned *__restrict__ dst, size_t n, unsigned v)
{
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) dst[i] = v;
}

hipError_t launch_fill_u32(unsigned *dst, size_t n, unsigned v, hipStream_t s)
{
    if (n == 0) return hipSuccess;
    size_t blocks = (n + 255) / 256;
    if (blocks > 1024) blocks = 1024;
    hipLaunchKernelGGL(fill_u32_kernel, dim3((unsigned)blocks), dim3(256), 0, s, dst, n, v);
    return hipGetLastError();
}

hipError_t launch_rms_norm(const float *x, const float *w, int n, int batch, float eps, float *out, hipStream_t s)
{
    hipLaunchKernelGGL(rms_norm_kernel, dim3(batch), dim3(QMV_NORM_THREADS), 0, s, x, w, n, eps, out);
    return hipGetLastError();
}

} // namespace qmv
