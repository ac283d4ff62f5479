// Device helpers shared by the gfx950 kernels of the dequant+GEMV path.
//
// Central trick (used by every GEMV kernel): two b-bit codes are turned into a
// pair of bf16 values with ONE v_and_or_b32, by OR-ing the code bits into the
// mantissa of the bf16 constant 128.0 (bits 0x4300):
//     bf16(0x4300 | (q << e)) = 128 + q * 2^e          (e + b <= 7)
// A v_dot2c_f32_bf16 against a pair (v_lo, v_hi) of bf16 operands scaled by
// 2^-e then accumulates 128*(v_lo + v_hi) + q_lo*v_lo' + q_hi*v_hi' in fp32;
// the constant 128*sum(v) is removed by starting the accumulator at
// -128*sum(v). Products of a <=15-bit integer with a bf16 are exact in fp32.
// Which two codes share a pair, and the exponent e of each, is fixed per bit
// width by PairMap<BITS> below; the operand (a bf16 x for gate/up) is arranged
// in the same pair order.
//
// Second trick (fp32 operands: the activation of the down projection, a fp16
// or fp32 x): a code masked in place inside a 16-bit half reads as the fp16
// subnormal q * 2^(p-24), so one v_fma_mix_f32 multiplies it by a fp32 value
// exactly (chunk_dot_f32 below).
//
// A "chunk" is 32 consecutive codes of one matrix row (BITS*4 bytes); the 16
// pairs of a chunk are numbered P = 0..15.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wisp {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

constexpr uint32_t kBias2 = 0x43004300u;  // two bf16 128.0
constexpr float kBiasF = 128.0f;

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c,
                                          false);
}

// round-to-nearest-even float -> bf16 pair (v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    bf16x2_t v;
    v.x = (__bf16)lo;
    v.y = (__bf16)hi;
    return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    return (uint16_t)(pack_bf16x2(f, 0.f) & 0xFFFFu);
}
__device__ __forceinline__ float bf16_lo(uint32_t p) { return __uint_as_float(p << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t p) { return __uint_as_float(p & 0xFFFF0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }
__device__ __forceinline__ float h2f(uint16_t h) { return __half2float(__ushort_as_half(h)); }

// (w & m) | bias in ONE v_and_or_b32. Written as inline asm because the
// compiler otherwise splits it into v_and_b32 + v_or_b32 with literals (a
// gfx9 VOP3 takes no literal and at most one SGPR): the mask goes in an SGPR,
// the bias in a VGPR that bias_vgpr() materialises once per kernel.
__device__ __forceinline__ uint32_t ao(uint32_t w, uint32_t m, uint32_t bias) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(w), "s"(m), "v"(bias));
    return r;
}
__device__ __forceinline__ uint32_t bias_vgpr() {
    uint32_t b;
    asm volatile("v_mov_b32 %0, %1" : "=v"(b) : "s"(kBias2));
    return b;
}
__device__ __forceinline__ uint32_t alignbit(uint32_t hi, uint32_t lo, uint32_t s) {
    return __builtin_amdgcn_alignbit(hi, lo, s);
}

// The workgroup's (bx, by, bz) of a logical nx x ny x nz grid launched as T = nx ny nz
// workgroups in one dimension. Workgroup i runs on XCD i % 8; the logical order (bx fastest)
// is dealt to the XCDs in contiguous runs (XCD x takes the x-th run of about T / 8: logical
// index (i % 8) floor(T / 8) + min(i % 8, T mod 8) + floor(i / 8), a bijection for every T),
// so workgroups that differ only in bx mostly share an XCD, and lines they all read (a row's
// quant-group scales, a token tile, partial sums) are fetched into one XCD's L2 once instead
// of into up to nx of them.
__device__ __forceinline__ void xcd_block(int nx, int ny, int nz, int& bx, int& by, int& bz) {
    const int T = nx * ny * nz, i = blockIdx.x;
    const int q = T >> 3, r = T & 7, x = i & 7, j = i >> 3;
    const int p = x * q + min(x, r) + j;
    bx = p % nx;
    by = (p / nx) % ny;
    bz = p / (nx * ny);
}

// As xcd_block, but the groups of nx workgroups (one (by, bz)) are dealt to the XCDs round
// robin, group g to XCD g % 8, each group's nx workgroups on that XCD: for groups of unequal
// work (work items of different token counts), which contiguous runs would pile onto a few
// XCDs. The last (ny nz) mod 8 groups keep the plain order (no XCD in common).
__device__ __forceinline__ void xcd_rr_block(int nx, int ny, int nz, int& bx, int& by, int& bz) {
    const int i = blockIdx.x, ng = ny * nz, ng8 = ng & ~7, t8 = ng8 * nx;
    int g;
    if (i < t8) {
        const int j = i >> 3;
        g = (i & 7) + 8 * (j / nx);
        bx = j % nx;
    } else {
        g = ng8 + (i - t8) / nx;
        bx = (i - t8) % nx;
    }
    by = g % ny;
    bz = g / ny;
}

// ---------------------------------------------------------------------------
// Pair maps: for pair P of a chunk, the chunk-relative code index of its low
// and high half and the power-of-two exponent e of each half (the code sits at
// mantissa bits e..e+BITS-1, so the operand is stored multiplied by 2^-e).
// ---------------------------------------------------------------------------
template <int BITS>
struct PairMap;

// 4-bit: dword d holds codes 8d..8d+7 (nibble i at bits 4i). Window w >> (4p - 3) puts
// codes 8d+p and 8d+p+4 at bits 3-6 and 19-22: the pair reads as (128 + 8q, 128 + 8q'),
// so the bias 128 is 16 times the code's top value instead of 128 (the accumulator
// cancels 3 bits less), with the operand stored times 2^-3 (exact).
template <>
struct PairMap<4> {
    static constexpr int lo(int P) { return 8 * (P >> 2) + (P & 3); }
    static constexpr int hi(int P) { return lo(P) + 4; }
    static constexpr int elo(int) { return 3; }
    static constexpr int ehi(int) { return 3; }
};

// 3-bit: 32 codes in 96 bits (code c at bit 3c). Pairs (c, c+5) for
// c in 0..4 and 10..14 with the low code at window bits 4-6 (e=4) and the high
// code at bits 19-21 (e=3); pairs (c, c+6) for c in 20..25 with the low code at
// bits 2-4 (e=2) and the high code at bits 20-22 (e=4). The codes sit as high
// in the mantissa as their spacing allows, so the bias 128 stays small against
// 2^e * q.
template <>
struct PairMap<3> {
    static constexpr int lo(int P) { return P < 5 ? P : (P < 10 ? 10 + (P - 5) : 20 + (P - 10)); }
    static constexpr int hi(int P) { return P < 5 ? P + 5 : (P < 10 ? 15 + (P - 5) : 26 + (P - 10)); }
    static constexpr int elo(int P) { return P < 10 ? 4 : 2; }
    static constexpr int ehi(int P) { return P < 10 ? 3 : 4; }
};

// 2-bit: dword d holds codes 16d..16d+15 (code i at bits 2i). Window w >> (4m - 3)
// puts codes 2m, 2m+1 at bits 3-4 and 5-6 and codes 2m+8, 2m+9 at bits 19-20 and
// 21-22: pairs (i, i+8) at e = 3 (i even) or 5 (i odd).
template <>
struct PairMap<2> {
    static constexpr int lo(int P) { return 16 * (P >> 3) + (P & 7); }
    static constexpr int hi(int P) { return lo(P) + 8; }
    static constexpr int elo(int P) { return (P & 1) ? 5 : 3; }
    static constexpr int ehi(int P) { return elo(P); }
};

// chunk dwords -> 16 biased bf16 code pairs
template <int BITS>
__device__ __forceinline__ void code_pairs(const uint32_t* d, uint32_t* p, uint32_t B);

template <>
__device__ __forceinline__ void code_pairs<4>(const uint32_t* d, uint32_t* p, uint32_t B) {
    constexpr uint32_t M = 0x00780078u;  // bits 3-6 of each half
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t w = d[i];
        p[4 * i + 0] = ao(w << 3, M, B);
        p[4 * i + 1] = ao(w >> 1, M, B);
        p[4 * i + 2] = ao(w >> 5, M, B);
        p[4 * i + 3] = ao(w >> 9, M, B);
    }
}

template <>
__device__ __forceinline__ void code_pairs<3>(const uint32_t* d, uint32_t* p, uint32_t B) {
    constexpr uint32_t MA = 0x00380070u;  // low code at bits 4-6, high code at bits 19-21
    constexpr uint32_t MC = 0x0070001Cu;  // low code at bits 2-4, high code at bits 20-22
    const uint32_t d0 = d[0], d1 = d[1], d2 = d[2];
    // window start 3c-4 for c = 0..4
    p[0] = ao(d0 << 4, MA, B);
    p[1] = ao(d0 << 1, MA, B);
    p[2] = ao(alignbit(d1, d0, 2), MA, B);
    p[3] = ao(alignbit(d1, d0, 5), MA, B);
    p[4] = ao(alignbit(d1, d0, 8), MA, B);
    // window start 3c-4 for c = 10..14
    p[5] = ao(alignbit(d1, d0, 26), MA, B);
    p[6] = ao(alignbit(d1, d0, 29), MA, B);
    p[7] = ao(d1, MA, B);
    p[8] = ao(alignbit(d2, d1, 3), MA, B);
    p[9] = ao(alignbit(d2, d1, 6), MA, B);
    // window start 3c-2 for c = 20..25
    p[10] = ao(alignbit(d2, d1, 26), MC, B);
    p[11] = ao(alignbit(d2, d1, 29), MC, B);
    p[12] = ao(d2, MC, B);
    p[13] = ao(d2 >> 3, MC, B);
    p[14] = ao(d2 >> 6, MC, B);
    p[15] = ao(d2 >> 9, MC, B);
}

template <>
__device__ __forceinline__ void code_pairs<2>(const uint32_t* d, uint32_t* p, uint32_t B) {
    constexpr uint32_t M3 = 0x00180018u, M5 = 0x00600060u;  // bits 3-4 / 5-6 of each half
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t w = d[i];
        const uint32_t w0 = w << 3, w1 = w >> 1, w2 = w >> 5, w3 = w >> 9;
        p[8 * i + 0] = ao(w0, M3, B);
        p[8 * i + 1] = ao(w0, M5, B);
        p[8 * i + 2] = ao(w1, M3, B);
        p[8 * i + 3] = ao(w1, M5, B);
        p[8 * i + 4] = ao(w2, M3, B);
        p[8 * i + 5] = ao(w2, M5, B);
        p[8 * i + 6] = ao(w3, M3, B);
        p[8 * i + 7] = ao(w3, M5, B);
    }
}

// exact multiplication by 2^-e for the small e used here
__device__ __forceinline__ float scale_pow2(float v, int e) {
    return v * __uint_as_float((uint32_t)(127 - e) << 23);
}

// load one chunk (BITS dwords) from a BITS*4-aligned address (4-aligned for
// 3-bit); non-temporal: every expert byte is read exactly once per layer.
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x3_t __attribute__((ext_vector_type(3)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

template <int BITS>
__device__ __forceinline__ void load_chunk(const uint8_t* p, uint32_t* d);
template <>
__device__ __forceinline__ void load_chunk<4>(const uint8_t* p, uint32_t* d) {
    const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
    d[0] = v.x; d[1] = v.y; d[2] = v.z; d[3] = v.w;
}
template <>
__device__ __forceinline__ void load_chunk<3>(const uint8_t* p, uint32_t* d) {
    const u32x3_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x3_t*>(p));
    d[0] = v.x; d[1] = v.y; d[2] = v.z;
}
template <>
__device__ __forceinline__ void load_chunk<2>(const uint8_t* p, uint32_t* d) {
    const u32x2_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(p));
    d[0] = v.x; d[1] = v.y;
}

// The 32 codes of one loaded chunk (BITS dwords, little-endian): element i
// sits at bit BITS*i (the packing of quant.py:25-40; 3-bit codes may straddle
// dwords).
template <int BITS>
__device__ __forceinline__ void chunk_codes(const uint32_t* d, uint32_t* q) {
    if constexpr (BITS == 4) {
#pragma unroll
        for (int i = 0; i < 32; ++i) q[i] = (d[i >> 3] >> (4 * (i & 7))) & 15u;
    } else if constexpr (BITS == 2) {
#pragma unroll
        for (int i = 0; i < 32; ++i) q[i] = (d[i >> 4] >> (2 * (i & 15))) & 3u;
    } else {
        static_assert(BITS == 3, "chunk_codes: 4, 3 or 2 bits");
        const uint64_t lo = (uint64_t)d[0] | ((uint64_t)d[1] << 32);
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            const int b = 3 * i;
            if (b + 3 <= 64)
                q[i] = (uint32_t)(lo >> b) & 7u;
            else if (b >= 64)
                q[i] = (d[2] >> (b - 64)) & 7u;
            else
                q[i] = (uint32_t)((lo >> b) | ((uint64_t)d[2] << (64 - b))) & 7u;
        }
    }
}

// The binary32 value of one 16-bit half of x read as fp16. A half whose
// exponent field (bits 10-14) and sign are zero is the subnormal
// (bits) * 2^-24, converted exactly.
__device__ __forceinline__ float half_lo_f(uint32_t x) { return (float)__builtin_bit_cast(_Float16, (uint16_t)x); }
__device__ __forceinline__ float half_hi_f(uint32_t x) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(x >> 16));
}

// Dequantize one chunk of 32 codes (BITS = 4 or 2; BITS dwords d, element i at
// bit BITS*i) of a group whose fp16 scale s and min m are packed in
// sm = s | m << 16, into 32 binary32 values in element order: q*s + m rounded
// once, the value quant.py:76-87 computes (q*s is exact in binary32) before its
// bf16 rounding. No code is converted to float: a code masked in place at bit p < 8 of a
// 16-bit half is the fp16 subnormal q * 2^(p-24), and fma(q * 2^(p-24),
// s * 2^(24-p), m) has the exact product q*s and one rounding. s * 2^(24-p) is
// exact (a power-of-two scaling of an fp16 value stays in binary32 range).
// The results are 0 or at least 2^-24 in magnitude (s and m are multiples of
// 2^-24), so no binary32 subnormal arises. One mask yields a code of each half.
template <int BITS>
__device__ __forceinline__ void dequant32_f32(const uint32_t* d, uint32_t sm, float* v) {
    const float s = h2f((uint16_t)sm), m = h2f((uint16_t)(sm >> 16));
    if constexpr (BITS == 4) {
        const float s0 = s * 0x1p24f, s4 = s * 0x1p20f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const uint32_t x = d[w], y = x >> 8;
            const uint32_t a = x & 0x000F000Fu, b = x & 0x00F000F0u, c = y & 0x000F000Fu, e = y & 0x00F000F0u;
            v[8 * w + 0] = __builtin_fmaf(half_lo_f(a), s0, m);
            v[8 * w + 1] = __builtin_fmaf(half_lo_f(b), s4, m);
            v[8 * w + 2] = __builtin_fmaf(half_lo_f(c), s0, m);
            v[8 * w + 3] = __builtin_fmaf(half_lo_f(e), s4, m);
            v[8 * w + 4] = __builtin_fmaf(half_hi_f(a), s0, m);
            v[8 * w + 5] = __builtin_fmaf(half_hi_f(b), s4, m);
            v[8 * w + 6] = __builtin_fmaf(half_hi_f(c), s0, m);
            v[8 * w + 7] = __builtin_fmaf(half_hi_f(e), s4, m);
        }
    } else {
        static_assert(BITS == 2, "dequant32_f32: 4 or 2 bits");
        const float sk[4] = {s * 0x1p24f, s * 0x1p22f, s * 0x1p20f, s * 0x1p18f};
#pragma unroll
        for (int w = 0; w < 2; ++w) {
            const uint32_t x = d[w], y = x >> 8;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t a = x & (0x00030003u << (2 * k)), b = y & (0x00030003u << (2 * k));
                v[16 * w + k] = __builtin_fmaf(half_lo_f(a), sk[k], m);
                v[16 * w + 4 + k] = __builtin_fmaf(half_lo_f(b), sk[k], m);
                v[16 * w + 8 + k] = __builtin_fmaf(half_hi_f(a), sk[k], m);
                v[16 * w + 12 + k] = __builtin_fmaf(half_hi_f(b), sk[k], m);
            }
        }
    }
}

// Sum of q_i * a_i over one 32-code chunk (BITS dwords d, element i at bit BITS*i) against 32 fp32 values a[i]
// in element order: exact products, fp32 accumulation (the fp32 q*a of the reference's down kernels,
// kernels.py:107-111, 166-184). Each code is masked in place inside a 16-bit half, where it reads as the fp16
// subnormal q * 2^(p-24) for its bit offset p in the half (p + BITS <= 10, so the exponent field stays zero),
// and one v_fma_mix_f32 multiplies that half by a[i] exactly and adds in fp32. Codes at the same offset share
// accumulators, which are scaled back by 2^(24-p) (exact) at the end. 13 VALU instructions per 8 codes at 4 bits.
template <int BITS>
__device__ __forceinline__ float chunk_dot_f32(const uint32_t* d, const float* a);

template <>
__device__ __forceinline__ float chunk_dot_f32<4>(const uint32_t* d, const float* a) {
    // dword w: nibbles 0/4 at p = 0 of the two halves, 1/5 at p = 4; after >> 8: 2/6 at p = 0, 3/7 at p = 4
    float s0a = 0.f, s0b = 0.f, s4a = 0.f, s4b = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const uint32_t x = d[w], y = x >> 8;
        const uint32_t c0 = x & 0x000F000Fu, c1 = x & 0x00F000F0u, c2 = y & 0x000F000Fu, c3 = y & 0x00F000F0u;
        const float* v = a + 8 * w;
        s0a = __builtin_fmaf(half_lo_f(c0), v[0], s0a);
        s0b = __builtin_fmaf(half_hi_f(c0), v[4], s0b);
        s4a = __builtin_fmaf(half_lo_f(c1), v[1], s4a);
        s4b = __builtin_fmaf(half_hi_f(c1), v[5], s4b);
        s0a = __builtin_fmaf(half_lo_f(c2), v[2], s0a);
        s0b = __builtin_fmaf(half_hi_f(c2), v[6], s0b);
        s4a = __builtin_fmaf(half_lo_f(c3), v[3], s4a);
        s4b = __builtin_fmaf(half_hi_f(c3), v[7], s4b);
    }
    return (s0a + s0b) * 0x1p24f + (s4a + s4b) * 0x1p20f;
}

template <>
__device__ __forceinline__ float chunk_dot_f32<2>(const uint32_t* d, const float* a) {
    // dword w holds codes 16w .. 16w + 15; mask 3 << 2k takes code k (low half) and 8 + k (high half) of x, and
    // codes 4 + k and 12 + k of x >> 8, all at p = 2k
    float s[4][2] = {{0.f, 0.f}, {0.f, 0.f}, {0.f, 0.f}, {0.f, 0.f}};
#pragma unroll
    for (int w = 0; w < 2; ++w) {
        const uint32_t x = d[w], y = x >> 8;
        const float* v = a + 16 * w;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t M = 0x00030003u << (2 * k);
            const uint32_t cx = x & M, cy = y & M;
            s[k][0] = __builtin_fmaf(half_lo_f(cx), v[k], s[k][0]);
            s[k][1] = __builtin_fmaf(half_hi_f(cx), v[8 + k], s[k][1]);
            s[k][0] = __builtin_fmaf(half_lo_f(cy), v[4 + k], s[k][0]);
            s[k][1] = __builtin_fmaf(half_hi_f(cy), v[12 + k], s[k][1]);
        }
    }
    return ((s[0][0] + s[0][1]) * 0x1p24f + (s[1][0] + s[1][1]) * 0x1p22f) +
           ((s[2][0] + s[2][1]) * 0x1p20f + (s[3][0] + s[3][1]) * 0x1p18f);
}

template <>
__device__ __forceinline__ float chunk_dot_f32<3>(const uint32_t* d, const float* a) {
    // 24-bit windows, masked without the bias: window P holds code PairMap<3>::lo(P) in the low half and code
    // PairMap<3>::hi(P) in the high half at the offsets below (0, 1 or 2; fp16 subnormals need p + 3 <= 10)
    constexpr uint32_t MA = 0x0007000Eu, MC = 0x001C0007u;  // (c, c+5): p = 1 / 0; (c, c+6): p = 0 / 2
    const uint32_t d0 = d[0], d1 = d[1], d2 = d[2];
    const uint32_t w[16] = {(d0 << 1) & MA,
                            alignbit(d1, d0, 2) & MA,
                            alignbit(d1, d0, 5) & MA,
                            alignbit(d1, d0, 8) & MA,
                            alignbit(d1, d0, 11) & MA,
                            alignbit(d1, d0, 29) & MA,
                            d1 & MA,
                            alignbit(d2, d1, 3) & MA,
                            alignbit(d2, d1, 6) & MA,
                            alignbit(d2, d1, 9) & MA,
                            alignbit(d2, d1, 28) & MC,
                            alignbit(d2, d1, 31) & MC,
                            (d2 >> 2) & MC,
                            (d2 >> 5) & MC,
                            (d2 >> 8) & MC,
                            (d2 >> 11) & MC};
    float s[3][2] = {{0.f, 0.f}, {0.f, 0.f}, {0.f, 0.f}};  // by offset p, two chains each
#pragma unroll
    for (int P = 0; P < 16; ++P) {
        const int pl = P < 10 ? 1 : 0, ph = P < 10 ? 0 : 2;
        s[pl][P & 1] = __builtin_fmaf(half_lo_f(w[P]), a[PairMap<3>::lo(P)], s[pl][P & 1]);
        s[ph][(P + 1) & 1] = __builtin_fmaf(half_hi_f(w[P]), a[PairMap<3>::hi(P)], s[ph][(P + 1) & 1]);
    }
    return ((s[0][0] + s[0][1]) * 0x1p24f + (s[1][0] + s[1][1]) * 0x1p23f) + (s[2][0] + s[2][1]) * 0x1p22f;
}

// Sum of the 32 fp32 values of one chunk, two chains (pairs of elements) then combined.
__device__ __forceinline__ float chunk_sum_f32(const float* a) {
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i += 2) {
        s0 += a[i];
        s1 += a[i + 1];
    }
    return s0 + s1;
}

// dequant32_f32 rounded to bf16 (RTNE), as 16 pairs in element order.
template <int BITS>
__device__ __forceinline__ void dequant32(const uint32_t* d, uint32_t sm, uint32_t* out) {
    float v[32];
    dequant32_f32<BITS>(d, sm, v);
#pragma unroll
    for (int i = 0; i < 16; ++i) out[i] = pack_bf16x2(v[2 * i], v[2 * i + 1]);
}

// bf16 pair (2^elo(P), 2^ehi(P)): dot2 of a stored operand pair with it gives
// the sum of the two true (unscaled) operand values.
template <int BITS>
__device__ __forceinline__ constexpr uint32_t unscale_pair(int P) {
    return ((uint32_t)(0x3F80 + (PairMap<BITS>::ehi(P) << 7)) << 16) | (uint32_t)(0x3F80 + (PairMap<BITS>::elo(P) << 7));
}
constexpr uint32_t kOnes2 = 0x3F803F80u;  // bf16 pair (1, 1)

// Operand pairs of one chunk from the 16 dwords w[] holding 32 consecutive
// bf16 values (value c = half c&1 of w[c>>1]): pair P = (v[lo]*2^-elo,
// v[hi]*2^-ehi). Exact for bf16 inputs. SCALED false: the values as they are,
// (v[lo], v[hi]) -- for a width whose pairs all share one e, the dots are then
// 2^e times the scaled ones, with the same bits once multiplied by 2^-e.
template <int BITS, bool SCALED = true>
__device__ __forceinline__ void operand_pairs(const uint32_t* w, uint32_t* pr) {
#pragma unroll
    for (int P = 0; P < 16; ++P) {
        const int lo = PairMap<BITS>::lo(P), hi = PairMap<BITS>::hi(P);
        const uint32_t wl = w[lo >> 1], wh = w[hi >> 1];
        if (!SCALED || (PairMap<BITS>::elo(P) == 0 && PairMap<BITS>::ehi(P) == 0)) {
            // pure 16-bit shuffle, one v_perm_b32: result bytes 0-1 from wl (selectors 0-3), 2-3 from
            // wh (selectors 4-7), each the low or the high half
            const uint32_t sl = (lo & 1) ? 0x0302u : 0x0100u, sh = (hi & 1) ? 0x0706u : 0x0504u;
            pr[P] = __builtin_amdgcn_perm(wh, wl, (sh << 16) | sl);
        } else {
            const float fl = (lo & 1) ? bf16_hi(wl) : bf16_lo(wl);
            const float fh = (hi & 1) ? bf16_hi(wh) : bf16_lo(wh);
            pr[P] = pack_bf16x2(scale_pow2(fl, PairMap<BITS>::elo(P)), scale_pow2(fh, PairMap<BITS>::ehi(P)));
        }
    }
}

// Sum of the stored operand values (for the bias) and of the true values.
template <int BITS>
__device__ __forceinline__ void operand_sums(const uint32_t* pr, float& vsum, float& tsum) {
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int P = 0; P < 16; P += 2) {
        a0 = dot2(pr[P], kOnes2, a0);
        a1 = dot2(pr[P + 1], kOnes2, a1);
    }
    vsum = a0 + a1;
    if (BITS == 4) {
        tsum = vsum * 8.0f;  // every 4-bit operand is stored times 2^-3 (exact scalings)
    } else {
        float b0 = 0.f, b1 = 0.f;
#pragma unroll
        for (int P = 0; P < 16; P += 2) {
            b0 = dot2(pr[P], unscale_pair<BITS>(P), b0);
            b1 = dot2(pr[P + 1], unscale_pair<BITS>(P + 1), b1);
        }
        tsum = b0 + b1;
    }
}

// Broadcast lane I of each quad to the whole quad (DPP quad_perm [I,I,I,I]).
template <int I>
__device__ __forceinline__ uint32_t quad_bcast(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, I * 0x55, 0xF, 0xF, false);
}

// v from the lane selected by the DPP control CTRL (0 where the source lane is
// outside the row, bound_ctrl).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}

// Wave-wide sum and maximum (wave64) with DPP: the 16 lanes of each row in four steps
// (quad_perm xor 1, xor 2, row_half_mirror, row_mirror), then the four row totals read
// from lanes 0, 16, 32 and 48 and combined in that order. No LDS round trip, so a run of
// independent reductions costs a few VALU cycles each; the result is wave-uniform. The
// sum order differs from wave_sum's butterfly.
__device__ __forceinline__ float wave_sum_dpp(float v) {
    v += dpp_f<0xB1>(v);
    v += dpp_f<0x4E>(v);
    v += dpp_f<0x141>(v);
    v += dpp_f<0x140>(v);
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return (r0 + r1) + (r2 + r3);
}
__device__ __forceinline__ float wave_max_dpp(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    v = fmaxf(v, dpp_f<0x140>(v));
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// The value of lane l ^ 16 (xor16) or l ^ 32 (xor32) combined with lane l's, in every lane,
// without LDS: gfx950's permlane swaps exchange the odd rows (halves) of one copy of v with
// the even rows (halves) of another, after which each lane holds its own value in one result
// and its partner's in the other. Sums add the two in either order (addition commutes), so
// they equal the xor butterfly's own + partner bit for bit.
__device__ __forceinline__ float max_xor16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float add_xor16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float add_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// The xor butterfly's sum (partners l ^ 32, ^ 16, ^ 8, ^ 4, ^ 2, ^ 1 in that order, as
// torch's warp reductions take them), bit for bit, without LDS: ^ 32 and ^ 16 by the permlane
// swaps; ^ 8 is row_ror:8 exactly; after it every lane's value equals its ^ 8 partner's (the
// two added the same pair), so row_ror:4 (lane (l + 4) % 16, which differs from l ^ 4 at most
// in bit 3) reads the same value as l ^ 4, and likewise row_ror:2 and row_ror:1 after the
// steps before them.
__device__ __forceinline__ float wave_sum(float v) {
    v = add_xor32(v);
    v = add_xor16(v);
    v += dpp_f<0x128>(v);  // row_ror:8
    v += dpp_f<0x124>(v);  // row_ror:4
    v += dpp_f<0x122>(v);  // row_ror:2
    v += dpp_f<0x121>(v);  // row_ror:1
    return v;
}
__device__ __forceinline__ float wave_min(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fminf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

__device__ __forceinline__ float bf(uint32_t v16) { return __uint_as_float(v16 << 16); }
__device__ __forceinline__ float rbf(float v) { return bf(f32_to_bf16(v)); }  // round to bf16, as float

// One q or k head of the decoder on one wave (graphdec.py:163-170: q_norm / k_norm, the
// Qwen3 RMSNorm module in bf16, then rope_decode at one position): lane t takes the
// element pairs (i, i + D/2), i = t, t + 64, ...; the sum of squares adds a^2 + b^2 per
// pair in that order, then the xor butterfly over the 64 lanes; x * rsqrt(mean + eps) and
// the weight product are each rounded to bf16 as the module's bf16 tensors are; the
// rotation runs in binary32 on those values and the cos/sin rows, rounded once. The
// result goes to dst and, when non-null, to dst2 (bf16). Every lane of the wave calls it.
// In two steps: hnr_load reads the lane's inputs into registers (a caller issues these
// loads ahead of others whose data it needs later), hnr_finish does the arithmetic.
template <int D>
struct HnrIn {
    static constexpr int NP = (D / 2 + 63) / 64;
    uint16_t a[NP], b[NP], wa[NP], wb[NP], ca[NP], cb[NP], sa[NP], sb[NP];
};
template <int D>
__device__ __forceinline__ void hnr_load(const uint16_t* __restrict__ x, const uint16_t* __restrict__ nw,
                                         const uint16_t* __restrict__ cs, const uint16_t* __restrict__ sn, int lane,
                                         HnrIn<D>& in) {
    constexpr int HALF = D / 2;
#pragma unroll
    for (int t = 0; t < HnrIn<D>::NP; ++t) {
        const int i = min(lane + 64 * t, HALF - 1);  // lanes past the head repeat its last pair (unused)
        in.a[t] = x[i];
        in.b[t] = x[i + HALF];
        in.wa[t] = nw[i];
        in.wb[t] = nw[i + HALF];
        in.ca[t] = cs[i];
        in.cb[t] = cs[i + HALF];
        in.sa[t] = sn[i];
        in.sb[t] = sn[i + HALF];
    }
}
template <int D>
__device__ __forceinline__ void hnr_finish(const HnrIn<D>& in, float eps, uint16_t* dst, uint16_t* dst2, int lane) {
#pragma clang fp contract(off)
    constexpr int HALF = D / 2;
    constexpr int NP = HnrIn<D>::NP;
    float a[NP], b[NP];
    float ss = 0.f;
#pragma unroll
    for (int t = 0; t < NP; ++t) {
        const int i = lane + 64 * t;
        a[t] = i < HALF ? bf(in.a[t]) : 0.f;
        b[t] = i < HALF ? bf(in.b[t]) : 0.f;
        ss += a[t] * a[t];
        ss += b[t] * b[t];
    }
    ss = wave_sum(ss);
    const float rs = rsqrtf(ss * (1.0f / (float)D) + eps);
#pragma unroll
    for (int t = 0; t < NP; ++t) {
        const int i = lane + 64 * t;
        if (i < HALF) {
            const float na = rbf(bf(in.wa[t]) * rbf(a[t] * rs));
            const float nb = rbf(bf(in.wb[t]) * rbf(b[t] * rs));
            const float lo = na * bf(in.ca[t]) + (-nb) * bf(in.sa[t]);
            const float hi = nb * bf(in.cb[t]) + na * bf(in.sb[t]);
            const uint16_t l16 = f32_to_bf16(lo), h16 = f32_to_bf16(hi);
            dst[i] = l16;
            dst[i + HALF] = h16;
            if (dst2) {
                dst2[i] = l16;
                dst2[i + HALF] = h16;
            }
        }
    }
}
template <int D>
__device__ __forceinline__ void head_norm_rope(const uint16_t* __restrict__ x, const uint16_t* __restrict__ nw,
                                               float eps, const uint16_t* __restrict__ cs,
                                               const uint16_t* __restrict__ sn, uint16_t* dst, uint16_t* dst2,
                                               int lane) {
    HnrIn<D> in;
    hnr_load<D>(x, nw, cs, sn, lane, in);
    hnr_finish<D>(in, eps, dst, dst2, lane);
}

__device__ __forceinline__ float silu_mul(float g, float u) {
    // silu(g) * u = g * sigmoid(g) * u, as kernels.py:68 (fp32)
    return g * (1.0f / (1.0f + __expf(-g))) * u;
}

}  // namespace wisp
