/*
 * CPU oracle for the fused group-wise expert dequant+GEMV path.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker that the HIP kernels are
 * compared against; it is never linked into, loaded by or called from the
 * product library (wisp-runtime_amd/). Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may use it.
 *
 * It restates, in plain C with IEEE single/double arithmetic, the algorithm of
 * the reference (imronpuji/wisp-runtime):
 *   - expert buffer layout and size ........ wisp/quant.py:1-8, 17-22
 *   - code packing / unpacking (8/4/3/2) ... wisp/quant.py:25-57
 *   - RTN min-max quantize ................. wisp/quant.py:60-73
 *   - dequant to bf16 ...................... wisp/quant.py:76-87
 *   - 3-bit field read used by the kernels . wisp/kernels.py:206-217
 *   - fused MoE decode semantics ........... wisp/kernels.py:12, 20-69,
 *                                            72-112, 137, 140-185, 220-307
 *   - decode rotary embedding .............. wisp/kernels.py:325-349
 *
 * Build: see oracle/Makefile (gcc -O2 -ffp-contract=off: no FMA contraction,
 * so every float expression rounds exactly where the reference's torch ops
 * round).
 *
 * Pinning (each function is checked by something other than itself; in
 * tests/test_oracle.py, and against the reference's own outputs in
 * tests/test_golden.py):
 *   wo_f32_to_f16 / wo_f32_to_bf16 / wo_*_to_f32 .. torch's own conversions on
 *       random, tie, subnormal, overflow and NaN inputs
 *   wo_expert_nbytes ... reference KATs (test_quant.py:39-40, architecture.md:82)
 *   wo_pack / wo_unpack  hand-derived byte KATs for 4/3/2-bit, round trips
 *   wo_q3_field ........ the kernel's 3-bit read formula (kernels.py:206-217)
 *                        evaluated independently for every element
 *   wo_quantize ........ hand-derived KATs (half-even ties, constant group,
 *                        1e-5 clamp), nearest-level property, reference error
 *                        bounds and monotonicity (test_quant.py:15-34); the
 *                        reference quantize's bytes (sha256, 12 experts)
 *   wo_dequant ......... hand KATs incl. the fp32-then-bf16 double rounding,
 *                        numpy float32 elementwise semantics; the reference
 *                        dequant's bf16 output (sha256, 12 experts)
 *   wo_moe_layer_f64 ... dense numpy dequant->matvec (the unfolded form) at
 *                        several shapes and bit widths; the reference kernels'
 *                        outputs (q4, q4_fast, q3_fast), every element equal
 *                        under the fixture's bf16 rounding
 *   wo_rope ............ hand KAT (d = 2: complex multiplication), rotation
 *                        preserves the norm and composes (angle addition),
 *                        float64 textbook rotate-half formula; the reference
 *                        rope_decode's fp32 and bf16 outputs, bit for bit
 * No function is parity-unpinned.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define WO_EXPORT __attribute__((visibility("default")))

/* ------------------------------------------------------------------------ */
/* scalar conversions                                                        */
/* ------------------------------------------------------------------------ */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* IEEE binary32 -> binary16, round to nearest even, with subnormals,
 * overflow to infinity and quiet NaN. (torch Tensor.half(), quant.py:70) */
WO_EXPORT uint16_t wo_f32_to_f16(float f) {
    uint32_t x = f2u(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ex = (x >> 23) & 0xFFu;
    uint32_t man = x & 0x7FFFFFu;
    if (ex == 0xFFu) return (uint16_t)(sign | 0x7C00u | (man ? 0x200u : 0u));
    if (ex == 0) return (uint16_t)sign; /* fp32 subnormal << fp16 min subnormal */
    int e = (int)ex - 127 + 15;         /* biased fp16 exponent */
    uint32_t m = man | 0x800000u;       /* 24-bit significand */
    if (e >= 1) {
        uint32_t keep = m >> 13, rem = m & 0x1FFFu;
        if (rem > 0x1000u || (rem == 0x1000u && (keep & 1u))) keep++;
        /* keep is in [0x400, 0x800]; 0x800 carries into the exponent */
        uint32_t bits = ((uint32_t)e << 10) + (keep - 0x400u);
        if (bits >= 0x7C00u) return (uint16_t)(sign | 0x7C00u);
        return (uint16_t)(sign | bits);
    }
    /* fp16 subnormal (or zero): value = m * 2^(e-1-10-13) */
    int shift = 14 - e; /* 13 + (1 - e) */
    if (shift >= 32) return (uint16_t)sign;
    uint32_t keep = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (keep & 1u))) keep++;
    return (uint16_t)(sign | keep); /* keep == 0x400 is the min normal */
}

/* binary16 -> binary32 (exact). */
WO_EXPORT float wo_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t ex = ((uint32_t)h >> 10) & 0x1Fu;
    uint32_t man = (uint32_t)h & 0x3FFu;
    if (ex == 0x1Fu) return u2f(sign | 0x7F800000u | (man << 13));
    if (ex == 0) {
        if (man == 0) return u2f(sign);
        /* subnormal: man * 2^-24 */
        float v = (float)man * 5.9604644775390625e-08f; /* 2^-24, exact */
        return sign ? -v : v;
    }
    return u2f(sign | ((ex + 112u) << 23) | (man << 13));
}

/* binary32 -> bfloat16, round to nearest even (torch .to(torch.bfloat16),
 * quant.py:87). Integer-add formulation of RTNE; NaN -> quiet NaN. */
WO_EXPORT uint16_t wo_f32_to_bf16(float f) {
    uint32_t x = f2u(f);
    if ((x & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((x >> 16) | 0x40u);
    uint32_t bias = 0x7FFFu + ((x >> 16) & 1u);
    return (uint16_t)((x + bias) >> 16);
}

WO_EXPORT float wo_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

/* ------------------------------------------------------------------------ */
/* layout (quant.py:1-8, 17-22)                                              */
/* ------------------------------------------------------------------------ */

/* Bytes of one expert = [codes 3n*bits/8 | fp16 scales 3n/G | fp16 mins 3n/G];
 * bits == 16 is raw bf16. Returns -1 on an invalid (n, bits, group). */
WO_EXPORT int64_t wo_expert_nbytes(int64_t n, int bits, int64_t group) {
    if (n <= 0) return -1;
    if (bits == 16) return 3 * n * 2;
    if (!(bits == 8 || bits == 4 || bits == 3 || bits == 2)) return -1;
    if (group <= 0 || (3 * n) % group != 0 || (3 * n * bits) % 8 != 0) return -1;
    return (3 * n * bits) / 8 + 4 * (3 * n / group);
}

/* ------------------------------------------------------------------------ */
/* packing (quant.py:25-57)                                                  */
/* ------------------------------------------------------------------------ */

/* q: m codes (< 2^bits), m a multiple of the pack unit -> packed bytes.
 * 4-bit: element e is the low nibble of byte e/2 when e is even, else the high
 * nibble (quant.py:29-31). 2-bit: 4 per byte, LSB first (32-34). 3-bit: 8 codes
 * -> 24-bit little-endian -> 3 bytes, element e at bit 3e (35-40). */
WO_EXPORT int wo_pack(const uint8_t* q, int64_t m, int bits, uint8_t* out) {
    if (bits == 8) { memcpy(out, q, (size_t)m); return 0; }
    if (bits == 4) {
        if (m % 2) return -1;
        for (int64_t i = 0; i < m / 2; i++) out[i] = (uint8_t)(q[2 * i] | (q[2 * i + 1] << 4));
        return 0;
    }
    if (bits == 2) {
        if (m % 4) return -1;
        for (int64_t i = 0; i < m / 4; i++)
            out[i] = (uint8_t)(q[4 * i] | (q[4 * i + 1] << 2) | (q[4 * i + 2] << 4) | (q[4 * i + 3] << 6));
        return 0;
    }
    if (bits == 3) {
        if (m % 8) return -1;
        for (int64_t t = 0; t < m / 8; t++) {
            uint32_t v = 0;
            for (int i = 0; i < 8; i++) v |= (uint32_t)q[8 * t + i] << (3 * i);
            out[3 * t] = (uint8_t)(v & 255u);
            out[3 * t + 1] = (uint8_t)((v >> 8) & 255u);
            out[3 * t + 2] = (uint8_t)((v >> 16) & 255u);
        }
        return 0;
    }
    return -1;
}

/* Inverse of wo_pack: m codes out of packed bytes (quant.py:44-57). */
WO_EXPORT int wo_unpack(const uint8_t* c, int64_t m, int bits, uint8_t* out) {
    if (bits == 8) { memcpy(out, c, (size_t)m); return 0; }
    if (bits == 4) {
        for (int64_t e = 0; e < m; e++) out[e] = (e & 1) ? (c[e >> 1] >> 4) : (c[e >> 1] & 15);
        return 0;
    }
    if (bits == 2) {
        for (int64_t e = 0; e < m; e++) out[e] = (c[e >> 2] >> (2 * (e & 3))) & 3;
        return 0;
    }
    if (bits == 3) {
        if (m % 8) return -1;
        for (int64_t t = 0; t < m / 8; t++) {
            uint32_t v = (uint32_t)c[3 * t] | ((uint32_t)c[3 * t + 1] << 8) | ((uint32_t)c[3 * t + 2] << 16);
            for (int i = 0; i < 8; i++) out[8 * t + i] = (uint8_t)((v >> (3 * i)) & 7u);
        }
        return 0;
    }
    return -1;
}

/* The 3-bit field read exactly as the reference kernels state it
 * (kernels.py:209, 211-217): q = ((b[p>>3] | b[(p>>3)+1] << 8) >> (p & 7)) & 7,
 * p = 3e. A second, independent statement of the 3-bit layout. The caller
 * guarantees b[(p>>3)+1] is inside the expert buffer (it is for every code of
 * a bits<16 buffer: the scales follow the codes). */
WO_EXPORT int wo_q3_field(const uint8_t* b, int64_t e) {
    int64_t p = 3 * e;
    uint32_t lo = b[p >> 3], hi = b[(p >> 3) + 1];
    return (int)((((hi << 8) | lo) >> (p & 7)) & 7u);
}

/* code e of a packed stream (flat over the 3n elements) */
static inline uint32_t code_at(const uint8_t* c, int64_t e, int bits) {
    switch (bits) {
    case 8: return c[e];
    case 4: return (e & 1) ? (uint32_t)(c[e >> 1] >> 4) : (uint32_t)(c[e >> 1] & 15);
    case 2: return (uint32_t)(c[e >> 2] >> (2 * (e & 3))) & 3u;
    default: { /* 3 */
        int64_t p = 3 * e;
        int sh = (int)(p & 7);
        uint32_t v = c[p >> 3];
        if (sh > 5) v |= (uint32_t)c[(p >> 3) + 1] << 8;
        return (v >> sh) & 7u;
    }
    }
}

/* ------------------------------------------------------------------------ */
/* quantize (quant.py:60-73)                                                 */
/* ------------------------------------------------------------------------ */

/* w3: 3n float32 values (gate [I,H] | up [I,H] | down [H,I], flat) -> nbytes.
 * Per group of `group` consecutive values, in IEEE binary32:
 *   mn = min, mx = max
 *   scale = max((mx - mn) / levels, 1e-5f)            (quant.py:67-69)
 *   s16 = half(scale), m16 = half(mn)                 (quant.py:70)
 *   q = clamp(round_half_even((g - float(m16)) / float(s16)), 0, levels)
 *                                                     (quant.py:71)
 *   out = packed q | s16 bytes | m16 bytes            (quant.py:72-73)
 * bits == 16 stores the bf16 rounding of w3 (quant.py:63-64). */
WO_EXPORT int wo_quantize(const float* w3, int64_t n, int bits, int64_t group, uint8_t* out,
                          uint8_t* scratch_codes /* 3n bytes, may be NULL for bits 16 */) {
    int64_t nb = wo_expert_nbytes(n, bits, group);
    if (nb < 0) return -1;
    int64_t N = 3 * n;
    if (bits == 16) {
        for (int64_t i = 0; i < N; i++) {
            uint16_t b = wo_f32_to_bf16(w3[i]);
            out[2 * i] = (uint8_t)(b & 255u);
            out[2 * i + 1] = (uint8_t)(b >> 8);
        }
        return 0;
    }
    const float levels = (float)((1 << bits) - 1);
    const float eps = 1e-5f;
    int64_t ng = N / group;
    int64_t ncode = (N * bits) / 8;
    uint8_t* sc = out + ncode;
    uint8_t* mnb = out + ncode + 2 * ng;
    for (int64_t g = 0; g < ng; g++) {
        const float* v = w3 + g * group;
        float mn = v[0], mx = v[0];
        for (int64_t i = 1; i < group; i++) {
            if (v[i] < mn) mn = v[i];
            if (v[i] > mx) mx = v[i];
        }
        float diff = mx - mn;
        float s = diff / levels;
        if (s < eps) s = eps;
        uint16_t s16 = wo_f32_to_f16(s), m16 = wo_f32_to_f16(mn);
        float sf = wo_f16_to_f32(s16), mf = wo_f16_to_f32(m16);
        for (int64_t i = 0; i < group; i++) {
            float t = v[i] - mf;
            float r = t / sf;
            float q = nearbyintf(r); /* default rounding mode: half to even */
            if (q < 0.f) q = 0.f;
            if (q > levels) q = levels;
            scratch_codes[g * group + i] = (uint8_t)q;
        }
        sc[2 * g] = (uint8_t)(s16 & 255u);
        sc[2 * g + 1] = (uint8_t)(s16 >> 8);
        mnb[2 * g] = (uint8_t)(m16 & 255u);
        mnb[2 * g + 1] = (uint8_t)(m16 >> 8);
    }
    return wo_pack(scratch_codes, N, bits, out);
}

/* ------------------------------------------------------------------------ */
/* dequant (quant.py:76-87)                                                  */
/* ------------------------------------------------------------------------ */

static inline float scale_at(const uint8_t* buf, int64_t ncode, int64_t g) {
    return wo_f16_to_f32((uint16_t)(buf[ncode + 2 * g] | (buf[ncode + 2 * g + 1] << 8)));
}
static inline float min_at(const uint8_t* buf, int64_t ncode, int64_t ng, int64_t g) {
    return wo_f16_to_f32((uint16_t)(buf[ncode + 2 * ng + 2 * g] | (buf[ncode + 2 * ng + 2 * g + 1] << 8)));
}

/* One expert buffer -> 3n bf16 bit patterns.
 * w = float(q) * float(s)  (binary32, rounded)
 *   + float(m)             (binary32, rounded)   -- two ops, not an FMA
 * then round-to-nearest-even to bf16 (quant.py:86-87). */
WO_EXPORT int wo_dequant(const uint8_t* buf, int64_t n, int bits, int64_t group, uint16_t* out) {
    int64_t nb = wo_expert_nbytes(n, bits, group);
    if (nb < 0) return -1;
    int64_t N = 3 * n;
    if (bits == 16) {
        for (int64_t i = 0; i < N; i++) out[i] = (uint16_t)(buf[2 * i] | (buf[2 * i + 1] << 8));
        return 0;
    }
    int64_t ng = N / group, ncode = (N * bits) / 8;
    for (int64_t g = 0; g < ng; g++) {
        float s = scale_at(buf, ncode, g), m = min_at(buf, ncode, ng, g);
        for (int64_t i = 0; i < group; i++) {
            int64_t e = g * group + i;
            float t = (float)code_at(buf, e, bits) * s;
            float w = t + m;
            out[e] = wo_f32_to_bf16(w);
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* fused MoE decode semantics in binary64                                    */
/* ------------------------------------------------------------------------ */

/* Row dot of matrix `mat` (0 gate, 1 up, 2 down) of one expert buffer against
 * v (binary64), folded per group as the kernels do (kernels.py:12, 57-61):
 *   sum_c  s_c * (q . v)_c + m_c * (sum v)_c
 * Exact in binary64 up to rounding of the fp64 sums. */
static double row_dot(const uint8_t* buf, int64_t n, int bits, int64_t group, int mat, int64_t row,
                      int64_t len, const double* v) {
    int64_t N = 3 * n, ng = N / group, ncode = (N * bits) / 8;
    int64_t e0 = (int64_t)mat * n + row * len;
    double acc = 0.0;
    for (int64_t c0 = 0; c0 < len; c0 += group) {
        int64_t g = (e0 + c0) / group;
        double qv = 0.0, sv = 0.0;
        for (int64_t i = 0; i < group; i++) {
            qv += (double)code_at(buf, e0 + c0 + i, bits) * v[c0 + i];
            sv += v[c0 + i];
        }
        acc += (double)scale_at(buf, ncode, g) * qv + (double)min_at(buf, ncode, ng, g) * sv;
    }
    return acc;
}

/* One MoE layer at batch 1 (kernels.py:115-137 / 188-203 / 310-322 semantics):
 *   a[j,r] = silu(Wg_j[r].x) * (Wu_j[r].x)                       (20-69)
 *   y[j,h] = Wd_j[h].a_j                                          (72-112)
 *   out[h] = sum_j w_j * y[j,h]   (j in order 0..k-1)             (140-185)
 * pool: nslots rows of slot_bytes; slots[k]; w[k] routing weights as the
 * kernels see them (fp32 values of the bf16-rounded weights, moe.py:72);
 * xd: H values of x in binary64 (the reference kernels widen x of any float
 * type to fp32 exactly, kernels.py:51-52). Outputs (any may be NULL): a [k*I],
 * y [k*H], out [H], all binary64 and unrounded. Returns 0, or -1 on bad
 * arguments. */
WO_EXPORT int wo_moe_layer_f64x(const uint8_t* pool, int64_t slot_bytes, int64_t nslots, const int64_t* slots,
                                const float* w, int k, const double* xd, int64_t H, int64_t I, int bits,
                                int64_t group, double* a_out, double* y_out, double* out) {
    if (!(bits == 8 || bits == 4 || bits == 3 || bits == 2)) return -1;
    if (H <= 0 || I <= 0 || H % group || I % group) return -1;
    int64_t n = H * I;
    if (wo_expert_nbytes(n, bits, group) < 0 || wo_expert_nbytes(n, bits, group) > slot_bytes) return -1;
    double* ad = (double*)malloc(sizeof(double) * (size_t)I);
    if (!ad) return -1;
    if (out)
        for (int64_t h = 0; h < H; h++) out[h] = 0.0;
    for (int j = 0; j < k; j++) {
        if (slots[j] < 0 || slots[j] >= nslots) { free(ad); return -1; }
        const uint8_t* buf = pool + slots[j] * slot_bytes;
        for (int64_t r = 0; r < I; r++) {
            double g = row_dot(buf, n, bits, group, 0, r, H, xd);
            double u = row_dot(buf, n, bits, group, 1, r, H, xd);
            double a = g / (1.0 + exp(-g)) * u;
            ad[r] = a;
            if (a_out) a_out[(int64_t)j * I + r] = a;
        }
        for (int64_t h = 0; h < H; h++) {
            double y = row_dot(buf, n, bits, group, 2, h, I, ad);
            if (y_out) y_out[(int64_t)j * H + h] = y;
            if (out) out[h] += (double)w[j] * y;
        }
    }
    free(ad);
    return 0;
}

/* wo_moe_layer_f64x with x given as H bf16 bit patterns. */
WO_EXPORT int wo_moe_layer_f64(const uint8_t* pool, int64_t slot_bytes, int64_t nslots, const int64_t* slots,
                               const float* w, int k, const uint16_t* x, int64_t H, int64_t I, int bits,
                               int64_t group, double* a_out, double* y_out, double* out) {
    if (H <= 0) return -1;
    double* xd = (double*)malloc(sizeof(double) * (size_t)H);
    if (!xd) return -1;
    for (int64_t i = 0; i < H; i++) xd[i] = (double)wo_bf16_to_f32(x[i]);
    int rc = wo_moe_layer_f64x(pool, slot_bytes, nslots, slots, w, k, xd, H, I, bits, group, a_out, y_out, out);
    free(xd);
    return rc;
}

/* ------------------------------------------------------------------------ */
/* rotary embedding of one decode token (kernels.py:325-349)                */
/* ------------------------------------------------------------------------ */

/* x [nh, d] binary32 head vectors (already widened from their storage type),
 * cs/sn [d]; out[h, i] = x[i]*cs[i] + sign(i)*x[(i + d/2) % d]*sn[i] with
 * sign = -1 for i < d/2, else +1 (kernels.py:332-346). Each product and the
 * sum round separately in binary32 (this file builds with -ffp-contract=off). */
WO_EXPORT int wo_rope(const float* x, int64_t nh, int d, const float* cs, const float* sn, float* out) {
    if (nh < 0 || d < 2 || d % 2) return -1;
    const int half = d / 2;
    for (int64_t h = 0; h < nh; h++) {
        const float* xv = x + h * d;
        float* o = out + h * d;
        for (int i = 0; i < d; i++) {
            const int p = (i + half) % d;
            const float sign = i < half ? -1.0f : 1.0f;
            const float t1 = xv[i] * cs[i];
            const float t2 = (sign * xv[p]) * sn[i];
            o[i] = t1 + t2;
        }
    }
    return 0;
}
