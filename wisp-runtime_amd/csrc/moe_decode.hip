// Batch-1 MoE layer kernels for gfx950: gate_up+SiLU (kernel 1) and down with
// the routing-weighted expert sum (kernel 2), reading packed 4/3/2-bit experts
// straight out of the slot pool.
//
// Reference semantics: wisp/kernels.py:12 (folded dequant
// sum_i (q_i s + m) v_i = s (q.v) + m sum(v)), 20-69 (_gate_up_kernel),
// 72-112 (_down_kernel), 140-185 (_down_sum_kernel), 206-307 (3-bit twins).
//
// Work decomposition (MI355X: 256 CUs, wave64):
//  * A lane owns one 32-code chunk of a row (16/12/8 bytes for 4/3/2-bit), so
//    the codes stream through 128/96/64-bit loads that are contiguous across
//    the wave. All loads of a wave are issued before any math.
//  * Kernel 1: one wave = one expert x T*RPI rows (gate and up), RPI = rows
//    per wave-wide load (1 when H = 2048). With a bf16 x a chunk dot is
//    16 v_and_or_b32 + 16 v_dot2c_f32_bf16 against x in pair order (exact
//    products); a fp16 or fp32 x is used as 32 fp32 values with one
//    v_fma_mix_f32 per code (chunk_dot_f32). Per-lane partials are summed per
//    row through LDS; SiLU(gate)*up is formed by the lane holding the row.
//  * The activation between the kernels is fp32 in natural order,
//    act[j*I + r] (the reference's fp32 `a`, kernels.py:133, 197, 316).
//  * Kernel 2: the activation chunk of a lane is 32 fp32 values staged in LDS;
//    the codes enter v_fma_mix_f32 as fp16 subnormals (chunk_dot_f32), so every
//    product q*a is exact and the sums are fp32, as the reference's are.
#include <mutex>

#include "wisp_device.hpp"
#include "wisp_internal.hpp"

#ifndef WISP_QSC
#define WISP_QSC 1
#endif

namespace wisp {

// Layer constants, computed once on the host (no divisions in the kernels).
struct Layer {
    const uint8_t* pool;
    const float* meta;
    int64_t slot_bytes;
    int64_t nmb;  // code bytes of one matrix, n*BITS/8
    int nslots, k;
    int H, I, G;
    int rowb_gu;  // code bytes of one gate/up row, H*BITS/8
    int rowb_dn;  // code bytes of one down row, I*BITS/8
    int gpr_gu;   // groups per gate/up row, H/G
    int gpr_dn;   // groups per down row, I/G
    int NGM;      // groups per matrix, n/G
    int gsh;      // log2(G/32) when G/32 is a power of two, else -1
    int spr_gu;   // chunks per gate/up row, H/32
    int spr_dn;   // chunks per down row, I/32
    int odt;      // output dtype of the weighted sum: WISP_DT_BF16, WISP_DT_F16 or WISP_DT_F32
};

// The layer constants of the Qwen3-30B-A3B expert shape (H = 2048, I = 768, G = 128) as compile-time
// constants: the kernels specialised on it take no Layer argument (every field they need is a constant or one
// of their preloaded scalar arguments), so nothing is read from kernel-argument memory before their weight
// loads; other shapes take the Layer as passed.
constexpr int kC2H = 2048, kC2I = 768, kC2G = 128;

template <int BITS>
__device__ __forceinline__ Layer layer_c2(const uint8_t* pool, const float* meta, int64_t slot_bytes, int nslots) {
    Layer c;
    c.pool = pool;
    c.meta = meta;
    c.slot_bytes = slot_bytes;
    c.nmb = (int64_t)kC2H * kC2I * BITS / 8;
    c.nslots = nslots;
    c.k = 0;  // taken from the kernel's own argument where needed
    c.H = kC2H;
    c.I = kC2I;
    c.G = kC2G;
    c.rowb_gu = kC2H * BITS / 8;
    c.rowb_dn = kC2I * BITS / 8;
    c.gpr_gu = kC2H / kC2G;
    c.gpr_dn = kC2I / kC2G;
    c.NGM = kC2H * kC2I / kC2G;
    c.gsh = 2;  // log2(G / 32)
    c.spr_gu = kC2H / 32;
    c.spr_dn = kC2I / 32;
    c.odt = WISP_DT_BF16;  // kernels of this shape take the output dtype as a template argument
    return c;
}

// out[h] = v rounded once (round to nearest even) to the caller's dtype
__device__ __forceinline__ void store_out(void* out, int odt, int h, float v) {
    if (odt == WISP_DT_F32)
        reinterpret_cast<float*>(out)[h] = v;
    else if (odt == WISP_DT_F16)
        reinterpret_cast<__half*>(out)[h] = __float2half_rn(v);
    else
        reinterpret_cast<uint16_t*>(out)[h] = f32_to_bf16(v);
}

// ---------------------------------------------------------------------------
// x in any of the three float types. XT: WISP_DT_BF16 (the native operand of the
// dot2 path), WISP_DT_F16 or WISP_DT_F32: those are converted to 32 fp32
// values per chunk (exact) for the fma path, so every product with x is exact,
// as the reference's fp32 loads of x (kernels.py:51-52) give.
// ---------------------------------------------------------------------------
template <int XT>
struct XWords {
    static constexpr int n = XT == WISP_DT_F32 ? 32 : 16;  // dwords of 32 values
};

// raw dwords of the 32 x values of chunk c
template <int XT>
__device__ __forceinline__ void load_x_raw(const void* x, int c, uint32_t* w) {
    const uint4* q = reinterpret_cast<const uint4*>(reinterpret_cast<const uint8_t*>(x) +
                                                    (int64_t)c * 32 * (XT == WISP_DT_F32 ? 4 : 2));
#pragma unroll
    for (int i = 0; i < XWords<XT>::n / 4; ++i) {
        const uint4 v = q[i];
        w[4 * i] = v.x; w[4 * i + 1] = v.y; w[4 * i + 2] = v.z; w[4 * i + 3] = v.w;
    }
}

// raw dwords -> 32 fp32 values in element order (exact for every XT)
template <int XT>
__device__ __forceinline__ void x_to_f32(const uint32_t* w, float* xf) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        if constexpr (XT == WISP_DT_F32) {
            xf[2 * i] = __uint_as_float(w[2 * i]);
            xf[2 * i + 1] = __uint_as_float(w[2 * i + 1]);
        } else if constexpr (XT == WISP_DT_F16) {
            xf[2 * i] = half_lo_f(w[i]);
            xf[2 * i + 1] = half_hi_f(w[i]);
        } else {
            xf[2 * i] = bf16_lo(w[i]);
            xf[2 * i + 1] = bf16_hi(w[i]);
        }
    }
}

// slot id from the meta buffer: -1 unless an exact integer in [0, nslots)
__device__ __forceinline__ int slot_from(float f, int nslots) {
    const int s = (int)f;
    return (f >= 0.f && f < (float)nslots && (float)s == f) ? s : -1;
}
__device__ __forceinline__ int slot_of(const float* meta, int j, int nslots) { return slot_from(meta[j], nslots); }

__device__ __forceinline__ void wave_sync_lds() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// a[j, r] into the fp32 activation workspace
__device__ __forceinline__ void write_act(float* act, int j, int I, int r, float a) { act[(int64_t)j * I + r] = a; }

// dot of one chunk of codes against one bf16 operand in pair order, bias removed: sum q*v.
// Even pairs accumulate from b0, odd pairs from b1. 3-bit: the operand scaled per half
// (operand_pairs), b0 = -128 * (sum of its values), b1 = 0. 4- and 2-bit: the operand as
// the x values are (operand_pairs<BITS, false>), each accumulator's pairs at one e in both
// halves (4-bit 3; 2-bit 3 for even pairs, 5 for odd ones), so each accumulator's dot is
// 2^e times the scaled form's and is scaled back here. 4-bit with b0 = -128 * (sum of the
// values), b1 = 0: every product, partial sum and the bias are exactly 8 times the scaled
// form's, so the result has the same bits (for |x| between about 2^-120 and 2^120: past
// those the scaled form's operands leave bf16's normal range, or the products fp32's, one
// step earlier than the other form's). 2-bit: b0 and b1 = -128 * (sum of the values
// of the even / odd pairs), each accumulator cancelling its own bias.
template <int BITS>
__device__ __forceinline__ float chunk_dot(const uint32_t* codes, const uint32_t* opr, float b0, float b1,
                                           uint32_t B) {
    uint32_t p[16];
    code_pairs<BITS>(codes, p, B);
    float a0 = b0, a1 = b1;
#pragma unroll
    for (int P = 0; P < 16; P += 2) {
        a0 = dot2(p[P], opr[P], a0);
        a1 = dot2(p[P + 1], opr[P + 1], a1);
    }
    if constexpr (BITS == 4) return (a0 + a1) * 0.125f;
    if constexpr (BITS == 2) return __builtin_fmaf(a1, 0.03125f, a0 * 0.125f);
    return a0 + a1;
}

// Sum the SPR partials of row-set q (LDS floats src[0..SPR)) across the LPS
// lanes of its lane group (LPS a power of two <= 16, groups aligned inside a
// 16-lane DPP row); every lane of the group gets the total. The cross-lane
// steps are DPP adds (quad_perm xor 1 / xor 2, row_half_mirror, row_mirror).
template <int SPR_T>
__device__ __forceinline__ float group_sum(const float* src, int SPR, int sub, int LPS) {
    float v = 0.f;
    if (SPR_T && SPR_T % LPS == 0) {  // contiguous VPL values per lane
        const int VPL = SPR_T / LPS;
        const float* p = src + sub * VPL;
        for (int i = 0; i < VPL; ++i) v += p[i];
    } else {  // strided; lanes with sub >= SPR add nothing
        for (int i = sub; i < SPR; i += LPS) v += src[i];
    }
    if (LPS >= 2) v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
    if (LPS >= 4) v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
    if (LPS >= 8) v += dpp_f<0x141>(v);  // row_half_mirror
    if (LPS >= 16) v += dpp_f<0x140>(v); // row_mirror
    return v;
}

// lanes per row-set sum for NQ sums over 64 lanes: a power of two, at most 16
__device__ __forceinline__ int lanes_per_sum(int NQ) {
    int LPS = 1;
    while (LPS < 16 && LPS * 2 * NQ <= 64) LPS <<= 1;
    return LPS;
}

// ===========================================================================
// Kernel 1 body (fast path): H/32 <= 64 chunks per row, G/32 a power of two.
// One wave computes rows r0 .. r0 + T*RPI - 1 of expert j (slot valid), where
// RPI = rows per wave-wide load (1 when H = 2048). SPR_T = H/32 when known at
// compile time (64 for H = 2048), 0 = runtime.
// QSC: the 4 lanes of a quad share one (row, group) (G >= 128, H/32 % 4 == 0):
//      each quad fetches its 4 fp16 values (gate s, gate m, up s, up m) with one
//      16-bit load per lane and shares them with DPP broadcasts.
// XF: x arrives as 32 fp32 values xf (fp16 / fp32 x, fma path); else as 16
//     bf16 pair words xw (dot2 path).
// FULL: H/32 == 64 and every row r0 .. r0 + T - 1 exists (the Qwen3 shape), so
//     no lane is idle and no row index needs a clamp.
// part: this wave's LDS scratch, T*2*64 floats.
// ===========================================================================
template <int BITS, int SPR_T, int T, bool QSC, bool XF, bool FULL = false>
// The lanes' x (chunk `seg` of x) is loaded by the caller before the slot id is
// known; `ok` false (invalid slot id) reads slot 0 and writes NaN rows.
__device__ __forceinline__ void gate_up_rows(const Layer& L, const uint8_t* __restrict__ base, bool ok,
                                             const uint32_t (&xw)[16], const float (&xf)[32],
                                             float* __restrict__ act, int j, int r0, float* part) {
    static_assert(!FULL || SPR_T == 64, "FULL needs one row per wave-wide load");
    const int SPR = SPR_T ? SPR_T : L.spr_gu;
    const int RPI = 64 / SPR;
    const int lane = threadIdx.x & 63;
    int rr = FULL ? 0 : lane / SPR;
    const int seg = lane - rr * SPR;
    const bool lane_on = FULL || rr < RPI;
    rr = lane_on ? rr : RPI - 1;  // idle lanes repeat an active lane's addresses
    const uint16_t* sc = reinterpret_cast<const uint16_t*>(base + 3 * L.nmb);
    const uint16_t* mn = sc + 3 * L.NGM;
    const int gi = seg >> L.gsh;

    // the weight codes and fp16 scale/min loads, all issued before any use
    uint32_t cg[T][BITS], cu[T][BITS];
    uint32_t sv[T][QSC ? 1 : 4];
#pragma unroll
    for (int t = 0; t < T; ++t) {
        const int r = FULL ? r0 + t : min(r0 + t * RPI + rr, L.I - 1);
        const uint8_t* rp = base + (int64_t)r * L.rowb_gu + seg * (4 * BITS);
        load_chunk<BITS>(rp, cg[t]);
        load_chunk<BITS>(rp + L.nmb, cu[t]);
        const int gidx = r * L.gpr_gu + gi;
        if (QSC) {
            const int w = lane & 3;  // 0 gate s, 1 gate m, 2 up s, 3 up m
            sv[t][0] = ((w & 1) ? mn : sc)[((w & 2) ? L.NGM : 0) + gidx];
        } else {
            sv[t][0] = sc[gidx];
            sv[t][1 % (QSC ? 1 : 4)] = mn[gidx];
            sv[t][2 % (QSC ? 1 : 4)] = sc[L.NGM + gidx];
            sv[t][3 % (QSC ? 1 : 4)] = mn[L.NGM + gidx];
        }
    }
    uint32_t xp[16];
    float xs, b0 = 0.f, b1 = 0.f;
    if constexpr (XF) {
        xs = chunk_sum_f32(xf);
    } else if constexpr (BITS == 3) {
        float vs;
        operand_pairs<BITS>(xw, xp);
        operand_sums<BITS>(xp, vs, xs);
        b0 = -kBiasF * vs;
    } else {
        // the x values as they are, one v_perm each; the biases as chunk_dot takes them
        operand_pairs<BITS, false>(xw, xp);
        float se = 0.f, so = 0.f;
#pragma unroll
        for (int P = 0; P < 16; P += 2) {
            se = dot2(xp[P], kOnes2, se);
            so = dot2(xp[P + 1], kOnes2, so);
        }
        xs = se + so;
        if constexpr (BITS == 4) {
            b0 = -kBiasF * xs;
        } else {
            b0 = -kBiasF * se;
            b1 = -kBiasF * so;
        }
    }
    const uint32_t B = bias_vgpr();
#pragma unroll
    for (int t = 0; t < T; ++t) {
        const bool ok = FULL || (lane_on && (r0 + t * RPI + rr < L.I));
        float dg, du;
        if constexpr (XF) {
            dg = chunk_dot_f32<BITS>(cg[t], xf);
            du = chunk_dot_f32<BITS>(cu[t], xf);
        } else {
            dg = chunk_dot<BITS>(cg[t], xp, b0, b1, B);
            du = chunk_dot<BITS>(cu[t], xp, b0, b1, B);
        }
        uint32_t s_g, m_g, s_u, m_u;
        if (QSC) {
            s_g = quad_bcast<0>(sv[t][0]);
            m_g = quad_bcast<1>(sv[t][0]);
            s_u = quad_bcast<2>(sv[t][0]);
            m_u = quad_bcast<3>(sv[t][0]);
        } else {
            s_g = sv[t][0];
            m_g = sv[t][1 % (QSC ? 1 : 4)];
            s_u = sv[t][2 % (QSC ? 1 : 4)];
            m_u = sv[t][3 % (QSC ? 1 : 4)];
        }
        const float pg = h2f((uint16_t)s_g) * dg + h2f((uint16_t)m_g) * xs;
        const float pu = h2f((uint16_t)s_u) * du + h2f((uint16_t)m_u) * xs;
        part[(2 * t) * 64 + lane] = ok ? pg : 0.f;
        part[(2 * t + 1) * 64 + lane] = ok ? pu : 0.f;
    }
    wave_sync_lds();

    // row sums: NQ = 2*T*RPI sums (gate/up interleaved) of SPR partials each
    const int NQ = 2 * T * RPI;
    const int LPS = lanes_per_sum(NQ);
    const int QPR = 64 / LPS;
    for (int q0 = 0; q0 < NQ; q0 += QPR) {
        const int q = q0 + lane / LPS;
        const int sub = lane & (LPS - 1);
        const int qq = q < NQ ? q : NQ - 1;
        const int m = qq & 1, row = qq >> 1, t = row / RPI, rq = row - t * RPI;
        const float v = group_sum<SPR_T>(part + (2 * t + m) * 64 + rq * SPR, SPR, sub, LPS);
        // the up sum of the same row sits LPS lanes higher, in the same DPP row when LPS <= 8
        float u;
        switch (LPS) {
        case 1: u = dpp_f<0x101>(v); break;  // row_shl:1
        case 2: u = dpp_f<0x102>(v); break;
        case 4: u = dpp_f<0x104>(v); break;
        case 8: u = dpp_f<0x108>(v); break;
        default: u = __shfl_down(v, LPS, 64); break;
        }
        if (q < NQ && sub == 0 && m == 0) {
            const int r = r0 + t * RPI + rq;
            if (FULL || r < L.I) write_act(act, j, L.I, r, ok ? silu_mul(v, u) : __builtin_nanf(""));
        }
    }
}

// x of this lane's chunk: raw words (bf16) or 32 fp32 values (fp16 / fp32)
template <int XT>
__device__ __forceinline__ void x_operand(const uint32_t* xr, uint32_t (&xw)[16], float (&xf)[32]) {
    if constexpr (XT == WISP_DT_BF16) {
#pragma unroll
        for (int i = 0; i < 16; ++i) xw[i] = xr[i];
    } else {
        x_to_f32<XT>(xr, xf);
    }
}

// Kernel 1 (fast path), two-kernel form, any shape with H/32 <= 64.
// grid = (ceil(I / (NW*T*RPI)), k), block = 64*NW.
// The leading scalar arguments are preloaded into SGPRs at dispatch (kernarg
// preloading, built with -amdgpu-kernarg-preload-count): the slot-id read and
// the x loads need no kernel-argument fetch first, so the only memory round
// trip before the weight loads is the slot id itself.
template <int BITS, int SPR_T, int T, int NW, bool QSC, int XT>
__global__ __launch_bounds__(64 * NW) void k_gate_up(const float* __restrict__ meta,
                                                      const uint8_t* __restrict__ pool, int64_t slot_bytes,
                                                      int nslots, const void* __restrict__ x,
                                                      float* __restrict__ act, const Layer L) {
    __shared__ float part[NW][T * 2 * 64];
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int j = blockIdx.y;
    // issue the slot-id read and the x loads together; the scheduling barrier keeps every use (and so every
    // wait) after them
    const float f = meta[j];
    uint32_t xr[XWords<XT>::n];
    load_x_raw<XT>(x, (threadIdx.x & 63) % (SPR_T ? SPR_T : L.spr_gu), xr);
    __builtin_amdgcn_sched_barrier(0);
    const int slot = __builtin_amdgcn_readfirstlane(slot_from(f, nslots));
    const bool ok = slot >= 0;
    const uint8_t* base = pool + (int64_t)(ok ? slot : 0) * slot_bytes;
    const int RPI = 64 / (SPR_T ? SPR_T : L.spr_gu);
    const int r0 = (blockIdx.x * NW + wv) * (T * RPI);
    uint32_t xw[16];
    float xf[32];
    x_operand<XT>(xr, xw, xf);
    gate_up_rows<BITS, SPR_T, T, QSC, XT != WISP_DT_BF16>(L, base, ok, xw, xf, act, j, r0, part[wv]);
}

// Kernel 1 at the Qwen3-30B-A3B shape: the same body with every shape field a compile-time constant and no
// Layer argument.
template <int BITS, int T, int NW, bool QSC, int XT>
__global__ __launch_bounds__(64 * NW) void k_gate_up_c2(const float* __restrict__ meta,
                                                         const uint8_t* __restrict__ pool, int64_t slot_bytes,
                                                         int nslots, const void* __restrict__ x,
                                                         float* __restrict__ act) {
    static_assert(kC2I % (NW * T) == 0, "every row of the grid exists (gate_up_rows FULL)");
    __shared__ float part[NW][T * 2 * 64];
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int j = blockIdx.y;
    const float f = meta[j];
    const Layer Lc = layer_c2<BITS>(pool, meta, slot_bytes, nslots);
    uint32_t xr[XWords<XT>::n];
    load_x_raw<XT>(x, threadIdx.x & 63, xr);
    __builtin_amdgcn_sched_barrier(0);
    const int slot = __builtin_amdgcn_readfirstlane(slot_from(f, nslots));
    const bool ok = slot >= 0;
    const uint8_t* base = pool + (int64_t)(ok ? slot : 0) * slot_bytes;
    const int r0 = (blockIdx.x * NW + wv) * T;
    uint32_t xw[16];
    float xf[32];
    x_operand<XT>(xr, xw, xf);
    gate_up_rows<BITS, 64, T, QSC, XT != WISP_DT_BF16, true>(Lc, base, ok, xw, xf, act, j, r0, part[wv]);
}

// Kernel 1 (generic): any H, G; one wave per (row, expert); x as fp32 values (exact for every x dtype).
template <int BITS, int XT>
__global__ __launch_bounds__(64) void k_gate_up_generic(const Layer L, const void* __restrict__ x,
                                                        float* __restrict__ act) {
    const int lane = threadIdx.x;
    const int r = blockIdx.x, j = blockIdx.y;
    const int slot = __builtin_amdgcn_readfirstlane(slot_of(L.meta, j, L.nslots));
    float pg = 0.f, pu = 0.f;
    if (slot >= 0) {
        const uint8_t* base = L.pool + (int64_t)slot * L.slot_bytes;
        const uint16_t* sc = reinterpret_cast<const uint16_t*>(base + 3 * L.nmb);
        const uint16_t* mn = sc + 3 * L.NGM;
        for (int c = lane; c < L.spr_gu; c += 64) {
            uint32_t cg[BITS], cu[BITS], xr[XWords<XT>::n];
            float xf[32];
            const uint8_t* rp = base + (int64_t)r * L.rowb_gu + c * (4 * BITS);
            load_chunk<BITS>(rp, cg);
            load_chunk<BITS>(rp + L.nmb, cu);
            load_x_raw<XT>(x, c, xr);
            x_to_f32<XT>(xr, xf);
            const float xs = chunk_sum_f32(xf);
            const int gidx = r * L.gpr_gu + (c * 32) / L.G;
            pg += h2f(sc[gidx]) * chunk_dot_f32<BITS>(cg, xf) + h2f(mn[gidx]) * xs;
            pu += h2f(sc[L.NGM + gidx]) * chunk_dot_f32<BITS>(cu, xf) + h2f(mn[L.NGM + gidx]) * xs;
        }
        pg = wave_sum(pg);
        pu = wave_sum(pu);
    } else {
        pg = pu = __builtin_nanf("");
    }
    if (lane == 0) write_act(act, j, L.I, r, silu_mul(pg, pu));
}

// ===========================================================================
// Kernel 2 body (fast path): I/32 <= 64 chunks per row, G/32 a power of two.
// One workgroup computes output rows h0 .. h0 + T*RPI - 1; wave j handles
// expert j (waves j >= k idle). SPR_T = I/32 when known at compile time (24
// for I = 768), 0 = runtime.
// QSC: quads share one (row, group) (G >= 128, I/32 % 4 == 0, T even): lane i
//      of a quad loads one of (s, m) for rows t and t+1; DPP broadcasts share them.
// Each wave stages its expert's fp32 activation (I values, 32-value segments
// at a stride of 36 words against bank conflicts) in LDS once, so a lane reads
// its 128-byte operand from LDS instead of from L2.
// lds: (k*T*64 + k*T*RPI + k*I*36/32) floats.
// WSUM: out[h] = sum_j w_j y_j[h] rounded once (wave j scales its row sums by
// w_j, loaded at the start); else y[j*H + h] = y_j[h].
// ===========================================================================
template <int BITS, int SPR_T, int T, bool WSUM, bool QSC>
// `meta`, `pool`, `slot_bytes`, `nslots`, `k` and `I` repeat fields of L as
// the kernel's preloaded scalar arguments (no kernel-argument fetch before the
// activation loads and the slot-id read). An invalid slot id reads slot 0 and
// yields NaN partials.
__device__ __forceinline__ void down_rows(const Layer& L, const float* meta,
                                          const uint8_t* __restrict__ pool, int64_t slot_bytes, int nslots, int k,
                                          int I, const float* __restrict__ act, void* __restrict__ out,
                                          float* __restrict__ y, int h0, float* lds) {
    static_assert(!QSC || T % 2 == 0, "quad-shared scales cover two rows per load");
    const int SPR = SPR_T ? SPR_T : L.spr_dn;
    const int RPI = 64 / SPR;
    const int RW = T * RPI;
    const int lane = threadIdx.x & 63;
    const int j = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // expert; the block has k waves
    int rr = lane / SPR;
    const int seg = lane - rr * SPR;
    const bool lane_on = rr < RPI;
    rr = lane_on ? rr : RPI - 1;
    float* part = lds + j * (T * 64);   // [T][64], this wave's partials (j < k)
    float* rows = lds + k * (T * 64);   // [k][RW]
    uint32_t* stage = reinterpret_cast<uint32_t*>(rows + k * RW) + (int64_t)j * (I / 32 * 36);

    {
        // issue the activation loads (their address needs no memory read), the
        // slot-id and weight reads from meta together; the scheduling barrier keeps
        // every use (and so every wait) after them
        const float f = meta[j];
        const float wj = WSUM ? meta[k + j] : 0.f;  // used at the end
        const uint4* asrc = reinterpret_cast<const uint4*>(act + (int64_t)j * I);
        const int na16 = I >> 2;
        constexpr int APL = SPR_T ? (SPR_T * 8 + 63) / 64 : 8;
        uint4 apiece[APL];
#pragma unroll
        for (int k2 = 0; k2 < APL; ++k2) apiece[k2] = asrc[min(lane + 64 * k2, na16 - 1)];
        __builtin_amdgcn_sched_barrier(0);
        const int slot = __builtin_amdgcn_readfirstlane(slot_from(f, nslots));
        const bool ok = slot >= 0;
        float p[T];
        {
            const uint8_t* base = pool + (int64_t)(ok ? slot : 0) * slot_bytes;
            const uint8_t* dcodes = base + 2 * L.nmb;
            const uint16_t* sc = reinterpret_cast<const uint16_t*>(base + 3 * L.nmb) + 2 * L.NGM;
            const uint16_t* mn = sc + 3 * L.NGM;
            const int gi = seg >> L.gsh;
            uint32_t cd[T][BITS], sv[T];
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const int h = min(h0 + t * RPI + rr, L.H - 1);
                load_chunk<BITS>(dcodes + (int64_t)h * L.rowb_dn + seg * (4 * BITS), cd[t]);
                if (QSC) {
                    if (t % 2 == 0) {
                        const int w = lane & 3;  // 0 s(t), 1 m(t), 2 s(t+1), 3 m(t+1)
                        const int hh = (w & 2) ? min(h0 + (t + 1) * RPI + rr, L.H - 1) : h;
                        sv[t] = ((w & 1) ? mn : sc)[hh * L.gpr_dn + gi];
                    }
                } else {
                    sv[t] = (uint32_t)sc[h * L.gpr_dn + gi] | ((uint32_t)mn[h * L.gpr_dn + gi] << 16);
                }
            }
            // stage expert j's activation in LDS, segment stride 36 words
#pragma unroll
            for (int k2 = 0; k2 < APL; ++k2) {
                const int i = min(lane + 64 * k2, na16 - 1);
                // halves swapped, so the compiler cannot fold the load and this store
                // into one copy placed here (the loads must stay at the kernel's start)
                const uint4 a = apiece[k2];
                reinterpret_cast<uint4*>(stage)[i + (i >> 3)] = make_uint4(a.z, a.w, a.x, a.y);
            }
            wave_sync_lds();
            float A[32];
            const uint4* ap = reinterpret_cast<const uint4*>(stage + seg * 36);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint4 v = ap[i];  // halves swapped in the stage
                A[4 * i] = __uint_as_float(v.z); A[4 * i + 1] = __uint_as_float(v.w);
                A[4 * i + 2] = __uint_as_float(v.x); A[4 * i + 3] = __uint_as_float(v.y);
            }
            const float as = chunk_sum_f32(A);
            // the sum uses the staged activation only: keep it ahead of every wait for the codes
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const bool row_ok = lane_on && (h0 + t * RPI + rr < L.H);
                const float d = chunk_dot_f32<BITS>(cd[t], A);
                uint32_t s_, m_;
                if (QSC) {
                    const uint32_t v2 = sv[t & ~1];
                    s_ = (t & 1) ? quad_bcast<2>(v2) : quad_bcast<0>(v2);
                    m_ = (t & 1) ? quad_bcast<3>(v2) : quad_bcast<1>(v2);
                } else {
                    s_ = sv[t] & 0xFFFFu;
                    m_ = sv[t] >> 16;
                }
                const float v = h2f((uint16_t)s_) * d + h2f((uint16_t)m_) * as;
                p[t] = !ok ? __builtin_nanf("") : (row_ok ? v : 0.f);
            }
        }
#pragma unroll
        for (int t = 0; t < T; ++t) part[t * 64 + lane] = p[t];
        wave_sync_lds();

        // per-wave row sums: RW sums of SPR partials each
        const int LPS = lanes_per_sum(RW);
        const int QPR = 64 / LPS;
        for (int q0 = 0; q0 < RW; q0 += QPR) {
            const int q = q0 + lane / LPS;
            const int sub = lane & (LPS - 1);
            const int qq = q < RW ? q : RW - 1;
            const int t = qq / RPI, rq = qq - t * RPI;
            const float v = group_sum<SPR_T>(part + t * 64 + rq * SPR, SPR, sub, LPS);
            if (q < RW && sub == 0) {
                if (WSUM) {
                    rows[j * RW + q] = wj * v;
                } else {
                    const int h = h0 + q;
                    if (h < L.H) y[(int64_t)j * L.H + h] = v;
                }
            }
        }
    }
    if (WSUM) {
        __syncthreads();
        for (int q = threadIdx.x; q < RW; q += 64 * k) {  // the block is k waves
            const int h = h0 + q;
            if (h < L.H) {
                float acc = 0.f;
                for (int jj = 0; jj < k; ++jj) acc += rows[jj * RW + q];
                store_out(out, L.odt, h, acc);
            }
        }
    }
}

// ===========================================================================
// Kernel 2 for the Qwen3-30B-A3B shape (I = 768, k <= 8, 4/3/2-bit codes),
// weighted sum: one wave computes RPW whole output rows over all k experts.
// Lane l takes the (expert, chunk) pairs l, l + 64 and l + 128 of a row's
// k x 24 pairs, so all 64 lanes work, each lane keeps its three activation
// chunks (32 fp32 values each) in registers for the wave's rows, and a row
// total is one in-register reduction (DPP within 16-lane rows, then the four
// rows) -- no exchange between waves, and every wave stores its own rows as
// soon as they are done. Sum order: the three pairs of a lane, then the lanes;
// the k expert weights are applied per pair. The fp32 activations of all k
// experts (24 KB) are staged in LDS once per workgroup. No Layer argument:
// every argument arrives preloaded in SGPRs. The output dtype ODT is a template
// argument: a branch on it between the rows would make the compiler wait for the
// first row's store before the second row's arithmetic. Default launch: one row
// per wave, 4 waves per workgroup, 512 workgroups (two waves per SIMD).
// ===========================================================================
template <int BITS, int RPW, int NWV, int ODT>
__global__ __launch_bounds__(64 * NWV) void k_down_rows(const float* meta, const uint8_t* __restrict__ pool,
                                                        int64_t slot_bytes, int nslots, int k,
                                                        const float* __restrict__ act, void* __restrict__ out) {
    constexpr int SEG = kC2I / 32, NC = 3, ROWB = kC2I * BITS / 8;
    constexpr int64_t NMB = (int64_t)kC2H * kC2I * BITS / 8;
    constexpr int NGM = kC2H * kC2I / kC2G, GPR = kC2I / kC2G;
    constexpr int ROWS_WG = RPW * NWV, NB = kC2H / ROWS_WG;
    constexpr bool QS = (RPW % 2) == 0;
    constexpr int CW = 9;  // uint4 per (expert, chunk): 8 of values + 1 pad
    __shared__ uint4 stage[8 * SEG * CW];
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    int rb = blockIdx.x;
    if ((NB & 7) == 0) rb = (rb & 7) * (NB >> 3) + (rb >> 3);
    const int h0 = rb * ROWS_WG + wv * RPW;

    // Each lane reads the slot ids and weights of its three pairs' experts from meta
    // itself (one round trip, no cross-lane broadcast between the slot ids' arrival and
    // the code loads), slot ids first, then the activations of all k experts (k * 192
    // uint4, staged in LDS below): waiting for the slot ids does not wait for the rest.
    constexpr int APT = (8 * SEG * 8 + 64 * NWV - 1) / (64 * NWV);
    const int na = k * SEG * 8;
    int ec[NC], sg[NC];
    bool on[NC], okc[NC];
    float fs[NC], fw[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int combo = lane + 64 * c;
        ec[c] = combo / SEG;
        sg[c] = combo - ec[c] * SEG;
        on[c] = ec[c] < k;
        fs[c] = meta[on[c] ? ec[c] : 0];
    }
#pragma unroll
    for (int c = 0; c < NC; ++c) fw[c] = meta[k + (on[c] ? ec[c] : 0)];
    const uint4* a4 = reinterpret_cast<const uint4*>(act);
    uint4 ap[APT];
#pragma unroll
    for (int i = 0; i < APT; ++i) {
        const int idx = threadIdx.x + i * 64 * NWV;
        ap[i] = a4[min(idx, na - 1)];
    }
    __builtin_amdgcn_sched_barrier(0);
    const uint8_t* bc[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int slot = slot_from(fs[c], nslots);
        okc[c] = slot >= 0;
        bc[c] = pool + (int64_t)(okc[c] ? slot : 0) * slot_bytes;
    }
    uint32_t cd[RPW][NC][BITS];
    uint32_t sv[QS ? RPW / 2 : RPW][NC];
#pragma unroll
    for (int t = 0; t < RPW; ++t) {
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const uint8_t* row = bc[c] + 2 * NMB + (int64_t)(h0 + t) * ROWB + sg[c] * (4 * BITS);
            load_chunk<BITS>(row, cd[t][c]);
            const uint16_t* sc = reinterpret_cast<const uint16_t*>(bc[c] + 3 * NMB) + 2 * NGM;
            const uint16_t* mn = sc + 3 * NGM;
            const int g = sg[c] >> 2;
            if constexpr (QS) {
                if (t % 2 == 0) {
                    const int w = lane & 3;
                    const int hh = h0 + t + ((w >> 1) & 1);
                    sv[t / 2][c] = ((w & 1) ? mn : sc)[hh * GPR + g];
                }
            } else {
                sv[t][c] = (uint32_t)sc[(h0 + t) * GPR + g] | ((uint32_t)mn[(h0 + t) * GPR + g] << 16);
            }
        }
    }
    // every code load is issued before the staging below: a register copy placed among them
    // would wait for an activation load first
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < APT; ++i) {
        // every thread stores (clamped: duplicates rewrite the same value), halves swapped: a plain
        // copy would let the compiler sink the load past the code loads, next to this store
        const int idx = min((int)threadIdx.x + i * 64 * NWV, na - 1);
        const uint4 a = ap[i];
        stage[(idx >> 3) * CW + (idx & 7)] = make_uint4(a.z, a.w, a.x, a.y);
    }
    __syncthreads();
    float A[NC][32];
    float as[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int e = on[c] ? ec[c] : 0;
        const uint4* q = stage + (e * SEG + sg[c]) * CW;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint4 v = q[i];  // halves swapped in the stage
            A[c][4 * i] = __uint_as_float(v.z); A[c][4 * i + 1] = __uint_as_float(v.w);
            A[c][4 * i + 2] = __uint_as_float(v.x); A[c][4 * i + 3] = __uint_as_float(v.y);
        }
        as[c] = chunk_sum_f32(A[c]);
    }
    float wc[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) wc[c] = on[c] ? fw[c] : 0.f;
    // everything above uses the staged activation and meta only: keep it ahead of every wait for
    // the codes
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < RPW; ++t) {
        float p = 0.f;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const float d = chunk_dot_f32<BITS>(cd[t][c], A[c]);
            uint32_t s_, m_;
            if constexpr (QS) {
                const uint32_t v2 = sv[t / 2][c];
                s_ = (t & 1) ? quad_bcast<2>(v2) : quad_bcast<0>(v2);
                m_ = (t & 1) ? quad_bcast<3>(v2) : quad_bcast<1>(v2);
            } else {
                s_ = sv[t][c] & 0xFFFFu;
                m_ = sv[t][c] >> 16;
            }
            const float v = h2f((uint16_t)s_) * d + h2f((uint16_t)m_) * as[c];
            p += !okc[c] && on[c] ? __builtin_nanf("") : wc[c] * v;
        }
        // row sums by DPP within each 16-lane row, then the four rows through readlane
        p += dpp_f<0xB1>(p);
        p += dpp_f<0x4E>(p);
        p += dpp_f<0x141>(p);
        p += dpp_f<0x140>(p);
        const float tot = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), 0)) +
                          __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), 16)) +
                          __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), 32)) +
                          __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), 48));
        if (lane == 0) store_out(out, ODT, h0 + t, tot);
    }
}

// Kernel 2 (fast path), two-kernel form.
// grid = ceil(H / (T*RPI)), block = 64*k, dynamic LDS as for down_rows.
template <int BITS, int SPR_T, int T, bool WSUM, bool QSC>
// The leading scalar arguments are preloaded into SGPRs at dispatch, as for
// k_gate_up.
__global__ __launch_bounds__(1024) void k_down(const float* meta, const uint8_t* __restrict__ pool,
                                               int64_t slot_bytes, int nslots, int k, int I,
                                               const float* __restrict__ act, void* __restrict__ out,
                                               float* __restrict__ y, const Layer L) {
    extern __shared__ float lds[];
    const int RW = T * (64 / (SPR_T ? SPR_T : L.spr_dn));
    // XCD-aware row blocks: the dispatcher deals workgroups to the 8 XCDs in turn, so
    // workgroup b runs on XCD b % 8; give each XCD one contiguous range of row blocks,
    // so the scale/min lines neighbouring blocks share are fetched into one L2 only
    // (the grid size from the shape: gridDim would be a kernel-argument memory read)
    int rb = blockIdx.x;
    const int G = (L.H + RW - 1) / RW;
    if ((G & 7) == 0) rb = (rb & 7) * (G >> 3) + (rb >> 3);
    down_rows<BITS, SPR_T, T, WSUM, QSC>(L, meta, pool, slot_bytes, nslots, k, I, act, out, y, rb * RW, lds);
}

// Kernel 2 at the Qwen3-30B-A3B shape (3- and 2-bit codes, per-expert y, k <= 16): k_down's body with the
// shape fields compile-time constants and no Layer argument; odt is the output dtype of the weighted sum.
template <int BITS, int T, bool WSUM, bool QSC>
__global__ __launch_bounds__(1024) void k_down_c2(const float* meta, const uint8_t* __restrict__ pool,
                                                  int64_t slot_bytes, int nslots, int k,
                                                  const float* __restrict__ act, void* __restrict__ out,
                                                  float* __restrict__ y, int odt) {
    extern __shared__ float lds[];
    Layer L = layer_c2<BITS>(pool, meta, slot_bytes, nslots);
    L.odt = odt;
    constexpr int RW = T * (64 / (kC2I / 32));
    constexpr int NBLK = (kC2H + RW - 1) / RW;
    int rb = blockIdx.x;
    if ((NBLK & 7) == 0) rb = (rb & 7) * (NBLK >> 3) + (rb >> 3);
    down_rows<BITS, kC2I / 32, T, WSUM, QSC>(L, meta, pool, slot_bytes, nslots, k, kC2I, act, out, y, rb * RW, lds);
}

// Kernel 2 (generic): any I, G and k; one workgroup of min(k, 16) waves per
// output row, wave w takes experts w, w + 16, ...; the k expert sums meet in
// LDS (dynamic, k floats) and are combined in expert order.
template <int BITS, bool WSUM>
__global__ __launch_bounds__(1024) void k_down_generic(const Layer L, const float* __restrict__ act,
                                                       void* __restrict__ out, float* __restrict__ y) {
    extern __shared__ float rows[];
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nw = blockDim.x >> 6;
    const int h = blockIdx.x;
    for (int j = w; j < L.k; j += nw) {
        const int slot = __builtin_amdgcn_readfirstlane(slot_of(L.meta, j, L.nslots));
        float v = 0.f;
        if (slot >= 0) {
            const uint8_t* base = L.pool + (int64_t)slot * L.slot_bytes;
            const uint16_t* sc = reinterpret_cast<const uint16_t*>(base + 3 * L.nmb) + 2 * L.NGM;
            const uint16_t* mn = sc + 3 * L.NGM;
            for (int c = lane; c < L.spr_dn; c += 64) {
                uint32_t cd[BITS];
                float A[32];
                load_chunk<BITS>(base + 2 * L.nmb + (int64_t)h * L.rowb_dn + c * (4 * BITS), cd);
                const float4* ap = reinterpret_cast<const float4*>(act + (int64_t)j * L.I + c * 32);
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const float4 q = ap[i];
                    A[4 * i] = q.x; A[4 * i + 1] = q.y; A[4 * i + 2] = q.z; A[4 * i + 3] = q.w;
                }
                const int gidx = h * L.gpr_dn + (c * 32) / L.G;
                v += h2f(sc[gidx]) * chunk_dot_f32<BITS>(cd, A) + h2f(mn[gidx]) * chunk_sum_f32(A);
            }
            v = wave_sum(v);
        } else {
            v = __builtin_nanf("");
        }
        if (WSUM) {
            if (lane == 0) rows[j] = v;
        } else if (lane == 0) {
            y[(int64_t)j * L.H + h] = v;
        }
    }
    if (WSUM) {
        __syncthreads();
        if (threadIdx.x == 0) {
            float acc = 0.f;
            for (int jj = 0; jj < L.k; ++jj) acc += L.meta[L.k + jj] * rows[jj];
            store_out(out, L.odt, h, acc);
        }
    }
}

// Workspace decode: the fp32 activation, copied
__global__ void k_act_read(const float* __restrict__ act, int64_t n, float* __restrict__ a) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) a[i] = act[i];
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
static int make_layer(Layer& L, const uint8_t* pool, int64_t slot_bytes, int64_t nslots, const float* meta, int k,
                      int64_t H, int64_t I, int bits, int64_t group) {
    if (!pool || !meta) return fail_inval("null pool or meta");
    if (!(bits == 4 || bits == 3 || bits == 2)) return fail_inval("bits must be 4, 3 or 2 for the fused kernels");
    if (k < 1 || k > WISP_MAX_K) return fail_inval("k must be in [1, WISP_MAX_K = 8192]");
    if (H <= 0 || I <= 0 || group <= 0 || H % group || I % group)
        return fail_inval("H and I must be positive multiples of group (kernels.py:118)");
    if (group % 32) return fail_inval("group must be a multiple of 32");
    if (H > (1 << 16) || I > (1 << 16)) return fail_inval("H, I must be <= 65536");
    const int64_t n = H * I;
    const int64_t nb = wisp_expert_nbytes(n, bits, group);
    if (nb < 0 || slot_bytes < nb) return fail_inval("slot_bytes is smaller than one expert");
    if (nslots < 1 || nslots > (1 << 24)) return fail_inval("nslots must be in [1, 2^24] (exact float ids)");
    const int al = bits == 3 ? 4 : 4 * bits;
    if (!aligned(pool, al) || slot_bytes % al) {
        set_error("pool base and slot_bytes must be %d-byte aligned for %d-bit experts", al, bits);
        return WISP_EALIGN;
    }
    L.pool = pool;
    L.meta = meta;
    L.slot_bytes = slot_bytes;
    L.nmb = n * bits / 8;
    L.nslots = (int)nslots;
    L.k = k;
    L.H = (int)H;
    L.I = (int)I;
    L.G = (int)group;
    L.rowb_gu = (int)(H * bits / 8);
    L.rowb_dn = (int)(I * bits / 8);
    L.gpr_gu = (int)(H / group);
    L.gpr_dn = (int)(I / group);
    L.NGM = (int)(n / group);
    const int cpg = (int)(group / 32);
    L.gsh = (cpg & (cpg - 1)) ? -1 : __builtin_ctz(cpg);
    L.spr_gu = (int)(H / 32);
    L.spr_dn = (int)(I / 32);
    L.odt = WISP_DT_BF16;
    return WISP_OK;
}

static bool valid_dtype(int dt) { return dt == WISP_DT_BF16 || dt == WISP_DT_F16 || dt == WISP_DT_F32; }

static bool is_c2(const Layer& L) { return L.H == kC2H && L.I == kC2I && L.G == kC2G; }

template <int BITS, int SPR, int T, int NW, bool QSC, int XT>
static void launch_gu(const Layer& L, const void* x, float* act, hipStream_t st) {
    const int RPI = 64 / L.spr_gu;
    const int rows_wg = NW * T * RPI;
    const dim3 grid((L.I + rows_wg - 1) / rows_wg, L.k);
    if (SPR == 64 && is_c2(L))
        hipLaunchKernelGGL((k_gate_up_c2<BITS, T, NW, QSC, XT>), grid, dim3(64 * NW), 0, st, L.meta, L.pool,
                           L.slot_bytes, L.nslots, x, act);
    else
        hipLaunchKernelGGL((k_gate_up<BITS, SPR, T, NW, QSC, XT>), grid, dim3(64 * NW), 0, st, L.meta, L.pool,
                           L.slot_bytes, L.nslots, x, act, L);
}

template <int BITS, int XT>
static int gate_up_bits(const Layer& L, const void* x, float* act, hipStream_t st) {
    if (L.spr_gu > 64 || L.gsh < 0) {
        hipLaunchKernelGGL((k_gate_up_generic<BITS, XT>), dim3(L.I, L.k), dim3(64), 0, st, L, x, act);
        return check_launch("k_gate_up_generic");
    }
    if (L.spr_gu != 64 || L.gsh < 2) {
        launch_gu<BITS, 0, 2, 4, false, XT>(L, x, act, st);
        return check_launch("k_gate_up");
    }
    if constexpr (XT != WISP_DT_BF16) {
        // fp16 / fp32 x: the default launch shape only
        launch_gu<BITS, 64, 2, 4, (bool)WISP_QSC, XT>(L, x, act, st);
        return check_launch("k_gate_up");
    } else {
        const Tuning& tu = tuning();
#define WISP_GU(TT, WW)                                                 \
    if (tu.gu_rows == TT && tu.gu_waves == WW) {                        \
        launch_gu<BITS, 64, TT, WW, (bool)WISP_QSC, XT>(L, x, act, st); \
        return check_launch("k_gate_up");                               \
    }
        WISP_GU(2, 4)
        WISP_GU(4, 4)
        WISP_GU(8, 4)
        WISP_GU(1, 4)
        WISP_GU(4, 2)
        WISP_GU(2, 8)
        WISP_GU(4, 1)
        WISP_GU(8, 1)
#undef WISP_GU
        return fail_inval("unsupported tuning (gu_rows, gu_waves)");
    }
}

// dynamic LDS of the fast kernel 2 with T row iterations (see down_rows)
static size_t dn_lds_bytes(const Layer& L, int T) {
    const int RW = T * (64 / L.spr_dn);
    return sizeof(float) * ((size_t)L.k * T * 64 + (size_t)L.k * RW + (size_t)L.k * (L.I / 32 * 36));
}

template <int BITS, int SPR, int T, bool WSUM, bool QSC>
static void launch_dn(const Layer& L, const float* act, void* out, float* y, hipStream_t st) {
    const int RW = T * (64 / L.spr_dn);
    const size_t lds = dn_lds_bytes(L, T);
    const dim3 grid((L.H + RW - 1) / RW), block(64 * L.k);
    if (SPR == 24 && is_c2(L))
        hipLaunchKernelGGL((k_down_c2<BITS, T, WSUM, QSC>), grid, block, lds, st, L.meta, L.pool, L.slot_bytes,
                           L.nslots, L.k, act, out, y, L.odt);
    else
        hipLaunchKernelGGL((k_down<BITS, SPR, T, WSUM, QSC>), grid, block, lds, st, L.meta, L.pool, L.slot_bytes,
                           L.nslots, L.k, L.I, act, out, y, L);
}

template <int BITS, bool WSUM>
static int down_bits(const Layer& L, const float* act, void* out, float* y, hipStream_t st) {
    // the fast path has one wave per expert (k <= 16) and stages k*I activation
    // values in LDS: keep the whole LDS within 64 KB
    const bool tuned = L.spr_dn == 24 && L.gsh >= 2;
    if (L.k > 16 || L.spr_dn > 64 || L.gsh < 0 || dn_lds_bytes(L, tuned ? tuning().dn_iters : 4) > 65536) {
        const int nw = L.k < 16 ? L.k : 16;
        hipLaunchKernelGGL((k_down_generic<BITS, WSUM>), dim3(L.H), dim3(64 * nw), WSUM ? sizeof(float) * L.k : 0, st,
                           L, act, out, y);
        return check_launch("k_down_generic");
    }
    if (!tuned) {
        launch_dn<BITS, 0, 4, WSUM, false>(L, act, out, y, st);
        return check_launch("k_down");
    }
    switch (tuning().dn_iters) {
    case 1: launch_dn<BITS, 24, 1, WSUM, false>(L, act, out, y, st); break;
    case 2: launch_dn<BITS, 24, 2, WSUM, (bool)WISP_QSC>(L, act, out, y, st); break;
    case 4:
        if (WSUM && is_c2(L) && L.k <= 8) {  // the default tuning of the C2 shape: the row kernel
            constexpr int RPW = 1, NWV = 4;
            const dim3 grid(kC2H / (RPW * NWV)), block(64 * NWV);
            if (L.odt == WISP_DT_F32)
                hipLaunchKernelGGL((k_down_rows<BITS, RPW, NWV, WISP_DT_F32>), grid, block, 0, st, L.meta, L.pool,
                                   L.slot_bytes, L.nslots, L.k, act, out);
            else if (L.odt == WISP_DT_F16)
                hipLaunchKernelGGL((k_down_rows<BITS, RPW, NWV, WISP_DT_F16>), grid, block, 0, st, L.meta, L.pool,
                                   L.slot_bytes, L.nslots, L.k, act, out);
            else
                hipLaunchKernelGGL((k_down_rows<BITS, RPW, NWV, WISP_DT_BF16>), grid, block, 0, st, L.meta, L.pool,
                                   L.slot_bytes, L.nslots, L.k, act, out);
            return check_launch("k_down_rows");
        }
        launch_dn<BITS, 24, 4, WSUM, (bool)WISP_QSC>(L, act, out, y, st);
        break;
    case 8: launch_dn<BITS, 24, 8, WSUM, (bool)WISP_QSC>(L, act, out, y, st); break;
    default: return fail_inval("unsupported tuning dn_iters");
    }
    return check_launch("k_down");
}

template <int XT>
static int gate_up_xt(const Layer& L, int bits, const void* x, float* act, hipStream_t st) {
    switch (bits) {
    case 4: return gate_up_bits<4, XT>(L, x, act, st);
    case 3: return gate_up_bits<3, XT>(L, x, act, st);
    default: return gate_up_bits<2, XT>(L, x, act, st);
    }
}

// kernel 1 of a validated layer
static int gate_up_launch(const Layer& L, int bits, const void* x, int x_dtype, float* act, hipStream_t st) {
    switch (x_dtype) {
    case WISP_DT_F16: return gate_up_xt<WISP_DT_F16>(L, bits, x, act, st);
    case WISP_DT_F32: return gate_up_xt<WISP_DT_F32>(L, bits, x, act, st);
    default: return gate_up_xt<WISP_DT_BF16>(L, bits, x, act, st);
    }
}

// kernel 2 of a validated layer: weighted sum into out (L.odt) when out, else per-expert y
static int down_launch(const Layer& L, int bits, const float* act, void* out, float* y, hipStream_t st) {
    if (out) {
        switch (bits) {
        case 4: return down_bits<4, true>(L, act, out, nullptr, st);
        case 3: return down_bits<3, true>(L, act, out, nullptr, st);
        default: return down_bits<2, true>(L, act, out, nullptr, st);
        }
    }
    switch (bits) {
    case 4: return down_bits<4, false>(L, act, nullptr, y, st);
    case 3: return down_bits<3, false>(L, act, nullptr, y, st);
    default: return down_bits<2, false>(L, act, nullptr, y, st);
    }
}

static int check_x(const void* x, int x_dtype) {
    if (!x) return fail_inval("null x");
    if (!valid_dtype(x_dtype)) return fail_inval("x_dtype must be WISP_DT_BF16, WISP_DT_F16 or WISP_DT_F32");
    if (!aligned(x, 16)) {
        set_error("x must be 16-byte aligned");
        return WISP_EALIGN;
    }
    return WISP_OK;
}

static int check_act(const void* act) {
    if (!act) return fail_inval("null act");
    if (!aligned(act, 16)) {
        set_error("act must be 16-byte aligned");
        return WISP_EALIGN;
    }
    return WISP_OK;
}

// ---------------------------------------------------------------------------
// Allocation-free layer (wisp_moe_decode_noalloc): the activation workspace
// between the two kernels is a file-scope device array instead of a caller
// buffer. Each GPU holds its own copy until the process ends; its address on
// a device comes from hipGetSymbolAddress (with that device current), taken
// once per device and kept. In host code `scratch` names a host-side
// stand-in, never a device address: only the kept pointer is passed on.
// ---------------------------------------------------------------------------
static __device__ __align__(256) uint32_t scratch[WISP_NOALLOC_MAX_ACT];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static uint32_t* g_scratch_ptr[kMaxDevices] = {};

// The device address of `scratch` on the current device (looked up once).
static int scratch_ptr(hipStream_t st, uint32_t** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        set_error("hipGetDevice: %s", hipGetErrorString(e));
        return (int)e;
    }
    if (dev < 0 || dev >= kMaxDevices) return fail_inval("device index beyond the no-alloc scratch table");
    if (st) {
        int sdev = -1;
        e = hipStreamGetDevice(st, &sdev);
        if (e != hipSuccess) {
            set_error("hipStreamGetDevice: %s", hipGetErrorString(e));
            return (int)e;
        }
        if (sdev != dev) return fail_inval("the stream's device must be the current device");
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            set_error("hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
            return e != hipSuccess ? (int)e : WISP_EINVAL;
        }
        g_scratch_ptr[dev] = static_cast<uint32_t*>(p);
    }
    *out = g_scratch_ptr[dev];
    return WISP_OK;
}

}  // namespace wisp

using namespace wisp;

extern "C" int64_t wisp_act_bytes(int k, int64_t I) {
    if (k < 1 || I <= 0) return -1;
    return (int64_t)k * I * 4;
}

extern "C" int wisp_moe_gate_up(const uint8_t* pool, int64_t slot_bytes, int64_t nslots, const float* meta, int k,
                                const void* x, int x_dtype, int64_t H, int64_t I, int bits, int64_t group,
                                uint32_t* act, void* stream) {
    clear_error();
    Layer L;
    int rc = make_layer(L, pool, slot_bytes, nslots, meta, k, H, I, bits, group);
    if (!rc) rc = check_x(x, x_dtype);
    if (!rc) rc = check_act(act);
    if (rc) return rc;
    return gate_up_launch(L, bits, x, x_dtype, reinterpret_cast<float*>(act), (hipStream_t)stream);
}

extern "C" int wisp_moe_down_sum(const uint8_t* pool, int64_t slot_bytes, int64_t nslots, const float* meta, int k,
                                 const uint32_t* act, int64_t H, int64_t I, int bits, int64_t group, void* out,
                                 int out_dtype, void* stream) {
    clear_error();
    Layer L;
    int rc = make_layer(L, pool, slot_bytes, nslots, meta, k, H, I, bits, group);
    if (!rc) rc = check_act(act);
    if (rc) return rc;
    if (!out) return fail_inval("null out");
    if (!valid_dtype(out_dtype)) return fail_inval("out_dtype must be WISP_DT_BF16, WISP_DT_F16 or WISP_DT_F32");
    L.odt = out_dtype;
    return down_launch(L, bits, reinterpret_cast<const float*>(act), out, nullptr, (hipStream_t)stream);
}

extern "C" int wisp_moe_down(const uint8_t* pool, int64_t slot_bytes, int64_t nslots, const float* meta, int k,
                             const uint32_t* act, int64_t H, int64_t I, int bits, int64_t group, float* y,
                             void* stream) {
    clear_error();
    Layer L;
    int rc = make_layer(L, pool, slot_bytes, nslots, meta, k, H, I, bits, group);
    if (!rc) rc = check_act(act);
    if (rc) return rc;
    if (!y) return fail_inval("null y");
    return down_launch(L, bits, reinterpret_cast<const float*>(act), nullptr, y, (hipStream_t)stream);
}

extern "C" int wisp_moe_decode(const uint8_t* pool, int64_t slot_bytes, int64_t nslots, const float* meta, int k,
                               const void* x, int x_dtype, int64_t H, int64_t I, int bits, int64_t group,
                               uint32_t* act, void* out, int out_dtype, void* stream) {
    const int rc = wisp_moe_gate_up(pool, slot_bytes, nslots, meta, k, x, x_dtype, H, I, bits, group, act, stream);
    if (rc) return rc;
    return wisp_moe_down_sum(pool, slot_bytes, nslots, meta, k, act, H, I, bits, group, out, out_dtype, stream);
}

extern "C" int wisp_moe_decode_noalloc(const uint8_t* pool, int64_t slot_bytes, int64_t nslots, const float* meta,
                                       int k, const void* x, int x_dtype, int64_t H, int64_t I, int bits, int64_t group,
                                       void* out, int out_dtype, void* stream) {
    clear_error();
    Layer L;
    int rc = make_layer(L, pool, slot_bytes, nslots, meta, k, H, I, bits, group);
    if (!rc) rc = check_x(x, x_dtype);
    if (rc) return rc;
    if (!out) return fail_inval("null out");
    if (!valid_dtype(out_dtype)) return fail_inval("out_dtype must be WISP_DT_BF16, WISP_DT_F16 or WISP_DT_F32");
    if ((int64_t)k * I > WISP_NOALLOC_MAX_ACT)
        return fail_inval("k*I exceeds the no-alloc scratch (WISP_NOALLOC_MAX_ACT = 262144 activation values)");
    hipStream_t st = (hipStream_t)stream;
    uint32_t* act = nullptr;
    rc = scratch_ptr(st, &act);
    if (rc) return rc;
    // kernel 1 writes every activation value kernel 2 reads: nothing in the
    // scratch has to start at zero
    rc = gate_up_launch(L, bits, x, x_dtype, reinterpret_cast<float*>(act), st);
    if (rc) return rc;
    L.odt = out_dtype;
    return down_launch(L, bits, reinterpret_cast<const float*>(act), out, nullptr, st);
}

extern "C" int wisp_act_read(const uint32_t* act, int k, int64_t I, int bits, float* a, void* stream) {
    clear_error();
    if (!act || !a) return fail_inval("null pointer");
    if (k < 1 || I <= 0 || I % 32) return fail_inval("k >= 1 and I a positive multiple of 32");
    if (!(bits == 4 || bits == 3 || bits == 2)) return fail_inval("bits must be 4, 3 or 2");
    const int64_t total = (int64_t)k * I;
    const dim3 grid((unsigned)((total + 255) / 256));
    hipLaunchKernelGGL(k_act_read, grid, dim3(256), 0, (hipStream_t)stream, reinterpret_cast<const float*>(act), total,
                       a);
    return check_launch("k_act_read");
}
