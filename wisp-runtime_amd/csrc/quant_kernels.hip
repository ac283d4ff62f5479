// Format kernels for gfx950: bit-exact dequant (rows -> bf16), RTN group
// quantize, and code pack/unpack.
//
// Reference semantics: wisp/quant.py:17-22 (size), 25-57 (_pack/_unpack),
// 60-73 (quantize), 76-87 (dequant). Bit-exactness rules:
//  * dequant: w = float(q)*float(s) then + float(m), two separately rounded
//    binary32 ops, then round-to-nearest-even to bf16 (v_cvt_pk_bf16_f32).
//    q*s is exact in binary32 (q < 256, s an fp16 value: at most 8 + 11
//    significant bits), so rounding it changes nothing; the kernels are
//    written with plain operators under `#pragma clang fp contract(off)`,
//    which keeps mul and add separate in the ISA. The 4- and 2-bit chunk
//    path instead uses dequant32 (wisp_device.hpp), one fused multiply-add
//    with the exact product q*s: the same single rounding of q*s + m.
//  * quantize: binary32 sub/div with __fsub_rn/__fdiv_rn (IEEE, correctly
//    rounded), round-half-even (rintf), fp16 RTNE conversion with subnormals.
// Dequant is HBM-bound: it reads nbytes and writes 6n bytes per expert.
#include "wisp_device.hpp"
#include "wisp_internal.hpp"

namespace wisp {

// 32 codes of chunk c out of the packed stream (BITS in {8,4,3,2});
// chunk c starts at byte c*4*BITS.
template <int BITS>
__device__ __forceinline__ void unpack32(const uint8_t* codes, int64_t c, uint32_t* q) {
    if constexpr (BITS == 8) {
        const uint4* p = reinterpret_cast<const uint4*>(codes + c * 32);
        const uint4 a = p[0], b = p[1];
        const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int i = 0; i < 32; ++i) q[i] = (w[i >> 2] >> (8 * (i & 3))) & 255u;
    } else {
        uint32_t d[BITS];
        load_chunk<BITS>(codes + c * 4 * BITS, d);
        chunk_codes<BITS>(d, q);
    }
}

// one thread = one chunk of 32 codes of one expert row; G % 32 == 0
template <int BITS>
__global__ __launch_bounds__(256) void k_dequant(const uint8_t* __restrict__ rows, int64_t row_stride,
                                                 const int64_t* __restrict__ row_index, int64_t nbound, int64_t n,
                                                 int G, uint16_t* __restrict__ out) {
#pragma clang fp contract(off)
    const int64_t N = 3 * n;
    const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (c * 32 >= N) return;
    const int64_t b = blockIdx.y;
    const int64_t idx = row_index ? row_index[b] : b;
    uint4* o = reinterpret_cast<uint4*>(out + b * N + c * 32);
    if (idx < 0 || idx >= nbound) {
        const uint32_t nan2 = 0x7FC07FC0u;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = make_uint4(nan2, nan2, nan2, nan2);
        return;
    }
    const uint8_t* buf = rows + idx * row_stride;
    const int64_t ncode = N * BITS / 8;
    const int64_t ng = N / G;
    const int64_t g = (c * 32) / G;
    const uint16_t* sc = reinterpret_cast<const uint16_t*>(buf + ncode);
    uint32_t w[16];
    if constexpr (BITS == 4 || BITS == 2) {  // the same routine as the prefill kernels' B fragments
        uint32_t d[BITS];
        load_chunk<BITS>(buf + c * 4 * BITS, d);
        dequant32<BITS>(d, (uint32_t)sc[g] | ((uint32_t)sc[ng + g] << 16), w);
    } else {
        const float s = h2f(sc[g]), m = h2f(sc[ng + g]);
        uint32_t q[32];
        unpack32<BITS>(buf, c, q);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float a = (float)q[2 * i] * s + m;
            const float bb = (float)q[2 * i + 1] * s + m;
            w[i] = pack_bf16x2(a, bb);
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = make_uint4(w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]);
}

// generic group size: one thread = one element
template <int BITS>
__global__ __launch_bounds__(256) void k_dequant_any(const uint8_t* __restrict__ rows, int64_t row_stride,
                                                     const int64_t* __restrict__ row_index, int64_t nbound,
                                                     int64_t n, int64_t G, uint16_t* __restrict__ out) {
#pragma clang fp contract(off)
    const int64_t N = 3 * n;
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= N) return;
    const int64_t b = blockIdx.y;
    const int64_t idx = row_index ? row_index[b] : b;
    if (idx < 0 || idx >= nbound) {
        out[b * N + e] = 0x7FC0u;
        return;
    }
    const uint8_t* buf = rows + idx * row_stride;
    const int64_t ncode = N * BITS / 8;
    const int64_t ng = N / G;
    const int64_t g = e / G;
    uint32_t q;
    if (BITS == 8) {
        q = buf[e];
    } else if (BITS == 4) {
        q = (buf[e >> 1] >> (4 * (e & 1))) & 15u;
    } else if (BITS == 2) {
        q = (buf[e >> 2] >> (2 * (e & 3))) & 3u;
    } else {
        const int64_t p = 3 * e;
        const uint32_t lo = buf[p >> 3], hi = buf[(p >> 3) + 1];  // inside the buffer: scales follow the codes
        q = (((hi << 8) | lo) >> (p & 7)) & 7u;
    }
    const uint16_t* sc = reinterpret_cast<const uint16_t*>(buf + ncode);
    const float v = (float)q * h2f(sc[g]) + h2f(sc[ng + g]);
    out[b * N + e] = f32_to_bf16(v);
}

// Quantize: one wave per group of G values (any G <= 4096, 3n % G == 0).
// codes are staged per wave in LDS, then packed.
template <int BITS, bool BF16_IN>
__global__ __launch_bounds__(256) void k_quantize(const void* __restrict__ w3, int64_t n, int G,
                                                  uint8_t* __restrict__ out) {
#pragma clang fp contract(off)
    extern __shared__ uint8_t qbuf[];  // [4 waves][G]
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int64_t N = 3 * n;
    const int64_t ng = N / G;
    const int64_t g = (int64_t)blockIdx.x * 4 + wv;
    if (g >= ng) return;  // whole wave leaves together; no block barrier below
    uint8_t* qs = qbuf + wv * G;
    const int64_t e0 = g * G;
    auto ld = [&](int64_t e) -> float {
        if (BF16_IN) return bf16_to_f32(reinterpret_cast<const uint16_t*>(w3)[e]);
        return reinterpret_cast<const float*>(w3)[e];
    };
    float mn = __builtin_huge_valf(), mx = -__builtin_huge_valf();
    for (int i = lane; i < G; i += 64) {
        const float v = ld(e0 + i);
        mn = fminf(mn, v);
        mx = fmaxf(mx, v);
    }
    mn = wave_min(mn);
    mx = wave_max(mx);
    const float levels = (float)((1 << BITS) - 1);
    float scale = __fdiv_rn(__fsub_rn(mx, mn), levels);
    scale = scale < 1e-5f ? 1e-5f : scale;  // clamp_min(1e-5) in binary32
    const __half s16 = __float2half_rn(scale), m16 = __float2half_rn(mn);
    const float sf = __half2float(s16), mf = __half2float(m16);
    for (int i = lane; i < G; i += 64) {
        float q = rintf(__fdiv_rn(__fsub_rn(ld(e0 + i), mf), sf));  // round half to even
        q = q < 0.f ? 0.f : (q > levels ? levels : q);
        qs[i] = (uint8_t)q;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int64_t ncode = N * BITS / 8;
    uint8_t* dst = out + e0 * BITS / 8;
    if (BITS == 8) {
        for (int i = lane; i < G; i += 64) dst[i] = qs[i];
    } else if (BITS == 4) {
        for (int i = lane; i < G / 2; i += 64) dst[i] = (uint8_t)(qs[2 * i] | (qs[2 * i + 1] << 4));
    } else if (BITS == 2) {
        for (int i = lane; i < G / 4; i += 64)
            dst[i] = (uint8_t)(qs[4 * i] | (qs[4 * i + 1] << 2) | (qs[4 * i + 2] << 4) | (qs[4 * i + 3] << 6));
    } else {
        for (int t = lane; t < G / 8; t += 64) {
            uint32_t v = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) v |= (uint32_t)qs[8 * t + i] << (3 * i);
            dst[3 * t] = (uint8_t)(v & 255u);
            dst[3 * t + 1] = (uint8_t)((v >> 8) & 255u);
            dst[3 * t + 2] = (uint8_t)((v >> 16) & 255u);
        }
    }
    if (lane == 0) {
        uint16_t* sc = reinterpret_cast<uint16_t*>(out + ncode);
        sc[g] = __half_as_ushort(s16);
        sc[ng + g] = __half_as_ushort(m16);
    }
}

// pack: one thread per pack unit (2, 4 or 8 codes)
template <int BITS>
__global__ void k_pack(const uint8_t* __restrict__ q, int64_t units, uint8_t* __restrict__ out) {
    const int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (u >= units) return;
    if (BITS == 4) {
        out[u] = (uint8_t)(q[2 * u] | (q[2 * u + 1] << 4));
    } else if (BITS == 2) {
        out[u] = (uint8_t)(q[4 * u] | (q[4 * u + 1] << 2) | (q[4 * u + 2] << 4) | (q[4 * u + 3] << 6));
    } else if (BITS == 3) {
        uint32_t v = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) v |= (uint32_t)q[8 * u + i] << (3 * i);
        out[3 * u] = (uint8_t)(v & 255u);
        out[3 * u + 1] = (uint8_t)((v >> 8) & 255u);
        out[3 * u + 2] = (uint8_t)((v >> 16) & 255u);
    } else {
        out[u] = q[u];
    }
}

template <int BITS>
__global__ void k_unpack(const uint8_t* __restrict__ c, int64_t units, uint8_t* __restrict__ out) {
    const int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (u >= units) return;
    if (BITS == 4) {
        const uint8_t b = c[u];
        out[2 * u] = b & 15;
        out[2 * u + 1] = b >> 4;
    } else if (BITS == 2) {
        const uint8_t b = c[u];
#pragma unroll
        for (int i = 0; i < 4; ++i) out[4 * u + i] = (b >> (2 * i)) & 3;
    } else if (BITS == 3) {
        const uint32_t v = (uint32_t)c[3 * u] | ((uint32_t)c[3 * u + 1] << 8) | ((uint32_t)c[3 * u + 2] << 16);
#pragma unroll
        for (int i = 0; i < 8; ++i) out[8 * u + i] = (uint8_t)((v >> (3 * i)) & 7u);
    } else {
        out[u] = c[u];
    }
}

}  // namespace wisp

using namespace wisp;

extern "C" int wisp_dequant(const uint8_t* rows, int64_t row_stride, const int64_t* row_index, int64_t nrows,
                            int64_t nbound, int64_t n, int bits, int64_t group, uint16_t* out, void* stream) {
    clear_error();
    if (!rows || !out) return fail_inval("null rows or out");
    if (!(bits == 8 || bits == 4 || bits == 3 || bits == 2)) return fail_inval("bits must be 8, 4, 3 or 2");
    const int64_t nb = wisp_expert_nbytes(n, bits, group);
    if (nb < 0) return fail_inval("(n, bits, group) is not a valid expert shape (quant.py:21)");
    if (row_stride < nb) return fail_inval("row_stride is smaller than one expert");
    if (nrows < 0 || nrows > 65535) return fail_inval("nrows must be in [0, 65535]");
    if (nbound < 1) return fail_inval("nbound must be >= 1");
    if (nrows == 0) return WISP_OK;
    hipStream_t st = (hipStream_t)stream;
    const int64_t N = 3 * n;
    const bool fast = group % 32 == 0 && aligned(out, 16) && (N % 32) == 0 &&
                      aligned(rows, bits == 3 ? 4 : (bits == 8 ? 16 : 4 * bits)) &&
                      row_stride % (bits == 3 ? 4 : (bits == 8 ? 16 : 4 * bits)) == 0;
    if (fast) {
        const int64_t chunks = N / 32;
        const dim3 grid((unsigned)((chunks + 255) / 256), (unsigned)nrows);
#define WISP_DQ(B) \
    hipLaunchKernelGGL(k_dequant<B>, grid, dim3(256), 0, st, rows, row_stride, row_index, nbound, n, (int)group, out)
        switch (bits) {
        case 8: WISP_DQ(8); break;
        case 4: WISP_DQ(4); break;
        case 3: WISP_DQ(3); break;
        default: WISP_DQ(2); break;
        }
#undef WISP_DQ
        return check_launch("k_dequant");
    }
    const dim3 grid((unsigned)((N + 255) / 256), (unsigned)nrows);
#define WISP_DQA(B) \
    hipLaunchKernelGGL(k_dequant_any<B>, grid, dim3(256), 0, st, rows, row_stride, row_index, nbound, n, group, out)
    switch (bits) {
    case 8: WISP_DQA(8); break;
    case 4: WISP_DQA(4); break;
    case 3: WISP_DQA(3); break;
    default: WISP_DQA(2); break;
    }
#undef WISP_DQA
    return check_launch("k_dequant_any");
}

extern "C" int wisp_quantize(const void* w3, int w_dtype, int64_t n, int bits, int64_t group, uint8_t* out,
                             void* stream) {
    clear_error();
    if (!w3 || !out) return fail_inval("null w3 or out");
    if (!(bits == 8 || bits == 4 || bits == 3 || bits == 2)) return fail_inval("bits must be 8, 4, 3 or 2");
    if (w_dtype != 0 && w_dtype != 1) return fail_inval("w_dtype must be 0 (float32) or 1 (bfloat16)");
    if (wisp_expert_nbytes(n, bits, group) < 0) return fail_inval("(n, bits, group) is not a valid expert shape");
    if (group > 4096) return fail_inval("group must be <= 4096");
    if ((group * bits) % 8) return fail_inval("group*bits must be a multiple of 8");
    hipStream_t st = (hipStream_t)stream;
    const int64_t ng = 3 * n / group;
    const dim3 grid((unsigned)((ng + 3) / 4));
    const size_t lds = 4 * (size_t)group;
    const int G = (int)group;
#define WISP_Q(B)                                                                                      \
    if (w_dtype) hipLaunchKernelGGL((k_quantize<B, true>), grid, dim3(256), lds, st, w3, n, G, out); \
    else hipLaunchKernelGGL((k_quantize<B, false>), grid, dim3(256), lds, st, w3, n, G, out)
    switch (bits) {
    case 8: WISP_Q(8); break;
    case 4: WISP_Q(4); break;
    case 3: WISP_Q(3); break;
    default: WISP_Q(2); break;
    }
#undef WISP_Q
    return check_launch("k_quantize");
}

extern "C" int wisp_pack(const uint8_t* q, int64_t nq, int bits, uint8_t* out, void* stream) {
    clear_error();
    if (!q || !out) return fail_inval("null pointer");
    const int per = bits == 4 ? 2 : bits == 2 ? 4 : bits == 3 ? 8 : bits == 8 ? 1 : 0;
    if (!per) return fail_inval("bits must be 8, 4, 3 or 2");
    if (nq < 0 || nq % per) return fail_inval("nq must be a multiple of the pack unit");
    const int64_t units = nq / per;
    if (!units) return WISP_OK;
    const dim3 grid((unsigned)((units + 255) / 256));
    hipStream_t st = (hipStream_t)stream;
    switch (bits) {
    case 4: hipLaunchKernelGGL(k_pack<4>, grid, dim3(256), 0, st, q, units, out); break;
    case 3: hipLaunchKernelGGL(k_pack<3>, grid, dim3(256), 0, st, q, units, out); break;
    case 2: hipLaunchKernelGGL(k_pack<2>, grid, dim3(256), 0, st, q, units, out); break;
    default: hipLaunchKernelGGL(k_pack<8>, grid, dim3(256), 0, st, q, units, out); break;
    }
    return check_launch("k_pack");
}

extern "C" int wisp_unpack(const uint8_t* packed, int64_t nq, int bits, uint8_t* out, void* stream) {
    clear_error();
    if (!packed || !out) return fail_inval("null pointer");
    const int per = bits == 4 ? 2 : bits == 2 ? 4 : bits == 3 ? 8 : bits == 8 ? 1 : 0;
    if (!per) return fail_inval("bits must be 8, 4, 3 or 2");
    if (nq < 0 || nq % per) return fail_inval("nq must be a multiple of the pack unit");
    const int64_t units = nq / per;
    if (!units) return WISP_OK;
    const dim3 grid((unsigned)((units + 255) / 256));
    hipStream_t st = (hipStream_t)stream;
    switch (bits) {
    case 4: hipLaunchKernelGGL(k_unpack<4>, grid, dim3(256), 0, st, packed, units, out); break;
    case 3: hipLaunchKernelGGL(k_unpack<3>, grid, dim3(256), 0, st, packed, units, out); break;
    case 2: hipLaunchKernelGGL(k_unpack<2>, grid, dim3(256), 0, st, packed, units, out); break;
    default: hipLaunchKernelGGL(k_unpack<8>, grid, dim3(256), 0, st, packed, units, out); break;
    }
    return check_launch("k_unpack");
}
