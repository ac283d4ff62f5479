// Rotary position embedding for one decode token, q and k heads in one launch.
//
// Reference semantics: wisp/kernels.py:325-371 (_rope_kernel / rope_decode):
// for head vector x of length D, partner p(i) = (i + D/2) mod D and
// sign(i) = -1 for i < D/2, +1 otherwise,
//     out[i] = x[i] * cos[i] + sign(i) * x[p(i)] * sin[i]
// in binary32 from inputs widened to binary32, rounded once to the output
// type. The two products and the sum are rounded separately here (no FMA
// contraction; checked in the ISA: v_mul_f32 x2 + v_add_f32), so the result
// is reproducible bit for bit.
//
// One wave per head (Hq + Hk workgroups of 64 threads); lane t handles the
// element pairs (i, i + D/2) for i = t, t + 64, ..., which are each other's
// partners, so every input element is read once.
#include "wisp_device.hpp"
#include "wisp_internal.hpp"

namespace wisp {

template <typename T>
__device__ __forceinline__ float ld(const T* p, int64_t i);
template <>
__device__ __forceinline__ float ld<uint16_t>(const uint16_t* p, int64_t i) {
    return __uint_as_float((uint32_t)p[i] << 16);
}
template <>
__device__ __forceinline__ float ld<float>(const float* p, int64_t i) {
    return p[i];
}

template <typename T>
__device__ __forceinline__ void st(T* p, int64_t i, float v);
template <>
__device__ __forceinline__ void st<uint16_t>(uint16_t* p, int64_t i, float v) {
    p[i] = f32_to_bf16(v);
}
template <>
__device__ __forceinline__ void st<float>(float* p, int64_t i, float v) {
    p[i] = v;
}

template <typename T>
__global__ __launch_bounds__(64) void k_rope(const T* __restrict__ q, int64_t sq, const T* __restrict__ k, int64_t sk,
                                             const T* __restrict__ cs, const T* __restrict__ sn, int hq, int d,
                                             T* __restrict__ qo, T* __restrict__ ko) {
#pragma clang fp contract(off)
    const int h = blockIdx.x;
    const bool is_q = h < hq;
    const T* x = is_q ? q + (int64_t)h * sq : k + (int64_t)(h - hq) * sk;
    T* o = is_q ? qo + (int64_t)h * d : ko + (int64_t)(h - hq) * d;
    const int half = d >> 1;
    for (int i = threadIdx.x; i < half; i += 64) {
        const float a = ld(x, i), b = ld(x, i + half);
        // plain operators under contract(off): the header intrinsics (__fmul_rn, ...) would
        // still be fused into v_fma_f32 after inlining
        const float lo = a * ld(cs, i) + (-b) * ld(sn, i);
        const float hi = b * ld(cs, i + half) + a * ld(sn, i + half);
        st(o, i, lo);
        st(o, i + half, hi);
    }
}

}  // namespace wisp

using namespace wisp;

// kernels.py:352-371 (rope_decode)
extern "C" int wisp_rope_decode(const void* q, int64_t q_head_stride, const void* k, int64_t k_head_stride,
                                const void* cos, const void* sin, int hq, int hk, int d, int dtype, void* qo,
                                void* ko, void* stream) {
    clear_error();
    if (!q || !cos || !sin || !qo || (hk > 0 && (!k || !ko))) return fail_inval("null pointer");
    if (hq < 1 || hk < 0 || d < 2 || d % 2) return fail_inval("need hq >= 1, hk >= 0 and an even head dim d");
    if (q_head_stride < d || (hk > 0 && k_head_stride < d)) return fail_inval("head strides must be >= d");
    if (dtype != 0 && dtype != 1) return fail_inval("dtype must be 0 (float32) or 1 (bfloat16)");
    hipStream_t st = (hipStream_t)stream;
    const dim3 grid((unsigned)(hq + hk));
    if (dtype == 1)
        hipLaunchKernelGGL(k_rope<uint16_t>, grid, dim3(64), 0, st, (const uint16_t*)q, q_head_stride,
                           (const uint16_t*)k, k_head_stride, (const uint16_t*)cos, (const uint16_t*)sin, hq, d,
                           (uint16_t*)qo, (uint16_t*)ko);
    else
        hipLaunchKernelGGL(k_rope<float>, grid, dim3(64), 0, st, (const float*)q, q_head_stride, (const float*)k,
                           k_head_stride, (const float*)cos, (const float*)sin, hq, d, (float*)qo, (float*)ko);
    return check_launch("k_rope");
}
