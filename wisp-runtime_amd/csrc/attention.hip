// Grouped-query attention of one decode token over a static KV cache, for the
// graph decoder's segments (all Tmax slots allocated, positions > pos masked).
//
// Reference semantics: wisp/graphdec.py:171-174 -- scaled_dot_product_attention
// of q [1, Hk, G, D] (G = Hq/Hk query heads share a KV head) against the static
// cache [1, Hk, Tmax, D] with the mask (t <= pos), scale = the layer's scaling:
//     o[h] = sum_{t <= pos} softmax_t(scale * q[h].k[t]) v[t],  KV head = h / G.
// Here q.k is accumulated in fp32 from exact bf16 x bf16 products
// (v_dot2_f32_bf16), the softmax and the weighted sum are fp32, and o is
// rounded to bf16 once.
//
// Two launches (split-K over positions, then a combine):
//  k_attn_partial: one wave per (64-position chunk, KV head). Phase 1, lane =
//    position: the lane's K row (D bf16) against the G query rows held in LDS.
//    Phase 2: per-head max and sum of exponentials across the wave. Phase 3,
//    lane = D/64 dimensions: the exponentials (in LDS) times the V rows, read
//    coalesced. Writes (m, l, o[D]) per head. Chunks beyond pos exit at once.
//  k_attn_combine: one wave per query head merges the chunks' partials with
//    the usual max-rescaling and stores bf16.
// HBM-bound: reads 2 * (pos+1) * D * 2 bytes per KV head.
#include <math.h>

#include "wisp_device.hpp"
#include "wisp_internal.hpp"

namespace wisp {

constexpr int kChunk = 64;  // positions per partial workgroup (one wave)

template <int D>
struct VRow;
template <>
struct VRow<64> {
    static __device__ __forceinline__ void load(const uint16_t* p, float* v) { v[0] = __uint_as_float((uint32_t)p[0] << 16); }
};
template <>
struct VRow<128> {
    static __device__ __forceinline__ void load(const uint16_t* p, float* v) {
        const uint32_t w = *reinterpret_cast<const uint32_t*>(p);
        v[0] = __uint_as_float(w << 16);
        v[1] = __uint_as_float(w & 0xFFFF0000u);
    }
};
template <>
struct VRow<256> {
    static __device__ __forceinline__ void load(const uint16_t* p, float* v) {
        const uint2 w = *reinterpret_cast<const uint2*>(p);
        v[0] = __uint_as_float(w.x << 16);
        v[1] = __uint_as_float(w.x & 0xFFFF0000u);
        v[2] = __uint_as_float(w.y << 16);
        v[3] = __uint_as_float(w.y & 0xFFFF0000u);
    }
};

// partial record of one (KV head, chunk, query head g): [m, l, o[0..D-1]]
template <int G, int D>
__global__ __launch_bounds__(64) void k_attn_partial(const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc,
                                                     const uint16_t* __restrict__ vc, int64_t head_stride,
                                                     const int64_t* __restrict__ pos_ptr, int tmax, float scale,
                                                     float* __restrict__ part, int nsplit) {
    constexpr int DPL = D / 64;  // dimensions per lane in phase 3
    __shared__ uint4 qs[G][D / 8];
    __shared__ float es[kChunk][G];
    const int lane = threadIdx.x;
    const int split = blockIdx.x, hk = blockIdx.y;
    const int64_t pos = *pos_ptr;
    const int p0 = split * kChunk;
    if ((int64_t)p0 > pos) return;  // nothing valid here; the combine reads chunks <= pos only
    const int nvalid = (int)min<int64_t>(min<int64_t>(kChunk, pos - p0 + 1), tmax - p0);

    const uint4* qsrc = reinterpret_cast<const uint4*>(q + (int64_t)hk * G * D);
    for (int i = lane; i < G * D / 8; i += 64) qs[i / (D / 8)][i % (D / 8)] = qsrc[i];
    __syncthreads();

    // phase 1: scores of this lane's position
    const bool valid = lane < nvalid;
    float s[G];
#pragma unroll
    for (int g = 0; g < G; ++g) s[g] = 0.f;
    if (valid) {
        const uint4* kr = reinterpret_cast<const uint4*>(kc + hk * head_stride + (int64_t)(p0 + lane) * D);
        uint4 kk[D / 8];
#pragma unroll
        for (int c = 0; c < D / 8; ++c) kk[c] = kr[c];
#pragma unroll
        for (int c = 0; c < D / 8; ++c) {
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const uint4 qq = qs[g][c];
                s[g] = dot2(kk[c].x, qq.x, s[g]);
                s[g] = dot2(kk[c].y, qq.y, s[g]);
                s[g] = dot2(kk[c].z, qq.z, s[g]);
                s[g] = dot2(kk[c].w, qq.w, s[g]);
            }
        }
    }
    // phase 2: per-head max and exponentials over the chunk
    float m[G], l[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const float v = valid ? s[g] * scale : -INFINITY;
        m[g] = wave_max(v);
        const float e = valid ? expf(v - m[g]) : 0.f;
        es[lane][g] = e;
        l[g] = wave_sum(e);
    }
    __syncthreads();

    // phase 3: o[g][d] = sum_j e[j][g] v[j][d], in batches of VB rows whose loads
    // are all issued first (rows past the valid ones repeat the last valid row,
    // with weight 0)
    constexpr int VB = 64 / DPL;
    const uint16_t* vbase = vc + hk * head_stride + (int64_t)p0 * D + lane * DPL;
    float o[G][DPL];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int t = 0; t < DPL; ++t) o[g][t] = 0.f;
    for (int j0 = 0; j0 < nvalid; j0 += VB) {
        float vv[VB][DPL];
#pragma unroll
        for (int j = 0; j < VB; ++j) VRow<D>::load(vbase + (int64_t)min(j0 + j, nvalid - 1) * D, vv[j]);
#pragma unroll
        for (int j = 0; j < VB; ++j) {
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const float e = j0 + j < kChunk ? es[min(j0 + j, kChunk - 1)][g] : 0.f;
#pragma unroll
                for (int t = 0; t < DPL; ++t) o[g][t] += e * vv[j][t];
            }
        }
    }
    float* rec = part + ((int64_t)hk * nsplit + split) * G * (2 + D);
#pragma unroll
    for (int g = 0; g < G; ++g) {
        if (lane == 0) {
            rec[g * (2 + D)] = m[g];
            rec[g * (2 + D) + 1] = l[g];
        }
#pragma unroll
        for (int t = 0; t < DPL; ++t) rec[g * (2 + D) + 2 + lane * DPL + t] = o[g][t];
    }
}

// one wave per query head h: merge the partials of chunks 0 .. pos/64
template <int D>
__global__ __launch_bounds__(64) void k_attn_combine(const float* __restrict__ part, const int64_t* __restrict__ pos_ptr,
                                                     int G, int nsplit, uint16_t* __restrict__ out) {
    constexpr int DPL = D / 64;
    constexpr int U = 8;  // partials loaded per step
    const int lane = threadIdx.x;
    const int h = blockIdx.x, hk = h / G, g = h - hk * G;
    const int64_t pos = *pos_ptr;
    const int nv = (int)min<int64_t>(nsplit, pos / kChunk + 1);
    const float* base = part + ((int64_t)hk * nsplit * G + g) * (2 + D);
    const int64_t stride = (int64_t)G * (2 + D);  // between chunks of this head
    float M = -INFINITY;
    for (int i = lane; i < nv; i += 64) M = fmaxf(M, base[i * stride]);
    M = wave_max(M);
    float L = 0.f;
    for (int i = lane; i < nv; i += 64) L += base[i * stride + 1] * expf(base[i * stride] - M);
    L = wave_sum(L);
    float O[DPL];
#pragma unroll
    for (int t = 0; t < DPL; ++t) O[t] = 0.f;
    for (int i0 = 0; i0 < nv; i0 += U) {
        float w[U], ov[U][DPL];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int i = min(i0 + u, nv - 1);
            w[u] = (i0 + u < nv) ? expf(base[i * stride] - M) : 0.f;
#pragma unroll
            for (int t = 0; t < DPL; ++t) ov[u][t] = base[i * stride + 2 + lane * DPL + t];
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int t = 0; t < DPL; ++t) O[t] += w[u] * ov[u][t];
    }
    const float inv = 1.f / L;
#pragma unroll
    for (int t = 0; t < DPL; ++t) out[(int64_t)h * D + lane * DPL + t] = f32_to_bf16(O[t] * inv);
}

template <int G, int D>
static void launch_attn(const uint16_t* q, const uint16_t* kc, const uint16_t* vc, int64_t hs, const int64_t* pos,
                        int hk, int tmax, float scale, float* part, uint16_t* out, hipStream_t st) {
    const int nsplit = (tmax + kChunk - 1) / kChunk;
    hipLaunchKernelGGL((k_attn_partial<G, D>), dim3(nsplit, hk), dim3(64), 0, st, q, kc, vc, hs, pos, tmax, scale,
                       part, nsplit);
    hipLaunchKernelGGL((k_attn_combine<D>), dim3(hk * G), dim3(64), 0, st, part, pos, G, nsplit, out);
}

}  // namespace wisp

using namespace wisp;

extern "C" int64_t wisp_attn_ws_bytes(int hq, int d, int tmax) {
    if (hq < 1 || d < 1 || tmax < 1) return -1;
    return (int64_t)hq * ((tmax + kChunk - 1) / kChunk) * (2 + d) * 4;
}

// graphdec.py:171-174
extern "C" int wisp_attn_decode(const uint16_t* q, const uint16_t* kc, const uint16_t* vc, int64_t kv_head_stride,
                                const int64_t* pos, int hq, int hk, int d, int tmax, float scale, void* ws,
                                uint16_t* out, void* stream) {
    clear_error();
    if (!q || !kc || !vc || !pos || !ws || !out) return fail_inval("null pointer");
    if (hk < 1 || hq < hk || hq % hk) return fail_inval("hq must be a positive multiple of hk");
    if (tmax < 1 || kv_head_stride < (int64_t)tmax * d) return fail_inval("kv_head_stride must be >= tmax*d");
    if (!aligned(q, 16) || !aligned(kc, 16) || !aligned(vc, 16) || (kv_head_stride * 2) % 16) {
        set_error("q, kc, vc and the KV head stride must be 16-byte aligned");
        return WISP_EALIGN;
    }
    const int G = hq / hk;
    hipStream_t st = (hipStream_t)stream;
    float* part = static_cast<float*>(ws);
#define WISP_ATTN(GG, DD)                                                                         \
    if (G == GG && d == DD) {                                                                     \
        launch_attn<GG, DD>(q, kc, vc, kv_head_stride, pos, hk, tmax, scale, part, out, st);      \
        return check_launch("k_attn");                                                            \
    }
    WISP_ATTN(8, 128)
    WISP_ATTN(4, 128)
    WISP_ATTN(2, 128)
    WISP_ATTN(1, 128)
    WISP_ATTN(16, 128)
    WISP_ATTN(8, 64)
    WISP_ATTN(4, 64)
    WISP_ATTN(2, 64)
    WISP_ATTN(1, 64)
    WISP_ATTN(8, 256)
    WISP_ATTN(4, 256)
    WISP_ATTN(2, 256)
    WISP_ATTN(1, 256)
#undef WISP_ATTN
    return fail_inval("supported: head dim 64/128/256 with 1, 2, 4, 8 (and 16 at d=128) query heads per KV head");
}
