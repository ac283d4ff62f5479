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

// ---------------------------------------------------------------------------
// Wide form (D in {64, 128}, G <= 8): one workgroup of 4 waves per (64-position
// chunk, KV head); wave w owns positions p0 + 16w .. +15.
//  * Every K and V load of the wave is issued first. K: LPR = D/8 lanes per row,
//    16 bytes each (a wave load reads RPI = 64/LPR whole rows); V: lane = D/64
//    dimensions of every row.
//  * Scores: 4 v_dot2 per (row, head) and lane, summed over the LPR lanes of a
//    row with DPP row operations (every lane of the group gets the sum).
//  * Softmax statistics and the V sums are combined across the 4 waves in LDS;
//    the record (m, l, o[D]) per head has the layout of k_attn_partial.
// ---------------------------------------------------------------------------
template <int LPR>
__device__ __forceinline__ float row_group_sum(float v) {
    v += dpp_f<0xB1>(v);                  // quad_perm [1,0,3,2]
    v += dpp_f<0x4E>(v);                  // quad_perm [2,3,0,1]
    v += dpp_f<0x141>(v);                 // row_half_mirror: the two quads of 8 lanes
    if (LPR >= 16) v += dpp_f<0x140>(v);  // row_mirror: the two halves of 16 lanes
    return v;
}

template <int G, int D>
__global__ __launch_bounds__(256) void k_attn_wide(const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc,
                                                   const uint16_t* __restrict__ vc, int64_t head_stride,
                                                   const int64_t* __restrict__ pos_ptr, int tmax, float scale,
                                                   float* __restrict__ part, int nsplit) {
    static_assert(D == 64 || D == 128, "wide attention takes head dim 64 or 128");
    static_assert(G >= 1 && G <= 8, "wide attention takes at most 8 query heads per KV head");
    constexpr int LPR = D / 8, RPI = 64 / LPR, RW = kChunk / 4, NK = RW / RPI, DPL = D / 64;
    __shared__ uint4 qs[G][D / 8];
    __shared__ float es[4][RW][G];
    __shared__ float red_m[4][G], red_l[4][G];
    __shared__ float red_o[4][G][D];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int split = blockIdx.x, hk = blockIdx.y;
    const int64_t pos = *pos_ptr;
    const int p0 = split * kChunk;
    if ((int64_t)p0 > pos) return;  // the whole workgroup: chunks past pos are never read
    const int nvalid = (int)min<int64_t>(min<int64_t>(kChunk, pos - p0 + 1), tmax - p0);
    const int plast = p0 + nvalid - 1;
    const int pw = p0 + wv * RW;
    const int rg = lane / LPR, dg = lane - rg * LPR;
    const uint16_t* kh = kc + hk * head_stride;
    const uint16_t* vh = vc + hk * head_stride;

    uint4 kk[NK];
#pragma unroll
    for (int i = 0; i < NK; ++i) {
        const int p = min(pw + rg + RPI * i, plast);
        kk[i] = *reinterpret_cast<const uint4*>(kh + (int64_t)p * D + dg * 8);
    }
    uint32_t vv[RW];
#pragma unroll
    for (int r = 0; r < RW; ++r) {
        const int p = min(pw + r, plast);
        vv[r] = DPL == 2 ? *reinterpret_cast<const uint32_t*>(vh + (int64_t)p * D + lane * 2)
                         : (uint32_t)vh[(int64_t)p * D + lane];
    }
    const uint4* qsrc = reinterpret_cast<const uint4*>(q + (int64_t)hk * G * D);
    for (int i = threadIdx.x; i < G * D / 8; i += 256) qs[i / (D / 8)][i % (D / 8)] = qsrc[i];
    __syncthreads();

    // scores of this lane group's rows
    float s[NK][G];
#pragma unroll
    for (int i = 0; i < NK; ++i) {
        const bool valid = pw + rg + RPI * i <= plast;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const uint4 qq = qs[g][dg];
            float a = dot2(kk[i].x, qq.x, 0.f);
            a = dot2(kk[i].y, qq.y, a);
            a = dot2(kk[i].z, qq.z, a);
            a = dot2(kk[i].w, qq.w, a);
            a = row_group_sum<LPR>(a);
            s[i][g] = valid ? a * scale : -INFINITY;
        }
    }
    // softmax statistics of the workgroup's rows
#pragma unroll
    for (int g = 0; g < G; ++g) {
        float m = s[0][g];
#pragma unroll
        for (int i = 1; i < NK; ++i) m = fmaxf(m, s[i][g]);
        m = wave_max(m);
        if (lane == 0) red_m[wv][g] = m;
    }
    __syncthreads();
    float M[G];
#pragma unroll
    for (int g = 0; g < G; ++g) M[g] = fmaxf(fmaxf(red_m[0][g], red_m[1][g]), fmaxf(red_m[2][g], red_m[3][g]));
#pragma unroll
    for (int g = 0; g < G; ++g) {
        float l = 0.f;
#pragma unroll
        for (int i = 0; i < NK; ++i) {
            const bool valid = pw + rg + RPI * i <= plast;
            const float e = valid ? expf(s[i][g] - M[g]) : 0.f;
            if (dg == 0) es[wv][rg + RPI * i][g] = e;
            l += dg == 0 ? e : 0.f;
        }
        l = wave_sum(l);
        if (lane == 0) red_l[wv][g] = l;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // o[g][lane's dims] over the wave's rows
    float o[G][DPL];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int t = 0; t < DPL; ++t) o[g][t] = 0.f;
#pragma unroll
    for (int r = 0; r < RW; ++r) {
        float vf[DPL];
        vf[0] = __uint_as_float(vv[r] << 16);
        if (DPL == 2) vf[DPL - 1] = __uint_as_float(vv[r] & 0xFFFF0000u);
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float e = es[wv][r][g];
#pragma unroll
            for (int t = 0; t < DPL; ++t) o[g][t] += e * vf[t];
        }
    }
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int t = 0; t < DPL; ++t) red_o[wv][g][lane * DPL + t] = o[g][t];
    __syncthreads();
    float* rec = part + ((int64_t)hk * nsplit + split) * G * (2 + D);
    for (int idx = threadIdx.x; idx < G * D; idx += 256) {
        const int g = idx / D, d = idx - g * D;
        rec[g * (2 + D) + 2 + d] = red_o[0][g][d] + red_o[1][g][d] + red_o[2][g][d] + red_o[3][g][d];
    }
    if (threadIdx.x < G) {
        const int g = threadIdx.x;
        rec[g * (2 + D)] = M[g];
        rec[g * (2 + D) + 1] = red_l[0][g] + red_l[1][g] + red_l[2][g] + red_l[3][g];
    }
}

// One workgroup (4 waves) per query head: wave w merges chunks w, w+4, ... in
// batches of 16 whose loads are issued before the block-wide maximum is known.
template <int D>
__global__ __launch_bounds__(256) void k_attn_merge(const float* __restrict__ part, const int64_t* __restrict__ pos_ptr,
                                                    int G, int nsplit, uint16_t* __restrict__ out) {
    constexpr int DPL = D / 64, B = 16;
    __shared__ float red[4];
    __shared__ float red_l[4];
    __shared__ float red_o[4][D];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int h = blockIdx.x, hk = h / G, g = h - hk * G;
    const int64_t pos = *pos_ptr;
    const int nv = (int)min<int64_t>(nsplit, pos / kChunk + 1);
    const float* base = part + ((int64_t)hk * nsplit * G + g) * (2 + D);
    const int64_t stride = (int64_t)G * (2 + D);
    // first batch of this wave's chunks: o pieces and m, l
    float ov[B][DPL], mv[B], lv[B];
#pragma unroll
    for (int b = 0; b < B; ++b) {
        const int c = min(wv + 4 * b, nv - 1);
        mv[b] = base[c * stride];
        lv[b] = base[c * stride + 1];
#pragma unroll
        for (int t = 0; t < DPL; ++t) ov[b][t] = base[c * stride + 2 + lane * DPL + t];
    }
    // block maximum over all chunks
    float m = -INFINITY;
    for (int c = threadIdx.x; c < nv; c += 256) m = fmaxf(m, base[c * stride]);
    m = wave_max(m);
    if (lane == 0) red[wv] = m;
    __syncthreads();
    const float M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float L = 0.f, O[DPL];
#pragma unroll
    for (int t = 0; t < DPL; ++t) O[t] = 0.f;
    for (int c0 = 0;; c0 += 4 * B) {
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const bool use = c0 + wv + 4 * b < nv;
            const float w = use ? expf(mv[b] - M) : 0.f;
            L += w * lv[b];
#pragma unroll
            for (int t = 0; t < DPL; ++t) O[t] += w * ov[b][t];
        }
        if (c0 + 4 * B >= nv) break;
#pragma unroll
        for (int b = 0; b < B; ++b) {  // next batch
            const int c = min(c0 + 4 * B + wv + 4 * b, nv - 1);
            mv[b] = base[c * stride];
            lv[b] = base[c * stride + 1];
#pragma unroll
            for (int t = 0; t < DPL; ++t) ov[b][t] = base[c * stride + 2 + lane * DPL + t];
        }
    }
    if (lane == 0) red_l[wv] = L;
#pragma unroll
    for (int t = 0; t < DPL; ++t) red_o[wv][lane * DPL + t] = O[t];
    __syncthreads();
    if (threadIdx.x < D) {
        const int d = threadIdx.x;
        const float inv = 1.f / (red_l[0] + red_l[1] + red_l[2] + red_l[3]);
        const float v = red_o[0][d] + red_o[1][d] + red_o[2][d] + red_o[3][d];
        out[(int64_t)h * D + d] = f32_to_bf16(v * inv);
    }
}

template <int G, int D>
static void launch_attn(const uint16_t* q, const uint16_t* kc, const uint16_t* vc, int64_t hs, const int64_t* pos,
                        int hk, int tmax, float scale, float* part, uint16_t* out, hipStream_t st) {
    const int nsplit = (tmax + kChunk - 1) / kChunk;
    if constexpr ((D == 64 || D == 128) && G <= 8) {
        hipLaunchKernelGGL((k_attn_wide<G, D>), dim3(nsplit, hk), dim3(256), 0, st, q, kc, vc, hs, pos, tmax, scale,
                           part, nsplit);
        hipLaunchKernelGGL((k_attn_merge<D>), dim3(hk * G), dim3(256), 0, st, part, pos, G, nsplit, out);
    } else {
        hipLaunchKernelGGL((k_attn_partial<G, D>), dim3(nsplit, hk), dim3(64), 0, st, q, kc, vc, hs, pos, tmax,
                           scale, part, nsplit);
        hipLaunchKernelGGL((k_attn_combine<D>), dim3(hk * G), dim3(64), 0, st, part, pos, G, nsplit, out);
    }
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
