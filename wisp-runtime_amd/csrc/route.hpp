// The router's choice for one decode token on one wave (wisp/moe.py:41-47 at batch 1):
// softmax in float32 of the bf16 router logits, top-k with equal values going to the lower
// index, renormalised by the sum of the selected weights when `norm`, weights rounded to
// bf16. Shared by the route kernel (decode_layer.hip) and the route + paging kernel
// (cache.hip), so both produce the same bits.
#pragma once

#include "wisp_device.hpp"

namespace wisp {

// (value, index) maximum with equal values going to the lower index: a total order, so
// every reduction order selects the same entry. Wave-wide with DPP inside each 16-lane
// row (xor 1, xor 2, row_half_mirror, row_mirror), then the four row winners through
// readlane; the result is wave-uniform.
__device__ __forceinline__ void best_of(float& bv, int& bi, float ov, int oi) {
    if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
    }
}
template <int CTRL>
__device__ __forceinline__ void best_dpp(float& bv, int& bi) {
    const float ov = dpp_f<CTRL>(bv);
    const int oi = __builtin_amdgcn_update_dpp(0, bi, CTRL, 0xF, 0xF, true);
    best_of(bv, bi, ov, oi);
}
__device__ __forceinline__ void wave_best(float& bv, int& bi) {
    best_dpp<0xB1>(bv, bi);
    best_dpp<0x4E>(bv, bi);
    best_dpp<0x141>(bv, bi);
    best_dpp<0x140>(bv, bi);
    float v = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bv), 0));
    int i = __builtin_amdgcn_readlane(bi, 0);
#pragma unroll
    for (int r = 16; r < 64; r += 16)
        best_of(v, i, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bv), r)),
                __builtin_amdgcn_readlane(bi, r));
    bv = v;
    bi = i;
}

// Lane r < k returns expert id r (as a float), lane k + r weight r, other lanes 0. EPL =
// logits per lane (E <= 64 EPL); the logits are requested before any use.
template <int EPL>
__device__ __forceinline__ float route_select(const uint16_t* __restrict__ logits, int E, int k, int norm) {
#pragma clang fp contract(off)
    constexpr int kRouteMaxPerLane = EPL;
    const int lane = threadIdx.x;
    uint32_t raw[kRouteMaxPerLane];
#pragma unroll
    for (int t = 0; t < kRouteMaxPerLane; ++t) raw[t] = logits[min(lane + 64 * t, E - 1)];
    float v[kRouteMaxPerLane];
    float mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < kRouteMaxPerLane; ++t) {
        const int i = lane + 64 * t;
        v[t] = i < E ? bf(raw[t]) : -INFINITY;
        mx = fmaxf(mx, v[t]);
    }
    mx = wave_max_dpp(mx);  // exact in any order
    float sum = 0.f;
#pragma unroll
    for (int t = 0; t < kRouteMaxPerLane; ++t) {
        const int i = lane + 64 * t;
        v[t] = i < E ? expf(v[t] - mx) : 0.f;
        sum += v[t];
    }
    sum = wave_sum(sum);
#pragma unroll
    for (int t = 0; t < kRouteMaxPerLane; ++t) v[t] = lane + 64 * t < E ? v[t] / sum : -1.f;
    float sel_v[16];
    int sel_i[16];
    for (int r = 0; r < k; ++r) {
        // best of this lane (lowest index among equals), then across the wave
        float bv = -2.f;
        int bi = 1 << 30;
#pragma unroll
        for (int t = 0; t < kRouteMaxPerLane; ++t)
            if (v[t] > bv) {
                bv = v[t];
                bi = lane + 64 * t;
            }
        wave_best(bv, bi);
        sel_v[r] = bv;
        sel_i[r] = bi;
#pragma unroll
        for (int t = 0; t < kRouteMaxPerLane; ++t)
            if (lane + 64 * t == bi) v[t] = -1.f;
    }
    // every lane holds the same selection: lanes r < k store id r, lanes k + r weight r.
    // The renormalising sum adds adjacent pairs level by level (an odd last entry carried
    // up), which is the order torch's sum over the last dim takes for k = 1, 2, 4, 8 and 16
    // (checked bit for bit on MI355X; for other k torch's order differs and the sum may
    // differ in its last bit). The softmax above sums per lane in index order, then with the
    // xor butterfly over the 64 lanes, as torch's warp softmax does.
    float tree[16];
    for (int r = 0; r < k; ++r) tree[r] = sel_v[r];
    for (int n = k; n > 1; n = (n + 1) >> 1) {
        for (int i = 0; i < (n >> 1); ++i) tree[i] = tree[2 * i] + tree[2 * i + 1];
        if (n & 1) tree[n >> 1] = tree[n - 1];
    }
    const float tot = tree[0];
    float val = 0.f;
    for (int r = 0; r < k; ++r) {
        if (lane == r) val = (float)sel_i[r];
        if (lane == k + r) val = rbf(norm ? sel_v[r] / tot : sel_v[r]);
    }
    return val;
}

}  // namespace wisp
