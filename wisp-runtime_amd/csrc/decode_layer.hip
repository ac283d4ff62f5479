// The dense part of one decode step of the graph decoder, as few launches.
//
// Reference: wisp/graphdec.py:160-192 (_attn_router) and :195-203 (_seg), which
// run transformers' Qwen3-MoE modules at batch 1: RMSNorm (Qwen3MoeRMSNorm),
// the q/k/v/o and router nn.Linear layers in bf16, the per-head q/k RMSNorm,
// rope_decode, the KV store at `pos`, and route() (wisp/moe.py:41-47). On the
// GPU those modules are ~60 small kernels per layer; here they are five:
//
//   k_dl_gemv<NORM>   y = W x for bf16 W [O, K] (up to three row blocks, so
//                     q/k/v share one launch). NORM: the input is first
//                     h = a (+ b) and x = RMSNorm(h) * w, computed by every
//                     workgroup for itself (x is a few KB); workgroup 0 also
//                     stores h and x. RES: y = res + (W x).
//   k_dl_qkrope       per q/k head RMSNorm * w, rotary embedding at `pos`,
//                     q to a buffer, k and v into the static KV cache at `pos`.
//   k_dl_route        softmax over the router logits, top-k, renormalise,
//                     bf16 weights -> the host row [ids | weights].
// (attention itself is csrc/attention.hip.)
//
// Numerics follow the modules' bf16 rounding points: every tensor the
// reference holds in bf16 is rounded to bf16 (RTNE) at the same step:
//   RMSNorm: h in binary32, var = sum(h^2) * (1/n), h * rsqrt(var + eps)
//            rounded to bf16, times the bf16 weight, rounded to bf16;
//   Linear:  bf16 x bf16 products summed in binary32, rounded to bf16;
//   residual adds: bf16 + bf16 rounded to bf16;
//   rope:    binary32 x*cos - x'*sin from the bf16 inputs, rounded once.
// Sums are in a different order than the library kernels', so results agree
// to binary32 rounding, not bit for bit.
#include <math.h>

#include "route.hpp"
#include "wisp_device.hpp"
#include "wisp_internal.hpp"

namespace wisp {

struct GemvArgs {
    const uint16_t* a;      // input (bf16 [K]); row *a_row of a [*, K] when a_row is set
    const int64_t* a_row;   // optional device index of the input row (embedding lookup)
    const uint16_t* b;      // NORM: optional second input, h = a + b
    const uint16_t* nw;     // NORM: RMSNorm weight (bf16 [K])
    float eps;
    uint16_t* h_out;        // NORM: optional, workgroup 0 stores h
    uint16_t* x_out;        // NORM: optional, workgroup 0 stores x
    const uint16_t* w0;     // rows [0, r1)
    const uint16_t* w1;     // rows [r1, r2)
    const uint16_t* w2;     // rows [r2, O)
    int r1, r2, O, K;
    const uint16_t* res;    // optional residual (bf16 [O])
    uint16_t* y;            // bf16 [O]
};


// 8 bf16 of a 16-byte chunk -> floats
__device__ __forceinline__ void unpack8(const uint4 q, float* f) {
    f[0] = bf(q.x & 0xFFFFu); f[1] = __uint_as_float(q.x & 0xFFFF0000u);
    f[2] = bf(q.y & 0xFFFFu); f[3] = __uint_as_float(q.y & 0xFFFF0000u);
    f[4] = bf(q.z & 0xFFFFu); f[5] = __uint_as_float(q.z & 0xFFFF0000u);
    f[6] = bf(q.w & 0xFFFFu); f[7] = __uint_as_float(q.w & 0xFFFF0000u);
}
__device__ __forceinline__ uint4 pack8(const float* f) {
    return make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]),
                      pack_bf16x2(f[6], f[7]));
}

// Workgroup of 4 waves; wave w owns rows (blockIdx.x*4 + w)*R .. +R-1. A lane
// owns the 16-byte chunks lane, lane+64, ... (CPL = K/512 of them) of every
// row, so each load instruction of a wave reads 1 KB contiguous. The input's
// loads are issued first, then every weight load; the input is formed while the
// weights stream.
template <int CPL, int R, bool NORM>
__global__ __launch_bounds__(256) void k_dl_gemv(const GemvArgs g) {
#pragma clang fp contract(off)
    __shared__ uint4 xs[NORM ? CPL * 64 : 1];
    __shared__ float red[4];
    const int lane = threadIdx.x & 63;
    const int wv = threadIdx.x >> 6;
    const int K = CPL * 512;
    const int row0 = (blockIdx.x * 4 + wv) * R;

    // The operand's inputs are requested before the weight rows: vector loads retire in issue
    // order, so requested after them the RMSNorm below would start only once the wave's whole
    // weight stream had arrived.
    const uint16_t* A = g.a + (g.a_row ? *g.a_row * (int64_t)K : 0);
    const uint4* a4 = reinterpret_cast<const uint4*>(A);
    constexpr int PT = (CPL * 64 + 255) / 256;  // 16-byte chunks per thread (NORM)
    uint4 av[NORM ? PT : 1], bv[NORM ? PT : 1], nv[NORM ? PT : 1];
    uint4 xv[CPL];
    if constexpr (NORM) {
        const uint4* b4 = reinterpret_cast<const uint4*>(g.b);
        const uint4* n4 = reinterpret_cast<const uint4*>(g.nw);
#pragma unroll
        for (int t = 0; t < PT; ++t) {
            const int i = min((int)threadIdx.x + 256 * t, CPL * 64 - 1);
            av[t] = a4[i];
            if (g.b) bv[t] = b4[i];
            nv[t] = n4[i];
        }
    } else {
#pragma unroll
        for (int c = 0; c < CPL; ++c) xv[c] = a4[c * 64 + lane];
    }
    // NORM: the residual (no caller of the decoder passes one) under a branch that is skipped when
    // there is none
    uint16_t resv = 0;
    if constexpr (NORM) resv = g.res && lane < R ? g.res[min(row0 + lane, g.O - 1)] : (uint16_t)0;

    uint4 wr[R][CPL];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int o = min(row0 + r, g.O - 1);
        const uint16_t* W = o < g.r1 ? g.w0 + (int64_t)o * K
                          : o < g.r2 ? g.w1 + (int64_t)(o - g.r1) * K
                                     : g.w2 + (int64_t)(o - g.r2) * K;
        const u32x4_t* w4 = reinterpret_cast<const u32x4_t*>(W);
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            // non-temporal: each weight byte is read once per step
            const u32x4_t v = __builtin_nontemporal_load(&w4[c * 64 + lane]);
            wr[r][c] = make_uint4(v.x, v.y, v.z, v.w);
        }
    }
    // otherwise the residual, needed last, is requested last, by every lane (the input's first
    // element when there is none): loaded under a branch, its value was needed at the branch's end,
    // so the wave waited there for it and every earlier load before requesting the weight rows
    if constexpr (!NORM) resv = (g.res ? g.res : A)[g.res ? min(row0 + lane, g.O - 1) : 0];
    __builtin_amdgcn_sched_barrier(0);  // the prologue's arithmetic stays behind every load

    if constexpr (NORM) {
        // h = a (+ b) in bf16; x = bf16(w * bf16(h * rsqrt(mean(h^2) + eps)))
        float ss = 0.f;
#pragma unroll
        for (int t = 0; t < PT; ++t) {
            const int i = threadIdx.x + 256 * t;
            if (i >= CPL * 64) break;
            float h[8];
            unpack8(av[t], h);
            if (g.b) {
                float bb[8];
                unpack8(bv[t], bb);
#pragma unroll
                for (int e = 0; e < 8; ++e) h[e] = rbf(h[e] + bb[e]);
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) ss += h[e] * h[e];
            xs[i] = pack8(h);
        }
        ss = wave_sum_dpp(ss);
        if (lane == 0) red[wv] = ss;
        __syncthreads();
        const float var = (red[0] + red[1] + red[2] + red[3]) * (1.0f / (float)K);
        const float rs = rsqrtf(var + g.eps);
#pragma unroll
        for (int t = 0; t < PT; ++t) {
            const int i = threadIdx.x + 256 * t;
            if (i >= CPL * 64) break;
            const uint4 hq = xs[i];
            float h[8], w[8], x[8];
            unpack8(hq, h);
            unpack8(nv[t], w);
#pragma unroll
            for (int e = 0; e < 8; ++e) x[e] = w[e] * rbf(h[e] * rs);
            const uint4 xq = pack8(x);
            xs[i] = xq;
            if (blockIdx.x == 0) {
                if (g.h_out) reinterpret_cast<uint4*>(g.h_out)[i] = hq;
                if (g.x_out) reinterpret_cast<uint4*>(g.x_out)[i] = xq;
            }
        }
        __syncthreads();
#pragma unroll
        for (int c = 0; c < CPL; ++c) xv[c] = xs[c * 64 + lane];
    }

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            s0 = dot2(wr[r][c].x, xv[c].x, s0);
            s1 = dot2(wr[r][c].y, xv[c].y, s1);
            s0 = dot2(wr[r][c].z, xv[c].z, s0);
            s1 = dot2(wr[r][c].w, xv[c].w, s1);
        }
        acc[r] = wave_sum_dpp(s0 + s1);
    }
    if (lane < R) {
        float v = acc[0];
#pragma unroll
        for (int r = 1; r < R; ++r)
            if (lane == r) v = acc[r];
        const int o = row0 + lane;
        if (o < g.O) {
            float yv = rbf(v);
            if (g.res) yv = rbf(bf(resv) + yv);
            g.y[o] = f32_to_bf16(yv);
        }
    }
}

// Any K (a multiple of 8, at most 8192): the same work split with a runtime
// number of chunks per lane, loads issued per chunk.
template <int R, bool NORM>
__global__ __launch_bounds__(256) void k_dl_gemv_any(const GemvArgs g) {
#pragma clang fp contract(off)
    __shared__ uint4 xs[NORM ? 1024 : 1];
    __shared__ float red[4];
    const int lane = threadIdx.x & 63;
    const int wv = threadIdx.x >> 6;
    const int K = g.K, NC = K >> 3;
    const int row0 = (blockIdx.x * 4 + wv) * R;
    const uint16_t* A = g.a + (g.a_row ? *g.a_row * (int64_t)K : 0);
    const uint4* xsrc = reinterpret_cast<const uint4*>(A);
    if (NORM) {
        const uint4* b4 = reinterpret_cast<const uint4*>(g.b);
        float ss = 0.f;
        for (int i = threadIdx.x; i < NC; i += 256) {
            float h[8];
            unpack8(xsrc[i], h);
            if (g.b) {
                float bb[8];
                unpack8(b4[i], bb);
#pragma unroll
                for (int e = 0; e < 8; ++e) h[e] = rbf(h[e] + bb[e]);
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) ss += h[e] * h[e];
            xs[i] = pack8(h);
        }
        ss = wave_sum(ss);
        if (lane == 0) red[wv] = ss;
        __syncthreads();
        const float var = (red[0] + red[1] + red[2] + red[3]) * (1.0f / (float)K);
        const float rs = rsqrtf(var + g.eps);
        const uint4* n4 = reinterpret_cast<const uint4*>(g.nw);
        for (int i = threadIdx.x; i < NC; i += 256) {
            const uint4 hq = xs[i];
            float h[8], w[8], x[8];
            unpack8(hq, h);
            unpack8(n4[i], w);
#pragma unroll
            for (int e = 0; e < 8; ++e) x[e] = w[e] * rbf(h[e] * rs);
            const uint4 xq = pack8(x);
            xs[i] = xq;
            if (blockIdx.x == 0) {
                if (g.h_out) reinterpret_cast<uint4*>(g.h_out)[i] = hq;
                if (g.x_out) reinterpret_cast<uint4*>(g.x_out)[i] = xq;
            }
        }
        __syncthreads();
    }
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int o = min(row0 + r, g.O - 1);
        const uint16_t* W = o < g.r1 ? g.w0 + (int64_t)o * K
                          : o < g.r2 ? g.w1 + (int64_t)(o - g.r1) * K
                                     : g.w2 + (int64_t)(o - g.r2) * K;
        const uint4* w4 = reinterpret_cast<const uint4*>(W);
        float s0 = 0.f, s1 = 0.f;
        for (int c = lane; c < NC; c += 64) {
            const uint4 wq = w4[c];
            const uint4 xq = NORM ? xs[c] : xsrc[c];
            s0 = dot2(wq.x, xq.x, s0);
            s1 = dot2(wq.y, xq.y, s1);
            s0 = dot2(wq.z, xq.z, s0);
            s1 = dot2(wq.w, xq.w, s1);
        }
        acc[r] = wave_sum_dpp(s0 + s1);
    }
    if (lane < R) {
        float v = acc[0];
#pragma unroll
        for (int r = 1; r < R; ++r)
            if (lane == r) v = acc[r];
        const int o = row0 + lane;
        if (o < g.O) {
            float yv = rbf(v);
            if (g.res) yv = rbf(bf(g.res[o]) + yv);
            g.y[o] = f32_to_bf16(yv);
        }
    }
}

// One wave per head: heads [0, Hq) are q, [Hq, Hq+Hk) are k (RMSNorm * weight,
// rope at pos), [Hq+Hk, Hq+2Hk) are v (copied). qkv = [q | k | v] heads of D.
// Lane t handles the element pairs (i, i + D/2) for i = t, t + 64, ... < D/2.
template <int D>
__global__ __launch_bounds__(64) void k_dl_qkrope(const uint16_t* __restrict__ qkv, const uint16_t* __restrict__ qnw,
                                                  const uint16_t* __restrict__ knw, float eps,
                                                  const uint16_t* __restrict__ cos_t, const uint16_t* __restrict__ sin_t,
                                                  const int64_t* __restrict__ pos_ptr, int Hq, int Hk,
                                                  uint16_t* __restrict__ kc, uint16_t* __restrict__ vc,
                                                  int64_t head_stride, uint16_t* __restrict__ qo) {
    const int h = blockIdx.x, lane = threadIdx.x;
    const int64_t pos = *pos_ptr;
    const uint16_t* x = qkv + (int64_t)h * D;
    if (h >= Hq + Hk) {
        uint16_t* dst = vc + (int64_t)(h - Hq - Hk) * head_stride + pos * D;
        for (int i = lane; i < D; i += 64) dst[i] = x[i];
        return;
    }
    const bool isq = h < Hq;
    uint16_t* dst = isq ? qo + (int64_t)h * D : kc + (int64_t)(h - Hq) * head_stride + pos * D;
    head_norm_rope<D>(x, isq ? qnw : knw, eps, cos_t + pos * D, sin_t + pos * D, dst, nullptr, lane);
}

// softmax (binary32) over E bf16 logits, top-k (descending; equal values: lower
// index first), optional renormalisation over the k, weights rounded to bf16.
// row = [ids (k, as float) | weights (k, bf16 values as float)]. One wave.
// host_row / host_flag (optional, pinned host memory mapped for the device):
// the row is also written there with system-scope stores and, once those have
// completed, host_flag = ++*seq (seq: a device counter), so the host can wait
// for the row by watching host_flag instead of synchronising the stream.
// EPL = logits per lane (a power of two >= E/64): every load is issued before
// any use (addresses clamped into range, the extra values masked afterwards).
template <int EPL>
__global__ __launch_bounds__(64) void k_dl_route(const uint16_t* __restrict__ logits, int E, int k, int norm,
                                                 float* __restrict__ row, float* host_row, uint32_t* host_flag,
                                                 uint32_t* seq) {
    const int lane = threadIdx.x;
    const uint32_t seq0 = host_row ? *seq : 0u;  // requested with the logits
    const float val = route_select<EPL>(logits, E, k, norm);
    if (lane < 2 * k) {
        row[lane] = val;
        if (host_row) __hip_atomic_store(host_row + lane, val, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
    if (host_row) {
        // the barrier makes every lane's row store happen-before lane 0's flag store,
        // and the system-scope release orders them before the flag for the host
        __syncthreads();
        if (lane == 0) {
            *seq = seq0 + 1;
            __hip_atomic_store(host_flag, seq0 + 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
        }
    }
}

template <int CPL, int R, bool NORM>
static void launch_gemv(const GemvArgs& g, hipStream_t st) {
    const int rows_wg = 4 * R;
    hipLaunchKernelGGL((k_dl_gemv<CPL, R, NORM>), dim3((g.O + rows_wg - 1) / rows_wg), dim3(256), 0, st, g);
}

template <int CPL, bool NORM>
static void gemv_rows(const GemvArgs& g, hipStream_t st) {
    // as many waves as the rows allow up to ~1k, then rows per wave for more loads in flight
    if (g.O >= 4096 * (CPL >= 8 ? 1 : 2))
        (CPL >= 8) ? launch_gemv<CPL, 2, NORM>(g, st) : launch_gemv<CPL, 4, NORM>(g, st);
    else if (g.O >= 1024)
        launch_gemv<CPL, 2, NORM>(g, st);
    else
        launch_gemv<CPL, 1, NORM>(g, st);
}

}  // namespace wisp

using namespace wisp;

// graphdec.py:160-192 (the input RMSNorm and q/k/v projections, the post-attention
// RMSNorm and router gate, o_proj with the residual) and :195-203 (embedding and
// the final norm + lm_head of the last segment)
extern "C" int wisp_dl_gemv(const void* a, const int64_t* a_row, const void* b, const void* norm_w, float eps,
                            void* h_out, void* x_out, const void* w0, const void* w1, const void* w2, int64_t r1,
                            int64_t r2, int64_t O, int64_t K, const void* res, void* y, void* stream) {
    clear_error();
    if (!a || !w0 || !y) return fail_inval("null a, w0 or y");
    if (K < 8 || K % 8 || K > 8192) return fail_inval("K must be a multiple of 8 in [8, 8192]");
    if (O < 1 || O > (int64_t)1 << 30) return fail_inval("O must be in [1, 2^30]");
    if (r1 < 0 || r1 > r2 || r2 > O) return fail_inval("need 0 <= r1 <= r2 <= O");
    if (r2 > r1 && !w1) return fail_inval("w1 is null but rows [r1, r2) are non-empty");
    if (O > r2 && !w2) return fail_inval("w2 is null but rows [r2, O) are non-empty");
    if (!norm_w && (b || h_out || x_out)) return fail_inval("b, h_out and x_out need norm_w (the NORM prologue)");
    for (const void* p : {a, b, norm_w, (const void*)h_out, (const void*)x_out, w0, w1, w2})
        if (p && !aligned(p, 16)) {
            set_error("every vector and weight pointer must be 16-byte aligned");
            return WISP_EALIGN;
        }
    if (res && !aligned(res, 2)) return fail_inval("res must be 2-byte aligned");
    GemvArgs g;
    g.a = (const uint16_t*)a;
    g.a_row = a_row;
    g.b = (const uint16_t*)b;
    g.nw = (const uint16_t*)norm_w;
    g.eps = eps;
    g.h_out = (uint16_t*)h_out;
    g.x_out = (uint16_t*)x_out;
    g.w0 = (const uint16_t*)w0;
    g.w1 = (const uint16_t*)(w1 ? w1 : w0);
    g.w2 = (const uint16_t*)(w2 ? w2 : w0);
    g.r1 = (int)r1;
    g.r2 = (int)r2;
    g.O = (int)O;
    g.K = (int)K;
    g.res = (const uint16_t*)res;
    g.y = (uint16_t*)y;
    hipStream_t st = (hipStream_t)stream;
    const bool norm = norm_w != nullptr;
    switch (K % 512 ? 0 : K / 512) {
    case 1: norm ? gemv_rows<1, true>(g, st) : gemv_rows<1, false>(g, st); break;
    case 2: norm ? gemv_rows<2, true>(g, st) : gemv_rows<2, false>(g, st); break;
    case 4: norm ? gemv_rows<4, true>(g, st) : gemv_rows<4, false>(g, st); break;
    case 8: norm ? gemv_rows<8, true>(g, st) : gemv_rows<8, false>(g, st); break;
    case 16: norm ? gemv_rows<16, true>(g, st) : gemv_rows<16, false>(g, st); break;
    default: {  // other multiples of 8: runtime chunk count, one row per wave
        const dim3 grid((unsigned)((O + 3) / 4));
        if (norm)
            hipLaunchKernelGGL((k_dl_gemv_any<1, true>), grid, dim3(256), 0, st, g);
        else
            hipLaunchKernelGGL((k_dl_gemv_any<1, false>), grid, dim3(256), 0, st, g);
    }
    }
    return check_launch("k_dl_gemv");
}

// graphdec.py:163-172 (q_norm, k_norm, rope_decode, the KV store at pos)
extern "C" int wisp_dl_qk_rope(const void* qkv, const void* q_norm_w, const void* k_norm_w, float eps,
                               const void* cos, const void* sin, const int64_t* pos, int hq, int hk, int d, void* kc,
                               void* vc, int64_t head_stride, void* qo, void* stream) {
    clear_error();
    if (!qkv || !q_norm_w || !k_norm_w || !cos || !sin || !pos || !kc || !vc || !qo) return fail_inval("null pointer");
    if (hq < 1 || hk < 1) return fail_inval("need hq >= 1 and hk >= 1");
    if (head_stride < d) return fail_inval("head_stride must be >= d");
    hipStream_t st = (hipStream_t)stream;
    const dim3 grid((unsigned)(hq + 2 * hk));
    switch (d) {
    case 64:
        hipLaunchKernelGGL(k_dl_qkrope<64>, grid, dim3(64), 0, st, (const uint16_t*)qkv, (const uint16_t*)q_norm_w,
                           (const uint16_t*)k_norm_w, eps, (const uint16_t*)cos, (const uint16_t*)sin, pos, hq, hk,
                           (uint16_t*)kc, (uint16_t*)vc, head_stride, (uint16_t*)qo);
        break;
    case 128:
        hipLaunchKernelGGL(k_dl_qkrope<128>, grid, dim3(64), 0, st, (const uint16_t*)qkv, (const uint16_t*)q_norm_w,
                           (const uint16_t*)k_norm_w, eps, (const uint16_t*)cos, (const uint16_t*)sin, pos, hq, hk,
                           (uint16_t*)kc, (uint16_t*)vc, head_stride, (uint16_t*)qo);
        break;
    case 256:
        hipLaunchKernelGGL(k_dl_qkrope<256>, grid, dim3(64), 0, st, (const uint16_t*)qkv, (const uint16_t*)q_norm_w,
                           (const uint16_t*)k_norm_w, eps, (const uint16_t*)cos, (const uint16_t*)sin, pos, hq, hk,
                           (uint16_t*)kc, (uint16_t*)vc, head_stride, (uint16_t*)qo);
        break;
    default: return fail_inval("head dim d must be 64, 128 or 256");
    }
    return check_launch("k_dl_qkrope");
}

// wisp/moe.py:41-47 (route) at batch 1 + pack_meta's [ids | weights] order
extern "C" int wisp_dl_route(const void* logits, int E, int k, int norm_topk, float* row, float* host_row,
                             uint32_t* host_flag, uint32_t* seq, void* stream) {
    clear_error();
    if (!logits || !row) return fail_inval("null pointer");
    if (E < 1 || E > 1024) return fail_inval("E must be in [1, 1024]");
    if (k < 1 || k > 16 || k > E) return fail_inval("k must be in [1, min(16, E)]");
    if ((host_row != nullptr) != (host_flag != nullptr) || (host_row && !seq))
        return fail_inval("host_row, host_flag and seq go together");
    float* hr = nullptr;
    uint32_t* hf = nullptr;
    if (host_row) {  // device addresses of the pinned host buffers
        void* d1 = nullptr;
        void* d2 = nullptr;
        hipError_t e = hipHostGetDevicePointer(&d1, host_row, 0);
        if (e == hipSuccess) e = hipHostGetDevicePointer(&d2, host_flag, 0);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            set_error("host_row / host_flag are not pinned host memory mapped for the device: %s",
                      hipGetErrorString(e));
            return WISP_EINVAL;
        }
        hr = static_cast<float*>(d1);
        hf = static_cast<uint32_t*>(d2);
    }
    hipStream_t st = (hipStream_t)stream;
    const uint16_t* lg = (const uint16_t*)logits;
    const int nt = norm_topk ? 1 : 0;
    if (E <= 64) hipLaunchKernelGGL(k_dl_route<1>, dim3(1), dim3(64), 0, st, lg, E, k, nt, row, hr, hf, seq);
    else if (E <= 128) hipLaunchKernelGGL(k_dl_route<2>, dim3(1), dim3(64), 0, st, lg, E, k, nt, row, hr, hf, seq);
    else if (E <= 256) hipLaunchKernelGGL(k_dl_route<4>, dim3(1), dim3(64), 0, st, lg, E, k, nt, row, hr, hf, seq);
    else if (E <= 512) hipLaunchKernelGGL(k_dl_route<8>, dim3(1), dim3(64), 0, st, lg, E, k, nt, row, hr, hf, seq);
    else hipLaunchKernelGGL(k_dl_route<16>, dim3(1), dim3(64), 0, st, lg, E, k, nt, row, hr, hf, seq);
    return check_launch("k_dl_route");
}
