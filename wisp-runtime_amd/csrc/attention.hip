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
// Two launches (split-K over positions, then a merge):
//  k_attn_mfma: one workgroup of 4 waves per (64-position chunk, KV head); wave w
//    owns positions p0 + 16w .. +15 and all G query heads of the KV head. Scores and
//    the V sums run on the matrix cores; the waves' (m, l, o) are combined in LDS
//    into one record per (chunk, head). Chunks beyond pos exit at once.
//  k_attn_merge: one workgroup per query head merges the chunks' records with the
//    usual max-rescaling and stores bf16.
// HBM-bound in principle (2 * (pos+1) * D * 2 bytes per KV head); at decode sizes
// the two launches' dependent round trips dominate.
#include <math.h>

#include "wisp_device.hpp"
#include "wisp_internal.hpp"

namespace wisp {

constexpr int kChunk = 64;  // positions per k_attn_mfma workgroup (4 waves of 16)

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// v_mfma_f32_16x16x32_bf16, lane l: A[row l%16][k 8*(l/16) + 0..7], B[k 8*(l/16) + 0..7][col l%16]
__device__ __forceinline__ f32x4_t mfma_k32(uint4 a, uint4 b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                    c, 0, 0, 0);
}
// v_mfma_f32_16x16x16_bf16, lane l: A[row l%16][k 4*(l/16) + 0..3], B[k 4*(l/16) + 0..3][col l%16];
// both forms: D[row 4*(l/16) + i][col l%16] in element i
__device__ __forceinline__ f32x4_t mfma_k16(uint2 a, uint2 b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4_t, a), __builtin_bit_cast(i16x4_t, b),
                                                      c, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// k_attn_mfma (G <= 16 query heads per KV head, D in {64, 128, 256}); lane l,
// n = l%16, r = l/16, wave w:
//  * Scores S[pos][head] = K q^T, D/32 MFMAs of k = 32: A = the wave's 16 K rows
//    (row n, dims D/4*r .. +D/4-1 as D/32 16-byte loads), B = the query rows (column
//    n = head n; columns >= G repeat head G-1 and are masked). A and B take the dims
//    in the same order, so each score is the plain dot product over the head dim
//    (exact bf16 products, fp32 sums). The result holds S[pos 4r+i][head n]: a lane
//    has four positions of one head, so the wave's maximum and sum of exponentials
//    per head take two cross-lane steps for all heads at once.
//  * o[head][d] = sum_pos p v, D/16 MFMAs of k = 16 per term: A = p split into two
//    bf16 terms (p = hi + lo to 2^-17 relative), which is the score layout unchanged;
//    B = V rows 4r+i at dim 32u + 2n + b for tile 2u + b (one 4-byte load per row
//    covers both tiles of a pair). The product of two bf16 is exact and the sums are
//    fp32, so o carries fp32 rounding only.
//  * The four waves exchange their maxima through LDS before the exponentials, so
//    the workgroup's record (m, l, o[D]) per head is a plain sum of theirs. The PV
//    result of a lane is four heads of one dim: one 16-byte LDS store per tile.
//  * QK (the decoder's q/k head norm + rope + K/V store folded in, graphdec.py:163-172):
//    q is not read ready-made; every workgroup forms its G query heads from the raw
//    qkv with head_norm_rope (wave w: heads w, w+4, ...; the same arithmetic as
//    k_dl_qkrope) into LDS. The workgroup whose chunk holds pos also forms the new K row
//    (head_norm_rope) and copies the V row, stores both into the caches at pos and puts
//    them into its own operands for that row (its loads of row pos read the old cache).
//    The inputs of that arithmetic are loaded before the K/V rows: loads retire in
//    issue order, so the head norms run while the K/V data is still arriving.
// ---------------------------------------------------------------------------
struct QkPrep {
    const uint16_t* qkv;  // [q (Hq heads) | k (Hk) | v (Hk)] of D
    const uint16_t* qnw;
    const uint16_t* knw;
    const uint16_t* cos_t;  // [tmax, D]
    const uint16_t* sin_t;
    uint16_t* kc_w;  // the caches attention reads, written at pos
    uint16_t* vc_w;
    float eps;
    int hq, hk;
};
// The new row's inputs pass through here raw (no instruction): the compiler may not move their
// conversions ahead of this point, into the branch that loads them, where converting them would
// wait for those loads and every earlier one before the wave's K/V rows are requested.
template <int D>
__device__ __forceinline__ void opaque_raw(HnrIn<D>& in) {
#pragma unroll
    for (int t = 0; t < HnrIn<D>::NP; ++t)
        asm volatile("" : "+v"(in.a[t]), "+v"(in.b[t]), "+v"(in.wa[t]), "+v"(in.wb[t]), "+v"(in.ca[t]),
                     "+v"(in.cb[t]), "+v"(in.sa[t]), "+v"(in.sb[t]));
}

template <int G, int D, bool QK>
__global__ __launch_bounds__(256) void k_attn_mfma(const uint16_t* __restrict__ q, const uint16_t* kc,
                                                   const uint16_t* vc, int64_t head_stride,
                                                   const int64_t* __restrict__ pos_ptr, int tmax, float scale,
                                                   float* __restrict__ part, int nsplit, const QkPrep qp) {
    static_assert(G == 1 || G == 2 || G == 4 || G == 8 || G == 16, "1, 2, 4, 8 or 16 query heads per KV head");
    static_assert(D == 64 || D == 128 || D == 256, "head dim 64, 128 or 256");
    constexpr int KS = D / 32;  // score MFMAs = 16-byte K loads per lane
    constexpr int NU = D / 32;  // V tile pairs
    constexpr int HQ = (G + 3) / 4;  // lane groups r whose PV rows are real heads
    __shared__ f32x4_t red_o[4][HQ][D];  // heads 4hq .. 4hq+3 of dim d
    __shared__ float red_m[4][16], red_l[4][16];
    const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = lane & 15, r = lane >> 4;
    const int split = blockIdx.x, hk = blockIdx.y;
    const int64_t pos = *pos_ptr;
    const int p0 = split * kChunk;
    if ((int64_t)p0 > pos) return;  // the whole workgroup: chunks past pos are never read
    const int plast = (int)min<int64_t>(min<int64_t>(pos, (int64_t)p0 + kChunk - 1), (int64_t)tmax - 1);
    const int pw = p0 + 16 * wv;
    const uint16_t* kh = kc + hk * head_stride;
    const uint16_t* vh = vc + hk * head_stride;
    const bool own = pos <= (int64_t)plast;  // this chunk holds position pos

    // every load first: the head-norm inputs (QK), then K rows (A), query rows (B), V
    // pieces (rows past plast repeat row plast and are masked)
    constexpr int QPW = (G + 3) / 4;  // query heads this wave forms (QK)
    constexpr int VPL = (D + 63) / 64;
    HnrIn<D> qin[QPW], kin;
    uint32_t vnew[VPL];  // 16-bit values, one per register (packed pairs were formed at the load)
    if constexpr (QK) {
        const uint16_t* cs = qp.cos_t + pos * D;
        const uint16_t* sn = qp.sin_t + pos * D;
#pragma unroll
        for (int j = 0; j < QPW; ++j)
            hnr_load<D>(qp.qkv + ((int64_t)hk * G + min(wv + 4 * j, G - 1)) * D, qp.qnw, cs, sn, lane, qin[j]);
        // Only the two waves that use them load the new K and V rows' inputs, and the values stay
        // raw until their use (opaque_raw; the V row one value per register): converted at the
        // branch's end, they made those waves wait for these loads before requesting their K/V
        // rows (8.61 -> 8.42 us per call at 4,090 positions without that wait). Measured slower:
        // loading them in every wave (8.86 us: every wave's K/V data retires behind them), and
        // requesting them after the K/V rows (8.97-9.38 us: the new K row's head norm then runs
        // after all of that workgroup's data, and that workgroup finishes last).
        if (own && wv == (G & 3)) hnr_load<D>(qp.qkv + ((int64_t)qp.hq + hk) * D, qp.knw, cs, sn, lane, kin);
        if (own && wv == ((G + 1) & 3)) {
            const uint16_t* xv = qp.qkv + ((int64_t)qp.hq + qp.hk + hk) * D;
#pragma unroll
            for (int t = 0; t < VPL; ++t) vnew[t] = xv[min(lane + 64 * t, D - 1)];
        }
    }
    uint4 ka[KS], qb[KS];
    {
        const uint4* kr = reinterpret_cast<const uint4*>(kh + (int64_t)min(pw + n, plast) * D + (D / 4) * r);
#pragma unroll
        for (int s = 0; s < KS; ++s) ka[s] = kr[s];
        if constexpr (!QK) {
            const uint4* qr =
                reinterpret_cast<const uint4*>(q + ((int64_t)hk * G + min(n, G - 1)) * D + (D / 4) * r);
#pragma unroll
            for (int s = 0; s < KS; ++s) qb[s] = qr[s];
        }
    }
    uint32_t vw[4][NU];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t* vr = reinterpret_cast<const uint32_t*>(vh + (int64_t)min(pw + 4 * r + i, plast) * D + 2 * n);
#pragma unroll
        for (int u = 0; u < NU; ++u) vw[i][u] = vr[16 * u];
    }
    __builtin_amdgcn_sched_barrier(0);  // all loads in flight before the first wait
    if constexpr (QK) {
        __shared__ __align__(16) uint16_t q_l[G][D];
        __shared__ __align__(16) uint16_t kv_l[2][D];  // the new K and V rows (chunk of pos)
#pragma unroll
        for (int j = 0; j < QPW; ++j) {
            const int g = wv + 4 * j;
            if (g < G) hnr_finish<D>(qin[j], qp.eps, &q_l[g][0], nullptr, lane);
        }
        if (own) {
            const int64_t at = hk * head_stride + pos * D;
            if (wv == (G & 3)) {  // a wave with the fewest q heads
                opaque_raw(kin);
                hnr_finish<D>(kin, qp.eps, &kv_l[0][0], qp.kc_w + at, lane);
            } else if (wv == ((G + 1) & 3)) {
#pragma unroll
                for (int t = 0; t < VPL; ++t) asm volatile("" : "+v"(vnew[t]));
#pragma unroll
                for (int t = 0; t < VPL; ++t) {
                    const int i = lane + 64 * t;
                    if (i < D) {
                        kv_l[1][i] = (uint16_t)vnew[t];
                        qp.vc_w[at + i] = (uint16_t)vnew[t];
                    }
                }
            }
        }
        __syncthreads();
#pragma unroll
        for (int s = 0; s < KS; ++s)
            qb[s] = *reinterpret_cast<const uint4*>(&q_l[min(n, G - 1)][(D / 4) * r + 8 * s]);
        if (own) {  // the row at pos from the values just formed
            if (pw + n == (int)pos) {
#pragma unroll
                for (int s = 0; s < KS; ++s) ka[s] = *reinterpret_cast<const uint4*>(&kv_l[0][(D / 4) * r + 8 * s]);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (pw + 4 * r + i == (int)pos) {
#pragma unroll
                    for (int u = 0; u < NU; ++u)
                        vw[i][u] = *reinterpret_cast<const uint32_t*>(&kv_l[1][32 * u + 2 * n]);
                }
        }
    }

    f32x4_t sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KS; ++s) sc = mfma_k32(ka[s], qb[s], sc);

    // this wave's maximum and exponential sum per head
    float sv[4], m = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const bool ok = n < G && pw + 4 * r + i <= plast;
        sv[i] = ok ? sc[i] * scale : -INFINITY;
        m = fmaxf(m, sv[i]);
    }
    m = max_xor16(m);
    m = max_xor32(m);
    if (lane < 16) red_m[wv][n] = m;
    __syncthreads();
    // the workgroup's maximum (finite for n < G: position p0 <= pos is in wave 0)
    m = fmaxf(fmaxf(red_m[0][n], red_m[1][n]), fmaxf(red_m[2][n], red_m[3][n]));
    float pe[4], l = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        pe[i] = sv[i] == -INFINITY ? 0.f : expf(sv[i] - m);
        l += pe[i];
    }
    l = add_xor16(l);
    l = add_xor32(l);
    if (lane < 16) red_l[wv][n] = l;

    uint2 phi, plo;
    phi.x = pack_bf16x2(pe[0], pe[1]);
    phi.y = pack_bf16x2(pe[2], pe[3]);
    plo.x = pack_bf16x2(pe[0] - bf16_lo(phi.x), pe[1] - bf16_hi(phi.x));
    plo.y = pack_bf16x2(pe[2] - bf16_lo(phi.y), pe[3] - bf16_hi(phi.y));

    f32x4_t o[2 * NU];
#pragma unroll
    for (int t = 0; t < 2 * NU; ++t) o[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < NU; ++u) {
        uint2 b0, b1;  // dims 32u + 2n (low halves) and 32u + 2n + 1 (high halves) of rows 4r .. 4r+3
        b0.x = __builtin_amdgcn_perm(vw[1][u], vw[0][u], 0x05040100u);
        b0.y = __builtin_amdgcn_perm(vw[3][u], vw[2][u], 0x05040100u);
        b1.x = __builtin_amdgcn_perm(vw[1][u], vw[0][u], 0x07060302u);
        b1.y = __builtin_amdgcn_perm(vw[3][u], vw[2][u], 0x07060302u);
        o[2 * u] = mfma_k16(phi, b0, o[2 * u]);
        o[2 * u + 1] = mfma_k16(phi, b1, o[2 * u + 1]);
        o[2 * u] = mfma_k16(plo, b0, o[2 * u]);
        o[2 * u + 1] = mfma_k16(plo, b1, o[2 * u + 1]);
    }

    // o[t][i] = O[head 4r + i][dim 32(t/2) + 2n + t%2]
    if (r < HQ) {
#pragma unroll
        for (int t = 0; t < 2 * NU; ++t) red_o[wv][r][32 * (t >> 1) + 2 * n + (t & 1)] = o[t];
    }
    __syncthreads();

    float* rec = part + ((int64_t)hk * nsplit + split) * G * (2 + D);
    for (int e = threadIdx.x; e < HQ * D; e += 256) {
        const int hq = e / D, d = e - hq * D;
        const f32x4_t v = (red_o[0][hq][d] + red_o[1][hq][d]) + (red_o[2][hq][d] + red_o[3][hq][d]);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (4 * hq + j < G) rec[(4 * hq + j) * (2 + D) + 2 + d] = v[j];
    }
    if (threadIdx.x < G) {
        const int h = threadIdx.x;
        rec[h * (2 + D)] = fmaxf(fmaxf(red_m[0][h], red_m[1][h]), fmaxf(red_m[2][h], red_m[3][h]));
        rec[h * (2 + D) + 1] = (red_l[0][h] + red_l[1][h]) + (red_l[2][h] + red_l[3][h]);
    }
}

// Sum of (lanes 0..15: max) of v over the 16 lanes of row 0, read from lane 0.
__device__ __forceinline__ float row0_sum(float v) {
    v += dpp_f<0xB1>(v);
    v += dpp_f<0x4E>(v);
    v += dpp_f<0x141>(v);
    v += dpp_f<0x140>(v);
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
}
__device__ __forceinline__ float row0_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    v = fmaxf(v, dpp_f<0x140>(v));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
}

// One workgroup (4 waves) per query head: wave w merges chunks w, w+4, ... in
// batches of 16 with a running maximum. Lane b < 16 reads the m and l of the batch's
// chunk b and computes its weight (one exponential per chunk); the weights reach the
// o sums of every lane through readlane. The four waves' sums are rescaled to the
// common maximum in LDS. Only the chunks up to pos have records (pos read from device
// memory, so graphs follow it).
template <int D>
__global__ __launch_bounds__(256) void k_attn_merge(const float* __restrict__ part, const int64_t* __restrict__ pos_ptr,
                                                    int G, int nsplit, uint16_t* __restrict__ out) {
    constexpr int DPL = D / 64, B = 16;
    __shared__ float red_m[4], red_l[4];
    __shared__ float red_o[4][D];
    const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // chunk indices in SGPRs
    const int h = blockIdx.x, hk = h / G, g = h - hk * G;
    const int64_t pos = *pos_ptr;
    const float* base = part + ((int64_t)hk * nsplit * G + g) * (2 + D);
    const int stride = G * (2 + D);  // c * stride < nsplit * G * (2 + D): 32-bit offsets within one head's records
    float M = -INFINITY, L = 0.f, O[DPL];
#pragma unroll
    for (int t = 0; t < DPL; ++t) O[t] = 0.f;
    // A batch's records are requested without waiting for the position: chunk indices are
    // clamped to the workspace's nsplit chunks, and records past the position's last chunk
    // (stale or never written) are masked once it has arrived -- never multiplied, so their
    // bits cannot reach the sums. The first batch always exists (chunk 0).
    int c0 = 0, nv;
    do {
        float ov[B][DPL];
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const int c = min(c0 + wv + 4 * b, nsplit - 1);
#pragma unroll
            for (int t = 0; t < DPL; ++t) ov[b][t] = base[c * stride + 2 + lane * DPL + t];
        }
        const int cl = c0 + wv + 4 * (lane & 15);
        const int cc = min(cl, nsplit - 1);
        float mr = base[cc * stride], lr = base[cc * stride + 1];
        __builtin_amdgcn_sched_barrier(0);
        int64_t pv = pos;
        asm volatile("" : "+s"(pv));  // the position's first use stays here, after the batch's loads
        nv = (int)min<int64_t>(nsplit, pv / kChunk + 1);
        const bool have = lane < 16 && cl < nv;
        const float mc = have ? mr : -INFINITY;
        const float Mn = fmaxf(M, row0_max(mc));
        const float f = M == -INFINITY ? 0.f : expf(M - Mn);  // rescale of the sums so far
        const float w = have ? expf(mc - Mn) : 0.f;
        L = L * f + row0_sum(have ? w * lr : 0.f);
#pragma unroll
        for (int t = 0; t < DPL; ++t) O[t] *= f;
#pragma unroll
        for (int b = 0; b < B; ++b) {
            const float wb = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), b));
            const bool vb = c0 + wv + 4 * b < nv;  // the same in every lane
#pragma unroll
            for (int t = 0; t < DPL; ++t) O[t] += vb ? wb * ov[b][t] : 0.f;
        }
        M = Mn;
        c0 += 4 * B;
    } while (c0 < nv);
    if (lane == 0) {
        red_m[wv] = M;
        red_l[wv] = L;
    }
#pragma unroll
    for (int t = 0; t < DPL; ++t) red_o[wv][lane * DPL + t] = O[t];
    __syncthreads();
    if (threadIdx.x < D) {
        const int d = threadIdx.x;
        const float Mx = fmaxf(fmaxf(red_m[0], red_m[1]), fmaxf(red_m[2], red_m[3]));  // finite: chunk 0 exists
        float v = 0.f, Lt = 0.f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const float f = red_m[w] == -INFINITY ? 0.f : expf(red_m[w] - Mx);
            v += f * red_o[w][d];
            Lt += f * red_l[w];
        }
        out[(int64_t)h * D + d] = f32_to_bf16(v / Lt);
    }
}

template <int G, int D>
static void launch_attn(const uint16_t* q, const uint16_t* kc, const uint16_t* vc, int64_t hs, const int64_t* pos,
                        int hk, int tmax, float scale, float* part, uint16_t* out, const QkPrep* qp, hipStream_t st) {
    const int nsplit = (tmax + kChunk - 1) / kChunk;
    if (qp)
        hipLaunchKernelGGL((k_attn_mfma<G, D, true>), dim3(nsplit, hk), dim3(256), 0, st, q, kc, vc, hs, pos, tmax,
                           scale, part, nsplit, *qp);
    else
        hipLaunchKernelGGL((k_attn_mfma<G, D, false>), dim3(nsplit, hk), dim3(256), 0, st, q, kc, vc, hs, pos, tmax,
                           scale, part, nsplit, QkPrep{});
    hipLaunchKernelGGL((k_attn_merge<D>), dim3(hk * G), dim3(256), 0, st, part, pos, G, nsplit, out);
}

static int attn_dispatch(const uint16_t* q, const uint16_t* kc, const uint16_t* vc, int64_t kv_head_stride,
                         const int64_t* pos, int hq, int hk, int d, int tmax, float scale, void* ws, uint16_t* out,
                         const QkPrep* qp, void* stream) {
    const int G = hq / hk;
    hipStream_t st = (hipStream_t)stream;
    float* part = static_cast<float*>(ws);
#define WISP_ATTN(GG, DD)                                                                         \
    if (G == GG && d == DD) {                                                                     \
        launch_attn<GG, DD>(q, kc, vc, kv_head_stride, pos, hk, tmax, scale, part, out, qp, st);  \
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
    return attn_dispatch(q, kc, vc, kv_head_stride, pos, hq, hk, d, tmax, scale, ws, out, nullptr, stream);
}

// graphdec.py:163-174 in one pair of launches: dl_qk_rope's q/k head norm, rope and
// K/V store at pos folded into the attention kernel (same bits as wisp_dl_qk_rope
// followed by wisp_attn_decode on its qo).
extern "C" int wisp_attn_decode_qk(const uint16_t* qkv, const uint16_t* q_norm_w, const uint16_t* k_norm_w,
                                   float eps, const uint16_t* cos, const uint16_t* sin, const int64_t* pos, int hq,
                                   int hk, int d, uint16_t* kc, uint16_t* vc, int64_t kv_head_stride, int tmax,
                                   float scale, void* ws, uint16_t* out, void* stream) {
    clear_error();
    if (!qkv || !q_norm_w || !k_norm_w || !cos || !sin || !pos || !kc || !vc || !ws || !out)
        return fail_inval("null pointer");
    if (hk < 1 || hq < hk || hq % hk) return fail_inval("hq must be a positive multiple of hk");
    if (tmax < 1 || kv_head_stride < (int64_t)tmax * d) return fail_inval("kv_head_stride must be >= tmax*d");
    if (!aligned(kc, 16) || !aligned(vc, 16) || (kv_head_stride * 2) % 16) {
        set_error("kc, vc and the KV head stride must be 16-byte aligned");
        return WISP_EALIGN;
    }
    const QkPrep qp{qkv, q_norm_w, k_norm_w, cos, sin, kc, vc, eps, hq, hk};
    return attn_dispatch(nullptr, kc, vc, kv_head_stride, pos, hq, hk, d, tmax, scale, ws, out, &qp, stream);
}
