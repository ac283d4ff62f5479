// gpt-oss experts on the WiSP slot pool (gfx950).
//
// Reference: wisp/gptoss.py. A gpt-oss expert is gate_up [H, 2I] (gate and up
// interleaved on the output axis), down [I, H], plus two biases; with I == H it
// is stored in the framework's flat [3, n] layout as
//     [ gate_up.flat[:n] | gate_up.flat[n:] | down.flat ]      (gptoss.py:32-37)
// and quantized like any other expert (b-bit codes, fp16 scale and min per G
// consecutive flat elements). Unlike the Qwen experts, both matrices are stored
// input-major ([K, out]): a weight row is one input element's contribution to
// every output, so the GEMV walks rows and accumulates columns.
//
// Kernels:
//   k_mxfp4      MXFP4 blocks + power-of-two scales -> bf16 (gptoss.py:22-29)
//   k_go_gate_up partial gate_up GEMV: per expert, column block and block of
//                16 * go_pairs_gu(bits) input rows, fp32 partial sums of x . W_gu (bf16 weights)
//   k_go_down    sums the gate_up partials of its kGoRows activation rows, adds the
//                bias and applies the clamped SwiGLU with the reference's bf16
//                rounding steps, then the partial down GEMV over those rows
//   k_go_out     sums the down partials, adds the bias and the weighted sum over
//                the k experts (gptoss.py:126-131)
//
// Numerics follow the reference's decode path (PagedGptOssBlock, N == 1): the
// dequantized weights are bf16 (bit-exact with the dequant kernel), products
// and sums are fp32, and every value the reference holds as a bf16 tensor is
// rounded to bf16 at the same point: the two GEMV outputs, the bias sums, each
// step of the activation, and each weighted expert output.
#include <algorithm>

#include "wisp_device.hpp"
#include "wisp_internal.hpp"

namespace wisp {

// ---------------------------------------------------------------------------
// MXFP4 -> bf16. blocks [ngroups][16] (two e2m1 codes per byte, low nibble
// first), scales [ngroups] (exponent byte, bias 127). value = FP4[code] *
// 2^(scale - 127) in binary32 (exact: an FP4 value has two significant bits),
// then rounded to bf16 like torch's .to(bfloat16) (any NaN -> 0x7FC0).

__device__ __forceinline__ float fp4_value(uint32_t c) {
    // e2m1: sign bit 3, exponent bits 2..1, mantissa bit 0:
    // 0, 0.5, 1, 1.5, 2, 3, 4, 6 and their negatives
    const uint32_t e = (c >> 1) & 3u, m = c & 1u;
    const float mag = e == 0 ? 0.5f * (float)m : __uint_as_float((126u + e) << 23) * (1.f + 0.5f * (float)m);
    return (c & 8u) ? -mag : mag;
}

__device__ __forceinline__ float pow2_bias127(uint32_t s) {
    // 2^(s - 127) as torch.exp2 gives it in binary32: s = 0 is the subnormal
    // 2^-127, s = 255 overflows to +inf
    return s == 0 ? __uint_as_float(0x00400000u) : s == 255 ? __uint_as_float(0x7F800000u) : __uint_as_float(s << 23);
}

__device__ __forceinline__ uint16_t bf16_torch(float v) {
    return v != v ? (uint16_t)0x7FC0u : f32_to_bf16(v);
}

// one thread per 16-byte block: 32 outputs (64 bytes, four 16-byte stores)
__global__ __launch_bounds__(256) void k_mxfp4(const uint8_t* __restrict__ blocks, const uint8_t* __restrict__ scales,
                                               int64_t ngroups, uint16_t* __restrict__ out) {
    const int64_t gi = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (gi >= ngroups) return;
    const uint4 b = *reinterpret_cast<const uint4*>(blocks + gi * 16);
    const float sc = pow2_bias127(scales[gi]);
    const uint32_t w[4] = {b.x, b.y, b.z, b.w};
    uint4* dst = reinterpret_cast<uint4*>(out + gi * 32);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        uint32_t o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t byte = (w[q] >> (8 * i)) & 0xFFu;
            const uint16_t lo = bf16_torch(fp4_value(byte & 15u) * sc);
            const uint16_t hi = bf16_torch(fp4_value(byte >> 4) * sc);
            o[i] = (uint32_t)lo | ((uint32_t)hi << 16);
        }
        dst[q] = make_uint4(o[0], o[1], o[2], o[3]);
    }
}

// ---------------------------------------------------------------------------
// Decode layer.

constexpr int kGoWaves = 4;         // waves per workgroup
constexpr int kGoCols = 1024;       // output columns per workgroup (32 lanes x 32)
constexpr int kGoRedStride = 1056;  // LDS floats per partial vector (32 x 33: conflict-free transpose)
// Row pairs per half-wave: input rows per workgroup = 16 x pairs. Gate_up takes 80 rows, so its
// grid at the gpt-oss-20b shape (6 x 36 x 4 = 864 workgroups) is resident at once at four
// workgroups per CU; with 64 rows it was 1,080, whose last 56 ran as a second round. Down keeps
// 64 rows (its prologue pairs two threads with each gate_up column of its rows).
// 64 rows for 3-bit codes, whose decode needs more registers (80 rows spilled there).
constexpr int go_pairs_gu(int bits) { return bits == 3 ? 4 : 5; }
constexpr int kGoPairsDN = 4, kGoRows = 16 * kGoPairsDN;
constexpr int kGoMaxPart = 20;      // gate_up partials a down-prologue thread requests together (18 at H = 2880)

struct GoLayer {
    const uint8_t* pool;
    int64_t slot_bytes;
    int nslots, k, H, I, G, E;
    int gsh;            // log2(G) when G is a power of two, else -1
    int64_t n;          // H * I
    int64_t scale_off;  // byte offset of the fp16 scales in an expert (3n*bits/8)
    int64_t NG;         // groups per expert (3n/G); the mins follow the scales
    const float* meta;  // [slot ids (k) | routing weights (k) | expert ids (k)]
    const uint16_t* x;  // bf16 [H]
    const uint16_t* gub;  // bf16 [E, 2I]
    const uint16_t* db;   // bf16 [E, H]
    float alpha, limit;
    float* p1;  // [k][S1][2I]
    float* p2;  // [k][S2][H]
    int S1, S2;
    uint16_t* out;  // bf16 [H]
};

__device__ __forceinline__ float bf16r(float v) { return bf16_to_f32(f32_to_bf16(v)); }

__device__ __forceinline__ int go_slot(const GoLayer& L, int j) {
    const float f = L.meta[j];
    const int s = (int)f;
    return (f >= 0.f && f < (float)L.nslots && (float)s == f) ? s : -1;
}
__device__ __forceinline__ int go_expert(const GoLayer& L, int j) {
    const float f = L.meta[2 * L.k + j];
    const int e = (int)f;
    return (f >= 0.f && f < (float)L.E && (float)e == f) ? e : -1;
}

// The workgroup's column GEMV over rows [r0, r0 + 16*PAIRS) of a [R, C] input-major
// matrix whose element (r, c) is flat element e0 + r*C + c of the expert.
// Lane l of wave w owns columns col0 + 32*(l%32) .. +31 and, with half
// h = l/32, the row pairs r0 + 4*PAIRS*w + 2*PAIRS*h + 2p (p < PAIRS). xpair(r) returns the bf16
// pair (x[r], x[r+1]) of the operand. Rows past R and columns past C read
// clamped (in-bounds) weights and contribute nothing (zero operand / no
// store). pre() runs after the weight loads are issued and before the first
// xpair() (the down kernel forms its operand there). The partial sums of the 2*kGoWaves
// half-waves are reduced through LDS in a fixed order and stored as
// dst[c - col0] for c < C.
// POW2G: G = 2^gsh, so a chunk's quant group is its element index shifted (else a division).
// XFIRST: xpair reads global memory and needs nothing from pre(), so the operand pairs are
// requested before the weight rows (loads retire in issue order: requested after them, the
// first dot product would wait for the wave's whole weight stream).
template <int BITS, int PAIRS, bool POW2G, bool XFIRST, typename XPair, typename Pre>
__device__ __forceinline__ void go_colgemv(const uint8_t* __restrict__ base, int64_t e0, int R, int C, int G, int gsh,
                                           int64_t scale_off, int64_t NG, int r0, int col0, XPair xpair, Pre pre,
                                           float* red, float* __restrict__ dst, bool poison) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, h = lane >> 5, cl = lane & 31;
    const int c = col0 + 32 * cl;
    const bool col_on = c < C;
    const int cc = col_on ? c : C - 32;
    const uint16_t* sc = reinterpret_cast<const uint16_t*>(base + scale_off);
    const uint16_t* mn = sc + NG;
    uint32_t cd[PAIRS][2][BITS];
    uint32_t sv[PAIRS][2][2];
    uint32_t xp[PAIRS];
    if constexpr (XFIRST) {
#pragma unroll
        for (int p = 0; p < PAIRS; ++p) {
            const int r = r0 + 4 * PAIRS * wv + 2 * PAIRS * h + 2 * p;
            xp[p] = xpair(min(r, R - 2));
        }
    }
#pragma unroll
    for (int p = 0; p < PAIRS; ++p) {
        const int r = r0 + 4 * PAIRS * wv + 2 * PAIRS * h + 2 * p;
        const bool row_on = r < R;  // R is even: the pair is whole or absent
        const int rr = row_on ? r : R - 2;
        const int64_t eb = e0 + (int64_t)rr * C + cc;  // element of the pair's first row
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int64_t e = eb + (t ? C : 0);
            load_chunk<BITS>(base + e * BITS / 8, cd[p][t]);
            const int64_t g = POW2G ? e >> gsh : e / G;  // e is a multiple of 32: the chunk is in one group
            sv[p][t][0] = sc[g];
            sv[p][t][1] = mn[g];
        }
    }
    pre();  // runs while the weight loads are in flight
#pragma unroll
    for (int p = 0; p < PAIRS; ++p) {
        const int r = r0 + 4 * PAIRS * wv + 2 * PAIRS * h + 2 * p;
        if constexpr (!XFIRST) xp[p] = r < R ? xpair(r) : 0u;
        else if (r >= R) xp[p] = 0u;  // (the row pair is absent: its loads read a clamped, real pair)
    }
    float acc[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) acc[i] = 0.f;
#pragma unroll
    for (int p = 0; p < PAIRS; ++p) {
        // the two rows' bf16 weights (RTNE of fp32(q*s) + m, q*s exact), one dot2
        float w0[32], w1[32];
        if constexpr (BITS == 3) {
            uint32_t q0[32], q1[32];
            chunk_codes<BITS>(cd[p][0], q0);
            chunk_codes<BITS>(cd[p][1], q1);
            const float s0 = h2f((uint16_t)sv[p][0][0]), m0 = h2f((uint16_t)sv[p][0][1]);
            const float s1 = h2f((uint16_t)sv[p][1][0]), m1 = h2f((uint16_t)sv[p][1][1]);
#pragma unroll
            for (int i = 0; i < 32; ++i) {
                w0[i] = __builtin_fmaf((float)q0[i], s0, m0);
                w1[i] = __builtin_fmaf((float)q1[i], s1, m1);
            }
        } else {
            dequant32_f32<BITS>(cd[p][0], sv[p][0][0] | (sv[p][0][1] << 16), w0);
            dequant32_f32<BITS>(cd[p][1], sv[p][1][0] | (sv[p][1][1] << 16), w1);
        }
#pragma unroll
        for (int i = 0; i < 32; ++i) acc[i] = dot2(pack_bf16x2(w0[i], w1[i]), xp[p], acc[i]);
    }
    // partial vectors [2*kGoWaves][32 lanes x 33]: slot = 2w + h, column 32*cl + i at cl*33 + i
    float* mine = red + (2 * wv + h) * kGoRedStride + cl * 33;
#pragma unroll
    for (int i = 0; i < 32; ++i) mine[i] = acc[i];
    __syncthreads();
    for (int col = threadIdx.x; col < kGoCols; col += 64 * kGoWaves) {
        float s = 0.f;
        const int at = (col >> 5) * 33 + (col & 31);
#pragma unroll
        for (int q = 0; q < 2 * kGoWaves; ++q) s += red[q * kGoRedStride + at];
        if (col0 + col < C) dst[col] = poison ? __builtin_nanf("") : s;
    }
}

// Workgroups are launched in one dimension and placed by xcd_block: the column blocks of one
// row block and expert read the same lines of the rows' fp16 scales and mins (a row's groups
// are contiguous in the store; a block's 8 of them are 16 of a line's 128 bytes) and, in the
// down kernel, the same gate_up partial sums, so they share an XCD and its L2.
// T = ceil(2I / kGoCols) x S1 x k workgroups, S1 = ceil(H / (16 * go_pairs_gu(BITS)))
template <int BITS, bool POW2G>
__global__ __launch_bounds__(64 * kGoWaves, 4) void k_go_gate_up(const GoLayer L) {
    __shared__ float red[2 * kGoWaves * kGoRedStride];
    constexpr int PAIRS = go_pairs_gu(BITS);
    const int C = 2 * L.I;
    int bx, by, j;
    xcd_block((C + kGoCols - 1) / kGoCols, L.S1, L.k, bx, by, j);
    const int slot = go_slot(L, j);
    const uint8_t* base = L.pool + (int64_t)(slot >= 0 ? slot : 0) * L.slot_bytes;
    const int col0 = bx * kGoCols, r0 = by * 16 * PAIRS;
    const uint32_t* xw = reinterpret_cast<const uint32_t*>(L.x);
    // (3-bit codes keep the operand loads after the weights: requested first they spilled there)
    go_colgemv<BITS, PAIRS, POW2G, BITS != 3>(base, 0, L.H, C, L.G, L.gsh, L.scale_off, L.NG, r0, col0,
                                   [&](int r) { return xw[r >> 1]; },
                     [] {}, red, L.p1 + ((int64_t)j * L.S1 + by) * C + col0, slot < 0);
}

// T = ceil(H / kGoCols) x S2 x k workgroups, S2 = ceil(I / kGoRows)
template <int BITS, bool POW2G>
__global__ __launch_bounds__(64 * kGoWaves, 4) void k_go_down(const GoLayer L) {
    __shared__ float red[2 * kGoWaves * kGoRedStride];
    __shared__ float gu[2 * kGoRows];
    __shared__ float half_sum[2][2 * kGoRows];
    __shared__ uint32_t actp[kGoRows / 2];
    static_assert(64 * kGoWaves == 4 * kGoRows, "two threads per gate_up column");
    int bx, by, j;
    xcd_block((L.H + kGoCols - 1) / kGoCols, L.S2, L.k, bx, by, j);
    const int slot = go_slot(L, j), ex = go_expert(L, j);
    const int I2 = 2 * L.I, i0 = by * kGoRows;
    // gate_up outputs of activation rows i0 .. i0+kGoRows-1: gu = bf16(bf16(x . W) + bias). The S1 partial
    // sums of a column are split between two threads. The first kGoMaxPart of a thread's partials (all of
    // them at the gpt-oss shapes) and the column's bias are requested before the weight rows: vector loads
    // retire in issue order, so requested after them they would wait for the whole weight stream, and the
    // prologue below would start only once the weights were in. Indices are clamped so every load is
    // unconditional; only the sums are predicated.
    const int t = threadIdx.x & (2 * kGoRows - 1), hf = threadIdx.x / (2 * kGoRows);
    const int c = 2 * i0 + t, cl = min(c, I2 - 1);
    const int per = (L.S1 + 1) / 2, s0 = hf * per, s1 = min(L.S1, s0 + per);
    const float* pcol = L.p1 + (int64_t)j * L.S1 * I2 + cl;
    float u8[kGoMaxPart];
#pragma unroll
    for (int u = 0; u < kGoMaxPart; ++u) u8[u] = pcol[(int64_t)min(s0 + u, L.S1 - 1) * I2];
    const uint16_t bias = L.gub[(int64_t)(ex >= 0 ? ex : 0) * I2 + cl];
    __builtin_amdgcn_sched_barrier(0);
    auto prologue = [&] {
        float v = 0.f;
        if (c < I2) {
#pragma unroll
            for (int u = 0; u < kGoMaxPart; ++u)
                if (s0 + u < s1) v += u8[u];
            for (int sb = s0 + kGoMaxPart; sb < s1; sb += kGoMaxPart) {  // more than 2 kGoMaxPart row blocks
                float w8[kGoMaxPart];
#pragma unroll
                for (int u = 0; u < kGoMaxPart; ++u) w8[u] = pcol[(int64_t)min(sb + u, s1 - 1) * I2];
#pragma unroll
                for (int u = 0; u < kGoMaxPart; ++u)
                    if (sb + u < s1) v += w8[u];
            }
        }
        half_sum[hf][t] = v;
        __syncthreads();
        if (threadIdx.x < 2 * kGoRows) {
            float g = 0.f;
            if (c < I2) {
                g = half_sum[0][t] + half_sum[1][t];
                g = ex >= 0 ? bf16r(bf16r(g) + bf16_to_f32(bias)) : __builtin_nanf("");
            }
            gu[t] = g;
        }
        __syncthreads();
        // clamped SwiGLU, each step rounded to bf16 as the reference's bf16 tensor ops do
        // (gptoss.py:120-122): gate = min(g, limit), up = clamp(u, -limit, limit),
        // act = (up + 1) * (gate * sigmoid(gate * alpha))
        for (int t2 = threadIdx.x; t2 < kGoRows / 2; t2 += 64 * kGoWaves) {
            float a2[2];
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const int i = i0 + 2 * t2 + q;
                float a = 0.f;
                if (i < L.I) {
                    const float gg = fminf(gu[4 * t2 + 2 * q], L.limit);
                    const float uu = fmaxf(fminf(gu[4 * t2 + 2 * q + 1], L.limit), -L.limit);
                    const float ga = bf16r(gg * L.alpha);
                    const float sg = bf16r(1.f / (1.f + expf(-ga)));
                    const float glu = bf16r(gg * sg);
                    a = bf16r(bf16r(uu + 1.f) * glu);
                    // a NaN gate/up (invalid expert or slot) stays NaN through fminf/fmaxf only
                    // if both operands are NaN, so carry it explicitly
                    if (gu[4 * t2 + 2 * q] != gu[4 * t2 + 2 * q] || gu[4 * t2 + 2 * q + 1] != gu[4 * t2 + 2 * q + 1])
                        a = __builtin_nanf("");
                }
                a2[q] = a;
            }
            actp[t2] = pack_bf16x2(a2[0], a2[1]);
        }
        __syncthreads();
    };
    const uint8_t* base = L.pool + (int64_t)(slot >= 0 ? slot : 0) * L.slot_bytes;
    go_colgemv<BITS, kGoPairsDN, POW2G, false>(base, 2 * L.n, L.I, L.H, L.G, L.gsh, L.scale_off, L.NG, i0,
                                        bx * kGoCols,
                     [&](int r) { return actp[(r - i0) >> 1]; }, prologue, red,
                     L.p2 + ((int64_t)j * L.S2 + by) * L.H + bx * kGoCols, slot < 0);
}

// out[h] = bf16( sum_j bf16( w_j * bf16( bf16(sum_s p2[j][s][h]) + db[e_j][h] ) ) ), j ascending.
// A workgroup takes kGoOutCols columns and splits each column's S2 partial sums
// into kGoOutSlices slices, one per wave. Every lane requests the partials of
// up to B experts before adding any (the sums are latency-bound); the slice sums
// are added in slice order through LDS. B (experts per batch) and U (partials per
// request round) are chosen at launch to fit k and the slice length, so no lane
// requests a clamped duplicate: at the gpt-oss shapes B = 4 and U = 6, 24 requests per
// lane where B = U = 8 made 64 (the layer 28.0-28.4 -> 27.0-27.4 us).
// 32 columns per workgroup (90 workgroups at H = 2880): measured 33.4 us per layer against
// 34.1 with 64 (45 workgroups), the same as 16; with B = 4, U = 6 also 16 columns (180
// workgroups), 16 slices per column or 64 columns measured no faster.
constexpr int kGoOutCols = 32, kGoOutSlices = 8;
template <int B, int U>
__global__ __launch_bounds__(kGoOutCols * kGoOutSlices) void k_go_out(const GoLayer L) {
    constexpr int kGoOutBatch = B, kGoOutUnroll = U;
    __shared__ float part[kGoOutSlices][kGoOutBatch][kGoOutCols];
    const int c = threadIdx.x & (kGoOutCols - 1), sl = threadIdx.x / kGoOutCols;
    const int h = blockIdx.x * kGoOutCols + c, hh = min(h, L.H - 1);
    const int per = (L.S2 + kGoOutSlices - 1) / kGoOutSlices, s0 = sl * per, s1 = min(L.S2, s0 + per);
    float y = 0.f;
    for (int j0 = 0; j0 < L.k; j0 += kGoOutBatch) {
        float v[kGoOutBatch];
#pragma unroll
        for (int jj = 0; jj < kGoOutBatch; ++jj) v[jj] = 0.f;
        // The batch's routing weights, expert ids and down biases are requested right after the first
        // partials: not before them (the expert ids are a round trip that would hold up the partials'
        // issue) and not after the sums (a round trip of its own at the end). Indices are clamped, so
        // every load is unconditional.
        float wj[kGoOutBatch];
        int exj[kGoOutBatch];
        uint16_t dbv[kGoOutBatch];
#pragma unroll
        for (int jj = 0; jj < kGoOutBatch; ++jj) {  // (set below in the slice's first step; slice 0 has one)
            wj[jj] = 0.f;
            exj[jj] = -1;
            dbv[jj] = 0;
        }
        for (int sb = s0; sb < s1; sb += kGoOutUnroll) {
            float t[kGoOutBatch][kGoOutUnroll];
#pragma unroll
            for (int jj = 0; jj < kGoOutBatch; ++jj)
#pragma unroll
                for (int u = 0; u < kGoOutUnroll; ++u) {
                    const int j = min(j0 + jj, L.k - 1), s = min(sb + u, s1 - 1);
                    t[jj][u] = L.p2[((int64_t)j * L.S2 + s) * L.H + hh];
                }
            if (sb == s0) {
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int jj = 0; jj < kGoOutBatch; ++jj) {
                    const int j = min(j0 + jj, L.k - 1);
                    exj[jj] = go_expert(L, j);
                    wj[jj] = L.meta[L.k + j];
                    dbv[jj] = L.db[(int64_t)(exj[jj] >= 0 ? exj[jj] : 0) * L.H + hh];
                }
            }
#pragma unroll
            for (int jj = 0; jj < kGoOutBatch; ++jj)
#pragma unroll
                for (int u = 0; u < kGoOutUnroll; ++u)
                    if (sb + u < s1) v[jj] += t[jj][u];
        }
#pragma unroll
        for (int jj = 0; jj < kGoOutBatch; ++jj) part[sl][jj][c] = v[jj];
        __syncthreads();
        if (sl == 0) {
#pragma unroll
            for (int jj = 0; jj < kGoOutBatch; ++jj) {
                if (j0 + jj >= L.k) break;
                float sum = part[0][jj][c];
#pragma unroll
                for (int q = 1; q < kGoOutSlices; ++q) sum += part[q][jj][c];
                const float w = bf16r(wj[jj]);
                const float o = exj[jj] >= 0 ? bf16r(bf16r(sum) + bf16_to_f32(dbv[jj])) : __builtin_nanf("");
                y += bf16r(o * w);
            }
        }
        __syncthreads();
    }
    if (sl == 0 && h < L.H) L.out[h] = f32_to_bf16(y);
}

template <int BITS, bool POW2G>
static void launch_go(const GoLayer& L, hipStream_t st) {
    const int C1 = 2 * L.I;
    hipLaunchKernelGGL((k_go_gate_up<BITS, POW2G>), dim3((C1 + kGoCols - 1) / kGoCols * L.S1 * L.k),
                       dim3(64 * kGoWaves), 0, st, L);
    hipLaunchKernelGGL((k_go_down<BITS, POW2G>), dim3((L.H + kGoCols - 1) / kGoCols * L.S2 * L.k),
                       dim3(64 * kGoWaves), 0, st, L);
    const dim3 og((L.H + kGoOutCols - 1) / kGoOutCols), ob(kGoOutCols * kGoOutSlices);
    const int per = (L.S2 + kGoOutSlices - 1) / kGoOutSlices;
    if (L.k <= 4 && per <= 6)
        hipLaunchKernelGGL((k_go_out<4, 6>), og, ob, 0, st, L);
    else
        hipLaunchKernelGGL((k_go_out<8, 8>), og, ob, 0, st, L);
}

}  // namespace wisp

using namespace wisp;

// gptoss.py:22-29
extern "C" int wisp_mxfp4_to_bf16(const uint8_t* blocks, const uint8_t* scales, int64_t ngroups, uint16_t* out,
                                  void* stream) {
    clear_error();
    if (!blocks || !scales || !out) return fail_inval("null pointer");
    if (ngroups < 0 || ngroups > ((int64_t)1 << 40)) return fail_inval("ngroups out of range");
    if (!aligned(blocks, 16) || !aligned(out, 16)) {
        set_error("blocks and out must be 16-byte aligned");
        return WISP_EALIGN;
    }
    if (ngroups == 0) return WISP_OK;
    hipLaunchKernelGGL(k_mxfp4, dim3((unsigned)((ngroups + 255) / 256)), dim3(256), 0, (hipStream_t)stream, blocks,
                       scales, ngroups, out);
    return check_launch("k_mxfp4");
}

extern "C" int64_t wisp_gptoss_ws_bytes(int k, int64_t H, int64_t I) {
    if (k < 1 || H < 1 || I < 1) return -1;
    const int64_t S1 = (H + 63) / 64, S2 = (I + kGoRows - 1) / kGoRows;  // S1: the most gate_up row blocks
    return 4 * ((int64_t)k * S1 * 2 * I + (int64_t)k * S2 * H);
}

// gptoss.py:126-131 (PagedGptOssBlock.forward, N == 1)
extern "C" int wisp_gptoss_decode(const uint8_t* pool, int64_t slot_bytes, int64_t nslots, const float* meta, int k,
                                  int64_t H, int64_t I, int bits, int64_t group, const uint16_t* x,
                                  const uint16_t* gate_up_bias, const uint16_t* down_bias, int64_t n_experts,
                                  float alpha, float limit, void* ws, uint16_t* out, void* stream) {
    clear_error();
    if (!pool || !meta || !x || !gate_up_bias || !down_bias || !ws || !out) return fail_inval("null pointer");
    if (!(bits == 4 || bits == 3 || bits == 2)) return fail_inval("bits must be 4, 3 or 2 for the fused kernels");
    if (k < 1 || k > 64) return fail_inval("k must be in [1, 64]");
    if (H < 32 || I < 16 || H % 32 || I % 16 || H > (1 << 16) || I > (1 << 16))
        return fail_inval("H a multiple of 32 and I of 16 (both <= 65536)");
    if (group < 32 || group % 32) return fail_inval("group must be a positive multiple of 32");
    if (n_experts < 1 || n_experts > (1 << 24)) return fail_inval("n_experts out of range");
    if (nslots < 1 || nslots > (1 << 24)) return fail_inval("nslots must be in [1, 2^24] (exact float ids)");
    const int64_t n = H * I;
    const int64_t nb = wisp_expert_nbytes(n, bits, group);
    if (nb < 0 || slot_bytes < nb) return fail_inval("slot_bytes is smaller than one expert");
    const int al = bits == 3 ? 4 : 4 * bits;
    if (!aligned(pool, al) || slot_bytes % al || !aligned(x, 4) || !aligned(ws, 16)) {
        set_error("pool base and slot_bytes must be %d-byte aligned for %d-bit experts; x 4, ws 16", al, bits);
        return WISP_EALIGN;
    }
    GoLayer L;
    L.pool = pool;
    L.slot_bytes = slot_bytes;
    L.nslots = (int)nslots;
    L.k = k;
    L.H = (int)H;
    L.I = (int)I;
    L.G = (int)group;
    L.E = (int)n_experts;
    L.n = n;
    L.scale_off = 3 * n * bits / 8;
    L.NG = 3 * n / group;
    L.meta = meta;
    L.x = x;
    L.gub = gate_up_bias;
    L.db = down_bias;
    L.alpha = alpha;
    L.limit = limit;
    const int rows_gu = 16 * go_pairs_gu(bits);
    L.S1 = (int)((H + rows_gu - 1) / rows_gu);
    L.S2 = (int)((I + kGoRows - 1) / kGoRows);
    L.p1 = static_cast<float*>(ws);
    L.p2 = L.p1 + (int64_t)k * L.S1 * 2 * I;
    L.out = out;
    hipStream_t st = (hipStream_t)stream;
    L.gsh = (group & (group - 1)) == 0 ? __builtin_ctzll((unsigned long long)group) : -1;
    const bool p2 = L.gsh >= 0;
    switch (bits) {
    case 4: p2 ? launch_go<4, true>(L, st) : launch_go<4, false>(L, st); break;
    case 3: p2 ? launch_go<3, true>(L, st) : launch_go<3, false>(L, st); break;
    default: p2 ? launch_go<2, true>(L, st) : launch_go<2, false>(L, st); break;
    }
    return check_launch("k_go");
}
