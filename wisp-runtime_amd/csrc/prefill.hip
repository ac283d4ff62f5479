// Grouped MoE prefill on gfx950: T tokens, each routed to k experts; per expert
// the token group runs gate/up (+ SiLU * up) and down as bf16 MFMA GEMMs whose
// weight tiles are dequantized into LDS from the packed slot-pool rows.
//
// Reference semantics: wisp/moe.py:131-137 (with 147-151): for every routed
// expert, dequantize its buffer to bf16 (quant.py:76-87, bit-exact here), run
// the expert MLP down(SiLU(gate x) * up x) on its tokens, weight by the token's
// routing weight and accumulate into the token's output, experts in ascending
// id order. Here the GEMMs accumulate in fp32 (MFMA), the activation between
// them is rounded to bf16 once (the MFMA operand type), the per-token sum is
// fp32 and the output is rounded to bf16 once.
//
// Data (all device, built by the caller from the routing):
//   pairs: the T*k (token, expert) pairs sorted by expert; tok[p] the token of
//          pair p, w[p] its routing weight; groups[u] = (slot, first pair,
//          pair count) of the u-th routed expert; back[t*k + j] = the pair of
//          token t's j-th expert in ascending expert id.
//   ws:    act bf16 [P, I] (gate_up output) | y fp32 [P, H] (weighted down output)
// Kernels:
//   k_pf_gate_up  grid (I/128, U, Z), 8 waves: per wave 16 act columns of one
//                 expert (their gate and up rows); K = H.
//   k_pf_down     grid (H/256, U, Z), 8 waves: per wave 32 down rows; K = I.
//   (workgroup z takes the group's token passes z, z+Z, ...)
//   k_pf_combine  out[t] = bf16(sum_j y[back[t, j]]).
// A wave owns 32 weight rows (two 16-row tiles), streams their codes one step
// (a pair of 128-wide quant groups, so whole 128-byte lines of a row) ahead,
// dequantizes them in registers straight into MFMA B fragments, and multiplies
// them against up to MT 16-token tiles of the group staged in LDS
// (v_mfma_f32_16x16x32_bf16, tokens as M, rows as N); each token fragment is
// reused by the two row tiles.
// K order inside a group: lane group g = lane/16 holds the group's 32-code
// chunk g, and MFMA k-substep s takes its codes 8s..8s+7; the A operand uses the
// same order, which leaves the dot products unchanged.
// Groups larger than one pass (MT*16 tokens) spread over Z workgroups.
// MFMA 16x16x32 bf16 lane layout (lane l): A[row l%16][k 8*(l/16) + 0..7],
// B[k 8*(l/16) + 0..7][col l%16], D[row 4*(l/16) + 0..3][col l%16].
// With the weights read once per expert the path is HBM-bound for T <= 512.
// 4-bit codes with an even number of K groups (the Qwen3 shapes) take the LDS-DMA
// form of the two GEMMs (k_pf_gate_up_dmag / k_pf_down_dmag, described at
// pf_gemm_dmag): the codes of a K step arrive as whole 128-byte lines straight into
// LDS, one step ahead, and the scales with them.
#include <math.h>

#include <algorithm>
#include <type_traits>

#include "wisp_device.hpp"
#include "wisp_internal.hpp"

namespace wisp {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// A workgroup owns 256 weight rows as NW waves x TPW 16-row tiles (NW * TPW = 16):
// 4 waves x 4 tiles for passes of up to two token tiles, 8 waves x 2 tiles for
// four (measured on C5: fewer, larger waves are faster while the passes are
// short, more waves once the 4-tile passes need registers).
constexpr int kPfMaxTiles = 4;

struct Prefill {
    const uint8_t* pool;
    int64_t slot_bytes, nmb;  // nmb: code bytes of one matrix
    int nslots, H, I, NGM, P, T;
    const int32_t* groups;  // [U][3]
    const int32_t* tok;     // [P]
    const float* w;         // [P]
    const uint16_t* x;      // [T, H]
    uint16_t* act;          // [P, I]
    float* y;               // [P, H]
    int gy, gz;             // the LDS-DMA kernels' logical grid: work items, workgroups per item's passes
};

__device__ __forceinline__ f32x4_t mfma16(uint4 a, uint4 b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                    c, 0, 0, 0);
}

// byte N of v as a float (v_cvt_f32_ubyteN: one instruction, no extract)
__device__ __forceinline__ float ubyte0(uint32_t v) { float r; asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(v)); return r; }
__device__ __forceinline__ float ubyte1(uint32_t v) { float r; asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(v)); return r; }
__device__ __forceinline__ float ubyte2(uint32_t v) { float r; asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(v)); return r; }
__device__ __forceinline__ float ubyte3(uint32_t v) { float r; asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(v)); return r; }
template <int B>
__device__ __forceinline__ float ubyte(uint32_t v) {
    return B == 0 ? ubyte0(v) : B == 1 ? ubyte1(v) : B == 2 ? ubyte2(v) : ubyte3(v);
}

// Dequantize 32 consecutive weights (one chunk) to 16 bf16 pairs, bit-exact with
// the dequant kernel: w = RTNE_bf16(fp32(q*s) + m). q*s is exact in binary32
// (q < 16, s an fp16 value), so a fused multiply-add rounds exactly where the
// separate multiply and add would. 4- and 2-bit codes are first spread one per
// byte, so that each becomes a float with one v_cvt_f32_ubyteN.
template <int BITS>
__device__ __forceinline__ void dequant_chunk(const uint32_t* d, float s, float m, uint32_t* out) {
    if constexpr (BITS == 4) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const uint32_t e = d[w] & 0x0F0F0F0Fu;         // codes 8w, 8w+2, 8w+4, 8w+6
            const uint32_t o = (d[w] >> 4) & 0x0F0F0F0Fu;  // codes 8w+1, 8w+3, 8w+5, 8w+7
            out[4 * w + 0] = pack_bf16x2(__builtin_fmaf(ubyte<0>(e), s, m), __builtin_fmaf(ubyte<0>(o), s, m));
            out[4 * w + 1] = pack_bf16x2(__builtin_fmaf(ubyte<1>(e), s, m), __builtin_fmaf(ubyte<1>(o), s, m));
            out[4 * w + 2] = pack_bf16x2(__builtin_fmaf(ubyte<2>(e), s, m), __builtin_fmaf(ubyte<2>(o), s, m));
            out[4 * w + 3] = pack_bf16x2(__builtin_fmaf(ubyte<3>(e), s, m), __builtin_fmaf(ubyte<3>(o), s, m));
        }
    } else if constexpr (BITS == 2) {
#pragma unroll
        for (int w = 0; w < 2; ++w) {
            uint32_t f[4];  // f[j] byte b = code 16w + 4b + j
#pragma unroll
            for (int j = 0; j < 4; ++j) f[j] = (d[w] >> (2 * j)) & 0x03030303u;
#define WISP_Q2(B)                                                                                      \
    out[8 * w + 2 * B] = pack_bf16x2(__builtin_fmaf(ubyte<B>(f[0]), s, m), __builtin_fmaf(ubyte<B>(f[1]), s, m));  \
    out[8 * w + 2 * B + 1] = pack_bf16x2(__builtin_fmaf(ubyte<B>(f[2]), s, m), __builtin_fmaf(ubyte<B>(f[3]), s, m));
            WISP_Q2(0)
            WISP_Q2(1)
            WISP_Q2(2)
            WISP_Q2(3)
#undef WISP_Q2
        }
    } else {
        uint32_t q[32];
        chunk_codes<BITS>(d, q);
#pragma unroll
        for (int i = 0; i < 16; ++i)
            out[i] = pack_bf16x2(__builtin_fmaf((float)q[2 * i], s, m), __builtin_fmaf((float)q[2 * i + 1], s, m));
    }
}

// Group u's (slot, first pair, count). Returns 0 for a group whose pair range is
// invalid (nothing is written), 1 for an invalid slot id (its rows are written
// as NaN, nothing is read from the pool), 2 for a valid group.
__device__ __forceinline__ int group_state(const Prefill& F, int u, int& slot, int& p0, int& cnt) {
    slot = F.groups[3 * u];
    p0 = F.groups[3 * u + 1];
    cnt = F.groups[3 * u + 2];
    if (!(p0 >= 0 && cnt > 0 && p0 + cnt <= F.P)) return 0;
    return (slot >= 0 && slot < F.nslots) ? 2 : 1;
}

// A wave's weight row tiles: the lane's code and scale pointers for tile 0
// (its row and chunk) and the tiles' offsets from them (wave-uniform).
// Scale/min table of a workgroup's 256 weight rows, staged in LDS when a row has
// at most kPfSmSteps quant groups (K <= 2048): entry [K step][local row] =
// s | m << 16 (fp16 bits). K-step major, so the 16 rows of a tile that one read
// touches are 16 consecutive words (distinct banks).
constexpr int kPfSmSteps = 16;

struct PfRows {
    const uint8_t* rc;   // codes of tile 0 at the lane's row and chunk
    const uint16_t* sp;  // fp16 scales of tile 0's row (one per 128-code group), global
    int64_t mn_off;      // mins - scales, in fp16 elements
    int64_t code_off[kPfMaxTiles], scale_off[kPfMaxTiles];
    const uint32_t* sml;  // LDS table at tile 0's row (nullptr: read sp/mn from global memory)
    int sml_off[kPfMaxTiles];  // per-tile local row offsets in the LDS table
};

// One K step's codes and fp16 scale/min (packed s | m << 16) of a lane's row in tile j.
// SMR > 0: the scale/min come from the workgroup's LDS table (row stride SMR); SMR == 0:
// from global memory. A compile-time choice: a run-time one compiled to a divergent branch
// whose loads made the compiler drain every outstanding load at the step loop's head.
template <int BITS, int SMR>
__device__ __forceinline__ void pf_load(const PfRows& R, int j, int kc, uint32_t* cd, uint32_t& sm) {
    load_chunk<BITS>(R.rc + R.code_off[j] + (int64_t)kc * 16 * BITS, cd);  // 128 codes per K step
    if constexpr (SMR > 0) {  // the LDS table (row stride SMR)
        sm = R.sml[R.sml_off[j] + kc * SMR];
    } else {
        const uint16_t* s = R.sp + R.scale_off[j] + kc;
        sm = (uint32_t)s[0] | ((uint32_t)s[R.mn_off] << 16);
    }
}

// Stage nrows * nk scale/min pairs (two contiguous fp16 runs, [row][K step],
// scales at `sc`, mins at sc + mn_off) into sml[kc * kPfSmRows + local0 + row]
// packed s | m << 16, with 16-byte loads (nrows * nk a multiple of 8; both runs
// 16-byte aligned). All threads of the workgroup take part.
__device__ __forceinline__ void pf_stage_scales(const uint16_t* sc, int64_t mn_off, int nrows, int nk, int local0,
                                                uint32_t* sml, int smr) {
    const int total = nrows * nk;  // entries, 8 per 16-byte load
    for (int e = (int)threadIdx.x * 8; e < total; e += (int)blockDim.x * 8) {
        const uint4 vs = *reinterpret_cast<const uint4*>(sc + e);
        const uint4 vm = *reinterpret_cast<const uint4*>(sc + mn_off + e);
        const uint32_t s4[4] = {vs.x, vs.y, vs.z, vs.w}, m4[4] = {vm.x, vm.y, vm.z, vm.w};
        int r = e / nk, kc = e - r * nk;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t sv = i & 1 ? s4[i >> 1] >> 16 : s4[i >> 1] & 0xFFFFu;
            const uint32_t mv = i & 1 ? m4[i >> 1] & 0xFFFF0000u : m4[i >> 1] << 16;
            sml[kc * smr + local0 + r] = sv | mv;
            if (++kc == nk) {
                kc = 0;
                ++r;
            }
        }
    }
}

// The step's 4 MFMA B fragments (k-substeps 0..3) from the lane's chunk.
template <int BITS>
__device__ __forceinline__ void pf_bfrag(const uint32_t* cd, uint32_t sm, uint4* b) {
    uint32_t v[16];
    if constexpr (BITS == 3)
        dequant_chunk<BITS>(cd, h2f((uint16_t)(sm & 0xFFFFu)), h2f((uint16_t)(sm >> 16)), v);
    else
        dequant32<BITS>(cd, sm, v);
#pragma unroll
    for (int s = 0; s < 4; ++s) b[s] = make_uint4(v[4 * s], v[4 * s + 1], v[4 * s + 2], v[4 * s + 3]);
}

// LDS row stride of a staged A tile in uint4: 32 (two K groups, 256 bf16) + 1
// pad, so the 16 rows one fragment read touches start 4 banks apart (no bank
// conflicts for the 128-bit reads).
constexpr int kArs = 33;

// One pass of the workgroup GEMM. The NW waves share the pass's NT*16 A rows
// (the token or activation rows of the group's pairs), staged a PAIR of K groups
// (256 values) at a time in LDS, double-buffered with one barrier per pair:
// thread t copies the pieces t + k*64*NW (k < RPT) of a pair, piece i being A
// row i/32, group half (i/16)&1, 16-byte column i%16; crow[k] = the start of
// its k-th row plus its column.
// Weight reads: a step covers two of the wave's row tiles over one group pair
// (TPW/2 steps per pair), so a lane requests its pieces of groups 2q and 2q+1
// of a row back to back -- the two halves of one 128-byte line. (Half lines
// requested one K step apart, ~1.5 us, reach HBM separately; a loads-only
// measurement with compute between the steps: 3.7 TB/s against 5.4 TB/s for
// whole lines.) Each step's codes are requested one step ahead, the next
// pair's A pieces at the start of a pair and written to LDS at its end.
// Loads go into register sets that swap roles (the loop is unrolled by two
// steps), never through a register copy: on this hardware a copy of a load's
// destination waits for the load, which would serialise the prefetch. Every
// thread of the workgroup calls it with the same nk; NT is the pass's exact
// tile count, so the loop has no per-tile branches.
template <int BITS>
struct PfStep {
    uint32_t cd[2][2][BITS], sm[2][2];  // [row tile of the step][group of the pair]: codes, s | m << 16
};

template <int BITS, int NT, int NW, int TPW, int SMR>
__device__ __forceinline__ void pf_gemm(const PfRows& R, const uint4* const* crow, uint4* lds, int nk,
                                        f32x4_t (*acc)[TPW]) {
    constexpr int TP = TPW / 2;  // steps per group pair
    constexpr int RPT = 8 * NT / NW;           // A pieces per thread and pair
    constexpr int BUF = NT * 16 * kArs;
    const int lane = threadIdx.x & 63, n = lane & 15, g = lane >> 4;
    const int cm = threadIdx.x >> 5, hh = (threadIdx.x >> 4) & 1, cc = threadIdx.x & 15;
    const int npairs = (nk + 1) >> 1, nsteps = npairs * TP;
    u32x4_t* ldv = reinterpret_cast<u32x4_t*>(lds);
#pragma unroll
    for (int mt = 0; mt < NT; ++mt)
#pragma unroll
        for (int j = 0; j < TPW; ++j) acc[mt][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    // step st: row tiles 2*(st%TP) + {0, 1}, groups 2*(st/TP) + {0, 1} (past the end: reload, in bounds)
    auto load_step = [&](PfStep<BITS>& S, int st) {
        const int q = st / TP, t0 = 2 * (st - q * TP);
        const int k0 = min(2 * q, nk - 1), k1 = min(2 * q + 1, nk - 1);
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
            pf_load<BITS, SMR>(R, t0 + jj, k0, S.cd[jj][0], S.sm[jj][0]);
            pf_load<BITS, SMR>(R, t0 + jj, k1, S.cd[jj][1], S.sm[jj][1]);
        }
    };
    auto load_a = [&](u32x4_t* av, int q) {
        const int kg = min(2 * q + hh, nk - 1);
#pragma unroll
        for (int k = 0; k < RPT; ++k) av[k] = *reinterpret_cast<const u32x4_t*>(crow[k] + kg * 16);
    };
    auto put_a = [&](const u32x4_t* av, int buf) {
#pragma unroll
        for (int k = 0; k < RPT; ++k) ldv[buf * BUF + (cm + 2 * NW * k) * kArs + 16 * hh + cc] = av[k];
    };
    // the MFMAs of step st: its two row tiles against the pair's A tile (buffer q&1)
    auto compute = [&](const PfStep<BITS>& S, int st) {
        const int q = st / TP, t0 = 2 * (st - q * TP);
        const uint4* A = lds + (q & 1) * BUF;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            if (2 * q + h >= nk) break;  // odd nk: the last pair has one group
            uint4 xa[NT][4];
#pragma unroll
            for (int mt = 0; mt < NT; ++mt)
#pragma unroll
                for (int s = 0; s < 4; ++s) xa[mt][s] = A[(mt * 16 + n) * kArs + 16 * h + 4 * g + s];
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
                uint4 b[4];
                pf_bfrag<BITS>(S.cd[jj][h], S.sm[jj][h], b);
#pragma unroll
                for (int s = 0; s < 4; ++s)
#pragma unroll
                    for (int mt = 0; mt < NT; ++mt)
                        acc[mt][t0 + jj] = mfma16(xa[mt][s], b[s], acc[mt][t0 + jj]);
            }
        }
    };
    // the A tile around step st: the next pair's pieces requested (and the barrier)
    // at a pair's first step, written to LDS after its last
    auto step = [&](const PfStep<BITS>& C, PfStep<BITS>& N, u32x4_t* an, int st) {
        const int q = st / TP;
        if (st == q * TP) {
            load_a(an, min(q + 1, npairs - 1));
            load_step(N, st + 1);
            __syncthreads();  // pair q's A tile is in buffer q&1; pair q-1's reads are done
        } else {
            load_step(N, st + 1);
        }
        compute(C, st);
        if (st == q * TP + TP - 1 && q + 1 < npairs) put_a(an, (q + 1) & 1);  // buffer last read in pair q-1
    };
    PfStep<BITS> S0, S1;
    u32x4_t an[RPT];
    load_a(an, 0);
    load_step(S0, 0);
    put_a(an, 0);
    // whole rounds of two steps, then the odd one: no exit from inside a round, so the
    // compiler's load counting is the same on every path into the loop head (an exit
    // mid-round made it drain every load there, prefetch included)
    int st = 0;
    for (const int nr = nsteps & ~1; st < nr; st += 2) {
        step(S0, S1, an, st);
        step(S1, S0, an, st + 1);
    }
    if (st < nsteps) step(S0, S1, an, st);
}

// One pass of kernel gate_up over NT 16-token tiles starting at pair mb of the
// group: A rows are the pairs' tokens (rows past cnt repeat the last pair).
// The wave's tiles j < TPW/2 are gate rows c0 + 16j, the others the same up rows.
template <int BITS, int NT, int NW, int TPW, int SMR>
__device__ __forceinline__ void pf_gate_up_pass(const Prefill& F, const PfRows& R, int nk, int c0, int p0, int cnt,
                                                int mb, uint4* lds) {
    constexpr int HT = TPW / 2, RPT = 8 * NT / NW;
    const int lane = threadIdx.x & 63, n = lane & 15, g = lane >> 4;
    const uint4* crow[RPT];
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
        int t = F.tok[p0 + min(mb + (int)(threadIdx.x >> 5) + 2 * NW * k, cnt - 1)];
        t = min(max(t, 0), F.T - 1);
        crow[k] = reinterpret_cast<const uint4*>(F.x + (int64_t)t * F.H) + (threadIdx.x & 15);
    }
    f32x4_t acc[NT][TPW];
    pf_gemm<BITS, NT, NW, TPW, SMR>(R, crow, lds, nk, acc);
    // D layout: acc[mt][j][i] = token mb + mt*16 + 4g + i, row tile j column n
#pragma unroll
    for (int mt = 0; mt < NT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int m = mb + mt * 16 + 4 * g + i;
            if (m < cnt) {
                uint16_t* dst = F.act + (int64_t)(p0 + m) * F.I + c0 + n;
#pragma unroll
                for (int j = 0; j < HT; ++j) dst[16 * j] = f32_to_bf16(silu_mul(acc[mt][j][i], acc[mt][j + HT][i]));
            }
        }
}

// One pass of kernel down (A rows: the pairs' activations), stores w * y.
template <int BITS, int NT, int NW, int TPW, int SMR>
__device__ __forceinline__ void pf_down_pass(const Prefill& F, const PfRows& R, int nk, int h0, int p0, int cnt,
                                             int mb, uint4* lds) {
    constexpr int RPT = 8 * NT / NW;
    const int lane = threadIdx.x & 63, n = lane & 15, g = lane >> 4;
    const uint4* crow[RPT];
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
        const int m = min(mb + (int)(threadIdx.x >> 5) + 2 * NW * k, cnt - 1);
        crow[k] = reinterpret_cast<const uint4*>(F.act + (int64_t)(p0 + m) * F.I) + (threadIdx.x & 15);
    }
    f32x4_t acc[NT][TPW];
    pf_gemm<BITS, NT, NW, TPW, SMR>(R, crow, lds, nk, acc);
#pragma unroll
    for (int mt = 0; mt < NT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int m = mb + mt * 16 + 4 * g + i;
            if (m < cnt) {
                const float wp = F.w[p0 + m];
                float* dst = F.y + (int64_t)(p0 + m) * F.H + h0 + n;
#pragma unroll
                for (int j = 0; j < TPW; ++j) dst[j * 16] = wp * acc[mt][j][i];
            }
        }
}

// ---------------------------------------------------------------------------
// gate_up: act[p][r] = bf16(silu(g) * u), g/u = x[tok[p]] . W{gate,up}[r]
// grid (I/128, U, Z), NW waves; wave w of workgroup x owns act columns
// c0 = x*128 + w*8*TPW .. +8*TPW-1: row tiles {gate c0 + 16j, up c0 + 16j}.
template <int BITS, int MT, int NW, int RWG, bool SML>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2))) void k_pf_gate_up(const Prefill F) {
    constexpr int SMR = SML ? RWG : 0;
    constexpr int TPW = RWG / (16 * NW), HT = TPW / 2, CW = 8 * TPW, HR = RWG / 2;
    __shared__ uint4 lds[2 * MT * 16 * kArs];
    __shared__ uint32_t sml[RWG * kPfSmSteps];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int n = lane & 15, g = lane >> 4;
    const int c0 = blockIdx.x * HR + wv * CW, u = blockIdx.y;
    int slot, p0, cnt;
    const int gs = group_state(F, u, slot, p0, cnt);
    if (gs == 0) return;
    if (gs == 1) {
        for (int i = lane; i < cnt * CW; i += 64)
            F.act[(int64_t)(p0 + i / CW) * F.I + c0 + (i % CW)] = 0x7FC0;  // bf16 NaN
        return;
    }
    const uint8_t* base = F.pool + (int64_t)slot * F.slot_bytes;
    const uint16_t* sc = reinterpret_cast<const uint16_t*>(base + 3 * F.nmb);
    const uint16_t* mn = sc + 3 * F.NGM;
    const int nk = F.H / 128;
    const int64_t rowb = (int64_t)F.H * BITS / 8;
    PfRows R;
    R.rc = base + (int64_t)(c0 + n) * rowb + g * 4 * BITS;
    R.sp = sc + (int64_t)(c0 + n) * nk;
    R.mn_off = mn - sc;
    R.sml = nullptr;
#pragma unroll
    for (int j = 0; j < TPW; ++j) {  // tiles gate c0 + 16j (j < HT), up c0 + 16(j - HT)
        const int mat = j / HT, dr = (j % HT) * 16;
        R.code_off[j] = mat * F.nmb + dr * rowb;
        R.scale_off[j] = (int64_t)mat * F.NGM + (int64_t)dr * nk;
        R.sml_off[j] = mat * HR + dr;  // local rows: gate 0..HR-1, up HR..RWG-1
    }
    if constexpr (SML) {  // the workgroup's HR gate and HR up rows' scale/min, once (nk <= kPfSmSteps)
        const int r0 = blockIdx.x * HR;
        pf_stage_scales(sc + (int64_t)r0 * nk, mn - sc, HR, nk, 0, sml, RWG);
        pf_stage_scales(sc + F.NGM + (int64_t)r0 * nk, mn - sc, HR, nk, HR, sml, RWG);
        __syncthreads();
        R.sml = sml + wv * CW + n;
    }
    constexpr int MB = MT * 16;
    for (int mb = blockIdx.z * MB; mb < cnt; mb += gridDim.z * MB) {
        const int nt = min(MT, (cnt - mb + 15) / 16);  // 16-token tiles in this pass (workgroup-uniform)
        if (MT >= 4 && nt >= 4) pf_gate_up_pass<BITS, (MT >= 4 ? 4 : 1), NW, TPW, SMR>(F, R, nk, c0, p0, cnt, mb, lds);
        else if (MT >= 3 && nt == 3) pf_gate_up_pass<BITS, (MT >= 3 ? 3 : 1), NW, TPW, SMR>(F, R, nk, c0, p0, cnt, mb, lds);
        else if (MT >= 2 && nt == 2) pf_gate_up_pass<BITS, (MT >= 2 ? 2 : 1), NW, TPW, SMR>(F, R, nk, c0, p0, cnt, mb, lds);
        else pf_gate_up_pass<BITS, 1, NW, TPW, SMR>(F, R, nk, c0, p0, cnt, mb, lds);
        __syncthreads();  // the next pass restages LDS buffer 0
    }
}

// ---------------------------------------------------------------------------
// down: y[p][h] = w[p] * (act[p] . Wdown[h]), fp32
// grid (H/256, U, Z), NW waves; wave w of workgroup x owns rows
// x*256 + w*16*TPW .. +16*TPW-1.
template <int BITS, int MT, int NW, int RWG, bool SML>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2))) void k_pf_down(const Prefill F) {
    constexpr int SMR = SML ? RWG : 0;
    constexpr int TPW = RWG / (16 * NW), RW = 16 * TPW;
    __shared__ uint4 lds[2 * MT * 16 * kArs];
    __shared__ uint32_t sml[RWG * kPfSmSteps];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int n = lane & 15, g = lane >> 4;
    const int h0 = blockIdx.x * RWG + wv * RW, u = blockIdx.y;
    int slot, p0, cnt;
    const int gs = group_state(F, u, slot, p0, cnt);
    if (gs == 0) return;
    if (gs == 1) {
        for (int i = lane; i < cnt * RW; i += 64)
            F.y[(int64_t)(p0 + i / RW) * F.H + h0 + (i % RW)] = __builtin_nanf("");
        return;
    }
    const uint8_t* base = F.pool + (int64_t)slot * F.slot_bytes;
    const uint16_t* sc = reinterpret_cast<const uint16_t*>(base + 3 * F.nmb);
    const uint16_t* mn = sc + 3 * F.NGM;
    const int nk = F.I / 128;
    const int64_t rowb = (int64_t)F.I * BITS / 8;
    PfRows R;
    R.rc = base + 2 * F.nmb + (int64_t)(h0 + n) * rowb + g * 4 * BITS;
    R.sp = sc + 2 * (int64_t)F.NGM + (int64_t)(h0 + n) * nk;
    R.mn_off = mn - sc;
    R.sml = nullptr;
#pragma unroll
    for (int j = 0; j < TPW; ++j) {  // tiles h0 + 16j
        R.code_off[j] = (int64_t)j * 16 * rowb;
        R.scale_off[j] = (int64_t)j * 16 * nk;
        R.sml_off[j] = j * 16;
    }
    if constexpr (SML) {  // the workgroup's RWG rows' scale/min, once (nk <= kPfSmSteps)
        const int hb = blockIdx.x * RWG;
        pf_stage_scales(sc + 2 * (int64_t)F.NGM + (int64_t)hb * nk, mn - sc, RWG, nk, 0, sml, RWG);
        __syncthreads();
        R.sml = sml + wv * RW + n;
    }
    constexpr int MB = MT * 16;
    for (int mb = blockIdx.z * MB; mb < cnt; mb += gridDim.z * MB) {
        const int nt = min(MT, (cnt - mb + 15) / 16);
        if (MT >= 4 && nt >= 4) pf_down_pass<BITS, (MT >= 4 ? 4 : 1), NW, TPW, SMR>(F, R, nk, h0, p0, cnt, mb, lds);
        else if (MT >= 3 && nt == 3) pf_down_pass<BITS, (MT >= 3 ? 3 : 1), NW, TPW, SMR>(F, R, nk, h0, p0, cnt, mb, lds);
        else if (MT >= 2 && nt == 2) pf_down_pass<BITS, (MT >= 2 ? 2 : 1), NW, TPW, SMR>(F, R, nk, h0, p0, cnt, mb, lds);
        else pf_down_pass<BITS, 1, NW, TPW, SMR>(F, R, nk, h0, p0, cnt, mb, lds);
        __syncthreads();
    }
}

// ===========================================================================
// LDS-DMA form (4-bit codes, an even number nk <= kPfSmSteps of K groups):
// pf_gemm_dmag, k_pf_gate_up_dmag, k_pf_down_dmag.
// A workgroup of 4 waves owns 128 weight rows, a wave 32 (two 16-row tiles).
// A K step is one pair of groups (256 K): for each row the step's codes are one
// whole 128-byte line, and every line is fetched by ONE request:
// global_load_lds_dwordx4 moves 64 lanes x 16 bytes = 8 rows x 128 bytes
// straight into LDS (no VGPRs held while in flight), where each lane then reads
// its MFMA fragment chunk. (Loads into registers in the fragment layout can only
// cover 16 rows x 64 bytes per instruction, i.e. every line in two halves, which
// measured 23 % slower in a loads-only run.)
//   * codes: per wave one private slot of 4 KB codes + 256 B of the rows' fp16
//     scale and min pairs; it is read into registers at the step's start and
//     then refilled with the next step's codes, which have the whole step to
//     arrive.
//   * tokens (A): the NT*16 rows x 256 bytes of one quant group, double-
//     buffered, loaded by all waves (DMA as well) and published by a barrier
//     per group. A workgroup holds 2 x NT*16*256 B + 17 KB of LDS, so three
//     (NT = 4) or four (NT = 2) workgroups share a CU: measured on C5 at T = 512,
//     three workgroups with one slot per wave beat two with two slots (125-129 µs
//     against 142-145), the SIMDs' dequantisation, MFMA and LDS work then
//     covering each other's waits.
//   * A(2st+1) is issued before the step's code DMAs, so the step's one inner
//     wait (for A(2st+1)) leaves the next step's codes in flight.
//   * in LDS, piece p (16 bytes) of row r is stored at position p ^ (r & 7):
//     the 8 lanes of a 128-bit LDS read phase (rows n..n+7, one piece) then hit
//     8 different bank groups.
// The compiler neither emits nor counts these loads, so every wait for them is
// an explicit s_waitcnt vmcnt(n), n = the number of DMA instructions this wave
// issued after the awaited ones (vector memory loads complete in order), and
// nothing else in the loop issues vector memory loads. Where fewer DMAs follow
// near the end of a tile the count is smaller: waiting longer is always safe.
// ===========================================================================
__device__ __forceinline__ uint32_t lds_addr(const void* p) { return (uint32_t)(uintptr_t)p; }
// s_waitcnt vmcnt(n) (expcnt and lgkmcnt not waited for), gfx9 encoding
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | 0x70 | 0xF00 | ((N >> 4) << 14));
    asm volatile("" ::: "memory");
}
__device__ __forceinline__ void wait_lgkm0() {
    __builtin_amdgcn_s_waitcnt(0xC07F);
    asm volatile("" ::: "memory");
}

// 64 lanes x 16 (dma16s) or 4 (dma4s) bytes from sbase + each lane's 32-bit offset to
// LDS [lds, lds + 64*size): the base in an SGPR pair, no 64-bit address arithmetic per lane.
// M0 carries the LDS address and is declared clobbered. The backend reserves M0, so that
// clobber is advisory (hence the silenced warning); what makes the write safe is that no
// compiler-emitted instruction in these kernels uses M0, which tests/test_build_isa.py
// checks on the generated gfx950 assembly.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16s(uint32_t lds, const void* sbase, uint32_t voff) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
                 :
                 : "s"(lds), "v"(voff), "s"(sbase)
                 : "memory", "m0");
}
__device__ __forceinline__ void dma4s(uint32_t lds, const void* sbase, uint32_t voff) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, %2"
                 :
                 : "s"(lds), "v"(voff), "s"(sbase)
                 : "memory", "m0");
}
#pragma clang diagnostic pop
__device__ __forceinline__ const uint8_t* uniform_ptr(const void* p) {
    const uint64_t v = (uint64_t)(uintptr_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return reinterpret_cast<const uint8_t*>((uintptr_t)(((uint64_t)hi << 32) | lo));
}

// One wave's view of a tile for the LDS-DMA GEMM (all byte offsets).
struct PfDma {
    const uint8_t* cb[2];  // code base of row tile jj (its first row, pair 0), wave-uniform
    const uint8_t* sb;     // scale base: fp16 scales of the wave's row 0, pair 0, wave-uniform
    int64_t rowb;          // code bytes of one row
    uint32_t voc;          // lane code offset: row lane>>3 of an 8-row block, piece (lane&7)^(lane>>3)
    uint32_t vos;          // lane scale offset: lanes 0-31 scale pair, 32-63 min pair of the wave's row lane&31
};

// per wave: one slot of 4 KB codes + 256 B scales
constexpr int kDmaSlot = 4096 + 256;

// NT token tiles, NW waves of two 16-row tiles each; abase: uniform A base (group 0),
// avo[k]: the lane's A offset for its k-th piece; abuf: 2 x NT*16 rows x 256 B;
// ring: this wave's slot. Issue order of step st (C = the step's 5 code and scale DMAs,
// A(G) = the RPTG token DMAs of group G):
//   wait all, barrier | A(2st+1) | read the slot | C(st+1) | group 2st
//   wait A(2st+1) (C(st+1) stays in flight), barrier | A(2st+2) | group 2st+1
template <int NT, int NW>
__device__ __forceinline__ void pf_gemm_dmag(const PfDma& R, const uint8_t* abase, const uint32_t* avo, uint8_t* abuf,
                                             uint8_t* ring, int nk, f32x4_t (*acc)[2]) {
    constexpr int RPTG = 4 * NT / NW;  // A DMA instructions per wave and group
    static_assert(RPTG >= 1 && (4 * NT) % NW == 0, "A pieces per wave");
    constexpr int ABUF = NT * 16 * 256;
    constexpr int CN = 5;  // code and scale DMA instructions per step
    const int lane = threadIdx.x & 63, n = lane & 15, g = lane >> 4;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nsteps = nk >> 1;
#pragma unroll
    for (int mt = 0; mt < NT; ++mt) acc[mt][0] = acc[mt][1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    const uint32_t ring_l = lds_addr(ring), abuf_l = lds_addr(abuf);
    auto issue_c = [&](int st) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            dma16s(ring_l + i * 1024, R.cb[i >> 1] + (i & 1) * 8 * R.rowb + (int64_t)st * 128, R.voc);
        dma4s(ring_l + 4096, R.sb + st * 4, R.vos);
    };
    auto issue_a = [&](int G) {
        const uint32_t dst = abuf_l + (G & 1) * ABUF;
#pragma unroll
        for (int k = 0; k < RPTG; ++k) dma16s(dst + 1024 * (wv + NW * k), abase + G * 256, avo[k]);
    };
    const uint32_t co0 = 128 * n + 16 * ((0 + g) ^ (n & 7)), co1 = 128 * n + 16 * ((4 + g) ^ (n & 7));
    issue_c(0);
    issue_a(0);
    for (int st = 0; st < nsteps; ++st) {
        wait_vm<0>();     // C(st) and A(2st)
        __syncthreads();  // every wave's part of A(2st) landed; every read of group 2st-1 ended
        issue_a(2 * st + 1);
        uint32_t cd[2][2][4], sm[2][2];
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
            const uint4 v0 = *reinterpret_cast<const uint4*>(ring + 2048 * jj + co0);
            const uint4 v1 = *reinterpret_cast<const uint4*>(ring + 2048 * jj + co1);
            cd[jj][0][0] = v0.x; cd[jj][0][1] = v0.y; cd[jj][0][2] = v0.z; cd[jj][0][3] = v0.w;
            cd[jj][1][0] = v1.x; cd[jj][1][1] = v1.y; cd[jj][1][2] = v1.z; cd[jj][1][3] = v1.w;
            const uint32_t sp = *reinterpret_cast<const uint32_t*>(ring + 4096 + 4 * (16 * jj + n));
            const uint32_t mp = *reinterpret_cast<const uint32_t*>(ring + 4096 + 128 + 4 * (16 * jj + n));
            sm[jj][0] = __builtin_amdgcn_perm(mp, sp, 0x05040100u);
            sm[jj][1] = __builtin_amdgcn_perm(mp, sp, 0x07060302u);
        }
        wait_lgkm0();  // the slot is read: it may be refilled
        if (st + 1 < nsteps) issue_c(st + 1);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int G = 2 * st + h;
            if (h == 1) {
                if (st + 1 < nsteps) wait_vm<CN>(); else wait_vm<0>();  // A(2st+1)
                __syncthreads();  // every wave's part of A(2st+1) landed; every read of group 2st ended
                if (G + 1 < nk) issue_a(G + 1);
            }
            const uint8_t* A = abuf + (G & 1) * ABUF;
            uint4 xa[NT][4];
#pragma unroll
            for (int mt = 0; mt < NT; ++mt)
#pragma unroll
                for (int s = 0; s < 4; ++s)
                    xa[mt][s] = *reinterpret_cast<const uint4*>(A + 256 * (16 * mt + n) + 16 * ((4 * g + s) ^ (n & 7)));
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
                uint4 b[4];
                pf_bfrag<4>(cd[jj][h], sm[jj][h], b);
#pragma unroll
                for (int s = 0; s < 4; ++s)
#pragma unroll
                    for (int mt = 0; mt < NT; ++mt) acc[mt][jj] = mfma16(xa[mt][s], b[s], acc[mt][jj]);
            }
        }
    }
}

// Passes of NT = 5..8 token tiles (items of 65-128 pairs) in the same LDS: the token
// tile is staged half a quant group at a time (NT*16 rows x 128 bytes: the pieces of
// K substeps 2hh and 2hh+1 of every lane group, 8 per row, piece p of row r at
// p ^ (r & 7)), double-buffered with one barrier per half group, so a 128-token tile
// needs no more LDS than a 64-token tile staged per group. Each group's codes are
// dequantized once (both halves of the group use the same B fragments), so an item of
// up to 128 pairs pays one dequantisation of its rows instead of two.
// Issue order of step st (stages q = 4st .. 4st+3, stage q = half q&1 of group q>>1):
//   wait all, barrier | A(4st+1) | read the slot | C(st+1) | stage 4st
//   wait A(4st+1) (C(st+1) in flight), barrier | A(4st+2) | stage 4st+1
//   wait all, barrier | A(4st+3) | stage 4st+2
//   wait all, barrier | A(4st+4) | stage 4st+3
// avo[k]: the lane's offset of its k-th A piece for group 0, half 0 (the lane's logical
// piece p = 2g + s' maps to the group's byte 16 * (4g + 2hh + s')).
template <int NT, int NW>
__device__ __forceinline__ void pf_gemm_dmag_h(const PfDma& R, const uint8_t* abase, const uint32_t* avo,
                                               uint8_t* abuf, uint8_t* ring, int nk, f32x4_t (*acc)[2]) {
    constexpr int RPTS = 2 * NT / NW;  // A DMA instructions per wave and stage
    static_assert(RPTS >= 1 && (2 * NT) % NW == 0, "A pieces per wave");
    constexpr int SBUF = NT * 16 * 128;
    constexpr int CN = 5;
    const int lane = threadIdx.x & 63, n = lane & 15, g = lane >> 4;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nsteps = nk >> 1, nst = 2 * nk;
#pragma unroll
    for (int mt = 0; mt < NT; ++mt) acc[mt][0] = acc[mt][1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    const uint32_t ring_l = lds_addr(ring), abuf_l = lds_addr(abuf);
    auto issue_c = [&](int st) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            dma16s(ring_l + i * 1024, R.cb[i >> 1] + (i & 1) * 8 * R.rowb + (int64_t)st * 128, R.voc);
        dma4s(ring_l + 4096, R.sb + st * 4, R.vos);
    };
    auto issue_a = [&](int q) {
        const uint32_t dst = abuf_l + (q & 1) * SBUF;
        const uint8_t* src = abase + (q >> 1) * 256 + (q & 1) * 32;
#pragma unroll
        for (int k = 0; k < RPTS; ++k) dma16s(dst + 1024 * (wv + NW * k), src, avo[k]);
    };
    const uint32_t co0 = 128 * n + 16 * ((0 + g) ^ (n & 7)), co1 = 128 * n + 16 * ((4 + g) ^ (n & 7));
    issue_c(0);
    issue_a(0);
    for (int st = 0; st < nsteps; ++st) {
        uint32_t cd[2][2][4], sm[2][2];
        uint4 b[2][4];  // B fragments of the current group, kept across its half-group barrier
#pragma unroll
        for (int hq = 0; hq < 4; ++hq) {
            const int q = 4 * st + hq, h = hq >> 1, hh = hq & 1;
            if (hq == 1 && st + 1 < nsteps) wait_vm<CN>(); else wait_vm<0>();  // A(q) (and at hq 0, C(st))
            __syncthreads();  // every wave's part of A(q) landed; every read of stage q-1 ended
            if (q + 1 < nst) issue_a(q + 1);
            if (hq == 0) {
#pragma unroll
                for (int jj = 0; jj < 2; ++jj) {
                    const uint4 v0 = *reinterpret_cast<const uint4*>(ring + 2048 * jj + co0);
                    const uint4 v1 = *reinterpret_cast<const uint4*>(ring + 2048 * jj + co1);
                    cd[jj][0][0] = v0.x; cd[jj][0][1] = v0.y; cd[jj][0][2] = v0.z; cd[jj][0][3] = v0.w;
                    cd[jj][1][0] = v1.x; cd[jj][1][1] = v1.y; cd[jj][1][2] = v1.z; cd[jj][1][3] = v1.w;
                    const uint32_t sp = *reinterpret_cast<const uint32_t*>(ring + 4096 + 4 * (16 * jj + n));
                    const uint32_t mp = *reinterpret_cast<const uint32_t*>(ring + 4096 + 128 + 4 * (16 * jj + n));
                    sm[jj][0] = __builtin_amdgcn_perm(mp, sp, 0x05040100u);
                    sm[jj][1] = __builtin_amdgcn_perm(mp, sp, 0x07060302u);
                }
                wait_lgkm0();  // the slot is read: it may be refilled
                if (st + 1 < nsteps) issue_c(st + 1);
            }
            const uint8_t* A = abuf + (q & 1) * SBUF;
            if (hh == 0) {
#pragma unroll
                for (int jj = 0; jj < 2; ++jj) pf_bfrag<4>(cd[jj][h], sm[jj][h], b[jj]);
            }
#pragma unroll
            for (int mt = 0; mt < NT; ++mt) {
                uint4 xa[2];
#pragma unroll
                for (int s = 0; s < 2; ++s)
                    xa[s] = *reinterpret_cast<const uint4*>(A + 128 * (16 * mt + n) + 16 * ((2 * g + s) ^ (n & 7)));
#pragma unroll
                for (int s = 0; s < 2; ++s)
#pragma unroll
                    for (int jj = 0; jj < 2; ++jj) acc[mt][jj] = mfma16(xa[s], b[jj][2 * hh + s], acc[mt][jj]);
            }
        }
    }
}

template <int MT, int NW, bool GATE_UP, class Epi>
__device__ __forceinline__ void pf_dmag_passes(const Prefill& F, const PfDma& R, int p0, int cnt, uint8_t* ab,
                                               uint8_t* ringw, int nk, int bz, int nz, Epi epi) {
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    constexpr int MB = MT * 16;
    for (int mb = bz * MB; mb < cnt; mb += nz * MB) {
        const int nt = min(MT, (cnt - mb + 15) / 16);
        auto pass = [&](auto NTc) {
            constexpr int NT = decltype(NTc)::value, RPTG = 4 * NT / NW;
            uint32_t avo[RPTG];
            const uint8_t* abase;
            if constexpr (GATE_UP) {
                abase = uniform_ptr(F.x);
#pragma unroll
                for (int k = 0; k < RPTG; ++k) {
                    const int r = 4 * (wv + NW * k) + (lane >> 4);
                    int t = F.tok[p0 + min(mb + r, cnt - 1)];
                    t = min(max(t, 0), F.T - 1);
                    avo[k] = (uint32_t)t * (uint32_t)F.H * 2u + 16u * ((lane & 15) ^ (r & 7));
                }
            } else {
                abase = uniform_ptr(F.act + (int64_t)p0 * F.I);
#pragma unroll
                for (int k = 0; k < RPTG; ++k) {
                    const int r = 4 * (wv + NW * k) + (lane >> 4);
                    const int m = min(mb + r, cnt - 1);
                    avo[k] = (uint32_t)m * (uint32_t)F.I * 2u + 16u * ((lane & 15) ^ (r & 7));
                }
            }
            f32x4_t acc[NT][2];
            pf_gemm_dmag<NT, NW>(R, abase, avo, ab, ringw, nk, acc);
            epi(acc, mb);
        };
        // 5..8 tiles: staged half a group at a time (pf_gemm_dmag_h); lane l of A DMA
        // instruction k covers row 8 (wv + NW k) + l/8 at LDS position l%8
        auto pass_h = [&](auto NTc) {
            constexpr int NT = decltype(NTc)::value, RPTS = 2 * NT / NW;
            uint32_t avo[RPTS];
            const uint8_t* abase;
#pragma unroll
            for (int k = 0; k < RPTS; ++k) {
                const int r = 8 * (wv + NW * k) + (lane >> 3);
                const int p = (lane & 7) ^ (r & 7);
                const uint32_t piece = 16u * (uint32_t)(4 * (p >> 1) + (p & 1));
                const int m = min(mb + r, cnt - 1);
                if constexpr (GATE_UP) {
                    int t = F.tok[p0 + m];
                    t = min(max(t, 0), F.T - 1);
                    avo[k] = (uint32_t)t * (uint32_t)F.H * 2u + piece;
                } else {
                    avo[k] = (uint32_t)m * (uint32_t)F.I * 2u + piece;
                }
            }
            if constexpr (GATE_UP) abase = uniform_ptr(F.x);
            else abase = uniform_ptr(F.act + (int64_t)p0 * F.I);
            f32x4_t acc[NT][2];
            pf_gemm_dmag_h<NT, NW>(R, abase, avo, ab, ringw, nk, acc);
            epi(acc, mb);
        };
        bool half = false;
        if constexpr (MT >= 8) {
            half = nt >= 5;
            if (nt >= 7) pass_h(std::integral_constant<int, 8>{});
            else if (nt >= 5) pass_h(std::integral_constant<int, 6>{});
        }
        if (half) {
        } else if (MT >= 4 && nt >= 4) pass(std::integral_constant<int, (MT >= 4 ? 4 : 1)>{});
        else if (MT >= 3 && nt == 3) pass(std::integral_constant<int, (MT >= 3 ? 3 : 1)>{});
        else if (MT >= 2 && nt == 2) pass(std::integral_constant<int, (MT >= 2 ? 2 : 1)>{});
        else pass(std::integral_constant<int, 1>{});
        __syncthreads();
    }
}

template <int MT, int NW>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2))) void k_pf_gate_up_dmag(const Prefill F) {
    constexpr int RWG = 32 * NW, HR = RWG / 2, CW = 16;
    __shared__ uint4 abuf[2 * (MT > 4 ? 4 : MT) * 16 * 16];  // 5..8 tiles: staged per half group
    __shared__ uint4 ring[NW * kDmaSlot / 16];
    const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = lane & 15, g = lane >> 4;
    // one-dimensional launch of (I / HR) x gy x gz workgroups: an item's row blocks share an
    // XCD (items dealt round robin), so its token tile is fetched into one L2
    int bx, u, bz;
    xcd_rr_block(F.I / HR, F.gy, F.gz, bx, u, bz);
    const int c0 = bx * HR + wv * CW;
    int slot, p0, cnt;
    const int gs = group_state(F, u, slot, p0, cnt);
    if (gs == 0) return;
    if (gs == 1) {
        for (int i = lane; i < cnt * CW; i += 64)
            F.act[(int64_t)(p0 + i / CW) * F.I + c0 + (i % CW)] = 0x7FC0;
        return;
    }
    const uint8_t* base = F.pool + (int64_t)slot * F.slot_bytes;
    const int nk = F.H / 128;
    PfDma R;
    R.rowb = (int64_t)F.H / 2;
    R.cb[0] = uniform_ptr(base + (int64_t)c0 * R.rowb);
    R.cb[1] = uniform_ptr(base + F.nmb + (int64_t)c0 * R.rowb);
    R.voc = (uint32_t)((lane >> 3) * R.rowb + 16 * ((lane & 7) ^ (lane >> 3)));
    const uint8_t* sc = base + 3 * F.nmb;
    R.sb = uniform_ptr(sc + (int64_t)c0 * nk * 2);
    R.vos = (uint32_t)((lane >= 32 ? 3 * (int64_t)F.NGM * 2 : 0) + ((lane & 31) >> 4) * (int64_t)F.NGM * 2 +
                       (lane & 15) * nk * 2);
    uint8_t* ringw = reinterpret_cast<uint8_t*>(ring) + wv * kDmaSlot;
    uint8_t* ab = reinterpret_cast<uint8_t*>(abuf);
    pf_dmag_passes<MT, NW, true>(F, R, p0, cnt, ab, ringw, nk, bz, F.gz, [&](auto& acc, int mb) {
        constexpr int NT = sizeof(acc) / sizeof(acc[0]);
#pragma unroll
        for (int mt = 0; mt < NT; ++mt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = mb + mt * 16 + 4 * g + i;
                if (m < cnt) F.act[(int64_t)(p0 + m) * F.I + c0 + n] = f32_to_bf16(silu_mul(acc[mt][0][i], acc[mt][1][i]));
            }
    });
}

template <int MT, int NW>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2))) void k_pf_down_dmag(const Prefill F) {
    constexpr int RWG = 32 * NW, RW = 32;
    __shared__ uint4 abuf[2 * (MT > 4 ? 4 : MT) * 16 * 16];  // 5..8 tiles: staged per half group
    __shared__ uint4 ring[NW * kDmaSlot / 16];
    const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n = lane & 15, g = lane >> 4;
    // one-dimensional launch of (H / RWG) x gy x gz workgroups: an item's row blocks share an
    // XCD (items dealt round robin), so its activation tile is fetched into one L2
    int bx, u, bz;
    xcd_rr_block(F.H / RWG, F.gy, F.gz, bx, u, bz);
    const int h0 = bx * RWG + wv * RW;
    int slot, p0, cnt;
    const int gs = group_state(F, u, slot, p0, cnt);
    if (gs == 0) return;
    if (gs == 1) {
        for (int i = lane; i < cnt * RW; i += 64)
            F.y[(int64_t)(p0 + i / RW) * F.H + h0 + (i % RW)] = __builtin_nanf("");
        return;
    }
    const uint8_t* base = F.pool + (int64_t)slot * F.slot_bytes;
    const int nk = F.I / 128;
    PfDma R;
    R.rowb = (int64_t)F.I / 2;
    R.cb[0] = uniform_ptr(base + 2 * F.nmb + (int64_t)h0 * R.rowb);
    R.cb[1] = uniform_ptr(base + 2 * F.nmb + (int64_t)(h0 + 16) * R.rowb);
    R.voc = (uint32_t)((lane >> 3) * R.rowb + 16 * ((lane & 7) ^ (lane >> 3)));
    const uint8_t* sc = base + 3 * F.nmb;
    R.sb = uniform_ptr(sc + (2 * (int64_t)F.NGM + (int64_t)h0 * nk) * 2);
    R.vos = (uint32_t)((lane >= 32 ? 3 * (int64_t)F.NGM * 2 : 0) + (lane & 31) * nk * 2);
    uint8_t* ringw = reinterpret_cast<uint8_t*>(ring) + wv * kDmaSlot;
    uint8_t* ab = reinterpret_cast<uint8_t*>(abuf);
    pf_dmag_passes<MT, NW, false>(F, R, p0, cnt, ab, ringw, nk, bz, F.gz, [&](auto& acc, int mb) {
        constexpr int NT = sizeof(acc) / sizeof(acc[0]);
#pragma unroll
        for (int mt = 0; mt < NT; ++mt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = mb + mt * 16 + 4 * g + i;
                if (m < cnt) {
                    const float wp = F.w[p0 + m];
                    float* dst = F.y + (int64_t)(p0 + m) * F.H + h0 + n;
                    dst[0] = wp * acc[mt][0][i];
                    dst[16] = wp * acc[mt][1][i];
                }
            }
    });
}

// s = sum_j y[back[t*k + j]][h], j in ascending expert id (back = -1: no pair in
// this call); out[t][h] = bf16(s), or acc[t][h] += s when acc is given.
// A thread takes 4 consecutive h of one token; its up to KMAX y rows are all
// requested before the ordered sum (k <= KMAX; H % 4 == 0).
template <int KMAX>
__global__ __launch_bounds__(256) void k_pf_combine(const float* __restrict__ y, const int32_t* __restrict__ back,
                                                    int T, int k, int H, int P, uint16_t* __restrict__ out,
                                                    float* __restrict__ acc) {
    const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i >= (int64_t)T * H) return;
    const int t = (int)(i / H), h = (int)(i - (int64_t)t * H);
    // Every request unconditional and issued before any use: the token's k pair indices, then
    // its k rows of y at clamped indices (a load under a per-lane condition was merged at the
    // branch's end, so each pair's round trip waited for the previous one's). Pairs past k
    // repeat the last (cached) and are skipped below; P >= 1 whenever this kernel runs.
    int pj[KMAX];
#pragma unroll
    for (int j = 0; j < KMAX; ++j) pj[j] = back[t * k + min(j, k - 1)];
    __builtin_amdgcn_sched_barrier(0);
    float4 v[KMAX];
#pragma unroll
    for (int j = 0; j < KMAX; ++j) {
        const int q = min(max(pj[j], 0), P - 1);
        v[j] = *reinterpret_cast<const float4*>(y + (int64_t)q * H + h);
    }
    __builtin_amdgcn_sched_barrier(0);
    float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int j = 0; j < KMAX; ++j) {
        if (j >= k || pj[j] == -1) continue;
        if (pj[j] < 0 || pj[j] >= P) {
            const float nan = __builtin_nanf("");
            v[j] = make_float4(nan, nan, nan, nan);
        }
        s.x += v[j].x; s.y += v[j].y; s.z += v[j].z; s.w += v[j].w;
    }
    if (acc) {
        float4* a = reinterpret_cast<float4*>(acc + i);
        float4 o = *a;
        o.x += s.x; o.y += s.y; o.z += s.z; o.w += s.w;
        *a = o;
    } else {
        *reinterpret_cast<uint2*>(out + i) = make_uint2(pack_bf16x2(s.x, s.y), pack_bf16x2(s.z, s.w));
    }
}

// MT (16-token tiles per wave and pass) from the largest group; Z workgroups
// share a larger group's passes
template <int BITS, int MT>
static void launch_pf_mt(const Prefill& F, int ngroups, int max_group, hipStream_t st) {
    if constexpr (BITS == 4) {
        const unsigned z = (unsigned)std::min(64, std::max(1, (max_group + MT * 16 - 1) / (MT * 16)));
        // the LDS-DMA form: an even number of K groups in both GEMMs, at most kPfSmSteps, and
        // x and act addressable with 32-bit offsets
        const int nkg = F.H / 128, nkd = F.I / 128;
        const bool off32 = (int64_t)F.T * F.H * 2 < (int64_t(1) << 31) && (int64_t)F.P * F.I * 2 < (int64_t(1) << 31);
        if (nkg % 2 == 0 && nkd % 2 == 0 && nkg <= kPfSmSteps && nkd <= kPfSmSteps && off32) {
            // 4-wave workgroups of 128 rows, token tiles staged per quant group: two or three
            // workgroups share a CU (measured on C5 against 8-wave workgroups with the tile
            // staged per group pair, one per CU: T = 256 119.7 -> 114.3 us, 512 150.5 -> 142.3)
            if (F.I % 64 == 0 && F.H % 128 == 0) {
                Prefill G = F;
                G.gy = ngroups;
                G.gz = (int)z;
                hipLaunchKernelGGL((k_pf_gate_up_dmag<MT, 4>), dim3((unsigned)(F.I / 64) * (unsigned)ngroups * z),
                                   dim3(256), 0, st, G);
                hipLaunchKernelGGL((k_pf_down_dmag<MT, 4>), dim3((unsigned)(F.H / 128) * (unsigned)ngroups * z),
                                   dim3(256), 0, st, G);
                return;
            }
        }
    }
    if constexpr (MT > 4) {
        launch_pf_mt<BITS, 4>(F, ngroups, max_group, st);  // passes of more than 4 tiles: LDS-DMA form only
        return;
    }
    constexpr int MTR = MT > 4 ? 4 : MT;  // the register form's tile count (MT <= 4 here)
    constexpr int NW = MTR >= 4 ? 8 : 4, RWG = 256;
    const unsigned z = (unsigned)std::min(64, std::max(1, (max_group + MTR * 16 - 1) / (MTR * 16)));
    const dim3 ggu((unsigned)(F.I / (RWG / 2)), (unsigned)ngroups, z), gdn((unsigned)(F.H / RWG), (unsigned)ngroups, z);
    if (F.H / 128 <= kPfSmSteps)
        hipLaunchKernelGGL((k_pf_gate_up<BITS, MTR, NW, RWG, true>), ggu, dim3(64 * NW), 0, st, F);
    else
        hipLaunchKernelGGL((k_pf_gate_up<BITS, MTR, NW, RWG, false>), ggu, dim3(64 * NW), 0, st, F);
    if (F.I / 128 <= kPfSmSteps)
        hipLaunchKernelGGL((k_pf_down<BITS, MTR, NW, RWG, true>), gdn, dim3(64 * NW), 0, st, F);
    else
        hipLaunchKernelGGL((k_pf_down<BITS, MTR, NW, RWG, false>), gdn, dim3(64 * NW), 0, st, F);
}
template <int BITS>
static void launch_pf(const Prefill& F, int ngroups, int max_group, hipStream_t st) {
    if (max_group <= 16)
        launch_pf_mt<BITS, 1>(F, ngroups, max_group, st);
    else if (max_group <= 32)
        launch_pf_mt<BITS, 2>(F, ngroups, max_group, st);
    else if (max_group <= 64)
        launch_pf_mt<BITS, 4>(F, ngroups, max_group, st);
    else
        launch_pf_mt<BITS, 8>(F, ngroups, max_group, st);
}

}  // namespace wisp

using namespace wisp;

extern "C" int64_t wisp_prefill_ws_bytes(int64_t pairs, int64_t H, int64_t I) {
    if (pairs < 1 || H < 1 || I < 1) return -1;
    return (pairs * I * 2 + 255) / 256 * 256 + pairs * H * 4;
}

// moe.py:131-151 (grouped: one launch per GEMM for all routed experts)
extern "C" int wisp_moe_prefill(const uint8_t* pool, int64_t slot_bytes, int64_t nslots, const int32_t* groups,
                                int ngroups, int max_group, const int32_t* tok, const float* w, const int32_t* back, int64_t pairs,
                                const uint16_t* x, int T, int k, int64_t H, int64_t I, int bits, int64_t group,
                                void* ws, uint16_t* out, float* acc, void* stream) {
    clear_error();
    if (!pool || !groups || !tok || !w || !back || !x || !ws || (!out && !acc)) return fail_inval("null pointer");
    if (!(bits == 4 || bits == 3 || bits == 2)) return fail_inval("bits must be 4, 3 or 2");
    if (group != 128) return fail_inval("the grouped prefill needs group 128 (one quant group per K step)");
    if (H % 256 || I % 128 || H > (1 << 16) || I > (1 << 16))
        return fail_inval("H a multiple of 256 and I of 128, both <= 65536");
    if (T < 1 || k < 1 || k > 32 || ngroups < 1 || pairs < 1 || pairs > (int64_t)T * k)
        return fail_inval("need 1 <= k <= 32, 1 <= pairs <= T*k and at least one group");
    if (nslots < 1 || nslots > (1 << 24)) return fail_inval("nslots out of range");
    const int64_t n = H * I;
    if (slot_bytes < wisp_expert_nbytes(n, bits, group)) return fail_inval("slot_bytes < expert size");
    if (!aligned(pool, 16) || slot_bytes % 16 || !aligned(x, 16) || !aligned(ws, 256) || (out && !aligned(out, 8)) ||
        (acc && !aligned(acc, 16))) {
        set_error("pool, x, ws, out and acc must be 16/16/256/8/16-byte aligned, slot_bytes a multiple of 16");
        return WISP_EALIGN;
    }
    Prefill F;
    F.pool = pool;
    F.slot_bytes = slot_bytes;
    F.nmb = n * bits / 8;
    F.nslots = (int)nslots;
    F.H = (int)H;
    F.I = (int)I;
    F.NGM = (int)(n / group);
    F.P = (int)pairs;
    F.T = T;
    F.groups = groups;
    F.tok = tok;
    F.w = w;
    F.x = x;
    F.act = static_cast<uint16_t*>(ws);
    F.y = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + (pairs * I * 2 + 255) / 256 * 256);
    F.gy = F.gz = 1;  // set per launch for the LDS-DMA kernels
    hipStream_t st = (hipStream_t)stream;
    max_group = std::max(1, std::min(max_group, T));  // a launch-shape hint; any value is correct
    switch (bits) {
    case 4: launch_pf<4>(F, ngroups, max_group, st); break;
    case 3: launch_pf<3>(F, ngroups, max_group, st); break;
    default: launch_pf<2>(F, ngroups, max_group, st); break;
    }
    const unsigned nblk = (unsigned)(((int64_t)T * H / 4 + 255) / 256);
    if (k <= 8)
        hipLaunchKernelGGL(k_pf_combine<8>, dim3(nblk), dim3(256), 0, st, (const float*)F.y, back, T, k, (int)H,
                           (int)pairs, out, acc);
    else
        hipLaunchKernelGGL(k_pf_combine<32>, dim3(nblk), dim3(256), 0, st, (const float*)F.y, back, T, k, (int)H,
                           (int)pairs, out, acc);
    return check_launch("k_pf");
}
