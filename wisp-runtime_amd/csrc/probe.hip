// Measurement probes: the floors the decode kernels are measured against
// (bench.py --workload floor). No reference counterpart; nothing on the
// product path calls them.
//
//  * k_probe_empty: a kernel that does nothing (the per-launch cost inside a
//    graph).
//  * k_probe_read: a plain streaming read of `bytes` bytes with 16-byte
//    non-temporal loads, one pass, the values folded into a register and
//    stored only if they equal an impossible pattern (so the loads are kept
//    and nothing is written). With `slot` non-null the base address is
//    base + s * stride, s = slot[0] (a float slot id, 0 unless an integer in
//    [0, nslots)) read from device memory first: the dependent round trip
//    (slot id -> data) the decode kernels pay before their weight loads.
//  * k_probe_stamp: one lane reads the GPU's constant-rate real-time counter
//    (s_memrealtime) and writes it to dst with a vector store. Two stamps
//    captured in a graph around a run of steps time those steps on the GPU's
//    own clock, without the graph's launch latency.
//  * The C2 layer's skeleton, every data movement of the two decode kernels
//    without their arithmetic: k_probe_skel_a (768 workgroups, as kernel 1)
//    reads the gate_up bytes after the slot-id read and writes the 6144-value
//    activation (8 values per workgroup); k_probe_skel_b (512 workgroups, as
//    kernel 2) issues its share of the down bytes first, stages the whole
//    activation in LDS, folds a token value per wave and writes the 2048
//    outputs. k_probe_skel_one is the same work as ONE launch: the 512
//    consuming workgroups wait at a grid barrier (per-group counters, then a
//    top counter and a generation word, all agent-scope atomics; the
//    activation written and read as agent-scope atomics, so it is coherent
//    across the XCDs' L2s without an L2 write-back or invalidate), with their
//    down bytes already loaded into registers. Every wait is bounded: a
//    workgroup that spins 2^22 times sets an error bit and goes on, so every
//    wave exits; the host launches it only when all 768 workgroups can be
//    resident at once.
#include "wisp_device.hpp"
#include "wisp_internal.hpp"

namespace wisp {

__global__ void k_probe_empty() {}

__global__ __launch_bounds__(64) void k_probe_stamp(uint64_t* __restrict__ dst) {
    const uint64_t t = __builtin_amdgcn_s_memrealtime();
    if (threadIdx.x == 0) {
        volatile uint64_t* d = dst;  // an ordinary (vector) global store
        *d = t;
    }
}

constexpr int kProbeThreads = 256;
constexpr int kProbeUnroll = 4;  // 16-byte loads in flight per thread and step

__global__ __launch_bounds__(kProbeThreads) void k_probe_read(const uint8_t* __restrict__ base,
                                                              const float* __restrict__ slot, int64_t stride,
                                                              int nslots, int64_t n16, uint32_t* __restrict__ sink) {
    const uint8_t* p = base;
    if (slot) {
        const float f = slot[0];
        const int s = (int)f;
        const bool ok = f >= 0.f && f < (float)nslots && (float)s == f;
        p += (int64_t)__builtin_amdgcn_readfirstlane(ok ? s : 0) * stride;
    }
    const u32x4_t* q = reinterpret_cast<const u32x4_t*>(p);
    const int64_t step = (int64_t)gridDim.x * kProbeThreads * kProbeUnroll;
    uint32_t acc = 0;
    for (int64_t i0 = (int64_t)blockIdx.x * kProbeThreads * kProbeUnroll + threadIdx.x; i0 < n16; i0 += step) {
        u32x4_t v[kProbeUnroll];
#pragma unroll
        for (int u = 0; u < kProbeUnroll; ++u) {
            const int64_t i = i0 + (int64_t)u * kProbeThreads;
            v[u] = i < n16 ? __builtin_nontemporal_load(q + i) : u32x4_t{0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < kProbeUnroll; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    if (acc == 0x9E3779B9u && threadIdx.x == 0x3FF) sink[blockIdx.x] = acc;  // never true: threadIdx.x < 256
}

// ---- the C2 layer's skeleton --------------------------------------------------------------
constexpr int kSkelP = 768, kSkelC = 512, kSkelAct = 8 * 768;  // 4 outputs per consumer: 2,048
constexpr int kSkelPerA = 8, kSkelPerB = 4;  // 16-byte loads per thread at most (bytes checked on the host)
constexpr unsigned kSkelSpin = 1u << 22;

// sync words, each on its own 256-byte line: 8 group counters, the top counter, the generation, errors
struct SkelSync {
    unsigned grp[8 * 64];
    unsigned top[64];
    unsigned gen[64];
    unsigned err[64];
};

__device__ __forceinline__ unsigned ld_agent(const unsigned* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(unsigned* p, unsigned v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned add_agent(unsigned* p, unsigned v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ const uint8_t* skel_base(const uint8_t* base, const float* slot, int64_t stride,
                                                    int nslots) {
    if (!slot) return base;
    const float f = slot[0];
    const int s = (int)f;
    const bool ok = f >= 0.f && f < (float)nslots && (float)s == f;
    return base + (int64_t)__builtin_amdgcn_readfirstlane(ok ? s : 0) * stride;
}

// this workgroup's share of n16 16-byte words, strided by the grid (nwg workgroups), folded to one word
__device__ __forceinline__ uint32_t skel_read_a(const uint8_t* p, int64_t n16, int b) {
    const u32x4_t* q = reinterpret_cast<const u32x4_t*>(p);
    u32x4_t v[kSkelPerA];
#pragma unroll
    for (int u = 0; u < kSkelPerA; ++u) {
        const int64_t i = (int64_t)u * kSkelP * kProbeThreads + (int64_t)b * kProbeThreads + threadIdx.x;
        v[u] = i < n16 ? __builtin_nontemporal_load(q + i) : u32x4_t{0, 0, 0, 0};
    }
    uint32_t acc = 0;
#pragma unroll
    for (int u = 0; u < kSkelPerA; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    return acc;
}
__device__ __forceinline__ void skel_load_b(const uint8_t* p, int64_t n16, int b, u32x4_t (&d)[kSkelPerB]) {
    const u32x4_t* q = reinterpret_cast<const u32x4_t*>(p);
#pragma unroll
    for (int u = 0; u < kSkelPerB; ++u) {
        const int64_t i = (int64_t)u * kSkelC * kProbeThreads + (int64_t)b * kProbeThreads + threadIdx.x;
        d[u] = i < n16 ? __builtin_nontemporal_load(q + i) : u32x4_t{0, 0, 0, 0};
    }
}
// one value per wave from the staged activation and the down words, written as bf16 bits
__device__ __forceinline__ void skel_out(const float* a_l, const u32x4_t (&d)[kSkelPerB], uint32_t extra,
                                         uint16_t* __restrict__ out, int b) {
    float y = (float)(extra & 1u);
#pragma unroll
    for (int u = 0; u < kSkelPerB; ++u) y += a_l[(threadIdx.x * 7 + u * 131) % kSkelAct] * (float)(d[u].x & 15u);
    for (int o = 32; o; o >>= 1) y += __shfl_xor(y, o, 64);
    if ((threadIdx.x & 63) == 0) out[b * 4 + (threadIdx.x >> 6)] = (uint16_t)(__float_as_uint(y) >> 16);
}

__global__ __launch_bounds__(kProbeThreads) void k_probe_skel_a(const uint8_t* base, const float* slot,
                                                                int64_t stride, int nslots, int64_t na16,
                                                                float* __restrict__ act) {
    const uint8_t* p = skel_base(base, slot, stride, nslots);
    const uint32_t acc = skel_read_a(p, na16, blockIdx.x);
    if (threadIdx.x < 8) act[blockIdx.x * 8 + threadIdx.x] = (float)(acc & 255u) * 1e-3f;
}

__global__ __launch_bounds__(kProbeThreads) void k_probe_skel_b(const uint8_t* base, const float* slot,
                                                                int64_t stride, int nslots, int64_t na16,
                                                                int64_t nb16, const float* __restrict__ act,
                                                                uint16_t* __restrict__ out) {
    __shared__ float a_l[kSkelAct];
    const uint8_t* p = skel_base(base, slot, stride, nslots) + na16 * 16;
    u32x4_t d[kSkelPerB];
    skel_load_b(p, nb16, blockIdx.x, d);
#pragma unroll
    for (int u = 0; u < kSkelAct / kProbeThreads; ++u) a_l[threadIdx.x + kProbeThreads * u] = act[threadIdx.x + kProbeThreads * u];
    __syncthreads();
    skel_out(a_l, d, 0u, out, blockIdx.x);
}

__global__ __launch_bounds__(kProbeThreads) void k_probe_skel_one(const uint8_t* base, const float* slot,
                                                                  int64_t stride, int nslots, int64_t na16,
                                                                  int64_t nb16, float* __restrict__ act,
                                                                  SkelSync* __restrict__ sy,
                                                                  uint16_t* __restrict__ out) {
    __shared__ float a_l[kSkelAct];
    __shared__ unsigned g0s;
    const int b = blockIdx.x;
    const bool cons = b < kSkelC;
    if (cons && threadIdx.x == 0) g0s = ld_agent(&sy->gen[0]);  // before arriving: the barrier cannot pass yet
    const uint8_t* p = skel_base(base, slot, stride, nslots);
    u32x4_t d[kSkelPerB];
    if (cons) skel_load_b(p + na16 * 16, nb16, b, d);
    const uint32_t acc = skel_read_a(p, na16, b);
    if (threadIdx.x < 8) st_agent(reinterpret_cast<unsigned*>(act) + b * 8 + threadIdx.x,
                                  __float_as_uint((float)(acc & 255u) * 1e-3f));
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");  // this wave's activation stores are complete
    __syncthreads();
    if (threadIdx.x == 0) {
        bool last = add_agent(&sy->grp[64 * (b & 7)], 1u) == kSkelP / 8 - 1;
        if (last) {
            st_agent(&sy->grp[64 * (b & 7)], 0u);
            last = add_agent(&sy->top[0], 1u) == 7;
            if (last) {
                st_agent(&sy->top[0], 0u);
                st_agent(&sy->gen[0], ld_agent(&sy->gen[0]) + 1u);
            }
        }
        if (cons && !last) {
            unsigned n = 0;
            while (ld_agent(&sy->gen[0]) == g0s) {
                if (++n > kSkelSpin) {
                    __hip_atomic_fetch_or(&sy->err[0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
        }
    }
    if (!cons) return;
    __syncthreads();
    const unsigned* au = reinterpret_cast<const unsigned*>(act);
#pragma unroll
    for (int u = 0; u < kSkelAct / kProbeThreads; ++u)
        a_l[threadIdx.x + kProbeThreads * u] = __uint_as_float(ld_agent(au + threadIdx.x + kProbeThreads * u));
    __syncthreads();
    skel_out(a_l, d, acc, out, b);
}

}  // namespace wisp

using namespace wisp;

extern "C" int wisp_probe_empty(void* stream) {
    clear_error();
    hipLaunchKernelGGL(k_probe_empty, dim3(1), dim3(64), 0, (hipStream_t)stream);
    return check_launch("k_probe_empty");
}

extern "C" int wisp_probe_stamp(uint64_t* dst, void* stream) {
    clear_error();
    if (!dst || !aligned(dst, 8)) return fail_inval("probe_stamp: dst must be an 8-byte aligned device pointer");
    hipLaunchKernelGGL(k_probe_stamp, dim3(1), dim3(64), 0, (hipStream_t)stream, dst);
    return check_launch("k_probe_stamp");
}

extern "C" int wisp_probe_read(const uint8_t* base, const float* slot, int64_t stride, int64_t nslots, int64_t bytes,
                               int workgroups, uint32_t* sink, void* stream) {
    clear_error();
    if (!base || !sink || bytes <= 0 || bytes % 16 || workgroups < 1 || workgroups > 65535)
        return fail_inval("probe_read: base, sink, bytes > 0 (a multiple of 16) and 1..65535 workgroups");
    if (slot && (nslots < 1 || nslots > (1 << 24))) return fail_inval("probe_read: nslots must be in [1, 2^24]");
    if (!aligned(base, 16) || stride % 16) {
        set_error("probe_read: base and stride must be 16-byte aligned");
        return WISP_EALIGN;
    }
    hipLaunchKernelGGL(k_probe_read, dim3(workgroups), dim3(kProbeThreads), 0, (hipStream_t)stream, base, slot, stride,
                       (int)nslots, bytes / 16, sink);
    return check_launch("k_probe_read");
}

extern "C" int wisp_probe_skeleton(const uint8_t* base, const float* slot, int64_t stride, int64_t nslots,
                                   int64_t gu_bytes, int64_t dn_bytes, float* act, uint16_t* out, void* sync,
                                   int one_launch, void* stream) {
    clear_error();
    const int64_t maxa = (int64_t)kSkelP * kProbeThreads * kSkelPerA * 16, maxb = (int64_t)kSkelC * kProbeThreads * kSkelPerB * 16;
    if (!base || !act || !out || gu_bytes <= 0 || dn_bytes <= 0 || gu_bytes % 16 || dn_bytes % 16 || gu_bytes > maxa ||
        dn_bytes > maxb)
        return fail_inval("probe_skeleton: base, act, out; byte counts > 0, multiples of 16, at most 25 MB / 8.4 MB");
    if (slot && (nslots < 1 || nslots > (1 << 24))) return fail_inval("probe_skeleton: nslots must be in [1, 2^24]");
    if (!aligned(base, 16) || stride % 16 || !aligned(act, 4) || !aligned(out, 2)) {
        set_error("probe_skeleton: base and stride 16-byte aligned, act 4, out 2");
        return WISP_EALIGN;
    }
    hipStream_t st = (hipStream_t)stream;
    if (!one_launch) {
        hipLaunchKernelGGL(k_probe_skel_a, dim3(kSkelP), dim3(kProbeThreads), 0, st, base, slot, stride, (int)nslots,
                           gu_bytes / 16, act);
        int rc = check_launch("k_probe_skel_a");
        if (rc) return rc;
        hipLaunchKernelGGL(k_probe_skel_b, dim3(kSkelC), dim3(kProbeThreads), 0, st, base, slot, stride, (int)nslots,
                           gu_bytes / 16, dn_bytes / 16, act, out);
        return check_launch("k_probe_skel_b");
    }
    if (!sync || !aligned(sync, 256)) return fail_inval("probe_skeleton: one_launch needs a 256-byte aligned sync buffer");
    int dev = 0, ncu = 0, occ = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, k_probe_skel_one, kProbeThreads, 0) != hipSuccess)
        return fail_inval("probe_skeleton: could not read the device's occupancy");
    if ((int64_t)occ * ncu < kSkelP) return fail_inval("probe_skeleton: the 768 workgroups cannot all be resident");
    hipLaunchKernelGGL(k_probe_skel_one, dim3(kSkelP), dim3(kProbeThreads), 0, st, base, slot, stride, (int)nslots,
                       gu_bytes / 16, dn_bytes / 16, act, static_cast<SkelSync*>(sync), out);
    return check_launch("k_probe_skel_one");
}

extern "C" int64_t wisp_probe_skeleton_sync_bytes(void) { return (int64_t)sizeof(SkelSync); }
