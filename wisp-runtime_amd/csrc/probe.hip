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
