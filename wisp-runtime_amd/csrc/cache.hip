// Expert cache for batch-1 MoE decode: slot bookkeeping (CacheCore) and the
// hipMalloc slot pool filled from a pinned host store by hipMemcpyAsync on a
// side stream or by a page kernel that reads the pinned rows itself
// (ExpertCache); optionally the LRU step on the GPU (device paging), so a
// captured decode step needs no host decision between layers. The
// decode-on-load mode reuses the dequant kernel.
//
// Reference semantics:
//   CacheCore  wisp/cache_core.py:15-149 (LRU / WSA / static policies, ensure,
//              split, admit, preload, resized)
//   ExpertCache wisp/cache.py:9-162 (pool, _issue ordering, sync_compute,
//              ensure, decode_on_load, resize)
//   one layer's host step of the graph decoder, wisp/graphdec.py:216-231
//              (ensure the routed experts, write [slots | weights] into the
//              pinned meta buffer, copy it to the device on the compute stream)
//
// Arithmetic of the bookkeeping (ticks, decayed frequencies, renormalisation at
// 1e100, first-index argmin over the dynamic region, stable hottest-first sort
// in resized) is binary64, in the reference's order, so slot choices match it
// exactly. A persistent native core removes the per-layer Python bookkeeping
// between graph replays (48 host decisions per token).
#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <new>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "route.hpp"
#include "wisp_internal.hpp"

namespace wisp {

enum Policy { kLRU = 0, kWSA = 1, kStatic = 2 };

struct Core {
    int64_t nslots = 0, n_static = 0;
    int policy = kLRU;
    double decay = 0.9995, admit_after = 2.0;
    std::vector<int64_t> slot_key;
    std::vector<double> last, score;
    std::unordered_map<int64_t, int64_t> key2slot;
    std::vector<int64_t> free;  // a stack: back() is handed out next
    int64_t tick = 0;
    double inc = 1.0;
    std::unordered_map<int64_t, double> freq;
    std::vector<int64_t> freq_order;  // insertion order of freq's keys
    int64_t hits = 0, misses = 0, evictions = 0, calls = 0;
    // protected slots of the current request: pmark[s] == pgen (one array pass per victim search)
    std::vector<uint32_t> pmark;
    uint32_t pgen = 0;

    Core(int64_t n, int pol, double dec, int64_t nst, double adm)
        : nslots(n), n_static(nst), policy(pol), decay(dec), admit_after(adm), slot_key(n, -1), last(n, 0.0),
          score(n, 0.0), pmark(n, 0) {
        for (int64_t s = n - 1; s >= nst; --s) free.push_back(s);
    }

    // start a new protected set (empty)
    void prot_begin() {
        if (++pgen == 0) {  // wrapped: clear the marks once
            std::fill(pmark.begin(), pmark.end(), 0u);
            pgen = 1;
        }
    }
    void prot_add(int64_t s) {
        if (s >= 0 && s < nslots) pmark[s] = pgen;
    }

    double& freq_at(int64_t k) {  // defaultdict(float) access
        auto it = freq.find(k);
        if (it != freq.end()) return it->second;
        freq_order.push_back(k);
        return freq.emplace(k, 0.0).first->second;
    }

    void step() {
        tick += 1;
        inc /= decay;
        if (inc > 1e100) {
            for (auto& kv : freq) kv.second /= 1e100;
            for (double& v : score) v /= 1e100;
            inc /= 1e100;
        }
    }

    void note(const int64_t* keys, int64_t n) {
        for (int64_t i = 0; i < n; ++i) {
            double& f = freq_at(keys[i]);
            f += inc;
            auto it = key2slot.find(keys[i]);
            if (it != key2slot.end()) {
                last[it->second] = (double)tick;
                score[it->second] = f;
            }
        }
    }

    double norm_freq(int64_t k) const {
        auto it = freq.find(k);
        return (it == freq.end() ? 0.0 : it->second) / inc;
    }

    int64_t lookup(int64_t k) const {
        auto it = key2slot.find(k);
        return it == key2slot.end() ? -1 : it->second;
    }

    // cache_core.py:64-84; returns -1 when nothing is evictable
    // (the protected slots are those marked since the last prot_begin)
    int64_t acquire(int64_t key) {
        int64_t s;
        if (!free.empty()) {
            s = free.back();
            free.pop_back();
        } else {
            const std::vector<double>& src = policy == kLRU ? last : score;
            int64_t j = -1;
            double best = INFINITY;
            for (int64_t i = n_static; i < nslots; ++i) {
                const double v = pmark[i] == pgen ? INFINITY : src[i];
                if (j < 0 || v < best) {
                    best = v;
                    j = i;
                }
            }
            if (j < 0 || !std::isfinite(best)) return -1;
            s = j;
            key2slot.erase(slot_key[s]);
            evictions += 1;
        }
        slot_key[s] = key;
        key2slot[key] = s;
        last[s] = (double)tick;
        score[s] = freq_at(key);
        return s;
    }
};

static int no_slot() {
    set_error("no evictable slot: dynamic region smaller than the working request");
    return WISP_EINVAL;
}

// ---------------------------------------------------------------------------
// slot pool memory shared between the cache and DLPack views of it
struct PoolBlock {
    void* ptr = nullptr;
    int device = 0;
    std::atomic<int> refs{1};
};

static void pool_release(PoolBlock* b) {
    if (b && b->refs.fetch_sub(1) == 1) {
        int cur = 0;
        (void)hipGetDevice(&cur);
        (void)hipSetDevice(b->device);
        (void)hipFree(b->ptr);
        (void)hipSetDevice(cur);
        delete b;
    }
}

// DLPack (unversioned ABI) structures, as consumed by torch.utils.dlpack
struct DLDevice {
    int32_t device_type;
    int32_t device_id;
};
struct DLDataType {
    uint8_t code;
    uint8_t bits;
    uint16_t lanes;
};
struct DLTensor {
    void* data;
    DLDevice device;
    int32_t ndim;
    DLDataType dtype;
    int64_t* shape;
    int64_t* strides;
    uint64_t byte_offset;
};
struct DLManagedTensor {
    DLTensor dl_tensor;
    void* manager_ctx;
    void (*deleter)(DLManagedTensor*);
};
struct PoolView {
    DLManagedTensor m;
    int64_t shape[2];
    int64_t strides[2];
    PoolBlock* block;
};
static void view_deleter(DLManagedTensor* m) {
    PoolView* v = reinterpret_cast<PoolView*>(m);
    pool_release(v->block);
    delete v;
}

// Device paging: the core's state in device memory (one allocation) while it is on.
constexpr int kDevMaxK = 16;  // keys per step
// The step holds every dynamic slot's eviction key in registers for the whole step:
// kLruSmall keys per lane of one wave for pools of at most 64 kLruSmall dynamic slots, else
// kLruBig keys per thread of up to 15 waves beside the wave that routes (16 in all).
constexpr int kLruSmall = 16, kLruBig = 28;
constexpr int kDevMaxSlots = 15 * 64 * kLruBig;  // 26880 dynamic slots
enum { kCtrTick, kCtrNextFree, kCtrHits, kCtrMisses, kCtrEvict, kCtrCalls, kCtrLoads, kCtrErr, kCtrOn, kCtrInc, kCtrN };
enum { kDevErrSlot = 1, kDevErrKey = 2 };
constexpr int64_t kFirstBefore = -2, kFirstNever = -1;  // DevPaging::first, besides a device stamp
struct DevPaging {
    int32_t* slot_key = nullptr;  // [nslots], -1 empty
    int64_t* last = nullptr;      // [nslots], tick of the last use
    double* score = nullptr;      // [nslots], the decayed frequency of the slot's key at its last note
    int32_t* key2slot = nullptr;  // [nkeys], -1 not resident
    double* freq = nullptr;       // [nkeys], decayed access frequency (0 for keys never noted)
    int64_t* first = nullptr;     // [nkeys], kFirstBefore: in the core's table before device paging began;
                                  // kFirstNever; else 64 tick + position of the key's first note on the device
    int64_t* ctr = nullptr;       // [kCtrN]: tick, next free slot, hits, misses, evictions, calls, loads, error
                                  // bits, on (1 while the device holds the state), the bits of inc (binary64)
    int32_t* miss = nullptr;      // [1 + 2 kDevMaxK]: count, keys, slots of the last step's loads
    double decay = 1.0;
    int64_t nslots = 0, nkeys = 0, n_static = 0;
};

struct Cache {
    Core* core = nullptr;
    PoolBlock* pool = nullptr;
    int device = 0;
    int64_t nslots = 0, slot_bytes = 0;
    const uint8_t* host = nullptr;  // pinned store rows (caller-owned)
    int64_t host_rows = 0, row_bytes = 0;
    int bits = 4;
    int64_t n = 0, group = 128;
    bool decode_on_load = false;
    uint8_t* staging = nullptr;  // decode_on_load: staging rows of quantized bytes
    int64_t staging_rows = 0;
    hipStream_t copy = nullptr;
    hipEvent_t order = nullptr, done = nullptr;
    int copy_mode = 0;                   // 0: hipMemcpyAsync per row, 1: k_page_rows
    const uint8_t* host_dev = nullptr;   // the host store's device address (copy_mode 1)
    bool pending = false;
    int64_t bytes_h2d = 0, n_loads = 0;
    // the device paging state: allocated by the first wisp_cache_device_begin and kept (at the
    // same address, so captured steps stay valid) until the cache is destroyed or its slot
    // count changes
    void* dev_block = nullptr;
    DevPaging dev;
    bool dev_on = false;
    bool dev_score = false;      // the core's policy evicts by score (WSA, static), not by last use
    int64_t dev_loads_seen = 0;  // device loads already added to bytes_h2d / n_loads
};

static int hip_fail(hipError_t e, const char* what) {
    set_error("%s: %s", what, hipGetErrorString(e));
    return (int)e;
}

// A resize whose new pool could not be allocated leaves the cache without one;
// every entry point that would touch the pool reports it instead.
static int no_pool() { return fail_inval("pool not allocated: the last resize failed to allocate it"); }

static int alloc_pool(Cache& c) {
    PoolBlock* b = new (std::nothrow) PoolBlock();
    if (!b) return fail_inval("out of host memory");
    b->device = c.device;
    const hipError_t e = hipMalloc(&b->ptr, (size_t)(c.nslots * c.slot_bytes));
    if (e != hipSuccess) {
        delete b;
        (void)hipGetLastError();  // consume it here: a later launch check must not report it
        return hip_fail(e, "hipMalloc(slot pool)");
    }
    c.pool = b;
    return WISP_OK;
}

// Copy mode 1: the GPU reads the pinned host rows itself over PCIe. Grid
// (kPageSplit, pairs): each workgroup copies one contiguous part of one row
// with 16-byte loads, 4 in flight per thread. On MI355X this streams
// 53-56 GB/s for 4+ rows against 46-47 GB/s for one hipMemcpyAsync per row.
constexpr int kPageMax = 16;    // pairs per launch
constexpr int kPageSplit = 32;  // workgroups per row
struct PagePairs {
    int64_t key[kPageMax];
    int64_t slot[kPageMax];
};
// optional payload: workgroup (0, 0) also stores n floats to dst (the layer's meta)
struct PageMeta {
    float v[32];
    float* dst;
    int n;
};
typedef uint32_t pg_u32x4 __attribute__((ext_vector_type(4)));
// workgroup blockIdx.x's part [b0, b1) of one row (16-byte units), 4 loads in flight per thread
__device__ __forceinline__ void page_part(const pg_u32x4* __restrict__ src, pg_u32x4* __restrict__ dst, int64_t row16,
                                          int64_t per) {
    const int64_t b0 = (int64_t)blockIdx.x * per, b1 = min(row16, b0 + per);
    constexpr int U = 4;
    for (int64_t i = b0 + threadIdx.x; i < b1; i += 256 * U) {
        pg_u32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t ii = i + (int64_t)u * 256;
            if (ii < b1) v[u] = __builtin_nontemporal_load(src + ii);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t ii = i + (int64_t)u * 256;
            if (ii < b1) dst[ii] = v[u];
        }
    }
}

__global__ __launch_bounds__(256) void k_page_rows(const pg_u32x4* __restrict__ host, pg_u32x4* __restrict__ pool,
                                                   const PagePairs p, int64_t row16, int64_t slot16, int64_t per,
                                                   const PageMeta pm) {
    const int r = blockIdx.y;
    if (blockIdx.x == 0 && r == 0 && (int)threadIdx.x < pm.n) pm.dst[threadIdx.x] = pm.v[threadIdx.x];
    page_part(host + p.key[r] * row16, pool + p.slot[r] * slot16, row16, per);
}

// The rows of the miss list that k_lru_step left in device memory: grid
// (kPageSplit, k), row blockIdx.y if it is below the list's count.
__global__ __launch_bounds__(256) void k_page_list(const pg_u32x4* __restrict__ host, pg_u32x4* __restrict__ pool,
                                                   const int32_t* __restrict__ miss, int64_t row16, int64_t slot16,
                                                   int64_t per) {
    const int r = blockIdx.y;
    if (r >= miss[0]) return;
    page_part(host + (int64_t)miss[1 + r] * row16, pool + (int64_t)miss[1 + kDevMaxK + r] * slot16, row16, per);
}

// Wave-wide minimum of a 64-bit value (every lane active; the result is wave-uniform):
// DPP inside each 16-lane row (quad_perm xor 1, xor 2, row_half_mirror, row_mirror), then
// the four row minima through readlane.
template <int CTRL>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)v, CTRL, 0xF, 0xF, true);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(v >> 32), CTRL, 0xF, 0xF, true);
    return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t min_u64(uint64_t a, uint64_t b) { return a < b ? a : b; }
__device__ __forceinline__ uint64_t readlane_u64(uint64_t v, int l) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), l);
    return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t wave_min_u64(uint64_t v) {
    v = min_u64(v, dpp_u64<0xB1>(v));
    v = min_u64(v, dpp_u64<0x4E>(v));
    v = min_u64(v, dpp_u64<0x141>(v));
    v = min_u64(v, dpp_u64<0x140>(v));
    return min_u64(min_u64(readlane_u64(v, 0), readlane_u64(v, 16)), min_u64(readlane_u64(v, 32), readlane_u64(v, 48)));
}

// The step's counters and its clock (cache_core.py:30-38, step): tick + 1, inc / decay, and
// when that passes 1e100 every frequency, every score and inc itself divided by 1e100 (the
// renormalisation, applied by lru_commit). Uniform scalar reads, taken by every wave.
struct LruCtr {
    int64_t tick, nf;
    double inc;
    bool on, renorm;
};
__device__ __forceinline__ LruCtr lru_counters(const DevPaging& d) {
    LruCtr st;
    st.on = d.ctr[kCtrOn] != 0;
    st.tick = d.ctr[kCtrTick] + 1;
    st.nf = d.ctr[kCtrNextFree];
    double inc = __longlong_as_double((long long)d.ctr[kCtrInc]) / d.decay;
    st.renorm = inc > 1e100;
    if (st.renorm) inc = inc / 1e100;
    st.inc = inc;
    return st;
}

// Which threads hold eviction keys: every lane of the one wave (R = kLruSmall), else the
// threads past wave 0 (wave 0 routes and classifies, and its registers stay free for that).
// Key holder t of nt holds dynamic slot i = t + nt u (u < R).
template <int R>
__device__ __forceinline__ int lru_holder() {
    return R == kLruSmall ? (int)threadIdx.x : (int)threadIdx.x - 64;
}
template <int R>
__device__ __forceinline__ int lru_holders() {
    return R == kLruSmall ? (int)blockDim.x : (int)blockDim.x - 64;
}

// Eviction keys in registers, dynamic slot i (slot n_static + i) of holder t in key[u],
// i = t + nt u, ~0 past the pool. LRU (SC false): (last, slot) + 1 as one integer (never 0,
// so 0 is below every key). Score policies (SC true): the bits of the slot's score (a
// non-negative binary64, so its bits order as its value; divided by 1e100 first when this step
// renormalises), the slot implied by the position. One request per key, all before any use;
// 32-bit slot indexes (nd <= kDevMaxSlots), so each request needs one offset register. The
// one-wave form also holds each slot's key (owner) in `own`, so the victims' old keys need no
// dependent read.
template <int R, bool SC>
__device__ __forceinline__ void lru_stage(const DevPaging& d, int nd, bool renorm, uint64_t (&key)[R],
                                          int32_t (&own)[R]) {
    const int t = lru_holder<R>(), nt = lru_holders<R>();
    const int64_t* __restrict__ lp = d.last + d.n_static;
    const double* __restrict__ sp = d.score + d.n_static;
    const int32_t* __restrict__ op = d.slot_key + d.n_static;
    uint64_t v[R];
#pragma unroll
    for (int u = 0; u < R; ++u) {
        const int i = min(t + nt * u, nd - 1);
        v[u] = SC ? (uint64_t)__double_as_longlong(sp[i]) : (uint64_t)lp[i];
        if constexpr (R == kLruSmall) own[u] = op[i];
    }
#pragma unroll
    for (int u = 0; u < R; ++u) {
        const int i = t + nt * u;
        uint64_t kv;
        if constexpr (SC) {
            kv = renorm ? (uint64_t)__double_as_longlong(__longlong_as_double((long long)v[u]) / 1e100) : v[u];
        } else {
            kv = ((v[u] << 20) | (uint64_t)(d.n_static + i)) + 1ull;
        }
        key[u] = i < nd ? kv : ~0ull;
    }
}

// The one-wave form's owner of dynamic slot i (0 <= i < 64 kLruSmall), held by lane i % 64
// in own[i / 64]; every lane of the wave active (the lane reads go through ds_bpermute).
__device__ __forceinline__ int lru_owner_of(const int32_t (&own)[kLruSmall], int i) {
    const int src = i & 63, reg = i >> 6;
    int v = -1;
#pragma unroll
    for (int u = 0; u < kLruSmall; ++u) {
        const int o = __shfl(own[u], src, 64);
        v = reg == u ? o : v;
    }
    return v;
}

// What wave 0 tells the other waves of the step (through LDS, before the eviction rounds).
struct LruShared {
    uint64_t wmin[2][16];     // per-wave round minima, two buffers (rounds alternate)
    int32_t wslot[2][16];     // their slots (score policies)
    int32_t hits[kDevMaxK];   // this step's hit slots
    int32_t nhit, m;          // hits, misses that evict
    int64_t nc;               // dynamic slots in use at the step's start
};

// Wave 0's per-lane view of the step.
struct LruLane {
    int key, slot, rank, from_free, nmiss;
    int lead, mult;  // the first lane holding this lane's key; on that lane, how many lanes hold it
    float w;
    bool miss, hit, on;
    uint64_t hm, bad;
    double fq;       // freq[key] at the step's start (lead lanes)
    int64_t fst;     // first[key] (lead lanes)
};

// cache_core.py:86-106 (ensure) on the GPU, for one layer, in three parts: lru_classify
// (wave 0: lane j < k holds key j, -1 if its id was not valid, and its weight w), lru_evict
// (every wave of the workgroup) and lru_commit (wave 0). The step's clock and notes
// (cache_core.py:30-51: inc, every key's decayed frequency with one addition of inc per
// occurrence in key order, a resident key's tick and score) are kept for every policy, as
// the reference keeps them. Misses take free slots in ascending order, then the unprotected
// slot with the smallest eviction key: `last` (LRU) or `score` (WSA, static). The reference
// picks each victim by a first-index argmin over the unprotected dynamic slots, and every slot
// it hands out becomes protected, so the i-th evicting miss (in key order) gets the i-th
// smallest (key, slot) among the slots in [n_static, next free) that are not hits of this
// step (a score policy's notes change only hits' scores before the victims are chosen).
// meta = [slots (float) | the row's weights]; the loads go to the miss list for k_page_list.
// A key that is not valid or a miss without an evictable slot gets slot -1 in meta (the MoE
// kernels then write NaN rows) and sets an error bit that the host reads when it syncs the
// state. A launch while device paging is off (a captured step replayed after
// wisp_cache_device_end) does no step and writes slot -1 into meta.
// `resident` is key2slot[key] (-1 for key < 0), looked up by the caller.
// have_pre: pfq / pfst are freq[key] / first[key], requested by the caller at the step's start.
__device__ __forceinline__ LruLane lru_classify(const DevPaging& d, const LruCtr& st, int lane, int k, int key,
                                                int resident, float w, LruShared& sh, bool have_pre = false,
                                                double pfq = 0.0, int64_t pfst = 0) {
    LruLane ln{};
    ln.key = key;
    ln.w = w;
    ln.on = st.on;
    if (!st.on) {  // replayed while the host core holds the state: no step
        if (lane == 0) {
            sh.m = 0;
            sh.nhit = 0;
            sh.nc = 0;
        }
        return ln;
    }
    // the notes: the first lane of each key adds inc once per lane holding it (in lru_commit);
    // its frequency and first-note stamp are requested here and used after the rounds
    ln.lead = lane;
    ln.mult = 0;
    for (int j = 0; j < k; ++j) {
        const int kj = __builtin_amdgcn_readlane(key, j);  // j is uniform: no LDS round trip
        if (kj == key && j < ln.lead) ln.lead = j;
        ln.mult += kj == key ? 1 : 0;
    }
    if (key >= 0 && ln.lead == lane) {
        ln.fq = have_pre ? pfq : d.freq[key];
        ln.fst = have_pre ? pfst : d.first[key];
    }
    const int64_t nf = st.nf;
    int slot = key >= 0 ? resident : -1;
    ln.hit = slot >= 0;
    const uint64_t mm = __ballot(key >= 0 && !ln.hit);
    ln.hm = __ballot(ln.hit);
    ln.bad = __ballot(lane < k && key < 0);
    ln.miss = (mm >> lane) & 1ull;
    ln.nmiss = __popcll(mm);
    ln.rank = __popcll(mm & ((1ull << lane) - 1ull));
    const int64_t nfree = d.nslots - nf;
    ln.from_free = (int)((int64_t)ln.nmiss < nfree ? (int64_t)ln.nmiss : nfree);
    if (ln.miss && ln.rank < ln.from_free) slot = (int)(nf + ln.rank);
    ln.slot = slot;
    if (ln.hit) sh.hits[__popcll(ln.hm & ((1ull << lane) - 1ull))] = slot;
    if (lane == 0) {
        sh.m = ln.nmiss - ln.from_free;  // misses that evict
        sh.nhit = __popcll(ln.hm);
        sh.nc = nf - d.n_static;
    }
    return ln;
}

// The eviction rounds, run by every wave of the workgroup after the barrier that publishes
// `sh`: round r takes the smallest key above the last round's among the keys of the slots in
// use (each thread's R registers, then the wave's minimum by DPP, then the waves' minima
// through LDS), so every wave sees the same winner and runs the same number of rounds and
// barriers. A winner that is a hit of this step is protected: it is passed over (at most
// one round per hit). Returns the victims found; wave 0's evicting miss of rank
// from_free + i gets victim i in ln.slot.
// (value, slot) order of the score policies: value first, then the lower slot.
__device__ __forceinline__ bool pair_lt(uint64_t a, int sa, uint64_t b, int sb) {
    return a < b || (a == b && sa < sb);
}
template <int CTRL>
__device__ __forceinline__ void pair_min_dpp(uint64_t& v, int& s) {
    const uint64_t ov = dpp_u64<CTRL>(v);
    const int os = __builtin_amdgcn_update_dpp(0, s, CTRL, 0xF, 0xF, true);
    if (pair_lt(ov, os, v, s)) {
        v = ov;
        s = os;
    }
}
// wave-wide (value, slot) minimum, as wave_min_u64 (every lane active; wave-uniform result)
__device__ __forceinline__ void wave_min_pair(uint64_t& v, int& s) {
    pair_min_dpp<0xB1>(v, s);
    pair_min_dpp<0x4E>(v, s);
    pair_min_dpp<0x141>(v, s);
    pair_min_dpp<0x140>(v, s);
    uint64_t bv = readlane_u64(v, 0);
    int bs = __builtin_amdgcn_readlane(s, 0);
#pragma unroll
    for (int r = 16; r < 64; r += 16) {
        const uint64_t rv = readlane_u64(v, r);
        const int rs = __builtin_amdgcn_readlane(s, r);
        if (pair_lt(rv, rs, bv, bs)) {
            bv = rv;
            bs = rs;
        }
    }
    v = bv;
    s = bs;
}

template <int R, bool SC>
__device__ __forceinline__ int lru_evict(LruShared& sh, uint64_t (&key)[R], LruLane& ln, bool wave0, int n_static) {
    const int m = sh.m;
    if (m <= 0) return 0;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int nc = (int)sh.nc, t = lru_holder<R>(), nt = lru_holders<R>();
#pragma unroll
    for (int u = 0; u < R; ++u)
        if (t + nt * u >= nc) key[u] = ~0ull;  // free slots are not candidates (wave 0 of R = kLruBig holds none)
    const int nhit = sh.nhit;
    const int hs = lane < nhit ? sh.hits[lane] : -1;
    int found = 0, buf = 0;
    if constexpr (!SC) {
        uint64_t prev = 0;
        while (found < m) {
            uint64_t best = ~0ull;
#pragma unroll
            for (int u = 0; u < R; ++u) best = (key[u] > prev && key[u] < best) ? key[u] : best;
            best = wave_min_u64(best);
            if (nw > 1) {
                if (lane == 0) sh.wmin[buf][wv] = best;
                __syncthreads();
                best = ~0ull;
                for (int w = 0; w < nw; ++w) best = min_u64(best, sh.wmin[buf][w]);
                buf ^= 1;
            }
            if (best == ~0ull) break;  // nothing evictable is left
            prev = best;
            const int s = (int)((best - 1ull) & 0xFFFFFull);
            if (__ballot(hs == s)) continue;  // a hit of this step
            if (wave0 && ln.miss && ln.rank == ln.from_free + found) ln.slot = s;
            ++found;
        }
    } else {
        uint64_t pv = 0;  // the last round's (score bits, slot); slot -1 is below every slot
        int ps = -1;
        while (found < m) {
            uint64_t bv = ~0ull;
            int bs = 0x7FFFFFFF;
#pragma unroll
            for (int u = 0; u < R; ++u) {
                const int s = n_static + t + nt * u;
                if (key[u] != ~0ull && pair_lt(pv, ps, key[u], s) && pair_lt(key[u], s, bv, bs)) {
                    bv = key[u];
                    bs = s;
                }
            }
            wave_min_pair(bv, bs);
            if (nw > 1) {
                if (lane == 0) {
                    sh.wmin[buf][wv] = bv;
                    sh.wslot[buf][wv] = bs;
                }
                __syncthreads();
                bv = ~0ull;
                bs = 0x7FFFFFFF;
                for (int w = 0; w < nw; ++w)
                    if (pair_lt(sh.wmin[buf][w], sh.wslot[buf][w], bv, bs)) {
                        bv = sh.wmin[buf][w];
                        bs = sh.wslot[buf][w];
                    }
                buf ^= 1;
            }
            if (bv == ~0ull) break;  // nothing evictable is left
            pv = bv;
            ps = bs;
            if (__ballot(hs == bs)) continue;  // a hit of this step
            if (wave0 && ln.miss && ln.rank == ln.from_free + found) ln.slot = bs;
            ++found;
        }
    }
    return found;
}

// Wave 0: the step's writes (the clock and notes, slot table, ticks and scores, the miss
// list, meta and counters).
template <int R>
__device__ __forceinline__ void lru_commit(const DevPaging& d, const LruCtr& st, int lane, int k, const LruLane& ln,
                                           int evicted, const int32_t (&own)[R], float* __restrict__ meta) {
    if (!ln.on) {
        if (lane < k) meta[lane] = -1.f;
        if (lane == 0) d.miss[0] = 0;
        return;
    }
    const int64_t tick = st.tick, nf = st.nf;
    const int key = ln.key, slot = ln.slot;
    const int got = ln.from_free + evicted;  // misses with a slot
    // the renormalisation (every frequency and score / 1e100), before this step's own writes
    // of the same entries, which follow in this wave's program order
    if (st.renorm) {
        for (int64_t i = lane; i < d.nkeys; i += 64) d.freq[i] = d.freq[i] / 1e100;
        for (int64_t i = lane; i < d.nslots; i += 64) d.score[i] = d.score[i] / 1e100;
    }
    // the notes: a key's lead lane adds inc once per lane holding the key, one addition at a
    // time as the reference's loop does; a key first noted here gets its order stamp
    double f = 0.0;
    if (key >= 0 && ln.lead == lane) {
        f = st.renorm ? ln.fq / 1e100 : ln.fq;
        for (int j = 0; j < ln.mult; ++j) f = f + st.inc;
        d.freq[key] = f;
        if (ln.fst == kFirstNever) d.first[key] = tick * 64 + lane;
    }
    // every lane of a key takes the lead's frequency: the score of its slot if it is resident
    // or loaded now (cache_core.py:46 and :82)
    const long long fb = __double_as_longlong(f);
    const uint32_t flo = (uint32_t)__shfl((int)(uint32_t)fb, ln.lead, 64);
    const uint32_t fhi = (uint32_t)__shfl((int)(uint32_t)((uint64_t)fb >> 32), ln.lead, 64);
    const double fk = __longlong_as_double((long long)(((uint64_t)fhi << 32) | flo));
    // the key this lane's victim held: from the staged owners (one wave), else read
    const bool evicts = ln.miss && ln.rank >= ln.from_free && slot >= 0;
    int old_key = -1;
    if constexpr (R == kLruSmall) {
        const int o = lru_owner_of(own, evicts ? slot - (int)d.n_static : 0);
        old_key = evicts ? o : -1;
    } else {
        old_key = evicts ? d.slot_key[slot] : -1;
    }
    // a key repeated later in the step: the later lane's slot is the one key2slot keeps
    bool later = false;
    for (int j = 0; j < k; ++j) {
        const int kj = __builtin_amdgcn_readlane(key, j);
        later = later || (j > lane && kj == key);
    }
    const bool gets = ln.miss && slot >= 0;
    if (ln.hit) {
        d.last[slot] = tick;
        d.score[slot] = fk;
    }
    if (gets) {
        if (old_key >= 0) d.key2slot[old_key] = -1;
        d.slot_key[slot] = key;
        if (!later) d.key2slot[key] = slot;
        d.last[slot] = tick;
        d.score[slot] = fk;
        d.miss[1 + ln.rank] = key;
        d.miss[1 + kDevMaxK + ln.rank] = slot;
    }
    if (lane < k) {
        meta[lane] = (key >= 0 && slot >= 0) ? (float)slot : -1.f;
        meta[k + lane] = ln.w;
    }
    if (lane == 0) {
        d.miss[0] = got;
        d.ctr[kCtrTick] = tick;
        d.ctr[kCtrInc] = (int64_t)__double_as_longlong(st.inc);
        d.ctr[kCtrNextFree] = nf + ln.from_free;
        d.ctr[kCtrHits] += __popcll(ln.hm);
        d.ctr[kCtrMisses] += got;
        d.ctr[kCtrEvict] += evicted;
        d.ctr[kCtrCalls] += 1;
        d.ctr[kCtrLoads] += got;
        d.ctr[kCtrErr] |= (got < ln.nmiss ? kDevErrSlot : 0) | (ln.bad ? kDevErrKey : 0);
    }
}

// key of lane j < k: key_base + id when id is in [0, n_ids) and the key in the store, else -1
__device__ __forceinline__ int lru_key(const DevPaging& d, int64_t id, int64_t key_base, int64_t n_ids) {
    return (id >= 0 && id < n_ids && key_base + id >= 0 && key_base + id < d.nkeys) ? (int)(key_base + id) : -1;
}

// Launch shape of the step kernels for nd >= 1 dynamic slots: one wave of kLruSmall keys per
// lane, or wave 0 plus waves of kLruBig keys per thread (at most 16 in all).
static inline int lru_threads(int64_t nd) {
    return nd <= 64 * kLruSmall ? 64 : (int)(64 * (1 + (nd + 64 * kLruBig - 1) / (64 * kLruBig)));
}

// Wave 0's part of a step before the eviction rounds, `classify` (route / read the keys and
// classify them), and the key holders' staging: one wave requests its keys first, then does
// the rest; with kLruBig keys the other waves stage while wave 0 works, in disjoint branches
// (so wave 0's registers never hold keys and the keys' registers never hold its state).
template <int R, bool SC, typename Classify>
__device__ __forceinline__ LruLane lru_begin(const DevPaging& d, bool renorm, uint64_t (&key)[R], int32_t (&own)[R],
                                             Classify classify) {
    const int nd = (int)(d.nslots - d.n_static);  // in [1, kDevMaxSlots] (device_begin)
    LruLane ln{};
    if constexpr (R == kLruSmall) {
        lru_stage<R, SC>(d, nd, renorm, key, own);
        ln = classify();
    } else if (threadIdx.x < 64) {
        ln = classify();
#pragma unroll
        for (int u = 0; u < R; ++u) key[u] = ~0ull;
    } else {
        lru_stage<R, SC>(d, nd, renorm, key, own);
    }
    return ln;
}

// The step for key_base + id_j, id_j = ids[j] if ids and ids[j] >= 0, else the route row's id
// j (an integer in [0, n_ids)); weights from the row. k <= 0: a warm-up launch that only
// clears the miss list. R keys per key holder, blockDim.x = lru_threads(dynamic slots); SC:
// a score policy (WSA, static) rather than LRU.
template <int R, bool SC>
__global__ __launch_bounds__(R == kLruSmall ? 64 : 1024) void k_lru_step(const DevPaging d,
                                                                          const float* __restrict__ row,
                                                                          const int64_t* __restrict__ ids,
                                                                          int64_t key_base, int64_t n_ids, int k,
                                                                          float* __restrict__ meta) {
    __shared__ LruShared sh;
    const int lane = threadIdx.x & 63;
    const bool wave0 = threadIdx.x < 64;
    if (k <= 0) {
        if (threadIdx.x == 0) d.miss[0] = 0;
        return;
    }
    const LruCtr st = lru_counters(d);
    uint64_t key[R];
    int32_t own[R];
    LruLane ln = lru_begin<R, SC>(d, st.renorm, key, own, [&] {
        int kk = -1;
        float w = 0.f;
        if (lane < k) {
            int64_t id = ids ? ids[lane] : -1;
            if (id < 0) {  // the row's id
                const float f = row[lane];
                id = (f >= 0.f && f < 16777216.f && (float)(int64_t)f == f) ? (int64_t)f : -1;
            }
            kk = lru_key(d, id, key_base, n_ids);
            w = row[k + lane];
        }
        return lru_classify(d, st, lane, k, kk, kk >= 0 ? d.key2slot[kk] : -1, w, sh);
    });
    __syncthreads();
    const int evicted = lru_evict<R, SC>(sh, key, ln, wave0, (int)d.n_static);
    if (wave0) lru_commit<R>(d, st, lane, k, ln, evicted, own, meta);
}

// The route kernel's choice (route.hpp: softmax, top-k, renormalised bf16 weights; row =
// [ids | weights]) and the LRU step of those experts in one launch: wave 0 routes while the
// eviction keys are in flight. ids (optional) replace the chosen expert ids where they are
// >= 0; the weights are the router's. The key -> slot entries of ids 0 .. 64 EPL - 1 (every
// expert the router can pick) are requested at the start with the rest, so the chosen keys'
// residency needs no dependent read (a forced id past them is read). Launch shape and SC as
// for k_lru_step.
template <int EPL, int R, bool SC>
__global__ __launch_bounds__(R == kLruSmall ? 64 : 1024) void k_route_lru(const DevPaging d,
                                                                           const uint16_t* __restrict__ logits, int E,
                                                                           int k, int norm, float* __restrict__ row,
                                                                           const int64_t* __restrict__ ids,
                                                                           int64_t key_base, int64_t n_ids,
                                                                           float* __restrict__ meta) {
    __shared__ LruShared sh;
    const int lane = threadIdx.x & 63;
    const bool wave0 = threadIdx.x < 64;
    if (k <= 0) {
        if (threadIdx.x == 0) d.miss[0] = 0;
        return;
    }
    const LruCtr st = lru_counters(d);
    int64_t forced = -1;
    // key2slot, freq and first of key_base + lane + 64 t (clamped into the table), requested
    // at the start: the chosen keys' entries then need no round trip after the top-k
    int32_t pre[EPL];
    double pfq[EPL];
    int64_t pfst[EPL];
    if (wave0) {
        forced = ids ? ids[lane < k ? lane : 0] : -1;
#pragma unroll
        for (int t = 0; t < EPL; ++t) {
            const int64_t kq = key_base + lane + 64 * t;
            const int64_t kc = kq < 0 ? 0 : (kq < d.nkeys ? kq : d.nkeys - 1);
            pre[t] = d.key2slot[kc];
            pfq[t] = d.freq[kc];
            pfst[t] = d.first[kc];
        }
    }
    uint64_t key[R];
    int32_t own[R];
    LruLane ln = lru_begin<R, SC>(d, st.renorm, key, own, [&] {
        const float val = route_select<EPL>(logits, E, k, norm);
        if (lane < 2 * k) row[lane] = val;
        const float w = __shfl(val, (k + lane) & 63, 64);
        int kk = -1;
        if (lane < k) kk = lru_key(d, forced >= 0 ? forced : (int64_t)val, key_base, n_ids);
        // residency of key_base + id from the requested entries (every lane takes part in the
        // lane reads), or read for an id past them
        const int64_t id = kk >= 0 ? (int64_t)kk - key_base : 0;
        const int src = (int)(id & 63), reg = (int)(id >> 6);
        int res = -1;
        double fq = 0.0;
        int64_t fst = 0;
#pragma unroll
        for (int t = 0; t < EPL; ++t) {
            const int o = __shfl(pre[t], src, 64);
            const long long fb = __double_as_longlong(pfq[t]);
            const uint32_t flo = (uint32_t)__shfl((int)(uint32_t)fb, src, 64);
            const uint32_t fhi = (uint32_t)__shfl((int)(uint32_t)((uint64_t)fb >> 32), src, 64);
            const uint32_t slo = (uint32_t)__shfl((int)(uint32_t)pfst[t], src, 64);
            const uint32_t shi = (uint32_t)__shfl((int)(uint32_t)((uint64_t)pfst[t] >> 32), src, 64);
            if (reg == t) {
                res = o;
                fq = __longlong_as_double((long long)(((uint64_t)fhi << 32) | flo));
                fst = (int64_t)(((uint64_t)shi << 32) | slo);
            }
        }
        const bool have = kk >= 0 && id < 64 * EPL;  // else read after the top-k
        if (kk >= 0 && !have) res = d.key2slot[kk];
        return lru_classify(d, st, lane, k, kk, kk >= 0 ? res : -1, w, sh, have, fq, fst);
    });
    __syncthreads();
    const int evicted = lru_evict<R, SC>(sh, key, ln, wave0, (int)d.n_static);
    if (wave0) lru_commit<R>(d, st, lane, k, ln, evicted, own, meta);
}

__global__ __launch_bounds__(64) void k_write_meta(const PageMeta pm) {
    if ((int)threadIdx.x < pm.n) pm.dst[threadIdx.x] = pm.v[threadIdx.x];
}

// Copy mode 1, misses of one layer on the compute stream itself (ordered after
// the queued reads of the evicted slots by stream order), the layer's meta
// written by the first launch (or by k_write_meta when nothing is missing).
static int page_on_stream(Cache& c, const int64_t* keys, const int64_t* slots, int64_t n, const float* meta, int nmeta,
                          float* meta_dev, hipStream_t st) {
    PageMeta pm;
    for (int i = 0; i < nmeta; ++i) pm.v[i] = meta[i];
    pm.dst = meta_dev;
    pm.n = nmeta;
    hipError_t e;
    if (n == 0) {
        hipLaunchKernelGGL(k_write_meta, dim3(1), dim3(64), 0, st, pm);
        e = hipGetLastError();
        return e == hipSuccess ? WISP_OK : hip_fail(e, "k_write_meta launch");
    }
    for (int64_t i = 0; i < n; ++i)
        if (keys[i] < 0 || keys[i] >= c.host_rows || slots[i] < 0 || slots[i] >= c.nslots)
            return fail_inval("key outside the host store or slot outside the pool");
    if (!c.pool) return no_pool();
    uint8_t* pool = static_cast<uint8_t*>(c.pool->ptr);
    const int64_t row16 = c.row_bytes / 16, slot16 = c.slot_bytes / 16;
    const int64_t per = ((row16 + kPageSplit - 1) / kPageSplit + 1023) / 1024 * 1024;
    for (int64_t i0 = 0; i0 < n; i0 += kPageMax) {
        const int m = (int)std::min<int64_t>(kPageMax, n - i0);
        PagePairs pp;
        for (int j = 0; j < kPageMax; ++j) {
            pp.key[j] = keys[i0 + std::min(j, m - 1)];
            pp.slot[j] = slots[i0 + std::min(j, m - 1)];
        }
        hipLaunchKernelGGL(k_page_rows, dim3(kPageSplit, m), dim3(256), 0, st,
                           reinterpret_cast<const pg_u32x4*>(c.host_dev), reinterpret_cast<pg_u32x4*>(pool), pp, row16,
                           slot16, per, pm);
        e = hipGetLastError();
        if (e != hipSuccess) return hip_fail(e, "k_page_rows launch");
        pm.n = 0;  // meta once
    }
    c.bytes_h2d += n * c.row_bytes;
    c.n_loads += n;
    return WISP_OK;
}

// cache.py:50-76: copies of [(key, slot)] on the side stream, ordered after
// the work already queued on the compute stream (those slots may still be read)
static int issue(Cache& c, const int64_t* keys, const int64_t* slots, int64_t n, hipStream_t compute) {
    if (n <= 0) return WISP_OK;
    for (int64_t i = 0; i < n; ++i)
        if (keys[i] < 0 || keys[i] >= c.host_rows || slots[i] < 0 || slots[i] >= c.nslots)
            return fail_inval("key outside the host store or slot outside the pool");
    if (!c.pool) return no_pool();
    hipError_t e = hipEventRecord(c.order, compute);
    if (e == hipSuccess) e = hipStreamWaitEvent(c.copy, c.order, 0);
    if (e != hipSuccess) return hip_fail(e, "ordering the copy stream");
    uint8_t* pool = static_cast<uint8_t*>(c.pool->ptr);
    if (!c.decode_on_load && c.copy_mode == 1) {
        const int64_t row16 = c.row_bytes / 16, slot16 = c.slot_bytes / 16;
        const int64_t per = ((row16 + kPageSplit - 1) / kPageSplit + 1023) / 1024 * 1024;
        for (int64_t i0 = 0; i0 < n; i0 += kPageMax) {
            const int m = (int)std::min<int64_t>(kPageMax, n - i0);
            PagePairs pp;
            for (int j = 0; j < kPageMax; ++j) {
                pp.key[j] = keys[i0 + std::min(j, m - 1)];
                pp.slot[j] = slots[i0 + std::min(j, m - 1)];
            }
            PageMeta none;
            none.dst = nullptr;
            none.n = 0;
            hipLaunchKernelGGL(k_page_rows, dim3(kPageSplit, m), dim3(256), 0, c.copy,
                               reinterpret_cast<const pg_u32x4*>(c.host_dev), reinterpret_cast<pg_u32x4*>(pool), pp,
                               row16, slot16, per, none);
            e = hipGetLastError();
            if (e != hipSuccess) return hip_fail(e, "k_page_rows launch");
        }
    } else if (!c.decode_on_load) {
        for (int64_t i = 0; i < n; ++i) {
            e = hipMemcpyAsync(pool + slots[i] * c.slot_bytes, c.host + keys[i] * c.row_bytes, (size_t)c.row_bytes,
                               hipMemcpyHostToDevice, c.copy);
            if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync(expert row)");
        }
    } else {
        // cache.py:62-71: quantized rows cross PCIe into staging, then are
        // dequantized once into the bf16 slots
        for (int64_t i0 = 0; i0 < n; i0 += c.staging_rows) {
            const int64_t m = std::min<int64_t>(c.staging_rows, n - i0);
            for (int64_t j = 0; j < m; ++j) {
                e = hipMemcpyAsync(c.staging + j * c.row_bytes, c.host + keys[i0 + j] * c.row_bytes,
                                   (size_t)c.row_bytes, hipMemcpyHostToDevice, c.copy);
                if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync(staging row)");
            }
            for (int64_t j = 0; j < m; ++j) {
                const int rc = wisp_dequant(c.staging + j * c.row_bytes, c.row_bytes, nullptr, 1, 1, c.n, c.bits,
                                            c.group, reinterpret_cast<uint16_t*>(pool + slots[i0 + j] * c.slot_bytes),
                                            c.copy);
                if (rc) return rc;
            }
        }
    }
    e = hipEventRecord(c.done, c.copy);
    if (e != hipSuccess) return hip_fail(e, "hipEventRecord(copies done)");
    c.pending = true;
    c.bytes_h2d += n * c.row_bytes;
    c.n_loads += n;
    return WISP_OK;
}

static int sync_compute(Cache& c, hipStream_t compute) {
    if (!c.pending) return WISP_OK;
    const hipError_t e = hipStreamWaitEvent(compute, c.done, 0);
    return e == hipSuccess ? WISP_OK : hip_fail(e, "hipStreamWaitEvent(copies done)");
}

// cache_core.py:87-106; loads (key, slot) pairs are returned in order
static int core_ensure(Core& c, const int64_t* keys, int64_t n, int64_t* slots, std::vector<int64_t>& lk,
                       std::vector<int64_t>& ls) {
    c.step();
    c.note(keys, n);
    c.calls += 1;
    c.prot_begin();
    for (int64_t i = 0; i < n; ++i) {
        const int64_t s = c.lookup(keys[i]);
        slots[i] = s;
        if (s >= 0) {
            c.prot_add(s);
            c.hits += 1;
        }
    }
    for (int64_t i = 0; i < n; ++i) {
        if (slots[i] >= 0) continue;
        const int64_t s = c.acquire(keys[i]);
        if (s < 0) return no_slot();
        slots[i] = s;
        c.prot_add(s);
        lk.push_back(keys[i]);
        ls.push_back(s);
        c.misses += 1;
    }
    return WISP_OK;
}

static Core* as_core(void* h) { return static_cast<Core*>(h); }
static Cache* as_cache(void* h) { return static_cast<Cache*>(h); }

// host-side bookkeeping while the device holds the LRU state would diverge from it
static int dev_refuse(const Cache& c) {
    return c.dev_on ? fail_inval("device paging is on: end it (wisp_cache_device_end) first") : WISP_OK;
}

}  // namespace wisp

using namespace wisp;

// ------------------------------------------------------------------ CacheCore
extern "C" int wisp_core_create(int64_t nslots, int policy, double decay, int64_t n_static, double admit_after,
                                void** out) {
    clear_error();
    if (!out) return fail_inval("null out");
    if (nslots < 1 || n_static < 0 || n_static > nslots) return fail_inval("need 0 <= n_static <= nslots, nslots >= 1");
    if (policy < kLRU || policy > kStatic) return fail_inval("policy must be 0 (lru), 1 (wsa) or 2 (static)");
    if (!(decay > 0.0)) return fail_inval("decay must be > 0");
    Core* c = new (std::nothrow) Core(nslots, policy, decay, n_static, admit_after);
    if (!c) return fail_inval("out of host memory");
    *out = c;
    return WISP_OK;
}

extern "C" void wisp_core_destroy(void* h) { delete as_core(h); }

extern "C" void wisp_core_step(void* h) { as_core(h)->step(); }

extern "C" void wisp_core_note(void* h, const int64_t* keys, int64_t n) { as_core(h)->note(keys, n); }

extern "C" double wisp_core_norm_freq(void* h, int64_t key) { return as_core(h)->norm_freq(key); }

extern "C" int64_t wisp_core_lookup(void* h, int64_t key) { return as_core(h)->lookup(key); }

extern "C" int wisp_core_ensure(void* h, const int64_t* keys, int64_t n, int64_t* slots, int64_t* load_keys,
                                int64_t* load_slots, int64_t* nloads) {
    clear_error();
    std::vector<int64_t> lk, ls;
    const int rc = core_ensure(*as_core(h), keys, n, slots, lk, ls);
    for (size_t i = 0; i < lk.size(); ++i) {
        load_keys[i] = lk[i];
        load_slots[i] = ls[i];
    }
    *nloads = (int64_t)lk.size();
    return rc;
}

extern "C" int wisp_core_split(void* h, const int64_t* keys, int64_t n, int64_t* hit_keys, int64_t* hit_slots,
                               int64_t* nhit, int64_t* miss_keys, int64_t* nmiss) {
    clear_error();
    Core& c = *as_core(h);
    c.step();
    c.note(keys, n);
    c.calls += 1;
    int64_t a = 0, b = 0;
    for (int64_t i = 0; i < n; ++i) {
        const int64_t s = c.lookup(keys[i]);
        if (s < 0) {
            miss_keys[b++] = keys[i];
        } else {
            hit_keys[a] = keys[i];
            hit_slots[a++] = s;
        }
    }
    c.hits += a;
    c.misses += b;
    *nhit = a;
    *nmiss = b;
    return WISP_OK;
}

extern "C" int wisp_core_acquire(void* h, int64_t key, const int64_t* prot, int64_t nprot, int64_t* slot) {
    clear_error();
    Core& c = *as_core(h);
    c.prot_begin();
    for (int64_t i = 0; i < nprot; ++i) c.prot_add(prot[i]);
    const int64_t s = c.acquire(key);
    if (s < 0) return no_slot();
    *slot = s;
    return WISP_OK;
}

// cache_core.py:125-132: slot, or -1 when resident already, not worth it, or nothing evictable
extern "C" int64_t wisp_core_admit(void* h, int64_t key, const int64_t* prot, int64_t nprot) {
    Core& c = *as_core(h);
    if (c.lookup(key) >= 0 || !(c.norm_freq(key) >= c.admit_after)) return -1;
    c.prot_begin();
    for (int64_t i = 0; i < nprot; ++i) c.prot_add(prot[i]);
    return c.acquire(key);
}

extern "C" int wisp_core_preload(void* h, const int64_t* keys, int64_t n) {
    clear_error();
    Core& c = *as_core(h);
    if (n > c.n_static) return fail_inval("more preload keys than static slots");
    for (int64_t s = 0; s < n; ++s) {
        c.slot_key[s] = keys[s];
        c.key2slot[keys[s]] = s;
    }
    return WISP_OK;
}

// cache_core.py:135-149: new core keeping the hottest resident keys
extern "C" int wisp_core_resized(void* h, int64_t nslots, void** out, int64_t* keys, int64_t* slots, int64_t* n) {
    clear_error();
    Core& c = *as_core(h);
    if (c.n_static != 0) return fail_inval("resize is not supported with a static region");
    if (nslots < 1) return fail_inval("nslots must be >= 1");
    Core* nc = new (std::nothrow) Core(nslots, c.policy, c.decay, 0, c.admit_after);
    if (!nc) return fail_inval("out of host memory");
    nc->tick = c.tick;
    nc->inc = c.inc;
    nc->freq = c.freq;
    nc->freq_order = c.freq_order;
    nc->hits = c.hits;
    nc->misses = c.misses;
    nc->evictions = c.evictions;
    nc->calls = c.calls;
    const std::vector<double>& rank = c.policy == kLRU ? c.last : c.score;
    std::vector<int64_t> live;
    for (int64_t s = 0; s < c.nslots; ++s)
        if (c.slot_key[s] >= 0) live.push_back(s);
    std::stable_sort(live.begin(), live.end(), [&](int64_t a, int64_t b) { return -rank[a] < -rank[b]; });
    const int64_t keep = std::min<int64_t>(nslots, (int64_t)live.size());
    for (int64_t ns = 0; ns < keep; ++ns) {
        const int64_t s = live[ns];
        nc->slot_key[ns] = c.slot_key[s];
        nc->key2slot[c.slot_key[s]] = ns;
        nc->last[ns] = c.last[s];
        nc->score[ns] = c.score[s];
        keys[ns] = c.slot_key[s];
        slots[ns] = ns;
    }
    nc->free.clear();
    for (int64_t s = nslots - 1; s >= keep; --s) nc->free.push_back(s);
    *n = keep;
    *out = nc;
    return WISP_OK;
}

// scalars: [nslots, policy, n_static, tick, hits, misses, evictions, calls, nfree, nresident, nfreq]
// doubles: [decay, admit_after, inc]
extern "C" void wisp_core_state(void* h, int64_t* s, double* d) {
    const Core& c = *as_core(h);
    const int64_t v[11] = {c.nslots, c.policy,  c.n_static, c.tick, c.hits,
                           c.misses, c.evictions, c.calls, (int64_t)c.free.size(), (int64_t)c.key2slot.size(),
                           (int64_t)c.freq.size()};
    for (int i = 0; i < 11; ++i) s[i] = v[i];
    d[0] = c.decay;
    d[1] = c.admit_after;
    d[2] = c.inc;
}

// snapshots: slot_key/last/score [nslots], free [nfree] (bottom of the stack first),
// freq keys/values [nfreq] in insertion order
extern "C" void wisp_core_arrays(void* h, int64_t* slot_key, double* last, double* score, int64_t* free_list,
                                 int64_t* freq_keys, double* freq_vals) {
    const Core& c = *as_core(h);
    for (int64_t s = 0; s < c.nslots; ++s) {
        if (slot_key) slot_key[s] = c.slot_key[s];
        if (last) last[s] = c.last[s];
        if (score) score[s] = c.score[s];
    }
    if (free_list)
        for (size_t i = 0; i < c.free.size(); ++i) free_list[i] = c.free[i];
    if (freq_keys || freq_vals)
        for (size_t i = 0; i < c.freq_order.size(); ++i) {
            if (freq_keys) freq_keys[i] = c.freq_order[i];
            if (freq_vals) freq_vals[i] = c.freq.at(c.freq_order[i]);
        }
}

// ------------------------------------------------------------------ ExpertCache
extern "C" int wisp_cache_create(void* core, int64_t slot_bytes, const uint8_t* host, int64_t host_rows,
                                 int64_t row_bytes, int bits, int64_t n, int64_t group, int decode_on_load,
                                 int64_t staging_rows, int device, void** out) {
    clear_error();
    if (!core || !host || !out) return fail_inval("null core, host or out");
    if (host_rows < 1 || row_bytes < 1) return fail_inval("empty host store");
    if (decode_on_load && bits < 16) {
        if (wisp_expert_nbytes(n, bits, group) != row_bytes) return fail_inval("row_bytes != expert_nbytes(n, bits)");
        if (slot_bytes != 3 * n * 2) return fail_inval("decode_on_load slots hold 3n bf16 values");
        if (staging_rows < 1) return fail_inval("staging_rows must be >= 1");
    } else if (slot_bytes < row_bytes) {
        return fail_inval("slot_bytes < row_bytes");
    }
    if (slot_bytes % 16) return fail_inval("slot_bytes must be a multiple of 16");
    Cache* c = new (std::nothrow) Cache();
    if (!c) return fail_inval("out of host memory");
    c->core = as_core(core);
    c->device = device;
    c->nslots = c->core->nslots;
    c->slot_bytes = slot_bytes;
    c->host = host;
    c->host_rows = host_rows;
    c->row_bytes = row_bytes;
    c->bits = bits;
    c->n = n;
    c->group = group;
    c->decode_on_load = decode_on_load && bits < 16;
    c->staging_rows = c->decode_on_load ? staging_rows : 0;
    int cur = 0;
    (void)hipGetDevice(&cur);
    hipError_t e = hipSetDevice(device);
    int rc = e == hipSuccess ? alloc_pool(*c) : hip_fail(e, "hipSetDevice");
    if (!rc && c->decode_on_load) {
        e = hipMalloc(reinterpret_cast<void**>(&c->staging), (size_t)(c->staging_rows * row_bytes));
        if (e != hipSuccess) rc = hip_fail(e, "hipMalloc(staging)");
    }
    if (!rc) {
        e = hipStreamCreateWithFlags(&c->copy, hipStreamNonBlocking);  // default priority
        if (e == hipSuccess) e = hipEventCreateWithFlags(&c->order, hipEventDisableTiming);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&c->done, hipEventDisableTiming);
        if (e != hipSuccess) rc = hip_fail(e, "creating the copy stream / events");
    }
    (void)hipSetDevice(cur);
    if (rc) {
        if (c->done) (void)hipEventDestroy(c->done);
        if (c->order) (void)hipEventDestroy(c->order);
        if (c->copy) (void)hipStreamDestroy(c->copy);
        if (c->staging) (void)hipFree(c->staging);
        pool_release(c->pool);
        delete c;
        return rc;
    }
    *out = c;
    return WISP_OK;
}

// Frees the cache's share of the pool (views keep it alive) and its core.
extern "C" void wisp_cache_destroy(void* h) {
    Cache* c = as_cache(h);
    if (!c) return;
    int cur = 0;
    (void)hipGetDevice(&cur);
    (void)hipSetDevice(c->device);
    (void)hipStreamSynchronize(c->copy);
    (void)hipEventDestroy(c->done);
    (void)hipEventDestroy(c->order);
    (void)hipStreamDestroy(c->copy);
    if (c->staging) (void)hipFree(c->staging);
    if (c->dev_block) (void)hipFree(c->dev_block);
    (void)hipSetDevice(cur);
    pool_release(c->pool);
    delete c->core;
    delete c;
}

extern "C" void* wisp_cache_core(void* h) { return as_cache(h)->core; }
extern "C" void* wisp_cache_pool(void* h) {
    Cache* c = as_cache(h);
    return c->pool ? c->pool->ptr : nullptr;
}
extern "C" void* wisp_cache_copy_stream(void* h) { return as_cache(h)->copy; }

extern "C" void wisp_cache_counters(void* h, int64_t* bytes_h2d, int64_t* n_loads) {
    *bytes_h2d = as_cache(h)->bytes_h2d;
    *n_loads = as_cache(h)->n_loads;
}

// A DLPack view [nslots, slot_bytes] uint8 of the pool on the ROCm device; the
// view holds a reference, so the memory outlives the cache while it is used.
extern "C" void* wisp_cache_pool_dlpack(void* h) {
    Cache* c = as_cache(h);
    if (!c->pool) {
        no_pool();
        return nullptr;
    }
    PoolView* v = new (std::nothrow) PoolView();
    if (!v) return nullptr;
    c->pool->refs.fetch_add(1);
    v->block = c->pool;
    v->shape[0] = c->nslots;
    v->shape[1] = c->slot_bytes;
    v->strides[0] = c->slot_bytes;
    v->strides[1] = 1;
    v->m.dl_tensor.data = c->pool->ptr;
    v->m.dl_tensor.device = DLDevice{10 /* kDLROCM */, c->device};
    v->m.dl_tensor.ndim = 2;
    v->m.dl_tensor.dtype = DLDataType{1 /* kDLUInt */, 8, 1};
    v->m.dl_tensor.shape = v->shape;
    v->m.dl_tensor.strides = v->strides;
    v->m.dl_tensor.byte_offset = 0;
    v->m.manager_ctx = v;
    v->m.deleter = view_deleter;
    return &v->m;
}

// Delete a view that was never handed to a consumer.
extern "C" void wisp_cache_pool_dlpack_free(void* m) {
    if (m) view_deleter(static_cast<DLManagedTensor*>(m));
}

extern "C" int wisp_cache_issue(void* h, const int64_t* keys, const int64_t* slots, int64_t n, void* compute) {
    clear_error();
    if (dev_refuse(*as_cache(h))) return WISP_EINVAL;
    return issue(*as_cache(h), keys, slots, n, (hipStream_t)compute);
}

extern "C" int wisp_cache_sync_compute(void* h, void* compute) {
    clear_error();
    return sync_compute(*as_cache(h), (hipStream_t)compute);
}

// cache.py:87-91: ensure residency, issue the misses' copies, order compute after them
extern "C" int wisp_cache_ensure(void* h, const int64_t* keys, int64_t n, int64_t* slots, void* compute) {
    clear_error();
    if (dev_refuse(*as_cache(h))) return WISP_EINVAL;
    Cache& c = *as_cache(h);
    std::vector<int64_t> lk, ls;
    int rc = core_ensure(*c.core, keys, n, slots, lk, ls);
    if (rc) return rc;
    rc = issue(c, lk.data(), ls.data(), (int64_t)lk.size(), (hipStream_t)compute);
    if (rc) return rc;
    return sync_compute(c, (hipStream_t)compute);
}

// graphdec.py:216-231 for one layer: slots = ensure(keys); meta_host = [slots |
// weights] (pinned, float32 [2k]); meta_dev <- meta_host on the compute stream,
// ordered after the expert copies. Returns the slots in `slots` (may be NULL).
extern "C" int wisp_cache_prepare_layer(void* h, const int64_t* keys, const float* weights, int k, float* meta_host,
                                        float* meta_dev, int64_t* slots, void* compute) {
    clear_error();
    if (k < 1 || k > 64 || !keys || !weights || !meta_host || !meta_dev) return fail_inval("bad prepare_layer args");
    int64_t sl[64];
    int rc = wisp_cache_ensure(h, keys, k, sl, compute);
    if (rc) return rc;
    for (int j = 0; j < k; ++j) {
        meta_host[j] = (float)sl[j];
        meta_host[k + j] = weights[j];
        if (slots) slots[j] = sl[j];
    }
    const hipError_t e = hipMemcpyAsync(meta_dev, meta_host, sizeof(float) * 2 * k, hipMemcpyHostToDevice,
                                        (hipStream_t)compute);
    return e == hipSuccess ? WISP_OK : hip_fail(e, "hipMemcpyAsync(meta)");
}

// graphdec.py:216-231 + :305-306 for one layer, the router row included: copy
// row_dev = [expert ids (k) | weights (k)] (float32, on the device) into the
// pinned row_host on the compute stream and wait for it (the one sync per
// layer), then prepare_layer with keys key_base + id, id in [0, n_ids). ids (may be NULL)
// replaces the row's expert ids (a caller's own routing); the weights always
// come from the row.
extern "C" int wisp_cache_prepare_row(void* h, const float* row_dev, float* row_host, int k, int64_t key_base,
                                      int64_t n_ids, const int64_t* ids, float* meta_host, float* meta_dev,
                                      int64_t* slots, void* compute) {
    clear_error();
    if (k < 1 || k > 64 || !row_dev || !row_host || !meta_host || !meta_dev) return fail_inval("bad prepare_row args");
    hipStream_t st = (hipStream_t)compute;
    hipError_t e = hipMemcpyAsync(row_host, row_dev, sizeof(float) * 2 * k, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) return hip_fail(e, "reading the router row");
    int64_t keys[64];
    for (int j = 0; j < k; ++j) {
        int64_t id;
        if (ids) {
            id = ids[j];
        } else {
            const float f = row_host[j];
            if (!(f >= 0.f && f < 16777216.f) || (float)(int64_t)f != f) return fail_inval("router row holds a bad id");
            id = (int64_t)f;
        }
        if (id < 0 || id >= n_ids) return fail_inval("expert id outside [0, n_ids)");
        keys[j] = key_base + id;
    }
    return wisp_cache_prepare_layer(h, keys, row_host + k, k, meta_host, meta_dev, slots, compute);
}

// prepare_row for a row the GPU writes into pinned host memory itself (the
// route kernel's host_row / host_flag): spin until the flag moves, then the
// layer's step. Copy mode 1 pages on the compute stream with the meta written
// by the page kernel; mode 0 goes through prepare_layer.
extern "C" int wisp_cache_prepare_signaled(void* h, float* row_host, const volatile uint32_t* flag,
                                           uint32_t flag_before, uint32_t* flag_after, int timeout_ms, int k,
                                           int64_t key_base, int64_t n_ids, const int64_t* ids, float* meta_host,
                                           float* meta_dev, void* compute) {
    clear_error();
    if (dev_refuse(*as_cache(h))) return WISP_EINVAL;
    if (k < 1 || k > 16 || !row_host || !flag || !meta_host || !meta_dev) return fail_inval("bad prepare_signaled args");
    const auto t0 = std::chrono::steady_clock::now();
    uint32_t f;
    unsigned spins = 0;
    while ((f = *flag) == flag_before) {
        if ((++spins & 4095u) == 0 &&
            std::chrono::duration_cast<std::chrono::milliseconds>(std::chrono::steady_clock::now() - t0).count() >
                timeout_ms) {
            set_error("timed out after %d ms waiting for the router row", timeout_ms);
            return WISP_EINVAL;
        }
        __builtin_ia32_pause();
    }
    std::atomic_thread_fence(std::memory_order_acquire);
    if (flag_after) *flag_after = f;
    const volatile float* row = row_host;
    int64_t keys[16];
    float w[16];
    for (int j = 0; j < k; ++j) {
        int64_t id;
        if (ids) {
            id = ids[j];
        } else {
            const float v = row[j];
            if (!(v >= 0.f && v < 16777216.f) || (float)(int64_t)v != v) return fail_inval("router row holds a bad id");
            id = (int64_t)v;
        }
        if (id < 0 || id >= n_ids) return fail_inval("expert id outside [0, n_ids)");
        keys[j] = key_base + id;
        w[j] = row[k + j];
    }
    Cache& c = *as_cache(h);
    hipStream_t st = (hipStream_t)compute;
    if (c.copy_mode != 1) return wisp_cache_prepare_layer(h, keys, w, k, meta_host, meta_dev, nullptr, compute);
    int64_t sl[16];
    std::vector<int64_t> lk, ls;
    int rc = core_ensure(*c.core, keys, k, sl, lk, ls);
    if (rc) return rc;
    for (int j = 0; j < k; ++j) {
        meta_host[j] = (float)sl[j];
        meta_host[k + j] = w[j];
    }
    rc = sync_compute(c, st);  // copies still pending on the side stream (prefetch, admit)
    if (rc) return rc;
    return page_on_stream(c, lk.data(), ls.data(), (int64_t)lk.size(), meta_host, 2 * k, meta_dev, st);
}

// Copy mode: 0 = one hipMemcpyAsync per row (the DMA engines), 1 = k_page_rows
// (the GPU reads the pinned host rows over PCIe). Mode 1 needs a host store
// mapped into the device's address space (pinned by hipHostMalloc or
// registered) and 16-byte rows; otherwise it is refused.
extern "C" int wisp_cache_set_copy_mode(void* h, int mode) {
    clear_error();
    Cache& c = *as_cache(h);
    if (mode == 0) {
        c.copy_mode = 0;
        return WISP_OK;
    }
    if (mode != 1) return fail_inval("copy mode must be 0 (hipMemcpyAsync) or 1 (page kernel)");
    if (c.decode_on_load) return fail_inval("the page kernel does not stage decode-on-load rows");
    if (c.row_bytes % 16 || c.slot_bytes % 16 || !aligned(c.host, 16))
        return fail_inval("the page kernel needs 16-byte rows and a 16-byte aligned host store");
    void* dptr = nullptr;
    const hipError_t e = hipHostGetDevicePointer(&dptr, const_cast<uint8_t*>(c.host), 0);
    if (e != hipSuccess || !dptr) {
        (void)hipGetLastError();
        set_error("the host store is not mapped for the device (not pinned): %s", hipGetErrorString(e));
        return WISP_EINVAL;
    }
    c.host_dev = static_cast<const uint8_t*>(dptr);
    c.copy_mode = 1;
    return WISP_OK;
}

// cache.py:144-158: keep the hottest experts in a pool of `nslots` rows. The
// device is synchronised, the old pool released before the new one is
// allocated, and the kept experts re-copied from the host store.
extern "C" int wisp_cache_resize(void* h, int64_t nslots) {
    clear_error();
    if (dev_refuse(*as_cache(h))) return WISP_EINVAL;
    Cache& c = *as_cache(h);
    if (c.decode_on_load) return fail_inval("resize is not supported with decode_on_load");
    if (nslots == c.nslots) return WISP_OK;
    std::vector<int64_t> keys(std::max<int64_t>(nslots, 1)), slots(keys.size());
    int64_t nk = 0;
    void* nc = nullptr;
    int rc = wisp_core_resized(c.core, nslots, &nc, keys.data(), slots.data(), &nk);
    if (rc) return rc;
    int cur = 0;
    (void)hipGetDevice(&cur);
    (void)hipSetDevice(c.device);
    hipError_t e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        wisp_core_destroy(nc);
        (void)hipSetDevice(cur);
        return hip_fail(e, "hipDeviceSynchronize");
    }
    delete c.core;
    c.core = as_core(nc);
    pool_release(c.pool);
    c.pool = nullptr;
    c.pending = false;
    c.nslots = nslots;
    rc = alloc_pool(c);
    if (!rc) rc = issue(c, keys.data(), slots.data(), nk, c.copy);
    if (!rc) {
        e = hipStreamSynchronize(c.copy);
        if (e != hipSuccess) rc = hip_fail(e, "hipStreamSynchronize(copy)");
    }
    (void)hipSetDevice(cur);
    return rc;
}

// ------------------------------------------------------------------ device paging
// The graph decoder's paging point on the GPU: wisp_cache_device_step queues
// k_lru_step (the LRU ensure of one layer) and k_page_list (its misses, read from
// the pinned store over PCIe) on a stream, with no host decision, so a whole decode
// step can be one graph. While device paging is on, the LRU state lives in device
// memory and the host core is stale: entry points that would read or change it are
// refused until wisp_cache_device_sync / _end copy the state back.

namespace wisp {

static size_t align256(size_t b) { return (b + 255) / 256 * 256; }

// the device state -> the host core (and the cache's load counters)
static int dev_download(Cache& c, hipStream_t st) {
    hipError_t e = hipStreamSynchronize(st);
    if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize (device paging)");
    const DevPaging& d = c.dev;
    std::vector<int32_t> sk(d.nslots), k2s(d.nkeys);
    std::vector<int64_t> last(d.nslots), ctr(kCtrN), first(d.nkeys);
    std::vector<double> score(d.nslots), freq(d.nkeys);
    e = hipMemcpy(sk.data(), d.slot_key, sizeof(int32_t) * d.nslots, hipMemcpyDeviceToHost);
    if (e == hipSuccess) e = hipMemcpy(last.data(), d.last, sizeof(int64_t) * d.nslots, hipMemcpyDeviceToHost);
    if (e == hipSuccess) e = hipMemcpy(score.data(), d.score, sizeof(double) * d.nslots, hipMemcpyDeviceToHost);
    if (e == hipSuccess) e = hipMemcpy(k2s.data(), d.key2slot, sizeof(int32_t) * d.nkeys, hipMemcpyDeviceToHost);
    if (e == hipSuccess) e = hipMemcpy(freq.data(), d.freq, sizeof(double) * d.nkeys, hipMemcpyDeviceToHost);
    if (e == hipSuccess) e = hipMemcpy(first.data(), d.first, sizeof(int64_t) * d.nkeys, hipMemcpyDeviceToHost);
    if (e == hipSuccess) e = hipMemcpy(ctr.data(), d.ctr, sizeof(int64_t) * kCtrN, hipMemcpyDeviceToHost);
    if (e != hipSuccess) return hip_fail(e, "hipMemcpy (device paging state)");
    Core& core = *c.core;
    for (int64_t s = 0; s < d.nslots; ++s) {
        core.slot_key[s] = sk[s];
        core.last[s] = (double)last[s];
        core.score[s] = score[s];
    }
    core.key2slot.clear();
    for (int64_t key = 0; key < d.nkeys; ++key)
        if (k2s[key] >= 0) core.key2slot[key] = k2s[key];
    // the frequency table: keys noted before device paging began keep their place; keys first
    // noted on the device join it in the order of their first notes (step, then position)
    std::vector<std::pair<int64_t, int64_t>> fresh_keys;
    for (int64_t key = 0; key < d.nkeys; ++key) {
        if (first[key] == kFirstBefore) core.freq[key] = freq[key];
        else if (first[key] >= 0) fresh_keys.emplace_back(first[key], key);
    }
    std::sort(fresh_keys.begin(), fresh_keys.end());
    for (const auto& fk : fresh_keys) core.freq_at(fk.second) = freq[fk.second];
    core.inc = __builtin_bit_cast(double, ctr[kCtrInc]);
    core.free.clear();
    for (int64_t s = d.nslots - 1; s >= ctr[kCtrNextFree]; --s) core.free.push_back(s);
    core.tick = ctr[kCtrTick];
    core.hits = ctr[kCtrHits];
    core.misses = ctr[kCtrMisses];
    core.evictions = ctr[kCtrEvict];
    core.calls = ctr[kCtrCalls];
    const int64_t fresh = ctr[kCtrLoads] - c.dev_loads_seen;
    c.bytes_h2d += fresh * c.row_bytes;
    c.n_loads += fresh;
    c.dev_loads_seen = ctr[kCtrLoads];
    if (ctr[kCtrErr]) {
        const int64_t zero = 0;
        (void)hipMemcpy(d.ctr + kCtrErr, &zero, sizeof(int64_t), hipMemcpyHostToDevice);
        set_error("device paging: %s%s", (ctr[kCtrErr] & kDevErrKey) ? "a routed id outside [0, n_ids) or the store; " : "",
                  (ctr[kCtrErr] & kDevErrSlot) ? "no evictable slot for a miss (dynamic region smaller than k)" : "");
        return WISP_EINVAL;
    }
    return WISP_OK;
}

}  // namespace wisp

// Copy the host core's state to the device and turn device paging on (a no-op when it
// is on). Any policy (LRU evicts by last use, WSA and static by score); needs the
// page-kernel copy mode, at most 26880 dynamic slots (2^20 in all), the free slots at
// the top of the pool (the order the core hands them out) and every noted key in the
// store. Stream-ordered after the copies already issued.
extern "C" int wisp_cache_device_begin(void* h, void* stream) {
    clear_error();
    Cache& c = *as_cache(h);
    if (c.dev_on) return WISP_OK;
    const Core& core = *c.core;
    if (c.copy_mode != 1 || !c.host_dev) return fail_inval("device paging needs the page-kernel copy mode");
    if (!c.pool) return no_pool();
    if (c.nslots > (1 << 20) || c.nslots - core.n_static > kDevMaxSlots)
        return fail_inval("device paging: at most 26880 dynamic slots and 2^20 slots in all");
    if (c.host_rows > INT32_MAX) return fail_inval("device paging: at most 2^31 - 1 store rows");
    if (core.tick > (int64_t(1) << 42)) return fail_inval("device paging: tick beyond 2^42");
    const int64_t nfree = (int64_t)core.free.size(), nf = c.nslots - nfree;
    for (int64_t i = 0; i < nfree; ++i)
        if (core.free[i] != c.nslots - 1 - i) return fail_inval("device paging needs the free slots at the top of the pool");
    DevPaging d;
    d.nslots = c.nslots;
    d.nkeys = c.host_rows;
    d.n_static = core.n_static;
    d.decay = core.decay;
    std::vector<int32_t> sk(d.nslots), k2s(d.nkeys, -1);
    std::vector<int64_t> last(d.nslots), first(d.nkeys, kFirstNever);
    std::vector<double> freq(d.nkeys, 0.0);
    for (int64_t s = 0; s < d.nslots; ++s) {
        sk[s] = (int32_t)core.slot_key[s];
        last[s] = (int64_t)core.last[s];
    }
    for (const auto& kv : core.key2slot) {
        if (kv.first < 0 || kv.first >= d.nkeys) return fail_inval("device paging: a resident key outside the store");
        k2s[kv.first] = (int32_t)kv.second;
    }
    for (const auto& kv : core.freq) {
        if (kv.first < 0 || kv.first >= d.nkeys) return fail_inval("device paging: a noted key outside the store");
        freq[kv.first] = kv.second;
        first[kv.first] = kFirstBefore;
    }
    const int64_t ctr[kCtrN] = {core.tick, nf, core.hits, core.misses, core.evictions, core.calls, 0, 0, 1,
                                __builtin_bit_cast(int64_t, core.inc)};
    const size_t b_sk = align256(sizeof(int32_t) * d.nslots), b_last = align256(sizeof(int64_t) * d.nslots),
                 b_score = align256(sizeof(double) * d.nslots), b_k2s = align256(sizeof(int32_t) * d.nkeys),
                 b_freq = align256(sizeof(double) * d.nkeys), b_first = align256(sizeof(int64_t) * d.nkeys),
                 b_ctr = align256(sizeof(int64_t) * kCtrN), b_miss = align256(sizeof(int32_t) * (1 + 2 * kDevMaxK));
    int cur = 0;
    (void)hipGetDevice(&cur);
    (void)hipSetDevice(c.device);
    hipStream_t st = (hipStream_t)stream;
    hipError_t e;
    if (c.dev_block && (c.dev.nslots != d.nslots || c.dev.nkeys != d.nkeys)) {  // the slot count changed
        e = hipDeviceSynchronize();
        if (e != hipSuccess) {
            (void)hipSetDevice(cur);
            return hip_fail(e, "hipDeviceSynchronize (device paging state)");
        }
        (void)hipFree(c.dev_block);
        c.dev_block = nullptr;
    }
    void* block = c.dev_block;
    if (!block) {
        e = hipMalloc(&block, b_sk + b_last + b_score + b_k2s + b_freq + b_first + b_ctr + b_miss);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            (void)hipSetDevice(cur);
            return hip_fail(e, "hipMalloc (device paging state)");
        }
    }
    uint8_t* p = static_cast<uint8_t*>(block);
    d.slot_key = reinterpret_cast<int32_t*>(p);
    p += b_sk;
    d.last = reinterpret_cast<int64_t*>(p);
    p += b_last;
    d.score = reinterpret_cast<double*>(p);
    p += b_score;
    d.key2slot = reinterpret_cast<int32_t*>(p);
    p += b_k2s;
    d.freq = reinterpret_cast<double*>(p);
    p += b_freq;
    d.first = reinterpret_cast<int64_t*>(p);
    p += b_first;
    d.ctr = reinterpret_cast<int64_t*>(p);
    p += b_ctr;
    d.miss = reinterpret_cast<int32_t*>(p);
    int rc = sync_compute(c, st);  // copies still pending on the side stream
    if (!rc) {
        e = hipMemcpyAsync(d.slot_key, sk.data(), sizeof(int32_t) * d.nslots, hipMemcpyHostToDevice, st);
        if (e == hipSuccess) e = hipMemcpyAsync(d.last, last.data(), sizeof(int64_t) * d.nslots, hipMemcpyHostToDevice, st);
        if (e == hipSuccess)
            e = hipMemcpyAsync(d.score, core.score.data(), sizeof(double) * d.nslots, hipMemcpyHostToDevice, st);
        if (e == hipSuccess) e = hipMemcpyAsync(d.key2slot, k2s.data(), sizeof(int32_t) * d.nkeys, hipMemcpyHostToDevice, st);
        if (e == hipSuccess) e = hipMemcpyAsync(d.freq, freq.data(), sizeof(double) * d.nkeys, hipMemcpyHostToDevice, st);
        if (e == hipSuccess) e = hipMemcpyAsync(d.first, first.data(), sizeof(int64_t) * d.nkeys, hipMemcpyHostToDevice, st);
        if (e == hipSuccess) e = hipMemcpyAsync(d.ctr, ctr, sizeof(int64_t) * kCtrN, hipMemcpyHostToDevice, st);
        if (e == hipSuccess) e = hipMemsetAsync(d.miss, 0, sizeof(int32_t) * (1 + 2 * kDevMaxK), st);
        if (e == hipSuccess) e = hipStreamSynchronize(st);  // the host vectors go out of scope
        if (e != hipSuccess) rc = hip_fail(e, "uploading the device paging state");
    }
    (void)hipSetDevice(cur);
    c.dev = d;
    c.dev_block = block;
    if (rc) return rc;  // the block is kept (device paging stays off)
    c.dev_on = true;
    c.dev_score = core.policy != kLRU;
    c.dev_loads_seen = 0;
    return WISP_OK;
}

// k distinct keys can always be placed when k <= the dynamic slots: the step's hits
// are protected, and the misses take the other dynamic slots. With fewer dynamic
// slots than k a miss can find no evictable slot (the reference's CacheCore.acquire
// raises on it, cache_core.py:64-84), so the step is refused on the host before any
// launch rather than left to the device report that only the next sync reads.
static int no_slot_for_k(const Cache& c, int k) {
    char msg[160];
    std::snprintf(msg, sizeof msg, "device paging: top-k %d exceeds the %lld dynamic slots (no evictable slot)", k,
                  (long long)(c.nslots - c.dev.n_static));
    return fail_inval(msg);
}

// the step kernels' launch for nd dynamic slots (one wave up to 64 kLruSmall, else lru_threads)
template <bool SC>
static void launch_lru_step(const Cache& c, int64_t nd, hipStream_t st, const float* row, const int64_t* ids,
                            int64_t key_base, int64_t n_ids, int k, float* meta) {
    if (nd <= 64 * kLruSmall)
        hipLaunchKernelGGL((k_lru_step<kLruSmall, SC>), dim3(1), dim3(64), 0, st, c.dev, row, ids, key_base, n_ids, k,
                           meta);
    else
        hipLaunchKernelGGL((k_lru_step<kLruBig, SC>), dim3(1), dim3(lru_threads(nd)), 0, st, c.dev, row, ids,
                           key_base, n_ids, k, meta);
}
template <int EPL, bool SC>
static void launch_route_lru(const Cache& c, int64_t nd, hipStream_t st, const uint16_t* logits, int E, int k, int nt,
                             float* row, const int64_t* ids, int64_t key_base, int64_t n_ids, float* meta) {
    if (nd <= 64 * kLruSmall)
        hipLaunchKernelGGL((k_route_lru<EPL, kLruSmall, SC>), dim3(1), dim3(64), 0, st, c.dev, logits, E, k, nt, row,
                           ids, key_base, n_ids, meta);
    else
        hipLaunchKernelGGL((k_route_lru<EPL, kLruBig, SC>), dim3(1), dim3(lru_threads(nd)), 0, st, c.dev, logits, E,
                           k, nt, row, ids, key_base, n_ids, meta);
}

// One layer's paging point on `stream` (capturable: no host sync, no allocation):
// ensure the keys key_base + id (ids: device int64 [k], else the route row's ids,
// row = device float32 [ids (k) | weights (k)]), meta (device float32 [2k]) =
// [slots | weights], then the page kernel for the misses. k in [1, 16]; k = 0
// launches both kernels without a step (a warm-up before graph capture).
extern "C" int wisp_cache_device_step(void* h, const float* row, const int64_t* ids, int64_t key_base, int64_t n_ids,
                                      int k, float* meta, void* stream) {
    clear_error();
    Cache& c = *as_cache(h);
    if (!c.dev_on) return fail_inval("device paging is off (wisp_cache_device_begin)");
    if (k < 0 || k > kDevMaxK) return fail_inval("device paging takes 0 <= k <= 16");
    if (k > 0 && (!row || !meta || n_ids < 1)) return fail_inval("device paging step: null row / meta or n_ids < 1");
    if (k > c.nslots - c.dev.n_static) return no_slot_for_k(c, k);
    if (!c.pool) return no_pool();
    hipStream_t st = (hipStream_t)stream;
    const int64_t nd = c.nslots - c.dev.n_static;
    if (c.dev_score)
        launch_lru_step<true>(c, nd, st, row, ids, key_base, n_ids, k, meta);
    else
        launch_lru_step<false>(c, nd, st, row, ids, key_base, n_ids, k, meta);
    int rc = check_launch("k_lru_step");
    if (rc) return rc;
    const int64_t row16 = c.row_bytes / 16, slot16 = c.slot_bytes / 16;
    const int64_t per = ((row16 + kPageSplit - 1) / kPageSplit + 1023) / 1024 * 1024;
    hipLaunchKernelGGL(k_page_list, dim3(kPageSplit, k > 0 ? k : 1), dim3(256), 0, st,
                       reinterpret_cast<const pg_u32x4*>(c.host_dev), reinterpret_cast<pg_u32x4*>(c.pool->ptr),
                       c.dev.miss, row16, slot16, per);
    return check_launch("k_page_list");
}

// wisp_dl_route (moe.py:41-47: softmax, top-k, renormalised bf16 weights into row) and
// wisp_cache_device_step on its choice in one launch, then the page kernel.
extern "C" int wisp_cache_device_route_step(void* h, const uint16_t* logits, int E, int k, int norm_topk, float* row,
                                            const int64_t* ids, int64_t key_base, int64_t n_ids, float* meta,
                                            void* stream) {
    clear_error();
    Cache& c = *as_cache(h);
    if (!c.dev_on) return fail_inval("device paging is off (wisp_cache_device_begin)");
    if (k < 0 || k > kDevMaxK) return fail_inval("device paging takes 0 <= k <= 16");
    if (k > 0 && (!logits || !row || !meta || n_ids < 1 || E < k || E > 1024))
        return fail_inval("device route step: null logits / row / meta, n_ids < 1 or E outside [k, 1024]");
    if (k > c.nslots - c.dev.n_static) return no_slot_for_k(c, k);
    if (!c.pool) return no_pool();
    hipStream_t st = (hipStream_t)stream;
    const int nt = norm_topk ? 1 : 0;
    const int64_t nd = c.nslots - c.dev.n_static;
#define WISP_RL(EPL)                                                                                   \
    if (c.dev_score)                                                                                   \
        launch_route_lru<EPL, true>(c, nd, st, logits, E, k, nt, row, ids, key_base, n_ids, meta);     \
    else                                                                                               \
        launch_route_lru<EPL, false>(c, nd, st, logits, E, k, nt, row, ids, key_base, n_ids, meta)
    if (E <= 64) {
        WISP_RL(1);
    } else if (E <= 128) {
        WISP_RL(2);
    } else if (E <= 256) {
        WISP_RL(4);
    } else if (E <= 512) {
        WISP_RL(8);
    } else {
        WISP_RL(16);
    }
#undef WISP_RL
    int rc = check_launch("k_route_lru");
    if (rc) return rc;
    const int64_t row16 = c.row_bytes / 16, slot16 = c.slot_bytes / 16;
    const int64_t per = ((row16 + kPageSplit - 1) / kPageSplit + 1023) / 1024 * 1024;
    hipLaunchKernelGGL(k_page_list, dim3(kPageSplit, k > 0 ? k : 1), dim3(256), 0, st,
                       reinterpret_cast<const pg_u32x4*>(c.host_dev), reinterpret_cast<pg_u32x4*>(c.pool->ptr),
                       c.dev.miss, row16, slot16, per);
    return check_launch("k_page_list");
}

// Wait for `stream` and copy the device state into the host core (device paging
// stays on). Reports (once) a step that met a bad id or had no evictable slot.
extern "C" int wisp_cache_device_sync(void* h, void* stream) {
    clear_error();
    Cache& c = *as_cache(h);
    if (!c.dev_on) return WISP_OK;
    int cur = 0;
    (void)hipGetDevice(&cur);
    (void)hipSetDevice(c.device);
    const int rc = dev_download(c, (hipStream_t)stream);
    (void)hipSetDevice(cur);
    return rc;
}

// wisp_cache_device_sync, then device paging off. The state stays allocated at the same
// address; a captured step replayed while it is off does nothing but write slot -1 into meta.
extern "C" int wisp_cache_device_end(void* h, void* stream) {
    clear_error();
    Cache& c = *as_cache(h);
    if (!c.dev_on) return WISP_OK;
    int cur = 0;
    (void)hipGetDevice(&cur);
    (void)hipSetDevice(c.device);
    int rc = dev_download(c, (hipStream_t)stream);
    const int64_t off = 0;
    const hipError_t e = hipMemcpy(c.dev.ctr + kCtrOn, &off, sizeof(int64_t), hipMemcpyHostToDevice);
    if (e != hipSuccess && !rc) rc = hip_fail(e, "hipMemcpy (device paging off)");
    (void)hipSetDevice(cur);
    c.dev_on = false;
    return rc;
}

extern "C" int wisp_cache_device_active(void* h) { return as_cache(h)->dev_on ? 1 : 0; }
