/*
 * wisp_hip.h -- C ABI of the MI355X (gfx950) fused group-wise expert
 * dequant+GEMV path.
 *
 * Plain pointers, sizes and a stream handle; no torch types. Every device
 * pointer is a HIP device address; `stream` is a hipStream_t passed as void*
 * (NULL = the default stream). The kernel entry points are asynchronous: they
 * enqueue kernels on `stream` and return; none allocates, frees or
 * synchronises, so all of them may be captured into a hipGraph. The expert
 * cache entry points (wisp_core_*, wisp_cache_*) are host-side: they allocate,
 * copy and synchronise where stated and run between graph replays, as the
 * reference's paging step does.
 *
 * Return value: WISP_OK (0) on success; WISP_EINVAL (-1) when an argument
 * precondition fails (the reference raises AssertionError for the same
 * cases); WISP_EALIGN (-2) when a pointer or row stride is not aligned for the
 * vector loads; a positive value is a hipError_t from the launch.
 * wisp_last_error() gives a message for the last failure on the calling
 * thread.
 *
 * Expert buffer layout (reference wisp/quant.py:1-8, docs/architecture.md:72-82):
 *   one expert = gate [I,H] | up [I,H] | down [H,I], flat as [3, n], n = H*I
 *   bits < 16 : [ codes 3n*bits/8 B | fp16 scales 3n/G | fp16 mins 3n/G ]
 *   w = q * s + m per group of G consecutive flat elements.
 * Slot pool: nslots rows of slot_bytes (>= the expert size), row-contiguous;
 * expert in slot s starts at pool + s*slot_bytes (reference kernels.py:39).
 * Routing meta: float32 [2k] on the device = [slot ids as float ..., weights ...]
 * (reference kernels.py:189-190).
 */
#ifndef WISP_HIP_H
#define WISP_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WISP_OK 0
#define WISP_EINVAL (-1)
#define WISP_EALIGN (-2)

#define WISP_ABI_VERSION 2

/* Float types of x and of the layer output (the reference kernels take any
 * float x and return x.dtype, wisp/kernels.py:132-137, 196-203, 315-322). */
#define WISP_DT_BF16 0
#define WISP_DT_F16 1
#define WISP_DT_F32 2

/* Largest k (experts per token) the decode entry points take. */
#define WISP_MAX_K 8192

/* ABI version of the loaded library (WISP_ABI_VERSION). No reference
 * counterpart: lets a binding check it loaded the library it was written for. */
int wisp_abi_version(void);

/* Message for the last non-zero return on the calling thread ("" if none). */
const char* wisp_last_error(void);

/* Size in bytes of one quantized expert; -1 if (n, bits, group) is invalid.
 * Replaces wisp/quant.py:17-22 (expert_nbytes). */
int64_t wisp_expert_nbytes(int64_t n, int bits, int64_t group);

/* Bytes of the activation workspace `act` used between the two decode
 * kernels: k*I*4 (same size as the reference's fp32 `a` [k, I],
 * wisp/kernels.py:197). */
int64_t wisp_act_bytes(int k, int64_t I);

/* RTN min-max group quantization of one expert, w3 [3n] -> nbytes.
 * w_dtype 0 = float32, 1 = bfloat16 (converted exactly to float32 first).
 * bits in {8,4,3,2}. Bit-exact with wisp/quant.py:60-73 (quantize). */
int wisp_quantize(const void* w3, int w_dtype, int64_t n, int bits, int64_t group, uint8_t* out, void* stream);

/* Pack nq codes (< 2^bits) into nq*bits/8 bytes / unpack them back.
 * Replaces wisp/quant.py:25-41 (_pack) and 44-57 (_unpack). */
int wisp_pack(const uint8_t* q, int64_t nq, int bits, uint8_t* out, void* stream);
int wisp_unpack(const uint8_t* packed, int64_t nq, int bits, uint8_t* out, void* stream);

/* Dequantize nrows experts to bf16: out [nrows, 3n] (bf16 bit patterns).
 * Row r is read at rows + idx(r)*row_stride, idx(r) = row_index[r] (device
 * int64, may be NULL for idx(r) = r). nbound: rows available at `rows`
 * (row_index entries outside [0, nbound) produce NaN rows, no read).
 * Bit-exact with wisp/quant.py:76-87 (dequant) and therefore with
 * quant.py:94-111 (dequant_fast); with row_index it is
 * wisp/cache.py:121-135 (weights_batched: index_select + dequant). */
int wisp_dequant(const uint8_t* rows, int64_t row_stride, const int64_t* row_index, int64_t nrows, int64_t nbound,
                 int64_t n, int bits, int64_t group, uint16_t* out, void* stream);

/* Kernel 1 of a batch-1 MoE layer: for each of the k experts in meta and each
 * row r < I, a[j,r] = silu(Wg_j[r].x) * (Wu_j[r].x), fp32 accumulation,
 * written to the workspace `act` (wisp_act_bytes(k, I) bytes: a as fp32 in
 * the order a[j*I + r], the reference's fp32 `a`; wisp_act_read copies it
 * out). x: H values of type x_dtype (WISP_DT_BF16, WISP_DT_F16 or
 * WISP_DT_F32; every product of a code with x is exact), 16-byte aligned.
 * bits in {4,3,2}; 1 <= k <= WISP_MAX_K.
 * Replaces wisp/kernels.py:20-69 (_gate_up_kernel, 4-bit) and 220-263
 * (_gate_up_kernel3, 3-bit); the 2-bit variant has no reference kernel. */
int wisp_moe_gate_up(const uint8_t* pool, int64_t slot_bytes, int64_t nslots, const float* meta, int k,
                     const void* x, int x_dtype, int64_t H, int64_t I, int bits, int64_t group, uint32_t* act,
                     void* stream);

/* Kernel 2, weighted sum: out[h] = sum_{j=0..k-1} w_j * (Wd_j[h].a_j), fp32,
 * experts reduced in order, rounded once (to nearest even) to out_dtype
 * (WISP_DT_BF16, WISP_DT_F16 or WISP_DT_F32). Replaces
 * wisp/kernels.py:140-185 (_down_sum_kernel) and 266-307 (_down_sum_kernel3). */
int wisp_moe_down_sum(const uint8_t* pool, int64_t slot_bytes, int64_t nslots, const float* meta, int k,
                      const uint32_t* act, int64_t H, int64_t I, int bits, int64_t group, void* out, int out_dtype,
                      void* stream);

/* Kernel 2, per expert: y[j,h] = Wd_j[h].a_j (fp32 [k, H]).
 * Replaces wisp/kernels.py:72-112 (_down_kernel). */
int wisp_moe_down(const uint8_t* pool, int64_t slot_bytes, int64_t nslots, const float* meta, int k,
                  const uint32_t* act, int64_t H, int64_t I, int bits, int64_t group, float* y, void* stream);

/* Both kernels of one layer (gate_up, then down_sum) on `stream`.
 * Replaces wisp/kernels.py:188-203 (moe_decode_q4_fast) and 310-322
 * (moe_decode_q3_fast), which return x.dtype: pass out_dtype = x_dtype.
 * act: caller-owned workspace of wisp_act_bytes(k, I). */
int wisp_moe_decode(const uint8_t* pool, int64_t slot_bytes, int64_t nslots, const float* meta, int k,
                    const void* x, int x_dtype, int64_t H, int64_t I, int bits, int64_t group, uint32_t* act,
                    void* out, int out_dtype, void* stream);

/* Largest k*I of wisp_moe_decode_noalloc (its activation scratch: 1 MiB). */
#define WISP_NOALLOC_MAX_ACT 262144

/* wisp_moe_decode without the caller's `act` workspace, allocating nothing:
 * the activation between the two kernels lives in a 1 MiB array of device
 * memory inside the library (a file-scope __device__ array; each GPU the
 * library runs on holds its own copy until the process ends). No reference
 * counterpart: for callers that cannot allocate (code under graph capture
 * that may not call hipMalloc, tight serving loops, harnesses that forbid
 * allocation). Refuses k*I > WISP_NOALLOC_MAX_ACT (WISP_EINVAL). The stream
 * must belong to the current device. Every call on one GPU shares that GPU's
 * scratch: calls that overlap in time on one GPU (different streams) race;
 * calls in one stream are ordered. Nothing in the scratch needs clearing:
 * kernel 1 writes every value kernel 2 reads. Same results as
 * wisp_moe_decode (the same kernels). */
int wisp_moe_decode_noalloc(const uint8_t* pool, int64_t slot_bytes, int64_t nslots, const float* meta, int k,
                            const void* x, int x_dtype, int64_t H, int64_t I, int bits, int64_t group, void* out,
                            int out_dtype, void* stream);

/* Rotary embedding of one decode token, q and k heads in one launch:
 * out[i] = x[i]*cos[i] + sign(i)*x[(i + d/2) mod d]*sin[i], sign = -1 for
 * i < d/2, else +1; binary32 products and sum rounded separately, one
 * rounding to the output type. q: hq heads of d elements at q_head_stride
 * elements apart (unit element stride); k likewise (hk heads, may be 0);
 * cos, sin: d elements; qo [hq, d], ko [hk, d] contiguous. dtype 0 = float32,
 * 1 = bfloat16 (all tensors). Replaces wisp/kernels.py:325-371 (rope_decode). */
int wisp_rope_decode(const void* q, int64_t q_head_stride, const void* k, int64_t k_head_stride, const void* cos,
                     const void* sin, int hq, int hk, int d, int dtype, void* qo, void* ko, void* stream);

/* Workspace bytes of wisp_attn_decode: hq * ceil(tmax/64) * (2 + d) * 4. */
int64_t wisp_attn_ws_bytes(int hq, int d, int tmax);

/* Grouped-query attention of one decode token over a static KV cache:
 * o[h] = sum_{t <= *pos} softmax_t(scale * q[h].k[h/G][t]) v[h/G][t], G = hq/hk.
 * q: bf16 [hq, d] contiguous; kc, vc: bf16, KV head j's [tmax, d] rows start
 * at j*kv_head_stride elements; pos: device int64 (read when the kernels run,
 * so a captured graph follows it); ws: wisp_attn_ws_bytes; out: bf16 [hq, d].
 * fp32 scores (exact bf16 products), fp32 softmax and sum, bf16 store.
 * d in {64, 128, 256}, G in {1, 2, 4, 8} (and 16 at d = 128). Two launches.
 * Replaces the masked grouped scaled_dot_product_attention of
 * wisp/graphdec.py:171-174. */
int wisp_attn_decode(const uint16_t* q, const uint16_t* kc, const uint16_t* vc, int64_t kv_head_stride,
                     const int64_t* pos, int hq, int hk, int d, int tmax, float scale, void* ws, uint16_t* out,
                     void* stream);
/* graphdec.py:163-174 at batch 1 in one pair of launches: wisp_dl_qk_rope's per-head
 * RMSNorm of the q and k heads of qkv = [q (hq*d) | k (hk*d) | v (hk*d)], rope at *pos,
 * k and v stored into kc/vc at *pos, then wisp_attn_decode of those q heads; the same
 * bits as the two calls in sequence (the q heads never leave the attention workgroups).
 * Same shapes, alignment and workspace as wisp_attn_decode. */
int wisp_attn_decode_qk(const uint16_t* qkv, const uint16_t* q_norm_w, const uint16_t* k_norm_w, float eps,
                        const uint16_t* cos, const uint16_t* sin, const int64_t* pos, int hq, int hk, int d,
                        uint16_t* kc, uint16_t* vc, int64_t kv_head_stride, int tmax, float scale, void* ws,
                        uint16_t* out, void* stream);

/* Workspace bytes of wisp_moe_prefill: act bf16 [pairs, I] (rounded up to 256)
 * followed by y fp32 [pairs, H]. */
int64_t wisp_prefill_ws_bytes(int64_t pairs, int64_t H, int64_t I);

/* Grouped MoE prefill: for the (token, expert) pairs of a chunk of T tokens,
 * sorted by expert, every routed expert's token group runs gate/up + SiLU*up
 * and down as bf16 MFMA GEMMs on weight tiles dequantized (bit-exactly) in
 * registers from slot-pool rows; y = w * down(...) per pair in fp32; per token
 * s[t] = sum of its pairs' y in ascending expert id (fp32).
 * groups: device int32 [ngroups][3] = (slot, first pair, pair count);
 * max_group: the largest pair count (sets the launch shape; results do not
 * depend on it);
 * tok/w: device int32 / float [pairs] token and routing weight of each pair;
 * back: device int32 [T][k], the pair of token t's j-th expert (ascending id),
 * -1 if that expert is not in this call; x: bf16 [T, H]; ws:
 * wisp_prefill_ws_bytes(pairs, H, I), 256-byte aligned. out: bf16 [T, H] =
 * bf16(s) (8-byte aligned), or, when acc (fp32 [T, H], 16-byte aligned) is
 * not NULL, acc += s and out unused. group must be 128; H a multiple of 256,
 * I of 128; 1 <= k <= 32; bits 4/3/2. An invalid slot id
 * makes its pairs' outputs NaN. Replaces the per-expert dequant + F.linear of
 * wisp/moe.py:131-137 (three launches for all routed experts). */
int wisp_moe_prefill(const uint8_t* pool, int64_t slot_bytes, int64_t nslots, const int32_t* groups, int ngroups,
                     int max_group, const int32_t* tok, const float* w, const int32_t* back, int64_t pairs, const uint16_t* x, int T,
                     int k, int64_t H, int64_t I, int bits, int64_t group, void* ws, uint16_t* out, float* acc,
                     void* stream);

/* ---------------------------------------------------------------------------
 * Expert cache bookkeeping (host only, no device calls). Keys are
 * layer*n_experts + expert; slots [0, n_static) are the static region.
 * policy 0 = lru, 1 = wsa (decayed frequency), 2 = static. Arithmetic is
 * binary64 in the reference's order, so slot choices are identical.
 * Replaces wisp/cache_core.py:15-149 (CacheCore).
 * ------------------------------------------------------------------------- */
int wisp_core_create(int64_t nslots, int policy, double decay, int64_t n_static, double admit_after, void** out);
void wisp_core_destroy(void* core);
/* cache_core.py:30-37 (step), 39-45 (note), 47-48 (norm_freq), 54-55 (lookup: -1 if absent) */
void wisp_core_step(void* core);
void wisp_core_note(void* core, const int64_t* keys, int64_t n);
double wisp_core_norm_freq(void* core, int64_t key);
int64_t wisp_core_lookup(void* core, int64_t key);
/* cache_core.py:87-106 (ensure): slots[n] aligned with keys; the (key, slot)
 * pairs to load in load_keys/load_slots[*nloads] (capacity n). WISP_EINVAL if
 * no slot is evictable (the reference's RuntimeError). */
int wisp_core_ensure(void* core, const int64_t* keys, int64_t n, int64_t* slots, int64_t* load_keys,
                     int64_t* load_slots, int64_t* nloads);
/* cache_core.py:108-123 (split): hits and misses, nothing loaded */
int wisp_core_split(void* core, const int64_t* keys, int64_t n, int64_t* hit_keys, int64_t* hit_slots, int64_t* nhit,
                    int64_t* miss_keys, int64_t* nmiss);
/* cache_core.py:64-84 (acquire) and 125-132 (admit: slot, or -1) */
int wisp_core_acquire(void* core, int64_t key, const int64_t* prot, int64_t nprot, int64_t* slot);
int64_t wisp_core_admit(void* core, int64_t key, const int64_t* prot, int64_t nprot);
/* cache_core.py:57-62 (preload into the static region) */
int wisp_core_preload(void* core, const int64_t* keys, int64_t n);
/* cache_core.py:135-149 (resized): a new core in *out keeping the hottest
 * keys; the (key, new slot) pairs to copy in keys/slots[*n] (capacity nslots). */
int wisp_core_resized(void* core, int64_t nslots, void** out, int64_t* keys, int64_t* slots, int64_t* n);
/* Inspection: s[11] = nslots, policy, n_static, tick, hits, misses,
 * evictions, calls, nfree, nresident, nfreq; d[3] = decay, admit_after, inc.
 * Arrays (any may be NULL): slot_key/last/score [nslots], free [nfree] (next
 * slot handed out last), freq keys/values [nfreq] in first-use order. */
void wisp_core_state(void* core, int64_t* s, double* d);
void wisp_core_arrays(void* core, int64_t* slot_key, double* last, double* score, int64_t* free_list,
                      int64_t* freq_keys, double* freq_vals);

/* ---------------------------------------------------------------------------
 * Expert cache: a hipMalloc slot pool [nslots, slot_bytes] filled from a host
 * store (pinned rows of row_bytes, caller-owned, outliving the cache) by
 * hipMemcpyAsync on a side stream of default priority. Replaces
 * wisp/cache.py:9-162 (ExpertCache). The cache takes ownership of `core`.
 * decode_on_load: quantized rows are staged and dequantized once into bf16
 * slots (slot_bytes = 3n*2), cache.py:25-37, 62-71.
 * ------------------------------------------------------------------------- */
int wisp_cache_create(void* core, int64_t slot_bytes, const uint8_t* host, int64_t host_rows, int64_t row_bytes,
                      int bits, int64_t n, int64_t group, int decode_on_load, int64_t staging_rows, int device,
                      void** out);
void wisp_cache_destroy(void* cache);
void* wisp_cache_core(void* cache);
void* wisp_cache_pool(void* cache);
void* wisp_cache_copy_stream(void* cache);
void wisp_cache_counters(void* cache, int64_t* bytes_h2d, int64_t* n_loads);
/* A DLManagedTensor* (DLPack) viewing the pool as uint8 [nslots, slot_bytes]
 * on the ROCm device; the view keeps the pool memory alive. A view never
 * handed to a consumer is released with wisp_cache_pool_dlpack_free. */
void* wisp_cache_pool_dlpack(void* cache);
void wisp_cache_pool_dlpack_free(void* managed);
/* cache.py:50-76 (_issue): copies of host row keys[i] into slots[i] on the
 * side stream, ordered after the work queued on `compute`. */
int wisp_cache_issue(void* cache, const int64_t* keys, const int64_t* slots, int64_t n, void* compute);
/* cache.py:78-81 (sync_compute): `compute` waits for the issued copies. */
int wisp_cache_sync_compute(void* cache, void* compute);
/* cache.py:87-91 (ensure): residency, copies, ordering, in one call. */
int wisp_cache_ensure(void* cache, const int64_t* keys, int64_t n, int64_t* slots, void* compute);
/* One layer's host step of the graph decoder (graphdec.py:216-231): ensure the
 * k routed keys, write [slots | weights] into meta_host (pinned float32 [2k])
 * and copy it to meta_dev on `compute`. slots (may be NULL) receives the slots. */
int wisp_cache_prepare_layer(void* cache, const int64_t* keys, const float* weights, int k, float* meta_host,
                             float* meta_dev, int64_t* slots, void* compute);

/* graphdec.py:216-231 and :305-306 for one layer including the router row: copy
 * row_dev = float32 [ids (k) | weights (k)] (device) into the pinned row_host on
 * `compute` and wait for it (the decoder's one sync per layer), then
 * wisp_cache_prepare_layer with keys key_base + id, every id in [0, n_ids)
 * (else WISP_EINVAL). ids (may be NULL) replaces the row's expert ids; the
 * weights always come from the row. */
int wisp_cache_prepare_row(void* cache, const float* row_dev, float* row_host, int k, int64_t key_base,
                           int64_t n_ids, const int64_t* ids, float* meta_host, float* meta_dev, int64_t* slots,
                           void* compute);

/* wisp_cache_prepare_row for a row that the GPU writes into row_host itself
 * (wisp_dl_route with host_row/host_flag): wait until *flag != flag_before
 * (spinning, at most timeout_ms, then WISP_EINVAL), then as prepare_row.
 * In copy mode 1 the misses' page kernel runs on `compute` and also writes
 * meta_dev, so no copy-stream events or meta copy are needed; in mode 0 the
 * copies and the meta copy are those of prepare_layer. *flag_after receives
 * the flag value seen. */
int wisp_cache_prepare_signaled(void* cache, float* row_host, const volatile uint32_t* flag, uint32_t flag_before,
                                uint32_t* flag_after, int timeout_ms, int k, int64_t key_base, int64_t n_ids,
                                const int64_t* ids, float* meta_host, float* meta_dev, void* compute);

/* How misses cross PCIe: mode 0 (default) = one hipMemcpyAsync per expert row
 * on the side stream (cache.py:56-60, the DMA engines); mode 1 = a page kernel
 * on the side stream that reads the pinned store rows over PCIe (one launch per
 * 16 rows; MI355X: 53-56 GB/s for 4+ rows against 46-47 GB/s). Mode 1 needs a
 * store mapped for the device (hipHostGetDevicePointer succeeds), 16-byte rows
 * and no decode_on_load; otherwise WISP_EINVAL and the mode is unchanged. No
 * reference counterpart (the reference always uses tensor copies). */
int wisp_cache_set_copy_mode(void* cache, int mode);
/* cache.py:144-158 (resize): synchronises the device, keeps the hottest
 * experts, releases the old pool, allocates the new one, re-copies. */
int wisp_cache_resize(void* cache, int64_t nslots);

/* Device paging: the graph decoder's per-layer paging point (graphdec.py:216-231:
 * route row -> CacheCore.ensure -> copies of the misses -> meta) on the GPU, so
 * a captured decode step needs no host decision between layers. The bookkeeping
 * is cache_core.py:30-106 with any policy (the clock and its 1e100
 * renormalisation, decayed frequencies and scores, ticks per step, hits
 * protected, free slots in ascending order, then the first-index argmin of
 * `last` (lru) or `score` (wsa, static) over the unprotected dynamic slots),
 * kept in device memory while device paging is on. No reference counterpart as
 * an interface (the reference decides on the host).
 *
 * begin: copy the core's state to the device, ordered on `stream` after the
 * copies already issued. Needs copy mode 1, nslots - n_static <= 26880 (the
 * step holds every dynamic slot's eviction key in registers: one wave up to
 * 1024 slots, else up to 15 waves of 28 keys per thread), nslots <= 2^20, the
 * free slots at the top of the pool (as the core hands them out) and every
 * resident or noted key in the store; WISP_EINVAL otherwise. A no-op when
 * device paging is on.
 * While it is on, wisp_cache_issue / _ensure / _prepare_* / _resize return
 * WISP_EINVAL (the host core is stale until _sync or _end). */
int wisp_cache_device_begin(void* cache, void* stream);
/* One layer on `stream`, capturable (no host sync, no allocation): keys =
 * key_base + id_j, id_j = ids[j] (device int64 [k]) if ids and ids[j] >= 0, else row[j] (row:
 * device float32 [ids (k) | weights (k)], e.g. wisp_dl_route's row; an id must
 * be an integer in [0, n_ids)); meta (device float32 [2k]) = [slots | row's
 * weights]; the misses are paged by a kernel reading the pinned store. A bad id
 * or a miss with no evictable slot gets slot -1 (the MoE kernels then write NaN
 * rows) and is reported by the next _sync / _end. 1 <= k <= 16; k = 0 launches
 * both kernels without a step (a warm-up before capture). */
int wisp_cache_device_step(void* cache, const float* row, const int64_t* ids, int64_t key_base, int64_t n_ids,
                           int k, float* meta, void* stream);
/* wisp_dl_route (softmax of the bf16 logits [E], top-k, renormalised if norm_topk,
 * bf16 weights; row = [ids | weights]) and wisp_cache_device_step on that choice
 * (ids, if given, replace the chosen expert ids where >= 0; the weights are the router's)
 * in one launch, then the page kernel: the step's state reads overlap the
 * router's softmax and top-k. E <= 1024; k as for wisp_cache_device_step
 * (k = 0: warm-up launches). */
int wisp_cache_device_route_step(void* cache, const uint16_t* logits, int E, int k, int norm_topk, float* row,
                                 const int64_t* ids, int64_t key_base, int64_t n_ids, float* meta, void* stream);
/* Synchronise `stream` and copy the device state into the host core (keys first
 * noted on the device join its frequency table in the order of their first
 * notes) and the load counters; device paging stays on. WISP_EINVAL (once) if a
 * step since the last sync met a bad id or had no evictable slot. */
int wisp_cache_device_sync(void* cache, void* stream);
/* wisp_cache_device_sync, then device paging off. The device state stays allocated
 * at the same address (until the cache is destroyed or a begin finds a different
 * slot count), so steps captured in a graph stay valid across end / begin; a
 * captured step replayed while device paging is off does no step and writes
 * slot -1 into meta. */
int wisp_cache_device_end(void* cache, void* stream);
/* 1 while device paging is on, else 0. */
int wisp_cache_device_active(void* cache);

/* ---------------------------------------------------------------------------
 * gpt-oss experts (wisp/gptoss.py). An expert is gate_up [H, 2I] (gate/up
 * interleaved on the output axis) and down [I, H], input-major, stored in the
 * flat [3, n] slot layout [gate_up.flat[:n] | gate_up.flat[n:] | down.flat]
 * (gptoss.py:32-37), plus bf16 biases gate_up_bias [E, 2I], down_bias [E, H]
 * indexed by expert id.
 * ------------------------------------------------------------------------- */
/* gptoss.py:22-29 (mxfp4_to_bf16): blocks [ngroups, 16] uint8 (two e2m1 codes
 * per byte, low nibble first), scales [ngroups] uint8 (exponent, bias 127) ->
 * out bf16 [ngroups * 32], bit-exact with the reference's float32 product and
 * .to(bfloat16) (NaN -> 0x7FC0). blocks and out 16-byte aligned. */
int wisp_mxfp4_to_bf16(const uint8_t* blocks, const uint8_t* scales, int64_t ngroups, uint16_t* out, void* stream);

/* Bytes of the wisp_gptoss_decode workspace (fp32 partial sums). */
int64_t wisp_gptoss_ws_bytes(int k, int64_t H, int64_t I);

/* gptoss.py:126-131 (PagedGptOssBlock.forward, decode N == 1): for the k routed
 * experts, gu = x @ W_gu + gate_up_bias[e], the clamped SwiGLU
 * act = (clamp(up, -limit, limit) + 1) * gate * sigmoid(alpha * gate) with
 * gate = min(gu[2i], limit), up = gu[2i+1], o = act @ W_d + down_bias[e], and
 * out = sum_j w_j * o_j, with bf16 weights (bit-exact dequant) and the
 * reference's bf16 rounding of every intermediate tensor (fp32 products and
 * sums). meta = float32 [slot ids (k) | weights (k) | expert ids (k)] on the
 * device (read at run time, so graphs follow it); an invalid slot or expert id
 * makes the output NaN. bits 4/3/2; H % 32 == 0, I % 16 == 0, group % 32 == 0;
 * pool and slot_bytes aligned as for wisp_moe_decode; x 4-byte, ws 16-byte
 * aligned, ws of wisp_gptoss_ws_bytes(k, H, I). Three launches. */
int wisp_gptoss_decode(const uint8_t* pool, int64_t slot_bytes, int64_t nslots, const float* meta, int k, int64_t H,
                       int64_t I, int bits, int64_t group, const uint16_t* x, const uint16_t* gate_up_bias,
                       const uint16_t* down_bias, int64_t n_experts, float alpha, float limit, void* ws,
                       uint16_t* out, void* stream);

/* ---- dense part of a graph-decoder step (csrc/decode_layer.hip) ----
 * These replace the transformers modules that wisp/graphdec.py:160-203 runs at
 * batch 1 (Qwen3MoeRMSNorm, the bf16 nn.Linear q/k/v/o and router layers, the
 * residual adds, q_norm/k_norm + rope_decode + the KV store, route()), with the
 * modules' bf16 rounding points. All vectors bf16 unless stated; everything is
 * caller-owned and only enqueued on `stream` (graph-capture safe). */

/* y[o] = bf16(W[o] . x), W bf16 [O, K] row-major as up to three row blocks
 * (w0: rows [0, r1), w1: [r1, r2), w2: [r2, O); one launch for q/k/v).
 * norm_w == NULL: x = a. norm_w != NULL: h = a (+ b if b), bf16 add;
 * x = bf16(norm_w * bf16(h * rsqrt(sum(h^2)/K + eps))) (Qwen3MoeRMSNorm);
 * h_out / x_out (optional) receive h and x. a_row (optional, device int64):
 * a is a [*, K] table and its row *a_row is used (embedding lookup).
 * res (optional): y = bf16(res + bf16(W x)). K a multiple of 8 up to 8192;
 * a, b, norm_w, h_out, x_out and the weights 16-byte aligned.
 * Replaces graphdec.py:160-181 (input_layernorm, q/k/v_proj, o_proj + residual,
 * post_attention_layernorm, gate) and :195-203 (embed_tokens, norm, lm_head). */
int wisp_dl_gemv(const void* a, const int64_t* a_row, const void* b, const void* norm_w, float eps, void* h_out,
                 void* x_out, const void* w0, const void* w1, const void* w2, int64_t r1, int64_t r2, int64_t O,
                 int64_t K, const void* res, void* y, void* stream);

/* qkv = [q (hq*d) | k (hk*d) | v (hk*d)]: each q/k head RMSNorm'd over d with
 * q_norm_w / k_norm_w (as above), rotated by rope_decode's rule with the bf16
 * tables cos/sin [tmax, d] at row *pos (device int64); q -> qo [hq*d], k and v
 * -> kc/vc [hk, tmax, d] (head stride head_stride elements) at position *pos.
 * d in {64, 128, 256}. Replaces graphdec.py:163-172. */
int wisp_dl_qk_rope(const void* qkv, const void* q_norm_w, const void* k_norm_w, float eps, const void* cos,
                    const void* sin, const int64_t* pos, int hq, int hk, int d, void* kc, void* vc,
                    int64_t head_stride, void* qo, void* stream);

/* route() at batch 1 (wisp/moe.py:41-47) plus pack_meta's order: softmax in
 * float32 of the bf16 logits [E], top-k (descending, equal values by lower
 * index), divided by their sum if norm_topk, rounded to bf16; row (float32)
 * = [ids (k) | weights (k)]. E <= 1024, k <= 16. One launch.
 * host_row / host_flag (optional, together; pinned host memory) also receive
 * the row and then host_flag = ++*seq (seq: a device uint32), written with
 * system-scope stores in that order, so the host can wait for the row by
 * watching host_flag (graphdec.py:305's sync without a stream sync). */
int wisp_dl_route(const void* logits, int E, int k, int norm_topk, float* row, float* host_row, uint32_t* host_flag,
                  uint32_t* seq, void* stream);

/* Launch-shape tuning, process-wide: gu_rows = rows of one expert per wave in
 * kernel 1, gu_waves = waves per workgroup in kernel 1, dn_iters = row
 * iterations per workgroup in kernel 2 (each in {1,2,4,8}; 0 keeps the
 * current value; kernel 1 supports the pairs (4,4) (2,4) (8,4) (1,4) (4,2)
 * (2,8) (4,1) (8,1)). Defaults (2, 4, 4). No reference counterpart: the
 * reference's block_* keyword arguments are Triton tiling knobs of its own
 * kernels (wisp/kernels.py:115, 188, 310). */
int wisp_set_tuning(int gu_rows, int gu_waves, int dn_iters);

/* Copy the workspace written by wisp_moe_gate_up (fp32 a [k, I]) into a.
 * No reference counterpart (the reference's `a` is its own fp32 tensor);
 * used by tests to check kernel 1 on its own. `bits` is checked (4, 3 or 2)
 * but does not change the layout. */
int wisp_act_read(const uint32_t* act, int k, int64_t I, int bits, float* a, void* stream);

/* ------------------------------------------------------------------------
 * Measurement probes (no reference counterpart): the floors the decode
 * kernels are measured against (bench.py --workload floor). Not used by the
 * product path.
 * ------------------------------------------------------------------------ */

/* An empty kernel (one wave): the cost of one launch inside a graph. */
int wisp_probe_empty(void* stream);

/* The GPU's constant-rate real-time counter (s_memrealtime) written to *dst
 * (device uint64, 8-byte aligned) by one lane when the kernel runs: two of
 * them captured in a graph around a run of steps time exactly those steps on
 * the GPU's clock (bench.py). */
int wisp_probe_stamp(uint64_t* dst, void* stream);

/* A plain streaming read of `bytes` (a multiple of 16) from base with 16-byte
 * non-temporal loads over `workgroups` workgroups of 256 threads; nothing is
 * written to `sink` (a device buffer of `workgroups` uint32, kept so the loads
 * are not removed). With `slot` non-null (device float), the read starts at
 * base + s*stride, s = *slot when it is an integer in [0, nslots), else 0:
 * the caller guarantees base + (nslots-1)*stride + bytes is in bounds. */
int wisp_probe_read(const uint8_t* base, const float* slot, int64_t stride, int64_t nslots, int64_t bytes,
                    int workgroups, uint32_t* sink, void* stream);

/* The C2 layer's skeleton: every data movement of the two decode kernels
 * without their arithmetic. Reads gu_bytes from the (slot-selected, as in
 * wisp_probe_read) base over 768 workgroups and writes act (device float
 * [6144]); then reads the next dn_bytes over 512 workgroups, stages all of
 * act in LDS and writes out (device uint16 [2048]). one_launch = 0: as two
 * launches (the layer's structure); 1: as one launch whose 512 consuming
 * workgroups wait at a grid barrier, with `sync` a zeroed, 256-byte aligned
 * device buffer of wisp_probe_skeleton_sync_bytes() bytes kept between
 * calls; a nonzero uint32 at its last 256-byte line (byte offset
 * wisp_probe_skeleton_sync_bytes() - 256) means a bounded wait gave up.
 * EINVAL when the 768 workgroups cannot all be resident. gu_bytes <=
 * 25,165,824 and dn_bytes <= 8,388,608, multiples of 16. */
int wisp_probe_skeleton(const uint8_t* base, const float* slot, int64_t stride, int64_t nslots, int64_t gu_bytes,
                        int64_t dn_bytes, float* act, uint16_t* out, void* sync, int one_launch, void* stream);
int64_t wisp_probe_skeleton_sync_bytes(void);

#ifdef __cplusplus
}
#endif

#endif /* WISP_HIP_H */
