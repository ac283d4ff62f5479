/*
 * wisp_hip.h -- C ABI of the MI355X (gfx950) fused group-wise expert
 * dequant+GEMV path.
 *
 * Plain pointers, sizes and a stream handle; no torch types. Every device
 * pointer is a HIP device address; `stream` is a hipStream_t passed as void*
 * (NULL = the default stream). Entry points are asynchronous: they enqueue
 * kernels on `stream` and return; none allocates, frees or synchronises, so
 * all of them may be captured into a hipGraph.
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

#define WISP_ABI_VERSION 1

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
 * written to the workspace `act` (wisp_act_bytes(k, I) bytes, internal
 * layout; wisp_act_read decodes it). x: H bf16 values. bits in {4,3,2}.
 * Replaces wisp/kernels.py:20-69 (_gate_up_kernel, 4-bit) and 220-263
 * (_gate_up_kernel3, 3-bit); the 2-bit variant has no reference kernel. */
int wisp_moe_gate_up(const uint8_t* pool, int64_t slot_bytes, int64_t nslots, const float* meta, int k,
                     const uint16_t* x, int64_t H, int64_t I, int bits, int64_t group, uint32_t* act, void* stream);

/* Kernel 2, weighted sum: out[h] = sum_{j=0..k-1} w_j * (Wd_j[h].a_j), fp32,
 * experts reduced in order, stored once as bf16. Replaces
 * wisp/kernels.py:140-185 (_down_sum_kernel) and 266-307 (_down_sum_kernel3). */
int wisp_moe_down_sum(const uint8_t* pool, int64_t slot_bytes, int64_t nslots, const float* meta, int k,
                      const uint32_t* act, int64_t H, int64_t I, int bits, int64_t group, uint16_t* out,
                      void* stream);

/* Kernel 2, per expert: y[j,h] = Wd_j[h].a_j (fp32 [k, H]).
 * Replaces wisp/kernels.py:72-112 (_down_kernel). */
int wisp_moe_down(const uint8_t* pool, int64_t slot_bytes, int64_t nslots, const float* meta, int k,
                  const uint32_t* act, int64_t H, int64_t I, int bits, int64_t group, float* y, void* stream);

/* Both kernels of one layer (gate_up, then down_sum) on `stream`.
 * Replaces wisp/kernels.py:188-203 (moe_decode_q4_fast) and 310-322
 * (moe_decode_q3_fast). act: caller-owned workspace of wisp_act_bytes(k, I). */
int wisp_moe_decode(const uint8_t* pool, int64_t slot_bytes, int64_t nslots, const float* meta, int k,
                    const uint16_t* x, int64_t H, int64_t I, int bits, int64_t group, uint32_t* act, uint16_t* out,
                    void* stream);

/* Rotary embedding of one decode token, q and k heads in one launch:
 * out[i] = x[i]*cos[i] + sign(i)*x[(i + d/2) mod d]*sin[i], sign = -1 for
 * i < d/2, else +1; binary32 products and sum rounded separately, one
 * rounding to the output type. q: hq heads of d elements at q_head_stride
 * elements apart (unit element stride); k likewise (hk heads, may be 0);
 * cos, sin: d elements; qo [hq, d], ko [hk, d] contiguous. dtype 0 = float32,
 * 1 = bfloat16 (all tensors). Replaces wisp/kernels.py:325-371 (rope_decode). */
int wisp_rope_decode(const void* q, int64_t q_head_stride, const void* k, int64_t k_head_stride, const void* cos,
                     const void* sin, int hq, int hk, int d, int dtype, void* qo, void* ko, void* stream);

/* Launch-shape tuning, process-wide: gu_rows = rows of one expert per wave in
 * kernel 1, gu_waves = waves per workgroup in kernel 1, dn_iters = row
 * iterations per workgroup in kernel 2 (each in {1,2,4,8}; 0 keeps the
 * current value; kernel 1 supports the pairs (4,4) (2,4) (8,4) (1,4) (4,2)
 * (2,8) (4,1) (8,1)). Defaults (2, 4, 4). No reference counterpart: the
 * reference's block_* keyword arguments are Triton tiling knobs of its own
 * kernels (wisp/kernels.py:115, 188, 310). */
int wisp_set_tuning(int gu_rows, int gu_waves, int dn_iters);

/* Decode the workspace written by wisp_moe_gate_up into fp32 a [k, I].
 * No reference counterpart (the reference's `a` is already fp32); used by
 * tests to check kernel 1 on its own. */
int wisp_act_read(const uint32_t* act, int k, int64_t I, int bits, float* a, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* WISP_HIP_H */
