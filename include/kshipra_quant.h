/*
 * kshipra_quant.h -- C ABI of the MI355X (gfx950) weight-only quantized
 * linear path: symmetric per-output-channel INT8 and symmetric per-group INT4
 * quantize/pack, dequantize, and the fused dequant-matmul.
 *
 * Each entry point replaces one function of Kshipra's engine/quantization.py
 * (cited per declaration).  Conventions shared by every entry point:
 *
 *  - All pointers are device pointers (HIP global memory) owned by the caller;
 *    the library never allocates or frees them.  Matrices are row-major with
 *    an explicit leading dimension in elements.
 *  - fp16 values (scales) travel as their IEEE binary16 bit patterns (uint16).
 *  - `stream` is a hipStream_t (NULL = the legacy default stream).  Work is
 *    enqueued on it; no entry point synchronises the host.
 *  - Return value: KQ_OK, or an error code with a message retrievable through
 *    kq_last_error() (per calling thread).  Argument errors are detected on
 *    the host before any launch.  No C++ exception crosses this boundary.
 */
#ifndef KSHIPRA_QUANT_H
#define KSHIPRA_QUANT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* kq_stream_t; /* hipStream_t */

enum kq_status {
  KQ_OK = 0,
  KQ_ERR_ARG = 1,         /* bad shape / dtype / group size / alignment: maps to QuantizationError */
  KQ_ERR_HIP = 2,         /* a HIP runtime error: maps to RuntimeError */
  KQ_ERR_WORKSPACE = 3    /* workspace missing or too small */
};

enum kq_dtype { KQ_F32 = 0, KQ_F16 = 1, KQ_BF16 = 2 };

/* ABI version (major * 100 + minor); bump on any signature change. */
int kq_version(void);

/* Message for the last non-OK status returned on this thread. */
const char* kq_last_error(void);

/* Replaces the finiteness pass of _validate_weight, engine/quantization.py:187.
 * Sets *nonfinite_flag (device int32) to 1 if any w[r, c] (r < n, c < k) is
 * NaN or +-inf, else to 0. */
int kq_check_finite(const void* w, int w_dtype, int64_t n, int64_t k, int64_t ldw,
                    int32_t* nonfinite_flag, kq_stream_t stream);

/* Replaces quantize_int8_per_channel, engine/quantization.py:196-223.
 * w: [n, k] (ldw) of w_dtype.  payload: int8 [n, k] contiguous.  scales: fp16
 * bits [n].  Bit-exact with the reference: s = fp16(max(|w_r| / 127, 1e-8)),
 * q = clamp(rint(w / float(s)), -127, 127), NaN -> 0.  *nonfinite_flag is set
 * as by kq_check_finite (the caller discards the outputs when it is 1). */
int kq_quantize_int8(const void* w, int w_dtype, int64_t n, int64_t k, int64_t ldw,
                     int8_t* payload, uint16_t* scales, int32_t* nonfinite_flag,
                     kq_stream_t stream);

/* Replaces quantize_int4_per_group, engine/quantization.py:238-318.
 * group_size: positive and even.  k_padded = ceil(k / group_size) * group_size.
 * payload: uint8 [n, k_padded / 2] (low nibble = even column).  scales: fp16
 * bits [n, k_padded / group_size].  Columns k..k_padded-1 are zero padding. */
int kq_quantize_int4(const void* w, int w_dtype, int64_t n, int64_t k, int64_t ldw,
                     int64_t group_size, uint8_t* payload, uint16_t* scales,
                     int32_t* nonfinite_flag, kq_stream_t stream);

/* Replaces _dequantize_int8_per_channel (engine/quantization.py:226-230) and
 * the cast of QuantizedWeight.dequantize (:161-172).  out: [n, k] contiguous
 * of out_dtype; the exact fp32 product q * s rounded to out_dtype (RNE). */
int kq_dequantize_int8(const int8_t* payload, const uint16_t* scales, int64_t n, int64_t k,
                       void* out, int out_dtype, kq_stream_t stream);

/* Replaces _dequantize_int4_per_group (engine/quantization.py:321-344) and the
 * cast of :172.  out: [n, k] contiguous (the padding is sliced off). */
int kq_dequantize_int4(const uint8_t* payload, const uint16_t* scales, int64_t n, int64_t k,
                       int64_t group_size, int64_t k_padded, void* out, int out_dtype,
                       kq_stream_t stream);

/* Workspace (device bytes) that kq_linear_int8 / kq_linear_int4 need for
 * these sizes; 0 when none.  scheme: 8 or 4. */
size_t kq_linear_workspace_bytes(int scheme, int64_t m, int64_t n, int64_t k, int64_t group_size);

/* Replaces QuantizedLinear.forward for scheme "int8" (engine/quantization.py:
 * 394-396 over the payload of :196-223): y[m, n] = sum_k x[m, k] * q[n, k] *
 * s[n] + bias[n], fp32 in and out, fp32 accumulation.  x: [m, k] (ldx),
 * y: [m, n] (ldy), bias: [n] or NULL.  workspace: at least
 * kq_linear_workspace_bytes(8, ...) bytes (may be NULL when that is 0). */
int kq_linear_int8(const float* x, int64_t m, int64_t ldx, const int8_t* payload,
                   const uint16_t* scales, const float* bias, float* y, int64_t ldy,
                   int64_t n, int64_t k, void* workspace, size_t workspace_bytes,
                   kq_stream_t stream);

/* Replaces QuantizedLinear.forward for scheme "int4" (engine/quantization.py:
 * 394-396 over the payload of :238-318): y[m, n] = sum_k x[m, k] * q[n, k] *
 * s[n, k / group_size] + bias[n] over the first k columns. */
int kq_linear_int4(const float* x, int64_t m, int64_t ldx, const uint8_t* payload,
                   const uint16_t* scales, int64_t group_size, int64_t k_padded,
                   const float* bias, float* y, int64_t ldy, int64_t n, int64_t k,
                   void* workspace, size_t workspace_bytes, kq_stream_t stream);

/* Device scratch the no-allocation entry point below holds per GPU. */
#define KQ_NOALLOC_SCRATCH_BYTES (32u << 20)

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): kq_linear_int4 with the same arguments and results, but
 * no workspace argument -- the scratch it needs (at most
 * KQ_NOALLOC_SCRATCH_BYTES; larger shapes return KQ_ERR_WORKSPACE without
 * launching) is a static device array of the library, one per GPU, held
 * until the process ends.  Calls nothing that allocates.  Call it with the
 * stream's device current.  Calls that overlap on one GPU share that array
 * and race: order them on one stream or synchronise between them. */
int kq_linear_int4_noalloc(const float* x, int64_t m, int64_t ldx, const uint8_t* payload,
                           const uint16_t* scales, int64_t group_size, int64_t k_padded,
                           const float* bias, float* y, int64_t ldy, int64_t n, int64_t k,
                           kq_stream_t stream);

/* Workspace bytes for kq_linear_argmax_int8 / _int4 with these sizes (host
 * only; scheme 8 or 4). */
size_t kq_linear_argmax_workspace_bytes(int scheme, int64_t m, int64_t n, int64_t k,
                                        int64_t group_size);

/* Quantized vocab projection + greedy token (engine/model.py:151 computes the
 * logits, :187 and :200 take int(logits[0, -1].argmax())): the same sum as
 * kq_linear_int8, then tokens[r] = first index of the maximum of row r
 * (a NaN counts as the maximum, as torch.argmax).  logits: [m, n] (ldl) or
 * NULL to skip writing them; tokens: int64 [m].  m <= 65535, n < 2^31.
 * workspace: at least kq_linear_argmax_workspace_bytes(8, ...) bytes. */
int kq_linear_argmax_int8(const float* x, int64_t m, int64_t ldx, const int8_t* payload,
                          const uint16_t* scales, const float* bias, float* logits,
                          int64_t ldl, int64_t n, int64_t k, int64_t* tokens, void* workspace,
                          size_t workspace_bytes, kq_stream_t stream);

/* As kq_linear_argmax_int8 over the INT4 payload (engine/model.py:151,187,200
 * with the projection of kq_linear_int4). */
int kq_linear_argmax_int4(const float* x, int64_t m, int64_t ldx, const uint8_t* payload,
                          const uint16_t* scales, int64_t group_size, int64_t k_padded,
                          const float* bias, float* logits, int64_t ldl, int64_t n, int64_t k,
                          int64_t* tokens, void* workspace, size_t workspace_bytes,
                          kq_stream_t stream);

/* Workspace bytes for kq_linear_silu_mul_int8 / _int4 with these sizes
 * (host only; nh = gate / up out_features). */
size_t kq_linear_silu_mul_workspace_bytes(int scheme, int64_t m, int64_t nh, int64_t k,
                                          int64_t group_size);

/* The MLP input of the decoder layer (engine/model.py:147 runs layer.mlp, the
 * HF MLP down_proj(act_fn(gate_proj(x)) * up_proj(x)) whose gate_proj and
 * up_proj are QuantizedLinear after engine/model.py:80-91):
 * act[m, j] = silu(g) * u with g, u the kq_linear_int8 sums of gate row j and
 * up row j (silu(v) = v / (1 + exp(-v))).  payload / scales / bias hold the
 * two weights interleaved by 16-row tiles (rows 32 b .. 32 b + 15: gate rows
 * 16 b .., the next 16: the same up rows; 2 nh rows); nh % 16 == 0.
 * act: [m, nh] (ldact).  workspace: at least
 * kq_linear_silu_mul_workspace_bytes(8, ...) bytes. */
int kq_linear_silu_mul_int8(const float* x, int64_t m, int64_t ldx, const int8_t* payload,
                            const uint16_t* scales, const float* bias, float* act,
                            int64_t ldact, int64_t nh, int64_t k, void* workspace,
                            size_t workspace_bytes, kq_stream_t stream);

/* As kq_linear_silu_mul_int8 over interleaved INT4 payload and group scales
 * (the projections of kq_linear_int4; engine/model.py:147). */
int kq_linear_silu_mul_int4(const float* x, int64_t m, int64_t ldx, const uint8_t* payload,
                            const uint16_t* scales, int64_t group_size, int64_t k_padded,
                            const float* bias, float* act, int64_t ldact, int64_t nh, int64_t k,
                            void* workspace, size_t workspace_bytes, kq_stream_t stream);

/* ---- Paged K/V pool and chunked attention (fp32) -------------------------
 * Pool element (block, head, offset, d) of one layer's K (or V) half is at
 * pool[block * pool_ld_blk + head * pool_ld_head + offset * pool_ld_off + d]
 * (d contiguous): for Kshipra's pool [num_blocks, layers, 2, H_kv, B, D] the
 * layer-i K half pool[:, i, 0] has strides (layers*2*H_kv*B*D, B*D, D).
 * Pointers 16-byte aligned, strides multiples of 4 elements. */

/* Replaces the K/V store loop of KshipraModel.forward, engine/model.py:124-129:
 * for every t < tokens with 0 <= slot_mapping[t] < num_blocks * block_size,
 * K / V element (t, head, d) -- k[t * src_ld_tok + head * src_ld_head + d] --
 * goes to (slot / block_size, head, slot % block_size, d) of k_pool / v_pool.
 * Negative slots are skipped; non-negative slots must be distinct (the Python
 * mirror keeps the last writer of a repeated slot, as the reference loop does,
 * by passing -1 for the earlier ones).  slot_mapping: device int64 [tokens]. */
int kq_paged_kv_write_f32(const float* k, const float* v, int64_t tokens, int64_t kv_heads,
                          int64_t head_dim, int64_t src_ld_tok, int64_t src_ld_head,
                          const int64_t* slot_mapping, float* k_pool, float* v_pool,
                          int64_t num_blocks, int64_t block_size, int64_t pool_ld_blk,
                          int64_t pool_ld_head, int64_t pool_ld_off, kq_stream_t stream);

/* Workspace of kq_chunked_attention_f32 in bytes (0: none needed; 0 also for
 * invalid shapes, which the entry point then rejects). */
size_t kq_chunked_attention_workspace_bytes(int64_t q_heads, int64_t kv_heads, int64_t chunk_len,
                                            int64_t head_dim, int64_t prefix_len);

/* Replaces chunked_attention, engine/chunked_prefill.py:93-140.
 * q element (h, i, d) at q[h * q_ld_head + i * q_ld_tok + d], h < q_heads,
 * i < chunk_len; out likewise (out_ld_head, out_ld_tok).  Query i sits at
 * position prefix_len + i and attends, with scale 1/sqrt(head_dim) and the
 * online softmax, to keys 0 .. prefix_len + i of KV head h / (q_heads /
 * kv_heads); key position p lives in block block_table[p / block_size] at
 * offset p % block_size.  head_dim 64 or 128; q_heads % kv_heads == 0;
 * table_len >= ceil((prefix_len + chunk_len) / block_size); block_table is
 * device int32, entries in [0, num_blocks) (an entry outside is read as block
 * num_blocks - 1: memory-safe, result unspecified).  fp32 throughout. */
int kq_chunked_attention_f32(const float* q, int64_t q_heads, int64_t chunk_len, int64_t head_dim,
                             int64_t q_ld_head, int64_t q_ld_tok, const float* k_pool,
                             const float* v_pool, int64_t kv_heads, int64_t num_blocks,
                             int64_t block_size, int64_t pool_ld_blk, int64_t pool_ld_head,
                             int64_t pool_ld_off, const int32_t* block_table, int64_t table_len,
                             int64_t prefix_len, float* out, int64_t out_ld_head,
                             int64_t out_ld_tok, void* workspace, size_t workspace_bytes,
                             kq_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* KSHIPRA_QUANT_H */
