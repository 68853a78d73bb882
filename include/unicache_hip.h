/*
 * unicache_hip.h -- C ABI of libunicache_hip.so, the MI355X (gfx950) kernels
 * behind UniCache's physical KV-cache engine (KIVI pack, packed attention,
 * H2O selection and GQA compaction).
 *
 * Conventions shared by every entry point
 *  - Every pointer argument is a device pointer unless the comment says
 *    otherwise.  Sizes and strides are int64 element counts (not bytes).
 *  - Tensors named "dense" are token-major [tokens, heads, head_dim] as in
 *    UniCache (physical.py:242-246).  Packed KIVI tensors have the shapes of
 *    the kernel-native layout of kivi_cuda.py:177-182,
 *        key_code   int32 [Hkv, D, T*bits/32]   (codes LSB-first along tokens)
 *        key_scale  fp16  [Hkv, D, T/G]          key_min likewise
 *        value_code int32 [Hkv, T, D*bits/32]   (codes LSB-first along channels)
 *        value_scale fp16 [Hkv, T, D/G]          value_min likewise
 *    but are stored token-major in memory, each head's rows C tokens apart
 *    (C = the packed capacity, >= T, a multiple of G; C = T when tight):
 *        key_code   element (h, d, w) at h*(C*bits/32)*D + w*D + d
 *        key_scale  element (h, d, g) at h*(C/G)*D + g*D + d
 *        value_code element (h, t, w) at h*C*(D*bits/32) + t*(D*bits/32) + w
 *        value_scale element (h, t, g) at h*C*(D/G) + t*(D/G) + g
 *    so a token range of one head is one contiguous run of every tensor and a
 *    cache can grow by whole rows.  The pack/dequant entry points take explicit
 *    strides (any layout, including UniCache's non-native "reference" layout,
 *    physical.py:291-304); the attention entry points take this layout.
 *  - The library never allocates or frees device memory and never
 *    synchronises: callers own every output and workspace, and all work is
 *    enqueued on the hipStream_t passed as `stream` (NULL = default stream).
 *  - Return value: UC_OK (0), UC_EINVAL (-1, bad shape/bits/group: Python
 *    maps it to ValueError) or UC_ERUNTIME (-2, layout or HIP launch error:
 *    RuntimeError).  uc_last_error() returns the calling thread's message.
 */
#ifndef UNICACHE_HIP_H
#define UNICACHE_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define UC_ABI_VERSION 3

/* element type codes */
#define UC_BF16 0
#define UC_FP16 1
#define UC_FP32 2

/* return codes */
#define UC_OK 0
#define UC_EINVAL (-1)
#define UC_ERUNTIME (-2)

/* uc_workspace_bytes() operation codes */
#define UC_OP_KIVI_AV 2
#define UC_OP_H2O_SCORES 3

/* hipStream_t, kept opaque so the header needs no HIP include */
typedef void *uc_stream_t;

/* Version of this header the library was built from (UC_ABI_VERSION). */
int uc_abi_version(void);

/* Thread-local description of the last error ("" after a success). */
const char *uc_last_error(void);

/*
 * KIVI quantize + pack of one dense K/V segment.
 * Replaces: quant.new_pack.triton_quantize_and_pack_along_last_dim as called by
 * quantize_kivi_native (kivi_cuda.py:157-190) and, through the stride
 * arguments, _quantize_grouped / _pack_codes (physical.py:66-85, 139-175).
 * Arithmetic (fp32 throughout): mn/mx over each group, scale =
 * max((mx-mn)/(2^b-1), FLT_EPSILON), code = clamp(rint((x-mn)/scale)),
 * scale/mn stored as `stats_dtype` (round to nearest even).
 * Keys are grouped along tokens, values along channels (KIVI).
 *   key, value: dense [tokens, heads, head_dim] of `in_dtype`, strides (st,sh,sd)
 *   k_bits, v_bits in {2,4,8}; 8-bit codes are stored one per byte (uint8).
 *   group_size in {16,32,64,128}; tokens % group_size == 0,
 *   head_dim % group_size == 0.
 *   key_code element (h,d,w) at kc_sh*h + kc_sd*d + kc_sw*w (w = word, or
 *   token when k_bits==8); key stats (h,d,g) at ks_sh*h + ks_sd*d + ks_sg*g.
 *   value_code (h,t,w) at vc_sh*h + vc_st*t + vc_sw*w; value stats (h,t,g) at
 *   vs_sh*h + vs_st*t + vs_sg*g.
 */
int uc_kivi_pack(const void *key, int64_t k_st, int64_t k_sh, int64_t k_sd,
                 const void *value, int64_t v_st, int64_t v_sh, int64_t v_sd,
                 int in_dtype, int64_t tokens, int64_t heads, int64_t head_dim,
                 int k_bits, int v_bits, int group_size, int stats_dtype,
                 void *key_code, int64_t kc_sh, int64_t kc_sd, int64_t kc_sw,
                 void *key_scale, void *key_min, int64_t ks_sh, int64_t ks_sd, int64_t ks_sg,
                 void *value_code, int64_t vc_sh, int64_t vc_st, int64_t vc_sw,
                 void *value_scale, void *value_min, int64_t vs_sh, int64_t vs_st, int64_t vs_sg,
                 uc_stream_t stream);

/*
 * Dequantize tokens [start, stop) of a packed segment into dense outputs
 * out_key/out_value [n, heads, head_dim] (strides o_st,o_sh,o_sd) beginning at
 * row `output_offset`.  Bit-exact with PackedKIVICache.dequantize:
 * fp32 code*scale, then +min (two roundings, physical.py:190-201), then a
 * round-to-nearest-even cast to `out_dtype`.
 * Replaces: _dequantize_kv_chunk_kernel / dequantize_kv_chunk_tiled
 * (kivi_triton.py:385-502, 690-770) behind dequantize_kivi_chunk
 * (kivi_cuda.py:58-93), and the full dequantize (physical.py:379-423).
 * Code/stat strides follow uc_kivi_pack.  Either key_code or value_code may be
 * NULL to restore only the other tensor.
 */
int uc_kivi_dequant(const void *key_code, int64_t kc_sh, int64_t kc_sd, int64_t kc_sw,
                    const void *key_scale, const void *key_min, int64_t ks_sh, int64_t ks_sd, int64_t ks_sg,
                    const void *value_code, int64_t vc_sh, int64_t vc_st, int64_t vc_sw,
                    const void *value_scale, const void *value_min, int64_t vs_sh, int64_t vs_st, int64_t vs_sg,
                    int stats_dtype, int64_t heads, int64_t head_dim,
                    int k_bits, int v_bits, int group_size, int64_t start, int64_t stop,
                    void *out_key, void *out_value, int out_dtype,
                    int64_t o_st, int64_t o_sh, int64_t o_sd, int64_t output_offset,
                    uc_stream_t stream);

/*
 * KIVI fake quantization (quantize then dequantize, no packing) of a dense
 * [tokens, heads, head_dim] tensor, grouped along `dim` (0 = tokens for keys,
 * 2 = channels for values), written to `out` (same strides as the input).
 * Arithmetic of asymmetric_fake_quant (operators/builtin.py:31-53):
 * scale = max(mx-mn, FLT_EPSILON)/(2^b-1), out = code*scale + mn.
 * Groups are min(group_size, length) wide; the last one may be partial.
 * Replaces: kivi_fake_quant_key / kivi_fake_quant_value (builtin.py:56-65).
 */
int uc_kivi_fake_quant(const void *data, int64_t st, int64_t sh, int64_t sd,
                       int dtype, int64_t tokens, int64_t heads, int64_t head_dim,
                       int bits, int dim, int group_size,
                       void *out, uc_stream_t stream);

/*
 * Scaled logits over a packed segment plus its dense residual:
 *   logits[hq, i, t] = sm_scale * <query[i, hq, :], K[t, hq / group, :]>
 * for t < quantized_tokens from the packed keys (token-major with capacity
 * packed_capacity, 0 meaning quantized_tokens; see the top of this file)
 * and t >= quantized_tokens from the dense residual_key, element (t, h, d) at
 * r_st*t + r_sh*h + d.  logits is fp32 [Hq, Lq, Tq+Tr] (contiguous).  With
 * quantized_tokens == 0 this is the dense GQA QK of gqa_query_key_logits
 * (physical.py:20-39).
 * Replaces: the KIVI GEMV QK (cuda_bmm_fA_qB_outer, kivi_cuda.py:257-266),
 * packed_qk_tiled (kivi_triton.py:505-556) and the residual logits, concat and
 * 1/sqrt(D) scaling of packed_kivi_attention_parts (kivi_cuda.py:283-287).
 * bits in {2,4,8}; 8 uses UniCache's uint8 layout (codes [Tq,Hkv,D],
 * stats [Tq/G,Hkv,D] of stats_dtype).
 */
int uc_kivi_qk(const void *query, int q_dtype, int64_t query_len, int64_t heads_q,
               const void *key_code, const void *key_scale, const void *key_min, int stats_dtype,
               int64_t quantized_tokens, int64_t packed_capacity, int bits, int group_size,
               const void *residual_key, int res_dtype, int64_t residual_tokens,
               int64_t r_st, int64_t r_sh,
               int64_t heads_kv, int64_t head_dim, float sm_scale,
               float *logits, uc_stream_t stream);

/*
 * Probability-value product over a packed segment plus its residual:
 *   out[hq, i, :] = sum_t probs[hq, i, t] * V[t, hq / group, :]
 * packed values with capacity packed_capacity (0: quantized_tokens);
 * probs [Hq, Lq, Tq+Tr] of p_dtype with strides (p_sh, p_si, p_st); out is
 * [Hq, Lq, D] of out_dtype (contiguous); residual_value element (t, h, d) at
 * r_st*t + r_sh*h + d.  `workspace` must hold
 * uc_workspace_bytes(UC_OP_KIVI_AV, ...) bytes.  With quantized_tokens == 0
 * this is gqa_probability_value (physical.py:42-63); there, with 16-bit values
 * and >= 64 query rows per KV head, the MFMA path rounds P to the value dtype
 * first, as physical.py:59 does (the other paths multiply fp32 P).
 * Replaces: the KIVI GEMV AV (kivi_cuda.py:295-307), packed_av_tiled
 * (kivi_triton.py:559-612) and the residual AV + sum (kivi_cuda.py:324-327).
 */
int uc_kivi_av(const void *probs, int p_dtype, int64_t p_sh, int64_t p_si, int64_t p_st,
               int64_t query_len, int64_t heads_q,
               const void *value_code, const void *value_scale, const void *value_min, int stats_dtype,
               int64_t quantized_tokens, int64_t packed_capacity, int bits, int group_size,
               const void *residual_value, int res_dtype, int64_t residual_tokens,
               int64_t r_st, int64_t r_sh,
               int64_t heads_kv, int64_t head_dim,
               void *out, int out_dtype, void *workspace, uc_stream_t stream);

/*
 * One packed KIVI segment (native layout, contiguous) with its residual, and
 * the query/outputs of one attention call over it.  Used by the decode entry
 * points; a table of these lets one launch cover many sequences and layers.
 */
typedef struct uc_kivi_item {
  const void *key_code;      /* int32 [Hkv, D, Tq*bits/32], token-major (see the top of this file) */
  const void *key_scale;     /* fp16  [Hkv, D, Tq/G], token-major */
  const void *key_min;
  const void *value_code;    /* int32 [Hkv, Tq, D*bits/32] */
  const void *value_scale;   /* fp16  [Hkv, Tq, D/G] */
  const void *value_min;
  const void *residual_key;  /* [Tr, Hkv, D] of res_dtype, may be NULL if Tr==0 */
  const void *residual_value;
  const void *query;         /* [Lq, Hq, D] of q_dtype */
  void *out;                 /* [Lq, Hq, D] of out_dtype, normalised */
  float *lse;                /* [Hq, Lq] natural-log LSE, may be NULL */
  int64_t quantized_tokens;  /* Tq, a multiple of group_size */
  int64_t residual_tokens;   /* Tr */
  int64_t packed_capacity;   /* C: tokens between the heads of the packed tensors; 0 means Tq */
  /* residual element (t, h, d) at residual_key + t * residual_token_stride +
   * h * residual_head_stride + d (elements, multiples of 8); 0 and 0 mean
   * token-major rows [Tr, Hkv, D] (token stride Hkv * D, head stride D).  A
   * head-major [Hkv, Tr, D] segment (a GQA H2O cache) has token stride D and
   * head stride Tr * D.  uc_kivi_residual_append needs token-major rows. */
  int64_t residual_token_stride;
  int64_t residual_head_stride;
} uc_kivi_item;

/*
 * Fused dequant attention for short queries (decode) over one packed segment
 * plus residual: out = softmax(sm_scale * q K^T) V over all Tq+Tr keys, and
 * lse = log sum_t exp(sm_scale * q.k_t).  Split-K over tokens; the splits are
 * merged with a log-sum-exp combine.  group = Hq/Hkv query heads share one KV
 * head; group*query_len <= 16.
 * Replaces: the decode use of packed_kivi_attention_parts (kivi_cuda.py:238-329)
 * followed by the caller's softmax and AV (adapters/bagel.py:1205-1297), and
 * packed_kivi_quantized_attention_summary (kivi_cuda.py:96-120) for Lq small.
 * `workspace` must hold uc_kivi_decode_workspace_bytes(1, ...) bytes.
 * head_dim 128 with bits 2/4 and group 32/64/128 runs the MFMA kernel; other
 * shapes a generic split-K kernel.  The MFMA kernel takes fp16 operands: query,
 * residual and dequantized values must stay below 65504 in magnitude.
 */
int uc_kivi_attn_decode(const uc_kivi_item *item_host, int bits, int group_size,
                        int64_t heads_q, int64_t heads_kv, int64_t head_dim, int64_t query_len,
                        int q_dtype, int res_dtype, int out_dtype, float sm_scale,
                        void *workspace, int64_t workspace_bytes, uc_stream_t stream);

/*
 * uc_kivi_attn_decode without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No reference counterpart.  The split
 * partials go to a fixed scratch array inside the library, one per GPU, of
 * uc_kivi_decode_scratch_bytes() bytes (8 MiB: a 2-bit head_dim-128 segment of
 * about 400k tokens at 4 KV heads); a call that would need more returns
 * UC_EINVAL.  The call allocates nothing.  Every call on one GPU shares that
 * GPU's scratch: calls that overlap on one GPU (different streams or host
 * threads without ordering) race and give wrong results.  The device current
 * on the calling thread must be the one that owns the item's tensors and
 * `stream`.  Results equal uc_kivi_attn_decode's bit for bit.
 */
int uc_kivi_attn_decode_static(const uc_kivi_item *item_host, int bits, int group_size,
                               int64_t heads_q, int64_t heads_kv, int64_t head_dim, int64_t query_len,
                               int q_dtype, int res_dtype, int out_dtype, float sm_scale, uc_stream_t stream);

/* Size in bytes of the scratch array behind uc_kivi_attn_decode_static. */
int64_t uc_kivi_decode_scratch_bytes(void);

/*
 * The same kernel over `n_items` segments (sequences x layers) in one launch.
 * `items_device` is a device array of uc_kivi_item; every item shares bits,
 * group, head counts and query_len; token counts may differ, up to
 * max_quantized_tokens / max_residual_tokens.
 * Each item's query must be 16-byte aligned (rows are read as 16-byte vectors).
 * No reference counterpart: this is the all-layer decode launch.
 */
int uc_kivi_attn_decode_batch(const uc_kivi_item *items_device, int64_t n_items,
                              int bits, int group_size,
                              int64_t heads_q, int64_t heads_kv, int64_t head_dim, int64_t query_len,
                              int q_dtype, int res_dtype, int out_dtype, float sm_scale,
                              int64_t max_quantized_tokens, int64_t max_residual_tokens,
                              void *workspace, int64_t workspace_bytes, uc_stream_t stream);

/*
 * uc_kivi_attn_decode_segments for ONE query over n_items (1..8) segments
 * given in host memory: the items travel in the kernel arguments, so a call
 * copies nothing to the device (a decode step of one layer).  The group's
 * result goes to the first item's out / lse.  Workspace:
 * uc_kivi_decode_workspace_bytes(n_items, ...).  Items may give residual
 * strides (a head-major H2O segment as a dense item with quantized_tokens 0).
 * Replaces: _run_fused_mixed_attention's per-segment summaries and merge for
 * decode-length queries (adapters/bagel.py:1598-1858), without concatenating
 * the bf16 parts.
 */
int uc_kivi_attn_decode_segments_host(const uc_kivi_item *items_host, int64_t n_items, int bits, int group_size,
                                      int64_t heads_q, int64_t heads_kv, int64_t head_dim, int64_t query_len,
                                      int q_dtype, int res_dtype, int out_dtype, float sm_scale,
                                      void *workspace, int64_t workspace_bytes, uc_stream_t stream);

/*
 * Segment table: the n_items items form n_items / segments_per_query groups
 * of consecutive items that share one query (a KV cache split into segments,
 * e.g. a packed prefix and a dense bf16 segment given as an item with
 * quantized_tokens == 0).  Every group is attended as one softmax over all
 * its segments and written to its first item's out / lse; the other items'
 * out / lse are not used.  MFMA decode shapes only (head_dim 128, bits 2/4,
 * group 32/64/128, query heads per KV head * query_len <= 16).  Workspace as
 * for uc_kivi_attn_decode_batch over n_items.
 * Replaces: the per-segment summaries plus merge_attention_summaries of
 * _run_fused_mixed_attention (adapters/bagel.py:1598-1858) for decode.
 */
int uc_kivi_attn_decode_segments(const uc_kivi_item *items_device, int64_t n_items, int64_t segments_per_query,
                                 int bits, int group_size,
                                 int64_t heads_q, int64_t heads_kv, int64_t head_dim, int64_t query_len,
                                 int q_dtype, int res_dtype, int out_dtype, float sm_scale,
                                 int64_t max_quantized_tokens, int64_t max_residual_tokens,
                                 void *workspace, int64_t workspace_bytes, uc_stream_t stream);

/*
 * Attention for long queries (image editing: group*query_len rows per KV head
 * in the thousands) over one packed segment plus residual: same inputs,
 * outputs and semantics as uc_kivi_attn_decode.  head_dim 128, bits 2/4,
 * group_size 32/64/128, q and residual bf16/fp16, sm_scale > 0; the residual
 * (the dense keys) must be 16-byte aligned.  One kernel streams 64-key tiles
 * through LDS for MFMA, 128 query rows per workgroup: packed tiles are
 * dequantized from their codes into LDS inside the kernel (nothing is staged
 * in HBM), residual tiles are read where they lie.  Packed tiles take fp16
 * operands (the query and the dequantized values must stay below 65504 in
 * magnitude); residual tiles take the residual's dtype (bf16 keeps its range).
 * `workspace` is not used (uc_kivi_mq_workspace_bytes returns 0) and may be
 * NULL; the arguments stay for callers written against the staged version.
 * Replaces: _packed_attention_kernel / packed_attention_tiled
 * (kivi_triton.py:216-382, 615-687) behind packed_kivi_quantized_attention_summary
 * (kivi_cuda.py:96-120) with backend "triton_tiled", plus the residual part.
 */
int uc_kivi_attn_mq(const uc_kivi_item *item_host, int bits, int group_size,
                    int64_t heads_q, int64_t heads_kv, int64_t head_dim, int64_t query_len,
                    int q_dtype, int res_dtype, int out_dtype, float sm_scale,
                    void *workspace, int64_t workspace_bytes, uc_stream_t stream);

/* Workspace of uc_kivi_attn_mq and uc_kivi_attn_mq_batch: 0 bytes (-1 for bad arguments). */
int64_t uc_kivi_mq_workspace_bytes(int64_t heads_kv, int64_t head_dim, int64_t quantized_tokens,
                                   int64_t residual_tokens);

/*
 * uc_kivi_attn_mq over n_items (1..8) independent segments in one launch:
 * item i attends its query_lens[i] queries (item.query / item.out /
 * item.lse, laid out as in uc_kivi_attn_mq) to its own packed prefix and
 * residual.  Every item shares bits, group_size, heads, head_dim and dtypes.
 * `workspace` is not used and may be NULL.  Results equal n_items calls of
 * uc_kivi_attn_mq bit for bit.
 * Replaces: the per-sample loop of apply_static_physical_attention_batch
 * (adapters/bagel.py:773-980) for samples whose physical layout is one packed
 * KIVI segment plus dense keys (CFG branches packed with pack_naive_caches).
 */
int uc_kivi_attn_mq_batch(const uc_kivi_item *items_host, const int64_t *query_lens, int n_items,
                          int bits, int group_size, int64_t heads_q, int64_t heads_kv, int64_t head_dim,
                          int q_dtype, int res_dtype, int out_dtype, float sm_scale,
                          void *workspace, int64_t workspace_bytes, uc_stream_t stream);

/*
 * One dense 16-bit key/value segment of a segment-table call: key element
 * (token t, KV head h, channel d) at key + t * token_stride + h * head_stride
 * + d, strides in elements (multiples of 8), the same for value; key and
 * value 16-byte aligned.  [T, Hkv, D] rows: token_stride = Hkv * D,
 * head_stride = D; [Hkv, T, D] (an H2O segment): token_stride = D,
 * head_stride = T * D.
 */
typedef struct uc_dense_segment {
  const void *key;
  const void *value;
  int64_t tokens;
  int64_t token_stride;
  int64_t head_stride;
} uc_dense_segment;

/*
 * Segment table for long queries: one softmax of query [Lq, Hq, 128] over
 * the packed prefixes and residuals of `n_packed` items (their query / out /
 * lse fields are not used) and `n_dense` dense segments, in one launch with
 * no staging: out [Lq, Hq, 128] normalised, lse [Hq, Lq] natural-log (may be
 * NULL).  Limits per call: 8 packed prefixes, 16 dense segments counting the
 * items' residuals.  Shapes and dtypes as uc_kivi_attn_mq; dense_dtype is the
 * dtype of every residual and dense segment.
 * Replaces: for long queries, the concatenation of the bf16 segments, the
 * per-prefix fused summaries and merge_attention_summaries of
 * _run_fused_mixed_attention (adapters/bagel.py:1598-1858).
 */
int uc_kivi_attn_mq_segments(const uc_kivi_item *packed_host, int n_packed,
                             const uc_dense_segment *dense_host, int n_dense,
                             const void *query, void *out, float *lse,
                             int bits, int group_size, int64_t heads_q, int64_t heads_kv, int64_t head_dim,
                             int64_t query_len, int q_dtype, int dense_dtype, int out_dtype, float sm_scale,
                             uc_stream_t stream);

/*
 * One query of a multi-query table call: its query / out / lse (laid out as in
 * uc_kivi_attn_mq) and the runs of the call's packed items and dense segments
 * it attends.
 */
typedef struct uc_mq_query {
  const void *query;
  void *out;
  float *lse;
  int64_t query_len;
  int32_t packed_begin, n_packed;
  int32_t dense_begin, n_dense;
} uc_mq_query;

/*
 * uc_kivi_attn_mq_segments for up to 8 queries in one launch: query i attends,
 * as one softmax, the packed prefixes and residuals of items
 * packed_host[packed_begin .. + n_packed) and the dense segments
 * dense_host[dense_begin .. + n_dense) (runs of different queries may name the
 * same tensors).  Limits per call: 8 packed items and 16 dense segments,
 * counting each item's residual as one.  Results equal one
 * uc_kivi_attn_mq_segments call per query bit for bit.
 * Replaces: the per-sample loop of apply_static_physical_attention_batch
 * (adapters/bagel.py:773-980) for samples with long queries, whatever their
 * physical layout (CFG branches, H2O segments, several packed prefixes).
 */
int uc_kivi_attn_mq_table(const uc_mq_query *queries_host, int n_queries,
                          const uc_kivi_item *packed_host, int n_packed,
                          const uc_dense_segment *dense_host, int n_dense,
                          int bits, int group_size, int64_t heads_q, int64_t heads_kv, int64_t head_dim,
                          int q_dtype, int dense_dtype, int out_dtype, float sm_scale, uc_stream_t stream);

/*
 * Merge normalised attention summaries of n_segments disjoint key segments:
 *   lse = logsumexp_s lse_s;  out = sum_s out_s * exp(lse_s - lse)
 * outs[s] are [Lq, Hq, D] of out_dtype (contiguous), lses[s] fp32 [Hq, Lq].
 * `outs` and `lses` are HOST arrays of n_segments device pointers
 * (n_segments <= 16).  out_lse may be NULL.
 * Replaces: merge_attention_summaries (adapters/bagel.py:57-72).
 */
int uc_lse_merge(const void *const *outs, const float *const *lses, int n_segments,
                 int out_dtype, int64_t query_len, int64_t heads_q, int64_t head_dim,
                 void *out, float *out_lse, uc_stream_t stream);

/*
 * H2O per-KV-head attention mass received by each key:
 *   P = bf16(softmax_t(sm_scale * q_i . k_t))   per query head and query row
 *   scores[h, t] (+)= sum_{g < group} sum_i float(P[h*group+g, i, t])
 * query [Lq, Hq, D], key [T, Hkv, D] (strides given), fp32 scores [Hkv, T]
 * contiguous.  accumulate != 0 adds to the existing scores.
 * `workspace` must hold uc_workspace_bytes(UC_OP_H2O_SCORES, ...) bytes.
 * Replaces: the softmax + bf16 cast of adapters/bagel.py:1205-1243 followed
 * by H2OPhysicalGQAOperator.update_after_attention (operators/physical.py:62-65),
 * without materialising P in HBM.
 */
int uc_h2o_scores(const void *query, int64_t q_si, int64_t q_sh, int64_t q_sd,
                  const void *key, int64_t k_st, int64_t k_sh, int64_t k_sd, int dtype,
                  int64_t query_len, int64_t heads_q, int64_t tokens, int64_t heads_kv,
                  int64_t head_dim, float sm_scale, int accumulate,
                  float *scores, void *workspace, uc_stream_t stream);

/*
 * H2O column sums of given probabilities (no softmax):
 *   out[h, t] (+)= sum_{g<group} sum_i float(probs[h*group+g, i, t])
 * probs [Hq, Lq, T] of p_dtype with strides (p_sh, p_si, p_st).
 * Replaces: GQAH2OCache.update_scores (physical.py:598-610) and the reduction of
 * operators/physical.py:62-65 when P already exists.
 */
int uc_h2o_colsum(const void *probs, int p_dtype, int64_t p_sh, int64_t p_si, int64_t p_st,
                  int64_t heads_q, int64_t query_len, int64_t tokens, int64_t heads_kv,
                  int accumulate, float *out, uc_stream_t stream);

/*
 * H2O selection per KV head: the heavy_k highest scores among tokens
 * [0, tokens - recent) (ties broken by lowest token index, NaN ranked
 * highest), written in ascending token order, followed by the recent window
 * tokens-recent .. tokens-1.  scores fp32 [Hkv, tokens] with strides
 * (s_sh, s_st); indices int64 [Hkv, heavy_k + recent] contiguous.
 * Replaces: torch.topk(...).indices.sort() + arange + cat of
 * GQAH2OCache.from_dense / trim (physical.py:511-532, 624-649).
 */
int uc_h2o_select(const float *scores, int64_t s_sh, int64_t s_st,
                  int64_t heads_kv, int64_t tokens, int64_t heavy_k, int64_t recent,
                  int64_t *indices, uc_stream_t stream);

/*
 * GQA compaction gather: for each KV head h and slot j, r = indices[h, j]:
 *   out_key[h, j, :] = key[r, h, :]      out_value likewise
 *   out_ids[h, j]    = ids[r] (ids_sh == 0) or ids[h, r] (ids_sh != 0)
 *   out_scores[h, j] = scores[h, r]
 * key/value use (k_st, k_sh, k_sd) strides; out_key/out_value are contiguous
 * [Hkv, R, D].  ids/out_ids/scores/out_scores may be NULL to skip them.
 * Replaces: the torch.gather calls of GQAH2OCache.from_dense / trim
 * (physical.py:533-546, 650-654).
 */
int uc_gqa_gather(const void *key, const void *value, int64_t k_st, int64_t k_sh, int64_t k_sd,
                  int dtype, int64_t heads_kv, int64_t head_dim,
                  const int64_t *indices, int64_t retained,
                  const int64_t *ids, int64_t ids_sh, int64_t ids_st,
                  const float *scores, int64_t s_sh, int64_t s_st,
                  void *out_key, void *out_value, int64_t *out_ids, float *out_scores,
                  uc_stream_t stream);

/*
 * uc_h2o_select followed by uc_gqa_gather in one call: selects into
 * `indices` (int64 [Hkv, heavy_k + recent], caller-owned) and gathers K, V,
 * ids and scores through them.  Scores must be the [Hkv, tokens] fp32 rows
 * that are also gathered (strides s_sh, s_st).  Same results as the two calls.
 * Replaces: the whole selection + gather of GQAH2OCache.from_dense
 * (physical.py:511-546) in one host round trip.
 */
int uc_h2o_select_gather(const void *key, const void *value, int64_t k_st, int64_t k_sh, int64_t k_sd,
                         int dtype, int64_t heads_kv, int64_t tokens, int64_t head_dim,
                         const float *scores, int64_t s_sh, int64_t s_st, int64_t heavy_k, int64_t recent,
                         const int64_t *ids, int64_t ids_sh, int64_t ids_st, int64_t *indices,
                         void *out_key, void *out_value, int64_t *out_ids, float *out_scores,
                         uc_stream_t stream);

/*
 * One H2O segment of uc_h2o_select_gather_segments: the uc_h2o_select_gather
 * arguments of one segment (rows [tokens, Hkv, D] by element strides, fp32
 * scores [Hkv, tokens], optional int64 ids, outputs [Hkv, heavy_k + recent]).
 */
typedef struct uc_h2o_segment {
  const void *key, *value;
  int64_t k_st, k_sh, k_sd;
  const float *scores;
  int64_t s_sh, s_st;
  const int64_t *ids;  /* NULL: no ids (then out_ids NULL too) */
  int64_t ids_sh, ids_st;
  int64_t tokens, heavy_k, recent;
  int64_t *indices;
  void *out_key, *out_value;
  int64_t *out_ids;
  float *out_scores;   /* NULL: the scores are not gathered */
} uc_h2o_segment;

/*
 * uc_h2o_select_gather for several segments (same dtype, KV heads and
 * head_dim) in one launch: each (segment, KV head) selects in one workgroup
 * and gathers through the indices it keeps in LDS, split over up to 16
 * workgroups per head.  Results equal one uc_h2o_select_gather per segment.
 * Up to 8 segments of 16-bit rows (16-byte aligned, strides multiples of 8
 * elements) with at most 8192 tokens share the launch; any other segment runs
 * through uc_h2o_select_gather on the same stream.
 * No reference counterpart: GQAH2OCache.from_dense (physical.py:511-546) per
 * segment is what a caller with several H2O segments (the instruction and ViT
 * segments of one materialisation, storage/tensor_backend.py) replaces.
 */
int uc_h2o_select_gather_segments(const uc_h2o_segment *segments, int n_segments, int dtype,
                                  int64_t heads_kv, int64_t head_dim, uc_stream_t stream);

/*
 * uc_h2o_scores with the softmax normaliser given instead of computed:
 *   P = bf16(exp(sm_scale * q_i . k_t - lse[h, i]))
 * lse is fp32 [Hq, Lq] (natural log), e.g. the global LSE of a mixed-segment
 * attention call; the workspace is sized as for uc_h2o_scores.
 * Replaces: the H2O update of _run_fused_mixed_attention, exp(logits -
 * global_lse).to(bf16) followed by update_scores (adapters/bagel.py:1845-1856).
 */
int uc_h2o_scores_lse(const void *query, int64_t q_si, int64_t q_sh, int64_t q_sd,
                      const void *key, int64_t k_st, int64_t k_sh, int64_t k_sd, int dtype,
                      int64_t query_len, int64_t heads_q, int64_t tokens, int64_t heads_kv,
                      int64_t head_dim, float sm_scale, const float *lse, int accumulate,
                      float *scores, void *workspace, uc_stream_t stream);

/*
 * Keep-mask compaction, step 1: for the n rows of a packed dense cache,
 *   dst_index[t] = number of kept rows before t   if keep[t] != 0
 *                = -1                             otherwise
 * and *total (device int64) = number of kept rows.  keep is one byte per row
 * (torch.bool), 16-byte aligned; n < 2^31.
 * Replaces: the per-sample boolean masks of TensorCacheStorageBackend.compact
 * (tensor_backend.py:54-77).
 */
int uc_mask_scan(const uint8_t *keep, int64_t n, int32_t *dst_index, int64_t *total, uc_stream_t stream);

/*
 * Keep-mask compaction, step 2: row t of src (row_bytes contiguous bytes at
 * t * src_row_stride_bytes) is copied to dst + dst_index[t] * row_bytes for
 * every t with dst_index[t] >= 0 (the output of uc_mask_scan).  Used for the
 * key, value and type-id rows.
 * Replaces: key[mask], value[mask], key_type_ids[mask]
 * (tensor_backend.py:66-77).
 */
int uc_compact_rows(const void *src, int64_t src_row_stride_bytes, int64_t row_bytes,
                    const int32_t *dst_index, int64_t n, void *dst, uc_stream_t stream);

/*
 * Several uc_compact_rows copies that share one dst_index (the K and V rows
 * of a compaction) in one launch.  Copies whose pointers, stride and row size
 * are not all multiples of 16 bytes, and any past the fourth, run as
 * uc_compact_rows on the same stream.
 * Replaces: key[keep] and value[keep] of TensorCacheStorageBackend.compact
 * (tensor_backend.py:66-77) as one operation.
 */
typedef struct uc_row_copy {
  const void *src;
  int64_t src_row_stride_bytes, row_bytes;
  void *dst;
} uc_row_copy;

int uc_compact_rows_multi(const uc_row_copy *copies, int n_copies, const int32_t *dst_index, int64_t n,
                          uc_stream_t stream);

/*
 * The rows KIVIQuantizationOperator.execute fake-quantizes, in one launch:
 * segment tokens (bool bytes) except the last residual_length of them and,
 * with preserve_protected, the protected ones; none with bypass.  Writes
 * dst_index [n] (row in the compact order, or -1), src_index [selected] (the
 * inverse) and counts [3] = (segment tokens, selected tokens, protected
 * segment tokens), all on the device.
 * Replaces: the mask arithmetic and counts of operators/builtin.py:394-410.
 */
int uc_fake_quant_mask(const uint8_t *segment, const uint8_t *protected_mask, int64_t n, int64_t residual_length,
                       int preserve_protected, int bypass, int32_t *dst_index, int32_t *src_index, int64_t *counts,
                       uc_stream_t stream);

/*
 * The inverse of uc_compact_rows: for every t with dst_index[t] >= 0, the
 * compact row dst_index[t] of src (row_bytes each) is copied to out + t *
 * out_row_stride_bytes; other rows of out are left as they are.
 * Replaces: the masked write-back k_out[quant_mask] = fake_quant(...) of the
 * KIVI fake-quant operator (operators/builtin.py:420-430).
 */
int uc_scatter_rows(const void *src, int64_t row_bytes, const int32_t *dst_index, int64_t n, void *out,
                    int64_t out_row_stride_bytes, uc_stream_t stream);

/*
 * Up to 8 independent device-to-device copies (span i: `bytes` bytes from src
 * to dst, non-overlapping) in one launch; 16-byte units where a span's
 * addresses and size allow.
 * Replaces: the residual clones and the logical-id clone of
 * PackedKIVICache.from_dense (physical.py:316-330), one copy kernel each.
 */
typedef struct uc_copy_span {
  const void *src;
  void *dst;
  int64_t bytes;
} uc_copy_span;

int uc_copy_spans(const uc_copy_span *spans_host, int n, uc_stream_t stream);

/*
 * Streaming decode over a device item table (as built for
 * uc_kivi_attn_decode_batch / _segments): for each entry, first move the
 * item's residual window past a flush that the caller has just packed, then
 * append n_tokens rows to it, all in place on the device:
 *   1. a = advance: quantized_tokens += a, residual_key and residual_value move
 *      a rows forward, residual_tokens -= a (the caller has packed those a
 *      rows into the packed tensors, which must have room for them);
 *   2. key[e] / value[e] (rows [n_tokens, heads_kv, head_dim] of `dtype`, entry
 *      e's block of contiguous [n_entries, n_tokens, heads_kv, head_dim]
 *      tensors) are written at residual rows residual_tokens.. and
 *      residual_tokens += n_tokens; ids[e] (int64 [n_entries, n_tokens], may be
 *      NULL) go to entries[e].ids[quantized_tokens + residual_tokens ..]
 *      (entries[e].ids may be NULL).
 * Residual rows are [Tr, heads_kv, head_dim] contiguous and 16-byte aligned
 * and must have room behind them; entries name distinct items (at most 128).
 * Decode launches enqueued later on the stream see the new lengths.  No
 * reference counterpart: UniCache builds a packed segment once
 * (physical.py:228-332); this is the decode loop's per-step append, so the
 * host neither rebuilds nor copies the item table per step.
 */
typedef struct uc_append_entry {
  int64_t item;      /* index into the item table */
  int64_t advance;   /* tokens packed by a flush since the previous call (0: none) */
  int64_t *ids;      /* device int64 logical-id buffer of the segment, or NULL */
} uc_append_entry;

int uc_kivi_residual_append(uc_kivi_item *items_device, const uc_append_entry *entries_host, int n_entries,
                            const void *key, const void *value, const int64_t *ids, int64_t n_tokens,
                            int64_t heads_kv, int64_t head_dim, int dtype, uc_stream_t stream);

/*
 * Bytes of caller-provided workspace an operation needs.
 *   UC_OP_KIVI_AV:     (1, heads_q, query_len, head_dim, total_tokens)
 *                      = max(4 Hq Lq S (D + 2), Hq Lq >= 64 ? 2 Hq D ceil64(T) : 0),
 *                      S = ceil(T / (Hq Lq <= 64 ? 64 : 512)) + 1
 *   UC_OP_H2O_SCORES:  (1, heads_q, query_len, head_dim, tokens)
 *                      = max(8 Hq Lq, 2048 (B + 768) + 4 T B),
 *                      B = ceil(Hq Lq / 256) + Hq
 * Returns < 0 for an unknown op.
 */
int64_t uc_workspace_bytes(int op, int64_t n_items, int64_t heads_q, int64_t query_len,
                           int64_t head_dim, int64_t max_tokens);

/*
 * Bytes of workspace uc_kivi_attn_decode(_batch) needs for n_items items of
 * at most max_quantized_tokens packed and max_residual_tokens residual keys.
 */
int64_t uc_kivi_decode_workspace_bytes(int64_t n_items, int bits, int group_size, int64_t heads_q,
                                       int64_t heads_kv, int64_t head_dim, int64_t query_len,
                                       int64_t max_quantized_tokens, int64_t max_residual_tokens);

#ifdef __cplusplus
}
#endif

#endif /* UNICACHE_HIP_H */
