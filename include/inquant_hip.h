/*
 * inquant_hip.h -- C ABI of libinquant_hip.so, the MI355X (gfx950) packed-KV
 * hot path of InQuant: K4 neighbor-slot codec, V2/V4 group-wise value codec,
 * incremental decode-metadata append, fused packed-KV decode attention and
 * the paged (vLLM page layout) variants.
 *
 * Conventions
 *   - Every entry point returns IQ_OK (0) or a negative status; the message
 *     of the last failure on the calling thread is iq_last_error().
 *   - All tensor arguments are raw device pointers plus element strides;
 *     streams are hipStream_t passed as void*.  Nothing here allocates
 *     device memory, synchronizes, or keeps state between calls: the caller
 *     (the Python host layer, torch-owned buffers) owns every buffer.
 *   - Work is enqueued asynchronously on `stream`.  Device-side data errors
 *     (non-finite inputs, f16 overflow) are reported through a caller-owned
 *     device int `bad_flag` that the kernel sets to 1; callers read it where
 *     the reference already synchronizes.
 *   - dtype codes: IQ_F32, IQ_BF16, IQ_F16, IQ_F64 (inputs only).
 *
 * Reference interfaces replaced (paths into the reference checkout):
 *   iq_k4_quantize      src/inquant/codec.py:181-243        quantize()
 *   iq_reuse_map        src/inquant/triton_selection.py:46-60 reuse_map(),
 *                       src/inquant/codec.py:137-178         _reuse_map()
 *   iq_k4_dequantize    src/inquant/codec.py:112-134         PackedTensor.dequantize()
 *   iq_v_quantize       src/inquant/value_codec.py:51-72     quantize_values()
 *   iq_v_dequantize     src/inquant/value_codec.py:38-48     PackedValues.dequantize()
 *   iq_kv_quantize      src/inquant/cache.py:288-295 (the paired key / value block
 *                       encodes of an append: iq_k4_quantize + iq_v_quantize)
 *   iq_k4_quantize_kv   src/inquant/cache.py:288-291 (the same with K4-coded values)
 *   iq_decode_append    src/inquant/triton_attention.py:234-309 PackedDecodeState.extend/_write_maps
 *   iq_decode_attention src/inquant/triton_attention.py:317-388 PackedDecodeState.decode
 *                       (_attention_partials :67-165 + _reduce_partials :168-181)
 *   iq_write_pages      extensions/vllm/src/inquant_vllm/packing.py:41-55 write_codec_pages
 *                       (+ the role-map part of layout.py:66-81 pack_pages)
 *   iq_encode_pages     extensions/vllm/src/inquant_vllm/layout.py:103-115 pack_pages_into
 *                       (quantize + quantize_values + write_codec_pages, one launch)
 *   iq_unpack_pages     extensions/vllm/src/inquant_vllm/layout.py:84-100 unpack_pages_reference
 *   iq_paged_decode     extensions/vllm/src/inquant_vllm/kernels.py:66-88 paged_decode
 *   iq_prefill_attention extensions/vllm/src/inquant_vllm/backend.py:139-144
 *                       (flash_attn_varlen_func, causal prefill on exact K/V)
 *   iq_tail_append      src/inquant/cache.py:256-259,283-286 (the dense tail
 *                       concatenation of append_for_attention / _append)
 */
#ifndef INQUANT_HIP_H
#define INQUANT_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define IQ_ABI_VERSION 1

enum iq_status { IQ_OK = 0, IQ_ERR_ARG = -1, IQ_ERR_DEVICE = -2, IQ_ERR_UNSUPPORTED = -3 };
enum iq_dtype { IQ_F32 = 0, IQ_BF16 = 1, IQ_F16 = 2, IQ_F64 = 3 };

/* Columns of a decode state's pointer table: the reference's six (K payload,
 * K scales, K padding, V payload, V scales, V offsets-or-padding,
 * triton_attention.py:337-340) plus the K source and donor descriptors. */
#define IQ_TABLE_COLS 8

/* Library ABI version (IQ_ABI_VERSION) and last error text of this thread. */
int iq_abi_version(void);
const char *iq_last_error(void);

/*
 * K4 neighbor-slot encode of x[B, H, T, D] (element strides x_strides[4]).
 * count = floor(D * salient_fraction) (<= D/2); sample_stride >= 1;
 * min_error != 0 selects the "min_error" donor policy, else "neighbors".
 * Outputs (contiguous): payload u8 [B,H,T,D/2]; scales f32 [B,H,D];
 * src/don [B,H,count] of desc_bytes (1 = u8, 4 = i32, 8 = i64);
 * padding f32 [B,H,count].  D even, 2 <= D <= 1024.
 * Replaces codec.py:181-243 (statistics, selection, scales, 4/8-bit slots,
 * nibble packing, padding); bit-exact with the reference's CPU torch path.
 */
int iq_k4_quantize(const void *x, int x_dtype, const int64_t *x_strides,
                   int64_t B, int64_t H, int64_t T, int64_t D,
                   int64_t count, int64_t sample_stride, int min_error,
                   uint8_t *payload, float *scales, void *src, void *don, int desc_bytes,
                   float *padding, int *bad_flag, void *stream);

/*
 * Donor selection alone: saliency (and optional donor error) f32 [rows, D]
 * contiguous -> src/don i64 [rows, count].  Replaces reuse_map /
 * _reuse_map (triton_selection.py:46-60, codec.py:137-178).
 */
int iq_reuse_map(const float *saliency, const float *donor_error, int64_t rows, int64_t D,
                 int64_t count, int64_t *src, int64_t *don, void *stream);

/*
 * K4 decode to a dense tensor: out [rows, T, D] of out_dtype (rows = B*H).
 * Replaces PackedTensor.dequantize (codec.py:112-134).
 */
int iq_k4_dequantize(const uint8_t *payload, const float *scales, const void *src, const void *don,
                     int desc_bytes, const float *padding, int64_t rows, int64_t T, int64_t D,
                     int64_t count, void *out, int out_dtype, void *stream);

/*
 * Group-wise affine value encode of x[B, H, T, D] (strides x_strides[4]):
 * bits in {2, 4}, group in {32, 64, 128}, D % group == 0.  Outputs
 * payload u8 [B,H,T,D*bits/8]; scales/offsets f16 bits [B,H,T,D/group].
 * Replaces quantize_values (value_codec.py:51-72).
 */
int iq_v_quantize(const void *x, int x_dtype, const int64_t *x_strides,
                  int64_t B, int64_t H, int64_t T, int64_t D, int bits, int group,
                  uint8_t *payload, uint16_t *scales, uint16_t *offsets, int *bad_flag, void *stream);

/*
 * Keys and values of the same blocks in one call: iq_k4_quantize of
 * keys[B, H, T, D] plus iq_v_quantize of values[B, H, T, D] (value_bits 2 or
 * 4), with the same arguments, outputs and flags as those two.  Sealed
 * blocks (T = 256, D = 128, 16-bit rows) take one launch whose workgroups
 * encode a block's values while their first wavefront makes the donor
 * picks; other shapes run the two encoders back to back.  Replaces the
 * paired block encodes of a cache append (cache.py:288-295: keys through
 * _quantize_temporal_blocks, values through quantize_value_blocks).
 */
int iq_kv_quantize(const void *keys, const void *values, int dtype, const int64_t *k_strides,
                   const int64_t *v_strides, int64_t B, int64_t H, int64_t T, int64_t D,
                   int64_t count, int64_t sample_stride, int min_error, uint8_t *k_payload,
                   float *k_scales, void *src, void *don, int desc_bytes, float *padding,
                   int value_bits, int value_group, uint8_t *v_payload, uint16_t *v_scales,
                   uint16_t *v_offsets, int *key_bad, int *value_bad, void *stream);

/*
 * Keys and values of the same blocks, both K4-coded (the cache's default
 * value_bits = None), in one call: iq_k4_quantize of keys and of values with
 * the same arguments, outputs (k_* for keys, v_* for values) and flags as two
 * calls of it.  Tile shapes (16-bit rows of D = 128, T <= 256) take one
 * launch over (B, 2 H) rows; others run the two encodes back to back.
 * Replaces the paired block encodes of an append (cache.py:288-291).
 */
int iq_k4_quantize_kv(const void *keys, const void *values, int dtype, const int64_t *k_strides,
                      const int64_t *v_strides, int64_t B, int64_t H, int64_t T, int64_t D,
                      int64_t count, int64_t sample_stride, int min_error,
                      uint8_t *k_payload, float *k_scales, void *k_src, void *k_don, float *k_padding,
                      uint8_t *v_payload, float *v_scales, void *v_src, void *v_don, float *v_padding,
                      int desc_bytes, int *key_bad, int *value_bad, void *stream);

/* Value decode: out [rows, D] of out_dtype (rows = B*H*T); value_codec.py:38-48. */
int iq_v_dequantize(const uint8_t *payload, const uint16_t *scales, const uint16_t *offsets,
                    int64_t rows, int64_t D, int bits, int group, void *out, int out_dtype, void *stream);

/*
 * One sealed block's device addresses, as recorded in the decode state's
 * pointer table (triton_attention.py:337-340), plus its descriptors.
 * v_scales/v_offsets hold the V2 scales/offsets, or for a K4-coded V its
 * scales/padding; v_src/v_don are 0 unless V is K4-coded.
 */
typedef struct iq_block_ptrs {
    uint64_t k_payload, k_scales, k_padding;
    uint64_t v_payload, v_scales, v_offsets;
    uint64_t k_src, k_don, v_src, v_don;
} iq_block_ptrs;

/*
 * Append `count` blocks to a decode state: writes tables[first + i] (i64 [cap, IQ_TABLE_COLS])
 * and the int8 role maps key_map / value_map [cap, H, 128] (value_map may be
 * NULL for V2/V4 values).  Roles: -1 normal, donor channel for a source,
 * -2 - i for donor i.  `blocks` is a HOST array; its contents travel as
 * kernel arguments (no host-to-device copy).  Replaces
 * PackedDecodeState.extend / _write_maps (triton_attention.py:234-309).
 */
int iq_decode_append(int64_t *tables, int8_t *key_map, int8_t *value_map, int64_t first, int64_t count,
                     const iq_block_ptrs *blocks, int64_t H, int64_t S, int desc_bytes, void *stream);

/*
 * The leading blocks of a decode state that sit at a fixed stride from each
 * other (the per-block views of one batched encode): block i < blocks has
 * field f (pointer-table column order: K payload, K scales, K padding,
 * V payload, V scales, V offsets, K sources, K donors) at base[f] + i * that
 * field's bytes per block (H*B*64, H*512, H*S*4, H*B*D*bits/8, H*B*(D/group)*2
 * twice, H*S, H*S).  The decode reads these blocks' addresses from the
 * kernel arguments instead of the pointer table; the table stays valid for
 * every block.
 */
typedef struct iq_block_run {
    uint64_t base[IQ_TABLE_COLS];
    int64_t blocks;
} iq_block_run;

/*
 * Fused single-query GQA decode over [sink | packed blocks | tail].
 *   q [Hq, 128] (row stride q_stride_h) of q_dtype (f32, bf16, f16);
 *   tables i64 [n_blocks, IQ_TABLE_COLS], key_map/value_map int8 [n_blocks, H, 128]
 *   (value_map used only when value_bits == 0, i.e. K4-coded V);
 *   run: optional (NULL) fixed-stride run of the leading blocks;
 *   block_tokens tokens per packed block, S salient channels per block;
 *   value_bits in {0, 2, 4}, value_group in {32, 64, 128};
 *   sink/tail K/V of q_dtype with (head, token) element strides, lengths
 *   sink_t / tail_t (pointers may be NULL when the length is 0);
 *   workspace f32 with at least iq_decode_workspace_floats(...) elements
 *   (Hq * P * 130 floats: each partition's 128-float output rows, then its
 *   (max, sum) pairs; merged by a second kernel);
 *   out [Hq, 128] contiguous of out_dtype.
 * Keys/values are decoded and rounded to q_dtype exactly as the reference's
 * dequantize-then-attend path does; logits, softmax and P.V accumulate in
 * fp32.  Replaces PackedDecodeState.decode (triton_attention.py:317-388).
 */
int64_t iq_decode_workspace_floats(int64_t Hq, int64_t n_blocks, int64_t sink_t, int64_t tail_t);

int iq_decode_attention(const void *q, int q_dtype, int64_t q_stride_h, int64_t Hq,
                        const int64_t *tables, const int8_t *key_map, const int8_t *value_map,
                        const iq_block_run *run, int64_t n_blocks, int64_t block_tokens, int64_t H, int64_t S,
                        int value_bits, int value_group,
                        const void *sink_k, const void *sink_v, int64_t sink_k_sh, int64_t sink_k_st,
                        int64_t sink_v_sh, int64_t sink_v_st, int64_t sink_t,
                        const void *tail_k, const void *tail_v, int64_t tail_k_sh, int64_t tail_k_st,
                        int64_t tail_v_sh, int64_t tail_v_st, int64_t tail_t,
                        float scale, float *workspace, int64_t workspace_floats,
                        void *out, int out_dtype, void *stream);

/*
 * The partition merge alone: out [Hq, 128] of out_dtype from the `parts`
 * partials in workspace (the layout iq_decode_attention writes: [Hq, parts]
 * 128-float rows, then [Hq, parts] (max, sum) pairs, max in natural-log
 * units).  Replaces _reduce_partials (triton_attention.py:168-181); the
 * decode calls it itself, this entry point serves callers that produce
 * partials elsewhere and the timing of the merge on its own.
 */
int iq_decode_merge(const float *workspace, int64_t parts, int64_t Hq, void *out, int out_dtype, void *stream);

/* Partitions iq_decode_attention uses for a call: the matrix-core kernel's
 * (fast != 0: blocks + ceil((sink + tail) / 32)) or the general kernel's. */
int64_t iq_decode_partitions(int64_t n_blocks, int64_t sink_t, int64_t tail_t, int fast);

/*
 * iq_decode_attention without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  The
 * partials live in a file-scope device array of IQ_NOALLOC_SCRATCH_FLOATS
 * floats (16 MiB) that each GPU holds until the process ends; a call needing
 * more (Hq * partitions * 130 floats) returns IQ_ERR_ARG.  Allocates and
 * frees nothing.  Calls that overlap on one GPU share the array and race:
 * serialize them (one stream, or events).
 */
#define IQ_NOALLOC_SCRATCH_FLOATS (4LL << 20)

int iq_decode_attention_noalloc(const void *q, int q_dtype, int64_t q_stride_h, int64_t Hq,
                                const int64_t *tables, const int8_t *key_map, const int8_t *value_map,
                                const iq_block_run *run, int64_t n_blocks, int64_t block_tokens, int64_t H, int64_t S,
                                int value_bits, int value_group,
                                const void *sink_k, const void *sink_v, int64_t sink_k_sh, int64_t sink_k_st,
                                int64_t sink_v_sh, int64_t sink_v_st, int64_t sink_t,
                                const void *tail_k, const void *tail_v, int64_t tail_k_sh, int64_t tail_k_st,
                                int64_t tail_v_sh, int64_t tail_v_st, int64_t tail_t,
                                float scale, void *out, int out_dtype, void *stream);

/*
 * ---------------------------------------------------------------- paged cache
 * Page layout of the vLLM plugin (extensions/vllm/src/inquant_vllm/layout.py:8-53),
 * field-major per page, B tokens per page, H KV heads, D = 128, 16 salient channels:
 *   key_payload u8 [H,B,64] | key_scales f32 [H,128] | key_map i16 [H,128] |
 *   key_padding f32 [H,16] | value_payload u8 [H,B,32] | value_scales f16 [H,B,2] |
 *   value_offsets f16 [H,B,2];  page bytes = H * (104 B + 832).
 * key_map: -1 normal, the donor channel for a source, -2 - j for donor j.
 * B in {64, 128, 256} as in the reference, plus 16 and 32.
 */
int64_t iq_page_bytes(int64_t H, int64_t block_tokens);

/*
 * Scatter n_pages encoded pages into the pool by physical id (ids i32 or i64
 * per id_bytes; ids outside [0, pool_pages) are skipped).  Inputs are the
 * codec outputs of [n, H, B, 128] K (K4, 16 salient channels) and V (V2, group 64):
 * k_payload [n,H,B,64], k_scales [n,H,128], k_padding [n,H,16], k_src/k_don
 * [n,H,16] of desc_bytes, v_payload [n,H,B,32], v_scales/v_offsets f16 [n,H,B,2].
 * Replaces write_codec_pages (packing.py:7-55) and the field copies and role map
 * of pack_pages (layout.py:56-81).
 */
int iq_write_pages(const uint8_t *k_payload, const float *k_scales, const float *k_padding,
                   const void *k_src, const void *k_don, int desc_bytes, const uint8_t *v_payload,
                   const uint16_t *v_scales, const uint16_t *v_offsets, int64_t n_pages, int64_t H,
                   int64_t block_tokens, uint8_t *pool, int64_t pool_pages, const void *page_ids,
                   int id_bytes, void *stream);

/*
 * Encode n_pages full pages straight into the pool, one launch: keys/values
 * [n, H, B, 128] of dtype (bf16 or f16) with element strides k_strides /
 * v_strides (unit channel stride, 16-byte aligned rows), B in {16, 32, 64,
 * 128, 256}.  Page n goes to physical id page_ids[n] (i32 or i64 per
 * id_bytes; an id outside [0, pool_pages) writes nothing and sets flags[2]):
 * K4 min_error with stride 8 and 16 salient channels (payload, scales,
 * padding and the i16 role map) and V2 with 64-channel groups.  flags[0] /
 * flags[1] are set for non-finite keys / values; the launch zeroes
 * next_flags[0..2] (the triple the caller passes as flags to its next call,
 * so no clearing launch is needed).
 * Replaces pack_pages_into (layout.py:103-115: quantize, quantize_values,
 * write_codec_pages) and the encode of pack_pages (layout.py:56-81).
 */
int iq_encode_pages(const void *keys, const void *values, int dtype, const int64_t *k_strides,
                    const int64_t *v_strides, int64_t n_pages, int64_t H, int64_t block_tokens, uint8_t *pool,
                    int64_t pool_pages, const void *page_ids, int id_bytes, int *flags, int *next_flags,
                    void *stream);

/*
 * iq_encode_pages with pages at arbitrary token rows of one key and one value
 * tensor: page n reads tokens page_rows[n] .. page_rows[n] + B - 1 (element
 * offsets page_rows[n] * k_strides[2] and page_rows[n] * v_strides[2]; the
 * page strides k_strides[0] / v_strides[0] are unused), i64 device array, or
 * NULL for iq_encode_pages' layout.  One launch seals the full pages of
 * several requests of a batch (each at its own row of the batch's key/value
 * rows, or at its own slot of a dense page buffer).  Replaces the per-request
 * pack_pages_into calls of backend.py:106-116.
 */
int iq_encode_pages_at(const void *keys, const void *values, int dtype, const int64_t *k_strides,
                       const int64_t *v_strides, const int64_t *page_rows, int64_t n_pages, int64_t H,
                       int64_t block_tokens, uint8_t *pool, int64_t pool_pages, const void *page_ids,
                       int id_bytes, int *flags, int *next_flags, void *stream);

/*
 * Decode n_pages contiguous pages to keys/values [n, H, B, 128] of out_dtype.
 * Replaces unpack_pages_reference (layout.py:84-100).
 */
int iq_unpack_pages(const uint8_t *pages, int64_t n_pages, int64_t H, int64_t block_tokens, void *keys,
                    void *values, int out_dtype, void *stream);

/* fp32 workspace elements iq_paged_decode needs: n_seq * Hq * partitions * 130
 * (128-float output rows, then (max, sum) pairs). */
int64_t iq_paged_workspace_floats(int64_t Hq, int64_t n_seq, int64_t max_pages, int64_t block_tokens);

/*
 * Fused single-query decode over paged K4/V2 history plus a dense BF16 buffer,
 * for n_seq sequences in one launch.
 *   q bf16 [n_seq, Hq, 128] (element strides q_stride_seq, q_stride_h);
 *   block_tables i32 [n_seq, bt_stride] of physical page ids (ids outside the
 *   pool contribute nothing); max_pages bounds every sequence's page count;
 *   seq_info i32 [n_seq, 3] = (pages, tail tokens, sink tokens) on the device,
 *   or NULL with n_seq == 1 and the host values n_pages, tail_t, sink_t;
 *   dense bf16 [slots, 2, H, B + 4, 128] (stride dense_stride_seq elements):
 *   rows 0..3 the sink, 4.. the current partial page (kernels.py:37-48 masks:
 *   packed tokens before the sink length and tail slots inside the sink are
 *   skipped); sequence i reads dense slot dense_slots[i] (i32 device array of
 *   in-range slots), or slot i when dense_slots is NULL;
 *   work: NULL (one workgroup per (KV head, partition, sequence) up to the
 *   longest sequence), or n_work i32 items (sequence << 16 | partition) that
 *   list every partition of every sequence (packed partitions of 256 tokens,
 *   then the dense one: seq_info's pages decide how many) in the order they
 *   should start, so that no workgroup is launched for a partition past a
 *   short sequence's end (items outside the batch do nothing);
 *   out [n_seq, Hq, 128] (stride out_stride_seq) of out_dtype.
 * Keys/values are decoded and rounded to bf16 as dequantize-then-attend does;
 * logits, softmax and P.V accumulate in fp32.  Replaces paged_decode
 * (kernels.py:66-88, _paged_partials :8-63, which handles one sequence per launch).
 */
int iq_paged_decode(const void *q, int64_t q_stride_seq, int64_t q_stride_h, int64_t Hq, int64_t n_seq,
                    const uint8_t *pool, int64_t pool_pages, int64_t H, int64_t block_tokens,
                    const int32_t *block_tables, int64_t bt_stride, int64_t max_pages,
                    const int32_t *seq_info, int64_t n_pages, int64_t tail_t, int64_t sink_t,
                    const void *dense, int64_t dense_stride_seq, const int32_t *dense_slots,
                    const int32_t *work, int64_t n_work, float scale, float *workspace,
                    int64_t workspace_floats, void *out, int64_t out_stride_seq, int out_dtype, void *stream);

/*
 * Causal self-attention over exact K/V for prefill, vLLM token-major layout:
 * q [tokens, Hq, 128], k/v [tokens, H, 128] of dtype (bf16 or f16) with
 * element strides (token, head), 16-byte aligned rows, k/v token strides
 * below 2^25 elements (IQ_ERR_ARG otherwise); sequences
 * [cu_seqlens[i], cu_seqlens[i + 1]) (i32, on the device, n_seq + 1 values),
 * none longer than max_seqlen; query i of a sequence attends to its keys
 * 0..i; out [tokens, Hq, 128] of out_dtype with strides (o_st, o_sh).  fp32
 * logits, softmax and accumulation; softmax weights rounded to the K/V dtype
 * before P.V.  Replaces flash_attn_varlen_func(..., causal=True) in the
 * plugin's prefill (extensions/vllm/src/inquant_vllm/backend.py:139-144).
 */
int iq_prefill_attention(const void *q, const void *k, const void *v, int dtype, int64_t q_st, int64_t q_sh,
                         int64_t k_st, int64_t k_sh, int64_t v_st, int64_t v_sh, const int32_t *cu_seqlens,
                         int64_t n_seq, int64_t max_seqlen, int64_t Hq, int64_t H, int64_t head_dim, float scale,
                         void *out, int64_t o_st, int64_t o_sh, int out_dtype, void *stream);

/*
 * Dense tail append of a cache layer.  buf holds [2 (keys, values), H,
 * capacity, D] elements of elem_bytes (element strides buf_kv, buf_h,
 * buf_t); k / v hold n_new (<= 64) rows per head (element strides: head,
 * token).  One launch moves rows [shift_src, shift_src + shift_count) to
 * [0, shift_count) (the rows that survive a seal), then writes the new rows
 * at [slot, slot + n_new); the three row ranges must be disjoint.  With
 * `positions` (i32 or i64 per pos_bytes, n_new values on the device) the
 * kernel compares positions[i] with expected + i and sets *flag = 1 on any
 * mismatch.  Replaces the per-token concatenation of the dense tail in
 * InQuantCache.append_for_attention / _append (cache.py:256-259,283-286).
 */
int iq_tail_append(const void *k, const void *v, int64_t k_sh, int64_t k_st, int64_t v_sh, int64_t v_st,
                   int64_t H, int64_t n_new, int64_t D, int elem_bytes, void *buf, int64_t buf_kv,
                   int64_t buf_h, int64_t buf_t, int64_t capacity, int64_t slot, int64_t shift_src,
                   int64_t shift_count, const void *positions, int pos_bytes, int64_t expected, int *flag,
                   void *stream);

/*
 * The same append of one row with the parts that stay fixed across a
 * layer's decode steps in a descriptor (built once per layer, the row
 * strides refreshed when they change), for the per-token host path: buf with
 * element strides buf_kv, buf_h, buf_t; heads; row length dim; capacity
 * rows; elem_bytes per element; flag = the int the position check sets;
 * pos_bytes = 4 or 8; k_sh, k_st, v_sh, v_st = element strides (head,
 * token) of the new key and value rows.  Equivalent to iq_tail_append(k, v,
 * k_sh, k_st, v_sh, v_st, heads, 1, dim, elem_bytes, buf, buf_kv, buf_h,
 * buf_t, capacity, slot, shift_src, shift_count, positions, pos_bytes,
 * expected, flag, stream).
 */
typedef struct iq_tail_desc {
    uint64_t buf;
    int64_t buf_kv, buf_h, buf_t, heads, dim, capacity;
    int elem_bytes, pos_bytes;
    uint64_t flag;
    int64_t k_sh, k_st, v_sh, v_st;
} iq_tail_desc;

int iq_tail_append_row(const iq_tail_desc *desc, const void *k, const void *v, int64_t slot, int64_t shift_src,
                       int64_t shift_count, const void *positions, int64_t expected, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* INQUANT_HIP_H */
