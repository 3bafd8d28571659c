/*
 * vlc_capi.h -- C ABI of the gfx950 warm partial-recompute prefill kernels.
 *
 * Every entry point takes plain pointers and sizes.  Device pointers are HIP
 * device addresses; `stream` is a hipStream_t (NULL = the null stream).  No
 * entry point allocates device memory, synchronises the host with the device,
 * or keeps mutable global state: work is enqueued on `stream` and the caller
 * owns every buffer (inputs, outputs and workspace).
 *
 * Return value: VLC_OK (0) on success, a negative VLC_ERR_* for an argument
 * the kernels do not accept (mirroring the asserts of the reference's
 * store_kvcache, layers/attention.py:36-39), or a positive hipError_t when a
 * launch fails.  vlc_status_string() names a status.
 *
 * Element type: bf16 (2-byte elements) for attention and re-rotation; the KV
 * scatter is a bit copy and also accepts 4-byte elements.
 */
#ifndef VLC_CAPI_H
#define VLC_CAPI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VLC_ABI_VERSION 1

#define VLC_OK 0
#define VLC_ERR_INVALID (-1)     /* null pointer, bad size, stride or alignment */
#define VLC_ERR_UNSUPPORTED (-2) /* a shape the kernels do not implement (e.g. a head_dim other than 128 or 80) */
#define VLC_ERR_WORKSPACE (-3)   /* workspace smaller than the plan requires */
#define VLC_ERR_CAPACITY (-4)    /* host plan buffer too small */
#define VLC_ERR_PLAN (-5)        /* plan does not match the call's shapes */
#define VLC_ERR_SCRATCH (-6)     /* the call needs more than the fixed scratch of a *_noalloc entry */

const char* vlc_status_string(int status);
int vlc_abi_version(void);

/*
 * Paged KV-cache scatter of freshly computed tokens.
 * Replaces store_kvcache / store_kvcache_kernel (layers/attention.py:10-40).
 *
 * For every token n in [0, num_tokens): slot = slot_mapping[n]; if slot < 0 the
 * token is skipped (the reference skips slot == -1, layers/attention.py:23);
 * a slot >= num_slots (rows in each cache) is skipped as well instead of being
 * written out of bounds.  Otherwise row_elems elements of key row n and value row n are copied bit for
 * bit to row `slot` of k_cache and v_cache (cache rows are contiguous, row
 * stride row_elems).  key/value rows are row_elems contiguous elements at row
 * strides key_row_stride / value_row_stride (elements): the value view that
 * the caller passes is strided (models/qwen3.py:77-80).
 * elem_bytes is 2 (bf16/fp16) or 4.
 */
int vlc_store_kvcache(const void* key, int64_t key_row_stride,
                      const void* value, int64_t value_row_stride,
                      void* k_cache, void* v_cache,
                      int64_t num_slots, const int32_t* slot_mapping, int64_t num_tokens,
                      int64_t row_elems, int elem_bytes, void* stream);

/*
 * Rotary embedding of q and k fused with the paged KV store of k and v.
 * Replaces RotaryEmbedding.forward (layers/rotary_embedding.py:37-48) followed
 * by store_kvcache (layers/attention.py:33-40), the per-layer sequence at
 * models/qwen3.py:84-85, with one launch.
 *
 * q: [num_tokens, num_heads_q, head_dim] bf16 at row stride q_row_stride; the
 *   rotated q goes to q_out (row stride q_out_row_stride; q_out == q rotates in
 *   place).  k: [num_tokens, num_heads_kv, head_dim] likewise; the rotated k goes
 *   to row slot_mapping[n] of k_cache and, when k_out != NULL, to k_out.
 *   v: rows copied bit for bit to row slot_mapping[n] of v_cache.  Heads are
 *   contiguous rows of head_dim elements inside a token row; every pointer and
 *   row stride must give 16-byte aligned rows.
 * Pair i is dims (i, i + head_dim/2) (rotate-half).  Its angle comes from the
 *   caller's fp32 cache cos_sin_cache[max_positions][cache_row_stride], whose
 *   row p holds cos of pair i at column i and sin at column head_dim/2 + i (the
 *   reference's cos_sin_cache, layers/rotary_embedding.py:30-35), at position
 *   positions[section(i) * position_row_stride + n] (int64).
 *   num_position_rows = 1: 1-D positions, section(i) = 0 for every pair.
 *   num_position_rows = 3: M-RoPE rows (t, h, w); mrope_section is a HOST
 *   int32[3] summing to head_dim/2: section(i) = 0 for i < s0, 1 for i < s0+s1,
 *   else 2.
 *   A position outside [0, max_positions) is clamped to the nearest valid row
 *   (the reference's cache indexing raises instead).
 * Arithmetic: y1 = x1*c - x2*s, y2 = x2*c + x1*s in fp32, each product and sum
 *   rounded, then rounded to bf16 (nearest even): bit-identical to the
 *   reference's fp32 formula (layers/rotary_embedding.py:6-14).
 * k_cache/v_cache: rows of num_heads_kv*head_dim elements, num_slots rows each;
 *   both NULL = rotate only (no store; v and slot_mapping may be NULL).  A slot
 *   < 0 (the reference's -1) or >= num_slots is skipped.
 * q_out must not overlap k, v or the caches; k_out must not overlap q or v.
 */
int vlc_rope_store_kvcache(const void* q, int64_t q_row_stride, void* q_out, int64_t q_out_row_stride,
                           const void* k, int64_t k_row_stride, void* k_out, int64_t k_out_row_stride,
                           const void* v, int64_t v_row_stride,
                           int num_heads_q, int num_heads_kv, int head_dim,
                           const int64_t* positions, int num_position_rows,
                           int64_t position_row_stride, const int32_t* mrope_section,
                           const float* cos_sin_cache, int64_t cache_row_stride,
                           int64_t max_positions,
                           void* k_cache, void* v_cache, int64_t num_slots,
                           const int32_t* slot_mapping, int64_t num_tokens, void* stream);

/*
 * All-layer copy of reused image KV with M-RoPE re-rotation of K.
 * Replaces ModelRunner.copy_image_kv (engine/model_runner.py:170-180), which
 * copies flat[:, :, new_slots] = flat[:, :, old_slots] on the cache viewed as
 * [2, L, num_slots, Hkv*hd]; this entry point additionally rotates K by the
 * position delta of the token's image.
 *
 * kv_cache: bf16, plane 0 = K, plane 1 = V; element (plane, layer, slot, head, d)
 *   is at plane*plane_stride + layer*layer_stride + slot*(num_kv_heads*head_dim)
 *   + head*head_dim + d (strides in elements).
 * old_slots/new_slots: device int64 [num_tokens].  The two slot sets must not
 *   overlap except where old == new for the same token.  A token whose old or
 *   new slot lies outside [0, num_slots) is skipped.
 * seg_of_token: device int32 [num_tokens] segment (image) index of each token,
 *   or NULL for "all tokens in segment 0".
 * cos_sin: device fp32 [num_segments][head_dim/2][2] = (cos, sin) of the
 *   rotation angle of pair i, i.e. of delta_section(i) * inv_freq[i]; pair i is
 *   dims (i, i + head_dim/2) (rotate-half convention, layers/rotary_embedding.py:6-14).
 *   A pair whose entry is exactly (1, 0) is copied bit for bit.
 * rotate_k: 0 = plain copy of K and V (the reference's behaviour), 1 = rotate K.
 */
int vlc_rerotate_copy_kv(void* kv_cache, int64_t plane_stride, int64_t layer_stride,
                         int num_layers,
                         const int64_t* old_slots, const int64_t* new_slots,
                         int64_t num_tokens, int64_t num_slots, int num_kv_heads, int head_dim,
                         const int32_t* seg_of_token, const float* cos_sin,
                         int num_segments, int rotate_k, void* stream);

/*
 * Host-side work planner for vlc_varlen_attn_fwd (no device calls).
 * Replaces the scheduling that flash_attn_varlen_func performs inside the
 * external flash-attn library for the call at layers/attention.py:67-70.
 *
 * cu_seqlens_q/k: HOST int32 [num_seqs + 1] (the values prepare_prefill builds,
 *   engine/model_runner.py:197-198,256-259,284-285).
 * num_cus: compute units to plan for (256 on MI355X; 0 selects 256); a negative
 *   value plans one work item per query tile with no split of the key range.
 * Writes the plan into plan[0 .. *plan_len) (int32); returns VLC_ERR_CAPACITY
 * with *plan_len set to the required length when plan_capacity is too small.
 * *workspace_bytes receives the device workspace the plan needs.
 */
int vlc_attn_plan(const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                  int num_seqs, int num_heads_q, int num_heads_kv, int head_dim,
                  int causal, int num_cus,
                  int32_t* plan, int64_t plan_capacity, int64_t* plan_len,
                  int64_t* workspace_bytes);

/*
 * Varlen GQA attention over paged or contiguous K/V (bf16 in, fp32 accumulate,
 * bf16 out).  Replaces flash_attn_varlen_func(q, k, v, max_seqlen_q,
 * cu_seqlens_q, max_seqlen_k, cu_seqlens_k, softmax_scale, causal=True,
 * block_table) at layers/attention.py:67-70.
 *
 * q: [total_q, num_heads_q, head_dim], row stride q_row_stride elements.
 * Paged mode (block_table != NULL): k/v are caches [num_blocks, page_size,
 *   num_heads_kv, head_dim], page_size a multiple of 16 (VLC_ERR_UNSUPPORTED
 *   otherwise; the reference's pages are multiples of 256, config.py:24); key j of
 *   sequence b lives in row
 *   block_table[b*bt_row_stride + j/page_size]*page_size + j%page_size;
 *   k_row_stride/v_row_stride are elements per cache row.  Row b of the block
 *   table must hold at least ceil(sk_b / page_size) entries (the kernel reads
 *   entry j / page_size for every key j < sk_b; the table's width is not passed).
 *   A block id outside [0, num_blocks) reads as zeros (it is never dereferenced).
 * Contiguous mode (block_table == NULL): key j of sequence b is row
 *   cu_seqlens_k[b] + j of k/v, at k_row_stride / v_row_stride elements.
 * causal: row i of a sequence with lengths (sq, sk) sees keys j <= i + sk - sq
 *   (bottom-right alignment); rows that see no key produce zeros.
 * cu_seqlens_q/k: DEVICE int32 [num_seqs + 1] holding the boundaries the plan was
 *   built from, or NULL: the plan carries every boundary the kernels read.
 * plan_host / plan_dev: the plan from vlc_attn_plan, in host memory and as a
 *   device copy; plan_len its length.
 * workspace: device scratch of at least the planned workspace_bytes.
 * out: [total_q, num_heads_q, head_dim] bf16, row stride out_row_stride.
 * head_dim: 128, or 80 in contiguous mode (the vision tower's heads,
 *   flash_attn_varlen_func(..., causal=False) at models/qwen2_5_vl.py:200-210):
 *   heads stay rows of 128 elements in q, k, v and out, the products read dims
 *   0..79 of q and k and 0..95 of v; output dims 96..127 are zero and 80..95
 *   hold P.V of v's dims 80..95 (zero when v is zero-padded, as
 *   vlc_vision_rope_pad writes it).  The plan must be built with the same
 *   head_dim.
 */
int vlc_varlen_attn_fwd(const void* q, int64_t q_row_stride,
                        const void* k, int64_t k_row_stride,
                        const void* v, int64_t v_row_stride,
                        const int32_t* block_table, int64_t bt_row_stride, int page_size,
                        int64_t num_blocks,
                        const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                        int num_seqs, int num_heads_q, int num_heads_kv, int head_dim,
                        float softmax_scale, int causal,
                        const int32_t* plan_host, const int32_t* plan_dev, int64_t plan_len,
                        void* out, int64_t out_row_stride,
                        void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Host-side sizing for vlc_decode_attn (no device calls).
 * The reference's decode call, flash_attn_with_kvcache at layers/attention.py:71-74,
 * sizes its split-KV work inside the external flash-attn library; here the caller
 * asks once per step (or once per maximum context length) for:
 *   *key_chunk      keys per workgroup (a multiple of 128),
 *   *grid_splits    workgroups per (sequence, kv head) the launch provides, enough
 *                   for max_seqlen_k keys,
 *   *workspace_bytes  device workspace the call needs.
 *   *pipeline_out   the kernel shape to launch with.
 * num_splits > 0 forces the number of chunks for max_seqlen_k; 0 chooses one
 * wave of workgroups over the compute units (num_cus, 0 selects 256), at most 32
 * chunks per pair.  pipeline selects the kernel shape: 16 * waves per workgroup +
 * stages per wave, plus 0x100 for 16-key tiles (else 32): 0x42, 0x22, 0x23, 0x24,
 * 0x14, 0x142, 0x144, 0x182, 0x124; 0 chooses.
 * Requires head_dim == 128, num_heads_q / num_heads_kv <= 16 and page_size a
 * multiple of the shape's tile (16 or 32 keys).
 */
int vlc_decode_attn_plan(int batch, int num_heads_q, int num_heads_kv, int head_dim, int page_size,
                         int max_seqlen_k, int num_cus, int num_splits, int pipeline,
                         int32_t* key_chunk, int32_t* grid_splits, int32_t* pipeline_out,
                         int64_t* workspace_bytes);

/*
 * Paged GQA decode attention: one query per sequence against its paged cache.
 * Replaces flash_attn_with_kvcache(q.unsqueeze(1), k_cache, v_cache,
 * cache_seqlens=context_lens, block_table=block_tables, softmax_scale, causal=True)
 * at layers/attention.py:71-74.
 *
 * q: [batch, num_heads_q, head_dim] bf16, q_row_stride elements between sequences
 *   (heads are contiguous rows of head_dim).  out: same shape, out_row_stride.
 * k_cache/v_cache: [num_blocks, page_size, num_heads_kv, head_dim] bf16 with
 *   cache_row_stride elements per token row.  Key j of sequence b is row
 *   block_table[b*bt_row_stride + j/page_size]*page_size + j%page_size.
 * cache_seqlens: DEVICE int32 [batch], keys per sequence; sequence b attends keys
 *   [0, cache_seqlens[b]) (the query is the last position, so causal masking
 *   hides nothing).  Lengths are clamped to bt_cols*page_size and to
 *   grid_splits*key_chunk; a sequence with no key gets zeros; a block id outside
 *   [0, num_blocks) reads as zeros.
 * key_chunk, grid_splits, pipeline: from vlc_decode_attn_plan for an upper bound
 *   of the lengths.  workspace: device memory of at least the planned bytes, whose first
 *   batch*num_heads_kv 32-bit words must be zero before the first call; every
 *   call leaves them zero.  Calls that share a workspace must not overlap.
 */
int vlc_decode_attn(const void* q, int64_t q_row_stride, const void* k_cache, const void* v_cache,
                    int64_t cache_row_stride, int page_size, int64_t num_blocks,
                    const int32_t* block_table, int64_t bt_row_stride, int bt_cols,
                    const int32_t* cache_seqlens, int batch, int num_heads_q, int num_heads_kv,
                    int head_dim, float softmax_scale, int key_chunk, int grid_splits, int pipeline,
                    void* out, int64_t out_row_stride, void* workspace, int64_t workspace_bytes,
                    void* stream);

/*
 * Allocation-free variant of vlc_decode_attn.  It has no counterpart in the
 * reference: it is for callers that cannot allocate device memory or pass a
 * workspace -- code under HIP graph capture (the reference replays its decode
 * step from a captured CUDA graph, engine/model_runner.py:418-432,453-479), tight serving
 * loops, harnesses that forbid allocation.
 *
 * Arguments and results are those of vlc_decode_attn without workspace and
 * workspace_bytes: the ticket counters and split partials live in a fixed
 * device array inside the library, VLC_DECODE_NOALLOC_MAX_BYTES (16 MiB) per
 * device, held until the process ends.  A call whose plan has grid_splits > 1
 * and whose workspace (as vlc_decode_attn_plan sizes it) exceeds that returns
 * VLC_ERR_SCRATCH before any device work; with grid_splits == 1 no scratch is
 * used.  The first call on a device looks the array up and enqueues a small
 * kernel on `stream` that zeroes its counters; no call allocates, frees or
 * synchronises.  Every call on a device shares that device's array: calls that
 * overlap on one device (other streams, other host threads) race and must not
 * be issued.
 */
#define VLC_DECODE_NOALLOC_MAX_BYTES (((int64_t)16) << 20)
int vlc_decode_attn_noalloc(const void* q, int64_t q_row_stride, const void* k_cache, const void* v_cache,
                            int64_t cache_row_stride, int page_size, int64_t num_blocks,
                            const int32_t* block_table, int64_t bt_row_stride, int bt_cols,
                            const int32_t* cache_seqlens, int batch, int num_heads_q, int num_heads_kv,
                            int head_dim, float softmax_scale, int key_chunk, int grid_splits, int pipeline,
                            void* out, int64_t out_row_stride, void* stream);

/*
 * Vision tower: 2-D rotary embedding of q and k fused with the split of the QKV
 * projection into zero-padded head rows for vlc_varlen_attn_fwd.
 * Replaces qkv.split + reshape + apply_rotary_pos_emb_vision of q and k in
 * VisionAttention.forward (models/qwen2_5_vl.py:176-199).
 *
 * qkv: [num_tokens, 3 * num_heads * head_dim] bf16 at row stride qkv_row_stride
 *   (q heads, then k heads, then v heads; the checkpoint's packed layout).
 * pos_hw: int32 [num_tokens][2], (patch row, patch column) of each token.
 * cos_table / sin_table: bf16 [max_pos][head_dim / 4]; row p holds cos / sin of
 *   the angle p * inv_freq[i] (the reference rounds the angle to bf16 before
 *   taking cos / sin, models/qwen2_5_vl.py:486).  Dim j of a head, with
 *   a = j mod head_dim/2, uses column a of row pos_h for a < head_dim/4 and
 *   column a - head_dim/4 of row pos_w otherwise.  Positions are clamped to
 *   [0, max_pos).
 * y[j] = bf16(bf16(x[j]*cos) + bf16(rotate_half(x)[j]*sin)) for q and k, as the
 *   reference's bf16 tensor arithmetic rounds; v is copied.
 * out: [num_tokens][3][num_heads][padded_dim] bf16 at row stride out_row_stride;
 *   dims head_dim..padded_dim-1 of every head are written as zero.
 * head_dim % 16 == 0, padded_dim % 8 == 0, head_dim <= padded_dim <= 128; qkv,
 * out and their row strides 16-byte aligned, the tables 8-byte aligned.
 */
int vlc_vision_rope_pad(const void* qkv, int64_t qkv_row_stride, const int32_t* pos_hw,
                        const void* cos_table, const void* sin_table, int64_t max_pos,
                        int64_t num_tokens, int num_heads, int head_dim, int padded_dim,
                        void* out, int64_t out_row_stride, void* stream);

/*
 * RMSNorm, optionally with the residual add fused in front of it.
 * Replaces RMSNorm.rms_forward / add_rms_forward (layers/layernorm.py:16-40),
 * used by the decoder (models/qwen3.py:145-158, :184) and the vision tower
 * (models/qwen2_5_vl.py:292-305, :330).
 *
 * x, residual, residual_out, out: [num_rows, dim] bf16 at their row strides
 * (elements); weight: bf16 [dim].
 *   residual == NULL: out = bf16(bf16(x * r) * weight), r = rsqrt(mean(x^2) + eps);
 *   otherwise:        s = x + residual in fp32, residual_out = bf16(s),
 *                     out = bf16(bf16(s * r) * weight) with r from the fp32 s.
 * residual_out may be residual or x (each element is read before it is written);
 * out must not overlap residual_out.  dim % 8 == 0, dim <= 8192; pointers 16-byte
 * aligned and row strides multiples of 8 elements.
 */
int vlc_rms_norm(const void* x, int64_t x_row_stride, const void* residual, int64_t residual_row_stride,
                 void* residual_out, int64_t residual_out_row_stride, const void* weight, float eps,
                 int64_t num_rows, int64_t dim, void* out, int64_t out_row_stride, void* stream);

/*
 * SiLU-and-multiply of a packed [gate | up] projection.
 * Replaces SiluAndMul (layers/activation.py:8-14), used by the decoder MLP
 * (models/qwen3.py:97-110) and the vision MLP (models/qwen2_5_vl.py:219-243).
 *
 * gate_up: [num_rows, 2 * inter] bf16 at gate_up_row_stride (gate columns
 * [0, inter), up columns [inter, 2 * inter)); out[n][i] = bf16(silu(gate) * up)
 * with fp32 math, silu(g) = g / (1 + exp(-g)).  inter % 4 == 0; pointers 8-byte
 * aligned and row strides multiples of 4 elements.
 */
int vlc_silu_mul(const void* gate_up, int64_t gate_up_row_stride, int64_t num_rows, int64_t inter,
                 void* out, int64_t out_row_stride, void* stream);

/*
 * Skinny linear layer (M <= 16 rows): out[m][n] = bf16(sum_k x[m][k] * weight[n][k] + bias[n]),
 * fp32 accumulation.  Replaces the decode-step projections of the decoder
 * (QKVParallelLinear / RowParallelLinear / MergedColumnParallelLinear and the LM head,
 * models/qwen3.py:71-110, layers/embed_head.py:56-66) whose work is streaming the
 * weights once.
 *
 * x: [rows, in_features] bf16 at x_row_stride; weight: [out_features, in_features]
 * bf16 at w_row_stride (nn.Linear layout); bias: bf16 [out_features] or NULL;
 * out: [rows, out_features] bf16 at out_row_stride.  rows <= 16, in_features % 32 == 0,
 * out_features % 16 == 0; x and weight 16-byte aligned with row strides multiples of 8
 * elements; out and bias 8-byte aligned, out_row_stride a multiple of 4.
 */
int vlc_linear_skinny(const void* x, int64_t x_row_stride, int64_t rows, int64_t in_features,
                      const void* weight, int64_t w_row_stride, int64_t out_features, const void* bias,
                      void* out, int64_t out_row_stride, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* VLC_CAPI_H */
