/*
 * paged_kv.h — C ABI of the MI355X (gfx950) paged-KV hot path.
 *
 * Every entry point takes plain device pointers, element strides and sizes, a dtype
 * code and a hipStream_t passed as void*. None allocates device memory, copies
 * synchronously or synchronises, so every call can be recorded into a hipGraph.
 * Buffers are owned by the caller. Calls return 0 on success, a negative PKV_E_* code
 * when the arguments are rejected before anything is launched, or a positive
 * hipError_t when the launch itself fails.
 *
 * Pool layout (one layer): [num_slots, num_kv_heads, head_dim], slot = block * block_size
 * + offset, exactly the layout of PagedKVCache.k[layer] in
 * engine/runtime/paged_cache.py:32-35 of the reference.
 */
#ifndef PAGED_KV_H
#define PAGED_KV_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes */
#define PKV_F32 0
#define PKV_F16 1
#define PKV_BF16 2

/* validation errors (negative) */
#define PKV_E_DTYPE (-1)     /* unsupported dtype or dtype combination */
#define PKV_E_SHAPE (-2)     /* unsupported head_dim / group size / block size / sizes */
#define PKV_E_ALIGN (-3)     /* pointer or stride not aligned for 16-byte vector access */
#define PKV_E_WORKSPACE (-4) /* split-K workspace missing or too small */
#define PKV_E_NULL (-5)      /* required pointer is NULL */
#define PKV_E_HIP (-6)       /* a HIP device query failed (no usable GPU) */
#define PKV_E_SCRATCH (-7)   /* the call needs more than the no-alloc scratch holds */

/* Bytes of the static device scratch behind pkv_paged_decode_noalloc (per GPU). */
#define PKV_NOALLOC_SCRATCH_BYTES (32LL << 20)

/* ABI version, bumped on any signature change. */
int pkv_abi_version(void);

/* Human-readable text for a status code returned by any entry point. */
const char* pkv_status_string(int status);

/*
 * KV append: k_pool[slots[i]] = convert(k_new[i]), v_pool[slots[i]] = convert(v_new[i]).
 * Replaces PagedKVCache.write (reference engine/runtime/paged_cache.py:42-45), i.e.
 * two Tensor.index_copy_(0, slots, x.to(pool dtype)) calls. Conversions round to nearest
 * even (float -> bf16 maps NaN to 0x7FC0, as torch does). Rows whose slot is outside
 * [0, num_slots) are skipped (no write). Duplicate slots: one of the rows wins.
 * k_new / v_new: [n_tokens, num_kv_heads, head_dim] with unit stride in head_dim.
 */
int pkv_kv_append(void* k_pool, void* v_pool, int pool_dtype, int64_t pool_stride_slot,
                  int64_t pool_stride_head, int64_t num_slots, const void* k_new,
                  int64_t k_stride_tok, int64_t k_stride_head, const void* v_new,
                  int64_t v_stride_tok, int64_t v_stride_head, int new_dtype,
                  const int64_t* slots, int64_t n_tokens, int32_t num_kv_heads,
                  int32_t head_dim, void* stream);

/*
 * Block copy for prefix-cache copy-on-write. No counterpart exists in the reference
 * (its prefix cache only shares full, never-written blocks; see
 * engine/runtime/block_manager.py:130-150); this is the operation a block manager calls
 * before appending into a shared block. For every layer l < num_layers and pair i:
 *   pool[l, dst_i*block_size : (dst_i+1)*block_size] = pool[l, src_i*block_size : ...]
 * for both pools. block_mapping is a device int64 array [n_pairs, 2] of (src, dst).
 * block_bytes = block_size * num_kv_heads * head_dim * element size (a block is
 * contiguous inside one layer). Pairs with src or dst outside [0, num_blocks) are
 * skipped. A dst that is also some pair's src gives an unspecified result.
 */
int pkv_copy_blocks(void* k_pool, void* v_pool, int64_t layer_stride_bytes,
                    int32_t num_layers, int64_t block_bytes, int64_t num_blocks,
                    const int64_t* block_mapping, int64_t n_pairs, void* stream);

/*
 * Slot mapping of a decode step, built on the device: for each sequence b,
 *   slots[b] = block_tables[b, (n-1) / block_size] * block_size + (n-1) % block_size,
 * n = context_lens[b] (the new token included), or -1 -- which pkv_kv_append skips --
 * when n < 1, (n-1) / block_size >= max_blocks, or the slot is outside [0, num_slots).
 * Replaces the host-side slot lists of PagedBatch._decode and DecodeGraphs.run
 * (reference engine/runtime/paged_cache.py:140-143, engine/runtime/cuda_graphs.py:104,
 * engine/runtime/engine.py:208-210), so a captured decode step needs only the tables and
 * lengths copied in. slots: device int64 [batch].
 */
int pkv_decode_slots(int64_t* slots, const int32_t* block_tables, int64_t table_stride,
                     int32_t max_blocks, const int32_t* context_lens, int32_t batch,
                     int32_t block_size, int64_t num_slots, void* stream);

/*
 * Workgroups the decode kernel should use on the current device for this shape: as
 * many as the GPU holds resident at once (CUs x workgroups per CU). Depends only on the
 * device and static shapes, so a graph captured with it stays valid. Returns >= 1, or a
 * negative PKV_E_* code.
 */
int32_t pkv_decode_workgroups(int kv_dtype, int32_t head_dim, int32_t num_heads,
                              int32_t num_kv_heads);

/*
 * What num_workgroups = 0 (the default split) of pkv_paged_decode runs for this shape
 * without cascade extras: 0 for the one-kernel split pass (no workspace), else the
 * stream-K workgroup count (pkv_decode_workgroups), whose workspace the caller passes.
 * Depends on static shapes and the device only. Negative: a PKV_E_* code.
 */
int32_t pkv_decode_default_workgroups(int kv_dtype, int32_t head_dim, int32_t num_heads,
                                      int32_t num_kv_heads, int32_t batch, int32_t max_blocks,
                                      int32_t block_size);

/* Bytes of scratch pkv_paged_decode needs for num_workgroups (0 when it is 1): one
 * 16-byte merge plan per sequence, then the partial records of sequences cut by a
 * range boundary. Any contents. */
int64_t pkv_decode_workspace_bytes(int32_t num_workgroups, int32_t batch, int32_t num_heads,
                                   int32_t head_dim);

/*
 * Paged decode attention (GQA). Replaces paged_decode_attention and its Triton kernels
 * (reference engine/kernels/paged_attention.py:44-179). For sequence b and query head h:
 *   n    = clamp(context_lens[b], 0, max_blocks * block_size)
 *   slot = block_tables[b, p / block_size] * block_size + p % block_size, p < n
 *   out[b, h] = softmax_p(scale * q[b,h] . k[slot_p, h / G]) @ v[slot_p, h / G]
 * with G = num_heads / num_kv_heads, fp32 softmax and accumulation; n == 0 gives 0.
 * Tokens whose slot falls outside [0, num_slots) are left out of the softmax.
 * q: [batch, num_heads, head_dim] in kv_dtype; out: same shape, kv_dtype or PKV_F32.
 * k_cache / v_cache share strides (stride_slot, stride_head, 1).
 * block_tables: int32 [batch, >= max_blocks] with row stride table_stride.
 * head_dim in {16, 32, 64, 128, 256}.
 * Work split: the contexts of all sequences, laid end to end, are divided evenly among
 * num_workgroups workgroups; a second kernel merges the pieces of sequences cut by a
 * boundary. num_workgroups > 1 needs a 16-byte aligned scratch `workspace` of
 * pkv_decode_workspace_bytes() bytes (any contents). num_workgroups = 0 asks for the
 * library's default, chosen from static shapes only (so a captured graph stays valid
 * for every context length): small batches of 16-bit K/V at head_dim 64 or 128 whose
 * (sequence, KV head) pairs fit the CUs and whose table width is at most 2,048 tokens
 * run one kernel with one workgroup per (sequence, KV head, sub-group of its query
 * heads -- as few heads as keep the workgroups within the CUs) that splits the
 * sequence among its waves and merges in LDS (no workspace used); everything else the
 * split above with pkv_decode_workgroups() workgroups, whose workspace size the caller
 * passes.
 */
int pkv_paged_decode(void* out, int out_dtype, int64_t out_stride_b, int64_t out_stride_h,
                     const void* q, int64_t q_stride_b, int64_t q_stride_h,
                     const void* k_cache, const void* v_cache, int kv_dtype,
                     int64_t kv_stride_slot, int64_t kv_stride_head, int64_t num_slots,
                     const int32_t* block_tables, int64_t table_stride, int32_t max_blocks,
                     const int32_t* context_lens, int32_t batch, int32_t num_heads,
                     int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                     float scale, int32_t num_workgroups, void* workspace,
                     int64_t workspace_bytes, void* stream);

/*
 * pkv_paged_decode without a workspace argument, for callers that cannot allocate (code
 * under hipGraph capture that must not call hipMalloc, tight serving loops, harnesses
 * that forbid allocation). No counterpart in the reference: its Triton decode needs no
 * scratch. Same arguments, kernels and results as pkv_paged_decode at the same
 * num_workgroups; the split-K workspace is a static device array of
 * PKV_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends. Calls whose workspace
 * (pkv_decode_workspace_bytes) exceeds it return PKV_E_SCRATCH before any launch. The
 * first call on a device resolves the array's address (make it outside graph capture).
 * Calls on one GPU share the array: calls that overlap on one GPU (concurrent streams)
 * race on it and must be serialised by the caller. Nothing is allocated, copied
 * synchronously or synchronised.
 */
int pkv_paged_decode_noalloc(void* out, int out_dtype, int64_t out_stride_b,
                             int64_t out_stride_h, const void* q, int64_t q_stride_b,
                             int64_t q_stride_h, const void* k_cache, const void* v_cache,
                             int kv_dtype, int64_t kv_stride_slot, int64_t kv_stride_head,
                             int64_t num_slots, const int32_t* block_tables,
                             int64_t table_stride, int32_t max_blocks,
                             const int32_t* context_lens, int32_t batch, int32_t num_heads,
                             int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                             float scale, int32_t num_workgroups, void* stream);

/* Bytes of scratch pkv_paged_decode_ex needs with prefix parts (cascade): the split-K
 * scratch plus fp32 room for the sequences the stream pass finishes, [batch, num_heads,
 * head_dim + 1]. Needed at any num_workgroups, 1 included. */
int64_t pkv_cascade_workspace_bytes(int32_t num_workgroups, int32_t batch, int32_t num_heads,
                                    int32_t head_dim);

/*
 * pkv_paged_decode with optional extras for cascade decode over shared prefixes (no
 * counterpart in the reference, which reads every sequence's whole context):
 *   first_block (int32 [batch], or NULL = all 0): sequence b attends only to table columns
 *     first_block[b] onwards, i.e. to positions first_block[b] * block_size .. n - 1 (a
 *     shared prefix held in the earlier columns is handled by a separate call);
 *   prefix_out / prefix_lse / prefix_row (fp32 [rows, num_heads, head_dim] contiguous and
 *     16-byte aligned / fp32 [rows, num_heads] / int32 [batch]; prefix_row NULL or
 *     prefix_parts 0 = none): attentions of the same queries over other keys, merged
 *     into the result. For sequence b with prefix_row[b] >= 0, its parts are rows
 *     prefix_row[b] + k * prefix_stride, k < prefix_parts, each a normalised output O_k
 *     with log2 normaliser lse_k (pkv_paged_prefill_ex writes both); the result is the
 *     softmax over the union of the key sets,
 *       out = (sum_i 2^(lse_i - M) O_i) / (sum_i 2^(lse_i - M)),  M = max_i lse_i,
 *     over the parts and this call's own keys. The workspace must then hold
 *     pkv_cascade_workspace_bytes() bytes;
 *   lse (fp32 [batch, num_heads], or NULL): receives the result's log2 normaliser in the
 *     kernel's score units, max_p(s_p) + log2(sum_p exp2(s_p - max)), s_p = scale *
 *     log2(e) * q . k_p, parts included; -inf when no key was live.
 */
int pkv_paged_decode_ex(void* out, int out_dtype, int64_t out_stride_b, int64_t out_stride_h,
                        const void* q, int64_t q_stride_b, int64_t q_stride_h,
                        const void* k_cache, const void* v_cache, int kv_dtype,
                        int64_t kv_stride_slot, int64_t kv_stride_head, int64_t num_slots,
                        const int32_t* block_tables, int64_t table_stride, int32_t max_blocks,
                        const int32_t* context_lens, int32_t batch, int32_t num_heads,
                        int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                        float scale, int32_t num_workgroups, void* workspace,
                        int64_t workspace_bytes, const int32_t* first_block, float* lse,
                        const float* prefix_out, const float* prefix_lse,
                        const int32_t* prefix_row, int32_t prefix_parts,
                        int64_t prefix_stride, void* stream);

/* 1 when pkv_cascade_decode runs the prefix pass and the decode pass as one launch for
 * these shapes (at the library's default workgroup count), else 0. Callers that lay out
 * prefix groups use it to pick the pieces per prefix (no counterpart in the reference). */
int32_t pkv_cascade_one_launch(int kv_dtype, int32_t head_dim, int32_t num_heads,
                               int32_t num_kv_heads, int32_t block_size, int32_t batch);

/*
 * Cascade decode in one call (no counterpart in the reference, which reads every
 * sequence's whole context): the prefix pass -- pkv_paged_prefill_ex(prefix_out, PKV_F32,
 * row stride num_heads * head_dim, head stride head_dim, q, ..., prefix_tables,
 * prefix_table_stride, prefix_width, prefix_ctx, prefix_cu_q, prefix_chunks,
 * prefix_max_queries, ..., causal 0, prefix_q_rows, prefix_lse) -- followed by
 * pkv_paged_decode_ex(out, ..., first_block, lse, prefix_out, prefix_lse, prefix_row,
 * prefix_parts, prefix_stride), with the same arguments, results and errors as those two
 * calls. prefix_out (fp32 [rows, num_heads, head_dim], contiguous, 16-byte aligned) and
 * prefix_lse (fp32 [rows, num_heads]) are the caller's scratch for the parts.
 * An empty prefix layout (prefix_chunks or prefix_max_queries 0) returns PKV_E_SHAPE:
 * no part would be written for the merge to read.
 * prefix_workgroups < 0 runs the two passes as two launches. Otherwise, for 16-bit K/V at
 * head_dim 64 or 128, power-of-two blocks of at least 16 tokens, 65 to 1,024 sequences and
 * at least 8 (KV head, head sub-group) tasks, the two passes share one launch:
 * prefix_workgroups (0: the library's default) of the num_workgroups workgroups take the
 * prefix pass's items in turn while the others run the stream pass. Other shapes run two
 * launches. The workspace is pkv_cascade_workspace_bytes(num_workgroups, ...) bytes, as
 * for pkv_paged_decode_ex.
 */
int pkv_cascade_decode(void* out, int out_dtype, int64_t out_stride_b, int64_t out_stride_h,
                       const void* q, int64_t q_stride_b, int64_t q_stride_h,
                       const void* k_cache, const void* v_cache, int kv_dtype,
                       int64_t kv_stride_slot, int64_t kv_stride_head, int64_t num_slots,
                       const int32_t* block_tables, int64_t table_stride, int32_t max_blocks,
                       const int32_t* context_lens, int32_t batch, int32_t num_heads,
                       int32_t num_kv_heads, int32_t head_dim, int32_t block_size, float scale,
                       int32_t num_workgroups, void* workspace, int64_t workspace_bytes,
                       const int32_t* first_block, float* lse, const int32_t* prefix_tables,
                       int64_t prefix_table_stride, int32_t prefix_width,
                       const int32_t* prefix_ctx, const int32_t* prefix_cu_q,
                       int32_t prefix_chunks, int32_t prefix_max_queries,
                       const int32_t* prefix_q_rows, float* prefix_out, float* prefix_lse,
                       const int32_t* prefix_row, int32_t prefix_parts, int64_t prefix_stride,
                       int32_t prefix_workgroups, void* stream);

/*
 * Chunked-prefill attention over the paged pool, on the matrix cores. Replaces the
 * reference's gather of each chunk's context slots plus FlashAttention varlen call
 * (engine/model/layers.py:246-253, metadata from engine/runtime/paged_cache.py:159-202).
 * Chunk c owns query tokens cu_seqlens_q[c] .. cu_seqlens_q[c+1]-1 of q and a context
 * of n_c = clamp(context_lens[c], 0, max_blocks * block_size) tokens reached through
 * block_tables row c, its own tokens last: query i of a chunk of q_c tokens sits at
 * position n_c - q_c + i and attends to keys 0 .. n_c - q_c + i (bottom-right causal).
 *   out[t, h] = softmax(scale * q[t,h] . K^T) V over those keys, KV head h / G.
 * q, out: [tokens, num_heads, head_dim]; out in kv_dtype or PKV_F32. kv_dtype is bf16
 * or fp16; head_dim in {32, 64, 128, 256}. max_query_len bounds every chunk's length
 * (it sizes the grid, so one hipGraph capture serves every length up to it). Block ids
 * must address the pool (out-of-range ids are clamped for memory safety only).
 * scale must be positive and finite (PKV_E_SHAPE otherwise).
 * Softmax statistics are fp32; for the P.V product the probabilities enter the matrix
 * cores as fp16 (fp16 caches) or as a bf16 hi + lo pair (bf16 caches).
 */
int pkv_paged_prefill(void* out, int out_dtype, int64_t out_stride_tok, int64_t out_stride_h,
                      const void* q, int64_t q_stride_tok, int64_t q_stride_h,
                      const void* k_cache, const void* v_cache, int kv_dtype,
                      int64_t kv_stride_slot, int64_t kv_stride_head, int64_t num_slots,
                      const int32_t* block_tables, int64_t table_stride, int32_t max_blocks,
                      const int32_t* context_lens, const int32_t* cu_seqlens_q, int32_t n_chunks,
                      int32_t max_query_len, int32_t num_heads, int32_t num_kv_heads,
                      int32_t head_dim, int32_t block_size, float scale, void* stream);

/*
 * pkv_paged_prefill with three extras, for the shared-prefix part of cascade decode (no
 * counterpart in the reference):
 *   causal = 0: every query of chunk c attends to all n_c keys of its context (the
 *     shared prefix), instead of the bottom-right causal limit;
 *   q_rows (int32 [tokens], or NULL = identity): query token t of the step reads q row
 *     q_rows[t] (a chunk's queries can be rows scattered over the batch); out and lse
 *     stay in step order; a negative q_rows[t] means no query at t: nothing is read
 *     for it and its out and lse rows are left untouched (padding in a fixed layout);
 *   lse (fp32 [tokens, num_heads], or NULL): log2 normalisers as in pkv_paged_decode_ex.
 */
int pkv_paged_prefill_ex(void* out, int out_dtype, int64_t out_stride_tok, int64_t out_stride_h,
                         const void* q, int64_t q_stride_tok, int64_t q_stride_h,
                         const void* k_cache, const void* v_cache, int kv_dtype,
                         int64_t kv_stride_slot, int64_t kv_stride_head, int64_t num_slots,
                         const int32_t* block_tables, int64_t table_stride, int32_t max_blocks,
                         const int32_t* context_lens, const int32_t* cu_seqlens_q,
                         int32_t n_chunks, int32_t max_query_len, int32_t num_heads,
                         int32_t num_kv_heads, int32_t head_dim, int32_t block_size, float scale,
                         int32_t causal, const int32_t* q_rows, float* lse, void* stream);

/*
 * Bytes of workspace pkv_paged_prefill_ws needs for the fp16 V copy at these static
 * shapes: about n_chunks x (max_blocks * block_size rounded up to 256) x num_kv_heads x
 * head_dim x 2, plus one scale byte per 256 tokens of each. 0 for shapes that take no
 * copy (fp16 or fp32 caches, head_dim 16, tables of more than 65,536 tokens); negative:
 * PKV_E_DTYPE or PKV_E_SHAPE. No counterpart in the reference (whose varlen path
 * gathers each chunk's K and V into new tensors itself).
 */
int64_t pkv_prefill_workspace_bytes(int kv_dtype, int32_t head_dim, int32_t num_kv_heads,
                                    int32_t n_chunks, int32_t max_blocks, int32_t block_size);

/*
 * pkv_paged_prefill with a workspace; replaces the same reference call (engine/model/
 * layers.py:246-253). When workspace_bytes >= pkv_prefill_workspace_bytes (> 0) for
 * these shapes, a first kernel writes each chunk's V (its clamped context, per KV head)
 * as fp16 into the workspace, each 256-token tile times a power of two 2^-k that keeps
 * its largest |V| below 2^16 (k = 0 unless some |V| >= 2^16), and the matrix cores then
 * multiply P by that copy in fp16 (P rounded once, as for fp16 caches) instead of as a
 * bf16 hi + lo pair: one P.V product instead of two. The scaled bf16 -> fp16 conversion
 * is exact down to 2^-14 (times 2^k); smaller values keep an absolute error below
 * 2^-25 (times 2^k). With a smaller workspace (NULL and 0 included) the call is
 * pkv_paged_prefill. The workspace is scratch (its contents on entry do not matter; the
 * call overwrites them) and 16-byte aligned (PKV_E_ALIGN otherwise; PKV_E_WORKSPACE for
 * negative bytes, or bytes without a pointer).
 */
int pkv_paged_prefill_ws(void* out, int out_dtype, int64_t out_stride_tok, int64_t out_stride_h,
                         const void* q, int64_t q_stride_tok, int64_t q_stride_h,
                         const void* k_cache, const void* v_cache, int kv_dtype,
                         int64_t kv_stride_slot, int64_t kv_stride_head, int64_t num_slots,
                         const int32_t* block_tables, int64_t table_stride, int32_t max_blocks,
                         const int32_t* context_lens, const int32_t* cu_seqlens_q,
                         int32_t n_chunks, int32_t max_query_len, int32_t num_heads,
                         int32_t num_kv_heads, int32_t head_dim, int32_t block_size, float scale,
                         void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Fused element-wise kernels (csrc/fused.hip). Replace the reference's Triton kernels of
 * engine/kernels/fused.py:47-131 (rms_norm, rope_, silu_mul), with the same contract:
 * every result is bitwise identical to the PyTorch ops they stand for.
 *
 * RMSNorm tail (reference fused.py:47-59, :93-111): for row r and column c,
 *   out[r, c] = w[c] * (x[r, c] (as fp32) * inv_rms[r]).to(x dtype)
 * inv_rms (fp32 [rows]) = rsqrt(mean(x[r]^2) + eps) is computed by the caller with
 * PyTorch: the reference leaves the mean to PyTorch (a fused sum adds in another order),
 * and PyTorch's ROCm rsqrt can differ from the device library's in the last fp32 bit.
 * out_dtype must be the promotion of x_dtype and w_dtype (equal dtypes stay; mixed ones
 * give PKV_F32). Columns are unit-stride.
 */
int pkv_rms_norm(void* out, int out_dtype, int64_t out_stride_row, const void* x, int x_dtype,
                 int64_t x_stride_row, const float* inv_rms, const void* weight, int w_dtype,
                 int64_t rows, int64_t cols, void* stream);

/*
 * RoPE in place (reference fused.py:61-80, :114-121): x [n_tokens, heads, head_dim]
 * (unit stride in head_dim) becomes x * cos + rotate_half(x) * sin, rotate_half(x) =
 * cat(-x[half:], x[:half]); cos / sin are fp32 [n_tokens, head_dim] with row stride
 * cs_stride_tok, cast to x's dtype first; each product and the sum round to the dtype.
 */
int pkv_rope(void* x, int dtype, int64_t stride_tok, int64_t stride_head, const float* cos,
             const float* sin, int64_t cs_stride_tok, int64_t n_tokens, int32_t heads,
             int32_t head_dim, void* stream);

/*
 * SiLU and multiply (reference fused.py:82-90, :124-131): out = silu(gate) * up, silu
 * computed in fp32 as g / (1 + exp(-g)) and rounded to the dtype, then the product
 * rounded. gate, up, out: n contiguous elements of one dtype.
 */
int pkv_silu_mul(void* out, const void* gate, const void* up, int dtype, int64_t n,
                 void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PAGED_KV_H */
