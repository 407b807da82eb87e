// cascade.h -- host-side functions that decode.hip, prefill.hip and cascade.hip share for
// cascade decode in one launch. The argument blocks themselves are defined with their
// kernels (decode_kernels.h: DecodeArgs, prefill_kernels.h: PrefillArgs).

#pragma once

#include "common.h"

namespace pkv {

struct DecodeArgs;
struct PrefillArgs;

// prefill.hip: checks the arguments of a pkv_paged_prefill_ex call and fills *a and *rows
// (the query rows of the longest chunk for one KV head: max_query_len x group). Returns 0,
// 1 when the call has nothing to do (no chunk or no query), or a PKV_E_* code.
int prefill_args(PrefillArgs* a, int64_t* rows, void* out, int out_dtype, int64_t out_stride_tok,
                 int64_t out_stride_h, const void* q, int64_t q_stride_tok, int64_t q_stride_h,
                 const void* k_cache, const void* v_cache, int kv_dtype, int64_t kv_stride_slot,
                 int64_t kv_stride_head, int64_t num_slots, const int32_t* block_tables,
                 int64_t table_stride, int32_t max_blocks, const int32_t* context_lens,
                 const int32_t* cu_seqlens_q, int32_t n_chunks, int32_t max_query_len,
                 int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                 float scale, int32_t causal, const int32_t* q_rows, float* lse);

// One-launch cascade: the prefix pass's arguments, its query rows per chunk and KV head
// (max_query_len x group) and how many workgroups take it. Once its items are done, each
// prefix workgroup streams tail_slots / wslots of a stream workgroup's share of the
// units (tail_slots 0: none).
struct CascadeLaunch {
  const PrefillArgs* p;
  int64_t rows;
  int prefix_wg;
  int wslots, tail_slots;
};

// decode.hip: pkv_paged_decode_ex; with `one`, the stream pass runs in one launch with
// the prefix pass `one` describes (PKV_E_SHAPE where cascade_prefix_wg gives 0). With
// check_only, every argument check runs and nothing is launched.
int decode_ex(void* out, int out_dtype, int64_t out_stride_b, int64_t out_stride_h,
              const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k_cache,
              const void* v_cache, int kv_dtype, int64_t kv_stride_slot, int64_t kv_stride_head,
              int64_t num_slots, const int32_t* block_tables, int64_t table_stride,
              int32_t max_blocks, const int32_t* context_lens, int32_t batch, int32_t num_heads,
              int32_t num_kv_heads, int32_t head_dim, int32_t block_size, float scale,
              int32_t num_workgroups, void* workspace, int64_t workspace_bytes,
              const int32_t* first_block, float* lse, const float* prefix_out,
              const float* prefix_lse, const int32_t* prefix_row, int32_t prefix_parts,
              int64_t prefix_stride, void* stream, const CascadeLaunch* one,
              bool check_only);

// decode.hip: the prefix workgroups of a one-launch cascade for these shapes with `items`
// prefix items (requested > 0: that many; 0: the library's choice), or 0 when the call
// takes two launches (requested < 0, or shapes without a one-launch form).
int cascade_prefix_wg(int kv_dtype, int head_dim, int num_heads, int num_kv_heads,
                      int block_size, int batch, int num_workgroups, int64_t items,
                      int requested);

// cascade.hip: whether the one-launch cascade has an instantiation for these shapes
// (16-bit K/V at head_dim 64 or 128, power-of-two blocks of at least 16 tokens, 65 to
// 1,024 sequences: the stream pass's LDS-staged form, full 8-wave workgroups).
bool cascade_one_launch_shape(int kv_dtype, int head_dim, int block_size, int batch,
                              int waves_per_wg);

// cascade.hip: launches the prefix pass p (prefix_wg x ygrid workgroups, each taking
// items in turn, then stream ranges d.full_wg + x if d.num_wg > d.full_wg) and the stream
// pass d (ranges 0 .. d.full_wg - 1) as one grid of (prefix_wg + d.full_wg) x ygrid.
// gpw: query heads per wave of the stream pass.
hipError_t launch_cascade(const DecodeArgs& d, const PrefillArgs& p, int64_t rows, int kv_dtype,
                          int head_dim, int gpw, int prefix_wg, int ygrid, hipStream_t st);

}  // namespace pkv
