// cascade.hip -- cascade decode's prefix pass and tail pass in one launch
// (include/paged_kv.h: pkv_cascade_decode).
//
// Run one after the other, the prefix pass (each group's queries against its shared
// blocks, on the matrix cores) holds the whole GPU while its short items wait on memory,
// and the tail pass (the HBM-bound stream over each sequence's private blocks) waits for
// it. Run on separate streams, the two grids cannot share a CU (one workgroup of either
// fills a CU's registers), so the dispatcher's interleaving decides. Here one grid holds
// both: its first prefix_wg workgroups along x take the prefix items in turn (item
// w, w + W, ...) and then stream a smaller share of the units (the weighted split of
// range_start<true>); the other workgroups are the stream pass's full ranges. A few CUs
// do the matrix work while the rest stream, and the prefix items can be long (few
// pieces). The stream pass leaves the sequences with prefix parts to the combine, which
// runs after this launch as before.

#include "cascade.h"
#include "decode_kernels.h"
#include "prefill_kernels.h"

namespace {

using namespace pkv;

// Stream share of a prefix workgroup, in eighths of a stream workgroup's.
constexpr int kCascadeTailEighths = PKV_CASCADE_TAIL_EIGHTHS;

// Work items of the prefix pass: (chunk, row block, KV head); 128-row blocks below
// head_dim 256, 64-row blocks at 256.
int64_t prefix_items(const PrefillArgs& p, int64_t rows, int head_dim) {
  const int64_t bm = head_dim >= 256 ? PrefillShape<256>::BM : PrefillShape<128>::BM;
  return (rows + bm - 1) / bm * p.nkv * p.n_chunks;
}

template <int DT, int GPW, int HD>
__global__ void __launch_bounds__(512)
cascade_decode_kernel(const DecodeArgs d, const PrefillArgs p, const int prefix_wg,
                      const int items) {
  const int bx = (int)blockIdx.x;
  if (bx < prefix_wg) {
    const int workers = prefix_wg * (int)gridDim.y;
    for (int it = (int)blockIdx.y * prefix_wg + bx; it < items; it += workers) {
      prefill_item<DT, HD, true>(p, it);
      __syncthreads();  // the item's merge used the rings the next item's loads fill
    }
    if (d.num_wg == d.full_wg) return;  // no stream share for prefix workgroups
    decode_mfma_body<DT, GPW, true, HD, false, true, true>(d, d.full_wg + bx, (int)blockIdx.y);
    return;
  }
  decode_mfma_body<DT, GPW, true, HD, false, true, true>(d, bx - prefix_wg, (int)blockIdx.y);
}

template <int DT, int HD>
hipError_t launch_hd(const DecodeArgs& d, PrefillArgs p, int64_t rows, int gpw, int prefix_wg,
                     int ygrid, hipStream_t st) {
  constexpr int BM = PrefillShape<HD>::BM;
  p.row_blocks = (int)((rows + BM - 1) / BM);
  const int64_t items = (int64_t)p.row_blocks * p.nkv * p.n_chunks;
  const int64_t gx = (int64_t)prefix_wg + d.full_wg;
  if (items > 0x7FFFFFFF || gx > 0x7FFFFFFF || prefix_wg < 1 || d.full_wg < 1 ||
      (d.num_wg != d.full_wg && d.num_wg != d.full_wg + prefix_wg))
    return hipErrorInvalidValue;
  const dim3 grid((unsigned)gx, (unsigned)ygrid), block(512);
  const int n = (int)items;
  switch (gpw) {
    case 1:
      hipLaunchKernelGGL((cascade_decode_kernel<DT, 1, HD>), grid, block, 0, st, d, p, prefix_wg, n);
      break;
    case 2:
      hipLaunchKernelGGL((cascade_decode_kernel<DT, 2, HD>), grid, block, 0, st, d, p, prefix_wg, n);
      break;
    case 3:
      hipLaunchKernelGGL((cascade_decode_kernel<DT, 3, HD>), grid, block, 0, st, d, p, prefix_wg, n);
      break;
    default:
      hipLaunchKernelGGL((cascade_decode_kernel<DT, 4, HD>), grid, block, 0, st, d, p, prefix_wg, n);
      break;
  }
  return hipGetLastError();
}

}  // namespace

namespace pkv {

bool cascade_one_launch_shape(int kv_dtype, int head_dim, int block_size, int batch,
                              int waves_per_wg) {
  return (kv_dtype == PKV_BF16 || kv_dtype == PKV_F16) && (head_dim == 64 || head_dim == 128) &&
         PKV_DECODE_USE_MFMA && block_size >= 16 && (block_size & (block_size - 1)) == 0 &&
         batch > kWave && batch <= kLdsBatch && waves_per_wg == 8;
}

hipError_t launch_cascade(const DecodeArgs& d, const PrefillArgs& p, int64_t rows, int kv_dtype,
                          int head_dim, int gpw, int prefix_wg, int ygrid, hipStream_t st) {
  if (!cascade_one_launch_shape(kv_dtype, head_dim, d.bs, d.batch, 8) || gpw < 1 || gpw > 4 ||
      p.bs_shift < 0)
    return hipErrorInvalidValue;
  if (kv_dtype == PKV_BF16)
    return head_dim == 64 ? launch_hd<PKV_BF16, 64>(d, p, rows, gpw, prefix_wg, ygrid, st)
                          : launch_hd<PKV_BF16, 128>(d, p, rows, gpw, prefix_wg, ygrid, st);
  return head_dim == 64 ? launch_hd<PKV_F16, 64>(d, p, rows, gpw, prefix_wg, ygrid, st)
                        : launch_hd<PKV_F16, 128>(d, p, rows, gpw, prefix_wg, ygrid, st);
}

}  // namespace pkv

extern "C" {

int32_t pkv_cascade_one_launch(int kv_dtype, int32_t head_dim, int32_t num_heads,
                               int32_t num_kv_heads, int32_t block_size, int32_t batch) {
  return cascade_prefix_wg(kv_dtype, head_dim, num_heads, num_kv_heads, block_size, batch, 0, 1,
                           0) > 0;
}

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
                       int32_t prefix_workgroups, void* stream) {
  if (!prefix_out || !prefix_lse || !prefix_row) return PKV_E_NULL;
  if (prefix_parts <= 0 || num_heads <= 0 || head_dim <= 0) return PKV_E_SHAPE;
  // The prefix pass: non-causal chunks over the shared blocks, fp32 parts [rows, nh, hd]
  // and their log2 normalisers.
  PrefillArgs p;
  int64_t rows = 0;
  const int st = prefill_args(&p, &rows, prefix_out, PKV_F32, (int64_t)num_heads * head_dim,
                              head_dim, q, q_stride_b, q_stride_h, k_cache, v_cache, kv_dtype,
                              kv_stride_slot, kv_stride_head, num_slots, prefix_tables,
                              prefix_table_stride, prefix_width, prefix_ctx, prefix_cu_q,
                              prefix_chunks, prefix_max_queries, num_heads, num_kv_heads,
                              head_dim, block_size, scale, 0, prefix_q_rows, prefix_lse);
  if (st < 0) return st;
  // An empty prefix layout (no chunks or no queries) writes no parts, yet the merge
  // would read prefix_parts of them for every sequence with a prefix row: refused.
  if (st == 1) return PKV_E_SHAPE;
  const int64_t items = prefix_items(p, rows, head_dim);
  const int wg = cascade_prefix_wg(kv_dtype, head_dim, num_heads, num_kv_heads, block_size, batch,
                                   num_workgroups, items, prefix_workgroups);
  if (wg > 0) {
    const CascadeLaunch one{&p, rows, wg, 8, kCascadeTailEighths};
    return decode_ex(out, out_dtype, out_stride_b, out_stride_h, q, q_stride_b, q_stride_h,
                     k_cache, v_cache, kv_dtype, kv_stride_slot, kv_stride_head, num_slots,
                     block_tables, table_stride, max_blocks, context_lens, batch, num_heads,
                     num_kv_heads, head_dim, block_size, scale, num_workgroups, workspace,
                     workspace_bytes, first_block, lse, prefix_out, prefix_lse, prefix_row,
                     prefix_parts, prefix_stride, stream, &one, false);
  }
  // Two launches: the prefix pass, then the stream pass (whose arguments are checked
  // before either launches).
  const int bad = decode_ex(out, out_dtype, out_stride_b, out_stride_h, q, q_stride_b,
                            q_stride_h, k_cache, v_cache, kv_dtype, kv_stride_slot,
                            kv_stride_head, num_slots, block_tables, table_stride, max_blocks,
                            context_lens, batch, num_heads, num_kv_heads, head_dim, block_size,
                            scale, num_workgroups, workspace, workspace_bytes, first_block, lse,
                            prefix_out, prefix_lse, prefix_row, prefix_parts, prefix_stride,
                            stream, nullptr, true);
  if (bad) return bad;
  {
    const int e = pkv_paged_prefill_ex(
        prefix_out, PKV_F32, (int64_t)num_heads * head_dim, head_dim, q, q_stride_b, q_stride_h,
        k_cache, v_cache, kv_dtype, kv_stride_slot, kv_stride_head, num_slots, prefix_tables,
        prefix_table_stride, prefix_width, prefix_ctx, prefix_cu_q, prefix_chunks,
        prefix_max_queries, num_heads, num_kv_heads, head_dim, block_size, scale, 0,
        prefix_q_rows, prefix_lse, stream);
    if (e) return e;
  }
  return pkv_paged_decode_ex(out, out_dtype, out_stride_b, out_stride_h, q, q_stride_b,
                             q_stride_h, k_cache, v_cache, kv_dtype, kv_stride_slot,
                             kv_stride_head, num_slots, block_tables, table_stride, max_blocks,
                             context_lens, batch, num_heads, num_kv_heads, head_dim, block_size,
                             scale, num_workgroups, workspace, workspace_bytes, first_block, lse,
                             prefix_out, prefix_lse, prefix_row, prefix_parts, prefix_stride,
                             stream);
}

}  // extern "C"
