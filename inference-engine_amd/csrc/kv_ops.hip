// kv_ops.hip -- slot-mapped KV append, block copy (copy-on-write) and the device-side
// decode slot mapping, plus the ABI version and status strings of include/paged_kv.h.

#include "common.h"

namespace {

using namespace pkv;

// ---------------------------------------------------------------------------------
// KV append.
// ---------------------------------------------------------------------------------

template <int DIN, int DOUT, int VEC>
__global__ void __launch_bounds__(256)
kv_append_kernel(typename Elt<DOUT>::S* __restrict__ k_pool,
                 typename Elt<DOUT>::S* __restrict__ v_pool, int64_t ps_slot,
                 int64_t ps_head, int64_t num_slots,
                 const typename Elt<DIN>::S* __restrict__ k_new, int64_t ks_tok,
                 int64_t ks_head, const typename Elt<DIN>::S* __restrict__ v_new,
                 int64_t vs_tok, int64_t vs_head, const int64_t* __restrict__ slots,
                 int64_t n_tokens, int nkv, int hd) {
  using SI = typename Elt<DIN>::S;
  using SO = typename Elt<DOUT>::S;
  const int chunks = hd / VEC;
  const int64_t per_tok = (int64_t)2 * nkv * chunks;
  const int64_t total = n_tokens * per_tok;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t tok = i / per_tok;
    int r = (int)(i - tok * per_tok);
    const int c = r % chunks;
    r /= chunks;
    const int head = r % nkv;
    const bool is_v = r >= nkv;
    const int64_t slot = slots[tok];
    if (slot < 0 || slot >= num_slots) continue;
    const SI* src = is_v ? v_new + tok * vs_tok + head * vs_head
                         : k_new + tok * ks_tok + head * ks_head;
    SO* dst = (is_v ? v_pool : k_pool) + slot * ps_slot + head * ps_head;
    src += c * VEC;
    dst += c * VEC;
    if constexpr (DIN == DOUT && VEC * sizeof(SI) % 16 == 0) {
#pragma unroll
      for (int j = 0; j < (int)(VEC * sizeof(SI) / 16); ++j)
        reinterpret_cast<uint4*>(dst)[j] = reinterpret_cast<const uint4*>(src)[j];
    } else if constexpr (DIN == DOUT) {
#pragma unroll
      for (int j = 0; j < VEC; ++j) dst[j] = src[j];
    } else {
      SI in[VEC];
      SO o[VEC];
#pragma unroll
      for (int j = 0; j < VEC; ++j) in[j] = src[j];
#pragma unroll
      for (int j = 0; j < VEC; ++j) o[j] = Elt<DOUT>::from_f32(Elt<DIN>::to_f32(in[j]));
#pragma unroll
      for (int j = 0; j < VEC; ++j) dst[j] = o[j];
    }
  }
}

// ---------------------------------------------------------------------------------
// Block copy (copy-on-write). One workgroup moves up to 32 KiB of one (pair, layer,
// pool) block: 8 independent 16-byte loads per thread, then the 8 stores.
// ---------------------------------------------------------------------------------

// Non-temporal store of one copy element (16-byte elements through the native vector type).
template <typename U> __device__ __forceinline__ void stream_store(U* p, const U& v) {
  if constexpr (sizeof(U) == 16)
    __builtin_nontemporal_store(__builtin_bit_cast(u32x4, v), reinterpret_cast<u32x4*>(p));
  else
    __builtin_nontemporal_store(v, p);
}

template <typename U>
__global__ void __launch_bounds__(256)
copy_blocks_kernel(char* __restrict__ k_pool, char* __restrict__ v_pool,
                   int64_t layer_stride_bytes, int64_t block_bytes, int64_t num_blocks,
                   const int64_t* __restrict__ mapping) {
  constexpr int kUnroll = 8, kThreads = 256;
  // Grid (chunks, 2 x layers, pairs): consecutive workgroups walk the (layer, K/V)
  // planes first, so with workgroups dealt round-robin to the 8 XCDs every pair of one
  // plane lands on the same XCD, whose L2 then serves a source block shared by many
  // pairs (copy-on-write of one prefix block) to all of them.
  const int64_t pair = blockIdx.z;
  const int layer = blockIdx.y >> 1;
  char* pool = (blockIdx.y & 1) ? v_pool : k_pool;
  const int64_t src = mapping[2 * pair], dst = mapping[2 * pair + 1];
  if (src < 0 || src >= num_blocks || dst < 0 || dst >= num_blocks) return;
  const int64_t n = block_bytes / (int64_t)sizeof(U);
  const U* s = reinterpret_cast<const U*>(pool + layer * layer_stride_bytes + src * block_bytes);
  U* d = reinterpret_cast<U*>(pool + layer * layer_stride_bytes + dst * block_bytes);
  constexpr int64_t span = (int64_t)kThreads * kUnroll;
  for (int64_t base = (int64_t)blockIdx.x * span + threadIdx.x; base < n;
       base += (int64_t)gridDim.x * span) {
    U r[kUnroll];
#pragma unroll
    for (int j = 0; j < kUnroll; ++j) {
      const int64_t e = base + j * kThreads;
      r[j] = e < n ? s[e] : U{};
    }
#pragma unroll
    for (int j = 0; j < kUnroll; ++j) {  // streaming stores: the copies are not read back here
      const int64_t e = base + j * kThreads;
      if (e < n) stream_store(d + e, r[j]);
    }
  }
}

// ---------------------------------------------------------------------------------
// Decode slot mapping on the device: the slot of each sequence's newest token,
// table[(n-1) / bs] * bs + (n-1) % bs with n = context_lens[b] (the token appended this
// step is counted). -1 (skipped by the append) when n < 1, when its block lies past
// max_blocks, or when the slot falls outside the pool.
// ---------------------------------------------------------------------------------

__global__ void __launch_bounds__(256)
decode_slots_kernel(int64_t* __restrict__ slots, const int32_t* __restrict__ tables,
                    int64_t table_stride, int32_t max_blocks, const int32_t* __restrict__ ctx,
                    int32_t batch, int32_t bs, int64_t num_slots) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= batch) return;
  const int n = ctx[b];
  int64_t slot = -1;
  if (n >= 1) {
    const int blk = (n - 1) / bs;
    if (blk < max_blocks) {
      const int64_t s = (int64_t)tables[(int64_t)b * table_stride + blk] * bs + (n - 1) % bs;
      if (s >= 0 && s < num_slots) slot = s;
    }
  }
  slots[b] = slot;
}

// ---------------------------------------------------------------------------------
// Host-side dispatch.
// ---------------------------------------------------------------------------------

template <int DIN, int DOUT, int VEC>
hipError_t launch_append(void* kp, void* vp, int64_t ps_slot, int64_t ps_head,
                         int64_t num_slots, const void* kn, int64_t ks_tok, int64_t ks_head,
                         const void* vn, int64_t vs_tok, int64_t vs_head,
                         const int64_t* slots, int64_t n_tokens, int nkv, int hd,
                         hipStream_t st) {
  const int64_t total = n_tokens * 2 * nkv * (hd / VEC);
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65535 * 8) blocks = 65535 * 8;
  hipLaunchKernelGGL((kv_append_kernel<DIN, DOUT, VEC>), dim3((unsigned)blocks), dim3(256), 0,
                     st, (typename Elt<DOUT>::S*)kp, (typename Elt<DOUT>::S*)vp, ps_slot,
                     ps_head, num_slots, (const typename Elt<DIN>::S*)kn, ks_tok, ks_head,
                     (const typename Elt<DIN>::S*)vn, vs_tok, vs_head, slots, n_tokens, nkv,
                     hd);
  return hipGetLastError();
}

template <int DIN, int DOUT>
hipError_t append_vec_or_scalar(bool vec, void* kp, void* vp, int64_t ps_slot,
                                int64_t ps_head, int64_t num_slots, const void* kn,
                                int64_t ks_tok, int64_t ks_head, const void* vn,
                                int64_t vs_tok, int64_t vs_head, const int64_t* slots,
                                int64_t n_tokens, int nkv, int hd, hipStream_t st) {
  if (vec)
    return launch_append<DIN, DOUT, 8>(kp, vp, ps_slot, ps_head, num_slots, kn, ks_tok,
                                       ks_head, vn, vs_tok, vs_head, slots, n_tokens, nkv,
                                       hd, st);
  return launch_append<DIN, DOUT, 1>(kp, vp, ps_slot, ps_head, num_slots, kn, ks_tok, ks_head,
                                     vn, vs_tok, vs_head, slots, n_tokens, nkv, hd, st);
}

template <int DIN>
hipError_t append_out(int dout, bool vec, void* kp, void* vp, int64_t ps_slot,
                      int64_t ps_head, int64_t num_slots, const void* kn, int64_t ks_tok,
                      int64_t ks_head, const void* vn, int64_t vs_tok, int64_t vs_head,
                      const int64_t* slots, int64_t n_tokens, int nkv, int hd,
                      hipStream_t st) {
  switch (dout) {
    case PKV_F32:
      return append_vec_or_scalar<DIN, PKV_F32>(vec, kp, vp, ps_slot, ps_head, num_slots, kn,
                                                ks_tok, ks_head, vn, vs_tok, vs_head, slots,
                                                n_tokens, nkv, hd, st);
    case PKV_F16:
      return append_vec_or_scalar<DIN, PKV_F16>(vec, kp, vp, ps_slot, ps_head, num_slots, kn,
                                                ks_tok, ks_head, vn, vs_tok, vs_head, slots,
                                                n_tokens, nkv, hd, st);
    default:
      return append_vec_or_scalar<DIN, PKV_BF16>(vec, kp, vp, ps_slot, ps_head, num_slots,
                                                 kn, ks_tok, ks_head, vn, vs_tok, vs_head,
                                                 slots, n_tokens, nkv, hd, st);
  }
}

}  // namespace

extern "C" {

int pkv_abi_version(void) { return 5; }

const char* pkv_status_string(int status) {
  switch (status) {
    case 0: return "ok";
    case PKV_E_DTYPE: return "unsupported dtype";
    case PKV_E_SHAPE: return "unsupported shape (head_dim, group size, block size or sizes)";
    case PKV_E_ALIGN: return "pointer or stride not aligned for 16-byte access";
    case PKV_E_WORKSPACE: return "split-K workspace missing or too small";
    case PKV_E_NULL: return "required pointer is NULL";
    case PKV_E_HIP: return "HIP device query failed (no usable GPU?)";
    case PKV_E_SCRATCH: return "the call needs more scratch than the no-alloc entry point holds";
    default: return status > 0 ? hipGetErrorString((hipError_t)status) : "unknown error";
  }
}

int pkv_kv_append(void* k_pool, void* v_pool, int pool_dtype, int64_t pool_stride_slot,
                  int64_t pool_stride_head, int64_t num_slots, const void* k_new,
                  int64_t k_stride_tok, int64_t k_stride_head, const void* v_new,
                  int64_t v_stride_tok, int64_t v_stride_head, int new_dtype,
                  const int64_t* slots, int64_t n_tokens, int32_t num_kv_heads,
                  int32_t head_dim, void* stream) {
  if (!valid_dtype(pool_dtype) || !valid_dtype(new_dtype)) return PKV_E_DTYPE;
  if (n_tokens < 0 || num_kv_heads <= 0 || head_dim <= 0 || num_slots < 0) return PKV_E_SHAPE;
  if (n_tokens == 0) return 0;
  if (!k_pool || !v_pool || !k_new || !v_new || !slots) return PKV_E_NULL;
  // 8-element vectors need every row start 8-element aligned and 16-byte aligned bases.
  const bool vec = head_dim % 8 == 0 && pool_stride_slot % 8 == 0 &&
                   pool_stride_head % 8 == 0 && k_stride_tok % 8 == 0 &&
                   k_stride_head % 8 == 0 && v_stride_tok % 8 == 0 &&
                   v_stride_head % 8 == 0 && aligned16(k_pool) && aligned16(v_pool) &&
                   aligned16(k_new) && aligned16(v_new);
  hipStream_t st = (hipStream_t)stream;
  hipError_t e;
  switch (new_dtype) {
    case PKV_F32:
      e = append_out<PKV_F32>(pool_dtype, vec, k_pool, v_pool, pool_stride_slot,
                              pool_stride_head, num_slots, k_new, k_stride_tok, k_stride_head,
                              v_new, v_stride_tok, v_stride_head, slots, n_tokens,
                              num_kv_heads, head_dim, st);
      break;
    case PKV_F16:
      e = append_out<PKV_F16>(pool_dtype, vec, k_pool, v_pool, pool_stride_slot,
                              pool_stride_head, num_slots, k_new, k_stride_tok, k_stride_head,
                              v_new, v_stride_tok, v_stride_head, slots, n_tokens,
                              num_kv_heads, head_dim, st);
      break;
    default:
      e = append_out<PKV_BF16>(pool_dtype, vec, k_pool, v_pool, pool_stride_slot,
                               pool_stride_head, num_slots, k_new, k_stride_tok,
                               k_stride_head, v_new, v_stride_tok, v_stride_head, slots,
                               n_tokens, num_kv_heads, head_dim, st);
  }
  return (int)e;
}

int pkv_copy_blocks(void* k_pool, void* v_pool, int64_t layer_stride_bytes,
                    int32_t num_layers, int64_t block_bytes, int64_t num_blocks,
                    const int64_t* block_mapping, int64_t n_pairs, void* stream) {
  if (num_layers < 0 || block_bytes <= 0 || num_blocks < 0 || n_pairs < 0) return PKV_E_SHAPE;
  if (n_pairs == 0 || num_layers == 0) return 0;
  if (!k_pool || !v_pool || !block_mapping) return PKV_E_NULL;
  if (n_pairs > 65535 || num_layers > 32767) return PKV_E_SHAPE;
  hipStream_t st = (hipStream_t)stream;
  const dim3 block(256);
  auto grid_for = [&](int64_t unit) {
    const int64_t n = block_bytes / unit;
    int64_t gx = (n + 256 * 8 - 1) / (256 * 8);
    if (gx > 65535) gx = 65535;
    return dim3((unsigned)gx, (unsigned)(2 * num_layers), (unsigned)n_pairs);
  };
  const bool a16 = aligned16(k_pool) && aligned16(v_pool) && layer_stride_bytes % 16 == 0;
  if (a16 && block_bytes % 16 == 0) {
    hipLaunchKernelGGL(copy_blocks_kernel<uint4>, grid_for(16), block, 0, st, (char*)k_pool,
                       (char*)v_pool, layer_stride_bytes, block_bytes, num_blocks,
                       block_mapping);
  } else if (((uintptr_t)k_pool & 3) == 0 && ((uintptr_t)v_pool & 3) == 0 &&
             layer_stride_bytes % 4 == 0 && block_bytes % 4 == 0) {
    hipLaunchKernelGGL(copy_blocks_kernel<uint32_t>, grid_for(4), block, 0, st, (char*)k_pool,
                       (char*)v_pool, layer_stride_bytes, block_bytes, num_blocks,
                       block_mapping);
  } else {
    hipLaunchKernelGGL(copy_blocks_kernel<uint8_t>, grid_for(1), block, 0, st, (char*)k_pool,
                       (char*)v_pool, layer_stride_bytes, block_bytes, num_blocks,
                       block_mapping);
  }
  return (int)hipGetLastError();
}

int pkv_decode_slots(int64_t* slots, const int32_t* block_tables, int64_t table_stride,
                     int32_t max_blocks, const int32_t* context_lens, int32_t batch,
                     int32_t block_size, int64_t num_slots, void* stream) {
  if (batch < 0 || max_blocks < 0 || block_size <= 0 || num_slots < 0) return PKV_E_SHAPE;
  if (batch == 0) return 0;
  if (!slots || !context_lens || (max_blocks > 0 && !block_tables)) return PKV_E_NULL;
  hipLaunchKernelGGL(decode_slots_kernel, dim3((unsigned)((batch + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, slots, block_tables, table_stride, max_blocks,
                     context_lens, batch, block_size, num_slots);
  return (int)hipGetLastError();
}

}  // extern "C"
