// common.h -- what the gfx950 kernels of the paged-KV hot path share: element types
// and conversions, 16-byte vector loads and stores, cross-lane reductions (DPP,
// permlane), the compile-time tuning knobs, and the host-side argument checks. The
// kernels themselves live in kv_ops.hip (append, block copy, decode slots),
// decode_kernels.h (split-K paged decode and its combine; launched by decode.hip),
// prefill_kernels.h (chunked prefill on the matrix cores; launched by prefill.hip),
// cascade.hip (cascade decode's two passes in one launch) and fused.hip (RMSNorm tail,
// RoPE, SiLU x up); the C ABI is include/paged_kv.h.
//
// Written for CDNA4 wave64: 16-byte global loads, DPP row reductions, v_exp_f32 for
// the softmax (exp2 with log2(e) folded into the query scale), fp32 accumulation.

#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "paged_kv.h"

namespace pkv {

constexpr int kWave = 64;

// Tuning knobs (compile-time; the defaults are the measured best on MI355X).
#ifndef PKV_DECODE_WAVES_PER_WG
#define PKV_DECODE_WAVES_PER_WG 8
#endif
#ifndef PKV_DECODE_NLOAD_MAX
#define PKV_DECODE_NLOAD_MAX 4
#endif
#ifndef PKV_DECODE_STREAM_LOADS
#define PKV_DECODE_STREAM_LOADS 1
#endif
#ifndef PKV_DECODE_USE_MFMA
#define PKV_DECODE_USE_MFMA 1
#endif
#ifndef PKV_DECODE_PREFETCH
#define PKV_DECODE_PREFETCH 1
#endif
#ifndef PKV_DECODE_COMBINE_CHUNK
#define PKV_DECODE_COMBINE_CHUNK 4
#endif
// Accumulator rows per load batch of the combine after a one-launch cascade, where
// every (sequence, head) also folds a prefix part: 2 (measured at config 3: 110.5-110.9
// against 111.1-111.3 µs with 4, 113.6 with 8).
#ifndef PKV_CASCADE_COMBINE_CHUNK
#define PKV_CASCADE_COMBINE_CHUNK 2
#endif
#ifndef PKV_DECODE_COMBINE_SPLIT_PAIRS
#define PKV_DECODE_COMBINE_SPLIT_PAIRS 1024
#endif
// 1: the MFMA stream-K decode pass at head_dim 64 runs P.V on the matrix cores; 0: on
// the VALU.
#ifndef PKV_DECODE_PV_MFMA
#define PKV_DECODE_PV_MFMA 1
#endif
// One-launch cascade: the share of the unit stream each prefix workgroup takes after its
// prefix items, in eighths of a stream workgroup's share (measured at config 3: 3 against
// 1, 2, 4 and 5; 2 had been best before the prefix items got faster).
#ifndef PKV_CASCADE_TAIL_EIGHTHS
#define PKV_CASCADE_TAIL_EIGHTHS 3
#endif
#ifndef PKV_PREFILL_SWZ
#define PKV_PREFILL_SWZ 1
#endif

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// 16-byte K/V load. Streaming (non-temporal) by default: each K/V row is read once per
// layer-step, so it should not displace reusable lines in L2 and the last-level cache.
__device__ __forceinline__ uint4 load_kv16(const void* p) {
#if PKV_DECODE_STREAM_LOADS
  const u32x4 x = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(x.x, x.y, x.z, x.w);
#else
  return *reinterpret_cast<const uint4*>(p);
#endif
}

// ---------------------------------------------------------------------------------
// Element types. 16-bit types are stored as raw uint16_t bits.
// ---------------------------------------------------------------------------------

template <int DT> struct Elt;
template <> struct Elt<PKV_F32> {
  using S = float;
  __device__ static float to_f32(S x) { return x; }
  __device__ static S from_f32(float f) { return f; }
};
template <> struct Elt<PKV_F16> {
  using S = uint16_t;
  __device__ static float to_f32(S x) { return (float)__builtin_bit_cast(_Float16, x); }
  // v_cvt_f16_f32: round to nearest even, as torch's float -> half on the GPU. The empty
  // asm pins f as an fp32 register value: without it the compiler may fuse the producing
  // multiply with the conversion (v_fma_mixlo_f16, one rounding of the exact product),
  // which differs in the last bit from rounding the fp32 result as torch's .to() does.
  __device__ static S from_f32(float f) {
    __asm__ volatile("" : "+v"(f));
    return __builtin_bit_cast(uint16_t, (_Float16)f);
  }
};
template <> struct Elt<PKV_BF16> {
  using S = uint16_t;
  __device__ static float to_f32(S x) { return __uint_as_float(uint32_t(x) << 16); }
  // IEEE round to nearest even on the upper 16 bits; NaN becomes the canonical quiet
  // NaN 0x7FC0, which is what torch produces for float -> bfloat16.
  __device__ static S from_f32(float f) {
    if (f != f) return 0x7FC0;
    uint32_t u = __float_as_uint(f);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
  }
};

// 16-byte chunk -> floats. Returns the number of elements (8 for 16-bit, 4 for fp32).
template <int DT> __device__ __forceinline__ void unpack16(const uint4& r, float* f);
template <> __device__ __forceinline__ void unpack16<PKV_BF16>(const uint4& r, float* f) {
  const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(w[i] << 16);
    f[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
  }
}
template <> __device__ __forceinline__ void unpack16<PKV_F16>(const uint4& r, float* f) {
  const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[i] & 0xFFFFu));
    f[2 * i + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[i] >> 16));
  }
}
template <> __device__ __forceinline__ void unpack16<PKV_F32>(const uint4& r, float* f) {
  f[0] = __uint_as_float(r.x);
  f[1] = __uint_as_float(r.y);
  f[2] = __uint_as_float(r.z);
  f[3] = __uint_as_float(r.w);
}

template <int DT> constexpr int vec16() { return DT == PKV_F32 ? 4 : 8; }

// Store n (= 4 or 8) floats as out dtype DTO at p (aligned to the vector size).
template <int DTO, int N> __device__ __forceinline__ void store_vec(void* p, const float* f) {
  if constexpr (DTO == PKV_F32) {
#pragma unroll
    for (int i = 0; i < N; i += 4)
      reinterpret_cast<float4*>(p)[i / 4] = make_float4(f[i], f[i + 1], f[i + 2], f[i + 3]);
  } else {
    uint32_t w[N / 2];
#pragma unroll
    for (int i = 0; i < N / 2; ++i)
      w[i] = (uint32_t)Elt<DTO>::from_f32(f[2 * i]) |
             ((uint32_t)Elt<DTO>::from_f32(f[2 * i + 1]) << 16);
    if constexpr (N == 8) {
      *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
    } else {
      *reinterpret_cast<uint2*>(p) = make_uint2(w[0], w[1]);
    }
  }
}

// ---------------------------------------------------------------------------------
// Cross-lane helpers (wave64).
// ---------------------------------------------------------------------------------

template <int CTRL> __device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}
constexpr int kQuadXor1 = 0xB1;     // quad_perm [1,0,3,2]
constexpr int kQuadXor2 = 0x4E;     // quad_perm [2,3,0,1]
constexpr int kRowHalfMirror = 0x141;
constexpr int kRowMirror = 0x140;
constexpr int kRowRor8 = 0x128;  // rotate by 8 within each 16-lane row: lane c <-> c ^ 8

// Sum over aligned groups of W lanes; every lane of a group gets the group's sum.
// After the two quad steps the value is uniform inside each quad, so the half-mirror
// (lane i <-> 7-i) pairs each quad with the other quad of its 8-lane half exactly as an
// xor-4 would; the same argument makes the row mirror an xor-8.
template <int W> __device__ __forceinline__ float group_sum(float x) {
  if constexpr (W >= 2) x += dpp<kQuadXor1>(x);
  if constexpr (W >= 4) x += dpp<kQuadXor2>(x);
  if constexpr (W >= 8) x += dpp<kRowHalfMirror>(x);
  if constexpr (W >= 16) x += dpp<kRowMirror>(x);
  if constexpr (W >= 32) x += __shfl_xor(x, 16);
  if constexpr (W >= 64) x += __shfl_xor(x, 32);
  return x;
}

// Max / sum across groups: lanes l and l ^ m for m = W, 2W, ..., 32, where the value is
// already uniform inside each aligned group of W lanes (so mirrors stand in for xors).
template <int W> __device__ __forceinline__ float across_max(float x) {
  if constexpr (W <= 1) x = fmaxf(x, dpp<kQuadXor1>(x));
  if constexpr (W <= 2) x = fmaxf(x, dpp<kQuadXor2>(x));
  if constexpr (W <= 4) x = fmaxf(x, dpp<kRowHalfMirror>(x));
  if constexpr (W <= 8) x = fmaxf(x, dpp<kRowMirror>(x));
  if constexpr (W <= 16) x = fmaxf(x, __shfl_xor(x, 16));
  if constexpr (W <= 32) x = fmaxf(x, __shfl_xor(x, 32));
  return x;
}
template <int W> __device__ __forceinline__ float across_sum(float x) {
  if constexpr (W <= 1) x += dpp<kQuadXor1>(x);
  if constexpr (W <= 2) x += dpp<kQuadXor2>(x);
  if constexpr (W <= 4) x += dpp<kRowHalfMirror>(x);
  if constexpr (W <= 8) x += dpp<kRowMirror>(x);
  if constexpr (W <= 16) x += __shfl_xor(x, 16);
  if constexpr (W <= 32) x += __shfl_xor(x, 32);
  return x;
}
// Exact xor-butterfly sum over lanes l ^ m, m = W..32 (values differ inside groups).
template <int W> __device__ __forceinline__ float across_sum_exact(float x) {
#pragma unroll
  for (int m = W; m < kWave; m <<= 1) x += __shfl_xor(x, m);
  return x;
}

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;  // LDS operand of ds_read_tr16_b64

// Eight fp32 probabilities as the P operand fragment of a 16x16x32 MFMA (four dwords of
// 16-bit pairs) in the K/V type. bf16: hi = bf16(p) (v_cvt_pk_bf16_f32, round to nearest
// even) plus lo = bf16(p - hi), two MFMAs -- p - hi is exact, and one bf16 rounding of P
// (8 significant bits) misses a 2e-3 bar on peaked attention. fp16: one rounding (11
// bits), lo zero -- or, with LO16, lo = fp16(p - hi) as well (22 bits: results then do
// not depend on where a context is cut into pieces, beyond fp32 rounding).
template <int DT, bool LO16 = false>
__device__ __forceinline__ void pack_p8(const float* p, u32x4& hi, u32x4& lo) {
  if constexpr (DT == PKV_BF16) {
    typedef __bf16 v2 __attribute__((ext_vector_type(2)));
    uint32_t h[4], l[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      h[i] = __builtin_bit_cast(uint32_t, v2{(__bf16)p[2 * i], (__bf16)p[2 * i + 1]});
      // the empty asm keeps h[i] one value (no second conversion to rebuild its low half);
      // on h[i] itself, so no copy of it is made
      __asm__("" : "+v"(h[i]));
      const float r0 = p[2 * i] - __uint_as_float(h[i] << 16);
      const float r1 = p[2 * i + 1] - __uint_as_float(h[i] & 0xFFFF0000u);
      l[i] = __builtin_bit_cast(uint32_t, v2{(__bf16)r0, (__bf16)r1});
    }
    hi = u32x4{h[0], h[1], h[2], h[3]};
    lo = u32x4{l[0], l[1], l[2], l[3]};
  } else {
    typedef _Float16 v2 __attribute__((ext_vector_type(2)));
    uint32_t h[4], l[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const v2 hp = v2{(_Float16)p[2 * i], (_Float16)p[2 * i + 1]};
      h[i] = __builtin_bit_cast(uint32_t, hp);
      if constexpr (LO16)  // p - hi is exact in fp32
        l[i] = __builtin_bit_cast(uint32_t, v2{(_Float16)(p[2 * i] - (float)hp[0]),
                                               (_Float16)(p[2 * i + 1] - (float)hp[1])});
    }
    hi = u32x4{h[0], h[1], h[2], h[3]};
    lo = u32x4{l[0], l[1], l[2], l[3]};
  }
}

// Lane h of every 16-lane row, broadcast to its row (DPP row_newbcast).
template <int H> __device__ __forceinline__ float row_bcast(float x) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x150 + H, 0xF, 0xF, false));
}
__device__ __forceinline__ float row_bcast(float x, int h) {
  switch (h) {
    case 0: return row_bcast<0>(x);
    case 1: return row_bcast<1>(x);
    case 2: return row_bcast<2>(x);
    default: return row_bcast<3>(x);
  }
}

// Reductions over lanes l, l^16, l^32, l^48 (the four rows of a column).
__device__ __forceinline__ float rows_max(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float rows_sum(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

inline int dtype_bytes(int dt) { return dt == PKV_F32 ? 4 : 2; }
inline bool valid_dtype(int dt) { return dt == PKV_F32 || dt == PKV_F16 || dt == PKV_BF16; }

}  // namespace pkv
