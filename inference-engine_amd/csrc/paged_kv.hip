// paged_kv.hip — gfx950 kernels for the paged-KV hot path behind the C ABI of
// include/paged_kv.h: slot-mapped KV append, block copy, and split-K paged decode
// attention with its combine pass.
//
// Written for CDNA4 wave64: 16-byte global loads, DPP row reductions, v_exp_f32 for
// the softmax (exp2 with log2(e) folded into the query scale), fp32 accumulation.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "paged_kv.h"

namespace {

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
#ifndef PKV_PREFILL_SETPRIO
#define PKV_PREFILL_SETPRIO 0
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

template <typename U>
__global__ void __launch_bounds__(256)
copy_blocks_kernel(char* __restrict__ k_pool, char* __restrict__ v_pool,
                   int64_t layer_stride_bytes, int64_t block_bytes, int64_t num_blocks,
                   const int64_t* __restrict__ mapping) {
  constexpr int kUnroll = 8, kThreads = 256;
  const int64_t pair = blockIdx.y;
  const int layer = blockIdx.z >> 1;
  char* pool = (blockIdx.z & 1) ? v_pool : k_pool;
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
    for (int j = 0; j < kUnroll; ++j) {
      const int64_t e = base + j * kThreads;
      if (e < n) d[e] = r[j];
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
// Paged decode attention: stream-K pass.
//
// The contexts of all sequences are cut into units of TILE tokens (a sequence with an
// empty context owns one unit) and laid end to end, sequence by sequence. The grid has
// exactly as many workgroups along x as the GPU holds at once, and workgroup w takes
// the contiguous unit range [w*U/G, (w+1)*U/G): every CU streams the same number of
// K/V bytes whatever the context lengths, and since workgroups are dealt to the 8 XCDs
// round-robin, so does every XCD. A sequence that lies wholly inside one range gets its
// output written directly; a sequence cut by a range boundary leaves one (m, l, acc)
// record per piece (at most two per workgroup: its first and its last piece), which the
// combine pass merges. Ranges are computed on the device from context_lens, so the
// launch shape depends only on static shapes and one hipGraph serves every length.
//
// One wave = one KV head (and up to GPW of its query heads). A workgroup holds the
// waves of consecutive KV heads over the same unit range, so together they stream each
// block's whole [block_size, nkv, hd] span, which is contiguous. Inside a wave a K/V row
// of hd elements is LPT lanes x 16 bytes; one 16-byte load per lane covers TPL = 64/LPT
// tokens, and a tile is NLOAD such loads. The next tile's K and V loads are issued
// before the current tile is reduced.
// ---------------------------------------------------------------------------------

template <int DT, int HD> struct DecodeShape {
  static constexpr int VEC = vec16<DT>();
  static constexpr int LPT = HD / VEC;
  static constexpr int TPL = kWave / LPT;
  static constexpr int NLOAD = (16 / TPL) < 1 ? 1
                               : ((16 / TPL) > PKV_DECODE_NLOAD_MAX ? PKV_DECODE_NLOAD_MAX
                                                                   : 16 / TPL);
  static constexpr int TILE = NLOAD * TPL;
  static_assert(LPT >= 1 && LPT <= kWave, "head_dim out of range");
};

struct DecodeArgs {
  void* out;
  int64_t out_sb, out_sh;
  const void* q;
  int64_t q_sb, q_sh;
  const void* k;
  const void* v;
  int64_t kv_ss, kv_sh, num_slots;
  const int32_t* tables;
  int64_t table_stride;
  int32_t max_blocks;
  const int32_t* ctx;
  int32_t batch, nh, nkv, groups, nsub, bs, bs_shift;  // bs_shift < 0: block_size not pow2
  int32_t unit_tokens;  // TILE of the instantiated kernel
  int32_t num_wg;       // workgroups along x sharing the unit stream
  float scale_log2;     // scale * log2(e)
  int4* desc;           // [batch] per-sequence merge plan (see SeqDesc)
  float* ws_acc;        // [num_wg, 2, nh, HD] partial records
  float* ws_ml;         // [num_wg, 2, nh, 2]   their (max, sum)
  int out_f32;
  const int32_t* first_block;  // [batch] or null: attend from table column first_block[b]
  float* lse;                  // [batch, nh] or null: log2 of each softmax's normaliser
  // Cascade (pre_row non-null): normalised attentions of the same queries over other
  // keys (a shared prefix's pieces), merged into the result by the combine pass. Part k
  // of sequence b is row pre_row[b] + k * pre_stride of pre_o [rows, nh, HD] / pre_lse
  // [rows, nh] (pre_row[b] < 0: none). The stream pass then writes the sequences it
  // finishes to out / lse as fp32 scratch, and the combine pass writes every sequence's
  // result to fin (fin_f32: fp32, else DT) and its normaliser to fin_lse (if non-null).
  const float* pre_o;
  const float* pre_lse;
  const int32_t* pre_row;
  int32_t pre_parts;
  int64_t pre_stride;
  void* fin;
  int64_t fin_sb, fin_sh;
  int fin_f32;
  float* fin_lse;
};

// Table column sequence b starts from (a shared prefix handled elsewhere is skipped).
__device__ __forceinline__ int first_blk(const DecodeArgs& a, int b) {
  if (!a.first_block) return 0;
  const int f = a.first_block[b];
  return f < 0 ? 0 : (f > a.max_blocks ? a.max_blocks : f);
}

// Tokens sequence b attends to, clamped: 0 <= n <= (max_blocks - first) * block_size.
// They are positions first * block_size + p, p < n.
__device__ __forceinline__ int clamped_ctx(const DecodeArgs& a, int b) {
  const int fb = first_blk(a, b);
  const int n = a.ctx[b] - fb * a.bs;
  const int cap = (a.max_blocks - fb) * a.bs;
  return n < 0 ? 0 : (n > cap ? cap : n);
}

// Log2 of the softmax normaliser in the kernel's score units (scores x scale x log2 e):
// max + log2(sum of exp2(score - max)); -inf when no key was live.
__device__ __forceinline__ float lse_of(float m, float l) {
  return l > 0.f ? m + __log2f(l) : -INFINITY;
}

// Folds sequence b's prefix parts for head h into a wave's running softmax state (m, l,
// acc), lane holding head dims lane + 64 c (c < DPL; dims >= HD skipped). A part is a
// normalised output O_k with log2 normaliser lse_k, i.e. the state (lse_k, 1, O_k):
// with M the new max, l <- l 2^(m - M) + sum_k 2^(lse_k - M) and likewise acc. Parts
// are loaded eight at a time, every load issued before any is used.
template <int HD, int DPL>
__device__ __forceinline__ void fold_prefix(const DecodeArgs& a, int b, int h, float& m,
                                            float& l, float (&acc)[DPL]) {
  const int r = a.pre_row[b];
  if (r < 0) return;
  const int lane = threadIdx.x & (kWave - 1);
  constexpr int C = 8;
  for (int k0 = 0; k0 < a.pre_parts; k0 += C) {
    float lk[C], x[C][DPL];
#pragma unroll
    for (int jj = 0; jj < C; ++jj) {
      const int k = k0 + jj;
      const bool live = k < a.pre_parts;
      const int64_t row = ((int64_t)r + (int64_t)(live ? k : 0) * a.pre_stride) * a.nh + h;
      lk[jj] = live ? a.pre_lse[row] : -INFINITY;
      const float* p = a.pre_o + row * HD;
#pragma unroll
      for (int c = 0; c < DPL; ++c) x[jj][c] = lane + kWave * c < HD ? p[lane + kWave * c] : 0.f;
    }
    float mn = m;
#pragma unroll
    for (int jj = 0; jj < C; ++jj) mn = fmaxf(mn, lk[jj]);
    const float mref = mn == -INFINITY ? 0.f : mn;  // nothing live yet: weights 0
    const float alpha = __builtin_amdgcn_exp2f(m - mref);
    m = mn;
    l *= alpha;
#pragma unroll
    for (int c = 0; c < DPL; ++c) acc[c] *= alpha;
#pragma unroll
    for (int jj = 0; jj < C; ++jj) {
      const float wj = __builtin_amdgcn_exp2f(lk[jj] - mref);  // dead or empty: 0
      l += wj;
#pragma unroll
      for (int c = 0; c < DPL; ++c) acc[c] = __builtin_fmaf(wj, x[jj][c], acc[c]);
    }
  }
}

__device__ __forceinline__ int units_of(const DecodeArgs& a, int n) {
  return n == 0 ? 1 : (n + a.unit_tokens - 1) / a.unit_tokens;
}

// Wave-wide walk over the unit prefix sums. With target >= 0 returns the sequence b
// that owns unit `target` and its first unit in *ustart; with target < 0 (or past the
// end) returns batch and the total unit count in *ustart. Call from whole waves.
__device__ int find_unit(const DecodeArgs& a, int64_t target, int64_t* ustart) {
  const int lane = threadIdx.x & (kWave - 1);
  int64_t base = 0;
  for (int c0 = 0; c0 < a.batch; c0 += kWave) {
    const int bb = c0 + lane;
    const int cnt = bb < a.batch ? units_of(a, clamped_ctx(a, bb)) : 0;
    int incl = cnt;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
      const int t = __shfl_up(incl, off);
      if (lane >= off) incl += t;
    }
    const int chunk_total = __shfl(incl, kWave - 1);
    if (target >= 0 && target < base + chunk_total) {
      const unsigned long long hit = __ballot(base + incl > target);
      const int l = __ffsll((long long)hit) - 1;
      *ustart = base + __shfl(incl - cnt, l);
      return c0 + l;
    }
    base += chunk_total;
  }
  *ustart = base;
  return a.batch;
}

__device__ __forceinline__ int64_t range_start(int64_t w, int64_t units, int64_t wgs) {
  return w * units / wgs;
}
// The workgroup whose range holds unit u: the largest w with range_start(w) <= u.
__device__ __forceinline__ int64_t wg_of_unit(int64_t u, int64_t units, int64_t wgs) {
  return ((u + 1) * wgs - 1) / units;
}

// Merge plan of one sequence, written by the workgroup that holds its first unit (so
// every sequence gets exactly one, every call): the first workgroup w0 of its pieces,
// the number of workgroups w0..w1 it spans (1: written directly), the record slot its
// piece has in w0, and whether every range is non-empty (units >= workgroups).
__device__ __forceinline__ void write_desc(const DecodeArgs& a, int b, int w, int64_t ub,
                                           int64_t ue, int64_t rs, int64_t total) {
  if (!a.desc) return;
  const int64_t w1 = wg_of_unit(ue - 1, total, a.num_wg);
  a.desc[b] = make_int4(w, (int)(w1 - w + 1), rs < ub ? 1 : 0, total >= a.num_wg ? 1 : 0);
}

template <int DT, int HD, int GPW>
__global__ void __launch_bounds__(512)
paged_decode_stream_kernel(const DecodeArgs a) {
  using Sh = DecodeShape<DT, HD>;
  constexpr int VEC = Sh::VEC, LPT = Sh::LPT, TPL = Sh::TPL, NLOAD = Sh::NLOAD;
  constexpr int TILE = Sh::TILE;
  using S = typename Elt<DT>::S;

  const int lane = threadIdx.x & (kWave - 1);
  const int task = blockIdx.y * (blockDim.x / kWave) + (threadIdx.x / kWave);
  const int kvh = task / a.nsub;
  if (kvh >= a.nkv) return;
  const int h0 = kvh * a.groups + (task - kvh * a.nsub) * GPW;
  const int w = blockIdx.x;

  int64_t total;
  find_unit(a, -1, &total);
  const int64_t rs = range_start(w, total, a.num_wg);
  const int64_t re = range_start(w + 1, total, a.num_wg);
  if (rs >= re) return;
  int64_t ub;
  int b = find_unit(a, rs, &ub);

  const int row = lane / LPT;         // token sub-index inside a load
  const int d0 = (lane % LPT) * VEC;  // this lane's first head_dim element
  const S* kbase = reinterpret_cast<const S*>(a.k) + (int64_t)kvh * a.kv_sh + d0;
  const S* vbase = reinterpret_cast<const S*>(a.v) + (int64_t)kvh * a.kv_sh + d0;

  for (int64_t u = rs; u < re && b < a.batch; ++b) {
    const int n = clamped_ctx(a, b);
    const int64_t ue = ub + units_of(a, n);
    const int64_t seg_end = ue < re ? ue : re;
    const bool whole = (u == ub) && (seg_end == ue);
    const int slot = (u == rs) ? 0 : 1;  // which record a cut piece goes to
    const int t0 = (int)(u - ub) * a.unit_tokens;
    const int t1 = min(n, (int)(seg_end - ub) * a.unit_tokens);
    if (u == ub && task == 0 && lane == 0) write_desc(a, b, w, ub, ue, rs, total);
    u = seg_end;
    ub = ue;

    // Query rows of this wave for sequence b, pre-scaled into the exp2 domain.
    float qf[GPW][VEC];
#pragma unroll
    for (int g = 0; g < GPW; ++g) {
      const S* qp = reinterpret_cast<const S*>(a.q) + b * a.q_sb + (int64_t)(h0 + g) * a.q_sh + d0;
      float t[VEC];
      unpack16<DT>(*reinterpret_cast<const uint4*>(qp), t);
#pragma unroll
      for (int i = 0; i < VEC; ++i) qf[g][i] = t[i] * a.scale_log2;
    }

    // Block ids of up to 64 consecutive blocks starting at cb, one per lane.
    int cb = 0, tbl = 0;
    const int fb = first_blk(a, b);
    auto load_table = [&](int first_block) {
      cb = first_block;
      const int j = cb + lane;
      tbl = j < a.max_blocks - fb ? a.tables[b * a.table_stride + fb + j] : 0;
    };
    auto block_of = [&](int p) { return a.bs_shift >= 0 ? (p >> a.bs_shift) : p / a.bs; };

    // Slot of this lane's token in load i of the tile starting at tb (-1: masked).
    auto slot_of = [&](int tb, int i) -> int64_t {
      const int p = tb + i * TPL + row;
      const int blk = block_of(p);
      const int bid = __shfl(tbl, blk - cb);
      const int off = p - blk * a.bs;
      const int64_t sl = (int64_t)bid * a.bs + off;
      return (p < t1 && sl >= 0 && sl < a.num_slots) ? sl : (int64_t)-1;
    };
    // Issue the K/V loads of the tile at tb (first making sure the table window
    // covers it); bit i of the result: load i holds a live token for this lane.
    auto load_tile = [&](int tb, uint4* kr, uint4* vr) -> unsigned {
      if (tb < t1 && block_of(min(tb + TILE, t1) - 1) - cb >= kWave) load_table(block_of(tb));
      unsigned ok = 0;
#pragma unroll
      for (int i = 0; i < NLOAD; ++i) {
        const int64_t sl = slot_of(tb, i);
        uint4 kk = make_uint4(0, 0, 0, 0), vv = make_uint4(0, 0, 0, 0);
        if (sl >= 0) {
          kk = load_kv16(kbase + sl * a.kv_ss);
          vv = load_kv16(vbase + sl * a.kv_ss);
          ok |= 1u << i;
        }
        kr[i] = kk;
        vr[i] = vv;
      }
      return ok;
    };

    float m[GPW], l[GPW], acc[GPW][VEC];
#pragma unroll
    for (int g = 0; g < GPW; ++g) {
      m[g] = -INFINITY;
      l[g] = 0.f;
#pragma unroll
      for (int i = 0; i < VEC; ++i) acc[g][i] = 0.f;
    }

    if (t0 < t1) {
      load_table(block_of(t0));
      uint4 kc[NLOAD], vc[NLOAD];
      unsigned okc = load_tile(t0, kc, vc);
      for (int tb = t0; tb < t1; tb += TILE) {
        uint4 kn[NLOAD], vn[NLOAD];
        const unsigned okn = load_tile(tb + TILE, kn, vn);  // past t1 every lane is masked

        float sc[NLOAD][GPW];
#pragma unroll
        for (int i = 0; i < NLOAD; ++i) {
          float kf[VEC];
          unpack16<DT>(kc[i], kf);
#pragma unroll
          for (int g = 0; g < GPW; ++g) {
            float d = 0.f;
#pragma unroll
            for (int c = 0; c < VEC; ++c) d = __builtin_fmaf(qf[g][c], kf[c], d);
            sc[i][g] = group_sum<LPT>(d);
          }
        }
#pragma unroll
        for (int g = 0; g < GPW; ++g) {
          float mx = -INFINITY;
#pragma unroll
          for (int i = 0; i < NLOAD; ++i) {
            sc[i][g] = ((okc >> i) & 1u) ? sc[i][g] : -INFINITY;
            mx = fmaxf(mx, sc[i][g]);
          }
          mx = across_max<LPT>(mx);
          const float mn = fmaxf(m[g], mx);
          // While every token so far is masked the max is -inf; exponents are then
          // taken against 0 so exp2(-inf - -inf) never turns the empty state into NaN.
          const float mref = mn == -INFINITY ? 0.f : mn;
          const float alpha = __builtin_amdgcn_exp2f(m[g] - mref);
          m[g] = mn;
          l[g] *= alpha;
#pragma unroll
          for (int c = 0; c < VEC; ++c) acc[g][c] *= alpha;
#pragma unroll
          for (int i = 0; i < NLOAD; ++i) sc[i][g] = __builtin_amdgcn_exp2f(sc[i][g] - mref);
        }
#pragma unroll
        for (int i = 0; i < NLOAD; ++i) {
          float vf[VEC];
          unpack16<DT>(vc[i], vf);
#pragma unroll
          for (int g = 0; g < GPW; ++g) {
            l[g] += sc[i][g];
#pragma unroll
            for (int c = 0; c < VEC; ++c) acc[g][c] = __builtin_fmaf(sc[i][g], vf[c], acc[g][c]);
          }
        }
#pragma unroll
        for (int i = 0; i < NLOAD; ++i) {
          kc[i] = kn[i];
          vc[i] = vn[i];
        }
        okc = okn;
      }
    }

    // Combine the TPL token rows of the wave.
#pragma unroll
    for (int g = 0; g < GPW; ++g) {
      l[g] = across_sum<LPT>(l[g]);
#pragma unroll
      for (int c = 0; c < VEC; ++c) acc[g][c] = across_sum_exact<LPT>(acc[g][c]);
    }

    if (lane < LPT) {
      if (whole) {  // the whole context was in this range: final output directly
#pragma unroll
        for (int g = 0; g < GPW; ++g) {
          // no live token (empty context): 0, the reference oracle's einsum over no keys
          const float inv = l[g] > 0.f ? 1.f / l[g] : 0.f;
          float o[VEC];
#pragma unroll
          for (int c = 0; c < VEC; ++c) o[c] = acc[g][c] * inv;
          const int64_t e = b * a.out_sb + (int64_t)(h0 + g) * a.out_sh + d0;
          if (a.out_f32) store_vec<PKV_F32, VEC>((float*)a.out + e, o);
          else store_vec<DT, VEC>((S*)a.out + e, o);
          if (a.lse && lane == 0) a.lse[(int64_t)b * a.nh + h0 + g] = lse_of(m[g], l[g]);
        }
      } else {
#pragma unroll
        for (int g = 0; g < GPW; ++g) {
          const int64_t rec = ((int64_t)w * 2 + slot) * a.nh + h0 + g;
          store_vec<PKV_F32, VEC>(a.ws_acc + rec * HD + d0, acc[g]);
          if (lane == 0) *reinterpret_cast<float2*>(a.ws_ml + 2 * rec) = make_float2(m[g], l[g]);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------------
// MFMA variant of the stream pass for 16-bit K/V at head_dim 128 (the Llama-3 shapes).
//
// Same stream-K ranges, records and outputs as paged_decode_stream_kernel; only the
// per-tile arithmetic differs. A tile is 16 tokens. Lane l is (col = l % 16, grp =
// l / 16).
//   * Scores on the matrix cores: S[16 tokens x 16 cols] = K_tile . Q^T with four
//     v_mfma_f32_16x16x32 (32 head dims each). A operand: lane (t, g) holds K[token t]
//     dims 32m + 8g .. +8 (one 16-byte load per MFMA); B operand: lane (j, g) holds
//     Q[head j] at the same dims (zero for j >= GPW). Result: lane (j, g) holds the
//     scores of tokens 4g + r (r < 4) for query head j.
//   * Softmax in that layout: per-head max over the 16 tokens with two permlane swaps
//     (v_permlane16/32_swap give {x[l], x[l^16]} / {x[l], x[l^32]}: no LDS trip).
//   * PV on the VALU in fp32: lane (c, g) holds V[token 4g + r] dims 8c .. +8; each
//     head's probabilities reach it with DPP row_newbcast (lane h of each 16-lane row
//     to the whole row), since token 4g + r's score sits in lane (h, g) of that row.
// When block_size is a multiple of 16 a tile lies inside one block: its block id is
// read with v_readlane into a scalar and every lane's address is a fixed offset from it.
// ---------------------------------------------------------------------------------

typedef float f32x4 __attribute__((ext_vector_type(4)));

template <int DT> struct Mfma16x16x32;
template <> struct Mfma16x16x32<PKV_BF16> {
  typedef __bf16 v8 __attribute__((ext_vector_type(8)));
  __device__ static f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8, a),
                                                   __builtin_bit_cast(v8, b), c, 0, 0, 0);
  }
};
template <> struct Mfma16x16x32<PKV_F16> {
  typedef _Float16 v8 __attribute__((ext_vector_type(8)));
  __device__ static f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8, a),
                                                  __builtin_bit_cast(v8, b), c, 0, 0, 0);
  }
};

__device__ __forceinline__ u32x4 load_kv16v(const void* p) {
#if PKV_DECODE_STREAM_LOADS
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
#else
  return *reinterpret_cast<const u32x4*>(p);
#endif
}

template <int DT> __device__ __forceinline__ void unpack16v(u32x4 r, float* f) {
  unpack16<DT>(make_uint4(r.x, r.y, r.z, r.w), f);
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

template <int DT, int GPW, bool FAST>
__global__ void __launch_bounds__(512)
paged_decode_mfma_kernel(const DecodeArgs a) {
  constexpr int HD = 128, TILE = 16;
  static_assert(GPW >= 1 && GPW <= 4, "at most 4 query heads per wave");
  using S = typename Elt<DT>::S;
  using MMA = Mfma16x16x32<DT>;

  const int lane = threadIdx.x & (kWave - 1);
  const int task = blockIdx.y * (blockDim.x / kWave) + (threadIdx.x / kWave);
  const int kvh = task / a.nsub;
  if (kvh >= a.nkv) return;
  const int h0 = kvh * a.groups + (task - kvh * a.nsub) * GPW;
  const int w = blockIdx.x;

  int64_t total;
  find_unit(a, -1, &total);
  const int64_t rs = range_start(w, total, a.num_wg);
  const int64_t re = range_start(w + 1, total, a.num_wg);
  if (rs >= re) return;
  int64_t ub;
  int b = find_unit(a, rs, &ub);

  const int col = lane & 15, grp = lane >> 4;
  // FAST: block_size is a multiple of 16, so a tile never crosses a block.
  const S* kbase = reinterpret_cast<const S*>(a.k) + (int64_t)kvh * a.kv_sh;
  const S* vbase = reinterpret_cast<const S*>(a.v) + (int64_t)kvh * a.kv_sh;
  // Fixed per-lane element offsets from a tile's first slot (fast path).
  const int64_t k_off = col * a.kv_ss + 8 * grp;
  int64_t v_off[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) v_off[r] = (4 * grp + r) * a.kv_ss + 8 * col;

  for (int64_t u = rs; u < re && b < a.batch; ++b) {
    const int n = clamped_ctx(a, b);
    const int64_t ue = ub + units_of(a, n);
    const int64_t seg_end = ue < re ? ue : re;
    const bool whole = (u == ub) && (seg_end == ue);
    const int slot = (u == rs) ? 0 : 1;
    const int t0 = (int)(u - ub) * TILE;
    const int t1 = min(n, (int)(seg_end - ub) * TILE);
    if (u == ub && task == 0 && lane == 0) write_desc(a, b, w, ub, ue, rs, total);
    u = seg_end;
    ub = ue;

    // Q^T as the B operand: column col = query head h0 + col.
    u32x4 qb[4];
    {
      const S* qp = reinterpret_cast<const S*>(a.q) + b * a.q_sb + (int64_t)(h0 + col) * a.q_sh + 8 * grp;
#pragma unroll
      for (int m = 0; m < 4; ++m)
        qb[m] = col < GPW ? *reinterpret_cast<const u32x4*>(qp + 32 * m) : u32x4{0, 0, 0, 0};
    }

    int cb = 0, tbl = 0;
    const int fb = first_blk(a, b);
    auto load_table = [&](int first_block) {
      cb = first_block;
      const int j = cb + lane;
      tbl = j < a.max_blocks - fb ? a.tables[b * a.table_stride + fb + j] : 0;
    };
    auto block_of = [&](int p) { return a.bs_shift >= 0 ? (p >> a.bs_shift) : p / a.bs; };

    // Issue a tile's K (MFMA A layout) and V (row layout) loads; returns, per lane,
    // bit r set when token 4*grp + r of the tile is live.
    auto load_tile = [&](int tb, u32x4* kr, u32x4* vr) -> unsigned {
      const u32x4 z = {0, 0, 0, 0};
      if (tb >= t1) {
#pragma unroll
        for (int i = 0; i < 4; ++i) kr[i] = vr[i] = z;
        return 0;
      }
      if (block_of(min(tb + TILE, t1) - 1) - cb >= kWave) load_table(block_of(tb));
      unsigned ok = 0;
      if constexpr (FAST) {
        const int blk = block_of(tb);
        const int bid = __builtin_amdgcn_readlane(tbl, blk - cb);
        const int64_t slot0 = (int64_t)bid * a.bs + (tb - blk * a.bs);
        const int live = (bid >= 0 && slot0 + TILE <= a.num_slots) ? min(TILE, t1 - tb) : 0;
        const S* kt = kbase + slot0 * a.kv_ss;
        const S* vt = vbase + slot0 * a.kv_ss;
        if (live == TILE) {  // full tile: every lane loads, no predication
#pragma unroll
          for (int m = 0; m < 4; ++m) kr[m] = load_kv16v(kt + k_off + 32 * m);
#pragma unroll
          for (int r = 0; r < 4; ++r) vr[r] = load_kv16v(vt + v_off[r]);
          return 0xFu;
        }
        if (live == 0) {  // block id outside the pool: the tile is masked
#pragma unroll
          for (int i = 0; i < 4; ++i) kr[i] = vr[i] = z;
          return 0;
        }
        // Last, partial tile of a piece: lanes past the end re-read the last live
        // token (finite data) and are masked out of the softmax (P = 0).
        const int kt_tok = min(col, live - 1);
#pragma unroll
        for (int m = 0; m < 4; ++m)
          kr[m] = load_kv16v(kt + kt_tok * a.kv_ss + 8 * grp + 32 * m);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int tok = 4 * grp + r;
          vr[r] = load_kv16v(vt + min(tok, live - 1) * a.kv_ss + 8 * col);
          ok |= (unsigned)(tok < live) << r;
        }
      } else {
        // K token tb + col; the V lanes fetch their tokens' slots from those lanes.
        const int p = tb + col;
        const int blk = block_of(p);
        const int bid = __shfl(tbl, blk - cb);
        const int64_t sl = (int64_t)bid * a.bs + (p - blk * a.bs);
        const bool kon = p < t1 && sl >= 0 && sl < a.num_slots;
        const int64_t kslot = kon ? sl : -1;
#pragma unroll
        for (int m = 0; m < 4; ++m)
          kr[m] = kon ? load_kv16v(kbase + kslot * a.kv_ss + 8 * grp + 32 * m) : z;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int src = 4 * grp + r;
          const int lo = __shfl((int)(kslot & 0xFFFFFFFF), src);
          const int hi = __shfl((int)(kslot >> 32), src);
          const int64_t vs = ((int64_t)hi << 32) | (uint32_t)lo;
          const bool on = vs >= 0;
          vr[r] = on ? load_kv16v(vbase + vs * a.kv_ss + 8 * col) : z;
          ok |= (unsigned)on << r;
        }
      }
      return ok;
    };

    float m_run = -INFINITY;  // running max of head column col (same in all 4 rows)
    float l_run = 0.f;        // this row's share of the running sum
    float acc[GPW][8];
#pragma unroll
    for (int g = 0; g < GPW; ++g)
#pragma unroll
      for (int d = 0; d < 8; ++d) acc[g][d] = 0.f;

    auto tile = [&](const u32x4* kr, const u32x4* vr, unsigned ok) {
      f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int m = 0; m < 4; ++m) s = MMA::mma(kr[m], qb[m], s);
      float p[4];
      float mx = -INFINITY;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        p[r] = ((ok >> r) & 1u) ? s[r] * a.scale_log2 : -INFINITY;
        mx = fmaxf(mx, p[r]);
      }
      mx = rows_max(mx);
      const float mn = fmaxf(m_run, mx);
      const float mref = mn == -INFINITY ? 0.f : mn;  // all masked so far: stay at 0
      const float alpha = __builtin_amdgcn_exp2f(m_run - mref);
      m_run = mn;
#pragma unroll
      for (int r = 0; r < 4; ++r) p[r] = __builtin_amdgcn_exp2f(p[r] - mref);
      l_run = __builtin_fmaf(l_run, alpha, (p[0] + p[1]) + (p[2] + p[3]));
      float vf[4][8];
#pragma unroll
      for (int r = 0; r < 4; ++r) unpack16v<DT>(vr[r], vf[r]);
#pragma unroll
      for (int g = 0; g < GPW; ++g) {
        const float al = row_bcast(alpha, g);
#pragma unroll
        for (int d = 0; d < 8; ++d) acc[g][d] *= al;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float pr = row_bcast(p[r], g);
#pragma unroll
          for (int d = 0; d < 8; ++d) acc[g][d] = __builtin_fmaf(pr, vf[r][d], acc[g][d]);
        }
      }
    };

    if (t0 < t1) {
      load_table(block_of(t0));
#if PKV_DECODE_PREFETCH >= 2
      // Three tile buffers in rotation: two tiles in flight while one is reduced.
      u32x4 k0[4], v0[4], k1[4], v1[4], k2[4], v2[4];
      unsigned ok0 = load_tile(t0, k0, v0);
      unsigned ok1 = load_tile(t0 + TILE, k1, v1);
      unsigned ok2;
      for (int tb = t0; tb < t1; tb += 3 * TILE) {
        ok2 = load_tile(tb + 2 * TILE, k2, v2);
        tile(k0, v0, ok0);
        if (tb + TILE >= t1) break;
        ok0 = load_tile(tb + 3 * TILE, k0, v0);
        tile(k1, v1, ok1);
        if (tb + 2 * TILE >= t1) break;
        ok1 = load_tile(tb + 4 * TILE, k1, v1);
        tile(k2, v2, ok2);
      }
#else
      // Two tile buffers in ping-pong: the next tile is in flight while one is reduced.
      u32x4 ka[4], va[4], kb2[4], vb2[4];
      unsigned oka = load_tile(t0, ka, va);
      for (int tb = t0; tb < t1; tb += 2 * TILE) {
        const unsigned okb = load_tile(tb + TILE, kb2, vb2);
        tile(ka, va, oka);
        if (tb + TILE >= t1) break;
        oka = load_tile(tb + 2 * TILE, ka, va);
        tile(kb2, vb2, okb);
      }
#endif
    }

    // Totals: l over the four rows of each column, acc over the four rows.
    const float l_tot = rows_sum(l_run);
#pragma unroll
    for (int g = 0; g < GPW; ++g)
#pragma unroll
      for (int d = 0; d < 8; ++d) acc[g][d] = rows_sum(acc[g][d]);
    float lh[GPW], mh[GPW];
#pragma unroll
    for (int g = 0; g < GPW; ++g) {
      lh[g] = row_bcast(l_tot, g);
      mh[g] = row_bcast(m_run, g);
    }

    if (grp == 0) {  // lane c writes head dims 8c .. 8c + 7
      const int d0 = 8 * col;
      if (whole) {
#pragma unroll
        for (int g = 0; g < GPW; ++g) {
          const float inv = lh[g] > 0.f ? 1.f / lh[g] : 0.f;
          float o[8];
#pragma unroll
          for (int d = 0; d < 8; ++d) o[d] = acc[g][d] * inv;
          const int64_t e = b * a.out_sb + (int64_t)(h0 + g) * a.out_sh + d0;
          if (a.out_f32) store_vec<PKV_F32, 8>((float*)a.out + e, o);
          else store_vec<DT, 8>((S*)a.out + e, o);
          if (a.lse && col == 0) a.lse[(int64_t)b * a.nh + h0 + g] = lse_of(mh[g], lh[g]);
        }
      } else {
#pragma unroll
        for (int g = 0; g < GPW; ++g) {
          const int64_t rec = ((int64_t)w * 2 + slot) * a.nh + h0 + g;
          store_vec<PKV_F32, 8>(a.ws_acc + rec * HD + d0, acc[g]);
          if (col == 0) *reinterpret_cast<float2*>(a.ws_ml + 2 * rec) = make_float2(mh[g], lh[g]);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------------
// Combine pass: merges the pieces of sequences cut by a range boundary.
//
// Sequence b (units [ub, ue)) spans workgroups w0..w1; each non-empty range among them
// holds one piece and wrote one record per query head (in w0 it is the range's last
// piece, slot 1, unless the range starts with it). One wave per (sequence, query head)
// merges them: out = sum_j w_j acc_j / sum_j w_j l_j with w_j = exp2(m_j - max m). The
// sequence's merge plan (16 bytes written by the stream pass) says which records to
// read; then one round trip per 4 records loads their (m, l) pairs and accumulator
// rows together (4 keeps the kernel near 64 VGPRs, so a whole batch's waves are
// resident at once). Cascade prefix parts are folded in after the records. Sequences
// that were not cut exit after reading the plan: the stream pass finished them.
// ---------------------------------------------------------------------------------

// Total units, and the unit range [ub, ue) of sequence b, in one pass over the lengths.
__device__ void seq_units(const DecodeArgs& a, int b, int64_t* ub, int64_t* ue, int64_t* total) {
  const int lane = threadIdx.x & (kWave - 1);
  int64_t before = 0, all = 0;
  int mine = 0;
  for (int c0 = 0; c0 < a.batch; c0 += kWave) {
    const int bb = c0 + lane;
    const int cnt = bb < a.batch ? units_of(a, clamped_ctx(a, bb)) : 0;
    int lt = bb < b ? cnt : 0;
    int tot = cnt;
    if (bb == b) mine = cnt;
#pragma unroll
    for (int s = 1; s < kWave; s <<= 1) {
      lt += __shfl_xor(lt, s);
      tot += __shfl_xor(tot, s);
    }
    before += lt;
    all += tot;
  }
#pragma unroll
  for (int s = 1; s < kWave; s <<= 1) mine += __shfl_xor(mine, s);
  *ub = before;
  *ue = before + mine;
  *total = all;
}

template <int DT, int HD>
__global__ void __launch_bounds__(256)
paged_decode_combine_kernel(const DecodeArgs a) {
  constexpr int DPL = HD >= kWave ? HD / kWave : 1;  // head dims per lane
  constexpr int kChunk = 4;                           // records loaded per round trip
  const int lane = threadIdx.x & (kWave - 1);
  const int wid = blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  if (wid >= a.batch * a.nh) return;  // uniform per wave
  const int b = wid / a.nh, h = wid - b * a.nh;

  const int4 plan = a.desc[b];
  const int nrec = plan.y;
  const bool cascade = a.pre_row != nullptr;
  if (nrec <= 1 && !cascade) return;  // written directly by the stream pass
  const int64_t w0 = plan.x;
  // Units fewer than workgroups leave some ranges empty: then find the live ones.
  int64_t ub = 0, ue = 0, total = 0;
  if (!plan.w) seq_units(a, b, &ub, &ue, &total);
  const int64_t row0 = (w0 * 2 + plan.z) * a.nh + h;  // record 0: always live

  float out_acc[DPL], lsum = 0.f, mmax = -INFINITY;
#pragma unroll
  for (int k = 0; k < DPL; ++k) out_acc[k] = 0.f;
  // Fold records [j0, j0 + C) into the running (max, sum, acc). Every load is issued
  // before any is used. Dead slots (past the last record, or an empty range) re-read
  // record 0 -- finite data -- and get weight 0: records that were never written are
  // not read, the scratch may hold NaN bit patterns.
  // Liveness of records j0 .. j0 + 63, one per lane (a range can be empty only when
  // units < workgroups; the test divides, so it is done once per lane, not per record).
  uint64_t live_bits = 0;
  auto live_block = [&](int j0) {
    const int j = j0 + lane;
    bool live = j < nrec;
    if (!plan.w && live) {
      const int64_t ww = w0 + j;
      live = range_start(ww, total, a.num_wg) < range_start(ww + 1, total, a.num_wg);
    }
    live_bits = __ballot(live);
  };
  auto fold = [&](auto chunk, int j0) {
    constexpr int C = decltype(chunk)::value;
    float m[C], l[C], x[C][DPL];
#pragma unroll
    for (int jj = 0; jj < C; ++jj) {
      const int j = j0 + jj;
      const bool live = (live_bits >> (j & (kWave - 1))) & 1;
      const int64_t row = (live && j > 0) ? (w0 + j) * 2 * a.nh + h : row0;
      const float2 ml = *reinterpret_cast<const float2*>(a.ws_ml + 2 * row);
      m[jj] = live ? ml.x : -INFINITY;
      l[jj] = ml.y;
      const float* rowp = a.ws_acc + row * HD;
#pragma unroll
      for (int k = 0; k < DPL; ++k) x[jj][k] = (lane + kWave * k < HD) ? rowp[lane + kWave * k] : 0.f;
    }
    float mn = mmax;
#pragma unroll
    for (int jj = 0; jj < C; ++jj) mn = fmaxf(mn, m[jj]);
    const float mref = mn == -INFINITY ? 0.f : mn;  // no live token yet: weights 0
    const float alpha = __builtin_amdgcn_exp2f(mmax - mref);
    mmax = mn;
    lsum *= alpha;
#pragma unroll
    for (int k = 0; k < DPL; ++k) out_acc[k] *= alpha;
#pragma unroll
    for (int jj = 0; jj < C; ++jj) {
      const float wj = __builtin_amdgcn_exp2f(m[jj] - mref);  // dead: exp2(-inf) = 0
      lsum = __builtin_fmaf(wj, l[jj], lsum);
#pragma unroll
      for (int k = 0; k < DPL; ++k) out_acc[k] = __builtin_fmaf(wj, x[jj][k], out_acc[k]);
    }
  };
  if (nrec <= 1) {
    // Cascade, finished by the stream pass: its normalised fp32 output and log2
    // normaliser are the state (lse, 1, O); an empty context (-inf) weighs nothing.
    const float lt = a.lse[(int64_t)b * a.nh + h];
    mmax = lt;
    lsum = lt == -INFINITY ? 0.f : 1.f;
    const float* t = reinterpret_cast<const float*>(a.out) + b * a.out_sb + (int64_t)h * a.out_sh;
#pragma unroll
    for (int k = 0; k < DPL; ++k) out_acc[k] = (lane + kWave * k < HD) ? t[lane + kWave * k] : 0.f;
  } else {
    for (int j0 = 0; j0 < nrec; j0 += kChunk) {
      if ((j0 & (kWave - 1)) == 0) live_block(j0);
      fold(std::integral_constant<int, kChunk>{}, j0);
    }
  }
  if (cascade) fold_prefix<HD, DPL>(a, b, h, mmax, lsum, out_acc);
  const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
  float* lse_dst = cascade ? a.fin_lse : a.lse;
  if (lse_dst && lane == 0) lse_dst[(int64_t)b * a.nh + h] = lse_of(mmax, lsum);
  void* dst = cascade ? a.fin : a.out;
  const int64_t sb = cascade ? a.fin_sb : a.out_sb, sh = cascade ? a.fin_sh : a.out_sh;
  const bool f32 = cascade ? a.fin_f32 : a.out_f32;
#pragma unroll
  for (int k = 0; k < DPL; ++k) {
    const int d = lane + kWave * k;
    if (d >= HD) break;
    const float o = out_acc[k] * inv;
    const int64_t e = b * sb + (int64_t)h * sh + d;
    if (f32) reinterpret_cast<float*>(dst)[e] = o;
    else reinterpret_cast<typename Elt<DT>::S*>(dst)[e] = Elt<DT>::from_f32(o);
  }
}

// ---------------------------------------------------------------------------------
// Chunked-prefill attention on the matrix cores (16-bit K/V, head_dim 32/64/128/256).
//
// Chunk c has q_c query tokens (rows cu_q[c] .. cu_q[c+1] of q) and a context of n_c
// tokens in the paged pool (its own tokens last): query i sits at position n_c - q_c + i
// and attends to keys 0 .. n_c - q_c + i (bottom-right causal, as the reference's
// PagedBatch._mixed / varlen path). For KV head g the query rows are (token, head j of
// g's group) pairs, rho = token * G + j. A workgroup of 8 waves takes 128 of them, one
// work item, and fills a CU:
//   * Key halves. Waves 0-3 take the item's first half of 64-key tiles, waves 4-7 the
//     rest; wave w of each half holds rows 32 w .. 32 w + 31 (two 16-row MFMA tiles), and
//     the two waves of one SIMD (w and w + 4) belong to different halves. At the end the
//     halves' softmax states (m, l, O) merge through LDS.
//   * Ping-pong. The halves run one barrier interval apart, alternating a matrix phase
//     (P.V of the previous tile, QK^T of this one) with a VALU phase (the K/V loads of
//     later tiles, the softmax of this one), so each SIMD overlaps one wave's MFMAs with
//     the other's softmax.
//   * K and V tiles go from the pool straight into LDS (global_load_lds), three
//     intervals ahead, the 16-byte chunks of each token row XOR-swizzled by the token
//     index (conflict-free operand reads).
//   * S^T = K . Q^T with v_mfma_f32_16x16x32 (K rows from LDS as A, Q rows kept in
//     VGPRs as B): lane (row n, grp g) gets keys 4g + r of each 16-key block for query
//     row n. fp32 online softmax per row (cross-row max/sum with permlane16/32 swaps).
//   * O^T += V^T . P^T: P^T's fragment is the lane's own S^T values (the MFMA's
//     contraction order over keys is chosen to match), so P needs no lane exchange and
//     takes the registers S had; V^T comes from two ds_read_b64_tr_b16 transpose reads
//     per MFMA. The rescale factor of row n lives in the lanes that hold O^T's row n.
// P enters the second product in the K/V type; for bf16 as a hi + lo pair (fp32-like
// accuracy), for fp16 rounded once.
// ---------------------------------------------------------------------------------

struct PrefillArgs {
  void* out;
  int64_t out_st, out_sh;
  const void* q;
  int64_t q_st, q_sh;
  const void* k;
  const void* v;
  int64_t kv_ss, kv_sh, num_slots;
  const int32_t* tables;
  int64_t table_stride;
  int32_t max_blocks;
  const int32_t* ctx;   // [n_chunks] context tokens (the chunk's own included)
  const int32_t* cu_q;  // [n_chunks + 1] query row offsets
  int32_t n_chunks, nh, nkv, groups, bs, bs_shift;
  int32_t row_blocks;   // 128-row blocks per chunk (static bound)
  float scale_log2;
  int out_f32;
  int32_t causal;         // 0: every query of chunk c sees all its n_c keys
  const int32_t* q_rows;  // [tokens] or null: query token t reads q row q_rows[t]
  float* lse;             // [tokens, nh] or null: log2 of each softmax's normaliser
};

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

template <int DT> struct Mfma16x16x32Bits;  // MFMA on raw 16-bit bit patterns
template <> struct Mfma16x16x32Bits<PKV_BF16> {
  typedef __bf16 v8 __attribute__((ext_vector_type(8)));
  typedef __bf16 v2 __attribute__((ext_vector_type(2)));
  // bf16 keeps 8 significant bits, too few for softmax weights at a 2e-3 output bar, so
  // P enters the product as hi = bf16(P) plus lo = bf16(P - hi) (two MFMAs).
  static constexpr bool kSplit = true;
  __device__ static f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8, a),
                                                   __builtin_bit_cast(v8, b), c, 0, 0, 0);
  }
  // 8 finite fp32 -> hi and lo operand fragments (v_cvt_pk_bf16_f32, round to nearest
  // even).
  __device__ static void pack8(const float* p, u32x4& hi, u32x4& lo) {
    uint32_t h[4], l[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      h[i] = __builtin_bit_cast(uint32_t, v2{(__bf16)p[2 * i], (__bf16)p[2 * i + 1]});
      // the empty asm keeps h[i] one value (no second conversion to rebuild its low half)
      uint32_t hv = h[i];
      __asm__("" : "+v"(hv));
      const float r0 = p[2 * i] - __uint_as_float(hv << 16);
      const float r1 = p[2 * i + 1] - __uint_as_float(hv & 0xFFFF0000u);
      l[i] = __builtin_bit_cast(uint32_t, v2{(__bf16)r0, (__bf16)r1});
    }
    hi = u32x4{h[0], h[1], h[2], h[3]};
    lo = u32x4{l[0], l[1], l[2], l[3]};
  }
};
template <> struct Mfma16x16x32Bits<PKV_F16> {
  typedef _Float16 v8 __attribute__((ext_vector_type(8)));
  typedef _Float16 v2 __attribute__((ext_vector_type(2)));
  static constexpr bool kSplit = false;  // fp16 keeps 11 bits: P rounded once
  __device__ static f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8, a),
                                                  __builtin_bit_cast(v8, b), c, 0, 0, 0);
  }
  __device__ static void pack8(const float* p, u32x4& hi, u32x4& lo) {
    uint32_t h[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      h[i] = __builtin_bit_cast(uint32_t, v2{(_Float16)p[2 * i], (_Float16)p[2 * i + 1]});
    hi = u32x4{h[0], h[1], h[2], h[3]};
    lo = hi;
  }
};

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding: vmcnt in
// bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8). Direct-to-LDS loads count in vmcnt and
// complete in issue order like every other vector-memory load.
template <int N> __device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit field");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
// Wait for every outstanding LDS access of this wave.
__device__ __forceinline__ void wait_lgkm0() {
  __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4));
}

typedef __attribute__((address_space(3))) void lds_void;

// LDS byte address of a __shared__ object.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const lds_void*)p;
}

// Global memory straight into LDS, one wave at a time: lane i's 16 (4) bytes land at LDS
// address lds_base + 16 i (+ 4 i); lds_base is wave-uniform and travels in M0. Written
// as inline asm on purpose: the compiler then neither treats the load as a pending LDS
// write (which makes it wait for every outstanding load before each later LDS read) nor
// counts it when it sizes its own vmcnt waits. Kernels that use these issue no other
// vector-memory loads in the same loop and order everything with wait_vmcnt and
// barriers themselves.
__device__ __forceinline__ void dma16_to_lds(const void* src, uint32_t lds_base) {
  asm volatile("global_load_lds_dwordx4 %0, off" : : "v"(src), "{m0}"(lds_base) : "memory");
}
// The same with a wave-uniform 64-bit base in SGPRs and a 32-bit per-lane byte offset.
__device__ __forceinline__ void dma16_to_lds_s(const void* base, uint32_t off, uint32_t lds_base) {
  asm volatile("global_load_lds_dwordx4 %0, %1" : : "v"(off), "s"(base), "{m0}"(lds_base)
               : "memory");
}
__device__ __forceinline__ void dma4_to_lds(const void* src, uint32_t lds_base) {
  asm volatile("global_load_lds_dword %0, off" : : "v"(src), "{m0}"(lds_base) : "memory");
}

// Wave priority around runs of MFMAs: when two waves share a SIMD, the one about to
// issue matrix instructions goes first while the other does its softmax arithmetic.
__device__ __forceinline__ void mfma_phase_begin() {
#if PKV_PREFILL_SETPRIO
  __builtin_amdgcn_s_setprio(1);
#endif
}
__device__ __forceinline__ void mfma_phase_end() {
#if PKV_PREFILL_SETPRIO
  __builtin_amdgcn_s_setprio(0);
#endif
}

template <int HD> struct PrefillShape {
  static constexpr int RT = HD >= 256 ? 1 : 2;   // 16-row MFMA tiles per wave
  static constexpr int BM = 4 * 16 * RT;         // query rows per workgroup (4 waves a half)
  static constexpr int KT = HD >= 256 ? 32 : 64; // keys per tile
  static constexpr int CH = HD / 8;              // 16-byte granules per K/V row
  static constexpr int NBETA = KT / 16;          // 16-key blocks of S^T per tile
  static constexpr int NSG = KT / 32;            // 32-key contraction steps of O^T per tile
  static constexpr int KS = HD / 32;             // contraction steps over head_dim
  static constexpr int DTL = HD / 16;            // 16-dim tiles of O^T
  static constexpr int NLD = KT * CH / 256;      // granules per thread per tile, K and V each
  static constexpr int TILE = KT * CH;           // granules of one K (or V) tile
  static_assert(NLD >= 1 && KT * CH % 256 == 0, "tile must split evenly over 256 threads");
  static_assert(2 * NLD < 64, "vmcnt range");
  static_assert(KT <= kWave, "a tile's block ids must fit one 64-entry table window");
  // LDS position of chunk c of key t's row is c ^ swz(t). Rows are 256 bytes (head dim
  // 128, 16 chunks), so a chunk's bank group is its position mod 8 (a 128-byte access
  // window). The K operand reads (ds_read_b128: 8 lanes = 8 consecutive keys, one chunk,
  // per access) are conflict-free when swz's low 3 bits are a bijection of the key's low
  // 3 bits; the V^T transpose reads (4 consecutive keys x chunks 2d, 2d + 1 per 16
  // lanes) when swz's bits 1-2 are a bijection of the key's bits 0-1. swz(t) = (t2, t0,
  // t1, t3) -- bits 0..3 -- satisfies both.
  __device__ static int swz(int t) {
    if constexpr (CH == 16) return ((t << 1) & 6) | ((t >> 2) & 1) | (t & 8);
    else return t % CH;
  }
};

template <int DT, int HD, bool POW2>
__global__ void __launch_bounds__(512)
paged_prefill_kernel(const PrefillArgs a) {
  using SH = PrefillShape<HD>;
  constexpr int RT = SH::RT, BM = SH::BM, KT = SH::KT, CH = SH::CH, NBETA = SH::NBETA;
  constexpr int NSG = SH::NSG, KS = SH::KS, DTL = SH::DTL, NLD = SH::NLD, TILE = SH::TILE;
  static_assert(HD % 32 == 0 && HD <= 256, "head_dim must be 32..256, a multiple of 32");
  using MMA = Mfma16x16x32Bits<DT>;
  using S = typename Elt<DT>::S;
  // ring[half][0 = K, 1 = V][stage]: each key half's K and V tiles, two stages each.
  __shared__ __align__(16) u32x4 ring[2][2][2][TILE];
  // Block-table windows, per half and wave, in a ring of three (one per tile in flight).
  __shared__ __align__(16) int32_t idring[2][3][4][kWave];

  const int tid = threadIdx.x;
  const int half = __builtin_amdgcn_readfirstlane(tid >> 8);  // which half of the key tiles
  const int htid = tid & 255;                                 // thread index inside the half
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(htid / kWave);  // rows 32 wave .. (RT = 2)
  const int col = lane & 15, grp = lane >> 4;
  // Work items (chunk, row block, KV head), heaviest first: chunks by context length
  // (longest first), then row blocks from the last (it sees the most keys), KV heads
  // innermost. One workgroup fills a CU, so a grid larger than the GPU runs the items
  // in this order as CUs free up: the longest start earliest.
  const int item = (int)blockIdx.x;
  const int kvh = item % a.nkv;
  const int rbi = (item / a.nkv) % a.row_blocks;
  const int crank = item / (a.nkv * a.row_blocks);
  // Each wave ranks up to 64 chunks by itself; larger batches keep their order.
  int c = crank;
  if (a.n_chunks <= kWave) {
    const int cap0 = a.max_blocks * a.bs;
    const int mine = lane < a.n_chunks ? min(max(a.ctx[lane], 0), cap0) : -1;
    int rank = 0;
    for (int j = 0; j < a.n_chunks; ++j) {
      const int other = __shfl(mine, j);
      rank += (other > mine) || (other == mine && j < lane);
    }
    const uint64_t hit = __ballot(lane < a.n_chunks && rank == crank);
    c = __builtin_ctzll(hit);
  }
  const int q0 = a.cu_q[c], qlen = a.cu_q[c + 1] - q0;
  const int G = a.groups;
  const int nrows = qlen * G;
  const int rho0 = (a.row_blocks - 1 - rbi) * BM;
  if (qlen <= 0 || rho0 >= nrows) return;  // uniform per workgroup
  const int cap = a.max_blocks * a.bs;
  const int n = min(max(a.ctx[c], 0), cap);
  const int base_pos = n - qlen;  // position of query token 0

  // This lane's query row in each of its wave's 16-row tiles (B operand column). Both
  // halves hold the same rows.
  int row_tok[RT];
  bool row_ok[RT];
  u32x4 qf[RT][KS];
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    const int rho = rho0 + 16 * RT * wave + 16 * t + col;
    row_ok[t] = rho < nrows;
    const int rr = row_ok[t] ? rho : 0;
    row_tok[t] = rr / G;
    const int64_t qrow = a.q_rows ? a.q_rows[q0 + row_tok[t]] : q0 + row_tok[t];
    const S* qp = reinterpret_cast<const S*>(a.q) + qrow * a.q_st +
                  (int64_t)(kvh * G + rr % G) * a.q_sh + 8 * grp;
#pragma unroll
    for (int s = 0; s < KS; ++s) qf[t][s] = *reinterpret_cast<const u32x4*>(qp + 32 * s);
  }
  // Keys any row of this workgroup attends to: [0, kend), in ntiles tiles; half 0 takes
  // tiles 0 .. ns - 1, half 1 the other ntiles - ns.
  const int last_row = min(nrows - 1, rho0 + BM - 1);
  const int kend = a.causal ? min(n, base_pos + last_row / G + 1) : n;
  const int ntiles = kend > 0 ? (kend + KT - 1) / KT : 0;
  const int ns = (ntiles + 1) / 2;
  const int tbeg = half ? ns : 0;
  const int nt = half ? ntiles - ns : ns;

  // Tile j's K (or V) rows go from the pool straight into LDS. Instruction r of wave w
  // fills granules r*256 + 64w .. +63 of the tile, one per lane; granule (token t,
  // position p) holds chunk p ^ swz(t) of that token's row, so the MFMA operand reads
  // below are conflict-free. Positions past the context re-read the last context token
  // (finite, masked out of the softmax). The 64 block-table entries from the tile's first
  // block on reach LDS the same way, two tiles ahead of the K/V loads that need them.
  // Granule r of this thread: token tok_of(r) of the tile, LDS position chk_of(r).
  auto tok_of = [&](int r) { return (r * 256 + htid) / CH; };
  auto chk_of = [&](int r) { return ((r * 256 + htid) % CH) ^ SH::swz(tok_of(r)); };
  const int32_t* trow = a.tables + (int64_t)c * a.table_stride;
  const int nlast = max(n - 1, 0);
  auto blk_of = [&](int p) { return POW2 ? (p >> a.bs_shift) : p / a.bs; };
  const int blast = blk_of(nlast);
  const uint32_t ring_lds = lds_addr(&ring[half][0][0][0]);
  const uint32_t ids_lds = lds_addr(&idring[half][0][wave][0]);
  // Local tile m of this half is tile tbeg + m; past the half's end, the last one (the
  // loads keep their count; their stages are free).
  auto gtile = [&](int m) { return tbeg + min(m, nt - 1); };
  auto issue_ids = [&](int m) __attribute__((always_inline)) {
    const int b = min(blk_of(gtile(m) * KT) + lane, blast);
    dma4_to_lds(trow + b, ids_lds + (uint32_t)((m % 3) * 4 * kWave * 4));
  };
  // One DMA instruction of one wave covers SEG consecutive keys of a tile. When the block
  // size is a power of two >= SEG those keys share one block: its id is wave-uniform and
  // the address is scalar math plus one per-lane offset.
  constexpr int SEG = kWave / CH;
  const bool seg_uniform = POW2 && a.bs >= SEG;
  // Fast path (power-of-two blocks of at least SEG keys, tile inside the context): the
  // lane's byte offset inside its block is the same for every tile, plus a uniform part
  // when blocks are longer than a tile.
  uint32_t lane_off[NLD];
#pragma unroll
  for (int r = 0; r < NLD; ++r)
    lane_off[r] = (uint32_t)(((tok_of(r) & (a.bs - 1)) * a.kv_ss + chk_of(r) * 8) * (int64_t)sizeof(S));
  const int64_t blk_bytes = (int64_t)a.bs * a.kv_ss * (int64_t)sizeof(S);
  const int64_t kvh_bytes = (int64_t)kvh * a.kv_sh * (int64_t)sizeof(S);
  // Per round only a 32 x 32-bit multiply-add in SGPRs: block bytes must fit 32 bits
  // (they do for any real pool), block ids past the pool read block 0.
  const bool fast = seg_uniform && blk_bytes <= 0xFFFFFFFFll;
  const uint32_t blk_bytes32 = (uint32_t)blk_bytes;
  const uint32_t pool_blocks = (uint32_t)min(a.num_slots / a.bs, (int64_t)0x7FFFFFFF);
  const char* kv_base[2] = {reinterpret_cast<const char*>(a.k) + kvh_bytes,
                            reinterpret_cast<const char*>(a.v) + kvh_bytes};
  // K (kv = 0) or V (kv = 1) of local tile m into stage m % 2.
  auto issue_tile = [&](int m, int kv) __attribute__((always_inline)) {
    const int j = gtile(m);
    const int32_t* ids = &idring[half][m % 3][wave][0];
    const int b0 = blk_of(j * KT);
    const char* src = reinterpret_cast<const char*>(kv ? a.v : a.k);
    const uint32_t dst = ring_lds + (uint32_t)(((kv * 2 + (m & 1)) * TILE) * 16);
    if constexpr (POW2) {
      if (fast && (j + 1) * KT <= n) {
        int id[NLD];
#pragma unroll
        for (int r = 0; r < NLD; ++r)  // every id read before the first DMA
          id[r] = ids[((j * KT + (r * 256 + wave * kWave) / CH) >> a.bs_shift) - b0];
        const char* base = kv_base[kv] + (uint32_t)(((j * KT) & (a.bs - 1)) * a.kv_ss * (int)sizeof(S));
#pragma unroll
        for (int r = 0; r < NLD; ++r) {
          uint32_t bid = (uint32_t)__builtin_amdgcn_readfirstlane(id[r]);
          bid = bid < pool_blocks ? bid : 0u;  // memory safety only
          dma16_to_lds_s(base + (uint64_t)bid * blk_bytes32, lane_off[r],
                         dst + (uint32_t)((r * 256 + wave * kWave) * 16));
        }
        return;
      }
      if (seg_uniform) {  // the context's last tile: positions past it re-read its last token
        int id[NLD];
#pragma unroll
        for (int r = 0; r < NLD; ++r) {  // every id read before the first DMA
          const int seg = j * KT + (r * 256 + wave * kWave) / CH;  // first key, uniform
          id[r] = ids[min(seg >> a.bs_shift, blast) - b0];
        }
#pragma unroll
        for (int r = 0; r < NLD; ++r) {
          const int seg = j * KT + (r * 256 + wave * kWave) / CH;
          const int blk = min(seg >> a.bs_shift, blast);
          int64_t bid = __builtin_amdgcn_readfirstlane(id[r]);
          if (bid < 0 || (bid + 1) * a.bs > a.num_slots) bid = 0;  // memory safety only
          const int64_t base = (bid * a.bs * a.kv_ss + (int64_t)kvh * a.kv_sh) * (int64_t)sizeof(S);
          const int in_blk = min(seg + lane / CH, nlast) - blk * a.bs;
          const uint32_t lo = (uint32_t)((in_blk * a.kv_ss + chk_of(r) * 8) * (int64_t)sizeof(S));
          dma16_to_lds(src + base + lo, dst + (uint32_t)((r * 256 + wave * kWave) * 16));
        }
        return;
      }
    }
#pragma unroll
    for (int r = 0; r < NLD; ++r) {
      const int p = min(j * KT + tok_of(r), nlast);
      const int blk = blk_of(p);
      int64_t sl = (int64_t)ids[blk - b0] * a.bs + (p - blk * a.bs);
      sl = (sl >= 0 && sl < a.num_slots) ? sl : 0;
      const int64_t off = (sl * a.kv_ss + (int64_t)kvh * a.kv_sh + chk_of(r) * 8) * (int64_t)sizeof(S);
      dma16_to_lds(src + off, dst + (uint32_t)((r * 256 + wave * kWave) * 16));
    }
  };

  float m_run[RT], l_run[RT];
  f32x4 o[RT][DTL];
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    m_run[t] = -INFINITY;
    l_run[t] = 0.f;
#pragma unroll
    for (int d = 0; d < DTL; ++d) o[t][d] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // Rows whose causal limit a tile can cross: tile j needs the mask only if it reaches
  // past the smallest limit among this workgroup's rows (its first row's).
  const int limit_min = a.causal ? min(n - 1, base_pos + rho0 / G) : n - 1;
  const int j_mask = min(ntiles, max(0, (limit_min + 1) / KT));
  int limit[RT];  // last key each of this lane's rows sees
#pragma unroll
  for (int t = 0; t < RT; ++t) limit[t] = a.causal ? min(n - 1, base_pos + row_tok[t]) : n - 1;

  // Per-lane LDS byte offsets of the operand fragments inside a tile, recomputed where
  // they are used (a few VALU instructions; holding them would cost 12 registers).
  //   K: lane (col, grp) reads key 16 beta + col, chunk 4 s + grp. swz(key) depends on
  //      beta only when a row has more than 16 chunks (head_dim 256).
  //   V^T: lane (col, grp) reads key 32 sg + 16 h2 + 4 grp + col / 4, dims 16 d +
  //      4 (col % 4) .. +4 (chunk 2 d + (col % 4) / 2, half (col % 4) & 1).
  constexpr int KSW = CH > 16 ? NBETA : 1;
  constexpr int VSW = CH > 16 ? 2 : 1;
  auto fresh_lane = [&]() {  // lane, as a value the compiler must not hoist
    int l = lane;
    __asm__ volatile("" : "+v"(l));
    return l;
  };
  auto koff = [&](int l, int b, int s) {
    const int tk = 16 * b + (l & 15);
    return (uint32_t)(((4 * s + (l >> 4)) ^ SH::swz(tk)) * 16 + (l & 15) * CH * 16);
  };
  auto voff = [&](int l, int h2, int d) {
    const int c4 = l & 3, tr = 4 * (l >> 4) + ((l & 15) >> 2);
    const int tk = 16 * h2 + tr;
    return (uint32_t)((((2 * d + c4 / 2) ^ SH::swz(tk)) * 16 + (c4 & 1) * 8) + tr * CH * 16);
  };

  // S^T of a tile from its QK^T to its softmax, then in the same registers its
  // probabilities P^T until its P.V (the first 32-key step's already packed as operand
  // fragments: hi in block 0, lo in block 1).
  static_assert(NBETA == 2 * NSG, "two score blocks per P^T fragment pair");
  f32x4 sc[RT][NBETA];

  // S^T = K . Q^T of local tile m: block beta holds keys 16 beta + 4 grp + r for query
  // row col.
  auto qk = [&](int m) __attribute__((always_inline)) {
    const char* stage = reinterpret_cast<const char*>(&ring[half][0][m & 1][0]);
    const int l = fresh_lane();
#pragma unroll
    for (int beta = 0; beta < NBETA; ++beta) {
      if (beta) __builtin_amdgcn_sched_barrier(0);  // one 16-key block's K fragments at a time
#pragma unroll
      for (int t = 0; t < RT; ++t) sc[t][beta] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const u32x4 kf = *reinterpret_cast<const u32x4*>(stage + beta * 16 * CH * 16 +
                                                         koff(l, KSW == 1 ? 0 : beta, s));
#pragma unroll
        for (int t = 0; t < RT; ++t) sc[t][beta] = MMA::mma(kf, qf[t][s], sc[t][beta]);
      }
    }
  };
  // O^T += V^T . P^T of local tile m; each V^T fragment (two ds_read_b64_tr_b16
  // transpose reads) serves every row tile. P arrives as fp32 probabilities; each 32-key
  // step packs its operand fragments here, in the matrix phase, whose VALU is otherwise
  // idle (the softmax phase is the longer one).
  auto pv = [&](int m) __attribute__((always_inline)) {
    const char* vstage = reinterpret_cast<const char*>(&ring[half][1][m & 1][0]);
    const int l = fresh_lane();
#pragma unroll
    for (int sg = 0; sg < NSG; ++sg) {
      if (sg) __builtin_amdgcn_sched_barrier(0);  // one 32-key step's fragments at a time
      // P^T fragment of row tile t: the lane's own 8 probabilities (keys 32 sg + 16
      // (e / 4) + 4 grp + e % 4), matching the transpose-read order of V^T. Step 0 was
      // packed by the softmax; the later steps are packed here, while step 0's MFMAs run.
      u32x4 phi[RT], plo[RT];
#pragma unroll
      for (int t = 0; t < RT; ++t) {
        if (sg == 0) {
          phi[t] = __builtin_bit_cast(u32x4, sc[t][0]);
          plo[t] = __builtin_bit_cast(u32x4, sc[t][1]);
        } else {
          float p8[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) p8[e] = sc[t][2 * sg + e / 4][e % 4];
          MMA::pack8(p8, phi[t], plo[t]);
        }
      }
#pragma unroll
      for (int d = 0; d < DTL; ++d) {
        u32x4 vf;
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
          // generic -> LDS address space (an addrspacecast of a __shared__ pointer)
          const s16x4 x = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_s16x4*)(vstage + (32 * sg + 16 * h2) * CH * 16 + voff(l, VSW == 1 ? 0 : h2, d)));
          const uint32_t lo = (uint32_t)(uint16_t)x[0] | ((uint32_t)(uint16_t)x[1] << 16);
          const uint32_t hi = (uint32_t)(uint16_t)x[2] | ((uint32_t)(uint16_t)x[3] << 16);
          if (h2 == 0) { vf.x = lo; vf.y = hi; } else { vf.z = lo; vf.w = hi; }
        }
#pragma unroll
        for (int t = 0; t < RT; ++t) {
          o[t][d] = MMA::mma(vf, phi[t], o[t][d]);
          if constexpr (MMA::kSplit) o[t][d] = MMA::mma(vf, plo[t], o[t][d]);
        }
      }
    }
  };
  // Online softmax of global tile j's scores into P^T fragments; masked: some key of the
  // tile is past some row's causal limit (the tiles on the diagonal and the context end;
  // a wave-uniform branch around the mask only: one copy of the rest, whose registers a
  // second copy would double).
  auto softmax = [&](int j, bool masked) __attribute__((always_inline)) {
    const int kt0 = j * KT;
    // p = exp2(scale_log2 * s - m_run). The reference m_run is raised only when a score
    // exceeds it by more than 2^8: a stale reference changes nothing in O / l (both carry
    // the same factor), keeps p <= 256, and leaves O untouched on most tiles. The row
    // tiles are independent chains: maxima first, one rescale branch, then every exp.
    float mx[RT];
    bool raise[RT];
    bool any = false;
#pragma unroll
    for (int t = 0; t < RT; ++t) {
      if (masked) {
        const int lim = limit[t] - kt0 - 4 * grp;  // keys 16 beta + r past it are out
#pragma unroll
        for (int beta = 0; beta < NBETA; ++beta)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (16 * beta + r > lim) sc[t][beta][r] = -INFINITY;
      }
      float x = -INFINITY;
#pragma unroll
      for (int beta = 0; beta < NBETA; ++beta)
#pragma unroll
        for (int r = 0; r < 4; ++r) x = fmaxf(x, sc[t][beta][r]);
      mx[t] = rows_max(x) * a.scale_log2;
      raise[t] = mx[t] > m_run[t] + 8.f;  // also true the first time (m_run = -inf)
      any = any || raise[t];
    }
    if (__builtin_amdgcn_ballot_w64(any)) {  // wave-uniform
#pragma unroll
      for (int t = 0; t < RT; ++t) {
        // Rows that do not raise keep their factor 1 (their m_run may still be -inf: a
        // half's tiles can all lie past a row's causal limit).
        const float alpha = raise[t] ? __builtin_amdgcn_exp2f(m_run[t] - mx[t]) : 1.f;
        m_run[t] = raise[t] ? mx[t] : m_run[t];
        l_run[t] *= alpha;
#pragma unroll
        for (int d = 0; d < DTL; ++d) o[t][d] *= alpha;
      }
    }
#pragma unroll
    for (int t = 0; t < RT; ++t) {
      const float mref = m_run[t] == -INFINITY ? 0.f : m_run[t];
      float psum = 0.f;
#pragma unroll
      for (int beta = 0; beta < NBETA; ++beta)
#pragma unroll
        for (int r = 0; r < 4; ++r) {  // probabilities replace the scores
          const float pr = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[t][beta][r], a.scale_log2, -mref));
          sc[t][beta][r] = pr;
          psum += pr;
        }
      // The first 32-key step's P^T fragments are packed here (hi and lo into score
      // blocks 0 and 1); P.V packs the others, balancing the two phases.
      {
        float p8[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) p8[e] = sc[t][e / 4][e % 4];
        u32x4 hi, lo;
        MMA::pack8(p8, hi, lo);
        sc[t][0] = __builtin_bit_cast(f32x4, hi);
        sc[t][1] = __builtin_bit_cast(f32x4, lo);
      }
      l_run[t] += psum;
    }
  };

  // Ping-pong schedule. Interval k (k = 0 .. 2 ns + 1) starts at a workgroup barrier; a
  // half is at local phase p = k - half, so when one half issues matrix work the other
  // does its softmax, and each SIMD (one wave of each half) overlaps the two.
  //   p = 2m (matrix phase):  P.V of tile m - 1, QK^T of tile m.
  //   p = 2m + 1 (VALU phase): loads of block ids (tile m + 3), V (m + 1), K (m + 2);
  //                            softmax of tile m.
  // A K tile is used at phase 2m, its V at 2m + 2; both were issued at 2m - 3, into the
  // stage that tile m - 2 freed at 2m - 2. Before each matrix phase a wave waits for all
  // but the loads of the previous VALU phase (2 NLD + 1), before each VALU phase for
  // all but that phase's K and V loads (its block ids must be in). Loads complete in
  // issue order.
  if (nt > 0) {  // prologue: block ids of tiles 0-2, K of 0 and 1, V of 0
    issue_ids(0);
    issue_ids(1);
    wait_vmcnt<0>();
    issue_tile(0, 0);
    issue_ids(2);
    issue_tile(0, 1);
    issue_tile(1, 0);
    wait_vmcnt<0>();
  }
  // Matrix phase of iteration m and VALU phase of iteration m, each closed by its
  // barrier. Half 0 runs intervals (M0 V0)(M1 V1)..(M_ns V_ns); half 1 one interval
  // later: idle, (M0 V0)..(M_ns-1 V_ns-1) M_ns. Both pass 2 ns + 2 barriers.
  auto interval_m = [&](int m) __attribute__((always_inline)) {
    if (m >= 1 && m - 1 < nt) wait_vmcnt<2 * NLD + 1>();
    else wait_vmcnt<0>();
    wait_lgkm0();
    __builtin_amdgcn_s_barrier();
    mfma_phase_begin();
    if (m >= 1 && m - 1 < nt) pv(m - 1);  // first: P's registers then hold S
    // Nothing crosses: the V^T and K fragments of the two products are never all live.
    __builtin_amdgcn_sched_barrier(0);
    if (m < nt) qk(m);
    mfma_phase_end();
  };
  auto interval_v = [&](int m) __attribute__((always_inline)) {
    if (m < nt) wait_vmcnt<2 * NLD>();
    wait_lgkm0();
    __builtin_amdgcn_s_barrier();
    if (m >= nt) return;
    issue_ids(m + 3);
    issue_tile(m + 1, 1);
    issue_tile(m + 2, 0);
    softmax(tbeg + m, tbeg + m >= j_mask);
  };
  if (half == 0) {
    for (int m = 0; m <= ns; ++m) {
      interval_m(m);
      interval_v(m);
    }
  } else {
    wait_lgkm0();
    __builtin_amdgcn_s_barrier();
    for (int m = 0; m < ns; ++m) {
      interval_m(m);
      interval_v(m);
    }
    interval_m(ns);
  }

  // Merge the halves' softmax states through LDS (the rings are free now): half 1
  // writes (m, l, O) per lane, half 0 reads its partner lane's (same rows, same lane
  // layout) and scales both by 2^(m_half - max).
  constexpr int NE = RT * (2 + 4 * DTL);  // floats per lane
  static_assert(4 * NE * kWave * 4 <= (int)sizeof(ring), "merge exchange must fit the rings");
  float* xch = reinterpret_cast<float*>(&ring[0][0][0][0]) + wave * NE * kWave + lane;
  // The last VALU phases issued loads nothing waited for (past the half's end, into
  // free stages); they must land before the rings are reused.
  wait_vmcnt<0>();
  __syncthreads();
  if (half) {
#pragma unroll
    for (int t = 0; t < RT; ++t) {
      float* x = xch + t * (2 + 4 * DTL) * kWave;
      x[0] = m_run[t];
      x[kWave] = l_run[t];
#pragma unroll
      for (int d = 0; d < DTL; ++d)
#pragma unroll
        for (int r = 0; r < 4; ++r) x[(2 + 4 * d + r) * kWave] = o[t][d][r];
    }
  }
  __syncthreads();
  if (half) return;
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    const float* x = xch + t * (2 + 4 * DTL) * kWave;
    const float mb = x[0];
    const float mn = fmaxf(m_run[t], mb);
    const float mref = mn == -INFINITY ? 0.f : mn;  // both empty: weights 0
    const float sa = __builtin_amdgcn_exp2f(m_run[t] - mref);
    const float sb = __builtin_amdgcn_exp2f(mb - mref);
    m_run[t] = mn;
    l_run[t] = l_run[t] * sa + x[kWave] * sb;
#pragma unroll
    for (int d = 0; d < DTL; ++d)
#pragma unroll
      for (int r = 0; r < 4; ++r) o[t][d][r] = o[t][d][r] * sa + x[(2 + 4 * d + r) * kWave] * sb;
  }

  // O^T lane (row col, grp) holds dims 16 d + 4 grp + r of query row col.
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    const float l_tot = rows_sum(l_run[t]);
    if (!row_ok[t]) continue;
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    const int rho = rho0 + 16 * RT * wave + 16 * t + col;
    if (a.lse && grp == 0)  // log2 normaliser: the exponent reference m_run plus log2(sum)
      a.lse[(int64_t)(q0 + rho / G) * a.nh + kvh * G + rho % G] =
          l_tot > 0.f ? m_run[t] + __log2f(l_tot) : -INFINITY;
    const int64_t e0 = (int64_t)(q0 + rho / G) * a.out_st + (int64_t)(kvh * G + rho % G) * a.out_sh;
#pragma unroll
    for (int d = 0; d < DTL; ++d) {
      const int64_t e = e0 + 16 * d + 4 * grp;
      const float v4[4] = {o[t][d][0] * inv, o[t][d][1] * inv, o[t][d][2] * inv, o[t][d][3] * inv};
      if (a.out_f32) {
        *reinterpret_cast<float4*>((float*)a.out + e) = make_float4(v4[0], v4[1], v4[2], v4[3]);
      } else {
        *reinterpret_cast<uint2*>((S*)a.out + e) =
            make_uint2((uint32_t)Elt<DT>::from_f32(v4[0]) | ((uint32_t)Elt<DT>::from_f32(v4[1]) << 16),
                       (uint32_t)Elt<DT>::from_f32(v4[2]) | ((uint32_t)Elt<DT>::from_f32(v4[3]) << 16));
      }
    }
  }
}

// ---------------------------------------------------------------------------------
// Host-side dispatch.
// ---------------------------------------------------------------------------------

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Decode scratch, byte offsets of its areas (each 256-byte aligned): the merge plans
// [batch] int4 (split or cascade), the partial records [num_wg, 2, nh, hd] fp32 and
// their (max, sum) pairs (split: num_wg > 1), and the finished-sequence outputs
// [batch, nh, hd] fp32 with their normalisers [batch, nh] (cascade). total = 0: no
// scratch needed.
struct DecodeWs {
  int64_t desc = -1, acc = -1, ml = -1, tail_o = -1, tail_lse = -1, total = 0;
};
DecodeWs decode_ws(int32_t num_wg, int32_t batch, int32_t nh, int32_t hd, bool cascade) {
  DecodeWs w;
  const bool split = num_wg > 1;
  if (batch <= 0 || nh <= 0 || hd <= 0 || !(split || cascade)) return w;
  int64_t at = 0;
  auto place = [&](int64_t bytes) {
    const int64_t off = (at + 255) / 256 * 256;
    at = off + bytes;
    return off;
  };
  w.desc = place((int64_t)batch * 16);
  if (split) {
    const int64_t recs = (int64_t)num_wg * 2 * nh;
    w.acc = place(recs * hd * 4);
    w.ml = place(recs * 2 * 4);
  }
  if (cascade) {
    w.tail_o = place((int64_t)batch * nh * hd * 4);
    w.tail_lse = place((int64_t)batch * nh * 4);
  }
  w.total = at;
  return w;
}
inline int dtype_bytes(int dt) { return dt == PKV_F32 ? 4 : 2; }
inline bool valid_dtype(int dt) { return dt == PKV_F32 || dt == PKV_F16 || dt == PKV_BF16; }

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

// Run f.run<DT, HD, GPW>() for the runtime (dtype, head_dim, heads per wave).
template <int DT, int HD, class F> hipError_t by_gpw(int gpw, const F& f) {
  switch (gpw) {
    case 1: return f.template run<DT, HD, 1>();
    case 2: return f.template run<DT, HD, 2>();
    case 3: return f.template run<DT, HD, 3>();
    default: return f.template run<DT, HD, 4>();
  }
}
template <int DT, class F> hipError_t by_hd(int hd, int gpw, const F& f) {
  switch (hd) {
    case 16: return by_gpw<DT, 16>(gpw, f);
    case 32: return by_gpw<DT, 32>(gpw, f);
    case 64: return by_gpw<DT, 64>(gpw, f);
    case 128: return by_gpw<DT, 128>(gpw, f);
    default: return by_gpw<DT, 256>(gpw, f);
  }
}
template <class F> hipError_t by_dtype(int dt, int hd, int gpw, const F& f) {
  switch (dt) {
    case PKV_F32: return by_hd<PKV_F32>(hd, gpw, f);
    case PKV_F16: return by_hd<PKV_F16>(hd, gpw, f);
    default: return by_hd<PKV_BF16>(hd, gpw, f);
  }
}

// The MFMA kernel serves 16-bit K/V at head_dim 128; every other shape uses the
// generic stream kernel.
template <int DT, int HD> constexpr bool use_mfma() {
  return DT != PKV_F32 && HD == 128 && PKV_DECODE_USE_MFMA;
}
template <int DT, int HD, int GPW> const void* decode_kernel() {
  if constexpr (use_mfma<DT, HD>())
    return reinterpret_cast<const void*>(&paged_decode_mfma_kernel<DT, GPW, true>);
  else
    return reinterpret_cast<const void*>(&paged_decode_stream_kernel<DT, HD, GPW>);
}

struct LaunchDecode {
  const DecodeArgs* a;
  int wpg, ygrid;
  hipStream_t st;
  template <int DT, int HD, int GPW> hipError_t run() const {
    const dim3 grid((unsigned)a->num_wg, (unsigned)ygrid), block(kWave * wpg);
    if constexpr (use_mfma<DT, HD>()) {
      if (a->bs % 16 == 0)
        hipLaunchKernelGGL((paged_decode_mfma_kernel<DT, GPW, true>), grid, block, 0, st, *a);
      else
        hipLaunchKernelGGL((paged_decode_mfma_kernel<DT, GPW, false>), grid, block, 0, st, *a);
    } else {
      hipLaunchKernelGGL((paged_decode_stream_kernel<DT, HD, GPW>), grid, block, 0, st, *a);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || (a->num_wg <= 1 && !a->pre_row)) return e;
    const int waves = a->batch * a->nh;
    hipLaunchKernelGGL((paged_decode_combine_kernel<DT, HD>), dim3((unsigned)((waves + 3) / 4)),
                       dim3(256), 0, st, *a);
    return hipGetLastError();
  }
};

// Unit size (TILE tokens) of an instantiation, and how many of its workgroups one CU
// holds at once.
struct QueryDecode {
  int wpg;
  int* tile;
  int* per_cu;  // may be null: tile only
  template <int DT, int HD, int GPW> hipError_t run() const {
    *tile = DecodeShape<DT, HD>::TILE;
    if (!per_cu) return hipSuccess;
    return hipOccupancyMaxActiveBlocksPerMultiprocessor(per_cu, decode_kernel<DT, HD, GPW>(),
                                                         kWave * wpg, 0);
  }
};

// Query heads per wave: the whole group when it has at most 4 heads (the register
// budget of 4 heads x 8 fp32 accumulators keeps the kernel spill-free at hd 256), else
// the largest of {4, 3, 2} that divides the group, else 1. Waves that share a KV head
// read the same rows within a few hundred cycles of each other, so the repeat is served
// from L2, not HBM.
int pick_gpw(int groups) {
  if (groups <= 4) return groups;
  const int cands[3] = {4, 3, 2};
  for (int c : cands)
    if (groups % c == 0) return c;
  return 1;
}

// Waves per workgroup and workgroups along y for num_kv_heads x (groups / gpw) tasks.
struct DecodePlan {
  int gpw, nsub, wpg, ygrid;
};
DecodePlan plan_decode(int num_heads, int num_kv_heads) {
  DecodePlan p;
  const int groups = num_heads / num_kv_heads;
  p.gpw = pick_gpw(groups);
  p.nsub = groups / p.gpw;
  const int tasks = num_kv_heads * p.nsub;
  p.wpg = tasks < PKV_DECODE_WAVES_PER_WG ? tasks : PKV_DECODE_WAVES_PER_WG;
  p.ygrid = (tasks + p.wpg - 1) / p.wpg;
  return p;
}

int check_decode_shape(int kv_dtype, int head_dim, int num_heads, int num_kv_heads) {
  if (!valid_dtype(kv_dtype)) return PKV_E_DTYPE;
  if (num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0) return PKV_E_SHAPE;
  if (!(head_dim == 16 || head_dim == 32 || head_dim == 64 || head_dim == 128 ||
        head_dim == 256))
    return PKV_E_SHAPE;
  return 0;
}


template <int DT, int HD>
hipError_t launch_prefill_hd(PrefillArgs a, int64_t rows, hipStream_t st) {
  constexpr int BM = PrefillShape<HD>::BM;
  a.row_blocks = (int)((rows + BM - 1) / BM);
  const int64_t items = (int64_t)a.row_blocks * a.nkv * a.n_chunks;
  if (items > 0x7FFFFFFF) return hipErrorInvalidValue;
  const dim3 grid((unsigned)items), block(512);
  if (a.bs_shift >= 0)
    hipLaunchKernelGGL((paged_prefill_kernel<DT, HD, true>), grid, block, 0, st, a);
  else
    hipLaunchKernelGGL((paged_prefill_kernel<DT, HD, false>), grid, block, 0, st, a);
  return hipGetLastError();
}

template <int DT>
hipError_t launch_prefill(const PrefillArgs& a, int hd, int64_t rows, hipStream_t st) {
  switch (hd) {
    case 32: return launch_prefill_hd<DT, 32>(a, rows, st);
    case 64: return launch_prefill_hd<DT, 64>(a, rows, st);
    case 128: return launch_prefill_hd<DT, 128>(a, rows, st);
    default: return launch_prefill_hd<DT, 256>(a, rows, st);
  }
}

}  // namespace

extern "C" {

int pkv_abi_version(void) { return 2; }

const char* pkv_status_string(int status) {
  switch (status) {
    case 0: return "ok";
    case PKV_E_DTYPE: return "unsupported dtype";
    case PKV_E_SHAPE: return "unsupported shape (head_dim, group size, block size or sizes)";
    case PKV_E_ALIGN: return "pointer or stride not aligned for 16-byte access";
    case PKV_E_WORKSPACE: return "split-K workspace missing or too small";
    case PKV_E_NULL: return "required pointer is NULL";
    case PKV_E_HIP: return "HIP device query failed (no usable GPU?)";
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
    return dim3((unsigned)gx, (unsigned)n_pairs, (unsigned)(2 * num_layers));
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

int32_t pkv_decode_workgroups(int kv_dtype, int32_t head_dim, int32_t num_heads,
                              int32_t num_kv_heads) {
  const int bad = check_decode_shape(kv_dtype, head_dim, num_heads, num_kv_heads);
  if (bad) return bad;
  const DecodePlan p = plan_decode(num_heads, num_kv_heads);
  int dev = 0, cus = 0, per_cu = 0, tile = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e == hipSuccess) e = by_dtype(kv_dtype, head_dim, p.gpw, QueryDecode{p.wpg, &tile, &per_cu});
  if (e != hipSuccess) return PKV_E_HIP;
  const int g = cus * (per_cu < 1 ? 1 : per_cu) / p.ygrid;
  return g < 1 ? 1 : g;
}

int64_t pkv_decode_workspace_bytes(int32_t num_workgroups, int32_t batch, int32_t num_heads,
                                   int32_t head_dim) {
  return decode_ws(num_workgroups, batch, num_heads, head_dim, false).total;
}

int64_t pkv_cascade_workspace_bytes(int32_t num_workgroups, int32_t batch, int32_t num_heads,
                                    int32_t head_dim) {
  return decode_ws(num_workgroups, batch, num_heads, head_dim, true).total;
}

int pkv_paged_decode(void* out, int out_dtype, int64_t out_stride_b, int64_t out_stride_h,
                     const void* q, int64_t q_stride_b, int64_t q_stride_h,
                     const void* k_cache, const void* v_cache, int kv_dtype,
                     int64_t kv_stride_slot, int64_t kv_stride_head, int64_t num_slots,
                     const int32_t* block_tables, int64_t table_stride, int32_t max_blocks,
                     const int32_t* context_lens, int32_t batch, int32_t num_heads,
                     int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                     float scale, int32_t num_workgroups, void* workspace,
                     int64_t workspace_bytes, void* stream) {
  return pkv_paged_decode_ex(out, out_dtype, out_stride_b, out_stride_h, q, q_stride_b,
                             q_stride_h, k_cache, v_cache, kv_dtype, kv_stride_slot,
                             kv_stride_head, num_slots, block_tables, table_stride, max_blocks,
                             context_lens, batch, num_heads, num_kv_heads, head_dim, block_size,
                             scale, num_workgroups, workspace, workspace_bytes, nullptr,
                             nullptr, nullptr, nullptr, nullptr, 0, 0, stream);
}

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
                        int64_t prefix_stride, void* stream) {
  const int bad = check_decode_shape(kv_dtype, head_dim, num_heads, num_kv_heads);
  if (bad) return bad;
  const bool cascade = prefix_row != nullptr && prefix_parts > 0;
  if (prefix_parts < 0 || prefix_stride < 0) return PKV_E_SHAPE;
  if (cascade && (!prefix_out || !prefix_lse)) return PKV_E_NULL;
  if (cascade && !aligned16(prefix_out)) return PKV_E_ALIGN;
  if (!(out_dtype == kv_dtype || out_dtype == PKV_F32)) return PKV_E_DTYPE;
  if (batch < 0 || block_size <= 0 || max_blocks < 0 || num_workgroups < 1 ||
      num_workgroups > (1 << 24) || batch > (1 << 24))
    return PKV_E_SHAPE;
  if ((int64_t)max_blocks * block_size > (int64_t)1 << 30) return PKV_E_SHAPE;
  if (batch == 0) return 0;
  if (!out || !q || !k_cache || !v_cache || !context_lens || (max_blocks > 0 && !block_tables))
    return PKV_E_NULL;
  const int vec = kv_dtype == PKV_F32 ? 4 : 8;
  if (!aligned16(q) || !aligned16(k_cache) || !aligned16(v_cache) || !aligned16(out) ||
      q_stride_b % vec || q_stride_h % vec || kv_stride_slot % vec || kv_stride_head % vec ||
      out_stride_b % vec || out_stride_h % vec)
    return PKV_E_ALIGN;
  const DecodePlan p = plan_decode(num_heads, num_kv_heads);

  DecodeArgs a;
  a.out = out;
  a.out_sb = out_stride_b;
  a.out_sh = out_stride_h;
  a.q = q;
  a.q_sb = q_stride_b;
  a.q_sh = q_stride_h;
  a.k = k_cache;
  a.v = v_cache;
  a.kv_ss = kv_stride_slot;
  a.kv_sh = kv_stride_head;
  a.num_slots = num_slots;
  a.tables = block_tables;
  a.table_stride = table_stride;
  a.max_blocks = max_blocks;
  a.ctx = context_lens;
  a.batch = batch;
  a.nh = num_heads;
  a.nkv = num_kv_heads;
  a.groups = num_heads / num_kv_heads;
  a.nsub = p.nsub;
  a.bs = block_size;
  a.bs_shift = (block_size & (block_size - 1)) == 0 ? __builtin_ctz(block_size) : -1;
  int tile = 0;
  (void)by_dtype(kv_dtype, head_dim, p.gpw, QueryDecode{p.wpg, &tile, nullptr});
  a.unit_tokens = tile;
  a.num_wg = num_workgroups;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.out_f32 = out_dtype == PKV_F32;
  a.first_block = first_block;
  a.lse = lse;
  a.pre_o = cascade ? prefix_out : nullptr;
  a.pre_lse = cascade ? prefix_lse : nullptr;
  a.pre_row = cascade ? prefix_row : nullptr;
  a.pre_parts = cascade ? prefix_parts : 0;
  a.pre_stride = prefix_stride;
  a.fin = nullptr;
  a.fin_lse = nullptr;
  a.fin_sb = a.fin_sh = 0;
  a.fin_f32 = 0;
  a.desc = nullptr;
  a.ws_acc = nullptr;
  a.ws_ml = nullptr;
  const DecodeWs ws = decode_ws(num_workgroups, batch, num_heads, head_dim, cascade);
  if (ws.total) {
    if (!workspace || workspace_bytes < ws.total || !aligned16(workspace)) return PKV_E_WORKSPACE;
    char* base = (char*)workspace;
    a.desc = (int4*)(base + ws.desc);
    if (ws.acc >= 0) {
      a.ws_acc = (float*)(base + ws.acc);
      a.ws_ml = (float*)(base + ws.ml);
    }
    if (cascade) {  // the stream pass finishes sequences into fp32 scratch; combine merges
      a.fin = out;
      a.fin_sb = out_stride_b;
      a.fin_sh = out_stride_h;
      a.fin_f32 = a.out_f32;
      a.fin_lse = lse;
      a.out = base + ws.tail_o;
      a.out_sb = (int64_t)num_heads * head_dim;
      a.out_sh = head_dim;
      a.out_f32 = 1;
      a.lse = (float*)(base + ws.tail_lse);
    }
  }

  hipStream_t st = (hipStream_t)stream;
  return (int)by_dtype(kv_dtype, head_dim, p.gpw, LaunchDecode{&a, p.wpg, p.ygrid, st});
}

int pkv_paged_prefill(void* out, int out_dtype, int64_t out_stride_tok, int64_t out_stride_h,
                      const void* q, int64_t q_stride_tok, int64_t q_stride_h,
                      const void* k_cache, const void* v_cache, int kv_dtype,
                      int64_t kv_stride_slot, int64_t kv_stride_head, int64_t num_slots,
                      const int32_t* block_tables, int64_t table_stride, int32_t max_blocks,
                      const int32_t* context_lens, const int32_t* cu_seqlens_q, int32_t n_chunks,
                      int32_t max_query_len, int32_t num_heads, int32_t num_kv_heads,
                      int32_t head_dim, int32_t block_size, float scale, void* stream) {
  return pkv_paged_prefill_ex(out, out_dtype, out_stride_tok, out_stride_h, q, q_stride_tok,
                              q_stride_h, k_cache, v_cache, kv_dtype, kv_stride_slot,
                              kv_stride_head, num_slots, block_tables, table_stride, max_blocks,
                              context_lens, cu_seqlens_q, n_chunks, max_query_len, num_heads,
                              num_kv_heads, head_dim, block_size, scale, 1, nullptr, nullptr,
                              stream);
}

int pkv_paged_prefill_ex(void* out, int out_dtype, int64_t out_stride_tok, int64_t out_stride_h,
                         const void* q, int64_t q_stride_tok, int64_t q_stride_h,
                         const void* k_cache, const void* v_cache, int kv_dtype,
                         int64_t kv_stride_slot, int64_t kv_stride_head, int64_t num_slots,
                         const int32_t* block_tables, int64_t table_stride, int32_t max_blocks,
                         const int32_t* context_lens, const int32_t* cu_seqlens_q,
                         int32_t n_chunks, int32_t max_query_len, int32_t num_heads,
                         int32_t num_kv_heads, int32_t head_dim, int32_t block_size, float scale,
                         int32_t causal, const int32_t* q_rows, float* lse, void* stream) {
  if (!(kv_dtype == PKV_BF16 || kv_dtype == PKV_F16)) return PKV_E_DTYPE;
  if (!(out_dtype == kv_dtype || out_dtype == PKV_F32)) return PKV_E_DTYPE;
  if (num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads || block_size <= 0 ||
      max_blocks < 0 || n_chunks < 0 || n_chunks > 65535 || max_query_len < 0 ||
      num_kv_heads > 65535)
    return PKV_E_SHAPE;
  if (!(head_dim == 32 || head_dim == 64 || head_dim == 128 || head_dim == 256)) return PKV_E_SHAPE;
  if ((int64_t)max_blocks * block_size > (int64_t)1 << 30) return PKV_E_SHAPE;
  if (!(scale > 0.f && scale < INFINITY)) return PKV_E_SHAPE;  // softmax scale
  const int64_t rows = (int64_t)max_query_len * (num_heads / num_kv_heads);
  if (rows > (int64_t)1 << 30) return PKV_E_SHAPE;
  if (n_chunks == 0 || max_query_len == 0) return 0;
  if (!out || !q || !k_cache || !v_cache || !context_lens || !cu_seqlens_q ||
      (max_blocks > 0 && !block_tables))
    return PKV_E_NULL;
  if (!aligned16(q) || !aligned16(k_cache) || !aligned16(v_cache) || !aligned16(out) ||
      q_stride_tok % 8 || q_stride_h % 8 || kv_stride_slot % 8 || kv_stride_head % 8 ||
      out_stride_tok % 8 || out_stride_h % 8)
    return PKV_E_ALIGN;
  PrefillArgs a;
  a.out = out;
  a.out_st = out_stride_tok;
  a.out_sh = out_stride_h;
  a.q = q;
  a.q_st = q_stride_tok;
  a.q_sh = q_stride_h;
  a.k = k_cache;
  a.v = v_cache;
  a.kv_ss = kv_stride_slot;
  a.kv_sh = kv_stride_head;
  a.num_slots = num_slots;
  a.tables = block_tables;
  a.table_stride = table_stride;
  a.max_blocks = max_blocks;
  a.ctx = context_lens;
  a.cu_q = cu_seqlens_q;
  a.n_chunks = n_chunks;
  a.nh = num_heads;
  a.nkv = num_kv_heads;
  a.groups = num_heads / num_kv_heads;
  a.bs = block_size;
  a.bs_shift = (block_size & (block_size - 1)) == 0 ? __builtin_ctz(block_size) : -1;
  a.row_blocks = 0;  // set per head_dim by launch_prefill
  a.causal = causal != 0;
  a.q_rows = q_rows;
  a.lse = lse;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.out_f32 = out_dtype == PKV_F32;
  hipStream_t st = (hipStream_t)stream;
  return (int)(kv_dtype == PKV_BF16 ? launch_prefill<PKV_BF16>(a, head_dim, rows, st)
                                    : launch_prefill<PKV_F16>(a, head_dim, rows, st));
}

}  // extern "C"
