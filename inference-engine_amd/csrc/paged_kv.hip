// paged_kv.hip — gfx950 kernels for the paged-KV hot path behind the C ABI of
// include/paged_kv.h: slot-mapped KV append, block copy, and split-K paged decode
// attention with its combine pass.
//
// Written for CDNA4 wave64: 16-byte global loads, DPP row reductions, v_exp_f32 for
// the softmax (exp2 with log2(e) folded into the query scale), fp32 accumulation.

#include <hip/hip_runtime.h>
#include <stdint.h>

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
  float* ws_acc;        // [num_wg, 2, nh, HD] partial records
  float* ws_ml;         // [num_wg, 2, nh, 2]   their (max, sum)
  int out_f32;
};

// Clamped context length of sequence b: 0 <= n <= max_blocks * block_size.
__device__ __forceinline__ int clamped_ctx(const DecodeArgs& a, int b) {
  const int n = a.ctx[b];
  const int cap = a.max_blocks * a.bs;
  return n < 0 ? 0 : (n > cap ? cap : n);
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
    auto load_table = [&](int first_block) {
      cb = first_block;
      const int j = cb + lane;
      tbl = j < a.max_blocks ? a.tables[b * a.table_stride + j] : 0;
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

// Second stage: one wave per (sequence, query head). A sequence whose units span
// workgroups w0..w1 (w0 < w1) has one record in each non-empty range among them (in
// w0 it is the range's last piece, slot 1, unless the range starts with it); they are
// merged with log-sum-exp weights w_j = exp2(m_j - max m), out = sum w_j acc_j /
// sum w_j l_j. Lane j holds record j's weight; eight records are loaded per step.
template <int DTO>
__global__ void __launch_bounds__(256)
paged_decode_combine_kernel(const DecodeArgs a, int hd) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wid = blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  if (wid >= a.batch * a.nh) return;  // uniform per wave
  const int b = wid / a.nh, h = wid - b * a.nh;

  int64_t total, ub;
  find_unit(a, -1, &total);
  // first unit of sequence b: the units of sequences before it
  {
    int64_t base = 0;
    for (int c0 = 0; c0 < b; c0 += kWave) {
      const int bb = c0 + lane;
      int cnt = bb < b ? units_of(a, clamped_ctx(a, bb)) : 0;
#pragma unroll
      for (int m = 1; m < kWave; m <<= 1) cnt += __shfl_xor(cnt, m);
      base += cnt;
    }
    ub = base;
  }
  const int64_t ue = ub + units_of(a, clamped_ctx(a, b));
  const int64_t G = a.num_wg;
  const int64_t w0 = wg_of_unit(ub, total, G), w1 = wg_of_unit(ue - 1, total, G);
  if (w0 == w1) return;  // written directly by the split pass
  const int nrec = (int)(w1 - w0 + 1);

  auto record = [&](int j, bool* live) -> int64_t {
    const int64_t ww = w0 + j;
    const int64_t s0 = range_start(ww, total, G);
    *live = s0 < range_start(ww + 1, total, G);
    const int slot = (ww == w0 && s0 < ub) ? 1 : 0;
    return (ww * 2 + slot) * a.nh + h;
  };

  float mmax = -INFINITY;
  for (int j = lane; j < nrec; j += kWave) {
    bool live;
    const int64_t r = record(j, &live);
    if (live) mmax = fmaxf(mmax, a.ws_ml[2 * r]);
  }
#pragma unroll
  for (int m = 1; m < kWave; m <<= 1) mmax = fmaxf(mmax, __shfl_xor(mmax, m));
  if (mmax == -INFINITY) mmax = 0.f;  // no live token in any piece: weights 0, output 0

  float out_acc[4] = {0.f, 0.f, 0.f, 0.f};  // dims lane + 64 k
  float lsum = 0.f;
  for (int c0 = 0; c0 < nrec; c0 += kWave) {
    const int j = c0 + lane;
    float wgt = 0.f;
    int64_t r = 0;
    if (j < nrec) {
      bool live;
      r = record(j, &live);
      if (live) {
        const float2 ml = *reinterpret_cast<const float2*>(a.ws_ml + 2 * r);
        wgt = __builtin_amdgcn_exp2f(ml.x - mmax);
        lsum = __builtin_fmaf(wgt, ml.y, lsum);
      } else {
        r = 0;
      }
    }
    const int cn = min(kWave, nrec - c0);
    for (int j0 = 0; j0 < cn; j0 += 8) {
      float wv[8];
      float x[8][4];
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) {
        const int src = min(j0 + jj, cn - 1);  // clamped duplicates get weight 0 below
        wv[jj] = j0 + jj < cn
                     ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wgt), src))
                     : 0.f;
        const int lo = __builtin_amdgcn_readlane((int)(r & 0xFFFFFFFF), src);
        const int hi = __builtin_amdgcn_readlane((int)(r >> 32), src);
        const int64_t rr = ((int64_t)hi << 32) | (uint32_t)lo;
        const float* rowp = a.ws_acc + rr * hd;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          // rows of dead or duplicate records are never read: the workspace holds
          // whatever the allocator left there, possibly NaN bit patterns
          x[jj][k] = (wv[jj] != 0.f && lane + 64 * k < hd) ? rowp[lane + 64 * k] : 0.f;
        }
      }
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) {
#pragma unroll
        for (int k = 0; k < 4; ++k) out_acc[k] = __builtin_fmaf(wv[jj], x[jj][k], out_acc[k]);
      }
    }
  }
#pragma unroll
  for (int m = 1; m < kWave; m <<= 1) lsum += __shfl_xor(lsum, m);
  const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int d = lane + 64 * k;
    if (d >= hd) break;
    const float o = out_acc[k] * inv;
    const int64_t e = b * a.out_sb + (int64_t)h * a.out_sh + d;
    if constexpr (DTO == PKV_F32) reinterpret_cast<float*>(a.out)[e] = o;
    else reinterpret_cast<typename Elt<DTO>::S*>(a.out)[e] = Elt<DTO>::from_f32(o);
  }
}

// ---------------------------------------------------------------------------------
// Host-side dispatch.
// ---------------------------------------------------------------------------------

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }
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

struct LaunchDecode {
  const DecodeArgs* a;
  int wpg, ygrid;
  hipStream_t st;
  template <int DT, int HD, int GPW> hipError_t run() const {
    hipLaunchKernelGGL((paged_decode_stream_kernel<DT, HD, GPW>),
                       dim3((unsigned)a->num_wg, (unsigned)ygrid), dim3(kWave * wpg), 0, st, *a);
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
    return hipOccupancyMaxActiveBlocksPerMultiprocessor(
        per_cu, reinterpret_cast<const void*>(&paged_decode_stream_kernel<DT, HD, GPW>),
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

}  // namespace

extern "C" {

int pkv_abi_version(void) { return 1; }

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

int64_t pkv_decode_workspace_bytes(int32_t num_workgroups, int32_t num_heads,
                                   int32_t head_dim) {
  if (num_workgroups <= 1 || num_heads <= 0 || head_dim <= 0) return 0;
  const int64_t recs = (int64_t)num_workgroups * 2 * num_heads;
  return (recs * head_dim * 4 + 255) / 256 * 256 + recs * 2 * 4;
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
  const int bad = check_decode_shape(kv_dtype, head_dim, num_heads, num_kv_heads);
  if (bad) return bad;
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
  a.ws_acc = nullptr;
  a.ws_ml = nullptr;
  if (num_workgroups > 1) {
    const int64_t need = pkv_decode_workspace_bytes(num_workgroups, num_heads, head_dim);
    if (!workspace || workspace_bytes < need || !aligned16(workspace)) return PKV_E_WORKSPACE;
    const int64_t recs = (int64_t)num_workgroups * 2 * num_heads;
    a.ws_acc = (float*)workspace;
    a.ws_ml = (float*)((char*)workspace + (recs * head_dim * 4 + 255) / 256 * 256);
  }

  hipStream_t st = (hipStream_t)stream;
  hipError_t e = by_dtype(kv_dtype, head_dim, p.gpw, LaunchDecode{&a, p.wpg, p.ygrid, st});
  if (e != hipSuccess || num_workgroups <= 1) return (int)e;

  const int waves = batch * num_heads;
  const dim3 cgrid((unsigned)((waves + 3) / 4));
  switch (out_dtype) {
    case PKV_F32:
      hipLaunchKernelGGL(paged_decode_combine_kernel<PKV_F32>, cgrid, dim3(256), 0, st, a,
                         head_dim);
      break;
    case PKV_F16:
      hipLaunchKernelGGL(paged_decode_combine_kernel<PKV_F16>, cgrid, dim3(256), 0, st, a,
                         head_dim);
      break;
    default:
      hipLaunchKernelGGL(paged_decode_combine_kernel<PKV_BF16>, cgrid, dim3(256), 0, st, a,
                         head_dim);
  }
  return (int)hipGetLastError();
}

}  // extern "C"
