// prefill_kernels.h -- chunked-prefill attention on the matrix cores (gfx950 device
// code). prefill.hip launches it for chunked prefill and cascade decode's prefix pass;
// cascade.hip runs the same item code inside the one-launch cascade.

#pragma once

#include "common.h"

namespace pkv {

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
  // bf16 caches: an fp16 copy of each chunk's V (null: none; the kernel with the copy is
  // launched only with one). Part (c, h) (chunk c, KV head h) starts at token slot
  // (c * nkv + h) * PM, PM = max_blocks * bs rounded up to kV16Rows, a slot being
  // head_dim fp16 values, and covers the chunk's clamped context rounded up to kV16Rows
  // (tokens past the context are zero). Each KT-token tile of the prefill (PrefillShape)
  // is stored in V^T operand order, not by rows: its fragment (32-key step sg, 16-dim
  // tile d) is 1 KiB, lane l's 16 bytes (dims 16 d + l % 16 of the tile's keys 32 sg +
  // 16 (e / 4) + 4 (l / 16) + e % 4, e = 0 .. 7) at l * 16. Region tile i (tokens i
  // kV16Rows ..) of part (c, h) holds V * 2^-k with k = v16_k[(c * nkv + h) * v16_kstride
  // + i] (0 unless some |V| of the tile is 2^16 or more), so every value fits fp16.
  const void* v16;
  const uint8_t* v16_k;
  int32_t v16_kstride;
};

// Tokens per region tile of the fp16 V copy (one workgroup of the copy kernel, one scale
// exponent); regions are padded to a multiple of it.
constexpr int kV16Rows = 256;
// Threads of a workgroup of the copy (one per region tile).
constexpr int kV16Threads = 512;
// Longest context the copy takes: a wave holds one chunk's scale exponents, four per lane.
constexpr int kV16MaxTokens = kV16Rows * 4 * kWave;
__host__ __device__ __forceinline__ int v16_pad(int n) {
  return (n + kV16Rows - 1) / kV16Rows * kV16Rows;
}

}  // namespace pkv

// Tuning knobs of the matrix-core prefill (compile-time; the defaults are the measured
// best on MI355X).
// Matrix phase: operand fragments read this many fragment steps ahead of their MFMAs.
#ifndef PKV_PREFILL_PIPE
#define PKV_PREFILL_PIPE 2
#endif
// The softmax packs every 32-key step's P fragments (1) or only the first (0; the matrix
// phase packs the others).
#ifndef PKV_PREFILL_PACK_ALL
#define PKV_PREFILL_PACK_ALL 1
#endif
// P's lo half (bf16 caches) from v_dot2c_f32_bf16 (1) or unpack-and-subtract (0).
#ifndef PKV_PREFILL_DOT2LO
#define PKV_PREFILL_DOT2LO 0
#endif
// Wave priority (s_setprio): 1 raises the softmax phase's, 2 raises half 1's waves'
// (younger, so otherwise second in issue arbitration), 0 leaves both at 0.
// 1: a VALU phase whose two tiles take the 16-token-block fast path fetches both tiles'
// block ids before waiting on either (one scalar-load round trip, not two; measured
// 0.7% faster at config 5); 0: one fetch and wait per tile.
#ifndef PKV_PREFILL_IDS2
#define PKV_PREFILL_IDS2 1
#endif
#ifndef PKV_PREFILL_VALU_PRIO
#define PKV_PREFILL_VALU_PRIO 0
#endif
// 1: the matrix-core prefill raises a wave's priority for its matrix phases (measured
// with the fp16 P.V: 80.1-80.2 against 81.1-81.6 µs per config-5 call, config 3's
// cascade unchanged; with the bf16 hi + lo product it had cost 2%); 0: no priorities.
#ifndef PKV_PREFILL_SETPRIO
#define PKV_PREFILL_SETPRIO 1
#endif
// Waves of a half (of 4) that issue their VALU phase's K/V loads after the softmax
// instead of before it.
#ifndef PKV_PREFILL_LATE_DMA
#define PKV_PREFILL_LATE_DMA 2
#endif
// 1: a wave masks its tile's scores and takes their row maxima at the end of the matrix
// phase that computed them, not at the start of the softmax phase.
#ifndef PKV_PREFILL_EARLY_MAX
#define PKV_PREFILL_EARLY_MAX 1
#endif
// 1: the steady-state matrix phase issues QK^T of its tile before P.V of the previous
// one, so the scores are in when the phase ends and takes their row maxima (measured at
// config 5: 77.75-77.80 against 77.56-77.64 µs per call for 0, 16 more VGPRs).
#ifndef PKV_PREFILL_QK_FIRST
#define PKV_PREFILL_QK_FIRST 0
#endif

namespace {

using namespace pkv;

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


template <int DT> struct Mfma16x16x32Bits;  // MFMA on raw 16-bit bit patterns
template <> struct Mfma16x16x32Bits<PKV_BF16> {
  typedef __bf16 v8 __attribute__((ext_vector_type(8)));
  typedef __bf16 v2 __attribute__((ext_vector_type(2)));
  // bf16 keeps 8 significant bits, too few for softmax weights at a 2e-3 output bar, so
  // P enters the product as hi = bf16(P) plus lo = bf16(P - hi) (two MFMAs).
  static constexpr bool kSplit = true;
  static constexpr uint32_t kOnePair = 0x3F803F80u;  // two bf16 1.0
  static constexpr float kPLog2 = 0.f;  // bf16's exponent range holds every weight
  __device__ static f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8, a),
                                                   __builtin_bit_cast(v8, b), c, 0, 0, 0);
  }
  // 8 finite fp32 -> hi and lo operand fragments (pack_p8: v_cvt_pk_bf16_f32, round to
  // nearest even; lo = p - hi is exact).
  __device__ static void pack8(const float* p, u32x4& hi, u32x4& lo) {
#if PKV_PREFILL_DOT2LO
    // lo from one v_dot2c_f32_bf16 per value (p + hi_pair . (-1, 0)). The pairs (-1, 0)
    // and (0, -1) go in as registers with these exact bits: left to itself the compiler
    // encodes the first as the inline constant -1.0, whose 32-bit pattern is the second
    // pair (lo of p0 then came out as p0 - hi of p1). Measured slower than pack_p8's two
    // plain instructions per value (the dot product issues at a lower rate).
    uint32_t h[4], l[4];
    uint32_t neg_lo = 0x0000BF80u, neg_hi = 0xBF800000u;
    __asm__("" : "+v"(neg_lo), "+v"(neg_hi));
    const v2 c0 = __builtin_bit_cast(v2, neg_lo), c1 = __builtin_bit_cast(v2, neg_hi);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const v2 hp = v2{(__bf16)p[2 * i], (__bf16)p[2 * i + 1]};
      h[i] = __builtin_bit_cast(uint32_t, hp);
      const float r0 = __builtin_amdgcn_fdot2_f32_bf16(hp, c0, p[2 * i], false);
      const float r1 = __builtin_amdgcn_fdot2_f32_bf16(hp, c1, p[2 * i + 1], false);
      l[i] = __builtin_bit_cast(uint32_t, v2{(__bf16)r0, (__bf16)r1});
    }
    hi = u32x4{h[0], h[1], h[2], h[3]};
    lo = u32x4{l[0], l[1], l[2], l[3]};
#else
    pack_p8<PKV_BF16>(p, hi, lo);
#endif
  }
};
template <> struct Mfma16x16x32Bits<PKV_F16> {
  typedef _Float16 v8 __attribute__((ext_vector_type(8)));
  typedef _Float16 v2 __attribute__((ext_vector_type(2)));
  static constexpr bool kSplit = false;  // fp16 keeps 11 bits: P rounded once
  static constexpr uint32_t kOnePair = 0x3C003C00u;  // two fp16 1.0
  // P carries a factor 2^kPLog2 (folded into the exponent's offset): weights down to
  // 2^-31 of the reference stay at or above fp16's smallest subnormal (2^-24) instead of
  // rounding to zero, and the largest, below 2^(8 + 7), stays below fp16's maximum. The
  // row sums carry the same factor, so O / l is unchanged; the log-sum-exp takes it out.
  static constexpr float kPLog2 = 7.f;
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

// Maximum over lanes l, l^16, l^32, l^48 (the four rows of a column) of scores that are
// finite or -inf. The swaps return raw bits, which fmaxf would first canonicalise (two
// extra instructions per step); these values are never signalling NaNs, so v_max_f32
// takes them as they are.
__device__ __forceinline__ float score_rows_max(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  float y;
  __asm__("v_max_f32 %0, %1, %2" : "=v"(y) : "v"(__uint_as_float(a[0])), "v"(__uint_as_float(a[1])));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(y), __float_as_uint(y), false, false);
  __asm__("v_max_f32 %0, %1, %2" : "=v"(y) : "v"(__uint_as_float(b[0])), "v"(__uint_as_float(b[1])));
  return y;
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
  // 128, 16 chunks). With 64 banks (a 256-byte window), a ds_read_b128 serves 16 lanes
  // and a ds_read_b64 32 lanes per pass: the K operand reads (16 consecutive keys, one
  // chunk) are conflict-free when swz is a bijection of the key's low 4 bits, the V^T
  // transpose reads (8 consecutive keys x chunks 2d, 2d + 1 per 32 lanes) when swz's
  // bits 1-3 are a bijection of the key's bits 0-2. swz(t) = (t3, t0, t1, t2) -- bits
  // 0..3 -- satisfies both (PKV_PREFILL_SWZ 1; measured at config 5: half the bank-
  // conflict cycles of the 32-bank layout (t2, t0, t1, t3), same results, same time).
  __device__ static int swz(int t) {
#if PKV_PREFILL_SWZ == 1
    if constexpr (CH == 16) return ((t & 7) << 1) | ((t >> 3) & 1);
#else
    if constexpr (CH == 16) return ((t << 1) & 6) | ((t >> 2) & 1) | (t & 8);
#endif
    else return t % CH;
  }
  // LDS byte offset (inside a 32-key step of a tile) of lane l's V^T transpose read:
  // lane (col, grp) reads key 16 h2 + 4 grp + col / 4, dims 16 d + 4 (col % 4) .. +4
  // (chunk 2 d + (col % 4) / 2, half (col % 4) & 1); h2 > 0 only when rows have more
  // than 16 chunks.
  __device__ static uint32_t voff(int l, int h2, int d) {
    const int c4 = l & 3, tr = 4 * (l >> 4) + ((l & 15) >> 2);
    const int tk = 16 * h2 + tr;
    return (uint32_t)((((2 * d + c4 / 2) ^ swz(tk)) * 16 + (c4 & 1) * 8) + tr * CH * 16);
  }
};

// The V^T operand fragment (32-key step sg, 16-dim tile d) of a V tile held in LDS in the
// swizzled row layout: two ds_read_b64_tr_b16 transpose reads per lane. Lane (col, grp)
// gets dims 16 d + col of keys 32 sg + 16 (e / 4) + 4 grp + e % 4, e = 0 .. 7 -- the
// order in which a lane holds its own probabilities P^T.
template <int HD>
__device__ __forceinline__ u32x4 vt_frag_tr(const char* vstage, int l, int sg, int d) {
  using SH = PrefillShape<HD>;
  constexpr int CH = SH::CH, VSW = CH > 16 ? 2 : 1;
  u32x4 f;
#pragma unroll
  for (int h2 = 0; h2 < 2; ++h2) {
    // generic -> LDS address space (an addrspacecast of a __shared__ pointer)
    const s16x4 x = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_s16x4*)(vstage + (32 * sg + 16 * h2) * CH * 16 + SH::voff(l, VSW == 1 ? 0 : h2, d)));
    const uint32_t lo = (uint32_t)(uint16_t)x[0] | ((uint32_t)(uint16_t)x[1] << 16);
    const uint32_t hi = (uint32_t)(uint16_t)x[2] | ((uint32_t)(uint16_t)x[3] << 16);
    if (h2 == 0) { f.x = lo; f.y = hi; } else { f.z = lo; f.w = hi; }
  }
  return f;
}

// Coordinates of a work item: chunk c (query rows q0 .. q1 - 1, n context tokens), its
// 128-row block rbi and KV head kvh.
struct PrefillItem {
  int c, q0, q1, n, kvh, rbi;
};

// The K/V rings of an item: ring[half][0 = K, 1 = V][stage] holds each key half's K and V
// tiles, two stages each; idring the block-table windows, per half and wave, in a ring
// of three (one per tile in flight).
template <int HD> struct PrefillLds {
  u32x4 ring[2][2][2][PrefillShape<HD>::TILE];
  int32_t idring[2][3][4][kWave];
};

// One work item on a workgroup of 512 threads. V16: P.V in fp16 with V from the fp16
// copy. Every exit is workgroup-uniform except half 1's after the merge; a caller that
// runs several items on one workgroup puts a barrier between them (the merge reuses the
// rings).
template <int DT, int HD, bool POW2, bool V16>
__device__ __forceinline__ void prefill_body(const PrefillArgs& a, const PrefillItem& it,
                                             PrefillLds<HD>& lds) {
  using SH = PrefillShape<HD>;
  constexpr int RT = SH::RT, BM = SH::BM, KT = SH::KT, CH = SH::CH, NBETA = SH::NBETA;
  constexpr int NSG = SH::NSG, KS = SH::KS, DTL = SH::DTL, NLD = SH::NLD, TILE = SH::TILE;
  static_assert(HD % 32 == 0 && HD <= 256, "head_dim must be 32..256, a multiple of 32");
  static_assert(!V16 || DT == PKV_BF16, "the fp16 V copy serves bf16 caches");
  using MMA = Mfma16x16x32Bits<DT>;                   // Q.K^T
  using PM = Mfma16x16x32Bits<V16 ? PKV_F16 : DT>;    // P.V and the row sums
  using S = typename Elt<DT>::S;
  auto& ring = lds.ring;
  auto& idring = lds.idring;

  const int tid = threadIdx.x;
  const int half = __builtin_amdgcn_readfirstlane(tid >> 8);  // which half of the key tiles
  const int htid = tid & 255;                                 // thread index inside the half
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(htid / kWave);  // rows 32 wave .. (RT = 2)
  const int col = lane & 15, grp = lane >> 4;
  const int c = it.c, q0 = it.q0, q1 = it.q1, n = it.n, kvh = it.kvh, rbi = it.rbi;
  const int qlen = q1 - q0;
  const int G = a.groups;
  const int nrows = qlen * G;
  const int rho0 = (a.row_blocks - 1 - rbi) * BM;
  if (qlen <= 0 || rho0 >= nrows) return;  // uniform per workgroup
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
    int64_t qrow = q0 + row_tok[t];
    if (a.q_rows) {  // a negative entry: no query there (nothing read or written)
      const int qr = a.q_rows[q0 + row_tok[t]];
      row_ok[t] = row_ok[t] && qr >= 0;
      qrow = qr >= 0 ? qr : 0;
    }
    const S* qp = reinterpret_cast<const S*>(a.q) + qrow * a.q_st +
                  (int64_t)(kvh * G + rr % G) * a.q_sh + 8 * grp;
#pragma unroll
    for (int s = 0; s < KS; ++s) qf[t][s] = *reinterpret_cast<const u32x4*>(qp + 32 * s);
  }
  // V16: the scale exponents of this chunk's KV head part, four per lane (byte i of lane
  // l: region tile 4 l + i); O^T (d < DTL) then holds the outputs times 2^-kcur.
  uint32_t kwin = 0;
  int kcur = 0;
  if constexpr (V16) {
    const int kt16 = v16_pad(n) / kV16Rows;
    const uint8_t* kp = a.v16_k + ((int64_t)c * a.nkv + kvh) * a.v16_kstride;
    kwin = 4 * lane < kt16 ? *reinterpret_cast<const uint32_t*>(kp + 4 * lane) : 0u;
  }
  // A row block of padding only (every q_rows entry negative: a fixed-shape layout's
  // spare rows) leaves before any key tile; the test is workgroup-uniform.
  if (a.q_rows) {
    bool any = false;
#pragma unroll
    for (int t = 0; t < RT; ++t) any = any || row_ok[t];
    if (!__syncthreads_or(any)) return;
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
  // This wave's first granule of a stage: the DMA of instruction r then lands at a
  // compile-time offset r * 4 KiB from it (no per-r register for the wave's part).
  const uint32_t ring_lds = lds_addr(&ring[half][0][0][0]) + (uint32_t)(wave * kWave * 16);
  const uint32_t ids_lds = lds_addr(&idring[half][0][wave][0]);
  // Local tile m of this half is tile tbeg + m; past the half's end, the last one (the
  // loads keep their count; their stages are free).
  auto gtile = [&](int m) { return tbeg + min(m, nt - 1); };
  // One DMA instruction of one wave covers SEG consecutive keys of a tile. When the block
  // size is a power of two >= SEG those keys share one block: its id is wave-uniform and
  // the address is scalar math plus one per-lane offset. The ids then come straight from
  // the table through the scalar cache (s_load, counted in lgkmcnt), not through the LDS
  // ring, whose reads queue behind the matrix waves' operand reads (~1,200 cycles of the
  // VALU phase went to issuing the DMAs that way).
  constexpr int SEG = kWave / CH;
  const bool seg_uniform = POW2 && a.bs >= SEG;
  const uint64_t trow_u = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)trow)) |
                          ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)((uintptr_t)trow >> 32)) << 32);
  typedef __attribute__((address_space(4))) const int32_t c_i32;
  typedef int32_t i32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));
  typedef __attribute__((address_space(4))) const i32x4_a4 c_i32x4;
  auto sid = [&](int b) { return *(c_i32*)(uintptr_t)(trow_u + 4ull * (uint32_t)b); };
  auto sid4 = [&](int b) { return *(c_i32x4*)(uintptr_t)(trow_u + 4ull * (uint32_t)b); };
  // The LDS ring of block ids (other block sizes): the 64 entries from tile m's first
  // block on, two tiles ahead of the K/V loads that read them.
  auto issue_ids = [&](int m) __attribute__((always_inline)) {
    if (seg_uniform) return;
    const int b = min(blk_of(gtile(m) * KT) + lane, blast);
    dma4_to_lds(trow + b, ids_lds + (uint32_t)((m % 3) * 4 * kWave * 4));
  };
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
  // The 16-token-block fast path of K (kv = 0) or V (kv = 1) of local tile m, with the
  // tile's four block ids already fetched (v4).
  auto issue_fast = [&](int m, int kv, const i32x4_a4 v4) __attribute__((always_inline)) {
    const int j = gtile(m);
    const uint32_t dst = ring_lds + (uint32_t)(((kv * 2 + (m & 1)) * TILE) * 16);
    const char* base = kv_base[kv] + (uint32_t)(((j * KT) & (a.bs - 1)) * a.kv_ss * (int)sizeof(S));
#pragma unroll
    for (int r = 0; r < NLD; ++r) {
      uint32_t bid = (uint32_t)__builtin_amdgcn_readfirstlane(v4[r & 3]);
      bid = bid < pool_blocks ? bid : 0u;  // memory safety only
      dma16_to_lds_s(base + (uint64_t)bid * blk_bytes32, lane_off[r], dst + (uint32_t)(r * 256 * 16));
    }
  };
  // 16-token blocks at head_dim 128 (a tile is four blocks, a half four waves; callers
  // check the block size and that the tile lies inside the context): wave w loads block
  // w of the tile, its four DMAs (tokens 4 r .. 4 r + 3 of the block) from one base. The
  // tile's LDS layout is the one above; only which wave fills which granules differs
  // (wave w: granules 256 w .. 256 w + 255), so each wave needs one block id and one
  // address per tile, not four.
  constexpr bool kBlockWave = CH == 16 && NLD == 4 && KT == 64;
  uint32_t lane_offb[NLD];
#pragma unroll
  for (int r = 0; r < NLD; ++r) {
    const int t = 4 * r + lane / CH;  // token inside the block (and its low 4 bits in the tile)
    lane_offb[r] = (uint32_t)((t * a.kv_ss + ((lane % CH) ^ SH::swz(t)) * 8) * (int64_t)sizeof(S));
  }
  const uint32_t ring_lds_bw = lds_addr(&ring[half][0][0][0]) + (uint32_t)(wave * NLD * kWave * 16);
  // This wave's block id of local tile m (a scalar load; the tile is inside the context).
  auto wave_id = [&](int m) { return sid(blk_of(gtile(m) * KT) + wave); };
  auto issue_block = [&](int m, int kv, int id) __attribute__((always_inline)) {
    const uint32_t dst = ring_lds_bw + (uint32_t)(((kv * 2 + (m & 1)) * TILE) * 16);
    uint32_t bid = (uint32_t)id;
    bid = bid < pool_blocks ? bid : 0u;  // memory safety only
    const char* base = kv_base[kv] + (uint64_t)bid * blk_bytes32;
#pragma unroll
    for (int r = 0; r < NLD; ++r) dma16_to_lds_s(base, lane_offb[r], dst + (uint32_t)(r * kWave * 16));
  };
  // V16: local tile m's V from the chunk's fp16 copy, tile j of this KV head's part of the
  // region (zeros past the context, so no clamping), already in operand order: the tile's
  // granules land in LDS in their own order.
  const char* const v16_head =
      V16 ? reinterpret_cast<const char*>(a.v16) +
                ((int64_t)c * a.nkv + kvh) * v16_pad(a.max_blocks * a.bs) * (HD * 2)
          : nullptr;
  auto issue_v16 = [&](int m) __attribute__((always_inline)) {
    const int j = gtile(m);
    const uint32_t dst = ring_lds + (uint32_t)(((2 + (m & 1)) * TILE) * 16);
    const char* base = v16_head + (int64_t)j * (KT * HD * 2);
#pragma unroll
    for (int r = 0; r < NLD; ++r)
      dma16_to_lds_s(base + r * 256 * 16, (uint32_t)(htid * 16), dst + (uint32_t)(r * 256 * 16));
  };
  // K (kv = 0) or V (kv = 1) of local tile m into stage m % 2.
  auto issue_tile = [&](int m, int kv) __attribute__((always_inline)) {
    if (V16 && kv) {
      issue_v16(m);
      return;
    }
    const int j = gtile(m);
    const int32_t* ids = &idring[half][m % 3][wave][0];
    const int b0 = blk_of(j * KT);
    const char* src = reinterpret_cast<const char*>(kv ? a.v : a.k);
    const uint32_t dst = ring_lds + (uint32_t)(((kv * 2 + (m & 1)) * TILE) * 16);
    if constexpr (POW2) {
      if (fast && (j + 1) * KT <= n) {
        int id[NLD];
        if (CH == 16 && NLD == 4 && a.bs_shift == 4) {
          // 16-token blocks at head_dim 128: DMA r covers keys 16 r + 4 wave .. + 3, all
          // in block r of the tile, so the four ids are the table's entries b0 .. b0 + 3:
          // one 16-byte scalar load (inside the table: the tile is inside the context).
          const i32x4_a4 v4 = sid4(b0);
#pragma unroll
          for (int r = 0; r < NLD; ++r) id[r] = v4[r & 3];
        } else {
#pragma unroll
          for (int r = 0; r < NLD; ++r)  // every id read before the first DMA
            id[r] = sid((j * KT + (r * 256 + wave * kWave) / CH) >> a.bs_shift);
        }
        const char* base = kv_base[kv] + (uint32_t)(((j * KT) & (a.bs - 1)) * a.kv_ss * (int)sizeof(S));
#pragma unroll
        for (int r = 0; r < NLD; ++r) {
          uint32_t bid = (uint32_t)__builtin_amdgcn_readfirstlane(id[r]);
          bid = bid < pool_blocks ? bid : 0u;  // memory safety only
          dma16_to_lds_s(base + (uint64_t)bid * blk_bytes32, lane_off[r],
                         dst + (uint32_t)(r * 256 * 16));
        }
        return;
      }
      if (seg_uniform) {  // the context's last tile: positions past it re-read its last token
        int id[NLD];
#pragma unroll
        for (int r = 0; r < NLD; ++r) {  // every id read before the first DMA
          const int seg = j * KT + (r * 256 + wave * kWave) / CH;  // first key, uniform
          id[r] = sid(min(seg >> a.bs_shift, blast));
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
          dma16_to_lds(src + base + lo, dst + (uint32_t)(r * 256 * 16));
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
      dma16_to_lds(src + off, dst + (uint32_t)(r * 256 * 16));
    }
  };

  float m_run[RT];
  float nref[RT];  // the exponent's offset: kPLog2 - m_run, or 0 while m_run is -inf
  // O^T tiles d < DTL; tile DTL is the softmax normaliser: the matrix cores multiply each
  // P^T fragment by an all-ones V^T fragment too, so every lane of row n's column holds
  // row n's sum of the same (hi + lo) weights O carries -- no VALU adds, no cross-lane sum.
  f32x4 o[RT][DTL + 1];
  const u32x4 ones = {PM::kOnePair, PM::kOnePair, PM::kOnePair, PM::kOnePair};
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    m_run[t] = -INFINITY;
    nref[t] = 0.f;
#pragma unroll
    for (int d = 0; d <= DTL; ++d) o[t][d] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // V16: O^T (d < DTL, not the row sums) from scale 2^-kcur to 2^-k (a power of two,
  // exact); uniform, and a no-op unless a tile of the copy was scaled down.
  auto v16_rescale = [&](int k) __attribute__((always_inline)) {
    if (k == kcur) return;
    const float f = __builtin_amdgcn_ldexpf(1.f, kcur - k);
#pragma unroll
    for (int t = 0; t < RT; ++t)
#pragma unroll
      for (int d = 0; d < DTL; ++d) o[t][d] *= f;
    kcur = k;
  };
  // Before the P.V of local tile m: its region tile's exponent.
  auto v16_tile_scale = [&](int m) __attribute__((always_inline)) {
    const int ri = gtile(m) * KT / kV16Rows;
    v16_rescale((int)((__builtin_amdgcn_readlane(kwin, ri >> 2) >> (8 * (ri & 3))) & 0xFFu));
  };

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
  //   V^T: see PrefillShape::voff (pool rows), or one 16-byte read (the fp16 copy).
  constexpr int KSW = CH > 16 ? NBETA : 1;
  auto fresh_lane = [&]() {  // lane, as a value the compiler must not hoist
    int l = lane;
    __asm__ volatile("" : "+v"(l));
    return l;
  };
  auto koff = [&](int l, int b, int s) {
    const int tk = 16 * b + (l & 15);
    return (uint32_t)(((4 * s + (l >> 4)) ^ SH::swz(tk)) * 16 + (l & 15) * CH * 16);
  };
  // V^T operand fragment (32-key step sg, 16-dim tile d) of the V tile at vstage. The
  // fp16 copy stores every tile in operand order (fragment (sg, d) is 1 KiB, lane l's 16
  // bytes at l * 16), so a fragment is one conflict-free ds_read_b128; V from the pool
  // takes two transpose reads of the swizzled rows (a timing copy that read V^T with one
  // 16-byte read per fragment ran 1.5 µs faster per config-5 call).
  auto vt_frag = [&](const char* vstage, int l, int sg, int d) __attribute__((always_inline)) {
    if constexpr (V16) return *reinterpret_cast<const u32x4*>(vstage + ((sg * DTL + d) * kWave + l) * 16);
    else return vt_frag_tr<HD>(vstage, l, sg, d);
  };

  // S^T of a tile from its QK^T to its softmax, then in the same registers its
  // probabilities P^T until its P.V (the first 32-key step's already packed as operand
  // fragments: hi in block 0, lo in block 1).
  static_assert(NBETA == 2 * NSG, "two score blocks per P^T fragment pair");
  // 32-key steps whose P^T fragments the softmax packs (the rest: the matrix phase)
  constexpr int kPackedSteps = PKV_PREFILL_PACK_ALL ? NSG : 1;
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
    if constexpr (V16) v16_tile_scale(m);
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
        if (sg < kPackedSteps) {
          phi[t] = __builtin_bit_cast(u32x4, sc[t][2 * sg]);
          plo[t] = __builtin_bit_cast(u32x4, sc[t][2 * sg + 1]);
        } else {
          float p8[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) p8[e] = sc[t][2 * sg + e / 4][e % 4];
          PM::pack8(p8, phi[t], plo[t]);
        }
      }
#pragma unroll
      for (int d = 0; d < DTL; ++d) {
        const u32x4 vf = vt_frag(vstage, l, sg, d);
#pragma unroll
        for (int t = 0; t < RT; ++t) {
          o[t][d] = PM::mma(vf, phi[t], o[t][d]);
          if constexpr (PM::kSplit) o[t][d] = PM::mma(vf, plo[t], o[t][d]);
        }
      }
#pragma unroll
      for (int t = 0; t < RT; ++t) {  // the row sums
        o[t][DTL] = PM::mma(ones, phi[t], o[t][DTL]);
        if constexpr (PM::kSplit) o[t][DTL] = PM::mma(ones, plo[t], o[t][DTL]);
      }
    }
  };
  // The steady-state matrix phase: P.V of local tile mp, then QK^T of tile mq, as one
  // software pipeline over their NV + NK operand fragments: step i issues the LDS reads of
  // fragment i + PIPE, then the MFMAs of fragment i, and a scheduling fence closes each
  // step. Left to itself the compiler moves every read down to just before its own MFMAs,
  // so each group of MFMAs waits out a whole LDS round trip: a timing kernel of this phase
  // (4 waves of 96 MFMAs on LDS fragments, 256 CUs) took 2,000 cycles that way and 1,520
  // (its MFMA time) with the reads two fragments ahead. Same products, same order of
  // accumulation as pv then qk.
  constexpr int PIPE = PKV_PREFILL_PIPE > 0 ? PKV_PREFILL_PIPE : 1;
  constexpr int NV = NSG * DTL, NK = NBETA * KS;
  auto pv_qk = [&](int mp, int mq) __attribute__((always_inline)) {
    if constexpr (V16) v16_tile_scale(mp);
    const char* vstage = reinterpret_cast<const char*>(&ring[half][1][mp & 1][0]);
    const char* kstage = reinterpret_cast<const char*>(&ring[half][0][mq & 1][0]);
    const int l = fresh_lane();
    u32x4 phi[NSG][RT], plo[NSG][RT];
#pragma unroll
    for (int sg = 0; sg < kPackedSteps; ++sg)
#pragma unroll
      for (int t = 0; t < RT; ++t) {
        phi[sg][t] = __builtin_bit_cast(u32x4, sc[t][2 * sg]);
        plo[sg][t] = __builtin_bit_cast(u32x4, sc[t][2 * sg + 1]);
      }
#pragma unroll
    for (int sg = kPackedSteps; sg < NSG; ++sg)
#pragma unroll
      for (int t = 0; t < RT; ++t) {
        float p8[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) p8[e] = sc[t][2 * sg + e / 4][e % 4];
        PM::pack8(p8, phi[sg][t], plo[sg][t]);
      }
    // fragment i: V^T (sg, d) = (iv / DTL, iv % DTL) for a V fragment, K (beta, s) = (ik /
    // KS, ik % KS) for a K one; K fragments first with PKV_PREFILL_QK_FIRST.
    constexpr bool QKF = PKV_PREFILL_QK_FIRST;
    auto is_v = [&](int i) { return QKF ? i >= NK : i < NV; };
    auto vi = [&](int i) { return QKF ? i - NK : i; };
    auto ki = [&](int i) { return QKF ? i : i - NV; };
    auto read_frag = [&](int i) __attribute__((always_inline)) {
      u32x4 f;
      if (is_v(i)) {
        f = vt_frag(vstage, l, vi(i) / DTL, vi(i) % DTL);
      } else {
        const int beta = ki(i) / KS, s = ki(i) % KS;
        f = *reinterpret_cast<const u32x4*>(kstage + beta * 16 * CH * 16 +
                                            koff(l, KSW == 1 ? 0 : beta, s));
      }
      return f;
    };
    auto mma_frag = [&](int i, const u32x4& f) __attribute__((always_inline)) {
      if (is_v(i)) {
        const int sg = vi(i) / DTL, d = vi(i) % DTL;
#pragma unroll
        for (int t = 0; t < RT; ++t) {
          o[t][d] = PM::mma(f, phi[sg][t], o[t][d]);
          if constexpr (PM::kSplit) o[t][d] = PM::mma(f, plo[sg][t], o[t][d]);
        }
        if (d == DTL - 1)
#pragma unroll
          for (int t = 0; t < RT; ++t) {  // the row sums
            o[t][DTL] = PM::mma(ones, phi[sg][t], o[t][DTL]);
            if constexpr (PM::kSplit) o[t][DTL] = PM::mma(ones, plo[sg][t], o[t][DTL]);
          }
      } else {
        const int beta = ki(i) / KS, s = ki(i) % KS;
#pragma unroll
        for (int t = 0; t < RT; ++t)
          sc[t][beta] = MMA::mma(f, qf[t][s], s == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : sc[t][beta]);
      }
    };
    u32x4 buf[PIPE + 1];
#pragma unroll
    for (int i = 0; i < PIPE; ++i) buf[i] = read_frag(i);
#pragma unroll
    for (int i = 0; i < NV + NK; ++i) {
      if (i + PIPE < NV + NK) buf[(i + PIPE) % (PIPE + 1)] = read_frag(i + PIPE);
      mma_frag(i, buf[i % (PIPE + 1)]);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // Online softmax of global tile j's scores into P^T fragments; masked: some key of the
  // tile is past some row's causal limit (the tiles on the diagonal and the context end;
  // a wave-uniform branch around the mask only: one copy of the rest, whose registers a
  // second copy would double).
  // The first part of the softmax of tile j: the causal mask and each row's maximum
  // (scaled to log2 units) into mx.
  float mx[RT];
  auto row_max = [&](int j, bool masked) __attribute__((always_inline)) {
    const int kt0 = j * KT;
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
      mx[t] = score_rows_max(x) * a.scale_log2;
    }
  };
  auto softmax = [&](int j, bool masked) __attribute__((always_inline)) {
    // p = exp2(scale_log2 * s - m_run + kPLog2) (kPLog2 of the P.V type). The reference
    // m_run is raised only when a score exceeds it by more than 2^8: a stale reference
    // changes nothing in O / l (both carry the same factor), keeps p <= 2^(8 + kPLog2),
    // and leaves O untouched on most tiles. The row tiles are independent chains: maxima
    // first, one rescale branch, then every exp.
    if (!PKV_PREFILL_EARLY_MAX) row_max(j, masked);
    bool raise[RT];
    bool any = false;
#pragma unroll
    for (int t = 0; t < RT; ++t) {
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
        nref[t] = raise[t] ? PM::kPLog2 - mx[t] : nref[t];  // a raise sets a finite maximum
#pragma unroll
        for (int d = 0; d <= DTL; ++d) o[t][d] *= alpha;
      }
    }
#pragma unroll
    for (int t = 0; t < RT; ++t) {
#pragma unroll
      for (int beta = 0; beta < NBETA; ++beta)
#pragma unroll
        for (int r = 0; r < 4; ++r)  // probabilities replace the scores
          sc[t][beta][r] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[t][beta][r], a.scale_log2, nref[t]));
      // The P^T fragments of the first kPackedSteps 32-key steps are packed here (hi and
      // lo of step sg into score blocks 2 sg and 2 sg + 1); P.V packs the others.
#pragma unroll
      for (int sg = 0; sg < kPackedSteps; ++sg) {
        float p8[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) p8[e] = sc[t][2 * sg + e / 4][e % 4];
        u32x4 hi, lo;
        PM::pack8(p8, hi, lo);
        sc[t][2 * sg] = __builtin_bit_cast(f32x4, hi);
        sc[t][2 * sg + 1] = __builtin_bit_cast(f32x4, lo);
      }
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
  // V from the fp16 copy and both first K tiles inside 16-token blocks: their block ids
  // come in one scalar trip, V0 (no ids) goes out before it returns, and K1 goes out
  // last, so the first matrix phase waits for V0 and K0 only (one trip fewer before it).
  const bool pro2 = PKV_PREFILL_IDS2 && V16 && kBlockWave && POW2 && fast && a.bs_shift == 4 &&
                    nt > 0 && (gtile(1) + 1) * KT <= n;
  if (pro2) {
    const int k0 = wave_id(0), k1 = wave_id(1);
    issue_v16(0);
    issue_block(0, 0, k0);
    issue_block(1, 0, k1);
  } else if (nt > 0) {  // prologue: block ids of tiles 0-2, K of 0 and 1, V of 0
    if (!seg_uniform) {  // the LDS ring's ids must land first; scalar-loaded ids need not
      issue_ids(0);      // wait for the query loads still in flight
      issue_ids(1);
      wait_vmcnt<0>();
    }
    issue_tile(0, 0);
    issue_ids(2);
    issue_tile(0, 1);
    issue_tile(1, 0);
    wait_vmcnt<0>();
  }
  // Matrix phase of iteration m and VALU phase of iteration m, each opened by its
  // barrier. Half 0 runs intervals (M0 V0)(M1 V1)..(M_ns V_ns); half 1 one interval
  // later: idle, (M0 V0)..(M_ns-1 V_ns-1) M_ns. Both pass 2 ns + 2 barriers. The steady
  // state M1 .. M_nt-1 is the pipelined pv_qk in a loop of its own; M0 (QK^T only) and
  // M_nt (P.V only) are peeled off, so that loop holds one matrix-phase variant (two in
  // one loop body cost ~70 more VGPRs and spilled).
  auto open_m = [&](int m) __attribute__((always_inline)) {
    if (m >= 1 && m - 1 < nt) {
      // all but the previous VALU phase's loads: K and V (and the ids, through the LDS)
      if (seg_uniform) wait_vmcnt<2 * NLD>();
      else wait_vmcnt<2 * NLD + 1>();
    } else if (m == 0 && pro2) {
      wait_vmcnt<NLD>();  // all but K1
    } else {
      wait_vmcnt<0>();
    }
    wait_lgkm0();
    __builtin_amdgcn_s_barrier();
  };
  auto interval_v = [&](int m) __attribute__((always_inline)) {
    if (m < nt) wait_vmcnt<2 * NLD>();
    wait_lgkm0();
    __builtin_amdgcn_s_barrier();
    if (m >= nt) return;
#if PKV_PREFILL_VALU_PRIO == 1
    __builtin_amdgcn_s_setprio(1);
#endif
    issue_ids(m + 3);
    // The phase's K/V loads: V of tile m + 1, K of tile m + 2, both used three phases on.
    auto loads = [&]() __attribute__((always_inline)) {
#if PKV_PREFILL_IDS2
      if (kBlockWave && POW2 && fast && a.bs_shift == 4 && (gtile(m + 2) + 1) * KT <= n) {
        if constexpr (V16) {  // V from the copy: no block ids
          const int k2 = wave_id(m + 2);
          issue_v16(m + 1);
          issue_block(m + 2, 0, k2);
        } else {
          const int v1 = wave_id(m + 1), k2 = wave_id(m + 2);
          issue_block(m + 1, 1, v1);
          issue_block(m + 2, 0, k2);
        }
      } else {
        issue_tile(m + 1, 1);
        issue_tile(m + 2, 0);
      }
#else
      issue_tile(m + 1, 1);
      issue_tile(m + 2, 0);
#endif
    };
    // The four waves' loads of a phase are 32 DMA instructions of 1 KiB, ~512 cycles of
    // the CU's address unit (64 bytes a cycle); a wave cannot start its softmax until its
    // own have been taken. The last PKV_PREFILL_LATE_DMA waves of the half issue theirs
    // after the softmax, by when the others' have drained.
    const bool late = wave >= 4 - PKV_PREFILL_LATE_DMA;  // wave-uniform
    if (!late) loads();
    softmax(tbeg + m, tbeg + m >= j_mask);
    if (late) loads();
#if PKV_PREFILL_VALU_PRIO == 1
    __builtin_amdgcn_s_setprio(0);
#endif
  };
  const int v_last = half ? ns - 1 : ns;  // this half's last VALU interval
#if PKV_PREFILL_VALU_PRIO == 2
  if (half) __builtin_amdgcn_s_setprio(1);
#endif
  if (half) {
    wait_lgkm0();
    __builtin_amdgcn_s_barrier();
  }
  open_m(0);
  mfma_phase_begin();
  if (nt > 0) qk(0);
  mfma_phase_end();
  if (PKV_PREFILL_EARLY_MAX && nt > 0) row_max(tbeg, tbeg >= j_mask);
  if (v_last >= 0) interval_v(0);
  for (int m = 1; m < nt; ++m) {
    open_m(m);
    mfma_phase_begin();
    pv_qk(m - 1, m);
    mfma_phase_end();
    if (PKV_PREFILL_EARLY_MAX) row_max(tbeg + m, tbeg + m >= j_mask);
    interval_v(m);
  }
  for (int m = max(nt, 1); m <= ns; ++m) {
    open_m(m);
    if (m == nt) {
      mfma_phase_begin();
      pv(m - 1);
      mfma_phase_end();
    }
    if (m <= v_last) interval_v(m);
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
  if constexpr (V16) v16_rescale(0);  // O^T back to the values' own scale
  __syncthreads();
  if (half) {
#pragma unroll
    for (int t = 0; t < RT; ++t) {
      float* x = xch + t * (2 + 4 * DTL) * kWave;
      x[0] = m_run[t];
      x[kWave] = o[t][DTL][0];
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
    const float l_sum = o[t][DTL][0] * sa + x[kWave] * sb;
    o[t][DTL][0] = l_sum;
#pragma unroll
    for (int d = 0; d < DTL; ++d)
#pragma unroll
      for (int r = 0; r < 4; ++r) o[t][d][r] = o[t][d][r] * sa + x[(2 + 4 * d + r) * kWave] * sb;
  }

  // O^T lane (row col, grp) holds dims 16 d + 4 grp + r of query row col.
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    const float l_tot = o[t][DTL][0];  // the whole row's sum, in every lane of its column
    if (!row_ok[t]) continue;
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    const int rho = rho0 + 16 * RT * wave + 16 * t + col;
    if (a.lse && grp == 0)  // log2 normaliser: the exponent reference m_run plus log2(sum)
      a.lse[(int64_t)(q0 + rho / G) * a.nh + kvh * G + rho % G] =
          l_tot > 0.f ? m_run[t] + (__log2f(l_tot) - PM::kPLog2) : -INFINITY;
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

// One work item (chunk, 128-row block, KV head) on a workgroup of 512 threads. Every
// exit is workgroup-uniform except half 1's after the merge; a caller that runs several
// items on one workgroup puts a barrier between them (the merge reuses the rings).
// V16: V from the fp16 copy (bf16 caches; the launch guarantees every chunk's region).
template <int DT, int HD, bool POW2, bool V16 = false>
__device__ __forceinline__ void prefill_item(const PrefillArgs& a, const int item) {
  __shared__ __align__(16) PrefillLds<HD> lds;
  const int lane = threadIdx.x & (kWave - 1);
  // Work items (chunk, row block, KV head), heaviest first: chunks by context length
  // (longest first), then row blocks from the last (it sees the most keys), KV heads
  // innermost. One workgroup fills a CU, so a grid larger than the GPU runs the items
  // in this order as CUs free up: the longest start earliest.
  PrefillItem it;
  it.kvh = item % a.nkv;
  it.rbi = (item / a.nkv) % a.row_blocks;
  const int crank = item / (a.nkv * a.row_blocks);
  // Each wave ranks up to 63 chunks by itself; larger batches keep their order. Lane j
  // fetches chunk j's length and query offset (and lane n_chunks the end offset) in one
  // round trip, so the chunk's numbers come from the lanes, not a second dependent load.
  const int cap = a.max_blocks * a.bs;
  it.c = crank;
  if (a.n_chunks < kWave) {
    const int mine = lane < a.n_chunks ? min(max(a.ctx[lane], 0), cap) : -1;
    const int cq = lane <= a.n_chunks ? a.cu_q[lane] : 0;
    int rank = 0;
    for (int j = 0; j < a.n_chunks; ++j) {
      const int other = __shfl(mine, j);
      rank += (other > mine) || (other == mine && j < lane);
    }
    const uint64_t hit = __ballot(lane < a.n_chunks && rank == crank);
    it.c = __builtin_ctzll(hit);
    it.q0 = __builtin_amdgcn_readlane(cq, it.c);
    it.q1 = __builtin_amdgcn_readlane(cq, it.c + 1);  // c + 1 <= n_chunks < 64
    it.n = __builtin_amdgcn_readlane(mine, it.c);
  } else {
    it.q0 = a.cu_q[it.c];
    it.q1 = a.cu_q[it.c + 1];
    it.n = min(max(a.ctx[it.c], 0), cap);
  }
  prefill_body<DT, HD, POW2, V16>(a, it, lds);
}

template <int DT, int HD, bool POW2, bool V16>
__global__ void __launch_bounds__(512)
paged_prefill_kernel(const PrefillArgs a) {
  prefill_item<DT, HD, POW2, V16>(a, (int)blockIdx.x);
}

// The fp16 copy of the chunks' V for the bf16 matrix-core prefill (PrefillArgs::v16):
// workgroup h + nkv (i + T c) (T tiles per chunk at the table's width) converts tokens
// i kV16Rows .. i kV16Rows + kV16Rows - 1 of chunk c's KV head h (zeros past the
// context), stores them in operand order through LDS, and writes the tile's scale
// exponent k: the
// largest finite |V| of the tile is below 2^(16 + k), so V * 2^-k lies below 2^16, where
// the largest bf16 value is 65280 and the conversion cannot overflow. bf16 -> fp16 is
// exact for scaled values of fp16's normal range (2^-14 up); smaller ones round to
// fp16's subnormal spacing, 2^-24 (times 2^k). Infinities and NaNs stay what they are.
template <int HD>
__global__ void __launch_bounds__(kV16Threads)
prefill_v16_kernel(const PrefillArgs a) {
  constexpr int NT = kV16Threads, NW = NT / kWave;
  constexpr int GPR = HD / 8;  // 16-byte granules per row
  constexpr int PER = kV16Rows * GPR / NT;
  static_assert(PER >= 1 && kV16Rows * GPR % NT == 0 && kV16Rows == 256 && NT >= kV16Rows,
                "granules split evenly over the threads, one thread per token for the ids");
  using SH = PrefillShape<HD>;
  constexpr int KT = SH::KT, NSG = SH::NSG, DTL = SH::DTL;
  constexpr int TILES = kV16Rows / KT;  // matrix-core prefill tiles per region tile
  constexpr int NFRAG = TILES * NSG * DTL;  // V^T operand fragments per region tile
  static_assert(GPR == SH::CH, "rows of CH granules");
  __shared__ int slots[kV16Rows];
  __shared__ uint32_t wmax[NW];
  // The converted region tile in the prefill's LDS layout for V rows (granule (token t,
  // position p) holds chunk p ^ swz(t)), read back as V^T operand fragments.
  __shared__ __align__(16) u32x4 stage[kV16Rows * GPR];
  // KV head innermost: workgroups are dealt to the XCDs round-robin, so with a multiple
  // of 8 KV heads head h's copy is written from XCD h mod 8, as the prefill's work items
  // of head h run there.
  const int cap = a.max_blocks * a.bs;
  const int tiles = (cap + kV16Rows - 1) / kV16Rows;
  const int h = (int)(blockIdx.x % (unsigned)a.nkv);
  const int rest = (int)(blockIdx.x / (unsigned)a.nkv);
  const int i = rest % tiles, c = rest / tiles;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int tok0 = i * kV16Rows;
  // One memory trip: the chunk's length and the tile's block ids (every token up to the
  // table's width; those past the context are not used).
  const bool id_thread = threadIdx.x < kV16Rows;  // thread t: token tok0 + t's id
  const int t = tok0 + (int)threadIdx.x;
  const int blk = a.bs_shift >= 0 ? (t >> a.bs_shift) : t / a.bs;
  const int bid = id_thread && t < cap ? a.tables[(int64_t)c * a.table_stride + blk] : 0;
  const int n = min(max(a.ctx[c], 0), cap);
  if (tok0 >= v16_pad(n)) return;  // uniform
  if (id_thread) {  // the tile's slots (block ids outside the pool read slot 0)
    int sl = -1;
    if (t < n) {
      const int64_t s64 = (int64_t)bid * a.bs + (t - blk * a.bs);
      sl = (s64 >= 0 && s64 < a.num_slots) ? (int)s64 : 0;  // num_slots < 2^31 (launch)
    }
    slots[threadIdx.x] = sl;
  }
  __syncthreads();
  const char* vsrc = reinterpret_cast<const char*>(a.v) + (int64_t)h * a.kv_sh * 2;
  u32x4 x[PER];
  uint32_t emax = 0;  // largest biased exponent of a finite value
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int g = k * NT + (int)threadIdx.x;
    const int sl = slots[g / GPR];
    x[k] = sl >= 0 ? *reinterpret_cast<const u32x4*>(vsrc + ((int64_t)sl * a.kv_ss + (g % GPR) * 8) * 2)
                   : u32x4{0u, 0u, 0u, 0u};
  }
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const uint32_t w[4] = {x[k].x, x[k].y, x[k].z, x[k].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t e0 = (w[e] >> 7) & 0xFFu, e1 = (w[e] >> 23) & 0xFFu;
      emax = max(emax, max(e0 == 0xFFu ? 0u : e0, e1 == 0xFFu ? 0u : e1));
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) emax = max(emax, (uint32_t)__shfl_xor((int)emax, off));
  if (lane == 0) wmax[wave] = emax;
  __syncthreads();
  emax = wmax[0];
#pragma unroll
  for (int k = 1; k < NW; ++k) emax = max(emax, wmax[k]);
  const int ks = max(0, (int)emax - 127 - 15);  // |V| < 2^(emax - 126)
  const float f = __builtin_amdgcn_ldexpf(1.f, -ks);
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  char* dst = reinterpret_cast<char*>(const_cast<void*>(a.v16)) +
              (((int64_t)c * a.nkv + h) * v16_pad(cap) + tok0) * (HD * 2);
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int g = k * NT + (int)threadIdx.x;
    uint32_t w[4] = {x[k].x, x[k].y, x[k].z, x[k].w};
#pragma unroll
    for (int e = 0; e < 4; ++e)
      w[e] = __builtin_bit_cast(uint32_t, h2{(_Float16)(__uint_as_float(w[e] << 16) * f),
                                             (_Float16)(__uint_as_float(w[e] & 0xFFFF0000u) * f)});
    const int t = g / GPR, ch = g % GPR;  // token of the region tile, 16-byte chunk of its row
    stage[t * GPR + (ch ^ SH::swz(t))] = u32x4{w[0], w[1], w[2], w[3]};
  }
  __syncthreads();
  // The region tile's prefill tiles in operand order: fragment (sg, d) of a tile is 1
  // KiB, lane l's 16 bytes at l * 16 (what the prefill reads with one ds_read_b128);
  // wave w writes fragments w, w + NW, .. of the region tile. Streaming stores: the copy
  // is not kept dirty in this XCD's L2 (no write-back at the kernel's end); the prefill
  // reads it once per XCD, then from its own L2.
#pragma unroll
  for (int fi = wave; fi < NFRAG; fi += NW) {
    const int q = fi / (NSG * DTL), sg = (fi / DTL) % NSG, d = fi % DTL;
    const char* tile = reinterpret_cast<const char*>(&stage[q * KT * GPR]);
    __builtin_nontemporal_store(vt_frag_tr<HD>(tile, lane, sg, d),
                                reinterpret_cast<u32x4*>(dst + (int64_t)fi * (kWave * 16) + lane * 16));
  }
  if (threadIdx.x == 0)
    const_cast<uint8_t*>(a.v16_k)[((int64_t)c * a.nkv + h) * a.v16_kstride + i] = (uint8_t)ks;
}

}  // namespace
