// decode_kernels.h -- split-K (stream-K) paged decode attention and its combine pass
// (gfx950 device code). decode.hip launches them; cascade.hip runs the MFMA stream
// pass beside cascade decode's prefix pass in one launch.

#pragma once

#include "common.h"

namespace pkv {

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
  int32_t num_wg;       // unit ranges (workgroups along x) sharing the unit stream
  // One-launch cascade (kernels instantiated with WT): the stream is cut into `slots`
  // equal slots; ranges 0 .. full_wg - 1 take wslots each, the others tail_slots each.
  // Otherwise num_wg equal ranges (and full_wg = slots = num_wg).
  int32_t full_wg, wslots, tail_slots, slots;
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
  // [rows, nh] (pre_row[b] < 0: none). The stream pass then writes the sequences with
  // parts it finishes to out / lse as fp32 scratch, and the combine pass writes every
  // other sequence's result to fin (fin_f32: fp32, else DT) and its normaliser to
  // fin_lse (if non-null); a whole sequence without parts the stream pass writes there.
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

}  // namespace pkv

namespace {

using namespace pkv;

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


// Table column sequence b starts from (a shared prefix handled elsewhere is skipped).
__device__ __forceinline__ int first_blk(const DecodeArgs& a, int b) {
  if (!a.first_block) return 0;
  const int f = a.first_block[b];
  return f < 0 ? 0 : (f > a.max_blocks ? a.max_blocks : f);
}

// Where the stream pass writes a sequence it finishes whole: the result (out), except
// in cascade for a sequence with prefix parts (pre_b >= 0), whose fp32 state goes to
// scratch (out, lse at that point) for the combine to merge; without parts it is final.
struct WholeDst {
  void* p;
  int64_t sb, sh;
  bool f32;
  float* lse;
};
__device__ __forceinline__ WholeDst whole_dst(const DecodeArgs& a, int pre_b) {
  if (a.pre_row && pre_b < 0) return {a.fin, a.fin_sb, a.fin_sh, a.fin_f32 != 0, a.fin_lse};
  return {a.out, a.out_sb, a.out_sh, a.out_f32 != 0, a.lse};
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

// A sequence's cascade prefix parts for head h, eight at a time. Part k is a normalised
// output O_k (row pre + k * pre_stride of pre_o) with log2 normaliser lse_k, i.e. the
// softmax state (lse_k, 1, O_k); folding it into a wave's running state (m, l, acc)
// (lane holding head dims lane + 64 c, c < DPL) is, with M the new max,
// l <- l 2^(m - M) + sum_k 2^(lse_k - M) and likewise acc. load() issues a chunk's loads
// (lane j < 8 fetches part k0 + j's normaliser, one vector load for the chunk), fold()
// consumes them, so the first chunk can be in flight while the records are merged.
template <int HD, int DPL> struct PrefixParts {
  static constexpr int C = 8;
  float lk;         // lane j: lse of part k0 + (j mod 8), -inf past the last part
  float x[C][DPL];  // the chunk's output rows

  __device__ __forceinline__ static int64_t row(const DecodeArgs& a, int pre, int h, int k) {
    return ((int64_t)pre + (int64_t)(k < a.pre_parts ? k : 0) * a.pre_stride) * a.nh + h;
  }
  __device__ __forceinline__ void load(const DecodeArgs& a, int pre, int h, int k0) {
    const int lane = threadIdx.x & (kWave - 1);
    const int kl = k0 + (lane & (C - 1));
    lk = kl < a.pre_parts ? a.pre_lse[row(a, pre, h, kl)] : -INFINITY;
#pragma unroll
    for (int j = 0; j < C; ++j) {
      const float* p = a.pre_o + row(a, pre, h, k0 + j) * HD;
#pragma unroll
      for (int c = 0; c < DPL; ++c) x[j][c] = lane + kWave * c < HD ? p[lane + kWave * c] : 0.f;
    }
  }
  __device__ __forceinline__ void fold(float& m, float& l, float (&acc)[DPL]) const {
    float lj[C];
#pragma unroll
    for (int j = 0; j < C; ++j) lj[j] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lk), j));
    float mn = m;
#pragma unroll
    for (int j = 0; j < C; ++j) mn = fmaxf(mn, lj[j]);
    const float mref = mn == -INFINITY ? 0.f : mn;  // nothing live yet: weights 0
    const float alpha = __builtin_amdgcn_exp2f(m - mref);
    m = mn;
    l *= alpha;
#pragma unroll
    for (int c = 0; c < DPL; ++c) acc[c] *= alpha;
#pragma unroll
    for (int j = 0; j < C; ++j) {
      const float wj = __builtin_amdgcn_exp2f(lj[j] - mref);  // dead or empty: 0
      l += wj;
#pragma unroll
      for (int c = 0; c < DPL; ++c) acc[c] = __builtin_fmaf(wj, x[j][c], acc[c]);
    }
  }
};

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

// First unit of range w (w = num_wg: the end of the stream). WT: the slots of the
// one-launch cascade; else num_wg equal ranges.
template <bool WT = false>
__device__ __forceinline__ int64_t range_start(const DecodeArgs& a, int64_t w, int64_t units) {
  if constexpr (!WT) return w * units / a.num_wg;
  const int64_t slot = w <= a.full_wg ? w * a.wslots
                                      : (int64_t)a.full_wg * a.wslots + (w - a.full_wg) * a.tail_slots;
  return slot * units / a.slots;
}

// Workgroup w's unit range [*rs, *re) and the sequence b owning unit *rs (first unit
// *ub); returns batch when the range is empty. A batch that fits one wave is scanned
// once (the lengths' prefix sums give both the total and the owner); larger batches
// take two passes of find_unit. Call from whole waves.
__device__ int locate_range(const DecodeArgs& a, int w, int64_t* total, int64_t* rs,
                            int64_t* re, int64_t* ub) {
  if (a.batch <= kWave) {
    const int lane = threadIdx.x & (kWave - 1);
    const int cnt = lane < a.batch ? units_of(a, clamped_ctx(a, lane)) : 0;
    int incl = cnt;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
      const int t = __shfl_up(incl, off);
      if (lane >= off) incl += t;
    }
    *total = __shfl(incl, kWave - 1);
    *rs = range_start(a, w, *total);
    *re = range_start(a, w + 1, *total);
    if (*rs >= *re) return a.batch;
    const unsigned long long hit = __ballot(incl > *rs);
    const int l = __ffsll((long long)hit) - 1;
    *ub = __shfl(incl - cnt, l);
    return l;
  }
  find_unit(a, -1, total);
  *rs = range_start(a, w, *total);
  *re = range_start(a, w + 1, *total);
  if (*rs >= *re) return a.batch;
  return find_unit(a, *rs, ub);
}
// The range holding unit u: the largest w with range_start(w) <= u. The largest slot s
// with s * units / slots <= u is ((u + 1) * slots - 1) / units; w is the range that
// slot belongs to.
template <bool WT = false>
__device__ __forceinline__ int64_t wg_of_unit(const DecodeArgs& a, int64_t u, int64_t units) {
  if constexpr (!WT) return ((u + 1) * a.num_wg - 1) / units;
  const int64_t s = ((u + 1) * a.slots - 1) / units;
  const int64_t full = (int64_t)a.full_wg * a.wslots;
  return s < full ? s / a.wslots : a.full_wg + (s - full) / a.tail_slots;
}

// Merge plan of one sequence, written by the workgroup that holds its first unit (so
// every sequence gets exactly one, every call): the first workgroup w0 of its pieces,
// the number of workgroups w0..w1 it spans (1: written directly), the record slot its
// piece has in w0, and whether every range is non-empty (units >= slots).
template <bool WT = false>
__device__ __forceinline__ void write_desc(const DecodeArgs& a, int b, int w, int64_t ub,
                                           int64_t ue, int64_t rs, int64_t total) {
  if (!a.desc) return;
  const int64_t w1 = wg_of_unit<WT>(a, ue - 1, total);
  const int64_t slots = WT ? a.slots : a.num_wg;
  a.desc[b] = make_int4(w, (int)(w1 - w + 1), rs < ub ? 1 : 0, total >= slots ? 1 : 0);
}

// Batches of kWave + 1 .. kLdsBatch sequences: every sequence's clamped context, first
// table column, cascade prefix row and first unit, staged in LDS by the whole workgroup.
// All lengths arrive in one memory trip (find_unit takes one dependent trip per 64
// sequences, twice), the range's first sequence is a binary search in LDS, and a
// sequence boundary inside a range needs no trip for the next sequence's length.
constexpr int kLdsBatch = 1024;
struct BatchLds {
  int64_t ub[kLdsBatch + 1];  // first unit of each sequence; ub[batch] = total units
  int n[kLdsBatch], fb[kLdsBatch], pre[kLdsBatch];
  int64_t wsum[PKV_DECODE_WAVES_PER_WG];  // per-wave unit sums of the scan
};
// Fill s (whole workgroup; blockDim.x <= 64 * PKV_DECODE_WAVES_PER_WG). Thread t takes a
// contiguous run of sequences, so one wave scan plus the waves' totals give every prefix.
__device__ void stage_batch(const DecodeArgs& a, BatchLds& s) {
  const int tid = threadIdx.x, nt = blockDim.x;
  const int lane = tid & (kWave - 1), wave = tid / kWave;
  const int per = (a.batch + nt - 1) / nt;
  const int b0 = tid * per, b1 = min(a.batch, b0 + per);
  int64_t mine = 0;
  for (int b = b0; b < b1; ++b) {
    const int fb = first_blk(a, b);
    const int n = clamped_ctx(a, b);
    s.n[b] = n;
    s.fb[b] = fb;
    s.pre[b] = a.pre_row ? a.pre_row[b] : -1;
    mine += units_of(a, n);
  }
  int64_t incl = mine;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int64_t t = __shfl_up(incl, off);
    if (lane >= off) incl += t;
  }
  if (lane == kWave - 1) s.wsum[wave] = incl;
  __syncthreads();
  int64_t before = incl - mine;
  for (int w = 0; w < wave; ++w) before += s.wsum[w];
  for (int b = b0; b < b1; ++b) {
    s.ub[b] = before;
    before += units_of(a, s.n[b]);
  }
  if (tid == nt - 1) s.ub[a.batch] = before;  // the last thread's run ends the batch
  __syncthreads();
}
// The sequence owning unit u < total: the last b with ub[b] <= u (every sequence owns at
// least one unit, so ub is strictly increasing).
__device__ __forceinline__ int staged_owner(const DecodeArgs& a, const BatchLds& s, int64_t u) {
  int lo = 0, hi = a.batch - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (s.ub[mid] <= u) lo = mid;
    else hi = mid - 1;
  }
  return lo;
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

  int64_t total, rs, re, ub;
  int b = locate_range(a, w, &total, &rs, &re, &ub);
  if (rs >= re) return;

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
    const int pre_b = a.pre_row ? a.pre_row[b] : -1;  // cascade: b's prefix row, or none
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
        const WholeDst dst = whole_dst(a, pre_b);
#pragma unroll
        for (int g = 0; g < GPW; ++g) {
          // no live token (empty context): 0, the reference oracle's einsum over no keys
          const float inv = l[g] > 0.f ? 1.f / l[g] : 0.f;
          float o[VEC];
#pragma unroll
          for (int c = 0; c < VEC; ++c) o[c] = acc[g][c] * inv;
          const int64_t e = b * dst.sb + (int64_t)(h0 + g) * dst.sh + d0;
          if (dst.f32) store_vec<PKV_F32, VEC>((float*)dst.p + e, o);
          else store_vec<DT, VEC>((S*)dst.p + e, o);
          if (dst.lse && lane == 0) dst.lse[(int64_t)b * a.nh + h0 + g] = lse_of(m[g], l[g]);
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
// MFMA variant of the stream pass for 16-bit K/V at head_dim 128 (the Llama-3 shapes)
// and 64 (Llama-3.2-1B).
//
// Same stream-K ranges, records and outputs as paged_decode_stream_kernel; only the
// per-tile arithmetic differs. A tile is 16 tokens. Lane l is (col = l % 16, grp =
// l / 16). (hd 64 takes two tiles per step: two k-blocks per score block, and the V
// rows of the second tile on lane columns 8 .. 15; see the kernel.)
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



template <int DT> struct Mfma16x16x32;
template <> struct Mfma16x16x32<PKV_BF16> {
  static constexpr bool kSplit = true;  // P.V on the matrix cores: P as hi + lo (pack_p8)
  typedef __bf16 v8 __attribute__((ext_vector_type(8)));
  __device__ static f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8, a),
                                                   __builtin_bit_cast(v8, b), c, 0, 0, 0);
  }
};
template <> struct Mfma16x16x32<PKV_F16> {
  static constexpr bool kSplit = true;  // P.V on the matrix cores: P as hi + lo (pack_p8 LO16)
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


// ---------------------------------------------------------------------------------
// Per-sequence split pass for small batches (one launch, no combine, no workspace):
// paged_decode_mfma_kernel with SPLIT. Workgroup (b, task) takes sequence b for one KV
// head's query heads h0 .. h0 + GPW - 1; its kSplitWaves waves take equal 16-token-
// aligned shares of the context (each the same matrix-core piece as a stream-K wave)
// and merge their softmax states through LDS: with M = max_s m_s,
// out = sum_s 2^(m_s - M) acc_s / sum_s 2^(m_s - M) l_s. Chosen by the host only from
// static shapes (batch, KV heads, table width), so a graph captured with it serves every
// context length: when the (sequence, task) pairs fit the CUs and the table's width
// bounds every wave's share to kSplitMaxTiles tiles. The step is then a few dependent
// memory trips long instead of two launches.
// ---------------------------------------------------------------------------------

constexpr int kSplitWaves = 8;
constexpr int kSplitMaxTiles = 16;      // per wave, from the table width (static)
constexpr int kSplitMaxColumns = 2048;  // table columns staged in LDS

// The split pass's merge: every wave's state (lanes grp == 0, col < HD / 8 hold acc[g]
// for head dims 8 col .. 8 col + 7; lh, mh are the same in every lane) goes to LDS, then
// wave g < GPW merges query head h0 + g and stores it. All waves call it.
template <int DT, int GPW, int HD>
__device__ __forceinline__ void split_merge(const DecodeArgs& a, int b, int h0,
                                            const float (&acc)[GPW][8], const float (&lh)[GPW],
                                            const float (&mh)[GPW]) {
  constexpr int W = kSplitWaves, VC = HD / 8;
  constexpr int DPL = HD / kWave;  // head dims per lane in the merge (2 or 1)
  using S = typename Elt<DT>::S;
  __shared__ __attribute__((aligned(16))) float part_acc[W][GPW][HD];
  __shared__ float part_ml[W][GPW][2];
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int col = lane & 15, grp = lane >> 4;
  if (grp == 0 && col < VC) {
#pragma unroll
    for (int g = 0; g < GPW; ++g) {
      float4* dst = reinterpret_cast<float4*>(&part_acc[wave][g][8 * col]);
      dst[0] = make_float4(acc[g][0], acc[g][1], acc[g][2], acc[g][3]);
      dst[1] = make_float4(acc[g][4], acc[g][5], acc[g][6], acc[g][7]);
      if (col == 0) {
        part_ml[wave][g][0] = mh[g];
        part_ml[wave][g][1] = lh[g];
      }
    }
  }
  __syncthreads();
  if (wave >= GPW) return;
  const int g = wave;
  float mmax = -INFINITY;
#pragma unroll
  for (int s = 0; s < W; ++s) mmax = fmaxf(mmax, part_ml[s][g][0]);
  const float mref = mmax == -INFINITY ? 0.f : mmax;  // nothing live: weights 0
  float l = 0.f, o[DPL];
#pragma unroll
  for (int k = 0; k < DPL; ++k) o[k] = 0.f;
#pragma unroll
  for (int s = 0; s < W; ++s) {
    const float wgt = __builtin_amdgcn_exp2f(part_ml[s][g][0] - mref);  // empty share: 0
    l = __builtin_fmaf(wgt, part_ml[s][g][1], l);
#pragma unroll
    for (int k = 0; k < DPL; ++k) o[k] = __builtin_fmaf(wgt, part_acc[s][g][DPL * lane + k], o[k]);
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;  // empty context: 0
  const int64_t e = b * a.out_sb + (int64_t)(h0 + g) * a.out_sh + DPL * lane;
#pragma unroll
  for (int k = 0; k < DPL; ++k) {
    const float v = o[k] * inv;
    if (a.out_f32) reinterpret_cast<float*>(a.out)[e + k] = v;
    else reinterpret_cast<S*>(a.out)[e + k] = Elt<DT>::from_f32(v);
  }
}

// The MFMA stream pass of workgroup (bx, by): bx indexes the unit ranges (or, SPLIT, the
// sequence), by the task group.
template <int DT, int GPW, bool FAST, int HD, bool SPLIT, bool STAGED = false, bool WT = false>
__device__ __forceinline__ void decode_mfma_body(const DecodeArgs& a, const int bx, const int by) {
  static_assert(!WT || STAGED, "the one-launch cascade's split takes the staged pass");
  // hd 128: a step is one 16-token tile, four 32-dim MFMA k-blocks, V rows over all 16
  // lane columns (8 dims each). hd 64: a step is two 16-token sub-tiles (the same 8 KB
  // per wave in flight as at hd 128), two k-blocks each, the V rows of sub-tile u on
  // lane columns 8u .. 8u + 7, the two halves of the accumulator added at the end.
  static_assert(HD == 64 || HD == 128, "MFMA decode: hd 64 or 128");
  constexpr int TILE = 16, KB = HD / 32, VC = HD / 8, NS = 128 / HD, STEP = NS * TILE;
  constexpr bool kDeep = PKV_DECODE_PREFETCH >= 2;
  static_assert(GPW >= 1 && GPW <= 4, "at most 4 query heads per wave");
  using S = typename Elt<DT>::S;
  using MMA = Mfma16x16x32<DT>;
  // hd 64: P.V on the matrix cores (PKV_DECODE_PV_MFMA; 5.6% faster than the VALU form,
  // a row broadcast and 8 FMAs per query head and V row, at config 2's batch and
  // contexts; at hd 128, a timing copy without any P.V ran only 1% faster, so it keeps
  // the VALU form). Each wave stages its step's V rows (32 tokens x 64 dims, 4 KiB)
  // in its own LDS slot, reads them back as V^T operand fragments with transpose reads,
  // and multiplies them by P^T: the lane's own probabilities, in the order the transpose
  // delivers the tokens, as a hi + lo pair in either 16-bit type (fp32-like P, as the
  // VALU form had: every work split then agrees to fp32 rounding). O^T lane (head col,
  // grp) holds dims 16 d + 4 grp + r.
  // (The stream-K pass only: the split pass's few short steps per wave are latency-bound,
  // and the LDS round trip cost config 1 0.2 us.)
  constexpr bool PVM = HD == 64 && !SPLIT && PKV_DECODE_PV_MFMA;
  __shared__ __align__(16) u32x4 v_lds[PVM ? PKV_DECODE_WAVES_PER_WG * 256 : 1];
  char* const vslot = reinterpret_cast<char*>(&v_lds[PVM ? (threadIdx.x / kWave) * 256 : 0]);

  const int lane = threadIdx.x & (kWave - 1);
  // Stream-K: wave = task (KV head and head sub-group), workgroup x = unit range.
  // SPLIT: workgroup = (sequence bx, task by), wave = share of it.
  const int task = SPLIT ? (int)by
                         : (int)(by * (blockDim.x / kWave) + (threadIdx.x / kWave));
  const int kvh = task / a.nsub;
  if (!SPLIT && !STAGED && kvh >= a.nkv) return;
  const int h0 = kvh * a.groups + (task - kvh * a.nsub) * GPW;
  // Unit range of this workgroup, XCD-blocked when the grid is a multiple of 8:
  // workgroups are dealt to the 8 XCDs round-robin, so workgroup bx (XCD bx % 8) takes
  // range (bx % 8) G / 8 + bx / 8, and each XCD streams one contiguous eighth of the
  // units (a sequence's pieces mostly on one XCD): 0.4-0.8% faster at configs 2 and 4
  // and the hd-64 shape than ranges dealt round-robin over the XCDs.
  const int w = (!SPLIT && !WT && (gridDim.x & 7) == 0)
                    ? (int)((bx & 7) * (gridDim.x >> 3) + (bx >> 3)) : bx;

  int64_t total, rs, re, ub;
  int b;
  // SPLIT: the sequence's block table row is staged in LDS by the whole workgroup, in
  // the same memory trip as each wave's context length (the split's tables hold at most
  // kSplitMaxColumns entries), so no wave waits for its length before its block ids.
  __shared__ int split_table[SPLIT ? kSplitMaxColumns : 1];
  // STAGED (stream-K over kWave + 1 .. kLdsBatch sequences): the batch's metadata in LDS.
  // Smaller batches keep their lengths in lanes; larger ones walk them with find_unit.
  static_assert(!(SPLIT && STAGED), "the split pass takes one sequence per workgroup");
  __shared__ BatchLds batch_lds[1];  // unused (and dropped) unless STAGED
  constexpr bool staged = STAGED;
  int split_n = 0;
  if constexpr (SPLIT) {
    total = rs = ub = 0;
    re = 1;
    b = bx;
    split_n = clamped_ctx(a, b);
    for (int j = threadIdx.x; j < a.max_blocks; j += blockDim.x)
      split_table[j] = a.tables[(int64_t)b * a.table_stride + j];
    __syncthreads();
  } else if constexpr (STAGED) {  // every wave of the workgroup stages, then idle ones leave
    stage_batch(a, batch_lds[0]);
    total = batch_lds[0].ub[a.batch];
    rs = range_start<WT>(a, w, total);
    re = range_start<WT>(a, w + 1, total);
    b = rs < re ? staged_owner(a, batch_lds[0], rs) : a.batch;
    ub = rs < re ? batch_lds[0].ub[b] : 0;
  } else {
    b = locate_range(a, w, &total, &rs, &re, &ub);
  }
  if (STAGED && kvh >= a.nkv) return;
  if (rs >= re) return;

  const int col = lane & 15, grp = lane >> 4;
  // FAST: block_size is a multiple of 16, so a tile never crosses a block.
  const S* kbase = reinterpret_cast<const S*>(a.k) + (int64_t)kvh * a.kv_sh;
  const S* vbase = reinterpret_cast<const S*>(a.v) + (int64_t)kvh * a.kv_sh;
  // Fixed per-lane element offsets from a tile's first slot (fast path).
  const int64_t k_off = col * a.kv_ss + 8 * grp;
  int64_t v_off[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) v_off[r] = (4 * grp + r) * a.kv_ss + 8 * (HD == 64 ? (col & 7) : col);

  for (int64_t u = rs; u < re && b < a.batch; ++b) {
    int n;
    if constexpr (SPLIT) n = split_n;
    else n = staged ? batch_lds[0].n[b] : clamped_ctx(a, b);
    int t0, t1, slot = 0;
    bool whole = true;
    if constexpr (SPLIT) {  // this wave's 16-token-aligned share of the context
      constexpr int W = kSplitWaves;
      // Wave-uniform (readfirstlane): the full / partial / empty tile branches below are
      // then scalar branches, and the compiler does not wait for one step's loads before
      // issuing the next step's.
      const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
      const int nu = __builtin_amdgcn_readfirstlane(n);
      const int units = (nu + TILE - 1) / TILE;
      t0 = (wave * units / W) * TILE;
      t1 = min(nu, ((wave + 1) * units / W) * TILE);
      u = re;
    } else {
      const int64_t ue = ub + units_of(a, n);
      const int64_t seg_end = ue < re ? ue : re;
      whole = (u == ub) && (seg_end == ue);
      slot = (u == rs) ? 0 : 1;
      t0 = (int)(u - ub) * TILE;
      t1 = min(n, (int)(seg_end - ub) * TILE);
      // Wave-uniform (readfirstlane): the full / partial / empty tile branches of the
      // loads are then scalar branches, so the compiler does not wait for one tile's
      // loads before issuing the next tile's.
      t0 = __builtin_amdgcn_readfirstlane(t0);
      t1 = __builtin_amdgcn_readfirstlane(t1);
      if (u == ub && task == 0 && lane == 0) write_desc<WT>(a, b, w, ub, ue, rs, total);
      u = seg_end;
      ub = ue;
    }

    // Q^T as the B operand: column col = query head h0 + col.
    u32x4 qb[4];
    {
      const S* qp = reinterpret_cast<const S*>(a.q) + b * a.q_sb + (int64_t)(h0 + col) * a.q_sh + 8 * grp;
#pragma unroll
      for (int m = 0; m < KB; ++m)
        qb[m] = col < GPW ? *reinterpret_cast<const u32x4*>(qp + 32 * m) : u32x4{0, 0, 0, 0};
    }

    int cb = 0, tbl = 0;
    const int fb = staged ? batch_lds[0].fb[b] : first_blk(a, b);
    // cascade: b's prefix row, or none
    const int pre_b = staged ? batch_lds[0].pre[b] : (a.pre_row ? a.pre_row[b] : -1);
    auto load_table = [&](int first_block) {
      cb = first_block;
      const int j = cb + lane;
      if constexpr (SPLIT)  // first_block is null on the split path: fb == 0
        tbl = j < a.max_blocks ? split_table[j] : 0;
      else
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
          for (int m = 0; m < KB; ++m) kr[m] = load_kv16v(kt + k_off + 32 * m);
#pragma unroll
          for (int r = 0; r < 4; ++r) vr[r] = col < VC ? load_kv16v(vt + v_off[r]) : z;
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
        for (int m = 0; m < KB; ++m)
          kr[m] = load_kv16v(kt + kt_tok * a.kv_ss + 8 * grp + 32 * m);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int tok = 4 * grp + r;
          vr[r] = col < VC ? load_kv16v(vt + min(tok, live - 1) * a.kv_ss + 8 * col) : z;
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
        for (int m = 0; m < KB; ++m)
          kr[m] = kon ? load_kv16v(kbase + kslot * a.kv_ss + 8 * grp + 32 * m) : z;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int src = 4 * grp + r;
          const int lo = __shfl((int)(kslot & 0xFFFFFFFF), src);
          const int hi = __shfl((int)(kslot >> 32), src);
          const int64_t vs = ((int64_t)hi << 32) | (uint32_t)lo;
          const bool on = vs >= 0;
          vr[r] = on && col < VC ? load_kv16v(vbase + vs * a.kv_ss + 8 * col) : z;
          ok |= (unsigned)on << r;
        }
      }
      return ok;
    };

    // hd 64: both 16-token sub-tiles of a step. Sub-tile u's K goes to kr[KB u ..]; the
    // V rows on lane columns 8u .. 8u + 7 come from sub-tile u, one load per row for all
    // lanes (lanes 0-7 address sub-tile 0's slots, lanes 8-15 sub-tile 1's), so no
    // register is written by two loads. Bits 4u .. 4u + 3 of the result: token 4*grp + r
    // of sub-tile u is live.
    const bool vlane0 = col < 8;  // hd 64: this lane's V rows come from sub-tile 0
    const int vd = 8 * (col & 7);
    auto load_pair = [&](int tb, u32x4* kr, u32x4* vr) -> unsigned {
      const u32x4 z = {0, 0, 0, 0};
      if (tb >= t1) {
#pragma unroll
        for (int i = 0; i < 2 * KB; ++i) kr[i] = z;
#pragma unroll
        for (int r = 0; r < 4; ++r) vr[r] = z;
        return 0;
      }
      if (block_of(min(tb + STEP, t1) - 1) - cb >= kWave) load_table(block_of(tb));
      unsigned ok = 0;
      if constexpr (FAST) {
        // One load form for full and partial sub-tiles (token index clamped to the last
        // live one), so the only branches are on the wave-uniform live counts.
        int live[2];
        const S* vt[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int tu = tb + TILE * u;
          const int blk = block_of(tu);
          const int bid = __builtin_amdgcn_readlane(tbl, blk - cb);
          const int64_t slot0 = (int64_t)bid * a.bs + (tu - blk * a.bs);
          live[u] = (tu < t1 && bid >= 0 && slot0 + TILE <= a.num_slots) ? min(TILE, t1 - tu) : 0;
          // a dead sub-tile's lanes read pool row 0 (in bounds when any tile is live) and
          // are masked out
          vt[u] = vbase + (live[u] ? slot0 : 0) * a.kv_ss;
          if (live[u] > 0) {
            const S* kt = kbase + slot0 * a.kv_ss + min(col, live[u] - 1) * a.kv_ss + 8 * grp;
#pragma unroll
            for (int m = 0; m < KB; ++m) kr[KB * u + m] = load_kv16v(kt + 32 * m);
#pragma unroll
            for (int r = 0; r < 4; ++r) ok |= (unsigned)(4 * grp + r < live[u]) << (4 * u + r);
          } else {
#pragma unroll
            for (int m = 0; m < KB; ++m) kr[KB * u + m] = z;
          }
        }
        if (live[0] + live[1] > 0) {
          const S* vl = vlane0 ? vt[0] : vt[1];
          const int lv = max(vlane0 ? live[0] : live[1], 1);
#pragma unroll
          for (int r = 0; r < 4; ++r) vr[r] = load_kv16v(vl + min(4 * grp + r, lv - 1) * a.kv_ss + vd);
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r) vr[r] = z;
        }
      } else {
        int64_t kslot[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int p = tb + TILE * u + col;
          const int blk = block_of(p);
          const int bid = __shfl(tbl, blk - cb);
          const int64_t sl = (int64_t)bid * a.bs + (p - blk * a.bs);
          const bool kon = p < t1 && sl >= 0 && sl < a.num_slots;
          kslot[u] = kon ? sl : -1;
#pragma unroll
          for (int m = 0; m < KB; ++m)
            kr[KB * u + m] = kon ? load_kv16v(kbase + kslot[u] * a.kv_ss + 8 * grp + 32 * m) : z;
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int src = 4 * grp + r;  // the K lane holding this row's token
          int64_t vs[2];
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const int lo = __shfl((int)(kslot[u] & 0xFFFFFFFF), src);
            const int hi = __shfl((int)(kslot[u] >> 32), src);
            vs[u] = ((int64_t)hi << 32) | (uint32_t)lo;
            ok |= (unsigned)(vs[u] >= 0) << (4 * u + r);
          }
          const int64_t v = vlane0 ? vs[0] : vs[1];
          vr[r] = v >= 0 ? load_kv16v(vbase + v * a.kv_ss + vd) : z;
        }
      }
      return ok;
    };
    // A step's loads; ok bits 4u .. 4u + 3 mark sub-tile u's live tokens.
    auto load_step = [&](int tb, u32x4* kr, u32x4* vr) -> unsigned {
      if constexpr (NS == 1) return load_tile(tb, kr, vr);
      else return load_pair(tb, kr, vr);
    };

    float m_run = -INFINITY;  // exponent reference of head column col (same in all 4 rows)
    float l_run = 0.f;        // this row's share of the running sum
    float acc[GPW][8];
#pragma unroll
    for (int g = 0; g < GPW; ++g)
#pragma unroll
      for (int d = 0; d < 8; ++d) acc[g][d] = 0.f;
    f32x4 ov[PVM ? 4 : 1];  // PVM: O^T, dims 16 d .. 16 d + 15
#pragma unroll
    for (int d = 0; d < (PVM ? 4 : 1); ++d) ov[d] = f32x4{0.f, 0.f, 0.f, 0.f};

    // The exponent reference of head column col is raised only when a tile's maximum
    // exceeds it by more than 2^8 (or it is still -inf): a stale reference changes
    // nothing in acc / l (both carry the same factor) and keeps p <= 256, and most tiles
    // then skip the rescale of the accumulators. Returns the reference to subtract (0
    // while every score so far was masked).
    auto raise_ref = [&](float mx) __attribute__((always_inline)) {
      const bool raise = mx > m_run + 8.f;  // m_run = -inf: any live score raises
      if (__builtin_amdgcn_ballot_w64(raise)) {  // wave-uniform
        const float mn = raise ? mx : m_run;
        // mn = -inf only where m_run stays -inf (acc, l are 0 there): factor 1
        const float alpha = mn == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m_run - mn);
        m_run = mn;
        l_run *= alpha;
        if constexpr (PVM) {  // O^T column col is head col: its own factor
#pragma unroll
          for (int d = 0; d < 4; ++d) ov[d] *= alpha;
        } else {
#pragma unroll
          for (int g = 0; g < GPW; ++g) {
            const float al = row_bcast(alpha, g);
#pragma unroll
            for (int d = 0; d < 8; ++d) acc[g][d] *= al;
          }
        }
      }
      return m_run == -INFINITY ? 0.f : m_run;
    };
    auto tile = [&](const u32x4* kr, const u32x4* vr, unsigned ok) {
      if constexpr (NS == 1) {
        f32x4 s = {0.f, 0.f, 0.f, 0.f};
  #pragma unroll
        for (int m = 0; m < KB; ++m) s = MMA::mma(kr[m], qb[m], s);
        float p[4];
        float mx = -INFINITY;
  #pragma unroll
        for (int r = 0; r < 4; ++r) {
          p[r] = ((ok >> r) & 1u) ? s[r] * a.scale_log2 : -INFINITY;
          mx = fmaxf(mx, p[r]);
        }
        const float mref = raise_ref(rows_max(mx));
  #pragma unroll
        for (int r = 0; r < 4; ++r) p[r] = __builtin_amdgcn_exp2f(p[r] - mref);
        l_run += (p[0] + p[1]) + (p[2] + p[3]);
        float vf[4][8];
  #pragma unroll
        for (int r = 0; r < 4; ++r) unpack16v<DT>(vr[r], vf[r]);
  #pragma unroll
        for (int g = 0; g < GPW; ++g) {
  #pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float pr = row_bcast(p[r], g);
  #pragma unroll
            for (int d = 0; d < 8; ++d) acc[g][d] = __builtin_fmaf(pr, vf[r][d], acc[g][d]);
          }
        }
      } else {
        // PVM: the step's V goes through the wave's LDS slot first, so the transpose
        // reads' latency runs under the scores and the softmax. V rows: tokens 16 u +
        // 4 grp + r of the step (u = the lane's sub-tile), 16-byte chunk col % 8 of the
        // row, at byte 128 tk + 16 (c ^ (tk % 8)) (the transpose reads then hit distinct
        // banks). V^T fragment d: lane (dim 16 d + col, grp) gets tokens 4 grp .. + 3 of
        // each sub-tile h2 -- it addresses token 4 grp + col / 4 of sub-tile h2, dims
        // 16 d + 4 (col % 4) .. + 3 (chunk 2 d + (col % 4) / 2, half (col % 4) % 2).
        u32x4 vtf[PVM ? 4 : 1];
        if constexpr (PVM) {
          const int u = vlane0 ? 0 : 1, c = col & 7;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int tk = 16 * u + 4 * grp + r;
            *reinterpret_cast<u32x4*>(vslot + tk * 128 + ((c ^ (tk & 7)) << 4)) = vr[r];
          }
          const int c4 = col & 3, tr = 4 * grp + (col >> 2);
#pragma unroll
          for (int d = 0; d < 4; ++d) {
#pragma unroll
            for (int h2 = 0; h2 < 2; ++h2) {
              const int off = (16 * h2 + tr) * 128 + (((2 * d + (c4 >> 1)) ^ (tr & 7)) << 4) + ((c4 & 1) << 3);
              const s16x4 x = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vslot + off));
              const uint32_t lo = (uint32_t)(uint16_t)x[0] | ((uint32_t)(uint16_t)x[1] << 16);
              const uint32_t hi = (uint32_t)(uint16_t)x[2] | ((uint32_t)(uint16_t)x[3] << 16);
              if (h2 == 0) { vtf[d].x = lo; vtf[d].y = hi; } else { vtf[d].z = lo; vtf[d].w = hi; }
            }
          }
          __builtin_amdgcn_sched_barrier(0);  // the reads stay ahead of the scores
        }
        float p[2][4];
        float mx = -INFINITY;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int m = 0; m < KB; ++m) s = MMA::mma(kr[KB * u + m], qb[m], s);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            p[u][r] = ((ok >> (4 * u + r)) & 1u) ? s[r] * a.scale_log2 : -INFINITY;
            mx = fmaxf(mx, p[u][r]);
          }
        }
        const float mref = raise_ref(rows_max(mx));
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int r = 0; r < 4; ++r) p[u][r] = __builtin_amdgcn_exp2f(p[u][r] - mref);
        l_run += ((p[0][0] + p[0][1]) + (p[0][2] + p[0][3])) +
                 ((p[1][0] + p[1][1]) + (p[1][2] + p[1][3]));
        if constexpr (PVM) {
          // P^T: lane (head col, grp) holds tokens 4 grp + r of sub-tile 0, then of
          // sub-tile 1 -- the order of the two transpose reads of each V^T fragment.
          // fp16: P scaled by 2^7 (exact; P <= 2^8 keeps it below fp16's maximum), so
          // that weights down to ~5e-10 stay above fp16's smallest subnormal instead of
          // flushing to zero; the epilogue scales O back.
          constexpr float kPScale = DT == PKV_F16 ? 128.f : 1.f;
          float p8[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) p8[e] = p[e / 4][e % 4] * kPScale;
          u32x4 phi, plo;
          pack_p8<DT, true>(p8, phi, plo);
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            ov[d] = MMA::mma(vtf[d], phi, ov[d]);
            if constexpr (MMA::kSplit) ov[d] = MMA::mma(vtf[d], plo, ov[d]);
          }
        } else {
        float vf[4][8];
#pragma unroll
        for (int r = 0; r < 4; ++r) unpack16v<DT>(vr[r], vf[r]);
#pragma unroll
        for (int g = 0; g < GPW; ++g) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            // This lane's V rows are sub-tile (col / 8)'s: that sub-tile's weights. Both
            // broadcasts run in every lane before the select: a DPP broadcast on the
            // untaken side would read its source lane (column g < 8) while inactive.
            const float p0 = row_bcast(p[0][r], g), p1 = row_bcast(p[1][r], g);
            const float pr = vlane0 ? p0 : p1;
#pragma unroll
            for (int d = 0; d < 8; ++d) acc[g][d] = __builtin_fmaf(pr, vf[r][d], acc[g][d]);
          }
        }
        }
      }
    };

    if (t0 < t1) {
      load_table(block_of(t0));
      if constexpr (kDeep) {
        // Three tile buffers in rotation: two tiles in flight while one is reduced.
        u32x4 k0[4], v0[4], k1[4], v1[4], k2[4], v2[4];
        unsigned ok0 = load_step(t0, k0, v0);
        unsigned ok1 = load_step(t0 + STEP, k1, v1);
        unsigned ok2;
        for (int tb = t0; tb < t1; tb += 3 * STEP) {
          ok2 = load_step(tb + 2 * STEP, k2, v2);
          tile(k0, v0, ok0);
          if (tb + STEP >= t1) break;
          ok0 = load_step(tb + 3 * STEP, k0, v0);
          tile(k1, v1, ok1);
          if (tb + 2 * STEP >= t1) break;
          ok1 = load_step(tb + 4 * STEP, k1, v1);
          tile(k2, v2, ok2);
        }
      } else {
        // Two tile buffers in ping-pong: the next tile is in flight while one is reduced.
        u32x4 ka[4], va[4], kb2[4], vb2[4];
        unsigned oka = load_step(t0, ka, va);
        for (int tb = t0; tb < t1; tb += 2 * STEP) {
          const unsigned okb = load_step(tb + STEP, kb2, vb2);
          tile(ka, va, oka);
          if (tb + STEP >= t1) break;
          oka = load_step(tb + 2 * STEP, ka, va);
          tile(kb2, vb2, okb);
        }
      }
    }

    // Totals: l over the four rows of each column, acc over the four rows (and, at hd 64,
    // over the two sub-tiles' lane columns c and c + 8, which hold the same dims).
    const float l_tot = rows_sum(l_run);
    if constexpr (PVM) {
      // O^T (already summed over every token) to acc's layout below -- lanes grp 0, col
      // < 8: head g's dims 8 col .. 8 col + 7 -- through the wave's slot, after the last
      // step's reads of it (LDS keeps one wave's accesses in order).
      float* xs = reinterpret_cast<float*>(vslot);  // [GPW][64]
      constexpr float kOScale = DT == PKV_F16 ? 1.f / 128.f : 1.f;  // P's fp16 scale undone
      if (col < GPW) {
#pragma unroll
        for (int d = 0; d < 4; ++d)
          *reinterpret_cast<f32x4*>(xs + col * 64 + 16 * d + 4 * grp) = ov[d] * kOScale;
      }
#pragma unroll
      for (int g = 0; g < GPW; ++g)
#pragma unroll
        for (int d = 0; d < 8; ++d) acc[g][d] = (grp == 0 && col < 8) ? xs[g * 64 + 8 * col + d] : 0.f;
    } else {
#pragma unroll
      for (int g = 0; g < GPW; ++g)
#pragma unroll
        for (int d = 0; d < 8; ++d) {
          acc[g][d] = rows_sum(acc[g][d]);
          if constexpr (NS == 2) acc[g][d] += dpp<kRowRor8>(acc[g][d]);  // lanes c, c ^ 8
        }
    }
    float lh[GPW], mh[GPW];
#pragma unroll
    for (int g = 0; g < GPW; ++g) {
      lh[g] = row_bcast(l_tot, g);
      mh[g] = row_bcast(m_run, g);
    }

    if constexpr (SPLIT) {
      split_merge<DT, GPW, HD>(a, b, h0, acc, lh, mh);
      return;
    }
    if (grp == 0 && col < VC) {  // lane c writes head dims 8c .. 8c + 7
      const int d0 = 8 * col;
      if (whole) {
        const WholeDst dst = whole_dst(a, pre_b);
#pragma unroll
        for (int g = 0; g < GPW; ++g) {
          const float inv = lh[g] > 0.f ? 1.f / lh[g] : 0.f;
          float o[8];
#pragma unroll
          for (int d = 0; d < 8; ++d) o[d] = acc[g][d] * inv;
          const int64_t e = b * dst.sb + (int64_t)(h0 + g) * dst.sh + d0;
          if (dst.f32) store_vec<PKV_F32, 8>((float*)dst.p + e, o);
          else store_vec<DT, 8>((S*)dst.p + e, o);
          if (dst.lse && col == 0) dst.lse[(int64_t)b * a.nh + h0 + g] = lse_of(mh[g], lh[g]);
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

template <int DT, int GPW, bool FAST, int HD, bool SPLIT, bool STAGED = false>
__global__ void __launch_bounds__(512)
paged_decode_mfma_kernel(const DecodeArgs a) {
  decode_mfma_body<DT, GPW, FAST, HD, SPLIT, STAGED>(a, (int)blockIdx.x, (int)blockIdx.y);
}

// ---------------------------------------------------------------------------------
// Combine pass: merges the pieces of sequences cut by a range boundary.
//
// Sequence b (units [ub, ue)) spans workgroups w0..w1; each non-empty range among them
// holds one piece and wrote one record per query head (in w0 it is the range's last
// piece, slot 1, unless the range starts with it). One wave per (sequence, query head)
// merges them: out = sum_j w_j acc_j / sum_j w_j l_j with w_j = exp2(m_j - max m). The
// sequence's merge plan (16 bytes written by the stream pass) says which records to
// read. Then one round trip loads up to 64 records' (m, l) pairs (one per lane), and
// the accumulator rows follow in chunks whose loads overlap: a sequence cut into many
// pieces (a long context) costs about three round trips, not one per few records.
// Cascade prefix parts are folded in after the records. Sequences that were not cut
// exit after reading the plan: the stream pass finished them.
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

// SP = 1: one wave per (sequence, query head). SP = 2 (batches with few such pairs):
// two waves per pair, each folding half of the records, their states merged through
// LDS -- half the dependent round trips for a sequence cut into many pieces.
template <int DT, int HD, int SP, bool WT = false>
__global__ void __launch_bounds__(256)
paged_decode_combine_kernel(const DecodeArgs a) {
  static_assert(SP == 1 || SP == 2, "one or two waves per (sequence, head)");
  constexpr int DPL = HD >= kWave ? HD / kWave : 1;  // head dims per lane
  constexpr int kChunk = WT ? PKV_CASCADE_COMBINE_CHUNK : PKV_DECODE_COMBINE_CHUNK;  // rows per load batch
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int part = SP == 2 ? (wave & 1) : 0;  // which half of the records (SP = 2)
  // Wave-uniform by construction; readfirstlane lets the compiler keep the plan, record
  // indices and row bases in scalar registers.
  const int wid = __builtin_amdgcn_readfirstlane(blockIdx.x * (blockDim.x / kWave / SP) + wave / SP);
  const bool active = wid < a.batch * a.nh;
  if (SP == 1 && !active) return;
  const int pw = active ? wid : 0;  // SP = 2: an idle pair still meets the barrier
  const int b = pw / a.nh, h = pw - b * a.nh;

  const int4 plan = a.desc[b];
  const bool cascade = a.pre_row != nullptr;
  const int pre_b = cascade ? a.pre_row[b] : -1;  // fetched with the plan
  const int pre = part == 0 ? pre_b : -1;
  const int nrec = plan.y;
  // Written directly by the stream pass (or past the batch): nothing to merge -- in
  // cascade, a whole sequence without prefix parts.
  const bool skip = !active || (nrec <= 1 && pre_b < 0);
  if (SP == 1 && skip) return;
  // This wave's records [jb, je): all of them, or one half of them.
  const int jb = part == 0 ? 0 : (nrec + 1) / 2;
  const int je = SP == 1 || part == 1 ? nrec : (nrec + 1) / 2;
  // The first prefix parts' loads go out before the records are merged.
  PrefixParts<HD, DPL> parts;
  if (pre >= 0) parts.load(a, pre, h, 0);
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
    bool live = j < je;
    if (!plan.w && live) {
      const int64_t ww = w0 + j;
      live = range_start<WT>(a, ww, total) < range_start<WT>(a, ww + 1, total);
    }
    live_bits = __ballot(live);
  };
  if (skip) {
  } else if (nrec <= 1) {
    // Cascade, finished by the stream pass: its normalised fp32 output and log2
    // normaliser are the state (lse, 1, O); an empty context (-inf) weighs nothing.
    // (With SP = 2 the first half takes it; the second contributes an empty state.)
    if (part == 0) {
    const float lt = a.lse[(int64_t)b * a.nh + h];
    mmax = lt;
    lsum = lt == -INFINITY ? 0.f : 1.f;
    const float* t = reinterpret_cast<const float*>(a.out) + b * a.out_sb + (int64_t)h * a.out_sh;
#pragma unroll
    for (int k = 0; k < DPL; ++k) out_acc[k] = (lane + kWave * k < HD) ? t[lane + kWave * k] : 0.f;
    }
  } else {
    // Records in blocks of up to 64: lane r of a block loads record j0 + r's (m, l), one
    // wave reduction gives the block's max M, and with every weight 2^(m - M) known up
    // front the accumulator rows stream in chunks of kChunk records, each chunk's loads
    // issued before the previous chunk is consumed (no round trip waits on another).
    for (int j0 = jb; j0 < je; j0 += kWave) {
      live_block(j0);
      const int n = min(kWave, je - j0);
      auto row_of = [&](int r) -> int64_t {  // r < n: record j0 + r, else record 0
        const bool lv = r < n && ((live_bits >> r) & 1);
        return (lv && j0 + r > 0) ? (w0 + j0 + r) * 2 * a.nh + h : row0;
      };
      float xa[kChunk][DPL], xb[kChunk][DPL];
      auto load_rows = [&](float (&x)[kChunk][DPL], int c) {
#pragma unroll
        for (int jj = 0; jj < kChunk; ++jj) {
          const float* rowp = a.ws_acc + row_of(c + jj) * HD;
#pragma unroll
          for (int k = 0; k < DPL; ++k) x[jj][k] = (lane + kWave * k < HD) ? rowp[lane + kWave * k] : 0.f;
        }
      };
      // The first rows go out with the (m, l) pairs: addresses do not need the weights.
      const float2 ml = *reinterpret_cast<const float2*>(a.ws_ml + 2 * row_of(lane));
      load_rows(xa, 0);
      const bool mine = lane < n && ((live_bits >> lane) & 1);
      const float mj = mine ? ml.x : -INFINITY;
      const float mn = fmaxf(mmax, across_max<1>(mj));
      const float mref = mn == -INFINITY ? 0.f : mn;  // no live token yet: weights 0
      const float alpha = __builtin_amdgcn_exp2f(mmax - mref);
      mmax = mn;
      const float wj = __builtin_amdgcn_exp2f(mj - mref);  // dead: exp2(-inf) = 0
      lsum = __builtin_fmaf(lsum, alpha, across_sum<1>(wj * ml.y));
#pragma unroll
      for (int k = 0; k < DPL; ++k) out_acc[k] *= alpha;
      auto consume = [&](const float (&x)[kChunk][DPL], int c) {
#pragma unroll
        for (int jj = 0; jj < kChunk; ++jj) {
          const int r = c + jj;
          const float w = r < n ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wj), r)) : 0.f;
#pragma unroll
          for (int k = 0; k < DPL; ++k) out_acc[k] = __builtin_fmaf(w, x[jj][k], out_acc[k]);
        }
      };
      for (int c = 0; c < n; c += 2 * kChunk) {
        if (c + kChunk < n) load_rows(xb, c + kChunk);
        consume(xa, c);
        if (c + kChunk >= n) break;
        if (c + 2 * kChunk < n) load_rows(xa, c + 2 * kChunk);
        consume(xb, c + kChunk);
      }
    }
  }
  if constexpr (SP == 2) {  // the second half's state joins the first's
    __shared__ float xch[2][2 + DPL * kWave];
    float* x = xch[wave >> 1];
    if (part == 1) {
      if (lane == 0) x[0] = mmax, x[1] = lsum;
#pragma unroll
      for (int k = 0; k < DPL; ++k) x[2 + lane + kWave * k] = out_acc[k];
    }
    __syncthreads();
    if (part == 1 || skip) return;
    const float mb = x[0];
    const float mn = fmaxf(mmax, mb);
    const float mref = mn == -INFINITY ? 0.f : mn;  // both empty: weights 0
    const float sa = __builtin_amdgcn_exp2f(mmax - mref), sb = __builtin_amdgcn_exp2f(mb - mref);
    mmax = mn;
    lsum = lsum * sa + x[1] * sb;
#pragma unroll
    for (int k = 0; k < DPL; ++k) out_acc[k] = out_acc[k] * sa + x[2 + lane + kWave * k] * sb;
  }
  if (pre >= 0) {
    parts.fold(mmax, lsum, out_acc);
    for (int k0 = PrefixParts<HD, DPL>::C; k0 < a.pre_parts; k0 += PrefixParts<HD, DPL>::C) {
      parts.load(a, pre, h, k0);
      parts.fold(mmax, lsum, out_acc);
    }
  }
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
}  // namespace
