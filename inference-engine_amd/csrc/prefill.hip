// prefill.hip -- chunked-prefill attention (include/paged_kv.h: pkv_paged_prefill*): the
// argument checks and launches of the matrix-core kernel (prefill_kernels.h, also
// cascade decode's prefix pass), and the VALU kernel for fp32 K/V and head_dim 16.

#include "cascade.h"
#include "prefill_kernels.h"

namespace {

using namespace pkv;

// ---------------------------------------------------------------------------------
// Chunked-prefill attention on the VALU, for the shapes the matrix-core kernel does not
// take: fp32 K/V (any supported head_dim) and 16-bit K/V at head_dim 16. Same contract
// and arguments as paged_prefill_kernel (causal / non-causal, q_rows, lse).
//
// A workgroup of 4 waves takes 16 consecutive query tokens of one chunk and GPW query
// heads of one KV head; wave w holds tokens 4w .. 4w + 3, so P = 4 * GPW (token, head)
// pairs per wave. Per tile of TK keys the workgroup stages K and V (converted to fp32)
// and a liveness flag per key in LDS once, so every K/V row is read once per 16 query
// tokens rather than once per token. Then, per wave:
//   * scores with lane j = key j (TK = 32 at head_dim 256: lanes j and j + 32 split the
//     head dims), the pairs' pre-scaled queries read from LDS as broadcast float4s;
//   * fp32 online softmax per pair (tile max across lanes; each lane keeps its own share
//     of the running sum), the probabilities of the tile written to LDS;
//   * P.V with lane = head dim, the probabilities read back four keys at a time.
// ---------------------------------------------------------------------------------

template <int HD> struct RowsShape {
  static constexpr int TK = HD >= 256 ? 32 : 64;  // keys per tile
  static constexpr int KS = kWave / TK;            // lane groups splitting head_dim
  static constexpr int DPL = HD >= kWave ? HD / kWave : 1;  // head dims per lane (P.V)
  static constexpr int TOK = 16;                   // query tokens per workgroup
  static constexpr int TPW = 4;                    // query tokens per wave
};

template <int DT, int HD, int GPW>
__global__ void __launch_bounds__(256)
paged_prefill_rows_kernel(const PrefillArgs a) {
  using SH = RowsShape<HD>;
  constexpr int TK = SH::TK, KS = SH::KS, DPL = SH::DPL, TOK = SH::TOK, TPW = SH::TPW;
  constexpr int P = TPW * GPW;
  constexpr int VEC = vec16<DT>();
  constexpr int CPR = HD / VEC;  // 16-byte chunks per K/V row
  using S = typename Elt<DT>::S;
  __shared__ float ks[TK][HD + 1];  // padded: lane j reads row j conflict-free
  __shared__ float vs[TK][HD];
  __shared__ int live[TK];
  __shared__ __attribute__((aligned(16))) float qs[4][P][HD];
  __shared__ __attribute__((aligned(16))) float es[4][P][TK];

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int tiles = (int)gridDim.x / a.n_chunks;  // query tiles per chunk (static bound)
  const int c = blockIdx.x / tiles;
  const int tt = blockIdx.x - c * tiles;
  const int nsub = (a.groups + GPW - 1) / GPW;
  const int kvh = blockIdx.y / nsub;
  const int h0 = kvh * a.groups + (blockIdx.y - kvh * nsub) * GPW;
  const int hend = (kvh + 1) * a.groups;  // heads of this KV head end here

  const int q0 = a.cu_q[c], ql = a.cu_q[c + 1] - q0;
  if (tt * TOK >= ql) return;  // workgroup-uniform
  int n = a.ctx[c];
  const int cap = a.max_blocks * a.bs;
  n = n < 0 ? 0 : (n > cap ? cap : n);
  const int last_tok = min(ql, (tt + 1) * TOK) - 1;  // last valid token of the tile
  // Keys the tile's queries may see: 0 .. kmax - 1.
  const int kmax = a.causal ? max(0, min(n, n - ql + last_tok + 1)) : n;

  // This wave's pairs: pair p = (token i = p / GPW, head h0 + p % GPW).
  const int tok0 = tt * TOK + TPW * wave;
  for (int e = lane; e < P * HD; e += kWave) {
    const int p = e / HD, d = e - p * HD;
    const int i = tok0 + p / GPW, h = h0 + p % GPW;
    float x = 0.f;
    const int row = i < ql ? (a.q_rows ? a.q_rows[q0 + i] : q0 + i) : -1;
    if (row >= 0 && h < hend)  // a negative q_rows entry: no query there
      x = Elt<DT>::to_f32(reinterpret_cast<const S*>(a.q)[(int64_t)row * a.q_st +
                                                        (int64_t)h * a.q_sh + d]);
    qs[wave][p][d] = x * a.scale_log2;
  }
  int qpos[TPW];  // position of each token of the wave (keys <= qpos are visible)
#pragma unroll
  for (int i = 0; i < TPW; ++i) qpos[i] = a.causal ? n - ql + tok0 + i : n - 1;

  float m[P], l[P], acc[P][DPL];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    m[p] = -INFINITY;
    l[p] = 0.f;
#pragma unroll
    for (int k = 0; k < DPL; ++k) acc[p][k] = 0.f;
  }
  const int j = lane % TK;    // this lane's key in the score phase
  const int part = lane / TK; // which share of head_dim it sums (KS > 1)
  const int64_t head_off = (int64_t)kvh * a.kv_sh;

  for (int kt = 0; kt < kmax; kt += TK) {
    __syncthreads();  // the previous tile's readers are done
    for (int e = threadIdx.x; e < TK * CPR; e += blockDim.x) {
      const int r = e / CPR, ch = e - r * CPR;
      const int pos = kt + r;
      int64_t slot = -1;
      if (pos < kmax) {
        const int blk = a.bs_shift >= 0 ? pos >> a.bs_shift : pos / a.bs;
        const int64_t sl = (int64_t)a.tables[(int64_t)c * a.table_stride + blk] * a.bs +
                           (pos - blk * a.bs);
        slot = (sl >= 0 && sl < a.num_slots) ? sl : -1;
      }
      float kf[VEC], vf[VEC];
      if (slot >= 0) {
        const int64_t off = slot * a.kv_ss + head_off + ch * VEC;
        unpack16<DT>(*reinterpret_cast<const uint4*>(reinterpret_cast<const S*>(a.k) + off), kf);
        unpack16<DT>(*reinterpret_cast<const uint4*>(reinterpret_cast<const S*>(a.v) + off), vf);
      } else {
#pragma unroll
        for (int i = 0; i < VEC; ++i) kf[i] = vf[i] = 0.f;
      }
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        ks[r][ch * VEC + i] = kf[i];
        vs[r][ch * VEC + i] = vf[i];
      }
      if (ch == 0) live[r] = slot >= 0;
    }
    __syncthreads();

    // Scores of key kt + j for every pair.
    float sc[P];
#pragma unroll
    for (int p = 0; p < P; ++p) sc[p] = 0.f;
    constexpr int DS = HD / KS;  // head dims per lane share
#pragma unroll 2
    for (int d = part * DS; d < (part + 1) * DS; d += 4) {
      const float k0 = ks[j][d], k1 = ks[j][d + 1], k2 = ks[j][d + 2], k3 = ks[j][d + 3];
#pragma unroll
      for (int p = 0; p < P; ++p) {
        const float4 qv = *reinterpret_cast<const float4*>(&qs[wave][p][d]);
        sc[p] = __builtin_fmaf(k0, qv.x, __builtin_fmaf(k1, qv.y,
                 __builtin_fmaf(k2, qv.z, __builtin_fmaf(k3, qv.w, sc[p]))));
      }
    }
    const int kpos = kt + j;
    const bool key_ok = kpos < kmax && live[j];
#pragma unroll
    for (int p = 0; p < P; ++p) {
      if constexpr (KS > 1) sc[p] += __shfl_xor(sc[p], TK);
      const bool vis = key_ok && kpos <= qpos[p / GPW];
      const float s = vis ? sc[p] : -INFINITY;
      const float mx = across_max<1>(s);  // the same for every lane
      const float mn = fmaxf(m[p], mx);
      const float mref = mn == -INFINITY ? 0.f : mn;  // nothing visible yet: stay at 0
      const float alpha = __builtin_amdgcn_exp2f(m[p] - mref);
      const float pr = __builtin_amdgcn_exp2f(s - mref);
      m[p] = mn;
      l[p] = l[p] * alpha + (part == 0 ? pr : 0.f);
#pragma unroll
      for (int k = 0; k < DPL; ++k) acc[p][k] *= alpha;
      if (part == 0) es[wave][p][j] = pr;
    }
    __syncthreads();

    // P.V: lane d accumulates head dims d + 64 k.
#pragma unroll 2
    for (int jj = 0; jj < TK; jj += 4) {
      float vv[4][DPL];
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int k = 0; k < DPL; ++k)
          vv[r][k] = (lane + kWave * k < HD) ? vs[jj + r][lane + kWave * k] : 0.f;
#pragma unroll
      for (int p = 0; p < P; ++p) {
        const float4 w = *reinterpret_cast<const float4*>(&es[wave][p][jj]);
#pragma unroll
        for (int k = 0; k < DPL; ++k)
          acc[p][k] = __builtin_fmaf(w.x, vv[0][k], __builtin_fmaf(w.y, vv[1][k],
                      __builtin_fmaf(w.z, vv[2][k], __builtin_fmaf(w.w, vv[3][k], acc[p][k]))));
      }
    }
  }

#pragma unroll
  for (int p = 0; p < P; ++p) {
    const float lt = across_sum_exact<1>(l[p]);
    const int i = tok0 + p / GPW, h = h0 + p % GPW;
    if (i >= ql || h >= hend || (a.q_rows && a.q_rows[q0 + i] < 0)) continue;
    const float inv = lt > 0.f ? 1.f / lt : 0.f;  // nothing visible: 0
    const int64_t t = q0 + i;
#pragma unroll
    for (int k = 0; k < DPL; ++k) {
      const int d = lane + kWave * k;
      if (d >= HD) break;
      const int64_t e = t * a.out_st + (int64_t)h * a.out_sh + d;
      const float o = acc[p][k] * inv;
      if (a.out_f32) reinterpret_cast<float*>(a.out)[e] = o;
      else reinterpret_cast<S*>(a.out)[e] = Elt<DT>::from_f32(o);
    }
    if (a.lse && lane == 0) a.lse[t * a.nh + h] = lt > 0.f ? m[p] + __log2f(lt) : -INFINITY;
  }
}

// ---------------------------------------------------------------------------------
// Host-side dispatch.
// ---------------------------------------------------------------------------------

template <int DT, int HD>
hipError_t launch_prefill_hd(PrefillArgs a, int64_t rows, hipStream_t st) {
  constexpr int BM = PrefillShape<HD>::BM;
  a.row_blocks = (int)((rows + BM - 1) / BM);
  const int64_t items = (int64_t)a.row_blocks * a.nkv * a.n_chunks;
  if (items > 0x7FFFFFFF) return hipErrorInvalidValue;
  const dim3 grid((unsigned)items), block(512);
  if constexpr (DT == PKV_BF16) {
    if (a.v16) {  // P.V in fp16 against the copy of V
      if (a.bs_shift >= 0)
        hipLaunchKernelGGL((paged_prefill_kernel<DT, HD, true, true>), grid, block, 0, st, a);
      else
        hipLaunchKernelGGL((paged_prefill_kernel<DT, HD, false, true>), grid, block, 0, st, a);
      return hipGetLastError();
    }
  }
  if (a.bs_shift >= 0)
    hipLaunchKernelGGL((paged_prefill_kernel<DT, HD, true, false>), grid, block, 0, st, a);
  else
    hipLaunchKernelGGL((paged_prefill_kernel<DT, HD, false, false>), grid, block, 0, st, a);
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

// The fp16 V copy ahead of a bf16 matrix-core prefill: one workgroup per (region tile of
// the widest possible context, KV head, chunk), KV head innermost; workgroups past their
// chunk's context leave.
hipError_t launch_v16(const PrefillArgs& a, int hd, hipStream_t st) {
  const int64_t tiles = ((int64_t)a.max_blocks * a.bs + kV16Rows - 1) / kV16Rows;
  const int64_t wgs = tiles * a.nkv * a.n_chunks;
  if (wgs < 1) return hipSuccess;
  if (wgs > 0x7FFFFFFF) return hipErrorInvalidValue;
  const dim3 grid((unsigned)wgs), block(kV16Threads);
  switch (hd) {
    case 32: hipLaunchKernelGGL((prefill_v16_kernel<32>), grid, block, 0, st, a); break;
    case 64: hipLaunchKernelGGL((prefill_v16_kernel<64>), grid, block, 0, st, a); break;
    case 128: hipLaunchKernelGGL((prefill_v16_kernel<128>), grid, block, 0, st, a); break;
    default: hipLaunchKernelGGL((prefill_v16_kernel<256>), grid, block, 0, st, a); break;
  }
  return hipGetLastError();
}

// The VALU kernel: grid (chunks x query tiles, KV heads x head sub-groups).
template <int DT, int HD, int GPW>
hipError_t launch_rows_gpw(const PrefillArgs& a, int max_query_len, hipStream_t st) {
  constexpr int TOK = RowsShape<HD>::TOK;
  const int64_t tiles = (max_query_len + TOK - 1) / TOK;
  const int64_t x = tiles * a.n_chunks;
  const int64_t y = (int64_t)a.nkv * ((a.groups + GPW - 1) / GPW);
  if (x > 0x7FFFFFFF || y > 65535) return hipErrorInvalidValue;
  hipLaunchKernelGGL((paged_prefill_rows_kernel<DT, HD, GPW>), dim3((unsigned)x, (unsigned)y),
                     dim3(256), 0, st, a);
  return hipGetLastError();
}
template <int DT, int HD>
hipError_t launch_rows_hd(const PrefillArgs& a, int max_query_len, hipStream_t st) {
  if (a.groups == 1) return launch_rows_gpw<DT, HD, 1>(a, max_query_len, st);
  if (a.groups == 2) return launch_rows_gpw<DT, HD, 2>(a, max_query_len, st);
  return launch_rows_gpw<DT, HD, 4>(a, max_query_len, st);
}
template <int DT>
hipError_t launch_rows(const PrefillArgs& a, int hd, int max_query_len, hipStream_t st) {
  switch (hd) {
    case 16: return launch_rows_hd<DT, 16>(a, max_query_len, st);
    case 32: return launch_rows_hd<DT, 32>(a, max_query_len, st);
    case 64: return launch_rows_hd<DT, 64>(a, max_query_len, st);
    case 128: return launch_rows_hd<DT, 128>(a, max_query_len, st);
    default: return launch_rows_hd<DT, 256>(a, max_query_len, st);
  }
}

}  // namespace

namespace pkv {

int prefill_args(PrefillArgs* out_args, int64_t* rows_out, void* out, int out_dtype,
                 int64_t out_stride_tok, int64_t out_stride_h, const void* q,
                 int64_t q_stride_tok, int64_t q_stride_h, const void* k_cache,
                 const void* v_cache, int kv_dtype, int64_t kv_stride_slot,
                 int64_t kv_stride_head, int64_t num_slots, const int32_t* block_tables,
                 int64_t table_stride, int32_t max_blocks, const int32_t* context_lens,
                 const int32_t* cu_seqlens_q, int32_t n_chunks, int32_t max_query_len,
                 int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                 float scale, int32_t causal, const int32_t* q_rows, float* lse) {
  if (!valid_dtype(kv_dtype)) return PKV_E_DTYPE;
  if (!(out_dtype == kv_dtype || out_dtype == PKV_F32)) return PKV_E_DTYPE;
  if (num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads || block_size <= 0 ||
      max_blocks < 0 || n_chunks < 0 || n_chunks > 65535 || max_query_len < 0 ||
      num_kv_heads > 65535)
    return PKV_E_SHAPE;
  if (!(head_dim == 16 || head_dim == 32 || head_dim == 64 || head_dim == 128 ||
        head_dim == 256))
    return PKV_E_SHAPE;
  if ((int64_t)max_blocks * block_size > (int64_t)1 << 30) return PKV_E_SHAPE;
  if (!(scale > 0.f && scale < INFINITY)) return PKV_E_SHAPE;  // softmax scale
  const int64_t rows = (int64_t)max_query_len * (num_heads / num_kv_heads);
  if (rows > (int64_t)1 << 30) return PKV_E_SHAPE;
  if (n_chunks == 0 || max_query_len == 0) return 1;
  if (!out || !q || !k_cache || !v_cache || !context_lens || !cu_seqlens_q ||
      (max_blocks > 0 && !block_tables))
    return PKV_E_NULL;
  const int vec = kv_dtype == PKV_F32 ? 4 : 8;
  if (!aligned16(q) || !aligned16(k_cache) || !aligned16(v_cache) || !aligned16(out) ||
      q_stride_tok % vec || q_stride_h % vec || kv_stride_slot % vec || kv_stride_head % vec ||
      out_stride_tok % vec || out_stride_h % vec)
    return PKV_E_ALIGN;
  *rows_out = rows;
  PrefillArgs& a = *out_args;
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
  a.row_blocks = 0;  // set per head_dim at launch
  a.causal = causal != 0;
  a.q_rows = q_rows;
  a.lse = lse;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.out_f32 = out_dtype == PKV_F32;
  a.v16 = nullptr;
  a.v16_k = nullptr;
  a.v16_kstride = 0;
  return 0;
}

}  // namespace pkv

namespace {

// Launches for checked arguments: the matrix cores take 16-bit K/V at head_dim 32..256
// (a bf16 call with a.v16 set converts the chunks' V first), the VALU kernel the rest.
int run_prefill(const PrefillArgs& a, int64_t rows, int kv_dtype, int head_dim,
                int max_query_len, hipStream_t st) {
  if (kv_dtype == PKV_F32) return (int)launch_rows<PKV_F32>(a, head_dim, max_query_len, st);
  if (head_dim == 16) {
    return (int)(kv_dtype == PKV_BF16 ? launch_rows<PKV_BF16>(a, head_dim, max_query_len, st)
                                      : launch_rows<PKV_F16>(a, head_dim, max_query_len, st));
  }
  if (kv_dtype == PKV_F16) return (int)launch_prefill<PKV_F16>(a, head_dim, rows, st);
  if (a.v16) {
    const hipError_t e = launch_v16(a, head_dim, st);
    if (e != hipSuccess) return (int)e;
  }
  return (int)launch_prefill<PKV_BF16>(a, head_dim, rows, st);
}

// Whether a call of these shapes can use the fp16 V copy: bf16 at head_dim 32..256,
// tables of at most kV16MaxTokens tokens, slot indices within 31 bits.
bool v16_shapes(int kv_dtype, int head_dim, int32_t max_blocks, int32_t block_size,
                int64_t num_slots) {
  return kv_dtype == PKV_BF16 && head_dim >= 32 && head_dim <= 256 &&
         (int64_t)max_blocks * block_size <= kV16MaxTokens && num_slots <= 0x7FFFFFFF;
}

// Workspace of the fp16 V copy: the scale exponents (a row of kstride bytes per chunk and
// KV head, the area rounded up to 256 bytes), then every chunk's region at its widest.
struct V16Layout {
  int64_t kstride, k_bytes, total;
};
V16Layout v16_layout(int32_t head_dim, int32_t num_kv_heads, int32_t n_chunks,
                     int32_t max_blocks, int32_t block_size) {
  const int64_t pad = v16_pad(max_blocks * block_size);
  V16Layout l;
  l.kstride = (pad / kV16Rows + 3) / 4 * 4;
  l.k_bytes = ((int64_t)n_chunks * num_kv_heads * l.kstride + 255) / 256 * 256;
  l.total = l.k_bytes + (int64_t)n_chunks * pad * num_kv_heads * head_dim * 2;
  return l;
}

}  // namespace

extern "C" {

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
  PrefillArgs a;
  int64_t rows = 0;
  const int bad = prefill_args(&a, &rows, out, out_dtype, out_stride_tok, out_stride_h, q,
                               q_stride_tok, q_stride_h, k_cache, v_cache, kv_dtype,
                               kv_stride_slot, kv_stride_head, num_slots, block_tables,
                               table_stride, max_blocks, context_lens, cu_seqlens_q, n_chunks,
                               max_query_len, num_heads, num_kv_heads, head_dim, block_size,
                               scale, causal, q_rows, lse);
  if (bad) return bad == 1 ? 0 : bad;
  return run_prefill(a, rows, kv_dtype, head_dim, max_query_len, (hipStream_t)stream);
}

int64_t pkv_prefill_workspace_bytes(int kv_dtype, int32_t head_dim, int32_t num_kv_heads,
                                    int32_t n_chunks, int32_t max_blocks, int32_t block_size) {
  if (!valid_dtype(kv_dtype)) return PKV_E_DTYPE;
  if (!(head_dim == 16 || head_dim == 32 || head_dim == 64 || head_dim == 128 ||
        head_dim == 256) ||
      num_kv_heads <= 0 || n_chunks < 0 || max_blocks < 0 || block_size <= 0 ||
      (int64_t)max_blocks * block_size > (int64_t)1 << 30)
    return PKV_E_SHAPE;
  if (!v16_shapes(kv_dtype, head_dim, max_blocks, block_size, 0)) return 0;
  return v16_layout(head_dim, num_kv_heads, n_chunks, max_blocks, block_size).total;
}

int pkv_paged_prefill_ws(void* out, int out_dtype, int64_t out_stride_tok, int64_t out_stride_h,
                         const void* q, int64_t q_stride_tok, int64_t q_stride_h,
                         const void* k_cache, const void* v_cache, int kv_dtype,
                         int64_t kv_stride_slot, int64_t kv_stride_head, int64_t num_slots,
                         const int32_t* block_tables, int64_t table_stride, int32_t max_blocks,
                         const int32_t* context_lens, const int32_t* cu_seqlens_q,
                         int32_t n_chunks, int32_t max_query_len, int32_t num_heads,
                         int32_t num_kv_heads, int32_t head_dim, int32_t block_size, float scale,
                         void* workspace, int64_t workspace_bytes, void* stream) {
  PrefillArgs a;
  int64_t rows = 0;
  const int bad = prefill_args(&a, &rows, out, out_dtype, out_stride_tok, out_stride_h, q,
                               q_stride_tok, q_stride_h, k_cache, v_cache, kv_dtype,
                               kv_stride_slot, kv_stride_head, num_slots, block_tables,
                               table_stride, max_blocks, context_lens, cu_seqlens_q, n_chunks,
                               max_query_len, num_heads, num_kv_heads, head_dim, block_size,
                               scale, 1, nullptr, nullptr);
  if (bad) return bad == 1 ? 0 : bad;
  if (workspace_bytes < 0 || (workspace_bytes > 0 && !workspace)) return PKV_E_WORKSPACE;
  if (workspace && !aligned16(workspace)) return PKV_E_ALIGN;
  if (workspace && v16_shapes(kv_dtype, head_dim, max_blocks, block_size, num_slots)) {
    const V16Layout l = v16_layout(head_dim, num_kv_heads, n_chunks, max_blocks, block_size);
    if (workspace_bytes >= l.total) {
      a.v16_k = static_cast<const uint8_t*>(workspace);
      a.v16_kstride = (int32_t)l.kstride;
      a.v16 = static_cast<const char*>(workspace) + l.k_bytes;
    }
  }
  return run_prefill(a, rows, kv_dtype, head_dim, max_query_len, (hipStream_t)stream);
}

}  // extern "C"
