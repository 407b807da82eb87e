// decode.hip -- host side of paged decode attention (include/paged_kv.h:
// pkv_paged_decode*, pkv_decode_*): argument checks, the choice of split, the workspace
// layout and the launches of the stream-K pass, the per-sequence split pass and the
// combine (kernels in decode_kernels.h).

#include "cascade.h"
#include "decode_kernels.h"

#include <mutex>

namespace {

using namespace pkv;

// ---------------------------------------------------------------------------------
// Host-side dispatch.
// ---------------------------------------------------------------------------------

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
  return DT != PKV_F32 && (HD == 128 || HD == 64) && PKV_DECODE_USE_MFMA;
}
template <int DT, int HD, int GPW> const void* decode_kernel() {
  if constexpr (use_mfma<DT, HD>())
    return reinterpret_cast<const void*>(&paged_decode_mfma_kernel<DT, GPW, true, HD, false>);
  else
    return reinterpret_cast<const void*>(&paged_decode_stream_kernel<DT, HD, GPW>);
}

// Up to this many (sequence, head) pairs the combine gives each pair two waves (at most
// 4,096 waves: all resident on a 256-CU part); larger batches get one wave per pair.
constexpr int kCombineSplitPairs = PKV_DECODE_COMBINE_SPLIT_PAIRS;

struct LaunchDecode {
  const DecodeArgs* a;
  int wpg, ygrid;
  hipStream_t st;
  const CascadeLaunch* one = nullptr;  // non-null: the stream pass shares a launch with a prefix pass
  template <int DT, int HD, int GPW> hipError_t run() const {
    const dim3 grid((unsigned)a->num_wg, (unsigned)ygrid), block(kWave * wpg);
    if constexpr (use_mfma<DT, HD>()) {
      const bool staged = a->batch > kWave && a->batch <= kLdsBatch;
      if (one) {
        const hipError_t e = launch_cascade(*a, *one->p, one->rows, DT, HD, GPW, one->prefix_wg,
                                            ygrid, st);
        if (e != hipSuccess) return e;
      } else if (a->bs % 16 == 0 && staged)
        hipLaunchKernelGGL((paged_decode_mfma_kernel<DT, GPW, true, HD, false, true>), grid, block, 0, st, *a);
      else if (a->bs % 16 == 0)
        hipLaunchKernelGGL((paged_decode_mfma_kernel<DT, GPW, true, HD, false>), grid, block, 0, st, *a);
      else if (staged)
        hipLaunchKernelGGL((paged_decode_mfma_kernel<DT, GPW, false, HD, false, true>), grid, block, 0, st, *a);
      else
        hipLaunchKernelGGL((paged_decode_mfma_kernel<DT, GPW, false, HD, false>), grid, block, 0, st, *a);
    } else {
      hipLaunchKernelGGL((paged_decode_stream_kernel<DT, HD, GPW>), grid, block, 0, st, *a);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || (a->num_wg <= 1 && !a->pre_row)) return e;
    const int pairs = a->batch * a->nh;  // (sequence, query head) pairs
    const dim3 g2((unsigned)((pairs + 1) / 2)), g1((unsigned)((pairs + 3) / 4));
    if (one && pairs <= kCombineSplitPairs)  // after a one-launch cascade: its unit split
      hipLaunchKernelGGL((paged_decode_combine_kernel<DT, HD, 2, true>), g2, dim3(256), 0, st, *a);
    else if (one)
      hipLaunchKernelGGL((paged_decode_combine_kernel<DT, HD, 1, true>), g1, dim3(256), 0, st, *a);
    else if (pairs <= kCombineSplitPairs)
      hipLaunchKernelGGL((paged_decode_combine_kernel<DT, HD, 2>), g2, dim3(256), 0, st, *a);
    else
      hipLaunchKernelGGL((paged_decode_combine_kernel<DT, HD, 1>), g1, dim3(256), 0, st, *a);
    return hipGetLastError();
  }
};

// The per-sequence split pass (16-bit K/V at head_dim 64 or 128 only).
struct LaunchSplit {
  const DecodeArgs* a;
  int ytasks;
  hipStream_t st;
  template <int DT, int HD, int GPW> hipError_t run() const {
    if constexpr (use_mfma<DT, HD>()) {
      const dim3 grid((unsigned)a->batch, (unsigned)ytasks), block(kWave * kSplitWaves);
      if (a->bs % 16 == 0)
        hipLaunchKernelGGL((paged_decode_mfma_kernel<DT, GPW, true, HD, true>), grid, block, 0, st, *a);
      else
        hipLaunchKernelGGL((paged_decode_mfma_kernel<DT, GPW, false, HD, true>), grid, block, 0, st, *a);
      return hipGetLastError();
    } else {
      return hipErrorInvalidValue;  // never chosen for these shapes
    }
  }
};

// Unit size (TILE tokens) of an instantiation, and how many of its workgroups one CU
// holds at once.
struct QueryDecode {
  int wpg;
  int* tile;
  int* per_cu;  // may be null: tile only
  template <int DT, int HD, int GPW> hipError_t run() const {
    static_assert(!use_mfma<DT, HD>() || DecodeShape<DT, HD>::TILE == 16,
                  "the MFMA kernel's unit is 16 tokens");
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

// Scratch of pkv_paged_decode_noalloc: the decode workspace (merge plans and partial
// records) for callers that cannot allocate. Each GPU the library runs on holds its own
// copy until the process ends. Host code must never pass `scratch` itself to a kernel (in
// host code the name is only a stand-in for the device symbol): it uses the per-device
// address hipGetSymbolAddress returns, kept in g_scratch_ptr.
static __device__ __align__(256) unsigned char scratch[PKV_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
void* g_scratch_ptr[kMaxDevices] = {};
std::mutex g_scratch_mu;

// CU count of the current device, queried once per device.
int g_cus[kMaxDevices] = {};
std::mutex g_cus_mu;
int device_cus(int* cus) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return PKV_E_HIP;
  std::lock_guard<std::mutex> lock(g_cus_mu);
  if (!g_cus[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n < 1)
      return PKV_E_HIP;
    g_cus[dev] = n;
  }
  *cus = g_cus[dev];
  return 0;
}

// Whether a default-split call (num_workgroups == 0) takes the per-sequence split pass,
// and with how many query heads per wave (*gpw, 0 = no): 16-bit K/V at head_dim 64 or
// 128, no cascade extras, the table width bounds every wave's share to kSplitMaxTiles
// tiles, and the (sequence, KV head, head sub-group) workgroups fit the CUs. The split
// pass is bound by each wave's VALU work (its P.V runs per query head), so the fewest
// heads per wave whose workgroups still fit the CUs is taken: more CUs at work, each
// wave's K/V re-read by the head sub-groups from cache. Static shapes only, so a
// captured graph stays valid for every context length.
int choose_split(int kv_dtype, int head_dim, int batch, int num_heads, int num_kv_heads,
                 int max_columns, int64_t max_tokens, bool extras, int* gpw) {
  *gpw = 0;
  const bool mfma = kv_dtype != PKV_F32 && (head_dim == 64 || head_dim == 128) &&
                    PKV_DECODE_USE_MFMA;
  if (!mfma || extras) return 0;
  const int64_t tiles = (max_tokens + 15) / 16;
  if (tiles > (int64_t)kSplitWaves * kSplitMaxTiles || max_columns > kSplitMaxColumns) return 0;
  int cus = 0;
  const int st = device_cus(&cus);
  if (st) return st;
  const int groups = num_heads / num_kv_heads;
  for (int g = 1; g <= 4; ++g)
    if (groups % g == 0 && (int64_t)batch * num_kv_heads * (groups / g) <= cus) {
      *gpw = g;
      break;
    }
  return 0;
}

// The current device's address of `scratch`, resolved on the first call per device (with
// that device current) and cached. Returns 0 or a PKV_E_* / hipError_t status.
int scratch_address(void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return PKV_E_HIP;
  if (dev >= kMaxDevices) return PKV_E_SHAPE;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (!p) return PKV_E_HIP;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

}  // namespace

namespace pkv {

int decode_ex(void* out, int out_dtype, int64_t out_stride_b, int64_t out_stride_h,
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
              int64_t prefix_stride, void* stream,
              const CascadeLaunch* one, bool check_only) {
  const int bad = check_decode_shape(kv_dtype, head_dim, num_heads, num_kv_heads);
  if (bad) return bad;
  const bool cascade = prefix_row != nullptr && prefix_parts > 0;
  if (prefix_parts < 0 || prefix_stride < 0) return PKV_E_SHAPE;
  if (cascade && (!prefix_out || !prefix_lse)) return PKV_E_NULL;
  if (cascade && !aligned16(prefix_out)) return PKV_E_ALIGN;
  if (!(out_dtype == kv_dtype || out_dtype == PKV_F32)) return PKV_E_DTYPE;
  if (batch < 0 || block_size <= 0 || max_blocks < 0 || num_workgroups < 0 ||
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
  DecodePlan p = plan_decode(num_heads, num_kv_heads);
  bool split = false;
  if (num_workgroups == 0) {  // the library's default split of the work
    int split_gpw = 0;
    const int st = choose_split(kv_dtype, head_dim, batch, num_heads, num_kv_heads, max_blocks,
                                (int64_t)max_blocks * block_size,
                                cascade || first_block || lse, &split_gpw);
    if (st) return st;
    split = split_gpw > 0;
    if (split) {
      p.gpw = split_gpw;
      p.nsub = num_heads / num_kv_heads / split_gpw;
    } else {
      num_workgroups = pkv_decode_workgroups(kv_dtype, head_dim, num_heads, num_kv_heads);
      if (num_workgroups < 1) return num_workgroups < 0 ? num_workgroups : PKV_E_HIP;
    }
  }

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
  a.full_wg = a.slots = num_workgroups;  // one slot per range
  a.wslots = a.tail_slots = 1;
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
  hipStream_t st = (hipStream_t)stream;
  if (split) {
    if (check_only) return 0;
    a.num_wg = a.full_wg = a.slots = 1;
    return (int)by_dtype(kv_dtype, head_dim, p.gpw,
                         LaunchSplit{&a, num_kv_heads * p.nsub, st});
  }
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

  if (one) {  // the prefix pass takes one->prefix_wg of the num_workgroups
    if (split || !cascade || one->prefix_wg < 1 || num_workgroups - one->prefix_wg < 1 ||
        !cascade_one_launch_shape(kv_dtype, head_dim, block_size, batch, p.wpg))
      return PKV_E_SHAPE;
    // Ranges 0 .. D - 1 belong to the stream workgroups, D .. D + P - 1 (tail_slots > 0)
    // to the prefix workgroups, which stream a smaller share once their items are done.
    const int d = num_workgroups - one->prefix_wg;
    a.full_wg = d;
    if (one->tail_slots > 0) {
      a.num_wg = num_workgroups;
      a.wslots = one->wslots;
      a.tail_slots = one->tail_slots;
      a.slots = d * one->wslots + one->prefix_wg * one->tail_slots;
    } else {
      a.num_wg = a.slots = d;
    }
  }
  if (check_only) return 0;
  return (int)by_dtype(kv_dtype, head_dim, p.gpw, LaunchDecode{&a, p.wpg, p.ygrid, st, one});
}

int cascade_prefix_wg(int kv_dtype, int head_dim, int num_heads, int num_kv_heads,
                      int block_size, int batch, int num_workgroups, int64_t items,
                      int requested) {
  if (requested < 0 || items < 1 || check_decode_shape(kv_dtype, head_dim, num_heads, num_kv_heads))
    return 0;
  const DecodePlan p = plan_decode(num_heads, num_kv_heads);
  if (!cascade_one_launch_shape(kv_dtype, head_dim, block_size, batch, p.wpg)) return 0;
  if (num_workgroups == 0)
    num_workgroups = pkv_decode_workgroups(kv_dtype, head_dim, num_heads, num_kv_heads);
  if (num_workgroups < 2) return 0;
  int64_t wg = requested;
  if (wg == 0) {
    // Measured on 256 CUs (prefix of 2,048 tokens, private tails of 0-1,024, 96-512
    // sequences): best with one item per prefix workgroup, plus one spare prefix
    // workgroup per 32 resident ones (it only streams its tail share) up to 56 items;
    // past 80 items, two items each. The thresholds scale with the workgroups the GPU
    // holds at once (prefix workers are wg x ygrid).
    const int64_t slots = (int64_t)num_workgroups * p.ygrid;
    const int64_t quarter = slots / 4 > 0 ? slots / 4 : 1;
    int64_t workers = items;
    if (items <= 7 * slots / 32) workers = items + slots / 32;
    else if (items > 5 * slots / 16) {
      const int64_t rounds = (items + quarter - 1) / quarter;
      workers = (items + rounds - 1) / rounds;
    }
    wg = (workers + p.ygrid - 1) / p.ygrid;
  }
  return wg >= 1 && num_workgroups - wg >= 1 ? (int)wg : 0;
}
}  // namespace pkv

extern "C" {

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

int32_t pkv_decode_default_workgroups(int kv_dtype, int32_t head_dim, int32_t num_heads,
                                      int32_t num_kv_heads, int32_t batch, int32_t max_blocks,
                                      int32_t block_size) {
  const int bad = check_decode_shape(kv_dtype, head_dim, num_heads, num_kv_heads);
  if (bad) return bad;
  if (batch < 0 || max_blocks < 0 || block_size <= 0) return PKV_E_SHAPE;
  int split_gpw = 0;
  const int st = choose_split(kv_dtype, head_dim, batch, num_heads, num_kv_heads, max_blocks,
                              (int64_t)max_blocks * block_size, false, &split_gpw);
  if (st) return st;
  return split_gpw ? 0 : pkv_decode_workgroups(kv_dtype, head_dim, num_heads, num_kv_heads);
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
  return decode_ex(out, out_dtype, out_stride_b, out_stride_h, q, q_stride_b, q_stride_h, k_cache,
                   v_cache, kv_dtype, kv_stride_slot, kv_stride_head, num_slots, block_tables,
                   table_stride, max_blocks, context_lens, batch, num_heads, num_kv_heads,
                   head_dim, block_size, scale, num_workgroups, workspace, workspace_bytes,
                   first_block, lse, prefix_out, prefix_lse, prefix_row, prefix_parts,
                   prefix_stride, stream, nullptr, false);
}

int pkv_paged_decode_noalloc(void* out, int out_dtype, int64_t out_stride_b,
                             int64_t out_stride_h, const void* q, int64_t q_stride_b,
                             int64_t q_stride_h, const void* k_cache, const void* v_cache,
                             int kv_dtype, int64_t kv_stride_slot, int64_t kv_stride_head,
                             int64_t num_slots, const int32_t* block_tables,
                             int64_t table_stride, int32_t max_blocks,
                             const int32_t* context_lens, int32_t batch, int32_t num_heads,
                             int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                             float scale, int32_t num_workgroups, void* stream) {
  const int bad = check_decode_shape(kv_dtype, head_dim, num_heads, num_kv_heads);
  if (bad) return bad;
  if (batch < 0 || num_workgroups < 0 || num_workgroups > (1 << 24) || batch > (1 << 24))
    return PKV_E_SHAPE;
  // The same workspace layout the allocating entry point asks its caller for; it must
  // fit the static array (no contents need clearing: every record is written before
  // the combine reads it, within the call). The default split (0) is sized by what it
  // runs: the one-launch split pass needs no workspace (and no symbol lookup), stream-K
  // its workgroup count's records.
  int sized = num_workgroups;
  if (sized == 0 && batch > 0) {
    sized = pkv_decode_default_workgroups(kv_dtype, head_dim, num_heads, num_kv_heads, batch,
                                          max_blocks, block_size);
    if (sized < 0) return sized;
  }
  const int64_t need = decode_ws(sized, batch, num_heads, head_dim, false).total;
  if (need > PKV_NOALLOC_SCRATCH_BYTES) return PKV_E_SCRATCH;
  void* ws = nullptr;
  if (need > 0 && batch > 0) {
    const int st = scratch_address(&ws);
    if (st) return st;
  }
  return pkv_paged_decode_ex(out, out_dtype, out_stride_b, out_stride_h, q, q_stride_b,
                             q_stride_h, k_cache, v_cache, kv_dtype, kv_stride_slot,
                             kv_stride_head, num_slots, block_tables, table_stride, max_blocks,
                             context_lens, batch, num_heads, num_kv_heads, head_dim, block_size,
                             scale, num_workgroups, ws, ws ? PKV_NOALLOC_SCRATCH_BYTES : 0,
                             nullptr, nullptr, nullptr, nullptr, nullptr, 0, 0, stream);
}

}  // extern "C"
