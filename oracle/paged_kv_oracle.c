/*
 * paged_kv_oracle.c — CPU restatement of the reference's paged-KV path.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg load this (through oracle/oracle.py), and only as the checker or the
 * timed CPU baseline. The product path never does.
 *
 * Functions and the reference code they restate:
 *   or_f32_to_bf16 / or_f32_to_f16 / or_f16_to_f32  torch's Tensor.to() rounding, used
 *       by PagedKVCache.write (reference engine/runtime/paged_cache.py:44-45)
 *   or_kv_append         PagedKVCache.write, two index_copy_ (paged_cache.py:42-45)
 *   or_copy_blocks       build-defined copy-on-write block copy (no reference code)
 *   or_decode_attention  reference_decode_attention (engine/kernels/paged_attention.py:
 *                        192-211): per sequence gather slots = table[p/bs]*bs + p%bs,
 *                        query head h reads KV head h/G (repeat_interleave), softmax of
 *                        scale*q.k, times V. Accumulated in double; fp32 output (the
 *                        reference casts to q.dtype afterwards).
 *   or_decode_partials / or_combine   the split-K decomposition of the same sum and its
 *                        log-sum-exp merge (flash-decoding; absent in the reference).
 *   or_prefill_attention chunk attention with the bottom-right causal mask of
 *                        PagedBatch._mixed (paged_cache.py:187-194): query i of a chunk
 *                        of q tokens with context ctx sees keys k <= ctx - q + i.
 *
 * dtype codes: 0 float32, 1 float16, 2 bfloat16 (as include/paged_kv.h).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ---- IEEE conversions, written from the format definitions ---- */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float or_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* Round to nearest, ties to even, on the top 16 bits; NaN -> 0x7FC0 (torch's choice). */
uint16_t or_f32_to_bf16(float f) {
  if (f != f) return 0x7FC0;
  uint32_t u = f2u(f);
  uint32_t lsb = (u >> 16) & 1u;
  return (uint16_t)((u + 0x7FFFu + lsb) >> 16);
}

float or_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  int exp = (h >> 10) & 0x1F;
  uint32_t man = h & 0x3FFu;
  if (exp == 0x1F) return u2f(sign | 0x7F800000u | (man << 13)); /* inf / nan */
  if (exp == 0) {
    if (man == 0) return u2f(sign);
    /* subnormal: man * 2^-24 exactly */
    float v = (float)man * 5.9604644775390625e-08f;
    return sign ? -v : v;
  }
  return u2f(sign | ((uint32_t)(exp - 15 + 127) << 23) | (man << 13));
}

/* Round to nearest even. NaN keeps its sign and top payload bits and is made quiet. */
uint16_t or_f32_to_f16(float f) {
  uint32_t u = f2u(f);
  uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  uint32_t a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return (uint16_t)(sign | 0x7E00u | ((a >> 13) & 0x3FFu));
  if (a >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* rounds to >= 65520: inf */
  if (a < 0x38800000u) {                                    /* below 2^-14: subnormal */
    /* value / 2^-24, rounded to nearest even integer */
    float v = u2f(a) * 16777216.0f; /* exact: scaling by a power of two */
    float r = nearbyintf(v);        /* default rounding mode: ties to even */
    return (uint16_t)(sign | (uint16_t)r);
  }
  uint32_t exp = (a >> 23) - 127 + 15;
  uint32_t man = a & 0x7FFFFFu;
  uint32_t h = (exp << 10) | (man >> 13);
  uint32_t rem = man & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1; /* carry may bump exponent */
  return (uint16_t)(sign | h);
}

static inline float load_elt(const void* base, int64_t i, int dt) {
  switch (dt) {
    case 0: return ((const float*)base)[i];
    case 1: return or_f16_to_f32(((const uint16_t*)base)[i]);
    default: return or_bf16_to_f32(((const uint16_t*)base)[i]);
  }
}

static inline void store_elt(void* base, int64_t i, int dt, float f) {
  switch (dt) {
    case 0: ((float*)base)[i] = f; break;
    case 1: ((uint16_t*)base)[i] = or_f32_to_f16(f); break;
    default: ((uint16_t*)base)[i] = or_f32_to_bf16(f);
  }
}

static inline int dt_size(int dt) { return dt == 0 ? 4 : 2; }

/* ---- KV append ---- */

/* pool[slots[i], h, :] = convert(new[i, h, :]) for K and V; out-of-range slots skipped.
 * Same dtype: the bits are copied untouched (Tensor.to(same dtype) is the identity). */
void or_kv_append(void* k_pool, void* v_pool, int pool_dt, int64_t ps_slot, int64_t ps_head,
                  int64_t num_slots, const void* k_new, int64_t ks_tok, int64_t ks_head,
                  const void* v_new, int64_t vs_tok, int64_t vs_head, int new_dt,
                  const int64_t* slots, int64_t n, int nkv, int hd) {
  for (int64_t i = 0; i < n; ++i) {
    int64_t s = slots[i];
    if (s < 0 || s >= num_slots) continue;
    for (int which = 0; which < 2; ++which) {
      void* pool = which ? v_pool : k_pool;
      const void* src = which ? v_new : k_new;
      int64_t st = which ? vs_tok : ks_tok, sh = which ? vs_head : ks_head;
      for (int h = 0; h < nkv; ++h) {
        for (int d = 0; d < hd; ++d) {
          int64_t si = i * st + h * sh + d, di = s * ps_slot + h * ps_head + d;
          if (pool_dt == new_dt) {
            memcpy((char*)pool + di * dt_size(pool_dt), (const char*)src + si * dt_size(new_dt),
                   dt_size(pool_dt));
          } else {
            store_elt(pool, di, pool_dt, load_elt(src, si, new_dt));
          }
        }
      }
    }
  }
}

/* ---- block copy ---- */

void or_copy_blocks(void* k_pool, void* v_pool, int64_t layer_stride_bytes, int num_layers,
                    int64_t block_bytes, int64_t num_blocks, const int64_t* mapping,
                    int64_t n_pairs) {
  for (int64_t p = 0; p < n_pairs; ++p) {
    int64_t src = mapping[2 * p], dst = mapping[2 * p + 1];
    if (src < 0 || src >= num_blocks || dst < 0 || dst >= num_blocks) continue;
    for (int l = 0; l < num_layers; ++l) {
      for (int which = 0; which < 2; ++which) {
        char* pool = (char*)(which ? v_pool : k_pool) + l * layer_stride_bytes;
        memmove(pool + dst * block_bytes, pool + src * block_bytes, (size_t)block_bytes);
      }
    }
  }
}

/* ---- decode attention ---- */

typedef struct {
  const void* q; int64_t q_sb, q_sh;
  const void* k; const void* v; int dt; int64_t kv_ss, kv_sh;
  const int32_t* tables; int64_t t_sb;
  const int32_t* ctx;
  int nh, nkv, hd, bs;
  double scale;
} dec_t;

static inline int64_t slot_at(const dec_t* a, int b, int64_t p) {
  return (int64_t)a->tables[b * a->t_sb + p / a->bs] * a->bs + p % a->bs;
}

/* Partial softmax state of query head h of sequence b over positions [p0, p1):
 * m = max score, l = sum exp(score - m), acc = sum exp(score - m) v. */
static void partial(const dec_t* a, int b, int h, int64_t p0, int64_t p1, double* qv,
                    double* sc, double* m_out, double* l_out, double* acc) {
  const int g = h / (a->nh / a->nkv);
  for (int d = 0; d < a->hd; ++d) qv[d] = load_elt(a->q, b * a->q_sb + h * a->q_sh + d, a->dt);
  double m = -INFINITY;
  for (int64_t p = p0; p < p1; ++p) {
    const int64_t base = slot_at(a, b, p) * a->kv_ss + g * a->kv_sh;
    double s = 0.0;
    for (int d = 0; d < a->hd; ++d) s += qv[d] * (double)load_elt(a->k, base + d, a->dt);
    s *= a->scale;
    sc[p - p0] = s;
    if (s > m) m = s;
  }
  double l = 0.0;
  for (int d = 0; d < a->hd; ++d) acc[d] = 0.0;
  for (int64_t p = p0; p < p1; ++p) {
    const double e = exp(sc[p - p0] - m);
    l += e;
    const int64_t base = slot_at(a, b, p) * a->kv_ss + g * a->kv_sh;
    for (int d = 0; d < a->hd; ++d) acc[d] += e * (double)load_elt(a->v, base + d, a->dt);
  }
  *m_out = m;
  *l_out = l;
}

static int max_ctx(const int32_t* ctx, int batch) {
  int mx = 0;
  for (int b = 0; b < batch; ++b) mx = ctx[b] > mx ? ctx[b] : mx;
  return mx;
}

/* out: float32 [batch, nh, hd] contiguous. Context lengths must be >= 0 and covered by
 * the table row (the reference indexes the table directly). n == 0 gives zeros. */
int or_decode_attention(float* out, const void* q, int64_t q_sb, int64_t q_sh,
                        const void* k, const void* v, int dt, int64_t kv_ss, int64_t kv_sh,
                        const int32_t* tables, int64_t t_sb, const int32_t* ctx, int batch,
                        int nh, int nkv, int hd, int bs, double scale, int threads) {
  dec_t a = {q, q_sb, q_sh, k, v, dt, kv_ss, kv_sh, tables, t_sb, ctx, nh, nkv, hd, bs, scale};
  if (nkv <= 0 || nh % nkv || bs <= 0) return -1;
  const int mc = max_ctx(ctx, batch);
  int err = 0;
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel
#endif
  {
    double* qv = (double*)malloc(sizeof(double) * hd);
    double* acc = (double*)malloc(sizeof(double) * hd);
    double* sc = (double*)malloc(sizeof(double) * (mc > 0 ? mc : 1));
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
    for (int64_t w = 0; w < (int64_t)batch * nh; ++w) {
      const int b = (int)(w / nh), h = (int)(w % nh);
      const int n = ctx[b];
      float* o = out + w * hd;
      if (n < 0) { err = -2; continue; }
      if (n == 0) { for (int d = 0; d < hd; ++d) o[d] = 0.f; continue; }
      double m, l;
      partial(&a, b, h, 0, n, qv, sc, &m, &l, acc);
      for (int d = 0; d < hd; ++d) o[d] = (float)(acc[d] / l);
    }
    free(qv); free(acc); free(sc);
  }
  return err;
}

/* Split-K partials: split s covers positions [s*split, min(n, (s+1)*split)).
 * ml: float64 [batch, nh, n_splits, 2] (m, l); acc: float64 [batch, nh, n_splits, hd].
 * Splits past the context get m = -inf, l = 0, acc = 0. */
int or_decode_partials(double* ml, double* acc, const void* q, int64_t q_sb, int64_t q_sh,
                       const void* k, const void* v, int dt, int64_t kv_ss, int64_t kv_sh,
                       const int32_t* tables, int64_t t_sb, const int32_t* ctx, int batch,
                       int nh, int nkv, int hd, int bs, double scale, int split_tokens,
                       int n_splits) {
  dec_t a = {q, q_sb, q_sh, k, v, dt, kv_ss, kv_sh, tables, t_sb, ctx, nh, nkv, hd, bs, scale};
  if (nkv <= 0 || nh % nkv || bs <= 0 || split_tokens <= 0) return -1;
  double* qv = (double*)malloc(sizeof(double) * hd);
  double* sc = (double*)malloc(sizeof(double) * split_tokens);
  for (int b = 0; b < batch; ++b) {
    for (int h = 0; h < nh; ++h) {
      for (int s = 0; s < n_splits; ++s) {
        const int64_t row = ((int64_t)b * nh + h) * n_splits + s;
        const int64_t p0 = (int64_t)s * split_tokens;
        int64_t p1 = p0 + split_tokens;
        if (p1 > ctx[b]) p1 = ctx[b];
        if (p0 >= p1) {
          ml[2 * row] = -INFINITY;
          ml[2 * row + 1] = 0.0;
          for (int d = 0; d < hd; ++d) acc[row * hd + d] = 0.0;
          continue;
        }
        partial(&a, b, h, p0, p1, qv, sc, &ml[2 * row], &ml[2 * row + 1], &acc[row * hd]);
      }
    }
  }
  free(qv); free(sc);
  return 0;
}

/* Merge n_splits partial states per row: M = max m_s, w_s = exp(m_s - M),
 * out = sum w_s acc_s / sum w_s l_s. Rows with no live split give 0. */
void or_combine(float* out, const double* ml, const double* acc, int64_t rows, int n_splits,
                int hd) {
  for (int64_t r = 0; r < rows; ++r) {
    double M = -INFINITY;
    for (int s = 0; s < n_splits; ++s) {
      const double m = ml[2 * (r * n_splits + s)];
      if (m > M) M = m;
    }
    float* o = out + r * hd;
    if (M == -INFINITY) { for (int d = 0; d < hd; ++d) o[d] = 0.f; continue; }
    double L = 0.0;
    for (int s = 0; s < n_splits; ++s) {
      const double m = ml[2 * (r * n_splits + s)];
      if (m == -INFINITY) continue;
      L += exp(m - M) * ml[2 * (r * n_splits + s) + 1];
    }
    for (int d = 0; d < hd; ++d) {
      double x = 0.0;
      for (int s = 0; s < n_splits; ++s) {
        const double m = ml[2 * (r * n_splits + s)];
        if (m == -INFINITY) continue;
        x += exp(m - M) * acc[(r * n_splits + s) * hd + d];
      }
      o[d] = (float)(x / L);
    }
  }
}

/* ---- chunked prefill (bottom-right causal) ---- */

/* q: [n_tokens, nh, hd] (rows of all chunks back to back, strides q_st, q_sh);
 * chunk c owns query rows [cu_q[c], cu_q[c+1]) and its context is the first ctx_c
 * positions of sequence table row c (ctx_c >= q_c; its last q_c positions are the
 * chunk's own tokens). out: float32 [n_tokens, nh, hd] contiguous. */
int or_prefill_attention(float* out, const void* q, int64_t q_st, int64_t q_sh,
                         const void* k, const void* v, int dt, int64_t kv_ss, int64_t kv_sh,
                         const int32_t* tables, int64_t t_sb, const int32_t* cu_q,
                         const int32_t* ctx, int n_chunks, int nh, int nkv, int hd, int bs,
                         double scale, int threads) {
  dec_t a = {q, q_st, q_sh, k, v, dt, kv_ss, kv_sh, tables, t_sb, ctx, nh, nkv, hd, bs, scale};
  if (nkv <= 0 || nh % nkv || bs <= 0) return -1;
  const int mc = max_ctx(ctx, n_chunks);
  const int64_t total = cu_q[n_chunks];
  int err = 0;
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel
#endif
  {
    double* qv = (double*)malloc(sizeof(double) * hd);
    double* acc = (double*)malloc(sizeof(double) * hd);
    double* sc = (double*)malloc(sizeof(double) * (mc > 0 ? mc : 1));
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 4)
#endif
    for (int64_t w = 0; w < total * nh; ++w) {
      const int64_t t = w / nh;
      const int h = (int)(w % nh);
      int c = 0;
      while (cu_q[c + 1] <= t) ++c;
      const int qlen = cu_q[c + 1] - cu_q[c];
      const int i = (int)(t - cu_q[c]);
      if (ctx[c] < qlen) { err = -2; continue; }
      const int64_t last = (int64_t)ctx[c] - qlen + i; /* keys 0..last visible */
      /* q row t lives at t * q_st; partial() addresses q by (b, h) with q_sb. */
      dec_t at = a;
      at.q = (const char*)q + t * q_st * dt_size(dt);
      at.q_sb = 0;
      double m, l;
      partial(&at, c, h, 0, last + 1, qv, sc, &m, &l, acc);
      float* o = out + w * hd;
      for (int d = 0; d < hd; ++d) o[d] = (float)(acc[d] / l);
    }
    free(qv); free(acc); free(sc);
  }
  return err;
}

/* ---- array conversions (for checking Tensor.to() rounding) ---- */

void or_cvt_f32_to_bf16_n(const float* x, uint16_t* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = or_f32_to_bf16(x[i]);
}
void or_cvt_f32_to_f16_n(const float* x, uint16_t* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = or_f32_to_f16(x[i]);
}
void or_cvt_f16_to_f32_n(const uint16_t* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = or_f16_to_f32(x[i]);
}
void or_cvt_bf16_to_f32_n(const uint16_t* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = or_bf16_to_f32(x[i]);
}
