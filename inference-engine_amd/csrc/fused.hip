// fused.hip — gfx950 element-wise kernels beside the paged-KV path: the RMSNorm tail,
// in-place RoPE and SiLU-and-multiply, each one launch instead of PyTorch's chain of
// small kernels, 16 bytes per access where pointers, strides and widths allow (one
// element per thread otherwise). C ABI in include/paged_kv.h.
//
// Each kernel rounds exactly where the PyTorch ops it replaces round, so results are
// bitwise identical to them: every product and sum is one fp32 operation rounded to the
// tensor dtype at the points PyTorch rounds, exp and division are the device library's
// and IEEE (as in PyTorch's ROCm SiLU), and multiply-add contraction is off for the whole
// file (PyTorch's separate kernels round between the multiply and the add). RMSNorm
// takes its per-row scale rsqrt(mean(x^2) + eps) from the caller: the device library's
// rsqrtf and PyTorch's ROCm rsqrt can differ in the last fp32 bit.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "paged_kv.h"

#pragma clang fp contract(off)

namespace {

template <int DT> struct F;
template <> struct F<PKV_F32> {
  using S = float;
  __device__ static float up(S x) { return x; }
  __device__ static S down(float f) { return f; }
};
template <> struct F<PKV_F16> {
  using S = uint16_t;
  __device__ static float up(S x) { return (float)__builtin_bit_cast(_Float16, x); }
  // v_cvt_f16_f32, round to nearest even; the empty asm keeps f an fp32 value (no fused
  // multiply-and-convert, which would round once instead of twice).
  __device__ static S down(float f) {
    __asm__ volatile("" : "+v"(f));
    return __builtin_bit_cast(uint16_t, (_Float16)f);
  }
};
template <> struct F<PKV_BF16> {
  using S = uint16_t;
  __device__ static float up(S x) { return __uint_as_float(uint32_t(x) << 16); }
  // Round to nearest even on the upper half; NaN becomes 0x7FC0 (torch's float ->
  // bfloat16).
  __device__ static S down(float f) {
    if (f != f) return 0x7FC0;
    const uint32_t u = __float_as_uint(f);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
  }
};

// Value as it is after a cast to DT and back to fp32.
template <int DT> __device__ __forceinline__ float through(float f) {
  return F<DT>::up(F<DT>::down(f));
}

// 16 bytes of DT: VN<DT> elements (8 of a 16-bit type, 4 floats).
template <int DT> constexpr int VN = DT == PKV_F32 ? 4 : 8;
template <int DT> __device__ __forceinline__ void load16(const typename F<DT>::S* p, float* f) {
  const uint4 r = *reinterpret_cast<const uint4*>(p);
  const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if constexpr (DT == PKV_F32) {
      f[i] = __uint_as_float(w[i]);
    } else {
      f[2 * i] = F<DT>::up((uint16_t)(w[i] & 0xFFFFu));
      f[2 * i + 1] = F<DT>::up((uint16_t)(w[i] >> 16));
    }
  }
}
template <int DT> __device__ __forceinline__ void store16(typename F<DT>::S* p, const float* f) {
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if constexpr (DT == PKV_F32)
      w[i] = __float_as_uint(f[i]);
    else
      w[i] = (uint32_t)F<DT>::down(f[2 * i]) | ((uint32_t)F<DT>::down(f[2 * i + 1]) << 16);
  }
  *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
}
// n fp32 values (n a multiple of 4) from a 16-byte aligned address.
template <int N> __device__ __forceinline__ void load_f32(const float* p, float* f) {
#pragma unroll
  for (int i = 0; i < N; i += 4) {
    const float4 v = *reinterpret_cast<const float4*>(p + i);
    f[i] = v.x, f[i + 1] = v.y, f[i + 2] = v.z, f[i + 3] = v.w;
  }
}

// out[r, c] = DO( f32(w[c]) * f32(DX( f32(x[r, c]) * inv[r] )) ): PyTorch's
// w * (x.float() * inv).to(x.dtype), inv = torch.rsqrt(mean(x.float()^2) + eps) per row.
template <int DX, int DW, int DO>
__global__ void __launch_bounds__(256)
rms_norm_tail_kernel(typename F<DO>::S* __restrict__ out, int64_t so,
                     const typename F<DX>::S* __restrict__ x, int64_t sx,
                     const float* __restrict__ inv_rms, const typename F<DW>::S* __restrict__ w,
                     int64_t rows, int cols) {
  for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
    const float inv = inv_rms[r];
    for (int c = blockIdx.x * blockDim.x + threadIdx.x; c < cols; c += gridDim.x * blockDim.x) {
      const float normed = through<DX>(F<DX>::up(x[r * sx + c]) * inv);
      out[r * so + c] = F<DO>::down(F<DW>::up(w[c]) * normed);
    }
  }
}

// In place, x [n, heads, hd]: x = x * cos + rotate_half(x) * sin, rotate_half(x) =
// cat(-x2, x1), with cos / sin (fp32 [n, hd]) cast to the dtype first and every product
// and the sum rounded to it (HF's apply_rotary_pos_emb in the model dtype).
template <int DT>
__global__ void __launch_bounds__(256)
rope_kernel(typename F<DT>::S* __restrict__ x, int64_t sn, int64_t sh,
            const float* __restrict__ cs, const float* __restrict__ sn_, int64_t sc,
            int64_t n, int heads, int half) {
  const int64_t total = n * heads * half;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int d = (int)(i % half);
    const int64_t nh = i / half;
    const int h = (int)(nh % heads);
    const int64_t t = nh / heads;
    typename F<DT>::S* p = x + t * sn + h * sh;
    const float x1 = F<DT>::up(p[d]), x2 = F<DT>::up(p[d + half]);
    const float* c = cs + t * sc;
    const float* s = sn_ + t * sc;
    const float c1 = through<DT>(c[d]), c2 = through<DT>(c[d + half]);
    const float s1 = through<DT>(s[d]), s2 = through<DT>(s[d + half]);
    const float o1 = through<DT>(x1 * c1) + through<DT>(-x2 * s1);
    const float o2 = through<DT>(x2 * c2) + through<DT>(x1 * s2);
    p[d] = F<DT>::down(o1);
    p[d + half] = F<DT>::down(o2);
  }
}

// out = DT( f32(DT( g / (1 + exp(-g)) )) * u ): PyTorch's F.silu(gate) * up (SiLU in
// fp32 with the library exp and IEEE division, rounded, then the rounded product).
template <int DT>
__global__ void __launch_bounds__(256)
silu_mul_kernel(typename F<DT>::S* __restrict__ out, const typename F<DT>::S* __restrict__ g,
                const typename F<DT>::S* __restrict__ u, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const float gf = F<DT>::up(g[i]);
    const float silu = through<DT>(gf / (1.0f + expf(-gf)));
    out[i] = F<DT>::down(silu * F<DT>::up(u[i]));
  }
}

// The same three operations, 16 bytes per access (x, weight and output of one dtype for
// the RMSNorm tail; the launchers take these when pointers, strides and widths allow).
// Each element goes through exactly the scalar kernels' operations.
template <int DT>
__global__ void __launch_bounds__(256)
rms_norm_tail_vec_kernel(typename F<DT>::S* __restrict__ out, int64_t so,
                         const typename F<DT>::S* __restrict__ x, int64_t sx,
                         const float* __restrict__ inv_rms,
                         const typename F<DT>::S* __restrict__ w, int64_t rows, int cvec) {
  constexpr int V = VN<DT>;
  for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
    const float inv = inv_rms[r];
    for (int c = blockIdx.x * blockDim.x + threadIdx.x; c < cvec; c += gridDim.x * blockDim.x) {
      float xf[V], wf[V], o[V];
      load16<DT>(x + r * sx + (int64_t)c * V, xf);
      load16<DT>(w + (int64_t)c * V, wf);
#pragma unroll
      for (int j = 0; j < V; ++j) o[j] = wf[j] * through<DT>(xf[j] * inv);
      store16<DT>(out + r * so + (int64_t)c * V, o);
    }
  }
}

template <int DT>
__global__ void __launch_bounds__(256)
rope_vec_kernel(typename F<DT>::S* __restrict__ x, int64_t sn, int64_t sh,
                const float* __restrict__ cs, const float* __restrict__ sn_, int64_t sc,
                int64_t n, int heads, int half) {
  constexpr int V = VN<DT>;
  const int hv = half / V;
  const int64_t total = n * heads * hv;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int d = (int)(i % hv) * V;
    const int64_t nh = i / hv;
    const int h = (int)(nh % heads);
    const int64_t t = nh / heads;
    typename F<DT>::S* p = x + t * sn + h * sh;
    float x1[V], x2[V], c1[V], c2[V], s1[V], s2[V], o1[V], o2[V];
    load16<DT>(p + d, x1);
    load16<DT>(p + d + half, x2);
    load_f32<V>(cs + t * sc + d, c1);
    load_f32<V>(cs + t * sc + d + half, c2);
    load_f32<V>(sn_ + t * sc + d, s1);
    load_f32<V>(sn_ + t * sc + d + half, s2);
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const float cc1 = through<DT>(c1[j]), cc2 = through<DT>(c2[j]);
      const float ss1 = through<DT>(s1[j]), ss2 = through<DT>(s2[j]);
      o1[j] = through<DT>(x1[j] * cc1) + through<DT>(-x2[j] * ss1);
      o2[j] = through<DT>(x2[j] * cc2) + through<DT>(x1[j] * ss2);
    }
    store16<DT>(p + d, o1);
    store16<DT>(p + d + half, o2);
  }
}

template <int DT>
__global__ void __launch_bounds__(256)
silu_mul_vec_kernel(typename F<DT>::S* __restrict__ out, const typename F<DT>::S* __restrict__ g,
                    const typename F<DT>::S* __restrict__ u, int64_t nvec) {
  constexpr int V = VN<DT>;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nvec;
       i += (int64_t)gridDim.x * blockDim.x) {
    float gf[V], uf[V], o[V];
    load16<DT>(g + i * V, gf);
    load16<DT>(u + i * V, uf);
#pragma unroll
    for (int j = 0; j < V; ++j) o[j] = through<DT>(gf[j] / (1.0f + expf(-gf[j]))) * uf[j];
    store16<DT>(out + i * V, o);
  }
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

bool valid(int dt) { return dt == PKV_F32 || dt == PKV_F16 || dt == PKV_BF16; }

// The dtype PyTorch promotes x (DX) and w (DW) to: equal dtypes stay, every mixed pair
// of the three floating types promotes to fp32.
int promoted(int dx, int dw) { return dx == dw ? dx : PKV_F32; }

unsigned blocks_for(int64_t n) {
  int64_t b = (n + 255) / 256;
  return (unsigned)(b < 1 ? 1 : (b > 8192 ? 8192 : b));
}

template <int DX, int DW>
hipError_t launch_rms(void* out, int64_t so, const void* x, int64_t sx, const float* inv,
                      const void* w, int64_t rows, int cols, hipStream_t st) {
  constexpr int DO = DX == DW ? DX : PKV_F32;
  const unsigned gy = (unsigned)(rows < 65535 ? rows : 65535);
  if constexpr (DX == DW) {
    constexpr int V = VN<DX>;
    if (cols % V == 0 && sx % V == 0 && so % V == 0 && aligned16(out) && aligned16(x) &&
        aligned16(w)) {
      const int cvec = cols / V;
      hipLaunchKernelGGL((rms_norm_tail_vec_kernel<DX>), dim3((unsigned)((cvec + 255) / 256), gy),
                         dim3(256), 0, st, (typename F<DX>::S*)out, so,
                         (const typename F<DX>::S*)x, sx, inv, (const typename F<DX>::S*)w, rows,
                         cvec);
      return hipGetLastError();
    }
  }
  const unsigned gx = (unsigned)((cols + 255) / 256);
  hipLaunchKernelGGL((rms_norm_tail_kernel<DX, DW, DO>), dim3(gx, gy), dim3(256), 0, st,
                     (typename F<DO>::S*)out, so, (const typename F<DX>::S*)x, sx, inv,
                     (const typename F<DW>::S*)w, rows, cols);
  return hipGetLastError();
}

template <int DX>
hipError_t rms_by_w(int dw, void* out, int64_t so, const void* x, int64_t sx, const float* inv,
                    const void* w, int64_t rows, int cols, hipStream_t st) {
  switch (dw) {
    case PKV_F32: return launch_rms<DX, PKV_F32>(out, so, x, sx, inv, w, rows, cols, st);
    case PKV_F16: return launch_rms<DX, PKV_F16>(out, so, x, sx, inv, w, rows, cols, st);
    default: return launch_rms<DX, PKV_BF16>(out, so, x, sx, inv, w, rows, cols, st);
  }
}

}  // namespace

extern "C" {

int pkv_rms_norm(void* out, int out_dtype, int64_t out_stride_row, const void* x, int x_dtype,
                 int64_t x_stride_row, const float* inv_rms, const void* weight, int w_dtype,
                 int64_t rows, int64_t cols, void* stream) {
  if (!valid(x_dtype) || !valid(w_dtype) || out_dtype != promoted(x_dtype, w_dtype))
    return PKV_E_DTYPE;
  if (rows < 0 || cols < 0 || cols > (1 << 30)) return PKV_E_SHAPE;
  if (rows == 0 || cols == 0) return 0;
  if (!out || !x || !inv_rms || !weight) return PKV_E_NULL;
  hipStream_t st = (hipStream_t)stream;
  const int c = (int)cols;
  switch (x_dtype) {
    case PKV_F32:
      return (int)rms_by_w<PKV_F32>(w_dtype, out, out_stride_row, x, x_stride_row, inv_rms,
                                    weight, rows, c, st);
    case PKV_F16:
      return (int)rms_by_w<PKV_F16>(w_dtype, out, out_stride_row, x, x_stride_row, inv_rms,
                                    weight, rows, c, st);
    default:
      return (int)rms_by_w<PKV_BF16>(w_dtype, out, out_stride_row, x, x_stride_row, inv_rms,
                                     weight, rows, c, st);
  }
}

int pkv_rope(void* x, int dtype, int64_t stride_tok, int64_t stride_head, const float* cos,
             const float* sin, int64_t cs_stride_tok, int64_t n_tokens, int32_t heads,
             int32_t head_dim, void* stream) {
  if (!valid(dtype)) return PKV_E_DTYPE;
  if (n_tokens < 0 || heads < 0 || head_dim < 0 || head_dim % 2) return PKV_E_SHAPE;
  if (n_tokens == 0 || heads == 0 || head_dim == 0) return 0;
  if (!x || !cos || !sin) return PKV_E_NULL;
  hipStream_t st = (hipStream_t)stream;
  const int half = head_dim / 2;
  const int v = dtype == PKV_F32 ? 4 : 8;  // elements per 16-byte access
  if (half % v == 0 && stride_tok % v == 0 && stride_head % v == 0 && cs_stride_tok % 4 == 0 &&
      aligned16(x) && aligned16(cos) && aligned16(sin)) {
    const unsigned nbv = blocks_for(n_tokens * heads * (half / v));
    switch (dtype) {
      case PKV_F32:
        hipLaunchKernelGGL(rope_vec_kernel<PKV_F32>, dim3(nbv), dim3(256), 0, st, (float*)x,
                           stride_tok, stride_head, cos, sin, cs_stride_tok, n_tokens, heads, half);
        break;
      case PKV_F16:
        hipLaunchKernelGGL(rope_vec_kernel<PKV_F16>, dim3(nbv), dim3(256), 0, st, (uint16_t*)x,
                           stride_tok, stride_head, cos, sin, cs_stride_tok, n_tokens, heads, half);
        break;
      default:
        hipLaunchKernelGGL(rope_vec_kernel<PKV_BF16>, dim3(nbv), dim3(256), 0, st, (uint16_t*)x,
                           stride_tok, stride_head, cos, sin, cs_stride_tok, n_tokens, heads, half);
    }
    return (int)hipGetLastError();
  }
  const unsigned nb = blocks_for(n_tokens * heads * half);
  switch (dtype) {
    case PKV_F32:
      hipLaunchKernelGGL(rope_kernel<PKV_F32>, dim3(nb), dim3(256), 0, st, (float*)x,
                         stride_tok, stride_head, cos, sin, cs_stride_tok, n_tokens, heads, half);
      break;
    case PKV_F16:
      hipLaunchKernelGGL(rope_kernel<PKV_F16>, dim3(nb), dim3(256), 0, st, (uint16_t*)x,
                         stride_tok, stride_head, cos, sin, cs_stride_tok, n_tokens, heads, half);
      break;
    default:
      hipLaunchKernelGGL(rope_kernel<PKV_BF16>, dim3(nb), dim3(256), 0, st, (uint16_t*)x,
                         stride_tok, stride_head, cos, sin, cs_stride_tok, n_tokens, heads, half);
  }
  return (int)hipGetLastError();
}

int pkv_silu_mul(void* out, const void* gate, const void* up, int dtype, int64_t n,
                 void* stream) {
  if (!valid(dtype)) return PKV_E_DTYPE;
  if (n < 0) return PKV_E_SHAPE;
  if (n == 0) return 0;
  if (!out || !gate || !up) return PKV_E_NULL;
  hipStream_t st = (hipStream_t)stream;
  const int v = dtype == PKV_F32 ? 4 : 8;  // elements per 16-byte access
  if (n % v == 0 && aligned16(out) && aligned16(gate) && aligned16(up)) {
    const unsigned nbv = blocks_for(n / v);
    switch (dtype) {
      case PKV_F32:
        hipLaunchKernelGGL(silu_mul_vec_kernel<PKV_F32>, dim3(nbv), dim3(256), 0, st,
                           (float*)out, (const float*)gate, (const float*)up, n / v);
        break;
      case PKV_F16:
        hipLaunchKernelGGL(silu_mul_vec_kernel<PKV_F16>, dim3(nbv), dim3(256), 0, st,
                           (uint16_t*)out, (const uint16_t*)gate, (const uint16_t*)up, n / v);
        break;
      default:
        hipLaunchKernelGGL(silu_mul_vec_kernel<PKV_BF16>, dim3(nbv), dim3(256), 0, st,
                           (uint16_t*)out, (const uint16_t*)gate, (const uint16_t*)up, n / v);
    }
    return (int)hipGetLastError();
  }
  const unsigned nb = blocks_for(n);
  switch (dtype) {
    case PKV_F32:
      hipLaunchKernelGGL(silu_mul_kernel<PKV_F32>, dim3(nb), dim3(256), 0, st, (float*)out,
                         (const float*)gate, (const float*)up, n);
      break;
    case PKV_F16:
      hipLaunchKernelGGL(silu_mul_kernel<PKV_F16>, dim3(nb), dim3(256), 0, st,
                         (uint16_t*)out, (const uint16_t*)gate, (const uint16_t*)up, n);
      break;
    default:
      hipLaunchKernelGGL(silu_mul_kernel<PKV_BF16>, dim3(nb), dim3(256), 0, st,
                         (uint16_t*)out, (const uint16_t*)gate, (const uint16_t*)up, n);
  }
  return (int)hipGetLastError();
}

}  // extern "C"
