// Fused SwiGLU forward/backward for gfx950.
//
// Layout: the up-projection u is [rows, ld_u] (ld_u >= 2*width) with gate in
// columns [0, width) and value in [width, 2*width); o and dy are
// [rows, width]; du has u's layout.  The vector path moves 16 bytes per
// operand per thread (8 halves or 4 floats): for width = 1024 fp16 a row's
// gate half is 128 consecutive 16-byte loads, coalesced across the wave.
// Each thread handles UNROLL vectors, all loads issued before any math.
//
// Arithmetic follows src/reversibility/kernels.py:88-110: FP32 math, silu
// rounded to the I/O dtype before the multiply, dy*value rounded to the I/O
// dtype before the sigmoid-derivative product.  The sigmoid uses the hardware
// exp2/reciprocal instructions (v_exp_f32, v_rcp_f32); the reference's Triton
// kernels likewise use approximate exp and division.

#include "rv_device.h"

namespace {

// Division by a run-time invariant divisor d > 0 for n < 2^32, after
// Granlund & Montgomery, "Division by Invariant Integers using
// Multiplication" (PLDI 1994), Fig. 4.1: l = ceil(log2 d),
// m = floor(2^32 (2^l - d) / d) + 1, q = (mulhi(m, n) + n) >> l.
struct FastDiv {
  uint32_t d, m, l;
};

FastDiv make_fastdiv(uint32_t d) {
  FastDiv f;
  f.d = d;
  uint32_t l = 0;
  while ((uint64_t(1) << l) < d) ++l;
  f.l = l;
  f.m = (uint32_t)((((uint64_t(1) << l) - d) << 32) / d + 1);
  return f;
}

__device__ __forceinline__ uint32_t fdiv(uint32_t n, const FastDiv& f) {
  return (uint32_t)(((uint64_t)__umulhi(n, f.m) + n) >> f.l);
}

constexpr int kThreads = 256;

template <typename T, int UNROLL>
__global__ __launch_bounds__(kThreads)
void swiglu_fwd_vec(const T* __restrict__ u, int64_t ld_u, T* __restrict__ o,
                    int64_t width, FastDiv vpr, uint32_t total) {
  using V = rv::Vec16<T>;
  constexpr int N = V::N;
  const uint32_t i0 = blockIdx.x * (uint32_t)(kThreads * UNROLL) + threadIdx.x;
  V g[UNROLL], v[UNROLL];
  int64_t orow[UNROLL];
#pragma unroll
  for (int k = 0; k < UNROLL; ++k) {
    const uint32_t i = i0 + k * kThreads;
    if (i < total) {
      const uint32_t row = fdiv(i, vpr);
      const int64_t c = (int64_t)(i - row * vpr.d) * N;
      const T* src = u + (int64_t)row * ld_u + c;
      g[k] = rv::load16(src);
      v[k] = rv::load16(src + width);
      orow[k] = (int64_t)row * width + c;
    }
  }
#pragma unroll
  for (int k = 0; k < UNROLL; ++k) {
    const uint32_t i = i0 + k * kThreads;
    if (i < total) {
      V out;
#pragma unroll
      for (int e = 0; e < N; ++e) {
        const float gf = rv::Conv<T>::to_f(g[k].v[e]);
        const float silu = rv::round_to<T>(gf * rv::fast_sigmoid(gf));
        out.v[e] = rv::Conv<T>::from_f(silu * rv::Conv<T>::to_f(v[k].v[e]));
      }
      rv::store16(o + orow[k], out);
    }
  }
}

template <typename T, int UNROLL>
__global__ __launch_bounds__(kThreads)
void swiglu_bwd_vec(const T* __restrict__ u, int64_t ld_u,
                    const T* __restrict__ dy, T* __restrict__ du,
                    int64_t width, FastDiv vpr, uint32_t total) {
  using V = rv::Vec16<T>;
  constexpr int N = V::N;
  const uint32_t i0 = blockIdx.x * (uint32_t)(kThreads * UNROLL) + threadIdx.x;
  V g[UNROLL], v[UNROLL], d[UNROLL];
  int64_t urow[UNROLL];
#pragma unroll
  for (int k = 0; k < UNROLL; ++k) {
    const uint32_t i = i0 + k * kThreads;
    if (i < total) {
      const uint32_t row = fdiv(i, vpr);
      const int64_t c = (int64_t)(i - row * vpr.d) * N;
      const T* src = u + (int64_t)row * ld_u + c;
      g[k] = rv::load16(src);
      v[k] = rv::load16(src + width);
      d[k] = rv::load16(dy + (int64_t)row * width + c);
      urow[k] = (int64_t)row * ld_u + c;
    }
  }
#pragma unroll
  for (int k = 0; k < UNROLL; ++k) {
    const uint32_t i = i0 + k * kThreads;
    if (i < total) {
      V dg, dv;
#pragma unroll
      for (int e = 0; e < N; ++e) {
        const float gf = rv::Conv<T>::to_f(g[k].v[e]);
        const float vf = rv::Conv<T>::to_f(v[k].v[e]);
        const float df = rv::Conv<T>::to_f(d[k].v[e]);
        const float s = rv::fast_sigmoid(gf);
        const float silu = rv::round_to<T>(gf * s);
        const float dgi = rv::round_to<T>(df * vf);
        dg.v[e] = rv::Conv<T>::from_f(dgi * (s * (1.0f + gf * (1.0f - s))));
        dv.v[e] = rv::Conv<T>::from_f(df * silu);
      }
      rv::store16(du + urow[k], dg);
      rv::store16(du + urow[k] + width, dv);
    }
  }
}

// Scalar fallbacks: any width / leading dimension / alignment.
template <typename T>
__global__ __launch_bounds__(kThreads)
void swiglu_fwd_scalar(const T* __restrict__ u, int64_t ld_u,
                       T* __restrict__ o, int64_t rows, int64_t width) {
  const int64_t n = rows * width;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kThreads) {
    const int64_t row = i / width, c = i - row * width;
    const float gf = rv::Conv<T>::to_f(u[row * ld_u + c]);
    const float vf = rv::Conv<T>::to_f(u[row * ld_u + width + c]);
    const float silu = rv::round_to<T>(gf * rv::fast_sigmoid(gf));
    o[i] = rv::Conv<T>::from_f(silu * vf);
  }
}

template <typename T>
__global__ __launch_bounds__(kThreads)
void swiglu_bwd_scalar(const T* __restrict__ u, int64_t ld_u,
                       const T* __restrict__ dy, T* __restrict__ du,
                       int64_t rows, int64_t width) {
  const int64_t n = rows * width;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kThreads) {
    const int64_t row = i / width, c = i - row * width;
    const float gf = rv::Conv<T>::to_f(u[row * ld_u + c]);
    const float vf = rv::Conv<T>::to_f(u[row * ld_u + width + c]);
    const float df = rv::Conv<T>::to_f(dy[i]);
    const float s = rv::fast_sigmoid(gf);
    const float silu = rv::round_to<T>(gf * s);
    const float dgi = rv::round_to<T>(df * vf);
    du[row * ld_u + c] =
        rv::Conv<T>::from_f(dgi * (s * (1.0f + gf * (1.0f - s))));
    du[row * ld_u + width + c] = rv::Conv<T>::from_f(df * silu);
  }
}

constexpr int kUnroll = 2;

template <typename T>
bool vec_ok(const void* a, const void* b, const void* c, int64_t ld_u,
            int64_t rows, int64_t width) {
  constexpr int N = 16 / sizeof(T);
  return width % N == 0 && ld_u % N == 0 && rv_host::aligned16(a) &&
         rv_host::aligned16(b) && (c == nullptr || rv_host::aligned16(c)) &&
         rows * (width / N) < (int64_t(1) << 31);
}

unsigned scalar_grid(int64_t n) {
  int64_t blocks = (n + kThreads - 1) / kThreads;
  const int64_t cap = (int64_t)rv_host::cu_count() * 64;
  return (unsigned)(blocks < cap ? blocks : cap);
}

template <typename T>
int launch_fwd(const T* u, int64_t ld_u, T* o, int64_t rows, int64_t width,
               hipStream_t s) {
  if (vec_ok<T>(u, o, nullptr, ld_u, rows, width)) {
    constexpr int N = 16 / sizeof(T);
    const uint32_t total = (uint32_t)(rows * (width / N));
    const FastDiv vpr = make_fastdiv((uint32_t)(width / N));
    const unsigned grid = (total + kThreads * kUnroll - 1) / (kThreads * kUnroll);
    hipLaunchKernelGGL((swiglu_fwd_vec<T, kUnroll>), dim3(grid), dim3(kThreads),
                       0, s, u, ld_u, o, width, vpr, total);
  } else {
    hipLaunchKernelGGL((swiglu_fwd_scalar<T>), dim3(scalar_grid(rows * width)),
                       dim3(kThreads), 0, s, u, ld_u, o, rows, width);
  }
  return rv_host::check_launch();
}

template <typename T>
int launch_bwd(const T* u, int64_t ld_u, const T* dy, T* du, int64_t rows,
               int64_t width, hipStream_t s) {
  if (vec_ok<T>(u, du, dy, ld_u, rows, width)) {
    constexpr int N = 16 / sizeof(T);
    const uint32_t total = (uint32_t)(rows * (width / N));
    const FastDiv vpr = make_fastdiv((uint32_t)(width / N));
    const unsigned grid = (total + kThreads * kUnroll - 1) / (kThreads * kUnroll);
    hipLaunchKernelGGL((swiglu_bwd_vec<T, kUnroll>), dim3(grid), dim3(kThreads),
                       0, s, u, ld_u, dy, du, width, vpr, total);
  } else {
    hipLaunchKernelGGL((swiglu_bwd_scalar<T>), dim3(scalar_grid(rows * width)),
                       dim3(kThreads), 0, s, u, ld_u, dy, du, rows, width);
  }
  return rv_host::check_launch();
}

}  // namespace

extern "C" {

int rv_swiglu_fwd(const void* u, int64_t ld_u, void* o, int64_t rows,
                  int64_t width, int dtype, void* stream) {
  if (!u || !o) return RV_ERR_NULL_POINTER;
  if (rows <= 0 || width <= 0 || ld_u < 2 * width) return RV_ERR_BAD_SIZE;
  const hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case RV_F16:
      return launch_fwd<__half>((const __half*)u, ld_u, (__half*)o, rows, width, s);
    case RV_F32:
      return launch_fwd<float>((const float*)u, ld_u, (float*)o, rows, width, s);
    default:
      return RV_ERR_UNSUPPORTED;
  }
}

int rv_swiglu_bwd(const void* u, int64_t ld_u, const void* dy, void* du,
                  int64_t rows, int64_t width, int dtype, void* stream) {
  if (!u || !dy || !du) return RV_ERR_NULL_POINTER;
  if (rows <= 0 || width <= 0 || ld_u < 2 * width) return RV_ERR_BAD_SIZE;
  const hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case RV_F16:
      return launch_bwd<__half>((const __half*)u, ld_u, (const __half*)dy,
                                (__half*)du, rows, width, s);
    case RV_F32:
      return launch_bwd<float>((const float*)u, ld_u, (const float*)dy,
                               (float*)du, rows, width, s);
    default:
      return RV_ERR_UNSUPPORTED;
  }
}

}  // extern "C"
