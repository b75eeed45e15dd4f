// Fused SwiGLU forward/backward for gfx950.
//
// Layout: the up-projection u is [rows, ld_u] (ld_u >= 2*width) with gate in
// columns [0, width) and value in [width, 2*width); o and dy are
// [rows, width]; du has u's layout.  The vector path moves 16 bytes per
// operand per thread (8 halves or 4 floats): for width = 1024 fp16 a row's
// gate half is 128 consecutive 16-byte loads, coalesced across the wave.
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

// Cache hints chosen by timing sweeps on MI355X at [14848, 1024] fp16 over
// > 1.5 GB of rotating buffers: streaming (nt) loads in both directions,
// streaming stores in the backward, plain stores in the forward.
constexpr bool kFwdNtStore = false;
constexpr bool kBwdNtStore = true;

// A grid with one thread per U 16-byte vectors of every operand (vector
// index blockIdx.x * 256 U + k * 256 + threadIdx.x, k < U), no loop; every
// load of a thread is issued before its first wait, and the sigmoid's
// transcendental work of one wave overlaps the loads of the others.  C2
// (same rotating-buffer timing as above): forward with U = 2 15.8 us and
// backward with U = 1 25.2 us, against 16.5 and 25.8 for a persistent
// grid-stride loop with the next vector's loads issued before the current
// one's math.
template <typename T, bool BWD, int U>
__global__ __launch_bounds__(kThreads)
void swiglu_once(const T* __restrict__ u, int64_t ld_u, const T* __restrict__ dy,
                 T* __restrict__ out, int64_t width, FastDiv vpr, uint32_t total) {
  using V = rv::Vec16<T>;
  constexpr int N = V::N;
  const uint32_t first = blockIdx.x * (uint32_t)(kThreads * U) + threadIdx.x;
  V g[U], v[U], d[BWD ? U : 1];
#pragma unroll
  for (int k = 0; k < U; ++k) {
    uint32_t i = first + k * kThreads;
    i = i < total ? i : total - 1;  // clamp: always a valid address
    const uint32_t row = fdiv(i, vpr);
    const int64_t c = (int64_t)(i - row * vpr.d) * N;
    const T* src = u + (int64_t)row * ld_u + c;
    g[k] = rv::load16<true>(src);
    v[k] = rv::load16<true>(src + width);
    if constexpr (BWD) d[k] = rv::load16<true>(dy + (int64_t)row * width + c);
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int k = 0; k < U; ++k) {
    const uint32_t i = first + k * kThreads;
    V a, b;
#pragma unroll
    for (int e = 0; e < N; ++e) {
      const float gf = rv::Conv<T>::to_f(g[k].v[e]);
      const float vf = rv::Conv<T>::to_f(v[k].v[e]);
      if constexpr (BWD) {
        const float df = rv::Conv<T>::to_f(d[k].v[e]);
        const float sg = rv::fast_sigmoid(gf);
        const float silu = rv::round_to<T>(gf * sg);
        const float dgi = rv::round_to<T>(df * vf);
        a.v[e] = rv::Conv<T>::from_f(dgi * (sg * (1.0f + gf * (1.0f - sg))));
        b.v[e] = rv::Conv<T>::from_f(df * silu);
      } else {
        const float silu = rv::round_to<T>(gf * rv::fast_sigmoid(gf));
        a.v[e] = rv::Conv<T>::from_f(silu * vf);
      }
    }
    if (i < total) {
      const uint32_t row = fdiv(i, vpr);
      const int64_t c = (int64_t)(i - row * vpr.d) * N;
      if constexpr (BWD) {
        T* dst = out + (int64_t)row * ld_u + c;
        rv::store16<kBwdNtStore>(dst, a);
        rv::store16<kBwdNtStore>(dst + width, b);
      } else {
        rv::store16<kFwdNtStore>(out + (int64_t)row * width + c, a);
      }
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

unsigned once_grid(uint32_t total, int vectors_per_thread) {
  const int64_t per_block = (int64_t)kThreads * vectors_per_thread;
  return (unsigned)(((int64_t)total + per_block - 1) / per_block);
}


template <typename T>
int launch_fwd(const T* u, int64_t ld_u, T* o, int64_t rows, int64_t width,
               hipStream_t s) {
  if (vec_ok<T>(u, o, nullptr, ld_u, rows, width)) {
    constexpr int N = 16 / sizeof(T);
    const uint32_t total = (uint32_t)(rows * (width / N));
    const FastDiv vpr = make_fastdiv((uint32_t)(width / N));
    constexpr int U = 2;
    hipLaunchKernelGGL((swiglu_once<T, false, U>), dim3(once_grid(total, U)), dim3(kThreads), 0,
                       s, u, ld_u, (const T*)nullptr, o, width, vpr, total);
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
    constexpr int U = 1;
    hipLaunchKernelGGL((swiglu_once<T, true, U>), dim3(once_grid(total, U)), dim3(kThreads), 0,
                       s, u, ld_u, dy, du, width, vpr, total);
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
