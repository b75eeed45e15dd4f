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

// Launch shapes and cache hints chosen by timing sweeps on MI355X at
// [14848, 1024] fp16 over > 1.5 GB of rotating buffers: one 16-byte vector
// per operand per thread per iteration; forward 4 blocks per CU with
// streaming loads, backward 2 blocks per CU with streaming loads and stores.
#ifndef RV_SWIGLU_VPT
#define RV_SWIGLU_VPT 1
#endif
#ifndef RV_SWIGLU_FWD_BLOCKS_PER_CU
#define RV_SWIGLU_FWD_BLOCKS_PER_CU 4
#endif
#ifndef RV_SWIGLU_BWD_BLOCKS_PER_CU
#define RV_SWIGLU_BWD_BLOCKS_PER_CU 2
#endif
constexpr int kVpt = RV_SWIGLU_VPT;
constexpr bool kFwdNtStore = false;
constexpr bool kBwdNtStore = true;

// Persistent, software-pipelined streaming: each block walks the vector index
// space with a grid-sized stride, alternating between two register tiles.
// The loads of the next tile are issued before the math of the current one,
// so the sigmoid's transcendental work (two quarter-rate ops per element)
// overlaps HBM latency instead of alternating with it.  Prefetches are
// unconditional: an index past the end is clamped to the last vector, so
// those loads all hit one cached line, and no branch forces the compiler to
// drain the load queue (s_waitcnt vmcnt(0)) inside the loop.
template <typename T>
struct SwiGLUTile {
  using V = rv::Vec16<T>;
  V g[kVpt], v[kVpt], d[kVpt];
};

template <typename T, bool BWD>
__device__ __forceinline__ void swiglu_load(SwiGLUTile<T>& t, const T* __restrict__ u,
                                            int64_t ld_u, const T* __restrict__ dy,
                                            int64_t width, const FastDiv& vpr,
                                            uint32_t first, uint32_t total) {
  constexpr int N = rv::Vec16<T>::N;
#pragma unroll
  for (int k = 0; k < kVpt; ++k) {
    uint32_t i = first + k * kThreads;
    i = i < total ? i : total - 1;  // clamp: always a valid address
    const uint32_t row = fdiv(i, vpr);
    const int64_t c = (int64_t)(i - row * vpr.d) * N;
    const T* src = u + (int64_t)row * ld_u + c;
    t.g[k] = rv::load16<true>(src);
    t.v[k] = rv::load16<true>(src + width);
    if constexpr (BWD) t.d[k] = rv::load16<true>(dy + (int64_t)row * width + c);
  }
}

template <typename T>
__device__ __forceinline__ void swiglu_fwd_compute(const SwiGLUTile<T>& t, T* __restrict__ o,
                                                   int64_t width, const FastDiv& vpr,
                                                   uint32_t first, uint32_t total) {
  using V = rv::Vec16<T>;
  constexpr int N = V::N;
#pragma unroll
  for (int k = 0; k < kVpt; ++k) {
    const uint32_t i = first + k * kThreads;
    V out;
#pragma unroll
    for (int e = 0; e < N; ++e) {
      const float gf = rv::Conv<T>::to_f(t.g[k].v[e]);
      const float silu = rv::round_to<T>(gf * rv::fast_sigmoid(gf));
      out.v[e] = rv::Conv<T>::from_f(silu * rv::Conv<T>::to_f(t.v[k].v[e]));
    }
    if (i < total) {
      const uint32_t row = fdiv(i, vpr);
      const int64_t c = (int64_t)(i - row * vpr.d) * N;
      rv::store16<kFwdNtStore>(o + (int64_t)row * width + c, out);
    }
  }
}

template <typename T>
__device__ __forceinline__ void swiglu_bwd_compute(const SwiGLUTile<T>& t, T* __restrict__ du,
                                                   int64_t ld_u, int64_t width,
                                                   const FastDiv& vpr, uint32_t first,
                                                   uint32_t total) {
  using V = rv::Vec16<T>;
  constexpr int N = V::N;
#pragma unroll
  for (int k = 0; k < kVpt; ++k) {
    const uint32_t i = first + k * kThreads;
    V dg, dv;
#pragma unroll
    for (int e = 0; e < N; ++e) {
      const float gf = rv::Conv<T>::to_f(t.g[k].v[e]);
      const float vf = rv::Conv<T>::to_f(t.v[k].v[e]);
      const float df = rv::Conv<T>::to_f(t.d[k].v[e]);
      const float s = rv::fast_sigmoid(gf);
      const float silu = rv::round_to<T>(gf * s);
      const float dgi = rv::round_to<T>(df * vf);
      dg.v[e] = rv::Conv<T>::from_f(dgi * (s * (1.0f + gf * (1.0f - s))));
      dv.v[e] = rv::Conv<T>::from_f(df * silu);
    }
    if (i < total) {
      const uint32_t row = fdiv(i, vpr);
      const int64_t c = (int64_t)(i - row * vpr.d) * N;
      T* dst = du + (int64_t)row * ld_u + c;
      rv::store16<kBwdNtStore>(dst, dg);
      rv::store16<kBwdNtStore>(dst + width, dv);
    }
  }
}

template <typename T, bool BWD>
__device__ __forceinline__ void swiglu_compute(const SwiGLUTile<T>& t, T* __restrict__ out,
                                               int64_t ld_u, int64_t width, const FastDiv& vpr,
                                               uint32_t first, uint32_t total) {
  if constexpr (BWD)
    swiglu_bwd_compute<T>(t, out, ld_u, width, vpr, first, total);
  else
    swiglu_fwd_compute<T>(t, out, width, vpr, first, total);
}

template <typename T, bool BWD>
__global__ __launch_bounds__(kThreads)
void swiglu_stream(const T* __restrict__ u, int64_t ld_u, const T* __restrict__ dy,
                   T* __restrict__ out, int64_t width, FastDiv vpr, uint32_t total) {
  const uint32_t step = gridDim.x * (uint32_t)(kThreads * kVpt);
  const uint32_t block_first = blockIdx.x * (uint32_t)(kThreads * kVpt);
  if (block_first >= total) return;  // block-uniform
  // iterations of this block: block_first + k*step < total
  const uint32_t iters = (total - 1 - block_first) / step + 1;
  uint32_t first = block_first + threadIdx.x;
  SwiGLUTile<T> a, b;
  swiglu_load<T, BWD>(a, u, ld_u, dy, width, vpr, first, total);
  for (uint32_t k = 0; k < iters; k += 2) {
    swiglu_load<T, BWD>(b, u, ld_u, dy, width, vpr, first + step, total);
    swiglu_compute<T, BWD>(a, out, ld_u, width, vpr, first, total);
    if (k + 1 >= iters) break;
    first += step;
    swiglu_load<T, BWD>(a, u, ld_u, dy, width, vpr, first + step, total);
    swiglu_compute<T, BWD>(b, out, ld_u, width, vpr, first, total);
    first += step;
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

unsigned stream_grid(uint32_t total, int blocks_per_cu) {
  const int64_t tiles = ((int64_t)total + kThreads * kVpt - 1) / (kThreads * kVpt);
  const int64_t cap = (int64_t)rv_host::cu_count() * blocks_per_cu;
  return (unsigned)(tiles < cap ? tiles : cap);
}

template <typename T>
int launch_fwd(const T* u, int64_t ld_u, T* o, int64_t rows, int64_t width,
               hipStream_t s) {
  if (vec_ok<T>(u, o, nullptr, ld_u, rows, width)) {
    constexpr int N = 16 / sizeof(T);
    const uint32_t total = (uint32_t)(rows * (width / N));
    const FastDiv vpr = make_fastdiv((uint32_t)(width / N));
    hipLaunchKernelGGL((swiglu_stream<T, false>),
                       dim3(stream_grid(total, RV_SWIGLU_FWD_BLOCKS_PER_CU)), dim3(kThreads),
                       0, s, u, ld_u, (const T*)nullptr, o, width, vpr, total);
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
    hipLaunchKernelGGL((swiglu_stream<T, true>),
                       dim3(stream_grid(total, RV_SWIGLU_BWD_BLOCKS_PER_CU)), dim3(kThreads),
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
