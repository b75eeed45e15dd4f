// Fused reversible residual updates for gfx950.
//
// Midpoint (paper Eq. 2.4/2.5; src/reversibility/reversible.py:16-32):
//   forward_pair:  next_q = p + 2h * (A(q) + M(q + A(q)))
//   inverse_pair:  prev_p = q - 2h * (A(p) + M(p + A(p)))
// Under fp16 autocast the reference evaluates this in three eager kernels
// with rounding points  f = fp16(a + m),  c = fp16(f * 2h),  out = p +/- float(c).
// One kernel here reads p (state dtype), a and m (force dtype) once and
// writes out, with the same rounding points, so results are bit-identical to
// the eager expression.
//
// Hamiltonian-Euler (Eq. 2.8/2.9; reversible.py:24-25, 31-32):
//   out = x +/- f, with f widened to the state dtype.
//
// Each thread moves groups of 4 consecutive elements (16-byte FP32 state,
// 8-byte FP16 force), grid-stride; a scalar tail covers n % 4 (and the whole
// range when a pointer is not aligned to a 4-element group).

#include "rv_device.h"

namespace {

template <typename T> struct Compute { using type = float; };
template <> struct Compute<double> { using type = double; };

template <typename T> __device__ __forceinline__ typename Compute<T>::type widen(T v) {
  return rv::Conv<T>::to_f(v);
}
template <> __device__ __forceinline__ double widen<double>(double v) { return v; }

template <typename T> __device__ __forceinline__ T narrow(typename Compute<T>::type v) {
  return rv::Conv<T>::from_f(v);
}
template <> __device__ __forceinline__ double narrow<double>(double v) { return v; }

template <typename T>
struct alignas(4 * sizeof(T)) Pack4 {
  T v[4];
};

template <typename S, typename T>
__device__ __forceinline__ S midpoint_one(S p, T a, T m,
                                          typename Compute<T>::type scale,
                                          int sign) {
  const T f = narrow<T>(widen<T>(a) + widen<T>(m));
  const T c = narrow<T>(widen<T>(f) * scale);
  const S cs = (S)widen<T>(c);
  return sign > 0 ? p + cs : p - cs;
}

template <typename S, typename T>
__global__ __launch_bounds__(256)
void midpoint_update_k(const S* p, const T* __restrict__ a,
                       const T* __restrict__ m, S* out,
                       typename Compute<T>::type scale, int sign, int64_t n,
                       int64_t groups) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (int64_t i = tid; i < groups; i += stride) {
    const Pack4<S> pv = reinterpret_cast<const Pack4<S>*>(p)[i];
    const Pack4<T> av = reinterpret_cast<const Pack4<T>*>(a)[i];
    const Pack4<T> mv = reinterpret_cast<const Pack4<T>*>(m)[i];
    Pack4<S> o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o.v[e] = midpoint_one<S, T>(pv.v[e], av.v[e], mv.v[e], scale, sign);
    reinterpret_cast<Pack4<S>*>(out)[i] = o;
  }
  for (int64_t i = groups * 4 + tid; i < n; i += stride)
    out[i] = midpoint_one<S, T>(p[i], a[i], m[i], scale, sign);
}

template <typename S, typename T>
__global__ __launch_bounds__(256)
void midpoint_bwd_k(const S* __restrict__ dout, T* __restrict__ da,
                    typename Compute<T>::type scale, int sign, int64_t n,
                    int64_t groups) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (int64_t i = tid; i < groups; i += stride) {
    const Pack4<S> g = reinterpret_cast<const Pack4<S>*>(dout)[i];
    Pack4<T> o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const S gs = sign > 0 ? g.v[e] : -g.v[e];
      const T gt = narrow<T>((typename Compute<T>::type)gs);
      o.v[e] = narrow<T>(widen<T>(gt) * scale);
    }
    reinterpret_cast<Pack4<T>*>(da)[i] = o;
  }
  for (int64_t i = groups * 4 + tid; i < n; i += stride) {
    const S gs = sign > 0 ? dout[i] : -dout[i];
    const T gt = narrow<T>((typename Compute<T>::type)gs);
    da[i] = narrow<T>(widen<T>(gt) * scale);
  }
}

template <typename S, typename T>
__global__ __launch_bounds__(256)
void axpy_k(const S* x, const T* __restrict__ f, S* out, int sign, int64_t n,
            int64_t groups) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (int64_t i = tid; i < groups; i += stride) {
    const Pack4<S> xv = reinterpret_cast<const Pack4<S>*>(x)[i];
    const Pack4<T> fv = reinterpret_cast<const Pack4<T>*>(f)[i];
    Pack4<S> o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const S fs = (S)widen<T>(fv.v[e]);
      o.v[e] = sign > 0 ? xv.v[e] + fs : xv.v[e] - fs;
    }
    reinterpret_cast<Pack4<S>*>(out)[i] = o;
  }
  for (int64_t i = groups * 4 + tid; i < n; i += stride) {
    const S fs = (S)widen<T>(f[i]);
    out[i] = sign > 0 ? x[i] + fs : x[i] - fs;
  }
}

unsigned grid_for(int64_t n) {
  const int64_t groups = (n + 3) / 4;
  int64_t blocks = (groups + 255) / 256;
  const int64_t cap = (int64_t)rv_host::cu_count() * 32;
  if (blocks > cap) blocks = cap;
  if (blocks < 1) blocks = 1;
  return (unsigned)blocks;
}

bool packs_aligned(const void* p, int bytes_per_pack) {
  return (reinterpret_cast<uintptr_t>(p) % (uintptr_t)bytes_per_pack) == 0;
}

template <typename S, typename T>
int launch_midpoint(const void* p, const void* a, const void* m, void* out,
                    double scale, int sign, int64_t n, hipStream_t s) {
  const bool vec =
      packs_aligned(p, 4 * sizeof(S)) && packs_aligned(out, 4 * sizeof(S)) &&
      packs_aligned(a, 4 * sizeof(T)) && packs_aligned(m, 4 * sizeof(T));
  using C = typename Compute<T>::type;
  hipLaunchKernelGGL((midpoint_update_k<S, T>), dim3(grid_for(n)), dim3(256), 0,
                     s, (const S*)p, (const T*)a, (const T*)m, (S*)out,
                     (C)scale, sign, n, vec ? n / 4 : (int64_t)0);
  return rv_host::check_launch();
}

template <typename S, typename T>
int launch_midpoint_bwd(const void* dout, void* da, double scale, int sign,
                        int64_t n, hipStream_t s) {
  const bool vec =
      packs_aligned(dout, 4 * sizeof(S)) && packs_aligned(da, 4 * sizeof(T));
  using C = typename Compute<T>::type;
  hipLaunchKernelGGL((midpoint_bwd_k<S, T>), dim3(grid_for(n)), dim3(256), 0, s,
                     (const S*)dout, (T*)da, (C)scale, sign, n,
                     vec ? n / 4 : (int64_t)0);
  return rv_host::check_launch();
}

template <typename S, typename T>
int launch_axpy(const void* x, const void* f, void* out, int sign, int64_t n,
                hipStream_t s) {
  const bool vec = packs_aligned(x, 4 * sizeof(S)) &&
                   packs_aligned(out, 4 * sizeof(S)) &&
                   packs_aligned(f, 4 * sizeof(T));
  hipLaunchKernelGGL((axpy_k<S, T>), dim3(grid_for(n)), dim3(256), 0, s,
                     (const S*)x, (const T*)f, (S*)out, sign, n,
                     vec ? n / 4 : (int64_t)0);
  return rv_host::check_launch();
}

// Dispatch over the supported (state, force) pairs.
#define RV_DISPATCH_PAIRS(FN, ...)                                        \
  do {                                                                    \
    if (state_dtype == RV_F32 && force_dtype == RV_F16)                   \
      return FN<float, __half>(__VA_ARGS__);                              \
    if (state_dtype == RV_F32 && force_dtype == RV_BF16)                  \
      return FN<float, __hip_bfloat16>(__VA_ARGS__);                      \
    if (state_dtype == RV_F32 && force_dtype == RV_F32)                   \
      return FN<float, float>(__VA_ARGS__);                               \
    if (state_dtype == RV_F64 && force_dtype == RV_F64)                   \
      return FN<double, double>(__VA_ARGS__);                             \
    return RV_ERR_UNSUPPORTED;                                            \
  } while (0)

}  // namespace

extern "C" {

int rv_midpoint_update(const void* p, const void* a, const void* m, void* out,
                       double scale, int sign, int64_t n, int state_dtype,
                       int force_dtype, void* stream) {
  if (!p || !a || !m || !out) return RV_ERR_NULL_POINTER;
  if (n <= 0 || (sign != 1 && sign != -1)) return RV_ERR_BAD_SIZE;
  const hipStream_t s = (hipStream_t)stream;
  RV_DISPATCH_PAIRS(launch_midpoint, p, a, m, out, scale, sign, n, s);
}

int rv_midpoint_update_bwd(const void* dout, void* da, double scale, int sign,
                           int64_t n, int state_dtype, int force_dtype,
                           void* stream) {
  if (!dout || !da) return RV_ERR_NULL_POINTER;
  if (n <= 0 || (sign != 1 && sign != -1)) return RV_ERR_BAD_SIZE;
  const hipStream_t s = (hipStream_t)stream;
  RV_DISPATCH_PAIRS(launch_midpoint_bwd, dout, da, scale, sign, n, s);
}

int rv_residual_axpy(const void* x, const void* f, void* out, int sign,
                     int64_t n, int state_dtype, int force_dtype,
                     void* stream) {
  if (!x || !f || !out) return RV_ERR_NULL_POINTER;
  if (n <= 0 || (sign != 1 && sign != -1)) return RV_ERR_BAD_SIZE;
  const hipStream_t s = (hipStream_t)stream;
  RV_DISPATCH_PAIRS(launch_axpy, x, f, out, sign, n, s);
}

}  // extern "C"
