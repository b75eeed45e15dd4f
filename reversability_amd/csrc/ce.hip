// Fused cross-entropy over vocabulary rows for gfx950 (the loss of the tied
// LM head, src/reversibility/kernels.py:14-77).
//
// Layout: logits x [rows][ld] (fp16 or fp32, cols <= ld used), labels int64
// [rows]; per-row statistics rmax, rlse, loss fp32 [rows]; dx has x's layout.
//
// Forward: one workgroup (8 waves) per row reads the row once, keeping an
// online (max, sum of exp) per lane over 16-byte vectors, merges lanes with
// DPP / LDS, and writes
//     m = max_j x_j,  lse = log(sum_j exp(x_j - m)),
//     loss = -round_T((x_t - m) - lse)        (0 when label == ignore)
// -- the reference's Half-logsoftmax -> fp32 NLL rounding points (_ce_rows).
// Backward: one pass per row,
//     dx_j = round_T([j == t] neg - exp(round_T((x_j - m) - lse)) neg),
//     neg  = round_T(-grad)                    (_ce_grad)
// with zero rows for ignore.  A label outside [0, cols) other than ignore
// gives a NaN loss and a NaN gradient row (the reference indexes out of
// bounds there; this kernel never reads outside the row).
//
// Rows of an odd vocabulary (50257) start at any 2-byte alignment: each row
// is a scalar head up to the first 16-byte boundary, 16-byte vectors, and a
// scalar tail.  Both passes are HBM-bound: the forward reads 2 bytes per fp16
// logit, the backward reads 2 and writes 2.

#include <cmath>

#include "rv_device.h"

namespace {

// 512 threads per row: the fused kernel's 50257-column rows at 13 vectors per
// thread (C4's 16896 x 50257 logits 626 -> 592 us against 256 threads)
constexpr int kThreads = 512;
constexpr int kWaves = kThreads / 64;

template <typename T>
struct Elem;
template <>
struct Elem<__half> {
  static constexpr int kPerVec = 8;
  __device__ __forceinline__ static float get(const rv::u32x4& v, int i) {
    const uint32_t w = v[i >> 1];
    const unsigned short b = (unsigned short)((i & 1) ? (w >> 16) : (w & 0xffffu));
    return __half2float(__ushort_as_half(b));
  }
  __device__ __forceinline__ static void set(rv::u32x4& v, int i, float f) {
    const uint32_t b = __half_as_ushort(__float2half_rn(f));
    const uint32_t w = v[i >> 1];
    v[i >> 1] = (i & 1) ? ((w & 0xffffu) | (b << 16)) : ((w & 0xffff0000u) | b);
  }
};
template <>
struct Elem<float> {
  static constexpr int kPerVec = 4;
  __device__ __forceinline__ static float get(const rv::u32x4& v, int i) {
    return __uint_as_float(v[i]);
  }
  __device__ __forceinline__ static void set(rv::u32x4& v, int i, float f) { v[i] = __float_as_uint(f); }
};

// Row split into a scalar head (up to the first 16-byte boundary), nvec
// 16-byte vectors, and a scalar tail.
template <typename T>
struct RowSplit {
  int64_t head, nvec, tail0;
  __device__ __forceinline__ RowSplit(const T* row, int64_t cols) {
    constexpr int V = Elem<T>::kPerVec;
    const int64_t h = (int64_t)(((16 - (reinterpret_cast<uintptr_t>(row) & 15)) & 15) / sizeof(T));
    head = h < cols ? h : cols;
    nvec = (cols - head) / V;
    tail0 = head + nvec * V;
  }
};

// Online softmax statistics: (m, s) with s = sum exp(x - m).
__device__ __forceinline__ void merge(float& m, float& s, float m2, float s2) {
  const float n = fmaxf(m, m2);
  if (n == -INFINITY) return;  // both empty
  s = s * __expf(m - n) + s2 * __expf(m2 - n);
  m = n;
}
__device__ __forceinline__ void add(float& m, float& s, float x) {
  if (x > m) {
    s = s * __expf(m - x) + 1.0f;
    m = x;
  } else {
    s = s + __expf(x - m);
  }
}

template <typename T>
__device__ __forceinline__ float load1(const T* p) {
  return rv::Conv<T>::to_f(*p);
}

template <typename T>
__global__ __launch_bounds__(kThreads)
void ce_fwd_k(const T* __restrict__ x, int64_t ld, const int64_t* __restrict__ labels,
              int64_t cols, int64_t ignore, float* __restrict__ rmax, float* __restrict__ rlse,
              float* __restrict__ loss) {
  constexpr int V = Elem<T>::kPerVec;
  const int64_t row = blockIdx.x;
  const T* xr = x + row * ld;
  const RowSplit<T> sp(xr, cols);
  float m = -INFINITY, s = 0.f;
  for (int64_t c = threadIdx.x; c < sp.head; c += kThreads) add(m, s, load1(xr + c));
  const rv::u32x4* xv = reinterpret_cast<const rv::u32x4*>(xr + sp.head);
#pragma unroll 4
  for (int64_t v = threadIdx.x; v < sp.nvec; v += kThreads) {
    const rv::u32x4 w = __builtin_nontemporal_load(xv + v);
    float e[V];
    float vm = -INFINITY;
#pragma unroll
    for (int i = 0; i < V; ++i) {
      e[i] = Elem<T>::get(w, i);
      vm = fmaxf(vm, e[i]);
    }
    const float n = fmaxf(m, vm);
    float acc = m == -INFINITY ? 0.f : s * __expf(m - n);
#pragma unroll
    for (int i = 0; i < V; ++i) acc = acc + __expf(e[i] - n);
    // NaN logits propagate through the sum (n may be NaN as well)
    m = n;
    s = acc;
  }
  for (int64_t c = sp.tail0 + threadIdx.x; c < cols; c += kThreads) add(m, s, load1(xr + c));

  // wave merge (butterfly over 64 lanes), then across the waves in order
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float m2 = __shfl_xor(m, off, 64);
    const float s2 = __shfl_xor(s, off, 64);
    merge(m, s, m2, s2);
  }
  __shared__ float wm[kWaves], ws[kWaves];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    wm[wave] = m;
    ws[wave] = s;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float M = wm[0], S = ws[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) merge(M, S, wm[w], ws[w]);
    const float lse = logf(S);
    rmax[row] = M;
    rlse[row] = lse;
    const int64_t t = labels[row];
    float l;
    if (t == ignore) l = 0.f;
    else if (t < 0 || t >= cols) l = NAN;
    else l = -rv::round_to<T>((load1(xr + t) - M) - lse);
    loss[row] = l;
  }
}

template <typename T>
__device__ __forceinline__ float grad_of(float xv, int64_t col, int64_t t, float m, float lse,
                                         float neg) {
  const float logp = rv::round_to<T>((xv - m) - lse);
  return (col == t ? neg : 0.f) - __expf(logp) * neg;
}

// Non-target column: grad_of's value with the label test dropped.
template <typename T>
__device__ __forceinline__ float grad_off(float xv, float m, float lse, float neg) {
  return 0.f - __expf(rv::round_to<T>((xv - m) - lse)) * neg;
}

template <typename T>
__global__ __launch_bounds__(kThreads)
void ce_bwd_k(const T* __restrict__ x, int64_t ld, const int64_t* __restrict__ labels,
              const float* __restrict__ rmax, const float* __restrict__ rlse,
              const float* __restrict__ grad, int64_t cols, int64_t ignore, T* __restrict__ dx) {
  constexpr int V = Elem<T>::kPerVec;
  const int64_t row = blockIdx.x;
  const T* xr = x + row * ld;
  T* dr = dx + row * ld;
  const RowSplit<T> sp(xr, cols);
  const int64_t t = labels[row];
  const rv::u32x4* xv = reinterpret_cast<const rv::u32x4*>(xr + sp.head);
  rv::u32x4* dv = reinterpret_cast<rv::u32x4*>(dr + sp.head);
  if (t == ignore) {  // an ignored row has a zero gradient
    for (int64_t c = threadIdx.x; c < sp.head; c += kThreads) dr[c] = rv::Conv<T>::from_f(0.f);
    for (int64_t v = threadIdx.x; v < sp.nvec; v += kThreads)
      __builtin_nontemporal_store(rv::u32x4{0u, 0u, 0u, 0u}, dv + v);
    for (int64_t c = sp.tail0 + threadIdx.x; c < cols; c += kThreads)
      dr[c] = rv::Conv<T>::from_f(0.f);
    return;
  }
  const bool bad = t < 0 || t >= cols;
  const float m = rmax[row], lse = rlse[row];
  const float neg = bad ? NAN : rv::round_to<T>(-grad[0]);
  for (int64_t c = threadIdx.x; c < sp.head; c += kThreads)
    dr[c] = rv::Conv<T>::from_f(grad_of<T>(load1(xr + c), c, t, m, lse, neg));
#pragma unroll 4
  for (int64_t v = threadIdx.x; v < sp.nvec; v += kThreads) {
    const rv::u32x4 w = __builtin_nontemporal_load(xv + v);
    rv::u32x4 o;
#pragma unroll
    for (int i = 0; i < V; ++i) Elem<T>::set(o, i, grad_off<T>(Elem<T>::get(w, i), m, lse, neg));
    const int64_t c0 = sp.head + v * V;
    if (static_cast<uint64_t>(t - c0) < static_cast<uint64_t>(V)) {  // the target's vector
#pragma unroll
      for (int i = 0; i < V; ++i)
        if (c0 + i == t) Elem<T>::set(o, i, grad_of<T>(Elem<T>::get(w, i), c0 + i, t, m, lse, neg));
    }
    __builtin_nontemporal_store(o, dv + v);
  }
  for (int64_t c = sp.tail0 + threadIdx.x; c < cols; c += kThreads)
    dr[c] = rv::Conv<T>::from_f(grad_of<T>(load1(xr + c), c, t, m, lse, neg));
}

// Forward and backward of one row in one pass over HBM: the row's 16-byte
// vectors stay in registers (NV per thread, the same thread-to-vector
// assignment and reduction order as ce_fwd_k), so the statistics, the loss and
// the gradient are those of ce_fwd_k followed by ce_bwd_k, bit for bit, with
// the row read once.  Needs the upstream gradient before the pass (the tied
// head's trainer knows it: scale / denominator).
template <typename T, int NV>
__global__ __launch_bounds__(kThreads)
void ce_fused_k(const T* __restrict__ x, int64_t ld, const int64_t* __restrict__ labels,
                int64_t cols, int64_t ignore, const float* __restrict__ grad,
                float* __restrict__ rmax, float* __restrict__ rlse, float* __restrict__ loss,
                T* __restrict__ dx) {
  constexpr int V = Elem<T>::kPerVec;
  const int64_t row = blockIdx.x;
  const T* xr = x + row * ld;
  T* dr = dx + row * ld;
  const RowSplit<T> sp(xr, cols);
  const rv::u32x4* xv = reinterpret_cast<const rv::u32x4*>(xr + sp.head);
  rv::u32x4* dv = reinterpret_cast<rv::u32x4*>(dr + sp.head);
  rv::u32x4 r[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t v = threadIdx.x + (int64_t)i * kThreads;
    r[i] = v < sp.nvec ? __builtin_nontemporal_load(xv + v) : rv::u32x4{0u, 0u, 0u, 0u};
  }
  float m = -INFINITY, s = 0.f;
  for (int64_t c = threadIdx.x; c < sp.head; c += kThreads) add(m, s, load1(xr + c));
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    if (threadIdx.x + (int64_t)i * kThreads >= sp.nvec) break;
    float e[V];
    float vm = -INFINITY;
#pragma unroll
    for (int k = 0; k < V; ++k) {
      e[k] = Elem<T>::get(r[i], k);
      vm = fmaxf(vm, e[k]);
    }
    const float n = fmaxf(m, vm);
    float acc = m == -INFINITY ? 0.f : s * __expf(m - n);
#pragma unroll
    for (int k = 0; k < V; ++k) acc = acc + __expf(e[k] - n);
    m = n;
    s = acc;
  }
  for (int64_t c = sp.tail0 + threadIdx.x; c < cols; c += kThreads) add(m, s, load1(xr + c));
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float m2 = __shfl_xor(m, off, 64);
    const float s2 = __shfl_xor(s, off, 64);
    merge(m, s, m2, s2);
  }
  __shared__ float wm[kWaves], ws[kWaves], stat[2];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    wm[wave] = m;
    ws[wave] = s;
  }
  __syncthreads();
  const int64_t t = labels[row];
  if (threadIdx.x == 0) {
    float M = wm[0], S = ws[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) merge(M, S, wm[w], ws[w]);
    const float lse = logf(S);
    rmax[row] = M;
    rlse[row] = lse;
    float l;
    if (t == ignore) l = 0.f;
    else if (t < 0 || t >= cols) l = NAN;
    else l = -rv::round_to<T>((load1(xr + t) - M) - lse);
    loss[row] = l;
    stat[0] = M;
    stat[1] = lse;
  }
  __syncthreads();
  if (t == ignore) {
    for (int64_t c = threadIdx.x; c < sp.head; c += kThreads) dr[c] = rv::Conv<T>::from_f(0.f);
    for (int64_t v = threadIdx.x; v < sp.nvec; v += kThreads)
      __builtin_nontemporal_store(rv::u32x4{0u, 0u, 0u, 0u}, dv + v);
    for (int64_t c = sp.tail0 + threadIdx.x; c < cols; c += kThreads)
      dr[c] = rv::Conv<T>::from_f(0.f);
    return;
  }
  const float M = stat[0], lse = stat[1];
  const bool bad = t < 0 || t >= cols;
  const float neg = bad ? NAN : rv::round_to<T>(-grad[0]);
  for (int64_t c = threadIdx.x; c < sp.head; c += kThreads)
    dr[c] = rv::Conv<T>::from_f(grad_of<T>(load1(xr + c), c, t, M, lse, neg));
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int64_t v = threadIdx.x + (int64_t)i * kThreads;
    if (v >= sp.nvec) break;
    rv::u32x4 o;
#pragma unroll
    for (int k = 0; k < V; ++k) Elem<T>::set(o, k, grad_off<T>(Elem<T>::get(r[i], k), M, lse, neg));
    const int64_t c0 = sp.head + v * V;
    if (static_cast<uint64_t>(t - c0) < static_cast<uint64_t>(V)) {
#pragma unroll
      for (int k = 0; k < V; ++k)
        if (c0 + k == t) Elem<T>::set(o, k, grad_of<T>(Elem<T>::get(r[i], k), c0 + k, t, M, lse, neg));
    }
    __builtin_nontemporal_store(o, dv + v);
  }
  for (int64_t c = sp.tail0 + threadIdx.x; c < cols; c += kThreads)
    dr[c] = rv::Conv<T>::from_f(grad_of<T>(load1(xr + c), c, t, M, lse, neg));
}

}  // namespace

extern "C" {

int rv_ce_fwd(const void* logits, int dtype, int64_t ld, const int64_t* labels, int64_t rows,
              int64_t cols, int64_t ignore_index, float* row_max, float* row_lse, float* loss,
              void* stream) {
  if (!logits || !labels || !row_max || !row_lse || !loss) return RV_ERR_NULL_POINTER;
  if (rows < 0 || cols <= 0 || ld < cols) return RV_ERR_BAD_SIZE;
  if (rows == 0) return RV_OK;
  if (rows > 0x7fffffff) return RV_ERR_UNSUPPORTED;
  const hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)rows), block(kThreads);
  if (dtype == RV_F16)
    hipLaunchKernelGGL(ce_fwd_k<__half>, grid, block, 0, s, static_cast<const __half*>(logits),
                       ld, labels, cols, ignore_index, row_max, row_lse, loss);
  else if (dtype == RV_F32)
    hipLaunchKernelGGL(ce_fwd_k<float>, grid, block, 0, s, static_cast<const float*>(logits), ld,
                       labels, cols, ignore_index, row_max, row_lse, loss);
  else
    return RV_ERR_UNSUPPORTED;
  return rv_host::check_launch();
}

int rv_ce_bwd(const void* logits, int dtype, int64_t ld, const int64_t* labels,
              const float* row_max, const float* row_lse, const float* grad, int64_t rows,
              int64_t cols, int64_t ignore_index, void* dlogits, void* stream) {
  if (!logits || !labels || !row_max || !row_lse || !grad || !dlogits) return RV_ERR_NULL_POINTER;
  if (rows < 0 || cols <= 0 || ld < cols) return RV_ERR_BAD_SIZE;
  if (rows == 0) return RV_OK;
  if (rows > 0x7fffffff) return RV_ERR_UNSUPPORTED;
  // the vector path walks x and dx with the same split: same 16-byte phase
  if ((reinterpret_cast<uintptr_t>(logits) & 15) != (reinterpret_cast<uintptr_t>(dlogits) & 15))
    return RV_ERR_UNSUPPORTED;
  const hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)rows), block(kThreads);
  if (dtype == RV_F16)
    hipLaunchKernelGGL(ce_bwd_k<__half>, grid, block, 0, s, static_cast<const __half*>(logits),
                       ld, labels, row_max, row_lse, grad, cols, ignore_index,
                       static_cast<__half*>(dlogits));
  else if (dtype == RV_F32)
    hipLaunchKernelGGL(ce_bwd_k<float>, grid, block, 0, s, static_cast<const float*>(logits), ld,
                       labels, row_max, row_lse, grad, cols, ignore_index,
                       static_cast<float*>(dlogits));
  else
    return RV_ERR_UNSUPPORTED;
  return rv_host::check_launch();
}

int rv_ce_fused(const void* logits, int dtype, int64_t ld, const int64_t* labels, int64_t rows,
                int64_t cols, int64_t ignore_index, const float* grad, float* row_max,
                float* row_lse, float* loss, void* dlogits, void* stream) {
  if (!logits || !labels || !grad || !row_max || !row_lse || !loss || !dlogits)
    return RV_ERR_NULL_POINTER;
  if (rows < 0 || cols <= 0 || ld < cols) return RV_ERR_BAD_SIZE;
  if (rows == 0) return RV_OK;
  if (rows > 0x7fffffff || dtype != RV_F16) return RV_ERR_UNSUPPORTED;
  if (cols > 65536) return RV_ERR_UNSUPPORTED;  // wider rows take the two-pass kernels
  if ((reinterpret_cast<uintptr_t>(logits) & 15) != (reinterpret_cast<uintptr_t>(dlogits) & 15))
    return RV_ERR_UNSUPPORTED;
  // vectors per thread the row needs (upper bound: the scalar head takes < 8)
  const int64_t per = (cols / 8 + kThreads - 1) / kThreads;
  const hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)rows), block(kThreads);
  const __half* x = static_cast<const __half*>(logits);
  __half* d = static_cast<__half*>(dlogits);
#define RV_CE_FUSED(NV)                                                                      \
  case NV:                                                                                   \
    hipLaunchKernelGGL((ce_fused_k<__half, NV>), grid, block, 0, s, x, ld, labels, cols,      \
                       ignore_index, grad, row_max, row_lse, loss, d);                       \
    break
  // registers per thread: the row's vectors (one instantiation per count, so a
  // row holds no more registers than it needs and occupancy stays as high as
  // it can: 50257 columns take 13 vectors per thread, 65536 take 16)
  switch (per < 1 ? 1 : per) {
    RV_CE_FUSED(1); RV_CE_FUSED(2); RV_CE_FUSED(3); RV_CE_FUSED(4);
    RV_CE_FUSED(5); RV_CE_FUSED(6); RV_CE_FUSED(7); RV_CE_FUSED(8);
    RV_CE_FUSED(9); RV_CE_FUSED(10); RV_CE_FUSED(11); RV_CE_FUSED(12);
    RV_CE_FUSED(13); RV_CE_FUSED(14); RV_CE_FUSED(15); RV_CE_FUSED(16);
    default:
      return RV_ERR_UNSUPPORTED;
  }
#undef RV_CE_FUSED
  return rv_host::check_launch();
}

}  // extern "C"
