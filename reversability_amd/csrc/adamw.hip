// Multi-tensor AdamW step for gfx950 (the optimizer update of the training
// step, scripts/benchmark_optimized.py:38-40, 66-80; torch.optim.AdamW with
// decoupled weight decay, driven through torch.amp.GradScaler).
//
// One launch updates up to kMaxTensors fp32 parameter tensors: the pointer
// table and the per-tensor chunk prefix sums travel in the kernel arguments
// (gradients are fresh tensors every step), each workgroup updates one chunk of
// kChunk elements of one tensor with 16-byte accesses:
//
//     p  = p * (1 - lr wd)
//     m  = lerp(m, g, 1 - b1)                       (torch's lerp formula)
//     v  = v * b2 + (1 - b2) g g
//     p  = p - (lr / (1 - b1^t)) * m / (sqrt(v) / sqrt(1 - b2^t) + eps)
//
// in fp32 with torch's operation order (foreach AdamW, whose lerp, addcmul
// and addcdiv each contract to one fused multiply-add); g is multiplied by
// *inv_scale when given.  The step count t lives on the device (one fp32 per
// parameter group): rv_adamw_advance adds 1 unless *found_inf != 0, and the
// update kernel skips every element when *found_inf != 0, so a skipped step
// (GradScaler overflow) changes nothing and needs no host synchronisation.
// The bias corrections are computed per workgroup in double from t.

#include <cmath>

#include "rv_device.h"

namespace {

constexpr int kThreads = 256;
constexpr int kMaxTensors = 48;
// elements per workgroup: 16384 (C4's 20.3M parameters in ~1250 workgroups
// rather than ~330; C4 step 6.93 -> 6.87 ms against 65536 in same-box runs)
constexpr int64_t kChunk = 16384;

struct TensorTable {
  float* p[kMaxTensors];
  const float* g[kMaxTensors];
  float* m[kMaxTensors];
  float* v[kMaxTensors];
  int64_t n[kMaxTensors];
  int chunk_start[kMaxTensors + 1];  // prefix sums of per-tensor chunk counts
  int count;
};

struct Hyper {
  float lr, beta1, beta2, eps, decay;  // decay = fp32(1 - lr * wd)
  double lr_d, beta1_d, beta2_d;       // the bias corrections are formed in double
  const float* step;                   // t after this update (already advanced)
  const float* found_inf;              // nullable
  const float* inv_scale;              // nullable
  const float* clip;                   // nullable: clip_grad_norm_'s clamped coefficient
};

// torch's lerp, addcmul and addcdiv as its ROCm build evaluates them: the
// multiply-add of each is one fused multiply-add.
__device__ __forceinline__ float lerp_t(float a, float b, float w) {
  // weight < 0.5 ? a + w (b - a) : b - (b - a) (1 - w)
  return fabsf(w) < 0.5f ? __builtin_fmaf(w, b - a, a) : __builtin_fmaf(-(b - a), 1.0f - w, b);
}

struct Scalars {
  float w1, one_minus_b2, step_size, bc2_sqrt, inv, clip;
};

__device__ __forceinline__ void update1(float& p, float g, float& m, float& v, const Hyper& h,
                                        const Scalars& s) {
  g = g * s.inv;   // GradScaler.unscale_ (exact when inv == 1)
  g = g * s.clip;  // clip_grad_norm_'s multiply (exact when clip == 1)
  p = p * h.decay;
  m = lerp_t(m, g, s.w1);
  v = v * h.beta2;
  v = __builtin_fmaf(s.one_minus_b2 * g, g, v);        // addcmul
  const float denom = sqrtf(v) / s.bc2_sqrt + h.eps;
  p = __builtin_fmaf(-s.step_size, m / denom, p);     // addcdiv
}

__global__ __launch_bounds__(kThreads)
void adamw_k(TensorTable tab, Hyper h) {
  if (h.found_inf != nullptr && *h.found_inf != 0.0f) return;  // uniform skip
  // tensor of this chunk: last t with chunk_start[t] <= blockIdx.x
  int t = 0;
  for (int i = 1; i < tab.count; ++i)
    if (tab.chunk_start[i] <= (int)blockIdx.x) t = i;
  const int64_t off = (int64_t)(blockIdx.x - tab.chunk_start[t]) * kChunk;
  const int64_t end = off + kChunk < tab.n[t] ? off + kChunk : tab.n[t];
  const double step = (double)*h.step;
  Scalars s;
  s.w1 = (float)(1.0 - h.beta1_d);
  s.one_minus_b2 = (float)(1.0 - h.beta2_d);
  s.step_size = (float)(h.lr_d / (1.0 - pow(h.beta1_d, step)));
  s.bc2_sqrt = (float)sqrt(1.0 - pow(h.beta2_d, step));
  s.inv = h.inv_scale != nullptr ? *h.inv_scale : 1.0f;
  s.clip = h.clip != nullptr ? *h.clip : 1.0f;
  float* p = tab.p[t];
  const float* g = tab.g[t];
  float* m = tab.m[t];
  float* v = tab.v[t];
  const bool vec = ((reinterpret_cast<uintptr_t>(p) | reinterpret_cast<uintptr_t>(g) |
                     reinterpret_cast<uintptr_t>(m) | reinterpret_cast<uintptr_t>(v)) & 15) == 0;
  int64_t i = off + threadIdx.x * 4;
  if (vec) {
    for (; i + 4 <= end; i += kThreads * 4) {
      float4 pp = *reinterpret_cast<const float4*>(p + i);
      const float4 gg = *reinterpret_cast<const float4*>(g + i);
      float4 mm = *reinterpret_cast<const float4*>(m + i);
      float4 vv = *reinterpret_cast<const float4*>(v + i);
      update1(pp.x, gg.x, mm.x, vv.x, h, s);
      update1(pp.y, gg.y, mm.y, vv.y, h, s);
      update1(pp.z, gg.z, mm.z, vv.z, h, s);
      update1(pp.w, gg.w, mm.w, vv.w, h, s);
      *reinterpret_cast<float4*>(p + i) = pp;
      *reinterpret_cast<float4*>(m + i) = mm;
      *reinterpret_cast<float4*>(v + i) = vv;
    }
    // tail (< 4 elements at the very end of the tensor)
    for (int64_t j = (i < end ? i : end); j < end; ++j) update1(p[j], g[j], m[j], v[j], h, s);
  } else {
    for (int64_t j = off + threadIdx.x; j < end; j += kThreads) update1(p[j], g[j], m[j], v[j], h, s);
  }
}

// Gradient-norm pass of GradScaler.unscale_ + clip_grad_norm_(p, max_norm, 2):
// per chunk of one tensor (same table and chunking as the update) the fp32 sum
// of squares of the unscaled gradient g * inv (the value unscale_ would write)
// and whether any unscaled element is non-finite.  Fixed summation order:
// each thread its elements in order, then a wave butterfly, then the waves in
// order.  Partials go to part[first + chunk], flags to flag[first + chunk].
struct GradTable {
  const float* g[kMaxTensors];
  int64_t n[kMaxTensors];
  int chunk_start[kMaxTensors + 1];
  int count;
};

__global__ __launch_bounds__(kThreads)
void grad_sq_k(GradTable tab, const float* __restrict__ inv_scale, float* __restrict__ part,
               float* __restrict__ flag, int first) {
  int t = 0;
  for (int i = 1; i < tab.count; ++i)
    if (tab.chunk_start[i] <= (int)blockIdx.x) t = i;
  const int64_t off = (int64_t)(blockIdx.x - tab.chunk_start[t]) * kChunk;
  const int64_t end = off + kChunk < tab.n[t] ? off + kChunk : tab.n[t];
  const float inv = inv_scale != nullptr ? *inv_scale : 1.0f;
  const float* g = tab.g[t];
  float ss = 0.f;
  bool bad = false;
  auto add = [&](float x) {
    const float u = x * inv;
    bad = bad || !isfinite(u);
    ss = __builtin_fmaf(u, u, ss);
  };
  int64_t i = off + threadIdx.x * 4;
  if ((reinterpret_cast<uintptr_t>(g) & 15) == 0) {
    for (; i + 4 <= end; i += kThreads * 4) {
      const float4 q = *reinterpret_cast<const float4*>(g + i);
      add(q.x);
      add(q.y);
      add(q.z);
      add(q.w);
    }
    for (int64_t j = (i < end ? i : end); j < end; ++j) add(g[j]);
  } else {
    for (int64_t j = off + threadIdx.x; j < end; j += kThreads) add(g[j]);
  }
  ss = rv::wave_sum(ss);
  const bool wave_bad = __any(bad);
  __shared__ float ws[kThreads / 64];
  __shared__ int wb[kThreads / 64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    ws[wave] = ss;
    wb[wave] = wave_bad;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float tot = ws[0];
    int any = wb[0];
#pragma unroll
    for (int w = 1; w < kThreads / 64; ++w) {
      tot = tot + ws[w];
      any |= wb[w];
    }
    part[first + blockIdx.x] = tot;
    flag[first + blockIdx.x] = any ? 1.0f : 0.0f;
  }
}

// total = sqrt(sum of the partials, in order), clip = min(max_norm / (total +
// 1e-6), 1) (clip_grad_norm_'s fp32 formulas), found_inf = 1 if any chunk had
// a non-finite unscaled gradient.  One workgroup.
__global__ __launch_bounds__(kThreads)
void grad_clip_k(const float* __restrict__ part, const float* __restrict__ flag, int n,
                 float max_norm, float* __restrict__ total, float* __restrict__ clip,
                 float* __restrict__ found_inf) {
  float ss = 0.f;
  float any = 0.f;
  // each thread's partials in the same order as one at a time, loaded eight
  // at a time (C5's 15583 partials: one memory round trip per eight)
  int i = threadIdx.x;
  for (; i + 7 * kThreads < n; i += 8 * kThreads) {
    float p[8], f[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      p[j] = part[i + j * kThreads];
      f[j] = flag[i + j * kThreads];
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      ss = ss + p[j];
      any = fmaxf(any, f[j]);
    }
  }
  for (; i < n; i += kThreads) {
    ss = ss + part[i];
    any = fmaxf(any, flag[i]);
  }
  ss = rv::wave_sum(ss);
  for (int o = 32; o >= 1; o >>= 1) any = fmaxf(any, __shfl_xor(any, o, 64));
  __shared__ float ws[kThreads / 64], wa[kThreads / 64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    ws[wave] = ss;
    wa[wave] = any;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float tot = ws[0], a = wa[0];
#pragma unroll
    for (int w = 1; w < kThreads / 64; ++w) {
      tot = tot + ws[w];
      a = fmaxf(a, wa[w]);
    }
    const float norm = sqrtf(tot);
    const float coef = max_norm / (norm + 1e-6f);
    *total = norm;
    *clip = coef < 1.0f ? coef : 1.0f;
    *found_inf = a;
  }
}

__global__ void adamw_advance_k(float* step, const float* found_inf) {
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    if (found_inf == nullptr || *found_inf == 0.0f) *step = *step + 1.0f;
  }
}

}  // namespace

extern "C" {

int rv_adamw_max_tensors(void) { return kMaxTensors; }

int rv_adamw_advance(float* step, const float* found_inf, void* stream) {
  if (!step) return RV_ERR_NULL_POINTER;
  hipLaunchKernelGGL(adamw_advance_k, dim3(1), dim3(64), 0, (hipStream_t)stream, step, found_inf);
  return rv_host::check_launch();
}

int rv_grad_chunks(const int64_t* numel, int count) {
  if (count < 0 || (count > 0 && !numel)) return -RV_ERR_BAD_SIZE;
  int64_t chunks = 0;
  for (int i = 0; i < count; ++i) {
    if (numel[i] < 0) return -RV_ERR_BAD_SIZE;
    chunks += (numel[i] + kChunk - 1) / kChunk;
    if (chunks > 0x7fffffff) return -RV_ERR_UNSUPPORTED;
  }
  return (int)chunks;
}

int rv_grad_sq_partials(int count, const float* const* grads, const int64_t* numel,
                        const float* inv_scale, float* partials, float* flags, int first,
                        void* stream) {
  if (count <= 0) return count == 0 ? RV_OK : RV_ERR_BAD_SIZE;
  if (count > kMaxTensors) return RV_ERR_UNSUPPORTED;
  if (!grads || !numel || !partials || !flags) return RV_ERR_NULL_POINTER;
  if (first < 0) return RV_ERR_BAD_SIZE;
  GradTable tab{};
  int chunks = 0;
  for (int i = 0; i < count; ++i) {
    if (!grads[i]) return RV_ERR_NULL_POINTER;
    if (numel[i] <= 0) return RV_ERR_BAD_SIZE;
    tab.g[i] = grads[i];
    tab.n[i] = numel[i];
    tab.chunk_start[i] = chunks;
    const int64_t c = (numel[i] + kChunk - 1) / kChunk;
    if ((int64_t)chunks + c > 0x7fffffff) return RV_ERR_UNSUPPORTED;
    chunks += (int)c;
  }
  tab.chunk_start[count] = chunks;
  tab.count = count;
  hipLaunchKernelGGL(grad_sq_k, dim3((unsigned)chunks), dim3(kThreads), 0, (hipStream_t)stream,
                     tab, inv_scale, partials, flags, first);
  return rv_host::check_launch();
}

int rv_grad_clip_coef(const float* partials, const float* flags, int n, double max_norm,
                      float* total_norm, float* clip_coef, float* found_inf, void* stream) {
  if (n <= 0) return RV_ERR_BAD_SIZE;
  if (!partials || !flags || !total_norm || !clip_coef || !found_inf) return RV_ERR_NULL_POINTER;
  hipLaunchKernelGGL(grad_clip_k, dim3(1), dim3(kThreads), 0, (hipStream_t)stream, partials, flags,
                     n, (float)max_norm, total_norm, clip_coef, found_inf);
  return rv_host::check_launch();
}

int rv_adamw_step(int count, float* const* params, const float* const* grads,
                  float* const* exp_avg, float* const* exp_avg_sq, const int64_t* numel,
                  double lr, double beta1, double beta2, double eps, double weight_decay,
                  const float* step, const float* found_inf, const float* inv_scale,
                  void* stream) {
  return rv_adamw_step_clipped(count, params, grads, exp_avg, exp_avg_sq, numel, lr, beta1, beta2,
                               eps, weight_decay, step, found_inf, inv_scale, nullptr, stream);
}

int rv_adamw_step_clipped(int count, float* const* params, const float* const* grads,
                          float* const* exp_avg, float* const* exp_avg_sq, const int64_t* numel,
                          double lr, double beta1, double beta2, double eps, double weight_decay,
                          const float* step, const float* found_inf, const float* inv_scale,
                          const float* clip_coef, void* stream) {
  if (count <= 0) return count == 0 ? RV_OK : RV_ERR_BAD_SIZE;
  if (count > kMaxTensors) return RV_ERR_UNSUPPORTED;
  if (!params || !grads || !exp_avg || !exp_avg_sq || !numel || !step) return RV_ERR_NULL_POINTER;
  TensorTable tab{};
  Hyper h{};
  int chunks = 0;
  for (int i = 0; i < count; ++i) {
    if (!params[i] || !grads[i] || !exp_avg[i] || !exp_avg_sq[i]) return RV_ERR_NULL_POINTER;
    if (numel[i] <= 0) return RV_ERR_BAD_SIZE;
    tab.p[i] = params[i];
    tab.g[i] = grads[i];
    tab.m[i] = exp_avg[i];
    tab.v[i] = exp_avg_sq[i];
    tab.n[i] = numel[i];
    tab.chunk_start[i] = chunks;
    const int64_t c = (numel[i] + kChunk - 1) / kChunk;
    if ((int64_t)chunks + c > 0x7fffffff) return RV_ERR_UNSUPPORTED;
    chunks += (int)c;
  }
  tab.chunk_start[count] = chunks;
  tab.count = count;
  h.lr = (float)lr;
  h.beta1 = (float)beta1;
  h.beta2 = (float)beta2;
  h.eps = (float)eps;
  h.decay = (float)(1.0 - lr * weight_decay);
  h.lr_d = lr;
  h.beta1_d = beta1;
  h.beta2_d = beta2;
  h.step = step;
  h.found_inf = found_inf;
  h.inv_scale = inv_scale;
  h.clip = clip_coef;
  hipLaunchKernelGGL(adamw_k, dim3((unsigned)chunks), dim3(kThreads), 0, (hipStream_t)stream, tab,
                     h);
  return rv_host::check_launch();
}

}  // extern "C"
