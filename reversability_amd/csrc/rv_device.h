// Device-side helpers shared by the gfx950 kernels: wave64 reductions built
// on DPP and v_readlane, 16-byte vector loads/stores, dtype conversions and
// the per-device launch context.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <hip/hip_bf16.h>
#include <stdint.h>

#include "../../include/reversibility_hip.h"

namespace rv {

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// Wave64 sum.  Inside each 16-lane DPP row: xor-1 and xor-2 via quad_perm,
// then rotate-by-4 and rotate-by-8 (row_ror), after which every lane of a row
// holds that row's sum.  The four row sums are combined with v_readlane in a
// fixed order, so every lane returns the same, run-to-run identical value.
// All 64 lanes must be active.
// ---------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(
      0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

__device__ __forceinline__ float wave_sum(float v) {
  v = v + dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]
  v = v + dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]
  v = v + dpp_mov<0x124>(v);  // row_ror:4
  v = v + dpp_mov<0x128>(v);  // row_ror:8
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return ((r0 + r1) + r2) + r3;
}

// Sum over each 16-lane DPP row, the same bits in all 16 lanes: xor-1 and
// xor-2 (quad_perm) leave every lane of a quad with the same quad sum, then
// row_half_mirror (lane i with 7 - i of its 8-lane half) and row_mirror (i
// with 15 - i) add partners that hold the same-order partial sums, so each
// add is a + b in one lane and b + a in its partner: bitwise equal.  The
// result is ((q0 + q1) + (q2 + q3)) of the four quad sums q.
__device__ __forceinline__ float row16_sum(float v) {
  v = v + dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]
  v = v + dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]
  v = v + dpp_mov<0x141>(v);  // row_half_mirror
  v = v + dpp_mov<0x140>(v);  // row_mirror
  return v;
}

// Sum over a group of G lanes (a row of the RMSNorm layouts), the same value
// in every lane of the group: G = 16 (one DPP row) or 64 (the wave).
template <int G>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(G == 16 || G == 64, "lane groups of 16 or 64");
  if constexpr (G == 16) return row16_sum(v);
  else return wave_sum(v);
}

// ---------------------------------------------------------------------------
// dtype plumbing
// ---------------------------------------------------------------------------
template <typename T> struct Conv;
template <> struct Conv<float> {
  __device__ __forceinline__ static float to_f(float v) { return v; }
  __device__ __forceinline__ static float from_f(float v) { return v; }
};
template <> struct Conv<__half> {
  __device__ __forceinline__ static float to_f(__half v) { return __half2float(v); }
  __device__ __forceinline__ static __half from_f(float v) { return __float2half_rn(v); }
};
template <> struct Conv<__hip_bfloat16> {
  __device__ __forceinline__ static float to_f(__hip_bfloat16 v) { return __bfloat162float(v); }
  __device__ __forceinline__ static __hip_bfloat16 from_f(float v) { return __float2bfloat16(v); }
};

// Round a float through dtype T and back (identity for float).
template <typename T>
__device__ __forceinline__ float round_to(float v) {
  return Conv<T>::to_f(Conv<T>::from_f(v));
}

// 16-byte global accesses, plain or streaming.  Streaming (NT = true) puts
// the nt hint on the instruction for data touched exactly once, so a stream
// of hundreds of MB does not evict reusable lines; each kernel picks per
// operand what measured fastest.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <bool NT>
__device__ __forceinline__ uint4 ld16(const void* p) {
  if constexpr (NT) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
  } else {
    return *reinterpret_cast<const uint4*>(p);
  }
}
template <bool NT>
__device__ __forceinline__ void st16(void* p, uint4 v) {
  if constexpr (NT) {
    u32x4 t;
    t.x = v.x; t.y = v.y; t.z = v.z; t.w = v.w;
    __builtin_nontemporal_store(t, reinterpret_cast<u32x4*>(p));
  } else {
    *reinterpret_cast<uint4*>(p) = v;
  }
}

// 16-byte vector of T.
template <typename T>
struct alignas(16) Vec16 {
  static constexpr int N = 16 / sizeof(T);
  T v[N];
};

template <bool NT = false, typename T>
__device__ __forceinline__ Vec16<T> load16(const T* p) {
  Vec16<T> r;
  *reinterpret_cast<uint4*>(&r) = ld16<NT>(p);
  return r;
}
template <bool NT = false, typename T>
__device__ __forceinline__ void store16(T* p, const Vec16<T>& r) {
  st16<NT>(p, *reinterpret_cast<const uint4*>(&r));
}

// float4 access; NT = streaming.
__device__ __forceinline__ float4 ld_f4(const float* p) {
  return *reinterpret_cast<const float4*>(p);
}
__device__ __forceinline__ void st_f4(float* p, float4 v) {
  *reinterpret_cast<float4*>(p) = v;
}
__device__ __forceinline__ float4 ld_f4s(const float* p) {
  const uint4 u = ld16<true>(p);
  return make_float4(__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z),
                     __uint_as_float(u.w));
}
__device__ __forceinline__ void st_f4s(float* p, float4 v) {
  st16<true>(p, make_uint4(__float_as_uint(v.x), __float_as_uint(v.y), __float_as_uint(v.z),
                           __float_as_uint(v.w)));
}

// Branch-free select: v if keep, else +0.0 (bit mask, so NaN/Inf inputs are
// cleared as well).
__device__ __forceinline__ float keep_if(float v, bool keep) {
  return __uint_as_float(__float_as_uint(v) & (keep ? 0xffffffffu : 0u));
}
__device__ __forceinline__ float4 keep_if(float4 v, bool keep) {
  return make_float4(keep_if(v.x, keep), keep_if(v.y, keep),
                     keep_if(v.z, keep), keep_if(v.w, keep));
}

// Four consecutive elements of T (aligned to 4*sizeof(T)) widened to float.
__device__ __forceinline__ float4 load4f(const float* p) { return ld_f4(p); }
__device__ __forceinline__ float4 load4f(const __half* p) {
  const uint2 raw = *reinterpret_cast<const uint2*>(p);
  const __half2 lo = *reinterpret_cast<const __half2*>(&raw.x);
  const __half2 hi = *reinterpret_cast<const __half2*>(&raw.y);
  return make_float4(__low2float(lo), __high2float(lo), __low2float(hi),
                     __high2float(hi));
}
__device__ __forceinline__ float4 load4f(const __hip_bfloat16* p) {
  const uint2 raw = *reinterpret_cast<const uint2*>(p);
  // bf16 -> f32 is a 16-bit left shift of the bit pattern.
  return make_float4(__uint_as_float(raw.x << 16),
                     __uint_as_float(raw.x & 0xffff0000u),
                     __uint_as_float(raw.y << 16),
                     __uint_as_float(raw.y & 0xffff0000u));
}

// Fast sigmoid: v_exp_f32 (via __expf) and v_rcp_f32.  The kernels are
// memory bound only if their VALU work stays near a dozen ops per element;
// the correctly-rounded exp/divide sequences would double that.
__device__ __forceinline__ float fast_sigmoid(float g) {
  return __builtin_amdgcn_rcpf(1.0f + __expf(-g));
}

}  // namespace rv

// ---------------------------------------------------------------------------
// Host-side helpers (status plumbing, device properties).
// ---------------------------------------------------------------------------
namespace rv_host {

// Record a HIP error text for rv_last_error() and map to RV_ERR_HIP.
int hip_fail(hipError_t err);

// Check for a launch error right after a kernel launch.
int check_launch();

// Number of compute units of the current device (cached per device).
int cu_count();

inline bool aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

}  // namespace rv_host
