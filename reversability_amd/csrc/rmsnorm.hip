// Fused RMSNorm forward/backward for gfx950.
//
// Layout: x, y, dy, dx are [rows, width] FP32 row-major; w and dw are
// [width]; rstd is [rows].  A row belongs to a group of G lanes of one wave
// (G = 16 for width <= 256: four rows per wave, each lane holding VEC float4
// of its row at float4 indices v*16 + lane%16, so one load instruction reads
// four 256-byte row segments; G = 64 for wider rows: one row per wave, VEC
// float4 per lane).  The row sums are DPP reductions inside the group.
//
// Backward is a single pass over x and dy: every wave computes dx for its
// rows and accumulates dy * (x * rstd) per column in registers; the waves of
// a block combine through LDS and the block writes one contiguous partial row
// of dw ([nparts][width]).  A second small kernel sums each column's partials
// in a fixed order.
//
// Under fp16 autocast the normalized output's only consumers are fp16 GEMMs,
// which read it through autocast's fp16 cast; the _f16 entry points write that
// fp16 value directly (y rounded to nearest even, the cast's rounding) and take
// the incoming gradient as fp16 (the GEMM's fp16 product, which autocast widens
// to fp32 unchanged), so the results are bit-identical to the fp32 y / dy path
// followed by the cast, with half of y's and dy's bytes and no cast launch.
//
// Arithmetic follows src/reversibility/kernels_v3.py:9-48 operation by
// operation (sum/width + eps, x*r*w, g*x reduction, (g - x*c)*r, and the
// forward multiply order x*r inside the dweight sum); the build disables FMA
// contraction to match the reference's enable_fp_fusion=False.

#include <mutex>
#include <type_traits>

#include "rv_device.h"

namespace {

using rv::wave_sum;

// Launch shapes chosen by timing sweeps on MI355X at the configs' shapes
// (x [14848, 256] fp32), over > 1.5 GB of rotating buffers:
//   forward, width <= 256  16 lanes per row, one group of four rows per
//                          wave, a grid that covers every row (no loop):
//                          every load is in flight at once (C1: 7.6 -> 6.1 us
//                          against the one-row-per-wave persistent grid)
//   forward, wider rows    8 blocks of 4 waves per CU, persistent, one row per
//                          wave in flight
//   backward, width <= 256 the same layout, blocks of 4 waves x 4 .. 8 four-row
//                          groups, the rows spread evenly over 256 blocks (C1:
//                          256 blocks of 58 rows), every row of a block in
//                          flight at once (13.1 -> 11.9 us; even spread 11.85)
//   backward, wider rows   256 blocks of 4 .. 16 waves, ~128 rows per block
// Stores of y / dx are streaming.
#ifndef RV_RMS_FWD_BLOCKS_PER_CU
#define RV_RMS_FWD_BLOCKS_PER_CU 8
#endif
#ifndef RV_RMS_BWD_WAVES
#define RV_RMS_BWD_WAVES 16
#endif
#ifndef RV_RMS_BWD_BLOCKS
#define RV_RMS_BWD_BLOCKS 256
#endif



constexpr int kFwdWaves = 4;                 // waves per block, forward
constexpr int kBwdWaves = RV_RMS_BWD_WAVES;  // waves per block, backward (scalar path, width <= 512)
// Waves per backward block by vector count per lane (width <= 256 * VEC):
// 2 rows x (x, dy) x VEC float4 per register tile, two tiles in flight.
constexpr int bwd_waves(int vec) { return vec <= 2 ? kBwdWaves : (vec == 4 ? 8 : 4); }
// With dh accumulated the tiles are 1.5x larger: fewer waves, more registers
// each (no scratch at width 1024).  dweight's per-row terms are then summed in
// another fixed order (rows are dealt to waves by index) -- dx is unaffected.
constexpr int bwd_waves(int vec, bool acc) {
  return !acc ? bwd_waves(vec) : (vec <= 1 ? kBwdWaves : (vec == 2 ? 8 : 4));
}
constexpr int kMaxVec = 16;      // float4 per lane => width <= 4096
constexpr int kMaxEpl = 64;      // scalar path: elements per lane <= 64

// ---------------------------------------------------------------------------
// Forward, width % 4 == 0, width <= 4 * G * VEC.  A wave handles groups of
// 64/G consecutive rows (lane l works on row group_first + l/G).  Persistent
// (rms_fwd_vec): wave w of the grid handles groups w, w + W, w + 2W, ...
// (W = waves in the grid) and alternates between two register tiles, issuing
// the next group's loads before reducing the current one.  Rows past the end
// are clamped to the last row for loading (one cached line, no branch) and
// never stored.  With ADD the row input is
// x + float(f) (fused residual add) and that sum is also written to h.
// ---------------------------------------------------------------------------
// Four normalized values to y (fp32: one streaming 16-byte store; fp16:
// rounded to nearest even, one streaming 8-byte store).  The fp16 values are
// the fp32 products rounded once more: without the empty asm the compiler
// folds "fp16(a * b)" into v_fma_mixlo_f16, a single rounding of the exact
// product, which differs from autocast's cast of the fp32 y.
__device__ __forceinline__ void store_y(float* p, float4 v) { rv::st_f4s(p, v); }
__device__ __forceinline__ void store_y(__half* p, float4 v) {
  typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
  asm volatile("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w));
  const uint32_t lo = (uint32_t)__half_as_ushort(__float2half_rn(v.x)) |
                      ((uint32_t)__half_as_ushort(__float2half_rn(v.y)) << 16);
  const uint32_t hi = (uint32_t)__half_as_ushort(__float2half_rn(v.z)) |
                      ((uint32_t)__half_as_ushort(__float2half_rn(v.w)) << 16);
  __builtin_nontemporal_store(u32x2{lo, hi}, reinterpret_cast<u32x2*>(p));
}

// Lane l's first column of its row's float4 number v (G lanes per row).
template <int G>
__device__ __forceinline__ int lane_col(int v, int lane) {
  return (v * G + (lane & (G - 1))) * 4;
}

// TWO: a second force operand g (the midpoint update's M(...) beside f = A(...)).
template <int VEC, typename F, bool ADD, bool TWO = false>
struct RowTile {
  float4 x[VEC];
  float4 f[ADD ? VEC : 1];
  float4 g[TWO ? VEC : 1];
};

// FULL: width == 4 * G * VEC (no column clamp).
template <int VEC, int G, bool FULL = false, typename F, bool ADD, bool TWO>
__device__ __forceinline__ void rms_load(RowTile<VEC, F, ADD, TWO>& t,
                                         const float* __restrict__ x, const F* __restrict__ f,
                                         int64_t row0, int64_t rows, int width, int lane,
                                         const F* __restrict__ g = nullptr) {
  const int64_t r = row0 + lane / G;
  const int64_t row = r < rows ? r : rows - 1;
#pragma unroll
  for (int v = 0; v < VEC; ++v) {
    const int col = lane_col<G>(v, lane);
    const int col_c = FULL || col < width ? col : width - 4;
    t.x[v] = rv::ld_f4(x + row * width + col_c);
    if constexpr (ADD) t.f[v] = rv::load4f(f + row * width + col_c);
    if constexpr (TWO) t.g[v] = rv::load4f(g + row * width + col_c);
  }
}

// The midpoint update of one element with the eager expression's rounding
// points (fp16 force): c = fp16(fp16(a + m) * scale), x +/- c.  The empty asm
// keeps the fp32 product from being folded into a mixed-precision FMA that
// would round the exact product to fp16 once.
__device__ __forceinline__ float midpoint_elem(float x, float a, float m, float scale, int sign) {
  const float fsum = __half2float(__float2half_rn(a + m));
  float prod = fsum * scale;
  asm volatile("" : "+v"(prod));
  const float c = __half2float(__float2half_rn(prod));
  return sign > 0 ? x + c : x - c;
}

// SUBM (with ADD): 0 -- the row input is x + f; 1 -- it is x - f; 2 -- d = x - f
// is stored and the row input is d + f; 3 -- it is the midpoint update of x
// with the force terms f and g (midpoint_elem).  The row input is stored in h
// for every SUBM but 0 without h.
// FULL: width == 4 * G * VEC (every lane's columns exist: no column masks, and
// the stores sit under the row predicate alone).
template <int VEC, int G, typename F, bool ADD, typename Y, int SUBM = 0, bool FULL = false>
__device__ __forceinline__ void rms_finish(RowTile<VEC, F, ADD, SUBM == 3>& t,
                                           const float4 (&wv)[VEC],
                                           float* __restrict__ h, Y* __restrict__ y,
                                           float* __restrict__ rstd, int64_t row0, int64_t rows,
                                           int width, float eps, int lane,
                                           float* __restrict__ d = nullptr, float scale = 0.f,
                                           int sign = 1) {
  const int64_t row = row0 + lane / G;
  float ss = 0.f;
#pragma unroll
  for (int v = 0; v < VEC; ++v) {
    const bool ok = FULL || lane_col<G>(v, lane) < width;
    if constexpr (ADD && SUBM == 0) {
      t.x[v].x = t.x[v].x + t.f[v].x;
      t.x[v].y = t.x[v].y + t.f[v].y;
      t.x[v].z = t.x[v].z + t.f[v].z;
      t.x[v].w = t.x[v].w + t.f[v].w;
    } else if constexpr (ADD && SUBM == 3) {
      t.x[v].x = midpoint_elem(t.x[v].x, t.f[v].x, t.g[v].x, scale, sign);
      t.x[v].y = midpoint_elem(t.x[v].y, t.f[v].y, t.g[v].y, scale, sign);
      t.x[v].z = midpoint_elem(t.x[v].z, t.f[v].z, t.g[v].z, scale, sign);
      t.x[v].w = midpoint_elem(t.x[v].w, t.f[v].w, t.g[v].w, scale, sign);
    } else if constexpr (ADD) {
      t.x[v].x = t.x[v].x - t.f[v].x;
      t.x[v].y = t.x[v].y - t.f[v].y;
      t.x[v].z = t.x[v].z - t.f[v].z;
      t.x[v].w = t.x[v].w - t.f[v].w;
      if constexpr (SUBM == 2) {
        if (row < rows && ok) rv::st_f4s(d + row * width + lane_col<G>(v, lane), t.x[v]);
        t.x[v].x = t.x[v].x + t.f[v].x;
        t.x[v].y = t.x[v].y + t.f[v].y;
        t.x[v].z = t.x[v].z + t.f[v].z;
        t.x[v].w = t.x[v].w + t.f[v].w;
      }
    }
    const float4 q = rv::keep_if(t.x[v], ok);
    ss = ss + q.x * q.x;
    ss = ss + q.y * q.y;
    ss = ss + q.z * q.z;
    ss = ss + q.w * q.w;
  }
  ss = rv::group_sum<G>(ss);
  const float rs = rsqrtf(ss / (float)width + eps);
  float4 o[VEC];
#pragma unroll
  for (int v = 0; v < VEC; ++v) {
    const float4 q = t.x[v];
    o[v].x = (q.x * rs) * wv[v].x;
    o[v].y = (q.y * rs) * wv[v].y;
    o[v].z = (q.z * rs) * wv[v].z;
    o[v].w = (q.w * rs) * wv[v].w;
  }
  const bool row_ok = row < rows;
  if constexpr (FULL) {
    if (row_ok) {
#pragma unroll
      for (int v = 0; v < VEC; ++v) {
        const int col = lane_col<G>(v, lane);
        store_y(y + row * width + col, o[v]);
        if constexpr (ADD) rv::st_f4s(h + row * width + col, t.x[v]);
      }
      if ((lane & (G - 1)) == 0) rstd[row] = rs;
    }
  } else {
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      const int col = lane_col<G>(v, lane);
      if (row_ok && col < width) {
        store_y(y + row * width + col, o[v]);
        if constexpr (ADD) rv::st_f4s(h + row * width + col, t.x[v]);
      }
    }
    if (row_ok && (lane & (G - 1)) == 0) rstd[row] = rs;
  }
}

// One four-row group per wave, 16 lanes per row (width <= 256), no loop: the
// grid covers every row and each wave's row loads are its first memory
// instructions, so every row load of the launch is in flight at once.
// FULL (width = 64 VEC): the weight loads follow the row sum (the compiler
// places them in the store branch): 3712 waves loading the same 1 KiB of w
// together with their rows made every wave wait on those few L2 lines (C1:
// 7.15 us with w loaded beside x, 6.84 staged once per block through LDS, 6.3
// after the row sum).  Other widths keep w beside x: an empty asm consumes it
// there, or the compiler would sink each column's weight load into that
// column's store branch, one round trip after another.
template <int VEC, bool FULL, typename F, bool ADD, typename Y, int SUBM = 0>
__global__ __launch_bounds__(kFwdWaves * 64)
void rms_fwd_grp(const float* __restrict__ x, const F* __restrict__ f,
                 const float* __restrict__ w, float* __restrict__ h,
                 Y* __restrict__ y, float* __restrict__ rstd,
                 int64_t rows, int width, float eps, float* __restrict__ d = nullptr,
                 const F* __restrict__ g = nullptr, float scale = 0.f, int sign = 1) {
  const int lane = threadIdx.x & 63;
  const int64_t row0 = ((int64_t)blockIdx.x * kFwdWaves + (threadIdx.x >> 6)) * 4;
  if (row0 >= rows) return;  // wave-uniform
  RowTile<VEC, F, ADD, SUBM == 3> a;
  rms_load<VEC, 16, FULL>(a, x, f, row0, rows, width, lane, g);
  // the row loads all issued before the row sum starts waiting on them
  __builtin_amdgcn_sched_barrier(0);
  float4 wv[VEC];
#pragma unroll
  for (int v = 0; v < VEC; ++v) {
    const int col = lane_col<16>(v, lane);
    wv[v] = rv::ld_f4(w + (FULL ? col : (col < width ? col : width - 4)));
  }
  if constexpr (!FULL) {
#pragma unroll
    for (int v = 0; v < VEC; ++v)
      asm volatile("" ::"v"(wv[v].x), "v"(wv[v].y), "v"(wv[v].z), "v"(wv[v].w));
    __builtin_amdgcn_sched_barrier(0);
  }
  rms_finish<VEC, 16, F, ADD, Y, SUBM, FULL>(a, wv, h, y, rstd, row0, rows, width, eps, lane,
                                             d, scale, sign);
}

template <int VEC, int G, typename F, bool ADD, typename Y, int SUBM = 0>
__global__ __launch_bounds__(kFwdWaves * 64)
void rms_fwd_vec(const float* __restrict__ x, const F* __restrict__ f,
                 const float* __restrict__ w, float* __restrict__ h,
                 Y* __restrict__ y, float* __restrict__ rstd,
                 int64_t rows, int width, float eps, float* __restrict__ d = nullptr,
                 const F* __restrict__ g = nullptr, float scale = 0.f, int sign = 1) {
  constexpr int RW = 64 / G;  // rows per wave group
  const int lane = threadIdx.x & 63;
  const int64_t nwaves = (int64_t)gridDim.x * kFwdWaves;
  const int64_t wave = (int64_t)blockIdx.x * kFwdWaves + (threadIdx.x >> 6);
  const int64_t groups = (rows + RW - 1) / RW;
  if (wave >= groups) return;  // wave-uniform
  const int64_t iters = (groups - 1 - wave) / nwaves + 1;

  // w of a column >= width only meets outputs that are never stored.
  float4 wv[VEC];
#pragma unroll
  for (int v = 0; v < VEC; ++v) {
    const int col = lane_col<G>(v, lane);
    wv[v] = rv::ld_f4(w + (col < width ? col : width - 4));
  }
  const int64_t stride = nwaves * RW;
  int64_t row0 = wave * RW;
  RowTile<VEC, F, ADD, SUBM == 3> a, b;
  rms_load<VEC, G>(a, x, f, row0, rows, width, lane, g);
  for (int64_t k = 0; k < iters; k += 2) {
    rms_load<VEC, G>(b, x, f, row0 + stride, rows, width, lane, g);
    rms_finish<VEC, G, F, ADD, Y, SUBM>(a, wv, h, y, rstd, row0, rows, width, eps, lane, d,
                                        scale, sign);
    if (k + 1 >= iters) break;
    row0 += stride;
    rms_load<VEC, G>(a, x, f, row0 + stride, rows, width, lane, g);
    rms_finish<VEC, G, F, ADD, Y, SUBM>(b, wv, h, y, rstd, row0, rows, width, eps, lane, d,
                                        scale, sign);
    row0 += stride;
  }
}

// ---------------------------------------------------------------------------
// Forward, any width <= 64 * EPL (scalar, element j of a lane is column
// j*64 + lane).
// ---------------------------------------------------------------------------
template <int EPL, typename F, bool ADD>
__global__ __launch_bounds__(kFwdWaves * 64)
void rms_fwd_scalar(const float* __restrict__ x, const F* __restrict__ f,
                    const float* __restrict__ w, float* __restrict__ h,
                    float* __restrict__ y, float* __restrict__ rstd,
                    int64_t rows, int width, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kFwdWaves + (threadIdx.x >> 6);
  if (row >= rows) return;
  float xv[EPL];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int col = j * 64 + lane;
    float t = 0.f;
    if (col < width) {
      t = x[row * width + col];
      if constexpr (ADD) t = t + rv::Conv<F>::to_f(f[row * width + col]);
    }
    xv[j] = t;
    ss = ss + t * t;
  }
  ss = wave_sum(ss);
  const float rs = rsqrtf(ss / (float)width + eps);
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int col = j * 64 + lane;
    if (col < width) {
      y[row * width + col] = (xv[j] * rs) * w[col];
      if constexpr (ADD) h[row * width + col] = xv[j];
    }
  }
  if (lane == 0) rstd[row] = rs;
}

// ---------------------------------------------------------------------------
// Backward, width % 4 == 0.  Block b owns rows [b*rpb, min((b+1)*rpb, rows)).
// Wave k of the block handles row pairs start + 2k, start + 2k + 2*WAVES, ...
// alternating between two register tiles (the next pair's loads are issued
// before the current pair is reduced).  Writes dx and the block's dw partial
// as one contiguous row, partial[block * width + col].
// ---------------------------------------------------------------------------
// ACC: the row gradient also receives dh (the gradient of the normalized
// input's other use: dx = dh + norm backward, the sum autograd would form).
// PASS: the input also has a pass-through use whose gradient dpass joins dx
// after the fp16 copy (that copy is the force term's gradient, which does not
// include it).
template <int VEC, bool ACC, bool PASS = false>
struct BwdTile {
  float4 x[2][VEC], g[2][VEC];
  float4 h[ACC ? 2 : 1][ACC ? VEC : 1];
  float4 p[PASS ? 2 : 1][PASS ? VEC : 1];
  float rs[2];
};

// The fp32 rows (x, dh, dpass) with streaming loads: C5's width-1024
// accumulating backward on rotating cold buffers 105.6 -> 93.3 us (dx16
// written too), 91.5 -> 78.3 us; inside the C5 training step, where dh was
// just written, the step time did not move (85.7 ms either way).
template <int VEC, bool ACC, bool PASS, typename G>
__device__ __forceinline__ void bwd_load(BwdTile<VEC, ACC, PASS>& t, const float* __restrict__ x,
                                         const G* __restrict__ dy,
                                         const float* __restrict__ rstd,
                                         const float* __restrict__ dh,
                                         const float* __restrict__ dpass, int64_t row0,
                                         int64_t end, int width, int lane) {
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int64_t row = row0 + r < end ? row0 + r : end - 1;  // clamped, valid
    t.rs[r] = rstd[row];
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      const int col = (v * 64 + lane) * 4;
      const int col_c = col < width ? col : width - 4;
      t.x[r][v] = rv::ld_f4s(x + row * width + col_c);
      t.g[r][v] = rv::load4f(dy + row * width + col_c);
      if constexpr (ACC) t.h[r][v] = rv::ld_f4s(dh + row * width + col_c);
      if constexpr (PASS) t.p[r][v] = rv::ld_f4s(dpass + row * width + col_c);
    }
  }
}

template <int VEC, bool ACC, bool H16, bool PASS>
__device__ __forceinline__ void bwd_finish(BwdTile<VEC, ACC, PASS>& t, const float4 (&wv)[VEC],
                                           float4 (&acc)[VEC], float* __restrict__ dx,
                                           __half* __restrict__ dx16,
                                           int64_t row0, int64_t end, int width, int lane) {
  const float fwidth = (float)width;
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int64_t row = row0 + r;
    const bool row_ok = row < end;
    const float rs = rv::keep_if(t.rs[r], row_ok);
    float dot = 0.f;
    float4 g[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      const bool ok = row_ok && (v * 64 + lane) * 4 < width;
      t.x[r][v] = rv::keep_if(t.x[r][v], ok);
      t.g[r][v] = rv::keep_if(t.g[r][v], ok);
      g[v].x = t.g[r][v].x * wv[v].x;
      g[v].y = t.g[r][v].y * wv[v].y;
      g[v].z = t.g[r][v].z * wv[v].z;
      g[v].w = t.g[r][v].w * wv[v].w;
      dot = dot + g[v].x * t.x[r][v].x;
      dot = dot + g[v].y * t.x[r][v].y;
      dot = dot + g[v].z * t.x[r][v].z;
      dot = dot + g[v].w * t.x[r][v].w;
    }
    dot = wave_sum(dot);
    const float c = ((dot / fwidth) * rs) * rs;
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      const float4 q = t.x[r][v];
      // dweight partial: dy * (x * r), forward multiply order.
      acc[v].x = acc[v].x + t.g[r][v].x * (q.x * rs);
      acc[v].y = acc[v].y + t.g[r][v].y * (q.y * rs);
      acc[v].z = acc[v].z + t.g[r][v].z * (q.z * rs);
      acc[v].w = acc[v].w + t.g[r][v].w * (q.w * rs);
      const int col = (v * 64 + lane) * 4;
      if (row_ok && col < width) {
        float4 o;
        o.x = (g[v].x - q.x * c) * rs;
        o.y = (g[v].y - q.y * c) * rs;
        o.z = (g[v].z - q.z * c) * rs;
        o.w = (g[v].w - q.w * c) * rs;
        if constexpr (ACC) {
          o.x = o.x + t.h[r][v].x;
          o.y = o.y + t.h[r][v].y;
          o.z = o.z + t.h[r][v].z;
          o.w = o.w + t.h[r][v].w;
        }
        if constexpr (H16) store_y(dx16 + row * width + col, o);
        if constexpr (PASS) {
          o.x = o.x + t.p[r][v].x;
          o.y = o.y + t.p[r][v].y;
          o.z = o.z + t.p[r][v].z;
          o.w = o.w + t.p[r][v].w;
        }
        rv::st_f4s(dx + row * width + col, o);
      }
    }
  }
}

// WAVES per block: wide rows keep fewer waves so that their two-row
// ping-pong tiles stay in registers (no scratch).
template <int VEC, int WAVES, typename G, bool ACC = false, bool H16 = false, bool PASS = false>
__global__ __launch_bounds__(WAVES * 64)
void rms_bwd_vec(const float* __restrict__ x, const float* __restrict__ w,
                 const G* __restrict__ dy, const float* __restrict__ rstd,
                 float* __restrict__ dx, float* __restrict__ partial,
                 int64_t rows, int width, int64_t rows_per_block,
                 const float* __restrict__ dh = nullptr, __half* __restrict__ dx16 = nullptr,
                 const float* __restrict__ dpass = nullptr) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t start = (int64_t)blockIdx.x * rows_per_block;
  const int64_t end = start + rows_per_block < rows ? start + rows_per_block : rows;

  float4 wv[VEC];
  float4 acc[VEC];
#pragma unroll
  for (int v = 0; v < VEC; ++v) {
    const int col = (v * 64 + lane) * 4;
    wv[v] = rv::keep_if(rv::ld_f4(w + (col < width ? col : width - 4)), col < width);
    acc[v] = make_float4(0.f, 0.f, 0.f, 0.f);
  }

  const int64_t first = start + 2 * wave;
  const int64_t stride = 2 * WAVES;
  if (first < end) {  // wave-uniform
    const int64_t iters = (end - 1 - first) / stride + 1;
    int64_t row0 = first;
    BwdTile<VEC, ACC, PASS> a, b;
    bwd_load(a, x, dy, rstd, dh, dpass, row0, end, width, lane);
    for (int64_t k = 0; k < iters; k += 2) {
      bwd_load(b, x, dy, rstd, dh, dpass, row0 + stride, end, width, lane);
      bwd_finish<VEC, ACC, H16, PASS>(a, wv, acc, dx, dx16, row0, end, width, lane);
      if (k + 1 >= iters) break;
      row0 += stride;
      bwd_load(a, x, dy, rstd, dh, dpass, row0 + stride, end, width, lane);
      bwd_finish<VEC, ACC, H16, PASS>(b, wv, acc, dx, dx16, row0, end, width, lane);
      row0 += stride;
    }
  }

  // Combine the waves' column partials in wave order, at most 4 float4 per
  // lane per pass.
  constexpr int kPass = VEC < 4 ? VEC : 4;
  __shared__ float4 red[WAVES][kPass * 64];
#pragma unroll
  for (int v0 = 0; v0 < VEC; v0 += kPass) {
#pragma unroll
    for (int v = 0; v < kPass; ++v) red[wave][v * 64 + lane] = acc[v0 + v];
    __syncthreads();
    for (int s = threadIdx.x; s < kPass * 64; s += WAVES * 64) {
      float4 t = red[0][s];
#pragma unroll
      for (int k = 1; k < WAVES; ++k) {
        t.x = t.x + red[k][s].x;
        t.y = t.y + red[k][s].y;
        t.z = t.z + red[k][s].z;
        t.w = t.w + red[k][s].w;
      }
      const int col = (v0 * 64 + s) * 4;
      if (col < width) rv::st_f4(partial + (int64_t)blockIdx.x * width + col, t);
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Backward, width % 4 == 0 and width <= 256: the forward's 16-lanes-per-row
// layout (four rows per wave, lane l on row l/16 of its group, float4 number
// v*16 + l%16 of the row).  Block b owns rows [b*R, min((b+1)*R, rows)),
// R = ceil(rows / 256) (16 .. 128): the rows spread evenly over 256 blocks,
// one per compute unit (C1: 256 blocks of 58 rows), so no compute unit streams
// two blocks' rows while others idle.  The block's 4 NG four-row slots (NG =
// 4, 5, 6 or 8, the fewest with 16 NG >= R; slots past R are masked) are
// dealt to the four waves round-robin, and each wave issues the loads of its
// NG groups before finishing any of them: every row of the block is in
// flight at once.  dweight per column: each lane sums its own rows in order,
// then the block sums (wave, row-in-group) in order through LDS and writes
// one contiguous partial row.
// ---------------------------------------------------------------------------
template <int VEC, bool ACC, bool PASS>
struct GrpTile {
  float4 x[VEC], g[VEC];
  float4 h[ACC ? VEC : 1];
  float4 p[PASS ? VEC : 1];
  float rs;
};

constexpr int kGrpWaves = 4;    // waves per block
constexpr int kGrpMinLoads = 4;  // four-row groups in flight per wave: 4 .. 8,
constexpr int kGrpMaxLoads = 8;  // the fewest that keep the grid at <= 256 blocks

// Loads of group k of the block: rows base + (k * kGrpWaves + wave) * 4 + lane/16,
// clamped to end - 1; addresses are block-uniform base pointers plus 32-bit
// lane offsets (a block's 16 NG rows).  The backward is the last reader of the
// fp32 rows and of an fp32 dy: streaming loads (x: C1 12.3 -> 11.95 us, dy as
// well: 11.77 -> 11.51 us; the forward keeps plain loads, whose lines the
// backward of the same batch may still find cached).  dx stores are streaming
// too (plain stores: 11.77 -> 14.07 us).
template <int VEC, int NG, bool FULL, typename G, bool ACC, bool PASS>
__device__ __forceinline__ void grp_load(GrpTile<VEC, ACC, PASS> (&t)[NG],
                                         const float* __restrict__ x, const G* __restrict__ dy,
                                         const float* __restrict__ rstd,
                                         const float* __restrict__ dh,
                                         const float* __restrict__ dpass, int64_t base,
                                         int64_t end, int width, int wave, int lane) {
  const int nrows = (int)(end - base);  // 1 .. 16 NG
  const float* xb = x + base * width;
  const G* gb = dy + base * width;
  const float* hb = ACC ? dh + base * width : nullptr;
  const float* pb = PASS ? dpass + base * width : nullptr;
#pragma unroll
  for (int k = 0; k < NG; ++k) {
    const int r = (k * kGrpWaves + wave) * 4 + (lane >> 4);
    const int rc = r < nrows ? r : nrows - 1;  // clamped, valid
    t[k].rs = rstd[base + rc];
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      const int col = lane_col<16>(v, lane);
      const unsigned off = (unsigned)(rc * width + (FULL || col < width ? col : width - 4));
      t[k].x[v] = rv::ld_f4s(xb + off);
      if constexpr (std::is_same<G, float>::value) t[k].g[v] = rv::ld_f4s(gb + off);
      else t[k].g[v] = rv::load4f(gb + off);
      if constexpr (ACC) t[k].h[v] = rv::ld_f4s(hb + off);
      if constexpr (PASS) t[k].p[v] = rv::ld_f4s(pb + off);
    }
  }
}

template <int VEC, int NG, bool FULL, typename G, bool ACC, bool H16, bool PASS>
__global__ __launch_bounds__(kGrpWaves * 64)
void rms_bwd_grp(const float* __restrict__ x, const float* __restrict__ w,
                 const G* __restrict__ dy, const float* __restrict__ rstd,
                 float* __restrict__ dx, float* __restrict__ partial,
                 int64_t rows, int width, int rows_per_block,
                 const float* __restrict__ dh = nullptr, __half* __restrict__ dx16 = nullptr,
                 const float* __restrict__ dpass = nullptr) {
  constexpr int GL = 16;  // lanes per row
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int sub = lane >> 4;
  // rows_per_block <= kGrpWaves * NG * 4 (the plan picks NG so); slots past
  // the block's rows load a valid row and are masked out
  const int64_t start = (int64_t)blockIdx.x * rows_per_block;
  const int64_t end = start + rows_per_block < rows ? start + rows_per_block : rows;
  const float fwidth = (float)width;

  // The weight is staged once per block through LDS: wave 0 loads it ahead of
  // its row loads (a few L2 lines that every block reads: loaded by every wave
  // beside its rows they held each wave's first wait), every wave then issues
  // all of its row loads, and the block meets at one barrier before the row
  // math (w of a column >= width only meets masked values).
  __shared__ float4 wlds[VEC * GL];
  float4 wr[VEC];
  if (wave == 0) {
#pragma unroll
    for (int v = 0; v < VEC; ++v)
      if (v * 64 + lane < VEC * GL) {
        const int col = (v * 64 + lane) * 4;
        wr[v] = rv::ld_f4(w + (FULL || col < width ? col : width - 4));
      }
  }
  GrpTile<VEC, ACC, PASS> t[NG];
  grp_load<VEC, NG, FULL, G, ACC, PASS>(t, x, dy, rstd, dh, dpass, start, end, width, wave,
                                        lane);
  // every row load issued before the first wait (the scheduler would otherwise
  // interleave the first group's math, and its waits, with the later loads)
  __builtin_amdgcn_sched_barrier(0);
  if (wave == 0) {
#pragma unroll
    for (int v = 0; v < VEC; ++v)
      if (v * 64 + lane < VEC * GL) wlds[v * 64 + lane] = wr[v];
  }
  __syncthreads();
  float4 wv[VEC], acc[VEC];
#pragma unroll
  for (int v = 0; v < VEC; ++v) {
    wv[v] = wlds[v * GL + (lane & (GL - 1))];
    acc[v] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
  {
    const int nrows = (int)(end - start);  // 1 .. rows_per_block
    float* dxb = dx + start * width;
    __half* d16b = H16 ? dx16 + start * width : nullptr;
#pragma unroll
    for (int k = 0; k < NG; ++k) {
      const int r = (k * kGrpWaves + wave) * 4 + sub;
      const bool row_ok = r < nrows;
      const float rs = rv::keep_if(t[k].rs, row_ok);
      float dot = 0.f;
      float4 g[VEC];
#pragma unroll
      for (int v = 0; v < VEC; ++v) {
        const bool ok = row_ok && (FULL || lane_col<GL>(v, lane) < width);
        t[k].x[v] = rv::keep_if(t[k].x[v], ok);
        t[k].g[v] = rv::keep_if(t[k].g[v], ok);
        g[v].x = t[k].g[v].x * wv[v].x;
        g[v].y = t[k].g[v].y * wv[v].y;
        g[v].z = t[k].g[v].z * wv[v].z;
        g[v].w = t[k].g[v].w * wv[v].w;
        g[v] = rv::keep_if(g[v], ok);
        dot = dot + g[v].x * t[k].x[v].x;
        dot = dot + g[v].y * t[k].x[v].y;
        dot = dot + g[v].z * t[k].x[v].z;
        dot = dot + g[v].w * t[k].x[v].w;
      }
      dot = rv::group_sum<GL>(dot);
      const float c = ((dot / fwidth) * rs) * rs;
#pragma unroll
      for (int v = 0; v < VEC; ++v) {
        const float4 q = t[k].x[v];
        // dweight partial: dy * (x * r), forward multiply order.
        acc[v].x = acc[v].x + t[k].g[v].x * (q.x * rs);
        acc[v].y = acc[v].y + t[k].g[v].y * (q.y * rs);
        acc[v].z = acc[v].z + t[k].g[v].z * (q.z * rs);
        acc[v].w = acc[v].w + t[k].g[v].w * (q.w * rs);
        const int col = lane_col<GL>(v, lane);
        if (row_ok && (FULL || col < width)) {
          const unsigned off = (unsigned)(r * width + col);
          float4 o;
          o.x = (g[v].x - q.x * c) * rs;
          o.y = (g[v].y - q.y * c) * rs;
          o.z = (g[v].z - q.z * c) * rs;
          o.w = (g[v].w - q.w * c) * rs;
          if constexpr (ACC) {
            o.x = o.x + t[k].h[v].x;
            o.y = o.y + t[k].h[v].y;
            o.z = o.z + t[k].h[v].z;
            o.w = o.w + t[k].h[v].w;
          }
          if constexpr (H16) store_y(d16b + off, o);
          if constexpr (PASS) {
            o.x = o.x + t[k].p[v].x;
            o.y = o.y + t[k].p[v].y;
            o.z = o.z + t[k].p[v].z;
            o.w = o.w + t[k].p[v].w;
          }
          rv::st_f4s(dxb + off, o);
        }
      }
    }
  }

  // Column partials of the block's (wave, row-in-group) slots, summed in slot
  // order: slot s = wave * 4 + sub holds float4 number v*16 + l%16 at [s][v*16 + l%16].
  __shared__ float4 red[kGrpWaves * 4][VEC * GL];
#pragma unroll
  for (int v = 0; v < VEC; ++v) red[wave * 4 + sub][v * GL + (lane & (GL - 1))] = acc[v];
  __syncthreads();
  const int s = threadIdx.x;
  if (s < VEC * GL) {
    float4 q[kGrpWaves * 4];
#pragma unroll
    for (int k = 0; k < kGrpWaves * 4; ++k) q[k] = red[k][s];
    float4 tsum = q[0];
#pragma unroll
    for (int k = 1; k < kGrpWaves * 4; ++k) {
      tsum.x = tsum.x + q[k].x;
      tsum.y = tsum.y + q[k].y;
      tsum.z = tsum.z + q[k].z;
      tsum.w = tsum.w + q[k].w;
    }
    const int col = s * 4;  // float4 number s of the row
    if (col < width) rv::st_f4(partial + (int64_t)blockIdx.x * width + col, tsum);
  }
}

// ---------------------------------------------------------------------------
// Backward, any width <= 64 * EPL (scalar).  Same structure as the vector
// kernel; element j of a lane is column j*64 + lane.
// ---------------------------------------------------------------------------
template <int EPL>
__global__ __launch_bounds__(kBwdWaves * 64)
void rms_bwd_scalar(const float* __restrict__ x, const float* __restrict__ w,
                    const float* __restrict__ dy, const float* __restrict__ rstd,
                    float* __restrict__ dx, float* __restrict__ partial,
                    int64_t rows, int width, int64_t rows_per_block) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t start = (int64_t)blockIdx.x * rows_per_block;
  const int64_t end = start + rows_per_block < rows ? start + rows_per_block : rows;
  float wv[EPL], acc[EPL];
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int col = j * 64 + lane;
    wv[j] = col < width ? w[col] : 0.f;
    acc[j] = 0.f;
  }
  for (int64_t row = start + wave; row < end; row += kBwdWaves) {
    const float rs = rstd[row];
    float xv[EPL], gv[EPL], g[EPL];
    float dot = 0.f;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      const int col = j * 64 + lane;
      xv[j] = col < width ? x[row * width + col] : 0.f;
      gv[j] = col < width ? dy[row * width + col] : 0.f;
      g[j] = gv[j] * wv[j];
      dot = dot + g[j] * xv[j];
    }
    dot = wave_sum(dot);
    const float c = ((dot / (float)width) * rs) * rs;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      const int col = j * 64 + lane;
      acc[j] = acc[j] + gv[j] * (xv[j] * rs);
      if (col < width) dx[row * width + col] = (g[j] - xv[j] * c) * rs;
    }
  }
  __shared__ float red[kBwdWaves][64];
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    red[wave][lane] = acc[j];
    __syncthreads();
    if (threadIdx.x < 64) {
      float t = red[0][threadIdx.x];
#pragma unroll
      for (int k = 1; k < kBwdWaves; ++k) t = t + red[k][threadIdx.x];
      const int col = j * 64 + threadIdx.x;
      if (col < width) partial[(int64_t)blockIdx.x * width + col] = t;
    }
    __syncthreads();
  }
}

// dw[col] = sum over parts of partial[part][col] (row-major, one contiguous
// row per backward block).  A block covers kRedCols columns with kRedGroups
// groups of kRedCols threads (thread = group * kRedCols + column): group g
// sums parts g, g + kRedGroups, ... in order, in batches of kRedPerGroup parts
// whose loads are all issued before the batch's first add (one memory round
// trip per batch), then the groups' sums are added in group order through
// LDS.  Fixed order throughout.  Narrow blocks spread the partial rows' reads
// over many compute units: at width 256, 32 blocks of 8 KB each (C1 backward
// with its reduce 11.51 -> 11.20 us against 4 blocks of 64 columns, one CU
// pulling 64 KB; 16 or 32 columns per block 11.29).
constexpr int kRedGroups = 16;
constexpr int kRedCols = 8;
constexpr int kRedPerGroup = 16;

__global__ __launch_bounds__(kRedGroups * kRedCols)
void rms_dw_reduce(const float* __restrict__ partial, float* __restrict__ dw,
                   int width, int nparts) {
  const int g = threadIdx.x / kRedCols, cl = threadIdx.x % kRedCols;
  const int col = blockIdx.x * kRedCols + cl;
  const int col_c = col < width ? col : width - 1;
  float s = 0.f;
  for (int p0 = 0; p0 < nparts; p0 += kRedGroups * kRedPerGroup) {
    float v[kRedPerGroup];
#pragma unroll
    for (int i = 0; i < kRedPerGroup; ++i) {
      const int part = p0 + g + i * kRedGroups;
      v[i] = partial[(int64_t)(part < nparts ? part : nparts - 1) * width + col_c];
    }
#pragma unroll
    for (int i = 0; i < kRedPerGroup; ++i)
      if (p0 + g + i * kRedGroups < nparts) s = s + v[i];
  }
  __shared__ float red[kRedGroups][kRedCols];
  red[g][cl] = s;
  __syncthreads();
  if (threadIdx.x < kRedCols) {
    float t = red[0][cl];
#pragma unroll
    for (int k = 1; k < kRedGroups; ++k) t = t + red[k][cl];
    if (col < width) dw[col] = t;
  }
}

// ---------------------------------------------------------------------------
// Launch plumbing
// ---------------------------------------------------------------------------
struct BwdPlan {
  int64_t rows_per_block;
  int nparts;  // backward blocks = partial rows
};

// Wide rows (width > 256): 256 blocks = one per compute unit on a 256-CU
// MI355X, all resident at once, every block with the same number of rows (no
// partial second wave of blocks).  Rows of width <= 256 (rms_bwd_grp): 256
// blocks of ceil(rows / 256) rows (at least 16, at most 128: more blocks
// beyond 32768 rows).  The counts depend on rows and width only, not on the
// device, so the dw summation order -- and therefore dw bit for bit -- does
// not depend on the device.  (Reducing the partials inside the backward
// kernel instead -- the last block to finish sums them -- needs device-scope
// release/acquire fences, which write back the per-XCD L2 on MI355X and
// measured 4-15x slower than this second launch.)
constexpr int64_t kBwdTargetBlocks = RV_RMS_BWD_BLOCKS;

// Whether the backward of this width runs rms_bwd_grp (when the pointers allow
// the vector path): the partial-row plan depends on it.
constexpr bool bwd_narrow(int64_t width) { return width <= 256; }

// Rows per block of rms_bwd_grp: the rows spread evenly over
// kBwdTargetBlocks blocks (every compute unit of a 256-CU MI355X gets one
// block), at least 16 and at most kGrpWaves * 4 * kGrpMaxLoads = 128 rows per
// block (more blocks beyond 32768 rows).  C1: 14848 rows -> 256 blocks of 58
// rows (232 blocks of 64 rows left 24 CUs idle: backward 11.99-12.04 ->
// 11.85-11.86 us).
int64_t grp_rows_per_block(int64_t rows) {
  int64_t rpb = (rows + kBwdTargetBlocks - 1) / kBwdTargetBlocks;
  if (rpb < 16) rpb = 16;
  if (rpb > kGrpWaves * 4 * kGrpMaxLoads) rpb = kGrpWaves * 4 * kGrpMaxLoads;
  return rpb;
}

// Four-row groups per wave of rms_bwd_grp holding a block of rpb rows: 4, 5,
// 6 or 8 (the instantiated counts), the fewest with kGrpWaves * 4 * NG >= rpb.
int grp_loads(int64_t rpb) {
  const int64_t per_wave = (rpb + kGrpWaves * 4 - 1) / (kGrpWaves * 4);
  if (per_wave <= kGrpMinLoads) return kGrpMinLoads;
  if (per_wave <= 6) return (int)per_wave;
  return kGrpMaxLoads;
}

BwdPlan plan_bwd(int64_t rows, int64_t width) {
  int64_t rpb = bwd_narrow(width) ? grp_rows_per_block(rows)
                                  : (rows + kBwdTargetBlocks - 1) / kBwdTargetBlocks;
  if (rpb < 1) rpb = 1;
  BwdPlan p;
  p.rows_per_block = rpb;
  p.nparts = (int)((rows + rpb - 1) / rpb);
  return p;
}

// Forward grid: with 16 lanes per row a wave per four-row group
// (rms_fwd_grp); with 64 a persistent grid of RV_RMS_FWD_BLOCKS_PER_CU blocks
// per CU (rms_fwd_vec).
dim3 fwd_grid(int64_t rows, int lanes_per_row) {
  const int64_t rows_per_block = (int64_t)kFwdWaves * (64 / lanes_per_row);
  int64_t blocks = (rows + rows_per_block - 1) / rows_per_block;
  if (lanes_per_row == 64) {
    const int64_t cap = (int64_t)rv_host::cu_count() * RV_RMS_FWD_BLOCKS_PER_CU;
    if (blocks > cap) blocks = cap;
  }
  return dim3((unsigned)blocks);
}

// Vector layout by width: 16 lanes per row with 1, 2 or 4 float4 per lane up to
// width 256; 64 lanes per row with 2 .. 16 float4 per lane above.
#define RV_FWD_DISPATCH(W, LAUNCH)       \
  do {                                   \
    if ((W) <= 64) LAUNCH(1, 16);        \
    else if ((W) <= 128) LAUNCH(2, 16);  \
    else if ((W) <= 256) LAUNCH(4, 16);  \
    else if ((W) <= 512) LAUNCH(2, 64);  \
    else if ((W) <= 1024) LAUNCH(4, 64); \
    else if ((W) <= 2048) LAUNCH(8, 64); \
    else LAUNCH(16, 64);                 \
  } while (0)

template <typename F, bool ADD, typename Y = float>
int launch_fwd(const float* x, const F* f, const float* w, float* h, Y* y,
               float* rstd, int64_t rows, int width, float eps,
               hipStream_t stream) {
  const bool vec = (width % 4 == 0) && rv_host::aligned16(x) &&
                   rv_host::aligned16(w) &&
                   (reinterpret_cast<uintptr_t>(y) % (4 * sizeof(Y))) == 0 &&
                   (h == nullptr || rv_host::aligned16(h)) &&
                   (f == nullptr ||
                    (reinterpret_cast<uintptr_t>(f) % (4 * sizeof(F))) == 0);
  if (vec && width <= 256 * kMaxVec) {
#define RV_FWD_VEC(V, G)                                                                      \
  if constexpr (G == 16) {                                                                    \
    if (width == 64 * (V))                                                                    \
      hipLaunchKernelGGL((rms_fwd_grp<V, true, F, ADD, Y>), fwd_grid(rows, G),                \
                         dim3(kFwdWaves * 64), 0, stream, x, f, w, h, y, rstd, rows, width, eps); \
    else                                                                                      \
      hipLaunchKernelGGL((rms_fwd_grp<V, false, F, ADD, Y>), fwd_grid(rows, G),               \
                         dim3(kFwdWaves * 64), 0, stream, x, f, w, h, y, rstd, rows, width, eps); \
  } else                                                                                      \
    hipLaunchKernelGGL((rms_fwd_vec<V, G, F, ADD, Y>), fwd_grid(rows, G), dim3(kFwdWaves * 64), \
                       0, stream, x, f, w, h, y, rstd, rows, width, eps)
    RV_FWD_DISPATCH(width, RV_FWD_VEC);
#undef RV_FWD_VEC
    return rv_host::check_launch();
  }
  if constexpr (!std::is_same<Y, float>::value) {
    return RV_ERR_UNSUPPORTED;  // fp16 output: vector path only
  } else {
  if (width > 64 * kMaxEpl) return RV_ERR_UNSUPPORTED;
  const dim3 grid((unsigned)((rows + kFwdWaves - 1) / kFwdWaves));
  const dim3 block(kFwdWaves * 64);
  const int epl = (width + 63) / 64;
#define RV_FWD_SC(E)                                                         \
  hipLaunchKernelGGL((rms_fwd_scalar<E, F, ADD>), grid, block, 0, stream, x, f, w, \
                     h, y, rstd, rows, width, eps)
  if (epl <= 1) RV_FWD_SC(1);
  else if (epl <= 2) RV_FWD_SC(2);
  else if (epl <= 4) RV_FWD_SC(4);
  else if (epl <= 8) RV_FWD_SC(8);
  else if (epl <= 16) RV_FWD_SC(16);
  else if (epl <= 32) RV_FWD_SC(32);
  else RV_FWD_SC(64);
#undef RV_FWD_SC
  return rv_host::check_launch();
  }
}

// x - f (SUBM 1: stored in h, the norm's input), d = x - f and h = d + f
// (SUBM 2), or the midpoint update of x with f and g (SUBM 3, stored in h):
// vector path, fp16 y only.
template <typename F, int SUBM>
int launch_fwd_sub(const float* x, const F* f, const float* w, float* d, float* h, __half* y,
                   float* rstd, int64_t rows, int width, float eps, hipStream_t stream,
                   const F* g = nullptr, float scale = 0.f, int sign = 1) {
  const bool vec = (width % 4 == 0) && rv_host::aligned16(x) && rv_host::aligned16(w) &&
                   rv_host::aligned16(h) && (d == nullptr || rv_host::aligned16(d)) &&
                   (reinterpret_cast<uintptr_t>(y) % 8) == 0 &&
                   (reinterpret_cast<uintptr_t>(f) % (4 * sizeof(F))) == 0 &&
                   (reinterpret_cast<uintptr_t>(g) % (4 * sizeof(F))) == 0;
  if (!vec || width > 256 * kMaxVec) return RV_ERR_UNSUPPORTED;
#define RV_FWD_SUB(V, G)                                                                       \
  if constexpr (G == 16) {                                                                     \
    if (width == 64 * (V))                                                                     \
      hipLaunchKernelGGL((rms_fwd_grp<V, true, F, true, __half, SUBM>), fwd_grid(rows, G),     \
                         dim3(kFwdWaves * 64), 0, stream, x, f, w, h, y, rstd, rows, width,    \
                         eps, d, g, scale, sign);                                              \
    else                                                                                       \
      hipLaunchKernelGGL((rms_fwd_grp<V, false, F, true, __half, SUBM>), fwd_grid(rows, G),    \
                         dim3(kFwdWaves * 64), 0, stream, x, f, w, h, y, rstd, rows, width,    \
                         eps, d, g, scale, sign);                                              \
  } else                                                                                       \
    hipLaunchKernelGGL((rms_fwd_vec<V, G, F, true, __half, SUBM>), fwd_grid(rows, G),          \
                       dim3(kFwdWaves * 64), 0, stream, x, f, w, h, y, rstd, rows, width, eps, \
                       d, g, scale, sign)
  RV_FWD_DISPATCH(width, RV_FWD_SUB);
#undef RV_FWD_SUB
  return rv_host::check_launch();
}

template <typename G>
int launch_bwd(const float* x, const float* w, const G* dy, const float* rstd, float* dx,
               float* dw, void* workspace, int64_t workspace_bytes, int64_t rows,
               int64_t width, hipStream_t s, const float* dh = nullptr,
               __half* dx16 = nullptr, const float* dpass = nullptr) {
  if (!x || !w || !dy || !rstd || !dx || !dw) return RV_ERR_NULL_POINTER;
  if (rows <= 0 || width <= 0) return RV_ERR_BAD_SIZE;
  if (width > 4096) return RV_ERR_UNSUPPORTED;
  const BwdPlan p = plan_bwd(rows, width);
  const int64_t need = (int64_t)p.nparts * width * (int64_t)sizeof(float);
  if (workspace == nullptr || workspace_bytes < need) return RV_ERR_WORKSPACE;
  if (!rv_host::aligned16(workspace)) return RV_ERR_WORKSPACE;
  float* partial = (float*)workspace;
  const dim3 grid((unsigned)p.nparts);
  const dim3 block(kBwdWaves * 64);
  const int iw = (int)width;
  const bool vec = (width % 4 == 0) && rv_host::aligned16(x) &&
                   rv_host::aligned16(w) &&
                   (reinterpret_cast<uintptr_t>(dy) % (4 * sizeof(G))) == 0 &&
                   rv_host::aligned16(dx) && (dh == nullptr || rv_host::aligned16(dh)) &&
                   (dpass == nullptr || rv_host::aligned16(dpass)) &&
                   (reinterpret_cast<uintptr_t>(dx16) % 8) == 0;
  if (!vec && (dh != nullptr || dx16 != nullptr || dpass != nullptr)) return RV_ERR_UNSUPPORTED;
  // the pass-through gradient: with the fp16 copy and without dh only
  if (dpass != nullptr && (dh != nullptr || dx16 == nullptr)) return RV_ERR_UNSUPPORTED;
  if (vec && bwd_narrow(iw)) {
    const dim3 gblock(kGrpWaves * 64);
    const int ng = grp_loads(p.rows_per_block);
    const int rpb = (int)p.rows_per_block;
#define RV_BWD_GRP_K(V, NG, ACC, H16, PASS)                                                       \
  do {                                                                                            \
    if (iw == 64 * (V))                                                                           \
      hipLaunchKernelGGL((rms_bwd_grp<V, NG, true, G, ACC, H16, PASS>), grid, gblock, 0, s, x, w, \
                         dy, rstd, dx, partial, rows, iw, rpb, dh, dx16, dpass);                  \
    else                                                                                          \
      hipLaunchKernelGGL((rms_bwd_grp<V, NG, false, G, ACC, H16, PASS>), grid, gblock, 0, s, x,   \
                         w, dy, rstd, dx, partial, rows, iw, rpb, dh, dx16, dpass);               \
  } while (0)
#define RV_BWD_GRP_NG(V, NG)                                                      \
  do {                                                                            \
    if (dpass != nullptr) RV_BWD_GRP_K(V, NG, false, true, true);                 \
    else if (dh != nullptr && dx16 != nullptr) RV_BWD_GRP_K(V, NG, true, true, false); \
    else if (dh != nullptr) RV_BWD_GRP_K(V, NG, true, false, false);              \
    else if (dx16 != nullptr) RV_BWD_GRP_K(V, NG, false, true, false);            \
    else RV_BWD_GRP_K(V, NG, false, false, false);                                \
  } while (0)
#define RV_BWD_GRP(V)                          \
  do {                                         \
    if (ng <= 4) RV_BWD_GRP_NG(V, 4);          \
    else if (ng == 5) RV_BWD_GRP_NG(V, 5);     \
    else if (ng == 6) RV_BWD_GRP_NG(V, 6);     \
    else RV_BWD_GRP_NG(V, 8);                  \
  } while (0)
    if (iw <= 64) RV_BWD_GRP(1);
    else if (iw <= 128) RV_BWD_GRP(2);
    else RV_BWD_GRP(4);
#undef RV_BWD_GRP
#undef RV_BWD_GRP_NG
#undef RV_BWD_GRP_K
  } else if (vec) {
    const int vecs = (iw + 255) / 256;
#define RV_BWD_VEC_K(V, ACC, H16)                                                         \
  hipLaunchKernelGGL((rms_bwd_vec<V, bwd_waves(V, ACC), G, ACC, H16>), grid,              \
                     dim3(bwd_waves(V, ACC) * 64), 0, s, x, w, dy, rstd, dx, partial, rows,  \
                     iw, p.rows_per_block, dh, dx16, nullptr)
#define RV_BWD_VEC(V)                                                \
  do {                                                               \
    if (dpass != nullptr)                                            \
      hipLaunchKernelGGL((rms_bwd_vec<V, bwd_waves(V, true), G, false, true, true>), grid, \
                         dim3(bwd_waves(V, true) * 64), 0, s, x, w, dy, rstd, dx, partial, \
                         rows, iw, p.rows_per_block, nullptr, dx16, dpass);          \
    else if (dh != nullptr && dx16 != nullptr) RV_BWD_VEC_K(V, true, true);   \
    else if (dh != nullptr) RV_BWD_VEC_K(V, true, false);            \
    else if (dx16 != nullptr) RV_BWD_VEC_K(V, false, true);          \
    else RV_BWD_VEC_K(V, false, false);                              \
  } while (0)
    if (vecs <= 1) RV_BWD_VEC(1);
    else if (vecs <= 2) RV_BWD_VEC(2);
    else if (vecs <= 4) RV_BWD_VEC(4);
    else if (vecs <= 8) RV_BWD_VEC(8);
    else RV_BWD_VEC(16);
#undef RV_BWD_VEC
#undef RV_BWD_VEC_K
  } else if constexpr (!std::is_same<G, float>::value) {
    return RV_ERR_UNSUPPORTED;  // fp16 gradient: vector path only
  } else {
    const int epl = (iw + 63) / 64;
#define RV_BWD_SC(E)                                                          \
  hipLaunchKernelGGL((rms_bwd_scalar<E>), grid, block, 0, s, x, w, dy, rstd, dx, \
                     partial, rows, iw, p.rows_per_block)
    if (epl <= 1) RV_BWD_SC(1);
    else if (epl <= 2) RV_BWD_SC(2);
    else if (epl <= 4) RV_BWD_SC(4);
    else if (epl <= 8) RV_BWD_SC(8);
    else if (epl <= 16) RV_BWD_SC(16);
    else if (epl <= 32) RV_BWD_SC(32);
    else RV_BWD_SC(64);
#undef RV_BWD_SC
  }
  int st = rv_host::check_launch();
  if (st != RV_OK) return st;
  hipLaunchKernelGGL(rms_dw_reduce, dim3((unsigned)((iw + kRedCols - 1) / kRedCols)),
                     dim3(kRedGroups * kRedCols), 0, s, partial, dw, iw, p.nparts);
  return rv_host::check_launch();
}

// ---------------------------------------------------------------------------
// Scratch of the backward entry point that allocates nothing
// (rv_rmsnorm_bwd_noalloc): the dweight partial rows, at most
// kBwdTargetBlocks x 4096 fp32 (4 MiB).  Every GPU the library runs on holds
// its own copy of this array until the process ends.  Host code never passes
// the array's name to a kernel (on the host it is only a stand-in for the
// symbol): the device address comes from hipGetSymbolAddress, queried once
// per device with that device current, and is cached per device.
// ---------------------------------------------------------------------------
constexpr int kNoallocMaxWidth = 4096;
constexpr int64_t kNoallocScratchFloats = kBwdTargetBlocks * kNoallocMaxWidth;

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxScratchDevices];  // device address of `scratch`, per device

}  // namespace

static __device__ __align__(256) float scratch[kNoallocScratchFloats];

namespace {

// The current device's address of `scratch` (queried on its first use on that
// device), or an rv_status.  A stream of another device is refused: the
// kernels would run there with this device's address.
int scratch_address(hipStream_t stream, float** out) {
  int dev = 0;
  const hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return rv_host::hip_fail(e);
  if (dev < 0 || dev >= kMaxScratchDevices) return RV_ERR_UNSUPPORTED;
  if (stream != nullptr) {
    int sdev = -1;
    const hipError_t es = hipStreamGetDevice(stream, &sdev);
    if (es != hipSuccess) return rv_host::hip_fail(es);
    if (sdev != dev) return RV_ERR_UNSUPPORTED;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    const hipError_t err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess) return rv_host::hip_fail(err);
    if (ptr == nullptr) return RV_ERR_HIP;
    g_scratch_ptr[dev] = ptr;
  }
  *out = static_cast<float*>(g_scratch_ptr[dev]);
  return RV_OK;
}

}  // namespace

extern "C" {

int rv_rmsnorm_fwd(const float* x, const float* w, float* y, float* rstd,
                   int64_t rows, int64_t width, float eps, void* stream) {
  if (!x || !w || !y || !rstd) return RV_ERR_NULL_POINTER;
  if (rows <= 0 || width <= 0) return RV_ERR_BAD_SIZE;
  if (width > 4096) return RV_ERR_UNSUPPORTED;
  return launch_fwd<float, false>(x, nullptr, w, nullptr, y, rstd, rows,
                                  (int)width, eps, (hipStream_t)stream);
}

int rv_add_rmsnorm_fwd(const float* x, const void* f, int force_dtype,
                       const float* w, float* h, float* y, float* rstd,
                       int64_t rows, int64_t width, float eps, void* stream) {
  if (!x || !f || !w || !h || !y || !rstd) return RV_ERR_NULL_POINTER;
  if (rows <= 0 || width <= 0) return RV_ERR_BAD_SIZE;
  if (width > 4096) return RV_ERR_UNSUPPORTED;
  const hipStream_t s = (hipStream_t)stream;
  switch (force_dtype) {
    case RV_F32:
      return launch_fwd<float, true>(x, (const float*)f, w, h, y, rstd, rows,
                                     (int)width, eps, s);
    case RV_F16:
      return launch_fwd<__half, true>(x, (const __half*)f, w, h, y, rstd,
                                      rows, (int)width, eps, s);
    case RV_BF16:
      return launch_fwd<__hip_bfloat16, true>(x, (const __hip_bfloat16*)f, w,
                                              h, y, rstd, rows, (int)width,
                                              eps, s);
    default:
      return RV_ERR_UNSUPPORTED;
  }
}

int rv_sub_rmsnorm_fwd_f16(const float* x, const void* f, int force_dtype, int readd,
                           const float* w, float* d, float* h, void* y, float* rstd,
                           int64_t rows, int64_t width, float eps, void* stream) {
  if (!x || !f || !w || !d || !y || !rstd || (readd && !h)) return RV_ERR_NULL_POINTER;
  if (rows <= 0 || width <= 0) return RV_ERR_BAD_SIZE;
  if (width > 4096) return RV_ERR_UNSUPPORTED;
  const hipStream_t s = (hipStream_t)stream;
  __half* y16 = static_cast<__half*>(y);
  switch (force_dtype) {
    case RV_F32:
      return readd ? launch_fwd_sub<float, 2>(x, (const float*)f, w, d, h, y16, rstd, rows,
                                              (int)width, eps, s)
                   : launch_fwd_sub<float, 1>(x, (const float*)f, w, nullptr, d, y16, rstd,
                                              rows, (int)width, eps, s);
    case RV_F16:
      return readd ? launch_fwd_sub<__half, 2>(x, (const __half*)f, w, d, h, y16, rstd, rows,
                                               (int)width, eps, s)
                   : launch_fwd_sub<__half, 1>(x, (const __half*)f, w, nullptr, d, y16, rstd,
                                               rows, (int)width, eps, s);
    default:
      return RV_ERR_UNSUPPORTED;
  }
}

int rv_midpoint_rmsnorm_fwd_f16(const float* p, const void* a, const void* m, int force_dtype,
                                double scale, int sign, const float* w, float* out, void* y,
                                float* rstd, int64_t rows, int64_t width, float eps,
                                void* stream) {
  if (!p || !a || !m || !w || !out || !y || !rstd) return RV_ERR_NULL_POINTER;
  if (rows <= 0 || width <= 0) return RV_ERR_BAD_SIZE;
  if (width > 4096 || force_dtype != RV_F16) return RV_ERR_UNSUPPORTED;
  return launch_fwd_sub<__half, 3>(p, static_cast<const __half*>(a), w, nullptr, out,
                                   static_cast<__half*>(y), rstd, rows, (int)width, eps,
                                   (hipStream_t)stream, static_cast<const __half*>(m),
                                   (float)scale, sign);
}

int64_t rv_rmsnorm_bwd_workspace_bytes(int64_t rows, int64_t width) {
  if (rows <= 0 || width <= 0) return -(int64_t)RV_ERR_BAD_SIZE;
  const BwdPlan p = plan_bwd(rows, width);
  return (int64_t)p.nparts * width * (int64_t)sizeof(float);
}

int rv_rmsnorm_bwd(const float* x, const float* w, const float* dy,
                   const float* rstd, float* dx, float* dw, void* workspace,
                   int64_t workspace_bytes, int64_t rows, int64_t width,
                   void* stream) {
  return launch_bwd<float>(x, w, dy, rstd, dx, dw, workspace, workspace_bytes, rows, width,
                           (hipStream_t)stream);
}

int rv_rmsnorm_bwd_noalloc(const float* x, const float* w, const float* dy, const float* rstd,
                           float* dx, float* dw, int64_t rows, int64_t width, void* stream) {
  // Argument checks first: a rejected call touches no device state.
  if (!x || !w || !dy || !rstd || !dx || !dw) return RV_ERR_NULL_POINTER;
  if (rows <= 0 || width <= 0) return RV_ERR_BAD_SIZE;
  if (width > kNoallocMaxWidth) return RV_ERR_UNSUPPORTED;
  const int64_t need = (int64_t)plan_bwd(rows, width).nparts * width * (int64_t)sizeof(float);
  if (need > kNoallocScratchFloats * (int64_t)sizeof(float)) return RV_ERR_WORKSPACE;
  float* ws = nullptr;
  const int st = scratch_address((hipStream_t)stream, &ws);
  if (st != RV_OK) return st;
  // The partial rows are written in full before the reduce reads them, so the
  // previous call's contents need no clearing.
  return launch_bwd<float>(x, w, dy, rstd, dx, dw, ws, need, rows, width, (hipStream_t)stream);
}

int rv_rmsnorm_fwd_f16(const float* x, const float* w, void* y, float* rstd, int64_t rows,
                       int64_t width, float eps, void* stream) {
  if (!x || !w || !y || !rstd) return RV_ERR_NULL_POINTER;
  if (rows <= 0 || width <= 0) return RV_ERR_BAD_SIZE;
  if (width > 4096) return RV_ERR_UNSUPPORTED;
  return launch_fwd<float, false, __half>(x, nullptr, w, nullptr, static_cast<__half*>(y), rstd,
                                          rows, (int)width, eps, (hipStream_t)stream);
}

int rv_rmsnorm_bwd_f16(const float* x, const float* w, const void* dy, const float* rstd,
                       float* dx, float* dw, void* workspace, int64_t workspace_bytes,
                       int64_t rows, int64_t width, void* stream) {
  return launch_bwd<__half>(x, w, static_cast<const __half*>(dy), rstd, dx, dw, workspace,
                            workspace_bytes, rows, width, (hipStream_t)stream);
}

int rv_add_rmsnorm_fwd_f16(const float* x, const void* f, int force_dtype, const float* w,
                           float* h, void* y, float* rstd, int64_t rows, int64_t width,
                           float eps, void* stream) {
  if (!x || !f || !w || !h || !y || !rstd) return RV_ERR_NULL_POINTER;
  if (rows <= 0 || width <= 0) return RV_ERR_BAD_SIZE;
  if (width > 4096) return RV_ERR_UNSUPPORTED;
  const hipStream_t s = (hipStream_t)stream;
  __half* y16 = static_cast<__half*>(y);
  switch (force_dtype) {
    case RV_F32:
      return launch_fwd<float, true, __half>(x, (const float*)f, w, h, y16, rstd, rows,
                                             (int)width, eps, s);
    case RV_F16:
      return launch_fwd<__half, true, __half>(x, (const __half*)f, w, h, y16, rstd, rows,
                                              (int)width, eps, s);
    default:
      return RV_ERR_UNSUPPORTED;
  }
}

int rv_rmsnorm_bwd_acc(const float* x, const float* w, const void* dy, int dy_dtype,
                       const float* rstd, const float* dh, float* dx, void* dx16, float* dw,
                       void* workspace, int64_t workspace_bytes, int64_t rows, int64_t width,
                       void* stream) {
  return rv_rmsnorm_bwd_acc_pass(x, w, dy, dy_dtype, rstd, dh, nullptr, dx, dx16, dw, workspace,
                                 workspace_bytes, rows, width, stream);
}

int rv_rmsnorm_bwd_acc_pass(const float* x, const float* w, const void* dy, int dy_dtype,
                            const float* rstd, const float* dh, const float* dpass, float* dx,
                            void* dx16, float* dw, void* workspace, int64_t workspace_bytes,
                            int64_t rows, int64_t width, void* stream) {
  const hipStream_t s = (hipStream_t)stream;
  __half* d16 = static_cast<__half*>(dx16);
  switch (dy_dtype) {
    case RV_F32:
      return launch_bwd<float>(x, w, static_cast<const float*>(dy), rstd, dx, dw, workspace,
                               workspace_bytes, rows, width, s, dh, d16, dpass);
    case RV_F16:
      return launch_bwd<__half>(x, w, static_cast<const __half*>(dy), rstd, dx, dw, workspace,
                                workspace_bytes, rows, width, s, dh, d16, dpass);
    default:
      return RV_ERR_UNSUPPORTED;
  }
}

}  // extern "C"
