// MFMA GEMMs for the SwiGLU MLP projections on gfx950, with fused epilogues.
//
// The six contractions of one TiledMLP tile (src/reversibility/optimized_v3.py:
// 10-18, 47-63) under fp16 autocast, in the canonical form
//     C[i][j] = sum_k A(i, k) * B(j, k)      (fp16 operands, fp32 accumulate)
//
//   up + SwiGLU   A = x[m][d]      B = W_up[g|v][d]   -> o = fp16(silu(fp16 u_g)) * fp16 u_v
//   down          A = o[m][f]      B = W_down[d][f]   -> y = fp16(acc)
//   d_o + SwiGLU' A = dy[m][d]     B(f, d) = W_down[d][f] -> du = swiglu_bwd(u, fp16(acc))
//   dx            A = du[m][j]     B(d, j) = W_up[j][d]   -> dx = fp32(fp16(acc))
//   dW_down       A(d, m) = dy[m][d]   B(f, m) = o[m][f]   (reduce over tokens, split-K)
//   dW_up         A(j, m) = du[m][j]   B(d, m) = x[m][d]   (reduce over tokens, split-K)
//
// Operands are read in their stored layout: "KC" sources are k-contiguous
// ([rows][k]); "RC" sources are [k][rows] (rows contiguous) and are transposed
// on the way into LDS.  fp32 sources (the fp32 master weights, the fp32
// normalized activations) are rounded to fp16 while loading, which is the
// cast autocast's F.linear performs, so no separate cast kernels run.
//
// Tiling: a workgroup of 4 waves (2 x 2) owns a (64*TM) x 128 tile of C; each
// wave owns TM x 2 tiles of 32 x 32 computed with v_mfma_f32_32x32x16_f16.
// K advances 32 at a time through two LDS buffers: the next stage's global
// loads are issued before the current stage's MFMAs, then written to the
// other buffer; one barrier per stage.  LDS rows are padded by 8 halves
// against bank conflicts.
//
// MFMA 32x32x16 lane layout (gfx950, verified on the device): lane l supplies
// A row / B column (l % 32) and 8 k values; the 16 accumulator values of lane
// l are C[(j/4)*8 + (l/32)*4 + j%4][l % 32], j = 0..15.  Any k order is valid
// as long as A and B agree; here lane l carries k = (l/32)*8 + 0..7.

#include "rv_device.h"

namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int kBN = 128;        // B rows (output columns) per workgroup
constexpr int kBK = 32;         // k per pipeline stage
constexpr int kLds = kBK + 8;   // padded LDS row, halves (80 bytes)

// ---------------------------------------------------------------------------
// fp32 / fp16 -> packed fp16 helpers
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  const __half2 h = __floats2half2_rn(a, b);
  return *reinterpret_cast<const uint32_t*>(&h);
}
__device__ __forceinline__ uint4 pack8(const float* v) {
  return make_uint4(pack2(v[0], v[1]), pack2(v[2], v[3]), pack2(v[4], v[5]), pack2(v[6], v[7]));
}

// 8 consecutive elements of a row, returned as 8 packed fp16.
template <typename T> __device__ __forceinline__ uint4 load8(const T* p);
template <> __device__ __forceinline__ uint4 load8<__half>(const __half* p) {
  return *reinterpret_cast<const uint4*>(p);
}
template <> __device__ __forceinline__ uint4 load8<float>(const float* p) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  const float4 b = *reinterpret_cast<const float4*>(p + 4);
  const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  return pack8(v);
}

// ---------------------------------------------------------------------------
// Tile loaders.  A loader moves one [ROWS][kBK] fp16 tile of an operand into
// LDS (row-major, row stride kLds).  load() issues the global loads into
// registers; store() writes them to LDS.  Rows past `rows` are clamped to a
// valid row (their results are never stored); k past `kmax` load zeros.
// ---------------------------------------------------------------------------

// Source [rows][ld], k contiguous.  A row may be remapped (gate/value gather).
template <typename T, int ROWS>
struct LoadKC {
  static constexpr int kVec = ROWS * kBK / 8 / kThreads;  // 16-byte vectors per thread
  uint4 r[kVec];
  template <class RowMap>
  __device__ __forceinline__ void load(const T* __restrict__ base, int64_t ld, const RowMap& map,
                                       int64_t k0) {
#pragma unroll
    for (int i = 0; i < kVec; ++i) {
      const int v = threadIdx.x + i * kThreads;
      const int row = v / (kBK / 8);
      const int kv = (v % (kBK / 8)) * 8;
      r[i] = load8<T>(base + map(row) * ld + k0 + kv);
    }
  }
  __device__ __forceinline__ void store(_Float16* lds) const {
#pragma unroll
    for (int i = 0; i < kVec; ++i) {
      const int v = threadIdx.x + i * kThreads;
      const int row = v / (kBK / 8);
      const int kv = (v % (kBK / 8)) * 8;
      *reinterpret_cast<uint4*>(lds + row * kLds + kv) = r[i];
    }
  }
};

// Source [k][ld] with the tile's rows contiguous (a transposed operand).  Each
// thread owns 8 consecutive rows x 2 consecutive k: two row-vector loads, then
// eight 4-byte LDS writes of (k, k+1) pairs.  k >= kmax reads as zero.
template <typename T, int ROWS>
struct LoadRC {
  static constexpr int kChunks = ROWS / 8;                   // 8-row chunks per k
  static constexpr int kPairs = kThreads / kChunks;          // k pairs covered per pass
  static constexpr int kPass = kBK / 2 / kPairs;             // passes per stage
  static_assert(kPass >= 1 && kChunks * kPairs == kThreads, "RC tile shape");
  uint4 r[kPass][2];
  __device__ __forceinline__ void load(const T* __restrict__ base, int64_t ld, int64_t row0,
                                       int64_t k0, int64_t kmax) {
    const int chunk = threadIdx.x % kChunks;
#pragma unroll
    for (int p = 0; p < kPass; ++p) {
      const int kk = ((threadIdx.x / kChunks) + p * kPairs) * 2;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int64_t k = k0 + kk + h;
        const int64_t kc = k < kmax ? k : kmax - 1;  // clamp, then zero below
        uint4 v = load8<T>(base + kc * ld + row0 + chunk * 8);
        if (k >= kmax) v = make_uint4(0u, 0u, 0u, 0u);
        r[p][h] = v;
      }
    }
  }
  __device__ __forceinline__ void store(_Float16* lds) const {
    const int chunk = threadIdx.x % kChunks;
#pragma unroll
    for (int p = 0; p < kPass; ++p) {
      const int kk = ((threadIdx.x / kChunks) + p * kPairs) * 2;
      const uint32_t* lo = reinterpret_cast<const uint32_t*>(&r[p][0]);
      const uint32_t* hi = reinterpret_cast<const uint32_t*>(&r[p][1]);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        // element e of the row chunk: low/high halves of word e/2
        const uint32_t a = (e & 1) ? (lo[e >> 1] >> 16) : (lo[e >> 1] & 0xffffu);
        const uint32_t b = (e & 1) ? (hi[e >> 1] >> 16) : (hi[e >> 1] & 0xffffu);
        *reinterpret_cast<uint32_t*>(lds + (chunk * 8 + e) * kLds + kk) = a | (b << 16);
      }
    }
  }
};

struct RowsDirect {  // LDS row r -> source row row0 + r, clamped to [0, rows)
  int64_t row0, rows;
  __device__ __forceinline__ int64_t operator()(int r) const {
    const int64_t g = row0 + r;
    return g < rows ? g : rows - 1;
  }
};
struct RowsGateValue {  // LDS rows 0..63 -> gate rows n0.., 64..127 -> value rows F + n0..
  int64_t n0, f;
  __device__ __forceinline__ int64_t operator()(int r) const {
    return r < 64 ? n0 + r : f + n0 + (r - 64);
  }
};

// ---------------------------------------------------------------------------
// MFMA core: acc[tm][tn] += A_tile * B_tile^T over one LDS stage.
// Wave (wm, wn): A rows wm*32*TM + tm*32 + (l%32); B rows tn*64 + wn*32 + (l%32).
// ---------------------------------------------------------------------------
template <int TM>
__device__ __forceinline__ void mfma_stage(const _Float16* __restrict__ a_lds,
                                           const _Float16* __restrict__ b_lds,
                                           f32x16 (&acc)[TM][2], int wm, int wn, int lane) {
#pragma unroll
  for (int ks = 0; ks < kBK / 16; ++ks) {
    const int k = ks * 16 + (lane / 32) * 8;
    f16x8 a[TM], b[2];
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
      a[tm] = *reinterpret_cast<const f16x8*>(a_lds + (wm * 32 * TM + tm * 32 + lane % 32) * kLds + k);
#pragma unroll
    for (int tn = 0; tn < 2; ++tn)
      b[tn] = *reinterpret_cast<const f16x8*>(b_lds + (tn * 64 + wn * 32 + lane % 32) * kLds + k);
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
      for (int tn = 0; tn < 2; ++tn)
        acc[tm][tn] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[tm], b[tn], acc[tm][tn], 0, 0, 0);
  }
}

// Row of accumulator element j of lane `lane` inside a 32x32 tile.
__device__ __forceinline__ int acc_row(int j, int lane) {
  return (j / 4) * 8 + (lane / 32) * 4 + (j % 4);
}

// ---------------------------------------------------------------------------
// Kernel 1: activation GEMMs, C[m][n] over m-tiles of 64*TM rows and
// n-tiles of 128 B rows; A is a KC source; B is KC (forward) or RC (backward).
// ---------------------------------------------------------------------------
enum class Epi { SwiGLU, StoreF16, SwiGLUBwd, StoreF32OfF16 };

struct ActArgs {
  const void* a; int64_t lda;         // A source
  const void* b; int64_t ldb;         // B source
  int64_t m, n, k;                    // rows of C, columns of C (F for SwiGLU), reduction
  void* c; int64_t ldc;               // output (o, y, du, dx)
  void* u; int64_t ldu;               // SwiGLU: optional u output; SwiGLUBwd: u input
};

template <int TM, typename TA, typename TB, bool B_RC, Epi EPI>
__global__ __launch_bounds__(kThreads, 2)
void act_gemm(ActArgs args) {
  constexpr int BM = 64 * TM;
  __shared__ __attribute__((aligned(16))) _Float16 lds_a[2][BM * kLds];
  __shared__ __attribute__((aligned(16))) _Float16 lds_b[2][kBN * kLds];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // SwiGLU: a block covers 64 output columns (64 gate + 64 value B rows).
  constexpr int kCols = (EPI == Epi::SwiGLU) ? 64 : kBN;
  const int64_t n_blocks = args.n / kCols;
  const int64_t mb = blockIdx.x / n_blocks;
  const int64_t nb = blockIdx.x % n_blocks;
  const int64_t m0 = mb * BM, n0 = nb * kCols;

  const TA* A = static_cast<const TA*>(args.a);
  const TB* B = static_cast<const TB*>(args.b);
  LoadKC<TA, BM> la;
  const RowsDirect amap{m0, args.m};
  LoadKC<TB, kBN> lb_kc;
  LoadRC<TB, kBN> lb_rc;

  auto issue = [&](int64_t k0) {
    la.load(A, args.lda, amap, k0);
    if constexpr (B_RC) {
      lb_rc.load(B, args.ldb, n0, k0, args.k);
    } else if constexpr (EPI == Epi::SwiGLU) {
      lb_kc.load(B, args.ldb, RowsGateValue{n0, args.n}, k0);
    } else {
      lb_kc.load(B, args.ldb, RowsDirect{n0, args.n}, k0);
    }
  };
  auto commit = [&](int buf) {
    la.store(lds_a[buf]);
    if constexpr (B_RC) lb_rc.store(lds_b[buf]); else lb_kc.store(lds_b[buf]);
  };

  f32x16 acc[TM][2];
#pragma unroll
  for (int tm = 0; tm < TM; ++tm)
#pragma unroll
    for (int tn = 0; tn < 2; ++tn)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[tm][tn][j] = 0.f;

  const int64_t stages = args.k / kBK;
  issue(0);
  commit(0);
  __syncthreads();
  for (int64_t s = 0; s < stages; ++s) {
    const int buf = (int)(s & 1);
    if (s + 1 < stages) issue((s + 1) * kBK);
    mfma_stage<TM>(lds_a[buf], lds_b[buf], acc, wm, wn, lane);
    if (s + 1 < stages) commit(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue ----
#pragma unroll
  for (int tm = 0; tm < TM; ++tm) {
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int64_t row = m0 + wm * 32 * TM + tm * 32 + acc_row(j, lane);
      if (row >= args.m) continue;
      if constexpr (EPI == Epi::SwiGLU) {
        const int64_t col = n0 + wn * 32 + (lane % 32);
        const float g = rv::round_to<__half>(acc[tm][0][j]);
        const float v = rv::round_to<__half>(acc[tm][1][j]);
        const float silu = rv::round_to<__half>(g * rv::fast_sigmoid(g));
        static_cast<__half*>(args.c)[row * args.ldc + col] = __float2half_rn(silu * v);
        if (args.u != nullptr) {
          __half* u = static_cast<__half*>(args.u) + row * args.ldu;
          u[col] = __float2half_rn(g);
          u[args.n + col] = __float2half_rn(v);
        }
      } else {
#pragma unroll
        for (int tn = 0; tn < 2; ++tn) {
          const int64_t col = n0 + tn * 64 + wn * 32 + (lane % 32);
          const float d = rv::round_to<__half>(acc[tm][tn][j]);
          if constexpr (EPI == Epi::StoreF16) {
            static_cast<__half*>(args.c)[row * args.ldc + col] = __float2half_rn(d);
          } else if constexpr (EPI == Epi::StoreF32OfF16) {
            static_cast<float*>(args.c)[row * args.ldc + col] = d;
          } else {  // SwiGLUBwd: du from u = [gate | value] and d_o = d
            const __half* u = static_cast<const __half*>(args.u) + row * args.ldu;
            const float g = __half2float(u[col]);
            const float v = __half2float(u[args.n + col]);
            const float s = rv::fast_sigmoid(g);
            const float silu = rv::round_to<__half>(g * s);
            const float dgi = rv::round_to<__half>(d * v);
            __half* du = static_cast<__half*>(args.c) + row * args.ldc;
            du[col] = __float2half_rn(dgi * (s * (1.0f + g * (1.0f - s))));
            du[args.n + col] = __float2half_rn(d * silu);
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Kernel 2: weight gradients, C[i][j] = sum_m A(i, m) B(j, m) with both
// operands RC sources ([m][i], [m][j]).  blockIdx -> (i-tile, j-tile, split);
// split s reduces m in [s*chunk, min((s+1)*chunk, m)) and writes its fp32
// partial tile to part[s][i][j].
// ---------------------------------------------------------------------------
struct WgradArgs {
  const void* a; int64_t lda;   // [m][ni]
  const void* b; int64_t ldb;   // [m][nj]
  int64_t m, ni, nj, chunk;     // tokens, output rows, output cols, tokens per split
  float* part;                  // [splits][ni][nj]
};

template <typename TA, typename TB>
__global__ __launch_bounds__(kThreads, 2)
void wgrad_gemm(WgradArgs args) {
  constexpr int TM = 2, BM = 128;
  __shared__ __attribute__((aligned(16))) _Float16 lds_a[2][BM * kLds];
  __shared__ __attribute__((aligned(16))) _Float16 lds_b[2][kBN * kLds];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t ti = args.ni / BM, tj = args.nj / kBN;
  const int64_t s = blockIdx.x / (ti * tj);
  const int64_t rem = blockIdx.x % (ti * tj);
  const int64_t i0 = (rem / tj) * BM, j0 = (rem % tj) * kBN;
  const int64_t kbeg = s * args.chunk;
  const int64_t kend = kbeg + args.chunk < args.m ? kbeg + args.chunk : args.m;

  const TA* A = static_cast<const TA*>(args.a);
  const TB* B = static_cast<const TB*>(args.b);
  LoadRC<TA, BM> la;
  LoadRC<TB, kBN> lb;

  f32x16 acc[TM][2];
#pragma unroll
  for (int tm = 0; tm < TM; ++tm)
#pragma unroll
    for (int tn = 0; tn < 2; ++tn)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[tm][tn][j] = 0.f;

  const int64_t stages = (kend - kbeg + kBK - 1) / kBK;
  if (stages > 0) {
    la.load(A, args.lda, i0, kbeg, kend);
    lb.load(B, args.ldb, j0, kbeg, kend);
    la.store(lds_a[0]);
    lb.store(lds_b[0]);
  }
  __syncthreads();
  for (int64_t st = 0; st < stages; ++st) {
    const int buf = (int)(st & 1);
    if (st + 1 < stages) {
      la.load(A, args.lda, i0, kbeg + (st + 1) * kBK, kend);
      lb.load(B, args.ldb, j0, kbeg + (st + 1) * kBK, kend);
    }
    mfma_stage<TM>(lds_a[buf], lds_b[buf], acc, wm, wn, lane);
    if (st + 1 < stages) {
      la.store(lds_a[buf ^ 1]);
      lb.store(lds_b[buf ^ 1]);
    }
    __syncthreads();
  }
  float* out = args.part + s * args.ni * args.nj;
#pragma unroll
  for (int tm = 0; tm < TM; ++tm)
#pragma unroll
    for (int tn = 0; tn < 2; ++tn)
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int64_t row = i0 + wm * 64 + tm * 32 + acc_row(j, lane);
        const int64_t col = j0 + tn * 64 + wn * 32 + (lane % 32);
        out[row * args.nj + col] = acc[tm][tn][j];
      }
}

// acc[i] (+)= fp32(fp16(sum_s part[s][i])), splits summed in order.  This is
// autocast's weight gradient: the fp16 GEMM result, cast to the fp32 weight
// and added to the running per-tile sum.
__global__ __launch_bounds__(256)
void wgrad_reduce(const float* __restrict__ part, int splits, int64_t n, float* acc_out,
                  int accumulate) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  float s = 0.f;
  for (int k = 0; k < splits; ++k) s = s + part[k * n + i];
  const float g = rv::round_to<__half>(s);
  acc_out[i] = accumulate ? acc_out[i] + g : g;
}

// ---------------------------------------------------------------------------
// Host launch helpers
// ---------------------------------------------------------------------------
template <int TM, typename TA, typename TB, bool B_RC, Epi EPI>
int launch_act(const ActArgs& a, hipStream_t s) {
  constexpr int BM = 64 * TM;
  const int64_t cols = (EPI == Epi::SwiGLU) ? 64 : kBN;
  const int64_t blocks = ((a.m + BM - 1) / BM) * (a.n / cols);
  hipLaunchKernelGGL((act_gemm<TM, TA, TB, B_RC, EPI>), dim3((unsigned)blocks), dim3(kThreads),
                     0, s, a);
  return rv_host::check_launch();
}

bool f16_or_f32(int dt) { return dt == RV_F16 || dt == RV_F32; }

// Split-K plan for an ni x nj weight gradient over `rows` tokens: enough
// splits to give ~256 workgroups (at most 16), each split a multiple of kBK
// tokens.  Depends only on the sizes, so results are device-independent.
struct WgradPlan {
  int64_t tiles, splits, chunk;
};
WgradPlan plan_wgrad(int64_t rows, int64_t ni, int64_t nj) {
  WgradPlan p;
  p.tiles = (ni / 128) * (nj / kBN);
  int64_t want = 256 / (p.tiles > 0 ? p.tiles : 1);
  if (want < 1) want = 1;
  if (want > 16) want = 16;
  int64_t chunk = (rows + want - 1) / want;
  chunk = (chunk + kBK - 1) / kBK * kBK;
  p.chunk = chunk;
  p.splits = (rows + chunk - 1) / chunk;
  return p;
}

}  // namespace

extern "C" {

int rv_mlp_up_swiglu(const void* x, int x_dtype, int64_t ldx, const float* w_up,
                     int64_t rows, int64_t d, int64_t f, void* o, void* u, void* stream) {
  if (!x || !w_up || !o) return RV_ERR_NULL_POINTER;
  if (rows <= 0 || d <= 0 || f <= 0 || ldx < d) return RV_ERR_BAD_SIZE;
  if (!f16_or_f32(x_dtype) || d % kBK || f % 64 || ldx % 8) return RV_ERR_UNSUPPORTED;
  if (!rv_host::aligned16(x) || !rv_host::aligned16(w_up)) return RV_ERR_UNSUPPORTED;
  ActArgs a{x, ldx, w_up, d, rows, f, d, o, f, u, 2 * f};
  const hipStream_t s = (hipStream_t)stream;
  return x_dtype == RV_F32 ? launch_act<2, float, float, false, Epi::SwiGLU>(a, s)
                           : launch_act<2, __half, float, false, Epi::SwiGLU>(a, s);
}

int rv_mlp_down(const void* o, const float* w_down, int64_t rows, int64_t d, int64_t f,
                void* y, void* stream) {
  if (!o || !w_down || !y) return RV_ERR_NULL_POINTER;
  if (rows <= 0 || d <= 0 || f <= 0) return RV_ERR_BAD_SIZE;
  if (f % kBK || d % kBN) return RV_ERR_UNSUPPORTED;
  if (!rv_host::aligned16(o) || !rv_host::aligned16(w_down)) return RV_ERR_UNSUPPORTED;
  ActArgs a{o, f, w_down, f, rows, d, f, y, d, nullptr, 0};
  return launch_act<1, __half, float, false, Epi::StoreF16>(a, (hipStream_t)stream);
}

int rv_mlp_dgate(const void* dy, const float* w_down, const void* u, int64_t rows, int64_t d,
                 int64_t f, void* du, void* stream) {
  if (!dy || !w_down || !u || !du) return RV_ERR_NULL_POINTER;
  if (rows <= 0 || d <= 0 || f <= 0) return RV_ERR_BAD_SIZE;
  if (d % kBK || f % kBN) return RV_ERR_UNSUPPORTED;
  if (!rv_host::aligned16(dy) || !rv_host::aligned16(w_down)) return RV_ERR_UNSUPPORTED;
  ActArgs a{dy, d, w_down, f, rows, f, d, du, 2 * f, const_cast<void*>(u), 2 * f};
  return launch_act<2, __half, float, true, Epi::SwiGLUBwd>(a, (hipStream_t)stream);
}

int rv_mlp_dx(const void* du, const float* w_up, int64_t rows, int64_t d, int64_t f,
              float* dx, void* stream) {
  if (!du || !w_up || !dx) return RV_ERR_NULL_POINTER;
  if (rows <= 0 || d <= 0 || f <= 0) return RV_ERR_BAD_SIZE;
  if ((2 * f) % kBK || d % kBN) return RV_ERR_UNSUPPORTED;
  if (!rv_host::aligned16(du) || !rv_host::aligned16(w_up)) return RV_ERR_UNSUPPORTED;
  ActArgs a{du, 2 * f, w_up, d, rows, d, 2 * f, dx, d, nullptr, 0};
  return launch_act<1, __half, float, true, Epi::StoreF32OfF16>(a, (hipStream_t)stream);
}

int64_t rv_mlp_wgrad_workspace_bytes(int64_t rows, int64_t d, int64_t f) {
  if (rows <= 0 || d <= 0 || f <= 0) return -(int64_t)RV_ERR_BAD_SIZE;
  const WgradPlan pd = plan_wgrad(rows, d, f), pu = plan_wgrad(rows, 2 * f, d);
  const int64_t a = pd.splits * d * f, b = pu.splits * 2 * f * d;
  return (a > b ? a : b) * (int64_t)sizeof(float);
}

int rv_mlp_wgrad(const void* dy, const void* o, const void* du, const void* x, int x_dtype,
                 int64_t ldx, int64_t rows, int64_t d, int64_t f, float* ddown, float* dup,
                 int accumulate, void* workspace, int64_t workspace_bytes, void* stream) {
  if (!dy || !o || !du || !x || !ddown || !dup) return RV_ERR_NULL_POINTER;
  if (rows <= 0 || d <= 0 || f <= 0 || ldx < d) return RV_ERR_BAD_SIZE;
  if (!f16_or_f32(x_dtype) || d % kBN || f % kBN || ldx % 8) return RV_ERR_UNSUPPORTED;
  const int64_t need = rv_mlp_wgrad_workspace_bytes(rows, d, f);
  if (workspace == nullptr || workspace_bytes < need) return RV_ERR_WORKSPACE;
  const hipStream_t s = (hipStream_t)stream;
  float* part = static_cast<float*>(workspace);
  // dW_down[d][f] = sum_m dy[m][d] o[m][f]
  {
    const WgradPlan p = plan_wgrad(rows, d, f);
    WgradArgs a{dy, d, o, f, rows, d, f, p.chunk, part};
    hipLaunchKernelGGL((wgrad_gemm<__half, __half>), dim3((unsigned)(p.splits * p.tiles)),
                       dim3(kThreads), 0, s, a);
    int st = rv_host::check_launch();
    if (st != RV_OK) return st;
    const int64_t n = d * f;
    hipLaunchKernelGGL(wgrad_reduce, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, part,
                       (int)p.splits, n, ddown, accumulate);
    st = rv_host::check_launch();
    if (st != RV_OK) return st;
  }
  // dW_up[2f][d] = sum_m du[m][j] x16[m][d]
  {
    const WgradPlan p = plan_wgrad(rows, 2 * f, d);
    WgradArgs a{du, 2 * f, x, ldx, rows, 2 * f, d, p.chunk, part};
    if (x_dtype == RV_F32)
      hipLaunchKernelGGL((wgrad_gemm<__half, float>), dim3((unsigned)(p.splits * p.tiles)),
                         dim3(kThreads), 0, s, a);
    else
      hipLaunchKernelGGL((wgrad_gemm<__half, __half>), dim3((unsigned)(p.splits * p.tiles)),
                         dim3(kThreads), 0, s, a);
    int st = rv_host::check_launch();
    if (st != RV_OK) return st;
    const int64_t n = 2 * f * d;
    hipLaunchKernelGGL(wgrad_reduce, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, part,
                       (int)p.splits, n, dup, accumulate);
    return rv_host::check_launch();
  }
}

}  // extern "C"
