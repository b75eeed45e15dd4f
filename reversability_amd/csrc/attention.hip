// Causal self-attention for gfx950 on MFMA (the attention inside the force,
// src/reversibility/model.py:26-45: F.scaled_dot_product_attention(q, k, v,
// is_causal=True) with the default scale 1/sqrt(head_dim), under fp16
// autocast).
//
// Layouts: qkv fp16 [B][T][3][H][HD] -- the packed projection exactly as the
// qkv GEMM writes it, read in place (no split, permute or copy); out and dout
// fp16 [B][T][H][HD], i.e. [B][T][d], what the output projection reads; lse
// and delta fp32 [B*H][T]; dqkv fp16 in qkv's layout.
//
// Forward (one workgroup = 4 waves = 128 queries of one (b, h); key tiles of
// 64 streamed through LDS, double buffered): each wave keeps its 32 queries'
// Q fragments in registers and computes S^T = K Q^T with
// v_mfma_f32_32x32x16_f16, so every lane holds the scores of one query (16
// keys per 32-key half tile, the other 16 in lane l ^ 32).  Online softmax in
// base 2 (c = scale * log2 e): m = running max of S c, p = 2^(S c - m) in
// fp32, l = sum p; O^T += V^T P^T on MFMA with P rounded to fp16, so the
// accumulator holds one query's outputs per lane and the rescale by
// 2^(m_old - m_new) is lane-local; m moves only when a score exceeds it by
// more than 2^8, so most tiles skip the rescale.  Tiles the causal diagonal
// does not cross run a code path without masking.
// lse = m + log2 l (base-2 units) is kept for the backward.
//
// Backward (FA2 order, no atomics, deterministic), two launches:
//   dQ: one workgroup = 128 queries; key tiles streamed; each lane first
//     forms its query's delta = rowsum(dO * O) from the dO and O fragments it
//     holds (its half of the row, then the other half from lane l ^ 32) and
//     writes it for the next kernel; then
//     S^T, dP^T (queries in lanes), dQ^T += K^T dS^T           attn_bwd_q_k
//   dK, dV: one workgroup = 128 keys; query tiles of 64 streamed; per wave
//     S = Q K^T, dP = dO V^T (keys in lanes), P = 2^(S c - lse),
//     dS = P (dP - delta), dV^T += dO^T P, dK^T += Q^T dS      attn_bwd_kv_k
//   dK and dQ are multiplied by the scale once, at the end.
//
// MFMA operand layout (gfx950, 32x32x16 f16): mfma(X, Y, acc) takes 8
// halves of row l % 32 of X and of Y at k = (l/32)*8 + 0..7 from lane l, and
// acc value j of lane l is sum_k X[(j/4)*8 + (l/32)*4 + j%4][k] Y[l%32][k].
// A product contracted over keys (or queries) takes its k order from the
// accumulator that produced P or dS: k index (l/32)*8 + i stands for tile row
// sigma = (i/4)*8 + (l/32)*4 + i%4, so a lane passes its own accumulator
// values 0..7 (and 8..15 for the next 16 rows) as the operand unchanged, and
// the other operand is read with ds_read_b64_tr_b16 from those rows.
//
// LDS tiles are [row][HD] fp16 with the 16-byte chunk index XOR-swizzled per
// row (swz); for HD = 32, 64, 128 both the row reads (ds_read_b128, lane ->
// row l % 32) and the transposed reads (rows sigma, 16 columns per 16 lanes)
// are free of bank conflicts for 32- and 64-bank LDS models.

#include <cmath>

#include "rv_device.h"

namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
#define RV_LDS __attribute__((address_space(3)))

constexpr int kThreads = 256;
constexpr int kWaveRows = 32;    // queries (forward, dQ) or keys (dK/dV) per wave
constexpr int kBlockRows = 128;  // per workgroup
constexpr int kTile = 64;        // rows per streamed LDS tile

// Workgroups per CU the register budget is sized for: two for HD <= 64; one
// for HD = 128, whose accumulators need the whole 512-register file.
template <int HD>
constexpr int kMinBlocks = HD == 128 ? 1 : 2;
// The forward keeps fewer live registers: three workgroups per CU at HD = 64.
template <int HD>
constexpr int kFwdMinBlocks = HD == 128 ? 1 : (HD == 64 ? 3 : 2);
// So does the dQ kernel: at HD = 64 three workgroups per CU fit in 168
// registers with two spilled outside the key loop (C5 backward 652-658 ->
// 633-638 us against two workgroups at 176 registers).
template <int HD>
constexpr int kQMinBlocks = HD == 128 ? 1 : (HD == 64 ? 3 : 2);

template <int HD>
__device__ __forceinline__ int swz(int r, int c) {
  if constexpr (HD == 32) return c ^ (((r >> 2) & 1) | ((((r >> 1) ^ (r >> 3)) & 1) << 1));
  else if constexpr (HD == 64) return c ^ (((r >> 2) ^ ((r & 3) << 1)) & 7);
  else return c ^ ((r & 3) | (((r ^ (r >> 2)) & 1) << 2) | ((((r >> 1) ^ (r >> 3)) & 1) << 3));
}

// Half index of tile element (r, col).
template <int HD>
__device__ __forceinline__ int lds_at(int r, int col) {
  return r * HD + (swz<HD>(r, col >> 3) << 3) + (col & 7);
}

__device__ __forceinline__ f32x16 mfma(f16x8 x, f16x8 y, f32x16 acc) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(x, y, acc, 0, 0, 0);
}

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int e = 0; e < 16; ++e) z[e] = 0.f;
  return z;
}

// Values 8 h .. 8 h + 7 of an accumulator as an fp16 operand.
__device__ __forceinline__ f16x8 pack8(const f32x16& v, int h) {
  f16x8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = (_Float16)v[8 * h + i];
  return r;
}

constexpr int kRsrcWord3 = 0x00020000;  // raw buffer resource, gfx9 data format

// Global -> registers -> LDS copy of a tile of kTile rows x HD halves.  The
// loads go through a buffer resource that starts at the tile's first row and
// ends with row `valid - 1`'s HD halves: rows at or past `valid` read as zero
// (the buffer range check), so no row needs a predicate, and a thread's byte
// offset inside a tile is the same for every tile (row stride `stride`
// halves; launch checks keep kTile rows of it below 2 GiB).
template <int HD>
struct TileCopy {
  static constexpr int kPer = kTile * HD / 8 / kThreads;
  static_assert(kPer >= 1, "tile smaller than one chunk per thread");
  u32x4 v[kPer];
  uint32_t off[kPer];
  __device__ __forceinline__ explicit TileCopy(int64_t stride) {
#pragma unroll
    for (int it = 0; it < kPer; ++it) {
      const int ch = it * kThreads + threadIdx.x;
      const int r = ch / (HD / 8), c = ch % (HD / 8);
      off[it] = (uint32_t)(((int64_t)r * stride + c * 8) * 2);
    }
  }
  __device__ __forceinline__ void load(const __half* base, int64_t stride, int row0, int valid) {
    const int rows = min(valid - row0, kTile);
    const int bytes = rows > 0 ? (int)(((int64_t)(rows - 1) * stride + HD) * 2) : 0;
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<__half*>(base + (int64_t)row0 * stride), 0, bytes, kRsrcWord3);
#pragma unroll
    for (int it = 0; it < kPer; ++it)
      v[it] = __builtin_amdgcn_raw_buffer_load_b128(rsrc, (int)off[it], 0, 0);
  }
  __device__ __forceinline__ void store(_Float16* t) const {
#pragma unroll
    for (int it = 0; it < kPer; ++it) {
      const int ch = it * kThreads + threadIdx.x;
      const int r = ch / (HD / 8), c = ch % (HD / 8);
      *reinterpret_cast<u32x4*>(t + r * HD + (swz<HD>(r, c) << 3)) = v[it];
    }
  }
};

// 64 fp32 per-row values (lse or delta) of a tile into LDS; rows past
// `valid` get 0.
__device__ __forceinline__ float load_rowval(const float* src, int row0, int valid) {
  const int r = row0 + (int)threadIdx.x;
  return (threadIdx.x < kTile && r < valid) ? src[r] : 0.f;
}

// Store 4 consecutive fp16 values (8 bytes).
__device__ __forceinline__ void store4(__half* dst, float a, float b, float c, float d) {
  f16x4 v = {(_Float16)a, (_Float16)b, (_Float16)c, (_Float16)d};
  *reinterpret_cast<f16x4*>(dst) = v;
}

// ---------------------------------------------------------------------------
// Forward.
// ---------------------------------------------------------------------------
// Value of lane l ^ 32 combined with the lane's own (v_permlane32_swap: the
// two 32-lane halves exchange; both halves get the same combination, lower
// half's value first).
__device__ __forceinline__ float pair_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Row of tile element j of a 32 x 32 accumulator, relative to the lane's own
// first row (l/32)*4: (j/4)*8 + j%4.
__device__ __forceinline__ constexpr int acc_row(int j) { return (j >> 2) * 8 + (j & 3); }

// Wave priorities inside one SIMD: a wave issues its score MFMA chains (S,
// and dP in the backward) at priority 2, the forward's P V chain at 1 and its
// softmax arithmetic at 0, so that the instruction arbiter prefers the wave
// with matrix work ready and the other waves' exponentials fill the matrix
// core's gaps (C5 forward 214-219 -> 208 us, backward -1%; results unchanged).
__device__ __forceinline__ void prio_mfma() { __builtin_amdgcn_s_setprio(2); }
__device__ __forceinline__ void prio_mfma_tail() { __builtin_amdgcn_s_setprio(1); }
__device__ __forceinline__ void prio_valu() { __builtin_amdgcn_s_setprio(0); }

// The running max is moved only when a score exceeds it by more than kLazy
// (base-2 units): p = 2^(S c - m) then stays below 2^kLazy (exact in fp16's
// exponent range), and the rescale of o and l is skipped on most tiles.
constexpr float kLazy = 8.0f;

template <int HD>
struct FwdState {
  f32x16 o[HD / 32];
  float m, l;
};

// A lane's LDS offsets (halves) inside one [64][HD] tile, fixed for the whole
// kernel: row operands of rows 0..31 (rows 32..63 add 32 HD: the swizzle
// depends on the row's low five bits only) and transposed operands of the
// rows sigma of each 16-row group, upper half of each read pair included.
template <int HD>
struct FragOffsets {
  int row[HD / 16];           // frag_row(t, lane % 32, kk, hl)
  int tr[2][HD / 32][2];      // frag_tr(t, cc * 16, dt * 32, lane): [cc][dt][first / second]
  __device__ __forceinline__ explicit FragOffsets(int lane) {
    const int hl = lane >> 5, g = lane >> 4, i = lane & 15;
#pragma unroll
    for (int kk = 0; kk < HD / 16; ++kk)
      row[kk] = (lane & 31) * HD + (swz<HD>(lane & 31, kk * 2 + hl) << 3);
#pragma unroll
    for (int cc = 0; cc < 2; ++cc)
#pragma unroll
      for (int dt = 0; dt < HD / 32; ++dt) {
        const int r = cc * 16 + (g >> 1) * 4 + (i >> 2);
        const int col = dt * 32 + (g & 1) * 16 + 4 * (i & 3);
        tr[cc][dt][0] = lds_at<HD>(r, col);
        tr[cc][dt][1] = lds_at<HD>(r + 8, col);
      }
  }
  __device__ __forceinline__ f16x8 rowf(const _Float16* t, int sub, int kk) const {
    return *reinterpret_cast<const f16x8*>(t + sub * 32 * HD + row[kk]);
  }
  __device__ __forceinline__ f16x8 trf(const _Float16* t, int sub, int cc, int dt) const {
    const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (RV_LDS i16x4*)(t + sub * 32 * HD + tr[cc][dt][0]));
    const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (RV_LDS i16x4*)(t + sub * 32 * HD + tr[cc][dt][1]));
    const f16x4 a = __builtin_bit_cast(f16x4, lo), b = __builtin_bit_cast(f16x4, hi);
    return f16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
  }
};

// One 64-key tile for one wave.  MASK: the causal diagonal crosses the tile;
// key offset (within the tile) k is visible to the lane's query iff
// k <= rel, rel = q - k0.  live1: the second 32-key half has a visible key
// for some query of the wave.
template <int HD, bool MASK>
__device__ __forceinline__ void fwd_tile(FwdState<HD>& st, const _Float16* Ks, const _Float16* Vs,
                                         const FragOffsets<HD>& fo, const f16x8 (&qf)[HD / 16],
                                         bool live1, int rel, float c, int lane) {
  constexpr int KK = HD / 16, DT = HD / 32;
  const int hl = lane >> 5;
  f32x16 s[2];
  prio_mfma();
#pragma unroll
  for (int sub = 0; sub < 2; ++sub) {
    if (sub == 1 && MASK && !live1) break;
    s[sub] = mfma(fo.rowf(Ks, sub, 0), qf[0], zero16());
#pragma unroll
    for (int kk = 1; kk < KK; ++kk) s[sub] = mfma(fo.rowf(Ks, sub, kk), qf[kk], s[sub]);
  }
  const bool two = !MASK || live1;
  prio_valu();
  float mx = -INFINITY;
#pragma unroll
  for (int sub = 0; sub < 2; ++sub) {
    if (sub == 1 && !two) break;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      if constexpr (MASK) {
        if (sub * 32 + acc_row(j) + hl * 4 > rel) s[sub][j] = -INFINITY;
      }
      mx = fmaxf(mx, s[sub][j]);
    }
  }
  const float mxc = pair_max(mx) * c;
  if (__any(mxc > st.m + kLazy)) {
    const float m_new = fmaxf(st.m, mxc);
    const float alpha = __builtin_amdgcn_exp2f(st.m - m_new);
    st.m = m_new;
    st.l *= alpha;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int e = 0; e < 16; ++e) st.o[dt][e] *= alpha;
  }
  const float neg_m = -st.m;
#pragma unroll
  for (int sub = 0; sub < 2; ++sub) {
    if (sub == 1 && !two) break;
    float rowsum = 0.f;
    prio_valu();
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const float p = __builtin_amdgcn_exp2f(fmaf(s[sub][j], c, neg_m));
      rowsum += p;
      s[sub][j] = p;
    }
    st.l += rowsum;
    prio_mfma_tail();
#pragma unroll
    for (int cc = 0; cc < 2; ++cc) {
      const f16x8 pf = pack8(s[sub], cc);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) st.o[dt] = mfma(fo.trf(Vs, sub, cc, dt), pf, st.o[dt]);
    }
  }
}

template <int HD>
__global__ __launch_bounds__(kThreads, kFwdMinBlocks<HD>)
void attn_fwd_k(const __half* __restrict__ qkv, __half* __restrict__ out, float* __restrict__ lse,
                int T, int H, int n_qt, float c) {
  constexpr int KK = HD / 16, DT = HD / 32;
  __shared__ __attribute__((aligned(16))) _Float16 lds[2][2][kTile * HD];
  const int BH = (int)(gridDim.x / n_qt);
  const int qt = n_qt - 1 - (int)(blockIdx.x / BH);  // longest rows first
  const int bh = (int)(blockIdx.x % BH);
  const int b = bh / H, h = bh % H;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, hl = lane >> 5;
  const int64_t rs = (int64_t)3 * H * HD;
  const __half* qb = qkv + (int64_t)b * T * rs + (int64_t)h * HD;
  const __half* kb = qb + (int64_t)H * HD;
  const __half* vb = qb + (int64_t)2 * H * HD;
  const int q0 = qt * kBlockRows + wave * kWaveRows;
  const int q = q0 + (lane & 31);
  const FragOffsets<HD> fo(lane);

  f16x8 qf[KK];
#pragma unroll
  for (int kk = 0; kk < KK; ++kk)
    qf[kk] = q < T ? *reinterpret_cast<const f16x8*>(qb + (int64_t)q * rs + kk * 16 + hl * 8)
                   : f16x8{0, 0, 0, 0, 0, 0, 0, 0};
  FwdState<HD> st;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) st.o[dt] = zero16();
  st.m = -INFINITY;
  st.l = 0.f;

  const int kv_end = min(T, qt * kBlockRows + kBlockRows);
  const int n_kt = (kv_end + kTile - 1) / kTile;
  TileCopy<HD> ck(rs), cv(rs);
  ck.load(kb, rs, 0, T);
  cv.load(vb, rs, 0, T);
  ck.store(lds[0][0]);
  cv.store(lds[0][1]);
  __syncthreads();
  // Tile t lives in buffer t % 2; the loop body is written out for both
  // buffers so that each buffer's LDS address is a constant.
#define RV_FWD_STEP(BUF)                                                                    \
  {                                                                                         \
    const int k0 = t * kTile;                                                               \
    const bool more = t + 1 < n_kt;                                                         \
    if (more) {                                                                             \
      ck.load(kb, rs, k0 + kTile, T);                                                       \
      cv.load(vb, rs, k0 + kTile, T);                                                       \
    }                                                                                       \
    if (k0 + kTile - 1 <= q0)                                                               \
      fwd_tile<HD, false>(st, lds[BUF][0], lds[BUF][1], fo, qf, true, 0, c, lane);          \
    else if (k0 <= q0 + kWaveRows - 1)                                                      \
      fwd_tile<HD, true>(st, lds[BUF][0], lds[BUF][1], fo, qf,                              \
                         k0 + 32 <= q0 + kWaveRows - 1, q - k0, c, lane);                    \
    if (more) {                                                                             \
      ck.store(lds[1 - (BUF)][0]);                                                          \
      cv.store(lds[1 - (BUF)][1]);                                                          \
    }                                                                                       \
    __syncthreads();                                                                        \
  }
  for (int t = 0; t < n_kt; ++t) {
    RV_FWD_STEP(0)
    if (++t >= n_kt) break;
    RV_FWD_STEP(1)
  }
#undef RV_FWD_STEP
  const float l = pair_sum(st.l);
  if (q < T) {
    const float inv = 1.0f / l;
    __half* orow = out + ((int64_t)b * T + q) * H * HD + (int64_t)h * HD;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int jg = 0; jg < 4; ++jg)
        store4(orow + dt * 32 + jg * 8 + hl * 4, st.o[dt][4 * jg] * inv,
               st.o[dt][4 * jg + 1] * inv, st.o[dt][4 * jg + 2] * inv,
               st.o[dt][4 * jg + 3] * inv);
    if (hl == 0) lse[(int64_t)bh * T + q] = st.m + __log2f(l);
  }
}

// ---------------------------------------------------------------------------
// Backward.
// ---------------------------------------------------------------------------
// dK/dV contribution of 32 staged queries (tile rows r0 .. r0 + 31 of Q / dO)
// to one wave's 32 keys (lanes).  MASK: the causal diagonal crosses the pair;
// tile row r is visible to the lane's key iff r >= krel = key - (first query
// of the tile).  Query rows past the sequence hold zeros (Q, dO, lse, delta):
// their P is 1 but dS = 0 and dO = 0, so they add nothing.
template <int HD, bool MASK>
__device__ __forceinline__ void kv_rows(f32x16 (&dk)[HD / 32], f32x16 (&dv)[HD / 32],
                                        const _Float16* Qs, const _Float16* Gs, const float* Ls,
                                        const float* Ds, const FragOffsets<HD>& fo,
                                        const f16x8 (&kf)[HD / 16],
                                        const f16x8 (&vf)[HD / 16], int r0, int krel, float c,
                                        int lane) {
  constexpr int KK = HD / 16, DT = HD / 32;
  const int hl = lane >> 5;
  const int sub = r0 / 32;
  prio_mfma();
  f32x16 s = mfma(fo.rowf(Qs, sub, 0), kf[0], zero16());
  f32x16 dp = mfma(fo.rowf(Gs, sub, 0), vf[0], zero16());
#pragma unroll
  for (int kk = 1; kk < KK; ++kk) {
    s = mfma(fo.rowf(Qs, sub, kk), kf[kk], s);
    dp = mfma(fo.rowf(Gs, sub, kk), vf[kk], dp);
  }
  prio_valu();
#pragma unroll
  for (int jg = 0; jg < 4; ++jg) {
    const int r4 = r0 + jg * 8 + hl * 4;
    const float4 L4 = *reinterpret_cast<const float4*>(Ls + r4);
    const float4 D4 = *reinterpret_cast<const float4*>(Ds + r4);
    const float Lr[4] = {L4.x, L4.y, L4.z, L4.w};
    const float Dr[4] = {D4.x, D4.y, D4.z, D4.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int j = 4 * jg + e;
      float p = __builtin_amdgcn_exp2f(fmaf(s[j], c, -Lr[e]));
      if constexpr (MASK) {
        if (r4 + e < krel) p = 0.f;
      }
      s[j] = p;
      dp[j] = p * (dp[j] - Dr[e]);
    }
  }
#pragma unroll
  for (int cc = 0; cc < 2; ++cc) {
    const f16x8 pf = pack8(s, cc), dsf = pack8(dp, cc);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      dv[dt] = mfma(fo.trf(Gs, sub, cc, dt), pf, dv[dt]);
      dk[dt] = mfma(fo.trf(Qs, sub, cc, dt), dsf, dk[dt]);
    }
  }
}

// dQ contribution of 32 staged keys (tile rows r0 .. r0 + 31 of K / V) to one
// wave's 32 queries (lanes).  MASK: tile row r is visible iff r <= qrel =
// query - (first key of the tile).
template <int HD, bool MASK>
__device__ __forceinline__ void q_rows(f32x16 (&dq)[HD / 32], const _Float16* Ks,
                                       const _Float16* Vs, const FragOffsets<HD>& fo,
                                       const f16x8 (&qf)[HD / 16],
                                       const f16x8 (&gf)[HD / 16], float Lq, float Dq, int r0,
                                       int qrel, float c, int lane) {
  constexpr int KK = HD / 16, DT = HD / 32;
  const int hl = lane >> 5;
  const int sub = r0 / 32;
  prio_mfma();
  f32x16 s = mfma(fo.rowf(Ks, sub, 0), qf[0], zero16());
  f32x16 dp = mfma(fo.rowf(Vs, sub, 0), gf[0], zero16());
#pragma unroll
  for (int kk = 1; kk < KK; ++kk) {
    s = mfma(fo.rowf(Ks, sub, kk), qf[kk], s);
    dp = mfma(fo.rowf(Vs, sub, kk), gf[kk], dp);
  }
  const float neg_l = -Lq;
  prio_valu();
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    float p = __builtin_amdgcn_exp2f(fmaf(s[j], c, neg_l));
    if constexpr (MASK) {
      if (r0 + acc_row(j) + hl * 4 > qrel) p = 0.f;
    }
    dp[j] = p * (dp[j] - Dq);
  }
#pragma unroll
  for (int cc = 0; cc < 2; ++cc) {
    const f16x8 dsf = pack8(dp, cc);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
      dq[dt] = mfma(fo.trf(Ks, sub, cc, dt), dsf, dq[dt]);
  }
}

template <int HD>
__global__ __launch_bounds__(kThreads, kMinBlocks<HD>)
void attn_bwd_kv_k(const __half* __restrict__ qkv, const __half* __restrict__ dout,
                   const float* __restrict__ lse, const float* __restrict__ delta,
                   __half* __restrict__ dqkv, int T, int H, int n_kt, float c, float scale) {
  constexpr int KK = HD / 16, DT = HD / 32;
  __shared__ __attribute__((aligned(16))) _Float16 lds[2][2][kTile * HD];  // [buf][Q / dO]
  __shared__ __attribute__((aligned(16))) float rowv[2][2][kTile];          // [buf][lse / delta]
  const int BH = (int)(gridDim.x / n_kt);
  const int kt = (int)(blockIdx.x / BH);  // earliest keys (most queries) first
  const int bh = (int)(blockIdx.x % BH);
  const int b = bh / H, h = bh % H;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, hl = lane >> 5;
  const int64_t rs = (int64_t)3 * H * HD, os = (int64_t)H * HD;
  const __half* qb = qkv + (int64_t)b * T * rs + (int64_t)h * HD;
  const __half* kb = qb + os;
  const __half* vb = qb + 2 * os;
  const __half* gb = dout + (int64_t)b * T * os + (int64_t)h * HD;
  const float* lb = lse + (int64_t)bh * T;
  const float* db = delta + (int64_t)bh * T;
  const int kbase = kt * kBlockRows;
  const int k0w = kbase + wave * kWaveRows;
  const int key = k0w + (lane & 31);

  f16x8 kf[KK], vf[KK];
#pragma unroll
  for (int kk = 0; kk < KK; ++kk) {
    const bool ok = key < T;
    kf[kk] = ok ? *reinterpret_cast<const f16x8*>(kb + (int64_t)key * rs + kk * 16 + hl * 8)
                : f16x8{0, 0, 0, 0, 0, 0, 0, 0};
    vf[kk] = ok ? *reinterpret_cast<const f16x8*>(vb + (int64_t)key * rs + kk * 16 + hl * 8)
                : f16x8{0, 0, 0, 0, 0, 0, 0, 0};
  }
  f32x16 dk[DT], dv[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    dk[dt] = zero16();
    dv[dt] = zero16();
  }

  const int n_qtiles = (T - kbase + kTile - 1) / kTile;
  TileCopy<HD> cq(rs), cg(os);
  cq.load(qb, rs, kbase, T);
  cg.load(gb, os, kbase, T);
  float lv = load_rowval(lb, kbase, T), dvv = load_rowval(db, kbase, T);
  cq.store(lds[0][0]);
  cg.store(lds[0][1]);
  if (threadIdx.x < kTile) {
    rowv[0][0][threadIdx.x] = lv;
    rowv[0][1][threadIdx.x] = dvv;
  }
  __syncthreads();
  const FragOffsets<HD> fo(lane);
#define RV_KV_STEP(BUF)                                                                     \
  {                                                                                         \
    const int qt0 = kbase + t * kTile;                                                      \
    const bool more = t + 1 < n_qtiles;                                                     \
    if (more) {                                                                             \
      cq.load(qb, rs, qt0 + kTile, T);                                                      \
      cg.load(gb, os, qt0 + kTile, T);                                                      \
      lv = load_rowval(lb, qt0 + kTile, T);                                                 \
      dvv = load_rowval(db, qt0 + kTile, T);                                                \
    }                                                                                       \
    _Pragma("unroll") for (int sub = 0; sub < 2; ++sub) {                                   \
      const int qs = qt0 + sub * 32;                                                        \
      if (qs + kWaveRows - 1 < k0w) continue; /* every query precedes every key */          \
      if (qs >= k0w + kWaveRows - 1)                                                        \
        kv_rows<HD, false>(dk, dv, lds[BUF][0], lds[BUF][1], rowv[BUF][0], rowv[BUF][1], fo, \
                           kf, vf, sub * 32, 0, c, lane);                                   \
      else                                                                                  \
        kv_rows<HD, true>(dk, dv, lds[BUF][0], lds[BUF][1], rowv[BUF][0], rowv[BUF][1], fo,  \
                          kf, vf, sub * 32, key - qt0, c, lane);                            \
    }                                                                                       \
    if (more) {                                                                             \
      cq.store(lds[1 - (BUF)][0]);                                                          \
      cg.store(lds[1 - (BUF)][1]);                                                          \
      if (threadIdx.x < kTile) {                                                            \
        rowv[1 - (BUF)][0][threadIdx.x] = lv;                                               \
        rowv[1 - (BUF)][1][threadIdx.x] = dvv;                                              \
      }                                                                                     \
    }                                                                                       \
    __syncthreads();                                                                        \
  }
  for (int t = 0; t < n_qtiles; ++t) {
    RV_KV_STEP(0)
    if (++t >= n_qtiles) break;
    RV_KV_STEP(1)
  }
#undef RV_KV_STEP
  if (key < T) {
    __half* krow = dqkv + ((int64_t)b * T + key) * rs + os + (int64_t)h * HD;
    __half* vrow = krow + os;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int jg = 0; jg < 4; ++jg) {
        const int col = dt * 32 + jg * 8 + hl * 4;
        store4(krow + col, dk[dt][4 * jg] * scale, dk[dt][4 * jg + 1] * scale,
               dk[dt][4 * jg + 2] * scale, dk[dt][4 * jg + 3] * scale);
        store4(vrow + col, dv[dt][4 * jg], dv[dt][4 * jg + 1], dv[dt][4 * jg + 2],
               dv[dt][4 * jg + 3]);
      }
  }
}

template <int HD>
__global__ __launch_bounds__(kThreads, kQMinBlocks<HD>)
void attn_bwd_q_k(const __half* __restrict__ qkv, const __half* __restrict__ out,
                  const __half* __restrict__ dout, const float* __restrict__ lse,
                  float* __restrict__ delta, __half* __restrict__ dqkv, int T, int H, int n_qt,
                  float c, float scale) {
  constexpr int KK = HD / 16, DT = HD / 32;
  __shared__ __attribute__((aligned(16))) _Float16 lds[2][2][kTile * HD];  // [buf][K / V]
  const int BH = (int)(gridDim.x / n_qt);
  const int qt = n_qt - 1 - (int)(blockIdx.x / BH);
  const int bh = (int)(blockIdx.x % BH);
  const int b = bh / H, h = bh % H;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, hl = lane >> 5;
  const int64_t rs = (int64_t)3 * H * HD, os = (int64_t)H * HD;
  const __half* qb = qkv + (int64_t)b * T * rs + (int64_t)h * HD;
  const __half* kb = qb + os;
  const __half* vb = qb + 2 * os;
  const __half* gb = dout + (int64_t)b * T * os + (int64_t)h * HD;
  const int q0 = qt * kBlockRows + wave * kWaveRows;
  const int q = q0 + (lane & 31);
  const bool qok = q < T;

  f16x8 qf[KK], gf[KK];
#pragma unroll
  for (int kk = 0; kk < KK; ++kk) {
    qf[kk] = qok ? *reinterpret_cast<const f16x8*>(qb + (int64_t)q * rs + kk * 16 + hl * 8)
                 : f16x8{0, 0, 0, 0, 0, 0, 0, 0};
    gf[kk] = qok ? *reinterpret_cast<const f16x8*>(gb + (int64_t)q * os + kk * 16 + hl * 8)
                 : f16x8{0, 0, 0, 0, 0, 0, 0, 0};
  }
  const float Lq = qok ? lse[(int64_t)bh * T + q] : 0.f;
  // delta = sum_d dO O over the query's row: this lane's HD / 2 columns (the
  // fragments' layout), then the other half from lane l ^ 32
  float dsum = 0.f;
  {
    const __half* ob = out + (int64_t)b * T * os + (int64_t)h * HD;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      const f16x8 of = qok ? *reinterpret_cast<const f16x8*>(ob + (int64_t)q * os + kk * 16 +
                                                             hl * 8)
                           : f16x8{0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
      for (int i = 0; i < 8; ++i) dsum = fmaf((float)gf[kk][i], (float)of[i], dsum);
    }
  }
  const float Dq = pair_sum(dsum);
  if (qok && hl == 0) delta[(int64_t)bh * T + q] = Dq;
  f32x16 dq[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) dq[dt] = zero16();

  const int kv_end = min(T, qt * kBlockRows + kBlockRows);
  const int n_kt = (kv_end + kTile - 1) / kTile;
  TileCopy<HD> ck(rs), cv(rs);
  ck.load(kb, rs, 0, T);
  cv.load(vb, rs, 0, T);
  ck.store(lds[0][0]);
  cv.store(lds[0][1]);
  __syncthreads();
  const FragOffsets<HD> fo(lane);
#define RV_Q_STEP(BUF)                                                                      \
  {                                                                                         \
    const int k0 = t * kTile;                                                               \
    const bool more = t + 1 < n_kt;                                                         \
    if (more) {                                                                             \
      ck.load(kb, rs, k0 + kTile, T);                                                       \
      cv.load(vb, rs, k0 + kTile, T);                                                       \
    }                                                                                       \
    _Pragma("unroll") for (int sub = 0; sub < 2; ++sub) {                                   \
      const int ks = k0 + sub * 32;                                                         \
      if (ks > q0 + kWaveRows - 1) continue; /* every key follows every query */            \
      if (ks + kWaveRows - 1 <= q0)                                                         \
        q_rows<HD, false>(dq, lds[BUF][0], lds[BUF][1], fo, qf, gf, Lq, Dq, sub * 32, 0, c, \
                          lane);                                                            \
      else                                                                                  \
        q_rows<HD, true>(dq, lds[BUF][0], lds[BUF][1], fo, qf, gf, Lq, Dq, sub * 32, q - k0, \
                         c, lane);                                                          \
    }                                                                                       \
    if (more) {                                                                             \
      ck.store(lds[1 - (BUF)][0]);                                                          \
      cv.store(lds[1 - (BUF)][1]);                                                          \
    }                                                                                       \
    __syncthreads();                                                                        \
  }
  for (int t = 0; t < n_kt; ++t) {
    RV_Q_STEP(0)
    if (++t >= n_kt) break;
    RV_Q_STEP(1)
  }
#undef RV_Q_STEP
  if (qok) {
    __half* qrow = dqkv + ((int64_t)b * T + q) * rs + (int64_t)h * HD;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int jg = 0; jg < 4; ++jg)
        store4(qrow + dt * 32 + jg * 8 + hl * 4, dq[dt][4 * jg] * scale,
               dq[dt][4 * jg + 1] * scale, dq[dt][4 * jg + 2] * scale,
               dq[dt][4 * jg + 3] * scale);
  }
}

// Sizes the kernels take: a kTile-row tile of qkv (row stride 3 H hd halves)
// spans less than 2 GiB, so a tile's buffer resource and byte offsets fit.
bool dims_ok(int64_t batch, int64_t seq, int64_t heads, int64_t hd) {
  return batch > 0 && seq > 0 && heads > 0 && (hd == 32 || hd == 64 || hd == 128) &&
         seq < (1 << 30) && heads < (1 << 20) && batch * heads < (1 << 24) &&
         (int64_t)kTile * 3 * heads * hd * 2 < (int64_t(1) << 31);
}

template <int HD>
int launch_fwd(const __half* qkv, int64_t B, int64_t T, int64_t H, __half* out, float* lse,
               hipStream_t s) {
  const int n_qt = (int)((T + kBlockRows - 1) / kBlockRows);
  const float c = (float)(1.4426950408889634 / std::sqrt((double)HD));
  hipLaunchKernelGGL(attn_fwd_k<HD>, dim3((unsigned)(n_qt * B * H)), dim3(kThreads), 0, s, qkv,
                     out, lse, (int)T, (int)H, n_qt, c);
  return rv_host::check_launch();
}

template <int HD>
int launch_bwd(const __half* qkv, const __half* out, const __half* dout, const float* lse,
               int64_t B, int64_t T, int64_t H, __half* dqkv, float* delta, hipStream_t s) {
  const int n_t = (int)((T + kBlockRows - 1) / kBlockRows);
  const double scale = 1.0 / std::sqrt((double)HD);
  const float c = (float)(1.4426950408889634 * scale);
  const dim3 grid((unsigned)(n_t * B * H));
  // the dQ kernel writes delta, which the dK/dV kernel reads
  hipLaunchKernelGGL(attn_bwd_q_k<HD>, grid, dim3(kThreads), 0, s, qkv, out, dout, lse, delta,
                     dqkv, (int)T, (int)H, n_t, c, (float)scale);
  int rc = rv_host::check_launch();
  if (rc != RV_OK) return rc;
  hipLaunchKernelGGL(attn_bwd_kv_k<HD>, grid, dim3(kThreads), 0, s, qkv, dout, lse, delta, dqkv,
                     (int)T, (int)H, n_t, c, (float)scale);
  return rv_host::check_launch();
}

}  // namespace

extern "C" {

int rv_attn_fwd(const void* qkv, int64_t batch, int64_t seq, int64_t heads, int64_t head_dim,
                void* out, float* lse, void* stream) {
  if (!qkv || !out || !lse) return RV_ERR_NULL_POINTER;
  if (batch <= 0 || seq <= 0 || heads <= 0 || head_dim <= 0) return RV_ERR_BAD_SIZE;
  if (!dims_ok(batch, seq, heads, head_dim)) return RV_ERR_UNSUPPORTED;
  if (!rv_host::aligned16(qkv) || !rv_host::aligned16(out)) return RV_ERR_UNSUPPORTED;
  const __half* q = static_cast<const __half*>(qkv);
  __half* o = static_cast<__half*>(out);
  const hipStream_t s = (hipStream_t)stream;
  switch (head_dim) {
    case 32: return launch_fwd<32>(q, batch, seq, heads, o, lse, s);
    case 64: return launch_fwd<64>(q, batch, seq, heads, o, lse, s);
    default: return launch_fwd<128>(q, batch, seq, heads, o, lse, s);
  }
}

int64_t rv_attn_bwd_workspace_bytes(int64_t batch, int64_t seq, int64_t heads) {
  if (batch <= 0 || seq <= 0 || heads <= 0) return -RV_ERR_BAD_SIZE;
  return batch * heads * seq * 4;
}

int rv_attn_bwd(const void* qkv, const void* out, const void* dout, const float* lse,
                int64_t batch, int64_t seq, int64_t heads, int64_t head_dim, void* dqkv,
                void* workspace, int64_t workspace_bytes, void* stream) {
  if (!qkv || !out || !dout || !lse || !dqkv) return RV_ERR_NULL_POINTER;
  if (batch <= 0 || seq <= 0 || heads <= 0 || head_dim <= 0) return RV_ERR_BAD_SIZE;
  if (!dims_ok(batch, seq, heads, head_dim)) return RV_ERR_UNSUPPORTED;
  if (!rv_host::aligned16(qkv) || !rv_host::aligned16(out) || !rv_host::aligned16(dout) ||
      !rv_host::aligned16(dqkv))
    return RV_ERR_UNSUPPORTED;
  if (!workspace || workspace_bytes < batch * heads * seq * 4) return RV_ERR_WORKSPACE;
  const __half* q = static_cast<const __half*>(qkv);
  const __half* o = static_cast<const __half*>(out);
  const __half* g = static_cast<const __half*>(dout);
  __half* dq = static_cast<__half*>(dqkv);
  float* delta = static_cast<float*>(workspace);
  const hipStream_t s = (hipStream_t)stream;
  switch (head_dim) {
    case 32: return launch_bwd<32>(q, o, g, lse, batch, seq, heads, dq, delta, s);
    case 64: return launch_bwd<64>(q, o, g, lse, batch, seq, heads, dq, delta, s);
    default: return launch_bwd<128>(q, o, g, lse, batch, seq, heads, dq, delta, s);
  }
}

}  // extern "C"
