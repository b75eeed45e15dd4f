// MFMA GEMMs for the SwiGLU MLP projections on gfx950, with fused epilogues.
//
// The six contractions of one TiledMLP tile (src/reversibility/optimized_v3.py:
// 10-18, 47-63) under fp16 autocast, in the canonical form
//     C[i][j] = sum_k A(i, k) * B(j, k)      (fp16 operands, fp32 accumulate)
//
//   up + SwiGLU   A = x16[m][d]    B = Wup16[g|v][d]    -> o = fp16(silu(fp16 u_g)) * fp16 u_v
//   down          A = o[m][f]      B = Wdown16[d][f]    -> y = fp16(acc)
//   d_o + SwiGLU' A = dy[m][d]     B(f, d) = Wdown16[d][f] -> du = swiglu_bwd(u, fp16(acc))
//   dx            A = du[m][j]     B(d, j) = Wup16[j][d]   -> dx = fp32(fp16(acc))
//   dW_down       A(d, m) = dy[m][d]   B(f, m) = o[m][f]     -> (+)= fp32(fp16(acc))
//   dW_up         A(j, m) = du[m][j]   B(d, m) = x16[m][d]   -> (+)= fp32(fp16(acc))
//
// Every operand is fp16 and is read in its stored layout.  A "KC" source is
// [rows][k] (k contiguous) and is staged in LDS as [row][k]; fragments are one
// ds_read_b128 per lane.  An "RC" source is [k][rows] (rows contiguous) and is
// staged as [k][row]; fragments are two ds_read_b64_tr_b16 per lane, the
// gfx950 LDS transpose read.  Global -> LDS copies are therefore plain 16-byte
// row segments for both kinds, with no scatter.  The fp32 master weights and
// the fp32 normalized activations are cast to fp16 once per call
// (rv_cast_f32_f16) -- the cast autocast's F.linear performs.
//
// Tiling: a workgroup of 4 waves (2 x 2) owns a BM x BN tile of C; each wave
// owns (BM/2) x (BN/2) = TM x TN tiles of 32 x 32 computed with
// v_mfma_f32_32x32x16_f16.  K advances 64 per stage through two LDS buffers:
// the next stage's global loads are issued before the current stage's MFMAs
// and written to the other buffer afterwards; one barrier per stage.
// Tile sizes 256x256, 128x256, 128x128 and 64x128 are chosen per shape (the
// largest one that still gives about one workgroup per CU); the choice does
// not change any result bit, because every output element sums its k blocks
// in the same order in every tile shape.  Weight gradients over few output
// tiles may split the token reduction (split-K) into fp32 partials summed by a
// second kernel in a fixed order.
//
// LDS layouts (bank-conflict free for the fragment reads):
//   KC  row stride 72 halves (144 B): the 16 rows a ds_read_b128 pass touches
//       start at 16 distinct 4-bank groups.
//   RC  row (= k) stride chosen so that its byte size is 64 mod 256: the four
//       k rows one 32-lane pass of ds_read_b64_tr_b16 touches fill 4 disjoint
//       64-byte bank ranges.
//
// MFMA 32x32x16 lane layout (gfx950): lane l supplies A row / B row (l % 32)
// with k = (l/32)*8 + 0..7; accumulator value j of lane l is
// C[(j/4)*8 + (l/32)*4 + j%4][l % 32].  The kernel issues the product as
// B * A^T, so its accumulator holds the transposed tile: lane l owns C row
// l % 32 and four consecutive columns per group of four values.
//
// ds_read_b64_tr_b16 (gfx950): within each 16-lane group, lane i receives
// element (i % 4) of the 8-byte chunks addressed by lanes 4e + i/4, e = 0..3.
// With lanes 4e..4e+3 addressing 16 consecutive halves of LDS row e, lane i
// receives column i of rows 0..3: a 4 (k) x 16 (row) block, transposed.

#include <atomic>
#include <cstdlib>
#include <map>
#include <mutex>
#include <tuple>

#include "rv_device.h"

namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));  // 16-byte staging word
#define RV_LDS __attribute__((address_space(3)))

constexpr int kThreads = 256;
constexpr int kBK = 32;             // k per pipeline stage
#ifndef RV_ST_256x256
#define RV_ST_256x256 4
#endif
#ifndef RV_ST_128x256
#define RV_ST_128x256 3
#endif
#ifndef RV_ST_128x128
#define RV_ST_128x128 4
#endif
#ifndef RV_ST_64x128
#define RV_ST_64x128 4
#endif
// depth of the LDS ring per tile shape
constexpr int stages_for(int bm, int bn) {
  return bm == 256 ? RV_ST_256x256 : bn == 256 ? RV_ST_128x256 : bm == 128 ? RV_ST_128x128 : RV_ST_64x128;
}
constexpr int kCUs = 256;           // MI355X compute units (tile-shape choice only)
constexpr int kRsrcWord3 = 0x00020000;  // raw buffer resource, gfx9 data format

// XOR swizzles of the 16-byte chunk index inside one LDS row (see the layout
// notes at the top of the file).
__device__ __forceinline__ int f_kc(int row) { return ((row >> 2) & 3) ^ (row & 2); }
template <int ROWS>
__device__ __forceinline__ int f_rc(int k) {
  return ((ROWS >= 128 ? 0xCA60 : 0x6420) >> ((k & 3) * 4)) & 0xF;
}

// s_waitcnt with vmcnt = N and the other counters left alone (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Workgroup barrier that orders this wave's LDS accesses in program order
// (compiler barriers on both sides) without the release fence of
// __syncthreads, which would wait for every outstanding LDS DMA.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// ---------------------------------------------------------------------------
// Row maps for KC sources: LDS row r of the tile -> source row.
// ---------------------------------------------------------------------------
struct MapDirect {  // row0 + r, clamped to the last valid row (results never stored)
  int64_t row0, rows;
  __device__ __forceinline__ int64_t operator()(int r) const {
    const int64_t g = row0 + r;
    return g < rows ? g : rows - 1;
  }
};
// SwiGLU up projection: a BN-row B tile holds BN/2 output columns, as gate
// and value halves per wave column (WCOLS of them, C = BN/WCOLS rows each):
// rows [wn*C, wn*C + C/2) are gate rows col0 + wn*C/2 + w, the next C/2 are
// the value rows f + the same.
template <int BN, int WCOLS>
struct MapGateValue {
  int64_t col0, f;
  __device__ __forceinline__ int64_t operator()(int r) const {
    constexpr int kCol = BN / WCOLS, kHalf = kCol / 2;
    const int wn = r / kCol, w = r % kCol;
    return w < kHalf ? col0 + wn * kHalf + w : f + col0 + wn * kHalf + (w - kHalf);
  }
};

// ---------------------------------------------------------------------------
// Global -> LDS copies: direct-to-LDS buffer loads (buffer_load_dwordx4 ...
// lds).  One wave instruction fills 1 KB of LDS, lane L's 16 bytes at byte
// 16 L; each lane loads the source chunk whose swizzled LDS slot that is.
// A tile of ROWS rows is ROWS * 64 bytes per stage (kBK = 32 halves per row,
// or 32 k rows of ROWS halves), i.e. ROWS / 16 wave instructions, ROWS / 64
// per wave.  Per-lane source offsets are fixed; each stage adds a constant.
// ---------------------------------------------------------------------------
template <bool RC, int ROWS, int WAVES>
struct Dma {
  static constexpr int kPerWave = ROWS / 16 / WAVES;
  uint32_t off[kPerWave];  // byte offset of this lane's chunk at k = 0 of the kernel's range
  uint32_t kstep;          // bytes per stage
  __amdgpu_buffer_rsrc_t rsrc;

  // KC source [rows][ld] (k contiguous), tile rows row0..; rows past `rows`
  // are clamped (their results are never stored); map() gathers B rows.
  template <class Map>
  __device__ __forceinline__ void init_kc(const __half* base, int64_t bytes, int64_t ld,
                                          const Map& map, int64_t kbeg) {
    rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<__half*>(base), 0, (int)bytes, kRsrcWord3);
    kstep = kBK * 2;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
    for (int it = 0; it < kPerWave; ++it) {
      const int b = (it * WAVES + wave) * 1024 + lane * 16;
      const int row = b >> 6, chunk = ((b >> 4) & 3) ^ f_kc(row);
      off[it] = (uint32_t)((map(row) * ld + kbeg + chunk * 8) * 2);
    }
  }
  // RC source [k][ld] (tile rows contiguous from row0); k rows past the
  // resource's end read as zero (the buffer range check).
  __device__ __forceinline__ void init_rc(const __half* base, int64_t bytes, int64_t ld,
                                          int64_t row0, int64_t kbeg) {
    rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<__half*>(base), 0, (int)bytes, kRsrcWord3);
    kstep = (uint32_t)(kBK * ld * 2);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
    for (int it = 0; it < kPerWave; ++it) {
      const int b = (it * WAVES + wave) * 1024 + lane * 16;
      const int krow = b / (ROWS * 2), chunk = ((b % (ROWS * 2)) >> 4) ^ f_rc<ROWS>(krow);
      off[it] = (uint32_t)(((kbeg + krow) * ld + row0 + chunk * 8) * 2);
    }
  }
  // Issue wave instruction `it` of stage `st` into the tile at `lds`; with
  // live = false the offset is beyond any buffer's range (2 GiB > the
  // largest operand the entry points accept): no memory is read and the
  // lanes write zeros.
  __device__ __forceinline__ void issue_one(_Float16* lds, int st, int it, bool live) const {
    const int wave = threadIdx.x >> 6;
    const uint32_t voff = live ? off[it] + (uint32_t)st * kstep : 0x80000000u;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        rsrc, (RV_LDS void*)(lds + (it * WAVES + wave) * 512), 16, voff, 0, 0, 0);
  }
  // Issue stage `st` (relative to the kernel's first k) into the tile at `lds`.
  __device__ __forceinline__ void issue(_Float16* lds, int st) const {
    const int wave = threadIdx.x >> 6;
#pragma unroll
    for (int it = 0; it < kPerWave; ++it)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rsrc, (RV_LDS void*)(lds + (it * WAVES + wave) * 512), 16, off[it] + (uint32_t)st * kstep,
          0, 0, 0);
  }
};

// ---------------------------------------------------------------------------
// MFMA fragments: lane l -> tile row r0 + l%32, k = ks*16 + (l/32)*8 + 0..7.
// ---------------------------------------------------------------------------
__device__ __forceinline__ f16x8 frag_kc(const _Float16* lds, int r0, int ks, int lane) {
  const int row = r0 + (lane & 31);
  const int chunk = ks * 2 + (lane >> 5);
  return *reinterpret_cast<const f16x8*>(lds + row * kBK + ((chunk ^ f_kc(row)) << 3));
}

// ds_read_b64_tr_b16 as inline assembly: through the builtin, the compiler
// cannot tell the read from the in-flight LDS DMA writes and drains every
// outstanding DMA (vmcnt(0)) before each one.  Its result is therefore not
// tracked by the compiler's LDS counter: the k-step code waits for it
// explicitly (lds_ready) before the MFMAs that use it.
__device__ __forceinline__ i16x4 tr_read(const _Float16* p) {
  i16x4 r;
  asm volatile("ds_read_b64_tr_b16 %0, %1"
               : "=v"(r)
               : "v"((uint32_t)(size_t)(RV_LDS const void*)p));
  return r;
}

template <int ROWS>
__device__ __forceinline__ f16x8 frag_rc(const _Float16* lds, int r0, int ks, int lane) {
  const int g = lane >> 4, i = lane & 15;
  const int m = r0 + (g & 1) * 16 + 4 * (i & 3);
  const int k = ks * 16 + (g >> 1) * 8 + (i >> 2);
  const int k4 = k + 4;
  const i16x4 lo = tr_read(lds + k * ROWS + ((f_rc<ROWS>(k) ^ (m >> 3)) << 3) + (m & 7));
  const i16x4 hi = tr_read(lds + k4 * ROWS + ((f_rc<ROWS>(k4) ^ (m >> 3)) << 3) + (m & 7));
  const f16x4 a = __builtin_bit_cast(f16x4, lo), b = __builtin_bit_cast(f16x4, hi);
  return f16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// Wait for every LDS read of this wave, and pass a fragment through an empty
// asm after that wait so that its users cannot be scheduled before it.
__device__ __forceinline__ void lds_wait_all() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
__device__ __forceinline__ void after_wait(f16x8& v) { asm volatile("" : "+v"(v)); }

template <bool RC, int ROWS>
__device__ __forceinline__ f16x8 frag(const _Float16* lds, int r0, int ks, int lane) {
  if constexpr (RC) return frag_rc<ROWS>(lds, r0, ks, lane);
  else return frag_kc(lds, r0, ks, lane);
}

// ---------------------------------------------------------------------------
// The GEMM kernel.
// ---------------------------------------------------------------------------
enum class Epi {
  SwiGLU,         // c = o fp16 [m][n/2... per MapGateValue], optional u = [u_g | u_v]
  StoreF16,       // c fp16 = fp16(acc)
  SwiGLUBwd,      // c = du fp16 [m][2f] from u and d_o = fp16(acc)
  StoreF32OfF16,  // c fp32 = fp32(fp16(acc))
  AccF32OfF16,    // c fp32 (+)= fp32(fp16(acc))
  PartialF32,     // c fp32 partial [split][m][n] = acc
};

struct GemmArgs {
  const __half* a; int64_t lda; int64_t a_bytes;   // source, row stride, bytes addressable
  const __half* b; int64_t ldb; int64_t b_bytes;
  int64_t m, n, k;         // C rows, C columns (B rows), reduction length
  int64_t k_chunk;         // tokens per split (multiple of kBK); == k without split
  int64_t tiles_m, tiles_n;
  void* c; int64_t ldc;
  void* u; int64_t ldu;    // SwiGLU: optional u output; SwiGLUBwd: u input
  int64_t f;               // SwiGLU / SwiGLUBwd: value column offset
  int accumulate;          // AccF32OfF16
};

// Workgroups are dispatched to the 8 XCDs round robin.  Tiles are numbered in
// groups of 8 M-tiles (M fastest inside a group), and each XCD receives a
// contiguous range of tile numbers, so the workgroups sharing one XCD's L2 at
// a time cover a compact block of M x N tiles.
__device__ __forceinline__ void tile_of(int64_t t, int64_t tiles_m, int64_t tiles_n,
                                        int64_t& tm, int64_t& tn) {
  const int64_t tiles = tiles_m * tiles_n;
  if ((tiles & 7) == 0) t = (t & 7) * (tiles >> 3) + (t >> 3);
  const int64_t group = 8 * tiles_n;
  const int64_t g = t / group, r = t % group;
  const int64_t first = g * 8;
  const int64_t gm = tiles_m - first < 8 ? tiles_m - first : 8;
  tm = first + r % gm;
  tn = r / gm;
}

template <int BM, int BN, bool A_RC, bool B_RC, Epi EPI, int WAVES>
__global__ __launch_bounds__(WAVES * 64)
void gemm_kernel(GemmArgs args) {
  // waves: 2 rows x WCOLS columns, each owning a WM x WN block of the tile
  constexpr int WCOLS = WAVES / 2, WM = BM / 2, WN = BN / WCOLS;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int kStages = stages_for(BM, BN);
  constexpr int kA = BM * kBK, kB = BN * kBK;          // halves per stage and operand
  constexpr int kRing = kStages * (kA + kB);
  constexpr int kStaging = WAVES * WM * (WN + 8);  // fp16 epilogue staging
  __shared__ __attribute__((aligned(16))) _Float16 lds[kRing > kStaging ? kRing : kStaging];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave / WCOLS, wn = wave % WCOLS;

  const int64_t tiles = args.tiles_m * args.tiles_n;
  const int64_t split = blockIdx.x / tiles;
  int64_t tm, tn;
  tile_of(blockIdx.x % tiles, args.tiles_m, args.tiles_n, tm, tn);
  const int64_t m0 = tm * BM;
  const int64_t n0 = (EPI == Epi::SwiGLU) ? tn * (BN / 2) : tn * BN;
  const int64_t kbeg = split * args.k_chunk;
  const int64_t kend = kbeg + args.k_chunk < args.k ? kbeg + args.k_chunk : args.k;
  const int stages = kend > kbeg ? (int)((kend - kbeg + kBK - 1) / kBK) : 0;

  Dma<A_RC, BM, WAVES> da;
  Dma<B_RC, BN, WAVES> db;
  if constexpr (A_RC) da.init_rc(args.a, args.a_bytes, args.lda, m0, kbeg);
  else da.init_kc(args.a, args.a_bytes, args.lda, MapDirect{m0, args.m}, kbeg);
  if constexpr (B_RC) db.init_rc(args.b, args.b_bytes, args.ldb, n0, kbeg);
  else if constexpr (EPI == Epi::SwiGLU)
    db.init_kc(args.b, args.b_bytes, args.ldb, MapGateValue<BN, WCOLS>{n0, args.f}, kbeg);
  else db.init_kc(args.b, args.b_bytes, args.ldb, MapDirect{n0, args.n}, kbeg);

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  // Ring: stage st lives in buffer st % kStages.  The prologue issues the
  // DMA groups of stages 0 .. kStages-2 and loads the first k step's
  // fragments.  Iteration st then
  //   * waits for its own DMA of stage st + 1 and joins the workgroup, so all
  //     of stage st + 1 has landed and every wave is done with stage st - 1;
  //   * runs stage st's two k steps of MFMAs, issuing between them -- at
  //     fixed points (sched_barrier) -- the DMA group of stage
  //     st + kStages - 1 into stage st - 1's buffer, the fragments of its
  //     second k step, and the fragments of stage st + 1's first k step.
  // A group for a stage past the end is still issued, with an offset beyond
  // the buffer's range: it reads nothing from memory and writes zeros into a
  // buffer no later stage uses, and every iteration waits for the same
  // vmcnt.  Fragments prefetched past the last stage are never used.
  constexpr int kPerWaveA = Dma<A_RC, BM, WAVES>::kPerWave;
  constexpr int kPerWave = kPerWaveA + Dma<B_RC, BN, WAVES>::kPerWave;
  constexpr int kM = TM * TN, kF = TM + TN;
  f16x8 fa[2][TM], fb[2][TN];

#define RV_FRAG(SLOT, LA, LB, KS, P)                                                        \
  do {                                                                                      \
    if ((P) < TM) fa[SLOT][(P)] = frag<A_RC, BM>((LA), wm * WM + (P) * 32, (KS), lane);     \
    else fb[SLOT][(P) - TM] = frag<B_RC, BN>((LB), wn * WN + ((P) - TM) * 32, (KS), lane);  \
  } while (0)
#define RV_DMA(D, BUF, ST, LIVE)                                                            \
  do {                                                                                      \
    if ((D) < kPerWaveA) da.issue_one((BUF), (ST), (D), (LIVE));                             \
    else db.issue_one((BUF) + kA, (ST), (D) - kPerWaveA, (LIVE));                            \
  } while (0)
  // MFMAs of fragment slot SLOT; after MFMA q, DMA instruction d goes where
  // d * kM / kPerWave == q (if DO_DMA) and fragment f of (LA2, LB2, KS2) into
  // slot SLOT ^ 1 where f * kM / kF == q.
#define RV_KSTEP(SLOT, DO_DMA, DMABUF, DMAST, LIVE, LA2, LB2, KS2)                           \
  do {                                                                                      \
    if constexpr (A_RC || B_RC) {                                                           \
      lds_wait_all();                                                                       \
      _Pragma("unroll") for (int i_ = 0; i_ < TM; ++i_) after_wait(fa[SLOT][i_]);           \
      _Pragma("unroll") for (int j_ = 0; j_ < TN; ++j_) after_wait(fb[SLOT][j_]);           \
      __builtin_amdgcn_sched_barrier(0);                                                    \
    }                                                                                       \
    _Pragma("unroll") for (int q = 0; q < kM; ++q) {                                        \
      acc[q / TN][q % TN] = __builtin_amdgcn_mfma_f32_32x32x16_f16(                          \
          fb[SLOT][q % TN], fa[SLOT][q / TN], acc[q / TN][q % TN], 0, 0, 0);                \
      if (DO_DMA) {                                                                         \
        _Pragma("unroll") for (int d = 0; d < kPerWave; ++d) if (d * kM / kPerWave == q)    \
          RV_DMA(d, (DMABUF), (DMAST), (LIVE));                                             \
      }                                                                                     \
      _Pragma("unroll") for (int f = 0; f < kF; ++f) if (f * kM / kF == q)                  \
        RV_FRAG((SLOT) ^ 1, (LA2), (LB2), (KS2), f);                                        \
      __builtin_amdgcn_sched_barrier(0);                                                    \
    }                                                                                       \
  } while (0)

  if (stages > 0) {
#pragma unroll
    for (int p = 0; p < kStages - 1; ++p) {
      _Float16* buf = lds + p * (kA + kB);
#pragma unroll
      for (int d = 0; d < kPerWave; ++d) RV_DMA(d, buf, p, p < stages);
    }
    wait_vmcnt<(kStages - 2) * kPerWave>();
    lds_barrier();
#pragma unroll
    for (int f = 0; f < kF; ++f) RV_FRAG(0, lds, lds + kA, 0, f);
  }
  for (int st = 0; st < stages; ++st) {
    wait_vmcnt<(kStages - 3) * kPerWave>();
    lds_barrier();
    const _Float16* la = lds + (st % kStages) * (kA + kB);
    const _Float16* ln = lds + ((st + 1) % kStages) * (kA + kB);
    _Float16* dbuf = lds + ((st + kStages - 1) % kStages) * (kA + kB);
    const int dst = st + kStages - 1;
    RV_KSTEP(0, true, dbuf, dst, dst < stages, la, la + kA, 1);
    RV_KSTEP(1, false, dbuf, dst, false, ln, ln + kA, 0);
  }
  wait_vmcnt<0>();  // the trailing groups' zero writes land before the ring is reused
#undef RV_KSTEP
#undef RV_DMA
#undef RV_FRAG
  __syncthreads();  // every wave is done with the ring before the epilogue reuses it

  // ---- epilogue ----
  // The MFMA is issued as B * A^T, so each lane holds C row (lane % 32) of
  // its 32x32 tile and, for q = 0..3, the 4 consecutive columns
  // q*8 + (lane/32)*4 + 0..3 (accumulator values 4q..4q+3).
  const int cq = (lane >> 5) * 4;
  if constexpr (EPI == Epi::PartialF32 || EPI == Epi::StoreF32OfF16 ||
                EPI == Epi::AccF32OfF16) {
    // fp32 outputs: 16-byte stores straight from the accumulators.
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int64_t row = m0 + wm * WM + i * 32 + (lane & 31);
      if (row >= args.m) continue;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int64_t col = n0 + wn * WN + j * 32 + q * 8 + cq;
          const float a0 = acc[i][j][q * 4], a1 = acc[i][j][q * 4 + 1];
          const float a2 = acc[i][j][q * 4 + 2], a3 = acc[i][j][q * 4 + 3];
          if constexpr (EPI == Epi::PartialF32) {
            *reinterpret_cast<float4*>(static_cast<float*>(args.c) +
                                       (split * args.m + row) * args.ldc + col) =
                make_float4(a0, a1, a2, a3);
          } else {
            float4 r = make_float4(rv::round_to<__half>(a0), rv::round_to<__half>(a1),
                                   rv::round_to<__half>(a2), rv::round_to<__half>(a3));
            float4* c = reinterpret_cast<float4*>(static_cast<float*>(args.c) + row * args.ldc + col);
            if constexpr (EPI == Epi::AccF32OfF16) {
              if (args.accumulate) {
                const float4 p = *c;
                r = make_float4(p.x + r.x, p.y + r.y, p.z + r.z, p.w + r.w);
              }
            }
            *c = r;
          }
        }
      }
    }
  } else {
    // fp16 outputs: each wave stages fp16(acc) for its WM x WN block in LDS
    // (row stride WN + 8 halves), then moves whole rows, 16 bytes per lane,
    // so every global access instruction covers full row segments.  The
    // stores are streaming (nt): measured 1-5% faster per GEMM and 0.3-0.5%
    // per configs[3]/[4] training step, consumers included.
    constexpr int S = WN + 8;
    _Float16* stage = lds + wave * (WM * S);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const __half2 h01 = __floats2half2_rn(acc[i][j][q * 4], acc[i][j][q * 4 + 1]);
          const __half2 h23 = __floats2half2_rn(acc[i][j][q * 4 + 2], acc[i][j][q * 4 + 3]);
          uint2 p;
          p.x = *reinterpret_cast<const uint32_t*>(&h01);
          p.y = *reinterpret_cast<const uint32_t*>(&h23);
          *reinterpret_cast<uint2*>(stage + (i * 32 + (lane & 31)) * S + j * 32 + q * 8 + cq) = p;
        }
    // each wave reads back only its own staged block: a wave-local wait
    // instead of a workgroup barrier, so a wave stores as soon as it has staged
    lds_wait_all();
    __builtin_amdgcn_wave_barrier();
    const int64_t row0 = m0 + wm * WM;
    if constexpr (EPI == Epi::SwiGLU) {
      // gate in staged columns [0, WN/2), value in [WN/2, WN)
      constexpr int CPR = WN / 16, RPP = 64 / CPR;
      const int c = lane % CPR;
      __half* u = static_cast<__half*>(args.u);
      const int64_t col = n0 + wn * (WN / 2) + c * 8;
#pragma unroll 4
      for (int r = lane / CPR; r < WM; r += RPP) {
        const int64_t row = row0 + r;
        if (row >= args.m) break;
        const u32x4 gw = *reinterpret_cast<const u32x4*>(stage + r * S + c * 8);
        const u32x4 vw = *reinterpret_cast<const u32x4*>(stage + r * S + WN / 2 + c * 8);
        const __half* gh = reinterpret_cast<const __half*>(&gw);
        const __half2* vh2 = reinterpret_cast<const __half2*>(&vw);
        // silu rounded to fp16, times v: the exact product of two fp16 values
        // rounded once, so the packed fp16 multiply gives the fp32 expression's
        // bits two values per instruction
        __half2 oh[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float g0 = __half2float(gh[2 * e]), g1 = __half2float(gh[2 * e + 1]);
          const __half2 silu = __floats2half2_rn(g0 * rv::fast_sigmoid(g0),
                                                 g1 * rv::fast_sigmoid(g1));
          oh[e] = __hmul2(silu, vh2[e]);
        }
        __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>(oh), reinterpret_cast<u32x4*>(static_cast<__half*>(args.c) + row * args.ldc + col));
        if (u != nullptr) {
          __builtin_nontemporal_store(gw, reinterpret_cast<u32x4*>(u + row * args.ldu + col));
          __builtin_nontemporal_store(vw, reinterpret_cast<u32x4*>(u + row * args.ldu + args.f + col));
        }
      }
    } else if constexpr (EPI == Epi::StoreF16) {
      constexpr int CPR = WN / 8, RPP = 64 / CPR;
      const int c = lane % CPR;
      const int64_t col = n0 + wn * WN + c * 8;
#pragma unroll 4
      for (int r = lane / CPR; r < WM; r += RPP) {
        const int64_t row = row0 + r;
        if (row >= args.m) break;
        const u32x4 dw = *reinterpret_cast<const u32x4*>(stage + r * S + c * 8);
        __builtin_nontemporal_store(dw, reinterpret_cast<u32x4*>(static_cast<__half*>(args.c) + row * args.ldc + col));
      }
    } else {
      // SwiGLUBwd: du from u = [gate | value] and d_o = fp16(acc).  The u
      // reads of up to 16 of a lane's rows are issued together (the
      // accumulators are in LDS by now, their registers free), so the tile's
      // epilogue waits on one memory round trip per 16 rows instead of one
      // per 4; rows past m read the last row and store nothing.
      constexpr int CPR = WN / 8, RPP = 64 / CPR;
      constexpr int ITER = WM / RPP;              // rows per lane
      constexpr int CH = ITER < 16 ? ITER : 16;   // rows whose u reads are in flight together
      static_assert(ITER % CH == 0, "epilogue row chunks");
      const int c = lane % CPR;
      const int64_t col = n0 + wn * WN + c * 8;
      const __half* ubase = static_cast<const __half*>(args.u);
#pragma unroll
      for (int r0 = 0; r0 < ITER; r0 += CH) {
        u32x4 gw[CH], vw[CH];
#pragma unroll
        for (int i = 0; i < CH; ++i) {
          const int64_t rr = row0 + lane / CPR + (r0 + i) * RPP;
          const __half* ur = ubase + (rr < args.m ? rr : args.m - 1) * args.ldu;
          gw[i] = *reinterpret_cast<const u32x4*>(ur + col);
          vw[i] = *reinterpret_cast<const u32x4*>(ur + args.f + col);
        }
#pragma unroll
        for (int i = 0; i < CH; ++i) {
          const int r = lane / CPR + (r0 + i) * RPP;
          const int64_t row = row0 + r;
          if (row < args.m) {
            const u32x4 dw = *reinterpret_cast<const u32x4*>(stage + r * S + c * 8);
            const __half2* dh2 = reinterpret_cast<const __half2*>(&dw);
            const __half* gh = reinterpret_cast<const __half*>(&gw[i]);
            const __half2* vh2 = reinterpret_cast<const __half2*>(&vw[i]);
            // d*v and d*silu are products of two fp16 values rounded to fp16
            // once: packed fp16 multiplies, the same bits as the fp32 forms
            __half2 dgo[4], dvo[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float g0 = __half2float(gh[2 * e]), g1 = __half2float(gh[2 * e + 1]);
              const float s0 = rv::fast_sigmoid(g0), s1 = rv::fast_sigmoid(g1);
              const __half2 silu = __floats2half2_rn(g0 * s0, g1 * s1);
              const __half2 dgi = __hmul2(dh2[e], vh2[e]);
              dgo[e] = __floats2half2_rn(__low2float(dgi) * (s0 * (1.0f + g0 * (1.0f - s0))),
                                         __high2float(dgi) * (s1 * (1.0f + g1 * (1.0f - s1))));
              dvo[e] = __hmul2(dh2[e], silu);
            }
            __half* du = static_cast<__half*>(args.c) + row * args.ldc;
            __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>(dgo), reinterpret_cast<u32x4*>(du + col));
            __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>(dvo), reinterpret_cast<u32x4*>(du + args.f + col));
          }
        }
      }
    }
  }
}

// Explicit instantiations of every (tile shape, operand layout, epilogue) the
// host dispatch can launch.  Without them this compiler emits the host-side
// launch stubs of only some of the kernels reached through the dispatch
// switch, and the library fails to load with undefined symbols.
template __global__ void gemm_kernel<256, 256, false, false, Epi::SwiGLU, 4>(GemmArgs);
template __global__ void gemm_kernel<256, 256, false, false, Epi::StoreF16, 4>(GemmArgs);
template __global__ void gemm_kernel<256, 256, false, true, Epi::SwiGLUBwd, 4>(GemmArgs);
template __global__ void gemm_kernel<256, 256, false, true, Epi::StoreF32OfF16, 4>(GemmArgs);
template __global__ void gemm_kernel<256, 256, true, true, Epi::AccF32OfF16, 4>(GemmArgs);
template __global__ void gemm_kernel<256, 256, true, true, Epi::PartialF32, 4>(GemmArgs);
template __global__ void gemm_kernel<128, 256, false, false, Epi::SwiGLU, 4>(GemmArgs);
template __global__ void gemm_kernel<128, 256, false, false, Epi::StoreF16, 4>(GemmArgs);
template __global__ void gemm_kernel<128, 256, false, true, Epi::SwiGLUBwd, 4>(GemmArgs);
template __global__ void gemm_kernel<128, 256, false, true, Epi::StoreF32OfF16, 4>(GemmArgs);
template __global__ void gemm_kernel<128, 256, true, true, Epi::AccF32OfF16, 4>(GemmArgs);
template __global__ void gemm_kernel<128, 256, true, true, Epi::PartialF32, 4>(GemmArgs);
template __global__ void gemm_kernel<128, 128, false, false, Epi::SwiGLU, 4>(GemmArgs);
template __global__ void gemm_kernel<128, 128, false, false, Epi::StoreF16, 4>(GemmArgs);
template __global__ void gemm_kernel<128, 128, false, true, Epi::SwiGLUBwd, 4>(GemmArgs);
template __global__ void gemm_kernel<128, 128, false, true, Epi::StoreF32OfF16, 4>(GemmArgs);
template __global__ void gemm_kernel<128, 128, true, true, Epi::AccF32OfF16, 4>(GemmArgs);
template __global__ void gemm_kernel<128, 128, true, true, Epi::PartialF32, 4>(GemmArgs);
template __global__ void gemm_kernel<64, 128, false, false, Epi::SwiGLU, 4>(GemmArgs);
template __global__ void gemm_kernel<64, 128, false, false, Epi::StoreF16, 4>(GemmArgs);
template __global__ void gemm_kernel<64, 128, false, true, Epi::SwiGLUBwd, 4>(GemmArgs);
template __global__ void gemm_kernel<64, 128, false, true, Epi::StoreF32OfF16, 4>(GemmArgs);
template __global__ void gemm_kernel<64, 128, true, true, Epi::AccF32OfF16, 4>(GemmArgs);
template __global__ void gemm_kernel<64, 128, true, true, Epi::PartialF32, 4>(GemmArgs);

template __global__ void gemm_kernel<256, 256, false, true, Epi::StoreF16, 4>(GemmArgs);
template __global__ void gemm_kernel<128, 256, false, true, Epi::StoreF16, 4>(GemmArgs);
template __global__ void gemm_kernel<128, 128, false, true, Epi::StoreF16, 4>(GemmArgs);
template __global__ void gemm_kernel<64, 128, false, true, Epi::StoreF16, 4>(GemmArgs);
template __global__ void gemm_kernel<256, 256, false, false, Epi::SwiGLU, 8>(GemmArgs);
template __global__ void gemm_kernel<256, 256, false, false, Epi::StoreF16, 8>(GemmArgs);
template __global__ void gemm_kernel<256, 256, false, true, Epi::SwiGLUBwd, 8>(GemmArgs);
template __global__ void gemm_kernel<256, 256, false, true, Epi::StoreF32OfF16, 8>(GemmArgs);
template __global__ void gemm_kernel<256, 256, true, true, Epi::AccF32OfF16, 8>(GemmArgs);
template __global__ void gemm_kernel<256, 256, true, true, Epi::PartialF32, 8>(GemmArgs);
template __global__ void gemm_kernel<256, 256, false, true, Epi::StoreF16, 8>(GemmArgs);

// acc[i] (+)= fp32(fp16(sum_s part[s][i])), splits summed in order.  This is
// autocast's weight gradient: the fp16 GEMM result, cast to the fp32 weight
// and added to the running per-tile sum.  n % 4 == 0.  One launch finishes up
// to two weight gradients: blocks [0, a.blocks) reduce segment a, the rest b.
struct ReduceSeg {
  const float* part;
  float* out;
  int64_t n;
  int splits;
  int64_t blocks;  // 0: nothing to reduce
};

__global__ __launch_bounds__(256)
void wgrad_reduce(ReduceSeg a, ReduceSeg b, int accumulate) {
  const bool second = (int64_t)blockIdx.x >= a.blocks;
  const float* part = second ? b.part : a.part;
  float* out = second ? b.out : a.out;
  const int64_t n = second ? b.n : a.n;
  const int splits = second ? b.splits : a.splits;
  const int64_t blk = second ? (int64_t)blockIdx.x - a.blocks : (int64_t)blockIdx.x;
  const int64_t i = (blk * 256 + threadIdx.x) * 4;
  if (i >= n) return;
  float4 s = *reinterpret_cast<const float4*>(part + i);
  // the partials of eight splits loaded before the first of their adds (one
  // memory round trip per eight splits instead of per split); same order
  int k = 1;
  for (; k + 8 <= splits; k += 8) {
    float4 t[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      t[j] = *reinterpret_cast<const float4*>(part + (int64_t)(k + j) * n + i);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      s.x = s.x + t[j].x; s.y = s.y + t[j].y; s.z = s.z + t[j].z; s.w = s.w + t[j].w;
    }
  }
  for (; k < splits; ++k) {
    const float4 t = *reinterpret_cast<const float4*>(part + (int64_t)k * n + i);
    s.x = s.x + t.x; s.y = s.y + t.y; s.z = s.z + t.z; s.w = s.w + t.w;
  }
  float4 r = make_float4(rv::round_to<__half>(s.x), rv::round_to<__half>(s.y),
                         rv::round_to<__half>(s.z), rv::round_to<__half>(s.w));
  float4* o = reinterpret_cast<float4*>(out + i);
  if (accumulate) {
    const float4 p = *o;
    r = make_float4(p.x + r.x, p.y + r.y, p.z + r.z, p.w + r.w);
  }
  *o = r;
}

// dst = fp16(src), round to nearest even; 8 elements per thread.
__global__ __launch_bounds__(256)
void cast_f32_f16(const float* __restrict__ src, __half* __restrict__ dst, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * 256 * 8;
  for (int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8; i < n; i += stride) {
    if (i + 8 <= n) {
      const float4 a = *reinterpret_cast<const float4*>(src + i);
      const float4 b = *reinterpret_cast<const float4*>(src + i + 4);
      const __half2 h0 = __floats2half2_rn(a.x, a.y), h1 = __floats2half2_rn(a.z, a.w);
      const __half2 h2 = __floats2half2_rn(b.x, b.y), h3 = __floats2half2_rn(b.z, b.w);
      uint4 v;
      v.x = *reinterpret_cast<const uint32_t*>(&h0);
      v.y = *reinterpret_cast<const uint32_t*>(&h1);
      v.z = *reinterpret_cast<const uint32_t*>(&h2);
      v.w = *reinterpret_cast<const uint32_t*>(&h3);
      *reinterpret_cast<uint4*>(dst + i) = v;
    } else {
      for (int64_t j = i; j < n; ++j) dst[j] = __float2half_rn(src[j]);
    }
  }
}

// dst[t] = fp16(src[t]) for up to kCastTensors tensors in one launch: the
// pointer table and per-tensor chunk prefix sums travel in the kernel
// arguments; each workgroup casts one kCastChunk-element chunk of one tensor
// with cast_f32_f16's arithmetic.
constexpr int kCastTensors = 64;
constexpr int64_t kCastChunk = 256 * 8 * 16;
struct CastTable {
  const float* src[kCastTensors];
  __half* dst[kCastTensors];
  int64_t n[kCastTensors];
  int chunk_start[kCastTensors + 1];
  int count;
};

__global__ __launch_bounds__(256)
void cast_multi_k(CastTable tab) {
  int t = 0;
  for (int i = 1; i < tab.count; ++i)
    if (tab.chunk_start[i] <= (int)blockIdx.x) t = i;
  const int64_t base = (int64_t)(blockIdx.x - tab.chunk_start[t]) * kCastChunk;
  const int64_t n = tab.n[t];
  const float* src = tab.src[t];
  __half* dst = tab.dst[t];
  const int64_t end = base + kCastChunk < n ? base + kCastChunk : n;
  for (int64_t i = base + threadIdx.x * 8; i < end; i += 256 * 8) {
    if (i + 8 <= end) {
      const float4 a = *reinterpret_cast<const float4*>(src + i);
      const float4 b = *reinterpret_cast<const float4*>(src + i + 4);
      const __half2 h0 = __floats2half2_rn(a.x, a.y), h1 = __floats2half2_rn(a.z, a.w);
      const __half2 h2 = __floats2half2_rn(b.x, b.y), h3 = __floats2half2_rn(b.z, b.w);
      uint4 v;
      v.x = *reinterpret_cast<const uint32_t*>(&h0);
      v.y = *reinterpret_cast<const uint32_t*>(&h1);
      v.z = *reinterpret_cast<const uint32_t*>(&h2);
      v.w = *reinterpret_cast<const uint32_t*>(&h3);
      *reinterpret_cast<uint4*>(dst + i) = v;
    } else {
      for (int64_t j = i; j < end; ++j) dst[j] = __float2half_rn(src[j]);
    }
  }
}

// ---------------------------------------------------------------------------
// Host side: tile-shape choice and launches.
// ---------------------------------------------------------------------------
struct TileShape {
  int bm, bn, waves;
};
// The first kRuleShapes are the ones pick_act's rule and the weight-gradient
// plan choose from; the tuner also times the rest (256 x 256 with 8 waves:
// two waves per SIMD, each owning a 128 x 64 block).
constexpr int kNumShapes = 5, kRuleShapes = 4;
constexpr TileShape kShapes[kNumShapes] = {
    {256, 256, 4}, {128, 256, 4}, {128, 128, 4}, {64, 128, 4}, {256, 256, 8}};

template <bool A_RC, bool B_RC, Epi EPI>
int launch(int shape, const GemmArgs& a, int64_t splits, hipStream_t s) {
  const dim3 grid((unsigned)(a.tiles_m * a.tiles_n * splits)), block(kShapes[shape].waves * 64);
  switch (shape) {
    case 0: hipLaunchKernelGGL((gemm_kernel<256, 256, A_RC, B_RC, EPI, 4>), grid, block, 0, s, a); break;
    case 1: hipLaunchKernelGGL((gemm_kernel<128, 256, A_RC, B_RC, EPI, 4>), grid, block, 0, s, a); break;
    case 2: hipLaunchKernelGGL((gemm_kernel<128, 128, A_RC, B_RC, EPI, 4>), grid, block, 0, s, a); break;
    case 3: hipLaunchKernelGGL((gemm_kernel<64, 128, A_RC, B_RC, EPI, 4>), grid, block, 0, s, a); break;
    default: hipLaunchKernelGGL((gemm_kernel<256, 256, A_RC, B_RC, EPI, 8>), grid, block, 0, s, a); break;
  }
  return rv_host::check_launch();
}

// Activation GEMMs: C is m x n_out where n_out = n (or n/2 output columns for
// SwiGLU, whose tile covers bn/2 of them).  The largest tile that gives at
// least one workgroup per CU; otherwise the one with the most workgroups.
int pick_act(int64_t m, int64_t n_cols, bool swiglu) {
  int best = -1;
  int64_t best_blocks = -1;
  for (int i = 0; i < kRuleShapes; ++i) {
    const int64_t cols = swiglu ? kShapes[i].bn / 2 : kShapes[i].bn;
    if (n_cols % cols) continue;
    const int64_t blocks = ((m + kShapes[i].bm - 1) / kShapes[i].bm) * (n_cols / cols);
    if (blocks >= kCUs) return i;
    if (blocks > best_blocks) best = i, best_blocks = blocks;
  }
  return best;
}

// Measured tile choice.  The fastest tile shape of an activation GEMM depends
// on more than the grid size (how the last round of workgroups fills the
// chip, two workgroups per CU overlapping one's epilogue with the other's
// MFMAs, the k loop's length), and the shape never changes a result bit: every
// output element sums its k blocks in the same order in every shape.  So the
// first call for each (epilogue and its outputs, operand layouts, m, n, k)
// times every shape that fits (one warm-up launch, then two timed ones on the
// caller's stream, which is synchronised after each shape; two sweeps, each
// shape's faster one counting) and keeps the fastest.  The epilogues tuned
// here overwrite their outputs, so the extra launches write the same values.
// A call made while its stream is being captured into a graph never tunes
// (that would synchronise): it takes the shape already chosen for its key,
// else pick_act's rule.  RV_GEMM_TUNE=0 in the environment turns tuning off.
using TuneKey = std::tuple<int, int, int, int64_t, int64_t, int64_t>;
std::atomic<int> g_forced_shape{-1};  // rv_gemm_force_shape; -1: measured / rule choice
std::mutex g_tune_mu;
std::map<TuneKey, int> g_tuned;

bool tuning_enabled() {
  static const bool on = [] {
    const char* v = std::getenv("RV_GEMM_TUNE");
    return !(v && v[0] == '0');
  }();
  return on;
}

bool capturing(hipStream_t s) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &st) != hipSuccess) return true;  // then do not tune
  return st != hipStreamCaptureStatusNone;
}

template <bool A_RC, bool B_RC, Epi EPI>
int launch_shape(int shape, GemmArgs a, int64_t n_cols, hipStream_t s) {
  const bool swiglu = EPI == Epi::SwiGLU;
  const TileShape t = kShapes[shape];
  a.tiles_m = (a.m + t.bm - 1) / t.bm;
  a.tiles_n = n_cols / (swiglu ? t.bn / 2 : t.bn);
  a.k_chunk = a.k;
  return launch<A_RC, B_RC, EPI>(shape, a, 1, s);
}

template <bool A_RC, bool B_RC, Epi EPI>
int tune_act(const GemmArgs& a, int64_t n_cols, hipStream_t s, int fallback) {
  const bool swiglu = EPI == Epi::SwiGLU;
  hipEvent_t e0, e1;
  if (hipEventCreate(&e0) != hipSuccess) return fallback;
  if (hipEventCreate(&e1) != hipSuccess) {
    (void)hipEventDestroy(e0);
    return fallback;
  }
  // two sweeps over the shapes, each shape keeping its faster one: a clock or
  // cache transient during one sweep does not decide the choice alone
  float ms_of[kNumShapes] = {};
  for (int sweep = 0; sweep < 2; ++sweep)
    for (int i = 0; i < kNumShapes; ++i) {
      const int64_t cols = swiglu ? kShapes[i].bn / 2 : kShapes[i].bn;
      if (n_cols % cols) continue;
      if (launch_shape<A_RC, B_RC, EPI>(i, a, n_cols, s) != RV_OK) continue;
      bool ok = hipEventRecord(e0, s) == hipSuccess;
      ok = ok && launch_shape<A_RC, B_RC, EPI>(i, a, n_cols, s) == RV_OK;
      ok = ok && launch_shape<A_RC, B_RC, EPI>(i, a, n_cols, s) == RV_OK;
      ok = ok && hipEventRecord(e1, s) == hipSuccess && hipEventSynchronize(e1) == hipSuccess;
      float ms = 0.f;
      ok = ok && hipEventElapsedTime(&ms, e0, e1) == hipSuccess;
      if (ok && ms > 0.f && (ms_of[i] == 0.f || ms < ms_of[i])) ms_of[i] = ms;
    }
  int best = fallback;
  float best_ms = 0.f;
  for (int i = 0; i < kNumShapes; ++i)
    if (ms_of[i] > 0.f && (best_ms == 0.f || ms_of[i] < best_ms)) best = i, best_ms = ms_of[i];
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  return best;
}

template <bool A_RC, bool B_RC, Epi EPI>
int run_act(GemmArgs a, int64_t n_cols, hipStream_t s) {
  const bool swiglu = EPI == Epi::SwiGLU;
  int shape = pick_act(a.m, n_cols, swiglu);
  if (shape < 0) return RV_ERR_UNSUPPORTED;
  const int forced = g_forced_shape.load();
  if (forced >= 0) {
    if (n_cols % (swiglu ? kShapes[forced].bn / 2 : kShapes[forced].bn)) return RV_ERR_UNSUPPORTED;
    return launch_shape<A_RC, B_RC, EPI>(forced, a, n_cols, s);
  }
  if (tuning_enabled()) {
    int device = 0;
    (void)hipGetDevice(&device);
    // the SwiGLU epilogue with and without its u output store different
    // amounts and are tuned apart
    const int variant = (EPI == Epi::SwiGLU && a.u != nullptr) ? 1 : 0;
    const TuneKey key{(int)EPI * 4 + (A_RC ? 2 : 0) + (B_RC ? 1 : 0), device, variant, a.m,
                      n_cols, a.k};
    std::lock_guard<std::mutex> lock(g_tune_mu);
    const auto it = g_tuned.find(key);
    if (it != g_tuned.end()) {
      shape = it->second;
    } else if (!capturing(s)) {
      shape = tune_act<A_RC, B_RC, EPI>(a, n_cols, s, shape);
      g_tuned[key] = shape;
    }
  }
  return launch_shape<A_RC, B_RC, EPI>(shape, a, n_cols, s);
}

// Weight-gradient plan for an ni x nj output reduced over `rows` tokens: tile
// shape and split count minimising a simple cost (MFMA time at a per-shape
// efficiency, divided by the fraction of the grid's CU rounds that hold a
// workgroup, plus the partial sums' HBM round trip at ~250 flop per byte; at
// 500 the 8192-token tiles' weight gradients kept fewer splits on smaller
// tiles and took 45.3 us (d 256, f 1024) and 267 us (d 1024, f 4096) against
// 42.6 and 261 us).
// The split count is the largest that keeps tiles x splits within one round
// of the CUs: a grid a few workgroups past the CU count (C5's qkv weight
// gradient: 96 tiles x 3 splits = 288) leaves those CUs a second turn and
// nearly doubles the kernel.  Depends only on the sizes, so results are
// device-independent.
struct WgradPlan {
  int shape;
  int64_t tiles_m, tiles_n, splits, chunk;
};
WgradPlan plan_wgrad(int64_t rows, int64_t ni, int64_t nj) {
  // per-shape efficiencies measured on the split-K weight gradients (the
  // 128 x 256 tile's 0.55: at C5's attention-projection shape, 1024 x 1024
  // over 32768 tokens, it took 113 us with 8 splits where 256 x 256 with 16
  // takes 85 us, partial sums and their reduce included)
  static const double eff[kRuleShapes] = {0.8, 0.55, 0.5, 0.35};
  WgradPlan best{-1, 0, 0, 0, 0};
  double best_cost = 0;
  for (int i = 0; i < kRuleShapes; ++i) {
    const TileShape t = kShapes[i];
    if (ni % t.bm || nj % t.bn) continue;
    const int64_t tiles = (ni / t.bm) * (nj / t.bn);
    int64_t splits = tiles >= kCUs ? 1 : kCUs / tiles;
    const int64_t max_splits = (rows + 4 * kBK - 1) / (4 * kBK);  // >= 4 stages per split
    if (splits > max_splits) splits = max_splits;
    if (splits > 64) splits = 64;
    if (splits < 1) splits = 1;
    int64_t chunk = (rows + splits - 1) / splits;
    chunk = (chunk + kBK - 1) / kBK * kBK;
    splits = (rows + chunk - 1) / chunk;
    const int64_t wgs = tiles * splits, rounds = (wgs + kCUs - 1) / kCUs;
    const double fill = (double)wgs / (double)(rounds * kCUs);
    const double flops = 2.0 * rows * ni * nj / (eff[i] * fill);
    const double bytes = splits > 1 ? 8.0 * splits * ni * nj : 0.0;
    const double cost = flops + 250.0 * bytes;
    if (best.shape < 0 || cost < best_cost) {
      best = WgradPlan{i, ni / t.bm, nj / t.bn, splits, chunk};
      best_cost = cost;
    }
  }
  return best;
}

// The weight-gradient GEMM.  Unsplit, it writes (or adds) the result itself;
// split, its fp32 partial sums go to `part` and `seg` describes the reduction
// still to launch (seg.blocks == 0 otherwise).
int launch_wgrad(const __half* a, int64_t lda, const __half* b, int64_t ldb, int64_t rows,
                 int64_t ni, int64_t nj, float* out, int accumulate, float* part,
                 ReduceSeg& seg, hipStream_t s) {
  seg = ReduceSeg{nullptr, nullptr, 0, 0, 0};
  const WgradPlan p = plan_wgrad(rows, ni, nj);
  if (p.shape < 0) return RV_ERR_UNSUPPORTED;
  GemmArgs g{};
  g.a = a; g.lda = lda; g.a_bytes = rows * lda * 2;
  g.b = b; g.ldb = ldb; g.b_bytes = rows * ldb * 2;
  g.m = ni; g.n = nj; g.k = rows; g.k_chunk = p.chunk;
  g.tiles_m = p.tiles_m; g.tiles_n = p.tiles_n;
  g.ldc = nj; g.accumulate = accumulate;
  if (p.splits == 1) {
    g.c = out;
    return launch<true, true, Epi::AccF32OfF16>(p.shape, g, 1, s);
  }
  g.c = part;
  const int st = launch<true, true, Epi::PartialF32>(p.shape, g, p.splits, s);
  if (st != RV_OK) return st;
  const int64_t n = ni * nj;
  seg = ReduceSeg{part, out, n, (int)p.splits, (n / 4 + 255) / 256};
  return RV_OK;
}

int launch_reduce(const ReduceSeg& a, const ReduceSeg& b, int accumulate, hipStream_t s) {
  const int64_t blocks = a.blocks + b.blocks;
  if (blocks == 0) return RV_OK;
  hipLaunchKernelGGL(wgrad_reduce, dim3((unsigned)blocks), dim3(256), 0, s, a, b, accumulate);
  return rv_host::check_launch();
}

int run_wgrad(const __half* a, int64_t lda, const __half* b, int64_t ldb, int64_t rows,
              int64_t ni, int64_t nj, float* out, int accumulate, float* part, hipStream_t s) {
  ReduceSeg seg;
  const int st = launch_wgrad(a, lda, b, ldb, rows, ni, nj, out, accumulate, part, seg, s);
  if (st != RV_OK) return st;
  return launch_reduce(seg, ReduceSeg{nullptr, nullptr, 0, 0, 0}, accumulate, s);
}

int64_t wgrad_part_bytes(int64_t rows, int64_t ni, int64_t nj) {
  const WgradPlan p = plan_wgrad(rows, ni, nj);
  if (p.shape < 0) return -1;
  return p.splits > 1 ? p.splits * ni * nj * (int64_t)sizeof(float) : 0;
}

bool ok16(const void* p) { return rv_host::aligned16(p); }

int64_t align256(int64_t bytes) { return (bytes + 255) & ~(int64_t)255; }

// Buffer loads address an operand with 32-bit byte offsets.
bool fits32(int64_t elems) { return elems > 0 && elems * 2 <= (int64_t)INT32_MAX - (int64_t)(1 << 24); }

}  // namespace

extern "C" {

int rv_gemm_num_shapes(void) { return kNumShapes; }

int rv_gemm_force_shape(int shape) {
  if (shape < -1 || shape >= kNumShapes) return RV_ERR_BAD_SIZE;
  g_forced_shape.store(shape);
  return RV_OK;
}

int rv_cast_f32_f16(const float* src, void* dst, int64_t n, void* stream) {
  if (!src || !dst) return RV_ERR_NULL_POINTER;
  if (n < 0) return RV_ERR_BAD_SIZE;
  if (n == 0) return RV_OK;
  if (!ok16(src) || !ok16(dst)) return RV_ERR_UNSUPPORTED;
  int64_t blocks = (n + 256 * 8 - 1) / (256 * 8);
  if (blocks > 8 * kCUs) blocks = 8 * kCUs;
  hipLaunchKernelGGL(cast_f32_f16, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, src,
                     static_cast<__half*>(dst), n);
  return rv_host::check_launch();
}

int rv_cast_f32_f16_max_tensors(void) { return kCastTensors; }

int rv_cast_f32_f16_multi(int count, const float* const* src, void* const* dst,
                          const int64_t* numel, void* stream) {
  if (count < 0) return RV_ERR_BAD_SIZE;
  if (count == 0) return RV_OK;
  if (!src || !dst || !numel) return RV_ERR_NULL_POINTER;
  if (count > kCastTensors) return RV_ERR_UNSUPPORTED;
  CastTable tab{};
  int64_t chunks = 0;
  for (int i = 0; i < count; ++i) {
    if (!src[i] || !dst[i]) return RV_ERR_NULL_POINTER;
    if (numel[i] < 0) return RV_ERR_BAD_SIZE;
    if (!ok16(src[i]) || !ok16(dst[i])) return RV_ERR_UNSUPPORTED;
    tab.src[i] = src[i];
    tab.dst[i] = static_cast<__half*>(dst[i]);
    tab.n[i] = numel[i];
    tab.chunk_start[i] = (int)chunks;
    chunks += (numel[i] + kCastChunk - 1) / kCastChunk;
    if (chunks > 0x7fffffff) return RV_ERR_UNSUPPORTED;
  }
  tab.chunk_start[count] = (int)chunks;
  tab.count = count;
  if (chunks == 0) return RV_OK;
  hipLaunchKernelGGL(cast_multi_k, dim3((unsigned)chunks), dim3(256), 0, (hipStream_t)stream, tab);
  return rv_host::check_launch();
}

int rv_mlp_up_swiglu(const void* x, int64_t ldx, const void* w_up, int64_t rows, int64_t d,
                     int64_t f, void* o, void* u, void* stream) {
  if (!x || !w_up || !o) return RV_ERR_NULL_POINTER;
  if (rows <= 0 || d <= 0 || f <= 0 || ldx < d) return RV_ERR_BAD_SIZE;
  if (d % kBK || f % 64 || ldx % 8) return RV_ERR_UNSUPPORTED;
  if (!ok16(x) || !ok16(w_up) || !ok16(o) || (u && !ok16(u))) return RV_ERR_UNSUPPORTED;
  if (!fits32(rows * ldx) || !fits32(2 * f * d)) return RV_ERR_UNSUPPORTED;
  GemmArgs a{};
  a.a = static_cast<const __half*>(x); a.lda = ldx; a.a_bytes = rows * ldx * 2;
  a.b = static_cast<const __half*>(w_up); a.ldb = d; a.b_bytes = 2 * f * d * 2;
  a.m = rows; a.n = 2 * f; a.k = d;
  a.c = o; a.ldc = f; a.u = u; a.ldu = 2 * f; a.f = f;
  return run_act<false, false, Epi::SwiGLU>(a, f, (hipStream_t)stream);
}

int rv_mlp_down(const void* o, const void* w_down, int64_t rows, int64_t d, int64_t f, void* y,
                void* stream) {
  if (!o || !w_down || !y) return RV_ERR_NULL_POINTER;
  if (rows <= 0 || d <= 0 || f <= 0) return RV_ERR_BAD_SIZE;
  if (f % kBK || d % 128) return RV_ERR_UNSUPPORTED;
  if (!ok16(o) || !ok16(w_down) || !ok16(y)) return RV_ERR_UNSUPPORTED;
  if (!fits32(rows * f) || !fits32(d * f)) return RV_ERR_UNSUPPORTED;
  GemmArgs a{};
  a.a = static_cast<const __half*>(o); a.lda = f; a.a_bytes = rows * f * 2;
  a.b = static_cast<const __half*>(w_down); a.ldb = f; a.b_bytes = d * f * 2;
  a.m = rows; a.n = d; a.k = f;
  a.c = y; a.ldc = d;
  return run_act<false, false, Epi::StoreF16>(a, d, (hipStream_t)stream);
}

int rv_mlp_dgate(const void* dy, const void* w_down, const void* u, int64_t rows, int64_t d,
                 int64_t f, void* du, void* stream) {
  if (!dy || !w_down || !u || !du) return RV_ERR_NULL_POINTER;
  if (rows <= 0 || d <= 0 || f <= 0) return RV_ERR_BAD_SIZE;
  if (d % kBK || f % 128) return RV_ERR_UNSUPPORTED;
  if (!ok16(dy) || !ok16(w_down) || !ok16(u) || !ok16(du)) return RV_ERR_UNSUPPORTED;
  if (!fits32(rows * d) || !fits32(d * f)) return RV_ERR_UNSUPPORTED;
  GemmArgs a{};
  a.a = static_cast<const __half*>(dy); a.lda = d; a.a_bytes = rows * d * 2;
  a.b = static_cast<const __half*>(w_down); a.ldb = f;  // B(f, d) = W_down[d][f]: RC
  a.b_bytes = d * f * 2;
  a.m = rows; a.n = f; a.k = d;
  a.c = du; a.ldc = 2 * f; a.u = const_cast<void*>(u); a.ldu = 2 * f; a.f = f;
  return run_act<false, true, Epi::SwiGLUBwd>(a, f, (hipStream_t)stream);
}

int rv_mlp_dx(const void* du, const void* w_up, int64_t rows, int64_t d, int64_t f, float* dx,
              void* stream) {
  if (!du || !w_up || !dx) return RV_ERR_NULL_POINTER;
  if (rows <= 0 || d <= 0 || f <= 0) return RV_ERR_BAD_SIZE;
  if ((2 * f) % kBK || d % 128) return RV_ERR_UNSUPPORTED;
  if (!ok16(du) || !ok16(w_up) || !ok16(dx)) return RV_ERR_UNSUPPORTED;
  if (!fits32(rows * 2 * f) || !fits32(2 * f * d)) return RV_ERR_UNSUPPORTED;
  GemmArgs a{};
  a.a = static_cast<const __half*>(du); a.lda = 2 * f; a.a_bytes = rows * 2 * f * 2;
  a.b = static_cast<const __half*>(w_up); a.ldb = d;  // B(d, j) = W_up[j][d]: RC
  a.b_bytes = 2 * f * d * 2;
  a.m = rows; a.n = d; a.k = 2 * f;
  a.c = dx; a.ldc = d;
  return run_act<false, true, Epi::StoreF32OfF16>(a, d, (hipStream_t)stream);
}

int rv_linear_fwd(const void* x, int64_t ldx, const void* w, int64_t rows, int64_t in,
                  int64_t out, void* y, void* stream) {
  if (!x || !w || !y) return RV_ERR_NULL_POINTER;
  if (rows <= 0 || in <= 0 || out <= 0 || ldx < in) return RV_ERR_BAD_SIZE;
  if (in % 128 || out % 128 || ldx % 8) return RV_ERR_UNSUPPORTED;
  if (!ok16(x) || !ok16(w) || !ok16(y)) return RV_ERR_UNSUPPORTED;
  if (!fits32(rows * ldx) || !fits32(out * in)) return RV_ERR_UNSUPPORTED;
  GemmArgs a{};
  a.a = static_cast<const __half*>(x); a.lda = ldx; a.a_bytes = rows * ldx * 2;
  a.b = static_cast<const __half*>(w); a.ldb = in; a.b_bytes = out * in * 2;
  a.m = rows; a.n = out; a.k = in;
  a.c = y; a.ldc = out;
  return run_act<false, false, Epi::StoreF16>(a, out, (hipStream_t)stream);
}

int rv_linear_dx(const void* dy, const void* w, int64_t rows, int64_t in, int64_t out, void* dx,
                 int dx_dtype, void* stream) {
  if (!dy || !w || !dx) return RV_ERR_NULL_POINTER;
  if (rows <= 0 || in <= 0 || out <= 0) return RV_ERR_BAD_SIZE;
  if (in % 128 || out % 128) return RV_ERR_UNSUPPORTED;
  if (dx_dtype != RV_F16 && dx_dtype != RV_F32) return RV_ERR_UNSUPPORTED;
  if (!ok16(dy) || !ok16(w) || !ok16(dx)) return RV_ERR_UNSUPPORTED;
  if (!fits32(rows * out) || !fits32(out * in)) return RV_ERR_UNSUPPORTED;
  GemmArgs a{};
  a.a = static_cast<const __half*>(dy); a.lda = out; a.a_bytes = rows * out * 2;
  a.b = static_cast<const __half*>(w); a.ldb = in;  // B(i, o) = W[o][i]: RC
  a.b_bytes = out * in * 2;
  a.m = rows; a.n = in; a.k = out;
  a.c = dx; a.ldc = in;
  const hipStream_t s = (hipStream_t)stream;
  return dx_dtype == RV_F16 ? run_act<false, true, Epi::StoreF16>(a, in, s)
                            : run_act<false, true, Epi::StoreF32OfF16>(a, in, s);
}

int64_t rv_linear_dw_workspace_bytes(int64_t rows, int64_t in, int64_t out) {
  if (rows <= 0 || in <= 0 || out <= 0) return -(int64_t)RV_ERR_BAD_SIZE;
  const int64_t b = wgrad_part_bytes(rows, out, in);
  return b < 0 ? -(int64_t)RV_ERR_UNSUPPORTED : b;
}

int rv_linear_dw(const void* dy, const void* x, int64_t ldx, int64_t rows, int64_t in,
                 int64_t out, float* dw, int accumulate, void* workspace, int64_t workspace_bytes,
                 void* stream) {
  if (!dy || !x || !dw) return RV_ERR_NULL_POINTER;
  if (rows <= 0 || in <= 0 || out <= 0 || ldx < in) return RV_ERR_BAD_SIZE;
  if (in % 128 || out % 128 || ldx % 8) return RV_ERR_UNSUPPORTED;
  if (!ok16(dy) || !ok16(x) || !ok16(dw)) return RV_ERR_UNSUPPORTED;
  if (!fits32(rows * out) || !fits32(rows * ldx)) return RV_ERR_UNSUPPORTED;
  const int64_t need = rv_linear_dw_workspace_bytes(rows, in, out);
  if (need < 0) return (int)-need;
  if (need > 0 && (workspace == nullptr || workspace_bytes < need || !ok16(workspace)))
    return RV_ERR_WORKSPACE;
  // dW[out][in] = sum_m dy[m][o] x[m][i]
  return run_wgrad(static_cast<const __half*>(dy), out, static_cast<const __half*>(x), ldx, rows,
                   out, in, dw, accumulate, static_cast<float*>(workspace), (hipStream_t)stream);
}

int64_t rv_mlp_wgrad_workspace_bytes(int64_t rows, int64_t d, int64_t f) {
  if (rows <= 0 || d <= 0 || f <= 0) return -(int64_t)RV_ERR_BAD_SIZE;
  const int64_t a = wgrad_part_bytes(rows, d, f), b = wgrad_part_bytes(rows, 2 * f, d);
  if (a < 0 || b < 0) return -(int64_t)RV_ERR_UNSUPPORTED;
  return (b > 0 ? align256(a) : a) + b;  // both partial sets at once (one reduction launch)
}

int rv_mlp_wgrad(const void* dy, const void* o, const void* du, const void* x, int64_t ldx,
                 int64_t rows, int64_t d, int64_t f, float* ddown, float* dup, int accumulate,
                 void* workspace, int64_t workspace_bytes, void* stream) {
  if (!dy || !o || !du || !x || !ddown || !dup) return RV_ERR_NULL_POINTER;
  if (rows <= 0 || d <= 0 || f <= 0 || ldx < d) return RV_ERR_BAD_SIZE;
  if (d % 128 || f % 128 || ldx % 8) return RV_ERR_UNSUPPORTED;
  if (!ok16(dy) || !ok16(o) || !ok16(du) || !ok16(x) || !ok16(ddown) || !ok16(dup))
    return RV_ERR_UNSUPPORTED;
  if (!fits32(rows * 2 * f) || !fits32(rows * ldx) || !fits32(rows * f)) return RV_ERR_UNSUPPORTED;
  const int64_t need = rv_mlp_wgrad_workspace_bytes(rows, d, f);
  if (need < 0) return (int)-need;
  if (need > 0 && (workspace == nullptr || workspace_bytes < need || !ok16(workspace)))
    return RV_ERR_WORKSPACE;
  const hipStream_t s = (hipStream_t)stream;
  // the two GEMMs' partial sums side by side, reduced by one launch
  float* part_down = static_cast<float*>(workspace);
  float* part_up = part_down + align256(wgrad_part_bytes(rows, d, f)) / (int64_t)sizeof(float);
  ReduceSeg seg_down, seg_up;
  // dW_down[d][f] = sum_m dy[m][d] o[m][f]
  int st = launch_wgrad(static_cast<const __half*>(dy), d, static_cast<const __half*>(o), f, rows,
                        d, f, ddown, accumulate, part_down, seg_down, s);
  if (st != RV_OK) return st;
  // dW_up[2f][d] = sum_m du[m][j] x16[m][d]
  st = launch_wgrad(static_cast<const __half*>(du), 2 * f, static_cast<const __half*>(x), ldx,
                    rows, 2 * f, d, dup, accumulate, part_up, seg_up, s);
  if (st != RV_OK) return st;
  return launch_reduce(seg_down, seg_up, accumulate, s);
}

}  // extern "C"
