// Token pipeline and token + position embedding for gfx950: the steps in
// front of the reversible stack.
//
//   batch      scripts/train_baseline.py:50-63 (batch_at): a window of
//              count + 1 uint16 tokens becomes x = window[:-1] and
//              y = window[1:] as int64, padded to whole sequences with x = 0
//              and y = -100.
//   forward    src/reversibility/reversible.py:105-106 and model.py (the
//              boundary p = q = token_embedding(ids) +
//              position_embedding(arange(T))).
//   backward   the gradients nn.Embedding's backward and the broadcast add
//              produce: dtok[v] = sum of dout rows whose id is v, dpos[t] =
//              sum over the batch of dout[:, t].
//
// Layouts (row-major): window uint16 [count + 1]; x, y int64 [sequences *
// seq]; ids int64 [batch * seq]; token table fp32 [vocab][d]; position table
// fp32 [max_seq][d]; activations fp32 [batch * seq][d]; d a multiple of 4 and
// the fp32 tables / activations 16-byte aligned.
//
// Every kernel is HBM-bound and touches each byte once:
//   batch_k        one thread per output position (2 bytes in, 16 out).
//   embed_fwd_k    one wave per token row, 16-byte accesses: reads the token
//                  row (4 d bytes; the position rows stay in L2), writes
//                  4 d.  An id outside [0, vocab) gives a NaN row.
//   embed_bwd_pos_k one wave per (t, 256 columns), summing the batch in
//                  order (4 d bytes read per token).
//   token gradient, deterministic (no floating-point atomics): the ids are
//                  sorted stably (rocPRIM radix sort, id as key, token index
//                  as value), so each id's occurrences form a run in
//                  ascending token order.  The sorted array is cut into
//                  blocks of kRun entries, one wave each (embed_bwd_tok_k):
//                  the wave sums the rows of each run piece of its block in
//                  order; a run that starts and ends inside the block is
//                  added to dtok directly, a piece that continues from the
//                  previous block goes to the block's head slot, a piece
//                  that continues into the next block to its tail slot.
//                  embed_bwd_chain_k then adds, for every run that crosses a
//                  block boundary, its tail piece and the following head
//                  pieces in block order.  The result is a fixed function of
//                  the ids (bit-identical run to run); reads 4 d bytes per
//                  token plus a read-modify-write of each touched dtok row.

#include <rocprim/device/device_radix_sort.hpp>
#include <rocprim/iterator/counting_iterator.hpp>

#include "rv_device.h"

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / rv::kWave;
constexpr int kCols = 4 * rv::kWave;  // columns one wave covers with a float4 per lane
constexpr int kChunks = 4;            // float4 per lane held at once: 1024 columns per pass
constexpr int kRun = 16;              // sorted entries per wave in the token gradient
constexpr int kPrefetch = 4;          // rows in flight per wave
constexpr int64_t kIgnore = -100;

__device__ __forceinline__ void add4(float4& a, const float4& b) {
  a.x = a.x + b.x;
  a.y = a.y + b.y;
  a.z = a.z + b.z;
  a.w = a.w + b.w;
}

__global__ __launch_bounds__(kThreads)
void batch_k(const uint16_t* __restrict__ w, int64_t count, int64_t total,
             int64_t* __restrict__ x, int64_t* __restrict__ y) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= total) return;
  const bool live = i < count;
  x[i] = live ? (int64_t)w[i] : 0;
  y[i] = live ? (int64_t)w[i + 1] : kIgnore;
}

__global__ __launch_bounds__(kThreads)
void embed_fwd_k(const int64_t* __restrict__ ids, int64_t n, int64_t seq,
                 const float* __restrict__ tok, int64_t vocab, const float* __restrict__ pos,
                 int64_t d, float* __restrict__ out) {
  const int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (row >= n) return;
  const int lane = threadIdx.x & 63;
  const int64_t id = ids[row];
  const bool ok = id >= 0 && id < vocab;
  const float* tr = tok + (ok ? id : 0) * d;
  const float* pr = pos + (row % seq) * d;
  float* o = out + row * d;
  for (int64_t c = 4 * lane; c < d; c += kCols) {
    float4 r = rv::ld_f4(tr + c);
    add4(r, rv::ld_f4(pr + c));
    if (!ok) r = make_float4(NAN, NAN, NAN, NAN);
    rv::st_f4(o + c, r);
  }
}

__global__ __launch_bounds__(kThreads)
void fill_zero_k(float* __restrict__ p, int64_t n4) {
  const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n4;
       i += (int64_t)gridDim.x * kThreads)
    rv::st_f4(p + 4 * i, z);
}

// dpos[t] (+)= sum_b dout[b * seq + t] for t < seq (batch order); rows
// seq <= t < max_seq are zeroed unless accumulating.
__global__ __launch_bounds__(kThreads)
void embed_bwd_pos_k(const float* __restrict__ dout, int64_t batch, int64_t seq,
                     int64_t max_seq, int64_t d, int64_t col_chunks, float* __restrict__ dpos,
                     int accumulate) {
  const int64_t wid = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (wid >= max_seq * col_chunks) return;
  const int64_t t = wid / col_chunks;
  const int64_t c = (wid % col_chunks) * kCols + 4 * (threadIdx.x & 63);
  if (c >= d) return;
  float* dst = dpos + t * d + c;
  if (t >= seq) {
    if (!accumulate) rv::st_f4(dst, make_float4(0.f, 0.f, 0.f, 0.f));
    return;
  }
  const float* src = dout + t * d + c;
  const int64_t stride = seq * d;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  int64_t b = 0;
  for (; b + 8 <= batch; b += 8) {
    float4 r[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) r[u] = rv::ld_f4s(src + (b + u) * stride);
#pragma unroll
    for (int u = 0; u < 8; ++u) add4(acc, r[u]);
  }
  for (; b < batch; ++b) add4(acc, rv::ld_f4s(src + b * stride));
  if (accumulate) {
    float4 old = rv::ld_f4(dst);
    add4(old, acc);
    acc = old;
  }
  rv::st_f4(dst, acc);
}

// Sort keys: the id, or vocab for an id outside [0, vocab) (sorted last and
// given no gradient).
__global__ __launch_bounds__(kThreads)
void keys_k(const int64_t* __restrict__ ids, int64_t n, int64_t vocab, uint32_t* __restrict__ key) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= n) return;
  const int64_t id = ids[i];
  key[i] = (id >= 0 && id < vocab) ? (uint32_t)id : (uint32_t)vocab;
}

// One wave per block of kRun sorted entries; see the header for the slots.
__global__ __launch_bounds__(kThreads)
void embed_bwd_tok_k(const uint32_t* __restrict__ key, const int32_t* __restrict__ src, int64_t n,
                     const float* __restrict__ dout, int64_t d, uint32_t vocab,
                     float* __restrict__ dtok, float* __restrict__ part) {
  const int64_t blk = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  const int64_t beg = blk * kRun;
  if (beg >= n) return;
  const int64_t end = beg + kRun < n ? beg + kRun : n;
  const int lane = threadIdx.x & 63;
  const bool head_cont = beg > 0 && key[beg] == key[beg - 1];
  const bool tail_cont = end < n && key[end - 1] == key[end];
  float* head_slot = part + 2 * blk * d;
  float* tail_slot = head_slot + d;
  for (int64_t c0 = 4 * lane; c0 < d; c0 += kCols * kChunks) {
    float4 acc[kChunks];
#pragma unroll
    for (int j = 0; j < kChunks; ++j) acc[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    int64_t piece = beg;  // first entry of the current run piece
    for (int64_t i0 = beg; i0 < end; i0 += kPrefetch) {
      float4 r[kPrefetch][kChunks];
#pragma unroll
      for (int u = 0; u < kPrefetch; ++u) {
        if (i0 + u < end) {
          const float* row = dout + (int64_t)src[i0 + u] * d;
#pragma unroll
          for (int j = 0; j < kChunks; ++j)
            r[u][j] = c0 + j * kCols < d ? rv::ld_f4s(row + c0 + j * kCols)
                                         : make_float4(0.f, 0.f, 0.f, 0.f);
        }
      }
#pragma unroll
      for (int u = 0; u < kPrefetch; ++u) {
        const int64_t i = i0 + u;
        if (i >= end) break;
#pragma unroll
        for (int j = 0; j < kChunks; ++j) add4(acc[j], r[u][j]);
        const uint32_t v = key[i];
        if (i + 1 < end && key[i + 1] == v) continue;  // the piece goes on
        if (v < vocab) {
          float* dst;
          bool final_row = false;
          if (piece == beg && head_cont) dst = head_slot;
          else if (i + 1 == end && tail_cont) dst = tail_slot;
          else {
            dst = dtok + (int64_t)v * d;
            final_row = true;
          }
#pragma unroll
          for (int j = 0; j < kChunks; ++j) {
            const int64_t c = c0 + j * kCols;
            if (c < d) {
              float4 o = acc[j];
              if (final_row) {
                o = rv::ld_f4(dst + c);
                add4(o, acc[j]);
              }
              rv::st_f4(dst + c, o);
            }
          }
        }
#pragma unroll
        for (int j = 0; j < kChunks; ++j) acc[j] = make_float4(0.f, 0.f, 0.f, 0.f);
        piece = i + 1;
      }
    }
  }
}

// For each run that crosses a block boundary, owned by the block where it
// starts: dtok[v] += ((tail piece + next head piece) + ...), in block order.
__global__ __launch_bounds__(kThreads)
void embed_bwd_chain_k(const uint32_t* __restrict__ key, int64_t n, int64_t d, uint32_t vocab,
                       float* __restrict__ dtok, const float* __restrict__ part) {
  const int64_t blk = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  const int64_t beg = blk * kRun;
  if (beg >= n) return;
  const int64_t end = beg + kRun < n ? beg + kRun : n;
  if (!(end < n && key[end - 1] == key[end])) return;           // nothing continues
  if (beg > 0 && key[beg] == key[beg - 1] && key[beg] == key[end - 1])
    return;  // the whole block continues a run owned by an earlier block
  const uint32_t v = key[end - 1];
  if (v >= vocab) return;
  const int64_t nblocks = (n + kRun - 1) / kRun;
  const int lane = threadIdx.x & 63;
  for (int64_t c0 = 4 * lane; c0 < d; c0 += kCols * kChunks) {
    float4 acc[kChunks];
#pragma unroll
    for (int j = 0; j < kChunks; ++j)
      acc[j] = c0 + j * kCols < d ? rv::ld_f4(part + (2 * blk + 1) * d + c0 + j * kCols)
                                  : make_float4(0.f, 0.f, 0.f, 0.f);
    bool go = true;
    for (int64_t b0 = blk + 1; go; b0 += kPrefetch) {
      float4 r[kPrefetch][kChunks];
      bool more[kPrefetch];
#pragma unroll
      for (int u = 0; u < kPrefetch; ++u) {
        const int64_t b = b0 + u;
        more[u] = false;
        if (b < nblocks) {
          const int64_t be = (b + 1) * kRun < n ? (b + 1) * kRun : n;
          more[u] = be < n && key[be - 1] == v && key[be] == v;
#pragma unroll
          for (int j = 0; j < kChunks; ++j)
            r[u][j] = c0 + j * kCols < d ? rv::ld_f4(part + 2 * b * d + c0 + j * kCols)
                                         : make_float4(0.f, 0.f, 0.f, 0.f);
        }
      }
#pragma unroll
      for (int u = 0; u < kPrefetch; ++u) {
        if (!go) break;
#pragma unroll
        for (int j = 0; j < kChunks; ++j) add4(acc[j], r[u][j]);
        go = more[u];
      }
    }
    float* dst = dtok + (int64_t)v * d;
#pragma unroll
    for (int j = 0; j < kChunks; ++j) {
      const int64_t c = c0 + j * kCols;
      if (c < d) {
        float4 o = rv::ld_f4(dst + c);
        add4(o, acc[j]);
        rv::st_f4(dst + c, o);
      }
    }
  }
}

int64_t align256(int64_t b) { return (b + 255) & ~(int64_t)255; }

unsigned key_bits(int64_t vocab) {
  unsigned bits = 0;
  while (bits < 32 && (vocab >> bits) != 0) ++bits;  // keys go up to vocab itself
  return bits;
}

// Workspace layout: keys in, keys out, sorted token indices, piece slots,
// rocPRIM's temporary storage.
struct Layout {
  int64_t keys_in, keys_out, values, part, temp, total;
  size_t temp_bytes;
};

int plan(int64_t tokens, int64_t vocab, int64_t d, Layout& L) {
  size_t temp = 0;
  const hipError_t e = rocprim::radix_sort_pairs(
      nullptr, temp, static_cast<const uint32_t*>(nullptr), static_cast<uint32_t*>(nullptr),
      rocprim::counting_iterator<int32_t>(0), static_cast<int32_t*>(nullptr), (size_t)tokens, 0u,
      key_bits(vocab), (hipStream_t)0);
  if (e != hipSuccess) return rv_host::hip_fail(e);
  const int64_t nblocks = (tokens + kRun - 1) / kRun;
  L.keys_in = 0;
  L.keys_out = L.keys_in + align256(4 * tokens);
  L.values = L.keys_out + align256(4 * tokens);
  L.part = L.values + align256(4 * tokens);
  L.temp = L.part + align256(2 * nblocks * d * 4);
  L.temp_bytes = temp;
  L.total = L.temp + align256((int64_t)temp);
  return RV_OK;
}

bool shape_ok(int64_t vocab, int64_t max_seq, int64_t d) {
  return vocab > 0 && vocab < 0x7fffffff && max_seq > 0 && d > 0 && d % 4 == 0;
}

unsigned grid_for(int64_t items, int per_block) {
  return (unsigned)((items + per_block - 1) / per_block);
}

}  // namespace

extern "C" {

int rv_batch_from_tokens(const uint16_t* window, int64_t count, int64_t seq_len, int64_t* x,
                         int64_t* y, void* stream) {
  if (!window || !x || !y) return RV_ERR_NULL_POINTER;
  if (count <= 0 || seq_len <= 0) return RV_ERR_BAD_SIZE;
  const int64_t total = (count + seq_len - 1) / seq_len * seq_len;
  if (total / kThreads >= 0x7fffffff) return RV_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(batch_k, dim3(grid_for(total, kThreads)), dim3(kThreads), 0,
                     (hipStream_t)stream, window, count, total, x, y);
  return rv_host::check_launch();
}

int rv_embed_fwd(const int64_t* ids, int64_t batch, int64_t seq, const float* tok, int64_t vocab,
                 const float* pos, int64_t max_seq, int64_t d, float* out, void* stream) {
  if (!ids || !tok || !pos || !out) return RV_ERR_NULL_POINTER;
  if (batch < 0 || seq <= 0 || !shape_ok(vocab, max_seq, d) || seq > max_seq) return RV_ERR_BAD_SIZE;
  if (!rv_host::aligned16(tok) || !rv_host::aligned16(pos) || !rv_host::aligned16(out))
    return RV_ERR_UNSUPPORTED;
  const int64_t n = batch * seq;
  if (n == 0) return RV_OK;
  if (n / kWaves >= 0x7fffffff) return RV_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(embed_fwd_k, dim3(grid_for(n, kWaves)), dim3(kThreads), 0,
                     (hipStream_t)stream, ids, n, seq, tok, vocab, pos, d, out);
  return rv_host::check_launch();
}

int64_t rv_embed_bwd_workspace_bytes(int64_t tokens, int64_t vocab, int64_t d) {
  if (tokens < 0 || !shape_ok(vocab, 1, d)) return -RV_ERR_BAD_SIZE;
  if (tokens >= 0x7fffffff) return -RV_ERR_UNSUPPORTED;
  if (tokens == 0) return 0;
  Layout L;
  const int rc = plan(tokens, vocab, d, L);
  return rc == RV_OK ? L.total : -rc;
}

int rv_embed_bwd(const int64_t* ids, int64_t batch, int64_t seq, const float* dout, int64_t vocab,
                 int64_t max_seq, int64_t d, float* dtok, int tok_accumulate, float* dpos,
                 int pos_accumulate, void* workspace, int64_t workspace_bytes, void* stream) {
  if (!ids || !dout) return RV_ERR_NULL_POINTER;
  if (batch < 0 || seq <= 0 || !shape_ok(vocab, max_seq, d) || seq > max_seq) return RV_ERR_BAD_SIZE;
  if (!rv_host::aligned16(dout) || (dtok && !rv_host::aligned16(dtok)) ||
      (dpos && !rv_host::aligned16(dpos)))
    return RV_ERR_UNSUPPORTED;
  const int64_t n = batch * seq;
  if (n >= 0x7fffffff) return RV_ERR_UNSUPPORTED;
  const hipStream_t s = (hipStream_t)stream;
  int rc;
  if (dpos) {
    const int64_t chunks = (d + kCols - 1) / kCols;
    hipLaunchKernelGGL(embed_bwd_pos_k, dim3(grid_for(max_seq * chunks, kWaves)), dim3(kThreads), 0,
                       s, dout, batch, seq, max_seq, d, chunks, dpos, pos_accumulate);
    if ((rc = rv_host::check_launch()) != RV_OK) return rc;
  }
  if (!dtok) return RV_OK;
  if (!tok_accumulate) {
    const int64_t n4 = vocab * d / 4;
    const int64_t blocks = n4 / kThreads + 1 < 4096 ? n4 / kThreads + 1 : 4096;
    hipLaunchKernelGGL(fill_zero_k, dim3((unsigned)blocks), dim3(kThreads), 0, s, dtok, n4);
    if ((rc = rv_host::check_launch()) != RV_OK) return rc;
  }
  if (n == 0) return RV_OK;
  Layout L;
  if ((rc = plan(n, vocab, d, L)) != RV_OK) return rc;
  if (!workspace) return RV_ERR_WORKSPACE;
  if (workspace_bytes < L.total) return RV_ERR_WORKSPACE;
  char* ws = static_cast<char*>(workspace);
  uint32_t* keys_in = reinterpret_cast<uint32_t*>(ws + L.keys_in);
  uint32_t* keys_out = reinterpret_cast<uint32_t*>(ws + L.keys_out);
  int32_t* values = reinterpret_cast<int32_t*>(ws + L.values);
  float* part = reinterpret_cast<float*>(ws + L.part);
  hipLaunchKernelGGL(keys_k, dim3(grid_for(n, kThreads)), dim3(kThreads), 0, s, ids, n, vocab,
                     keys_in);
  if ((rc = rv_host::check_launch()) != RV_OK) return rc;
  size_t temp = L.temp_bytes;
  const hipError_t e = rocprim::radix_sort_pairs(
      ws + L.temp, temp, keys_in, keys_out, rocprim::counting_iterator<int32_t>(0), values,
      (size_t)n, 0u, key_bits(vocab), s);
  if (e != hipSuccess) return rv_host::hip_fail(e);
  const int64_t nblocks = (n + kRun - 1) / kRun;
  const dim3 grid(grid_for(nblocks, kWaves));
  hipLaunchKernelGGL(embed_bwd_tok_k, grid, dim3(kThreads), 0, s, keys_out, values, n, dout, d,
                     (uint32_t)vocab, dtok, part);
  if ((rc = rv_host::check_launch()) != RV_OK) return rc;
  hipLaunchKernelGGL(embed_bwd_chain_k, grid, dim3(kThreads), 0, s, keys_out, n, d,
                     (uint32_t)vocab, dtok, part);
  return rv_host::check_launch();
}

}  // extern "C"
