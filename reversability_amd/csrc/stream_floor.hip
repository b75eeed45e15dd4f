// Streaming floor kernels: measurement only, no part of any hot-path result.
//
// A bandwidth-bound kernel's time at a given size is bounded below by the time
// the chip needs to move the same bytes with the simplest possible kernel.  These
// kernels read NR arrays and write NW arrays of the same byte size, 16 bytes per
// access, in the shape the product's one-shot kernels use: a grid that covers
// every vector once (no loop), each thread loading V vectors of each input
// (vectors blockIdx * 256 V + v * 256 + threadIdx, coalesced) before its first
// wait, then storing.  Every output is a bitwise function of the inputs (xor), so
// nothing is dead code and no floating-point work is added.  The benchmark sweeps
// V and the cache hints and keeps the fastest as the floor for each kernel's
// read/write shape at its exact byte count.

#include "rv_device.h"

namespace {

struct StreamArgs {
  const uint4* in[3];
  uint4* out[2];
  int64_t n;  // 16-byte vectors per array
};

template <int NR, int NW, int V, bool NTL, bool NTS>
__global__ __launch_bounds__(256) void stream_floor_k(StreamArgs a) {
  const int64_t base = (int64_t)blockIdx.x * (256 * V) + threadIdx.x;
  uint4 r[NR][V];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int64_t i = base + (int64_t)v * 256;
    const int64_t ic = i < a.n ? i : a.n - 1;
#pragma unroll
    for (int j = 0; j < NR; ++j) r[j][v] = rv::ld16<NTL>(a.in[j] + ic);
  }
  __builtin_amdgcn_sched_barrier(0);  // every load in flight before the first wait
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int64_t i = base + (int64_t)v * 256;
    if (i >= a.n) continue;
    uint4 o = r[0][v];
#pragma unroll
    for (int j = 1; j < NR; ++j) {
      o.x ^= r[j][v].x; o.y ^= r[j][v].y; o.z ^= r[j][v].z; o.w ^= r[j][v].w;
    }
#pragma unroll
    for (int k = 0; k < NW; ++k) {
      const uint4 ok = make_uint4(o.x ^ k, o.y, o.z, o.w);
      rv::st16<NTS>(a.out[k] + i, ok);
    }
  }
}

__global__ void empty_k() {}

template <int NR, int NW, int V>
int launch_v(const StreamArgs& a, int hints, hipStream_t st) {
  const dim3 grid((unsigned)((a.n + 256 * V - 1) / (256 * V)));
  switch (hints & 3) {
    case 0: stream_floor_k<NR, NW, V, false, false><<<grid, 256, 0, st>>>(a); break;
    case 1: stream_floor_k<NR, NW, V, true, false><<<grid, 256, 0, st>>>(a); break;
    case 2: stream_floor_k<NR, NW, V, false, true><<<grid, 256, 0, st>>>(a); break;
    default: stream_floor_k<NR, NW, V, true, true><<<grid, 256, 0, st>>>(a); break;
  }
  return rv_host::check_launch();
}

template <int NR, int NW>
int launch_rw(const StreamArgs& a, int vec, int hints, hipStream_t st) {
  switch (vec) {
    case 1: return launch_v<NR, NW, 1>(a, hints, st);
    case 2: return launch_v<NR, NW, 2>(a, hints, st);
    case 4: return launch_v<NR, NW, 4>(a, hints, st);
    case 8: return launch_v<NR, NW, 8>(a, hints, st);
    default: return RV_ERR_UNSUPPORTED;
  }
}

}  // namespace

extern "C" {

int rv_stream_floor(const void* const* in, int nin, void* const* out, int nout, int64_t bytes,
                    int vec, int hints, void* stream) {
  if (in == nullptr || out == nullptr) return RV_ERR_NULL_POINTER;
  if (nin < 1 || nin > 3 || nout < 1 || nout > 2 || bytes <= 0 || (bytes & 15) != 0)
    return RV_ERR_BAD_SIZE;
  if (hints < 0 || hints > 3) return RV_ERR_UNSUPPORTED;
  StreamArgs a{};
  for (int j = 0; j < nin; ++j) {
    if (in[j] == nullptr) return RV_ERR_NULL_POINTER;
    if (!rv_host::aligned16(in[j])) return RV_ERR_UNSUPPORTED;
    a.in[j] = static_cast<const uint4*>(in[j]);
  }
  for (int k = 0; k < nout; ++k) {
    if (out[k] == nullptr) return RV_ERR_NULL_POINTER;
    if (!rv_host::aligned16(out[k])) return RV_ERR_UNSUPPORTED;
    a.out[k] = static_cast<uint4*>(out[k]);
  }
  a.n = bytes / 16;
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (nin * 4 + nout) {
    case 5: return launch_rw<1, 1>(a, vec, hints, st);
    case 6: return launch_rw<1, 2>(a, vec, hints, st);
    case 9: return launch_rw<2, 1>(a, vec, hints, st);
    case 10: return launch_rw<2, 2>(a, vec, hints, st);
    case 13: return launch_rw<3, 1>(a, vec, hints, st);
    default: return launch_rw<3, 2>(a, vec, hints, st);
  }
}

int rv_empty_kernel(int blocks, void* stream) {
  if (blocks < 1) return RV_ERR_BAD_SIZE;
  empty_k<<<dim3((unsigned)blocks), 64, 0, static_cast<hipStream_t>(stream)>>>();
  return rv_host::check_launch();
}

}  // extern "C"
