// HBM rate probes for gfx950: what the memory delivers for the standalone dequant's access
// pattern with none of its arithmetic, and for pure load and pure store streams.  bench.py
// reports them beside the dequant so that its fraction of peak can be read against what this
// part reaches for the same mix of reads and writes.  Built into libmxs_probe.so, apart from the
// product library.
//
//   kind 0, the dequant's pattern (k_dequant_wide): 256 lanes per workgroup, lane t loads the
//     dwords c0 + t + 256 u (u < 4) non-temporally and stores 16 bytes per dword loaded at the
//     same chunk index (the dword repeated), non-temporally: every wave load covers 256
//     contiguous bytes and every wave store 1 KiB.  Reads 4 B and writes 16 B per chunk.
//   kind 1, loads only: the same grid reading 16 bytes per chunk (1 KiB per wave load); each
//     wave XORs what it read and one lane stores 4 bytes per wave.
//   kind 2, stores only: 16 bytes per chunk, as kind 0 stores.
#include "common.h"
#include "mxs_nf4.h"
#include "mxs_probe.h"

namespace mxs {

constexpr int kProbeThreads = 256;
constexpr int kProbeUnroll = 4;
constexpr int kProbeChunks = kProbeThreads * kProbeUnroll;  // chunks per workgroup

__global__ __launch_bounds__(kProbeThreads) void k_probe_pattern(const uint32_t* src, u32x4* dst,
                                                                 int64_t n_chunks) {
  const int64_t c0 = (int64_t)blockIdx.x * kProbeChunks + threadIdx.x;
  uint32_t w[kProbeUnroll];
#pragma unroll
  for (int u = 0; u < kProbeUnroll; u++) {
    const int64_t c = c0 + u * kProbeThreads;
    w[u] = c < n_chunks ? __builtin_nontemporal_load(src + c) : 0u;
  }
#pragma unroll
  for (int u = 0; u < kProbeUnroll; u++) {
    const int64_t c = c0 + u * kProbeThreads;
    if (c >= n_chunks) break;
    const u32x4 v = {w[u], w[u], w[u], w[u]};
    __builtin_nontemporal_store(v, dst + c);
  }
}

__global__ __launch_bounds__(kProbeThreads) void k_probe_load(const u32x4* src, uint32_t* dst,
                                                              int64_t n_chunks) {
  const int64_t c0 = (int64_t)blockIdx.x * kProbeChunks + threadIdx.x;
  u32x4 v[kProbeUnroll];
#pragma unroll
  for (int u = 0; u < kProbeUnroll; u++) {
    const int64_t c = c0 + u * kProbeThreads;
    v[u] = c < n_chunks ? __builtin_nontemporal_load(src + c) : (u32x4){};
  }
  uint32_t x = 0;
#pragma unroll
  for (int u = 0; u < kProbeUnroll; u++) x ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
#pragma unroll
  for (int s = 32; s > 0; s >>= 1) x ^= (uint32_t)__shfl_xor((int)x, s, 64);
  if ((threadIdx.x & 63) == 0)
    dst[(int64_t)blockIdx.x * (kProbeThreads / 64) + (threadIdx.x >> 6)] = x;
}

__global__ __launch_bounds__(kProbeThreads) void k_probe_store(u32x4* dst, int64_t n_chunks) {
  const int64_t c0 = (int64_t)blockIdx.x * kProbeChunks + threadIdx.x;
#pragma unroll
  for (int u = 0; u < kProbeUnroll; u++) {
    const int64_t c = c0 + u * kProbeThreads;
    if (c >= n_chunks) break;
    const uint32_t lo = (uint32_t)c;
    const u32x4 v = {lo, lo ^ 1u, lo ^ 2u, lo ^ 3u};
    __builtin_nontemporal_store(v, dst + c);
  }
}

}  // namespace mxs

using namespace mxs;

extern "C" {

int mxs_hbm_probe(int kind, const void* src, void* dst, int64_t n_chunks, hipStream_t stream) {
  if (n_chunks < 0 || kind < 0 || kind > 2 || !dst || (kind != 2 && !src)) return MXS_ERR_ARG;
  if (n_chunks == 0) return MXS_OK;
  if ((uintptr_t)dst % 16 || (kind == 1 && (uintptr_t)src % 16) || (uintptr_t)src % 4)
    return MXS_ERR_ALIGN;
  const int64_t blocks = (n_chunks + kProbeChunks - 1) / kProbeChunks;
  if (blocks > 0x7fffffff) return MXS_ERR_SIZE;
  const dim3 grid((unsigned)blocks);
  if (kind == 0)
    hipLaunchKernelGGL(k_probe_pattern, grid, dim3(kProbeThreads), 0, stream,
                       static_cast<const uint32_t*>(src), static_cast<u32x4*>(dst), n_chunks);
  else if (kind == 1)
    hipLaunchKernelGGL(k_probe_load, grid, dim3(kProbeThreads), 0, stream,
                       static_cast<const u32x4*>(src), static_cast<uint32_t*>(dst), n_chunks);
  else
    hipLaunchKernelGGL(k_probe_store, grid, dim3(kProbeThreads), 0, stream,
                       static_cast<u32x4*>(dst), n_chunks);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? MXS_OK : (int)e;
}

}  // extern "C"
