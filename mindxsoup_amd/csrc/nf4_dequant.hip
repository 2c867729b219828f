// NF4 -> fp16/fp32 dequantization for gfx950 (standalone, HBM-bound).
//
// Replaces the reference's Triton kernels nf4_unpack_wide_kernel (solution/nf4.py:54-86),
// nf4_unpack_kernel (solution/nf4.py:31-51) and nf4_layer_kernel (solution/nf4.py:89-110).
//
// Layout: packed NF4 is u8 [(N*K)/2] (byte i = values 2i high nibble, 2i+1 low nibble),
// 64 values (32 bytes) per first-level block.  A "chunk" is one dword = 8 values = 16 output
// bytes.  A workgroup of 256 lanes takes 1024 consecutive chunks (128 blocks): lane t handles
// chunks t, t+256, t+512, t+768, so each wave's dword load reads 256 contiguous bytes and each
// wave's 16-byte store writes 1 KiB contiguous (fully coalesced both ways).  The
// 128 block scales of the workgroup are decoded once (one lane per block) into LDS.
#include "common.h"
#include "mxs_nf4.h"

namespace mxs {

constexpr int kDqThreads = 256;
constexpr int kDqUnroll = 4;                          // chunks per lane
constexpr int kDqChunks = kDqThreads * kDqUnroll;     // chunks per workgroup
constexpr int kDqBlocks = kDqChunks / 8;              // 128 first-level blocks per workgroup

struct DequantArgs {
  const uint32_t* packed;  // dwords
  void* out;
  const uint8_t* absmax8;
  const float* code;       // [n_modules * 256]
  const float* absmax2;
  const float* offset;     // [n_modules]
  const float* absmax_f32; // non-nested first-level scales
  const int64_t* block0;   // [n_modules + 1] first block of each module (multi-module only)
  const int64_t* scale0;   // [n_modules] first absmax2 index of each module
  const int16_t* wg_module;  // per workgroup: its module, or -1 if it straddles two (or NULL)
  int64_t n_chunks;
  int64_t n_blocks;
  int n_modules;
};

// Module holding block `blk`: the last m with block0[m] <= blk (block0 ascending).
__device__ __forceinline__ int find_module(const int64_t* block0, int n, int64_t blk) {
  int lo = 0, hi = n;  // invariant: block0[lo] <= blk < block0[hi]
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (block0[mid] <= blk) lo = mid; else hi = mid;
  }
  return lo;
}

template <bool NESTED, bool MULTI, bool F32_OUT>
__global__ __launch_bounds__(kDqThreads) void k_dequant_wide(DequantArgs a) {
  __shared__ float s_nf4[16];
  __shared__ float s_scale[kDqBlocks];
  const int t = threadIdx.x;
  const int64_t c0 = (int64_t)blockIdx.x * kDqChunks;

  // Issue the packed loads first; their latency overlaps the scale decode below.
  uint32_t w[kDqUnroll];
#pragma unroll
  for (int u = 0; u < kDqUnroll; u++) {
    const int64_t c = c0 + u * kDqThreads + t;
    w[u] = c < a.n_chunks ? __builtin_nontemporal_load(a.packed + c) : 0u;
  }

  if (t < 16) s_nf4[t] = kNF4[t];
  if (t < kDqBlocks) {
    const int64_t blk = (c0 >> 3) + t;
    float s = 0.0f;
    if (blk < a.n_blocks) {
      if (NESTED) {
        int m = 0;
        int64_t first_blk = 0, first_a2 = 0;
        if (MULTI) {
          // workgroup-uniform module from the plan; a binary search only where the workgroup
          // straddles two modules (or no plan was given)
          const int wm = a.wg_module ? (int)a.wg_module[blockIdx.x] : -1;
          m = wm >= 0 ? wm : find_module(a.block0, a.n_modules, blk);
          first_blk = a.block0[m];
          first_a2 = a.scale0[m];
        }
        const float c = a.code[m * 256 + a.absmax8[blk]];
        const float a2 = a.absmax2[first_a2 + ((blk - first_blk) >> 8)];
        s = nested_scale(c, a2, a.offset[m]);
      } else {
        s = a.absmax_f32[blk];
      }
    }
    s_scale[t] = s;
  }
  __syncthreads();

#pragma unroll
  for (int u = 0; u < kDqUnroll; u++) {
    const int local = u * kDqThreads + t;
    const int64_t c = c0 + local;
    if (c >= a.n_chunks) break;
    const float s = s_scale[local >> 3];
    if (F32_OUT) {
      float4_t lo, hi;
      const uint32_t x = w[u];
#pragma unroll
      for (int j = 0; j < 2; j++) {
        lo[2 * j] = s_nf4[(x >> (8 * j + 4)) & 15u] * s;
        lo[2 * j + 1] = s_nf4[(x >> (8 * j)) & 15u] * s;
        hi[2 * j] = s_nf4[(x >> (8 * j + 20)) & 15u] * s;
        hi[2 * j + 1] = s_nf4[(x >> (8 * j + 16)) & 15u] * s;
      }
      float4_t* o = reinterpret_cast<float4_t*>(a.out) + 2 * c;
      __builtin_nontemporal_store(lo, o);
      __builtin_nontemporal_store(hi, o + 1);
    } else {
      const u32x4 v = decode8(w[u], s, s_nf4);
      __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(a.out) + c);
    }
  }
}

// One byte per lane (any size, any alignment): solution/nf4.py:31-51.  Kept as the fallback for
// sizes that are not whole 32-byte blocks and as an independent cross-check of the wide kernel.
template <bool NESTED, bool F32_OUT>
__global__ __launch_bounds__(256) void k_dequant_bytes(const uint8_t* __restrict__ packed,
                                                      void* __restrict__ out,
                                                      const uint8_t* __restrict__ absmax8,
                                                      const float* __restrict__ code,
                                                      const float* __restrict__ absmax2,
                                                      const float* __restrict__ offset,
                                                      const float* __restrict__ absmax_f32,
                                                      int64_t n_bytes) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_bytes; i += stride) {
    const int64_t blk = i >> 5;
    const float s = NESTED ? nested_scale(code[absmax8[blk]], absmax2[blk >> 8], offset[0])
                           : absmax_f32[blk];
    const uint32_t b = packed[i];
    const float hi = kNF4[b >> 4] * s;
    const float lo = kNF4[b & 15u] * s;
    if (F32_OUT) {
      float* o = reinterpret_cast<float*>(out);
      o[2 * i] = hi;
      o[2 * i + 1] = lo;
    } else {
      const uint32_t pk = pack_f16x2(hi, lo);
      uint16_t* o = reinterpret_cast<uint16_t*>(out);
      o[2 * i] = (uint16_t)(pk & 0xffffu);
      o[2 * i + 1] = (uint16_t)(pk >> 16);
    }
  }
}

static int launch_wide(const DequantArgs& a, bool nested, bool multi, bool f32_out,
                       hipStream_t stream) {
  if (a.n_chunks <= 0) return MXS_OK;
  const int64_t grid = (a.n_chunks + kDqChunks - 1) / kDqChunks;
  if (grid > 0x7fffffff) return MXS_ERR_SIZE;
  const dim3 g((unsigned)grid), b(kDqThreads);
#define MXS_LAUNCH(N, M, F) hipLaunchKernelGGL((k_dequant_wide<N, M, F>), g, b, 0, stream, a)
  if (nested) {
    if (multi) {
      if (f32_out) MXS_LAUNCH(true, true, true); else MXS_LAUNCH(true, true, false);
    } else {
      if (f32_out) MXS_LAUNCH(true, false, true); else MXS_LAUNCH(true, false, false);
    }
  } else {
    if (f32_out) MXS_LAUNCH(false, false, true); else MXS_LAUNCH(false, false, false);
  }
#undef MXS_LAUNCH
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? MXS_OK : (int)e;
}

}  // namespace mxs

using namespace mxs;

extern "C" {

int mxs_nf4_dequant_bytewise(const void* packed, int64_t n_bytes, const void* absmax8,
                             const float* code, const float* absmax2, const float* offset,
                             const float* absmax_f32, void* out, int out_dtype,
                             hipStream_t stream) {
  if (n_bytes < 0) return MXS_ERR_ARG;
  if (out_dtype != MXS_DTYPE_F16 && out_dtype != MXS_DTYPE_F32) return MXS_ERR_DTYPE;
  if (n_bytes == 0) return MXS_OK;  // empty tensors may carry null pointers
  if (!packed || !out) return MXS_ERR_ARG;
  const bool nested = absmax8 != nullptr;
  if (nested ? (!code || !absmax2 || !offset) : !absmax_f32) return MXS_ERR_ARG;
  int64_t grid = (n_bytes + 1023) / 1024;
  if (grid > 65536) grid = 65536;
  const dim3 g((unsigned)grid), b(256);
  const uint8_t* p = static_cast<const uint8_t*>(packed);
  const uint8_t* q8 = static_cast<const uint8_t*>(absmax8);
#define MXS_LAUNCH(N, F) \
  hipLaunchKernelGGL((k_dequant_bytes<N, F>), g, b, 0, stream, p, out, q8, code, absmax2, \
                     offset, absmax_f32, n_bytes)
  if (nested) {
    if (out_dtype == MXS_DTYPE_F32) MXS_LAUNCH(true, true); else MXS_LAUNCH(true, false);
  } else {
    if (out_dtype == MXS_DTYPE_F32) MXS_LAUNCH(false, true); else MXS_LAUNCH(false, false);
  }
#undef MXS_LAUNCH
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? MXS_OK : (int)e;
}

int mxs_nf4_dequant(const void* packed, int64_t n_bytes, const void* absmax8, const float* code,
                    const float* absmax2, const float* offset, const float* absmax_f32,
                    void* out, int out_dtype, hipStream_t stream) {
  if (n_bytes < 0) return MXS_ERR_ARG;
  if (out_dtype != MXS_DTYPE_F16 && out_dtype != MXS_DTYPE_F32) return MXS_ERR_DTYPE;
  if (n_bytes == 0) return MXS_OK;  // empty tensors may carry null pointers
  if (!packed || !out) return MXS_ERR_ARG;
  const bool nested = absmax8 != nullptr;
  if (nested ? (!code || !absmax2 || !offset) : !absmax_f32) return MXS_ERR_ARG;
  // The wide kernel needs whole 32-byte blocks, dword-aligned packed bytes and 16-byte aligned
  // output rows (solution/nf4.py:145-148 uses the same rule with 16-byte alignment).
  const bool wide = n_bytes % 32 == 0 && ((uintptr_t)packed % 16) == 0 &&
                    ((uintptr_t)out % 16) == 0;
  if (!wide)
    return mxs_nf4_dequant_bytewise(packed, n_bytes, absmax8, code, absmax2, offset, absmax_f32,
                                    out, out_dtype, stream);
  DequantArgs a{};
  a.packed = static_cast<const uint32_t*>(packed);
  a.out = out;
  a.absmax8 = static_cast<const uint8_t*>(absmax8);
  a.code = code;
  a.absmax2 = absmax2;
  a.offset = offset;
  a.absmax_f32 = absmax_f32;
  a.n_chunks = n_bytes / 4;
  a.n_blocks = n_bytes / 32;
  a.n_modules = 1;
  return launch_wide(a, nested, false, out_dtype == MXS_DTYPE_F32, stream);
}

int64_t mxs_nf4_dequant_layer_plan(const int64_t* block0, int n_modules, int16_t* wg_module,
                                   int64_t capacity) {
  if (!block0 || n_modules < 1 || n_modules > 32767 || capacity < 0) return MXS_ERR_ARG;
  const int64_t n_blocks = block0[n_modules];
  const int64_t n_wg = (n_blocks + kDqBlocks - 1) / kDqBlocks;
  if (!wg_module) return n_wg;
  if (capacity < n_wg) return MXS_ERR_SIZE;
  int m = 0;
  for (int64_t g = 0; g < n_wg; g++) {
    const int64_t first = g * kDqBlocks;
    const int64_t last = (first + kDqBlocks < n_blocks ? first + kDqBlocks : n_blocks) - 1;
    while (m + 1 <= n_modules && block0[m + 1] <= first) m++;
    wg_module[g] = (int16_t)(last < block0[m + 1] ? m : -1);
  }
  return n_wg;
}

int mxs_nf4_dequant_layer(const void* packed, int64_t n_blocks, const void* absmax8,
                          const float* code, const float* absmax2, const float* offset,
                          const int64_t* block0, const int64_t* scale0, int n_modules,
                          const int16_t* wg_module, int64_t n_plan, void* out,
                          hipStream_t stream) {
  if (n_blocks == 0 && n_modules >= 1) return MXS_OK;
  if (n_blocks < 0 || n_modules < 1 || !packed || !out || !absmax8 || !code || !absmax2 ||
      !offset || !block0 || !scale0)
    return MXS_ERR_ARG;
  // every workgroup reads its entry of the plan: one of another length belongs to another layout
  if (wg_module && n_plan != (n_blocks + kDqBlocks - 1) / kDqBlocks) return MXS_ERR_SIZE;
  if (((uintptr_t)packed % 16) != 0 || ((uintptr_t)out % 16) != 0) return MXS_ERR_ALIGN;
  DequantArgs a{};
  a.packed = static_cast<const uint32_t*>(packed);
  a.out = out;
  a.absmax8 = static_cast<const uint8_t*>(absmax8);
  a.code = code;
  a.absmax2 = absmax2;
  a.offset = offset;
  a.block0 = block0;
  a.scale0 = scale0;
  a.wg_module = wg_module;
  a.n_chunks = n_blocks * 8;
  a.n_blocks = n_blocks;
  a.n_modules = n_modules;
  return launch_wide(a, true, n_modules > 1, false, stream);
}

}  // extern "C"
