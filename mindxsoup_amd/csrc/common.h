// Shared definitions for the gfx950 NF4 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mxs {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// The 16 NF4 code values (QLoRA, arXiv 2305.14314, Appendix E), fp32, ascending; index 7 is 0.
__device__ __constant__ static const float kNF4[16] = {
    -1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f,
    -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f,
    0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f,
    0.33791524171829224f, 0.44070982933044434f, 0.5626170039176941f,
    0.7229568362236023f, 1.0f};

constexpr int kBlock = 64;      // NF4 values per first-level absmax
constexpr int kGroup = 256;     // first-level blocks per second-level absmax

// Dropout keep masks travel as bits: row m of a mask over K columns is keep_words(K) 32-bit
// words (keep_row_bytes(K) bytes), bit k % 32 of word k / 32 set where element (m, k) is kept;
// bits past K are zero.  Byte k / 8 of a row holds columns k & ~7 .. +7, bit k % 8 for column k.
__host__ __device__ constexpr int keep_words(int K) { return (K + 31) / 32; }
__host__ __device__ constexpr int64_t keep_row_bytes(int K) { return 4 * (int64_t)keep_words(K); }

// Two fp32 values -> two fp16 (round to nearest even) packed low-first in a dword.
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  float2_t v = {lo, hi};
  half2_t h = __builtin_convertvector(v, half2_t);
  return __builtin_bit_cast(uint32_t, h);
}

// fp16 of an fp32 value computed as it is: a product rounded to fp32 and then to fp16, as the
// reference's kernels compute in fp32 and cast.  Left alone the compiler contracts a multiply
// and the conversion into one mixed-precision FMA (whatever the contract pragma says), which
// rounds the exact product once: one fp16 ulp off where the fp32 product lands on an fp16
// rounding tie.  The empty asm keeps the fp32 value.
__device__ __forceinline__ _Float16 f16_of(float p) {
  __asm__("" : "+v"(p));
  return (_Float16)p;
}

// fp16(fp32(x) * s), the reference's dropout (solution/dropout.py:33-35).  Rounded once instead,
// hundreds of the 63 488 finite inputs come out one ulp off at some rates (over 700 at p = 0.04;
// none at p = 0.05).
__device__ __forceinline__ _Float16 scale_round2(_Float16 x, float s) {
  return f16_of((float)x * s);
}

// Decoded block scale of the double-quantized absmax: code[q8] * absmax2 + offset, one fused
// multiply-add in fp32 (the contraction Triton applies to the reference kernel).
__device__ __forceinline__ float nested_scale(float code_q8, float absmax2, float offset) {
  return __builtin_fmaf(code_q8, absmax2, offset);
}

// Eight NF4 values of one packed dword (byte j holds values 2j high nibble, 2j+1 low nibble)
// times `s`, as eight fp16 in four dwords.  `tab` is the NF4 table in LDS.
__device__ __forceinline__ u32x4 decode8(uint32_t w, float s, const float* tab) {
  u32x4 r;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const uint32_t hi = (w >> (8 * j + 4)) & 15u;
    const uint32_t lo = (w >> (8 * j)) & 15u;
    r[j] = pack_f16x2(tab[hi] * s, tab[lo] * s);
  }
  return r;
}

// vmcnt(0): every vector memory access this wave issued has completed (gfx9 s_waitcnt encoding,
// expcnt and lgkmcnt left at their maxima).
__device__ __forceinline__ void wait_vmem_all() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Workgroup barrier that waits only for this wave's LDS operations (lgkmcnt(0)), not for its
// global loads: __syncthreads() adds a workgroup fence that waits for every outstanding vector
// memory instruction, which would drain a multi-stage load pipeline at each barrier.  The empty
// asm statements keep the compiler from moving memory accesses across the barrier.  Use only
// where no global store must become visible to the workgroup at this barrier, and wait for
// direct-to-LDS loads (counted in vmcnt) explicitly before it.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt left at their maxima
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// vmcnt(N): at most the N most recently issued vector memory instructions of this wave are still
// outstanding (they complete in issue order).  gfx9 encoding: vmcnt bits 3:0 and 15:14.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N <= 63, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

// Global loads issued as inline asm: uniform base in SGPRs plus a 32-bit per-lane byte offset.
// Like the direct-to-LDS copies, the compiler neither counts them in the vmcnt waits it
// inserts for its own loads (so none of those waits drains them) nor waits for them itself:
// read a result only after wait_vmcnt<N>() has covered its load and vm_ready() has passed it
// through.  vm_ready is ordered after the wait (both have side effects) and redefines the
// value, so no use of it can be scheduled above the wait.
__device__ __forceinline__ uint32_t gload_u8(const void* base, uint32_t off) {
  uint32_t v;
  asm volatile("global_load_ubyte %0, %1, %2" : "=v"(v) : "v"(off), "s"(base));
  return v;
}
__device__ __forceinline__ float gload_f32(const void* base, uint32_t off) {
  float v;
  asm volatile("global_load_dword %0, %1, %2" : "=v"(v) : "v"(off), "s"(base));
  return v;
}
__device__ __forceinline__ uint32_t gload_b32(const void* base, uint32_t off) {
  uint32_t v;
  asm volatile("global_load_dword %0, %1, %2" : "=v"(v) : "v"(off), "s"(base));
  return v;
}
__device__ __forceinline__ u32x2 gload_b64(const void* base, uint32_t off) {
  u32x2 v;
  asm volatile("global_load_dwordx2 %0, %1, %2" : "=v"(v) : "v"(off), "s"(base));
  return v;
}
__device__ __forceinline__ u32x4 gload_b128(const void* base, uint32_t off) {
  u32x4 v;
  asm volatile("global_load_dwordx4 %0, %1, %2" : "=v"(v) : "v"(off), "s"(base));
  return v;
}
template <typename T>
__device__ __forceinline__ void vm_ready(T& v) {
  asm volatile("" : "+v"(v));
}

}  // namespace mxs
