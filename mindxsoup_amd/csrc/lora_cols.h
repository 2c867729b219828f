// LoRA gradient columns (dA = dHs^T . drop(X), dB = dY^T . Hs) for one workgroup: the body of
// the cols kernel in lora.hip, also run by extra workgroups of the backward GEMM launch
// (nf4_gemm.hip), which then computes dX and both gradients in one launch.
#pragma once

#include <string.h>

#include <mutex>

#include "common.h"
#include "mxs_nf4.h"

namespace mxs {

constexpr int kMaxWaves = 16;        // waves per workgroup (1024 threads)
constexpr int kColsLds = 64 * 1024;  // LDS budget for the cross-wave sums (bytes)

// Columns per lane for n_tot gradient columns: the widest that still gives the launch enough
// workgroups.
inline int cols_cpl(int n_tot) { return n_tot / 128 >= 160 ? 8 : n_tot / 64 >= 96 ? 4 : 2; }

// Most waves a gradient workgroup of CPL columns per lane uses (register budget).
template <int CPL>
constexpr int cols_max_waves() { return CPL >= 8 ? 8 : CPL >= 4 ? 12 : kMaxWaves; }

// Waves that share a gradient workgroup's tokens: about three 32-token steps each, 4 to
// max_waves, and their cross-wave sums within the LDS budget.  The split of the tokens over
// waves sets the summation order, so every launch of these columns uses this rule.
inline int cols_waves(int M, int r, int cpl, int max_waves) {
  int w = ((M + 31) / 32 + 2) / 3;
  w = w < 4 ? 4 : w > max_waves ? max_waves : w;
  const int per_wave = r * (16 * cpl + 1) * (int)sizeof(float);
  while (w > 1 && w * per_wave > kColsLds) w--;
  return w;
}

// Whether rounding the exact product x * s once to fp16 gives the reference's dropout,
// fp16(fp32(x) * s), for every finite fp16 x (so at p = 0.05, not at p = 0.04).  Where it does,
// the kernels let the compiler fuse the multiply and the conversion (one mixed-precision FMA);
// where it does not they round twice (scale_round2), at a few more instructions and registers.
// Checked on the host once per scale (63 488 products), the last few scales kept.
inline bool round_once_exact(float s) {
  static std::mutex mu;
  static float seen[4];
  static bool exact[4];
  static int n = 0;
  std::lock_guard<std::mutex> lock(mu);
  for (int i = 0; i < n; i++)
    if (memcmp(&seen[i], &s, sizeof s) == 0) return exact[i];
  bool ok = true;
  for (uint32_t b = 0; b < 65536 && ok; b++) {
    const uint16_t bits = (uint16_t)b;
    _Float16 x;
    memcpy(&x, &bits, sizeof x);
    if (!__builtin_isfinite((float)x)) continue;
    const _Float16 twice = (_Float16)((float)x * s);
    const _Float16 once = (_Float16)((double)x * (double)s);  // the product is exact in double
    ok = memcmp(&twice, &once, sizeof once) == 0;
  }
  const int slot = n < 4 ? n++ : 3;
  seen[slot] = s;
  exact[slot] = ok;
  return ok;
}

struct ColsProblem {
  const _Float16* PT;     // [r, ldt] (transposed LoRA activations, zeros past M)
  const _Float16* Q;      // [M, Nq] row-major
  const uint8_t* mask;    // keep bits of [M, Nq] (keep_row_bytes(Nq) per row) or null
  float mscale;
  int round2;             // dropout rounded twice (round_once_exact(mscale) is false)
  int Nq;
  float* out;             // [r, Nq] (out_rn) or [Nq, r]
  int out_rn;
};

template <int CPL> struct ColsVec;
template <> struct ColsVec<2> { typedef uint32_t T; };
template <> struct ColsVec<4> { typedef u32x2 T; };
template <> struct ColsVec<8> { typedef u32x4 T; };

// out[j][n] = sum_m PT[j][m] * Q[m][n] over all tokens, for the 16*CPL columns of workgroup
// `block`: block < cb0 is problem p0 (dA), the rest p1 (dB).  The first nw waves (at most
// blockDim.x / 64) take 32-token steps in turn and add their accumulators in LDS (`red`,
// [nw][r][16*CPL + 1] floats) in wave order; further waves only help store.  Every thread of
// the workgroup calls it (it synchronizes the workgroup once).  MASK: the problem has a keep
// mask (uniform over the workgroup).  R2: the dropout's product is rounded to fp32 and then to
// fp16 (scale_round2), else in one mixed-precision FMA (where that is the same:
// round_once_exact).
template <int CPL, bool MASK, bool R2 = false>
__device__ __forceinline__ void lora_cols_body(const ColsProblem& a, int nb, int M, int ldt,
                                               int r, int nw, float* red) {
  typedef typename ColsVec<CPL>::T VT;
  constexpr int WC = 16 * CPL;  // columns per workgroup
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int ln = lane & 15;  // columns nb + CPL*ln .. +CPL
  const int lg = lane >> 4;  // tokens t0 + 8*lg .. +8
  const int col = nb + CPL * ln;
  const bool col_ok = col < a.Nq;
  const int ccol = col_ok ? col : 0;  // a column the loads may touch
  // the lane's CPL keep bits of a row: bits col % 8 .. of byte col / 8 (CPL divides 8)
  const int64_t kst = keep_row_bytes(a.Nq);
  const int kbyte = ccol >> 3, kshift = ccol & 7;
  const int ld = WC + 1;
  // U token blocks of 32 per batch, all loaded before any is multiplied (one memory round trip
  // per batch instead of one per block).  The loads are unconditional (token and column clamped
  // into the tensors) so that a batch issues back to back; values past M or Nq are zeroed after.
  constexpr int U = CPL == 8 ? 2 : 3;
  for (int b = 0; wave < nw && b < (r >> 4); b++) {  // r-blocks of 16 (input re-read per block)
    float4_t acc[CPL];
#pragma unroll
    for (int c = 0; c < CPL; c++) acc[c] = (float4_t){0.f, 0.f, 0.f, 0.f};
    for (int t0 = wave * 32; t0 < M; t0 += nw * 32 * U) {
      half8_t av[U];
      VT rows[U][8];
      uint32_t mks[U][8];
#pragma unroll
      for (int u = 0; u < U; u++) {
        const int mb = t0 + u * nw * 32 + 8 * lg;
        av[u] = *reinterpret_cast<const half8_t*>(a.PT + (int64_t)(16 * b + ln) * ldt +
                                                  min(mb, ldt - 8));
#pragma unroll
        for (int e = 0; e < 8; e++) {
          const int64_t m = min(mb + e, M - 1);
          rows[u][e] = *reinterpret_cast<const VT*>(a.Q + m * a.Nq + ccol);
          if constexpr (MASK) mks[u][e] = a.mask[m * kst + kbyte];
        }
      }
      // the whole batch issues before any of its values is used
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < U; u++) {
        const int mb = t0 + u * nw * 32 + 8 * lg;
        if (mb >= ldt) av[u] = (half8_t){};
        _Float16 hv[8][CPL];
#pragma unroll
        for (int e = 0; e < 8; e++) {
          if (!(mb + e < M && col_ok)) rows[u][e] = VT{};
          __builtin_memcpy(hv[e], &rows[u][e], sizeof(VT));
          if constexpr (MASK) {
#pragma unroll
            for (int c = 0; c < CPL; c++)
              hv[e][c] = ((mks[u][e] >> (kshift + c)) & 1u)
                             ? (R2 ? scale_round2(hv[e][c], a.mscale)
                                   : (_Float16)((float)hv[e][c] * a.mscale))
                             : (_Float16)0.0f;
          }
        }
#pragma unroll
        for (int c = 0; c < CPL; c++) {
          half8_t bv;
#pragma unroll
          for (int e = 0; e < 8; e++) bv[e] = hv[e][c];
          acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[u], bv, acc[c], 0, 0, 0);
        }
      }
    }
    // acc[c][v] = C[j = 16*b + 4*lg + v][column nb + CPL*ln + c]
#pragma unroll
    for (int c = 0; c < CPL; c++)
#pragma unroll
      for (int v = 0; v < 4; v++)
        red[(wave * r + 16 * b + 4 * lg + v) * ld + CPL * ln + c] = acc[c][v];
  }
  __syncthreads();
  for (int i = threadIdx.x; i < r * WC; i += blockDim.x) {
    const int j = i / WC, n = nb + i % WC;
    if (n >= a.Nq) continue;
    float sum = 0.f;
    for (int w = 0; w < nw; w++) sum += red[(w * r + j) * ld + i % WC];
    if (a.out_rn) a.out[(int64_t)j * a.Nq + n] = sum;
    else a.out[(int64_t)n * r + j] = sum;
  }
}

template <int CPL>
__device__ __forceinline__ void lora_cols_block(const ColsProblem& p0, const ColsProblem& p1,
                                                int cb0, int M, int ldt, int r, int block,
                                                int nw, float* red) {
  const bool second = block >= cb0;
  const ColsProblem& a = second ? p1 : p0;
  const int nb = (second ? block - cb0 : block) * 16 * CPL;
  if (!a.mask) lora_cols_body<CPL, false>(a, nb, M, ldt, r, nw, red);
  else if (a.round2) lora_cols_body<CPL, true, true>(a, nb, M, ldt, r, nw, red);
  else lora_cols_body<CPL, true, false>(a, nb, M, ldt, r, nw, red);
}

// dA / dB of several projections in one launch (gate's and up's arrive together): pair i owns
// workgroups [start[i], start[i+1]), laid out as its own launch's grid (dA blocks, then dB).
// All pairs share the columns per lane and the waves, which is what their own launches would
// use when their shapes agree.
constexpr int kMaxColsGroup = 4;
struct ColsGroup {
  ColsProblem pa[kMaxColsGroup], pb[kMaxColsGroup];
  int start[kMaxColsGroup + 1];
  int cb0[kMaxColsGroup];
  int n;
};

// Pair i of a gradient group: dA [r, K] = dHs^T . drop(X) from dht [r, ldt], x [M, K] and the
// keep bits (or null), dB [N, r] = dY^T . Hs from ht [r, ldt] and dy [M, N], with the checks of
// mxs_lora_grads.  MXS_OK or an error code.
inline int cols_group_set(ColsGroup& g, int i, const void* dht, const void* ht, int ldt,
                          const void* x, const void* dy, int M, int K, int N, const void* mask,
                          float mask_scale, float* da, float* db) {
  if (K <= 0 || N <= 0 || !dht || !ht || !x || !dy || !da || !db) return MXS_ERR_ARG;
  if (K % 8 || N % 8 || ldt < M || ldt % 8) return MXS_ERR_SIZE;
  if ((uintptr_t)x % 16 || (uintptr_t)dht % 16 || (uintptr_t)dy % 16 || (uintptr_t)ht % 16 ||
      (mask && ((uintptr_t)mask % 4)))
    return MXS_ERR_ALIGN;
  ColsProblem& pa = g.pa[i];
  pa.PT = static_cast<const _Float16*>(dht);
  pa.Q = static_cast<const _Float16*>(x);
  pa.mask = static_cast<const uint8_t*>(mask);
  pa.mscale = mask_scale;
  pa.round2 = mask && !round_once_exact(mask_scale);
  pa.Nq = K;
  pa.out = da;
  pa.out_rn = 1;
  ColsProblem& pb = g.pb[i];
  pb.PT = static_cast<const _Float16*>(ht);
  pb.Q = static_cast<const _Float16*>(dy);
  pb.mask = nullptr;
  pb.mscale = 1.0f;
  pb.round2 = 0;
  pb.Nq = N;
  pb.out = db;
  pb.out_rn = 0;
  return MXS_OK;
}

// Lays out the group's workgroups for CPL columns per lane (16 * CPL columns a workgroup);
// returns their number.
inline int cols_group_layout(ColsGroup& g, int cpl) {
  const int wc = 16 * cpl;
  int total = 0;
  for (int i = 0; i < g.n; i++) {
    g.cb0[i] = (g.pa[i].Nq + wc - 1) / wc;
    g.start[i] = total;
    total += g.cb0[i] + (g.pb[i].Nq + wc - 1) / wc;
  }
  g.start[g.n] = total;
  return total;
}

// Workgroup `bid` (< g.start[g.n]) of a gradient group, with nw summing waves.
template <int CPL>
__device__ __forceinline__ void lora_cols_group_block(const ColsGroup& g, int M, int ldt, int r,
                                                      int bid, int nw, float* red) {
  int i = 0;
  while (i + 1 < g.n && bid >= g.start[i + 1]) i++;
  lora_cols_block<CPL>(g.pa[i], g.pb[i], g.cb0[i], M, ldt, r, bid - g.start[i], nw, red);
}

}  // namespace mxs
