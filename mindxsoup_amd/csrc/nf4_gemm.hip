// Fused NF4-dequant GEMMs for gfx950: the frozen Linear4bit forward and its input gradient.
//
//   forward  (solution/linear4bit.py:47-49):  Y[M,N]  = X[M,K] . W[N,K]^T  (+ bias) (+ LoRA)
//   backward (solution/linear4bit.py:51-57):  dX[M,K] = dY[M,N] . W[N,K]            (+ LoRA)
//
// Both are one kernel, C[M,Nc] = A[M,Kr] . B[Nc,Kr]^T with B decoded from NF4 on the fly:
//   forward:  B = W   (Nc = N, Kr = K; NF4 contiguous along B's reduction dim)
//   backward: B = W^T (Nc = K, Kr = N; NF4 contiguous along B's output dim)
// Each K-step of 64 reduction indices stages A (fp16, straight copy) and B (NF4 decoded to the
// exact fp16 the standalone dequant writes) into LDS, double buffered, and feeds
// v_mfma_f32_32x32x16_f16 with fp32 accumulation.  The NF4 bytes of the next K-step are loaded
// while the current one multiplies.  LDS rows are 64 fp16 (128 B) with the 16-byte segments
// XOR-swizzled by the row index, so MFMA operand reads and the tile writes are bank-conflict
// free.
//
// Epilogue: + bias, + the LoRA term as one more MFMA per 32x32 tile (K = r), dropout mask on the
// LoRA term of the input gradient, fp16 store.  With split-K (gridDim.z > 1) each split writes
// fp32 partials and k_splitk_reduce sums them (split 0 carries bias and LoRA).
#include "common.h"
#include "mxs_nf4.h"

namespace mxs {

constexpr int kBK = 64;           // reduction indices per K-step (one NF4 block in forward)
constexpr int kThreads = 256;     // 4 waves

struct GemmArgs {
  const _Float16* A;        // [M, lda]
  int64_t lda;
  const uint8_t* packed;    // NF4 W [Nw, Kw] (Nw = out_features, Kw = in_features)
  const uint8_t* absmax8;
  const float* code;
  const float* absmax2;
  const float* offset;
  int M, Nc, Kr;            // C is [M, Nc], reduction Kr
  int Kw;                   // in_features (row length of W)
  // epilogue
  const _Float16* bias;     // [Nc] (forward) or null
  const _Float16* lora_h;   // [M, r]: s*H (forward) or s*dH (backward), or null
  const _Float16* lora_w;   // forward: lora_B [Nc, r]; backward: lora_A [r, Nc]
  int r;
  const uint8_t* mask;      // backward: dropout keep mask [M, Nc] or null
  float mask_scale;         // 1 / (1 - p)
  _Float16* C;              // [M, ldc]
  int64_t ldc;
  float* ws;                // split-K partials [splits, M, Nc]
  int steps_per_split;
};

// LDS offset (in halfs) of 16-byte segment `seg` (0..7) of row `row` in a [rows][64] tile.
__device__ __forceinline__ int lds_off(int row, int seg) {
  return row * kBK + (((seg ^ row ^ (row >> 3)) & 7) << 3);
}

__device__ __forceinline__ float block_scale_at(const GemmArgs& a, int64_t blk) {
  return nested_scale(a.code[a.absmax8[blk]], a.absmax2[blk >> 8], a.offset[0]);
}

template <int BM, int BN, int WAVES_M, bool BWD>
struct Tile {
  static constexpr int WAVES_N = 4 / WAVES_M;
  static constexpr int WM = BM / WAVES_M;
  static constexpr int WN = BN / WAVES_N;
  static constexpr int TM = WM / 32;               // 32x32 MFMA tiles per wave along M
  static constexpr int TN = WN / 32;
  static constexpr int A_ITEMS = BM * 8 / kThreads;  // 16-byte A segments per thread
  // forward B items: (row, half) = 32 NF4 values; backward: 4 W rows x 8 cols
  static constexpr int B_ITEMS = BWD ? (BN / 8) * (kBK / 4) / kThreads : BN * 2 / kThreads;
  static_assert(WM % 32 == 0 && WN % 32 == 0, "wave tile");
  static_assert(A_ITEMS >= 1 && B_ITEMS >= 1, "tile too small for 256 threads");
  static constexpr int LDS_A = BM * kBK;            // halfs per buffer
  static constexpr int LDS_B = BN * kBK;
};

template <int BM, int BN, int WAVES_M, bool BWD>
__global__ __launch_bounds__(kThreads, 1) void k_nf4_gemm(GemmArgs a) {
  using T = Tile<BM, BN, WAVES_M, BWD>;
  extern __shared__ __attribute__((aligned(16))) _Float16 smem[];
  _Float16* As = smem;                      // [2][BM][64]
  _Float16* Bs = smem + 2 * T::LDS_A;       // [2][BN][64]
  __shared__ float s_nf4[16];

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int wm0 = (wave / T::WAVES_N) * T::WM;
  const int wn0 = (wave % T::WAVES_N) * T::WN;
  const int m0 = blockIdx.y * BM;
  const int n0 = blockIdx.x * BN;
  const int n_steps = a.Kr / kBK;
  const int kt0 = blockIdx.z * a.steps_per_split;
  const int kt1 = min(n_steps, kt0 + a.steps_per_split);
  if (t < 16) s_nf4[t] = kNF4[t];

  // ---- prefetch registers ----
  u32x4 a_pf[T::A_ITEMS];
  uint32_t b_pf[T::B_ITEMS][4];
  float b_sc[T::B_ITEMS][BWD ? 4 : 1];

  auto load_tile = [&](int kt) {
    const int k0 = kt * kBK;
#pragma unroll
    for (int u = 0; u < T::A_ITEMS; u++) {
      const int q = t + u * kThreads;
      const int row = q >> 3, seg = q & 7;
      const int m = m0 + row;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (m < a.M) v = *reinterpret_cast<const u32x4*>(a.A + (int64_t)m * a.lda + k0 + seg * 8);
      a_pf[u] = v;
    }
#pragma unroll
    for (int u = 0; u < T::B_ITEMS; u++) {
      const int q = t + u * kThreads;
      if (!BWD) {
        // W row n = n0 + q/2, values k0 + 32*(q&1) .. +32 (16 bytes, inside one NF4 block)
        const int n = n0 + (q >> 1);
        const int half = q & 1;
        if (n < a.Nc) {
          const int64_t byte = (int64_t)n * (a.Kw / 2) + k0 / 2 + half * 16;
          const u32x4 w = *reinterpret_cast<const u32x4*>(a.packed + byte);
#pragma unroll
          for (int j = 0; j < 4; j++) b_pf[u][j] = w[j];
          b_sc[u][0] = block_scale_at(a, ((int64_t)n * a.Kw + k0) >> 6);
        } else {
#pragma unroll
          for (int j = 0; j < 4; j++) b_pf[u][j] = 0x77777777u;  // NF4 index 7 = 0.0
          b_sc[u][0] = 0.0f;
        }
      } else {
        // W rows k0 + 4*rg .. +4 (reduction), cols n0 + 8*chunk .. +8 (output)
        const int chunk = q % (BN / 8);
        const int rg = q / (BN / 8);
        const int col = n0 + chunk * 8;
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int wrow = k0 + rg * 4 + i;
          if (col < a.Nc) {
            const int64_t idx = (int64_t)wrow * a.Kw + col;
            b_pf[u][i] = *reinterpret_cast<const uint32_t*>(a.packed + (idx >> 1));
            b_sc[u][i] = block_scale_at(a, idx >> 6);
          } else {
            b_pf[u][i] = 0x77777777u;
            b_sc[u][i] = 0.0f;
          }
        }
      }
    }
  };

  auto store_tile = [&](int buf) {
    _Float16* as = As + buf * T::LDS_A;
    _Float16* bs = Bs + buf * T::LDS_B;
#pragma unroll
    for (int u = 0; u < T::A_ITEMS; u++) {
      const int q = t + u * kThreads;
      *reinterpret_cast<u32x4*>(as + lds_off(q >> 3, q & 7)) = a_pf[u];
    }
#pragma unroll
    for (int u = 0; u < T::B_ITEMS; u++) {
      const int q = t + u * kThreads;
      if (!BWD) {
        const int row = q >> 1, half = q & 1;
        const float s = b_sc[u][0];
#pragma unroll
        for (int d = 0; d < 4; d++)
          *reinterpret_cast<u32x4*>(bs + lds_off(row, half * 4 + d)) = decode8(b_pf[u][d], s, s_nf4);
      } else {
        const int chunk = q % (BN / 8);
        const int rg = q / (BN / 8);
        // column c of the 8: values of rows rg*4 .. +4 -> 4 fp16 along the reduction dim
#pragma unroll
        for (int c = 0; c < 8; c++) {
          const int sh = 8 * (c >> 1) + ((c & 1) ? 0 : 4);
          u32x2 v;
          v[0] = pack_f16x2(s_nf4[(b_pf[u][0] >> sh) & 15u] * b_sc[u][0],
                            s_nf4[(b_pf[u][1] >> sh) & 15u] * b_sc[u][1]);
          v[1] = pack_f16x2(s_nf4[(b_pf[u][2] >> sh) & 15u] * b_sc[u][2],
                            s_nf4[(b_pf[u][3] >> sh) & 15u] * b_sc[u][3]);
          const int row = chunk * 8 + c;
          *reinterpret_cast<u32x2*>(bs + lds_off(row, rg >> 1) + (rg & 1) * 4) = v;
        }
      }
    }
  };

  float16_t acc[T::TM][T::TN];
#pragma unroll
  for (int i = 0; i < T::TM; i++)
#pragma unroll
    for (int j = 0; j < T::TN; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[i][j][e] = 0.0f;

  const int lrow = lane & 31;
  const int lseg = lane >> 5;

  if (kt0 < kt1) {
    load_tile(kt0);
    __syncthreads();  // s_nf4 ready
    store_tile(0);
    __syncthreads();
    for (int kt = kt0; kt < kt1; kt++) {
      const int cur = (kt - kt0) & 1;
      if (kt + 1 < kt1) load_tile(kt + 1);
      const _Float16* as = As + cur * T::LDS_A;
      const _Float16* bs = Bs + cur * T::LDS_B;
#pragma unroll
      for (int kk = 0; kk < kBK / 16; kk++) {
        half8_t af[T::TM], bf[T::TN];
#pragma unroll
        for (int i = 0; i < T::TM; i++)
          af[i] = *reinterpret_cast<const half8_t*>(as + lds_off(wm0 + i * 32 + lrow, 2 * kk + lseg));
#pragma unroll
        for (int j = 0; j < T::TN; j++)
          bf[j] = *reinterpret_cast<const half8_t*>(bs + lds_off(wn0 + j * 32 + lrow, 2 * kk + lseg));
#pragma unroll
        for (int i = 0; i < T::TM; i++)
#pragma unroll
          for (int j = 0; j < T::TN; j++)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
      }
      if (kt + 1 < kt1) store_tile(cur ^ 1);
      __syncthreads();
    }
  }

  // ---- epilogue ----
  const bool first_split = blockIdx.z == 0;
  const bool split = gridDim.z > 1;
  // LoRA term: (s*H)[M, r] . lora_B[N, r]^T  (forward)  or  (s*dH)[M, r] . lora_A[r, N] (backward,
  // times the dropout keep mask and 1/(1-p) when a mask is given).  One 32x32x16 MFMA per tile
  // and 16 LoRA ranks, done one 32-row tile at a time to keep few registers live.
  if (a.lora_h && first_split) {
#pragma unroll
    for (int i = 0; i < T::TM; i++) {
      float16_t lacc[T::TN];
#pragma unroll
      for (int j = 0; j < T::TN; j++)
#pragma unroll
        for (int e = 0; e < 16; e++) lacc[j][e] = 0.0f;
      const int mrow = m0 + wm0 + i * 32 + lrow;
      for (int r0 = 0; r0 < a.r; r0 += 16) {
        half8_t hf = {};
        if (mrow < a.M) hf = *reinterpret_cast<const half8_t*>(a.lora_h + (int64_t)mrow * a.r + r0 + 8 * lseg);
#pragma unroll
        for (int j = 0; j < T::TN; j++) {
          const int n = n0 + wn0 + j * 32 + lrow;
          half8_t wf = {};
          if (n < a.Nc) {
            if (!BWD) {
              wf = *reinterpret_cast<const half8_t*>(a.lora_w + (int64_t)n * a.r + r0 + 8 * lseg);
            } else {
#pragma unroll
              for (int e = 0; e < 8; e++) wf[e] = a.lora_w[(int64_t)(r0 + 8 * lseg + e) * a.Nc + n];
            }
          }
          lacc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(hf, wf, lacc[j], 0, 0, 0);
        }
      }
#pragma unroll
      for (int j = 0; j < T::TN; j++)
#pragma unroll
        for (int e = 0; e < 16; e++) {
          float l = lacc[j][e];
          if (BWD && a.mask) {
            const int m = m0 + wm0 + i * 32 + 8 * (e >> 2) + 4 * lseg + (e & 3);
            const int n = n0 + wn0 + j * 32 + lrow;
            const bool keep = m < a.M && n < a.Nc && a.mask[(int64_t)m * a.Nc + n] != 0;
            l = keep ? l * a.mask_scale : 0.0f;
          }
          acc[i][j][e] += l;
        }
    }
  }

#pragma unroll
  for (int j = 0; j < T::TN; j++) {
    const int n = n0 + wn0 + j * 32 + lrow;
    if (n >= a.Nc) continue;
    const float b = (a.bias && first_split) ? (float)a.bias[n] : 0.0f;
#pragma unroll
    for (int i = 0; i < T::TM; i++) {
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const int m = m0 + wm0 + i * 32 + 8 * (e >> 2) + 4 * lseg + (e & 3);
        if (m >= a.M) continue;
        const float v = acc[i][j][e] + b;
        if (split)
          a.ws[((int64_t)blockIdx.z * a.M + m) * a.Nc + n] = v;
        else
          a.C[(int64_t)m * a.ldc + n] = (_Float16)v;
      }
    }
  }
}

// Sum of split-K partials -> fp16.  ws [splits, M, Nc] fp32.
__global__ __launch_bounds__(256) void k_splitk_reduce(const float* __restrict__ ws, int splits,
                                                      int M, int Nc, _Float16* __restrict__ C,
                                                      int64_t ldc) {
  const int64_t total = (int64_t)M * Nc;
  const int64_t plane = total;
  for (int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4; i < total;
       i += (int64_t)gridDim.x * 256 * 4) {
    float4_t s = {0.f, 0.f, 0.f, 0.f};
    const bool vec = (Nc % 4 == 0) && i + 3 < total;
    if (vec) {
      for (int z = 0; z < splits; z++) s += *reinterpret_cast<const float4_t*>(ws + z * plane + i);
      const int64_t m = i / Nc, n = i % Nc;
      half4_t h = __builtin_convertvector(s, half4_t);
      *reinterpret_cast<half4_t*>(C + m * ldc + n) = h;
    } else {
      for (int64_t e = i; e < i + 4 && e < total; e++) {
        float v = 0.f;
        for (int z = 0; z < splits; z++) v += ws[z * plane + e];
        C[(e / Nc) * ldc + e % Nc] = (_Float16)v;
      }
    }
  }
}

template <int BM, int BN, int WAVES_M, bool BWD>
static int launch_cfg(const GemmArgs& a0, int splits, hipStream_t stream) {
  using T = Tile<BM, BN, WAVES_M, BWD>;
  GemmArgs a = a0;
  const int n_steps = a.Kr / kBK;
  if (splits < 1) splits = 1;
  if (splits > n_steps) splits = n_steps > 0 ? n_steps : 1;
  a.steps_per_split = (n_steps + splits - 1) / splits;
  splits = n_steps > 0 ? (n_steps + a.steps_per_split - 1) / a.steps_per_split : 1;
  if (splits > 1 && !a.ws) return MXS_ERR_ARG;
  const dim3 grid((a.Nc + BN - 1) / BN, (a.M + BM - 1) / BM, splits);
  const size_t lds = (size_t)2 * (T::LDS_A + T::LDS_B) * sizeof(_Float16);
  static bool lds_set = false;  // idempotent attribute; a benign race between threads
  if (!lds_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_nf4_gemm<BM, BN, WAVES_M, BWD>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return (int)e;
    lds_set = true;
  }
  hipLaunchKernelGGL((k_nf4_gemm<BM, BN, WAVES_M, BWD>), grid, dim3(kThreads), lds, stream, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return (int)e;
  if (splits > 1) {
    const int64_t total = (int64_t)a.M * a.Nc;
    int64_t blocks = (total / 4 + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL(k_splitk_reduce, dim3((unsigned)blocks), dim3(256), 0, stream, a.ws, splits,
                       a.M, a.Nc, a.C, a.ldc);
    e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
  }
  return MXS_OK;
}

// Tile configurations, by id (mxs_nf4_gemm_config_*): BM x BN, waves along M.
template <bool BWD>
static int launch_by_id(int cfg, const GemmArgs& a, int splits, hipStream_t s) {
  switch (cfg) {
    case 0: return launch_cfg<256, 128, 2, BWD>(a, splits, s);
    case 1: return launch_cfg<128, 128, 2, BWD>(a, splits, s);
    case 2: return launch_cfg<128, 256, 2, BWD>(a, splits, s);
    case 3: return launch_cfg<256, 256, 2, BWD>(a, splits, s);
    case 4: return launch_cfg<64, 128, 1, BWD>(a, splits, s);
    default: return MXS_ERR_ARG;
  }
}

static const int kCfgBM[] = {256, 128, 128, 256, 64};
static const int kCfgBN[] = {128, 128, 256, 256, 128};
constexpr int kNumCfg = 5;

// Tile and split choice for one GEMM: fill the 256 CUs with whole tiles where the shape allows,
// else split the reduction (each split keeps at least 4 K-steps).
static void choose(int M, int Nc, int Kr, int* cfg, int* splits) {
  const int n_steps = Kr / kBK;
  const int order[] = {0, 2, 1, 4};
  int best = 0, best_split = 1;
  double best_score = -1.0;
  for (int c : order) {
    const int64_t tiles = (int64_t)((M + kCfgBM[c] - 1) / kCfgBM[c]) * ((Nc + kCfgBN[c] - 1) / kCfgBN[c]);
    for (int sp = 1; sp <= 16; sp *= 2) {
      if (sp > 1 && n_steps / sp < 4) break;
      const int64_t wgs = tiles * sp;
      const double waves = (double)wgs / 256.0;
      const double fill = waves / ((double)((wgs + 255) / 256));
      // efficiency: CU fill x tile-size factor (bigger tiles reuse more) x split-K overhead
      const double tile_eff = (kCfgBM[c] * kCfgBN[c]) / (kCfgBM[c] + kCfgBN[c]) / 85.3;
      const double split_pen = sp > 1 ? 1.0 / (1.0 + 0.08 * sp) : 1.0;
      const double score = fill * (tile_eff > 1.0 ? 1.0 : tile_eff) * split_pen;
      if (score > best_score + 1e-9) {
        best_score = score;
        best = c;
        best_split = sp;
      }
    }
  }
  *cfg = best;
  *splits = best_split;
}

static int gemm_entry(bool bwd, const GemmArgs& a, int cfg, int splits, hipStream_t stream) {
  if (a.M < 0 || a.Nc < 0 || a.Kr < 0) return MXS_ERR_ARG;
  if (a.M == 0 || a.Nc == 0) return MXS_OK;
  if (!a.A || !a.packed || !a.absmax8 || !a.code || !a.absmax2 || !a.offset || !a.C)
    return MXS_ERR_ARG;
  if (a.Kr % kBK != 0 || a.Kw % kBK != 0) return MXS_ERR_SIZE;
  if (bwd && a.Nc % 8 != 0) return MXS_ERR_SIZE;
  if (a.lda % 8 != 0 || ((uintptr_t)a.A % 16) != 0 || ((uintptr_t)a.packed % 16) != 0)
    return MXS_ERR_ALIGN;
  if (a.lora_h && (!a.lora_w || a.r <= 0 || a.r % 16 != 0)) return MXS_ERR_SIZE;
  if (a.lora_h && (((uintptr_t)a.lora_h % 16) != 0 || (!bwd && ((uintptr_t)a.lora_w % 16) != 0)))
    return MXS_ERR_ALIGN;
  if (cfg < 0) choose(a.M, a.Nc, a.Kr, &cfg, &splits);
  if (cfg >= kNumCfg) return MXS_ERR_ARG;
  return bwd ? launch_by_id<true>(cfg, a, splits, stream)
             : launch_by_id<false>(cfg, a, splits, stream);
}

}  // namespace mxs

using namespace mxs;

extern "C" {

int64_t mxs_nf4_gemm_workspace_bytes(int M, int Nc, int Kr, int cfg, int splits) {
  if (cfg < 0) choose(M, Nc, Kr, &cfg, &splits);
  if (splits <= 1) return 0;
  return (int64_t)splits * M * Nc * (int64_t)sizeof(float);
}

int mxs_nf4_linear_fwd(const void* x, int M, int K, int N, const void* packed,
                       const void* absmax8, const float* code, const float* absmax2,
                       const float* offset, const void* bias, const void* lora_h,
                       const void* lora_b, int r, void* y, void* workspace, int cfg, int splits,
                       hipStream_t stream) {
  GemmArgs a{};
  a.A = static_cast<const _Float16*>(x);
  a.lda = K;
  a.packed = static_cast<const uint8_t*>(packed);
  a.absmax8 = static_cast<const uint8_t*>(absmax8);
  a.code = code;
  a.absmax2 = absmax2;
  a.offset = offset;
  a.M = M;
  a.Nc = N;
  a.Kr = K;
  a.Kw = K;
  a.bias = static_cast<const _Float16*>(bias);
  a.lora_h = static_cast<const _Float16*>(lora_h);
  a.lora_w = static_cast<const _Float16*>(lora_b);
  a.r = r;
  a.C = static_cast<_Float16*>(y);
  a.ldc = N;
  a.ws = static_cast<float*>(workspace);
  return gemm_entry(false, a, cfg, splits, stream);
}

int mxs_nf4_linear_bwd_dx(const void* dy, int M, int N, int K, const void* packed,
                          const void* absmax8, const float* code, const float* absmax2,
                          const float* offset, const void* lora_dh, const void* lora_a, int r,
                          const void* mask, float mask_scale, void* dx, void* workspace, int cfg,
                          int splits, hipStream_t stream) {
  GemmArgs a{};
  a.A = static_cast<const _Float16*>(dy);
  a.lda = N;
  a.packed = static_cast<const uint8_t*>(packed);
  a.absmax8 = static_cast<const uint8_t*>(absmax8);
  a.code = code;
  a.absmax2 = absmax2;
  a.offset = offset;
  a.M = M;
  a.Nc = K;
  a.Kr = N;
  a.Kw = K;
  a.lora_h = static_cast<const _Float16*>(lora_dh);
  a.lora_w = static_cast<const _Float16*>(lora_a);
  a.r = r;
  a.mask = static_cast<const uint8_t*>(mask);
  a.mask_scale = mask_scale;
  a.C = static_cast<_Float16*>(dx);
  a.ldc = K;
  a.ws = static_cast<float*>(workspace);
  return gemm_entry(true, a, cfg, splits, stream);
}

}  // extern "C"
