/*
 * CPU oracle for the NF4 quantized-linear hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the HIP path is compared
 * against (tests/, the smoke check and the CPU-baseline leg of the bench).  The
 * product library never links, loads or calls it.
 *
 * Every function restates the reference's algorithm in plain scalar C, citing
 * the reference file:line it follows (paths relative to the MindXSoup tree).
 *
 * Pinning (what checks each function independently of this restatement):
 *   nf4_table            - recomputed from the normal-quantile definition
 *                          (scipy norm.ppf) and the QLoRA paper's table.
 *   f32_to_f16_rne       - numpy's IEEE float16 conversion over every class of
 *                          input (normals, subnormals, ties, overflow, NaN).
 *   dequant_nf4          - closed-form special cases (code index 7 -> +-0,
 *                          index 15 -> +s), a brute force over all 256 byte
 *                          values, the fused/unfused 1-ulp bound, an
 *                          independent numpy vectorised restatement, and the
 *                          quantize -> dequantize error bound, which fails for
 *                          a swapped nibble order or a wrong block index.
 *   quantize_nf4 / quantize_absmax_256 / dynamic_map
 *                        - round-trip bounds and the nearest-code property
 *                          (brute force over every candidate code).
 *   silu_mul / silu_mul_bwd
 *                        - float64 evaluation of the same formulas (within one
 *                          fp16 ulp), closed forms at gate = 0 (out = 0,
 *                          d_up = 0, d_gate = dh * up / 2) and for large |gate|
 *                          (silu -> gate or 0), and the differently ordered
 *                          derivative of solution/test_silu_mul.py:13-19.
 *   qkv_rope             - float64 rotate-half RoPE (transformers'
 *                          apply_rotary_pos_emb, solution/test_rope.py:19-23)
 *                          within one fp16 ulp; forward then backward restores
 *                          the input (a rotation and its inverse); pair norms
 *                          preserved; closed forms (cos = 1, sin = 0 is the
 *                          identity; cos = 0, sin = 1 maps (x1, x2) to
 *                          (-x2, x1)); a power-of-two LoRA scale equals adding
 *                          the pre-scaled LoRA (solution/test_attention.py:226).
 *   The GEMM / LoRA references live in oracle/oracle.py (numpy) and are pinned
 *   against float64 torch autograd.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <stdlib.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* The 16 NF4 values, QLoRA (Dettmers et al. 2023, arXiv 2305.14314) Appendix E;
 * bitsandbytes' get_4bit_type("nf4") returns the same list (called at
 * solution/nf4.py:116-123). Index 7 is the exact zero. */
static const float NF4[16] = {
    -1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f,
    -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f,
    0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f,
    0.33791524171829224f, 0.44070982933044434f, 0.5626170039176941f,
    0.7229568362236023f, 1.0f};

void oracle_nf4_table(float *out) { memcpy(out, NF4, sizeof(NF4)); }

/* IEEE-754 binary32 -> binary16, round to nearest, ties to even, with
 * subnormals, overflow to infinity and NaN kept quiet.  This is the rounding
 * Triton's `.to(tl.float16)` applies at solution/nf4.py:50 and :80. */
uint16_t oracle_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    if (exp == 0xffu) { /* inf / nan */
        return (uint16_t)(sign | 0x7c00u | (man ? (0x200u | (man >> 13)) : 0));
    }
    int e = (int)exp - 127 + 15; /* biased half exponent */
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        /* subnormal half (or zero): value = man_full * 2^(exp-150); half ulp = 2^-24 */
        if (e < -10) return (uint16_t)sign; /* below half of the smallest subnormal */
        uint32_t full = man | 0x800000u;
        uint32_t shift = (uint32_t)(14 - e); /* 24-bit significand -> 10-bit field */
        uint32_t q = full >> shift;
        uint32_t rem = full & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q); /* q may carry into the exponent field: correct */
    }
    uint32_t q = ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++; /* carry into exponent ok */
    return (uint16_t)(sign | q);
}

float oracle_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t x;
    if (exp == 0) {
        if (man == 0) {
            x = sign;
        } else { /* subnormal: normalise */
            int e = -1;
            do { man <<= 1; e++; } while (!(man & 0x400u));
            man &= 0x3ffu;
            x = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 31) {
        x = sign | 0x7f800000u | (man << 13);
    } else {
        x = sign | ((exp - 15 + 127) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/* Block scale of the double-quantized absmax: solution/nf4.py:40-43 / :70-73,
 * code[q8] * absmax2[blk // 256] + offset in fp32.  Triton contracts the
 * multiply-add into one FMA by default (the "one fp16 ulp" note at
 * solution/test_nf4.py:41); `fused` selects that (1) or the two roundings (0). */
static inline float block_scale(const uint8_t *absmax8, const float *code,
                                const float *absmax2, float offset, int64_t blk, int fused) {
    float c = code[absmax8[blk]];
    float a2 = absmax2[blk >> 8];
    if (fused) return fmaf(c, a2, offset);
    volatile float prod = c * a2; /* force the separate rounding */
    return prod + offset;
}

/* One-byte restatement of nf4_unpack_kernel (solution/nf4.py:31-51) which the
 * wide kernel (:54-86) must match bit for bit: byte i holds values 2i (high
 * nibble) and 2i+1 (low nibble); block = i // 32; out = fp16(NF4[q] * scale).
 * nested != 0: scale from (absmax8, code, absmax2, offset); else absmax_f32[blk]
 * (solution/nf4.py:44-45).  Output is fp16 bit patterns, 2*n_bytes of them. */
void oracle_dequant_nf4(const uint8_t *packed, int64_t n_bytes, const uint8_t *absmax8,
                        const float *code, const float *absmax2, float offset,
                        const float *absmax_f32, int nested, int fused, uint16_t *out) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n_bytes; i++) {
        int64_t blk = i >> 5;
        float s = nested ? block_scale(absmax8, code, absmax2, offset, blk, fused)
                         : absmax_f32[blk];
        uint8_t b = packed[i];
        out[2 * i] = oracle_f32_to_f16(NF4[b >> 4] * s);
        out[2 * i + 1] = oracle_f32_to_f16(NF4[b & 15] * s);
    }
}

/* fp32 output variant (unpack_nf4's dtype=torch.float32 case, nf4.py:166). */
void oracle_dequant_nf4_f32(const uint8_t *packed, int64_t n_bytes, const uint8_t *absmax8,
                            const float *code, const float *absmax2, float offset,
                            const float *absmax_f32, int nested, int fused, float *out) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n_bytes; i++) {
        int64_t blk = i >> 5;
        float s = nested ? block_scale(absmax8, code, absmax2, offset, blk, fused)
                         : absmax_f32[blk];
        uint8_t b = packed[i];
        out[2 * i] = NF4[b >> 4] * s;
        out[2 * i + 1] = NF4[b & 15] * s;
    }
}

/* The grouped (whole-layer) form of solution/nf4.py:89-110: several weights,
 * each with its own code book, second-level scales and offset, decoded in one
 * call.  Here simply a loop over the per-weight form. */
void oracle_dequant_nf4_grouped(int n_weights, const uint8_t *const *packed,
                                const int64_t *n_bytes, const uint8_t *const *absmax8,
                                const float *const *code, const float *const *absmax2,
                                const float *offset, uint16_t *const *out) {
    for (int w = 0; w < n_weights; w++)
        oracle_dequant_nf4(packed[w], n_bytes[w], absmax8[w], code[w], absmax2[w], offset[w],
                           NULL, 1, 1, out[w]);
}

/* ---------------------------------------------------------------------------
 * Quantizer (upstream of the path: makes synthetic NF4 weights).  Restates the
 * published bitsandbytes algorithm behind quantize_4bit(..., quant_type="nf4",
 * compress_statistics=True) as the reference calls it (solution/test_nf4.py:33,
 * tools/bench_nf4.py:30-35).  Exact equality with bitsandbytes is not required:
 * the path's contract starts at the packed tensors.
 * ------------------------------------------------------------------------- */

/* Signed dynamic-tree code book, 8 bits, 7 exponent bits (Dettmers, "8-bit
 * approximations for parallelism in deep learning", arXiv 1511.04561): for
 * decade i = 0..6 the 2^i midpoints of an even split of [0.1, 1] scaled by
 * 10^(i-6), both signs, plus 0 and 1; sorted ascending. */
void oracle_dynamic_map(float *out) {
    float v[256];
    int n = 0;
    for (int i = 0; i < 7; i++) {
        int items = (1 << i) + 1; /* boundaries in [0.1, 1] */
        double scale = pow(10.0, (double)(i - 6));
        for (int j = 0; j + 1 < items; j++) {
            /* boundaries as fp32 like a float32 linspace, midpoint in fp32 */
            float b0 = (float)(0.1 + 0.9 * (double)j / (double)(items - 1));
            float b1 = (float)(0.1 + 0.9 * (double)(j + 1) / (double)(items - 1));
            float mid = (b0 + b1) / 2.0f;
            v[n++] = (float)(scale * (double)mid);
            v[n++] = (float)(-scale * (double)mid);
        }
    }
    v[n++] = 0.0f;
    v[n++] = 1.0f;
    /* n == 256 */
    for (int i = 1; i < n; i++) { /* insertion sort */
        float key = v[i];
        int j = i - 1;
        while (j >= 0 && v[j] > key) { v[j + 1] = v[j]; j--; }
        v[j + 1] = key;
    }
    memcpy(out, v, sizeof(float) * 256);
}

/* Nearest NF4 index of a value already divided by the block absmax: the index
 * of the first table entry whose upper midpoint is >= x (ties go down). */
static inline int nf4_nearest(float x) {
    int q = 0;
    for (int i = 0; i < 15; i++) {
        float mid = (float)(((double)NF4[i] + (double)NF4[i + 1]) * 0.5);
        if (x > mid) q = i + 1;
    }
    return q;
}

/* Per-64 absmax and packed nibbles, high nibble first.  w: fp16 bit patterns,
 * n a multiple of 64 (all Qwen2.5-1.5B shapes are). */
void oracle_quantize_nf4(const uint16_t *w, int64_t n, uint8_t *packed, float *absmax) {
    int64_t n_blocks = n / 64;
#pragma omp parallel for schedule(static)
    for (int64_t b = 0; b < n_blocks; b++) {
        float m = 0.0f;
        for (int j = 0; j < 64; j++) {
            float a = fabsf(oracle_f16_to_f32(w[b * 64 + j]));
            if (a > m) m = a;
        }
        absmax[b] = m;
        float inv = m > 0.0f ? 1.0f / m : 0.0f;
        for (int j = 0; j < 64; j += 2) {
            int hi = nf4_nearest(oracle_f16_to_f32(w[b * 64 + j]) * inv);
            int lo = nf4_nearest(oracle_f16_to_f32(w[b * 64 + j + 1]) * inv);
            packed[b * 32 + j / 2] = (uint8_t)((hi << 4) | lo);
        }
    }
}

/* Mean of the block absmax values (bitsandbytes: absmax.mean()), summed in double in a fixed
 * order: spans of 4096 blocks, each summed by 256 lane-strided partials combined pairwise
 * (d = 128, 64, ..., 1), then the span sums in index order.  A fixed order makes the quantizer
 * reproducible; the order itself is a choice of this build, not of the reference. */
float oracle_absmax_mean(const float *absmax, int64_t n_blocks) {
    double total = 0.0;
    for (int64_t base = 0; base < n_blocks; base += 4096) {
        double lane[256];
        for (int t = 0; t < 256; t++) {
            double acc = 0.0;
            for (int i = t; i < 4096; i += 256)
                if (base + i < n_blocks) acc += (double)absmax[base + i];
            lane[t] = acc;
        }
        for (int d = 128; d > 0; d >>= 1)
            for (int t = 0; t < d; t++) lane[t] += lane[t + d];
        total += lane[0];
    }
    return (float)(total / (double)n_blocks);
}

/* Index of the code entry nearest to x (code sorted ascending; ties -> lower). */
static inline int code_nearest(const float *code, float x) {
    int lo = 0, hi = 255;
    while (hi - lo > 1) { /* largest index with code[idx] <= x */
        int mid = (lo + hi) >> 1;
        if (code[mid] <= x) lo = mid; else hi = mid;
    }
    if (x <= code[0]) return 0;
    if (x >= code[255]) return 255;
    float dlo = x - code[lo], dhi = code[hi] - x;
    return dhi < dlo ? hi : lo;
}

/* Second level: (absmax - offset) quantized blockwise (256 per block) with the
 * signed dynamic code book: absmax2 = max |v| per 256-block, q8 = nearest code
 * of v / absmax2.  Decoded scale = code[q8] * absmax2 + offset (nf4.py:70-73). */
void oracle_quantize_absmax_256(const float *absmax, int64_t n_blocks, float offset,
                                const float *code, uint8_t *q8, float *absmax2) {
    int64_t n_groups = (n_blocks + 255) / 256;
#pragma omp parallel for schedule(static)
    for (int64_t g = 0; g < n_groups; g++) {
        int64_t b0 = g * 256, b1 = b0 + 256 < n_blocks ? b0 + 256 : n_blocks;
        float m = 0.0f;
        for (int64_t b = b0; b < b1; b++) {
            float a = fabsf(absmax[b] - offset);
            if (a > m) m = a;
        }
        absmax2[g] = m;
        float inv = m > 0.0f ? 1.0f / m : 0.0f;
        for (int64_t b = b0; b < b1; b++) q8[b] = (uint8_t)code_nearest(code, (absmax[b] - offset) * inv);
    }
}

/* Threads the OpenMP loops above use (1 without OpenMP). */
int oracle_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void oracle_set_num_threads(int n) {
#ifdef _OPENMP
    omp_set_num_threads(n);
#else
    (void)n;
#endif
}

/* SwiGLU of the fp16 MLP, solution/silu_mul.py:26-44 (silu_mul_kernel): values are computed
 * in fp32 from the fp16 inputs and rounded to fp16 once.  sigmoid(g) = 1 / (1 + exp(-g)).
 * Forward: out = fp16(up * (g * sigmoid(g))). */
static inline float sigmoid_f32(float g) { return 1.0f / (1.0f + expf(-g)); }

void oracle_silu_mul(const uint16_t *gate, const uint16_t *up, uint16_t *out, int64_t n) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) {
        const float g = oracle_f16_to_f32(gate[i]), u = oracle_f16_to_f32(up[i]);
        const float s = sigmoid_f32(g);
        const float silu = g * s;
        out[i] = oracle_f32_to_f16(u * silu);
    }
}

/* Backward (BACKWARD=True branch, silu_mul.py:35-41), for the incoming d(out) = dh:
 * d(gate) = fp16((dh * up) * (s + silu * (1 - s))), d(up) = fp16(dh * silu). */
void oracle_silu_mul_bwd(const uint16_t *dh, const uint16_t *gate, const uint16_t *up,
                         uint16_t *d_gate, uint16_t *d_up, int64_t n) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) {
        const float g = oracle_f16_to_f32(gate[i]), u = oracle_f16_to_f32(up[i]);
        const float d = oracle_f16_to_f32(dh[i]);
        const float s = sigmoid_f32(g);
        const float silu = g * s;
        d_gate[i] = oracle_f32_to_f16((d * u) * (s + silu * (1.0f - s)));
        d_up[i] = oracle_f32_to_f16(d * silu);
    }
}

/* q/k/v of Qwen2 attention, solution/attention.py:28-82 (qkv_rope_kernel, _qkv_heads): per
 * position (b, t) and head of 128 values, x = a (+ b * scale) in fp32; q and k heads rotated,
 * v heads not; one rounding to the output type.  With x1 = x[0:64], x2 = x[64:128], the cos
 * row c = (c1, c2) and the sin row s = (s1, s2) of the position:
 *   forward   y1 = x1 * c1 + x2 * (-s1)    y2 = x2 * c2 + x1 * s2
 *   backward  y1 = x1 * c1 + x2 * s2       y2 = x2 * c2 + x1 * (-s1)
 * (attention.py:70-74, rope.py:54-66: sign +1 / -1 with the sin halves swapped).  Each product
 * and sum is one fp32 operation (no contraction).  Layouts: inputs and outputs [B, T, H * 128]
 * contiguous (a [B, H, T, 128] view with [B, T, H, 128] memory, as the projections write it);
 * cos / sin fp32 [Bc, T, 128] with Bc = 1 (shared over the batch) or B.  q_b / v_b / v_a may
 * be NULL (no LoRA term; no v).  in_f32 / out_f32 select fp32 (1) or fp16 (0) storage. */
static inline float rope_load(const void *p, int64_t i, int f32) {
    return f32 ? ((const float *)p)[i] : oracle_f16_to_f32(((const uint16_t *)p)[i]);
}

static inline void rope_store(void *p, int64_t i, float v, int f32) {
    if (f32) ((float *)p)[i] = v;
    else ((uint16_t *)p)[i] = oracle_f32_to_f16(v);
}

static void rope_heads(const void *a, const void *b, float scale, void *y, int64_t row, int heads,
                       const float *c, const float *sn, int rotate, int backward, int in_f32,
                       int out_f32) {
    for (int h = 0; h < heads; h++) {
        const int64_t base = (row * heads + h) * 128;
        for (int j = 0; j < 64; j++) {
            float x1 = rope_load(a, base + j, in_f32), x2 = rope_load(a, base + 64 + j, in_f32);
            if (b) {
                x1 = x1 + rope_load(b, base + j, in_f32) * scale;
                x2 = x2 + rope_load(b, base + 64 + j, in_f32) * scale;
            }
            float y1 = x1, y2 = x2;
            if (rotate) {
                const float c1 = c[j], c2 = c[64 + j];
                const float p = backward ? sn[64 + j] : -sn[j];
                const float r = backward ? -sn[j] : sn[64 + j];
                y1 = x1 * c1 + x2 * p;
                y2 = x2 * c2 + x1 * r;
            }
            rope_store(y, base + j, y1, out_f32);
            rope_store(y, base + 64 + j, y2, out_f32);
        }
    }
}

void oracle_qkv_rope(const void *q_a, const void *q_b, const void *k, const void *v_a,
                     const void *v_b, const float *cos, const float *sin, int cos_batch,
                     void *q_o, void *k_o, void *v_o, int batch, int n_tokens, int n_q, int n_kv,
                     int in_f32, int out_f32, int backward, float q_scale, float v_scale) {
#pragma omp parallel for schedule(static)
    for (int64_t row = 0; row < (int64_t)batch * n_tokens; row++) {
        const int64_t crow = cos_batch == 1 ? row % n_tokens : row;
        const float *c = cos + crow * 128, *sn = sin + crow * 128;
        rope_heads(q_a, q_b, q_scale, q_o, row, n_q, c, sn, 1, backward, in_f32, out_f32);
        rope_heads(k, NULL, 1.0f, k_o, row, n_kv, c, sn, 1, backward, in_f32, out_f32);
        if (v_a) rope_heads(v_a, v_b, v_scale, v_o, row, n_kv, c, sn, 0, backward, in_f32, out_f32);
    }
}
