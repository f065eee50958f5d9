// ftm_cpu.cpp -- the host-CPU half of the hybrid CPU || GPU MoE split: routed
// experts computed on the host cores straight from the packed, pinned host
// banks (the slot pool's sources), so a decode step's misses can be shared
// between the PCIe fetch + GPU kernels and the CPU.
//
// The reference's CPU MoE kernel (python/freetoken/kernel/csrc/cpu_moe/
// cpu_moe.cpp:75-154, 470-528) only takes dense fp32 / bf16 banks, so its
// hybrid backend forces quantized checkpoints to pure offload
// (python/freetoken/models/qwen3_moe/__init__.py:730-733).  Here every bank
// format of the GPU kernels is decoded on the fly:
//   * K-major rows (FP8 e4m3 + 128x128 block scales, INT8 offset-binary +
//     group scales, MXFP4 e2m1 + e8m0, bf16, fp32): 16 weights of a row are
//     decoded into one AVX-512 register (bit arithmetic, no tables in memory;
//     MXFP4 through a 16-entry in-register permute), multiplied by their
//     group scale (the reference's fp32 dequant product, rounded once), then
//     one FMA per routed token of the expert;
//   * GPTQ (qweight [K/8, N], N contiguous): blocks of 16 output columns
//     accumulate the outer products of each packed row's 8 K values, so
//     every cache line of qweight is read once.
// Math as the reference CPU backend: fp32 gu, fp32 h (act(gate) * up, with
// the clamped GLU and the projection biases of gpt-oss), fp32 down
// projection, out[t] += w[t, j] * y, experts split into contiguous ranges
// over threads with private partial outputs summed at the end
// (cpu_moe.cpp:485-527).  A scalar path with the same arithmetic serves
// hosts without AVX-512.
//
// ftm_cpu_moe_submit / ftm_cpu_moe_wait run one such call on a persistent
// worker thread, one job at a time, so the caller enqueues the GPU half in
// the meantime (the reference's async worker: cpu_moe.cpp:596-706, 820-853).
#include <immintrin.h>
#include <math.h>
#include <string.h>

#include <algorithm>
#include <condition_variable>
#include <mutex>
#include <thread>
#include <vector>

#include "ftmoe.h"

namespace {

// ------------------------------------------------------------------ scalars
float bf16_f(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}
float f16_f(uint16_t h) {
  const uint32_t s = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 1023u;
  uint32_t u;
  if (e == 0) {
    float f = (float)m * 0x1p-24f;
    memcpy(&u, &f, 4);
    u |= s;
  } else if (e == 31) {
    u = s | 0x7f800000u | (m << 13);
  } else {
    u = s | ((e + 112u) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &u, 4);
  return f;
}
float load_dt(const void* p, int64_t i, int dt) {
  if (dt == FTM_DT_F32) return ((const float*)p)[i];
  if (dt == FTM_DT_F16) return f16_f(((const uint16_t*)p)[i]);
  return bf16_f(((const uint16_t*)p)[i]);
}
// OCP e4m3fn: bias 7, no infinities, S.1111.111 is NaN
float e4m3_f(uint32_t b) {
  const uint32_t s = (b & 0x80u) << 24, e = (b >> 3) & 15u, m = b & 7u;
  uint32_t u;
  if (e == 15 && m == 7) {
    u = s | 0x7fc00000u;
  } else if (e == 0) {
    float f = (float)m * 0x1p-9f;
    memcpy(&u, &f, 4);
    u |= s;
  } else {
    u = s | ((e + 120u) << 23) | (m << 20);
  }
  float f;
  memcpy(&f, &u, 4);
  return f;
}
float e5m2_f(uint32_t b) { return f16_f((uint16_t)(b << 8)); }
const float kE2M1[16] = {0.f, .5f, 1.f, 1.5f, 2.f, 3.f, 4.f, 6.f, -0.f, -.5f, -1.f, -1.5f, -2.f, -3.f, -4.f, -6.f};
// e8m0 as the reference decodes it (torch.exp2(e - 127)): the fp32 with
// exponent field e; 0 -> 2^-127 (subnormal), 255 -> inf
inline float e8m0_f(uint32_t e) {
  const uint32_t u = e == 0 ? 0x00400000u : e == 255 ? 0x7f800000u : e << 23;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

struct Slot {  // one slot of a projection bank, host pointers
  const char *w, *s, *z, *bias;
  int fmt, s_dt, bias_dt, group, N, K;
};
Slot slot_of(const ftm_proj& P, int slot) {
  Slot v;
  v.w = (const char*)P.w + (int64_t)slot * P.w_stride;
  v.s = P.s ? (const char*)P.s + (int64_t)slot * P.s_stride : nullptr;
  v.z = P.z ? (const char*)P.z + (int64_t)slot * P.z_stride : nullptr;
  v.bias = P.bias ? (const char*)P.bias + (int64_t)slot * P.bias_stride : nullptr;
  v.fmt = P.fmt;
  v.s_dt = P.s_dtype;
  v.bias_dt = P.bias_dtype;
  v.group = P.group;
  v.N = P.N;
  v.K = P.K;
  return v;
}

// Element (n, k) of the reference's dequantized weight (fp32 product, one rounding).
float deq(const Slot& W, int n, int k) {
  const int N = W.N, K = W.K;
  switch (W.fmt) {
    case FTM_FMT_FP8_BLOCK:
    case FTM_FMT_FP8_E5M2_BLOCK: {
      const uint32_t b = (uint8_t)W.w[(int64_t)n * K + k];
      const float v = W.fmt == FTM_FMT_FP8_BLOCK ? e4m3_f(b) : e5m2_f(b);
      const int nkb = (K + W.group - 1) / W.group;
      return v * load_dt(W.s, (int64_t)(n / W.group) * nkb + k / W.group, W.s_dt);
    }
    case FTM_FMT_GPTQ_INT4: {
      const uint32_t word = ((const uint32_t*)W.w)[(int64_t)(k / 8) * N + n];
      const int q = (int)((word >> (4 * (k & 7))) & 15u);
      const int g = k / W.group;
      const uint32_t zw = ((const uint32_t*)W.z)[(int64_t)g * (N / 8) + n / 8];
      const int z = (int)((zw >> (4 * (n & 7))) & 15u) + 1;
      return load_dt(W.s, (int64_t)g * N + n, W.s_dt) * (float)(q - z);
    }
    case FTM_FMT_INT8_PACKED: {
      const int v = (int)((uint8_t)W.w[(int64_t)n * K + k]) - 128;
      return (float)v * load_dt(W.s, (int64_t)n * (K / W.group) + k / W.group, W.s_dt);
    }
    case FTM_FMT_MXFP4: {
      const uint32_t b = (uint8_t)W.w[(int64_t)n * (K / 2) + k / 2];
      return kE2M1[(k & 1) ? b >> 4 : b & 15u] * e8m0_f((uint8_t)W.s[(int64_t)n * (K / 32) + k / 32]);
    }
    case FTM_FMT_FP32:
      return ((const float*)W.w)[(int64_t)n * K + k];
    default:
      return bf16_f(((const uint16_t*)W.w)[(int64_t)n * K + k]);
  }
}

float act_f(int act, float g, float u, float alpha, float limit) {
  if (act == FTM_ACT_SILU) return g / (1.0f + expf(-g)) * u;
  if (act == FTM_ACT_GELU) return 0.5f * g * (1.0f + erff(g * 0.70710678118654752f)) * u;
  if (act == FTM_ACT_RELU) return (g > 0.0f ? g : 0.0f) * u;
  g = g < limit ? g : limit;
  u = u < -limit ? -limit : (u > limit ? limit : u);
  return (u + 1.0f) * (g / (1.0f + expf(-alpha * g)));
}

// ------------------------------------------------------------------ projections
// y[t][n] = sum_k x[t][k] * W[n][k] (+ bias[n]) for t < M; x rows ldx apart, y rows ldy apart.
void proj_scalar(const Slot& W, const float* x, int ldx, int M, float* y, int ldy) {
  for (int n = 0; n < W.N; ++n) {
    const float b = W.bias ? load_dt(W.bias, n, W.bias_dt) : 0.0f;
    for (int t = 0; t < M; ++t) {
      float acc = 0.0f;
      for (int k = 0; k < W.K; ++k) acc = fmaf(x[(int64_t)t * ldx + k], deq(W, n, k), acc);
      y[(int64_t)t * ldy + n] = acc + b;
    }
  }
}

#define FTM_AVX512 __attribute__((target("avx512f,avx512bw,avx512vl,avx512dq")))

// K-major formats of the vector path
enum KFmt { kE4M3, kE5M2, kI8, kFP4, kF32, kBF16 };

// 16 weights [k, k + 16) of one K-major row, before the group scale.  E4M3
// comes out as value * 2^-8: its byte, widened to 16 bits as s.eeee.mmm <<
// 7, is the fp16 of value * 2^-8 (normals and subnormals alike), and the
// scale factor carries the 2^8; 0x7f / 0xff (NaN) are patched.  E5M2 is the
// high byte of an fp16.  INT8 offset-binary: b ^ 0x80 is b - 128 as int8.
template <int F>
FTM_AVX512 inline __m512 dec16(const char* row, int k) {
  if constexpr (F == kE4M3) {
    const __m256i b = _mm256_cvtepu8_epi16(_mm_loadu_si128((const __m128i*)(row + k)));
    const __m256i mag = _mm256_and_si256(b, _mm256_set1_epi16(0x7f));
    const __m256i h = _mm256_or_si256(_mm256_slli_epi16(_mm256_and_si256(b, _mm256_set1_epi16(0x80)), 8),
                                      _mm256_slli_epi16(mag, 7));
    const __mmask16 nan = _mm256_cmpeq_epi16_mask(mag, _mm256_set1_epi16(0x7f));
    return _mm512_mask_mov_ps(_mm512_cvtph_ps(h), nan, _mm512_set1_ps(__builtin_nanf("")));
  } else if constexpr (F == kE5M2) {
    const __m256i b = _mm256_cvtepu8_epi16(_mm_loadu_si128((const __m128i*)(row + k)));
    return _mm512_cvtph_ps(_mm256_slli_epi16(b, 8));
  } else if constexpr (F == kI8) {
    const __m128i b = _mm_xor_si128(_mm_loadu_si128((const __m128i*)(row + k)), _mm_set1_epi8((char)0x80));
    return _mm512_cvtepi32_ps(_mm512_cvtepi8_epi32(b));
  } else if constexpr (F == kFP4) {
    // 8 bytes hold elements k .. k + 15, low nibble first
    uint64_t b8;
    memcpy(&b8, row + k / 2, 8);
    const __m512i bytes = _mm512_cvtepu8_epi32(_mm_set_epi64x(0, (long long)b8));
    const __m512i pair = _mm512_permutexvar_epi32(_mm512_set_epi32(7, 7, 6, 6, 5, 5, 4, 4, 3, 3, 2, 2, 1, 1, 0, 0), bytes);
    const __m512i nib = _mm512_and_si512(
        _mm512_srlv_epi32(pair, _mm512_set_epi32(4, 0, 4, 0, 4, 0, 4, 0, 4, 0, 4, 0, 4, 0, 4, 0)), _mm512_set1_epi32(15));
    return _mm512_permutexvar_ps(nib, _mm512_loadu_ps(kE2M1));
  } else if constexpr (F == kF32) {
    return _mm512_loadu_ps((const float*)row + k);
  } else {
    const __m256i h = _mm256_loadu_si256((const __m256i*)((const uint16_t*)row + k));
    return _mm512_castsi512_ps(_mm512_slli_epi32(_mm512_cvtepu16_epi32(h), 16));
  }
}

template <int F>
constexpr int row_bytes(int K) {
  return F == kFP4 ? K / 2 : F == kF32 ? 4 * K : F == kBF16 ? 2 * K : K;
}

// The group scale of row n at column k (1 for the unscaled formats).
template <int F>
inline float group_scale(const Slot& W, int n, int k) {
  if constexpr (F == kE4M3 || F == kE5M2) {
    const int nkb = (W.K + W.group - 1) / W.group;
    return load_dt(W.s, (int64_t)(n / W.group) * nkb + k / W.group, W.s_dt);
  } else if constexpr (F == kI8) {
    return load_dt(W.s, (int64_t)n * (W.K / W.group) + k / W.group, W.s_dt);
  } else if constexpr (F == kFP4) {
    return e8m0_f((uint8_t)W.s[(int64_t)n * (W.K / 32) + k / 32]);
  } else {
    return 1.0f;
  }
}

// Rows [n0, n0 + R) for tokens [t0, t0 + tm), tm <= TB: R x TB accumulators,
// each decoded vector shared by the block's tokens, scales hoisted per group.
// Each weight is the reference's fp32 product value * scale rounded once;
// an E4M3 group whose scale times 2^8 could leave the exact range takes the
// two-multiply form.
template <int F, int R, int TB>
FTM_AVX512 void kmajor_rows(const Slot& W, int n0, const float* x, int ldx, int t0, int tm, float* y, int ldy) {
  const int K = W.K, K16 = K / 16 * 16;
  constexpr bool scaled = F == kE4M3 || F == kE5M2 || F == kI8 || F == kFP4;
  const int GS = F == kFP4 ? 32 : scaled ? W.group : K16;
  const char* rows[R];
  for (int r = 0; r < R; ++r) rows[r] = W.w + (int64_t)(n0 + r) * row_bytes<F>(K);
  const float* xr[TB];
  for (int i = 0; i < TB; ++i) xr[i] = x + (int64_t)(t0 + (i < tm ? i : 0)) * ldx;
  __m512 acc[R][TB];
  for (int r = 0; r < R; ++r)
    for (int i = 0; i < TB; ++i) acc[r][i] = _mm512_setzero_ps();
  for (int g0 = 0; g0 < K16; g0 += GS) {
    const int g1 = std::min(g0 + GS, K16);
    __m512 sv[R];
    bool wide = false;
    for (int r = 0; r < R; ++r) {
      float s = group_scale<F>(W, n0 + r, g0);
      if constexpr (F == kE4M3) {
        wide |= !(fabsf(s) < 0x1p100f);
        s *= 256.0f;
      }
      sv[r] = _mm512_set1_ps(s);
    }
    if (F == kE4M3 && wide) {
      for (int r = 0; r < R; ++r) sv[r] = _mm512_set1_ps(group_scale<F>(W, n0 + r, g0));
      for (int k = g0; k < g1; k += 16)
        for (int r = 0; r < R; ++r) {
          const __m512 w = _mm512_mul_ps(_mm512_mul_ps(dec16<F>(rows[r], k), _mm512_set1_ps(256.0f)), sv[r]);
          for (int i = 0; i < TB; ++i)
            if (i < tm) acc[r][i] = _mm512_fmadd_ps(_mm512_loadu_ps(xr[i] + k), w, acc[r][i]);
        }
      continue;
    }
    for (int k = g0; k < g1; k += 16) {
      __m512 xv[TB];
      for (int i = 0; i < TB; ++i) xv[i] = _mm512_loadu_ps(xr[i] + k);
      for (int r = 0; r < R; ++r) {
        __m512 w = dec16<F>(rows[r], k);
        if constexpr (scaled) w = _mm512_mul_ps(w, sv[r]);
        for (int i = 0; i < TB; ++i)
          if (i < tm) acc[r][i] = _mm512_fmadd_ps(xv[i], w, acc[r][i]);
      }
    }
  }
  for (int r = 0; r < R; ++r) {
    const int n = n0 + r;
    const float b = W.bias ? load_dt(W.bias, n, W.bias_dt) : 0.0f;
    for (int i = 0; i < tm; ++i) {
      float s = _mm512_reduce_add_ps(acc[r][i]);
      for (int k = K16; k < K; ++k) s = fmaf(xr[i][k], deq(W, n, k), s);
      y[(int64_t)(t0 + i) * ldy + n] = s + b;
    }
  }
}

// K-major projection: blocks of rows (4 for one or two tokens, 2 for up to
// four, else 1) against blocks of up to 8 tokens, so a decode step keeps
// several independent FMA chains in flight.
template <int F>
FTM_AVX512 void kmajor(const Slot& W, const float* x, int ldx, int M, float* y, int ldy) {
  const int N = W.N;
  int n = 0;
  if (M <= 2) {
    for (; n + 4 <= N; n += 4) {
      if (M == 1)
        kmajor_rows<F, 4, 1>(W, n, x, ldx, 0, 1, y, ldy);
      else
        kmajor_rows<F, 4, 2>(W, n, x, ldx, 0, 2, y, ldy);
    }
  } else if (M <= 4) {
    for (; n + 2 <= N; n += 2) kmajor_rows<F, 2, 4>(W, n, x, ldx, 0, M, y, ldy);
  }
  for (; n < N; ++n)
    for (int t0 = 0; t0 < M; t0 += 8) kmajor_rows<F, 1, 8>(W, n, x, ldx, t0, std::min(8, M - t0), y, ldy);
}

FTM_AVX512 void proj_kmajor_avx512(const Slot& W, const float* x, int ldx, int M, float* y, int ldy) {
  switch (W.fmt) {
    case FTM_FMT_FP8_BLOCK: return kmajor<kE4M3>(W, x, ldx, M, y, ldy);
    case FTM_FMT_FP8_E5M2_BLOCK: return kmajor<kE5M2>(W, x, ldx, M, y, ldy);
    case FTM_FMT_INT8_PACKED: return kmajor<kI8>(W, x, ldx, M, y, ldy);
    case FTM_FMT_MXFP4: return kmajor<kFP4>(W, x, ldx, M, y, ldy);
    case FTM_FMT_FP32: return kmajor<kF32>(W, x, ldx, M, y, ldy);
    default: return kmajor<kBF16>(W, x, ldx, M, y, ldy);
  }
}

// GPTQ, AVX-512 (N % 16 == 0, K % 8 == 0, group % 8 == 0; else the scalar
// path).  qweight is [K/8, N] with N contiguous, so the walk is row by row of
// packed words across all N columns -- one contiguous stream -- with the
// accumulators of up to two tokens in the output rows (L1-resident) and each
// group's scales and zero points unpacked once into fp32 rows.
FTM_AVX512 void proj_gptq_avx512(const Slot& W, const float* x, int ldx, int M, float* y, int ldy) {
  const int N = W.N, K = W.K, G = W.group;
  const uint32_t* qw = (const uint32_t*)W.w;
  const uint32_t* qz = (const uint32_t*)W.z;
  std::vector<float> sbuf((size_t)N), zbuf((size_t)N);
  for (int t0 = 0; t0 < M; t0 += 2) {
    const int tm = std::min(2, M - t0);
    float* y0 = y + (int64_t)t0 * ldy;
    float* y1 = y + (int64_t)(t0 + tm - 1) * ldy;  // == y0 for one token
    const float* x0 = x + (int64_t)t0 * ldx;
    const float* x1 = x + (int64_t)(t0 + tm - 1) * ldx;
    memset(y0, 0, sizeof(float) * N);
    if (tm == 2) memset(y1, 0, sizeof(float) * N);
    for (int g0 = 0; g0 < K; g0 += G) {
      const int g = g0 / G, g1 = std::min(g0 + G, K);
      for (int n = 0; n < N; ++n) {  // zero stored minus one
        sbuf[(size_t)n] = load_dt(W.s, (int64_t)g * N + n, W.s_dt);
        zbuf[(size_t)n] = (float)((int)((qz[(int64_t)g * (N / 8) + n / 8] >> (4 * (n & 7))) & 15u) + 1);
      }
      for (int k = g0; k < g1; k += 8) {
        const uint32_t* row = qw + (int64_t)(k / 8) * N;
        __m512 xb0[8], xb1[8];
        for (int j = 0; j < 8; ++j) {
          xb0[j] = _mm512_set1_ps(x0[k + j]);
          xb1[j] = _mm512_set1_ps(x1[k + j]);
        }
        for (int n0 = 0; n0 < N; n0 += 16) {
          const __m512i word = _mm512_loadu_si512((const void*)(row + n0));
          const __m512 s = _mm512_loadu_ps(&sbuf[(size_t)n0]), zp = _mm512_loadu_ps(&zbuf[(size_t)n0]);
          __m512 a0 = _mm512_loadu_ps(y0 + n0), a1 = _mm512_loadu_ps(y1 + n0);
#pragma GCC unroll 8
          for (int j = 0; j < 8; ++j) {
            const __m512i q = _mm512_and_si512(_mm512_srli_epi32(word, 4 * j), _mm512_set1_epi32(15));
            // s * (q - (z + 1)): the integer difference is exact in fp32, one rounding
            const __m512 w = _mm512_mul_ps(s, _mm512_sub_ps(_mm512_cvtepi32_ps(q), zp));
            a0 = _mm512_fmadd_ps(xb0[j], w, a0);
            if (tm == 2) a1 = _mm512_fmadd_ps(xb1[j], w, a1);
          }
          _mm512_storeu_ps(y0 + n0, a0);
          if (tm == 2) _mm512_storeu_ps(y1 + n0, a1);
        }
      }
    }
    if (W.bias)
      for (int i = 0; i < tm; ++i)
        for (int n = 0; n < N; ++n) y[(int64_t)(t0 + i) * ldy + n] += load_dt(W.bias, n, W.bias_dt);
  }
}

bool have_avx512() {
  static const bool ok = __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
                         __builtin_cpu_supports("avx512vl") && __builtin_cpu_supports("avx512dq");
  return ok;
}

void proj(const Slot& W, const float* x, int ldx, int M, float* y, int ldy, bool vec) {
  if (vec && W.fmt == FTM_FMT_GPTQ_INT4 && W.N % 16 == 0 && W.K % 8 == 0 && W.group % 8 == 0) {
    proj_gptq_avx512(W, x, ldx, M, y, ldy);
  } else if (vec && W.fmt != FTM_FMT_GPTQ_INT4 && W.K % 16 == 0 && (W.fmt != FTM_FMT_MXFP4 || W.K % 32 == 0) &&
             ((W.fmt != FTM_FMT_FP8_BLOCK && W.fmt != FTM_FMT_FP8_E5M2_BLOCK && W.fmt != FTM_FMT_INT8_PACKED) ||
              W.group % 16 == 0)) {  // a 16-wide vector never straddles two scale groups
    proj_kmajor_avx512(W, x, ldx, M, y, ldy);
  } else {
    proj_scalar(W, x, ldx, M, y, ldy);
  }
}

// ------------------------------------------------------------------ the layer half
struct Call {
  ftm_moe_layer L;
  const float* x;
  int T;
  const int32_t* ids;
  const float* w;
  const uint8_t* mask;
  int threads;
  int force_scalar;
  float* out;
};

// Experts [e0, e1) of the call, accumulated into out (zeroed by the caller).
void run_range(const Call& c, int e0, int e1, float* out, bool vec) {
  const ftm_moe_layer& L = c.L;
  const int H = L.hidden, I = L.inter, k = L.topk, T = c.T;
  std::vector<int> rows;
  std::vector<float> wts, xe, gu, h, y;
  for (int e = e0; e < e1; ++e) {
    if (c.mask != nullptr && c.mask[e] == 0) continue;
    rows.clear();
    wts.clear();
    for (int t = 0; t < T; ++t)  // token-major, then column: the reference's pair order within an expert
      for (int j = 0; j < k; ++j)
        if (c.ids[(int64_t)t * k + j] == e) {
          rows.push_back(t);
          wts.push_back(c.w[(int64_t)t * k + j]);
        }
    const int M = (int)rows.size();
    if (M == 0) continue;
    const int slot = L.slot_of_expert ? L.slot_of_expert[e] : e;
    const Slot W13 = slot_of(L.w13, slot), W2 = slot_of(L.w2, slot);
    xe.resize((size_t)M * H);
    for (int m = 0; m < M; ++m) memcpy(&xe[(size_t)m * H], c.x + (int64_t)rows[m] * H, sizeof(float) * H);
    gu.resize((size_t)M * 2 * I);
    proj(W13, xe.data(), H, M, gu.data(), 2 * I, vec);
    h.resize((size_t)M * I);
    for (int m = 0; m < M; ++m)
      for (int i = 0; i < I; ++i)
        h[(size_t)m * I + i] =
            act_f(L.act, gu[(size_t)m * 2 * I + i], gu[(size_t)m * 2 * I + I + i], L.swiglu_alpha, L.swiglu_limit);
    y.resize((size_t)M * H);
    proj(W2, h.data(), I, M, y.data(), H, vec);
    for (int m = 0; m < M; ++m) {
      float* o = out + (int64_t)rows[m] * H;
      const float wt = wts[m];
      const float* yr = &y[(size_t)m * H];
      for (int n = 0; n < H; ++n) o[n] += wt * yr[n];
    }
  }
}

int validate(const ftm_moe_layer* L, const float* x, int T, const int32_t* ids, const float* w, const float* out) {
  if (L == nullptr) return FTM_ERR_NULL;
  if (T < 0 || L->num_experts <= 0 || L->hidden <= 0 || L->inter <= 0 || L->topk <= 0) return FTM_ERR_DIM;
  if (T > 0 && (x == nullptr || ids == nullptr || w == nullptr || out == nullptr)) return FTM_ERR_NULL;
  if (L->w13.w == nullptr || L->w2.w == nullptr) return FTM_ERR_NULL;
  if (L->w13.N != 2 * L->inter || L->w13.K != L->hidden || L->w2.N != L->hidden || L->w2.K != L->inter)
    return FTM_ERR_DIM;
  if (L->w13.fmt != L->w2.fmt) return FTM_ERR_FORMAT;
  for (const ftm_proj* P : {&L->w13, &L->w2}) {
    switch (P->fmt) {
      case FTM_FMT_BF16:
      case FTM_FMT_FP32:
        break;
      case FTM_FMT_FP8_BLOCK:
      case FTM_FMT_FP8_E5M2_BLOCK:
      case FTM_FMT_INT8_PACKED:
        if (P->s == nullptr) return FTM_ERR_NULL;
        if (P->group <= 0 || (P->fmt == FTM_FMT_INT8_PACKED && P->K % P->group != 0)) return FTM_ERR_DIM;
        break;
      case FTM_FMT_GPTQ_INT4:
        if (P->s == nullptr || P->z == nullptr) return FTM_ERR_NULL;
        if (P->group <= 0 || P->K % 8 != 0 || P->N % 8 != 0) return FTM_ERR_DIM;
        break;
      case FTM_FMT_MXFP4:
        if (P->s == nullptr) return FTM_ERR_NULL;
        if (P->K % 32 != 0) return FTM_ERR_DIM;
        break;
      default:
        return FTM_ERR_FORMAT;
    }
  }
  if (L->act < FTM_ACT_SILU || L->act > FTM_ACT_SWIGLU_OAI) return FTM_ERR_FORMAT;
  return FTM_OK;
}

int run_call(const Call& c) {
  const int E = c.L.num_experts, H = c.L.hidden, T = c.T;
  if (T == 0) return FTM_OK;  // (out may be null then)
  memset(c.out, 0, sizeof(float) * (size_t)T * H);
  for (int64_t i = 0; i < (int64_t)T * c.L.topk; ++i)
    if (c.ids[i] >= E) return FTM_ERR_DIM;
  const bool vec = have_avx512() && !c.force_scalar;
  int threads = c.threads;
  if (threads <= 0) {
    const unsigned hw = std::thread::hardware_concurrency();
    threads = hw > 0 ? (int)hw : 1;
  }
  threads = std::max(1, std::min(threads, E));
  if (threads == 1) {
    run_range(c, 0, E, c.out, vec);
    return FTM_OK;
  }
  // contiguous expert ranges, private partial outputs, summed in thread order
  std::vector<std::vector<float>> part((size_t)threads);
  std::vector<std::thread> pool;
  const int base = E / threads, rem = E % threads;
  int b = 0;
  for (int p = 0; p < threads; ++p) {
    const int e1 = b + base + (p < rem ? 1 : 0);
    part[(size_t)p].assign((size_t)T * H, 0.0f);
    pool.emplace_back([&c, &part, p, b, e1, vec] { run_range(c, b, e1, part[(size_t)p].data(), vec); });
    b = e1;
  }
  for (auto& th : pool) th.join();
  for (int p = 0; p < threads; ++p) {
    const float* src = part[(size_t)p].data();
    for (size_t i = 0; i < (size_t)T * H; ++i) c.out[i] += src[i];
  }
  return FTM_OK;
}

// ------------------------------------------------------------------ async worker
// One job at a time on a persistent thread: submit waits for the slot to be
// free, hands the job over and returns its handle; wait blocks until that
// job has run and frees the slot.
class Worker {
 public:
  Worker() : th_([this] { loop(); }) {}
  ~Worker() {
    {
      std::lock_guard<std::mutex> lk(mu_);
      stop_ = true;
    }
    cv_.notify_all();
    th_.join();
  }
  int64_t submit(const Call& c) {
    std::unique_lock<std::mutex> lk(mu_);
    cv_.wait(lk, [this] { return state_ == kFree; });
    job_ = c;
    state_ = kQueued;
    handle_ = ++last_;
    const int64_t h = handle_;
    lk.unlock();
    cv_.notify_all();
    return h;
  }
  int wait(int64_t h) {
    std::unique_lock<std::mutex> lk(mu_);
    if (state_ == kFree || h != handle_) return FTM_ERR_HANDLE;
    cv_.wait(lk, [this] { return state_ == kDone; });
    const int rc = rc_;
    state_ = kFree;
    lk.unlock();
    cv_.notify_all();
    return rc;
  }

 private:
  enum State { kFree, kQueued, kRunning, kDone };
  void loop() {
    std::unique_lock<std::mutex> lk(mu_);
    for (;;) {
      cv_.wait(lk, [this] { return stop_ || state_ == kQueued; });
      if (state_ != kQueued) return;  // stopping with nothing queued
      state_ = kRunning;
      const Call c = job_;
      lk.unlock();
      const int rc = run_call(c);
      lk.lock();
      rc_ = rc;
      state_ = kDone;
      cv_.notify_all();
    }
  }
  std::mutex mu_;
  std::condition_variable cv_;
  Call job_{};
  State state_ = kFree;
  bool stop_ = false;
  int rc_ = 0;
  int64_t handle_ = 0, last_ = 0;
  std::thread th_;
};

Worker& worker() {
  static Worker w;
  return w;
}

Call make_call(const ftm_moe_layer* L, const float* x, int T, const int32_t* ids, const float* w, const uint8_t* mask,
               int threads, int force_scalar, float* out) {
  Call c;
  c.L = *L;
  c.x = x;
  c.T = T;
  c.ids = ids;
  c.w = w;
  c.mask = mask;
  c.threads = threads;
  c.force_scalar = force_scalar;
  c.out = out;
  return c;
}

}  // namespace

extern "C" {

int ftm_cpu_moe_forward(const ftm_moe_layer* layer, const float* x, int32_t num_tokens, const int32_t* topk_ids,
                        const float* topk_w, const uint8_t* expert_mask, int32_t threads, int32_t force_scalar,
                        float* out) {
  const int rc = validate(layer, x, num_tokens, topk_ids, topk_w, out);
  if (rc != FTM_OK) return rc;
  return run_call(make_call(layer, x, num_tokens, topk_ids, topk_w, expert_mask, threads, force_scalar, out));
}

int64_t ftm_cpu_moe_submit(const ftm_moe_layer* layer, const float* x, int32_t num_tokens, const int32_t* topk_ids,
                           const float* topk_w, const uint8_t* expert_mask, int32_t threads, float* out) {
  const int rc = validate(layer, x, num_tokens, topk_ids, topk_w, out);
  if (rc != FTM_OK) return rc;
  return worker().submit(make_call(layer, x, num_tokens, topk_ids, topk_w, expert_mask, threads, 0, out));
}

int ftm_cpu_moe_wait(int64_t handle) { return worker().wait(handle); }

int ftm_cpu_avx512(void) { return have_avx512() ? 1 : 0; }

}  // extern "C"
