// ftm_device.h -- gfx950 device building blocks for the fused quantized MoE layer.
//
// Everything here is written for CDNA4 wave64 and the gfx950 bf16 matrix core
// (v_mfma_f32_16x16x32_bf16).  Quantized weights are decoded in registers to
// their *exact* bf16 code values (no scale, no rounding); per-group scales and
// zero points are applied in fp32 to the MFMA partial sums, so the arithmetic
// equals an fp32 dot product of the reference's dequantized weights up to fp32
// summation order (the reference fused kernels also accumulate in fp32:
// python/freetoken/kernel/triton/fused_fp8_linear.py:69-89,
// gptq_fused_linear.py:290-318, fused_int8_linear.py:78-103,
// fused_mxfp4_linear.py:307-343).
//
// MFMA 16x16x32 bf16 operand layout (lane l of the wave):
//   A[i][k]: i = l % 16, k = 8*(l/16) + e   (e = element 0..7 of the lane's bf16x8)
//   B[k][j]: j = l % 16, k = 8*(l/16) + e
//   D[i][j]: j = l % 16, i = 4*(l/16) + r   (r = 0..3 of the lane's f32x4)
// Any permutation of k applied identically to A and B leaves the product
// unchanged, which the loaders below use to keep every weight load a single
// coalesced 16-byte access per lane.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ftmoe.h"

namespace ftm {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;
constexpr int kBlock = 256;  // 4 waves per workgroup everywhere

// ---------------------------------------------------------------- scalars

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

__device__ __forceinline__ float f16_to_f32(uint16_t bits) {
  return (float)__builtin_bit_cast(_Float16, bits);
}

// Round-to-nearest-even fp32 -> bf16 (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  bf16x2 v = __builtin_convertvector((f32x2){f, 0.0f}, bf16x2);
  return (uint16_t)(__builtin_bit_cast(uint32_t, v) & 0xffffu);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  bf16x2 v = __builtin_convertvector((f32x2){lo, hi}, bf16x2);
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// Round to the given storage dtype and back (the value a tensor of that dtype holds).
__device__ __forceinline__ float round_to(float v, int dt) {
  if (dt == FTM_DT_BF16) return bf16_to_f32(f32_to_bf16(v));
  if (dt == FTM_DT_F16) return f16_to_f32(f32_to_f16(v));
  return v;
}

__device__ __forceinline__ float load_scalar(const void* p, int64_t i, int dt) {
  if (dt == FTM_DT_F32) return ((const float*)p)[i];
  if (dt == FTM_DT_F16) return f16_to_f32(((const uint16_t*)p)[i]);
  return bf16_to_f32(((const uint16_t*)p)[i]);
}

__device__ __forceinline__ void store_scalar(void* p, int64_t i, int dt, float v) {
  if (dt == FTM_DT_F32) ((float*)p)[i] = v;
  else if (dt == FTM_DT_F16) ((uint16_t*)p)[i] = f32_to_f16(v);
  else ((uint16_t*)p)[i] = f32_to_bf16(v);
}

__device__ __forceinline__ int dt_size(int dt) { return dt == FTM_DT_F32 ? 4 : 2; }

// e8m0 shared exponent -> fp32 2^(s-127), bit-exact with torch.exp2(s - 127)
// (python/freetoken/kernel/triton/mxfp4_linear.py:74): s = 0 gives the fp32
// subnormal 2^-127, s = 255 gives +inf.
__device__ __forceinline__ float e8m0_to_f32(uint32_t s) {
  return __uint_as_float(s == 0 ? 0x00400000u : (s << 23));
}

__device__ __forceinline__ f32x4 mfma_bf16(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

__device__ __forceinline__ float wave_sum(float v) {
  v += __shfl_xor(v, 32);
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 8);
  v += __shfl_xor(v, 4);
  v += __shfl_xor(v, 2);
  v += __shfl_xor(v, 1);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, __shfl_xor(v, 32));
  v = fmaxf(v, __shfl_xor(v, 16));
  v = fmaxf(v, __shfl_xor(v, 8));
  v = fmaxf(v, __shfl_xor(v, 4));
  v = fmaxf(v, __shfl_xor(v, 2));
  v = fmaxf(v, __shfl_xor(v, 1));
  return v;
}

// ---------------------------------------------------------------- B decoders
// Each returns the 8 bf16 values (as 4 packed dwords) one lane feeds to one MFMA.

// 8 e4m3fn bytes (two dwords) -> 8 exact bf16 values.  OCP e4m3 values are all
// representable in bf16, so scale 1.0 makes the conversion exact.
__device__ __forceinline__ u32x4 fp8x8_to_bf16(uint32_t w0, uint32_t w1) {
  u32x4 r;
  r.x = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w0, 1.0f, false));
  r.y = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w0, 1.0f, true));
  r.z = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w1, 1.0f, false));
  r.w = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w1, 1.0f, true));
  return r;
}

// 8 offset-binary int8 bytes (value = byte - 128, compressed-tensors
// pack-quantized, int8_packed_linear.py:74-93) -> 8 exact bf16 values.
__device__ __forceinline__ uint32_t u8pair_to_bf16(uint32_t w, int hi) {
  uint32_t b0 = (w >> (16 * hi)) & 0xffu, b1 = (w >> (16 * hi + 8)) & 0xffu;
  return pack_bf16x2((float)b0 - 128.0f, (float)b1 - 128.0f);
}
__device__ __forceinline__ u32x4 i8x8_to_bf16(uint32_t w0, uint32_t w1) {
  u32x4 r;
  r.x = u8pair_to_bf16(w0, 0);
  r.y = u8pair_to_bf16(w0, 1);
  r.z = u8pair_to_bf16(w1, 0);
  r.w = u8pair_to_bf16(w1, 1);
  return r;
}

// 8 e2m1 nibbles (one dword, low nibble = even element) scaled by the block's
// e8m0 factor -> 8 bf16.  LUT * 2^e is exact in bf16 for every e8m0 byte >= 2.
__device__ __forceinline__ u32x4 fp4x8_to_bf16(uint32_t w, float scale) {
  u32x4 r;
  r.x = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4((int)w, scale, 0));
  r.y = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4((int)w, scale, 1));
  r.z = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4((int)w, scale, 2));
  r.w = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4((int)w, scale, 3));
  return r;
}

// One GPTQ int32 word (8 nibbles along K, LSB first, gptq_linear.py:39-52) ->
// bf16 values 128 + q in the element order [q0,q4,q1,q5,q2,q6,q3,q7].
// 0x4300 is bf16 128.0 and the nibble lands in its low mantissa bits, so each
// value is exactly 128 + q; the 128 and the zero point are removed afterwards
// with one fp32 correction per group.
__device__ __forceinline__ u32x4 gptq_word_to_bf16(uint32_t w) {
  u32x4 r;
  r.x = (w & 0x000f000fu) | 0x43004300u;
  r.y = ((w >> 4) & 0x000f000fu) | 0x43004300u;
  r.z = ((w >> 8) & 0x000f000fu) | 0x43004300u;
  r.w = ((w >> 12) & 0x000f000fu) | 0x43004300u;
  return r;
}

// Reorder 8 bf16 activations x0..x7 to [x0,x4,x1,x5,x2,x6,x3,x7] (the GPTQ
// element order above).
__device__ __forceinline__ u32x4 perm_gptq(u32x4 d) {
  u32x4 r;
  r.x = __builtin_amdgcn_perm(d.z, d.x, 0x05040100u);  // (x0, x4)
  r.y = __builtin_amdgcn_perm(d.z, d.x, 0x07060302u);  // (x1, x5)
  r.z = __builtin_amdgcn_perm(d.w, d.y, 0x05040100u);  // (x2, x6)
  r.w = __builtin_amdgcn_perm(d.w, d.y, 0x07060302u);  // (x3, x7)
  return r;
}

// ---------------------------------------------------------------- A operand
// Each lane owns one A row (its l % 16) of the current 16-row M tile.
struct ARow {
  const char* p;  // row base, NULL -> zero row
  float mul;      // multiplier applied before rounding (router weight on input), 1 = none
  int dt;         // FTM_DT_* of the row
};

// 8 consecutive activations starting at element kk, as bf16 hi (+ lo remainder
// when the source is fp32/fp16, so hi + lo carries 16 significant bits).
template <bool SPLIT>
__device__ __forceinline__ void load_a8(const ARow& a, int kk, u32x4& hi, u32x4& lo) {
  if (a.p == nullptr) {
    hi = (u32x4){0, 0, 0, 0};
    lo = hi;
    return;
  }
  if (a.dt == FTM_DT_BF16 && a.mul == 1.0f) {
    hi = *(const u32x4*)(a.p + 2 * (int64_t)kk);
    lo = (u32x4){0, 0, 0, 0};
    return;
  }
  float v[8];
  if (a.dt == FTM_DT_F32) {
    u32x4 q0 = *(const u32x4*)(a.p + 4 * (int64_t)kk);
    u32x4 q1 = *(const u32x4*)(a.p + 4 * (int64_t)kk + 16);
    v[0] = __uint_as_float(q0.x); v[1] = __uint_as_float(q0.y);
    v[2] = __uint_as_float(q0.z); v[3] = __uint_as_float(q0.w);
    v[4] = __uint_as_float(q1.x); v[5] = __uint_as_float(q1.y);
    v[6] = __uint_as_float(q1.z); v[7] = __uint_as_float(q1.w);
  } else {
    u32x4 q = *(const u32x4*)(a.p + 2 * (int64_t)kk);
    uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (a.dt == FTM_DT_BF16) {
        v[2 * i] = bf16_to_f32(w[i] & 0xffffu);
        v[2 * i + 1] = bf16_to_f32(w[i] >> 16);
      } else {
        v[2 * i] = f16_to_f32((uint16_t)(w[i] & 0xffffu));
        v[2 * i + 1] = f16_to_f32((uint16_t)(w[i] >> 16));
      }
    }
  }
  if (a.mul != 1.0f) {
    // x * router_weight rounded to the activation dtype (fused_moe.py:139-140).
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = round_to(v[i] * a.mul, a.dt);
  }
  uint32_t h[4], l[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    h[i] = pack_bf16x2(v[2 * i], v[2 * i + 1]);
    if (SPLIT) {
      float r0 = v[2 * i] - bf16_to_f32(h[i] & 0xffffu);
      float r1 = v[2 * i + 1] - bf16_to_f32(h[i] >> 16);
      l[i] = pack_bf16x2(r0, r1);
    } else {
      l[i] = 0;
    }
  }
  hi = (u32x4){h[0], h[1], h[2], h[3]};
  lo = (u32x4){l[0], l[1], l[2], l[3]};
}

// Sum of the 8 activations a lane feeds for element offset kk (fp32), used by
// the GPTQ zero-point correction.
__device__ __forceinline__ float sum_a8(u32x4 hi, u32x4 lo) {
  float s = 0.0f;
  uint32_t h[4] = {hi.x, hi.y, hi.z, hi.w};
  uint32_t l[4] = {lo.x, lo.y, lo.z, lo.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    s += bf16_to_f32(h[i] & 0xffffu) + bf16_to_f32(l[i] & 0xffffu);
    s += bf16_to_f32(h[i] >> 16) + bf16_to_f32(l[i] >> 16);
  }
  return s;
}

// ---------------------------------------------------------------- projection view
// One slot of one projection, resolved to raw pointers.
struct ProjSlot {
  const char* w;
  const char* s;
  const char* z;
  const char* bias;
  int fmt, s_dt, bias_dt, group, N, K;
};

__device__ __forceinline__ ProjSlot proj_slot(const ftm_proj& P, int slot) {
  ProjSlot v;
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

// ---------------------------------------------------------------- K-major engine
// Formats whose weight rows are contiguous along K: FP8 block, INT8 packed,
// MXFP4, BF16.  One "wave-load" = every lane loading 16 bytes of its row
// (row = col0 + l%16, 4 lane groups side by side along K).
template <int FMT>
struct KMajor;

template <>
struct KMajor<FTM_FMT_FP8_BLOCK> {
  static constexpr int kLaneK = 16, kLoadK = 64, kMfma = 2, kChunk = 8;
  static constexpr bool kPostScale = true;
  __device__ static int64_t row_bytes(int K) { return K; }
  __device__ static int64_t elem_off(int kk) { return kk; }
};
template <>
struct KMajor<FTM_FMT_INT8_PACKED> {
  static constexpr int kLaneK = 16, kLoadK = 64, kMfma = 2, kChunk = 8;
  static constexpr bool kPostScale = true;
  __device__ static int64_t row_bytes(int K) { return K; }
  __device__ static int64_t elem_off(int kk) { return kk; }
};
template <>
struct KMajor<FTM_FMT_MXFP4> {
  static constexpr int kLaneK = 32, kLoadK = 128, kMfma = 4, kChunk = 4;
  static constexpr bool kPostScale = false;
  __device__ static int64_t row_bytes(int K) { return K / 2; }
  __device__ static int64_t elem_off(int kk) { return kk / 2; }
};
template <>
struct KMajor<FTM_FMT_BF16> {
  static constexpr int kLaneK = 8, kLoadK = 32, kMfma = 1, kChunk = 8;
  static constexpr bool kPostScale = false;
  __device__ static int64_t row_bytes(int K) { return 2 * (int64_t)K; }
  __device__ static int64_t elem_off(int kk) { return 2 * (int64_t)kk; }
};

// Number of wave-loads covering K for a format.
template <int FMT>
__device__ __forceinline__ int kmajor_loads(int K) {
  return (K + KMajor<FMT>::kLoadK - 1) / KMajor<FMT>::kLoadK;
}

// Wave-loads covering K for any format (GPTQ: 32 k per wave-load).
template <int FMT>
__device__ __forceinline__ int fmt_loads(int K) {
  if constexpr (FMT == FTM_FMT_GPTQ_INT4) {
    return (K + 31) / 32;
  } else {
    return kmajor_loads<FMT>(K);
  }
}

// acc[r] += sum over wave-loads [L_lo, L_hi) of A(16 x K) * W(rows col0[r]..+16)^T.
// Rows >= N and k >= K read as zero.  For post-scaled formats the partial sum of
// each quantisation group is multiplied by the group's fp32 scale before it
// joins acc (FP8: one scale per 128x128 block; INT8: one per (row, group)).
template <int FMT, int NR, bool SPLIT>
__device__ __forceinline__ void wave_gemm_kmajor(const ProjSlot& W, const int (&col0)[NR], int L_lo,
                                                 int L_hi, const ARow& ar, f32x4 (&acc)[NR]) {
  using F = KMajor<FMT>;
  constexpr int CH = SPLIT ? (F::kChunk / 2 > 0 ? F::kChunk / 2 : 1) : F::kChunk;
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4;
  const int rl = lane & 15;
  const int K = W.K;
  const int64_t rb = F::row_bytes(K);

  const char* wrow[NR];
  const char* srow[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const int n = col0[r] + rl;
    wrow[r] = (n < W.N) ? W.w + (int64_t)n * rb : nullptr;
    srow[r] = nullptr;
    if (FMT == FTM_FMT_FP8_BLOCK) {
      // scale row of the 128-row block holding this 16-row tile
      const int nkb = (K + W.group - 1) / W.group;
      srow[r] = (col0[r] < W.N) ? W.s + (int64_t)(col0[r] / W.group) * nkb * (W.s_dt == FTM_DT_F32 ? 4 : 2)
                                : nullptr;
    } else if (FMT == FTM_FMT_INT8_PACKED) {
      const int ng = K / W.group;
      srow[r] = (n < W.N) ? W.s + (int64_t)n * ng * (W.s_dt == FTM_DT_F32 ? 4 : 2) : nullptr;
    } else if (FMT == FTM_FMT_MXFP4) {
      srow[r] = (n < W.N) ? W.s + (int64_t)n * (K / 32) : nullptr;
    }
  }

  f32x4 tmp[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) tmp[r] = (f32x4){0.f, 0.f, 0.f, 0.f};

  for (int Lc = L_lo; Lc < L_hi; Lc += CH) {
    u32x4 raw[NR][CH];
    float msc[NR][CH];
    u32x4 ahi[CH][F::kMfma], alo[CH][F::kMfma];
#pragma unroll
    for (int b = 0; b < CH; ++b) {
      const int L = Lc + b;
      const int kk = L * F::kLoadK + F::kLaneK * g;
      const bool kok = (L < L_hi) && (kk < K);
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        raw[r][b] = (kok && wrow[r]) ? *(const u32x4*)(wrow[r] + F::elem_off(kk)) : (u32x4){0, 0, 0, 0};
        if (FMT == FTM_FMT_MXFP4)
          msc[r][b] = (kok && srow[r]) ? e8m0_to_f32((uint8_t)srow[r][kk / 32]) : 0.0f;
      }
#pragma unroll
      for (int q = 0; q < F::kMfma; ++q) {
        if (kok) {
          load_a8<SPLIT>(ar, kk + 8 * q, ahi[b][q], alo[b][q]);
        } else {
          ahi[b][q] = (u32x4){0, 0, 0, 0};
          alo[b][q] = ahi[b][q];
        }
      }
    }
#pragma unroll
    for (int b = 0; b < CH; ++b) {
      const int L = Lc + b;
      if (L >= L_hi) break;
#pragma unroll
      for (int q = 0; q < F::kMfma; ++q) {
#pragma unroll
        for (int r = 0; r < NR; ++r) {
          u32x4 bq;
          if (FMT == FTM_FMT_FP8_BLOCK) {
            bq = q == 0 ? fp8x8_to_bf16(raw[r][b].x, raw[r][b].y) : fp8x8_to_bf16(raw[r][b].z, raw[r][b].w);
          } else if (FMT == FTM_FMT_INT8_PACKED) {
            bq = q == 0 ? i8x8_to_bf16(raw[r][b].x, raw[r][b].y) : i8x8_to_bf16(raw[r][b].z, raw[r][b].w);
          } else if (FMT == FTM_FMT_MXFP4) {
            const uint32_t wq = q == 0 ? raw[r][b].x : q == 1 ? raw[r][b].y : q == 2 ? raw[r][b].z : raw[r][b].w;
            bq = fp4x8_to_bf16(wq, msc[r][b]);
          } else {
            bq = raw[r][b];
          }
          tmp[r] = mfma_bf16(ahi[b][q], bq, tmp[r]);
          if (SPLIT) tmp[r] = mfma_bf16(alo[b][q], bq, tmp[r]);
        }
      }
      if (F::kPostScale) {
        const int k_first = L * F::kLoadK;
        const int grp = k_first / W.group;
        const bool last = (L + 1 == L_hi) || (((L + 1) * F::kLoadK) / W.group != grp);
        if (last) {
#pragma unroll
          for (int r = 0; r < NR; ++r) {
            // FP8: one scale for the whole 16-row tile; INT8: the scale of row
            // col0 + l%16, which is exactly the D column this lane holds.
            const float s = (srow[r] != nullptr) ? load_scalar(srow[r], grp, W.s_dt) : 0.0f;
            acc[r] += tmp[r] * s;
            tmp[r] = (f32x4){0.f, 0.f, 0.f, 0.f};
          }
        }
      }
    }
  }
  if (!F::kPostScale) {
#pragma unroll
    for (int r = 0; r < NR; ++r) acc[r] += tmp[r];
  }
}

// ---------------------------------------------------------------- GPTQ engine
// qweight [K/8, N] int32 is contiguous along N.  One wave-load: lane group g
// reads packed row 4L+g (k = 32L + 8g .. +8) for columns col0 + 4*(l%16) + c,
// c = 0..3 (16 bytes).  A wave therefore produces 64 columns as 4 interleaved
// MFMA sub-tiles: sub-tile c, MFMA column j <-> output column col0 + 4j + c.
// Per quantisation group the zero point and the +128 decode bias are removed
// with  acc += s * (tmp - (128 + zp) * sum_k x_k)  (gptq_linear.py:88-99).
template <int NR, bool SPLIT>
__device__ __forceinline__ void wave_gemm_gptq(const ProjSlot& W, const int (&col0)[NR], int L_lo, int L_hi,
                                               const ARow& ar, f32x4 (&acc)[NR][4]) {
  constexpr int CH = 4;
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4;
  const int rl = lane & 15;
  const int N = W.N;
  const int K = W.K;
  const int G = W.group;
  const int ngroups = (K + G - 1) / G;

  f32x4 tmp[NR][4];
#pragma unroll
  for (int r = 0; r < NR; ++r)
#pragma unroll
    for (int c = 0; c < 4; ++c) tmp[r][c] = (f32x4){0.f, 0.f, 0.f, 0.f};
  float xs = 0.0f;  // this lane's partial sum of x over the current group

  for (int Lc = L_lo; Lc < L_hi; Lc += CH) {
    u32x4 raw[NR][CH];
    u32x4 ahi[CH], alo[CH];
#pragma unroll
    for (int b = 0; b < CH; ++b) {
      const int L = Lc + b;
      const int prow = 4 * L + g;
      const bool kok = (L < L_hi) && (8 * prow < K);
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        const int n = col0[r] + 4 * rl;
        raw[r][b] = (kok && n < N) ? *(const u32x4*)(W.w + ((int64_t)prow * N + n) * 4) : (u32x4){0, 0, 0, 0};
      }
      if (kok) {
        u32x4 h, l;
        load_a8<SPLIT>(ar, 8 * prow, h, l);
        ahi[b] = perm_gptq(h);
        alo[b] = perm_gptq(l);
      } else {
        ahi[b] = (u32x4){0, 0, 0, 0};
        alo[b] = ahi[b];
      }
    }
#pragma unroll
    for (int b = 0; b < CH; ++b) {
      const int L = Lc + b;
      if (L >= L_hi) break;
      xs += sum_a8(ahi[b], alo[b]);
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        const uint32_t wv[4] = {raw[r][b].x, raw[r][b].y, raw[r][b].z, raw[r][b].w};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const u32x4 bq = gptq_word_to_bf16(wv[c]);
          tmp[r][c] = mfma_bf16(ahi[b], bq, tmp[r][c]);
          if (SPLIT) tmp[r][c] = mfma_bf16(alo[b], bq, tmp[r][c]);
        }
      }
      const int grp = (32 * L) / G;
      const bool last = (L + 1 == L_hi) || ((32 * (L + 1)) / G != grp);
      if (last) {
        // Row sums of x over this group: reduce the 4 lane groups (same l%16).
        float sx = xs;
        sx += __shfl_xor(sx, 16);
        sx += __shfl_xor(sx, 32);
        // D row i = 4*(l/16) + rr lives at lane i's sum.
        float sxr[4];
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) sxr[rr] = __shfl(sx, 4 * g + rr);
        xs = 0.0f;
        if (grp < ngroups) {
#pragma unroll
          for (int r = 0; r < NR; ++r) {
            const int nb = col0[r] + 4 * rl;  // columns nb + c
            float sc[4], zp[4];
            if (nb < N) {
              const uint32_t zw = *(const uint32_t*)(W.z + ((int64_t)grp * (N / 8) + nb / 8) * 4);
#pragma unroll
              for (int c = 0; c < 4; ++c) {
                sc[c] = load_scalar(W.s, (int64_t)grp * N + nb + c, W.s_dt);
                zp[c] = (float)(((zw >> (4 * ((nb + c) & 7))) & 0xfu) + 1u);
              }
            } else {
#pragma unroll
              for (int c = 0; c < 4; ++c) { sc[c] = 0.0f; zp[c] = 0.0f; }
            }
#pragma unroll
            for (int c = 0; c < 4; ++c) {
              f32x4 corr;
              corr.x = tmp[r][c].x - (128.0f + zp[c]) * sxr[0];
              corr.y = tmp[r][c].y - (128.0f + zp[c]) * sxr[1];
              corr.z = tmp[r][c].z - (128.0f + zp[c]) * sxr[2];
              corr.w = tmp[r][c].w - (128.0f + zp[c]) * sxr[3];
              acc[r][c] += corr * sc[c];
              tmp[r][c] = (f32x4){0.f, 0.f, 0.f, 0.f};
            }
          }
        }
      }
    }
  }
}

}  // namespace ftm
