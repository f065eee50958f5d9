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
typedef int i32x8 __attribute__((ext_vector_type(8)));  // operands of the scaled (f8f6f4) MFMAs

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

// e^x in fp32 for the routing arithmetic (softmax numerators, the gpt-oss
// top-k softmax, the shared expert's sigmoid gate).  Every step is one IEEE
// operation with a fixed operand order, so a host restatement that performs
// the same steps (fmaf, rintf, multiplies; no contraction) returns the same
// bits:
//   * Cody & Waite range reduction, x = n ln2 + r with n = rint(x log2 e),
//     ln 2 split into the float nearest it and the float nearest the
//     remainder, each product folded in by one fused multiply-add;
//   * e^r on |r| <= ln2 / 2 by its Taylor polynomial of degree 7 in Horner
//     form (truncation below 2^-27 relative);
//   * 2^n applied as two exact powers of two (the second product rounds
//     once, into the subnormal range where the result lies there).
// x is clamped to [-104, 89] first (e^-104 is below half the smallest
// subnormal, e^89 above FLT_MAX), so NaN gives 0.  Measured over every float
// in [-104, 88.7] with a normal result: at most 0.94 ulp from e^x.
__device__ __forceinline__ float ftm_expf(float x) {
#pragma clang fp contract(off)
  const float xc = fminf(fmaxf(x, -104.0f), 89.0f);
  const float n = rintf(xc * 0x1.715476p+0f);
  float r = fmaf(n, -0x1.62e43p-1f, xc);
  r = fmaf(n, 0x1.05c61p-29f, r);
  float p = 0x1.a01a02p-13f;    // 1/7!
  p = fmaf(p, r, 0x1.6c16c2p-10f);  // 1/6!
  p = fmaf(p, r, 0x1.111112p-7f);   // 1/5!
  p = fmaf(p, r, 0x1.555556p-5f);   // 1/4!
  p = fmaf(p, r, 0x1.555556p-3f);   // 1/3!
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  const int ni = (int)n, h = ni >> 1;
  // the last product as fmaf(., ., +0): an explicit fused op leaves the
  // caller's sums nothing to contract into an FMA
  return fmaf(p * __uint_as_float((uint32_t)(h + 127) << 23), __uint_as_float((uint32_t)(ni - h + 127) << 23), 0.0f);
}

// The router's sigmoid gate weight 1 / (1 + e^-z), on ftm_expf.
__device__ __forceinline__ float ftm_sigmoidf(float z) { return 1.0f / (1.0f + ftm_expf(-z)); }

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

// Raw bits of element i of a scalar array (2- or 4-byte dtype) and their
// value, for loads issued ahead of a kernel's weight stream but used only in
// its epilogue: vector loads complete in order, so converting right after the
// load would wait for every weight load issued before it.  opaque_bits at the
// point of use pins the conversion (and the wait) there; without it the
// compiler may hoist a loop-invariant conversion back up to the load.
__device__ __forceinline__ uint32_t load_bits(const void* p, int64_t i, int dt) {
  return dt == FTM_DT_F32 ? ((const uint32_t*)p)[i] : (uint32_t)((const uint16_t*)p)[i];
}
__device__ __forceinline__ float bits_to_f32(uint32_t b, int dt) {
  if (dt == FTM_DT_F32) return __uint_as_float(b);
  if (dt == FTM_DT_F16) return f16_to_f32((uint16_t)b);
  return __uint_as_float(b << 16);
}
__device__ __forceinline__ uint32_t opaque_bits(uint32_t b) {
  asm volatile("" : "+v"(b));
  return b;
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

// s_waitcnt vmcnt(n), other counters untouched (gfx9 encoding), n < 64:
// the oldest vector-memory loads of this wave have landed, up to n are still
// in flight (they complete in issue order).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xf << 8));
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

// Wave64 reductions on DPP inside each 16-lane row (xor 1, xor 2, half-row
// mirror, row mirror) and v_readlane across the four rows: no LDS round trip,
// unlike __shfl_xor.  Every lane returns the result.  wave_sum above keeps the
// xor-32..1 order that the router's bit-exact contract fixes; wave_sum_dpp
// associates as quad -> 8 -> 16 lanes -> (row0 + row1) + (row2 + row3).
constexpr int kDppXor1 = 0xB1;        // quad_perm [1, 0, 3, 2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2, 3, 0, 1]
constexpr int kDppHalfMirror = 0x141; // lane i <- 7 - i within 8
constexpr int kDppMirror = 0x140;     // lane i <- 15 - i within 16

template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(dpp_i<CTRL>(__float_as_int(v)));
}
__device__ __forceinline__ float readlane_f(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

__device__ __forceinline__ float wave_max_dpp(float v) {
  v = fmaxf(v, dpp_f<kDppXor1>(v));
  v = fmaxf(v, dpp_f<kDppXor2>(v));
  v = fmaxf(v, dpp_f<kDppHalfMirror>(v));
  v = fmaxf(v, dpp_f<kDppMirror>(v));
  return fmaxf(fmaxf(readlane_f(v, 0), readlane_f(v, 16)), fmaxf(readlane_f(v, 32), readlane_f(v, 48)));
}

__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += dpp_f<kDppXor1>(v);
  v += dpp_f<kDppXor2>(v);
  v += dpp_f<kDppHalfMirror>(v);
  v += dpp_f<kDppMirror>(v);
  return (readlane_f(v, 0) + readlane_f(v, 16)) + (readlane_f(v, 32) + readlane_f(v, 48));
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
// The same with the mask and the 128.0 pattern in VGPRs (gq_decode_consts):
// each value is one v_and_or_b32 (after a shift) instead of an AND and an OR
// with literal operands -- a VOP3 on this target takes no literal.  7 VALU
// per word instead of 11.
struct GqConsts {
  uint32_t m, c;
};
__device__ __forceinline__ GqConsts gq_decode_consts() {
  GqConsts k;
  asm("v_mov_b32 %0, 0xf000f" : "=v"(k.m));
  asm("v_mov_b32 %0, 0x43004300" : "=v"(k.c));
  return k;
}
__device__ __forceinline__ u32x4 gptq_word_to_bf16(uint32_t w, GqConsts k) {
  u32x4 r;
  r.x = (w & k.m) | k.c;
  r.y = ((w >> 4) & k.m) | k.c;
  r.z = ((w >> 8) & k.m) | k.c;
  r.w = ((w >> 12) & k.m) | k.c;
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

// ---------------------------------------------------------------- buffer loads
// Raw buffer loads return 0 for any byte offset at or past the descriptor's
// size, so padding rows, rows past N and K tails are expressed as an
// out-of-range offset instead of a branch: every load is issued
// unconditionally and the waves keep many loads in flight.
typedef __amdgpu_buffer_rsrc_t Rsrc;
constexpr uint32_t kOOB = 0x80000000u;

__device__ __forceinline__ Rsrc make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ u32x4 bload16(Rsrc r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}
__device__ __forceinline__ uint32_t bload4(Rsrc r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
// XCD-aware order: consecutive workgroups go to different XCDs (round robin),
// so workgroup b runs item xcd * per + min(xcd, rem) + b / 8, which keeps
// runs of consecutive items on one XCD's L2 (a bijection on [0, G)).
__device__ __forceinline__ int xcd_item(int b, int G) {
  const int xcd = b & 7, per = G >> 3, rem = G & 7;
  return xcd * per + (xcd < rem ? xcd : rem) + (b >> 3);
}

// Device-coherent accesses (the SC1 cache-policy bit): the load misses every
// cache another XCD's writes could leave stale, the store is written through
// to where every XCD reads it.  Data one workgroup hands to another inside a
// launch travels this way; a producer waits for its stores' acknowledgement
// (s_waitcnt) before its arrival, a consumer loads after seeing the count.
// An agent-scope fence would write back (release: buffer_wbl2) or invalidate
// (acquire: buffer_inv) the whole L2 of the XCD instead, once per workgroup.
// This ordering is a property of the gfx942 / gfx950 memory system (the SC1
// bit's write-through and miss-on-load, vector memory returning in order for
// one wave), not of the HIP memory model: the relaxed arrival atomic itself
// orders nothing.  Other targets would need the release / acquire pair on the
// arrival counter, so the build refuses them.
#if defined(__HIP_DEVICE_COMPILE__) && !defined(__gfx942__) && !defined(__gfx950__)
#error "the fence-free cross-workgroup hand-over (store_dev / load_dev) assumes gfx942 / gfx950 SC1 coherence"
#endif
constexpr int kAuxDev = 16;
__device__ __forceinline__ uint32_t bload4_dev(Rsrc r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, kAuxDev);
}
template <class V>
__device__ __forceinline__ void store_dev(V* p, V v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <class V>
__device__ __forceinline__ V load_dev(const V* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t bload2(Rsrc r, uint32_t off) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}
__device__ __forceinline__ uint32_t bload1(Rsrc r, uint32_t off) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(r, off, 0, 0);
}
// Scalars are fetched as the aligned 4-byte word holding element i (0 when
// !ok) and decoded later, so no dtype-dependent code sits between the loads.
__device__ __forceinline__ uint32_t bload_scalar_word(Rsrc r, uint32_t i, int dt, bool ok) {
  const uint32_t byte = dt == FTM_DT_F32 ? 4u * i : 2u * i;
  return bload4(r, ok ? (byte & ~3u) : kOOB);
}
// Branch-free (selects only): a branch here would separate an MFMA from the
// VALU read of its result by a block boundary (see wave_gemm_kmajor).
__device__ __forceinline__ float decode_scalar_word(uint32_t w, uint32_t i, int dt) {
  const uint32_t h = (w >> ((i & 1u) * 16u)) & 0xffffu;
  const float f16v = f16_to_f32((uint16_t)h);
  const float bf16v = __uint_as_float(h << 16);
  const float narrow = dt == FTM_DT_F16 ? f16v : bf16v;
  return dt == FTM_DT_F32 ? __uint_as_float(w) : narrow;
}

// ---------------------------------------------------------------- A operand
// Each lane owns one A row (its l % 16) of the current 16-row M tile: the
// byte offset of that row in the activation buffer, or kOOB for a padding row.
// AT is the activation dtype: bf16 feeds the MFMA directly; fp32 / fp16 are
// split into bf16 hi + lo halves (16 significant bits) and cost two MFMAs.
template <int AT>
struct AType {
  static constexpr bool kSplit = AT != FTM_DT_BF16;
  static constexpr int kBytes = AT == FTM_DT_F32 ? 4 : 2;
};

template <int AT>
__device__ __forceinline__ void load_a8(Rsrc r, uint32_t row_off, int kk, u32x4& hi, u32x4& lo) {
  if constexpr (AT == FTM_DT_BF16) {
    hi = bload16(r, row_off + 2u * (uint32_t)kk);
    lo = (u32x4){0, 0, 0, 0};
  } else {
    float v[8];
    if constexpr (AT == FTM_DT_F32) {
      const u32x4 q0 = bload16(r, row_off + 4u * (uint32_t)kk);
      const u32x4 q1 = bload16(r, row_off + 4u * (uint32_t)kk + 16u);
      v[0] = __uint_as_float(q0.x); v[1] = __uint_as_float(q0.y);
      v[2] = __uint_as_float(q0.z); v[3] = __uint_as_float(q0.w);
      v[4] = __uint_as_float(q1.x); v[5] = __uint_as_float(q1.y);
      v[6] = __uint_as_float(q1.z); v[7] = __uint_as_float(q1.w);
    } else {
      const u32x4 q = bload16(r, row_off + 2u * (uint32_t)kk);
      const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[2 * i] = f16_to_f32((uint16_t)(w[i] & 0xffffu));
        v[2 * i + 1] = f16_to_f32((uint16_t)(w[i] >> 16));
      }
    }
    uint32_t h[4], l[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      h[i] = pack_bf16x2(v[2 * i], v[2 * i + 1]);
      l[i] = pack_bf16x2(v[2 * i] - bf16_to_f32(h[i] & 0xffffu), v[2 * i + 1] - bf16_to_f32(h[i] >> 16));
    }
    hi = (u32x4){h[0], h[1], h[2], h[3]};
    lo = (u32x4){l[0], l[1], l[2], l[3]};
  }
}

// Sum of the 8 activations a lane feeds (hi + lo), for the GPTQ zero-point correction.
__device__ __forceinline__ float sum_a8(u32x4 hi, u32x4 lo) {
  float s = 0.0f;
  const uint32_t h[4] = {hi.x, hi.y, hi.z, hi.w};
  const uint32_t l[4] = {lo.x, lo.y, lo.z, lo.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    s += bf16_to_f32(h[i] & 0xffffu) + bf16_to_f32(l[i] & 0xffffu);
    s += bf16_to_f32(h[i] >> 16) + bf16_to_f32(l[i] >> 16);
  }
  return s;
}

// ---------------------------------------------------------------- projection view
// One slot of one projection: raw pointers and the byte sizes of its banks.
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

// e4m3fn conversions on the hardware converts (v_cvt_pk_fp8_f32 rounds to
// nearest even; checked on MI355X bit for bit against a software RNE over
// every f32 with |v| < 448 and 12 trailing zero bits, subnormals and ties
// included, and v_cvt_f32_fp8 over all 256 codes).  The callers keep |v| <
// 257, so nothing saturates.
// Two values -> two codes in bits 0-7 and 8-15.
__device__ __forceinline__ uint32_t f32x2_to_e4m3(float a, float b) {
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false) & 0xffffu;
}
// Four values -> four codes, a in bits 0-7.
__device__ __forceinline__ uint32_t f32x4_to_e4m3(float a, float b, float c, float d) {
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false), true);
}
// Code in byte B of w -> its value.
template <int B>
__device__ __forceinline__ float e4m3_at(uint32_t w) {
  return __builtin_amdgcn_cvt_f32_fp8((int)w, B);
}

// ---------------------------------------------------------------- K-major engine
// Formats whose weight rows are contiguous along K: FP8 block, INT8 packed,
// MXFP4, BF16.  One "wave-load" = every lane loading 16 bytes of its row
// (row = col0 + l%16, the 4 lane groups side by side along K).
template <int FMT>
struct KMajor;

template <>
struct KMajor<FTM_FMT_FP8_BLOCK> {
  static constexpr int kLaneK = 16, kLoadK = 64, kMfma = 2;
  static constexpr bool kPostScale = true;
  __device__ static uint32_t row_bytes(int K) { return (uint32_t)K; }
  __device__ static uint32_t elem_off(int kk) { return (uint32_t)kk; }
};
template <>
struct KMajor<FTM_FMT_INT8_PACKED> {
  static constexpr int kLaneK = 16, kLoadK = 64, kMfma = 2;
  static constexpr bool kPostScale = true;
  __device__ static uint32_t row_bytes(int K) { return (uint32_t)K; }
  __device__ static uint32_t elem_off(int kk) { return (uint32_t)kk; }
};
template <>
struct KMajor<FTM_FMT_MXFP4> {
  static constexpr int kLaneK = 32, kLoadK = 128, kMfma = 4;
  static constexpr bool kPostScale = false;
  __device__ static uint32_t row_bytes(int K) { return (uint32_t)K / 2; }
  __device__ static uint32_t elem_off(int kk) { return (uint32_t)kk / 2; }
};
template <>
struct KMajor<FTM_FMT_BF16> {
  static constexpr int kLaneK = 8, kLoadK = 32, kMfma = 1;
  static constexpr bool kPostScale = false;
  __device__ static uint32_t row_bytes(int K) { return 2u * (uint32_t)K; }
  __device__ static uint32_t elem_off(int kk) { return 2u * (uint32_t)kk; }
};

template <int FMT>
__device__ __forceinline__ int fmt_loads(int K) {
  if constexpr (FMT == FTM_FMT_GPTQ_INT4) {
    return (K + 31) / 32;
  } else {
    return (K + KMajor<FMT>::kLoadK - 1) / KMajor<FMT>::kLoadK;
  }
}

// Wave-loads issued together before their MFMAs (registers vs loads in flight).
template <int FMT, int NR, int AT>
struct Chunk {
  static constexpr int v = (KMajor<FMT>::kMfma >= 4 || AType<AT>::kSplit || NR > 1) ? 4 : 8;
};

// acc[r] += A(16 x K-range) * W(rows col0[r] .. +16)^T over wave-loads [L_lo, L_hi).
// Rows >= N and k >= K read as zero.  For post-scaled formats the partial sum of
// each quantisation group is multiplied by the group's fp32 scale before it
// joins acc (FP8: one scale per 128x128 block; INT8: one per (row, group)).
template <int FMT, int NR, int AT>
__device__ __forceinline__ void wave_gemm_kmajor(const ProjSlot& W, const int (&col0)[NR], int L_lo, int L_hi,
                                                 Rsrc ares, uint32_t arow, f32x4 (&acc)[NR]) {
  using F = KMajor<FMT>;
  constexpr bool SPLIT = AType<AT>::kSplit;
  constexpr int CH = Chunk<FMT, NR, AT>::v;
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4;
  const int rl = lane & 15;
  const int K = W.K;
  const uint32_t rb = F::row_bytes(K);
  const Rsrc wres = make_rsrc(W.w, rb * (uint32_t)W.N);
  uint32_t woff[NR];
  Rsrc sres = wres;
  uint32_t soff[NR];
  if constexpr (FMT == FTM_FMT_FP8_BLOCK) {
    const int nkb = (K + W.group - 1) / W.group;
    const int nrb = (W.N + W.group - 1) / W.group;
    sres = make_rsrc(W.s, (uint32_t)(nrb * nkb) * (W.s_dt == FTM_DT_F32 ? 4u : 2u));
#pragma unroll
    for (int r = 0; r < NR; ++r) soff[r] = (col0[r] < W.N) ? (uint32_t)((col0[r] / W.group) * nkb) : kOOB;
  } else if constexpr (FMT == FTM_FMT_INT8_PACKED) {
    const int ng = K / W.group;
    sres = make_rsrc(W.s, (uint32_t)(W.N * ng) * (W.s_dt == FTM_DT_F32 ? 4u : 2u));
#pragma unroll
    for (int r = 0; r < NR; ++r) soff[r] = (col0[r] + rl < W.N) ? (uint32_t)((col0[r] + rl) * ng) : kOOB;
  } else if constexpr (FMT == FTM_FMT_MXFP4) {
    sres = make_rsrc(W.s, (uint32_t)W.N * (uint32_t)(K / 32));
#pragma unroll
    for (int r = 0; r < NR; ++r) soff[r] = (col0[r] + rl < W.N) ? (uint32_t)((col0[r] + rl) * (K / 32)) : kOOB;
  }
#pragma unroll
  for (int r = 0; r < NR; ++r) woff[r] = (col0[r] + rl < W.N) ? (uint32_t)(col0[r] + rl) * rb : kOOB;

  f32x4 tmp[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) tmp[r] = (f32x4){0.f, 0.f, 0.f, 0.f};

  // Post-scaled formats: wave-loads per quantisation group (the host requires
  // group % kLoadK == 0 or a single group), and the group / position of the
  // current wave-load, advanced by selects rather than per-load divisions.
  const int lpg = F::kPostScale ? (W.group + F::kLoadK - 1) / F::kLoadK : 1;
  int gcur = L_lo / lpg;
  int gpos = L_lo - gcur * lpg;

  for (int Lc = L_lo; Lc < L_hi; Lc += CH) {
    u32x4 raw[NR][CH];
    float sc[NR][CH];      // MXFP4: e8m0 factor of the lane's block
    uint32_t scw[NR][CH];  // FP8 / INT8: raw scale word of the wave-load's group
    int grp_b[CH];         // FP8 / INT8: group of wave-load b
    bool last_b[CH];       // FP8 / INT8: wave-load b ends its group or the range
    u32x4 ahi[CH][F::kMfma], alo[CH][F::kMfma];
#pragma unroll
    for (int b = 0; b < CH; ++b) {
      const int L = Lc + b;
      const int kk = L * F::kLoadK + F::kLaneK * g;
      const bool kok = (L < L_hi) && (kk < K);
      if constexpr (F::kPostScale) {
        const bool wrap = gpos == lpg - 1;
        grp_b[b] = gcur;
        last_b[b] = wrap | (L + 1 == L_hi);
        gpos = wrap ? 0 : gpos + 1;
        gcur += wrap ? 1 : 0;
      }
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        raw[r][b] = bload16(wres, kok ? woff[r] + F::elem_off(kk) : kOOB);
        if constexpr (F::kPostScale) {
          scw[r][b] = bload_scalar_word(sres, soff[r] + (uint32_t)grp_b[b], W.s_dt, L < L_hi && soff[r] != kOOB);
        }
      }
    }
    if constexpr (FMT == FTM_FMT_MXFP4) {
      // row r's e8m0 bytes of wave-loads b = 0 .. CH-1 sit 4 bytes apart
      // (group 4 (Lc + b) + g): byte sh / 8 of CH consecutive dwords, fetched
      // by ceil(CH / 4) 16-byte loads rather than one byte load per wave-load;
      // wave-loads outside the range take scale byte 0 (their weights are 0)
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        const uint32_t b0 = soff[r] != kOOB ? soff[r] + 4u * (uint32_t)Lc + (uint32_t)g : kOOB;
        const uint32_t sh = b0 != kOOB ? 8u * (b0 & 3u) : 0u;
        uint32_t dw[(CH + 3) / 4 * 4];
#pragma unroll
        for (int q = 0; q < (CH + 3) / 4; ++q) {
          const u32x4 v = bload16(sres, b0 != kOOB ? (b0 & ~3u) + 16u * (uint32_t)q : kOOB);
          dw[4 * q] = v.x;
          dw[4 * q + 1] = v.y;
          dw[4 * q + 2] = v.z;
          dw[4 * q + 3] = v.w;
        }
#pragma unroll
        for (int b = 0; b < CH; ++b) {
          const int L = Lc + b;
          const bool kok = (L < L_hi) && (L * F::kLoadK + F::kLaneK * g < K);
          sc[r][b] = e8m0_to_f32(kok ? (dw[b] >> sh) & 0xffu : 0u);
        }
      }
    }
    // Activation fragments after every weight load of the chunk: their row
    // offsets come from the expert's token list, so the weight stream is not
    // held up behind that dependent load.
#pragma unroll
    for (int b = 0; b < CH; ++b) {
      const int L = Lc + b;
      const int kk = L * F::kLoadK + F::kLaneK * g;
      const bool kok = (L < L_hi) && (kk < K);
#pragma unroll
      for (int q = 0; q < F::kMfma; ++q) load_a8<AT>(ares, kok ? arow : kOOB, kk + 8 * q, ahi[b][q], alo[b][q]);
    }
    // Wave-loads past L_hi read zeros, so the MFMAs below are unconditional
    // (no branch the compiler could sink the loads into).
#pragma unroll
    for (int b = 0; b < CH; ++b) {
      const int L = Lc + b;
#pragma unroll
      for (int q = 0; q < F::kMfma; ++q) {
#pragma unroll
        for (int r = 0; r < NR; ++r) {
          u32x4 bq;
          if constexpr (FMT == FTM_FMT_FP8_BLOCK) {
            bq = q == 0 ? fp8x8_to_bf16(raw[r][b].x, raw[r][b].y) : fp8x8_to_bf16(raw[r][b].z, raw[r][b].w);
          } else if constexpr (FMT == FTM_FMT_INT8_PACKED) {
            bq = q == 0 ? i8x8_to_bf16(raw[r][b].x, raw[r][b].y) : i8x8_to_bf16(raw[r][b].z, raw[r][b].w);
          } else if constexpr (FMT == FTM_FMT_MXFP4) {
            const uint32_t wq = q == 0 ? raw[r][b].x : q == 1 ? raw[r][b].y : q == 2 ? raw[r][b].z : raw[r][b].w;
            bq = fp4x8_to_bf16(wq, sc[r][b]);
          } else {
            bq = raw[r][b];
          }
          tmp[r] = mfma_bf16(ahi[b][q], bq, tmp[r]);
          if constexpr (SPLIT) tmp[r] = mfma_bf16(alo[b][q], bq, tmp[r]);
        }
      }
      if constexpr (F::kPostScale) {
        // End of a quantisation group (or of the wave's range): fold in its
        // scale.  Straight-line code on purpose: with a branch between the
        // MFMAs above and these reads of tmp, the gfx950 compiler has placed
        // too few wait states on the taken path and read stale accumulators.
        const bool fold = last_b[b] & (L < L_hi);
#pragma unroll
        for (int r = 0; r < NR; ++r) {
          const float s_grp = decode_scalar_word(scw[r][b], soff[r] + (uint32_t)grp_b[b], W.s_dt);
          const float f = fold ? s_grp : 0.0f;
          acc[r] += tmp[r] * f;
          const float keep = last_b[b] ? 0.0f : 1.0f;
          tmp[r] *= keep;
        }
      }
    }
  }
  if constexpr (!F::kPostScale) {
#pragma unroll
    for (int r = 0; r < NR; ++r) acc[r] += tmp[r];
  }
}

// ---------------------------------------------------------------- row-item engine
// A 4-byte word at a wave-uniform byte offset, read through the constant
// address space so the compiler emits a scalar (s_load) read.
__device__ __forceinline__ uint32_t sload4(const void* base, uint32_t off) {
  typedef const __attribute__((address_space(4))) uint32_t* CPtr;
  return *(CPtr)((const char*)base + off);
}
// Element i (wave-uniform) of an int32 table written by an earlier kernel,
// e.g. the routed-expert list: a scalar load keeps the value (and every
// address derived from it) in SGPRs whatever the rest of the kernel does.
__device__ __forceinline__ int sload_i32(const int32_t* p, int i) { return (int)sload4(p, 4u * (uint32_t)i); }
typedef uint32_t u32x8 __attribute__((ext_vector_type(8)));
// Eight consecutive int32 at a wave-uniform, 32-byte aligned address (one
// scalar load).
__device__ __forceinline__ u32x8 sload32(const void* base, uint32_t off) {
  typedef const __attribute__((address_space(4))) u32x8* CPtr;
  return *(CPtr)((const char*)base + off);
}

// acc += A(16 tokens x K range) * W(16 rows)^T, where lane l supplies weight
// row lrow (its MFMA column l % 16; -1 = no row, reads zero).  Unlike
// wave_gemm_kmajor the 16 rows need not be consecutive: stage A pairs 8 gate
// rows with their 8 up rows.  FP8 block scales are read with scalar loads:
// lanes l % 16 < 8 use scale row-block sb_lo, the others sb_hi (each uniform).
template <int FMT, int AT, int CH>
__device__ __forceinline__ void wave_rows_kmajor(const ProjSlot& W, int lrow, int sb_lo, int sb_hi, int L_lo,
                                                 int L_hi, Rsrc ares, uint32_t arow, f32x4& acc) {
  using F = KMajor<FMT>;
  constexpr bool SPLIT = AType<AT>::kSplit;
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4;
  const bool upper = (lane & 15) >= 8;
  const int K = W.K;
  const uint32_t rb = F::row_bytes(K);
  const Rsrc wres = make_rsrc(W.w, rb * (uint32_t)W.N);
  const uint32_t woff = lrow >= 0 ? (uint32_t)lrow * rb : kOOB;
  Rsrc sres = wres;
  uint32_t soff = kOOB;
  uint32_t fp8_lo = 0, fp8_hi = 0;  // FP8: byte offsets of the two scale rows
  int gmax = 0;                     // FP8: last K block (clamps the scalar reads)
  const uint32_t sesz = W.s_dt == FTM_DT_F32 ? 4u : 2u;
  if constexpr (FMT == FTM_FMT_FP8_BLOCK) {
    const int nkb = (K + W.group - 1) / W.group;
    gmax = nkb - 1;
    fp8_lo = (uint32_t)(sb_lo * nkb) * sesz;
    fp8_hi = (uint32_t)(sb_hi * nkb) * sesz;
  } else if constexpr (FMT == FTM_FMT_INT8_PACKED) {
    const int ng = K / W.group;
    sres = make_rsrc(W.s, (uint32_t)(W.N * ng) * sesz);
    soff = lrow >= 0 ? (uint32_t)(lrow * ng) : kOOB;
  } else if constexpr (FMT == FTM_FMT_MXFP4) {
    sres = make_rsrc(W.s, (uint32_t)W.N * (uint32_t)(K / 32));
    soff = lrow >= 0 ? (uint32_t)(lrow * (K / 32)) : kOOB;
  }
  const int lpg = F::kPostScale ? (W.group + F::kLoadK - 1) / F::kLoadK : 1;
  int gcur = L_lo / lpg;
  int gpos = L_lo - gcur * lpg;
  f32x4 tmp = (f32x4){0.f, 0.f, 0.f, 0.f};

  for (int Lc = L_lo; Lc < L_hi; Lc += CH) {
    u32x4 raw[CH];
    float sc[CH];       // MXFP4: e8m0 factor of the lane's block
    uint32_t scw[CH];   // FP8 / INT8: raw scale word of the wave-load's group
    int grp_b[CH];
    bool last_b[CH];
    u32x4 ahi[CH][F::kMfma], alo[CH][F::kMfma];
#pragma unroll
    for (int b = 0; b < CH; ++b) {
      const int L = Lc + b;
      const int kk = L * F::kLoadK + F::kLaneK * g;
      const bool kok = (L < L_hi) && (kk < K);
      if constexpr (F::kPostScale) {
        const bool wrap = gpos == lpg - 1;
        grp_b[b] = gcur;
        last_b[b] = wrap | (L + 1 == L_hi);
        gpos = wrap ? 0 : gpos + 1;
        gcur += wrap ? 1 : 0;
      }
      raw[b] = bload16(wres, kok ? woff + F::elem_off(kk) : kOOB);
      if constexpr (FMT == FTM_FMT_MXFP4) {
        sc[b] = e8m0_to_f32(bload1(sres, kok ? soff + (uint32_t)(kk / 32) : kOOB));
      } else if constexpr (FMT == FTM_FMT_FP8_BLOCK) {
        // both halves' words, uniform offsets -> scalar loads
        const uint32_t gb = (uint32_t)min(grp_b[b], gmax) * sesz;
        const uint32_t w_lo = sload4(W.s, (fp8_lo + gb) & ~3u);
        const uint32_t w_hi = sload4(W.s, (fp8_hi + gb) & ~3u);
        scw[b] = upper ? w_hi : w_lo;
      } else if constexpr (FMT == FTM_FMT_INT8_PACKED) {
        scw[b] = bload_scalar_word(sres, soff + (uint32_t)grp_b[b], W.s_dt, L < L_hi && soff != kOOB);
      }
    }
#pragma unroll
    for (int b = 0; b < CH; ++b) {
      const int L = Lc + b;
      const int kk = L * F::kLoadK + F::kLaneK * g;
      const bool kok = (L < L_hi) && (kk < K);
#pragma unroll
      for (int q = 0; q < F::kMfma; ++q) load_a8<AT>(ares, kok ? arow : kOOB, kk + 8 * q, ahi[b][q], alo[b][q]);
    }
#pragma unroll
    for (int b = 0; b < CH; ++b) {
      const int L = Lc + b;
#pragma unroll
      for (int q = 0; q < F::kMfma; ++q) {
        u32x4 bq;
        if constexpr (FMT == FTM_FMT_FP8_BLOCK) {
          bq = q == 0 ? fp8x8_to_bf16(raw[b].x, raw[b].y) : fp8x8_to_bf16(raw[b].z, raw[b].w);
        } else if constexpr (FMT == FTM_FMT_INT8_PACKED) {
          bq = q == 0 ? i8x8_to_bf16(raw[b].x, raw[b].y) : i8x8_to_bf16(raw[b].z, raw[b].w);
        } else if constexpr (FMT == FTM_FMT_MXFP4) {
          const uint32_t wq = q == 0 ? raw[b].x : q == 1 ? raw[b].y : q == 2 ? raw[b].z : raw[b].w;
          bq = fp4x8_to_bf16(wq, sc[b]);
        } else {
          bq = raw[b];
        }
        tmp = mfma_bf16(ahi[b][q], bq, tmp);
        if constexpr (SPLIT) tmp = mfma_bf16(alo[b][q], bq, tmp);
      }
      if constexpr (F::kPostScale) {
        // group end (or range end): fold in the group's scale; straight-line
        // code, see wave_gemm_kmajor
        const bool fold = last_b[b] & (L < L_hi);
        uint32_t sidx;
        if constexpr (FMT == FTM_FMT_FP8_BLOCK)
          sidx = ((upper ? fp8_hi : fp8_lo) / sesz) + (uint32_t)grp_b[b];
        else
          sidx = soff + (uint32_t)grp_b[b];
        const float s_grp = decode_scalar_word(scw[b], sidx, W.s_dt);
        acc += tmp * (fold ? s_grp : 0.0f);
        tmp *= last_b[b] ? 0.0f : 1.0f;
      }
    }
  }
  if constexpr (!F::kPostScale) acc += tmp;
}

// ---------------------------------------------------------------- prefetched row streams
// The per-lane-row GEMV of wave_rows_kmajor split into a weight half and an
// activation half.  rows_issue starts up to NLW wave-loads [Lw, min(Lw + NLW,
// L_hi)) of the lane's row (plus their scale words) and returns at once, so a
// workgroup's whole weight window is in flight behind one memory latency while
// the caller resolves its tokens; rows_consume_lds then runs the MFMAs with
// the activations taken from LDS.
//   lrow         weight row of lane l (its MFMA column l % 16); < 0 reads zero
//   sb_lo/sb_hi  FP8 only: 128-row scale block of lanes l % 16 < 8 / >= 8;
//                PAIRED = false when every lane's row is in block sb_lo
template <int FMT, int NLW>
struct RowStream {
  u32x4 raw[NLW];
  uint32_t sw[NLW];  // FP8 / INT8: scale word of the wave-load's group; MXFP4: the dword holding its e8m0 byte
  uint32_t sh;       // MXFP4: bit position of the byte in those dwords
  uint32_t vmask;    // MXFP4: wave-loads inside the lane's K range (the others decode with scale byte 0)
};

template <int FMT>
struct RowGeom {
  Rsrc wres, sres;
  uint32_t woff, soff;   // lane's row start in w / in its scale row (INT8, MXFP4)
  uint32_t fp8_lo, fp8_hi, sesz;
  int gmax, lpg;
  __device__ __forceinline__ RowGeom() = default;
  __device__ __forceinline__ RowGeom(const ProjSlot& W, int lrow, int sb_lo, int sb_hi) {
    using F = KMajor<FMT>;
    const int K = W.K;
    const uint32_t rb = F::row_bytes(K);
    wres = make_rsrc(W.w, rb * (uint32_t)W.N);
    woff = lrow >= 0 ? (uint32_t)lrow * rb : kOOB;
    sres = wres;
    soff = kOOB;
    fp8_lo = fp8_hi = 0;
    gmax = 0;
    sesz = W.s_dt == FTM_DT_F32 ? 4u : 2u;
    if constexpr (FMT == FTM_FMT_FP8_BLOCK) {
      const int nkb = (K + W.group - 1) / W.group;
      const int nrb = (W.N + W.group - 1) / W.group;
      gmax = nkb - 1;
      fp8_lo = (uint32_t)(sb_lo * nkb) * sesz;
      fp8_hi = (uint32_t)(sb_hi * nkb) * sesz;
      sres = make_rsrc(W.s, (uint32_t)(nrb * nkb) * sesz);
    } else if constexpr (FMT == FTM_FMT_INT8_PACKED) {
      const int ng = K / W.group;
      sres = make_rsrc(W.s, (uint32_t)(W.N * ng) * sesz);
      soff = lrow >= 0 ? (uint32_t)(lrow * ng) : kOOB;
    } else if constexpr (FMT == FTM_FMT_MXFP4) {
      sres = make_rsrc(W.s, (uint32_t)W.N * (uint32_t)(K / 32));
      soff = lrow >= 0 ? (uint32_t)(lrow * (K / 32)) : kOOB;
    }
    lpg = F::kPostScale ? (W.group + F::kLoadK - 1) / F::kLoadK : 1;
  }
};

template <int FMT, int NLW, bool PAIRED>
__device__ __forceinline__ void rows_issue(const ProjSlot& W, const RowGeom<FMT>& G, int Lw, int L_hi,
                                           RowStream<FMT, NLW>& S) {
  using F = KMajor<FMT>;
  const int g = (threadIdx.x & 63) >> 4;
  const bool upper = (threadIdx.x & 15) >= 8;
  const int K = W.K;
  int gcur = Lw / G.lpg;
  int gpos = Lw - gcur * G.lpg;
  if constexpr (FMT == FTM_FMT_MXFP4) S.vmask = 0u;
#pragma unroll
  for (int b = 0; b < NLW; ++b) {
    const int L = Lw + b;
    const int kk = L * F::kLoadK + F::kLaneK * g;
    const bool kok = (L < L_hi) && (kk < K);
    S.raw[b] = bload16(G.wres, kok ? G.woff + F::elem_off(kk) : kOOB);
    if constexpr (FMT == FTM_FMT_MXFP4) {
      S.vmask |= kok ? 1u << b : 0u;
    } else if constexpr (FMT == FTM_FMT_FP8_BLOCK) {
      // each lane reads its own row block's word with the weights (a vector
      // load: nothing waits for it until the MFMAs)
      const uint32_t gb = (uint32_t)min(gcur, G.gmax) * G.sesz;
      const uint32_t rb = (PAIRED && upper) ? G.fp8_hi : G.fp8_lo;
      S.sw[b] = bload4(G.sres, (L < L_hi) ? ((rb + gb) & ~3u) : kOOB);
    } else if constexpr (FMT == FTM_FMT_INT8_PACKED) {
      S.sw[b] = bload_scalar_word(G.sres, G.soff + (uint32_t)gcur, W.s_dt, L < L_hi && G.soff != kOOB);
    }
    if constexpr (F::kPostScale) {
      const bool wrap = gpos == G.lpg - 1;
      gpos = wrap ? 0 : gpos + 1;
      gcur += wrap ? 1 : 0;
    }
  }
  if constexpr (FMT == FTM_FMT_MXFP4) {
    // the lane's e8m0 bytes of wave-loads b = 0 .. NLW-1 sit 4 bytes apart in
    // its scale row (group 4 (Lw + b) + g), so they are byte sh / 8 of NLW
    // consecutive dwords: ceil(NLW / 4) 16-byte loads instead of one byte
    // load per wave-load (half the vector-memory instructions of the stream)
    const uint32_t b0 = G.soff != kOOB ? G.soff + 4u * (uint32_t)Lw + (uint32_t)g : kOOB;
    S.sh = b0 != kOOB ? 8u * (b0 & 3u) : 0u;
#pragma unroll
    for (int q = 0; q < (NLW + 3) / 4; ++q) {
      const u32x4 v = bload16(G.sres, b0 != kOOB ? (b0 & ~3u) + 16u * (uint32_t)q : kOOB);
      if (4 * q + 0 < NLW) S.sw[4 * q + 0] = v.x;
      if (4 * q + 1 < NLW) S.sw[4 * q + 1] = v.y;
      if (4 * q + 2 < NLW) S.sw[4 * q + 2] = v.z;
      if (4 * q + 3 < NLW) S.sw[4 * q + 3] = v.w;
    }
  }
}

// rows_consume_lds: the MFMAs of NT row tiles at once, activations from LDS.  xs
// holds the current block's token rows from element k0 on (bf16, `pitch`
// elements apart, nb of them) and, as row zr, a row of zeros at least as long
// as the wave's range; lane l feeds token row l % 16 of the MFMA, and rows >=
// nb as well as lanes whose K position is out of range read the zero row, so
// one address select per wave-load replaces a select per activation register
// and the reads of a wave-load use immediate offsets.  Each activation read
// feeds all NT tiles' MFMAs.
// Post-scaled formats accumulate each quantisation group in its own register
// (LPG wave-loads per group, the window starting on a group boundary, or the
// whole window inside one group when LPG == NLW) and apply the scales once at
// the end, so no MFMA waits on a VALU read of its own result mid-window.
// NOZ: no zero row (zr unused).  MFMA rows >= nb read row 0 instead (their
// outputs are never stored; an MFMA row depends on its own A row only), a
// wave-load past L_hi reads the last one in range against zero weights
// (out-of-range weight loads return 0, post-scales 0), and lanes past K read
// the region's tail, which the caller keeps at zero.
template <int FMT, int NLW, int NT, int LPG, bool PAIRED, bool NOZ = false>
__device__ __forceinline__ void rows_consume_lds(const ProjSlot& W, const RowGeom<FMT> (&G)[NT], int Lw, int L_hi,
                                                 const RowStream<FMT, NLW> (&S)[NT], const uint16_t* xs, int k0,
                                                 int pitch, int nb, int zr, f32x4 (&acc)[NT]) {
  using F = KMajor<FMT>;
  static_assert(NLW % LPG == 0, "groups tile the window");
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4;
  const int m = lane & 15;
  const bool upper = m >= 8;
  const int K = W.K;
  const uint16_t* zrow = xs + zr * pitch;
  const int rbase = (m < nb ? m : NOZ ? 0 : zr) * pitch - k0;  // lane's row, element kk at rbase + kk
  constexpr int NP = F::kPostScale ? NLW / LPG : 1;
  f32x4 part[NT][NP];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int i = 0; i < NP; ++i) part[t][i] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int b = 0; b < NLW; ++b) {
    const int L = Lw + b;
    const int kk = (NOZ ? min(L, L_hi - 1) : L) * F::kLoadK + F::kLaneK * g;
    const uint16_t* xb = NOZ ? xs + (rbase + kk) : (L < L_hi) && (kk < K) ? xs + (rbase + kk) : zrow;
#pragma unroll
    for (int q = 0; q < F::kMfma; ++q) {
      const u32x4 av = *(const u32x4*)(xb + 8 * q);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const u32x4 r = S[t].raw[b];
        u32x4 bq;
        if constexpr (FMT == FTM_FMT_FP8_BLOCK) {
          bq = q == 0 ? fp8x8_to_bf16(r.x, r.y) : fp8x8_to_bf16(r.z, r.w);
        } else if constexpr (FMT == FTM_FMT_INT8_PACKED) {
          bq = q == 0 ? i8x8_to_bf16(r.x, r.y) : i8x8_to_bf16(r.z, r.w);
        } else if constexpr (FMT == FTM_FMT_MXFP4) {
          const uint32_t wq = q == 0 ? r.x : q == 1 ? r.y : q == 2 ? r.z : r.w;
          const uint32_t e8 = ((S[t].vmask >> b) & 1u) ? (S[t].sw[b] >> S[t].sh) & 0xffu : 0u;
          bq = fp4x8_to_bf16(wq, e8m0_to_f32(e8));
        } else {
          bq = r;
        }
        f32x4& pt = part[t][F::kPostScale ? b / LPG : 0];
        pt = mfma_bf16(av, bq, pt);
      }
    }
  }
  if constexpr (F::kPostScale) {
    const int g0 = Lw / G[0].lpg;
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      const int b = i * LPG;  // first wave-load of the group
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        uint32_t sidx;
        if constexpr (FMT == FTM_FMT_FP8_BLOCK)
          sidx = (((PAIRED && upper) ? G[t].fp8_hi : G[t].fp8_lo) / G[t].sesz) + (uint32_t)(g0 + i);
        else
          sidx = G[t].soff + (uint32_t)(g0 + i);
        const float s_grp = decode_scalar_word(S[t].sw[b], sidx, W.s_dt);
        acc[t] += part[t][i] * ((Lw + b < L_hi) ? s_grp : 0.0f);
      }
    }
  } else {
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] += part[t][0];
  }
}

// ---------------------------------------------------------------- GPTQ engine
// qweight [K/8, N] int32 is contiguous along N.  One wave-load: lane group g
// reads packed row 4L+g (k = 32L + 8g .. +8) for columns col0 + 4*(l%16) + c,
// c = 0..3 (16 bytes).  A wave therefore produces 64 columns as 4 interleaved
// MFMA sub-tiles: sub-tile c, MFMA column j <-> output column col0 + 4j + c.
// The wave walks whole quantisation groups [grp_lo, grp_hi); each group's
// scales and zero word are loaded with its first weights, and at the group's
// end the zero point and the +128 decode bias are removed in fp32:
//   acc += s * (tmp - (128 + zp) * sum_k x_k)        (gptq_linear.py:88-99)
template <int NR, int AT>
__device__ __forceinline__ void wave_gemm_gptq(const ProjSlot& W, const int (&col0)[NR], int grp_lo, int grp_hi,
                                               Rsrc ares, uint32_t arow, f32x4 (&acc)[NR][4]) {
  constexpr bool SPLIT = AType<AT>::kSplit;
  constexpr int CH = 4;
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4;
  const int rl = lane & 15;
  const int N = W.N;
  const int K = W.K;
  const int G = W.group;
  const int ngroups = (K + G - 1) / G;
  const int nL = (K + 31) / 32;
  const uint32_t sbytes = W.s_dt == FTM_DT_F32 ? 4u : 2u;
  const Rsrc wres = make_rsrc(W.w, (uint32_t)(K / 8) * (uint32_t)N * 4u);
  const Rsrc zres = make_rsrc(W.z, (uint32_t)ngroups * (uint32_t)(N / 8) * 4u);
  const Rsrc sres = make_rsrc(W.s, (uint32_t)ngroups * (uint32_t)N * sbytes);
  uint32_t ncol[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) ncol[r] = (col0[r] + 4 * rl < N) ? (uint32_t)(col0[r] + 4 * rl) : kOOB;

  for (int grp = grp_lo; grp < grp_hi; ++grp) {
    const int L0 = grp * G / 32;
    const int L1 = min((grp + 1) * G / 32, nL);
    // this group's 4 scales and zero word per row tile (16 bytes covers 4 fp32 or 8 fp16 scales)
    u32x4 scv[NR];
    uint32_t zw[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const bool ok = ncol[r] != kOOB;
      scv[r] = bload16(sres, ok ? ((uint32_t)grp * (uint32_t)N + ncol[r]) * sbytes : kOOB);
      zw[r] = bload4(zres, ok ? ((uint32_t)grp * (uint32_t)(N / 8) + ncol[r] / 8) * 4u : kOOB);
    }
    f32x4 tmp[NR][4];
#pragma unroll
    for (int r = 0; r < NR; ++r)
#pragma unroll
      for (int c = 0; c < 4; ++c) tmp[r][c] = (f32x4){0.f, 0.f, 0.f, 0.f};
    float xs = 0.0f;
    for (int Lc = L0; Lc < L1; Lc += CH) {
      u32x4 raw[NR][CH];
      u32x4 ahi[CH], alo[CH];
#pragma unroll
      for (int b = 0; b < CH; ++b) {
        const int L = Lc + b;
        const int prow = 4 * L + g;
        const bool kok = (L < L1) && (8 * prow < K);
#pragma unroll
        for (int r = 0; r < NR; ++r)
          raw[r][b] = bload16(wres, (kok && ncol[r] != kOOB) ? ((uint32_t)prow * (uint32_t)N + ncol[r]) * 4u : kOOB);
        u32x4 h, l;
        load_a8<AT>(ares, kok ? arow : kOOB, 8 * prow, h, l);
        ahi[b] = perm_gptq(h);
        alo[b] = perm_gptq(l);
      }
      // wave-loads past the group read zeros: x sums and MFMAs stay unconditional
#pragma unroll
      for (int b = 0; b < CH; ++b) {
        xs += sum_a8(ahi[b], alo[b]);
#pragma unroll
        for (int r = 0; r < NR; ++r) {
          const uint32_t wv[4] = {raw[r][b].x, raw[r][b].y, raw[r][b].z, raw[r][b].w};
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const u32x4 bq = gptq_word_to_bf16(wv[c], gq_decode_consts());
            tmp[r][c] = mfma_bf16(ahi[b], bq, tmp[r][c]);
            if constexpr (SPLIT) tmp[r][c] = mfma_bf16(alo[b], bq, tmp[r][c]);
          }
        }
      }
    }
    // Row sums of x over this group: reduce the 4 lane groups (same l%16), then
    // fetch the sums of the D rows this lane holds (row 4g+rr lives at lane 4g+rr).
    float sx = xs;
    sx += __shfl_xor(sx, 16);
    sx += __shfl_xor(sx, 32);
    float sxr[4];
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) sxr[rr] = __shfl(sx, 4 * g + rr);
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const uint32_t sw[4] = {scv[r].x, scv[r].y, scv[r].z, scv[r].w};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        float sc;
        if (sbytes == 4u) sc = __uint_as_float(sw[c]);
        else {
          const uint32_t h = (sw[c >> 1] >> (16 * (c & 1))) & 0xffffu;
          sc = W.s_dt == FTM_DT_F16 ? f16_to_f32((uint16_t)h) : bf16_to_f32(h);
        }
        const float zp = (float)(((zw[r] >> (4 * ((ncol[r] + c) & 7))) & 0xfu) + 1u);
        f32x4 corr;
        corr.x = tmp[r][c].x - (128.0f + zp) * sxr[0];
        corr.y = tmp[r][c].y - (128.0f + zp) * sxr[1];
        corr.z = tmp[r][c].z - (128.0f + zp) * sxr[2];
        corr.w = tmp[r][c].w - (128.0f + zp) * sxr[3];
        acc[r][c] += corr * sc;
      }
    }
  }
}

}  // namespace ftm
