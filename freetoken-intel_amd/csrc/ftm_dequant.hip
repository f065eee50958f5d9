// ftm_dequant.hip -- bit-exact dense dequantization of one bank slot.
//
// Each element is the reference's fp32 product rounded once to the output
// dtype (round-to-nearest-even):
//   FP8   w = fp32(e4m3) * s[n/B][k/B]                 fp8_block_linear.py:48-91
//         (e5m2 bytes: the same product; an e5m2 byte is the high byte of the
//         fp16 with the same value, so its decode is exact)
//   GPTQ  w = s[g][n] * (q[k][n] - (z[g][n] + 1))      gptq_linear.py:55-124 (output [K, N])
//   INT8  w = (byte - 128) * s[n][k/gs]                int8_packed_linear.py:74-125
//   MXFP4 w = LUT[nibble] * 2^(e8m0 - 127)             mxfp4_linear.py:38-76
//   BF16  w = bf16 value
// The e4m3 decode uses the gfx950 hardware conversion (v_cvt_pk_f32_fp8, OCP
// e4m3fn), which is exact; tests compare every one of the 256 codes with the
// OCP definition.
#include "ftm_device.h"
#include "ftm_internal.h"

namespace ftm {

__constant__ float kE2M1[16] = {0.0f,  0.5f,  1.0f,  1.5f,  2.0f,  3.0f,  4.0f,  6.0f,
                                -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};

// e5m2 (sign, 5 exponent bits with bias 15, 2 mantissa bits: the high byte of
// an IEEE fp16) -> its exact fp32 value, infinities and NaN included.
__device__ __forceinline__ float e5m2_to_f32(uint32_t b) {
  const uint32_t sign = (b & 0x80u) << 24, e = (b >> 2) & 31u, m = b & 3u;
  if (e == 31u) return __uint_as_float(sign | 0x7f800000u | (m << 21));
  if (e == 0u) return __uint_as_float(sign | __float_as_uint((float)m * 0x1p-16f));
  return __uint_as_float(sign | ((e + 112u) << 23) | (m << 21));
}

__device__ __forceinline__ float dequant_elem(const ProjSlot& W, int n, int k) {
  const int N = W.N, K = W.K;
  switch (W.fmt) {
    case FTM_FMT_FP8_BLOCK: {
      const uint32_t b = (uint8_t)W.w[(int64_t)n * K + k];
      const f32x2 f = __builtin_amdgcn_cvt_pk_f32_fp8((int)b, false);
      const int nkb = (K + W.group - 1) / W.group;
      const float s = load_scalar(W.s, (int64_t)(n / W.group) * nkb + k / W.group, W.s_dt);
      return f.x * s;
    }
    case FTM_FMT_FP8_E5M2_BLOCK: {
      const float f = e5m2_to_f32((uint8_t)W.w[(int64_t)n * K + k]);
      const int nkb = (K + W.group - 1) / W.group;
      const float s = load_scalar(W.s, (int64_t)(n / W.group) * nkb + k / W.group, W.s_dt);
      return f * s;
    }
    case FTM_FMT_GPTQ_INT4: {
      const uint32_t word = ((const uint32_t*)W.w)[(int64_t)(k / 8) * N + n];
      const int q = (int)((word >> (4 * (k & 7))) & 0xfu);
      const int g = k / W.group;
      const uint32_t zw = ((const uint32_t*)W.z)[(int64_t)g * (N / 8) + n / 8];
      const int z = (int)((zw >> (4 * (n & 7))) & 0xfu) + 1;
      const float s = load_scalar(W.s, (int64_t)g * N + n, W.s_dt);
      return s * (float)(q - z);
    }
    case FTM_FMT_INT8_PACKED: {
      const uint32_t word = ((const uint32_t*)W.w)[(int64_t)n * (K / 4) + k / 4];
      const int v = (int)((word >> (8 * (k & 3))) & 0xffu) - 128;
      const int ng = K / W.group;
      const float s = load_scalar(W.s, (int64_t)n * ng + k / W.group, W.s_dt);
      return (float)v * s;
    }
    case FTM_FMT_MXFP4: {
      const uint32_t b = (uint8_t)W.w[(int64_t)n * (K / 2) + k / 2];
      const uint32_t nib = (k & 1) ? (b >> 4) : (b & 0xfu);
      const uint32_t e = (uint8_t)W.s[(int64_t)n * (K / 32) + k / 32];
      return kE2M1[nib] * e8m0_to_f32(e);
    }
    case FTM_FMT_FP32:
      return ((const float*)W.w)[(int64_t)n * K + k];
    default:  // FTM_FMT_BF16
      return bf16_to_f32(((const uint16_t*)W.w)[(int64_t)n * K + k]);
  }
}

__global__ __launch_bounds__(kBlock) void k_dequant(const ftm_proj P, int slot, void* out, int out_dt,
                                                    int transpose) {
  const ProjSlot W = proj_slot(P, slot);
  const int64_t total = (int64_t)W.N * W.K;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    // Walk in output order so stores are coalesced.
    int n, k;
    if (transpose) {
      k = (int)(idx / W.N);
      n = (int)(idx % W.N);
    } else {
      n = (int)(idx / W.K);
      k = (int)(idx % W.K);
    }
    store_scalar(out, idx, out_dt, dequant_elem(W, n, k));
  }
}

// ============================================================== generic path
// Scalar fp32 kernels for every shape / dtype / format the reference API
// accepts but the MFMA engine does not take (K not a multiple of 16, INT8
// groups below 64, fp32 dense banks, tiny fused_moe test shapes): each output
// is a sequential fp32 fma over the reference's dequantized weights.
__global__ __launch_bounds__(kBlock) void k_linear_generic(const ftm_proj P, int slot, const void* x, int x_dt,
                                                           int M, void* out, int out_dt, const void* bias,
                                                           int bias_dt, int final_dt) {
  const ProjSlot W = proj_slot(P, slot);
  const int N = W.N, K = W.K;
  const int64_t total = (int64_t)M * N;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int m = (int)(idx / N), n = (int)(idx % N);
    float acc = 0.0f;
    for (int k = 0; k < K; ++k) acc = __builtin_fmaf(load_scalar(x, (int64_t)m * K + k, x_dt), dequant_elem(W, n, k), acc);
    float v = round_to(acc, out_dt);
    if (bias != nullptr) v = round_to(v + load_scalar(bias, n, bias_dt), final_dt);
    store_scalar(out, idx, final_dt, v);
  }
}

struct GenArgs {
  ftm_moe_layer L;
  const void* x;
  void* out;
  int T, KP, Imax;
  const int32_t* ids;
  const float* wts;
  char* hbuf;
  float* ybuf;
};

__device__ __forceinline__ float gen_act(int act, float g, float u, float alpha, float limit) {
  if (act == FTM_ACT_SILU) return g / (1.0f + expf(-g)) * u;
  if (act == FTM_ACT_GELU) return 0.5f * g * (1.0f + erff(g * 0.70710678118654752f)) * u;
  if (act == FTM_ACT_RELU) return fmaxf(g, 0.0f) * u;
  g = fminf(g, limit);
  u = fminf(fmaxf(u, -limit), limit);
  return (u + 1.0f) * (g / (1.0f + expf(-alpha * g)));
}

// Resolve pair p = t*KP + j to its projection slot view; false if not resident.
__device__ __forceinline__ bool gen_pair(const GenArgs& a, int p, bool down, ProjSlot& W, int& Iu) {
  const int k = a.L.topk, t = p / a.KP, j = p % a.KP;
  if (j == k) {  // shared expert
    Iu = a.L.shared_inter;
    W.w = (const char*)(down ? a.L.shared_w2 : a.L.shared_w13);
    W.s = W.z = W.bias = nullptr;
    W.fmt = FTM_FMT_BF16;
    W.s_dt = W.bias_dt = FTM_DT_BF16;
    W.group = 0;
    W.N = down ? a.L.hidden : 2 * Iu;
    W.K = down ? Iu : a.L.hidden;
    return true;
  }
  const int e = a.ids[(int64_t)t * k + j];
  if (e < 0 || e >= a.L.num_experts) return false;
  const int slot = a.L.slot_of_expert ? a.L.slot_of_expert[e] : e;
  const ftm_proj& P = down ? a.L.w2 : a.L.w13;
  if (slot < 0 || slot >= P.num_slots) return false;
  W = proj_slot(P, slot);
  Iu = a.L.inter;
  return true;
}

__global__ __launch_bounds__(kBlock) void k_gen_stage_a(const GenArgs a) {
  const int H = a.L.hidden, KP = a.KP, dt = a.L.act_dtype;
  const int64_t total = (int64_t)a.T * KP * a.Imax;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int p = (int)(idx / a.Imax), i = (int)(idx % a.Imax);
    ProjSlot W;
    int Iu;
    if (!gen_pair(a, p, false, W, Iu) || i >= Iu) continue;
    const int t = p / KP;
    const bool on_in = a.L.apply_router_weight_on_input && (p % KP) < a.L.topk;
    const float mul = on_in ? a.wts[p] : 1.0f;
    float g = 0.0f, u = 0.0f;
    for (int k = 0; k < H; ++k) {
      float xv = load_scalar(a.x, (int64_t)t * H + k, dt);
      if (on_in) xv = round_to(xv * mul, dt);
      g = __builtin_fmaf(xv, dequant_elem(W, i, k), g);
      u = __builtin_fmaf(xv, dequant_elem(W, Iu + i, k), u);
    }
    if (W.bias != nullptr) {
      g += load_scalar(W.bias, i, W.bias_dt);
      u += load_scalar(W.bias, Iu + i, W.bias_dt);
    }
    store_scalar(a.hbuf, (int64_t)p * a.Imax + i, dt,
                 round_to(gen_act(a.L.act, g, u, a.L.swiglu_alpha, a.L.swiglu_limit), a.L.h_dtype));
  }
}

__global__ __launch_bounds__(kBlock) void k_gen_stage_b(const GenArgs a) {
  const int H = a.L.hidden, KP = a.KP, dt = a.L.act_dtype;
  const int64_t total = (int64_t)a.T * KP * H;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int p = (int)(idx / H), n = (int)(idx % H);
    ProjSlot W;
    int Iu;
    float y = 0.0f;
    if (gen_pair(a, p, true, W, Iu)) {
      for (int i = 0; i < Iu; ++i)
        y = __builtin_fmaf(load_scalar(a.hbuf, (int64_t)p * a.Imax + i, dt), dequant_elem(W, n, i), y);
      if (W.bias != nullptr) y += load_scalar(W.bias, n, W.bias_dt);
      const bool on_in = a.L.apply_router_weight_on_input && (p % KP) < a.L.topk;
      if (!on_in) y *= a.wts[p];
    }
    a.ybuf[idx] = y;
  }
}

__global__ __launch_bounds__(kBlock) void k_gen_combine(const GenArgs a) {
  const int H = a.L.hidden, KP = a.KP;
  const int64_t total = (int64_t)a.T * H;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int t = (int)(idx / H), n = (int)(idx % H);
    float s = 0.0f;
    for (int j = 0; j < KP; ++j) s += a.ybuf[((int64_t)t * KP + j) * H + n];
    store_scalar(a.out, idx, a.L.act_dtype, s);
  }
}

static unsigned gen_blocks(int64_t total) {
  int64_t b = (total + kBlock - 1) / kBlock;
  if (b > 4096) b = 4096;
  return (unsigned)(b < 1 ? 1 : b);
}

hipError_t launch_linear_generic(const ftm_proj& P, int slot, const void* x, int x_dt, int M, void* out,
                                 int out_dt, const void* bias, int bias_dt, int final_dt, hipStream_t st) {
  hipLaunchKernelGGL(k_linear_generic, dim3(gen_blocks((int64_t)M * P.N)), dim3(kBlock), 0, st, P, slot, x, x_dt, M,
                     out, out_dt, bias, bias_dt, final_dt);
  return hipGetLastError();
}

hipError_t launch_experts_generic(const ftm_moe_layer& L, const void* x, int T, void* out, char* ws,
                                  const WsLayout& wl, hipStream_t st) {
  GenArgs a;
  a.L = L;
  a.x = x;
  a.out = out;
  a.T = T;
  a.KP = wl.KP;
  a.Imax = wl.Imax;
  a.ids = (const int32_t*)(ws + wl.ids);
  a.wts = (const float*)(ws + wl.wts);
  a.hbuf = ws + wl.hbuf;
  a.ybuf = (float*)(ws + wl.ybuf);
  hipLaunchKernelGGL(k_gen_stage_a, dim3(gen_blocks((int64_t)T * wl.KP * wl.Imax)), dim3(kBlock), 0, st, a);
  hipLaunchKernelGGL(k_gen_stage_b, dim3(gen_blocks((int64_t)T * wl.KP * L.hidden)), dim3(kBlock), 0, st, a);
  hipLaunchKernelGGL(k_gen_combine, dim3(gen_blocks((int64_t)T * L.hidden)), dim3(kBlock), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_dequant(const ftm_proj& P, int slot, void* out, int out_dt, int transpose, hipStream_t st) {
  const int64_t total = (int64_t)P.N * P.K;
  int64_t blocks = (total + kBlock - 1) / kBlock;
  if (blocks > 8192) blocks = 8192;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(k_dequant, dim3((unsigned)blocks), dim3(kBlock), 0, st, P, slot, out, out_dt, transpose);
  return hipGetLastError();
}

}  // namespace ftm
