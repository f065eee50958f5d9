/*
 * oracle_core.c -- TEST INFRASTRUCTURE ONLY.  CPU restatement of the reference
 * algorithms of FreeToken-Intel's quantized MoE layer, used by tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg as the checker.
 * Never linked into, loaded by, or called from the product library.
 *
 * Every function cites the reference file:line (under /root/reference) whose
 * arithmetic it restates.  Build: oracle/Makefile (gcc -O2 -ffp-contract=off,
 * so every product below is a separately rounded IEEE multiply unless fmaf is
 * written explicitly).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* Same field layout as ftm_proj of the product header, restated so the oracle
 * depends on nothing in the product. */
typedef struct orc_proj {
  const void* w;
  const void* s;
  const void* z;
  const void* bias;
  int64_t w_stride, s_stride, z_stride, bias_stride;
  int32_t fmt, s_dtype, bias_dtype, group, N, K, num_slots, reserved;
} orc_proj;

enum { F_BF16 = 0, F_FP8 = 1, F_GPTQ = 2, F_INT8 = 3, F_MXFP4 = 4, F_FP32 = 5 };
enum { D_F32 = 0, D_F16 = 1, D_BF16 = 2 };
enum { A_SILU = 0, A_GELU = 1, A_RELU = 2, A_OAI = 3 };

/* ------------------------------------------------------------------ scalars */
float orc_bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* round-to-nearest-even, NaN -> quiet NaN (c10::BFloat16 semantics) */
uint16_t orc_f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float orc_round_bf16(float f) { return orc_bf16_to_f32(orc_f32_to_bf16(f)); }

/* IEEE binary16 decode (exact). */
float orc_f16_to_f32(uint16_t h) {
  const int s = h >> 15, e = (h >> 10) & 0x1f, m = h & 0x3ff;
  float v;
  if (e == 0) v = ldexpf((float)m, -24);
  else if (e == 31) v = m ? NAN : INFINITY;
  else v = ldexpf((float)(m + 1024), e - 25);
  return s ? -v : v;
}

/* OCP FP8 e4m3fn: bias 7, no infinities, S.1111.111 = NaN, subnormal m*2^-9.
 * torch.float8_e4m3fn -> float32 (python/freetoken/kernel/triton/fp8_block_linear.py:70). */
float orc_e4m3_to_f32(uint8_t b) {
  const int s = b >> 7, e = (b >> 3) & 0xf, m = b & 7;
  float v;
  if (e == 15 && m == 7) return NAN;
  if (e == 0) v = ldexpf((float)m, -9);
  else v = ldexpf((float)(8 + m), e - 10);
  return s ? -v : v;
}

/* e8m0 -> torch.exp2(s - 127) (python/freetoken/kernel/triton/mxfp4_linear.py:74):
 * exact power of two, 2^-127 is an fp32 subnormal, 2^128 overflows to +inf. */
float orc_e8m0_to_f32(uint8_t s) {
  if (s == 255) return INFINITY;
  return ldexpf(1.0f, (int)s - 127);
}

/* python/freetoken/kernel/triton/mxfp4_linear.py:38-41 */
static const float kLut[16] = {0.0f,  0.5f,  1.0f,  1.5f,  2.0f,  3.0f,  4.0f,  6.0f,
                               -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};

static float load_dt(const void* p, int64_t i, int dt) {
  if (dt == D_F32) return ((const float*)p)[i];
  if (dt == D_F16) return orc_f16_to_f32(((const uint16_t*)p)[i]);
  return orc_bf16_to_f32(((const uint16_t*)p)[i]);
}

/* --------------------------------------------------------------- dequant
 * One element W[n][k] (logical [out, in]) of one slot, as the fp32 value the
 * reference computes before its final cast:
 *   FP8   fp8_block_linear.py:86-91    fp32(e4m3) * fp32(scale[n/B][k/B])
 *   GPTQ  gptq_linear.py:88-99         fp32(scale[g][n]) * (fp32(q) - fp32(z + 1))
 *   INT8  int8_packed_linear.py:89-93,122-125   fp32(byte - 128) * fp32(scale[n][k/gs])
 *   MXFP4 mxfp4_linear.py:75-79        LUT[nibble] * exp2(e8m0 - 127)
 */
float orc_deq(const orc_proj* P, int slot, int n, int k) {
  const int N = P->N, K = P->K;
  const char* w = (const char*)P->w + (int64_t)slot * P->w_stride;
  const char* s = P->s ? (const char*)P->s + (int64_t)slot * P->s_stride : NULL;
  const char* z = P->z ? (const char*)P->z + (int64_t)slot * P->z_stride : NULL;
  switch (P->fmt) {
    case F_FP8: {
      const int B = P->group, nkb = (K + B - 1) / B;
      const float sc = load_dt(s, (int64_t)(n / B) * nkb + k / B, P->s_dtype);
      return orc_e4m3_to_f32((uint8_t)w[(int64_t)n * K + k]) * sc;
    }
    case F_GPTQ: {
      const uint32_t word = ((const uint32_t*)w)[(int64_t)(k / 8) * N + n];
      const int q = (int)((word >> (4 * (k % 8))) & 0xfu);
      const int g = k / P->group;
      const uint32_t zw = ((const uint32_t*)z)[(int64_t)g * (N / 8) + n / 8];
      const int zp = (int)((zw >> (4 * (n % 8))) & 0xfu) + 1;
      const float sc = load_dt(s, (int64_t)g * N + n, P->s_dtype);
      return sc * ((float)q - (float)zp);
    }
    case F_INT8: {
      const uint32_t word = ((const uint32_t*)w)[(int64_t)n * (K / 4) + k / 4];
      const int v = (int)((word >> (8 * (k % 4))) & 0xffu) - 128;
      const int ng = K / P->group;
      return (float)v * load_dt(s, (int64_t)n * ng + k / P->group, P->s_dtype);
    }
    case F_MXFP4: {
      const uint8_t b = (uint8_t)w[(int64_t)n * (K / 2) + k / 2];
      const int nib = (k % 2) ? (b >> 4) : (b & 0xf);
      return kLut[nib] * orc_e8m0_to_f32((uint8_t)s[(int64_t)n * (K / 32) + k / 32]);
    }
    case F_FP32:
      return ((const float*)w)[(int64_t)n * K + k];
    default:
      return orc_bf16_to_f32(((const uint16_t*)w)[(int64_t)n * K + k]);
  }
}

/* Dense [N, K] fp32 dequant of one slot. */
void orc_dequant(const orc_proj* P, int slot, float* out) {
  for (int n = 0; n < P->N; ++n)
    for (int k = 0; k < P->K; ++k) out[(int64_t)n * P->K + k] = orc_deq(P, slot, n, k);
}

/* --------------------------------------------------------------- router
 * logits[t][r] = round_bf16( S(x_t, G_r) (+ bias_r) ), the bf16 Linear of
 * python/freetoken/models/qwen3_5_moe/__init__.py:1224 (LinearReplicated, bf16)
 * and gpt_oss/__init__.py:348 (nn.Linear with bias).  The fp32 sum S is the
 * fixed-order reduction the gfx950 router kernel performs: 64 lane partials,
 * lane l accumulating fmaf over 8-element chunks c = l, l+64, ... in order,
 * then a xor-32,16,8,4,2,1 butterfly.  (The reference's own Linear leaves its
 * summation order to the BLAS; this order is the one the tests pin.) */
static float gpu_order_dot(const float* x, const float* g, int H) {
  float v[64];
  for (int l = 0; l < 64; ++l) {
    float acc = 0.0f;
    for (int c = l; 8 * c < H; c += 64)
      for (int e = 0; e < 8; ++e) acc = fmaf(x[8 * c + e], g[8 * c + e], acc);
    v[l] = acc;
  }
  for (int off = 32; off >= 1; off >>= 1) {
    float nv[64];
    for (int l = 0; l < 64; ++l) nv[l] = v[l] + v[l ^ off];
    memcpy(v, nv, sizeof(v));
  }
  return v[0];
}

void orc_router_logits(const uint16_t* x, int T, int H, const uint16_t* G, int R, const uint16_t* bias,
                       float* out) {
  float* xf = (float*)malloc(sizeof(float) * (size_t)H);
  float* gf = (float*)malloc(sizeof(float) * (size_t)H);
  for (int r = 0; r < R; ++r) {
    for (int k = 0; k < H; ++k) gf[k] = orc_bf16_to_f32(G[(int64_t)r * H + k]);
    for (int t = 0; t < T; ++t) {
      for (int k = 0; k < H; ++k) xf[k] = orc_bf16_to_f32(x[(int64_t)t * H + k]);
      float z = gpu_order_dot(xf, gf, H);
      if (bias) z = z + orc_bf16_to_f32(bias[r]);
      out[(int64_t)t * R + r] = orc_round_bf16(z);
    }
  }
  free(xf);
  free(gf);
}

/* --------------------------------------------------------------- routing
 * Router softmax / top-k / renorm with the GPU's IEEE operations step for
 * step, so that routing indices AND router weights are bitwise equal to the
 * kernel's (route_token_pre / ftm_expf in the product's device code).  The
 * arithmetic follows the reference:
 *   mode 0  softmax over E in fp32, top-k, renorm      qwen3_5_moe/__init__.py:1225-1227
 *   mode 1  softmax in the logits' dtype, top-k on those probabilities,
 *           renorm divided in that dtype               fused_moe.py:92-96, qwen3_moe/__init__.py:473-475
 *   mode 2  top-k on the logits, softmax over the k    gpt_oss/__init__.py:350-352
 * and the weights are rounded to the activation dtype (fused_moe.py:96).
 * The reference leaves exp and the summation order to torch; the order
 * here is the kernel's: lane l of one wave holds experts l, l + 64, ...,
 * sums their exponentials in that order, and the 64 lane sums are reduced
 * by wave_sum_tree below.  Ties break to the lower expert index. */

/* e^x: Cody & Waite range reduction x = n ln2 + r (n = rint(x log2 e), ln 2
 * split into the float nearest it and the float nearest the remainder, each
 * product folded in by one fmaf), the degree-7 Taylor polynomial of e^r in
 * Horner form, and 2^n as two exact powers of two.  x is clamped to
 * [-104, 89] (NaN gives 0).  Within 0.94 ulp of e^x over every float in
 * [-104, 88.7] whose result is normal (tests/test_oracle.py pins it against
 * float64 exp). */
float orc_expf(float x) {
  const float xc = fminf(fmaxf(x, -104.0f), 89.0f);
  const float n = rintf(xc * 0x1.715476p+0f);
  float r = fmaf(n, -0x1.62e43p-1f, xc);
  r = fmaf(n, 0x1.05c61p-29f, r);
  float p = 0x1.a01a02p-13f;
  p = fmaf(p, r, 0x1.6c16c2p-10f);
  p = fmaf(p, r, 0x1.111112p-7f);
  p = fmaf(p, r, 0x1.555556p-5f);
  p = fmaf(p, r, 0x1.555556p-3f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  const int ni = (int)n, h = ni >> 1;
  uint32_t b1 = (uint32_t)(h + 127) << 23, b2 = (uint32_t)(ni - h + 127) << 23;
  float s1, s2;
  memcpy(&s1, &b1, 4);
  memcpy(&s2, &b2, 4);
  return fmaf(p * s1, s2, 0.0f);
}

void orc_expf_n(const float* x, int64_t n, float* y) {
  for (int64_t i = 0; i < n; ++i) y[i] = orc_expf(x[i]);
}

/* The shared expert's gate weight sigmoid(z) = 1 / (1 + e^-z)
 * (qwen3_5_moe/__init__.py:1229-1230), on orc_expf. */
float orc_sigmoidf(float z) { return 1.0f / (1.0f + orc_expf(-z)); }

/* fp32 -> IEEE binary16, round to nearest even (subnormals kept), as fp32. */
float orc_round_f16(float f) {
  if (f != f) return f;
  const float a = fabsf(f);
  if (a >= 65520.0f) return copysignf(INFINITY, f);
  if (a == 0.0f) return f;
  int e;
  frexpf(a, &e);
  int q = (e - 1) - 10; /* quantum exponent of the binary16 value */
  if (q < -24) q = -24;
  return copysignf(ldexpf(rintf(ldexpf(a, -q)), q), f);
}

static float round_dt(float v, int dt) {
  if (dt == D_BF16) return orc_round_bf16(v);
  if (dt == D_F16) return orc_round_f16(v);
  return v;
}

/* The wave-wide sum of 64 lane values in the kernel's DPP order
 * (wave_sum_dpp): lane pairs i ^ 1, then i ^ 2, then the mirror within 8
 * lanes (i <-> 7 - i), within 16 (i <-> 15 - i), then
 * (lane 0 + lane 16) + (lane 32 + lane 48). */
float orc_wave_sum(const float* v64) {
  float a[64], b[64];
  for (int i = 0; i < 64; ++i) a[i] = v64[i] + v64[i ^ 1];
  for (int i = 0; i < 64; ++i) b[i] = a[i] + a[i ^ 2];
  for (int i = 0; i < 64; ++i) a[i] = b[i] + b[(i & ~7) | (7 - (i & 7))];
  for (int i = 0; i < 64; ++i) b[i] = a[i] + a[(i & ~15) | (15 - (i & 15))];
  return (b[0] + b[16]) + (b[32] + b[48]);
}

/* Order-preserving image of a key: larger float -> larger image, -0 as +0,
 * NaN below everything (pack_key's order). */
static uint32_t key_image(float v) {
  if (v != v) return 0u;
  if (v == 0.0f) v = 0.0f;
  uint32_t b;
  memcpy(&b, &v, 4);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

/* logits fp32 [T, E] (the values of the logits' dtype); pdt: dtype the
 * LOWP probabilities are rounded to; wdt: the activation dtype.  ids int32
 * [T, k], w fp32 [T, k].  Returns 0, or -2 for a bad shape. */
int orc_route(const float* logits, int T, int E, int k, int mode, int renorm, int pdt, int wdt, int32_t* ids,
              float* w) {
  if (T < 0 || E <= 0 || k <= 0 || k > E || k > 64) return -2;
  float* key = (float*)malloc(sizeof(float) * (size_t)E);
  char* used = (char*)malloc((size_t)E);
  for (int t = 0; t < T; ++t) {
    const float* v = logits + (int64_t)t * E;
    float m = 0.0f, s = 1.0f;
    if (mode != 2) {
      m = -INFINITY;
      for (int e = 0; e < E; ++e) m = fmaxf(m, v[e]);
      float lanes[64];
      for (int l = 0; l < 64; ++l) {
        float ps = 0.0f;
        for (int e = l; e < E; e += 64) ps += orc_expf(v[e] - m);
        lanes[l] = ps;
      }
      s = orc_wave_sum(lanes);
    }
    for (int e = 0; e < E; ++e) key[e] = mode == 1 ? round_dt(orc_expf(v[e] - m) / s, pdt) : v[e];
    memset(used, 0, (size_t)E);
    float sel[64] = {0};
    for (int j = 0; j < k; ++j) {
      int best = -1;
      uint32_t bi = 0;
      for (int e = 0; e < E; ++e) {
        if (used[e]) continue;
        const uint32_t im = key_image(key[e]);
        if (best < 0 || im > bi) {
          best = e;
          bi = im;
        }
      }
      used[best] = 1;
      ids[(int64_t)t * k + j] = best;
      sel[j] = key[best] == 0.0f ? 0.0f : key[best];
    }
    float p[64] = {0};
    for (int j = 0; j < k; ++j) {
      if (mode == 0) p[j] = orc_expf(sel[j] - m) / s;
      else if (mode == 1) p[j] = sel[j];
      else p[j] = orc_expf(sel[j] - sel[0]);
    }
    const float tot = orc_wave_sum(p);
    for (int j = 0; j < k; ++j) {
      float wj;
      if (mode == 0) wj = renorm ? p[j] / tot : p[j];
      else if (mode == 1) wj = renorm ? round_dt(p[j] / round_dt(tot, pdt), pdt) : p[j];
      else wj = p[j] / tot;
      w[(int64_t)t * k + j] = round_dt(wj, wdt);
    }
  }
  free(key);
  free(used);
  return 0;
}

/* --------------------------------------------------------------- expert
 * One expert (or the dense shared expert) on M rows, double accumulation:
 *   gu = x . W13^T (+ b13)                 fused_fp8_linear.py:172 (fp32 gu)
 *   h  = act(gu[:, :I], gu[:, I:])         fused_moe.py:53-61,145 / gpt_oss/__init__.py:306-310
 *   h rounded to bf16 when h_bf16         fused_fp8_linear.py:174 (.to(out_dtype))
 *   y  = h . W2^T (+ b2)                   fused_fp8_linear.py:175
 * x: fp32 [M, H] (exact bf16 values), y: double [M, H]. */
static double act_d(int act, double g, double u, double alpha, double limit) {
  switch (act) {
    case A_SILU: return g / (1.0 + exp(-g)) * u;
    case A_GELU: return 0.5 * g * (1.0 + erf(g / sqrt(2.0))) * u;
    case A_RELU: return (g > 0.0 ? g : 0.0) * u;
    default: {
      if (g > limit) g = limit;
      if (u > limit) u = limit;
      if (u < -limit) u = -limit;
      const double glu = g / (1.0 + exp(-alpha * g));
      return (u + 1.0) * glu;
    }
  }
}

/* The activation alone, for the tests that pin it against library routines. */
double orc_act(int act, double g, double u, double alpha, double limit) { return act_d(act, g, u, alpha, limit); }

static float bias_val(const orc_proj* P, int slot, int n) {
  if (P->bias == NULL) return 0.0f;
  const char* b = (const char*)P->bias + (int64_t)slot * P->bias_stride;
  return load_dt(b, n, P->bias_dtype);
}

/* w13/w2 deq to fp32 once per call (rows of this slot), then the SwiGLU. */
int orc_expert_forward(const orc_proj* w13, const orc_proj* w2, int slot, const float* x, int M, int act,
                       float alpha, float limit, int h_bf16, double* y) {
  const int H = w13->K, I2 = w13->N, I = I2 / 2;
  if (w2->N != H || w2->K != I) return -2;
  float* W13 = (float*)malloc(sizeof(float) * (size_t)I2 * H);
  float* W2 = (float*)malloc(sizeof(float) * (size_t)H * I);
  double* h = (double*)malloc(sizeof(double) * (size_t)I);
  if (!W13 || !W2 || !h) return -1;
  orc_dequant(w13, slot, W13);
  orc_dequant(w2, slot, W2);
  for (int m = 0; m < M; ++m) {
    const float* xr = x + (int64_t)m * H;
    for (int i = 0; i < I; ++i) {
      double g = 0.0, u = 0.0;
      const float* wg = W13 + (int64_t)i * H;
      const float* wu = W13 + (int64_t)(I + i) * H;
      for (int k = 0; k < H; ++k) {
        g += (double)xr[k] * (double)wg[k];
        u += (double)xr[k] * (double)wu[k];
      }
      g += (double)bias_val(w13, slot, i);
      u += (double)bias_val(w13, slot, I + i);
      double hv = act_d(act, g, u, alpha, limit);
      if (h_bf16) hv = (double)orc_round_bf16((float)hv);
      h[i] = hv;
    }
    for (int n = 0; n < H; ++n) {
      double acc = 0.0;
      const float* wr = W2 + (int64_t)n * I;
      for (int i = 0; i < I; ++i) acc += h[i] * (double)wr[i];
      y[(int64_t)m * H + n] = acc + (double)bias_val(w2, slot, n);
    }
  }
  free(W13);
  free(W2);
  free(h);
  return 0;
}

/* --------------------------------------------------------------- layer
 * Routed experts + combine for given routing, double accumulation:
 *   out[t] = sum_j w[t][j] * expert_{ids[t][j]}(x[t])   (+ shared_w[t] * shared(x[t]))
 * python/freetoken/models/qwen3_5_moe/__init__.py:1732-1737,1229,1252 and
 * python/freetoken/kernel/triton/fused_moe.py:129-161, with the reference's
 * bf16 running sum replaced by an exact-as-possible double sum.
 * slot_of_expert may be NULL (identity).  on_input: x is scaled by w (rounded
 * to bf16 when x_bf16) instead of the output (fused_moe.py:139-148). */
int orc_moe_experts(const orc_proj* w13, const orc_proj* w2, const int32_t* slot_of_expert, int E,
                    const float* x, int T, int topk, const int32_t* ids, const float* w, int act, float alpha,
                    float limit, int h_bf16, int on_input, int x_bf16, double* out) {
  const int H = w13->K;
  memset(out, 0, sizeof(double) * (size_t)T * H);
  int32_t* rows = (int32_t*)malloc(sizeof(int32_t) * (size_t)T * topk);
  float* xs = (float*)malloc(sizeof(float) * (size_t)T * topk * H);
  double* y = (double*)malloc(sizeof(double) * (size_t)T * topk * H);
  if (!rows || !xs || !y) return -1;
  for (int e = 0; e < E; ++e) {
    int M = 0;
    for (int t = 0; t < T; ++t)
      for (int j = 0; j < topk; ++j)
        if (ids[t * topk + j] == e) {
          rows[M] = t * topk + j;
          for (int k = 0; k < H; ++k) {
            float v = x[(int64_t)t * H + k];
            if (on_input) {
              v = v * w[t * topk + j];
              if (x_bf16) v = orc_round_bf16(v);
            }
            xs[(int64_t)M * H + k] = v;
          }
          ++M;
        }
    if (M == 0) continue;
    const int slot = slot_of_expert ? slot_of_expert[e] : e;
    int rc = orc_expert_forward(w13, w2, slot, xs, M, act, alpha, limit, h_bf16, y);
    if (rc != 0) return rc;
    for (int m = 0; m < M; ++m) {
      const int p = rows[m], t = p / topk;
      const double wt = on_input ? 1.0 : (double)w[p];
      for (int n = 0; n < H; ++n) out[(int64_t)t * H + n] += wt * y[(int64_t)m * H + n];
    }
  }
  free(rows);
  free(xs);
  free(y);
  return 0;
}
