// ftm_moe.hip -- the fused quantized MoE layer on gfx950.
//
// One layer forward is five launches on the caller's stream:
//   k_router   router GEMV  logits[t, e] = round(x[t] . G[e] (+ b[e]))
//              (one WG per expert row and 16-token block)
//   k_topk1    softmax / top-k / renorm, one wave per token, and compaction
//              of the routed experts (ascending id); one WG for T <= 256
//   k_topk     the same for larger T over many WGs; the last-arriving WG
//              compacts
//   k_stage_a  per (routed expert, 16-channel tile): gate and up rows of w13,
//              K split over the 4 waves, fused activation -> h (act dtype)
//   k_stage_b  per (expert, 64-column tile of H): w2 . h, bias, router weight,
//              written to the [T, k(+1), H] fp32 slot buffer
//   k_combine  out[t] = sum of the token's k(+1) slots in fixed order
// The shared expert (dense bf16) rides along as one more expert in stages A/B.
// No float atomics anywhere: the output is bitwise reproducible run to run.
//
// Reference semantics followed (file:line under /root/reference):
//   routing      python/freetoken/models/qwen3_5_moe/__init__.py:1224-1227,
//                python/freetoken/kernel/triton/fused_moe.py:91-97,
//                python/freetoken/models/gpt_oss/__init__.py:347-352
//   expert       python/freetoken/kernel/triton/fused_fp8_linear.py:154-175 (fp32 gu,
//                h rounded to the activation dtype, fp32 down projection)
//   clamped GLU  python/freetoken/models/gpt_oss/__init__.py:306-310
//   combine      python/freetoken/models/qwen3_5_moe/__init__.py:1732-1737,1252
//   shared       python/freetoken/models/qwen3_5_moe/__init__.py:1229,1752-1768
#include <math.h>

#include "ftm_layer.h"

#include <algorithm>
#include <mutex>

namespace ftm {

// ---------------------------------------------------------------- MXFP4 decode on scaled MFMAs
// The routed MXFP4 rows of stage A run on v_mfma_scale_f32_16x16x128_f8f6f4:
// the weights go in as they are stored (e2m1 nibbles, e8m0 block scales) and
// the activations as two e4m3 terms with e8m0 block scales (k_quant_mx), so
// no weight is decoded by the vector ALUs.  Operand layout of one 16 x 16 x
// 128 step (columns = 16 weight rows, K = one wave-load):
//   B (e2m1): lane l holds K [32 g, 32 g + 32) of column l % 16 (g = l / 16)
//             in its 4 low registers -- the 16 bytes a K-major wave-load
//             puts there -- and that block's scale in scale_b;
//   A (e4m3): lane l holds token row l % 16 at K [16 g, 16 g + 16) and
//             [64 + 16 g, 64 + 16 g + 16) (8 registers), and in scale_a the
//             scale of the row's block g (K [32 g, 32 g + 32)).
// One 32-element block of a token row (T rows of H bf16) per 4 lanes, 8
// elements a lane: with E = floor(log2 max|x|) the hi scale is 2^(E - 7), so
// the block maps into [-256, 256); hi = e4m3(x / s_hi) and lo = e4m3((x /
// s_hi - hi) * 16) with s_lo = s_hi / 16.  The residual of a bf16 value is
// exact in fp32 and, for |x| >= 2^(E - 13), exact in e4m3, so hi + lo is the
// input itself there (the smaller ones are off by at most 2^(E - 21)).
// Blocks past H are zeros; a block holding Inf or NaN gets NaN scales (0xff).
// Piece i (8 elements) of the T x H input; callers run whole quads of lanes
// (i and the piece count are multiples of 4 at every quad boundary).
__device__ __forceinline__ void quant_mx_piece(const uint16_t* __restrict__ x, int T, int H,
                                               uint8_t* __restrict__ xq, int i) {
  const int nq = (H + 127) / 128 * 16;  // 8-element pieces of a row, padding included
  if (i >= T * nq) return;  // whole quads (blocks) leave together
  const int t = i / nq, q = i - t * nq;
  const int k0 = 8 * q;
  u32x4 w = (u32x4){0u, 0u, 0u, 0u};
  if (k0 < H) w = *(const u32x4*)(x + (size_t)t * H + k0);  // H % 32 == 0: a block is whole or past the end
  float v[8];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    v[2 * j] = __uint_as_float(w[j] << 16);
    v[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
  }
  // largest |x| bit pattern of the block (Inf and NaN: >= 0x7f800000)
  int mb = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) mb = max(mb, (int)(__float_as_uint(v[j]) & 0x7fffffffu));
  mb = max(mb, dpp_i<kDppXor1>(mb));
  mb = max(mb, dpp_i<kDppXor2>(mb));
  // E + 120 clamped to >= 0 (amax < 2^-120 keeps |x / s_hi| < 2^8 as well)
  const uint32_t chi = (uint32_t)max((mb >> 23) - 7, 0);
  const uint32_t clo = chi >= 4u ? chi - 4u : 0u;
  const float inv = __uint_as_float((254u - chi) << 23);        // 1 / s_hi
  const float flo = __uint_as_float((127u + chi - clo) << 23);  // s_hi / s_lo
  uint32_t hw[2], lw[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const float s0 = v[4 * h] * inv, s1 = v[4 * h + 1] * inv, s2 = v[4 * h + 2] * inv, s3 = v[4 * h + 3] * inv;
    hw[h] = f32x4_to_e4m3(s0, s1, s2, s3);
    lw[h] = f32x4_to_e4m3((s0 - e4m3_at<0>(hw[h])) * flo, (s1 - e4m3_at<1>(hw[h])) * flo,
                          (s2 - e4m3_at<2>(hw[h])) * flo, (s3 - e4m3_at<3>(hw[h])) * flo);
  }
  const int c = q >> 4, p = q & 15;
  uint8_t* o = xq + (size_t)t * (size_t)((H + 127) / 128 * kMxChunk) + (size_t)c * kMxChunk;
  *(u32x2*)(o + 8 * p) = (u32x2){hw[0], hw[1]};
  *(u32x2*)(o + 128 + 8 * p) = (u32x2){lw[0], lw[1]};
  if ((p & 3) == 0) *(uint16_t*)(o + 256 + (p >> 1)) = (uint16_t)(mb < 0x7f800000 ? (chi | (clo << 8)) : 0xffffu);
  if (p == 0) *(u32x2*)(o + 264) = (u32x2){0u, 0u};
}

__host__ __device__ __forceinline__ int quant_mx_threads(int T, int H) { return T * ((H + 127) / 128 * 16); }

// The quantisation as a launch of its own (when no router launch carries it).
__global__ __launch_bounds__(kBlock) void k_quant_mx(const uint16_t* __restrict__ x, int T, int H,
                                                     uint8_t* __restrict__ xq) {
  quant_mx_piece(x, T, H, xq, blockIdx.x * kBlock + threadIdx.x);
}

// ============================================================== router GEMV
// logit = round_act( sum_k x[k]*G[k] (+ b) ).  The fp32 sum has a fixed order
// (per lane: 8-element chunks c = lane + 64*s in ascending s, fma in element
// order; then the xor-32/16/8/4/2/1 butterfly) that the C oracle replays with
// fmaf, so logits and therefore routing indices are bit-reproducible.
// Grid: (expert row [+ the shared-gate row], block of 16 tokens); wave w
// takes tokens 16*blockIdx.y + w + 4*i, i < 4.  Every load of a step group
// (4 chunk steps: the gate row and the wave's 4 token rows) is issued before
// any fma, with buffer loads that read zeros past the end, so one wave has
// 20 x 16 B per lane in flight.  Chunks past H are masked by a select.
constexpr int kRouterTPW = 4;  // tokens per wave
constexpr int kRouterSteps = 4;  // 512-element chunk steps per load group

// Logits of row r for tokens tb + ts i (i < NT), by one wave, NS chunk steps
// per load group (COH: stored device-coherent, for a reader in the same
// launch).  NT, ts and NS change which loads are in flight together, not the
// order of any sum.
template <bool COH = false, int NT = kRouterTPW, int NS = kRouterSteps>
__device__ __forceinline__ void router_row_tile(const LayerArgs& a, int r, int tb, int ts = 4) {
  const int E = a.L.num_experts, H = a.L.hidden, T = a.T;
  const void* grow = (r < E) ? (const void*)((const uint16_t*)a.L.gate_w + (size_t)r * H) : a.L.shared_gate;
  const int lane = threadIdx.x & 63;
  const Rsrc gres = make_rsrc(grow, (uint32_t)H * 2u);
  const Rsrc xres = make_rsrc(a.x, (uint32_t)T * (uint32_t)H * 2u);
  const int nsteps = (H + 511) / 512;
  float acc[NT];
#pragma unroll
  for (int i = 0; i < NT; ++i) acc[i] = 0.0f;
  for (int s0 = 0; s0 < nsteps; s0 += NS) {
    u32x4 gv[NS], xv[NS][NT];
#pragma unroll
    for (int q = 0; q < NS; ++q) {
      const int c = lane + 64 * (s0 + q);
      const bool ok = (s0 + q < nsteps) && (8 * c < H);
      gv[q] = bload16(gres, ok ? 16u * (uint32_t)c : kOOB);
#pragma unroll
      for (int i = 0; i < NT; ++i) {
        const int t = tb + ts * i;
        xv[q][i] = bload16(xres, (ok && t < T) ? ((uint32_t)t * (uint32_t)H + 8u * (uint32_t)c) * 2u : kOOB);
      }
    }
#pragma unroll
    for (int q = 0; q < NS; ++q) {
      const int c = lane + 64 * (s0 + q);
      const bool ok = (s0 + q < nsteps) && (8 * c < H);
      const uint32_t gw[4] = {gv[q].x, gv[q].y, gv[q].z, gv[q].w};
#pragma unroll
      for (int i = 0; i < NT; ++i) {
        const uint32_t xw[4] = {xv[q][i].x, xv[q][i].y, xv[q][i].z, xv[q][i].w};
        float t8 = acc[i];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          t8 = __builtin_fmaf(bf16_to_f32(xw[e] & 0xffffu), bf16_to_f32(gw[e] & 0xffffu), t8);
          t8 = __builtin_fmaf(bf16_to_f32(xw[e] >> 16), bf16_to_f32(gw[e] >> 16), t8);
        }
        acc[i] = ok ? t8 : acc[i];
      }
    }
  }
#pragma unroll
  for (int i = 0; i < NT; ++i) {
    const float v = wave_sum(acc[i]);
    const int t = tb + ts * i;
    if (lane == 0 && t < T) {
      float z = v;
      if (r < E && a.L.gate_b != nullptr) z = v + bf16_to_f32(((const uint16_t*)a.L.gate_b)[r]);
      if constexpr (COH)
        store_dev(&a.logits[(size_t)t * (E + 1) + r], round_to(z, a.L.act_dtype));
      else
        a.logits[(size_t)t * (E + 1) + r] = round_to(z, a.L.act_dtype);
    }
  }
}

// Workgroups past `rows` quantise the input for the MXFP4 scaled-MFMA stage
// A instead (quant_mx_piece), off its critical path: quantisation block
// (x - rows) * gridDim.y + y.
__device__ __forceinline__ void router_quant_block(const LayerArgs& a, int qb) {
  quant_mx_piece((const uint16_t*)a.x, a.T, a.L.hidden, a.xq, qb * kBlock + threadIdx.x);
}

// NT = 1: wave w takes token 4 blockIdx.y + w alone, with every chunk step of
// the row in one load group (a 2880-wide row is 6 steps: one round trip
// instead of two), while the grid stays within kRouterOneMaxWgs workgroups.
// Measured on MI355X against four tokens per wave (us): C4 (32 rows) T=1 /
// 17 / 32 / 64 / 128 2.9 / 3.3 / 3.3 / 3.7 / 4.9 against 4.8 / 5.8 / 5.9 / 5.9 /
// 6.0; C2 (128 rows) T=1 2.8 against 3.7, T=17 3.8 against 4.4, T=32 4.5 both,
// T=64 6.6 against 5.5; C3 (257 rows) T=1 2.8 against 4.0, T=17 5.2 against
// 5.5, T=32 7.3 against 6.0.
constexpr int kRouterOneMaxWgs = 1300;
template <int NT>
__global__ __launch_bounds__(kBlock) void k_router(const LayerArgs a, int row_begin, int rows) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if ((int)blockIdx.x >= rows) {
    router_quant_block(a, ((int)blockIdx.x - rows) * (int)gridDim.y + (int)blockIdx.y);
    return;
  }
  if constexpr (NT == 1) {
    const int t = 4 * (int)blockIdx.y + wave;
    if (t < a.T) router_row_tile<false, 1, 8>(a, row_begin + blockIdx.x, t);
  } else {
    router_row_tile(a, row_begin + blockIdx.x, blockIdx.y * 4 * kRouterTPW + wave);
  }
}

// Large T: one WG per (8 expert rows, 16 tokens), so x is read once per 8
// rows instead of once per row.  Every (token, row) logit keeps k_router's
// arithmetic exactly: lane l accumulates chunks c = l, l + 64, ... (8
// elements each, in order) with one fma chain, and the wave sums the 64
// partials with the same xor-32..1 butterfly (wave_sum).
constexpr int kRouterRB = 8;   // expert rows per WG
constexpr int kRouterMinT = 64;  // from here on k_router_rows (x re-reads dominate k_router) ...
// ... once k_router's input re-reads (rows x T x H elements, one pass of x per
// row) pass 40 M elements.  Measured on MI355X, k_router against
// k_router_rows in us: C4 (32 rows, H 2880) T=64/128/256 5.7/5.8/8.5 against
// 9.8/9.8/10.0, T=512 13.0 against 11.9; C2 (128 rows) T=64/128 5.2/6.9
// against 7.4/7.5; C3 (257 rows) T=64 7.5 against 7.9, T=128 11.2 against 9.2.
constexpr double kRouterRowsMinElems = 40e6;
__host__ __forceinline__ bool router_by_rows(int rows, int T, int H) {
  return T >= kRouterMinT && (double)rows * T * H > kRouterRowsMinElems;
}

// One level of the transposing butterfly: lanes with bit M set keep values
// [N, 2N), the others [0, N); each adds the partner's copy of what it keeps.
template <int M, int N>
__device__ __forceinline__ void router_halve(float (&v)[32], int lane) {
  const bool up = (lane & M) != 0;
#pragma unroll
  for (int q = 0; q < N; ++q) {
    const float mine = up ? v[q + N] : v[q];
    const float give = up ? v[q] : v[q + N];
    v[q] = mine + __shfl_xor(give, M);
  }
}

// Logits of rows [r0, r0 + kRouterRB) (below row_end) for tokens [t0, t0 +
// kRouterTPW), by one wave.
__device__ __forceinline__ void router_rows_tile(const LayerArgs& a, int r0, int row_end, int t0) {
  const int E = a.L.num_experts, H = a.L.hidden, T = a.T;
  const int lane = threadIdx.x & 63;
  Rsrc gres[kRouterRB];
#pragma unroll
  for (int j = 0; j < kRouterRB; ++j) {
    const int r = r0 + j;
    const void* grow = r < E ? (const void*)((const uint16_t*)a.L.gate_w + (size_t)r * H) : a.L.shared_gate;
    gres[j] = make_rsrc(grow, r < row_end ? (uint32_t)H * 2u : 0u);
  }
  const Rsrc xres = make_rsrc(a.x, (uint32_t)T * (uint32_t)H * 2u);
  const int nq = (H / 8 + 63) / 64;
  float acc[kRouterTPW][kRouterRB];
#pragma unroll
  for (int i = 0; i < kRouterTPW; ++i)
#pragma unroll
    for (int j = 0; j < kRouterRB; ++j) acc[i][j] = 0.0f;
  // chunk q in gc/xc while chunk q + 1 loads into gn/xn
  u32x4 gc[kRouterRB], xc[kRouterTPW], gn[kRouterRB], xn[kRouterTPW];
  auto load = [&](int q, u32x4 (&g)[kRouterRB], u32x4 (&x)[kRouterTPW]) {
    const int c = lane + 64 * q;
    const bool ok = q < nq && 8 * c < H;
#pragma unroll
    for (int j = 0; j < kRouterRB; ++j) g[j] = bload16(gres[j], ok ? 16u * (uint32_t)c : kOOB);
#pragma unroll
    for (int i = 0; i < kRouterTPW; ++i) {
      const int t = t0 + i;
      x[i] = bload16(xres, (ok && t < T) ? ((uint32_t)t * (uint32_t)H + 8u * (uint32_t)c) * 2u : kOOB);
    }
  };
  load(0, gc, xc);
  for (int q = 0; q < nq; ++q) {
    load(q + 1, gn, xn);
    const bool ok = 8 * (lane + 64 * q) < H;
    float xf[kRouterTPW][8];
#pragma unroll
    for (int i = 0; i < kRouterTPW; ++i) {
      const uint32_t w4[4] = {xc[i].x, xc[i].y, xc[i].z, xc[i].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        xf[i][2 * e] = bf16_to_f32(w4[e] & 0xffffu);
        xf[i][2 * e + 1] = bf16_to_f32(w4[e] >> 16);
      }
    }
#pragma unroll
    for (int j = 0; j < kRouterRB; ++j) {
      const uint32_t w4[4] = {gc[j].x, gc[j].y, gc[j].z, gc[j].w};
      float gf[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        gf[2 * e] = bf16_to_f32(w4[e] & 0xffffu);
        gf[2 * e + 1] = bf16_to_f32(w4[e] >> 16);
      }
#pragma unroll
      for (int i = 0; i < kRouterTPW; ++i) {
        float t8 = acc[i][j];
#pragma unroll
        for (int e = 0; e < 8; ++e) t8 = __builtin_fmaf(xf[i][e], gf[e], t8);
        acc[i][j] = ok ? t8 : acc[i][j];
      }
    }
#pragma unroll
    for (int j = 0; j < kRouterRB; ++j) gc[j] = gn[j];
#pragma unroll
    for (int i = 0; i < kRouterTPW; ++i) xc[i] = xn[i];
  }
  // 32 butterfly sums at once: at xor level m a lane keeps the half of its
  // values whose index bit matches its lane bit and adds the partner's copy
  // (sent by the partner), so every value sees the pairs of wave_sum (xor 32,
  // 16, 8, 4, 2, then 1) and the same bits, in 16+8+4+2+1+1 shuffles.
  static_assert(kRouterTPW * kRouterRB == 32, "one value per lane pair after 5 halvings");
  float v[32];
#pragma unroll
  for (int i = 0; i < kRouterTPW; ++i)
#pragma unroll
    for (int j = 0; j < kRouterRB; ++j) v[i * kRouterRB + j] = acc[i][j];
  router_halve<32, 16>(v, lane);
  router_halve<16, 8>(v, lane);
  router_halve<8, 4>(v, lane);
  router_halve<4, 2>(v, lane);
  router_halve<2, 1>(v, lane);
  const float tot = v[0] + __shfl_xor(v[0], 1);
  // lane bits 5..1 name the value this lane holds: index = bit5*16 + bit4*8 + ... + bit1
  const int idx = ((lane >> 5) & 1) * 16 + ((lane >> 4) & 1) * 8 + ((lane >> 3) & 1) * 4 + ((lane >> 2) & 1) * 2 +
                  ((lane >> 1) & 1);
  const int t = t0 + idx / kRouterRB, r = r0 + idx % kRouterRB;
  if ((lane & 1) == 0 && t < T && r < row_end) {
    float z = tot;
    if (r < E && a.L.gate_b != nullptr) z = tot + bf16_to_f32(((const uint16_t*)a.L.gate_b)[r]);
    a.logits[(size_t)t * (E + 1) + r] = round_to(z, a.L.act_dtype);
  }
}

__global__ __launch_bounds__(kBlock) void k_router_rows(const LayerArgs a, int row_begin, int row_end) {
  const int wave = threadIdx.x >> 6;
  const int rb = (row_end - row_begin + kRouterRB - 1) / kRouterRB;
  if ((int)blockIdx.x >= rb) {  // as in k_router
    router_quant_block(a, ((int)blockIdx.x - rb) * (int)gridDim.y + (int)blockIdx.y);
    return;
  }
  router_rows_tile(a, row_begin + blockIdx.x * kRouterRB, row_end, blockIdx.y * 4 * kRouterTPW + wave * kRouterTPW);
}

// ============================================================== top-k + grouping

// Selection keys: (key desc, expert id asc) packed into one u64 that orders
// the same way -- the key's order-preserving bit image (+0 for either zero,
// the bottom for NaN) above ~expert.  0 is below every real key.
__device__ __forceinline__ uint64_t pack_key(float v, int e) {
  uint32_t b = __float_as_uint(v == 0.0f ? 0.0f : v);
  b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  b = (v != v) ? 0u : b;
  return ((uint64_t)b << 32) | (uint32_t)~(uint32_t)e;
}
__device__ __forceinline__ float key_value(uint64_t k) {
  const uint32_t b = (uint32_t)(k >> 32);
  return __uint_as_float((b & 0x80000000u) ? (b & 0x7fffffffu) : ~b);
}
__device__ __forceinline__ int key_expert(uint64_t k) { return (int)~(uint32_t)k; }

// The same order in 32 bits for bf16-exact keys (the low 16 bits of the key
// are zero, so the top half of its image decides): image >> 16 above ~expert
// (16 bits, E <= 65536).
__device__ __forceinline__ uint32_t pack_key32(float v, int e) {
  return (uint32_t)(pack_key(v, e) >> 48) << 16 | (~(uint32_t)e & 0xffffu);
}
__device__ __forceinline__ float key32_value(uint32_t k) {
  const uint32_t hi = k >> 16;
  // the image's low half: 0 for non-negative keys, 0xffff for negative ones
  const uint32_t b = (hi << 16) | ((hi & 0x8000u) ? 0u : 0xffffu);
  return __uint_as_float((b & 0x80000000u) ? (b & 0x7fffffffu) : ~b);
}
__device__ __forceinline__ int key32_expert(uint32_t k) { return (int)(~k & 0xffffu); }

template <int CTRL>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t x) {
  const uint32_t lo = (uint32_t)dpp_i<CTRL>((int)(uint32_t)x);
  const uint32_t hi = (uint32_t)dpp_i<CTRL>((int)(uint32_t)(x >> 32));
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t umax64(uint64_t a, uint64_t b) { return a > b ? a : b; }

// Wave max of a u64 (DPP within rows, v_readlane across rows); all lanes get it.
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t x) {
  x = umax64(x, dpp_u64<kDppXor1>(x));
  x = umax64(x, dpp_u64<kDppXor2>(x));
  x = umax64(x, dpp_u64<kDppHalfMirror>(x));
  x = umax64(x, dpp_u64<kDppMirror>(x));
  uint64_t r[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)x, 16 * q);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(x >> 32), 16 * q);
    r[q] = ((uint64_t)hi << 32) | lo;
  }
  return umax64(umax64(r[0], r[1]), umax64(r[2], r[3]));
}

// Wave max of a u32 (DPP within rows, v_readlane across rows); all lanes get it.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t x) {
  x = max(x, (uint32_t)dpp_i<kDppXor1>((int)x));
  x = max(x, (uint32_t)dpp_i<kDppXor2>((int)x));
  x = max(x, (uint32_t)dpp_i<kDppHalfMirror>((int)x));
  x = max(x, (uint32_t)dpp_i<kDppMirror>((int)x));
  const uint32_t r0 = (uint32_t)__builtin_amdgcn_readlane((int)x, 0), r1 = (uint32_t)__builtin_amdgcn_readlane((int)x, 16);
  const uint32_t r2 = (uint32_t)__builtin_amdgcn_readlane((int)x, 32), r3 = (uint32_t)__builtin_amdgcn_readlane((int)x, 48);
  return max(max(r0, r1), max(r2, r3));
}

// Wave max of a u32 in every lane without a scalar round trip: DPP within
// rows, then the gfx950 row swaps (v_permlane16_swap: rows 0 <-> 1, 2 <-> 3;
// v_permlane32_swap: halves) -- eight VALU instructions.
__device__ __forceinline__ uint32_t wave_max_u32_v(uint32_t x) {
  x = max(x, (uint32_t)dpp_i<kDppXor1>((int)x));
  x = max(x, (uint32_t)dpp_i<kDppXor2>((int)x));
  x = max(x, (uint32_t)dpp_i<kDppHalfMirror>((int)x));
  x = max(x, (uint32_t)dpp_i<kDppMirror>((int)x));
  const auto r16 = __builtin_amdgcn_permlane16_swap(x, x, false, false);
  x = max((uint32_t)r16[0], (uint32_t)r16[1]);
  const auto r32 = __builtin_amdgcn_permlane32_swap(x, x, false, false);
  return max((uint32_t)r32[0], (uint32_t)r32[1]);
}

__device__ __forceinline__ void cas_desc(uint64_t& a, uint64_t& b) {
  const uint64_t hi = umax64(a, b), lo = a > b ? b : a;
  a = hi;
  b = lo;
}
// Descending sorting networks for a lane's candidates (4: 5 comparators,
// 8: Batcher's 19).
template <int NV>
__device__ __forceinline__ void sort_desc(uint64_t (&k)[NV]) {
  if constexpr (NV == 4) {
    cas_desc(k[0], k[1]); cas_desc(k[2], k[3]);
    cas_desc(k[0], k[2]); cas_desc(k[1], k[3]);
    cas_desc(k[1], k[2]);
  } else {
    static_assert(NV == 8, "4 or 8 candidates per lane");
    cas_desc(k[0], k[1]); cas_desc(k[2], k[3]); cas_desc(k[4], k[5]); cas_desc(k[6], k[7]);
    cas_desc(k[0], k[2]); cas_desc(k[1], k[3]); cas_desc(k[4], k[6]); cas_desc(k[5], k[7]);
    cas_desc(k[1], k[2]); cas_desc(k[5], k[6]);
    cas_desc(k[0], k[4]); cas_desc(k[1], k[5]); cas_desc(k[2], k[6]); cas_desc(k[3], k[7]);
    cas_desc(k[2], k[4]); cas_desc(k[3], k[5]);
    cas_desc(k[1], k[2]); cas_desc(k[3], k[4]); cas_desc(k[5], k[6]);
  }
}

__device__ __forceinline__ void cas_desc32(uint32_t& a, uint32_t& b) {
  const uint32_t hi = max(a, b), lo = min(a, b);
  a = hi;
  b = lo;
}
template <int NV>
__device__ __forceinline__ void sort_desc32(uint32_t (&k)[NV]) {
  if constexpr (NV == 4) {
    cas_desc32(k[0], k[1]); cas_desc32(k[2], k[3]);
    cas_desc32(k[0], k[2]); cas_desc32(k[1], k[3]);
    cas_desc32(k[1], k[2]);
  } else {
    cas_desc32(k[0], k[1]); cas_desc32(k[2], k[3]); cas_desc32(k[4], k[5]); cas_desc32(k[6], k[7]);
    cas_desc32(k[0], k[2]); cas_desc32(k[1], k[3]); cas_desc32(k[4], k[6]); cas_desc32(k[5], k[7]);
    cas_desc32(k[1], k[2]); cas_desc32(k[5], k[6]);
    cas_desc32(k[0], k[4]); cas_desc32(k[1], k[5]); cas_desc32(k[2], k[6]); cas_desc32(k[3], k[7]);
    cas_desc32(k[2], k[4]); cas_desc32(k[3], k[5]);
    cas_desc32(k[1], k[2]); cas_desc32(k[3], k[4]); cas_desc32(k[5], k[6]);
  }
}

// Routing of token t by one wave: lanes j < k end with (sel_e, sel_w).
// NV = candidates per lane (E <= 64 * NV).
// The router's logits of token t, lane l holding experts l + 64 i (issued
// ahead of use by the multi-token top-k loop).
template <int NV, bool COH = false>
__device__ __forceinline__ void route_load(const LayerArgs& a, int t, uint32_t (&raw)[NV]) {
  const int E = a.L.num_experts;
  const int lane = threadIdx.x & 63;
  const Rsrc lres = make_rsrc(a.logits, (uint32_t)a.T * (uint32_t)(E + 1) * 4u);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int e = lane + 64 * i;
    const uint32_t off = (e < E && t < a.T) ? ((uint32_t)t * (uint32_t)(E + 1) + (uint32_t)e) * 4u : kOOB;
    raw[i] = COH ? bload4_dev(lres, off) : bload4(lres, off);
  }
}

// Caller routing may list one expert more than once for a token; the
// reference's per-pair loop (python/freetoken/models/qwen3_5_moe/__init__.py:
// 1732-1737) then applies the expert once per listing.  The repeats' weights
// are added, in listing order, to the expert's first listing and the repeats
// become pairs without an expert: y * ((w1 + w2) + ...) for y * w1 + y * w2 +
// ..., and no expert's list can hold more than T pairs.  Whole wave; lanes >= k
// hold sel_e = -1.
__device__ __forceinline__ void fold_repeats(int& sel_e, float& sel_w, int E, int k) {
  const int lane = threadIdx.x & 63;
  const bool valid = lane < k && sel_e >= 0 && sel_e < E;
  bool repeat = false;
  float tot = sel_w;
  for (int j = 0; j < k; ++j) {
    const int ej = __shfl(sel_e, j);
    const float wj = __shfl(sel_w, j);
    if (valid && ej == sel_e) {
      repeat = repeat || j < lane;
      tot = j > lane ? tot + wj : tot;
    }
  }
  if (valid) {
    sel_e = repeat ? -1 : sel_e;
    sel_w = repeat ? 0.0f : tot;
  }
}

// use_pre: take the router logits of t from pre (route_load, router path only).
template <int MODE, int NV, bool COH = false>
__device__ __forceinline__ void route_token_pre(const LayerArgs& a, int t, const void* logits_in, int logits_dt,
                                                const int32_t* ids_in, const float* w_in, float* logits_out,
                                                int& sel_e, float& sel_w, bool use_pre,
                                                const uint32_t (&pre)[NV]) {
  const int E = a.L.num_experts, k = a.L.topk;
  const int lane = threadIdx.x & 63;
  const int act_dt = a.L.act_dtype;
  sel_e = -1;
  sel_w = 0.0f;
  if (ids_in != nullptr) {
    if (lane < k) {
      sel_e = ids_in[(size_t)t * k + lane];
      sel_w = w_in[(size_t)t * k + lane];
    }
    fold_repeats(sel_e, sel_w, E, k);
    return;
  }
  const int pdt = logits_in ? logits_dt : act_dt;  // dtype the probabilities live in (LOWP)
  float v[NV], key[NV];
  float vmax = -INFINITY;
  if (logits_in == nullptr) {
    // the router's [T, E+1] fp32 logits: all loads issued before any use
    uint32_t raw[NV];
    if (use_pre) {
#pragma unroll
      for (int i = 0; i < NV; ++i) raw[i] = pre[i];
    } else {
      route_load<NV, COH>(a, t, raw);
    }
#pragma unroll
    for (int i = 0; i < NV; ++i) v[i] = (lane + 64 * i < E) ? __uint_as_float(raw[i]) : -INFINITY;
  } else {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int e = lane + 64 * i;
      v[i] = (e < E) ? load_scalar(logits_in, (size_t)t * E + e, logits_dt) : -INFINITY;
    }
  }
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int e = lane + 64 * i;
    if (logits_out && e < E) logits_out[(size_t)t * E + e] = v[i];
    vmax = fmaxf(vmax, v[i]);
  }
  float m = 0.0f, s = 1.0f;
  if (MODE != FTM_ROUTE_TOPK_SOFTMAX) {
    m = wave_max_dpp(vmax);
    float ps = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i)
      if (lane + 64 * i < E) ps += ftm_expf(v[i] - m);
    s = wave_sum_dpp(ps);
  }
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    if (MODE == FTM_ROUTE_SOFTMAX_TOPK_LOWP)
      key[i] = (lane + 64 * i < E) ? round_to(ftm_expf(v[i] - m) / s, pdt) : -INFINITY;
    else
      key[i] = v[i];
  }
  // Each lane sorts its candidates; k rounds take the wave max of the lanes'
  // heads, and the lane holding it pops its head.  When every key is
  // bf16-exact (router logits and LOWP probabilities are rounded to bf16) the
  // (key, expert) pair packs into 32 bits with the same order, and each round
  // is a 32-bit max.
  bool exact16 = true;
#pragma unroll
  for (int i = 0; i < NV; ++i)
    exact16 &= (lane + 64 * i >= E) | (key[i] != key[i]) | ((__float_as_uint(key[i]) & 0xffffu) == 0u);
  float top0;
  if (__all(exact16)) {
    uint32_t lst[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) lst[i] = (lane + 64 * i < E) ? pack_key32(key[i], lane + 64 * i) : 0u;
    sort_desc32<NV>(lst);
    // k rounds: the wave max of the lanes' heads is the next key (in every
    // lane), the lane holding it pops its head
    uint32_t mine = 0u;
    const uint32_t first = wave_max_u32_v(lst[0]);
    for (int j = 0; j < k; ++j) {
      const uint32_t best = j == 0 ? first : wave_max_u32_v(lst[0]);
      mine = lane == j ? best : mine;
      // the lane holding the key pops its head: one select per candidate,
      // written out so the shift stays NV v_cndmask (left to itself the
      // compiler tracks the rotation with index compares, ~2x the VALU); the
      // s_nop gives the VALU-written mask the two wait states the compiler
      // puts between a v_cmp and its v_cndmask on this target
      const uint64_t pop = __ballot(lst[0] == best);
      asm volatile("s_nop 1\n\tv_cndmask_b32_e64 %0, %0, %1, %2" : "+v"(lst[0]) : "v"(lst[1]), "s"(pop));
#pragma unroll
      for (int i = 1; i + 1 < NV; ++i)
        asm volatile("v_cndmask_b32_e64 %0, %0, %1, %2" : "+v"(lst[i]) : "v"(lst[i + 1]), "s"(pop));
      asm volatile("v_cndmask_b32_e64 %0, %0, 0, %1" : "+v"(lst[NV - 1]) : "s"(pop));
    }
    top0 = key32_value(first);
    if (lane < k) {
      sel_e = key32_expert(mine);
      sel_w = key32_value(mine);  // the key; converted to a weight below
    }
  } else {
    uint64_t lst[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) lst[i] = (lane + 64 * i < E) ? pack_key(key[i], lane + 64 * i) : 0ull;
    sort_desc<NV>(lst);
    uint64_t mine = 0ull, first = 0ull;
    for (int j = 0; j < k; ++j) {
      const uint64_t best = wave_max_u64(lst[0]);
      first = j == 0 ? best : first;
      mine = lane == j ? best : mine;
      const bool pop = lst[0] == best;
#pragma unroll
      for (int i = 0; i + 1 < NV; ++i) lst[i] = pop ? lst[i + 1] : lst[i];
      lst[NV - 1] = pop ? 0ull : lst[NV - 1];
    }
    top0 = key_value(first);
    if (lane < k) {
      sel_e = key_expert(mine);
      sel_w = key_value(mine);  // the key; converted to a weight below
    }
  }
  float p = 0.0f;
  if (lane < k) {
    if (MODE == FTM_ROUTE_SOFTMAX_TOPK) p = ftm_expf(sel_w - m) / s;
    else if (MODE == FTM_ROUTE_SOFTMAX_TOPK_LOWP) p = sel_w;
    else p = ftm_expf(sel_w - top0);
  }
  const float tot = wave_sum_dpp(lane < k ? p : 0.0f);
  if (MODE == FTM_ROUTE_SOFTMAX_TOPK) {
    sel_w = a.L.renormalize ? p / tot : p;
  } else if (MODE == FTM_ROUTE_SOFTMAX_TOPK_LOWP) {
    sel_w = a.L.renormalize ? round_to(p / round_to(tot, pdt), pdt) : p;
  } else {
    sel_w = p / tot;
  }
  sel_w = round_to(sel_w, act_dt);
}

template <int MODE, int NV, bool COH = false>
__device__ __forceinline__ void route_token(const LayerArgs& a, int t, const void* logits_in, int logits_dt,
                                            const int32_t* ids_in, const float* w_in, float* logits_out,
                                            int& sel_e, float& sel_w) {
  const uint32_t none[NV] = {};
  route_token_pre<MODE, NV, COH>(a, t, logits_in, logits_dt, ids_in, w_in, logits_out, sel_e, sel_w, false, none);
}

// Zero the slot rows of token t's pairs that have no expert (caller routing
// with id < 0: no stage writes them, and k_combine sums every slot).  Called
// by the whole wave; skip: this lane's pair (lane < k) has no expert.
__device__ __forceinline__ void zero_skipped_slots(const LayerArgs& a, int t, bool skip) {
  uint64_t m = __ballot(skip);
  const int H = a.L.hidden, lane = threadIdx.x & 63;
  while (m) {
    const int j = __builtin_ctzll(m);
    m &= m - 1;
    float* row = a.ybuf + (size_t)(t * a.KP + j) * H;
    if (H % 4 == 0) {
      for (int i = lane; i < H / 4; i += 64) ((f32x4*)row)[i] = (f32x4){0.f, 0.f, 0.f, 0.f};
    } else {
      for (int i = lane; i < H; i += 64) row[i] = 0.0f;
    }
  }
}

// Record token t's selection: weights, ids, and one list entry per pair in
// the expert's list (cnt: per-expert counters, in LDS or global memory;
// s_first: null, or an LDS copy of each list's first kRecPairs entries).
__device__ __forceinline__ void emit_token(const LayerArgs& a, int t, int sel_e, float sel_w, int32_t* ids_out,
                                           float* w_out, int32_t* cnt, int32_t* s_first = nullptr,
                                           const float* sh_logit = nullptr) {
  const int E = a.L.num_experts, k = a.L.topk, T = a.T, KP = a.KP;
  const int lane = threadIdx.x & 63;
  bool listed = false;
  if (lane < k) {
    const int p = t * KP + lane;
    if (sel_e >= 0 && sel_e < E) {
      a.wts[p] = sel_w;
      a.ids[(size_t)t * k + lane] = sel_e;
      if (ids_out) ids_out[(size_t)t * k + lane] = sel_e;
      if (w_out) w_out[(size_t)t * k + lane] = sel_w;
      const int pos = atomicAdd(&cnt[sel_e], 1);
      if (pos < T) {
        store_dev(&a.lists[(size_t)sel_e * T + pos], p);  // k_topk's last workgroup reads the lists
        if (s_first != nullptr && pos < kRecPairs) s_first[sel_e * kRecPairs + pos] = p;
        listed = true;
      } else {  // more than T pairs for one expert (fold_repeats rules it out): dropped, flagged
        atomicSub(&cnt[sel_e], 1);
        atomicOr(&a.ctrl[kCtrlError], 4);
        a.ids[(size_t)t * k + lane] = -1;
      }
    } else {
      // caller-supplied id < 0: the pair has no expert in this call (it is in
      // no list and its slot is zeroed below); >= E: an error
      a.ids[(size_t)t * k + lane] = -1;
      if (sel_e >= E) atomicOr(&a.ctrl[kCtrlError], 2);
    }
  }
  // every slot no stage writes is zeroed (k_combine sums all of a token's slots)
  zero_skipped_slots(a, t, lane < k && !listed);
  if (lane == 0 && a.L.shared_inter > 0) {
    // k_route_topk1: another workgroup's logit (sh_logit: loaded with the routing logits)
    const float sl = sh_logit != nullptr ? *sh_logit : load_dev(&a.logits[(size_t)t * (E + 1) + E]);
    a.wts[t * KP + k] = round_to(ftm_sigmoidf(sl), a.L.act_dtype);
  }
}

// Compaction of the routed experts (ascending id) by one workgroup of NW
// waves from the per-expert counters; counters are cleared when global.
// s_first: null (records read the lists' heads from global memory), or the
// LDS copy emit_token kept.
template <int NW>
__device__ __forceinline__ void compact_experts(const LayerArgs& a, int32_t* cnt, bool global_cnt, int* s_wsum,
                                                const int32_t* s_first = nullptr) {
  const int E = a.L.num_experts;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  int running = 0;
  for (int base = 0; base < E; base += NW * 64) {
    const int e = base + threadIdx.x;
    int c = 0;
    if (e < E) c = global_cnt ? __hip_atomic_load(&cnt[e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : cnt[e];
    c = c < a.T ? c : a.T;  // a list holds at most T pairs (the overflow was flagged)
    const bool f = c > 0;
    const uint64_t mask = __ballot(f);
    const int pre = __popcll(mask & ((1ull << lane) - 1ull));
    if (lane == 0) s_wsum[wave] = __popcll(mask);
    __syncthreads();
    int wpre = 0, tot = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      if (w < wave) wpre += s_wsum[w];
      tot += s_wsum[w];
    }
    if (f) {
      const int u = running + wpre + pre;
      a.uniq[u] = e;
      a.ucnt[u] = c;
    }
    if (f && (a.T <= kRecMaxT || a.lean)) {
      // work record for the LDS-activation stages: the list of expert e is
      // complete here
      const int u = running + wpre + pre;
      const int32_t* list = a.lists + (size_t)e * a.T;
      int rec[kRecWords];
      rec[0] = e;
      rec[1] = c;
      rec[2] = a.L.slot_of_expert ? a.L.slot_of_expert[e] : e;
#pragma unroll
      for (int i = 0; i < kRecPairs; ++i)
        rec[3 + i] = i < c ? (s_first != nullptr ? s_first[e * kRecPairs + i] : load_dev(&list[i])) : -1;
      rec[kRecWords - 1] = 0;
      int32_t* dst = a.recs + (size_t)u * kRecWords;
#pragma unroll
      for (int i = 0; i < kRecWords; ++i) dst[i] = rec[i];
    }
    if (global_cnt && e < E) cnt[e] = 0;
    running += tot;
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    a.ctrl[kCtrlNRouted] = running;
    a.ctrl[kCtrlNU] = running + (a.L.shared_inter > 0 ? 1 : 0);
  }
}

// Small batches: one workgroup of 16 waves routes every token (wave w takes
// t = w, w + 16, ...) with per-expert counters in LDS, then compacts.  No
// cross-workgroup traffic, so no device-scope fences.  Measured on MI355X
// (C3, 256 experts, top-8): 6.1 us at T <= 4 against 7.9-8.9 us for the
// multi-workgroup kernel, 8.1 against 9.3 at 12, 8.9 against 9.2 at 16;
// they tie at 20 and from 24 on the multi-workgroup kernel wins (9.8 vs 13.3
// us at 32, 10.0 vs 17.3 at 48).
constexpr int kTopk1Waves = 16;
constexpr int kTopk1MaxT = 16;

template <int MODE, int NV>
__global__ __launch_bounds__(64 * kTopk1Waves) void k_topk1(const LayerArgs a, const void* logits_in,
                                                            int logits_dt, const int32_t* ids_in,
                                                            const float* w_in, int32_t* ids_out, float* w_out,
                                                            float* logits_out) {
  __shared__ int32_t s_cnt[kMaxExperts];
  __shared__ int32_t s_first[kMaxExperts * kRecPairs];  // each list's first pairs, for the records
  __shared__ int s_wsum[kTopk1Waves];
  const int E = a.L.num_experts, T = a.T;
  for (int e = threadIdx.x; e < E; e += 64 * kTopk1Waves) s_cnt[e] = 0;
  __syncthreads();
  for (int t = threadIdx.x >> 6; t < T; t += kTopk1Waves) {
    int sel_e;
    float sel_w;
    route_token<MODE, NV>(a, t, logits_in, logits_dt, ids_in, w_in, logits_out, sel_e, sel_w);
    emit_token(a, t, sel_e, sel_w, ids_out, w_out, s_cnt, s_first);
  }
  __syncthreads();
  compact_experts<kTopk1Waves>(a, s_cnt, false, s_wsum, s_first);
}

// Router and top-k in one launch for T <= kTopk1MaxT: workgroup g computes
// the logits of rows [rpw g, rpw g + rpw) for every token (route_rpw: about
// 128 workgroups), wpr = 16 / rpw waves per row; wave w takes row rpw g + w /
// wpr and tokens w % wpr + wpr i (i < NT) exactly as a k_router wave does
// (router_row_tile: the loads of every chunk of the gate row and the tokens
// in flight, the same fp32 order).  The last workgroup to arrive runs
// k_topk1's body -- one wave per token, per-expert counters in LDS,
// compaction and work records.  Takes the top-k launch and its ramp out of
// the chain router -> top-k -> stage A.
constexpr int kRouteWgs = 136;  // router workgroups aimed at
__host__ __device__ constexpr int route_rpw(int rows) {
  return rows <= kRouteWgs ? 1 : rows <= 2 * kRouteWgs ? 2 : 4;
}
template <int MODE, int NV, int NT>
__global__ __launch_bounds__(64 * kTopk1Waves) void k_route_topk1(
    const LayerArgs a, int row_end, int32_t* ids_out, float* w_out, float* logits_out) {
  __shared__ int32_t s_cnt[kMaxExperts];
  __shared__ int32_t s_first[kMaxExperts * kRecPairs];
  __shared__ int s_wsum[kTopk1Waves];
  __shared__ int s_last;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: scalar gate-row descriptors
  static_assert(kTopk1Waves == 16 && kTopk1MaxT <= 16, "16 waves: wpr >= 4 waves per row, NT <= 4 tokens each");
  const int rpw = route_rpw(row_end), wpr = kTopk1Waves / rpw;
  const int nrwg = (row_end + rpw - 1) / rpw;
  if ((int)blockIdx.x >= nrwg) {  // workgroups past the router's quantise the input (as in k_router)
    quant_mx_piece((const uint16_t*)a.x, a.T, a.L.hidden, a.xq,
                   ((int)blockIdx.x - nrwg) * (64 * kTopk1Waves) + threadIdx.x);
    return;
  }
  const int r = (int)blockIdx.x * rpw + wave / wpr, tb = wave % wpr;
  if (r < row_end && tb < a.T) router_row_tile<true, NT, 4>(a, r, tb, wpr);
  // publish this workgroup's logits (device-coherent stores, acknowledged
  // before the arrival); the last arrival reads every workgroup's
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) s_last = (atomicAdd(&a.ctrl[kCtrlArriveTopk], 1) == nrwg - 1);
  __syncthreads();
  if (!s_last) return;
  const int E = a.L.num_experts, T = a.T;
  for (int e = threadIdx.x; e < E; e += 64 * kTopk1Waves) s_cnt[e] = 0;
  __syncthreads();
  for (int t = wave; t < T; t += kTopk1Waves) {
    int sel_e;
    float sel_w;
    // the shared-gate logit requested before the routing logits (one round trip for both)
    const float shl = a.L.shared_inter > 0 ? load_dev(&a.logits[(size_t)t * (E + 1) + E]) : 0.0f;
    route_token<MODE, NV, true>(a, t, nullptr, 0, nullptr, nullptr, logits_out, sel_e, sel_w);
    emit_token(a, t, sel_e, sel_w, ids_out, w_out, s_cnt, s_first, &shl);
  }
  __syncthreads();
  compact_experts<kTopk1Waves>(a, s_cnt, false, s_wsum, s_first);
  if (threadIdx.x == 0) a.ctrl[kCtrlArriveTopk] = 0;
}

// Large batches: one wave per token, 4 per workgroup; the last-arriving
// workgroup compacts from the global counters and clears them.
template <int MODE, int NV>
__global__ __launch_bounds__(kBlock) void k_topk(const LayerArgs a, const void* logits_in, int logits_dt,
                                                 const int32_t* ids_in, const float* w_in, int32_t* ids_out,
                                                 float* w_out, float* logits_out) {
  const int T = a.T;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  int32_t* cnt = a.ctrl + kCtrlExpertCnt;
  if (t < T) {
    int sel_e;
    float sel_w;
    route_token<MODE, NV>(a, t, logits_in, logits_dt, ids_in, w_in, logits_out, sel_e, sel_w);
    emit_token(a, t, sel_e, sel_w, ids_out, w_out, cnt);
  }
  __shared__ int s_last;
  __shared__ int s_wsum[4];
  // the lists' device-coherent stores acknowledged before the arrival
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) s_last = (atomicAdd(&a.ctrl[kCtrlArriveTopk], 1) == (int)gridDim.x - 1);
  __syncthreads();
  if (!s_last) return;
  compact_experts<4>(a, cnt, true, s_wsum);
  if (threadIdx.x == 0) a.ctrl[kCtrlArriveTopk] = 0;
}

// Large batches: workgroups of 16 waves, one token per wave up to
// kTopkBlkMaxWG workgroups (then each wave loops, t = g, g + 16 * gridDim.x,
// ...).  A workgroup counts its pairs per expert in LDS, reserves one range
// per expert in the global list with one atomic, and writes its pairs there;
// the last workgroup to arrive compacts.  Against k_topk (one workgroup per 4
// tokens, every pair a global atomic) this cuts the same-address atomics (the
// arrival counter, the per-expert counters) and the device-scope fences 4x
// and more.  Measured on MI355X (C3, 256 experts, top-8): 13.3 us at T=256
// (k_topk 14.8), 18.9 us at T=2048 (k_topk 58); k_topk stays ahead at 64
// (10.6 against 13.4).  One token per wave beat four per wave (32.5 us at
// every T from 64 to 2048).
constexpr int kTopkBlkWaves = 16;
constexpr int kTopkBlkMaxWG = 128;
constexpr int kTopkBlkSlots = 8192;  // LDS pair slots per workgroup
constexpr int kTopkBlkMinT = 256;    // from here on k_topk_blk

__host__ __device__ __forceinline__ int topk_blk_grid(int T, int k) {
  int g = (T + kTopkBlkWaves - 1) / kTopkBlkWaves;
  g = g < kTopkBlkMaxWG ? g : kTopkBlkMaxWG;
  // every workgroup's tokens x k must fit its pair slots
  const int tpw = (kTopkBlkSlots / (k > 0 ? k : 1)) / kTopkBlkWaves * kTopkBlkWaves;  // tokens per WG
  const int need = (T + tpw - 1) / tpw;
  return g > need ? g : need;
}

template <int MODE, int NV>
__global__ __launch_bounds__(64 * kTopkBlkWaves) void k_topk_blk(const LayerArgs a, const void* logits_in,
                                                                 int logits_dt, const int32_t* ids_in,
                                                                 const float* w_in, int32_t* ids_out,
                                                                 float* w_out, float* logits_out) {
  __shared__ int32_t s_cnt[kMaxExperts];    // local pair count, then the reserved base, per expert
  __shared__ int32_t s_slot[kTopkBlkSlots];  // expert | local position << 9 per pair slot, -1: none
  __shared__ int s_last;
  __shared__ int s_wsum[kTopkBlkWaves];
  const int E = a.L.num_experts, T = a.T, k = a.L.topk, KP = a.KP;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int e = threadIdx.x; e < E; e += 64 * kTopkBlkWaves) s_cnt[e] = 0;
  __syncthreads();
  const int stride = kTopkBlkWaves * (int)gridDim.x;
  int li = wave;  // local token index: slot base li * k
  // router path: the next token's logits load while this one is routed
  const bool pre = logits_in == nullptr && ids_in == nullptr;
  uint32_t raw[NV];
  if (pre) route_load<NV>(a, blockIdx.x * kTopkBlkWaves + wave, raw);
  for (int t = blockIdx.x * kTopkBlkWaves + wave; t < T; t += stride, li += kTopkBlkWaves) {
    uint32_t nxt[NV];
    if (pre) route_load<NV>(a, t + stride, nxt);
    int sel_e;
    float sel_w;
    route_token_pre<MODE, NV>(a, t, logits_in, logits_dt, ids_in, w_in, logits_out, sel_e, sel_w, pre, raw);
#pragma unroll
    for (int i = 0; i < NV; ++i) raw[i] = nxt[i];
    if (lane < k) {
      const int p = t * KP + lane;
      int slot = -1;
      if (sel_e >= 0 && sel_e < E) {
        a.wts[p] = sel_w;
        a.ids[(size_t)t * k + lane] = sel_e;
        if (ids_out) ids_out[(size_t)t * k + lane] = sel_e;
        if (w_out) w_out[(size_t)t * k + lane] = sel_w;
        slot = sel_e | (atomicAdd(&s_cnt[sel_e], 1) << 9);
      } else {
        // id < 0: no expert for this pair (caller routing); >= E: an error
        a.ids[(size_t)t * k + lane] = -1;
        if (sel_e >= E) atomicOr(&a.ctrl[kCtrlError], 2);
      }
      s_slot[li * k + lane] = slot;
    }
    zero_skipped_slots(a, t, lane < k && !(sel_e >= 0 && sel_e < E));
    if (lane == 0 && a.L.shared_inter > 0) {
      const float sl = a.logits[(size_t)t * (E + 1) + E];
      a.wts[t * KP + k] = round_to(ftm_sigmoidf(sl), a.L.act_dtype);
    }
  }
  __syncthreads();
  int32_t* gcnt = a.ctrl + kCtrlExpertCnt;
  for (int e = threadIdx.x; e < E; e += 64 * kTopkBlkWaves) {
    const int c = s_cnt[e];
    s_cnt[e] = c > 0 ? atomicAdd(&gcnt[e], c) : 0;
  }
  __syncthreads();
  li = wave;
  for (int t = blockIdx.x * kTopkBlkWaves + wave; t < T; t += stride, li += kTopkBlkWaves) {
    if (lane < k) {
      const int slot = s_slot[li * k + lane];
      if (slot >= 0) {
        const int e = slot & 511, pos = s_cnt[e] + (slot >> 9);
        if (pos < T) {
          store_dev(&a.lists[(size_t)e * T + pos], t * KP + lane);
        } else {  // more than T pairs for one expert (fold_repeats rules it out): dropped, flagged, slot zeroed
          atomicOr(&a.ctrl[kCtrlError], 4);
          float* row = a.ybuf + (size_t)(t * KP + lane) * a.L.hidden;
          for (int i = 0; i < a.L.hidden; ++i) row[i] = 0.0f;
        }
      }
    }
  }
  // Every wave's device-coherent list stores acknowledged, then the arrival
  // (the last workgroup reads the lists device-coherent: no fence, which
  // would write back or invalidate the whole L2 of the XCD).
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) s_last = (atomicAdd(&a.ctrl[kCtrlArriveTopk], 1) == (int)gridDim.x - 1);
  __syncthreads();
  if (!s_last) return;
  compact_experts<kTopkBlkWaves>(a, gcnt, true, s_wsum);
  if (threadIdx.x == 0) a.ctrl[kCtrlArriveTopk] = 0;
}

// ============================================================== activation
// ============================================================== stage A (w13 + act)
// Split-K over the 4 waves: wave-load range of wave w (GPTQ: whole groups).
template <int EFMT>
__device__ __forceinline__ void wave_k_range(const ProjSlot& W, int wave, int nwaves, int& lo, int& hi) {
  if constexpr (EFMT == FTM_FMT_GPTQ_INT4) {
    const int ng = (W.K + W.group - 1) / W.group;
    lo = wave * ng / nwaves;
    hi = (wave + 1) * ng / nwaves;
  } else {
    const int nL = fmt_loads<EFMT>(W.K);
    lo = wave * nL / nwaves;
    hi = (wave + 1) * nL / nwaves;
  }
}

template <int EFMT, int AT, int NT>
__device__ void stage_a_body(const LayerArgs& a, const ProjSlot& W, int Iu, int it, int cnt,
                             const int32_t* list, int shared_col, f32x4* red) {
  constexpr bool kG = EFMT == FTM_FMT_GPTQ_INT4;
  constexpr int NSUB = kG ? 4 : 1;
  constexpr int XB = AType<AT>::kBytes;
  constexpr int EPI = 16 * NT / kBlock;  // epilogue elements per thread
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int H = a.L.hidden, KP = a.KP;
  int lo, hi;
  wave_k_range<EFMT>(W, wave, 4, lo, hi);
  const int col0[2] = {it * NT, Iu + it * NT};
  const Rsrc xres = make_rsrc(a.x, (uint32_t)a.T * (uint32_t)H * XB);
  const Rsrc lres = make_rsrc(list, list ? (uint32_t)cnt * 4u : 0u);
  // epilogue element q of this thread: row i, channel j of the tile
  float bias_g[EPI], bias_u[EPI];
#pragma unroll
  for (int q = 0; q < EPI; ++q) {
    const int j = (threadIdx.x + q * kBlock) % NT;
    bias_g[q] = W.bias != nullptr ? load_scalar(W.bias, it * NT + j, W.bias_dt) : 0.0f;
    bias_u[q] = W.bias != nullptr ? load_scalar(W.bias, Iu + it * NT + j, W.bias_dt) : 0.0f;
  }
  for (int mb = 0; mb < cnt; mb += 16) {
    // every list lookup of this row block is issued before the weight stream
    const int pa = pair_of_row(lres, list != nullptr, mb + (lane & 15), cnt, KP, shared_col);
    int pe[EPI];
#pragma unroll
    for (int q = 0; q < EPI; ++q)
      pe[q] = pair_of_row(lres, list != nullptr, mb + (threadIdx.x + q * kBlock) / NT, cnt, KP, shared_col);
    const uint32_t arow = pa >= 0 ? (uint32_t)(pa / KP) * (uint32_t)H * XB : kOOB;
    if constexpr (kG) {
      f32x4 acc[2][4];
#pragma unroll
      for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[r][c] = (f32x4){0.f, 0.f, 0.f, 0.f};
      wave_gemm_gptq<2, AT>(W, col0, lo, hi, xres, arow, acc);
#pragma unroll
      for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) red[((wave * 2 + r) * NSUB + c) * 64 + lane] = acc[r][c];
    } else {
      f32x4 acc[2] = {(f32x4){0.f, 0.f, 0.f, 0.f}, (f32x4){0.f, 0.f, 0.f, 0.f}};
      wave_gemm_kmajor<EFMT, 2, AT>(W, col0, lo, hi, xres, arow, acc);
#pragma unroll
      for (int r = 0; r < 2; ++r) red[(wave * 2 + r) * 64 + lane] = acc[r];
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < EPI; ++q) {
      const int idx = threadIdx.x + q * kBlock;
      const int i = idx / NT, j = idx % NT;
      const int c = kG ? (j & 3) : 0, jj = kG ? (j >> 2) : j;
      const int ln = jj + 16 * (i >> 2), rr = i & 3;
      float g4 = 0.0f, u4 = 0.0f;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        g4 += red[((w * 2 + 0) * NSUB + c) * 64 + ln][rr];
        u4 += red[((w * 2 + 1) * NSUB + c) * 64 + ln][rr];
      }
      const float gs = W.bias != nullptr ? g4 + bias_g[q] : g4;
      const float us = W.bias != nullptr ? u4 + bias_u[q] : u4;
      if (pe[q] >= 0) {
        const float h = round_to(act_fn(a.L.act, gs, us, a.L.swiglu_alpha, a.L.swiglu_limit), a.L.h_dtype);
        store_scalar(a.hbuf, (size_t)pe[q] * a.Imax + it * NT + j, AT, h);
      }
    }
    __syncthreads();
  }
}

template <int FMT, int AT>
__global__ __launch_bounds__(kBlock) void k_stage_a(const LayerArgs a) {
  constexpr bool kG = FMT == FTM_FMT_GPTQ_INT4;
  constexpr int NT = kG ? 64 : 16;
  __shared__ f32x4 red[4 * 2 * (kG ? 4 : 1) * 64];
  const int I = a.L.inter;
  const int tilesR = I / NT;
  int item = blockIdx.x;
  // The expert table is read before the routed count so both loads are in
  // flight together (uniq / ucnt hold E + 1 entries).
  const int u = min(item / tilesR, a.L.num_experts), it = item % tilesR;
  const int e = sload_i32(a.uniq, u), cnt = sload_i32(a.ucnt, u);
  const int nRouted = sload_i32(a.ctrl, kCtrlNRouted);
  if (item < nRouted * tilesR) {
    const int slot = a.L.slot_of_expert ? sload_i32(a.L.slot_of_expert, e) : e;
    if (slot < 0 || slot >= a.L.w13.num_slots) {
      if (threadIdx.x == 0) atomicOr(&a.ctrl[kCtrlError], 1);
      return;
    }
    const ProjSlot W = proj_slot(a.L.w13, slot);
    stage_a_body<FMT, AT, NT>(a, W, I, it, cnt, a.lists + (size_t)e * a.T, 0, red);
  } else {
    item -= nRouted * tilesR;
    const int Is = a.L.shared_inter;
    if (Is <= 0 || item >= Is / 16) return;
    const ProjSlot W = shared_view(a.L.shared_w13, 2 * Is, a.L.hidden);
    stage_a_body<FTM_FMT_BF16, AT, 16>(a, W, Is, item, a.T, nullptr, a.L.topk, red);
  }
}

// ---------------------------------------------------------------- work records
// One routed expert's work record: expert id, pair count, bank slot and its
// first kRecPairs pairs (stage kernels read it with one scalar load).
struct ExpertRec {
  int e, cnt, slot;
  int p[kRecPairs];
};
__device__ __forceinline__ ExpertRec load_rec(const LayerArgs& a, int u) {
  const u32x8 v = sload32(a.recs, (uint32_t)u * (uint32_t)(4 * kRecWords));
  ExpertRec r;
  r.e = (int)v[0];
  r.cnt = (int)v[1];
  r.slot = (int)v[2];
#pragma unroll
  for (int i = 0; i < kRecPairs; ++i) r.p[i] = (int)v[3 + i];
  return r;
}

// Rank u of the set bits of m[0..nwords) (-1 if u >= total) and the total.
__device__ __forceinline__ int mask_rank(const uint32_t* m, int nwords, int u, int& total) {
  int e = -1, run = 0;
  for (int w = 0; w < nwords; ++w) {
    uint32_t b = m[w];
    const int c = __popc(b);
    if (e < 0 && u < run + c) {
      for (int q = 0; q < u - run; ++q) b &= b - 1;
      e = 32 * w + __builtin_ctz(b);
    }
    run += c;
  }
  total = run;
  return e;
}

// Record of expert e from the LDS selections sel[T * k]: every pair of it (T
// <= kRecPairs), in token order (per lane: e may differ between lanes).
__device__ __forceinline__ ExpertRec route_rec(const LayerArgs& a, const int* sel, int e) {
  const int k = a.L.topk, n = a.T * k;
  ExpertRec r;
  r.e = e;
  r.cnt = 0;
#pragma unroll
  for (int q = 0; q < kRecPairs; ++q) r.p[q] = -1;
  for (int i = 0; i < n; ++i) {
    if (sel[i] == e) {
      const int p = (i / k) * a.KP + i % k;
#pragma unroll
      for (int q = 0; q < kRecPairs; ++q) r.p[q] = r.cnt == q ? p : r.p[q];
      ++r.cnt;
    }
  }
  r.slot = a.L.slot_of_expert ? a.L.slot_of_expert[e] : e;
  return r;
}

// The same record when every lane asks for the same expert: scalar fields.
__device__ __forceinline__ ExpertRec route_rec_uniform(const LayerArgs& a, const int* sel, int e) {
  ExpertRec r = route_rec(a, sel, __builtin_amdgcn_readfirstlane(e));
  r.e = __builtin_amdgcn_readfirstlane(r.e);
  r.cnt = __builtin_amdgcn_readfirstlane(r.cnt);
  r.slot = __builtin_amdgcn_readfirstlane(r.slot);
#pragma unroll
  for (int q = 0; q < kRecPairs; ++q) r.p[q] = __builtin_amdgcn_readfirstlane(r.p[q]);
  return r;
}

// ---- routing inside stage A for small batches (route_a): every stage-A
// workgroup routes the call's T <= kRouteAMaxT tokens itself from the router
// logits (one wave per token, the top-k kernels' arithmetic), ranks the routed
// experts by id in an LDS bitmap and takes the expert of its item; workgroup
// 0 publishes what the compaction would have -- the ids, router weights and
// shared-expert gate weights, the work records, the expert table, the lists
// and the routed count -- for stage B, the combine and the caller.  This takes
// the top-k launch out of the chain router -> top-k -> stage A -> ...
struct RouteA {
  int sel[kRouteAMaxT * kLeanRouteMaxK];
  float w[kRouteAMaxT * kLeanRouteMaxK];
  uint32_t mask[256 / 32];
};

template <int MODE>
__device__ __forceinline__ void route_a_token(const LayerArgs& a, RouteA& s, bool lead) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, k = a.L.topk;
  if (wave >= a.T) return;
  int sel_e;
  float sel_w;
  route_token<MODE, 4>(a, wave, nullptr, 0, nullptr, nullptr, lead ? a.logits_out : nullptr, sel_e, sel_w);
  if (lane < k) {
    s.sel[wave * k + lane] = sel_e;
    s.w[wave * k + lane] = sel_w;
    atomicOr(&s.mask[sel_e >> 5], 1u << (sel_e & 31));
  }
}

// Routes the tokens (whole workgroup; every thread must call it) and returns
// the number of routed experts.
__device__ __forceinline__ int route_a_prologue(const LayerArgs& a, RouteA& s, bool lead) {
  if (threadIdx.x < 256 / 32) s.mask[threadIdx.x] = 0u;
  __syncthreads();
  if (a.L.route_mode == FTM_ROUTE_SOFTMAX_TOPK)
    route_a_token<FTM_ROUTE_SOFTMAX_TOPK>(a, s, lead);
  else if (a.L.route_mode == FTM_ROUTE_SOFTMAX_TOPK_LOWP)
    route_a_token<FTM_ROUTE_SOFTMAX_TOPK_LOWP>(a, s, lead);
  else
    route_a_token<FTM_ROUTE_TOPK_SOFTMAX>(a, s, lead);
  __syncthreads();
  int n;
  mask_rank(s.mask, (a.L.num_experts + 31) / 32, 0, n);
  return __builtin_amdgcn_readfirstlane(n);
}

// Workgroup 0's publication (whole workgroup).
__device__ void route_a_publish(const LayerArgs& a, const RouteA& s, int nRouted) {
  const int T = a.T, k = a.L.topk, E = a.L.num_experts, KP = a.KP;
  const int nw = (E + 31) / 32;
  for (int i = threadIdx.x; i < T * k; i += blockDim.x) {
    const int p = (i / k) * KP + i % k;
    a.wts[p] = s.w[i];
    a.ids[i] = s.sel[i];
    if (a.ids_out) a.ids_out[i] = s.sel[i];
    if (a.w_out) a.w_out[i] = s.w[i];
  }
  if (a.L.shared_inter > 0) {
    for (int t = threadIdx.x; t < T; t += blockDim.x) {
      const float sl = a.logits[(size_t)t * (E + 1) + E];
      a.wts[t * KP + k] = round_to(ftm_sigmoidf(sl), a.L.act_dtype);
    }
  }
  for (int u = threadIdx.x; u < nRouted; u += blockDim.x) {
    int tot;
    const ExpertRec r = route_rec(a, s.sel, mask_rank(s.mask, nw, u, tot));
    int32_t* dst = a.recs + (size_t)u * kRecWords;
    dst[0] = r.e;
    dst[1] = r.cnt;
    dst[2] = r.slot;
#pragma unroll
    for (int q = 0; q < kRecPairs; ++q) dst[3 + q] = r.p[q];
    dst[kRecWords - 1] = 0;
    a.uniq[u] = r.e;
    a.ucnt[u] = r.cnt;
#pragma unroll
    for (int q = 0; q < kRecPairs; ++q)
      if (q < r.cnt) a.lists[(size_t)r.e * T + q] = r.p[q];
  }
  if (threadIdx.x == 0) {
    a.ctrl[kCtrlNRouted] = nRouted;
    a.ctrl[kCtrlNU] = nRouted + (a.L.shared_inter > 0 ? 1 : 0);
  }
}

// Pair m (< cnt) of a routed expert: from its record when the record holds
// every pair (route_a), else from its list in global memory.
__device__ __forceinline__ int pair_rec_or_list(const ExpertRec* rec, Rsrc lres, int m, int cnt, int KP) {
  if (rec != nullptr) {
    int p = -1;
#pragma unroll
    for (int q = 0; q < kRecPairs; ++q) p = (m == q && m < cnt) ? rec->p[q] : p;
    return p;
  }
  return pair_of_row(lres, true, m, cnt, KP, 0);
}

// ---------------------------------------------------------------- stage A, GPTQ decode (activations in LDS)
// The arithmetic of wave_gemm_gptq / stage_a_body (each nibble decoded as
// 128 + q in bf16, per-group scale and zero-point correction from the group's
// row sums of x) with the data path of the lean FP8 kernels: the block's token
// rows of a wave's K range are copied to LDS once (global_load_lds), and the
// next 128-wide group's weights, scales and zero words are in flight while the
// current group is multiplied.  bf16 activations, group 128, a wave's K range
// of at most kGqMaxKR; blocks of kGqXT tokens (MFMA rows past them read a zero row).
extern __shared__ __align__(16) uint16_t ftm_xl_lds[];  // dynamic LDS of the decode stages

constexpr int kGqXT = 4;
constexpr int kGqMaxKR = 1024;
// Larger batches keep the 16-token blocks of k_stage_a: measured on C2, this
// kernel ties it at T=32 (64.7 against 64.5 us) and loses at T=64 (91 against 67).
constexpr int kGqMaxT = 16;

__host__ __device__ __forceinline__ constexpr int gq_pitch(int KR) { return KR + 8; }

// LDS layout of the GPTQ decode stages: wave w's kGqXT token rows at
// w * kGqXT * pitch, pitch = gq_pitch(the layer's per-wave K range), so the
// region is no larger than the layer needs; the reduction buffer (red_bytes)
// aliases the start of it; then ONE zero row, past both, that MFMA rows past
// the block's tokens read (shared by the workgroup's waves).
__host__ __device__ __forceinline__ int gq_wave_kr(int K, int ks) { return ((K + 127) / 128 + ks - 1) / ks * 128; }
__host__ __device__ __forceinline__ int gq_zrow_off(int waves, int pitch, int red_bytes) {
  const int rows = waves * kGqXT * pitch;
  return rows > red_bytes / 2 ? rows : red_bytes / 2;  // in elements
}
__host__ __device__ __forceinline__ size_t gq_lds_bytes(int waves, int K, int ks, int red_bytes) {
  const int pitch = gq_pitch(gq_wave_kr(K, ks));
  return ((size_t)gq_zrow_off(waves, pitch, red_bytes) + (size_t)pitch) * 2u;
}
// Each wave writes the whole zero row itself (identical values) before it
// reads it, so no barrier is needed.
__device__ __forceinline__ void gq_zero_row(uint16_t* zrow, int kr) {
  const int lane = threadIdx.x & 63;
  for (int e = 8 * lane; e < kr; e += 8 * 64) *(u32x4*)(zrow + e) = (u32x4){0u, 0u, 0u, 0u};
}

// NCOL columns per lane: 4 (a wave covers 64 columns, 16-byte loads) or 2
// (32 columns, 8-byte loads: twice the items for one or two tokens).
template <int NCOL>
struct GqGroupT {
  typedef uint32_t V __attribute__((ext_vector_type(NCOL)));
  V raw[4];  // 4 wave-loads of 32 K: lane (g, rl) holds k8 row 4 b + g, columns ncol .. ncol + NCOL - 1
  V scv;     // the columns' scales (fp32: NCOL words; fp16 / bf16: NCOL halves in the first words)
  uint32_t zw;
};
typedef GqGroupT<4> GqGroup;

template <int NCOL>
__device__ __forceinline__ typename GqGroupT<NCOL>::V gq_bload(Rsrc r, uint32_t off) {
  if constexpr (NCOL == 4) return bload16(r, off);
  else return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
}

template <int NCOL = 4>
__device__ __forceinline__ void gq_issue(Rsrc wres, Rsrc sres, Rsrc zres, uint32_t ncol, int N, int grp,
                                         uint32_t sbytes, GqGroupT<NCOL>& G) {
  const int g = (threadIdx.x & 63) >> 4;
  const bool ok = ncol != kOOB;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const uint32_t prow = (uint32_t)(grp * 16 + 4 * b + g);
    G.raw[b] = gq_bload<NCOL>(wres, ok ? (prow * (uint32_t)N + ncol) * 4u : kOOB);
  }
  G.scv = gq_bload<NCOL>(sres, ok ? ((uint32_t)grp * (uint32_t)N + ncol) * sbytes : kOOB);
  G.zw = bload4(zres, ok ? ((uint32_t)grp * (uint32_t)(N / 8) + ncol / 8) * 4u : kOOB);
}
constexpr int kGqLoads = 6;  // vector loads per gq_issue

// One group: MFMAs over its 4 wave-loads, then acc += s * (partial - (128 + z + 1) * sum x).
// The token rows' sums over the group come from one more MFMA per wave-load
// against a tile of ones, already in the output layout (lane (g, j) holds
// rows 4 g .. 4 g + 3), instead of VALU sums and cross-lane shuffles.
template <int NCOL = 4>
__device__ __forceinline__ void gq_group(const GqGroupT<NCOL>& G, const uint16_t* xrow, int kofs, uint32_t ncol,
                                         uint32_t sbytes, int s_dt, f32x4 (&acc)[NCOL]) {
  const int lane = threadIdx.x & 63, g = lane >> 4;
  const u32x4 ones = (u32x4){0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u};  // bf16 1.0
  const GqConsts kc = gq_decode_consts();
  f32x4 tmp[NCOL];
#pragma unroll
  for (int c = 0; c < NCOL; ++c) tmp[c] = (f32x4){0.f, 0.f, 0.f, 0.f};
  f32x4 sxr = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const u32x4 av = perm_gptq(*(const u32x4*)(xrow + kofs + 32 * b + 8 * g));
    sxr = mfma_bf16(av, ones, sxr);
#pragma unroll
    for (int c = 0; c < NCOL; ++c) tmp[c] = mfma_bf16(av, gptq_word_to_bf16(G.raw[b][c], kc), tmp[c]);
  }
  uint32_t sw[NCOL];
#pragma unroll
  for (int c = 0; c < NCOL; ++c) sw[c] = G.scv[c];
#pragma unroll
  for (int c = 0; c < NCOL; ++c) {
    float sc;
    if (sbytes == 4u) {
      sc = __uint_as_float(sw[c]);
    } else {
      const uint32_t h = (sw[c >> 1] >> (16 * (c & 1))) & 0xffffu;
      sc = s_dt == FTM_DT_F16 ? f16_to_f32((uint16_t)h) : bf16_to_f32(h);
    }
    const float zp = (float)(((G.zw >> (4 * ((ncol + c) & 7))) & 0xfu) + 1u);
    f32x4 corr;
    corr.x = tmp[c].x - (128.0f + zp) * sxr[0];
    corr.y = tmp[c].y - (128.0f + zp) * sxr[1];
    corr.z = tmp[c].z - (128.0f + zp) * sxr[2];
    corr.w = tmp[c].w - (128.0f + zp) * sxr[3];
    acc[c] += corr * sc;
  }
}

// Copy elements [k0, k0 + kr) of the rows of pairs pr[0..nb) into xw (row r
// at xw + r * pitch); the row of pair p starts at src + (p / div) * row_elems.
__device__ __forceinline__ void gq_fill(const int (&pr)[kGqXT], int nb, const void* src, int div, int row_elems,
                                        int k0, int kr, int pitch, uint16_t* xw) {
  typedef __attribute__((address_space(1))) const void* GPtr;
  typedef __attribute__((address_space(3))) void* LPtr;
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int r = 0; r < kGqXT; ++r) {
    if (r < nb) {
      const char* row = (const char*)src + ((size_t)(pr[r] / div) * (size_t)row_elems + (size_t)k0) * 2u;
      for (int c = 0; c * 1024 < 2 * kr; ++c) {
        if (c * 1024 + 16 * lane < 2 * kr)
          __builtin_amdgcn_global_load_lds((GPtr)(row + c * 1024 + 16 * lane),
                                           (LPtr)((char*)(xw + r * pitch) + c * 1024), 16, 0, 0);
      }
    }
  }
}

// A wave's groups [lo, hi) through two group buffers: group g + 1 is in
// flight while group g is multiplied.  GA already holds group lo (issued
// before the caller's token-row copy).  A third buffer (group g + 2 in flight
// too) measured slower on C2 at T=16: w13 37.1 -> 39.3 us, w2 23.4 -> 30.5.
__device__ __forceinline__ void gq_pipeline(Rsrc wres, Rsrc sres, Rsrc zres, uint32_t ncol, int N, uint32_t sbytes,
                                            int s_dt, int lo, int hi, const uint16_t* xrow, GqGroup& GA,
                                            f32x4 (&acc)[4]) {
  GqGroup GB;
  for (int grp = lo; grp < hi; grp += 2) {
    const bool two = grp + 1 < hi;
    if (two) {
      gq_issue(wres, sres, zres, ncol, N, grp + 1, sbytes, GB);
      wait_vm<kGqLoads>();  // group grp (and the copy) landed
    } else {
      __builtin_amdgcn_s_waitcnt(0);
    }
    gq_group(GA, xrow, (grp - lo) * 128, ncol, sbytes, s_dt, acc);
    if (two) {
      if (grp + 2 < hi) {
        gq_issue(wres, sres, zres, ncol, N, grp + 2, sbytes, GA);
        wait_vm<kGqLoads>();
      } else {
        __builtin_amdgcn_s_waitcnt(0);
      }
      gq_group(GB, xrow, (grp + 1 - lo) * 128, ncol, sbytes, s_dt, acc);
    }
  }
}

// Small batches (a workgroup or two per CU): every group of the wave's range
// [lo, hi), at most NG, issued at once before the token-row copy -- one
// round trip instead of one per group pair -- then multiplied in order (the
// same arithmetic as gq_pipeline).
template <int NG, int NCOL>
__device__ __forceinline__ void gq_issue_all(Rsrc wres, Rsrc sres, Rsrc zres, uint32_t ncol, int N, uint32_t sbytes,
                                             int lo, int hi, GqGroupT<NCOL> (&G)[NG]) {
#pragma unroll
  for (int i = 0; i < NG; ++i) gq_issue<NCOL>(wres, sres, zres, lo + i < hi ? ncol : kOOB, N, lo + i, sbytes, G[i]);
}
template <int NG, int NCOL>
__device__ __forceinline__ void gq_run_all(uint32_t ncol, uint32_t sbytes, int s_dt, int lo, int hi,
                                           const uint16_t* xrow, const GqGroupT<NCOL> (&G)[NG],
                                           f32x4 (&acc)[NCOL]) {
  __builtin_amdgcn_s_waitcnt(0);  // every group and the copy landed
#pragma unroll
  for (int i = 0; i < NG; ++i)
    if (lo + i < hi) gq_group<NCOL>(G[i], xrow, i * 128, ncol, sbytes, s_dt, acc);
}
// Measured on MI355X (C2, us): stage A (k_stage_a_gq<4>, one or two
// tokens) T=1 13.5 -> 12.8, T=2 15.4 -> 14.8; stage B T=1 7.8 -> 7.4, T=2
// 8.9 either way, T=3 / 4 10.1 / 10.7 -> 10.5 / 11.2 (two workgroups per CU
// at 188 registers), so stage B issues them all for one token only, on
// items of 64 columns (6.9 -> 6.3 against 128: twice the workgroups).
constexpr int kGqAllNG = 4;   // groups per wave issued at once
constexpr int kGqBAllMaxT = 1;  // stage B issues them all up to this many tokens

// Item: 64 channels of one expert; waves [0, KS) take the 64 gate columns and
// waves [KS, 2 KS) the 64 up columns, each over 1 / KS of the K groups (KS = 2:
// a 256-thread workgroup, rows of up to kGqMaxKR elements per wave; KS = 4: 512
// threads, half the rows per wave, twice the waves -- and bytes in flight --
// per CU at the same LDS).
// Channels per stage-A item: 32 for one token (twice the items, so twice
// the CUs stream the eight experts: C2 w13 T=1 11.9 -> 10.9 us; at T=2 the
// 64-channel items are 0.2 us faster), else 64.
__host__ __device__ constexpr int gq_nt(int ks, int T) { return ks == 4 && T == 1 ? 32 : 64; }

template <int KS>
struct GqA {
  static constexpr int kThreads = 2 * KS * 64;
  static constexpr int kKR = kGqMaxKR * 2 / KS;  // a wave's K range bound
  // token rows + zero row, at least the reduction buffer (32 KiB: 8 waves x
  // 4 sub-tiles, or the shared-expert body's)
  static constexpr int kRedBytes = 32768;
  static size_t lds(int K) { return gq_lds_bytes(2 * KS, K, KS, kRedBytes); }
};

// rec: null (pairs from list), or a record holding every pair (route_a).
template <int NT, int KS>
__device__ void stage_a_gq(const LayerArgs& a, const ProjSlot& W, int Iu, int it, int cnt, const ExpertRec* rec,
                           const int32_t* list, f32x4* red) {
  constexpr int EPI = 16 * NT / GqA<KS>::kThreads;
  constexpr int NCOL = NT / 16;  // columns per lane
  static_assert(NCOL == 4 || (NCOL == 2 && KS == 4), "64-column tiles, or 32 with every group issued at once");
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int rl = lane & 15;
  const int H = a.L.hidden, KP = a.KP, N = W.N;
  const int tile = wave / KS;
  int lo, hi;
  wave_k_range<FTM_FMT_GPTQ_INT4>(W, wave % KS, KS, lo, hi);
  const int k0 = lo * 128, kr = (hi - lo) * 128;
  const uint32_t sbytes = W.s_dt == FTM_DT_F32 ? 4u : 2u;
  const int ngroups = (W.K + 127) / 128;
  const Rsrc wres = make_rsrc(W.w, (uint32_t)(W.K / 8) * (uint32_t)N * 4u);
  const Rsrc zres = make_rsrc(W.z, (uint32_t)ngroups * (uint32_t)(N / 8) * 4u);
  const Rsrc sres = make_rsrc(W.s, (uint32_t)ngroups * (uint32_t)N * sbytes);
  const int col0 = (tile == 0 ? 0 : Iu) + it * NT;
  const uint32_t ncol = col0 + NCOL * rl < N ? (uint32_t)(col0 + NCOL * rl) : kOOB;
  const Rsrc lres = make_rsrc(list, (uint32_t)cnt * 4u);
  const int kr_max = gq_wave_kr(W.K, KS);
  const int pitch = gq_pitch(kr_max);
  uint16_t* xw = ftm_xl_lds + wave * kGqXT * pitch;
  uint16_t* zrow = ftm_xl_lds + gq_zrow_off(2 * KS, pitch, GqA<KS>::kRedBytes);
  gq_zero_row(zrow, kr_max);
  float bias_g[EPI], bias_u[EPI];
#pragma unroll
  for (int q = 0; q < EPI; ++q) {
    const int j = (threadIdx.x + q * GqA<KS>::kThreads) % NT;
    bias_g[q] = W.bias != nullptr ? load_scalar(W.bias, it * NT + j, W.bias_dt) : 0.0f;
    bias_u[q] = W.bias != nullptr ? load_scalar(W.bias, Iu + it * NT + j, W.bias_dt) : 0.0f;
  }
  for (int mb = 0; mb < cnt; mb += kGqXT) {
    const int nb = min(kGqXT, cnt - mb);
    int pr[kGqXT];
#pragma unroll
    for (int i = 0; i < kGqXT; ++i) pr[i] = pair_rec_or_list(rec, lres, mb + i, cnt, KP);
    int pe[EPI];
#pragma unroll
    for (int q = 0; q < EPI; ++q) {
      const int i = (threadIdx.x + q * GqA<KS>::kThreads) / NT;
      pe[q] = i < kGqXT ? pair_rec_or_list(rec, lres, mb + i, cnt, KP) : -1;
    }
    f32x4 acc[NCOL];
#pragma unroll
    for (int c = 0; c < NCOL; ++c) acc[c] = (f32x4){0.f, 0.f, 0.f, 0.f};
    if (hi > lo) {
      const uint16_t* xrow = rl < nb ? xw + rl * pitch : zrow;
      if constexpr (KS == 4) {  // one or two tokens: a wave's <= 4 groups in flight at once
        GqGroupT<NCOL> G[kGqAllNG];
        gq_issue_all<kGqAllNG, NCOL>(wres, sres, zres, ncol, N, sbytes, lo, hi, G);
        gq_fill(pr, nb, a.x, KP, H, k0, kr, pitch, xw);
        gq_run_all<kGqAllNG, NCOL>(ncol, sbytes, W.s_dt, lo, hi, xrow, G, acc);
      } else {
        GqGroup GA;
        gq_issue(wres, sres, zres, ncol, N, lo, sbytes, GA);  // weights first,
        gq_fill(pr, nb, a.x, KP, H, k0, kr, pitch, xw);       // then the token rows
        gq_pipeline(wres, sres, zres, ncol, N, sbytes, W.s_dt, lo, hi, xrow, GA, acc);
      }
    }
    __syncthreads();  // red aliases the token rows: every wave is past its MFMAs
#pragma unroll
    for (int c = 0; c < NCOL; ++c) red[(wave * NCOL + c) * 64 + lane] = acc[c];
    __syncthreads();
#pragma unroll
    for (int q = 0; q < EPI; ++q) {
      const int idx = threadIdx.x + q * GqA<KS>::kThreads;
      const int i = idx / NT, j = idx % NT;
      const int c = j % NCOL, jj = j / NCOL;
      const int ln = jj + 16 * (i >> 2), rr = i & 3;
      float g4 = 0.0f, u4 = 0.0f;
#pragma unroll
      for (int p = 0; p < KS; ++p) {
        g4 += red[(p * NCOL + c) * 64 + ln][rr];
        u4 += red[((KS + p) * NCOL + c) * 64 + ln][rr];
      }
      const float gs = W.bias != nullptr ? g4 + bias_g[q] : g4;
      const float us = W.bias != nullptr ? u4 + bias_u[q] : u4;
      if (pe[q] >= 0) {
        const float h = act_fn(a.L.act, gs, us, a.L.swiglu_alpha, a.L.swiglu_limit);
        store_scalar(a.hbuf, (size_t)pe[q] * a.Imax + it * NT + j, FTM_DT_BF16, h);
      }
    }
    __syncthreads();
  }
}

// Layers the GPTQ decode stage A with activations in LDS takes (0 = none),
// and its K split: 4 for one or two tokens when every wave's quarter of the K
// groups fits and there is no shared expert (whose body needs 256-thread
// workgroups), else 2.  Measured on C2 (w13 us, KS 2 -> 4): T=1 15.9 -> 11.5,
// T=4 19.1 -> 21.4, T=16 37.6 -> 44.2.
static int gq_ks(const ftm_moe_layer& L, int T) {
  const ftm_proj& A = L.w13;
  if (A.fmt != FTM_FMT_GPTQ_INT4 || L.act_dtype != FTM_DT_BF16 || A.group != 128) return 0;
  if (L.hidden % 128 != 0 || L.inter % 64 != 0 || T > kGqMaxT) return 0;
  if (T <= 2 && L.shared_inter <= 0 && (L.hidden / 128 + 3) / 4 * 128 <= GqA<4>::kKR) return 4;
  return (L.hidden / 128 + 1) / 2 * 128 <= GqA<2>::kKR ? 2 : 0;  // half of the K groups per wave
}
static bool gq_ok(const ftm_moe_layer& L, int T) { return gq_ks(L, T) != 0; }

// KS = 2: three 4-wave workgroups' worth of waves per SIMD (amdgpu_waves_per_eu
// 3: 147 VGPRs and no accumulators parked in AGPRs, against 156 + 20 and two
// waves per SIMD left to the compiler): C2 w13 T=16 / 32 35.7 / 60.2 ->
// 35.4 / 60.0 us, w2 (the same for k_stage_b_gq) 21.1 / 30.1 -> 20.8 / 29.5.
template <int KS, int NT>
__global__ __launch_bounds__(GqA<KS>::kThreads) __attribute__((amdgpu_waves_per_eu(KS == 2 ? 3 : 1))) void k_stage_a_gq(
    const LayerArgs a) {
  // The reduction buffer (16 KiB routed, 32 KiB for the shared-expert body)
  // aliases the dynamic token-row regions (41 KiB), so a workgroup holds 41
  // KiB of LDS and three fit a CU.
  f32x4* red = (f32x4*)ftm_xl_lds;
  __shared__ RouteA sra;
  const int I = a.L.inter;
  const int tilesR = I / NT;
  int item = blockIdx.x;
  if (a.route_a) {
    // the shared expert's items first (they need no routing), then the routed ones
    const int nSh = KS == 2 && a.L.shared_inter > 0 ? a.L.shared_inter / 16 : 0;
    if (item < nSh) {
      if constexpr (KS == 2) {
        const int Is = a.L.shared_inter;
        const ProjSlot W = shared_view(a.L.shared_w13, 2 * Is, a.L.hidden);
        stage_a_body<FTM_FMT_BF16, FTM_DT_BF16, 16>(a, W, Is, item, a.T, nullptr, a.L.topk, red);
      }
      return;
    }
    item -= nSh;
    const int nR = route_a_prologue(a, sra, item == 0);
    if (item == 0) route_a_publish(a, sra, nR);
    if (item >= nR * tilesR) return;
    int tot;
    const ExpertRec rec = route_rec_uniform(a, sra.sel, mask_rank(sra.mask, (a.L.num_experts + 31) / 32,
                                                                  item / tilesR, tot));
    if (rec.slot < 0 || rec.slot >= a.L.w13.num_slots) {
      if (threadIdx.x == 0) atomicOr(&a.ctrl[kCtrlError], 1);
      return;
    }
    stage_a_gq<NT, KS>(a, proj_slot(a.L.w13, rec.slot), I, item % tilesR, rec.cnt, &rec, nullptr, red);
    return;
  }
  const int u = min(item / tilesR, a.L.num_experts), it = item % tilesR;
  const int e = sload_i32(a.uniq, u), cnt = sload_i32(a.ucnt, u);
  const int nRouted = sload_i32(a.ctrl, kCtrlNRouted);
  if (item < nRouted * tilesR) {
    const int slot = a.L.slot_of_expert ? sload_i32(a.L.slot_of_expert, e) : e;
    if (slot < 0 || slot >= a.L.w13.num_slots) {
      if (threadIdx.x == 0) atomicOr(&a.ctrl[kCtrlError], 1);
      return;
    }
    stage_a_gq<NT, KS>(a, proj_slot(a.L.w13, slot), I, it, cnt, nullptr, a.lists + (size_t)e * a.T, red);
  } else if constexpr (KS == 2) {
    item -= nRouted * tilesR;
    const int Is = a.L.shared_inter;
    if (Is <= 0 || item >= Is / 16) return;
    const ProjSlot W = shared_view(a.L.shared_w13, 2 * Is, a.L.hidden);
    stage_a_body<FTM_FMT_BF16, FTM_DT_BF16, 16>(a, W, Is, item, a.T, nullptr, a.L.topk, red);
  }
}

// ---------------------------------------------------------------- stage B, GPTQ decode (h rows in LDS)
// The data path of k_stage_a_gq for w2: an item is 128 output columns of one
// expert; waves 0-1 take columns [0, 64) of it and waves 2-3 [64, 128), each
// over half of the K groups (K = I), the next group's weights, scales and zero
// word in flight while the current one is multiplied; the two halves are
// summed through LDS, router-weighted, and written to the slot buffer rows
// (k_combine sums them).
constexpr int kGqNB = 128;  // output columns per stage-B item
constexpr int kGqNB1 = 64;  // ... for one token (every group issued at once)
constexpr int kGqBRedBytes = 16384;  // its reduction buffer: 4 waves x 4 sub-tiles x 64 lanes x 16 B
// Measured on C2 (w2, against the register-fed k_stage_b): T=4 18.6 -> 11.6
// us, T=16 39.5 -> 29.3, T=24 46.3 -> 36.0, T=32 49.6 -> 41.0; T=64 55.3 ->
// 56.5, so it stops at 32 tokens.
constexpr int kGqBMaxT = 32;

template <bool ALL, int NB>
__device__ void stage_b_gq(const LayerArgs& a, const ProjSlot& W, int it, int cnt, const int32_t* list,
                           f32x4* red) {
  constexpr int EPI = kGqXT * NB / kBlock;
  constexpr int NCOL = NB / 32;  // columns per lane: two column halves of NB / 2
  static_assert(NCOL == 4 || (NCOL == 2 && ALL), "128-column items, or 64 with every group issued at once");
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int rl = lane & 15;
  const int H = a.L.hidden, KP = a.KP, N = W.N;
  const int tile = wave >> 1;
  int lo, hi;
  wave_k_range<FTM_FMT_GPTQ_INT4>(W, wave & 1, 2, lo, hi);
  const int k0 = lo * 128, kr = (hi - lo) * 128;
  const uint32_t sbytes = W.s_dt == FTM_DT_F32 ? 4u : 2u;
  const int ngroups = (W.K + 127) / 128;
  const Rsrc wres = make_rsrc(W.w, (uint32_t)(W.K / 8) * (uint32_t)N * 4u);
  const Rsrc zres = make_rsrc(W.z, (uint32_t)ngroups * (uint32_t)(N / 8) * 4u);
  const Rsrc sres = make_rsrc(W.s, (uint32_t)ngroups * (uint32_t)N * sbytes);
  const int col0 = it * NB + (NB / 2) * tile;
  const uint32_t ncol = col0 + NCOL * rl < N ? (uint32_t)(col0 + NCOL * rl) : kOOB;
  const Rsrc lres = make_rsrc(list, (uint32_t)cnt * 4u);
  const Rsrc wtres = make_rsrc(a.wts, (uint32_t)a.T * (uint32_t)KP * 4u);
  const int kr_max = gq_wave_kr(W.K, 2);
  const int pitch = gq_pitch(kr_max);
  uint16_t* xw = ftm_xl_lds + wave * kGqXT * pitch;
  uint16_t* zrow = ftm_xl_lds + gq_zrow_off(4, pitch, kGqBRedBytes);
  gq_zero_row(zrow, kr_max);
  float bias_n[EPI];
#pragma unroll
  for (int q = 0; q < EPI; ++q) {
    const int n = it * NB + (threadIdx.x + q * kBlock) % NB;
    bias_n[q] = (W.bias != nullptr && n < H) ? load_scalar(W.bias, n, W.bias_dt) : 0.0f;
  }
  for (int mb = 0; mb < cnt; mb += kGqXT) {
    const int nb = min(kGqXT, cnt - mb);
    int pr[kGqXT];
#pragma unroll
    for (int i = 0; i < kGqXT; ++i) pr[i] = pair_of_row(lres, true, mb + i, cnt, KP, 0);
    int pe[EPI];
    float we[EPI];
#pragma unroll
    for (int q = 0; q < EPI; ++q) {
      const int i = (threadIdx.x + q * kBlock) / NB;
      pe[q] = pair_of_row(lres, true, mb + i, cnt, KP, 0);
      we[q] = __uint_as_float(bload4(wtres, pe[q] >= 0 ? 4u * (uint32_t)pe[q] : kOOB));
    }
    f32x4 acc[NCOL];
#pragma unroll
    for (int c = 0; c < NCOL; ++c) acc[c] = (f32x4){0.f, 0.f, 0.f, 0.f};
    if (hi > lo) {
      const uint16_t* xrow = rl < nb ? xw + rl * pitch : zrow;
      if constexpr (ALL) {
        GqGroupT<NCOL> G[kGqAllNG];
        gq_issue_all<kGqAllNG, NCOL>(wres, sres, zres, ncol, N, sbytes, lo, hi, G);
        gq_fill(pr, nb, a.hbuf, 1, a.Imax, k0, kr, pitch, xw);
        gq_run_all<kGqAllNG, NCOL>(ncol, sbytes, W.s_dt, lo, hi, xrow, G, acc);
      } else {
        GqGroup GA;
        gq_issue(wres, sres, zres, ncol, N, lo, sbytes, GA);       // weights first,
        gq_fill(pr, nb, a.hbuf, 1, a.Imax, k0, kr, pitch, xw);     // then the h rows
        gq_pipeline(wres, sres, zres, ncol, N, sbytes, W.s_dt, lo, hi, xrow, GA, acc);
      }
    }
    __syncthreads();  // red aliases the h rows: every wave is past its MFMAs
#pragma unroll
    for (int c = 0; c < NCOL; ++c) red[(wave * NCOL + c) * 64 + lane] = acc[c];
    __syncthreads();
#pragma unroll
    for (int q = 0; q < EPI; ++q) {
      const int idx = threadIdx.x + q * kBlock;
      const int i = idx / NB, j = idx % NB;
      const int t = j / (NB / 2), jl = j % (NB / 2);
      const int c = jl % NCOL, ln = jl / NCOL + 16 * (i >> 2), rr = i & 3;
      const int n = it * NB + j;
      float y = red[((2 * t) * NCOL + c) * 64 + ln][rr] + red[((2 * t + 1) * NCOL + c) * 64 + ln][rr];
      if (pe[q] >= 0 && n < H) {
        if (W.bias != nullptr) y += bias_n[q];
        a.ybuf[(size_t)pe[q] * H + n] = y * we[q];
      }
    }
    __syncthreads();
  }
}

// Layers the GPTQ decode stage B with h rows in LDS takes.
template <int EFMT, int AT>
__device__ void stage_b_body(const LayerArgs& a, const ProjSlot& W, int cnt, const int32_t* list, int shared_col,
                             int nt, f32x4* red);

// Routed items (expert, 128 columns) first, then the shared expert's 64-column tiles.
// ---------------------------------------------------------------- stage A, K-major formats
// Work item: 8 channels of one expert = 16 weight rows (the 8 gate rows and
// their 8 up rows), K split over the 4 waves of a workgroup and reduced
// through LDS.  Lanes l % 16 < 8 produce gate sums, the others the matching
// up sums; a DPP row shift brings each up sum next to its gate sum for the
// activation.  Compared with 16-channel tiles (16 gate + 16 up rows), the
// workgroup needs half the activation registers per weight byte in flight.
constexpr int kDppRowShl8 = 0x108;  // lane i <- lane i + 8 within a 16-lane row

constexpr int kRowsNLW = 8;  // wave-loads of a wave's K range in one prefetch window

template <int EFMT, int AT>
__device__ void stage_a_rows(const LayerArgs& a, const ProjSlot& W, int Iu, int c0, int cnt, const int32_t* list,
                             int shared_col, int kp, f32x4* red) {
  constexpr int CH = 4;
  constexpr int KS = 4;
  const int lane = threadIdx.x & 63;
  const int n = lane & 15;
  const int H = a.L.hidden, KP = a.KP;
  constexpr int XB = AType<AT>::kBytes;
  const int lrow = n < 8 ? c0 + n : Iu + c0 + (n - 8);
  const int sb_lo = W.group > 0 ? c0 / W.group : 0;
  const int sb_hi = W.group > 0 ? (Iu + c0) / W.group : 0;
  const int nL = fmt_loads<EFMT>(W.K);
  const int L_lo = kp * nL / KS, L_hi = (kp + 1) * nL / KS;
  const Rsrc xres = make_rsrc(a.x, (uint32_t)a.T * (uint32_t)H * XB);
  const Rsrc lres = make_rsrc(list, list ? (uint32_t)cnt * 4u : 0u);
  float bg = 0.0f, bu = 0.0f;
  if (W.bias != nullptr && n < 8) {
    bg = load_scalar(W.bias, c0 + n, W.bias_dt);
    bu = load_scalar(W.bias, Iu + c0 + n, W.bias_dt);
  }
  for (int mb = 0; mb < cnt; mb += 16) {
    const int pa = pair_of_row(lres, list != nullptr, mb + n, cnt, KP, shared_col);
    int pe[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) pe[r] = pair_of_row(lres, list != nullptr, mb + 4 * (lane >> 4) + r, cnt, KP, shared_col);
    const uint32_t arow = pa >= 0 ? (uint32_t)(pa / KP) * (uint32_t)H * XB : kOOB;
    f32x4 acc = (f32x4){0.f, 0.f, 0.f, 0.f};
    wave_rows_kmajor<EFMT, AT, CH>(W, lrow, sb_lo, sb_hi, L_lo, L_hi, xres, arow, acc);
    red[kp * 64 + lane] = acc;
    __syncthreads();
    if (kp == 0) {
      acc = red[lane];
#pragma unroll
      for (int j = 1; j < KS; ++j) acc += red[j * 64 + lane];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float gs = acc[r] + bg;
        const float us = dpp_f<kDppRowShl8>(acc[r]) + bu;
        if (n < 8 && pe[r] >= 0) {
          const float h = round_to(act_fn(a.L.act, gs, us, a.L.swiglu_alpha, a.L.swiglu_limit), a.L.h_dtype);
          store_scalar(a.hbuf, (size_t)pe[r] * a.Imax + c0 + n, AT, h);
        }
      }
    }
    __syncthreads();
  }
}

// One 8-channel item per workgroup (routed items first, then the shared expert's).
template <int FMT, int AT>
__global__ __launch_bounds__(kBlock) void k_stage_a_rows(const LayerArgs a) {
  __shared__ f32x4 red[4 * 64];
  // wave index as a wave-uniform (scalar) value, so the FP8 scale addresses
  // stay in SGPRs and use scalar loads
  const int kp = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int I = a.L.inter;
  const int t8 = I / 8;
  const int item = blockIdx.x;
  // expert table and routed count in flight together (uniq / ucnt hold E + 1)
  const int u = min(item / t8, a.L.num_experts);
  const int e = a.uniq[u], cnt = a.ucnt[u];
  const int nRouted = a.ctrl[kCtrlNRouted];
  if (item < nRouted * t8) {
    const int slot = a.L.slot_of_expert ? a.L.slot_of_expert[e] : e;
    if (slot < 0 || slot >= a.L.w13.num_slots) {
      if (threadIdx.x == 0) atomicOr(&a.ctrl[kCtrlError], 1);
      return;
    }
    const ProjSlot W = proj_slot(a.L.w13, slot);
    stage_a_rows<FMT, AT>(a, W, I, (item % t8) * 8, cnt, a.lists + (size_t)e * a.T, 0, kp, red);
  } else {
    const int sitem = item - nRouted * t8;
    const int Is = a.L.shared_inter;
    if (Is <= 0 || sitem >= Is / 8) return;
    const ProjSlot W = shared_view(a.L.shared_w13, 2 * Is, a.L.hidden);
    stage_a_rows<FTM_FMT_BF16, AT>(a, W, Is, sitem * 8, a.T, nullptr, a.L.topk, kp, red);
  }
}

// ============================================================== stage B (w2 -> slot buffer)
// 64 output columns per workgroup.  K-major formats: 4 waves side by side,
// 16 columns each, full K.  GPTQ: one 64-column wave tile, K split over the
// 4 waves on group edges and reduced through LDS.
template <int EFMT, int AT>
__device__ void stage_b_body(const LayerArgs& a, const ProjSlot& W, int cnt, const int32_t* list,
                             int shared_col, int nt, f32x4* red) {
  constexpr bool kG = EFMT == FTM_FMT_GPTQ_INT4;
  constexpr int XB = AType<AT>::kBytes;
  constexpr int EPI = kG ? 16 * 64 / kBlock : 4;  // output elements per thread
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int H = a.L.hidden, KP = a.KP;
  int lo, hi;
  if (kG) {
    wave_k_range<EFMT>(W, wave, 4, lo, hi);
  } else {
    lo = 0;
    hi = fmt_loads<EFMT>(W.K);
  }
  const int col0[1] = {kG ? nt * 64 : nt * 64 + 16 * wave};
  const Rsrc hres = make_rsrc(a.hbuf, (uint32_t)a.T * (uint32_t)KP * (uint32_t)a.Imax * XB);
  const Rsrc lres = make_rsrc(list, list ? (uint32_t)cnt * 4u : 0u);
  const Rsrc wres = make_rsrc(a.wts, (uint32_t)a.T * (uint32_t)KP * 4u);
  // output element q of this thread: (row, column)
  auto elem = [&](int q, int& i, int& n) {
    if constexpr (kG) {
      const int idx = threadIdx.x + q * kBlock;
      i = idx / 64;
      n = nt * 64 + idx % 64;
    } else {
      i = 4 * (lane >> 4) + q;
      n = col0[0] + (lane & 15);
    }
  };
  float bias_n[EPI];
#pragma unroll
  for (int q = 0; q < EPI; ++q) {
    int i, n;
    elem(q, i, n);
    bias_n[q] = (W.bias != nullptr && n < H) ? load_scalar(W.bias, n, W.bias_dt) : 0.0f;
  }
  for (int mb = 0; mb < cnt; mb += 16) {
    // list lookups and router weights of the block are issued before the
    // weight stream; only the activation loads wait for them
    const int pa = pair_of_row(lres, list != nullptr, mb + (lane & 15), cnt, KP, shared_col);
    int pe[EPI];
    float we[EPI];
#pragma unroll
    for (int q = 0; q < EPI; ++q) {
      int i, n;
      elem(q, i, n);
      pe[q] = pair_of_row(lres, list != nullptr, mb + i, cnt, KP, shared_col);
    }
#pragma unroll
    for (int q = 0; q < EPI; ++q) we[q] = __uint_as_float(bload4(wres, pe[q] >= 0 ? 4u * (uint32_t)pe[q] : kOOB));
    const uint32_t arow = pa >= 0 ? (uint32_t)pa * (uint32_t)a.Imax * XB : kOOB;
    float yv[EPI];
    if constexpr (kG) {
      f32x4 acc[1][4];
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[0][c] = (f32x4){0.f, 0.f, 0.f, 0.f};
      wave_gemm_gptq<1, AT>(W, col0, lo, hi, hres, arow, acc);
#pragma unroll
      for (int c = 0; c < 4; ++c) red[(wave * 4 + c) * 64 + lane] = acc[0][c];
      __syncthreads();
#pragma unroll
      for (int q = 0; q < EPI; ++q) {
        const int idx = threadIdx.x + q * kBlock;
        const int i = idx / 64, j = idx % 64;
        const int c = j & 3, ln = (j >> 2) + 16 * (i >> 2), rr = i & 3;
        float y = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) y += red[(w * 4 + c) * 64 + ln][rr];
        yv[q] = y;
      }
      __syncthreads();
    } else {
      f32x4 acc[1] = {(f32x4){0.f, 0.f, 0.f, 0.f}};
      wave_gemm_kmajor<EFMT, 1, AT>(W, col0, lo, hi, hres, arow, acc);
#pragma unroll
      for (int q = 0; q < EPI; ++q) yv[q] = acc[0][q];
    }
#pragma unroll
    for (int q = 0; q < EPI; ++q) {
      int i, n;
      elem(q, i, n);
      if (pe[q] >= 0 && n < H) {
        float y = yv[q];
        if (W.bias != nullptr) y += bias_n[q];
        y *= we[q];  // router weight (routed) or sigmoid gate (shared)
        a.ybuf[(size_t)pe[q] * H + n] = y;
      }
    }
  }
}

template <int FMT, int AT>
__global__ __launch_bounds__(kBlock) void k_stage_b(const LayerArgs a) {
  __shared__ f32x4 red[4 * 4 * 64];
  const int H = a.L.hidden;
  const int tiles = H / 64;
  const int u = blockIdx.x / tiles, nt = blockIdx.x % tiles;
  const int uc = min(u, a.L.num_experts);  // uniq / ucnt hold E + 1 entries
  const int e = a.uniq[uc], cnt = a.ucnt[uc];
  const int nU = a.ctrl[kCtrlNU], nRouted = a.ctrl[kCtrlNRouted];
  if (u >= nU) return;
  if (u < nRouted) {
    const int32_t* list = a.lists + (size_t)e * a.T;
    const int slot = a.L.slot_of_expert ? a.L.slot_of_expert[e] : e;
    if (slot < 0 || slot >= a.L.w2.num_slots) {
      // non-resident expert: contribute zeros, flag the error
      for (int idx = threadIdx.x; idx < cnt * 64; idx += kBlock) {
        const int m = idx / 64, n = nt * 64 + idx % 64;
        a.ybuf[(size_t)list[m] * H + n] = 0.0f;
      }
      if (threadIdx.x == 0) atomicOr(&a.ctrl[kCtrlError], 1);
    } else {
      const ProjSlot W = proj_slot(a.L.w2, slot);
      stage_b_body<FMT, AT>(a, W, cnt, list, 0, nt, red);
    }
  } else {
    const ProjSlot W = shared_view(a.L.shared_w2, H, a.L.shared_inter);
    stage_b_body<FTM_FMT_BF16, AT>(a, W, a.T, nullptr, a.L.topk, nt, red);
  }
}

// ============================================================== decode stages, activations in LDS
// Each wave starts its weight window as soon as the expert is known, then
// resolves the token list with scalar loads and copies its K range of the
// block's token rows into its own LDS region by direct global->LDS loads.
// Those copies complete behind the weights (vector loads finish in issue
// order) but hold no registers and depend on nothing the weights wait for,
// so the whole dependent chain (expert table -> token list -> activations)
// overlaps the weight latency.  The MFMAs read the activations from LDS right
// where they are used.  Tokens are taken kXT at a time; each wave's region
// holds kXT token rows and a zero row (index kXT) that MFMA rows kXT..15 and
// out-of-range lanes read.
constexpr int kXT = 4;
constexpr int kXR = kXT + 1;  // LDS rows per wave region
// Dynamic LDS a launch may ask for without raising the kernel's attribute.
constexpr int kDynLdsMax = 65536;
extern __shared__ __align__(16) uint16_t ftm_xl_lds[];

// LDS elements per token row of one wave's region: its K range plus 8 (shifts
// banks).  A wave's range is ceil(ceil(K / kLoadK) / split) wave-loads, at most
// ceil(ceil(K / 128) / split) * 128 elements for every format (kLoadK = 32,
// 64 or 128).
__host__ __device__ __forceinline__ int xl_pitch(int K, int split) {
  return ((K + 127) / 128 + split - 1) / split * 128 + 8;
}

// Zero row kXT of a wave's region (the whole pitch; only this wave reads it).
__device__ __forceinline__ void xl_zero_row(uint16_t* xw, int pitch) {
  const int lane = threadIdx.x & 63;
  for (int e = 8 * lane; e < pitch; e += 8 * 64) *(u32x4*)(xw + kXT * pitch + e) = (u32x4){0u, 0u, 0u, 0u};
}

// Work record of routed expert u (see kRecWords).

// Pairs of tokens [mb, mb + kXT) of a routed expert (block 0 from its record,
// later blocks from its list) or of the shared expert; -1 past cnt.
__device__ __forceinline__ void block_pairs(const LayerArgs& a, const ExpertRec* rec, const int32_t* list,
                                            int shared_col, int cnt, int mb, int (&pr)[kXT]) {
  static_assert(kXT <= kRecPairs, "block 0 pairs come from the record");
#pragma unroll
  for (int i = 0; i < kXT; ++i) {
    const bool ok = mb + i < cnt;
    int p;
    if (list == nullptr)
      p = (mb + i) * a.KP + shared_col;
    else if (mb == 0)
      p = rec->p[i];
    else
      p = ok ? sload_i32(list, mb + i) : -1;
    pr[i] = ok ? p : -1;
  }
}

// Copies bytes [b0, b0 + nbytes) of the rows of the pairs pr (-1 = none)
// into dst (row i at dst + i * pitch bytes).  Row of pair p: src + (p / div) *
// row_bytes.  Returns after issuing the direct global->LDS loads (16 bytes a
// lane; b0, nbytes, row_bytes and pitch are multiples of 16).
__device__ __forceinline__ void lds_fill_rows(const int (&pr)[kXT], const void* src, int div, size_t row_bytes,
                                              size_t b0, uint32_t nbytes, char* dst, uint32_t pitch) {
  typedef __attribute__((address_space(1))) const void* GPtr;
  typedef __attribute__((address_space(3))) void* LPtr;
  const uint32_t lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < kXT; ++i) {
    if (pr[i] >= 0) {
      const char* row = (const char*)src + (size_t)(pr[i] / div) * row_bytes + b0;
      char* d = dst + i * pitch;
      for (uint32_t c = 0; c < nbytes; c += 16u * kWave) {
        if (c + 16u * lane < nbytes)
          __builtin_amdgcn_global_load_lds((GPtr)(row + c + 16u * lane), (LPtr)(d + c), 16, 0, 0);
      }
    }
  }
}

// Elements [k0, k1) of bf16 rows of row_elems elements (see lds_fill_rows).
__device__ __forceinline__ void xl_fill_wave(const int (&pr)[kXT], const void* src, int div, int row_elems, int k0,
                                             int k1, uint16_t* xw, int pitch) {
  lds_fill_rows(pr, src, div, 2u * (size_t)row_elems, 2u * (size_t)k0, 2u * (uint32_t)(k1 - k0), (char*)xw,
                2u * (uint32_t)pitch);
}

// LDS bytes per token row of one wave's region on the MX path: its wave-loads'
// chunks plus 16 (shifts banks).
__host__ __device__ __forceinline__ int mx_pitch(int nL, int split) {
  return (nL + split - 1) / split * kMxChunk + 16;
}

// rows_consume_lds for the MX path: xs holds the block's token rows as
// chunks from wave-load L_lo on (nb rows, `pitch` bytes apart).  No zero
// row: MFMA rows >= nb read row 0 (their outputs are never stored; an MFMA
// row depends on its own A row only), and wave-loads past L_hi read the last
// chunk in range against zero weights (out-of-range weight loads return 0,
// scale 2^-127), which adds 0 since every quantised value is finite.
template <int NLW, int NT>
__device__ __forceinline__ void rows_consume_mx(int Lw, int L_lo, int L_hi,
                                                const RowStream<FTM_FMT_MXFP4, NLW> (&S)[NT], const uint8_t* xs,
                                                int pitch, int nb, f32x4 (&acc)[NT]) {
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4;
  const int m = lane & 15;
  const uint8_t* rb = xs + (m < nb ? m : 0) * pitch - L_lo * kMxChunk;
#pragma unroll
  for (int b = 0; b < NLW; ++b) {
    const int L = Lw + b;
    const uint8_t* cb = rb + min(L, L_hi - 1) * kMxChunk;
    const u32x4 h0 = *(const u32x4*)(cb + 16 * g);
    const u32x4 h1 = *(const u32x4*)(cb + 64 + 16 * g);
    const u32x4 l0 = *(const u32x4*)(cb + 128 + 16 * g);
    const u32x4 l1 = *(const u32x4*)(cb + 192 + 16 * g);
    const uint32_t sc = *(const uint16_t*)(cb + 256 + 2 * g);
    const i32x8 ahi = {(int)h0.x, (int)h0.y, (int)h0.z, (int)h0.w, (int)h1.x, (int)h1.y, (int)h1.z, (int)h1.w};
    const i32x8 alo = {(int)l0.x, (int)l0.y, (int)l0.z, (int)l0.w, (int)l1.x, (int)l1.y, (int)l1.z, (int)l1.w};
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const u32x4 r = S[t].raw[b];
      const i32x8 bw = {(int)r.x, (int)r.y, (int)r.z, (int)r.w, 0, 0, 0, 0};
      const int e8 = ((S[t].vmask >> b) & 1u) ? (int)((S[t].sw[b] >> S[t].sh) & 0xffu) : 0;
      acc[t] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(ahi, bw, acc[t], 0, 4, 0, (int)(sc & 0xffu), 0, e8);
      acc[t] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(alo, bw, acc[t], 0, 4, 0, (int)(sc >> 8), 0, e8);
    }
  }
}

// Stage A item body: NT x 8 channels (per tile 8 gate + 8 up rows) of one
// expert, K split over the 4 waves and reduced through LDS.
// MX: MXFP4 rows on scaled MFMAs, activations from the quantised input xq.
// NLW: wave-loads per prefetch window.
template <int EFMT, int NT, int LPG, bool MX = false, int NLW = kRowsNLW>
__device__ void stage_a_xl_body(const LayerArgs& a, const ProjSlot& W, int Iu, int c0, int cnt,
                                const ExpertRec* rec, const int32_t* list, int shared_col, int kp, f32x4* red) {
  static_assert(!MX || EFMT == FTM_FMT_MXFP4, "scaled MFMAs take MXFP4 rows");
  using F = KMajor<EFMT>;
  constexpr int KS = 4;
  const int lane = threadIdx.x & 63;
  const int n = lane & 15;
  const int H = a.L.hidden;
  const int nL = fmt_loads<EFMT>(W.K);
  const int L_lo = kp * nL / KS, L_hi = (kp + 1) * nL / KS;
  const bool multi = L_hi - L_lo > NLW;
  RowGeom<EFMT> G[NT];
  RowStream<EFMT, NLW> S[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int ct = c0 + 8 * t;
    const int lrow = n < 8 ? ct + n : Iu + ct + (n - 8);
    G[t] = RowGeom<EFMT>(W, lrow, W.group > 0 ? ct / W.group : 0, W.group > 0 ? (Iu + ct) / W.group : 0);
    rows_issue<EFMT, NLW, true>(W, G[t], L_lo, L_hi, S[t]);
  }
  const int pitch = MX ? mx_pitch(nL, KS) : xl_pitch(H, KS);
  uint16_t* xw = ftm_xl_lds + kp * kXR * pitch;
  uint8_t* xm = (uint8_t*)ftm_xl_lds + kp * kXT * pitch;  // MX: kXT rows, no zero row
  if constexpr (!MX) xl_zero_row(xw, pitch);
  const int k0 = L_lo * F::kLoadK, k1 = min(L_hi * F::kLoadK, W.K);
  uint32_t bg[NT], bu[NT];  // bias bits, converted in the epilogue
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    bg[t] = bu[t] = 0u;
    if (W.bias != nullptr && n < 8 && kp == 0) {
      bg[t] = load_bits(W.bias, c0 + 8 * t + n, W.bias_dt);
      bu[t] = load_bits(W.bias, Iu + c0 + 8 * t + n, W.bias_dt);
    }
  }
  for (int mb = 0; mb < cnt; mb += kXT) {
    const int nb = min(kXT, cnt - mb);
    int pr[kXT];
    block_pairs(a, rec, list, shared_col, cnt, mb, pr);
    if constexpr (MX)
      lds_fill_rows(pr, a.xq, a.KP, (size_t)mx_row_bytes(H), (size_t)L_lo * kMxChunk,
                    (uint32_t)(L_hi - L_lo) * kMxChunk, (char*)xm, (uint32_t)pitch);
    else
      xl_fill_wave(pr, a.x, a.KP, H, k0, k1, xw, pitch);
    f32x4 acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = (f32x4){0.f, 0.f, 0.f, 0.f};
    for (int Lw = L_lo; Lw < L_hi; Lw += NLW) {
      // further windows, or the first again for a later token block when the
      // range needs several (re-reads hit L2)
      if (Lw != L_lo || (mb > 0 && multi)) {
#pragma unroll
        for (int t = 0; t < NT; ++t) rows_issue<EFMT, NLW, true>(W, G[t], Lw, L_hi, S[t]);
      }
      __builtin_amdgcn_s_waitcnt(0);  // weights and this wave's LDS copy have landed
      if constexpr (MX)
        rows_consume_mx<NLW, NT>(Lw, L_lo, L_hi, S, xm, pitch, nb, acc);
      else
        rows_consume_lds<EFMT, NLW, NT, LPG, true>(W, G, Lw, L_hi, S, xw, k0, pitch, nb, kXT, acc);
    }
    // MFMA rows 0..kXT-1 (the block's tokens) live in lanes 0..15
    if (lane < 16) {
#pragma unroll
      for (int t = 0; t < NT; ++t) red[(t * KS + kp) * 16 + lane] = acc[t];
    }
    __syncthreads();
    if (kp == 0) {
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        f32x4 v = red[t * KS * 16 + n];
#pragma unroll
        for (int j = 1; j < KS; ++j) v += red[(t * KS + j) * 16 + n];
        const float bgf = bits_to_f32(opaque_bits(bg[t]), W.bias_dt);
        const float buf = bits_to_f32(opaque_bits(bu[t]), W.bias_dt);
#pragma unroll
        for (int r = 0; r < kXT; ++r) {
          const float gs = v[r] + bgf;
          const float us = dpp_f<kDppRowShl8>(v[r]) + buf;
          if (lane < 8 && r < nb) {
            const float h = act_fn(a.L.act, gs, us, a.L.swiglu_alpha, a.L.swiglu_limit);
            store_scalar(a.hbuf, (size_t)pr[r] * a.Imax + c0 + 8 * t + n, FTM_DT_BF16, h);
          }
        }
      }
    }
    __syncthreads();
  }
}

// Minimum waves per SIMD the LDS-activation kernels are compiled for: 5 (<=
// 102 registers) for MXFP4 rows in windows of up to 6 wave-loads without a
// shared expert's bf16 body, where that needs no spills; otherwise the
// compiler's choice.  Measured on MI355X (C4 MXFP4 T=32, k_stage_a_xl with
// scaled-MFMA rows): 72.2 us against 76.8 at the compiler's 116 registers
// (4 waves) and 92.2 at 6 waves (spills).
template <int FMT, int NLW, bool SH, int NT = 1>
constexpr int kXlWaves = (FMT == FTM_FMT_MXFP4 && NLW <= 6 && !SH) ? (NT == 1 ? 5 : 3) : 1;

// NT x 8 channels per workgroup: routed items first, then the shared expert's
// (SH = false: a layer without one, and no bf16 body in the kernel).
template <int FMT, int NT, int LPG, int NLWM = kRowsNLW, bool SH = true>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(kXlWaves<FMT, NLWM, SH, NT>))) void k_stage_a_xl(
    const LayerArgs a) {
  __shared__ f32x4 red[NT * 4 * 16];
  __shared__ RouteA sra;
  const int kp = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int I = a.L.inter;
  const int ti = I / (8 * NT);
  int item = blockIdx.x;
  if (a.route_a) {
    // the shared expert's items first (they need no routing), then the routed ones
    const int nSh = SH && a.L.shared_inter > 0 ? a.L.shared_inter / (8 * NT) : 0;
    if (item < nSh) {
      if constexpr (SH) {
        const int Is = a.L.shared_inter;
        const ProjSlot W = shared_view(a.L.shared_w13, 2 * Is, a.L.hidden);
        stage_a_xl_body<FTM_FMT_BF16, NT, kRowsNLW>(a, W, Is, item * 8 * NT, a.T, nullptr, nullptr, a.L.topk, kp,
                                                     red);
      }
      return;
    }
    item -= nSh;
    const int nR = route_a_prologue(a, sra, item == 0);
    if (item == 0) route_a_publish(a, sra, nR);
    if (item >= nR * ti) return;
    int tot;
    const ExpertRec rec = route_rec_uniform(a, sra.sel, mask_rank(sra.mask, (a.L.num_experts + 31) / 32,
                                                                  item / ti, tot));
    if (rec.slot < 0 || rec.slot >= a.L.w13.num_slots) {
      if (threadIdx.x == 0) atomicOr(&a.ctrl[kCtrlError], 1);
      return;
    }
    const ProjSlot W = proj_slot(a.L.w13, rec.slot);
    stage_a_xl_body<FMT, NT, LPG, FMT == FTM_FMT_MXFP4, NLWM>(a, W, I, (item % ti) * 8 * NT, rec.cnt, &rec,
                                                         a.lists + (size_t)rec.e * a.T, 0, kp, red);
    return;
  }
  const int u = min(item / ti, a.L.num_experts);
  const ExpertRec rec = load_rec(a, u);
  const int nRouted = sload_i32(a.ctrl, kCtrlNRouted);
  if (item < nRouted * ti) {
    if (rec.slot < 0 || rec.slot >= a.L.w13.num_slots) {
      if (threadIdx.x == 0) atomicOr(&a.ctrl[kCtrlError], 1);
      return;
    }
    const ProjSlot W = proj_slot(a.L.w13, rec.slot);
    stage_a_xl_body<FMT, NT, LPG, FMT == FTM_FMT_MXFP4, NLWM>(a, W, I, (item % ti) * 8 * NT, rec.cnt, &rec,
                                                         a.lists + (size_t)rec.e * a.T, 0, kp, red);
  } else if constexpr (SH) {
    const int sitem = item - nRouted * ti;
    const int Is = a.L.shared_inter;
    if (Is <= 0 || sitem >= Is / (8 * NT)) return;
    const ProjSlot W = shared_view(a.L.shared_w13, 2 * Is, a.L.hidden);
    stage_a_xl_body<FTM_FMT_BF16, NT, kRowsNLW>(a, W, Is, sitem * 8 * NT, a.T, nullptr, nullptr, a.L.topk, kp, red);
  }
}

// Stage B item with K split: 16 output columns (w2 rows c0 .. c0 + 15) of one
// expert, K split over the 4 waves and reduced through LDS (the stage-A xl
// data path with plain rows).  For small batches whose 64-column items would
// leave CUs idle and whose rows are too long for one window per wave.
// NLW: wave-loads per prefetch window; NOZ: regions of kXT rows without the
// zero row (rows_consume_lds), their tails past K cleared once here.
// PART: one token block (cnt <= kXT) and no reduction here -- lanes 0..15 store
// this wave's accumulator at red[kp * 16 + lane] and the caller sums the K
// quarters (k_stage_bc_ks); rg: the wave's LDS region (-1: kp).
template <int EFMT, int LPG, int NLW = kRowsNLW, bool NOZ = false, bool PART = false>
__device__ void stage_b_ks_body(const LayerArgs& a, const ProjSlot& W, int c0, int cnt, const ExpertRec* rec,
                                const int32_t* list, int shared_col, int kp, f32x4* red, int mb0 = 0,
                                int rg = -1) {
  using F = KMajor<EFMT>;
  constexpr int KS = 4;
  const int lane = threadIdx.x & 63;
  const int n = lane & 15;
  const int H = a.L.hidden;
  const int nL = fmt_loads<EFMT>(W.K);
  const int L_lo = kp * nL / KS, L_hi = (kp + 1) * nL / KS;
  const bool multi = L_hi - L_lo > NLW;
  RowGeom<EFMT> G[1];
  RowStream<EFMT, NLW> S[1];
  G[0] = RowGeom<EFMT>(W, c0 + n, W.group > 0 ? c0 / W.group : 0, W.group > 0 ? (c0 + 8) / W.group : 0);
  rows_issue<EFMT, NLW, true>(W, G[0], L_lo, L_hi, S[0]);
  const int pitch = xl_pitch(a.Imax, KS);
  uint16_t* xw = ftm_xl_lds + (rg < 0 ? kp : rg) * (NOZ ? kXT : kXR) * pitch;
  const int k0 = L_lo * F::kLoadK, k1 = min(L_hi * F::kLoadK, W.K);
  if constexpr (PART) cnt = min(cnt, mb0 + kXT);
  if constexpr (NOZ) {
    // elements [k1, L_hi * kLoadK) of each row (the last wave's only): read by
    // lanes past K, never filled
    const int t0 = k1 - k0, tl = L_hi * F::kLoadK - k1;
    if (tl > 0) {
      for (int e = lane; e < kXT * tl; e += 64) {
        const int r = e / tl;
        xw[r * pitch + t0 + (e - r * tl)] = 0;
      }
    }
  } else {
    xl_zero_row(xw, pitch);
  }
  const uint32_t bn = (W.bias != nullptr && kp == 0) ? load_bits(W.bias, c0 + n, W.bias_dt) : 0u;  // epilogue
  for (int mb = mb0; mb < cnt; mb += kXT) {
    const int nb = min(kXT, cnt - mb);
    int pr[kXT];
    block_pairs(a, rec, list, shared_col, cnt, mb, pr);
    xl_fill_wave(pr, a.hbuf, 1, a.Imax, k0, k1, xw, pitch);
    f32x4 acc[1] = {(f32x4){0.f, 0.f, 0.f, 0.f}};
    for (int Lw = L_lo; Lw < L_hi; Lw += NLW) {
      if (Lw != L_lo || (mb > mb0 && multi)) rows_issue<EFMT, NLW, true>(W, G[0], Lw, L_hi, S[0]);
      __builtin_amdgcn_s_waitcnt(0);  // weights and this wave's LDS copy have landed
      rows_consume_lds<EFMT, NLW, 1, LPG, true, NOZ>(W, G, Lw, L_hi, S, xw, k0, pitch, nb, kXT, acc);
    }
    // MFMA rows 0..kXT-1 (the block's tokens) live in lanes 0..15, lane n = column c0 + n
    if (lane < 16) red[kp * 16 + lane] = acc[0];
    if constexpr (PART) continue;
    __syncthreads();
    if (kp == 0 && lane < 16) {
      f32x4 v = red[n];
#pragma unroll
      for (int j = 1; j < KS; ++j) v += red[j * 16 + n];
      const float bnf = bits_to_f32(opaque_bits(bn), W.bias_dt);
#pragma unroll
      for (int r = 0; r < kXT; ++r)
        if (r < nb) {
          const float wr = __uint_as_float(sload4(a.wts, 4u * (uint32_t)pr[r]));  // router weight or shared gate
          a.ybuf[(size_t)pr[r] * H + c0 + n] = (v[r] + bnf) * wr;
        }
    }
    __syncthreads();
  }
}

// 16 output columns per workgroup: routed items first, then the shared
// expert's.  SH = false (a layer without one): no bf16 body, and NOZ regions
// for the formats whose zero byte decodes to 0 (the zero weights of
// rows_consume_lds's NOZ contract; INT8's offset-binary 0 is -128).
template <int FMT>
constexpr bool kKsNoz = FMT != FTM_FMT_INT8_PACKED;
template <int FMT, int LPG, int NLWM = kRowsNLW, bool SH = true>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(kXlWaves<FMT, NLWM, SH>))) void k_stage_b_ks(
    const LayerArgs a) {
  __shared__ f32x4 red[4 * 16];
  const int kp = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int H = a.L.hidden;
  const int tn = H / 16;
  const int item = blockIdx.x;
  const int u = min(item / tn, a.L.num_experts);
  const ExpertRec rec = load_rec(a, u);
  const int nRouted = sload_i32(a.ctrl, kCtrlNRouted);
  if (item < nRouted * tn) {
    const int c0 = (item % tn) * 16;
    const int32_t* list = a.lists + (size_t)rec.e * a.T;
    if (rec.slot < 0 || rec.slot >= a.L.w2.num_slots) {
      // non-resident expert: contribute zeros, flag the error
      for (int idx = threadIdx.x; idx < rec.cnt * 16; idx += kBlock)
        a.ybuf[(size_t)list[idx / 16] * H + c0 + idx % 16] = 0.0f;
      if (threadIdx.x == 0) atomicOr(&a.ctrl[kCtrlError], 1);
      return;
    }
    stage_b_ks_body<FMT, LPG, NLWM, !SH && kKsNoz<FMT>>(a, proj_slot(a.L.w2, rec.slot), c0, rec.cnt, &rec, list, 0,
                                                        kp, red);
  } else if constexpr (SH) {
    const int sitem = item - nRouted * tn;
    const int Is = a.L.shared_inter;
    if (Is <= 0 || sitem >= tn) return;
    const ProjSlot W = shared_view(a.L.shared_w2, H, Is);
    stage_b_ks_body<FTM_FMT_BF16, kRowsNLW>(a, W, sitem * 16, a.T, nullptr, nullptr, a.L.topk, kp, red);
  }
}

// ---- K-split stage B and the combine in one launch for up to kBcKsMaxU
// routed experts and kXT tokens (no shared expert; bcks_ok): one workgroup of
// kBcKsWaves waves per 16 output columns takes every routed expert.  Wave w streams K quarter w % 4 of the experts
// w / 4, w / 4 + 4, ... (stage_b_ks_body, PART); the quarters are summed in
// order with the bias and the router weight as k_stage_b_ks does, into the
// pair's slot row in LDS, and the workgroup sums each token's slots in slot
// order (k_combine's order and rounding) into the output.  Saves the combine
// launch and the slot buffer's round trip: at one token the two launches are
// each a ramp and a few dependent round trips over a few MB.  Up to two
// routed experts per wave: measured on MI355X (C4, stage B + combine, us per
// layer): T=1 (4 experts) 26.4 -> 24.4, T=2 (8) 36.9 -> 35.9-36.5, T=4 (16,
// four a wave, one after another) 50.3 -> 50.9-51.2.
constexpr int kBcKsWaves = 16;
constexpr int kBcKsMaxU = 8;    // routed experts (two per wave group of four)
constexpr int kBcKsMaxKP = 64;  // top-k (no shared expert)
template <int FMT, int LPG, int NLW>
__global__ __launch_bounds__(64 * kBcKsWaves) void k_stage_bc_ks(const LayerArgs a) {
  constexpr bool NOZ = kKsNoz<FMT>;
  __shared__ f32x4 red[kBcKsMaxU * 4 * 16];
  __shared__ float s_y[kXT * kBcKsMaxKP * 16];
  __shared__ uint32_t s_bias[kBcKsMaxU * 16];
  __shared__ float s_wr[kBcKsMaxU * kXT];
  __shared__ int s_pr[kBcKsMaxU * kXT];
  __shared__ int s_cnt[kBcKsMaxU];
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kp = wv & 3, ug = wv >> 2;
  const int lane = threadIdx.x & 63;
  const int H = a.L.hidden, T = a.T, KP = a.KP;
  const int c0 = blockIdx.x * 16;
  const int nRouted = sload_i32(a.ctrl, kCtrlNRouted);
  // slots of pairs without an expert stay zero (as their slot-buffer rows would be)
  for (int i = threadIdx.x; i < T * KP * 16; i += 64 * kBcKsWaves) s_y[i] = 0.0f;
  for (int u = ug; u < nRouted; u += 4) {
    const ExpertRec rec = load_rec(a, u);
    const bool ok = rec.slot >= 0 && rec.slot < a.L.w2.num_slots;
    if (!ok) {  // non-resident expert: contributes zeros, flags the error
      if (kp == 0 && lane == 0) {
        s_cnt[u] = 0;
        atomicOr(&a.ctrl[kCtrlError], 1);
      }
      continue;
    }
    const ProjSlot W = proj_slot(a.L.w2, rec.slot);
    // the epilogue's operands, requested before the weights' wait in the body
    uint32_t bb = 0u;
    float wr = 0.0f;
    int pr = -1;
    if (kp == 0) {
      if (W.bias != nullptr && lane < 16) bb = load_bits(W.bias, c0 + lane, W.bias_dt);
      pr = lane == 0 ? rec.p[0] : lane == 1 ? rec.p[1] : lane == 2 ? rec.p[2] : rec.p[3];
      if (lane < kXT && lane < rec.cnt) wr = a.wts[pr];
    }
    stage_b_ks_body<FMT, LPG, NLW, NOZ, true>(a, W, c0, rec.cnt, &rec, a.lists + (size_t)rec.e * T, 0, kp,
                                              red + u * 4 * 16, 0, wv);
    if (kp == 0) {
      if (lane < 16) s_bias[u * 16 + lane] = bb;
      if (lane < kXT) {
        s_wr[u * kXT + lane] = wr;
        s_pr[u * kXT + lane] = pr;
      }
      if (lane == 0) s_cnt[u] = rec.cnt;
    }
  }
  __syncthreads();
  // slot rows: the K quarters in order, + bias, x router weight (k_stage_b_ks's epilogue)
  for (int i = threadIdx.x; i < nRouted * 16; i += 64 * kBcKsWaves) {
    const int u = i >> 4, n = i & 15;
    const int cnt = s_cnt[u];
    if (cnt == 0) continue;
    f32x4 v = red[(u * 4) * 16 + n];
#pragma unroll
    for (int j = 1; j < 4; ++j) v += red[(u * 4 + j) * 16 + n];
    const float bnf = bits_to_f32(opaque_bits(s_bias[u * 16 + n]), a.L.w2.bias_dtype);
#pragma unroll
    for (int r = 0; r < kXT; ++r)
      if (r < cnt) s_y[s_pr[u * kXT + r] * 16 + n] = (v[r] + bnf) * s_wr[u * kXT + r];
  }
  __syncthreads();
  for (int i = threadIdx.x; i < T * 16; i += 64 * kBcKsWaves) {
    const int t = i >> 4, n = i & 15;
    float sum = s_y[(t * KP) * 16 + n];
    for (int j = 1; j < KP; ++j) sum += s_y[(t * KP + j) * 16 + n];
    ((uint16_t*)a.out)[(size_t)t * H + c0 + n] = f32_to_bf16(sum);
  }
}

// ---------------------------------------------------------------- token-resident stages
// For about 6 to 16 tokens per routed expert (MXFP4 decode batches): the
// LDS-activation kernels above take a token block of kXT rows at a time and
// split K over the 4 waves of a 16-row item, so every item copies its tokens'
// rows from L2 once per block -- about four times its weight bytes at 16
// tokens per expert, in four dependent round trips.  Here a workgroup of 8
// waves copies one block of up to kTokMaxRows token rows of its expert (bf16,
// the whole K range) into LDS once, and each wave streams 16 weight rows over
// the whole K range through registers, two windows of kTokNLW wave-loads in
// flight, multiplying each window against every token of the block (one or
// two 16-row MFMA tiles).  The copy is shared by the workgroup's 128 weight
// rows and no cross-wave reduction is needed.
//   stage A: wave w takes channels c0 + 8 w .. + 7 (8 gate and the matching 8
//            up rows of w13) and writes their h;
//   stage B: wave w takes output columns c0 + 16 w .. + 15 of w2 and writes
//            router-weighted fp32 rows into the slot buffer (k_combine sums).
// Blocks beyond kTokMaxRows tokens (or what the LDS holds) stream the weights
// again.  Formats whose zero byte decodes to 0 (the NOZ contract of
// rows_consume_lds), no shared expert.  One workgroup fits a CU (the rows take
// the LDS).  Measured on MI355X (C4, us per layer, T = 64 / 128): 175 / 243
// on k_stage_a_xl + k_stage_b_ks; here one tile per workgroup 146 / 161, runs
// of tiles per workgroup 128 / 142.  Not faster: windows of 6, 8 or 12
// wave-loads (8 and 12: 136 / 156), 12 waves per workgroup (130 / 145), K
// split over two wave groups (152 / 199) or over four quarters per row group
// (140 / 216); the weight stream without the MFMAs runs at the same speed
// (128 / 139), so it is the loads of 16 rows x 64 bytes per wave-load with one
// workgroup per CU, at ~4 TB/s, that bound it.
constexpr int kTokWaves = 8;
constexpr int kTokThreads = 64 * kTokWaves;
constexpr int kTokMaxRows = 32;  // two MFMA row tiles
constexpr int kTokNLW = 4;  // wave-loads per window (two windows in flight)
constexpr int kTokMaxTiles = 8;  // column tiles per workgroup
constexpr int kTokTileVals = 128;  // bias values per column tile (A: 64 gate + 64 up, B: 128 columns)
// dynamic LDS: the CU's 160 KiB less the static pairs, router weights and biases
constexpr int kTokLdsMax = 160 * 1024 - 2 * 4 * kTokMaxRows - 4 * kTokMaxTiles * kTokTileVals - 256;

// LDS row pitch (elements) of K-element bf16 rows read by K-major wave-loads of
// kload elements: the K range rounded up to whole wave-loads (the tail stays
// zero), plus 8 so that the 16 rows of one MFMA operand read fall on
// different banks.
__host__ __device__ __forceinline__ int tok_pitch(int K, int kload) { return (K + kload - 1) / kload * kload + 8; }
__host__ __device__ __forceinline__ int tok_rows(int K, int kload) {
  const int r = kTokLdsMax / (2 * tok_pitch(K, kload));
  return r < kTokMaxRows ? r : kTokMaxRows;
}

// Weight row of lane row n (0..15) of wave `wave` in column tile ct: stage A
// the 8 gate rows of channels c0 .. c0 + 7 then their 8 up rows, stage B
// output columns c0 .. c0 + 15; -1 past the projection or for ct < 0 (a tile
// past the workgroup's run, whose prefetch must load nothing).
template <bool STB>
__device__ __forceinline__ int tok_row(const LayerArgs& a, int ct, int wave, int n, int& c0) {
  const int H = a.L.hidden, I = a.L.inter;
  if constexpr (STB) {
    c0 = ct * (16 * kTokWaves) + 16 * wave;
    return ct >= 0 && c0 + n < H ? c0 + n : -1;
  } else {
    c0 = ct * (8 * kTokWaves) + 8 * wave;
    return ct >= 0 && c0 + (n & 7) < I ? (n < 8 ? c0 + n : I + c0 + n - 8) : -1;
  }
}

template <int EFMT, bool STB>
__device__ __forceinline__ RowGeom<EFMT> tok_geom(const LayerArgs& a, const ProjSlot& W, int ct, int wave, int n) {
  int c0;
  const int lrow = tok_row<STB>(a, ct, wave, n, c0);
  const int sb_lo = W.group > 0 ? c0 / W.group : 0;
  const int sb_hi = W.group > 0 ? (STB ? c0 : a.L.inter + c0) / W.group : 0;
  return RowGeom<EFMT>(W, lrow, sb_lo, sb_hi);
}

// The MFMAs of one weight window against one or two 16-row token tiles (TWO)
// of the resident rows.  Each wave-load's weights are decoded once for both
// tiles, and the LDS reads of wave-load b + 1 are issued before the MFMAs of b
// (one wave-load ahead, not the whole window: the registers go to the weight
// windows in flight).  NOZ semantics of rows_consume_lds: rows >= nb read the
// tile's first row, wave-loads past L_hi the last one in range against zero
// weights, lanes past K the zeroed row tails.
template <int FMT, int NLW, int LPG, bool PAIRED, bool TWO>
__device__ __forceinline__ void tok_consume(const ProjSlot& W, const RowGeom<FMT>& G, int Lw, int L_hi,
                                            const RowStream<FMT, NLW>& S, const uint16_t* xs, int pitch, int nb,
                                            f32x4& acc0, f32x4& acc1) {
  using F = KMajor<FMT>;
  static_assert(NLW % LPG == 0, "groups tile the window");
  constexpr int QM = F::kMfma;
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4, m = lane & 15;
  const bool upper = m >= 8;
  const uint16_t* x0 = xs + (m < nb ? m : 0) * pitch + F::kLaneK * g;
  const uint16_t* x1 = xs + (16 + m < nb ? 16 + m : 16) * pitch + F::kLaneK * g;
  constexpr int NP = F::kPostScale ? NLW / LPG : 1;
  f32x4 p0[NP], p1[NP];
#pragma unroll
  for (int i = 0; i < NP; ++i) p0[i] = p1[i] = (f32x4){0.f, 0.f, 0.f, 0.f};
  // the first tile's reads run one wave-load ahead; the second tile's are
  // issued with the wave-load's own MFMAs
  u32x4 n0[QM];
  {
    const int kk = min(Lw, L_hi - 1) * F::kLoadK;
#pragma unroll
    for (int q = 0; q < QM; ++q) n0[q] = *(const u32x4*)(x0 + kk + 8 * q);
  }
#pragma unroll
  for (int b = 0; b < NLW; ++b) {
    u32x4 c0[QM], c1[QM];
#pragma unroll
    for (int q = 0; q < QM; ++q) c0[q] = n0[q];
    if constexpr (TWO) {
      const int kk = min(Lw + b, L_hi - 1) * F::kLoadK;
#pragma unroll
      for (int q = 0; q < QM; ++q) c1[q] = *(const u32x4*)(x1 + kk + 8 * q);
    }
    if (b + 1 < NLW) {
      const int kk = min(Lw + b + 1, L_hi - 1) * F::kLoadK;
#pragma unroll
      for (int q = 0; q < QM; ++q) n0[q] = *(const u32x4*)(x0 + kk + 8 * q);
    }
    const u32x4 r = S.raw[b];
    const int pi = F::kPostScale ? b / LPG : 0;
#pragma unroll
    for (int q = 0; q < QM; ++q) {
      u32x4 bq;
      if constexpr (FMT == FTM_FMT_FP8_BLOCK) {
        bq = q == 0 ? fp8x8_to_bf16(r.x, r.y) : fp8x8_to_bf16(r.z, r.w);
      } else if constexpr (FMT == FTM_FMT_MXFP4) {
        const uint32_t wq = q == 0 ? r.x : q == 1 ? r.y : q == 2 ? r.z : r.w;
        const uint32_t e8 = ((S.vmask >> b) & 1u) ? (S.sw[b] >> S.sh) & 0xffu : 0u;
        bq = fp4x8_to_bf16(wq, e8m0_to_f32(e8));
      } else {
        bq = r;
      }
      p0[pi] = mfma_bf16(c0[q], bq, p0[pi]);
      if constexpr (TWO) p1[pi] = mfma_bf16(c1[q], bq, p1[pi]);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  if constexpr (F::kPostScale) {
    const int g0 = Lw / G.lpg;
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      const int b = i * LPG;  // first wave-load of the group
      uint32_t sidx;
      if constexpr (FMT == FTM_FMT_FP8_BLOCK)
        sidx = (((PAIRED && upper) ? G.fp8_hi : G.fp8_lo) / G.sesz) + (uint32_t)(g0 + i);
      else
        sidx = G.soff + (uint32_t)(g0 + i);
      const float s_grp = (Lw + b < L_hi) ? decode_scalar_word(S.sw[b], sidx, W.s_dt) : 0.0f;
      acc0 += p0[i] * s_grp;
      if constexpr (TWO) acc1 += p1[i] * s_grp;
    }
  } else {
    acc0 += p0[0];
    if constexpr (TWO) acc1 += p1[0];
  }
}

// One workgroup per (routed expert, group of ni consecutive column tiles):
// the expert's token rows are copied once and the weight stream runs on
// through the tiles (the next tile's first windows in flight during the
// current tile's last), so the launch is about one workgroup per CU, each
// streaming without a gap between its tiles.
template <int EFMT, bool STB>
__device__ __forceinline__ void stage_tok_body(const LayerArgs& a, int ni) {
  using F = KMajor<EFMT>;
  constexpr int NLW = kTokNLW;
  constexpr int LPG = F::kPostScale ? 2 : NLW;
  typedef __attribute__((address_space(1))) const void* GPtr;
  typedef __attribute__((address_space(3))) void* LPtr;
  __shared__ int s_pr[kTokMaxRows];
  __shared__ float s_w[kTokMaxRows];                      // stage B: the block's router weights
  __shared__ float s_bias[kTokMaxTiles * kTokTileVals];  // the tiles' biases (f32)
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, n = lane & 15, g = lane >> 4;
  const int H = a.L.hidden, I = a.L.inter;
  const int K = STB ? I : H;
  const int nct = ((STB ? H : I) + (STB ? 16 : 8) * kTokWaves - 1) / ((STB ? 16 : 8) * kTokWaves);
  const int ngrp = (nct + ni - 1) / ni;
  // an expert's runs on one XCD: its token rows are fetched into one L2
  const int b = xcd_item((int)blockIdx.x, (int)gridDim.x);
  const int u = b / ngrp;
  const int ct0 = (b % ngrp) * ni;
  const int nti = min(ni, nct - ct0);  // column tiles of this workgroup
  const int nRouted = sload_i32(a.ctrl, kCtrlNRouted);
  if (u >= nRouted) return;
  const ExpertRec rec = load_rec(a, u);
  const int32_t* list = a.lists + (size_t)rec.e * a.T;
  const ftm_proj& P = STB ? a.L.w2 : a.L.w13;
  if (rec.slot < 0 || rec.slot >= P.num_slots) {
    // non-resident expert: stage B contributes zeros; both flag the error
    if constexpr (STB) {
      for (int it = 0; it < nti; ++it) {
        int c0;
        (void)tok_row<true>(a, ct0 + it, wave, 0, c0);
        for (int idx = lane; idx < rec.cnt * 16; idx += 64) {
          const int col = c0 + idx % 16;
          if (col < H) a.ybuf[(size_t)sload_i32(list, idx / 16) * H + col] = 0.0f;
        }
      }
    }
    if (threadIdx.x == 0) atomicOr(&a.ctrl[kCtrlError], 1);
    return;
  }
  const ProjSlot W = proj_slot(P, rec.slot);
  const int nL = fmt_loads<EFMT>(K);
  const int nwin = ((nL + NLW - 1) / NLW + 1) / 2 * 2;  // windows per tile, even (a pad window loads nothing)
  const int pitch = tok_pitch(K, F::kLoadK);
  const int rows_max = tok_rows(K, F::kLoadK);
  const uint32_t pb = 2u * (uint32_t)pitch;  // row pitch in bytes
  uint16_t* xs = ftm_xl_lds;
  // the rows' tails [K, pitch) are never copied: zero them once
  {
    const int tq = (pitch - K) / 8;  // 16-byte pieces per tail
    for (int i = threadIdx.x; i < rows_max * tq; i += kTokThreads) {
      const int r = i / tq, q = i % tq;
      *(u32x4*)(xs + r * pitch + K + 8 * q) = (u32x4){0u, 0u, 0u, 0u};
    }
  }
  const char* src = STB ? (const char*)a.hbuf : (const char*)a.x;
  const size_t src_row = STB ? 2u * (size_t)a.Imax : 2u * (size_t)H;  // bytes per source row
  const int div = STB ? 1 : a.KP;                                      // source row of pair p: p / div
  for (int mb = 0; mb < rec.cnt; mb += rows_max) {
    const int nb = min(rows_max, rec.cnt - mb);
    const bool two = nb > 16;
    __syncthreads();  // the previous block's reads of s_pr and the rows are done
    // The epilogues take the pairs, router weights and biases from LDS: a
    // vector load used after the window loop would wait for the next tile's
    // windows in flight.  The loads issue here and land with the copies.
    float wv = 0.0f;
    if (threadIdx.x < nb) {
      const int m = mb + threadIdx.x;
      int p = -1;
#pragma unroll
      for (int q = 0; q < kRecPairs; ++q) p = m == q ? rec.p[q] : p;
      p = m < kRecPairs ? p : list[m];
      s_pr[threadIdx.x] = p;
      if constexpr (STB) wv = a.wts[p];
    }
    uint32_t bv[2] = {0u, 0u};  // raw bits, converted once the copies have landed
    if (W.bias != nullptr) {
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int i = threadIdx.x + q * kTokThreads;
        const int it = i / kTokTileVals, j = i % kTokTileVals;
        int col = -1;
        if (it < nti) {
          if constexpr (STB) {
            col = (ct0 + it) * kTokTileVals + j;
            col = col < H ? col : -1;
          } else {
            const int c = (ct0 + it) * (8 * kTokWaves) + (j & 63);
            col = c < I ? (j < 64 ? c : I + c) : -1;
          }
        }
        if (col >= 0) bv[q] = load_bits(W.bias, col, W.bias_dt);
      }
    }
    // the first tile's first two windows, then the block's rows
    RowGeom<EFMT> G[1] = {tok_geom<EFMT, STB>(a, W, ct0, wave, n)};
    RowStream<EFMT, NLW> S0[1], S1[1];
    rows_issue<EFMT, NLW, !STB>(W, G[0], 0, nL, S0[0]);
    rows_issue<EFMT, NLW, !STB>(W, G[0], NLW, nL, S1[0]);
    __syncthreads();  // s_pr
    const uint32_t nbytes = (uint32_t)nb * pb;
    for (uint32_t c = (uint32_t)wave * 1024u; c < nbytes; c += 1024u * kTokWaves) {
      const uint32_t d = c + 16u * (uint32_t)lane;
      const uint32_t r = d / pb, off = d - r * pb;
      if (r < (uint32_t)nb && off < 2u * (uint32_t)K) {
        const char* row = src + (size_t)(s_pr[r] / div) * src_row + off;
        __builtin_amdgcn_global_load_lds((GPtr)row, (LPtr)((char*)xs + c), 16, 0, 0);
      }
    }
    __builtin_amdgcn_s_waitcnt(0);  // this wave's copies (and the first windows) have landed
    if (STB && threadIdx.x < nb) s_w[threadIdx.x] = wv;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int i = threadIdx.x + q * kTokThreads;
      if (i < kTokMaxTiles * kTokTileVals) s_bias[i] = bits_to_f32(opaque_bits(bv[q]), W.bias_dt);
    }
    __syncthreads();                // every wave's copies
    for (int it = 0; it < nti; ++it) {
      // acc0 / acc1: tokens 0-15 / 16-31 of the block (MFMA row tiles)
      f32x4 acc0[1] = {(f32x4){0.f, 0.f, 0.f, 0.f}}, acc1[1] = {(f32x4){0.f, 0.f, 0.f, 0.f}};
      const RowGeom<EFMT> Gc[1] = {G[0]};
      // the windows after this tile's last two are the next tile's first two
      // (nothing past the run: those tiles are another workgroup's)
      const RowGeom<EFMT> Gn = tok_geom<EFMT, STB>(a, W, it + 1 < nti ? ct0 + it + 1 : -1, wave, n);
      int c0;
      const int lrow = tok_row<STB>(a, ct0 + it, wave, n, c0);
      for (int w = 0; w < nwin; w += 2) {
        const bool last = w + 2 >= nwin;
        const int Lw = w * NLW;
        if (two)
          tok_consume<EFMT, NLW, LPG, !STB, true>(W, Gc[0], Lw, nL, S0[0], xs, pitch, nb, acc0[0], acc1[0]);
        else
          tok_consume<EFMT, NLW, LPG, !STB, false>(W, Gc[0], Lw, nL, S0[0], xs, pitch, nb, acc0[0], acc1[0]);
        // unconditional: past the tiles and past K the loads fetch nothing
        rows_issue<EFMT, NLW, !STB>(W, last ? Gn : Gc[0], last ? 0 : Lw + 2 * NLW, nL, S0[0]);
        if (two)
          tok_consume<EFMT, NLW, LPG, !STB, true>(W, Gc[0], Lw + NLW, nL, S1[0], xs, pitch, nb, acc0[0], acc1[0]);
        else
          tok_consume<EFMT, NLW, LPG, !STB, false>(W, Gc[0], Lw + NLW, nL, S1[0], xs, pitch, nb, acc0[0], acc1[0]);
        rows_issue<EFMT, NLW, !STB>(W, last ? Gn : Gc[0], last ? NLW : Lw + 3 * NLW, nL, S1[0]);
      }
      G[0] = Gn;
      // MFMA lane (g, n) holds tokens 4 g + r (r = 0..3) of its tile, weight row n of the wave's 16
      const float* sb = s_bias + it * kTokTileVals;
      const float bgf = STB ? sb[16 * wave + n] : sb[8 * wave + (n & 7)];
      const float buf = STB ? 0.0f : sb[64 + 8 * wave + (n & 7)];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const f32x4 acc = t == 0 ? acc0[0] : acc1[0];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int tok = 16 * t + 4 * g + r;
          if constexpr (STB) {
            if (tok < nb && lrow >= 0) a.ybuf[(size_t)s_pr[tok] * H + c0 + n] = (acc[r] + bgf) * s_w[tok];
          } else {
            const float gs = acc[r] + bgf;
            const float us = dpp_f<kDppRowShl8>(acc[r]) + buf;
            if (n < 8 && tok < nb && lrow >= 0) {
              const float h = act_fn(a.L.act, gs, us, a.L.swiglu_alpha, a.L.swiglu_limit);
              store_scalar(a.hbuf, (size_t)s_pr[tok] * a.Imax + c0 + n, FTM_DT_BF16, h);
            }
          }
        }
      }
    }
  }
}

// Stage A (w13 + activation) and stage B (w2) on the token-resident body.
template <int EFMT>
__global__ __launch_bounds__(kTokThreads) void k_stage_tok_a(const LayerArgs a, int ni) {
  stage_tok_body<EFMT, false>(a, ni);
}
template <int EFMT>
__global__ __launch_bounds__(kTokThreads) void k_stage_tok_b(const LayerArgs a, int ni) {
  stage_tok_body<EFMT, true>(a, ni);
}

// GPTQ stage B: the shared expert's items first, 16 output columns each with
// K split over the 4 waves (stage_b_ks_body) and its tokens in blocks of
// kGqBShXT, one workgroup per (block, 16 columns); then the routed experts'
// 128-column items (stage_b_gq).  Measured on MI355X with a Qwen1.5-MoE-A2.7B
// shaped layer (60 GPTQ experts of 1408, top-4, a bf16 shared expert of
// 5632): stage B T=1 35.4 -> 15.2 us, T=16 60.8 -> 34.8, T=32 101 -> 61
// against 64-column shared items over every token (H / 64 = 32 workgroups of
// 720 KB each); blocks of 4 or 16 tokens: within 1 us of 8 up to T=16.
constexpr int kGqBShXT = 8;
__host__ __device__ __forceinline__ int gq_b_sh_items(const ftm_moe_layer& L, int T) {
  return L.shared_inter > 0 ? (L.hidden / 16) * ((T + kGqBShXT - 1) / kGqBShXT) : 0;
}

// Layers the GPTQ decode stage B takes: the routed items' K halves within
// kGqMaxKR, the shared expert's LDS regions (4 waves x kXT rows of a quarter
// of K) within 64 KiB.
static bool gq_b_ok(const ftm_moe_layer& L, int T) {
  const ftm_proj& B = L.w2;
  if (B.fmt != FTM_FMT_GPTQ_INT4 || L.act_dtype != FTM_DT_BF16 || B.group != 128) return false;
  if (L.hidden % kGqNB != 0 || L.inter % 128 != 0 || T > kGqBMaxT) return false;
  if (L.shared_inter > 0) {
    const int imax = L.inter > L.shared_inter ? L.inter : L.shared_inter;
    if (L.shared_inter % 8 != 0 || 4 * kXR * xl_pitch(imax, 4) * 2 > kDynLdsMax) return false;
  }
  return (L.inter / 128 + 1) / 2 * 128 <= kGqMaxKR;
}

template <bool ALL, int NB>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(ALL ? 1 : 3))) void k_stage_b_gq(const LayerArgs a) {
  // routed items: the reduction buffer (16 KiB) aliases the h-row regions;
  // the shared expert's K-split items keep a small one of their own (their
  // waves' regions are in use while other waves reduce)
  __shared__ f32x4 red_s[4 * 16];
  const int H = a.L.hidden;
  const int tilesR = H / NB;
  const int nSh = gq_b_sh_items(a.L, a.T);
  const int item = (int)blockIdx.x;
  if (item < nSh) {
    const int tn = H / 16, b = item / tn, c0 = (item % tn) * 16;
    const int kp = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const ProjSlot W = shared_view(a.L.shared_w2, H, a.L.shared_inter);
    stage_b_ks_body<FTM_FMT_BF16, kRowsNLW>(a, W, c0, min(a.T, (b + 1) * kGqBShXT), nullptr, nullptr, a.L.topk, kp,
                                            red_s, b * kGqBShXT);
    return;
  }
  const int ritem = item - nSh;
  const int nRouted = sload_i32(a.ctrl, kCtrlNRouted);
  if (ritem >= nRouted * tilesR) return;
  const int u = ritem / tilesR, it = ritem % tilesR;
  const int e = sload_i32(a.uniq, u), cnt = sload_i32(a.ucnt, u);
  const int32_t* list = a.lists + (size_t)e * a.T;
  const int slot = a.L.slot_of_expert ? sload_i32(a.L.slot_of_expert, e) : e;
  if (slot < 0 || slot >= a.L.w2.num_slots) {
    // non-resident expert: contribute zeros, flag the error
    for (int idx = threadIdx.x; idx < cnt * NB; idx += kBlock) {
      const int m = idx / NB, n = it * NB + idx % NB;
      a.ybuf[(size_t)list[m] * H + n] = 0.0f;
    }
    if (threadIdx.x == 0) atomicOr(&a.ctrl[kCtrlError], 1);
    return;
  }
  stage_b_gq<ALL, NB>(a, proj_slot(a.L.w2, slot), it, cnt, list, (f32x4*)ftm_xl_lds);
}

// Stage B item body: NT x 64 output columns of one expert; in each 64-column
// tile wave w owns columns 16w .. 16w + 15, over the full K (no cross-wave
// reduction).
template <int EFMT, int NT, int LPG>
__device__ void stage_b_xl_body(const LayerArgs& a, const ProjSlot& W, int cnt, const ExpertRec* rec,
                                const int32_t* list, int shared_col, int nt, int wv) {
  const int lane = threadIdx.x & 63;
  const int n = lane & 15;
  const int H = a.L.hidden;
  const int lo = 0, hi = fmt_loads<EFMT>(W.K);
  const bool multi = hi - lo > kRowsNLW;
  RowGeom<EFMT> G[NT];
  RowStream<EFMT, kRowsNLW> S[NT];
  int brow[NT];
  float bias_n[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int col0 = (nt * NT + t) * 64 + 16 * wv;
    brow[t] = col0 + n;
    const int sb = W.group > 0 ? col0 / W.group : 0;
    G[t] = RowGeom<EFMT>(W, brow[t] < W.N ? brow[t] : -1, sb, sb);
    rows_issue<EFMT, kRowsNLW, false>(W, G[t], lo, hi, S[t]);
    bias_n[t] = (W.bias != nullptr && brow[t] < H) ? load_scalar(W.bias, brow[t], W.bias_dt) : 0.0f;
  }
  const int K = W.K;
  const int pitch = xl_pitch(a.Imax, 1);
  uint16_t* xw = ftm_xl_lds + wv * kXR * pitch;
  xl_zero_row(xw, pitch);
  for (int mb = 0; mb < cnt; mb += kXT) {
    const int nb = min(kXT, cnt - mb);
    int pr[kXT];
    block_pairs(a, rec, list, shared_col, cnt, mb, pr);
    xl_fill_wave(pr, a.hbuf, 1, a.Imax, 0, K, xw, pitch);
    float wr[kXT];
#pragma unroll
    for (int r = 0; r < kXT; ++r) wr[r] = pr[r] >= 0 ? __uint_as_float(sload4(a.wts, 4u * (uint32_t)pr[r])) : 0.0f;
    f32x4 acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = (f32x4){0.f, 0.f, 0.f, 0.f};
    for (int Lw = lo; Lw < hi; Lw += kRowsNLW) {
      if (Lw != lo || (mb > 0 && multi)) {
#pragma unroll
        for (int t = 0; t < NT; ++t) rows_issue<EFMT, kRowsNLW, false>(W, G[t], Lw, hi, S[t]);
      }
      __builtin_amdgcn_s_waitcnt(0);  // weights and this wave's LDS copy have landed
      rows_consume_lds<EFMT, kRowsNLW, NT, LPG, false>(W, G, Lw, hi, S, xw, 0, pitch, nb, kXT, acc);
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
#pragma unroll
      for (int r = 0; r < kXT; ++r) {
        if (lane < 16 && r < nb && brow[t] < H) {
          float y = acc[t][r];
          if (W.bias != nullptr) y += bias_n[t];
          y *= wr[r];  // router weight (routed) or sigmoid gate (shared)
          a.ybuf[(size_t)pr[r] * H + brow[t]] = y;
        }
      }
    }
  }
}

template <int FMT, int NT, int LPG>
__global__ __launch_bounds__(kBlock) void k_stage_b_xl(const LayerArgs a) {
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int H = a.L.hidden;
  const int tiles = H / (64 * NT);
  const int u = blockIdx.x / tiles, nt = blockIdx.x % tiles;
  const int uc = min(u, a.L.num_experts);
  const ExpertRec rec = load_rec(a, uc);
  const int nU = sload_i32(a.ctrl, kCtrlNU), nRouted = sload_i32(a.ctrl, kCtrlNRouted);
  if (u >= nU) return;
  if (u < nRouted) {
    const int32_t* list = a.lists + (size_t)rec.e * a.T;
    if (rec.slot < 0 || rec.slot >= a.L.w2.num_slots) {
      // non-resident expert: contribute zeros, flag the error
      for (int idx = threadIdx.x; idx < rec.cnt * 64 * NT; idx += kBlock) {
        const int m = idx / (64 * NT), c = nt * 64 * NT + idx % (64 * NT);
        a.ybuf[(size_t)list[m] * H + c] = 0.0f;
      }
      if (threadIdx.x == 0) atomicOr(&a.ctrl[kCtrlError], 1);
      return;
    }
    const ProjSlot W = proj_slot(a.L.w2, rec.slot);
    stage_b_xl_body<FMT, NT, LPG>(a, W, rec.cnt, &rec, list, 0, nt, wv);
  } else {
    const ProjSlot W = shared_view(a.L.shared_w2, H, a.L.shared_inter);
    stage_b_xl_body<FTM_FMT_BF16, NT, kRowsNLW>(a, W, a.T, nullptr, nullptr, a.L.topk, nt, wv);
  }
}

// ============================================================== lean decode stages (FP8 block-128 layers)
// The hot decode shape (FP8 block-128 experts with fp32 scales, bf16
// activations, no projection biases, optional dense bf16 shared expert) gets
// kernels with nothing else in them: per wave one window of weights issued as
// soon as the expert record is read, the scale words with two scalar loads,
// the block's activation rows copied to LDS by one direct global->LDS load per
// token, LDS reads at fixed offsets (MFMA rows past the block read a zero
// row), one accumulator per quantisation group.  Measured with a stripped
// probe of this pattern on MI355X: 6.1 TB/s on the C3 T=16 w13 bytes, where
// per-lane activation loads cap the same stream at 4.7 TB/s (they triple the
// vector memory instructions per weight byte).
constexpr int kLeanXT = 4;  // tokens per block (MFMA rows 0..3; rows 4..15 read the zero row)

// LDS elements per token row of a wave's region (K range + 8: shifts banks).
__host__ __device__ __forceinline__ constexpr int lean_pitch(int KR) { return KR + 8; }

// One wave's weight window: NLW wave-loads of 16 bytes per lane.
template <int NLW>
struct LeanWin {
  u32x4 raw[NLW];
};

// Issue window [w0, w0 + NLW) wave-loads of a row-major weight matrix:
// lane (n, g) reads row `row` (< 0: none) at byte (kbase + (w0 + b) * 64 + 16 g).
template <int NLW>
__device__ __forceinline__ void lean_issue(Rsrc wres, int row, uint32_t row_bytes, uint32_t kbase, int w0,
                                           LeanWin<NLW>& S) {
  const int g = (threadIdx.x & 63) >> 4;
  const uint32_t base = row >= 0 ? (uint32_t)row * row_bytes + kbase + 16u * (uint32_t)g : kOOB;
#pragma unroll
  for (int b = 0; b < NLW; ++b) S.raw[b] = bload16(wres, base == kOOB ? kOOB : base + 64u * (uint32_t)(w0 + b));
}

// Copy elements [k0, k0 + KR) of the rows of pairs pr[0..nb) into xw (row r at
// xw + r * pitch); row of pair p at src + (p / div) * row_elems elements.
template <int KR>
__device__ __forceinline__ void lean_fill(const int (&pr)[kLeanXT], int nb, const void* src, int div, int row_elems,
                                          int k0, uint16_t* xw) {
  typedef __attribute__((address_space(1))) const void* GPtr;
  typedef __attribute__((address_space(3))) void* LPtr;
  const uint32_t lane = threadIdx.x & 63;
#pragma unroll
  for (int r = 0; r < kLeanXT; ++r) {
    if (r < nb) {
      const char* row = (const char*)src + ((size_t)(pr[r] / div) * (size_t)row_elems + (size_t)k0) * 2u;
#pragma unroll
      for (int c = 0; c < (2 * KR + 1023) / 1024; ++c) {
        if (c * 1024 + 16 * (int)lane < 2 * KR)
          __builtin_amdgcn_global_load_lds((GPtr)(row + c * 1024 + 16 * lane),
                                           (LPtr)((char*)(xw + r * lean_pitch(KR)) + c * 1024), 16, 0, 0);
      }
    }
  }
}

// MFMAs of one window.  FP8: wave-load b of window w belongs to group
// (w * NLW + b) / 2 (64 K per wave-load, 128 per group), accumulated in
// part[]; BF16: one accumulator part[0].  xrow: this lane's LDS row
// (token l % 16, or the zero row), element kw = the window's first K offset
// within the wave's range.
template <bool FP8, int NLW, int NP>
__device__ __forceinline__ void lean_mfma(const LeanWin<NLW>& S, const uint16_t* xrow, int kw, f32x4 (&part)[NP],
                                          int pbase) {
  const int g = (threadIdx.x & 63) >> 4;
  constexpr int kLoadK = FP8 ? 64 : 32, kLaneK = FP8 ? 16 : 8;
  const uint16_t* xl = xrow + kw + kLaneK * g;
#pragma unroll
  for (int b = 0; b < NLW; ++b) {
    const u32x4 r = S.raw[b];
    if constexpr (FP8) {
      const u32x4 x0 = *(const u32x4*)(xl + b * kLoadK);
      const u32x4 x1 = *(const u32x4*)(xl + b * kLoadK + 8);
      f32x4& t = part[pbase + b / 2];
      t = mfma_bf16(x0, fp8x8_to_bf16(r.x, r.y), t);
      t = mfma_bf16(x1, fp8x8_to_bf16(r.z, r.w), t);
      // interleave: two LDS reads, then their two MFMAs.  Left alone, the
      // scheduler issues all 2 * NLW activation reads up front (8 VGPRs each),
      // which costs k_stage_b_lean a wave per SIMD (114 -> 102 VGPRs).
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
    } else {
      const u32x4 x0 = *(const u32x4*)(xl + b * kLoadK);
      part[0] = mfma_bf16(x0, r, part[0]);
    }
  }
}

// Pairs of tokens [mb, mb + kLeanXT): block 0 of a routed expert from its
// record, later blocks from its list, the shared expert's from the token index.
__device__ __forceinline__ void lean_pairs(const LayerArgs& a, const ExpertRec* rec, const int32_t* list,
                                           int shared_col, int cnt, int mb, int (&pr)[kLeanXT]) {
#pragma unroll
  for (int i = 0; i < kLeanXT; ++i) {
    int p = -1;
    if (mb + i < cnt) p = list == nullptr ? (mb + i) * a.KP + shared_col : mb == 0 ? rec->p[i] : sload_i32(list, mb + i);
    pr[i] = p;
  }
}

// Stage A item: 8 channels (8 gate + 8 up rows) of one expert, the hidden K
// split over the 4 waves (KR = H / 4 each).  FP8: one window of KR / 64
// wave-loads, fp32 scale words sc_lo (gate rows' block) / sc_hi (up rows').
// BF16 (shared expert): NWIN windows of KR / (32 NWIN) wave-loads.
// The shared expert's tokens split into blocks of kLeanAShXT for stage A,
// one workgroup per (block, 8 channels), so its workgroups take no longer
// than a routed expert's.  Measured on MI355X (C3, stage A): T=64 92.4 ->
// 87.7 us against one workgroup per 8 channels taking every token (4: 88.4,
// 16: 88.9); no change up to T=32.
constexpr int kLeanAShXT = 8;
static_assert(kLeanRouteMaxT <= kLeanAShXT, "the routing stage A takes the shared expert as one block");
__host__ __device__ __forceinline__ int lean_a_sh_blocks(const ftm_moe_layer& L, int T) {
  return L.shared_inter > 0 ? (T + kLeanAShXT - 1) / kLeanAShXT : 0;
}

template <bool FP8, int KR, int NWIN>
__device__ void lean_a_item(const LayerArgs& a, const char* w, const float* sc, int Iu, int c0, int cnt,
                            const ExpertRec* rec, const int32_t* list, int shared_col, int kp, f32x4* red,
                            int mb0 = 0) {
  constexpr int NLW = (FP8 ? KR / 64 : KR / 32) / NWIN;
  constexpr int NP = FP8 ? NLW / 2 : 1;
  static_assert(!FP8 || NWIN == 1, "FP8 rows: one window per wave");
  const int lane = threadIdx.x & 63;
  const int n = lane & 15;
  const int H = a.L.hidden;
  const uint32_t row_bytes = (FP8 ? 1u : 2u) * (uint32_t)H;
  const Rsrc wres = make_rsrc(w, row_bytes * (uint32_t)(2 * Iu));
  const int lrow = n < 8 ? c0 + n : Iu + c0 + (n - 8);
  const int k0 = kp * KR;
  const uint32_t kbase = (FP8 ? 1u : 2u) * (uint32_t)k0;
  LeanWin<NLW> S;
  lean_issue<NLW>(wres, lrow, row_bytes, kbase, 0, S);
  // fp32 scale words of this wave's K blocks: gate rows' block, up rows' block
  float s_lo[NP], s_hi[NP];
  if constexpr (FP8) {
    const int nkb = H / 128;
    const uint32_t lo = (uint32_t)(((c0 / 128) * nkb + k0 / 128) * 4);
    const uint32_t hi = (uint32_t)((((Iu + c0) / 128) * nkb + k0 / 128) * 4);
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      s_lo[i] = __uint_as_float(sload4(sc, lo + 4u * (uint32_t)i));
      s_hi[i] = __uint_as_float(sload4(sc, hi + 4u * (uint32_t)i));
    }
  }
  constexpr int pitch = lean_pitch(KR);
  uint16_t* xw = ftm_xl_lds + kp * (kLeanXT + 1) * pitch;
  // zero row for MFMA rows without a token (this wave's region only)
  for (int e = 8 * lane; e < KR; e += 8 * 64) *(u32x4*)(xw + kLeanXT * pitch + e) = (u32x4){0u, 0u, 0u, 0u};
  for (int mb = mb0; mb < cnt; mb += kLeanXT) {
    const int nb = min(kLeanXT, cnt - mb);
    int pr[kLeanXT];
    lean_pairs(a, rec, list, shared_col, cnt, mb, pr);
    lean_fill<KR>(pr, nb, a.x, a.KP, H, k0, xw);
    const uint16_t* xrow = xw + ((n < nb) ? n : kLeanXT) * pitch;
    f32x4 part[NP];
#pragma unroll
    for (int i = 0; i < NP; ++i) part[i] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int wi = 0; wi < NWIN; ++wi) {
      if (wi > 0 || (NWIN > 1 && mb > mb0)) lean_issue<NLW>(wres, lrow, row_bytes, kbase, wi * NLW, S);
      __builtin_amdgcn_s_waitcnt(0);  // weights and this wave's LDS rows have landed
      lean_mfma<FP8, NLW, NP>(S, xrow, wi * NLW * (FP8 ? 64 : 32), part, 0);
    }
    f32x4 acc;
    if constexpr (FP8) {
      const bool upper = n >= 8;
      acc = part[0] * (upper ? s_hi[0] : s_lo[0]);
#pragma unroll
      for (int i = 1; i < NP; ++i) acc += part[i] * (upper ? s_hi[i] : s_lo[i]);
    } else {
      acc = part[0];
    }
    if (lane < 16) red[kp * 16 + lane] = acc;
    __syncthreads();
    if (kp == 0) {
      f32x4 t = red[n] + red[16 + n] + red[32 + n] + red[48 + n];
#pragma unroll
      for (int r = 0; r < kLeanXT; ++r) {
        const float gs = t[r];
        const float us = dpp_f<kDppRowShl8>(t[r]);
        if (lane < 8 && r < nb) {
          const float h = act_fn(a.L.act, gs, us, a.L.swiglu_alpha, a.L.swiglu_limit);
          ((uint16_t*)a.hbuf)[(size_t)pr[r] * a.Imax + c0 + n] = f32_to_bf16(h);
        }
      }
    }
    __syncthreads();
  }
}

template <int KR, int NWS>
__global__ __launch_bounds__(kBlock) void k_stage_a_lean(const LayerArgs a) {
  __shared__ f32x4 red[4 * 16];
  const int kp = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int I = a.L.inter;
  const int t8 = I / 8;
  // the shared expert's (token block, 8-channel) items first, so they start
  // early instead of trailing the grid
  const int ts = a.L.shared_inter / 8;
  const int nShared = ts * lean_a_sh_blocks(a.L, a.T);
  if ((int)blockIdx.x < nShared) {
    const int b = (int)blockIdx.x / ts, c = (int)blockIdx.x % ts;
    lean_a_item<false, KR, NWS>(a, (const char*)a.L.shared_w13, nullptr, a.L.shared_inter, c * 8,
                                min(a.T, (b + 1) * kLeanAShXT), nullptr, nullptr, a.L.topk, kp, red,
                                b * kLeanAShXT);
    return;
  }
  const int item = blockIdx.x - nShared;
  const ExpertRec rec = load_rec(a, min(item / t8, a.L.num_experts));
  const int nRouted = sload_i32(a.ctrl, kCtrlNRouted);
  if (item >= nRouted * t8) return;
  if (rec.slot < 0 || rec.slot >= a.L.w13.num_slots) {
    if (threadIdx.x == 0) atomicOr(&a.ctrl[kCtrlError], 1);
    return;
  }
  const char* w = (const char*)a.L.w13.w + (int64_t)rec.slot * a.L.w13.w_stride;
  const float* sc = (const float*)((const char*)a.L.w13.s + (int64_t)rec.slot * a.L.w13.s_stride);
  lean_a_item<true, KR, 1>(a, w, sc, I, (item % t8) * 8, rec.cnt, &rec, a.lists + (size_t)rec.e * a.T, 0, kp, red);
}

// ---- stage A that routes (T <= kLeanRouteMaxT): every workgroup routes the
// call's tokens itself (route_token, one wave per token) and takes the
// routed expert of rank u (ascending id) from an LDS expert mask; workgroup 0
// of the routed items publishes ids, weights, records and the routed count for
// stage B, the combine and the caller.  Replaces the top-k launch.

template <int KR, int NWS, int MODE>
__global__ __launch_bounds__(kBlock) void k_stage_a_lean_route(const LayerArgs a) {
  __shared__ f32x4 red[4 * 16];
  __shared__ int s_sel[kLeanRouteMaxT * kLeanRouteMaxK];
  __shared__ float s_w[kLeanRouteMaxT * kLeanRouteMaxK];
  __shared__ uint32_t s_mask[256 / 32];
  const int kp = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int I = a.L.inter, t8 = I / 8, T = a.T, k = a.L.topk, E = a.L.num_experts, KP = a.KP;
  const int nShared = a.L.shared_inter > 0 ? a.L.shared_inter / 8 : 0;
  if ((int)blockIdx.x < nShared) {  // shared-expert items need no routing
    lean_a_item<false, KR, NWS>(a, (const char*)a.L.shared_w13, nullptr, a.L.shared_inter, blockIdx.x * 8, T,
                                nullptr, nullptr, k, kp, red);
    return;
  }
  const int item = blockIdx.x - nShared;
  const bool lead = item == 0;
  if (threadIdx.x < 256 / 32) s_mask[threadIdx.x] = 0u;
  __syncthreads();
  if (kp < T) {
    int sel_e;
    float sel_w;
    route_token<MODE, 4>(a, kp, nullptr, 0, nullptr, nullptr, lead ? a.logits_out : nullptr, sel_e, sel_w);
    if (lane < k) {
      s_sel[kp * k + lane] = sel_e;
      s_w[kp * k + lane] = sel_w;
      atomicOr(&s_mask[sel_e >> 5], 1u << (sel_e & 31));
    }
  }
  __syncthreads();
  const int nw = (E + 31) / 32;
  int nRouted;
  mask_rank(s_mask, nw, 0, nRouted);
  nRouted = __builtin_amdgcn_readfirstlane(nRouted);
  if (lead) {
    for (int i = threadIdx.x; i < T * k; i += kBlock) {
      const int p = (i / k) * KP + i % k;
      a.wts[p] = s_w[i];
      a.ids[i] = s_sel[i];
      if (a.ids_out) a.ids_out[i] = s_sel[i];
      if (a.w_out) a.w_out[i] = s_w[i];
    }
    if (a.L.shared_inter > 0) {
      for (int t = threadIdx.x; t < T; t += kBlock) {
        const float sl = a.logits[(size_t)t * (E + 1) + E];
        a.wts[t * KP + k] = round_to(ftm_sigmoidf(sl), a.L.act_dtype);
      }
    }
    for (int u2 = threadIdx.x; u2 < nRouted; u2 += kBlock) {
      int tot;
      const ExpertRec r = route_rec(a, s_sel, mask_rank(s_mask, nw, u2, tot));
      int32_t* dst = a.recs + (size_t)u2 * kRecWords;
      dst[0] = r.e;
      dst[1] = r.cnt;
      dst[2] = r.slot;
#pragma unroll
      for (int q = 0; q < kRecPairs; ++q) dst[3 + q] = r.p[q];
      dst[kRecWords - 1] = 0;
    }
    if (threadIdx.x == 0) {
      a.ctrl[kCtrlNRouted] = nRouted;
      a.ctrl[kCtrlNU] = nRouted + (a.L.shared_inter > 0 ? 1 : 0);
    }
  }
  const int u = item / t8;
  if (u >= nRouted) return;
  int tot;
  const ExpertRec rec = route_rec_uniform(a, s_sel, mask_rank(s_mask, nw, u, tot));
  if (rec.slot < 0 || rec.slot >= a.L.w13.num_slots) {
    if (threadIdx.x == 0) atomicOr(&a.ctrl[kCtrlError], 1);
    return;
  }
  const char* w = (const char*)a.L.w13.w + (int64_t)rec.slot * a.L.w13.w_stride;
  const float* sc = (const float*)((const char*)a.L.w13.s + (int64_t)rec.slot * a.L.w13.s_stride);
  lean_a_item<true, KR, 1>(a, w, sc, I, (item % t8) * 8, rec.cnt, &rec, a.lists + (size_t)rec.e * T, 0, kp, red);
}

// Stage B item: 64 output columns of one expert, wave w owns 16 of them over
// the full K (= I routed / Is shared); y = acc * router weight -> slot buffer.
// col0: first of the wave's ncols (16 or 8) output columns; wv: the wave's LDS
// region; s_y: null -> slot buffer rows, else LDS s_y[pair * 16 + column];
// token blocks from mb0 (a multiple of kLeanXT) up to cnt.
template <bool FP8, int KB, int NWIN>
__device__ void lean_b_item(const LayerArgs& a, const char* w, const float* sc, int cnt, const ExpertRec* rec,
                            const int32_t* list, int shared_col, int col0, int wv, float* s_y = nullptr,
                            int ncols = 16, int mb0 = 0) {
  constexpr int NLW = (FP8 ? KB / 64 : KB / 32) / NWIN;
  constexpr int NP = FP8 ? NLW / 2 : 1;
  static_assert(!FP8 || NWIN == 1, "FP8 rows: one window per wave");
  const int lane = threadIdx.x & 63;
  const int n = lane & 15;
  const int H = a.L.hidden;
  const uint32_t row_bytes = (FP8 ? 1u : 2u) * (uint32_t)KB;
  const Rsrc wres = make_rsrc(w, row_bytes * (uint32_t)H);
  const int brow = col0 + n;
  const int wrow = n < ncols ? brow : -1;  // rows past ncols load nothing
  LeanWin<NLW> S;
  lean_issue<NLW>(wres, wrow, row_bytes, 0u, 0, S);
  float sv[NP];
  if constexpr (FP8) {
    const uint32_t off = (uint32_t)((col0 / 128) * (KB / 128) * 4);
#pragma unroll
    for (int i = 0; i < NP; ++i) sv[i] = __uint_as_float(sload4(sc, off + 4u * (uint32_t)i));
  }
  constexpr int pitch = lean_pitch(KB);
  uint16_t* xw = ftm_xl_lds + wv * (kLeanXT + 1) * pitch;
  for (int e = 8 * lane; e < KB; e += 8 * 64) *(u32x4*)(xw + kLeanXT * pitch + e) = (u32x4){0u, 0u, 0u, 0u};
  for (int mb = mb0; mb < cnt; mb += kLeanXT) {
    const int nb = min(kLeanXT, cnt - mb);
    int pr[kLeanXT];
    lean_pairs(a, rec, list, shared_col, cnt, mb, pr);
    lean_fill<KB>(pr, nb, a.hbuf, 1, a.Imax, 0, xw);
    float wr[kLeanXT];
#pragma unroll
    for (int r = 0; r < kLeanXT; ++r) wr[r] = r < nb ? __uint_as_float(sload4(a.wts, 4u * (uint32_t)pr[r])) : 0.0f;
    const uint16_t* xrow = xw + ((n < nb) ? n : kLeanXT) * pitch;
    f32x4 part[NP];
#pragma unroll
    for (int i = 0; i < NP; ++i) part[i] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int wi = 0; wi < NWIN; ++wi) {
      if (wi > 0 || (NWIN > 1 && mb > mb0)) lean_issue<NLW>(wres, wrow, row_bytes, 0u, wi * NLW, S);
      __builtin_amdgcn_s_waitcnt(0);  // weights and this wave's LDS rows have landed
      lean_mfma<FP8, NLW, NP>(S, xrow, wi * NLW * (FP8 ? 64 : 32), part, 0);
    }
    f32x4 acc;
    if constexpr (FP8) {
      acc = part[0] * sv[0];
#pragma unroll
      for (int i = 1; i < NP; ++i) acc += part[i] * sv[i];
    } else {
      acc = part[0];
    }
#pragma unroll
    for (int r = 0; r < kLeanXT; ++r)
      if (lane < ncols && r < nb) {
        if (s_y != nullptr)
          s_y[pr[r] * 16 + n] = acc[r] * wr[r];
        else
          a.ybuf[(size_t)pr[r] * H + brow] = acc[r] * wr[r];
      }
  }
}

// The shared expert's tokens split into blocks of kLeanBShXT, one workgroup
// per (block, column tile), so its workgroups take no longer than a routed
// expert's.  Measured on MI355X (C3, stage B): T=32 37.3 -> 33.7 us, T=48
// 50.3 -> 41.7, T=64 60.9 -> 48.6 against one workgroup per tile taking every
// token (blocks of 4: 34.5 at T=32; 16: as 8).
constexpr int kLeanBShXT = 8;
__host__ __device__ __forceinline__ int lean_b_sh_blocks(const ftm_moe_layer& L, int T) {
  return L.shared_inter > 0 ? (T + kLeanBShXT - 1) / kLeanBShXT : 0;
}

template <int KB, int NWS>
__global__ __launch_bounds__(kBlock) void k_stage_b_lean(const LayerArgs a) {
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int H = a.L.hidden;
  const int tiles = H / 64;
  // the shared expert's (token block, column tile) units first
  const int hasSh = lean_b_sh_blocks(a.L, a.T);
  const int u0 = (int)blockIdx.x / tiles, nt = (int)blockIdx.x % tiles;
  if (u0 < hasSh) {
    lean_b_item<false, KB, NWS>(a, (const char*)a.L.shared_w2, nullptr, min(a.T, (u0 + 1) * kLeanBShXT), nullptr,
                                nullptr, a.L.topk, nt * 64 + 16 * wv, wv, nullptr, 16, u0 * kLeanBShXT);
    return;
  }
  const int u = u0 - hasSh;
  const ExpertRec rec = load_rec(a, min(u, a.L.num_experts));
  const int nRouted = sload_i32(a.ctrl, kCtrlNRouted);
  if (u >= nRouted) return;
  const int32_t* list = a.lists + (size_t)rec.e * a.T;
  if (rec.slot < 0 || rec.slot >= a.L.w2.num_slots) {
    // non-resident expert: contribute zeros, flag the error
    for (int idx = threadIdx.x; idx < rec.cnt * 64; idx += kBlock) {
      const int m = idx / 64, c = nt * 64 + idx % 64;
      a.ybuf[(size_t)list[m] * H + c] = 0.0f;
    }
    if (threadIdx.x == 0) atomicOr(&a.ctrl[kCtrlError], 1);
    return;
  }
  const char* w = (const char*)a.L.w2.w + (int64_t)rec.slot * a.L.w2.w_stride;
  const float* sc = (const float*)((const char*)a.L.w2.s + (int64_t)rec.slot * a.L.w2.s_stride);
  lean_b_item<true, KB, 1>(a, w, sc, rec.cnt, &rec, list, 0, nt * 64 + 16 * wv, wv);
}

// ---- stage B and the combine in one launch for T <= kBcMaxT (lean kernels):
// one workgroup of kBcWaves waves per kBcCols output columns.  Its units are
// the shared expert's blocks of kLeanXT tokens (first: each takes every token
// of its block, and as one unit they made the longest wave) and then the
// routed experts; wave w takes units w, w + kBcWaves, ...  Their
// router-weighted rows land in LDS by pair, and the workgroup sums each
// token's slots in slot order (k_combine's order and rounding) into the
// output.  Saves the combine launch and the slot buffer's round trip.
// Measured on MI355X (C3), stage B + combine with the shared expert as one
// unit against split by token block: T=8 17.2 -> 15.8 us, T=16 25.5 -> 24.0.
// Neither a software pipeline over a wave's experts (8 waves, 198 VGPRs: the
// compiler's vmcnt tracking across the loop still serialises the loads; 18.3
// and 28.9 us) nor 16 waves (128 VGPRs; 18.6 and 28.1 us) was faster, nor two
// routed experts per wave in the 16 MFMA rows (8 weight rows each, twice the
// bytes in flight for the same registers): a pair took 3.8 us where one unit
// takes 2.0 (s_memrealtime per unit, T=16), so the CU's memory pipeline, not
// a wave's latency, bounds the loop (stage B + combine T=16 23.3 -> 24.3 us).
constexpr int kBcWaves = 12;  // 768 threads: 170 VGPRs per lane (16 waves spill at 128)
constexpr int kBcCols = 8;    // output columns per workgroup: H / 8 workgroups fill the CUs
// Measured on MI355X (C3), stage B + combine: T=5 12.7 us against 12.2 + 4.8,
// T=8 17.1 against 15.3 + 4.6, T=16 26.0 against 22.5 + 5.3.
constexpr int kBcMaxT = 16;
constexpr int kBcMaxKP = 65;  // top-k <= 64, + the shared expert

template <int KB, int NWS>
__global__ __launch_bounds__(64 * kBcWaves) void k_stage_bc_lean(const LayerArgs a) {
  __shared__ float s_y[kBcMaxT * kBcMaxKP * 16];
  __shared__ int s_next;  // the next unit a wave takes
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int H = a.L.hidden, T = a.T, KP = a.KP;
  const int col0 = blockIdx.x * kBcCols;
  const int nSh = a.L.shared_inter > 0 ? (T + kLeanXT - 1) / kLeanXT : 0;
  // Each routed unit's record is loaded one unit ahead, one word a lane
  // (lanes 0..kRecWords-1, a vector load the current unit's full wait
  // covers), so a unit's weight loads issue without waiting for its record
  // (a scalar prefetch was waited for at the loop head: its registers are
  // recycled); the first one is requested beside the routed count (any of
  // the E + 1 records: the loop reads it only for a routed unit).  C3 stage
  // B + combine, us: T=16 23.5 -> 22.9, T=8 14.5 -> 13.9, T=1 5.5 -> 5.4.
  const int rl = threadIdx.x & 63;
  const Rsrc rall = make_rsrc(a.recs, (uint32_t)(a.L.num_experts + 1) * (uint32_t)(4 * kRecWords));
  uint32_t nrec = bload4(rall, wv >= nSh && rl < kRecWords ? (uint32_t)((wv - nSh) * kRecWords + rl) * 4u : kOOB);
  const int nRouted = sload_i32(a.ctrl, kCtrlNRouted);
  // slots of pairs without an expert stay zero (as their slot-buffer rows would be)
  for (int i = threadIdx.x; i < T * KP * 16; i += 64 * kBcWaves) s_y[i] = 0.0f;
  if (threadIdx.x == 0) s_next = kBcWaves;
  __syncthreads();
  const int nU = nSh + nRouted;
  const Rsrc rres = make_rsrc(a.recs, (uint32_t)nRouted * (uint32_t)(4 * kRecWords));
  auto rec_load = [&](int uu) {
    const int u = uu - nSh;
    return bload4(rres, uu < nU && u >= 0 && rl < kRecWords ? (uint32_t)(u * kRecWords + rl) * 4u : kOOB);
  };
  // units handed out on demand: wave w starts with unit w, then takes the next
  // free one (an LDS counter), so waves whose units ran short take more (C3
  // stage B + combine, us: T=16 23.0 -> 22.7, T=8 14.1 -> 13.8, T=4 9.4 -> 9.3)
  int nx = 0;
  for (int uu = wv; uu < nU; uu = nx) {
    ExpertRec rec;
    rec.e = __builtin_amdgcn_readlane((int)nrec, 0);
    rec.cnt = __builtin_amdgcn_readlane((int)nrec, 1);
    rec.slot = __builtin_amdgcn_readlane((int)nrec, 2);
#pragma unroll
    for (int i = 0; i < kRecPairs; ++i) rec.p[i] = __builtin_amdgcn_readlane((int)nrec, 3 + i);
    int t = 0;
    if (rl == 0) t = atomicAdd(&s_next, 1);
    nx = __builtin_amdgcn_readfirstlane(t);
    nrec = rec_load(nx);
    if (uu >= nSh) {
      if (rec.slot < 0 || rec.slot >= a.L.w2.num_slots) {  // non-resident: contributes zeros
        if ((threadIdx.x & 63) == 0) atomicOr(&a.ctrl[kCtrlError], 1);
        continue;
      }
      const char* w = (const char*)a.L.w2.w + (int64_t)rec.slot * a.L.w2.w_stride;
      const float* sc = (const float*)((const char*)a.L.w2.s + (int64_t)rec.slot * a.L.w2.s_stride);
      lean_b_item<true, KB, 1>(a, w, sc, rec.cnt, &rec, a.lists + (size_t)rec.e * T, 0, col0, wv, s_y, kBcCols);
    } else {
      lean_b_item<false, KB, NWS>(a, (const char*)a.L.shared_w2, nullptr, min(T, (uu + 1) * kLeanXT), nullptr,
                                  nullptr, a.L.topk, col0, wv, s_y, kBcCols, uu * kLeanXT);
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < T * kBcCols; i += 64 * kBcWaves) {
    const int t = i / kBcCols, c = i % kBcCols;
    float sum = s_y[(t * KP) * 16 + c];
    for (int j = 1; j < KP; ++j) sum += s_y[(t * KP + j) * 16 + c];
    ((uint16_t*)a.out)[(size_t)t * H + col0 + c] = f32_to_bf16(sum);
  }
}

// ============================================================== combine
// out[t, n] = sum_j ybuf[t*KP + j, n] in slot order (deterministic, no atomics).
template <int AT>
__global__ __launch_bounds__(kBlock) void k_combine(const LayerArgs a) {
  const int H = a.L.hidden, KP = a.KP;
  const int H4 = H / 4;
  const int idx = blockIdx.x * kBlock + threadIdx.x;
  if (idx >= a.T * H4) return;
  const int t = idx / H4, n4 = idx % H4;
  const f32x4* yb = (const f32x4*)(a.ybuf + (size_t)t * KP * H) + n4;
  // slots in order (a pair without an expert has a zeroed slot); the loads
  // of 8 slots issue together before their adds, which keep slot order
  f32x4 s = yb[0];
  int j = 1;
  for (; j + 8 <= KP; j += 8) {
    f32x4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = yb[(size_t)(j + u) * H4];
#pragma unroll
    for (int u = 0; u < 8; ++u) s += v[u];
  }
  for (; j < KP; ++j) s += yb[(size_t)j * H4];
  if constexpr (AT == FTM_DT_F32) {
    ((f32x4*)a.out)[(size_t)t * H4 + n4] = s;
  } else {
    u32x2 o;
    o.x = pack_bf16x2(s.x, s.y);
    o.y = pack_bf16x2(s.z, s.w);
    ((u32x2*)a.out)[(size_t)t * H4 + n4] = o;
  }
}

// ============================================================== single projection
struct LinArgs {
  ftm_proj P;
  int slot;
  const void* x;
  int M;
  void* out;
  int out_dt;
  const void* bias;
  int bias_dt, final_dt;
};

template <int FMT, int AT>
__global__ __launch_bounds__(kBlock) void k_linear(const LinArgs a) {
  constexpr bool kG = FMT == FTM_FMT_GPTQ_INT4;
  constexpr int XB = AType<AT>::kBytes;
  __shared__ f32x4 red[4 * 4 * 64];
  const ProjSlot W = proj_slot(a.P, a.slot);
  const int N = W.N, K = W.K;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int nt = blockIdx.x, mt = blockIdx.y;
  int lo, hi;
  if (kG) {
    wave_k_range<FMT>(W, wave, 4, lo, hi);
  } else {
    lo = 0;
    hi = fmt_loads<FMT>(K);
  }
  const int col0[1] = {kG ? nt * 64 : nt * 64 + 16 * wave};
  const Rsrc xres = make_rsrc(a.x, (uint32_t)a.M * (uint32_t)K * XB);
  const int m = mt * 16 + (lane & 15);
  const uint32_t arow = (m < a.M) ? (uint32_t)m * (uint32_t)K * XB : kOOB;
  auto emit = [&](int m2, int n, float y) {
    if (m2 < a.M && n < N) {
      float v = round_to(y, a.out_dt);
      if (a.bias != nullptr) v = round_to(v + load_scalar(a.bias, n, a.bias_dt), a.final_dt);
      store_scalar(a.out, (size_t)m2 * N + n, a.final_dt, v);
    }
  };
  if constexpr (kG) {
    f32x4 acc[1][4];
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[0][c] = (f32x4){0.f, 0.f, 0.f, 0.f};
    wave_gemm_gptq<1, AT>(W, col0, lo, hi, xres, arow, acc);
#pragma unroll
    for (int c = 0; c < 4; ++c) red[(wave * 4 + c) * 64 + lane] = acc[0][c];
    __syncthreads();
    for (int idx = threadIdx.x; idx < 16 * 64; idx += kBlock) {
      const int i = idx / 64, j = idx % 64;
      const int c = j & 3, ln = (j >> 2) + 16 * (i >> 2), rr = i & 3;
      float y = 0.0f;
#pragma unroll
      for (int w = 0; w < 4; ++w) y += red[(w * 4 + c) * 64 + ln][rr];
      emit(mt * 16 + i, nt * 64 + j, y);
    }
  } else {
    f32x4 acc[1] = {(f32x4){0.f, 0.f, 0.f, 0.f}};
    wave_gemm_kmajor<FMT, 1, AT>(W, col0, lo, hi, xres, arow, acc);
    const int n = col0[0] + (lane & 15);
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) emit(mt * 16 + 4 * (lane >> 4) + rr, n, acc[0][rr]);
  }
}

// ============================================================== small helpers
__global__ void k_fill_routing(int T, int32_t slot, int32_t* slot_word, int32_t* ids, float* w) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t == 0) *slot_word = slot;
  if (t < T) {
    ids[t] = 0;
    w[t] = 1.0f;
  }
}

__global__ void k_zero_words(int32_t* p, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0;
}

// ============================================================== launchers
hipError_t launch_ws_init(void* ws, hipStream_t st) {
  hipLaunchKernelGGL(k_zero_words, dim3(4), dim3(kBlock), 0, st, (int32_t*)ws, FTM_WS_CTRL_BYTES / 4);
  return hipGetLastError();
}

hipError_t launch_router(const ftm_moe_layer& L, const void* x, int T, int row_begin, int row_end, char* ws,
                         const WsLayout& wl, hipStream_t st, bool quant) {
  const LayerArgs a = make_args(L, x, nullptr, T, ws, wl);
  if (row_end - row_begin <= 0 || T <= 0) return hipSuccess;
  const bool one = (row_end - row_begin) * ((T + 3) / 4) <= kRouterOneMaxWgs;  // k_router<1>: 4 tokens per workgroup
  const int tpb = one ? 4 : 4 * kRouterTPW;
  const int ty = (T + tpb - 1) / tpb;
  // quantisation blocks spread over the grid's token-block rows (ceil(nq / ty) columns)
  const int nq = quant && mx_input(L, T) ? (quant_mx_threads(T, L.hidden) + kBlock - 1) / kBlock : 0;
  const int qx = (nq + ty - 1) / ty;
  if (router_by_rows(row_end - row_begin, T, L.hidden))
    hipLaunchKernelGGL(k_router_rows, dim3((row_end - row_begin + kRouterRB - 1) / kRouterRB + qx, ty),
                       dim3(kBlock), 0, st, a, row_begin, row_end);
  else if (one)
    hipLaunchKernelGGL(k_router<1>, dim3(row_end - row_begin + qx, ty), dim3(kBlock), 0, st, a, row_begin,
                       row_end - row_begin);
  else
    hipLaunchKernelGGL(k_router<kRouterTPW>, dim3(row_end - row_begin + qx, ty), dim3(kBlock), 0, st, a, row_begin,
                       row_end - row_begin);
  return hipGetLastError();
}

bool route_topk_fused(const ftm_moe_layer& L, int T) {
  return T >= 1 && T <= kTopk1MaxT && L.gate_w != nullptr && L.act_dtype == FTM_DT_BF16 && L.hidden % 8 == 0 &&
         !route_a_ok(L, T);
}

hipError_t launch_route_topk(const ftm_moe_layer& L, const void* x, int T, int32_t* ids_out, float* w_out,
                             float* logits_out, char* ws, const WsLayout& wl, hipStream_t st, bool quant) {
  const LayerArgs a = make_args(L, x, nullptr, T, ws, wl);
  const int rows = L.num_experts + (L.shared_inter > 0 ? 1 : 0);
  const int nq = quant && mx_input(L, T) ? (quant_mx_threads(T, L.hidden) + 64 * kTopk1Waves - 1) / (64 * kTopk1Waves) : 0;
  const int rpw = route_rpw(rows), wpr = kTopk1Waves / rpw, nt = (T + wpr - 1) / wpr;
  const dim3 grid((rows + rpw - 1) / rpw + nq), block(64 * kTopk1Waves);
#define FTM_RT_NT(M, NV)                                                                                       \
  if (nt <= 1)                                                                                                 \
    hipLaunchKernelGGL((k_route_topk1<M, NV, 1>), grid, block, 0, st, a, rows, ids_out, w_out, logits_out);   \
  else if (nt <= 2)                                                                                            \
    hipLaunchKernelGGL((k_route_topk1<M, NV, 2>), grid, block, 0, st, a, rows, ids_out, w_out, logits_out);   \
  else                                                                                                         \
    hipLaunchKernelGGL((k_route_topk1<M, NV, 4>), grid, block, 0, st, a, rows, ids_out, w_out, logits_out);
#define FTM_RT_NV(M)      \
  if (L.num_experts <= 256) { \
    FTM_RT_NT(M, 4)       \
  } else {                \
    FTM_RT_NT(M, 8)       \
  }
  switch (L.route_mode) {
    case FTM_ROUTE_SOFTMAX_TOPK: FTM_RT_NV(FTM_ROUTE_SOFTMAX_TOPK) break;
    case FTM_ROUTE_SOFTMAX_TOPK_LOWP: FTM_RT_NV(FTM_ROUTE_SOFTMAX_TOPK_LOWP) break;
    default: FTM_RT_NV(FTM_ROUTE_TOPK_SOFTMAX) break;
  }
#undef FTM_RT_NV
#undef FTM_RT_NT
  return hipGetLastError();
}

hipError_t launch_topk(const ftm_moe_layer& L, int T, const void* logits_in, int logits_dt,
                       const int32_t* ids_in, const float* w_in, int32_t* ids_out, float* w_out,
                       float* logits_out, char* ws, const WsLayout& wl, hipStream_t st) {
  const LayerArgs a = make_args(L, nullptr, nullptr, T, ws, wl);
  const bool one = T <= kTopk1MaxT, blk = T >= kTopkBlkMinT;
  const dim3 grid(one ? 1 : (T + 3) / 4), block(one ? 64 * kTopk1Waves : kBlock);
  const dim3 gblk(topk_blk_grid(T, L.topk)), bblk(64 * kTopkBlkWaves);
#define FTM_TOPK_LAUNCH(M, NV)                                                                                 \
  if (one)                                                                                                     \
    hipLaunchKernelGGL((k_topk1<M, NV>), grid, block, 0, st, a, logits_in, logits_dt, ids_in, w_in, ids_out,    \
                       w_out, logits_out);                                                                     \
  else if (blk)                                                                                                \
    hipLaunchKernelGGL((k_topk_blk<M, NV>), gblk, bblk, 0, st, a, logits_in, logits_dt, ids_in, w_in,           \
                       ids_out, w_out, logits_out);                                                            \
  else                                                                                                         \
    hipLaunchKernelGGL((k_topk<M, NV>), grid, block, 0, st, a, logits_in, logits_dt, ids_in, w_in, ids_out,     \
                       w_out, logits_out);
#define FTM_TOPK_NV(M)            \
  if (L.num_experts <= 256) {     \
    FTM_TOPK_LAUNCH(M, 4)         \
  } else {                        \
    FTM_TOPK_LAUNCH(M, 8)         \
  }
  switch (L.route_mode) {
    case FTM_ROUTE_SOFTMAX_TOPK: FTM_TOPK_NV(FTM_ROUTE_SOFTMAX_TOPK) break;
    case FTM_ROUTE_SOFTMAX_TOPK_LOWP: FTM_TOPK_NV(FTM_ROUTE_SOFTMAX_TOPK_LOWP) break;
    default: FTM_TOPK_NV(FTM_ROUTE_TOPK_SOFTMAX) break;
  }
#undef FTM_TOPK_NV
#undef FTM_TOPK_LAUNCH
  return hipGetLastError();
}

// Does one prefetch window hold a wave's share of K when K is split over
// `split` waves?  (A wave's range is at most ceil(loads / split) wave-loads.)
template <int FMT>
static bool pf_window_fits(int K, int split) {
  if constexpr (FMT == FTM_FMT_GPTQ_INT4) {
    return false;
  } else {
    const int kload = FMT == FTM_FMT_MXFP4 ? 128 : FMT == FTM_FMT_BF16 ? 32 : 64;
    const int loads = (K + kload - 1) / kload;
    return (loads + split - 1) / split <= kRowsNLW;
  }
}

// Launch plan of the LDS-activation decode stages: eligible (bf16
// activations, K-major format, a wave's K range in one prefetch window, its
// quantisation groups aligned as rows_consume_lds needs), row tiles per
// workgroup and wave-loads per scale group.
struct XlPlan {
  bool ok;
  int nt, lpg;
};


template <int FMT>
static int kload_of() {
  return FMT == FTM_FMT_MXFP4 ? 128 : FMT == FTM_FMT_BF16 ? 32 : 64;
}

// Group layout for one projection whose K is split over `split` waves: 2 =
// two wave-loads per group with every wave range starting on a group
// boundary; kRowsNLW = every wave range inside one group (or no post-scale);
// 0 = neither.
template <int FMT>
static int xl_lpg(const ftm_proj& P, int split) {
  if (FMT != FTM_FMT_FP8_BLOCK && FMT != FTM_FMT_INT8_PACKED) return kRowsNLW;
  const int kload = kload_of<FMT>();
  const int nL = (P.K + kload - 1) / kload;
  if (P.group <= 0 || (P.group % kload != 0 && P.group < P.K)) return 0;
  const int lpg = P.group >= P.K ? nL : P.group / kload;
  bool two = lpg == 2, one = true;
  for (int w = 0; w < split; ++w) {
    const int lo = w * nL / split, hi = (w + 1) * nL / split;
    if (lo % 2 != 0) two = false;
    if (hi > lo && lo / lpg != (hi - 1) / lpg) one = false;
  }
  return two ? 2 : one ? kRowsNLW : 0;
}

// Compute units of the current device (cached per device).
static int device_cus() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cus[dev] == 0) {
    int v = 0;
    cus[dev] = hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0 ? v : 256;
  }
  return cus[dev];
}

template <int FMT, int AT>
static XlPlan xl_plan_a(const ftm_moe_layer& L, int T) {
  XlPlan p{false, 1, kRowsNLW};
  if constexpr (FMT == FTM_FMT_GPTQ_INT4 || AT != FTM_DT_BF16) {
    return p;
  } else {
    if (T > (FMT == FTM_FMT_MXFP4 ? kXlMaxTMx : kXlMaxT)) return p;
    // routed rows: one window per wave (the bf16 shared rows may take several)
    if (!pf_window_fits<FMT>(L.hidden, 4)) return p;
    if (L.hidden % 8 != 0) return p;
    if (4 * kXR * xl_pitch(L.hidden, 4) * 2 > kDynLdsMax) return p;
    if (FMT == FTM_FMT_MXFP4 && 4 * kXT * mx_pitch((L.hidden + 127) / 128, 4) > kDynLdsMax) return p;
    p.lpg = xl_lpg<FMT>(L.w13, 4);
    if (p.lpg == 0) return p;
    // MXFP4 without a shared expert: 16-channel items (5 workgroups per CU at
    // 8 channels, 3 at 16: kXlWaves) where the 8-channel grid would need a
    // second round of workgroups and the 16-channel one fits one.  Measured on
    // MI355X (C4, w13 us): T = 1 (1,440 / 720 workgroups) 13.5 -> 11.9; T = 2
    // (two rounds either way) 15.8 -> 20.9.
    p.nt = 1;
    if (FMT == FTM_FMT_MXFP4 && L.shared_inter == 0 && L.inter % 16 == 0) {
      const int maxU = L.num_experts < T * L.topk ? L.num_experts : T * L.topk;
      const int items = maxU * (L.inter / 8), cus = device_cus();
      if (items > 5 * cus && items / 2 <= 3 * cus) p.nt = 2;
    }
    p.ok = true;
    return p;
  }
}

// Token-resident stages (k_stage_tok_a / _b) for both projections: MXFP4 layers with
// bf16 activations and no shared expert, below the GEMM crossover, from
// kTokMinAvg tokens per routed expert on average (up to kRecMaxT tokens: the
// kernels read the work records).  Measured on MI355X (C4, us per layer,
// against k_stage_a_xl + k_stage_b_ks): 2 tokens per expert (T=16) 113.4
// against 96.9, 3 (T=24) 113.7 / 109.9, 4 (T=32) 116.9 / 123.2, 5 (T=40)
// 117.8 / 133.4.
constexpr int kTokMinAvg = 4;
static bool tok_ok(const ftm_moe_layer& L, int T) {
  if (L.w13.fmt != FTM_FMT_MXFP4 || L.w2.fmt != FTM_FMT_MXFP4 || L.act_dtype != FTM_DT_BF16) return false;
  if (L.shared_inter > 0 || L.hidden % 8 != 0 || L.inter % 8 != 0 || T > kRecMaxT || gemm_path_ok(L, T)) return false;
  const long pairs = (long)T * L.topk;
  const long maxU = L.num_experts < pairs ? L.num_experts : pairs;
  if (pairs < (long)kTokMinAvg * maxU) return false;
  return tok_rows(L.hidden, 128) >= 16 && tok_rows(L.inter, 128) >= 16;
}

template <int FMT, bool STB>
static void launch_tok(const LayerArgs& a, int maxU, hipStream_t st) {
  constexpr int kload = FMT == FTM_FMT_MXFP4 ? 128 : FMT == FTM_FMT_BF16 ? 32 : 64;
  const int K = STB ? a.L.inter : a.L.hidden;
  const size_t lds = (size_t)tok_rows(K, kload) * 2u * (size_t)tok_pitch(K, kload);
  static bool attr = false;
  if (!attr) {
    const void* fn = STB ? reinterpret_cast<const void*>(&k_stage_tok_b<FMT>)
                         : reinterpret_cast<const void*>(&k_stage_tok_a<FMT>);
    (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, kTokLdsMax);
    attr = true;
  }
  const int cols = STB ? 16 * kTokWaves : 8 * kTokWaves;
  const int nct = ((STB ? a.L.hidden : a.L.inter) + cols - 1) / cols;
  // column tiles per workgroup: about one workgroup per CU (one fits a CU's LDS)
  int ni = (maxU * nct + device_cus() - 1) / device_cus();
  ni = ni < kTokMaxTiles ? ni : kTokMaxTiles;
  const int ngrp = (nct + ni - 1) / ni;
  if constexpr (STB)
    hipLaunchKernelGGL((k_stage_tok_b<FMT>), dim3(maxU * ngrp), dim3(kTokThreads), lds, st, a, ni);
  else
    hipLaunchKernelGGL((k_stage_tok_a<FMT>), dim3(maxU * ngrp), dim3(kTokThreads), lds, st, a, ni);
}

bool mx_stage_a(const ftm_moe_layer& L, int T) {
  return L.w13.fmt == FTM_FMT_MXFP4 && L.act_dtype == FTM_DT_BF16 && !gemm_path_ok(L, T) && !tok_ok(L, T) &&
         xl_plan_a<FTM_FMT_MXFP4, FTM_DT_BF16>(L, T).ok;
}

bool mx_input(const ftm_moe_layer& L, int T) {
  return mx_stage_a(L, T) || (gemm_path_ok(L, T) && mx_gemm_ok(L));
}

void launch_quant_mx(const void* x, int T, int H, uint8_t* xq, hipStream_t st) {
  hipLaunchKernelGGL(k_quant_mx, dim3((quant_mx_threads(T, H) + kBlock - 1) / kBlock), dim3(kBlock), 0, st,
                     (const uint16_t*)x, T, H, xq);
}

template <int FMT, int AT>
static XlPlan xl_plan_b(const ftm_moe_layer& L, int T) {
  XlPlan p{false, 1, kRowsNLW};
  if constexpr (FMT == FTM_FMT_GPTQ_INT4 || AT != FTM_DT_BF16) {
    return p;
  } else {
    if (T > kXlMaxT) return p;
    if (!pf_window_fits<FMT>(L.inter, 1)) return p;
    if (L.inter % 8 != 0 || (L.shared_inter > 0 && L.shared_inter % 8 != 0)) return p;
    // the LDS regions are sized for the wider of the routed and shared rows
    const int imax = L.inter > L.shared_inter ? L.inter : L.shared_inter;
    if (4 * kXR * xl_pitch(imax, 1) * 2 > kDynLdsMax) return p;
    p.lpg = xl_lpg<FMT>(L.w2, 1);
    if (p.lpg == 0) return p;
    p.nt = 1;
    p.ok = true;
    return p;
  }
}

// Stage B with K split over the waves (k_stage_b_ks): small batches whose w2
// rows do not fit one window per wave (the full-K xl kernel's condition).
// Measured on MI355X (C4 w2, against the register-fed k_stage_b): T=1 13.9 ->
// 9.7 us, T=4 29.5 -> 20.9, T=8 38.0 -> 28.6, T=16 48.3 -> 38.3, T=24 56.2 ->
// 46.3, T=32 60.3 -> 52.2.
constexpr int kBksMaxT = 32;
constexpr int kBksMaxTMx = kXlMaxTMx;  // MXFP4: beside the scaled-MFMA stage A
template <int FMT, int AT>
static XlPlan ks_plan_b(const ftm_moe_layer& L, int T) {
  XlPlan p{false, 1, kRowsNLW};
  if constexpr (FMT == FTM_FMT_GPTQ_INT4 || AT != FTM_DT_BF16) {
    return p;
  } else {
    if (T > (FMT == FTM_FMT_MXFP4 ? kBksMaxTMx : kBksMaxT) || T > kRecMaxT || L.hidden % 16 != 0) return p;
    if (!pf_window_fits<FMT>(L.inter, 4) || L.inter % 8 != 0) return p;
    if (L.shared_inter > 0 && (!pf_window_fits<FTM_FMT_BF16>(L.shared_inter, 4) || L.shared_inter % 8 != 0))
      return p;
    const int imax = L.inter > L.shared_inter ? L.inter : L.shared_inter;
    if (4 * kXR * xl_pitch(imax, 4) * 2 > kDynLdsMax) return p;
    p.lpg = xl_lpg<FMT>(L.w2, 4);
    p.ok = p.lpg != 0;
    return p;
  }
}

// K-split stage B and the combine as one launch (k_stage_bc_ks): bf16
// activations, stage B on k_stage_b_ks, no shared expert, up to kBcKsMaxT
// tokens (one token block: kXT), at most kBcKsMaxU routed experts (min(E, T
// k)) and kBcKsMaxKP slots a token, the 16 wave regions within the CU's LDS.
constexpr int kBcKsMaxT = kXT;
constexpr size_t kBcKsLdsMax = 160u * 1024u - 40u * 1024u;  // the CU's LDS less the kernel's static arrays
template <int FMT>
static size_t bcks_lds(const ftm_moe_layer& L) {
  return (size_t)kBcKsWaves * (kKsNoz<FMT> ? kXT : kXR) * (size_t)xl_pitch(L.inter, 4) * 2u;
}
template <int FMT>
static bool bcks_ok(const ftm_moe_layer& L, int T) {
  if constexpr (FMT == FTM_FMT_GPTQ_INT4) {
    return false;
  } else {
    if (L.act_dtype != FTM_DT_BF16 || L.shared_inter > 0 || T < 1 || T > kBcKsMaxT) return false;
    const int maxU = L.num_experts < T * L.topk ? L.num_experts : T * L.topk;
    if (maxU > kBcKsMaxU || L.topk > kBcKsMaxKP || bcks_lds<FMT>(L) > kBcKsLdsMax) return false;
    if (FMT == FTM_FMT_FP8_BLOCK && lean_ok(L, T)) return false;
    if constexpr (FMT == FTM_FMT_MXFP4) {
      if (tok_ok(L, T)) return false;
    }
    if (!ks_plan_b<FMT, FTM_DT_BF16>(L, T).ok) return false;
    // Where a w2 row fits one wave's window (k_stage_b_xl, H / 64 workgroups
    // per expert) only up to 2 routed experts: measured on MI355X (C1, H =
    // 1024, us per layer) T=1 (2 experts) 18.3 -> 17.4, T=2 (4) 18.5 -> 19.4,
    // T=4 (8) 19.9 -> 23.0.
    return maxU <= 2 || !xl_plan_b<FMT, FTM_DT_BF16>(L, T).ok;
  }
}
static bool bcks_fused(const ftm_moe_layer& L, int T) {
  if (gemm_path_ok(L, T)) return false;
  switch (L.w13.fmt) {
    case FTM_FMT_BF16: return bcks_ok<FTM_FMT_BF16>(L, T);
    case FTM_FMT_FP8_BLOCK: return bcks_ok<FTM_FMT_FP8_BLOCK>(L, T);
    case FTM_FMT_INT8_PACKED: return bcks_ok<FTM_FMT_INT8_PACKED>(L, T);
    case FTM_FMT_MXFP4: return bcks_ok<FTM_FMT_MXFP4>(L, T);
    default: return false;
  }
}
template <int FMT, int LPG, int NLW>
static void launch_bcks(const LayerArgs& a, hipStream_t st) {
  static bool attr = false;
  if (!attr) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&k_stage_bc_ks<FMT, LPG, NLW>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)kBcKsLdsMax);
    attr = true;
  }
  hipLaunchKernelGGL((k_stage_bc_ks<FMT, LPG, NLW>), dim3(a.L.hidden / 16), dim3(64 * kBcKsWaves), bcks_lds<FMT>(a.L),
                     st, a);
}

// which: bit 0 = stage A (w13 + act), bit 1 = stage B (w2), bit 2 = combine
template <int FMT, int AT>
static void launch_stages(const LayerArgs& a, int gridA, int gridB, hipStream_t st, int which, bool xq_ready) {
  const bool lean = FMT == FTM_FMT_FP8_BLOCK && AT == FTM_DT_BF16 && a.lean;
  if (lean) {
    const int maxU = a.L.num_experts < a.T * a.L.topk ? a.L.num_experts : a.T * a.L.topk;
    const size_t lds = 4u * (kLeanXT + 1) * (size_t)lean_pitch(512) * 2u;
    if (which & 1) {
      const int items = maxU * (a.L.inter / 8) + (a.L.shared_inter / 8) * lean_a_sh_blocks(a.L, a.T);
      if (a.route_a) {
        if (a.L.route_mode == FTM_ROUTE_SOFTMAX_TOPK)
          hipLaunchKernelGGL((k_stage_a_lean_route<512, 2, FTM_ROUTE_SOFTMAX_TOPK>), dim3(items), dim3(kBlock), lds, st, a);
        else if (a.L.route_mode == FTM_ROUTE_SOFTMAX_TOPK_LOWP)
          hipLaunchKernelGGL((k_stage_a_lean_route<512, 2, FTM_ROUTE_SOFTMAX_TOPK_LOWP>), dim3(items), dim3(kBlock), lds,
                             st, a);
        else
          hipLaunchKernelGGL((k_stage_a_lean_route<512, 2, FTM_ROUTE_TOPK_SOFTMAX>), dim3(items), dim3(kBlock), lds, st,
                             a);
      } else {
        hipLaunchKernelGGL((k_stage_a_lean<512, 2>), dim3(items), dim3(kBlock), lds, st, a);
      }
    }
    const bool bc = a.T <= kBcMaxT && a.KP <= kBcMaxKP;  // stage B and the combine in one launch
    if (which & 2) {
      if (bc) {
        const size_t ldsb = (size_t)kBcWaves * (kLeanXT + 1) * (size_t)lean_pitch(512) * 2u;
        hipLaunchKernelGGL((k_stage_bc_lean<512, 2>), dim3(a.L.hidden / kBcCols), dim3(64 * kBcWaves), ldsb, st, a);
      } else {
        const int grid = (maxU + lean_b_sh_blocks(a.L, a.T)) * (a.L.hidden / 64);
        hipLaunchKernelGGL((k_stage_b_lean<512, 2>), dim3(grid), dim3(kBlock), lds, st, a);
      }
    }
    which &= bc ? 0 : 4;
  }
  if (which & 1) {
    if constexpr (FMT == FTM_FMT_GPTQ_INT4) {
      if (const int ks = gq_ks(a.L, a.T); ks != 0 && AT == FTM_DT_BF16) {
        if (ks == 4 && gq_nt(ks, a.T) == 32)
          hipLaunchKernelGGL((k_stage_a_gq<4, 32>), dim3(gridA), dim3(GqA<4>::kThreads), GqA<4>::lds(a.L.hidden), st, a);
        else if (ks == 4)
          hipLaunchKernelGGL((k_stage_a_gq<4, 64>), dim3(gridA), dim3(GqA<4>::kThreads), GqA<4>::lds(a.L.hidden), st, a);
        else
          hipLaunchKernelGGL((k_stage_a_gq<2, 64>), dim3(gridA), dim3(GqA<2>::kThreads), GqA<2>::lds(a.L.hidden), st, a);
      } else {
        hipLaunchKernelGGL((k_stage_a<FMT, AT>), dim3(gridA), dim3(kBlock), 0, st, a);
      }
    } else {
      // one workgroup per 8-channel item (routed upper bound + shared)
      const int maxU = a.L.num_experts < a.T * a.L.topk ? a.L.num_experts : a.T * a.L.topk;
      const int items = maxU * (a.L.inter / 8) + (a.L.shared_inter > 0 ? a.L.shared_inter / 8 : 0);
      const XlPlan pa = xl_plan_a<FMT, AT>(a.L, a.T);
      bool tok = false;
      if constexpr (FMT == FTM_FMT_MXFP4 && AT == FTM_DT_BF16) tok = tok_ok(a.L, a.T);
      if (tok) {
        if constexpr (FMT == FTM_FMT_MXFP4 && AT == FTM_DT_BF16) launch_tok<FMT, false>(a, maxU, st);
      } else if (pa.ok) {
        size_t lds = 4u * kXR * (size_t)xl_pitch(a.L.hidden, 4) * 2u;
        if (FMT == FTM_FMT_MXFP4) {
          // routed MXFP4 rows on scaled MFMAs: quantise the input first; the
          // bf16 regions only for a shared expert's items
          const size_t ldm = 4u * kXT * (size_t)mx_pitch((a.L.hidden + 127) / 128, 4);
          lds = a.L.shared_inter > 0 && lds > ldm ? lds : ldm;
          if (!xq_ready)  // else the router launch has quantised it
            hipLaunchKernelGGL(k_quant_mx, dim3((quant_mx_threads(a.T, a.L.hidden) + kBlock - 1) / kBlock),
                               dim3(kBlock), 0, st, (const uint16_t*)a.x, a.T, a.L.hidden, a.xq);
        }
        const int nt = pa.nt;
        const int itemsx = maxU * (a.L.inter / (8 * nt)) + (a.L.shared_inter > 0 ? a.L.shared_inter / (8 * nt) : 0);
#define FTM_XLA(NT, LPG, NLW) \
  hipLaunchKernelGGL((k_stage_a_xl<FMT, NT, LPG, NLW>), dim3(itemsx), dim3(kBlock), lds, st, a)
#define FTM_XLM(NLW)                                                                                          \
  if (a.L.shared_inter > 0)                                                                                   \
    hipLaunchKernelGGL((k_stage_a_xl<FMT, 1, kRowsNLW, NLW, true>), dim3(itemsx), dim3(kBlock), lds, st, a); \
  else if (nt == 2)                                                                                           \
    hipLaunchKernelGGL((k_stage_a_xl<FMT, 2, kRowsNLW, NLW, false>), dim3(itemsx), dim3(kBlock), lds, st, a); \
  else                                                                                                        \
    hipLaunchKernelGGL((k_stage_a_xl<FMT, 1, kRowsNLW, NLW, false>), dim3(itemsx), dim3(kBlock), lds, st, a)
        if constexpr (FMT == FTM_FMT_MXFP4) {
          // the window sized to a wave's range: no wave-loads past it issued or multiplied
          const int r = ((a.L.hidden + 127) / 128 + 3) / 4;
          if (r <= 4) { FTM_XLM(4); } else if (r <= 6) { FTM_XLM(6); } else { FTM_XLM(8); }
#undef FTM_XLM
        } else {
          if (pa.lpg == 2) FTM_XLA(1, 2, kRowsNLW); else FTM_XLA(1, kRowsNLW, kRowsNLW);
        }
#undef FTM_XLA
      } else {
        hipLaunchKernelGGL((k_stage_a_rows<FMT, AT>), dim3(items), dim3(kBlock), 0, st, a);
      }
    }
  }
  bool bcks = false;  // stage B and the combine in one launch
  if constexpr (AT == FTM_DT_BF16) bcks = bcks_ok<FMT>(a.L, a.T);
  if (which & 2) {
    const XlPlan pb = xl_plan_b<FMT, AT>(a.L, a.T);
    bool tok = false;
    if constexpr (FMT == FTM_FMT_MXFP4 && AT == FTM_DT_BF16) tok = tok_ok(a.L, a.T);
    if (tok) {
      if constexpr (FMT == FTM_FMT_MXFP4 && AT == FTM_DT_BF16) {
        const int maxU = a.L.num_experts < a.T * a.L.topk ? a.L.num_experts : a.T * a.L.topk;
        launch_tok<FMT, true>(a, maxU, st);
      }
    } else if constexpr (FMT == FTM_FMT_GPTQ_INT4) {
      if (gq_b_ok(a.L, a.T) && AT == FTM_DT_BF16) {
        // the shared expert's (token block, 16 columns) items + routed items of 128 columns
        const size_t lds_r = gq_lds_bytes(4, a.L.inter, 2, kGqBRedBytes);
        const size_t lds_s = a.L.shared_inter > 0 ? 4u * kXR * (size_t)xl_pitch(a.Imax, 4) * 2u : 0u;
        const int maxU = a.L.num_experts < a.T * a.L.topk ? a.L.num_experts : a.T * a.L.topk;
        const size_t lds = lds_r > lds_s ? lds_r : lds_s;
        // a wave's half of the K groups issued at once for a few tokens (a
        // workgroup or two per CU), two groups in flight above; one token
        // takes 64-column items (twice the CUs stream the eight experts)
        if (a.T <= kGqBAllMaxT && ((a.L.inter + 127) / 128 + 1) / 2 <= kGqAllNG) {
          const int grid = gq_b_sh_items(a.L, a.T) + maxU * (a.L.hidden / kGqNB1);
          hipLaunchKernelGGL((k_stage_b_gq<true, kGqNB1>), dim3(grid), dim3(kBlock), lds, st, a);
        } else {
          const int grid = gq_b_sh_items(a.L, a.T) + maxU * (a.L.hidden / kGqNB);
          hipLaunchKernelGGL((k_stage_b_gq<false, kGqNB>), dim3(grid), dim3(kBlock), lds, st, a);
        }
      } else {
        hipLaunchKernelGGL((k_stage_b<FMT, AT>), dim3(gridB), dim3(kBlock), 0, st, a);
      }
    } else if (pb.ok && !bcks) {
      const size_t lds = 4u * kXR * (size_t)xl_pitch(a.Imax, 1) * 2u;
      const int nt = pb.nt;
      const int maxU = a.L.num_experts < a.T * a.L.topk ? a.L.num_experts : a.T * a.L.topk;
      const int gridx = (maxU + (a.L.shared_inter > 0 ? 1 : 0)) * (a.L.hidden / (64 * nt));
#define FTM_XLB(NT, LPG) hipLaunchKernelGGL((k_stage_b_xl<FMT, NT, LPG>), dim3(gridx), dim3(kBlock), lds, st, a)
      if (pb.lpg == 2) FTM_XLB(1, 2); else FTM_XLB(1, kRowsNLW);
#undef FTM_XLB
    } else if (const XlPlan pk = ks_plan_b<FMT, AT>(a.L, a.T); pk.ok) {
      const int maxU = a.L.num_experts < a.T * a.L.topk ? a.L.num_experts : a.T * a.L.topk;
      const bool sh = a.L.shared_inter > 0;
      // the regions stage_b_ks_body lays out (kXT rows each when NOZ)
      const size_t lds = 4u * (sh || !kKsNoz<FMT> ? kXR : kXT) * (size_t)xl_pitch(a.Imax, 4) * 2u;
      const int gridk = (maxU + (sh ? 1 : 0)) * (a.L.hidden / 16);
#define FTM_KSB(LPG, NLW)                                                                          \
  if (bcks)                                                                                        \
    launch_bcks<FMT, LPG, NLW>(a, st);                                                             \
  else if (sh)                                                                                     \
    hipLaunchKernelGGL((k_stage_b_ks<FMT, LPG, NLW, true>), dim3(gridk), dim3(kBlock), lds, st, a); \
  else                                                                                             \
    hipLaunchKernelGGL((k_stage_b_ks<FMT, LPG, NLW, false>), dim3(gridk), dim3(kBlock), lds, st, a)
      if constexpr (FMT == FTM_FMT_MXFP4) {
        // the window sized to a wave's range (no post-scale groups to align)
        const int r = ((a.L.inter + 127) / 128 + 3) / 4;
        if (r <= 4) { FTM_KSB(4, 4); } else if (r <= 6) { FTM_KSB(6, 6); } else { FTM_KSB(kRowsNLW, kRowsNLW); }
      } else if (pk.lpg == 2) {
        FTM_KSB(2, kRowsNLW);
      } else {
        FTM_KSB(kRowsNLW, kRowsNLW);
      }
#undef FTM_KSB
    } else {
      hipLaunchKernelGGL((k_stage_b<FMT, AT>), dim3(gridB), dim3(kBlock), 0, st, a);
    }
  }
  if ((which & 4) && !bcks) {
    const int n4 = a.T * (a.L.hidden / 4);
    hipLaunchKernelGGL((k_combine<AT>), dim3((n4 + kBlock - 1) / kBlock), dim3(kBlock), 0, st, a);
  }
}

template <int FMT>
static void launch_stages_dt(const LayerArgs& a, int gridA, int gridB, hipStream_t st, int which, bool xq_ready) {
  if (a.L.act_dtype == FTM_DT_F32)
    launch_stages<FMT, FTM_DT_F32>(a, gridA, gridB, st, which, xq_ready);
  else
    launch_stages<FMT, FTM_DT_BF16>(a, gridA, gridB, st, which, xq_ready);
}

bool route_a_ok(const ftm_moe_layer& L, int T) {
  if (lean_route_ok(L, T)) return true;
  if (T < 1 || T > kRouteAMaxT || L.gate_w == nullptr || L.act_dtype != FTM_DT_BF16 || L.hidden % 8 != 0)
    return false;
  if (L.num_experts > 256 || L.topk > kLeanRouteMaxK || lean_ok(L, T) || gemm_path_ok(L, T)) return false;
  const int maxU = L.num_experts < T * L.topk ? L.num_experts : T * L.topk;
  int items, nt = 1;
  switch (L.w13.fmt) {
    case FTM_FMT_GPTQ_INT4:
      if (!gq_ok(L, T)) return false;
      items = maxU * (L.inter / gq_nt(gq_ks(L, T), T)) + (L.shared_inter > 0 ? L.shared_inter / 16 : 0);
      break;
    case FTM_FMT_BF16:
      if (!xl_plan_a<FTM_FMT_BF16, FTM_DT_BF16>(L, T).ok) return false;
      items = 0;
      break;
    case FTM_FMT_FP8_BLOCK:
      if (!xl_plan_a<FTM_FMT_FP8_BLOCK, FTM_DT_BF16>(L, T).ok) return false;
      items = 0;
      break;
    case FTM_FMT_INT8_PACKED:
      if (!xl_plan_a<FTM_FMT_INT8_PACKED, FTM_DT_BF16>(L, T).ok) return false;
      items = 0;
      break;
    case FTM_FMT_MXFP4: {
      const XlPlan p = xl_plan_a<FTM_FMT_MXFP4, FTM_DT_BF16>(L, T);
      if (!p.ok) return false;
      nt = p.nt;
      items = 0;
      break;
    }
    default: return false;
  }
  if (L.w13.fmt != FTM_FMT_GPTQ_INT4)  // k_stage_a_xl, NT x 8 channels an item
    items = maxU * (L.inter / (8 * nt)) + (L.shared_inter > 0 ? L.shared_inter / (8 * nt) : 0);
  return items <= kRouteAMaxItems;
}

hipError_t launch_experts(const ftm_moe_layer& L, const void* x, int T, void* out, char* ws,
                          const WsLayout& wl, hipStream_t st, int which, const RouteOut* ro, bool xq_ready) {
  if (gemm_path_ok(L, T)) {
    // above the token crossover the expert stages are tiled GEMMs
    if (which & 3) launch_gemm_stages(L, x, T, out, ws, wl, st, which & 3, xq_ready);
    which &= 4;
    if (which == 0) return hipGetLastError();
  }
  LayerArgs a = make_args(L, x, out, T, ws, wl);
  if (ro != nullptr && route_a_ok(L, T)) {
    a.route_a = true;
    a.ids_out = ro->ids;
    a.w_out = ro->w;
    a.logits_out = ro->logits;
  }
  const int maxU = L.num_experts < T * L.topk ? L.num_experts : T * L.topk;
  const int NT = L.w13.fmt == FTM_FMT_GPTQ_INT4 ? gq_nt(gq_ks(L, T), T) : 16;
  const int has_sh = L.shared_inter > 0 ? 1 : 0;
  const int gridA = maxU * (L.inter / NT) + (has_sh ? L.shared_inter / 16 : 0);
  const int gridB = (maxU + has_sh) * (L.hidden / 64);
  switch (L.w13.fmt) {
    case FTM_FMT_BF16: launch_stages_dt<FTM_FMT_BF16>(a, gridA, gridB, st, which, xq_ready); break;
    case FTM_FMT_FP8_BLOCK: launch_stages_dt<FTM_FMT_FP8_BLOCK>(a, gridA, gridB, st, which, xq_ready); break;
    case FTM_FMT_GPTQ_INT4: launch_stages_dt<FTM_FMT_GPTQ_INT4>(a, gridA, gridB, st, which, xq_ready); break;
    case FTM_FMT_INT8_PACKED: launch_stages_dt<FTM_FMT_INT8_PACKED>(a, gridA, gridB, st, which, xq_ready); break;
    case FTM_FMT_MXFP4: launch_stages_dt<FTM_FMT_MXFP4>(a, gridA, gridB, st, which, xq_ready); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// Name of the kernel launch_router / launch_topk / launch_experts start for
// `stage` (FTM_STAGE_*) of layer L at T tokens: the same predicates as the
// launchers above, for profilers and benchmarks that attribute time by name.
// Stage B and the combine run as one launch (k_stage_bc_lean).
static bool bc_fused(const ftm_moe_layer& L, int T) {
  return lean_ok(L, T) && L.w13.fmt == FTM_FMT_FP8_BLOCK && L.act_dtype == FTM_DT_BF16 && T <= kBcMaxT &&
         L.topk + (L.shared_inter > 0 ? 1 : 0) <= kBcMaxKP;
}

template <int FMT, int AT>
static const char* expert_kernel_name(const ftm_moe_layer& L, int T, int stage) {
  const bool lean = FMT == FTM_FMT_FP8_BLOCK && AT == FTM_DT_BF16 && lean_ok(L, T);
  if (stage == FTM_STAGE_W13) {
    if (lean) return lean_route_ok(L, T) ? "k_stage_a_lean_route" : "k_stage_a_lean";
    if (FMT == FTM_FMT_GPTQ_INT4) return AT == FTM_DT_BF16 && gq_ok(L, T) ? "k_stage_a_gq" : "k_stage_a";
    if (AT == FTM_DT_BF16 && tok_ok(L, T)) return "k_stage_tok_a";
    return xl_plan_a<FMT, AT>(L, T).ok ? "k_stage_a_xl" : "k_stage_a_rows";
  }
  if (lean) return L.topk + (L.shared_inter > 0 ? 1 : 0) <= kBcMaxKP && T <= kBcMaxT ? "k_stage_bc_lean" : "k_stage_b_lean";
  if (FMT == FTM_FMT_GPTQ_INT4) return AT == FTM_DT_BF16 && gq_b_ok(L, T) ? "k_stage_b_gq" : "k_stage_b";
  if (AT == FTM_DT_BF16 && tok_ok(L, T)) return "k_stage_tok_b";
  if (AT == FTM_DT_BF16 && bcks_ok<FMT>(L, T)) return "k_stage_bc_ks";
  if (xl_plan_b<FMT, AT>(L, T).ok) return "k_stage_b_xl";
  return ks_plan_b<FMT, AT>(L, T).ok ? "k_stage_b_ks" : "k_stage_b";
}

template <int FMT>
static const char* expert_kernel_name_dt(const ftm_moe_layer& L, int T, int stage) {
  return L.act_dtype == FTM_DT_F32 ? expert_kernel_name<FMT, FTM_DT_F32>(L, T, stage)
                                   : expert_kernel_name<FMT, FTM_DT_BF16>(L, T, stage);
}

const char* stage_kernel_name(const ftm_moe_layer& L, int T, int stage) {
  switch (stage) {
    case FTM_STAGE_ROUTER:
      if (route_topk_fused(L, T)) return "k_route_topk1";
      return router_by_rows(L.num_experts + (L.shared_inter > 0 ? 1 : 0), T, L.hidden) ? "k_router_rows" : "k_router";
    case FTM_STAGE_TOPK:
      if (route_a_ok(L, T) || route_topk_fused(L, T)) return "";  // routed inside stage A / the router
      return T <= kTopk1MaxT ? "k_topk1" : T >= kTopkBlkMinT ? "k_topk_blk" : "k_topk";
    case FTM_STAGE_COMBINE: return bc_fused(L, T) || bcks_fused(L, T) ? "" : "k_combine";  // "": done by stage B
    case FTM_STAGE_W13:
    case FTM_STAGE_W2: break;
    default: return nullptr;
  }
  if (gemm_path_ok(L, T)) return stage == FTM_STAGE_W13 ? gemm_a_kernel_name(L) : gemm_b_kernel_name(L, T);
  switch (L.w13.fmt) {
    case FTM_FMT_BF16: return expert_kernel_name_dt<FTM_FMT_BF16>(L, T, stage);
    case FTM_FMT_FP8_BLOCK: return expert_kernel_name_dt<FTM_FMT_FP8_BLOCK>(L, T, stage);
    case FTM_FMT_GPTQ_INT4: return expert_kernel_name_dt<FTM_FMT_GPTQ_INT4>(L, T, stage);
    case FTM_FMT_INT8_PACKED: return expert_kernel_name_dt<FTM_FMT_INT8_PACKED>(L, T, stage);
    case FTM_FMT_MXFP4: return expert_kernel_name_dt<FTM_FMT_MXFP4>(L, T, stage);
    default: return nullptr;
  }
}

template <int FMT>
static void launch_linear_t(const LinArgs& a, dim3 grid, int x_dt, hipStream_t st) {
  if (x_dt == FTM_DT_F32)
    hipLaunchKernelGGL((k_linear<FMT, FTM_DT_F32>), grid, dim3(kBlock), 0, st, a);
  else if (x_dt == FTM_DT_F16)
    hipLaunchKernelGGL((k_linear<FMT, FTM_DT_F16>), grid, dim3(kBlock), 0, st, a);
  else
    hipLaunchKernelGGL((k_linear<FMT, FTM_DT_BF16>), grid, dim3(kBlock), 0, st, a);
}

hipError_t launch_linear(const ftm_proj& P, int slot, const void* x, int x_dt, int M, void* out, int out_dt,
                         const void* bias, int bias_dt, int final_dt, hipStream_t st) {
  LinArgs a;
  a.P = P;
  a.slot = slot;
  a.x = x;
  a.M = M;
  a.out = out;
  a.out_dt = out_dt;
  a.bias = bias;
  a.bias_dt = bias_dt;
  a.final_dt = final_dt;
  const dim3 grid((P.N + 63) / 64, (M + 15) / 16);
  switch (P.fmt) {
    case FTM_FMT_BF16: launch_linear_t<FTM_FMT_BF16>(a, grid, x_dt, st); break;
    case FTM_FMT_FP8_BLOCK: launch_linear_t<FTM_FMT_FP8_BLOCK>(a, grid, x_dt, st); break;
    case FTM_FMT_GPTQ_INT4: launch_linear_t<FTM_FMT_GPTQ_INT4>(a, grid, x_dt, st); break;
    case FTM_FMT_INT8_PACKED: launch_linear_t<FTM_FMT_INT8_PACKED>(a, grid, x_dt, st); break;
    case FTM_FMT_MXFP4: launch_linear_t<FTM_FMT_MXFP4>(a, grid, x_dt, st); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_fill_routing(int T, int32_t slot, int32_t* slot_word, int32_t* ids, float* w, hipStream_t st) {
  const int blocks = (T + 255) / 256 > 0 ? (T + 255) / 256 : 1;
  hipLaunchKernelGGL(k_fill_routing, dim3(blocks), dim3(256), 0, st, T, slot, slot_word, ids, w);
  return hipGetLastError();
}

}  // namespace ftm
