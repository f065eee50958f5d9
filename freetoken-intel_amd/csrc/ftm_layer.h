// ftm_layer.h -- the per-call argument block of the layer kernels and the small
// device helpers shared by the decode kernels (ftm_moe.hip) and the tiled
// prefill GEMMs (ftm_gemm.hip).
#pragma once

#include <math.h>

#include "ftm_device.h"
#include "ftm_internal.h"

namespace ftm {

struct LayerArgs {
  ftm_moe_layer L;
  const void* x;
  void* out;
  int T, KP, Imax;
  bool lean;        // decode stages use the lean FP8 kernels (they read the work records)
  bool route_a;     // stage A routes the tokens itself (no top-k launch, route_a_ok)
  int32_t* ids_out; // route_a: the caller's routing outputs (each may be null)
  float* w_out;
  float* logits_out;
  int32_t* ctrl;
  float* logits;    // [T, E+1]   (column E = shared-expert gate logit)
  float* wts;       // [T*KP]     router weight of pair p = t*KP + j (j == k: shared gate)
  int32_t* ids;     // [T*k]
  int32_t* lists;   // [E, T]     pair ids routed to expert e (order within an expert is free)
  int32_t* uniq;    // [E+1]      routed experts with >= 1 pair, ascending
  int32_t* ucnt;    // [E+1]
  int32_t* recs;    // [E+1, kRecWords] work records of the routed experts
  char* hbuf;       // [T*KP, Imax] act dtype
  float* ybuf;      // [T*KP, H]
  uint8_t* hq;      // [T*KP, mx_row_bytes(Imax)]  mx_fmt layers: h quantised by stage A's scaled-MFMA tiles
  uint8_t* xq;      // [T, mx_row_bytes(H)]  mx_fmt layers: the quantised input (kMxChunk layout)
};

inline LayerArgs make_args(const ftm_moe_layer& L, const void* x, void* out, int T, char* ws,
                           const WsLayout& wl) {
  LayerArgs a;
  a.L = L;
  a.x = x;
  a.out = out;
  a.T = T;
  a.KP = wl.KP;
  a.Imax = wl.Imax;
  a.lean = lean_ok(L, T);
  a.route_a = false;
  a.ids_out = nullptr;
  a.w_out = nullptr;
  a.logits_out = nullptr;
  a.ctrl = (int32_t*)ws;
  a.logits = (float*)(ws + wl.logits);
  a.wts = (float*)(ws + wl.wts);
  a.ids = (int32_t*)(ws + wl.ids);
  a.lists = (int32_t*)(ws + wl.lists);
  a.uniq = (int32_t*)(ws + wl.uniq);
  a.ucnt = (int32_t*)(ws + wl.ucnt);
  a.recs = (int32_t*)(ws + wl.recs);
  a.hbuf = ws + wl.hbuf;
  a.ybuf = (float*)(ws + wl.ybuf);
  a.hq = (uint8_t*)(ws + wl.hq);
  a.xq = (uint8_t*)(ws + wl.xq);
  return a;
}

// Pair slot p of row m of an expert's token list (the shared expert has no
// list: its rows are the tokens, p = m*KP + shared_col), or -1 past cnt.
// A buffer load, so callers issue it early without a branch around it.
__device__ __forceinline__ int pair_of_row(Rsrc lres, bool has_list, int m, int cnt, int KP, int shared_col) {
  const uint32_t v = bload4(lres, (has_list && m < cnt) ? 4u * (uint32_t)m : kOOB);
  return m < cnt ? (has_list ? (int)v : m * KP + shared_col) : -1;
}

// Gate activation h = act(g) * u; FTM_ACT_SWIGLU_OAI is gpt-oss's clamped form
// (python/freetoken/models/gpt_oss/__init__.py:306-310).
__device__ __forceinline__ float act_fn(int act, float g, float u, float alpha, float limit) {
  if (act == FTM_ACT_SILU) return g / (1.0f + expf(-g)) * u;
  if (act == FTM_ACT_GELU) return 0.5f * g * (1.0f + erff(g * 0.70710678118654752f)) * u;
  if (act == FTM_ACT_RELU) return fmaxf(g, 0.0f) * u;
  // FTM_ACT_SWIGLU_OAI
  g = fminf(g, limit);
  u = fminf(fmaxf(u, -limit), limit);
  const float glu = g / (1.0f + expf(-alpha * g));
  return (u + 1.0f) * glu;
}

// The dense bf16 shared expert as a one-slot projection.
__device__ __forceinline__ ProjSlot shared_view(const void* w, int N, int K) {
  ProjSlot v;
  v.w = (const char*)w;
  v.s = v.z = v.bias = nullptr;
  v.fmt = FTM_FMT_BF16;
  v.s_dt = v.bias_dt = FTM_DT_BF16;
  v.group = 0;
  v.N = N;
  v.K = K;
  return v;
}

}  // namespace ftm
