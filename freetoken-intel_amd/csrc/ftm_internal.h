// ftm_internal.h -- host-side layout of the layer workspace and the kernel
// launchers shared by the C ABI (ftm_capi.cpp) and the kernel files.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "ftmoe.h"

namespace ftm {

// ---- control region (first FTM_WS_CTRL_BYTES of a workspace, int32 words).
// Zero between calls: every counter is reset by the workgroup that consumes it.
// Work record of routed expert u (recs[u], kRecWords int32): expert id, token
// count, bank slot (-1 = not resident), the pairs of its first kRecPairs
// tokens (-1 past the count), one pad word.  Written by the top-k compaction,
// read by the decode stages with one scalar load.
constexpr int kRecWords = 8;
constexpr int kRecPairs = 4;
// Batches up to kXlMaxT tokens run the decode stages with activations in LDS
// and per-expert work records (latency-bound there); larger batches keep the
// register-fed chunked kernels, which sustain more bytes in flight per CU.
// Measured on MI355X (C3 layer before its lean kernels, w13 + w2 us): T=1 15.9
// vs 16.7, T=4 30.7 vs 34.5, T=8 54.5 vs 54.5, T=16 92.4 vs 88.1.  MXFP4
// stage A (C4, w13 us) keeps the LDS path up to kXlMaxTMx: T=8 67.4 -> 54.8,
// T=16 90.9 -> 76.7, and with its scale bytes fetched 16 at a time T=24
// 106.6 -> 89.3, T=32 115.6 -> 100.1.  On scaled MFMAs (and the K-split
// stage B beside it) it also beats the register-fed kernels and the GEMM
// tiles up to 16 tokens per expert (C4, w13 + w2 us): T=64 200 -> 153 (rows
// kernels), T=128 288 -> 235 (tiles); at T=256 (32 per expert) the tiles win,
// 326 against 401.  MXFP4 layers therefore take the tiles only above 16
// tokens per expert (gemm_path_ok) and the LDS path up to kXlMaxTMx tokens.
constexpr int kXlMaxT = 4;
constexpr int kXlMaxTMx = 256;
// the top-k compaction writes work records up to this many tokens (the xl
// stage A and the K-split stage B read them)
constexpr int kRecMaxT = 256;
// Decode batches up to kLeanRouteMaxT tokens (top-k up to kLeanRouteMaxK) route
// inside the lean stage A, which takes the top-k launch out of the layer's
// chain of dependent launches.  Every stage-A workgroup then spends ~3 us
// routing before its weight loads, which pays while the grid fits one round
// of workgroups: measured on MI355X (C3), T = 1: 27.0 us per layer against
// 29.6 with the top-k launch; T = 4: 47.8 against 42.7 (2,112 workgroups);
// measured again beside k_route_topk1 (us per layer): T = 3 30.5 against
// 29.5, T = 4 34.6 against 32.5.
// A record holds every pair of such an expert.
constexpr int kLeanRouteMaxT = 2;
constexpr int kLeanRouteMaxK = 16;
// The same routing inside the GPTQ and LDS-activation stage A kernels
// (k_stage_a_gq, k_stage_a_xl) up to kRouteAMaxT tokens, while the stage-A
// grid stays within kRouteAMaxItems workgroups (about one round of them: a
// second round would pay the routing again).
constexpr int kRouteAMaxT = 4;
constexpr int kRouteAMaxItems = 1536;
static_assert(kLeanRouteMaxT <= kRouteAMaxT && kRouteAMaxT <= kRecPairs, "records hold all pairs of a routed expert");
constexpr int kCtrlArriveTopk = 0;  // arrivals of the top-k workgroups
constexpr int kCtrlNRouted = 1;     // routed experts with >= 1 token (written per call)
constexpr int kCtrlNU = 2;          // nRouted + shared expert
constexpr int kCtrlError = 3;       // sticky error bits (FTM_WS_ERR_*), read and cleared by the caller
static_assert(kCtrlError * 4 == FTM_WS_ERROR_OFFSET, "error word offset of the C ABI");
constexpr int kCtrlExpertCnt = 16;  // [E] per-expert pair counters (E <= kMaxExperts)
constexpr int kMaxExperts = 512;
constexpr int kCtrlTileCnt = kCtrlExpertCnt + kMaxExperts;  // [H/64] combine arrivals
constexpr int kMaxColTiles = FTM_WS_CTRL_BYTES / 4 - kCtrlTileCnt;

// MXFP4 decode: the layer input quantised for the scaled fp8 x fp4 MFMAs.
// Per token row, per 128-element chunk of the hidden dimension, kMxChunk
// bytes: 128 e4m3 "hi" values, 128 e4m3 "lo" values, then the e8m0 scale
// bytes of the chunk's four 32-element blocks as (hi, lo) pairs and 8 zero
// bytes.  x = hi * 2^(s_hi - 127) + lo * 2^(s_lo - 127) reproduces every bf16
// input within 2^-13 of its block's maximum exactly (rows past the hidden
// size are zeros).
constexpr int kMxChunk = 272;
__host__ __device__ inline int mx_row_bytes(int H) { return (H + 127) / 128 * kMxChunk; }
// Weight formats the scaled-MFMA stages take (bf16 activations): MXFP4, and
// FP8 e4m3 with 128 x 128 blocks (the block scale applied to each K step's
// partial sums).
inline bool mx_fmt(const ftm_moe_layer& L) {
  if (L.act_dtype != FTM_DT_BF16) return false;
  if (L.w13.fmt == FTM_FMT_MXFP4) return true;
  return L.w13.fmt == FTM_FMT_FP8_BLOCK && L.w13.group == 128 && L.w2.group == 128 &&
         L.w13.s_dtype == FTM_DT_F32 && L.w2.s_dtype == FTM_DT_F32 && L.hidden % 128 == 0 && L.inter % 128 == 0;
}

struct WsLayout {
  size_t misc, logits, wts, ids, lists, uniq, ucnt, recs, hbuf, ybuf, hq, xq, total;
  int T, E, KP, Imax;
};

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

inline WsLayout ws_layout(const ftm_moe_layer& L, int T) {
  WsLayout w;
  w.T = T;
  w.E = L.num_experts;
  w.KP = L.topk + (L.shared_inter > 0 ? 1 : 0);
  w.Imax = L.inter > L.shared_inter ? L.inter : L.shared_inter;
  const size_t Tt = (size_t)(T > 0 ? T : 1);
  const size_t act = L.act_dtype == FTM_DT_F32 ? 4 : 2;
  size_t o = FTM_WS_CTRL_BYTES;
  w.misc = o;   o = align_up(o + 256, 256);
  w.logits = o; o = align_up(o + 4 * Tt * (w.E + 1), 256);
  w.wts = o;    o = align_up(o + 4 * Tt * w.KP, 256);
  w.ids = o;    o = align_up(o + 4 * Tt * L.topk, 256);
  w.lists = o;  o = align_up(o + 4 * (size_t)w.E * Tt, 256);
  w.uniq = o;   o = align_up(o + 4 * (size_t)(w.E + 1), 256);
  w.ucnt = o;   o = align_up(o + 4 * (size_t)(w.E + 1), 256);
  w.recs = o;   o = align_up(o + 4 * (size_t)kRecWords * (w.E + 1), 256);
  w.hbuf = o;   o = align_up(o + act * Tt * w.KP * w.Imax, 256);
  w.ybuf = o;   o = align_up(o + 4 * Tt * w.KP * (size_t)L.hidden, 256);
  // layers the scaled-MFMA stages take: the input and h quantised (kMxChunk
  // layout, by token and by pair)
  const bool mx = mx_fmt(L);
  w.hq = o;     o = align_up(o + (mx ? Tt * w.KP * (size_t)mx_row_bytes(w.Imax) : 0), 256);
  w.xq = o;     o = align_up(o + (mx ? Tt * (size_t)mx_row_bytes(L.hidden) : 0), 256);
  w.total = o;
  return w;
}

// ---- launchers (ftm_moe.hip); all return hipError_t of the launch
// quant: also quantise the input for the MXFP4 stage A (mx_stage_a) in the
// same launch; the expert stages are then launched with xq_ready.
hipError_t launch_router(const ftm_moe_layer& L, const void* x, int T, int row_begin, int row_end, char* ws,
                         const WsLayout& wl, hipStream_t st, bool quant = false);
hipError_t launch_topk(const ftm_moe_layer& L, int T, const void* logits_in, int logits_dt,
                       const int32_t* ids_in, const float* w_in, int32_t* ids_out, float* w_out,
                       float* logits_out, char* ws, const WsLayout& wl, hipStream_t st);
// The caller's routing outputs of ftm_moe_forward (each may be null).
struct RouteOut {
  int32_t* ids;
  float* w;
  float* logits;
};
// ro: route inside the expert stages where lean_route_ok allows it (the caller
// then launches no top-k); which: bit 0 = stage A, bit 1 = stage B, bit 2 = combine;
// xq_ready: the router launch has quantised the input (launch_router's quant).
hipError_t launch_experts(const ftm_moe_layer& L, const void* x, int T, void* out, char* ws,
                          const WsLayout& wl, hipStream_t st, int which = 7, const RouteOut* ro = nullptr,
                          bool xq_ready = false);
// Stage A of MXFP4 layers on scaled MFMAs over the quantised input (the xq
// workspace region, written by k_quant_mx or a router launch with quant):
// the LDS decode stage (mx_stage_a) or the GEMM tiles (mx_gemm_ok above the
// crossover); mx_input: either.
bool mx_stage_a(const ftm_moe_layer& L, int T);
bool mx_input(const ftm_moe_layer& L, int T);
// Prefill side of the crossover (ftm_gemm.hip): whether the tiled GEMM stages
// take this layer at T tokens, and their launch (which: bit 0 = w13, bit 1 = w2).
bool gemm_path_ok(const ftm_moe_layer& L, int T);
const char* gemm_a_kernel_name(const ftm_moe_layer& L);  // the stage A tile kernel the layer takes
const char* gemm_b_kernel_name(const ftm_moe_layer& L, int T);  // the stage B tile kernel at T tokens
void launch_gemm_stages(const ftm_moe_layer& L, const void* x, int T, void* out, char* ws, const WsLayout& wl,
                        hipStream_t st, int which, bool xq_ready = false);
// MXFP4 stage A on the scaled-MFMA tiles (k_gemm_a_mx) above the crossover.
bool mx_gemm_ok(const ftm_moe_layer& L);
// k_quant_mx: the input (T x H bf16) into the xq region's two-term e4m3 split.
void launch_quant_mx(const void* x, int T, int H, uint8_t* xq, hipStream_t st);
// The lean FP8 decode kernels (ftm_moe.hip) cover H = 2048 (a 512-element K
// range per wave in stage A), I = 512 (one 8-load window per wave in stage
// B), fp32 block-128 scales, no projection biases, bf16 activations and a
// shared expert (if any) of the routed width, below the GEMM crossover.
inline bool lean_ok(const ftm_moe_layer& L, int T) {
  const ftm_proj &A = L.w13, &B = L.w2;
  if (A.fmt != FTM_FMT_FP8_BLOCK || L.act_dtype != FTM_DT_BF16) return false;
  if (A.group != 128 || B.group != 128 || A.s_dtype != FTM_DT_F32 || B.s_dtype != FTM_DT_F32) return false;
  if (A.bias != nullptr || B.bias != nullptr) return false;
  if (L.hidden != 2048 || L.inter != 512) return false;
  if (L.shared_inter != 0 && L.shared_inter != L.inter) return false;
  return !gemm_path_ok(L, T);
}

// Small decode batches on the lean kernels: stage A routes the T <=
// kLeanRouteMaxT tokens in every workgroup (one wave per token) instead of
// waiting for a top-k launch; E <= 256 (four candidates per lane) and k <=
// kLeanRouteMaxK.
inline bool lean_route_ok(const ftm_moe_layer& L, int T) {
  return lean_ok(L, T) && T <= kLeanRouteMaxT && L.num_experts <= 256 && L.topk <= kLeanRouteMaxK;
}

// Small decode batches whose stage A routes the tokens itself (route_a): the
// lean kernels (lean_route_ok), or k_stage_a_gq / k_stage_a_xl with bf16
// activations and a router matrix, T <= kRouteAMaxT, E <= 256, k <=
// kLeanRouteMaxK and a stage-A grid of at most kRouteAMaxItems workgroups.
bool route_a_ok(const ftm_moe_layer& L, int T);

// Router and top-k as one launch (k_route_topk1) for small batches that do
// not route inside stage A: bf16 activations, a router matrix, T <= 16.
bool route_topk_fused(const ftm_moe_layer& L, int T);
hipError_t launch_route_topk(const ftm_moe_layer& L, const void* x, int T, int32_t* ids_out, float* w_out,
                             float* logits_out, char* ws, const WsLayout& wl, hipStream_t st, bool quant = false);

hipError_t launch_linear(const ftm_proj& P, int slot, const void* x, int x_dt, int M, void* out,
                         int out_dt, const void* bias, int bias_dt, int final_dt, hipStream_t st);
hipError_t launch_fill_routing(int T, int32_t slot, int32_t* slot_word, int32_t* ids, float* w, hipStream_t st);
hipError_t launch_ws_init(void* ws, hipStream_t st);
// Base name of the kernel a stage (FTM_STAGE_*) launches for L at T tokens.
const char* stage_kernel_name(const ftm_moe_layer& L, int T, int stage);
// ftm_dequant.hip
hipError_t launch_linear_generic(const ftm_proj& P, int slot, const void* x, int x_dt, int M, void* out,
                                 int out_dt, const void* bias, int bias_dt, int final_dt, hipStream_t st);
hipError_t launch_experts_generic(const ftm_moe_layer& L, const void* x, int T, void* out, char* ws,
                                  const WsLayout& wl, hipStream_t st);
hipError_t launch_dequant(const ftm_proj& P, int slot, void* out, int out_dt, int transpose,
                          hipStream_t st);

}  // namespace ftm
