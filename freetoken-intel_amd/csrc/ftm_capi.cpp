// ftm_capi.cpp -- extern "C" entry points of libftmoe.so.
//
// Every entry point validates its arguments completely before it touches the
// HIP runtime, so argument errors are reported identically with or without a
// GPU.  Error codes follow the reference CPU MoE ABI
// (python/freetoken/kernel/csrc/cpu_moe/cpu_moe.cpp:733-739).
#include <hip/hip_runtime.h>
#include <string.h>

#include <mutex>

#include "ftm_internal.h"

using namespace ftm;

// ---- scratch of ftm_moe_forward_noalloc: the layer workspace as a file-scope
// device array, FTM_NOALLOC_SCRATCH_BYTES per GPU, held until the process
// ends.  In host code `scratch` is only a stand-in for the symbol: the device
// address of each GPU's copy comes from hipGetSymbolAddress, once per device,
// and only that address is handed to kernels.
static __device__ __align__(256) char scratch[FTM_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// This device's scratch address, looked up once per device.
int scratch_of_current_device(void** ptr) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    (void)hipGetLastError();
    return FTM_ERR_HIP;
  }
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) {
      (void)hipGetLastError();
      return FTM_ERR_HIP;
    }
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return FTM_OK;
}

bool dt_ok(int dt) { return dt == FTM_DT_F32 || dt == FTM_DT_F16 || dt == FTM_DT_BF16; }

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Whether the register-dequant MFMA engine takes this projection (else the
// generic scalar kernels run it).
int check_proj(const ftm_proj* P) {
  if (P == nullptr || P->w == nullptr) return FTM_ERR_NULL;
  if (P->N <= 0 || P->K <= 0 || P->num_slots <= 0) return FTM_ERR_DIM;
  if (P->w_stride < 0 || P->s_stride < 0 || P->z_stride < 0 || P->bias_stride < 0) return FTM_ERR_DIM;
  if (P->bias != nullptr && !dt_ok(P->bias_dtype)) return FTM_ERR_FORMAT;
  if (!aligned16(P->w) || (P->num_slots > 1 && (P->w_stride & 15) != 0)) return FTM_ERR_ALIGN;
  switch (P->fmt) {
    case FTM_FMT_BF16:
      if (P->K % 8 != 0) return FTM_ERR_DIM;
      return FTM_OK;
    case FTM_FMT_FP8_BLOCK:
      if (P->s == nullptr) return FTM_ERR_NULL;
      if (!dt_ok(P->s_dtype)) return FTM_ERR_FORMAT;
      if (P->group <= 0 || P->group % 64 != 0) return FTM_ERR_DIM;
      if (P->K % 16 != 0) return FTM_ERR_DIM;
      return FTM_OK;
    case FTM_FMT_GPTQ_INT4:
      if (P->s == nullptr || P->z == nullptr) return FTM_ERR_NULL;
      if (!dt_ok(P->s_dtype)) return FTM_ERR_FORMAT;
      if (P->group <= 0 || P->group % 32 != 0) return FTM_ERR_DIM;
      if (P->K % 8 != 0 || P->N % 8 != 0) return FTM_ERR_DIM;
      return FTM_OK;
    case FTM_FMT_INT8_PACKED:
      if (P->s == nullptr) return FTM_ERR_NULL;
      if (!dt_ok(P->s_dtype)) return FTM_ERR_FORMAT;
      if (P->group <= 0 || P->K % P->group != 0) return FTM_ERR_DIM;
      if (P->K % 16 != 0) return FTM_ERR_DIM;
      if (P->group % 64 != 0 && P->group != P->K) return FTM_ERR_DIM;
      return FTM_OK;
    case FTM_FMT_MXFP4:
      if (P->s == nullptr) return FTM_ERR_NULL;
      if (P->group != 32 || P->K % 32 != 0) return FTM_ERR_DIM;
      return FTM_OK;
    default:
      return FTM_ERR_FORMAT;
  }
}

// Looser check for the dequant kernel (any element layout the format allows).
int check_proj_dequant(const ftm_proj* P) {
  if (P == nullptr || P->w == nullptr) return FTM_ERR_NULL;
  if (P->N <= 0 || P->K <= 0 || P->num_slots <= 0) return FTM_ERR_DIM;
  switch (P->fmt) {
    case FTM_FMT_BF16:
    case FTM_FMT_FP32:
      return FTM_OK;
    case FTM_FMT_FP8_BLOCK:
    case FTM_FMT_FP8_E5M2_BLOCK:
      if (P->s == nullptr) return FTM_ERR_NULL;
      if (!dt_ok(P->s_dtype)) return FTM_ERR_FORMAT;
      return P->group > 0 ? FTM_OK : FTM_ERR_DIM;
    case FTM_FMT_GPTQ_INT4:
      if (P->s == nullptr || P->z == nullptr) return FTM_ERR_NULL;
      if (!dt_ok(P->s_dtype)) return FTM_ERR_FORMAT;
      if (P->group <= 0 || P->K % 8 != 0 || P->N % 8 != 0) return FTM_ERR_DIM;
      return FTM_OK;
    case FTM_FMT_INT8_PACKED:
      if (P->s == nullptr) return FTM_ERR_NULL;
      if (!dt_ok(P->s_dtype)) return FTM_ERR_FORMAT;
      if (P->group <= 0 || P->K % P->group != 0 || P->K % 4 != 0) return FTM_ERR_DIM;
      return FTM_OK;
    case FTM_FMT_MXFP4:
      if (P->s == nullptr) return FTM_ERR_NULL;
      if (P->K % 32 != 0) return FTM_ERR_DIM;
      return FTM_OK;
    default:
      return FTM_ERR_FORMAT;
  }
}

// Validity for the layer entry points (any shape the generic path can run).
int check_layer(const ftm_moe_layer* L, bool need_router) {
  if (L == nullptr) return FTM_ERR_NULL;
  const int E = L->num_experts, H = L->hidden, I = L->inter, k = L->topk;
  if (E <= 0 || E > kMaxExperts || H <= 0 || I <= 0 || k <= 0 || k > E || k > 64) return FTM_ERR_DIM;
  if (L->act_dtype != FTM_DT_BF16 && L->act_dtype != FTM_DT_F32) return FTM_ERR_FORMAT;
  // bf16 activations hold h in bf16: only the no-op roundings fit them
  if (!dt_ok(L->h_dtype) || (L->act_dtype == FTM_DT_BF16 && L->h_dtype == FTM_DT_F16)) return FTM_ERR_FORMAT;
  if (L->route_mode < FTM_ROUTE_SOFTMAX_TOPK || L->route_mode > FTM_ROUTE_TOPK_SOFTMAX) return FTM_ERR_FORMAT;
  if (L->act < FTM_ACT_SILU || L->act > FTM_ACT_SWIGLU_OAI) return FTM_ERR_FORMAT;
  int rc = check_proj_dequant(&L->w13);
  if (rc != FTM_OK) return rc;
  rc = check_proj_dequant(&L->w2);
  if (rc != FTM_OK) return rc;
  if (L->w13.fmt != L->w2.fmt) return FTM_ERR_FORMAT;
  if (L->w13.N != 2 * I || L->w13.K != H || L->w2.N != H || L->w2.K != I) return FTM_ERR_DIM;
  if ((L->w13.bias != nullptr && !dt_ok(L->w13.bias_dtype)) || (L->w2.bias != nullptr && !dt_ok(L->w2.bias_dtype)))
    return FTM_ERR_FORMAT;
  if (L->shared_inter < 0) return FTM_ERR_DIM;
  if (L->shared_inter > 0) {
    if (L->shared_w13 == nullptr || L->shared_w2 == nullptr || L->shared_gate == nullptr) return FTM_ERR_NULL;
    // the shared-expert gate logit comes from the bf16 router kernel
    if (L->act_dtype != FTM_DT_BF16) return FTM_ERR_FORMAT;
    if (H % 8 != 0) return FTM_ERR_DIM;
    if (!aligned16(L->shared_gate)) return FTM_ERR_ALIGN;
  }
  if (need_router) {
    if (L->gate_w == nullptr) return FTM_ERR_NULL;
    if (L->act_dtype != FTM_DT_BF16) return FTM_ERR_FORMAT;
    if (H % 8 != 0) return FTM_ERR_DIM;
    if (!aligned16(L->gate_w)) return FTM_ERR_ALIGN;
  }
  return FTM_OK;
}

// Whether the MFMA engine takes this layer (else the generic scalar path runs).
bool fast_layer(const ftm_moe_layer* L, const void* x) {
  const int H = L->hidden, I = L->inter;
  if (L->apply_router_weight_on_input) return false;  // scaled inputs: generic path
  if (check_proj(&L->w13) != FTM_OK || check_proj(&L->w2) != FTM_OK) return false;
  if (H % 64 != 0 || H / 64 > kMaxColTiles) return false;
  const int nt = L->w13.fmt == FTM_FMT_GPTQ_INT4 ? 64 : 16;
  if (I % nt != 0) return false;
  if (L->w13.fmt == FTM_FMT_FP8_BLOCK && I % L->w13.group != 0) return false;
  if (L->shared_inter > 0 &&
      (L->shared_inter % 16 != 0 || !aligned16(L->shared_w13) || !aligned16(L->shared_w2)))
    return false;
  return aligned16(x);
}

// xq_ready: the router launch quantised the input (launch_router's quant)
hipError_t run_experts(const ftm_moe_layer& L, const void* x, int T, void* out, char* ws, const WsLayout& wl,
                       hipStream_t st, bool xq_ready = false) {
  return fast_layer(&L, x) ? launch_experts(L, x, T, out, ws, wl, st, 7, nullptr, xq_ready)
                           : launch_experts_generic(L, x, T, out, ws, wl, st);
}

int check_ws(const ftm_moe_layer* L, int T, const void* ws, size_t ws_bytes) {
  if (ws == nullptr) return FTM_ERR_WORKSPACE;
  if (((uintptr_t)ws & 255u) != 0) return FTM_ERR_ALIGN;
  if (ws_bytes < ws_layout(*L, T).total) return FTM_ERR_WORKSPACE;
  return FTM_OK;
}

int hip_rc(hipError_t e) { return e == hipSuccess ? FTM_OK : FTM_ERR_HIP; }

}  // namespace

extern "C" {

int ftm_version(void) { return FTM_ABI_VERSION; }

size_t ftm_moe_workspace_bytes(const ftm_moe_layer* layer, int32_t num_tokens) {
  if (layer == nullptr || num_tokens < 0) return 0;
  return ws_layout(*layer, num_tokens).total;
}

int ftm_workspace_init(void* workspace, size_t ws_bytes, void* stream) {
  if (workspace == nullptr) return FTM_ERR_NULL;
  if (ws_bytes < (size_t)FTM_WS_CTRL_BYTES) return FTM_ERR_WORKSPACE;
  if (((uintptr_t)workspace & 255u) != 0) return FTM_ERR_ALIGN;
  return hip_rc(launch_ws_init(workspace, (hipStream_t)stream));
}

int ftm_moe_forward(const ftm_moe_layer* layer, const void* x, int32_t num_tokens, void* out, int32_t* topk_ids,
                    float* topk_w, float* logits, void* workspace, size_t ws_bytes, void* stream) {
  int rc = check_layer(layer, true);
  if (rc != FTM_OK) return rc;
  if (num_tokens < 0) return FTM_ERR_DIM;
  if (num_tokens == 0) return FTM_OK;
  if (x == nullptr || out == nullptr) return FTM_ERR_NULL;
  if (!aligned16(x)) return FTM_ERR_ALIGN;
  rc = check_ws(layer, num_tokens, workspace, ws_bytes);
  if (rc != FTM_OK) return rc;
  const WsLayout wl = ws_layout(*layer, num_tokens);
  hipStream_t st = (hipStream_t)stream;
  char* ws = (char*)workspace;
  const int rows = layer->num_experts + (layer->shared_inter > 0 ? 1 : 0);
  // small decode batches route inside stage A (no top-k launch)
  const bool fused = fast_layer(layer, x) && route_a_ok(*layer, num_tokens);
  // the router launch also quantises the input of an MXFP4 stage A
  const bool xq = mx_input(*layer, num_tokens);
  if (!fused && route_topk_fused(*layer, num_tokens)) {  // router + top-k in one launch
    hipError_t e = launch_route_topk(*layer, x, num_tokens, topk_ids, topk_w, logits, ws, wl, st, true);
    if (e == hipSuccess) e = run_experts(*layer, x, num_tokens, out, ws, wl, st, xq);
    return hip_rc(e);
  }
  hipError_t e = launch_router(*layer, x, num_tokens, 0, rows, ws, wl, st, true);
  if (fused) {
    const RouteOut ro = {topk_ids, topk_w, logits};
    if (e == hipSuccess) e = launch_experts(*layer, x, num_tokens, out, ws, wl, st, 7, &ro, xq);
    return hip_rc(e);
  }
  if (e == hipSuccess)
    e = launch_topk(*layer, num_tokens, nullptr, 0, nullptr, nullptr, topk_ids, topk_w, logits, ws, wl, st);
  if (e == hipSuccess) e = run_experts(*layer, x, num_tokens, out, ws, wl, st, xq);
  return hip_rc(e);
}

int ftm_moe_forward_noalloc(const ftm_moe_layer* layer, const void* x, int32_t num_tokens, void* out,
                            int32_t* topk_ids, float* topk_w, float* logits, void* stream) {
  int rc = check_layer(layer, true);
  if (rc != FTM_OK) return rc;
  if (num_tokens < 0) return FTM_ERR_DIM;
  if (num_tokens == 0) return FTM_OK;
  if (x == nullptr || out == nullptr) return FTM_ERR_NULL;
  if (!aligned16(x)) return FTM_ERR_ALIGN;
  const size_t need = ws_layout(*layer, num_tokens).total;
  if (need > (size_t)FTM_NOALLOC_SCRATCH_BYTES) return FTM_ERR_WORKSPACE;
  void* ws = nullptr;
  rc = scratch_of_current_device(&ws);
  if (rc != FTM_OK) return rc;
  // The scratch keeps whatever the last call on this GPU left, on whichever
  // stream it ran, and a call that failed part way can leave its counters
  // set: each call clears the control region with a fill kernel on its own
  // stream first, so its kernels are ordered after that clear (a kernel, not a
  // memset, so the call can be captured in a HIP graph).
  if (launch_ws_init(ws, (hipStream_t)stream) != hipSuccess) return FTM_ERR_HIP;
  return ftm_moe_forward(layer, x, num_tokens, out, topk_ids, topk_w, logits, ws, need, stream);
}

int ftm_moe_forward_stage(const ftm_moe_layer* layer, const void* x, int32_t num_tokens, void* out, int32_t stage,
                          void* workspace, size_t ws_bytes, void* stream) {
  int rc = check_layer(layer, true);
  if (rc != FTM_OK) return rc;
  if (stage < FTM_STAGE_ROUTER || stage > FTM_STAGE_COMBINE) return FTM_ERR_DIM;
  if (num_tokens < 0) return FTM_ERR_DIM;
  if (num_tokens == 0) return FTM_OK;
  if (x == nullptr || out == nullptr) return FTM_ERR_NULL;
  if (!aligned16(x)) return FTM_ERR_ALIGN;
  rc = check_ws(layer, num_tokens, workspace, ws_bytes);
  if (rc != FTM_OK) return rc;
  if (!fast_layer(layer, x)) return FTM_ERR_FORMAT;  // stages exist for the MFMA path only
  const WsLayout wl = ws_layout(*layer, num_tokens);
  hipStream_t st = (hipStream_t)stream;
  char* ws = (char*)workspace;
  hipError_t e = hipSuccess;
  const bool fused = route_a_ok(*layer, num_tokens);  // routing runs in stage A
  const bool rt = !fused && route_topk_fused(*layer, num_tokens);  // the router launch also routes
  const RouteOut ro = {nullptr, nullptr, nullptr};
  // the router stage quantises the input of an MXFP4 stage A, as ftm_moe_forward's router launch does
  if (stage == FTM_STAGE_ROUTER)
    e = rt ? launch_route_topk(*layer, x, num_tokens, nullptr, nullptr, nullptr, ws, wl, st, true)
           : launch_router(*layer, x, num_tokens, 0, layer->num_experts + (layer->shared_inter > 0 ? 1 : 0), ws, wl,
                           st, true);
  else if (stage == FTM_STAGE_TOPK)
    e = fused || rt
            ? hipSuccess
            : launch_topk(*layer, num_tokens, nullptr, 0, nullptr, nullptr, nullptr, nullptr, nullptr, ws, wl, st);
  else
    e = launch_experts(*layer, x, num_tokens, out, ws, wl, st,
                       stage == FTM_STAGE_W13 ? 1 : stage == FTM_STAGE_W2 ? 2 : 4, fused ? &ro : nullptr,
                       mx_input(*layer, num_tokens));
  return hip_rc(e);
}

const char* ftm_moe_stage_kernel(const ftm_moe_layer* layer, int32_t num_tokens, int32_t stage) {
  if (check_layer(layer, true) != FTM_OK || num_tokens <= 0) return nullptr;
  // x only matters for its alignment, which the caller guarantees when it launches
  if (!fast_layer(layer, reinterpret_cast<const void*>(uintptr_t{256}))) return nullptr;
  return stage_kernel_name(*layer, num_tokens, stage);
}

int ftm_moe_forward_routed(const ftm_moe_layer* layer, const void* x, int32_t num_tokens,
                           const int32_t* topk_ids, const float* topk_w, void* out, void* workspace,
                           size_t ws_bytes, void* stream) {
  int rc = check_layer(layer, false);
  if (rc != FTM_OK) return rc;
  if (num_tokens < 0) return FTM_ERR_DIM;
  if (num_tokens == 0) return FTM_OK;
  if (x == nullptr || out == nullptr || topk_ids == nullptr || topk_w == nullptr) return FTM_ERR_NULL;
  rc = check_ws(layer, num_tokens, workspace, ws_bytes);
  if (rc != FTM_OK) return rc;
  const WsLayout wl = ws_layout(*layer, num_tokens);
  hipStream_t st = (hipStream_t)stream;
  char* ws = (char*)workspace;
  hipError_t e = hipSuccess;
  if (layer->shared_inter > 0) {
    if (layer->act_dtype != FTM_DT_BF16) return FTM_ERR_FORMAT;
    e = launch_router(*layer, x, num_tokens, layer->num_experts, layer->num_experts + 1, ws, wl, st);
  }
  if (e == hipSuccess)
    e = launch_topk(*layer, num_tokens, nullptr, 0, topk_ids, topk_w, nullptr, nullptr, nullptr, ws, wl, st);
  if (e == hipSuccess) e = run_experts(*layer, x, num_tokens, out, ws, wl, st);
  return hip_rc(e);
}

int ftm_route(const ftm_moe_layer* layer, const void* x, int32_t num_tokens, const void* logits_in,
              int32_t logits_dtype, float* logits_out, int32_t* topk_ids, float* topk_w, void* workspace,
              size_t ws_bytes, void* stream) {
  if (layer == nullptr) return FTM_ERR_NULL;
  const int E = layer->num_experts, k = layer->topk;
  if (E <= 0 || E > kMaxExperts || k <= 0 || k > E || k > 64) return FTM_ERR_DIM;
  if (layer->route_mode < FTM_ROUTE_SOFTMAX_TOPK || layer->route_mode > FTM_ROUTE_TOPK_SOFTMAX)
    return FTM_ERR_FORMAT;
  if (layer->act_dtype != FTM_DT_BF16 && layer->act_dtype != FTM_DT_F32) return FTM_ERR_FORMAT;
  if (num_tokens < 0) return FTM_ERR_DIM;
  if (num_tokens == 0) return FTM_OK;
  if (logits_in == nullptr) {
    if (layer->gate_w == nullptr || x == nullptr) return FTM_ERR_NULL;
    if (layer->act_dtype != FTM_DT_BF16) return FTM_ERR_FORMAT;
    if (layer->hidden <= 0 || layer->hidden % 8 != 0) return FTM_ERR_DIM;
    if (!aligned16(x) || !aligned16(layer->gate_w)) return FTM_ERR_ALIGN;
  } else if (!dt_ok(logits_dtype)) {
    return FTM_ERR_FORMAT;
  }
  if (topk_ids == nullptr || topk_w == nullptr) return FTM_ERR_NULL;
  int rc = check_ws(layer, num_tokens, workspace, ws_bytes);
  if (rc != FTM_OK) return rc;
  // Routing only: no shared expert bookkeeping.
  ftm_moe_layer L = *layer;
  L.shared_inter = 0;
  const WsLayout wl = ws_layout(L, num_tokens);
  hipStream_t st = (hipStream_t)stream;
  char* ws = (char*)workspace;
  hipError_t e = hipSuccess;
  if (logits_in == nullptr) e = launch_router(L, x, num_tokens, 0, E, ws, wl, st);
  if (e == hipSuccess)
    e = launch_topk(L, num_tokens, logits_in, logits_dtype, nullptr, nullptr, topk_ids, topk_w, logits_out, ws,
                    wl, st);
  return hip_rc(e);
}

int ftm_linear(const ftm_proj* proj, int32_t slot, const void* x, int32_t x_dtype, int32_t M, void* out,
               int32_t out_dtype, const void* bias, int32_t bias_dtype, int32_t final_dtype, void* stream) {
  int rc = check_proj_dequant(proj);
  if (rc != FTM_OK) return rc;
  if (slot < 0 || slot >= proj->num_slots) return FTM_ERR_DIM;
  if (!dt_ok(x_dtype) || !dt_ok(out_dtype) || !dt_ok(final_dtype)) return FTM_ERR_FORMAT;
  if (bias != nullptr && !dt_ok(bias_dtype)) return FTM_ERR_FORMAT;
  if (M < 0) return FTM_ERR_DIM;
  if (M == 0) return FTM_OK;
  if (x == nullptr || out == nullptr) return FTM_ERR_NULL;
  hipStream_t st = (hipStream_t)stream;
  if (check_proj(proj) == FTM_OK && aligned16(x))
    return hip_rc(launch_linear(*proj, slot, x, x_dtype, M, out, out_dtype, bias, bias_dtype, final_dtype, st));
  return hip_rc(launch_linear_generic(*proj, slot, x, x_dtype, M, out, out_dtype, bias, bias_dtype, final_dtype, st));
}

int ftm_expert_forward(const ftm_moe_layer* layer, int32_t slot, const void* x, int32_t M, void* out,
                       void* workspace, size_t ws_bytes, void* stream) {
  if (layer == nullptr) return FTM_ERR_NULL;
  ftm_moe_layer L = *layer;
  L.num_experts = 1;
  L.topk = 1;
  L.shared_inter = 0;
  L.gate_w = nullptr;
  L.gate_b = nullptr;
  L.apply_router_weight_on_input = 0;
  L.route_mode = FTM_ROUTE_SOFTMAX_TOPK;
  int rc = check_layer(&L, false);
  if (rc != FTM_OK) return rc;
  if (slot < 0 || slot >= layer->w13.num_slots || slot >= layer->w2.num_slots) return FTM_ERR_DIM;
  if (M < 0) return FTM_ERR_DIM;
  if (M == 0) return FTM_OK;
  if (x == nullptr || out == nullptr) return FTM_ERR_NULL;
  rc = check_ws(&L, M, workspace, ws_bytes);
  if (rc != FTM_OK) return rc;
  const WsLayout wl = ws_layout(L, M);
  char* ws = (char*)workspace;
  int32_t* slot_word = (int32_t*)(ws + wl.misc);
  int32_t* ids = (int32_t*)(ws + wl.logits);  // logits region: 4*M*(1+1) bytes
  float* w = (float*)(ws + wl.logits) + M;
  L.slot_of_expert = slot_word;
  hipStream_t st = (hipStream_t)stream;
  hipError_t e = launch_fill_routing(M, slot, slot_word, ids, w, st);
  if (e == hipSuccess) e = launch_topk(L, M, nullptr, 0, ids, w, nullptr, nullptr, nullptr, ws, wl, st);
  if (e == hipSuccess) e = run_experts(L, x, M, out, ws, wl, st);
  return hip_rc(e);
}

int ftm_dequant(const ftm_proj* proj, int32_t slot, void* out, int32_t out_dtype, int32_t transpose_out,
                void* stream) {
  int rc = check_proj_dequant(proj);
  if (rc != FTM_OK) return rc;
  if (slot < 0 || slot >= proj->num_slots) return FTM_ERR_DIM;
  if (!dt_ok(out_dtype)) return FTM_ERR_FORMAT;
  if (out == nullptr) return FTM_ERR_NULL;
  return hip_rc(launch_dequant(*proj, slot, out, out_dtype, transpose_out ? 1 : 0, (hipStream_t)stream));
}

int ftm_copy_slots(void* dev_pool, const void* host_bank, int64_t row_bytes, const int32_t* evict_slots,
                   const int32_t* src_rows, int32_t n, void* stream, void* done_event) {
  if (n < 0 || row_bytes <= 0) return FTM_ERR_DIM;
  if (n > 0 && (dev_pool == nullptr || host_bank == nullptr || evict_slots == nullptr || src_rows == nullptr))
    return FTM_ERR_NULL;
  for (int i = 0; i < n; ++i)
    if (evict_slots[i] < 0 || src_rows[i] < 0) return FTM_ERR_DIM;
  hipStream_t st = (hipStream_t)stream;
  // Coalesce runs where both the slot and the host row advance by one.
  int i = 0;
  while (i < n) {
    int j = i + 1;
    while (j < n && evict_slots[j] == evict_slots[j - 1] + 1 && src_rows[j] == src_rows[j - 1] + 1) ++j;
    const size_t bytes = (size_t)(j - i) * (size_t)row_bytes;
    char* dst = (char*)dev_pool + (size_t)evict_slots[i] * (size_t)row_bytes;
    const char* src = (const char*)host_bank + (size_t)src_rows[i] * (size_t)row_bytes;
    if (hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, st) != hipSuccess) return FTM_ERR_HIP;
    i = j;
  }
  if (done_event != nullptr && hipEventRecord((hipEvent_t)done_event, st) != hipSuccess) return FTM_ERR_HIP;
  return FTM_OK;
}

}  // extern "C"
