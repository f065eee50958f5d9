/*
 * ftmoe.h -- C ABI of the MI355X (gfx950) fused quantized MoE expert layer.
 *
 * Every entry point is `extern "C"`, takes plain pointers and sizes, and never
 * allocates device memory: the caller owns every buffer (weights, activations,
 * outputs, workspace) and passes the HIP stream the work is enqueued on as an
 * opaque `void*` (a `hipStream_t`; NULL = the null stream).  All device
 * pointers must stay valid until the stream reaches the enqueued work.
 *
 * Return codes follow the reference's CPU MoE ABI convention
 * (python/freetoken/kernel/csrc/cpu_moe/cpu_moe.cpp:733-739: -1 null pointer,
 * -2 bad dimensions; :638-650: -100 unknown handle) and extend it with -3..-6.
 *
 * Layouts (all row-major, "slot" = one expert's bank row in a [S, ...] pool):
 *   FTM_FMT_BF16        w: bf16 [N, K]
 *   FTM_FMT_FP32        w: f32  [N, K]
 *   FTM_FMT_FP8_BLOCK   w: e4m3fn bytes [N, K]; s: [ceil(N/B), ceil(K/B)] (B = group)
 *                       python/freetoken/kernel/triton/fp8_block_linear.py:48-91
 *   FTM_FMT_FP8_E5M2_BLOCK  the same with e5m2 bytes (fused_fp8_linear.py:123 accepts
 *                       torch.float8_e5m2 weights); runs on the generic GPU kernels
 *   FTM_FMT_GPTQ_INT4   w: int32 qweight [K/8, N] (8 nibbles along K, LSB first);
 *                       z: int32 qzeros [K/group, N/8]; s: scales [K/group, N]
 *                       python/freetoken/kernel/triton/gptq_linear.py:39-124
 *   FTM_FMT_INT8_PACKED w: int32 [N, K/4] (4 offset-binary bytes along K, +128);
 *                       s: [N, K/group]
 *                       python/freetoken/kernel/triton/int8_packed_linear.py:74-125
 *   FTM_FMT_MXFP4       w: uint8 blocks [N, K/32, 16] (low nibble = even element);
 *                       s: uint8 e8m0 [N, K/32]
 *                       python/freetoken/kernel/triton/mxfp4_linear.py:38-76
 */
#ifndef FTMOE_H
#define FTMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FTM_ABI_VERSION 1

/* ---- return codes ---- */
#define FTM_OK 0
#define FTM_ERR_NULL (-1)       /* a required pointer is NULL */
#define FTM_ERR_DIM (-2)        /* a dimension is out of range or inconsistent */
#define FTM_ERR_FORMAT (-3)     /* unsupported format / dtype / mode combination */
#define FTM_ERR_HIP (-4)        /* a HIP runtime call failed */
#define FTM_ERR_WORKSPACE (-5)  /* workspace missing or smaller than required */
#define FTM_ERR_ALIGN (-6)      /* a pointer or stride violates the alignment contract */
#define FTM_ERR_HANDLE (-100)   /* unknown handle */

/* ---- weight formats (bank schemas of python/freetoken/moe/offload_cache.py:140-173) ---- */
#define FTM_FMT_BF16 0
#define FTM_FMT_FP8_BLOCK 1
#define FTM_FMT_GPTQ_INT4 2
#define FTM_FMT_INT8_PACKED 3
#define FTM_FMT_MXFP4 4
#define FTM_FMT_FP32 5
#define FTM_FMT_FP8_E5M2_BLOCK 6

/* ---- scalar dtypes (activations, scales, outputs, biases) ---- */
#define FTM_DT_F32 0
#define FTM_DT_F16 1
#define FTM_DT_BF16 2

/* ---- routing modes ---- */
/* fp32 softmax over all E, top-k on it, optional renorm, weights rounded to the
 * activation dtype: python/freetoken/models/qwen3_5_moe/__init__.py:1224-1227 */
#define FTM_ROUTE_SOFTMAX_TOPK 0
/* softmax kept in the logits' dtype before top-k (bf16 probabilities), renorm in
 * that dtype: python/freetoken/kernel/triton/fused_moe.py:91-97,
 * python/freetoken/models/qwen3_moe/__init__.py:472-475 */
#define FTM_ROUTE_SOFTMAX_TOPK_LOWP 1
/* top-k on the (biased) logits, then fp32 softmax over the k selected values:
 * python/freetoken/models/gpt_oss/__init__.py:347-352 */
#define FTM_ROUTE_TOPK_SOFTMAX 2

/* ---- expert activations (python/freetoken/kernel/triton/fused_moe.py:53-61) ---- */
#define FTM_ACT_SILU 0
#define FTM_ACT_GELU 1
#define FTM_ACT_RELU 2
/* gpt-oss clamped GLU: g=min(g,L); u=clamp(u,-L,L); h=(u+1)*g*sigmoid(alpha*g)
 * python/freetoken/models/gpt_oss/__init__.py:306-310 */
#define FTM_ACT_SWIGLU_OAI 3

/* One projection bank: logical weight [N, K] per slot, `num_slots` slots. */
typedef struct ftm_proj {
  const void* w;        /* packed weights of slot 0 (layout per format, above) */
  const void* s;        /* scales of slot 0 (NULL for BF16/FP32) */
  const void* z;        /* GPTQ qzeros of slot 0, else NULL */
  const void* bias;     /* per-slot bias [N] in bias_dtype, or NULL */
  int64_t w_stride;     /* bytes between consecutive slots of w */
  int64_t s_stride;     /* bytes between consecutive slots of s */
  int64_t z_stride;     /* bytes between consecutive slots of z */
  int64_t bias_stride;  /* bytes between consecutive slots of bias */
  int32_t fmt;          /* FTM_FMT_* */
  int32_t s_dtype;      /* FTM_DT_* of s (FP8/GPTQ/INT8); ignored otherwise */
  int32_t bias_dtype;   /* FTM_DT_* of bias */
  int32_t group;        /* FP8 block edge; GPTQ group_size; INT8 K/num_groups; MXFP4 32 */
  int32_t N;            /* out features */
  int32_t K;            /* in features */
  int32_t num_slots;    /* slots in the pool (bounds check for slot ids) */
  int32_t flags;        /* 0, or FTM_PROJ_* below */
} ftm_proj;

/* ftm_proj.flags.  FTM_PROJ_RING_B, on w2: FP8 stage B above the token
 * crossover runs on the ring tile (k_gemm_mx) even where the register-fed
 * tile (k_gemm_mxb_f8) would; both compute the same products, block scales
 * and epilogue in the same order, and tests compare their outputs bitwise. */
#define FTM_PROJ_RING_B 1

/* One MoE layer: routed banks (w13 = gate||up [2I, H], w2 = down [H, I]),
 * router, activation and an optional always-on dense bf16 shared expert. */
typedef struct ftm_moe_layer {
  ftm_proj w13;                 /* N = 2*inter, K = hidden; rows [0,I) gate, [I,2I) up */
  ftm_proj w2;                  /* N = hidden, K = inter */
  const int32_t* slot_of_expert;/* device [E]: slot holding expert e, or NULL = identity */
  const void* gate_w;           /* router weight, bf16 [E, H] (NULL when routing is given) */
  const void* gate_b;           /* router bias, bf16 [E], or NULL */
  const void* shared_w13;       /* bf16 [2*shared_inter, H] or NULL */
  const void* shared_w2;        /* bf16 [H, shared_inter] or NULL */
  const void* shared_gate;      /* bf16 [1, H]: out += sigmoid(x.g) * shared(x) */
  int32_t num_experts;          /* E */
  int32_t hidden;               /* H */
  int32_t inter;                /* I */
  int32_t topk;                 /* k */
  int32_t shared_inter;         /* 0 = no shared expert */
  int32_t route_mode;           /* FTM_ROUTE_* */
  int32_t renormalize;          /* divide the k weights by their sum */
  int32_t act;                  /* FTM_ACT_* */
  float swiglu_alpha;           /* FTM_ACT_SWIGLU_OAI alpha (1.702) */
  float swiglu_limit;           /* FTM_ACT_SWIGLU_OAI clamp limit (7.0) */
  int32_t apply_router_weight_on_input; /* scale x by the router weight instead of y */
  int32_t act_dtype;            /* FTM_DT_BF16 or FTM_DT_F32: x, h and out dtype */
  int32_t h_dtype;              /* FTM_DT_*: h is rounded to it before w2 (then held in
                                   act_dtype); FTM_DT_F32 = no extra rounding;
                                   FTM_DT_F16 needs act_dtype FTM_DT_F32.  The
                                   reference rounds h to out_dtype
                                   (python/freetoken/kernel/triton/fused_fp8_linear.py:172-175) */
} ftm_moe_layer;

/* ABI version (FTM_ABI_VERSION). Never fails. */
int ftm_version(void);

/* Device workspace bytes ftm_moe_forward / ftm_moe_forward_routed / ftm_route
 * need for `num_tokens` tokens.  The first FTM_WS_CTRL_BYTES of a workspace
 * must be zero before its first use (ftm_workspace_init does that); every call
 * leaves them zero again, except the sticky error word (int32 at byte
 * FTM_WS_ERROR_OFFSET), whose bits the kernels OR in and the caller reads and
 * clears: FTM_WS_ERR_SLOT a routed expert had no resident slot (it contributed
 * zeros: the reference raises IndexError on such a stale slot,
 * python/freetoken/models/qwen3_5_moe/__init__.py:1676-1685), FTM_WS_ERR_ID an
 * expert id >= E (the pair contributed zeros), FTM_WS_ERR_LIST more than T pairs
 * for one expert (the pair was dropped).  Replaces the per-call host buffers of
 * python/freetoken/moe/offload_cache.py:560-674 and fused_moe.py:106-161. */
#define FTM_WS_CTRL_BYTES 4096
#define FTM_WS_ERROR_OFFSET 12
#define FTM_WS_ERR_SLOT 1
#define FTM_WS_ERR_ID 2
#define FTM_WS_ERR_LIST 4
size_t ftm_moe_workspace_bytes(const ftm_moe_layer* layer, int32_t num_tokens);
int ftm_workspace_init(void* workspace, size_t ws_bytes, void* stream);

/* Whole MoE layer: router GEMV -> softmax/top-k -> token->expert grouping ->
 * w13 + activation -> w2 + router-weighted deterministic combine (+ shared).
 * Replaces _Qwen35MoE.forward (python/freetoken/models/qwen3_5_moe/__init__.py:
 * 1221-1252) routed through _forward_offload_core (:1609-1749), and
 * _GptOssMoE.forward (python/freetoken/models/gpt_oss/__init__.py:347-365).
 *   x          [T, H] act_dtype            out [T, H] act_dtype
 *   topk_ids   optional int32 [T, k] output (selection order: descending)
 *   topk_w     optional f32 [T, k] output (router weights as used)
 *   logits     optional f32 [T, E] output (router logits, act_dtype-rounded) */
int ftm_moe_forward(const ftm_moe_layer* layer, const void* x, int32_t num_tokens,
                    void* out, int32_t* topk_ids, float* topk_w, float* logits,
                    void* workspace, size_t ws_bytes, void* stream);

/* ftm_moe_forward without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  The
 * workspace is a static device array of FTM_NOALLOC_SCRATCH_BYTES per GPU (the
 * library's own, held until the process ends; FTM_ERR_WORKSPACE when the layer
 * needs more at num_tokens: ftm_moe_workspace_bytes tells); the call allocates
 * nothing.  Each call first clears the array's control region with a small
 * fill kernel on `stream` (one launch more than ftm_moe_forward), so a call on
 * any stream, or after a failed call, starts from a cleared region.  Every call
 * on one GPU shares that array: calls that overlap on one GPU (several streams
 * or host threads) race.  Its sticky error word is not readable here: use
 * ftm_moe_forward with a workspace to check it.  Same kernels and result as
 * ftm_moe_forward. */
#define FTM_NOALLOC_SCRATCH_BYTES (16u << 20)
int ftm_moe_forward_noalloc(const ftm_moe_layer* layer, const void* x, int32_t num_tokens,
                            void* out, int32_t* topk_ids, float* topk_w, float* logits,
                            void* stream);

/* One stage of ftm_moe_forward, for per-kernel timing with events on `stream`:
 *   0 = router GEMV, 1 = softmax/top-k/grouping, 2 = w13 + activation,
 *   3 = w2 (router-weighted slots), 4 = combine of the slots into `out`.
 * Calling stages 0..4 in order on one stream launches exactly the kernels
 * ftm_moe_forward launches. */
#define FTM_STAGE_ROUTER 0
#define FTM_STAGE_TOPK 1
#define FTM_STAGE_W13 2
#define FTM_STAGE_W2 3
#define FTM_STAGE_COMBINE 4
int ftm_moe_forward_stage(const ftm_moe_layer* layer, const void* x, int32_t num_tokens, void* out,
                          int32_t stage, void* workspace, size_t ws_bytes, void* stream);

/* Base name (no namespace or template arguments) of the kernel that stage
 * `stage` of ftm_moe_forward launches for this layer at `num_tokens` tokens,
 * as a static string; NULL when the layer is invalid, takes the generic path
 * (which has no stages) or `stage` is out of range.  Touches no device state.
 * No counterpart in the reference: it names what ftm_moe_forward_stage runs,
 * for profilers and benchmarks that attribute time by kernel name. */
const char* ftm_moe_stage_kernel(const ftm_moe_layer* layer, int32_t num_tokens, int32_t stage);

/* Routed experts (+ shared expert if the layer has one) with routing supplied
 * by the caller: the grouped replacement of the per-(token, expert) loop in
 * python/freetoken/models/qwen3_5_moe/__init__.py:1732-1737 and of
 * fused_moe's per-expert loop (python/freetoken/kernel/triton/fused_moe.py:129-161).
 *   topk_ids int32 [T, k] expert ids; topk_w f32 [T, k] router weights.
 * An id < 0 marks a pair with no expert in this call: it contributes nothing
 * and raises no error (the padding an expert-parallel shard or a slot pool
 * smaller than the routed set uses; the reference has no such case). */
int ftm_moe_forward_routed(const ftm_moe_layer* layer, const void* x, int32_t num_tokens,
                           const int32_t* topk_ids, const float* topk_w, void* out,
                           void* workspace, size_t ws_bytes, void* stream);

/* Router only: logits (from x and layer->gate_w, or taken from `logits_in` of
 * dtype `logits_dtype` when gate_w is NULL), then the layer's route_mode
 * softmax/top-k.  Matches fused_moe's routing (fused_moe.py:91-97) and the
 * model routers (qwen3_5_moe/__init__.py:1224-1227, gpt_oss/__init__.py:347-352). */
int ftm_route(const ftm_moe_layer* layer, const void* x, int32_t num_tokens,
              const void* logits_in, int32_t logits_dtype, float* logits_out,
              int32_t* topk_ids, float* topk_w, void* workspace, size_t ws_bytes,
              void* stream);

/* One quantized projection: out[M, N] = cast(x[M, K] @ deq(W[slot]).T) (+ bias),
 * fp32 accumulation, weights never materialised densely.  Replaces
 * fused_{fp8,gptq,int8,mxfp4}_linear (python/freetoken/kernel/triton/
 * fused_fp8_linear.py:95-151, gptq_fused_linear.py:131-196,
 * fused_int8_linear.py:109-173, fused_mxfp4_linear.py:129-188).
 * `out` holds round(acc, out_dtype) (+ bias in fp32, rounded to final_dtype). */
int ftm_linear(const ftm_proj* proj, int32_t slot, const void* x, int32_t x_dtype,
               int32_t M, void* out, int32_t out_dtype, const void* bias,
               int32_t bias_dtype, int32_t final_dtype, void* stream);

/* One expert's SwiGLU forward against packed banks:
 * down(act(gate(x)) * up(x)), h rounded to out_dtype between the projections.
 * Replaces fused_*_expert_forward (e.g. fused_fp8_linear.py:154-175) and
 * SlotWeightAccessor.expert_forward (python/freetoken/moe/offload_cache.py:926-996). */
int ftm_expert_forward(const ftm_moe_layer* layer, int32_t slot, const void* x,
                       int32_t M, void* out, void* workspace, size_t ws_bytes,
                       void* stream);

/* Dequantize one slot of a projection to a dense [N, K] (or [K, N] when
 * transpose_out) tensor of out_dtype, bit-exact with the reference formulas
 * (fp32 product, then one round-to-nearest-even).  Replaces dequantize_block_fp8
 * (fp8_block_linear.py:48-91), dequantize_gptq_int4_sequential_groups
 * (gptq_linear.py:102-124, whose natural output is [K, N]: pass transpose_out=1),
 * dequantize_int8_packed (int8_packed_linear.py:96-125) and
 * dequantize_mxfp4_blocks (mxfp4_linear.py:46-76). */
int ftm_dequant(const ftm_proj* proj, int32_t slot, void* out, int32_t out_dtype,
                int32_t transpose_out, void* stream);

/* ---- offload slot pool (python/freetoken/moe/offload_cache.py:218-694) ---- */

/* Host-side global timestamp LRU over num_layers*E expert ids and S slots.
 * Mirrors OffloadMoeCache.ensure_experts (offload_cache.py:560-647): hits
 * stamp usage=step; misses (in ascending expert order) evict
 * argmin(usage, slot).  All arrays are host memory owned by the caller:
 *   slot_for_id [L*E] int32, id_of_slot [S] int32, usage [S] int64,
 *   step (in/out) int64, evict_slots / src_rows [max(E,S)] int32 (out),
 *   num_staged (out).  expert_ids [n] routed expert ids (duplicates allowed).
 * Returns the number of misses (>= 0) or a negative error code. */
int ftm_lru_ensure(int32_t layer_id, int32_t num_layers, int32_t num_experts,
                   int32_t cache_size, const int64_t* expert_ids, int32_t n,
                   int32_t* slot_for_id, int32_t* id_of_slot, int64_t* usage,
                   int64_t* step, int32_t* evict_slots, int32_t* src_rows,
                   int32_t* num_staged);

/* Whole-layer variant for prefill (OffloadMoeCache.materialize_layer,
 * offload_cache.py:461-556): every expert of the layer becomes resident;
 * misses take a free slot (lowest id_of_slot == -1) or the LRU victim. */
int ftm_lru_materialize(int32_t layer_id, int32_t num_layers, int32_t num_experts,
                        int32_t cache_size, int32_t* slot_for_id, int32_t* id_of_slot,
                        int64_t* usage, int64_t* step, int32_t* evict_slots,
                        int32_t* src_rows, int32_t* num_staged);

/* Enqueue the staged copies: for i < n, bytes [src_rows[i]*row_bytes, +row_bytes)
 * of `host_bank` (pinned host memory) -> [evict_slots[i]*row_bytes, +row_bytes)
 * of `dev_pool`, on `stream` (a side stream), then record `done_event` (a
 * hipEvent_t, may be NULL) on it.  Replaces OffloadMoeCache.copy_missing
 * (offload_cache.py:651-674).  Host arrays; the copies are asynchronous. */
int ftm_copy_slots(void* dev_pool, const void* host_bank, int64_t row_bytes,
                   const int32_t* evict_slots, const int32_t* src_rows, int32_t n,
                   void* stream, void* done_event);

/* ---- the same LRU and copy engine on the GPU (no host round trip) ----
 * Upstream's device-side lru_ensure (described at offload_cache.py:14-30) and
 * the batched copy its port leaves as stubs (python/freetoken/kernel/sycl/
 * batch_memcpy.py:11-12, python/freetoken/kernel/sycl/index.py:11-12). */

/* ensure_experts (offload_cache.py:560-647) as one kernel on `stream` over
 * device-resident state: slot_for_id [L*E] int32, id_of_slot [S] int32,
 * usage [S] int64, step [1] int64, the plan evict_slots / src_rows [>= E]
 * int32 and num_staged [1] int32 (all device memory, updated in place; the
 * same values ftm_lru_ensure computes).  expert_ids [n] int32 device: the
 * routed ids of the step (ids < 0 are pairs without an expert; ids >= E set
 * status bit 1 and are ignored).  The call takes the routed experts of ranks
 * [chunk * chunk_cap, (chunk + 1) * chunk_cap) in ascending id; chunk 0
 * is always an LRU step (as a call with no routed expert is), a later chunk
 * past the last routed expert changes nothing (num_staged = 0).  ids_chunk [n] int32 (device, may
 * be NULL): each pair's id if its expert is in the chunk, else -1.  stats
 * [2] int64 (device, may be NULL): += misses, += 1 call.  status [1] int32
 * (device, may be NULL): error bits OR-ed in.  num_experts <= 512,
 * cache_size <= 2^21. */
int ftm_lru_ensure_dev(int32_t layer_id, int32_t num_layers, int32_t num_experts,
                       int32_t cache_size, const int32_t* expert_ids, int32_t n,
                       int32_t chunk, int32_t chunk_cap, int32_t* slot_for_id,
                       int32_t* id_of_slot, int64_t* usage, int64_t* step,
                       int32_t* evict_slots, int32_t* src_rows, int32_t* num_staged,
                       int32_t* ids_chunk, int64_t* stats, int32_t* status, void* stream);

/* One bank of a layer for ftm_copy_slots_dev: host_bank (pinned host memory,
 * rows of row_bytes) -> dev_pool (slot rows of row_bytes). */
typedef struct ftm_bank_copy {
  const void* host_bank;
  void* dev_pool;
  int64_t row_bytes;
} ftm_bank_copy;

/* copy_missing (offload_cache.py:651-674) as one kernel on `stream`: for i <
 * min(*num_staged, max_rows) (device values, as ftm_lru_ensure_dev leaves
 * them), row src_rows[i] of every bank -> slot evict_slots[i], read from the
 * pinned host banks by the kernel.  Plan entries outside [0, host_rows) /
 * [0, pool_slots) are skipped.  Up to 8 banks; a host bank that is not
 * pinned, mapped host memory returns FTM_ERR_HIP before anything is
 * launched. */
int ftm_copy_slots_dev(const ftm_bank_copy* banks, int32_t num_banks, int32_t host_rows,
                       int32_t pool_slots, const int32_t* evict_slots, const int32_t* src_rows,
                       const int32_t* num_staged, int32_t max_rows, void* stream);

/* ---- the host-CPU half of the hybrid CPU || GPU split ----
 * Routed experts of `layer` computed on the host cores from packed HOST banks
 * (every format the GPU kernels take, decoded per element as the reference
 * dequantizes: fp32 product, one rounding): fp32 gu, fp32 h = act(gate) * up
 * (+ the projection biases), fp32 down projection, out[t] += w[t, j] * y, for
 * the pairs whose expert has expert_mask[e] != 0 (expert_mask NULL = all).
 * x [T, H] f32, topk_ids [T, k] int32, topk_w [T, k] f32, out [T, H] f32
 * (overwritten).  Experts split into contiguous ranges over `threads` host
 * threads (0 = hardware concurrency clamped to E) with private partial sums.
 * The shared expert is not included.  Replaces freetoken_cpu_moe_forward_fast
 * (python/freetoken/kernel/csrc/cpu_moe/cpu_moe.cpp:470-528, 763-786), which
 * takes only dense fp32 / bf16 banks.  force_scalar: skip the AVX-512 path. */
int ftm_cpu_moe_forward(const ftm_moe_layer* layer, const float* x, int32_t num_tokens,
                        const int32_t* topk_ids, const float* topk_w, const uint8_t* expert_mask,
                        int32_t threads, int32_t force_scalar, float* out);

/* The same call on the library's persistent worker thread, one job at a time
 * (submit waits for the previous job to be collected): returns a handle > 0
 * (or a negative error code before anything runs); every pointer must stay
 * valid until ftm_cpu_moe_wait(handle) returns the call's code
 * (FTM_ERR_HANDLE for an unknown handle).  Replaces freetoken_cpu_moe_submit /
 * _wait (cpu_moe.cpp:596-706, 820-853). */
int64_t ftm_cpu_moe_submit(const ftm_moe_layer* layer, const float* x, int32_t num_tokens,
                           const int32_t* topk_ids, const float* topk_w, const uint8_t* expert_mask,
                           int32_t threads, float* out);
int ftm_cpu_moe_wait(int64_t handle);

/* 1 when the host CPU runs the AVX-512 path (freetoken_cpu_moe_avx512_available). */
int ftm_cpu_avx512(void);

#ifdef __cplusplus
}
#endif

#endif /* FTMOE_H */
