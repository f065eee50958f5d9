// ftm_gemm.hip -- the MoE expert stages above the token crossover: grouped,
// LDS-tiled GEMMs on bf16 MFMA (v_mfma_f32_16x16x32_bf16).
//
// Below the crossover every expert sees a handful of tokens and the stages are
// weight-streaming GEMVs (ftm_moe.hip).  Above it (prefill) each expert's
// weights are reused by many tokens, so a tile of 64 tokens x 64 channels
// loads its weights once per K step into LDS, decoded to bf16 exactly (FP8
// e4m3 and INT8 codes are exact in bf16, MXFP4 e2m1 times its power-of-two
// scale is exact), and four waves run 16x16x32 MFMAs out of LDS.  FP8 block
// and INT8 group scales multiply the fp32 partial sums of each quantisation
// group, as in the GEMV path, so both paths share one numerical contract.
//
// Tiles: the routed experts' token lists are cut into 64-row M tiles
// (ascending compact expert index u), then the shared expert's tokens.  Stage
// A (w13 + activation): a tile covers 64 channels, i.e. the 64 gate rows and
// the matching 64 up rows of w13, and writes h.  Stage B (w2): a tile covers
// 64 output columns and writes router-weighted fp32 rows into the slot buffer
// that k_combine reduces.
#include "ftm_layer.h"

namespace ftm {

constexpr int kGM = 64;            // tokens per tile
constexpr int kGK = 64;            // K per step
constexpr int kGPitch = kGK + 8;   // LDS row pitch in bf16 (144 B: rows do not share a bank period)
// Crossover, in average tokens per routed expert.  Measured on MI355X (C3 FP8
// and C4 MXFP4 layers): the tiles win from 16 on (C3 T=512: 466 us against
// 723 us on the GEMVs; C4 T=128: 360 us against 380 us) and lose at 8 and
// below (C4 T=64: 341 us against 236 us; C4 T=32: 333 us against 193 us).
constexpr int kGemmMinRows = 16;

// Weight bytes per element and 16-byte pieces per tile row per K step.
template <int WFMT>
struct GemmW {
  static constexpr int kPieces = WFMT == FTM_FMT_BF16 ? 8 : WFMT == FTM_FMT_MXFP4 ? 2 : 4;
  static constexpr int kElems = kGK / kPieces;  // elements per piece
  static constexpr bool kPostScale = WFMT == FTM_FMT_FP8_BLOCK || WFMT == FTM_FMT_INT8_PACKED;
  __device__ static uint32_t row_bytes(int K) {
    return WFMT == FTM_FMT_BF16 ? 2u * (uint32_t)K : WFMT == FTM_FMT_MXFP4 ? (uint32_t)K / 2 : (uint32_t)K;
  }
};

// M tile -> (compact expert u, first row, token count).  u == nRouted is the
// shared expert; u < 0: past the last tile.  Every lane of the calling wave
// gets the same answer (wave-uniform, no LDS).
struct GemmTile {
  int u, m0, cnt;
};

template <int MT = kGM>
__device__ __forceinline__ GemmTile gemm_find_tile(const LayerArgs& a, int mtile, int nRouted, bool shared) {
  const int lane = threadIdx.x & 63;
  // lane l owns compact experts 8l .. 8l+7 (E <= 512)
  const Rsrc cres = make_rsrc(a.ucnt, (uint32_t)(a.L.num_experts + 1) * 4u);
  int v[8], c[8];
  int lsum = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int u = 8 * lane + j;
    c[j] = u < nRouted ? (int)bload4(cres, 4u * (uint32_t)u) : 0;
    v[j] = (c[j] + MT - 1) / MT;
    lsum += v[j];
  }
  // exclusive prefix over lanes
  int incl = lsum;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int o = __shfl_up(incl, off);
    if (lane >= off) incl += o;
  }
  const int total = __shfl(incl, 63);
  GemmTile t = {-1, 0, 0};
  if (mtile < total) {
    int base = incl - lsum;
    int found_u = -1, found_m0 = 0, found_cnt = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (found_u < 0 && mtile >= base && mtile < base + v[j]) {
        found_u = 8 * lane + j;
        found_m0 = (mtile - base) * MT;
        found_cnt = c[j];
      }
      base += v[j];
    }
    const uint64_t who = __ballot(found_u >= 0);
    const int src = (int)__builtin_ctzll(who);
    t.u = __shfl(found_u, src);
    t.m0 = __shfl(found_m0, src);
    t.cnt = __shfl(found_cnt, src);
  } else if (shared) {
    const int st = mtile - total;
    if (st * MT < a.T) {
      t.u = nRouted;
      t.m0 = st * MT;
      t.cnt = a.T;
    }
  }
  return t;
}

// Routed M tiles (device total) for the item -> tile mapping of a stage whose
// routed part has ntn N tiles per M tile.
template <int MT = kGM>
__device__ __forceinline__ int gemm_routed_mtiles(const LayerArgs& a, int nRouted) {
  const int lane = threadIdx.x & 63;
  const Rsrc cres = make_rsrc(a.ucnt, (uint32_t)(a.L.num_experts + 1) * 4u);
  int lsum = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int u = 8 * lane + j;
    lsum += u < nRouted ? ((int)bload4(cres, 4u * (uint32_t)u) + MT - 1) / MT : 0;
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) lsum += __shfl_xor(lsum, off);
  return lsum;
}

// One 64-token x (NWR weight rows) tile over the whole K range.
//   WFMT: weight format; NWR = 128 (stage A: 64 gate + 64 up rows) or 64 (stage B)
//   grow(r): global weight row of tile row r
//   arow[i]: byte offset of the activation row of A piece i of this thread (kOOB = zero row)
//   acc[mi][nj]: wave (wm, wn) tile: tokens 32wm + 16mi, tile rows nrow(nj)
template <int WFMT, int NWR, int AXB>
struct GemmTileRun {
  static constexpr int NB = NWR == 128 ? 4 : 2;  // 16-column MFMA blocks per wave
  static constexpr int kWPieces = NWR * GemmW<WFMT>::kPieces;
  static constexpr int kWLoads = (kWPieces + kBlock - 1) / kBlock;

  // tile row of MFMA column block nj of wave column wn
  __device__ static int nrow(int nj, int wn) {
    if constexpr (NWR == 128) return nj < 2 ? 32 * wn + 16 * nj : 64 + 32 * wn + 16 * (nj - 2);
    return 32 * wn + 16 * nj;
  }
};

template <int WFMT, int NWR>
__device__ __forceinline__ void gemm_tile(const ProjSlot& W, int c0, int Iu, Rsrc ares, const uint32_t (&arow)[2],
                                          uint16_t* sA, uint16_t* sB, f32x4 (&acc)[2][NWR == 128 ? 4 : 2]) {
  using G = GemmW<WFMT>;
  using R = GemmTileRun<WFMT, NWR, 2>;
  constexpr int NB = R::NB;
  constexpr int kSA = kGM * kGPitch, kSB = NWR * kGPitch;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;
  const int K = W.K;
  const int nsteps = (K + kGK - 1) / kGK;
  auto grow = [&](int r) { return NWR == 128 ? (r < 64 ? c0 + r : Iu + c0 + (r - 64)) : c0 + r; };

  const uint32_t rb = G::row_bytes(K);
  const Rsrc wres = make_rsrc(W.w, rb * (uint32_t)W.N);
  uint32_t woff[R::kWLoads];
  int wtr[R::kWLoads], wpc[R::kWLoads];
#pragma unroll
  for (int i = 0; i < R::kWLoads; ++i) {
    const int c = tid + kBlock * i;
    wtr[i] = c / G::kPieces;
    wpc[i] = c % G::kPieces;
    const int r = grow(wtr[i]);
    woff[i] = (c < R::kWPieces && r < W.N) ? (uint32_t)r * rb + (uint32_t)wpc[i] * 16u : kOOB;
  }
  Rsrc sres = wres;  // MXFP4 e8m0 scales: one byte per (row, 32 elements)
  uint32_t moff[R::kWLoads];
  if constexpr (WFMT == FTM_FMT_MXFP4) {
    sres = make_rsrc(W.s, (uint32_t)W.N * (uint32_t)(K / 32));
#pragma unroll
    for (int i = 0; i < R::kWLoads; ++i) {
      const int r = grow(wtr[i]);
      moff[i] = woff[i] != kOOB ? (uint32_t)(r * (K / 32) + wpc[i]) : kOOB;
    }
  }
  // post-scale sources: FP8 block rows (uniform per column block), INT8 rows (per lane)
  const int lpg = G::kPostScale ? W.group / kGK : 1;
  int srow[NB];
#pragma unroll
  for (int nj = 0; nj < NB; ++nj) srow[nj] = grow(R::nrow(nj, wn));
  const uint32_t sesz = W.s_dt == FTM_DT_F32 ? 4u : 2u;
  Rsrc i8res = wres;
  if constexpr (WFMT == FTM_FMT_INT8_PACKED) i8res = make_rsrc(W.s, (uint32_t)(W.N * (K / W.group)) * sesz);

  u32x4 rw[R::kWLoads], ra[2];
  uint32_t rs[R::kWLoads];
  auto issue = [&](int kb) {
    const uint32_t kbyte = (uint32_t)kb * (uint32_t)(kGK * (WFMT == FTM_FMT_BF16 ? 2 : 1));
    const uint32_t kbw = WFMT == FTM_FMT_MXFP4 ? kbyte / 2 : kbyte;
#pragma unroll
    for (int i = 0; i < R::kWLoads; ++i) {
      rw[i] = bload16(wres, woff[i] != kOOB ? woff[i] + kbw : kOOB);
      if constexpr (WFMT == FTM_FMT_MXFP4) rs[i] = bload1(sres, moff[i] != kOOB ? moff[i] + (uint32_t)(2 * kb) : kOOB);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int piece = (tid + kBlock * i) & 7;
      ra[i] = bload16(ares, arow[i] != kOOB ? arow[i] + (uint32_t)(kb * kGK + piece * 8) * 2u : kOOB);
    }
  };
  auto stage = [&](int buf) {
    uint16_t* a_ = sA + buf * kSA;
    uint16_t* b_ = sB + buf * kSB;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int c = tid + kBlock * i;
      *(u32x4*)(a_ + (c >> 3) * kGPitch + (c & 7) * 8) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < R::kWLoads; ++i) {
      if (tid + kBlock * i >= R::kWPieces) continue;
      uint16_t* dst = b_ + wtr[i] * kGPitch + wpc[i] * G::kElems;
      if constexpr (WFMT == FTM_FMT_FP8_BLOCK) {
        *(u32x4*)dst = fp8x8_to_bf16(rw[i].x, rw[i].y);
        *(u32x4*)(dst + 8) = fp8x8_to_bf16(rw[i].z, rw[i].w);
      } else if constexpr (WFMT == FTM_FMT_INT8_PACKED) {
        *(u32x4*)dst = i8x8_to_bf16(rw[i].x, rw[i].y);
        *(u32x4*)(dst + 8) = i8x8_to_bf16(rw[i].z, rw[i].w);
      } else if constexpr (WFMT == FTM_FMT_MXFP4) {
        const float sc = e8m0_to_f32(rs[i]);
        *(u32x4*)dst = fp4x8_to_bf16(rw[i].x, sc);
        *(u32x4*)(dst + 8) = fp4x8_to_bf16(rw[i].y, sc);
        *(u32x4*)(dst + 16) = fp4x8_to_bf16(rw[i].z, sc);
        *(u32x4*)(dst + 24) = fp4x8_to_bf16(rw[i].w, sc);
      } else {
        *(u32x4*)dst = rw[i];
      }
    }
  };

  f32x4 tmp[2][NB];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int nj = 0; nj < NB; ++nj) tmp[mi][nj] = (f32x4){0.f, 0.f, 0.f, 0.f};

  issue(0);
  for (int kb = 0; kb < nsteps; ++kb) {
    const int buf = kb & 1;
    stage(buf);
    __syncthreads();
    if (kb + 1 < nsteps) issue(kb + 1);
    const uint16_t* a_ = sA + buf * kSA;
    const uint16_t* b_ = sB + buf * kSB;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int ko = ks * 32 + 8 * (lane >> 4);
      u32x4 af[2], bf[NB];
#pragma unroll
      for (int mi = 0; mi < 2; ++mi) af[mi] = *(const u32x4*)(a_ + (32 * wm + 16 * mi + (lane & 15)) * kGPitch + ko);
#pragma unroll
      for (int nj = 0; nj < NB; ++nj) bf[nj] = *(const u32x4*)(b_ + (R::nrow(nj, wn) + (lane & 15)) * kGPitch + ko);
#pragma unroll
      for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int nj = 0; nj < NB; ++nj) tmp[mi][nj] = mfma_bf16(af[mi], bf[nj], tmp[mi][nj]);
    }
    if constexpr (G::kPostScale) {
      // end of a quantisation group: acc += group partial * scale (straight-line)
      const bool last = ((kb + 1) % lpg == 0) | (kb + 1 == nsteps);
      const int grp = kb / lpg;
#pragma unroll
      for (int nj = 0; nj < NB; ++nj) {
        float s;
        if constexpr (WFMT == FTM_FMT_FP8_BLOCK) {
          const int nkb = (K + W.group - 1) / W.group;
          const uint32_t idx = (uint32_t)((srow[nj] / W.group) * nkb + grp);
          s = decode_scalar_word(sload4(W.s, (idx * sesz) & ~3u), idx, W.s_dt);
        } else {
          const uint32_t idx = (uint32_t)((srow[nj] + (lane & 15)) * (K / W.group) + grp);
          s = decode_scalar_word(bload_scalar_word(i8res, idx, W.s_dt, srow[nj] + (lane & 15) < W.N), idx, W.s_dt);
        }
        const float f = last ? s : 0.0f;
        const float keep = last ? 0.0f : 1.0f;
#pragma unroll
        for (int mi = 0; mi < 2; ++mi) {
          acc[mi][nj] += tmp[mi][nj] * f;
          tmp[mi][nj] *= keep;
        }
      }
    }
  }
  if constexpr (!G::kPostScale) {
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
      for (int nj = 0; nj < NB; ++nj) acc[mi][nj] += tmp[mi][nj];
  }
  __syncthreads();  // the LDS tiles are reused by the caller's next tile
}

// ---------------------------------------------------------------- LDS ring tiles (stage A)
// The stage A tiles for FP8 / INT8 / MXFP4 / bf16 weights, fed by a ring of up to
// four LDS stages that direct global-to-LDS copies (global_load_lds, 16 B per
// lane) fill three K steps ahead of the MFMAs.  Activations (bf16) and the raw
// weight bytes both land in LDS undecoded; a wave decodes its own weight rows
// after its LDS read.  Each 1 KiB copy writes 64 consecutive 16-byte slots, so
// the bank-conflict swizzle is applied on the read side of the copy: the lane
// filling slot s of row r fetches piece s ^ f(r) of that row, and a reader
// finds piece p of row r in slot p ^ f(r).  With f below, the rows one MFMA
// operand read touches (16 rows, one piece each) hit distinct 16-byte bank
// groups.  The tile's quantisation-group scales are copied to LDS once, before
// the K loop, so no scale load waits inside it.

// Raw weight bytes per row per K step and rows per 1 KiB copy.
template <int WFMT>
struct RingW {
  static constexpr int kRowBytes = WFMT == FTM_FMT_BF16 ? 2 * kGK : WFMT == FTM_FMT_MXFP4 ? kGK / 2 : kGK;
  static constexpr int kRowsPerCopy = 1024 / kRowBytes;
};
// Ring bytes per workgroup: 64 KiB (FP8/INT8: 4 stages, bf16: 2).  The
// tile's scales follow the ring (at most kRingScaleBytes; the launch sizes the
// dynamic LDS to what the layer needs).
constexpr int kRingA = 64 * 1024;
constexpr int kRingScaleBytes = 16 * 1024;

template <int WFMT, int NWR, int RB>
struct RingPlan {
  static constexpr int kA = kGM * 2 * kGK;  // 64 token rows x 64 bf16
  static constexpr int kW = NWR * RingW<WFMT>::kRowBytes;
  static constexpr int kStage = kA + kW;
  static constexpr int kStages = RB / kStage < 4 ? RB / kStage : 4;
  static constexpr int kALoads = kA / 1024 / 4;  // 1 KiB copies per wave per stage
  static constexpr int kWLoads = kW / 1024 / 4;
  static constexpr int kLoads = kALoads + kWLoads;
  static_assert(kStages >= 2 && kA % 4096 == 0 && kW % 4096 == 0, "ring shape");
};

__device__ __forceinline__ int ring_fa(int r) { return (r ^ (r >> 3)) & 7; }         // 8 pieces per row
__device__ __forceinline__ int ring_fw(int r) { return ((r >> 1) ^ (r >> 3)) & 3; }  // 4 pieces per row
__device__ __forceinline__ int ring_fm(int r) { return (r >> 3) & 1; }                // 2 pieces per row (MXFP4)

// Wait until at most `stages` ring stages of this wave's copies are in flight.
template <int LOADS, int MAXS>
__device__ __forceinline__ void wait_ring(int stages) {
  if (MAXS >= 3 && stages >= 3) wait_vm<3 * LOADS>();
  else if (MAXS >= 2 && stages == 2) wait_vm<2 * LOADS>();
  else if (stages == 1) wait_vm<LOADS>();
  else wait_vm<0>();
}

// One 64-token x NWR-row tile over the whole K range (FP8, INT8 or bf16
// weights).  Wave w owns tile rows 64 j + 16 w .. + 15 (j < NWR / 64: for
// stage A the gate rows and the matching up rows) for all 64 tokens, so each
// weight byte is decoded once.  LPG: K steps per quantisation group, the loop
// unrolled so the group partial is scaled once, straight after the group's
// last MFMAs (2: 128-wide groups); 0: no intermediate scaling (bf16, or one
// group over K); -1: any group size (scaled with selects every step).
//   arow[i]: activation row of this lane's slot in A copy i (always a valid row;
//            padding rows repeat a real one and their outputs are dropped)
//   acc[mi][j]: tokens 16 mi + 4 (lane / 16) + r, tile row 64 j + 16 w + lane % 16
template <int WFMT, int NWR, int RB, int LPG>
__device__ __forceinline__ void gemm_tile_ring(const ProjSlot& W, int c0, int Iu,
                                               const char* const (&arow)[RingPlan<WFMT, NWR, RB>::kALoads],
                                               char* lds, f32x4 (&acc)[4][NWR / 64]) {
  using P = RingPlan<WFMT, NWR, RB>;
  using RW = RingW<WFMT>;
  typedef __attribute__((address_space(1))) const void* GPtr;
  typedef __attribute__((address_space(3))) void* LPtr;
  constexpr int NB = NWR / 64;
  constexpr int S = P::kStages;
  constexpr bool kPost = WFMT == FTM_FMT_FP8_BLOCK || WFMT == FTM_FMT_INT8_PACKED;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int K = W.K;
  const int nsteps = K / kGK;
  auto grow = [&](int r) { return NWR == 128 ? (r < 64 ? c0 + r : Iu + c0 + (r - 64)) : c0 + r; };
  const uint32_t rb = GemmW<WFMT>::row_bytes(K);
  float* sS = (float*)(lds + RB);

  // ---- this lane's copy sources (K offset added per step)
  const char* asrc[P::kALoads];
#pragma unroll
  for (int i = 0; i < P::kALoads; ++i) {
    const int r = 8 * (wave * P::kALoads + i) + (lane >> 3);
    asrc[i] = arow[i] + 16 * ((lane & 7) ^ ring_fa(r));
  }
  const char* wsrc[P::kWLoads];
#pragma unroll
  for (int i = 0; i < P::kWLoads; ++i) {
    const int j = wave * P::kWLoads + i;
    int r, piece;
    if constexpr (WFMT == FTM_FMT_BF16) {
      r = 8 * j + (lane >> 3);
      piece = (lane & 7) ^ ring_fa(r);
    } else if constexpr (WFMT == FTM_FMT_MXFP4) {
      r = 32 * j + (lane >> 1);
      piece = (lane & 1) ^ ring_fm(r);
    } else {
      r = 16 * j + (lane >> 2);
      piece = (lane & 3) ^ ring_fw(r);
    }
    wsrc[i] = W.w + (size_t)grow(r) * rb + 16 * piece;
  }
  auto issue = [&](int kb, int slot) {
    char* st = lds + slot * P::kStage;
#pragma unroll
    for (int i = 0; i < P::kALoads; ++i)
      __builtin_amdgcn_global_load_lds((GPtr)(asrc[i] + kb * 2 * kGK),
                                       (LPtr)(st + 1024 * (wave * P::kALoads + i)), 16, 0, 0);
#pragma unroll
    for (int i = 0; i < P::kWLoads; ++i)
      __builtin_amdgcn_global_load_lds((GPtr)(wsrc[i] + kb * RW::kRowBytes),
                                       (LPtr)(st + P::kA + 1024 * (wave * P::kWLoads + i)), 16, 0, 0);
  };

  // ---- group scales of the tile -> LDS as fp32 (FP8: one row per 64-row
  // half, INT8: one row per tile row), loads issued before the ring prologue
  const int ngroups = kPost ? (K + W.group - 1) / W.group : 0;
  constexpr int kScaleRows = WFMT == FTM_FMT_INT8_PACKED ? NWR : NWR / 64;
  constexpr int kScalePer = WFMT == FTM_FMT_INT8_PACKED || WFMT == FTM_FMT_MXFP4
                                ? (kRingScaleBytes / 4 + kBlock - 1) / kBlock : 1;
  uint32_t sw[kScalePer];
  uint32_t sidx[kScalePer];
  // MXFP4: the e8m0 bytes [NWR rows][K / 32], copied as words; each 64-row
  // half of the tile is one contiguous run of 64 * K / 32 bytes
  const int kgb = K / 32;                 // scale bytes per row
  const int mwords = 64 * kgb / 4;        // words per 64-row half
  if constexpr (WFMT == FTM_FMT_MXFP4) {
    const Rsrc mres = make_rsrc(W.s, (uint32_t)W.N * (uint32_t)kgb);
#pragma unroll
    for (int q = 0; q < kScalePer; ++q) {
      const int e = tid + kBlock * q;
      const int half = e / mwords, wi = e - half * mwords;
      const bool ok = e < (NWR / 64) * mwords;
      sw[q] = bload4(mres, ok ? (uint32_t)(grow(64 * half) * kgb + 4 * wi) : kOOB);
    }
  }
  if constexpr (kPost) {
    const uint32_t sesz = W.s_dt == FTM_DT_F32 ? 4u : 2u;
    const int nsc = kScaleRows * ngroups;
    const Rsrc sres = make_rsrc(W.s, WFMT == FTM_FMT_FP8_BLOCK
                                         ? (uint32_t)(((W.N + W.group - 1) / W.group) * ngroups) * sesz
                                         : (uint32_t)(W.N * ngroups) * sesz);
#pragma unroll
    for (int q = 0; q < kScalePer; ++q) {
      const int e = tid + kBlock * q;
      const int sr = e / (ngroups > 0 ? ngroups : 1), g = e - sr * ngroups;
      const int wrow = WFMT == FTM_FMT_FP8_BLOCK ? grow(64 * sr) / W.group : grow(sr);
      sidx[q] = (uint32_t)(wrow * ngroups + g);
      sw[q] = bload_scalar_word(sres, sidx[q], W.s_dt, e < nsc);
    }
  }
  const int pro = nsteps < S - 1 ? nsteps : S - 1;
  for (int kb = 0; kb < pro; ++kb) issue(kb, kb);
  if constexpr (WFMT == FTM_FMT_MXFP4) {
    wait_ring<P::kLoads, S - 1>(pro);
#pragma unroll
    for (int q = 0; q < kScalePer; ++q) {
      const int e = tid + kBlock * q;
      if (e < (NWR / 64) * mwords) ((uint32_t*)sS)[e] = sw[q];
    }
  }
  if constexpr (kPost) {
    wait_ring<P::kLoads, S - 1>(pro);
#pragma unroll
    for (int q = 0; q < kScalePer; ++q) {
      const int e = tid + kBlock * q;
      if (e < kScaleRows * ngroups) sS[e] = decode_scalar_word(sw[q], sidx[q], W.s_dt);
    }
  }

  const int g4 = lane >> 4;
  int arr[4], wrr[NB];
#pragma unroll
  for (int mi = 0; mi < 4; ++mi) arr[mi] = 16 * mi + (lane & 15);
#pragma unroll
  for (int nj = 0; nj < NB; ++nj) wrr[nj] = 64 * nj + 16 * wave + (lane & 15);

  // one K step into d: wait for its stage, refill the ring, LDS -> MFMAs
  auto step = [&](int kb, f32x4 (&d)[4][NB]) {
    const int ahead = nsteps - 1 - kb < S - 2 ? nsteps - 1 - kb : S - 2;
    wait_ring<P::kLoads, S - 2>(ahead);
    __syncthreads();  // stage kb is in LDS for every wave; every wave is done with stage kb - 1
    if (kb + S - 1 < nsteps) issue(kb + S - 1, (kb + S - 1) % S);
    const char* st = lds + (kb % S) * P::kStage;
    u32x4 b0[NB], b1[NB];
#pragma unroll
    for (int nj = 0; nj < NB; ++nj) {
      const char* row = st + P::kA + wrr[nj] * RW::kRowBytes;
      if constexpr (WFMT == FTM_FMT_BF16) {
        b0[nj] = *(const u32x4*)(row + 16 * ((2 * g4) ^ ring_fa(wrr[nj])));
        b1[nj] = *(const u32x4*)(row + 16 * ((2 * g4 + 1) ^ ring_fa(wrr[nj])));
      } else if constexpr (WFMT == FTM_FMT_MXFP4) {
        // 16 e2m1 codes (K 16 g .. 16 g + 15), one 32-wide e8m0 group
        const u32x2 raw = *(const u32x2*)(row + 16 * ((g4 >> 1) ^ ring_fm(wrr[nj])) + 8 * (g4 & 1));
        const float sc = e8m0_to_f32(((const uint8_t*)sS)[wrr[nj] * kgb + 2 * kb + (g4 >> 1)]);
        b0[nj] = fp4x8_to_bf16(raw.x, sc);
        b1[nj] = fp4x8_to_bf16(raw.y, sc);
      } else {
        const u32x4 raw = *(const u32x4*)(row + 16 * (g4 ^ ring_fw(wrr[nj])));
        if constexpr (WFMT == FTM_FMT_FP8_BLOCK) {
          b0[nj] = fp8x8_to_bf16(raw.x, raw.y);
          b1[nj] = fp8x8_to_bf16(raw.z, raw.w);
        } else {
          b0[nj] = i8x8_to_bf16(raw.x, raw.y);
          b1[nj] = i8x8_to_bf16(raw.z, raw.w);
        }
      }
    }
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
      const char* row = st + arr[mi] * (2 * kGK);
      const u32x4 a0 = *(const u32x4*)(row + 16 * ((2 * g4) ^ ring_fa(arr[mi])));
      const u32x4 a1 = *(const u32x4*)(row + 16 * ((2 * g4 + 1) ^ ring_fa(arr[mi])));
#pragma unroll
      for (int nj = 0; nj < NB; ++nj) {
        d[mi][nj] = mfma_bf16(a0, b0[nj], d[mi][nj]);
        d[mi][nj] = mfma_bf16(a1, b1[nj], d[mi][nj]);
      }
    }
  };
  auto scale_of = [&](int nj, int grp) {
    return sS[(WFMT == FTM_FMT_FP8_BLOCK ? nj : wrr[nj]) * ngroups + grp];
  };

  if constexpr (!kPost) {
    for (int kb = 0; kb < nsteps; ++kb) step(kb, acc);
  } else {
    f32x4 tmp[4][NB];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int nj = 0; nj < NB; ++nj) tmp[mi][nj] = (f32x4){0.f, 0.f, 0.f, 0.f};
    if constexpr (LPG > 0) {
      // nsteps % LPG == 0 (checked at launch): whole groups per iteration
      for (int kb = 0, grp = 0; kb < nsteps; kb += LPG, ++grp) {
#pragma unroll
        for (int q = 0; q < LPG; ++q) step(kb + q, tmp);
#pragma unroll
        for (int nj = 0; nj < NB; ++nj) {
          const float sc = scale_of(nj, grp);
#pragma unroll
          for (int mi = 0; mi < 4; ++mi) {
            acc[mi][nj] += tmp[mi][nj] * sc;
            tmp[mi][nj] = (f32x4){0.f, 0.f, 0.f, 0.f};
          }
        }
      }
    } else if constexpr (LPG == 0) {
      for (int kb = 0; kb < nsteps; ++kb) step(kb, tmp);
#pragma unroll
      for (int nj = 0; nj < NB; ++nj) {
        const float sc = scale_of(nj, 0);
#pragma unroll
        for (int mi = 0; mi < 4; ++mi) acc[mi][nj] += tmp[mi][nj] * sc;
      }
    } else {
      const int lpg = W.group / kGK;
      for (int kb = 0; kb < nsteps; ++kb) {
        step(kb, tmp);
        // end of a quantisation group: acc += group partial * scale (straight-line)
        const bool last = ((kb + 1) % lpg == 0) | (kb + 1 == nsteps);
        const int grp = kb / lpg;
#pragma unroll
        for (int nj = 0; nj < NB; ++nj) {
          const float sc = scale_of(nj, grp);
          const float f = last ? sc : 0.0f;
          const float keep = last ? 0.0f : 1.0f;
#pragma unroll
          for (int mi = 0; mi < 4; ++mi) {
            acc[mi][nj] += tmp[mi][nj] * f;
            tmp[mi][nj] *= keep;
          }
        }
      }
    }
  }
  __syncthreads();  // the ring is reused by the caller's next tile
}

// K-loop group structure of a projection: 2 (128-wide groups), 0 (one group
// over K, or no scales), -1 (other).
__host__ __device__ __forceinline__ int ring_lpg(int fmt, int group, int K) {
  if (fmt != FTM_FMT_FP8_BLOCK && fmt != FTM_FMT_INT8_PACKED) return 0;
  if (group >= K) return 0;
  if (group == 2 * kGK && (K / kGK) % 2 == 0) return 2;
  return -1;
}

// Stage A body on the ring tiles: item -> rows, tile, activation epilogue.
template <int WFMT, int LPG>
__device__ void gemm_a_ring_body(const LayerArgs& a, const ProjSlot& W, int Iu, int c0, int m0, int cnt,
                                 const int32_t* list, int shared_col, char* lds) {
  using P = RingPlan<WFMT, 128, kRingA>;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int H = a.L.hidden, KP = a.KP;
  const Rsrc lres = make_rsrc(list, list ? (uint32_t)a.T * 4u : 0u);
  const int p0 = pair_of_row(lres, list != nullptr, m0, cnt, KP, shared_col);
  const char* ap[P::kALoads];
#pragma unroll
  for (int i = 0; i < P::kALoads; ++i) {
    int p = pair_of_row(lres, list != nullptr, m0 + 8 * (wave * P::kALoads + i) + (lane >> 3), cnt, KP, shared_col);
    p = p >= 0 ? p : p0;
    ap[i] = (const char*)a.x + (size_t)(p / KP) * (size_t)H * 2u;
  }
  f32x4 acc[4][2];
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int nj = 0; nj < 2; ++nj) acc[mi][nj] = (f32x4){0.f, 0.f, 0.f, 0.f};
  gemm_tile_ring<WFMT, 128, kRingA, LPG>(W, c0, Iu, ap, lds, acc);
  const int ch = c0 + 16 * wave + (lane & 15);
  const float bg = W.bias != nullptr ? load_scalar(W.bias, ch, W.bias_dt) : 0.0f;
  const float bu = W.bias != nullptr ? load_scalar(W.bias, Iu + ch, W.bias_dt) : 0.0f;
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int pe = pair_of_row(lres, list != nullptr, m0 + 16 * mi + 4 * (lane >> 4) + r, cnt, KP, shared_col);
      if (pe >= 0) {
        const float h = act_fn(a.L.act, acc[mi][0][r] + bg, acc[mi][1][r] + bu, a.L.swiglu_alpha, a.L.swiglu_limit);
        store_scalar(a.hbuf, (size_t)pe * a.Imax + ch, FTM_DT_BF16, h);
      }
    }
}

// ---------------------------------------------------------------- stage A (w13 + activation)
template <int WFMT>
__device__ void gemm_a_body(const LayerArgs& a, const ProjSlot& W, int Iu, int c0, int m0, int cnt,
                            const int32_t* list, int shared_col, uint16_t* sA, uint16_t* sB) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;
  const int H = a.L.hidden, KP = a.KP;
  const Rsrc lres = make_rsrc(list, list ? (uint32_t)a.T * 4u : 0u);
  const Rsrc xres = make_rsrc(a.x, (uint32_t)a.T * (uint32_t)H * 2u);
  uint32_t arow[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int p = pair_of_row(lres, list != nullptr, m0 + ((tid + kBlock * i) >> 3), cnt, KP, shared_col);
    arow[i] = p >= 0 ? (uint32_t)(p / KP) * (uint32_t)H * 2u : kOOB;
  }
  int pe[2][4];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      pe[mi][r] = pair_of_row(lres, list != nullptr, m0 + 32 * wm + 16 * mi + 4 * (lane >> 4) + r, cnt, KP,
                              shared_col);
  float bg[2], bu[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int ch = c0 + 32 * wn + 16 * j + (lane & 15);
    bg[j] = W.bias != nullptr ? load_scalar(W.bias, ch, W.bias_dt) : 0.0f;
    bu[j] = W.bias != nullptr ? load_scalar(W.bias, Iu + ch, W.bias_dt) : 0.0f;
  }
  f32x4 acc[2][4];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int nj = 0; nj < 4; ++nj) acc[mi][nj] = (f32x4){0.f, 0.f, 0.f, 0.f};
  gemm_tile<WFMT, 128>(W, c0, Iu, xres, arow, sA, sB, acc);
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int ch = c0 + 32 * wn + 16 * j + (lane & 15);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if (pe[mi][r] >= 0) {
          const float h = act_fn(a.L.act, acc[mi][j][r] + bg[j], acc[mi][2 + j][r] + bu[j], a.L.swiglu_alpha,
                                 a.L.swiglu_limit);
          store_scalar(a.hbuf, (size_t)pe[mi][r] * a.Imax + ch, FTM_DT_BF16, h);
        }
      }
    }
}

// Stage A ring body by K-loop group structure (ring_lpg): FP8 128x128 blocks
// take LPG 2; INT8 per-channel (one group over K) 0, 128-wide groups 2; bf16 0.
template <int WFMT>
__device__ __forceinline__ void ring_a(const LayerArgs& a, const ProjSlot& W, int Iu, int c0, int m0, int cnt,
                                       const int32_t* list, int shared_col, char* lds) {
  const int lpg = ring_lpg(WFMT, W.group, W.K);
  if constexpr (WFMT == FTM_FMT_BF16 || WFMT == FTM_FMT_MXFP4) {  // no group post-scale
    gemm_a_ring_body<WFMT, 0>(a, W, Iu, c0, m0, cnt, list, shared_col, lds);
  } else if constexpr (WFMT == FTM_FMT_FP8_BLOCK) {
    if (lpg == 2) gemm_a_ring_body<WFMT, 2>(a, W, Iu, c0, m0, cnt, list, shared_col, lds);
    else gemm_a_ring_body<WFMT, -1>(a, W, Iu, c0, m0, cnt, list, shared_col, lds);
  } else {
    if (lpg == 0) gemm_a_ring_body<WFMT, 0>(a, W, Iu, c0, m0, cnt, list, shared_col, lds);
    else if (lpg == 2) gemm_a_ring_body<WFMT, 2>(a, W, Iu, c0, m0, cnt, list, shared_col, lds);
    else gemm_a_ring_body<WFMT, -1>(a, W, Iu, c0, m0, cnt, list, shared_col, lds);
  }
}

// SONLY: the shared expert's items only (its routed experts run elsewhere)
template <int FMT, bool RING, bool SONLY = false>
__device__ __forceinline__ void gemm_a_item(const LayerArgs& a, int item, uint16_t* sA, uint16_t* sB) {
  const int I = a.L.inter, Is = a.L.shared_inter;
  const int nRouted = a.ctrl[kCtrlNRouted];
  const int ntn = I / 64;
  const int routed_items = SONLY ? 0 : gemm_routed_mtiles(a, nRouted) * ntn;
  if (item < routed_items) {
    const GemmTile t = gemm_find_tile(a, item / ntn, nRouted, false);
    if (t.u < 0) return;
    const int e = a.uniq[t.u];
    const int slot = a.L.slot_of_expert ? a.L.slot_of_expert[e] : e;
    if (slot < 0 || slot >= a.L.w13.num_slots) {
      if (threadIdx.x == 0) atomicOr(&a.ctrl[kCtrlError], 1);
      return;
    }
    const ProjSlot W = proj_slot(a.L.w13, slot);
    if constexpr (RING)
      ring_a<FMT>(a, W, I, (item % ntn) * 64, t.m0, t.cnt, a.lists + (size_t)e * a.T, 0, (char*)sA);
    else
      gemm_a_body<FMT>(a, W, I, (item % ntn) * 64, t.m0, t.cnt, a.lists + (size_t)e * a.T, 0, sA, sB);
  } else if (Is > 0) {
    const int sitem = item - routed_items, nts = Is / 64;
    const int m0 = (sitem / nts) * kGM;
    if (m0 >= a.T) return;
    const ProjSlot W = shared_view(a.L.shared_w13, 2 * Is, a.L.hidden);
    if constexpr (RING)
      ring_a<FTM_FMT_BF16>(a, W, Is, (sitem % nts) * 64, m0, a.T, nullptr, a.L.topk, (char*)sA);
    else
      gemm_a_body<FTM_FMT_BF16>(a, W, Is, (sitem % nts) * 64, m0, a.T, nullptr, a.L.topk, sA, sB);
  }
}

template <int FMT>
__global__ __launch_bounds__(kBlock) void k_gemm_a(const LayerArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t sA[2 * kGM * kGPitch];
  __shared__ __attribute__((aligned(16))) uint16_t sB[2 * 128 * kGPitch];
  gemm_a_item<FMT, false>(a, blockIdx.x, sA, sB);
}

extern __shared__ __attribute__((aligned(16))) uint16_t ftm_ring_lds[];

// The ring tiles (dynamic LDS: ring + the layer's tile scales), items in
// XCD-aware order.
template <int FMT, bool SONLY = false>
__global__ __launch_bounds__(kBlock) void k_gemm_a_ring(const LayerArgs a) {
  gemm_a_item<FMT, true, SONLY>(a, xcd_item(blockIdx.x, gridDim.x), ftm_ring_lds, nullptr);
}

// ---------------------------------------------------------------- scaled-MFMA tiles (MXFP4)
// The expert stages of MXFP4 layers above the crossover on
// v_mfma_scale_f32_16x16x128_f8f6f4 with the decode path's operand layouts
// (ftm_moe.hip): the weights go in as stored (e2m1 nibbles, e8m0 block
// scales), the activations as their two-term e4m3 split (kMxChunk bytes per
// row and 128 K: the input by token in the xq region, written by the router
// launch or k_quant_mx; h by pair in the h buffer, written by stage A's
// epilogue).  No weight is decoded.
// Tile: MT rows (pairs) x 256 weight rows -- stage A 128 gate + 128 up
// channels, stage B 256 output columns -- K steps of 128.  Eight waves sit
// 2 x 4, each MT/2 rows x 64 weight rows (MT/32 x 4 blocks of 16 x 16), so
// one A read feeds four weight blocks and one B read MT/32 row blocks, and
// each byte copied to LDS feeds 4-8x as many MFMAs as a 64 x 64-channel tile
// (the copies, not the MFMAs, bound the smaller tiles).  A three-stage LDS
// ring is filled by direct global->LDS copies two K steps ahead: per stage
// the tile's row chunks (16-byte slots in order), its weight rows (64 bytes
// per row, slot q of row r holding piece q ^ ring_fw(r), so the 16 rows of
// one B read hit distinct banks) and the rows' four e8m0 bytes of the step
// (16-bit copies, which land one per 4-byte LDS slot).
constexpr int kMxK = 128;      // K per step
constexpr int kMxThreads = 512;
constexpr int kMxNR = 256;     // weight rows per tile
template <int MT, int S = 3, bool F8 = false>
struct MxPlan {
  static constexpr int kMI = MT / 32;                            // 16-row blocks per wave
  static constexpr int kACopies = MT * (kMxChunk / 16) / 64;     // 16-byte copies of the A chunks per stage
  static constexpr int kABytes = kACopies * 1024;
  static constexpr int kWRow = F8 ? 128 : 64;                    // weight bytes per row per step
  static constexpr int kWPieces = kWRow / 16;
  static constexpr int kWBytes = kMxNR * kWRow;
  static constexpr int kSBytes = F8 ? 0 : kMxNR * 2 * 4;         // e8m0: 2 halves per row, one 4-byte slot each
  static constexpr int kStage = kABytes + kWBytes + kSBytes;
  static constexpr int kStages = S;
  static constexpr int kLds = kStages * kStage;
  // copies per wave per stage: A copies w, w + 8, ...; kWPieces / 2 W copies; one e8m0 copy
  static constexpr int kAMax = (kACopies + 7) / 8;
  static constexpr int kWCopies = kWPieces / 2;
  static constexpr int kLoadsMax = kAMax + kWCopies + (F8 ? 0 : 1);
  static_assert(MT * (kMxChunk / 16) % 64 == 0 && kLoadsMax < 64, "copy shape");
  static_assert(MT * kMxChunk + MT * 4 <= kStage, "stage A's output rows fit one ring slot");
  static_assert(S == 2 || S == 3, "ring depth");
};

template <int MT, int S, bool F8>
__host__ __device__ __forceinline__ size_t mx_tile_lds() { return (size_t)MxPlan<MT, S, F8>::kLds; }

// NT consecutive N tiles of one M tile (stage A: 128 channels each; stage B,
// STB: 256 output columns each).  The A rows' sources and the epilogue's
// pairs are resolved once, and the next tile's first two stages are issued
// before this tile's epilogue.
template <int WFMT, int MT, int S, bool STB>
__device__ void gemm_mx_body(const LayerArgs& a, const ProjSlot& W, int Iu, int c0, int NT, int m0, int cnt,
                             const int32_t* list, char* lds) {
  constexpr bool F8 = WFMT == FTM_FMT_FP8_BLOCK;
  using P = MxPlan<MT, S, F8>;
  constexpr int MI = P::kMI;
  constexpr int kTileN = STB ? kMxNR : kMxNR / 2;
  typedef __attribute__((address_space(1))) const void* GPtr;
  typedef __attribute__((address_space(3))) void* LPtr;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;
  const int g = lane >> 4, m = lane & 15;
  const int K = W.K, KP = a.KP, H = a.L.hidden;
  const int nsteps = (K + kMxK - 1) / kMxK;
  const uint32_t rb = F8 ? (uint32_t)K : (uint32_t)K / 2;  // bytes per weight row (a multiple of 16)
  const uint32_t kgb = (uint32_t)K / 32;  // MXFP4: e8m0 bytes per row (even: K % 64 == 0)
  const int nkb = K / 128;                 // FP8: 128-wide scale blocks along K
  const Rsrc lres = make_rsrc(list, (uint32_t)a.T * 4u);
  const int p0 = pair_of_row(lres, true, m0, cnt, KP, 0);
  const int na = (P::kACopies - wave + 7) / 8;  // this wave's A copies per stage
  // A rows: stage A the quantised input by token, stage B the quantised h by pair
  const uint8_t* abase = STB ? a.hq : a.xq;
  const size_t arow = (size_t)mx_row_bytes(STB ? a.Imax : H);
  const int adiv = STB ? 1 : KP;

  // ---- A copy sources: slot s = tile row s / 17, piece s % 17 (rows past
  // the tile's pairs repeat its first)
  const char* asrc[P::kAMax];
#pragma unroll
  for (int i = 0; i < P::kAMax; ++i) {
    const int sl = 64 * (8 * i + wave) + lane;
    const int r = sl / (kMxChunk / 16), pc = sl - r * (kMxChunk / 16);
    int pr = r < MT ? pair_of_row(lres, true, m0 + r, cnt, KP, 0) : -1;
    pr = pr >= 0 ? pr : p0;
    asrc[i] = (const char*)abase + (size_t)(pr / adiv) * arow + 16 * pc;
  }
  // the pairs of this lane's output rows (epilogue) and, stage B, their router weights
  int pe[MI][4];
  float we[MI][4];
  const Rsrc wres = make_rsrc(a.wts, (uint32_t)a.T * (uint32_t)KP * 4u);
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      pe[mi][r] = pair_of_row(lres, true, m0 + (MT / 2) * wm + 16 * mi + 4 * g + r, cnt, KP, 0);
      we[mi][r] = STB ? __uint_as_float(bload4(wres, pe[mi][r] >= 0 ? 4u * (uint32_t)pe[mi][r] : kOOB)) : 0.0f;
    }

  // ---- per-tile weight sources.  W slot s = row s / kWPieces, slot s %
  // kWPieces holding that piece xor a swizzle of the row (ring_fw for 4
  // pieces, ring_fa for 8); a piece past the row's end (last K step) re-reads
  // the row's first: finite codes against zero activations.  Rows past the
  // projection (the last tile) repeat its last row; their outputs are
  // dropped (stage B) or zeroed (stage A's channels past I).  MXFP4 scale
  // slot s = row s / 2, bytes 2 (s % 2), +1 of the step's four (past the
  // row's end its first two, against zero activations).
  constexpr int WC = P::kWCopies;
  const char* wrow[WC];
  uint32_t wpo[WC];
  const char* srow = nullptr;
  auto swz = [](int r) { return F8 ? ring_fa(r) : ring_fw(r); };
  auto grow = [&](int cc, int r) {
    int row;
    if constexpr (STB) row = cc + r;
    else row = r < kMxNR / 2 ? cc + r : Iu + cc + (r - kMxNR / 2);
    return row < W.N ? row : W.N - 1;
  };
  auto tile_sources = [&](int cc) {
#pragma unroll
    for (int i = 0; i < WC; ++i) {
      const int sl = 64 * (8 * i + wave) + lane;
      const int r = sl / P::kWPieces;
      wrow[i] = (const char*)W.w + (size_t)grow(cc, r) * rb;
      wpo[i] = 16u * (uint32_t)((sl % P::kWPieces) ^ swz(r));
    }
    if constexpr (!F8) srow = (const char*)W.s + (size_t)grow(cc, (64 * wave + lane) >> 1) * kgb;
  };
  const uint32_t sho = 2u * (uint32_t)(lane & 1);
  auto issue = [&](int kb, int slot) {
    char* st = lds + slot * P::kStage;
#pragma unroll
    for (int i = 0; i < P::kAMax; ++i)
      if (i < na)
        __builtin_amdgcn_global_load_lds((GPtr)(asrc[i] + (size_t)kb * kMxChunk),
                                         (LPtr)(st + 1024 * (8 * i + wave)), 16, 0, 0);
#pragma unroll
    for (int i = 0; i < WC; ++i) {
      const uint32_t off = (uint32_t)P::kWRow * (uint32_t)kb + wpo[i];
      __builtin_amdgcn_global_load_lds((GPtr)(wrow[i] + (off + 16u <= rb ? off : 0u)),
                                       (LPtr)(st + P::kABytes + 1024 * (8 * i + wave)), 16, 0, 0);
    }
    if constexpr (!F8) {
      const uint32_t so = 4u * (uint32_t)kb + sho;
      __builtin_amdgcn_global_load_lds((GPtr)(srow + (so + 2u <= kgb ? so : 0u)),
                                       (LPtr)(st + P::kABytes + P::kWBytes + 256 * wave), 2, 0, 0);
    }
  };
  const int pro = nsteps < P::kStages - 1 ? nsteps : P::kStages - 1;
  tile_sources(c0);
  for (int kb = 0; kb < pro; ++kb) issue(kb, kb);

  int brow[4];
#pragma unroll
  for (int nj = 0; nj < 4; ++nj)
    brow[nj] = (STB ? 64 * wn + 16 * nj : nj < 2 ? 32 * wn + 16 * nj : kMxNR / 2 + 32 * wn + 16 * (nj - 2)) + m;
  for (int t = 0; t < NT; ++t) {
    const int cc = c0 + kTileN * t;
    uint32_t bb[4];  // bias bits (converted in the epilogue): stage A gate j, up j; stage B column nj
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      int ch;
      if constexpr (STB) ch = cc + 64 * wn + 16 * j + m;
      else ch = (j < 2 ? 0 : Iu) + cc + 32 * wn + 16 * (j & 1) + m;
      bb[j] = W.bias != nullptr && ch < W.N ? load_bits(W.bias, ch, W.bias_dt) : 0u;
    }
    f32x4 acc[MI][4];
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
      for (int nj = 0; nj < 4; ++nj) acc[mi][nj] = (f32x4){0.f, 0.f, 0.f, 0.f};
    for (int kb = 0; kb < nsteps; ++kb) {
      // this wave's copies of stage kb have landed (the next stage's, and
      // loads issued after them, may be in flight), then every wave's have;
      // every wave is also done with stage kb - 1 (its reads fed MFMAs that
      // have issued).  A plain barrier: __syncthreads' release fence would
      // wait for every copy in flight, the next stage's too.
      if (S == 3 && kb + 1 < nsteps) {
        if (na == P::kAMax) wait_vm<P::kLoadsMax>(); else wait_vm<P::kLoadsMax - 1>();
      } else {
        wait_vm<0>();  // two stages: nothing is issued past stage kb yet
      }
      asm volatile("s_barrier" ::: "memory");
      if (kb + P::kStages - 1 < nsteps) issue(kb + P::kStages - 1, (kb + P::kStages - 1) % P::kStages);
      const char* st = lds + (kb % P::kStages) * P::kStage;
      // FP8: the step's fp32 block scales of this wave's rows (stage A: gate, up; stage B: its 64 columns)
      float fs0 = 1.0f, fs1 = 1.0f;
      if constexpr (F8) {
        const int b0 = STB ? (cc + 64 * wn) / 128 : cc / 128, b1 = STB ? b0 : (Iu + cc) / 128;
        fs0 = __uint_as_float(sload4(W.s, 4u * (uint32_t)(b0 * nkb + kb)));
        fs1 = __uint_as_float(sload4(W.s, 4u * (uint32_t)(b1 * nkb + kb)));
      }
      i32x8 bw[4];
      int sb[4];
#pragma unroll
      for (int nj = 0; nj < 4; ++nj) {
        const char* wr = st + P::kABytes + brow[nj] * P::kWRow;
        if constexpr (F8) {
          // e4m3 B operand: K [16 g, 16 g + 16) and [64 + 16 g, ...) of the step
          const u32x4 r0 = *(const u32x4*)(wr + 16 * (g ^ ring_fa(brow[nj])));
          const u32x4 r1 = *(const u32x4*)(wr + 16 * ((4 + g) ^ ring_fa(brow[nj])));
          bw[nj] = (i32x8){(int)r0.x, (int)r0.y, (int)r0.z, (int)r0.w, (int)r1.x, (int)r1.y, (int)r1.z, (int)r1.w};
          sb[nj] = 127;
        } else {
          const u32x4 r = *(const u32x4*)(wr + 16 * (g ^ ring_fw(brow[nj])));
          bw[nj] = (i32x8){(int)r.x, (int)r.y, (int)r.z, (int)r.w, 0, 0, 0, 0};
          const uint32_t sv = *(const uint32_t*)(st + P::kABytes + P::kWBytes + 4 * (2 * brow[nj] + (g >> 1)));
          sb[nj] = (int)((sv >> (8 * (g & 1))) & 0xffu);
        }
      }
#pragma unroll
      for (int mi = 0; mi < MI; ++mi) {
        const char* cb = st + ((MT / 2) * wm + 16 * mi + m) * kMxChunk;
        const u32x4 h0 = *(const u32x4*)(cb + 16 * g);
        const u32x4 h1 = *(const u32x4*)(cb + 64 + 16 * g);
        const u32x4 l0 = *(const u32x4*)(cb + 128 + 16 * g);
        const u32x4 l1 = *(const u32x4*)(cb + 192 + 16 * g);
        const uint32_t sc = *(const uint16_t*)(cb + 256 + 2 * g);
        const i32x8 ahi = {(int)h0.x, (int)h0.y, (int)h0.z, (int)h0.w, (int)h1.x, (int)h1.y, (int)h1.z, (int)h1.w};
        const i32x8 alo = {(int)l0.x, (int)l0.y, (int)l0.z, (int)l0.w, (int)l1.x, (int)l1.y, (int)l1.z, (int)l1.w};
#pragma unroll
        for (int nj = 0; nj < 4; ++nj) {
          constexpr int kB = F8 ? 0 : 4;  // B format: e4m3 or e2m1
          if constexpr (F8) {
            // the step's partial sums scaled by the block scale of these rows
            f32x4 tq = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(ahi, bw[nj], (f32x4){0.f, 0.f, 0.f, 0.f},
                                                                        0, kB, 0, (int)(sc & 0xffu), 0, sb[nj]);
            tq = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(alo, bw[nj], tq, 0, kB, 0, (int)(sc >> 8), 0,
                                                                  sb[nj]);
            acc[mi][nj] += tq * ((STB || nj < 2) ? fs0 : fs1);
          } else {
            acc[mi][nj] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(ahi, bw[nj], acc[mi][nj], 0, kB, 0,
                                                                           (int)(sc & 0xffu), 0, sb[nj]);
            acc[mi][nj] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(alo, bw[nj], acc[mi][nj], 0, kB, 0,
                                                                           (int)(sc >> 8), 0, sb[nj]);
          }
        }
      }
    }
    // every wave is done with the ring (its last reads fed MFMAs that have
    // issued): the next tile's first stages go out before this epilogue, into
    // slots 0 .. S - 2; stage A stages its output rows in slot S - 1
    asm volatile("s_barrier" ::: "memory");
    if (t + 1 < NT) {
      tile_sources(cc + kTileN);
      for (int kb = 0; kb < pro; ++kb) issue(kb, kb);
    }

    if constexpr (STB) {
      // ---- stage B epilogue: router-weighted fp32 rows into the slot buffer
#pragma unroll
      for (int nj = 0; nj < 4; ++nj) {
        const int col = cc + 64 * wn + 16 * nj + m;
        const float bn = bits_to_f32(opaque_bits(bb[nj]), W.bias_dt);
#pragma unroll
        for (int mi = 0; mi < MI; ++mi)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (pe[mi][r] >= 0 && col < W.N) a.ybuf[(size_t)pe[mi][r] * H + col] = (acc[mi][nj][r] + bn) * we[mi][r];
      }
    } else {
      // ---- stage A epilogue: h = bf16(act(gate + b_g, up + b_u)) (zero for
      // channels past I), split into e4m3 hi + lo over the wave's 32-channel
      // block of each row; the tile's 128 channels are one whole chunk, staged
      // in slot 2 in the chunk layout and copied out in 16-byte pieces
      char* stg = lds + (S - 1) * P::kStage;
      int* stg_pe = (int*)(stg + MT * kMxChunk);
      const float bg0 = bits_to_f32(opaque_bits(bb[0]), W.bias_dt), bg1 = bits_to_f32(opaque_bits(bb[1]), W.bias_dt);
      const float bu0 = bits_to_f32(opaque_bits(bb[2]), W.bias_dt), bu1 = bits_to_f32(opaque_bits(bb[3]), W.bias_dt);
      const bool in0 = cc + 32 * wn + m < Iu, in1 = cc + 32 * wn + 16 + m < Iu;
#pragma unroll
      for (int mi = 0; mi < MI; ++mi)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int tr = (MT / 2) * wm + 16 * mi + 4 * g + r;
          float h0 = bf16_to_f32(f32_to_bf16(
              act_fn(a.L.act, acc[mi][0][r] + bg0, acc[mi][2][r] + bu0, a.L.swiglu_alpha, a.L.swiglu_limit)));
          float h1 = bf16_to_f32(f32_to_bf16(
              act_fn(a.L.act, acc[mi][1][r] + bg1, acc[mi][3][r] + bu1, a.L.swiglu_alpha, a.L.swiglu_limit)));
          h0 = in0 ? h0 : 0.0f;
          h1 = in1 ? h1 : 0.0f;
          // the block's largest |h| bit pattern over the row's 16 lanes (Inf / NaN: >= 0x7f800000)
          int mb = max((int)(__float_as_uint(h0) & 0x7fffffffu), (int)(__float_as_uint(h1) & 0x7fffffffu));
          mb = max(mb, dpp_i<kDppXor1>(mb));
          mb = max(mb, dpp_i<kDppXor2>(mb));
          mb = max(mb, dpp_i<kDppHalfMirror>(mb));
          mb = max(mb, dpp_i<kDppMirror>(mb));
          const uint32_t chi = (uint32_t)max((mb >> 23) - 7, 0);
          const uint32_t clo = chi >= 4u ? chi - 4u : 0u;
          const float inv = __uint_as_float((254u - chi) << 23);
          const float flo = __uint_as_float((127u + chi - clo) << 23);
          const float s0 = h0 * inv, s1 = h1 * inv;
          const uint32_t q = f32x2_to_e4m3(s0, s1);
          const uint32_t l = f32x2_to_e4m3((s0 - e4m3_at<0>(q)) * flo, (s1 - e4m3_at<1>(q)) * flo);
          char* row = stg + tr * kMxChunk;
          row[32 * wn + m] = (char)q;
          row[32 * wn + 16 + m] = (char)(q >> 8);
          row[128 + 32 * wn + m] = (char)l;
          row[128 + 32 * wn + 16 + m] = (char)(l >> 8);
          if (m == 0) {
            *(uint16_t*)(row + 256 + 2 * wn) = (uint16_t)(mb < 0x7f800000 ? (chi | (clo << 8)) : 0xffffu);
            stg_pe[tr] = pe[mi][r];
          }
        }
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      // copy out the chunk of each real row (its last 16 bytes: 8 scale bytes
      // and 8 bytes nothing reads)
      uint8_t* hq = a.hq;
      const size_t hrow = (size_t)mx_row_bytes(a.Imax);
      for (int q = tid; q < MT * (kMxChunk / 16); q += kMxThreads) {
        const int tr = q / (kMxChunk / 16), k = q - tr * (kMxChunk / 16);
        const int p = stg_pe[tr];
        if (p >= 0)
          *(u32x4*)(hq + (size_t)p * hrow + (size_t)(cc / 128) * kMxChunk + 16 * k) =
              *(const u32x4*)(stg + tr * kMxChunk + 16 * k);
      }
    }
  }
}

// Routed MXFP4 expert tiles on the scaled MFMAs (a layer without a shared
// expert, mx_gemm_ok): one workgroup per (M tile, ntpw consecutive N
// tiles), items in XCD-aware order.  STB: stage B (w2, the quantised h).
// N tiles per workgroup: stage A 1, stage B 2.  Measured on MI355X (prefill,
// w13 / w2 us): C4 T=4096 one tile 829-834 / 421, two 861 / 399, three 913 /
// 425; C3 T=2048 one 297-303 / 218, two 304 / 191, three 412 / 185.
constexpr int kMxNTA = 1;
constexpr int kMxNTB = 2;
template <int WFMT, int MT, int S, bool STB>
__global__ __launch_bounds__(kMxThreads) void k_gemm_mx(const LayerArgs a, int ntpw) {
  const int item = xcd_item(blockIdx.x, gridDim.x);
  const int nRouted = a.ctrl[kCtrlNRouted];
  const int tiles = STB ? (a.L.hidden + kMxNR - 1) / kMxNR : (a.L.inter + kMxNR / 2 - 1) / (kMxNR / 2);
  const int ntn = (tiles + ntpw - 1) / ntpw;
  const int routed_items = gemm_routed_mtiles<MT>(a, nRouted) * ntn;
  if (item >= routed_items) return;
  const GemmTile t = gemm_find_tile<MT>(a, item / ntn, nRouted, false);
  if (t.u < 0) return;
  // wave-uniform values in scalar registers, so the buffer descriptors built
  // from them are scalar too (no per-load waterfall loops)
  const int e = __builtin_amdgcn_readfirstlane(a.uniq[t.u]);
  const int slot = __builtin_amdgcn_readfirstlane(a.L.slot_of_expert ? a.L.slot_of_expert[e] : e);
  const ftm_proj& PW = STB ? a.L.w2 : a.L.w13;
  const int n0 = (item % ntn) * ntpw;
  const int nt = tiles - n0 < ntpw ? tiles - n0 : ntpw;
  const int tn = STB ? kMxNR : kMxNR / 2;
  const int32_t* list = a.lists + (size_t)e * a.T;
  const int m0 = __builtin_amdgcn_readfirstlane(t.m0), cnt = __builtin_amdgcn_readfirstlane(t.cnt);
  if (slot < 0 || slot >= PW.num_slots) {
    if (STB) {  // non-resident expert: its rows contribute zeros
      const int H = a.L.hidden;
      for (int idx = threadIdx.x; idx < MT * tn * nt; idx += kMxThreads) {
        const int mm = m0 + idx / (tn * nt), col = tn * n0 + idx % (tn * nt);
        if (mm < cnt && col < H) a.ybuf[(size_t)list[mm] * H + col] = 0.0f;
      }
    }
    if (threadIdx.x == 0) atomicOr(&a.ctrl[kCtrlError], 1);
    return;
  }
  gemm_mx_body<WFMT, MT, S, STB>(a, proj_slot(PW, slot), a.L.inter, tn * n0, nt, m0, cnt, list, (char*)ftm_ring_lds);
}

// Stage B (w2) of FP8 routed experts with weights fed from registers: the
// tile's quantised h rows (64 rows x K / 128 chunks, at most 69.6 KB) are
// copied into LDS once and stay there; each wave loads the e4m3 B operands
// of its 32 columns straight into VGPRs with buffer loads (no LDS ring, no
// per-step barrier), the next N tile's operands in flight during the current
// tile's MFMAs.  One workgroup per (M tile, ntpw consecutive 128-column N
// tiles), four waves, two workgroups per CU.  K = I, a multiple of 128 up to
// 512.  The products, the per-step fp32 block scales and the epilogue are
// those of gemm_mx_body's stage B, in the same order, so the output is the same.
constexpr int kRbThreads = 256;
constexpr int kRbMT = 64;
constexpr int kRbKS = 4;     // K steps at most (K <= 512)
constexpr int kRbNT = 128;   // output columns per N tile (one FP8 scale block)
constexpr int kRbNTW = 8;    // N tiles per workgroup
constexpr int kRbA = kRbMT * kRbKS * kMxChunk;
constexpr int kRbLds = kRbA + kRbMT * 8;  // + the rows' pairs and router weights
static_assert(2 * kRbLds <= 160 * 1024, "two workgroups per CU");

__global__ __launch_bounds__(kRbThreads, 2) void k_gemm_mxb_f8(const LayerArgs a, int ntpw) {
  const int item = xcd_item(blockIdx.x, gridDim.x);
  const int nRouted = a.ctrl[kCtrlNRouted];
  const int H = a.L.hidden;
  const int tiles = (H + kRbNT - 1) / kRbNT;
  const int ntn = (tiles + ntpw - 1) / ntpw;
  const int routed_items = gemm_routed_mtiles<kRbMT>(a, nRouted) * ntn;
  if (item >= routed_items) return;
  const GemmTile t = gemm_find_tile<kRbMT>(a, item / ntn, nRouted, false);
  if (t.u < 0) return;
  const int e = __builtin_amdgcn_readfirstlane(a.uniq[t.u]);
  const int slot = __builtin_amdgcn_readfirstlane(a.L.slot_of_expert ? a.L.slot_of_expert[e] : e);
  const int n0 = __builtin_amdgcn_readfirstlane((item % ntn) * ntpw);
  const int nt = tiles - n0 < ntpw ? tiles - n0 : ntpw;
  const int32_t* list = a.lists + (size_t)e * a.T;
  const int m0 = __builtin_amdgcn_readfirstlane(t.m0), cnt = __builtin_amdgcn_readfirstlane(t.cnt);
  const int tid = threadIdx.x;
  if (slot < 0 || slot >= a.L.w2.num_slots) {  // non-resident expert: its rows contribute zeros
    for (int idx = tid; idx < kRbMT * kRbNT * nt; idx += kRbThreads) {
      const int mm = m0 + idx / (kRbNT * nt), col = kRbNT * n0 + idx % (kRbNT * nt);
      if (mm < cnt && col < H) a.ybuf[(size_t)list[mm] * H + col] = 0.0f;
    }
    if (tid == 0) atomicOr(&a.ctrl[kCtrlError], 1);
    return;
  }
  const ProjSlot W = proj_slot(a.L.w2, slot);
  char* lds = (char*)ftm_ring_lds;
  int* lpe = (int*)(lds + kRbA);
  float* lwe = (float*)(lpe + kRbMT);
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, m = lane & 15;
  const int K = W.K, KP = a.KP;
  const int nsteps = K / 128;
  const Rsrc lres = make_rsrc(list, (uint32_t)a.T * 4u);
  const int p0 = pair_of_row(lres, true, m0, cnt, KP, 0);
  const size_t hrow = (size_t)mx_row_bytes(a.Imax);

  // the rows' pairs (rows past the tile's pairs: -1) and router weights
  if (tid < kRbMT) {
    const int pr = pair_of_row(lres, true, m0 + tid, cnt, KP, 0);
    lpe[tid] = pr;
    lwe[tid] = pr >= 0 ? a.wts[pr] : 0.0f;
  }

  // ---- B operands: column c = 128 tile + 32 wave + 16 nj + m, K bytes
  // [16 g, 16 g + 16) and [64 + 16 g, ...) of each 128-wide step (the
  // operand layout of gemm_mx_body).  Every load is issued unconditionally
  // (columns past N and tiles past the item's last read as zeros through an
  // out-of-range offset, without memory traffic), so each tile's loads are
  // the same 16 in flight whatever the branches did and the compiler's
  // counted waits stop at the tile being used.
  const Rsrc wres = make_rsrc(W.w, (uint32_t)K * (uint32_t)W.N);
  // the columns' bias bits, in the same batch (a layer without bias: an
  // empty descriptor, zeros); converted in the epilogue
  const bool b32 = W.bias_dt == FTM_DT_F32;
  const Rsrc bres = make_rsrc(W.bias, W.bias != nullptr ? (uint32_t)W.N * (b32 ? 4u : 2u) : 0u);
  const int nkb = nsteps;
  // tile t's operands (and bias bits) into w / bb; tiles past the item's
  // last read nothing (an out-of-range offset), so every iteration issues
  // the same loads and the compiler's counted waits stop at the tile in use
  auto load_w = [&](int t, u32x4 (&w)[2][kRbKS][2], uint32_t (&bb)[2]) {
    const bool live = t < nt;
#pragma unroll
    for (int nj = 0; nj < 2; ++nj) {
      const uint32_t col = (uint32_t)(kRbNT * (n0 + t) + 32 * wave + 16 * nj + m);
      const uint32_t bo = live ? col * (b32 ? 4u : 2u) : kOOB;
      bb[nj] = b32 ? __builtin_amdgcn_raw_buffer_load_b32(bres, bo, 0, 0)
                   : (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(bres, bo, 0, 0);
    }
#pragma unroll
    for (int nj = 0; nj < 2; ++nj) {
      const uint32_t rowoff =
          (uint32_t)(kRbNT * (n0 + t) + 32 * wave + 16 * nj + m) * (uint32_t)K + 16u * (uint32_t)g;
#pragma unroll
      for (int kb = 0; kb < kRbKS; ++kb)
#pragma unroll
        for (int h = 0; h < 2; ++h)
          w[nj][kb][h] =
              bload16(wres, live && kb < nsteps ? rowoff + 128u * (uint32_t)kb + 64u * (uint32_t)h : kOOB);
    }
  };

  // ---- the A tile: piece q (16 bytes) = step q / 1088, row (q / 17) % 64,
  // piece q % 17 of that step's 272-byte chunk, at LDS byte 16 q (rows past
  // the tile's pairs repeat its first; steps past K re-read step 0 and are
  // never used)
  constexpr int kPieces = kRbMT * kRbKS * (kMxChunk / 16);
  constexpr int kPPT = kPieces / kRbThreads;
  static_assert(kPieces % kRbThreads == 0, "A pieces per thread");
  u32x4 wa[2][kRbKS][2], wb[2][kRbKS][2];
  uint32_t ba[2], bb2[2];
  load_w(0, wa, ba);
  __syncthreads();  // the rows' pairs
  {
    u32x4 av[kPPT];
#pragma unroll
    for (int i = 0; i < kPPT; ++i) {
      const int q = tid + kRbThreads * i;
      const int kb = q / (kRbMT * (kMxChunk / 16)), rem = q - kb * (kRbMT * (kMxChunk / 16));
      const int r = rem / (kMxChunk / 16), pc = rem - r * (kMxChunk / 16);
      const int pr = lpe[r];
      const int kc = kb < nsteps ? kb : 0;
      av[i] = *(const u32x4*)(a.hq + (size_t)(pr >= 0 ? pr : p0) * hrow + (size_t)kc * kMxChunk + 16 * pc);
    }
    load_w(1, wb, bb2);
#pragma unroll
    for (int i = 0; i < kPPT; ++i) *(u32x4*)(lds + 16 * (tid + kRbThreads * i)) = av[i];
  }
  __syncthreads();  // the A tile is in LDS

  // router-weighted fp32 rows into the slot buffer: rows past the tile's
  // pairs and columns past H are stored to an out-of-range offset (dropped)
  const Rsrc yres = make_rsrc(a.ybuf, (uint32_t)a.T * (uint32_t)KP * (uint32_t)H * 4u);
  auto run_tile = [&](int t, const u32x4 (&w)[2][kRbKS][2], const uint32_t (&bb)[2]) {
    const int tile = n0 + t;
    f32x4 acc[4][2];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int nj = 0; nj < 2; ++nj) acc[mi][nj] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < kRbKS; ++kb) {
      if (kb < nsteps) {
        // the step's fp32 block scale of this wave's columns (one 128-block per N tile)
        const float fs = __uint_as_float(sload4(W.s, 4u * (uint32_t)(tile * nkb + kb)));
#pragma unroll
        for (int mi = 0; mi < 4; ++mi) {
          const char* cb = lds + (kb * kRbMT + 16 * mi + m) * kMxChunk;
          const u32x4 h0 = *(const u32x4*)(cb + 16 * g);
          const u32x4 h1 = *(const u32x4*)(cb + 64 + 16 * g);
          const u32x4 l0 = *(const u32x4*)(cb + 128 + 16 * g);
          const u32x4 l1 = *(const u32x4*)(cb + 192 + 16 * g);
          const uint32_t sc = *(const uint16_t*)(cb + 256 + 2 * g);
          const i32x8 ahi = {(int)h0.x, (int)h0.y, (int)h0.z, (int)h0.w, (int)h1.x, (int)h1.y, (int)h1.z, (int)h1.w};
          const i32x8 alo = {(int)l0.x, (int)l0.y, (int)l0.z, (int)l0.w, (int)l1.x, (int)l1.y, (int)l1.z, (int)l1.w};
#pragma unroll
          for (int nj = 0; nj < 2; ++nj) {
            const u32x4 r0 = w[nj][kb][0], r1 = w[nj][kb][1];
            const i32x8 bw = {(int)r0.x, (int)r0.y, (int)r0.z, (int)r0.w, (int)r1.x, (int)r1.y, (int)r1.z, (int)r1.w};
            f32x4 tq = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(ahi, bw, (f32x4){0.f, 0.f, 0.f, 0.f}, 0, 0,
                                                                        0, (int)(sc & 0xffu), 0, 127);
            tq = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(alo, bw, tq, 0, 0, 0, (int)(sc >> 8), 0, 127);
            acc[mi][nj] += tq * fs;
          }
        }
      }
    }
#pragma unroll
    for (int nj = 0; nj < 2; ++nj) {
      const int col = kRbNT * tile + 32 * wave + 16 * nj + m;
      const float bn = bits_to_f32(opaque_bits(bb[nj]), W.bias_dt);
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = 16 * mi + 4 * g + r;
          const int pe = lpe[row];
          const uint32_t off = pe >= 0 && col < H ? 4u * ((uint32_t)pe * (uint32_t)H + (uint32_t)col) : kOOB;
          __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint((acc[mi][nj][r] + bn) * lwe[row]), yres, off, 0, 0);
        }
    }
  };

  // tiles in pairs: tile t's operands are in flight during tile t - 1's MFMAs
  for (int t = 0; t < nt; t += 2) {
    run_tile(t, wa, ba);
    load_w(t + 2, wa, ba);
    if (t + 1 < nt) run_tile(t + 1, wb, bb2);
    load_w(t + 3, wb, bb2);
  }
}

// ---------------------------------------------------------------- stage B (w2 -> slot buffer)
template <int WFMT>
__device__ void gemm_b_body(const LayerArgs& a, const ProjSlot& W, int n0, int m0, int cnt, const int32_t* list,
                            int shared_col, uint16_t* sA, uint16_t* sB) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;
  const int H = a.L.hidden, KP = a.KP;
  const Rsrc lres = make_rsrc(list, list ? (uint32_t)a.T * 4u : 0u);
  const Rsrc hres = make_rsrc(a.hbuf, (uint32_t)a.T * (uint32_t)KP * (uint32_t)a.Imax * 2u);
  const Rsrc wres = make_rsrc(a.wts, (uint32_t)a.T * (uint32_t)KP * 4u);
  uint32_t arow[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int p = pair_of_row(lres, list != nullptr, m0 + ((tid + kBlock * i) >> 3), cnt, KP, shared_col);
    arow[i] = p >= 0 ? (uint32_t)p * (uint32_t)a.Imax * 2u : kOOB;
  }
  int pe[2][4];
  float we[2][4];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      pe[mi][r] = pair_of_row(lres, list != nullptr, m0 + 32 * wm + 16 * mi + 4 * (lane >> 4) + r, cnt, KP,
                              shared_col);
      we[mi][r] = __uint_as_float(bload4(wres, pe[mi][r] >= 0 ? 4u * (uint32_t)pe[mi][r] : kOOB));
    }
  float bn[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = n0 + 32 * wn + 16 * j + (lane & 15);
    bn[j] = W.bias != nullptr ? load_scalar(W.bias, n, W.bias_dt) : 0.0f;
  }
  f32x4 acc[2][2];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int nj = 0; nj < 2; ++nj) acc[mi][nj] = (f32x4){0.f, 0.f, 0.f, 0.f};
  gemm_tile<WFMT, 64>(W, n0, 0, hres, arow, sA, sB, acc);
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = n0 + 32 * wn + 16 * j + (lane & 15);
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (pe[mi][r] >= 0) {
          float y = acc[mi][j][r];
          if (W.bias != nullptr) y += bn[j];
          a.ybuf[(size_t)pe[mi][r] * H + n] = y * we[mi][r];
        }
    }
}

template <int FMT, bool SONLY = false>
__device__ __forceinline__ void gemm_b_item(const LayerArgs& a, int item, uint16_t* sA, uint16_t* sB) {
  const int H = a.L.hidden, Is = a.L.shared_inter;
  const int nRouted = a.ctrl[kCtrlNRouted];
  const int ntn = H / 64;
  const int routed_items = SONLY ? 0 : gemm_routed_mtiles(a, nRouted) * ntn;
  if (item < routed_items) {
    const GemmTile t = gemm_find_tile(a, item / ntn, nRouted, false);
    if (t.u < 0) return;
    const int e = a.uniq[t.u];
    const int32_t* list = a.lists + (size_t)e * a.T;
    const int slot = a.L.slot_of_expert ? a.L.slot_of_expert[e] : e;
    const int n0 = (item % ntn) * 64;
    if (slot < 0 || slot >= a.L.w2.num_slots) {
      // non-resident expert: its rows contribute zeros
      for (int idx = threadIdx.x; idx < kGM * 64; idx += kBlock) {
        const int m = t.m0 + idx / 64;
        if (m < t.cnt) a.ybuf[(size_t)list[m] * H + n0 + idx % 64] = 0.0f;
      }
      if (threadIdx.x == 0) atomicOr(&a.ctrl[kCtrlError], 1);
      return;
    }
    const ProjSlot W = proj_slot(a.L.w2, slot);
    gemm_b_body<FMT>(a, W, n0, t.m0, t.cnt, list, 0, sA, sB);
  } else if (Is > 0) {
    const int sitem = item - routed_items;
    const int m0 = (sitem / ntn) * kGM;
    if (m0 >= a.T) return;
    const ProjSlot W = shared_view(a.L.shared_w2, H, Is);
    gemm_b_body<FTM_FMT_BF16>(a, W, (sitem % ntn) * 64, m0, a.T, nullptr, a.L.topk, sA, sB);
  }
}

template <int FMT, bool SONLY = false>
__global__ __launch_bounds__(kBlock) void k_gemm_b(const LayerArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t sA[2 * kGM * kGPitch];
  __shared__ __attribute__((aligned(16))) uint16_t sB[2 * 64 * kGPitch];
  gemm_b_item<FMT, SONLY>(a, blockIdx.x, sA, sB);
}

// ---------------------------------------------------------------- launch
bool gemm_path_ok(const ftm_moe_layer& L, int T) {
  if (L.act_dtype != FTM_DT_BF16) return false;
  const int f = L.w13.fmt;
  if (f != FTM_FMT_FP8_BLOCK && f != FTM_FMT_INT8_PACKED && f != FTM_FMT_MXFP4 && f != FTM_FMT_BF16) return false;
  if (L.hidden % 64 != 0 || L.inter % 64 != 0 || (L.shared_inter > 0 && L.shared_inter % 64 != 0)) return false;
  if ((f == FTM_FMT_FP8_BLOCK || f == FTM_FMT_INT8_PACKED) &&
      (L.w13.group % kGK != 0 || L.w2.group % kGK != 0))
    return false;
  if (L.apply_router_weight_on_input) return false;
  // above the crossover: on average at least kGemmMinRows tokens per routed
  // expert (MXFP4: more than that, up to which its scaled-MFMA decode path wins)
  const long pairs = (long)T * L.topk;
  const long maxU = L.num_experts < pairs ? L.num_experts : pairs;
  if (f == FTM_FMT_MXFP4 && T <= kXlMaxTMx) return pairs > (long)kGemmMinRows * maxU;
  return pairs >= (long)kGemmMinRows * maxU;
}

// Whether the ring tiles take this layer: weights whose tile scales fit the
// LDS scale area (INT8: one fp32 per tile row and group; MXFP4: one e8m0 byte
// per tile row and 32 K).
static bool ring_ok(const ftm_moe_layer& L) {
  const int f = L.w13.fmt;
  if (f == FTM_FMT_MXFP4 && 128 * (L.hidden / 32) > kRingScaleBytes) return false;  // e8m0 bytes of the tile
  if (f == FTM_FMT_INT8_PACKED || f == FTM_FMT_FP8_BLOCK) {
    const long g13 = (L.hidden + L.w13.group - 1) / L.w13.group;
    if (f == FTM_FMT_INT8_PACKED && 128 * g13 * 4 > kRingScaleBytes) return false;
    if (f == FTM_FMT_FP8_BLOCK && 2 * g13 > kBlock) return false;  // one scale per thread
  }
  return true;
}

// Dynamic LDS of the ring kernels for this layer: ring + tile scales.
static size_t ring_lds_a(const ftm_moe_layer& L) {
  const int f = L.w13.fmt;
  if (f == FTM_FMT_MXFP4) return (size_t)kRingA + 128u * (size_t)(L.hidden / 32);
  const int g = (L.hidden + L.w13.group - 1) / (L.w13.group > 0 ? L.w13.group : 1);
  const int rows = f == FTM_FMT_FP8_BLOCK ? 2 : f == FTM_FMT_INT8_PACKED ? 128 : 0;
  return (size_t)kRingA + (size_t)rows * g * 4;
}
bool mx_gemm_ok(const ftm_moe_layer& L) {
  static_assert(MxPlan<128, 3, false>::kLds <= 160 * 1024 && MxPlan<64, 3, true>::kLds <= 160 * 1024,
                "the tiles' rings fit a CU's LDS");
  // the ring tiles take the shared expert's items (their tile scales fit)
  return mx_fmt(L) && (L.shared_inter == 0 || ring_ok(L));
}

const char* gemm_a_kernel_name(const ftm_moe_layer& L) {
  return mx_gemm_ok(L) ? "k_gemm_mx" : ring_ok(L) ? "k_gemm_a_ring" : "k_gemm_a";
}

template <int FMT, bool SONLY = false>
static void ring_lds_attr() {
  static bool done = false;  // once per instantiation (setting it twice is harmless)
  if (!done) {
    // a failure here surfaces as the launch error that follows
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&k_gemm_a_ring<FMT, SONLY>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, kRingA + kRingScaleBytes);
    done = true;
  }
}

// Stage B on k_gemm_mxb_f8: FP8 weights, K = I a multiple of 128 up to 512
// (the whole A tile resident in LDS), and a slot buffer that one buffer
// descriptor spans (below 2 GiB, so the out-of-range store offset is past it).
static bool mxb_reg_ok(const ftm_moe_layer& L, long T, int KP) {
  return L.w2.fmt == FTM_FMT_FP8_BLOCK && (L.w2.flags & FTM_PROJ_RING_B) == 0 && L.w2.K == L.inter &&
         L.inter % 128 == 0 && L.inter <= 128 * kRbKS && 4.0 * (double)T * (double)KP * (double)L.hidden < 2147483648.0;
}

const char* gemm_b_kernel_name(const ftm_moe_layer& L, int T) {
  if (!mx_gemm_ok(L)) return "k_gemm_b";
  return mxb_reg_ok(L, T, L.topk + (L.shared_inter > 0 ? 1 : 0)) ? "k_gemm_mxb_f8" : "k_gemm_mx";
}

template <int WFMT, int MT, int S>
static void launch_gemm_mx(const LayerArgs& a, hipStream_t st, int which, bool xq_ready, long pairs, long maxU) {
  constexpr bool F8 = WFMT == FTM_FMT_FP8_BLOCK;
  const ftm_moe_layer& L = a.L;
  static bool attr = false;
  if (!attr) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&k_gemm_mx<WFMT, MT, S, false>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)MxPlan<MT, S, F8>::kLds);
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&k_gemm_mx<WFMT, MT, S, true>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)MxPlan<MT, S, F8>::kLds);
    attr = true;
  }
  const long mt = pairs / MT + maxU + 1;
  const size_t lds = mx_tile_lds<MT, S, F8>();
  // the bf16 shared expert (if any) on the bf16 tiles, its items only
  const long mt_shared = L.shared_inter > 0 ? (a.T + kGM - 1) / kGM : 0;
  if (which & 1) {
    if (!xq_ready) launch_quant_mx(a.x, a.T, L.hidden, a.xq, st);
    const int ntA = kMxNTA;
    const long items = mt * (((L.inter + kMxNR / 2 - 1) / (kMxNR / 2) + ntA - 1) / ntA);
    hipLaunchKernelGGL((k_gemm_mx<WFMT, MT, S, false>), dim3((unsigned)items), dim3(kMxThreads), lds, st, a, ntA);
    if (mt_shared > 0) {
      ring_lds_attr<WFMT, true>();
      hipLaunchKernelGGL((k_gemm_a_ring<WFMT, true>), dim3((unsigned)(mt_shared * (L.shared_inter / 64))),
                         dim3(kBlock), (size_t)kRingA, st, a);
    }
  }
  if (which & 2) {
    if (mxb_reg_ok(a.L, a.T, a.KP) && MT == kRbMT) {
      static bool rb_attr = false;
      if (!rb_attr) {
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&k_gemm_mxb_f8),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, kRbLds);
        rb_attr = true;
      }
      const long items = mt * (((L.hidden + kRbNT - 1) / kRbNT + kRbNTW - 1) / kRbNTW);
      hipLaunchKernelGGL(k_gemm_mxb_f8, dim3((unsigned)items), dim3(kRbThreads), (size_t)kRbLds, st, a, kRbNTW);
    } else {
      const int ntB = kMxNTB;
      const long items = mt * (((L.hidden + kMxNR - 1) / kMxNR + ntB - 1) / ntB);
      hipLaunchKernelGGL((k_gemm_mx<WFMT, MT, S, true>), dim3((unsigned)items), dim3(kMxThreads), lds, st, a, ntB);
    }
    if (mt_shared > 0)
      hipLaunchKernelGGL((k_gemm_b<WFMT, true>), dim3((unsigned)(mt_shared * (L.hidden / 64))), dim3(kBlock), 0,
                         st, a);
  }
}

template <int FMT>
static void launch_gemm_t(const LayerArgs& a, hipStream_t st, int which, bool xq_ready) {
  const ftm_moe_layer& L = a.L;
  const long pairs = (long)a.T * L.topk;
  const long maxU = L.num_experts < pairs ? L.num_experts : pairs;
  if constexpr (FMT == FTM_FMT_MXFP4 || FMT == FTM_FMT_FP8_BLOCK) {
    if (mx_gemm_ok(L)) {
      // both stages' routed experts on the scaled-MFMA tiles: stage A over the
      // quantised input, writing h quantised the same way for stage B.  MXFP4:
      // 128-row M tiles from 128 pairs per expert on average, 64 below; FP8
      // (twice the weight bytes in the ring): 64.
      if constexpr (FMT == FTM_FMT_MXFP4) {
        if (pairs >= 128 * maxU) {
          launch_gemm_mx<FMT, 128, 3>(a, st, which, xq_ready, pairs, maxU);
          return;
        }
      }
      launch_gemm_mx<FMT, 64, 3>(a, st, which, xq_ready, pairs, maxU);
      return;
    }
  }
  const long mt_routed = pairs / kGM + maxU + 1;
  const long mt_shared = L.shared_inter > 0 ? (a.T + kGM - 1) / kGM : 0;
  const long items_a = mt_routed * (L.inter / 64) + mt_shared * (L.shared_inter > 0 ? L.shared_inter / 64 : 0);
  const long items_b = (mt_routed + mt_shared) * (L.hidden / 64);
  // Stage A on the ring tiles where they apply (measured on MI355X, C3 FP8:
  // w13 285 us against 343 at T=2048, 179 against 239 at T=512; C1 INT8 T=1024:
  // 29 against 42; C4 MXFP4 T=4096: 1045 against 1415).  Stage B keeps the register-staged tiles: with K = I its
  // tiles are 8 K steps long and 4 workgroups per CU beat the deeper ring
  // (C3 T=2048 w2 259 us against 377).
  const bool ring = ring_ok(L);
  if (which & 1) {
    if (ring) {
      ring_lds_attr<FMT>();
      hipLaunchKernelGGL((k_gemm_a_ring<FMT>), dim3((unsigned)items_a), dim3(kBlock), ring_lds_a(L), st, a);
    } else {
      hipLaunchKernelGGL((k_gemm_a<FMT>), dim3((unsigned)items_a), dim3(kBlock), 0, st, a);
    }
  }
  if (which & 2) hipLaunchKernelGGL((k_gemm_b<FMT>), dim3((unsigned)items_b), dim3(kBlock), 0, st, a);
}

void launch_gemm_stages(const ftm_moe_layer& L, const void* x, int T, void* out, char* ws, const WsLayout& wl,
                        hipStream_t st, int which, bool xq_ready) {
  const LayerArgs a = make_args(L, x, out, T, ws, wl);
  switch (L.w13.fmt) {
    case FTM_FMT_FP8_BLOCK: launch_gemm_t<FTM_FMT_FP8_BLOCK>(a, st, which, xq_ready); break;
    case FTM_FMT_INT8_PACKED: launch_gemm_t<FTM_FMT_INT8_PACKED>(a, st, which, xq_ready); break;
    case FTM_FMT_MXFP4: launch_gemm_t<FTM_FMT_MXFP4>(a, st, which, xq_ready); break;
    default: launch_gemm_t<FTM_FMT_BF16>(a, st, which, xq_ready); break;
  }
}

}  // namespace ftm
