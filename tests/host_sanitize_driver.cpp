// Host-code driver for the sanitizer runs of the library's host-only parts:
// the slot-pool LRU (ftm_offload.cpp) and the CPU expert kernel of the hybrid
// split (ftm_cpu.cpp).  Built by tests/test_host_sanitize.py with g++
// -fsanitize=address,undefined (no argument: every check below) and with
// -fsanitize=thread (argument "threads": several host threads submitting to
// and waiting on the async worker, ftm_cpu_moe_submit / ftm_cpu_moe_wait,
// beside synchronous multi-threaded calls); any sanitizer report fails the
// process.  Every call is made with random
// (seeded) shapes, routings, caller state -- valid, and corrupt where the
// API takes caller-owned state -- and argument errors, and the results are
// checked for the invariants the Python tests check on the real data.
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <random>
#include <thread>
#include <vector>

#include "ftmoe.h"

#define CHECK(c)                                                        \
  do {                                                                  \
    if (!(c)) {                                                         \
      fprintf(stderr, "check failed %s:%d: %s\n", __FILE__, __LINE__, #c); \
      return 1;                                                         \
    }                                                                   \
  } while (0)

static int lru_run(std::mt19937& g) {
  for (int trial = 0; trial < 300; ++trial) {
    const int L = 1 + (int)(g() % 3), E = 1 + (int)(g() % 40);
    const int S = 1 + (int)(g() % (E + 6));
    std::vector<int32_t> sfi((size_t)L * E, -1), ios((size_t)S, -1), ev((size_t)(E > S ? E : S)), src(ev.size());
    std::vector<int64_t> usage((size_t)S, 0);
    int64_t step = 0;
    int32_t staged = 0;
    if (trial % 7 == 3) {  // corrupt caller state: ids and slots out of range
      for (auto& v : ios) v = (int32_t)(g() % (3 * L * E + 3)) - 1;
      for (auto& v : sfi) v = (int32_t)(g() % (3 * S + 3)) - 1;
    }
    for (int call = 0; call < 20; ++call) {
      const int layer = (int)(g() % L);
      if (S >= E && g() % 5 == 0) {
        const int rc = ftm_lru_materialize(layer, L, E, S, sfi.data(), ios.data(), usage.data(), &step, ev.data(),
                                           src.data(), &staged);
        CHECK(rc >= 0 && rc == staged && staged <= E);
      } else {
        const int n = (int)(g() % 24);
        std::vector<int64_t> ids((size_t)n);
        for (auto& v : ids) v = (int64_t)(g() % E);
        const int rc = ftm_lru_ensure(layer, L, E, S, ids.data(), n, sfi.data(), ios.data(), usage.data(), &step,
                                      ev.data(), src.data(), &staged);
        CHECK(rc >= 0 && rc == staged && staged <= E);
      }
      for (int i = 0; i < staged; ++i) CHECK(ev[i] >= 0 && ev[i] < S && src[i] >= 0 && src[i] < E);
      for (int id = 0; id < L * E; ++id) CHECK(sfi[id] >= -1 && sfi[id] < S);  // rebuilt from id_of_slot
    }
    // argument errors: no state is touched past the checks
    const int64_t bad[1] = {E};
    CHECK(ftm_lru_ensure(0, L, E, S, bad, 1, sfi.data(), ios.data(), usage.data(), &step, ev.data(), src.data(),
                         &staged) == FTM_ERR_DIM);
    CHECK(ftm_lru_ensure(L, L, E, S, nullptr, 0, sfi.data(), ios.data(), usage.data(), &step, ev.data(), src.data(),
                         &staged) == FTM_ERR_DIM);
    CHECK(ftm_lru_ensure(0, L, E, S, nullptr, 1, sfi.data(), ios.data(), usage.data(), &step, ev.data(), src.data(),
                         &staged) == FTM_ERR_NULL);
    CHECK(ftm_lru_materialize(0, L, E, S, nullptr, ios.data(), usage.data(), &step, ev.data(), src.data(),
                              &staged) == (S < E ? FTM_ERR_DIM : FTM_ERR_NULL));
  }
  return 0;
}

// Random bytes for packed weights; scales drawn as finite floats.
struct Bank {
  std::vector<uint8_t> w, s, z, bias;
};

static void fill(std::vector<uint8_t>& v, size_t n, std::mt19937& g) {
  v.resize(n);
  for (auto& b : v) b = (uint8_t)g();
}
static void fill_scales(std::vector<uint8_t>& v, size_t n, int dt, std::mt19937& g) {
  std::uniform_real_distribution<float> u(0.001f, 0.1f);
  const size_t es = dt == FTM_DT_F32 ? 4 : 2;
  v.resize(n * es);
  for (size_t i = 0; i < n; ++i) {
    const float f = u(g);
    uint32_t bits;
    memcpy(&bits, &f, 4);
    if (es == 4) {
      memcpy(&v[4 * i], &bits, 4);
    } else {
      const uint16_t h = (uint16_t)(bits >> 16);  // bf16 of f (finite, positive)
      memcpy(&v[2 * i], &h, 2);
    }
  }
}

// One projection [N, K] of E slots in format fmt; returns false for a shape the format cannot hold.
static bool make_proj(int fmt, int E, int N, int K, std::mt19937& g, Bank& b, ftm_proj& p) {
  memset(&p, 0, sizeof(p));
  p.fmt = fmt;
  p.N = N;
  p.K = K;
  p.num_slots = E;
  p.s_dtype = (g() & 1) ? FTM_DT_F32 : FTM_DT_BF16;
  size_t wb = 0, sb = 0, zb = 0;
  switch (fmt) {
    case FTM_FMT_FP8_BLOCK:
    case FTM_FMT_FP8_E5M2_BLOCK:
      p.group = (g() & 1) ? 16 : 32;
      wb = (size_t)N * K;
      sb = (size_t)((N + p.group - 1) / p.group) * ((K + p.group - 1) / p.group);
      break;
    case FTM_FMT_INT8_PACKED:
      p.group = (K % 32 == 0 && (g() & 1)) ? 32 : K;
      wb = (size_t)N * K;
      sb = (size_t)N * (K / p.group);
      break;
    case FTM_FMT_MXFP4:
      if (K % 32 != 0) return false;
      p.group = 32;
      wb = (size_t)N * K / 2;
      sb = (size_t)N * (K / 32);
      break;
    case FTM_FMT_GPTQ_INT4:
      if (K % 8 != 0 || N % 8 != 0) return false;
      p.group = (K % 16 == 0 && (g() & 1)) ? 16 : 8;
      p.s_dtype = (g() & 1) ? FTM_DT_F32 : FTM_DT_F16;
      wb = (size_t)(K / 8) * N * 4;
      sb = (size_t)((K + p.group - 1) / p.group) * N;
      zb = (size_t)((K + p.group - 1) / p.group) * (N / 8) * 4;
      break;
    case FTM_FMT_BF16:
      wb = (size_t)N * K * 2;
      break;
    default:  // FP32
      wb = (size_t)N * K * 4;
      break;
  }
  fill(b.w, wb * E, g);
  if (fmt == FTM_FMT_BF16 || fmt == FTM_FMT_FP32) {  // finite values: sign, small exponent
    const size_t es = fmt == FTM_FMT_BF16 ? 2 : 4;
    for (size_t i = 0; i < b.w.size(); i += es) b.w[i + es - 1] &= 0xbf;
  }
  p.w = b.w.data();
  p.w_stride = (int64_t)wb;
  if (sb) {
    if (fmt == FTM_FMT_MXFP4) {
      fill(b.s, sb * E, g);
    } else if (fmt == FTM_FMT_GPTQ_INT4 && p.s_dtype == FTM_DT_F16) {
      b.s.resize(sb * E * 2);
      for (size_t i = 0; i < sb * E; ++i) {
        const uint16_t h = (uint16_t)(0x2000 + g() % 0x1000);  // small positive fp16
        memcpy(&b.s[2 * i], &h, 2);
      }
    } else {
      fill_scales(b.s, sb * E, p.s_dtype, g);
    }
    p.s = b.s.data();
    p.s_stride = (int64_t)(b.s.size() / E);
  }
  if (zb) {
    fill(b.z, zb * E, g);
    p.z = b.z.data();
    p.z_stride = (int64_t)zb;
  }
  if (g() % 3 == 0) {
    fill_scales(b.bias, (size_t)N * E, FTM_DT_BF16, g);
    p.bias = b.bias.data();
    p.bias_dtype = FTM_DT_BF16;
    p.bias_stride = (int64_t)N * 2;
  }
  return true;
}

static int cpu_moe_run(std::mt19937& g) {
  const int fmts[] = {FTM_FMT_FP8_BLOCK, FTM_FMT_FP8_E5M2_BLOCK, FTM_FMT_INT8_PACKED, FTM_FMT_MXFP4,
                      FTM_FMT_GPTQ_INT4, FTM_FMT_BF16, FTM_FMT_FP32};
  int runs = 0;
  for (int trial = 0; trial < 140; ++trial) {
    const int fmt = fmts[trial % 7];
    const int E = 1 + (int)(g() % 6), H = 8 * (1 + (int)(g() % 12)), I = 8 * (1 + (int)(g() % 8));
    const int k = 1 + (int)(g() % (E < 4 ? E : 4));
    Bank b13, b2;
    ftm_moe_layer L;
    memset(&L, 0, sizeof(L));
    if (!make_proj(fmt, E, 2 * I, H, g, b13, L.w13) || !make_proj(fmt, E, H, I, g, b2, L.w2)) continue;
    L.num_experts = E;
    L.hidden = H;
    L.inter = I;
    L.topk = k;
    L.act = (int)(g() % 4);
    L.swiglu_alpha = 1.702f;
    L.swiglu_limit = 7.0f;
    L.act_dtype = FTM_DT_F32;
    L.h_dtype = FTM_DT_F32;
    const int T = (int)(g() % 10);
    std::vector<float> x((size_t)T * H), w((size_t)T * k), out((size_t)T * H);
    std::normal_distribution<float> nd(0.0f, 1.0f);
    for (auto& v : x) v = nd(g);
    for (auto& v : w) v = nd(g);
    std::vector<int32_t> ids((size_t)T * k);
    for (auto& v : ids) v = (int32_t)(g() % (E + 1)) - 1;  // -1: a pair without an expert
    std::vector<uint8_t> mask((size_t)E);
    for (auto& v : mask) v = (uint8_t)(g() & 1);
    const uint8_t* mp = (g() & 1) ? mask.data() : nullptr;
    const int threads = (g() & 1) ? 1 : 3;
    for (int scalar = 0; scalar < 2; ++scalar) {
      CHECK(ftm_cpu_moe_forward(&L, x.data(), T, ids.data(), w.data(), mp, threads, scalar, out.data()) == FTM_OK);
      ++runs;
    }
    const int64_t h = ftm_cpu_moe_submit(&L, x.data(), T, ids.data(), w.data(), mp, threads, out.data());
    CHECK(h > 0);
    CHECK(ftm_cpu_moe_wait(h) == FTM_OK);
    CHECK(ftm_cpu_moe_wait(h) == FTM_ERR_HANDLE);
    if (T > 0) {  // an id >= E is an argument error, before any work
      std::vector<int32_t> bad(ids);
      bad[0] = E;
      CHECK(ftm_cpu_moe_forward(&L, x.data(), T, bad.data(), w.data(), nullptr, 1, 0, out.data()) == FTM_ERR_DIM);
    }
  }
  ftm_moe_layer Z;
  memset(&Z, 0, sizeof(Z));
  CHECK(ftm_cpu_moe_forward(nullptr, nullptr, 0, nullptr, nullptr, nullptr, 0, 0, nullptr) == FTM_ERR_NULL);
  CHECK(ftm_cpu_moe_forward(&Z, nullptr, 0, nullptr, nullptr, nullptr, 0, 0, nullptr) == FTM_ERR_DIM);
  CHECK(ftm_cpu_moe_wait(123456) == FTM_ERR_HANDLE);
  CHECK(runs > 100);
  return 0;
}

// One host thread's share of the threaded run: its own layer and buffers,
// async jobs (the worker holds one job at a time, so submits from other
// threads wait for this thread's wait) alternating with synchronous calls
// that fan out over their own pool threads; each result is compared with the
// same call run synchronously on one thread.
static int threaded_client(unsigned seed, int iters, std::atomic<int>* failures, std::atomic<int>* done) {
  std::mt19937 g(seed);
  const int fmts[] = {FTM_FMT_FP8_BLOCK, FTM_FMT_INT8_PACKED, FTM_FMT_MXFP4, FTM_FMT_GPTQ_INT4, FTM_FMT_BF16};
  for (int it = 0; it < iters; ++it) {
    const int fmt = fmts[(seed + it) % 5];
    const int E = 2 + (int)(g() % 5), H = 64, I = 32, k = 2;
    Bank b13, b2;
    ftm_moe_layer L;
    memset(&L, 0, sizeof(L));
    if (!make_proj(fmt, E, 2 * I, H, g, b13, L.w13) || !make_proj(fmt, E, H, I, g, b2, L.w2)) continue;
    L.num_experts = E;
    L.hidden = H;
    L.inter = I;
    L.topk = k;
    L.swiglu_alpha = 1.702f;
    L.swiglu_limit = 7.0f;
    L.act_dtype = FTM_DT_F32;
    L.h_dtype = FTM_DT_F32;
    const int T = 1 + (int)(g() % 4);
    std::vector<float> x((size_t)T * H), w((size_t)T * k), a((size_t)T * H), b((size_t)T * H), c((size_t)T * H);
    std::normal_distribution<float> nd(0.0f, 1.0f);
    for (auto& v : x) v = nd(g);
    for (auto& v : w) v = nd(g);
    std::vector<int32_t> ids((size_t)T * k);
    for (int t = 0; t < T; ++t) {
      ids[(size_t)t * k] = (int32_t)(g() % E);
      ids[(size_t)t * k + 1] = (ids[(size_t)t * k] + 1) % E;
    }
    const int64_t h = ftm_cpu_moe_submit(&L, x.data(), T, ids.data(), w.data(), nullptr, 2, a.data());
    const int rc_sync = ftm_cpu_moe_forward(&L, x.data(), T, ids.data(), w.data(), nullptr, 3, 0, b.data());
    const int rc_async = h > 0 ? ftm_cpu_moe_wait(h) : (int)h;
    const int rc_one = ftm_cpu_moe_forward(&L, x.data(), T, ids.data(), w.data(), nullptr, 1, 0, c.data());
    if (h <= 0 || rc_async != FTM_OK || rc_sync != FTM_OK || rc_one != FTM_OK) {
      fprintf(stderr, "threaded client %u: rc submit %lld wait %d sync %d one %d\n", seed, (long long)h, rc_async,
              rc_sync, rc_one);
      failures->fetch_add(1);
      return 1;
    }
    for (size_t i = 0; i < c.size(); ++i) {
      const float tol = 1e-4f * (1.0f + (c[i] < 0 ? -c[i] : c[i]));
      const float da = a[i] - c[i], db = b[i] - c[i];
      if (da > tol || da < -tol || db > tol || db < -tol) {
        fprintf(stderr, "threaded client %u: result %zu differs (%g %g %g)\n", seed, i, a[i], b[i], c[i]);
        failures->fetch_add(1);
        return 1;
      }
    }
    done->fetch_add(1);
  }
  return 0;
}

static int threads_run() {
  std::atomic<int> failures{0}, done{0};
  std::vector<std::thread> pool;
  for (unsigned s = 0; s < 4; ++s)
    pool.emplace_back([s, &failures, &done] { threaded_client(1000u + s, 25, &failures, &done); });
  for (auto& t : pool) t.join();
  printf("threaded iterations: %d\n", done.load());
  return failures.load() == 0 && done.load() >= 60 ? 0 : 1;
}

int main(int argc, char** argv) {
  if (argc > 1 && strcmp(argv[1], "threads") == 0) {
    if (threads_run() != 0) return 1;
    printf("host sanitize driver (threads): ok\n");
    return 0;
  }
  std::mt19937 g(20261202u);
  if (lru_run(g) != 0) return 1;
  if (cpu_moe_run(g) != 0) return 1;
  printf("host sanitize driver: ok\n");
  return 0;
}
