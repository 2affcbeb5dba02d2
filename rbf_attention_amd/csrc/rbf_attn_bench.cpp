// rbf_attn_bench: native timing harness for the C ABI (no Python).
//
// Allocates a workload's tensors with hipMalloc, fills them on the host with
// seeded inputs of the benchmark's distributions, and times one training
// step (rbf_attn_fwd then rbf_attn_bwd) on its own stream with HIP events:
//   * warm: after a clock ramp and warm-up steps, K back-to-back steps
//     between two events;
//   * per kernel, right after the step loop: fwd, bwd and the backward's two
//     stages (rbf_attn_bwd_stage 1 and 2) each in a loop of its own of at
//     least 200 launches and 0.2 s;
//   * cold: the median over reps of one step timed alone after a 512 MiB
//     write that evicts L2 and MALL (outside the events), and likewise of the
//     forward alone and of the backward alone (from the saved forward
//     outputs).
// Prints one JSON line.  Built by rbf_attention_amd/build.py next to
// librbfattn.so (found through the binary's rpath).
//
//   rbf_attn_bench [--workload c2_model_bf16|c3_long_bf16|c4_nonsoftmax_bf16]
//                  [--steps K] [--warmup W] [--cold-reps R] [--ramp-seconds S]
//
// The inputs follow the benchmark's distributions (q, v, dO ~ N(0, std^2);
// content key rows scaled by exp(sigma z); the 4 register rows of q, k, v
// zero) from this program's own generator, so they are not the values that
// bench.py's torch generator draws: the harness times the kernels, it does
// not check results.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "rbf_attn.h"

namespace {

struct Workload {
  const char* name;
  int B, H, content, D;
  int dtype;
  bool softmax;
  float std;
  float key_lognormal;
};

const Workload kWorkloads[] = {
    {"c2_model_bf16", 32, 8, 512, 64, RBF_ATTN_BF16, true, 1.0f, 0.5f},
    {"c3_long_bf16", 4, 16, 8192, 128, RBF_ATTN_BF16, true, 1.0f, 0.5f},
    {"c4_nonsoftmax_bf16", 16, 8, 2048, 64, RBF_ATTN_BF16, false, 0.5f, 0.0f},
};
constexpr int kRegisters = 4;
constexpr size_t kFlushBytes = size_t(512) << 20;

void die(const char* what, const char* detail) {
  fprintf(stderr, "rbf_attn_bench: %s: %s\n", what, detail);
  exit(1);
}

void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) die(what, hipGetErrorString(e));
}

void abi_check(int rc, const char* what) {
  if (rc != RBF_ATTN_OK) die(what, rbf_attn_last_error());
}

// splitmix64 stream -> standard normals (Box-Muller)
struct Rng {
  uint64_t s;
  explicit Rng(uint64_t seed) : s(seed) {}
  uint64_t next() {
    uint64_t z = (s += 0x9e3779b97f4a7c15ULL);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
  }
  double uniform() { return ((next() >> 11) + 0.5) * (1.0 / 9007199254740992.0); }
  float normal() {
    const double u1 = uniform(), u2 = uniform();
    return (float)(std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2));
  }
};

// round to nearest even, 16-bit patterns
uint16_t to_bf16(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

uint16_t to_fp16(float x) {
  const _Float16 h = (_Float16)x;
  uint16_t u;
  memcpy(&u, &h, 2);
  return u;
}

size_t elem_size(int dtype) { return dtype == RBF_ATTN_FP32 ? 4 : 2; }

// host values of a (B, H, N, D) tensor in the element type
std::vector<uint8_t> make_tensor(const Workload& w, int N, Rng& rng, bool zero_registers, bool key_scale) {
  const size_t n = (size_t)w.B * w.H * N * w.D, esz = elem_size(w.dtype);
  std::vector<uint8_t> out(n * esz);
  std::vector<float> row(w.D);
  size_t idx = 0;
  for (int bh = 0; bh < w.B * w.H; ++bh)
    for (int t = 0; t < N; ++t) {
      const bool reg = t < kRegisters;
      const float scale = key_scale && !reg ? std::exp(w.key_lognormal * rng.normal()) : 1.0f;
      for (int d = 0; d < w.D; ++d) row[d] = (zero_registers && reg) ? 0.0f : w.std * rng.normal() * scale;
      for (int d = 0; d < w.D; ++d, ++idx) {
        if (w.dtype == RBF_ATTN_FP32) {
          memcpy(&out[idx * 4], &row[d], 4);
        } else {
          const uint16_t u = w.dtype == RBF_ATTN_BF16 ? to_bf16(row[d]) : to_fp16(row[d]);
          memcpy(&out[idx * 2], &u, 2);
        }
      }
    }
  return out;
}

rbf_attn_tensor desc(void* p, const Workload& w, int N) {
  rbf_attn_tensor t;
  t.ptr = p;
  t.stride_n = w.D;
  t.stride_h = (int64_t)N * w.D;
  t.stride_b = (int64_t)w.H * N * w.D;
  return t;
}

double median(std::vector<double> v) {
  std::sort(v.begin(), v.end());
  const size_t m = v.size() / 2;
  return v.size() % 2 ? v[m] : 0.5 * (v[m - 1] + v[m]);
}

}  // namespace

int main(int argc, char** argv) {
  std::string wname = "c2_model_bf16";
  int steps = 200, warmup = 20, cold_reps = 25;
  double ramp_s = 0.4;
  for (int i = 1; i < argc; ++i) {
    const std::string a = argv[i];
    auto val = [&]() -> const char* {
      if (i + 1 >= argc) die("missing value for", a.c_str());
      return argv[++i];
    };
    if (a == "--workload") wname = val();
    else if (a == "--steps") steps = atoi(val());
    else if (a == "--warmup") warmup = atoi(val());
    else if (a == "--cold-reps") cold_reps = atoi(val());
    else if (a == "--ramp-seconds") ramp_s = atof(val());
    else die("unknown argument", a.c_str());
  }
  const Workload* wp = nullptr;
  for (const Workload& w : kWorkloads)
    if (wname == w.name) wp = &w;
  if (!wp) die("unknown workload", wname.c_str());
  if (steps < 1 || cold_reps < 1 || warmup < 0) die("bad counts", "steps and cold reps must be >= 1");
  const Workload& w = *wp;
  const int N = w.content + kRegisters;
  if (rbf_attn_abi_version() != RBF_ATTN_ABI_VERSION) die("library", "ABI version mismatch");

  // inputs in the benchmark's order: q, k, v, dO
  Rng rng(42);
  std::vector<uint8_t> hq = make_tensor(w, N, rng, true, false);
  std::vector<uint8_t> hk = make_tensor(w, N, rng, true, w.key_lognormal > 0.0f);
  std::vector<uint8_t> hv = make_tensor(w, N, rng, true, false);
  std::vector<uint8_t> hdo = make_tensor(w, N, rng, false, false);
  const size_t bytes = hq.size(), rows = (size_t)w.B * w.H * N;

  hip_check(hipSetDevice(0), "hipSetDevice");
  void *q, *k, *v, *o, *dout, *dq, *dk, *dv, *flush;
  float *lse, *delta;
  for (void** p : {&q, &k, &v, &o, &dout, &dq, &dk, &dv}) hip_check(hipMalloc(p, bytes), "hipMalloc");
  hip_check(hipMalloc((void**)&lse, rows * 4), "hipMalloc");
  hip_check(hipMalloc((void**)&delta, rows * 4), "hipMalloc");
  hip_check(hipMalloc(&flush, kFlushBytes), "hipMalloc");
  hip_check(hipMemcpy(q, hq.data(), bytes, hipMemcpyHostToDevice), "hipMemcpy");
  hip_check(hipMemcpy(k, hk.data(), bytes, hipMemcpyHostToDevice), "hipMemcpy");
  hip_check(hipMemcpy(v, hv.data(), bytes, hipMemcpyHostToDevice), "hipMemcpy");
  hip_check(hipMemcpy(dout, hdo.data(), bytes, hipMemcpyHostToDevice), "hipMemcpy");

  rbf_attn_args a;
  memset(&a, 0, sizeof(a));
  a.abi_version = RBF_ATTN_ABI_VERSION;
  a.variant = w.softmax ? RBF_ATTN_SOFTMAX : RBF_ATTN_NON_SOFTMAX;
  a.dtype = w.dtype;
  a.B = w.B;
  a.H = w.H;
  a.N = N;
  a.D = w.D;
  a.causal = 1;
  a.num_prefix = 0;
  a.gamma = (float)(1.0 / (2.0 * std::sqrt((double)w.D)));
  a.q = desc(q, w, N);
  a.k = desc(k, w, N);
  a.v = desc(v, w, N);
  a.o = desc(o, w, N);
  a.dout = desc(dout, w, N);
  a.dq = desc(dq, w, N);
  a.dk = desc(dk, w, N);
  a.dv = desc(dv, w, N);
  a.lse = lse;
  a.delta = delta;

  hipStream_t st;
  hip_check(hipStreamCreate(&st), "hipStreamCreate");
  hipEvent_t e0, e1;
  hip_check(hipEventCreate(&e0), "hipEventCreate");
  hip_check(hipEventCreate(&e1), "hipEventCreate");
  auto fwd = [&]() { abi_check(rbf_attn_fwd(&a, st), "rbf_attn_fwd"); };
  auto bwd = [&]() { abi_check(rbf_attn_bwd(&a, st), "rbf_attn_bwd"); };
  auto stage1 = [&]() { abi_check(rbf_attn_bwd_stage(&a, st, 1), "rbf_attn_bwd_stage 1"); };
  auto stage2 = [&]() { abi_check(rbf_attn_bwd_stage(&a, st, 2), "rbf_attn_bwd_stage 2"); };
  auto step = [&]() {
    fwd();
    bwd();
  };
  // mean ms of n calls between two events
  auto loop = [&](auto&& fn, int n) {
    hip_check(hipStreamSynchronize(st), "sync");
    hip_check(hipEventRecord(e0, st), "hipEventRecord");
    for (int i = 0; i < n; ++i) fn();
    hip_check(hipEventRecord(e1, st), "hipEventRecord");
    hip_check(hipEventSynchronize(e1), "hipEventSynchronize");
    float ms = 0.f;
    hip_check(hipEventElapsedTime(&ms, e0, e1), "hipEventElapsedTime");
    return (double)ms / n;
  };

  // clock ramp, then warm-up
  const auto t0 = std::chrono::steady_clock::now();
  int ramp_n = 0;
  while (std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count() < ramp_s) {
    for (int i = 0; i < 10; ++i) step();
    hip_check(hipStreamSynchronize(st), "sync");
    ramp_n += 10;
  }
  for (int i = 0; i < warmup; ++i) step();
  const double ms_step = loop(step, steps);

  // one kernel: at least 200 launches and 0.2 s, the count from a short loop
  auto kernel_loop = [&](auto&& fn) {
    const double est = loop(fn, 20);
    long long n = (long long)std::ceil(200.0 / std::max(est, 1e-4));
    n = std::min<long long>(std::max<long long>(n, 200), 20000);
    return loop(fn, (int)n);
  };
  const double ms_fwd = kernel_loop(fwd), ms_bwd = kernel_loop(bwd);
  const double ms_dq = kernel_loop(stage1), ms_dkdv = kernel_loop(stage2);
  const int bwd_launches = rbf_attn_bwd_kernels(&a, nullptr);

  auto cold_median = [&](auto&& fn) {
    std::vector<double> t;
    for (int r = 0; r < cold_reps; ++r) {
      hip_check(hipMemsetAsync(flush, r & 0xff, kFlushBytes, st), "hipMemsetAsync");
      t.push_back(loop(fn, 1));
    }
    return median(t);
  };
  const double cold_step = cold_median(step), cold_fwd = cold_median(fwd);
  step();  // the backward alone reads the outputs the last forward saved
  const double cold_bwd = cold_median(bwd);

  const double P = (double)N * (N + 1) / 2.0 * w.B * w.H;
  const double flops = 14.0 * w.D * P;
  printf("{\"harness\": \"rbf_attn_bench (C ABI, no Python)\", \"workload\": \"%s\", \"steps\": %d, \"warmup\": %d, "
         "\"ramp_steps\": %d, \"step_us\": %.3f, \"tflops\": %.3f, \"fwd_us\": %.3f, \"bwd_us\": %.3f, "
         "\"bwd_dq_us\": %.3f, \"bwd_dkdv_us\": %.3f, \"bwd_launches\": %d, "
         "\"cold\": {\"step_us_median\": %.3f, \"fwd_us_median\": %.3f, \"bwd_us_median\": %.3f, \"reps\": %d}}\n",
         w.name, steps, warmup, ramp_n, ms_step * 1e3, flops / (ms_step * 1e-3) / 1e12, ms_fwd * 1e3, ms_bwd * 1e3,
         ms_dq * 1e3, ms_dkdv * 1e3, bwd_launches, cold_step * 1e3, cold_fwd * 1e3, cold_bwd * 1e3, cold_reps);

  hip_check(hipStreamSynchronize(st), "sync");
  hip_check(hipEventDestroy(e0), "hipEventDestroy");
  hip_check(hipEventDestroy(e1), "hipEventDestroy");
  hip_check(hipStreamDestroy(st), "hipStreamDestroy");
  for (void* p : {q, k, v, o, dout, dq, dk, dv, (void*)lse, (void*)delta, flush}) hip_check(hipFree(p), "hipFree");
  return 0;
}
