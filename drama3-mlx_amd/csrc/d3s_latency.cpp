/* Host-side latency of one-row d3s_sample calls as a C caller of the library
 * sees them (tower_decode_step samples one row at a time, src/tower.c:420-446):
 * per call, the wall time from the call to its return (the enqueue) and to the
 * return of hipStreamSynchronize;
 * in a second pass, from the call until hipStreamQuery reports the stream
 * done (the caller polls instead of blocking); in a third, HIP events around
 * the launch.  With "spin" as the last argument the process asks for
 * spin-wait scheduling (hipDeviceScheduleSpin) before any other HIP call, so
 * hipStreamSynchronize polls too.
 *
 * Input: a raw file holding fp32 logits [n_rows, V] then fp32 uniforms
 * [n_rows, k] (bench.py writes it).  Calls cycle over the rows.  Output: one
 * JSON line on stdout.
 *   usage: d3s_latency <file> <n_rows> <V> <k> <calls> <temperature> <top_p> [spin] */
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdlib.h>
#include <time.h>

#include <algorithm>
#include <string>
#include <vector>

#include "../../include/d3s_sampler.h"

namespace {

[[noreturn]] void fail(const char *what, int code) {
  fprintf(stderr, "d3s_latency: %s (%d)\n", what, code);
  exit(1);
}

void check(hipError_t e, const char *what) {
  if (e != hipSuccess) fail(what, (int)e);
}

double now_us() {
  timespec t;
  clock_gettime(CLOCK_MONOTONIC, &t);
  return t.tv_sec * 1e6 + t.tv_nsec * 1e-3;
}

double pct(std::vector<double> v, double q) {
  std::sort(v.begin(), v.end());
  return v[(size_t)(q * (double)(v.size() - 1) + 0.5)];
}

}  // namespace

int main(int argc, char **argv) {
  if (argc != 8 && argc != 9) fail("usage: d3s_latency <file> <n_rows> <V> <k> <calls> <temperature> <top_p> [spin]", argc);
  const bool spin = argc == 9 && std::string(argv[8]) == "spin";
  if (argc == 9 && !spin) fail("the last argument, when given, is spin", 0);
  if (spin) check(hipSetDeviceFlags(hipDeviceScheduleSpin), "hipSetDeviceFlags");
  const int n_rows = atoi(argv[2]), V = atoi(argv[3]), k = atoi(argv[4]), calls = atoi(argv[5]);
  const float T = (float)atof(argv[6]), top_p = (float)atof(argv[7]);
  if (n_rows < 1 || V < 1 || k < 1 || calls < 1) fail("bad sizes", 0);
  std::vector<float> host((size_t)n_rows * (V + k));
  FILE *f = fopen(argv[1], "rb");
  if (!f) fail("cannot open the input file", 0);
  if (fread(host.data(), sizeof(float), host.size(), f) != host.size()) fail("short input file", 0);
  fclose(f);
  float *logits = nullptr, *u = nullptr;
  int32_t *ids = nullptr;
  check(hipMalloc(&logits, (size_t)n_rows * V * sizeof(float)), "hipMalloc");
  check(hipMalloc(&u, (size_t)n_rows * k * sizeof(float)), "hipMalloc");
  check(hipMalloc(&ids, sizeof(int32_t)), "hipMalloc");
  check(hipMemcpy(logits, host.data(), (size_t)n_rows * V * sizeof(float), hipMemcpyHostToDevice), "copy");
  check(hipMemcpy(u, host.data() + (size_t)n_rows * V, (size_t)n_rows * k * sizeof(float),
                  hipMemcpyHostToDevice),
        "copy");
  hipStream_t s;
  check(hipStreamCreate(&s), "hipStreamCreate");
  hipEvent_t a, b;
  check(hipEventCreate(&a), "hipEventCreate");
  check(hipEventCreate(&b), "hipEventCreate");
  const int warm = 100;
  std::vector<double> host_us, call_us, event_us;
  for (int i = 0; i < warm + calls; i++) {
    const int r = i % n_rows;
    const double t0 = now_us();
    const int rc = d3s_sample(logits + (size_t)r * V, D3S_DTYPE_F32, 1, V, V, u + (size_t)r * k, k, nullptr,
                              nullptr, T, top_p, nullptr, ids, nullptr, nullptr, nullptr, 0u, s);
    const double tc = now_us();
    check(hipStreamSynchronize(s), "hipStreamSynchronize");
    const double t1 = now_us();
    if (rc != D3S_OK) fail("d3s_sample", rc);
    if (i >= warm) {
      host_us.push_back(t1 - t0);
      call_us.push_back(tc - t0);
    }
  }
  std::vector<double> poll_us;
  for (int i = 0; i < warm + calls; i++) {
    const int r = i % n_rows;
    const double t0 = now_us();
    const int rc = d3s_sample(logits + (size_t)r * V, D3S_DTYPE_F32, 1, V, V, u + (size_t)r * k, k, nullptr,
                              nullptr, T, top_p, nullptr, ids, nullptr, nullptr, nullptr, 0u, s);
    hipError_t q;
    while ((q = hipStreamQuery(s)) == hipErrorNotReady) {
    }
    check(q, "hipStreamQuery");
    const double t1 = now_us();
    if (rc != D3S_OK) fail("d3s_sample", rc);
    if (i >= warm) poll_us.push_back(t1 - t0);
  }
  for (int i = 0; i < warm + calls; i++) {
    const int r = i % n_rows;
    check(hipEventRecord(a, s), "hipEventRecord");
    const int rc = d3s_sample(logits + (size_t)r * V, D3S_DTYPE_F32, 1, V, V, u + (size_t)r * k, k, nullptr,
                              nullptr, T, top_p, nullptr, ids, nullptr, nullptr, nullptr, 0u, s);
    check(hipEventRecord(b, s), "hipEventRecord");
    check(hipEventSynchronize(b), "hipEventSynchronize");
    if (rc != D3S_OK) fail("d3s_sample", rc);
    float ms = 0.0f;
    check(hipEventElapsedTime(&ms, a, b), "hipEventElapsedTime");
    if (i >= warm) event_us.push_back(ms * 1e3);
  }
  printf("{\"calls\": %d, \"rows\": %d, \"spin\": %s, \"call_p50_us\": %.3f, \"host_p50_us\": %.3f, \"host_p90_us\": %.3f, "
         "\"host_poll_p50_us\": %.3f, \"host_poll_p90_us\": %.3f, "
         "\"event_p50_us\": %.3f, \"event_p90_us\": %.3f}\n",
         calls, n_rows, spin ? "true" : "false", pct(call_us, 0.5), pct(host_us, 0.5), pct(host_us, 0.9), pct(poll_us, 0.5),
         pct(poll_us, 0.9), pct(event_us, 0.5), pct(event_us, 0.9));
  (void)hipEventDestroy(a);
  (void)hipEventDestroy(b);
  (void)hipStreamDestroy(s);
  (void)hipFree(logits);
  (void)hipFree(u);
  (void)hipFree(ids);
  return 0;
}
