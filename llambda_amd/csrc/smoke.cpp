// smoke.cpp -- llambda_hip_smoke, the command-line check of one packed
// projection through the C ABI, the counterpart of the reference's
// native/llambda_npu_smoke.cpp:41-151: probe, create a session from the file
// the :hip exporter writes, run it on an input of 0.5 everywhere (warm-up
// runs, then timed runs) and print one line with the runtime version, the
// element counts, the session set-up and warm run times and the first
// output.
//
//   llambda_hip_smoke PROJECTION_FILE [WARMUP_RUNS] [TIMED_RUNS]
//
// Exit status: 0 on success, 1 when the device or a call fails, 2 on bad
// arguments.
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "../../include/llambda_hip.h"

int main(int argc, char** argv) {
  if (argc < 2 || argc > 4) {
    std::fprintf(stderr, "usage: llambda_hip_smoke PROJECTION_FILE [WARMUP_RUNS] [TIMED_RUNS]\n");
    return 2;
  }
  const char* path = argv[1];
  const int warmup_runs = argc > 2 ? std::atoi(argv[2]) : 1;
  const int timed_runs = argc > 3 ? std::atoi(argv[3]) : 1;
  if (warmup_runs < 0 || timed_runs <= 0) {
    std::fprintf(stderr, "Warmup runs must be nonnegative and timed runs positive.\n");
    return 2;
  }

  const auto session_start = std::chrono::steady_clock::now();
  if (llambda_hip_probe() != 1) {
    std::fprintf(stderr, "HIP probe failed: %s\n", llambda_hip_last_error());
    return 1;
  }
  llambda_hip_session* session = nullptr;
  if (llambda_hip_session_create(path, nullptr, nullptr, &session) != 0) {
    std::fprintf(stderr, "Session creation failed: %s\n", llambda_hip_last_error());
    return 1;
  }
  const auto session_end = std::chrono::steady_clock::now();

  const size_t input_count = llambda_hip_session_input_element_count(session);
  const size_t output_count = llambda_hip_session_output_element_count(session);
  std::vector<float> input(input_count, 0.5f);
  std::vector<float> output(output_count);
  auto run = [&](const char* what) {
    if (llambda_hip_session_run(session, input.data(), input.size(), output.data(),
                                output.size()) != 0) {
      std::fprintf(stderr, "%s failed: %s\n", what, llambda_hip_last_error());
      llambda_hip_session_destroy(session);
      return false;
    }
    return true;
  };
  for (int i = 0; i < warmup_runs; ++i)
    if (!run("Warmup")) return 1;
  const auto run_start = std::chrono::steady_clock::now();
  for (int i = 0; i < timed_runs; ++i)
    if (!run("Inference")) return 1;
  const auto run_end = std::chrono::steady_clock::now();

  const double session_ms =
      std::chrono::duration<double, std::milli>(session_end - session_start).count();
  const double run_ms =
      std::chrono::duration<double, std::milli>(run_end - run_start).count() / timed_runs;
  std::printf("%s (%s): %zu inputs -> %zu outputs; session = %.3f ms; warm run = %.4f ms; "
              "first output = %.9g\n",
              llambda_hip_runtime_version(), llambda_hip_bridge_version(), input_count,
              output_count, session_ms, run_ms, output.empty() ? 0.0 : (double)output.front());
  llambda_hip_session_destroy(session);
  return 0;
}
