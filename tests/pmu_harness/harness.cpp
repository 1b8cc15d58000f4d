// SPDX-License-Identifier: BSD-3-Clause
// Replays, on the CPU, the calls that loop-explore with a GPU hardware
// counter makes into libxtc_hip_pmu (xtc_amd/csrc/pmu.cpp), linked against
// the rocprofiler-sdk stand-in of fake_rocprofiler.cpp (test infrastructure).
//
// Per sample, as xtc_amd/search/explore.py drives HipEvaluator and as
// xtc_hip_evaluate_perf (xtc_amd/csrc/runtime.hip) drives the counter hooks:
//   open(counters) -> validation call -> warm-up call ->
//   repeat x { start -> call x attempts -> device synchronize -> stop }
//   -> close
// where a call is the payload's kernel plus the one-wave completion kernel of
// xtc_hip_synchronize, waited for.  Meanwhile a second thread loads and
// unloads payload libraries (dlopen/dlclose), as the explorer's compile
// threads and the evaluator's unload do, and at the end it is joined (the
// pool's shutdown).
//
// usage: harness <scenario> <samples> <payload.so>
//   scenario "explore":  one counter per sample
//   scenario "switch":   counter sets alternate between samples
//   scenario "lost":     one record of the first window is lost; that stop
//                        must fail within its bounded wait, and the next
//                        samples must count correctly
// Prints one line per sample; exit 0 when every count is right and no wait
// of the stand-in reached its deadline, 1 on a wrong count, 2 on a stall,
// 3 when the watchdog fires.
#include <dlfcn.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include <atomic>
#include <chrono>
#include <string>
#include <thread>

#include "xtc_hip_pmu.h"

extern "C" {
int fake_runtime_start(void);
void fake_runtime_stop(void);
int fake_dispatch(int waves);
int fake_device_synchronize(void);
void fake_drop_next_record(void);
int fake_stalls(void);
const char* fake_stall_where(void);
int fake_configs_alive(void);
}

namespace {

std::atomic<const char*> g_phase{"start"};
std::atomic<int> g_sample{-1};

constexpr int kGemmWaves = 64 * 4;  // a 512^3 tile of 64 workgroups x 4 waves

// one payload call: the GEMM, then xtc_hip_synchronize's completion kernel,
// waited for
bool payload_call() {
  return fake_dispatch(kGemmWaves) == 0 && fake_dispatch(1) == 0 && fake_device_synchronize() == 0;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc != 4) {
    fprintf(stderr, "usage: %s explore|switch|lost <samples> <payload.so>\n", argv[0]);
    return 64;
  }
  const std::string scenario = argv[1];
  const int samples = atoi(argv[2]);
  const char* payload = argv[3];

  std::atomic<bool> done{false};
  std::thread watchdog([&] {
    const auto t0 = std::chrono::steady_clock::now();
    while (!done.load()) {
      std::this_thread::sleep_for(std::chrono::milliseconds(20));
      if (std::chrono::steady_clock::now() - t0 > std::chrono::seconds(60)) {
        fprintf(stdout, "WATCHDOG: sample %d stuck in %s\n", g_sample.load(), g_phase.load());
        fflush(stdout);
        _exit(3);
      }
    }
  });

  if (xtc_hip_pmu_enable() != 0) {
    printf("enable failed: %s\n", xtc_hip_pmu_last_error());
    return 1;
  }
  if (fake_runtime_start() != 0 || !xtc_hip_pmu_ready()) {
    printf("tool did not initialise: %s\n", xtc_hip_pmu_last_error());
    return 1;
  }
  // the explorer's peak probe: kernels with the context stopped
  for (int i = 0; i < 4; ++i) fake_dispatch(8);
  fake_device_synchronize();

  // the compile/unload side: payload libraries loaded and unloaded while
  // samples are evaluated
  std::atomic<int> loads{0};
  std::thread loader([&] {
    while (!done.load()) {
      void* h = dlopen(payload, RTLD_NOW | RTLD_LOCAL);
      if (h) {
        dlsym(h, "payload_entry");
        dlclose(h);
        ++loads;
      }
      xtc_hip_pmu_ready();
      std::this_thread::sleep_for(std::chrono::microseconds(200));
    }
  });

  int wrong = 0;
  const char* one[] = {"SQ_WAVES"};
  const char* two[] = {"GRBM_GUI_ACTIVE", "SQ_WAVES", "NOT_A_COUNTER"};
  for (int s = 0; s < samples; ++s) {
    g_sample = s;
    const bool alt = scenario == "switch" && (s & 1);
    const char** names = alt ? two : one;
    const int n = alt ? 3 : 1;
    int slots[3] = {-2, -2, -2};
    g_phase = "open";
    if (xtc_hip_pmu_open(0, n, names, slots) != 0) {
      printf("sample %d: open failed: %s\n", s, xtc_hip_pmu_last_error());
      return 1;
    }
    const int waves_slot = alt ? slots[1] : slots[0];
    if (alt && (slots[0] < 0 || slots[2] != -1)) {
      printf("sample %d: slots %d %d %d\n", s, slots[0], slots[1], slots[2]);
      ++wrong;
    }
    g_phase = "validation call";
    if (!payload_call()) break;
    g_phase = "warm-up call";
    if (!payload_call()) break;
    double waves[2] = {0, 0};
    int stop_rc[2] = {0, 0};
    for (int r = 0; r < 2; ++r) {
      g_phase = "start";
      if (xtc_hip_pmu_start() != 0) {
        printf("sample %d: start failed: %s\n", s, xtc_hip_pmu_last_error());
        return 1;
      }
      if (scenario == "lost" && s == 0 && r == 0) fake_drop_next_record();
      g_phase = "timed call";
      if (!payload_call()) break;
      g_phase = "device synchronize";
      if (fake_device_synchronize() != 0) break;
      g_phase = "stop";
      double sums[4] = {0, 0, 0, 0};
      stop_rc[r] = xtc_hip_pmu_stop(sums, 4);
      waves[r] = waves_slot >= 0 ? sums[waves_slot] : -1;
    }
    g_phase = "close";
    xtc_hip_pmu_close();
    const bool lost_window = scenario == "lost" && s == 0;
    for (int r = 0; r < 2; ++r) {
      const bool expect_fail = lost_window && r == 0;
      if (expect_fail) {
        if (stop_rc[r] != 1 || !strstr(xtc_hip_pmu_last_error(), "unreported")) {
          printf("sample %d repeat %d: a lost record gave stop rc %d (%s)\n", s, r, stop_rc[r],
                 xtc_hip_pmu_last_error());
          ++wrong;
        }
      } else if (stop_rc[r] != 0 || waves[r] != kGemmWaves + 1) {
        printf("sample %d repeat %d: stop rc %d, SQ_WAVES %.0f (expected %d)\n", s, r, stop_rc[r], waves[r],
               kGemmWaves + 1);
        ++wrong;
      }
    }
    printf("sample %d/%d ok: SQ_WAVES %.0f %.0f\n", s + 1, samples, waves[0], waves[1]);
    fflush(stdout);
    if (fake_stalls()) break;
  }
  g_phase = "pool shutdown";
  done = true;
  loader.join();
  watchdog.join();
  fake_runtime_stop();
  const int alive = fake_configs_alive();
  printf("payload loads %d, counter configurations alive %d, stalls %d%s%s\n", loads.load(), alive, fake_stalls(),
         fake_stalls() ? ": " : "", fake_stall_where());
  if (fake_stalls()) return 2;
  return wrong || alive ? 1 : 0;
}
