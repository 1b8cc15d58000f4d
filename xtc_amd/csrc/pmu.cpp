// SPDX-License-Identifier: BSD-3-Clause
// libxtc_hip_pmu: GPU hardware counters for the evaluator's pmu_counters
// ("gpu.<counter>"), through rocprofiler-sdk's dispatch counting service.
//
// Replaces the reference's CUPTI range profiler
// (src/xtc/csrcs/runtimes/accelerator/gpu/perf_event_gpu.cpp:56-233): the
// counters of every kernel dispatched while collection is started are summed
// (over dispatches and over the counter's hardware instances: XCDs, SEs, ...),
// as the range profiler accumulates its ranges (perf_event_gpu.cpp:140-197).
//
// rocprofiler-sdk accepts a tool only before the ROCm runtime initialises, so
// xtc_hip_pmu_enable() must run before the first GPU call of the process.  It
// registers a tool whose one context carries a callback dispatch counting
// service; the context stays stopped (no dispatch is touched) until
// xtc_hip_pmu_start().  While it runs, every dispatch is profiled and
// serialised by the service, so timings taken in that window are perturbed,
// as they are under CUPTI.
//
// Counter names are rocprofiler's (rocprofv3 --list-avail): SQ_WAVES,
// GRBM_GUI_ACTIVE, FETCH_SIZE, ...  One configuration must fit the hardware
// counter blocks of a single pass; create_counter_config rejects more.
#include <rocprofiler-sdk/agent.h>
#include <rocprofiler-sdk/context.h>
#include <rocprofiler-sdk/counter_config.h>
#include <rocprofiler-sdk/counters.h>
#include <rocprofiler-sdk/dispatch_counting_service.h>
#include <rocprofiler-sdk/registration.h>

#include "xtc_hip_pmu.h"

#include <dirent.h>
#include <stdio.h>
#include <string.h>
#include <time.h>
#include <unistd.h>

#include <atomic>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

namespace {

std::mutex g_mu;
std::string g_error;
std::atomic<int> g_state{0};  // 0 not registered, 1 registered (waiting for init), 2 initialised, -1 failed
rocprofiler_context_id_t g_ctx{0};
rocprofiler_client_id_t* g_client = nullptr;

struct Agent {
  rocprofiler_agent_id_t id;
  int gpu_index;  // logical index among GPU agents
};
std::vector<Agent> g_agents;

// the open configuration
bool g_have_config = false;
rocprofiler_counter_config_id_t g_config{0};
rocprofiler_agent_id_t g_config_agent{0};
std::unordered_map<uint64_t, int> g_slot_of_counter;  // counter id handle -> slot
std::vector<double> g_sums;
std::atomic<uint64_t> g_issued{0}, g_completed{0};

void set_error(const std::string& e) {
  std::lock_guard<std::mutex> lk(g_mu);
  g_error = e;
}

int fail(const std::string& e) {
  set_error(e);
  return 1;
}

rocprofiler_status_t collect_agents(rocprofiler_agent_version_t, const void** agents, size_t n, void*) {
  int gpu = 0;
  for (size_t i = 0; i < n; ++i) {
    const auto* a = static_cast<const rocprofiler_agent_v0_t*>(agents[i]);
    if (a->type != ROCPROFILER_AGENT_TYPE_GPU) continue;
    g_agents.push_back(Agent{a->id, gpu++});
  }
  return ROCPROFILER_STATUS_SUCCESS;
}

// rocprofiler calls the two callbacks below from its own code paths; they
// take g_mu, so this file never calls into rocprofiler while holding g_mu
// (a rocprofiler lock held around a callback would otherwise order against
// g_mu both ways).
void dispatch_cb(rocprofiler_dispatch_counting_service_data_t data, rocprofiler_counter_config_id_t* config,
                 rocprofiler_user_data_t*, void*) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (!g_have_config || data.dispatch_info.agent_id.handle != g_config_agent.handle) return;
  *config = g_config;
  g_issued.fetch_add(1);
}

void record_cb(rocprofiler_dispatch_counting_service_data_t, rocprofiler_counter_record_t* records, size_t n,
               rocprofiler_user_data_t, void*) {
  // decode the records first, then add them up under g_mu
  std::vector<std::pair<uint64_t, double>> vals;
  vals.reserve(n);
  for (size_t i = 0; i < n; ++i) {
    rocprofiler_counter_id_t cid{0};
    if (rocprofiler_query_record_counter_id(records[i].id, &cid) == ROCPROFILER_STATUS_SUCCESS)
      vals.emplace_back(cid.handle, records[i].counter_value);
  }
  {
    std::lock_guard<std::mutex> lk(g_mu);
    for (const auto& v : vals) {
      auto it = g_slot_of_counter.find(v.first);
      if (it != g_slot_of_counter.end()) g_sums[it->second] += v.second;
    }
  }
  g_completed.fetch_add(1);
}

int tool_init(rocprofiler_client_finalize_t, void*) {
  if (rocprofiler_query_available_agents(ROCPROFILER_AGENT_INFO_VERSION_0, collect_agents,
                                         sizeof(rocprofiler_agent_v0_t), nullptr) != ROCPROFILER_STATUS_SUCCESS) {
    set_error("rocprofiler_query_available_agents failed");
    g_state = -1;
    return -1;
  }
  if (rocprofiler_create_context(&g_ctx) != ROCPROFILER_STATUS_SUCCESS) {
    set_error("rocprofiler_create_context failed");
    g_state = -1;
    return -1;
  }
  if (rocprofiler_configure_callback_dispatch_counting_service(g_ctx, dispatch_cb, nullptr, record_cb, nullptr) !=
      ROCPROFILER_STATUS_SUCCESS) {
    set_error("rocprofiler_configure_callback_dispatch_counting_service failed");
    g_state = -1;
    return -1;
  }
  g_state = 2;
  return 0;
}

void tool_fini(void*) {}

rocprofiler_tool_configure_result_t g_cfg = {sizeof(rocprofiler_tool_configure_result_t), tool_init, tool_fini,
                                             nullptr};

rocprofiler_tool_configure_result_t* configure(uint32_t, const char*, uint32_t, rocprofiler_client_id_t* id) {
  if (id) {
    id->name = "xtc_hip_pmu";
    g_client = id;
  }
  return &g_cfg;
}

// True when this process holds /dev/kfd open: the ROCm runtime (HSA) has
// started, whoever started it.  Read from /proc only; touches no runtime.
bool runtime_started() {
  DIR* d = opendir("/proc/self/fd");
  if (!d) return false;
  bool found = false;
  char path[64], target[256];
  for (struct dirent* e; !found && (e = readdir(d)) != nullptr;) {
    if (e->d_name[0] == '.') continue;
    snprintf(path, sizeof(path), "/proc/self/fd/%s", e->d_name);
    const ssize_t n = readlink(path, target, sizeof(target) - 1);
    if (n <= 0) continue;
    target[n] = 0;
    found = strcmp(target, "/dev/kfd") == 0;
  }
  closedir(d);
  return found;
}

const Agent* agent_of_device(int device) {
  for (const auto& a : g_agents)
    if (a.gpu_index == device) return &a;
  return nullptr;
}

struct CounterList {
  std::vector<rocprofiler_counter_id_t> ids;
};

rocprofiler_status_t collect_counters(rocprofiler_agent_id_t, rocprofiler_counter_id_t* counters, size_t n,
                                      void* user) {
  auto* out = static_cast<CounterList*>(user);
  out->ids.assign(counters, counters + n);
  return ROCPROFILER_STATUS_SUCCESS;
}

bool counter_name(rocprofiler_counter_id_t id, std::string* name) {
  rocprofiler_counter_info_v0_t info{};
  if (rocprofiler_query_counter_info(id, ROCPROFILER_COUNTER_INFO_VERSION_0, &info) != ROCPROFILER_STATUS_SUCCESS ||
      !info.name)
    return false;
  *name = info.name;
  return true;
}

}  // namespace

extern "C" {

const char* xtc_hip_pmu_last_error(void) {
  static thread_local std::string copy;
  std::lock_guard<std::mutex> lk(g_mu);
  copy = g_error;
  return copy.c_str();
}

// Registers the counter tool.  0 on success (the tool initialises with the
// ROCm runtime, on its first use); 1 when rocprofiler is already configured,
// i.e. the runtime started before this call.
int xtc_hip_pmu_enable(void) {
  if (g_state.load() > 0) return 0;
  if (runtime_started())
    return fail("the ROCm runtime of this process has already started: enable GPU counters before the first GPU call");
  int inited = 0;
  rocprofiler_is_initialized(&inited);
  if (inited != 0) return fail("rocprofiler is already configured in this process");
  if (rocprofiler_force_configure(configure) != ROCPROFILER_STATUS_SUCCESS)
    return fail("rocprofiler_force_configure failed (rocprofiler already configured)");
  if (g_state.load() == 0) g_state = 1;
  return 0;
}

// 1 when the tool is initialised and counters can be opened.
int xtc_hip_pmu_ready(void) { return g_state.load() == 2 ? 1 : 0; }

// Number of counters the GPU `device` supports (-1 on error); their names
// through xtc_hip_pmu_counter_name.
int xtc_hip_pmu_counter_count(int device) {
  const Agent* a = agent_of_device(device);
  if (g_state.load() != 2 || !a) return -1;
  CounterList l;
  if (rocprofiler_iterate_agent_supported_counters(a->id, collect_counters, &l) != ROCPROFILER_STATUS_SUCCESS)
    return -1;
  return (int)l.ids.size();
}

int xtc_hip_pmu_counter_name(int device, int index, char* buf, int len) {
  const Agent* a = agent_of_device(device);
  if (g_state.load() != 2 || !a || !buf || len <= 0) return 1;
  CounterList l;
  if (rocprofiler_iterate_agent_supported_counters(a->id, collect_counters, &l) != ROCPROFILER_STATUS_SUCCESS ||
      index < 0 || index >= (int)l.ids.size())
    return 1;
  std::string name;
  if (!counter_name(l.ids[index], &name)) return 1;
  snprintf(buf, (size_t)len, "%s", name.c_str());
  return 0;
}

// Opens a configuration of `n` counters on GPU `device`.  slots[i] is the
// index of names[i] in the sums xtc_hip_pmu_stop writes, or -1 for a name the
// device does not support (left out; the evaluator reports -1 for it).
// 0 on success.
int xtc_hip_pmu_open(int device, int n, const char** names, int* slots) {
  if (g_state.load() != 2) return fail("GPU counters are not enabled (xtc_hip_pmu_enable before the first GPU call)");
  const Agent* a = agent_of_device(device);
  if (!a) return fail("no rocprofiler agent for GPU " + std::to_string(device));
  CounterList l;
  if (rocprofiler_iterate_agent_supported_counters(a->id, collect_counters, &l) != ROCPROFILER_STATUS_SUCCESS)
    return fail("rocprofiler_iterate_agent_supported_counters failed");
  std::unordered_map<std::string, rocprofiler_counter_id_t> by_name;
  for (auto id : l.ids) {
    std::string nm;
    if (counter_name(id, &nm)) by_name.emplace(nm, id);
  }
  std::vector<rocprofiler_counter_id_t> chosen;
  std::unordered_map<uint64_t, int> slot_of;
  for (int i = 0; i < n; ++i) {
    slots[i] = -1;
    if (!names[i]) continue;
    auto it = by_name.find(names[i]);
    if (it == by_name.end()) continue;
    auto seen = slot_of.find(it->second.handle);
    if (seen != slot_of.end()) {
      slots[i] = seen->second;
      continue;
    }
    slots[i] = (int)chosen.size();
    slot_of[it->second.handle] = (int)chosen.size();
    chosen.push_back(it->second);
  }
  // take the open configuration out under g_mu, destroy it and create the
  // new one without it, then publish the new one under g_mu
  rocprofiler_counter_config_id_t old{0};
  bool had = false;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    had = g_have_config;
    old = g_config;
    g_have_config = false;
    g_slot_of_counter = slot_of;
    g_sums.assign(chosen.size(), 0.0);
  }
  if (had) rocprofiler_destroy_counter_config(old);
  if (chosen.empty()) return 0;
  rocprofiler_counter_config_id_t cfg{0};
  if (rocprofiler_create_counter_config(a->id, chosen.data(), chosen.size(), &cfg) != ROCPROFILER_STATUS_SUCCESS)
    return fail("rocprofiler_create_counter_config failed (unsupported set, or more counters than one pass holds)");
  std::lock_guard<std::mutex> lk(g_mu);
  g_config = cfg;
  g_config_agent = a->id;
  g_have_config = true;
  return 0;
}

// Zeroes the sums and starts collection.
int xtc_hip_pmu_start(void) {
  if (g_state.load() != 2) return fail("GPU counters are not enabled");
  {
    std::lock_guard<std::mutex> lk(g_mu);
    for (double& s : g_sums) s = 0.0;
  }
  g_issued = 0;
  g_completed = 0;
  if (rocprofiler_start_context(g_ctx) != ROCPROFILER_STATUS_SUCCESS) return fail("rocprofiler_start_context failed");
  return 0;
}

// Stops collection once every profiled dispatch has reported (at most
// ~2 s of host-side waiting after the caller's own synchronisation) and
// copies the sums, one per opened counter slot.
int xtc_hip_pmu_stop(double* sums, int n) {
  if (g_state.load() != 2) return fail("GPU counters are not enabled");
  const struct timespec pause = {0, 1000000};
  for (int i = 0; i < 2000 && g_completed.load() < g_issued.load(); ++i) nanosleep(&pause, nullptr);
  const bool complete = g_completed.load() >= g_issued.load();
  rocprofiler_stop_context(g_ctx);
  std::lock_guard<std::mutex> lk(g_mu);
  for (int i = 0; i < n && i < (int)g_sums.size(); ++i) sums[i] = g_sums[i];
  if (!complete) {
    g_error = "GPU counters: dispatches still unreported when collection stopped";
    return 1;
  }
  return 0;
}

// Drops the open configuration.
void xtc_hip_pmu_close(void) {
  rocprofiler_counter_config_id_t old{0};
  bool had = false;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    had = g_have_config;
    old = g_config;
    g_have_config = false;
    g_slot_of_counter.clear();
    g_sums.clear();
  }
  if (had) rocprofiler_destroy_counter_config(old);
}

}  // extern "C"
