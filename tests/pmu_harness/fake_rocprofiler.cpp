// SPDX-License-Identifier: BSD-3-Clause
// A CPU stand-in for the part of rocprofiler-sdk that libxtc_hip_pmu
// (xtc_amd/csrc/pmu.cpp) calls, so that pmu.cpp's own locking and waiting
// can be exercised on a host without a GPU (test infrastructure only; the
// product links the real rocprofiler-sdk).
//
// It keeps the documented threading of the dispatch counting service
// (rocprofiler-sdk/dispatch_counting_service.h): the dispatch callback runs in
// the thread that enqueues the kernel, before the enqueue; the record callback
// runs in another thread once the kernel has completed.  Where the documents
// leave the semantics open it takes the strictest reading, so that a lock
// order or wait in pmu.cpp that could block against a real implementation
// blocks here:
//   * the dispatch callback is called while a per-queue lock is held, and the
//     completion thread takes the same lock around the record callback;
//   * rocprofiler_stop_context waits until every dispatch counted in the
//     window has delivered its record callback;
//   * rocprofiler_destroy_counter_config waits until no dispatch still in
//     flight uses the configuration;
//   * rocprofiler_create_counter_config and the counter queries take the
//     service's registry lock, which the dispatch path also takes.
// Every such internal wait has a deadline (FAKE_WAIT_S); a wait that reaches
// it records a stall (fake_stalls()), so the harness ends and names it
// instead of hanging.  Waits poll (lock attempts and state checks with short
// sleeps) rather than block on condition variables, so that a thread
// sanitizer build sees only plain mutex lock and unlock calls.
#include <rocprofiler-sdk/agent.h>
#include <rocprofiler-sdk/context.h>
#include <rocprofiler-sdk/counter_config.h>
#include <rocprofiler-sdk/counters.h>
#include <rocprofiler-sdk/dispatch_counting_service.h>
#include <rocprofiler-sdk/registration.h>

#include <atomic>
#include <chrono>
#include <cstdio>
#include <cstring>
#include <deque>
#include <map>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

namespace {

using clk = std::chrono::steady_clock;
constexpr double FAKE_WAIT_S = 5.0;

const char* const kCounterNames[] = {"SQ_WAVES", "GRBM_GUI_ACTIVE", "FETCH_SIZE", "SQ_BUSY_CYCLES"};
constexpr int kCounters = 4;
constexpr int kInstances = 8;  // hardware instances per counter (one per XCD)

std::mutex g_registry;  // contexts, configurations, counter queries
std::mutex g_queue;     // held around the dispatch callback and the record callback
std::mutex g_state_mu;  // jobs and counts

rocprofiler_configure_func_t g_configure = nullptr;
rocprofiler_tool_configure_result_t* g_tool = nullptr;
bool g_initialized = false;

rocprofiler_dispatch_counting_service_cb_t g_dispatch_cb = nullptr;
rocprofiler_dispatch_counting_record_cb_t g_record_cb = nullptr;
void* g_dispatch_arg = nullptr;
void* g_record_arg = nullptr;
bool g_ctx_created = false;
std::atomic<bool> g_ctx_started{false};

struct Config {
  std::vector<int> counters;  // indices into kCounterNames
  int in_flight = 0;
};
std::map<uint64_t, Config> g_configs;
uint64_t g_next_config = 1;

struct Job {
  uint64_t dispatch_id;
  int waves;
  uint64_t config;  // 0: not counted
  bool drop_record;
};
std::deque<Job> g_jobs;
uint64_t g_dispatched = 0, g_kernels_done = 0;
int g_counted_pending = 0;  // counted dispatches whose record callback has not returned
std::atomic<int> g_stalls{0};
std::string g_stall_where;
std::atomic<bool> g_drop_next{false};
std::atomic<int> g_kernel_us{50};
std::thread g_worker;
std::atomic<bool> g_stop_worker{false};

void stall(const char* where) {
  std::lock_guard<std::mutex> lk(g_state_mu);
  ++g_stalls;
  if (g_stall_where.empty()) g_stall_where = where;
}

rocprofiler_agent_v0_t make_agent(int i, rocprofiler_agent_type_t type) {
  rocprofiler_agent_v0_t a;
  memset(&a, 0, sizeof(a));
  a.size = sizeof(a);
  a.id.handle = 100 + i;
  a.type = type;
  return a;
}
rocprofiler_agent_v0_t g_agent_list[2] = {make_agent(0, ROCPROFILER_AGENT_TYPE_CPU),
                                          make_agent(1, ROCPROFILER_AGENT_TYPE_GPU)};

// takes `m`, or gives up at the deadline
bool lock_before_deadline(std::mutex& m) {
  const auto deadline = clk::now() + std::chrono::duration<double>(FAKE_WAIT_S);
  while (!m.try_lock()) {
    if (clk::now() > deadline) return false;
    std::this_thread::sleep_for(std::chrono::microseconds(5));
  }
  return true;
}

// the completion side: the kernel runs for g_kernel_us, then (for a counted
// dispatch) the record callback delivers one record per counter instance
void worker_main() {
  for (;;) {
    Job j;
    bool have = false;
    {
      std::lock_guard<std::mutex> lk(g_state_mu);
      if (!g_jobs.empty()) {
        j = g_jobs.front();
        g_jobs.pop_front();
        have = true;
      }
    }
    if (!have) {
      if (g_stop_worker.load()) return;
      std::this_thread::sleep_for(std::chrono::microseconds(10));
      continue;
    }
    std::this_thread::sleep_for(std::chrono::microseconds(g_kernel_us.load()));
    {
      std::lock_guard<std::mutex> lk(g_state_mu);
      ++g_kernels_done;
    }
    if (!j.config) continue;
    std::vector<rocprofiler_counter_record_t> recs;
    std::vector<int> counters;
    {
      std::lock_guard<std::mutex> lk(g_registry);
      auto it = g_configs.find(j.config);
      if (it != g_configs.end()) counters = it->second.counters;
    }
    for (int c : counters)
      for (int inst = 0; inst < kInstances; ++inst) {
        rocprofiler_counter_record_t r;
        memset(&r, 0, sizeof(r));
        r.id = ((uint64_t)c << 32) | (uint64_t)inst;  // counter in the high word
        // SQ_WAVES: the dispatch's waves spread over the instances; others: 1 per instance
        r.counter_value = c == 0 ? (double)(j.waves / kInstances + (inst < j.waves % kInstances ? 1 : 0)) : 1.0;
        r.dispatch_id = j.dispatch_id;
        recs.push_back(r);
      }
    if (!j.drop_record) {
      if (!lock_before_deadline(g_queue)) {
        stall("completion thread: queue lock for the record callback");
      } else {
        rocprofiler_dispatch_counting_service_data_t d;
        memset(&d, 0, sizeof(d));
        d.size = sizeof(d);
        d.dispatch_info.agent_id.handle = 101;
        d.dispatch_info.dispatch_id = j.dispatch_id;
        rocprofiler_user_data_t u;
        u.value = 0;
        g_record_cb(d, recs.data(), recs.size(), u, g_record_arg);
        g_queue.unlock();
      }
    }
    {
      std::lock_guard<std::mutex> lk(g_registry);
      auto it = g_configs.find(j.config);
      if (it != g_configs.end()) --it->second.in_flight;
    }
    {
      std::lock_guard<std::mutex> lk(g_state_mu);
      --g_counted_pending;
    }
  }
}

// true once pred() holds (checked under g_state_mu), false at the deadline
template <class Pred>
bool wait_for(Pred pred) {
  const auto deadline = clk::now() + std::chrono::duration<double>(FAKE_WAIT_S);
  for (;;) {
    {
      std::lock_guard<std::mutex> lk(g_state_mu);
      if (pred()) return true;
    }
    if (clk::now() > deadline) return false;
    std::this_thread::sleep_for(std::chrono::microseconds(10));
  }
}

}  // namespace

extern "C" {

// ---- the rocprofiler-sdk entry points pmu.cpp calls

rocprofiler_status_t rocprofiler_is_initialized(int* status) {
  *status = g_initialized ? 1 : 0;
  return ROCPROFILER_STATUS_SUCCESS;
}

rocprofiler_status_t rocprofiler_force_configure(rocprofiler_configure_func_t f) {
  if (g_initialized || g_configure) return ROCPROFILER_STATUS_ERROR_CONFIGURATION_LOCKED;
  g_configure = f;
  static rocprofiler_client_id_t id{};
  g_tool = f(10000, "fake", 0, &id);
  return ROCPROFILER_STATUS_SUCCESS;
}

rocprofiler_status_t rocprofiler_query_available_agents(rocprofiler_agent_version_t version,
                                                        rocprofiler_query_available_agents_cb_t cb, size_t,
                                                        void* user) {
  const void* ptrs[2] = {&g_agent_list[0], &g_agent_list[1]};
  return cb(version, ptrs, 2, user);
}

rocprofiler_status_t rocprofiler_create_context(rocprofiler_context_id_t* ctx) {
  std::lock_guard<std::mutex> lk(g_registry);
  g_ctx_created = true;
  ctx->handle = 7;
  return ROCPROFILER_STATUS_SUCCESS;
}

rocprofiler_status_t rocprofiler_configure_callback_dispatch_counting_service(
    rocprofiler_context_id_t, rocprofiler_dispatch_counting_service_cb_t dcb, void* darg,
    rocprofiler_dispatch_counting_record_cb_t rcb, void* rarg) {
  std::lock_guard<std::mutex> lk(g_registry);
  g_dispatch_cb = dcb;
  g_dispatch_arg = darg;
  g_record_cb = rcb;
  g_record_arg = rarg;
  return ROCPROFILER_STATUS_SUCCESS;
}

rocprofiler_status_t rocprofiler_start_context(rocprofiler_context_id_t) {
  std::lock_guard<std::mutex> lk(g_registry);
  g_ctx_started = true;
  return ROCPROFILER_STATUS_SUCCESS;
}

rocprofiler_status_t rocprofiler_stop_context(rocprofiler_context_id_t) {
  // strict: returns once every counted dispatch has delivered its record
  if (!wait_for([] { return g_counted_pending == 0; })) {
    stall("rocprofiler_stop_context: records still pending");
    return ROCPROFILER_STATUS_ERROR;
  }
  std::lock_guard<std::mutex> lk(g_registry);
  g_ctx_started = false;
  return ROCPROFILER_STATUS_SUCCESS;
}

rocprofiler_status_t rocprofiler_iterate_agent_supported_counters(rocprofiler_agent_id_t agent,
                                                                  rocprofiler_available_counters_cb_t cb,
                                                                  void* user) {
  std::lock_guard<std::mutex> lk(g_registry);
  if (agent.handle != 101) return ROCPROFILER_STATUS_ERROR_AGENT_NOT_FOUND;
  rocprofiler_counter_id_t ids[kCounters];
  for (int i = 0; i < kCounters; ++i) ids[i].handle = (uint64_t)i;
  return cb(agent, ids, kCounters, user);
}

rocprofiler_status_t rocprofiler_query_counter_info(rocprofiler_counter_id_t id, rocprofiler_counter_info_version_id_t,
                                                    void* info) {
  std::lock_guard<std::mutex> lk(g_registry);
  if (id.handle >= (uint64_t)kCounters) return ROCPROFILER_STATUS_ERROR_COUNTER_NOT_FOUND;
  auto* out = static_cast<rocprofiler_counter_info_v0_t*>(info);
  memset(out, 0, sizeof(*out));
  out->id = id;
  out->name = kCounterNames[id.handle];
  return ROCPROFILER_STATUS_SUCCESS;
}

rocprofiler_status_t rocprofiler_query_record_counter_id(rocprofiler_counter_instance_id_t id,
                                                         rocprofiler_counter_id_t* cid) {
  cid->handle = id >> 32;
  return ROCPROFILER_STATUS_SUCCESS;
}

rocprofiler_status_t rocprofiler_create_counter_config(rocprofiler_agent_id_t agent, rocprofiler_counter_id_t* list,
                                                       size_t n, rocprofiler_counter_config_id_t* cfg) {
  std::lock_guard<std::mutex> lk(g_registry);
  if (agent.handle != 101 || n == 0) return ROCPROFILER_STATUS_ERROR_INVALID_ARGUMENT;
  Config c;
  for (size_t i = 0; i < n; ++i) c.counters.push_back((int)list[i].handle);
  cfg->handle = g_next_config++;
  g_configs[cfg->handle] = c;
  return ROCPROFILER_STATUS_SUCCESS;
}

rocprofiler_status_t rocprofiler_destroy_counter_config(rocprofiler_counter_config_id_t cfg) {
  // strict: waits until no dispatch in flight uses the configuration
  const auto deadline = clk::now() + std::chrono::duration<double>(FAKE_WAIT_S);
  for (;;) {
    {
      std::lock_guard<std::mutex> lk(g_registry);
      auto it = g_configs.find(cfg.handle);
      if (it == g_configs.end()) return ROCPROFILER_STATUS_ERROR_INVALID_ARGUMENT;
      if (it->second.in_flight == 0) {
        g_configs.erase(it);
        return ROCPROFILER_STATUS_SUCCESS;
      }
    }
    if (clk::now() > deadline) {
      stall("rocprofiler_destroy_counter_config: configuration still in flight");
      return ROCPROFILER_STATUS_ERROR;
    }
    std::this_thread::sleep_for(std::chrono::microseconds(100));
  }
}

// ---- the harness side: runtime start, kernel dispatch, device synchronisation

// The ROCm runtime starts: the registered tool initialises.
int fake_runtime_start(void) {
  if (g_initialized) return 0;
  g_initialized = true;
  g_worker = std::thread(worker_main);
  if (g_tool && g_tool->initialize) return g_tool->initialize(nullptr, g_tool->tool_data);
  return 0;
}

void fake_runtime_stop(void) {
  g_stop_worker = true;
  if (g_worker.joinable()) g_worker.join();
}

// Enqueues a kernel of `waves` waves from the calling thread.
int fake_dispatch(int waves) {
  if (!lock_before_deadline(g_queue)) {
    stall("dispatch: queue lock");
    return 1;
  }
  Job j{0, waves, 0, false};
  {
    std::lock_guard<std::mutex> lk(g_state_mu);
    j.dispatch_id = ++g_dispatched;
  }
  if (g_ctx_started.load() && g_dispatch_cb) {
    rocprofiler_dispatch_counting_service_data_t d;
    memset(&d, 0, sizeof(d));
    d.size = sizeof(d);
    d.dispatch_info.agent_id.handle = 101;
    d.dispatch_info.dispatch_id = j.dispatch_id;
    rocprofiler_counter_config_id_t cfg{0};
    rocprofiler_user_data_t u;
    u.value = 0;
    g_dispatch_cb(d, &cfg, &u, g_dispatch_arg);
    if (cfg.handle) {
      std::lock_guard<std::mutex> lk(g_registry);
      auto it = g_configs.find(cfg.handle);
      if (it != g_configs.end()) {
        ++it->second.in_flight;
        j.config = cfg.handle;
      }
    }
  }
  j.drop_record = j.config && g_drop_next.exchange(false);
  {
    std::lock_guard<std::mutex> lk(g_state_mu);
    if (j.config) ++g_counted_pending;
    g_jobs.push_back(j);
  }
  g_queue.unlock();
  return 0;
}

// Waits for every kernel enqueued so far (hipDeviceSynchronize).
int fake_device_synchronize(void) {
  if (!wait_for([] { return g_kernels_done == g_dispatched; })) {
    stall("device synchronize");
    return 1;
  }
  return 0;
}

// The next counted dispatch never delivers its record (a lost record).
void fake_drop_next_record(void) { g_drop_next = true; }
void fake_set_kernel_us(int us) { g_kernel_us = us; }
int fake_stalls(void) { return g_stalls.load(); }
const char* fake_stall_where(void) {
  static std::string copy;
  std::lock_guard<std::mutex> lk(g_state_mu);
  copy = g_stall_where;
  return copy.c_str();
}
int fake_configs_alive(void) {
  std::lock_guard<std::mutex> lk(g_registry);
  return (int)g_configs.size();
}

}  // extern "C"
