/* SPDX-License-Identifier: BSD-3-Clause */
/* libxtc_hip_pmu: GPU hardware counters ("gpu.<counter>" pmu_counters of the
 * XTC evaluators) through rocprofiler-sdk's dispatch counting service.
 *
 * Replaces the reference's CUPTI range profiler,
 * src/xtc/csrcs/runtimes/accelerator/gpu/perf_event_gpu.cpp:56-233
 * (open/start/stop/close_perf_events__gpu and get_perf_event_config__gpu),
 * which src/xtc/csrcs/runtimes/host/perf_event_linux.c:133-221 dispatches to
 * for names starting with "gpu.".  Counters are summed over every kernel
 * dispatched between start and stop, and over the counter's hardware
 * instances, as perf_event_gpu.cpp:140-197 accumulates its ranges.
 *
 * xtc_hip_evaluate_perf, declared in xtc_hip.h, finds these entry points in the process
 * when the library is loaded with global symbols, and uses them for every
 * "gpu.<name>" event other than gpu.time / gpu.clocks; "gpu.cycles" reads
 * GRBM_GUI_ACTIVE.  Plain C types only; 0 = success unless stated. */
#ifndef XTC_HIP_PMU_H
#define XTC_HIP_PMU_H

#ifdef __cplusplus
extern "C" {
#endif

/* Message of the last failure. */
const char *xtc_hip_pmu_last_error(void);

/* Registers the counter tool with rocprofiler-sdk.  Must run before the first
 * GPU call of the process (rocprofiler accepts tools only then); 1 if the
 * runtime already started. */
int xtc_hip_pmu_enable(void);

/* 1 once the tool has initialised with the runtime. */
int xtc_hip_pmu_ready(void);

/* Counters GPU `device` supports (-1 on error) and the name of the
 * index-th (rocprofv3 --list-avail names: SQ_WAVES, GRBM_GUI_ACTIVE, ...). */
int xtc_hip_pmu_counter_count(int device);
int xtc_hip_pmu_counter_name(int device, int index, char *buf, int len);

/* Opens one configuration of n counters on GPU `device` (replaces
 * get_perf_event_config__gpu + open_perf_events__gpu).  slots[i] receives
 * the index of names[i] in the sums of xtc_hip_pmu_stop, or -1 when the
 * device does not have it.  Fails when the set does not fit one pass. */
int xtc_hip_pmu_open(int device, int n, const char **names, int *slots);

/* Zeroes the sums and starts collection (start_perf_events__gpu). */
int xtc_hip_pmu_start(void);

/* Stops collection after every profiled dispatch has reported and writes up
 * to n sums (stop_perf_events__gpu + read_perf_events__gpu). */
int xtc_hip_pmu_stop(double *sums, int n);

/* Drops the open configuration (close_perf_events__gpu). */
void xtc_hip_pmu_close(void);

#ifdef __cplusplus
}
#endif

#endif /* XTC_HIP_PMU_H */
